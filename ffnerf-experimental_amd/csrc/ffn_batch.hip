// ffn_batch.hip -- training batches made on the GPU: uniform or error-weighted
// pixel draws over all resident training images and their pinhole rays and
// target colours.
//
// Reference: the host-side producer and ray builder (run_ffnerf_OG.py:585-686,
// ffnerf_tools.py:175-234).  The ray math is the reference's: OpenCV camera
// axes, pixel centre ((u + 0.5 - cx) / fx, (v + 0.5 - cy) / fy, 1), rotated by
// the camera-to-world matrix, normalised with +1e-12; origin = camera centre.
// Pixel r of a batch is pixel floor(h * P / 2^32) of the P = n W H pixels,
// h = lowbias32(seed ^ r * 2654435769), so a batch is a pure function of its
// seed (the CPU tests draw the same pixels).
#include "ffn_device.h"
#include "ffn_kernels.h"

namespace ffn {

// ray and target colour of pixel p (flat index over the n W H pixels of the resident images)
__device__ __forceinline__ void emit_pixel_ray(const float* __restrict__ images, uint32_t W, uint32_t H,
                                               const float* __restrict__ c2w, const float* __restrict__ K,
                                               uint32_t p, uint32_t r, float4* __restrict__ rays,
                                               float4* __restrict__ targets, uint32_t* __restrict__ pixel_ids) {
  const uint32_t per_image = W * H;
  const uint32_t im = p / per_image, rem = p - im * per_image;
  const uint32_t v = rem / W, u = rem - v * W;
  const float fx = K[0], cx = K[2], fy = K[4], cy = K[5];
  const float x = ((float)u + 0.5f - cx) / fx;
  const float y = ((float)v + 0.5f - cy) / fy;
  const float* m = c2w + 16 * (size_t)im;
  float d[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) d[i] = (m[4 * i] * x + m[4 * i + 1] * y) + m[4 * i + 2];
  const float nrm = sqrtf(d[0] * d[0] + d[1] * d[1] + d[2] * d[2]) + 1e-12f;
  rays[2 * (size_t)r] = make_float4(m[3], m[7], m[11], 1.0f);
  rays[2 * (size_t)r + 1] = make_float4(d[0] / nrm, d[1] / nrm, d[2] / nrm, 0.0f);
  const float* px = images + ((size_t)p) * 3;
  targets[r] = make_float4(px[0], px[1], px[2], 0.0f);
  if (pixel_ids) pixel_ids[r] = p;
}

__global__ __launch_bounds__(256) void k_make_batch(const float* __restrict__ images, uint32_t n_images, uint32_t W,
                                                    uint32_t H, const float* __restrict__ c2w,
                                                    const float* __restrict__ K, uint32_t num_rays, uint32_t seed,
                                                    float4* __restrict__ rays, float4* __restrict__ targets,
                                                    uint32_t* __restrict__ pixel_ids) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= num_rays) return;
  const uint32_t total = W * H * n_images;
  const uint32_t h = hash_u32(seed ^ (r * 2654435769u));
  const uint32_t p = (uint32_t)(((uint64_t)h * total) >> 32);
  emit_pixel_ray(images, W, H, c2w, K, p, r, rays, targets, pixel_ids);
}

// Error-weighted draws (the reference's producer, run_ffnerf_OG.py:490-516 and 635-677): ray r's image is
// im = floor(h0 n / 2^32), h0 = lowbias32(seed ^ r * 2654435769).  Proposal t (t = 0, 1, ...) is pixel
// floor(h_t W H / 2^32) of that image, h_t = lowbias32(h0 ^ (t + 1) * 0x9E3779B9), accepted when
// lowbias32(h_t ^ 0x5BD1E995) & 255 <= its weight, i.e. with probability (w + 1) / 256 as the reference's
// rng.integers(0, 256) <= w.  Rays r < uniform_rays keep proposal 0; the others keep the first accepted
// proposal, or proposal max_tries - 1 when none is.  Two deliberate departures from the reference: its
// rejection loop has no bound (run_ffnerf_OG.py:508-514; at max_tries = 4096 every weight >= 1 leaves a ray
// on its last proposal with probability <= (254/256)^4096 < 2e-14, all weights 0 <= 1.2e-7), and its uniform
// share is int(0.2 B_im) rays within each image's group (run_ffnerf_OG.py:503,677), here the first
// uniform_rays rays of the batch, whose images are drawn like every ray's.
__global__ __launch_bounds__(256) void k_make_batch_weighted(
    const float* __restrict__ images, uint32_t n_images, uint32_t W, uint32_t H, const float* __restrict__ c2w,
    const float* __restrict__ K, const uint8_t* __restrict__ weights, uint32_t num_rays, uint32_t uniform_rays,
    uint32_t max_tries, uint32_t seed, float4* __restrict__ rays, float4* __restrict__ targets,
    uint32_t* __restrict__ pixel_ids) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= num_rays) return;
  const uint32_t per_image = W * H;
  const uint32_t h0 = hash_u32(seed ^ (r * 2654435769u));
  const uint32_t im = (uint32_t)(((uint64_t)h0 * n_images) >> 32);
  const uint8_t* wmap = weights + (size_t)im * per_image;
  const uint32_t tries = r < uniform_rays ? 1u : max_tries;
  uint32_t q = 0;
  for (uint32_t t = 0; t < tries; ++t) {
    const uint32_t ht = hash_u32(h0 ^ ((t + 1u) * 0x9E3779B9u));
    q = (uint32_t)(((uint64_t)ht * per_image) >> 32);
    if (r < uniform_rays || (hash_u32(ht ^ 0x5BD1E995u) & 255u) <= (uint32_t)wmap[q]) break;
  }
  emit_pixel_ray(images, W, H, c2w, K, im * per_image + q, r, rays, targets, pixel_ids);
}

hipError_t launch_make_batch(const float* images, uint32_t n_images, uint32_t W, uint32_t H, const float* c2w,
                             const float* K, uint32_t num_rays, uint32_t seed, float4* rays, float4* targets,
                             uint32_t* pixel_ids, hipStream_t st) {
  if (num_rays == 0) return hipSuccess;
  hipLaunchKernelGGL(k_make_batch, dim3((num_rays + 255) / 256), dim3(256), 0, st, images, n_images, W, H, c2w, K,
                     num_rays, seed, rays, targets, pixel_ids);
  return hipGetLastError();
}

hipError_t launch_make_batch_weighted(const float* images, uint32_t n_images, uint32_t W, uint32_t H,
                                      const float* c2w, const float* K, const uint8_t* weights, uint32_t num_rays,
                                      uint32_t uniform_rays, uint32_t max_tries, uint32_t seed, float4* rays,
                                      float4* targets, uint32_t* pixel_ids, hipStream_t st) {
  if (num_rays == 0) return hipSuccess;
  hipLaunchKernelGGL(k_make_batch_weighted, dim3((num_rays + 255) / 256), dim3(256), 0, st, images, n_images, W, H,
                     c2w, K, weights, num_rays, uniform_rays, max_tries, seed, rays, targets, pixel_ids);
  return hipGetLastError();
}

}  // namespace ffn
