// ffn_sample.hip -- occupancy-weighted importance resampler
// (reference: ffnerf_OG.cl:1002-1250, one work-group of S work-items per ray).
//
// MI355X mapping: one ray per S-lane segment of a 64-lane wavefront; the
// reference's LDS Blelloch scans/reductions become lane shuffles with the same
// trees, so the sample times are bit-identical to the CPU restatement.
#include "ffn_device.h"
#include "ffn_kernels.h"

namespace ffn {

struct SampleOut {
  float t, dt;
  bool run_start;
};

// One lane = one sample of one ray.  All lanes of the wave must call this
// (it shuffles); lanes with valid == false get benign values.
__device__ __forceinline__ SampleOut sample_lane(const DevCfg& c, const float4* __restrict__ rays, uint32_t ray_id,
                                                 bool valid, int lid, int S, int base, uint32_t seed,
                                                 const uint32_t* __restrict__ occ_in, int do_train) {
  float o[3] = {0.f, 0.f, 0.f}, d[3] = {0.f, 0.f, 1.f};
  if (valid) {
    float4 ro = rays[2 * ray_id], rd = rays[2 * ray_id + 1];
    o[0] = ro.x; o[1] = ro.y; o[2] = ro.z;
    d[0] = rd.x; d[1] = rd.y; d[2] = rd.z;
  }
  const uint32_t WG = (uint32_t)S;
  float t0 = 0.0f, t1 = 0.0f;
  bool hit = ray_aabb(o, d, c.bmin, c.bmax, t0, t1);
  float t0_l = 0.0f, t1_l = 0.0f;
  bool hit_l = false;
  if (hit) {
    t0 = fmaxf(t0, c.t_near);
    t1 = fminf(t1, c.t_far);
    if (!(t1 <= t0)) {
      hit_l = true;
      t0_l = t0 + 1.0e-6f;
      t1_l = t1;
    }
  }
  hit_l = hit_l && valid;
  float dtb = hit_l ? ((t1_l - t0_l) * (1.0f / (float)WG)) : 0.0f;
  dtb = fminf(c.dt_max, fmaxf(c.dt_min, dtb));
  const float dt_base = hit_l ? dtb : 0.0f;
  // hit_l is uniform over the segment (every lane of a ray computes the same
  // values), so the shuffles below stay inside rays that all take this path.
  uint32_t rng0 = hash_u32(seed ^ ray_id * 1597334677u);
  const float u0 = rand01(rng0) * (1.0f / (float)WG);

  const float* inv_box = c.inv_bs;  // 1.0f / (bmax - bmin), computed on the host
  const int G = c.G;

  uint32_t rng = hash_u32(seed ^ ray_id * 747796405u ^ (uint32_t)lid * 2891336453u);
  float u = ((float)lid + rand01(rng)) * (1.0f / (float)WG);
  float tk = t0_l + (t1_l - t0_l) * u;
  float gm[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    float xk = o[i] + tk * d[i];
    gm[i] = (xk - c.bmin[i]) * inv_box[i] * (float)G;
  }
  float occ = 0.0f;
  if (hit_l && gm[0] >= 0.0f && gm[0] < (float)G && gm[1] >= 0.0f && gm[1] < (float)G && gm[2] >= 0.0f &&
      gm[2] < (float)G) {
    int im[3];
    uint32_t sub = 0;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      int v = (int)floorf(gm[i]);
      im[i] = v < 0 ? 0 : (v > G - 1 ? G - 1 : v);
      float f = gm[i] - floorf(gm[i]);
      f = fminf(fmaxf(f, 0.0f), 1.0f - 1e-7f);
      sub += (f > 0.5f ? 1u : 0u) << i;
    }
    int cell = im[0] + G * (im[1] + G * im[2]);
    uint32_t occ4 = (occ_in[cell] >> (4u * sub)) & 0xFu;
    uint32_t q_eff = do_train ? (occ4 + 1u) : ((occ4 > 2u) ? (occ4 - 2u) : 0u);
    occ = (float)q_eff * (1.0f / 16.0f);
  }
  float infer_f = do_train ? 0.0f : 1.0f;
  float active = (occ > 0.0f) ? 1.0f : 0.0f;
  float rho_base = c.rho_min + (c.rho_max - c.rho_min) * occ;
  float rho = rho_base * (1.0f - infer_f + infer_f * active);
  float wp = safe_pow_pos(rho * dt_base, 1.3f);

  // Wtot/pref only enter through exp(-LAMBDA_FOCUS * pi) with LAMBDA_FOCUS = 0
  // (ffnerf_OG.cl:57,1173-1175): the gain is exactly 1, so g = wp.
  const float g = wp;
  float gtot = fmaxf(seg_reduce_add(g, lid, S, base), 1.0e-12f);
  float active_count = seg_reduce_add(active, lid, S, base);
  float any_active = (active_count > 0.5f) ? 1.0f : 0.0f;
  float inv_active = 1.0f / fmaxf(active_count, 1.0f);
  float uta = active * inv_active;
  float lo_u = 1.0f / (float)WG;
  float uniform_term = lo_u + (uta - lo_u) * any_active;
  float proposal_term = any_active * (g / gtot);
  float p = 0.3f * uniform_term + (1.0f - 0.3f) * proposal_term;
  float cdf = seg_scan_excl_add(p, lid, S, base) + p;

  float uk = u0 + (float)lid * (1.0f / (float)WG);
  uk = fminf(uk, 0.99999994f);
  int lo = 0, hi = S - 1;
  for (int it = 1; it < S; it <<= 1) {
    int mid = (lo + hi) >> 1;
    float cm = __shfl(cdf, base + mid);
    if (lo < hi) {
      if (cm >= uk) hi = mid;
      else lo = mid + 1;
    }
  }
  float t_out = __shfl(tk, base + lo);

  uint32_t key = 0xFFFFFFFEu;
  {
    float go[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      float xo = o[i] + t_out * d[i];
      go[i] = (xo - c.bmin[i]) * inv_box[i] * (float)G;
    }
    int ix = (int)floorf(go[0]), iy = (int)floorf(go[1]), iz = (int)floorf(go[2]);
    if ((uint32_t)ix < (uint32_t)G && (uint32_t)iy < (uint32_t)G && (uint32_t)iz < (uint32_t)G) {
      uint32_t sub = 0;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        float f = go[i] - floorf(go[i]);
        f = fminf(fmaxf(f, 0.0f), 1.0f - 1e-7f);
        sub += (f >= 0.5f ? 1u : 0u) << i;
      }
      int cell = ix + G * (iy + G * iz);
      key = (((uint32_t)cell) << 3) | (sub & 7u);
    }
  }
  uint32_t prev_key = __shfl(key, base + lid - 1);
  SampleOut r;
  if (hit_l) {
    r.t = t_out;
    r.dt = dt_base;
    r.run_start = (lid == 0) || (key != prev_key);
  } else {
    r.t = 0.0f;
    r.dt = 0.0f;
    r.run_start = true;
  }
  return r;
}

__global__ __launch_bounds__(256) void k_sample(DevCfg c, const float4* __restrict__ rays, uint32_t num_rays,
                                                int S, int log2S, uint32_t seed, const uint32_t* __restrict__ occ_in,
                                                int do_train, float* __restrict__ Ts, float* __restrict__ DTs,
                                                uint32_t* __restrict__ flags, uint32_t* __restrict__ tile_busy) {
  const uint64_t gtid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int lane = threadIdx.x & 63;
  const int lid = lane & (S - 1);
  const int base = lane - lid;
  const uint64_t ray64 = gtid >> log2S;
  const bool valid = ray64 < num_rays;
  const uint32_t ray_id = valid ? (uint32_t)ray64 : 0u;
  SampleOut so = sample_lane(c, rays, ray_id, valid, lid, S, base, seed, occ_in, do_train);
  const uint64_t bal = __ballot(so.run_start);
  // a wavefront's 64 lanes are the 64 samples of one MLP tile: whether any of them is active (dt > 0)
  const uint64_t busy = __ballot(valid && so.dt > 0.0f);
  if (tile_busy && lane == 0 && (uint64_t)(gtid >> log2S) < num_rays) tile_busy[gtid >> 6] = busy != 0ull ? 1u : 0u;
  if (!valid) return;
  Ts[gtid] = so.t;
  DTs[gtid] = so.dt;
  if (lid == 0) {
    uint64_t segmask = (S == 64) ? bal : ((bal >> base) & ((1ull << S) - 1ull));
    flags[2 * ray_id] = (uint32_t)segmask;
    flags[2 * ray_id + 1] = (uint32_t)(segmask >> 32);
  }
}

hipError_t launch_sample(const DevCfg& c, const float4* rays, uint32_t num_rays, int S, uint32_t seed,
                         const uint32_t* occ_in, int do_train, float* Ts, float* DTs, uint32_t* flags,
                         hipStream_t st, uint32_t* tile_busy) {
  int log2S = 0;
  while ((1 << log2S) < S) ++log2S;
  const uint64_t threads = (uint64_t)num_rays * (uint64_t)S;
  const uint64_t blocks = (threads + 255) / 256;
  hipLaunchKernelGGL(k_sample, dim3((unsigned)blocks), dim3(256), 0, st, c, rays, num_rays, S, log2S, seed, occ_in,
                     do_train, Ts, DTs, flags, tile_busy);
  return hipGetLastError();
}

}  // namespace ffn
