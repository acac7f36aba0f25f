// ffn_hash.hip -- multiresolution hash-grid encoding, forward gather and
// backward scatter-add (reference: ffnerf_OG.cl:1286-1364 and 2090-2173).
//
// One thread per sample.  Per level the 8 corner indices are formed first and
// the 8 corner loads (one F-wide vector each) are issued back to back before
// the trilinear sums, so each thread keeps 8 independent gathers in flight.
// The sums run corner by corner without FMA contraction, which makes the
// encodings bit-identical to the CPU restatement.
#include "ffn_device.h"
#include "ffn_kernels.h"

namespace ffn {

template <int F>
struct FVec;
template <>
struct FVec<1> {
  typedef float T;
  static __device__ __forceinline__ void unpack(const T& v, float* o) { o[0] = v; }
};
template <>
struct FVec<2> {
  typedef float2 T;
  static __device__ __forceinline__ void unpack(const T& v, float* o) {
    o[0] = v.x;
    o[1] = v.y;
  }
};
template <>
struct FVec<4> {
  typedef float4 T;
  static __device__ __forceinline__ void unpack(const T& v, float* o) {
    o[0] = v.x;
    o[1] = v.y;
    o[2] = v.z;
    o[3] = v.w;
  }
};

__device__ __forceinline__ void sample_position(const float* __restrict__ x, const float4* __restrict__ rays,
                                                const float* __restrict__ Ts, int log2S, int64_t b, float pos[3]) {
  if (rays) {
    const int64_t r = b >> log2S;
    const float4 o = rays[2 * r], d = rays[2 * r + 1];
    const float t = Ts[b];
    pos[0] = o.x + t * d.x;
    pos[1] = o.y + t * d.y;
    pos[2] = o.z + t * d.z;
  } else {
    pos[0] = x[3 * b + 0];
    pos[1] = x[3 * b + 1];
    pos[2] = x[3 * b + 2];
  }
}

template <int F>
__global__ __launch_bounds__(256) void k_hash_fwd(DevCfg c, const float* __restrict__ x,
                                                  const float4* __restrict__ rays, const float* __restrict__ Ts,
                                                  int log2S, int64_t n, const float* __restrict__ table,
                                                  float* __restrict__ a0, uint32_t* __restrict__ idx_out) {
  typedef typename FVec<F>::T V;
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n) return;
  float pos[3], p[3];
  sample_position(x, rays, Ts, log2S, b, pos);
  normalize_pos(c, pos, p);
  const int L = c.L, LF = c.LF;
  float* out = a0 + b * LF;
  for (int l = 0; l < L; ++l) {
    const LevelCell lc = level_cell(c.res[l], p);
    const uint32_t mask = c.mask[l], off = c.offset[l];
    uint32_t fb[8];
    V val[8];
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      fb[cc] = (off + corner_entry(lc, cc, l, mask)) * (uint32_t)F;
      val[cc] = *reinterpret_cast<const V*>(table + fb[cc]);
    }
    float acc[F];
#pragma unroll
    for (int f = 0; f < F; ++f) acc[f] = 0.0f;
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      const float w = corner_weight(lc, cc);
      float t[F];
      FVec<F>::unpack(val[cc], t);
#pragma unroll
      for (int f = 0; f < F; ++f) acc[f] += w * t[f];
    }
#pragma unroll
    for (int f = 0; f < F; ++f) out[l * F + f] = acc[f];
    if (idx_out) {
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) idx_out[(b * L + l) * 8 + cc] = fb[cc];
    }
  }
}

template <int F, int MODE>
__global__ __launch_bounds__(256) void k_hash_bwd(DevCfg c, const float* __restrict__ x,
                                                  const float4* __restrict__ rays, const float* __restrict__ Ts,
                                                  int log2S, int64_t n, const float* __restrict__ g,
                                                  float* __restrict__ dst, float lr) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n) return;
  float pos[3], p[3];
  sample_position(x, rays, Ts, log2S, b, pos);
  normalize_pos(c, pos, p);
  const int L = c.L, LF = c.LF;
  const float* gin = g + b * LF;
  for (int l = 0; l < L; ++l) {
    float gf[F];
    bool any = false;
#pragma unroll
    for (int f = 0; f < F; ++f) {
      float v = gin[l * F + f];
      // non-finite gradients are dropped (ffnerf_OG.cl:2162); exact zeros add nothing
      if (!isfinite(v)) v = 0.0f;
      if (MODE == 1) v = -(lr * c.lvl_lr_scale[l]) * 0.5f * v;
      gf[f] = v;
      any |= (v != 0.0f);
    }
    if (!any) continue;
    const LevelCell lc = level_cell(c.res[l], p);
    const uint32_t mask = c.mask[l], off = c.offset[l];
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      const float w = corner_weight(lc, cc);
      const uint32_t fb = (off + corner_entry(lc, cc, l, mask)) * (uint32_t)F;
#pragma unroll
      for (int f = 0; f < F; ++f)
        if (gf[f] != 0.0f) unsafeAtomicAdd(dst + fb + f, gf[f] * w);
    }
  }
}

hipError_t launch_hash_fwd(const DevCfg& c, const float* x, const float4* rays, const float* Ts, int log2S,
                           int64_t n, const float* table, float* a0, uint32_t* idx_out, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  switch (c.F) {
    case 1: hipLaunchKernelGGL(k_hash_fwd<1>, grid, block, 0, st, c, x, rays, Ts, log2S, n, table, a0, idx_out); break;
    case 2: hipLaunchKernelGGL(k_hash_fwd<2>, grid, block, 0, st, c, x, rays, Ts, log2S, n, table, a0, idx_out); break;
    case 4: hipLaunchKernelGGL(k_hash_fwd<4>, grid, block, 0, st, c, x, rays, Ts, log2S, n, table, a0, idx_out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_hash_bwd(const DevCfg& c, const float* x, const float4* rays, const float* Ts, int log2S,
                           int64_t n, const float* g, float* dst, int mode, float lr, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
#define FFN_BWD(FV, MV) hipLaunchKernelGGL((k_hash_bwd<FV, MV>), grid, block, 0, st, c, x, rays, Ts, log2S, n, g, dst, lr)
  if (mode == 0) {
    switch (c.F) {
      case 1: FFN_BWD(1, 0); break;
      case 2: FFN_BWD(2, 0); break;
      case 4: FFN_BWD(4, 0); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (c.F) {
      case 1: FFN_BWD(1, 1); break;
      case 2: FFN_BWD(2, 1); break;
      case 4: FFN_BWD(4, 1); break;
      default: return hipErrorInvalidValue;
    }
  }
#undef FFN_BWD
  return hipGetLastError();
}

}  // namespace ffn
