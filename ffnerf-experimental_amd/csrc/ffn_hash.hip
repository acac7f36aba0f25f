// ffn_hash.hip -- multiresolution hash-grid encoding: forward gather and
// backward scatter (reference: ffnerf_OG.cl:1286-1364 and 2090-2173).
//
// MI355X design
//   Forward: one pass per level (grid.y = level).  A level's table (2^19
//   entries x F floats = 4 MiB at the benchmark shape) then stays resident in
//   every XCD's 4 MB L2 while all samples gather from it; the encodings are
//   stored level-major ([L][N][F]), so each pass writes one contiguous array.
//   The trilinear sums run corner by corner without FMA contraction, which
//   makes them bit-identical to the CPU restatement.
//
//   Backward: scattered float atomics run at ~21 G lanes/s on this chip
//   (measured), far below what the HBM can stream, so the scatter is done
//   without global atomics, as a bucketed reduction:
//     1. count  -- per (level, sample chunk), how many corner contributions
//                  land in each bucket (BE consecutive table entries of one
//                  level); LDS histogram, one row of counts per block;
//     2. scan   -- exclusive prefix over the (bucket, block) counts, so every
//                  block owns a contiguous slot range inside every bucket;
//     3. emit   -- recompute the corners and write (entry-in-bucket, value)
//                  pairs to the slots (LDS cursors, streaming writes);
//     4. reduce -- one block per bucket sums its pairs into an LDS copy of
//                  the bucket and applies the update to its own slice of the
//                  table: gradient add, the reference SGD, or Adam.  No
//                  gradient table is materialised for Adam.
//   LDS float atomics (ds_add_f32) sustain only ~0.33 lanes/clk/CU here while
//   ds_add_u64 sustains ~4.9 (both measured), so the reduce accumulates in
//   64-bit fixed point: the emit pass records each bucket's largest |value|
//   (integer max on the float bits), and the reduce scales by the power of two
//   that keeps the bucket's total below 2^62 -- an exact scaling, one
//   round-to-nearest per pair, ~2^-34 of the bucket's largest value per entry.
//   Levels are processed in groups so the pair buffer stays bounded.
#include "ffn_device.h"
#include "ffn_kernels.h"

namespace ffn {

template <int F>
struct FVec;
template <>
struct FVec<1> {
  typedef float T;
  static __device__ __forceinline__ void unpack(const T& v, float* o) { o[0] = v; }
  static __device__ __forceinline__ T pack(const float* o) { return o[0]; }
};
template <>
struct FVec<2> {
  typedef float2 T;
  static __device__ __forceinline__ void unpack(const T& v, float* o) {
    o[0] = v.x;
    o[1] = v.y;
  }
  static __device__ __forceinline__ T pack(const float* o) { return make_float2(o[0], o[1]); }
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
  static __device__ __forceinline__ T pack(const float* o) { return make_float4(o[0], o[1], o[2], o[3]); }
};

__device__ __forceinline__ void sample_position(const PosSrc& s, int64_t b, float pos[3]) {
  if (s.rays) {
    const int64_t r = b >> s.log2S;
    const float4 o = s.rays[2 * r], d = s.rays[2 * r + 1];
    const float t = s.Ts[b];
    pos[0] = o.x + t * d.x;
    pos[1] = o.y + t * d.y;
    pos[2] = o.z + t * d.z;
  } else {
    const float* xb = s.x + (int64_t)s.x_stride * b;
    pos[0] = xb[0];
    pos[1] = xb[1];
    pos[2] = xb[2];
  }
}

// ---------------------------------------------------------------------------
// forward

template <int F>
__global__ __launch_bounds__(256) void k_hash_fwd(DevCfg c, PosSrc src, int64_t n, int level0,
                                                  const float* __restrict__ table, float* __restrict__ a0,
                                                  FeatLayout lay, uint32_t* __restrict__ idx_out) {
  typedef typename FVec<F>::T V;
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n) return;
  const int l = level0 + (int)blockIdx.y;
  float pos[3], p[3];
  sample_position(src, b, pos);
  normalize_pos(c, pos, p);
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
  *reinterpret_cast<V*>(a0 + l * lay.stride_l + b * lay.stride_b) = FVec<F>::pack(acc);
  if (idx_out) {
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) idx_out[(b * c.L + l) * 8 + cc] = fb[cc];
  }
}

// ---------------------------------------------------------------------------
// backward: bucketed scatter

// The gradient of one (sample, level): scaled as the mode needs, non-finite
// components dropped (ffnerf_OG.cl:2162).  Returns false when it is all zero.
template <int F, int MODE>
__device__ __forceinline__ bool level_grad(const DevCfg& c, const float* __restrict__ g, const FeatLayout& lay,
                                           int64_t b, int l, float lr, float gf[F]) {
  typedef typename FVec<F>::T V;
  float v[F];
  FVec<F>::unpack(*reinterpret_cast<const V*>(g + l * lay.stride_l + b * lay.stride_b), v);
  bool any = false;
#pragma unroll
  for (int f = 0; f < F; ++f) {
    float x = v[f];
    if (!isfinite(x)) x = 0.0f;
    if (MODE == BIN_SGD) x = -(lr * c.lvl_lr_scale[l]) * 0.5f * x;
    gf[f] = x;
    any |= (x != 0.0f);
  }
  return any;
}

template <int F, int MODE>
__global__ __launch_bounds__(256) void k_bin_count(DevCfg c, PosSrc src, int64_t n, BinGroup grp,
                                                   const float* __restrict__ g, FeatLayout lay, float lr,
                                                   uint32_t* __restrict__ cnt, uint32_t* __restrict__ bmax) {
  extern __shared__ uint32_t hist[];
  const int l = grp.level0 + (int)blockIdx.y;
  const int nbl = grp.nbl[l - grp.level0];
  const int chunk = blockIdx.x;
  if (chunk == 0)
    for (int j = threadIdx.x; j < nbl; j += blockDim.x) bmax[grp.bucket_rel[l - grp.level0] + j] = 0u;
  for (int j = threadIdx.x; j < nbl; j += blockDim.x) hist[j] = 0u;
  __syncthreads();
  const int64_t b0 = (int64_t)chunk * grp.chunk;
  const int64_t b1 = b0 + grp.chunk < n ? b0 + grp.chunk : n;
  for (int64_t b = b0 + threadIdx.x; b < b1; b += blockDim.x) {
    float gf[F];
    if (!level_grad<F, MODE>(c, g, lay, b, l, lr, gf)) continue;
    float pos[3], p[3];
    sample_position(src, b, pos);
    normalize_pos(c, pos, p);
    const LevelCell lc = level_cell(c.res[l], p);
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) atomicAdd(&hist[corner_entry(lc, cc, l, c.mask[l]) >> grp.log2_be], 1u);
  }
  __syncthreads();
  const int rel0 = grp.bucket_rel[l - grp.level0];
  for (int j = threadIdx.x; j < nbl; j += blockDim.x) cnt[(int64_t)(rel0 + j) * grp.nblk + chunk] = hist[j];
}

// Block-wide exclusive scan of cnt[0..n) into off[0..n) (256 threads; n may exceed 256).
__device__ __forceinline__ uint32_t block_scan_excl(const uint32_t* cnt, uint32_t* off, int n, uint32_t* wsum) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int per = (n + 255) / 256;
  const int j0 = tid * per;
  uint32_t s = 0;
  for (int j = j0; j < j0 + per && j < n; ++j) s += cnt[j];
  uint32_t incl = s;
  for (int d = 1; d < 64; d <<= 1) {
    uint32_t o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == 63) wsum[wv] = incl;
  __syncthreads();
  uint32_t run = incl - s;
  for (int k = 0; k < wv; ++k) run += wsum[k];
  const uint32_t total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
  for (int j = j0; j < j0 + per && j < n; ++j) {
    off[j] = run;
    run += cnt[j];
  }
  return total;
}

// Emit the (entry, value) pairs of 256 samples at a time: rank them by bucket
// in LDS (a local counting sort), then copy each bucket's run to its slots
// with consecutive lanes on consecutive addresses.
template <int F, int MODE>
__global__ __launch_bounds__(256) void k_bin_emit(DevCfg c, PosSrc src, int64_t n, BinGroup grp,
                                                  const float* __restrict__ g, FeatLayout lay, float lr,
                                                  const uint32_t* __restrict__ off, uint16_t* __restrict__ pair_idx,
                                                  float* __restrict__ pair_val, uint32_t* __restrict__ bmax) {
  typedef typename FVec<F>::T V;
  extern __shared__ uint32_t sm[];
  const int l = grp.level0 + (int)blockIdx.y;
  const int nbl = grp.nbl[l - grp.level0];
  const int chunk = blockIdx.x;
  const int rel0 = grp.bucket_rel[l - grp.level0];
  uint32_t* gcur = sm;             // [nbl] next global slot of each bucket
  uint32_t* lcnt = gcur + nbl;     // [nbl] pairs of the round per bucket
  uint32_t* loff = lcnt + nbl;     // [nbl] their offsets in the stage
  uint32_t* lmax = loff + nbl;     // [nbl] float bits of the largest |value| per bucket
  uint32_t* wsum = lmax + nbl;     // [4]
  // the stage starts 16-byte aligned: (4 nbl + 4) header words rounded up to a multiple of 4
  uint16_t* st_idx = reinterpret_cast<uint16_t*>(sm + ((4 * nbl + 4 + 3) & ~3));  // [2048]
  uint16_t* st_bkt = st_idx + 2048;                          // [2048]
  V* st_val = reinterpret_cast<V*>(st_bkt + 2048);           // [2048]
  const int tid = threadIdx.x;
  for (int j = tid; j < nbl; j += 256) {
    gcur[j] = off[(int64_t)(rel0 + j) * grp.nblk + chunk];
    lmax[j] = 0u;
  }
  const uint32_t be_mask = (1u << grp.log2_be) - 1u;
  V* vals = reinterpret_cast<V*>(pair_val);
  const int64_t b_begin = (int64_t)chunk * grp.chunk;
  const int64_t b_end = b_begin + grp.chunk < n ? b_begin + grp.chunk : n;
  for (int64_t rb = b_begin; rb < b_end; rb += 256) {
    for (int j = tid; j < nbl; j += 256) lcnt[j] = 0u;
    __syncthreads();
    const int64_t b = rb + tid;
    float gf[F];
    bool act = b < b_end && level_grad<F, MODE>(c, g, lay, b, l, lr, gf);
    uint32_t ent[8], rank[8];
    LevelCell lc;
    if (act) {
      float pos[3], p[3];
      sample_position(src, b, pos);
      normalize_pos(c, pos, p);
      lc = level_cell(c.res[l], p);
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) {
        ent[cc] = corner_entry(lc, cc, l, c.mask[l]);
        rank[cc] = atomicAdd(&lcnt[ent[cc] >> grp.log2_be], 1u);
      }
    }
    __syncthreads();
    const uint32_t total = block_scan_excl(lcnt, loff, nbl, wsum);
    __syncthreads();
    if (act) {
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) {
        const uint32_t bk = ent[cc] >> grp.log2_be;
        const uint32_t pos = loff[bk] + rank[cc];
        const float w = corner_weight(lc, cc);
        float v[F];
        float amax = 0.0f;
#pragma unroll
        for (int f = 0; f < F; ++f) {
          v[f] = gf[f] * w;
          amax = fmaxf(amax, fabsf(v[f]));
        }
        st_idx[pos] = (uint16_t)(ent[cc] & be_mask);
        st_bkt[pos] = (uint16_t)bk;
        st_val[pos] = FVec<F>::pack(v);
        atomicMax(&lmax[bk], __float_as_uint(amax));
      }
    }
    __syncthreads();
    for (uint32_t i = tid; i < total; i += 256) {
      const uint32_t bk = st_bkt[i];
      const uint32_t dst = gcur[bk] + (i - loff[bk]);
      pair_idx[dst] = st_idx[i];
      vals[dst] = st_val[i];
    }
    __syncthreads();
    for (int j = tid; j < nbl; j += 256) gcur[j] += lcnt[j];
  }
  __syncthreads();
  for (int j = tid; j < nbl; j += 256)
    if (lmax[j]) atomicMax(&bmax[rel0 + j], lmax[j]);
}

template <int F, int MODE>
__global__ __launch_bounds__(1024) void k_bin_reduce(DevCfg c, BinGroup grp, const uint32_t* __restrict__ off,
                                                     const uint16_t* __restrict__ pair_idx,
                                                     const float* __restrict__ pair_val,
                                                     const uint32_t* __restrict__ bmax, BinApply ap) {
  typedef typename FVec<F>::T V;
  extern __shared__ unsigned long long acc[];
  const int j = blockIdx.x;  // bucket, relative to the group
  int li = 0;
  while (li + 1 < grp.n_levels && j >= grp.bucket_rel[li + 1]) ++li;
  const int l = grp.level0 + li;
  const int be = 1 << grp.log2_be;
  const uint32_t entry_lo = (uint32_t)(j - grp.bucket_rel[li]) << grp.log2_be;
  const uint32_t level_T = c.mask[l] + 1u;
  const int count = (int)((level_T - entry_lo) < (uint32_t)be ? (level_T - entry_lo) : (uint32_t)be);
  const int tid = threadIdx.x;
  for (int e = tid; e < count * F; e += 1024) acc[e] = 0ull;
  __syncthreads();
  const uint32_t start = off[(int64_t)j * grp.nblk];
  const uint32_t end = off[(int64_t)(j + 1) * grp.nblk];
  // fixed-point scale 2^k with (pairs + 1) * max|v| * 2^k < 2^62: no partial sum can overflow
  const float mx = __uint_as_float(bmax[j]);
  int k = 0;
  if (mx > 0.0f) {
    int e_mx, e_n;
    frexpf(mx, &e_mx);                       // mx < 2^e_mx
    frexp((double)(end - start) + 1.0, &e_n);  // pairs + 1 <= 2^e_n
    k = 62 - e_mx - e_n;
  }
  const double scale = ldexp(1.0, k);
  const V* vals = reinterpret_cast<const V*>(pair_val);
  auto q = [&](float v) -> unsigned long long { return (unsigned long long)__double2ll_rn((double)v * scale); };
  auto add1 = [&](uint32_t i) {
    const uint32_t e = pair_idx[i];
    float v[F];
    FVec<F>::unpack(vals[i], v);
#pragma unroll
    for (int f = 0; f < F; ++f) atomicAdd(&acc[e * F + f], q(v[f]));
  };
  if (mx > 0.0f) {
    if constexpr (F == 2) {
      // two pairs per 16-byte load; a block step covers 4 rows of 2048 pairs and every thread issues its
      // 8 loads before its 16 LDS adds (each wave load reads 1 KiB / 256 B of contiguous memory)
      const uint32_t even0 = (start + 1u) & ~1u;
      if (start < even0 && start < end && tid == 0) add1(start);
      uint32_t i = even0;
      for (; i + 8192u <= end; i += 8192u) {
        uint32_t e2[4];
        float4 v4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t kk = i + (uint32_t)r * 2048u + 2u * (uint32_t)tid;
          e2[r] = *reinterpret_cast<const uint32_t*>(pair_idx + kk);
          v4[r] = *reinterpret_cast<const float4*>(pair_val + 2 * (size_t)kk);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t ea = e2[r] & 0xFFFFu, eb = e2[r] >> 16;
          atomicAdd(&acc[2 * ea], q(v4[r].x));
          atomicAdd(&acc[2 * ea + 1], q(v4[r].y));
          atomicAdd(&acc[2 * eb], q(v4[r].z));
          atomicAdd(&acc[2 * eb + 1], q(v4[r].w));
        }
      }
      if (i < end) {
        for (uint32_t kk = i + 2u * (uint32_t)tid; kk + 1u < end; kk += 2048u) {
          const uint32_t e2 = *reinterpret_cast<const uint32_t*>(pair_idx + kk);
          const float4 v = *reinterpret_cast<const float4*>(pair_val + 2 * (size_t)kk);
          atomicAdd(&acc[2 * (e2 & 0xFFFFu)], q(v.x));
          atomicAdd(&acc[2 * (e2 & 0xFFFFu) + 1], q(v.y));
          atomicAdd(&acc[2 * (e2 >> 16)], q(v.z));
          atomicAdd(&acc[2 * (e2 >> 16) + 1], q(v.w));
        }
        if (((end - i) & 1u) && tid == 0) add1(end - 1u);
      }
    } else {
      for (uint32_t i = start + tid; i < end; i += 1024) add1(i);
    }
  }
  __syncthreads();
  const double inv = ldexp(1.0, -k);
  const int64_t base = ((int64_t)c.offset[l] + entry_lo) * F;
  for (int e = tid; e < count * F; e += 1024) {
    const int64_t gi = base + e;
    const float gsum = (float)((double)(long long)acc[e] * inv);
    if (MODE == BIN_GRAD || MODE == BIN_SGD) {
      ap.dst[gi] += gsum;
    } else {
      if (ap.g_tap) ap.g_tap[gi] = gsum;
      float pp = ap.dst[gi], mm = ap.m[gi], vv = ap.v[gi];
      float mi = fmaf(1.0f - ap.beta1, gsum, ap.beta1 * mm);
      float vi = fmaf(1.0f - ap.beta2, gsum * gsum, ap.beta2 * vv);
      pp = pp - ap.lr_t * (mi / (sqrtf(vi) + ap.eps));
      ap.dst[gi] = pp;
      ap.m[gi] = mi;
      ap.v[gi] = vi;
    }
  }
}

// ---------------------------------------------------------------------------
// exclusive scan of n uint32 (n + 1 outputs: the last one is the total)

// in has n_in elements; out gets n elements (n >= n_in; the missing inputs count as 0)
__global__ __launch_bounds__(1024) void k_scan_tiles(const uint32_t* __restrict__ in, int64_t n_in,
                                                     uint32_t* __restrict__ out, int64_t n,
                                                     uint32_t* __restrict__ tile_sums) {
  __shared__ uint32_t wsum[16];
  const int64_t base = (int64_t)blockIdx.x * 4096;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  uint32_t v[4], s = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t i = base + tid * 4 + q;
    v[q] = i < n_in ? in[i] : 0u;
    s += v[q];
  }
  uint32_t incl = s;
  for (int d = 1; d < 64; d <<= 1) {
    uint32_t o = __shfl_up(incl, d);
    if (lane >= d) incl += o;
  }
  if (lane == 63) wsum[wv] = incl;
  __syncthreads();
  uint32_t wpre = 0;
  for (int k = 0; k < wv; ++k) wpre += wsum[k];
  uint32_t run = wpre + incl - s;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t i = base + tid * 4 + q;
    if (i < n) out[i] = run;
    run += v[q];
  }
  if (tid == 1023) tile_sums[blockIdx.x] = wpre + incl;
}

__global__ __launch_bounds__(1024) void k_scan_sums(uint32_t* __restrict__ sums, int64_t n_tiles,
                                                    uint32_t* __restrict__ total_out) {
  __shared__ uint32_t wsum[16];
  __shared__ uint32_t carry;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (tid == 0) carry = 0;
  __syncthreads();
  for (int64_t c0 = 0; c0 < n_tiles; c0 += 1024) {
    const int64_t i = c0 + tid;
    const uint32_t s = i < n_tiles ? sums[i] : 0u;
    uint32_t incl = s;
    for (int d = 1; d < 64; d <<= 1) {
      uint32_t o = __shfl_up(incl, d);
      if (lane >= d) incl += o;
    }
    if (lane == 63) wsum[wv] = incl;
    __syncthreads();
    uint32_t wpre = 0;
    for (int k = 0; k < wv; ++k) wpre += wsum[k];
    const uint32_t cbase = carry;
    if (i < n_tiles) sums[i] = cbase + wpre + incl - s;
    __syncthreads();
    if (tid == 1023) carry = cbase + wpre + incl;
    __syncthreads();
  }
  if (tid == 0) *total_out = carry;
}

__global__ __launch_bounds__(1024) void k_scan_add(uint32_t* __restrict__ out, int64_t n,
                                                   const uint32_t* __restrict__ tile_pre) {
  const int64_t base = (int64_t)blockIdx.x * 4096;
  const uint32_t add = tile_pre[blockIdx.x];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t i = base + threadIdx.x * 4 + q;
    if (i < n) out[i] += add;
  }
}

// ---------------------------------------------------------------------------
// launchers

// exclusive scan of in[0..n) into out[0..n]; out[n] and *total get the sum; sums has (n + 4096) / 4096 slots
hipError_t launch_scan_u32(const uint32_t* in, int64_t n, uint32_t* out, uint32_t* sums, uint32_t* total,
                           hipStream_t st) {
  const int64_t tiles = (n + 1 + 4095) / 4096;
  hipLaunchKernelGGL(k_scan_tiles, dim3((unsigned)tiles), dim3(1024), 0, st, in, n, out, n + 1, sums);
  hipLaunchKernelGGL(k_scan_sums, dim3(1), dim3(1024), 0, st, sums, tiles, total);
  hipLaunchKernelGGL(k_scan_add, dim3((unsigned)tiles), dim3(1024), 0, st, out, n + 1, sums);
  return hipGetLastError();
}

hipError_t launch_hash_fwd(const DevCfg& c, const PosSrc& src, int64_t n, const float* table, float* a0,
                           const FeatLayout& lay, uint32_t* idx_out, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const dim3 grid((unsigned)((n + 255) / 256), (unsigned)c.L), block(256);
  switch (c.F) {
    case 1: hipLaunchKernelGGL(k_hash_fwd<1>, grid, block, 0, st, c, src, n, 0, table, a0, lay, idx_out); break;
    case 2: hipLaunchKernelGGL(k_hash_fwd<2>, grid, block, 0, st, c, src, n, 0, table, a0, lay, idx_out); break;
    case 4: hipLaunchKernelGGL(k_hash_fwd<4>, grid, block, 0, st, c, src, n, 0, table, a0, lay, idx_out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

BinPlan plan_bins(const DevCfg& c, int64_t n, size_t pair_budget_bytes) {
  BinPlan p{};
  // int64 LDS accumulator of one bucket: 2^log2_be * F * 8 bytes = 64 KiB
  p.log2_be = c.F == 4 ? 11 : (c.F == 2 ? 12 : 13);
  p.chunk = 4096;
  p.nblk = (int)((n + p.chunk - 1) / p.chunk);
  const int64_t per_level_pairs = n * 8;
  const int64_t pair_bytes = 2 + 4 * (int64_t)c.F;
  int lg = (int)(pair_budget_bytes / (size_t)(per_level_pairs * pair_bytes));
  // slot offsets are 32-bit: keep a group's pair count below 2^32
  const int lg32 = (int)((((int64_t)1 << 32) - 1) / per_level_pairs);
  if (lg > lg32) lg = lg32;
  if (lg < 1) lg = 1;
  if (lg > c.L) lg = c.L;
  p.levels_per_group = lg;
  int max_buckets = 0, max_nbl = 0;
  for (int g0 = 0; g0 < c.L; g0 += lg) {
    int nb = 0;
    for (int l = g0; l < g0 + lg && l < c.L; ++l) {
      const int nbl = (int)(((int64_t)c.mask[l] + 1 + (1 << p.log2_be) - 1) >> p.log2_be);
      nb += nbl;
      if (nbl > max_nbl) max_nbl = nbl;
    }
    if (nb > max_buckets) max_buckets = nb;
  }
  p.max_buckets = max_buckets;
  p.max_nbl = max_nbl;
  p.max_pairs = per_level_pairs * lg;
  p.cnt_elems = (int64_t)max_buckets * p.nblk + 1;
  p.tiles = (p.cnt_elems + 4095) / 4096;
  return p;
}

hipError_t launch_hash_bwd(const DevCfg& c, const PosSrc& src, int64_t n, const float* g, const FeatLayout& lay,
                           int mode, float lr, const BinApply& ap, const BinPlan& plan, const BinScratch& s,
                           hipStream_t st) {
  if (n <= 0) return hipSuccess;
  for (int g0 = 0; g0 < c.L; g0 += plan.levels_per_group) {
    BinGroup grp{};
    grp.level0 = g0;
    grp.n_levels = (g0 + plan.levels_per_group <= c.L) ? plan.levels_per_group : c.L - g0;
    grp.log2_be = plan.log2_be;
    grp.chunk = plan.chunk;
    grp.nblk = plan.nblk;
    int rel = 0;
    for (int li = 0; li < grp.n_levels; ++li) {
      const int l = g0 + li;
      grp.nbl[li] = (int)(((int64_t)c.mask[l] + 1 + (1 << plan.log2_be) - 1) >> plan.log2_be);
      grp.bucket_rel[li] = rel;
      rel += grp.nbl[li];
    }
    grp.bucket_rel[grp.n_levels] = rel;
    const int n_buckets = rel;
    const int64_t n_cnt = (int64_t)n_buckets * plan.nblk;
    int max_nbl = 0;
    for (int li = 0; li < grp.n_levels; ++li) max_nbl = grp.nbl[li] > max_nbl ? grp.nbl[li] : max_nbl;
    const dim3 grid_bl((unsigned)plan.nblk, (unsigned)grp.n_levels);
    const size_t lds_hist = sizeof(uint32_t) * (size_t)max_nbl;
    const size_t lds_acc = sizeof(unsigned long long) * ((size_t)1 << plan.log2_be) * (size_t)c.F;
    const size_t lds_emit =
        sizeof(uint32_t) * ((4 * (size_t)max_nbl + 4 + 3) & ~(size_t)3) + 2048 * (4 + sizeof(float) * (size_t)c.F);
#define FFN_BIN(FV, MV)                                                                                             \
  do {                                                                                                              \
    hipLaunchKernelGGL((k_bin_count<FV, MV>), grid_bl, dim3(256), lds_hist, st, c, src, n, grp, g, lay, lr,       \
                       s.cnt, s.bmax);                                                                              \
    const int64_t tiles = (n_cnt + 1 + 4095) / 4096;                                                                \
    hipLaunchKernelGGL(k_scan_tiles, dim3((unsigned)tiles), dim3(1024), 0, st, s.cnt, n_cnt, s.off, n_cnt + 1,     \
                       s.sums);                                                                                     \
    hipLaunchKernelGGL(k_scan_sums, dim3(1), dim3(1024), 0, st, s.sums, tiles, s.total);                           \
    hipLaunchKernelGGL(k_scan_add, dim3((unsigned)tiles), dim3(1024), 0, st, s.off, n_cnt + 1, s.sums);            \
    hipLaunchKernelGGL((k_bin_emit<FV, MV>), grid_bl, dim3(256), lds_emit, st, c, src, n, grp, g, lay, lr, s.off, \
                       s.pair_idx, s.pair_val, s.bmax);                                                             \
    hipLaunchKernelGGL((k_bin_reduce<FV, MV>), dim3((unsigned)n_buckets), dim3(1024), lds_acc, st, c, grp, s.off, \
                       s.pair_idx, s.pair_val, s.bmax, ap);                                                         \
  } while (0)
#define FFN_BIN_F(MV)                  \
  switch (c.F) {                       \
    case 1: FFN_BIN(1, MV); break;     \
    case 2: FFN_BIN(2, MV); break;     \
    case 4: FFN_BIN(4, MV); break;     \
    default: return hipErrorInvalidValue; \
  }
    // the scan writes n_cnt + 1 offsets: the last one is the group's pair total
    if (mode == BIN_GRAD) {
      FFN_BIN_F(BIN_GRAD)
    } else if (mode == BIN_SGD) {
      FFN_BIN_F(BIN_SGD)
    } else {
      FFN_BIN_F(BIN_ADAM)
    }
#undef FFN_BIN_F
#undef FFN_BIN
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// level-major [L][N][F] <-> sample-major [N][L*F] copies (for taps)
__global__ __launch_bounds__(256) void k_feat_relayout(const float* __restrict__ src, FeatLayout ls,
                                                       float* __restrict__ dst, FeatLayout ld, int64_t n, int L,
                                                       int F) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= n) return;
  for (int l = 0; l < L; ++l)
    for (int f = 0; f < F; ++f) dst[l * ld.stride_l + b * ld.stride_b + f] = src[l * ls.stride_l + b * ls.stride_b + f];
}

hipError_t launch_feat_relayout(const float* src, const FeatLayout& ls, float* dst, const FeatLayout& ld, int64_t n,
                                int L, int F, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_feat_relayout, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, src, ls, dst, ld, n, L,
                     F);
  return hipGetLastError();
}

}  // namespace ffn
