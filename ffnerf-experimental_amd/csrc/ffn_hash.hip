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
//     1. emit      -- per (level, sample chunk), rounds of 1024 samples (512
//                     at F = 4): each
//                     round ranks its (entry-in-bucket, value) pairs by bucket
//                     (BE consecutive table entries of one level) with an LDS
//                     counting sort and writes them contiguously into its own
//                     slots, plus a run table (offset, length per bucket);
//                     consecutive samples in the same cell of the level are
//                     merged first, one pair per corner for the whole run;
//     2. transpose -- the run table turned bucket-major;
//     3. reduce    -- one block per bucket sums its runs from every round into
//                     an LDS copy of the bucket and applies the update to its
//                     own slice of the table: gradient add, the reference SGD,
//                     or Adam.  No gradient table is materialised for Adam.
//   LDS float atomics (ds_add_f32) sustain only ~0.33 lanes/clk/CU here while
//   ds_add_u64 sustains ~4.9 (both measured), so the reduce accumulates in
//   64-bit fixed point: the emit records a bound on every |value| of a chunk
//   (the largest it wrote), the reduce takes the largest over the level's
//   chunks and scales by the power of two that keeps a bucket's total below
//   2^62 -- an exact scaling, one round-to-nearest per pair, ~2^-40 of the
//   level's largest value per entry at the benchmark shape.
//   Pair stores went through the L2 as 2-byte and 8-byte scattered writes and
//   stalled the address/data path (measured: write data stalled by the cache),
//   so every bucket run of an emit round is padded with zero pairs to a
//   multiple of 8 and the pairs move in 16-byte aligned blocks of 8 (values,
//   then entries), one block per lane.
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

// F features of a binary16 table entry: one 2-, 4- or 8-byte load, widened exactly to fp32
template <int F>
struct HVec;
template <>
struct HVec<1> {
  typedef _Float16 T;
  static __device__ __forceinline__ void unpack(const T& v, float* o) { o[0] = (float)v; }
};
template <>
struct HVec<2> {
  typedef _Float16 T __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ void unpack(const T& v, float* o) {
    o[0] = (float)v.x;
    o[1] = (float)v.y;
  }
};
template <>
struct HVec<4> {
  typedef _Float16 T __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ void unpack(const T& v, float* o) {
    o[0] = (float)v.x;
    o[1] = (float)v.y;
    o[2] = (float)v.z;
    o[3] = (float)v.w;
  }
};
template <int F, typename TT>
struct TabVec {
  typedef FVec<F> V;
};
template <int F>
struct TabVec<F, _Float16> {
  typedef HVec<F> V;
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

// Dense copies of the coarse levels.  A level whose R^3 vertices are few gets its vertex values copied
// out of the hash table before the gather, in vertex order: the 64 samples of a wavefront, one ray, walk
// through neighbouring cells, so a load instruction touches a few lines instead of 64 random ones, and no
// corner is hashed.  Small copies are row-major ([z][y][x]: the eight corners of a cell are four pairs of
// x-neighbours, each pair one load where it fits 16 bytes); larger ones (bricked) are stored in 4x4x4
// bricks of 64 vertices, [brick z][y][x][z & 3][y & 3][x & 3], so that the corners of a cell and the cells
// a ray crosses share lines in every direction, not only along x.  The values are the table's, so the
// gather is unchanged bit for bit.
template <int F, typename TT>
__global__ __launch_bounds__(256) void k_hash_densify(DevCfg c, const TT* __restrict__ table, DenseLevels dl) {
  const int l = (int)blockIdx.y;
  if (dl.off[l] == DENSE_NONE) return;
  const uint32_t R = (uint32_t)c.res[l];
  const bool brick = (dl.bricked >> l) & 1u;
  const uint32_t NB = (R + 3) / 4;
  const uint32_t cells = brick ? NB * NB * NB * 64 : R * R * R;
  TT* __restrict__ grid = static_cast<TT*>(dl.grid) + (size_t)dl.off[l] * F;
  const uint32_t base = c.offset[l], mask = c.mask[l];
  for (uint32_t v = blockIdx.x * blockDim.x + threadIdx.x; v < cells; v += gridDim.x * blockDim.x) {
    uint32_t x, y, z;
    if (brick) {
      const uint32_t b = v >> 6, i = v & 63;
      x = (b % NB) * 4 + (i & 3);
      y = ((b / NB) % NB) * 4 + ((i >> 2) & 3);
      z = (b / (NB * NB)) * 4 + (i >> 4);
    } else {
      x = v % R;
      y = (v / R) % R;
      z = v / (R * R);
    }
    if (x < R && y < R && z < R) {
      const uint32_t e = (base + level_entry(x, y, z, l, mask)) * (uint32_t)F;
#pragma unroll
      for (int f = 0; f < F; ++f) grid[(size_t)v * F + f] = table[e + f];
    }
  }
}

// the x-neighbour pair of a dense row: one 8- or 16-byte load where the pair has that size
template <int F, typename TT>
__device__ __forceinline__ void load_xpair(const TT* p, typename TabVec<F, TT>::V::T& a,
                                           typename TabVec<F, TT>::V::T& b) {
  typedef typename TabVec<F, TT>::V::T V;
  constexpr int BYTES = 2 * F * (int)sizeof(TT);
  if constexpr (BYTES == 8 || BYTES == 16) {
    typedef unsigned int W __attribute__((ext_vector_type(BYTES / 4), aligned(BYTES / 2)));
    struct Pair {
      V a, b;
    };
    static_assert(sizeof(Pair) == BYTES, "two entries, no padding");
    const Pair pr = __builtin_bit_cast(Pair, *reinterpret_cast<const W*>(p));
    a = pr.a;
    b = pr.b;
  } else {
    a = *reinterpret_cast<const V*>(p);
    b = *reinterpret_cast<const V*>(p + F);
  }
}

// one sample at one level: the eight corners (from the dense copy or through the hash), the trilinear sum,
// the store of the encoding (and of the corner indices when idx_out is given)
template <int F, typename TT>
__device__ __forceinline__ void gather_level(const DevCfg& c, const float (&p)[3], int l, const TT* __restrict__ table,
                                             const DenseLevels& dl, int64_t b, float* __restrict__ a0,
                                             const FeatLayout& lay, uint32_t* __restrict__ idx_out) {
  typedef typename TabVec<F, TT>::V TV;
  typedef typename TV::T V;
  const LevelCell lc = level_cell(c.res[l], p);
  const uint32_t mask = c.mask[l], off = c.offset[l];
  uint32_t fb[8];
  V val[8];
  if (dl.off[l] != DENSE_NONE && ((dl.bricked >> l) & 1u)) {
    const uint32_t NB = ((uint32_t)c.res[l] + 3) / 4;
    uint32_t X[2], Y[2], Z[2];
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const uint32_t cx = (uint32_t)lc.i0[0] + d, cy = (uint32_t)lc.i0[1] + d, cz = (uint32_t)lc.i0[2] + d;
      X[d] = (cx >> 2) * 64 + (cx & 3);
      Y[d] = (cy >> 2) * (NB * 64) + (cy & 3) * 4;
      Z[d] = (cz >> 2) * (NB * NB * 64) + (cz & 3) * 16;
    }
    const TT* g = static_cast<const TT*>(dl.grid) + (size_t)dl.off[l] * F;
#pragma unroll
    for (int cc = 0; cc < 8; ++cc)
      val[cc] = *reinterpret_cast<const V*>(g + (size_t)(X[cc & 1] + Y[(cc >> 1) & 1] + Z[cc >> 2]) * F);
    if (idx_out) {
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) fb[cc] = (off + corner_entry(lc, cc, l, mask)) * (uint32_t)F;
    }
  } else if (dl.off[l] != DENSE_NONE) {  // the same for the whole block
    const size_t R = (size_t)c.res[l];
    const TT* g = static_cast<const TT*>(dl.grid) +
                  ((size_t)dl.off[l] + ((size_t)lc.i0[2] * R + (size_t)lc.i0[1]) * R + (size_t)lc.i0[0]) * F;
#pragma unroll
    for (int q = 0; q < 4; ++q)  // corners 2q (dx = 0) and 2q + 1 (dx = 1) of row dy = q & 1, dz = q >> 1
      load_xpair<F, TT>(g + ((size_t)(q >> 1) * R * R + (size_t)(q & 1) * R) * F, val[2 * q], val[2 * q + 1]);
    if (idx_out) {
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) fb[cc] = (off + corner_entry(lc, cc, l, mask)) * (uint32_t)F;
    }
  } else {
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      fb[cc] = (off + corner_entry(lc, cc, l, mask)) * (uint32_t)F;
      val[cc] = *reinterpret_cast<const V*>(table + fb[cc]);
    }
  }
  float acc[F];
#pragma unroll
  for (int f = 0; f < F; ++f) acc[f] = 0.0f;
#pragma unroll
  for (int cc = 0; cc < 8; ++cc) {
    const float w = corner_weight(lc, cc);
    float t[F];
    TV::unpack(val[cc], t);
#pragma unroll
    for (int f = 0; f < F; ++f) acc[f] += w * t[f];
  }
  // a streaming store: the encodings are read by the next pass, while this one gathers from the level's
  // table in the L2 (3 % faster than a plain store at the benchmark shape)
  store_stream(reinterpret_cast<typename FVec<F>::T*>(a0 + l * lay.stride_l + b * lay.stride_b),
               FVec<F>::pack(acc));
  if (idx_out) {
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) idx_out[(b * c.L + l) * 8 + cc] = fb[cc];
  }
}

// the grid row's level(s) of sample b
template <int F, typename TT>
__device__ __forceinline__ void gather_row(const DevCfg& c, const PosSrc& src, int64_t b, const TT* __restrict__ table,
                                           float* __restrict__ a0, const FeatLayout& lay,
                                           uint32_t* __restrict__ idx_out, const DenseLevels& dl) {
  float pos[3], p[3];
  sample_position(src, b, pos);
  normalize_pos(c, pos, p);
  const int row = (int)blockIdx.y;
  if (dl.n_multi > 0 && row == 0) {
#pragma unroll 1
    for (int l = 0; l < dl.n_multi; ++l) gather_level<F, TT>(c, p, l, table, dl, b, a0, lay, idx_out);
  } else {
    gather_level<F, TT>(c, p, row + (dl.n_multi > 0 ? dl.n_multi - 1 : 0), table, dl, b, a0, lay, idx_out);
  }
}

// Grid row y gathers level y + (n_multi - 1) for one sample per thread; with n_multi > 0, row 0 gathers the
// n_multi coarsest levels (small dense copies, together a working set of a few MB) in one pass, so their
// sample positions are read and computed once.  DEV: the count min(n, *n_dev) is read on the device and the
// threads walk it with the grid's stride (a grid sized for a capacity n whose use is known only there).
template <int F, typename TT, bool DEV>
__global__ __launch_bounds__(256) void k_hash_fwd(DevCfg c, PosSrc src, int64_t n, const TT* __restrict__ table,
                                                  float* __restrict__ a0, FeatLayout lay,
                                                  uint32_t* __restrict__ idx_out, DenseLevels dl,
                                                  const uint32_t* __restrict__ n_dev) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if constexpr (DEV) {
    const int64_t nd = (int64_t)*n_dev, nn = nd < n ? nd : n;
    for (int64_t bb = b; bb < nn; bb += (int64_t)gridDim.x * blockDim.x)
      gather_row<F, TT>(c, src, bb, table, a0, lay, idx_out, dl);
  } else {
    if (b >= n) return;
    gather_row<F, TT>(c, src, b, table, a0, lay, idx_out, dl);
  }
}

// ---------------------------------------------------------------------------
// backward: bucketed scatter

// The raw inputs of one (sample, level) of the scatter: its upstream gradient and what its position is
// made of.  Loaded one emit/count round ahead of their use, so the loads' latency overlaps the round.
template <int F>
struct RawSample {
  float g[F];
  float4 o, d;  // ray origin / direction, or the stored position in o.xyz
  float t;
};

template <int F>
__device__ __forceinline__ void load_raw(const PosSrc& s, const float* __restrict__ g, const FeatLayout& lay,
                                         int64_t b, int l, RawSample<F>& r) {
  typedef typename FVec<F>::T V;
  {
    // each level's gradients are read by this pass once: streamed past the caches
    const float* gp = g + l * lay.stride_l + b * lay.stride_b;
    if constexpr (F == 1) {
      r.g[0] = __builtin_nontemporal_load(gp);
    } else {
      typedef float fv __attribute__((ext_vector_type(F)));
      const fv v = __builtin_nontemporal_load(reinterpret_cast<const fv*>(gp));
#pragma unroll
      for (int f = 0; f < F; ++f) r.g[f] = v[f];
    }
  }
  if (s.rays) {
    const int64_t ray = b >> s.log2S;
    r.o = s.rays[2 * ray];
    r.d = s.rays[2 * ray + 1];
    r.t = s.Ts[b];
  } else {
    const float* xb = s.x + (int64_t)s.x_stride * b;
    r.o = make_float4(xb[0], xb[1], xb[2], 0.0f);
  }
}

// the sample position, computed exactly as sample_position does
template <int F>
__device__ __forceinline__ void raw_position(const PosSrc& s, const RawSample<F>& r, float pos[3]) {
  if (s.rays) {
    pos[0] = r.o.x + r.t * r.d.x;
    pos[1] = r.o.y + r.t * r.d.y;
    pos[2] = r.o.z + r.t * r.d.z;
  } else {
    pos[0] = r.o.x;
    pos[1] = r.o.y;
    pos[2] = r.o.z;
  }
}

// The gradient of one (sample, level): scaled as the mode needs, non-finite
// components dropped (ffnerf_OG.cl:2162).  Returns false when it is all zero.
template <int F, int MODE>
__device__ __forceinline__ bool level_grad(const DevCfg& c, const float (&v)[F], int l, float lr, float gf[F]) {
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

// One step of the emit's segmented suffix sum: lane i adds lane i + D's values when both are in its run
// (take).  Runs lie inside aligned groups of at most 16 lanes, so lane i + D is in the same 16-lane row and
// the DPP row shift reaches it.
template <int D, int F>
__device__ __forceinline__ void merge_step(float (&v)[8][F], bool take) {
  static_assert(D < 16, "a row shift");
#pragma unroll
  for (int cc = 0; cc < 8; ++cc)
#pragma unroll
    for (int f = 0; f < F; ++f) {
      // row_shl:D, zero past the row's end: the read folds into the add as a DPP operand
      const float u = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[cc][f]), 0x100 + D, 0xF, 0xF, true));
      const float t = v[cc][f] + u;
      v[cc][f] = take ? t : v[cc][f];
    }
}

// Emit rounds: one sample per thread, emit_nt(F) samples per round (the stage of a round's pairs must fit
// in LDS at 2 + 4F bytes per pair), and every bucket's run of a round is padded with zero pairs to a
// multiple of PAD_RUN.  The pair buffer is a sequence of blocks of PAD_RUN pairs, each 16-byte aligned:
// the block's 8F values, then its 8 entries (pair_block_words(F) 16-byte words), so a run is one
// contiguous range for the reduction (with entries and values in separate arrays, a run of a few dozen
// pairs was two short ranges whose edge sectors were fetched twice).
// Same-cell samples merge within aligned groups of MERGE_BLK lanes (a run never crosses one), which keeps
// the merge to log2(MERGE_BLK) register steps inside a 16-lane DPP row; longer groups would merge little
// more (at the benchmark shape 73 % of the pairs remain with unbounded runs, 76 % with groups of 8; groups
// of 16 took the scatter from 7.23 to 7.19 ms).
constexpr int PAD_RUN = 8;
__host__ __device__ constexpr int pair_block_words(int F) { return 2 * F + 1; }
constexpr int MERGE_BLK = 16;
__host__ __device__ constexpr int emit_nt(int F) { return F >= 4 ? 512 : 1024; }
__device__ __forceinline__ uint32_t pad_run(uint32_t n) { return (n + (PAD_RUN - 1)) & ~(uint32_t)(PAD_RUN - 1); }

// LDS of k_bin_emit: counters, run offsets, the round totals and wavefront maxima (32-bit words), then the
// stage: values [np][F] and entries [np]
__host__ __device__ constexpr int emit_words(int nbl, int F) { return (3 * nbl + 4 + emit_nt(F) / 64 + 3) & ~3; }
__host__ __device__ constexpr int emit_stage_pairs(int nbl, int F) {
  return 8 * emit_nt(F) + (PAD_RUN - 1) * (nbl < 8 * emit_nt(F) ? nbl : 8 * emit_nt(F));
}
__host__ __device__ constexpr int round8(int x) { return (x + 7) & ~7; }
__host__ __device__ constexpr size_t emit_lds_bytes(int nbl, int F) {
  return (size_t)emit_words(nbl, F) * 4 + (size_t)round8(emit_stage_pairs(nbl, F)) * (2 + 4 * (size_t)F);
}

// Inclusive sum over the 64 lanes: DPP row shifts within 16-lane rows, then row broadcasts of lanes 15
// and 31 into the rows above (all VALU).
__device__ __forceinline__ uint32_t wave_incl_sum(uint32_t x) {
  int v = (int)x;
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1 and 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2 and 3
  return (uint32_t)v;
}

// One sample of an emit round, ready to rank: its cell at the level and, at a run's head, the run's eight
// corner sums.
template <int F>
struct EmitSample {
  bool head;
  int i0[3];
  float v[8][F];
};

// Form a sample's corner values g_f * w_corner and merge same-cell runs: a sample in the same cell as the
// previous lane's (within its group of MERGE_BLK lanes) continues that lane's run; a segmented suffix sum
// over the lanes (DPP row shifts by 1, 2, 4, a step taken only when some run of the wavefront is longer
// than its stride) leaves each run's first lane, its head, with the run's sums.  The additions follow a
// fixed tree, so the values are deterministic.
template <int F, int MODE>
__device__ __forceinline__ void emit_prepare(const DevCfg& c, const PosSrc& src, const RawSample<F>& in, bool valid,
                                             int l, float lr, int lane, EmitSample<F>& es) {
  float gf[F];
  const bool act = valid && level_grad<F, MODE>(c, in.g, l, lr, gf);
  LevelCell lc;
  lc.i0[0] = lc.i0[1] = lc.i0[2] = -1;
  if (act) {
    float pos[3], p[3];
    raw_position<F>(src, in, pos);
    normalize_pos(c, pos, p);
    lc = level_cell(c.res[l], p);
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      const float w = corner_weight(lc, cc);
#pragma unroll
      for (int f = 0; f < F; ++f) es.v[cc][f] = gf[f] * w;
    }
  } else {
#pragma unroll
    for (int cc = 0; cc < 8; ++cc)
#pragma unroll
      for (int f = 0; f < F; ++f) es.v[cc][f] = 0.0f;
  }
  // the previous lane's cell by DPP row_shr:1 (a run never starts a 16-lane row's first lane, which gets -1)
  const int p0 = __builtin_amdgcn_update_dpp(-1, lc.i0[0], 0x111, 0xF, 0xF, false);
  const int p1 = __builtin_amdgcn_update_dpp(-1, lc.i0[1], 0x111, 0xF, 0xF, false);
  const int p2 = __builtin_amdgcn_update_dpp(-1, lc.i0[2], 0x111, 0xF, 0xF, false);
  const bool cont = act && (lane & (MERGE_BLK - 1)) != 0 && p0 == lc.i0[0] && p1 == lc.i0[1] && p2 == lc.i0[2];
  const uint64_t cm = __ballot(cont);
  if (cm != 0ull) {
    // lanes from this one to its run's end (the next lane that continues nothing); at most MERGE_BLK
    const uint64_t starts_above = lane == 63 ? 0ull : (~cm >> (lane + 1));
    const int len = starts_above == 0ull ? 64 - lane : 1 + (int)__builtin_ctzll(starts_above);
    merge_step<1, F>(es.v, len > 1);
    if (__ballot(len > 2) != 0ull) {
      merge_step<2, F>(es.v, len > 2);
      if (__ballot(len > 4) != 0ull) {
        merge_step<4, F>(es.v, len > 4);
        if (__ballot(len > 8) != 0ull) merge_step<8, F>(es.v, len > 8);
      }
    }
  }
  es.head = act && !cont;
  es.i0[0] = lc.i0[0];
  es.i0[1] = lc.i0[1];
  es.i0[2] = lc.i0[2];
}

// Emit the (entry, value) pairs of emit_nt(F) samples at a time.  Only run heads (emit_prepare) rank and
// stage pairs: along a ray the coarse levels hold many samples per cell (at the benchmark shape the pairs
// fall to ~76 % over the 16 levels, to ~30 % at the coarsest).  A round ranks the heads' pairs by bucket
// in LDS (a local counting sort into runs padded to PAD_RUN with zero pairs), stages them (entry in
// bucket, values), and writes the stage contiguously into the round's own slots (np pairs per round),
// plus its row of the run table (each bucket's run offset and length in the slots).  Every write of the
// pass is so a sequential stream, and no counting pass or global offsets are needed; the reduction reads
// each bucket's runs from all rounds.
// Order within a round: prepare the round's samples; issue the next round's loads; rank; barrier; copy
// out the previous round's stage (complete since that barrier) while wavefront 0 scans the counts (stage
// offsets, the run-table row straight to memory, the other counter buffer cleared for the next round);
// barrier; stage the pairs.  Two barriers a round: the copy-out fills the time the other wavefronts
// waited for the scan, and the next round's first barrier orders the stage before its copy-out (with a
// third barrier before an in-round copy-out the pass took 7.55 instead of 7.28 ms with its reduce).  The
// wavefronts spend most of their time waiting (barriers, LDS returns); with a 1024-thread block that
// needs 87 KB of LDS, one block per CU gives four wavefronts per SIMD.  Measured slower at the benchmark
// shape: preparing the next round's samples before the copy-out (6.2 against 5.5 ms), and splitting the
// wavefronts into loaders that never store and writers that never load (7.3 ms: the loaders' ALU work
// per wavefront doubles).  The block also writes
// cmax[level in group][chunk], a bound on every |value| of its pairs: the largest it staged.
// Write one round's stage (total padded pairs) as a sequence of 16-byte words, lane t on word t: every
// store instruction writes 1 KB contiguously (a lane per block would store at the block stride)
template <int F>
__device__ __forceinline__ void copy_out_round(uint4* __restrict__ pbuf, const BinGroup& grp, int li, int64_t round,
                                               const float* st_val, const uint16_t* st_idx, uint32_t total,
                                               int tid) {
  constexpr int NT = emit_nt(F);
  constexpr uint32_t W = pair_block_words(F);
  const uint32_t nw = min(total, (uint32_t)grp.np) / PAD_RUN * W;  // the round's slots bound the copy
  uint4* dst = pbuf + ((int64_t)li * grp.n_rounds + round) * (grp.np / PAD_RUN) * W;
  for (uint32_t w = (uint32_t)tid; w < nw; w += NT) {
    const uint32_t blk = w / W, k = w - blk * W;
    const uint4 v = k < 2 * F ? reinterpret_cast<const uint4*>(st_val)[blk * 2 * F + k]
                              : reinterpret_cast<const uint4*>(st_idx)[blk];
    // streamed past the caches: the reduce reads the pairs back only after the whole pass (13 GB at the
    // benchmark shape, far beyond the L2 and the MALL): scatter 6.87 -> 6.83 ms
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(u4{v.x, v.y, v.z, v.w}, reinterpret_cast<u4*>(dst + w));
  }
}

// n_dev (may be NULL): the sample count is min(n, *n_dev); a block past it writes only its zero bound, and
// the rounds past it are not read (k_bin_meta_transpose, k_bin_reduce bound them by the same count)
template <int F, int MODE>
__global__ __launch_bounds__(emit_nt(F)) void k_bin_emit(DevCfg c, PosSrc src, int64_t n, BinGroup grp,
                                                         const float* __restrict__ g, FeatLayout lay, float lr,
                                                         uint32_t* __restrict__ meta, float* __restrict__ cmax,
                                                         uint4* __restrict__ pbuf, const uint32_t* __restrict__ n_dev) {
  typedef typename FVec<F>::T V;
  constexpr int NT = emit_nt(F);
  extern __shared__ uint32_t sm[];
  const int li = (int)blockIdx.y, l = grp.level0 + li;
  const int nbl = grp.nbl[li];
  const int chunk = blockIdx.x;
  uint32_t* lcnt = sm;              // [2][nbl] pairs of the round per bucket
  uint32_t* loff = lcnt + 2 * nbl;  // [nbl] run offsets in the stage
  uint32_t* total_s = loff + nbl;   // [2] padded pairs of the round, by round parity
  float* wmax = reinterpret_cast<float*>(total_s + 4);                          // [NT / 64]
  float* st_val = reinterpret_cast<float*>(sm + emit_words(nbl, F));            // [np][F]
  uint16_t* st_idx = reinterpret_cast<uint16_t*>(st_val + (size_t)grp.np * F);  // [np]
  const int tid = threadIdx.x, lane = tid & 63;
  for (int j = tid; j < nbl; j += NT) lcnt[j] = 0u;
  const uint32_t be_mask = (1u << grp.log2_be) - 1u;
  if (n_dev) {
    const int64_t nd = (int64_t)*n_dev;
    n = nd < n ? nd : n;
  }
  const int64_t b_begin = (int64_t)chunk * grp.chunk;
  const int64_t b_end = b_begin + grp.chunk < n ? b_begin + grp.chunk : n;
  const int kb = (nbl + 63) >> 6;  // counters per lane in the scan
  RawSample<F> in;
  if (b_begin + tid < b_end) load_raw<F>(src, g, lay, b_begin + tid, l, in);
  __syncthreads();
  float bound = 0.0f;
  int r = 0;
  for (int64_t rb = b_begin; rb < b_end; rb += NT, r ^= 1) {
    const int64_t round = rb / NT;  // the round's index in the level
    uint32_t* cur = lcnt + r * nbl;
    uint32_t* nxt = lcnt + (r ^ 1) * nbl;
    EmitSample<F> es;
    emit_prepare<F, MODE>(c, src, in, rb + tid < b_end, l, lr, lane, es);
    if (rb + NT + tid < b_end) load_raw<F>(src, g, lay, rb + NT + tid, l, in);
    uint32_t ent[8], rank[8];
    if (es.head) {
      LevelCell lc;
      lc.i0[0] = es.i0[0];
      lc.i0[1] = es.i0[1];
      lc.i0[2] = es.i0[2];
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) {
#pragma unroll
        for (int f = 0; f < F; ++f) bound = fmaxf(bound, fabsf(es.v[cc][f]));
        ent[cc] = corner_entry(lc, cc, l, c.mask[l]);
        rank[cc] = atomicAdd(&cur[ent[cc] >> grp.log2_be], 1u);
      }
    }
    __syncthreads();
    // the previous round's stage, complete since the barrier above, goes out while wavefront 0 scans
    if (rb != b_begin) copy_out_round<F>(pbuf, grp, li, round - 1, st_val, st_idx, total_s[r ^ 1], tid);
    uint32_t* mrow = meta + ((int64_t)li * grp.n_rounds + round) * grp.meta_stride;
    if (tid < 64) {
      // lane t scans counters [t * kb, t * kb + kb); nbl is a power of two, so from 256 buckets on every
      // lane holds a multiple of 4 of them, read and written 16 bytes at a time
      const int j0 = lane * kb;
      uint32_t own = 0;
      if (j0 < nbl) {
        if (kb >= 4) {
          for (int k = 0; k < kb; k += 4) {
            const uint4 c4 = *reinterpret_cast<const uint4*>(cur + j0 + k);
            own += pad_run(c4.x) + pad_run(c4.y) + pad_run(c4.z) + pad_run(c4.w);
          }
        } else {
          for (int k = 0; k < kb; ++k) own += pad_run(cur[j0 + k]);
        }
      }
      const uint32_t incl = wave_incl_sum(own);
      uint32_t o = incl - own;
      if (j0 < nbl) {
        if (kb >= 4) {
          for (int k = 0; k < kb; k += 4) {
            const uint4 c4 = *reinterpret_cast<const uint4*>(cur + j0 + k);
            const uint32_t n0 = pad_run(c4.x), n1 = pad_run(c4.y), n2 = pad_run(c4.z), n3 = pad_run(c4.w);
            const uint4 of = make_uint4(o, o + n0, o + n0 + n1, o + n0 + n1 + n2);
            *reinterpret_cast<uint4*>(loff + j0 + k) = of;
            *reinterpret_cast<uint4*>(mrow + j0 + k) =
                make_uint4((of.x << 16) | n0, (of.y << 16) | n1, (of.z << 16) | n2, (of.w << 16) | n3);
            *reinterpret_cast<uint4*>(nxt + j0 + k) = make_uint4(0u, 0u, 0u, 0u);
            o = of.w + n3;
          }
        } else {
          for (int k = 0; k < kb; ++k) {
            const int j = j0 + k;
            const uint32_t cn = pad_run(cur[j]);
            loff[j] = o;
            mrow[j] = (o << 16) | cn;
            nxt[j] = 0u;
            o += cn;
          }
        }
      }
      if (lane == 63) total_s[r] = incl;
    }
    __syncthreads();
    if (es.head) {
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) {
        const uint32_t slot = loff[ent[cc] >> grp.log2_be] + rank[cc];
        st_idx[slot] = (uint16_t)(ent[cc] & be_mask);
        reinterpret_cast<V*>(st_val)[slot] = FVec<F>::pack(es.v[cc]);
      }
    }
    // zero pairs pad every run to a multiple of PAD_RUN
    for (int j = tid; j < nbl; j += NT) {
      const uint32_t c0 = cur[j], c1 = pad_run(c0), o = loff[j];
      for (uint32_t k = c0; k < c1; ++k) {
        st_idx[o + k] = 0;
        float z[F];
#pragma unroll
        for (int f = 0; f < F; ++f) z[f] = 0.0f;
        reinterpret_cast<V*>(st_val)[o + k] = FVec<F>::pack(z);
      }
    }
  }
  // the last round's stage
  __syncthreads();
  if (b_end > b_begin) copy_out_round<F>(pbuf, grp, li, (b_end - 1) / NT, st_val, st_idx, total_s[r ^ 1], tid);
  bound = wave_max_nonneg(bound);
  if (lane == 0) wmax[tid >> 6] = bound;
  __syncthreads();
  if (tid == 0) {
    float m = 0.0f;
    for (int w = 0; w < NT / 64; ++w) m = fmaxf(m, wmax[w]);
    cmax[(int64_t)li * grp.nblk + chunk] = m;
  }
}

// The run table as emit writes it, [level][round][bucket], turned bucket-major, [level][bucket][round],
// so that each reduce block reads its bucket's runs as one contiguous row (a strided column read costs a
// memory sector per round once the table outgrows the caches).  64x64 tiles through LDS.
// the rounds with samples (rounds_used: fewer when the count is read on the device)
__device__ __forceinline__ int rounds_used(int n_rounds, const uint32_t* n_dev, int nt) {
  if (!n_dev) return n_rounds;
  const int64_t r = ((int64_t)*n_dev + nt - 1) / nt;
  return r < n_rounds ? (int)r : n_rounds;
}

__global__ __launch_bounds__(256) void k_bin_meta_transpose(const uint32_t* __restrict__ meta,
                                                            uint32_t* __restrict__ meta_t, int n_rounds,
                                                            int stride, const uint32_t* __restrict__ n_dev,
                                                            int nt) {
  __shared__ uint32_t tile[64][65];
  const int r0 = blockIdx.x * 64, b0 = blockIdx.y * 64, li = blockIdx.z;
  if (r0 >= rounds_used(n_rounds, n_dev, nt)) return;  // the same for the whole block
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const uint32_t* src = meta + (int64_t)li * n_rounds * stride;
  uint32_t* dst = meta_t + (int64_t)li * stride * n_rounds;
  for (int i = ty; i < 64; i += 4) {
    const int r = r0 + i, bk = b0 + tx;
    tile[i][tx] = (r < n_rounds && bk < stride) ? src[(int64_t)r * stride + bk] : 0u;
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int bk = b0 + i, r = r0 + tx;
    if (bk < stride && r < n_rounds) dst[(int64_t)bk * n_rounds + r] = tile[tx][i];
  }
}

// One block per bucket: sum its pairs in 64-bit fixed point in LDS, then apply the mode's update to the
// bucket's slice of the table.  The bucket's pairs are one run in each round's slots (its row of the
// bucket-major run table gives offset and length); a first pass over the row counts them (for the
// fixed-point scale), the second walks SEG rounds per wavefront at a time with every lane on one block of 8
// pairs: 16 rounds (a block's run found by selects over the 16 running ends in scalars) or 64 (a binary
// search over the lanes' running ends).  Zero pairs (the run padding) are skipped.
template <int F, int MODE, int SEG>
__global__ __launch_bounds__(1024) void k_bin_reduce(DevCfg c, BinGroup grp, const uint32_t* __restrict__ meta,
                                                     const uint4* __restrict__ pbuf,
                                                     const float* __restrict__ cmax, BinApply ap,
                                                     const uint32_t* __restrict__ n_dev) {
  extern __shared__ unsigned long long acc[];
  __shared__ float wmax[16];
  __shared__ uint32_t wtot[16];
  // bucket, relative to the group, finest levels first: their buckets hold the most pairs, and the lighter
  // coarse-level blocks then fill the last wave of blocks (scatter 7.01 -> 6.91 ms at the benchmark shape)
  const int j = (int)gridDim.x - 1 - (int)blockIdx.x;
  int li = 0;
  while (li + 1 < grp.n_levels && j >= grp.bucket_rel[li + 1]) ++li;
  const int l = grp.level0 + li;
  const int jb = j - grp.bucket_rel[li];
  const int be = 1 << grp.log2_be;
  const uint32_t entry_lo = (uint32_t)jb << grp.log2_be;
  const uint32_t level_T = c.mask[l] + 1u;
  const int count = (int)((level_T - entry_lo) < (uint32_t)be ? (level_T - entry_lo) : (uint32_t)be);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nr = grp.n_rounds;
  const int nr_use = rounds_used(nr, n_dev, emit_nt(F));  // rounds with samples
  if (nr_use == 0) return;  // no samples: nothing is applied (the same for the whole block)
  for (int e = tid; e < count * F; e += 1024) acc[e] = 0ull;
  const uint32_t* mrow = meta + ((int64_t)li * grp.meta_stride + jb) * nr;  // bucket-major: round rr at mrow[rr]
  // bound on every |value| of the level (the largest of its chunks' bounds) and the bucket's pair count
  float mxl = 0.0f;
  for (int ch = tid; ch < grp.nblk; ch += 1024) mxl = fmaxf(mxl, cmax[(int64_t)li * grp.nblk + ch]);
  uint32_t cnt = 0;
  for (int rr = tid; rr < nr_use; rr += 1024) cnt += mrow[rr] & 0xFFFFu;
  mxl = wave_max_nonneg(mxl);
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) cnt += __shfl_xor(cnt, d);
  if (lane == 0) {
    wmax[wave] = mxl;
    wtot[wave] = cnt;
  }
  __syncthreads();
  float mx = 0.0f;
  uint32_t pairs = 0;
#pragma unroll
  for (int w = 0; w < 16; ++w) {
    mx = fmaxf(mx, wmax[w]);
    pairs += wtot[w];
  }
  // fixed-point scale 2^k with (pairs + 1) * bound * 2^k < 2^62: no partial sum can overflow
  int k = 0;
  if (mx > 0.0f) {
    int e_mx, e_n;
    frexpf(mx, &e_mx);                   // mx < 2^e_mx
    frexp((double)pairs + 1.0, &e_n);    // pairs + 1 <= 2^e_n
    k = 62 - e_mx - e_n;
  }
  const double scale = ldexp(1.0, k);
  auto add = [&](uint32_t e, float v, int f) {
    if (v != 0.0f) atomicAdd(&acc[e * F + f], (unsigned long long)__double2ll_rn((double)v * scale));
  };
  // one block of PAD_RUN pairs: PAD_RUN * F values, then the PAD_RUN entries
  auto add_block = [&](const uint4* src) {
    float v[PAD_RUN * F];
#pragma unroll
    for (int qq = 0; qq < 2 * F; ++qq) {
      const float4 t4 = *reinterpret_cast<const float4*>(src + qq);
      v[4 * qq] = t4.x;
      v[4 * qq + 1] = t4.y;
      v[4 * qq + 2] = t4.z;
      v[4 * qq + 3] = t4.w;
    }
    const uint4 e8 = src[2 * F];
    const uint32_t ev[PAD_RUN] = {e8.x & 0xFFFFu, e8.x >> 16, e8.y & 0xFFFFu, e8.y >> 16,
                                  e8.z & 0xFFFFu, e8.z >> 16, e8.w & 0xFFFFu, e8.w >> 16};
#pragma unroll
    for (int p = 0; p < PAD_RUN; ++p)
#pragma unroll
      for (int f = 0; f < F; ++f) add(ev[p], v[p * F + f], f);
  };
  if (mx > 0.0f) {
    const int64_t bpr = grp.np / PAD_RUN;  // pair blocks per round
    const int64_t blk_lvl = (int64_t)li * nr * bpr;
    for (int r0 = wave * SEG; r0 < nr_use; r0 += 16 * SEG) {
      if constexpr (SEG == 16) {
        // lanes 0..SEG-1 hold rounds r0 + lane: run offset and block count, then the blocks' running ends
        uint32_t m = 0;
        if (lane < SEG && r0 + lane < nr_use) m = mrow[r0 + lane];
        uint32_t incl = lane < SEG ? (m & 0xFFFFu) / PAD_RUN : 0u;
#pragma unroll
        for (int d = 1; d < SEG; d <<= 1) {
          const uint32_t o = __shfl_up(incl, d);
          if (lane >= d) incl += o;
        }
        uint32_t ends[SEG], offs[SEG];
#pragma unroll
        for (int t = 0; t < SEG; ++t) {
          ends[t] = __builtin_amdgcn_readlane(incl, t);
          offs[t] = __builtin_amdgcn_readlane(m >> 16, t);
        }
        for (uint32_t q = (uint32_t)lane; q < ends[SEG - 1]; q += 64) {
          // the run holding block q: the last round whose running start is <= q
          uint32_t qb = 0, off = offs[0];
          int sg = 0;
#pragma unroll
          for (int t = 1; t < SEG; ++t) {
            if (q >= ends[t - 1]) {
              qb = ends[t - 1];
              off = offs[t];
              sg = t;
            }
          }
          add_block(pbuf + (blk_lvl + (int64_t)(r0 + sg) * bpr + off / PAD_RUN + (q - qb)) * pair_block_words(F));
        }
      } else {
        // lane t holds round r0 + t, and the wavefront's blocks are dealt over its lanes in order; block q
        // belongs to the first round whose running end exceeds q, found by a binary search over the lanes'
        // running ends.  Every lane runs every search step (the loop count is the same for the whole
        // wavefront), so the shuffles never read an inactive lane.
        uint32_t m = 0;
        if (r0 + lane < nr_use) m = mrow[r0 + lane];
        const uint32_t nb = (m & 0xFFFFu) / PAD_RUN;
        const uint32_t incl = wave_incl_sum(nb);
        const uint32_t excl = incl - nb;
        const uint32_t total = __builtin_amdgcn_readlane(incl, 63);
        for (uint32_t q0 = 0; q0 < total; q0 += 64) {
          const uint32_t q = q0 + (uint32_t)lane;
          int t = 0;
#pragma unroll
          for (int step = 32; step >= 1; step >>= 1) {
            const uint32_t v = (uint32_t)__shfl((int)incl, t + step - 1);
            if (v <= q) t += step;
          }
          const uint32_t qb = (uint32_t)__shfl((int)excl, t);
          const uint32_t off = (uint32_t)__shfl((int)(m >> 16), t);
          if (q < total)
            add_block(pbuf + (blk_lvl + (int64_t)(r0 + t) * bpr + off / PAD_RUN + (q - qb)) * pair_block_words(F));
        }
      }
    }
  }
  __syncthreads();
  const double inv = ldexp(1.0, -k);
  const int64_t base = ((int64_t)c.offset[l] + entry_lo) * F;
  float* dst32 = static_cast<float*>(ap.dst);
  _Float16* dst16 = static_cast<_Float16*>(ap.dst);
  for (int e = tid; e < count * F; e += 1024) {
    const int64_t gi = base + e;
    const float gsum = (float)((double)(long long)acc[e] * inv);
    float pp = ap.dst_f16 ? (float)dst16[gi] : dst32[gi];
    if (MODE == BIN_GRAD || MODE == BIN_SGD) {
      pp = pp + gsum;
    } else {
      if (ap.g_tap) ap.g_tap[gi] = gsum;
      float mm = ap.m[gi], vv = ap.v[gi];
      float mi = fmaf(1.0f - ap.beta1, gsum, ap.beta1 * mm);
      float vi = fmaf(1.0f - ap.beta2, gsum * gsum, ap.beta2 * vv);
      pp = pp - ap.lr_t * (mi / (sqrtf(vi) + ap.eps));
      ap.m[gi] = mi;
      ap.v[gi] = vi;
    }
    if (ap.dst_f16)
      dst16[gi] = (_Float16)pp;  // round to nearest even, once per entry and step
    else
      dst32[gi] = pp;
  }
}

// ---------------------------------------------------------------------------
// exclusive scan of n uint32 (n + 1 outputs: the last one is the total)

// in has n_in elements; out gets n elements (n >= n_in; the missing inputs count as 0)
// gate (may be NULL): each of the scan's kernels does nothing when *gate == 0 on entry
__global__ __launch_bounds__(1024) void k_scan_tiles(const uint32_t* __restrict__ in, int64_t n_in,
                                                     uint32_t* __restrict__ out, int64_t n,
                                                     uint32_t* __restrict__ tile_sums, const uint32_t* gate) {
  if (gate && *gate == 0u) return;
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
                                                    uint32_t* total_out, const uint32_t* gate) {
  if (gate && *gate == 0u) return;
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
                                                   const uint32_t* __restrict__ tile_pre, const uint32_t* gate) {
  if (gate && *gate == 0u) return;  // a zero total: every input and every tile prefix is zero
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
                           hipStream_t st, bool gated) {
  const int64_t tiles = (n + 1 + 4095) / 4096;
  const uint32_t* gate = gated ? total : nullptr;
  hipLaunchKernelGGL(k_scan_tiles, dim3((unsigned)tiles), dim3(1024), 0, st, in, n, out, n + 1, sums, gate);
  hipLaunchKernelGGL(k_scan_sums, dim3(1), dim3(1024), 0, st, sums, tiles, total, gate);
  hipLaunchKernelGGL(k_scan_add, dim3((unsigned)tiles), dim3(1024), 0, st, out, n + 1, sums, gate);
  return hipGetLastError();
}

template <typename TT, bool DEV>
static hipError_t launch_hash_fwd_d(const DevCfg& c, const PosSrc& src, int64_t n, const TT* table, float* a0,
                                    const FeatLayout& lay, uint32_t* idx_out, const DenseLevels& dl,
                                    const uint32_t* n_dev, hipStream_t st) {
  const int rows = dl.n_multi > 0 ? c.L - dl.n_multi + 1 : c.L;
  int64_t bx = (n + 255) / 256;
  if (DEV && bx > HASH_FWD_DEV_BLOCKS) bx = HASH_FWD_DEV_BLOCKS;
  const dim3 grid((unsigned)bx, (unsigned)rows), block(256);
#define FFN_FWD(FV) \
  hipLaunchKernelGGL((k_hash_fwd<FV, TT, DEV>), grid, block, 0, st, c, src, n, table, a0, lay, idx_out, dl, n_dev)
  switch (c.F) {
    case 1: FFN_FWD(1); break;
    case 2: FFN_FWD(2); break;
    case 4: FFN_FWD(4); break;
    default: return hipErrorInvalidValue;
  }
#undef FFN_FWD
  return hipGetLastError();
}

template <typename TT>
static hipError_t launch_hash_fwd_t(const DevCfg& c, const PosSrc& src, int64_t n, const TT* table, float* a0,
                                    const FeatLayout& lay, uint32_t* idx_out, const DenseLevels& dl,
                                    hipStream_t st, const uint32_t* n_dev) {
  if (n_dev) return launch_hash_fwd_d<TT, true>(c, src, n, table, a0, lay, idx_out, dl, n_dev, st);
  return launch_hash_fwd_d<TT, false>(c, src, n, table, a0, lay, idx_out, dl, nullptr, st);
}

hipError_t launch_hash_fwd(const DevCfg& c, const PosSrc& src, int64_t n, const void* table, float* a0,
                           const FeatLayout& lay, uint32_t* idx_out, const DenseLevels* dl, hipStream_t st,
                           const uint32_t* n_dev) {
  if (n <= 0) return hipSuccess;
  DenseLevels none{};
  none.grid = nullptr;
  none.n_multi = 0;
  none.bricked = 0u;
  for (int l = 0; l < FFN_MAX_LEVELS; ++l) none.off[l] = DENSE_NONE;
  const DenseLevels& d = (dl && dl->grid) ? *dl : none;
  if (c.table_f16)
    return launch_hash_fwd_t(c, src, n, static_cast<const _Float16*>(table), a0, lay, idx_out, d, st, n_dev);
  return launch_hash_fwd_t(c, src, n, static_cast<const float*>(table), a0, lay, idx_out, d, st, n_dev);
}

template <typename TT>
static hipError_t launch_densify_t(const DevCfg& c, const TT* table, const DenseLevels& dl, hipStream_t st) {
  uint32_t max_cells = 0;
  for (int l = 0; l < c.L; ++l)
    if (dl.off[l] != DENSE_NONE) {
      const uint32_t R = (uint32_t)c.res[l], NB = (R + 3) / 4;
      const uint32_t cells = ((dl.bricked >> l) & 1u) ? NB * NB * NB * 64 : R * R * R;
      max_cells = cells > max_cells ? cells : max_cells;
    }
  if (max_cells == 0) return hipSuccess;
  const unsigned bx = (unsigned)((max_cells + 255) / 256 < 2048 ? (max_cells + 255) / 256 : 2048);
  const dim3 grid(bx, (unsigned)c.L), block(256);
  switch (c.F) {
    case 1: hipLaunchKernelGGL((k_hash_densify<1, TT>), grid, block, 0, st, c, table, dl); break;
    case 2: hipLaunchKernelGGL((k_hash_densify<2, TT>), grid, block, 0, st, c, table, dl); break;
    case 4: hipLaunchKernelGGL((k_hash_densify<4, TT>), grid, block, 0, st, c, table, dl); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_hash_densify(const DevCfg& c, const void* table, const DenseLevels& dl, hipStream_t st) {
  if (!dl.grid) return hipSuccess;
  if (c.table_f16) return launch_densify_t(c, static_cast<const _Float16*>(table), dl, st);
  return launch_densify_t(c, static_cast<const float*>(table), dl, st);
}

BinPlan plan_bins(const DevCfg& c, int64_t n, size_t pair_budget_bytes) {
  BinPlan p{};
  // int64 LDS accumulator of one bucket: 2^log2_be * F * 8 bytes = 64 KiB (two reduce blocks per CU), or
  // 128 KiB (one) when a level would otherwise have more than 64 buckets.  An emit round's pairs spread
  // over the buckets, and every run costs its two edge sectors twice (the neighbouring buckets' blocks
  // read them too) plus its padding: at the benchmark shape 64 buckets per level measured emit 4.95 and
  // reduce 2.81 ms against 5.12 and 3.19 ms with 128.  Small tables keep the small buckets, so that the
  // reduction still has blocks for every CU.
  p.log2_be = c.F == 4 ? 11 : (c.F == 2 ? 12 : 13);
  {
    uint32_t max_T = 0;
    for (int l = 0; l < c.L; ++l) max_T = c.mask[l] + 1 > max_T ? c.mask[l] + 1 : max_T;
    if ((max_T >> p.log2_be) > 64u) ++p.log2_be;
  }
  const int rs = emit_nt(c.F);  // samples per emit round
  p.n_rounds = (int)((n + rs - 1) / rs);
  // rounds per emit block: 32 where a level still has at least 256 blocks (a block's set-up, first load and
  // last copy-out are paid once per 32 rounds: at the benchmark shape the scatter took 7.15 ms with 8 rounds,
  // 7.04 with 16 and 7.02 with 32), fewer for small batches so that every CU gets blocks
  int rpb = 32;
  while (rpb > 8 && (p.n_rounds + rpb - 1) / rpb < 256) rpb >>= 1;
  p.chunk = rpb * rs;
  p.nblk = (int)((n + p.chunk - 1) / p.chunk);
  int max_nbl = 0;
  for (int l = 0; l < c.L; ++l) {
    const int nbl = (int)(((int64_t)c.mask[l] + 1 + (1 << p.log2_be) - 1) >> p.log2_be);
    if (nbl > max_nbl) max_nbl = nbl;
  }
  // every round of a level has its own np pair slots (its pairs and at most PAD_RUN - 1 padding pairs per
  // bucket that receives any)
  p.np = round8(emit_stage_pairs(max_nbl, c.F));
  const int64_t per_level_pairs = (int64_t)p.n_rounds * p.np;
  const int64_t pair_bytes = 2 + 4 * (int64_t)c.F;
  int lg = (int)(pair_budget_bytes / (size_t)(per_level_pairs * pair_bytes));
  if (lg < 1) lg = 1;
  if (lg > c.L) lg = c.L;
  p.levels_per_group = lg;
  int max_buckets = 0;
  for (int g0 = 0; g0 < c.L; g0 += lg) {
    int nb = 0;
    for (int l = g0; l < g0 + lg && l < c.L; ++l)
      nb += (int)(((int64_t)c.mask[l] + 1 + (1 << p.log2_be) - 1) >> p.log2_be);
    if (nb > max_buckets) max_buckets = nb;
  }
  p.max_buckets = max_buckets;
  p.max_nbl = max_nbl;
  p.max_pairs = per_level_pairs * lg;
  p.meta_elems = (int64_t)lg * p.n_rounds * max_nbl;
  return p;
}

bool scatter_supported(const DevCfg& c) {
  const BinPlan p = plan_bins(c, 1, (size_t)1 << 30);  // the stage size depends on the table, not on n
  return p.np <= 65535 && emit_lds_bytes(p.max_nbl, c.F) <= 160 * 1024;
}

hipError_t launch_hash_bwd(const DevCfg& c, const PosSrc& src, int64_t n, const float* g, const FeatLayout& lay,
                           int mode, float lr, const BinApply& ap, const BinPlan& plan, const BinScratch& s,
                           hipStream_t st, const uint32_t* n_dev) {
  if (n <= 0) return hipSuccess;
  // run offsets and lengths are 16-bit, and a round's stage must fit in LDS
  const size_t lds_emit = emit_lds_bytes(plan.max_nbl, c.F);
  if (plan.np > 65535 || lds_emit > 160 * 1024) return hipErrorInvalidConfiguration;  // table too large
  const size_t lds_acc = sizeof(unsigned long long) * ((size_t)1 << plan.log2_be) * (size_t)c.F;
  for (int g0 = 0; g0 < c.L; g0 += plan.levels_per_group) {
    BinGroup grp{};
    grp.level0 = g0;
    grp.n_levels = (g0 + plan.levels_per_group <= c.L) ? plan.levels_per_group : c.L - g0;
    grp.log2_be = plan.log2_be;
    grp.chunk = plan.chunk;
    grp.nblk = plan.nblk;
    grp.n_rounds = plan.n_rounds;
    grp.np = plan.np;
    grp.meta_stride = plan.max_nbl;
    int rel = 0;
    for (int li = 0; li < grp.n_levels; ++li) {
      const int l = g0 + li;
      grp.nbl[li] = (int)(((int64_t)c.mask[l] + 1 + (1 << plan.log2_be) - 1) >> plan.log2_be);
      grp.bucket_rel[li] = rel;
      rel += grp.nbl[li];
    }
    grp.bucket_rel[grp.n_levels] = rel;
    const int n_buckets = rel;
    // The reduce walks 64 rounds per wavefront step where a level has many buckets (2^22-entry levels: 512
    // buckets of 8192 entries, runs of about two pair blocks, which left half the lanes of a 16-round step
    // idle; cfg3 backward 15.2 -> 14.2 ms uniform, 16.9 -> 16.1 ms shell) or enough rounds to give every
    // wavefront of a block 64 (the benchmark shape: 16,384 rounds, scatter 6.83 -> 6.74 ms); small batches
    // keep 16 rounds so that their few rounds spread over the block's wavefronts.  FFN_REDUCE_WALK64=0
    // keeps the 16-round walk everywhere (the sums are exact, so both give the same table bit for bit).
    const char* w_env = getenv("FFN_REDUCE_WALK64");
    const bool walk64 = (plan.max_nbl >= 256 || plan.n_rounds >= 16 * 64) && !(w_env && atoi(w_env) == 0);
    const dim3 grid_bl((unsigned)plan.nblk, (unsigned)grp.n_levels);
    const dim3 grid_tr((unsigned)((plan.n_rounds + 63) / 64), (unsigned)((plan.max_nbl + 63) / 64),
                       (unsigned)grp.n_levels);
#define FFN_BIN(FV, MV)                                                                                            \
  do {                                                                                                             \
    hipLaunchKernelGGL((k_bin_emit<FV, MV>), grid_bl, dim3(emit_nt(FV)), lds_emit, st, c, src, n, grp, g, lay,   \
                       lr, s.meta, s.cmax, s.pairs, n_dev);                                                        \
    hipLaunchKernelGGL(k_bin_meta_transpose, grid_tr, dim3(256), 0, st, s.meta, s.meta_t, grp.n_rounds,            \
                       grp.meta_stride, n_dev, emit_nt(FV));                                                       \
    if (walk64)                                                                                                    \
      hipLaunchKernelGGL((k_bin_reduce<FV, MV, 64>), dim3((unsigned)n_buckets), dim3(1024), lds_acc, st, c, grp,   \
                         s.meta_t, s.pairs, s.cmax, ap, n_dev);                                                    \
    else                                                                                                           \
      hipLaunchKernelGGL((k_bin_reduce<FV, MV, 16>), dim3((unsigned)n_buckets), dim3(1024), lds_acc, st, c, grp,   \
                         s.meta_t, s.pairs, s.cmax, ap, n_dev);                                                    \
  } while (0)
#define FFN_BIN_F(MV)                     \
  switch (c.F) {                          \
    case 1: FFN_BIN(1, MV); break;        \
    case 2: FFN_BIN(2, MV); break;        \
    case 4: FFN_BIN(4, MV); break;        \
    default: return hipErrorInvalidValue; \
  }
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

// level-major [L][N][F] <-> sample-major [N][L*F] transposes (the encode entry points' sample-major
// buffers, taps).  A block moves RL_TB samples through an LDS tile [RL_TB][L*F + 1] (odd pitch: the
// level-major side's column accesses spread over the banks): the sample-major side is one contiguous
// range, the level-major side one contiguous range per level, so every global access is coalesced.
constexpr int RL_TB = 128;
template <bool TO_LEVEL_MAJOR>
__global__ __launch_bounds__(256) void k_feat_relayout(const float* __restrict__ src, float* __restrict__ dst,
                                                       int64_t n, int L, int F) {
  extern __shared__ float tile[];
  const int LF = L * F, pitch = LF + 1, lgF = F >> 1;  // F is 1, 2 or 4
  const int64_t b0 = (int64_t)blockIdx.x * RL_TB;
  const int nb = (int)(n - b0 < RL_TB ? n - b0 : RL_TB);
  const int tid = threadIdx.x;
  // sample-major side: element i of the range is (sample i / LF, feature i % LF); the quotient and
  // remainder advance by a fixed step per iteration
  const int qs = 256 / LF, rs = 256 % LF;
  if (TO_LEVEL_MAJOR) {
    int bq = tid / LF, kr = tid % LF;
    for (int i = tid; i < nb * LF; i += 256) {
      tile[bq * pitch + kr] = src[b0 * LF + i];
      bq += qs;
      kr += rs;
      if (kr >= LF) {
        kr -= LF;
        ++bq;
      }
    }
    __syncthreads();
    for (int l = 0; l < L; ++l)
      for (int j = tid; j < nb * F; j += 256)
        dst[(int64_t)l * n * F + b0 * F + j] = tile[(j >> lgF) * pitch + l * F + (j & (F - 1))];
  } else {
    for (int l = 0; l < L; ++l)
      for (int j = tid; j < nb * F; j += 256)
        tile[(j >> lgF) * pitch + l * F + (j & (F - 1))] = src[(int64_t)l * n * F + b0 * F + j];
    __syncthreads();
    int bq = tid / LF, kr = tid % LF;
    for (int i = tid; i < nb * LF; i += 256) {
      dst[b0 * LF + i] = tile[bq * pitch + kr];
      bq += qs;
      kr += rs;
      if (kr >= LF) {
        kr -= LF;
        ++bq;
      }
    }
  }
}

hipError_t launch_feat_relayout(const float* src, const FeatLayout& ls, float* dst, const FeatLayout& ld, int64_t n,
                                int L, int F, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const FeatLayout sm = sample_major(L, F), lm = level_major(n, F);
  const bool s_sm = ls.stride_l == sm.stride_l && ls.stride_b == sm.stride_b;
  const bool s_lm = ls.stride_l == lm.stride_l && ls.stride_b == lm.stride_b;
  const bool d_sm = ld.stride_l == sm.stride_l && ld.stride_b == sm.stride_b;
  const bool d_lm = ld.stride_l == lm.stride_l && ld.stride_b == lm.stride_b;
  if (!((s_sm && d_lm) || (s_lm && d_sm)) || (F != 1 && F != 2 && F != 4)) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((n + RL_TB - 1) / RL_TB));
  const size_t lds = sizeof(float) * (size_t)RL_TB * (size_t)(L * F + 1);
  if (s_sm)
    hipLaunchKernelGGL(k_feat_relayout<true>, grid, dim3(256), lds, st, src, dst, n, L, F);
  else
    hipLaunchKernelGGL(k_feat_relayout<false>, grid, dim3(256), lds, st, src, dst, n, L, F);
  return hipGetLastError();
}

}  // namespace ffn
