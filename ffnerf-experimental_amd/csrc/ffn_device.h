// ffn_device.h -- device-side helpers shared by the gfx950 kernels.
//
// All kernels of this library are compiled with -ffp-contract=off: every
// multiply and add rounds on its own, so the integer-valued outputs that
// depend on floats (sample positions, hash corner indices, occupancy words)
// are reproducible operation for operation.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ffnerf_hip.h"

#define FFN_M 64
#define FFN_D_OUT 16
#define FFN_L_DIR 16
#define FFN_C_IN 32
#define FFN_C_OUT 3
#define FFN_S_MAX 64

typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace ffn {

// Everything a kernel needs from ffn_config, flattened into a kernel argument.
struct DevCfg {
  int L, F, LF;
  uint32_t mask[FFN_MAX_LEVELS];    // 2^log2_T - 1
  uint32_t offset[FFN_MAX_LEVELS];  // level offset in entries
  int res[FFN_MAX_LEVELS];
  float lvl_lr_scale[FFN_MAX_LEVELS];
  int nd, nc, G;
  float bmin[3], bmax[3];
  float inv_extent[3];  // 1 / (bmax - bmin) when that extent is a power of two (exact), else 0
  // Uniform constants of the occupancy grid and the proposals, computed on the host with the same single-
  // precision operations the device code would use (IEEE division and square root), so that they arrive
  // as kernel arguments (scalar registers) instead of being recomputed on the vector ALU and held, or
  // spilled, in vector registers for a whole kernel
  float inv_bs[3];   // 1.0f / (bmax - bmin)
  float occ_cell[3]; // (bmax - bmin) * (1.0f / G): an occupancy cell's extent
  float Gf;          // (float)G
  float dhalf;       // half the box diagonal, 0.5f * sqrtf(dx dx + dy dy + dz dz)
  float occ_lat;     // fmaxf(occ_cell[0], 1e-12f): the proposals' lattice step
  float occ_den;     // fmaxf(Dl Dl + Dl + 1/3, 1e-12f) with Dl = dhalf / occ_lat: the keep draw's denominator
  float rho_min, rho_max, dt_min, dt_max, t_near, t_far;
  int background, hash_opt;
  int table_f16;  // the table is IEEE binary16 (FFN_TABLE_FP16)
};

// ---------------------------------------------------------------------------
// integer hash and xorshift (ffnerf_OG.cl:293-311)

__device__ __forceinline__ uint32_t hash_u32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

__device__ __forceinline__ float rand01(uint32_t& state) {
  uint32_t x = state;
  x ^= x << 13;
  x ^= x >> 17;
  x ^= x << 5;
  state = x;
  return (float)(x & 0x00FFFFFFu) * (1.0f / 16777216.0f);
}

// ---------------------------------------------------------------------------
// powr(x, y) for the sampler weights: double-precision exp(y * log(x)) from
// + - * / only (log: exponent split + atanh series; exp: Cody-Waite reduction
// by ln2 + Taylor series to degree 13), then rounded once to float.
// Deterministic across CPU and GPU; within one float ulp of the true power.

__device__ __forceinline__ double det_log(double x) {
  const double LN2_HI = 6.93147180369123816490e-01;
  const double LN2_LO = 1.90821492927058770002e-10;
  uint64_t bits = (uint64_t)__double_as_longlong(x);
  int e = (int)((bits >> 52) & 0x7ff) - 1023;
  bits = (bits & 0x000fffffffffffffULL) | 0x3ff0000000000000ULL;
  double m = __longlong_as_double((long long)bits);
  if (m > 1.4142135623730951) {
    m = m * 0.5;
    e += 1;
  }
  double s = (m - 1.0) / (m + 1.0);
  double s2 = s * s;
  double p = 1.0 / 25.0;
  p = p * s2 + 1.0 / 23.0;
  p = p * s2 + 1.0 / 21.0;
  p = p * s2 + 1.0 / 19.0;
  p = p * s2 + 1.0 / 17.0;
  p = p * s2 + 1.0 / 15.0;
  p = p * s2 + 1.0 / 13.0;
  p = p * s2 + 1.0 / 11.0;
  p = p * s2 + 1.0 / 9.0;
  p = p * s2 + 1.0 / 7.0;
  p = p * s2 + 1.0 / 5.0;
  p = p * s2 + 1.0 / 3.0;
  p = p * s2 + 1.0;
  double lnm = 2.0 * s * p;
  double de = (double)e;
  return de * LN2_HI + (de * LN2_LO + lnm);
}

__device__ __forceinline__ double det_exp(double z) {
  const double LN2_HI = 6.93147180369123816490e-01;
  const double LN2_LO = 1.90821492927058770002e-10;
  double k = floor(z * 1.4426950408889634 + 0.5);
  double r = (z - k * LN2_HI) - k * LN2_LO;
  double p = 1.0 / 6227020800.0;
  p = p * r + 1.0 / 479001600.0;
  p = p * r + 1.0 / 39916800.0;
  p = p * r + 1.0 / 3628800.0;
  p = p * r + 1.0 / 362880.0;
  p = p * r + 1.0 / 40320.0;
  p = p * r + 1.0 / 5040.0;
  p = p * r + 1.0 / 720.0;
  p = p * r + 1.0 / 120.0;
  p = p * r + 1.0 / 24.0;
  p = p * r + 1.0 / 6.0;
  p = p * r + 0.5;
  p = p * r + 1.0;
  p = p * r + 1.0;
  int ki = (int)k;
  if (ki < -1022) return 0.0;
  if (ki > 1023) return __longlong_as_double(0x7ff0000000000000LL);
  double two_k = __longlong_as_double((long long)((uint64_t)(ki + 1023) << 52));
  return p * two_k;
}

__device__ __forceinline__ float safe_pow_pos(float x, float y) {  // ffnerf_OG.cl:665-671
  x = fmaxf(x, 0.0f);
  if (x <= 0.0f) return 0.0f;
  if (!(x < __builtin_huge_valf())) return x;
  return (float)det_exp((double)y * det_log((double)x));
}

// ---------------------------------------------------------------------------
// ray / box slab test (ffnerf_OG.cl:322-343)

__device__ __forceinline__ bool ray_aabb(const float o[3], const float d[3], const float bmin[3],
                                         const float bmax[3], float& t0, float& t1) {
  float tmin3[3], tmax3[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    float invd = (d[i] != 0.0f) ? (1.0f / d[i]) : __builtin_huge_valf();
    float tb = (bmin[i] - o[i]) * invd;
    float tt = (bmax[i] - o[i]) * invd;
    tmin3[i] = fminf(tb, tt);
    tmax3[i] = fmaxf(tb, tt);
  }
  float tmin = fmaxf(tmin3[0], fmaxf(tmin3[1], tmin3[2]));
  float tmax = fminf(tmax3[0], fminf(tmax3[1], tmax3[2]));
  if (tmax < tmin) return false;
  t0 = tmin;
  t1 = tmax;
  return true;
}

// ---------------------------------------------------------------------------
// hash grid corner math (ffnerf_OG.cl:1286-1364); bit-identical to the oracle

// (x - bmin) / (bmax - bmin), clamped.  For a power-of-two extent the product with its reciprocal is the
// same correctly rounded value as the quotient (both round d * 2^-k), at a fraction of the cost of a
// division; the branch is uniform.
__device__ __forceinline__ void normalize_pos(const DevCfg& c, const float x[3], float p[3]) {
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const float d = x[i] - c.bmin[i];
    float v;
    if (c.inv_extent[i] != 0.0f) {
      v = d * c.inv_extent[i];
    } else {
      const float bs = c.bmax[i] - c.bmin[i];
      v = d / bs;
    }
    p[i] = fminf(fmaxf(v, 0.0f), 1.0f - 1.0e-6f);
  }
}

struct LevelCell {
  int i0[3];
  float f[3];
};

__device__ __forceinline__ LevelCell level_cell(int R, const float p[3]) {
  LevelCell lc;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    float u = p[i] * (float)R;
    int v = (int)floorf(u);
    v = v < 0 ? 0 : (v > R - 2 ? R - 2 : v);
    lc.i0[i] = v;
    lc.f[i] = u - (float)v;
  }
  return lc;
}

__device__ __forceinline__ float corner_weight(const LevelCell& lc, int cc) {
  float wx = (cc & 1) ? lc.f[0] : 1.0f - lc.f[0];
  float wy = (cc & 2) ? lc.f[1] : 1.0f - lc.f[1];
  float wz = (cc & 4) ? lc.f[2] : 1.0f - lc.f[2];
  return wx * wy * wz;
}

// table entry of grid vertex (ix, iy, iz) at level lvl
__device__ __forceinline__ uint32_t level_entry(uint32_t ix, uint32_t iy, uint32_t iz, int lvl, uint32_t mask) {
  return hash_u32(ix * 73856093u ^ iy * 19349663u ^ iz * 83492791u ^ (uint32_t)lvl * 2654435761u) & mask;
}

__device__ __forceinline__ uint32_t corner_entry(const LevelCell& lc, int cc, int lvl, uint32_t mask) {
  return level_entry((uint32_t)(lc.i0[0] + (cc & 1)), (uint32_t)(lc.i0[1] + ((cc >> 1) & 1)),
                     (uint32_t)(lc.i0[2] + ((cc >> 2) & 1)), lvl, mask);
}

// ---------------------------------------------------------------------------
// Streaming stores: the non-temporal hint (`nt`) lets the written lines leave the L2 first, so that data a
// kernel writes once for a later pass does not evict what the kernel itself still gathers from the caches

__device__ __forceinline__ void store_stream(float* p, float v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void store_stream(float2* p, float2 v) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  __builtin_nontemporal_store(f2{v.x, v.y}, reinterpret_cast<f2*>(p));
}
__device__ __forceinline__ void store_stream(float4* p, float4 v) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(f4{v.x, v.y, v.z, v.w}, reinterpret_cast<f4*>(p));
}
__device__ __forceinline__ void store_stream(uint4* p, uint4 v) {
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(u4{v.x, v.y, v.z, v.w}, reinterpret_cast<u4*>(p));
}

// ---------------------------------------------------------------------------
// activations (ffnerf_OG.cl:214-253) and SH degree 3 (ffnerf_OG.cl:572-602)

// e^x as 2^(x log2 e) on v_exp_f32 instead of the range-reduced correctly rounded expf: relative error
// below 2e-6 for the arguments used here (|x| <= 20; the rounding of x log2 e dominates); used where the
// result is checked within a relative tolerance
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// log(1 + e^x): log1p of y = e^x as log(u) * y / (u - 1), u = 1 + y (exact for the rounded u, so accurate
// for small y; Goldberg's method), on v_log_f32 and v_rcp_f32
// ReLU as one integer maximum of the bit pattern: a float with the sign bit clear is a non-negative integer,
// one with it set a negative one, so max_i32(bits, 0) keeps x > 0 (and +0) and maps every negative value and
// -0 to +0 -- the values of x > 0 ? x : 0.  Written as a float comparison, the compiler lowers it to an IEEE
// maximum that first canonicalises its MFMA-produced operand (two vector instructions per value).
__device__ __forceinline__ float relu_f(float x) {
  const int b = __float_as_int(x);
  return __int_as_float(b > 0 ? b : 0);
}

__device__ __forceinline__ float softplus(float x) {
  if (x > 20.0f) return x;
  const float y = fast_exp(x);
  if (x < -20.0f) return y;
  const float u = 1.0f + y;
  if (u == 1.0f) return y;
  return __builtin_amdgcn_logf(u) * 0.69314718055994531f * y * __builtin_amdgcn_rcpf(u - 1.0f);
}
// The MLP's per-sample activation and loss derivatives use the hardware reciprocal and reciprocal square
// root (v_rcp_f32 / v_rsq_f32, about 1 ulp) instead of IEEE division: they feed outputs checked against
// the CPU restatement within a relative tolerance, and a correctly rounded division costs about ten vector
// instructions per lane.
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float softplus_prime_from_pre(float x) {
  if (x >= 0.0f) return fast_rcp(1.0f + fast_exp(-x));
  float e = fast_exp(x);
  return e * fast_rcp(1.0f + e);
}
__device__ __forceinline__ float sigmoid_soft(float x) {
  x *= 0.5f;
  x = fminf(fmaxf(x, -18.0f), 18.0f);
  if (x >= 0.0f) return fast_rcp(1.0f + fast_exp(-x));
  float e = fast_exp(x);
  return e * fast_rcp(1.0f + e);
}
__device__ __forceinline__ float charbonnier_prime(float x) {
  const float e2 = 1.0e-3f * 1.0e-3f;
  return x * __builtin_amdgcn_rsqf(x * x + e2);
}

__device__ __forceinline__ float sh_component(const float d[3], int i) {
  const float x = d[0], y = d[1], z = d[2];
  switch (i) {
    case 0: return 0.28209479177387814f;
    case 1: return 0.4886025119029199f * y;
    case 2: return 0.4886025119029199f * z;
    case 3: return 0.4886025119029199f * x;
    case 4: return 1.0925484305920792f * x * y;
    case 5: return 1.0925484305920792f * y * z;
    case 6: return 0.31539156525252005f * (3.0f * z * z - 1.0f);
    case 7: return 1.0925484305920792f * x * z;
    case 8: return 0.5462742152960396f * (x * x - y * y);
    case 9: return 0.5900435899266435f * y * (3.0f * x * x - y * y);
    case 10: return 2.890611442640554f * x * y * z;
    case 11: return 0.4570457994644658f * y * (5.0f * z * z - 1.0f);
    case 12: return 0.3731763325901154f * (5.0f * z * z * z - 3.0f * z);
    case 13: return 0.4570457994644658f * x * (5.0f * z * z - 1.0f);
    case 14: return 1.445305721320277f * z * (x * x - y * y);
    default: return 0.5900435899266435f * x * (x * x - 3.0f * y * y);
  }
}

// ---------------------------------------------------------------------------
// Work-group scans of the reference restated on wave lanes.  A "segment" is
// S consecutive lanes (S a power of two <= 64) holding one ray; lid is the
// lane's index inside it and base the segment's first lane.  The trees and
// the operand order of every combine are those of ffnerf_OG.cl:619-646 and
// 691-735 (including the down-sweep's new_right = combine(old_left,
// old_right)), so results are bit-identical to the CPU restatement.

__device__ __forceinline__ bool is_right(int lid, int stride) { return ((lid + 1) & (2 * stride - 1)) == 0; }
__device__ __forceinline__ bool is_left(int lid, int stride) {
  return ((lid + 1 + stride) & (2 * stride - 1)) == 0;
}

// Lane movement of the trees.  At stride s the "right" lane of every aligned
// 2s-lane block reads its partner s lanes below and the "left" lane reads the
// one s lanes above.  Inside a 16-lane row (s <= 8) that is a DPP row shift;
// for s = 16 and 32 the lower partner of the served lanes (31, 63 and 63) is
// what DPP row_bcast:15 / row_bcast:31 deliver, and the upper partner of the
// served lanes (15, 47 and 31) what v_permlane16_swap / v_permlane32_swap
// deliver (the odd row of each row pair, the upper half of the wave: checked
// on the device).  All of them are VALU operations: no LDS round trip.  Lanes
// that are not served get unspecified values, exactly as the tree ignores them.
template <int S_>
__device__ __forceinline__ float from_lower(float v) {
  const int x = __float_as_int(v);
  int r;
  if constexpr (S_ < 16)
    r = __builtin_amdgcn_update_dpp(x, x, 0x110 + S_, 0xF, 0xF, false);  // row_shr:S_
  else if constexpr (S_ == 16)
    r = __builtin_amdgcn_update_dpp(x, x, 0x142, 0xF, 0xF, false);  // row_bcast:15
  else
    r = __builtin_amdgcn_update_dpp(x, x, 0x143, 0xF, 0xF, false);  // row_bcast:31
  return __int_as_float(r);
}
template <int S_>
__device__ __forceinline__ float from_upper(float v) {
  const int x = __float_as_int(v);
  if constexpr (S_ < 16) {
    return __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x100 + S_, 0xF, 0xF, false));  // row_shl:S_
  } else if constexpr (S_ == 16) {
    return __int_as_float((int)__builtin_amdgcn_permlane16_swap(x, x, false, false)[1]);  // lane i <- odd row
  } else {
    return __int_as_float((int)__builtin_amdgcn_permlane32_swap(x, x, false, false)[1]);  // lanes 0-31 <- 32-63
  }
}

template <int ST>
__device__ __forceinline__ void scan_add_up(float& v, int lid, int S) {
  if (ST < S) {
    const float o = from_lower<ST>(v);
    if (is_right(lid, ST)) v = v + o;
  }
}
template <int ST>
__device__ __forceinline__ void scan_add_down(float& v, int lid, int S) {
  if (ST < S) {
    const float from_l = from_lower<ST>(v);
    const float from_r = from_upper<ST>(v);
    if (is_right(lid, ST)) v = v + from_l;
    else if (is_left(lid, ST)) v = from_r;
  }
}

__device__ __forceinline__ float seg_scan_excl_add(float v, int lid, int S, int base) {
  (void)base;
  scan_add_up<1>(v, lid, S);
  scan_add_up<2>(v, lid, S);
  scan_add_up<4>(v, lid, S);
  scan_add_up<8>(v, lid, S);
  scan_add_up<16>(v, lid, S);
  scan_add_up<32>(v, lid, S);
  if (lid == S - 1) v = 0.0f;
  scan_add_down<32>(v, lid, S);
  scan_add_down<16>(v, lid, S);
  scan_add_down<8>(v, lid, S);
  scan_add_down<4>(v, lid, S);
  scan_add_down<2>(v, lid, S);
  scan_add_down<1>(v, lid, S);
  return v;
}

// ffnerf_OG.cl:639-646: a[lid] += a[lid + stride] for lid < stride; result a[0] broadcast
template <int ST>
__device__ __forceinline__ void reduce_add_step(float& v, int lid, int S) {
  if (ST < S) {
    float o;
    o = from_upper<ST>(v);  // lanes below ST read lid + ST
    if (lid < ST) v = v + o;
  }
}
__device__ __forceinline__ float seg_reduce_add(float v, int lid, int S, int base) {
  reduce_add_step<32>(v, lid, S);
  reduce_add_step<16>(v, lid, S);
  reduce_add_step<8>(v, lid, S);
  reduce_add_step<4>(v, lid, S);
  reduce_add_step<2>(v, lid, S);
  reduce_add_step<1>(v, lid, S);
  return __shfl(v, base);
}

struct Seg {
  float a, v0, v1, v2;
};
__device__ __forceinline__ Seg seg_combine(const Seg& L, const Seg& R) {
  Seg O;
  O.a = L.a * R.a;
  O.v0 = L.v0 + L.a * R.v0;
  O.v1 = L.v1 + L.a * R.v1;
  O.v2 = L.v2 + L.a * R.v2;
  return O;
}
__device__ __forceinline__ Seg shfl_seg(const Seg& s, int src) {
  Seg o;
  o.a = __shfl(s.a, src);
  o.v0 = __shfl(s.v0, src);
  o.v1 = __shfl(s.v1, src);
  o.v2 = __shfl(s.v2, src);
  return o;
}
template <int ST>
__device__ __forceinline__ Seg seg_lower(const Seg& s) {
  return Seg{from_lower<ST>(s.a), from_lower<ST>(s.v0), from_lower<ST>(s.v1), from_lower<ST>(s.v2)};
}
template <int ST>
__device__ __forceinline__ Seg seg_upper(const Seg& s) {
  return Seg{from_upper<ST>(s.a), from_upper<ST>(s.v0), from_upper<ST>(s.v1), from_upper<ST>(s.v2)};
}
template <int ST>
__device__ __forceinline__ void seg_up(Seg& v, int lid, int S) {
  if (ST < S) {
    const Seg o = seg_lower<ST>(v);
    if (is_right(lid, ST)) v = seg_combine(o, v);
  }
}
template <int ST>
__device__ __forceinline__ void seg_down(Seg& v, int lid, int S) {
  if (ST < S) {
    const Seg from_l = seg_lower<ST>(v);
    const Seg from_r = seg_upper<ST>(v);
    if (is_right(lid, ST)) v = seg_combine(from_l, v);
    else if (is_left(lid, ST)) v = from_r;
  }
}

// exclusive Seg scan; returns the lane's prefix, total of the segment in *total
__device__ __forceinline__ Seg seg_scan_excl_seg(Seg v, int lid, int S, int base, Seg* total) {
  seg_up<1>(v, lid, S);
  seg_up<2>(v, lid, S);
  seg_up<4>(v, lid, S);
  seg_up<8>(v, lid, S);
  seg_up<16>(v, lid, S);
  seg_up<32>(v, lid, S);
  *total = shfl_seg(v, base + S - 1);
  if (lid == S - 1) {
    v.a = 1.0f;
    v.v0 = v.v1 = v.v2 = 0.0f;
  }
  seg_down<32>(v, lid, S);
  seg_down<16>(v, lid, S);
  seg_down<8>(v, lid, S);
  seg_down<4>(v, lid, S);
  seg_down<2>(v, lid, S);
  seg_down<1>(v, lid, S);
  return v;
}

struct Aff {
  float a, b;
};
__device__ __forceinline__ Aff aff_combine_rev(const Aff& L, const Aff& R) {
  Aff O;
  O.a = R.a * L.a;
  O.b = R.a * L.b + R.b;
  return O;
}
__device__ __forceinline__ Aff shfl_aff(const Aff& s, int src) {
  Aff o;
  o.a = __shfl(s.a, src);
  o.b = __shfl(s.b, src);
  return o;
}
template <int ST>
__device__ __forceinline__ void aff_up(Aff& v, int lid, int S) {
  if (ST < S) {
    const Aff o{from_lower<ST>(v.a), from_lower<ST>(v.b)};
    if (is_right(lid, ST)) v = aff_combine_rev(o, v);
  }
}
template <int ST>
__device__ __forceinline__ void aff_down(Aff& v, int lid, int S) {
  if (ST < S) {
    const Aff from_l{from_lower<ST>(v.a), from_lower<ST>(v.b)};
    const Aff from_r{from_upper<ST>(v.a), from_upper<ST>(v.b)};
    if (is_right(lid, ST)) v = aff_combine_rev(from_l, v);
    else if (is_left(lid, ST)) v = from_r;
  }
}
// exclusive scan with aff_combine_rev over the segment's lanes in lane order
__device__ __forceinline__ Aff seg_scan_excl_aff_rev(Aff v, int lid, int S, int base) {
  (void)base;
  aff_up<1>(v, lid, S);
  aff_up<2>(v, lid, S);
  aff_up<4>(v, lid, S);
  aff_up<8>(v, lid, S);
  aff_up<16>(v, lid, S);
  aff_up<32>(v, lid, S);
  if (lid == S - 1) {
    v.a = 1.0f;
    v.b = 0.0f;
  }
  aff_down<32>(v, lid, S);
  aff_down<16>(v, lid, S);
  aff_down<8>(v, lid, S);
  aff_down<4>(v, lid, S);
  aff_down<2>(v, lid, S);
  aff_down<1>(v, lid, S);
  return v;
}

// largest value over the wavefront (v >= 0): row-wise prefix maxima with DPP row shifts, then the rows
// combined with row_bcast:15/31; lane 63 ends with the maximum
__device__ __forceinline__ float wave_max_nonneg(float v) {
  auto step = [](float x, int ctrl) {
    const int xi = __float_as_int(x);
    int r;
    switch (ctrl) {
      case 1: r = __builtin_amdgcn_update_dpp(xi, xi, 0x111, 0xF, 0xF, false); break;
      case 2: r = __builtin_amdgcn_update_dpp(xi, xi, 0x112, 0xF, 0xF, false); break;
      case 4: r = __builtin_amdgcn_update_dpp(xi, xi, 0x114, 0xF, 0xF, false); break;
      case 8: r = __builtin_amdgcn_update_dpp(xi, xi, 0x118, 0xF, 0xF, false); break;
      case 15: r = __builtin_amdgcn_update_dpp(xi, xi, 0x142, 0xF, 0xF, false); break;
      default: r = __builtin_amdgcn_update_dpp(xi, xi, 0x143, 0xF, 0xF, false); break;
    }
    return fmaxf(x, __int_as_float(r));
  };
  v = step(v, 1);
  v = step(v, 2);
  v = step(v, 4);
  v = step(v, 8);
  v = step(v, 15);
  v = step(v, 31);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// next set bit strictly after lid inside the segment's 64-bit run mask, or S
__device__ __forceinline__ int find_next_flag(uint64_t segmask, int lid, int S) {
  if (lid + 1 >= S) return S;
  uint64_t m = segmask >> (lid + 1);
  if (m == 0) return S;
  int r = lid + 1 + (int)__builtin_ctzll(m);
  return r < S ? r : S;
}

// CAS nibble max into an occupancy word (ffnerf_OG.cl:486-512)
__device__ __forceinline__ void occ_nibble_atomic_max(uint32_t* grid, int cell, uint32_t sub, uint32_t proposed_q) {
  const uint32_t shift = 4u * sub;
  const uint32_t mask = 0xFu << shift;
  uint32_t old_u = __hip_atomic_load(grid + cell, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (;;) {
    uint32_t old_q = ((old_u >> shift) & 0xFu) + 1u;
    if (proposed_q <= old_q) return;
    uint32_t new_u = (old_u & ~mask) | (((proposed_q - 1u) & 0xFu) << shift);
    uint32_t prev = atomicCAS(grid + cell, old_u, new_u);
    if (prev == old_u) return;
    old_u = prev;
  }
}


// grid coordinates of a point for the occupancy proposals (ffnerf_OG.cl:1660-1690); the same operations
// serve the early load of the cell's occupancy word, the runs of the marched samples and the proposal itself
__device__ __forceinline__ void occ_grid_pos(const DevCfg& c, const float (&o)[3], const float (&d)[3], float t,
                                             float (&gpos)[3]) {
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const float bs = c.bmax[i] - c.bmin[i];
    const float xi = o[i] + t * d[i];
    gpos[i] = (xi - c.bmin[i]) * c.inv_bs[i] * c.Gf;
  }
}

__device__ __forceinline__ float half_box_diagonal(const DevCfg& c) { return c.dhalf; }

// The occupancy proposal of one run: the samples of ray rj that lie in one subcell, from sample lid (time t_j,
// transmittance Tr_j arriving at it) to sample `last` (t_last, T_last).  (t_prev, T_prev) is the sample
// before the run (the run's first when it is the ray's first); (t_nx, T_nx) the first sample after the run
// when has_next, else the cell's exit and the ray's final transmittance T_final.  The transmittance is
// interpolated to the cell's entry and exit; 16 times the predicted absorption, rounded stochastically,
// becomes the proposed level, which raises the subcell's nibble of occ_st (an atomic max) when it exceeds the
// occ_in level (occ_word: the cell's occ_in word) and the distance-dependent keep draw accepts it
// (ffnerf_OG.cl:1640-1821).  Dhalf: half the box diagonal.
__device__ __forceinline__ void occ_propose_run(const DevCfg& c, const float (&o)[3], const float (&d)[3], float t_j,
                                                float Tr_j, float t_prev, float T_prev, float t_last, float T_last,
                                                bool has_next, float t_nx, float T_nx, float T_final,
                                                uint32_t occ_word, uint32_t seed, uint32_t rj, uint32_t lid,
                                                float Dhalf, uint32_t* occ_st) {
  const int G = c.G;
  float gpos[3];
  occ_grid_pos(c, o, d, t_j, gpos);
  const int ix = (int)floorf(gpos[0]), iy = (int)floorf(gpos[1]), iz = (int)floorf(gpos[2]);
  if (!((uint32_t)ix < (uint32_t)G && (uint32_t)iy < (uint32_t)G && (uint32_t)iz < (uint32_t)G)) return;
  uint32_t sub = 0;
#pragma unroll
  for (int i = 0; i < 3; ++i) sub += ((gpos[i] - floorf(gpos[i])) >= 0.5f ? 1u : 0u) << i;
  const int cell = ix + G * (iy + G * iz);
  float pred = 0.0f;
  {
    const int ii[3] = {ix, iy, iz};
    float cmin[3], cmax[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      cmin[i] = c.bmin[i] + (float)ii[i] * c.occ_cell[i];
      cmax[i] = cmin[i] + c.occ_cell[i];
    }
    float t_enter, t_exit;
    if (ray_aabb(o, d, cmin, cmax, t_enter, t_exit)) {
      t_enter = fmaxf(t_enter, c.t_near);
      t_exit = fminf(t_exit, c.t_far);
      if (t_exit > t_enter) {
        const float denom0 = t_j - t_prev;
        float u0 = (fabsf(denom0) > 1.0e-8f) ? (t_enter - t_prev) / denom0 : 0.0f;
        u0 = fminf(fmaxf(u0, 0.0f), 1.0f);
        const float T_enter = T_prev + (Tr_j - T_prev) * u0;
        const float t_next = has_next ? t_nx : t_exit;
        const float T_next = has_next ? T_nx : T_final;
        const float denom1 = t_next - t_last;
        float u1 = (fabsf(denom1) > 1.0e-8f) ? (t_exit - t_last) / denom1 : 1.0f;
        u1 = fminf(fmaxf(u1, 0.0f), 1.0f);
        const float T_exit = T_last + (T_next - T_last) * u1;
        pred = fminf(1.0f, fmaxf(0.0f, (T_enter - T_exit) / fmaxf(T_enter, 1.0e-12f)));
      }
    }
  }
  const uint32_t old_q = ((occ_word >> (4u * sub)) & 0xFu) + 1u;
  uint32_t proposed_q = old_q;
  const float pred16 = pred * 16.0f;
  const uint32_t hseed =
      hash_u32(seed ^ rj * 747796405u ^ lid * 2891336453u ^ (uint32_t)cell * 9781u ^ sub * 6271u);
  if (pred16 > (float)old_q && old_q < 16u) {
    const float f0 = floorf(pred16);
    const float frac = pred16 - f0;
    const uint32_t q0 = (uint32_t)f0;
    const uint32_t thresh = (uint32_t)(frac * 16777216.0f);
    const uint32_t q_stoch = ((hseed & 0x00FFFFFFu) < thresh) ? (q0 + 1u) : q0;
    proposed_q = q_stoch > 16u ? 16u : q_stoch;
  }
  // occ_st equals occ_in after every decay and proposals only raise it, so a proposal that does not exceed
  // the occ_in nibble cannot change occ_st: skip the keep draw and the atomic
  if (proposed_q > old_q) {
    (void)Dhalf;  // in c.occ_den
    const float tl = t_j / c.occ_lat;
    const float num = tl * tl + tl + (1.0f / 3.0f);
    const float keep_p = fminf(num / c.occ_den, 1.0f);
    bool keep = keep_p >= 1.0f;
    if (!keep) {
      uint32_t rk = hseed;
      keep = rand01(rk) <= keep_p;
    }
    if (keep) occ_nibble_atomic_max(occ_st, cell, sub, proposed_q);
  }
}

}  // namespace ffn
