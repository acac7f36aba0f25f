// ffn_mlp_common.h -- pieces shared by the fp32 and the fp16/bf16 MLP kernels:
// the per-ray compositing with the photometric loss gradient, the reversed
// affine scan and the occupancy proposals (ffnerf_OG.cl:1505-1821), and the
// output deltas with the distance gate (ffnerf_OG.cl:1863-1914).
#pragma once
#include "ffn_device.h"
#include "ffn_kernels.h"

namespace ffn {

// Make LDS writes of this wavefront visible to its own later LDS reads and
// keep the compiler from moving LDS accesses across this point.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// the background colour of ray rj (black, white, or the seeded random colour while training;
// ffnerf_OG.cl:1534-1541)
__device__ __forceinline__ void background(const MlpArgs& a, int64_t rj, bool train, float (&bg)[3]) {
  bg[0] = bg[1] = bg[2] = 0.0f;
  if (train) {
    if (a.c.background == FFN_BG_WHITE) {
      bg[0] = bg[1] = bg[2] = 1.0f;
    } else if (a.c.background == FFN_BG_RANDOM) {
      uint32_t rb = hash_u32(a.seed ^ (uint32_t)rj * 747796405u ^ 0xA511E9B3u);
      bg[0] = rand01(rb);
      bg[1] = rand01(rb);
      bg[2] = rand01(rb);
    }
  }
}

// per-sample inputs of the compositing; lane j holds sample j of the 64-sample tile
struct CompLane {
  int64_t bj, rj;
  bool vj;
  float dt_j, t_j;
  float4 tg;
  uint64_t segmask;
  uint32_t occ_word;  // occ_in word of the sample's cell (proposal lanes), loaded early for its latency
};

// prop_wave: this wavefront composites the tile and makes its occupancy proposals (one wavefront per tile,
// all 64 lanes); the others load only what the empty-tile test needs (validity and dt).
// SC: the samples per ray when fixed at compile time (64, the benchmark's), else 0 and a.S at run time; a
// fixed S turns the segment logic of the compositing's scans into constants.
template <int SC>
__device__ __forceinline__ CompLane load_comp_lane(const MlpArgs& a, int64_t tile, int lane, bool prop_wave,
                                                   uint64_t n_samples, int log2S, bool proposals) {
  const int S = SC > 0 ? SC : a.S;
  CompLane L;
  L.bj = tile * 64 + lane;
  L.vj = (uint64_t)L.bj < n_samples;
  L.rj = L.vj ? (L.bj >> log2S) : 0;
  L.dt_j = L.vj ? a.DTs[L.bj] : 0.0f;
  L.tg = make_float4(0.f, 0.f, 0.f, 0.f);
  if (prop_wave && L.vj && a.targets) L.tg = a.targets[L.rj];
  L.t_j = 0.0f;
  L.segmask = 0;
  L.occ_word = 0;
  if (prop_wave && proposals && L.vj) {
    L.t_j = a.Ts[L.bj];
    L.segmask = (uint64_t)a.flags[2 * L.rj] | ((uint64_t)a.flags[2 * L.rj + 1] << 32);
    const int lid = lane & (S - 1);
    if (((L.segmask >> lid) & 1ull) && L.dt_j > 0.0f) {
      const float4 ro = a.rays[2 * L.rj], rdv = a.rays[2 * L.rj + 1];
      const float o[3] = {ro.x, ro.y, ro.z}, d[3] = {rdv.x, rdv.y, rdv.z};
      float gpos[3];
      occ_grid_pos(a.c, o, d, L.t_j, gpos);
      const int G = a.c.G;
      const int ix = (int)floorf(gpos[0]), iy = (int)floorf(gpos[1]), iz = (int)floorf(gpos[2]);
      if ((uint32_t)ix < (uint32_t)G && (uint32_t)iy < (uint32_t)G && (uint32_t)iz < (uint32_t)G)
        L.occ_word = a.occ_in[ix + G * (iy + G * iz)];
    }
  }
  return L;
}

// The compositing's transmittance and colour prefix on DPP: Hillis-Steele steps inside 16-lane rows, then
// across rows.  Segments are S consecutive lanes (one ray), S a power of two <= 64.  The combine order is
// not the reference's work-group tree (the results agree to fp32 rounding: the prefix multiplies both
// terms of every gradient alike), and the scan takes about a third of the tree's vector instructions.

// v read from the lane CTRL selects (row masks ROW_MASK), `old` where the source lane is invalid
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_or(float old, float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ Seg seg_dpp(const Seg& v) {  // identity (1, 0) where the source is invalid
  return Seg{dpp_or<CTRL, ROW_MASK>(1.0f, v.a), dpp_or<CTRL, ROW_MASK>(0.0f, v.v0),
             dpp_or<CTRL, ROW_MASK>(0.0f, v.v1), dpp_or<CTRL, ROW_MASK>(0.0f, v.v2)};
}

// v read from the lane CTRL selects, 0 where the source lane is invalid (bound_ctrl): for the row shifts
// whose result the invalid lanes discard, so the read needs no copy of an `old` value and can fold into
// the combine's arithmetic
template <int CTRL>
__device__ __forceinline__ Seg seg_dpp_z(const Seg& v) {
  auto z = [](float x) { return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true)); };
  return Seg{z(v.a), z(v.v0), z(v.v1), z(v.v2)};
}

// exclusive prefix of seg_combine over each segment (identity at its first lane); *total = the segment's
// combination of all its lanes
__device__ __forceinline__ Seg comp_seg_prefix(Seg v, int lane, int S, Seg* total) {
  const int key = lane & 15 & (S - 1);  // position inside the segment's part of the row
  // row_shr:k: lanes with key < k (the row's first k lanes among them) keep v, so their reads are unused
  if (S > 1) {
    const Seg n = seg_combine(seg_dpp_z<0x111>(v), v);  // row_shr:1
    if (key >= 1) v = n;
  }
  if (S > 2) {
    const Seg n = seg_combine(seg_dpp_z<0x112>(v), v);
    if (key >= 2) v = n;
  }
  if (S > 4) {
    const Seg n = seg_combine(seg_dpp_z<0x114>(v), v);
    if (key >= 4) v = n;
  }
  if (S > 8) {
    const Seg n = seg_combine(seg_dpp_z<0x118>(v), v);
    if (key >= 8) v = n;
  }
  if (S >= 32) v = seg_combine(seg_dpp<0x142, 0xA>(v), v);  // row_bcast:15 into rows 1 and 3
  if (S >= 64) v = seg_combine(seg_dpp<0x143, 0xC>(v), v);  // row_bcast:31 into rows 2 and 3
  if (S == 64) {  // one segment: its total is lane 63's, read into scalar registers (no LDS round trip)
    auto rl = [](float x) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63)); };
    *total = Seg{rl(v.a), rl(v.v0), rl(v.v1), rl(v.v2)};
  } else {
    *total = shfl_seg(v, (lane & ~(S - 1)) + S - 1);
  }
  Seg e = seg_dpp<0x138>(v);  // wave_shr:1
  if ((lane & (S - 1)) == 0) e = Seg{1.0f, 0.0f, 0.0f, 0.0f};
  return e;
}

// Compositing of the tile's rays on the wavefront's 64 lanes (S lanes per ray), the loss gradient, the
// output colour (wavefront 0), taps (wavefront 0) and, on the tile's proposal wavefront, the occupancy
// proposals of all its samples; returns dL/dsigma and dL/dc of lane j's sample.  sSig/sRgb hold
// sigma[64] and rgb[64][3] of the tile.
template <bool TAPS, int SC>
__device__ __forceinline__ void composite_tile(const MlpArgs& a, const float* __restrict__ sSig,
                                               const float* __restrict__ sRgb, const CompLane& L, int lane,
                                               int wave, bool prop_wave, bool train, bool proposals, float Dhalf,
                                               float& dLds_j, float (&dLdc_j)[3]) {
  const DevCfg& c = a.c;
  const int S = SC > 0 ? SC : a.S;
  const int64_t bj = L.bj, rj = L.rj;
  const bool vj = L.vj;
  const float dt_j = L.dt_j, t_j = L.t_j;
  const float4 tg = L.tg;
  const uint64_t segmask = L.segmask;
  {
    const int j = lane;
    const int lid = j & (S - 1);
    const int base = j - lid;
    const float sig_j = sSig[j];
    const float c0 = sRgb[3 * j], c1 = sRgb[3 * j + 1], c2 = sRgb[3 * j + 2];
    float alpha = 0.0f;
    if (dt_j > 0.0f) alpha = 1.0f - fast_exp(fminf(fmaxf(-sig_j * dt_j, -5.0f), 18.0f));
    const float oma = 1.0f - alpha;
    Seg my;
    my.a = oma;
    my.v0 = alpha * c0;
    my.v1 = alpha * c1;
    my.v2 = alpha * c2;
    Seg tot;
    const Seg pre = comp_seg_prefix(my, lane, S, &tot);
    const float Tr = pre.a, T_final = tot.a;
    float bg[3];
    background(a, rj, train, bg);
    const float Cf0 = tot.v0 + T_final * bg[0];
    const float Cf1 = tot.v1 + T_final * bg[1];
    const float Cf2 = tot.v2 + T_final * bg[2];
    const float gr0 = charbonnier_prime(Cf0 - tg.x);
    const float gr1 = charbonnier_prime(Cf1 - tg.y);
    const float gr2 = charbonnier_prime(Cf2 - tg.z);
    const float gT_end = gr0 * bg[0] + gr1 * bg[1] + gr2 * bg[2];
    if (wave == 0 && lid == 0 && vj)
      a.out_rgb[rj] = make_float4(fminf(fmaxf(Cf0, 0.0f), 1.0f), fminf(fmaxf(Cf1, 0.0f), 1.0f),
                                  fminf(fmaxf(Cf2, 0.0f), 1.0f), train ? 4.0f : 0.0f);
    const float ws = Tr * alpha;
    dLdc_j[0] = ws * gr0;
    dLdc_j[1] = ws * gr1;
    dLdc_j[2] = ws * gr2;
    Aff f;
    f.a = oma;
    f.b = gr0 * (alpha * c0) + gr1 * (alpha * c1) + gr2 * (alpha * c2);
    // gT after sample j, in the reference's tree order: dL/dsigma is Tr (sum g c - gT_next) with the two
    // terms nearly equal for many samples, so another combine order (rounding differences of 1e-7 in
    // gT_next) moves it by up to 1e-2 of its range against the CPU restatement; the prefix above has no
    // such cancellation
    const Aff f_rev = shfl_aff(f, base + (S - 1 - lid));  // lane k holds the element of sample S-1-k
    const Aff scn = seg_scan_excl_aff_rev(f_rev, lid, S, base);
    const int m = (lid <= S - 2) ? (S - 2 - lid) : 0;
    const Aff sm = shfl_aff(scn, base + m);
    const Aff em = shfl_aff(f_rev, base + m);
    float gT_next = gT_end;
    if (lid <= S - 2) {
      const Aff incl = aff_combine_rev(sm, em);
      gT_next = incl.a * gT_end + incl.b;
    }
    const float gA = gr0 * (Tr * c0) + gr1 * (Tr * c1) + gr2 * (Tr * c2);
    const float gAlpha = gA - gT_next * Tr;
    const float dads = (dt_j > 0.0f) ? (dt_j * oma) : 0.0f;
    const float regu = (dt_j > 0.0f) ? (5e-3f * dt_j * ldexpf(1.0f, -a.log2S)) : 0.0f;  // / S, exactly
    dLds_j = gAlpha * dads + regu;

    if (TAPS && wave == 0) {
      if (vj) {
        if (a.t_sigma) a.t_sigma[bj] = sig_j;
        if (a.t_rgb) {
          a.t_rgb[3 * bj] = c0;
          a.t_rgb[3 * bj + 1] = c1;
          a.t_rgb[3 * bj + 2] = c2;
        }
        if (a.t_Tr) a.t_Tr[bj] = Tr;
        if (a.t_Tfinal && lid == 0) a.t_Tfinal[rj] = T_final;
        if (a.t_color && lid == 0) a.t_color[rj] = make_float4(Cf0, Cf1, Cf2, 0.0f);
        if (a.t_dLds) a.t_dLds[bj] = dLds_j;
        if (a.t_dLdc) {
          a.t_dLdc[3 * bj] = dLdc_j[0];
          a.t_dLdc[3 * bj + 1] = dLdc_j[1];
          a.t_dLdc[3 * bj + 2] = dLdc_j[2];
        }
      }
    }
    {
      // occupancy proposals for run-representative samples (ffnerf_OG.cl:1640-1821); every wavefront
      // holds the whole ray here, and one per tile (rotating) makes the proposals of all 64 samples
      if (proposals && prop_wave) {
        const int nxt = find_next_flag(segmask, lid, S);
        const int prev_end = lid > 0 ? lid - 1 : 0;
        const int last = nxt < S ? nxt - 1 : S - 1;
        const int nsrc = nxt < S ? nxt : lid;
        const float t_prev = __shfl(t_j, base + prev_end), T_prev = __shfl(Tr, base + prev_end);
        const float t_last = __shfl(t_j, base + last), T_last = __shfl(Tr, base + last);
        const float t_nx = __shfl(t_j, base + nsrc), T_nx = __shfl(Tr, base + nsrc);
        const bool is_rep = (segmask >> lid) & 1ull;
        // Early out, exact: transmittance never rises along the ray, so the run's predicted absorption
        // pred = 1 - T_exit / T_enter below is at most (T_prev - T_next) / T_prev.  When 16 times that bound
        // cannot exceed the smallest level in the cell's occupancy word, no subcell of the cell can take a
        // proposal, and the lane would neither draw nor write.  The scan's products may exceed monotonicity
        // by a few ulps (< 1e-6 relative); the 1e-4 margin covers that, so only such lanes are skipped.
        uint32_t wmin = 15u;  // smallest nibble of the word (its subcells' level - 1)
#pragma unroll
        for (int q = 0; q < 8; ++q) wmin = min(wmin, (L.occ_word >> (4 * q)) & 0xFu);
        const float T_nb = nxt < S ? T_nx : T_final;
        const bool may_rise = 16.0f * (T_prev - T_nb) > (float)(wmin + 1u) * T_prev * (1.0f - 1.0e-4f);
        if (vj && is_rep && dt_j > 0.0f && may_rise) {
          const float4 ro = a.rays[2 * rj], rdv = a.rays[2 * rj + 1];
          const float o[3] = {ro.x, ro.y, ro.z}, d[3] = {rdv.x, rdv.y, rdv.z};
          occ_propose_run(c, o, d, t_j, Tr, t_prev, T_prev, t_last, T_last, nxt < S, t_nx, T_nx, T_final, L.occ_word,
                          a.seed, (uint32_t)rj, (uint32_t)lid, Dhalf, a.occ_st);
        }
      }
    }
  }
}

// Output deltas of one sample (ffnerf_OG.cl:1863-1914): colour-head pre-activation deltas dco[0..2] and the
// density-head delta dd0 (the other 15 density outputs get none), scaled by the distance gate f_vol.
__device__ __forceinline__ void output_deltas(float t_b, float dt_b, float Dhalf, float dLds, float dLdc0,
                                              float dLdc1, float dLdc2, const float (&rgb_s)[3], float dout0,
                                              float (&dco)[3], float& dd0) {
  // hardware reciprocal, exp2 and log2 (about 1 ulp each) in place of division and powf
  const float num = t_b * t_b + t_b * dt_b + dt_b * dt_b * (1.0f / 3.0f);
  const float den = Dhalf * Dhalf + Dhalf * dt_b + dt_b * dt_b * (1.0f / 3.0f);
  const float xg = t_b * fast_rcp(fmaxf(Dhalf, 1.0e-12f));
  const float sg = (xg >= 1.0f) ? 0.0f : 1.0f;
  const float pw = __builtin_amdgcn_exp2f(0.2f * __builtin_amdgcn_logf(fmaxf(xg, 1.0e-12f)));  // xg^0.2
  const float gate = (1.0f - sg) * 1.0f + sg * pw;
  const float f_vol = gate * num * fast_rcp(fmaxf(den, 1.0e-12f));
  dco[0] = (f_vol * dLdc0) * ((rgb_s[0] * (1.0f - rgb_s[0])) * 0.5f);
  dco[1] = (f_vol * dLdc1) * ((rgb_s[1] * (1.0f - rgb_s[1])) * 0.5f);
  dco[2] = (f_vol * dLdc2) * ((rgb_s[2] * (1.0f - rgb_s[2])) * 0.5f);
  dd0 = 1.0f * (f_vol * dLds) * softplus_prime_from_pre(fminf(fmaxf(dout0, -18.0f), 18.0f));
}

// dL/da0 of this lane's sample b: tile t holds encoding neurons 16t + 4g + r (level n / F, feature n % F)
template <int LF, int FEAT>
__device__ __forceinline__ void store_enc_grad(const MlpArgs& a, int64_t b, int g, const floatx4 (&ga)[LF / 16]) {
#pragma unroll
  for (int t = 0; t < LF / 16; ++t) {
#pragma unroll
    for (int r = 0; r < 4; r += 2) {  // neurons 16t+4g+r, r+1: one level when F >= 2
      const int nn = 16 * t + 4 * g + r;
      const int l = nn / FEAT, f = nn - l * FEAT;
      float* dst = a.dL_da0 + l * a.feat.stride_l + b * a.feat.stride_b + f;
      if constexpr (FEAT >= 2) {
        *reinterpret_cast<float2*>(dst) = make_float2(ga[t][r], ga[t][r + 1]);
      } else {
        dst[0] = ga[t][r];
        a.dL_da0[(l + 1) * a.feat.stride_l + b * a.feat.stride_b] = ga[t][r + 1];
      }
    }
  }
}

// A tile whose samples are all inactive (dt <= 0, e.g. a ray that misses the box) composites to exactly
// the background (every alpha is 0, so T = 1 and the colour sum is 0) and every gradient of its samples is
// zero; this writes what the full path would write for it -- the rays' colours and zero encoding
// gradients -- so the MLP can be skipped.  Taps, which expose per-sample MLP outputs, take the full path.
template <int LF, int FEAT, int SC>
__device__ __forceinline__ void empty_tile(const MlpArgs& a, const CompLane& L, int lane, int wave, int64_t b,
                                           bool valid, bool train, int g) {
  const int lid = lane & ((SC > 0 ? SC : a.S) - 1);
  if (wave == 0 && lid == 0 && L.vj) {
    float bg[3];
    background(a, L.rj, train, bg);
    a.out_rgb[L.rj] = make_float4(fminf(fmaxf(bg[0], 0.0f), 1.0f), fminf(fmaxf(bg[1], 0.0f), 1.0f),
                                  fminf(fmaxf(bg[2], 0.0f), 1.0f), train ? 4.0f : 0.0f);
  }
  if (train && valid) {
    floatx4 z[LF / 16];
#pragma unroll
    for (int t = 0; t < LF / 16; ++t) z[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    store_enc_grad<LF, FEAT>(a, b, g, z);
  }
}

// Whether any per-sample tap is bound.  The MLP kernels take it as a template parameter (TAPS): without
// taps the tap pointers and their tests leave the kernel, which keeps its scalar registers within the
// hardware's limit (the test-only taps otherwise cost spills to vector-register lanes in every tile).
__host__ __device__ __forceinline__ bool taps_requested(const MlpArgs& a) {
  return a.t_sigma || a.t_rgb || a.t_Tr || a.t_Tfinal || a.t_dLds || a.t_dLdc || a.t_relu || a.t_color;
}

// ReLU-branch tap of hidden layer slot h (0..2 density, 3..6 colour) for this lane's sample: bit n of the
// record's words 2h, 2h + 1 is set when unit n's activation (as the backward reads it) is positive.  Lane
// (g, s) holds units 16t + 4g + r; the four lane groups of a sample combine their bits.  Every lane of the
// wavefront must call this (rec may be NULL for lanes without a sample).
template <typename V>
__device__ __forceinline__ void tap_relu(uint32_t* rec, int h, const V (&act)[4], int g) {
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t on = (float)act[t][r] > 0.0f ? 1u : 0u;
      const int n = 16 * t + 4 * g + r;
      if (t < 2) lo |= on << (n & 31);
      else hi |= on << (n & 31);
    }
  lo |= __shfl_xor(lo, 16);
  lo |= __shfl_xor(lo, 32);
  hi |= __shfl_xor(hi, 16);
  hi |= __shfl_xor(hi, 32);
  if (rec && g == 0) {
    rec[2 * h] = lo;
    rec[2 * h + 1] = hi;
  }
}

// Weight-gradient tiles (T, Tp) of one layer (OT x IT tiles of 16x16) dealt over the four wavefronts:
// wavefront w's m-th tile.  The tiles with Tp = 0 also sum the bias gradient, so they are spread: with
// IT = 4 (or 2) every wavefront holds one Tp = 0 tile per four (two) of its tiles.
template <int IT>
__device__ __forceinline__ void deal_tile(int m, int wave, int& T, int& Tp) {
  if constexpr (IT == 4) {
    T = m;
    Tp = (wave + m) & 3;
  } else if constexpr (IT == 2) {
    T = 2 * m + (wave >> 1);
    Tp = (wave + (wave >> 1) + m) & 1;
  } else {
    static_assert(IT == 1, "16, 32 or 64 input neurons per layer");
    T = 4 * m + wave;
    Tp = 0;
  }
}

}  // namespace ffn
