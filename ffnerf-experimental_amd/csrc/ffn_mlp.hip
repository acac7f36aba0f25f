// ffn_mlp.hip -- fused density+color MLP forward, volume compositing,
// photometric loss gradient, compositing backward, occupancy proposals, MLP
// backward and weight-gradient accumulation.
//
// Reference: ffnerf_OG.cl:1373-1466 (MLP fwd), 1505-1634 (compositing, loss,
// reverse affine scan), 1640-1821 (proposals), 1863-2082 (deltas, backward),
// weight_update.cl:210-341 (weight-gradient GEMM over the staged SoA buffers).
//
// MI355X design
//   * A 256-thread block (4 wavefronts) walks 64-sample tiles in a persistent
//     loop.  Each wavefront owns 16 samples of the tile and runs every layer
//     as 16x16x4 fp32 MFMAs with the samples as the N dimension
//     (out[o][s] = W[o][:] . act[:][s]).
//   * An MFMA result tile leaves lane (g, s) holding neurons 16t+4g+r of
//     sample s.  The next layer consumes it unchanged: its K index is
//     permuted so that k-step (t, r) takes neuron 16t+4g+r from lane group g
//     and the weights are read with the same permutation.  Activations and
//     deltas therefore never move between lanes.
//   * Compositing needs the whole ray: sigma/rgb go to LDS, one barrier, and
//     every wavefront runs the reference's scan trees on 64 lanes (one lane
//     per sample, S lanes per ray) and picks its own samples' gradients.
//   * Weight gradients dW = sum_s delta[o][s] act[i][s] are MFMAs with the
//     samples as K: each 16x16 tile is transposed through a per-wave LDS
//     scratch (4 ds_write_b32 + 1 ds_read_b128) and accumulated with
//     ds_add_f32 into a per-block LDS copy of the gradient; each block writes
//     one partial at the end (no staging buffers in HBM, unlike the
//     reference's ~1.8 KB/sample SoA traffic).
#include "ffn_device.h"
#include "ffn_kernels.h"
#include "ffn_mlp_common.h"

namespace ffn {

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int LF_, int ND_, int NC_>
struct Arch {
  static constexpr int LF = LF_, ND = ND_, NC = NC_;
  static constexpr int rows_pad(int k) { return k == FFN_WC_OUT ? 16 : layer_out(k); }
  static constexpr int pitch(int k) { return layer_in(k, LF) + 1; }
  static constexpr int wsz(int k) { return layer_active(k, ND, NC) ? rows_pad(k) * pitch(k) + rows_pad(k) : 0; }
  static constexpr int w_off(int k) {
    int o = 0;
    for (int j = 0; j < k; ++j) o += wsz(j);
    return o;
  }
  static constexpr int b_off(int k) { return w_off(k) + rows_pad(k) * pitch(k); }
  static constexpr int w_total() { return w_off(FFN_N_LAYERS); }
  static constexpr int gsz(int k) {
    return layer_active(k, ND, NC) ? layer_out(k) * layer_in(k, LF) + layer_out(k) : 0;
  }
  static constexpr int g_off(int k) {
    int o = 0;
    for (int j = 0; j < k; ++j) o += gsz(j);
    return o;
  }
  static constexpr int gb_off(int k) { return g_off(k) + layer_out(k) * layer_in(k, LF); }
  static constexpr int g_total() { return g_off(FFN_N_LAYERS); }
  static constexpr int XP = 20;  // transpose scratch pitch: 16 samples + 4 pad
  static constexpr int x_per_wave = 64 * XP;
  static constexpr int comp_floats = 2 * 256;  // double-buffered sigma[64] + rgb[64][3]
  static constexpr int lds_floats() { return w_total() + g_total() + 4 * x_per_wave + comp_floats; }
};

// out tiles (D layout) = act(W . in + b), in given as D-layout tiles.  The
// output tiles are interleaved inside each k-step so consecutive MFMAs are
// independent.
template <int OT, int IT>
__device__ __forceinline__ void fwd_tiles(const float* __restrict__ W, const float* __restrict__ B, int P,
                                          const floatx4 (&in)[IT], floatx4 (&out)[OT], int g, int s, bool relu) {
  floatx4 acc[OT];
#pragma unroll
  for (int t = 0; t < OT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[t][r] = B[16 * t + 4 * g + r];
  const float* wrow = W + s * P + 4 * g;
#pragma unroll
  for (int tp = 0; tp < IT; ++tp)
#pragma unroll
    for (int rp = 0; rp < 4; ++rp)
#pragma unroll
      for (int t = 0; t < OT; ++t) acc[t] = mfma4(wrow[16 * t * P + 16 * tp + rp], in[tp][rp], acc[t]);
#pragma unroll
  for (int t = 0; t < OT; ++t) {
    if (relu) {
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[t][r] = acc[t][r] > 0.0f ? acc[t][r] : 0.0f;
    }
    out[t] = acc[t];
  }
}

// res tiles (D layout over input neurons, first RT tiles) = W^T . delta (+ init)
template <int RT, int DT>
__device__ __forceinline__ void bwd_tiles(const float* __restrict__ W, int P, const floatx4 (&delta)[DT],
                                          floatx4 (&res)[RT], int g, int s) {
#pragma unroll
  for (int tp = 0; tp < DT; ++tp)
#pragma unroll
    for (int rp = 0; rp < 4; ++rp)
#pragma unroll
      for (int t = 0; t < RT; ++t) res[t] = mfma4(W[(16 * tp + 4 * g + rp) * P + 16 * t + s], delta[tp][rp], res[t]);
}

template <int NT>
__device__ __forceinline__ void relu_mask(floatx4 (&d)[NT], const floatx4 (&act)[NT]) {
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) d[t][r] = act[t][r] > 0.0f ? d[t][r] : 0.0f;
}

template <int NT>
__device__ __forceinline__ void stash_D(float* __restrict__ sx, const floatx4 (&v)[NT], int g, int s) {
  constexpr int XP = 20;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) sx[(16 * t + 4 * g + r) * XP + s] = v[t][r];
}

template <int NT>
__device__ __forceinline__ void load_op(const float* __restrict__ sx, floatx4 (&op)[NT], int g, int m) {
  constexpr int XP = 20;
#pragma unroll
  for (int t = 0; t < NT; ++t) op[t] = *reinterpret_cast<const floatx4*>(sx + (16 * t + m) * XP + 4 * g);
}

// dW[o][i] += sum_s delta[o][s] act[i][s] and db[o] += sum_s delta[o][s] over the wave's 16 samples.
// dop: delta operands (OT tiles), aop: activation operands (IT tiles), already transposed.
template <int OT, int IT>
__device__ __forceinline__ void accum_dW(float* __restrict__ gW, float* __restrict__ gB, int out_dim, int in_dim,
                                         const floatx4 (&dop)[OT], const floatx4 (&aop)[IT], int g, int s) {
#pragma unroll
  for (int T = 0; T < OT; ++T) {
    float bs = (dop[T][0] + dop[T][1]) + (dop[T][2] + dop[T][3]);
    bs += __shfl_xor(bs, 16);
    bs += __shfl_xor(bs, 32);
    if (g == 0 && 16 * T + s < out_dim) atomicAdd(gB + 16 * T + s, bs);
  }
#pragma unroll
  for (int T = 0; T < OT; ++T) {
#pragma unroll
    for (int Tp = 0; Tp < IT; ++Tp) {
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) acc = mfma4(dop[T][q], aop[Tp][q], acc);
      const int col = 16 * Tp + s;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * T + 4 * g + r;
        if (row < out_dim && col < in_dim) atomicAdd(gW + row * in_dim + col, acc[r]);
      }
    }
  }
}

// Weight-gradient accumulators of one layer held in registers (AGPRs) for all
// the tiles a wavefront processes: w[T][Tp] is the D-layout 16x16 tile
// (rows 16T + 4g + r, columns 16Tp + lane%16), b[T] a per-lane partial bias sum.
template <int OT, int IT>
struct GradAcc {
  floatx4 w[OT][IT];
  float b[OT];
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int T = 0; T < OT; ++T) {
      b[T] = 0.0f;
#pragma unroll
      for (int Tp = 0; Tp < IT; ++Tp) w[T][Tp] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // dW += delta . act^T and db += delta over the wave's 16 samples (operands already transposed)
  __device__ __forceinline__ void add(const floatx4 (&dop)[OT], const floatx4 (&aop)[IT]) {
#pragma unroll
    for (int T = 0; T < OT; ++T) b[T] += (dop[T][0] + dop[T][1]) + (dop[T][2] + dop[T][3]);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int T = 0; T < OT; ++T)
#pragma unroll
        for (int Tp = 0; Tp < IT; ++Tp) w[T][Tp] = mfma4(dop[T][q], aop[Tp][q], w[T][Tp]);
  }
  // add this wavefront's sums into the block's LDS gradient (callers serialise the waves)
  __device__ __forceinline__ void flush(float* __restrict__ gW, float* __restrict__ gB, int out_dim, int in_dim,
                                        int g, int s) {
#pragma unroll
    for (int T = 0; T < OT; ++T) {
      float bs = b[T];
      bs += __shfl_xor(bs, 16);
      bs += __shfl_xor(bs, 32);
      if (g == 0 && 16 * T + s < out_dim) gB[16 * T + s] += bs;
#pragma unroll
      for (int Tp = 0; Tp < IT; ++Tp) {
        const int col = 16 * Tp + s;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * T + 4 * g + r;
          if (row < out_dim && col < in_dim) gW[row * in_dim + col] += w[T][Tp][r];
        }
      }
    }
  }
};

template <int OT, int IT>
__device__ __forceinline__ void transpose_ops(float* __restrict__ sx, const floatx4 (&delta)[OT],
                                              const floatx4 (&act)[IT], floatx4 (&dop)[OT], floatx4 (&aop)[IT],
                                              int g, int s) {
  stash_D(sx, delta, g, s);
  wave_lds_sync();
  load_op(sx, dop, g, s);
  wave_lds_sync();
  stash_D(sx, act, g, s);
  wave_lds_sync();
  load_op(sx, aop, g, s);
  wave_lds_sync();
}

template <int OT, int IT>
__device__ __forceinline__ void layer_grad_reg(float* __restrict__ sx, GradAcc<OT, IT>& acc,
                                               const floatx4 (&delta)[OT], const floatx4 (&act)[IT], int g, int s) {
  floatx4 dop[OT], aop[IT];
  transpose_ops(sx, delta, act, dop, aop, g, s);
  acc.add(dop, aop);
}

template <int OT, int IT>
__device__ __forceinline__ void layer_grad(float* __restrict__ sx, float* __restrict__ gW, float* __restrict__ gB,
                                           int out_dim, int in_dim, const floatx4 (&delta)[OT],
                                           const floatx4 (&act)[IT], int g, int s) {
  floatx4 dop[OT], aop[IT];
  stash_D(sx, delta, g, s);
  wave_lds_sync();
  load_op(sx, dop, g, s);
  wave_lds_sync();
  stash_D(sx, act, g, s);
  wave_lds_sync();
  load_op(sx, aop, g, s);
  wave_lds_sync();
  accum_dW(gW, gB, out_dim, in_dim, dop, aop, g, s);
}

// Register-resident gradient accumulators of every layer (used when they fit:
// at most 48 16x16 tiles = 192 AGPRs per lane); otherwise the block
// accumulates in LDS.
template <int LF, int ND, int NC>
constexpr int acc_tiles() {
  return 4 + 16 * (NC - 1) + 8 + 4 + 16 * (ND - 1) + 4 * (LF / 16);
}

template <int LF, int ND, int NC, bool REG>
struct AccSet {
  __device__ __forceinline__ void zero() {}
};
template <int LF, int ND, int NC>
struct AccSet<LF, ND, NC, true> {
  GradAcc<1, 4> c_out;
  GradAcc<4, 4> c_h[NC > 1 ? NC - 1 : 1];  // Wc_01, Wc_12, Wc_23
  GradAcc<4, 2> c_in;
  GradAcc<1, 4> d_out;
  GradAcc<4, 4> d_h[ND > 1 ? ND - 1 : 1];  // Wd_01, Wd_12
  GradAcc<4, LF / 16> d_in;
  __device__ __forceinline__ void zero() {
    c_out.zero();
#pragma unroll
    for (int i = 0; i < NC - 1; ++i) c_h[i].zero();
    c_in.zero();
    d_out.zero();
#pragma unroll
    for (int i = 0; i < ND - 1; ++i) d_h[i].zero();
    d_in.zero();
  }
};

// stage the weights of every active layer into LDS (zero-padded rows, pitch in+1)
template <int LF, int ND, int NC>
__device__ __forceinline__ void stage_weights(float* __restrict__ sW, const MlpPtrs& wp, int tid, int nthreads) {
  using A = Arch<LF, ND, NC>;
#pragma unroll
  for (int k = 0; k < FFN_N_LAYERS; ++k) {
    if (!layer_active(k, ND, NC)) continue;
    const int O = layer_out(k), I = layer_in(k, LF), R = A::rows_pad(k), P = A::pitch(k);
    float* w = sW + A::w_off(k);
    float* bb = sW + A::b_off(k);
    const float* gw = wp.W[k];
    const float* gbias = wp.b[k];
    for (int e = tid; e < R * P; e += nthreads) {
      const int r = e / P, col = e - r * P;
      w[e] = (r < O && col < I) ? gw[r * I + col] : 0.0f;
    }
    for (int e = tid; e < R; e += nthreads) bb[e] = e < O ? gbias[e] : 0.0f;
  }
}

// a0r[kk] = encoding neuron (LF/4) g + kk (= level n / F, feature n % F) of sample b
template <int LF, int FEAT>
__device__ __forceinline__ void load_a0(const float* __restrict__ a0, const FeatLayout& feat, int64_t b, bool valid,
                                        int g, float (&a0r)[LF / 4]) {
  constexpr int KA = LF / 4;
  if (valid) {
    if constexpr (FEAT >= 2 && KA % 2 == 0) {
#pragma unroll
      for (int kk = 0; kk < KA; kk += 2) {
        const int nn = KA * g + kk;
        const int l = nn / FEAT, f = nn - l * FEAT;
        const float2 v = *reinterpret_cast<const float2*>(a0 + l * feat.stride_l + b * feat.stride_b + f);
        a0r[kk] = v.x;
        a0r[kk + 1] = v.y;
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < KA; ++kk) {
        const int nn = KA * g + kk;
        const int l = nn / FEAT, f = nn - l * FEAT;
        a0r[kk] = a0[l * feat.stride_l + b * feat.stride_b + f];
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < KA; ++q) a0r[q] = 0.0f;
  }
}

// forward of the wavefront's 16 samples through both MLPs (ffnerf_OG.cl:1373-1466): hidden activations
// (kept for the backward), the colour-net input [dout | SH * mult] and the sigmoid colours
template <int LF, int ND, int NC>
__device__ __forceinline__ void mlp_fwd_tile(const float* __restrict__ sW, const float (&a0r)[LF / 4],
                                             const float (&dirv)[3], float sh_mult, int g, int s,
                                             floatx4 (&hd)[ND][4], floatx4 (&acin)[2], floatx4 (&hc)[NC][4],
                                             float (&rgb_s)[3]) {
  using A = Arch<LF, ND, NC>;
  constexpr int KA = LF / 4;
  {
    const float* W = sW + A::w_off(FFN_WD_IN);
    const float* B = sW + A::b_off(FFN_WD_IN);
    constexpr int P = A::pitch(FFN_WD_IN);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      floatx4 acc;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = B[16 * t + 4 * g + r];
      const float* wrow = W + (16 * t + s) * P + KA * g;
#pragma unroll
      for (int kk = 0; kk < KA; ++kk) acc = mfma4(wrow[kk], a0r[kk], acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = acc[r] > 0.0f ? acc[r] : 0.0f;
      hd[0][t] = acc;
    }
  }
  if constexpr (ND >= 2)
    fwd_tiles<4, 4>(sW + A::w_off(FFN_WD_01), sW + A::b_off(FFN_WD_01), A::pitch(FFN_WD_01), hd[0], hd[1], g, s,
                    true);
  if constexpr (ND >= 3)
    fwd_tiles<4, 4>(sW + A::w_off(FFN_WD_12), sW + A::b_off(FFN_WD_12), A::pitch(FFN_WD_12), hd[1], hd[2], g, s,
                    true);
  {
    floatx4 o1[1];
    fwd_tiles<1, 4>(sW + A::w_off(FFN_WD_OUT), sW + A::b_off(FFN_WD_OUT), A::pitch(FFN_WD_OUT), hd[ND - 1], o1, g,
                    s, false);
    acin[0] = o1[0];
#pragma unroll
    for (int r = 0; r < 4; ++r) acin[1][r] = sh_component(dirv, 4 * g + r) * sh_mult;
  }
  fwd_tiles<4, 2>(sW + A::w_off(FFN_WC_IN), sW + A::b_off(FFN_WC_IN), A::pitch(FFN_WC_IN), acin, hc[0], g, s, true);
  if constexpr (NC >= 2)
    fwd_tiles<4, 4>(sW + A::w_off(FFN_WC_01), sW + A::b_off(FFN_WC_01), A::pitch(FFN_WC_01), hc[0], hc[1], g, s,
                    true);
  if constexpr (NC >= 3)
    fwd_tiles<4, 4>(sW + A::w_off(FFN_WC_12), sW + A::b_off(FFN_WC_12), A::pitch(FFN_WC_12), hc[1], hc[2], g, s,
                    true);
  if constexpr (NC >= 4)
    fwd_tiles<4, 4>(sW + A::w_off(FFN_WC_23), sW + A::b_off(FFN_WC_23), A::pitch(FFN_WC_23), hc[2], hc[3], g, s,
                    true);
  floatx4 co[1];
  fwd_tiles<1, 4>(sW + A::w_off(FFN_WC_OUT), sW + A::b_off(FFN_WC_OUT), A::pitch(FFN_WC_OUT), hc[NC - 1], co, g, s,
                  false);
  rgb_s[0] = sigmoid_soft(co[0][0]);
  rgb_s[1] = sigmoid_soft(co[0][1]);
  rgb_s[2] = sigmoid_soft(co[0][2]);
}

template <int LF, int ND, int NC, int FEAT>
__global__ __launch_bounds__(256, 1) void k_mlp(MlpArgs a) {
  using A = Arch<LF, ND, NC>;
  constexpr int KA = LF / 4;  // a0 values per lane (k-steps of the first layer)
  extern __shared__ float smem[];
  float* sW = smem;
  float* sG = smem + A::w_total();
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
  float* sX = sG + A::g_total() + wave * A::x_per_wave;
  float* sC = smem + A::w_total() + A::g_total() + 4 * A::x_per_wave;
  const bool train = a.do_train != 0;
  const DevCfg& c = a.c;
  const int S = a.S, log2S = a.log2S;
  const uint64_t n_samples = (uint64_t)a.num_rays << log2S;

  // stage weights and clear the gradient accumulators
  stage_weights<LF, ND, NC>(sW, a.w, tid, 256);
  if (train)
    for (int e = tid; e < A::g_total(); e += 256) sG[e] = 0.0f;
  __syncthreads();

  const float Dhalf = half_box_diagonal(c);
  const bool proposals = train && a.occ_strength > 0.0f;

  constexpr bool REG_ACC = acc_tiles<LF, ND, NC>() <= 48;
  AccSet<LF, ND, NC, REG_ACC> ga;
  ga.zero();

  int parity = 0;
  for (int64_t tile = blockIdx.x; tile < a.n_tiles; tile += gridDim.x, parity ^= 1) {
    float* sSig = sC + parity * 256;
    float* sRgb = sSig + 64;
    // ------------------------------------------------------------------
    // forward: this lane's sample in the MLP layout
    const int64_t b = tile * 64 + wave * 16 + s;
    const bool valid = (uint64_t)b < n_samples;
    const int64_t ray = valid ? (b >> log2S) : 0;
    float a0r[KA];
    load_a0<LF, FEAT>(a.a0, a.feat, b, valid, g, a0r);
    float dirv[3];
    {
      const float4 rd = a.rays[2 * ray + 1];
      dirv[0] = rd.x;
      dirv[1] = rd.y;
      dirv[2] = rd.z;
    }
    const float dt_b = valid ? a.DTs[b] : 0.0f;
    const float t_b = valid ? a.Ts[b] : 0.0f;
    // per-sample inputs of the compositing (lane j = sample j of the tile), loaded before the forward so
    // that their latency hides behind it
    const CompLane CL = load_comp_lane(a, tile, lane, wave, n_samples, log2S, proposals);

    floatx4 hd[ND][4];
    floatx4 acin[2];  // [dout(16) | SH*mult(16)] as two D-layout tiles
    floatx4 hc[NC][4];
    float rgb_s[3];
    mlp_fwd_tile<LF, ND, NC>(sW, a0r, dirv, a.sh_mult, g, s, hd, acin, hc, rgb_s);
    const float dout0 = acin[0][0];
    if (g == 0) {
      float sig = softplus(fminf(fmaxf(dout0, -10.0f), 10.0f));
      if (dt_b <= 0.0f) sig = 0.0f;
      sSig[wave * 16 + s] = sig;
      sRgb[(wave * 16 + s) * 3 + 0] = rgb_s[0];
      sRgb[(wave * 16 + s) * 3 + 1] = rgb_s[1];
      sRgb[(wave * 16 + s) * 3 + 2] = rgb_s[2];
    }
    __syncthreads();

    // ------------------------------------------------------------------
    // compositing on 64 lanes: lane j = sample j of the tile (every wave)
    float dLds_j, dLdc_j[3];
    composite_tile(a, sSig, sRgb, CL, lane, wave, train, proposals, Dhalf, dLds_j, dLdc_j);
    if (!train) continue;

    // ------------------------------------------------------------------
    // backward of this wave's 16 samples
    const int src = wave * 16 + s;
    const float dLds = __shfl(dLds_j, src);
    const float dLdc0 = __shfl(dLdc_j[0], src), dLdc1 = __shfl(dLdc_j[1], src), dLdc2 = __shfl(dLdc_j[2], src);
    floatx4 dco[1] = {{0.f, 0.f, 0.f, 0.f}};
    floatx4 ddo[1] = {{0.f, 0.f, 0.f, 0.f}};
    if (g == 0 && valid) {
      float d3[3], dd0;
      output_deltas(t_b, dt_b, Dhalf, dLds, dLdc0, dLdc1, dLdc2, rgb_s, dout0, d3, dd0);
      dco[0][0] = d3[0];
      dco[0][1] = d3[1];
      dco[0][2] = d3[2];
      ddo[0][0] = dd0;
    }
    // color backward
    floatx4 dc[NC][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) dc[NC - 1][t] = floatx4{0.f, 0.f, 0.f, 0.f};
    bwd_tiles<4, 1>(sW + A::w_off(FFN_WC_OUT), A::pitch(FFN_WC_OUT), dco, dc[NC - 1], g, s);
    relu_mask(dc[NC - 1], hc[NC - 1]);
    if constexpr (REG_ACC) layer_grad_reg(sX, ga.c_out, dco, hc[NC - 1], g, s);
    else layer_grad<1, 4>(sX, sG + A::g_off(FFN_WC_OUT), sG + A::gb_off(FFN_WC_OUT), FFN_C_OUT, FFN_M, dco,
                          hc[NC - 1], g, s);
    if constexpr (NC >= 4) {
#pragma unroll
      for (int t = 0; t < 4; ++t) dc[2][t] = floatx4{0.f, 0.f, 0.f, 0.f};
      bwd_tiles<4, 4>(sW + A::w_off(FFN_WC_23), A::pitch(FFN_WC_23), dc[3], dc[2], g, s);
      relu_mask(dc[2], hc[2]);
      if constexpr (REG_ACC) layer_grad_reg(sX, ga.c_h[2], dc[3], hc[2], g, s);
      else layer_grad<4, 4>(sX, sG + A::g_off(FFN_WC_23), sG + A::gb_off(FFN_WC_23), FFN_M, FFN_M, dc[3], hc[2], g, s);
    }
    if constexpr (NC >= 3) {
#pragma unroll
      for (int t = 0; t < 4; ++t) dc[1][t] = floatx4{0.f, 0.f, 0.f, 0.f};
      bwd_tiles<4, 4>(sW + A::w_off(FFN_WC_12), A::pitch(FFN_WC_12), dc[2], dc[1], g, s);
      relu_mask(dc[1], hc[1]);
      if constexpr (REG_ACC) layer_grad_reg(sX, ga.c_h[1], dc[2], hc[1], g, s);
      else layer_grad<4, 4>(sX, sG + A::g_off(FFN_WC_12), sG + A::gb_off(FFN_WC_12), FFN_M, FFN_M, dc[2], hc[1], g, s);
    }
    if constexpr (NC >= 2) {
#pragma unroll
      for (int t = 0; t < 4; ++t) dc[0][t] = floatx4{0.f, 0.f, 0.f, 0.f};
      bwd_tiles<4, 4>(sW + A::w_off(FFN_WC_01), A::pitch(FFN_WC_01), dc[1], dc[0], g, s);
      relu_mask(dc[0], hc[0]);
      if constexpr (REG_ACC) layer_grad_reg(sX, ga.c_h[0], dc[1], hc[0], g, s);
      else layer_grad<4, 4>(sX, sG + A::g_off(FFN_WC_01), sG + A::gb_off(FFN_WC_01), FFN_M, FFN_M, dc[1], hc[0], g, s);
    }
    // color input layer: its gradient, and the dout part of its input delta
    if constexpr (REG_ACC) layer_grad_reg(sX, ga.c_in, dc[0], acin, g, s);
    else layer_grad<4, 2>(sX, sG + A::g_off(FFN_WC_IN), sG + A::gb_off(FFN_WC_IN), FFN_M, FFN_C_IN, dc[0], acin, g, s);
    bwd_tiles<1, 4>(sW + A::w_off(FFN_WC_IN), A::pitch(FFN_WC_IN), dc[0], ddo, g, s);
    // density backward
    floatx4 dd[ND][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) dd[ND - 1][t] = floatx4{0.f, 0.f, 0.f, 0.f};
    bwd_tiles<4, 1>(sW + A::w_off(FFN_WD_OUT), A::pitch(FFN_WD_OUT), ddo, dd[ND - 1], g, s);
    relu_mask(dd[ND - 1], hd[ND - 1]);
    if constexpr (REG_ACC) layer_grad_reg(sX, ga.d_out, ddo, hd[ND - 1], g, s);
    else layer_grad<1, 4>(sX, sG + A::g_off(FFN_WD_OUT), sG + A::gb_off(FFN_WD_OUT), FFN_D_OUT, FFN_M, ddo,
                          hd[ND - 1], g, s);
    if constexpr (ND >= 3) {
#pragma unroll
      for (int t = 0; t < 4; ++t) dd[1][t] = floatx4{0.f, 0.f, 0.f, 0.f};
      bwd_tiles<4, 4>(sW + A::w_off(FFN_WD_12), A::pitch(FFN_WD_12), dd[2], dd[1], g, s);
      relu_mask(dd[1], hd[1]);
      if constexpr (REG_ACC) layer_grad_reg(sX, ga.d_h[1], dd[2], hd[1], g, s);
      else layer_grad<4, 4>(sX, sG + A::g_off(FFN_WD_12), sG + A::gb_off(FFN_WD_12), FFN_M, FFN_M, dd[2], hd[1], g, s);
    }
    if constexpr (ND >= 2) {
#pragma unroll
      for (int t = 0; t < 4; ++t) dd[0][t] = floatx4{0.f, 0.f, 0.f, 0.f};
      bwd_tiles<4, 4>(sW + A::w_off(FFN_WD_01), A::pitch(FFN_WD_01), dd[1], dd[0], g, s);
      relu_mask(dd[0], hd[0]);
      if constexpr (REG_ACC) layer_grad_reg(sX, ga.d_h[0], dd[1], hd[0], g, s);
      else layer_grad<4, 4>(sX, sG + A::g_off(FFN_WD_01), sG + A::gb_off(FFN_WD_01), FFN_M, FFN_M, dd[1], hd[0], g, s);
    }
    // encoding gradient dL/da0 = Wd_in^T . delta_d1 -> HBM for the hash scatter
    {
      floatx4 ga[LF / 16];
#pragma unroll
      for (int t = 0; t < LF / 16; ++t) ga[t] = floatx4{0.f, 0.f, 0.f, 0.f};
      bwd_tiles<LF / 16, 4>(sW + A::w_off(FFN_WD_IN), A::pitch(FFN_WD_IN), dd[0], ga, g, s);
      if (valid) {
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
    }
    // first-layer weight gradient: a0 is held with the permuted neuron order
    {
      floatx4 dop[4], aop[LF / 16];
      stash_D(sX, dd[0], g, s);
      wave_lds_sync();
      load_op(sX, dop, g, s);
      wave_lds_sync();
#pragma unroll
      for (int kk = 0; kk < KA; ++kk) sX[(KA * g + kk) * A::XP + s] = a0r[kk];
      wave_lds_sync();
      load_op(sX, aop, g, s);
      wave_lds_sync();
      if constexpr (REG_ACC) ga.d_in.add(dop, aop);
      else accum_dW(sG + A::g_off(FFN_WD_IN), sG + A::gb_off(FFN_WD_IN), FFN_M, LF, dop, aop, g, s);
    }
  }

  if (train) {
    if constexpr (REG_ACC) {
      // add the four wavefronts' register sums into the block's LDS gradient, one wave at a time
      for (int w = 0; w < 4; ++w) {
        __syncthreads();
        if (wave == w) {
          ga.c_out.flush(sG + A::g_off(FFN_WC_OUT), sG + A::gb_off(FFN_WC_OUT), FFN_C_OUT, FFN_M, g, s);
          if constexpr (NC >= 2) ga.c_h[0].flush(sG + A::g_off(FFN_WC_01), sG + A::gb_off(FFN_WC_01), FFN_M, FFN_M, g, s);
          if constexpr (NC >= 3) ga.c_h[1].flush(sG + A::g_off(FFN_WC_12), sG + A::gb_off(FFN_WC_12), FFN_M, FFN_M, g, s);
          if constexpr (NC >= 4) ga.c_h[2].flush(sG + A::g_off(FFN_WC_23), sG + A::gb_off(FFN_WC_23), FFN_M, FFN_M, g, s);
          ga.c_in.flush(sG + A::g_off(FFN_WC_IN), sG + A::gb_off(FFN_WC_IN), FFN_M, FFN_C_IN, g, s);
          ga.d_out.flush(sG + A::g_off(FFN_WD_OUT), sG + A::gb_off(FFN_WD_OUT), FFN_D_OUT, FFN_M, g, s);
          if constexpr (ND >= 2) ga.d_h[0].flush(sG + A::g_off(FFN_WD_01), sG + A::gb_off(FFN_WD_01), FFN_M, FFN_M, g, s);
          if constexpr (ND >= 3) ga.d_h[1].flush(sG + A::g_off(FFN_WD_12), sG + A::gb_off(FFN_WD_12), FFN_M, FFN_M, g, s);
          ga.d_in.flush(sG + A::g_off(FFN_WD_IN), sG + A::gb_off(FFN_WD_IN), FFN_M, LF, g, s);
        }
      }
    }
    __syncthreads();
    float* dst = a.partials + (int64_t)blockIdx.x * A::g_total();
    for (int e = tid; e < A::g_total(); e += 256) dst[e] = sG[e];
  }
}

// ---------------------------------------------------------------------------

template <int LF, int ND, int NC, int FEAT>
static hipError_t launch_f(const MlpArgs& a, int n_blocks, hipStream_t st) {
  using A = Arch<LF, ND, NC>;
  const size_t lds = sizeof(float) * (size_t)A::lds_floats();
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)k_mlp<LF, ND, NC, FEAT>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((k_mlp<LF, ND, NC, FEAT>), dim3(n_blocks), dim3(256), lds, st, a);
  return hipGetLastError();
}

template <int LF, int ND, int NC>
static hipError_t launch_t(const MlpArgs& a, int n_blocks, hipStream_t st) {
  switch (a.c.F) {
    case 1: return launch_f<LF, ND, NC, 1>(a, n_blocks, st);
    case 2: return launch_f<LF, ND, NC, 2>(a, n_blocks, st);
    case 4: return launch_f<LF, ND, NC, 4>(a, n_blocks, st);
    default: return hipErrorInvalidValue;
  }
}

// forward only, over a flat list of samples (the render path): 16 samples per wavefront per step
template <int LF, int ND, int NC, int FEAT>
__global__ __launch_bounds__(256) void k_mlp_fwd(MlpPtrs wp, const float* __restrict__ a0, FeatLayout feat,
                                                 const float4* __restrict__ rays, const uint32_t* __restrict__ ray_ids,
                                                 int64_t n, float sh_mult, float* __restrict__ sigma,
                                                 float* __restrict__ rgb) {
  extern __shared__ float smem[];
  float* sW = smem;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
  stage_weights<LF, ND, NC>(sW, wp, tid, 256);
  __syncthreads();
  for (int64_t grp = (int64_t)blockIdx.x * 4 + wave; grp * 16 < n; grp += (int64_t)gridDim.x * 4) {
    const int64_t b = grp * 16 + s;
    const bool valid = b < n;
    float a0r[LF / 4];
    load_a0<LF, FEAT>(a0, feat, b, valid, g, a0r);
    float dirv[3] = {0.0f, 0.0f, 1.0f};
    if (valid) {
      const float4 rd = rays[2 * (size_t)ray_ids[b] + 1];
      dirv[0] = rd.x;
      dirv[1] = rd.y;
      dirv[2] = rd.z;
    }
    floatx4 hd[ND][4];
    floatx4 acin[2];
    floatx4 hc[NC][4];
    float rgb_s[3];
    mlp_fwd_tile<LF, ND, NC>(sW, a0r, dirv, sh_mult, g, s, hd, acin, hc, rgb_s);
    if (g == 0 && valid) {
      sigma[b] = softplus(fminf(fmaxf(acin[0][0], -10.0f), 10.0f));
      rgb[3 * b] = rgb_s[0];
      rgb[3 * b + 1] = rgb_s[1];
      rgb[3 * b + 2] = rgb_s[2];
    }
  }
}

template <int LF, int ND, int NC, int FEAT>
static hipError_t launch_fwd_f(const MlpPtrs& w, const float* a0, const FeatLayout& feat, const float4* rays,
                               const uint32_t* ray_ids, int64_t n, float sh_mult, float* sigma, float* rgb,
                               int n_blocks, hipStream_t st) {
  using A = Arch<LF, ND, NC>;
  const size_t lds = sizeof(float) * (size_t)A::w_total();
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)k_mlp_fwd<LF, ND, NC, FEAT>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((k_mlp_fwd<LF, ND, NC, FEAT>), dim3(n_blocks), dim3(256), lds, st, w, a0, feat, rays, ray_ids, n,
                     sh_mult, sigma, rgb);
  return hipGetLastError();
}

template <int LF, int ND, int NC>
static hipError_t launch_fwd_t(const DevCfg& c, const MlpPtrs& w, const float* a0, const FeatLayout& feat,
                               const float4* rays, const uint32_t* ray_ids, int64_t n, float sh_mult, float* sigma,
                               float* rgb, int n_blocks, hipStream_t st) {
  switch (c.F) {
    case 1: return launch_fwd_f<LF, ND, NC, 1>(w, a0, feat, rays, ray_ids, n, sh_mult, sigma, rgb, n_blocks, st);
    case 2: return launch_fwd_f<LF, ND, NC, 2>(w, a0, feat, rays, ray_ids, n, sh_mult, sigma, rgb, n_blocks, st);
    case 4: return launch_fwd_f<LF, ND, NC, 4>(w, a0, feat, rays, ray_ids, n, sh_mult, sigma, rgb, n_blocks, st);
    default: return hipErrorInvalidValue;
  }
}

#define FFN_MLP_CONFIGS(X) \
  X(16, 1, 2)              \
  X(32, 1, 2)              \
  X(64, 1, 2)              \
  X(16, 2, 2)              \
  X(32, 2, 2)              \
  X(64, 2, 2)

bool mlp_supported(int LF, int nd, int nc) {
#define X(l, d, n) \
  if (LF == l && nd == d && nc == n) return true;
  FFN_MLP_CONFIGS(X)
#undef X
  return false;
}

size_t mlp_lds_bytes(int LF, int nd, int nc) {
#define X(l, d, n) \
  if (LF == l && nd == d && nc == n) return sizeof(float) * (size_t)Arch<l, d, n>::lds_floats();
  FFN_MLP_CONFIGS(X)
#undef X
  return 0;
}

hipError_t launch_mlp_fwd(const DevCfg& c, const MlpPtrs& w, const float* a0, const FeatLayout& feat,
                          const float4* rays, const uint32_t* ray_ids, int64_t n, float sh_mult, float* sigma,
                          float* rgb, int LF, int nd, int nc, int n_blocks, hipStream_t st) {
  if (n <= 0) return hipSuccess;
#define X(l, d, nn)                   \
  if (LF == l && nd == d && nc == nn) \
    return launch_fwd_t<l, d, nn>(c, w, a0, feat, rays, ray_ids, n, sh_mult, sigma, rgb, n_blocks, st);
  FFN_MLP_CONFIGS(X)
#undef X
  return hipErrorInvalidValue;
}

hipError_t launch_mlp(const MlpArgs& a, int LF, int nd, int nc, int n_blocks, hipStream_t st) {
#define X(l, d, n) \
  if (LF == l && nd == d && nc == n) return launch_t<l, d, n>(a, n_blocks, st);
  FFN_MLP_CONFIGS(X)
#undef X
  return hipErrorInvalidValue;
}

}  // namespace ffn
