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
//     one wavefront per tile (rotating) runs the reference's scan trees on 64
//     lanes (one lane per sample, S lanes per ray) and leaves the loss
//     gradients in LDS; after a second barrier every wavefront reads its own
//     samples'.
//   * Weight gradients dW = sum_s delta[o][s] act[i][s] need the samples as
//     K.  Layer by layer in the backward, every wavefront writes its 16
//     samples' deltas and input activations into a block-shared fp32 stash
//     (rows = neurons, 64 sample columns); after a barrier the layer's 16x16
//     gradient tiles are dealt round-robin over the four wavefronts, each
//     accumulating its tiles over the 64 samples (16 MFMAs per tile) in
//     registers for the whole kernel.  A wavefront so holds a quarter of the
//     gradient (40 registers at the cfg2 shape), the weights are kept once
//     (the backward reads them transposed), and two blocks fit on a CU.  At
//     the end every wavefront stores its tiles into the block's partial
//     (no staging buffers in HBM, unlike the reference's ~1.8 KB/sample SoA
//     traffic).
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
  // row pitch in+4 (4 mod 32 for in = 16, 32, 64): the forward's 16-byte reads of four k-steps and the
  // backward's transposed 4-byte reads both fall on distinct banks
  static constexpr int pitch(int k) { return layer_in(k, LF) + 4; }
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
  static constexpr int PSF = 64 + 4;       // stash pitch: 64 sample columns + 4 pad (conflict-free b128 reads)
  static constexpr int stash_rows = 128;   // one layer's delta rows (<= 64) + input activation rows (<= 64)
  // sigma[64] + rgb[64][3] of the tile: one slot when training (the stash barriers separate a tile's
  // compositing from the next tile's writes), two alternating slots for a forward-only launch
  static constexpr int comp_floats(bool train) { return train ? 256 : 512; }
  static constexpr int lds_floats(bool train = true) { return w_total() + stash_rows * PSF + comp_floats(train); }
  // two blocks per CU when the LDS allows it (160 KiB per CU)
  static constexpr int blocks_per_cu() { return lds_floats() * 4 <= 80 * 1024 ? 2 : 1; }
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
  // Software-pipelined weight reads: output tile t's four k-steps of input tile tp run back to back (each
  // accumulator still takes its k-steps in (tp, rp) order, the same sums), and the registers they free take
  // tile t's weights of input tile tp + 1 while the other output tiles' MFMAs run, so no read waits at the
  // head of the next k block.  A single output tile (the 16-row heads) double-buffers its weights instead.
  auto wread = [&](int t, int tp) { return *reinterpret_cast<const floatx4*>(wrow + 16 * t * P + 16 * tp); };
  if constexpr (OT == 1) {
    floatx4 w_cur = wread(0, 0);
#pragma unroll
    for (int tp = 0; tp < IT; ++tp) {
      floatx4 w_nxt = w_cur;
      if (tp + 1 < IT) w_nxt = wread(0, tp + 1);
#pragma unroll
      for (int rp = 0; rp < 4; ++rp) acc[0] = mfma4(w_cur[rp], in[tp][rp], acc[0]);
      w_cur = w_nxt;
    }
  } else {
    floatx4 w4[OT];
#pragma unroll
    for (int t = 0; t < OT; ++t) w4[t] = wread(t, 0);
#pragma unroll
    for (int tp = 0; tp < IT; ++tp) {
#pragma unroll
      for (int t = 0; t < OT; ++t) {
#pragma unroll
        for (int rp = 0; rp < 4; ++rp) acc[t] = mfma4(w4[t][rp], in[tp][rp], acc[t]);
        if (tp + 1 < IT) w4[t] = wread(t, tp + 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < OT; ++t) {
    if (relu) {
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[t][r] = relu_f(acc[t][r]);
    }
    out[t] = acc[t];
  }
}

// res tiles (D layout over input neurons, first RT tiles) = W^T . delta (+ init)
template <int RT, int DT>
__device__ __forceinline__ void bwd_tiles(const float* __restrict__ W, int P, const floatx4 (&delta)[DT],
                                          floatx4 (&res)[RT], int g, int s) {
#pragma unroll
  for (int tp = 0; tp < DT; ++tp) {
    float w[4][RT];  // the delta tile's weights, all read before its MFMAs
#pragma unroll
    for (int rp = 0; rp < 4; ++rp)
#pragma unroll
      for (int t = 0; t < RT; ++t) w[rp][t] = W[(16 * tp + 4 * g + rp) * P + 16 * t + s];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int rp = 0; rp < 4; ++rp)
#pragma unroll
      for (int t = 0; t < RT; ++t) res[t] = mfma4(w[rp][t], delta[tp][rp], res[t]);
  }
}

// The colour output layer's backward: res tiles = W^T . delta over the 64 hidden units, with the delta's
// three rows held by lane group 0 (r = 0, 1, 2; the padded tile's other rows are zero).  Rows 1 and 2 move to
// lane groups 1 and 2 (permlane row swaps with a zero partner, so every other row stays zero), which makes
// the delta one K = 4 step (K index g, row 3 of the padded weights zero): four MFMAs where the padded tile's
// four k-steps took sixteen.
__device__ __forceinline__ void bwd_color_out(const float* __restrict__ W, int P, const floatx4 (&delta)[1],
                                              floatx4 (&res)[4], int g, int s) {
  const int d1 = __float_as_int(delta[0][1]), d2 = __float_as_int(delta[0][2]);
  const int m1 = (int)__builtin_amdgcn_permlane16_swap(0, d1, false, false)[0];  // row 1 <- row 0
  const int m2 = (int)__builtin_amdgcn_permlane32_swap(0, d2, false, false)[0];  // row 2 <- row 0
  const float bk = __int_as_float(__float_as_int(delta[0][0]) | m1 | m2);
  float w[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) w[t] = W[g * P + 16 * t + s];
#pragma unroll
  for (int t = 0; t < 4; ++t) res[t] = mfma4(w[t], bk, floatx4{0.f, 0.f, 0.f, 0.f});
}

// The activation passes through an empty asm first: otherwise the compiler proves act > 0 equal to the
// forward ReLU's own comparison and keeps that lane mask (two SGPRs per value, 48 values) live from the
// forward to the backward, which spilled SGPRs to VGPR lanes by the hundred per tile.  Here the test is
// made where it is used, on the value the backward holds anyway.
template <int NT>
__device__ __forceinline__ void relu_mask(floatx4 (&d)[NT], const floatx4 (&act)[NT]) {
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = act[t][r];
      __asm__("" : "+v"(v));
      d[t][r] = v > 0.0f ? d[t][r] : 0.0f;
    }
}

// Weight-gradient tiles of one layer held by one wavefront: the layer's 16x16 tile (T, Tp) (rows 16T..,
// columns 16Tp..) dealt to it as its m-th by deal_tile in w[m] (D layout), and in b a per-lane partial
// of the bias gradient of its tile with Tp = 0 (deal_tile gives a wavefront at most one per layer).
template <int OT, int IT>
struct WaveGrad {
  static constexpr int N = OT * IT / 4;
  static_assert(OT * IT % 4 == 0, "a layer's gradient tiles split evenly over four wavefronts");
  floatx4 w[N];
  float b;
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int m = 0; m < N; ++m) w[m] = floatx4{0.f, 0.f, 0.f, 0.f};
    b = 0.0f;
  }
};

// this wavefront's samples (stash column col) of a layer: delta rows [0, 16 OT), activation rows
// [16 OT, 16 (OT + IT)); both given as D-layout tiles (lane (g, s) holds neurons 16t + 4g + r)
template <int OT, int IT, int PSF>
__device__ __forceinline__ void stash_layer(float* __restrict__ st, const floatx4 (&d)[OT], const floatx4 (&act)[IT],
                                            int g, int col) {
#pragma unroll
  for (int t = 0; t < OT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) st[(16 * t + 4 * g + r) * PSF + col] = d[t][r];
#pragma unroll
  for (int t = 0; t < IT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) st[(16 * (OT + t) + 4 * g + r) * PSF + col] = act[t][r];
}

// dW tiles of this wavefront over the 64 stashed samples: 16 k-steps of 4, lane group g taking sample
// 16g + kk at k-step kk (the same permutation for both operands)
template <int OT, int IT, int PSF>
__device__ __forceinline__ void layer_dw(const float* __restrict__ st, WaveGrad<OT, IT>& acc, int wave, int g, int s) {
#pragma unroll
  for (int m = 0; m < WaveGrad<OT, IT>::N; ++m) {
    int T, Tp;
    deal_tile<IT>(m, wave, T, Tp);
    const float* drow = st + (16 * T + s) * PSF + 16 * g;
    const float* arow = st + (16 * (OT + Tp) + s) * PSF + 16 * g;
    floatx4 dv[4], av[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      dv[q] = *reinterpret_cast<const floatx4*>(drow + 4 * q);
      av[q] = *reinterpret_cast<const floatx4*>(arow + 4 * q);
    }
    floatx4 c = acc.w[m];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) c = mfma4(dv[q][e], av[q][e], c);
    acc.w[m] = c;
    if (Tp == 0) {
      float bs = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q) bs += (dv[q][0] + dv[q][1]) + (dv[q][2] + dv[q][3]);
      acc.b += bs;
    }
  }
}

// The colour output layer's weight gradient dW[o][k] = sum_s delta[o][s] act[k][s] (three rows, 64 inputs)
// on v_mfma_f32_4x4x1f32 (layout at fwd_color_out): wavefront w takes inputs 16w .. 16w + 15; lane l = 16 kq +
// 4 sg + j is lane j of block 4 kq + sg and supplies, at step n, delta row j of sample 16 sg + n (A; row 3 is
// the padding's zero row) and the activation of input 16w + 4 kq + j for that sample (B), so its register o
// accumulates sample group sg's share of dW[o][16w + 4 kq + j]; the groups are summed at the flush.  16
// instructions of 8 cycles where the padded 16-row tile took 16 of 32.  Wavefront 0 also sums the bias
// gradient (lane l: delta row j over sample group sg).  The stash holds the 16 delta rows, then the inputs.
template <int PSF>
__device__ __forceinline__ void layer_dw_color_out(const float* __restrict__ st, WaveGrad<1, 4>& acc, int wave,
                                                   int lane) {
  const int j = lane & 3, sg = (lane >> 2) & 3, kq = lane >> 4;
  const float* drow = st + j * PSF + 16 * sg;
  const float* arow = st + (16 + 16 * wave + 4 * kq + j) * PSF + 16 * sg;
  floatx4 dv[4], av[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    dv[q] = *reinterpret_cast<const floatx4*>(drow + 4 * q);
    av[q] = *reinterpret_cast<const floatx4*>(arow + 4 * q);
  }
  floatx4 c = acc.w[0];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int e = 0; e < 4; ++e) c = __builtin_amdgcn_mfma_f32_4x4x1f32(dv[q][e], av[q][e], c, 0, 0, 0);
  acc.w[0] = c;
  if (wave == 0) {
    float bs = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) bs += (dv[q][0] + dv[q][1]) + (dv[q][2] + dv[q][3]);
    acc.b += bs;
  }
}
__device__ __forceinline__ void flush_color_out(float* __restrict__ dst, const WaveGrad<1, 4>& acc, int wave,
                                                int lane) {
  constexpr int O = FFN_C_OUT, In = FFN_M;
  const int j = lane & 3, sg = (lane >> 2) & 3, kq = lane >> 4;
#pragma unroll
  for (int o = 0; o < O; ++o) {
    float v = acc.w[0][o];
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 8);
    if (sg == 0) dst[o * In + 16 * wave + 4 * kq + j] = v;
  }
  if (wave == 0) {
    float bs = acc.b;
    bs += __shfl_xor(bs, 4);
    bs += __shfl_xor(bs, 8);
    if (lane < O) dst[O * In + lane] = bs;
  }
}

// store this wavefront's tiles of a layer into the block's partial gradient (packed [O][In] + [O])
template <int OT, int IT>
__device__ __forceinline__ void flush_layer(float* __restrict__ dst, int O, int In, const WaveGrad<OT, IT>& acc,
                                            int wave, int g, int s) {
#pragma unroll
  for (int m = 0; m < WaveGrad<OT, IT>::N; ++m) {
    int T, Tp;
    deal_tile<IT>(m, wave, T, Tp);
    const int col = 16 * Tp + s;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * T + 4 * g + r;
      if (row < O && col < In) dst[row * In + col] = acc.w[m][r];
    }
    if (Tp == 0) {
      float bs = acc.b;
      bs += __shfl_xor(bs, 16);
      bs += __shfl_xor(bs, 32);
      if (g == 0 && 16 * T + s < O) dst[O * In + 16 * T + s] = bs;
    }
  }
}

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

// The colour output layer's forward (three rows of 64 inputs) on v_mfma_f32_4x4x1f32, whose 16 blocks of
// four lanes each add a 4x4 outer product (block b: lane 4b + i supplies row i of A, lane 4b + j column j of
// B, and lane 4b + j receives column j in its four registers; pinned by a probe).  Lane (g, s) is lane j =
// s % 4 of block 4g + s / 4: it supplies weight row s % 4 (row 3 is the padding's zero row) of input unit
// 16t + 4g + r and the activation of that unit for its sample, so after the 16 (t, r) steps it holds lane
// group g's share of its sample's three outputs (and a zero fourth); two row swaps sum the four groups.
// 16 instructions of 8 cycles where the padded 16-row tile took 16 of 32.  Every lane gets its sample's
// colours.
__device__ __forceinline__ void fwd_color_out(const float* __restrict__ W, const float* __restrict__ B, int P,
                                              const floatx4 (&act)[4], int g, int s, float (&rgb)[3]) {
  floatx4 part = {0.f, 0.f, 0.f, 0.f};
  const float* wrow = W + (s & 3) * P + 4 * g;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const floatx4 w4 = *reinterpret_cast<const floatx4*>(wrow + 16 * t);
#pragma unroll
    for (int r = 0; r < 4; ++r) part = __builtin_amdgcn_mfma_f32_4x4x1f32(w4[r], act[t][r], part, 0, 0, 0);
  }
#pragma unroll
  for (int o = 0; o < 3; ++o) {
    const int x = __float_as_int(part[o]);
    const auto h = __builtin_amdgcn_permlane32_swap(x, x, false, false);  // {lower half twice, upper half twice}
    const int y = __float_as_int(__int_as_float((int)h[0]) + __int_as_float((int)h[1]));
    const auto q = __builtin_amdgcn_permlane16_swap(y, y, false, false);  // {even rows twice, odd rows twice}
    rgb[o] = sigmoid_soft((__int_as_float((int)q[0]) + __int_as_float((int)q[1])) + B[o]);
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
      for (int kq = 0; kq < KA; kq += 4) {
        const floatx4 w4 = *reinterpret_cast<const floatx4*>(wrow + kq);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) acc = mfma4(w4[kk], a0r[kq + kk], acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = relu_f(acc[r]);
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
  fwd_color_out(sW + A::w_off(FFN_WC_OUT), sW + A::b_off(FFN_WC_OUT), A::pitch(FFN_WC_OUT), hc[NC - 1], g, s, rgb_s);
}

// MARCHED: the backward over marched samples -- sample b is a.smp[b] of ray a.ray_ids[b], its loss gradients
// are read (a.in_dLds, a.in_dLdc), and there is no compositing and no proposal.  TRAIN (a.do_train) is a
// template parameter: a forward-only tile leaves the loop after its compositing, and that exit, taken at run
// time, made the register allocator copy the activations and gradient accumulators (90 moves per tile) on
// the training path too.
template <int LF, int ND, int NC, int FEAT, bool TAPS, bool MARCHED, int SC, bool TRAIN>
__global__ __launch_bounds__(256, (Arch<LF, ND, NC>::blocks_per_cu())) void k_mlp(MlpArgs a) {
  static_assert(TRAIN || !MARCHED, "marched launches train");
  using A = Arch<LF, ND, NC>;
  constexpr int KA = LF / 4;  // a0 values per lane (k-steps of the first layer)
  constexpr int PSF = A::PSF;
  extern __shared__ float smem[];
  float* sW = smem;
  float* sS = smem + A::w_total();            // per-layer stash of deltas and activations
  float* sC = sS + A::stash_rows * A::PSF;    // compositing inputs (double-buffered)
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
  const int col = wave * 16 + s;              // this lane's stash column
  constexpr bool train = TRAIN;
  const DevCfg& c = a.c;
  const int log2S = a.log2S;
  uint64_t n_samples = (uint64_t)a.num_rays << log2S;
  int64_t n_tiles = a.n_tiles;
  if (a.n_dev) {  // the count of a launch sized for a capacity, read on the device
    const uint64_t nd = *a.n_dev;
    n_samples = nd < n_samples ? nd : n_samples;
    n_tiles = (int64_t)((n_samples + 63) / 64);
  }

  stage_weights<LF, ND, NC>(sW, a.w, tid, 256);
  __syncthreads();

  const float Dhalf = half_box_diagonal(c);
  constexpr bool taps = TAPS;
  const bool proposals = train && a.occ_strength > 0.0f;

  WaveGrad<1, 4> gc_out;
  WaveGrad<4, 4> gc_h[NC > 1 ? NC - 1 : 1];  // Wc_01, Wc_12, Wc_23
  WaveGrad<4, 2> gc_in;
  WaveGrad<1, 4> gd_out;
  WaveGrad<4, 4> gd_h[ND > 1 ? ND - 1 : 1];  // Wd_01, Wd_12
  WaveGrad<4, LF / 16> gd_in;
  gc_out.zero();
#pragma unroll
  for (int i = 0; i < (NC > 1 ? NC - 1 : 1); ++i) gc_h[i].zero();
  gc_in.zero();
  gd_out.zero();
#pragma unroll
  for (int i = 0; i < (ND > 1 ? ND - 1 : 1); ++i) gd_h[i].zero();
  gd_in.zero();

  // The busy tiles (a sample with dt > 0), which the tile order puts first, take the full path; a tile
  // whose samples are all inactive (e.g. a ray that misses the box) composites to exactly the background
  // and all its gradients are zero, so the later positions only write that (empty_tile).  Taps, which expose
  // per-sample MLP outputs, take the full path for every tile.  (Two loops: an exit from the full path for
  // the empty tiles had the register allocator copy the gradient accumulators on every tile.)
  const int64_t n_full = (TAPS || MARCHED || !a.n_busy) ? n_tiles : (int64_t)*a.n_busy;
  int parity = 0;
  int64_t ti = blockIdx.x;
  // Issue priority.  The two blocks a CU holds (blocks b and b + gridDim.x / 2, as the dispatcher deals
  // the grid) take turns at the higher of two levels, twice a tile (the forward with the compositing, then
  // the backward): the favoured block's wavefronts reach its barriers together while the other block fills
  // the issue slots they leave (fp32 MFMAs and vector instructions never issue together), where equal levels
  // let both blocks' wavefronts drift apart and wait at every barrier for the slowest (fp32 MLP 7.29 ->
  // 7.13-7.19 ms with one turn per tile, 7.09-7.11 with two; one turn every 2 or 4 tiles 7.20-7.22, four per
  // tile 7.14-7.30).  The compositing wavefront, which the rest of its block waits for, runs above both.
  const int gang = (int)(blockIdx.x >= gridDim.x / 2);
#pragma unroll 1
  for (; ti < n_full; ti += gridDim.x, parity ^= 1) {
    const bool gang_hi = (parity ^ gang) != 0;
    if (gang_hi) __builtin_amdgcn_s_setprio(2);
    else __builtin_amdgcn_s_setprio(1);
    __builtin_amdgcn_sched_barrier(0);  // the turn starts here (the scheduler would sink it to the forward's end)
    const int64_t tile = a.tile_order ? (int64_t)a.tile_order[ti] : ti;
    float* sSig = sC + (train ? 0 : parity * 256);
    float* sRgb = sSig + 64;
    // ------------------------------------------------------------------
    // forward: this lane's sample in the MLP layout
    const int64_t b = tile * 64 + col;
    const bool valid = (uint64_t)b < n_samples;
    const int64_t ray = valid ? (MARCHED ? (int64_t)a.ray_ids[b] : (b >> log2S)) : 0;
    float a0r[KA];
    load_a0<LF, FEAT>(a.a0, a.feat, b, valid, g, a0r);
    float dirv[3];
    {
      const float4 rd = a.rays[2 * ray + 1];
      dirv[0] = rd.x;
      dirv[1] = rd.y;
      dirv[2] = rd.z;
    }
    const float dt_b = valid ? (MARCHED ? a.march_dt : a.DTs[b]) : 0.0f;
    const float t_b = valid ? (MARCHED ? a.smp[b].w : a.Ts[b]) : 0.0f;
    // per-sample inputs of the compositing (lane j = sample j of the tile), loaded before the forward so
    // that their latency hides behind it
    const bool prop_wave = (int)(tile & 3) == wave;  // this wavefront makes the tile's proposals
    CompLane CL{};
    if constexpr (!MARCHED) {
      CL = load_comp_lane<SC>(a, tile, lane, prop_wave, n_samples, log2S, proposals);
    }

    floatx4 hd[ND][4];
    floatx4 acin[2];  // [dout(16) | SH*mult(16)] as two D-layout tiles
    floatx4 hc[NC][4];
    float rgb_s[3];
    mlp_fwd_tile<LF, ND, NC>(sW, a0r, dirv, a.sh_mult, g, s, hd, acin, hc, rgb_s);
    if constexpr (TAPS) {
      if (a.t_relu) {
        uint32_t* rec = valid ? a.t_relu + (int64_t)RELU_WORDS * b : nullptr;
#pragma unroll
        for (int i = 0; i < ND; ++i) tap_relu(rec, i, hd[i], g);
#pragma unroll
        for (int i = 0; i < NC; ++i) tap_relu(rec, 3 + i, hc[i], g);
      }
    }
    const float dout0 = acin[0][0];
    float dLds, dLdc0, dLdc1, dLdc2;
    if constexpr (MARCHED) {
      __syncthreads();  // the previous tile's last weight-gradient tiles have read the stash
      dLds = valid ? a.in_dLds[b] : 0.0f;
      dLdc0 = valid ? a.in_dLdc[3 * b] : 0.0f;
      dLdc1 = valid ? a.in_dLdc[3 * b + 1] : 0.0f;
      dLdc2 = valid ? a.in_dLdc[3 * b + 2] : 0.0f;
    } else {
      if (g == 0) {
        float sig = softplus(fminf(fmaxf(dout0, -10.0f), 10.0f));
        if (dt_b <= 0.0f) sig = 0.0f;
        sSig[col] = sig;
        sRgb[col * 3 + 0] = rgb_s[0];
        sRgb[col * 3 + 1] = rgb_s[1];
        sRgb[col * 3 + 2] = rgb_s[2];
      }
      __syncthreads();

      // ------------------------------------------------------------------
      // compositing on 64 lanes (lane j = sample j of the tile) by one wavefront, the tile's proposal
      // wavefront, which also writes the output colour (and taps); its loss gradients replace sigma and rgb
      // in LDS (only it reads them), and after a barrier every wavefront reads its own samples'.  The other
      // three wavefronts' SIMDs meanwhile run the CU's other block.
      if (prop_wave) {
        float dLds_j, dLdc_j[3];
        __builtin_amdgcn_s_setprio(3);
        composite_tile<TAPS, SC>(a, sSig, sRgb, CL, lane, 0, true, train, proposals, Dhalf, dLds_j, dLdc_j);
        if (train) {
          sSig[lane] = dLds_j;
          sRgb[3 * lane] = dLdc_j[0];
          sRgb[3 * lane + 1] = dLdc_j[1];
          sRgb[3 * lane + 2] = dLdc_j[2];
        }
      }
      // the tile's second turn: the block that led the forward yields the backward
      if (gang_hi) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(2);
      if (!train) continue;
      __syncthreads();
      dLds = sSig[col];
      dLdc0 = sRgb[3 * col];
      dLdc1 = sRgb[3 * col + 1];
      dLdc2 = sRgb[3 * col + 2];
    }

    // ------------------------------------------------------------------
    // backward of this wave's 16 samples; every layer's deltas and inputs go through the stash for the
    // block's weight-gradient tiles (barrier, this wave's tiles, barrier before the stash is reused)
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
    // colour output layer
    floatx4 dc[NC][4];
    stash_layer<1, 4, PSF>(sS, dco, hc[NC - 1], g, col);
    bwd_color_out(sW + A::w_off(FFN_WC_OUT), A::pitch(FFN_WC_OUT), dco, dc[NC - 1], g, s);
    relu_mask(dc[NC - 1], hc[NC - 1]);
    __syncthreads();
    layer_dw_color_out<PSF>(sS, gc_out, wave, lane);
    __syncthreads();
    // hidden colour layers (Wc_23, Wc_12, Wc_01)
#pragma unroll
    for (int i = NC - 1; i >= 1; --i) {
      const int k = i == 1 ? FFN_WC_01 : (i == 2 ? FFN_WC_12 : FFN_WC_23);
      stash_layer<4, 4, PSF>(sS, dc[i], hc[i - 1], g, col);
#pragma unroll
      for (int t = 0; t < 4; ++t) dc[i - 1][t] = floatx4{0.f, 0.f, 0.f, 0.f};
      bwd_tiles<4, 4>(sW + A::w_off(k), A::pitch(k), dc[i], dc[i - 1], g, s);
      relu_mask(dc[i - 1], hc[i - 1]);
      __syncthreads();
      layer_dw<4, 4, PSF>(sS, gc_h[i - 1], wave, g, s);
      __syncthreads();
    }
    // colour input layer: its gradient, and the dout part of its input delta
    stash_layer<4, 2, PSF>(sS, dc[0], acin, g, col);
    bwd_tiles<1, 4>(sW + A::w_off(FFN_WC_IN), A::pitch(FFN_WC_IN), dc[0], ddo, g, s);
    __syncthreads();
    layer_dw<4, 2, PSF>(sS, gc_in, wave, g, s);
    __syncthreads();
    // density output layer
    floatx4 dd[ND][4];
    stash_layer<1, 4, PSF>(sS, ddo, hd[ND - 1], g, col);
#pragma unroll
    for (int t = 0; t < 4; ++t) dd[ND - 1][t] = floatx4{0.f, 0.f, 0.f, 0.f};
    bwd_tiles<4, 1>(sW + A::w_off(FFN_WD_OUT), A::pitch(FFN_WD_OUT), ddo, dd[ND - 1], g, s);
    relu_mask(dd[ND - 1], hd[ND - 1]);
    __syncthreads();
    layer_dw<1, 4, PSF>(sS, gd_out, wave, g, s);
    __syncthreads();
    // hidden density layers (Wd_12, Wd_01)
#pragma unroll
    for (int i = ND - 1; i >= 1; --i) {
      const int k = i == 1 ? FFN_WD_01 : FFN_WD_12;
      stash_layer<4, 4, PSF>(sS, dd[i], hd[i - 1], g, col);
#pragma unroll
      for (int t = 0; t < 4; ++t) dd[i - 1][t] = floatx4{0.f, 0.f, 0.f, 0.f};
      bwd_tiles<4, 4>(sW + A::w_off(k), A::pitch(k), dd[i], dd[i - 1], g, s);
      relu_mask(dd[i - 1], hd[i - 1]);
      __syncthreads();
      layer_dw<4, 4, PSF>(sS, gd_h[i - 1], wave, g, s);
      __syncthreads();
    }
    // density input layer: deltas in rows [0, 64), the encoding (neuron KA g + kk in a0r[kk]) in rows 64..
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) sS[(16 * t + 4 * g + r) * PSF + col] = dd[0][t][r];
#pragma unroll
    for (int kk = 0; kk < KA; ++kk) sS[(64 + KA * g + kk) * PSF + col] = a0r[kk];
    // encoding gradient dL/da0 = Wd_in^T . delta_d1 -> HBM for the hash scatter
    {
      floatx4 ga[LF / 16];
#pragma unroll
      for (int t = 0; t < LF / 16; ++t) ga[t] = floatx4{0.f, 0.f, 0.f, 0.f};
      bwd_tiles<LF / 16, 4>(sW + A::w_off(FFN_WD_IN), A::pitch(FFN_WD_IN), dd[0], ga, g, s);
      if (valid) store_enc_grad<LF, FEAT>(a, b, g, ga);
    }
    __syncthreads();
    layer_dw<4, LF / 16, PSF>(sS, gd_in, wave, g, s);
    // no barrier: the stash is next written after the next tile's compositing barrier
  }
  if constexpr (!MARCHED) {
#pragma unroll 1
    for (; ti < n_tiles; ti += gridDim.x) {
      const int64_t tile = a.tile_order ? (int64_t)a.tile_order[ti] : ti;
      const int64_t b = tile * 64 + col;
      const CompLane CL = load_comp_lane<SC>(a, tile, lane, false, n_samples, log2S, false);
      empty_tile<LF, FEAT, SC>(a, CL, lane, wave, b, (uint64_t)b < n_samples, train, g);
    }
  }

  if (train) {
    // every wavefront stores its tiles into the block's partial gradient
    float* dst = a.partials + (int64_t)blockIdx.x * A::g_total();
    flush_color_out(dst + A::g_off(FFN_WC_OUT), gc_out, wave, lane);
    if constexpr (NC >= 2) flush_layer(dst + A::g_off(FFN_WC_01), FFN_M, FFN_M, gc_h[0], wave, g, s);
    if constexpr (NC >= 3) flush_layer(dst + A::g_off(FFN_WC_12), FFN_M, FFN_M, gc_h[1], wave, g, s);
    if constexpr (NC >= 4) flush_layer(dst + A::g_off(FFN_WC_23), FFN_M, FFN_M, gc_h[2], wave, g, s);
    flush_layer(dst + A::g_off(FFN_WC_IN), FFN_M, FFN_C_IN, gc_in, wave, g, s);
    flush_layer(dst + A::g_off(FFN_WD_OUT), FFN_D_OUT, FFN_M, gd_out, wave, g, s);
    if constexpr (ND >= 2) flush_layer(dst + A::g_off(FFN_WD_01), FFN_M, FFN_M, gd_h[0], wave, g, s);
    if constexpr (ND >= 3) flush_layer(dst + A::g_off(FFN_WD_12), FFN_M, FFN_M, gd_h[1], wave, g, s);
    flush_layer(dst + A::g_off(FFN_WD_IN), FFN_M, LF, gd_in, wave, g, s);
  }
}

// ---------------------------------------------------------------------------

template <int LF, int ND, int NC, int FEAT, bool TAPS, bool MARCHED, int SC, bool TRAIN>
static hipError_t launch_k(const MlpArgs& a, int n_blocks, hipStream_t st) {
  using A = Arch<LF, ND, NC>;
  const size_t lds = sizeof(float) * (size_t)A::lds_floats(TRAIN);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)k_mlp<LF, ND, NC, FEAT, TAPS, MARCHED, SC, TRAIN>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((k_mlp<LF, ND, NC, FEAT, TAPS, MARCHED, SC, TRAIN>), dim3(n_blocks), dim3(256), lds, st, a);
  return hipGetLastError();
}

template <int LF, int ND, int NC, int FEAT, bool TAPS, bool MARCHED, int SC>
static hipError_t launch_f(const MlpArgs& a, int n_blocks, hipStream_t st) {
  if constexpr (MARCHED) {
    return launch_k<LF, ND, NC, FEAT, TAPS, true, SC, true>(a, n_blocks, st);
  } else {
    return a.do_train ? launch_k<LF, ND, NC, FEAT, TAPS, false, SC, true>(a, n_blocks, st)
                      : launch_k<LF, ND, NC, FEAT, TAPS, false, SC, false>(a, n_blocks, st);
  }
}

template <int LF, int ND, int NC, bool MARCHED, int SC>
static hipError_t launch_t(const MlpArgs& a, int n_blocks, hipStream_t st) {
  const bool taps = taps_requested(a);
  switch (a.c.F) {
    case 1:
      return taps ? launch_f<LF, ND, NC, 1, true, MARCHED, SC>(a, n_blocks, st)
                  : launch_f<LF, ND, NC, 1, false, MARCHED, SC>(a, n_blocks, st);
    case 2:
      return taps ? launch_f<LF, ND, NC, 2, true, MARCHED, SC>(a, n_blocks, st)
                  : launch_f<LF, ND, NC, 2, false, MARCHED, SC>(a, n_blocks, st);
    case 4:
      return taps ? launch_f<LF, ND, NC, 4, true, MARCHED, SC>(a, n_blocks, st)
                  : launch_f<LF, ND, NC, 4, false, MARCHED, SC>(a, n_blocks, st);
    default: return hipErrorInvalidValue;
  }
}

// forward only, over a flat list of samples (the render path): 16 samples per wavefront per step
template <int LF, int ND, int NC, int FEAT>
__global__ __launch_bounds__(256) void k_mlp_fwd(MlpPtrs wp, const float* __restrict__ a0, FeatLayout feat,
                                                 const float4* __restrict__ rays, const uint32_t* __restrict__ ray_ids,
                                                 int64_t n, float sh_mult, float* __restrict__ sigma,
                                                 float* __restrict__ rgb, const uint32_t* __restrict__ n_dev) {
  extern __shared__ float smem[];
  if (n_dev) {  // the count of a launch sized for a capacity, read on the device
    const int64_t nd = (int64_t)*n_dev;
    n = nd < n ? nd : n;
  }
  if ((int64_t)blockIdx.x * 64 >= n) return;  // no samples for this block: skip staging the weights
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
                               int n_blocks, hipStream_t st, const uint32_t* n_dev) {
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
                     sh_mult, sigma, rgb, n_dev);
  return hipGetLastError();
}

template <int LF, int ND, int NC>
static hipError_t launch_fwd_t(const DevCfg& c, const MlpPtrs& w, const float* a0, const FeatLayout& feat,
                               const float4* rays, const uint32_t* ray_ids, int64_t n, float sh_mult, float* sigma,
                               float* rgb, int n_blocks, hipStream_t st, const uint32_t* n_dev) {
  switch (c.F) {
    case 1: return launch_fwd_f<LF, ND, NC, 1>(w, a0, feat, rays, ray_ids, n, sh_mult, sigma, rgb, n_blocks, st, n_dev);
    case 2: return launch_fwd_f<LF, ND, NC, 2>(w, a0, feat, rays, ray_ids, n, sh_mult, sigma, rgb, n_blocks, st, n_dev);
    case 4: return launch_fwd_f<LF, ND, NC, 4>(w, a0, feat, rays, ray_ids, n, sh_mult, sigma, rgb, n_blocks, st, n_dev);
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

int mlp_blocks_per_cu(int LF, int nd, int nc) {
#define X(l, d, n) \
  if (LF == l && nd == d && nc == n) return Arch<l, d, n>::blocks_per_cu();
  FFN_MLP_CONFIGS(X)
#undef X
  return 1;
}

hipError_t launch_mlp_fwd(const DevCfg& c, const MlpPtrs& w, const float* a0, const FeatLayout& feat,
                          const float4* rays, const uint32_t* ray_ids, int64_t n, float sh_mult, float* sigma,
                          float* rgb, int LF, int nd, int nc, int n_blocks, hipStream_t st, const uint32_t* n_dev) {
  if (n <= 0) return hipSuccess;
#define X(l, d, nn)                   \
  if (LF == l && nd == d && nc == nn) \
    return launch_fwd_t<l, d, nn>(c, w, a0, feat, rays, ray_ids, n, sh_mult, sigma, rgb, n_blocks, st, n_dev);
  FFN_MLP_CONFIGS(X)
#undef X
  return hipErrorInvalidValue;
}

// Tile order of a step: the sampler flags each 64-sample tile with a sample of dt > 0 (the tiles the MLP
// computes; the others composite to the background); the scan of the flags places the busy tiles first, in
// index order, then the others.  With the busy tiles dealt round-robin the blocks get equal shares of them
// (with tiles dealt in index order, a quarter of the rays missing the box left the busiest of 512 blocks
// 8.5 % above the mean).  The order depends on the data alone, so steps stay deterministic.
__global__ __launch_bounds__(256) void k_tile_place(const uint32_t* __restrict__ flags,
                                                    const uint32_t* __restrict__ off, int64_t n_tiles,
                                                    uint32_t* __restrict__ order) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_tiles) return;
  const uint32_t o = off[t], n_busy = off[n_tiles];
  order[flags[t] ? o : n_busy + ((uint32_t)t - o)] = (uint32_t)t;
}

hipError_t launch_tile_order(int64_t n_tiles, const uint32_t* flags, uint32_t* off, uint32_t* sums, uint32_t* total,
                             uint32_t* order, hipStream_t st) {
  if (n_tiles <= 0) return hipSuccess;
  hipError_t e = launch_scan_u32(flags, n_tiles, off, sums, total, st);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_tile_place, dim3((unsigned)((n_tiles + 255) / 256)), dim3(256), 0, st, flags, off, n_tiles,
                     order);
  return hipGetLastError();
}

hipError_t launch_mlp(const MlpArgs& a, int LF, int nd, int nc, int n_blocks, hipStream_t st) {
#define X(l, d, n) \
  if (LF == l && nd == d && nc == n)                                                         \
    return a.S == 64 ? launch_t<l, d, n, false, 64>(a, n_blocks, st) : launch_t<l, d, n, false, 0>(a, n_blocks, st);
  FFN_MLP_CONFIGS(X)
#undef X
  return hipErrorInvalidValue;
}

hipError_t launch_mlp_marched(const MlpArgs& a, int LF, int nd, int nc, int n_blocks, hipStream_t st) {
#define X(l, d, n) \
  if (LF == l && nd == d && nc == n) return launch_t<l, d, n, true, 0>(a, n_blocks, st);
  FFN_MLP_CONFIGS(X)
#undef X
  return hipErrorInvalidValue;
}

}  // namespace ffn
