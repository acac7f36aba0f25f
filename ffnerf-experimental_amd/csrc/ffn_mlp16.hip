// ffn_mlp16.hip -- the fused MLP step on 16-bit MFMAs with fp32 accumulation:
// forward and backward chains in fp16 (v_mfma_f32_16x16x16_f16; each layer's
// deltas are scaled by a per-wavefront power of two that puts their largest
// magnitude just below 2^14, so small deltas neither underflow nor lose bits),
// weight gradients in bf16 (v_mfma_f32_16x16x16_bf16, whose fp32-sized
// exponent takes the unscaled deltas of all four wavefronts).  Same semantics as the fp32
// kernel (ffnerf_OG.cl:1373-2082, weight_update.cl:210-341): compositing, loss
// gradient, proposals and output deltas are the shared fp32 code.
//
// MI355X design
//   * A 256-thread block (4 wavefronts) walks 64-sample tiles; each wavefront
//     runs the layers for its 16 samples.  With K = 16 per MFMA a layer's
//     output tile (lane (g, s) holds neurons 16t + 4g + r of sample s) is, once
//     converted to four 16-bit values, exactly the B operand of k-block t of
//     the next layer: activations never move between lanes.
//   * Weights live in LDS twice, fp16 row-major for the forward (A = W) and
//     fp16 transposed for the backward (A = W^T); every A operand is one
//     8-byte LDS read.
//   * Weight gradients dW = delta . act^T need the samples as K.  Layer by
//     layer in the backward, every wavefront writes its deltas and the layer's
//     input activations, transposed, into a block-shared bf16 stash (rows =
//     neurons, 64 samples per row); after a barrier the layer's 16x16 gradient
//     tiles are dealt round-robin over the four wavefronts, each of which
//     accumulates its tiles over the tile's 64 samples (4 MFMAs per tile) in
//     registers for the whole kernel and stores them into the block's partial
//     at the end.  A wavefront so holds about a quarter of the gradient, and
//     the one-layer stash lets two blocks share a CU.
#include "ffn_device.h"
#include "ffn_kernels.h"
#include "ffn_mlp_common.h"

namespace ffn {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma_f16(const half4& a, const half4& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma_bf16(const bf16x4& a, const bf16x4& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ half4 to_half4(const floatx4& v) {
  half4 h;
#pragma unroll
  for (int r = 0; r < 4; ++r) h[r] = (_Float16)v[r];
  return h;
}
__device__ __forceinline__ bf16x4 to_bf16x4(const floatx4& v) {
  bf16x4 h;
#pragma unroll
  for (int r = 0; r < 4; ++r) h[r] = (__bf16)v[r];
  return h;
}

// power of two that maps the largest |d| of the wavefront's tiles into [2^13, 2^14) (1 if all zero)
template <int NT>
__device__ __forceinline__ float delta_scale(const floatx4 (&d)[NT]) {
  float m = 0.0f;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) m = fmaxf(m, fabsf(d[t][r]));
  m = wave_max_nonneg(m);
  if (!(m > 0.0f) || !(m < 3.0e38f)) return 1.0f;
  int e;
  frexpf(m, &e);  // m < 2^e
  e = 14 - e;
  e = e > 100 ? 100 : (e < -100 ? -100 : e);
  return ldexpf(1.0f, e);
}

template <int NT>
__device__ __forceinline__ void scaled_half(const floatx4 (&d)[NT], float sc, half4 (&op)[NT]) {
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) op[t][r] = (_Float16)(d[t][r] * sc);
}

template <int LF_, int ND_, int NC_>
struct Arch16 {
  static constexpr int LF = LF_, ND = ND_, NC = NC_;
  static constexpr int rows_pad(int k) { return k == FFN_WC_OUT ? 16 : layer_out(k); }
  static constexpr int pf(int k) { return layer_in(k, LF) + 4; }  // fp16 forward row pitch (halves)
  static constexpr int pt(int k) { return rows_pad(k) + 4; }      // fp16 transposed row pitch
  static constexpr int wf_sz(int k) { return layer_active(k, ND, NC) ? rows_pad(k) * pf(k) : 0; }
  static constexpr int wt_sz(int k) { return layer_active(k, ND, NC) ? layer_in(k, LF) * pt(k) : 0; }
  static constexpr int wf_off(int k) {  // in halves
    int o = 0;
    for (int j = 0; j < k; ++j) o += wf_sz(j);
    return o;
  }
  static constexpr int wt_off(int k) {
    int o = wf_off(FFN_N_LAYERS);
    for (int j = 0; j < k; ++j) o += wt_sz(j);
    return o;
  }
  static constexpr int w_halves() { return wt_off(FFN_N_LAYERS); }
  static constexpr int b_off(int k) {  // in floats, after the 16-bit weights
    int o = 0;
    for (int j = 0; j < k; ++j) o += layer_active(j, ND, NC) ? rows_pad(j) : 0;
    return o;
  }
  static constexpr int b_floats() { return b_off(FFN_N_LAYERS); }
  // one layer's stash (bf16, PS per row): delta rows, then the layer's input activation rows
  static constexpr int PS = 64 + 4;
  static constexpr int stash_rows = 128;
  static constexpr int stash_halves() { return stash_rows * PS; }
  // packed gradient (same layout as make_layout)
  static constexpr int gsz(int k) {
    return layer_active(k, ND, NC) ? layer_out(k) * layer_in(k, LF) + layer_out(k) : 0;
  }
  static constexpr int g_off(int k) {
    int o = 0;
    for (int j = 0; j < k; ++j) o += gsz(j);
    return o;
  }
  static constexpr int g_total() { return g_off(FFN_N_LAYERS); }
  static constexpr int comp_floats = 2 * 256;
  static constexpr size_t lds_bytes() {
    return (size_t)w_halves() * 2 + (size_t)b_floats() * 4 + (size_t)stash_halves() * 2 + comp_floats * 4;
  }
  static constexpr int blocks_per_cu() { return lds_bytes() <= 80 * 1024 ? 2 : 1; }
};

// forward layer: out tiles = act(W . in + b); in[kb] is the fp16 B operand of k-block kb
template <int OT, int KB>
__device__ __forceinline__ void fwd16(const _Float16* __restrict__ W, int P, const float* __restrict__ B,
                                      const half4 (&in)[KB], floatx4 (&out)[OT], int g, int s, bool relu) {
  floatx4 acc[OT];
#pragma unroll
  for (int t = 0; t < OT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[t][r] = B[16 * t + 4 * g + r];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int t = 0; t < OT; ++t) {
      const half4 a = *reinterpret_cast<const half4*>(W + (16 * t + s) * P + 16 * kb + 4 * g);
      acc[t] = mfma_f16(a, in[kb], acc[t]);
    }
#pragma unroll
  for (int t = 0; t < OT; ++t) {
    if (relu) {
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[t][r] = acc[t][r] > 0.0f ? acc[t][r] : 0.0f;
    }
    out[t] = acc[t];
  }
}

// backward layer: res tiles over input neurons += (W^T . (delta * sc)) / sc; Wt is [in][out_pad] fp16 and
// op the scaled fp16 deltas
template <int RT, int KB>
__device__ __forceinline__ void bwd16(const _Float16* __restrict__ Wt, int P, const half4 (&op)[KB], float sc,
                                      floatx4 (&res)[RT], int g, int s) {
  floatx4 acc[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      const half4 a = *reinterpret_cast<const half4*>(Wt + (16 * t + s) * P + 16 * kb + 4 * g);
      acc[t] = mfma_f16(a, op[kb], acc[t]);
    }
  int e;
  frexpf(sc, &e);  // sc = 2^(e - 1)
  const float inv = ldexpf(1.0f, 1 - e);  // 1 / sc, exactly
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) res[t][r] = res[t][r] + acc[t][r] * inv;
}

// zero the deltas of inactive ReLUs (mask from the forward activations)
template <int NT>
__device__ __forceinline__ void relu_mask16(floatx4 (&d)[NT], const half4 (&act)[NT]) {
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) d[t][r] = (float)act[t][r] > 0.0f ? d[t][r] : 0.0f;
}

// the next layer's operands: scale and fp16 deltas
template <int NT>
__device__ __forceinline__ float make_op(const floatx4 (&d)[NT], half4 (&op)[NT]) {
  const float sc = delta_scale<NT>(d);
  scaled_half<NT>(d, sc, op);
  return sc;
}

// write NT D-layout tiles of this wavefront's samples into stash rows row0 + 16t + 4g + r, column 16w + s
template <int NT, typename V>
__device__ __forceinline__ void stash_tiles(__bf16* __restrict__ st, int row0, const V (&v)[NT], int g, int col) {
  constexpr int PS = 64 + 4;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) st[(row0 + 16 * t + 4 * g + r) * PS + col] = (__bf16)(float)v[t][r];
}

// Weight-gradient tiles of one layer held by one wavefront: tiles i = T * IT + Tp dealt round-robin,
// wavefront w holding i = 4m + w (D layout) and a per-lane partial of the bias gradient when Tp = 0.
template <int OT, int IT>
struct WaveGrad16 {
  static constexpr int N = OT * IT / 4;
  static_assert(OT * IT % 4 == 0, "a layer's gradient tiles split evenly over four wavefronts");
  floatx4 w[N];
  float b[N];
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int m = 0; m < N; ++m) {
      w[m] = floatx4{0.f, 0.f, 0.f, 0.f};
      b[m] = 0.0f;
    }
  }
};

// this wavefront's dW tiles over the 64 stashed samples (delta rows [0, 16 OT), activation rows after)
template <int OT, int IT, int PS>
__device__ __forceinline__ void layer_dw16(const __bf16* __restrict__ st, WaveGrad16<OT, IT>& acc, int wave, int g,
                                           int s) {
#pragma unroll
  for (int m = 0; m < WaveGrad16<OT, IT>::N; ++m) {
    const int i = 4 * m + wave, T = i / IT, Tp = i - T * IT;
    const __bf16* drow = st + (16 * T + s) * PS + 4 * g;
    const __bf16* arow = st + (16 * (OT + Tp) + s) * PS + 4 * g;
    floatx4 c = acc.w[m];
    float bs = acc.b[m];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bf16x4 dv = *reinterpret_cast<const bf16x4*>(drow + 16 * q);
      const bf16x4 av = *reinterpret_cast<const bf16x4*>(arow + 16 * q);
      c = mfma_bf16(dv, av, c);
      if (Tp == 0) bs += ((float)dv[0] + (float)dv[1]) + ((float)dv[2] + (float)dv[3]);
    }
    acc.w[m] = c;
    acc.b[m] = bs;
  }
}

// store this wavefront's tiles of a layer into the block's partial gradient (packed [O][In] + [O])
template <int OT, int IT>
__device__ __forceinline__ void flush_layer16(float* __restrict__ dst, int O, int In, const WaveGrad16<OT, IT>& acc,
                                              int wave, int g, int s) {
#pragma unroll
  for (int m = 0; m < WaveGrad16<OT, IT>::N; ++m) {
    const int i = 4 * m + wave, T = i / IT, Tp = i - T * IT;
    const int col = 16 * Tp + s;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * T + 4 * g + r;
      if (row < O && col < In) dst[row * In + col] = acc.w[m][r];
    }
    if (Tp == 0) {
      float bs = acc.b[m];
      bs += __shfl_xor(bs, 16);
      bs += __shfl_xor(bs, 32);
      if (g == 0 && 16 * T + s < O) dst[O * In + 16 * T + s] = bs;
    }
  }
}

template <int LF, int ND, int NC, int FEAT, bool TAPS>
__global__ __launch_bounds__(256, (Arch16<LF, ND, NC>::blocks_per_cu())) void k_mlp16(MlpArgs a) {
  using A = Arch16<LF, ND, NC>;
  constexpr int KB0 = LF / 16;  // k-blocks of the first layer
  extern __shared__ __align__(16) unsigned char smem16[];
  _Float16* sWf = reinterpret_cast<_Float16*>(smem16);
  _Float16* sWt = sWf;  // the transposed copies follow the forward weights (offsets in 16-bit units)
  float* sB = reinterpret_cast<float*>(smem16 + (size_t)A::w_halves() * 2);
  __bf16* sS = reinterpret_cast<__bf16*>(smem16 + (size_t)A::w_halves() * 2 + (size_t)A::b_floats() * 4);
  float* sC = reinterpret_cast<float*>(smem16 + (size_t)A::w_halves() * 2 + (size_t)A::b_floats() * 4 +
                                       (size_t)A::stash_halves() * 2);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
  const bool train = a.do_train != 0;
  const DevCfg& c = a.c;
  const int log2S = a.log2S;
  const uint64_t n_samples = (uint64_t)a.num_rays << log2S;

  // weights: fp16 [out_pad][in] and bf16 [in][out_pad] (zero padding), fp32 biases
#pragma unroll
  for (int k = 0; k < FFN_N_LAYERS; ++k) {
    if (!layer_active(k, ND, NC)) continue;
    const int O = layer_out(k), I = layer_in(k, LF), R = A::rows_pad(k);
    const int PF = A::pf(k), PT = A::pt(k);
    const float* gw = a.w.W[k];
    for (int e = tid; e < R * PF; e += 256) {
      const int r = e / PF, col = e - r * PF;
      sWf[A::wf_off(k) + e] = (_Float16)((r < O && col < I) ? gw[r * I + col] : 0.0f);
    }
    for (int e = tid; e < I * PT; e += 256) {
      const int i = e / PT, o = e - i * PT;
      sWt[A::wt_off(k) + e] = (_Float16)((o < O) ? gw[o * I + i] : 0.0f);
    }
    for (int e = tid; e < R; e += 256) sB[A::b_off(k) + e] = e < O ? a.w.b[k][e] : 0.0f;
  }
  __syncthreads();

  const float Dhalf = half_box_diagonal(c);
  constexpr bool taps = TAPS;
  const bool proposals = train && a.occ_strength > 0.0f;
  constexpr int PS = A::PS;
  WaveGrad16<1, 4> gc_out;
  WaveGrad16<4, 4> gc_h[NC > 1 ? NC - 1 : 1];  // Wc_01, Wc_12, Wc_23
  WaveGrad16<4, 2> gc_in;
  WaveGrad16<1, 4> gd_out;
  WaveGrad16<4, 4> gd_h[ND > 1 ? ND - 1 : 1];  // Wd_01, Wd_12
  WaveGrad16<4, KB0> gd_in;
  gc_out.zero();
#pragma unroll
  for (int i = 0; i < (NC > 1 ? NC - 1 : 1); ++i) gc_h[i].zero();
  gc_in.zero();
  gd_out.zero();
#pragma unroll
  for (int i = 0; i < (ND > 1 ? ND - 1 : 1); ++i) gd_h[i].zero();
  gd_in.zero();

  int parity = 0;
  for (int64_t tile = blockIdx.x; tile < a.n_tiles; tile += gridDim.x, parity ^= 1) {
    float* sSig = sC + parity * 256;
    float* sRgb = sSig + 64;
    const int64_t b = tile * 64 + wave * 16 + s;
    const bool valid = (uint64_t)b < n_samples;
    const int64_t ray = valid ? (b >> log2S) : 0;
    // a0v[4 kb + j] = encoding neuron 16 kb + 4 g + j of sample b
    float a0v[LF / 4];
    if (valid) {
#pragma unroll
      for (int kb = 0; kb < KB0; ++kb) {
        if constexpr (FEAT == 4) {
          const int l = 4 * kb + g;
          const float4 v = *reinterpret_cast<const float4*>(a.a0 + l * a.feat.stride_l + b * a.feat.stride_b);
          a0v[4 * kb] = v.x;
          a0v[4 * kb + 1] = v.y;
          a0v[4 * kb + 2] = v.z;
          a0v[4 * kb + 3] = v.w;
        } else if constexpr (FEAT == 2) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int l = 8 * kb + 2 * g + h;
            const float2 v = *reinterpret_cast<const float2*>(a.a0 + l * a.feat.stride_l + b * a.feat.stride_b);
            a0v[4 * kb + 2 * h] = v.x;
            a0v[4 * kb + 2 * h + 1] = v.y;
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) a0v[4 * kb + j] = a.a0[(16 * kb + 4 * g + j) * a.feat.stride_l + b * a.feat.stride_b];
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < LF / 4; ++q) a0v[q] = 0.0f;
    }
    float dirv[3];
    {
      const float4 rd = a.rays[2 * ray + 1];
      dirv[0] = rd.x;
      dirv[1] = rd.y;
      dirv[2] = rd.z;
    }
    const float dt_b = valid ? a.DTs[b] : 0.0f;
    const float t_b = valid ? a.Ts[b] : 0.0f;
    const bool prop_wave = (int)(tile & 3) == wave;  // this wavefront makes the tile's proposals
    const CompLane CL = load_comp_lane(a, tile, lane, prop_wave, n_samples, log2S, proposals);
    if (!taps && __ballot(CL.vj && CL.dt_j > 0.0f) == 0ull) {  // the same on every wavefront of the block
      empty_tile<LF, FEAT>(a, CL, lane, wave, b, valid, train, g);
      continue;
    }

    // ---- forward (fp16 operands, fp32 accumulation)
    half4 a0h[KB0];
#pragma unroll
    for (int kb = 0; kb < KB0; ++kb)
#pragma unroll
      for (int j = 0; j < 4; ++j) a0h[kb][j] = (_Float16)a0v[4 * kb + j];
    bf16x4 a0b[KB0];  // the encoding as the stash holds it (bf16), kept for the first layer's gradient
#pragma unroll
    for (int kb = 0; kb < KB0; ++kb)
#pragma unroll
      for (int j = 0; j < 4; ++j) a0b[kb][j] = (__bf16)a0v[4 * kb + j];
    floatx4 sh;  // this lane's four SH inputs of the colour net
#pragma unroll
    for (int r = 0; r < 4; ++r) sh[r] = sh_component(dirv, 4 * g + r) * a.sh_mult;
    // the network's activations: computed for the colours, dropped across the compositing (held there,
    // they spilled to scratch), and computed again, bit-identically, for the backward
    auto forward = [&](half4(&hdh)[ND][4], half4(&acinh)[2], bf16x4(&acb)[2], half4(&hch)[NC][4], float(&rgb_s)[3],
                       float& dout0) {
      {
        floatx4 o[4];
        fwd16<4, KB0>(sWf + A::wf_off(FFN_WD_IN), A::pf(FFN_WD_IN), sB + A::b_off(FFN_WD_IN), a0h, o, g, s, true);
#pragma unroll
        for (int t = 0; t < 4; ++t) hdh[0][t] = to_half4(o[t]);
      }
      if constexpr (ND >= 2) {
        floatx4 o[4];
        fwd16<4, 4>(sWf + A::wf_off(FFN_WD_01), A::pf(FFN_WD_01), sB + A::b_off(FFN_WD_01), hdh[0], o, g, s, true);
#pragma unroll
        for (int t = 0; t < 4; ++t) hdh[1][t] = to_half4(o[t]);
      }
      if constexpr (ND >= 3) {
        floatx4 o[4];
        fwd16<4, 4>(sWf + A::wf_off(FFN_WD_12), A::pf(FFN_WD_12), sB + A::b_off(FFN_WD_12), hdh[1], o, g, s, true);
#pragma unroll
        for (int t = 0; t < 4; ++t) hdh[2][t] = to_half4(o[t]);
      }
      floatx4 dout[1];
      fwd16<1, 4>(sWf + A::wf_off(FFN_WD_OUT), A::pf(FFN_WD_OUT), sB + A::b_off(FFN_WD_OUT), hdh[ND - 1], dout, g, s,
                  false);
      acinh[0] = to_half4(dout[0]);
      acinh[1] = to_half4(sh);
      acb[0] = to_bf16x4(dout[0]);  // colour-net input, for its gradient
      acb[1] = to_bf16x4(sh);
      {
        floatx4 o[4];
        fwd16<4, 2>(sWf + A::wf_off(FFN_WC_IN), A::pf(FFN_WC_IN), sB + A::b_off(FFN_WC_IN), acinh, o, g, s, true);
#pragma unroll
        for (int t = 0; t < 4; ++t) hch[0][t] = to_half4(o[t]);
      }
#pragma unroll
      for (int i = 1; i < NC; ++i) {
        const int k = i == 1 ? FFN_WC_01 : (i == 2 ? FFN_WC_12 : FFN_WC_23);
        floatx4 o[4];
        fwd16<4, 4>(sWf + A::wf_off(k), A::pf(k), sB + A::b_off(k), hch[i - 1], o, g, s, true);
#pragma unroll
        for (int t = 0; t < 4; ++t) hch[i][t] = to_half4(o[t]);
      }
      {
        floatx4 co[1];
        fwd16<1, 4>(sWf + A::wf_off(FFN_WC_OUT), A::pf(FFN_WC_OUT), sB + A::b_off(FFN_WC_OUT), hch[NC - 1], co, g, s,
                    false);
        rgb_s[0] = sigmoid_soft(co[0][0]);
        rgb_s[1] = sigmoid_soft(co[0][1]);
        rgb_s[2] = sigmoid_soft(co[0][2]);
      }
      dout0 = dout[0][0];
    };
    float rgb_s[3], dout0;
    {
      half4 hdh[ND][4], acinh[2], hch[NC][4];
      bf16x4 acb[2];
      forward(hdh, acinh, acb, hch, rgb_s, dout0);
      if constexpr (TAPS) {
        if (a.t_relu) {
          uint32_t* rec = valid ? a.t_relu + (int64_t)RELU_WORDS * b : nullptr;
#pragma unroll
          for (int i = 0; i < ND; ++i) tap_relu(rec, i, hdh[i], g);
#pragma unroll
          for (int i = 0; i < NC; ++i) tap_relu(rec, 3 + i, hch[i], g);
        }
      }
    }
    if (g == 0) {
      float sig = softplus(fminf(fmaxf(dout0, -10.0f), 10.0f));
      if (dt_b <= 0.0f) sig = 0.0f;
      sSig[wave * 16 + s] = sig;
      sRgb[(wave * 16 + s) * 3 + 0] = rgb_s[0];
      sRgb[(wave * 16 + s) * 3 + 1] = rgb_s[1];
      sRgb[(wave * 16 + s) * 3 + 2] = rgb_s[2];
    }
    __syncthreads();

    float dLds_j, dLdc_j[3];
    composite_tile<TAPS>(a, sSig, sRgb, CL, lane, wave, prop_wave, train, proposals, Dhalf, dLds_j, dLdc_j);
    if (!train) continue;
    half4 hdh[ND][4], acinh[2], hch[NC][4];
    bf16x4 acb[2];
    {
      float rgb_r[3], dout_r;
      forward(hdh, acinh, acb, hch, rgb_r, dout_r);
    }

    // ---- backward (fp16 chain with per-wavefront delta scaling, fp32 accumulation); every layer's deltas
    // and inputs go through the stash for the block's bf16 weight-gradient tiles (barrier, this wave's
    // tiles, barrier before the stash is reused)
    const int col = wave * 16 + s;
    const float dLds = __shfl(dLds_j, col);
    const float dLdc0 = __shfl(dLdc_j[0], col), dLdc1 = __shfl(dLdc_j[1], col), dLdc2 = __shfl(dLdc_j[2], col);
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
    half4 dop[4];
    float dsc;
    floatx4 dc[4];
    stash_tiles<1>(sS, 0, dco, g, col);
    stash_tiles<4>(sS, 16, hch[NC - 1], g, col);
    {
      half4 cop[1];
      const float csc = make_op<1>(dco, cop);
#pragma unroll
      for (int t = 0; t < 4; ++t) dc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
      bwd16<4, 1>(sWt + A::wt_off(FFN_WC_OUT), A::pt(FFN_WC_OUT), cop, csc, dc, g, s);
      relu_mask16<4>(dc, hch[NC - 1]);
      dsc = make_op<4>(dc, dop);
    }
    __syncthreads();
    layer_dw16<1, 4, PS>(sS, gc_out, wave, g, s);
    __syncthreads();
    // hidden colour layers (Wc_23, Wc_12, Wc_01): delta dc of layer i's output, input hch[i - 1]
#pragma unroll
    for (int i = NC - 1; i >= 1; --i) {
      const int k = i == 1 ? FFN_WC_01 : (i == 2 ? FFN_WC_12 : FFN_WC_23);
      stash_tiles<4>(sS, 0, dc, g, col);
      stash_tiles<4>(sS, 64, hch[i - 1], g, col);
#pragma unroll
      for (int t = 0; t < 4; ++t) dc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
      bwd16<4, 4>(sWt + A::wt_off(k), A::pt(k), dop, dsc, dc, g, s);
      relu_mask16<4>(dc, hch[i - 1]);
      dsc = make_op<4>(dc, dop);
      __syncthreads();
      layer_dw16<4, 4, PS>(sS, gc_h[i - 1], wave, g, s);
      __syncthreads();
    }
    // colour input layer: its gradient, and the dout part of its input delta joins the density head's delta
    stash_tiles<4>(sS, 0, dc, g, col);
    stash_tiles<2>(sS, 64, acb, g, col);
    bwd16<1, 4>(sWt + A::wt_off(FFN_WC_IN), A::pt(FFN_WC_IN), dop, dsc, ddo, g, s);
    __syncthreads();
    layer_dw16<4, 2, PS>(sS, gc_in, wave, g, s);
    __syncthreads();
    // density output layer
    floatx4 dd[4];
    stash_tiles<1>(sS, 0, ddo, g, col);
    stash_tiles<4>(sS, 16, hdh[ND - 1], g, col);
    {
      half4 dd_op[1];
      const float ssc = make_op<1>(ddo, dd_op);
#pragma unroll
      for (int t = 0; t < 4; ++t) dd[t] = floatx4{0.f, 0.f, 0.f, 0.f};
      bwd16<4, 1>(sWt + A::wt_off(FFN_WD_OUT), A::pt(FFN_WD_OUT), dd_op, ssc, dd, g, s);
      relu_mask16<4>(dd, hdh[ND - 1]);
      dsc = make_op<4>(dd, dop);
    }
    __syncthreads();
    layer_dw16<1, 4, PS>(sS, gd_out, wave, g, s);
    __syncthreads();
    // hidden density layers (Wd_12, Wd_01)
#pragma unroll
    for (int i = ND - 1; i >= 1; --i) {
      const int k = i == 1 ? FFN_WD_01 : FFN_WD_12;
      stash_tiles<4>(sS, 0, dd, g, col);
      stash_tiles<4>(sS, 64, hdh[i - 1], g, col);
#pragma unroll
      for (int t = 0; t < 4; ++t) dd[t] = floatx4{0.f, 0.f, 0.f, 0.f};
      bwd16<4, 4>(sWt + A::wt_off(k), A::pt(k), dop, dsc, dd, g, s);
      relu_mask16<4>(dd, hdh[i - 1]);
      dsc = make_op<4>(dd, dop);
      __syncthreads();
      layer_dw16<4, 4, PS>(sS, gd_h[i - 1], wave, g, s);
      __syncthreads();
    }
    // density input layer: deltas and the encoding; encoding gradient dL/da0 = Wd_in^T . delta -> HBM
    stash_tiles<4>(sS, 0, dd, g, col);
    stash_tiles<KB0>(sS, 64, a0b, g, col);
    {
      floatx4 ga0[KB0];
#pragma unroll
      for (int t = 0; t < KB0; ++t) ga0[t] = floatx4{0.f, 0.f, 0.f, 0.f};
      bwd16<KB0, 4>(sWt + A::wt_off(FFN_WD_IN), A::pt(FFN_WD_IN), dop, dsc, ga0, g, s);
      if (valid) store_enc_grad<LF, FEAT>(a, b, g, ga0);
    }
    __syncthreads();
    layer_dw16<4, KB0, PS>(sS, gd_in, wave, g, s);
    // no barrier: the stash is next written after the next tile's compositing barrier
  }

  if (train) {
    // every wavefront stores its tiles into the block's partial gradient
    float* dst = a.partials + (int64_t)blockIdx.x * A::g_total();
    flush_layer16(dst + A::g_off(FFN_WC_OUT), FFN_C_OUT, FFN_M, gc_out, wave, g, s);
    if constexpr (NC >= 2) flush_layer16(dst + A::g_off(FFN_WC_01), FFN_M, FFN_M, gc_h[0], wave, g, s);
    if constexpr (NC >= 3) flush_layer16(dst + A::g_off(FFN_WC_12), FFN_M, FFN_M, gc_h[1], wave, g, s);
    if constexpr (NC >= 4) flush_layer16(dst + A::g_off(FFN_WC_23), FFN_M, FFN_M, gc_h[2], wave, g, s);
    flush_layer16(dst + A::g_off(FFN_WC_IN), FFN_M, FFN_C_IN, gc_in, wave, g, s);
    flush_layer16(dst + A::g_off(FFN_WD_OUT), FFN_D_OUT, FFN_M, gd_out, wave, g, s);
    if constexpr (ND >= 2) flush_layer16(dst + A::g_off(FFN_WD_01), FFN_M, FFN_M, gd_h[0], wave, g, s);
    if constexpr (ND >= 3) flush_layer16(dst + A::g_off(FFN_WD_12), FFN_M, FFN_M, gd_h[1], wave, g, s);
    flush_layer16(dst + A::g_off(FFN_WD_IN), FFN_M, LF, gd_in, wave, g, s);
  }
}

// ---------------------------------------------------------------------------

template <int LF, int ND, int NC, int FEAT, bool TAPS>
static hipError_t launch16_f(const MlpArgs& a, int n_blocks, hipStream_t st) {
  using A = Arch16<LF, ND, NC>;
  const size_t lds = A::lds_bytes();
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)k_mlp16<LF, ND, NC, FEAT, TAPS>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((k_mlp16<LF, ND, NC, FEAT, TAPS>), dim3(n_blocks), dim3(256), lds, st, a);
  return hipGetLastError();
}

template <int LF, int ND, int NC>
static hipError_t launch16_t(const MlpArgs& a, int n_blocks, hipStream_t st) {
  const bool taps = taps_requested(a);
  switch (a.c.F) {
    case 1:
      return taps ? launch16_f<LF, ND, NC, 1, true>(a, n_blocks, st) : launch16_f<LF, ND, NC, 1, false>(a, n_blocks, st);
    case 2:
      return taps ? launch16_f<LF, ND, NC, 2, true>(a, n_blocks, st) : launch16_f<LF, ND, NC, 2, false>(a, n_blocks, st);
    case 4:
      return taps ? launch16_f<LF, ND, NC, 4, true>(a, n_blocks, st) : launch16_f<LF, ND, NC, 4, false>(a, n_blocks, st);
    default: return hipErrorInvalidValue;
  }
}

#define FFN_MLP16_CONFIGS(X) \
  X(16, 1, 2)                \
  X(32, 1, 2)                \
  X(64, 1, 2)                \
  X(16, 2, 2)                \
  X(32, 2, 2)                \
  X(64, 2, 2)

int mlp16_blocks_per_cu(int LF, int nd, int nc) {
#define X(l, d, n) \
  if (LF == l && nd == d && nc == n) return Arch16<l, d, n>::blocks_per_cu();
  FFN_MLP16_CONFIGS(X)
#undef X
  return 1;
}

bool mlp16_supported(int LF, int nd, int nc) {
#define X(l, d, n) \
  if (LF == l && nd == d && nc == n) return true;
  FFN_MLP16_CONFIGS(X)
#undef X
  return false;
}

hipError_t launch_mlp16(const MlpArgs& a, int LF, int nd, int nc, int n_blocks, hipStream_t st) {
#define X(l, d, n) \
  if (LF == l && nd == d && nc == n) return launch16_t<l, d, n>(a, n_blocks, st);
  FFN_MLP16_CONFIGS(X)
#undef X
  return hipErrorInvalidValue;
}

}  // namespace ffn
