// ffn_mlp16.hip -- the fused MLP step on 16-bit MFMAs with fp32 accumulation:
// forward and backward chains in fp16, weight gradients in bf16 (whose
// fp32-sized exponent takes the unscaled deltas of all four wavefronts); each
// layer's fp16 deltas are scaled by a per-sample power of two that puts their
// largest magnitude just below 2^14, so small deltas neither underflow nor
// lose bits.  Same semantics as the fp32 kernel (ffnerf_OG.cl:1373-2082,
// weight_update.cl:210-341): compositing, loss gradient, proposals and output
// deltas are the shared fp32 code.
//
// MI355X design
//   * A 256-thread block (4 wavefronts) walks 64-sample tiles in a persistent
//     loop.  Each wavefront runs the layers for its 16 samples of the tile; a
//     layer's output tile (lane (g, s) holds neurons 16t + 4g + r of sample s)
//     is exactly one half of the next layer's B operand.
//   * gfx950's K = 32 MFMAs (v_mfma_f32_16x16x32_f16 / _bf16): lane group g
//     supplies eight K values per operand.  Slot j of group g in K block kb
//     stands for neuron 32 kb + 16 (j / 4) + 4 g + j % 4, i.e. the four values
//     of output tile 2 kb and the four of tile 2 kb + 1 that the lane already
//     holds -- activations never move between lanes; the weights in LDS are
//     stored with their K columns in that order, so every A operand is one
//     16-byte LDS read.  Layers with K = 16 (the output layers' backward, a
//     16-wide encoding) keep v_mfma_f32_16x16x16.
//   * Per tile: every wavefront runs the forward of its samples, keeping the
//     hidden activations as bf16 K blocks, and leaves sigma and rgb in LDS;
//     after a barrier the tile's proposal wavefront composites it alone (64
//     lanes, its proposals too) and leaves dL/dsigma, dL/dc in LDS -- one
//     compositing per tile, not one per wavefront; the other SIMDs run the
//     CU's other block meanwhile.  After a second barrier, the backward.
//   * Weight gradients dW = delta . act^T need the samples as K.  Layer by
//     layer in the backward, every wavefront writes its deltas and the layer's
//     input activations, transposed, into a block-shared bf16 stash (rows =
//     neurons, 64 samples per row); after a barrier the layer's 16x16 gradient
//     tiles are dealt round-robin over the four wavefronts, each of which
//     accumulates its tiles over the tile's 64 samples (two K = 32 MFMAs per
//     tile) in registers for the whole kernel and stores them into the
//     block's partial at the end.
//   * The backward's fp16 deltas are scaled per sample (the column of the
//     next MFMA's B operand) by the power of two that puts the sample's
//     largest delta in [2^13, 2^14).
#include "ffn_device.h"
#include "ffn_kernels.h"
#include "ffn_mlp_common.h"

namespace ffn {

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ floatx4 mfma_k16(const half4& a, const half4& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma_k32(const half8& a, const half8& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mfma_k32b(const bf16x8& a, const bf16x8& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// neuron of K slot j of lane group g in K block kb (see the file comment)
__host__ __device__ constexpr int kslot_neuron(int kb, int g, int j) {
  return 32 * kb + 16 * (j >> 2) + 4 * g + (j & 3);
}
// the same for the position p = 32 kb + 8 g + j of a K-ordered row
__host__ __device__ constexpr int kpos_neuron(int p) { return kslot_neuron(p >> 5, (p >> 3) & 3, p & 7); }

__device__ __forceinline__ half4 to_half4(const floatx4& v) {
  half4 h;
#pragma unroll
  for (int r = 0; r < 4; ++r) h[r] = (_Float16)v[r];
  return h;
}
// K block of two D-layout tiles: slots 0-3 = tile lo, slots 4-7 = tile hi
__device__ __forceinline__ half8 to_half8(const floatx4& lo, const floatx4& hi) {
  half8 h;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    h[r] = (_Float16)lo[r];
    h[4 + r] = (_Float16)hi[r];
  }
  return h;
}
// the same K block in bf16 (two values per v_cvt_pk_bf16_f32)
__device__ __forceinline__ bf16x8 to_bf16x8(const floatx4& lo, const floatx4& hi) {
  typedef float float2_ __attribute__((ext_vector_type(2)));
  const bf16x2 p0 = __builtin_convertvector(float2_{lo[0], lo[1]}, bf16x2);
  const bf16x2 p1 = __builtin_convertvector(float2_{lo[2], lo[3]}, bf16x2);
  const bf16x2 p2 = __builtin_convertvector(float2_{hi[0], hi[1]}, bf16x2);
  const bf16x2 p3 = __builtin_convertvector(float2_{hi[2], hi[3]}, bf16x2);
  return bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}
__device__ __forceinline__ half8 join8(const half4& lo, const half4& hi) {
  return half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
__device__ __forceinline__ bf16x4 to_bf16x4(const floatx4& v) {
  bf16x4 h;
#pragma unroll
  for (int r = 0; r < 4; ++r) h[r] = (__bf16)v[r];
  return h;
}

// power of two per sample (column of the next backward MFMA's B operand, whose K values the sample's four
// lanes l, l ^ 16, l ^ 32, l ^ 48 hold) that maps the largest |d| of its deltas into [2^13, 2^14) (1 if all
// zero); *inv its reciprocal
template <int NT>
__device__ __forceinline__ float delta_scale(const floatx4 (&d)[NT], float* inv) {
  float m = 0.0f;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) m = fmaxf(m, fabsf(d[t][r]));
  {
    // the maxima of non-negative floats as unsigned maxima of their bit patterns (the float form
    // canonicalises both swapped operands first)
    const unsigned int u = __float_as_uint(m);
    const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const unsigned int u2 = p[0] > p[1] ? p[0] : p[1];
    const auto q = __builtin_amdgcn_permlane16_swap(u2, u2, false, false);
    m = __uint_as_float(q[0] > q[1] ? q[0] : q[1]);
  }
  int e = 0;
  if (m > 0.0f && m < 3.0e38f) {
    frexpf(m, &e);  // m < 2^e
    e = 14 - e;
    e = e > 100 ? 100 : (e < -100 ? -100 : e);
  }
  *inv = ldexpf(1.0f, -e);
  return ldexpf(1.0f, e);
}

template <int LF_, int ND_, int NC_>
struct Arch16 {
  static constexpr int LF = LF_, ND = ND_, NC = NC_;
  static constexpr int rows_pad(int k) { return k == FFN_WC_OUT ? 16 : layer_out(k); }
  // forward copy [rows_pad][in + 8] (columns in K-slot order when in is a multiple of 32); transposed copy
  // for the backward [in][rows_pad + 8] (columns in K-slot order when rows_pad is a multiple of 32).  The
  // 8-half pad keeps the 16-byte reads aligned and spreads a tile's 16 rows over distinct banks.
  static constexpr int pf(int k) { return layer_in(k, LF) + 8; }
  static constexpr int pt(int k) { return rows_pad(k) + 8; }
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
  static constexpr int PS = 64 + 8;
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
  // sigma[64] + rgb[64][3] of the tile (the compositing overwrites them with dL/dsigma, dL/dc): one slot
  // when training (the stash barriers separate a tile's compositing from the next tile's writes), two
  // alternating slots for a forward-only launch
  static constexpr int comp_floats = 512;
  static constexpr size_t lds_bytes() {
    return (size_t)w_halves() * 2 + (size_t)b_floats() * 4 + (size_t)stash_halves() * 2 + comp_floats * 4;
  }
  static constexpr int blocks_per_cu() { return lds_bytes() <= 80 * 1024 ? 2 : 1; }
};

// forward layer, K = 32 blocks: out tiles = act(W . in + b); W is the K-ordered forward copy
template <int OT, int KB>
__device__ __forceinline__ void fwd_k32(const _Float16* __restrict__ W, int P, const float* __restrict__ B,
                                        const half8 (&in)[KB], floatx4 (&out)[OT], int g, int s, bool relu) {
  floatx4 acc[OT];
#pragma unroll
  for (int t = 0; t < OT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[t][r] = B[16 * t + 4 * g + r];
  // Software-pipelined weight reads: the first K block's operands are all read before its MFMAs; then each
  // MFMA's weight register takes the next K block's operand of the same output tile while the other tiles'
  // MFMAs run (a single output tile double-buffers instead)
  auto wread = [&](int t, int kb) { return *reinterpret_cast<const half8*>(W + (16 * t + s) * P + 32 * kb + 8 * g); };
  if constexpr (OT == 1) {
    half8 w_cur = wread(0, 0);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      half8 w_nxt = w_cur;
      if (kb + 1 < KB) w_nxt = wread(0, kb + 1);
      acc[0] = mfma_k32(w_cur, in[kb], acc[0]);
      w_cur = w_nxt;
    }
  } else {
    half8 w[OT];
#pragma unroll
    for (int t = 0; t < OT; ++t) w[t] = wread(t, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
      for (int t = 0; t < OT; ++t) {
        acc[t] = mfma_k32(w[t], in[kb], acc[t]);
        if (kb + 1 < KB) w[t] = wread(t, kb + 1);
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

// forward layer with K = 16 (a 16-wide encoding): natural column order
template <int OT>
__device__ __forceinline__ void fwd_k16(const _Float16* __restrict__ W, int P, const float* __restrict__ B,
                                        const half4& in, floatx4 (&out)[OT], int g, int s, bool relu) {
  half4 w[OT];  // every weight operand read before the MFMAs
#pragma unroll
  for (int t = 0; t < OT; ++t) w[t] = *reinterpret_cast<const half4*>(W + (16 * t + s) * P + 4 * g);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < OT; ++t) {
    floatx4 acc;
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = B[16 * t + 4 * g + r];
    acc = mfma_k16(w[t], in, acc);
    if (relu) {
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = relu_f(acc[r]);
    }
    out[t] = acc;
  }
}

// backward layer over a 64-wide output (K = 32 blocks): res tiles over input neurons += (W^T . op) / sc (= when
// !ACC), with Wt the K-ordered transposed copy and op the scaled fp16 deltas
template <int RT, bool ACC = true>
__device__ __forceinline__ void bwd_k32(const _Float16* __restrict__ Wt, int P, const half8 (&op)[2], float inv,
                                        floatx4 (&res)[RT], int g, int s) {
  floatx4 acc[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  // weight reads pipelined as in fwd_k32
  auto wread = [&](int t, int kb) { return *reinterpret_cast<const half8*>(Wt + (16 * t + s) * P + 32 * kb + 8 * g); };
  if constexpr (RT == 1) {
    const half8 w0 = wread(0, 0), w1 = wread(0, 1);
    acc[0] = mfma_k32(w0, op[0], acc[0]);
    acc[0] = mfma_k32(w1, op[1], acc[0]);
  } else {
    half8 w[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) w[t] = wread(t, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        acc[t] = mfma_k32(w[t], op[kb], acc[t]);
        if (kb == 0) w[t] = wread(t, 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) res[t][r] = ACC ? res[t][r] + acc[t][r] * inv : acc[t][r] * inv;
}

// backward layer over a 16-wide output (K = 16): natural column order
template <int RT, bool ACC = true>
__device__ __forceinline__ void bwd_k16(const _Float16* __restrict__ Wt, int P, const half4& op, float inv,
                                        floatx4 (&res)[RT], int g, int s) {
  half4 w[RT];  // every weight operand read before the MFMAs
#pragma unroll
  for (int t = 0; t < RT; ++t) w[t] = *reinterpret_cast<const half4*>(Wt + (16 * t + s) * P + 4 * g);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const floatx4 acc = mfma_k16(w[t], op, floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
    for (int r = 0; r < 4; ++r) res[t][r] = ACC ? res[t][r] + acc[r] * inv : acc[r] * inv;
  }
}

// zero the deltas of inactive ReLUs (act: the forward's bf16 activations, two tiles per K block).  An
// activation is +0 or positive (the ReLU maps everything else to +0), so it is active when its bits are not
// all zero: tested on the packed words (low half: the low 16 bits; high half: the word above 0xffff)
__device__ __forceinline__ void relu_mask(floatx4 (&d)[4], const bf16x8 (&act)[2]) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const u32x4 wv = __builtin_bit_cast(u32x4, act[t >> 1]);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const unsigned int word = wv[(4 * (t & 1) + r) >> 1];
      const bool on = (r & 1) ? word > 0xffffu : (unsigned short)word != 0;
      d[t][r] = on ? d[t][r] : 0.0f;
    }
  }
}

// the next layer's operands from four delta tiles: scale and fp16 K blocks
__device__ __forceinline__ float make_op4(const floatx4 (&d)[4], half8 (&op)[2]) {
  float inv;
  const float sc = delta_scale<4>(d, &inv);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      op[kb][r] = (_Float16)(d[2 * kb][r] * sc);
      op[kb][4 + r] = (_Float16)(d[2 * kb + 1][r] * sc);
    }
  return inv;
}
__device__ __forceinline__ float make_op1(const floatx4 (&d)[1], half4& op) {
  float inv;
  const float sc = delta_scale<1>(d, &inv);
#pragma unroll
  for (int r = 0; r < 4; ++r) op[r] = (_Float16)(d[0][r] * sc);
  return inv;
}

// One packed word per lane into the stash: lane (g, s) holds rows n, n + 1 (n = row0 + 16 t + 4 g + r, r
// even) of sample column `col` as the low and high half.  Neighbouring lanes s, s ^ 1 swap their words (DPP
// quad permutation [1, 0, 3, 2]); the even lane then writes row n and the odd lane row n + 1, each for the
// column pair (col & ~1, col | 1) as one 32-bit store (sel: the byte selector stash_sel(s) gives the lane).
__device__ __forceinline__ unsigned int stash_sel(int s) { return (s & 1) ? 0x03020706u : 0x05040100u; }
__device__ __forceinline__ void stash_pair(__bf16* __restrict__ st, int n, int col, unsigned int sel,
                                           unsigned int w) {
  constexpr int PS = 64 + 8;
  // every lane receives a neighbour's word, so the move needs no old value (update_dpp with old = w had the
  // compiler copy w into the destination first: one more instruction per stashed word; 3.38 -> 3.33 ms)
  const unsigned int nb = (unsigned int)__builtin_amdgcn_mov_dpp((int)w, 0xB1, 0xF, 0xF, false);
  const unsigned int v = __builtin_amdgcn_perm(nb, w, sel);
  *reinterpret_cast<unsigned int*>(st + (n + (col & 1)) * PS + (col & ~1)) = v;
}

// stash rows row0 + 16 t + 4 g + r, column `col`, of NT D-layout tiles (value(t, r)); two values per
// conversion (v_cvt_pk_bf16_f32), the low and the high half of the packed word
template <int NT, typename F>
__device__ __forceinline__ void stash_rows(__bf16* __restrict__ st, int row0, int g, int col, F value) {
  const unsigned int sel = stash_sel(col);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; r += 2) {
      typedef float float2_ __attribute__((ext_vector_type(2)));
      const bf16x2 p = __builtin_convertvector(float2_{value(t, r), value(t, r + 1)}, bf16x2);
      stash_pair(st, row0 + 16 * t + 4 * g + r, col, sel, __builtin_bit_cast(unsigned int, p));
    }
}

// stash rows row0 + 16 t + 4 g + r, column `col`, of NT tiles given as packed bf16 words (word(t, r / 2)
// holds rows r and r + 1), no conversion
template <int NT, typename F>
__device__ __forceinline__ void stash_words(__bf16* __restrict__ st, int row0, int g, int col, F word) {
  const unsigned int sel = stash_sel(col);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; r += 2) stash_pair(st, row0 + 16 * t + 4 * g + r, col, sel, word(t, r >> 1));
}
// NT bf16 tiles held two per K block (act[t / 2], slots 4 (t % 2) + r)
template <int NT, int NB>
__device__ __forceinline__ void stash_act(__bf16* __restrict__ st, int row0, int g, int col, const bf16x8 (&act)[NB]) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  stash_words<NT>(st, row0, g, col, [&](int t, int p) {
    return __builtin_bit_cast(u32x4, act[t >> 1])[2 * (t & 1) + p];
  });
}

// One wavefront's weight-gradient tiles of a layer (D layout) and, for its tile with Tp = 0, a per-lane
// partial of the bias gradient.
template <int OT, int IT>
struct WaveGrad16 {
  static constexpr int N = OT * IT / 4;
  static_assert(OT * IT % 4 == 0, "a layer's gradient tiles split evenly over four wavefronts");
  floatx4 w[N];
  float b;  // the bias partial of the wavefront's tile with Tp = 0 (at most one per layer, deal_tile)
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int m = 0; m < N; ++m) w[m] = floatx4{0.f, 0.f, 0.f, 0.f};
    b = 0.0f;
  }
};

// this wavefront's dW tiles over the 64 stashed samples (delta rows [0, 16 OT), activation rows after): two
// K = 32 blocks of samples, lane group g reading samples 32 q + 8 g .. + 7 of both operands
template <int OT, int IT, int PS>
__device__ __forceinline__ void layer_dw(const __bf16* __restrict__ st, WaveGrad16<OT, IT>& acc, int wave, int g,
                                         int s) {
#pragma unroll
  for (int m = 0; m < WaveGrad16<OT, IT>::N; ++m) {
    int T, Tp;
    deal_tile<IT>(m, wave, T, Tp);
    const __bf16* drow = st + (16 * T + s) * PS + 8 * g;
    const __bf16* arow = st + (16 * (OT + Tp) + s) * PS + 8 * g;
    floatx4 c = acc.w[m];
    float bs = acc.b;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const bf16x8 dv = *reinterpret_cast<const bf16x8*>(drow + 32 * q);
      const bf16x8 av = *reinterpret_cast<const bf16x8*>(arow + 32 * q);
      c = mfma_k32b(dv, av, c);
      if (Tp == 0)
        bs += (((float)dv[0] + (float)dv[1]) + ((float)dv[2] + (float)dv[3])) +
              (((float)dv[4] + (float)dv[5]) + ((float)dv[6] + (float)dv[7]));
    }
    acc.w[m] = c;
    if (Tp == 0) acc.b = bs;
  }
}

// store this wavefront's tiles of a layer into the block's partial gradient (packed [O][In] + [O])
template <int OT, int IT>
__device__ __forceinline__ void flush_layer16(float* __restrict__ dst, int O, int In, const WaveGrad16<OT, IT>& acc,
                                              int wave, int g, int s) {
#pragma unroll
  for (int m = 0; m < WaveGrad16<OT, IT>::N; ++m) {
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

// this lane's encoding values: a0v[4 kb + j] = neuron 16 kb + 4 g + j of sample b (0 when !valid)
template <int LF, int FEAT>
__device__ __forceinline__ void load_a0(const float* __restrict__ a0, const FeatLayout& feat, int64_t b, bool valid,
                                        int g, float (&a0v)[LF / 4]) {
  if (!valid) {
#pragma unroll
    for (int q = 0; q < LF / 4; ++q) a0v[q] = 0.0f;
    return;
  }
#pragma unroll
  for (int kb = 0; kb < LF / 16; ++kb) {
    if constexpr (FEAT == 4) {
      const int l = 4 * kb + g;
      const float4 v = *reinterpret_cast<const float4*>(a0 + l * feat.stride_l + b * feat.stride_b);
      a0v[4 * kb] = v.x;
      a0v[4 * kb + 1] = v.y;
      a0v[4 * kb + 2] = v.z;
      a0v[4 * kb + 3] = v.w;
    } else if constexpr (FEAT == 2) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int l = 8 * kb + 2 * g + h;
        const float2 v = *reinterpret_cast<const float2*>(a0 + l * feat.stride_l + b * feat.stride_b);
        a0v[4 * kb + 2 * h] = v.x;
        a0v[4 * kb + 2 * h + 1] = v.y;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) a0v[4 * kb + j] = a0[(16 * kb + 4 * g + j) * feat.stride_l + b * feat.stride_b];
    }
  }
}

// The network's forward for this wavefront's 16 samples: a0 (fp16 K blocks, or one K = 16 operand when
// LF = 16) through the density net, [dout | SH] through the colour net, each layer's input an fp16
// operand.  With KEEP the hidden activations are also kept as bf16 K blocks (hd, hc; the colour net's
// input cin), which the backward's ReLU masks and weight-gradient stash read; rgb and the density head's
// first output for the lane.
template <int LF, int ND, int NC>
struct Fwd16 {
  bf16x8 hd[ND][2];
  bf16x8 cin;
  bf16x8 hc[NC][2];
  float rgb[3];
  float dout0;
};

template <int LF, int ND, int NC, typename A, bool KEEP>
__device__ __forceinline__ void forward16(const _Float16* __restrict__ sWf, const float* __restrict__ sB,
                                          const float (&a0v)[LF / 4], const floatx4& sh, int g, int s,
                                          Fwd16<LF, ND, NC>& f) {
  floatx4 o[4];
  if constexpr (LF >= 32) {
    half8 a0k[LF / 32];
#pragma unroll
    for (int kb = 0; kb < LF / 32; ++kb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        a0k[kb][j] = (_Float16)a0v[8 * kb + j];          // neuron 32 kb + 4 g + j
        a0k[kb][4 + j] = (_Float16)a0v[8 * kb + 4 + j];  // neuron 32 kb + 16 + 4 g + j
      }
    fwd_k32<4, LF / 32>(sWf + A::wf_off(FFN_WD_IN), A::pf(FFN_WD_IN), sB + A::b_off(FFN_WD_IN), a0k, o, g, s, true);
  } else {
    half4 a0q;
#pragma unroll
    for (int j = 0; j < 4; ++j) a0q[j] = (_Float16)a0v[j];
    fwd_k16<4>(sWf + A::wf_off(FFN_WD_IN), A::pf(FFN_WD_IN), sB + A::b_off(FFN_WD_IN), a0q, o, g, s, true);
  }
  half8 x[2] = {to_half8(o[0], o[1]), to_half8(o[2], o[3])};  // the next layer's input
  if constexpr (KEEP) {
    f.hd[0][0] = to_bf16x8(o[0], o[1]);
    f.hd[0][1] = to_bf16x8(o[2], o[3]);
  }
#pragma unroll
  for (int i = 1; i < ND; ++i) {
    const int k = i == 1 ? FFN_WD_01 : FFN_WD_12;
    fwd_k32<4, 2>(sWf + A::wf_off(k), A::pf(k), sB + A::b_off(k), x, o, g, s, true);
    x[0] = to_half8(o[0], o[1]);
    x[1] = to_half8(o[2], o[3]);
    if constexpr (KEEP) {
      f.hd[i][0] = to_bf16x8(o[0], o[1]);
      f.hd[i][1] = to_bf16x8(o[2], o[3]);
    }
  }
  floatx4 dout[1];
  fwd_k32<1, 2>(sWf + A::wf_off(FFN_WD_OUT), A::pf(FFN_WD_OUT), sB + A::b_off(FFN_WD_OUT), x, dout, g, s, false);
  if constexpr (KEEP) f.cin = to_bf16x8(dout[0], sh);
  {
    const half8 cin[1] = {to_half8(dout[0], sh)};
    fwd_k32<4, 1>(sWf + A::wf_off(FFN_WC_IN), A::pf(FFN_WC_IN), sB + A::b_off(FFN_WC_IN), cin, o, g, s, true);
  }
  x[0] = to_half8(o[0], o[1]);
  x[1] = to_half8(o[2], o[3]);
  if constexpr (KEEP) {
    f.hc[0][0] = to_bf16x8(o[0], o[1]);
    f.hc[0][1] = to_bf16x8(o[2], o[3]);
  }
#pragma unroll
  for (int i = 1; i < NC; ++i) {
    const int k = i == 1 ? FFN_WC_01 : (i == 2 ? FFN_WC_12 : FFN_WC_23);
    fwd_k32<4, 2>(sWf + A::wf_off(k), A::pf(k), sB + A::b_off(k), x, o, g, s, true);
    x[0] = to_half8(o[0], o[1]);
    x[1] = to_half8(o[2], o[3]);
    if constexpr (KEEP) {
      f.hc[i][0] = to_bf16x8(o[0], o[1]);
      f.hc[i][1] = to_bf16x8(o[2], o[3]);
    }
  }
  floatx4 co[1];
  fwd_k32<1, 2>(sWf + A::wf_off(FFN_WC_OUT), A::pf(FFN_WC_OUT), sB + A::b_off(FFN_WC_OUT), x, co, g, s, false);
  f.rgb[0] = sigmoid_soft(co[0][0]);
  f.rgb[1] = sigmoid_soft(co[0][1]);
  f.rgb[2] = sigmoid_soft(co[0][2]);
  f.dout0 = dout[0][0];
}

// ReLU taps from bf16 K blocks (two tiles each)
__device__ __forceinline__ void tap_relu8(uint32_t* rec, int h, const bf16x8 (&act)[2], int g) {
  bf16x4 t4[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) t4[t] = bf16x4{act[t >> 1][4 * (t & 1)], act[t >> 1][4 * (t & 1) + 1],
                                             act[t >> 1][4 * (t & 1) + 2], act[t >> 1][4 * (t & 1) + 3]};
  tap_relu(rec, h, t4, g);
}

// what a wavefront reads from HBM for its 16 samples of a tile; loaded one tile ahead of its use
template <int LF>
struct TileIn {
  float a0v[LF / 4];
  float4 rd;  // the ray direction
  float dt, t;
};
// MARCHED: sample b is a.smp[b] of ray a.ray_ids[b], lattice step a.march_dt
template <int LF, int FEAT, bool MARCHED>
__device__ __forceinline__ void load_tile_in(const MlpArgs& a, int64_t b, bool valid, int g, int log2S,
                                             TileIn<LF>& in) {
  load_a0<LF, FEAT>(a.a0, a.feat, b, valid, g, in.a0v);
  if constexpr (MARCHED) {
    in.rd = a.rays[2 * (valid ? (int64_t)a.ray_ids[b] : 0) + 1];
    in.dt = valid ? a.march_dt : 0.0f;
    in.t = valid ? a.smp[b].w : 0.0f;
  } else {
    in.rd = a.rays[2 * (valid ? (b >> log2S) : 0) + 1];
    in.dt = valid ? a.DTs[b] : 0.0f;
    in.t = valid ? a.Ts[b] : 0.0f;
  }
}

// MARCHED: the backward over marched samples (every tile busy): the loss gradients are read from a.in_dLds /
// a.in_dLdc, the samples' rays, times and step from the march; no compositing, no proposals.  TRAIN
// (a.do_train) is a template parameter for the reason given at k_mlp.
template <int LF, int ND, int NC, int FEAT, bool TAPS, bool MARCHED, int SC, bool TRAIN>
__global__ __launch_bounds__(256, (Arch16<LF, ND, NC>::blocks_per_cu())) void k_mlp16(MlpArgs a) {
  static_assert(TRAIN || !MARCHED, "marched launches train");
  using A = Arch16<LF, ND, NC>;
  constexpr int KB0 = LF / 16;  // D-layout tiles of the encoding
  extern __shared__ __align__(16) unsigned char smem16[];
  _Float16* sWf = reinterpret_cast<_Float16*>(smem16);
  _Float16* sWt = sWf;  // the transposed copies follow the forward weights (offsets in 16-bit units)
  float* sB = reinterpret_cast<float*>(smem16 + (size_t)A::w_halves() * 2);
  __bf16* sS = reinterpret_cast<__bf16*>(smem16 + (size_t)A::w_halves() * 2 + (size_t)A::b_floats() * 4);
  float* sC = reinterpret_cast<float*>(smem16 + (size_t)A::w_halves() * 2 + (size_t)A::b_floats() * 4 +
                                       (size_t)A::stash_halves() * 2);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
  const int col = wave * 16 + s;  // this lane's sample column in a tile
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

  // weights: fp16 [out_pad][in] and [in][out_pad] (K-ordered columns where K blocks are 32 wide, zero
  // padding), fp32 biases
#pragma unroll
  for (int k = 0; k < FFN_N_LAYERS; ++k) {
    if (!layer_active(k, ND, NC)) continue;
    const int O = layer_out(k), I = layer_in(k, LF), R = A::rows_pad(k);
    const int PF = A::pf(k), PT = A::pt(k);
    const bool kf = I % 32 == 0, kt = R % 32 == 0;
    const float* gw = a.w.W[k];
    for (int e = tid; e < R * PF; e += 256) {
      const int r = e / PF, p = e - r * PF;
      const int i = p < I ? (kf ? kpos_neuron(p) : p) : I;
      sWf[A::wf_off(k) + e] = (_Float16)((r < O && i < I) ? gw[r * I + i] : 0.0f);
    }
    for (int e = tid; e < I * PT; e += 256) {
      const int i = e / PT, p = e - i * PT;
      const int o = p < R ? (kt ? kpos_neuron(p) : p) : R;
      sWt[A::wt_off(k) + e] = (_Float16)((o < O) ? gw[o * I + i] : 0.0f);
    }
    for (int e = tid; e < R; e += 256) sB[A::b_off(k) + e] = e < O ? a.w.b[k][e] : 0.0f;
  }
  __syncthreads();

  const float Dhalf = half_box_diagonal(c);
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

  // The busy tiles (a sample with dt > 0), which the tile order puts first, take the full path; a tile
  // whose samples are all inactive (e.g. a ray that misses the box) composites to exactly the background
  // and all its gradients are zero, so the later positions only write that (empty_tile).  Taps, which expose
  // per-sample MLP outputs, take the full path for every tile.  (Two loops: an exit from the full path for
  // the empty tiles had the register allocator copy the gradient accumulators on every tile.)
  const int64_t n_full = (TAPS || MARCHED || !a.n_busy) ? n_tiles : (int64_t)*a.n_busy;
  int parity = 0;
  int64_t ti = blockIdx.x;
#pragma unroll 1
  for (; ti < n_full; ti += gridDim.x, parity ^= 1) {
    const int64_t tile = a.tile_order ? (int64_t)a.tile_order[ti] : ti;
    float* sSig = sC + (train ? 0 : parity * 256);
    float* sRgb = sSig + 64;
    const int64_t b = tile * 64 + col;
    const bool valid = (uint64_t)b < n_samples;
    TileIn<LF> cur;
    load_tile_in<LF, FEAT, MARCHED>(a, b, valid, g, log2S, cur);
    // per-sample inputs of the compositing (lane j = sample j of the tile), loaded before the forward so
    // that their latency hides behind it
    const bool prop_wave = (int)(tile & 3) == wave;  // this wavefront composites the tile
    CompLane CL{};
    if constexpr (!MARCHED) {
      CL = load_comp_lane<SC>(a, tile, lane, prop_wave, n_samples, log2S, proposals);
    }
    const float dirv[3] = {cur.rd.x, cur.rd.y, cur.rd.z};
    floatx4 sh;
#pragma unroll
    for (int r = 0; r < 4; ++r) sh[r] = sh_component(dirv, 4 * g + r) * a.sh_mult;
    const float dt_b = cur.dt, t_b = cur.t;
    Fwd16<LF, ND, NC> f;
    forward16<LF, ND, NC, A, true>(sWf, sB, cur.a0v, sh, g, s, f);
    if constexpr (TAPS) {
      if (a.t_relu) {
        uint32_t* rec = valid ? a.t_relu + (int64_t)RELU_WORDS * b : nullptr;
#pragma unroll
        for (int i = 0; i < ND; ++i) tap_relu8(rec, i, f.hd[i], g);
#pragma unroll
        for (int i = 0; i < NC; ++i) tap_relu8(rec, 3 + i, f.hc[i], g);
      }
    }
    unsigned int a0w[KB0][2];  // the encoding as the stash holds it: bf16 of the fp32 values, packed in pairs
#pragma unroll
    for (int t = 0; t < KB0; ++t)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        typedef float float2_ __attribute__((ext_vector_type(2)));
        a0w[t][p] = __builtin_bit_cast(unsigned int, __builtin_convertvector(
                                                         float2_{cur.a0v[4 * t + 2 * p], cur.a0v[4 * t + 2 * p + 1]},
                                                         bf16x2));
      }
    float dLds, dLdc0, dLdc1, dLdc2;
    if constexpr (MARCHED) {
      __syncthreads();  // the previous tile's last gradient tiles have read the stash
      dLds = valid ? a.in_dLds[b] : 0.0f;
      dLdc0 = valid ? a.in_dLdc[3 * b] : 0.0f;
      dLdc1 = valid ? a.in_dLdc[3 * b + 1] : 0.0f;
      dLdc2 = valid ? a.in_dLdc[3 * b + 2] : 0.0f;
    } else {
      if (g == 0) {
        float sig = softplus(fminf(fmaxf(f.dout0, -10.0f), 10.0f));
        if (dt_b <= 0.0f) sig = 0.0f;
        sSig[col] = sig;
        sRgb[col * 3 + 0] = f.rgb[0];
        sRgb[col * 3 + 1] = f.rgb[1];
        sRgb[col * 3 + 2] = f.rgb[2];
      }
      __syncthreads();
      // compositing on 64 lanes by the tile's proposal wavefront, which also writes the output colour (and
      // taps); its loss gradients replace sigma and rgb in LDS (only it reads them), and after a barrier
      // every wavefront reads its own samples'.  The other three SIMDs meanwhile run the CU's other block.
      // The compositing wavefront runs at a raised issue priority: the rest of its block waits for it
      // (3.44 -> 3.37 ms).  Turns of the two blocks at two levels, which the fp32 kernel takes, measured
      // 3.46-3.49 ms here, where MFMAs and vector instructions of the two blocks issue together.
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
        __builtin_amdgcn_s_setprio(0);
      }
      if (!train) continue;
      __syncthreads();
      dLds = sSig[col];
      dLdc0 = sRgb[3 * col];
      dLdc1 = sRgb[3 * col + 1];
      dLdc2 = sRgb[3 * col + 2];
    }
    floatx4 dco[1] = {{0.f, 0.f, 0.f, 0.f}};
    floatx4 ddo[1] = {{0.f, 0.f, 0.f, 0.f}};
    if (g == 0 && valid) {
      float d3[3], dd0;
      output_deltas(t_b, dt_b, Dhalf, dLds, dLdc0, dLdc1, dLdc2, f.rgb, f.dout0, d3, dd0);
      dco[0][0] = d3[0];
      dco[0][1] = d3[1];
      dco[0][2] = d3[2];
      ddo[0][0] = dd0;
    }
    // colour output layer
    half8 dop[2];
    float dsc;
    floatx4 dc[4];
    stash_rows<1>(sS, 0, g, col, [&](int t, int r) { return dco[t][r]; });
    stash_act<4>(sS, 16, g, col, f.hc[NC - 1]);
    {
      half4 cop;
      const float csc = make_op1(dco, cop);
      bwd_k16<4, false>(sWt + A::wt_off(FFN_WC_OUT), A::pt(FFN_WC_OUT), cop, csc, dc, g, s);
      relu_mask(dc, f.hc[NC - 1]);
      dsc = make_op4(dc, dop);
    }
    __syncthreads();
    layer_dw<1, 4, PS>(sS, gc_out, wave, g, s);
    __syncthreads();
    // hidden colour layers (Wc_23, Wc_12, Wc_01): delta dc of layer i's output, input hc[i - 1]
#pragma unroll
    for (int i = NC - 1; i >= 1; --i) {
      const int k = i == 1 ? FFN_WC_01 : (i == 2 ? FFN_WC_12 : FFN_WC_23);
      stash_rows<4>(sS, 0, g, col, [&](int t, int r) { return dc[t][r]; });
      stash_act<4>(sS, 64, g, col, f.hc[i - 1]);
      bwd_k32<4, false>(sWt + A::wt_off(k), A::pt(k), dop, dsc, dc, g, s);
      relu_mask(dc, f.hc[i - 1]);
      dsc = make_op4(dc, dop);
      __syncthreads();
      layer_dw<4, 4, PS>(sS, gc_h[i - 1], wave, g, s);
      __syncthreads();
    }
    // colour input layer: its gradient, and the dout part of its input delta joins the density head's delta
    stash_rows<4>(sS, 0, g, col, [&](int t, int r) { return dc[t][r]; });
    {
      const bf16x8 cin[1] = {f.cin};
      stash_act<2>(sS, 64, g, col, cin);
    }
    bwd_k32<1>(sWt + A::wt_off(FFN_WC_IN), A::pt(FFN_WC_IN), dop, dsc, ddo, g, s);
    __syncthreads();
    layer_dw<4, 2, PS>(sS, gc_in, wave, g, s);
    __syncthreads();
    // density output layer
    floatx4 dd[4];
    stash_rows<1>(sS, 0, g, col, [&](int t, int r) { return ddo[t][r]; });
    stash_act<4>(sS, 16, g, col, f.hd[ND - 1]);
    {
      half4 dd_op;
      const float ssc = make_op1(ddo, dd_op);
      bwd_k16<4, false>(sWt + A::wt_off(FFN_WD_OUT), A::pt(FFN_WD_OUT), dd_op, ssc, dd, g, s);
      relu_mask(dd, f.hd[ND - 1]);
      dsc = make_op4(dd, dop);
    }
    __syncthreads();
    layer_dw<1, 4, PS>(sS, gd_out, wave, g, s);
    __syncthreads();
    // hidden density layers (Wd_12, Wd_01)
#pragma unroll
    for (int i = ND - 1; i >= 1; --i) {
      const int k = i == 1 ? FFN_WD_01 : FFN_WD_12;
      stash_rows<4>(sS, 0, g, col, [&](int t, int r) { return dd[t][r]; });
      stash_act<4>(sS, 64, g, col, f.hd[i - 1]);
      bwd_k32<4, false>(sWt + A::wt_off(k), A::pt(k), dop, dsc, dd, g, s);
      relu_mask(dd, f.hd[i - 1]);
      dsc = make_op4(dd, dop);
      __syncthreads();
      layer_dw<4, 4, PS>(sS, gd_h[i - 1], wave, g, s);
      __syncthreads();
    }
    // density input layer: deltas and the encoding (bf16 of the fp32 values); dL/da0 = Wd_in^T . delta
    stash_rows<4>(sS, 0, g, col, [&](int t, int r) { return dd[t][r]; });
    stash_words<KB0>(sS, 64, g, col, [&](int t, int p) { return a0w[t][p]; });
    {
      floatx4 ga0[KB0];
      bwd_k32<KB0, false>(sWt + A::wt_off(FFN_WD_IN), A::pt(FFN_WD_IN), dop, dsc, ga0, g, s);
      if (valid) store_enc_grad<LF, FEAT>(a, b, g, ga0);
    }
    __syncthreads();
    layer_dw<4, KB0, PS>(sS, gd_in, wave, g, s);
    // no barrier: the stash is next written after the next tile's compositing barriers
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

template <int LF, int ND, int NC, int FEAT, bool TAPS, bool MARCHED, int SC, bool TRAIN>
static hipError_t launch16_k(const MlpArgs& a, int n_blocks, hipStream_t st) {
  using A = Arch16<LF, ND, NC>;
  const size_t lds = A::lds_bytes();
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)k_mlp16<LF, ND, NC, FEAT, TAPS, MARCHED, SC, TRAIN>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((k_mlp16<LF, ND, NC, FEAT, TAPS, MARCHED, SC, TRAIN>), dim3(n_blocks), dim3(256), lds, st, a);
  return hipGetLastError();
}

template <int LF, int ND, int NC, int FEAT, bool TAPS, bool MARCHED, int SC>
static hipError_t launch16_f(const MlpArgs& a, int n_blocks, hipStream_t st) {
  if constexpr (MARCHED) {
    return launch16_k<LF, ND, NC, FEAT, TAPS, true, SC, true>(a, n_blocks, st);
  } else {
    return a.do_train ? launch16_k<LF, ND, NC, FEAT, TAPS, false, SC, true>(a, n_blocks, st)
                      : launch16_k<LF, ND, NC, FEAT, TAPS, false, SC, false>(a, n_blocks, st);
  }
}

template <int LF, int ND, int NC, bool MARCHED, int SC>
static hipError_t launch16_t(const MlpArgs& a, int n_blocks, hipStream_t st) {
  const bool taps = taps_requested(a);
  switch (a.c.F) {
    case 1:
      return taps ? launch16_f<LF, ND, NC, 1, true, MARCHED, SC>(a, n_blocks, st)
                  : launch16_f<LF, ND, NC, 1, false, MARCHED, SC>(a, n_blocks, st);
    case 2:
      return taps ? launch16_f<LF, ND, NC, 2, true, MARCHED, SC>(a, n_blocks, st)
                  : launch16_f<LF, ND, NC, 2, false, MARCHED, SC>(a, n_blocks, st);
    case 4:
      return taps ? launch16_f<LF, ND, NC, 4, true, MARCHED, SC>(a, n_blocks, st)
                  : launch16_f<LF, ND, NC, 4, false, MARCHED, SC>(a, n_blocks, st);
    default: return hipErrorInvalidValue;
  }
}

// Forward only, for samples given by index (the marched training step's sigma and rgb, which its
// compositing kernel needs before the backward): the same fp16 forward as k_mlp16's, 16 samples per
// wavefront at a time; sample b belongs to ray ray_ids[b]
template <int LF, int ND, int NC, int FEAT>
__global__ __launch_bounds__(256) void k_mlp16_fwd(MlpPtrs wp, const float* __restrict__ a0, FeatLayout feat,
                                                   const float4* __restrict__ rays,
                                                   const uint32_t* __restrict__ ray_ids, int64_t n, float sh_mult,
                                                   float* __restrict__ sigma, float* __restrict__ rgb,
                                                   const uint32_t* __restrict__ n_dev) {
  using A = Arch16<LF, ND, NC>;
  if (n_dev) {  // the count of a launch sized for a capacity, read on the device
    const int64_t nd = (int64_t)*n_dev;
    n = nd < n ? nd : n;
  }
  if ((int64_t)blockIdx.x * 64 >= n) return;  // no samples for this block: skip staging the weights
  extern __shared__ __align__(16) unsigned char smem16f[];
  _Float16* sWf = reinterpret_cast<_Float16*>(smem16f);
  float* sB = reinterpret_cast<float*>(smem16f + (size_t)A::wf_off(FFN_N_LAYERS) * 2);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, s = lane & 15;
#pragma unroll
  for (int k = 0; k < FFN_N_LAYERS; ++k) {
    if (!layer_active(k, ND, NC)) continue;
    const int O = layer_out(k), I = layer_in(k, LF), R = A::rows_pad(k), PF = A::pf(k);
    const bool kf = I % 32 == 0;
    for (int e = tid; e < R * PF; e += 256) {
      const int r = e / PF, p = e - r * PF;
      const int i = p < I ? (kf ? kpos_neuron(p) : p) : I;
      sWf[A::wf_off(k) + e] = (_Float16)((r < O && i < I) ? wp.W[k][r * I + i] : 0.0f);
    }
    for (int e = tid; e < R; e += 256) sB[A::b_off(k) + e] = e < O ? wp.b[k][e] : 0.0f;
  }
  __syncthreads();
  for (int64_t grp = (int64_t)blockIdx.x * 4 + wave; grp * 16 < n; grp += (int64_t)gridDim.x * 4) {
    const int64_t b = grp * 16 + s;
    const bool valid = b < n;
    float a0v[LF / 4];
    load_a0<LF, FEAT>(a0, feat, b, valid, g, a0v);
    float dirv[3] = {0.0f, 0.0f, 1.0f};
    if (valid) {
      const float4 rd = rays[2 * (size_t)ray_ids[b] + 1];
      dirv[0] = rd.x;
      dirv[1] = rd.y;
      dirv[2] = rd.z;
    }
    floatx4 sh;
#pragma unroll
    for (int r = 0; r < 4; ++r) sh[r] = sh_component(dirv, 4 * g + r) * sh_mult;
    Fwd16<LF, ND, NC> f;
    forward16<LF, ND, NC, A, false>(sWf, sB, a0v, sh, g, s, f);
    if (g == 0 && valid) {
      sigma[b] = softplus(fminf(fmaxf(f.dout0, -10.0f), 10.0f));
      rgb[3 * b] = f.rgb[0];
      rgb[3 * b + 1] = f.rgb[1];
      rgb[3 * b + 2] = f.rgb[2];
    }
  }
}

template <int LF, int ND, int NC, int FEAT>
static hipError_t launch16_fwd_f(const MlpPtrs& w, const float* a0, const FeatLayout& feat, const float4* rays,
                                 const uint32_t* ray_ids, int64_t n, float sh_mult, float* sigma, float* rgb,
                                 int n_blocks, hipStream_t st, const uint32_t* n_dev) {
  using A = Arch16<LF, ND, NC>;
  const size_t lds = (size_t)A::wf_off(FFN_N_LAYERS) * 2 + (size_t)A::b_floats() * 4;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)k_mlp16_fwd<LF, ND, NC, FEAT>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((k_mlp16_fwd<LF, ND, NC, FEAT>), dim3(n_blocks), dim3(256), lds, st, w, a0, feat, rays,
                     ray_ids, n, sh_mult, sigma, rgb, n_dev);
  return hipGetLastError();
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
  if (LF == l && nd == d && nc == n)                                                     \
    return a.S == 64 ? launch16_t<l, d, n, false, 64>(a, n_blocks, st) : launch16_t<l, d, n, false, 0>(a, n_blocks, st);
  FFN_MLP16_CONFIGS(X)
#undef X
  return hipErrorInvalidValue;
}

hipError_t launch_mlp16_marched(const MlpArgs& a, int LF, int nd, int nc, int n_blocks, hipStream_t st) {
#define X(l, d, n) \
  if (LF == l && nd == d && nc == n) return launch16_t<l, d, n, true, 0>(a, n_blocks, st);
  FFN_MLP16_CONFIGS(X)
#undef X
  return hipErrorInvalidValue;
}

hipError_t launch_mlp16_fwd(const DevCfg& c, const MlpPtrs& w, const float* a0, const FeatLayout& feat,
                            const float4* rays, const uint32_t* ray_ids, int64_t n, float sh_mult, float* sigma,
                            float* rgb, int LF, int nd, int nc, int n_blocks, hipStream_t st, const uint32_t* n_dev) {
  if (n <= 0) return hipSuccess;
#define X(l, d, nn)                                                                                             \
  if (LF == l && nd == d && nc == nn) {                                                                         \
    switch (c.F) {                                                                                              \
      case 1: return launch16_fwd_f<l, d, nn, 1>(w, a0, feat, rays, ray_ids, n, sh_mult, sigma, rgb, n_blocks, st, n_dev); \
      case 2: return launch16_fwd_f<l, d, nn, 2>(w, a0, feat, rays, ray_ids, n, sh_mult, sigma, rgb, n_blocks, st, n_dev); \
      case 4: return launch16_fwd_f<l, d, nn, 4>(w, a0, feat, rays, ray_ids, n, sh_mult, sigma, rgb, n_blocks, st, n_dev); \
      default: return hipErrorInvalidValue;                                                                     \
    }                                                                                                           \
  }
  FFN_MLP16_CONFIGS(X)
#undef X
  return hipErrorInvalidValue;
}

}  // namespace ffn
