// ffn_kernels.h -- launchers of the gfx950 kernels (internal to the library).
#pragma once
#include "ffn_device.h"

namespace ffn {

// packed layout of the MLP parameters: per active layer slot, W [out][in] then b [out]
struct __attribute__((packed)) PackedLayout {
  int active[FFN_N_LAYERS];
  int out[FFN_N_LAYERS];
  int in[FFN_N_LAYERS];
  int w_off[FFN_N_LAYERS];
  int b_off[FFN_N_LAYERS];
  int total;
};

__host__ __device__ constexpr bool layer_active(int k, int nd, int nc) {
  return k == FFN_WD_IN || k == FFN_WD_OUT || k == FFN_WC_IN || k == FFN_WC_OUT || (k == FFN_WD_01 && nd >= 2) ||
         (k == FFN_WD_12 && nd >= 3) || (k == FFN_WC_01 && nc >= 2) || (k == FFN_WC_12 && nc >= 3) ||
         (k == FFN_WC_23 && nc >= 4);
}
__host__ __device__ constexpr int layer_out(int k) {
  return k == FFN_WD_OUT ? FFN_D_OUT : (k == FFN_WC_OUT ? FFN_C_OUT : FFN_M);
}
__host__ __device__ constexpr int layer_in(int k, int LF) {
  return k == FFN_WD_IN ? LF : (k == FFN_WC_IN ? FFN_C_IN : FFN_M);
}

inline PackedLayout make_layout(int LF, int nd, int nc) {
  PackedLayout p{};
  int o = 0;
  for (int k = 0; k < FFN_N_LAYERS; ++k) {
    p.active[k] = layer_active(k, nd, nc) ? 1 : 0;
    p.out[k] = layer_out(k);
    p.in[k] = layer_in(k, LF);
    if (!p.active[k]) {
      p.w_off[k] = p.b_off[k] = -1;
      continue;
    }
    p.w_off[k] = o;
    o += p.out[k] * p.in[k];
    p.b_off[k] = o;
    o += p.out[k];
  }
  p.total = o;
  return p;
}

// where sample positions come from: x[n][x_stride] (first three floats), or o + Ts[b] d of ray b >> log2S
struct PosSrc {
  const float* x;
  const float4* rays;
  const float* Ts;
  int log2S;
  int x_stride = 3;
};

// element (sample b, level l, feature f) of an encoding-shaped array is at
// l * stride_l + b * stride_b + f: sample-major [N][L*F] or level-major [L][N][F]
struct FeatLayout {
  int64_t stride_l, stride_b;
};
inline FeatLayout sample_major(int L, int F) { return FeatLayout{F, (int64_t)L * F}; }
inline FeatLayout level_major(int64_t n, int F) { return FeatLayout{n * F, F}; }

struct MlpPtrs {
  const float* W[FFN_N_LAYERS];
  const float* b[FFN_N_LAYERS];
};

constexpr int RELU_WORDS = 14;  // ReLU-branch tap words per sample: two per hidden layer slot (3 density, 4 colour)

struct MlpArgs {
  DevCfg c;
  MlpPtrs w;
  const float4* rays;
  const float4* targets;
  float4* out_rgb;
  const float* Ts;
  const float* DTs;
  const uint32_t* flags;
  const float* a0;
  float* dL_da0;
  FeatLayout feat;  // layout of a0 and dL_da0
  float* partials;  // [gridDim.x][layout.total]
  const uint32_t* occ_in;
  uint32_t* occ_st;
  uint32_t num_rays;
  int S, log2S;
  int64_t n_tiles;
  // k_mlp, k_mlp16: position i of the launch's tile sequence is tile tile_order[i] (launch_tile_order: the
  // busy tiles first, so that the round-robin deal gives every block the same share of them), or tile i when
  // NULL
  const uint32_t* tile_order;
  // with tile_order: the number of busy tiles (a sample with dt > 0), which the order puts first; the
  // kernels composite the later positions' tiles to the background without the MLP (NULL: every tile takes
  // the full path)
  const uint32_t* n_busy;
  float sh_mult, occ_strength;
  uint32_t seed;
  int do_train;
  // taps
  float* t_sigma;
  float* t_rgb;
  float* t_Tr;
  float* t_Tfinal;
  uint32_t* t_relu;  // [N][RELU_WORDS]
  float4* t_color;   // [num_rays] colour before clamping
  float* t_dLds;
  float* t_dLdc;
  // marched training (the backward over compacted samples): sample b is smp[b] = {x, y, z, t} of ray
  // ray_ids[b], lattice step march_dt; its loss gradients come from the compositing kernel
  const float4* smp;
  const uint32_t* ray_ids;
  const float* in_dLds;
  const float* in_dLdc;
  float march_dt;
  // when set, the sample count is min(*n_dev, num_rays << log2S) read on the device (num_rays << log2S the
  // capacity the buffers hold) and the kernel walks its tiles; n_tiles is then the capacity's
  const uint32_t* n_dev;
};

// bucketed backward scatter
enum { BIN_GRAD = 0, BIN_SGD = 1, BIN_ADAM = 2 };

struct BinGroup {
  int level0, n_levels, log2_be, chunk, nblk;
  int n_rounds;     // emit rounds per level (the samples in runs of the emit round size)
  int np;           // pair slots of one round (the stage size; a multiple of 8)
  int meta_stride;  // entries per round in the run table (the group's largest bucket count)
  int nbl[FFN_MAX_LEVELS];             // buckets of each level of the group
  int bucket_rel[FFN_MAX_LEVELS + 1];  // first bucket of each level, relative to the group
};

struct BinPlan {
  int log2_be, chunk, nblk, levels_per_group, max_buckets, max_nbl, n_rounds, np;
  int64_t max_pairs, meta_elems;
};

struct BinScratch {
  uint32_t* meta;      // [levels_per_group][n_rounds][max_nbl] each bucket's run in a round's slots: offset << 16 | length
  uint32_t* meta_t;    // the same, bucket-major: [levels_per_group][max_nbl][n_rounds]
  float* cmax;         // [levels_per_group][chunks] bound on every |value| of the chunk's pairs
  uint4* pairs;        // [max_pairs / 8] blocks of 8 pairs: 8 * F fp32 values, then 8 u16 entries (in bucket)
};

struct BinApply {
  void* dst;   // grad (BIN_GRAD), table (BIN_SGD, BIN_ADAM): float, or binary16 when dst_f16
  int dst_f16;
  float* m;
  float* v;
  float* g_tap;  // optional: the summed table gradient (BIN_ADAM)
  float lr_t, beta1, beta2, eps;
};

BinPlan plan_bins(const DevCfg& c, int64_t n, size_t pair_budget_bytes);
// whether the scatter is built for this table shape: a round's stage must fit in a CU's LDS and its run
// offsets in 16 bits (F = 4 with 2^22-entry levels does not)
bool scatter_supported(const DevCfg& c);

// tile_busy (may be NULL): word t = 1 when one of samples 64t .. 64t + 63 has dt > 0 (the MLP's busy tiles)
hipError_t launch_sample(const DevCfg& c, const float4* rays, uint32_t num_rays, int S, uint32_t seed,
                         const uint32_t* occ_in, int do_train, float* Ts, float* DTs, uint32_t* flags,
                         hipStream_t st, uint32_t* tile_busy = nullptr);

// table: float, or binary16 when c.table_f16 (widened exactly; the sums are the same fp32 operations)
// Dense copies of the coarse levels' vertex values (the table's element type, F per vertex) from
// grid + off[l] F: row-major, vertex (x, y, z) at (z R + y) R + x, or, for a level whose bit is set in
// `bricked`, in 4x4x4 bricks: ((z/4 NB + y/4) NB + x/4) 64 + (z%4) 16 + (y%4) 4 + x%4 (NB = ceil(R/4));
// off[l] = DENSE_NONE for a level read through its hash
constexpr uint32_t DENSE_NONE = 0xFFFFFFFFu;
struct DenseLevels {
  void* grid;
  uint32_t off[FFN_MAX_LEVELS];
  int n_multi;       // levels 0 .. n_multi - 1 (all with row-major copies) are gathered together in one pass
  uint32_t bricked;  // bit l: level l's copy is bricked
};
// fill the dense copies from the table (every level with off[l] != DENSE_NONE)
hipError_t launch_hash_densify(const DevCfg& c, const void* table, const DenseLevels& dl, hipStream_t st);
// dl (may be NULL): levels with a dense copy gather from it, with the same values and arithmetic.
// n_dev (may be NULL): the sample count is min(n, *n_dev), read on the device (n the capacity); the grid is
// then sized for at most HASH_FWD_DEV_BLOCKS blocks per level, each walking its samples with a grid stride
constexpr int64_t HASH_FWD_DEV_BLOCKS = 4096;
hipError_t launch_hash_fwd(const DevCfg& c, const PosSrc& src, int64_t n, const void* table, float* a0,
                           const FeatLayout& lay, uint32_t* idx_out, const DenseLevels* dl, hipStream_t st,
                           const uint32_t* n_dev = nullptr);
// BIN_GRAD: dst += scatter(g); BIN_SGD: table += scatter(-lr 2^(-0.1 l) 0.5 g) (reference SGD);
// BIN_ADAM: Adam on the table with the scattered gradient.  n_dev (may be NULL): the sample count is
// min(n, *n_dev), read on the device (the plan made for n, the capacity)
hipError_t launch_hash_bwd(const DevCfg& c, const PosSrc& src, int64_t n, const float* g, const FeatLayout& lay,
                           int mode, float lr, const BinApply& ap, const BinPlan& plan, const BinScratch& s,
                           hipStream_t st, const uint32_t* n_dev = nullptr);
hipError_t launch_feat_relayout(const float* src, const FeatLayout& ls, float* dst, const FeatLayout& ld, int64_t n,
                                int L, int F, hipStream_t st);

hipError_t launch_adam(float* p, float* m, float* v, float* g, int64_t n, float lr_t, float b1, float b2, float eps,
                       int zero_grad, hipStream_t st);
hipError_t launch_fill(float* p, int64_t n, float v, hipStream_t st);
hipError_t launch_occ_decay(uint32_t* occ_in, uint32_t* occ_st, uint32_t n_words, uint32_t decay_q24,
                            uint32_t seed, hipStream_t st);

// occupancy bitfield and DDA marcher (no counterpart in the reference; see ffn_march.hip)
struct MarchState {
  uint32_t k;      // next lattice index
  uint32_t cell;   // current cell, 10 bits per axis
  uint32_t n;      // samples emitted so far
  uint32_t flags;  // MARCH_FRESH, MARCH_DONE
};
enum { MARCH_FRESH = 1u, MARCH_DONE = 2u };

struct MarchArgs {
  float bmin[3], bmax[3], t_near, t_far;
  const float4* rays;
  uint32_t num_rays;
  const uint32_t* bits;
  int res;
  float dt;
  uint32_t max_steps;        // per ray in total
  uint32_t chunk;            // per call
  MarchState* state;         // NULL: every ray starts fresh and no state is kept
  uint32_t* counts;          // count pass: samples this call per ray
  const uint32_t* offsets;   // emit pass: first slot of each ray
  float4* samples;           // emit pass: {x, y, z, t}
  uint32_t* ray_ids;         // emit pass
  uint64_t capacity;         // slots of samples / ray_ids
  uint32_t slot_stride;      // emit pass into per-ray slots: ray r's samples at r * slot_stride (and its count
                             // written as the count pass does); 0: at offsets[r]
  const uint32_t* blocks;     // summary of `bits` per 8^3 block (launch_occ_blocks), or NULL: no block skipping
  const uint32_t* blocks_use;  // with it: the walk skips blocks when *blocks_use != 0
  // (may be NULL) the launch does nothing when *gate == 0: a render round after one without samples (every ray
  // has stopped, every count is already 0)
  const uint32_t* gate;
};

hipError_t launch_occ_bitfield(const uint32_t* occ, int G, uint32_t q_min, uint32_t* bits, hipStream_t st);
// one bit per 8^3 block of cells (x fastest, ceil(R / 8) blocks per axis), set when any cell of the block is
// occupied; *use = 1 when at least half the blocks are empty, else 0
hipError_t launch_occ_blocks(const uint32_t* bits, int R, uint32_t* blocks, uint32_t* use, hipStream_t st);
hipError_t launch_march(const MarchArgs& a, bool emit, hipStream_t st);
// per-ray slots (ray r's counts[r] samples at slots + r * stride) -> the compacted order (offsets), with ray ids
// (gate: as MarchArgs::gate)
hipError_t launch_march_compact(const uint32_t* counts, const uint32_t* offsets, const float4* slots,
                                uint32_t stride, uint32_t num_rays, float4* samples, uint32_t* ray_ids,
                                hipStream_t st, const uint32_t* gate = nullptr);
// sample budget of a step: the rays whose samples all lie below slot cap of the scanned order keep their
// counts, the others (a suffix of the rays) get count 0; *n_eff = the samples kept.  offsets [num_rays + 1]
// from launch_scan_u32 (offsets[num_rays] = the total)
hipError_t launch_march_clamp(uint32_t* counts, const uint32_t* offsets, uint32_t num_rays, uint32_t cap,
                              uint32_t* n_eff, hipStream_t st);
// (prime, may be NULL: set to 1, the open gate of a render's first round)
hipError_t launch_march_init(MarchState* state, float4* acc, uint32_t* n_used, uint32_t num_rays, hipStream_t st,
                             uint32_t* prime = nullptr);
hipError_t launch_render_composite(const uint32_t* offsets, const uint32_t* counts, uint32_t num_rays,
                                   const float* sigma, const float* rgb, float dt, float T_stop, MarchState* state,
                                   float4* acc, uint32_t* n_used, hipStream_t st, const uint32_t* gate = nullptr);
hipError_t launch_render_finish(const float4* acc, uint32_t num_rays, float4* out_rgb, hipStream_t st);
// exclusive scan of in[0..n) into out[0..n]; out[n] and *total get the sum.  gated: the kernels do nothing
// while *total == 0 on entry (a render round after one without samples: in is all zero and out already holds
// its scan)
hipError_t launch_scan_u32(const uint32_t* in, int64_t n, uint32_t* out, uint32_t* sums, uint32_t* total,
                           hipStream_t st, bool gated = false);

// compositing of a marched training batch (one lane per ray, front to back, stopping after the sample that
// leaves T < T_stop), the photometric loss gradient and the compositing backward of every sample
struct CompMarchArgs {
  const uint32_t* offsets;
  const uint32_t* counts;
  uint32_t num_rays;
  const float* sigma;
  const float* rgb;
  const float4* targets;
  float dt, T_stop, regu;  // regu = 5e-3 dt / max_steps, the density penalty of every composited sample
  int background;          // FFN_BG_*
  uint32_t seed;
  float4* out_rgb;         // {clamped rgb, 4}
  float* Tr;               // [n] transmittance before each sample
  float* dLds;             // [n]
  float* dLdc;             // [n][3]
  uint32_t* n_used;        // [num_rays] samples composited (optional)
  float* T_final;          // [num_rays] (optional)
  float4* color;           // [num_rays] colour before clamping (optional)
  // occupancy proposals of the marched runs, made when occ_st is set: the grid (c), the rays, the marched
  // samples (t in .w) and both occupancy grids
  DevCfg c;
  const float4* rays;
  const float4* samples;
  const uint32_t* occ_in;
  uint32_t* occ_st;
};
hipError_t launch_composite_marched(const CompMarchArgs& a, hipStream_t st);

// training batch on the GPU: uniform pixels of the resident images, their rays and targets
hipError_t launch_make_batch(const float* images, uint32_t n_images, uint32_t W, uint32_t H, const float* c2w,
                             const float* K, uint32_t num_rays, uint32_t seed, float4* rays, float4* targets,
                             uint32_t* pixel_ids, hipStream_t st);
hipError_t launch_make_batch_weighted(const float* images, uint32_t n_images, uint32_t W, uint32_t H,
                                      const float* c2w, const float* K, const uint8_t* weights, uint32_t num_rays,
                                      uint32_t uniform_rays, uint32_t max_tries, uint32_t seed, float4* rays,
                                      float4* targets, uint32_t* pixel_ids, hipStream_t st);

// forward-only MLP over n samples: encodings a0 (layout feat), view directions from rays[ray_ids[b]];
// sigma[n], rgb[n][3]
// (n_dev may be NULL: the count is then n; else min(n, *n_dev), read on the device)
hipError_t launch_mlp_fwd(const DevCfg& c, const MlpPtrs& w, const float* a0, const FeatLayout& feat,
                          const float4* rays, const uint32_t* ray_ids, int64_t n, float sh_mult, float* sigma,
                          float* rgb, int LF, int nd, int nc, int n_blocks, hipStream_t st,
                          const uint32_t* n_dev = nullptr);

// fused MLP forward + compositing + loss + backward + proposals, per 64-sample tile
bool mlp_supported(int LF, int nd, int nc);
int mlp_blocks_per_cu(int LF, int nd, int nc);  // blocks of launch_mlp that fit on one CU
int mlp16_blocks_per_cu(int LF, int nd, int nc);  // blocks of launch_mlp16 that fit on one CU
hipError_t launch_mlp(const MlpArgs& a, int LF, int nd, int nc, int n_blocks, hipStream_t st);
// order[n_tiles]: the tiles with a sample of dt > 0 in index order, then the others; scratch: flags and off
// n_tiles + 1 words each, sums (n_tiles + 4096) / 4096 + 1 words, total 1 word
// flags: the tiles' busy flags (launch_sample's tile_busy)
hipError_t launch_tile_order(int64_t n_tiles, const uint32_t* flags, uint32_t* off, uint32_t* sums, uint32_t* total,
                             uint32_t* order, hipStream_t st);
// the same kernel's backward over marched samples (a.smp, a.ray_ids, a.in_dLds, a.in_dLdc; a.num_rays = the
// sample count, log2S = 0): no compositing, no proposals
hipError_t launch_mlp_marched(const MlpArgs& a, int LF, int nd, int nc, int n_blocks, hipStream_t st);
// the same step on fp16 (forward) / bf16 (backward, weight gradients) MFMAs with fp32 accumulation
bool mlp16_supported(int LF, int nd, int nc);
hipError_t launch_mlp16(const MlpArgs& a, int LF, int nd, int nc, int n_blocks, hipStream_t st);
// the fp16 path of the marched training step: forward only over indexed samples, and the backward
hipError_t launch_mlp16_fwd(const DevCfg& c, const MlpPtrs& w, const float* a0, const FeatLayout& feat,
                            const float4* rays, const uint32_t* ray_ids, int64_t n, float sh_mult, float* sigma,
                            float* rgb, int LF, int nd, int nc, int n_blocks, hipStream_t st,
                            const uint32_t* n_dev = nullptr);
hipError_t launch_mlp16_marched(const MlpArgs& a, int LF, int nd, int nc, int n_blocks, hipStream_t st);

// sum the per-block gradient partials and apply Adam to the MLP parameters
struct MlpOptArgs {
  PackedLayout lay;
  float* W[FFN_N_LAYERS];
  float* b[FFN_N_LAYERS];
  float* mW[FFN_N_LAYERS];
  float* vW[FFN_N_LAYERS];
  float* mb[FFN_N_LAYERS];
  float* vb[FFN_N_LAYERS];
  float* gW[FFN_N_LAYERS];  // optional taps
  float* gb[FFN_N_LAYERS];
  const float* partials;
  int n_partials;
  float lr_t, color_rel_lr, beta1, beta2, eps;
};
hipError_t launch_mlp_adam(const MlpOptArgs& a, hipStream_t st);

}  // namespace ffn
