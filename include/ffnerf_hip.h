/*
 * ffnerf_hip.h -- C ABI of libffnerf_hip.so, the MI355X (gfx950) implementation
 * of the ffnerf fused NeRF training step.
 *
 * Plain C: no C++ or torch types cross this boundary.  Every buffer argument is
 * a caller-owned device pointer (hipMalloc / torch-ROCm storage); sizes are
 * passed explicitly; every call enqueues on the caller's hipStream_t (passed as
 * void*, NULL = default stream) and returns immediately.  Return value: 0 on
 * success, < 0 on failure with a message in ffn_last_error() (thread-local).
 * Unlike the reference kernels, nothing fails silently: a bad shape or an
 * unsupported configuration is an error.
 *
 * What each entry point replaces in the reference (/root/reference):
 *   ffn_create / ffn_bind_params   Nerf.from_kernels + Nerf.setup_buffers
 *                                  (ffnerf_tools.py:583-671, 926-977): program
 *                                  build options become a config struct,
 *                                  parameter buffers are bound, scratch sized.
 *   ffn_train_step                 the kernel pair enqueued by Nerf.step
 *                                  (ffnerf_tools.py:1439-1445 and 1479-1519):
 *                                  ffnerf_train_step (ffnerf_OG.cl:838-922) +
 *                                  update_ffnerf_oneWG (weight_update.cl:346-454),
 *                                  fused, without the SoA staging buffers.
 *   ffn_occ_decay                  occ_nibble_decay_write_both_q24
 *                                  (decay_occ_grid_in-st.cl:13-19), same
 *                                  arguments; launched by Nerf.step at
 *                                  ffnerf_tools.py:1452-1476.
 *   ffn_sample / ffn_hash_encode_fwd / ffn_hash_encode_bwd / ffn_adam
 *                                  stage entry points of the same path
 *                                  (ffnerf_OG.cl:1002-1250, 1286-1364,
 *                                  2090-2173; weight_update.cl:177-201) for
 *                                  parity tests and micro-benchmarks.
 */
#ifndef FFNERF_HIP_H
#define FFNERF_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2: ffn_taps gained T_final, relu and color; ffn_params.table became void* (binary16 tables).
 * 3: ffn_march_params' reserved words became sample_capacity and flags (zero keeps the version-2
 *    behaviour). */
#define FFN_ABI_VERSION 3
#define FFN_MAX_LEVELS 32

/* layer slots (reference kernel-argument order, ffnerf_tools.py:1210-1232) */
enum {
  FFN_WD_IN = 0, FFN_WD_01, FFN_WD_12, FFN_WD_OUT,
  FFN_WC_IN, FFN_WC_01, FFN_WC_12, FFN_WC_23, FFN_WC_OUT,
  FFN_N_LAYERS
};

enum { FFN_BG_BLACK = 0, FFN_BG_WHITE = 1, FFN_BG_RANDOM = 2 };     /* -DBACKGROUND_COLOR */
enum { FFN_HASH_SGD = 0, FFN_HASH_ADAM = 1 };                       /* table optimizer */
enum { FFN_MLP_FP32 = 0, FFN_MLP_FP16 = 1 };                        /* MLP arithmetic */
enum { FFN_TABLE_FP32 = 0, FFN_TABLE_FP16 = 1 };                    /* hash-table storage */
enum { FFN_SAMPLER_RESAMPLE = 0, FFN_SAMPLER_MARCH = 1 };           /* ffn_train_step's samples */

/* Build-time constants of the reference (ffnerf_OG.cl:16-81,161-200;
 * ffnerf_tools.py:23-69; run_ffnerf_OG.py:1044-1057) as runtime values. */
typedef struct ffn_config {
  int32_t n_levels;                     /* L   (reference: 16) */
  int32_t f_per_level;                  /* F   (reference: 4) */
  uint32_t log2_T[FFN_MAX_LEVELS];      /* per-level table size (reference LEVEL_LOG2) */
  int32_t res[FFN_MAX_LEVELS];          /* per-level resolution R_l, >= 2 */
  float lvl_lr_scale[FFN_MAX_LEVELS];   /* 2^(-0.1 l): per-level SGD scale */
  int32_t nd, nc;                       /* hidden layers: density 1..3, color 1..4 */
  int32_t occ_G;                        /* occupancy words per axis (8 nibbles each) */
  float box_min[3], box_max[3];
  float rho_min, rho_max, dt_min, dt_max, t_near, t_far;
  int32_t background;                   /* FFN_BG_* (training only; render is black) */
  int32_t hash_opt;                     /* FFN_HASH_* */
  int32_t mlp_precision;                /* FFN_MLP_* */
  int32_t table_dtype;                  /* FFN_TABLE_*: the table's storage (its Adam state stays fp32) */
  /* FFN_SAMPLER_MARCH: ffn_train_step samples by the bitfield march instead of the reference's
     importance resampler (no counterpart in the reference; see ffn_train_step) */
  int32_t sampler;                      /* FFN_SAMPLER_* */
  int32_t march_max_steps;              /* samples per ray at most (1..4096) */
  float march_dt;                       /* lattice step (> 0) */
  float march_T_stop;                   /* compositing stops after the sample that leaves T < T_stop, [0, 1) */
  int32_t march_q_min;                  /* bitfield predicate: occupancy level q = nibble + 1 >= q_min (1..17) */
  int32_t reserved[2];
} ffn_config;

/* Caller-owned device buffers of one model.  Weights are row-major
 * [out][in] float32 (the reference stores the same floats as int32 bit
 * patterns).  Inactive layers (depending on nd/nc) may be NULL. */
typedef struct ffn_params {
  float* W[FFN_N_LAYERS];
  float* b[FFN_N_LAYERS];
  float* mW[FFN_N_LAYERS];
  float* vW[FFN_N_LAYERS];
  float* mb[FFN_N_LAYERS];
  float* vb[FFN_N_LAYERS];
  void* table;                          /* [sum_l 2^log2_T[l]][F]: float32, or IEEE binary16 when
                                           table_dtype is FFN_TABLE_FP16 (updates round to nearest even) */
  float* m_table;                       /* Adam state, required for FFN_HASH_ADAM */
  float* v_table;
  uint32_t* occ_in;                     /* [G^3] 8 nibbles per word */
  uint32_t* occ_st;                     /* [G^3] proposals (training) */
} ffn_params;

/* Per-step scalars (ffnerf_tools.py:1197-1275, 1479-1482). */
typedef struct ffn_step_scalars {
  float lr;             /* lr_f; the table SGD uses lr * lvl_lr_scale[l] * 0.5 */
  float lr_t;           /* bias-corrected Adam step */
  float color_rel_lr;   /* color-MLP multiplier of lr_t */
  float sh_multiplier;
  float occ_strength;   /* proposals only if > 0 and training */
  float beta1, beta2, eps;
  uint32_t rng_seed;
  int32_t do_train;     /* 0: forward-only render (inference occupancy, black bg) */
} ffn_step_scalars;

/* Optional device taps of intermediate values (any pointer may be NULL).
 * N = num_rays * samples_per_ray; LF = n_levels * f_per_level. */
typedef struct ffn_taps {
  float* Ts;            /* [N] sample t */
  float* DTs;           /* [N] sample dt */
  uint32_t* flags;      /* [num_rays][2] run-start bits */
  float* a0;            /* [N][LF] encoding */
  float* sigma;         /* [N] */
  float* rgb;           /* [N][3] */
  float* Tr;            /* [N] transmittance before each sample */
  float* dL_dsigma;     /* [N] */
  float* dL_dc;         /* [N][3] */
  float* dL_da0;        /* [N][LF] */
  float* gW[FFN_N_LAYERS];  /* summed weight gradients (before Adam) */
  float* gb[FFN_N_LAYERS];
  float* g_table;       /* table gradient (FFN_HASH_ADAM), before Adam */
  float* T_final;       /* [num_rays] transmittance after each ray's last sample */
  uint32_t* relu;       /* [N][14] ReLU branches: words 2h, 2h+1 hold bit n set when hidden unit n of hidden
                           layer h (h = 0..2 density, 3..6 colour) has a positive activation */
  float* color;         /* [num_rays][4] composited colour before clamping, background included (the
                           photometric loss's input), 0 */
} ffn_taps;

int ffn_version(void);
const char* ffn_last_error(void);

int ffn_create(const ffn_config* cfg, void** handle);
/* Waits for the work the handle's calls enqueued (on every stream they were
 * given), then frees the handle and its scratch.  Calls captured into a HIP
 * graph run when the caller launches the graph: the caller finishes those
 * launches before ffn_destroy. */
int ffn_destroy(void* handle);
int ffn_bind_params(void* handle, const ffn_params* params);

/* One training step (do_train=1) or forward-only render (do_train=0).
 * rays: [num_rays] {float4 o (w=1), float4 d (w=0)} (ffnerf_tools.py:170-172);
 * targets, out_rgb: [num_rays] float4.  samples_per_ray: power of two <= 64.
 * With config sampler = FFN_SAMPLER_MARCH the step takes its samples from the
 * bitfield march instead (samples_per_ray is then ignored): the bitfield of
 * the (2 occ_G)^3 subcells with q >= march_q_min is built from occ_in, and
 * the step is ffn_train_step_marched with march_dt, march_max_steps and
 * march_T_stop (taps index the march's samples; the proposals of the marched
 * runs when occ_strength > 0, so that with the caller's decay the grid, and
 * the next step's bitfield, follow the density); a forward-only call is
 * ffn_render (out_rgb.w = T_final). */
int ffn_train_step(void* handle, const void* rays, const void* targets, void* out_rgb, uint32_t num_rays,
                   uint32_t samples_per_ray, const ffn_step_scalars* scalars, const ffn_taps* taps,
                   void* stream);

/* Occupancy decay/merge: same arguments as the reference kernel. */
int ffn_occ_decay(uint32_t* occ_grid_in, uint32_t* occ_grid_st, uint32_t n_words, uint32_t decay_q24,
                  uint32_t iter_seed, void* stream);

/* Sampler only: Ts/DTs [num_rays*spr], flags [num_rays][2]. */
int ffn_sample(void* handle, const void* rays, uint32_t num_rays, uint32_t samples_per_ray, uint32_t rng_seed,
               int32_t do_train, float* Ts, float* DTs, uint32_t* flags, void* stream);

/* Hash-grid encoding of n points x [n][3] (world space) with the bound table:
 * a0 [n][LF].  idx_out (optional) [n][L][8]: feature base index per corner.
 * Stages the encodings level-major in the handle's scratch (n * LF floats), so
 * calls on one handle must not overlap. */
int ffn_hash_encode_fwd(void* handle, const float* x, int64_t n, float* a0, uint32_t* idx_out, void* stream);

/* Scatter-add of the encoding gradient g [n][LF] of points x into grad
 * (table-shaped, caller-zeroed; of the table's storage type: with
 * FFN_TABLE_FP16 each entry takes its exactly summed gradient in one
 * round-to-nearest-even addition).  Non-finite gradients are skipped.  Stages g
 * level-major in the handle's scratch (n * LF floats), so calls on one handle
 * must not overlap. */
int ffn_hash_encode_bwd(void* handle, const float* x, const float* g, int64_t n, void* grad, void* stream);

/* Adam over n parameters (weight_update.cl:177-201 form).  If zero_grad,
 * g is cleared after it is read. */
int ffn_adam(float* p, float* m, float* v, float* g, int64_t n, float lr_t, float beta1, float beta2, float eps,
             int32_t zero_grad, void* stream);

/* ---- occupancy bitfield, DDA marcher, early-terminated render ----------
 * No counterpart in the reference, which samples every ray with S importance-
 * resampled points (ffnerf_OG.cl:1002-1250); its nearest analogues are the
 * occupancy nibble read (ffnerf_OG.cl:477-483) and the compositing recurrence
 * (ffnerf_OG.cl:1505-1591).  The CPU definitions ora_occ_bitfield,
 * ora_march_ray and ora_render_ray (oracle/) are the specification. */

/* Bitfield of (2G)^3 cells from the nibble grid occ [G^3]: bit = (q >= q_min)
 * with q = nibble + 1 of the cell's subcell; bit index x + R (y + R z),
 * R = 2G, 32 cells per word: bits holds ceil(R^3 / 32) words. */
int ffn_occ_bitfield(const uint32_t* occ, int32_t occ_G, uint32_t q_min, uint32_t* bits, void* stream);

typedef struct ffn_march_params {
  int32_t res;            /* cells per axis of the bitfield (<= 1024) */
  float dt;               /* lattice step: samples at t0 + (k + 1/2) dt, t0 the box entry */
  uint32_t max_steps;     /* samples per ray at most */
  float T_stop;           /* render: a ray stops after the sample that leaves T < T_stop */
  uint32_t chunk;         /* render: samples marched per ray per round */
  float sh_multiplier;    /* render: SH scale of the colour-net input */
  uint32_t sample_capacity; /* marched step: 0, or the most samples a step takes (no host wait, see below);
                             ffn_march and ffn_render refuse a nonzero value */
  uint32_t flags;         /* render: FFN_RENDER_NO_WAIT or 0 (the other entry points ignore that bit);
                             other bits are refused */
} ffn_march_params;

/* ffn_render enqueues all ceil(max_steps / chunk) rounds and never waits on
 * the stream: every launch is sized from device-side counts (rounds after the
 * last ray retires are empty launches). */
#define FFN_RENDER_NO_WAIT 1u

/* March every ray through the bitfield (box and t_near/t_far of the handle's
 * config) and compact the samples: counts/offsets [num_rays]; samples
 * [capacity] float4 {x, y, z, t}; ray_ids [capacity]; *total (device) = sum
 * of counts.  Slots at or beyond capacity are not written: compare *total
 * with capacity. */
int ffn_march(void* handle, const void* rays, uint32_t num_rays, const uint32_t* bits, const ffn_march_params* mp,
              uint32_t* counts, uint32_t* offsets, float* samples, uint32_t* ray_ids, uint64_t capacity,
              uint32_t* total, void* stream);

/* ffn_march without any allocation.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as ffn_march; the scan's offsets and partial sums live
 * in a fixed device array of the library (4 MiB, held on every GPU the
 * library runs on until the process ends), so num_rays may not exceed
 * FFN_MARCH_NOALLOC_MAX_RAYS (an error otherwise), and calls that overlap on
 * one GPU (other streams, other threads) race on that array. */
#define FFN_MARCH_NOALLOC_MAX_RAYS (1u << 20)
int ffn_march_noalloc(void* handle, const void* rays, uint32_t num_rays, const uint32_t* bits,
                      const ffn_march_params* mp, uint32_t* counts, uint32_t* offsets, float* samples,
                      uint32_t* ray_ids, uint64_t capacity, uint32_t* total, void* stream);

/* A training step over marched samples (the DDA march replaces the reference's
 * S importance-resampled samples per ray, ffnerf_OG.cl:1002-1250): march every
 * ray through the bitfield (as ffn_march: lattice samples of occupied cells,
 * at most mp->max_steps), encode, run the MLPs, composite front to back
 * stopping after the sample that leaves T < mp->T_stop (the later samples
 * contribute nothing and get no gradient), the photometric loss and its
 * gradient (ffnerf_OG.cl:1505-1634, as a sequential recurrence), the MLP
 * backward, the table update (reference SGD or Adam) and the MLP Adam.  The
 * density penalty of a composited sample is 5e-3 dt / max_steps (the
 * reference's 5e-3 dt / S).  The bitfield is an input (ffn_occ_bitfield).
 * When scalars->occ_strength > 0 the step makes the occupancy proposals of
 * its samples into occ_st: each ray's marched samples fall into runs of one
 * occupancy subcell, and every run proposes as a run of the resampled step
 * does (ffnerf_OG.cl:1640-1821), from the compositing's transmittances.
 * Specification: ora_train_step_marched (oracle/).
 * rays, targets, out_rgb as ffn_train_step (out_rgb.w = 4); n_samples
 * (optional) [num_rays] = samples composited per ray.  taps (optional) index
 * the step's samples in march order (ray by ray, front to back; at most
 * num_rays * max_steps): sigma, rgb, Tr, dL_dsigma, dL_dc, a0, dL_da0, relu,
 * the per-ray T_final and color, and the summed gradients.  A step whose
 * march finds no samples returns the background, leaves the table and its
 * moments as they are and runs the MLP's Adam on zero gradients.  Both MLP
 * paths (mlp_precision fp32 or fp16).
 * With mp->sample_capacity = 0 the step waits on the stream once, after the
 * march's count, to size its buffers and launches.  With sample_capacity = C
 * > 0 it never waits (it can be captured in a graph): buffers are sized for C
 * samples and every launch reads the count on the device.  The rays whose
 * samples all fit into the first C slots of the march order are trained;
 * the later rays (the first whose samples would pass slot C and every one
 * after it) are dropped: they get no samples, n_samples 0 and the background
 * colour, and no gradient.  With C >= the march's total the step is
 * bit-identical to the waiting one.  taps need sample_capacity = 0; C may not
 * exceed num_rays * max_steps. */
int ffn_train_step_marched(void* handle, const void* rays, const void* targets, void* out_rgb, uint32_t num_rays,
                           const uint32_t* bits, const ffn_march_params* mp, const ffn_step_scalars* scalars,
                           const ffn_taps* taps, uint32_t* n_samples, void* stream);

/* Forward render with the bound parameters: march `chunk` samples per live
 * ray, encode, run the MLPs, composite front to back, retire rays below
 * T_stop, repeat.  out_rgb [num_rays] float4 {r, g, b, T_final} (black
 * background); n_samples [num_rays] (optional) = samples composited.  Waits
 * on the stream once per round to size the round's launches, and stops after
 * the first round without samples; with mp->flags & FFN_RENDER_NO_WAIT it does
 * not wait (same results). */
int ffn_render(void* handle, const void* rays, uint32_t num_rays, const uint32_t* bits, const ffn_march_params* mp,
               void* out_rgb, uint32_t* n_samples, void* stream);

/* A training batch made on the GPU (replaces the host producer and ray builder,
 * run_ffnerf_OG.py:585-686 and ffnerf_tools.py:175-234): ray r is pixel
 * floor(h P / 2^32) of the P = n W H pixels of the resident images, with
 * h = lowbias32(seed ^ r * 2654435769).  images [n][H][W][3] float32 RGB,
 * c2w [n][4][4] row-major, K [3][3] shared intrinsics (OpenCV axes).
 * rays [num_rays] {o, 1, d, 0}; targets [num_rays] {rgb, 0}; pixel_ids
 * (optional) [num_rays] the drawn pixel index. */
int ffn_make_batch(const float* images, uint32_t n_images, uint32_t width, uint32_t height, const float* c2w,
                   const float* K, uint32_t num_rays, uint32_t seed, void* rays, void* targets, uint32_t* pixel_ids,
                   void* stream);

/* An error-weighted training batch (replaces the reference's producer with its
 * per-image uint8 weight maps and rejection sampler, run_ffnerf_OG.py:490-516,
 * 585-686): weights [n][H][W] uint8 (the caller's maps, updated from the loss).
 * Ray r's image is drawn uniformly (im = floor(h0 n / 2^32),
 * h0 = lowbias32(seed ^ r * 2654435769)); proposal t is pixel
 * floor(h_t W H / 2^32) of it, h_t = lowbias32(h0 ^ (t + 1) * 0x9E3779B9),
 * accepted when lowbias32(h_t ^ 0x5BD1E995) & 255 <= its weight (probability
 * (w + 1) / 256, as the reference's rng.integers(0, 256) <= w).  Rays
 * r < uniform_rays take proposal 0 (the reference's uniform share); the others
 * the first accepted proposal, or proposal max_tries - 1.  Outputs as
 * ffn_make_batch.  Errors: -1 for NULL buffers, uniform_rays > num_rays or
 * max_tries outside [1, 2^20]. */
int ffn_make_batch_weighted(const float* images, uint32_t n_images, uint32_t width, uint32_t height,
                            const float* c2w, const float* K, const uint8_t* weights, uint32_t num_rays,
                            uint32_t uniform_rays, uint32_t max_tries, uint32_t seed, void* rays, void* targets,
                            uint32_t* pixel_ids, void* stream);

/* Stage timing (the counterpart of the reference's profiling queue and
 * event_ms, ffnerf_tools.py:11-13,127-138,1521-1530).  When enabled, every
 * ffn_train_step records HIP events around its kernels on the caller's stream;
 * ffn_stage_times waits for the last step and returns the accumulated
 * milliseconds and launch counts per stage since the last reset.  The events
 * of at most 64 stages wait unread; past that the oldest are waited for and
 * added to the totals, so a long profiled run holds a bounded number of
 * events (and may wait on the GPU from inside ffn_train_step).  Stages:
 * 0 sample, 1 hash_fwd, 2 mlp, 3 hash_bwd, 4 mlp_adam, 5 table_adam.  No
 * counterpart in the reference's kernel ABI: it replaces the host-side event
 * reads above. */
#define FFN_N_STAGES 6
int ffn_set_profiling(void* handle, int32_t enable);
int ffn_stage_times(void* handle, float* total_ms, int32_t* launches, int32_t reset);

#ifdef __cplusplus
}
#endif

#endif /* FFNERF_HIP_H */
