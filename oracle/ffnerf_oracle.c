/*
 * ffnerf_oracle.c -- CPU restatement of the reference fused NeRF training step.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline).  The product path (the HIP library) never calls
 * anything in here.
 *
 * It restates, sequentially and in plain C, the semantics of
 *   /root/reference/ffnerf_OG.cl            ffnerf_train_step        (:838-2174)
 *   /root/reference/weight_update.cl        update_ffnerf_oneWG      (:346-577)
 *   /root/reference/decay_occ_grid_in-st.cl occ_nibble_decay_write_both_q24 (:13-113)
 * with every compile-time constant of the reference turned into a runtime
 * parameter (levels, features, per-level table sizes, per-level resolutions,
 * MLP depths, occupancy resolution, background, table optimizer).
 *
 * Floating-point rules (so the HIP path can be compared bit-for-bit where the
 * north star demands it):
 *   - built with -ffp-contract=off; every multiply and add rounds separately,
 *     explicit fmaf only where the reference writes fma();
 *   - work-group scans follow the reference's Blelloch trees operand for
 *     operand, including the reference's down-sweep operand order
 *     (new_right = combine(old_left, old_right), ffnerf_OG.cl:632-634,708-710,
 *     730-732), which composes non-commutative operators out of order;
 *   - powr(x, 1.3) of the sampler (ffnerf_OG.cl:665-671) is evaluated by a
 *     deterministic double-precision exp(y*log(x)) built from + - * / only
 *     (log: exponent split + atanh series; exp: Cody-Waite reduction by ln2 +
 *     Taylor series), identical to the device implementation;
 *   - other transcendentals use the C library (single precision).
 *
 * Built without OpenMP (liboracle.so, the checker) everything runs on one
 * thread in a fixed order.  The same source built with -fopenmp
 * (liboracle_omp.so) is the multi-core CPU baseline only: rays, points and
 * parameters are spread over threads, and the sums into shared arrays (table
 * gradient, reference SGD, proposals) become atomic, so their order varies.
 *
 * Where the reference's result depends on work-item interleaving (the Hogwild
 * CAS scatter into the hash table, ffnerf_OG.cl:2090-2173), the oracle uses
 * the synchronous interleaving: every forward read sees the table as it was
 * at the start of the step; updates are applied afterwards in sample order.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#define ORA_ATOMIC _Pragma("omp atomic")
#else
#define ORA_ATOMIC
#endif

#define ORA_M 64
#define ORA_D_OUT 16
#define ORA_L_DIR 16
#define ORA_C_IN 32
#define ORA_C_OUT 3
#define ORA_S_MAX 64
#define ORA_MAX_LEVELS 32
#define ORA_RELU_WORDS 14

/* layer slots, in the reference's kernel-argument order (ffnerf_tools.py:1210-1232) */
enum { L_WD_IN = 0, L_WD_01, L_WD_12, L_WD_OUT, L_WC_IN, L_WC_01, L_WC_12, L_WC_23, L_WC_OUT, L_COUNT };

typedef struct {
  int32_t n_levels;
  int32_t f_per_level;
  uint32_t log2_T[ORA_MAX_LEVELS];
  uint32_t offset[ORA_MAX_LEVELS];   /* entry offset of each level in the concatenated table */
  int32_t res[ORA_MAX_LEVELS];       /* per-level grid resolution R_l (host computed) */
  float lvl_lr_scale[ORA_MAX_LEVELS];/* 2^(-0.1*l) of the reference SGD (ffnerf_OG.cl:2108) */
  int32_t nd, nc;                    /* hidden layers of the density / color MLP */
  int32_t occ_G;
  float box_min[3], box_max[3];
  float rho_min, rho_max, dt_min, dt_max, t_near, t_far;
  int32_t background;                /* 0 black, 1 white, 2 random (train only) */
  int32_t hash_opt;                  /* 0 reference SGD in the step, 1 Adam */
  int32_t table_f16;                 /* the table is stored as IEEE binary16 (values here are its exact
                                        float32 widenings; every update rounds to nearest even, once per
                                        entry and step) */
} ora_cfg;

typedef struct {
  float lr;              /* lr_f: un-bias-corrected (used by the table SGD) */
  float lr_t;            /* bias-corrected Adam step (ffnerf_tools.py:1479-1482) */
  float color_rel_lr;
  float sh_multiplier;
  float occ_strength;
  float beta1, beta2, eps;
  uint32_t rng_seed;
  int32_t do_train;
} ora_scalars;

typedef struct {
  float* W[L_COUNT];
  float* b[L_COUNT];
  float* mW[L_COUNT];
  float* vW[L_COUNT];
  float* mb[L_COUNT];
  float* vb[L_COUNT];
  float* table;
  float* m_table;        /* Adam state of the table (hash_opt == 1) */
  float* v_table;
  uint32_t* occ_in;
  uint32_t* occ_st;
} ora_params;

/* optional intermediate taps; every pointer may be NULL */
typedef struct {
  float* Ts;          /* [N*S]        sample times */
  float* DTs;         /* [N*S]        sample dt */
  uint32_t* flags;    /* [N*2]        run-start bit flags */
  float* a0;          /* [N*S*LF]     hash encoding */
  float* sigma;       /* [N*S] */
  float* rgb;         /* [N*S*3] */
  float* Tr;          /* [N*S]        transmittance before each sample */
  float* T_final;     /* [N] */
  float* dL_dsigma;   /* [N*S] */
  float* dL_dc;       /* [N*S*3] */
  float* dL_da0;      /* [N*S*LF]     gradient of the encoding (gf of :2154-2156) */
  float* gW[L_COUNT]; /* weight gradients (sum over samples), sized like W */
  float* gb[L_COUNT];
  float* g_table;     /* table gradient (hash_opt == 1), sized like table */
  /* ReLU branches, ORA_RELU_WORDS words per sample: words 2h, 2h+1 hold bit n of hidden unit n of hidden
   * layer h (h = 0..2 density, 3..6 colour) */
  const uint32_t* relu_in; /* [N*S][14] input: the branch each unit takes (another implementation's) */
  uint32_t* relu_out;      /* [N*S][14] output: pre-activation > 0 as this restatement computes it */
  float* preact;           /* [N*S][7][64] output: hidden pre-activations */
  /* the composited colour before clamping, background included: the photometric loss's input */
  const float* C_in;       /* [N][4] input: evaluate the loss gradient at this colour (another implementation's) */
  float* C_out;            /* [N][4] output: the colour as composited here */
} ora_debug;

/* ------------------------------------------------------------------ */
/* integer helpers (ffnerf_OG.cl:293-311, decay_occ_grid_in-st.cl:2-10) */

/* ------------------------------------------------------------------ */
/* IEEE 754 binary16 rounding (round to nearest, ties to even), from   */
/* the format's definition: 1 sign, 5 exponent (bias 15), 10 fraction  */
/* bits; subnormals in units of 2^-24; overflow at 65520 to infinity.  */

uint16_t ora_f32_to_f16_bits(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) /* infinity, NaN (quiet, payload kept where it fits) */
    return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? (0x200u | ((ax >> 13) & 0x3FFu)) : 0u));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520: rounds to infinity */
  if (ax < 0x38800000u) {                                  /* below 2^-14: subnormal (or zero) */
    float a;
    memcpy(&a, &ax, 4);
    const float units = a * 16777216.0f; /* |f| / 2^-24, exact */
    float m = floorf(units);
    const float rem = units - m;
    if (rem > 0.5f || (rem == 0.5f && fmodf(m, 2.0f) != 0.0f)) m += 1.0f;
    return (uint16_t)(sign | (uint32_t)m); /* m = 1024 is the smallest normal, 0x0400 */
  }
  uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7FFFFFu) >> 13);
  const uint32_t rem = ax & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* a carry moves into the exponent */
  return (uint16_t)(sign | h);
}

float ora_f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  uint32_t x;
  if (e == 0) {
    float v = (float)m * (1.0f / 16777216.0f);
    memcpy(&x, &v, 4);
  } else if (e == 31) {
    x = 0x7F800000u | (m << 13);
  } else {
    x = ((e + 112u) << 23) | (m << 13);
  }
  x |= sign;
  float r;
  memcpy(&r, &x, 4);
  return r;
}

float ora_f16_round(float f) { return ora_f16_bits_to_f32(ora_f32_to_f16_bits(f)); }

/* thread count of the OpenMP build (the checker build has one) */
void ora_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}
int ora_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

uint32_t ora_hash_u32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

static float rand01(uint32_t* state) {
  uint32_t x = *state;
  x ^= x << 13;
  x ^= x >> 17;
  x ^= x << 5;
  *state = x;
  return (float)(x & 0x00FFFFFFu) * (1.0f / 16777216.0f);
}

float ora_rand01_first(uint32_t seed) { uint32_t s = seed; return rand01(&s); }
uint32_t ora_xorshift32(uint32_t x) { x ^= x << 13; x ^= x >> 17; x ^= x << 5; return x; }

/* ------------------------------------------------------------------ */
/* deterministic powr for the sampler weights (ffnerf_OG.cl:665-671)   */

static const double ORA_LN2_HI = 6.93147180369123816490e-01; /* 0x3fe62e42fee00000 */
static const double ORA_LN2_LO = 1.90821492927058770002e-10; /* 0x3dea39ef35793c76 */

double ora_det_log(double x) {
  uint64_t bits;
  memcpy(&bits, &x, 8);
  int e = (int)((bits >> 52) & 0x7ff) - 1023;
  bits = (bits & 0x000fffffffffffffULL) | 0x3ff0000000000000ULL;
  double m;
  memcpy(&m, &bits, 8);
  if (m > 1.4142135623730951) { m = m * 0.5; e += 1; }
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
  return de * ORA_LN2_HI + (de * ORA_LN2_LO + lnm);
}

double ora_det_exp(double z) {
  double k = floor(z * 1.4426950408889634 + 0.5);
  double r = (z - k * ORA_LN2_HI) - k * ORA_LN2_LO;
  double p = 1.0 / 6227020800.0;        /* 1/13! */
  p = p * r + 1.0 / 479001600.0;        /* 1/12! */
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
  if (ki > 1023) return INFINITY;
  uint64_t b = (uint64_t)(ki + 1023) << 52;
  double two_k;
  memcpy(&two_k, &b, 8);
  return p * two_k;
}

/* powr(x, y) for finite x > 0 */
float ora_det_powr(float x, float y) {
  return (float)ora_det_exp((double)y * ora_det_log((double)x));
}

static float safe_pow_pos(float x, float gamma) {
  x = fmaxf(x, 0.0f);
  if (x <= 0.0f) return 0.0f;
  if (!(x < INFINITY)) return x;
  return ora_det_powr(x, gamma);
}

/* ------------------------------------------------------------------ */
/* ray / AABB (ffnerf_OG.cl:322-343)                                  */

int ora_ray_aabb(const float o[3], const float d[3], const float bmin[3], const float bmax[3],
                 float* t0, float* t1) {
  float tmin3[3], tmax3[3];
  for (int i = 0; i < 3; ++i) {
    float invd = (d[i] != 0.0f) ? (1.0f / d[i]) : INFINITY;
    float tb = (bmin[i] - o[i]) * invd;
    float tt = (bmax[i] - o[i]) * invd;
    tmin3[i] = fminf(tb, tt);
    tmax3[i] = fmaxf(tb, tt);
  }
  float tmin = fmaxf(tmin3[0], fmaxf(tmin3[1], tmin3[2]));
  float tmax = fminf(tmax3[0], fminf(tmax3[1], tmax3[2]));
  if (tmax < tmin) return 0;
  *t0 = tmin;
  *t1 = tmax;
  return 1;
}

/* ------------------------------------------------------------------ */
/* work-group scans, restated sequentially phase by phase              */

static void scan_excl_f(float* a, int n) { /* ffnerf_OG.cl:619-637 */
  for (int stride = 1; stride < n; stride <<= 1)
    for (int lid = 0; lid < n; ++lid) {
      int idx = (lid + 1) * (stride << 1) - 1;
      if (idx < n) a[idx] += a[idx - stride];
    }
  a[n - 1] = 0.0f;
  for (int stride = n >> 1; stride >= 1; stride >>= 1) {
    for (int lid = 0; lid < n; ++lid) {
      int idx = (lid + 1) * (stride << 1) - 1;
      if (idx < n) {
        float t = a[idx - stride];
        a[idx - stride] = a[idx];
        a[idx] += t;
      }
    }
    if (stride == 1) break;
  }
}

static float reduce_sum_f(float* a, int n) { /* ffnerf_OG.cl:639-646 */
  for (int stride = n >> 1; stride >= 1; stride >>= 1) {
    for (int lid = 0; lid < stride; ++lid) a[lid] += a[lid + stride];
    if (stride == 1) break;
  }
  return a[0];
}

static int lower_bound_cdf(const float* cdf, int n, float u) { /* ffnerf_OG.cl:648-656 */
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi) >> 1;
    if (cdf[mid] >= u) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

typedef struct { float a; float v[3]; } Seg;
static Seg seg_combine(Seg L, Seg R) { /* ffnerf_OG.cl:683-684 */
  Seg O;
  O.a = L.a * R.a;
  for (int c = 0; c < 3; ++c) O.v[c] = L.v[c] + L.a * R.v[c];
  return O;
}

static void scan_excl_seg(Seg* s, int n, Seg* total) { /* ffnerf_OG.cl:691-713 */
  for (int stride = 1; stride < n; stride <<= 1)
    for (int lid = 0; lid < n; ++lid) {
      int idx = (lid + 1) * (stride << 1) - 1;
      if (idx < n) s[idx] = seg_combine(s[idx - stride], s[idx]);
    }
  *total = s[n - 1];
  s[n - 1].a = 1.0f;
  s[n - 1].v[0] = s[n - 1].v[1] = s[n - 1].v[2] = 0.0f;
  for (int stride = n >> 1; stride >= 1; stride >>= 1) {
    for (int lid = 0; lid < n; ++lid) {
      int idx = (lid + 1) * (stride << 1) - 1;
      if (idx < n) {
        Seg t = s[idx - stride];
        s[idx - stride] = s[idx];
        s[idx] = seg_combine(t, s[idx]);
      }
    }
    if (stride == 1) break;
  }
}

typedef struct { float a; float b; } Aff;
static Aff aff_combine_rev(Aff L, Aff R) { /* ffnerf_OG.cl:687-689 */
  Aff O;
  O.a = R.a * L.a;
  O.b = R.a * L.b + R.b;
  return O;
}

static void scan_excl_aff_rev(Aff* s, int n, Aff* total) { /* ffnerf_OG.cl:715-735 */
  for (int stride = 1; stride < n; stride <<= 1)
    for (int lid = 0; lid < n; ++lid) {
      int idx = (lid + 1) * (stride << 1) - 1;
      if (idx < n) s[idx] = aff_combine_rev(s[idx - stride], s[idx]);
    }
  *total = s[n - 1];
  s[n - 1].a = 1.0f;
  s[n - 1].b = 0.0f;
  for (int stride = n >> 1; stride >= 1; stride >>= 1) {
    for (int lid = 0; lid < n; ++lid) {
      int idx = (lid + 1) * (stride << 1) - 1;
      if (idx < n) {
        Aff t = s[idx - stride];
        s[idx - stride] = s[idx];
        s[idx] = aff_combine_rev(t, s[idx]);
      }
    }
    if (stride == 1) break;
  }
}

/* exported for tests: the two composite scans on plain arrays */
void ora_scan_excl_f(float* a, int n) { scan_excl_f(a, n); }
float ora_reduce_sum_f(float* a, int n) { return reduce_sum_f(a, n); }
void ora_scan_excl_aff_rev(float* a, float* b, int n, float* tot_a, float* tot_b) {
  Aff s[ORA_S_MAX], t;
  for (int i = 0; i < n; ++i) { s[i].a = a[i]; s[i].b = b[i]; }
  scan_excl_aff_rev(s, n, &t);
  for (int i = 0; i < n; ++i) { a[i] = s[i].a; b[i] = s[i].b; }
  *tot_a = t.a;
  *tot_b = t.b;
}

/* ------------------------------------------------------------------ */
/* occupancy nibble helpers (ffnerf_OG.cl:446-512)                    */

static uint32_t chg_get(const uint32_t* f, uint32_t idx) { return (f[idx >> 5] >> (idx & 31u)) & 1u; }

static uint32_t chg_find_next(const uint32_t* f, uint32_t idx, uint32_t WG) {
  uint32_t i = idx + 1u;
  if (i >= WG) return WG;
  uint32_t w = i >> 5, b = i & 31u;
  uint32_t mask = f[w] & (~0u << b);
  for (;;) {
    if (mask) {
      uint32_t off = (uint32_t)__builtin_ctz(mask);
      uint32_t res = (w << 5) + off;
      return (res < WG) ? res : WG;
    }
    w++;
    if ((w << 5) >= WG) break;
    mask = f[w];
  }
  return WG;
}

static void occ_nibble_max(uint32_t* grid, int cell, uint32_t sub, uint32_t proposed_q) {
  uint32_t shift = 4u * sub;
#ifdef _OPENMP
  uint32_t old_u = __atomic_load_n(&grid[cell], __ATOMIC_RELAXED);
  for (;;) {
    uint32_t old_q = ((old_u >> shift) & 0xFu) + 1u;
    if (proposed_q <= old_q) return;
    uint32_t nu = (old_u & ~(0xFu << shift)) | (((proposed_q - 1u) & 0xFu) << shift);
    if (__atomic_compare_exchange_n(&grid[cell], &old_u, nu, 0, __ATOMIC_RELAXED, __ATOMIC_RELAXED)) return;
  }
#else
  uint32_t old_u = grid[cell];
  uint32_t old_q = ((old_u >> shift) & 0xFu) + 1u;
  if (proposed_q <= old_q) return;
  grid[cell] = (old_u & ~(0xFu << shift)) | (((proposed_q - 1u) & 0xFu) << shift);
#endif
}

/* ------------------------------------------------------------------ */
/* sampler: occupancy-weighted importance resampling (ffnerf_OG.cl:1002-1250) */

void ora_sample_ray(const ora_cfg* c, const float* ray, uint32_t ray_id, int S, uint32_t seed,
                    const uint32_t* occ_in, int do_train, float* Ts, float* DTs, uint32_t* flags) {
  const float* o = ray;
  const float* d = ray + 4;
  const uint32_t WG = (uint32_t)S;
  flags[0] = flags[1] = 0u;

  float t0 = 0.0f, t1 = 0.0f;
  int hit = ora_ray_aabb(o, d, c->box_min, c->box_max, &t0, &t1);
  float t0_l = 0.0f, t1_l = 0.0f;
  int hit_l = 0;
  if (hit) {
    t0 = fmaxf(t0, c->t_near);
    t1 = fminf(t1, c->t_far);
    if (t1 <= t0) {
      hit_l = 0;
    } else {
      hit_l = 1;
      t0_l = t0 + 1.0e-6f;
      t1_l = t1;
    }
  }
  float dtb = hit_l ? ((t1_l - t0_l) * (1.0f / (float)WG)) : 0.0f;
  dtb = fminf(c->dt_max, fmaxf(c->dt_min, dtb));
  const float dt_base = hit_l ? dtb : 0.0f;

  if (!hit_l) {
    for (uint32_t i = 0; i < WG; ++i) {
      Ts[i] = 0.0f;
      DTs[i] = 0.0f;
      flags[i >> 5] |= 1u << (i & 31u);
    }
    return;
  }
  uint32_t rng0 = ora_hash_u32(seed ^ ray_id * 1597334677u);
  const float u0 = rand01(&rng0) * (1.0f / (float)WG);

  const int G = c->occ_G;
  float box_size[3], inv_box[3];
  for (int i = 0; i < 3; ++i) {
    box_size[i] = c->box_max[i] - c->box_min[i];
    inv_box[i] = 1.0f / box_size[i];
  }

  float cand_t[ORA_S_MAX], wp[ORA_S_MAX], act[ORA_S_MAX], buf[ORA_S_MAX];
  for (uint32_t lid = 0; lid < WG; ++lid) {
    uint32_t rng = ora_hash_u32(seed ^ ray_id * 747796405u ^ lid * 2891336453u);
    float u = ((float)lid + rand01(&rng)) * (1.0f / (float)WG);
    float tk = t0_l + (t1_l - t0_l) * u;
    cand_t[lid] = tk;
    float gm[3];
    for (int i = 0; i < 3; ++i) {
      float xk = o[i] + tk * d[i];
      gm[i] = (xk - c->box_min[i]) * inv_box[i] * (float)G;
    }
    float occ = 0.0f;
    if (gm[0] >= 0.0f && gm[0] < (float)G && gm[1] >= 0.0f && gm[1] < (float)G && gm[2] >= 0.0f &&
        gm[2] < (float)G) {
      int im[3];
      uint32_t sub = 0;
      for (int i = 0; i < 3; ++i) {
        int v = (int)floorf(gm[i]);
        im[i] = v < 0 ? 0 : (v > G - 1 ? G - 1 : v);
        float f = gm[i] - floorf(gm[i]);
        f = fminf(fmaxf(f, 0.0f), 1.0f - 1e-7f);
        sub += (f > 0.5f ? 1u : 0u) << i;
      }
      int cell = im[0] + G * (im[1] + G * im[2]);
      uint32_t occ4 = (occ_in[cell] >> (4u * sub)) & 0xFu;
      uint32_t q_train = occ4 + 1u;
      uint32_t q_infer = (occ4 > 2u) ? (occ4 - 2u) : 0u;
      uint32_t q_eff = do_train ? q_train : q_infer;
      occ = (float)q_eff * (1.0f / 16.0f);
    }
    float infer_f = do_train ? 0.0f : 1.0f;
    float active = (occ > 0.0f) ? 1.0f : 0.0f;
    float rho_base = c->rho_min + (c->rho_max - c->rho_min) * occ;
    float rho = rho_base * (1.0f - infer_f + infer_f * active);
    float w_raw = rho * dt_base;
    wp[lid] = safe_pow_pos(w_raw, 1.3f);
    act[lid] = active;
  }

  /* pref = exclusive scan of wp; Wtot; gtot (LAMBDA_FOCUS = 0 => exp(-0*pi) = 1); active count */
  float pref[ORA_S_MAX];
  memcpy(buf, wp, sizeof(float) * WG);
  scan_excl_f(buf, (int)WG);
  memcpy(pref, buf, sizeof(float) * WG);
  memcpy(buf, wp, sizeof(float) * WG);
  float Wtot = fmaxf(reduce_sum_f(buf, (int)WG), 1.0e-12f);
  /* g = wp * exp(-LAMBDA_FOCUS * pref/Wtot); LAMBDA_FOCUS is 0 (ffnerf_OG.cl:57), so the gain is exactly 1 */
  float g[ORA_S_MAX];
  for (uint32_t lid = 0; lid < WG; ++lid) g[lid] = wp[lid];
  (void)pref;
  (void)Wtot;
  memcpy(buf, g, sizeof(float) * WG);
  float gtot = fmaxf(reduce_sum_f(buf, (int)WG), 1.0e-12f);
  memcpy(buf, act, sizeof(float) * WG);
  float active_count = reduce_sum_f(buf, (int)WG);
  float any_active = (active_count > 0.5f) ? 1.0f : 0.0f;
  float inv_active = 1.0f / fmaxf(active_count, 1.0f);

  float p[ORA_S_MAX];
  const float uniform_part = 0.3f;
  for (uint32_t lid = 0; lid < WG; ++lid) {
    float uta = act[lid] * inv_active;
    float lo = 1.0f / (float)WG;
    float uniform_term = lo + (uta - lo) * any_active; /* mix() */
    float proposal_term = any_active * (g[lid] / gtot);
    p[lid] = uniform_part * uniform_term + (1.0f - uniform_part) * proposal_term;
  }
  float cdf[ORA_S_MAX];
  memcpy(buf, p, sizeof(float) * WG);
  scan_excl_f(buf, (int)WG);
  for (uint32_t lid = 0; lid < WG; ++lid) cdf[lid] = buf[lid] + p[lid];

  uint32_t key[ORA_S_MAX];
  for (uint32_t lid = 0; lid < WG; ++lid) {
    float uk = u0 + (float)lid * (1.0f / (float)WG);
    uk = fminf(uk, 0.99999994f);
    int idx = lower_bound_cdf(cdf, (int)WG, uk);
    float t_out = cand_t[idx];
    Ts[lid] = t_out;
    DTs[lid] = dt_base;
    float go[3];
    for (int i = 0; i < 3; ++i) {
      float xo = o[i] + t_out * d[i];
      go[i] = (xo - c->box_min[i]) * inv_box[i] * (float)G;
    }
    uint32_t k = 0xFFFFFFFEu;
    int ix = (int)floorf(go[0]), iy = (int)floorf(go[1]), iz = (int)floorf(go[2]);
    if ((uint32_t)ix < (uint32_t)G && (uint32_t)iy < (uint32_t)G && (uint32_t)iz < (uint32_t)G) {
      uint32_t sub = 0;
      for (int i = 0; i < 3; ++i) {
        float f = go[i] - floorf(go[i]);
        f = fminf(fmaxf(f, 0.0f), 1.0f - 1e-7f);
        sub += (f >= 0.5f ? 1u : 0u) << i;
      }
      int cell = ix + G * (iy + G * iz);
      k = (((uint32_t)cell) << 3) | (sub & 7u);
    }
    key[lid] = k;
  }
  for (uint32_t lid = 0; lid < WG; ++lid)
    if (lid == 0 || key[lid] != key[lid - 1]) flags[lid >> 5] |= 1u << (lid & 31u);
}

/* ------------------------------------------------------------------ */
/* hash grid (ffnerf_OG.cl:1286-1364 fwd, :2090-2173 bwd)              */

static void normalize_pos(const ora_cfg* c, const float x[3], float p[3]) {
  for (int i = 0; i < 3; ++i) {
    float bs = c->box_max[i] - c->box_min[i];
    float v = (x[i] - c->box_min[i]) / bs;
    p[i] = fminf(fmaxf(v, 0.0f), 1.0f - 1.0e-6f);
  }
}

static void level_corners(const ora_cfg* c, int lvl, const float p[3], uint32_t feat[8], float w[8]) {
  int R = c->res[lvl];
  int i0[3];
  float f[3];
  for (int i = 0; i < 3; ++i) {
    float u = p[i] * (float)R;
    int v = (int)floorf(u);
    v = v < 0 ? 0 : (v > R - 2 ? R - 2 : v);
    i0[i] = v;
    f[i] = u - (float)v;
  }
  const uint32_t mask = (1u << c->log2_T[lvl]) - 1u;
  for (int cc = 0; cc < 8; ++cc) {
    int dx = cc & 1, dy = (cc >> 1) & 1, dz = (cc >> 2) & 1;
    float wx = dx ? f[0] : 1.0f - f[0];
    float wy = dy ? f[1] : 1.0f - f[1];
    float wz = dz ? f[2] : 1.0f - f[2];
    w[cc] = wx * wy * wz;
    uint32_t h = ora_hash_u32((uint32_t)(i0[0] + dx) * 73856093u ^ (uint32_t)(i0[1] + dy) * 19349663u ^
                              (uint32_t)(i0[2] + dz) * 83492791u ^ (uint32_t)lvl * 2654435761u) & mask;
    feat[cc] = (c->offset[lvl] + h) * (uint32_t)c->f_per_level;
  }
}

/* encoding of one point x[3] -> a0[LF]; optionally its feature base indices [L*8] and weights [L*8] */
static void encode_point(const ora_cfg* c, const float* table, const float* x, float* a0, uint32_t* idx_out,
                         float* w_out) {
  const int L = c->n_levels, F = c->f_per_level;
  float p[3];
  normalize_pos(c, x, p);
  for (int l = 0; l < L; ++l) {
    uint32_t feat[8];
    float w[8];
    level_corners(c, l, p, feat, w);
    for (int f = 0; f < F; ++f) {
      float acc = 0.0f;
      for (int cc = 0; cc < 8; ++cc) acc += w[cc] * table[feat[cc] + (uint32_t)f];
      a0[l * F + f] = acc;
    }
    if (idx_out)
      for (int cc = 0; cc < 8; ++cc) idx_out[l * 8 + cc] = feat[cc];
    if (w_out)
      for (int cc = 0; cc < 8; ++cc) w_out[l * 8 + cc] = w[cc];
  }
}

/* encode n points x[n*3] -> a0[n*LF]; optionally the feature base index [n*L*8] and weights [n*L*8] */
void ora_hash_encode(const ora_cfg* c, const float* table, const float* x, int64_t n, float* a0,
                     uint32_t* idx_out, float* w_out) {
  const int L = c->n_levels, LF = L * c->f_per_level;
#pragma omp parallel for schedule(static)
  for (int64_t s = 0; s < n; ++s)
    encode_point(c, table, x + 3 * s, a0 + s * LF, idx_out ? idx_out + s * L * 8 : NULL,
                 w_out ? w_out + s * L * 8 : NULL);
}

/* scatter the encoding gradient g[n*LF] of points x into grad (plain sum, double accumulators) */
void ora_hash_backward(const ora_cfg* c, const float* x, const float* g, int64_t n, double* grad) {
  const int L = c->n_levels, F = c->f_per_level, LF = L * F;
#pragma omp parallel for schedule(static)
  for (int64_t s = 0; s < n; ++s) {
    float p[3];
    normalize_pos(c, x + 3 * s, p);
    for (int l = 0; l < L; ++l) {
      uint32_t feat[8];
      float w[8];
      level_corners(c, l, p, feat, w);
      for (int f = 0; f < F; ++f) {
        float gf = g[s * LF + l * F + f];
        if (!isfinite(gf)) continue;
        for (int cc = 0; cc < 8; ++cc) {
          ORA_ATOMIC
          grad[feat[cc] + (uint32_t)f] += (double)(gf * w[cc]);
        }
      }
    }
  }
}

/* ------------------------------------------------------------------ */
/* activations (ffnerf_OG.cl:214-253)                                 */

static float softplus(float x) {
  if (x > 20.0f) return x;
  if (x < -20.0f) return expf(x);
  return log1pf(expf(x));
}
static float softplus_prime_from_pre(float x) {
  if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
  return expf(x) / (1.0f + expf(x));
}
static float sigmoid_soft(float x) {
  x *= 0.5f;
  x = fminf(fmaxf(x, -18.0f), 18.0f);
  if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
  return expf(x) / (1.0f + expf(x));
}
static float charbonnier_prime(float x) {
  const float e2 = 1.0e-3f * 1.0e-3f;
  return x * (1.0f / sqrtf(x * x + e2));
}

void ora_sh_encode(const float d[3], float* sh) { /* ffnerf_OG.cl:572-602 */
  float x = d[0], y = d[1], z = d[2];
  sh[0] = 0.28209479177387814f;
  sh[1] = 0.4886025119029199f * y;
  sh[2] = 0.4886025119029199f * z;
  sh[3] = 0.4886025119029199f * x;
  sh[4] = 1.0925484305920792f * x * y;
  sh[5] = 1.0925484305920792f * y * z;
  sh[6] = 0.31539156525252005f * (3.0f * z * z - 1.0f);
  sh[7] = 1.0925484305920792f * x * z;
  sh[8] = 0.5462742152960396f * (x * x - y * y);
  sh[9] = 0.5900435899266435f * y * (3.0f * x * x - y * y);
  sh[10] = 2.890611442640554f * x * y * z;
  sh[11] = 0.4570457994644658f * y * (5.0f * z * z - 1.0f);
  sh[12] = 0.3731763325901154f * (5.0f * z * z * z - 3.0f * z);
  sh[13] = 0.4570457994644658f * x * (5.0f * z * z - 1.0f);
  sh[14] = 1.445305721320277f * z * (x * x - y * y);
  sh[15] = 0.5900435899266435f * x * (x * x - 3.0f * y * y);
}

/* out[i] = act(b[i] + sum_j W[i*in + j] * in[j]), sequential from the bias (ffnerf_OG.cl:754-806) */
static void fc(float* out, const float* in, int in_dim, int out_dim, const float* W, const float* b, int relu) {
  for (int i = 0; i < out_dim; ++i) {
    float sum = b ? b[i] : 0.0f;
    for (int j = 0; j < in_dim; ++j) sum += W[i * in_dim + j] * in[j];
    out[i] = relu ? (sum > 0.0f ? sum : 0.0f) : sum;
  }
}

/* delta_in[j] = sum_i W[i*in_dim + j] * delta_out[i] (ffnerf_OG.cl:811-835) */
static void fc_bwd(float* din, const float* dout, int out_dim, int in_dim, const float* W) {
  for (int j = 0; j < in_dim; ++j) {
    float s = 0.0f;
    for (int i = 0; i < out_dim; ++i) s += W[i * in_dim + j] * dout[i];
    din[j] = s;
  }
}

/* per-sample MLP state */
typedef struct {
  float a0[ORA_M];          /* LF <= 64 */
  float hd[3][ORA_M];       /* density hidden activations */
  float acin[ORA_C_IN];     /* [dout(16), SH*mult(16)] */
  float hc[4][ORA_M];       /* color hidden activations */
  uint64_t on[7];           /* ReLU branch of every hidden unit (h = 0..2 density, 3..6 colour) */
  uint64_t own[7];          /* pre-activation > 0, as computed here */
  float pre[7][ORA_M];      /* hidden pre-activations */
  float sigma;
  float rgb[3];
} mlp_state;

/* hidden layer h: pre-activations from fc, then the ReLU.  Unit n passes its pre-activation when its
 * branch is on: the branch is pre > 0 (ffnerf_OG.cl:754-791), or, when `force` is given, bit n of the
 * layer's words there (another implementation's decision; that unit's value is then passed unclamped). */
static void hidden(mlp_state* st, int h, float* out, const float* in, int in_dim, const float* W, const float* b,
                   const uint32_t* force) {
  fc(st->pre[h], in, in_dim, ORA_M, W, b, 0);
  uint64_t own = 0, on;
  for (int n = 0; n < ORA_M; ++n)
    if (st->pre[h][n] > 0.0f) own |= 1ull << n;
  on = force ? ((uint64_t)force[2 * h] | ((uint64_t)force[2 * h + 1] << 32)) : own;
  for (int n = 0; n < ORA_M; ++n) out[n] = ((on >> n) & 1ull) ? st->pre[h][n] : 0.0f;
  st->own[h] = own;
  st->on[h] = on;
}

static int unit_on(const mlp_state* st, int h, int n) { return (int)((st->on[h] >> n) & 1ull); }

static void mlp_forward(const ora_cfg* c, const ora_params* P, const float* dir, float sh_mult, mlp_state* st,
                        const uint32_t* force) {
  const int LF = c->n_levels * c->f_per_level;
  const int nd = c->nd, nc = c->nc;
  memset(st->on, 0, sizeof(st->on));
  memset(st->own, 0, sizeof(st->own));
  memset(st->pre, 0, sizeof(st->pre));
  hidden(st, 0, st->hd[0], st->a0, LF, P->W[L_WD_IN], P->b[L_WD_IN], force);
  if (nd >= 2) hidden(st, 1, st->hd[1], st->hd[0], ORA_M, P->W[L_WD_01], P->b[L_WD_01], force);
  if (nd >= 3) hidden(st, 2, st->hd[2], st->hd[1], ORA_M, P->W[L_WD_12], P->b[L_WD_12], force);
  float dout[ORA_D_OUT];
  fc(dout, st->hd[nd - 1], ORA_M, ORA_D_OUT, P->W[L_WD_OUT], P->b[L_WD_OUT], 0);
  for (int i = 0; i < ORA_D_OUT; ++i) st->acin[i] = dout[i];
  st->sigma = softplus(fminf(fmaxf(dout[0], -10.0f), 10.0f));
  ora_sh_encode(dir, st->acin + ORA_D_OUT);
  for (int i = 0; i < ORA_L_DIR; ++i) st->acin[ORA_D_OUT + i] *= sh_mult;
  hidden(st, 3, st->hc[0], st->acin, ORA_C_IN, P->W[L_WC_IN], P->b[L_WC_IN], force);
  static const int slot[4] = {0, L_WC_01, L_WC_12, L_WC_23};
  for (int k = 1; k < nc; ++k) hidden(st, 3 + k, st->hc[k], st->hc[k - 1], ORA_M, P->W[slot[k]], P->b[slot[k]], force);
  float cout[ORA_C_OUT];
  fc(cout, st->hc[nc - 1], ORA_M, ORA_C_OUT, P->W[L_WC_OUT], P->b[L_WC_OUT], 0);
  for (int i = 0; i < 3; ++i) st->rgb[i] = sigmoid_soft(cout[i]);
}

/* exported: forward of one sample given its encoding (for MLP tests) */
void ora_mlp_forward(const ora_cfg* c, const ora_params* P, const float* a0, const float* dir, float sh_mult,
                     float* sigma, float* rgb, float* dout) {
  mlp_state st;
  const int LF = c->n_levels * c->f_per_level;
  memcpy(st.a0, a0, sizeof(float) * LF);
  mlp_forward(c, P, dir, sh_mult, &st, NULL);
  *sigma = st.sigma;
  for (int i = 0; i < 3; ++i) rgb[i] = st.rgb[i];
  if (dout) memcpy(dout, st.acin, sizeof(float) * ORA_D_OUT);
}

static int dim_out(int slot, const ora_cfg* c, int* in_dim) {
  const int LF = c->n_levels * c->f_per_level;
  switch (slot) {
    case L_WD_IN: *in_dim = LF; return ORA_M;
    case L_WD_OUT: *in_dim = ORA_M; return ORA_D_OUT;
    case L_WC_IN: *in_dim = ORA_C_IN; return ORA_M;
    case L_WC_OUT: *in_dim = ORA_M; return ORA_C_OUT;
    default: *in_dim = ORA_M; return ORA_M;
  }
}

static int slot_active(int slot, const ora_cfg* c) {
  switch (slot) {
    case L_WD_01: return c->nd >= 2;
    case L_WD_12: return c->nd >= 3;
    case L_WC_01: return c->nc >= 2;
    case L_WC_12: return c->nc >= 3;
    case L_WC_23: return c->nc >= 4;
    default: return 1;
  }
}

int ora_layer_shape(const ora_cfg* c, int slot, int* out_dim, int* in_dim) {
  if (!slot_active(slot, c)) { *out_dim = 0; *in_dim = 0; return 0; }
  *out_dim = dim_out(slot, c, in_dim);
  return 1;
}

/* ------------------------------------------------------------------ */
/* occupancy proposals of one ray (ffnerf_OG.cl:1640-1821)            */

void ora_occ_propose_ray(const ora_cfg* c, const float* ray, uint32_t ray_id, int S, uint32_t seed,
                         const float* Ts, const float* DTs, const float* Tr, float T_final, const uint32_t* flags,
                         const uint32_t* occ_in, uint32_t* occ_st) {
  const float* o = ray;
  const float* d = ray + 4;
  const int G = c->occ_G;
  const uint32_t WG = (uint32_t)S;
  float box_size[3], inv_box[3], cell_size[3];
  for (int i = 0; i < 3; ++i) {
    box_size[i] = c->box_max[i] - c->box_min[i];
    inv_box[i] = 1.0f / box_size[i];
    cell_size[i] = box_size[i] * (1.0f / (float)G);
  }
  for (uint32_t lid = 0; lid < WG; ++lid) {
    float dt_s = DTs[lid];
    if (!(dt_s > 0.0f)) continue;
    if (!chg_get(flags, lid)) continue;
    float t = Ts[lid];
    float x[3], gpos[3];
    for (int i = 0; i < 3; ++i) {
      x[i] = o[i] + t * d[i];
      gpos[i] = (x[i] - c->box_min[i]) * inv_box[i] * (float)G;
    }
    int ix = (int)floorf(gpos[0]), iy = (int)floorf(gpos[1]), iz = (int)floorf(gpos[2]);
    if (!((uint32_t)ix < (uint32_t)G && (uint32_t)iy < (uint32_t)G && (uint32_t)iz < (uint32_t)G)) continue;
    uint32_t sub = 0;
    for (int i = 0; i < 3; ++i) {
      float f = gpos[i] - floorf(gpos[i]);
      sub += (f >= 0.5f ? 1u : 0u) << i;
    }
    int cell = ix + G * (iy + G * iz);
    uint32_t next = chg_find_next(flags, lid, WG);

    float pred = 0.0f;
    {
      float cmin[3], cmax[3];
      int ii[3] = {ix, iy, iz};
      for (int i = 0; i < 3; ++i) {
        cmin[i] = c->box_min[i] + (float)ii[i] * cell_size[i];
        cmax[i] = cmin[i] + cell_size[i];
      }
      float t_enter, t_exit;
      if (ora_ray_aabb(o, d, cmin, cmax, &t_enter, &t_exit)) {
        t_enter = fmaxf(t_enter, c->t_near);
        t_exit = fminf(t_exit, c->t_far);
        if (t_exit > t_enter) {
          uint32_t prev_end = lid > 0 ? lid - 1 : 0;
          float t_prev = Ts[prev_end], T_prev = Tr[prev_end];
          float t_cur = Ts[lid], T_cur = Tr[lid];
          float denom0 = t_cur - t_prev;
          float u0 = (fabsf(denom0) > 1.0e-8f) ? (t_enter - t_prev) / denom0 : 0.0f;
          u0 = fminf(fmaxf(u0, 0.0f), 1.0f);
          float T_enter = T_prev + (T_cur - T_prev) * u0;
          uint32_t last = (next < WG) ? (next - 1u) : (WG - 1u);
          float t_last = Ts[last], T_last = Tr[last];
          float t_next = (next < WG) ? Ts[next] : t_exit;
          float T_next = (next < WG) ? Tr[next] : T_final;
          float denom1 = t_next - t_last;
          float u1 = (fabsf(denom1) > 1.0e-8f) ? (t_exit - t_last) / denom1 : 1.0f;
          u1 = fminf(fmaxf(u1, 0.0f), 1.0f);
          float T_exit = T_last + (T_next - T_last) * u1;
          float pv = (T_enter - T_exit) / fmaxf(T_enter, 1.0e-12f);
          pred = fminf(1.0f, fmaxf(0.0f, pv));
        }
      }
    }
    uint32_t old_q = ((occ_in[cell] >> (4u * sub)) & 0xFu) + 1u;
    uint32_t proposed_q = old_q;
    float pred16 = pred * 16.0f;
    uint32_t hseed = ora_hash_u32(seed ^ ray_id * 747796405u ^ lid * 2891336453u ^ (uint32_t)cell * 9781u ^
                                  sub * 6271u);
    if (pred16 > (float)old_q && old_q < 16u) {
      float f0 = floorf(pred16);
      float frac = pred16 - f0;
      uint32_t q0 = (uint32_t)f0;
      uint32_t r24 = hseed & 0x00FFFFFFu;
      uint32_t thresh = (uint32_t)(frac * 16777216.0f);
      uint32_t q_stoch = (r24 < thresh) ? (q0 + 1u) : q0;
      if (q_stoch > 16u) q_stoch = 16u;
      proposed_q = q_stoch;
    }
    float lat = (c->box_max[0] - c->box_min[0]) * (1.0f / (float)G);
    float dd[3] = {c->box_max[0] - c->box_min[0], c->box_max[1] - c->box_min[1], c->box_max[2] - c->box_min[2]};
    float D = 0.5f * sqrtf(dd[0] * dd[0] + dd[1] * dd[1] + dd[2] * dd[2]);
    float tl = t / fmaxf(lat, 1.0e-12f);
    float Dl = D / fmaxf(lat, 1.0e-12f);
    float num = tl * tl + tl + (1.0f / 3.0f);
    float den = Dl * Dl + Dl + (1.0f / 3.0f);
    float f_keep = num / fmaxf(den, 1.0e-12f);
    float keep_p = fminf(f_keep, 1.0f);
    if (keep_p >= 1.0f) {
      occ_nibble_max(occ_st, cell, sub, proposed_q);
    } else {
      uint32_t rk = hseed;
      if (rand01(&rk) <= keep_p) occ_nibble_max(occ_st, cell, sub, proposed_q);
    }
  }
}

/* the proposals of a batch of rays (rays in order) from given per-sample times, transmittances and run
 * flags: the step's proposal pass (ffnerf_OG.cl:1640-1821) fed with another implementation's compositing
 * results, so that the integer outcome can be compared word for word */
void ora_occ_propose_batch(const ora_cfg* c, const float* rays, int32_t num_rays, int S, uint32_t seed,
                           const float* Ts, const float* DTs, const float* Tr, const float* T_final,
                           const uint32_t* flags, const uint32_t* occ_in, uint32_t* occ_st) {
  for (int32_t r = 0; r < num_rays; ++r) {
    const int64_t b0 = (int64_t)r * S;
    ora_occ_propose_ray(c, rays + 8 * (int64_t)r, (uint32_t)r, S, seed, Ts + b0, DTs + b0, Tr + b0, T_final[r],
                        flags + 2 * (int64_t)r, occ_in, occ_st);
  }
}

/* The occupancy proposals of one marched ray (no counterpart in the reference, whose samples come from the
 * resampler): its n samples at times ts, in march order, are cut into runs of one (cell, subcell) of the
 * occupancy grid -- the key the resampler's run flags use, from the grid position the proposal computes -- and
 * the proposal pass above runs over them as over a resampled ray of n samples (every sample's dt positive),
 * with the compositing's transmittances Tr (T_end after a termination) and T_end as the final one. */
void ora_occ_propose_marched_ray(const ora_cfg* c, const float* ray, uint32_t ray_id, int n, uint32_t seed,
                                 const float* ts, const float* Tr, float T_end, const uint32_t* occ_in,
                                 uint32_t* occ_st) {
  if (n <= 0) return;
  const int G = c->occ_G;
  uint32_t* flags = (uint32_t*)calloc((size_t)(n + 31) / 32, sizeof(uint32_t));
  float* dts = (float*)malloc(sizeof(float) * (size_t)n);
  uint64_t prev_key = 0;
  for (int j = 0; j < n; ++j) {
    float gpos[3];
    for (int i = 0; i < 3; ++i) {
      const float x = ray[i] + ts[j] * ray[4 + i];
      gpos[i] = (x - c->box_min[i]) * (1.0f / (c->box_max[i] - c->box_min[i])) * (float)G;
    }
    const int ix = (int)floorf(gpos[0]), iy = (int)floorf(gpos[1]), iz = (int)floorf(gpos[2]);
    uint64_t key = ~(uint64_t)1; /* outside the grid */
    if ((uint32_t)ix < (uint32_t)G && (uint32_t)iy < (uint32_t)G && (uint32_t)iz < (uint32_t)G) {
      uint32_t sub = 0;
      for (int i = 0; i < 3; ++i) sub += (gpos[i] - floorf(gpos[i]) >= 0.5f ? 1u : 0u) << i;
      key = ((uint64_t)(ix + G * (iy + G * iz)) << 3) | sub;
    }
    if (j == 0 || key != prev_key) flags[j >> 5] |= 1u << (j & 31);
    prev_key = key;
    dts[j] = 1.0f;
  }
  ora_occ_propose_ray(c, ray, ray_id, n, seed, ts, dts, Tr, T_end, flags, occ_in, occ_st);
  free(flags);
  free(dts);
}

/* the proposals of marched rays from another implementation's samples and compositing: counts [num_rays],
 * ts / Tr [sum of counts] in march order, T_final [num_rays] */
void ora_occ_propose_marched_batch(const ora_cfg* c, const float* rays, int32_t num_rays, const uint32_t* counts,
                                   uint32_t seed, const float* ts, const float* Tr, const float* T_final,
                                   const uint32_t* occ_in, uint32_t* occ_st) {
  int64_t base = 0;
  for (int32_t r = 0; r < num_rays; ++r) {
    ora_occ_propose_marched_ray(c, rays + 8 * (int64_t)r, (uint32_t)r, (int)counts[r], seed, ts + base, Tr + base,
                                T_final[r], occ_in, occ_st);
    base += counts[r];
  }
}

/* ------------------------------------------------------------------ */
/* compositing, loss gradient and its backward of one ray (ffnerf_OG.cl:1505-1634) */

/* C_force (optional): the loss gradient is evaluated at this colour instead of the composited one (the
 * Charbonnier derivative has slope up to 1/eps = 1000 near a zero residual, so comparisons with another
 * implementation feed it that implementation's colour); C_own (optional) receives the composited colour */
static void composite_ray(const ora_cfg* c, uint32_t ray_id, int S, uint32_t seed, int do_train,
                          const float* sigma, const float* rgb, const float* DTs, const float* target, float* out4,
                          float* Tr, float* T_final_out, float* dL_dc, float* dL_dsigma, const float* C_force,
                          float* C_own) {
  const uint32_t WG = (uint32_t)S;
  Seg segs[ORA_S_MAX], total;
  float alpha[ORA_S_MAX];
  for (uint32_t lid = 0; lid < WG; ++lid) {
    float dt_s = DTs[lid];
    float sg = (dt_s <= 0.0f) ? 0.0f : sigma[lid];
    float a = 0.0f;
    if (dt_s > 0.0f) {
      float xx = fminf(fmaxf(-sg * dt_s, -5.0f), 18.0f);
      a = 1.0f - expf(xx);
    }
    alpha[lid] = a;
    segs[lid].a = 1.0f - a;
    for (int k = 0; k < 3; ++k) segs[lid].v[k] = a * rgb[3 * lid + k];
  }
  scan_excl_seg(segs, (int)WG, &total);
  for (uint32_t lid = 0; lid < WG; ++lid) Tr[lid] = segs[lid].a;
  float T_final = total.a;
  *T_final_out = T_final;
  float bg[3] = {0.0f, 0.0f, 0.0f};
  if (do_train) {
    if (c->background == 1) {
      bg[0] = bg[1] = bg[2] = 1.0f;
    } else if (c->background == 2) {
      uint32_t r = ora_hash_u32(seed ^ ray_id * 747796405u ^ 0xA511E9B3u);
      bg[0] = rand01(&r);
      bg[1] = rand01(&r);
      bg[2] = rand01(&r);
    }
  }
  float gr[3];
  for (int k = 0; k < 3; ++k) {
    float Cf = total.v[k] + T_final * bg[k];
    out4[k] = fminf(fmaxf(Cf, 0.0f), 1.0f);
    if (C_own) C_own[k] = Cf;
    gr[k] = charbonnier_prime((C_force ? C_force[k] : Cf) - target[k]);
  }
  if (C_own) C_own[3] = 0.0f;
  out4[3] = 0.0f;
  float gT_end = gr[0] * bg[0] + gr[1] * bg[1] + gr[2] * bg[2];

  Aff elem[ORA_S_MAX], scan[ORA_S_MAX], tot_aff;
  for (uint32_t lid = 0; lid < WG; ++lid) {
    float a = alpha[lid];
    const float* cs = rgb + 3 * lid;
    float B = gr[0] * (a * cs[0]) + gr[1] * (a * cs[1]) + gr[2] * (a * cs[2]);
    uint32_t k = (WG - 1u) - lid;
    elem[k].a = 1.0f - a;
    elem[k].b = B;
    float ws = Tr[lid] * a;
    for (int q = 0; q < 3; ++q) dL_dc[3 * lid + q] = ws * gr[q];
  }
  memcpy(scan, elem, sizeof(Aff) * WG);
  scan_excl_aff_rev(scan, (int)WG, &tot_aff);
  for (uint32_t lid = 0; lid < WG; ++lid) {
    uint32_t k = (WG - 1u) - lid;
    float gT_next = gT_end;
    if (k >= 1u) {
      uint32_t m = k - 1u;
      Aff incl = aff_combine_rev(scan[m], elem[m]);
      gT_next = incl.a * gT_end + incl.b;
    }
    float a = alpha[lid];
    float Ts_ = Tr[lid];
    const float* cs = rgb + 3 * lid;
    float gA = gr[0] * (Ts_ * cs[0]) + gr[1] * (Ts_ * cs[1]) + gr[2] * (Ts_ * cs[2]);
    float gAlpha = gA - gT_next * Ts_;
    float dt_s = DTs[lid];
    float dads = (dt_s > 0.0f) ? (dt_s * (1.0f - a)) : 0.0f;
    float regu = (dt_s > 0.0f) ? (5e-3f * dt_s / (float)(uint32_t)S) : 0.0f;
    dL_dsigma[lid] = gAlpha * dads + regu;
  }
}

void ora_composite_ray(const ora_cfg* c, uint32_t ray_id, int S, uint32_t seed, int do_train,
                       const float* sigma, const float* rgb, const float* DTs, const float* target, float* out4,
                       float* Tr, float* T_final_out, float* dL_dc, float* dL_dsigma) {
  composite_ray(c, ray_id, S, seed, do_train, sigma, rgb, DTs, target, out4, Tr, T_final_out, dL_dc, dL_dsigma, NULL,
                NULL);
}

/* ------------------------------------------------------------------ */
/* Adam, reference form (weight_update.cl:177-201)                    */

void ora_adam(float* p, float* m, float* v, const float* g, int64_t n, float lr_t, float beta1, float beta2,
              float eps) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    float mi = fmaf(1.0f - beta1, g[i], beta1 * m[i]);
    float vi = fmaf(1.0f - beta2, g[i] * g[i], beta2 * v[i]);
    float denom = sqrtf(vi) + eps;
    p[i] = p[i] - lr_t * (mi / denom);
    m[i] = mi;
    v[i] = vi;
  }
}

/* ------------------------------------------------------------------ */
/* occupancy decay/merge (decay_occ_grid_in-st.cl:13-113)            */

void ora_occ_decay(uint32_t* occ_in, uint32_t* occ_st, uint32_t n_words, uint32_t decay_q24, uint32_t seed) {
  for (uint32_t gid = 0; gid < n_words; ++gid) {
    const uint32_t win = occ_in[gid], wst = occ_st[gid];
    uint32_t out = wst;
    const uint32_t x = wst ^ win;
    for (uint32_t s = 0; s < 8; ++s) {
      const uint32_t shift = s * 4u;
      if (wst != win && ((x >> shift) & 0xFu) != 0u) continue;
      const uint32_t q = ((wst >> shift) & 0xFu) + 1u;
      if (q <= 1u) continue;
      const uint32_t qd24 = q * decay_q24;
      uint32_t cand = (qd24 >> 24) + 1u;
      const uint32_t thresh = 0x01000000u - (qd24 & 0x00FFFFFFu);
      uint32_t hx = seed ^ (gid * 9781u) ^ (s * 6271u) ^ wst;
      if (wst != win) hx ^= (win * 1597u);
      const uint32_t r24 = ora_hash_u32(hx) & 0x00FFFFFFu;
      if (cand > 1u && r24 < thresh) cand -= 1u;
      if (cand < 1u) cand = 1u;
      if (cand > 16u) cand = 16u;
      out = (out & ~(0xFu << shift)) | (((cand - 1u) & 0xFu) << shift);
    }
    occ_st[gid] = out;
    occ_in[gid] = out;
  }
}

/* ------------------------------------------------------------------ */
/* the full step: sampler -> encode -> MLPs -> composite -> proposals  */
/* -> deltas -> MLP backward -> table update -> weight grads -> Adam   */

/* backward of one sample from its loss gradients (ffnerf_OG.cl:1863-2173): output deltas with the distance
 * gate f_vol, the colour and density MLP backward through the sample's ReLU branches, the weight gradients
 * added to gW/gb (weight_update.cl:260-314), the encoding gradient (written to gf_out when given) and the
 * table update -- summed into gtab (Adam, or a binary16 table's SGD) or added to the table one
 * contribution at a time (the reference SGD).  x is the sample's position, t/dtl its time and dt. */
/* the step's parameter updates: MLP Adam with colour layers at lr_t * color_rel_lr
 * (weight_update.cl:487-573) from the summed weight gradients, then the table -- Adam on its summed gradient,
 * or a binary16 table's summed SGD update added once (rounded to nearest even); the reference SGD on a float
 * table was applied during the backward.  gtab may be NULL (no table update). */
static void apply_updates(const ora_cfg* c, ora_params* P, const ora_scalars* sc, double** gW, double** gb,
                          const int* odim, const int* idim, double* gtab, int64_t table_n, ora_debug* dbg) {
  /* MLP Adam; color layers at lr_t * color_rel_lr (weight_update.cl:487-573) */
  for (int k = 0; k < L_COUNT; ++k) {
    if (!gW[k]) continue;
    int n = odim[k] * idim[k];
    float* gwf = (float*)malloc(sizeof(float) * n);
    float* gbf = (float*)malloc(sizeof(float) * odim[k]);
    for (int i = 0; i < n; ++i) gwf[i] = (float)gW[k][i];
    for (int i = 0; i < odim[k]; ++i) gbf[i] = (float)gb[k][i];
    float lrk = (k >= L_WC_IN) ? sc->lr_t * sc->color_rel_lr : sc->lr_t;
    if (dbg && dbg->gW[k]) memcpy(dbg->gW[k], gwf, sizeof(float) * n);
    if (dbg && dbg->gb[k]) memcpy(dbg->gb[k], gbf, sizeof(float) * odim[k]);
    ora_adam(P->W[k], P->mW[k], P->vW[k], gwf, n, lrk, sc->beta1, sc->beta2, sc->eps);
    ora_adam(P->b[k], P->mb[k], P->vb[k], gbf, odim[k], lrk, sc->beta1, sc->beta2, sc->eps);
    free(gwf);
    free(gbf);
  }
  if (gtab && c->hash_opt == 1) {
    float* gtf = (float*)malloc(sizeof(float) * (size_t)table_n);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < table_n; ++i) gtf[i] = (float)gtab[i];
    if (dbg && dbg->g_table) memcpy(dbg->g_table, gtf, sizeof(float) * (size_t)table_n);
    ora_adam(P->table, P->m_table, P->v_table, gtf, table_n, sc->lr_t, sc->beta1, sc->beta2, sc->eps);
    free(gtf);
    if (c->table_f16) {
#pragma omp parallel for schedule(static)
      for (int64_t i = 0; i < table_n; ++i) P->table[i] = ora_f16_round(P->table[i]);
    }
  } else if (gtab) { /* binary16 table, reference SGD: each entry's summed update in one rounding */
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < table_n; ++i) P->table[i] = ora_f16_round(P->table[i] + (float)gtab[i]);
  }
}

static void sample_backward(const ora_cfg* c, ora_params* P, const ora_scalars* sc, const mlp_state* m,
                            const float x[3], float t, float dtl, float D, float dLds, const float* dLdc,
                            double** lgW, double** lgb, double* gtab, float* gf_out) {
  static const int cslot[4] = {L_WC_IN, L_WC_01, L_WC_12, L_WC_23};
  static const int dslot[3] = {L_WD_IN, L_WD_01, L_WD_12};
  const int L = c->n_levels, F = c->f_per_level, LF = L * F;
  const int nd = c->nd, nc = c->nc;
  /* output deltas with the distance gate f_vol (ffnerf_OG.cl:1863-1891) */
  float num = t * t + t * dtl + (dtl * dtl / 3.0f);
  float den = D * D + D * dtl + (dtl * dtl / 3.0f);
  float xg = t / fmaxf(D, 1.0e-12f);
  float sg = (xg >= 1.0f) ? 0.0f : 1.0f;
  float gate = (1.0f - sg) * 1.0f + sg * powf(fmaxf(xg, 1.0e-12f), 0.2f);
  float f_vol = gate * num / fmaxf(den, 1.0e-12f);
  float d_sigma = f_vol * dLds;
  float dcout[ORA_C_OUT], ddout[ORA_D_OUT];
  for (int k = 0; k < 3; ++k) {
    float sk = m->rgb[k];
    dcout[k] = (f_vol * dLdc[k]) * ((sk * (1.0f - sk)) * 0.5f);
  }
  ddout[0] = 1.0f * d_sigma * softplus_prime_from_pre(fminf(fmaxf(m->acin[0], -18.0f), 18.0f));
  for (int i = 1; i < ORA_D_OUT; ++i) ddout[i] = 0.0f;

  /* color backward */
  float dc[4][ORA_M];
  fc_bwd(dc[nc - 1], dcout, ORA_C_OUT, ORA_M, P->W[L_WC_OUT]);
  for (int j = 0; j < ORA_M; ++j) dc[nc - 1][j] = unit_on(m, 3 + nc - 1, j) ? dc[nc - 1][j] : 0.0f;
  for (int k = nc - 1; k >= 1; --k) {
    fc_bwd(dc[k - 1], dc[k], ORA_M, ORA_M, P->W[cslot[k]]);
    for (int j = 0; j < ORA_M; ++j) dc[k - 1][j] = unit_on(m, 3 + k - 1, j) ? dc[k - 1][j] : 0.0f;
  }
  for (int i = 0; i < ORA_D_OUT; ++i) {
    float sacc = 0.0f;
    for (int j = 0; j < ORA_M; ++j) sacc += P->W[L_WC_IN][j * ORA_C_IN + i] * dc[0][j];
    ddout[i] += sacc;
  }
  /* density backward */
  float dd[3][ORA_M];
  fc_bwd(dd[nd - 1], ddout, ORA_D_OUT, ORA_M, P->W[L_WD_OUT]);
  for (int j = 0; j < ORA_M; ++j) dd[nd - 1][j] = unit_on(m, nd - 1, j) ? dd[nd - 1][j] : 0.0f;
  for (int k = nd - 1; k >= 1; --k) {
    fc_bwd(dd[k - 1], dd[k], ORA_M, ORA_M, P->W[dslot[k]]);
    for (int j = 0; j < ORA_M; ++j) dd[k - 1][j] = unit_on(m, k - 1, j) ? dd[k - 1][j] : 0.0f;
  }
  /* weight gradients: dW[o][i] += delta[o] * act_in[i] (weight_update.cl:260-314) */
#define ACC(slot, delta, act, od, id)                                                         \
  do {                                                                                        \
    for (int o_ = 0; o_ < (od); ++o_) {                                                       \
      double dv = (double)(delta)[o_];                                                        \
      lgb[slot][o_] += dv;                                                                    \
      for (int i_ = 0; i_ < (id); ++i_) lgW[slot][o_ * (id) + i_] += dv * (double)(act)[i_]; \
    }                                                                                         \
  } while (0)
  ACC(L_WC_OUT, dcout, m->hc[nc - 1], ORA_C_OUT, ORA_M);
  for (int k = nc - 1; k >= 1; --k) ACC(cslot[k], dc[k], m->hc[k - 1], ORA_M, ORA_M);
  ACC(L_WC_IN, dc[0], m->acin, ORA_M, ORA_C_IN);
  ACC(L_WD_OUT, ddout, m->hd[nd - 1], ORA_D_OUT, ORA_M);
  for (int k = nd - 1; k >= 1; --k) ACC(dslot[k], dd[k], m->hd[k - 1], ORA_M, ORA_M);
  ACC(L_WD_IN, dd[0], m->a0, ORA_M, LF);
#undef ACC
  /* encoding gradient and table update (ffnerf_OG.cl:2090-2173) */
  float gf[ORA_M];
  for (int k = 0; k < LF; ++k) {
    float sacc = 0.0f;
    for (int j = 0; j < ORA_M; ++j) sacc += P->W[L_WD_IN][j * LF + k] * dd[0][j];
    gf[k] = sacc;
  }
  if (gf_out) memcpy(gf_out, gf, sizeof(float) * LF);
  float p[3];
  normalize_pos(c, x, p);
  for (int l = 0; l < L; ++l) {
    uint32_t feat[8];
    float w[8];
    level_corners(c, l, p, feat, w);
    float lr_lvl = sc->lr * c->lvl_lr_scale[l];
    for (int f = 0; f < F; ++f) {
      float g = gf[l * F + f];
      if (!isfinite(g)) continue;
      for (int cc = 0; cc < 8; ++cc) {
        if (c->hash_opt == 1) {
          ORA_ATOMIC
          gtab[feat[cc] + (uint32_t)f] += (double)(g * w[cc]);
        } else if (c->table_f16) {
          ORA_ATOMIC
          gtab[feat[cc] + (uint32_t)f] += (double)(-lr_lvl * 0.5f * g * w[cc]);
        } else {
          ORA_ATOMIC
          P->table[feat[cc] + (uint32_t)f] += -lr_lvl * 0.5f * g * w[cc];
        }
      }
    }
  }
}

int ora_train_step(const ora_cfg* c, ora_params* P, const float* rays, const float* targets, float* out_rgb,
                   int32_t num_rays, int32_t S, const ora_scalars* sc, ora_debug* dbg) {
  if (S <= 0 || S > ORA_S_MAX || (S & (S - 1)) != 0) return -1;
  const int L = c->n_levels, F = c->f_per_level, LF = L * F;
  if (LF > ORA_M || c->nd < 1 || c->nd > 3 || c->nc < 1 || c->nc > 4) return -2;
  const int do_train = sc->do_train != 0;
  int64_t table_entries = 0;
  for (int l = 0; l < L; ++l) {
    int64_t e = (int64_t)c->offset[l] + ((int64_t)1 << c->log2_T[l]);
    if (e > table_entries) table_entries = e;
  }
  const int64_t table_n = table_entries * F;

  /* forward reads use the table as of the step start */
  float* table_read = (float*)malloc(sizeof(float) * (size_t)table_n);
  if (!table_read) return -3;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < table_n; ++i) table_read[i] = P->table[i];

  double* gW[L_COUNT];
  double* gb[L_COUNT];
  int odim[L_COUNT], idim[L_COUNT];
  for (int k = 0; k < L_COUNT; ++k) {
    gW[k] = NULL;
    gb[k] = NULL;
    if (!ora_layer_shape(c, k, &odim[k], &idim[k])) continue;
    gW[k] = (double*)calloc((size_t)odim[k] * idim[k], sizeof(double));
    gb[k] = (double*)calloc((size_t)odim[k], sizeof(double));
  }
  /* the summed table gradient (Adam), or for a binary16 table the summed SGD update of each entry, added once */
  const int sum_table = do_train && (c->hash_opt == 1 || c->table_f16);
  double* gtab = sum_table ? (double*)malloc(sizeof(double) * (size_t)table_n) : NULL;
  if (gtab) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < table_n; ++i) gtab[i] = 0.0;
  }

  ora_params PR = *P;
  PR.table = table_read;

  const float D = 0.5f * sqrtf((c->box_max[0] - c->box_min[0]) * (c->box_max[0] - c->box_min[0]) +
                               (c->box_max[1] - c->box_min[1]) * (c->box_max[1] - c->box_min[1]) +
                               (c->box_max[2] - c->box_min[2]) * (c->box_max[2] - c->box_min[2]));
#pragma omp parallel
  {
  mlp_state* st = (mlp_state*)malloc(sizeof(mlp_state) * (size_t)S);
  /* weight-gradient sums: the shared ones, or per thread in the OpenMP build (added together at the end) */
  double* lgW[L_COUNT];
  double* lgb[L_COUNT];
  for (int k = 0; k < L_COUNT; ++k) {
    lgW[k] = gW[k];
    lgb[k] = gb[k];
#ifdef _OPENMP
    if (gW[k]) {
      lgW[k] = (double*)calloc((size_t)odim[k] * idim[k], sizeof(double));
      lgb[k] = (double*)calloc((size_t)odim[k], sizeof(double));
    }
#endif
  }
#pragma omp for schedule(dynamic, 4)
  for (int32_t r = 0; r < num_rays; ++r) {
    const float* ray = rays + 8 * (int64_t)r;
    float Ts[ORA_S_MAX], DTs[ORA_S_MAX], Tr[ORA_S_MAX], sig[ORA_S_MAX], rgb[3 * ORA_S_MAX];
    float dLdc[3 * ORA_S_MAX], dLds[ORA_S_MAX], T_final;
    uint32_t flags[2];
    ora_sample_ray(c, ray, (uint32_t)r, S, sc->rng_seed, P->occ_in, do_train, Ts, DTs, flags);
    for (int s = 0; s < S; ++s) {
      float x[3];
      for (int i = 0; i < 3; ++i) x[i] = ray[i] + Ts[s] * ray[4 + i];
      encode_point(c, table_read, x, st[s].a0, NULL, NULL);
      const int64_t bs_ = (int64_t)r * S + s;
      mlp_forward(c, &PR, ray + 4, sc->sh_multiplier, &st[s],
                  (dbg && dbg->relu_in) ? dbg->relu_in + ORA_RELU_WORDS * bs_ : NULL);
      if (dbg && dbg->relu_out)
        for (int h = 0; h < 7; ++h) {
          dbg->relu_out[ORA_RELU_WORDS * bs_ + 2 * h] = (uint32_t)st[s].own[h];
          dbg->relu_out[ORA_RELU_WORDS * bs_ + 2 * h + 1] = (uint32_t)(st[s].own[h] >> 32);
        }
      if (dbg && dbg->preact) memcpy(dbg->preact + 7 * ORA_M * bs_, st[s].pre, sizeof(float) * 7 * ORA_M);
      sig[s] = (DTs[s] <= 0.0f) ? 0.0f : st[s].sigma;
      for (int k = 0; k < 3; ++k) rgb[3 * s + k] = st[s].rgb[k];
    }
    float* o4 = out_rgb + 4 * (int64_t)r;
    composite_ray(c, (uint32_t)r, S, sc->rng_seed, do_train, sig, rgb, DTs, targets + 4 * (int64_t)r, o4, Tr,
                  &T_final, dLdc, dLds, (dbg && dbg->C_in) ? dbg->C_in + 4 * (int64_t)r : NULL,
                  (dbg && dbg->C_out) ? dbg->C_out + 4 * (int64_t)r : NULL);
    if (sc->occ_strength > 0.0f && do_train)
      ora_occ_propose_ray(c, ray, (uint32_t)r, S, sc->rng_seed, Ts, DTs, Tr, T_final, flags, P->occ_in, P->occ_st);

    if (dbg) {
      int64_t b0 = (int64_t)r * S;
      if (dbg->Ts) memcpy(dbg->Ts + b0, Ts, sizeof(float) * S);
      if (dbg->DTs) memcpy(dbg->DTs + b0, DTs, sizeof(float) * S);
      if (dbg->flags) { dbg->flags[2 * r] = flags[0]; dbg->flags[2 * r + 1] = flags[1]; }
      if (dbg->sigma) memcpy(dbg->sigma + b0, sig, sizeof(float) * S);
      if (dbg->rgb) memcpy(dbg->rgb + 3 * b0, rgb, sizeof(float) * 3 * S);
      if (dbg->Tr) memcpy(dbg->Tr + b0, Tr, sizeof(float) * S);
      if (dbg->T_final) dbg->T_final[r] = T_final;
      if (dbg->dL_dsigma) memcpy(dbg->dL_dsigma + b0, dLds, sizeof(float) * S);
      if (dbg->dL_dc) memcpy(dbg->dL_dc + 3 * b0, dLdc, sizeof(float) * 3 * S);
      if (dbg->a0)
        for (int s = 0; s < S; ++s) memcpy(dbg->a0 + (b0 + s) * LF, st[s].a0, sizeof(float) * LF);
    }
    if (!do_train) continue;
    o4[3] += 4.0f; /* ffnerf_OG.cl:2091 */

    for (int s = 0; s < S; ++s) {
      float x[3];
      for (int i = 0; i < 3; ++i) x[i] = ray[i] + Ts[s] * ray[4 + i];
      sample_backward(c, P, sc, &st[s], x, Ts[s], DTs[s], D, dLds[s], dLdc + 3 * s, lgW, lgb, gtab,
                      (dbg && dbg->dL_da0) ? dbg->dL_da0 + ((int64_t)r * S + s) * LF : NULL);
    }
  }
#ifdef _OPENMP
#pragma omp critical
  for (int k = 0; k < L_COUNT; ++k) {
    if (!gW[k]) continue;
    for (int i = 0; i < odim[k] * idim[k]; ++i) gW[k][i] += lgW[k][i];
    for (int i = 0; i < odim[k]; ++i) gb[k][i] += lgb[k][i];
    free(lgW[k]);
    free(lgb[k]);
  }
#endif
  free(st);
  }

  if (do_train) apply_updates(c, P, sc, gW, gb, odim, idim, gtab, table_n, dbg);
  for (int k = 0; k < L_COUNT; ++k) { free(gW[k]); free(gb[k]); }
  free(gtab);
  free(table_read);
  return 0;
}

/* ------------------------------------------------------------------ */
/* R4: occupancy bitfield, DDA marcher, early-terminated render.      */
/* New in this build (the reference samples with R3 only); the        */
/* definitions below are the specification the HIP kernels follow    */
/* operation for operation.  Nearest reference analogues: the         */
/* occupancy nibble read (ffnerf_OG.cl:477-483) and the compositing   */
/* recurrence (ffnerf_OG.cl:1505-1591).                               */

typedef struct {
  int32_t res;         /* cells per axis of the bitfield */
  float dt;            /* lattice step: samples at t0 + (k + 0.5) dt */
  uint32_t max_steps;  /* emitted samples per ray at most */
  float T_stop;        /* render: stop once the transmittance drops below */
  float sh_multiplier;
} ora_march_cfg;

/* bit (x, y, z) of the (2G)^3 bitfield = (nibble q of that subcell >= q_min); bit index x + R (y + R z),
 * 32 bits per word.  Subcell (x, y, z) is nibble (x&1) | (y&1)<<1 | (z&1)<<2 of word (x>>1, y>>1, z>>1). */
void ora_occ_bitfield(const uint32_t* occ, int32_t G, uint32_t q_min, uint32_t* bits) {
  const int R = 2 * G;
  const int64_t n = (int64_t)R * R * R;
  memset(bits, 0, sizeof(uint32_t) * (size_t)((n + 31) / 32));
  for (int z = 0; z < R; ++z)
    for (int y = 0; y < R; ++y)
      for (int x = 0; x < R; ++x) {
        const uint32_t w = occ[(x >> 1) + G * ((y >> 1) + G * (z >> 1))];
        const uint32_t sub = (uint32_t)((x & 1) | ((y & 1) << 1) | ((z & 1) << 2));
        const uint32_t q = ((w >> (4u * sub)) & 0xFu) + 1u;
        if (q >= q_min) {
          const int64_t i = x + (int64_t)R * (y + (int64_t)R * z);
          bits[i >> 5] |= 1u << (i & 31);
        }
      }
}

static int bit_at(const uint32_t* bits, int R, const int c[3]) {
  const int64_t i = c[0] + (int64_t)R * (c[1] + (int64_t)R * c[2]);
  return (bits[i >> 5] >> (i & 31)) & 1u;
}

/* The march of one ray.  The cells come from a DDA that starts at the cell of o + t0 d (clamped into the
 * grid) and leaves each cell at the nearest face plane crossed, t = (bmin + (c + (d > 0)) cell - o) / d.
 * A lattice time t_k = t0 + (k + 0.5) dt belongs to the cell whose interval [t_enter, t_exit) holds it;
 * it is emitted when that cell's bit is set, until t_k >= t1 or max_steps samples.  Here every lattice
 * point is visited one by one (the brute force of the specification). */
int ora_march_ray(const ora_cfg* c, const ora_march_cfg* m, const uint32_t* bits, const float* ray, float* t_out) {
  const float* o = ray;
  const float* d = ray + 4;
  float ta, tb;
  if (!ora_ray_aabb(o, d, c->box_min, c->box_max, &ta, &tb)) return 0;
  const float t0 = fmaxf(ta, c->t_near), t1 = fminf(tb, c->t_far);
  if (!(t1 > t0)) return 0;
  const int R = m->res;
  float cell[3], inv[3], invd[3];
  int cc[3], step[3];
  for (int i = 0; i < 3; ++i) {
    const float size = c->box_max[i] - c->box_min[i];
    cell[i] = size / (float)R;
    inv[i] = (float)R / size;
    invd[i] = (d[i] != 0.0f) ? (1.0f / d[i]) : INFINITY;
    step[i] = d[i] > 0.0f ? 1 : (d[i] < 0.0f ? -1 : 0);
    const float p = o[i] + t0 * d[i];
    int ci = (int)floorf((p - c->box_min[i]) * inv[i]);
    cc[i] = ci < 0 ? 0 : (ci > R - 1 ? R - 1 : ci);
  }
  uint32_t k = 0, n = 0;
  for (int iter = 0; iter < 3 * R + 3; ++iter) {
    float t_exit = t1;
    int axis = -1;
    for (int i = 0; i < 3; ++i) {
      if (step[i] == 0) continue;
      const float bound = c->box_min[i] + (float)(cc[i] + (step[i] > 0 ? 1 : 0)) * cell[i];
      const float te = (bound - o[i]) * invd[i];
      if (te < t_exit) {
        t_exit = te;
        axis = i;
      }
    }
    const int occ = bit_at(bits, R, cc);
    for (;;) {
      const float tk = t0 + ((float)k + 0.5f) * m->dt;
      if (!(tk < t_exit)) break;
      if (occ) {
        if (n >= m->max_steps) return (int)n;
        t_out[n++] = tk;
      }
      ++k;
    }
    if (axis < 0) break;  /* the interval reached t1 */
    cc[axis] += step[axis];
    if (cc[axis] < 0 || cc[axis] >= R) break;
  }
  return (int)n;
}

/* Forward render of one ray: the marched samples in order, sigma and rgb from the MLP, front-to-back
 * compositing (alpha as in ffnerf_OG.cl:1505-1520) stopped after the first sample that leaves
 * T < T_stop; black background.  out = {r, g, b, T_final}; returns the samples evaluated. */
int ora_render_ray(const ora_cfg* c, const ora_params* P, const ora_march_cfg* m, const uint32_t* bits,
                   const float* ray, float* out) {
  float* ts = (float*)malloc(sizeof(float) * (m->max_steps ? m->max_steps : 1));
  const int n = ora_march_ray(c, m, bits, ray, ts);
  float T = 1.0f, C[3] = {0.0f, 0.0f, 0.0f};
  int used = 0;
  for (int j = 0; j < n; ++j) {
    float x[3], a0[ORA_M], sigma, rgb[3];
    for (int i = 0; i < 3; ++i) x[i] = ray[i] + ts[j] * ray[4 + i];
    ora_hash_encode(c, P->table, x, 1, a0, NULL, NULL);
    ora_mlp_forward(c, P, a0, ray + 4, m->sh_multiplier, &sigma, rgb, NULL);
    const float alpha = 1.0f - expf(fminf(fmaxf(-sigma * m->dt, -5.0f), 18.0f));
    const float w = T * alpha;
    for (int i = 0; i < 3; ++i) C[i] = C[i] + w * rgb[i];
    T = T * (1.0f - alpha);
    ++used;
    if (T < m->T_stop) break;
  }
  out[0] = C[0];
  out[1] = C[1];
  out[2] = C[2];
  out[3] = T;
  free(ts);
  return used;
}

/* ------------------------------------------------------------------ */
/* training over marched samples: the specification of                */
/* ffn_train_step_marched (no counterpart in the reference, whose     */
/* training samples every ray with S resampled points)                */

/* Compositing of one marched ray of n samples and its backward.  Front to back with
 * alpha_i = 1 - exp(clamp(-sigma_i dt, -5, 18)) (ffnerf_OG.cl:1505-1520), stopping after the sample that leaves
 * T < T_stop (or after exactly used_force samples when that is >= 0: another implementation's termination);
 * Cf = sum T_i alpha_i c_i + T_end bg; the Charbonnier gradient g at Cf (or at C_force); then back to front
 * gT_end = g.bg, dL/dsigma_i = (g.(T_i c_i) - gT_(i+1) T_i) dt (1 - alpha_i) + regu, dL/dc_i = T_i alpha_i g,
 * gT_i = g.(alpha_i c_i) + (1 - alpha_i) gT_(i+1) (ffnerf_OG.cl:1593-1634 as a sequential recurrence).  Samples
 * after the stop get no gradient and Tr = T_end.  Returns the samples composited. */
int ora_composite_marched(const float* sig, const float* rgb, int n, float dt, float T_stop, const float* bg,
                          const float* target, const float* C_force, int used_force, float regu, float* Tr,
                          float* dLds, float* dLdc, float* Cf, float* T_end) {
  float T = 1.0f, C[3] = {0.0f, 0.0f, 0.0f};
  int used = 0;
  for (int j = 0; j < n; ++j) {
    if (used_force >= 0 && j >= used_force) break;
    const float alpha = 1.0f - expf(fminf(fmaxf(-sig[j] * dt, -5.0f), 18.0f));
    Tr[j] = T;
    const float w = T * alpha;
    for (int k = 0; k < 3; ++k) C[k] = C[k] + w * rgb[3 * j + k];
    T = T * (1.0f - alpha);
    ++used;
    if (used_force < 0 && T < T_stop) break;
  }
  for (int j = used; j < n; ++j) Tr[j] = T;
  float gr[3];
  for (int k = 0; k < 3; ++k) {
    Cf[k] = C[k] + T * bg[k];
    gr[k] = charbonnier_prime((C_force ? C_force[k] : Cf[k]) - target[k]);
  }
  *T_end = T;
  float gT = gr[0] * bg[0] + gr[1] * bg[1] + gr[2] * bg[2];
  for (int j = n - 1; j >= 0; --j) {
    if (j >= used) {
      dLds[j] = 0.0f;
      dLdc[3 * j] = dLdc[3 * j + 1] = dLdc[3 * j + 2] = 0.0f;
      continue;
    }
    const float alpha = 1.0f - expf(fminf(fmaxf(-sig[j] * dt, -5.0f), 18.0f));
    const float Ti = Tr[j];
    const float* cs = rgb + 3 * j;
    const float gA = gr[0] * (Ti * cs[0]) + gr[1] * (Ti * cs[1]) + gr[2] * (Ti * cs[2]);
    const float gAlpha = gA - gT * Ti;
    dLds[j] = gAlpha * (dt * (1.0f - alpha)) + regu;
    const float ws = Ti * alpha;
    for (int k = 0; k < 3; ++k) dLdc[3 * j + k] = ws * gr[k];
    gT = (gr[0] * (alpha * cs[0]) + gr[1] * (alpha * cs[1]) + gr[2] * (alpha * cs[2])) + (1.0f - alpha) * gT;
  }
  return used;
}

/* Per ray: the march's samples (ora_march_ray), their encodings and MLP outputs, front-to-back compositing
 * with alpha = 1 - exp(clamp(-sigma dt, -5, 18)) (ffnerf_OG.cl:1505-1520) that stops after the sample leaving
 * T < T_stop, the Charbonnier loss gradient at the composited colour plus background
 * (ffnerf_OG.cl:1534-1562), and its backward as a back-to-front recurrence of dL/dT
 * (gT_i = g.(alpha_i c_i) + (1 - alpha_i) gT_(i+1), gT_end = g.bg; dL/dsigma_i = (g.(T_i c_i) - gT_(i+1) T_i)
 * dt (1 - alpha_i) + 5e-3 dt / max_steps, dL/dc_i = T_i alpha_i g: ffnerf_OG.cl:1593-1634 sequentially);
 * samples past the termination get no gradient.  Then every sample's backward (sample_backward) and the
 * parameter updates.  A step without samples leaves the table and its moments as they are (no table update
 * runs) while the MLP's Adam runs on zero gradients.  Taps index samples in march order.
 * n_used (optional) [num_rays] = samples composited; used_in (optional) [num_rays]: composite exactly that
 * many samples per ray (another implementation's termination).  With occ_strength > 0, the occupancy
 * proposals of every ray's runs (ora_occ_propose_marched_ray). */
int ora_train_step_marched(const ora_cfg* c, ora_params* P, const ora_march_cfg* m, const uint32_t* bits,
                           const float* rays, const float* targets, float* out_rgb, int32_t num_rays,
                           const ora_scalars* sc, ora_debug* dbg, const uint32_t* used_in, uint32_t* n_used) {
  const int L = c->n_levels, F = c->f_per_level, LF = L * F;
  if (LF > ORA_M || c->nd < 1 || c->nd > 3 || c->nc < 1 || c->nc > 4 || m->max_steps == 0) return -2;
  int64_t table_entries = 0;
  for (int l = 0; l < L; ++l) {
    int64_t e = (int64_t)c->offset[l] + ((int64_t)1 << c->log2_T[l]);
    if (e > table_entries) table_entries = e;
  }
  const int64_t table_n = table_entries * F;
  float* table_read = (float*)malloc(sizeof(float) * (size_t)table_n);
  if (!table_read) return -3;
  memcpy(table_read, P->table, sizeof(float) * (size_t)table_n);
  double* gW[L_COUNT];
  double* gb[L_COUNT];
  int odim[L_COUNT], idim[L_COUNT];
  for (int k = 0; k < L_COUNT; ++k) {
    gW[k] = NULL;
    gb[k] = NULL;
    if (!ora_layer_shape(c, k, &odim[k], &idim[k])) continue;
    gW[k] = (double*)calloc((size_t)odim[k] * idim[k], sizeof(double));
    gb[k] = (double*)calloc((size_t)odim[k], sizeof(double));
  }
  double* gtab = (c->hash_opt == 1 || c->table_f16) ? (double*)calloc((size_t)table_n, sizeof(double)) : NULL;
  ora_params PR = *P;
  PR.table = table_read;
  const float D = 0.5f * sqrtf((c->box_max[0] - c->box_min[0]) * (c->box_max[0] - c->box_min[0]) +
                               (c->box_max[1] - c->box_min[1]) * (c->box_max[1] - c->box_min[1]) +
                               (c->box_max[2] - c->box_min[2]) * (c->box_max[2] - c->box_min[2]));
  const float dt = m->dt;
  const float regu = 5e-3f * dt / (float)m->max_steps;
  float* ts = (float*)malloc(sizeof(float) * m->max_steps);
  mlp_state* st = (mlp_state*)malloc(sizeof(mlp_state) * m->max_steps);
  float* sig = (float*)malloc(sizeof(float) * m->max_steps);
  float* rgb = (float*)malloc(sizeof(float) * 3 * m->max_steps);
  float* Tr = (float*)malloc(sizeof(float) * m->max_steps);
  float* dLds = (float*)malloc(sizeof(float) * m->max_steps);
  float* dLdc = (float*)malloc(sizeof(float) * 3 * m->max_steps);
  int64_t base = 0;
  for (int32_t r = 0; r < num_rays; ++r) {
    const float* ray = rays + 8 * (int64_t)r;
    const int n = ora_march_ray(c, m, bits, ray, ts);
    for (int j = 0; j < n; ++j) {
      float x[3];
      for (int i = 0; i < 3; ++i) x[i] = ray[i] + ts[j] * ray[4 + i];
      encode_point(c, table_read, x, st[j].a0, NULL, NULL);
      const int64_t b = base + j;
      mlp_forward(c, &PR, ray + 4, sc->sh_multiplier, &st[j],
                  (dbg && dbg->relu_in) ? dbg->relu_in + ORA_RELU_WORDS * b : NULL);
      if (dbg && dbg->relu_out)
        for (int h = 0; h < 7; ++h) {
          dbg->relu_out[ORA_RELU_WORDS * b + 2 * h] = (uint32_t)st[j].own[h];
          dbg->relu_out[ORA_RELU_WORDS * b + 2 * h + 1] = (uint32_t)(st[j].own[h] >> 32);
        }
      if (dbg && dbg->preact) memcpy(dbg->preact + 7 * ORA_M * b, st[j].pre, sizeof(float) * 7 * ORA_M);
      if (dbg && dbg->a0) memcpy(dbg->a0 + b * LF, st[j].a0, sizeof(float) * LF);
      sig[j] = st[j].sigma;
      for (int k = 0; k < 3; ++k) rgb[3 * j + k] = st[j].rgb[k];
    }
    float bg[3] = {0.0f, 0.0f, 0.0f};
    if (c->background == 1) {
      bg[0] = bg[1] = bg[2] = 1.0f;
    } else if (c->background == 2) {
      uint32_t rr = ora_hash_u32(sc->rng_seed ^ (uint32_t)r * 747796405u ^ 0xA511E9B3u);
      bg[0] = rand01(&rr);
      bg[1] = rand01(&rr);
      bg[2] = rand01(&rr);
    }
    float Cf[3], T;
    const int used = ora_composite_marched(sig, rgb, n, dt, m->T_stop, bg, targets + 4 * (int64_t)r,
                                           (dbg && dbg->C_in) ? dbg->C_in + 4 * (int64_t)r : NULL,
                                           used_in ? (int)used_in[r] : -1, regu, Tr, dLds, dLdc, Cf, &T);
    for (int k = 0; k < 3; ++k) out_rgb[4 * (int64_t)r + k] = fminf(fmaxf(Cf[k], 0.0f), 1.0f);
    out_rgb[4 * (int64_t)r + 3] = 4.0f; /* the training output's marker (ffnerf_OG.cl:2091) */
    if (n_used) n_used[r] = (uint32_t)used;
    if (dbg) {
      if (dbg->Ts) memcpy(dbg->Ts + base, ts, sizeof(float) * n);
      if (dbg->sigma) memcpy(dbg->sigma + base, sig, sizeof(float) * n);
      if (dbg->rgb) memcpy(dbg->rgb + 3 * base, rgb, sizeof(float) * 3 * n);
      if (dbg->Tr) memcpy(dbg->Tr + base, Tr, sizeof(float) * n);
      if (dbg->T_final) dbg->T_final[r] = T;
      if (dbg->C_out)
        for (int k = 0; k < 4; ++k) dbg->C_out[4 * (int64_t)r + k] = k < 3 ? Cf[k] : 0.0f;
      if (dbg->dL_dsigma) memcpy(dbg->dL_dsigma + base, dLds, sizeof(float) * n);
      if (dbg->dL_dc) memcpy(dbg->dL_dc + 3 * base, dLdc, sizeof(float) * 3 * n);
    }
    if (sc->occ_strength > 0.0f && P->occ_st)
      ora_occ_propose_marched_ray(c, ray, (uint32_t)r, n, sc->rng_seed, ts, Tr, T, P->occ_in, P->occ_st);
    for (int j = 0; j < n; ++j) {
      float x[3];
      for (int i = 0; i < 3; ++i) x[i] = ray[i] + ts[j] * ray[4 + i];
      sample_backward(c, P, sc, &st[j], x, ts[j], dt, D, dLds[j], dLdc + 3 * j, gW, gb, gtab,
                      (dbg && dbg->dL_da0) ? dbg->dL_da0 + (base + j) * LF : NULL);
    }
    base += n;
  }
  apply_updates(c, P, sc, gW, gb, odim, idim, base > 0 ? gtab : NULL, table_n, dbg);
  for (int k = 0; k < L_COUNT; ++k) { free(gW[k]); free(gb[k]); }
  free(gtab);
  free(table_read);
  free(ts);
  free(st);
  free(sig);
  free(rgb);
  free(Tr);
  free(dLds);
  free(dLdc);
  return 0;
}
