// ffn_capi.hip -- the extern "C" boundary of libffnerf_hip.so (declared in
// include/ffnerf_hip.h).  Owns a handle per model configuration, the scratch
// buffers of one step, and the launch sequence of a training step.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <cmath>
#include <mutex>
#include <string>
#include <vector>

#include "ffn_device.h"
#include "ffn_kernels.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define FFN_HIP(call)                                                                     \
  do {                                                                                    \
    hipError_t e_ = (call);                                                               \
    if (e_ != hipSuccess) return fail(-3, "%s: %s", #call, hipGetErrorString(e_));        \
  } while (0)

struct Scratch {
  void* p = nullptr;
  size_t bytes = 0;
  hipError_t ensure(size_t need) {
    if (need <= bytes) return hipSuccess;
    if (p) {
      hipError_t e = hipFree(p);
      if (e != hipSuccess) return e;
      p = nullptr;
      bytes = 0;
    }
    hipError_t e = hipMalloc(&p, need);
    if (e != hipSuccess) return e;
    bytes = need;
    return hipSuccess;
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
};

struct StageEvent {
  int stage;
  hipEvent_t start, stop;
};

// the event recorded after the last work a call on the handle enqueued on one stream
struct StreamUse {
  hipStream_t st;
  hipEvent_t ev;
};

struct Handle {
  std::vector<StreamUse> uses;  // one per stream the handle has been used on: ffn_destroy waits for these
  bool uses_lost = false;       // an event could not be created: ffn_destroy waits for the whole device
  bool prof = false;
  std::vector<StageEvent> events;    // recorded, not yet folded into the totals
  std::vector<hipEvent_t> event_pool;  // created events free for reuse
  double stage_ms[FFN_N_STAGES] = {};
  int32_t stage_n[FFN_N_STAGES] = {};
  ffn_config cfg;
  ffn::DevCfg dc;
  ffn::PackedLayout lay;
  ffn_params params;
  bool bound = false;
  int64_t table_floats = 0;
  int n_cu = 0;
  Scratch Ts, DTs, flags, a0, dLda0, partials;
  Scratch bin_meta, bin_meta_t, bin_pairs, bin_max;
  // marcher / render
  Scratch m_state, m_acc, m_counts, m_offsets, m_sums, m_total, m_samples, m_ids, m_a0, m_sigma, m_rgb;
  // marched training
  Scratch m_Tr, m_dLds, m_dLdc;
  Scratch m_bits;  // the bitfield of ffn_train_step's march sampler
  Scratch m_blocks;  // the march's summary of the bitfield per 8^3 block, and its use flag
  Scratch m_slots;  // the marched step's per-ray sample slots (one walk instead of count + emit)
  Scratch dense;    // dense vertex copies of the coarse levels (the gather's)
  Scratch tile_sched;  // the MLP's tile order: busy flags, their scan, scan sums, total, order
  uint32_t* host_total = nullptr;  // pinned
};

// A scratch buffer may grow to `need` bytes when it is no larger than what it already holds plus half of the
// device memory free now, so that other allocations of the process (a second handle, torch's cache) keep room
bool growth_fits_free(const Scratch& held, size_t need) {
  if (need <= held.bytes) return true;
  size_t fr = 0, tot = 0;
  if (hipMemGetInfo(&fr, &tot) != hipSuccess) return true;  // unknown: let the allocation itself decide
  return need <= held.bytes + fr / 2;
}

// Pair-buffer budget of the scatter: FFN_BIN_BUDGET_MB (MiB, clamped to [64, 2^22]) when set, else 32 GiB
// limited by growth_fits_free (the levels are then split into more groups)
size_t bin_budget_bytes(bool* from_env) {
  const char* e = getenv("FFN_BIN_BUDGET_MB");
  *from_env = e != nullptr;
  long long mb = e ? atoll(e) : 32768;
  if (mb < 64) mb = 64;
  if (mb > (1ll << 22)) mb = 1ll << 22;
  return (size_t)mb << 20;
}

// Per-ray slot budget of the marched step and render: FFN_MARCH_SLOT_BUDGET_MB (MiB, default 8 GiB, limited by
// growth_fits_free; 0 walks twice)
bool march_slots_fit(const Scratch& held, size_t need) {
  const char* e = getenv("FFN_MARCH_SLOT_BUDGET_MB");
  long long mb = e ? atoll(e) : 8192;
  if (mb < 0) mb = 0;
  if (mb > (1ll << 22)) mb = 1ll << 22;
  return need <= ((size_t)mb << 20) && growth_fits_free(held, need);
}

// The gather's dense vertex copies: every level with 2 <= R and R^3 <= FFN_DENSE_MAX_CELLS (default 2^21:
// 16 MB at F = 2 in fp32) vertices gets one, filled from `table` on the stream (they follow the table, so
// they are rebuilt before every gather that follows a table update).  At the benchmark shape the row-major
// copies of levels 0-6 (res 16-111) took the gather from 5.22 to 4.61 ms (adding level 7, res 154, 4.71;
// all levels up to res 406 6.24); with levels 5-6 bricked 4.42 (level 7 bricked as well: no change).
hipError_t build_dense_levels(Handle* h, const void* table, ffn::DenseLevels* dl, hipStream_t st) {
  const char* env = getenv("FFN_DENSE_MAX_CELLS");
  const long long max_cells = env ? atoll(env) : (1ll << 21);
  const ffn::DevCfg& c = h->dc;
  const size_t elem = c.table_f16 ? 2 : 4;
  uint64_t total = 0;
  for (int l = 0; l < FFN_MAX_LEVELS; ++l) dl->off[l] = ffn::DENSE_NONE;
  dl->n_multi = 0;
  dl->bricked = 0u;
  bool leading = true;
  for (int l = 0; l < c.L; ++l) {
    const long long R = c.res[l];
    if (R >= 2 && R * R * R <= max_cells) {
      // copies of at most 2 MiB are row-major and the leading ones share one gather pass
      // (FFN_DENSE_MULTI=0: none); larger copies are bricked (4x4x4 vertices, the grid padded to whole bricks)
      const bool small = (size_t)(R * R * R) * (size_t)c.F * elem <= ((size_t)2 << 20);
      const long long NB = (R + 3) / 4;
      const long long cells = small ? R * R * R : NB * NB * NB * 64;
      dl->off[l] = (uint32_t)total;
      total += (uint64_t)((cells + 63) & ~63ll);  // each level's copy starts 256-byte aligned
      if (!small) dl->bricked |= 1u << l;
      if (leading && small) ++dl->n_multi;
      else leading = false;
    } else {
      leading = false;
    }
  }
  if (const char* m = getenv("FFN_DENSE_MULTI")) {
    if (atoi(m) == 0) dl->n_multi = 0;
  }
  dl->grid = nullptr;
  if (total == 0) {
    dl->n_multi = 0;
    return hipSuccess;
  }
  hipError_t e = h->dense.ensure((size_t)total * (size_t)c.F * elem);
  if (e != hipSuccess) return e;
  dl->grid = h->dense.p;
  return ffn::launch_hash_densify(c, table, *dl, st);
}

// size the bucketed-scatter scratch for n samples and fill the views
hipError_t ensure_bins(Handle* h, int64_t n, ffn::BinPlan* plan, ffn::BinScratch* s) {
  bool from_env = false;
  const size_t budget = bin_budget_bytes(&from_env);
  const size_t pair_bytes = 2 + 4 * (size_t)h->dc.F;
  *plan = ffn::plan_bins(h->dc, n, budget);
  if (!from_env && !growth_fits_free(h->bin_pairs, pair_bytes * (size_t)plan->max_pairs)) {
    size_t fr = 0, tot = 0;
    if (hipMemGetInfo(&fr, &tot) == hipSuccess) {
      const size_t cap = h->bin_pairs.bytes + fr / 2;
      *plan = ffn::plan_bins(h->dc, n, cap < ((size_t)64 << 20) ? ((size_t)64 << 20) : cap);
    }
  }
  hipError_t e;
  if ((e = h->bin_meta.ensure(sizeof(uint32_t) * (size_t)plan->meta_elems)) != hipSuccess) return e;
  if ((e = h->bin_meta_t.ensure(sizeof(uint32_t) * (size_t)plan->meta_elems)) != hipSuccess) return e;
  if ((e = h->bin_pairs.ensure((2 + 4 * (size_t)h->dc.F) * (size_t)plan->max_pairs)) != hipSuccess) return e;
  if ((e = h->bin_max.ensure(sizeof(float) * (size_t)plan->levels_per_group * plan->nblk)) != hipSuccess) return e;
  s->meta = (uint32_t*)h->bin_meta.p;
  s->meta_t = (uint32_t*)h->bin_meta_t.p;
  s->pairs = (uint4*)h->bin_pairs.p;
  s->cmax = (float*)h->bin_max.p;
  return hipSuccess;
}

bool is_pow2(uint32_t v) { return v && !(v & (v - 1)); }

uint32_t max_level_entries(const ffn::DevCfg& c) {
  uint32_t m = 0;
  for (int l = 0; l < c.L; ++l) m = c.mask[l] + 1 > m ? c.mask[l] + 1 : m;
  return m;
}

int validate_config(const ffn_config* c, int64_t* table_entries) {
  if (!c) return fail(-1, "config is NULL");
  if (c->n_levels < 1 || c->n_levels > FFN_MAX_LEVELS) return fail(-1, "n_levels=%d out of [1,%d]", c->n_levels, FFN_MAX_LEVELS);
  if (c->f_per_level != 1 && c->f_per_level != 2 && c->f_per_level != 4)
    return fail(-1, "f_per_level=%d unsupported (1, 2 or 4)", c->f_per_level);
  int64_t tot = 0;
  for (int l = 0; l < c->n_levels; ++l) {
    if (c->log2_T[l] < 1 || c->log2_T[l] > 26) return fail(-1, "log2_T[%d]=%u out of [1,26]", l, c->log2_T[l]);
    if (c->res[l] < 2) return fail(-1, "res[%d]=%d must be >= 2", l, c->res[l]);
    tot += (int64_t)1 << c->log2_T[l];
  }
  if (tot * c->f_per_level >= ((int64_t)1 << 32)) return fail(-1, "hash table too large for 32-bit feature indices");
  *table_entries = tot;
  if (c->nd < 1 || c->nd > 3) return fail(-1, "nd=%d out of [1,3]", c->nd);
  if (c->nc < 1 || c->nc > 4) return fail(-1, "nc=%d out of [1,4]", c->nc);
  if (c->occ_G < 1 || c->occ_G > 1024) return fail(-1, "occ_G=%d out of [1,1024]", c->occ_G);
  for (int i = 0; i < 3; ++i)
    if (!(c->box_max[i] > c->box_min[i])) return fail(-1, "box_max must exceed box_min on every axis");
  if (c->background < 0 || c->background > 2) return fail(-1, "background=%d unknown", c->background);
  if (c->hash_opt != FFN_HASH_SGD && c->hash_opt != FFN_HASH_ADAM) return fail(-1, "hash_opt=%d unknown", c->hash_opt);
  if (c->mlp_precision != FFN_MLP_FP32 && c->mlp_precision != FFN_MLP_FP16)
    return fail(-1, "mlp_precision=%d unknown", c->mlp_precision);
  if (c->table_dtype != FFN_TABLE_FP32 && c->table_dtype != FFN_TABLE_FP16)
    return fail(-1, "table_dtype=%d unknown", c->table_dtype);
  if (c->sampler != FFN_SAMPLER_RESAMPLE && c->sampler != FFN_SAMPLER_MARCH)
    return fail(-1, "sampler=%d unknown", c->sampler);
  if (c->sampler == FFN_SAMPLER_MARCH) {
    if (c->march_max_steps < 1 || c->march_max_steps > 4096)
      return fail(-1, "march_max_steps=%d out of [1,4096]", c->march_max_steps);
    if (!(c->march_dt > 0.0f)) return fail(-1, "march_dt must be > 0");
    if (!(c->march_T_stop >= 0.0f && c->march_T_stop < 1.0f)) return fail(-1, "march_T_stop must be in [0,1)");
    if (c->march_q_min < 1 || c->march_q_min > 17) return fail(-1, "march_q_min=%d out of [1,17]", c->march_q_min);
    if (2 * c->occ_G > 1024) return fail(-1, "the march's bitfield has at most 1024 cells per axis (occ_G <= 512)");
  }
  return 0;
}

ffn::DevCfg make_devcfg(const ffn_config* c) {
  ffn::DevCfg d{};
  d.L = c->n_levels;
  d.F = c->f_per_level;
  d.LF = c->n_levels * c->f_per_level;
  uint32_t off = 0;
  for (int l = 0; l < c->n_levels; ++l) {
    d.mask[l] = (1u << c->log2_T[l]) - 1u;
    d.offset[l] = off;
    off += 1u << c->log2_T[l];
    d.res[l] = c->res[l];
    d.lvl_lr_scale[l] = c->lvl_lr_scale[l];
  }
  d.nd = c->nd;
  d.nc = c->nc;
  d.G = c->occ_G;
  for (int i = 0; i < 3; ++i) {
    d.bmin[i] = c->box_min[i];
    d.bmax[i] = c->box_max[i];
    // the extent as the device computes it; its reciprocal is exact when it is a power of two
    const float bs = d.bmax[i] - d.bmin[i];
    int e = 0;
    d.inv_extent[i] = (std::isfinite(bs) && bs > 0.0f && std::frexp(bs, &e) == 0.5f) ? std::ldexp(1.0f, 1 - e) : 0.0f;
    // the occupancy grid's uniform constants, in the device code's single-precision operations
    d.inv_bs[i] = 1.0f / bs;
    d.occ_cell[i] = bs * (1.0f / (float)c->occ_G);
  }
  d.Gf = (float)c->occ_G;
  {
    const float dx = d.bmax[0] - d.bmin[0], dy = d.bmax[1] - d.bmin[1], dz = d.bmax[2] - d.bmin[2];
    d.dhalf = 0.5f * std::sqrt(dx * dx + dy * dy + dz * dz);
    d.occ_lat = std::fmax(d.occ_cell[0], 1.0e-12f);
    const float Dl = d.dhalf / d.occ_lat;
    d.occ_den = std::fmax(Dl * Dl + Dl + (1.0f / 3.0f), 1.0e-12f);
  }
  d.rho_min = c->rho_min;
  d.rho_max = c->rho_max;
  d.dt_min = c->dt_min;
  d.dt_max = c->dt_max;
  d.t_near = c->t_near;
  d.t_far = c->t_far;
  d.background = c->background;
  d.hash_opt = c->hash_opt;
  d.table_f16 = c->table_dtype == FFN_TABLE_FP16 ? 1 : 0;
  return d;
}

Handle* as_handle(void* h) { return static_cast<Handle*>(h); }

// ---- the march's scratch for callers that cannot allocate (ffn_march_noalloc) ------------------------
// The march's exclusive scan needs num_rays + 1 offsets and one partial sum per 4096 of them.  This array
// holds them for up to FFN_MARCH_NOALLOC_MAX_RAYS rays, once per GPU for the life of the process (4 MiB).
// Host code never uses the array's name as an address: the per-device address comes from
// hipGetSymbolAddress, taken once per device with that device current (at ffn_create, or at the first
// ffn_march_noalloc call on a device that has no handle).
constexpr uint64_t kNoallocScanWords = (uint64_t)FFN_MARCH_NOALLOC_MAX_RAYS + 1;
constexpr uint64_t kNoallocSumWords = (kNoallocScanWords + 4095) / 4096 + 1;
static __device__ __align__(256) uint32_t scratch[kNoallocScanWords + kNoallocSumWords];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint32_t* g_scratch_ptr[kMaxDevices] = {};

// the current device's address of `scratch` (looked up once per device); NULL with an error message
uint32_t* noalloc_scratch() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    fail(-3, "hipGetDevice: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    fail(-3, "device %d beyond the %d devices this library tracks", dev, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      fail(-3, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = static_cast<uint32_t*>(ptr);
  }
  return g_scratch_ptr[dev];
}

hipError_t take_event(Handle* h, hipEvent_t* e) {
  if (!h->event_pool.empty()) {
    *e = h->event_pool.back();
    h->event_pool.pop_back();
    return hipSuccess;
  }
  return hipEventCreate(e);
}

// Fold the oldest `count` recorded stages into the per-stage totals (waiting for each) and return their
// events to the pool.
hipError_t fold_events(Handle* h, size_t count) {
  if (count > h->events.size()) count = h->events.size();
  hipError_t err = hipSuccess;
  for (size_t i = 0; i < count; ++i) {
    StageEvent& e = h->events[i];
    float ms = 0.0f;
    hipError_t r = hipEventSynchronize(e.stop);
    if (r == hipSuccess) r = hipEventElapsedTime(&ms, e.start, e.stop);
    if (r == hipSuccess) {
      h->stage_ms[e.stage] += ms;
      h->stage_n[e.stage] += 1;
    } else if (err == hipSuccess) {
      err = r;
    }
    h->event_pool.push_back(e.start);
    h->event_pool.push_back(e.stop);
  }
  h->events.erase(h->events.begin(), h->events.begin() + (std::ptrdiff_t)count);
  return err;
}

// Brackets one stage of a step with HIP events when profiling is on.  At most kMaxPending stages wait
// unfolded, so a long profiled run holds a bounded number of events.
struct StageTimer {
  static constexpr size_t kMaxPending = 64;
  Handle* h;
  hipStream_t st;
  StageEvent ev{};
  bool on;
  StageTimer(Handle* h_, int stage, hipStream_t s) : h(h_), st(s), on(h_->prof) {
    if (!on) return;
    ev.stage = stage;
    if (take_event(h, &ev.start) != hipSuccess) {
      on = false;
      return;
    }
    if (take_event(h, &ev.stop) != hipSuccess) {
      h->event_pool.push_back(ev.start);
      on = false;
      return;
    }
    (void)hipEventRecord(ev.start, st);
  }
  ~StageTimer() {
    if (!on) return;
    (void)hipEventRecord(ev.stop, st);
    h->events.push_back(ev);
    if (h->events.size() > kMaxPending) (void)fold_events(h, h->events.size() - kMaxPending / 2);
  }
};

// Records the handle's last work on stream st (re-recording the stream's event), so that ffn_destroy waits
// for the work of this handle only, not for the device's other streams.
void note_use(Handle* h, hipStream_t st) {
  // a call captured into a graph runs when the graph is launched, not here: the caller orders those launches
  // before ffn_destroy (no event is recorded into the capture)
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) return;
  for (StreamUse& u : h->uses) {
    if (u.st == st) {
      if (hipEventRecord(u.ev, st) != hipSuccess) h->uses_lost = true;
      return;
    }
  }
  hipEvent_t ev;
  if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
    h->uses_lost = true;
    return;
  }
  h->uses.push_back(StreamUse{st, ev});
  if (hipEventRecord(ev, st) != hipSuccess) h->uses_lost = true;
}

// note_use at the end of an entry point's scope (every return path), after everything it enqueued
struct UseMark {
  Handle* h;
  hipStream_t st;
  ~UseMark() {
    if (h) note_use(h, st);
  }
};

void destroy_events(Handle* h) {
  for (auto& e : h->events) {
    (void)hipEventDestroy(e.start);
    (void)hipEventDestroy(e.stop);
  }
  h->events.clear();
  for (hipEvent_t e : h->event_pool) (void)hipEventDestroy(e);
  h->event_pool.clear();
}

}  // namespace

extern "C" {

int ffn_version(void) { return FFN_ABI_VERSION; }

const char* ffn_last_error(void) { return g_err.c_str(); }

int ffn_create(const ffn_config* cfg, void** handle) {
  if (!handle) return fail(-1, "handle out-pointer is NULL");
  *handle = nullptr;
  int64_t entries = 0;
  int rc = validate_config(cfg, &entries);
  if (rc) return rc;
  Handle* h = new Handle();
  h->cfg = *cfg;
  h->dc = make_devcfg(cfg);
  h->lay = ffn::make_layout(h->dc.LF, cfg->nd, cfg->nc);
  h->table_floats = entries * cfg->f_per_level;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&h->n_cu, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) {
    delete h;
    return fail(-3, "no HIP device: %s", hipGetErrorString(e));
  }
  // the address of this device's ffn_march_noalloc scratch, taken here rather than inside a caller's
  // no-allocation region
  if (!noalloc_scratch()) {
    delete h;
    return -3;
  }
  *handle = h;
  g_err.clear();
  return 0;
}

int ffn_destroy(void* handle) {
  Handle* h = as_handle(handle);
  if (!h) return 0;
  // the handle's buffers may still be in use by work it enqueued: wait for that work (the last call's event on
  // every stream the handle was used on) before freeing them
  if (h->uses_lost) (void)hipDeviceSynchronize();
  for (StreamUse& u : h->uses) {
    (void)hipEventSynchronize(u.ev);
    (void)hipEventDestroy(u.ev);
  }
  h->uses.clear();
  destroy_events(h);
  h->Ts.release();
  h->DTs.release();
  h->flags.release();
  h->a0.release();
  h->dLda0.release();
  h->partials.release();
  h->bin_meta.release();
  h->bin_meta_t.release();
  h->bin_pairs.release();
  h->bin_max.release();
  for (Scratch* sc : {&h->m_state, &h->m_acc, &h->m_counts, &h->m_offsets, &h->m_sums, &h->m_total, &h->m_samples,
                      &h->m_ids, &h->m_a0, &h->m_sigma, &h->m_rgb, &h->m_Tr, &h->m_dLds, &h->m_dLdc, &h->m_bits,
                      &h->m_blocks, &h->m_slots, &h->dense, &h->tile_sched})
    sc->release();
  if (h->host_total) (void)hipHostFree(h->host_total);
  delete h;
  return 0;
}

int ffn_bind_params(void* handle, const ffn_params* p) {
  Handle* h = as_handle(handle);
  if (!h || !p) return fail(-1, "NULL handle or params");
  for (int k = 0; k < FFN_N_LAYERS; ++k) {
    if (!ffn::layer_active(k, h->cfg.nd, h->cfg.nc)) continue;
    if (!p->W[k] || !p->b[k] || !p->mW[k] || !p->vW[k] || !p->mb[k] || !p->vb[k])
      return fail(-1, "layer slot %d is active but a parameter/optimizer pointer is NULL", k);
  }
  if (!p->table) return fail(-1, "table is NULL");
  if (h->cfg.hash_opt == FFN_HASH_ADAM && (!p->m_table || !p->v_table))
    return fail(-1, "FFN_HASH_ADAM needs m_table and v_table");
  if (!p->occ_in) return fail(-1, "occ_in is NULL");
  h->params = *p;
  h->bound = true;
  return 0;
}

int ffn_occ_decay(uint32_t* occ_in, uint32_t* occ_st, uint32_t n_words, uint32_t decay_q24, uint32_t iter_seed,
                  void* stream) {
  if (!occ_in || !occ_st) return fail(-1, "occupancy grids must not be NULL");
  if (decay_q24 > (1u << 24)) return fail(-1, "decay_q24=%u exceeds 2^24", decay_q24);
  FFN_HIP(ffn::launch_occ_decay(occ_in, occ_st, n_words, decay_q24, iter_seed, (hipStream_t)stream));
  return 0;
}

int ffn_adam(float* p, float* m, float* v, float* g, int64_t n, float lr_t, float beta1, float beta2, float eps,
             int32_t zero_grad, void* stream) {
  if (n < 0) return fail(-1, "negative size");
  if (n > 0 && (!p || !m || !v || !g)) return fail(-1, "NULL buffer");
  FFN_HIP(ffn::launch_adam(p, m, v, g, n, lr_t, beta1, beta2, eps, zero_grad, (hipStream_t)stream));
  return 0;
}

int ffn_sample(void* handle, const void* rays, uint32_t num_rays, uint32_t spr, uint32_t rng_seed, int32_t do_train,
               float* Ts, float* DTs, uint32_t* flags, void* stream) {
  Handle* h = as_handle(handle);
  if (!h) return fail(-1, "NULL handle");
  if (!is_pow2(spr) || spr > FFN_S_MAX) return fail(-1, "samples_per_ray=%u must be a power of two <= %d", spr, FFN_S_MAX);
  if (!rays || !Ts || !DTs || !flags) return fail(-1, "NULL buffer");
  if (!h->params.occ_in) return fail(-1, "bind params (occ_in) first");
  if (num_rays == 0) return 0;
  UseMark um{h, (hipStream_t)stream};
  FFN_HIP(ffn::launch_sample(h->dc, (const float4*)rays, num_rays, (int)spr, rng_seed, h->params.occ_in, do_train, Ts,
                             DTs, flags, (hipStream_t)stream));
  return 0;
}

int ffn_hash_encode_fwd(void* handle, const float* x, int64_t n, float* a0, uint32_t* idx_out, void* stream) {
  Handle* h = as_handle(handle);
  if (!h) return fail(-1, "NULL handle");
  if (n < 0) return fail(-1, "negative size");
  if (n > 0 && (!x || !a0)) return fail(-1, "NULL buffer");
  if (!h->params.table) return fail(-1, "bind params (table) first");
  if (n == 0) return 0;
  // the gather writes level-major (one contiguous array per level pass) into the handle's scratch, and one
  // tiled transpose makes the caller's sample-major rows: the passes would otherwise write F floats out
  // of every L * F
  const hipStream_t st = (hipStream_t)stream;
  UseMark um{h, st};
  FFN_HIP(h->a0.ensure(sizeof(float) * (size_t)n * h->dc.LF));
  const ffn::FeatLayout lm = ffn::level_major(n, h->dc.F);
  ffn::PosSrc src{x, nullptr, nullptr, 0};
  ffn::DenseLevels dl;
  FFN_HIP(build_dense_levels(h, h->params.table, &dl, st));
  FFN_HIP(ffn::launch_hash_fwd(h->dc, src, n, h->params.table, (float*)h->a0.p, lm, idx_out, &dl, st));
  FFN_HIP(ffn::launch_feat_relayout((const float*)h->a0.p, lm, a0, ffn::sample_major(h->dc.L, h->dc.F), n, h->dc.L,
                                    h->dc.F, st));
  return 0;
}

int ffn_hash_encode_bwd(void* handle, const float* x, const float* g, int64_t n, void* grad, void* stream) {
  Handle* h = as_handle(handle);
  if (!h) return fail(-1, "NULL handle");
  if (n < 0) return fail(-1, "negative size");
  if (n > 0 && (!x || !g || !grad)) return fail(-1, "NULL buffer");
  if (n == 0) return 0;
  if (!ffn::scatter_supported(h->dc))
    return fail(-2, "ffn_hash_encode_bwd: the scatter is not built for this table shape (F=%d with %u-entry levels)",
                h->dc.F, max_level_entries(h->dc));
  UseMark um{h, (hipStream_t)stream};
  ffn::BinPlan plan;
  ffn::BinScratch bs;
  FFN_HIP(ensure_bins(h, n, &plan, &bs));
  // the scatter reads one level per pass: the caller's sample-major rows are transposed to level-major
  // first (the passes would otherwise fetch every row once per level for F floats of it)
  const hipStream_t st = (hipStream_t)stream;
  FFN_HIP(h->dLda0.ensure(sizeof(float) * (size_t)n * h->dc.LF));
  const ffn::FeatLayout lm = ffn::level_major(n, h->dc.F);
  FFN_HIP(ffn::launch_feat_relayout(g, ffn::sample_major(h->dc.L, h->dc.F), (float*)h->dLda0.p, lm, n, h->dc.L,
                                    h->dc.F, st));
  ffn::PosSrc src{x, nullptr, nullptr, 0};
  ffn::BinApply ap{};
  ap.dst = grad;
  ap.dst_f16 = h->dc.table_f16;
  FFN_HIP(ffn::launch_hash_bwd(h->dc, src, n, (const float*)h->dLda0.p, lm, ffn::BIN_GRAD, 0.0f, ap, plan, bs, st));
  return 0;
}

// ffn_train_step with the march sampler: the bitfield from occ_in, then the marched step (or the render)
static int step_by_march(Handle* h, const void* rays, const void* targets, void* out_rgb, uint32_t num_rays,
                         const ffn_step_scalars* sc, const ffn_taps* taps, void* stream) {
  const int G = h->cfg.occ_G, R = 2 * G;
  const size_t words = ((size_t)R * R * R + 31) / 32;
  FFN_HIP(h->m_bits.ensure(sizeof(uint32_t) * words));
  uint32_t* bits = (uint32_t*)h->m_bits.p;
  FFN_HIP(ffn::launch_occ_bitfield(h->params.occ_in, G, (uint32_t)h->cfg.march_q_min, bits, (hipStream_t)stream));
  ffn_march_params mp{};
  mp.res = R;
  mp.dt = h->cfg.march_dt;
  mp.max_steps = (uint32_t)h->cfg.march_max_steps;
  mp.T_stop = h->cfg.march_T_stop;
  mp.chunk = 32;
  mp.sh_multiplier = sc->sh_multiplier;
  if (!sc->do_train) return ffn_render(h, rays, num_rays, bits, &mp, out_rgb, nullptr, stream);
  return ffn_train_step_marched(h, rays, targets, out_rgb, num_rays, bits, &mp, sc, taps, nullptr, stream);
}

int ffn_train_step(void* handle, const void* rays, const void* targets, void* out_rgb, uint32_t num_rays,
                   uint32_t spr, const ffn_step_scalars* sc, const ffn_taps* taps, void* stream) {
  Handle* h = as_handle(handle);
  if (!h) return fail(-1, "NULL handle");
  if (!h->bound) return fail(-1, "ffn_bind_params must be called before ffn_train_step");
  if (!sc) return fail(-1, "NULL scalars");
  if (h->cfg.sampler == FFN_SAMPLER_MARCH) return step_by_march(h, rays, targets, out_rgb, num_rays, sc, taps, stream);
  if (!is_pow2(spr) || spr > FFN_S_MAX) return fail(-1, "samples_per_ray=%u must be a power of two <= %d", spr, FFN_S_MAX);
  if (num_rays == 0) return fail(-1, "num_rays must be > 0");
  if (!rays || !out_rgb) return fail(-1, "NULL rays/out_rgb");
  const bool train = sc->do_train != 0;
  if (train && !targets) return fail(-1, "training needs targets");
  if (train && sc->occ_strength > 0.0f && !h->params.occ_st) return fail(-1, "proposals need occ_st");
  const int LF = h->dc.LF;
  const bool mlp16 = h->cfg.mlp_precision == FFN_MLP_FP16;
  if (mlp16 ? !ffn::mlp16_supported(LF, h->cfg.nd, h->cfg.nc) : !ffn::mlp_supported(LF, h->cfg.nd, h->cfg.nc))
    return fail(-2, "MLP shape LF=%d nd=%d nc=%d is not built", LF, h->cfg.nd, h->cfg.nc);
  // refused before any launch, so that a step is applied whole or not at all
  if (train && !ffn::scatter_supported(h->dc))
    return fail(-2, "ffn_train_step: the scatter is not built for this table shape (F=%d with %u-entry levels)",
                h->dc.F, max_level_entries(h->dc));
  hipStream_t st = (hipStream_t)stream;
  UseMark um{h, st};
  int log2S = 0;
  while ((1u << log2S) < spr) ++log2S;
  const int64_t N = (int64_t)num_rays * spr;
  const int64_t n_tiles = (N + 63) / 64;
  int n_blocks = (h->n_cu > 0 ? h->n_cu : 256) * (mlp16 ? ffn::mlp16_blocks_per_cu(LF, h->cfg.nd, h->cfg.nc)
                                                          : ffn::mlp_blocks_per_cu(LF, h->cfg.nd, h->cfg.nc));
  if (n_blocks > n_tiles) n_blocks = (int)n_tiles;

  FFN_HIP(h->Ts.ensure(sizeof(float) * N));
  FFN_HIP(h->DTs.ensure(sizeof(float) * N));
  FFN_HIP(h->flags.ensure(sizeof(uint32_t) * 2 * (size_t)num_rays));
  FFN_HIP(h->a0.ensure(sizeof(float) * N * LF));
  if (train) {
    FFN_HIP(h->dLda0.ensure(sizeof(float) * N * LF));
    FFN_HIP(h->partials.ensure(sizeof(float) * (size_t)n_blocks * h->lay.total));
  }
  ffn::BinPlan plan{};
  ffn::BinScratch bs{};
  if (train) FFN_HIP(ensure_bins(h, N, &plan, &bs));
  const ffn::FeatLayout feat = ffn::level_major(N, h->dc.F);
  const ffn::PosSrc src{nullptr, (const float4*)rays, nullptr, log2S};
  float* Ts = (float*)h->Ts.p;
  float* DTs = (float*)h->DTs.p;
  uint32_t* flags = (uint32_t*)h->flags.p;
  float* a0 = (float*)h->a0.p;
  float* dLda0 = (float*)h->dLda0.p;
  const ffn_params& P = h->params;

  // the MLP's tile order (below): the sampler writes the tiles' busy flags
  const size_t nt1 = (size_t)n_tiles + 1, n_sums = ((size_t)n_tiles + 4096) / 4096 + 2;
  FFN_HIP(h->tile_sched.ensure(sizeof(uint32_t) * (3 * nt1 + n_sums + 4)));
  uint32_t* tile_flags = (uint32_t*)h->tile_sched.p;
  {
    StageTimer tm(h, 0, st);
    FFN_HIP(ffn::launch_sample(h->dc, (const float4*)rays, num_rays, (int)spr, sc->rng_seed, P.occ_in,
                               train ? 1 : 0, Ts, DTs, flags, st, tile_flags));
  }
  {
    StageTimer tm(h, 1, st);
    ffn::PosSrc s2 = src;
    s2.Ts = Ts;
    ffn::DenseLevels dl;
    FFN_HIP(build_dense_levels(h, P.table, &dl, st));
    FFN_HIP(ffn::launch_hash_fwd(h->dc, s2, N, P.table, a0, feat, nullptr, &dl, st));
  }

  ffn::MlpArgs a{};
  a.c = h->dc;
  for (int k = 0; k < FFN_N_LAYERS; ++k) {
    a.w.W[k] = P.W[k];
    a.w.b[k] = P.b[k];
  }
  a.rays = (const float4*)rays;
  a.targets = (const float4*)targets;
  a.out_rgb = (float4*)out_rgb;
  a.Ts = Ts;
  a.DTs = DTs;
  a.flags = flags;
  a.a0 = a0;
  a.dL_da0 = dLda0;
  a.feat = feat;
  a.partials = (float*)h->partials.p;
  a.occ_in = P.occ_in;
  a.occ_st = P.occ_st;
  a.num_rays = num_rays;
  a.S = (int)spr;
  a.log2S = log2S;
  a.n_tiles = n_tiles;
  a.sh_mult = sc->sh_multiplier;
  a.occ_strength = sc->occ_strength;
  a.seed = sc->rng_seed;
  a.do_train = train ? 1 : 0;
  // the MLP's tile order: the busy tiles first, so that every block gets the same share of them (fp32 MLP
  // 8.41 -> 8.30 ms at the benchmark shape)
  a.tile_order = tile_flags + 2 * nt1;
  a.n_busy = tile_flags + nt1 + n_tiles;  // the scan's total (offsets[n_tiles])
  if (taps) {
    a.t_sigma = taps->sigma;
    a.t_rgb = taps->rgb;
    a.t_Tr = taps->Tr;
    a.t_Tfinal = taps->T_final;
    a.t_relu = taps->relu;
    a.t_color = (float4*)taps->color;
    a.t_dLds = taps->dL_dsigma;
    a.t_dLdc = taps->dL_dc;
  }
  {
    StageTimer tm(h, 2, st);
    FFN_HIP(ffn::launch_tile_order(n_tiles, tile_flags, tile_flags + nt1, tile_flags + 3 * nt1,
                                   tile_flags + 3 * nt1 + n_sums, const_cast<uint32_t*>(a.tile_order), st));
    if (mlp16)
      FFN_HIP(ffn::launch_mlp16(a, LF, h->cfg.nd, h->cfg.nc, n_blocks, st));
    else
      FFN_HIP(ffn::launch_mlp(a, LF, h->cfg.nd, h->cfg.nc, n_blocks, st));
  }

  if (taps) {
    if (taps->Ts) FFN_HIP(hipMemcpyAsync(taps->Ts, Ts, sizeof(float) * N, hipMemcpyDeviceToDevice, st));
    if (taps->DTs) FFN_HIP(hipMemcpyAsync(taps->DTs, DTs, sizeof(float) * N, hipMemcpyDeviceToDevice, st));
    if (taps->flags)
      FFN_HIP(hipMemcpyAsync(taps->flags, flags, sizeof(uint32_t) * 2 * num_rays, hipMemcpyDeviceToDevice, st));
    const ffn::FeatLayout sm = ffn::sample_major(h->dc.L, h->dc.F);
    if (taps->a0) FFN_HIP(ffn::launch_feat_relayout(a0, feat, taps->a0, sm, N, h->dc.L, h->dc.F, st));
    if (train && taps->dL_da0)
      FFN_HIP(ffn::launch_feat_relayout(dLda0, feat, taps->dL_da0, sm, N, h->dc.L, h->dc.F, st));
  }
  if (!train) return 0;

  {
    StageTimer tm(h, 3, st);
    ffn::PosSrc s2 = src;
    s2.Ts = Ts;
    ffn::BinApply ap{};
    ap.dst = P.table;
    ap.dst_f16 = h->dc.table_f16;
    int mode = ffn::BIN_SGD;
    if (h->cfg.hash_opt == FFN_HASH_ADAM) {
      mode = ffn::BIN_ADAM;
      ap.m = P.m_table;
      ap.v = P.v_table;
      ap.g_tap = taps ? taps->g_table : nullptr;
      ap.lr_t = sc->lr_t;
      ap.beta1 = sc->beta1;
      ap.beta2 = sc->beta2;
      ap.eps = sc->eps;
    }
    FFN_HIP(ffn::launch_hash_bwd(h->dc, s2, N, dLda0, feat, mode, sc->lr, ap, plan, bs, st));
  }

  ffn::MlpOptArgs o{};
  o.lay = h->lay;
  for (int k = 0; k < FFN_N_LAYERS; ++k) {
    o.W[k] = P.W[k];
    o.b[k] = P.b[k];
    o.mW[k] = P.mW[k];
    o.vW[k] = P.vW[k];
    o.mb[k] = P.mb[k];
    o.vb[k] = P.vb[k];
    if (taps) {
      o.gW[k] = taps->gW[k];
      o.gb[k] = taps->gb[k];
    }
  }
  o.partials = (const float*)h->partials.p;
  o.n_partials = n_blocks;
  o.lr_t = sc->lr_t;
  o.color_rel_lr = sc->color_rel_lr;
  o.beta1 = sc->beta1;
  o.beta2 = sc->beta2;
  o.eps = sc->eps;
  {
    StageTimer tm(h, 4, st);
    FFN_HIP(ffn::launch_mlp_adam(o, st));
  }

  return 0;
}

int ffn_occ_bitfield(const uint32_t* occ, int32_t occ_G, uint32_t q_min, uint32_t* bits, void* stream) {
  if (!occ || !bits) return fail(-1, "NULL buffer");
  if (occ_G < 1 || occ_G > 512) return fail(-1, "occ_G=%d out of [1,512]", occ_G);
  FFN_HIP(ffn::launch_occ_bitfield(occ, occ_G, q_min, bits, (hipStream_t)stream));
  return 0;
}

namespace {

int check_march(Handle* h, const void* rays, const uint32_t* bits, const ffn_march_params* mp) {
  if (!h) return fail(-1, "NULL handle");
  if (!rays || !bits || !mp) return fail(-1, "NULL buffer");
  if (mp->res < 1 || mp->res > 1024) return fail(-1, "march res=%d out of [1,1024]", mp->res);
  if (!(mp->dt > 0.0f)) return fail(-1, "march dt must be > 0");
  if (mp->max_steps == 0 || mp->max_steps > (1u << 20)) return fail(-1, "max_steps=%u out of [1,2^20]", mp->max_steps);
  if (mp->flags & ~FFN_RENDER_NO_WAIT) return fail(-1, "unknown march flags 0x%x", mp->flags);
  return 0;
}

ffn::MarchArgs march_args(Handle* h, const void* rays, uint32_t num_rays, const uint32_t* bits,
                          const ffn_march_params* mp) {
  ffn::MarchArgs a{};
  for (int i = 0; i < 3; ++i) {
    a.bmin[i] = h->cfg.box_min[i];
    a.bmax[i] = h->cfg.box_max[i];
  }
  a.t_near = h->cfg.t_near;
  a.t_far = h->cfg.t_far;
  a.rays = (const float4*)rays;
  a.num_rays = num_rays;
  a.bits = bits;
  a.res = mp->res;
  a.dt = mp->dt;
  a.max_steps = mp->max_steps;
  a.chunk = mp->max_steps;
  return a;
}

// The walk crosses empty 8^3 blocks in one step from a summary of the bitfield built here, on the stream, for
// this call's bitfield, when at least half the blocks are empty (decided on the device; FFN_MARCH_BLOCKS=0: no
// summary, every cell walked).  The samples are the same either way.
hipError_t set_march_blocks(Handle* h, ffn::MarchArgs& a, hipStream_t st) {
  const char* env = getenv("FFN_MARCH_BLOCKS");
  a.blocks = a.blocks_use = nullptr;
  if (env && env[0] == '0') return hipSuccess;
  const size_t NB = ((size_t)a.res + 7) / 8;
  const size_t words = (NB * NB * NB + 31) / 32;
  hipError_t e = h->m_blocks.ensure(sizeof(uint32_t) * (words + 1));
  if (e != hipSuccess) return e;
  uint32_t* b = (uint32_t*)h->m_blocks.p;
  e = ffn::launch_occ_blocks(a.bits, a.res, b, b + words, st);
  if (e == hipSuccess) {
    a.blocks = b;
    a.blocks_use = b + words;
  }
  return e;
}

}  // namespace

int ffn_march(void* handle, const void* rays, uint32_t num_rays, const uint32_t* bits, const ffn_march_params* mp,
              uint32_t* counts, uint32_t* offsets, float* samples, uint32_t* ray_ids, uint64_t capacity,
              uint32_t* total, void* stream) {
  Handle* h = as_handle(handle);
  int rc = check_march(h, rays, bits, mp);
  if (rc) return rc;
  if (!counts || !offsets || !total || (capacity > 0 && (!samples || !ray_ids))) return fail(-1, "NULL buffer");
  if (mp->sample_capacity) return fail(-1, "sample_capacity is the marched step's (the march takes `capacity`)");
  if (num_rays == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  UseMark um{h, st};
  ffn::MarchArgs a = march_args(h, rays, num_rays, bits, mp);
  FFN_HIP(set_march_blocks(h, a, st));
  a.counts = counts;
  FFN_HIP(ffn::launch_march(a, false, st));
  // offsets needs num_rays + 1 slots for the scan's total; use the handle's buffer for it
  const size_t n1 = (size_t)num_rays + 1;
  FFN_HIP(h->m_offsets.ensure(sizeof(uint32_t) * n1));
  FFN_HIP(h->m_sums.ensure(sizeof(uint32_t) * ((n1 + 4095) / 4096 + 1)));
  uint32_t* off = (uint32_t*)h->m_offsets.p;
  FFN_HIP(ffn::launch_scan_u32(counts, num_rays, off, (uint32_t*)h->m_sums.p, total, st));
  FFN_HIP(hipMemcpyAsync(offsets, off, sizeof(uint32_t) * num_rays, hipMemcpyDeviceToDevice, st));
  a.offsets = off;
  a.samples = (float4*)samples;
  a.ray_ids = ray_ids;
  a.capacity = capacity;
  FFN_HIP(ffn::launch_march(a, true, st));
  return 0;
}

int ffn_march_noalloc(void* handle, const void* rays, uint32_t num_rays, const uint32_t* bits,
                      const ffn_march_params* mp, uint32_t* counts, uint32_t* offsets, float* samples,
                      uint32_t* ray_ids, uint64_t capacity, uint32_t* total, void* stream) {
  Handle* h = as_handle(handle);
  int rc = check_march(h, rays, bits, mp);
  if (rc) return rc;
  if (!counts || !offsets || !total || (capacity > 0 && (!samples || !ray_ids))) return fail(-1, "NULL buffer");
  if (mp->sample_capacity) return fail(-1, "sample_capacity is the marched step's (the march takes `capacity`)");
  if (num_rays > FFN_MARCH_NOALLOC_MAX_RAYS)
    return fail(-1, "ffn_march_noalloc: num_rays=%u exceeds its scratch of %u rays (use ffn_march)", num_rays,
                (uint32_t)FFN_MARCH_NOALLOC_MAX_RAYS);
  if (num_rays == 0) return 0;
  uint32_t* off = noalloc_scratch();  // [num_rays + 1] offsets, then the scan's tile sums
  if (!off) return -3;
  uint32_t* sums = off + kNoallocScanWords;
  hipStream_t st = (hipStream_t)stream;
  UseMark um{h, st};
  ffn::MarchArgs a = march_args(h, rays, num_rays, bits, mp);
  a.counts = counts;
  FFN_HIP(ffn::launch_march(a, false, st));
  // every word the scan reads is written by it first (offsets, tile sums, total): nothing to clear
  FFN_HIP(ffn::launch_scan_u32(counts, num_rays, off, sums, total, st));
  FFN_HIP(hipMemcpyAsync(offsets, off, sizeof(uint32_t) * num_rays, hipMemcpyDeviceToDevice, st));
  a.offsets = off;
  a.samples = (float4*)samples;
  a.ray_ids = ray_ids;
  a.capacity = capacity;
  FFN_HIP(ffn::launch_march(a, true, st));
  return 0;
}

int ffn_train_step_marched(void* handle, const void* rays, const void* targets, void* out_rgb, uint32_t num_rays,
                           const uint32_t* bits, const ffn_march_params* mp, const ffn_step_scalars* sc,
                           const ffn_taps* taps, uint32_t* n_samples, void* stream) {
  Handle* h = as_handle(handle);
  int rc = check_march(h, rays, bits, mp);
  if (rc) return rc;
  if (!h->bound) return fail(-1, "ffn_bind_params must be called before ffn_train_step_marched");
  if (!sc || !targets || !out_rgb) return fail(-1, "NULL scalars/targets/out_rgb");
  if (num_rays == 0) return fail(-1, "num_rays must be > 0");
  if (!sc->do_train) return fail(-1, "ffn_train_step_marched trains; ffn_render is the marched forward render");
  if (sc->occ_strength > 0.0f && !h->params.occ_st) return fail(-1, "proposals need occ_st");
  if (!(mp->T_stop >= 0.0f && mp->T_stop < 1.0f)) return fail(-1, "T_stop must be in [0,1)");
  if ((uint64_t)num_rays * mp->max_steps >= ((uint64_t)1 << 32))
    return fail(-1, "num_rays * max_steps must stay below 2^32 samples");
  // sample_capacity > 0: no host wait; buffers and launches for that many samples, the count read on the device
  const uint32_t cap = mp->sample_capacity;
  if (cap > 0 && taps) return fail(-1, "taps need sample_capacity = 0 (the per-sample taps are sized on the host)");
  if ((uint64_t)cap > (uint64_t)num_rays * mp->max_steps)
    return fail(-1, "sample_capacity=%u exceeds num_rays * max_steps = %llu", cap,
                (unsigned long long)num_rays * mp->max_steps);
  const int LF = h->dc.LF;
  const bool mlp16 = h->cfg.mlp_precision == FFN_MLP_FP16;
  if (mlp16 ? !ffn::mlp16_supported(LF, h->cfg.nd, h->cfg.nc) : !ffn::mlp_supported(LF, h->cfg.nd, h->cfg.nc))
    return fail(-2, "MLP shape LF=%d nd=%d nc=%d is not built", LF, h->cfg.nd, h->cfg.nc);
  if (!ffn::scatter_supported(h->dc))
    return fail(-2, "ffn_train_step_marched: the scatter is not built for this table shape (F=%d with %u-entry "
                    "levels)", h->dc.F, max_level_entries(h->dc));
  hipStream_t st = (hipStream_t)stream;
  UseMark um{h, st};
  const ffn_params& P = h->params;

  // 1. march.  With room for max_steps samples per ray, one walk writes each ray's samples to its own slots
  // and its count; the scan of the counts sizes the step (its total comes back to the host) and a copy packs
  // the slots into the scanned order.  Otherwise the walk runs twice: count, scan, emit to the scanned slots.
  // Both give the same samples in the same order.  With a sample capacity the total stays on the device: the
  // rays past the capacity get count 0 (launch_march_clamp) and every later launch reads the kept count.
  const size_t n1 = (size_t)num_rays + 1;
  FFN_HIP(h->m_counts.ensure(sizeof(uint32_t) * n1));
  FFN_HIP(h->m_offsets.ensure(sizeof(uint32_t) * n1));
  FFN_HIP(h->m_sums.ensure(sizeof(uint32_t) * ((n1 + 4095) / 4096 + 1)));
  FFN_HIP(h->m_total.ensure(sizeof(uint32_t) * 4));
  if (!h->host_total) FFN_HIP(hipHostMalloc((void**)&h->host_total, sizeof(uint32_t) * 4, hipHostMallocDefault));
  uint32_t* counts = (uint32_t*)h->m_counts.p;
  uint32_t* off = (uint32_t*)h->m_offsets.p;
  ffn::MarchArgs ma = march_args(h, rays, num_rays, bits, mp);
  FFN_HIP(set_march_blocks(h, ma, st));
  ma.counts = counts;
  int64_t n = 0;                     // the samples (waiting) or the capacity
  const uint32_t* n_dev = nullptr;   // with a capacity: the samples kept, on the device
  {
    StageTimer tm(h, 0, st);
    const uint64_t slot_n = (uint64_t)num_rays * mp->max_steps;
    const bool one_walk = march_slots_fit(h->m_slots, slot_n * sizeof(float4));
    if (one_walk) {
      FFN_HIP(h->m_slots.ensure(sizeof(float4) * (size_t)slot_n));
      ma.slot_stride = mp->max_steps;
      ma.samples = (float4*)h->m_slots.p;
      ma.ray_ids = nullptr;
      ma.capacity = slot_n;
      FFN_HIP(ffn::launch_march(ma, true, st));
    } else {
      FFN_HIP(ffn::launch_march(ma, false, st));
    }
    FFN_HIP(ffn::launch_scan_u32(counts, num_rays, off, (uint32_t*)h->m_sums.p, (uint32_t*)h->m_total.p, st));
    if (cap > 0) {
      uint32_t* kept = (uint32_t*)h->m_total.p + 1;
      FFN_HIP(ffn::launch_march_clamp(counts, off, num_rays, cap, kept, st));
      n = cap;
      n_dev = kept;
    } else {
      FFN_HIP(hipMemcpyAsync(h->host_total, h->m_total.p, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
      FFN_HIP(hipStreamSynchronize(st));
      n = *h->host_total;
    }
    FFN_HIP(h->m_samples.ensure(sizeof(float4) * (size_t)(n > 0 ? n : 1)));
    FFN_HIP(h->m_ids.ensure(sizeof(uint32_t) * (size_t)(n > 0 ? n : 1)));
    if (one_walk) {
      FFN_HIP(ffn::launch_march_compact(counts, off, (const float4*)h->m_slots.p, mp->max_steps, num_rays,
                                        (float4*)h->m_samples.p, (uint32_t*)h->m_ids.p, st));
    } else {
      ma.offsets = off;
      ma.samples = (float4*)h->m_samples.p;
      ma.ray_ids = (uint32_t*)h->m_ids.p;
      ma.capacity = (uint64_t)n;
      FFN_HIP(ffn::launch_march(ma, true, st));
    }
  }
  const float4* smp = (const float4*)h->m_samples.p;
  const uint32_t* ids = (const uint32_t*)h->m_ids.p;
  const size_t nz = (size_t)(n > 0 ? n : 1);
  FFN_HIP(h->a0.ensure(sizeof(float) * nz * LF));
  FFN_HIP(h->dLda0.ensure(sizeof(float) * nz * LF));
  FFN_HIP(h->m_sigma.ensure(sizeof(float) * nz));
  FFN_HIP(h->m_rgb.ensure(sizeof(float) * nz * 3));
  FFN_HIP(h->m_Tr.ensure(sizeof(float) * nz));
  FFN_HIP(h->m_dLds.ensure(sizeof(float) * nz));
  FFN_HIP(h->m_dLdc.ensure(sizeof(float) * nz * 3));
  float* a0 = (float*)h->a0.p;
  float* dLda0 = (float*)h->dLda0.p;
  float* sigma = (float*)h->m_sigma.p;
  float* rgb = (float*)h->m_rgb.p;
  const ffn::FeatLayout feat = ffn::level_major(n, h->dc.F);
  ffn::PosSrc src{(const float*)smp, nullptr, nullptr, 0};
  src.x_stride = 4;

  // 2. encode the samples
  {
    StageTimer tm(h, 1, st);
    ffn::DenseLevels dl;
    FFN_HIP(build_dense_levels(h, P.table, &dl, st));
    FFN_HIP(ffn::launch_hash_fwd(h->dc, src, n, P.table, a0, feat, nullptr, &dl, st, n_dev));
  }
  // 3-5. forward MLP, compositing with early termination and the loss, MLP backward.  (With a capacity the
  // blocks are those of the capacity's tiles: a block's tiles and the order of the partials' sum are the same
  // as for the kept count, the further blocks add zero partials.)
  const int64_t n_tiles = (n + 63) / 64;
  int n_blocks = (h->n_cu > 0 ? h->n_cu : 256) * (mlp16 ? ffn::mlp16_blocks_per_cu(LF, h->cfg.nd, h->cfg.nc)
                                                         : ffn::mlp_blocks_per_cu(LF, h->cfg.nd, h->cfg.nc));
  if (n_blocks > n_tiles) n_blocks = (int)(n_tiles > 0 ? n_tiles : 1);
  FFN_HIP(h->partials.ensure(sizeof(float) * (size_t)n_blocks * h->lay.total));
  ffn::MlpPtrs w{};
  for (int k = 0; k < FFN_N_LAYERS; ++k) {
    w.W[k] = P.W[k];
    w.b[k] = P.b[k];
  }
  {
    StageTimer tm(h, 2, st);
    if (mlp16)
      FFN_HIP(ffn::launch_mlp16_fwd(h->dc, w, a0, feat, (const float4*)rays, ids, n, sc->sh_multiplier, sigma, rgb,
                                    LF, h->cfg.nd, h->cfg.nc, n_blocks, st, n_dev));
    else
      FFN_HIP(ffn::launch_mlp_fwd(h->dc, w, a0, feat, (const float4*)rays, ids, n, sc->sh_multiplier, sigma, rgb,
                                  LF, h->cfg.nd, h->cfg.nc, n_blocks, st, n_dev));
    ffn::CompMarchArgs ca{};
    ca.offsets = off;
    ca.counts = counts;
    ca.num_rays = num_rays;
    ca.sigma = sigma;
    ca.rgb = rgb;
    ca.targets = (const float4*)targets;
    ca.dt = mp->dt;
    ca.T_stop = mp->T_stop;
    ca.regu = 5e-3f * mp->dt / (float)mp->max_steps;
    ca.background = h->cfg.background;
    ca.seed = sc->rng_seed;
    ca.out_rgb = (float4*)out_rgb;
    ca.Tr = (float*)h->m_Tr.p;
    ca.dLds = (float*)h->m_dLds.p;
    ca.dLdc = (float*)h->m_dLdc.p;
    ca.n_used = n_samples;
    ca.T_final = taps ? taps->T_final : nullptr;
    ca.color = taps ? (float4*)taps->color : nullptr;
    ca.c = h->dc;
    ca.rays = (const float4*)rays;
    ca.samples = smp;
    ca.occ_in = P.occ_in;
    ca.occ_st = sc->occ_strength > 0.0f ? P.occ_st : nullptr;
    FFN_HIP(ffn::launch_composite_marched(ca, st));
    ffn::MlpArgs a{};
    a.c = h->dc;
    a.w = w;
    a.rays = (const float4*)rays;
    a.a0 = a0;
    a.dL_da0 = dLda0;
    a.feat = feat;
    a.partials = (float*)h->partials.p;
    a.num_rays = (uint32_t)n;  // one "ray" per sample: the kernel walks n samples in tiles of 64
    a.S = 1;
    a.log2S = 0;
    a.n_tiles = n_tiles;
    a.sh_mult = sc->sh_multiplier;
    a.occ_strength = 0.0f;
    a.seed = sc->rng_seed;
    a.do_train = 1;
    a.smp = smp;
    a.ray_ids = ids;
    a.in_dLds = ca.dLds;
    a.in_dLdc = ca.dLdc;
    a.march_dt = mp->dt;
    a.n_dev = n_dev;
    if (taps) a.t_relu = taps->relu;
    if (n > 0 && mlp16) FFN_HIP(ffn::launch_mlp16_marched(a, LF, h->cfg.nd, h->cfg.nc, n_blocks, st));
    else if (n > 0) FFN_HIP(ffn::launch_mlp_marched(a, LF, h->cfg.nd, h->cfg.nc, n_blocks, st));
    else FFN_HIP(ffn::launch_fill((float*)h->partials.p, h->lay.total, 0.0f, st));
  }
  if (taps) {
    if (taps->sigma) FFN_HIP(hipMemcpyAsync(taps->sigma, sigma, sizeof(float) * n, hipMemcpyDeviceToDevice, st));
    if (taps->rgb) FFN_HIP(hipMemcpyAsync(taps->rgb, rgb, sizeof(float) * 3 * n, hipMemcpyDeviceToDevice, st));
    if (taps->Tr) FFN_HIP(hipMemcpyAsync(taps->Tr, h->m_Tr.p, sizeof(float) * n, hipMemcpyDeviceToDevice, st));
    if (taps->dL_dsigma)
      FFN_HIP(hipMemcpyAsync(taps->dL_dsigma, h->m_dLds.p, sizeof(float) * n, hipMemcpyDeviceToDevice, st));
    if (taps->dL_dc)
      FFN_HIP(hipMemcpyAsync(taps->dL_dc, h->m_dLdc.p, sizeof(float) * 3 * n, hipMemcpyDeviceToDevice, st));
    const ffn::FeatLayout sm = ffn::sample_major(h->dc.L, h->dc.F);
    if (taps->a0) FFN_HIP(ffn::launch_feat_relayout(a0, feat, taps->a0, sm, n, h->dc.L, h->dc.F, st));
    if (taps->dL_da0) FFN_HIP(ffn::launch_feat_relayout(dLda0, feat, taps->dL_da0, sm, n, h->dc.L, h->dc.F, st));
  }
  // 6. the table update from the samples' encoding gradients
  {
    StageTimer tm(h, 3, st);
    ffn::BinPlan plan{};
    ffn::BinScratch bs{};
    FFN_HIP(ensure_bins(h, n > 0 ? n : 1, &plan, &bs));
    ffn::BinApply ap{};
    ap.dst = P.table;
    ap.dst_f16 = h->dc.table_f16;
    int mode = ffn::BIN_SGD;
    if (h->cfg.hash_opt == FFN_HASH_ADAM) {
      mode = ffn::BIN_ADAM;
      ap.m = P.m_table;
      ap.v = P.v_table;
      ap.g_tap = taps ? taps->g_table : nullptr;
      ap.lr_t = sc->lr_t;
      ap.beta1 = sc->beta1;
      ap.beta2 = sc->beta2;
      ap.eps = sc->eps;
    }
    // with no samples nothing runs: the table and its moments stay as they are
    FFN_HIP(ffn::launch_hash_bwd(h->dc, src, n, dLda0, feat, mode, sc->lr, ap, plan, bs, st, n_dev));
  }
  // 7. MLP Adam
  ffn::MlpOptArgs o{};
  o.lay = h->lay;
  for (int k = 0; k < FFN_N_LAYERS; ++k) {
    o.W[k] = P.W[k];
    o.b[k] = P.b[k];
    o.mW[k] = P.mW[k];
    o.vW[k] = P.vW[k];
    o.mb[k] = P.mb[k];
    o.vb[k] = P.vb[k];
    if (taps) {
      o.gW[k] = taps->gW[k];
      o.gb[k] = taps->gb[k];
    }
  }
  o.partials = (const float*)h->partials.p;
  o.n_partials = n_blocks;
  o.lr_t = sc->lr_t;
  o.color_rel_lr = sc->color_rel_lr;
  o.beta1 = sc->beta1;
  o.beta2 = sc->beta2;
  o.eps = sc->eps;
  {
    StageTimer tm(h, 4, st);
    FFN_HIP(ffn::launch_mlp_adam(o, st));
  }
  return 0;
}

int ffn_render(void* handle, const void* rays, uint32_t num_rays, const uint32_t* bits, const ffn_march_params* mp,
               void* out_rgb, uint32_t* n_samples, void* stream) {
  Handle* h = as_handle(handle);
  int rc = check_march(h, rays, bits, mp);
  if (rc) return rc;
  if (!out_rgb) return fail(-1, "NULL buffer");
  if (!h->bound) return fail(-1, "bind params first");
  if (mp->chunk == 0 || mp->chunk > 1024) return fail(-1, "chunk=%u out of [1,1024]", mp->chunk);
  if (!(mp->T_stop >= 0.0f && mp->T_stop < 1.0f)) return fail(-1, "T_stop must be in [0,1)");
  if (mp->sample_capacity) return fail(-1, "sample_capacity is the marched step's (the render sizes its rounds)");
  if (num_rays == 0) return 0;
  hipStream_t st = (hipStream_t)stream;
  UseMark um{h, st};
  const bool no_wait = (mp->flags & FFN_RENDER_NO_WAIT) != 0;
  const int LF = h->dc.LF;
  const size_t n1 = (size_t)num_rays + 1;
  const size_t cap = (size_t)num_rays * mp->chunk;
  if (no_wait && cap >= ((size_t)1 << 32)) return fail(-1, "num_rays * chunk must stay below 2^32 samples");
  FFN_HIP(h->m_state.ensure(sizeof(ffn::MarchState) * num_rays));
  FFN_HIP(h->m_acc.ensure(sizeof(float4) * num_rays));
  FFN_HIP(h->m_counts.ensure(sizeof(uint32_t) * n1));
  FFN_HIP(h->m_offsets.ensure(sizeof(uint32_t) * n1));
  FFN_HIP(h->m_sums.ensure(sizeof(uint32_t) * ((n1 + 4095) / 4096 + 1)));
  FFN_HIP(h->m_total.ensure(sizeof(uint32_t) * 4));
  FFN_HIP(h->m_samples.ensure(sizeof(float4) * cap));
  FFN_HIP(h->m_ids.ensure(sizeof(uint32_t) * cap));
  FFN_HIP(h->m_a0.ensure(sizeof(float) * cap * LF));
  FFN_HIP(h->m_sigma.ensure(sizeof(float) * cap));
  FFN_HIP(h->m_rgb.ensure(sizeof(float) * cap * 3));
  if (!h->host_total) FFN_HIP(hipHostMalloc((void**)&h->host_total, sizeof(uint32_t) * 4, hipHostMallocDefault));
  ffn::MarchState* state = (ffn::MarchState*)h->m_state.p;
  float4* acc = (float4*)h->m_acc.p;
  uint32_t* counts = (uint32_t*)h->m_counts.p;
  uint32_t* off = (uint32_t*)h->m_offsets.p;
  uint32_t* total = (uint32_t*)h->m_total.p;
  float4* samples = (float4*)h->m_samples.p;
  uint32_t* ids = (uint32_t*)h->m_ids.p;
  float* a0 = (float*)h->m_a0.p;
  float* sigma = (float*)h->m_sigma.p;
  float* rgb = (float*)h->m_rgb.p;
  // without waits, the scan's total is each round's sample count on the device and the gate of the next round's
  // launches (primed open here): a round after one without samples does nothing
  FFN_HIP(ffn::launch_march_init(state, acc, n_samples, num_rays, st, no_wait ? total : nullptr));
  ffn::MarchArgs a = march_args(h, rays, num_rays, bits, mp);
  FFN_HIP(set_march_blocks(h, a, st));
  a.chunk = mp->chunk;
  a.state = state;
  a.counts = counts;
  a.offsets = off;
  a.samples = samples;
  a.ray_ids = ids;
  a.capacity = cap;
  ffn::MlpPtrs w{};
  for (int k = 0; k < FFN_N_LAYERS; ++k) {
    w.W[k] = h->params.W[k];
    w.b[k] = h->params.b[k];
  }
  // Each round walks every live ray once into its own chunk of slots (its count and walk state written by the
  // same pass), then packs the slots into the scanned order; without room for the slots (the budget of the
  // marched step) it walks twice, count then emit.  The samples, their order and the walk states agree.
  const bool one_walk = march_slots_fit(h->m_slots, cap * sizeof(float4));
  if (one_walk) FFN_HIP(h->m_slots.ensure(sizeof(float4) * cap));
  if (no_wait) a.gate = total;
  ffn::MarchArgs a1 = a;
  a1.slot_stride = mp->chunk;
  a1.samples = (float4*)h->m_slots.p;
  a1.ray_ids = nullptr;
  int n_blocks = h->n_cu > 0 ? 2 * h->n_cu : 512;
  const uint32_t rounds = (mp->max_steps + mp->chunk - 1) / mp->chunk;
  ffn::DenseLevels dl;  // the table does not change during the render: one copy serves every round
  FFN_HIP(build_dense_levels(h, h->params.table, &dl, st));
  // (without waits: the round's count is *total, read on the device; n the capacity)
  const uint32_t* n_dev = no_wait ? total : nullptr;
  for (uint32_t round = 0; round < rounds; ++round) {
    FFN_HIP(ffn::launch_march(one_walk ? a1 : a, one_walk, st));
    FFN_HIP(ffn::launch_scan_u32(counts, num_rays, off, (uint32_t*)h->m_sums.p, total, st, no_wait));
    int64_t n = (int64_t)cap;
    if (!no_wait) {
      FFN_HIP(hipMemcpyAsync(h->host_total, total, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
      FFN_HIP(hipStreamSynchronize(st));
      n = *h->host_total;
      if (n == 0) break;
    }
    if (one_walk) {
      FFN_HIP(ffn::launch_march_compact(counts, off, (const float4*)h->m_slots.p, mp->chunk, num_rays, samples, ids,
                                        st, n_dev));
    } else {
      FFN_HIP(ffn::launch_march(a, true, st));
    }
    ffn::PosSrc src{(const float*)samples, nullptr, nullptr, 0};
    src.x_stride = 4;
    const ffn::FeatLayout feat = ffn::level_major(n, h->dc.F);
    FFN_HIP(ffn::launch_hash_fwd(h->dc, src, n, h->params.table, a0, feat, nullptr, &dl, st, n_dev));
    int nb = (int)((n + 63) / 64);
    if (nb > n_blocks) nb = n_blocks;
    FFN_HIP(ffn::launch_mlp_fwd(h->dc, w, a0, feat, (const float4*)rays, ids, n, mp->sh_multiplier, sigma, rgb, LF,
                                h->cfg.nd, h->cfg.nc, nb, st, n_dev));
    FFN_HIP(ffn::launch_render_composite(off, counts, num_rays, sigma, rgb, mp->dt, mp->T_stop, state, acc,
                                         n_samples, st, n_dev));
  }
  FFN_HIP(ffn::launch_render_finish(acc, num_rays, (float4*)out_rgb, st));
  return 0;
}

int ffn_make_batch(const float* images, uint32_t n_images, uint32_t width, uint32_t height, const float* c2w,
                   const float* K, uint32_t num_rays, uint32_t seed, void* rays, void* targets, uint32_t* pixel_ids,
                   void* stream) {
  if (!images || !c2w || !K || !rays || !targets) return fail(-1, "NULL buffer");
  if (n_images == 0 || width == 0 || height == 0) return fail(-1, "empty image set");
  if ((uint64_t)n_images * width * height >= ((uint64_t)1 << 32)) return fail(-1, "more than 2^32 - 1 pixels");
  FFN_HIP(ffn::launch_make_batch(images, n_images, width, height, c2w, K, num_rays, seed, (float4*)rays,
                                 (float4*)targets, pixel_ids, (hipStream_t)stream));
  return 0;
}

int ffn_make_batch_weighted(const float* images, uint32_t n_images, uint32_t width, uint32_t height,
                            const float* c2w, const float* K, const uint8_t* weights, uint32_t num_rays,
                            uint32_t uniform_rays, uint32_t max_tries, uint32_t seed, void* rays, void* targets,
                            uint32_t* pixel_ids, void* stream) {
  if (!images || !c2w || !K || !weights || !rays || !targets) return fail(-1, "NULL buffer");
  if (n_images == 0 || width == 0 || height == 0) return fail(-1, "empty image set");
  if ((uint64_t)n_images * width * height >= ((uint64_t)1 << 32)) return fail(-1, "more than 2^32 - 1 pixels");
  if (uniform_rays > num_rays) return fail(-1, "uniform_rays=%u exceeds num_rays=%u", uniform_rays, num_rays);
  if (max_tries == 0 || max_tries > (1u << 20)) return fail(-1, "max_tries=%u out of [1,2^20]", max_tries);
  FFN_HIP(ffn::launch_make_batch_weighted(images, n_images, width, height, c2w, K, weights, num_rays, uniform_rays,
                                          max_tries, seed, (float4*)rays, (float4*)targets, pixel_ids,
                                          (hipStream_t)stream));
  return 0;
}

int ffn_set_profiling(void* handle, int32_t enable) {
  Handle* h = as_handle(handle);
  if (!h) return fail(-1, "NULL handle");
  h->prof = enable != 0;
  return 0;
}

int ffn_stage_times(void* handle, float* total_ms, int32_t* launches, int32_t reset) {
  Handle* h = as_handle(handle);
  if (!h || !total_ms || !launches) return fail(-1, "NULL argument");
  FFN_HIP(fold_events(h, h->events.size()));
  for (int i = 0; i < FFN_N_STAGES; ++i) {
    total_ms[i] = (float)h->stage_ms[i];
    launches[i] = h->stage_n[i];
    if (reset) {
      h->stage_ms[i] = 0.0;
      h->stage_n[i] = 0;
    }
  }
  return 0;
}

}  // extern "C"
