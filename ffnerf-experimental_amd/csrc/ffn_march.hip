// ffn_march.hip -- occupancy bitfield, DDA marcher with stream compaction, and
// the early-terminated front-to-back compositing of the forward render.
//
// The reference has no marcher: every ray gets S importance-resampled samples
// (ffnerf_OG.cl:1002-1250).  This path is new; its specification is the CPU
// definition in the oracle (ora_occ_bitfield, ora_march_ray, ora_render_ray),
// which these kernels follow operation for operation (no contraction), so the
// marched sample times are bit-identical.  Nearest reference analogues: the
// occupancy nibble read (ffnerf_OG.cl:477-483) and the compositing recurrence
// (ffnerf_OG.cl:1505-1591).
//
// MI355X design
//   * The bitfield holds one bit per cell (x fastest, 32 cells per word):
//     128^3 cells = 256 KiB, 256^3 = 2 MiB -- resident in each XCD's L2, so the
//     DDA's bit lookups never reach HBM after the first touch.
//   * One lane per ray.  Empty cells are skipped in one step: the first lattice
//     index past the cell's exit is computed directly and corrected to the exact
//     index the one-by-one walk of the specification reaches.
//   * Empty 8^3 blocks are crossed in one step: a summary (one bit per block,
//     4 KiB at 256^3) marks the blocks with any occupied cell, and in an empty
//     block the walk moves straight to the first cell past the block -- the
//     same cell, lattice index and step count the one-cell-at-a-time walk
//     reaches, because every crossing of a cell boundary is an event ordered
//     by (time, axis) and the block's first face event and the interior events
//     before it follow from the same boundary-time formula.  A jump costs
//     several cell steps and diverges from the lanes that step cells, so the
//     walk uses the summary only when at least half the blocks are empty (a
//     flag computed on the device with it): a field with isolated occupied
//     cells scattered everywhere, where nearly every block holds one, walks
//     cell by cell.
//   * Compaction: one walk writes each ray's samples to its own fixed run of
//     slots (max_steps, or the chunk, per ray) and its count; a scan of the
//     counts and a wavefront-per-ray copy pack them.  Where those slots do not
//     fit, two passes over the same deterministic walk: count, scan, emit to the
//     scanned slots.  A chunked variant keeps a 16-byte state per
//     ray so that the render can march, shade and composite a few samples per
//     ray per round and retire rays whose transmittance fell below T_stop.
#include "ffn_device.h"
#include "ffn_kernels.h"

namespace ffn {

__global__ __launch_bounds__(256) void k_occ_bitfield(const uint32_t* __restrict__ occ, int G, uint32_t q_min,
                                                      uint32_t* __restrict__ bits, int64_t n_words) {
  const int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= n_words) return;
  const int R = 2 * G;
  const int64_t n_cells = (int64_t)R * R * R;
  uint32_t out = 0;
  for (int j = 0; j < 32; ++j) {
    const int64_t i = w * 32 + j;
    if (i >= n_cells) break;
    const int x = (int)(i % R), y = (int)((i / R) % R), z = (int)(i / ((int64_t)R * R));
    const uint32_t word = occ[(x >> 1) + G * ((y >> 1) + G * (z >> 1))];
    const uint32_t sub = (uint32_t)((x & 1) | ((y & 1) << 1) | ((z & 1) << 2));
    const uint32_t q = ((word >> (4u * sub)) & 0xFu) + 1u;
    if (q >= q_min) out |= 1u << j;
  }
  bits[w] = out;
}

// Block summary: bit (bx + NB (by + NB bz)) of `blocks` is set when any cell of the 8^3 block (bx, by, bz) is
// occupied (NB = ceil(R / 8); the last block of an axis is partial when 8 does not divide R).  One lane per
// block, 64 blocks (two words) per wavefront.
__global__ __launch_bounds__(256) void k_occ_blocks(const uint32_t* __restrict__ bits, int R,
                                                    uint32_t* __restrict__ blocks, int64_t n_blocks) {
  constexpr int B = 8;
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int NB = (R + B - 1) / B;
  bool any = false;
  if (b < n_blocks) {
    const int bx = (int)(b % NB), by = (int)((b / NB) % NB), bz = (int)(b / ((int64_t)NB * NB));
    const int x0 = B * bx, n = (R - x0 < B ? R - x0 : B);
    const uint32_t mask = (1u << n) - 1u;
    const int y1 = (B * by + B < R ? B * by + B : R), z1 = (B * bz + B < R ? B * bz + B : R);
    uint32_t acc = 0;
    for (int z = B * bz; z < z1; ++z)
      for (int y = B * by; y < y1; ++y) {
        const int64_t i0 = x0 + (int64_t)R * (y + (int64_t)R * z);
        const uint32_t sh = (uint32_t)(i0 & 31);
        uint32_t w = bits[i0 >> 5] >> sh;
        if (sh + (uint32_t)n > 32u) w |= bits[(i0 >> 5) + 1] << (32u - sh);
        acc |= w & mask;
      }
    any = acc != 0;
  }
  const uint64_t bal = __ballot(any);
  const int lane = threadIdx.x & 63;
  const int64_t w0 = (b - lane) >> 5;  // the wavefront's first word (64 blocks, 64-aligned)
  const int64_t n_words = (n_blocks + 31) >> 5;
  if (lane == 0 && w0 < n_words) blocks[w0] = (uint32_t)bal;
  if (lane == 32 && w0 + 1 < n_words) blocks[w0 + 1] = (uint32_t)(bal >> 32);
}

// *use = 1 when at least half of the n_blocks summary bits are clear (one workgroup; fixed-order sum)
__global__ __launch_bounds__(256) void k_blocks_use(const uint32_t* __restrict__ blocks, int64_t n_blocks,
                                                    uint32_t* __restrict__ use) {
  __shared__ uint32_t part[256];
  const int64_t n_words = (n_blocks + 31) >> 5;
  uint32_t c = 0;
  for (int64_t w = threadIdx.x; w < n_words; w += 256) c += (uint32_t)__popc(blocks[w]);
  part[threadIdx.x] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t t = 0;
    for (int i = 0; i < 256; ++i) t += part[i];
    use[0] = 2 * t <= (uint64_t)n_blocks ? 1u : 0u;
  }
}

__device__ __forceinline__ float lattice_t(float t0, uint32_t k, float dt) { return t0 + ((float)k + 0.5f) * dt; }

// the first lattice index k' >= k with t_k' >= t_exit, as the one-cell-at-a-time walk reaches it
__device__ __forceinline__ uint32_t skip_lattice(float t0, uint32_t k, float dt, float t_exit) {
  if (!(lattice_t(t0, k, dt) < t_exit)) return k;
  float est = ceilf((t_exit - t0) / dt - 0.5f);
  uint32_t ke = k + 1;
  if (est > (float)ke) ke = est < 4.0e9f ? (uint32_t)est : 4000000000u;
  while (ke > k + 1 && !(lattice_t(t0, ke - 1, dt) < t_exit)) --ke;
  while (lattice_t(t0, ke, dt) < t_exit) ++ke;
  return ke;
}

// Rays per wavefront of k_march.  A lane walks one ray at a time and, when that ray is finished (or paused at
// the chunk budget), takes the next unclaimed ray of its wavefront's range: walks are 37 % as long as
// their wavefront's longest on average, so a lane per ray would leave most lanes idle.
constexpr uint32_t MARCH_RPW = 256;
constexpr int MARCH_CELLS_PER_CLAIM = 8;

// One lane's walk of one ray, advanced a cell at a time.  The sequence of operations per ray is the
// specification's (ora_march_ray): the same cells, exit times and lattice indices, so the emitted samples
// are bit-identical whatever order the lane meets its rays in.
template <bool EMIT>
struct RayWalk {
  MarchState st;
  float o[3], d[3], invd[3], t0, t1;
  int cc[3], step[3];
  uint32_t r, k, emitted;
  uint64_t base;
  int iter;
  // Exit time of the last empty cell walked, not yet applied to k.  The one-cell-at-a-time walk moves k past
  // every empty cell's exit time; those times never decrease along the walk and k' = first index >= k with
  // t_k' >= t is the same whether applied once per cell or once for the last cell of a run, so k is brought up
  // to date only where it is used: on entering an occupied cell and when the walk state is saved.
  float t_pend;
  bool done, paused;

  // claim ray rr; returns false when the ray has nothing to walk (it is then already finished)
  __device__ __forceinline__ bool start(const MarchArgs& a, uint32_t rr, const float (&cell)[3]) {
    r = rr;
    emitted = 0;
    iter = 0;
    t_pend = -__builtin_huge_valf();
    done = false;
    paused = false;
    st = a.state ? a.state[r] : MarchState{0u, 0u, 0u, MARCH_FRESH};
    if (st.flags & MARCH_DONE) return false;  // no state change, no samples
    const float4 ro = a.rays[2 * (size_t)r], rd = a.rays[2 * (size_t)r + 1];
    o[0] = ro.x; o[1] = ro.y; o[2] = ro.z;
    d[0] = rd.x; d[1] = rd.y; d[2] = rd.z;
    base = EMIT ? (a.slot_stride ? (uint64_t)r * a.slot_stride : (uint64_t)a.offsets[r]) : 0;
    float ta, tb;
    if (!ray_aabb(o, d, a.bmin, a.bmax, ta, tb)) {
      done = true;
      finish_state(a, false);
      return false;
    }
    t0 = fmaxf(ta, a.t_near);
    t1 = fminf(tb, a.t_far);
    if (!(t1 > t0)) {
      done = true;
      finish_state(a, false);
      return false;
    }
    const int R = a.res;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      invd[i] = (d[i] != 0.0f) ? (1.0f / d[i]) : __builtin_huge_valf();
      step[i] = d[i] > 0.0f ? 1 : (d[i] < 0.0f ? -1 : 0);
    }
    if (st.flags & MARCH_FRESH) {
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const float inv = (float)R / (a.bmax[i] - a.bmin[i]);
        const float p = o[i] + t0 * d[i];
        const int ci = (int)floorf((p - a.bmin[i]) * inv);
        cc[i] = ci < 0 ? 0 : (ci > R - 1 ? R - 1 : ci);
      }
      st.k = 0;
      st.n = 0;
    } else {
      cc[0] = (int)(st.cell & 1023u);
      cc[1] = (int)((st.cell >> 10) & 1023u);
      cc[2] = (int)((st.cell >> 20) & 1023u);
    }
    k = st.k;
    return true;
  }

  // The current cell's 8^3 block is empty: move to the first cell past it.  Every boundary crossing of the
  // one-cell-at-a-time walk is an event (time, axis) -- the walk takes the smallest time, the lower axis on
  // ties, and the ray's end t1 before any axis at equal time -- and an axis' crossing times do not decrease
  // along it.  So the walk leaves the block by the first of the block's faces in that order (or ends inside
  // it at t1), after exactly the interior crossings that precede that event; each time below is the walk's
  // own formula for the same boundary.  The caller guarantees at least 24 steps of iteration budget.
  __device__ __forceinline__ bool jump_block(const MarchArgs& a, const float (&cell)[3]) {
    constexpr int B = 8;
    const int R = a.res;
    int face[3];
    float e_best = t1;
    int j_best = -1;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int b0 = cc[i] & ~(B - 1), b1 = (b0 + B - 1 < R - 1 ? b0 + B - 1 : R - 1);
      face[i] = step[i] > 0 ? b1 : b0;
      if (step[i] == 0) continue;
      const float bound = a.bmin[i] + (float)(face[i] + (step[i] > 0 ? 1 : 0)) * cell[i];
      const float te = (bound - o[i]) * invd[i];
      if (te < e_best) {
        e_best = te;
        j_best = i;
      }
    }
    int n_steps = 0;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (step[i] == 0) continue;
      if (i == j_best) {
        n_steps += (face[i] - cc[i]) * step[i] + 1;
        cc[i] = face[i] + step[i];
        continue;
      }
      // this axis' crossings before the exit event (at most B - 1: its own face comes after that event)
      int c = cc[i];
      for (;;) {
        const float bound = a.bmin[i] + (float)(c + (step[i] > 0 ? 1 : 0)) * cell[i];
        const float te = (bound - o[i]) * invd[i];
        if (!(te < e_best || (te == e_best && i < j_best))) break;
        c += step[i];
        ++n_steps;
      }
      cc[i] = c;
    }
    t_pend = e_best;  // k past the block's cells, where it is next used
    if (j_best < 0) {  // the ray ends inside the block
      done = true;
      return true;
    }
    bool out = false;  // static indices: a dynamic cc[j_best] would put the walk state in scratch memory
#pragma unroll
    for (int i = 0; i < 3; ++i)
      if (i == j_best) out = cc[i] < 0 || cc[i] >= R;
    if (out) {
      done = true;
      return true;
    }
    iter += n_steps;
    return false;
  }

  // one cell of the walk; returns true when the ray is finished or paused for this call
  __device__ __forceinline__ bool advance(const MarchArgs& a, const float (&cell)[3], bool use_blocks) {
    const int R = a.res;
    // the cell's bit and its block's bit, loaded together
    const int64_t bi = cc[0] + (int64_t)R * (cc[1] + (int64_t)R * cc[2]);
    const uint32_t wcell = a.bits[bi >> 5];
    if (use_blocks && iter + 24 < 3 * R + 2) {
      const int NB = (R + 7) >> 3;
      const int64_t bb = (cc[0] >> 3) + (int64_t)NB * ((cc[1] >> 3) + (int64_t)NB * (cc[2] >> 3));
      if (!((a.blocks[bb >> 5] >> (bb & 31)) & 1u)) return jump_block(a, cell);
    }
    float t_exit = t1;
    int axis = -1;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (step[i] == 0) continue;
      const float bound = a.bmin[i] + (float)(cc[i] + (step[i] > 0 ? 1 : 0)) * cell[i];
      const float te = (bound - o[i]) * invd[i];
      if (te < t_exit) {
        t_exit = te;
        axis = i;
      }
    }
    const bool occ = (wcell >> (bi & 31)) & 1u;
    if (occ) {
      k = skip_lattice(t0, k, a.dt, t_pend);
      for (;;) {
        const float tk = lattice_t(t0, k, a.dt);
        if (!(tk < t_exit)) break;
        if (st.n + emitted >= a.max_steps) {
          done = true;
          break;
        }
        if (emitted >= a.chunk) {
          paused = true;
          break;
        }
        if (EMIT) {
          const uint64_t slot = base + emitted;
          if (slot < a.capacity) {
            a.samples[slot] = make_float4(o[0] + tk * d[0], o[1] + tk * d[1], o[2] + tk * d[2], tk);
            if (a.ray_ids) a.ray_ids[slot] = r;
          }
        }
        ++emitted;
        ++k;
      }
      if (done || paused) return true;
    } else {
      t_pend = t_exit;  // skip the empty cell (k is brought past t_exit where it is next used)
    }
    if (axis < 0) {
      done = true;
      return true;
    }
    // step into the next cell (static indices: the walk state stays in registers)
    int ncc = 0;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (i == axis) {
        cc[i] += step[i];
        ncc = cc[i];
      }
    }
    if (ncc < 0 || ncc >= R) {
      done = true;
      return true;
    }
    if (iter == 3 * R + 2) {
      done = true;
      return true;
    }
    ++iter;
    return false;
  }

  // the state kept for the next call (walked rays only)
  __device__ __forceinline__ void finish_state(const MarchArgs& a, bool walked) {
    if (EMIT && a.state) {
      if (walked) {
        st.k = skip_lattice(t0, k, a.dt, t_pend);
        st.cell = (uint32_t)cc[0] | ((uint32_t)cc[1] << 10) | ((uint32_t)cc[2] << 20);
      }
      st.n += emitted;
      st.flags = (st.flags & ~MARCH_FRESH) | (done ? MARCH_DONE : 0u);
      a.state[r] = st;
    }
  }
};

template <bool EMIT>
__global__ __launch_bounds__(256) void k_march(MarchArgs a) {
  if (a.gate && *a.gate == 0u) return;  // the whole launch: every ray has stopped
  const int lane = threadIdx.x & 63;
  const uint64_t wave = (uint64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const uint64_t r_begin = wave * MARCH_RPW;
  if (r_begin >= a.num_rays) return;  // the same on every lane of the wavefront
  const uint32_t r_end = (uint32_t)(r_begin + MARCH_RPW < a.num_rays ? r_begin + MARCH_RPW : a.num_rays);
  float cell[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) cell[i] = (a.bmax[i] - a.bmin[i]) / (float)a.res;
  const bool use_blocks = a.blocks && *a.blocks_use != 0u;  // the same for every lane
  uint32_t next = (uint32_t)r_begin;  // the wavefront's next unclaimed ray
  RayWalk<EMIT> w;
  bool have = false;  // this lane walks a ray
  for (;;) {
    // lanes without a ray claim the next rays of the range, in lane order
    const uint64_t need = __ballot(!have);
    if (!have) {
      const uint32_t rr = next + (uint32_t)__popcll(need & ((1ull << lane) - 1ull));
      if (rr < r_end) {
        if (w.start(a, rr, cell)) {
          have = true;
        } else if (!EMIT || a.slot_stride) {
          a.counts[rr] = 0u;
        }
      }
    }
    next = next + (uint32_t)__popcll(need);
    if (next > r_end) next = r_end;
    if (__ballot(have) == 0ull) {
      if (next >= r_end) break;
      continue;
    }
    // a few cells per lane between claims: the claim's wavefront-wide bookkeeping is paid once per batch
#pragma unroll 1
    for (int j = 0; j < MARCH_CELLS_PER_CLAIM; ++j) {
      if (have && w.advance(a, cell, use_blocks)) {
        w.finish_state(a, true);
        if (!EMIT || a.slot_stride) a.counts[w.r] = w.emitted;
        have = false;
      }
    }
  }
}

// One wavefront per ray at a time: the ray's samples from its slots to its compacted range, 64 at a time
__global__ __launch_bounds__(256) void k_march_compact(const uint32_t* __restrict__ counts,
                                                       const uint32_t* __restrict__ offsets,
                                                       const float4* __restrict__ slots, uint32_t stride,
                                                       uint32_t num_rays, float4* __restrict__ samples,
                                                       uint32_t* __restrict__ ray_ids,
                                                       const uint32_t* __restrict__ gate) {
  if (gate && *gate == 0u) return;
  const int lane = threadIdx.x & 63;
  const uint32_t n_waves = gridDim.x * (blockDim.x >> 6);
  for (uint32_t r = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); r < num_rays; r += n_waves) {
    const uint32_t c = counts[r], o = offsets[r];
    const float4* src = slots + (uint64_t)r * stride;
    for (uint32_t k = lane; k < c; k += 64) {
      samples[(uint64_t)o + k] = src[k];
      ray_ids[(uint64_t)o + k] = r;
    }
  }
}

// sample budget of a marched step (launch_march_clamp): offsets [num_rays + 1], offsets[r + 1] the end of ray r
__global__ __launch_bounds__(256) void k_march_clamp(uint32_t* __restrict__ counts, const uint32_t* __restrict__ offsets,
                                                     uint32_t num_rays, uint32_t cap, uint32_t* __restrict__ n_eff) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= num_rays) return;
  const uint32_t end = offsets[r + 1];
  const bool fits = end <= cap;
  if (!fits) counts[r] = 0u;
  // the rays that fit are a prefix (offsets never decrease): its last ray writes the samples kept
  const bool next_fits = r + 1 < num_rays && offsets[r + 2] <= cap;
  if (fits && !next_fits) *n_eff = end;
  if (r == 0 && !fits) *n_eff = 0u;
}

__global__ __launch_bounds__(256) void k_march_init(MarchState* __restrict__ state, float4* __restrict__ acc,
                                                    uint32_t* __restrict__ n_used, uint32_t num_rays,
                                                    uint32_t* __restrict__ prime) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  if (prime && r == 0) *prime = 1u;
  if (r >= num_rays) return;
  state[r] = MarchState{0u, 0u, 0u, MARCH_FRESH};
  acc[r] = make_float4(0.0f, 0.0f, 0.0f, 1.0f);
  if (n_used) n_used[r] = 0u;
}

// front-to-back compositing of this round's samples of each ray (alpha as ffnerf_OG.cl:1505-1520);
// a ray whose transmittance drops below T_stop is retired
__global__ __launch_bounds__(256) void k_render_composite(const uint32_t* __restrict__ offsets,
                                                          const uint32_t* __restrict__ counts, uint32_t num_rays,
                                                          const float* __restrict__ sigma,
                                                          const float* __restrict__ rgb, float dt, float T_stop,
                                                          MarchState* __restrict__ state, float4* __restrict__ acc,
                                                          uint32_t* __restrict__ n_used,
                                                          const uint32_t* __restrict__ gate) {
  if (gate && *gate == 0u) return;
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= num_rays) return;
  const uint32_t cnt = counts[r];
  if (cnt == 0) return;
  const uint32_t off = offsets[r];
  float4 cv = acc[r];
  float T = cv.w;
  if (!(T >= T_stop)) return;  // retired in an earlier round
  float C0 = cv.x, C1 = cv.y, C2 = cv.z;
  uint32_t used = 0;
  for (uint32_t j = 0; j < cnt; ++j) {
    const uint32_t b = off + j;
    const float alpha = 1.0f - fast_exp(fminf(fmaxf(-sigma[b] * dt, -5.0f), 18.0f));
    const float w = T * alpha;
    C0 = C0 + w * rgb[3 * (size_t)b];
    C1 = C1 + w * rgb[3 * (size_t)b + 1];
    C2 = C2 + w * rgb[3 * (size_t)b + 2];
    T = T * (1.0f - alpha);
    ++used;
    if (T < T_stop) {
      state[r].flags |= MARCH_DONE;
      break;
    }
  }
  acc[r] = make_float4(C0, C1, C2, T);
  if (n_used) n_used[r] += used;
}

__global__ __launch_bounds__(256) void k_render_finish(const float4* __restrict__ acc, uint32_t num_rays,
                                                       float4* __restrict__ out_rgb) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= num_rays) return;
  out_rgb[r] = acc[r];  // black background: C + T * 0; w = T_final
}

// Compositing of marched training rays: one lane per ray walks its samples front to back (the order of the
// specification, ora_train_step_marched), keeping the transmittance before every sample for the backward
// sweep, which walks them back to front with dL/dT of the next sample (ffnerf_OG.cl:1593-1634 restated as a
// sequential recurrence: gT_i = g . (alpha_i c_i) + (1 - alpha_i) gT_(i+1), gT_end = g . bg).
// (cell, subcell) of the occupancy grid holding the point at time t of ray (o, d), as the proposals compute it;
// kOutsideGrid for a point outside the grid
constexpr uint64_t kOutsideGrid = ~(uint64_t)1;
__device__ __forceinline__ uint64_t occ_run_key(const DevCfg& c, const float (&o)[3], const float (&d)[3], float t) {
  float gpos[3];
  occ_grid_pos(c, o, d, t, gpos);
  const int G = c.G;
  const int ix = (int)floorf(gpos[0]), iy = (int)floorf(gpos[1]), iz = (int)floorf(gpos[2]);
  if (!((uint32_t)ix < (uint32_t)G && (uint32_t)iy < (uint32_t)G && (uint32_t)iz < (uint32_t)G)) return kOutsideGrid;
  uint32_t sub = 0;
#pragma unroll
  for (int i = 0; i < 3; ++i) sub += ((gpos[i] - floorf(gpos[i])) >= 0.5f ? 1u : 0u) << i;
  return ((uint64_t)(ix + G * (iy + G * iz)) << 3) | sub;
}

// The occupancy proposals of marched ray r: its samples, in order, fall into runs of one (cell, subcell) of the
// occupancy grid, and each run inside the grid proposes as a run of the resampled step does
// (ffnerf_OG.cl:1640-1821), from the compositing's transmittances (T_end past a termination, so those runs
// propose nothing).
__device__ void propose_marched_runs(const CompMarchArgs& a, uint32_t r, uint32_t off, uint32_t cnt, float T_end) {
  if (cnt == 0) return;
  const float4 ro = a.rays[2 * r], rdv = a.rays[2 * r + 1];
  const float o[3] = {ro.x, ro.y, ro.z}, d[3] = {rdv.x, rdv.y, rdv.z};
  const float Dhalf = half_box_diagonal(a.c);
  uint32_t s = 0;
  float t_s = a.samples[off].w;
  uint64_t key_s = occ_run_key(a.c, o, d, t_s);
  for (uint32_t j = 1; j <= cnt; ++j) {
    float t_j = 0.0f;
    uint64_t key_j = ~(uint64_t)0;
    if (j < cnt) {
      t_j = a.samples[off + j].w;
      key_j = occ_run_key(a.c, o, d, t_j);
    }
    if (key_j == key_s) continue;
    if (key_s != kOutsideGrid) {  // the run [s, j) ends here
      const uint32_t prev = s > 0 ? s - 1 : 0;
      const bool has_next = j < cnt;
      occ_propose_run(a.c, o, d, t_s, a.Tr[off + s], a.samples[off + prev].w, a.Tr[off + prev],
                      a.samples[off + j - 1].w, a.Tr[off + j - 1], has_next, t_j, has_next ? a.Tr[off + j] : 0.0f,
                      T_end, a.occ_in[key_s >> 3], a.seed, r, s, Dhalf, a.occ_st);
    }
    s = j;
    t_s = t_j;
    key_s = key_j;
  }
}

__global__ __launch_bounds__(256) void k_composite_marched(CompMarchArgs a) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= a.num_rays) return;
  const uint32_t cnt = a.counts[r], off = a.offsets[r];
  float T = 1.0f, C0 = 0.0f, C1 = 0.0f, C2 = 0.0f;
  uint32_t used = 0;
  for (uint32_t j = 0; j < cnt; ++j) {
    const uint32_t b = off + j;
    const float alpha = 1.0f - fast_exp(fminf(fmaxf(-a.sigma[b] * a.dt, -5.0f), 18.0f));
    a.Tr[b] = T;
    const float w = T * alpha;
    C0 = C0 + w * a.rgb[3 * (size_t)b];
    C1 = C1 + w * a.rgb[3 * (size_t)b + 1];
    C2 = C2 + w * a.rgb[3 * (size_t)b + 2];
    T = T * (1.0f - alpha);
    ++used;
    if (T < a.T_stop) break;
  }
  float bg[3] = {0.0f, 0.0f, 0.0f};
  if (a.background == FFN_BG_WHITE) {
    bg[0] = bg[1] = bg[2] = 1.0f;
  } else if (a.background == FFN_BG_RANDOM) {
    uint32_t rb = hash_u32(a.seed ^ r * 747796405u ^ 0xA511E9B3u);
    bg[0] = rand01(rb);
    bg[1] = rand01(rb);
    bg[2] = rand01(rb);
  }
  const float4 tg = a.targets[r];
  const float Cf0 = C0 + T * bg[0], Cf1 = C1 + T * bg[1], Cf2 = C2 + T * bg[2];
  const float gr0 = charbonnier_prime(Cf0 - tg.x), gr1 = charbonnier_prime(Cf1 - tg.y),
              gr2 = charbonnier_prime(Cf2 - tg.z);
  a.out_rgb[r] = make_float4(fminf(fmaxf(Cf0, 0.0f), 1.0f), fminf(fmaxf(Cf1, 0.0f), 1.0f),
                             fminf(fmaxf(Cf2, 0.0f), 1.0f), 4.0f);
  if (a.n_used) a.n_used[r] = used;
  if (a.T_final) a.T_final[r] = T;
  if (a.color) a.color[r] = make_float4(Cf0, Cf1, Cf2, 0.0f);
  float gT = gr0 * bg[0] + gr1 * bg[1] + gr2 * bg[2];
  for (uint32_t j = used; j-- > 0;) {
    const uint32_t b = off + j;
    const float alpha = 1.0f - fast_exp(fminf(fmaxf(-a.sigma[b] * a.dt, -5.0f), 18.0f));
    const float Ti = a.Tr[b];
    const float c0 = a.rgb[3 * (size_t)b], c1 = a.rgb[3 * (size_t)b + 1], c2 = a.rgb[3 * (size_t)b + 2];
    const float gA = gr0 * (Ti * c0) + gr1 * (Ti * c1) + gr2 * (Ti * c2);
    const float gAlpha = gA - gT * Ti;
    a.dLds[b] = gAlpha * (a.dt * (1.0f - alpha)) + a.regu;
    const float ws = Ti * alpha;
    a.dLdc[3 * (size_t)b] = ws * gr0;
    a.dLdc[3 * (size_t)b + 1] = ws * gr1;
    a.dLdc[3 * (size_t)b + 2] = ws * gr2;
    gT = (gr0 * (alpha * c0) + gr1 * (alpha * c1) + gr2 * (alpha * c2)) + (1.0f - alpha) * gT;
  }
  for (uint32_t j = used; j < cnt; ++j) {  // past the termination: no contribution, no gradient
    const uint32_t b = off + j;
    a.Tr[b] = T;
    a.dLds[b] = 0.0f;
    a.dLdc[3 * (size_t)b] = a.dLdc[3 * (size_t)b + 1] = a.dLdc[3 * (size_t)b + 2] = 0.0f;
  }
  if (a.occ_st) propose_marched_runs(a, r, off, cnt, T);
}

hipError_t launch_composite_marched(const CompMarchArgs& a, hipStream_t st) {
  if (a.num_rays == 0) return hipSuccess;
  hipLaunchKernelGGL(k_composite_marched, dim3((a.num_rays + 255) / 256), dim3(256), 0, st, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------

hipError_t launch_occ_bitfield(const uint32_t* occ, int G, uint32_t q_min, uint32_t* bits, hipStream_t st) {
  const int64_t R = 2 * (int64_t)G;
  const int64_t n_words = (R * R * R + 31) / 32;
  hipLaunchKernelGGL(k_occ_bitfield, dim3((unsigned)((n_words + 255) / 256)), dim3(256), 0, st, occ, G, q_min,
                     bits, n_words);
  return hipGetLastError();
}

hipError_t launch_occ_blocks(const uint32_t* bits, int R, uint32_t* blocks, uint32_t* use, hipStream_t st) {
  const int64_t NB = (R + 7) / 8;
  const int64_t n_blocks = NB * NB * NB;
  hipLaunchKernelGGL(k_occ_blocks, dim3((unsigned)((n_blocks + 255) / 256)), dim3(256), 0, st, bits, R, blocks,
                     n_blocks);
  hipLaunchKernelGGL(k_blocks_use, dim3(1), dim3(256), 0, st, blocks, n_blocks, use);
  return hipGetLastError();
}

hipError_t launch_march(const MarchArgs& a, bool emit, hipStream_t st) {
  if (a.num_rays == 0) return hipSuccess;
  const uint64_t waves = (a.num_rays + MARCH_RPW - 1) / MARCH_RPW;
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  if (emit)
    hipLaunchKernelGGL(k_march<true>, grid, block, 0, st, a);
  else
    hipLaunchKernelGGL(k_march<false>, grid, block, 0, st, a);
  return hipGetLastError();
}

hipError_t launch_march_compact(const uint32_t* counts, const uint32_t* offsets, const float4* slots,
                                uint32_t stride, uint32_t num_rays, float4* samples, uint32_t* ray_ids,
                                hipStream_t st, const uint32_t* gate) {
  if (num_rays == 0) return hipSuccess;
  const uint32_t blocks = (num_rays + 3) / 4 < 4096 ? (num_rays + 3) / 4 : 4096;
  hipLaunchKernelGGL(k_march_compact, dim3(blocks), dim3(256), 0, st, counts, offsets, slots, stride, num_rays,
                     samples, ray_ids, gate);
  return hipGetLastError();
}

hipError_t launch_march_clamp(uint32_t* counts, const uint32_t* offsets, uint32_t num_rays, uint32_t cap,
                              uint32_t* n_eff, hipStream_t st) {
  if (num_rays == 0) return hipSuccess;
  hipLaunchKernelGGL(k_march_clamp, dim3((num_rays + 255) / 256), dim3(256), 0, st, counts, offsets, num_rays, cap,
                     n_eff);
  return hipGetLastError();
}

hipError_t launch_march_init(MarchState* state, float4* acc, uint32_t* n_used, uint32_t num_rays, hipStream_t st,
                             uint32_t* prime) {
  if (num_rays == 0) return hipSuccess;
  hipLaunchKernelGGL(k_march_init, dim3((num_rays + 255) / 256), dim3(256), 0, st, state, acc, n_used, num_rays,
                     prime);
  return hipGetLastError();
}

hipError_t launch_render_composite(const uint32_t* offsets, const uint32_t* counts, uint32_t num_rays,
                                   const float* sigma, const float* rgb, float dt, float T_stop, MarchState* state,
                                   float4* acc, uint32_t* n_used, hipStream_t st, const uint32_t* gate) {
  if (num_rays == 0) return hipSuccess;
  hipLaunchKernelGGL(k_render_composite, dim3((num_rays + 255) / 256), dim3(256), 0, st, offsets, counts, num_rays,
                     sigma, rgb, dt, T_stop, state, acc, n_used, gate);
  return hipGetLastError();
}

hipError_t launch_render_finish(const float4* acc, uint32_t num_rays, float4* out_rgb, hipStream_t st) {
  if (num_rays == 0) return hipSuccess;
  hipLaunchKernelGGL(k_render_finish, dim3((num_rays + 255) / 256), dim3(256), 0, st, acc, num_rays, out_rgb);
  return hipGetLastError();
}

}  // namespace ffn
