// The LM head's Q8_0 product fused with the whole sampled output of
// fg_output_sample (src/output.c:702-756): per token, the logits of the
// vocabulary (fg_output_logits), penalties over the token's history counts
// (fg_vk_apply_penalties, C rounding as src/sampler.c:55-58), then either
// the greedy argmax ladder (T == 0) or the top-k ladder
// (output_topk_in_batch, src/output.c:681-700) and fg_sampler_select
// (src/sampler.c:80-122).  No logit leaves the chip: a token costs one pass
// over the weights plus a few KB of candidate lists.
//
// Grid: one 16-row cooked tile per wave, as dense_q8_finalist_kernel.
// Sampled tokens are reduced in three steps:
//   workgroup  its 64 penalised logits (4 waves x 16 rows) sorted by one
//              wave; the best kk are published with their count;
//   group      of 64 consecutive workgroups: the last to count in merges
//              the group's lists (one list per lane, a round per list
//              position, a list stopping at its first entry the merged list
//              has beaten), publishes the group's best kk and raises the
//              token's bound to its kk-th (kk entries of the row are at or
//              above it: later merges skip what is below);
//   token      the last group merges the groups' lists the same way (in the
//              same pass as its own when it sees every other group in
//              already) and runs the select (finish_row, the sampler's own
//              f64 arithmetic).
// Greedy tokens keep the finalist kernel's single atomic-max step (with
// penalised values).  Hand-offs use agent-scope atomics and wait_memory()
// (see its comment for the argument).
#pragma once

#include "fg_dense_kernels.hpp"
#include "fg_sample_kernels.hpp"

namespace fg {

constexpr uint32_t kLmGroup = 64;  // workgroups per merge group
constexpr uint32_t kLmLine64 = kLineWords / 2u;  // u64 per 128-byte line
constexpr uint32_t kLmCand = (kDenseBlock / kWave) * kCookRows;  // 64 logits per workgroup
static_assert(kLmCand == static_cast<uint32_t>(kWave), "one candidate per lane");

// The slice's workspace, in device memory (written once at create): the
// kernel reads it only in its closing steps, so none of it occupies scalar
// registers during the product.
struct LmWork {
  uint32_t vocab;             // full vocabulary (ids < vocab)
  uint32_t wg_cap, grp_cap;   // workgroups and groups the workspace holds
  // Every counter and running value below sits on its own 128-byte line
  // (kLineWords u32): thousands of workgroups update them, and updates to
  // one line queue behind each other.
  unsigned long long* keys;   // [2][line] greedy composites, zero between launches
  uint32_t* arrivals;         // [2][line] greedy arrivals, zero between launches
  // sampled tokens, token-major (zero between launches where noted)
  uint64_t* wg_lists;         // [2][grp_cap][kMaxK][kLmGroup] (position-major per group)
  uint32_t* wg_count;         // [2][wg_cap]
  uint32_t* grp_arrivals;     // [2][grp_cap][line], zero between launches
  uint64_t* grp_lists;        // [2][kMaxK][grp_cap] each group's best kk (position-major)
  uint32_t* grp_count;        // [2][grp_cap]
  uint32_t* fin_arrivals;     // [2][line], zero between launches
  unsigned long long* bound;  // [2][line] best group kk-th so far, zero between launches
};

struct LmSampleArgs {
  DenseArgs d;                // the product; values/ids/status receive the tokens
  RowParams p[2];             // controls of the pass's tokens (token0 + t)
  const uint32_t* counts;     // [token][cstride] history counts by vocabulary id, or NULL
  uint64_t cstride;
  const float* uniforms;      // [token]
  const LmWork* work;
};

// The controls of the pass's token t (selected, so that a runtime t does not
// index the kernel-argument array).
__device__ __forceinline__ RowParams lm_params(const LmSampleArgs& s, uint32_t t) {
  return t == 0u ? s.p[0] : s.p[1];
}

// The kk best entries of nl sorted lists (list l: cnt[l] entries at
// lists + l * kMaxK, descending; list `skip` left out), by one wave: lane i
// of the result is the i-th best (0 past the end).  `floor` is a lower bound
// of the row's kk-th (or 0): nothing below it is needed.  Lists are taken 64 at a
// time, one per lane, their first kLmAhead entries loaded at once with the
// counts (coherently: other workgroups published them).  Each round stages
// the lanes' next entries that beat the running list (a TopList: staged
// entries are sorted into it 64 at a time, which raises its bar), and a list
// stops at its first entry that does not (the rest are smaller); the few
// lists that put more than kLmAhead entries past the bar read on one entry
// per round.  `buf` is kLmStage u64 of wave-private LDS.
constexpr uint32_t kLmAhead = 16;
constexpr uint32_t kNoList = 0xffffffffu;  // lm_merge: skip nothing
constexpr uint32_t kLmStage = 3u * kWave;  // < 64 left + one round of 64, spare slots
__device__ __forceinline__ uint64_t lm_merge(const uint64_t* lists, uint32_t es,
                                             const uint32_t* cnt, uint32_t nl, uint32_t kk,
                                             uint32_t skip, uint64_t floor, uint64_t* buf) {
  const uint32_t lane = lane_id();
  // Entries below floor (a lower bound of the row's kk-th) cannot enter.
  const uint64_t R0 = floor > kFiniteComp ? floor - 1ull : kFiniteComp - 1ull;
  TopList t{0ull, R0, buf, 0u, kk, -3.402823466e38f, nullptr, 0xffffffffu};
  for (uint32_t l0 = 0; l0 < nl; l0 += kWave) {
    const uint32_t l = l0 + lane;
    const bool use = l < nl && l != skip;
    const uint64_t* mine = lists + l;  // entry j at mine + j * es
    uint32_t c = use ? load_coherent(cnt + l) : 0u;
    uint64_t head[kLmAhead];
#pragma unroll
    for (uint32_t j = 0; j < kLmAhead; j++)
      head[j] = use ? load_coherent(mine + static_cast<uint64_t>(j) * es) : 0ull;
    c = c < kk ? c : kk;
    for (uint32_t j = 0; ballot(j < c) != 0ull; j++) {
      uint64_t x = 0ull;
#pragma unroll
      for (uint32_t q = 0; q < kLmAhead; q++) x = q == j ? head[q] : x;
      if (j >= kLmAhead && j < c) x = load_coherent(mine + static_cast<uint64_t>(j) * es);
      const bool beats = j < c && x > t.R;
      if (!beats) c = j;  // sorted: the rest of this list cannot enter either
      top_stage(t, beats ? x : 0ull);
      if (t.n >= static_cast<uint32_t>(kWave)) top_drain(t, false);
    }
  }
  top_drain(t, true);
  return lane < kk ? t.top : 0ull;
}

#ifdef FG_LM_TRACE
// Phase timestamps of trace builds: [workgroup][8] (s_memrealtime, 100 MHz),
// kept in LDS and copied out where the workgroup's work ends (FG_LMT_FLUSH):
// a global store per stamp would make the compiler wait for its completion
// before reusing its registers.
__device__ uint64_t g_lm_trace[8192 * 8];
__shared__ uint64_t s_lm_trace[8];
#define FG_LMT(slot)                                                      \
  do {                                                                    \
    if (lane_id() == 0) s_lm_trace[slot] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#define FG_LMT_INIT                                                       \
  do {                                                                    \
    if (threadIdx.x < 8u) s_lm_trace[threadIdx.x] = 0ull;                 \
  } while (0)
#define FG_LMT_FLUSH                                                      \
  do {                                                                    \
    if (lane_id() == 0)                                                   \
      for (int i_ = 0; i_ < 8; i_++) g_lm_trace[blockIdx.x * 8u + i_] = s_lm_trace[i_]; \
  } while (0)
#else
#define FG_LMT(slot) \
  do {               \
  } while (0)
#define FG_LMT_INIT \
  do {              \
  } while (0)
#define FG_LMT_FLUSH \
  do {               \
  } while (0)
#endif

// Greedy close of token t (the last workgroup of the grid for it): the
// finalist kernel's decode, with penalised values.  One wave.
template <int B>
__device__ inline void lm_close_greedy(const LmSampleArgs& s, const float* s_x, uint32_t t) {
  const DenseArgs& a = s.d;
  const uint32_t lane = lane_id();
  const uint32_t tok = a.token0 + t;
  const RowParams p = lm_params(s, t);
  const bool pen = (p.flags & kRowPenalties) && s.counts;
  uint64_t k = 0ull;
  if (lane == 0) {
    k = __hip_atomic_exchange(s.work->keys + t * kLmLine64, 0ull, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(s.work->arrivals + t * kLineWords, 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  k = readlane64(k, 0);
  const uint32_t id = greedy_id(k);
  const uint32_t row = id - a.first_row;
  const uint32_t hi = static_cast<uint32_t>(k >> 32);
  float v = key_to_float(hi);
  if (k != 0ull && (hi == 0xffffffffu || hi == 0x80000000u)) {
    // Non-finite or zero: recompute the winner's logit (exact bits).
    float out[B];
    tile_rows<B>(a, row / kCookRows, s_x, out);
    float mine = 0.0f;
#pragma unroll
    for (int u = 0; u < B; u++)
      if (static_cast<uint32_t>(u) == t) mine = out[u];
    v = __uint_as_float(__builtin_amdgcn_readlane(static_cast<int>(__float_as_uint(mine)),
                                                  static_cast<int>(4u * (row % kCookRows))));
    if (pen)
      v = penalise(v, s.counts[static_cast<uint64_t>(tok) * s.cstride + id], p.presence,
                   p.frequency, p.repetition);
  }
  if (lane == 0) {
    const bool ok = k != 0ull && is_finite_bits(__float_as_uint(v));
    a.values[tok] = v;  // token logits
    a.ids[tok] = ok ? id : kInvalidId;
    a.status[tok] = ok ? kStOk : (pen ? kStFormat : kStMismatch);
  }
}

template <int B>
__global__ __launch_bounds__(kDenseBlock) void dense_q8_sample_kernel(LmSampleArgs s) {
  const DenseArgs& a = s.d;
  extern __shared__ float s_x[];  // staged inputs (read only after staging)
  __shared__ uint64_t s_cand[B][kLmCand];
  __shared__ uint64_t s_best[kDenseBlock / kWave][B];
  __shared__ uint64_t s_stage[B][kLmStage];
  FG_LMT_INIT;
  if (threadIdx.x == 0) FG_LMT(0);
  stage_inputs<B>(a, s_x);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t lane = lane_id();
  const uint64_t tiles = (a.rows + kCookRows - 1u) / kCookRows;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * (kDenseBlock / kWave);
  const uint32_t r = lane >> 2;
  uint64_t best[B], cand[B];
#pragma unroll
  for (int t = 0; t < B; t++) best[t] = cand[t] = 0ull;
  for (uint64_t tile = static_cast<uint64_t>(blockIdx.x) * (kDenseBlock / kWave) + wave;
       tile < tiles; tile += stride) {
    const uint64_t row = tile * kCookRows + r;
    const bool live = (lane & 3u) == 0u && row < a.rows;
    const uint32_t id = a.first_row + static_cast<uint32_t>(row);
    // The history counts of the tile's rows, loaded before the product so
    // their latency hides behind it.
    uint32_t cnt[B];
#pragma unroll
    for (int t = 0; t < B; t++) {
      const RowParams p = lm_params(s, t);
      cnt[t] = live && t < (int)a.tokens && (p.flags & kRowPenalties) && s.counts
                   ? s.counts[static_cast<uint64_t>(a.token0 + t) * s.cstride + id]
                   : 0u;
    }
    float out[B];
    tile_rows<B>(a, tile, s_x, out);
#pragma unroll
    for (int t = 0; t < B; t++) {
      if (!live || t >= (int)a.tokens) continue;
      const RowParams p = lm_params(s, t);
      float v = out[t];
      if ((p.flags & kRowPenalties) && s.counts)
        v = penalise(v, cnt[t], p.presence, p.frequency, p.repetition);
      if (p.temperature == 0.0f) best[t] = max(best[t], greedy_comp(v, id));
      else cand[t] = make_comp(float_key(v), id);  // one tile per wave on this grid
    }
  }
  // ---- workgroup: wave t carries token t from here ----
#pragma unroll
  for (int t = 0; t < B; t++) {
    const uint64_t m = wave_max_u64(best[t]);
    if (lane == 0) s_best[wave][t] = m;
    // Lane 4i holds row i of the wave's tile: candidate slot wave*16 + i.
    if ((lane & 3u) == 0u) s_cand[t][wave * kCookRows + r] = cand[t];
  }
  __syncthreads();
  if (wave == 0) FG_LMT(1);
  if (wave >= static_cast<uint32_t>(B) || wave >= a.tokens) return;
  const uint32_t t = wave;
  const uint32_t tok = a.token0 + t;
  const RowParams p = lm_params(s, t);
  if (p.temperature == 0.0f) {
    // Greedy (src/output.c:728-741 with penalties, fg_output_greedy without).
    uint64_t m = 0ull;
#pragma unroll
    for (uint32_t w = 0; w < kDenseBlock / kWave; w++) m = max(m, s_best[w][t]);
    uint32_t arrived = 0u;
    if (lane == 0) {
      __hip_atomic_fetch_max(s.work->keys + t * kLmLine64, static_cast<unsigned long long>(m),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      wait_memory();  // hand-off ordering: see wait_memory()
      arrived = __hip_atomic_fetch_add(s.work->arrivals + t * kLineWords, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
    }
    arrived = __builtin_amdgcn_readfirstlane(arrived);
    if (arrived + 1u == gridDim.x) lm_close_greedy<B>(s, s_x, t);
    return;
  }
  // Sampled: this workgroup's best kk, published.
  const LmWork& w = *s.work;
  const uint32_t kk = p.top_k;
  const uint64_t grp = blockIdx.x / kLmGroup;
  const uint32_t grp_size = min(kLmGroup, gridDim.x - static_cast<uint32_t>(grp) * kLmGroup);
  const uint32_t ngroups = (gridDim.x + kLmGroup - 1u) / kLmGroup;
  const uint64_t sorted = wave_sort_desc(s_cand[t][lane]);
  const uint32_t n = static_cast<uint32_t>(__popcll(ballot(lane < kk && sorted != 0ull)));
  const uint64_t slot = static_cast<uint64_t>(t) * w.wg_cap + blockIdx.x;
  // Position-major within the group: the merging workgroup's loads of one
  // position of all 64 lists are one contiguous 512-byte run.
  if (lane < n)
    store_coherent(w.wg_lists + ((static_cast<uint64_t>(t) * w.grp_cap + grp) * kMaxK + lane) *
                                    kLmGroup + blockIdx.x % kLmGroup,
                   sorted);
  if (lane == 0) store_coherent(w.wg_count + slot, n);
  wait_memory();  // hand-off ordering: see wait_memory()
  uint32_t arrived = 0u;
  const uint64_t gslot = static_cast<uint64_t>(t) * w.grp_cap + grp;
  if (lane == 0)
    arrived = __hip_atomic_fetch_add(w.grp_arrivals + gslot * kLineWords, 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
  arrived = __builtin_amdgcn_readfirstlane(arrived);
  if (t == 0) FG_LMT(2);
  if (arrived + 1u != grp_size) {
    if (t == 0) FG_LMT_FLUSH;
    return;
  }

  // Group: merge its workgroups' lists.  When every other group has
  // counted in already, this group is the token's last: it merges the
  // other groups' lists in the same pass and runs the select itself.
  if (lane == 0) store_coherent(w.grp_arrivals + gslot * kLineWords, 0u);  // all are in
  const uint32_t groups_in =
      __builtin_amdgcn_readfirstlane(load_coherent(w.fin_arrivals + t * kLineWords));
  const uint64_t wslot = static_cast<uint64_t>(t) * w.wg_cap + grp * kLmGroup;
  const uint64_t* grp_lists = w.grp_lists + static_cast<uint64_t>(t) * kMaxK * w.grp_cap;
  const uint32_t* grp_count = w.grp_count + static_cast<uint64_t>(t) * w.grp_cap;
  const bool last_group = groups_in + 1u == ngroups;
  // The row's kk-th is at or above every finished group's kk-th.
  unsigned long long* bound = w.bound + t * kLmLine64;
  const uint64_t floor_g =
      __hip_atomic_load(bound, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint64_t fin = lm_merge(w.wg_lists + (static_cast<uint64_t>(t) * w.grp_cap + grp) * kMaxK * kLmGroup,
                          kLmGroup, w.wg_count + wslot, grp_size, kk, kNoList, floor_g, s_stage[t]);
  if (last_group)
    fin = wave_merge_desc(fin, lm_merge(grp_lists, w.grp_cap, grp_count, ngroups, kk,
                                        static_cast<uint32_t>(grp), floor_g, s_stage[t]));
  fin = lane < kk ? fin : 0ull;
  if (t == 0) FG_LMT(3);
  if (!last_group) {
    const uint32_t gn = static_cast<uint32_t>(__popcll(ballot(fin != 0ull)));
    if (lane < gn)
      store_coherent(w.grp_lists + (static_cast<uint64_t>(t) * kMaxK + lane) * w.grp_cap + grp, fin);
    const uint64_t kth = readlane64(fin, kk - 1u);
    if (lane == 0) {
      store_coherent(w.grp_count + gslot, gn);
      // kk entries of the row are at or above the group's kk-th.
      if (gn >= kk)
        __hip_atomic_fetch_max(bound, static_cast<unsigned long long>(kth), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    wait_memory();  // hand-off ordering: see wait_memory()
    if (lane == 0)
      arrived = __hip_atomic_fetch_add(w.fin_arrivals + t * kLineWords, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
    arrived = __builtin_amdgcn_readfirstlane(arrived);
    if (t == 0) FG_LMT(4);
    if (arrived + 1u != ngroups) {
      if (t == 0) FG_LMT_FLUSH;
      return;
    }
    // Token: the last group to count in merges the groups' lists.
    const uint64_t floor_t = __hip_atomic_load(bound, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    fin = lm_merge(grp_lists, w.grp_cap, grp_count, ngroups, kk, kNoList, floor_t, s_stage[t]);
  }
  if (lane == 0) {
    store_coherent(w.fin_arrivals + t * kLineWords, 0u);
    store_coherent(w.bound + t * kLmLine64, 0ull);
  }
  if (t == 0) FG_LMT(5);
  SampleArgs fa{};
  fa.vocab = w.vocab;
  fa.tokens = a.ids;
  fa.token_logits = a.values;
  fa.row_status = a.status;
  const bool pen = (p.flags & kRowPenalties) && s.counts;
  finish_row(fa, p, tok, fin, 0ull, -INFINITY, 0.0, Mass{-INFINITY, 0.0, 0.0}, nullptr, nullptr,
             pen, s.uniforms[tok], 1.0 / static_cast<double>(p.temperature));
  if (t == 0) FG_LMT(6);
  if (t == 0) FG_LMT_FLUSH;
}

}  // namespace fg
