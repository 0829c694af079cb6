// gfx950 kernel of the batched sampler: one fused streaming pass over
// rows x vocab f32 logits (+ u32 history counts) that ends in a token per row.
//
// Grid: rows x chunks workgroups of 256 threads (4 waves).  Each wave streams
// a contiguous slice of its row from HBM exactly once: 16-byte non-temporal
// loads of logits and counts, double-buffered so the next step's loads are in
// flight while the current step is processed.  In registers each wave keeps
// only what the row's result needs:
//   * penalties (src/sampler.c:55-58) applied in registers;
//   * greedy: the best greedy composite (src/output.c:484-492);
//   * top-k:  a sorted register list of its best 64 composites behind a
//             rising filter; candidates that pass are staged in LDS and merged
//             64 at a time with bitonic networks built from DPP / permlane
//             moves (the reference's per-tile select, shaders/fg_topk_select.comp,
//             recast as a streaming merge);
//   * log-probs: per-lane online (max, sum exp) in f32.
// Row hand-off: when a row spans several workgroups, every wave publishes its
// top-kk list, greedy winner and (max, sum) with device-coherent (sc1) stores
// and waits for them; the workgroup then bumps the row's arrival counter (one
// cache line per row, so rows never contend).  The last workgroup to arrive
// reads the row's partials with sc1 loads, merges the sorted lists and runs
// the select arithmetic of src/sampler.c:80-122 in one wave, then resets the
// row's counter for the next launch.  No L2 write-back or invalidate is
// needed.  A row that fits one workgroup is
// merged straight from LDS.
#pragma once

#include "fg_device.hpp"

namespace fg {

struct RowParams {
  float temperature;
  float top_p;
  uint32_t top_k;
  float presence;
  float frequency;
  float repetition;
  uint32_t flags;
  uint32_t reserved;
};
constexpr uint32_t kRowPenalties = 1u;

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kMaxStepVec = 4;  // quads (4 elements) per lane per streaming step, at most
constexpr uint32_t kStepElems = kWave * kMaxStepVec * 4u;  // elements per step, at most
// LDS staging per wave: fewer than 64 left over plus one full step.
constexpr uint32_t kCap = 64u + kStepElems;
constexpr uint32_t kMaxK = 64;       // largest top-k / log-prob count
constexpr uint32_t kXcds = 8;  // XCDs of an MI355X (workgroups go round robin)
constexpr uint32_t kSpecMinK = 32;   // top lists longer than this stage speculatively
constexpr uint32_t kSpecMaxElems = 24u * 1024u;  // ... over wave slices of at most this many steps
constexpr uint32_t kMaxChunks = 64;  // workgroups per row
constexpr uint32_t kDefaultGroups = 512;   // chunking: ceil(512 / rows) chunks per row
constexpr uint32_t kNucleusGroups = 768;   // chunking with whole-row nucleus rows
constexpr uint32_t kMaxGroups = 1024;      // workspace: workgroups a launch may use beyond rows
constexpr uint32_t kLineWords = 32;  // u32 per 128-byte cache line (row counters)

constexpr int32_t kStOk = 0;
constexpr int32_t kStFormat = 4;
constexpr int32_t kStMismatch = 5;
constexpr int32_t kStLimit = 8;  // whole-row nucleus cut deeper than the kMaxK best

// Rows of controls a sampling launch can carry in its own arguments.
constexpr uint32_t kInlineRows = 64;

struct SampleArgs {
  const float* logits;
  uint64_t lstride;
  const uint32_t* counts;
  uint64_t cstride;
  const float* uniforms;
  RowParams* params;      // the device table of controls (read, or written from inline)
  uint32_t vocab;
  uint32_t rows;
  uint32_t chunks;      // workgroups per row
  uint32_t wave_elems;  // elements per wave slice of chunks < split (multiple of 4)
  uint32_t wave_elems_b;  // elements per wave slice of chunks >= split (multiple of 4)
  uint32_t pace;          // 1: waves step their issue priority down as they progress
  uint32_t split;         // chunks [0, split) run in the grid's first half, the
                          // rest in its second half (split == chunks: one layout)
  uint32_t logprobs;
  uint32_t finisher;      // bits 0-7: c + 1, chunk c finishes each row (tagged
                          // words, no counter), 0 the last arriver does; bits
                          // 16-28: the launch's epoch (1..kMaxEpoch)
  uint32_t wait_ticks;    // finisher hand-off: wait limit, s_memrealtime ticks
  uint32_t* tokens;
  float* token_logits;
  int32_t* row_status;
  float* penalised;
  float* lp_values;
  uint32_t* lp_ids;
  // workspace, indexed by wave slot = (row * chunks + chunk) * kWaves + wave
  uint64_t* cand;        // [slot][kMaxK] top-kk composites of the wave, descending, 0 = empty
  uint64_t* greedy;      // [slot] greedy composite
  uint64_t* spec;        // [slot] the wave's speculative stream key (0 = none; a
                         // tagged word in the finisher hand-off)
  double* lse;           // [slot][2] (max s, sum exp((s - max)/T))
  double* zsum;          // [slot][3] whole-row nucleus mass (max, sum, error bound)
  uint32_t* row_done;    // [rows * kLineWords] arrivals, one cache line per row,
                         // reset by the last workgroup
  uint64_t* trace;       // FG_SAMPLE_TRACE builds only: [workgroup][16] timestamps
  // Controls carried by value (inline > 0): rows [0, inline) of the table,
  // read from here and written to `params` by workgroup 0 for later
  // launches that read the table.
  uint32_t inline_rows;
  RowParams row_inline[kInlineRows];
};

// Row r's controls (r wave-uniform), read with scalar loads from one place
// or the other under a uniform branch.  A launch reads the table only when
// it carries no controls of its own, so the table never changes while it is
// read: it is read as constant memory (scalar loads, whatever the launch
// stores elsewhere).  The empty asm keeps the two loads apart: merged into
// one load from a selected address, the load would be a flat, per-lane one.
typedef const __attribute__((address_space(4))) RowParams* ConstRowParams;
__device__ __forceinline__ RowParams row_controls(const SampleArgs& a, uint32_t r) {
  RowParams p;
  if (a.inline_rows) {
    p = a.row_inline[r];
    asm volatile("" ::: "memory");
  } else {
#if defined(__HIP_DEVICE_COMPILE__)
    const ConstRowParams q = (ConstRowParams)(a.params) + r;
    p.temperature = q->temperature;
    p.top_p = q->top_p;
    p.top_k = q->top_k;
    p.presence = q->presence;
    p.frequency = q->frequency;
    p.repetition = q->repetition;
    p.flags = q->flags;
    p.reserved = q->reserved;
#else
    p = a.params[r];
#endif
  }
  return p;
}
// Workgroup 0 of a launch with inline controls writes them to the table.
__device__ __forceinline__ void store_inline_controls(const SampleArgs& a) {
  if (a.inline_rows && blockIdx.x == 0u && threadIdx.x < a.inline_rows)
    a.params[threadIdx.x] = a.row_inline[threadIdx.x];
}

// Phase timestamps (s_memrealtime, 100 MHz) for builds with FG_SAMPLE_TRACE;
// compiled out otherwise.
// The stamps go to LDS and are copied out where the workgroup's work ends
// (FG_TRACE_FLUSH): a global store per stamp would make the compiler wait for
// its completion before reusing the stamp's registers.
#ifdef FG_SAMPLE_TRACE
#define FG_TRACE_DECL __shared__ uint64_t s_trace[16]
#define FG_TRACE_INIT                                     \
  do {                                                    \
    if (threadIdx.x == 0)                                 \
      for (int i_ = 0; i_ < 16; i_++) s_trace[i_] = 0ull; \
  } while (0)
#define FG_TRACE(a, slot)                                              \
  do {                                                                 \
    if (threadIdx.x == 0) s_trace[slot] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#define FG_TRACE_FLUSH(a)                                                      \
  do {                                                                         \
    if (threadIdx.x == 0 && (a).trace)                                         \
      for (int i_ = 0; i_ < 16; i_++)                                          \
        (a).trace[static_cast<uint64_t>(blockIdx.x) * 16u + i_] = s_trace[i_]; \
  } while (0)
// Event counters of FG_SAMPLE_TRACE builds (FG_SAMPLE_COUNT also set; they
// slow the launch down): g_trace_counters[i].
__device__ uint64_t* g_trace_counters;
#else
#define FG_TRACE_DECL static_assert(true, "")
#define FG_TRACE_INIT \
  do {                \
  } while (0)
#define FG_TRACE(a, slot) \
  do {                    \
  } while (0)
#define FG_TRACE_FLUSH(a) \
  do {                    \
  } while (0)
#endif
#if defined(FG_SAMPLE_TRACE) && defined(FG_SAMPLE_COUNT)
#define FG_COUNT(i, v)                                                             \
  do {                                                                             \
    if (g_trace_counters && lane_id() == 0) atomicAdd(&g_trace_counters[i], (v));  \
  } while (0)
#else
#define FG_COUNT(i, v) \
  do {                 \
  } while (0)
#endif

// Device-coherent (sc1) accesses for the cross-workgroup hand-off.
template <typename T>
__device__ __forceinline__ void store_coherent(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T load_coherent(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent_f64(double* p, double v) {
  store_coherent(reinterpret_cast<uint64_t*>(p), static_cast<uint64_t>(__double_as_longlong(v)));
}
__device__ __forceinline__ double load_coherent_f64(const double* p) {
  return __longlong_as_double(
      static_cast<long long>(load_coherent(reinterpret_cast<const uint64_t*>(p))));
}

// ---- per-wave top list ------------------------------------------------------
//
// Each wave keeps its best 64 composites so far as one sorted register list
// (lane i holds the i-th best, descending; 0 = empty).  Streamed candidates
// that beat the filter R are staged in wave-private LDS; every 64 staged
// entries are sorted across the lanes and merged into the list.  R rises to
// the list's kk-th entry after each merge: nothing at or below it can enter
// the top-kk.

constexpr uint64_t kRawTag = 1ull << 63;  // a staged raw entry; composites stay below 2^63

struct TopList {
  uint64_t top;    // lane i: i-th best composite
  uint64_t R;      // filter: a candidate must be > R (wave-uniform)
  uint64_t* buf;   // kCap staged composites + one spare slot per lane (wave-private LDS)
  uint32_t n;      // staged entries (wave-uniform)
  uint32_t kk;     // entries of the list that matter (1..64)
  float fM;        // float form of R for elements later in the stream
  uint32_t* wg_key;  // LDS, shared by the workgroup's waves: the largest key K
                     // such that some wave holds kk composites with key >= K
  uint32_t shared;   // largest key this wave has published
};

// Raises R.  For an element later in the stream than every list member, a
// key above comp_key(R) is needed (a tie on the key loses on the id), so the
// stream filter is v >= fM with fM the float of key comp_key(R) + 1; it may
// let a few extra values through (-0 against +0), never too few.
__device__ __forceinline__ void top_raise(TopList& t, uint64_t R) {
  if (R <= t.R) return;
  t.R = R;
  const uint32_t m = comp_key(R) + 1u;
  t.fM = m < 0x00800000u ? -3.402823466e38f : key_to_float(m);
}

// The workgroup's waves share their bounds: kk composites with key >= K in
// one wave mean that no element with a lower key, in any wave of the row, is
// in the row's top-kk.  Ties on K are kept (their ids may rank either way).
// (Sharing across the row's workgroups through a global atomic measured
// slower: a slice is a few steps long, so the bound arrives after most of its
// staging is done.)
__device__ __forceinline__ void top_share(TopList& t, uint32_t key) {
  if (key <= t.shared) return;
  t.shared = key;
  if (lane_id() == 0) atomicMax(t.wg_key, key);
}
__device__ __forceinline__ void top_adopt(TopList& t) {
  const uint32_t K = __hip_atomic_load(t.wg_key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  if (K) top_raise(t, key_floor(K));
}

__device__ __forceinline__ void top_merge_sorted(TopList& t, uint64_t sorted_desc) {
  t.top = wave_merge_desc(t.top, sorted_desc);
  const uint64_t kth = readlane64(t.top, t.kk - 1u);
  top_raise(t, kth);
  top_share(t, comp_key(kth));
}

__device__ __forceinline__ uint64_t staged_comp(uint64_t x) {
  return (x & kRawTag) ? make_comp(float_key(__uint_as_float(static_cast<uint32_t>(x))),
                                   static_cast<uint32_t>(x >> 32) & 0x7fffffffu)
                       : x;
}

// Drops the staged entries that no longer beat R, keeping the rest in
// order at the front of the stage (a chunk is read before anything is
// written over it).
__device__ __forceinline__ void top_compact(TopList& t) {
  const uint32_t lane = lane_id();
  uint32_t w = 0u;
  for (uint32_t c = 0; c < t.n; c += kWave) {
    const uint64_t x = c + lane < t.n ? staged_comp(t.buf[c + lane]) : 0ull;
    wave_lds_sync();
    const bool keep = x > t.R;
    const uint64_t m = ballot(keep);
    if (keep) t.buf[w + lanes_below(m)] = x;
    w += static_cast<uint32_t>(__popcll(m));
    wave_lds_sync();
  }
  t.n = w;
}

// Raises the filter from the staged entries alone and drops those it beats,
// without sorting: the kk-th largest of the lanes' maximum staged keys (a
// ballot radix search, to 2^12 key units) has at least kk staged entries at
// or above it.  Cheaper than sorting 64 entries into the list, it usually
// leaves fewer than 64 staged.
__device__ __forceinline__ void top_select(TopList& t) {
  const uint32_t lane = lane_id();
  uint32_t kmax = 0u;
  for (uint32_t i = lane; i < t.n; i += kWave) {
    const uint32_t k = comp_key(staged_comp(t.buf[i]));
    kmax = k > kmax ? k : kmax;
  }
  uint32_t T = 0u;
#pragma unroll
  for (int b = 31; b >= 12; b--) {
    const uint32_t c = T | (1u << b);
    if (static_cast<uint32_t>(__popcll(ballot(kmax >= c))) >= t.kk) T = c;
  }
  if (T) {
    top_raise(t, key_floor(T));
    top_share(t, T);
  }
  top_compact(t);
}

// Moves staged entries into the list: whole groups of 64, or everything when
// `all` is set.  While streaming (kk <= 32), a full stage is first thinned by
// top_select; only what still fills 64 entries is sorted in.  (For larger kk
// the lanes' maxima rarely raise the filter.)  An empty list takes a sorted
// group as it is.
__device__ __forceinline__ void top_drain(TopList& t, bool all) {
  const uint32_t lane = lane_id();
  if (!all && t.kk <= 32u && t.n >= static_cast<uint32_t>(kWave)) top_select(t);
  while (t.n >= static_cast<uint32_t>(kWave) || (all && t.n > 0u)) {
    const uint32_t take = t.n < static_cast<uint32_t>(kWave) ? t.n : static_cast<uint32_t>(kWave);
    const uint32_t at = t.n - take;
    uint64_t x = lane < take ? t.buf[at + lane] : 0ull;
    wave_lds_sync();
    t.n = at;
    x = staged_comp(x);
    if (x <= t.R) x = 0ull;  // beaten by a list that grew after it was staged
    if (ballot(x != 0ull) == 0ull) continue;
    FG_COUNT(all ? 3 : 0, 1ull);
    const uint64_t sorted = wave_sort_desc_first(x, take);
    if (ballot(t.top != 0ull) == 0ull) {
      t.top = sorted;
      const uint64_t kth = readlane64(t.top, t.kk - 1u);
      top_raise(t, kth);
      top_share(t, comp_key(kth));
    } else {
      top_merge_sorted(t, sorted);
    }
  }
}

// The final drain of a list of at most 32 when the list is still empty and
// 17-64 entries are staged (the usual case at top-k 20: while streaming,
// top_select thins the stage instead of sorting it).  Each staged entry's
// rank among the others is counted in one pass over the stage, and the kk
// best are written at their ranks into the spare slots: a few LDS rounds and
// ~2n VALU operations instead of a 64-entry bitonic sort (21 dependent
// exchange steps).  It keeps the same entries as top_drain, in the same
// order (staged entries are distinct: one per element).  Returns false,
// changing nothing, in the other cases (measured: config 2 19.50 -> 19.34
// us; the whole-row nucleus at top-k 64, few staged, slowed by 1 us when it
// took this path).
__device__ __forceinline__ bool top_drain_rank(TopList& t) {
  const uint32_t n = t.n;
  if (t.kk > 32u || n <= 16u || n > static_cast<uint32_t>(kWave) || ballot(t.top != 0ull) != 0ull)
    return false;
  const uint32_t lane = lane_id();
  uint64_t x = lane < n ? staged_comp(t.buf[lane]) : 0ull;
  if (x <= t.R) x = 0ull;  // beaten by a list that grew after it was staged
  uint64_t* const out = t.buf + kCap;
  wave_lds_sync();
  t.buf[lane] = x;
  out[lane] = 0ull;
  wave_lds_sync();
  // The stage is scanned in blocks of 32 (zeros past n count nothing), each
  // block's reads issued together: a loop of dependent reads would pay the
  // LDS latency per iteration.
  uint32_t r = 0u;
  for (uint32_t b = 0; b < 2u; b++) {
    if (b * 32u >= n) break;
    uint64_t y[32];
#pragma unroll
    for (int j = 0; j < 32; j++) y[j] = t.buf[b * 32u + j];
#pragma unroll
    for (int j = 0; j < 32; j++) r += y[j] > x ? 1u : 0u;
  }
  if (x != 0ull && r < t.kk) out[r] = x;
  wave_lds_sync();
  t.top = out[lane];
  wave_lds_sync();
  t.n = 0u;
  top_raise(t, readlane64(t.top, t.kk - 1u));
  return true;
}

// Stages this lane's composite if it beats R.  The caller keeps n + 64 <= kCap.
__device__ __forceinline__ void top_stage(TopList& t, uint64_t comp) {
  const bool pass = comp > t.R;
  const uint64_t m = ballot(pass);
  if (m == 0ull) return;
  if (pass) t.buf[t.n + lanes_below(m)] = comp;
  t.n += static_cast<uint32_t>(__popcll(m));
}

// Stream form: stages value v (element `id`, later in the stream than every
// list member) when it passes the float filter f (fM, or a higher
// speculative filter).  The entry is staged raw
// (id << 32 | float bits, marked by kRawTag) and becomes a composite when it
// is drained: the per-element cost stays a compare, a count and one store.
// +Inf passes the filter and is dropped at the drain (its key is 0).
__device__ __forceinline__ void top_stage_stream(TopList& t, float v, uint32_t id, float f) {
  const bool pass = v >= f;  // f is NaN for masked elements
  const uint64_t m = __builtin_amdgcn_ballot_w64(pass);
  if (m == 0ull) return;
  FG_COUNT(1, static_cast<unsigned long long>(__popcll(m)));
  // Every lane stores: those that fail to their own spare slot past kCap.
  const uint32_t slot = pass ? t.n + lanes_below(m) : kCap + lane_id();
  t.buf[slot] = kRawTag | (static_cast<uint64_t>(id) << 32) | __float_as_uint(v);
  t.n += static_cast<uint32_t>(__popcll(m));
}

// Value order of src/sampler.c:75-78 (value desc, id asc) as a composite:
// -0 folds onto +0 because the reference compares floats.
__device__ __forceinline__ uint64_t value_comp_from(uint64_t key_comp) {
  if (key_comp == 0ull) return 0ull;
  uint32_t k = comp_key(key_comp);
  if (k == 0x7fffffffu) k = 0x80000000u;  // key(-0) -> key(+0)
  return (static_cast<uint64_t>(k) << 31) | (key_comp & 0x7fffffffull);
}

// A key-ordered list re-ordered by value: only -0 entries can move.
__device__ __forceinline__ uint64_t value_order(uint64_t key_sorted) {
  const uint64_t v = value_comp_from(key_sorted);
  if (ballot(key_sorted != 0ull && comp_key(key_sorted) == 0x7fffffffu) == 0ull) return v;
  return wave_sort_desc(v);
}

// Combines per-lane (max s, sum exp((s - max)/T)) pairs of a wave in f64.
__device__ __forceinline__ void wave_lse_combine(double m, double z, double t, double* wm,
                                                 double* wz) {
  const double mm = wave_max_f64(m);
  const double zz = (m == -INFINITY) ? 0.0 : z * exp((m - mm) / t);
  *wm = mm;
  *wz = wave_sum_f64(zz);
}

// Folds one (max, sum exp((s - max)/t)) partial into a running pair.
__device__ __forceinline__ void lse_accumulate(double& m, double& z, double mi, double zi, double t) {
  if (mi == -INFINITY) return;
  if (mi > m) {
    z = (m == -INFINITY) ? 0.0 : z * exp((m - mi) / t);
    m = mi;
  }
  z += zi * exp((mi - m) / t);
}

// Whole-row mass for a nucleus row: (max s, z = sum exp(s - max), e = sum
// exp(s - max) * (max - s)).  The terms are f32 exp2, each within
// 1.2e-7 + 1.8e-7 |s - max| of exp (one ulp of v_exp_f32, plus the rounding of
// s - max, of log2(e) and of the product), so e bounds their error.  A
// streaming step (four quads per lane in launches with whole-row nucleus
// rows) sums its 16 terms per lane pairwise in f32 (four roundings,
// 2.4e-7 of the step's sum) before adding them in f64, so z is within
// 3.6e-7 z + 1.8e-7 e of the exact sum.
struct Mass {
  double m, z, e;
};

// Folds (mi, zi, ei) into a running mass (rescaling the one with the lower
// max: exp(-d) z and exp(-d) (e + d z)).
__device__ __forceinline__ void mass_accumulate(Mass& a, double mi, double zi, double ei) {
  if (mi == -INFINITY) return;
  if (mi > a.m) {
    if (a.m == -INFINITY) {
      a.z = a.e = 0.0;
    } else {
      const double d = mi - a.m, f = exp(-d);
      a.e = f * (a.e + d * a.z);
      a.z = f * a.z;
    }
    a.m = mi;
  }
  const double d = a.m - mi, f = exp(-d);
  a.z += f * zi;
  a.e += f * (ei + d * zi);
}

__device__ __forceinline__ Mass wave_mass_combine(double m, double z, double e) {
  const double mm = wave_max_f64(m);
  double zz = 0.0, ee = 0.0;
  if (m != -INFINITY) {
    const double d = mm - m, f = exp(-d);
    zz = f * z;
    ee = f * (e + d * z);
  }
  return Mass{mm, wave_sum_f64(zz), wave_sum_f64(ee)};
}

// ---- the row's final step (one wave) ---------------------------------------

// fin: lane i holds the row's i-th best composite in key order (0 past the
// end); gbest: the row's greedy composite; (m, z): the row's tempered
// log-sum-exp pair for log-probs; zs: the row's untempered mass for a
// whole-row nucleus.  Writes token, logit, status and log-probs.
__device__ inline int32_t finish_row(const SampleArgs& a, const RowParams& p, uint32_t row,
                                  uint64_t fin, uint64_t gbest, double m, double z, Mass zs,
                                  const float* lrow, const uint32_t* crow, bool pen, float u,
                                  double inv_t) {
  const uint32_t lane = lane_id();
  const bool greedy = p.temperature == 0.0f;
  const uint32_t L = a.logprobs;
  const bool nuc = !greedy && p.top_k == 0u;
  const uint32_t kk = greedy ? L : nuc ? kMaxK : (p.top_k > L ? p.top_k : L);
  fin = lane < kk ? fin : 0ull;  // past kk the lists are not exact
  int32_t status = kStOk;
  uint32_t token = kInvalidId;
  float token_logit = -INFINITY;

  if (greedy) {
    // src/output.c:560-599 / 728-741: a non-finite winner is an error.
    const uint32_t id = greedy_id(gbest);
    const uint32_t hi = static_cast<uint32_t>(gbest >> 32);
    float v = -INFINITY;
    if (gbest != 0ull && id < a.vocab) {
      if (hi != 0xffffffffu && hi != 0x80000000u) {
        v = key_to_float(hi);  // the penalised value itself
      } else {
        // Non-finite, or a zero whose sign the composite folded: re-read.
        v = lrow[id];
        if (pen) v = penalise(v, crow[id], p.presence, p.frequency, p.repetition);
      }
    }
    token_logit = v;
    if (gbest == 0ull || !is_finite_bits(__float_as_uint(v)))
      status = pen ? kStFormat : kStMismatch;
    else
      token = id;
  } else {
    // fg_sampler_select (src/sampler.c:80-122) over the exact top_k, in value
    // order; the f64 running sums are parallel prefix sums.  A whole-row
    // nucleus (top_k 0) runs the same steps with limit = every finite logit:
    // its raw sum is the row's mass zz, and the cut must fall inside the
    // kMaxK best (or the row has no more finite logits than that).
    const uint32_t topk = nuc ? kMaxK : p.top_k;
    const uint64_t sorted = value_order(lane < topk ? fin : 0ull);
    const uint32_t kept = static_cast<uint32_t>(__popcll(ballot(sorted != 0ull)));
    if (kept == 0u) {
      status = kStFormat;
    } else {
      const uint32_t limit = topk < kept ? topk : kept;
      const bool whole_row_listed = nuc && kept < kMaxK;
      const bool live = lane < limit;
      const double v = live ? static_cast<double>(key_to_float(comp_key(sorted))) : 0.0;
      const double vmax = __longlong_as_double(static_cast<long long>(
          readlane64(static_cast<uint64_t>(__double_as_longlong(v)), 0)));
      // Both running sums at once (independent chains): the tempered one is
      // read at the cut, and a prefix sum up to a lane ignores later lanes.
      // Every lane runs both exps (exp(-inf) = 0 past the list), so the two
      // chains interleave instead of running one after the other.
      const double d = live ? v - vmax : -INFINITY;
      const double e = exp(d);
      const double te = exp(d * inv_t);
      // Lists of at most 32 (every top-k up to 32) have no terms past lane
      // 31: the scans over two rows of 16 skip the upper rows' offsets.
      double ecum, tcum;
      if (topk <= 32u) {
        ecum = wave_prefix_sum_f64_lo32(e);
        tcum = wave_prefix_sum_f64_lo32(te);
      } else {
        ecum = wave_prefix_sum_f64(e);
        tcum = wave_prefix_sum_f64(te);
      }
      double sum = __longlong_as_double(static_cast<long long>(
          readlane64(static_cast<uint64_t>(__double_as_longlong(ecum)), limit - 1u)));
      // Relative error bound of the f32-term mass (see Mass).
      double bound = 0.0;
      if (nuc && !whole_row_listed) {
        sum = zs.z * exp(zs.m - vmax);
        bound = 3.6e-7 + 1.8e-7 * (zs.e / zs.z);
      }
      if (!(sum > 0.0) || !isfinite(sum)) {
        status = kStFormat;
      } else {
        // Running probability ecum / sum against top_p, as ecum >= top_p * sum
        // (the reference sums the quotients; both differ by rounding only).
        const double target = static_cast<double>(p.top_p) * sum;
        const uint64_t hit = ballot(live && ecum >= target);
        uint32_t cutoff = hit ? static_cast<uint32_t>(__builtin_ctzll(hit)) + 1u : limit;
        // A deeper cut, or a list that ends on zeros (where key order, +0
        // above -0, and value order, 0 == -0, may keep different entries),
        // is left to the deep-row kernel.
        if (nuc && !whole_row_listed) {
          const uint32_t edge_key = comp_key(readlane64(fin, kMaxK - 1u));
          const bool zero_edge = edge_key == 0x7fffffffu || edge_key == 0x80000000u;
          // So is a cut that the mass's error bound could move: the positions
          // either side of the cut must clear top_p by twice the bound.
          const double gap = lane < cutoff ? fabs(ecum - target) / sum : INFINITY;
          const bool close = -wave_max_f64(-gap) <= 2.0 * bound;
          if (hit == 0ull || zero_edge || close) status = kStLimit;
        }
        const double tsum = __longlong_as_double(static_cast<long long>(
            readlane64(static_cast<uint64_t>(__double_as_longlong(tcum)), cutoff - 1u)));
        if (status != kStOk) {
          // whole-row nucleus cut below the kMaxK best: no token
        } else if (!(tsum > 0.0) || !isfinite(tsum)) {
          status = kStFormat;
        } else {
          if (!is_finite_bits(__float_as_uint(u)) || u < 0.0f) u = 0.0f;
          if (u >= 1.0f) u = __uint_as_float(0x3f7fffffu);  // nextafterf(1, 0)
          const double draw = static_cast<double>(u) * tsum;
          const uint64_t hit2 = ballot(lane < cutoff && draw < tcum);
          const uint32_t pick = hit2 ? static_cast<uint32_t>(__builtin_ctzll(hit2)) : cutoff - 1u;
          const uint64_t picked = readlane64(sorted, pick);
          token = comp_id(picked);
          if (comp_key(picked) != 0x80000000u) {
            token_logit = key_to_float(comp_key(picked));  // the value's own key
          } else {
            // A zero keeps its sign: read it from the key-order list.
            const uint64_t owner = ballot(fin != 0ull && comp_id(fin) == token);
            token_logit = key_to_float(
                comp_key(readlane64(fin, static_cast<uint32_t>(__builtin_ctzll(owner)))));
          }
        }
      }
    }
  }

  if (L) {
    const double te = static_cast<double>(p.temperature > 0.0f ? p.temperature : 1.0f);
    const double lse = m / te + log(z);
    const uint64_t vs = value_order(fin);
    if (lane < L) {
      float lp = -INFINITY;
      uint32_t id = kInvalidId;
      if (vs != 0ull) {
        id = comp_id(vs);
        lp = static_cast<float>(static_cast<double>(key_to_float(comp_key(vs))) / te - lse);
      }
      a.lp_values[static_cast<uint64_t>(row) * L + lane] = lp;
      a.lp_ids[static_cast<uint64_t>(row) * L + lane] = id;
    }
  }
  if (lane == 0) {
    a.tokens[row] = token;
    if (a.token_logits) a.token_logits[row] = token_logit;
    if (a.row_status) a.row_status[row] = status;
  }
  return status;
}

// ---- streaming ---------------------------------------------------------------

// Which parts of the pass a launch needs (the union over its rows).  Each
// combination is its own instantiation, so a launch carries only its code.
template <bool kVec_, bool kPen_, bool kGreedy_, bool kTop_, bool kLse_, bool kNuc_,
          bool kSpec_>
struct Features {
  static constexpr bool kVec = kVec_;      // 16-byte aligned rows: vector loads
  static constexpr bool kPen = kPen_;      // some row applies penalties
  static constexpr bool kGreedy = kGreedy_;  // some row is greedy
  static constexpr bool kTop = kTop_;      // some row keeps a top list
  static constexpr bool kLse = kLse_;      // log-probs requested
  static constexpr bool kNuc = kNuc_;      // some row is a whole-row nucleus (top_k 0)
  static constexpr bool kSpec = kSpec_;    // some top list is longer than kSpecMinK
  // Quads per lane per streaming step: 2 (512 elements) for launches
  // without speculation or whole-row nucleus rows, 4 otherwise (measured:
  // config 2 21.9 -> 21.1 us at 512, config 4 greedy 22.4 -> 21.8; top-k 64
  // 23.1 -> 23.6 and config 3 79 -> 85 would lose).
  static constexpr int kStepVec = (kSpec_ || kNuc_) ? 4 : 2;
};

template <bool kVec>
__device__ __forceinline__ void load_quad(const float* lrow, const uint32_t* crow, bool pen,
                                          uint32_t q, f4& x, u4& y) {
  const uint32_t i = q * 4u;
  if (kVec) {
    x = __builtin_nontemporal_load(reinterpret_cast<const f4*>(lrow + i));
    y = pen ? __builtin_nontemporal_load(reinterpret_cast<const u4*>(crow + i))
            : u4{0u, 0u, 0u, 0u};
  } else {
    x = f4{lrow[i], lrow[i + 1], lrow[i + 2], lrow[i + 3]};
    y = pen ? u4{crow[i], crow[i + 1], crow[i + 2], crow[i + 3]} : u4{0u, 0u, 0u, 0u};
  }
}

// Vector path: raw buffer loads over the wave's slice.  The descriptor's
// range ends at the slice's last quad, so a load past it returns zeros
// without a memory request: the double-buffered loop loads the "next" step
// unconditionally, and the step after the slice costs nothing to wait for.
constexpr int32_t kBufferWord3 = 0x00020000;  // 32-bit data format, raw access
constexpr int32_t kLoadNT = 2;                // non-temporal (streamed once)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slice_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           kBufferWord3);
}
__device__ __forceinline__ void load_quad_buf(__amdgpu_buffer_rsrc_t rl, __amdgpu_buffer_rsrc_t rc,
                                              bool pen, uint32_t qrel, f4& x, u4& y) {
  // Counts are always loaded: without penalties rc has no records, so the
  // load returns zeros without touching memory (and needs no branch).
  (void)pen;
  x = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rl, qrel * 16u, 0, kLoadNT));
  y = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(rc, qrel * 16u, 0, kLoadNT));
}

struct WaveState {
  TopList t;
  float gv;      // greedy: best value seen by this lane (stream order breaks ties)
  uint32_t gid;  // greedy: its id
  uint32_t gnf;  // greedy: first non-finite id seen by this lane
  float lm;      // per-lane max of finite s
  float lz;      // per-lane sum exp2((s - lm) * log2e / T)
  float nm;      // nucleus: per-lane max of finite s
  double nz;     // nucleus: per-lane sum of f32 terms exp(s - nm)
  double ne;     // nucleus: per-lane sum exp(s - nm) (nm - s), the error bound
  bool first;
  uint32_t KS;   // speculative key: only elements with key >= KS are staged
  float fS;      // its float form (elements v >= fS are staged)
};

// Greedy update for one element in stream order (ids rise along a lane).
__device__ __forceinline__ void greedy_stream(WaveState& st, bool valid, float v, uint32_t id) {
  const bool bad = valid && !is_finite_bits(__float_as_uint(v));
  st.gnf = (bad && st.gnf == kInvalidId) ? id : st.gnf;
  const bool gt = valid && v > st.gv;
  st.gv = gt ? v : st.gv;
  st.gid = gt ? id : st.gid;
}

// Greedy update for an element that may come out of stream order.
__device__ __forceinline__ void greedy_any(WaveState& st, bool valid, float v, uint32_t id) {
  if (!valid) return;
  if (!is_finite_bits(__float_as_uint(v))) {
    st.gnf = id < st.gnf ? id : st.gnf;
    return;
  }
  if (v > st.gv || st.gid == kInvalidId || (v == st.gv && id < st.gid)) {
    st.gv = v;
    st.gid = id;
  }
}

__device__ __forceinline__ uint64_t greedy_lane_comp(const WaveState& st) {
  if (st.gnf != kInvalidId) return (0xffffffffull << 32) | static_cast<uint64_t>(~st.gnf);
  return st.gid != kInvalidId ? greedy_comp(st.gv, st.gid) : 0ull;
}

// One streaming step: x/y hold quads q0 + j*64 + lane (j < F::kStepVec); quads
// at or past q_end are clamped duplicates and are masked out.
template <class F>
__device__ __forceinline__ void process_step(WaveState& st, const RowParams& p, bool pen,
                                             bool greedy, bool lse, bool nuc, bool spec,
                                             float log2e_over_t,
                                             float* prow, const f4* x, const u4* y, uint32_t q0,
                                             uint32_t q_end) {
  const uint32_t lane = lane_id();
  float v[F::kStepVec][4];
  bool ok[F::kStepVec];
#pragma unroll
  for (int j = 0; j < F::kStepVec; j++) {
    const uint32_t q = q0 + j * kWave + lane;
    ok[j] = q < q_end;
    v[j][0] = x[j].x;
    v[j][1] = x[j].y;
    v[j][2] = x[j].z;
    v[j][3] = x[j].w;
  }
  if (F::kPen && pen) {
    // Penalties touch only elements with a nonzero count (sparse): a 64-lane
    // slot pays for the IEEE division only when one of its lanes needs it,
    // and then without branches.
#pragma unroll
    for (int j = 0; j < F::kStepVec; j++) {
      const uint32_t c4[4] = {y[j].x, y[j].y, y[j].z, y[j].w};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        if (__builtin_amdgcn_ballot_w64(c4[e] != 0u) != 0ull)
          v[j][e] = penalise_sel(v[j][e], c4[e], p.presence, p.frequency, p.repetition);
      }
    }
  }
  if (prow) {
#pragma unroll
    for (int j = 0; j < F::kStepVec; j++)
      if (ok[j]) {
        const uint32_t q = q0 + j * kWave + lane;
#pragma unroll
        for (int e = 0; e < 4; e++) prow[q * 4u + e] = v[j][e];
      }
  }
  if (F::kGreedy && greedy) {
#pragma unroll
    for (int j = 0; j < F::kStepVec; j++) {
      const uint32_t q = q0 + j * kWave + lane;
#pragma unroll
      for (int e = 0; e < 4; e++) greedy_stream(st, ok[j], v[j][e], q * 4u + e);
    }
  }
  if (F::kLse && lse) {
    float step_max = -INFINITY;
#pragma unroll
    for (int j = 0; j < F::kStepVec; j++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (ok[j] && is_finite_bits(__float_as_uint(v[j][e]))) step_max = fmaxf(step_max, v[j][e]);
    if (step_max > st.lm) {
      st.lz = (st.lm == -INFINITY) ? 0.0f : st.lz * exp2f((st.lm - step_max) * log2e_over_t);
      st.lm = step_max;
    }
#pragma unroll
    for (int j = 0; j < F::kStepVec; j++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (ok[j] && is_finite_bits(__float_as_uint(v[j][e])))
          st.lz += exp2f((v[j][e] - st.lm) * log2e_over_t);
  }
  if (F::kNuc && nuc) {
    float step_max = -INFINITY;
#pragma unroll
    for (int j = 0; j < F::kStepVec; j++)
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (ok[j] && is_finite_bits(__float_as_uint(v[j][e]))) step_max = fmaxf(step_max, v[j][e]);
    if (step_max > st.nm) {
      if (st.nm == -INFINITY) {
        st.nz = st.ne = 0.0;
      } else {
        const double d = static_cast<double>(step_max) - static_cast<double>(st.nm);
        const double f = exp(-d);
        st.ne = f * (st.ne + d * st.nz);
        st.nz = f * st.nz;
      }
      st.nm = step_max;
    }
    // The step's f32 terms summed pairwise in f32 (at most four roundings:
    // the mass bound assumes no more), then in f64; their error bound
    // sum w * (max - s) in f32.
    static_assert(F::kStepVec <= 4, "the nucleus mass bound covers 16 terms per step");
    float w[F::kStepVec * 4];
    float ef = 0.0f;
#pragma unroll
    for (int j = 0; j < F::kStepVec; j++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const bool use = ok[j] && is_finite_bits(__float_as_uint(v[j][e]));
        const float sd = use ? v[j][e] - st.nm : 0.0f;
        w[j * 4 + e] = use ? exp2f(sd * 1.4426950408889634f) : 0.0f;
        ef = fmaf(w[j * 4 + e], -sd, ef);
      }
#pragma unroll
    for (int h = F::kStepVec * 2; h >= 1; h /= 2)
#pragma unroll
      for (int i = 0; i < h; i++) w[i] = w[i] + w[i + h];
    st.nz += static_cast<double>(w[0]);
    st.ne += static_cast<double>(ef);
  }
  if (F::kTop && st.t.kk) {
    // The lane's largest value: +Inf counts here (it is dropped where it is
    // drained); NaN does not.
    float lane_max = -INFINITY;
#pragma unroll
    for (int j = 0; j < F::kStepVec; j++) {
      const float m = fmaxf(fmaxf(v[j][0], v[j][1]), fmaxf(v[j][2], v[j][3]));
      lane_max = ok[j] ? fmaxf(lane_max, m) : lane_max;
    }
    if (st.first) {
      // The kk-th largest lane maximum: at least kk keys of this step are >=
      // it, so it bounds the wave's kk-th key from below.  A lane whose
      // largest value is +Inf takes its largest finite key the long way.
      uint32_t lane_max_key = float_key(lane_max);
      if (ballot(lane_max == INFINITY) != 0ull) {
        lane_max_key = 0u;
#pragma unroll
        for (int j = 0; j < F::kStepVec; j++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const uint32_t key = ok[j] ? float_key(v[j][e]) : 0u;
            lane_max_key = key > lane_max_key ? key : lane_max_key;
          }
      }
      // Largest T (to 2^12 key units) with at least kk lane maxima >= T: a
      // ballot radix search, cheaper than sorting the 64 maxima.
      uint32_t T = 0u;
#pragma unroll
      for (int b = 31; b >= 12; b--) {
        const uint32_t c = T | (1u << b);
        if (static_cast<uint32_t>(__popcll(ballot(lane_max_key >= c))) >= st.t.kk) T = c;
      }
      if (T) top_raise(st.t, key_floor(T));
      top_share(st.t, T);
      if (spec) {
        // Speculation: stage only keys >= the m-th largest lane maximum of
        // this step, m a few more than the row's top-kk is expected to hold
        // here.  What it skips is checked when the row is merged: a wave
        // whose key lies above the row's kk-th is scanned again then.
        const uint32_t m = 7u;
        uint32_t S = 0u;
#pragma unroll
        for (int b = 31; b >= 12; b--) {
          const uint32_t c = S | (1u << b);
          if (static_cast<uint32_t>(__popcll(ballot(lane_max_key >= c))) >= m) S = c;
        }
        st.KS = S;
        st.fS = S >= 0x00800000u ? key_to_float(S) : -3.402823466e38f;
      }
      st.first = false;
    }
    top_adopt(st.t);  // the workgroup's bound (the other waves' first steps too)
    // Most steps hold no candidate once the filter has risen: one ballot on
    // the lane maxima (computed above) skips the per-element staging.
    const float f = F::kSpec ? fmaxf(st.t.fM, st.fS) : st.t.fM;
    if (ballot(lane_max >= f) != 0ull) {
      FG_COUNT(2, 1ull);
#pragma unroll
      for (int j = 0; j < F::kStepVec; j++) {
        const uint32_t q = q0 + j * kWave + lane;
        const float fj = ok[j] ? f : __builtin_nanf("");
#pragma unroll
        for (int e = 0; e < 4; e++) top_stage_stream(st.t, v[j][e], q * 4u + e, fj);
      }
      top_drain(st.t, false);
    }
  }
}

// ---- speculation check ------------------------------------------------------

// Wave slice i of a row (i = chunk * kWaves + wave): [begin, begin + len)
// clipped to the vocabulary.
__host__ __device__ inline uint32_t slice_begin_of(uint32_t i, uint32_t split, uint32_t ea,
                                                   uint32_t eb, uint32_t vocab) {
  const uint32_t na = split * kWaves;
  const uint32_t b = i < na ? i * ea : na * ea + (i - na) * eb;
  return b < vocab ? b : vocab;
}
__host__ __device__ inline uint32_t slice_end_of(uint32_t i, uint32_t split, uint32_t ea,
                                                 uint32_t eb, uint32_t vocab) {
  const uint32_t e = slice_begin_of(i, split, ea, eb, vocab) + (i < split * kWaves ? ea : eb);
  return e < vocab ? e : vocab;
}
__device__ __forceinline__ uint32_t slice_begin(const SampleArgs& a, uint32_t i) {
  return slice_begin_of(i, a.split, a.wave_elems, a.wave_elems_b, a.vocab);
}
__device__ __forceinline__ uint32_t slice_end(const SampleArgs& a, uint32_t i) {
  return slice_end_of(i, a.split, a.wave_elems, a.wave_elems_b, a.vocab);
}

// The row and chunk of workgroup b.  A row's chunks share one XCD (and its
// L2): the dispatcher hands workgroups to the kXcds XCDs round robin, so row
// r's chunks take blockIdx values of residue r % kXcds.  With split < chunks
// (rows a multiple of kXcds, two equal halves of chunks) chunks [0, split)
// sit in the grid's first half and the rest in its second: the
// first-dispatched workgroup of a CU streams faster than the second.  Rows
// past the last whole group of kXcds are laid out row-major after them.
// Only speed depends on the dispatch order; any order is correct.
__host__ __device__ inline void block_row_chunk(uint32_t b, uint32_t rows, uint32_t chunks,
                                                uint32_t split, uint32_t* row, uint32_t* chunk) {
  const uint32_t grouped = rows - rows % kXcds;
  if (split < chunks) {
    const uint32_t half = rows * split;  // workgroups per half
    const bool second = b >= half;
    const uint32_t bb = second ? b - half : b;
    const uint32_t hc = second ? chunks - split : split;
    const uint32_t q = bb / kXcds;
    const uint32_t g = q / hc;
    *row = g * kXcds + bb % kXcds;
    *chunk = q - g * hc + (second ? split : 0u);
  } else if (b < grouped * chunks) {
    const uint32_t q = b / kXcds;
    const uint32_t g = q / chunks;
    *row = g * kXcds + b % kXcds;
    *chunk = q - g * chunks;
  } else {
    const uint32_t r = (b - grouped * chunks) / chunks;
    *row = grouped + r;
    *chunk = b - grouped * chunks - r * chunks;
  }
}

// Reads wave slice `i` of the row again and merges into `fin` (the row's list)
// the elements the wave skipped under its speculative key ks that beat the
// list's kk-th entry.  One wave; `buf` is its free staging LDS.
__device__ inline uint64_t rescan_slice(const SampleArgs& a, const RowParams& p, bool pen,
                                        const float* lrow, const uint32_t* crow, uint64_t fin,
                                        uint32_t kk, uint32_t ks, uint32_t i, uint64_t* buf,
                                        uint32_t* wg_key) {
  const uint32_t lane = lane_id();
  const uint32_t wbegin = slice_begin(a, i);
  const uint32_t wend = slice_end(a, i);
  const float fS = ks >= 0x00800000u ? key_to_float(ks) : -3.402823466e38f;
  const uint64_t kth = readlane64(fin, kk - 1u);
  // shared = all ones: this list never publishes a workgroup bound.
  TopList t{fin, kth ? kth : kFiniteComp - 1ull, buf, 0u, kk, -3.402823466e38f, wg_key,
            0xffffffffu};
  constexpr uint32_t kPer = 16;
  for (uint32_t i0 = wbegin; i0 < wend; i0 += kPer * kWave) {
    float v[kPer];
    uint32_t c[kPer];
#pragma unroll
    for (uint32_t j = 0; j < kPer; j++) {
      const uint32_t idx = i0 + j * kWave + lane;
      const bool valid = idx < wend;
      v[j] = valid ? lrow[idx] : 0.0f;
      c[j] = valid && pen ? crow[idx] : 0u;
    }
#pragma unroll
    for (uint32_t j = 0; j < kPer; j++) {
      const uint32_t idx = i0 + j * kWave + lane;
      const bool valid = idx < wend;
      float x = v[j];
      if (c[j] != 0u) x = penalise(x, c[j], p.presence, p.frequency, p.repetition);
      // Exactly the elements the stream skipped for fS (x < fS); the others
      // were staged then or cannot enter the list.
      top_stage(t, valid && x < fS ? make_comp(float_key(x), idx) : 0ull);
    }
    // One drain call site (kept small: this path is rare); a round adds at
    // most 16 * 64 entries, which fit beside fewer than 64 left over.
    const bool last = i0 + kPer * kWave >= wend;
    if (last || t.n >= static_cast<uint32_t>(kWave)) top_drain(t, last);
  }
  return t.top;
}

// Every element a speculating wave skipped has a key below its key KS, so it
// cannot enter the row's top-kk when KS is at most the key of the list's
// kk-th entry; each wave of the row for which that fails is read again.
// ks_lds holds the keys when the row is one workgroup, else they are read
// from the workspace.
// The keys of waves 0..63 come in as ks0 (lane i: wave i), loaded early.
__device__ __forceinline__ uint32_t spec_key(const SampleArgs& a, uint32_t row, uint32_t i,
                                             const uint32_t* ks_lds) {
  const uint32_t n = a.chunks * static_cast<uint32_t>(kWaves);
  if (i >= n) return 0u;
  return a.chunks == 1u
             ? ks_lds[i]
             : static_cast<uint32_t>(load_coherent(a.spec + static_cast<uint64_t>(row) * n + i));
}

__device__ inline uint64_t spec_check(const SampleArgs& a, const RowParams& p, uint32_t row,
                                      bool pen, const float* lrow, const uint32_t* crow,
                                      uint64_t fin, uint32_t kk, const uint32_t* ks_lds,
                                      uint32_t ks0, uint64_t* buf, uint32_t* wg_key) {
  const uint32_t lane = lane_id();
  const uint32_t n = a.chunks * static_cast<uint32_t>(kWaves);
  for (uint32_t b = 0; b < n; b += kWave) {
    uint32_t ks = b == 0u ? ks0 : spec_key(a, row, b + lane, ks_lds);
    for (;;) {
      const uint32_t kkey = comp_key(readlane64(fin, kk - 1u));
      const uint64_t need = ballot(ks > kkey);
      if (need == 0ull) break;
      const uint32_t l = static_cast<uint32_t>(__builtin_ctzll(need));
      const uint32_t w_ks = readlane32(ks, l);
      FG_COUNT(4, 1ull);
      fin = rescan_slice(a, p, pen, lrow, crow, fin, kk, w_ks, b + l, buf, wg_key);
      if (lane == l) ks = 0u;
    }
  }
  return fin;
}

// ---- the finisher's tagged words ---------------------------------------------
//
// In the finisher hand-off the other chunks' lists (and greedy composites)
// travel as self-describing words: bit 63 set, bits 62-50 the launch's epoch
// (1-8191, advanced by the host every launch), bits 49-0 the payload,
// key << 18 | (2^18 - 1 - id) (larger payload = larger key, then lower id:
// the ladder's order; greedy words carry greedy_comp's high word as the
// key), 0 for an empty entry.  The finisher reads a word until it carries
// this launch's epoch, so slots are never cleared and a word stored late, by
// a launch whose finisher gave up, is never read as a later launch's; the
// host clears the workspace when the epoch wraps.  Ids must be below 2^18
// (larger vocabularies take the last-arriver hand-off).  A finisher that has
// not seen every word after the launch's wait limit (a.wait_ticks of the
// 100 MHz clock) reports kStTimeout for its row instead of a token.
constexpr int32_t kStTimeout = 7;     // FG_ERR_UNAVAILABLE: the finisher's wait gave up

// Payload of a composite (make_comp order); 0 stays 0.
__device__ __forceinline__ uint64_t wire_payload(uint64_t comp) {
  if (comp == 0ull) return 0ull;
  return (static_cast<uint64_t>(comp_key(comp)) << kWireIdBits) |
         static_cast<uint64_t>(kWireVocab - 1u - comp_id(comp));
}
__device__ __forceinline__ uint64_t comp_of_payload(uint64_t w) {
  if (w == 0ull) return 0ull;
  return make_comp(static_cast<uint32_t>(w >> kWireIdBits),
                   kWireVocab - 1u - static_cast<uint32_t>(w & (kWireVocab - 1u)));
}

// c + 1 when chunk c finishes each row (finisher hand-off), else 0.
__device__ __forceinline__ uint32_t finisher_of(const SampleArgs& a) { return a.finisher & 0xffu; }

// Whether the finisher's wait has passed its limit, at poll `spin` (0, 1,
// ...) of a wait whose first clock reading goes to t0.  The clock (a scalar
// memory read) is read at the first poll and every 32nd after it; a limit
// of 0 gives up at the first poll.
__device__ __forceinline__ bool wait_passed(const SampleArgs& a, uint32_t spin, uint64_t& t0) {
  if (a.wait_ticks == 0u) return true;
  if (spin % 32u) return false;
  const uint64_t now = __builtin_amdgcn_s_memrealtime();
  if (spin == 0u) t0 = now;
  return now - t0 > a.wait_ticks;
}

// The row's outputs when its finisher gave up waiting.
__device__ inline void timeout_row(const SampleArgs& a, uint32_t row) {
  if (lane_id() == 0u) {
    a.tokens[row] = kInvalidId;
    if (a.token_logits) a.token_logits[row] = -INFINITY;
    if (a.row_status) a.row_status[row] = kStTimeout;
  }
}

// ---- merging by rank ----------------------------------------------------------
//
// Lists of at most 32 entries are merged in LDS: every entry finds its rank
// in the union as the sum, over the lists, of the entries above it (a
// five-step binary search per list; the lists' searches are independent, so
// they overlap), and the entries ranked below kk are stored at their ranks.
// That is a few LDS round trips deep, where a bitonic merge tree runs six
// dependent exchange steps per level.  Entries are distinct within a row.

// Stores e (an entry of one of the kN descending lists at lists + i * stride,
// positions 0..31, zeros past their ends; or 0 for none) at out[rank] when
// its rank in their union is below kk.  The searches advance a step at a
// time over all lists, so each step's reads are issued together.
template <int kN>
__device__ __forceinline__ void rank_place(const uint64_t* lists, uint32_t stride, uint64_t e,
                                           uint32_t kk, uint64_t* out) {
  uint32_t lo[kN];
#pragma unroll
  for (int i = 0; i < kN; i++) lo[i] = lists[i * stride + 15u] > e ? 16u : 0u;
#pragma unroll
  for (uint32_t h = 8u; h >= 1u; h /= 2u) {
#pragma unroll
    for (int i = 0; i < kN; i++) lo[i] += lists[i * stride + lo[i] + h - 1u] > e ? h : 0u;
  }
  // The search tells 31 entries above e from 32 only with the last entry,
  // which is empty unless the lists hold 32.
  if (kk == 32u) {
#pragma unroll
    for (int i = 0; i < kN; i++) lo[i] += (lo[i] == 31u && lists[i * stride + 31u] > e) ? 1u : 0u;
  }
  uint32_t r = 0u;
#pragma unroll
  for (int i = 0; i < kN; i++) r += lo[i];
  if (e != 0ull && r < kk) out[r] = e;
}

// The same for lists of at most 64 entries (a six-step search; all 64
// entries above e are told from 63 by the last entry).
template <int kN>
__device__ __forceinline__ void rank_place64(const uint64_t* lists, uint32_t stride, uint64_t e,
                                             uint32_t kk, uint64_t* out) {
  uint32_t lo[kN];
#pragma unroll
  for (int i = 0; i < kN; i++) lo[i] = lists[i * stride + 31u] > e ? 32u : 0u;
#pragma unroll
  for (uint32_t h = 16u; h >= 1u; h /= 2u) {
#pragma unroll
    for (int i = 0; i < kN; i++) lo[i] += lists[i * stride + lo[i] + h - 1u] > e ? h : 0u;
  }
  if (kk == 64u) {
#pragma unroll
    for (int i = 0; i < kN; i++) lo[i] += (lo[i] == 63u && lists[i * stride + 63u] > e) ? 1u : 0u;
  }
  uint32_t r = 0u;
#pragma unroll
  for (int i = 0; i < kN; i++) r += lo[i];
  if (e != 0ull && r < kk) out[r] = e;
}

// The finisher's eight lists in LDS (lists past the row's chunk count
// empty, so with at most 4 chunks only lists 0-3 are searched).  Lists of at
// most 32 (list c at lists32 + 32 c): lanes 0-31 of wave w place the entries
// of list 2w, lanes 32-63 those of list 2w + 1.  Longer lists (list c at
// lists64 + 64 c): with at most 4 chunks wave w places list w's entries, a
// position per lane; else both of lists 2w and 2w + 1.
__device__ __forceinline__ void rank_place_lists(const uint64_t* lists32, const uint64_t* lists64,
                                                 uint32_t wave, uint32_t kk, uint32_t chunks,
                                                 uint64_t* out) {
  const uint32_t lane = lane_id();
  if (kk <= 32u) {
    const uint32_t c = 2u * wave + (lane >= 32u ? 1u : 0u);
    const uint32_t pos = lane & 31u;
    const uint64_t e = pos < kk ? lists32[c * 32u + pos] : 0ull;
    if (chunks <= 4u)
      rank_place<4>(lists32, 32u, e, kk, out);
    else
      rank_place<8>(lists32, 32u, e, kk, out);
  } else if (chunks <= 4u) {
    rank_place64<4>(lists64, 64u, lane < kk ? lists64[wave * 64u + lane] : 0ull, kk, out);
  } else {
#pragma unroll
    for (uint32_t h = 0; h < 2u; h++) {
      const uint32_t c = 2u * wave + h;
      rank_place64<8>(lists64, 64u, lane < kk ? lists64[c * 64u + lane] : 0ull, kk, out);
    }
  }
}

}  // namespace fg

#include "fg_nucleus_kernels.hpp"

namespace fg {

// ---- the fused kernel ------------------------------------------------------

template <class F>
__global__ __launch_bounds__(kBlock, 3) void sample_rows_kernel(SampleArgs a) {
  __shared__ uint64_t s_buf[F::kTop ? kWaves : 1][F::kTop ? kCap + kWave : 1];
  static_assert(!F::kTop || kWaves * (kCap + kWave) >= 8u * kMaxK, "finisher lists in s_buf");
  __shared__ uint64_t s_top[kWaves][kWave];
  __shared__ uint64_t s_greedy[kWaves];
  __shared__ uint32_t s_ks[kWaves];
  __shared__ double s_lm[kWaves];
  __shared__ double s_lz[kWaves];
  __shared__ double s_nm[kWaves];
  __shared__ double s_nz[kWaves];
  __shared__ double s_ne[kWaves];
  __shared__ uint32_t s_wg_key;
  __shared__ uint64_t s_rank[kWave];
  FG_TRACE_DECL;
  FG_TRACE_INIT;

  // readfirstlane: the wave index is uniform across the wave, so the slice
  // bounds, buffer descriptors and loop control stay scalar (the compiler
  // treats threadIdx.x / 64 as divergent, which wraps every buffer load in a
  // waterfall loop).
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t lane = lane_id();
  uint32_t row, chunk;
  block_row_chunk(blockIdx.x, a.rows, a.chunks, a.split, &row, &chunk);
  const RowParams p = row_controls(a, row);
  // After the read: a store to the table before it would keep the compiler
  // from reading the table with scalar loads.
  store_inline_controls(a);
  const float urow = a.uniforms[row];  // early: the row's last step needs it
  const bool greedy = p.temperature == 0.0f;
  const uint32_t L = a.logprobs;
  const bool lse = F::kLse && L != 0u;
  const bool nuc = F::kNuc && !greedy && p.top_k == 0u;
  const uint32_t kk = greedy ? L : nuc ? kMaxK : (p.top_k > L ? p.top_k : L);
  const bool pen = (p.flags & kRowPenalties) && a.counts != nullptr;
  // Speculative staging pays for top lists longer than kSpecMinK (top-k
  // rows and the whole-row nucleus's 64 best) over short wave slices
  // (measured: top-k 64 on 64 rows 16% faster, config 3 6%); over long
  // slices the exact filter soon passes it, and a check that fails would
  // read a long slice again.
  const bool spec = F::kSpec && !greedy && kk > kSpecMinK &&
                    max(a.wave_elems, a.wave_elems_b) <= kSpecMaxElems;
  const float t_eff = p.temperature > 0.0f ? p.temperature : 1.0f;
  const float log2e_over_t = 1.4426950408889634f / t_eff;
  // 1 / T for the finish, divided here where the loads' latency hides it.
  const double inv_t = 1.0 / static_cast<double>(p.temperature);

  const float* lrow = a.logits + static_cast<uint64_t>(row) * a.lstride;
  const uint32_t* crow = pen ? a.counts + static_cast<uint64_t>(row) * a.cstride : nullptr;
  float* prow = a.penalised ? a.penalised + static_cast<uint64_t>(row) * a.vocab : nullptr;

  const uint32_t wbegin = slice_begin(a, chunk * kWaves + wave);
  const uint32_t wend = slice_end(a, chunk * kWaves + wave);
  const uint32_t q_begin = wbegin / 4u;
  const uint32_t q_end = (wbegin + ((wend - wbegin) & ~3u)) / 4u;

  if (F::kTop) {
    if (threadIdx.x == 0) s_wg_key = 0u;
    __syncthreads();
  }
  WaveState st{{0ull, kFiniteComp - 1ull, F::kTop ? s_buf[wave] : nullptr, 0u, F::kTop ? kk : 0u,
                -3.402823466e38f, &s_wg_key, 0u},
               -INFINITY, kInvalidId, kInvalidId, -INFINITY, 0.0f, -INFINITY, 0.0, 0.0, true,
               0u, -3.402823466e38f};
  FG_TRACE(a, 0);

  if (q_end > q_begin) {
    // Double-buffered, the two buffers taking turns (no register copies,
    // which would wait for the loads on the back edge): step s+1 is loaded
    // before step s is processed.  (Loading further ahead measured slower.)
    f4 xa[F::kStepVec], xb[F::kStepVec];
    u4 ya[F::kStepVec], yb[F::kStepVec];
    const bool cnt = F::kPen && pen;
    const uint32_t slice_bytes = (q_end - q_begin) * 16u;
    const __amdgpu_buffer_rsrc_t rl = slice_rsrc(lrow + 4u * q_begin, slice_bytes);
    const __amdgpu_buffer_rsrc_t rc =
        slice_rsrc(cnt ? static_cast<const void*>(crow + 4u * q_begin) : lrow, cnt ? slice_bytes : 0u);
    auto load = [&](f4 (&x)[F::kStepVec], u4 (&y)[F::kStepVec], uint32_t qs) {
#pragma unroll
      for (int j = 0; j < F::kStepVec; j++) {
        if constexpr (F::kVec)
          load_quad_buf(rl, rc, cnt, qs - q_begin + j * kWave + lane, x[j], y[j]);
        else
          load_quad<false>(lrow, crow, cnt, min(qs + j * kWave + lane, q_end - 1u), x[j], y[j]);
      }
    };
    load(xa, ya, q_begin);
    // Fair progress between the waves sharing a SIMD: a wave starts at the
    // highest issue priority and steps down at each quarter of its slice, so
    // a wave that has fallen behind (the hardware favours older waves at
    // equal priority) is issued first until it catches up.
    const uint32_t quarter = (q_end - q_begin + 3u) / 4u;
    uint32_t next_drop = a.pace ? q_begin + quarter : 0xffffffffu;
    uint32_t level = 3u;
    if (a.pace) __builtin_amdgcn_s_setprio(3);
    auto pace = [&](uint32_t q) {
      if (q >= next_drop) {
        next_drop += quarter;
        level--;
        if (level == 2u) __builtin_amdgcn_s_setprio(2);
        else if (level == 1u) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
      }
    };
    for (uint32_t q0 = q_begin;;) {
      load(xb, yb, q0 + (kWave * F::kStepVec));
      process_step<F>(st, p, pen, greedy, lse, nuc, spec, log2e_over_t, prow, xa, ya, q0, q_end);
      if ((q0 += (kWave * F::kStepVec)) >= q_end) break;
      pace(q0);
      load(xa, ya, q0 + (kWave * F::kStepVec));
      process_step<F>(st, p, pen, greedy, lse, nuc, spec, log2e_over_t, prow, xb, yb, q0, q_end);
      if ((q0 += (kWave * F::kStepVec)) >= q_end) break;
      pace(q0);
    }
    if (a.pace) __builtin_amdgcn_s_setprio(3);  // the rest is the row's critical path
  }
  {
    // Fewer than 4 trailing elements (only at the end of a row): lane 0.
    const uint32_t tail = (wend - wbegin) & 3u;
    if (tail) {
      const uint32_t i0 = q_end * 4u;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const bool valid = lane == 0u && static_cast<uint32_t>(e) < tail;
        float v = valid ? lrow[i0 + e] : -INFINITY;
        const uint32_t c = (valid && pen) ? crow[i0 + e] : 0u;
        if (pen && valid) v = penalise(v, c, p.presence, p.frequency, p.repetition);
        if (prow && valid) prow[i0 + e] = v;
        if (F::kGreedy && greedy) greedy_stream(st, valid, v, i0 + e);
        if (lse && valid && is_finite_bits(__float_as_uint(v))) {
          if (v > st.lm) {
            st.lz = (st.lm == -INFINITY) ? 0.0f : st.lz * exp2f((st.lm - v) * log2e_over_t);
            st.lm = v;
          }
          st.lz += exp2f((v - st.lm) * log2e_over_t);
        }
        if (F::kNuc && nuc && valid && is_finite_bits(__float_as_uint(v))) {
          // Exact f64 terms here (error bound contribution 0).
          Mass ms{static_cast<double>(st.nm), st.nz, st.ne};
          mass_accumulate(ms, static_cast<double>(v), 1.0, 0.0);
          st.nm = static_cast<float>(ms.m);
          st.nz = ms.z;
          st.ne = ms.e;
        }
        // Below the speculative filter an element is left to the check.
        if (F::kTop && kk)
          top_stage(st.t, make_comp(valid && !(F::kSpec && v < st.fS) ? float_key(v) : 0u, i0 + e));
      }
    }
  }

  // ---- per-wave results ----
  FG_TRACE(a, 1);
  if (F::kTop && kk && !top_drain_rank(st.t)) top_drain(st.t, true);
  FG_TRACE(a, 2);
  const uint64_t mine = (F::kTop && kk && lane < kk) ? st.t.top : 0ull;
  const uint64_t gbest = (F::kGreedy && greedy) ? wave_max_u64(greedy_lane_comp(st)) : 0ull;
  double wm = -INFINITY, wz = 0.0;
  if (lse) wave_lse_combine(static_cast<double>(st.lm), static_cast<double>(st.lz), t_eff, &wm, &wz);
  Mass wmass{-INFINITY, 0.0, 0.0};
  if (F::kNuc && nuc) wmass = wave_mass_combine(static_cast<double>(st.nm), st.nz, st.ne);

  // ---- the workgroup's result: wave 0 combines the four waves from LDS ----
  // Finisher protocol (launches whose rows all keep top lists of at most 64
  // over 2-8 chunks, nothing else): one chunk finishes the row, reading the
  // other chunks' lists until every entry carries the tag; the others store
  // their lists tagged and end, with no wait for the stores and no arrival
  // count (measured at config 2: 0.3 us less than the last-arriver hand-off;
  // giving chunk 0 a longer slice, so that it would usually end last, cost
  // more stream time than the wait it saved).  All four waves of the
  // finishing workgroup rank the lists.
  const bool fin_mode = F::kTop && !F::kLse && !F::kNuc && finisher_of(a) != 0u &&
                        !greedy && kk != 0u && kk <= static_cast<uint32_t>(kMaxK) && a.chunks <= 8u;
  const bool fin_wg = fin_mode && a.chunks != 1u && chunk == finisher_of(a) - 1u;
  // The same for batches of greedy rows (no log-probs) over 2-64 chunks:
  // one composite per chunk.
  const bool gfin_mode = F::kGreedy && finisher_of(a) != 0u && greedy && L == 0u &&
                         a.chunks >= 2u && a.chunks <= static_cast<uint32_t>(kWave);
  // The four waves rank their own lists' entries (five- or six-step
  // searches): lists of at most 32, and longer ones in launches without
  // whole-row nucleus or log-prob rows (there, one wave's bitonic merges
  // measured faster: 69.3 against 71.1 us at config 3, 215.6 against 216.1
  // at config 5; at config 4's top-k 50, 27.64 against 27.95).
  const bool rank_wg = F::kTop && kk != 0u && (kk <= 32u || (!F::kNuc && !F::kLse));
  if (F::kTop) s_top[wave][lane] = mine;
  if (F::kTop && rank_wg && wave == 0) s_rank[lane] = 0ull;
  if (lane == 0) {
    // Only the partials some row of the launch reads.
    if (F::kGreedy) s_greedy[wave] = gbest;
    if (F::kSpec) s_ks[wave] = st.KS;
    if (F::kLse) {
      s_lm[wave] = wm;
      s_lz[wave] = wz;
    }
    if (F::kNuc) {
      s_nm[wave] = wmass.m;
      s_nz[wave] = wmass.z;
      s_ne[wave] = wmass.e;
    }
  }
  __syncthreads();
  if (F::kTop && rank_wg) {
    if (kk <= 32u)
      rank_place<kWaves>(&s_top[0][0], kWave, mine, kk, s_rank);
    else
      rank_place64<kWaves>(&s_top[0][0], kWave, mine, kk, s_rank);
    __syncthreads();
  }
  // Launches with whole-row nucleus rows: a workgroup's waves stay to the
  // end, where wave 0 tells them (through LDS, at one barrier every path of
  // every wave reaches) whether its row's cut lies below the kMaxK best; if
  // so all four run the deep-row descent, in the staging LDS.
  __shared__ uint32_t s_nuc_deep;
  __shared__ float s_nuc_vmax;
  auto nuc_tail = [&](bool deep, float vmax) __attribute__((always_inline)) {
    if (wave == 0 && lane == 0) {
      s_nuc_deep = deep ? 1u : 0u;
      s_nuc_vmax = vmax;
    }
    __syncthreads();
    // (Nucleus rows keep top lists, so launches with them have kTop.)
    if constexpr (F::kTop) {
      if (__builtin_expect(s_nuc_deep != 0u, 0)) {
        static_assert(sizeof(NucLds<FusedNuc>) <= sizeof(s_buf), "deep-row LDS");
        // Everything the descent needs is re-read here, so the streaming
        // code above carries none of it.
        const RowParams q = row_controls(a, row);
        const bool qpen = (q.flags & kRowPenalties) && a.counts != nullptr;
        nucleus_deep_row<FusedNuc>(
            a.logits + static_cast<uint64_t>(row) * a.lstride,
            qpen ? a.counts + static_cast<uint64_t>(row) * a.cstride : nullptr, q.temperature,
            q.top_p, q.presence, q.frequency, q.repetition, a.vocab, a.uniforms[row], s_nuc_vmax,
            a.tokens + row, a.token_logits ? a.token_logits + row : nullptr,
            a.row_status ? a.row_status + row : nullptr,
            *reinterpret_cast<NucLds<FusedNuc>*>(&s_buf[0][0]));
      }
    }
  };
  if (wave != 0) {
    if (F::kTop && fin_wg) {
      // The finisher's helpers: wave 0 fills the lists, all four rank them.
      __syncthreads();
      rank_place_lists(&s_top[0][0], &s_buf[0][0], wave, kk, a.chunks, s_rank);
      __syncthreads();
    }
    if constexpr (F::kNuc) nuc_tail(false, 0.0f);
    return;
  }
  uint64_t fin = 0ull;
  uint64_t g = 0ull;
  double m = -INFINITY, z = 0.0;
  Mass zs{-INFINITY, 0.0, 0.0};
  if (F::kTop && kk) {
    if (rank_wg) {
      fin = lane < kk ? s_rank[lane] : 0ull;
    } else {
      // (0,1) and (2,3) side by side, then the two results.
      uint64_t a0 = s_top[0][lane], a1 = s_top[2][lane];
      wave_merge_desc2(a0, s_top[1][lane], a1, s_top[3][lane]);
      fin = readlane64(a1, 0) > readlane64(a0, kk - 1u) ? wave_merge_desc(a0, a1) : a0;
    }
  }
  for (int w = 0; w < kWaves; w++) {
    if (F::kGreedy) g = s_greedy[w] > g ? s_greedy[w] : g;  // no greedy row: g stays 0
    if (lse) lse_accumulate(m, z, s_lm[w], s_lz[w], t_eff);
    if (F::kNuc && nuc) mass_accumulate(zs, s_nm[w], s_nz[w], s_ne[w]);
  }
  uint32_t ks0 = 0u;
  bool gave_up = false;  // the finisher's wait passed its limit
  if (a.chunks == 1u) {  // the whole row is in this workgroup
    if (spec) ks0 = spec_key(a, row, lane, s_ks);
  } else if ((fin_mode || gfin_mode) && chunk != finisher_of(a) - 1u) {
    const uint64_t slot = static_cast<uint64_t>(row) * a.chunks + chunk;
    const uint64_t header = wire_header(a.finisher >> 16u);
    if (fin_mode && lane < kk)
      store_coherent(a.cand + slot * kMaxK + lane, header | wire_payload(fin));
    if (fin_mode && spec && lane < static_cast<uint32_t>(kWaves))
      store_coherent(a.spec + slot * kWaves + lane, header | s_ks[lane]);
    if (gfin_mode && lane == 0) store_coherent(a.greedy + slot, header | greedy_payload(g));
    FG_TRACE(a, 3);
    FG_TRACE_FLUSH(a);
    return;
  } else {
    const uint64_t slot = static_cast<uint64_t>(row) * a.chunks + chunk;
    if (!fin_mode && !gfin_mode) {
      // Publish the workgroup's partials with device-coherent stores.
      if (F::kTop && kk && lane < kk) store_coherent(a.cand + slot * kMaxK + lane, fin);
      if (spec && lane < static_cast<uint32_t>(kWaves))
        store_coherent(a.spec + slot * kWaves + lane, static_cast<uint64_t>(s_ks[lane]));
      if (lane == 0) {
        if (F::kGreedy && greedy) store_coherent(a.greedy + slot, g);
        if (lse) {
          store_coherent_f64(a.lse + slot * 2, m);
          store_coherent_f64(a.lse + slot * 2 + 1, z);
        }
        if (F::kNuc && nuc) {
          store_coherent_f64(a.zsum + slot * 3, zs.m);
          store_coherent_f64(a.zsum + slot * 3 + 1, zs.z);
          store_coherent_f64(a.zsum + slot * 3 + 2, zs.e);
        }
      }
      wait_memory();  // hand-off ordering: see wait_memory()
      FG_TRACE(a, 3);
      uint32_t arrived = 0u;
      if (lane == 0) arrived = atomicAdd(&a.row_done[row * kLineWords], 1u);
      arrived = __builtin_amdgcn_readfirstlane(arrived);
      FG_TRACE(a, 4);
      if (arrived != a.chunks - 1u) {
        FG_TRACE_FLUSH(a);
        if constexpr (F::kNuc) nuc_tail(false, 0.0f);
        return;
      }
    }

    // ---- last workgroup of the row: merge the other workgroups' lists ----
    const uint64_t row_slot = static_cast<uint64_t>(row) * a.chunks;
    if (F::kTop && fin_mode) {
      // The finisher (at most 8 chunks): the others' lists are read until
      // every entry carries this launch's epoch, then placed in LDS beside
      // its own and ranked by all four waves (which meet at the barriers
      // below even when the wait gives up).
      const uint32_t own = finisher_of(a) - 1u;
      const uint64_t header = wire_header(a.finisher >> 16u);
      // Lists of at most 32: lanes 0-31 hold list 2t, lanes 32-63 list
      // 2t + 1 in x[t] (t < 4).  Longer lists: x[c] holds list c at
      // position `lane`.
      const bool wide = kk > 32u;
      const bool hi = lane >= 32u;
      const uint32_t pos = wide ? lane : (lane & 31u);
      uint64_t x[8];
      auto list_of = [&](int t) -> uint32_t { return wide ? static_cast<uint32_t>(t) : 2u * t + (hi ? 1u : 0u); };
      // Speculating rows: lane i also reads wave i's key (i < chunks * 4).
      const uint32_t ks_chunk = lane / static_cast<uint32_t>(kWaves);
      const bool ks_read = spec && ks_chunk < a.chunks && ks_chunk != own;
      uint64_t y = header;
      auto fetch = [&]() {
#pragma unroll
        for (int t = 0; t < 8; t++) {
          const uint32_t c = list_of(t);
          if ((wide || t < 4) && c != own && c < a.chunks && pos < kk)
            x[t] = load_coherent(a.cand + (row_slot + c) * kMaxK + pos);
        }
        if (ks_read) y = load_coherent(a.spec + row_slot * kWaves + lane);
      };
#pragma unroll
      for (int t = 0; t < 8; t++) x[t] = header;
      fetch();
      FG_TRACE(a, 8);
      uint64_t t0 = 0ull;
      for (uint32_t spin = 0;; spin++) {
        bool miss = !wire_current(y, header);
#pragma unroll
        for (int t = 0; t < 8; t++) miss |= !wire_current(x[t], header);
        if (ballot(miss) == 0ull) break;
        if (wait_passed(a, spin, t0)) {
          gave_up = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        fetch();
      }
      FG_TRACE(a, 4);
      uint64_t* const lists = wide ? &s_buf[0][0] : &s_top[0][0];
      const uint32_t stride = wide ? 64u : 32u;
#pragma unroll
      for (int t = 0; t < 8; t++) {
        const uint32_t c = list_of(t);
        if ((wide || t < 4) && c != own) lists[c * stride + pos] = comp_of_payload(x[t] & kWirePayload);
      }
      if (wide || lane < 32u) lists[own * stride + lane] = lane < kk ? fin : 0ull;
      s_rank[lane] = 0ull;
      __syncthreads();
      rank_place_lists(&s_top[0][0], &s_buf[0][0], 0u, kk, a.chunks, s_rank);
      __syncthreads();
      fin = lane < kk ? s_rank[lane] : 0ull;
      if (spec) {
        const uint32_t w = lane % static_cast<uint32_t>(kWaves);
        ks0 = ks_chunk == own ? s_ks[w]
              : ks_chunk < a.chunks ? static_cast<uint32_t>(y & kWirePayload) : 0u;
      }
      FG_TRACE(a, 5);
    } else if (F::kTop && kk) {
      if (kk <= 32u) {
        // Lists of at most 32: two per register, the second loaded in
        // reverse into lanes 32-63, so a pair is already a bitonic sequence
        // and one 64-wide merge stage leaves the pair's best 32 in lanes
        // 0-31.  Eight lists per round (this workgroup's own included) in
        // three levels; rounds fold into `fin`.
        const bool hi = lane >= 32u;
        const uint32_t pos = hi ? 63u - lane : lane;  // list position this lane holds
        uint64_t acc = 0ull;
        for (uint32_t c0 = 0; c0 < a.chunks; c0 += 8u) {
          uint64_t x[4];
#pragma unroll
          for (int t = 0; t < 4; t++) {
            const uint32_t c = c0 + 2u * t + (hi ? 1u : 0u);
            x[t] = (c < a.chunks && pos < kk)
                       ? load_coherent(a.cand + (row_slot + c) * kMaxK + pos)
                       : 0ull;
          }
          if (spec && c0 == 0u) {
            // The waves' speculative keys travel with the first lists (the
            // asm keeps the load here instead of after the merges).
            ks0 = spec_key(a, row, lane, s_ks);
            asm volatile("" ::"v"(ks0));
          }
#pragma unroll
          for (int t = 0; t < 4; t++) x[t] = bitonic_merge_stage<64>(x[t]);
          // The reversals run in every lane (a cross-lane read from a lane
          // that is switched off would not return its value), then select.
          const uint64_t r1 = lane_reverse64(x[1]), r3 = lane_reverse64(x[3]);
          x[0] = bitonic_merge_stage<64>(hi ? r1 : x[0]);
          x[2] = bitonic_merge_stage<64>(hi ? r3 : x[2]);
          const uint64_t r2 = lane_reverse64(x[2]);
          x[0] = bitonic_merge_stage<64>(hi ? r2 : x[0]);
          if (c0 == 0u) {
            acc = x[0];
          } else {
            const uint64_t r0 = lane_reverse64(x[0]);
            acc = bitonic_merge_stage<64>(hi ? r0 : acc);
          }
        }
        fin = acc;
      } else {
        // Eight lists per round, loaded together and merged as a tree of
        // side-by-side pairs; this workgroup's own list is already in `fin`.
        for (uint32_t c0 = 0; c0 < a.chunks; c0 += 8u) {
          uint64_t x[8];
#pragma unroll
          for (int t = 0; t < 8; t++) {
            const uint32_t c = c0 + t;
            x[t] = (c < a.chunks && c != chunk && lane < kk)
                       ? load_coherent(a.cand + (row_slot + c) * kMaxK + lane)
                       : 0ull;
          }
          if (spec && c0 == 0u) {
            ks0 = spec_key(a, row, lane, s_ks);
            asm volatile("" ::"v"(ks0));
          }
          wave_merge_desc2(x[0], x[1], x[2], x[3]);
          wave_merge_desc2(x[4], x[5], x[6], x[7]);
          wave_merge_desc2(x[0], x[2], x[4], x[6]);
          wave_merge_desc2(fin, x[0], x[4], 0ull);
          if (readlane64(x[4], 0) > readlane64(fin, kk - 1u)) fin = wave_merge_desc(fin, x[4]);
        }
      }
      FG_TRACE(a, 5);
    }
    if (F::kGreedy && greedy) {
      if (gfin_mode) {
        // The greedy finisher (at most 64 chunks, one per lane): the others'
        // words are read until every one carries this launch's epoch.
        const uint32_t own = finisher_of(a) - 1u;
        const uint64_t header = wire_header(a.finisher >> 16u);
        const bool other = lane < a.chunks && lane != own;
        const uint64_t* const at = a.greedy + row_slot + lane;
        uint64_t x = other ? load_coherent(at) : header;
        uint64_t t0 = 0ull;
        for (uint32_t spin = 0; ballot(!wire_current(x, header)) != 0ull; spin++) {
          if (wait_passed(a, spin, t0)) {
            gave_up = true;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
          if (!wire_current(x, header)) x = load_coherent(at);
        }
        const uint64_t xv = greedy_of_payload(x & kWirePayload);
        g = wave_max_u64(xv > g ? xv : g);
      } else {
        for (uint32_t i = lane; i < a.chunks; i += kWave) {
          const uint64_t x = load_coherent(a.greedy + row_slot + i);
          g = x > g ? x : g;
          // Cleared: a greedy finisher of a later launch must never find an
          // untagged composite here (its high bits could read as a tag).
          store_coherent(a.greedy + row_slot + i, uint64_t{0});
        }
        g = wave_max_u64(g);
      }
    }
    if (lse) {
      double lm = -INFINITY, lz = 0.0;
      for (uint32_t i = lane; i < a.chunks; i += kWave)
        lse_accumulate(lm, lz, load_coherent_f64(a.lse + (row_slot + i) * 2),
                       load_coherent_f64(a.lse + (row_slot + i) * 2 + 1), t_eff);
      wave_lse_combine(lm, lz, t_eff, &m, &z);
    }
    if (F::kNuc && nuc) {
      Mass lm{-INFINITY, 0.0, 0.0};
      for (uint32_t i = lane; i < a.chunks; i += kWave)
        mass_accumulate(lm, load_coherent_f64(a.zsum + (row_slot + i) * 3),
                        load_coherent_f64(a.zsum + (row_slot + i) * 3 + 1),
                        load_coherent_f64(a.zsum + (row_slot + i) * 3 + 2));
      zs = wave_mass_combine(lm.m, lm.z, lm.e);
    }
  }
  // One copy of the check and of the finish serves both paths.
  if (spec) fin = spec_check(a, p, row, pen, lrow, crow, fin, kk, s_ks, ks0, s_buf[0], &s_wg_key);
  FG_TRACE(a, 6);
  int32_t status = kStOk;
  if (gave_up)
    timeout_row(a, row);
  else
    status = finish_row(a, p, row, fin, g, m, z, zs, lrow, crow, pen, urow, inv_t);
  if (a.chunks != 1u && !fin_mode && !gfin_mode && lane == 0)
    store_coherent(&a.row_done[row * kLineWords], 0u);
  FG_TRACE(a, 7);
  FG_TRACE_FLUSH(a);
  if constexpr (F::kNuc)
    nuc_tail(nuc && status == kStLimit, key_to_float(comp_key(readlane64(fin, 0))));
}

}  // namespace fg
