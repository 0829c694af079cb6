// extern "C" entry points of include/fg_sampler_hip.h: argument checks,
// launch shapes and workspace ownership for the gfx950 sampling kernels.
#include <hip/hip_runtime.h>

#include <math.h>

#include <atomic>
#include <stdlib.h>
#include <string.h>

#include "fg_sampler_hip.h"
#include "fg_dense_kernels.hpp"
#include "fg_lmhead_sample_kernels.hpp"
#include "fg_sample_kernels.hpp"
#include "fg_split_kernels.hpp"
#include "fg_unit_kernels.hpp"

namespace {

using fg::RowParams;

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

fg_status hip_fail(fg_error* err, hipError_t e, const char* what) {
  fg_error_set(err, FG_ERR_UNAVAILABLE, "%s: %s", what, hipGetErrorString(e));
  return FG_ERR_UNAVAILABLE;
}

fg_status arg_fail(fg_error* err, const char* msg) {
  fg_error_set(err, FG_ERR_ARGUMENT, "%s", msg);
  return FG_ERR_ARGUMENT;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Validation of src/sampler.c:24-38, with top_k == 0 admitted when the
// whole-vocabulary extension is enabled.
bool config_ok(const fg_sampler_config* c, uint32_t flags) {
  if (c->top_k == 0u && (flags & FG_SAMPLER_HIP_ALLOW_FULL_VOCAB)) {
    fg_sampler_config probe = *c;
    probe.top_k = 1u;
    return fg_sampler_config_validate(&probe, nullptr) == FG_OK;
  }
  return fg_sampler_config_validate(c, nullptr) == FG_OK;
}

// One instantiation of the fused kernel per feature combination.
using SampleLaunch = void (*)(uint32_t, hipStream_t, const fg::SampleArgs&);

template <class F>
void launch_sample(uint32_t grid, hipStream_t s, const fg::SampleArgs& a) {
  fg::sample_rows_kernel<F><<<grid, fg::kBlock, 0, s>>>(a);
}

template <int kBits>
constexpr SampleLaunch vec_launch() {
  // The speculative-staging bit only exists alongside top lists.
  return launch_sample<fg::Features<true, (kBits & 1) != 0, (kBits & 2) != 0, (kBits & 4) != 0,
                                    (kBits & 8) != 0, (kBits & 16) != 0,
                                    (kBits & 4) != 0 && (kBits & 32) != 0>>;
}

template <int... kBits>
struct LaunchTable {
  static constexpr SampleLaunch table[sizeof...(kBits)] = {vec_launch<kBits>()...};
};

// Indexed by pen | greedy << 1 | top << 2 | lse << 3 | nucleus << 4 |
// speculative << 5.
const SampleLaunch* const kVecLaunch =
    LaunchTable<0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21,
                22, 23, 24, 25, 26, 27, 28, 29, 30, 31, 32, 33, 34, 35, 36, 37, 38, 39, 40, 41,
                42, 43, 44, 45, 46, 47, 48, 49, 50, 51, 52, 53, 54, 55, 56, 57, 58, 59, 60, 61,
                62, 63>::table;
// Rows that are not 16-byte aligned: scalar loads, every part compiled in.
const SampleLaunch kScalarLaunch =
    launch_sample<fg::Features<false, true, true, true, true, true, true>>;

// The same instantiations as kernel symbols (occupancy queries), index 64
// the scalar one.
template <int kBits>
const void* vec_kernel() {
  return reinterpret_cast<const void*>(
      &fg::sample_rows_kernel<fg::Features<true, (kBits & 1) != 0, (kBits & 2) != 0,
                                           (kBits & 4) != 0, (kBits & 8) != 0, (kBits & 16) != 0,
                                           (kBits & 4) != 0 && (kBits & 32) != 0>>);
}
template <int... kBits>
const void* kernel_of(int index) {
  static const void* const table[sizeof...(kBits)] = {vec_kernel<kBits>()...};
  return table[index];
}
const void* sample_kernel(int index) {
  if (index >= 64)
    return reinterpret_cast<const void*>(
        &fg::sample_rows_kernel<fg::Features<false, true, true, true, true, true, true>>);
  return kernel_of<0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16, 17, 18, 19, 20, 21,
                   22, 23, 24, 25, 26, 27, 28, 29, 30, 31, 32, 33, 34, 35, 36, 37, 38, 39, 40, 41,
                   42, 43, 44, 45, 46, 47, 48, 49, 50, 51, 52, 53, 54, 55, 56, 57, 58, 59, 60, 61,
                   62, 63>(index);
}

// Workgroups of one instantiation that a CU holds at once (0: unknown),
// queried once per process: every GPU this library runs on is a gfx950.
std::atomic<int> g_occupancy[65];
int occupancy(int index) {
  int n = g_occupancy[index].load(std::memory_order_relaxed);
  if (n) return n;
  const void* k = sample_kernel(index);
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, fg::kBlock, 0) != hipSuccess || n < 0)
    n = 0;
  g_occupancy[index].store(n, std::memory_order_relaxed);
  return n;
}

// ---- Q8_0 cooked matrix-vector launch shapes

constexpr uint32_t kDensePassTokens = 2;  // tokens per pass over the weights

bool dense_geometry(uint32_t in, uint32_t rows, fg::DenseArgs* a) {
  if (!in || in % 32u || in * kDensePassTokens > fg::kDenseLdsFloats || !rows) return false;
  const uint64_t blocks = in / 32u;
  a->quant_offset = (fg::kCookRows * blocks * 2u + 63u) & ~63ull;
  a->tile_bytes = (a->quant_offset + fg::kCookRows * blocks * 32u + 63u) & ~63ull;
  a->in = in;
  a->rows = rows;
  return a->tile_bytes <= UINT32_MAX;
}

// One tile per wave: the dispatcher balances waves better than a fixed
// tile stride (a persistent grid left a ragged last round).
uint32_t dense_groups(uint32_t rows) {
  const uint64_t tiles = (rows + fg::kCookRows - 1u) / fg::kCookRows;
  return static_cast<uint32_t>((tiles + 3u) / 4u);
}

template <bool kFused>
hipError_t dense_launch(fg::DenseArgs a, uint32_t tokens, hipStream_t stream) {
  const uint32_t groups = dense_groups(a.rows);
  for (uint32_t t0 = 0; t0 < tokens; t0 += kDensePassTokens) {
    a.token0 = t0;
    a.tokens = tokens - t0 < kDensePassTokens ? tokens - t0 : kDensePassTokens;
    if (a.tokens == 1u) {
      const size_t lds = sizeof(float) * a.in;
      if (kFused)
        fg::dense_q8_finalist_kernel<1><<<groups, fg::kDenseBlock, lds, stream>>>(a);
      else
        fg::dense_q8_cooked_kernel<1><<<groups, fg::kDenseBlock, lds, stream>>>(a);
    } else {
      const size_t lds = sizeof(float) * a.in * 2u;
      if (kFused)
        fg::dense_q8_finalist_kernel<2><<<groups, fg::kDenseBlock, lds, stream>>>(a);
      else
        fg::dense_q8_cooked_kernel<2><<<groups, fg::kDenseBlock, lds, stream>>>(a);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

// Paired layout (a row's chunks split between the grid's halves) for grids
// of at most this many workgroups (two per CU), and the share (per mille) of
// a row its first-half chunks stream: measured on MI355X at V = 151,936,
// 580 for two chunks per row (config 3 at 2 chunks: 79.5 -> 77.4 us), 530
// for more (config 2 at 8 chunks, 512-element steps: 21.1 us even, 20.65 at
// 520, 20.5 at 530, 20.55 at 535); grids of four workgroups per CU run
// slower paired (config 4: 28.5 -> 30.8 us).
constexpr uint32_t kPairedMaxGroups = 512u;
constexpr uint32_t kFrontPermilleTwo = 580u;
constexpr uint32_t kFrontPermilleMany = 530u;

namespace {

// Launch-geometry overrides read from the environment (0 / -1: the rule).
struct Tuning {
  uint32_t target_groups = 0u;   // FG_HIP_TARGET_GROUPS
  uint32_t front_permille = 0u;  // FG_HIP_FRONT_SHARE (500..749)
  int32_t paired = -1;           // FG_HIP_PAIRED (0 / 1)
  int32_t pace = -1;             // FG_HIP_PACE (0 / 1)
  int32_t finisher = -1;         // FG_HIP_FINISHER (0: off, c + 1: chunk c finishes)
  uint64_t wait_us = 100000u;    // FG_HIP_FINISHER_WAIT_US: the finisher's wait limit
};
Tuning tuning_from_env() {
  Tuning t;
  if (const char* v = getenv("FG_HIP_TARGET_GROUPS")) {
    const long x = strtol(v, nullptr, 10);
    if (x >= 1 && x <= 1 << 20) t.target_groups = static_cast<uint32_t>(x);
  }
  if (const char* v = getenv("FG_HIP_FRONT_SHARE")) {
    const long x = strtol(v, nullptr, 10);
    if (x >= 500 && x < 750) t.front_permille = static_cast<uint32_t>(x);
  }
  if (const char* v = getenv("FG_HIP_PAIRED")) t.paired = atoi(v) != 0;
  if (const char* v = getenv("FG_HIP_PACE")) t.pace = atoi(v) != 0;
  if (const char* v = getenv("FG_HIP_FINISHER")) t.finisher = atoi(v);  // 0: off, c + 1: chunk c
  if (const char* v = getenv("FG_HIP_FINISHER_WAIT_US")) {
    const long long x = strtoll(v, nullptr, 10);
    if (x >= 0 && x <= 60000000) t.wait_us = static_cast<uint64_t>(x);
  }
  return t;
}

// Launch geometry of a batch (see fg_sampler_hip_geometry).
//
// Chunking (measured on MI355X, V = 151,936): ceil(512 / rows) chunks, two
// workgroups per CU (config 2's 64 rows: 8 chunks, 21.5 us against 25.2 at
// 12; config 4's 128 rows: 4 chunks, 28.0 us against 29.2 at 6 and 29.9-31.1
// at 8; one row: 64 chunks, 5.97 us against 6.35 at 128).  Launches with
// whole-row nucleus rows (an exp per element) take ceil(768 / rows), three
// per CU (config 3's 256 rows: 3 chunks 69.1 us against 72.7 at 2 and 85.6
// at 4).  At most kMaxChunks per row; each wave slice a multiple of 4
// elements.
//
// Layout: the first workgroup dispatched to a CU streams faster than the
// second (measured: ~8% at 8 chunks of V = 151,936 per row, ~12% at 2).
// With the rows a multiple of the XCD count, an even chunk count, at most
// two workgroups per CU and rows of like cost, a row's first chunks go to
// the grid's first half (longer slices at two chunks per row), the others
// to its second half.  Rows of unlike cost keep the row-major halves: the
// costlier rows (first in the batch) then run in the faster first half
// (config 4, penalties on rows 0-63 only: 28.1 us against 30.2 paired).
void plan_geometry(uint32_t vocab, uint32_t rows, bool nuc_rows, bool same_cost, const Tuning& t,
                   fg_sampler_hip_geometry* g) {
  const uint32_t target = t.target_groups ? t.target_groups
                          : nuc_rows      ? fg::kNucleusGroups
                                          : fg::kDefaultGroups;
  uint32_t chunks = (target + rows - 1u) / rows;
  if (chunks > fg::kMaxChunks) chunks = fg::kMaxChunks;
  if (chunks < 1u) chunks = 1u;
  const uint32_t waves = chunks * fg::kWaves;
  uint32_t wave_elems = (vocab + waves - 1u) / waves;
  wave_elems = (wave_elems + 3u) & ~3u;
  if (wave_elems < 4u) wave_elems = 4u;
  chunks = (vocab + wave_elems * fg::kWaves - 1u) / (wave_elems * fg::kWaves);
  g->chunks = chunks;
  g->split = chunks;
  g->wave_elems = wave_elems;
  g->wave_elems_b = wave_elems;
  g->pace = t.pace >= 0 ? static_cast<uint32_t>(t.pace) : 1u;
  const bool paired_rule =
      same_cost && static_cast<uint64_t>(rows) * chunks <= kPairedMaxGroups;
  if (rows % fg::kXcds == 0u && chunks % 2u == 0u && (t.paired >= 0 ? t.paired != 0 : paired_rule)) {
    const uint32_t permille = t.front_permille ? t.front_permille
                              : chunks == 2u   ? kFrontPermilleTwo
                                               : kFrontPermilleMany;
    const uint32_t na = chunks / 2u * fg::kWaves;
    uint64_t ea = (static_cast<uint64_t>(vocab) * permille + 1000u * na - 1u) / (1000u * na);
    ea = (ea + 3u) & ~3ull;
    if (ea * na < vocab) {
      uint64_t eb = (vocab - ea * na + na - 1u) / na;
      eb = (eb + 3u) & ~3ull;
      g->wave_elems = static_cast<uint32_t>(ea);
      g->wave_elems_b = static_cast<uint32_t>(eb);
      g->split = chunks / 2u;
    }
  }
}

}  // namespace

// Device workspace of one sampling launch: the per-row controls and the
// hand-off buffers of the fused kernel (see fg::SampleArgs).
struct Workspace {
  uint32_t max_rows;
  uint64_t slots;           // wave slots
  RowParams* params;        // [max_rows]
  uint64_t* cand;           // [slots][kMaxK]
  uint64_t* greedy;         // [slots]
  uint64_t* spec;           // [slots] speculative stream keys
  double* lse;              // [slots][2]
  double* zsum;             // [slots][3]
  uint32_t* row_done;       // [max_rows * kLineWords], zero between launches
  uint64_t* trace;          // phase timestamps, FG_SAMPLE_TRACE builds only
  uint32_t* epoch;          // host: the last finisher launch's epoch (0: none yet)
  uint32_t cus;             // compute units of the device (co-residency check)
  Tuning tuning;            // environment overrides
};

struct fg_sampler_hip {
  int device;
  uint32_t vocab;
  Workspace ws;             // device workspace (hipMalloc'd at create)
  RowParams* h_params;      // host mirror of the uploaded table (launch-variant choice)
  uint32_t config_rows;     // rows configured by the last set_configs
  uint64_t* counters;       // event counters, FG_SAMPLE_TRACE builds only
  uint32_t epoch;           // the last finisher launch's epoch (Workspace::epoch)
  bool params_dirty;        // h_params not yet in the device table
};

namespace {

RowParams row_params(const fg_sampler_config* c) {
  RowParams p{};
  p.temperature = c->temperature;
  p.top_p = c->top_p;
  p.top_k = c->top_k;
  p.presence = c->presence_penalty;
  p.frequency = c->frequency_penalty;
  p.repetition = c->repetition_penalty;
  p.flags = fg_sampler_penalties_active(c) ? fg::kRowPenalties : 0u;
  return p;
}

// ---- Static workspace of fg_sampler_hip_sample_static
//
// A file-scope device array carved into the Workspace buffers for
// kStaticMaxRows rows.  Host code never uses the array's name as an address:
// each device's copy is found once with hipGetSymbolAddress and that pointer
// is used for every launch on the device.
constexpr uint32_t kStaticMaxRows = FG_SAMPLER_HIP_STATIC_MAX_ROWS;
constexpr uint64_t kStaticSlots = static_cast<uint64_t>(fg::kMaxGroups + kStaticMaxRows) * fg::kWaves;
constexpr size_t align256(size_t x) { return (x + 255u) & ~static_cast<size_t>(255u); }
constexpr size_t kOffParams = 0;
constexpr size_t kOffCand = align256(kOffParams + sizeof(RowParams) * kStaticMaxRows);
constexpr size_t kOffGreedy = align256(kOffCand + sizeof(uint64_t) * kStaticSlots * fg::kMaxK);
constexpr size_t kOffSpec = align256(kOffGreedy + sizeof(uint64_t) * kStaticSlots);
constexpr size_t kOffLse = align256(kOffSpec + sizeof(uint64_t) * kStaticSlots);
constexpr size_t kOffZsum = align256(kOffLse + sizeof(double) * kStaticSlots * 2u);
constexpr size_t kOffDone = align256(kOffZsum + sizeof(double) * (kStaticSlots / fg::kWaves) * 3u);
constexpr size_t kStaticBytes = align256(kOffDone + sizeof(uint32_t) * fg::kLineWords * kStaticMaxRows);
static_assert(kStaticBytes == FG_SAMPLER_HIP_STATIC_BYTES, "header size out of date");

static __device__ __align__(256) unsigned char scratch[kStaticBytes];

constexpr int kStaticMaxDevices = 64;
// Per device: the address of its copy of `scratch` (0 until first use), and
// the last finisher epoch used on it (calls that overlap on one device race,
// as they do on the array itself).
std::atomic<uintptr_t> g_scratch_addr[kStaticMaxDevices];
uint32_t g_static_epoch[kStaticMaxDevices];

hipError_t static_workspace(Workspace* w) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kStaticMaxDevices) return hipErrorInvalidDevice;
  uintptr_t base = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!base) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!ptr) return hipErrorInvalidSymbol;
    base = reinterpret_cast<uintptr_t>(ptr);
    g_scratch_addr[dev].store(base, std::memory_order_release);
  }
  unsigned char* p = reinterpret_cast<unsigned char*>(base);
  w->max_rows = kStaticMaxRows;
  w->slots = kStaticSlots;
  w->params = reinterpret_cast<RowParams*>(p + kOffParams);
  w->cand = reinterpret_cast<uint64_t*>(p + kOffCand);
  w->greedy = reinterpret_cast<uint64_t*>(p + kOffGreedy);
  w->spec = reinterpret_cast<uint64_t*>(p + kOffSpec);
  w->lse = reinterpret_cast<double*>(p + kOffLse);
  w->zsum = reinterpret_cast<double*>(p + kOffZsum);
  w->row_done = reinterpret_cast<uint32_t*>(p + kOffDone);
  w->trace = nullptr;
  w->epoch = &g_static_epoch[dev];
  int cus = 0;
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  w->cus = static_cast<uint32_t>(cus);
  // The environment is read once per process; the array holds kMaxGroups
  // workgroups' slots beyond the rows, so a larger target is clamped.
  static const Tuning tuning = [] {
    Tuning t = tuning_from_env();
    if (t.target_groups > fg::kMaxGroups) t.target_groups = fg::kMaxGroups;
    return t;
  }();
  w->tuning = tuning;
  return hipSuccess;
}

// Rows of controls per launch of params_fill_kernel (2 KiB of arguments).
constexpr uint32_t kParamsPerFill = 64;
struct ParamsFill {
  RowParams rows[kParamsPerFill];
  uint32_t first;
  uint32_t count;
};

// Writes rows [first, first + count) of the controls and clears their
// arrival counters (a fill kernel, not a memset, so the call can sit in a
// captured graph).
__global__ void __launch_bounds__(kParamsPerFill)
    params_fill_kernel(ParamsFill p, RowParams* params, uint32_t* row_done) {
  const uint32_t t = threadIdx.x;
  if (t < p.count) {
    params[p.first + t] = p.rows[t];
    row_done[static_cast<size_t>(p.first + t) * fg::kLineWords] = 0u;
  }
}

// Writes rows [0, rows) of the controls to w.params with params_fill_kernel
// launches on `stream` (the rows travel in the kernel arguments).
hipError_t fill_params(const Workspace& w, const RowParams* h, uint32_t rows, hipStream_t stream) {
  for (uint32_t first = 0; first < rows; first += kParamsPerFill) {
    ParamsFill p;
    p.first = first;
    p.count = rows - first < kParamsPerFill ? rows - first : kParamsPerFill;
    memcpy(p.rows, h + first, sizeof(RowParams) * p.count);
    params_fill_kernel<<<1, kParamsPerFill, 0, stream>>>(p, w.params, w.row_done);
  }
  return hipGetLastError();
}

// Returns the workspace's hand-off slots to zero (when the finisher epoch
// wraps, so that no word of an earlier launch can carry the new one).
__global__ void __launch_bounds__(256)
    epoch_clear_kernel(uint64_t* cand, uint64_t* greedy, uint64_t* spec, uint64_t slots) {
  // Every region that carries tagged words: lists, greedy composites and the
  // waves' speculative keys.
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < slots * fg::kMaxK; i += stride) {
    cand[i] = 0ull;
    if (i < slots) {  // greedy and spec: a word per wave slot at most
      greedy[i] = 0ull;
      spec[i] = 0ull;
    }
  }
}

// The next finisher epoch (1..kMaxEpoch); on a wrap the workspace is
// cleared first, on the same stream.
hipError_t next_epoch(const Workspace& w, hipStream_t stream, uint32_t* epoch) {
  uint32_t e = *w.epoch + 1u;
  if (e > fg::kMaxEpoch) {
    epoch_clear_kernel<<<256, 256, 0, stream>>>(w.cand, w.greedy, w.spec, w.slots);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    e = 1u;
  }
  *w.epoch = e;
  *epoch = e;
  return hipSuccess;
}

// One fused sampling launch (two with whole-row nucleus rows) over a batch
// whose per-row controls are h_params on the host (variant and layout choice)
// and w.params on the device, or, with inline_rows > 0, rows [0, inline_rows)
// of h_params carried in the launch's arguments (and written to w.params by
// the launch).  The caller has checked the batch against w.max_rows and the
// configured rows.
fg_status sample_launch(const Workspace& w, const RowParams* h_params, uint32_t vocab,
                        const fg_sampler_hip_batch* b, hipStream_t stream, uint32_t inline_rows,
                        fg_error* err) {
  if (!b->logits || !b->tokens || !b->uniforms || !b->rows || b->rows > w.max_rows ||
      b->logits_stride < vocab || (b->counts && b->counts_stride < vocab) ||
      b->logprobs > fg::kMaxK || (b->logprobs && (!b->logprob_values || !b->logprob_ids)))
    return arg_fail(err, "invalid sampled output arguments");
  bool same_cost = true;  // every row alike in penalties (for the paired layout)
  bool nuc_rows = false;
  for (uint32_t r = 0; r < b->rows; r++) {
    same_cost &= ((h_params[r].flags ^ h_params[0].flags) & fg::kRowPenalties) == 0u;
    nuc_rows |= h_params[r].temperature > 0.0f && h_params[r].top_k == 0u;
  }
  fg_sampler_hip_geometry geo;
  plan_geometry(vocab, b->rows, nuc_rows, same_cost, w.tuning, &geo);
  const uint32_t chunks = geo.chunks;
  if (static_cast<uint64_t>(b->rows) * chunks * fg::kWaves > w.slots) {
    fg_error_set(err, FG_ERR_LIMIT, "sampler workspace too small for %u rows", b->rows);
    return FG_ERR_LIMIT;
  }
  fg::SampleArgs a{};
  a.logits = b->logits;
  a.lstride = b->logits_stride;
  a.counts = b->counts;
  a.cstride = b->counts_stride;
  a.uniforms = b->uniforms;
  a.params = w.params;
  a.vocab = vocab;
  a.rows = b->rows;
  a.chunks = chunks;
  a.wave_elems = geo.wave_elems;
  a.wave_elems_b = geo.wave_elems_b;
  a.split = geo.split;
  uint32_t finisher = 0u;
  {
    // Finisher protocol (see the kernel): every row a top list of at most 64
    // (no greedy row, no log-probs) over 2-8 chunks, or every row greedy (no
    // log-probs) over 2-64 chunks; ids that fit a tagged word.  Not for a
    // launch being captured into a graph: its replays would all carry the
    // epoch it was captured with, so a word left by the previous replay
    // would pass for the current one; the last-arriver hand-off keeps no
    // state between launches.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &capture) != hipSuccess) capture = hipStreamCaptureStatusNone;
    const bool eager = capture == hipStreamCaptureStatusNone;
    bool ok = eager && w.tuning.finisher != 0 && chunks >= 2u && chunks <= 8u &&
              b->logprobs == 0u && vocab <= fg::kWireVocab;
    for (uint32_t r = 0; ok && r < b->rows; r++)
      ok = h_params[r].temperature > 0.0f && h_params[r].top_k >= 1u &&
           h_params[r].top_k <= static_cast<uint32_t>(fg::kMaxK);
    bool gok = eager && w.tuning.finisher != 0 && chunks >= 2u && chunks <= fg::kMaxChunks &&
               b->logprobs == 0u && vocab <= fg::kWireVocab;
    for (uint32_t r = 0; gok && r < b->rows; r++) gok = h_params[r].temperature == 0.0f;
    ok = ok || gok;
    const uint32_t which = w.tuning.finisher > 0 ? static_cast<uint32_t>(w.tuning.finisher) - 1u : 0u;
    finisher = ok && which < chunks ? which + 1u : 0u;
  }
  a.pace = geo.pace;
  a.logprobs = b->logprobs;
  a.tokens = b->tokens;
  a.token_logits = b->token_logits;
  a.row_status = b->row_status;
  a.penalised = b->penalised;
  a.lp_values = b->logprob_values;
  a.lp_ids = b->logprob_ids;
  a.cand = w.cand;
  a.greedy = w.greedy;
  a.spec = w.spec;
  a.lse = w.lse;
  a.zsum = w.zsum;
  a.row_done = w.row_done;
  a.trace = w.trace;
  a.inline_rows = inline_rows;
  if (inline_rows) memcpy(a.row_inline, h_params, sizeof(RowParams) * inline_rows);

  // The vector path addresses a slice with 32-bit byte offsets.
  const bool vec = aligned16(b->logits) && (b->logits_stride % 4u) == 0u &&
                   a.wave_elems < (1u << 28) && a.wave_elems_b < (1u << 28) &&
                   (!b->counts || (aligned16(b->counts) && (b->counts_stride % 4u) == 0u));
  bool any_pen = false, any_greedy = false, any_top = b->logprobs != 0u, any_nuc = false;
  bool any_spec = false;
  for (uint32_t r = 0; r < b->rows; r++) {
    const RowParams& rp = h_params[r];
    any_pen |= (rp.flags & fg::kRowPenalties) != 0u;
    any_greedy |= rp.temperature == 0.0f;
    any_top |= rp.temperature > 0.0f;
    any_nuc |= rp.temperature > 0.0f && rp.top_k == 0u;
    any_spec |= rp.temperature > 0.0f &&
                (rp.top_k == 0u ? fg::kMaxK : (rp.top_k > b->logprobs ? rp.top_k : b->logprobs)) >
                    fg::kSpecMinK;
  }
  any_pen = any_pen && b->counts != nullptr;
  // Speculation only runs over short slices (the kernel's own condition); a
  // launch without it streams in shorter steps.
  any_spec = any_spec && (a.wave_elems > a.wave_elems_b ? a.wave_elems : a.wave_elems_b) <=
                             fg::kSpecMaxElems;
  const int bits = (any_pen ? 1 : 0) | (any_greedy ? 2 : 0) | (any_top ? 4 : 0) |
                   (b->logprobs ? 8 : 0) | (any_nuc ? 16 : 0) | (any_spec ? 32 : 0);
  const uint32_t grid = b->rows * chunks;
  // The finisher waits for the other workgroups of its row: only when the
  // whole grid fits on the device at once (occupancy x CUs) is every one of
  // them sure to run while it waits.  Otherwise the last arriver finishes.
  if (finisher && static_cast<uint64_t>(grid) <=
                      static_cast<uint64_t>(occupancy(vec ? bits : 64)) * w.cus) {
    uint32_t epoch = 0u;
    const hipError_t e = next_epoch(w, stream, &epoch);
    if (e != hipSuccess) return hip_fail(err, e, "sampler epoch");
    a.finisher = finisher | epoch << 16;
    // s_memrealtime runs at 100 MHz; limits up to 42.9 s fit.
    const uint64_t ticks = w.tuning.wait_us * 100u;
    a.wait_ticks = ticks < UINT32_MAX ? static_cast<uint32_t>(ticks) : UINT32_MAX;
  }
  (vec ? kVecLaunch[bits] : kScalarLaunch)(grid, stream, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FG_OK : hip_fail(err, e, "sampler launch");
}

}  // namespace

extern "C" {

fg_status fg_hip_apply_penalties(float* logits, const uint32_t* counts, uint32_t values,
                                 float presence_penalty, float frequency_penalty,
                                 float repetition_penalty, void* stream, fg_error* err) {
  if (!logits || !counts || !values || !isfinite(presence_penalty) ||
      !isfinite(frequency_penalty) || !isfinite(repetition_penalty) ||
      repetition_penalty <= 0.0f)
    return arg_fail(err, "invalid vocabulary penalty dispatch");
  const uint32_t quads = (values + 3u) / 4u;
  const uint32_t blocks = (quads + 255u) / 256u;
  if (aligned16(logits) && aligned16(counts))
    fg::apply_penalties_kernel<true><<<blocks, 256, 0, as_stream(stream)>>>(
        logits, counts, values, presence_penalty, frequency_penalty, repetition_penalty);
  else
    fg::apply_penalties_kernel<false><<<blocks, 256, 0, as_stream(stream)>>>(
        logits, counts, values, presence_penalty, frequency_penalty, repetition_penalty);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FG_OK : hip_fail(err, e, "penalty launch");
}

fg_status fg_hip_argmax_reduce(float* output_scores, uint32_t* output_ids,
                               const float* input_scores, const uint32_t* input_ids,
                               uint32_t count, uint32_t* output_count, void* stream,
                               fg_error* err) {
  if (!output_scores || !output_ids || !input_scores || !count || !output_count)
    return arg_fail(err, "invalid argmax reduction dispatch");
  const uint32_t groups = (count + 4095u) / 4096u;
  fg::argmax_reduce_kernel<<<groups, 256, 0, as_stream(stream)>>>(output_scores, output_ids,
                                                                   input_scores, input_ids, count);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(err, e, "argmax launch");
  *output_count = groups;
  return FG_OK;
}

fg_status fg_hip_topk_select(float* output_scores, uint32_t* output_ids,
                             const float* input_scores, const uint32_t* input_ids,
                             uint32_t count, uint32_t k, uint32_t* output_count, void* stream,
                             fg_error* err) {
  const uint32_t groups = (count + 1023u) / 1024u;
  const uint64_t produced = static_cast<uint64_t>(groups) * k;
  if (!output_scores || !output_ids || !input_scores || !count || k < 1u || k > 64u ||
      !output_count || produced > UINT32_MAX)
    return arg_fail(err, "invalid generation top-k selection dispatch");
  fg::topk_select_kernel<<<groups, 256, 0, as_stream(stream)>>>(output_scores, output_ids,
                                                                 input_scores, input_ids, count, k);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(err, e, "top-k launch");
  *output_count = static_cast<uint32_t>(produced);
  return FG_OK;
}

fg_status fg_hip_topk_reduce(float* output_scores, uint32_t* output_ids,
                             const float* input_scores, const uint32_t* input_ids, uint32_t count,
                             uint32_t* output_count, void* stream, fg_error* err) {
  if (!output_scores || !output_ids || !input_scores || !count || !output_count) {
    fg_error_set(err, FG_ERR_ARGUMENT, "invalid top-k reduction dispatch");
    return FG_ERR_ARGUMENT;
  }
  const uint32_t tiles = (count + fg::kReduceTile - 1u) / fg::kReduceTile;
  const uint32_t produced = (tiles == 1u && count < fg::kReduceKeep) ? count : tiles * fg::kReduceKeep;
  const uint32_t per_tile = tiles == 1u ? produced : fg::kReduceKeep;
  fg::topk_reduce_kernel<<<tiles, fg::kReduceBlock, 0, as_stream(stream)>>>(
      output_scores, output_ids, input_scores, input_ids, count, per_tile);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(err, e, "top-k reduction launch");
  *output_count = produced;
  return FG_OK;
}

uint64_t fg_hip_topk_reduce_all_workspace_bytes(uint32_t count) {
  return fg::reduce_all_bytes((static_cast<uint64_t>(count) + fg::kReduceTile - 1u) / fg::kReduceTile);
}

fg_status fg_hip_topk_reduce_all(float* output_scores, uint32_t* output_ids,
                                 const float* input_scores, const uint32_t* input_ids,
                                 uint32_t count, void* workspace, uint32_t* output_count,
                                 void* stream, fg_error* err) {
  if (!output_scores || !output_ids || !input_scores || !count || !workspace || !output_count ||
      (reinterpret_cast<uintptr_t>(workspace) & 255u))
    return arg_fail(err, "invalid top-k reduction dispatch");
  const uint32_t tiles = (count + fg::kReduceTile - 1u) / fg::kReduceTile;
  // The grid-wide barriers need every tile's workgroup resident at once.
  static std::atomic<int> occ{0};
  int per_cu = occ.load(std::memory_order_relaxed);
  if (!per_cu) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(&fg::topk_reduce_all_kernel), fg::kReduceBlock,
            0) != hipSuccess || per_cu < 0)
      per_cu = 0;
    occ.store(per_cu, std::memory_order_relaxed);
  }
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return hip_fail(err, e, "top-k reduction device");
  if (tiles > fg::kReduceAllMaxTiles ||
      static_cast<uint64_t>(tiles) > static_cast<uint64_t>(per_cu) * static_cast<uint64_t>(cus)) {
    fg_error_set(err, FG_ERR_LIMIT, "%u tiles exceed the workgroups the device holds at once",
                 tiles);
    return FG_ERR_LIMIT;
  }
  const uint32_t out_n = count < fg::kReduceKeep ? count : fg::kReduceKeep;
  // Tiles on the two XCDs that start first, when the padded grid still fits.
  const uint64_t packed_grid = (static_cast<uint64_t>(tiles) + 1u) / 2u * 8u;
  const bool packed = packed_grid <= static_cast<uint64_t>(per_cu) * static_cast<uint64_t>(cus);
  const uint32_t grid = packed ? static_cast<uint32_t>(packed_grid) : tiles;
  fg::topk_reduce_all_kernel<<<grid, fg::kReduceBlock, 0, as_stream(stream)>>>(
      output_scores, output_ids, input_scores, input_ids, count, out_n,
      static_cast<uint8_t*>(workspace), tiles, packed ? 1u : 0u);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(err, e, "top-k reduction launch");
  *output_count = out_n;
  return FG_OK;
}

// Chunk layouts of the owner step's tagged hand-off: 2,048, 4,096 and 8,192
// logits a workgroup.
constexpr uint32_t kSliceLayouts = 3;

struct fg_hip_output_slice {
  uint32_t vocab, ways, first_row, rows, max_batch;
  unsigned long long* d_keys;  // per batch row; zero between calls
  uint32_t* d_arrivals;        // per batch row; zero between calls
  // Tagged hand-off (fg::slice_owner_kernel): words [batch row][chunk] and
  // per-row epochs; the wait limit in s_memrealtime ticks.
  uint64_t* d_words;
  uint32_t* d_epochs;
  uint32_t wait_ticks;
  // Sampled LM-head workspace (fg::LmSampleArgs), for whole-head slices.
  uint32_t wg_cap, grp_cap;
  uint64_t* d_wg_lists;
  uint32_t* d_wg_count;
  uint32_t* d_lm_lines;      // counters, a 128-byte line each; zero between calls
  uint64_t* d_grp_lists;
  uint32_t* d_grp_count;
  fg::LmWork* d_lmwork;         // the pointers above, for the kernel
};

fg_status fg_hip_output_slice_create(fg_hip_output_slice** out, uint32_t vocab, uint32_t ways,
                                     uint32_t first_row, uint32_t rows,
                                     uint32_t max_batch_rows, fg_error* err) {
  if (out) *out = nullptr;
  if (!out || !vocab || vocab == UINT32_MAX || !rows || first_row >= vocab ||
      rows > vocab - first_row || (ways != 1u && ways != 2u && ways != 4u) || !max_batch_rows ||
      max_batch_rows > 65535u)
    return arg_fail(err, "invalid output slice arguments");
  fg_hip_output_slice* s = static_cast<fg_hip_output_slice*>(calloc(1, sizeof(*s)));
  if (!s) {
    fg_error_set(err, FG_ERR_OOM, "output slice");
    return FG_ERR_OOM;
  }
  s->vocab = vocab;
  s->ways = ways;
  s->first_row = first_row;
  s->rows = rows;
  s->max_batch = max_batch_rows;
  hipError_t e = hipMalloc(&s->d_keys, sizeof(unsigned long long) * max_batch_rows);
  if (e == hipSuccess) e = hipMalloc(&s->d_arrivals, sizeof(uint32_t) * max_batch_rows);
  if (e == hipSuccess) e = hipMemset(s->d_keys, 0, sizeof(unsigned long long) * max_batch_rows);
  if (e == hipSuccess) e = hipMemset(s->d_arrivals, 0, sizeof(uint32_t) * max_batch_rows);
  {
    // Words and epochs for each of the owner step's chunk layouts.
    const size_t words = sizeof(uint64_t) * fg::kSliceWordStride * max_batch_rows * kSliceLayouts;
    const size_t epochs = sizeof(uint32_t) * max_batch_rows * kSliceLayouts;
    if (e == hipSuccess) e = hipMalloc(&s->d_words, words);
    if (e == hipSuccess) e = hipMalloc(&s->d_epochs, epochs);
    if (e == hipSuccess) e = hipMemset(s->d_words, 0, words);
    if (e == hipSuccess) e = hipMemset(s->d_epochs, 0, epochs);
    s->wait_ticks = static_cast<uint32_t>(
        std::min<uint64_t>(UINT32_MAX, tuning_from_env().wait_us * 100u));
  }
  if (ways == 1u) {
    // Two tokens per pass: lists of every workgroup and every group.
    s->wg_cap = dense_groups(rows);
    s->grp_cap = (s->wg_cap + fg::kLmGroup - 1u) / fg::kLmGroup;
    const size_t wl = sizeof(uint64_t) * 2u * s->grp_cap * fg::kMaxK * fg::kLmGroup;
    if (e == hipSuccess) e = hipMalloc(&s->d_wg_lists, wl);
    if (e == hipSuccess) e = hipMalloc(&s->d_wg_count, sizeof(uint32_t) * 2u * s->wg_cap);
    // Counters and running values, one 128-byte line each, then the running
    // lists (zero between calls).
    const size_t line = sizeof(uint32_t) * fg::kLineWords;
    const size_t lines = line * 2u * (4u + s->grp_cap);
    if (e == hipSuccess)
      e = hipMalloc(&s->d_grp_lists, sizeof(uint64_t) * 2u * s->grp_cap * fg::kMaxK);
    if (e == hipSuccess) e = hipMalloc(&s->d_grp_count, sizeof(uint32_t) * 2u * s->grp_cap);
    if (e == hipSuccess) e = hipMalloc(&s->d_lm_lines, lines);
    if (e == hipSuccess) e = hipMemset(s->d_lm_lines, 0, lines);
    uint8_t* base = reinterpret_cast<uint8_t*>(s->d_lm_lines);
    fg::LmWork w{};
    w.vocab = vocab;
    w.wg_cap = s->wg_cap;
    w.grp_cap = s->grp_cap;
    w.keys = reinterpret_cast<unsigned long long*>(base);
    w.arrivals = reinterpret_cast<uint32_t*>(base + 2u * line);
    w.bound = reinterpret_cast<unsigned long long*>(base + 4u * line);
    w.fin_arrivals = reinterpret_cast<uint32_t*>(base + 6u * line);
    w.grp_arrivals = reinterpret_cast<uint32_t*>(base + 8u * line);
    w.grp_lists = s->d_grp_lists;
    w.grp_count = s->d_grp_count;
    w.wg_lists = s->d_wg_lists;
    w.wg_count = s->d_wg_count;
    if (e == hipSuccess) e = hipMalloc(&s->d_lmwork, sizeof w);
    if (e == hipSuccess) e = hipMemcpy(s->d_lmwork, &w, sizeof w, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipDeviceSynchronize();
  }
  if (e != hipSuccess) {
    fg_hip_output_slice_destroy(s);
    return hip_fail(err, e, "output slice workspace");
  }
  *out = s;
  return FG_OK;
}

void fg_hip_output_slice_destroy(fg_hip_output_slice* s) {
  if (!s) return;
  (void)hipFree(s->d_keys);
  (void)hipFree(s->d_arrivals);
  (void)hipFree(s->d_words);
  (void)hipFree(s->d_epochs);
  (void)hipFree(s->d_wg_lists);
  (void)hipFree(s->d_wg_count);
  (void)hipFree(s->d_lm_lines);
  (void)hipFree(s->d_grp_lists);
  (void)hipFree(s->d_grp_count);
  (void)hipFree(s->d_lmwork);
  free(s);
}

uint32_t fg_hip_output_slice_ways(const fg_hip_output_slice* s) { return s ? s->ways : 0u; }

namespace {

extern "C++" {
// Whether every workgroup of a slice step's grid can be resident at once
// (the tagged hand-off's finisher waits for the row's other chunks).
template <uint32_t kChunk>
bool slice_grid_resident(uint32_t groups) {
  static std::atomic<int> occ{0};
  int per_cu = occ.load(std::memory_order_relaxed);
  if (!per_cu) {
    int a = 0, b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &a, reinterpret_cast<const void*>(&fg::slice_owner_kernel<true, kChunk>),
            fg::kSliceBlock, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &b, reinterpret_cast<const void*>(&fg::slice_owner_kernel<false, kChunk>),
            fg::kSliceBlock, 0) != hipSuccess)
      return false;
    per_cu = std::min(a, b);
    if (per_cu <= 0) return false;
    occ.store(per_cu, std::memory_order_relaxed);
  }
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return false;
  return static_cast<uint64_t>(groups) <= static_cast<uint64_t>(per_cu) * static_cast<uint64_t>(cus);
}

// The ways' spans checked (they tile [0, vocab)) into `spans`.
bool split_spans(uint32_t ways, uint32_t vocab, const uint32_t* span_first,
                 const uint32_t* span_rows, fg::SplitSpans* spans) {
  static const uint32_t kRanks[fg::kSplitWaysMax] = {4u, 0u, 1u, 2u};
  uint64_t cursor = 0;
  for (uint32_t w = 0; w < ways; w++) {
    if (span_first[w] != cursor || !span_rows[w]) return false;
    cursor += span_rows[w];
    spans->first[w] = span_first[w];
    spans->rows[w] = span_rows[w];
    spans->rank[w] = kRanks[w];
  }
  return cursor == vocab;
}

// The tagged owner step with kChunk logits per workgroup (chunk layout
// `layout`), if its grid has at most kSliceWordStride chunks a row and is
// resident at once.  Each layout has its own words and epochs: a launch
// then rewrites every word its finishers poll, so a word's previous tag is
// always the previous epoch of the same row and layout (with one shared set,
// a word that a layout of fewer chunks leaves alone could keep a tag until
// the row's epoch wraps back to it).
template <uint32_t kChunk>
bool slice_owner_launch(fg_hip_output_slice* s, const float* logits, uint64_t stride,
                        uint32_t batch_rows, float* values, uint32_t* ids, int32_t* row_status,
                        fg::SliceOwner o, uint32_t layout, bool vec, hipStream_t stream) {
  const dim3 grid((s->rows + kChunk - 1u) / kChunk, batch_rows);
  if (grid.x > fg::kSliceWordStride || !slice_grid_resident<kChunk>(grid.x * grid.y))
    return false;
  o.words = s->d_words + static_cast<size_t>(layout) * fg::kSliceWordStride * s->max_batch;
  o.epochs = s->d_epochs + static_cast<size_t>(layout) * s->max_batch;
  if (vec)
    fg::slice_owner_kernel<true, kChunk><<<grid, fg::kSliceBlock, 0, stream>>>(
        values, ids, row_status, logits, stride, s->first_row, s->rows, o);
  else
    fg::slice_owner_kernel<false, kChunk><<<grid, fg::kSliceBlock, 0, stream>>>(
        values, ids, row_status, logits, stride, s->first_row, s->rows, o);
  return true;
}
}  // extern "C++"

// One owner step over the slice: the tagged hand-off when the slice's ids fit
// a word and a grid of 2,048-, 4,096- or 8,192-logit chunks (the smallest
// that fits: more workgroups shorten each one's load chain) is resident at
// once, else one workgroup a row.
hipError_t slice_step(fg_hip_output_slice* s, const float* logits, uint64_t stride,
                      uint32_t batch_rows, float* values, uint32_t* ids, int32_t* row_status,
                      fg::SliceOwner o, hipStream_t stream) {
  const bool vec = aligned16(logits) && stride % 4u == 0u && s->rows % 4u == 0u;
  bool launched = false;
  if (static_cast<uint64_t>(s->first_row) + s->rows <= fg::kWireVocab) {
    o.wait_ticks = s->wait_ticks;
    launched = slice_owner_launch<2048>(s, logits, stride, batch_rows, values, ids, row_status, o,
                                        0u, vec, stream) ||
               slice_owner_launch<4096>(s, logits, stride, batch_rows, values, ids, row_status, o,
                                        1u, vec, stream) ||
               slice_owner_launch<8192>(s, logits, stride, batch_rows, values, ids, row_status, o,
                                        2u, vec, stream);
  }
  if (launched) return hipGetLastError();
  if (vec) {
    fg::slice_row_kernel<true><<<batch_rows, fg::kRowBlock, 0, stream>>>(
        values, ids, row_status, logits, stride, s->first_row, s->rows, o);
  } else {
    fg::slice_row_kernel<false><<<batch_rows, fg::kRowBlock, 0, stream>>>(
        values, ids, row_status, logits, stride, s->first_row, s->rows, o);
  }
  return hipGetLastError();
}

}  // namespace

fg_status fg_hip_output_slice_set_wait_limit(fg_hip_output_slice* s, uint64_t wait_us,
                                             fg_error* err) {
  if (!s || wait_us > 42000000u) return arg_fail(err, "invalid output slice wait limit");
  s->wait_ticks = static_cast<uint32_t>(wait_us * 100u);
  return FG_OK;
}

fg_status fg_hip_output_slice_reduce(fg_hip_output_slice* s, const float* logits,
                                     uint64_t stride, uint32_t batch_rows, float* values,
                                     uint32_t* ids, int32_t* row_status, void* stream,
                                     fg_error* err) {
  if (!s || !logits || !values || !ids || !row_status || !batch_rows ||
      batch_rows > s->max_batch || stride < s->rows)
    return arg_fail(err, "invalid output slice run arguments");
  const hipError_t e = slice_step(s, logits, stride, batch_rows, values, ids, row_status,
                                  fg::SliceOwner{}, as_stream(stream));
  return e == hipSuccess ? FG_OK : hip_fail(err, e, "output slice launch");
}

fg_status fg_hip_output_slice_reduce_combine(
    fg_hip_output_slice* s, const float* logits, uint64_t stride, uint32_t batch_rows,
    const float* part_values, const uint32_t* part_ids, const uint8_t* part_ranks,
    const uint32_t* span_first, const uint32_t* span_rows, uint32_t* tokens, float* logits_out,
    int32_t* row_status, void* stream, fg_error* err) {
  fg::SliceOwner o{};
  if (!s || !logits || !part_values || !part_ids || !part_ranks || !span_first || !span_rows ||
      !tokens || !row_status || !batch_rows || batch_rows > s->max_batch || stride < s->rows ||
      (s->ways != 2u && s->ways != 4u) ||
      !split_spans(s->ways, s->vocab, span_first, span_rows, &o.spans))
    return arg_fail(err, "invalid output slice step arguments");
  o.combine = 1u;
  o.ways = s->ways;
  o.vocab = s->vocab;
  o.part_values = part_values;
  o.part_ids = part_ids;
  o.part_ranks = part_ranks;
  o.tokens = tokens;
  o.logits_out = logits_out;
  const hipError_t e = slice_step(s, logits, stride, batch_rows, nullptr, nullptr, row_status,
                                  o, as_stream(stream));
  return e == hipSuccess ? FG_OK : hip_fail(err, e, "output slice step launch");
}

// ---- Q8_0 cooked matrix-vector products ------------------------------------


fg_status fg_hip_dense_q8_0_cooked(float* output, const void* weights, const float* input,
                                   uint32_t in, uint32_t rows, uint32_t tokens, float scale,
                                   void* stream, fg_error* err) {
  fg::DenseArgs a{};
  if (!output || !weights || !input || !tokens || !dense_geometry(in, rows, &a) ||
      !aligned16(weights) || !aligned16(input))
    return arg_fail(err, "invalid cooked Q8_0 dense dispatch");
  a.w = static_cast<const uint8_t*>(weights);
  a.x = input;
  a.y = output;
  a.scale = scale;
  const hipError_t e = dense_launch<false>(a, tokens, as_stream(stream));
  return e == hipSuccess ? FG_OK : hip_fail(err, e, "cooked Q8_0 dense launch");
}

fg_status fg_hip_output_slice_run_dense(fg_hip_output_slice* s, const void* weights,
                                        const float* hidden, uint32_t in, uint32_t tokens,
                                        float scale, float* values, uint32_t* ids,
                                        int32_t* row_status, float* logits, void* stream,
                                        fg_error* err) {
  fg::DenseArgs a{};
  if (!s || !weights || !hidden || !values || !ids || !row_status || !tokens ||
      tokens > s->max_batch || s->first_row % fg::kCookRows || !dense_geometry(in, s->rows, &a) ||
      !aligned16(weights) || !aligned16(hidden))
    return arg_fail(err, "invalid output slice run arguments");
  a.w = static_cast<const uint8_t*>(weights);
  a.x = hidden;
  a.y = logits;
  a.scale = scale;
  a.first_row = s->first_row;
  a.keys = s->d_keys;
  a.arrivals = s->d_arrivals;
  a.values = values;
  a.ids = ids;
  a.status = row_status;
  const hipError_t e = dense_launch<true>(a, tokens, as_stream(stream));
  return e == hipSuccess ? FG_OK : hip_fail(err, e, "output slice dense launch");
}

fg_status fg_hip_output_slice_run_dense_sampled(
    fg_hip_output_slice* s, const void* weights, const float* hidden, uint32_t in,
    uint32_t tokens, float scale, const fg_sampler_config* configs, const uint32_t* counts,
    uint64_t counts_stride, const float* uniforms, uint32_t* out_tokens, float* out_logits,
    int32_t* row_status, void* stream, fg_error* err) {
  fg::LmSampleArgs a{};
  if (!s || s->ways != 1u || s->first_row != 0u || s->rows != s->vocab || !weights || !hidden ||
      !configs || !uniforms || !out_tokens || !out_logits || !row_status || !tokens ||
      tokens > s->max_batch || (counts && counts_stride < s->vocab) ||
      !dense_geometry(in, s->rows, &a.d) || !aligned16(weights) || !aligned16(hidden))
    return arg_fail(err, "invalid sampled output arguments");
  for (uint32_t t = 0; t < tokens; t++) {
    // src/sampler.c:24-38: 1 <= top_k <= 64, which the candidate lists need.
    if (!config_ok(&configs[t], 0u)) {
      fg_error_set(err, FG_ERR_ARGUMENT, "invalid sampler controls (token %u)", t);
      return FG_ERR_ARGUMENT;
    }
  }
  a.d.w = static_cast<const uint8_t*>(weights);
  a.d.x = hidden;
  a.d.y = nullptr;
  a.d.scale = scale;
  a.d.first_row = 0u;
  a.d.values = out_logits;
  a.d.ids = out_tokens;
  a.d.status = row_status;
  a.counts = counts;
  a.cstride = counts_stride;
  a.uniforms = uniforms;
  a.work = s->d_lmwork;
  const uint32_t groups = dense_groups(s->rows);
  hipStream_t st = as_stream(stream);
  for (uint32_t t0 = 0; t0 < tokens; t0 += kDensePassTokens) {
    a.d.token0 = t0;
    a.d.tokens = tokens - t0 < kDensePassTokens ? tokens - t0 : kDensePassTokens;
    for (uint32_t t = 0; t < 2u; t++)
      a.p[t] = t < a.d.tokens ? row_params(&configs[t0 + t]) : RowParams{};
    // Dynamic LDS holds the staged inputs only (the merges use static arrays).
    if (a.d.tokens == 1u) {
      fg::dense_q8_sample_kernel<1><<<groups, fg::kDenseBlock, sizeof(float) * a.d.in, st>>>(a);
    } else {
      fg::dense_q8_sample_kernel<2><<<groups, fg::kDenseBlock, sizeof(float) * a.d.in * 2u, st>>>(a);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(err, e, "sampled output launch");
  }
  return FG_OK;
}

fg_status fg_hip_output_split_combine(uint32_t* tokens, float* logits_out, int32_t* row_status,
                                      const float* part_values, const uint32_t* part_ids,
                                      const uint8_t* part_ranks, uint32_t rows, uint32_t ways,
                                      uint32_t vocab, const uint32_t* span_first,
                                      const uint32_t* span_rows, void* stream, fg_error* err) {
  if (!tokens || !row_status || !part_values || !part_ids || !part_ranks || !rows ||
      (ways != 2u && ways != 4u) || !vocab || !span_first || !span_rows)
    return arg_fail(err, "invalid output split combine arguments");
  fg::SplitSpans spans{};
  if (!split_spans(ways, vocab, span_first, span_rows, &spans))
    return arg_fail(err, "invalid output split combine arguments");
  fg::split_combine_kernel<<<(rows + 255u) / 256u, 256, 0, as_stream(stream)>>>(
      tokens, logits_out, row_status, part_values, part_ids, part_ranks, rows, ways, vocab,
      spans);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FG_OK : hip_fail(err, e, "output split combine launch");
}

fg_status fg_hip_history_build_wire(uint32_t* counts, uint64_t counts_stride, uint32_t vocab,
                                    const uint8_t* payloads, const uint64_t* offsets,
                                    uint32_t rows, int32_t* row_status, uint8_t* row_slot,
                                    void* stream, fg_error* err) {
  if (!counts || !vocab || !payloads || !offsets || !row_status || !rows ||
      counts_stride < vocab)
    return arg_fail(err, "invalid output history payloads");
  hipStream_t s = as_stream(stream);
  const uint32_t chunks = (vocab + fg::kWireRegion - 1u) / fg::kWireRegion;
  if (static_cast<uint64_t>(rows) * chunks > 0x7fffffffu)
    return arg_fail(err, "invalid output history payloads");
  fg::history_wire_build_kernel<<<rows * chunks, fg::kWireBlock, 0, s>>>(
      counts, counts_stride, vocab, payloads, offsets, row_status, row_slot, chunks);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FG_OK : hip_fail(err, e, "history wire launch");
}

fg_status fg_hip_history_build(uint32_t* counts, uint64_t counts_stride, uint32_t vocab,
                               const uint32_t* ids, const uint64_t* offsets, uint32_t rows,
                               int32_t* row_status, void* stream, fg_error* err) {
  if (!counts || !vocab || !ids || !offsets || !rows || !row_status || counts_stride < vocab)
    return arg_fail(err, "invalid output history");
  const uint32_t chunks = (vocab + fg::kWireRegion - 1u) / fg::kWireRegion;
  if (static_cast<uint64_t>(rows) * chunks > 0x7fffffffull)
    return arg_fail(err, "invalid output history");
  fg::history_ids_build_kernel<<<rows * chunks, fg::kWireBlock, 0, as_stream(stream)>>>(
      counts, counts_stride, vocab, ids, offsets, row_status, chunks);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FG_OK : hip_fail(err, e, "history launch");
}

fg_status fg_sampler_hip_create(fg_sampler_hip** out, uint32_t vocab, uint32_t max_rows,
                                fg_error* err) {
  // Candidate composites hold a 31-bit id.
  if (!out || !vocab || vocab >= 0x80000000u || !max_rows)
    return arg_fail(err, "invalid sampler dimensions");
  *out = nullptr;
  fg_sampler_hip* s = static_cast<fg_sampler_hip*>(calloc(1, sizeof *s));
  if (!s) {
    fg_error_set(err, FG_ERR_OOM, "allocate sampler");
    return FG_ERR_OOM;
  }
  s->vocab = vocab;
  s->ws.max_rows = max_rows;
  s->ws.tuning = tuning_from_env();
  s->ws.epoch = &s->epoch;
  hipError_t e = hipGetDevice(&s->device);
  int cus = 0;
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, s->device);
  s->ws.cus = static_cast<uint32_t>(cus);
  // rows * chunks(rows) <= max(target, kMaxGroups) + rows for every batch
  // size.
  const uint64_t groups_cap =
      s->ws.tuning.target_groups > fg::kMaxGroups ? s->ws.tuning.target_groups : fg::kMaxGroups;
  const uint64_t slots = (groups_cap + max_rows) * fg::kWaves;
  s->ws.slots = slots;
  s->h_params = static_cast<RowParams*>(calloc(max_rows, sizeof(RowParams)));
  if (!s->h_params) {
    free(s);
    fg_error_set(err, FG_ERR_OOM, "allocate sampler");
    return FG_ERR_OOM;
  }
  if (e == hipSuccess) e = hipMalloc(&s->ws.params, sizeof(RowParams) * max_rows);
  if (e == hipSuccess) e = hipMalloc(&s->ws.cand, sizeof(uint64_t) * slots * fg::kMaxK);
  // Hand-off slots start cleared (no word carries an epoch yet).
  if (e == hipSuccess) e = hipMemset(s->ws.cand, 0, sizeof(uint64_t) * slots * fg::kMaxK);
  if (e == hipSuccess) e = hipMalloc(&s->ws.greedy, sizeof(uint64_t) * slots);
  if (e == hipSuccess) e = hipMemset(s->ws.greedy, 0, sizeof(uint64_t) * slots);
  if (e == hipSuccess) e = hipMalloc(&s->ws.spec, sizeof(uint64_t) * slots);
  if (e == hipSuccess) e = hipMalloc(&s->ws.lse, sizeof(double) * slots * 2);
  // (A workgroup slot each: wave slots / kWaves.)
  if (e == hipSuccess)
    e = hipMalloc(&s->ws.zsum, sizeof(double) * ((slots + fg::kWaves - 1) / fg::kWaves) * 3u);
  const size_t done_bytes = sizeof(uint32_t) * fg::kLineWords * max_rows;
  if (e == hipSuccess) e = hipMalloc(&s->ws.row_done, done_bytes);
  if (e == hipSuccess) e = hipMemset(s->ws.row_done, 0, done_bytes);
  if (e == hipSuccess) e = hipMemset(s->ws.params, 0, sizeof(RowParams) * max_rows);
#ifdef FG_SAMPLE_TRACE
  if (e == hipSuccess) e = hipMalloc(&s->ws.trace, sizeof(uint64_t) * 16u * (groups_cap + max_rows));
  if (e == hipSuccess) e = hipMemset(s->ws.trace, 0, sizeof(uint64_t) * 16u * (groups_cap + max_rows));
  if (e == hipSuccess) e = hipMalloc(&s->counters, sizeof(uint64_t) * 16u);
  if (e == hipSuccess) e = hipMemset(s->counters, 0, sizeof(uint64_t) * 16u);
  if (e == hipSuccess)
    e = hipMemcpyToSymbol(HIP_SYMBOL(fg::g_trace_counters), &s->counters, sizeof(uint64_t*));
#endif
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    fg_sampler_hip_destroy(s);
    return hip_fail(err, e, "sampler workspace");
  }
  *out = s;
  return FG_OK;
}

void fg_sampler_hip_destroy(fg_sampler_hip* s) {
  if (!s) return;
  (void)hipFree(s->ws.params);
  (void)hipFree(s->ws.cand);
  (void)hipFree(s->ws.greedy);
  (void)hipFree(s->ws.spec);
  (void)hipFree(s->ws.lse);
  (void)hipFree(s->ws.zsum);
  (void)hipFree(s->ws.row_done);
  (void)hipFree(s->ws.trace);
  free(s->h_params);
  free(s);
}

fg_status fg_sampler_hip_set_wait_limit(fg_sampler_hip* s, uint64_t wait_us, fg_error* err) {
  if (!s || wait_us > 60000000u) return arg_fail(err, "invalid finisher wait limit");
  s->ws.tuning.wait_us = wait_us;
  return FG_OK;
}

fg_status fg_sampler_hip_set_configs(fg_sampler_hip* s, const fg_sampler_config* configs,
                                     uint32_t rows, uint32_t flags, void* stream, fg_error* err) {
  if (!s || !configs || !rows || rows > s->ws.max_rows ||
      (flags & ~FG_SAMPLER_HIP_ALLOW_FULL_VOCAB))
    return arg_fail(err, "invalid sampler configuration batch");
  for (uint32_t r = 0; r < rows; r++) {
    if (!config_ok(&configs[r], flags)) {
      fg_error_set(err, FG_ERR_ARGUMENT, "invalid sampler controls (row %u)", r);
      return FG_ERR_ARGUMENT;
    }
  }
  for (uint32_t r = 0; r < rows; r++) {
    s->h_params[r] = row_params(&configs[r]);
  }
  // The controls travel with the next launch that reads them: in the
  // arguments of the next sample (batches of up to fg::kInlineRows
  // configured rows), else as arguments of fill kernels launched first on
  // that call's stream.  No host copy, no staging buffer, nothing to wait
  // for, and no launch of its own.
  (void)stream;
  s->config_rows = rows;
  s->params_dirty = true;
  return FG_OK;
}

namespace {
// Brings the device table up to date on `stream` with fill kernels.
fg_status flush_params(fg_sampler_hip* s, hipStream_t stream, fg_error* err) {
  if (!s->params_dirty) return FG_OK;
  const hipError_t e = fill_params(s->ws, s->h_params, s->config_rows, stream);
  if (e != hipSuccess) return hip_fail(err, e, "upload sampler configuration");
  s->params_dirty = false;
  return FG_OK;
}
}  // namespace

fg_status fg_sampler_hip_sample(fg_sampler_hip* s, const fg_sampler_hip_batch* b, void* stream,
                                fg_error* err) {
  if (!s || !b || b->rows > s->config_rows)
    return arg_fail(err, "invalid sampled output arguments");
  // Fresh controls ride in this launch's arguments when they fit.
  uint32_t inline_rows = 0u;
  if (s->params_dirty && s->config_rows <= fg::kInlineRows) {
    inline_rows = s->config_rows;
  } else {
    const fg_status st = flush_params(s, as_stream(stream), err);
    if (st != FG_OK) return st;
  }
  const fg_status st =
      sample_launch(s->ws, s->h_params, s->vocab, b, as_stream(stream), inline_rows, err);
  if (st == FG_OK) s->params_dirty = false;
  return st;
}

fg_status fg_sampler_hip_sample_static(uint32_t vocab, const fg_sampler_config* configs,
                                       uint32_t flags, const fg_sampler_hip_batch* b,
                                       void* stream, fg_error* err) {
  if (!configs || !b || !vocab || vocab >= 0x80000000u || !b->rows ||
      (flags & ~FG_SAMPLER_HIP_ALLOW_FULL_VOCAB))
    return arg_fail(err, "invalid sampled output arguments");
  if (b->rows > kStaticMaxRows) {
    fg_error_set(err, FG_ERR_LIMIT, "%u rows exceed the static sampler workspace (%u rows)",
                 b->rows, kStaticMaxRows);
    return FG_ERR_LIMIT;
  }
  RowParams h[kStaticMaxRows];
  for (uint32_t r = 0; r < b->rows; r++) {
    if (!config_ok(&configs[r], flags)) {
      fg_error_set(err, FG_ERR_ARGUMENT, "invalid sampler controls (row %u)", r);
      return FG_ERR_ARGUMENT;
    }
    h[r] = row_params(&configs[r]);
  }
  Workspace w;
  hipError_t e = static_workspace(&w);
  if (e != hipSuccess) return hip_fail(err, e, "static sampler workspace");
  // Controls by value: in the sampling launch's own arguments when they fit,
  // else as arguments of fill kernels launched first.
  uint32_t inline_rows = b->rows;
  if (b->rows > fg::kInlineRows) {
    e = fill_params(w, h, b->rows, as_stream(stream));
    if (e != hipSuccess) return hip_fail(err, e, "static sampler controls");
    inline_rows = 0u;
  }
  return sample_launch(w, h, vocab, b, as_stream(stream), inline_rows, err);
}

fg_status fg_sampler_hip_history_increment(fg_sampler_hip* s, uint32_t* counts,
                                           uint64_t counts_stride, const uint32_t* tokens,
                                           const int32_t* row_status, uint32_t rows, void* stream,
                                           fg_error* err) {
  if (!s || !counts || !tokens || !rows || rows > s->config_rows || counts_stride < s->vocab)
    return arg_fail(err, "invalid output history token");
  const fg_status st = flush_params(s, as_stream(stream), err);
  if (st != FG_OK) return st;
  fg::history_increment_kernel<<<(rows + 255u) / 256u, 256, 0, as_stream(stream)>>>(
      counts, counts_stride, s->vocab, tokens, row_status,
      reinterpret_cast<const uint32_t*>(s->ws.params) + offsetof(RowParams, flags) / 4u,
      sizeof(RowParams) / 4u, rows);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FG_OK : hip_fail(err, e, "history increment launch");
}

#ifdef FG_LM_TRACE
// Copies the sampled LM head's phase timestamps ([workgroup][8]) to the host.
fg_status fg_lm_trace_copy(uint64_t* host, uint64_t count) {
  const hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(fg::g_lm_trace), sizeof(uint64_t) * count);
  return e == hipSuccess ? FG_OK : FG_ERR_UNAVAILABLE;
}
#endif

#ifdef FG_REDUCE_TRACE
// Copies the top-512 reduction's phase timestamps ([tile][32]) to the host.
fg_status fg_reduce_trace_copy(uint64_t* host, uint64_t count) {
  const hipError_t e =
      hipMemcpyFromSymbol(host, HIP_SYMBOL(fg::g_reduce_trace), sizeof(uint64_t) * count);
  return e == hipSuccess ? FG_OK : FG_ERR_UNAVAILABLE;
}
#endif

#ifdef FG_SAMPLE_TRACE
// Copies the last launch's phase timestamps ([workgroup][8]) to the host.
fg_status fg_sampler_hip_trace_copy(fg_sampler_hip* s, uint64_t* host, uint64_t count) {
  const hipError_t e = hipMemcpy(host, s->ws.trace, sizeof(uint64_t) * count, hipMemcpyDeviceToHost);
  return e == hipSuccess ? FG_OK : FG_ERR_UNAVAILABLE;
}
// Copies the event counters (16 u64) to the host and clears them.
fg_status fg_sampler_hip_trace_counters(fg_sampler_hip* s, uint64_t* host) {
  hipError_t e = hipMemcpy(host, s->counters, sizeof(uint64_t) * 16u, hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = hipMemset(s->counters, 0, sizeof(uint64_t) * 16u);
  return e == hipSuccess ? FG_OK : FG_ERR_UNAVAILABLE;
}
#endif

}  // extern "C"

extern "C" fg_status fg_sampler_hip_plan(uint32_t vocab, uint32_t rows, uint32_t traits,
                                         fg_sampler_hip_geometry* out, fg_error* err) {
  if (!out || !vocab || vocab >= 0x80000000u || !rows || (traits & ~3u))
    return arg_fail(err, "invalid geometry arguments");
  plan_geometry(vocab, rows, (traits & FG_SAMPLER_HIP_ROWS_NUCLEUS) != 0u,
                (traits & FG_SAMPLER_HIP_ROWS_UNLIKE_COST) == 0u, tuning_from_env(), out);
  return FG_OK;
}

extern "C" fg_status fg_sampler_hip_block(const fg_sampler_hip_geometry* g, uint32_t vocab,
                                          uint32_t rows, uint32_t block, uint32_t wave,
                                          uint32_t* row, uint32_t* chunk, uint32_t* begin,
                                          uint32_t* end, fg_error* err) {
  if (!g || !row || !chunk || !begin || !end || !vocab || !rows || !g->chunks ||
      g->split > g->chunks || (g->split < g->chunks && (rows % fg::kXcds || 2u * g->split != g->chunks)) ||
      static_cast<uint64_t>(block) >= static_cast<uint64_t>(rows) * g->chunks ||
      wave >= static_cast<uint32_t>(fg::kWaves))
    return arg_fail(err, "invalid block arguments");
  fg::block_row_chunk(block, rows, g->chunks, g->split, row, chunk);
  const uint32_t i = *chunk * fg::kWaves + wave;
  *begin = fg::slice_begin_of(i, g->split, g->wave_elems, g->wave_elems_b, vocab);
  *end = fg::slice_end_of(i, g->split, g->wave_elems, g->wave_elems_b, vocab);
  return FG_OK;
}
