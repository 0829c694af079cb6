// Vocabulary-split greedy output on the device: each rank's slice of the
// logits reduced to one (value, id) finalist per decode row, and the owner's
// combine of the finalists (reference src/output.c:320-344, 484-497;
// src/runtime.c:2440-2466).  The order is fg_output_better's, which is
// greedy_comp's: padding last, non-finite first (lower id), then the larger
// value, then the lower id.
#pragma once

#include <float.h>

#include "fg_device.hpp"

namespace fg {

constexpr uint32_t kSliceBlock = 256;
constexpr uint32_t kSliceWordStride = kWave;  // hand-off words per row: chunks <= 64
constexpr uint32_t kSplitWaysMax = 4;
constexpr int32_t kStatusMismatch = 5;  // FG_ERR_MISMATCH

struct SplitSpans {
  uint32_t first[kSplitWaysMax];
  uint32_t rows[kSplitWaysMax];
  uint32_t rank[kSplitWaysMax];  // rank owning each way
};

// Four logits at x (16-byte aligned) with a non-temporal load: each is read
// once, so it need not stay in the caches (measured 6.00 against 6.46 us for
// the 64-row owner step, 27.1 against 30.4 us for the 1,024-row step).
__device__ __forceinline__ float4 load_quad_nt(const float* x) {
  typedef float v4f __attribute__((ext_vector_type(4)));
  const v4f w = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(x));
  return make_float4(w.x, w.y, w.z, w.w);
}

// The best composite key (greedy_comp order, ids first_row + position) of
// logits [base, base + kChunk) of one row, in every thread.
template <bool kVec, uint32_t kChunk>
__device__ __forceinline__ uint64_t slice_chunk_best(const float* x, uint32_t base,
                                                     uint32_t slice_rows, uint32_t first_row,
                                                     uint64_t* s_best) {
  // Each thread sees its ids in increasing order, so it keeps the first
  // position of its largest key (ties to the lower id) and builds the
  // composite once.
  uint32_t best_key = 0u, best_pos = 0u;
  auto visit = [&](float v, uint32_t pos) {
    uint32_t b = __float_as_uint(v);
    b = b == 0x80000000u ? 0u : b;  // -0 ranks with +0
    const uint32_t flipped = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    const uint32_t key = is_finite_bits(b) ? flipped : 0xffffffffu;
    const bool take = key > best_key;
    best_key = take ? key : best_key;
    best_pos = take ? pos : best_pos;
  };
  if (kVec) {
    constexpr uint32_t kLoads = kChunk / (4u * kSliceBlock);
    float4 q[kLoads];
#pragma unroll
    for (uint32_t l = 0; l < kLoads; l++) {
      const uint32_t i = base + 4u * (l * kSliceBlock + threadIdx.x);
      q[l] = i < slice_rows ? load_quad_nt(x + i)
                            : make_float4(-FLT_MAX, -FLT_MAX, -FLT_MAX, -FLT_MAX);
    }
    // Past the slice end the lanes hold -FLT_MAX, the smallest finite key:
    // it never beats an earlier real entry of the thread, and a thread whose
    // best is such a lane has best_pos past the end (masked below).
    // While every value is finite the float order is the key order (-0 and
    // +0 compare equal, as their keys do), so the scan keeps the first
    // largest value and its slot l * 4 + component (four instructions per
    // logit); v * 0 accumulates to NaN once a value is non-finite, and only
    // then are the keys built.
    float bv = -INFINITY, bad = 0.0f;
    uint32_t slot = 0u;
    auto scan = [&](float v, uint32_t s) {
      bad = __builtin_fmaf(v, 0.0f, bad);
      const bool take = v > bv;
      bv = take ? v : bv;
      slot = take ? s : slot;
    };
#pragma unroll
    for (uint32_t l = 0; l < kLoads; l++) {
      scan(q[l].x, 4u * l);
      scan(q[l].y, 4u * l + 1u);
      scan(q[l].z, 4u * l + 2u);
      scan(q[l].w, 4u * l + 3u);
    }
    if (bad == 0.0f) {
      uint32_t b = __float_as_uint(bv);
      b = b == 0x80000000u ? 0u : b;
      best_key = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
      best_pos = base + 4u * ((slot >> 2) * kSliceBlock + threadIdx.x) + (slot & 3u);
    } else {
#pragma unroll
      for (uint32_t l = 0; l < kLoads; l++) {
        const uint32_t i = base + 4u * (l * kSliceBlock + threadIdx.x);
        visit(q[l].x, i);
        visit(q[l].y, i + 1u);
        visit(q[l].z, i + 2u);
        visit(q[l].w, i + 3u);
      }
    }
  } else {
    const uint32_t end = min(base + kChunk, slice_rows);
    for (uint32_t i = base + threadIdx.x; i < end; i += kSliceBlock) visit(x[i], i);
  }
  uint64_t best = best_key && best_pos < slice_rows
                      ? (static_cast<uint64_t>(best_key) << 32) | ~(first_row + best_pos)
                      : 0ull;
  best = wave_max_u64(best);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  if (lane_id() == 0) s_best[wave] = best;
  __syncthreads();
#pragma unroll
  for (uint32_t w = 0; w < kSliceBlock / kWave; w++) best = max(best, s_best[w]);
  return best;
}

// A row's finalist from its best composite k (never 0: every slice row has
// a real id).  A finite nonzero value is its key unflipped; a non-finite one
// or a zero is reloaded so the finalist keeps its exact bits (NaN payload,
// sign of zero).
__device__ __forceinline__ float finalist_value(uint64_t k, const float* x, uint32_t first_row) {
  const uint32_t hi = static_cast<uint32_t>(k >> 32);
  return hi == 0xffffffffu || hi == 0x80000000u ? x[greedy_id(k) - first_row] : key_to_float(hi);
}

// The owner's combine of one row (src/runtime.c:2440-2466): finalist 0 is
// (value0, id0), the owner's own; finalist i >= 1 is part_*[row * ways + i],
// sent by rank part_ranks[...], and is checked against that rank's span
// before it is combined.  Ties keep the finalist combined so far.
struct RowParts {  // the finalists other ranks sent for one row (index i >= 1)
  float v[kSplitWaysMax];
  uint32_t id[kSplitWaysMax], rank[kSplitWaysMax];
};
__device__ __forceinline__ RowParts load_parts(uint32_t row, const float* part_values,
                                               const uint32_t* part_ids, const uint8_t* part_ranks,
                                               uint32_t ways) {
  const uint64_t at = static_cast<uint64_t>(row) * ways;
  RowParts p;
#pragma unroll
  for (uint32_t i = 0; i < kSplitWaysMax; i++) {
    const bool in = i >= 1u && i < ways;
    p.v[i] = in ? part_values[at + i] : 0.0f;
    p.id[i] = in ? part_ids[at + i] : 0u;
    p.rank[i] = in ? part_ranks[at + i] : 0u;
  }
  return p;
}
__device__ inline void combine_row(uint32_t row, float value0, uint32_t id0, const RowParts& parts,
                                   uint32_t ways, uint32_t vocab, const SplitSpans& spans,
                                   uint32_t* tokens, float* logits_out, int32_t* row_status) {
  const float* pv = parts.v;
  const uint32_t* pid = parts.id;
  const uint32_t* prank = parts.rank;
  float value = value0;
  uint32_t id = id0;
  uint64_t best = greedy_comp(value, id);
  bool ok = true;
#pragma unroll
  for (uint32_t i = 1; i < kSplitWaysMax; i++) {
    if (i >= ways) break;
    uint32_t way = kSplitWaysMax;
#pragma unroll
    for (uint32_t w = 0; w < kSplitWaysMax; w++)
      if (w < ways && spans.rank[w] == prank[i]) way = w;
    const uint32_t first = way < kSplitWaysMax ? spans.first[way] : 0u;
    const uint32_t n = way < kSplitWaysMax ? spans.rows[way] : 0u;
    ok = ok && way < kSplitWaysMax && pid[i] >= first && pid[i] - first < n;
    const uint64_t c = greedy_comp(pv[i], pid[i]);
    if (c > best) {
      best = c;
      value = pv[i];
      id = pid[i];
    }
  }
  ok = ok && id < vocab && is_finite_bits(__float_as_uint(value));
  tokens[row] = ok ? id : kInvalidId;
  if (logits_out) logits_out[row] = value;
  row_status[row] = ok ? 0 : kStatusMismatch;
}

// One thread per decode row; finalist 0 of a row is the owner's own.
__global__ __launch_bounds__(256) void split_combine_kernel(
    uint32_t* tokens, float* logits_out, int32_t* row_status, const float* part_values,
    const uint32_t* part_ids, const uint8_t* part_ranks, uint32_t rows, uint32_t ways,
    uint32_t vocab, SplitSpans spans) {
  const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  const uint64_t at = static_cast<uint64_t>(row) * ways;
  // All of the row's finalists are loaded before any is examined.
  const RowParts parts = load_parts(row, part_values, part_ids, part_ranks, ways);
  combine_row(row, part_values[at], part_ids[at], parts, ways, vocab, spans, tokens, logits_out,
              row_status);
}

// The owner's step: where the tagged hand-off's words and epochs live, and the
// combine's inputs (combine != 0).
struct SliceOwner {
  uint64_t* words;   // [row * kSliceWordStride + c]
  uint32_t* epochs;  // [row] launches of the row finished
  uint32_t wait_ticks;  // chunk 0's wait limit, s_memrealtime ticks (100 MHz)
  uint32_t combine;     // 1: combine with the other ways' finalists
  uint32_t ways, vocab;
  const float* part_values;
  const uint32_t* part_ids;
  const uint8_t* part_ranks;
  uint32_t* tokens;
  float* logits_out;
  SplitSpans spans;
};
constexpr int32_t kStatusUnavailable = 7;  // FG_ERR_UNAVAILABLE: the finisher's wait gave up

// ---- the owner's step, one workgroup a row ----------------------------------------
//
// Batches whose tagged-hand-off grid would not be resident at once (or
// slices whose ids reach kWireVocab): one workgroup of kRowBlock threads
// streams a row's whole slice in rounds (every thread's non-temporal float4
// loads of a kRowUnroll-deep round in flight at once) and finishes it, with
// no hand-off between workgroups.  At 1,024 rows of a 4-way slice: 27.1 us a
// step with the combine (512 threads; 1,024 threads 28.9, 256 threads 27.4;
// two buffers taking turns did not help), against 33.1 for the earlier
// per-chunk atomic hand-off plus a combine launch.  The scan is the chunk scan's (first
// largest value and its position per thread, keys only once a non-finite
// value shows up).
constexpr uint32_t kRowBlock = 512;
constexpr uint32_t kRowUnroll = 10;  // float4 loads per thread per round

template <bool kVec>
__global__ __launch_bounds__(kRowBlock) void slice_row_kernel(
    float* values, uint32_t* ids, int32_t* row_status, const float* logits, uint64_t stride,
    uint32_t first_row, uint32_t slice_rows, SliceOwner o) {
  __shared__ uint64_t s_best[kRowBlock / kWave];
  const uint32_t row = blockIdx.x;
  const float* x = logits + static_cast<uint64_t>(row) * stride;
  RowParts parts{};
  if (o.combine && threadIdx.x == 0u)
    parts = load_parts(row, o.part_values, o.part_ids, o.part_ranks, o.ways);
  uint32_t best_key = 0u, best_pos = 0u;
  auto visit = [&](float v, uint32_t pos) {
    uint32_t b = __float_as_uint(v);
    b = b == 0x80000000u ? 0u : b;
    const uint32_t flipped = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    const uint32_t key = is_finite_bits(b) ? flipped : 0xffffffffu;
    const bool take = key > best_key;
    best_key = take ? key : best_key;
    best_pos = take ? pos : best_pos;
  };
  if (kVec) {
    constexpr uint32_t kRound = 4u * kRowBlock * kRowUnroll;
    auto load = [&](float4 (&q)[kRowUnroll], uint32_t base) {
#pragma unroll
      for (uint32_t l = 0; l < kRowUnroll; l++) {
        const uint32_t i = base + 4u * (l * kRowBlock + threadIdx.x);
        q[l] = i < slice_rows ? load_quad_nt(x + i)
                              : make_float4(-FLT_MAX, -FLT_MAX, -FLT_MAX, -FLT_MAX);
      }
    };
    auto consume = [&](const float4 (&q)[kRowUnroll], uint32_t base) {
      // As in slice_chunk_best: float order while every value is finite.
      float bv = -INFINITY, bad = 0.0f;
      uint32_t slot = 0u;
      auto scan = [&](float v, uint32_t s) {
        bad = __builtin_fmaf(v, 0.0f, bad);
        const bool take = v > bv;
        bv = take ? v : bv;
        slot = take ? s : slot;
      };
#pragma unroll
      for (uint32_t l = 0; l < kRowUnroll; l++) {
        scan(q[l].x, 4u * l);
        scan(q[l].y, 4u * l + 1u);
        scan(q[l].z, 4u * l + 2u);
        scan(q[l].w, 4u * l + 3u);
      }
      if (bad == 0.0f) {
        const uint32_t pos = base + 4u * ((slot >> 2) * kRowBlock + threadIdx.x) + (slot & 3u);
        visit(bv, pos < slice_rows ? pos : 0xffffffffu);
      } else {
#pragma unroll
        for (uint32_t l = 0; l < kRowUnroll; l++) {
          const uint32_t i = base + 4u * (l * kRowBlock + threadIdx.x);
          visit(q[l].x, i);
          visit(q[l].y, i + 1u);
          visit(q[l].z, i + 2u);
          visit(q[l].w, i + 3u);
        }
      }
    };
    for (uint32_t base = 0; base < slice_rows; base += kRound) {
      float4 q[kRowUnroll];
      load(q, base);
      consume(q, base);
    }
  } else {
    for (uint32_t i = threadIdx.x; i < slice_rows; i += kRowBlock) visit(x[i], i);
  }
  uint64_t best = best_key && best_pos < slice_rows
                      ? (static_cast<uint64_t>(best_key) << 32) | ~(first_row + best_pos)
                      : 0ull;
  best = wave_max_u64(best);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  if (lane_id() == 0) s_best[wave] = best;
  __syncthreads();
  if (threadIdx.x != 0) return;
#pragma unroll
  for (uint32_t w = 1; w < kRowBlock / kWave; w++) best = max(best, s_best[w]);
  const float v = finalist_value(best, x, first_row);
  if (o.combine) {
    combine_row(row, v, greedy_id(best), parts, o.ways, o.vocab, o.spans, o.tokens, o.logits_out,
                row_status);
  } else {
    values[row] = v;
    ids[row] = greedy_id(best);
    row_status[row] = is_finite_bits(__float_as_uint(v)) ? 0 : kStatusMismatch;
  }
}

// ---- the owner's step with the tagged hand-off ------------------------------------
//
// Grid (chunks, batch rows), every workgroup resident at once.  The last
// chunk (the slice's remainder, usually the shortest) finishes the row: the
// others store their best as a tagged word (greedy payload: ids below
// kWireVocab) and end; it polls the row's words until each carries the row's
// epoch, takes the best, and either writes the row's finalist or combines it
// with the other ways' finalists (loaded when it starts).  The epoch of row r
// is epochs[r] % 8191 + 1, read by every chunk when it starts; the finisher
// advances epochs[r] once it has every word (or has given up), so a word
// left from an earlier launch always carries an older epoch, and replays of
// a captured launch stay exact.  The words and epochs passed in belong to
// this launch's chunk size (the host keeps a set per size, a row's words at a
// fixed stride), so every word a finisher polls was written by the previous
// launch of the same row and size.

template <bool kVec, uint32_t kChunk>
__global__ __launch_bounds__(kSliceBlock) void slice_owner_kernel(
    float* values, uint32_t* ids, int32_t* row_status, const float* logits, uint64_t stride,
    uint32_t first_row, uint32_t slice_rows, SliceOwner o) {
  __shared__ uint64_t s_best[kSliceBlock / kWave];
  const uint32_t row = blockIdx.y, chunk = blockIdx.x, chunks = gridDim.x;
  const uint32_t fin = chunks - 1u;
  const uint32_t lane = lane_id();
  // A plain load: only an earlier launch writes the row's epoch (this one's
  // finisher advances it after every chunk has read it and published), and
  // the kernel boundary makes that store visible.  A device-scope load here
  // would hold up the chunk's first data loads behind its longer round trip.
  const uint32_t launches = o.epochs[row];
  RowParts parts{};
  if (o.combine && chunk == fin && threadIdx.x == 0u)
    parts = load_parts(row, o.part_values, o.part_ids, o.part_ranks, o.ways);
  const float* x = logits + static_cast<uint64_t>(row) * stride;
  const uint64_t best = slice_chunk_best<kVec, kChunk>(x, chunk * kChunk, slice_rows, first_row, s_best);
  if (threadIdx.x >= static_cast<uint32_t>(kWave)) return;
  const uint64_t header = wire_header(launches % kMaxEpoch + 1u);
  uint64_t* const words = o.words + static_cast<uint64_t>(row) * kSliceWordStride;
  if (chunk != fin) {
    if (lane == 0u)
      __hip_atomic_store(words + chunk, header | greedy_payload(best), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  // Lane c (c < fin) polls chunk c's word.
  const bool mine = lane < fin;
  uint64_t w = 0ull;
  bool gave_up = false;
  uint64_t t0 = 0ull;
  for (uint32_t spin = 0;; spin++) {
    if (mine && !wire_current(w, header))
      w = __hip_atomic_load(words + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (ballot(mine && !wire_current(w, header)) == 0ull) break;
    if (o.wait_ticks == 0u) {
      gave_up = true;
      break;
    }
    if (spin % 32u == 0u) {
      const uint64_t now = __builtin_amdgcn_s_memrealtime();
      if (spin == 0u) t0 = now;
      if (now - t0 > o.wait_ticks) {
        gave_up = true;
        break;
      }
    }
    __builtin_amdgcn_s_sleep(1);
  }
  uint64_t k = mine ? greedy_of_payload(w & kWirePayload) : lane == fin ? best : 0ull;
  k = wave_max_u64(k);
  if (lane != 0u) return;
  __hip_atomic_store(o.epochs + row, launches + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (gave_up) {
    if (o.combine) {
      o.tokens[row] = kInvalidId;
      if (o.logits_out) o.logits_out[row] = -INFINITY;
    } else {
      values[row] = -INFINITY;
      ids[row] = kInvalidId;
    }
    row_status[row] = kStatusUnavailable;
    return;
  }
  const float v = finalist_value(k, x, first_row);
  if (o.combine) {
    combine_row(row, v, greedy_id(k), parts, o.ways, o.vocab, o.spans, o.tokens, o.logits_out,
                row_status);
  } else {
    values[row] = v;
    ids[row] = greedy_id(k);
    row_status[row] = is_finite_bits(__float_as_uint(v)) ? 0 : kStatusMismatch;
  }
}

}  // namespace fg
