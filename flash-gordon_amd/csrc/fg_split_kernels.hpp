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
constexpr uint32_t kSliceChunk = 8192;  // logits per workgroup: 8 float4 per thread
constexpr uint32_t kSplitWaysMax = 4;
constexpr int32_t kStatusMismatch = 5;  // FG_ERR_MISMATCH

struct SplitSpans {
  uint32_t first[kSplitWaysMax];
  uint32_t rows[kSplitWaysMax];
  uint32_t rank[kSplitWaysMax];  // rank owning each way
};

// Grid (chunks, batch rows).  Each workgroup reduces kSliceChunk logits of
// one row to its best composite key and folds it into keys[row] with an
// atomic max; the workgroup that arrives last decodes the row's finalist and
// returns keys[row] and arrivals[row] to zero for the next call.
template <bool kVec>
__global__ __launch_bounds__(kSliceBlock) void slice_finalist_kernel(
    float* values, uint32_t* ids, int32_t* row_status, const float* logits, uint64_t stride,
    uint32_t first_row, uint32_t slice_rows, unsigned long long* keys, uint32_t* arrivals) {
  __shared__ uint64_t s_best[kSliceBlock / kWave];
  const uint32_t row = blockIdx.y;
  const float* x = logits + static_cast<uint64_t>(row) * stride;
  const uint32_t base = blockIdx.x * kSliceChunk;
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
    constexpr uint32_t kLoads = kSliceChunk / (4u * kSliceBlock);
    float4 q[kLoads];
#pragma unroll
    for (uint32_t l = 0; l < kLoads; l++) {
      const uint32_t i = base + 4u * (l * kSliceBlock + threadIdx.x);
      q[l] = i < slice_rows ? *reinterpret_cast<const float4*>(x + i)
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
    const uint32_t end = min(base + kSliceChunk, slice_rows);
    for (uint32_t i = base + threadIdx.x; i < end; i += kSliceBlock) visit(x[i], i);
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
  for (uint32_t w = 1; w < kSliceBlock / kWave; w++) best = max(best, s_best[w]);
  // Device-scope (sc1) atomics meet at the device's coherence point; the
  // wait orders the max before the arrival count without the L2 write-back
  // and invalidate an acquire-release fence would cost every workgroup.
  __hip_atomic_fetch_max(keys + row, static_cast<unsigned long long>(best), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  wait_memory();  // hand-off ordering: see wait_memory()
  const uint32_t arrived =
      __hip_atomic_fetch_add(arrivals + row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (arrived + 1u != gridDim.x) return;
  const uint64_t k = __hip_atomic_exchange(keys + row, 0ull, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(arrivals + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // Every slice row has a real id, so k != 0.  A finite nonzero value is
  // its key unflipped; a non-finite one or a zero is reloaded so the
  // finalist keeps its exact bits (NaN payload, sign of zero).
  const uint32_t local = greedy_id(k) - first_row;
  const uint32_t hi = static_cast<uint32_t>(k >> 32);
  const float v = hi == 0xffffffffu || hi == 0x80000000u ? x[local] : key_to_float(hi);
  values[row] = v;
  ids[row] = first_row + local;
  row_status[row] = is_finite_bits(__float_as_uint(v)) ? 0 : kStatusMismatch;
}

// One thread per decode row.  Finalist 0 of a row is the owner's own; the
// others come with the rank that sent them and are checked against that
// rank's span before they are combined, as the owner checks them.
__global__ __launch_bounds__(256) void split_combine_kernel(
    uint32_t* tokens, float* logits_out, int32_t* row_status, const float* part_values,
    const uint32_t* part_ids, const uint8_t* part_ranks, uint32_t rows, uint32_t ways,
    uint32_t vocab, SplitSpans spans) {
  const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  const uint64_t at = static_cast<uint64_t>(row) * ways;
  // All of the row's finalists are loaded before any is examined.
  float pv[kSplitWaysMax];
  uint32_t pid[kSplitWaysMax], prank[kSplitWaysMax];
#pragma unroll
  for (uint32_t i = 0; i < kSplitWaysMax; i++) {
    const bool in = i < ways;
    pv[i] = in ? part_values[at + i] : 0.0f;
    pid[i] = in ? part_ids[at + i] : 0u;
    prank[i] = in && i ? part_ranks[at + i] : 0u;
  }
  float value = pv[0];
  uint32_t id = pid[0];
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
    if (c > best) {  // ties keep the finalist combined so far
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

}  // namespace fg
