// gfx950 kernels behind the unit entry points that stand in for the
// reference's Vulkan dispatches (src/vk.c:1808-1823, 2237-2260) and its
// history table upkeep (src/output.c:601-628).
#pragma once

#include "fg_device.hpp"

namespace fg {

// shaders/fg_apply_penalties.comp, with the C rounding of src/sampler.c:55-58.
// Each thread owns 4 consecutive logits (one 16-byte access when aligned).
template <bool kVec>
__global__ __launch_bounds__(256) void apply_penalties_kernel(float* logits, const uint32_t* counts,
                                                            uint32_t values, float pres, float freq,
                                                            float rep) {
  const uint32_t quads = (values + 3u) / 4u;
  for (uint32_t q = blockIdx.x * blockDim.x + threadIdx.x; q < quads; q += gridDim.x * blockDim.x) {
    const uint32_t i = q * 4u;
    if (kVec && i + 3u < values) {
      const u4 c = *reinterpret_cast<const u4*>(counts + i);
      if ((c.x | c.y | c.z | c.w) == 0u) continue;
      f4 v = *reinterpret_cast<const f4*>(logits + i);
      v.x = penalise(v.x, c.x, pres, freq, rep);
      v.y = penalise(v.y, c.y, pres, freq, rep);
      v.z = penalise(v.z, c.z, pres, freq, rep);
      v.w = penalise(v.w, c.w, pres, freq, rep);
      *reinterpret_cast<f4*>(logits + i) = v;
    } else {
      for (uint32_t e = 0; e < 4u && i + e < values; e++) {
        const uint32_t c = counts[i + e];
        if (c) logits[i + e] = penalise(logits[i + e], c, pres, freq, rep);
      }
    }
  }
}

// One argmax step over 4096-element slices (shaders/fg_argmax_reduce.comp):
// greedy composites are max-reduced, the winner's value travels with it.
__global__ __launch_bounds__(256) void argmax_reduce_kernel(float* out_scores, uint32_t* out_ids,
                                                          const float* in_scores,
                                                          const uint32_t* in_ids, uint32_t count) {
  __shared__ uint64_t s_comp[4];
  __shared__ float s_val[4];
  const uint32_t base = blockIdx.x * 4096u;
  uint64_t best = 0ull;
  float best_v = -INFINITY;
  for (uint32_t k = threadIdx.x; k < 4096u; k += 256u) {
    const uint32_t i = base + k;
    if (i >= count) break;
    const float v = in_scores[i];
    const uint32_t id = in_ids ? in_ids[i] : i;
    const uint64_t g = greedy_comp(v, id);
    if (g > best) { best = g; best_v = v; }
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const uint64_t o = __shfl_xor(best, d);
    const float ov = __shfl_xor(best_v, d);
    if (o > best) { best = o; best_v = ov; }
  }
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // uniform
  if (lane_id() == 0) { s_comp[wave] = best; s_val[wave] = best_v; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; w++)
      if (s_comp[w] > best) { best = s_comp[w]; best_v = s_val[w]; }
    out_scores[blockIdx.x] = best ? best_v : -INFINITY;
    out_ids[blockIdx.x] = best ? greedy_id(best) : kInvalidId;
  }
}

// One top-k step over 1024-element tiles (shaders/fg_topk_select.comp): exact
// top min(k, tile) finite entries by (key desc, position asc), emitted in tile
// order, padded with (-inf, invalid).  Thread t owns positions 4t..4t+3.
__global__ __launch_bounds__(256) void topk_select_kernel(float* out_scores, uint32_t* out_ids,
                                                        const float* in_scores,
                                                        const uint32_t* in_ids, uint32_t count,
                                                        uint32_t k) {
  __shared__ uint64_t s_buf[1024];
  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_wave_sel[4];
  __shared__ uint32_t s_finite;
  __shared__ uint64_t s_R;
  const uint32_t t = threadIdx.x;
  const uint32_t wave = t / kWave;
  const uint32_t lane = lane_id();
  const uint32_t base = blockIdx.x * 1024u;
  const uint32_t avail = min(1024u, count - base);
  const uint32_t limit = min(k, avail);
  if (t == 0) s_finite = 0u;
  __syncthreads();
  uint64_t comp[4];
  uint32_t nfin = 0;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const uint32_t pos = 4u * t + e;
    uint32_t key = 0u;
    if (pos < avail) key = float_key(in_scores[base + pos]);
    comp[e] = key ? make_comp(key, pos) : 0ull;
    s_buf[pos] = comp[e];
    nfin += key ? 1u : 0u;
  }
  atomicAdd(&s_finite, nfin);
  __syncthreads();
  const uint32_t take = min(limit, s_finite);
  if (wave == 0) {
    uint64_t R = kFiniteComp;  // every finite entry
    if (take > 0u && take < s_finite) R = wave_select_kth(s_buf, 1024u, take, s_hist);
    if (lane == 0) s_R = R;
  }
  __syncthreads();
  const uint64_t R = s_R;
  uint32_t mine = 0;
#pragma unroll
  for (int e = 0; e < 4; e++) mine += (take > 0u && comp[e] >= R && comp[e] >= kFiniteComp) ? 1u : 0u;
  // Exclusive prefix of `mine` over the workgroup in thread order.
  uint32_t incl = mine;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t o = __shfl_up(incl, d);
    if (lane >= static_cast<uint32_t>(d)) incl += o;
  }
  if (lane == kWave - 1) s_wave_sel[wave] = incl;
  __syncthreads();
  uint32_t off = incl - mine;
  for (uint32_t w = 0; w < wave; w++) off += s_wave_sel[w];
  const uint64_t out_base = static_cast<uint64_t>(blockIdx.x) * k;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    if (take > 0u && comp[e] >= R && comp[e] >= kFiniteComp) {
      const uint32_t pos = 4u * t + e;
      out_scores[out_base + off] = in_scores[base + pos];
      out_ids[out_base + off] = in_ids ? in_ids[base + pos] : base + pos;
      off++;
    }
  }
  for (uint32_t j = take + t; j < k; j += 256u) {
    out_scores[out_base + j] = -INFINITY;
    out_ids[out_base + j] = kInvalidId;
  }
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* dst, uint64_t stride, uint32_t width,
                                                     uint32_t rows, uint32_t value) {
  const uint64_t total = static_cast<uint64_t>(rows) * width;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint64_t r = i / width;
    dst[r * stride + (i - r * width)] = value;
  }
}

__device__ __forceinline__ void saturating_increment(uint32_t* p) {
  uint32_t old = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while (old != 0xffffffffu) {
    const uint32_t seen = atomicCAS(p, old, old + 1u);
    if (seen == old) break;
    old = seen;
  }
}

// src/output.c:601-617 for many rows: counts were cleared by fill_u32_kernel.
// Grid: (blocks per row, rows).  An id >= vocab sets *bad.
__global__ __launch_bounds__(256) void history_count_kernel(uint32_t* counts, uint64_t stride,
                                                          uint32_t vocab, const uint32_t* ids,
                                                          const uint64_t* offsets, uint32_t* bad) {
  const uint32_t r = blockIdx.y;
  const uint64_t b = offsets[r], e = offsets[r + 1];
  for (uint64_t i = b + static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < e;
       i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint32_t id = ids[i];
    if (id >= vocab) {
      atomicOr(bad, 1u);
      continue;
    }
    // A cleared row with fewer than UINT32_MAX ids cannot saturate: a plain
    // atomic add avoids compare-and-swap retries on repeated ids.
    uint32_t* c = counts + static_cast<uint64_t>(r) * stride + id;
    if (e - b < 0xffffffffull)
      atomicAdd(c, 1u);
    else
      saturating_increment(c);
  }
}

// src/output.c:752 / :619-628: one saturating increment per sampled row.
__global__ __launch_bounds__(256) void history_increment_kernel(uint32_t* counts, uint64_t stride,
                                                              uint32_t vocab, const uint32_t* tokens,
                                                              const int32_t* status,
                                                              const uint32_t* row_flags,
                                                              uint32_t flags_stride, uint32_t rows) {
  const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  if (!(row_flags[static_cast<uint64_t>(r) * flags_stride] & 1u)) return;
  if (status && status[r] != 0) return;
  const uint32_t tok = tokens[r];
  if (tok >= vocab) return;
  saturating_increment(counts + static_cast<uint64_t>(r) * stride + tok);
}

// FG_MSG_OUTPUT_HISTORY payloads (src/protocol.c:1348-1366) decoded on the
// device and turned into count tables (src/output.c:601-617), in two
// launches: kWireChunks workgroups per row each validate the whole payload
// and clear their part of the row (the first one writes the row's status),
// then a counting launch adds the row's ids.  A row that fails validation
// keeps its counts; its status says why (FG_ERR_ARGUMENT: shorter than the
// header; FG_ERR_FORMAT: the decoder's other checks).  Payload bytes are
// big-endian and need not be aligned.
constexpr int kWireBlock = 256;
constexpr uint32_t kWireChunks = 16u;  // clearing workgroups per row
constexpr uint32_t kWireHeader = 8u;
constexpr uint32_t kWireMaxCount = 262144u;
constexpr uint32_t kWireMaxSlots = 2u;

__device__ __forceinline__ uint32_t load_be32(const uint8_t* p) {
  return (static_cast<uint32_t>(p[0]) << 24) | (static_cast<uint32_t>(p[1]) << 16) |
         (static_cast<uint32_t>(p[2]) << 8) | static_cast<uint32_t>(p[3]);
}

// Status of row r's payload (0, 2 or 4) and its id count; every thread of
// the workgroup returns the same.
__device__ inline int32_t wire_validate(const uint8_t* p, uint64_t bytes, uint32_t vocab,
                                        uint32_t* count_out, uint8_t* slot_out) {
  __shared__ int32_t s_status;
  __shared__ uint32_t s_count;
  __shared__ uint8_t s_slot;
  if (threadIdx.x == 0) {
    int32_t st = 0;
    uint32_t count = 0u;
    uint8_t slot = 0u;
    if (bytes < kWireHeader) {
      st = 2;  // FG_ERR_ARGUMENT
    } else {
      count = load_be32(p);
      const uint32_t reserved = (static_cast<uint32_t>(p[5]) << 16) |
                                (static_cast<uint32_t>(p[6]) << 8) | p[7];
      if (reserved || p[4] >= kWireMaxSlots || count > kWireMaxCount ||
          kWireHeader + 4ull * count != bytes)
        st = 4;  // FG_ERR_FORMAT
      slot = p[4];
    }
    s_status = st;
    s_count = st == 0 ? count : 0u;
    s_slot = st == 0 ? slot : 0u;
  }
  __syncthreads();
  const uint32_t count = s_count;
  for (uint32_t i = threadIdx.x; i < count; i += kWireBlock)
    if (load_be32(p + kWireHeader + 4u * i) >= vocab) atomicOr(&s_status, 4);
  __syncthreads();
  *count_out = count;
  *slot_out = s_slot;
  return s_status;
}

// Grid kWireChunks * rows: workgroup b clears chunk b % kWireChunks of row
// b / kWireChunks.
__global__ __launch_bounds__(kWireBlock) void history_wire_clear_kernel(
    uint32_t* counts, uint64_t stride, uint32_t vocab, const uint8_t* payloads,
    const uint64_t* offsets, int32_t* row_status, uint8_t* row_slot) {
  const uint32_t r = blockIdx.x / kWireChunks;
  const uint32_t chunk = blockIdx.x - r * kWireChunks;
  const uint8_t* p = payloads + offsets[r];
  uint32_t count;
  uint8_t slot;
  const int32_t st = wire_validate(p, offsets[r + 1] - offsets[r], vocab, &count, &slot);
  if (chunk == 0 && threadIdx.x == 0) {
    row_status[r] = st;
    if (row_slot && st != 2) row_slot[r] = slot;
  }
  if (st != 0) return;
  const uint32_t per = (vocab + kWireChunks - 1u) / kWireChunks;
  const uint32_t begin = chunk * per;
  const uint32_t end = begin + per < vocab ? begin + per : vocab;
  uint32_t* crow = counts + static_cast<uint64_t>(r) * stride;
  for (uint32_t i = begin + threadIdx.x; i < end; i += kWireBlock) crow[i] = 0u;
}

// Grid kWireCountGroups * rows: the ids of each valid row, once the clearing
// launch is done.
constexpr uint32_t kWireCountGroups = 8u;
__global__ __launch_bounds__(kWireBlock) void history_wire_count_kernel(
    uint32_t* counts, uint64_t stride, const uint8_t* payloads, const uint64_t* offsets,
    const int32_t* row_status) {
  const uint32_t r = blockIdx.x / kWireCountGroups;
  const uint32_t g = blockIdx.x - r * kWireCountGroups;
  if (row_status[r] != 0) return;
  const uint8_t* p = payloads + offsets[r];
  const uint32_t count = load_be32(p);
  uint32_t* crow = counts + static_cast<uint64_t>(r) * stride;
  // The row was cleared and holds at most kWireMaxCount ids, so no count can
  // reach UINT32_MAX: a plain atomic add saturates nothing and keeps hot ids
  // (a Zipf history repeats its head tokens) free of compare-and-swap retries.
  for (uint32_t i = g * kWireBlock + threadIdx.x; i < count; i += kWireCountGroups * kWireBlock)
    atomicAdd(crow + load_be32(p + kWireHeader + 4u * i), 1u);
}

// Top-512 reduction of shaders/fg_topk_reduce_v2.comp (src/vk.c:2235): per
// 4096-element tile, the tile's entries in the greedy order of its
// comparator (:9; padding id 0xffffffff last, non-finite first with lower id
// first, then larger value, equal values (0 == -0) by lower id), the first
// min(512, n) written, the rest of the 512 slots padded with (-inf,
// 0xffffffff).  One workgroup per tile sorts (greedy composite, position)
// pairs with a bitonic network in LDS; scores and ids are then copied from
// the input by position, so every bit of a value (NaN payloads, -0) is kept.
constexpr int kReduceBlock = 512;
constexpr uint32_t kReduceTile = 4096u;
constexpr uint32_t kReduceKeep = 512u;

// Per tile: a radix select (eight 8-bit digits, most significant first)
// finds the composite of the tile's min(512, n)-th entry, the entries at or
// above it are compacted into LDS, and only those are sorted.
__global__ __launch_bounds__(kReduceBlock) void topk_reduce_kernel(
    float* out_scores, uint32_t* out_ids, const float* in_scores, const uint32_t* in_ids,
    uint32_t count, uint32_t out_per_tile) {
  constexpr uint32_t kPer = kReduceTile / kReduceBlock;  // entries per thread
  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_sel[3];  // chosen digit, entries above it, entries in it
  __shared__ uint64_t s_key[kReduceKeep];
  __shared__ uint16_t s_pos[kReduceKeep];
  __shared__ uint32_t s_n;
  const uint32_t tid = threadIdx.x;
  const uint32_t base = blockIdx.x * kReduceTile;
  const uint32_t n = min(kReduceTile, count - base);
  uint64_t key[kPer];
#pragma unroll
  for (uint32_t e = 0; e < kPer; e++) {
    const uint32_t i = e * kReduceBlock + tid;
    uint64_t k = 0ull;  // a fill slot of a partial tile: never selected
    if (i < n) {
      const uint32_t id = in_ids ? in_ids[base + i] : base + i;
      // Padding ids rank last among the entries (1).
      k = id == kInvalidId ? 1ull : greedy_comp(in_scores[base + i], id);
    }
    key[e] = k;
  }
  const uint32_t want = min(kReduceKeep, n);
  // Radix select: after digit d, `prefix` holds the top d bytes of the
  // want-th largest key and `rank` its rank among the keys sharing them.
  uint64_t prefix = 0ull;
  uint32_t rank = want;
  int last = 0;  // lowest digit selected: 4 when the top 32 bits settle it
  for (int d = 7; d >= 0; d--) {
    const uint32_t shift = 8u * static_cast<uint32_t>(d);
    const uint64_t hi_mask = d == 7 ? 0ull : ~0ull << (shift + 8u);
    if (tid < 256u) s_hist[tid] = 0u;
    __syncthreads();
#pragma unroll
    for (uint32_t e = 0; e < kPer; e++) {
      const uint32_t i = e * kReduceBlock + tid;
      if (i < n && (key[e] & hi_mask) == prefix)
        atomicAdd(&s_hist[(key[e] >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64u) {
      // Bins from the top: lane l owns bins 255 - 4l .. 252 - 4l.
      uint32_t c[4];
      uint32_t sum = 0u;
#pragma unroll
      for (int b = 0; b < 4; b++) {
        c[b] = s_hist[255u - 4u * tid - b];
        sum += c[b];
      }
      uint32_t before = sum;  // inclusive prefix over lanes, then made exclusive
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(before, o, 64);
        if (tid >= static_cast<uint32_t>(o)) before += t;
      }
      before -= sum;
      uint32_t acc = before;
#pragma unroll
      for (int b = 0; b < 4; b++) {
        if (acc < rank && acc + c[b] >= rank) {
          s_sel[0] = 255u - 4u * tid - b;
          s_sel[1] = acc;
          s_sel[2] = c[b];
        }
        acc += c[b];
      }
    }
    __syncthreads();
    prefix |= static_cast<uint64_t>(s_sel[0]) << shift;
    rank -= s_sel[1];
    const bool settled = d == 4 && s_sel[2] == rank;  // keep every key of this float key
    __syncthreads();
    if (settled) {
      last = 4;
      break;
    }
  }
  // Kept: keys above prefix, and `rank` keys equal to it in the digits
  // selected (all of them when the float key settled it).
  const uint64_t cmp_mask = last == 4 ? ~0ull << 32 : ~0ull;
  if (tid == 0) {
    s_n = 0u;
    s_sel[0] = 0u;
  }
  __syncthreads();
#pragma unroll
  for (uint32_t e = 0; e < kPer; e++) {
    const uint32_t i = e * kReduceBlock + tid;
    const uint64_t km = key[e] & cmp_mask;
    bool keep = i < n && km > prefix;
    if (i < n && km == prefix) keep = atomicAdd(&s_sel[0], 1u) < rank;
    if (keep) {
      const uint32_t at = atomicAdd(&s_n, 1u);
      s_key[at] = key[e];
      s_pos[at] = static_cast<uint16_t>(i);
    }
  }
  __syncthreads();
  // Sort the kept entries (want of them), padded to a power of two with 0.
  uint32_t P = 1u;
  while (P < want) P <<= 1;
  for (uint32_t i = want + tid; i < P; i += kReduceBlock) s_key[i] = 0ull;
  __syncthreads();
  for (uint32_t k = 2u; k <= P; k <<= 1) {
    for (uint32_t j = k >> 1; j > 0u; j >>= 1) {
      for (uint32_t q = tid; q < P / 2u; q += kReduceBlock) {
        const uint32_t lo = 2u * j * (q / j) + (q % j);
        const uint32_t hi = lo + j;
        const uint64_t a = s_key[lo], b = s_key[hi];
        const bool desc = (lo & k) == 0u;
        if (desc ? a < b : a > b) {
          s_key[lo] = b;
          s_key[hi] = a;
          const uint16_t t = s_pos[lo];
          s_pos[lo] = s_pos[hi];
          s_pos[hi] = t;
        }
      }
      __syncthreads();
    }
  }
  for (uint32_t i = tid; i < out_per_tile; i += kReduceBlock) {
    const uint64_t o = static_cast<uint64_t>(blockIdx.x) * kReduceKeep + i;
    if (i < want) {
      const uint32_t src = base + s_pos[i];
      out_scores[o] = in_scores[src];
      out_ids[o] = in_ids ? in_ids[src] : src;
    } else {
      out_scores[o] = -INFINITY;
      out_ids[o] = kInvalidId;
    }
  }
}

}  // namespace fg
