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

__device__ __forceinline__ void saturating_increment(uint32_t* p) {
  uint32_t old = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while (old != 0xffffffffu) {
    const uint32_t seen = atomicCAS(p, old, old + 1u);
    if (seen == old) break;
    old = seen;
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
// device and turned into count tables (src/output.c:601-617) in one launch:
// each workgroup owns kWireRegion counts of one row, validates the row's
// whole payload (a few KB, shared through the cache by the row's
// workgroups), counts the ids that fall in its region in LDS, and writes the
// region once (cleared and counted in one store per entry: no clearing pass
// and no global atomics).  The first workgroup of a row writes its status.  A
// row that fails validation keeps its counts; its status says why
// (FG_ERR_ARGUMENT: shorter than the header; FG_ERR_FORMAT: the decoder's
// other checks).  Payload bytes are big-endian and need not be aligned.
constexpr int kWireBlock = 256;
constexpr uint32_t kWireRegion = 8192u;  // counts per workgroup (32 KB of LDS)
constexpr uint32_t kWireHeader = 8u;
constexpr uint32_t kWireMaxCount = 262144u;
constexpr uint32_t kWireMaxSlots = 2u;

__device__ __forceinline__ uint32_t load_be32(const uint8_t* p) {
  return (static_cast<uint32_t>(p[0]) << 24) | (static_cast<uint32_t>(p[1]) << 16) |
         (static_cast<uint32_t>(p[2]) << 8) | static_cast<uint32_t>(p[3]);
}

// Id i of a payload (big-endian, at byte 8 + 4i): one dword load when the
// payload is 4-byte aligned, bytes otherwise.
__device__ __forceinline__ uint32_t wire_id(const uint8_t* p, bool aligned, uint32_t i) {
  if (aligned) return __builtin_bswap32(reinterpret_cast<const uint32_t*>(p + kWireHeader)[i]);
  return load_be32(p + kWireHeader + 4u * i);
}

// Writes counts [begin, end) of a row from the workgroup's LDS region:
// 16-byte non-temporal stores over the region's whole quads when they are
// aligned (the table is not read back by this launch; measured 8.80 against
// 9.73 us for 64 rows of 151,936), then the tail.
__device__ __forceinline__ void store_region(uint32_t* crow, uint32_t begin, uint32_t end,
                                             const uint32_t* s_cnt) {
  const uint32_t tid = threadIdx.x;
  if ((reinterpret_cast<uintptr_t>(crow + begin) & 15u) == 0u) {
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    const uint32_t quads = (end - begin) / 4u;
    for (uint32_t q = tid; q < quads; q += kWireBlock) {
      const u4 c = reinterpret_cast<const u4*>(s_cnt)[q];
      const v4u w = {c.x, c.y, c.z, c.w};
      __builtin_nontemporal_store(w, reinterpret_cast<v4u*>(crow + begin) + q);
    }
    for (uint32_t i = begin + 4u * quads + tid; i < end; i += kWireBlock) crow[i] = s_cnt[i - begin];
  } else {
    for (uint32_t i = begin + tid; i < end; i += kWireBlock) crow[i] = s_cnt[i - begin];
  }
}

// Grid chunks * rows (chunks = ceil(vocab / kWireRegion)): workgroup b owns
// region b % chunks of row b / chunks.  The ids are read once, right away
// (their number follows from the payload's size): each is checked against
// the vocabulary and, when it falls in the region, counted in LDS; the
// header is checked alongside.  The row's region is written only when the
// whole payload is valid.
__global__ __launch_bounds__(kWireBlock) void history_wire_build_kernel(
    uint32_t* counts, uint64_t stride, uint32_t vocab, const uint8_t* payloads,
    const uint64_t* offsets, int32_t* row_status, uint8_t* row_slot, uint32_t chunks) {
  __shared__ __align__(16) uint32_t s_cnt[kWireRegion];
  __shared__ int32_t s_status;
  const uint32_t tid = threadIdx.x;
  const uint32_t r = blockIdx.x / chunks;
  const uint32_t chunk = blockIdx.x - r * chunks;
  const uint8_t* p = payloads + offsets[r];
  const uint64_t bytes = offsets[r + 1] - offsets[r];
  const bool aligned = (reinterpret_cast<uintptr_t>(p) & 3u) == 0u;
  // As many ids as the size allows (the header must agree, checked below).
  const uint32_t n = bytes >= kWireHeader + 4ull * kWireMaxCount
                         ? kWireMaxCount
                         : (bytes >= kWireHeader ? static_cast<uint32_t>((bytes - kWireHeader) / 4u) : 0u);
  const uint32_t begin = chunk * kWireRegion;
  const uint32_t end = vocab - begin < kWireRegion ? vocab : begin + kWireRegion;
  for (uint32_t i = tid; i < kWireRegion / 4u; i += kWireBlock)
    reinterpret_cast<u4*>(s_cnt)[i] = u4{0u, 0u, 0u, 0u};
  if (tid == 0) s_status = 0;
  __syncthreads();
  int32_t bad = 0;
  for (uint32_t i = tid; i < n; i += kWireBlock) {
    const uint32_t id = wire_id(p, aligned, i);
    bad |= id >= vocab ? 4 : 0;
    if (id >= begin && id < end) atomicAdd(&s_cnt[id - begin], 1u);
  }
  uint8_t slot = 0u;
  if (tid == 0) {
    if (bytes < kWireHeader) {
      bad = 2;  // FG_ERR_ARGUMENT (a short payload has no ids)
    } else {
      const uint32_t count = load_be32(p);
      const uint32_t reserved = (static_cast<uint32_t>(p[5]) << 16) |
                                (static_cast<uint32_t>(p[6]) << 8) | p[7];
      slot = p[4];
      if (reserved || slot >= kWireMaxSlots || count > kWireMaxCount ||
          kWireHeader + 4ull * count != bytes)
        bad |= 4;  // FG_ERR_FORMAT
    }
  }
  if (bad) atomicOr(&s_status, bad);
  __syncthreads();
  // FG_ERR_ARGUMENT over FG_ERR_FORMAT, as the decoder checks the length
  // first.
  const int32_t st = (s_status & 2) ? 2 : s_status;
  if (chunk == 0 && tid == 0) {
    row_status[r] = st;
    if (row_slot && st != 2) row_slot[r] = st == 0 ? slot : 0u;
  }
  if (st != 0) return;
  store_region(counts + static_cast<uint64_t>(r) * stride, begin, end, s_cnt);
}

// src/output.c:601-617 (fg_output_history_reset) per row, from plain id
// lists, in one launch shaped like the wire builder: workgroup b owns region
// b % chunks (kWireRegion counts) of row b / chunks.  It reads the row's ids
// twice: first for the position of the first id outside the vocabulary (the
// reference stops there), then counting in LDS the ids before it that fall
// in its region.  The region is then written whole: cleared and counted in
// one store per entry, no clearing pass and no global atomics.  A row of
// more than kWireMaxCount ids is refused (FG_ERR_ARGUMENT, counts left as
// they were); a row with an id outside the vocabulary gets FG_ERR_FORMAT and
// the counts of the ids before it, as the reference leaves its table.  The
// first workgroup of a row writes the row's status.
__global__ __launch_bounds__(kWireBlock) void history_ids_build_kernel(
    uint32_t* counts, uint64_t stride, uint32_t vocab, const uint32_t* ids,
    const uint64_t* offsets, int32_t* row_status, uint32_t chunks) {
  __shared__ __align__(16) uint32_t s_cnt[kWireRegion];
  __shared__ uint32_t s_first_bad;
  const uint32_t tid = threadIdx.x;
  const uint32_t r = blockIdx.x / chunks;
  const uint32_t chunk = blockIdx.x - r * chunks;
  const uint64_t b = offsets[r], n64 = offsets[r + 1] - b;
  if (n64 > kWireMaxCount) {
    if (chunk == 0 && tid == 0) row_status[r] = 2;  // FG_ERR_ARGUMENT
    return;
  }
  const uint32_t n = static_cast<uint32_t>(n64);
  const uint32_t* row_ids = ids + b;
  const uint32_t begin = chunk * kWireRegion;
  const uint32_t end = vocab - begin < kWireRegion ? vocab : begin + kWireRegion;
  for (uint32_t i = tid; i < kWireRegion / 4u; i += kWireBlock)
    reinterpret_cast<u4*>(s_cnt)[i] = u4{0u, 0u, 0u, 0u};
  if (tid == 0) s_first_bad = n;
  __syncthreads();
  uint32_t first_bad = n;
  for (uint32_t i = tid; i < n; i += kWireBlock)
    if (row_ids[i] >= vocab && i < first_bad) first_bad = i;
  if (first_bad < n) atomicMin(&s_first_bad, first_bad);
  __syncthreads();
  const uint32_t stop = s_first_bad;
  for (uint32_t i = tid; i < stop; i += kWireBlock) {
    const uint32_t id = row_ids[i];
    if (id >= begin && id < end) atomicAdd(&s_cnt[id - begin], 1u);
  }
  if (chunk == 0 && tid == 0) row_status[r] = stop < n ? 4 : 0;  // FG_ERR_FORMAT / FG_OK
  __syncthreads();
  store_region(counts + static_cast<uint64_t>(r) * stride, begin, end, s_cnt);
}

// Top-512 reduction of shaders/fg_topk_reduce_v2.comp (src/vk.c:2235): per
// 4096-element tile, the tile's entries in the greedy order of its
// comparator (:9; padding id 0xffffffff last, non-finite first with lower id
// first, then larger value, equal values (0 == -0) by lower id), the first
// min(512, n) written, the rest of the 512 slots padded with (-inf,
// 0xffffffff).  Entries are ordered as 64-bit greedy composites (padding ids
// 1, the fill slots of a partial tile 0) carried with the score's bits, so
// every bit of a value (NaN payloads, -0) is written back; the id is the
// composite's low word.
//
// One 512-thread workgroup per tile; thread t holds positions t + 512 e.
// A tile of more than 1024 entries is bucketed:
//  1. The float keys (composite high words) at 64 sampled positions
//     (p % 64 == 37) are sorted by one wave; the region is every entry whose
//     float key is at or above the sample's 24th largest (about 37% of the
//     tile).
//  2. Region entries fall into 128 buckets by a monotone map of their
//     float key onto [region floor, tile maximum]; the
//     buckets are counted in LDS (spread over 128 addresses, so the atomics
//     rarely meet) and scanned from the top: the buckets down to the one
//     holding the 512th entry are kept and scattered into LDS in bucket
//     order.
//  3. Each wave sorts one 64-entry window of the entries above the boundary
//     bucket (a DPP/permlane bitonic network, no barriers), and a spare wave
//     sorts the boundary bucket; then a bucket that crosses a window edge
//     has its two sorted parts merged by one wave.  Buckets are ordered
//     intervals, so the array is then sorted.
// A bucket of more than 64 entries (heavily tied values) sends the tile to
// a workgroup-wide bitonic sort of the kept entries; a region with fewer
// than 512 entries (a sample unlike its tile) to an exact MSB-first radix
// select.  Tiles of at most 1024 entries keep them all and take the
// workgroup-wide sort.
constexpr int kReduceBlock = 512;
constexpr uint32_t kReduceTile = 4096u;
constexpr uint32_t kReduceKeep = 512u;
constexpr uint32_t kReduceSort = 1024u;      // most kept entries the sort takes
constexpr uint32_t kReduceBuckets = 128u;
constexpr uint32_t kReduceRegionRank = 23u;  // sample rank of the region floor
constexpr uint32_t kReduceSampleLane = 37u;  // lane whose entries form the sample
constexpr uint32_t kReduceNoBucket = 0xffu;

#ifdef FG_REDUCE_TRACE
// Phase timestamps of trace builds: [tile][32] (s_memrealtime, 100 MHz).
__device__ uint64_t g_reduce_trace[512 * 32];
#define FG_RDT(slot)                                                                    \
  do {                                                                                  \
    __builtin_amdgcn_s_waitcnt(0);                                                      \
    if (threadIdx.x == 0 && blockIdx.x < 512u)                                        \
      g_reduce_trace[blockIdx.x * 32u + (slot)] = __builtin_amdgcn_s_memrealtime();     \
  } while (0)
#define FG_RDTR(row, slot)                                                              \
  do {                                                                                  \
    __builtin_amdgcn_s_waitcnt(0);                                                      \
    if (threadIdx.x == 0 && (row) < 512u)                                               \
      g_reduce_trace[(row) * 32u + (slot)] = __builtin_amdgcn_s_memrealtime();          \
  } while (0)
#else
#define FG_RDT(slot) \
  do {               \
  } while (0)
#define FG_RDTR(row, slot) \
  do {                     \
  } while (0)
#endif

struct ReduceShared {
  uint64_t key[2][kReduceSort];  // kept entries in [0]; sort exchanges alternate
  uint32_t bits[2][kReduceSort];  // the entries' score bits
  uint32_t sample[kWave];        // sampled float keys, then sorted descending
  uint32_t wave_max[kReduceBlock / kWave];
  uint32_t hist[256];
  uint32_t start[kReduceBuckets];
  uint32_t straddle[kReduceBlock / kWave + 1u];
  uint32_t sel[4];
  uint32_t n_kept;      // radix fallback's kept entries
  uint32_t n_straddle;  // buckets across window edges
};

// Compare-exchange of (composite, score bits) with lane ^ J: the larger key stays
// where keep_min is false.  Composites of one tile are unique except for
// duplicate ids, whose entries are identical, so a strict compare suffices.
template <int J>
__device__ __forceinline__ void cx_lanes(uint64_t& k, uint32_t& p, bool keep_min) {
  const uint64_t ok = lane_xor64<J>(k);
  const uint32_t op = lane_xor<J>(p);
  const bool take = (ok > k) != keep_min;
  k = take ? ok : k;
  p = take ? op : p;
}

// The steps j, j/2, .., 1 (j <= 32) of the bitonic stage of block size kb for
// element idx (descending where idx & kb == 0).
__device__ __forceinline__ void cx_lane_steps(uint64_t& k, uint32_t& p, uint32_t idx, uint32_t kb,
                                              uint32_t j) {
  const bool asc = (idx & kb) != 0u;
  switch (j) {
    case 32u: cx_lanes<32>(k, p, asc != ((idx & 32u) != 0u)); [[fallthrough]];
    case 16u: cx_lanes<16>(k, p, asc != ((idx & 16u) != 0u)); [[fallthrough]];
    case 8u: cx_lanes<8>(k, p, asc != ((idx & 8u) != 0u)); [[fallthrough]];
    case 4u: cx_lanes<4>(k, p, asc != ((idx & 4u) != 0u)); [[fallthrough]];
    case 2u: cx_lanes<2>(k, p, asc != ((idx & 2u) != 0u)); [[fallthrough]];
    case 1u: cx_lanes<1>(k, p, asc != ((idx & 1u) != 0u)); break;
    default: break;
  }
}

// Sorts lanes [0, w) of one wave descending (w <= 64; lanes >= w must hold
// key 0): stages up to the first power of two >= w.
__device__ __forceinline__ void wave_sort_pairs(uint64_t& k, uint32_t& p, uint32_t w) {
  const uint32_t lane = lane_id();
  for (uint32_t kb = 2u; kb <= static_cast<uint32_t>(kWave); kb <<= 1) {
    cx_lane_steps(k, p, lane, kb, kb >> 1);
    if (kb >= w) break;
  }
}

// Appends this lane's entry where p holds, one LDS atomic per wave; returns
// its slot (meaningless where p is false).
__device__ __forceinline__ uint32_t wave_append(uint32_t* counter, bool p) {
  const uint64_t m = ballot(p);
  if (!m) return 0u;
  const uint32_t lead = static_cast<uint32_t>(__builtin_ctzll(m));
  uint32_t first = 0u;
  if (lane_id() == lead) first = atomicAdd(counter, static_cast<uint32_t>(__builtin_popcountll(m)));
  return readlane32(first, lead) + lanes_below(m);
}

// Exact fallback: the want-th largest of the tile's composites by an MSB-first
// radix select, then exactly `want` entries (those above it, and as many equal
// to it as needed) appended to the kept list.
__device__ __forceinline__ void reduce_radix_keep(ReduceShared& S, const uint64_t (&key)[8],
                                                  const uint32_t (&sbits)[8], uint32_t n,
                                                  uint32_t want) {
  constexpr uint32_t kPer = kReduceTile / kReduceBlock;
  const uint32_t tid = threadIdx.x;
  uint64_t prefix = 0ull;
  uint32_t rank = want;
  uint64_t cmp_mask = ~0ull;
  for (int d = 7; d >= 0; d--) {
    const uint32_t shift = 8u * static_cast<uint32_t>(d);
    const uint64_t hi_mask = d == 7 ? 0ull : ~0ull << (shift + 8u);
    if (tid < 256u) S.hist[tid] = 0u;
    __syncthreads();
#pragma unroll
    for (uint32_t e = 0; e < kPer; e++) {
      const uint32_t i = e * kReduceBlock + tid;
      if (i < n && (key[e] & hi_mask) == prefix) atomicAdd(&S.hist[(key[e] >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64u) {
      // Bins from the top: lane l owns bins 255 - 4l .. 252 - 4l.
      uint32_t c[4];
      uint32_t sum = 0u;
#pragma unroll
      for (int b = 0; b < 4; b++) {
        c[b] = S.hist[255u - 4u * tid - b];
        sum += c[b];
      }
      uint32_t before = sum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(before, o, 64);
        if (tid >= static_cast<uint32_t>(o)) before += t;
      }
      uint32_t acc = before - sum;
#pragma unroll
      for (int b = 0; b < 4; b++) {
        if (acc < rank && acc + c[b] >= rank) {
          S.sel[0] = 255u - 4u * tid - b;
          S.sel[1] = acc;
          S.sel[2] = c[b];
        }
        acc += c[b];
      }
    }
    __syncthreads();
    prefix |= static_cast<uint64_t>(S.sel[0]) << shift;
    rank -= S.sel[1];
    const bool settled = d == 4 && S.sel[2] == rank;  // every key of this float key is kept
    __syncthreads();
    if (settled) {
      cmp_mask = ~0ull << 32;
      break;
    }
  }
  if (tid == 0) {
    S.sel[3] = 0u;
    S.n_kept = 0u;
  }
  __syncthreads();
#pragma unroll
  for (uint32_t e = 0; e < kPer; e++) {
    const uint32_t i = e * kReduceBlock + tid;
    const uint64_t km = key[e] & cmp_mask;
    bool keep = i < n && km > prefix;
    if (i < n && km == prefix) keep = atomicAdd(&S.sel[3], 1u) < rank;
    const uint32_t at = wave_append(&S.n_kept, keep);
    if (keep) {
      S.key[0][at] = key[e];
      S.bits[0][at] = sbits[e];
    }
  }
}

// Bitonic sort of the n_sort (<= 1024) pairs in S.key[0] / S.bits[0], padded
// with 0 to a power of two: element idx = tid (+ 512 for the second, when
// more than 512), descending at the end; returns rank tid's pair.  Strides
// below 64 between lanes, 64 to 256 through LDS, 512 within a thread.
__device__ __forceinline__ void reduce_block_sort(ReduceShared& S, uint32_t n_sort, uint64_t& k0,
                                                  uint32_t& p0) {
  const uint32_t tid = threadIdx.x;
  uint32_t P = 1u;
  while (P < n_sort) P <<= 1;
  k0 = tid < n_sort ? S.key[0][tid] : 0ull;
  p0 = tid < n_sort ? S.bits[0][tid] : 0u;
  const uint32_t i1 = tid + kReduceBlock;
  uint64_t k1 = i1 < n_sort ? S.key[0][i1] : 0ull;
  uint32_t p1 = i1 < n_sort ? S.bits[0][i1] : 0u;
  uint32_t buf = 0u;
  for (uint32_t kb = 2u; kb <= P; kb <<= 1) {
    uint32_t j = kb >> 1;
    // The second element lives until the last stage's 512 step has given the
    // first one the larger of each pair.
    const bool two = P > kReduceBlock && kb < P;
    if (j == kReduceBlock) {
      if (k1 > k0) {
        const uint64_t tk = k0;
        k0 = k1;
        k1 = tk;
        const uint32_t tp = p0;
        p0 = p1;
        p1 = tp;
      }
      j >>= 1;
    }
    for (; j >= static_cast<uint32_t>(kWave); j >>= 1) {
      S.key[buf][tid] = k0;
      S.bits[buf][tid] = p0;
      if (two) {
        S.key[buf][i1] = k1;
        S.bits[buf][i1] = p1;
      }
      __syncthreads();
      {
        const uint64_t ok = S.key[buf][tid ^ j];
        const uint32_t op = S.bits[buf][tid ^ j];
        const bool take = (ok > k0) != (((tid & kb) != 0u) != ((tid & j) != 0u));
        k0 = take ? ok : k0;
        p0 = take ? op : p0;
      }
      if (two) {
        const uint64_t ok = S.key[buf][i1 ^ j];
        const uint32_t op = S.bits[buf][i1 ^ j];
        const bool take = (ok > k1) != (((i1 & kb) != 0u) != ((i1 & j) != 0u));
        k1 = take ? ok : k1;
        p1 = take ? op : p1;
      }
      buf ^= 1u;
    }
    cx_lane_steps(k0, p0, tid, kb, j);
    if (two) cx_lane_steps(k1, p1, i1, kb, j);
  }
}

__global__ __launch_bounds__(kReduceBlock) void topk_reduce_kernel(
    float* out_scores, uint32_t* out_ids, const float* in_scores, const uint32_t* in_ids,
    uint32_t count, uint32_t out_per_tile) {
  constexpr uint32_t kPer = kReduceTile / kReduceBlock;  // entries per thread
  __shared__ ReduceShared S;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & (kWave - 1u);
  const uint32_t wave = tid / kWave;
  const uint32_t base = blockIdx.x * kReduceTile;
  const uint32_t n = min(kReduceTile, count - base);
  const uint32_t want = min(kReduceKeep, n);
  FG_RDT(0);
  uint64_t key[kPer];
  uint32_t sbits[kPer], ids[kPer];
  // Every load is issued before the first is used.
  if (n == kReduceTile) {
#pragma unroll
    for (uint32_t e = 0; e < kPer; e++) sbits[e] = __float_as_uint(in_scores[base + e * kReduceBlock + tid]);
    if (in_ids) {
#pragma unroll
      for (uint32_t e = 0; e < kPer; e++) ids[e] = in_ids[base + e * kReduceBlock + tid];
    }
  } else {
#pragma unroll
    for (uint32_t e = 0; e < kPer; e++) {
      const uint32_t i = min(e * kReduceBlock + tid, n - 1u);
      sbits[e] = __float_as_uint(in_scores[base + i]);
      if (in_ids) ids[e] = in_ids[base + i];
    }
  }
  uint32_t hmax = 0u;  // largest float key (composite high word)
#pragma unroll
  for (uint32_t e = 0; e < kPer; e++) {
    const uint32_t i = e * kReduceBlock + tid;
    const uint32_t id = in_ids ? ids[e] : base + i;
    // Padding ids rank last among the entries (1); a fill slot of a partial
    // tile is 0 and never selected.
    const uint64_t k = i >= n ? 0ull : (id == kInvalidId ? 1ull : greedy_comp(__uint_as_float(sbits[e]), id));
    key[e] = k;
    hmax = max(hmax, static_cast<uint32_t>(k >> 32));
  }
  FG_RDT(1);
  uint64_t k0;
  uint32_t p0;
  if (n <= kReduceSort) {
    // Every entry is kept; positions below 1024 are e = 0, 1.
#pragma unroll
    for (uint32_t e = 0; e < 2u; e++) {
      const uint32_t i = e * kReduceBlock + tid;
      if (i < n) {
        S.key[0][i] = key[e];
        S.bits[0][i] = sbits[e];
      }
    }
    __syncthreads();
    reduce_block_sort(S, n, k0, p0);
  } else {
    hmax = max(hmax, lane_xor<1>(hmax));
    hmax = max(hmax, lane_xor<2>(hmax));
    hmax = max(hmax, lane_xor<4>(hmax));
    hmax = max(hmax, lane_xor<8>(hmax));
    hmax = max(hmax, lane_xor<16>(hmax));
    hmax = max(hmax, lane_xor<32>(hmax));
    if (lane == 0u) S.wave_max[wave] = hmax;
    if (lane == kReduceSampleLane) {
#pragma unroll
      for (uint32_t e = 0; e < kPer; e++) S.sample[wave * kPer + e] = static_cast<uint32_t>(key[e] >> 32);
    }
    if (tid < kReduceBuckets) S.hist[tid] = 0u;
    __syncthreads();
    if (wave == 0u) S.sample[lane] = wave_sort_desc_u32(S.sample[lane]);
    __syncthreads();
    FG_RDT(2);
    // The bucket map: region entries (float key >= the floor) linearly from
    // the floor to the tile's largest float key, onto [0, 128).
    const uint32_t floor_hi = S.sample[kReduceRegionRank];
    uint32_t top = S.wave_max[0];
#pragma unroll
    for (uint32_t w = 1; w < kReduceBlock / kWave; w++) top = max(top, S.wave_max[w]);
    const float scale = static_cast<float>(kReduceBuckets) / (static_cast<float>(top - floor_hi) + 1.0f);
    // The count's returned value is the entry's slot within its bucket.
    uint8_t bucket[kPer];
    uint32_t slot[kPer];
#pragma unroll
    for (uint32_t e = 0; e < kPer; e++) {
      const uint32_t i = e * kReduceBlock + tid;
      uint32_t c = kReduceNoBucket;
      slot[e] = 0u;
      if (i < n && static_cast<uint32_t>(key[e] >> 32) >= floor_hi) {
        const float f = static_cast<float>(static_cast<uint32_t>(key[e] >> 32) - floor_hi) * scale;
        c = min(static_cast<uint32_t>(f), kReduceBuckets - 1u);
        slot[e] = atomicAdd(&S.hist[c], 1u);
      }
      bucket[e] = static_cast<uint8_t>(c);
    }
    __syncthreads();
    FG_RDT(3);
    if (wave == 0u) {
      // Lane l holds buckets 127 - 2l and 126 - 2l, the highest first.
      const uint32_t ca = 127u - 2u * lane, cb = ca - 1u;
      const uint32_t ha = S.hist[ca], hb = S.hist[cb];
      const uint32_t cum = wave_prefix_sum_u32(ha + hb);
      const uint32_t start_a = cum - ha - hb, start_b = cum - hb;
      // The boundary bucket: the first whose inclusive count reaches want.
      const bool hit_a = start_a < want && start_a + ha >= want;
      const bool hit_b = start_b < want && start_b + hb >= want;
      const uint64_t hits = ballot(hit_a || hit_b);
      uint32_t mode = 2u, bnd = 0u, above = 0u, in_bnd = 0u;
      if (hits) {
        const uint32_t L = static_cast<uint32_t>(__builtin_ctzll(hits));
        const uint32_t la = readlane32(hit_a ? 1u : 0u, L);
        bnd = la ? 127u - 2u * L : 126u - 2u * L;
        above = la ? readlane32(start_a, L) : readlane32(start_b, L);
        in_bnd = la ? readlane32(ha, L) : readlane32(hb, L);
        // Buckets at or above the boundary must each fit one wave.
        const uint32_t big = max(ca >= bnd ? ha : 0u, cb >= bnd ? hb : 0u);
        const uint64_t over = ballot(big > static_cast<uint32_t>(kWave));
        mode = over ? (above + in_bnd <= kReduceSort ? 1u : 2u) : 0u;
      }
      S.start[ca] = start_a;
      S.start[cb] = start_b;
      // Buckets above the boundary that cross a 64-entry window edge: their
      // two sorted parts are merged after the windows are sorted.
      const bool st_a = ca > bnd && ha != 0u && (start_a / kWave) != ((start_a + ha - 1u) / kWave);
      const bool st_b = cb > bnd && hb != 0u && (start_b / kWave) != ((start_b + hb - 1u) / kWave);
      const uint64_t ma = ballot(st_a), mb = ballot(st_b);
      if (st_a) S.straddle[lanes_below(ma) + lanes_below(mb)] = ca;
      if (st_b) S.straddle[lanes_below(ma) + lanes_below(mb) + (st_a ? 1u : 0u)] = cb;
      if (lane == 0u) {
        S.sel[0] = mode;
        S.sel[1] = bnd;
        S.sel[2] = above;
        S.sel[3] = in_bnd;
        S.n_straddle = static_cast<uint32_t>(__builtin_popcountll(ma) + __builtin_popcountll(mb));
      }
    }
    __syncthreads();
    FG_RDT(4);
    const uint32_t mode = S.sel[0];
    const uint32_t bnd = S.sel[1];
    const uint32_t above = S.sel[2];  // entries in the buckets above the boundary
    const uint32_t in_bnd = S.sel[3];
    if (mode != 2u) {
      // Scatter in bucket order (every offset read before any write).
      uint32_t at[kPer];
#pragma unroll
      for (uint32_t e = 0; e < kPer; e++) at[e] = S.start[bucket[e] & (kReduceBuckets - 1u)] + slot[e];
#pragma unroll
      for (uint32_t e = 0; e < kPer; e++) {
        const uint32_t c = bucket[e];
        if (c != kReduceNoBucket && c >= bnd) {
          S.key[0][at[e]] = key[e];
          S.bits[0][at[e]] = sbits[e];
        }
      }
    } else {
      reduce_radix_keep(S, key, sbits, n, want);
    }
    __syncthreads();
    FG_RDT(5);
    if (mode == 0u) {
      // The entries above the boundary in windows of 64, one per wave; the
      // boundary bucket whole on the first free wave (the last wave after
      // the merges when all eight windows are taken).
      const uint32_t windows = (above + kWave - 1u) / kWave;
      if (wave < windows) {
        const uint32_t at = wave * kWave + lane;
        uint64_t k = at < above ? S.key[0][at] : 0ull;
        uint32_t p = at < above ? S.bits[0][at] : 0u;
        wave_sort_pairs(k, p, min(static_cast<uint32_t>(kWave), above - wave * kWave));
        if (at < above) {
          S.key[0][at] = k;
          S.bits[0][at] = p;
        }
      }
      const uint32_t bnd_wave = windows < kReduceBlock / kWave ? windows : kReduceBlock / kWave - 1u;
      const bool bnd_first = windows < kReduceBlock / kWave;
      if (bnd_first && wave == bnd_wave) {
        const uint32_t at = above + lane;
        uint64_t k = lane < in_bnd ? S.key[0][at] : 0ull;
        uint32_t p = lane < in_bnd ? S.bits[0][at] : 0u;
        wave_sort_pairs(k, p, in_bnd);
        if (lane < in_bnd) {
          S.key[0][at] = k;
          S.bits[0][at] = p;
        }
      }
      __syncthreads();
      FG_RDT(6);
      const uint32_t n_strad = S.n_straddle;
      if (wave < n_strad) {
        // Both parts of a bucket across a window edge are sorted: the first
        // descending in the low lanes, the second reversed in the high lanes
        // (zeros between) form a bitonic sequence, merged in six steps.
        const uint32_t c = S.straddle[wave];
        const uint32_t b0 = S.start[c], h = S.hist[c];
        const uint32_t edge = (b0 / kWave + 1u) * kWave;
        const uint32_t l1 = edge - b0, l2 = h - l1;
        const uint32_t src = lane < l1 ? b0 + lane : edge + (kWave - 1u - lane);
        const bool live = lane < l1 || kWave - 1u - lane < l2;
        uint64_t v = live ? S.key[0][src] : 0ull;
        uint32_t q = live ? S.bits[0][src] : 0u;
        cx_lane_steps(v, q, lane, kWave, kWave / 2u);
        if (lane < h) {
          S.key[0][b0 + lane] = v;
          S.bits[0][b0 + lane] = q;
        }
      } else if (!bnd_first && wave == bnd_wave) {
        const uint32_t at = above + lane;
        uint64_t k = lane < in_bnd ? S.key[0][at] : 0ull;
        uint32_t p = lane < in_bnd ? S.bits[0][at] : 0u;
        wave_sort_pairs(k, p, in_bnd);
        if (lane < in_bnd) {
          S.key[0][at] = k;
          S.bits[0][at] = p;
        }
      }
      __syncthreads();
      k0 = S.key[0][tid];
      p0 = S.bits[0][tid];
    } else {
      reduce_block_sort(S, mode == 1u ? above + in_bnd : want, k0, p0);
    }
  }
  FG_RDT(7);

  if (tid < out_per_tile) {
    const uint64_t o = static_cast<uint64_t>(blockIdx.x) * kReduceKeep + tid;
    if (tid < want) {
      out_scores[o] = __uint_as_float(p0);
      out_ids[o] = k0 == 1ull ? kInvalidId : ~static_cast<uint32_t>(k0);
    } else {
      out_scores[o] = -INFINITY;
      out_ids[o] = kInvalidId;
    }
  }
}

// ---- the whole top-512 scan in one launch --------------------------------------
// One workgroup per 4096-entry tile, all resident at once.  Composites are
// the 64-bit keys of fg_hip_topk_reduce's comparator (larger = earlier).
//  1. Each tile finds its K-th largest composite v_t by radix steps over
//     its composites in LDS (12 bits a step from the top, until the boundary
//     bucket holds at most 64 entries, which one wave then ranks), with
//     K = min(512, s + ceil(3 sqrt(s)) + 8) for the even share s =
//     ceil(512 / tiles) (every entry of a smaller tile, and of a single
//     tile), and publishes its entries at or above v_t and v_t itself; once
//     they have landed it stores its slot: this call's tag with their number.
//  2. Every workgroup waits for every slot to carry the tag, then gathers
//     the published entries at or above V = max v_t into LDS, in the same
//     order in every workgroup.  If there are at least 512, they hold the
//     global top 512: an entry above the 512th is above V, so its tile
//     published it.  Every workgroup then ranks its share of them against
//     all of them (ties by position) and writes those of rank < 512 to
//     their places.
// Otherwise (the top entries crowded into few tiles: sorted or skewed
// scores) every workgroup, deciding alike from the same data, takes a second
// route: a radix select over the whole input with a global digit histogram
// per round and a grid barrier after each, stopped once the entries at or
// above the boundary bucket fit in LDS (or the key is complete: then the
// boundary is one composite, repeated only by duplicate ids, and just the
// copies still needed are taken), and a global list of those entries,
// ranked the same way.
// The output is the comparator order of fg_hip_topk_reduce, so it is what
// iterating that kernel down to one tile leaves.
constexpr uint32_t kReduceAllDigit = 12u;
constexpr uint32_t kReduceAllBuckets = 1u << kReduceAllDigit;
constexpr uint32_t kReduceAllRounds = 6u;       // 12 x 5 + 4 bits
constexpr uint32_t kReduceAllList = 6144u;      // entries ranked in LDS
constexpr uint32_t kReduceAllRegion = 1024u;    // entries one tile's region holds
constexpr uint32_t kReduceAllSlack = 8u;        // K beyond a tile's share and its spread
constexpr uint32_t kReduceAllMaxTiles = 1024u;  // tiles the gather's offsets hold
struct ReduceAllWork {
  uint32_t count;   // arrivals at the second route's grid barrier (back to 0 every use)
  uint32_t gen;     // that barrier's uses so far (wraps)
  uint32_t listed;  // second-route list entries
  uint32_t ties;    // copies of an exact boundary composite taken
  uint32_t call;    // calls so far (wraps): the slots' tag is call + 1
};
constexpr uint32_t kReduceAllHeader = 64u;
constexpr uint64_t kReduceAllHistOffset = kReduceAllHeader;
constexpr uint64_t kReduceAllListOffset =
    kReduceAllHistOffset + uint64_t{kReduceAllRounds} * kReduceAllBuckets * sizeof(uint32_t);
constexpr uint64_t kReduceAllSlotOffset =
    kReduceAllListOffset + uint64_t{kReduceAllList} * (sizeof(uint64_t) + sizeof(uint32_t));
static_assert(sizeof(ReduceAllWork) <= kReduceAllHeader, "header");
static_assert(kReduceAllSlotOffset % 8u == 0u, "slot alignment");
// Bytes of the workspace for `tiles` tiles: the fixed part (with a bound
// (8 B) and a slot (8 B: tag << 32 | count) for each of kReduceAllMaxTiles
// tiles, at the same addresses for every tile count, so a slot word left by
// an earlier call always carries an older tag), then per tile a region of
// composites and score bits.
constexpr uint64_t kReduceAllRegionOffset =
    kReduceAllSlotOffset + uint64_t{kReduceAllMaxTiles} * 2u * sizeof(uint64_t);
__host__ __device__ constexpr uint64_t reduce_all_bytes(uint64_t tiles) {
  return kReduceAllRegionOffset + tiles * kReduceAllRegion * (sizeof(uint64_t) + sizeof(uint32_t));
}

// Sense-reversing grid barrier: the last workgroup in (its arrival number
// modulo `groups` is groups - 1) takes `groups` back off the count and
// advances the generation; the others wait for the generation to move past
// `gen`, which each workgroup read before its first arrival and counts along.
// A fast workgroup's next arrival may land before the last one's subtraction:
// arrival numbers are taken modulo `groups`, so it still counts right.
__device__ __forceinline__ void grid_sync(ReduceAllWork* w, uint32_t groups, uint32_t& gen) {
  wait_memory();  // this workgroup's published data first (see wait_memory)
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t o = atomicAdd(&w->count, 1u);
    if (o % groups == groups - 1u) {
      atomicSub(&w->count, groups);
      __hip_atomic_store(&w->gen, gen + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      while (__hip_atomic_load(&w->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gen)
        __builtin_amdgcn_s_sleep(1);
    }
  }
  gen++;
  __syncthreads();
}

// Workgroup barrier for LDS only: global loads already issued stay in flight
// (__syncthreads also waits for them).
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt left alone
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ uint32_t load_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t load_agent64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The bucket, counting 4096 buckets from the top (count(b) for bucket b),
// where the running count first reaches `need` (>= 1, at most the total):
// s_sel = {bucket, count above it, its count}.  All kReduceBlock threads.
template <class Count>
__device__ __forceinline__ void top_bucket(Count count, uint32_t need, uint32_t* s_wave,
                                           uint32_t* s_sel) {
  constexpr uint32_t kScan = kReduceAllBuckets / kReduceBlock;
  const uint32_t tid = threadIdx.x, lane = tid & (kWave - 1u), wave = tid / kWave;
  uint32_t c[kScan], sum = 0u;
#pragma unroll
  for (uint32_t j = 0; j < kScan; j++) {  // thread t: buckets 4095 - 8t down to 4088 - 8t
    c[j] = count(kReduceAllBuckets - 1u - (tid * kScan + j));
    sum += c[j];
  }
  const uint32_t incl = wave_prefix_sum_u32(sum);
  if (lane == kWave - 1u) s_wave[wave] = incl;
  __syncthreads();
  uint32_t start = incl - sum;
#pragma unroll
  for (uint32_t w = 0; w < kReduceBlock / kWave; w++) start += w < wave ? s_wave[w] : 0u;
#pragma unroll
  for (uint32_t j = 0; j < kScan; j++) {
    if (start < need && start + c[j] >= need) {
      s_sel[0] = kReduceAllBuckets - 1u - (tid * kScan + j);
      s_sel[1] = start;
      s_sel[2] = c[j];
    }
    start += c[j];
  }
  __syncthreads();
}

// LDS histogram of the next digit of the composites under `prefix`.
template <uint32_t kPer>
__device__ __forceinline__ void digit_hist(uint32_t* lh, const uint64_t (&key)[kPer],
                                           uint64_t prefix, uint32_t fixed, uint32_t width) {
  const uint32_t shift = 64u - fixed - width;
  const uint64_t hi_mask = fixed ? ~0ull << (64u - fixed) : 0ull;
#pragma unroll
  for (uint32_t j = 0; j < kReduceAllBuckets / kReduceBlock; j++) lh[j * kReduceBlock + threadIdx.x] = 0u;
  __syncthreads();
#pragma unroll
  for (uint32_t e = 0; e < kPer; e++)
    if (key[e] != 0ull && (key[e] & hi_mask) == prefix)
      atomicAdd(&lh[static_cast<uint32_t>(key[e] >> shift) & ((1u << width) - 1u)], 1u);
  __syncthreads();
}

// Workgroups go to the XCDs in turn (block b to XCD b % 8), and XCDs 0 and 1
// start a launch's workgroups about 2 us before the others.  With `packed`
// the grid is ceil(tiles / 2) * 8 workgroups and only blocks b % 8 < 2 take
// tiles (b / 8 * 2 + b % 8); the rest return at once.  Placement only: every
// exchange between tiles is coherent across the whole device.
__global__ __launch_bounds__(kReduceBlock) void topk_reduce_all_kernel(
    float* out_scores, uint32_t* out_ids, const float* in_scores, const uint32_t* in_ids,
    uint32_t count, uint32_t out_n, uint8_t* work_bytes, uint32_t tiles, uint32_t packed) {
  const uint32_t tile = packed ? (blockIdx.x >> 3) * 2u + (blockIdx.x & 7u) : blockIdx.x;
  if ((packed && (blockIdx.x & 7u) >= 2u) || tile >= tiles) return;
  constexpr uint32_t kPer = kReduceTile / kReduceBlock;  // entries per thread
  constexpr uint32_t kWaves = kReduceBlock / kWave;
  constexpr uint32_t kSweep = 4u;   // entries a wave ranks in one pass over the list
  constexpr uint32_t kUnroll = 4u;  // list entries a lane reads at once in that pass
  __shared__ uint64_t s_key[kReduceAllList];  // digit histogram, then the ranked entries
  __shared__ uint32_t s_bits[kReduceAllList];  // counts, then the tile map, then score bits
  __shared__ uint32_t s_off[kReduceAllMaxTiles + 1u];
  __shared__ uint32_t s_wave[kWaves];
  __shared__ uint32_t s_sel[3];
  __shared__ uint32_t s_n;
  __shared__ uint32_t s_tag;
  __shared__ uint64_t s_max;
  uint32_t* const lh = reinterpret_cast<uint32_t*>(s_key);
  static_assert(kReduceAllBuckets * sizeof(uint32_t) <= sizeof(s_key), "histogram in LDS");
  static_assert(kReduceAllList % (kUnroll * kWave) == 0u, "padded list");
  static_assert(kReduceAllMaxTiles <= kReduceAllList, "counts in s_bits");
  ReduceAllWork* const work = reinterpret_cast<ReduceAllWork*>(work_bytes);
  uint32_t* const hist = reinterpret_cast<uint32_t*>(work_bytes + kReduceAllHistOffset);
  uint64_t* const list_comp = reinterpret_cast<uint64_t*>(work_bytes + kReduceAllListOffset);
  uint32_t* const list_bits = reinterpret_cast<uint32_t*>(list_comp + kReduceAllList);
  uint64_t* const slot_bound = reinterpret_cast<uint64_t*>(work_bytes + kReduceAllSlotOffset);
  uint64_t* const slot_tag = slot_bound + kReduceAllMaxTiles;
  uint64_t* const region_comp = reinterpret_cast<uint64_t*>(work_bytes + kReduceAllRegionOffset);
  uint32_t* const region_bits = reinterpret_cast<uint32_t*>(region_comp + uint64_t{tiles} * kReduceAllRegion);
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & (kWave - 1u);
  const uint32_t wave = tid / kWave;
  const uint32_t base = tile * kReduceTile;
  const uint32_t n = min(kReduceTile, count - base);
  uint64_t key[kPer];  // 0 past the tile's entries; 1 for padding ids
  uint32_t sbits[kPer];
  FG_RDTR(tile, 0);
  // The call counter and the second route's barrier generation, read before
  // this workgroup publishes anything.
  uint32_t gen = 0u;
  if (tid == 0u) {
    gen = load_agent(&work->gen);
    s_tag = load_agent(&work->call) + 1u;
  }
  {
    uint32_t ids[kPer];
#pragma unroll
    for (uint32_t e = 0; e < kPer; e++) {
      const uint32_t i = min(e * kReduceBlock + tid, n - 1u);
      sbits[e] = __float_as_uint(in_scores[base + i]);
      ids[e] = in_ids ? in_ids[base + i] : base + i;
    }
#pragma unroll
    for (uint32_t e = 0; e < kPer; e++) {
      const uint32_t i = e * kReduceBlock + tid;
      key[e] = i >= n ? 0ull
                      : (ids[e] == kInvalidId ? 1ull : greedy_comp(__uint_as_float(sbits[e]), ids[e]));
    }
  }
  FG_RDTR(tile, 1);

  // ---- 1: this tile's top K (at least) published ----
  {
    // K: the tile's even share of the 512, three binomial standard
    // deviations and a margin; every entry of a single tile.
    const uint32_t share = (out_n + tiles - 1u) / tiles;
    const uint32_t spread = static_cast<uint32_t>(ceilf(3.0f * sqrtf(static_cast<float>(share))));
    const uint32_t k = min(tiles == 1u ? out_n : min(share + spread + kReduceAllSlack, kReduceKeep), n);
    uint64_t prefix = 0ull;  // ends as v_t: exactly the k-th largest composite
    uint32_t fixed = 0u, above = 0u;
    for (;;) {
      const uint32_t width = min(kReduceAllDigit, 64u - fixed);
      digit_hist(lh, key, prefix, fixed, width);
      if (fixed == 0u) FG_RDTR(tile, 10);
      top_bucket([&](uint32_t b) { return lh[b]; }, k - above, s_wave, s_sel);
      if (fixed == 0u) FG_RDTR(tile, 11);
      const uint64_t d = s_sel[0];
      const uint32_t before = s_sel[1], in_bucket = s_sel[2];
      __syncthreads();  // s_sel, s_wave and the histogram are written again
      fixed += width;
      prefix |= d << (64u - fixed);
      above += before;
      if (fixed == 64u) break;
      if (in_bucket <= kWave) {
        // The (k - above)-th largest of the boundary bucket's entries.
        uint64_t* const cand = s_key;
        const uint64_t mask = ~0ull << (64u - fixed);
        if (tid == 0u) s_n = 0u;
        __syncthreads();
#pragma unroll
        for (uint32_t e = 0; e < kPer; e++) {
          const bool in = key[e] != 0ull && (key[e] & mask) == prefix;
          const uint64_t m = ballot(in);
          if (m == 0ull) continue;
          const uint32_t leader = static_cast<uint32_t>(__builtin_ctzll(m));
          uint32_t first = 0u;
          if (lane == leader) first = atomicAdd(&s_n, static_cast<uint32_t>(__popcll(m)));
          first = readlane32(first, leader);
          if (in) cand[first + lanes_below(m)] = key[e];
        }
        __syncthreads();
        FG_RDTR(tile, 12);
        if (wave == 0u) {
          // Lane l's candidate is the r-th largest (from 0) when fewer than
          // r + 1 candidates exceed it and more than r reach it.
          const uint64_t c = lane < in_bucket ? cand[lane] : 0ull;
          const uint32_t r = k - above - 1u;
          uint32_t gt = 0u, ge = 0u;
#pragma unroll 8
          for (uint32_t i = 0; i < in_bucket; i++) {
            const uint64_t x = cand[i];
            gt += x > c ? 1u : 0u;
            ge += x >= c ? 1u : 0u;
          }
          if (lane < in_bucket && gt <= r && r < ge) s_max = c;
        }
        __syncthreads();
        prefix = s_max;
        break;
      }
    }
    FG_RDTR(tile, 7);
    if (tid == 0u) s_n = 0u;
    __syncthreads();
    uint64_t* const rc = region_comp + uint64_t{tile} * kReduceAllRegion;
    uint32_t* const rb = region_bits + uint64_t{tile} * kReduceAllRegion;
#pragma unroll
    for (uint32_t e = 0; e < kPer; e++) {
      const bool keep = key[e] != 0ull && key[e] >= prefix;
      const uint64_t m = ballot(keep);
      if (m == 0ull) continue;
      const uint32_t leader = static_cast<uint32_t>(__builtin_ctzll(m));
      uint32_t first = 0u;
      if (lane == leader) first = atomicAdd(&s_n, static_cast<uint32_t>(__popcll(m)));
      first = readlane32(first, leader);
      const uint32_t at = first + lanes_below(m);
      if (keep && at < kReduceAllRegion) {
        __hip_atomic_store(&rc[at], key[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&rb[at], sbits[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (tid == 0u) __hip_atomic_store(&slot_bound[tile], prefix, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#ifdef FG_REDUCE_TRACE
    if (threadIdx.x == 0 && tile < 512u) g_reduce_trace[tile * 32u + 13u] = __builtin_amdgcn_s_memrealtime();
#endif
    wait_memory();  // every store of this workgroup acknowledged ...
    __syncthreads();
    if (tid == 0u)  // ... before the slot says they are there
      __hip_atomic_store(&slot_tag[tile], (uint64_t{s_tag} << 32) | s_n, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  FG_RDTR(tile, 2);

  // ---- 2: every slot tagged; the published entries at or above V gathered ----
  if (wave == 0u) {
    const uint32_t tag = s_tag;
    for (uint32_t t0 = 0; t0 < tiles; t0 += kWave) {
      const uint32_t t = t0 + lane;
      bool ok = t >= tiles;
      uint64_t v = 0ull;
      for (;;) {
        if (!ok) {
          v = load_agent64(&slot_tag[t]);
          ok = static_cast<uint32_t>(v >> 32) == tag;
        }
        if (ballot(!ok) == 0ull) break;
        __builtin_amdgcn_s_sleep(1);
      }
      if (t < tiles) s_bits[t] = static_cast<uint32_t>(v);
    }
  }
  if (tid == 0u) s_max = 0ull;
  __syncthreads();
  FG_RDTR(tile, 3);
  if (tile == 0u && tid == 0u)  // every workgroup has read the call counter
    __hip_atomic_store(&work->call, s_tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint32_t M;
  bool complete;
  {
    // The bounds' loads stay in flight over the offsets' scan.
    uint64_t vb[kReduceAllMaxTiles / kReduceBlock];
#pragma unroll
    for (uint32_t u = 0; u < kReduceAllMaxTiles / kReduceBlock; u++) {
      const uint32_t t = u * kReduceBlock + tid;
      vb[u] = t < tiles ? load_agent64(&slot_bound[t]) : 0ull;
    }
    uint32_t over = 0u;
    for (uint32_t t0 = 0; t0 < tiles; t0 += kReduceBlock) {
      const uint32_t t = t0 + tid;
      const uint32_t c = t < tiles ? s_bits[t] : 0u;
      over |= c > kReduceAllRegion ? 1u : 0u;
      const uint32_t incl = wave_prefix_sum_u32(c);
      if (lane == kWave - 1u) s_wave[wave] = incl;
      lds_barrier();
      uint32_t start = (t0 ? s_off[t0] : 0u) + incl - c;
#pragma unroll
      for (uint32_t w = 0; w < kWaves; w++) start += w < wave ? s_wave[w] : 0u;
      lds_barrier();
      if (t < tiles) s_off[t + 1u] = start + c;
      if (t0 == 0u && tid == 0u) s_off[0] = 0u;
      lds_barrier();
    }
    M = s_off[tiles];
    const uint32_t wave_over = ballot(over != 0u) != 0ull ? 1u : 0u;
    if (lane == 0u) s_wave[wave] = wave_over;
    lds_barrier();
    over = M > kReduceAllList ? 1u : 0u;
#pragma unroll
    for (uint32_t w = 0; w < kWaves; w++) over |= s_wave[w];
    complete = false;
    FG_RDTR(tile, 8);
    if (!over) {
      lds_barrier();  // s_wave read by every wave
      // s_bits maps each published entry to its tile, then holds score bits.
      for (uint32_t t = wave; t < tiles; t += kWaves)
        for (uint32_t i = s_off[t] + lane; i < s_off[t + 1u]; i += kWave) s_bits[i] = t;
      lds_barrier();
      // Wave w loads entries [w P, w P + P), P = M / 8 rounded up to 64.
      constexpr uint32_t kLoads = kReduceAllList / kReduceBlock;
      const uint32_t P = ((M + kWaves - 1u) / kWaves + kWave - 1u) & ~(kWave - 1u);
      const uint32_t lo = min(wave * P, M), hi = min(lo + P, M);
      uint64_t x[kLoads];
      uint32_t xb[kLoads];
#pragma unroll
      for (uint32_t u = 0; u < kLoads; u++) {
        const uint32_t j = lo + u * kWave + lane;
        x[u] = 0ull;
        xb[u] = 0u;
        if (j < hi) {
          const uint32_t t = s_bits[j];
          const uint64_t at = uint64_t{t} * kReduceAllRegion + (j - s_off[t]);
          x[u] = load_agent64(&region_comp[at]);
          xb[u] = load_agent(&region_bits[at]);
        }
      }
      uint64_t vmax = 0ull;
#pragma unroll
      for (uint32_t u = 0; u < kReduceAllMaxTiles / kReduceBlock; u++) vmax = vb[u] > vmax ? vb[u] : vmax;
      vmax = wave_max_u64(vmax);
      if (lane == 0u) atomicMax(reinterpret_cast<unsigned long long*>(&s_max), vmax);
      __syncthreads();  // V known; every tile map entry read
      const uint64_t V = s_max;
      uint32_t kept = 0u;
#pragma unroll
      for (uint32_t u = 0; u < kLoads; u++) kept += __popcll(ballot(x[u] != 0ull && x[u] >= V));
      if (lane == 0u) s_wave[wave] = kept;
      FG_RDTR(tile, 9);
      lds_barrier();
      uint32_t pos = 0u, total = 0u;
#pragma unroll
      for (uint32_t w = 0; w < kWaves; w++) {
        pos += w < wave ? s_wave[w] : 0u;
        total += s_wave[w];
      }
#pragma unroll
      for (uint32_t u = 0; u < kLoads; u++) {
        const bool keep = x[u] != 0ull && x[u] >= V;
        const uint64_t m = ballot(keep);
        if (keep) {
          s_key[pos + lanes_below(m)] = x[u];
          s_bits[pos + lanes_below(m)] = xb[u];
        }
        pos += __popcll(m);
      }
      M = total;
      complete = total >= out_n;
    }
  }
  FG_RDTR(tile, 4);

  if (!complete) {
    // ---- second route: radix select over the whole input ----
    uint64_t prefix = 0ull;
    uint32_t fixed = 0u, above = 0u, round = 0u;
    uint64_t T = 0ull;
    bool capped = false;
    __syncthreads();  // every wave is past its reads of s_wave and the tile map
    for (;; round++) {
      const uint32_t width = min(kReduceAllDigit, 64u - fixed);
      uint32_t* const gh = hist + round * kReduceAllBuckets;
      digit_hist(lh, key, prefix, fixed, width);
#pragma unroll
      for (uint32_t j = 0; j < kReduceAllBuckets / kReduceBlock; j++) {
        const uint32_t c = lh[j * kReduceBlock + tid];
        if (c) __hip_atomic_fetch_add(&gh[j * kReduceBlock + tid], c, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
      }
      grid_sync(work, tiles, gen);
      if (round) {  // every workgroup has read the previous round's table
        uint32_t* const prev = hist + (round - 1u) * kReduceAllBuckets;
        for (uint32_t i = tile * kReduceBlock + tid; i < kReduceAllBuckets; i += tiles * kReduceBlock)
          __hip_atomic_store(&prev[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      top_bucket([&](uint32_t b) { return load_agent(&gh[b]); }, out_n - above, s_wave, s_sel);
      const uint64_t d = s_sel[0];
      const uint32_t before = s_sel[1], in_bucket = s_sel[2];
      __syncthreads();
      fixed += width;
      prefix |= d << (64u - fixed);
      const bool fits = above + before + in_bucket <= kReduceAllList;
      above += before;
      if (fits || fixed == 64u) {
        T = prefix;
        capped = !fits;
        break;
      }
    }
    const uint32_t tie_room = out_n - above;
#pragma unroll
    for (uint32_t e = 0; e < kPer; e++) {
      bool keep = key[e] != 0ull && key[e] >= T;
      if (capped && keep && key[e] == T) keep = atomicAdd(&work->ties, 1u) < tie_room;
      const uint64_t m = ballot(keep);
      if (m == 0ull) continue;
      const uint32_t leader = static_cast<uint32_t>(__builtin_ctzll(m));
      uint32_t first = 0u;
      if (lane == leader) first = atomicAdd(&work->listed, static_cast<uint32_t>(__popcll(m)));
      first = readlane32(first, leader);
      if (keep) {
        const uint32_t at = first + lanes_below(m);
        __hip_atomic_store(&list_comp[at], key[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&list_bits[at], sbits[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    grid_sync(work, tiles, gen);
    uint32_t* const last = hist + round * kReduceAllBuckets;
    for (uint32_t i = tile * kReduceBlock + tid; i < kReduceAllBuckets; i += tiles * kReduceBlock)
      __hip_atomic_store(&last[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    M = load_agent(&work->listed);
    for (uint32_t j = tid; j < M; j += kReduceBlock) {
      s_key[j] = load_agent64(&list_comp[j]);
      s_bits[j] = load_agent(&list_bits[j]);
    }
    grid_sync(work, tiles, gen);  // every workgroup has read the list's length
    if (tile == 0u && tid == 0u) {
      __hip_atomic_store(&work->listed, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&work->ties, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // Zeros past the list to a multiple of kUnroll * 64 (a zero composite
  // ranks no entry: every listed composite is at least 1).
  const uint32_t padded = (M + kUnroll * kWave - 1u) & ~(kUnroll * kWave - 1u);
  for (uint32_t j = M + tid; j < padded; j += kReduceBlock) s_key[j] = 0ull;
  __syncthreads();
  FG_RDTR(tile, 5);

  // ---- 3: places; wave w of workgroup g ranks entries g + tiles * (w + 8 i) ----
  const uint32_t stride = tiles * kWaves;
  for (uint32_t j0 = tile + tiles * wave; j0 < M; j0 += kSweep * stride) {
    uint64_t e[kSweep];
    uint32_t jq[kSweep], gt[kSweep], ge[kSweep];
#pragma unroll
    for (uint32_t q = 0; q < kSweep; q++) {
      jq[q] = j0 + q * stride;
      e[q] = jq[q] < M ? s_key[jq[q]] : ~0ull;
      gt[q] = 0u;
      ge[q] = 0u;
    }
    for (uint32_t i0 = 0; i0 < padded; i0 += kUnroll * kWave) {
      uint64_t x[kUnroll];
#pragma unroll
      for (uint32_t u = 0; u < kUnroll; u++) x[u] = s_key[i0 + u * kWave + lane];
#pragma unroll
      for (uint32_t u = 0; u < kUnroll; u++) {
#pragma unroll
        for (uint32_t q = 0; q < kSweep; q++) {
          gt[q] += x[u] > e[q] ? 1u : 0u;
          ge[q] += x[u] >= e[q] ? 1u : 0u;
        }
      }
    }
#pragma unroll
    for (uint32_t q = 0; q < kSweep; q++) {
      uint32_t rank = wave_reduce_sum_u32(gt[q]);
      if (wave_reduce_sum_u32(ge[q]) > rank + 1u && jq[q] < M) {
        // Copies of this composite (duplicate ids): those listed first rank first.
        uint32_t before = 0u;
        for (uint32_t i = lane; i < jq[q]; i += kWave) before += s_key[i] == e[q] ? 1u : 0u;
        rank += wave_reduce_sum_u32(before);
      }
      if (lane == 0u && jq[q] < M && rank < out_n) {
        out_scores[rank] = __uint_as_float(s_bits[jq[q]]);
        out_ids[rank] = e[q] == 1ull ? kInvalidId : ~static_cast<uint32_t>(e[q]);
      }
    }
  }
  FG_RDTR(tile, 6);
}

}  // namespace fg
