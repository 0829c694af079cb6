// Device primitives for the gfx950 sampling kernels (wave64).
//
// Keys: float_key is the order-preserving map of shaders/fg_topk_select.comp:27-31
// (NaN/Inf -> 0; +0 above -0).  A candidate is carried as one 64-bit
// "composite" (key << 31) | (2^31 - 1 - id), ids < 2^31: ids are unique within
// a row, so composites are unique and their unsigned order is exactly the
// top-k order of the reference's select ladder (key desc, then lower id
// first).  Composite 0 (and anything below 2^31) means "no candidate".  Bit 63
// is clear and a finite key is >= 2^23, so read as an f64 a composite is a
// positive normal number (or +0): f64 max/min order composites in one
// instruction each.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fg {

constexpr int kWave = 64;
constexpr uint32_t kInvalidId = 0xffffffffu;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t lane_id() {
  return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

// Number of set bits of `mask` below this lane.
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// Orders LDS traffic between lanes of one wave: LDS executes a wave's
// operations in issue order, so a compiler fence at wavefront scope suffices.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

__device__ __forceinline__ bool is_finite_bits(uint32_t b) {
  return (b & 0x7f800000u) != 0x7f800000u;
}

__device__ __forceinline__ uint32_t float_key(float v) {
  const uint32_t b = __float_as_uint(v);
  if (!is_finite_bits(b)) return 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float key_to_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

constexpr uint64_t kFiniteComp = 1ull << 31;  // smallest composite of a real candidate

__device__ __forceinline__ uint64_t make_comp(uint32_t key, uint32_t id) {
  return (static_cast<uint64_t>(key) << 31) | static_cast<uint64_t>(0x7fffffffu - id);
}
__device__ __forceinline__ uint32_t comp_key(uint64_t c) { return static_cast<uint32_t>(c >> 31); }
__device__ __forceinline__ uint32_t comp_id(uint64_t c) {
  return 0x7fffffffu - static_cast<uint32_t>(c & 0x7fffffffull);
}
// The largest composite below every composite with key >= T.
__device__ __forceinline__ uint64_t key_floor(uint32_t T) {
  return (static_cast<uint64_t>(T) << 31) - 1ull;
}

// Value-order composite: like make_comp, but -0 takes the key of +0, so two
// zeros of either sign tie on value and the lower id ranks first (the order
// of the select's sort, src/sampler.c:88-96).  0 for a non-finite value.
__device__ __forceinline__ uint64_t value_comp(float v, uint32_t id) {
  uint32_t b = __float_as_uint(v);
  if (!is_finite_bits(b)) return 0ull;
  if (b == 0x80000000u) b = 0u;
  return make_comp((b & 0x80000000u) ? ~b : (b | 0x80000000u), id);
}

// e^x in f64 for x <= 0, to a few ulp, by the table-driven method of
// P. T. P. Tang (ACM TOMS 15(2), 1989): x = (64k + j) ln2/64 + r with
// |r| <= ln2/128 (Cody-Waite reduction with a two-part ln2/64 and fma),
// e^x = 2^k 2^(j/64) e^r, e^r by its Taylor polynomial to r^6 (truncation
// below 3e-20).  The table holds 2^(j/64) rounded to nearest.  Used for the
// masses that a top-p cut compares, so that a cut agrees with an f64 libm
// reference to ~1e-15 of the row's mass.
__constant__ const double kExp2Frac64[64] = {
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,
    0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0,
};

__device__ __forceinline__ double exp_nonpos(double x) {
  x = fmax(x, -800.0);  // e^-800 underflows to 0 like libm exp
  const double n = rint(x * 0x1.71547652b82fep+6);  // x * 64 / ln2
  double r = fma(-n, 0x1.62e42fefa39efp-7, x);      // x - n * ln2/64 (high part)
  r = fma(-n, 0x1.abc9e3b39803fp-62, r);            // ... (low part)
  double q = fma(r, 1.0 / 720.0, 1.0 / 120.0);
  q = fma(r, q, 1.0 / 24.0);
  q = fma(r, q, 1.0 / 6.0);
  q = fma(r, q, 0.5);
  q = fma(r, q, 1.0);
  q = fma(r, q, 1.0);
  const int ni = static_cast<int>(n);
  return ldexp(kExp2Frac64[ni & 63] * q, ni >> 6);
}

// The same without the table: x = n ln2 + r, |r| <= ln2/2, e^r by its
// Taylor polynomial to r^12 (truncation below 2e-16).  No memory access, for
// use inside streaming loops.
__device__ __forceinline__ double exp_nonpos_poly(double x) {
  x = fmax(x, -800.0);
  const double n = rint(x * 0x1.71547652b82fep+0);  // x / ln2
  double r = fma(-n, 0x1.62e42fefa39efp-1, x);       // x - n ln2 (high part)
  r = fma(-n, 0x1.abc9e3b39803fp-56, r);             // ... (low part)
  double q = fma(r, 1.0 / 479001600.0, 1.0 / 39916800.0);
  q = fma(r, q, 1.0 / 3628800.0);
  q = fma(r, q, 1.0 / 362880.0);
  q = fma(r, q, 1.0 / 40320.0);
  q = fma(r, q, 1.0 / 5040.0);
  q = fma(r, q, 1.0 / 720.0);
  q = fma(r, q, 1.0 / 120.0);
  q = fma(r, q, 1.0 / 24.0);
  q = fma(r, q, 1.0 / 6.0);
  q = fma(r, q, 0.5);
  q = fma(r, q, 1.0);
  q = fma(r, q, 1.0);
  return ldexp(q, static_cast<int>(n));
}

// Greedy order of src/output.c:484-492 as one 64-bit max: non-finite values
// rank first (hi = all ones), finite ones by key with -0 folded onto +0 (the
// reference compares values, so 0 == -0 and the lower id wins), ties by lower
// id (lo = ~id).  Padding ids encode as 0 and lose to everything.
__device__ __forceinline__ uint64_t greedy_comp(float v, uint32_t id) {
  if (id == kInvalidId) return 0ull;
  uint32_t b = __float_as_uint(v);
  uint32_t hi;
  if (!is_finite_bits(b)) {
    hi = 0xffffffffu;
  } else {
    if (b == 0x80000000u) b = 0u;
    hi = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  }
  return (static_cast<uint64_t>(hi) << 32) | static_cast<uint64_t>(~id);
}
__device__ __forceinline__ uint32_t greedy_id(uint64_t c) { return ~static_cast<uint32_t>(c); }

// ---- tagged hand-off words ------------------------------------------------------
// A word one workgroup stores for another to poll: bit 63 set, bits 62-50 an
// epoch (1-8191), bits 49-0 a payload, 0 for nothing stored.  The reader polls
// until the word carries the epoch it expects, so words are never cleared.
constexpr uint32_t kWireIdBits = 18;
constexpr uint32_t kWireVocab = 1u << kWireIdBits;  // ids below this travel in a word
constexpr uint64_t kWirePayload = (1ull << 50) - 1ull;
constexpr uint32_t kMaxEpoch = 8191;  // epochs 1..8191

__device__ __forceinline__ uint64_t wire_header(uint32_t epoch) {
  return (0x2000ull | epoch) << 50;
}
__device__ __forceinline__ bool wire_current(uint64_t w, uint64_t header) {
  return (w >> 50) == (header >> 50);
}
// Greedy composite <-> payload (high word = greedy key, low word = ~id; ids
// below kWireVocab): a larger payload is a larger composite.
__device__ __forceinline__ uint64_t greedy_payload(uint64_t g) {
  if (g == 0ull) return 0ull;
  return ((g >> 32) << kWireIdBits) | static_cast<uint64_t>(kWireVocab - 1u - greedy_id(g));
}
__device__ __forceinline__ uint64_t greedy_of_payload(uint64_t w) {
  if (w == 0ull) return 0ull;
  const uint32_t id = kWireVocab - 1u - static_cast<uint32_t>(w & (kWireVocab - 1u));
  return ((w >> kWireIdBits) << 32) | static_cast<uint64_t>(~id);
}

// Penalty of src/sampler.c:55-58 for one logit seen c > 0 times.  The kernels
// are compiled with -ffp-contract=off so the product and the sum round
// separately, and '/' is the IEEE-rounded f32 division.
// The same value without branches: both the quotient and the product are
// formed and one is selected (s / 1 and s * 1 are exact, so a repetition of
// 1 needs no test); a zero count returns s.
__device__ __forceinline__ float penalise_sel(float s, uint32_t c, float pres, float freq,
                                              float rep) {
  const float q = s / rep;
  const float m = s * rep;
  const float r = s > 0.0f ? q : m;
  const float fc = freq * static_cast<float>(c);
  const float total = fc + pres;
  return c != 0u ? r - total : s;
}

__device__ __forceinline__ float penalise(float s, uint32_t c, float pres, float freq, float rep) {
  if (c == 0u) return s;
  if (rep != 1.0f) s = s > 0.0f ? s / rep : s * rep;
  const float fc = freq * static_cast<float>(c);
  const float total = fc + pres;
  return s - total;
}

// ---- cross-lane exchanges in VALU (DPP and gfx950 permlane swaps) ----------
//
// lane_xor<J>(v) returns v of lane (lane ^ J).  J = 1, 2: quad_perm; 4: the
// half-row mirror (^7) followed by the quad mirror (^3); 8: row rotate by 8;
// 16, 32: v_permlane16/32_swap, which hand every lane both members of its pair.

// Every control used here reads a valid lane for every lane, so the DPP
// "old" operand is never selected and needs no initialising move.
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_mov_dpp(static_cast<int>(v), kCtrl, 0xf, 0xf, false));
}

template <int J>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
  if constexpr (J == 1) {
    return dpp<0xB1>(v);
  } else if constexpr (J == 2) {
    return dpp<0x4E>(v);
  } else if constexpr (J == 4) {
    return dpp<0x1B>(dpp<0x141>(v));
  } else if constexpr (J == 8) {
    return dpp<0x128>(v);
  } else if constexpr (J == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane_id() & 16u) ? r[0] : r[1];
  } else {
    static_assert(J == 32, "lane_xor: J must be a power of two below 64");
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane_id() & 32u) ? r[0] : r[1];
  }
}

template <int J>
__device__ __forceinline__ uint64_t lane_xor64(uint64_t v) {
  const uint32_t lo = lane_xor<J>(static_cast<uint32_t>(v));
  const uint32_t hi = lane_xor<J>(static_cast<uint32_t>(v >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// v of lane 63 - lane.
__device__ __forceinline__ uint32_t lane_reverse(uint32_t v) {
  return lane_xor<32>(lane_xor<16>(dpp<0x140>(v)));
}
__device__ __forceinline__ uint64_t lane_reverse64(uint64_t v) {
  const uint32_t lo = lane_reverse(static_cast<uint32_t>(v));
  const uint32_t hi = lane_reverse(static_cast<uint32_t>(v >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t readlane64(uint64_t v, uint32_t lane) {
  const uint32_t lo = static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), static_cast<int>(lane)));
  const uint32_t hi = static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), static_cast<int>(lane)));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ uint32_t readlane32(uint32_t v, uint32_t lane) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_readlane(static_cast<int>(v), static_cast<int>(lane)));
}

// One compare-exchange step of a bitonic network over the 64 lanes: blocks of
// K lanes, partner at distance J; the final order is descending by lane.
template <int K, int J, typename T>
__device__ __forceinline__ T bitonic_step(T v) {
  const uint32_t lane = lane_id();
  const bool desc = (K == kWave) || ((lane & K) == 0);
  const bool lower = (lane & J) == 0;
  if constexpr (sizeof(T) == 8) {
    // One 64-bit compare and two selects; the lane pattern (lower == desc)
    // folds into the compare's mask.  (An f64 max/min pair would carry two
    // NaN-quieting canonicalisations per step.)
    const T o = lane_xor64<J>(v);
    const bool gt = o > v;
    return (gt == (lower == desc)) ? o : v;
  } else {
    const T o = lane_xor<J>(v);
    const T hi = o > v ? o : v;
    const T lo = o > v ? v : o;
    return (lower == desc) ? hi : lo;
  }
}

template <int K, typename T>
__device__ __forceinline__ T bitonic_merge_stage(T v) {
  if constexpr (K >= 64) v = bitonic_step<K, 32>(v);
  if constexpr (K >= 32) v = bitonic_step<K, 16>(v);
  if constexpr (K >= 16) v = bitonic_step<K, 8>(v);
  if constexpr (K >= 8) v = bitonic_step<K, 4>(v);
  if constexpr (K >= 4) v = bitonic_step<K, 2>(v);
  return bitonic_step<K, 1>(v);
}

// Sorts one value per lane across the wave, descending (lane 0 the largest).
template <typename T>
__device__ __forceinline__ T wave_sort_desc(T v) {
  v = bitonic_merge_stage<2>(v);
  v = bitonic_merge_stage<4>(v);
  v = bitonic_merge_stage<8>(v);
  v = bitonic_merge_stage<16>(v);
  v = bitonic_merge_stage<32>(v);
  return bitonic_merge_stage<64>(v);
}
// Sorts lanes [0, w) descending when every lane >= w holds 0.  After the
// stage of width K, lanes [0, K) form a descending block, so for w <= 16 or
// w <= 32 the later stages only reorder zeros and are skipped (10 or 15
// steps instead of 21; the width-16 stages stay inside a DPP row).  The
// result is a descending 64-lane sequence, zeros last.
__device__ __forceinline__ uint64_t wave_sort_desc_first(uint64_t v, uint32_t w) {
  v = bitonic_merge_stage<2>(v);
  v = bitonic_merge_stage<4>(v);
  v = bitonic_merge_stage<8>(v);
  v = bitonic_merge_stage<16>(v);
  if (w <= 16u) return v;
  v = bitonic_merge_stage<32>(v);
  if (w <= 32u) return v;
  return bitonic_merge_stage<64>(v);
}
__device__ __forceinline__ uint64_t wave_sort_desc_u64(uint64_t v) { return wave_sort_desc(v); }
__device__ __forceinline__ uint32_t wave_sort_desc_u32(uint32_t v) { return wave_sort_desc(v); }

// a and b are descending across the lanes; returns the 64 largest of both,
// descending.  max(a_i, b_{63-i}) is bitonic and holds the 64 largest.
__device__ __forceinline__ uint64_t wave_merge_desc(uint64_t a, uint64_t b) {
  const uint64_t r = lane_reverse64(b);
  return bitonic_merge_stage<64>(a > r ? a : r);
}

// Two independent merges, written side by side so their dependent chains
// interleave.
__device__ __forceinline__ void wave_merge_desc2(uint64_t& a0, uint64_t b0, uint64_t& a1,
                                                 uint64_t b1) {
  const uint64_t r0 = lane_reverse64(b0);
  const uint64_t r1 = lane_reverse64(b1);
  uint64_t x0 = a0 > r0 ? a0 : r0;
  uint64_t x1 = a1 > r1 ? a1 : r1;
  x0 = bitonic_step<64, 32>(x0); x1 = bitonic_step<64, 32>(x1);
  x0 = bitonic_step<64, 16>(x0); x1 = bitonic_step<64, 16>(x1);
  x0 = bitonic_step<64, 8>(x0);  x1 = bitonic_step<64, 8>(x1);
  x0 = bitonic_step<64, 4>(x0);  x1 = bitonic_step<64, 4>(x1);
  x0 = bitonic_step<64, 2>(x0);  x1 = bitonic_step<64, 2>(x1);
  x0 = bitonic_step<64, 1>(x0);  x1 = bitonic_step<64, 1>(x1);
  a0 = x0;
  a1 = x1;
}

// Waits until this wave's memory operations have completed; the signal
// fences keep the compiler from moving memory operations across the wait.
//
// Cross-workgroup hand-offs (publish, count in, the last one reads) use it
// instead of release/acquire fences.  In the HIP memory model a relaxed
// counter increment is ordered after earlier stores only by a release, and
// the reader's loads after it only by an acquire; at agent scope on gfx950
// those are an L2 write-back (buffer_wbl2) and an L2 invalidate (buffer_inv),
// which took a sampling launch from 20 us to 135 us.  The hand-offs get the
// same ordering from what the ISA guarantees for the accesses they use:
//  1. every published value is an agent-scope atomic store (sc1), written
//     through to the device-coherent level, never left dirty in one XCD's L2
//     (the write-back a release adds is for plain stores, and there are none);
//  2. s_waitcnt 0 returns only when those stores are acknowledged by that
//     level, and only then is the counter's agent-scope atomic issued;
//  3. the reader branches on the atomic's returned value before it issues
//     its loads, and those are agent-scope atomic loads (sc1), which do not
//     return a stale copy from its own caches (the invalidate an acquire adds
//     is for plain loads, and there are none).
// So a workgroup that learns from the counter that it is last reads every
// partial published before the others counted in.  The signal fences keep
// the compiler from moving the stores past the wait.
__device__ __forceinline__ void wait_memory() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ---- wave reductions and scans ------------------------------------------------

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = max(v, lane_xor64<1>(v));
  v = max(v, lane_xor64<2>(v));
  v = max(v, lane_xor64<4>(v));
  v = max(v, lane_xor64<8>(v));
  v = max(v, lane_xor64<16>(v));
  return max(v, lane_xor64<32>(v));
}

__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
  v = min(v, lane_xor64<1>(v));
  v = min(v, lane_xor64<2>(v));
  v = min(v, lane_xor64<4>(v));
  v = min(v, lane_xor64<8>(v));
  v = min(v, lane_xor64<16>(v));
  return min(v, lane_xor64<32>(v));
}

template <int J>
__device__ __forceinline__ double lane_xor_f64(double x) {
  return __longlong_as_double(static_cast<long long>(
      lane_xor64<J>(static_cast<uint64_t>(__double_as_longlong(x)))));
}

__device__ __forceinline__ double wave_max_f64(double x) {
  x = fmax(x, lane_xor_f64<1>(x));
  x = fmax(x, lane_xor_f64<2>(x));
  x = fmax(x, lane_xor_f64<4>(x));
  x = fmax(x, lane_xor_f64<8>(x));
  x = fmax(x, lane_xor_f64<16>(x));
  return fmax(x, lane_xor_f64<32>(x));
}

// Butterfly sum: every lane ends with the same total.
__device__ __forceinline__ double wave_sum_f64(double x) {
  x += lane_xor_f64<1>(x);
  x += lane_xor_f64<2>(x);
  x += lane_xor_f64<4>(x);
  x += lane_xor_f64<8>(x);
  x += lane_xor_f64<16>(x);
  return x + lane_xor_f64<32>(x);
}

// v of lane (lane - D) inside each row of 16 lanes, 0 for the first D lanes
// of a row (DPP row_shr with bound_ctrl).
template <int D>
__device__ __forceinline__ uint32_t row_shr(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x110 + D, 0xf, 0xf, true));
}

template <int D>
__device__ __forceinline__ double row_shr_f64(double x) {
  const uint64_t b = static_cast<uint64_t>(__double_as_longlong(x));
  const uint32_t lo = row_shr<D>(static_cast<uint32_t>(b));
  const uint32_t hi = row_shr<D>(static_cast<uint32_t>(b >> 32));
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

// Inclusive prefix sum over lanes 0..lane: a row-local Hillis-Steele scan,
// then each row adds the totals of the rows before it (read with readlane).
__device__ __forceinline__ double wave_prefix_sum_f64(double x) {
  x += row_shr_f64<1>(x);
  x += row_shr_f64<2>(x);
  x += row_shr_f64<4>(x);
  x += row_shr_f64<8>(x);
  const uint64_t b = static_cast<uint64_t>(__double_as_longlong(x));
  const double r0 = __longlong_as_double(static_cast<long long>(readlane64(b, 15)));
  const double r1 = __longlong_as_double(static_cast<long long>(readlane64(b, 31)));
  const double r2 = __longlong_as_double(static_cast<long long>(readlane64(b, 47)));
  // The rows' offsets without branches: 0, r0, r0 + r1, (r0 + r1) + r2.
  const uint32_t row = lane_id() >> 4;
  const double r01 = r0 + r1;
  const double r012 = r01 + r2;
  const double before = row < 2u ? (row == 0u ? 0.0 : r0) : (row == 2u ? r01 : r012);
  return x + before;
}

// The same scan where lanes 32-63 hold zeros: exact in lanes 0-31 (the
// upper lanes' results are not meaningful).
__device__ __forceinline__ double wave_prefix_sum_f64_lo32(double x) {
  x += row_shr_f64<1>(x);
  x += row_shr_f64<2>(x);
  x += row_shr_f64<4>(x);
  x += row_shr_f64<8>(x);
  const double r0 = __longlong_as_double(static_cast<long long>(
      readlane64(static_cast<uint64_t>(__double_as_longlong(x)), 15)));
  return (lane_id() >> 4) == 1u ? x + r0 : x;
}

// The same scan for u32 counts.
__device__ __forceinline__ uint32_t wave_prefix_sum_u32(uint32_t x) {
  x += row_shr<1>(x);
  x += row_shr<2>(x);
  x += row_shr<4>(x);
  x += row_shr<8>(x);
  const uint32_t r0 = readlane32(x, 15), r1 = readlane32(x, 31), r2 = readlane32(x, 47);
  const uint32_t row = lane_id() >> 4;
  return x + (row < 2u ? (row == 0u ? 0u : r0) : (row == 2u ? r0 + r1 : r0 + r1 + r2));
}

// The wave's total in every lane.
__device__ __forceinline__ uint32_t wave_reduce_sum_u32(uint32_t x) {
  x += lane_xor<1>(x);
  x += lane_xor<2>(x);
  x += lane_xor<4>(x);
  x += lane_xor<8>(x);
  x += lane_xor<16>(x);
  return x + lane_xor<32>(x);
}

// Inclusive sum over lanes >= this lane (used by the LDS radix select).
__device__ __forceinline__ uint32_t wave_suffix_sum(uint32_t v) {
  const uint32_t lane = lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const uint32_t o = __shfl_down(v, d);
    if (lane + d < kWave) v += o;
  }
  return v;
}

// ---- exact k-th largest composite over an LDS array, one wave -------------
//
// MSB-first radix select, 8 bits per round, on n unique composites in
// buf[0..n).  Requires 1 <= kk <= n.  Returns the kk-th largest composite R;
// exactly kk entries satisfy c >= R.  hist is 256 u32 of wave-private LDS.
__device__ inline uint64_t wave_select_kth(const uint64_t* buf, uint32_t n, uint32_t kk,
                                           uint32_t* hist) {
  const uint32_t lane = lane_id();
  uint64_t prefix = 0;
  uint32_t need = kk;
  for (int shift = 56; shift >= 0; shift -= 8) {
    for (uint32_t b = lane; b < 256u; b += kWave) hist[b] = 0u;
    wave_lds_sync();
    const uint64_t hi_mask = (shift == 56) ? 0ull : (~0ull << (shift + 8));
    for (uint32_t i = lane; i < n; i += kWave) {
      const uint64_t c = buf[i];
      if ((c & hi_mask) == prefix) atomicAdd(&hist[(c >> shift) & 255u], 1u);
    }
    wave_lds_sync();
    uint32_t h[4];
#pragma unroll
    for (int q = 0; q < 4; q++) h[q] = hist[4u * lane + q];
    wave_lds_sync();
    const uint32_t mine = h[0] + h[1] + h[2] + h[3];
    const uint32_t suf = wave_suffix_sum(mine);
    uint32_t above = suf - mine;
    const bool owner = above < need && need <= suf;
    uint32_t bin = 0, bin_above = 0, bin_count = 0;
    if (owner) {
#pragma unroll
      for (int q = 3; q >= 0; q--) {
        if (above + h[q] >= need) {
          bin = 4u * lane + q;
          bin_above = above;
          bin_count = h[q];
          break;
        }
        above += h[q];
      }
    }
    const uint64_t who = ballot(owner);
    const int src = __ffsll(static_cast<unsigned long long>(who)) - 1;
    bin = __shfl(bin, src);
    bin_above = __shfl(bin_above, src);
    bin_count = __shfl(bin_count, src);
    prefix |= static_cast<uint64_t>(bin) << shift;
    need -= bin_above;
    if (bin_count == need) {
      // Every entry of this bucket is in: the answer is the smallest entry
      // whose bits down to `shift` are >= prefix.
      uint64_t best = ~0ull;
      for (uint32_t i = lane; i < n; i += kWave) {
        const uint64_t c = buf[i];
        if (c >= prefix && c < best) best = c;
      }
      return wave_min_u64(best);
    }
  }
  return prefix;  // not reached: a bucket of one unique composite ends the loop
}

// Keeps the entries c >= R of buf[0..n) at the front, in their current order;
// returns how many were kept.
__device__ inline uint32_t wave_compact_ge(uint64_t* buf, uint32_t n, uint64_t R) {
  const uint32_t lane = lane_id();
  uint32_t kept = 0;
  for (uint32_t base = 0; base < n; base += kWave) {
    const uint32_t i = base + lane;
    const uint64_t c = i < n ? buf[i] : 0ull;
    const bool keep = i < n && c >= R;
    const uint64_t m = ballot(keep);
    wave_lds_sync();
    if (keep) buf[kept + lanes_below(m)] = c;
    wave_lds_sync();
    kept += __popcll(m);
  }
  return kept;
}

}  // namespace fg
