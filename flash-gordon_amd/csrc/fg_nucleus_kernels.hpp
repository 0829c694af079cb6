// Whole-row nucleus rows (top_k 0) whose top-p cut lies deeper than the 64
// best logits that the fused pass keeps: finished by the row's finishing
// workgroup of the fused kernel itself (all its waves), in the LDS of its
// staging buffers, so no second launch is needed.
//
// It computes what fg_sampler_select (src/sampler.c:80-122) computes over the
// whole row: sort by (value desc, id asc), cut at the first position where
// the running untempered mass reaches top_p, then draw from the cut set with
// the tempered weights.  Sorting 151,936 logits per row is not needed.  Both
// steps are a weighted select: find the first element, in that order, at
// which a running sum crosses a target.  One workgroup owns a row and
// descends through histograms of mass in LDS (sizes from NucCfg; the fused
// kernel's: 256 threads, 512 bins, 2,048 collected):
//   level 1  kBins bins of value, bin = floor((vmax - v) * kBins / 32)
//            computed in exact f64, so equal values share a bin and bins
//            follow the order (32 logit units below the maximum and beyond
//            share the last bin);
//   level n  the chosen bin as a range of 63-bit value-order composites
//            (value key << 31 | ~id, unique per element), split into kBins
//            equal sub-ranges, until a range is small enough;
//   collect  once the chosen bin holds at most kCollect elements they are
//            gathered into LDS, sorted with a bitonic network and scanned in
//            order.
// Every level is one coalesced pass over the row (16-byte loads, penalties
// re-applied in registers).  Masses are f64 sums of exp_nonpos terms (a few
// ulp each), so a cut agrees with the f64 reference except within ~1e-14 of a
// boundary.  The level-1 histogram carries both the untempered and the
// tempered mass, so the draw reuses it and the cut's sorted bin: a typical
// deep row takes two passes (level 1, collect), three when the draw lands in
// an earlier bin than the cut.
#pragma once

// Included by fg_sample_kernels.hpp, before the fused kernel (it uses the
// sampler's types and helpers defined there).

namespace fg {

// Sizes of the descent: threads of the workgroup, bins per level, entries a
// bin may hold to be collected and sorted.
template <int kBlock_, uint32_t kBins_, uint32_t kCollect_, uint32_t kQuads_>
struct NucCfg {
  static constexpr uint32_t kQuads = kQuads_;  // 16-byte quads per thread per loop step
  static constexpr int kBlock = kBlock_;
  static constexpr int kWaves = kBlock_ / kWave;
  static constexpr uint32_t kBins = kBins_;
  static constexpr uint32_t kBinsPer = kBins_ / kBlock_;
  static constexpr uint32_t kCollect = kCollect_;
  static constexpr uint32_t kListPer = kCollect_ / kBlock_;
  static constexpr double kValueBinScale = static_cast<double>(kBins_) / 32.0;
};
// The fused kernel's: four waves, in the LDS of the staging buffers, and
// few enough registers per thread that the kernel keeps three workgroups
// per CU with no stack.
using FusedNuc = NucCfg<256, 512, 1024, 1>;

constexpr uint32_t kMaxLevels = 8;
constexpr uint32_t kNoBin = 0xffffffffu;

template <class C>
struct NucLds {
  uint32_t cnt[C::kBins];
  double mass[C::kBins];    // untempered exp(v - vmax)
  double tmass[C::kBins];   // tempered exp((v - vmax) / T)
  double tmass1[C::kBins];  // level-1 tempered mass, kept for the draw
  uint32_t cnt1[C::kBins];  // level-1 counts, kept for the draw
  uint64_t list[C::kCollect];
  double wave_a[C::kWaves];
  double wave_b[C::kWaves];
  uint64_t lo, hi;  // composite range (refinement)
  uint32_t pick;    // chosen bin / list index (atomicMin)
  uint32_t last;    // last non-empty bin + 1 (atomicMax)
  uint32_t n;       // collected entries
  double res[4];    // results broadcast by one thread
};

// One level of the descent: which elements take part and their bin.
struct Level {
  bool value;       // level 1: value bins
  uint64_t lo, hi;  // range levels: inclusive composite range
  uint32_t shift;   // range levels: bin = (hi - c) >> shift
};

struct RowView {
  const float* lrow;
  const uint32_t* crow;  // null: no penalties
  RowParams p;
  uint32_t vocab;
  bool vec;  // 16-byte aligned logits (and counts)
  double vmax;
  double inv_t;
};

struct Pick {
  uint64_t comp;
  uint32_t idx;             // index in the sorted list
  double above_m, above_t;  // weight of the elements ranked before comp
  double w_m, w_t;          // weight of comp itself
};

template <class C>
__device__ __forceinline__ uint32_t value_bin(double vmax, float v) {
  const double d = (vmax - static_cast<double>(v)) * C::kValueBinScale;
  return d >= static_cast<double>(C::kBins - 1u) ? C::kBins - 1u : static_cast<uint32_t>(d);
}

__device__ __forceinline__ float pen_value(const RowView& r, float v, uint32_t c) {
  return r.crow ? penalise(v, c, r.p.presence, r.p.frequency, r.p.repetition) : v;
}

__device__ __forceinline__ float row_value(const RowView& r, uint32_t i) {
  return pen_value(r, r.lrow[i], r.crow ? r.crow[i] : 0u);
}

// Calls f(v, id) for every element of the row (penalised value), each once
// across the workgroup.  C::kQuads (1 or 2) 16-byte quads per thread are in
// flight.
template <class C, class Fn>
__device__ __forceinline__ void for_each_element(const RowView& r, Fn&& f) {
  const uint32_t tid = threadIdx.x;
  uint32_t head = 0u;
  if (r.vec) {
    const uint32_t nq = r.vocab / 4u;
    const f4* lq = reinterpret_cast<const f4*>(r.lrow);
    const u4* cq = reinterpret_cast<const u4*>(r.crow);
    for (uint32_t q = tid; q < nq; q += C::kQuads * C::kBlock) {
      const uint32_t q1 = q + C::kBlock;
      const bool ok1 = C::kQuads > 1u && q1 < nq;
      const uint32_t q1c = ok1 ? q1 : q;
      const f4 x0 = lq[q], x1 = lq[q1c];
      u4 y0 = {0u, 0u, 0u, 0u}, y1 = {0u, 0u, 0u, 0u};
      if (r.crow) {
        y0 = cq[q];
        y1 = cq[q1c];
      }
#pragma unroll
      for (int e = 0; e < 4; e++) f(pen_value(r, x0[e], y0[e]), 4u * q + e);
      if (ok1) {
#pragma unroll
        for (int e = 0; e < 4; e++) f(pen_value(r, x1[e], y1[e]), 4u * q1 + e);
      }
    }
    head = nq * 4u;
  }
  for (uint32_t i = head + tid; i < r.vocab; i += C::kBlock) f(row_value(r, i), i);
}

// Exclusive block scan of two f64 series (one value each per thread); also
// returns the totals.  All threads must call it.
template <class C>
__device__ inline void block_scan2(NucLds<C>& s, double a, double b, double* ea, double* eb,
                                   double* ta, double* tb) {
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // uniform
  const uint32_t lane = lane_id();
  const double ia = wave_prefix_sum_f64(a);
  const double ib = wave_prefix_sum_f64(b);
  if (lane == kWave - 1) {
    s.wave_a[wave] = ia;
    s.wave_b[wave] = ib;
  }
  __syncthreads();
  double oa = 0.0, ob = 0.0, sa = 0.0, sb = 0.0;
  for (uint32_t w = 0; w < C::kWaves; w++) {
    const double xa = s.wave_a[w], xb = s.wave_b[w];
    if (w < wave) {
      oa += xa;
      ob += xb;
    }
    sa += xa;
    sb += xb;
  }
  *ea = oa + ia - a;
  *eb = ob + ib - b;
  *ta = sa;
  *tb = sb;
  __syncthreads();
}

// Fills cnt / mass / tmass for one level over the elements with c >= floor.
template <class C>
__device__ inline void histogram_pass(NucLds<C>& s, const RowView& r, const Level& lv,
                                      uint64_t floor) {
  for (uint32_t b = threadIdx.x; b < C::kBins; b += C::kBlock) {
    s.cnt[b] = 0u;
    s.mass[b] = 0.0;
    s.tmass[b] = 0.0;
  }
  __syncthreads();
  for_each_element<C>(r, [&](float v, uint32_t i) {
    const uint64_t c = value_comp(v, i);
    if (c == 0ull || c < floor) return;
    uint32_t b;
    if (lv.value) {
      b = value_bin<C>(r.vmax, v);
    } else {
      if (c < lv.lo || c > lv.hi) return;
      b = static_cast<uint32_t>((lv.hi - c) >> lv.shift);
    }
    const double d = static_cast<double>(v) - r.vmax;
    atomicAdd(&s.cnt[b], 1u);
    atomicAdd(&s.mass[b], exp_nonpos(d));
    atomicAdd(&s.tmass[b], exp_nonpos(d * r.inv_t));
  });
  __syncthreads();
}

// The first bin (in order) at which  above + running weight  crosses the
// target (>= when inclusive, > otherwise); the last non-empty bin if none
// does.  The weight compared is tmass when tempered, else mass.  When
// `limit` is not kNoBin only bins below it take part, from the saved level-1
// series tmass1 / cnt1 (tempered only).
struct BinChoice {
  uint32_t bin;               // kNoBin: every bin empty
  uint32_t count;             // elements in the bin
  double before_c, before_o;  // compared / other weight of the bins before it
  double total_c;             // compared weight of all bins taking part
  bool crossed;
};

template <class C>
__device__ inline BinChoice choose_bin(NucLds<C>& s, double above, double target, bool tempered,
                                       bool inclusive, uint32_t limit) {
  constexpr uint32_t kBinsPer = C::kBinsPer;
  const uint32_t tid = threadIdx.x;
  const bool saved = limit != kNoBin;
  const uint32_t bb = tid * kBinsPer;
  double wc[kBinsPer], wo[kBinsPer], sc = 0.0, so = 0.0;
  uint32_t cn[kBinsPer];
#pragma unroll
  for (uint32_t e = 0; e < kBinsPer; e++) {
    const uint32_t b = bb + e;
    const bool in = !saved || b < limit;
    cn[e] = in ? (saved ? s.cnt1[b] : s.cnt[b]) : 0u;
    const double t = saved ? s.tmass1[b] : s.tmass[b];
    wc[e] = in ? (tempered ? t : s.mass[b]) : 0.0;
    wo[e] = in && !saved ? (tempered ? s.mass[b] : s.tmass[b]) : 0.0;
    sc += wc[e];
    so += wo[e];
  }
  if (tid == 0) {
    s.pick = kNoBin;
    s.last = 0u;
  }
  double ex, ex_o, tot, tot_o;
  block_scan2<C>(s, sc, so, &ex, &ex_o, &tot, &tot_o);  // its barriers order the resets
  {
    uint32_t last = 0u;
#pragma unroll
    for (uint32_t e = 0; e < kBinsPer; e++)
      if (cn[e]) last = bb + e + 1u;
    double c = above + ex;
#pragma unroll
    for (uint32_t e = 0; e < kBinsPer; e++) {
      c += wc[e];
      if (cn[e] && (inclusive ? c >= target : target < c)) {
        atomicMin(&s.pick, bb + e);
        break;
      }
    }
    if (last) atomicMax(&s.last, last);
  }
  __syncthreads();
  BinChoice out;
  out.crossed = s.pick != kNoBin;
  out.bin = out.crossed ? s.pick : (s.last ? s.last - 1u : kNoBin);
  out.total_c = tot;
  if (out.bin != kNoBin && out.bin / kBinsPer == tid) {
    double pc = ex, po = ex_o;
    uint32_t count = 0u;
#pragma unroll
    for (uint32_t e = 0; e < kBinsPer; e++) {
      if (bb + e < out.bin) {
        pc += wc[e];
        po += wo[e];
      }
      if (bb + e == out.bin) count = cn[e];
    }
    s.res[0] = pc;
    s.res[1] = po;
    s.res[2] = static_cast<double>(count);
  }
  __syncthreads();
  out.before_c = s.res[0];
  out.before_o = s.res[1];
  out.count = static_cast<uint32_t>(s.res[2]);
  __syncthreads();
  return out;
}

// Gathers the members of `bin` of level lv (c >= floor) into s.list, sorted
// descending; returns their number (<= kCollect).
template <class C>
__device__ inline uint32_t collect_sorted(NucLds<C>& s, const RowView& r, const Level& lv,
                                          uint32_t bin, uint64_t floor) {
  constexpr uint32_t kCollect = C::kCollect;
  const uint32_t tid = threadIdx.x;
  if (tid == 0) s.n = 0u;
  __syncthreads();
  for_each_element<C>(r, [&](float v, uint32_t i) {
    const uint64_t c = value_comp(v, i);
    if (c == 0ull || c < floor) return;
    bool in;
    if (lv.value)
      in = value_bin<C>(r.vmax, v) == bin;
    else
      in = c >= lv.lo && c <= lv.hi && static_cast<uint32_t>((lv.hi - c) >> lv.shift) == bin;
    if (in) {
      const uint32_t slot = atomicAdd(&s.n, 1u);
      if (slot < kCollect) s.list[slot] = c;
    }
  });
  __syncthreads();
  const uint32_t n = min(s.n, kCollect);
  uint32_t P = 1u;
  while (P < n) P <<= 1;
  for (uint32_t i = n + tid; i < P; i += C::kBlock) s.list[i] = 0ull;
  __syncthreads();
  for (uint32_t k = 2u; k <= P; k <<= 1) {
    for (uint32_t j = k >> 1; j > 0u; j >>= 1) {
      for (uint32_t i = tid; i < P; i += C::kBlock) {
        const uint32_t ixj = i ^ j;
        if (ixj > i) {
          const uint64_t x = s.list[i], y = s.list[ixj];
          const bool desc = (i & k) == 0u;
          if (desc ? x < y : x > y) {
            s.list[i] = y;
            s.list[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
  return n;
}

// Scans the first n (>= 1) entries of the sorted list in order (running
// weights start at above_m / above_t) and returns the first crossing entry,
// or the n-th if none crosses.
template <class C>
__device__ inline Pick scan_list(NucLds<C>& s, const RowView& r, uint32_t n, double above_m,
                                 double above_t, double target, bool tempered, bool inclusive) {
  constexpr uint32_t kListPer = C::kListPer;
  const uint32_t tid = threadIdx.x;
  double wm[kListPer], wt[kListPer], sm = 0.0, st = 0.0;
#pragma unroll
  for (uint32_t e = 0; e < kListPer; e++) {
    const uint32_t idx = tid * kListPer + e;
    wm[e] = wt[e] = 0.0;
    if (idx < n) {
      const double d = static_cast<double>(key_to_float(comp_key(s.list[idx]))) - r.vmax;
      wm[e] = exp_nonpos(d);
      wt[e] = exp_nonpos(d * r.inv_t);
    }
    sm += wm[e];
    st += wt[e];
  }
  if (tid == 0) s.pick = kNoBin;
  double exm, ext, totm, tott;
  block_scan2<C>(s, sm, st, &exm, &ext, &totm, &tott);
  {
    double cm = above_m + exm, ct = above_t + ext;
#pragma unroll
    for (uint32_t e = 0; e < kListPer; e++) {
      const uint32_t idx = tid * kListPer + e;
      cm += wm[e];
      ct += wt[e];
      const double c = tempered ? ct : cm;
      if (idx < n && (inclusive ? c >= target : target < c)) {
        atomicMin(&s.pick, idx);
        break;
      }
    }
  }
  __syncthreads();
  const uint32_t idx = s.pick != kNoBin ? s.pick : n - 1u;
  if (idx / kListPer == tid) {
    const uint32_t off = idx - tid * kListPer;
    double pm = above_m + exm, pt = above_t + ext, om = 0.0, ot = 0.0;
#pragma unroll
    for (uint32_t e = 0; e < kListPer; e++) {
      if (e < off) {
        pm += wm[e];
        pt += wt[e];
      }
      if (e == off) {
        om = wm[e];
        ot = wt[e];
      }
    }
    s.res[0] = pm;
    s.res[1] = pt;
    s.res[2] = om;
    s.res[3] = ot;
  }
  __syncthreads();
  Pick out{s.list[idx], idx, s.res[0], s.res[1], s.res[2], s.res[3]};
  __syncthreads();
  return out;
}

// The weighted select from a chosen bin of level lv on: collects the bin if
// it is small enough, else narrows the range and descends.  `above_*` are
// the weights ranked before the bin.  *refined reports whether the result
// came from a level below lv.
template <class C>
__device__ inline Pick descend_from(NucLds<C>& s, const RowView& r, Level lv, uint32_t bin,
                                    uint32_t count, double above_m, double above_t,
                                    uint64_t floor, double target, bool tempered, bool inclusive,
                                    bool* refined) {
  *refined = false;
  for (uint32_t level = 0; level < kMaxLevels; level++) {
    if (count <= C::kCollect) {
      const uint32_t n = collect_sorted<C>(s, r, lv, bin, floor);
      if (n == 0u) break;
      return scan_list<C>(s, r, n, above_m, above_t, target, tempered, inclusive);
    }
    *refined = true;
    // The chosen bin becomes the next level's composite range.
    if (lv.value) {
      if (threadIdx.x == 0) {
        s.lo = ~0ull;
        s.hi = 0ull;
      }
      __syncthreads();
      uint64_t mn = ~0ull, mx = 0ull;
      for_each_element<C>(r, [&](float v, uint32_t i) {
        const uint64_t c = value_comp(v, i);
        if (c == 0ull || c < floor || value_bin<C>(r.vmax, v) != bin) return;
        mn = c < mn ? c : mn;
        mx = c > mx ? c : mx;
      });
      mn = wave_min_u64(mn);
      mx = wave_max_u64(mx);
      if (lane_id() == 0) {
        atomicMin(reinterpret_cast<unsigned long long*>(&s.lo), mn);
        atomicMax(reinterpret_cast<unsigned long long*>(&s.hi), mx);
      }
      __syncthreads();
      lv.value = false;
      lv.lo = s.lo;
      lv.hi = s.hi;
      __syncthreads();
      if (lv.lo > lv.hi) break;
    } else {
      const uint64_t top = lv.hi - (static_cast<uint64_t>(bin) << lv.shift);
      const uint64_t width = (1ull << lv.shift) - 1ull;
      lv.lo = top - lv.lo > width ? top - width : lv.lo;
      lv.hi = top;
    }
    // Each range level narrows the range by kBins (512: 9 bits), so 63-bit
    // composites need at most 7 levels; kMaxLevels only bounds the loop.
    uint32_t sh = 0u;
    while (((lv.hi - lv.lo) >> sh) >= C::kBins) sh++;
    lv.shift = sh;
    histogram_pass<C>(s, r, lv, floor);
    const BinChoice ch =
        choose_bin<C>(s, tempered ? above_t : above_m, target, tempered, inclusive, kNoBin);
    if (ch.bin == kNoBin) break;
    bin = ch.bin;
    count = ch.count;
    above_m += tempered ? ch.before_o : ch.before_c;
    above_t += tempered ? ch.before_c : ch.before_o;
  }
  return Pick{0ull, 0u, 0.0, 0.0, 0.0, 0.0};  // not reached for a consistent row
}

// What the descent needs of one deep row (by value: the sampler's argument
// block is too large to pass to a function that is not inlined).
struct DeepRow {
  const float* lrow;
  const uint32_t* crow;  // null: no penalties
  RowParams p;
  uint32_t vocab;
  float u;               // the row's uniform
  float vmax;            // the row's largest finite (penalised) value
  uint32_t* token;
  float* token_logit;    // optional
  int32_t* status;       // optional
};

// The descent for one deep row; every thread of the workgroup calls it.
// Writes the row's token, logit and status.  Inlined: a call would give the
// whole kernel a stack (the callee-saved registers it uses).
template <class C>
__device__ __forceinline__ void nucleus_deep_row(
    const float* lrow, const uint32_t* crow, float temperature, float top_p, float presence,
    float frequency, float repetition, uint32_t vocab, float u_row, float vmax, uint32_t* token,
    float* token_logit, int32_t* status, NucLds<C>& s) {
  RowParams p{};
  p.temperature = temperature;
  p.top_p = top_p;
  p.presence = presence;
  p.frequency = frequency;
  p.repetition = repetition;
  const DeepRow dr{lrow, crow, p, vocab, u_row, vmax, token, token_logit, status};
  const uint32_t tid = threadIdx.x;
  const bool vec = (reinterpret_cast<uintptr_t>(dr.lrow) & 15u) == 0u &&
                   (!dr.crow || (reinterpret_cast<uintptr_t>(dr.crow) & 15u) == 0u);
  const RowView r{dr.lrow, dr.crow, p, dr.vocab, vec, static_cast<double>(dr.vmax),
                  1.0 / static_cast<double>(p.temperature)};

  // Level 1 over every finite element: both masses per value bin.
  const Level l1{true, 0ull, 0ull, 0u};
  histogram_pass<C>(s, r, l1, kFiniteComp);
  for (uint32_t b = tid; b < C::kBins; b += C::kBlock) {
    s.tmass1[b] = s.tmass[b];
    s.cnt1[b] = s.cnt[b];
  }
  double total_m, total_t;
  {
    double sm = 0.0, st = 0.0, e0, e1;
    for (uint32_t b = tid; b < C::kBins; b += C::kBlock) {
      sm += s.mass[b];
      st += s.tmass[b];
    }
    block_scan2<C>(s, sm, st, &e0, &e1, &total_m, &total_t);
  }

  float u = dr.u;
  if (!is_finite_bits(__float_as_uint(u)) || u < 0.0f) u = 0.0f;
  if (u >= 1.0f) u = __uint_as_float(0x3f7fffffu);  // nextafterf(1, 0)
  bool refined;
  Pick d{0ull, 0u, 0.0, 0.0, 0.0, 0.0};

  if (p.top_p >= 1.0f) {
    // The cut keeps every finite logit: draw from the level-1 histogram.
    const double target = static_cast<double>(u) * total_t;
    const BinChoice ch = choose_bin<C>(s, 0.0, target, true, false, kNoBin);
    if (ch.bin != kNoBin)
      d = descend_from<C>(s, r, l1, ch.bin, ch.count, ch.before_o, ch.before_c, kFiniteComp, target,
                       true, false, &refined);
  } else {
    // Cut: first position where the running mass reaches top_p of the total.
    const double target = static_cast<double>(p.top_p) * total_m;
    const BinChoice ch = choose_bin<C>(s, 0.0, target, false, true, kNoBin);
    Pick c{0ull, 0u, 0.0, 0.0, 0.0, 0.0};
    if (ch.bin != kNoBin)
      c = descend_from<C>(s, r, l1, ch.bin, ch.count, ch.before_c, ch.before_o, kFiniteComp, target,
                       false, true, &refined);
    if (c.comp != 0ull) {
      const double draw = static_cast<double>(u) * (c.above_t + c.w_t);
      // Bins before the cut's bin lie wholly inside the cut set.
      const BinChoice dh = choose_bin<C>(s, 0.0, draw, true, false, ch.bin);
      if (dh.crossed) {
        d = descend_from<C>(s, r, l1, dh.bin, dh.count, 0.0, dh.before_c, kFiniteComp, draw, true,
                         false, &refined);
      } else if (!refined) {
        // The cut's bin is still sorted in LDS: draw among its entries up
        // to the cut, after all the bins before it.
        d = scan_list<C>(s, r, c.idx + 1u, 0.0, dh.total_c, draw, true, false);
      } else {
        // Rare: the cut needed a finer level; rerun the descent above it.
        histogram_pass<C>(s, r, l1, c.comp);
        const BinChoice dd = choose_bin<C>(s, 0.0, draw, true, false, kNoBin);
        if (dd.bin != kNoBin)
          d = descend_from<C>(s, r, l1, dd.bin, dd.count, dd.before_o, dd.before_c, c.comp, draw,
                           true, false, &refined);
      }
    }
  }
  if (tid == 0) {
    if (d.comp == 0ull) {
      *dr.token = kInvalidId;
      if (dr.status) *dr.status = kStLimit;
    } else {
      const uint32_t id = comp_id(d.comp);
      *dr.token = id;
      // The logit keeps its sign of zero: read it back from the row.
      if (dr.token_logit) *dr.token_logit = row_value(r, id);
      if (dr.status) *dr.status = kStOk;
    }
  }
}

}  // namespace fg
