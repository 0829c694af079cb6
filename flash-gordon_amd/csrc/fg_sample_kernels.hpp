// gfx950 kernels of the batched sampler: one fused streaming pass over
// rows x vocab f32 logits (+ u32 history counts) that ends in a token per row.
//
// Grid: rows x chunks workgroups of 256 threads (4 waves).  Each wave streams
// a contiguous slice of its row once from HBM (16-byte non-temporal loads of
// logits and counts) and keeps in registers/LDS only what the row result
// needs:
//   * penalties (src/sampler.c:55-58) applied in registers;
//   * greedy: the best greedy composite (src/output.c:484-492);
//   * top-k:  an LDS candidate buffer filtered by a rising composite
//             threshold, cut back to the exact top-kk by an LDS radix select
//             when it fills (the per-tile radix idea of
//             shaders/fg_topk_select.comp:45-77, applied per wave);
//   * log-probs: per-lane online (max, sum exp) in f32.
// Each workgroup merges its 4 waves, publishes a sorted top-kk list, its
// greedy winner and its (max, sum) to the workspace, raises the row's key
// threshold (a lower bound on the row's kk-th key) and bumps the row's
// arrival counter.  The last workgroup of a row merges the row and runs the
// select arithmetic of src/sampler.c:80-122 in one wave, then resets the row's
// counter and threshold for the next launch.
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
constexpr uint32_t kCap = 256;       // per-wave candidate buffer (composites)
constexpr uint32_t kMaxK = 64;       // largest top-k / log-prob count
constexpr uint32_t kMaxChunks = 64;  // workgroups per row (one lane each in merges)
constexpr int kStepVec = 4;          // float4 per lane per streaming step

constexpr int32_t kStOk = 0;
constexpr int32_t kStFormat = 4;
constexpr int32_t kStMismatch = 5;

struct SampleArgs {
  const float* logits;
  uint64_t lstride;
  const uint32_t* counts;
  uint64_t cstride;
  const float* uniforms;
  const RowParams* params;
  uint32_t vocab;
  uint32_t rows;
  uint32_t chunks;      // workgroups per row
  uint32_t wave_elems;  // elements per wave slice (multiple of 4)
  uint32_t logprobs;
  uint32_t* tokens;
  float* token_logits;
  int32_t* row_status;
  float* penalised;
  float* lp_values;
  uint32_t* lp_ids;
  // workspace
  uint64_t* cand;        // [rows][chunks][kMaxK] sorted composites, 0 = empty
  uint64_t* greedy;      // [rows][chunks] greedy composites
  double* lse;           // [rows][chunks][2] (max s, sum exp((s - max)/T))
  uint32_t* row_thr;     // [rows] key lower bound, reset by the last workgroup
  uint32_t* row_done;    // [rows] arrivals, reset by the last workgroup
};

// ---- per-wave candidate buffer --------------------------------------------

struct Cand {
  uint64_t* buf;   // kCap composites, wave-private LDS
  uint32_t* hist;  // 256 u32, wave-private LDS
  uint32_t n;      // entries in buf (wave-uniform)
  uint64_t R;      // pass iff composite > R (wave-uniform)
  uint32_t kk;     // how many to keep
};

// Cuts the buffer back to its exact top-kk and raises the threshold to the
// kk-th composite: anything not above it can never enter the top-kk.
__device__ inline void cand_reduce(Cand& c) {
  if (c.n <= c.kk) return;
  const uint64_t R = wave_select_kth(c.buf, c.n, c.kk, c.hist);
  c.n = wave_compact_ge(c.buf, c.n, R);
  if (R > c.R) c.R = R;
}

__device__ __forceinline__ void cand_push(Cand& c, uint64_t comp) {
  bool pass = comp > c.R;
  uint64_t m = ballot(pass);
  if (m == 0ull) return;
  if (c.n + static_cast<uint32_t>(__popcll(m)) > kCap) {
    cand_reduce(c);
    pass = comp > c.R;
    m = ballot(pass);
    if (m == 0ull) return;
  }
  if (pass) c.buf[c.n + lanes_below(m)] = comp;
  c.n += static_cast<uint32_t>(__popcll(m));
}

// Wave 0 of a workgroup: gathers the 4 wave buffers (each <= kk entries) into
// buffer 0, cuts to the exact top-kk and returns this lane's entry of the
// descending list (0 past the end).  *count receives the list length.
__device__ inline uint64_t wave0_merge(uint64_t (*bufs)[kCap], const uint32_t* ns, uint32_t* hist,
                                       uint32_t kk, uint32_t* count) {
  const uint32_t lane = lane_id();
  uint32_t n = ns[0];
  for (int w = 1; w < kWaves; w++) {
    const uint32_t m = ns[w];
    for (uint32_t i = lane; i < m; i += kWave) bufs[0][n + i] = bufs[w][i];
    n += m;
  }
  wave_lds_sync();
  if (n > kk) {
    const uint64_t R = wave_select_kth(bufs[0], n, kk, hist);
    n = wave_compact_ge(bufs[0], n, R);
  }
  wave_lds_sync();
  const uint64_t mine = lane < n ? bufs[0][lane] : 0ull;
  *count = n;
  return wave_sort_desc_u64(mine);
}

__device__ __forceinline__ double wave_prefix_sum_f64(double x) {
  const uint32_t lane = lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const double o = __shfl_up(x, d);
    if (lane >= static_cast<uint32_t>(d)) x += o;
  }
  return x;
}

__device__ __forceinline__ double wave_max_f64(double x) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const double o = __shfl_xor(x, d);
    x = o > x ? o : x;
  }
  return x;
}

__device__ __forceinline__ double wave_sum_f64(double x) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) x += __shfl_xor(x, d);
  return x;
}

// Value order of src/sampler.c:75-78 (value desc, id asc) as a composite:
// -0 folds onto +0 because the reference compares floats.
__device__ __forceinline__ uint64_t value_comp_from(uint64_t key_comp) {
  if (key_comp == 0ull) return 0ull;
  uint32_t k = comp_key(key_comp);
  if (k == 0x7fffffffu) k = 0x80000000u;  // key(-0) -> key(+0)
  return (static_cast<uint64_t>(k) << 32) | (key_comp & 0xffffffffull);
}

// ---- the fused kernel ------------------------------------------------------

template <bool kVec>
__global__ __launch_bounds__(kBlock) void sample_rows_kernel(SampleArgs a) {
  __shared__ uint64_t s_buf[kWaves][kCap];
  __shared__ uint32_t s_hist[kWaves][256];
  __shared__ uint32_t s_n[kWaves];
  __shared__ uint64_t s_greedy[kWaves];
  __shared__ double s_lm[kWaves];
  __shared__ double s_lz[kWaves];
  __shared__ int s_last;

  const uint32_t wave = threadIdx.x / kWave;
  const uint32_t lane = lane_id();
  const uint32_t row = blockIdx.x / a.chunks;
  const uint32_t chunk = blockIdx.x - row * a.chunks;
  const RowParams p = a.params[row];
  const bool greedy = p.temperature == 0.0f;
  const uint32_t L = a.logprobs;
  const uint32_t kk = greedy ? L : (p.top_k > L ? p.top_k : L);
  const bool pen = (p.flags & kRowPenalties) && a.counts != nullptr;
  const float t_eff = p.temperature > 0.0f ? p.temperature : 1.0f;
  const float log2e_over_t = 1.4426950408889634f / t_eff;

  const float* lrow = a.logits + static_cast<uint64_t>(row) * a.lstride;
  const uint32_t* crow = pen ? a.counts + static_cast<uint64_t>(row) * a.cstride : nullptr;
  float* prow = a.penalised ? a.penalised + static_cast<uint64_t>(row) * a.vocab : nullptr;

  const uint32_t wbegin = (chunk * kWaves + wave) * a.wave_elems;
  const uint32_t wend = min(wbegin + a.wave_elems, a.vocab);

  Cand c{s_buf[wave], s_hist[wave], 0u, 0xffffffffull, kk};
  uint64_t gbest = 0ull;
  float lm = -INFINITY;
  float lz = 0.0f;
  bool first = true;

  for (uint32_t base = wbegin; base < wend; base += kWave * 4 * kStepVec) {
    float v[kStepVec][4];
    uint32_t cnt[kStepVec][4];
#pragma unroll
    for (int j = 0; j < kStepVec; j++) {
      const uint32_t idx = base + (j * kWave + lane) * 4u;
      if (kVec && idx + 3u < wend) {
        const f4 x = __builtin_nontemporal_load(reinterpret_cast<const f4*>(lrow + idx));
        v[j][0] = x.x; v[j][1] = x.y; v[j][2] = x.z; v[j][3] = x.w;
        if (pen) {
          const u4 y = __builtin_nontemporal_load(reinterpret_cast<const u4*>(crow + idx));
          cnt[j][0] = y.x; cnt[j][1] = y.y; cnt[j][2] = y.z; cnt[j][3] = y.w;
        } else {
          cnt[j][0] = cnt[j][1] = cnt[j][2] = cnt[j][3] = 0u;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const uint32_t i = idx + e;
          const bool ok = i < wend;
          v[j][e] = ok ? lrow[i] : -INFINITY;
          cnt[j][e] = (pen && ok) ? crow[i] : 0u;
        }
      }
    }
    // Penalties, write-back (verification only), greedy and log-sum-exp.
    float step_max = -INFINITY;
    uint32_t lane_max_key = 0u;
#pragma unroll
    for (int j = 0; j < kStepVec; j++) {
      const uint32_t idx = base + (j * kWave + lane) * 4u;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t i = idx + e;
        const bool ok = i < wend;
        if (pen) v[j][e] = penalise(v[j][e], cnt[j][e], p.presence, p.frequency, p.repetition);
        if (prow && ok) prow[i] = v[j][e];
        if (greedy) {
          const uint64_t g = greedy_comp(v[j][e], ok ? i : kInvalidId);
          gbest = g > gbest ? g : gbest;
        }
        const uint32_t key = ok ? float_key(v[j][e]) : 0u;
        if (key) {
          step_max = fmaxf(step_max, v[j][e]);
          lane_max_key = key > lane_max_key ? key : lane_max_key;
        }
      }
    }
    if (L) {
      if (step_max > lm) {
        lz = (lm == -INFINITY) ? 0.0f : lz * exp2f((lm - step_max) * log2e_over_t);
        lm = step_max;
      }
#pragma unroll
      for (int j = 0; j < kStepVec; j++) {
        const uint32_t idx = base + (j * kWave + lane) * 4u;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const bool ok = idx + e < wend;
          if (ok && is_finite_bits(__float_as_uint(v[j][e])))
            lz += exp2f((v[j][e] - lm) * log2e_over_t);
        }
      }
    }
    if (kk) {
      if (first) {
        // The kk-th largest lane maximum: at least kk keys of this step are
        // >= it, so it bounds the wave's kk-th key from below.
        const uint32_t sorted = wave_sort_desc_u32(lane_max_key);
        const uint32_t T = __shfl(sorted, static_cast<int>(kk - 1u));
        const uint64_t R = T ? ((static_cast<uint64_t>(T) << 32) - 1ull) : 0xffffffffull;
        if (R > c.R) c.R = R;
        first = false;
      }
#pragma unroll
      for (int j = 0; j < kStepVec; j++) {
        const uint32_t idx = base + (j * kWave + lane) * 4u;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const uint32_t i = idx + e;
          const uint32_t key = i < wend ? float_key(v[j][e]) : 0u;
          cand_push(c, make_comp(key, i));
        }
      }
    }
  }

  // ---- workgroup merge ----
  if (kk) cand_reduce(c);
  if (lane == 0) s_n[wave] = c.n;
  if (greedy) {
    gbest = wave_max_u64(gbest);
    if (lane == 0) s_greedy[wave] = gbest;
  }
  if (L) {
    const double wm = wave_max_f64(static_cast<double>(lm));
    const double lzd = (lm == -INFINITY) ? 0.0
        : static_cast<double>(lz) * exp((static_cast<double>(lm) - wm) / t_eff);
    const double wz = wave_sum_f64(lzd);
    if (lane == 0) { s_lm[wave] = wm; s_lz[wave] = wz; }
  }
  __syncthreads();

  const uint64_t slot = static_cast<uint64_t>(row) * a.chunks + chunk;
  if (wave == 0) {
    if (kk) {
      uint32_t n = 0;
      const uint64_t mine = wave0_merge(s_buf, s_n, s_hist[0], kk, &n);
      a.cand[slot * kMaxK + lane] = mine;
      if (n == kk) {
        const uint64_t kth = __shfl(mine, static_cast<int>(kk - 1u));
        if (lane == 0) atomicMax(&a.row_thr[row], comp_key(kth));
      }
    }
    if (lane == 0) {
      if (greedy) {
        uint64_t g = s_greedy[0];
        for (int w = 1; w < kWaves; w++) g = s_greedy[w] > g ? s_greedy[w] : g;
        a.greedy[slot] = g;
      }
      if (L) {
        double m = s_lm[0];
        for (int w = 1; w < kWaves; w++) m = s_lm[w] > m ? s_lm[w] : m;
        double z = 0.0;
        if (m != -INFINITY)
          for (int w = 0; w < kWaves; w++)
            if (s_lm[w] != -INFINITY) z += s_lz[w] * exp((s_lm[w] - m) / t_eff);
        a.lse[slot * 2] = m;
        a.lse[slot * 2 + 1] = z;
      }
    }
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = atomicAdd(&a.row_done[row], 1u);
    s_last = (old == a.chunks - 1u);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  // ---- last workgroup of the row: merge the row ----
  const uint64_t row_slot = static_cast<uint64_t>(row) * a.chunks;
  uint64_t fin = 0ull;   // wave 0: lane i holds the i-th best composite (key order)
  uint32_t fin_n = 0;
  if (kk) {
    const uint32_t thr = __hip_atomic_load(&a.row_thr[row], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    Cand m{s_buf[wave], s_hist[wave], 0u,
           thr ? ((static_cast<uint64_t>(thr) << 32) - 1ull) : 0xffffffffull, kk};
    for (uint32_t ch = wave; ch < a.chunks; ch += kWaves) {
      const uint64_t* list = a.cand + (row_slot + ch) * kMaxK;
      const uint64_t x = lane < kk
          ? __hip_atomic_load(list + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
      cand_push(m, x);
    }
    cand_reduce(m);
    if (lane == 0) s_n[wave] = m.n;
    __syncthreads();
    if (wave == 0) fin = wave0_merge(s_buf, s_n, s_hist[0], kk, &fin_n);
  }
  if (wave != 0) return;

  int32_t status = kStOk;
  uint32_t token = kInvalidId;
  float token_logit = -INFINITY;

  if (greedy) {
    const uint64_t g = lane < a.chunks
        ? __hip_atomic_load(a.greedy + row_slot + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
        : 0ull;
    const uint64_t best = wave_max_u64(g);
    const uint32_t id = comp_id(best);
    float v = -INFINITY;
    if (best != 0ull && id < a.vocab) {
      v = lrow[id];
      if (pen) v = penalise(v, crow[id], p.presence, p.frequency, p.repetition);
    }
    if (best == 0ull || !is_finite_bits(__float_as_uint(v))) {
      status = pen ? kStFormat : kStMismatch;
      token_logit = v;
    } else {
      token = id;
      token_logit = v;
    }
  } else {
    // fg_sampler_select (src/sampler.c:80-122) over the exact top_k, in value
    // order, with parallel prefix sums in f64.
    const uint32_t topk = p.top_k;
    const uint64_t sel_comp = value_comp_from(lane < topk ? fin : 0ull);
    const uint64_t sorted = wave_sort_desc_u64(sel_comp);
    const uint32_t kept = static_cast<uint32_t>(__popcll(ballot(sorted != 0ull)));
    if (kept == 0u) {
      status = kStFormat;
    } else {
      const uint32_t limit = topk < kept ? topk : kept;
      const bool live = lane < limit;
      const float vf = live ? key_to_float(comp_key(sorted)) : 0.0f;
      const double v = static_cast<double>(vf);
      const double vmax = __shfl(v, 0);
      const double e = live ? exp(v - vmax) : 0.0;
      const double esum_inc = wave_prefix_sum_f64(e);
      const double sum = __shfl(esum_inc, static_cast<int>(limit - 1u));
      if (!(sum > 0.0) || !isfinite(sum)) {
        status = kStFormat;
      } else {
        const double q = e / sum;
        const double cum = wave_prefix_sum_f64(q);
        const uint64_t hit = ballot(live && cum >= static_cast<double>(p.top_p));
        const uint32_t cutoff = hit ? static_cast<uint32_t>(__builtin_ctzll(hit)) + 1u : limit;
        const double t = static_cast<double>(p.temperature);
        const double vmax_t = vmax / t;
        const double te = lane < cutoff ? exp(v / t - vmax_t) : 0.0;
        const double tcum = wave_prefix_sum_f64(te);
        const double tsum = __shfl(tcum, static_cast<int>(cutoff - 1u));
        if (!(tsum > 0.0) || !isfinite(tsum)) {
          status = kStFormat;
        } else {
          float u = a.uniforms[row];
          if (!is_finite_bits(__float_as_uint(u)) || u < 0.0f) u = 0.0f;
          if (u >= 1.0f) u = __uint_as_float(0x3f7fffffu);
          const double draw = static_cast<double>(u) * tsum;
          const uint64_t hit2 = ballot(lane < cutoff && draw < tcum);
          const uint32_t pick = hit2 ? static_cast<uint32_t>(__builtin_ctzll(hit2)) : cutoff - 1u;
          const uint64_t chosen = __shfl(sorted, static_cast<int>(pick));
          token = comp_id(chosen);
          // The logit keeps its sign of zero: take it from the key-order list.
          const uint64_t owner = ballot(fin != 0ull && comp_id(fin) == token);
          const uint64_t orig = __shfl(fin, static_cast<int>(__builtin_ctzll(owner)));
          token_logit = key_to_float(comp_key(orig));
        }
      }
    }
  }

  if (L) {
    // Log-probs of the first L of the kk candidates in value order.
    double m = -INFINITY;
    double z = 0.0;
    const double le = lane < a.chunks ? __hip_atomic_load(a.lse + (row_slot + lane) * 2,
                                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                      : -INFINITY;
    const double lzz = lane < a.chunks ? __hip_atomic_load(a.lse + (row_slot + lane) * 2 + 1,
                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                       : 0.0;
    m = wave_max_f64(le);
    const double te = static_cast<double>(t_eff);
    z = wave_sum_f64(le == -INFINITY ? 0.0 : lzz * exp((le - m) / te));
    const double lse = m / te + log(z);
    const uint64_t vs = wave_sort_desc_u64(value_comp_from(fin));
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
    __hip_atomic_store(&a.row_thr[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&a.row_done[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace fg
