// Q8_0 matrix-vector products over the cooked weight layout (the LM head):
// y[t][row] = scale * sum_b d(row, b) * sum_i q(row, b, i) * x[t][32b + i]
// (shaders/fg_dense_q8_0_cooked.comp; layout src/quant.c:68-96), and the same
// product fused with the greedy finalist of each token (src/output.c:320-344)
// so the logits need not round-trip through HBM.
//
// Cooked layout, per tile of 16 rows (tile_bytes, 64-byte aligned):
//   [0, quant_offset)            f16 scales, [block][tile_row]
//   [quant_offset, +16*in)       int8 quants, [tile_row][in]
// One wave owns a tile at a time.  Lane l takes the 16-byte chunks
// c = l, l + 64, ... of the in/16 chunks of a row and, for each chunk, the
// 16 rows of the tile: 16 coalesced 16-byte loads (1 KiB per instruction
// across the wave), the chunk's 16 inputs per token from LDS once, and the
// block's 16 scales (32 bytes).  Each lane accumulates d * (16-term dot) per
// row and token; a butterfly reduce-scatter over the wave (permlane swaps for
// strides 32 and 16, DPP below) then leaves lane l with row l/4's total.
// Every row's arithmetic is the same in the plain and the fused kernel, so a
// fused finalist carries exactly the value the plain kernel writes.
#pragma once

#include "fg_device.hpp"

namespace fg {

constexpr uint32_t kCookRows = 16;
constexpr uint32_t kDenseBlock = 256;                // 4 waves
constexpr uint32_t kDenseLdsFloats = 16384;          // staged inputs: in * tokens per pass

struct DenseArgs {
  const uint8_t* w;       // cooked tiles
  const float* x;         // [tokens][in]
  float* y;               // [tokens][rows] (plain) or NULL (fused, logits not kept)
  uint32_t in, rows, tokens, token0;  // this pass: tokens [token0, token0 + tokens)
  uint64_t tile_bytes, quant_offset;
  float scale;
  // fused finalist (src/output.c:320-344)
  uint32_t first_row;
  unsigned long long* keys;
  uint32_t* arrivals;
  float* values;
  uint32_t* ids;
  int32_t* status;
};

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

__device__ __forceinline__ float swap_add32(float a, float b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                   false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap_add16(float a, float b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                   false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// v[r] (r < 16) summed over the 64 lanes; lane l returns the total of row l/4.
__device__ __forceinline__ float wave_rows_total(float (&v)[kCookRows]) {
  // stride 32: lanes 32-63 keep rows 8-15; permlane32_swap(v[i], v[i+8])
  // returns, in every lane, its kept value and the partner's.
#pragma unroll
  for (int i = 0; i < 8; i++) v[i] = swap_add32(v[i], v[i + 8]);
#pragma unroll
  for (int i = 0; i < 4; i++) v[i] = swap_add16(v[i], v[i + 4]);
  const uint32_t lane = lane_id();
  const bool b3 = lane & 8u, b2 = lane & 4u;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const float keep = b3 ? v[i + 2] : v[i];
    const float send = b3 ? v[i] : v[i + 2];
    v[i] = keep + __uint_as_float(lane_xor<8>(__float_as_uint(send)));
  }
  {
    const float keep = b2 ? v[1] : v[0];
    const float send = b2 ? v[0] : v[1];
    v[0] = keep + __uint_as_float(lane_xor<4>(__float_as_uint(send)));
  }
  float t = v[0];
  t += __uint_as_float(lane_xor<2>(__float_as_uint(t)));
  t += __uint_as_float(lane_xor<1>(__float_as_uint(t)));
  return t;
}

// One wave's pass over one tile: out[t] = row (lane/4)'s scaled total for
// token t (t < B).  s_x holds B rows of `in` inputs.
template <int B>
__device__ __forceinline__ void tile_rows(const DenseArgs& a, uint64_t tile, const float* s_x,
                                          float (&out)[B]) {
  const uint8_t* base = a.w + tile * a.tile_bytes;
  const uint8_t* quants = base + a.quant_offset;
  const uint32_t chunks = a.in / 16u;
  const uint32_t lane = lane_id();
  float acc[B][kCookRows];
#pragma unroll
  for (int t = 0; t < B; t++)
#pragma unroll
    for (int r = 0; r < (int)kCookRows; r++) acc[t][r] = 0.0f;
  for (uint32_t c = lane; c < chunks; c += kWave) {
    u4 q[kCookRows];
#pragma unroll
    for (int r = 0; r < (int)kCookRows; r++)  // streamed once: non-temporal
      q[r] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(quants + static_cast<uint64_t>(r) * a.in + 16u * c));
    const u4 s0 = *reinterpret_cast<const u4*>(base + 32u * (c >> 1));
    const u4 s1 = *reinterpret_cast<const u4*>(base + 32u * (c >> 1) + 16u);
    float xs[B][16];
#pragma unroll
    for (int t = 0; t < B; t++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const f4 v = *reinterpret_cast<const f4*>(s_x + t * a.in + 16u * c + 4u * j);
        xs[t][4 * j] = v.x;
        xs[t][4 * j + 1] = v.y;
        xs[t][4 * j + 2] = v.z;
        xs[t][4 * j + 3] = v.w;
      }
    const uint32_t sw[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int r = 0; r < (int)kCookRows; r++) {
      const float d = f16_bits_to_f32((sw[r >> 1] >> (16 * (r & 1))) & 0xffffu);
      const uint32_t qw[4] = {q[r].x, q[r].y, q[r].z, q[r].w};
      float qf[16];
#pragma unroll
      for (int j = 0; j < 16; j++)
        qf[j] = static_cast<float>(static_cast<int32_t>(qw[j >> 2] << (24 - 8 * (j & 3))) >> 24);
#pragma unroll
      for (int t = 0; t < B; t++) {
        float dot = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) dot = __builtin_fmaf(qf[j], xs[t][j], dot);
        acc[t][r] = __builtin_fmaf(d, dot, acc[t][r]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < B; t++) out[t] = wave_rows_total(acc[t]) * a.scale;
}

template <int B>
__device__ __forceinline__ void stage_inputs(const DenseArgs& a, float* s_x) {
  const uint32_t n = a.in * B;
  for (uint32_t i = 4u * threadIdx.x; i < n; i += 4u * kDenseBlock) {
    const uint32_t t = i / a.in;
    f4 v = {0.f, 0.f, 0.f, 0.f};
    if (t < a.tokens)
      v = *reinterpret_cast<const f4*>(a.x + static_cast<uint64_t>(a.token0 + t) * a.in + (i - t * a.in));
    *reinterpret_cast<f4*>(s_x + i) = v;
  }
  __syncthreads();
}

// Grid: one tile per wave (wave g of the grid takes tile g; the loop covers
// any grid).
template <int B>
__global__ __launch_bounds__(kDenseBlock) void dense_q8_cooked_kernel(DenseArgs a) {
  extern __shared__ float s_x[];
  stage_inputs<B>(a, s_x);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint64_t tiles = (a.rows + kCookRows - 1u) / kCookRows;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * (kDenseBlock / kWave);
  const uint32_t r = lane_id() >> 2;
  for (uint64_t tile = static_cast<uint64_t>(blockIdx.x) * (kDenseBlock / kWave) + wave;
       tile < tiles; tile += stride) {
    float out[B];
    tile_rows<B>(a, tile, s_x, out);
    const uint64_t row = tile * kCookRows + r;
    if ((lane_id() & 3u) == 0u && row < a.rows) {
#pragma unroll
      for (int t = 0; t < B; t++)
        if (t < (int)a.tokens) a.y[static_cast<uint64_t>(a.token0 + t) * a.rows + row] = out[t];
    }
  }
}

// The same product fused with each token's greedy finalist over the rows
// (ids first_row + row): per wave a running best composite per token, then
// per workgroup, then an atomic max into keys[token]; the workgroup that
// arrives last for a token decodes it and returns keys/arrivals to zero.  A
// finalist whose value is non-finite or zero is recomputed from its tile (the
// composite keeps neither NaN payloads nor the sign of zero), bit for bit the
// value the plain kernel writes.  y, when non-NULL, also receives the logits.
template <int B>
__global__ __launch_bounds__(kDenseBlock) void dense_q8_finalist_kernel(DenseArgs a) {
  extern __shared__ float s_x[];
  __shared__ uint64_t s_best[kDenseBlock / kWave][B];
  __shared__ uint32_t s_last[B];
  stage_inputs<B>(a, s_x);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint64_t tiles = (a.rows + kCookRows - 1u) / kCookRows;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * (kDenseBlock / kWave);
  const uint32_t r = lane_id() >> 2;
  uint64_t best[B];
#pragma unroll
  for (int t = 0; t < B; t++) best[t] = 0ull;
  for (uint64_t tile = static_cast<uint64_t>(blockIdx.x) * (kDenseBlock / kWave) + wave;
       tile < tiles; tile += stride) {
    float out[B];
    tile_rows<B>(a, tile, s_x, out);
    const uint64_t row = tile * kCookRows + r;
    const bool live = (lane_id() & 3u) == 0u && row < a.rows;
#pragma unroll
    for (int t = 0; t < B; t++) {
      if (live) best[t] = max(best[t], greedy_comp(out[t], a.first_row + static_cast<uint32_t>(row)));
      if (a.y && live && t < (int)a.tokens)
        a.y[static_cast<uint64_t>(a.token0 + t) * a.rows + row] = out[t];
    }
  }
#pragma unroll
  for (int t = 0; t < B; t++) {
    const uint64_t m = wave_max_u64(best[t]);
    if (lane_id() == 0) s_best[wave][t] = m;
  }
  __syncthreads();
  if (threadIdx.x < static_cast<uint32_t>(B)) {
    const uint32_t t = threadIdx.x;
    uint64_t m = 0ull;
#pragma unroll
    for (uint32_t w = 0; w < kDenseBlock / kWave; w++) m = max(m, s_best[w][t]);
    uint32_t last = 0u;
    if (t < a.tokens) {
      const uint32_t tok = a.token0 + t;
      __hip_atomic_fetch_max(a.keys + tok, static_cast<unsigned long long>(m), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      wait_memory();  // hand-off ordering: see wait_memory()
      const uint32_t arrived =
          __hip_atomic_fetch_add(a.arrivals + tok, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = arrived + 1u == gridDim.x;
    }
    s_last[t] = last;
  }
  __syncthreads();
  // Workgroup-uniform from here: each token this workgroup closes.
  for (int t = 0; t < B; t++) {
    if (!s_last[t]) continue;
    const uint32_t tok = a.token0 + t;
    uint64_t k = 0ull;
    if (threadIdx.x == 0)
      k = __hip_atomic_exchange(a.keys + tok, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (threadIdx.x == 0) {
      __hip_atomic_store(a.arrivals + tok, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_best[0][t] = k;
    }
    __syncthreads();
    k = s_best[0][t];
    const uint32_t row = greedy_id(k) - a.first_row;
    const uint32_t hi = static_cast<uint32_t>(k >> 32);
    float v = key_to_float(hi);
    if (hi == 0xffffffffu || hi == 0x80000000u) {
      // Recompute the winner's tile with wave 0 (uniform branch per workgroup).
      if (wave == 0) {
        float out[B];
        tile_rows<B>(a, row / kCookRows, s_x, out);
        float mine = 0.0f;
#pragma unroll
        for (int u = 0; u < B; u++)
          if (u == t) mine = out[u];
        const float got = __uint_as_float(__builtin_amdgcn_readlane(
            static_cast<int>(__float_as_uint(mine)), static_cast<int>(4u * (row % kCookRows))));
        if (threadIdx.x == 0) s_best[1][t] = __float_as_uint(got);
      }
      __syncthreads();
      v = __uint_as_float(static_cast<uint32_t>(s_best[1][t]));
    }
    if (threadIdx.x == 0) {
      a.values[tok] = v;
      a.ids[tok] = a.first_row + row;
      a.status[tok] = is_finite_bits(__float_as_uint(v)) ? 0 : 5;  // FG_ERR_MISMATCH
    }
  }
}

}  // namespace fg
