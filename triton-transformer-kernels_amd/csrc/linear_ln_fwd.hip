// Linear + residual add + LayerNorm forward for gfx950 (MI355X), bf16 / fp16,
// one kernel for the reference's
//
//   attn_out = F.linear(a, W, bias)                 (rounded to T)
//   r = x + attn_out                                (rounded to T)
//   y = LayerNorm(r) * gamma + beta                 (rounded to T)
//
// - the attention output projection followed by the fused residual +
// LayerNorm (transformer_opt/submission.py:497-505 and :457-479, with the
// kernel of transformer_opt/kernels/residual_layer_norm.py:73-126), at the
// reference's dtype boundaries: the projection is rounded to T before the
// residual add, the sum is rounded to T (it is the residual output) and the
// statistics are those of the rounded sum.  Width N = 1024.
//
// Design (one workgroup = 8 wavefronts, two per SIMD):
// * A LayerNorm row needs all 1024 features, so the projection is tiled by
//   row blocks: workgroups 2b and 2b + 1 compute tokens 64b .. 64b + 63, the
//   first features 0 .. 511, the second 512 .. 1023.  Each wavefront owns 64
//   features x 64 tokens: 2 x 2 v_mfma_f32_32x32x16 tiles (C^T = W . A^T, so
//   a lane ends holding one token and 4 consecutive features per register
//   group), 64 fp32 accumulators.  Workgroups are dealt round-robin to the 8
//   XCDs, so each XCD runs one feature half and streams half of W.
// * K advances 64 at a time.  W comes straight from global memory into a
//   two-stage register ring, pre-packed in MFMA fragment order (fragment
//   (feature block fb, k-step q) is 1 KB: lane 32h + r32 holds
//   W[32 fb + r32][16 q + 8h .. + 7]), one 1 KB load per fragment.  The 64
//   token rows of a stage are loaded into registers one stage ahead and
//   written to a 2-deep LDS ring (8 KB per stage, 16-byte chunks XOR-swizzled
//   by row), one barrier per stage.
// * Epilogue: bias, rounding, one v_permlane32_swap per dword (a lane then
//   holds 8 consecutive features of one token), the residual add with x and
//   its rounding, r stored.  Each workgroup then forms the statistics of its
//   half of every row (sum S and centred sum of squares M2) and publishes
//   them (system-scope atomic stores; the two halves run on different XCDs,
//   whose L2 caches are not coherent), then an agent-scope release fence
//   (L2 write-back and the wait for it, the memory model's release) orders
//   them before the workgroup counts itself in on its row block's counter.
//   Once both are in, each merges the two halves' statistics and writes y
//   for its own half.  The first of a pair polls for the second a
//   bounded number of times; if the second does not come, the first makes
//   its r visible (a release fence) and hands its half over (a
//   compare-and-swap on the counter), and the second then normalises both
//   halves, reading that r after an acquire fence.  Every wait ends, so no
//   co-residency is assumed.
// * Statistics in fp32 over the rounded r: per half S and M2 about S / 512,
//   merged as mean = (S0 + S1) / 1024, M2 = M2_0 + M2_1 + (S1/512 - S0/512)^2
//   * 256 (Chan et al.'s pairwise update), always half 0 first, so both
//   workgroups of a pair compute the same statistics whichever arrives
//   second; biased variance, rsqrt(var + eps), y = fma((r - mean) * rstd,
//   gamma, beta).
// Rows past M: the loads of a past row read the last row, stores outside
// the buffer resources are dropped, and coherent loads outside them read
// zeros.
#include <algorithm>
#include <type_traits>

#include "ttk_common.h"

namespace ttk {
namespace {

constexpr int kLlnN = 1024;            // features (LayerNorm width)
constexpr int kLlnHalf = kLlnN / 2;    // features per workgroup
constexpr int kLlnTokens = 64;         // tokens per workgroup
constexpr int kLlnWaves = 8;
constexpr int kLlnBK = 64;             // k per stage
constexpr int kLlnStageBytes = kLlnTokens * kLlnBK * 2;
constexpr int kLlnCoherent = 17;       // sc0 | sc1: system-coherent access

typedef __bf16 llbf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 llf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x16 llmfma(BF16, u16x8 a, u16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 llmfma(F16, u16x8 a, u16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ unsigned llpack(BF16, float a, float b) {
  const llbf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(unsigned, v);
}
__device__ __forceinline__ unsigned llpack(F16, float a, float b) {
  const llf16x2 v = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
  return __builtin_bit_cast(unsigned, v);
}
template <typename T>
__device__ __forceinline__ float lo_f32(unsigned d) {
  return to_f32(T{}, static_cast<unsigned short>(d));
}
template <typename T>
__device__ __forceinline__ float hi_f32(unsigned d) {
  return to_f32(T{}, static_cast<unsigned short>(d >> 16));
}

template <typename T, bool BIAS, bool LNB>
__global__ __launch_bounds__(64 * kLlnWaves) void linear_ln_kernel(LinearLnParams p) {
  __shared__ __attribute__((aligned(1024))) unsigned char xs[2][kLlnStageBytes];
  __shared__ float red[2][32][kLlnWaves];  // [token block][token][wave]
  __shared__ int sync_word[3];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31;
  const int h = lane >> 5;
  const int rb = static_cast<int>(blockIdx.x) >> 1;
  const int half = static_cast<int>(blockIdx.x) & 1;
  const int m0 = rb * kLlnTokens;
  const int NS = p.K / kLlnBK;
  const int fb0 = half * (kLlnN / 64) + 2 * wave;  // first 32-feature block of this wavefront

  // ---- main loop ------------------------------------------------------------
  const char* wp0 = static_cast<const char*>(p.wp) + static_cast<size_t>(fb0) * NS * 4096 + lane * 16;
  const char* wp1 = wp0 + static_cast<size_t>(NS) * 4096;
  // Stage copy: wavefront w moves token rows 8w .. 8w + 7, 8 lanes per
  // 128-byte row; chunk c of row q is stored at c ^ ((q >> 1) & 7).
  const int arow = wave * 8 + (lane >> 3);
  const char* ag = static_cast<const char*>(p.a) +
                   static_cast<size_t>(min(m0 + arow, p.M - 1)) * p.lda * 2 + 16 * (lane & 7);
  const int aw_off = arow * 128 + 16 * ((lane & 7) ^ ((arow >> 1) & 7));
  const int swz = (r32 >> 1) & 7;
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
  u16x8 wb[2][2][4], areg;
  auto loadw = [&](int s, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < 4; ++t) wb[buf][0][t] = *reinterpret_cast<const u16x8*>(wp0 + s * 4096 + 1024 * t);
#pragma unroll
    for (int t = 0; t < 4; ++t) wb[buf][1][t] = *reinterpret_cast<const u16x8*>(wp1 + s * 4096 + 1024 * t);
  };
  auto loada = [&](int s) __attribute__((always_inline)) {
    areg = *reinterpret_cast<const u16x8*>(ag + s * (kLlnBK * 2));
  };
  auto publish = [&](int buf) __attribute__((always_inline)) {
    *reinterpret_cast<u16x8*>(&xs[buf][aw_off]) = areg;
    __syncthreads();
  };
  auto compute = [&](int buf) __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      u16x8 af[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        af[j] = *reinterpret_cast<const u16x8*>(&xs[buf][(32 * j + r32) * 128 + 16 * ((2 * t + h) ^ swz)]);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = llmfma(T{}, wb[buf][i][t], af[j], acc[i][j]);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  loadw(0, 0);
  loada(0);
  __builtin_amdgcn_sched_barrier(0);
  publish(0);
  for (int s0 = 0; s0 < NS; s0 += 2) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int s = s0 + u;
      loada(min(s + 1, NS - 1));
      loadw(min(s + 1, NS - 1), u ^ 1);
      compute(u);
      publish(u ^ 1);
    }
  }

  // ---- epilogue: linear output, residual, r ---------------------------------
  // Chunk (i, j, gp) of a lane: token m0 + 32j + r32, features
  // 32 (fb0 + i) + 16 gp + 8h .. + 7 (after the swap).
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p.x), static_cast<short>(0), static_cast<int>(p.x_bytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t rr =
      __builtin_amdgcn_make_buffer_rsrc(p.r, static_cast<short>(0), static_cast<int>(p.r_bytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t yr =
      __builtin_amdgcn_make_buffer_rsrc(p.y, static_cast<short>(0), static_cast<int>(p.y_bytes), 0x00020000);
  auto offset = [&](int j, int f, int64_t ld) __attribute__((always_inline)) -> int {
    const int m = m0 + 32 * j + r32;
    return m < p.M ? static_cast<int>(static_cast<unsigned>(m) * static_cast<unsigned>(ld) * 2u + static_cast<unsigned>(f) * 2u)
                   : static_cast<int>(0x80000000u);
  };
  auto feature = [&](int which_half, int i, int gp) __attribute__((always_inline)) -> int {
    return 32 * (which_half * (kLlnN / 64) + 2 * wave + i) + 16 * gp + 8 * h;
  };
  u32x4 xin[2][2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int gp = 0; gp < 2; ++gp)
        xin[i][j][gp] = __builtin_amdgcn_raw_buffer_load_b128(xr, offset(j, feature(half, i, gp), p.ldx), 0, 0);
  u32x4 rown[2][2][2];  // r of this half, packed T
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float bq[4][4];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        bq[g][e] = BIAS ? to_f32(T{}, static_cast<const unsigned short*>(p.bias)[32 * (fb0 + i) + 8 * g + 4 * h + e])
                        : 0.0f;
      }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      unsigned o[4][2];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = BIAS ? acc[i][j][4 * g + e] + bq[g][e] : acc[i][j][4 * g + e];
        o[g][0] = llpack(T{}, v[0], v[1]);
        o[g][1] = llpack(T{}, v[2], v[3]);
      }
#pragma unroll
      for (int gp = 0; gp < 2; ++gp) {
        const auto s0 = __builtin_amdgcn_permlane32_swap(o[2 * gp][0], o[2 * gp + 1][0], false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(o[2 * gp][1], o[2 * gp + 1][1], false, false);
        const unsigned lin[4] = {s0[0], s1[0], s0[1], s1[1]};
        const u32x4 xv = xin[i][j][gp];
        u32x4 rv;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          rv[d] = llpack(T{}, lo_f32<T>(xv[d]) + lo_f32<T>(lin[d]), hi_f32<T>(xv[d]) + hi_f32<T>(lin[d]));
        }
        rown[i][j][gp] = rv;
        __builtin_amdgcn_raw_buffer_store_b128(rv, rr, offset(j, feature(half, i, gp), p.ldr), 0, 0);
      }
    }
  }

  // ---- statistics of this half ------------------------------------------------
  // Per token: the lane's 32 values in (i, gp, d) order, the two lane halves,
  // then the 8 wavefronts in order: the sum S, then the centred sum of
  // squares M2 about S / 512.
  auto token_total = [&](const float (&part)[2], float (&tot)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float v = part[j] + __shfl_xor(part[j], 32);
      if (h == 0) red[j][r32][wave] = v;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float t = 0.0f;
#pragma unroll
      for (int w = 0; w < kLlnWaves; ++w) t += red[j][r32][w];
      tot[j] = t;
    }
    __syncthreads();
  };
  float part[2], own_s[2], own_m2[2], own_mean[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int gp = 0; gp < 2; ++gp)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          t += lo_f32<T>(rown[i][j][gp][d]);
          t += hi_f32<T>(rown[i][j][gp][d]);
        }
    part[j] = t;
  }
  token_total(part, own_s);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    own_mean[j] = own_s[j] * (1.0f / kLlnHalf);
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int gp = 0; gp < 2; ++gp)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const float a = lo_f32<T>(rown[i][j][gp][d]) - own_mean[j];
          const float b = hi_f32<T>(rown[i][j][gp][d]) - own_mean[j];
          t = __builtin_fmaf(a, a, t);
          t = __builtin_fmaf(b, b, t);
        }
    part[j] = t;
  }
  token_total(part, own_m2);
  // Published for the other workgroup of the pair: (S, M2) of token
  // 32j + r32 at stats[((rb * 2 + half) * 2 + j) * 64 + 2 * r32 + {0, 1}].
  float* const stats_rb = p.stats + static_cast<int64_t>(rb) * 256;
  if (wave == 0) {
    if (h == 0) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float* st = stats_rb + (half * 2 + j) * 64 + 2 * r32;
        __hip_atomic_store(st, own_s[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(st + 1, own_m2[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
    }
    // The release that orders the statistics before the count-in below
    // (agent scope: L2 write-back, then the wait for it).
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  }

  // ---- pair hand-shake ----------------------------------------------------------
  // Counter states: 0 nobody, 1 first arrived, 2 both arrived, 3 the first
  // handed its half over, 4 the second took it.  The first polls (at most
  // max_polls times) for state 2; if it does not come, it releases its r and
  // swaps 1 -> 3, and the second, finding 3, normalises both halves.
  // Whoever uses the counter last clears it.
  __syncthreads();
  int* const counter = &p.counters[rb];
  // Each hand-shake word is written once by thread 0 and read by every
  // thread only after the barrier that follows the write.
  if (tid == 0) sync_word[0] = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  __syncthreads();
  const int arrived = sync_word[0];
  bool both_halves = false;
  if (arrived == 0) {
    if (tid == 0) {
      int state = 1;
      for (int n = 0; n < p.max_polls && state == 1; ++n) {
        __builtin_amdgcn_s_sleep(2);
        state = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
      sync_word[1] = state;
    }
    __syncthreads();
    if (sync_word[1] == 1) {
      // Hand over.  r of this half went out with ordinary stores and may
      // sit in this XCD's L2: a release fence (L2 write-back, then the wait
      // for it) in every wavefront makes it visible before the swap that
      // hands it over.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      __syncthreads();
      if (tid == 0) {
        int expected = 1;
        const bool handed = __hip_atomic_compare_exchange_strong(counter, &expected, 3, __ATOMIC_RELAXED,
                                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        sync_word[2] = handed ? 3 : expected;
      }
      __syncthreads();
      if (sync_word[2] == 3) return;  // the second workgroup normalises this half
    }
    // Both here: the second's count-in was its last use of the counter.
    if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  } else if (arrived == 3) {
    both_halves = true;
    if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }

  // ---- row statistics: both halves merged in half order --------------------------
  const int other = half ^ 1;
  float mean[2], rstd[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float* st = stats_rb + (other * 2 + j) * 64 + 2 * r32;
    const float oth_s = __hip_atomic_load(st, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const float oth_m2 = __hip_atomic_load(st + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const float s0 = half == 0 ? own_s[j] : oth_s, s1 = half == 0 ? oth_s : own_s[j];
    const float q0 = half == 0 ? own_m2[j] : oth_m2, q1 = half == 0 ? oth_m2 : own_m2[j];
    const float delta = s1 * (1.0f / kLlnHalf) - s0 * (1.0f / kLlnHalf);
    const float m2 = (q0 + q1) + delta * delta * (kLlnHalf / 2.0f);
    mean[j] = (s0 + s1) * (1.0f / kLlnN);
    rstd[j] = rsqrtf(m2 * (1.0f / kLlnN) + p.eps);
  }

  // ---- y ---------------------------------------------------------------------------
  auto normalise = [&](const u32x4 (&v)[2][2][2], int which_half) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int gp = 0; gp < 2; ++gp) {
        const int f = feature(which_half, i, gp);
        const u32x4 gw = *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.gamma) + 2 * f);
        const u32x4 gb = LNB ? *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.beta) + 2 * f)
                             : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          u32x4 yv;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const float na = (lo_f32<T>(v[i][j][gp][d]) - mean[j]) * rstd[j];
            const float nb = (hi_f32<T>(v[i][j][gp][d]) - mean[j]) * rstd[j];
            yv[d] = llpack(T{}, __builtin_fmaf(na, lo_f32<T>(gw[d]), lo_f32<T>(gb[d])),
                           __builtin_fmaf(nb, hi_f32<T>(gw[d]), hi_f32<T>(gb[d])));
          }
          __builtin_amdgcn_raw_buffer_store_b128(yv, yr, offset(j, f, p.ldy), 0, 0);
        }
      }
  };
  normalise(rown, half);
  if (both_halves) {
    // The other half's r: an acquire fence (this XCD's L2 invalidated)
    // pairs with the other workgroup's release before it is read.
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    u32x4 roth[2][2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int gp = 0; gp < 2; ++gp)
          roth[i][j][gp] = __builtin_amdgcn_raw_buffer_load_b128(rr, offset(j, feature(other, i, gp), p.ldr), 0,
                                                                 kLlnCoherent);
    normalise(roth, other);
  }
}

template <typename T>
hipError_t launch_ln_typed(LinearLnParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(2 * ((p.M + kLlnTokens - 1) / kLlnTokens)));
  const dim3 block(64 * kLlnWaves);
  if (p.bias) {
    if (p.beta) {
      linear_ln_kernel<T, true, true><<<grid, block, 0, stream>>>(p);
    } else {
      linear_ln_kernel<T, true, false><<<grid, block, 0, stream>>>(p);
    }
  } else if (p.beta) {
    linear_ln_kernel<T, false, true><<<grid, block, 0, stream>>>(p);
  } else {
    linear_ln_kernel<T, false, false><<<grid, block, 0, stream>>>(p);
  }
  return hipGetLastError();
}

// Packs W [N, K] (row stride ldw) into MFMA fragment order: 16-byte chunk
// (fb * (K/16) + q) * 64 + l of the output is W[32 fb + l % 32][16 q + 8 (l / 32) .. + 7].
__global__ __launch_bounds__(256) void pack_weight_kernel(const unsigned char* w, unsigned char* wp,
                                                          int N, int K, int64_t ldw) {
  const int64_t chunks = static_cast<int64_t>(N) * K / 8;
  const int kq = K / 16;
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; c < chunks;
       c += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int l = static_cast<int>(c & 63);
    const int64_t frag = c >> 6;
    const int q = static_cast<int>(frag % kq);
    const int fb = static_cast<int>(frag / kq);
    const int64_t n = 32 * static_cast<int64_t>(fb) + (l & 31);
    const int64_t k = 16 * static_cast<int64_t>(q) + 8 * (l >> 5);
    *reinterpret_cast<u32x4*>(wp + 16 * c) = *reinterpret_cast<const u32x4*>(w + 2 * (n * ldw + k));
  }
}

}  // namespace

hipError_t launch_linear_ln(int dtype, LinearLnParams& p, hipStream_t stream) {
  switch (dtype) {
    case 1: return launch_ln_typed<BF16>(p, stream);
    case 2: return launch_ln_typed<F16>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_pack_weight(const void* w, void* wp, int N, int K, int64_t ldw, hipStream_t stream) {
  const int64_t chunks = static_cast<int64_t>(N) * K / 8;
  const int64_t blocks = std::min<int64_t>((chunks + 255) / 256, 4096);
  pack_weight_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(
      static_cast<const unsigned char*>(w), static_cast<unsigned char*>(wp), N, K, ldw);
  return hipGetLastError();
}

}  // namespace ttk
