// Fused residual add + LayerNorm forward for gfx950.
//
// Semantics follow the reference kernel `_residual_layer_norm_fwd`
// (transformer_opt/kernels/residual_layer_norm.py:73-126): r = x + u, optional
// zeroing of invalid rows, store r, biased mean/variance of r in fp32,
// y = (r - mean) * rsqrt(var + eps) * w + b, optional zeroing, store y.
//
// The work is pure streaming (16 bytes of HBM traffic per fp32 element, no
// reuse), so the kernel is organised for bandwidth:
//  * every access is a 16-byte vector; consecutive lanes touch consecutive
//    16-byte chunks of a row, so each wave instruction moves whole 64-byte
//    segments;
//  * a row is owned by a group of `lanes_per_row` lanes of one wavefront
//    (8..64 lanes, several rows per wave for narrow rows), so no LDS and no
//    barrier is needed and every lane has several independent loads in flight;
//  * the row is held in registers between the statistics and the output pass
//    (one HBM read of x and u, one write of r and y);
//  * statistics: each lane computes the exact mean and centred sum of squares
//    of its own elements, then the lane group merges (mean, M2) pairs with
//    Chan's parallel-variance update over xor butterflies.  All partners merge
//    equal counts, so the update is mean = (ma + mb) / 2,
//    M2 = M2a + M2b + (mb - ma)^2 * n / 2, and every lane of the group ends
//    with bitwise-identical statistics.
// Rows whose width does not fit the register-resident form, or unaligned
// tensors, take a block-per-row fallback kernel with the same arithmetic.
#include "ttk_common.h"

namespace ttk {
namespace {

constexpr int kLnThreads = 256;

template <typename T>
struct Vec {
  static constexpr int N = 16 / T::kBytes;  // elements per 16-byte vector
};

__device__ __forceinline__ void unpack(F32, u32x4 raw, float (&o)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = __uint_as_float(raw[i]);
}
__device__ __forceinline__ void unpack(BF16, u32x4 raw, float (&o)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __uint_as_float(raw[i] << 16);
    o[2 * i + 1] = __uint_as_float(raw[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void unpack(F16, u32x4 raw, float (&o)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = to_f32(F16{}, static_cast<unsigned short>(raw[i] & 0xffffu));
    o[2 * i + 1] = to_f32(F16{}, static_cast<unsigned short>(raw[i] >> 16));
  }
}

__device__ __forceinline__ u32x4 pack(F32, const float (&v)[4]) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = __float_as_uint(v[i]);
  return r;
}
template <typename T>
__device__ __forceinline__ u32x4 pack(T tag, const float (&v)[8]) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = static_cast<unsigned int>(from_f32(tag, v[2 * i])) |
           (static_cast<unsigned int>(from_f32(tag, v[2 * i + 1])) << 16);
  }
  return r;
}

// Round an fp32 value to the storage type and back (identity for fp32): the
// residual is materialised in the tensor dtype before it is normalised.
template <typename T>
__device__ __forceinline__ float round_trip(float v) {
  if constexpr (T::kBytes == 4) {
    return v;
  } else {
    return to_f32(T{}, from_f32(T{}, v));
  }
}

// One wavefront handles `64 / lanes_per_row` consecutive rows (one row per
// lane group).  All loads of the group are straight-line code, issued back
// to back so they are in flight together: lanes past the last row read the
// last row instead (in bounds, never stored), and the presence of `u` is a
// kernel-wide template choice.  gamma/beta come in after the statistics, four
// vectors at a time, when the x/u registers are free again.
template <typename T, int VPL, bool HAS_U>
__device__ __forceinline__ void ln_rows(const LnParams& p) {
  constexpr int VN = Vec<T>::N;
  const int lane = threadIdx.x & 63;
  const int lpr = p.lanes_per_row;
  const int rows_per_wave = 64 / lpr;
  const int li = lane & (lpr - 1);
  const int64_t wave = static_cast<int64_t>(blockIdx.x) * (kLnThreads / 64) + (threadIdx.x >> 6);
  const int64_t row = wave * rows_per_wave + lane / lpr;
  if (wave * rows_per_wave >= p.rows) return;  // whole wavefront
  const bool active = row < p.rows;
  const int64_t lrow = active ? row : p.rows - 1;
  const int64_t vrow = p.N / VN;  // 16-byte vectors per row
  const int64_t base = row * vrow;

  const u32x4* __restrict__ xv = reinterpret_cast<const u32x4*>(p.x) + lrow * vrow;
  const u32x4* __restrict__ uv = HAS_U ? reinterpret_cast<const u32x4*>(p.u) + lrow * vrow : nullptr;
  const u32x4* __restrict__ wv = reinterpret_cast<const u32x4*>(p.w);
  const u32x4* __restrict__ bv = reinterpret_cast<const u32x4*>(p.b);

  u32x4 rawx[VPL], rawu[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    rawx[j] = __builtin_nontemporal_load(xv + j * lpr + li);
    if constexpr (HAS_U) rawu[j] = __builtin_nontemporal_load(uv + j * lpr + li);
  }
  const bool row_ok = p.valid == nullptr || p.valid[lrow] != 0;
  const bool zero_r = p.zero_res && !row_ok;

  float r[VPL][VN];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    float xf[VN];
    unpack(T{}, rawx[j], xf);
    if constexpr (HAS_U) {
      float uf[VN];
      unpack(T{}, rawu[j], uf);
#pragma unroll
      for (int i = 0; i < VN; ++i) r[j][i] = zero_r ? 0.0f : round_trip<T>(xf[i] + uf[i]);
    } else {
#pragma unroll
      for (int i = 0; i < VN; ++i) r[j][i] = zero_r ? 0.0f : xf[i];
    }
  }

  if (p.r_out != nullptr && active) {
    u32x4* __restrict__ ro = reinterpret_cast<u32x4*>(p.r_out) + base;
#pragma unroll
    for (int j = 0; j < VPL; ++j) __builtin_nontemporal_store(pack(T{}, r[j]), ro + j * lpr + li);
  }

  // Per-lane exact statistics of VPL*VN values.
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j)
#pragma unroll
    for (int i = 0; i < VN; ++i) sum += r[j][i];
  constexpr float kLaneCount = static_cast<float>(VPL * VN);
  float mean = sum * (1.0f / kLaneCount);
  float m2 = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j)
#pragma unroll
    for (int i = 0; i < VN; ++i) {
      const float d = r[j][i] - mean;
      m2 = __builtin_fmaf(d, d, m2);
    }
  // Chan merge across the lane group (equal counts on both sides).
  float half_count = 0.5f * kLaneCount;
  for (int off = 1; off < lpr; off <<= 1) {
    const float mo = __shfl_xor(mean, off);
    const float m2o = __shfl_xor(m2, off);
    const float delta = mo - mean;
    m2 = (m2 + m2o) + delta * delta * half_count;
    mean = 0.5f * (mean + mo);
    half_count *= 2.0f;
  }
  const float var = m2 / static_cast<float>(p.N);
  const float rstd = rsqrtf(var + p.eps);
  const bool zero_y = p.zero_norm && !row_ok;

  if (!active) return;
  u32x4* __restrict__ yo = reinterpret_cast<u32x4*>(p.y_out) + base;
#pragma unroll
  for (int j0 = 0; j0 < VPL; j0 += 4) {
    u32x4 cw[4], cb[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      if (j0 + jj < VPL) {
        cw[jj] = wv[(j0 + jj) * lpr + li];
        cb[jj] = bv != nullptr ? bv[(j0 + jj) * lpr + li] : u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = j0 + jj;
      if (j < VPL) {
        float wf[VN], bf[VN], y[VN];
        unpack(T{}, cw[jj], wf);
        unpack(T{}, cb[jj], bf);
#pragma unroll
        for (int i = 0; i < VN; ++i) {
          const float n = (r[j][i] - mean) * rstd;
          y[i] = zero_y ? 0.0f : __builtin_fmaf(n, wf[i], bf[i]);
        }
        __builtin_nontemporal_store(pack(T{}, y), yo + j * lpr + li);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <typename T, int VPL>
__global__ __launch_bounds__(kLnThreads) void residual_ln_vec_kernel(LnParams p) {
  if (p.u != nullptr) {
    ln_rows<T, VPL, true>(p);
  } else {
    ln_rows<T, VPL, false>(p);
  }
}

// Block-wide sum over 256 threads (4 wavefronts).
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // `red` may still be read by a previous reduction
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// Fallback: one 256-thread block per row, scalar accesses, three passes over
// the row (the row stays in L2 between passes).  Same arithmetic as above
// except that the mean and M2 are two block-wide sums.
template <typename T>
__global__ __launch_bounds__(kLnThreads) void residual_ln_generic_kernel(LnParams p) {
  using St = typename T::storage;
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int N = p.N;
  const St* __restrict__ x = static_cast<const St*>(p.x) + row * N;
  const St* __restrict__ u = p.u ? static_cast<const St*>(p.u) + row * N : nullptr;
  const St* __restrict__ w = static_cast<const St*>(p.w);
  const St* __restrict__ b = static_cast<const St*>(p.b);
  const bool row_ok = p.valid == nullptr || p.valid[row] != 0;
  const bool zero_r = p.zero_res && !row_ok;

  auto residual = [&](int c) -> float {
    if (zero_r) return 0.0f;
    const float xf = to_f32(T{}, x[c]);
    return u ? round_trip<T>(xf + to_f32(T{}, u[c])) : xf;
  };

  float s = 0.0f;
  for (int c = threadIdx.x; c < N; c += kLnThreads) {
    const float r = residual(c);
    if (p.r_out) static_cast<St*>(p.r_out)[row * N + c] = static_cast<St>(from_f32(T{}, r));
    s += r;
  }
  const float mean = block_sum(s, red) / static_cast<float>(N);
  float m2 = 0.0f;
  for (int c = threadIdx.x; c < N; c += kLnThreads) {
    const float d = residual(c) - mean;
    m2 = __builtin_fmaf(d, d, m2);
  }
  const float var = block_sum(m2, red) / static_cast<float>(N);
  const float rstd = rsqrtf(var + p.eps);
  const bool zero_y = p.zero_norm && !row_ok;
  St* __restrict__ y = static_cast<St*>(p.y_out) + row * N;
  for (int c = threadIdx.x; c < N; c += kLnThreads) {
    const float n = (residual(c) - mean) * rstd;
    const float bf = b ? to_f32(T{}, b[c]) : 0.0f;
    const float v = zero_y ? 0.0f : __builtin_fmaf(n, to_f32(T{}, w[c]), bf);
    y[c] = static_cast<St>(from_f32(T{}, v));
  }
}

template <typename T, int VPL>
hipError_t launch_vec(const LnParams& p, hipStream_t stream) {
  const int64_t rows_per_wave = 64 / p.lanes_per_row;
  const int64_t waves = (p.rows + rows_per_wave - 1) / rows_per_wave;
  const int64_t blocks = (waves + 3) / 4;
  residual_ln_vec_kernel<T, VPL><<<dim3(static_cast<unsigned>(blocks)), dim3(kLnThreads), 0, stream>>>(p);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_typed(const LnParams& p, bool vector_path, int vpl, hipStream_t stream) {
  if (!vector_path) {
    residual_ln_generic_kernel<T><<<dim3(static_cast<unsigned>(p.rows)), dim3(kLnThreads), 0, stream>>>(p);
    return hipGetLastError();
  }
  switch (vpl) {
    case 1: return launch_vec<T, 1>(p, stream);
    case 2: return launch_vec<T, 2>(p, stream);
    case 3: return launch_vec<T, 3>(p, stream);
    case 4: return launch_vec<T, 4>(p, stream);
    case 5: return launch_vec<T, 5>(p, stream);
    case 6: return launch_vec<T, 6>(p, stream);
    case 7: return launch_vec<T, 7>(p, stream);
    case 8: return launch_vec<T, 8>(p, stream);
    case 9: return launch_vec<T, 9>(p, stream);
    case 10: return launch_vec<T, 10>(p, stream);
    case 11: return launch_vec<T, 11>(p, stream);
    case 12: return launch_vec<T, 12>(p, stream);
    case 13: return launch_vec<T, 13>(p, stream);
    case 14: return launch_vec<T, 14>(p, stream);
    case 15: return launch_vec<T, 15>(p, stream);
    case 16: return launch_vec<T, 16>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_residual_layernorm(int dtype, const LnParams& p, bool vector_path,
                                     int vectors_per_lane, hipStream_t stream) {
  switch (dtype) {
    case 0: return launch_typed<F32>(p, vector_path, vectors_per_lane, stream);
    case 1: return launch_typed<BF16>(p, vector_path, vectors_per_lane, stream);
    case 2: return launch_typed<F16>(p, vector_path, vectors_per_lane, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ttk
