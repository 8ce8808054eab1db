// Exact (erf) GELU, elementwise, fp32 / bf16 / fp16:
//
//   y = gelu(x) = x * Phi(x)     (Phi the standard normal CDF)
//
// computed in fp32 with gelu_exact() (Abramowitz & Stegun 7.1.26 erfc, the
// same code as the fused Linear + GELU epilogue) and rounded once to the
// storage type.  It stands in for the encoder's F.gelu(..., approximate=
// "none") on the FFN activation (reference transformer_opt/submission.py:507,
// benchmarks/torch_transformer_benchmark.py:95-97).
//
// HBM-bound: a lane moves 16-byte vectors (8 bf16/fp16 or 4 fp32 values),
// kUnroll of them per pass, all loads issued before any store.  One vector
// per lane (the most workgroups in flight) measured fastest over inputs that
// exceed the 256 MB MALL: bf16 [8192, 4096] 28.5 / 25.3 / 23.8 us and fp32
// [32768, 2048] 95.5 / 94.4 / 90.6 us with 4 / 2 / 1 vectors per lane.  Loads are
// non-temporal; stores are ordinary, because the next GEMM reads the result
// right away and should find it in the caches (non-temporal stores made the
// config-4 encoder 0.8 % slower).  y == x (in place) is allowed:
// every element is read and written by the same lane.  Buffers that are not
// 16-byte aligned take a one-element-per-lane kernel.
#include "ttk_common.h"

namespace ttk {
namespace {

constexpr int kGeluThreads = 256;
constexpr int kUnroll = 1;

__device__ __forceinline__ u32x4 gelu_vec(F32, u32x4 raw) {
  u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = __float_as_uint(gelu_exact(__uint_as_float(raw[i])));
  return out;
}
// 16-bit pairs: unpacked with shifts, rounded back two at a time by the
// hardware conversion (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32: round to nearest
// even, NaN stays NaN).
typedef __bf16 gbf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 gf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ unsigned pack2(BF16, float a, float b) {
  const gbf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(unsigned, v);
}
__device__ __forceinline__ unsigned pack2(F16, float a, float b) {
  const gf16x2 v = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
  return __builtin_bit_cast(unsigned, v);
}
template <typename T>
__device__ __forceinline__ u32x4 gelu_vec(T, u32x4 raw) {
  u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = to_f32(T{}, static_cast<unsigned short>(raw[i]));
    const float hi = to_f32(T{}, static_cast<unsigned short>(raw[i] >> 16));
    out[i] = pack2(T{}, gelu_exact(lo), gelu_exact(hi));
  }
  return out;
}

// Vectors [0, nvec) of 16 bytes; block b covers kGeluThreads * kUnroll of
// them, lane-consecutive within each of its kUnroll passes.
template <typename T>
__global__ __launch_bounds__(kGeluThreads) void gelu_vec_kernel(const u32x4* x, u32x4* y, int64_t nvec) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kGeluThreads * kUnroll) + threadIdx.x;
  u32x4 raw[kUnroll];
#pragma unroll
  for (int i = 0; i < kUnroll; ++i) {
    const int64_t v = base + static_cast<int64_t>(i) * kGeluThreads;
    raw[i] = v < nvec ? __builtin_nontemporal_load(x + v) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int i = 0; i < kUnroll; ++i) {
    const int64_t v = base + static_cast<int64_t>(i) * kGeluThreads;
    if (v < nvec) y[v] = gelu_vec(T{}, raw[i]);
  }
}

// One element per lane: elements [first, n).
template <typename T>
__global__ __launch_bounds__(kGeluThreads) void gelu_scalar_kernel(const typename T::storage* x,
                                                                   typename T::storage* y, int64_t first,
                                                                   int64_t n) {
  const int64_t i = first + static_cast<int64_t>(blockIdx.x) * kGeluThreads + threadIdx.x;
  if (i < n) y[i] = from_f32(T{}, gelu_exact(to_f32(T{}, x[i])));
}

template <typename T>
hipError_t launch_typed(const void* x, void* y, int64_t n, hipStream_t stream) {
  using St = typename T::storage;
  constexpr int kPerVec = 16 / T::kBytes;
  const bool aligned = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15u) == 0;
  const int64_t nvec = aligned ? n / kPerVec : 0;
  if (nvec > 0) {
    const int64_t per_block = static_cast<int64_t>(kGeluThreads) * kUnroll;
    const int64_t blocks = (nvec + per_block - 1) / per_block;
    gelu_vec_kernel<T><<<dim3(static_cast<unsigned>(blocks)), dim3(kGeluThreads), 0, stream>>>(
        static_cast<const u32x4*>(x), static_cast<u32x4*>(y), nvec);
  }
  const int64_t first = nvec * kPerVec;
  if (first < n) {
    const int64_t blocks = (n - first + kGeluThreads - 1) / kGeluThreads;
    gelu_scalar_kernel<T><<<dim3(static_cast<unsigned>(blocks)), dim3(kGeluThreads), 0, stream>>>(
        static_cast<const St*>(x), static_cast<St*>(y), first, n);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gelu(int dtype, const void* x, void* y, int64_t n, hipStream_t stream) {
  switch (dtype) {
    case 0: return launch_typed<F32>(x, y, n, stream);
    case 1: return launch_typed<BF16>(x, y, n, stream);
    case 2: return launch_typed<F16>(x, y, n, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ttk
