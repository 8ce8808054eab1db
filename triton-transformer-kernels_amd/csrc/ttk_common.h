// Shared definitions of the gfx950 kernels and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace ttk {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Storage tags.  Device code moves 16-bit types as raw ushort bits and
// converts explicitly, so the numerics never depend on header operators.
struct F32 {
  using storage = float;
  static constexpr int kBytes = 4;
};
struct BF16 {
  using storage = unsigned short;
  static constexpr int kBytes = 2;
};
struct F16 {
  using storage = unsigned short;
  static constexpr int kBytes = 2;
};

__device__ __forceinline__ float to_f32(F32, float v) { return v; }
__device__ __forceinline__ float to_f32(BF16, unsigned short v) {
  return __uint_as_float(static_cast<unsigned int>(v) << 16);
}
__device__ __forceinline__ float to_f32(F16, unsigned short v) {
  _Float16 h = __builtin_bit_cast(_Float16, v);
  return static_cast<float>(h);
}

__device__ __forceinline__ float from_f32(F32, float v) { return v; }
// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN), the rounding torch uses:
// the gfx950 conversion instruction (v_cvt_pk_bf16_f32).
__device__ __forceinline__ unsigned short from_f32(BF16, float v) {
  return __builtin_bit_cast(unsigned short, static_cast<__bf16>(v));
}
__device__ __forceinline__ unsigned short from_f32(F16, float v) {
  _Float16 h = static_cast<_Float16>(v);  // v_cvt_f16_f32: round to nearest even
  return __builtin_bit_cast(unsigned short, h);
}

// gelu(v) = v * Phi(v), Phi the standard normal CDF, with
// Phi(v) = 1 - h(|v|) (v >= 0) or h(|v|) (v < 0), h(a) = erfc(a / sqrt(2)) / 2,
// and erfc(x) = t*(a1 + t*(a2 + t*(a3 + t*(a4 + t*a5)))) * exp(-x^2),
// t = 1/(1 + p*x): Abramowitz & Stegun, Handbook of Mathematical Functions,
// 7.1.26 (after Hastings), |error| <= 1.5e-7 on erf - far below the bf16 /
// fp16 rounding of the result.  With x = |v|/sqrt(2) the factor 1/2, the
// 1/sqrt(2) and log2(e) fold into the constants: t = 1/(1 + (p/sqrt2)|v|),
// h = t * (a1/2 + ... ) * 2^(-v^2 log2(e) / 2).  v * (1 - h) keeps
// gelu(+inf) = +inf and NaN in, NaN out.
__device__ __forceinline__ float gelu_exact(float v) {
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(fabsf(v), 0.23164188826636040f, 1.0f));
  float q = __builtin_fmaf(t, 0.5307027145f, -0.7265760135f);
  q = __builtin_fmaf(t, q, 0.7107068705f);
  q = __builtin_fmaf(t, q, -0.142248368f);
  q = __builtin_fmaf(t, q, 0.127414796f);
  const float e = __builtin_amdgcn_exp2f((v * v) * -0.72134752044448170f);
  const float te = t * e;
  const float phi = v >= 0.0f ? __builtin_fmaf(-te, q, 1.0f) : te * q;
  return v * phi;
}

// Launch parameters of the attention kernels (element strides).
struct AttnParams {
  const void* q;
  const void* k;
  const void* v;
  const uint8_t* mask;
  void* out;
  int64_t qb, qs, qh;
  int64_t kb, ks, kh;
  int64_t vb, vs, vh;
  int64_t mb, ms;
  int64_t ob, os, oh;
  int S, H, BH, nq;
  float scale_log2;  // softmax scale * log2(e)
  int xcd_swizzle;   // 1 when BH % 8 == 0: heads are pinned to XCDs
  int pair;          // causal: a workgroup runs query tiles nq-1-i and i
  int units;         // workgroups per (batch, head)
  int cu_count;      // compute units of the device (wave-priority phase)
  int twin;          // fp32, S <= 64: two (batch, head) pairs per workgroup
  int fold;          // causal, one resident round: heavy/light query-tile order
  // Key-split causal grid (16-bit): query tiles heavier than the average
  // workgroup slot are split into chunks of key tiles; unit u of a (batch,
  // head) runs query tile unit_tab[u] & 1023, chunk (unit_tab[u] >> 10) & 7
  // of ((unit_tab[u] >> 13) + 1).  Chunks of query tiles >= split_q0 leave
  // their partial state in ws_part and count themselves in ws_cnt; the last
  // one to arrive merges the partials and writes the rows.  Both are indexed
  // by the split slot bh * split_tiles + (query tile - split_q0).
  int split;
  int split_q0;
  int split_tiles;   // nq - split_q0
  int split_maxch;   // chunks of the heaviest query tile
  int* ws_cnt;       // [kSplitCounterSlots] arrival counters, zero between launches
  float* ws_part;    // [BH * split_tiles * split_maxch * 4 waves * lanes * state]
  unsigned short unit_tab[256];
};
constexpr int kMaxSplitUnits = 256;
// The key-split workspace starts with a counter block of fixed size, the
// same for every shape, so a launch never finds another launch's partial
// states where its counters are: the block is zero before the first launch
// and every launch leaves it zero.  A plan with more split slots than the
// block holds runs unsplit.
constexpr int kSplitCounterSlots = 4096;
constexpr int64_t kSplitCounterBytes = int64_t{kSplitCounterSlots} * 4;

// Launch parameters of the residual + LayerNorm kernels.
struct LnParams {
  const void* x;
  const void* u;
  const void* w;
  const void* b;
  const uint8_t* valid;
  void* r_out;
  void* y_out;
  int64_t rows;
  int N;
  int lanes_per_row;  // vector kernel: lanes that share one row (power of 2)
  float eps;
  int zero_res;
  int zero_norm;
};

// Launch parameters of the Linear (+ activation) kernel: Y = act(X W^T + b),
// X [M, K], W [N, K], Y [M, N] row-major with element leading dimensions.
struct LinearParams {
  const void* x;
  const void* w;
  const void* bias;  // [N] or null
  void* y;
  int64_t ldx, ldw, ldy;
  int M, N, K;
  int tiles_m, tiles_n, tiles;
  int per_xcd;       // tiles dealt to each XCD (the last may get fewer)
  int group_m;       // token tiles per band of the tile order
  unsigned y_bytes;  // bytes of Y addressed by the store resource
};

// Launch parameters of the Linear + residual + LayerNorm kernel (width 1024):
// attn_out = round(A W^T + bias), r = round(x + attn_out),
// y = round(LayerNorm(r) * gamma + beta); A [M, K], W packed in fragment
// order, x / r / y [M, 1024], element leading dimensions.
struct LinearLnParams {
  const void* a;
  const void* wp;     // W [1024, K] packed by launch_pack_weight
  const void* bias;   // [1024] or null
  const void* x;
  const void* gamma;  // [1024]
  const void* beta;   // [1024] or null
  void* r;
  void* y;
  int* counters;      // one per 64-row block: zero before a launch, left zero
  float* stats;       // 256 floats per 64-row block: the halves' row statistics
  int64_t lda, ldx, ldr, ldy;
  int M, K;
  float eps;
  int max_polls;      // polls of the first workgroup of a pair for the second
  unsigned x_bytes, r_bytes, y_bytes;  // extents of the buffer resources
};

// Host-side launchers (defined next to their kernels).  Return a HIP error.
// launch_attention fills p.pair / p.units / the split plan and sizes the
// grid itself.  `workspace` (workspace_bytes, 256-byte aligned) may be null;
// a launch whose split plan needs more than it gets runs unsplit.
hipError_t launch_attention(int dtype, int D, bool causal, bool has_mask,
                            AttnParams& p, void* workspace, int64_t workspace_bytes,
                            hipStream_t stream);
int attention_block_m(int dtype, int D);
// Workspace bytes the key-split schedule of this launch uses on the current
// device (0 when it runs unsplit).
int64_t attention_workspace_bytes(int dtype, int D, bool causal, int64_t BH, int64_t S);

hipError_t launch_residual_layernorm(int dtype, const LnParams& p, bool vector_path,
                                     int vectors_per_lane, hipStream_t stream);

// Exact GELU over n contiguous elements of dtype (0 fp32, 1 bf16, 2 fp16).
hipError_t launch_gelu(int dtype, const void* x, void* y, int64_t n, hipStream_t stream);

// Linear + activation (0 none, 1 exact GELU) for dtype 1 (bf16) or 2 (fp16);
// fills the tile fields of p and sizes the grid.
hipError_t launch_linear(int dtype, int activation, LinearParams& p, hipStream_t stream);

// Linear + residual + LayerNorm, dtype 1 (bf16) or 2 (fp16).
hipError_t launch_linear_ln(int dtype, LinearLnParams& p, hipStream_t stream);
// W [N, K] (16-bit, row stride ldw) into MFMA fragment order (N % 32 == 0,
// K % 16 == 0): 16-byte chunk (fb * K/16 + q) * 64 + l holds
// W[32 fb + l % 32][16 q + 8 (l / 32) .. + 7].
hipError_t launch_pack_weight(const void* w, void* wp, int N, int K, int64_t ldw, hipStream_t stream);

}  // namespace ttk
