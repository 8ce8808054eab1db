// Fused Linear + exact GELU forward for gfx950 (MI355X):
//
//   Y[m, n] = gelu( sum_k X[m, k] * W[n, k] + bias[n] ),
//   gelu(v) = 0.5 * v * (1 + erf(v / sqrt(2)))          (the exact form)
//
// X [M, K] and W [N, K] (the nn.Linear weight) are row-major bf16 or fp16 with
// K contiguous, bias [N] of the same type or NULL, Y [M, N] row-major.  The
// product accumulates in fp32, bias and GELU are applied to the fp32 value and
// the result is rounded once to the storage type.  This is the FFN input
// projection of the reference's encoder, `ffn_in` followed by
// F.gelu(approximate="none") (reference
// benchmarks/torch_transformer_benchmark.py:95-97, transformer_opt/
// submission.py:508-512), with the GELU pass folded into the GEMM epilogue.
//
// Design (one workgroup = 4 wavefronts = a 256 x 256 output tile):
// * The MFMA computes the TRANSPOSED tile C^T[n, m] = W . X^T with
//   v_mfma_f32_32x32x16_{bf16,f16}: both operands are 8 consecutive k of one
//   row (of W and of X), and in the result layout a lane holds one token m and
//   4 consecutive features n per register group.
// * Each wavefront owns 128 features x 128 tokens: 4 x 4 MFMA tiles whose
//   256 fp32 accumulators live in AGPRs (one wavefront per SIMD).
// * K advances in stages of 64.  The W and X tiles of a stage (256 rows x 64
//   k each) are copied global->LDS by LDS-DMA into rows padded to 144 bytes,
//   double-buffered with one barrier per stage; the 16-byte operand reads of
//   16 consecutive rows then start 36 dwords apart and cover all 64 banks.
//   Operand fragments are read one k-step ahead of the MFMAs.
// * The epilogue applies bias and GELU to the accumulators, stages the
//   rounded 256 x 256 tile in LDS (reusing the operand rings) and stores it
//   row by row, 16 bytes per lane, so every store instruction writes whole
//   512-byte row segments of Y.
// * Rows of a partial tile (M or N not a multiple of 256) copy the last row
//   of the matrix (in bounds) and are never stored.
#include <math.h>

#include <type_traits>

#include "ttk_common.h"

namespace ttk {
namespace {

constexpr int kGThreads = 256;
constexpr int kGTile = 256;                 // rows of W (features) and of X (tokens) per tile
// LDS row pitch (elements) of the staged output tile: 256 features + 8 pad, so
// the 8-byte writes of 32 consecutive token rows start 4 banks apart.
constexpr int kOutPitch = kGTile + 8;

// K per stage and number of stages in the LDS ring.
template <int BK_, int NSTAGE_>
struct GemmCfg {
  static constexpr int BK = BK_;
  static constexpr int NSTAGE = NSTAGE_;
  static constexpr int KSTEPS = BK / 16;              // MFMA k-steps per stage
  static constexpr int ROW_CHUNKS = BK / 8 + 1;       // 16-byte chunks per LDS row (+1 pad)
  static constexpr int ROW_ELEMS = ROW_CHUNKS * 8;
  static constexpr int TILE_ELEMS = kGTile * ROW_ELEMS;
  static constexpr int DMA = kGTile * ROW_CHUNKS / 64;  // DMA instructions per operand tile
  static constexpr int DMA_PER_WAVE = DMA / 4;
  static_assert(DMA % 4 == 0, "DMA instructions are dealt evenly to the wavefronts");
  static_assert(KSTEPS % 2 == 0, "fragment sets alternate per k-step");
};
using GCfg = GemmCfg<64, 2>;

#define TTK_GLDS(ptr) ((__attribute__((address_space(3))) void*)(ptr))

__device__ __forceinline__ f32x16 gmfma(BF16, u16x8 a, u16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 gmfma(F16, u16x8 a, u16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ unsigned short round_bits(BF16, float v) {
  return __builtin_bit_cast(unsigned short, static_cast<__bf16>(v));
}
__device__ __forceinline__ unsigned short round_bits(F16, float v) {
  return __builtin_bit_cast(unsigned short, static_cast<_Float16>(v));
}

// One 16-byte LDS-DMA per lane: global bytes [gbase + voff, +16) land at LDS
// byte address lds + 16 * lane.  Issued as inline assembly so that the
// compiler does not treat every later LDS read as a possible consumer of the
// copy (it would wait for all outstanding copies before the first LDS read of
// each stage); the kernel instead waits for exactly the stage it needs with
// explicit vmcnt waits.  M0 carries the LDS address; the one wait state after
// writing it is required before the copy reads it.
__device__ __forceinline__ void lds_dma16(const void* gbase, unsigned voff, unsigned lds) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(gbase), "s"(lds)
               : "memory", "m0");
#pragma clang diagnostic pop
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <typename T, bool HAS_BIAS>
__global__ __launch_bounds__(kGThreads, 1) void linear_gelu_kernel(LinearParams p) {
  using C = GCfg;
  constexpr int BK = C::BK, NSTAGE = C::NSTAGE, KSTEPS = C::KSTEPS, ROW_CHUNKS = C::ROW_CHUNKS,
                ROW_ELEMS = C::ROW_ELEMS, DMA_PER_WAVE = C::DMA_PER_WAVE;
  constexpr int NDMA = 2 * DMA_PER_WAVE;  // copies one wavefront issues per stage
  constexpr unsigned TILE_BYTES = 2u * C::TILE_ELEMS;
  // One LDS block: the W ring, then the X ring; after the K loop it holds the
  // output tile (kOutPitch elements per token row) for the coalesced stores.
  __shared__ __attribute__((aligned(16))) unsigned short smem[2 * NSTAGE * C::TILE_ELEMS];
  static_assert(2 * NSTAGE * C::TILE_ELEMS >= kGTile * kOutPitch, "output tile fits the operand rings");
  unsigned short(*smW)[C::TILE_ELEMS] = reinterpret_cast<unsigned short(*)[C::TILE_ELEMS]>(smem);
  unsigned short(*smX)[C::TILE_ELEMS] = reinterpret_cast<unsigned short(*)[C::TILE_ELEMS]>(smem + NSTAGE * C::TILE_ELEMS);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r32 = lane & 31;
  const int h = lane >> 5;
  const int wn = wave >> 1;  // feature half of the tile this wavefront owns
  const int wm = wave & 1;   // token half

  // Tile of this workgroup: features n0.., tokens m0.. (tokens fastest, so
  // the workgroups that share a W tile run side by side).
  const int tn = blockIdx.x / p.tiles_m;
  const int tm = blockIdx.x - tn * p.tiles_m;
  const int n0 = tn * kGTile;
  const int m0 = tm * kGTile;

  using St = unsigned short;
  const St* __restrict__ W = static_cast<const St*>(p.w);
  const St* __restrict__ X = static_cast<const St*>(p.x);

  // Per-lane DMA source byte offsets (stage-independent): copy j of an
  // operand fills LDS chunks [64j, 64j + 64) of its tile, chunk c of row r
  // holding k 8c..8c+7 (the pad chunk copies chunk 0); rows past the matrix
  // copy its last row.  Wavefront w issues copies j = w, w + 4, ...
  unsigned woff[DMA_PER_WAVE], xoff[DMA_PER_WAVE];
#pragma unroll
  for (int i = 0; i < DMA_PER_WAVE; ++i) {
    const int pos = 64 * (wave + 4 * i) + lane;
    const int row = pos / ROW_CHUNKS;
    const int cc = pos - row * ROW_CHUNKS;
    const int kc = cc < BK / 8 ? 8 * cc : 0;
    woff[i] = 2u * static_cast<unsigned>(min(n0 + row, p.N - 1) * p.ldw + kc);
    xoff[i] = 2u * static_cast<unsigned>(min(m0 + row, p.M - 1) * p.ldx + kc);
  }
  const unsigned ldsW = static_cast<unsigned>(reinterpret_cast<size_t>(TTK_GLDS(&smW[0][0])));
  const unsigned ldsX = static_cast<unsigned>(reinterpret_cast<size_t>(TTK_GLDS(&smX[0][0])));
  // Copy d (0 <= d < NDMA) of stage `stage` into ring buffer `buf`.
  auto dma = [&](int d, int buf, int stage) __attribute__((always_inline)) {
    const int i = d >> 1;
    const unsigned dst = static_cast<unsigned>(buf) * TILE_BYTES + 1024u * static_cast<unsigned>(wave + 4 * i);
    if (d & 1) lds_dma16(X + stage * BK, xoff[i], ldsX + dst);
    else lds_dma16(W + stage * BK, woff[i], ldsW + dst);
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  // Operand fragments of k-step kk (16 k) of a stage: W rows 128wn + 32i + r32
  // and X rows 128wm + 32j + r32, k = 16kk + 8h + 0..7.  Read r of a k-step
  // is fragment kRead[r]: the order in which the MFMAs below first use them.
  const int wrow = (128 * wn + r32) * ROW_ELEMS + 8 * h;
  const int xrow = (128 * wm + r32) * ROW_ELEMS + 8 * h;
  auto read_frag = [&](int r, int buf, int kk, u16x8 (&wf)[4], u16x8 (&xf)[4]) __attribute__((always_inline)) {
    // r: 0 -> W0, 1..4 -> X0..X3, 5..7 -> W1..W3
    if (r == 0 || r >= 5) {
      const int i = r == 0 ? 0 : r - 4;
      wf[i] = *reinterpret_cast<const u16x8*>(&smW[buf][wrow + 32 * i * ROW_ELEMS + 16 * kk]);
    } else {
      const int j = r - 1;
      xf[j] = *reinterpret_cast<const u16x8*>(&smX[buf][xrow + 32 * j * ROW_ELEMS + 16 * kk]);
    }
  };

  // One k-step: 16 MFMAs on (wf, xf), one instruction slot after each MFMA
  // for the next k-step's fragment reads (slots 0-7) and, when `dma_stage` is
  // a stage to copy, for its NDMA copies spread over all 16 slots.  The
  // scheduling barriers keep this order: an MFMA occupies the matrix core for
  // 32 cycles, and the reads and copies issue in its shadow.
  auto kstep = [&](auto rd, auto do_dma, const u16x8 (&wf)[4], const u16x8 (&xf)[4], int rbuf, int rkk,
                   u16x8 (&wn)[4], u16x8 (&xn)[4], int dma_stage, int dma_buf) __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const int i = m >> 2, j = m & 3;
      acc[i][j] = gmfma(T{}, wf[i], xf[j], acc[i][j]);
      if constexpr (decltype(rd)::value) {
        if (m < 8) read_frag(m, rbuf, rkk, wn, xn);
      }
      if constexpr (decltype(do_dma)::value) {
#pragma unroll
        for (int d = m * NDMA / 16; d < (m + 1) * NDMA / 16; ++d) dma(d, dma_buf, dma_stage);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Ring of NSTAGE buffers: stage s lives in buffer s % NSTAGE.  Stages
  // 0..NSTAGE-1 are copied up front; the copy of stage s + NSTAGE starts in
  // the last k-step of stage s, right after the barrier that retires buffer
  // s % NSTAGE.  Copies complete in issue order, so "stage s+1 has landed"
  // is "at most (stages issued after it) * NDMA copies outstanding".
  const int nstages = p.K / BK;
#pragma unroll
  for (int s = 0; s < NSTAGE; ++s)
    if (s < nstages)
      for (int d = 0; d < NDMA; ++d) dma(d, s, s);
  auto wait_stage = [&](int later) __attribute__((always_inline)) {
    // later: stages whose copies were issued after the one needed.
    if constexpr (NSTAGE >= 4) {
      if (later >= 3) { wait_vmcnt<3 * NDMA>(); return; }
    }
    if constexpr (NSTAGE >= 3) {
      if (later >= 2) { wait_vmcnt<2 * NDMA>(); return; }
    }
    if (later >= 1) { wait_vmcnt<NDMA>(); return; }
    wait_vmcnt<0>();
  };
  static_assert(NSTAGE <= 4, "wait_stage covers up to three later stages");
  wait_stage(min(NSTAGE, nstages) - 1);
  __syncthreads();

  constexpr std::true_type kYes{};
  constexpr std::false_type kNo{};
  u16x8 fa_w[4], fa_x[4], fb_w[4], fb_x[4];
#pragma unroll
  for (int r = 0; r < 8; ++r) read_frag(r, 0, 0, fa_w, fa_x);

  // Stage s: k-steps 0 .. KSTEPS-2 read the next k-step of the same stage
  // (KSTEPS is even, so the fragment sets alternate a, b, a, b ... and every
  // stage starts from set a); the last k-step lands stage s+1, retires buffer
  // s % NSTAGE, refills it with stage s + NSTAGE (do_dma) and reads k-step 0
  // of stage s+1 (has_next).  The three loops below keep each stage body free
  // of branches.
  auto stage_body = [&](auto do_dma, auto has_next, int s, int later) __attribute__((always_inline)) {
    const int buf = s % NSTAGE;
#pragma unroll
    for (int kk = 0; kk + 1 < KSTEPS; ++kk) {
      if (kk % 2 == 0) kstep(kYes, kNo, fa_w, fa_x, buf, kk + 1, fb_w, fb_x, 0, 0);
      else kstep(kYes, kNo, fb_w, fb_x, buf, kk + 1, fa_w, fa_x, 0, 0);
    }
    if constexpr (decltype(has_next)::value) {
      wait_stage(later);
      __syncthreads();
      kstep(kYes, do_dma, fb_w, fb_x, (s + 1) % NSTAGE, 0, fa_w, fa_x, s + NSTAGE, buf);
    } else {
      kstep(kNo, kNo, fb_w, fb_x, 0, 0, fa_w, fa_x, 0, 0);
    }
  };
  int s = 0;
  for (; s + NSTAGE < nstages; ++s) stage_body(kYes, kYes, s, NSTAGE - 2);
  for (; s + 1 < nstages; ++s) stage_body(kNo, kYes, s, nstages - 2 - s);
  stage_body(kNo, kNo, s, 0);

  // ---- epilogue ---------------------------------------------------------
  // 1. bias + exact GELU in fp32 on the accumulators, rounded once, written
  //    to the LDS output tile (token rows, feature columns): register group g
  //    of MFMA tile (i, j) holds features 32i + 8g + 4h .. +3 of token 32j + r32.
  // 2. the tile leaves LDS row by row: each lane stores 16 (or 8) consecutive
  //    bytes of one token row, so a store instruction covers whole rows.
  const St* __restrict__ bias = static_cast<const St*>(p.bias);
  St* __restrict__ Y = static_cast<St*>(p.y);
  __syncthreads();  // every wavefront is done with the operand rings
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int nl = 128 * wn + 32 * i + 8 * g + 4 * h;  // feature within the tile
      float bv[4] = {0.f, 0.f, 0.f, 0.f};
      if constexpr (HAS_BIAS) {
        // Features past N read the last bias quad (in bounds); never stored.
        const int nb = min(n0 + nl, p.N - 4);
        const u16x4 b4 = *reinterpret_cast<const u16x4*>(bias + nb);
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = to_f32(T{}, b4[e]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = round_bits(T{}, gelu_exact(acc[i][j][4 * g + e] + bv[e]));
        *reinterpret_cast<u16x4*>(&smem[(128 * wm + 32 * j + r32) * kOutPitch + nl]) = o;
      }
    }
  __syncthreads();
  const int rows = min(kGTile, p.M - m0);
  const int cols = min(kGTile, p.N - n0);  // a multiple of 4
  const bool wide = ((reinterpret_cast<size_t>(p.y) | (2u * static_cast<unsigned>(p.ldy))) & 15u) == 0;
  if (wide) {
    // Two token rows per instruction, 16 bytes per lane.
    const int c = 8 * (lane & 31);
#pragma unroll 4
    for (int t = 0; t < kGTile / 8; ++t) {
      const int r = 2 * (wave + 4 * t) + (lane >> 5);
      if (r < rows && c < cols) {
        St* dst = Y + static_cast<int64_t>(m0 + r) * p.ldy + n0 + c;
        if (c + 8 <= cols) {
          *reinterpret_cast<u16x8*>(dst) = *reinterpret_cast<const u16x8*>(&smem[r * kOutPitch + c]);
        } else {
          *reinterpret_cast<u16x4*>(dst) = *reinterpret_cast<const u16x4*>(&smem[r * kOutPitch + c]);
        }
      }
    }
  } else {
    // One token row per instruction, 8 bytes per lane.
    const int c = 4 * lane;
#pragma unroll 4
    for (int t = 0; t < kGTile / 4; ++t) {
      const int r = wave + 4 * t;
      if (r < rows && c < cols) {
        *reinterpret_cast<u16x4*>(Y + static_cast<int64_t>(m0 + r) * p.ldy + n0 + c) =
            *reinterpret_cast<const u16x4*>(&smem[r * kOutPitch + c]);
      }
    }
  }
}

}  // namespace

hipError_t launch_linear_gelu(int dtype, LinearParams& p, hipStream_t stream) {
  p.tiles_m = (p.M + kGTile - 1) / kGTile;
  const int tiles_n = (p.N + kGTile - 1) / kGTile;
  const dim3 grid(static_cast<unsigned>(p.tiles_m) * static_cast<unsigned>(tiles_n)), blk(kGThreads);
  const bool bias = p.bias != nullptr;
  switch (dtype) {
    case 1:
      if (bias) linear_gelu_kernel<BF16, true><<<grid, blk, 0, stream>>>(p);
      else linear_gelu_kernel<BF16, false><<<grid, blk, 0, stream>>>(p);
      break;
    case 2:
      if (bias) linear_gelu_kernel<F16, true><<<grid, blk, 0, stream>>>(p);
      else linear_gelu_kernel<F16, false><<<grid, blk, 0, stream>>>(p);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ttk
