// Linear (+ exact GELU) forward for gfx950 (MI355X), bf16 / fp16:
//
//   Y[m, n] = act( round( sum_k X[m, k] * W[n, k] + bias[n] ) )
//
// X [M, K] and W [N, K] (the nn.Linear weight) are row-major with K
// contiguous, bias [N] or none, Y [M, N] row-major.  The product accumulates
// in fp32 and bias is added in fp32; the sum is rounded to the storage type
// (the output of the reference's F.linear), and act is applied to that
// rounded value and rounded again - exactly the dtype boundaries of the
// reference's `F.gelu(layer.ffn_in(h))` (transformer_opt/submission.py:507;
// benchmarks/torch_transformer_benchmark.py:95-97), with the GELU pass
// folded into the GEMM's epilogue instead of a second trip through HBM.
//
// The GELU of a bf16 value is read from a table of the exact GELU of every
// bf16 input in (-8, -2^-16] and [2^-16, 8), correctly rounded
// (gelu_bf16_table.h, generated in float64), kept in LDS: per pair of
// outputs five packed 16-bit integer operations, two LDS reads and a byte
// permute replace the ~17 VALU operations per element of an erf evaluation.
// Inputs outside the table (rare: GELU is x there, or x/2 at bf16 precision)
// take gelu_exact().  fp16 evaluates gelu_exact() on every element.
//
// Design (one workgroup = 4 wavefronts, one per SIMD; a 256 x 256 tile):
// * The MFMA computes the transposed tile C^T[n, m] = W . X^T with
//   v_mfma_f32_32x32x16_{bf16,f16}: both operands are 8 consecutive k of one
//   row, and in the result a lane holds one token and 4 consecutive features
//   per register group.  Each wavefront owns 128 features x 128 tokens:
//   4 x 4 MFMA tiles, 256 fp32 accumulators (AGPRs).
// * K advances in stages of 64 through a 2-deep LDS ring per operand
//   (2 x 32 KB), after the 9.5 KB GELU table: 137.5 KB of LDS, one
//   workgroup per CU.  Stages are copied global -> LDS by LDS-DMA, spread
//   over the MFMAs of the k-steps around the barrier that frees their buffer
//   (one copy every 4 MFMAs), so a copy has about one stage of compute to
//   land.  Rows are 128 bytes of eight 16-byte chunks, chunk c of row r
//   stored at c ^ ((r >> 1) & 7): the 16-byte operand reads of 16
//   consecutive rows then cover all 64 banks.
// * Persistent grid: each workgroup walks its tiles, and the copies of the
//   next tile's first two stages are issued during the current tile's last
//   two, so they land while the epilogue runs and its stores drain while
//   the next tile computes.
// * Tile order: workgroups are dealt round-robin to the 8 XCDs, so the slots
//   of one workgroup stay on one XCD; each XCD gets a contiguous band of the
//   tile grid (group_m token tiles x all feature tiles), and the workgroups
//   of an XCD share their X and W strips in its L2.
// * Epilogue straight from the accumulators: bias (scalar loads), rounding,
//   activation, then one v_permlane32_swap per dword gives each lane 8
//   consecutive features of one token, stored as 16 bytes by a buffer store
//   whose resource covers Y: stores of rows >= M or features >= N fall
//   outside it and are dropped, so every wavefront issues the same number of
//   stores - which the copy waits count on.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "gelu_bf16_table.h"
#include "ttk_common.h"

namespace ttk {
namespace {

#ifndef TTK_LIN_WAVES
#define TTK_LIN_WAVES 4
#endif
constexpr int kLinWaves = TTK_LIN_WAVES;             // wavefronts per workgroup

constexpr int kLinTile = 256;                        // features and tokens per tile
constexpr int kLinBK = 64;                           // k per stage
constexpr int kLinStages = 2;                        // LDS ring depth
constexpr int kLinOpBytes = kLinTile * kLinBK * 2;   // one operand tile of one stage
constexpr int kLinTabBytes = kGeluBf16Entries * 2;
constexpr int kLinWRing = kLinTabBytes;              // LDS: table, W ring, X ring
constexpr int kLinXRing = kLinWRing + kLinStages * kLinOpBytes;
constexpr int kLinSmem = kLinXRing + kLinStages * kLinOpBytes;
static_assert(kLinTabBytes % 1024 == 0 || kLinTabBytes % 256 == 0, "ring starts 256-byte aligned");
static_assert(kLinSmem <= 160 * 1024, "LDS of one workgroup");

typedef unsigned short us2 __attribute__((ext_vector_type(2)));
typedef __bf16 lbf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 lf16x2 __attribute__((ext_vector_type(2)));
typedef const __attribute__((address_space(4))) unsigned* ConstU32;
#define TTK_LIN_LDS(ptr) ((__attribute__((address_space(3))) void*)(ptr))

__device__ __forceinline__ f32x16 lmfma(BF16, u16x8 a, u16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 lmfma(F16, u16x8 a, u16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Two fp32 values rounded to the storage type (round to nearest even, by the
// gfx950 conversion instructions), packed low / high.
__device__ __forceinline__ unsigned lpack(BF16, float a, float b) {
  const lbf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(unsigned, v);
}
__device__ __forceinline__ unsigned lpack(F16, float a, float b) {
  const lf16x2 v = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
  return __builtin_bit_cast(unsigned, v);
}

// Table index of two packed bf16 values: each 16-bit half rotated left by one
// (sign to bit 0) minus 2 * kGeluBf16First, i.e. 2 (magnitude - first) + sign
// modulo 2^16 - below kGeluBf16Entries exactly for the inputs the table holds.
// Three instructions: the sign bits, or-ed with -2 * first (0x9100), are the
// addend of a packed multiply-add of the bits by 2 (whose product drops the
// sign bit).
__device__ __forceinline__ unsigned gelu_table_index(unsigned pre) {
  static_assert(((0x10000 - 2 * kGeluBf16First) & 1) == 0, "the sign bit fits below the addend");
  const us2 bits = __builtin_bit_cast(us2, pre);
  const us2 addend = (bits >> static_cast<unsigned short>(15)) |
                     static_cast<unsigned short>(0x10000 - 2 * kGeluBf16First);
  unsigned r;
  asm("v_pk_mad_u16 %0, %1, 2, %2 op_sel_hi:[1,0,1]" : "=v"(r) : "v"(pre), "v"(__builtin_bit_cast(unsigned, addend)));
  return r;
}
// Exact GELU of two packed bf16 values from the table at the start of the
// kernel's LDS (`smem`), given their index pair r (gelu_table_index).  The index is clamped, so the
// reads stay inside the table for any input.
__device__ __forceinline__ unsigned gelu_pair_table(unsigned r, const unsigned char* smem) {
  const us2 last = {static_cast<unsigned short>(kGeluBf16Entries - 1),
                    static_cast<unsigned short>(kGeluBf16Entries - 1)};
  const unsigned c = __builtin_bit_cast(unsigned, __builtin_elementwise_min(__builtin_bit_cast(us2, r), last));
  unsigned lo_byte;  // 2 * low index: one multiply-add on the low half
  asm("v_mad_u32_u16 %0, %1, 2, 0" : "=v"(lo_byte) : "v"(c));
  const unsigned hi_byte = c >> 15;  // 2 * high index (the low index is below 2^15)
  // Two 16-bit reads, merged by one byte permute (16-bit loads into register
  // halves zero the other half on this GPU, so they cannot merge in place).
  const unsigned lo = *reinterpret_cast<const unsigned short*>(smem + lo_byte);
  const unsigned hi = *reinterpret_cast<const unsigned short*>(smem + hi_byte);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}
// Exact GELU of two packed values by evaluation (inputs outside the table,
// and fp16).
template <typename T>
__device__ __forceinline__ unsigned gelu_pair_eval(T, unsigned pre) {
  return lpack(T{}, gelu_exact(to_f32(T{}, static_cast<unsigned short>(pre))),
               gelu_exact(to_f32(T{}, static_cast<unsigned short>(pre >> 16))));
}
// Whether a bf16 value (low 16 bits of b) has a table entry.
__device__ __forceinline__ bool in_table(unsigned b) {
  return static_cast<unsigned short>((b & 0x7fffu) - kGeluBf16First) < kGeluBf16Pos;
}

// One 16-byte LDS-DMA per lane: global bytes [gbase + voff, +16) land at LDS
// byte address lds + 16 * lane.  Inline assembly, so that the compiler does
// not take every later LDS read for a consumer of the copy (it would wait for
// all outstanding copies before the first one); the kernel waits for exactly
// the stage it needs with explicit vmcnt waits.  M0 carries the LDS address;
// the one wait state after writing it is required before the copy reads it.
__device__ __forceinline__ void lin_dma16(const void* gbase, unsigned voff, unsigned lds) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(gbase), "s"(lds)
               : "memory", "m0");
#pragma clang diagnostic pop
}

// Wait until at most n vector-memory operations of this wavefront are
// outstanding, n rounded down to the nearest count the kernel uses (waiting
// for fewer outstanding operations is always safe).
__device__ __forceinline__ void lin_vm_wait(int n) {
  if (n >= 48) {
    asm volatile("s_waitcnt vmcnt(48)" ::: "memory");
  } else if (n >= 40) {
    asm volatile("s_waitcnt vmcnt(40)" ::: "memory");
  } else if (n >= 32) {
    asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
  } else if (n >= 24) {
    asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
  } else if (n >= 16) {
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
  } else if (n >= 12) {
    asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  } else if (n >= 8) {
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  } else if (n >= 4) {
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
}

// Tile of slot `slot` (see the tile order above); false for a slot past the
// last tile of its XCD.
__device__ __forceinline__ bool lin_tile(const LinearParams& p, int slot, int& m0, int& n0) {
  const int q = slot >> 3;
  const int o = (slot & 7) * p.per_xcd + q;
  if (q >= p.per_xcd || o >= p.tiles) return false;
  const int span = p.group_m * p.tiles_n;
  const int band = o / span;
  const int first = band * p.group_m;
  const int gs = min(p.group_m, p.tiles_m - first);
  const int rem = o - band * span;
  m0 = (first + rem % gs) * kLinTile;
  n0 = (rem / gs) * kLinTile;
  return true;
}

template <typename T, bool GELU, bool BIAS, int NW>
__global__ __launch_bounds__(64 * NW, 1) void linear_kernel(LinearParams p) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[kLinSmem];
  constexpr bool kTable = GELU && std::is_same<T, BF16>::value;
  static_assert(NW == 4 || NW == 8, "four or eight wavefronts per workgroup");
  constexpr int TJ = NW == 4 ? 4 : 2;       // 32-token MFMA blocks per wavefront
  constexpr int WT = 32 * TJ;               // tokens per wavefront
  constexpr int CPO = kLinTile / 8;         // copy instructions per operand per stage
  constexpr int DMA = 2 * CPO / NW;         // copies per wavefront per stage
  constexpr int HALF = DMA / 2;             // copies per k-step that issues any
  constexpr int KS = kLinBK / 16;           // k-steps per stage
  constexpr int MF = 4 * TJ;                // MFMAs per k-step
  constexpr int kGap = MF / HALF;           // MFMAs per copy
  constexpr int STORES = 8 * TJ;            // stores per wavefront per tile
  static_assert(kGap >= 1 && MF % HALF == 0, "copies spread evenly over a k-step");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31;
  const int h = lane >> 5;
  const int wn = wave & 1;   // feature half of the tile (128 features)
  const int wm = wave >> 1;  // token block of the tile (WT tokens)

  // The slots of this workgroup: blockIdx.x, + gridDim.x, ... (one XCD).
  const int grid = static_cast<int>(gridDim.x);
  const int slot_end = 8 * p.per_xcd;
  int slot = static_cast<int>(blockIdx.x);
  int cm = 0, cn = 0;
  while (slot < slot_end && !lin_tile(p, slot, cm, cn)) slot += grid;
  if (slot >= slot_end) return;
  int nm = 0, nn = 0;
  auto find_next = [&]() __attribute__((always_inline)) -> bool {
    slot += grid;
    while (slot < slot_end && !lin_tile(p, slot, nm, nn)) slot += grid;
    return slot < slot_end;
  };

  if constexpr (kTable) {
    const u32x4* src = reinterpret_cast<const u32x4*>(kGeluBf16Table);
    u32x4* dst = reinterpret_cast<u32x4*>(smem);
    for (int i = tid; i < kLinTabBytes / 16; i += 64 * NW) dst[i] = src[i];
  }

  // Copy lanes: lane L of copy instruction c fills LDS row 8c + L/8 of the
  // operand tile at physical chunk L%8, which holds logical chunk
  // (L%8) ^ ((row >> 1) & 7) = (L%8) ^ (4 (c & 1) + ((L >> 4) & 3)).
  // Wavefront w issues c = w, w + NW, ... (c & 1 == w & 1).  Rows past the
  // matrix copy its last row (in bounds, never stored).  Lane offsets are
  // recomputed at every issue rather than kept in registers across the loop.
  const int drow = lane >> 3;
  const unsigned dchunk = static_cast<unsigned>((lane & 7) ^ (((wave & 1) << 2) | ((lane >> 4) & 3))) * 16u;
  const unsigned wpitch = static_cast<unsigned>(p.ldw) * 2u;
  const unsigned xpitch = static_cast<unsigned>(p.ldx) * 2u;
  const unsigned lds0 = static_cast<unsigned>(reinterpret_cast<size_t>(TTK_LIN_LDS(smem)));
  // Copy c (0 .. DMA-1) of stage ks of the tile at (m0, n0) into ring buffer
  // buf: copy instruction wave + NW (c >> 1) of W (c even) or X (c odd).
  auto issue_one = [&](int m0, int n0, int ks, int buf, int c) __attribute__((always_inline)) {
    const int ci = wave + NW * (c >> 1);
    const int row = 8 * ci + drow;
    const unsigned blk = static_cast<unsigned>(buf * kLinOpBytes + ci * 1024);
    if (c & 1) {
      const char* xb = static_cast<const char*>(p.x) + static_cast<size_t>(ks) * (kLinBK * 2);
      lin_dma16(xb, static_cast<unsigned>(min(m0 + row, p.M - 1)) * xpitch + dchunk, lds0 + kLinXRing + blk);
    } else {
      const char* wb = static_cast<const char*>(p.w) + static_cast<size_t>(ks) * (kLinBK * 2);
      lin_dma16(wb, static_cast<unsigned>(min(n0 + row, p.N - 1)) * wpitch + dchunk, lds0 + kLinWRing + blk);
    }
  };

  // Operand fragments: W rows 128wn + 32i + r32 and X rows WT wm + 32j + r32,
  // k = 16kk + 8h .. + 7 (logical chunk 2kk + h of the stage, physical chunk
  // (2kk + h) ^ ((r32 >> 1) & 7)).  The 16-byte reads of 16 consecutive rows
  // then cover all 64 banks.
  const int swz = (r32 >> 1) & 7;
  const unsigned char* wfrag[KS];
  const unsigned char* xfrag[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    wfrag[kk] = smem + kLinWRing + (128 * wn + r32) * (kLinBK * 2) + 16 * ((2 * kk + h) ^ swz);
    xfrag[kk] = smem + kLinXRing + (WT * wm + r32) * (kLinBK * 2) + 16 * ((2 * kk + h) ^ swz);
  }

  f32x16 acc[4][TJ];
  // Copies of a stage go out as two halves: the first in the k-step right
  // after the barrier that frees their ring buffer, the second in the next
  // k-step.
  struct Pending {
    bool on;
    int m0, n0, ks, buf;
  };
  // One k-step: MF MFMAs on (wf, xf).  In their shadow go the fragment reads
  // of the next k-step (one after each of the first 4 + TJ MFMAs) and, when
  // d.on, copies HALF * half .. + HALF - 1 of stage d.ks of the tile at
  // (d.m0, d.n0) into ring buffer d.buf, one every kGap MFMAs - or, with
  // `both`, all DMA copies of the stage, evenly spread.
  auto kstep = [&](auto zero, const u16x8 (&wf)[4], const u16x8 (&xf)[TJ], int rbuf, int rkk,
                   u16x8 (&nw)[4], u16x8 (&nx)[TJ], const Pending& d, int half,
                   auto both) __attribute__((always_inline)) {
    const unsigned char* wb = wfrag[rkk] + rbuf * kLinOpBytes;
    const unsigned char* xb = xfrag[rkk] + rbuf * kLinOpBytes;
#pragma unroll
    for (int t = 0; t < MF; ++t) {
      const int i = t / TJ, j = t % TJ;
      if constexpr (decltype(zero)::value) {
        acc[i][j] = lmfma(T{}, wf[i], xf[j], f32x16{});
      } else {
        acc[i][j] = lmfma(T{}, wf[i], xf[j], acc[i][j]);
      }
      if (t < 4) nw[t] = *reinterpret_cast<const u16x8*>(wb + 32 * (kLinBK * 2) * t);
      else if (t < 4 + TJ) nx[t - 4] = *reinterpret_cast<const u16x8*>(xb + 32 * (kLinBK * 2) * (t - 4));
      if constexpr (decltype(both)::value) {
        constexpr int kGap2 = MF / DMA;
        static_assert(kGap2 >= 1 && MF % DMA == 0, "all copies fit one k-step");
        if (t % kGap2 == 0 && d.on) issue_one(d.m0, d.n0, d.ks, d.buf, t / kGap2);
      } else if (t % kGap == (kGap > 1 ? 1 : 0) && d.on) {
        issue_one(d.m0, d.n0, d.ks, d.buf, HALF * half + t / kGap);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Epilogue of the tile at (m0, n0).
  const unsigned y_pitch = static_cast<unsigned>(p.ldy) * 2u;
  const __amdgpu_buffer_rsrc_t yrsrc =
      __builtin_amdgcn_make_buffer_rsrc(p.y, static_cast<short>(0), static_cast<int>(p.y_bytes), 0x00020000);
  auto epilogue = [&](int m0, int n0) __attribute__((always_inline)) {
    // Lane-derived values are re-derived here from an opaque copy of the lane
    // index, so the compiler does not compute them once before the main loop
    // and keep them in registers through it.
    int el = lane;
    asm volatile("" : "+v"(el));
    const int eh = el >> 5;
    const int er = el & 31;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int fblock = n0 + 128 * wn + 32 * i;  // features fblock .. +31 (wave-uniform)
      float bq[4][4];
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) bq[g][e] = 0.0f;
      if constexpr (BIAS) {
        // 32 bias values by scalar loads (a block past N reads the last block:
        // in bounds, never stored); the lane keeps features 8g + 4h .. + 3.
        const int fb = __builtin_amdgcn_readfirstlane(min(fblock, p.N - 32));
        const ConstU32 cb = (ConstU32)(static_cast<const char*>(p.bias) + 2 * fb);
        unsigned d[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) d[t] = cb[t];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const unsigned lo = eh ? d[4 * g + 2] : d[4 * g];
          const unsigned hi = eh ? d[4 * g + 3] : d[4 * g + 1];
          bq[g][0] = to_f32(T{}, static_cast<unsigned short>(lo));
          bq[g][1] = to_f32(T{}, static_cast<unsigned short>(lo >> 16));
          bq[g][2] = to_f32(T{}, static_cast<unsigned short>(hi));
          bq[g][3] = to_f32(T{}, static_cast<unsigned short>(hi >> 16));
        }
        // Materialised once per feature block (otherwise the compiler
        // rebuilds them from the scalar registers for every token block).
#pragma unroll
        for (int g = 0; g < 4; ++g) asm volatile("" : "+v"(bq[g][0]), "+v"(bq[g][1]), "+v"(bq[g][2]), "+v"(bq[g][3]));
      }
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int m = m0 + WT * wm + 32 * j + er;
#pragma unroll
        for (int gp = 0; gp < 2; ++gp) {
          // Linear outputs rounded to T, two per dword (groups 2gp, 2gp+1).
          unsigned o[2][2];
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const int g = 2 * gp + k;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = BIAS ? acc[i][j][4 * g + e] + bq[g][e] : acc[i][j][4 * g + e];
            o[k][0] = lpack(T{}, v[0], v[1]);
            o[k][1] = lpack(T{}, v[2], v[3]);
            // Opaque, so the compiler keeps the packed conversion (it would
            // convert each half again to take the table index apart).
            asm volatile("" : "+v"(o[k][0]), "+v"(o[k][1]));
          }
          if constexpr (kTable) {
            // Table reads for all eight; in the rare group where some lane
            // holds an input outside the table (a wave-uniform branch), every
            // lane evaluates and keeps the evaluation for those inputs only.
            unsigned r[2][2], t[2][2];
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
              for (int d = 0; d < 2; ++d) {
                r[k][d] = gelu_table_index(o[k][d]);
                t[k][d] = gelu_pair_table(r[k][d], smem);
              }
            const us2 rmax = __builtin_elementwise_max(
                __builtin_elementwise_max(__builtin_bit_cast(us2, r[0][0]), __builtin_bit_cast(us2, r[0][1])),
                __builtin_elementwise_max(__builtin_bit_cast(us2, r[1][0]), __builtin_bit_cast(us2, r[1][1])));
            const bool all_ok = (rmax.x < kGeluBf16Entries) & (rmax.y < kGeluBf16Entries);
            if (__builtin_expect(__builtin_amdgcn_ballot_w64(!all_ok) != 0, 0)) {
#pragma unroll
              for (int k = 0; k < 2; ++k)
#pragma unroll
                for (int d = 0; d < 2; ++d) {
                  const unsigned e = gelu_pair_eval(T{}, o[k][d]);
                  const unsigned lo = in_table(o[k][d]) ? t[k][d] : e;
                  const unsigned hi = in_table(o[k][d] >> 16) ? t[k][d] : e;
                  t[k][d] = (lo & 0xffffu) | (hi & 0xffff0000u);
                }
            }
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
              for (int d = 0; d < 2; ++d) o[k][d] = t[k][d];
          } else if constexpr (GELU) {
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
              for (int d = 0; d < 2; ++d) o[k][d] = gelu_pair_eval(T{}, o[k][d]);
          }
          // Lanes < 32 keep group 2gp (features +0..3) and take its +4..7 from
          // lane + 32; lanes >= 32 get group 2gp+1's +8..11 from lane - 32 and
          // keep its +12..15.
          const auto s0 = __builtin_amdgcn_permlane32_swap(o[0][0], o[1][0], false, false);
          const auto s1 = __builtin_amdgcn_permlane32_swap(o[0][1], o[1][1], false, false);
          const u32x4 v = {s0[0], s1[0], s0[1], s1[1]};
          const int f = fblock + 16 * gp + 8 * eh;
          const unsigned off = (m < p.M && f < p.N)
              ? static_cast<unsigned>(m) * y_pitch + static_cast<unsigned>(f) * 2u
              : 0x80000000u;
          __builtin_amdgcn_raw_buffer_store_b128(v, yrsrc, static_cast<int>(off), 0, 0);
        }
        // Two groups of 8 outputs at a time (the table reads of one overlap
        // the other's arithmetic); unfenced, the scheduler hoists the table
        // reads of many groups and runs out of registers.
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // ---- the stage stream ----------------------------------------------------
  // Stages of KS k-steps through a two-buffer ring.  The barrier of stage s
  // sits before its last k-step: by then every wavefront has read all of
  // stage s's fragments (they are read one k-step ahead), so its buffer is
  // free, and stage s + 1 must be in LDS.  Stage s + 2's copies go into that
  // buffer in two halves, in the last k-step of s and the first of s + 1;
  // at stage s's barrier the only copies outstanding are stage s + 1's, so
  // the wait is vmcnt(0).  The exception is the tile boundary: the last
  // k-step of a tile issues all of the next tile's stage-1 copies, so that
  // the epilogue's STORES stores come after every copy the next tile's first
  // barrier waits for, and that barrier waits vmcnt(STORES) - the stores
  // drain while the next tile computes.  Stages run in pairs (one per
  // buffer): the first pair of a tile (accumulators start at zero), the
  // middle pairs and the last pair (copies of the next tile's first stages,
  // if any); NS >= 4 keeps the first and last apart.
  const int NS = p.K / kLinBK;
  bool has_next = find_next();
#pragma unroll
  for (int c = 0; c < DMA; ++c) issue_one(cm, cn, 0, 0, c);
#pragma unroll
  for (int c = 0; c < DMA; ++c) issue_one(cm, cn, 1, 1, c);
  lin_vm_wait(DMA);
  __syncthreads();  // stage 0 and the GELU table are in LDS
  u16x8 fw[2][4], fx[2][TJ];  // fragment sets of consecutive k-steps
#pragma unroll
  for (int i = 0; i < 4; ++i) fw[0][i] = *reinterpret_cast<const u16x8*>(wfrag[0] + 32 * (kLinBK * 2) * i);
#pragma unroll
  for (int j = 0; j < TJ; ++j) fx[0][j] = *reinterpret_cast<const u16x8*>(xfrag[0] + 32 * (kLinBK * 2) * j);

  constexpr std::true_type kYes{};
  constexpr std::false_type kNo{};
  constexpr std::integral_constant<int, 0> kFirst{};
  constexpr std::integral_constant<int, 1> kMiddle{};
  constexpr std::integral_constant<int, 2> kLast{};
  Pending pend{false, 0, 0, 0, 0};  // second half of the copies last issued
  const Pending none{false, 0, 0, 0, 0};
  bool first = true;
  for (;;) {
    auto pair = [&](auto kind, int s0) __attribute__((always_inline)) {
      constexpr int K = decltype(kind)::value;
#pragma unroll
      for (int u = 0; u < kLinStages; ++u) {
#pragma unroll
        for (int kk = 0; kk + 1 < KS; ++kk) {
          const int a = kk & 1;
          if (K == 0 && u == 0 && kk == 0) {
            kstep(kYes, fw[a], fx[a], u, kk + 1, fw[a ^ 1], fx[a ^ 1], none, 1, kNo);
          } else {
            kstep(kNo, fw[a], fx[a], u, kk + 1, fw[a ^ 1], fx[a ^ 1], kk == 0 ? pend : none, 1, kNo);
          }
        }
        // Last k-step: the barrier, then stage s + 2's first copies.
        constexpr int a = (KS - 1) & 1;
        if constexpr (K == 2) {
          // s = NS - 2 + u: s + 1 exists for u == 0 or with a next tile.
          if (u == 0 || has_next) {
            lin_vm_wait(0);
            __syncthreads();
          }
          pend = Pending{has_next, nm, nn, u, u};
        } else {
          // The first stage of a tile after the first: the previous tile's
          // stores came after all of stage 1's copies.
          lin_vm_wait((K == 0 && u == 0 && !first) ? STORES : 0);
          __syncthreads();
          pend = Pending{true, cm, cn, s0 + u + 2, u};
        }
        if (K == 2 && u == 1) {
          // The next tile's stage 1, all copies before the epilogue.
          kstep(kNo, fw[a], fx[a], u ^ 1, 0, fw[a ^ 1], fx[a ^ 1], pend, 0, kYes);
          pend = none;
        } else {
          kstep(kNo, fw[a], fx[a], u ^ 1, 0, fw[a ^ 1], fx[a ^ 1], pend, 0, kNo);
        }
      }
    };
    pair(kFirst, 0);
    for (int s0 = kLinStages; s0 < NS - kLinStages; s0 += kLinStages) pair(kMiddle, s0);
    pair(kLast, NS - kLinStages);
    epilogue(cm, cn);
    if (!has_next) break;
    cm = nm;
    cn = nn;
    has_next = find_next();
    first = false;
  }
}

template <typename T, bool GELU>
hipError_t launch_typed(LinearParams& p, dim3 grid, hipStream_t stream) {
  constexpr int NW = kLinWaves;
  if (p.bias) {
    linear_kernel<T, GELU, true, NW><<<grid, dim3(64 * NW), 0, stream>>>(p);
  } else {
    linear_kernel<T, GELU, false, NW><<<grid, dim3(64 * NW), 0, stream>>>(p);
  }
  return hipGetLastError();
}

int lin_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      n = 256;
    }
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace

hipError_t launch_linear(int dtype, int activation, LinearParams& p, hipStream_t stream) {
  p.tiles_m = (p.M + kLinTile - 1) / kLinTile;
  p.tiles_n = (p.N + kLinTile - 1) / kLinTile;
  p.tiles = p.tiles_m * p.tiles_n;
  p.per_xcd = (p.tiles + 7) / 8;
  // A band of the tile order covers about one XCD's share of the tiles.
  p.group_m = std::max(1, std::min(p.tiles_m, p.per_xcd / p.tiles_n));
  const int cus = lin_cu_count() / 8 * 8;
  const int groups = std::max(8, std::min(cus, 8 * p.per_xcd));
  const dim3 grid(static_cast<unsigned>(groups));
  const bool gelu = activation == 1;
  switch (dtype) {
    case 1: return gelu ? launch_typed<BF16, true>(p, grid, stream) : launch_typed<BF16, false>(p, grid, stream);
    case 2: return gelu ? launch_typed<F16, true>(p, grid, stream) : launch_typed<F16, false>(p, grid, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ttk
