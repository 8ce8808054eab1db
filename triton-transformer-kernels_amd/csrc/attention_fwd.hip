// Fused flash-style attention forward for gfx950 (MI355X).
//
// Semantics follow the reference kernel `_attention_fwd`
// (transformer_opt/kernels/attention.py:103-265): BSHD strided q/k/v, fp32
// running max / running sum / output accumulator, keys visited in tiles with
// an online softmax, key mask `valid[b, t]`, causal bound
// `end = min(S, (query_tile + 1) * BLOCK_M)`, and exact zeros for a query row
// without any allowed key.
//
// Design (one workgroup = 4 wavefronts = 128 queries of one (batch, head)):
//
// * Each wavefront owns 32 queries and the full head dimension.  It computes
//   the TRANSPOSED score tile S^T[key, query] = K . Q^T with the 32x32 MFMA.
//   In the 32x32 MFMA result layout a lane holds one column (query = lane%32)
//   and 16 rows (keys 8*(r/4) + 4*(lane/32) + r%4 for register r), so
//     - the softmax row statistics of a query are a reduction over the lane's
//       own registers plus ONE exchange with lane^32 (v_permlane32_swap), and
//     - the probabilities P^T already sit in the B-operand layout of the next
//       MFMA, O^T[d, query] += V^T[d, key] . P^T[key, query]: register r
//       feeds the k-step whose two keys are the ones that register holds in
//       lane halves 0 and 1.  No transpose, no LDS round trip for P.
// * K and V tiles are double-buffered in LDS with one barrier per tile.  K
//   rows are padded by 16 bytes, so the 16-byte MFMA operand reads of 16
//   consecutive key rows start on distinct banks and cover all 64 banks, and
//   every per-step operand address is the lane's base plus an immediate.
//     - fp32: the next tile's global loads are issued into registers before
//       the current tile's MFMAs and written to the other buffer after them.
//       The fp32 MFMA is 16 passes long, so the matrix core is the bound and
//       the softmax VALU of one wavefront runs under the MFMAs of the other
//       wavefront on the SIMD.
//     - bf16/fp16: the 8-pass MFMA leaves the softmax as the bound (per
//       64-key tile of the unmasked steady body a wavefront issues 16
//       (head_dim 64) or 32 (128) MFMAs against 134 other VALU instructions
//       in the compiled head_dim-64 loop: 114 of softmax (32 fma, 32
//       v_exp_f32, 16 conversions, 16 max3, 16 dot2 row-sum steps, the
//       cross-half max), 2 for the lagging-max test and 18 of copy
//       addressing; a masked tile costs ~280), so the loop is
//       software-pipelined.  Unmasked tiles run two phases per tile:
//       Q.K of tile t+1 interleaved with the exp2 and 16-bit rounding of
//       tile t's scores, then the P.V of tile t interleaved with the row max
//       of tile t+1.  Key-masked launches run one stream interleaving the
//       P.V of tile t-1 with the softmax of tile t.  K and V tiles are
//       copied global->LDS by LDS-DMA (global_load_lds_dwordx4, no register
//       staging), spread over the MFMA groups of the pipelined loop; V stays
//       row-major and the P.V operand is read with the transposing
//       ds_read_b64_tr_b16.
// * Masking: key validity (key mask and key < S) is a wave-uniform 64-bit
//   ballot per tile; with the lane's causal limit it becomes one bit mask per
//   32-key sub-block.  Only tiles that need it (diagonal, ragged end, key
//   mask) take the masked path; interior tiles run unmasked.  Causal
//   workgroups stop at their diagonal (future tiles are never loaded) and a
//   wavefront skips the 32-key sub-blocks entirely after its last query.
//   fp32 with 64-key tiles: in the last tile of a query tile, wavefront 0
//   (whose rows are complete) takes wavefront 3's diagonal sub-block and
//   hands its partial softmax state over through LDS, so the diagonal costs
//   3 sub-block times instead of 4.
// * fp32 head_dim 8 and 16: P.V runs on 16x16x4 MFMAs (a 32x32 O^T block
//   would leave 3/4 or half of its d-rows empty); v_permlane16_swap of two
//   score registers regroups them by 16 queries, see the tile body.
// * Scheduling: causal query tile i costs i+1 key blocks.  When the grid
//   still fills every workgroup slot of the GPU, a workgroup runs the query
//   tiles nq-1-i and i one after the other, so all workgroups carry the same
//   nq+1 blocks of work and the launch has no tail.  Otherwise the flat grid
//   is ordered heaviest query tile first, or, for an fp32 grid resident in
//   one round, folded so that the two workgroups of a CU hold a heavy and a
//   light tile.  fp32 non-causal with S <= 64 runs two (batch, head) pairs
//   per workgroup (the twin grid).  When B*H is a multiple of 8 all
//   workgroups of one head run on the same XCD (workgroups are dealt
//   round-robin to the 8 XCDs), so a head's K/V is fetched from HBM into one
//   XCD's L2 instead of eight.  The fp32 kernel alternates wave priority per
//   tile between the two workgroups of a CU (the age order otherwise favours
//   the older one throughout).
// * Output: the 16-bit kernel stages each wavefront's 32 x D tile in LDS so
//   that each store covers whole rows; fp32 stores straight from registers.
//
// fp32 path: v_mfma_f32_32x32x2_f32 (IEEE fp32 products, fp32 accumulate).
// Q is pre-multiplied by scale*log2(e) so scores are already in the exp2
// domain.  bf16/fp16 path: v_mfma_f32_32x32x16_{bf16,f16}; scores stay fp32,
// the row max is taken on raw scores and the scale is folded into one fma per
// element before exp2; P is rounded to the input type (v_cvt_pk_bf16_f32 /
// v_cvt_f16_f32) for the P.V product; the 16-bit A operand (8 keys of one d)
// is two transposing 8-byte LDS reads of the row-major V tile.
#include <algorithm>
#include <atomic>

#include "ttk_common.h"

namespace ttk {
namespace {

constexpr int kThreads = 256;
constexpr int kBM = 128;  // queries per workgroup (4 wavefronts x 32)

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 mfma_16(BF16, u16x8 a, u16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_16(F16, u16x8 a, u16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Hardware conversions (round to nearest even) of probabilities to 16 bits.
__device__ __forceinline__ unsigned short to_bits(BF16, float v) {
  return __builtin_bit_cast(unsigned short, static_cast<__bf16>(v));
}
__device__ __forceinline__ unsigned short to_bits(F16, float v) {
  return __builtin_bit_cast(unsigned short, static_cast<_Float16>(v));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Adds the 16-bit probabilities a lane holds for one tile (NP packed u16x8
// registers of 8 values) to the fp32 row sum acc with v_dot2c_f32_{bf16,f16}
// against (1, 1): one instruction per two values, accumulated straight into
// the running sum (no per-tile partial sums to clear and combine).  Summing
// the rounded P that the P.V product uses makes the weights applied to V sum
// to one exactly in the final division.
__device__ __forceinline__ float dot2_ones(BF16, unsigned pair, float acc) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair),
                                         __builtin_bit_cast(bf16x2, 0x3F803F80u), acc, false);
}
__device__ __forceinline__ float dot2_ones(F16, unsigned pair, float acc) {
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pair), __builtin_bit_cast(f16x2, 0x3C003C00u),
                                acc, false);
}
// Row sum of the first NU packed registers (all by default).
template <typename T, int NP, int NU = NP>
__device__ __forceinline__ float add_packed(const u16x8 (&pn)[NP], float acc) {
  static_assert(NU <= NP, "registers in use");
#pragma unroll
  for (int i = 0; i < NU; ++i) {
    const u32x4 w = __builtin_bit_cast(u32x4, pn[i]);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = dot2_ones(T{}, w[j], acc);
  }
  return acc;
}

__device__ __forceinline__ void fence() { __builtin_amdgcn_sched_barrier(0); }

// Max / sum of a value and the same value in lane ^ 32 (v_permlane32_swap:
// exchanges the upper half of the first operand with the lower half of the
// second, so the two results hold {x[l], x[l ^ 32]} in every lane).
// The maximum is one v_max_f32: fmaxf on the swapped words (integers to the
// compiler) would first quiet each of them with a v_max_f32 of its own.
__device__ __forceinline__ float max_with_other_half(float x) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  float m;
  asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(r[0]), "v"(r[1]));
  return m;
}
__device__ __forceinline__ float sum_with_other_half(float x) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Per-query value (32x32 result layout: query l % 32, equal in both lane
// halves) re-read for the 16x16 output layout through v_permlane16_swap of
// (x, x), which swaps the odd 16-lane rows of the first operand with the even
// rows of the second: lo = the value of query l % 16, hi = that of query
// 16 + l % 16.
__device__ __forceinline__ void by_query16(float x, float& lo, float& hi) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  lo = __uint_as_float(r[0]);
  hi = __uint_as_float(r[1]);
}

__device__ __forceinline__ f32x4 mfma_f32_16(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// LDS-DMA: each active lane copies the 16 bytes at gbase + voff (gbase
// wave-uniform, voff the lane's byte offset) to lds_base + 16 * lane
// (global_load_lds_dwordx4; lds_base is wave-uniform).  Completion is tracked
// by vmcnt only: callers wait with vm_wait() before the barrier that publishes
// the buffer.  Issued as inline assembly: the compiler cannot tell which LDS
// reads a copy feeds, and with the builtin it waits for every outstanding
// copy before the first LDS read after it - here, the K read right after the
// next tile's copies are issued.  M0 carries the LDS address; the one wait
// state after writing it is required before the copy reads it.
#define TTK_LDS(ptr) ((__attribute__((address_space(3))) void*)(ptr))
__device__ __forceinline__ void dma16(const void* gbase, unsigned voff, void* lds_base) {
  const unsigned lds = static_cast<unsigned>(reinterpret_cast<size_t>(TTK_LDS(lds_base)));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(gbase), "s"(lds)
               : "memory", "m0");
#pragma clang diagnostic pop
}
__device__ __forceinline__ void vm_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Key offset (inside a 32-key sub-block) held by register r of lane half h in
// the 32x32 MFMA result layout.
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// Work of one workgroup: a (batch, head) and one or two query tiles.
struct Work {
  int bh;
  int q_first;   // query tile of the first pass
  int q_second;  // query tile of the second pass (npass == 2)
  int npass;
  int chunk;     // key-split grid: chunk of q_first's key tiles (of nchunk)
  int nchunk;
};

__device__ __forceinline__ Work work_item(const AttnParams& p, bool causal) {
  const int id = blockIdx.x;
  int unit, bh;
  if (p.xcd_swizzle) {
    const int xcd = id & 7;
    const int j = id >> 3;
    const int hpx = p.BH >> 3;  // heads per XCD
    unit = j / hpx;
    bh = xcd + 8 * (j - unit * hpx);
  } else {
    unit = id / p.BH;
    bh = id - unit * p.BH;
  }
  Work w;
  w.bh = bh;
  w.chunk = 0;
  w.nchunk = 1;
  if (causal && p.split) {
    const unsigned e = p.unit_tab[unit];
    w.q_first = static_cast<int>(e & 1023u);
    w.chunk = static_cast<int>((e >> 10) & 7u);
    w.nchunk = static_cast<int>(e >> 13) + 1;
    w.q_second = w.q_first;
    w.npass = 1;
    return w;
  }
  if (causal && p.fold) {
    // Folded order: the first half of the units takes the heavy query tiles
    // (descending), the second half the light ones (ascending), so that the
    // workgroups i and i + CUs that share a CU hold tiles of opposite weight.
    const int half = (p.nq + 1) >> 1;
    w.q_first = unit < half ? p.nq - 1 - unit : unit - half;
  } else {
    w.q_first = causal ? p.nq - 1 - unit : unit;
  }
  w.q_second = unit;
  w.npass = (causal && p.pair && unit < w.q_first) ? 2 : 1;
  return w;
}

// Valid bits of the keys [k0, k0 + 64) that exist (key < S).
__device__ __forceinline__ uint64_t range_bits(int k0, int S) {
  const int n = S - k0;
  return n >= 64 ? ~uint64_t{0} : ((uint64_t{1} << n) - 1);
}

// Allowed-key bits of one 32-key sub-block (first key ks) for this lane, as
// a mask over the lane's registers: bit 8*(r/4) + r%4 <-> register r.
template <bool CAUSAL>
__device__ __forceinline__ uint32_t lane_allowed(uint32_t sub_valid, int ks, int qrow, int h) {
  uint32_t a = sub_valid;
  if constexpr (CAUSAL) {
    const int lim = qrow - ks;  // keys ks + i allowed for i <= lim
    const uint32_t cm = lim >= 31 ? 0xffffffffu : (lim < 0 ? 0u : ((2u << lim) - 1u));
    a &= cm;
  }
  return a >> (4 * h);
}

// Sets scores of disallowed keys to -inf (tile of NSB sub-blocks from k0;
// only the first NL are touched - the caller has not computed the others).
// BITSEL: per register, a signed one-bit field extract of the allowed bit
// gives an all-ones / all-zeros word and a bit-field insert selects the score
// or -inf - two VALU instructions and no compare, so no VCC write that the
// select has to wait for.  Otherwise a compare and a select per register
// (fewer live registers where the kernel is at its register limit).
template <int NSB, bool CAUSAL, bool BITSEL = true, int NL = NSB>
__device__ __forceinline__ void apply_mask(f32x16 (&s)[NSB], int k0, uint64_t kvalid, int qrow, int h) {
#pragma unroll
  for (int sb = 0; sb < NL; ++sb) {
    const uint32_t a =
        lane_allowed<CAUSAL>(static_cast<uint32_t>(kvalid >> (32 * sb)), k0 + sb * 32, qrow, h);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int bit = 8 * (r >> 2) + (r & 3);
      if constexpr (BITSEL) {
        const uint32_t keep = static_cast<uint32_t>(__builtin_amdgcn_sbfe(static_cast<int>(a), bit, 1));
        const uint32_t bits = __float_as_uint(s[sb][r]);
        s[sb][r] = __uint_as_float((bits & keep) | (0xff800000u & ~keep));
      } else {
        if (!((a >> bit) & 1u)) s[sb][r] = -INFINITY;
      }
    }
  }
}

// Waves per SIMD the register budget is sized for: two workgroups per CU,
// except fp32 head_dim 128, whose live state (64 accumulator + 64 Q registers
// + score tiles + staging) does not fit 256 registers; it runs one workgroup
// per CU with the accumulators in AGPRs; and 16-bit head_dim <= 64, sized for
// three (at most 168 VGPRs; the LDS of three workgroups fits).  The 16-bit
// loop is VALU-issue and latency bound, so the third workgroup pays: left to
// itself the compiler gave the causal head_dim-64 kernel 176 VGPRs (two
// workgroups per CU), and capping it at 168 - five registers spilled, reloaded
// only on the accumulator-rescale path - made config 4's attention 5-7 %
// faster.
template <bool F32, int D>
constexpr int kMinWaves = (D >= 128 && F32) ? 1 : ((!F32 && D <= 64) ? 3 : 2);

// ----------------------------------------------------------------------------
// fp32
// ----------------------------------------------------------------------------
template <int D, bool CAUSAL>
struct F32Cfg {
  // Keys per tile.  Head dim 128 runs one workgroup per CU; 64-key tiles fit
  // its LDS and halve the barriers (non-causal +5-7 %), but the causal
  // variants then spill 14-51 registers (with or without the diagonal
  // hand-off), so causal keeps 32-key tiles.
  static constexpr int BN = (D >= 128 && CAUSAL) ? 32 : 64;
  static constexpr int NSB = BN / 32;               // 32-key sub-blocks per tile
  static constexpr int CPR = D / 4;                 // 16-byte chunks per key row
  static constexpr int KS = D + 4;                  // LDS K row stride (floats, 16-byte pad)
  static constexpr int DB = D >= 32 ? D / 32 : 1;   // output blocks of 32 d-rows
  static constexpr int G = D / 8;                   // Q.K groups of 4 k-steps
  static constexpr int CHUNKS = BN * CPR;
  static constexpr int CPT = (CHUNKS + kThreads - 1) / kThreads;  // chunks per thread
};

template <int D>
struct VFrag32 {
  using type = float;
};
template <>
struct VFrag32<64> {
  using type = float2;
};
template <>
struct VFrag32<128> {
  using type = f32x4;
};

template <int D, bool CAUSAL, bool HAS_MASK>
__global__ __launch_bounds__(kThreads, (kMinWaves<true, D>)) void attn_fwd_f32_kernel(AttnParams p) {
  using C = F32Cfg<D, CAUSAL>;
  constexpr int BN = C::BN, NSB = C::NSB, CPR = C::CPR, KS = C::KS, DB = C::DB, CPT = C::CPT,
                G = C::G;
  using VF = typename VFrag32<D>::type;
  __shared__ __attribute__((aligned(16))) float smK[2][BN * KS];
  __shared__ __attribute__((aligned(16))) float smV[2][BN * D];
  // Causal hand-off (two-sub-block tiles): in the last key tile of a query
  // tile only wavefronts 2 (one sub-block) and 3 (two) have keys left, so
  // wavefront 0 - whose rows are complete by then - takes wavefront 3's
  // diagonal sub-block and passes its partial state through smX: per lane
  // 16*DB accumulator values, the row max and the lane half's row sum, as
  // 16-byte chunks at smX[(chunk * 64 + lane) * 4].
  constexpr bool kHandoff = CAUSAL && NSB == 2;
  // head_dim 8 and 16: P.V on 16x16x4 MFMAs (a 32x32 block would leave 3/4 or
  // half of its rows empty); the accumulator keeps the f32x16 storage,
  // elements 0-7 used.
  constexpr bool kNarrowD = D <= 16;
  constexpr int NX4 = 4 * DB + 1;
  __shared__ __attribute__((aligned(16))) float smX[kHandoff ? NX4 * 256 : 4];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int m = lane & 31;
  const int h = lane >> 5;

  const Work w = work_item(p, CAUSAL);
  // Twin grid (S <= 64, one key tile, rows only for wavefronts 0-1 of a
  // 128-query tile): workgroup i serves (batch, head) pairs 2i (wavefronts
  // 0-1, K/V buffer 0) and 2i + 1 (wavefronts 2-3, buffer 1).  The second
  // pair of the last workgroup may not exist (odd B*H): its wavefronts hold
  // no rows and read nothing.  Built into the non-causal kernels only (the
  // causal ones keep their register budget for the pairing and hand-off).
  constexpr bool kTwin = !CAUSAL && BN == 64;
  const bool twin = kTwin && p.twin != 0;
  const int slot = twin ? (wave >> 1) : 0;
  const int bh = twin ? 2 * static_cast<int>(blockIdx.x) + slot : w.bh;
  const bool head_live = bh < p.BH;
  const int b = head_live ? bh / p.H : 0;
  const int hh = head_live ? bh - b * p.H : 0;
  const int S = p.S;
  const float* __restrict__ Q = static_cast<const float*>(p.q) + b * p.qb + hh * p.qh;
  const float* __restrict__ K = static_cast<const float*>(p.k) + b * p.kb + hh * p.kh;
  const float* __restrict__ V = static_cast<const float*>(p.v) + b * p.vb + hh * p.vh;
  const uint8_t* __restrict__ M = HAS_MASK ? p.mask + b * p.mb : nullptr;

  // Every pass ends with a barrier after its last LDS read, so the next pass
  // may refill both buffers right away.
  f32x4 rk[C::CPT], rv[C::CPT];
  bool rm = false;
  bool staged = false;  // tile 0 of the coming pass already sits in rk / rv
  // Wave priority alternates tile by tile, in opposite phase for workgroups
  // whose index differs by the CU count.  The first grid fills every CU with
  // workgroups i and i + CUs; left to the age order, the older of the two
  // wins every issue conflict and finishes ~15 % earlier, and the younger
  // one runs alone to the end.  Alternating shares the CU evenly; a lone
  // workgroup keeps its CU nearly as busy, so the gain is small (~1 % at
  // S=1024).
  const int prio_phase = (static_cast<int>(blockIdx.x) / max(p.cu_count, 1)) & 1;
  // Folded grid: the heavy workgroup of a CU (the first CU-count workgroups)
  // keeps the high priority throughout and the light one fills its gaps
  // (0.5 % faster than alternating at config 2, S=512).
  const bool fold_fixed = p.fold != 0;
  const bool fold_heavy = prio_phase == 0;
  int tiles_done = 0;
  for (int pass = 0; pass < w.npass; ++pass) {
    const int qb = pass == 0 ? w.q_first : w.q_second;
    // First query of this wavefront (uniform); S, i.e. no rows, for the
    // missing second pair of a twin workgroup.
    const int q0 = !head_live ? S : qb * kBM + (twin ? (wave & 1) : wave) * 32;
    int qrow = q0 + m;                    // query of this lane (wavefront 3's on a hand-off)

    // B operand of S^T = K.Q^T: group g covers d = 8g..8g+7, lane half h
    // holds d = 8g+4h..8g+4h+3 (one element per k-step).  Pre-scaled into
    // exp2 units.
    f32x4 qf[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (qrow < S) {
        qf[g] = *reinterpret_cast<const f32x4*>(Q + qrow * p.qs + 8 * g + 4 * h) * p.scale_log2;
      } else {
        qf[g] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }

    const int kv_end = CAUSAL ? min(S, (qb + 1) * kBM) : S;
    const int ntiles = (kv_end + BN - 1) / BN;
    // Hand-off in this pass: the last tile starts half-way into the query
    // tile and wavefront 3 has rows (and keys of its second sub-block) < S.
    const bool handoff = kHandoff && (ntiles - 1) * BN == qb * kBM + 64 && qb * kBM + 96 < S;
    bool own_done = false;  // wavefront 0 stored its own rows early

    // Global loads of tile t into registers; rows past S read as zeros.
    auto gload = [&](int t) {
      const bool full = (t + 1) * BN <= S;
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int idx = tid + kThreads * i;
        if (C::CHUNKS % kThreads == 0 || idx < C::CHUNKS) {
          const int row = idx / CPR;
          const int c = idx - row * CPR;
          const int key = t * BN + row;
          if (full || key < S) {
            rk[i] = *reinterpret_cast<const f32x4*>(K + key * p.ks + 4 * c);
            rv[i] = *reinterpret_cast<const f32x4*>(V + key * p.vs + 4 * c);
          } else {
            rk[i] = f32x4{0.f, 0.f, 0.f, 0.f};
            rv[i] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
        }
      }
      if constexpr (HAS_MASK) {
        const int key = t * BN + lane;  // every wavefront reads the tile's mask bytes
        rm = lane < BN && key < S && M[key * p.ms] != 0;
      }
    };
    // Writes the staged tile into LDS buffer `buf`; returns the tile's
    // valid-key bits (key mask and key < S) as a wave-uniform 64-bit mask.
    auto lstore = [&](int buf, int t) -> uint64_t {
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int idx = tid + kThreads * i;
        if (C::CHUNKS % kThreads == 0 || idx < C::CHUNKS) {
          const int row = idx / CPR;
          const int c = idx - row * CPR;
          *reinterpret_cast<f32x4*>(&smK[buf][row * KS + 4 * c]) = rk[i];
          *reinterpret_cast<f32x4*>(&smV[buf][row * D + 4 * c]) = rv[i];
        }
      }
      if constexpr (HAS_MASK) {
        return __builtin_amdgcn_ballot_w64(rm);
      } else {
        return range_bits(t * BN, S);
      }
    };

    auto kread = [&](int buf, int sb, int g) -> f32x4 {
      const int row = sb * 32 + m;
      return *reinterpret_cast<const f32x4*>(&smK[buf][row * KS + 8 * g + 4 * h]);
    };
    auto vread = [&](int buf, int sb, int r) -> VF {
      const int krow = sb * 32 + acc_row(r, h);
      const float* vrow = &smV[buf][krow * D];
      if constexpr (DB == 1) {
        return (D >= 32 || m < D) ? vrow[m] : 0.0f;
      } else {
        return *reinterpret_cast<const VF*>(vrow + DB * m);
      }
    };

    float m_run = -INFINITY;
    float l_run = 0.0f;  // partial sum over this lane half's keys
    f32x16 acc[DB];
#pragma unroll
    for (int i = 0; i < DB; ++i) acc[i] = f32x16{};

    // One tile: S^T = K.Q^T, (mask), online softmax, O^T += V^T.P^T.
    // MASKED: apply the key / causal mask; PARTIAL: only the first of the two
    // sub-blocks holds keys this wavefront may see (the other is skipped).
    // Tiles with every sub-block live keep the branch-free, interleaved
    // sub-block chains even when masked.
    // SB0: index in the LDS tile of the first sub-block processed (k0 and
    // kvalid describe that sub-block onwards).
    auto tile = [&](auto masked_tag, auto partial_tag, auto sb0_tag, int buf, int k0, int nlive,
                    uint64_t kvalid) {
      constexpr bool MASKED = decltype(masked_tag)::value;
      constexpr bool PARTIAL = decltype(partial_tag)::value;
      constexpr int SB0 = decltype(sb0_tag)::value;
      // Live sub-blocks (nlive, 1 on partial tiles, which have two) as a
      // compile-time count: a run-time one puts every MFMA of sub-block 1
      // under its own branch, and the compiler copies its operands through
      // each (head_dim 64 causal: 337 -> 271 moves, config 2 -0.6 %).
      // Kernels that never run a partial tile at the measured shapes keep
      // the run-time form: non-causal (partial only at a ragged end) and
      // head dim 128 causal (one-sub-block tiles).  Their register
      // allocation moved with the shape of that dead path, and they ran
      // 0.8 % (non-causal head_dim 64) and 2-3 % (causal head_dim 128)
      // slower.
      constexpr bool kStaticLive = CAUSAL && D < 128;
      constexpr int NL = (PARTIAL && NSB == 2) ? 1 : NSB;
      auto live = [&](int sb) __attribute__((always_inline)) {
        return kStaticLive ? sb < NL : (!PARTIAL || sb < nlive);
      };
      f32x16 s[NSB];
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb)
        if (!kStaticLive || sb < NL) s[sb] = f32x16{};
      // ---- S^T = K . Q^T (K fragments read one group ahead) --------------
      f32x4 kf[NSB];
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb)
        if (live(sb)) kf[sb] = kread(buf, SB0 + sb, 0);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        f32x4 kn[NSB];
        if (g + 1 < G) {
#pragma unroll
          for (int sb = 0; sb < NSB; ++sb)
            if (live(sb)) kn[sb] = kread(buf, SB0 + sb, g + 1);
        }
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb) {
          if (!live(sb)) continue;
#pragma unroll
          for (int e = 0; e < 4; ++e) s[sb] = mfma_f32(kf[sb][e], qf[g][e], s[sb]);
        }
        if (g + 1 < G) {
#pragma unroll
          for (int sb = 0; sb < (kStaticLive ? NL : NSB); ++sb) kf[sb] = kn[sb];
        }
        fence();
      }
      constexpr int NS = kStaticLive ? NL : NSB;  // sub-blocks the softmax visits
      if constexpr (MASKED) apply_mask<NSB, CAUSAL, true, NS>(s, k0, kvalid, qrow, h);
      // ---- online softmax (exp2 domain) ------------------------------------
      float mt = s[0][0];
#pragma unroll
      for (int sb = 0; sb < NS; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[sb][r]);
      mt = max_with_other_half(mt);
      const float m_new = fmaxf(m_run, mt);
      // A fully masked row keeps m = -inf; use 0 so exp2(-inf - 0) = 0, never NaN.
      const float m_use = (MASKED && m_new == -INFINITY) ? 0.0f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      float ls = 0.0f;
#pragma unroll
      for (int sb = 0; sb < NS; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pr = fast_exp2(s[sb][r] - m_use);
          s[sb][r] = pr;
          ls += pr;
        }
      l_run = __builtin_fmaf(l_run, alpha, ls);
      if constexpr (kNarrowD) {
        float a_lo, a_hi;
        by_query16(alpha, a_lo, a_hi);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[0][e] *= a_lo;
          acc[0][4 + e] *= a_hi;
        }
      } else {
#pragma unroll
        for (int i = 0; i < DB; ++i) acc[i] *= alpha;
      }
      m_run = m_new;
      fence();
      if constexpr (kNarrowD) {
        // ---- head_dim <= 16: O^T += V^T . P^T on 16x16x4 MFMAs ------------
        // v_permlane16_swap of score registers r, r + 1 (keys k, k + 1 in lane
        // half 0, k + 4, k + 5 in half 1, k = 8(r/4) + r%4) leaves queries
        // 0-15 in the first and 16-31 in the second, with key k + {0,1,4,5}[g]
        // in 16-lane row g: the B operands of the two 16-query output blocks,
        // sharing one A operand V[key][d = l % 16].  Accumulator elements
        // 0-3 hold block 0 (d = 4(l/16) + e, query l % 16), 4-7 block 1;
        // for head_dim 8 the rows d >= 8 multiply zeros.
        const int g16 = lane >> 4;
        const int vkey = (g16 & 1) + 4 * (g16 >> 1);
        const bool d_ok = (lane & 15) < D;
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb) {
          if (!live(sb)) continue;
          const float* vb = &smV[buf][((SB0 + sb) * 32 + vkey) * D + (lane & 15 & (D - 1))];
#pragma unroll
          for (int r = 0; r < 16; r += 2) {
            const float va = d_ok ? vb[(8 * (r >> 2) + (r & 3)) * D] : 0.0f;
            const auto pq = __builtin_amdgcn_permlane16_swap(__float_as_uint(s[sb][r]),
                                                             __float_as_uint(s[sb][r + 1]), false, false);
            f32x4 lo = {acc[0][0], acc[0][1], acc[0][2], acc[0][3]};
            f32x4 hi = {acc[0][4], acc[0][5], acc[0][6], acc[0][7]};
            lo = mfma_f32_16(va, __uint_as_float(pq[0]), lo);
            hi = mfma_f32_16(va, __uint_as_float(pq[1]), hi);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              acc[0][e] = lo[e];
              acc[0][4 + e] = hi[e];
            }
          }
        }
        fence();
        return;
      }
      // ---- O^T += V^T . P^T (V fragments read one k-step ahead) -----------
      const int nsteps = kStaticLive ? NL * 16 : (PARTIAL ? nlive : NSB) * 16;
      VF vf = vread(buf, SB0, 0);
#pragma unroll
      for (int idx = 0; idx < NSB * 16; ++idx) {
        // Fixed trip count (fully unrolled, so s[][] stays in registers); the
        // dead sub-blocks' k-steps are skipped (at compile time below head
        // dim 128).
        if (idx < nsteps) {
          const int sb = idx >> 4;
          const int r = idx & 15;
          VF vn{};
          if (idx + 1 < NSB * 16 && idx + 1 < nsteps) {
            vn = vread(buf, SB0 + ((idx + 1) >> 4), (idx + 1) & 15);
          }
          const float pr = s[sb][r];
          if constexpr (DB == 1) {
            acc[0] = mfma_f32(vf, pr, acc[0]);
          } else if constexpr (DB == 2) {
            acc[0] = mfma_f32(vf.x, pr, acc[0]);
            acc[1] = mfma_f32(vf.y, pr, acc[1]);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = mfma_f32(vf[i], pr, acc[i]);
          }
          vf = vn;
        }
        fence();
      }
    };

    // O = acc / l for this lane's row.
    auto epilogue = [&]() __attribute__((always_inline)) {
      const float lt = sum_with_other_half(l_run);
      if constexpr (kNarrowD) {
        // Block 0: query base + l % 16, block 1: base + 16 + l % 16; d = 4(l/16) + e.
        float lt_lo, lt_hi;
        by_query16(lt, lt_lo, lt_hi);
        const float inv_lo = lt_lo > 0.0f ? 1.0f / lt_lo : 0.0f;
        const float inv_hi = lt_hi > 0.0f ? 1.0f / lt_hi : 0.0f;
        const int base = qrow - m;  // first query of the rows held (uniform)
        const int d0 = 4 * (lane >> 4);
        float* __restrict__ O = static_cast<float*>(p.out) + b * p.ob + hh * p.oh + d0;
        const int r_lo = base + (lane & 15), r_hi = r_lo + 16;
        if (d0 >= D) return;  // head_dim 8: d-rows 8-15 are empty
        if (r_lo < S)
          *reinterpret_cast<f32x4*>(O + r_lo * p.os) =
              f32x4{acc[0][0] * inv_lo, acc[0][1] * inv_lo, acc[0][2] * inv_lo, acc[0][3] * inv_lo};
        if (r_hi < S)
          *reinterpret_cast<f32x4*>(O + r_hi * p.os) =
              f32x4{acc[0][4] * inv_hi, acc[0][5] * inv_hi, acc[0][6] * inv_hi, acc[0][7] * inv_hi};
        return;
      }
      const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
      if (qrow < S) {
        float* __restrict__ O = static_cast<float*>(p.out) + b * p.ob + hh * p.oh + qrow * p.os;
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
          // Block i of the accumulator holds d = DB*row + i; register 4*j4+e
          // holds row 8*j4 + 4h + e, so a lane's d-values form one run of 4*DB.
          const int d0 = DB * (8 * j4 + 4 * h);
          if (D < 32 && d0 >= D) continue;
          float vals[4 * DB];
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int i = 0; i < DB; ++i) vals[DB * e + i] = acc[i][4 * j4 + e] * inv;
#pragma unroll
          for (int c = 0; c < DB; ++c) {
            *reinterpret_cast<f32x4*>(O + d0 + 4 * c) =
                f32x4{vals[4 * c], vals[4 * c + 1], vals[4 * c + 2], vals[4 * c + 3]};
          }
        }
      }
    };

    // Twin grid: both pairs' only key tile, pair 2i into buffer 0 and 2i + 1
    // into buffer 1, every load issued before the first LDS store; returns
    // this wavefront's valid-key bits.
    auto twin_stage = [&]() -> uint64_t {
      f32x4 tk[2][CPT], tv[2][CPT];
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const int bhx = 2 * static_cast<int>(blockIdx.x) + s2;
        const bool live = bhx < p.BH;
        const int bx = live ? bhx / p.H : 0;
        const int hx = live ? bhx - bx * p.H : 0;
        const float* Kx = static_cast<const float*>(p.k) + bx * p.kb + hx * p.kh;
        const float* Vx = static_cast<const float*>(p.v) + bx * p.vb + hx * p.vh;
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          const int idx = tid + kThreads * i;
          if (C::CHUNKS % kThreads == 0 || idx < C::CHUNKS) {
            const int row = idx / CPR;  // key: the tile starts at key 0
            const int c = idx - row * CPR;
            if (live && row < S) {
              tk[s2][i] = *reinterpret_cast<const f32x4*>(Kx + row * p.ks + 4 * c);
              tv[s2][i] = *reinterpret_cast<const f32x4*>(Vx + row * p.vs + 4 * c);
            } else {
              tk[s2][i] = f32x4{0.f, 0.f, 0.f, 0.f};
              tv[s2][i] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
          }
        }
      }
      bool valid = head_live && lane < S;
      if constexpr (HAS_MASK) valid = valid && M[lane * p.ms] != 0;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
          const int idx = tid + kThreads * i;
          if (C::CHUNKS % kThreads == 0 || idx < C::CHUNKS) {
            const int row = idx / CPR;
            const int c = idx - row * CPR;
            *reinterpret_cast<f32x4*>(&smK[s2][row * KS + 4 * c]) = tk[s2][i];
            *reinterpret_cast<f32x4*>(&smV[s2][row * D + 4 * c]) = tv[s2][i];
          }
        }
      }
      return HAS_MASK ? __builtin_amdgcn_ballot_w64(valid) : range_bits(0, S);
    };

    uint64_t kvalid;
    if (kTwin && twin) {
      kvalid = twin_stage();
    } else {
      if (!staged) gload(0);
      kvalid = lstore(0, 0);
    }
    __syncthreads();
    staged = false;

    for (int t = 0; t < ntiles; ++t) {
      const int buf = twin ? slot : (t & 1);
      if (fold_fixed ? fold_heavy : (((tiles_done + t) & 1) == prio_phase)) {
        __builtin_amdgcn_s_setprio(1);
      } else {
        __builtin_amdgcn_s_setprio(0);
      }
      if (t + 1 < ntiles) {
        gload(t + 1);
      } else if (pass + 1 < w.npass) {
        gload(0);  // the next pass's key tile 0 (same head, same rows)
        staged = true;
      }
      const int k0 = t * BN;
      if constexpr (kHandoff) {
        if (handoff && t == ntiles - 1 && wave == 0) {
          // Own rows are complete (their last keys were in tile t - 1): store
          // them, then run wavefront 3's second sub-block of this tile on
          // wavefront 3's rows from a fresh state and hand the state over.
          const int frow = qb * kBM + 96 + m;
          f32x4 fq[G];
#pragma unroll
          for (int g = 0; g < G; ++g) {
            fq[g] = frow < S ? *reinterpret_cast<const f32x4*>(Q + frow * p.qs + 8 * g + 4 * h) * p.scale_log2
                             : f32x4{0.f, 0.f, 0.f, 0.f};
          }
          epilogue();
          own_done = true;
          qrow = frow;
#pragma unroll
          for (int g = 0; g < G; ++g) qf[g] = fq[g];
          m_run = -INFINITY;
          l_run = 0.0f;
#pragma unroll
          for (int i = 0; i < DB; ++i) acc[i] = f32x16{};
          tile(std::true_type{}, std::true_type{}, std::integral_constant<int, 1>{}, buf, k0 + 32, 1,
               kvalid >> 32);
#pragma unroll
          for (int j = 0; j < 4 * DB; ++j) {
            const int i = j >> 2, r0 = 4 * (j & 3);
            *reinterpret_cast<f32x4*>(&smX[(j * 64 + lane) * 4]) =
                f32x4{acc[i][r0], acc[i][r0 + 1], acc[i][r0 + 2], acc[i][r0 + 3]};
          }
          *reinterpret_cast<f32x4*>(&smX[(4 * DB * 64 + lane) * 4]) = f32x4{m_run, l_run, 0.f, 0.f};
        }
      }
      if (q0 < S && (!CAUSAL || k0 <= q0 + 31) && !own_done) {
        // Leading sub-blocks that hold any key this wavefront may see.
        int nlive = NSB;
#pragma unroll
        for (int sb = NSB - 1; sb >= 0; --sb) {
          const int ks = k0 + sb * 32;
          if (ks >= S || (CAUSAL && ks > q0 + 31)) nlive = sb;
        }
        // On a hand-off wavefront 3 keeps only the first sub-block of the last
        // tile; its second sub-block's keys are cleared from the valid bits,
        // since the causal mask alone would leave them at score 0.
        uint64_t kv = kvalid;
        if (kHandoff && handoff && t == ntiles - 1 && wave == 3) {
          nlive = 1;
          kv &= 0xffffffffull;
        }
        const bool need_mask = HAS_MASK || (k0 + BN > S) || (CAUSAL && k0 + BN - 1 > q0);
        if (need_mask) {
          if (nlive < NSB) {
            tile(std::true_type{}, std::true_type{}, std::integral_constant<int, 0>{}, buf, k0, nlive, kv);
          } else {
            tile(std::true_type{}, std::false_type{}, std::integral_constant<int, 0>{}, buf, k0, NSB, kv);
          }
        } else {
          tile(std::false_type{}, std::false_type{}, std::integral_constant<int, 0>{}, buf, k0, NSB, kvalid);
        }
      }
      if (t + 1 < ntiles) kvalid = lstore(buf ^ 1, t + 1);
      __syncthreads();
    }

    if constexpr (kHandoff) {
      if (handoff && wave == 3) {
        // Merge wavefront 0's state for the second sub-block of the last
        // tile (written before the loop's final barrier).
        const f32x4 ml = *reinterpret_cast<const f32x4*>(&smX[(4 * DB * 64 + lane) * 4]);
        const float mx = fmaxf(m_run, ml[0]);
        const float mu = mx == -INFINITY ? 0.0f : mx;
        const float a = fast_exp2(m_run - mu);
        const float bb = fast_exp2(ml[0] - mu);
        l_run = __builtin_fmaf(l_run, a, ml[1] * bb);
        if constexpr (kNarrowD) {
          // Factors per output block (queries l % 16 and 16 + l % 16).
          float a_lo, a_hi, b_lo, b_hi;
          by_query16(a, a_lo, a_hi);
          by_query16(bb, b_lo, b_hi);
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const float fa = j == 0 ? a_lo : a_hi, fb = j == 0 ? b_lo : b_hi;
            const f32x4 x = *reinterpret_cast<const f32x4*>(&smX[(j * 64 + lane) * 4]);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[0][4 * j + e] = __builtin_fmaf(acc[0][4 * j + e], fa, x[e] * fb);
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4 * DB; ++j) {
            const int i = j >> 2, r0 = 4 * (j & 3);
            const f32x4 x = *reinterpret_cast<const f32x4*>(&smX[(j * 64 + lane) * 4]);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][r0 + e] = __builtin_fmaf(acc[i][r0 + e], a, x[e] * bb);
          }
        }
        m_run = mx;
      }
    }
    if (!own_done) epilogue();
    tiles_done += ntiles;
  }
  __builtin_amdgcn_s_setprio(0);
}

// ----------------------------------------------------------------------------
// fp32, short sequences: S <= 64, non-causal, head_dim 32 / 64
// ----------------------------------------------------------------------------
// The whole 64-key tile of one (batch, head) fits a wavefront's registers as
// MFMA operands (head_dim 64: K 64 + V 64 + Q 32 VGPRs), so one wavefront
// serves one (batch, head, 32-query half) on its own: no barrier.  The grid
// is persistent (two workgroups per CU); wavefront gw walks the items gw,
// gw + W, ... (item = 2 * (batch * H + head) + half, so the two halves of a
// head run side by side in one workgroup and the second K/V read hits L2).
// While the current item's softmax and P.V run, the next item's K and Q are
// in flight, and the next V while the current rows are stored.
//
// Global traffic is row-coalesced: K, Q and O move as whole rows (64 lanes x
// 16 bytes = 1 KB of consecutive rows per instruction) and are re-laid out
// through an LDS region private to the wavefront (64 rows, 16 KB at head_dim
// 64; 16-byte chunks XOR-swizzled by row so both layouts access LDS without
// bank conflicts): K and Q into the MFMA operand layout (key or query per lane,
// 4 head dims per register), O back from the accumulator layout.  The MFMA
// fragments read with a lane stride of a whole row (32 rows x 32 bytes per
// instruction) cost ~8 % more time at config 5b than whole rows.  V is read
// straight into its operand layout, 256 contiguous bytes per half-wavefront.
// Fragment layouts, accumulation order and softmax are those of
// attn_fwd_f32_kernel's single-tile pass, so the two kernels give identical
// results.
// MASKED: scores need the key mask (HAS_MASK, or S < 64 leaves padded keys).
template <int D, bool HAS_MASK, bool MASKED>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_f32_short_kernel(AttnParams p) {
  static_assert(D == 32 || D == 64, "short-sequence kernel: head_dim 32 or 64");
  constexpr int NSB = 2, DB = D / 32, G = D / 8;
  constexpr int CPR = D / 4;        // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;     // rows per row-coalesced instruction
  constexpr int NI = 32 / RPI;      // instructions per 32 rows (== G)
  static_assert(NI == G, "32 rows take as many instructions as Q has fragments");
  using VF = typename VFrag32<D>::type;
  __shared__ __attribute__((aligned(16))) float smem[kThreads / 64][64 * D];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int m = lane & 31;
  const int h = lane >> 5;
  const int S = p.S;
  const int hshift = S > 32 ? 1 : 0;  // 32-query halves per head: 2 or 1
  const int items = p.BH << hshift;
  const int stride = static_cast<int>(gridDim.x) * (kThreads / 64);
  int item = static_cast<int>(blockIdx.x) * (kThreads / 64) + wave;
  if (item >= items) return;
  float* const region = smem[wave];

  // Every global access is a buffer access whose resource covers exactly the
  // rows < S of one head (the host checks row stride >= head_dim and that
  // the offsets of all 64 rows a lane may address stay below 2^31): rows past
  // S read as zeros and are not written,
  // without a branch.  The range check covers the VGPR offset (plus the
  // instruction offset) but not soffset, so the row part of every offset is
  // in the VGPR.  The loads of the next item are issued unconditionally -
  // after the last item with an empty resource, which fetches nothing - so
  // every wait count is exact on the one path through the loop and waits only
  // for the operands it needs.
  auto head_of = [&](int it, int& b, int& hh) {
    const int bh = it >> hshift;
    b = bh / p.H;
    hh = bh - b * p.H;
  };
  auto rsrc = [&](const void* base, int64_t bo, int64_t ho, int64_t rs, int it, bool live) {
    int b, hh;
    head_of(it, b, hh);
    const float* ptr = static_cast<const float*>(base) + b * bo + hh * ho;
    const int bytes = live ? static_cast<int>(((S - 1) * rs + D) * 4) : 0;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ptr), static_cast<short>(0), bytes, 0x00020000);
  };
  // Row-coalesced lane position: instruction j covers rows RPI*j .. RPI*j + RPI - 1.
  const int crow = lane / CPR;
  const int cchunk = lane % CPR;
  // LDS float index of (row, 16-byte chunk) in the wavefront's region.
  auto slot = [](int row, int chunk) { return row * D + 4 * (chunk ^ (row & (CPR - 1))); };
  const int voff0 = static_cast<int>((4 * h * p.vs + DB * m) * 4);

  f32x4 kst[NSB][NI], qst[NI];  // K and Q as loaded (row-coalesced)
  VF vf[NSB][16];
  int key_ok = 0;  // HAS_MASK: this lane's key (= lane) exists and is not masked

  // 32 rows from row0 of one head, row-coalesced (the row offsets of the
  // instructions are added at each load, not hoisted into live registers).
  auto load_rows = [&](f32x4 (&dst)[NI], const __amdgpu_buffer_rsrc_t& rs, int64_t row_stride, int row0) {
    int off = static_cast<int>(((row0 + crow) * row_stride + 4 * cchunk) * 4);
    asm volatile("" : "+v"(off));
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      dst[j] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + static_cast<int>(RPI * j * row_stride * 4), 0, 0));
    }
  };
  auto load_q = [&](int it, bool live) {
    const auto rq = rsrc(p.q, p.qb, p.qh, p.qs, it, live);
    load_rows(qst, rq, p.qs, (it & hshift) << 5);
    if constexpr (HAS_MASK) {
      int b, hh;
      head_of(it, b, hh);
      const int bytes = live ? static_cast<int>((S - 1) * p.ms + 1) : 0;
      const auto rm = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p.mask + b * p.mb),
                                                        static_cast<short>(0), bytes, 0x00020000);
      key_ok = __builtin_amdgcn_raw_buffer_load_b8(rm, static_cast<int>(lane * p.ms), 0, 0);
    }
  };
  auto load_k = [&](int it, bool live, int sb) {
    const auto rk = rsrc(p.k, p.kb, p.kh, p.ks, it, live);
    load_rows(kst[sb], rk, p.ks, sb * 32);
  };
  // V as the A operand of O^T += V^T . P^T: register (sb, r) holds key
  // sb * 32 + acc_row(r, h), head dims DB * m .. DB * m + DB - 1.  The
  // per-register row offsets are added at each load (an opaque copy of the
  // lane offset keeps them from being hoisted into 32 live registers).
  auto load_v = [&](int it, bool live, int sb) {
    const auto rv = rsrc(p.v, p.vb, p.vh, p.vs, it, live);
    int voff = voff0;
    asm volatile("" : "+v"(voff));
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int off = voff + static_cast<int>((sb * 32 + acc_row(r, 0)) * p.vs * 4);
      if constexpr (DB == 1) {
        vf[sb][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rv, off, 0, 0));
      } else {
        vf[sb][r] = __builtin_bit_cast(VF, __builtin_amdgcn_raw_buffer_load_b64(rv, off, 0, 0));
      }
    }
  };
  // Row-coalesced registers -> LDS region rows row0 .. row0 + 31.
  auto put_rows = [&](const f32x4 (&src)[NI], int row0) {
#pragma unroll
    for (int j = 0; j < NI; ++j) *reinterpret_cast<f32x4*>(&region[slot(row0 + RPI * j + crow, cchunk)]) = src[j];
  };
  // MFMA operand fragments from the region: group g of lane (m, h) holds row
  // row0 + m, head dims 8g + 4h .. 8g + 4h + 3 (16-byte chunk 2g + h).
  auto get_frags = [&](f32x4 (&dst)[G], int row0) {
#pragma unroll
    for (int g = 0; g < G; ++g) dst[g] = *reinterpret_cast<const f32x4*>(&region[slot(row0 + m, 2 * g + h)]);
  };

  // Same memory-instruction sequence as the loop body issues before its head
  // (K, Q, NI row stores, V; the stores here go to an empty resource and
  // write nothing): vmcnt counts loads and stores together, so the wait
  // counts the compiler derives at the loop head then fit both paths into it
  // and none of them waits for the previous item's stores.
  load_k(item, true, 0);
  load_k(item, true, 1);
  load_q(item, true);
  {
    const auto none = __builtin_amdgcn_make_buffer_rsrc(p.out, static_cast<short>(0), 0, 0x00020000);
#pragma unroll
    for (int j = 0; j < NI; ++j) __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, none, 16 * j, 0, 0);
  }
  load_v(item, true, 0);
  load_v(item, true, 1);
  while (true) {
    const int next_raw = item + stride;
    const bool more = next_raw < items;
    const int next = more ? next_raw : item;
    const int half_row0 = (item & hshift) << 5;
    const int qrow = half_row0 + m;
    const uint64_t kv = HAS_MASK ? __builtin_amdgcn_ballot_w64(lane < S && key_ok != 0) : range_bits(0, S);
    const auto ro = [&] {
      int b, hh;
      head_of(item, b, hh);
      float* ptr = static_cast<float*>(p.out) + b * p.ob + hh * p.oh;
      const int bytes = static_cast<int>(((S - 1) * p.os + D) * 4);
      return __builtin_amdgcn_make_buffer_rsrc(ptr, static_cast<short>(0), bytes, 0x00020000);
    }();

    // ---- S^T = K . Q^T (sub-block by sub-block; each accumulates over d in
    // the same order as the tiled kernel).  Q, then K, passes through the LDS
    // region; one wavefront's LDS accesses complete in program order, so the
    // K rows overwrite Q's only after Q's fragments are read.
    f32x4 qf[G];
    put_rows(qst, 0);
    get_frags(qf, 0);
    put_rows(kst[0], 0);
    put_rows(kst[1], 32);
#pragma unroll
    for (int g = 0; g < G; ++g) qf[g] *= p.scale_log2;
    f32x16 s[NSB];
    f32x4 kf[NSB][G];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) get_frags(kf[sb], 32 * sb);
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
      s[sb] = f32x16{};
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) s[sb] = mfma_f32(kf[sb][g][e], qf[g][e], s[sb]);
    }
    fence();
    // The staging registers of K are free since its rows went to LDS.
    load_k(next, more, 0);
    load_k(next, more, 1);
    fence();

    // ---- softmax (exp2 domain, one tile: the running state starts empty) ----
    if constexpr (MASKED) apply_mask<NSB, false, false>(s, 0, kv, qrow, h);
    float mt = s[0][0];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[sb][r]);
    mt = fmaxf(-INFINITY, max_with_other_half(mt));
    // A fully masked row keeps m = -inf; use 0 so exp2(-inf - 0) = 0, never NaN.
    const float m_use = (MASKED && mt == -INFINITY) ? 0.0f : mt;
    float ls = 0.0f;
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = fast_exp2(s[sb][r] - m_use);
        s[sb][r] = pr;
        ls += pr;
      }
    fence();

    // ---- O^T = V^T . P^T ----------------------------------------------------
    f32x16 acc[DB];
#pragma unroll
    for (int i = 0; i < DB; ++i) acc[i] = f32x16{};
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = s[sb][r];
        if constexpr (DB == 1) {
          acc[0] = mfma_f32(vf[sb][r], pr, acc[0]);
        } else {
          acc[0] = mfma_f32(vf[sb][r].x, pr, acc[0]);
          acc[1] = mfma_f32(vf[sb][r].y, pr, acc[1]);
        }
      }
      fence();
    }
    load_q(next, more);
    fence();

    // ---- O = acc / l, through the LDS region into whole rows -----------------
    const float lt = sum_with_other_half(ls);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
#pragma unroll
    for (int j4 = 0; j4 < 4; ++j4) {
      // Block i holds d = DB * row + i; register 4 * j4 + e holds row 8 * j4 + 4h + e,
      // so a lane's d-values for one j4 form one run of 4 * DB (chunks d0 / 4 ..).
      const int d0 = DB * (8 * j4 + 4 * h);
      float vals[4 * DB];
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < DB; ++i) vals[DB * e + i] = acc[i][4 * j4 + e] * inv;
#pragma unroll
      for (int c = 0; c < DB; ++c) {
        *reinterpret_cast<f32x4*>(&region[slot(m, d0 / 4 + c)]) =
            f32x4{vals[4 * c], vals[4 * c + 1], vals[4 * c + 2], vals[4 * c + 3]};
      }
    }
    const int ooff = static_cast<int>(((half_row0 + crow) * p.os + 4 * cchunk) * 4);
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const f32x4 o4 = *reinterpret_cast<const f32x4*>(&region[slot(RPI * j + crow, cchunk)]);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o4), ro,
                                             ooff + static_cast<int>(RPI * j * p.os * 4), 0, 0);
    }
    fence();
    load_v(next, more, 0);
    load_v(next, more, 1);
    if (!more) break;
    item = next;
  }
}

// ----------------------------------------------------------------------------
// bf16 / fp16
// ----------------------------------------------------------------------------
template <int D, int BNK = 64>
struct H16Cfg {
  static constexpr int DK = D < 16 ? 16 : D;         // contraction length of Q.K (zero padded)
  static constexpr int BN = BNK;                     // keys per tile (64, or 32)
  static constexpr int NSB = BN / 32;
  static constexpr int CPR = D / 8;                  // 16-byte chunks per key row (8 elems)
  static constexpr int KS = DK + 8;                  // LDS K row stride (elements, 16-byte pad)
  static constexpr int NDB = (D + 31) / 32;          // output blocks of 32 d-rows
  static constexpr int G = DK / 16;                  // Q.K k-steps of 16
  // LDS V row stride (elements) of the row-major V tile.  The 4 key rows one
  // half-wave reads with the transposing load must fall on disjoint banks.
  // Rows stay unpadded and, for head_dim 64 and 128 (VSWZ), 32-column blocks
  // are permuted per row instead: 16-byte chunk c of row r sits in slot
  // c ^ 4*((r >> 1) & 1) (head_dim 64: 128-byte rows, rows r and r + 2 share
  // banks) or c ^ 4*(r & 3) (head_dim 128: 256-byte rows, every row starts on
  // bank 0).  That copies 8 / 16 chunks per row instead of the 12 / 20 of a
  // padded stride.
  static constexpr bool VSWZ = D == 64 || D == 128;
  static constexpr int VS = D;
  static constexpr int VCH = VS / 8;                 // 16-byte chunks per LDS V row
  // Head dims below 32 read up to d = 31 with the transposing load (rows
  // d >= D of the result are never stored); the slack keeps those reads of
  // the last rows inside the buffer.
  static constexpr int VSLACK = 32;
  static constexpr int NSTEP = NSB * 2 * NDB;        // P.V MFMAs per tile
  // Operand prefetch distances (ring depths) of the K and V fragments.
  static constexpr int PDK = 2;
  static constexpr int PDV = 2;
};

// Transposing LDS read (ds_read_b64_tr_b16).  Within each group of 16 lanes,
// lane 4a+c receives element c of the 8-byte rows addressed by lanes a, a+4,
// a+8 and a+12 of the group (in that order).
__device__ __forceinline__ u16x4 lds_read_tr16(const unsigned short* p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(p));
  return __builtin_bit_cast(u16x4, v);
}

// BNK = 32 (head_dim 128 only): 32-key tiles, sized for three workgroups per
// CU, run with the single-score-buffer body and never key-split - for the
// shorter launches, where more resident wavefronts hide more latency than the
// extra per-tile work costs.
template <typename T, int D, bool CAUSAL, bool HAS_MASK, int BNK = 64>
__global__ __launch_bounds__(kThreads, (BNK == 32 ? (D <= 64 ? 4 : 3) : kMinWaves<false, D>)) void attn_fwd_h16_kernel(AttnParams p) {
  using C = H16Cfg<D, BNK>;
  constexpr int BN = C::BN, NSB = C::NSB, CPR = C::CPR, KS = C::KS,
                NDB = C::NDB, VS = C::VS, VCH = C::VCH, G = C::G, NSTEP = C::NSTEP,
                PDK = C::PDK, PDV = C::PDV;
  static_assert(BNK == 64 || (BNK == 32 && D >= 32), "32-key tiles are built for head_dim 32, 64 and 128");
  // The K region also stages the output tile (4 wavefronts x 32 rows of D + 8).
  constexpr int KBUF = (BN * KS > 64 * (D + 8)) ? BN * KS : 64 * (D + 8);
  __shared__ __attribute__((aligned(16))) unsigned short smK[2][KBUF];
  __shared__ __attribute__((aligned(16))) unsigned short smV[2][BN * VS + C::VSLACK];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int m = lane & 31;
  const int h = lane >> 5;

  const Work w = work_item(p, CAUSAL);
  const int b = w.bh / p.H;
  const int hh = w.bh - b * p.H;
  const int S = p.S;
  using St = unsigned short;
  const St* __restrict__ Q = static_cast<const St*>(p.q) + b * p.qb + hh * p.qh;
  const St* __restrict__ K = static_cast<const St*>(p.k) + b * p.kb + hh * p.kh;
  const St* __restrict__ V = static_cast<const St*>(p.v) + b * p.vb + hh * p.vh;
  const uint8_t* __restrict__ M = HAS_MASK ? p.mask + b * p.mb : nullptr;

  // The row max is taken on raw scores, which needs a positive scale: a
  // negative scale is folded into Q as an exact sign flip.
  const bool negate = p.scale_log2 < 0.0f;
  float c = negate ? -p.scale_log2 : p.scale_log2;
  // Scale 0 (uniform weights): masked scores are -inf and -inf * 0 is NaN,
  // so 2^-100 stands in.  Masked scores stay -inf, and every allowed score
  // (|s| < 2^75) gives an exp2 argument below 2^-25, so P = 1 exactly.
  if (c == 0.0f) c = 0x1p-100f;
  // The reference max moves once a row's max passes it by more than 8 / c
  // (8 in log2 units, so P <= 2^8).
  float lag = 8.0f / c;
  // Both are wave-uniform: kept in SGPRs (a VOP3 instruction reads one SGPR
  // operand), they leave two more VGPRs to the loop.
  c = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(c)));
  lag = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(lag)));
  const unsigned short sign = negate ? 0x8000u : 0u;

  // K: LDS-DMA into padded rows of KCH 16-byte chunks; DMA instruction j
  // fills chunks [64j, 64j + 64) and the instructions are dealt round-robin
  // to the wavefronts.  A lane landing on the pad chunk - and for head_dim 8
  // on the zero-padded d 8..15, which meets zero Q entries - copies chunk 0
  // again; keys past S copy row S-1 (finite data that the mask neutralises).
  // The (row, chunk) a lane copies is the same for every tile, so its element
  // byte offset from the tile's first key row is computed once (row < 64 and
  // the ABI bounds the key stride below 2^25 elements, so 2 * (row * ks + col)
  // fits 32 bits); lanes past the tile are marked by pos >= BN * KCH.
  constexpr int KCH = KS / 8;
  constexpr int NK = (BN * KCH + 63) / 64;
  constexpr int NW = kThreads / 64;
  constexpr int KPW = (NK + NW - 1) / NW;
  unsigned koff[KPW];
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    const int pos = 64 * (wave + NW * i) + lane;
    const int row = pos / KCH;
    const int cc = pos - row * KCH;
    koff[i] = 2u * static_cast<unsigned>(row * static_cast<int>(p.ks) + 8 * (cc < CPR ? cc : 0));
  }
  // V: LDS-DMA into unpadded row-major rows of VCH 16-byte chunks (read back
  // with the transposing load); with VSWZ the lane filling slot (row, cc)
  // copies chunk cc ^ vswz(row).
  static_assert(VCH == CPR, "V rows are unpadded");
  auto vswz = [](int row) { return C::VSWZ ? (D == 128 ? 4 * (row & 3) : 4 * ((row >> 1) & 1)) : 0; };
  constexpr int NV = (BN * VCH + 63) / 64;
  constexpr int VPW = (NV + NW - 1) / NW;
  unsigned voff[VPW];
#pragma unroll
  for (int i = 0; i < VPW; ++i) {
    const int pos = 64 * (wave + NW * i) + lane;
    const int row = pos / VCH;
    const int cc = pos - row * VCH;
    voff[i] = 2u * static_cast<unsigned>(row * static_cast<int>(p.vs) + 8 * (cc ^ vswz(row)));
  }
  // Per-lane base of the transposing V reads: lane i of 16-lane group g
  // addresses key row 4*(g/2) + i/4 and d = 16*(g%2) + 4*(i%4), so lane
  // (m, h) receives V[4h + 0..3][m] (see lds_read_tr16); P.V step (kstep,
  // db) adds 16*kstep rows and 32*db columns, its upper four keys 8 rows.
  // With VSWZ the rows a lane reads all share their low two bits with lane
  // bits 2-3 (16*kstep and 8 rows leave them alone), so the block permutation
  // is one per-lane XOR of the db offset.
  const int vbase = (4 * h + ((lane & 15) >> 2)) * VS + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const int vflip = C::VSWZ ? (D == 128 ? 32 * ((lane >> 2) & 3) : 32 * ((lane >> 3) & 1)) : 0;

  {
    // 16-bit workgroups run one query tile (never paired: a second pass costs
    // this kernel more in register pressure than it gains in balance).
    const int qb = w.q_first;
    const int q0 = qb * kBM + wave * 32;
    const int qrow = q0 + m;

    // B operand of S^T = K.Q^T: k-step g covers d = 16g..16g+15, lane half h
    // holds d = 16g+8h..16g+8h+7.
    u16x8 qf[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int d = 16 * g + 8 * h;
      if (qrow < S && d < D) {
        qf[g] = *reinterpret_cast<const u16x8*>(Q + qrow * p.qs + d) ^ sign;
      } else {
        qf[g] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }

    const int kv_end = CAUSAL ? min(S, (qb + 1) * kBM) : S;
    const int ntiles = (kv_end + BN - 1) / BN;

    bool rm = false;
    auto dma_k = [&](int buf, int t) __attribute__((always_inline)) {
      if constexpr (HAS_MASK) {
        const int key = t * BN + lane;
        rm = lane < BN && key < S && M[key * p.ms] != 0;
      }
      const St* kt = K + static_cast<int64_t>(t) * BN * p.ks;
      const bool ragged = (t + 1) * BN > S;
#pragma unroll
      for (int i = 0; i < KPW; ++i) {
        const int j = wave + NW * i;
        const int pos = 64 * j + lane;
        if (j < NK && pos < BN * KCH) {
          if (!ragged) {
            dma16(kt, koff[i], &smK[buf][512 * j]);
          } else {
            // Keys past S copy row S-1 (at or after the tile's first key).
            const int row = pos / KCH;
            const int cc = pos - row * KCH;
            const int rrel = min(t * BN + row, S - 1) - t * BN;
            dma16(kt, 2u * static_cast<unsigned>(rrel * static_cast<int>(p.ks) + 8 * (cc < CPR ? cc : 0)),
                  &smK[buf][512 * j]);
          }
        }
      }
    };
    // Valid-key bits (key mask and key < S) of tile t as a wave-uniform mask;
    // with a key mask, call after vm_wait() (the mask bytes load in dma_k).
    auto key_bits = [&](int t) __attribute__((always_inline)) -> uint64_t {
      if constexpr (HAS_MASK) {
        return __builtin_amdgcn_ballot_w64(rm);
      } else {
        return range_bits(t * BN, S);
      }
    };
    auto dma_v = [&](int buf, int t) __attribute__((always_inline)) {
      const St* vt = V + static_cast<int64_t>(t) * BN * p.vs;
      const bool ragged = (t + 1) * BN > S;
#pragma unroll
      for (int i = 0; i < VPW; ++i) {
        const int j = wave + NW * i;
        const int pos = 64 * j + lane;
        if (j < NV && pos < BN * VCH) {
          if (!ragged) {
            dma16(vt, voff[i], &smV[buf][512 * j]);
          } else {
            const int row = pos / VCH;
            const int cc = pos - row * VCH;
            const int rrel = min(t * BN + row, S - 1) - t * BN;
            dma16(vt, 2u * static_cast<unsigned>(rrel * static_cast<int>(p.vs) + 8 * (cc ^ vswz(row))),
                  &smV[buf][512 * j]);
          }
        }
      }
    };

    // Copies of a tile that lies wholly before S (no ragged rows): the
    // (row, chunk) offsets computed once, no per-lane range test.  With whole
    // 64-lane DMA instructions (BN * VCH and, for 64-key tiles, BN * KCH
    // multiples of 64) the only guard left is the wave-uniform instruction
    // count; the 32-key K tile of head_dim 128 (544 chunks) ends on half an
    // instruction.
    static_assert((BN * VCH) % 64 == 0 && (BN == 32 || (BN * KCH) % 64 == 0), "whole DMA instructions");
    auto dma_k_full = [&](int buf, int t) __attribute__((always_inline)) {
      if constexpr (HAS_MASK) {
        const int key = t * BN + lane;
        rm = lane < BN && M[key * p.ms] != 0;
      }
      const St* kt = K + static_cast<int64_t>(t) * BN * p.ks;
#pragma unroll
      for (int i = 0; i < KPW; ++i) {
        const int j = wave + NW * i;
        if (j < NK && ((BN * KCH) % 64 == 0 || 64 * j + lane < BN * KCH)) {
          dma16(kt, koff[i], &smK[buf][512 * j]);
        }
      }
    };
    auto dma_v_full = [&](int buf, int t) __attribute__((always_inline)) {
      const St* vt = V + static_cast<int64_t>(t) * BN * p.vs;
#pragma unroll
      for (int i = 0; i < VPW; ++i) {
        const int j = wave + NW * i;
        if (j < NV) dma16(vt, voff[i], &smV[buf][512 * j]);
      }
    };

    auto kread = [&](int buf, int sb, int g) __attribute__((always_inline)) -> u16x8 {
      const int row = sb * 32 + m;
      return *reinterpret_cast<const u16x8*>(&smK[buf][row * KS + 16 * g + 8 * h]);
    };
    // A operand of P.V step idx = ((sb * 2 + j) * NDB + db): d-row 32*db + m,
    // keys sb*32 + 16j + 4h + {0..3} and sb*32 + 16j + 8 + 4h + {0..3}.  For
    // head dims below 32 the rows d >= D hold other data; they only reach
    // output rows that are never stored.
    auto vread = [&](int buf, int idx) __attribute__((always_inline)) -> u16x8 {
      const int db = idx % NDB;
      const int kstep = idx / NDB;  // sb * 2 + j
      const int col = C::VSWZ ? vbase + ((32 * db) ^ vflip) : vbase + 32 * db;
      const unsigned short* base = &smV[buf][col + 16 * kstep * VS];
      const u16x4 lo = lds_read_tr16(base);
      const u16x4 hi = lds_read_tr16(base + 8 * VS);
      return u16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    float m_run = -INFINITY;  // running max of RAW scores
    float m_exp = -INFINITY;  // ceil(m_run * c), kept with m_run
    float l_run = 0.0f;
    f32x16 acc[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i) acc[i] = f32x16{};
    // Probabilities of the pending tile in the B-operand layout of the
    // 32x32x16 MFMA: k-step (sb, j) takes registers 8j..8j+7 of sub-block sb,
    // i.e. keys 16j+4h+{0..3} and 16j+8+4h+{0..3}.
    u16x8 pk[NSB * 2];
#pragma unroll
    for (int i = 0; i < NSB * 2; ++i) pk[i] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};

    // S^T = K(buf) . Q^T.  K fragments run PDK groups ahead in a ring: the
    // slot of group g is refilled with group g + PDK right after group g's
    // MFMAs issue, so an LDS read has PDK - 1 groups of MFMAs to land.
    // Only the first L sub-blocks (a compile-time count: the live ones of a
    // masked tile) are computed; the others are left untouched.  A run-time
    // count would put every MFMA of sub-block 1 under its own branch, and the
    // compiler then copies its 16 accumulators through every branch.
    auto qk = [&](auto live_tag, int buf, f32x16 (&s)[NSB]) {
      constexpr int L = decltype(live_tag)::value;
      static_assert(L >= 1 && L <= NSB, "live sub-blocks");
#pragma unroll
      for (int sb = 0; sb < L; ++sb) s[sb] = f32x16{};
      u16x8 kr[PDK][NSB];
#pragma unroll
      for (int i = 0; i < PDK && i < G; ++i)
#pragma unroll
        for (int sb = 0; sb < L; ++sb) kr[i][sb] = kread(buf, sb, i);
#pragma unroll
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int sb = 0; sb < L; ++sb) s[sb] = mfma_16(T{}, kr[g % PDK][sb], qf[g], s[sb]);
        if (g + PDK < G) {
#pragma unroll
          for (int sb = 0; sb < L; ++sb) kr[g % PDK][sb] = kread(buf, sb, g + PDK);
        }
        fence();
      }
    };

    // O^T += V^T(buf) . P^T over the first L sub-blocks (compile-time, as in
    // qk); V fragments run PDV steps ahead in a ring.
    auto pv = [&](int buf, auto live_tag) __attribute__((always_inline)) {
      constexpr int L = decltype(live_tag)::value;
      constexpr int nsteps = L * 2 * NDB;
      u16x8 vr[PDV];
#pragma unroll
      for (int i = 0; i < PDV && i < nsteps; ++i) vr[i] = vread(buf, i);
#pragma unroll
      for (int idx = 0; idx < nsteps; ++idx) {
        acc[idx % NDB] = mfma_16(T{}, vr[idx % PDV], pk[idx / NDB], acc[idx % NDB]);
        if (idx + PDV < nsteps) vr[idx % PDV] = vread(buf, idx + PDV);
        fence();
      }
    };
    // Calls f with the live sub-block count n (1 .. NSB) as a compile-time
    // constant.
    auto with_live = [&](int n, auto&& f) __attribute__((always_inline)) {
      if constexpr (NSB == 2) {
        if (n == 2) {
          f(std::integral_constant<int, 2>{});
        } else {
          f(std::integral_constant<int, 1>{});
        }
      } else {
        f(std::integral_constant<int, NSB>{});
      }
    };
    constexpr std::integral_constant<int, NSB> kAllLive{};

    // Lazy reference max: probabilities are exp2(s * c - ceil(m_run * c))
    // against a per-row reference m_run that moves only when the row's max
    // exceeds it by more than 8 / c (so P <= 2^8); the accumulator and the
    // row sum are rescaled only then, for the whole wavefront at once.  The
    // reference exponent is rounded up to an integer, so P = 2^k * exp2(s * c
    // - ceil(max * c)) for an integer k whatever the lag: rounding P to 16
    // bits lands on the same grid as rounding it against the final row max
    // (a power-of-two scale commutes with rounding), and the rescale factor
    // is an exact power of two.  Call after the P.V MFMAs that use the
    // previous reference have been issued.
    auto rebase = [&](float mt) __attribute__((always_inline)) {
      const bool need = mt - m_run > lag;  // false for two -inf
      if (__builtin_amdgcn_ballot_w64(need) != 0) {
        const float m_new = need ? mt : m_run;
        // 1 where the reference stays (also at -inf, where the difference
        // would be NaN), 0 from -inf, else 2^-k.
        const float e_new = ceilf(m_new * c);
        const float alpha = m_new == m_run ? 1.0f : fast_exp2(m_exp - e_new);
        l_run *= alpha;
#pragma unroll
        for (int i = 0; i < NDB; ++i) acc[i] *= alpha;
        m_run = m_new;
        m_exp = e_new;
      }
    };
    // Softmax of the first L sub-blocks of s into pn (registers 2L and up of
    // pn are left as they are: P.V and the row sum of this tile skip them).
    auto softmax = [&](auto masked_tag, auto live_tag, f32x16 (&s)[NSB], u16x8 (&pn)[NSB * 2]) {
      constexpr bool MASKED = decltype(masked_tag)::value;
      constexpr int L = decltype(live_tag)::value;
      float mt = s[0][0];
#pragma unroll
      for (int sb = 0; sb < L; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[sb][r]);
      mt = max_with_other_half(mt);
      rebase(mt);
      const float mc = ceilf(((MASKED && m_run == -INFINITY) ? 0.0f : m_run) * c);
#pragma unroll
      for (int sb = 0; sb < L; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pr = fast_exp2(__builtin_fmaf(s[sb][r], c, -mc));
          pn[sb * 2 + (r >> 3)][r & 7] = to_bits(T{}, pr);
        }
      l_run = add_packed<T, NSB * 2, 2 * L>(pn, l_run);
    };

    // P.V of the pending tile interleaved with the softmax of s: the first
    // half of the k-steps carries the row max, the second half the exp2 and
    // conversion (the steady body of key-masked launches).
    auto fused = [&](int buf, f32x16 (&s)[NSB], u16x8 (&pn)[NSB * 2]) __attribute__((always_inline)) {
      constexpr int HALF = NSTEP / 2;
      constexpr int E = NSB * 16;      // score elements per lane
      constexpr int PER = E / HALF;    // elements per step in each phase
      float mt = -INFINITY;
      float m_use = 0.0f, alpha = 1.0f, mc = 0.0f;
      bool rebase_any = false;
      u16x8 vr[PDV];
#pragma unroll
      for (int i = 0; i < PDV && i < NSTEP; ++i) vr[i] = vread(buf, i);
#pragma unroll
      for (int idx = 0; idx < NSTEP; ++idx) {
        acc[idx % NDB] = mfma_16(T{}, vr[idx % PDV], pk[idx / NDB], acc[idx % NDB]);
        if (idx + PDV < NSTEP) vr[idx % PDV] = vread(buf, idx + PDV);
        if (idx < HALF) {
#pragma unroll
          for (int j = 0; j < PER; ++j) {
            const int e = PER * idx + j;
            mt = fmaxf(mt, s[e >> 4][e & 15]);
          }
          if (idx == HALF - 1) {
            mt = max_with_other_half(mt);
            // The reference for this tile: rebased now only if some row needs
            // it (the accumulator rescale waits for the last P.V step).
            const bool need = mt - m_run > lag;
            rebase_any = __builtin_amdgcn_ballot_w64(need) != 0;
            m_use = rebase_any && need ? mt : m_run;
            // 1 where the reference stays: a row still at -inf (no allowed
            // key so far) must not turn its zeros into NaN when another row
            // of the wavefront moves.
            alpha = m_use == m_run ? 1.0f : fast_exp2(m_exp - ceilf(m_use * c));
            mc = ceilf((m_use == -INFINITY ? 0.0f : m_use) * c);
          }
        } else {
#pragma unroll
          for (int j = 0; j < PER; ++j) {
            const int e = PER * (idx - HALF) + j;
            const float pr = fast_exp2(__builtin_fmaf(s[e >> 4][e & 15], c, -mc));
            pn[(e >> 4) * 2 + ((e & 15) >> 3)][e & 7] = to_bits(T{}, pr);
          }
        }
        fence();
      }
      if (rebase_any) {
        l_run *= alpha;
#pragma unroll
        for (int i = 0; i < NDB; ++i) acc[i] *= alpha;
        m_run = m_use;
        m_exp = ceilf(m_use * c);
      }
      l_run = add_packed<T>(pn, l_run);
    };
    // Pipelined full tiles (launches without a key mask).  Q.K runs one tile
    // ahead, so each wavefront has matrix-core work beside its softmax VALU
    // work in both halves of a tile (Q.K on its own was the longest stretch
    // of a tile in which the wavefront could issue nothing else):
    //   phase A: S(t+1) = K(t+1).Q^T, interleaved with the exp2 and 16-bit
    //            conversion of S(t) into P(t) against the reference mc;
    //   phase B: O^T += V(t)^T.P(t), interleaved with the row max of S(t+1);
    //            then the row sum of P(t) and the reference decision for
    //            tile t+1 (with the accumulator rescale when it moves).
    auto phase_a = [&](int kbuf, f32x16 (&sn)[NSB], const f32x16 (&s)[NSB], float mc, auto&& hook)
        __attribute__((always_inline)) {
      constexpr int NQK = G * NSB;  // Q.K MFMAs of a tile
      constexpr int E = NSB * 16;   // score elements per lane
      constexpr int PER = E / NQK;  // exp2 per MFMA
      static_assert(E % NQK == 0, "the softmax work divides over the Q.K steps");
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) sn[sb] = f32x16{};
      u16x8 kr[PDK][NSB];
#pragma unroll
      for (int i = 0; i < PDK && i < G; ++i)
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb) kr[i][sb] = kread(kbuf, sb, i);
#pragma unroll
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb) {
          sn[sb] = mfma_16(T{}, kr[g % PDK][sb], qf[g], sn[sb]);
#pragma unroll
          for (int j = 0; j < PER; ++j) {
            const int e = PER * (g * NSB + sb) + j;
            const float pr = fast_exp2(__builtin_fmaf(s[e >> 4][e & 15], c, -mc));
            pk[(e >> 4) * 2 + ((e & 15) >> 3)][e & 7] = to_bits(T{}, pr);
          }
        }
        if (g + PDK < G) {
#pragma unroll
          for (int sb = 0; sb < NSB; ++sb) kr[g % PDK][sb] = kread(kbuf, sb, g + PDK);
        }
        hook(g);
        fence();
      }
    };
    // ADD_SUM: whether P(t) still has to enter the row sum (the generic
    // softmax counts its P when producing it).
    auto phase_b = [&](auto add_sum_tag, int vbuf, const f32x16 (&sn)[NSB], auto&& hook)
        __attribute__((always_inline)) {
      constexpr bool ADD_SUM = decltype(add_sum_tag)::value;
      constexpr int E = NSB * 16;
      constexpr int PER = E / NSTEP;  // max operands per P.V MFMA
      static_assert(E % NSTEP == 0, "the row max divides over the P.V steps");
      float mt = -INFINITY;
      u16x8 vr[PDV];
#pragma unroll
      for (int i = 0; i < PDV && i < NSTEP; ++i) vr[i] = vread(vbuf, i);
#pragma unroll
      for (int idx = 0; idx < NSTEP; ++idx) {
        acc[idx % NDB] = mfma_16(T{}, vr[idx % PDV], pk[idx / NDB], acc[idx % NDB]);
        if (idx + PDV < NSTEP) vr[idx % PDV] = vread(vbuf, idx + PDV);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
          const int e = PER * idx + j;
          mt = fmaxf(mt, sn[e >> 4][e & 15]);
        }
        hook(idx);
        fence();
      }
      if constexpr (ADD_SUM) l_run = add_packed<T>(pk, l_run);
      rebase(max_with_other_half(mt));
    };
    // Reference exponent of the current tile (without a key mask every row
    // of a full tile has finite scores after tile 0).
    auto ref_exp = [&]() __attribute__((always_inline)) -> float { return m_exp; };

    // Key tiles [kt0, kt1) of this workgroup: all of the query tile's, or one
    // chunk of them on the key-split grid.
    int kt0 = 0, kt1 = ntiles;
    if (w.nchunk > 1) {
      const int csz = (ntiles + w.nchunk - 1) / w.nchunk;
      kt0 = w.chunk * csz;
      kt1 = min(ntiles, kt0 + csz);
    }

    dma_k(kt0 & 1, kt0);
    vm_wait();
    uint64_t kvalid = key_bits(kt0);
    __syncthreads();

    // Tiles before n_full are "full" for this wavefront: every sub-block
    // live, no causal or ragged-end masking (a key mask may still apply).
    // Tiles (kt0, n_full) run a branch-free steady body; tile kt0 and the
    // tail use the generic body.  Every path executes one barrier per tile,
    // so all wavefronts meet kt1 - kt0 barriers.
    const int n_full = q0 >= S ? 0
                               : min(kt1, min(S / BN, CAUSAL ? (q0 + 1) / BN : ntiles));
    bool pending = false;  // a tile's P.V is still to be accumulated (uniform)
    int pend_live = 0;     // its number of live sub-blocks

    auto finish_tile = [&](int t) __attribute__((always_inline)) {
      vm_wait();
      const uint64_t kvalid_next = key_bits(t + 1);
      __syncthreads();
      kvalid = kvalid_next;
    };
    auto generic_tile = [&](int t) __attribute__((always_inline)) {
      const int kb = t & 1;
      // K(t+1) goes to the buffer K(t-1) used, V(t) to the one V(t-2) used;
      // neither is read in this iteration.
      if (t + 1 < kt1) dma_k(kb ^ 1, t + 1);
      dma_v(kb, t);
      const int k0 = t * BN;
      const bool live = q0 < S && (!CAUSAL || k0 <= q0 + 31);
      int nlive = NSB;
#pragma unroll
      for (int sb = NSB - 1; sb >= 0; --sb) {
        const int ks = k0 + sb * 32;
        if (ks >= S || (CAUSAL && ks > q0 + 31)) nlive = sb;
      }
      if (pending) with_live(pend_live, [&](auto lt) __attribute__((always_inline)) { pv(kb ^ 1, lt); });
      if (live) {
        // pn registers past the live sub-blocks are left unset: P.V and the
        // row sum of this tile never read them.  The copy into pk stays out
        // of the branches (stores to pk that differ per branch would be
        // merged into one store at a selected index, which moves pk to
        // scratch memory).
        u16x8 pn[NSB * 2];
        with_live(nlive, [&](auto lt) __attribute__((always_inline)) {
          f32x16 s[NSB];
          qk(lt, kb, s);
          apply_mask<NSB, CAUSAL, true, decltype(lt)::value>(s, k0, kvalid, qrow, h);
          softmax(std::true_type{}, lt, s, pn);
        });
#pragma unroll
        for (int i = 0; i < NSB * 2; ++i) pk[i] = pn[i];
        pend_live = nlive;
      }
      pending = live;
      finish_tile(t);
    };

    generic_tile(kt0);
    if constexpr (HAS_MASK || BNK == 32) {
      // Key-masked launches keep one score buffer (the second one of the
      // pipelined body costs them an occupancy step at head_dim 64 and
      // spills at 128, which outweighs the overlap), and so do 32-key tiles,
      // whose three workgroups per CU leave no room for it.
      for (int t = kt0 + 1; t < n_full; ++t) {
        const int kb = t & 1;
        if (t + 1 < n_full) {
          dma_k_full(kb ^ 1, t + 1);
        } else if (t + 1 < kt1) {
          dma_k(kb ^ 1, t + 1);
        }
        dma_v_full(kb, t);
        f32x16 s[NSB];
        u16x8 pn[NSB * 2];
        qk(kAllLive, kb, s);
        if constexpr (HAS_MASK) apply_mask<NSB, false>(s, t * BN, kvalid, qrow, h);
        fused(kb ^ 1, s, pn);
#pragma unroll
        for (int i = 0; i < NSB * 2; ++i) pk[i] = pn[i];
        finish_tile(t);
      }
    } else if (n_full - kt0 >= 2) {
      // Every interval between two barriers copies and reads the same buffers
      // as the generic tile of that index (K(tau+1), V(tau) in; K(tau),
      // V(tau-1) read), so wavefronts on different paths stay in step.
      // S(t) lives in sa when t - kt0 is odd and in sb when it is even.
      f32x16 sa[NSB], sb[NSB];
      const int t1 = kt0 + 1;
      // Tile t1: S(t1) with nothing to overlap, then P.V(kt0) with its row max.
      if (t1 + 1 < n_full) {
        dma_k_full((t1 + 1) & 1, t1 + 1);
      } else if (t1 + 1 < kt1) {
        dma_k((t1 + 1) & 1, t1 + 1);
      }
      dma_v_full(t1 & 1, t1);
      qk(kAllLive, t1 & 1, sa);
      phase_b(std::false_type{}, kt0 & 1, sa, [](int) {});
      finish_tile(t1);
      // Tile t + 1 for t = t1 .. n_full - 2.
      auto steady = [&](int t, const f32x16 (&cur)[NSB], f32x16 (&nxt)[NSB])
          __attribute__((always_inline)) {
        const int kb = t & 1;
        // The copies of K(t+2) and V(t+1) are spread over the MFMA groups of
        // both phases instead of issued back to back at the top of the tile.
        static_assert(KPW <= G && 2 * VPW - 1 <= NSTEP, "a copy slot for every copy");
        const bool kfull = t + 2 < n_full;
        if (!kfull && t + 2 < kt1) dma_k(kb, t + 2);
        const St* kt = K + static_cast<int64_t>(t + 2) * BN * p.ks;
        const St* vt = V + static_cast<int64_t>(t + 1) * BN * p.vs;
        phase_a(kb ^ 1, nxt, cur, ref_exp(), [&](int g) __attribute__((always_inline)) {
          if (g < KPW) {
            const int j = wave + NW * g;
            if (kfull && j < NK) dma16(kt, koff[g], &smK[kb][512 * j]);
          }
        });
        phase_b(std::true_type{}, kb, nxt, [&](int idx) __attribute__((always_inline)) {
          if (idx % 2 == 0 && idx / 2 < VPW) {
            const int i = idx / 2;
            const int j = wave + NW * i;
            if (j < NV) dma16(vt, voff[i], &smV[kb ^ 1][512 * j]);
          }
        });
        finish_tile(t + 1);
      };
      int t = t1;
      for (; t + 2 < n_full; t += 2) {
        steady(t, sa, sb);
        steady(t + 1, sb, sa);
      }
      if (t + 1 < n_full) {
        steady(t, sa, sb);
        ++t;
      }
      // Tile n_full - 1: its P becomes the pending P.V of the next tile.
      const float mc = ref_exp();
      auto last_p = [&](const f32x16 (&cur)[NSB]) __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < NSB * 16; ++e) {
          const float pr = fast_exp2(__builtin_fmaf(cur[e >> 4][e & 15], c, -mc));
          pk[(e >> 4) * 2 + ((e & 15) >> 3)][e & 7] = to_bits(T{}, pr);
        }
      };
      if ((t - kt0) & 1) {
        last_p(sa);
      } else {
        last_p(sb);
      }
      l_run = add_packed<T>(pk, l_run);
      pending = true;
      pend_live = NSB;
    }
    for (int t = max(kt0 + 1, n_full); t < kt1; ++t) generic_tile(t);
    if (pending) with_live(pend_live, [&](auto lt) __attribute__((always_inline)) { pv((kt1 - 1) & 1, lt); });

    if (BNK == 64 && w.nchunk > 1) {
      // Key-split query tile: publish this chunk's state - per lane the
      // integer reference exponent E (-inf for a row with no key yet), the
      // lane half's row sum and the 16 * NDB accumulator values, stored
      // lane-major so every access is coalesced - then count the chunk in.
      // The chunk that arrives last merges all states; E differs between
      // chunks by integers, so every rescale is an exact power of two.
      //
      // Coherence without cache-wide maintenance: the chunks of a tile may
      // run on different XCDs, whose L2 caches are not coherent, and an
      // agent-scope fence would write back and invalidate a whole L2 (the
      // K/V tiles every other workgroup on that XCD streams from).  Instead
      // only the exchanged words are coherent: the states are written and
      // read with system-scope relaxed atomics (write-through stores,
      // cache-bypassing loads), each wavefront waits for its stores to
      // complete (vmcnt) before the barrier that precedes the counter
      // increment, and the last chunk reads the states only after its
      // increment has returned.
      constexpr int NV = NDB * 16 + 2;  // floats per lane
      const int slot = w.bh * p.split_tiles + (qb - p.split_q0);
      float* const base = p.ws_part + static_cast<int64_t>(slot) * p.split_maxch * 4 * NV * 64;
      auto state = [&](int ch) __attribute__((always_inline)) -> float* {
        return base + static_cast<int64_t>(ch * 4 + wave) * NV * 64 + lane;
      };
      auto put = [](float* a, float v) __attribute__((always_inline)) {
        __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      };
      auto get = [](const float* a) __attribute__((always_inline)) -> float {
        return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      };
      const float e_own = m_run == -INFINITY ? -INFINITY : ceilf(m_run * c);
      {
        float* st = state(w.chunk);
        put(st, e_own);
        put(st + 64, l_run);
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) put(st + (2 + db * 16 + r) * 64, acc[db][r]);
      }
      vm_wait();
      __syncthreads();
      int* const counter = &p.ws_cnt[slot];
      int* arrival = reinterpret_cast<int*>(&smV[0][0]);  // V buffers are idle now
      if (tid == 0) {
        *arrival = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
      __syncthreads();
      if (*arrival != w.nchunk - 1) return;  // another chunk finishes this tile
      float e_max = -INFINITY;
      for (int ch = 0; ch < w.nchunk; ++ch) e_max = fmaxf(e_max, ch == w.chunk ? e_own : get(state(ch)));
      // Sum the chunks in chunk order, so the result does not depend on which
      // one arrived last.
      f32x16 own[NDB];
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        own[db] = acc[db];
        acc[db] = f32x16{};
      }
      const float l_own = l_run;
      l_run = 0.0f;
      for (int ch = 0; ch < w.nchunk; ++ch) {
        const float* st = state(ch);
        const float e = ch == w.chunk ? e_own : get(st);
        const float a = (e == -INFINITY) ? 0.0f : fast_exp2(e - e_max);
        if (ch == w.chunk) {
          l_run += a * l_own;
#pragma unroll
          for (int db = 0; db < NDB; ++db) acc[db] += a * own[db];
        } else {
          l_run += a * get(st + 64);
#pragma unroll
          for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[db][r] += a * get(st + (2 + db * 16 + r) * 64);
        }
      }
      // Ready for the next launch (the launch boundary orders it).
      if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }

    // Output through LDS: the accumulator layout gives a lane 4 consecutive
    // d of one query per register group, so direct stores would write 16
    // bytes into each of 32 rows per instruction (partial cache lines).  The
    // wavefront's 32 x D tile goes to its own slice of the K buffers instead
    // (no K read or copy is pending after the loop's last barrier) and comes
    // back as whole 16-byte row chunks, so each store covers whole rows.
    const float lt = sum_with_other_half(l_run);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    constexpr int OS = D + 8;  // staged row stride (elements; 16-byte pad)
    static_assert(4 * 32 * OS <= 2 * KBUF, "output staging fits the K buffers");
    unsigned short* so = &smK[0][0] + wave * 32 * OS;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int j4 = 0; j4 < 4; ++j4) {
        const int d0 = 32 * db + 8 * j4 + 4 * h;  // 4 consecutive d-rows
        if (D < 32 && d0 >= D) continue;
        u16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = to_bits(T{}, acc[db][4 * j4 + e] * inv);
        *reinterpret_cast<u16x4*>(so + m * OS + d0) = o;
      }
    __builtin_amdgcn_wave_barrier();
    constexpr int OCH = D / 8;  // 16-byte chunks per output row
    St* __restrict__ O = static_cast<St*>(p.out) + b * p.ob + hh * p.oh;
#pragma unroll
    for (int i0 = 0; i0 < 32 * OCH; i0 += 64) {
      const int i = i0 + lane;
      const int row = i / OCH;
      const int cc = i - row * OCH;
      if ((32 * OCH % 64 == 0 || i < 32 * OCH) && q0 + row < S) {
        *reinterpret_cast<u16x8*>(O + (q0 + row) * p.os + 8 * cc) =
            *reinterpret_cast<const u16x8*>(so + row * OS + 8 * cc);
      }
    }
  }
}

// Compute units of the current device (queried once per device).
int device_cu_count() {
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

// Key-split plan of a causal 16-bit launch (see AttnParams::split).  When the
// heaviest query tile outweighs the average workgroup slot, the launch lasts
// as long as that workgroup: a query tile that sees more key tiles than the average
// workgroup slot carries is cut into chunks of at most that many (and at
// most 8), and all units are dispatched heaviest first.
struct SplitPlan {
  bool on = false;
  int units = 0;
  int q0 = 0;
  int maxch = 1;
  int64_t cnt_bytes = 0;
  int64_t bytes = 0;
  unsigned short tab[kMaxSplitUnits] = {};
};

// Workgroups of the 16-bit kernel resident per CU (registers / LDS).
int h16_slots_per_cu(int D) { return D >= 128 ? 2 : 3; }

SplitPlan plan_key_split(int dtype, int D, bool causal, int64_t BH, int64_t S) {
  SplitPlan sp;
  if (dtype == 0 || !causal || BH <= 0 || S <= 0) return sp;
  const int64_t nq = (S + kBM - 1) / kBM;
  if (nq < 2 || nq > 1024) return sp;
  const int64_t slots = static_cast<int64_t>(device_cu_count()) * h16_slots_per_cu(D);
  auto tiles = [&](int64_t i) { return (std::min<int64_t>(S, (i + 1) * kBM) + 63) / 64; };
  int64_t total = 0;
  for (int64_t i = 0; i < nq; ++i) total += tiles(i);
  total *= BH;
  const int64_t limit = std::max<int64_t>(8, (total + slots - 1) / slots);
  // Split only when the heaviest query tile carries over 1.5x the average
  // load of a workgroup slot.  Measured on the MI355X: config 4's attention
  // (B=4, H=16, S=2048, D=64; 1.41x) ran slower split (62.4 -> 66.6 us: the
  // extra prologues and the state exchange outweigh the shorter tail), as
  // did B=8, H=16, S=1024 (1.33x); B=1, H=4, S=4096 (11.6x) went 51.9 ->
  // 35.4 us and B=2, H=4, S=4096 52.3 -> 42.7 us.
  if (2 * tiles(nq - 1) <= 3 * limit) return sp;
  struct Unit {
    int work, q, c, n;
  };
  Unit units[kMaxSplitUnits];
  int nu = 0;
  int q0 = static_cast<int>(nq);
  for (int64_t i = nq - 1; i >= 0; --i) {
    const int64_t t = tiles(i);
    const int64_t n0 = std::min<int64_t>(8, (t + limit - 1) / limit);
    const int64_t csz = (t + n0 - 1) / n0;
    const int64_t n = (t + csz - 1) / csz;  // every chunk non-empty; ceil(t / n) == csz
    if (n > 1) q0 = static_cast<int>(i);
    for (int64_t c = 0; c < n; ++c) {
      if (nu == kMaxSplitUnits) return SplitPlan{};
      units[nu++] = Unit{static_cast<int>(std::min(t, (c + 1) * csz) - c * csz), static_cast<int>(i),
                         static_cast<int>(c), static_cast<int>(n)};
    }
  }
  std::stable_sort(units, units + nu, [](const Unit& a, const Unit& b) { return a.work > b.work; });
  for (int u = 0; u < nu; ++u) {
    sp.tab[u] = static_cast<unsigned short>(units[u].q | (units[u].c << 10) | ((units[u].n - 1) << 13));
    if (units[u].q == nq - 1) sp.maxch = units[u].n;
  }
  const int64_t nv = ((D + 31) / 32) * 16 + 2;  // floats of partial state per lane
  const int64_t split_tiles = nq - q0;
  // One counter per split slot (batch, head, split query tile), in the fixed
  // block that leads every workspace.
  if (BH * split_tiles > kSplitCounterSlots) return SplitPlan{};
  sp.q0 = q0;
  sp.units = nu;
  sp.cnt_bytes = kSplitCounterBytes;
  sp.bytes = sp.cnt_bytes + BH * split_tiles * sp.maxch * 4 * nv * 64 * 4;
  sp.on = true;
  return sp;
}

template <int D, bool CAUSAL, bool HAS_MASK>
hipError_t launch_d(int dtype, AttnParams& p, void* ws, int64_t ws_bytes, hipStream_t stream) {
  // Causal pairing (fp32 kernel only) halves the grid; use it only while the
  // paired grid still gives every workgroup slot of the GPU (CUs x resident
  // workgroups) one workgroup - below that, the tail of the unpaired grid is
  // cheaper than idle slots.
  const int64_t paired = static_cast<int64_t>((p.nq + 1) / 2) * p.BH;
  p.pair = (dtype == 0 && CAUSAL && p.nq >= 2 &&
            paired >= static_cast<int64_t>(device_cu_count()) * kMinWaves<true, D>) ? 1 : 0;
  p.units = p.pair ? (p.nq + 1) / 2 : p.nq;
  p.cu_count = device_cu_count();
  // Unpaired causal fp32 grid resident in one round (two workgroups per CU):
  // fold the query-tile order so each CU pairs a heavy tile with a light one.
  p.fold = (dtype == 0 && CAUSAL && !p.pair && kMinWaves<true, D> == 2 && p.nq >= 3 &&
            static_cast<int64_t>(p.nq) * p.BH <= 2 * static_cast<int64_t>(p.cu_count) &&
            static_cast<int64_t>(p.nq) * p.BH > static_cast<int64_t>(p.cu_count)) ? 1 : 0;
  // One 64-key tile per head and rows for wavefronts 0-1 only: two heads per
  // workgroup (fp32 non-causal kernels, whose second K/V buffer is free).
  p.twin = (dtype == 0 && !CAUSAL && F32Cfg<D, CAUSAL>::BN == 64 && p.S <= 64) ? 1 : 0;
  p.split = 0;
  if (dtype != 0 && CAUSAL && ws != nullptr) {
    const SplitPlan sp = plan_key_split(dtype, D, true, p.BH, p.S);
    if (sp.on && ws_bytes >= sp.bytes) {
      p.split = 1;
      p.units = sp.units;
      p.split_q0 = sp.q0;
      p.split_tiles = p.nq - sp.q0;
      p.split_maxch = sp.maxch;
      p.ws_cnt = static_cast<int*>(ws);
      p.ws_part = reinterpret_cast<float*>(static_cast<char*>(ws) + sp.cnt_bytes);
      std::copy(sp.tab, sp.tab + sp.units, p.unit_tab);
    }
  }
  if constexpr ((D == 64 || D == 32) && CAUSAL) {
    // 16-bit head_dim 64 and 32, causal, not key-split: 32-key tiles at four
    // workgroups per CU up to S = 1024 (head_dim 64 with a key mask: 2048).
    // Measured against the 64-key kernel (same box, alternating):
    // [16, 512, 16, 64] -13 %, [8, 1024, 16, 64] -4.5 %, key-masked fp16
    // [4, 2048, 16, 64] -2.5 %; config 4 (S = 2048, no mask) +6 %,
    // [1, 8192, 16, 64] +12 %, non-causal launches 6-9 % slower.  Head dim
    // 32: [32, 256, 16, 32] -15 %, [16, 512] -15 %, [8, 1024] -4 %, key-masked
    // fp16 [8, 1024] +2.7 %.
    const int bn32_max = HAS_MASK ? (D == 64 ? 2048 : 0) : 1024;
    if (dtype != 0 && !p.split && p.S <= bn32_max) {
      const dim3 g(static_cast<unsigned>(p.units) * static_cast<unsigned>(p.BH)), blk(kThreads);
      if (dtype == 1) {
        attn_fwd_h16_kernel<BF16, D, CAUSAL, HAS_MASK, 32><<<g, blk, 0, stream>>>(p);
      } else {
        attn_fwd_h16_kernel<F16, D, CAUSAL, HAS_MASK, 32><<<g, blk, 0, stream>>>(p);
      }
      return hipGetLastError();
    }
  }
  if constexpr (D == 128) {
    // 16-bit head_dim 128, not key-split: 32-key tiles, three workgroups per
    // CU, for causal or key-masked launches up to S = 4096 and unmasked
    // non-causal ones up to 1024.  Measured against the 64-key kernel (same
    // box, alternating): causal [16, 512, 16, 128] -19 %, [8, 1024, 16, 128]
    // -9.5 % (key-masked fp16 -19 %), [4, 2048, 16, 128] key-masked fp16
    // -14 %, [4, 4096, 16, 128] -4 %; non-causal [16, 512, 16, 128] -4 %,
    // [8, 1024, 16, 128] +0.7 %, [4, 2048, 16, 128] +4.6 % (key-masked fp16
    // -1 %), [4, 4096, 16, 128] +4.6 %; causal S = 16384 +3.6 %.
    const int bn32_max = (CAUSAL || HAS_MASK) ? 4096 : 1024;
    if (dtype != 0 && !p.split && p.S <= bn32_max) {
      const dim3 g(static_cast<unsigned>(p.units) * static_cast<unsigned>(p.BH)), blk(kThreads);
      if (dtype == 1) {
        attn_fwd_h16_kernel<BF16, D, CAUSAL, HAS_MASK, 32><<<g, blk, 0, stream>>>(p);
      } else {
        attn_fwd_h16_kernel<F16, D, CAUSAL, HAS_MASK, 32><<<g, blk, 0, stream>>>(p);
      }
      return hipGetLastError();
    }
  }
  if constexpr (!CAUSAL && (D == 32 || D == 64)) {
    // Its buffer resources span rows 0..S-1 of one head, and its lanes
    // address rows 0..63 (rows past S are padding) with 32-bit offsets: rows
    // must not overlap (sequence stride >= head_dim) and the offset of every
    // padded row must stay below 2^31 bytes, or it could wrap back inside the
    // resource instead of reading as zero (or being dropped, for stores).
    auto span_ok = [&](int64_t rs) { return rs >= D && (63 * rs + D) * 4 < (int64_t{1} << 31); };
    if (dtype == 0 && p.S <= 64 && span_ok(p.qs) && span_ok(p.ks) && span_ok(p.vs) && span_ok(p.os) &&
        63 * p.ms < (int64_t{1} << 31) - 1) {
      // Short sequences: one wavefront per (batch, head, 32-query half), a
      // persistent grid of two workgroups per CU (fewer when there are fewer
      // items than wavefronts).
      const int64_t items = static_cast<int64_t>(p.BH) * (p.S > 32 ? 2 : 1);
      const int64_t full = static_cast<int64_t>(p.cu_count) * 2;
      const int64_t groups = std::min<int64_t>((items + 3) / 4, full);
      if (HAS_MASK || p.S < 64) {
        attn_fwd_f32_short_kernel<D, HAS_MASK, true>
            <<<dim3(static_cast<unsigned>(groups)), dim3(kThreads), 0, stream>>>(p);
      } else {
        attn_fwd_f32_short_kernel<D, false, false>
            <<<dim3(static_cast<unsigned>(groups)), dim3(kThreads), 0, stream>>>(p);
      }
      return hipGetLastError();
    }
  }
  const unsigned groups = p.twin ? static_cast<unsigned>((p.BH + 1) / 2)
                                 : static_cast<unsigned>(p.units) * static_cast<unsigned>(p.BH);
  const dim3 g(groups), blk(kThreads);
  switch (dtype) {
    case 0: attn_fwd_f32_kernel<D, CAUSAL, HAS_MASK><<<g, blk, 0, stream>>>(p); break;
    case 1: attn_fwd_h16_kernel<BF16, D, CAUSAL, HAS_MASK><<<g, blk, 0, stream>>>(p); break;
    case 2: attn_fwd_h16_kernel<F16, D, CAUSAL, HAS_MASK><<<g, blk, 0, stream>>>(p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int D>
hipError_t launch_flags(int dtype, bool causal, bool has_mask, AttnParams& p, void* ws,
                        int64_t ws_bytes, hipStream_t stream) {
  if (causal) {
    return has_mask ? launch_d<D, true, true>(dtype, p, ws, ws_bytes, stream)
                    : launch_d<D, true, false>(dtype, p, ws, ws_bytes, stream);
  }
  return has_mask ? launch_d<D, false, true>(dtype, p, ws, ws_bytes, stream)
                  : launch_d<D, false, false>(dtype, p, ws, ws_bytes, stream);
}

}  // namespace

int attention_block_m(int /*dtype*/, int /*D*/) { return kBM; }

hipError_t launch_attention(int dtype, int D, bool causal, bool has_mask, AttnParams& p,
                            void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  switch (D) {
    case 8: return launch_flags<8>(dtype, causal, has_mask, p, workspace, workspace_bytes, stream);
    case 16: return launch_flags<16>(dtype, causal, has_mask, p, workspace, workspace_bytes, stream);
    case 32: return launch_flags<32>(dtype, causal, has_mask, p, workspace, workspace_bytes, stream);
    case 64: return launch_flags<64>(dtype, causal, has_mask, p, workspace, workspace_bytes, stream);
    case 128: return launch_flags<128>(dtype, causal, has_mask, p, workspace, workspace_bytes, stream);
    default: return hipErrorInvalidValue;
  }
}

int64_t attention_workspace_bytes(int dtype, int D, bool causal, int64_t BH, int64_t S) {
  const SplitPlan sp = plan_key_split(dtype, D, causal, BH, S);
  return sp.on ? sp.bytes : 0;
}

}  // namespace ttk
