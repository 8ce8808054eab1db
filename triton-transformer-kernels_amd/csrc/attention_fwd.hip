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
//       own registers plus ONE exchange with lane^32, and
//     - the probabilities P^T already sit in the B-operand layout of the next
//       MFMA, O^T[d, query] += V^T[d, key] . P^T[key, query]: register r
//       feeds the k-step whose two keys are the ones that register holds in
//       lane halves 0 and 1.  No transpose, no LDS round trip for P.
// * K and V tiles (BLOCK_N keys) are staged in LDS and double-buffered: the
//   next tile's global loads are issued before the current tile's MFMAs and
//   written to the other buffer afterwards, one barrier per tile.  K rows are
//   padded by 16 bytes, so the 16-byte MFMA operand reads of 16 consecutive
//   key rows start 4 banks apart and cover all 64 banks without conflict,
//   and every per-step operand address is the lane's base plus an immediate.
// * Inside a tile the LDS operand reads are software-pipelined one step ahead
//   of the MFMAs and fenced with scheduling barriers, which keeps the
//   register footprint inside the two-waves-per-SIMD budget (no spills).
// * Masking: key validity (key mask and key < S) is a wave-uniform 64-bit
//   ballot per tile; with the lane's causal limit it becomes one bit mask per
//   32-key sub-block.  Only tiles that need it (diagonal, ragged end, key
//   mask) take the masked path; full interior tiles run unmasked.  Causal
//   workgroups stop at their diagonal (future tiles are never loaded) and a
//   wavefront skips the 32-key sub-blocks entirely after its last query.
// * Scheduling: the flat grid is ordered heaviest query tile first (causal)
//   and, when B*H is a multiple of 8, all query tiles of one head run on the
//   same XCD (workgroups are dealt round-robin to the 8 XCDs), so a head's K/V
//   is fetched from HBM into one XCD's L2 instead of eight.
//
// fp32 path: v_mfma_f32_32x32x2_f32 (IEEE fp32 products, fp32 accumulate).
// Q is pre-multiplied by scale*log2(e) so scores are already in the exp2
// domain.  bf16/fp16 path: v_mfma_f32_32x32x16_{bf16,f16}; scores are kept
// in fp32 and scaled after the product, P is rounded to the input type for
// the P.V product, V is stored transposed in LDS so the 16-bit A operand
// (8 keys of one d) is two 8-byte LDS reads.
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

__device__ __forceinline__ void fence() { __builtin_amdgcn_sched_barrier(0); }

// Key offset (inside a 32-key sub-block) held by register r of lane half h in
// the 32x32 MFMA result layout.
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// Work item of this workgroup: (query tile, batch*head).
__device__ __forceinline__ void work_item(const AttnParams& p, bool causal, int& qb, int& bh) {
  const int id = blockIdx.x;
  int qrank;
  if (p.xcd_swizzle) {
    const int xcd = id & 7;
    const int j = id >> 3;
    const int hpx = p.BH >> 3;  // heads per XCD
    qrank = j / hpx;
    bh = xcd + 8 * (j - qrank * hpx);
  } else {
    qrank = id / p.BH;
    bh = id - qrank * p.BH;
  }
  qb = causal ? p.nq - 1 - qrank : qrank;
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

__device__ __forceinline__ bool reg_allowed(uint32_t a, int r) {
  return (a >> (8 * (r >> 2) + (r & 3))) & 1u;
}

// Online-softmax update of one tile in the exp2 domain.  `s` holds scaled
// scores (-inf where not allowed); on return it holds the probabilities.
template <int NSB, int NACC, bool MASKED>
__device__ __forceinline__ void online_softmax(f32x16 (&s)[NSB], float& m_run, float& l_run,
                                               f32x16 (&acc)[NACC]) {
  float mt = s[0][0];
#pragma unroll
  for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
    for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[sb][r]);
  mt = fmaxf(mt, __shfl_xor(mt, 32));
  const float m_new = fmaxf(m_run, mt);
  // A fully masked row keeps m = -inf; use 0 so exp2(-inf - 0) = 0, never NaN.
  const float m_use = (MASKED && m_new == -INFINITY) ? 0.0f : m_new;
  const float alpha = fast_exp2(m_run - m_use);
  float ls = 0.0f;
#pragma unroll
  for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pv = fast_exp2(s[sb][r] - m_use);
      s[sb][r] = pv;
      ls += pv;
    }
  l_run = __builtin_fmaf(l_run, alpha, ls);
#pragma unroll
  for (int i = 0; i < NACC; ++i) acc[i] *= alpha;
  m_run = m_new;
}

// Waves per SIMD the register budget is sized for: two workgroups per CU,
// except where the live state of head_dim 128 (fp32: every variant; 16-bit:
// non-causal unmasked) does not fit 256 registers without spilling - those
// run one workgroup per CU with the accumulators in AGPRs.
template <bool F32, int D, bool CAUSAL, bool HAS_MASK>
constexpr int kMinWaves = (D >= 128 && (F32 || (!CAUSAL && !HAS_MASK))) ? 1 : 2;

// ----------------------------------------------------------------------------
// fp32
// ----------------------------------------------------------------------------
template <int D>
struct F32Cfg {
  static constexpr int BN = D >= 128 ? 32 : 64;     // keys per tile
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
__global__ __launch_bounds__(kThreads, (kMinWaves<true, D, CAUSAL, HAS_MASK>)) void attn_fwd_f32_kernel(AttnParams p) {
  using C = F32Cfg<D>;
  constexpr int BN = C::BN, NSB = C::NSB, CPR = C::CPR, KS = C::KS, DB = C::DB, CPT = C::CPT,
                G = C::G;
  using VF = typename VFrag32<D>::type;
  __shared__ __attribute__((aligned(16))) float smK[2][BN * KS];
  __shared__ __attribute__((aligned(16))) float smV[2][BN * D];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int m = lane & 31;
  const int h = lane >> 5;

  int qb, bh;
  work_item(p, CAUSAL, qb, bh);
  const int b = bh / p.H;
  const int hh = bh - b * p.H;
  const int S = p.S;
  const float* __restrict__ Q = static_cast<const float*>(p.q) + b * p.qb + hh * p.qh;
  const float* __restrict__ K = static_cast<const float*>(p.k) + b * p.kb + hh * p.kh;
  const float* __restrict__ V = static_cast<const float*>(p.v) + b * p.vb + hh * p.vh;
  const uint8_t* __restrict__ M = HAS_MASK ? p.mask + b * p.mb : nullptr;

  const int q0 = qb * kBM + wave * 32;  // first query of this wavefront
  const int qrow = q0 + m;              // query of this lane

  // B operand of S^T = K.Q^T: group g covers d = 8g..8g+7, lane half h holds
  // d = 8g+4h..8g+4h+3 (one element per k-step).  Pre-scaled into exp2 units.
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

  f32x4 rk[CPT], rv[CPT];
  bool rm = false;
  auto gload = [&](int t) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int idx = tid + kThreads * i;
      if (C::CHUNKS % kThreads == 0 || idx < C::CHUNKS) {
        const int row = idx / CPR;
        const int c = idx - row * CPR;
        const int key = t * BN + row;
        if (key < S) {
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
  // Writes the staged tile into LDS buffer `buf`; returns the tile's valid-key
  // bits (key mask and key < S) as a wave-uniform 64-bit mask.
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
  // `nlive` = number of leading 32-key sub-blocks this wavefront needs.
  auto tile = [&](auto masked_tag, int buf, int k0, int nlive, uint64_t kvalid) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    f32x16 s[NSB];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) s[sb] = f32x16{};
    // ---- S^T = K . Q^T (K fragments read one group ahead) ----------------
    f32x4 kf[NSB];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
      if (!MASKED || sb < nlive) kf[sb] = kread(buf, sb, 0);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      f32x4 kn[NSB];
      if (g + 1 < G) {
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb)
          if (!MASKED || sb < nlive) kn[sb] = kread(buf, sb, g + 1);
      }
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) {
        if (MASKED && sb >= nlive) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) s[sb] = mfma_f32(kf[sb][e], qf[g][e], s[sb]);
      }
      if (g + 1 < G) {
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb) kf[sb] = kn[sb];
      }
      fence();
    }
    // ---- mask ------------------------------------------------------------
    if constexpr (MASKED) {
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) {
        const int ks = k0 + sb * 32;
        const uint32_t a = lane_allowed<CAUSAL>(static_cast<uint32_t>(kvalid >> (32 * sb)), ks, qrow, h);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (!reg_allowed(a, r)) s[sb][r] = -INFINITY;
      }
    }
    online_softmax<NSB, DB, MASKED>(s, m_run, l_run, acc);
    fence();
    // ---- O^T += V^T . P^T (V fragments read one k-step ahead) -------------
    const int nsteps = (MASKED ? nlive : NSB) * 16;
    VF vf = vread(buf, 0, 0);
#pragma unroll
    for (int idx = 0; idx < NSB * 16; ++idx) {
      // Fixed trip count (fully unrolled, so s[][] stays in registers); the
      // masked path skips the k-steps of dead sub-blocks with a uniform guard.
      if (!MASKED || idx < nsteps) {
        const int sb = idx >> 4;
        const int r = idx & 15;
        VF vn{};
        if (idx + 1 < NSB * 16 && (!MASKED || idx + 1 < nsteps)) {
          vn = vread(buf, (idx + 1) >> 4, (idx + 1) & 15);
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

  gload(0);
  uint64_t kvalid = lstore(0, 0);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) gload(t + 1);
    const int k0 = t * BN;
    if (q0 < S && (!CAUSAL || k0 <= q0 + 31)) {
      // Leading sub-blocks that hold any key this wavefront may see.
      int nlive = NSB;
#pragma unroll
      for (int sb = NSB - 1; sb >= 0; --sb) {
        const int ks = k0 + sb * 32;
        if (ks >= S || (CAUSAL && ks > q0 + 31)) nlive = sb;
      }
      const bool need_mask = HAS_MASK || (k0 + BN > S) || (CAUSAL && k0 + BN - 1 > q0);
      if (need_mask) {
        tile(std::true_type{}, buf, k0, nlive, kvalid);
      } else {
        tile(std::false_type{}, buf, k0, NSB, kvalid);
      }
    }
    if (t + 1 < ntiles) kvalid = lstore(buf ^ 1, t + 1);
    __syncthreads();
  }

  // ---- epilogue: O = acc / l ------------------------------------------------
  const float lt = l_run + __shfl_xor(l_run, 32);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  if (qrow >= S) return;
  float* __restrict__ O = static_cast<float*>(p.out) + b * p.ob + hh * p.oh + qrow * p.os;
#pragma unroll
  for (int j4 = 0; j4 < 4; ++j4) {
    // Block i of the accumulator holds d = DB*row + i; register 4*j4+e holds
    // row 8*j4 + 4h + e, so a lane's d-values form one run of 4*DB.
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

// ----------------------------------------------------------------------------
// bf16 / fp16
// ----------------------------------------------------------------------------
template <int D>
struct H16Cfg {
  static constexpr int DK = D < 16 ? 16 : D;         // contraction length of Q.K (zero padded)
  static constexpr int BN = 64;                      // keys per tile
  static constexpr int NSB = BN / 32;
  static constexpr int CPR = D / 8;                  // 16-byte chunks per key row (8 elems)
  static constexpr int KS = DK + 8;                  // LDS K row stride (elements, 16-byte pad)
  static constexpr int NDB = (D + 31) / 32;          // output blocks of 32 d-rows
  static constexpr int G = DK / 16;                  // Q.K k-steps of 16
  static constexpr int VTS = BN + 4;                 // V^T row stride (elements)
  static constexpr int CHUNKS = BN * CPR;
  static constexpr int CPT = (CHUNKS + kThreads - 1) / kThreads;
  // V^T store: a thread moves 4 keys x 8 d (four 16-byte global loads).
  static constexpr int VGROUPS = (BN / 4) * CPR;
  static constexpr int VPT = (VGROUPS + kThreads - 1) / kThreads;
};

template <typename T, int D, bool CAUSAL, bool HAS_MASK>
__global__ __launch_bounds__(kThreads, (kMinWaves<false, D, CAUSAL, HAS_MASK>)) void attn_fwd_h16_kernel(AttnParams p) {
  using C = H16Cfg<D>;
  constexpr int BN = C::BN, NSB = C::NSB, CPR = C::CPR, DK = C::DK, KS = C::KS,
                NDB = C::NDB, VTS = C::VTS, CPT = C::CPT, VPT = C::VPT, G = C::G;
  __shared__ __attribute__((aligned(16))) unsigned short smK[2][BN * KS];
  __shared__ __attribute__((aligned(16))) unsigned short smVt[2][D * VTS];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int m = lane & 31;
  const int h = lane >> 5;

  int qb, bh;
  work_item(p, CAUSAL, qb, bh);
  const int b = bh / p.H;
  const int hh = bh - b * p.H;
  const int S = p.S;
  using St = unsigned short;
  const St* __restrict__ Q = static_cast<const St*>(p.q) + b * p.qb + hh * p.qh;
  const St* __restrict__ K = static_cast<const St*>(p.k) + b * p.kb + hh * p.kh;
  const St* __restrict__ V = static_cast<const St*>(p.v) + b * p.vb + hh * p.vh;
  const uint8_t* __restrict__ M = HAS_MASK ? p.mask + b * p.mb : nullptr;

  const int q0 = qb * kBM + wave * 32;
  const int qrow = q0 + m;

  // B operand of S^T = K.Q^T: k-step g covers d = 16g..16g+15, lane half h
  // holds d = 16g+8h..16g+8h+7.
  u16x8 qf[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int d = 16 * g + 8 * h;
    if (qrow < S && d < D) {
      qf[g] = *reinterpret_cast<const u16x8*>(Q + qrow * p.qs + d);
    } else {
      qf[g] = u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }

  const int kv_end = CAUSAL ? min(S, (qb + 1) * kBM) : S;
  const int ntiles = (kv_end + BN - 1) / BN;

  // K: CPT chunks of 8 elements per thread.  V: VPT groups of 4 keys x 8 d.
  u32x4 rk[CPT];
  u32x4 rv[VPT][4];
  bool rm = false;
  auto gload = [&](int t) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int idx = tid + kThreads * i;
      if (C::CHUNKS % kThreads == 0 || idx < C::CHUNKS) {
        const int row = idx / CPR;
        const int c = idx - row * CPR;
        const int key = t * BN + row;
        rk[i] = key < S ? *reinterpret_cast<const u32x4*>(K + key * p.ks + 8 * c)
                        : u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int gi = tid + kThreads * i;
      if (C::VGROUPS % kThreads == 0 || gi < C::VGROUPS) {
        const int kq = gi / CPR;  // key quad
        const int c = gi - kq * CPR;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int key = t * BN + 4 * kq + e;
          rv[i][e] = key < S ? *reinterpret_cast<const u32x4*>(V + key * p.vs + 8 * c)
                             : u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
    if constexpr (HAS_MASK) {
      const int key = t * BN + lane;
      rm = lane < BN && key < S && M[key * p.ms] != 0;
    }
  };
  auto lstore = [&](int buf, int t) -> uint64_t {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int idx = tid + kThreads * i;
      if (C::CHUNKS % kThreads == 0 || idx < C::CHUNKS) {
        const int row = idx / CPR;
        const int c = idx - row * CPR;
        *reinterpret_cast<u32x4*>(&smK[buf][row * KS + 8 * c]) = rk[i];
      }
    }
    if constexpr (DK != D) {
      // Zero the padded tail of each K row (head_dim 8): logical chunk 1.
      if (tid < BN) {
        const int row = tid;
        *reinterpret_cast<u32x4*>(&smK[buf][row * KS + 8]) =
            u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int gi = tid + kThreads * i;
      if (C::VGROUPS % kThreads == 0 || gi < C::VGROUPS) {
        const int kq = gi / CPR;
        const int c = gi - kq * CPR;
        // Transpose 4 keys x 8 d into 8 rows of V^T (4 consecutive keys each).
#pragma unroll
        for (int dd = 0; dd < 8; ++dd) {
          const int word = dd >> 1;
          const int shift = (dd & 1) * 16;
          u32x2 packed;
          packed[0] = ((rv[i][0][word] >> shift) & 0xffffu) | (((rv[i][1][word] >> shift) & 0xffffu) << 16);
          packed[1] = ((rv[i][2][word] >> shift) & 0xffffu) | (((rv[i][3][word] >> shift) & 0xffffu) << 16);
          *reinterpret_cast<u32x2*>(&smVt[buf][(8 * c + dd) * VTS + 4 * kq]) = packed;
        }
      }
    }
    if constexpr (HAS_MASK) {
      return __builtin_amdgcn_ballot_w64(rm);
    } else {
      return range_bits(t * BN, S);
    }
  };

  auto kread = [&](int buf, int sb, int g) -> u16x8 {
    const int row = sb * 32 + m;
    return *reinterpret_cast<const u16x8*>(&smK[buf][row * KS + 16 * g + 8 * h]);
  };
  // A operand of the P.V k-step (sb, j) for d-block db: keys
  // sb*32 + 16j + 4h + {0..3} and sb*32 + 16j + 8 + 4h + {0..3} of d-row d.
  auto vread = [&](int buf, int sb, int j, int db) -> u16x8 {
    const int d = 32 * db + m;
    if (D < 32 && d >= D) return u16x8{0, 0, 0, 0, 0, 0, 0, 0};
    const int kbase = sb * 32 + 16 * j + 4 * h;
    const u16x4 lo = *reinterpret_cast<const u16x4*>(&smVt[buf][d * VTS + kbase]);
    const u16x4 hi = *reinterpret_cast<const u16x4*>(&smVt[buf][d * VTS + kbase + 8]);
    return u16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };

  float m_run = -INFINITY;
  float l_run = 0.0f;
  f32x16 acc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i) acc[i] = f32x16{};

  auto tile = [&](auto masked_tag, int buf, int k0, int nlive, uint64_t kvalid) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    f32x16 s[NSB];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) s[sb] = f32x16{};
    u16x8 kf[NSB];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
      if (!MASKED || sb < nlive) kf[sb] = kread(buf, sb, 0);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      u16x8 kn[NSB];
      if (g + 1 < G) {
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb)
          if (!MASKED || sb < nlive) kn[sb] = kread(buf, sb, g + 1);
      }
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) {
        if (MASKED && sb >= nlive) continue;
        s[sb] = mfma_16(T{}, kf[sb], qf[g], s[sb]);
      }
      if (g + 1 < G) {
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb) kf[sb] = kn[sb];
      }
      fence();
    }
    // Scores to the exp2 domain (fp32, after the product).
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) s[sb] *= p.scale_log2;
    if constexpr (MASKED) {
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) {
        const int ks = k0 + sb * 32;
        const uint32_t a = lane_allowed<CAUSAL>(static_cast<uint32_t>(kvalid >> (32 * sb)), ks, qrow, h);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (!reg_allowed(a, r)) s[sb][r] = -INFINITY;
      }
    }
    online_softmax<NSB, NDB, MASKED>(s, m_run, l_run, acc);
    // P^T in the B-operand layout of the 32x32x16 MFMA: k-step (sb, j) takes
    // registers 8j..8j+7, i.e. keys 16j+4h+{0..3} and 16j+8+4h+{0..3}.
    u16x8 pk[NSB][2];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
      for (int r = 0; r < 16; ++r) pk[sb][r >> 3][r & 7] = to_bits(T{}, s[sb][r]);
    fence();
    constexpr int NSTEP = NSB * 2 * NDB;
    const int nsteps = (MASKED ? nlive : NSB) * 2 * NDB;
    u16x8 vf = vread(buf, 0, 0, 0);
#pragma unroll
    for (int idx = 0; idx < NSTEP; ++idx) {
      if (!MASKED || idx < nsteps) {
        const int db = idx % NDB;
        const int j = (idx / NDB) & 1;
        const int sb = idx / (2 * NDB);
        u16x8 vn{};
        const int nx = idx + 1;
        if (nx < NSTEP && (!MASKED || nx < nsteps)) {
          vn = vread(buf, nx / (2 * NDB), (nx / NDB) & 1, nx % NDB);
        }
        acc[db] = mfma_16(T{}, vf, pk[sb][j], acc[db]);
        vf = vn;
      }
      fence();
    }
  };

  gload(0);
  uint64_t kvalid = lstore(0, 0);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) gload(t + 1);
    const int k0 = t * BN;
    if (q0 < S && (!CAUSAL || k0 <= q0 + 31)) {
      int nlive = NSB;
#pragma unroll
      for (int sb = NSB - 1; sb >= 0; --sb) {
        const int ks = k0 + sb * 32;
        if (ks >= S || (CAUSAL && ks > q0 + 31)) nlive = sb;
      }
      const bool need_mask = HAS_MASK || (k0 + BN > S) || (CAUSAL && k0 + BN - 1 > q0);
      if (need_mask) {
        tile(std::true_type{}, buf, k0, nlive, kvalid);
      } else {
        tile(std::false_type{}, buf, k0, NSB, kvalid);
      }
    }
    if (t + 1 < ntiles) kvalid = lstore(buf ^ 1, t + 1);
    __syncthreads();
  }

  const float lt = l_run + __shfl_xor(l_run, 32);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  if (qrow >= S) return;
  St* __restrict__ O = static_cast<St*>(p.out) + b * p.ob + hh * p.oh + qrow * p.os;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int j4 = 0; j4 < 4; ++j4) {
      const int d0 = 32 * db + 8 * j4 + 4 * h;  // 4 consecutive d-rows
      if (D < 32 && d0 >= D) continue;
      u16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = to_bits(T{}, acc[db][4 * j4 + e] * inv);
      *reinterpret_cast<u16x4*>(O + d0) = o;
    }
}

template <int D, bool CAUSAL, bool HAS_MASK>
hipError_t launch_d(int dtype, const AttnParams& p, int grid, hipStream_t stream) {
  const dim3 g(static_cast<unsigned>(grid)), blk(kThreads);
  switch (dtype) {
    case 0: attn_fwd_f32_kernel<D, CAUSAL, HAS_MASK><<<g, blk, 0, stream>>>(p); break;
    case 1: attn_fwd_h16_kernel<BF16, D, CAUSAL, HAS_MASK><<<g, blk, 0, stream>>>(p); break;
    case 2: attn_fwd_h16_kernel<F16, D, CAUSAL, HAS_MASK><<<g, blk, 0, stream>>>(p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int D>
hipError_t launch_flags(int dtype, bool causal, bool has_mask, const AttnParams& p, int grid,
                        hipStream_t stream) {
  if (causal) {
    return has_mask ? launch_d<D, true, true>(dtype, p, grid, stream)
                    : launch_d<D, true, false>(dtype, p, grid, stream);
  }
  return has_mask ? launch_d<D, false, true>(dtype, p, grid, stream)
                  : launch_d<D, false, false>(dtype, p, grid, stream);
}

}  // namespace

int attention_block_m(int /*dtype*/, int /*D*/) { return kBM; }

hipError_t launch_attention(int dtype, int D, bool causal, bool has_mask, const AttnParams& p,
                            int grid, hipStream_t stream) {
  switch (D) {
    case 8: return launch_flags<8>(dtype, causal, has_mask, p, grid, stream);
    case 16: return launch_flags<16>(dtype, causal, has_mask, p, grid, stream);
    case 32: return launch_flags<32>(dtype, causal, has_mask, p, grid, stream);
    case 64: return launch_flags<64>(dtype, causal, has_mask, p, grid, stream);
    case 128: return launch_flags<128>(dtype, causal, has_mask, p, grid, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ttk
