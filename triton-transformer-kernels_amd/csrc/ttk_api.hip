// C ABI of libttk_hip.so: argument validation and kernel dispatch.
//
// The entry points validate everything the kernels assume (non-null
// pointers, positive sizes, 16-byte row alignment, supported head dims and
// dtypes) BEFORE any HIP call, so a rejected call touches no device state.
// They never allocate, free, synchronise or keep pointers; the kernels are
// enqueued on the caller's stream, which keeps every call capturable in a
// hipGraph.  The only global state is the thread-local error message.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <atomic>
#include <limits>
#include <mutex>

#include "ttk_common.h"
#include "ttk_hip.h"

namespace {

thread_local char g_error[512] = "";

ttk_status fail(ttk_status status, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return status;
}

int elem_bytes(int dtype) {
  switch (dtype) {
    case TTK_F32: return 4;
    case TTK_BF16: return 2;
    case TTK_F16: return 2;
    default: return 0;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static_assert(ttk::kSplitCounterBytes == TTK_ATTENTION_WS_COUNTER_BYTES,
              "the counter block of the header is the kernels' one");

// HIP launches at most 2^32 - 1 work-items per grid dimension; every kernel
// here runs 256-thread workgroups on a 1-D grid.
constexpr int64_t kMaxGroups = int64_t{0xFFFFFFFF} / 256;

}  // namespace

extern "C" int ttk_abi_version(void) { return TTK_ABI_VERSION; }

extern "C" const char* ttk_last_error(void) { return g_error; }

namespace {

ttk_status attention_fwd(const void* q, const void* k, const void* v, const uint8_t* key_valid,
                         void* out, int dtype, int64_t B, int64_t S, int64_t H, int64_t D,
                         const int64_t q_strides[3], const int64_t k_strides[3],
                         const int64_t v_strides[3], const int64_t mask_strides[2],
                         const int64_t o_strides[3], float scale, int causal, void* workspace,
                         size_t workspace_bytes, void* stream) {
  g_error[0] = '\0';
  const int es = elem_bytes(dtype);
  if (es == 0) return fail(TTK_EUNSUPPORTED, "attention: unsupported dtype code %d", dtype);
  if (B < 0 || S <= 0 || H <= 0 || D <= 0) {
    return fail(TTK_EINVAL,
                "attention: sequence length, head count, and head dimension must be positive "
                "(B=%lld S=%lld H=%lld D=%lld)",
                (long long)B, (long long)S, (long long)H, (long long)D);
  }
  if (D != 8 && D != 16 && D != 32 && D != 64 && D != 128) {
    return fail(TTK_EUNSUPPORTED, "attention: head_dim=%lld is outside [8, 16, 32, 64, 128]",
                (long long)D);
  }
  if (!q_strides || !k_strides || !v_strides || !o_strides) {
    return fail(TTK_EINVAL, "attention: stride arrays must not be NULL");
  }
  if (key_valid != nullptr && mask_strides == nullptr) {
    return fail(TTK_EINVAL, "attention: key_valid given without mask_strides");
  }
  if (B == 0) return TTK_OK;  // empty batch: nothing to launch
  if (!q || !k || !v || !out) return fail(TTK_EINVAL, "attention: q, k, v and out must not be NULL");
  if (S > (int64_t{1} << 24)) {
    return fail(TTK_EUNSUPPORTED, "attention: seq_len=%lld exceeds the kernel limit %d",
                (long long)S, 1 << 24);
  }
  const int64_t bm = ttk::attention_block_m(dtype, static_cast<int>(D));
  const int64_t nq = (S + bm - 1) / bm;
  // The largest grid any schedule launches is one workgroup per (batch,
  // head, 128-query tile).
  if (B > kMaxGroups || H > kMaxGroups || B * H > kMaxGroups / nq) {
    return fail(TTK_EUNSUPPORTED,
                "attention: B*H*ceil(S/%lld) workgroups exceed the launch limit %lld "
                "(B=%lld S=%lld H=%lld)",
                (long long)bm, (long long)kMaxGroups, (long long)B, (long long)S, (long long)H);
  }
  const void* ptrs[4] = {q, k, v, out};
  const int64_t* strides[4] = {q_strides, k_strides, v_strides, o_strides};
  const char* names[4] = {"q", "k", "v", "out"};
  for (int i = 0; i < 4; ++i) {
    if (!aligned16(ptrs[i])) {
      return fail(TTK_EUNSUPPORTED, "attention: %s is not 16-byte aligned", names[i]);
    }
    for (int a = 0; a < 3; ++a) {
      if (strides[i][a] < 0 || (strides[i][a] * es) % 16 != 0) {
        return fail(TTK_EUNSUPPORTED,
                    "attention: %s stride[%d]=%lld is not a non-negative multiple of 16 bytes",
                    names[i], a, (long long)strides[i][a]);
      }
    }
  }
  // The kernels keep per-lane K/V offsets of up to 64 rows in 32-bit integers.
  if (k_strides[1] >= (int64_t{1} << 25) || v_strides[1] >= (int64_t{1} << 25)) {
    return fail(TTK_EUNSUPPORTED, "attention: k/v sequence stride exceeds %d elements", 1 << 25);
  }
  if (key_valid != nullptr && (mask_strides[0] < 0 || mask_strides[1] < 0)) {
    return fail(TTK_EINVAL, "attention: mask strides must be non-negative");
  }

  ttk::AttnParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.mask = key_valid;
  p.out = out;
  p.qb = q_strides[0]; p.qs = q_strides[1]; p.qh = q_strides[2];
  p.kb = k_strides[0]; p.ks = k_strides[1]; p.kh = k_strides[2];
  p.vb = v_strides[0]; p.vs = v_strides[1]; p.vh = v_strides[2];
  p.ob = o_strides[0]; p.os = o_strides[1]; p.oh = o_strides[2];
  p.mb = key_valid ? mask_strides[0] : 0;
  p.ms = key_valid ? mask_strides[1] : 0;
  p.S = static_cast<int>(S);
  p.H = static_cast<int>(H);
  p.BH = static_cast<int>(B * H);
  p.nq = static_cast<int>(nq);
  p.scale_log2 = scale * 1.4426950408889634f;
  p.xcd_swizzle = (p.BH % 8 == 0) ? 1 : 0;

  if (workspace != nullptr && (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0) {
    return fail(TTK_EINVAL, "attention: workspace is not 256-byte aligned");
  }
  const hipError_t err = ttk::launch_attention(
      dtype, static_cast<int>(D), causal != 0, key_valid != nullptr, p, workspace,
      static_cast<int64_t>(std::min<size_t>(workspace_bytes, size_t{1} << 62)),
      static_cast<hipStream_t>(stream));
  if (err != hipSuccess) {
    return fail(TTK_ELAUNCH, "attention: launch failed: %s", hipGetErrorString(err));
  }
  return TTK_OK;
}

}  // namespace

extern "C" ttk_status ttk_attention_fwd(const void* q, const void* k, const void* v,
                                        const uint8_t* key_valid, void* out, int dtype,
                                        int64_t B, int64_t S, int64_t H, int64_t D,
                                        const int64_t q_strides[3], const int64_t k_strides[3],
                                        const int64_t v_strides[3], const int64_t mask_strides[2],
                                        const int64_t o_strides[3], float scale, int causal,
                                        void* stream) {
  return attention_fwd(q, k, v, key_valid, out, dtype, B, S, H, D, q_strides, k_strides, v_strides,
                       mask_strides, o_strides, scale, causal, nullptr, 0, stream);
}

extern "C" size_t ttk_attention_workspace_size(int dtype, int64_t B, int64_t S, int64_t H, int64_t D,
                                               int causal) {
  if (elem_bytes(dtype) == 0 || B <= 0 || S <= 0 || H <= 0 || B > kMaxGroups || H > kMaxGroups ||
      (D != 8 && D != 16 && D != 32 && D != 64 && D != 128) || S > (int64_t{1} << 24)) {
    return 0;
  }
  return static_cast<size_t>(
      ttk::attention_workspace_bytes(dtype, static_cast<int>(D), causal != 0, B * H, S));
}

namespace {

// Scratch of ttk_attention_fwd_noalloc: the key-split schedule's counters and
// partial states live in this static device array instead of a caller's or
// an allocated workspace.  Every GPU the library runs on holds its own copy
// from module load until the process ends.  It starts zero-filled, and every
// launch leaves its counters zero again.
constexpr size_t kScratchBytes = size_t{32} << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

// Device address of `scratch` per device.  The array's name is only a
// host-side handle: kernels and copies get this address, looked up once per
// device with that device current.
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mutex;

ttk_status scratch_address(void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    return fail(TTK_ELAUNCH, "attention_noalloc: no current device (%s)", hipGetErrorString(err));
  }
  void* ptr = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ptr = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (err != hipSuccess || ptr == nullptr) {
        return fail(TTK_ELAUNCH, "attention_noalloc: scratch address lookup failed: %s",
                    hipGetErrorString(err));
      }
      g_scratch_addr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return TTK_OK;
}

}  // namespace

extern "C" ttk_status ttk_attention_fwd_noalloc(const void* q, const void* k, const void* v,
                                                const uint8_t* key_valid, void* out, int dtype,
                                                int64_t B, int64_t S, int64_t H, int64_t D,
                                                const int64_t q_strides[3],
                                                const int64_t k_strides[3],
                                                const int64_t v_strides[3],
                                                const int64_t mask_strides[2],
                                                const int64_t o_strides[3], float scale,
                                                int causal, void* stream) {
  g_error[0] = '\0';
  const size_t need = ttk_attention_workspace_size(dtype, B, S, H, D, causal);
  if (need > kScratchBytes) {
    return fail(TTK_EUNSUPPORTED,
                "attention_noalloc: this launch's key-split schedule needs %zu bytes of scratch, "
                "above the static maximum of %zu bytes (use ttk_attention_fwd_ws)",
                need, kScratchBytes);
  }
  void* ws = nullptr;
  if (need > 0) {
    const ttk_status st = scratch_address(&ws);
    if (st != TTK_OK) return st;
  }
  return attention_fwd(q, k, v, key_valid, out, dtype, B, S, H, D, q_strides, k_strides, v_strides,
                       mask_strides, o_strides, scale, causal, ws, need > 0 ? kScratchBytes : 0, stream);
}

extern "C" ttk_status ttk_attention_fwd_ws(const void* q, const void* k, const void* v,
                                           const uint8_t* key_valid, void* out, int dtype,
                                           int64_t B, int64_t S, int64_t H, int64_t D,
                                           const int64_t q_strides[3], const int64_t k_strides[3],
                                           const int64_t v_strides[3], const int64_t mask_strides[2],
                                           const int64_t o_strides[3], float scale, int causal,
                                           void* workspace, size_t workspace_bytes, void* stream) {
  return attention_fwd(q, k, v, key_valid, out, dtype, B, S, H, D, q_strides, k_strides, v_strides,
                       mask_strides, o_strides, scale, causal, workspace, workspace_bytes, stream);
}

extern "C" ttk_status ttk_residual_layernorm_fwd(const void* x, const void* u, const void* w,
                                                 const void* b, const uint8_t* row_valid,
                                                 void* residual_out, void* normalized_out,
                                                 int dtype, int64_t rows, int64_t N, float eps,
                                                 int zero_invalid_residual,
                                                 int zero_invalid_normalized, void* stream) {
  g_error[0] = '\0';
  const int es = elem_bytes(dtype);
  if (es == 0) return fail(TTK_EUNSUPPORTED, "layernorm: unsupported dtype code %d", dtype);
  if (rows < 0 || N <= 0) {
    return fail(TTK_EINVAL, "layernorm: rows must be >= 0 and N > 0 (rows=%lld N=%lld)",
                (long long)rows, (long long)N);
  }
  if (N > 65536) {
    return fail(TTK_EUNSUPPORTED,
                "layernorm: normalized feature dimension %lld exceeds the fused kernel limit 65536",
                (long long)N);
  }
  if ((zero_invalid_residual || zero_invalid_normalized) && row_valid == nullptr) {
    return fail(TTK_EINVAL, "layernorm: invalid-row zeroing requires valid_token_mask");
  }
  if (rows == 0) return TTK_OK;
  if (!x || !w || !normalized_out) {
    return fail(TTK_EINVAL, "layernorm: x, weight and normalized_out must not be NULL");
  }

  ttk::LnParams p{};
  p.x = x;
  p.u = u;
  p.w = w;
  p.b = b;
  p.valid = row_valid;
  p.r_out = residual_out;
  p.y_out = normalized_out;
  p.rows = rows;
  p.N = static_cast<int>(N);
  p.eps = eps;
  p.zero_res = zero_invalid_residual ? 1 : 0;
  p.zero_norm = zero_invalid_normalized ? 1 : 0;

  // Register-resident vector path: whole 16-byte vectors, aligned tensors,
  // at most 16 vectors per lane.
  const int vn = 16 / es;
  bool vector_path = (N % vn) == 0;
  for (const void* ptr : {x, u, w, b, static_cast<const void*>(residual_out),
                          static_cast<const void*>(normalized_out)}) {
    if (ptr != nullptr && !aligned16(ptr)) vector_path = false;
  }
  int vpl = 0;
  if (vector_path) {
    const int64_t nv = N / vn;
    int lpr = 1;
    while (lpr < 64 && nv % (2 * lpr) == 0) lpr *= 2;
    int64_t per_lane = nv / lpr;
    // Narrow rows: several rows per wavefront, >= 4 vectors per lane.
    while (per_lane < 4 && lpr > 8) {
      lpr /= 2;
      per_lane *= 2;
    }
    if (per_lane > 16) {
      vector_path = false;
    } else {
      p.lanes_per_row = lpr;
      vpl = static_cast<int>(per_lane);
    }
  }
  // Grid of the chosen path: one workgroup per row (fallback) or per four
  // wavefronts of 64 / lanes_per_row rows each (vector path).
  const int64_t groups = vector_path
      ? ((rows + 64 / p.lanes_per_row - 1) / (64 / p.lanes_per_row) + 3) / 4
      : rows;
  if (groups > kMaxGroups) {
    return fail(TTK_EUNSUPPORTED,
                "layernorm: %lld rows of width %lld need %lld workgroups, above the launch "
                "limit %lld",
                (long long)rows, (long long)N, (long long)groups, (long long)kMaxGroups);
  }
  const hipError_t err = ttk::launch_residual_layernorm(dtype, p, vector_path, vpl,
                                                        static_cast<hipStream_t>(stream));
  if (err != hipSuccess) {
    return fail(TTK_ELAUNCH, "layernorm: launch failed: %s", hipGetErrorString(err));
  }
  return TTK_OK;
}

extern "C" ttk_status ttk_gelu_fwd(const void* x, void* y, int dtype, int64_t n, void* stream) {
  g_error[0] = '\0';
  const int es = elem_bytes(dtype);
  if (es == 0) return fail(TTK_EUNSUPPORTED, "gelu: unsupported dtype code %d", dtype);
  if (n < 0) return fail(TTK_EINVAL, "gelu: negative element count %lld", (long long)n);
  // An unaligned buffer runs one element per work-item.
  if (n > kMaxGroups * 256) {
    return fail(TTK_EUNSUPPORTED, "gelu: element count %lld exceeds the launch limit %lld",
                (long long)n, (long long)(kMaxGroups * 256));
  }
  if (n == 0) return TTK_OK;
  if (!x || !y) return fail(TTK_EINVAL, "gelu: x and y must not be NULL");
  const uintptr_t xb = reinterpret_cast<uintptr_t>(x), yb = reinterpret_cast<uintptr_t>(y);
  const uintptr_t bytes = static_cast<uintptr_t>(n) * static_cast<uintptr_t>(es);
  if (xb != yb && xb < yb + bytes && yb < xb + bytes) {
    return fail(TTK_EINVAL, "gelu: x and y overlap without being the same buffer");
  }
  const hipError_t err = ttk::launch_gelu(dtype, x, y, n, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(TTK_ELAUNCH, "gelu: launch failed: %s", hipGetErrorString(err));
  return TTK_OK;
}

namespace {

bool overlaps(const void* a, uint64_t abytes, const void* b, uint64_t bbytes) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + bbytes && y < x + abytes;
}

}  // namespace

extern "C" ttk_status ttk_linear_fwd(const void* x, const void* w, const void* bias, void* y, int dtype,
                                     int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldw,
                                     int64_t ldy, int activation, void* stream) {
  g_error[0] = '\0';
  if (dtype != TTK_BF16 && dtype != TTK_F16) {
    return fail(TTK_EUNSUPPORTED, "linear: dtype code %d is not bf16 or fp16", dtype);
  }
  if (activation != TTK_ACT_NONE && activation != TTK_ACT_GELU) {
    return fail(TTK_EINVAL, "linear: unknown activation code %d", activation);
  }
  if (M < 0 || N <= 0 || K <= 0) {
    return fail(TTK_EINVAL, "linear: M must be >= 0 and N, K positive (M=%lld N=%lld K=%lld)",
                (long long)M, (long long)N, (long long)K);
  }
  if (M == 0) return TTK_OK;
  if (!x || !w || !y) return fail(TTK_EINVAL, "linear: x, w and y must not be NULL");
  if (K % 128 != 0 || K < 256) {
    return fail(TTK_EUNSUPPORTED, "linear: K=%lld must be a multiple of 128 and at least 256",
                (long long)K);
  }
  if (N % 32 != 0) return fail(TTK_EUNSUPPORTED, "linear: N=%lld must be a multiple of 32", (long long)N);
  if (!aligned16(x) || !aligned16(w) || !aligned16(y)) {
    return fail(TTK_EUNSUPPORTED, "linear: x, w and y must be 16-byte aligned");
  }
  if (ldx % 8 != 0 || ldw % 8 != 0 || ldy % 8 != 0 || ldx < K || ldw < K || ldy < N) {
    return fail(TTK_EUNSUPPORTED,
                "linear: row strides must be multiples of 8 elements with ldx, ldw >= K and "
                "ldy >= N (ldx=%lld ldw=%lld ldy=%lld)",
                (long long)ldx, (long long)ldw, (long long)ldy);
  }
  if (bias != nullptr && (reinterpret_cast<uintptr_t>(bias) & 3u) != 0) {
    return fail(TTK_EUNSUPPORTED, "linear: bias must be 4-byte aligned");
  }
  const uint64_t xbytes = (static_cast<uint64_t>(M - 1) * ldx + K) * 2;
  const uint64_t wbytes = (static_cast<uint64_t>(N - 1) * ldw + K) * 2;
  const uint64_t ybytes = static_cast<uint64_t>(M) * ldy * 2;
  if (xbytes >= (uint64_t{1} << 32) || wbytes >= (uint64_t{1} << 32) || ybytes >= (uint64_t{1} << 31)) {
    return fail(TTK_EUNSUPPORTED,
                "linear: x or w spans 2^32 bytes or more, or y 2^31 bytes or more (M=%lld N=%lld "
                "K=%lld)",
                (long long)M, (long long)N, (long long)K);
  }
  if (overlaps(y, ybytes, x, xbytes) || overlaps(y, ybytes, w, wbytes) ||
      (bias != nullptr && overlaps(y, ybytes, bias, static_cast<uint64_t>(N) * 2))) {
    return fail(TTK_EINVAL, "linear: y overlaps x, w or bias");
  }
  ttk::LinearParams p{};
  p.x = x;
  p.w = w;
  p.bias = bias;
  p.y = y;
  p.ldx = ldx;
  p.ldw = ldw;
  p.ldy = ldy;
  p.M = static_cast<int>(M);
  p.N = static_cast<int>(N);
  p.K = static_cast<int>(K);
  p.y_bytes = static_cast<unsigned>(ybytes);
  const hipError_t err = ttk::launch_linear(dtype, activation, p, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(TTK_ELAUNCH, "linear: launch failed: %s", hipGetErrorString(err));
  return TTK_OK;
}

namespace {
constexpr int64_t kLnRowsPerBlock = 64;
constexpr int64_t kLnWidth = 1024;

constexpr int kLnDefaultPolls = 4096;

// A counter block of fixed size (one counter per 64-row block of the largest
// M the entry point takes: x, r and y stay below 2^31 bytes, so M < 2^20),
// then the statistics area (1 KB per 64-row block).  The counters sit at the
// same bytes for every M, so launches of any shapes can share a workspace.
constexpr int64_t kLnCounterBytes = ((int64_t{1} << 20) / kLnRowsPerBlock) * 4;
int64_t ln_counter_bytes(int64_t) { return kLnCounterBytes; }
static_assert(kLnCounterBytes == TTK_LINEAR_LN_WS_COUNTER_BYTES, "the header's counter block");

}  // namespace

extern "C" int64_t ttk_linear_residual_ln_workspace_size(int64_t M) {
  if (M <= 0) return 0;
  return ln_counter_bytes(M) + (M + kLnRowsPerBlock - 1) / kLnRowsPerBlock * 1024;
}

extern "C" ttk_status ttk_linear_pack_weight(const void* w, void* w_packed, int dtype, int64_t N,
                                             int64_t K, int64_t ldw, void* stream) {
  g_error[0] = '\0';
  if (dtype != TTK_BF16 && dtype != TTK_F16) {
    return fail(TTK_EUNSUPPORTED, "pack weight: dtype code %d is not bf16 or fp16", dtype);
  }
  if (N <= 0 || K <= 0) {
    return fail(TTK_EINVAL, "pack weight: N and K must be positive (N=%lld K=%lld)", (long long)N,
                (long long)K);
  }
  if (!w || !w_packed) return fail(TTK_EINVAL, "pack weight: w and w_packed must not be NULL");
  if (N % 32 != 0 || K % 16 != 0) {
    return fail(TTK_EUNSUPPORTED, "pack weight: N=%lld must be a multiple of 32 and K=%lld of 16",
                (long long)N, (long long)K);
  }
  if (!aligned16(w) || !aligned16(w_packed) || ldw % 8 != 0 || ldw < K) {
    return fail(TTK_EUNSUPPORTED,
                "pack weight: w and w_packed must be 16-byte aligned, ldw a multiple of 8 and >= K "
                "(ldw=%lld)",
                (long long)ldw);
  }
  if (N > (int64_t{1} << 30) || K > (int64_t{1} << 30)) {
    return fail(TTK_EUNSUPPORTED, "pack weight: N or K too large");
  }
  const uint64_t wbytes = (static_cast<uint64_t>(N - 1) * ldw + K) * 2;
  if (overlaps(w_packed, static_cast<uint64_t>(N) * K * 2, w, wbytes)) {
    return fail(TTK_EINVAL, "pack weight: w_packed overlaps w");
  }
  const hipError_t err = ttk::launch_pack_weight(w, w_packed, static_cast<int>(N), static_cast<int>(K), ldw,
                                                 static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(TTK_ELAUNCH, "pack weight: launch failed: %s", hipGetErrorString(err));
  return TTK_OK;
}

extern "C" ttk_status ttk_linear_residual_ln_fwd(const void* a, const void* w_packed, const void* bias,
                                                 const void* x, const void* gamma, const void* beta,
                                                 void* r, void* y, void* workspace,
                                                 int64_t workspace_bytes, int dtype, int64_t M,
                                                 int64_t N, int64_t K, int64_t lda, int64_t ldx,
                                                 int64_t ldr, int64_t ldy, float eps, int max_polls,
                                                 void* stream) {
  g_error[0] = '\0';
  if (dtype != TTK_BF16 && dtype != TTK_F16) {
    return fail(TTK_EUNSUPPORTED, "linear+LN: dtype code %d is not bf16 or fp16", dtype);
  }
  if (M < 0 || N <= 0 || K <= 0) {
    return fail(TTK_EINVAL, "linear+LN: M must be >= 0 and N, K positive (M=%lld N=%lld K=%lld)",
                (long long)M, (long long)N, (long long)K);
  }
  if (N != kLnWidth) {
    return fail(TTK_EUNSUPPORTED, "linear+LN: N=%lld; the kernel normalises rows of 1024", (long long)N);
  }
  if (K % 128 != 0 || K > (int64_t{1} << 24)) {
    return fail(TTK_EUNSUPPORTED, "linear+LN: K=%lld must be a positive multiple of 128", (long long)K);
  }
  if (M == 0) return TTK_OK;
  if (!a || !w_packed || !x || !gamma || !r || !y || !workspace) {
    return fail(TTK_EINVAL, "linear+LN: a, w_packed, x, gamma, r, y and workspace must not be NULL");
  }
  if (!aligned16(a) || !aligned16(w_packed) || !aligned16(x) || !aligned16(gamma) || !aligned16(r) ||
      !aligned16(y) || (beta != nullptr && !aligned16(beta))) {
    return fail(TTK_EUNSUPPORTED, "linear+LN: a, w_packed, x, gamma, beta, r and y must be 16-byte aligned");
  }
  if (bias != nullptr && (reinterpret_cast<uintptr_t>(bias) & 1u) != 0) {
    return fail(TTK_EUNSUPPORTED, "linear+LN: bias must be 2-byte aligned");
  }
  if ((reinterpret_cast<uintptr_t>(workspace) & 3u) != 0 ||
      workspace_bytes < ttk_linear_residual_ln_workspace_size(M)) {
    return fail(TTK_EINVAL, "linear+LN: workspace must be 4-byte aligned and hold %lld bytes (got %lld)",
                (long long)ttk_linear_residual_ln_workspace_size(M), (long long)workspace_bytes);
  }
  if (lda % 8 != 0 || ldx % 8 != 0 || ldr % 8 != 0 || ldy % 8 != 0 || lda < K || ldx < N ||
      ldr < N || ldy < N) {
    return fail(TTK_EUNSUPPORTED,
                "linear+LN: row strides must be multiples of 8 elements with lda >= K and ldx, ldr, "
                "ldy >= N (lda=%lld ldx=%lld ldr=%lld ldy=%lld)",
                (long long)lda, (long long)ldx, (long long)ldr, (long long)ldy);
  }
  const uint64_t abytes = (static_cast<uint64_t>(M - 1) * lda + K) * 2;
  const uint64_t xbytes = static_cast<uint64_t>(M) * ldx * 2;
  const uint64_t rbytes = static_cast<uint64_t>(M) * ldr * 2;
  const uint64_t ybytes = static_cast<uint64_t>(M) * ldy * 2;
  if (xbytes >= (uint64_t{1} << 31) || rbytes >= (uint64_t{1} << 31) || ybytes >= (uint64_t{1} << 31) ||
      M > (int64_t{1} << 30)) {
    return fail(TTK_EUNSUPPORTED, "linear+LN: x, r or y spans 2^31 bytes or more (M=%lld)", (long long)M);
  }
  const uint64_t wbytes = static_cast<uint64_t>(N) * K * 2;
  const uint64_t ws_used = static_cast<uint64_t>(ttk_linear_residual_ln_workspace_size(M));
  struct Span {
    const void* p;
    uint64_t n;
  };
  const Span inputs[] = {{a, abytes}, {w_packed, wbytes}, {x, xbytes}, {gamma, static_cast<uint64_t>(N) * 2},
                         {beta, beta ? static_cast<uint64_t>(N) * 2 : 0},
                         {bias, bias ? static_cast<uint64_t>(N) * 2 : 0}, {workspace, ws_used}};
  for (const Span& in : inputs) {
    if (in.p != nullptr && (overlaps(r, rbytes, in.p, in.n) || overlaps(y, ybytes, in.p, in.n))) {
      return fail(TTK_EINVAL, "linear+LN: r or y overlaps an input or the workspace");
    }
  }
  if (overlaps(r, rbytes, y, ybytes)) return fail(TTK_EINVAL, "linear+LN: r overlaps y");
  ttk::LinearLnParams p{};
  p.a = a;
  p.wp = w_packed;
  p.bias = bias;
  p.x = x;
  p.gamma = gamma;
  p.beta = beta;
  p.r = r;
  p.y = y;
  p.counters = static_cast<int*>(workspace);
  p.stats = reinterpret_cast<float*>(static_cast<char*>(workspace) + ln_counter_bytes(M));
  p.max_polls = max_polls < 0 ? kLnDefaultPolls : max_polls;
  p.lda = lda;
  p.ldx = ldx;
  p.ldr = ldr;
  p.ldy = ldy;
  p.M = static_cast<int>(M);
  p.K = static_cast<int>(K);
  p.eps = eps;
  p.x_bytes = static_cast<unsigned>(xbytes);
  p.r_bytes = static_cast<unsigned>(rbytes);
  p.y_bytes = static_cast<unsigned>(ybytes);
  const hipError_t err = ttk::launch_linear_ln(dtype, p, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(TTK_ELAUNCH, "linear+LN: launch failed: %s", hipGetErrorString(err));
  return TTK_OK;
}
