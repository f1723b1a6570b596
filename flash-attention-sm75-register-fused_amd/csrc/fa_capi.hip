// C ABI of the library: argument validation, status codes, the stream-ordered
// entry points and the four reference-signature launchers.
//
// Every check runs before the first HIP call, so all error paths are
// reachable without a device.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <atomic>
#include <cstring>
#include <mutex>
#include <string>

#include "fa_internal.h"
#include "flash_attn_sm75.h"

namespace {

thread_local char g_last_error[512] = "";

// Which fused kernel fa_sm75_forward launches (process-wide).
std::atomic<int> g_kernel_policy{FA_POLICY_AUTO};

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Key/value rows of a call (seq_len_kv == 0 selects seq_len).
int64_t kv_rows(const fa_fwd_params* p) {
  return p->seq_len_kv != 0 ? p->seq_len_kv : p->seq_len;
}

// Shared validation of the fused and naive entry points.
int validate(const fa_fwd_params* p, bool fused) {
  if (p == nullptr) return fail(FA_ERR_INVALID_ARGUMENT, "params must not be NULL");
  if (p->batch < 0 || p->heads_q < 0 || p->heads_kv < 0 || p->seq_len < 0 ||
      p->head_dim < 0 || p->seq_len_kv < 0)
    return fail(FA_ERR_INVALID_ARGUMENT,
                "sizes must be non-negative (batch=%lld heads_q=%lld heads_kv=%lld "
                "seq_len=%lld head_dim=%lld)",
                (long long)p->batch, (long long)p->heads_q, (long long)p->heads_kv,
                (long long)p->seq_len, (long long)p->head_dim);
  if (fused) {
    if (p->head_dim != 64 && p->head_dim != 128)
      return fail(FA_ERR_UNSUPPORTED_HEAD_DIM,
                  "flash_attention_forward supports head_dim=64 or 128, got %lld",
                  (long long)p->head_dim);
  } else {
    if (p->head_dim < 1 || p->head_dim > 256 || (p->head_dim % 8) != 0)
      return fail(FA_ERR_UNSUPPORTED_HEAD_DIM,
                  "naive_attention supports head_dim multiple of 8 in [8, 256], got %lld",
                  (long long)p->head_dim);
  }
  if (p->heads_q > 0 && p->heads_kv == 0)
    return fail(FA_ERR_HEADS_NOT_DIVISIBLE, "heads_kv must be positive");
  if (p->heads_kv > 0 && (p->heads_q % p->heads_kv) != 0)
    return fail(FA_ERR_HEADS_NOT_DIVISIBLE,
                "heads mismatch: Q heads (%lld) not divisible by K/V heads (%lld)",
                (long long)p->heads_q, (long long)p->heads_kv);
  if (!std::isfinite(p->scale))
    return fail(FA_ERR_INVALID_ARGUMENT, "scale must be finite");
  if (p->causal < FA_CAUSAL_NONE || p->causal > FA_CAUSAL_BOTTOM_RIGHT)
    return fail(FA_ERR_INVALID_ARGUMENT, "causal must be 0, 1 (top-left) or 2 (bottom-right), got %d",
                p->causal);
  if (!fused && p->seq_len_kv != 0 && p->seq_len_kv != p->seq_len)
    return fail(FA_ERR_INVALID_ARGUMENT, "naive path needs seq_len_kv == seq_len");
  if (p->dtype != FA_DTYPE_FP16 && p->dtype != FA_DTYPE_BF16)
    return fail(FA_ERR_INVALID_ARGUMENT, "dtype must be 0 (binary16) or 1 (bfloat16), got %d",
                p->dtype);
  if (!fused && p->dtype != FA_DTYPE_FP16)
    return fail(FA_ERR_INVALID_ARGUMENT, "the naive path is binary16 only");
  const bool empty = p->batch == 0 || p->heads_q == 0 || p->seq_len == 0;
  if (empty) return FA_OK;
  if (!p->q || !p->k || !p->v || !p->o)
    return fail(FA_ERR_INVALID_ARGUMENT, "Q, K, V and O pointers must not be NULL");
  if (!aligned16(p->q) || !aligned16(p->k) || !aligned16(p->v) || !aligned16(p->o))
    return fail(FA_ERR_MISALIGNED, "Q, K, V and O must be 16-byte aligned");
  if (p->workspace != nullptr && !aligned16(p->workspace))
    return fail(FA_ERR_MISALIGNED, "workspace must be 16-byte aligned");
  if (p->workspace_bytes < 0)
    return fail(FA_ERR_INVALID_ARGUMENT, "workspace_bytes must be non-negative");
  if (p->mask_bits != nullptr) {
    if (!fused)
      return fail(FA_ERR_INVALID_ARGUMENT, "the naive path takes no mask");
    if ((reinterpret_cast<uintptr_t>(p->mask_bits) & 7u) != 0)
      return fail(FA_ERR_MISALIGNED, "mask_bits must be 8-byte aligned");
    if (p->mask_stride_b < 0 || p->mask_stride_h < 0 || p->mask_stride_q < 0)
      return fail(FA_ERR_INVALID_ARGUMENT, "mask strides must be non-negative");
    if (p->mask_stride_q != 0 && p->mask_stride_q < (kv_rows(p) + 63) / 64)
      return fail(FA_ERR_INVALID_ARGUMENT,
                  "mask row stride %lld is below ceil(seq_len_kv / 64) = %lld words",
                  (long long)p->mask_stride_q, (long long)((kv_rows(p) + 63) / 64));
  }
  if (p->mask_ranges != nullptr) {
    if (p->mask_bits == nullptr)
      return fail(FA_ERR_INVALID_ARGUMENT, "mask_ranges needs mask_bits");
    if ((reinterpret_cast<uintptr_t>(p->mask_ranges) & 7u) != 0)
      return fail(FA_ERR_MISALIGNED, "mask_ranges must be 8-byte aligned");
    if (p->mask_ranges_stride_b < 0 || p->mask_ranges_stride_h < 0 ||
        p->mask_ranges_stride_q < 0)
      return fail(FA_ERR_INVALID_ARGUMENT, "mask_ranges strides must be non-negative");
  }
  if (p->mask_keys != nullptr) {
    if (!fused)
      return fail(FA_ERR_INVALID_ARGUMENT, "the naive path takes no mask");
    if (p->mask_bits != nullptr)
      return fail(FA_ERR_INVALID_ARGUMENT, "mask_bits and mask_keys are exclusive");
    if (p->mask_keys_stride_b < 0 || p->mask_keys_stride_k < 0)
      return fail(FA_ERR_INVALID_ARGUMENT, "mask_keys strides must be non-negative");
  }
  const int64_t strides[12] = {p->q_stride_b, p->q_stride_h, p->q_stride_n,
                               p->k_stride_b, p->k_stride_h, p->k_stride_n,
                               p->v_stride_b, p->v_stride_h, p->v_stride_n,
                               p->o_stride_b, p->o_stride_h, p->o_stride_n};
  for (int i = 0; i < 12; ++i) {
    if (strides[i] < 0)
      return fail(FA_ERR_INVALID_ARGUMENT, "strides must be non-negative");
    if (strides[i] % 8 != 0)
      return fail(FA_ERR_MISALIGNED,
                  "batch/head/row strides must be multiples of 8 elements (16 bytes)");
  }
  if (p->q_stride_n < p->head_dim || p->k_stride_n < p->head_dim ||
      p->v_stride_n < p->head_dim || p->o_stride_n < p->head_dim)
    return fail(FA_ERR_INVALID_ARGUMENT, "row stride must be at least head_dim");
  const int64_t nk = kv_rows(p);
  if (p->seq_len > INT32_MAX / 2 || nk > INT32_MAX / 2)
    return fail(FA_ERR_TOO_LARGE, "seq_len %lld / seq_len_kv %lld exceeds the supported maximum",
                (long long)p->seq_len, (long long)nk);
  // K/V tiles are read through 32-bit buffer windows over one (batch, head),
  // with offsets up to one tile past the last key.
  if ((nk + 64) * p->k_stride_n * 2 > (int64_t)INT32_MAX ||
      (nk + 64) * p->v_stride_n * 2 > (int64_t)INT32_MAX)
    return fail(FA_ERR_TOO_LARGE, "seq_len_kv * row stride of K/V exceeds 2^31 bytes");
  // One 1-D grid of batch*heads_q*ceil(seq_len/128) workgroups of 256
  // threads; the thread count must stay below 2^32.
  const int64_t bm = fa::fused_block_m();
  if (p->batch * p->heads_q > (int64_t)(1u << 24) ||
      p->batch * p->heads_q * ((p->seq_len + bm - 1) / bm) >= (int64_t)(1u << 24))
    return fail(FA_ERR_TOO_LARGE, "batch*heads_q*ceil(seq_len/%lld) exceeds 2^24 workgroups",
                (long long)bm);
  return FA_OK;
}

fa::FwdArgs make_args(const fa_fwd_params* p) {
  fa::FwdArgs a;
  a.q = reinterpret_cast<const _Float16*>(p->q);
  a.k = reinterpret_cast<const _Float16*>(p->k);
  a.v = reinterpret_cast<const _Float16*>(p->v);
  a.o = reinterpret_cast<_Float16*>(p->o);
  a.lse = p->lse;
  a.qsb = p->q_stride_b; a.qsh = p->q_stride_h; a.qsn = p->q_stride_n;
  a.ksb = p->k_stride_b; a.ksh = p->k_stride_h; a.ksn = p->k_stride_n;
  a.vsb = p->v_stride_b; a.vsh = p->v_stride_h; a.vsn = p->v_stride_n;
  a.osb = p->o_stride_b; a.osh = p->o_stride_h; a.osn = p->o_stride_n;
  a.n = (int)p->seq_len;
  a.nk = (int)kv_rows(p);
  a.diag = p->causal == FA_CAUSAL_BOTTOM_RIGHT ? a.nk - a.n : 0;
  a.hq = (int)p->heads_q;
  a.group = (int)(p->heads_kv > 0 ? p->heads_q / p->heads_kv : 1);
  a.num_qblocks = 0;  // grid plan: filled by the launcher
  a.units = 0;
  a.xcds = 1;
  const float log2e = 1.4426950408889634f;
  float c = std::fabs(p->scale) * log2e;
  // scale == 0 must still give uniform weights over the visible keys; a tiny
  // positive factor keeps exp2(-inf * c) = 0 for masked keys.
  if (c < 1e-30f) c = 1e-30f;
  a.c = c;
  a.negate_q = p->scale < 0.0f ? 1 : 0;
  a.mbits = p->mask_bits;
  a.msb = p->mask_stride_b;
  a.msh = p->mask_stride_h;
  a.msq = p->mask_stride_q;
  a.mkeys = p->mask_keys;
  a.mksb = p->mask_keys_stride_b;
  a.mksk = p->mask_keys_stride_k;
  a.mranges = p->mask_ranges;
  a.mrsb = p->mask_ranges_stride_b;
  a.mrsh = p->mask_ranges_stride_h;
  a.mrsq = p->mask_ranges_stride_q;
  a.ctr = nullptr;
  a.items = 0;
  a.bf16 = p->dtype == FA_DTYPE_BF16 ? 1 : 0;
  a.pair_half = 0;
  a.pair_split = 0;
  return a;
}

int check_launch() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(FA_ERR_HIP, "HIP launch failed: %s", hipGetErrorString(e));
  return FA_OK;
}

// Shared body of the reference-signature launchers: contiguous, default
// stream, synchronous, message on stderr on failure.
void legacy_launch(const char* tag, const fa_half* Q, const fa_half* K, const fa_half* V,
                   fa_half* O, int batch, int heads, int seq_len, int head_dim,
                   float scale, bool causal, bool d64_only, float* workspace) {
  if (d64_only && head_dim != 64) {
    std::fprintf(stderr, "[%s] head_dim=%d not supported\n", tag, head_dim);
    return;
  }
  fa_fwd_params p;
  std::memset(&p, 0, sizeof(p));
  p.q = Q; p.k = K; p.v = V; p.o = O;
  p.batch = batch; p.heads_q = heads; p.heads_kv = heads;
  p.seq_len = seq_len; p.head_dim = head_dim;
  fa_sm75_set_contiguous_strides(&p);
  p.scale = scale;
  p.causal = causal ? 1 : 0;
  p.stream = nullptr;
  const int st = workspace ? fa_sm75_naive_forward(&p, workspace) : fa_sm75_forward(&p);
  if (st != FA_OK) {
    std::fprintf(stderr, "[%s] %s\n", tag, fa_sm75_last_error());
    return;
  }
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) std::fprintf(stderr, "[%s] %s\n", tag, hipGetErrorString(e));
}

int64_t bwd_kv_rows(const fa_bwd_params* p) {
  return p->seq_len_kv != 0 ? p->seq_len_kv : p->seq_len;
}

bool bwd_empty(const fa_bwd_params* p) {
  return p->batch == 0 || p->heads_q == 0 || (p->seq_len == 0 && bwd_kv_rows(p) == 0);
}

// Validation of fa_sm75_backward (the forward's rules for the shared
// fields, plus the gradient tensors, the LSE and the workspace).
int validate_bwd(const fa_bwd_params* p) {
  if (p == nullptr) return fail(FA_ERR_INVALID_ARGUMENT, "params must not be NULL");
  if (p->batch < 0 || p->heads_q < 0 || p->heads_kv < 0 || p->seq_len < 0 ||
      p->head_dim < 0 || p->seq_len_kv < 0)
    return fail(FA_ERR_INVALID_ARGUMENT,
                "sizes must be non-negative (batch=%lld heads_q=%lld heads_kv=%lld "
                "seq_len=%lld head_dim=%lld)",
                (long long)p->batch, (long long)p->heads_q, (long long)p->heads_kv,
                (long long)p->seq_len, (long long)p->head_dim);
  if (p->head_dim != 64 && p->head_dim != 128)
    return fail(FA_ERR_UNSUPPORTED_HEAD_DIM,
                "flash_attention_backward supports head_dim=64 or 128, got %lld",
                (long long)p->head_dim);
  if (p->heads_q > 0 && p->heads_kv == 0)
    return fail(FA_ERR_HEADS_NOT_DIVISIBLE, "heads_kv must be positive");
  if (p->heads_kv > 0 && (p->heads_q % p->heads_kv) != 0)
    return fail(FA_ERR_HEADS_NOT_DIVISIBLE,
                "heads mismatch: Q heads (%lld) not divisible by K/V heads (%lld)",
                (long long)p->heads_q, (long long)p->heads_kv);
  if (!std::isfinite(p->scale)) return fail(FA_ERR_INVALID_ARGUMENT, "scale must be finite");
  if (p->causal < FA_CAUSAL_NONE || p->causal > FA_CAUSAL_BOTTOM_RIGHT)
    return fail(FA_ERR_INVALID_ARGUMENT,
                "causal must be 0, 1 (top-left) or 2 (bottom-right), got %d", p->causal);
  if (p->dtype != FA_DTYPE_FP16 && p->dtype != FA_DTYPE_BF16)
    return fail(FA_ERR_INVALID_ARGUMENT, "dtype must be 0 (binary16) or 1 (bfloat16), got %d",
                p->dtype);
  if (bwd_empty(p)) return FA_OK;
  // With no query rows only dK and dV (zeros) are written, from K and V's shapes.
  const bool rows = p->seq_len > 0;
  const void* ptrs[9] = {p->k, p->v, p->dk, p->dv, p->q, p->o, p->dout, p->dq, p->workspace};
  for (int i = 0; i < (rows ? 9 : 4); ++i)
    if (ptrs[i] == nullptr)
      return fail(FA_ERR_INVALID_ARGUMENT,
                  "Q, K, V, O, dO, dQ, dK, dV and workspace pointers must not be NULL");
  for (int i = 0; i < (rows ? 9 : 4); ++i)
    if (!aligned16(ptrs[i]))
      return fail(FA_ERR_MISALIGNED, "tensor and workspace pointers must be 16-byte aligned");
  if (rows && p->lse == nullptr) return fail(FA_ERR_INVALID_ARGUMENT, "lse must not be NULL");
  if ((reinterpret_cast<uintptr_t>(p->lse) & 3u) != 0)
    return fail(FA_ERR_MISALIGNED, "lse must be 4-byte aligned");
  const int64_t strides[24] = {
      p->q_stride_b,  p->q_stride_h,  p->q_stride_n,  p->k_stride_b,  p->k_stride_h,
      p->k_stride_n,  p->v_stride_b,  p->v_stride_h,  p->v_stride_n,  p->o_stride_b,
      p->o_stride_h,  p->o_stride_n,  p->do_stride_b, p->do_stride_h, p->do_stride_n,
      p->dq_stride_b, p->dq_stride_h, p->dq_stride_n, p->dk_stride_b, p->dk_stride_h,
      p->dk_stride_n, p->dv_stride_b, p->dv_stride_h, p->dv_stride_n};
  for (int i = 0; i < 24; ++i) {
    if (strides[i] < 0) return fail(FA_ERR_INVALID_ARGUMENT, "strides must be non-negative");
    if (strides[i] % 8 != 0)
      return fail(FA_ERR_MISALIGNED,
                  "batch/head/row strides must be multiples of 8 elements (16 bytes)");
  }
  for (int i = 2; i < 24; i += 3)
    if (strides[i] < p->head_dim)
      return fail(FA_ERR_INVALID_ARGUMENT, "row stride must be at least head_dim");
  const int64_t nk = bwd_kv_rows(p);
  if (p->seq_len > INT32_MAX / 2 || nk > INT32_MAX / 2)
    return fail(FA_ERR_TOO_LARGE, "seq_len %lld / seq_len_kv %lld exceeds the supported maximum",
                (long long)p->seq_len, (long long)nk);
  if (nk == 0 && p->seq_len > 0)
    return fail(FA_ERR_INVALID_ARGUMENT, "K/V must hold at least one row");
  // Q and dO tiles (dK/dV kernel) and K and V tiles (dQ kernel) are read
  // through 32-bit buffer windows over one (batch, head).
  if ((p->seq_len + 64) * p->q_stride_n * 2 > (int64_t)INT32_MAX ||
      (p->seq_len + 64) * p->do_stride_n * 2 > (int64_t)INT32_MAX ||
      (nk + 64) * p->k_stride_n * 2 > (int64_t)INT32_MAX ||
      (nk + 64) * p->v_stride_n * 2 > (int64_t)INT32_MAX)
    return fail(FA_ERR_TOO_LARGE, "rows * row stride of Q, dO, K or V exceeds 2^31 bytes");
  if (p->batch * p->heads_q * ((p->seq_len + 63) / 64) >= (int64_t)(1u << 24) ||
      p->batch * p->heads_kv * ((nk + 127) / 128) >= (int64_t)(1u << 24))
    return fail(FA_ERR_TOO_LARGE, "the backward grids exceed 2^24 workgroups");
  if (p->mask_bits != nullptr) {
    if ((reinterpret_cast<uintptr_t>(p->mask_bits) & 7u) != 0)
      return fail(FA_ERR_MISALIGNED, "mask_bits must be 8-byte aligned");
    if (p->mask_stride_b < 0 || p->mask_stride_h < 0 || p->mask_stride_q < 0)
      return fail(FA_ERR_INVALID_ARGUMENT, "mask strides must be non-negative");
    const int64_t words = (nk + 63) / 64;
    if (p->mask_stride_q != 0 && p->mask_stride_q < words)
      return fail(FA_ERR_INVALID_ARGUMENT,
                  "mask row stride %lld is below ceil(seq_len_kv / 64) = %lld words",
                  (long long)p->mask_stride_q, (long long)words);
    // The dK/dV kernel reads a tile's mask words through a 32-bit buffer window.
    if ((p->seq_len * p->mask_stride_q + words) * 8 > (int64_t)INT32_MAX)
      return fail(FA_ERR_TOO_LARGE, "seq_len * mask row stride exceeds 2^31 bytes");
  }
  if (p->mask_ranges != nullptr) {
    if (p->mask_bits == nullptr)
      return fail(FA_ERR_INVALID_ARGUMENT, "mask_ranges needs mask_bits");
    if ((reinterpret_cast<uintptr_t>(p->mask_ranges) & 7u) != 0)
      return fail(FA_ERR_MISALIGNED, "mask_ranges must be 8-byte aligned");
    if (p->mask_ranges_stride_b < 0 || p->mask_ranges_stride_h < 0 ||
        p->mask_ranges_stride_q < 0)
      return fail(FA_ERR_INVALID_ARGUMENT, "mask_ranges strides must be non-negative");
  }
  const int64_t need = fa::bwd_workspace_bytes(p->batch, p->heads_q, p->seq_len);
  if (p->workspace_bytes < need)
    return fail(FA_ERR_INVALID_ARGUMENT, "workspace_bytes %lld is below the required %lld",
                (long long)p->workspace_bytes, (long long)need);
  return FA_OK;
}

}  // namespace

// Scratch of fa_sm75_forward_noalloc: the split-K partials or the dynamic
// schedule's queue counters that fa_sm75_forward otherwise takes from the
// caller's workspace.  Each GPU the library runs on holds its own copy until
// the process ends.  Host code never names this array as an address (its
// name is a host-side stand-in there): it uses the per-device pointer from
// hipGetSymbolAddress below.
static __device__ __align__(256) unsigned char scratch[FA_SM75_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxScratchDevices];

// The current device's copy of `scratch`, looked up once per device (with
// that device current) and kept.
int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FA_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(FA_ERR_INVALID_ARGUMENT, "device %d is beyond the %d devices the scratch covers",
                dev, kMaxScratchDevices);
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || ptr == nullptr)
        return fail(FA_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                    hipGetErrorString(e));
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return FA_OK;
}

}  // namespace

extern "C" {

void fa_sm75_set_contiguous_strides(fa_fwd_params* p) {
  const int64_t D = p->head_dim, N = p->seq_len, Nk = kv_rows(p);
  p->q_stride_n = D; p->q_stride_h = N * D; p->q_stride_b = p->heads_q * N * D;
  p->o_stride_n = D; p->o_stride_h = N * D; p->o_stride_b = p->heads_q * N * D;
  p->k_stride_n = D; p->k_stride_h = Nk * D; p->k_stride_b = p->heads_kv * Nk * D;
  p->v_stride_n = D; p->v_stride_h = Nk * D; p->v_stride_b = p->heads_kv * Nk * D;
}

int fa_sm75_forward(const fa_fwd_params* p) {
  g_last_error[0] = '\0';
  const int st = validate(p, true);
  if (st != FA_OK) return st;
  if (p->batch == 0 || p->heads_q == 0 || p->seq_len == 0) return FA_OK;
  const fa::FwdArgs a = make_args(p);
  const int policy = g_kernel_policy.load(std::memory_order_relaxed);
  const hipStream_t stream = reinterpret_cast<hipStream_t>(p->stream);
  if (policy == FA_POLICY_AUTO && fa::decode_eligible(a, (int)p->batch)) {
    const int64_t room = p->workspace != nullptr ? p->workspace_bytes : 0;
    const fa::DecodePlan plan =
        fa::plan_decode(a, (int)p->batch, (int)p->head_dim, p->causal != 0, room);
    fa::launch_decode_forward(a, plan, (int)p->head_dim, p->causal != 0, p->workspace, stream);
  } else {
    fa::FwdArgs f = a;
    // A workspace of kTicketBytes enables the dynamic (XCD-balanced) schedule;
    // it is 8-byte aligned (16 is required of every workspace).
    if (p->workspace != nullptr && p->workspace_bytes >= fa::kTicketBytes)
      f.ctr = static_cast<uint64_t*>(p->workspace);
    fa::launch_fused_forward(f, (int)p->batch, (int)p->head_dim, p->causal != 0, policy,
                             stream);
  }
  return check_launch();
}

int64_t fa_sm75_workspace_size(const fa_fwd_params* p) {
  const std::string saved = g_last_error;
  const int st = validate(p, true);
  std::snprintf(g_last_error, sizeof(g_last_error), "%s", saved.c_str());
  if (st != FA_OK || p->batch == 0 || p->heads_q == 0 || p->seq_len == 0) return 0;
  const fa::FwdArgs a = make_args(p);
  const int policy = g_kernel_policy.load(std::memory_order_relaxed);
  if (policy == FA_POLICY_AUTO && fa::decode_eligible(a, (int)p->batch))
    return fa::plan_decode(a, (int)p->batch, (int)p->head_dim, p->causal != 0, INT64_MAX)
        .workspace_bytes;
  // Fused kernel: the counters of the dynamic schedule, when it would run.
  return fa::fused_workspace_bytes(a, (int)p->batch, (int)p->head_dim, p->causal != 0, policy);
}

int fa_sm75_forward_noalloc(const fa_fwd_params* p) {
  g_last_error[0] = '\0';
  const int st = validate(p, true);
  if (st != FA_OK) return st;
  if (p->workspace != nullptr || p->workspace_bytes != 0)
    return fail(FA_ERR_INVALID_ARGUMENT,
                "fa_sm75_forward_noalloc takes no workspace (workspace must be NULL and "
                "workspace_bytes 0): it uses the library's own scratch");
  if (p->batch == 0 || p->heads_q == 0 || p->seq_len == 0) return FA_OK;
  const int64_t need = fa_sm75_workspace_size(p);
  if (need > (int64_t)FA_SM75_NOALLOC_SCRATCH_BYTES)
    return fail(FA_ERR_TOO_LARGE,
                "this call needs %lld bytes of scratch; fa_sm75_forward_noalloc holds %lld",
                (long long)need, (long long)FA_SM75_NOALLOC_SCRATCH_BYTES);
  void* ptr = nullptr;
  const int sst = scratch_of_current_device(&ptr);
  if (sst != FA_OK) return sst;
  fa_fwd_params q = *p;
  q.workspace = ptr;
  q.workspace_bytes = (int64_t)FA_SM75_NOALLOC_SCRATCH_BYTES;
  return fa_sm75_forward(&q);
}

namespace {

int pack_mask_impl(const uint8_t* mask, int64_t batch, int64_t heads, int64_t rows, int64_t cols,
                   int64_t stride_b, int64_t stride_h, int64_t stride_q, int64_t stride_k,
                   uint64_t* out, int32_t* ranges, void* stream) {
  g_last_error[0] = '\0';
  if (batch < 0 || heads < 0 || rows < 0 || cols < 0)
    return fail(FA_ERR_INVALID_ARGUMENT, "mask sizes must be non-negative");
  if (stride_b < 0 || stride_h < 0 || stride_q < 0 || stride_k < 0)
    return fail(FA_ERR_INVALID_ARGUMENT, "mask strides must be non-negative");
  if (cols > INT32_MAX / 2)
    return fail(FA_ERR_TOO_LARGE, "mask cols %lld exceeds the supported maximum",
                (long long)cols);
  if (batch == 0 || heads == 0 || rows == 0 || cols == 0) return FA_OK;
  if (mask == nullptr || out == nullptr)
    return fail(FA_ERR_INVALID_ARGUMENT, "mask and out must not be NULL");
  if ((reinterpret_cast<uintptr_t>(out) & 7u) != 0)
    return fail(FA_ERR_MISALIGNED, "out must be 8-byte aligned");
  if (ranges != nullptr && (reinterpret_cast<uintptr_t>(ranges) & 7u) != 0)
    return fail(FA_ERR_MISALIGNED, "ranges must be 8-byte aligned");
  fa::launch_pack_mask(mask, batch, heads, rows, cols, stride_b, stride_h, stride_q, stride_k,
                       out, ranges, reinterpret_cast<hipStream_t>(stream));
  return check_launch();
}

}  // namespace

int fa_sm75_pack_mask(const uint8_t* mask, int64_t batch, int64_t heads, int64_t rows,
                      int64_t cols, int64_t stride_b, int64_t stride_h, int64_t stride_q,
                      int64_t stride_k, uint64_t* out, void* stream) {
  return pack_mask_impl(mask, batch, heads, rows, cols, stride_b, stride_h, stride_q, stride_k,
                        out, nullptr, stream);
}

int fa_sm75_pack_mask_ranges(const uint8_t* mask, int64_t batch, int64_t heads, int64_t rows,
                             int64_t cols, int64_t stride_b, int64_t stride_h,
                             int64_t stride_q, int64_t stride_k, uint64_t* out,
                             int32_t* ranges, void* stream) {
  if (ranges == nullptr) {
    g_last_error[0] = '\0';
    return fail(FA_ERR_INVALID_ARGUMENT, "ranges must not be NULL");
  }
  return pack_mask_impl(mask, batch, heads, rows, cols, stride_b, stride_h, stride_q, stride_k,
                        out, ranges, stream);
}

int fa_sm75_set_kernel_policy(int policy) {
  if (policy < FA_POLICY_AUTO || policy > FA_POLICY_SPLIT_PAIRS) return FA_ERR_INVALID_ARGUMENT;
  g_kernel_policy.store(policy, std::memory_order_relaxed);
  return FA_OK;
}

int fa_sm75_get_kernel_policy(void) { return g_kernel_policy.load(std::memory_order_relaxed); }

int fa_sm75_naive_forward(const fa_fwd_params* p, float* workspace) {
  g_last_error[0] = '\0';
  const int st = validate(p, false);
  if (st != FA_OK) return st;
  if (p->batch == 0 || p->heads_q == 0 || p->seq_len == 0) return FA_OK;
  if (workspace == nullptr)
    return fail(FA_ERR_INVALID_ARGUMENT, "workspace must not be NULL");
  if (p->lse != nullptr)
    return fail(FA_ERR_INVALID_ARGUMENT, "the naive path does not produce LSE");
  if (p->seq_len > 65535)
    return fail(FA_ERR_TOO_LARGE, "naive path supports seq_len <= 65535");
  const fa::FwdArgs a = make_args(p);
  fa::launch_naive_forward(a, (int)p->batch, (int)p->head_dim, p->causal != 0, p->scale,
                           workspace, reinterpret_cast<hipStream_t>(p->stream));
  return check_launch();
}

void fa_sm75_set_contiguous_bwd_strides(fa_bwd_params* p) {
  const int64_t D = p->head_dim, N = p->seq_len, Nk = bwd_kv_rows(p);
  const int64_t qh = N * D, qb = p->heads_q * N * D, kh = Nk * D, kb = p->heads_kv * Nk * D;
  p->q_stride_n = D; p->q_stride_h = qh; p->q_stride_b = qb;
  p->o_stride_n = D; p->o_stride_h = qh; p->o_stride_b = qb;
  p->do_stride_n = D; p->do_stride_h = qh; p->do_stride_b = qb;
  p->dq_stride_n = D; p->dq_stride_h = qh; p->dq_stride_b = qb;
  p->k_stride_n = D; p->k_stride_h = kh; p->k_stride_b = kb;
  p->v_stride_n = D; p->v_stride_h = kh; p->v_stride_b = kb;
  p->dk_stride_n = D; p->dk_stride_h = kh; p->dk_stride_b = kb;
  p->dv_stride_n = D; p->dv_stride_h = kh; p->dv_stride_b = kb;
}

int fa_sm75_backward(const fa_bwd_params* p) {
  g_last_error[0] = '\0';
  const int st = validate_bwd(p);
  if (st != FA_OK) return st;
  if (bwd_empty(p)) return FA_OK;
  fa::BwdArgs a;
  std::memset(&a, 0, sizeof(a));
  a.q = reinterpret_cast<const _Float16*>(p->q);
  a.k = reinterpret_cast<const _Float16*>(p->k);
  a.v = reinterpret_cast<const _Float16*>(p->v);
  a.o = reinterpret_cast<const _Float16*>(p->o);
  a.dout = reinterpret_cast<const _Float16*>(p->dout);
  a.lse = p->lse;
  a.dq = reinterpret_cast<_Float16*>(p->dq);
  a.dk = reinterpret_cast<_Float16*>(p->dk);
  a.dv = reinterpret_cast<_Float16*>(p->dv);
  a.qsb = p->q_stride_b; a.qsh = p->q_stride_h; a.qsn = p->q_stride_n;
  a.ksb = p->k_stride_b; a.ksh = p->k_stride_h; a.ksn = p->k_stride_n;
  a.vsb = p->v_stride_b; a.vsh = p->v_stride_h; a.vsn = p->v_stride_n;
  a.osb = p->o_stride_b; a.osh = p->o_stride_h; a.osn = p->o_stride_n;
  a.dosb = p->do_stride_b; a.dosh = p->do_stride_h; a.dosn = p->do_stride_n;
  a.dqsb = p->dq_stride_b; a.dqsh = p->dq_stride_h; a.dqsn = p->dq_stride_n;
  a.dksb = p->dk_stride_b; a.dksh = p->dk_stride_h; a.dksn = p->dk_stride_n;
  a.dvsb = p->dv_stride_b; a.dvsh = p->dv_stride_h; a.dvsn = p->dv_stride_n;
  a.stats = static_cast<float*>(p->workspace);
  a.tspans = p->mask_ranges != nullptr
                 ? reinterpret_cast<int32_t*>(static_cast<char*>(p->workspace) +
                                              fa::bwd_stats_bytes(p->batch, p->heads_q,
                                                                  p->seq_len))
                 : nullptr;
  a.mbits = p->mask_bits;
  a.msb = p->mask_stride_b;
  a.msh = p->mask_stride_h;
  a.msq = p->mask_stride_q;
  a.mranges = p->mask_ranges;
  a.mrsb = p->mask_ranges_stride_b;
  a.mrsh = p->mask_ranges_stride_h;
  a.mrsq = p->mask_ranges_stride_q;
  a.n = (int)p->seq_len;
  a.nk = (int)bwd_kv_rows(p);
  a.diag = p->causal == FA_CAUSAL_BOTTOM_RIGHT ? a.nk - a.n : 0;
  a.hq = (int)p->heads_q;
  a.group = (int)(p->heads_q / p->heads_kv);
  a.c2 = p->scale * 1.4426950408889634f;
  a.scale = p->scale;
  fa::launch_backward(a, (int)p->batch, (int)p->head_dim, p->causal != FA_CAUSAL_NONE,
                      p->dtype == FA_DTYPE_BF16, reinterpret_cast<hipStream_t>(p->stream));
  return check_launch();
}

int64_t fa_sm75_backward_workspace_size(const fa_bwd_params* p) {
  if (p == nullptr || p->batch < 0 || p->heads_q < 0 || p->seq_len < 0) return 0;
  return fa::bwd_workspace_bytes(p->batch, p->heads_q, p->seq_len);
}

const char* fa_sm75_last_error(void) { return g_last_error; }

const char* fa_sm75_status_string(int status) {
  switch (status) {
    case FA_OK: return "ok";
    case FA_ERR_INVALID_ARGUMENT: return "invalid argument";
    case FA_ERR_UNSUPPORTED_HEAD_DIM: return "unsupported head_dim";
    case FA_ERR_HEADS_NOT_DIVISIBLE: return "heads_q not divisible by heads_kv";
    case FA_ERR_MISALIGNED: return "misaligned pointer or stride";
    case FA_ERR_TOO_LARGE: return "problem too large";
    case FA_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

int fa_sm75_abi_version(void) { return FA_SM75_ABI_VERSION; }

void launch_flash_attention_forward(const fa_half* Q, const fa_half* K, const fa_half* V,
                                    fa_half* O, int batch, int heads, int seq_len,
                                    int head_dim, float scale, bool causal) {
  legacy_launch("flash_attn", Q, K, V, O, batch, heads, seq_len, head_dim, scale, causal,
                false, nullptr);
}

void launch_flash_attention_forward_scalar(const fa_half* Q, const fa_half* K,
                                           const fa_half* V, fa_half* O, int batch,
                                           int heads, int seq_len, int head_dim,
                                           float scale, bool causal) {
  legacy_launch("flash_attn_scalar", Q, K, V, O, batch, heads, seq_len, head_dim, scale,
                causal, true, nullptr);
}

void launch_flash_attention_forward_wmma_qk(const fa_half* Q, const fa_half* K,
                                            const fa_half* V, fa_half* O, int batch,
                                            int heads, int seq_len, int head_dim,
                                            float scale, bool causal) {
  legacy_launch("flash_attn_wmma_qk", Q, K, V, O, batch, heads, seq_len, head_dim, scale,
                causal, true, nullptr);
}

void launch_naive_attention(const fa_half* Q, const fa_half* K, const fa_half* V,
                            fa_half* O, int batch, int heads, int seq_len, int head_dim,
                            float scale, bool causal, float* workspace) {
  if (workspace == nullptr) {
    std::fprintf(stderr, "[naive_attention] workspace must not be NULL\n");
    return;
  }
  legacy_launch("naive_attention", Q, K, V, O, batch, heads, seq_len, head_dim, scale,
                causal, false, workspace);
}

}  // extern "C"
