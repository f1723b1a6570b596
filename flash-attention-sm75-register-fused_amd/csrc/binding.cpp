// PyTorch binding: module `flash_attn_sm75_cuda`.
//
// Same op names, signatures and error texts as the reference binding
// (reference src/bindings/pytorch_extension.cpp:21-129):
//   naive_attention_forward, flash_attention_forward,
//   flash_attention_forward_scalar, flash_attention_forward_wmma_qk,
// each (Tensor Q, Tensor K, Tensor V, bool causal, float scale) -> Tensor.
// Additions: flash_attention_forward accepts grouped K/V heads (Hkv divides
// Hq) so no repeat_interleave copy is needed, flash_attention_forward_lse
// also returns the fp32 row log-sum-exp, and flash_attention_forward_ex takes
// strided views in place, Nq != Nk, either causal alignment, a boolean
// attn_mask and bfloat16 tensors (the reference ops stay FP16 only).
//
// All checks run before any device work; the kernels are enqueued on the
// current HIP stream of Q's device and the host is not blocked.
#include <torch/extension.h>

#include <ATen/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <string>
#include <tuple>

#include "flash_attn_sm75.h"

namespace {

void check_tensor(const torch::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), std::string(name) + " must be a CUDA tensor");
  TORCH_CHECK(t.dtype() == torch::kFloat16, std::string(name) + " must be FP16");
  TORCH_CHECK(t.is_contiguous(), std::string(name) + " must be contiguous");
  TORCH_CHECK(t.dim() == 4, std::string(name) + " must be [B, H, N, D]");
}

void check_same_device(const torch::Tensor& Q, const torch::Tensor& K,
                       const torch::Tensor& V) {
  TORCH_CHECK(Q.device() == K.device() && Q.device() == V.device(),
              "Q, K, V must be on the same device");
}

// Data pointers and element type of 16-bit tensors (binary16 or bfloat16,
// checked by the callers).
void set_tensors(fa_fwd_params& p, const torch::Tensor& Q, const torch::Tensor& K,
                 const torch::Tensor& V, torch::Tensor& O) {
  p.q = static_cast<const fa_half*>(Q.data_ptr());
  p.k = static_cast<const fa_half*>(K.data_ptr());
  p.v = static_cast<const fa_half*>(V.data_ptr());
  p.o = static_cast<fa_half*>(O.data_ptr());
  p.dtype = Q.scalar_type() == torch::kBFloat16 ? FA_DTYPE_BF16 : FA_DTYPE_FP16;
}

fa_fwd_params make_params(const torch::Tensor& Q, const torch::Tensor& K,
                          const torch::Tensor& V, torch::Tensor& O, float* lse,
                          bool causal, float scale) {
  fa_fwd_params p{};
  set_tensors(p, Q, K, V, O);
  p.lse = lse;
  p.batch = Q.size(0);
  p.heads_q = Q.size(1);
  p.heads_kv = K.size(1);
  p.seq_len = Q.size(2);
  p.head_dim = Q.size(3);
  p.q_stride_b = Q.stride(0); p.q_stride_h = Q.stride(1); p.q_stride_n = Q.stride(2);
  p.k_stride_b = K.stride(0); p.k_stride_h = K.stride(1); p.k_stride_n = K.stride(2);
  p.v_stride_b = V.stride(0); p.v_stride_h = V.stride(1); p.v_stride_n = V.stride(2);
  p.o_stride_b = O.stride(0); p.o_stride_h = O.stride(1); p.o_stride_n = O.stride(2);
  p.scale = scale;
  p.causal = causal ? 1 : 0;
  p.stream = nullptr;
  return p;
}

// Shape checks of the fused op (reference pytorch_extension.cpp:56-68), with
// the heads check widened from equality to divisibility.
void check_fused_shapes(const torch::Tensor& Q, const torch::Tensor& K,
                        const torch::Tensor& V) {
  check_tensor(Q, "Q");
  check_tensor(K, "K");
  check_tensor(V, "V");
  check_same_device(Q, K, V);
  TORCH_CHECK(Q.size(0) == K.size(0), "batch mismatch");
  TORCH_CHECK(K.size(1) > 0 && Q.size(1) % K.size(1) == 0,
              "heads mismatch after GQA expansion: Q heads (", Q.size(1),
              ") not divisible by K/V heads (", K.size(1), ")");
  TORCH_CHECK(Q.size(2) == K.size(2), "seq_len mismatch");
  TORCH_CHECK(Q.size(3) == K.size(3), "head_dim mismatch");
  TORCH_CHECK(K.sizes() == V.sizes(), "K and V must have identical shapes");
  const auto head_dim = Q.size(3);
  TORCH_CHECK(head_dim == 64 || head_dim == 128,
              "flash_attention_forward supports head_dim=64 or 128, got ", head_dim);
}

// Runs fa_sm75_forward with a workspace from torch's caching allocator when
// the call can use one (the split-K path's partials, or the ticket counters
// of the fused kernel's dynamic schedule).  The workspace is released when
// this returns; the allocator only hands it out again to work ordered after
// the launch on the same stream.
void forward_with_workspace(fa_fwd_params& p, const torch::Tensor& Q, const char* tag) {
  p.stream = c10::hip::getCurrentHIPStream(Q.device().index()).stream();
  const int64_t ws = fa_sm75_workspace_size(&p);
  torch::Tensor work;
  if (ws > 0) {
    work = torch::empty({ws}, Q.options().dtype(torch::kUInt8));
    p.workspace = work.data_ptr();
    p.workspace_bytes = ws;
  }
  const int st = fa_sm75_forward(&p);
  TORCH_CHECK(st == FA_OK, tag, ": ", fa_sm75_last_error());
}

void run_fused(const torch::Tensor& Q, const torch::Tensor& K, const torch::Tensor& V,
               torch::Tensor& O, float* lse, bool causal, float scale) {
  const at::OptionalDeviceGuard guard(at::device_of(Q));
  fa_fwd_params p = make_params(Q, K, V, O, lse, causal, scale);
  forward_with_workspace(p, Q, "flash_attention_forward");
}

torch::Tensor flash_attention_forward(torch::Tensor Q, torch::Tensor K, torch::Tensor V,
                                      bool causal, float scale) {
  check_fused_shapes(Q, K, V);
  auto O = torch::empty_like(Q);
  run_fused(Q, K, V, O, nullptr, causal, scale);
  return O;
}

std::tuple<torch::Tensor, torch::Tensor> flash_attention_forward_lse(
    torch::Tensor Q, torch::Tensor K, torch::Tensor V, bool causal, float scale) {
  check_fused_shapes(Q, K, V);
  auto O = torch::empty_like(Q);
  auto L = torch::empty({Q.size(0), Q.size(1), Q.size(2)},
                        Q.options().dtype(torch::kFloat32));
  run_fused(Q, K, V, O, L.data_ptr<float>(), causal, scale);
  return {O, L};
}

// ---- flash_attention_forward_ex: strided views, Nq != Nk, causal alignment --

// Whether the kernels can read t in place: head_dim contiguous, the other
// strides multiples of 8 elements, a 16-byte aligned base and (for K/V) a
// (batch, head) slice that fits the 32-bit buffer window.  Strides of size-1
// dimensions never matter and are ignored.
bool kernel_layout_ok(const torch::Tensor& t, bool kv) {
  if (t.stride(3) != 1) return false;
  if ((reinterpret_cast<uintptr_t>(t.data_ptr()) & 15u) != 0) return false;
  for (int i = 0; i < 3; ++i)
    if (t.size(i) > 1 && (t.stride(i) < 0 || t.stride(i) % 8 != 0)) return false;
  if (t.size(2) > 1 && t.stride(2) < t.size(3)) return false;
  // The library reads these through 32-bit buffer windows that reach one
  // 64-row tile past the last row (fa_capi.hip rejects (rows + 64) * row
  // stride * 2 > INT32_MAX); such views are copied to a contiguous layout.
  if (kv && (t.size(2) + 64) * (t.size(2) > 1 ? t.stride(2) : t.size(3)) * 2 >
                (int64_t)INT32_MAX)
    return false;
  return true;
}

torch::Tensor kernel_view(const torch::Tensor& t, bool kv) {
  return kernel_layout_ok(t, kv) ? t : t.contiguous();
}

// Stride of dimension i, or `fallback` for a size-1 dimension.
int64_t eff_stride(const torch::Tensor& t, int i, int64_t fallback) {
  return t.size(i) == 1 ? fallback : t.stride(i);
}

// Packs a boolean mask broadcastable to [B, Hq, Nq, Nk] into bit rows; the
// mask's own size-1 (or stride-0) batch, head and query dimensions stay size
// 1 in the packed tensor and get stride 0 in the params.  The forward
// and the backward also get each row's span of visible keys (mask_ranges),
// one int64 per row after the words, so the kernels skip the tiles no row
// of a block sees.
template <class Params>  // fa_fwd_params or fa_bwd_params (same mask fields)
torch::Tensor pack_mask(const torch::Tensor& mask, const torch::Tensor& Q, int64_t nk,
                        Params& p) {
  TORCH_CHECK(mask.dtype() == torch::kBool, "attn_mask must be a bool tensor");
  TORCH_CHECK(mask.device() == Q.device(), "attn_mask must be on Q's device");
  TORCH_CHECK(mask.dim() <= 4, "attn_mask must have at most 4 dimensions");
  const auto m = mask.expand({Q.size(0), Q.size(1), Q.size(2), nk});
  int64_t own[3];
  for (int d = 0; d < 3; ++d) own[d] = (m.size(d) == 1 || m.stride(d) == 0) ? 1 : m.size(d);
  const int64_t words = (nk + 63) / 64;
  const int64_t nrows = own[0] * own[1] * own[2];
  auto bits = torch::empty({nrows * (words + 1)}, Q.options().dtype(torch::kInt64));
  uint64_t* const out = reinterpret_cast<uint64_t*>(bits.data_ptr<int64_t>());
  int32_t* const ranges = reinterpret_cast<int32_t*>(out + nrows * words);
  const auto* src = reinterpret_cast<const uint8_t*>(m.data_ptr<bool>());
  const int64_t sb = own[0] > 1 ? m.stride(0) : 0, sh = own[1] > 1 ? m.stride(1) : 0,
                sq = own[2] > 1 ? m.stride(2) : 0;
  void* const stream = c10::hip::getCurrentHIPStream(Q.device().index()).stream();
  const int st = fa_sm75_pack_mask_ranges(src, own[0], own[1], own[2], nk, sb, sh, sq,
                                          m.stride(3), out, ranges, stream);
  TORCH_CHECK(st == FA_OK, "attn_mask packing: ", fa_sm75_last_error());
  p.mask_bits = out;
  p.mask_stride_b = own[0] > 1 ? own[1] * own[2] * words : 0;
  p.mask_stride_h = own[1] > 1 ? own[2] * words : 0;
  p.mask_stride_q = own[2] > 1 ? words : 0;
  p.mask_ranges = ranges;
  p.mask_ranges_stride_b = own[0] > 1 ? own[1] * own[2] : 0;
  p.mask_ranges_stride_h = own[1] > 1 ? own[2] : 0;
  p.mask_ranges_stride_q = own[2] > 1 ? 1 : 0;
  return bits;
}

// The forward's mask: a key-padding mask (the same for every head and query
// row, transformers' [B, 1, 1, Nk] for padded batches) goes to the kernels as
// its bytes, read in place (no packing launch); any other shape is packed
// into bit rows.  Returns the tensor the call's mask pointer refers to.
torch::Tensor forward_mask(const torch::Tensor& mask, const torch::Tensor& Q, int64_t nk,
                           fa_fwd_params& p) {
  TORCH_CHECK(mask.dtype() == torch::kBool, "attn_mask must be a bool tensor");
  TORCH_CHECK(mask.device() == Q.device(), "attn_mask must be on Q's device");
  TORCH_CHECK(mask.dim() <= 4, "attn_mask must have at most 4 dimensions");
  const auto m = mask.expand({Q.size(0), Q.size(1), Q.size(2), nk});
  const bool per_key = (m.size(1) == 1 || m.stride(1) == 0) && (m.size(2) == 1 || m.stride(2) == 0);
  if (!per_key) return pack_mask(mask, Q, nk, p);
  p.mask_keys = reinterpret_cast<const uint8_t*>(m.data_ptr<bool>());
  p.mask_keys_stride_b = m.size(0) > 1 ? m.stride(0) : 0;
  p.mask_keys_stride_k = m.stride(3);
  return mask;
}

std::tuple<torch::Tensor, c10::optional<torch::Tensor>> flash_attention_forward_ex(
    torch::Tensor Q, torch::Tensor K, torch::Tensor V, int64_t causal, double scale,
    bool return_lse, c10::optional<torch::Tensor> attn_mask) {
  for (auto* pr : {&Q, &K, &V}) {
    const torch::Tensor& t = *pr;
    TORCH_CHECK(t.is_cuda(), "inputs must be CUDA tensors");
    TORCH_CHECK(t.dtype() == torch::kFloat16 || t.dtype() == torch::kBFloat16,
                "inputs must be FP16 or BF16");
    TORCH_CHECK(t.dtype() == Q.dtype(), "Q, K and V must have the same dtype");
    TORCH_CHECK(t.dim() == 4, "inputs must be [B, H, N, D]");
  }
  check_same_device(Q, K, V);
  TORCH_CHECK(Q.size(0) == K.size(0), "batch mismatch");
  TORCH_CHECK(K.size(1) > 0 && Q.size(1) % K.size(1) == 0, "heads mismatch: Q heads (",
              Q.size(1), ") not divisible by K/V heads (", K.size(1), ")");
  TORCH_CHECK(Q.size(3) == K.size(3), "head_dim mismatch");
  TORCH_CHECK(K.sizes() == V.sizes(), "K and V must have identical shapes");
  TORCH_CHECK(causal >= 0 && causal <= 2,
              "causal must be 0 (none), 1 (top-left) or 2 (bottom-right), got ", causal);
  const auto D = Q.size(3);
  TORCH_CHECK(D == 64 || D == 128, "flash_attention_forward supports head_dim=64 or 128, got ", D);
  Q = kernel_view(Q, false);
  K = kernel_view(K, true);
  V = kernel_view(V, true);
  auto O = torch::empty_like(Q);  // keeps Q's dense layout (e.g. [B, N, H, D] storage)
  if (!kernel_layout_ok(O, false)) O = torch::empty(Q.sizes(), Q.options());
  c10::optional<torch::Tensor> L;
  if (return_lse)
    L = torch::empty({Q.size(0), Q.size(1), Q.size(2)}, Q.options().dtype(torch::kFloat32));
  if (Q.numel() == 0) return {O, L};
  TORCH_CHECK(K.size(2) > 0, "K/V must hold at least one row");
  const at::OptionalDeviceGuard guard(at::device_of(Q));
  fa_fwd_params p{};
  set_tensors(p, Q, K, V, O);
  p.lse = return_lse ? L->data_ptr<float>() : nullptr;
  p.batch = Q.size(0);
  p.heads_q = Q.size(1);
  p.heads_kv = K.size(1);
  p.seq_len = Q.size(2);
  p.seq_len_kv = K.size(2);
  p.head_dim = D;
  const int64_t qn = eff_stride(Q, 2, D), kn = eff_stride(K, 2, D), vn = eff_stride(V, 2, D),
                on = eff_stride(O, 2, D);
  p.q_stride_n = qn; p.q_stride_h = eff_stride(Q, 1, 0); p.q_stride_b = eff_stride(Q, 0, 0);
  p.k_stride_n = kn; p.k_stride_h = eff_stride(K, 1, 0); p.k_stride_b = eff_stride(K, 0, 0);
  p.v_stride_n = vn; p.v_stride_h = eff_stride(V, 1, 0); p.v_stride_b = eff_stride(V, 0, 0);
  p.o_stride_n = on; p.o_stride_h = eff_stride(O, 1, 0); p.o_stride_b = eff_stride(O, 0, 0);
  p.scale = (float)scale;
  p.causal = (int)causal;
  torch::Tensor bits;  // lives until the launch is enqueued (stream-ordered reuse)
  if (attn_mask.has_value()) bits = forward_mask(*attn_mask, Q, K.size(2), p);
  forward_with_workspace(p, Q, "flash_attention_forward_ex");
  return {O, L};
}

// ---- flash_attention_backward: dQ, dK, dV (no reference counterpart) ---------

// Gradients of flash_attention_forward_ex's O (causal code, scale and
// boolean attn_mask as given to it) from dO, the inputs, O and the fp32 row
// LSE it returned.
// Inputs are read in place when their layout allows; the gradients are
// dense tensors shaped like Q, K and V.
std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> flash_attention_backward(
    torch::Tensor dO, torch::Tensor Q, torch::Tensor K, torch::Tensor V, torch::Tensor O,
    torch::Tensor LSE, int64_t causal, double scale, c10::optional<torch::Tensor> attn_mask) {
  for (auto* pr : {&Q, &K, &V, &O, &dO}) {
    const torch::Tensor& t = *pr;
    TORCH_CHECK(t.is_cuda(), "inputs must be CUDA tensors");
    TORCH_CHECK(t.dtype() == torch::kFloat16 || t.dtype() == torch::kBFloat16,
                "inputs must be FP16 or BF16");
    TORCH_CHECK(t.dtype() == Q.dtype(), "Q, K, V, O and dO must have the same dtype");
    TORCH_CHECK(t.dim() == 4, "inputs must be [B, H, N, D]");
    TORCH_CHECK(t.device() == Q.device(), "inputs must be on the same device");
  }
  TORCH_CHECK(Q.size(0) == K.size(0), "batch mismatch");
  TORCH_CHECK(K.size(1) > 0 && Q.size(1) % K.size(1) == 0, "heads mismatch: Q heads (",
              Q.size(1), ") not divisible by K/V heads (", K.size(1), ")");
  TORCH_CHECK(Q.size(3) == K.size(3), "head_dim mismatch");
  TORCH_CHECK(K.sizes() == V.sizes(), "K and V must have identical shapes");
  TORCH_CHECK(O.sizes() == Q.sizes() && dO.sizes() == Q.sizes(), "O and dO must be shaped like Q");
  TORCH_CHECK(LSE.device() == Q.device() && LSE.dtype() == torch::kFloat32,
              "LSE must be a float32 tensor on Q's device");
  TORCH_CHECK(LSE.dim() == 3 && LSE.size(0) == Q.size(0) && LSE.size(1) == Q.size(1) &&
                  LSE.size(2) == Q.size(2),
              "LSE must be [B, Hq, N]");
  TORCH_CHECK(causal >= 0 && causal <= 2,
              "causal must be 0 (none), 1 (top-left) or 2 (bottom-right), got ", causal);
  const auto D = Q.size(3);
  TORCH_CHECK(D == 64 || D == 128, "flash_attention_backward supports head_dim=64 or 128, got ",
              D);
  Q = kernel_view(Q, true);  // Q and dO tiles go through buffer windows too
  dO = kernel_view(dO, true);
  K = kernel_view(K, true);
  V = kernel_view(V, true);
  O = kernel_view(O, false);
  LSE = LSE.contiguous();
  auto dQ = torch::empty(Q.sizes(), Q.options());
  auto dK = torch::empty(K.sizes(), K.options());
  auto dV = torch::empty(V.sizes(), V.options());
  if (Q.numel() == 0 && K.numel() == 0) return {dQ, dK, dV};
  if (Q.size(1) == 0) return {dQ, dK.zero_(), dV.zero_()};  // no query head reads K/V
  TORCH_CHECK(K.size(2) > 0 || Q.size(2) == 0, "K/V must hold at least one row");
  const at::OptionalDeviceGuard guard(at::device_of(Q));
  fa_bwd_params p{};
  p.q = static_cast<const fa_half*>(Q.data_ptr());
  p.k = static_cast<const fa_half*>(K.data_ptr());
  p.v = static_cast<const fa_half*>(V.data_ptr());
  p.o = static_cast<const fa_half*>(O.data_ptr());
  p.dout = static_cast<const fa_half*>(dO.data_ptr());
  p.lse = LSE.data_ptr<float>();
  p.dq = static_cast<fa_half*>(dQ.data_ptr());
  p.dk = static_cast<fa_half*>(dK.data_ptr());
  p.dv = static_cast<fa_half*>(dV.data_ptr());
  p.batch = Q.size(0);
  p.heads_q = Q.size(1);
  p.heads_kv = K.size(1);
  p.seq_len = Q.size(2);
  p.seq_len_kv = K.size(2);
  p.head_dim = D;
  auto strides = [&](const torch::Tensor& t, int64_t& sb, int64_t& sh, int64_t& sn) {
    sn = eff_stride(t, 2, D);
    sh = eff_stride(t, 1, 0);
    sb = eff_stride(t, 0, 0);
  };
  strides(Q, p.q_stride_b, p.q_stride_h, p.q_stride_n);
  strides(K, p.k_stride_b, p.k_stride_h, p.k_stride_n);
  strides(V, p.v_stride_b, p.v_stride_h, p.v_stride_n);
  strides(O, p.o_stride_b, p.o_stride_h, p.o_stride_n);
  strides(dO, p.do_stride_b, p.do_stride_h, p.do_stride_n);
  strides(dQ, p.dq_stride_b, p.dq_stride_h, p.dq_stride_n);
  strides(dK, p.dk_stride_b, p.dk_stride_h, p.dk_stride_n);
  strides(dV, p.dv_stride_b, p.dv_stride_h, p.dv_stride_n);
  p.scale = (float)scale;
  p.causal = (int)causal;
  p.dtype = Q.scalar_type() == torch::kBFloat16 ? FA_DTYPE_BF16 : FA_DTYPE_FP16;
  p.stream = c10::hip::getCurrentHIPStream(Q.device().index()).stream();
  torch::Tensor bits;  // lives until the launches are enqueued (stream-ordered reuse)
  if (attn_mask.has_value()) bits = pack_mask(*attn_mask, Q, K.size(2), p);
  const int64_t ws = fa_sm75_backward_workspace_size(&p);
  torch::Tensor work;  // released after the launch: stream-ordered reuse
  if (ws > 0) {
    work = torch::empty({ws}, Q.options().dtype(torch::kUInt8));
    p.workspace = work.data_ptr();
    p.workspace_bytes = ws;
  }
  const int st = fa_sm75_backward(&p);
  TORCH_CHECK(st == FA_OK, "flash_attention_backward: ", fa_sm75_last_error());
  return {dQ, dK, dV};
}

torch::Tensor d64_compat(const char* tag, torch::Tensor Q, torch::Tensor K,
                         torch::Tensor V, bool causal, float scale) {
  check_tensor(Q, "Q");
  check_tensor(K, "K");
  check_tensor(V, "V");
  check_same_device(Q, K, V);
  TORCH_CHECK(Q.sizes() == K.sizes() && Q.sizes() == V.sizes(),
              "Q, K, V must have identical shapes");
  TORCH_CHECK(Q.size(3) == 64, tag, " kernel supports head_dim=64 only");
  auto O = torch::empty_like(Q);
  run_fused(Q, K, V, O, nullptr, causal, scale);
  return O;
}

// reference pytorch_extension.cpp:84-102
torch::Tensor flash_attention_forward_scalar(torch::Tensor Q, torch::Tensor K,
                                             torch::Tensor V, bool causal, float scale) {
  return d64_compat("scalar", Q, K, V, causal, scale);
}

// reference pytorch_extension.cpp:104-122
torch::Tensor flash_attention_forward_wmma_qk(torch::Tensor Q, torch::Tensor K,
                                              torch::Tensor V, bool causal, float scale) {
  return d64_compat("wmma_qk", Q, K, V, causal, scale);
}

// reference pytorch_extension.cpp:28-50
torch::Tensor naive_attention_forward(torch::Tensor Q, torch::Tensor K, torch::Tensor V,
                                      bool causal, float scale) {
  check_tensor(Q, "Q");
  check_tensor(K, "K");
  check_tensor(V, "V");
  check_same_device(Q, K, V);
  TORCH_CHECK(Q.sizes() == K.sizes() && Q.sizes() == V.sizes(),
              "naive_attention: Q, K, V must have identical shapes");
  auto O = torch::empty_like(Q);
  auto ws = torch::empty({Q.size(0) * Q.size(1), Q.size(2), Q.size(2)},
                         Q.options().dtype(torch::kFloat32));
  const at::OptionalDeviceGuard guard(at::device_of(Q));
  fa_fwd_params p = make_params(Q, K, V, O, nullptr, causal, scale);
  p.stream = c10::hip::getCurrentHIPStream(Q.device().index()).stream();
  const int st = fa_sm75_naive_forward(&p, ws.data_ptr<float>());
  TORCH_CHECK(st == FA_OK, "naive_attention_forward: ", fa_sm75_last_error());
  return O;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "MI355X (gfx950) fused attention forward, reference-compatible op set";
  m.def("naive_attention_forward", &naive_attention_forward);
  m.def("flash_attention_forward", &flash_attention_forward);
  m.def("flash_attention_forward_scalar", &flash_attention_forward_scalar);
  m.def("flash_attention_forward_wmma_qk", &flash_attention_forward_wmma_qk);
  m.def("flash_attention_forward_lse", &flash_attention_forward_lse);
  m.def("flash_attention_forward_ex", &flash_attention_forward_ex,
        "O (and optionally the fp32 row LSE) for Q [B,Hq,Nq,D], K/V [B,Hkv,Nk,D]; "
        "strided views read in place; causal 0 none, 1 top-left, 2 bottom-right",
        pybind11::arg("Q"), pybind11::arg("K"), pybind11::arg("V"), pybind11::arg("causal"),
        pybind11::arg("scale"), pybind11::arg("return_lse") = false,
        pybind11::arg("attn_mask") = pybind11::none());
  m.def("flash_attention_backward", &flash_attention_backward,
        "(dQ, dK, dV) of flash_attention_forward_ex's output from dO, Q, K, V, O and the "
        "fp32 row LSE; causal 0 none, 1 top-left, 2 bottom-right",
        pybind11::arg("dO"), pybind11::arg("Q"), pybind11::arg("K"), pybind11::arg("V"),
        pybind11::arg("O"), pybind11::arg("LSE"), pybind11::arg("causal"),
        pybind11::arg("scale"), pybind11::arg("attn_mask") = pybind11::none());
  m.def("abi_version", []() { return fa_sm75_abi_version(); });
  m.def("set_kernel_policy", [](int policy) {
    TORCH_CHECK(fa_sm75_set_kernel_policy(policy) == FA_OK,
                "kernel policy must be 0 (auto), 1 (narrow), 2 (wide), 3 (dynamic), 4 (split) or "
                "5 (split pairs), got ",
                policy);
  });
  m.def("get_kernel_policy", []() { return fa_sm75_get_kernel_policy(); });
}
