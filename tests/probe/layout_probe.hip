// Device probes of the hardware semantics the attention kernels rely on.
// Test infrastructure: built by __graft_entry__.build() into
// tests/probe/liblayout_probe.so and driven by tests/test_gpu_layout_probe.py
// through ctypes; nothing in the product loads it.
//
//   fa_probe_mfma          v_mfma_f32_32x32x16_{f16,bf16} (Elem<>::mfma): the
//                          A, B and C register layouts the kernels assume
//                          (fa_fwd_kernel.h header): lane l holds
//                          A[m = l%32][k = 8(l/32) + j], B[k = 8(l/32) + j][n = l%32]
//                          and C[m = 8(i/4) + 4(l/32) + i%4][n = l%32].
//   fa_probe_tr16          ds_read_b64_tr_b16 (ds_read_tr16): within each
//                          16-lane group, lane i's element j is the 16-bit
//                          word at (address of group lane 4j + i/4) + i%4.
//   fa_probe_halves        halves_max / halves_sum (v_permlane32_swap):
//                          lanes l and l^32 exchange their values.
// One wave per launch; every access is inside the buffers the host passes.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa_kernel_common.h"

namespace {

using fa::float16v;
using fa::half4;
using fa::half8;

template <bool BF16>
__global__ void __launch_bounds__(64) probe_mfma(const uint16_t* A, const uint16_t* B, float* C) {
  const int l = (int)threadIdx.x;
  half8 a, b;
  for (int j = 0; j < 8; ++j) {
    a[j] = __builtin_bit_cast(_Float16, A[(l % 32) * 16 + 8 * (l / 32) + j]);
    b[j] = __builtin_bit_cast(_Float16, B[(8 * (l / 32) + j) * 32 + (l % 32)]);
  }
  const float16v c = fa::Elem<BF16>::mfma(a, b, (float16v)0.0f);
  for (int i = 0; i < 16; ++i) {
    const int m = 8 * (i / 4) + 4 * (l / 32) + i % 4;
    C[m * 32 + (l % 32)] = c[i];
  }
}

__global__ void __launch_bounds__(64) probe_tr16(const int* addr, const uint16_t* mem, int n,
                                                 uint16_t* out) {
  __shared__ __attribute__((aligned(16))) _Float16 lds[4096];
  for (int i = (int)threadIdx.x; i < n; i += 64) lds[i] = __builtin_bit_cast(_Float16, mem[i]);
  __syncthreads();
  const half4 r = fa::ds_read_tr16(lds + addr[threadIdx.x]);
  // One 8-byte store of the whole result, as the kernels consume it whole.
  // (Extracting the four elements one by one compiled, with this ROCm's
  // hipcc, into code that stored element 0 four times.)
  *(fa::short4v*)(out + threadIdx.x * 4) = __builtin_bit_cast(fa::short4v, r);
}

__global__ void __launch_bounds__(64) probe_halves(const float* x, float* mx, float* sm) {
  const int l = (int)threadIdx.x;
  mx[l] = fa::halves_max(x[l]);
  sm[l] = fa::halves_sum(x[l]);
}

int finish() { return hipGetLastError() == hipSuccess && hipDeviceSynchronize() == hipSuccess ? 0 : 1; }

}  // namespace

extern "C" {

// A: [32, 16] and B: [16, 32] row-major 16-bit (binary16, or bfloat16 when
// bf16 != 0) device buffers; C: [32, 32] fp32.  Returns 0 on success.
int fa_probe_mfma(const uint16_t* A, const uint16_t* B, float* C, int bf16) {
  if (bf16)
    hipLaunchKernelGGL(probe_mfma<true>, dim3(1), dim3(64), 0, 0, A, B, C);
  else
    hipLaunchKernelGGL(probe_mfma<false>, dim3(1), dim3(64), 0, 0, A, B, C);
  return finish();
}

// addr: 64 element offsets (multiples of 4, each + 4 <= n); mem: n <= 4096
// 16-bit words; out: [64, 4].
int fa_probe_tr16(const int* addr, const uint16_t* mem, int n, uint16_t* out) {
  if (n < 4 || n > 4096) return 2;
  hipLaunchKernelGGL(probe_tr16, dim3(1), dim3(64), 0, 0, addr, mem, n, out);
  return finish();
}

// x, mx, sm: 64 floats each.
int fa_probe_halves(const float* x, float* mx, float* sm) {
  hipLaunchKernelGGL(probe_halves, dim3(1), dim3(64), 0, 0, x, mx, sm);
  return finish();
}

}  // extern "C"
