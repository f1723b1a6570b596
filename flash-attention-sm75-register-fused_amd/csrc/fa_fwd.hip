// Fused attention forward for gfx950 (MI355X / CDNA4): kernel selection.
//
// The kernel itself (fa_fwd_kernel.h) is instantiated per head dimension and
// workgroup shape in fa_fwd_d{64,128}{,_w8,_mask}.hip, which compile in
// parallel; this file picks the instance for a call.
#include <hip/hip_runtime.h>

#include <atomic>

#include "fa_internal.h"

namespace fa {

namespace {

__global__ void fa_clear_tickets(uint64_t* ctr) {
  for (int i = threadIdx.x; i < kNumXcds; i += blockDim.x) ctr[i * kCtrStride] = 0ull;
}

template <int WAVES, bool MASK>
void launch_waves(const FwdArgs& a, int batch, int head_dim, bool causal, Schedule schedule,
                  hipStream_t stream) {
  if (head_dim == 128)
    launch_fused<128, WAVES, MASK>(a, batch, causal, schedule, stream);
  else
    launch_fused<64, WAVES, MASK>(a, batch, causal, schedule, stream);
}

}  // namespace

// The 8-wave (256-row, one workgroup per CU) kernel only runs when asked
// for (FA_POLICY_WIDE): measured on C4 it is ~4% slower than the 4-wave
// kernel -- with one workgroup per CU both waves of a SIMD stop at the same
// barrier, where two independent 4-wave workgroups cover each other's.
// Masked calls always take the 4-wave kernel.
int launch_fused_forward(const FwdArgs& a, int batch, int head_dim, bool causal,
                         int policy, hipStream_t stream) {
  const Schedule schedule =
      policy == 3 ? Schedule::kDynamic : policy == 0 ? Schedule::kAuto : Schedule::kStatic;
  if (a.mbits != nullptr)
    launch_waves<4, true>(a, batch, head_dim, causal, schedule, stream);
  else if (policy == 2)
    launch_waves<8, false>(a, batch, head_dim, causal, Schedule::kStatic, stream);
  else
    launch_waves<4, false>(a, batch, head_dim, causal, schedule, stream);
  return 0;
}

int fused_block_m() { return 128; }

int resident_fused_workgroups() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    n = 2 * cus;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

void launch_clear_tickets(uint64_t* ctr, hipStream_t stream) {
  hipLaunchKernelGGL(fa_clear_tickets, dim3(1), dim3(64), 0, stream, ctr);
}

}  // namespace fa
