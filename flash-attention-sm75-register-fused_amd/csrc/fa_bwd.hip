// Fused attention backward for gfx950: grid plan and instance selection.
// The kernels are in fa_bwd_kernel.h, instantiated per head dimension and
// mask mode in fa_bwd_d{64,128}{,_mask}.hip.
#include <hip/hip_runtime.h>

#include "fa_internal.h"

namespace fa {

int launch_backward(const BwdArgs& args, int batch, int head_dim, bool causal, bool bf16,
                    hipStream_t stream) {
  BwdArgs a = args;
  a.qtiles = (a.n + kBwdStatsTile - 1) / kBwdStatsTile;
  a.units = batch * (a.hq / a.group);
  a.xcds = a.units % kNumXcds == 0 ? kNumXcds : 1;
  a.num_qblocks = (a.n + kBwdBlockRows - 1) / kBwdBlockRows;
  a.items = batch * a.hq * a.num_qblocks;
  a.pair_half = 0;
  a.mwords = (a.nk + 63) / 64;
  const bool mask = a.mbits != nullptr;
  if (head_dim == 128) {
    if (mask) {
      if (bf16) launch_bwd<128, true, true>(a, batch, causal, stream);
      else launch_bwd<128, false, true>(a, batch, causal, stream);
    } else {
      if (bf16) launch_bwd<128, true, false>(a, batch, causal, stream);
      else launch_bwd<128, false, false>(a, batch, causal, stream);
    }
  } else {
    if (mask) {
      if (bf16) launch_bwd<64, true, true>(a, batch, causal, stream);
      else launch_bwd<64, false, true>(a, batch, causal, stream);
    } else {
      if (bf16) launch_bwd<64, true, false>(a, batch, causal, stream);
      else launch_bwd<64, false, false>(a, batch, causal, stream);
    }
  }
  return 0;
}

}  // namespace fa
