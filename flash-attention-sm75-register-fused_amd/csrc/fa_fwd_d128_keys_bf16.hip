// Fused forward instances (bfloat16): head_dim 128, 128-row workgroups (4 waves) with a key-padding mask read as bytes.
#include "fa_fwd_kernel.h"

namespace fa {
template void launch_fused<128, 4, 2, false, true>(const FwdArgs&, int, bool, Schedule,
                                                  hipStream_t);
}  // namespace fa
