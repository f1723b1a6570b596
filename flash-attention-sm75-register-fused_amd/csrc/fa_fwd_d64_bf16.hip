// Fused forward instances (bfloat16): head_dim 64, 128-row workgroups (4 waves), no explicit mask.
#include "fa_fwd_kernel.h"

namespace fa {
template void launch_fused<64, 4, 0, false, true>(const FwdArgs&, int, bool, Schedule,
                                                      hipStream_t);
}  // namespace fa
