// Fused forward instances (binary16): head_dim 128, 128-row workgroups (4 waves) with a boolean mask.
#include "fa_fwd_kernel.h"

namespace fa {
template void launch_fused<128, 4, 1, false, false>(const FwdArgs&, int, bool, Schedule,
                                                      hipStream_t);
}  // namespace fa
