// Fused forward instances (bfloat16): head_dim 128, 128-row workgroups of 8 waves splitting the keys.
#include "fa_fwd_kernel.h"

namespace fa {
template void launch_fused<128, 8, 0, true, true>(const FwdArgs&, int, bool, Schedule,
                                                      hipStream_t);
}  // namespace fa
