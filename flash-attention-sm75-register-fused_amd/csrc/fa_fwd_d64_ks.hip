// Fused forward instances (binary16): head_dim 64, 128-row workgroups of 8 waves splitting the keys.
#include "fa_fwd_kernel.h"

namespace fa {
template void launch_fused<64, 8, 0, true, false>(const FwdArgs&, int, bool, Schedule,
                                                      hipStream_t);
}  // namespace fa
