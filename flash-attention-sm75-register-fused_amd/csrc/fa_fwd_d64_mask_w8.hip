// Fused forward instances (binary16): head_dim 64, 256-row workgroups (8 waves), mask bits.
#include "fa_fwd_kernel.h"

namespace fa {
template void launch_fused<64, 8, 1, false, false>(const FwdArgs&, int, bool, Schedule,
                                                   hipStream_t);
}  // namespace fa
