// Fused forward instances (binary16): head_dim 64, 128-row workgroups (4 waves) with a key-padding mask read as bytes.
#include "fa_fwd_kernel.h"

namespace fa {
template void launch_fused<64, 4, 2, false, false>(const FwdArgs&, int, bool, Schedule,
                                                  hipStream_t);
}  // namespace fa
