// Backward instances: head_dim 64, binary16 and bfloat16 (stats, dK/dV and dQ kernels).
#include "fa_bwd_kernel.h"

namespace fa {
template void launch_bwd<64, false, false>(const BwdArgs&, int, bool, hipStream_t);
template void launch_bwd<64, true, false>(const BwdArgs&, int, bool, hipStream_t);
}  // namespace fa
