// Fused attention forward for gfx950 (MI355X / CDNA4): kernel selection.
//
// The kernel itself (fa_fwd_kernel.h) is instantiated per head dimension,
// workgroup shape and element type in fa_fwd_d*.hip, which compile in
// parallel; this file picks the instance for a call.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>

#include "fa_internal.h"

namespace fa {

namespace {

__global__ void fa_clear_tickets(uint64_t* ctr) {
  for (int i = threadIdx.x; i < kNumXcds; i += blockDim.x) ctr[i * kCtrStride] = 0ull;
}

template <int WAVES, int MASK, bool KSPLIT, bool BF16>
void launch_shape(const FwdArgs& a, int batch, int head_dim, bool causal, Schedule schedule,
                  hipStream_t stream) {
  if (head_dim == 128)
    launch_fused<128, WAVES, MASK, KSPLIT, BF16>(a, batch, causal, schedule, stream);
  else
    launch_fused<64, WAVES, MASK, KSPLIT, BF16>(a, batch, causal, schedule, stream);
}

// The 8-wave (256-row, one workgroup per CU) kernel runs when asked for
// (FA_POLICY_WIDE) and where AUTO picks it (use_wide_workgroups), also for
// calls with mask bits; calls with key-padding bytes take the 4-wave kernel.
template <bool BF16>
void launch_typed(const FwdArgs& a, int batch, int head_dim, bool causal, int policy,
                  hipStream_t stream) {
  const Schedule schedule = schedule_of_policy(policy);
  if (a.mkeys != nullptr) {
    launch_shape<4, 2, false, BF16>(a, batch, head_dim, causal, schedule, stream);
    return;
  }
  const bool wide = policy == 2 || use_wide_workgroups(a, batch, head_dim, causal, policy);
  if (a.mbits != nullptr) {
    if (wide)
      launch_shape<8, 1, false, BF16>(a, batch, head_dim, causal, Schedule::kStatic, stream);
    else
      launch_shape<4, 1, false, BF16>(a, batch, head_dim, causal, schedule, stream);
    return;
  }
  if (wide) {
    launch_shape<8, 0, false, BF16>(a, batch, head_dim, causal, Schedule::kStatic, stream);
    return;
  }
  if (use_key_split(a, batch, head_dim, causal, policy)) {
    FwdArgs k = a;
    k.pair_split = use_pair_split(a, batch, head_dim, causal, policy) ? 1 : 0;
    launch_shape<8, 0, true, BF16>(k, batch, head_dim, causal, Schedule::kStatic, stream);
  } else
    launch_shape<4, 0, false, BF16>(a, batch, head_dim, causal, schedule, stream);
}

}  // namespace

int launch_fused_forward(const FwdArgs& a, int batch, int head_dim, bool causal,
                         int policy, hipStream_t stream) {
  if (a.bf16)
    launch_typed<true>(a, batch, head_dim, causal, policy, stream);
  else
    launch_typed<false>(a, batch, head_dim, causal, policy, stream);
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

namespace {

// Key tiles all query blocks of one (batch, head) step through (64-key
// tiles, 128-row blocks).
int64_t tile_steps_per_head(const FwdArgs& a, bool causal) {
  const int64_t full = ((int64_t)a.nk + 63) / 64;
  if (!causal) return full * a.num_qblocks;
  int64_t steps = 0;
  for (int qb = 0; qb < a.num_qblocks; ++qb) {
    const int64_t kv = std::min<int64_t>(a.nk, std::max<int64_t>(0, (int64_t)qb * 128 + 128 +
                                                                        a.diag));
    steps += (kv + 63) / 64;
  }
  return steps;
}

// AUTO runs the dynamic schedule for long launches only: at least
// kDynamicMinSteps tile steps per resident workgroup (about 2 ms at C5
// scale).  It evens out XCDs that run at different clocks, which pays off
// once their drift over the launch exceeds the per-item cost of claiming
// work (measured on MI355X: +2.5-4.6% for B=2 Hq=64 N=16384 d=128 causal,
// neutral at N=8192, 2-5% slower for launches of short items).
constexpr int64_t kDynamicMinSteps = 1024;

// AUTO takes key-split workgroups (8 waves on one 128-row block, one per CU)
//  * for launches whose blocks all get a CU at once and whose rows are long
//    enough (split_pays): there a 4-wave workgroup runs alone on its CU, one
//    wave per SIMD, where its steps are bound by latency; two waves per SIMD
//    on half the key tiles each finish the block sooner, unless the rows
//    are short next to the merge through LDS.  Measured on MI355X
//    (interleaved A/B against the 4-wave kernel's static instance, 21
//    shapes): non-causal head_dim 64 from 16 key tiles 1.053-1.149x (8
//    tiles 0.972x); non-causal head_dim 128 from 24 tiles 1.051-1.078x, or
//    with at most a quarter of the CUs busy 1.099x (16 tiles on 128 or 256
//    blocks 1.003x / 0.968x, 8 tiles 0.920x); causal head_dim 128
//    1.011-1.242x; causal head_dim 64 with rows of 64 tiles 1.017x (16-32
//    tiles 0.934-0.990x).  Declined launches take the 4-wave kernel (the
//    256-row one runs them at 0.66-0.69x);
//  * at head_dim 128 for causal launches of at most this many 128-row
//    blocks per resident 128-row workgroup, each block row at least
//    kSplitMinBlocks long: the largest block's chain of key tiles sets the
//    launch time, and the split halves it (16 blocks per row 0.955x, 32
//    1.02-1.03x, 48-128 1.09x; with more blocks than slots 5-13% slower).
// Causal head_dim-64 launches whose blocks outnumber the CUs but whose pairs
// of blocks (block i with block nqb-1-i of the same head) do not, with rows
// of at least kSplitMinBlocks blocks, run the paired key split instead: one
// round of 8-wave workgroups, each pair's key tiles dealt evenly to the two
// groups (B=1 H=16 N=4096: 1.055x).  With shorter rows the 4-wave kernel's
// large/small block pairing on one CU does as well (C3, 16 blocks per row:
// 0.98x paired key split).  Two waves of one workgroup on a SIMD stop at the
// same barriers, and at head_dim 64 a step is bound by its VALU work (the
// 32 exponentials and the fp16 packing, row max and sum of 2048 scores per
// wave), which two waves on a SIMD share: a SIMD runs one 64-key step of
// two waves in about as many cycles as two steps of one.
constexpr int64_t kSplitMaxItems = 1;
constexpr int kSplitMinBlocks = 32;

int64_t compute_units() { return resident_fused_workgroups() / 2; }

}  // namespace

bool use_pair_split(const FwdArgs& a, int batch, int head_dim, bool causal, int policy) {
  if (has_mask(a) || !causal || head_dim != 64) return false;
  if (policy == 5) return true;
  if (policy != 0) return false;
  FwdArgs planned = a;
  if (plan_grid(planned, batch, 128) <= compute_units()) return false;  // plain key split
  if (planned.num_qblocks < kSplitMinBlocks) return false;
  return plan_pairs(planned, batch) <= compute_units();
}

bool use_key_split(const FwdArgs& a, int batch, int head_dim, bool causal, int policy) {
  if (has_mask(a)) return false;
  if (policy == 4 || policy == 5) return true;
  if (policy != 0) return false;
  FwdArgs planned = a;
  plan_grid(planned, batch, 128);
  if (planned.items <= compute_units()) {
    const int tiles = (a.nk + 63) / 64;  // key tiles of the longest block row
    const bool split_pays =
        causal ? head_dim == 128 || tiles >= 64
               : head_dim == 64 ? tiles >= 16
                                : tiles >= 24 || planned.items <= compute_units() / 4;
    return split_pays;
  }
  if (use_pair_split(a, batch, head_dim, causal, policy)) return true;
  return causal && head_dim == 128 && planned.num_qblocks >= kSplitMinBlocks &&
         planned.items <= kSplitMaxItems * resident_fused_workgroups();
}

// AUTO takes the 256-row workgroups of 8 waves (one per CU: every K/V tile
// serves 256 query rows, so each wave issues half the direct loads per step
// of the 4-wave kernel, which at ~30 cycles of its wave apiece are a tenth or
// more of a step) for launches without key-padding bytes that neither key
// split takes and the dynamic schedule would not run (interleaved A/B on
// MI355X against the 4-wave kernel's static instances):
//  * non-causal launches of more than one and at most two 128-row blocks
//    per CU, where the 4-wave kernel leaves some CUs with two workgroups and
//    others with one, and the 8-wave grid gives each CU at most one (with
//    at most one block per CU, 0.66-0.69x; C2 1.044x, B=3 H=16
//    N=1024 1.038x at head_dim 64 and 1.041x at 128, B=2 H=24 N=1024 d128
//    1.040x; B=4 H=12 N=1536, past two, 0.836x);
//  * rows of at least kWideMinRows queries and keys: causal (or with mask
//    bits, which may leave the blocks' work as uneven as the causal flag,
//    as transformers' causal bool mask does) at head_dim 64 (1.019-1.037x
//    over three shapes), non-causal at head_dim 128 (1.018-1.035x), and
//    causal head_dim 128 from twice that (C4 1.021x, B=2 Hq=32 Hkv=8
//    N=8192 1.003x).  Non-causal head_dim-64 rows stay on the 4-wave
//    kernel, whose static instance holds 168 VGPRs (0.914-1.003x over eight
//    shapes on 256-row workgroups).
// Shorter rows stay on the 4-wave kernel: its causal large/small pairing
// evens single-round launches out (C3 0.825x on 256-row workgroups), and the
// 256-row blocks' diagonal costs more of a short row (B=4 Hq=32 Hkv=8 N=2048
// d128 causal 0.916x, full 0.956x).
constexpr int kWideMinRows = 4096;

bool use_wide_workgroups(const FwdArgs& a, int batch, int head_dim, bool causal, int policy) {
  if (policy != 0 || a.mkeys != nullptr) return false;
  if (use_key_split(a, batch, head_dim, causal, policy)) return false;
  FwdArgs planned = a;
  plan_grid(planned, batch, 128);
  if (use_dynamic_schedule(planned, batch, causal, Schedule::kAuto)) return false;
  const bool uneven = causal || a.mbits != nullptr;
  if (!uneven && planned.items > compute_units() && planned.items <= 2 * compute_units())
    return true;
  const int rows = std::min(a.n, a.nk);
  if (rows < kWideMinRows) return false;
  return head_dim == 64 ? uneven : !uneven || rows >= 2 * kWideMinRows;
}

bool use_dynamic_schedule(const FwdArgs& planned, int batch, bool causal, Schedule schedule) {
  if (schedule == Schedule::kDynamic) return true;
  if (schedule != Schedule::kAuto) return false;
  const int64_t slots = resident_fused_workgroups();
  return planned.items > slots &&
         (int64_t)batch * planned.hq * tile_steps_per_head(planned, causal) >=
             kDynamicMinSteps * slots;
}

int64_t fused_workspace_bytes(const FwdArgs& a, int batch, int head_dim, bool causal,
                              int policy) {
  if (use_key_split(a, batch, head_dim, causal, policy)) return 0;
  FwdArgs planned = a;
  plan_grid(planned, batch, 128);
  return use_dynamic_schedule(planned, batch, causal, schedule_of_policy(policy)) ? kTicketBytes
                                                                                 : 0;
}

void launch_clear_tickets(uint64_t* ctr, hipStream_t stream) {
  hipLaunchKernelGGL(fa_clear_tickets, dim3(1), dim3(64), 0, stream, ctr);
}

}  // namespace fa
