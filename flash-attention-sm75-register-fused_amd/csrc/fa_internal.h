// Internal interface between the C ABI (fa_capi.hip) and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

// MI355X deals the workgroups of a launch to its 8 XCDs round-robin by
// linear workgroup id; each XCD has its own L2.
constexpr int kNumXcds = 8;

// Kernel arguments of the fused forward (passed by value).
struct FwdArgs {
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  _Float16* o;
  float* lse;  // [B*Hq, N] or nullptr
  int64_t qsb, qsh, qsn;
  int64_t ksb, ksh, ksn;
  int64_t vsb, vsh, vsn;
  int64_t osb, osh, osn;
  int n;            // query rows
  int nk;           // key/value rows
  int diag;         // causal: key j visible to query i iff j <= i + diag
  int hq;           // query heads
  int group;        // heads_q / heads_kv
  int num_qblocks;  // filled by the launcher
  int units;        // batch * heads_kv (one unit = one K/V pair of tensors)
  int xcds;         // 8: units split evenly over the XCDs, else 1 (launcher)
  float c;          // |scale| * log2(e), clamped away from 0
  int negate_q;     // scale < 0: Q fragments are negated (exact in fp16)
  const uint64_t* mbits;   // explicit mask bits or nullptr (see fa_fwd_params)
  int64_t msb, msh, msq;   // its strides in 64-bit words
  const uint8_t* mkeys;    // key-padding mask bytes or nullptr (fa_fwd_params.mask_keys);
  int64_t mksb, mksk;      //   exclusive with mbits; its batch and key strides in bytes
  const int32_t* mranges;  // per mask row (first, one past last) visible key, or nullptr
  int64_t mrsb, mrsh, mrsq;  // its strides in pairs (fa_fwd_params.mask_ranges)
  uint64_t* ctr;    // queue counters of the dynamic schedule, or nullptr (static)
  int items;        // work items (query blocks): filled by the launcher
  int bf16;         // elements are bfloat16 (else binary16)
  int pair_half;    // > 0: single-round causal order pairing (launcher; block_work)
  int pair_split;   // 1: key-split workgroups take pairs of query blocks (launcher)
};

// Whether a call carries an explicit mask (bits or key-padding bytes): the
// kernels' MASK instances serve both.
inline bool has_mask(const FwdArgs& a) { return a.mbits != nullptr || a.mkeys != nullptr; }

// Dynamic schedule of the fused kernel: one 64-bit (head, tail) counter per
// XCD queue, kCtrStride counters (256 bytes) apart, in a caller workspace of
// kTicketBytes.
constexpr int kCtrStride = 32;
constexpr int64_t kTicketBytes = (int64_t)kNumXcds * kCtrStride * 8;
// Workgroups of the 4-wave fused kernel resident on the current device at once
// (two per CU); the dynamic schedule launches this many.
int resident_fused_workgroups();
// Zeroes the ticket counters (a small kernel, so the call stays capturable).
void launch_clear_tickets(uint64_t* ctr, hipStream_t stream);

// Launches the fused MFMA kernel; all arguments already validated.
// policy (fa_kernel_policy): 0 = automatic, 1 = 128-row workgroups of 4
// waves (two per CU) on the static schedule, 2 = 256-row workgroups of 8
// waves (one per CU; K/V triple-buffered at head_dim 64, double at 128),
// 3 = 128-row workgroups on the
// dynamic schedule (when a.ctr is set), 4 = 128-row workgroups of 8 waves
// splitting the keys (one per CU).
int launch_fused_forward(const FwdArgs& a, int batch, int head_dim, bool causal,
                         int policy, hipStream_t stream);
// Schedules of the 4-wave kernel: the long-launch rule, or forced.
enum class Schedule { kAuto, kStatic, kDynamic };
inline Schedule schedule_of_policy(int policy) {
  return policy == 3 ? Schedule::kDynamic : policy == 0 ? Schedule::kAuto : Schedule::kStatic;
}

// Fills num_qblocks, units, xcds and items of the fused kernel's work plan
// for query blocks of block_m rows; returns the number of work items (the
// grid size of the static schedule).
inline int64_t plan_grid(FwdArgs& a, int batch, int block_m) {
  a.num_qblocks = (int)(((int64_t)a.n + block_m - 1) / block_m);
  a.units = batch * (a.hq / a.group);
  a.xcds = a.units % kNumXcds == 0 ? kNumXcds : 1;
  a.items = batch * a.hq * a.num_qblocks;
  a.pair_half = 0;
  a.pair_split = 0;
  return a.items;
}
// Plan of the paired key split: work item = a pair of query blocks of one
// (batch, query head), ceil(num_qblocks / 2) per head (128-row blocks);
// returns the number of items.
inline int64_t plan_pairs(FwdArgs& a, int batch) {
  plan_grid(a, batch, 128);
  a.num_qblocks = (a.num_qblocks + 1) / 2;
  a.items = batch * a.hq * a.num_qblocks;
  a.pair_split = 1;
  return a.items;
}
// Whether the 4-wave kernel runs the dynamic schedule for a planned call
// (plan_grid done, 128-row blocks), given counters to run it with (on its
// instances that carry the item loop, DYN).
bool use_dynamic_schedule(const FwdArgs& planned, int batch, bool causal, Schedule schedule);
// Workspace bytes the fused path uses for a call (the dynamic schedule's
// counters, or 0), under a kernel policy.
int64_t fused_workspace_bytes(const FwdArgs& a, int batch, int head_dim, bool causal,
                              int policy);
// One instance family of the fused kernel (fa_fwd_kernel.h), explicitly
// instantiated in fa_fwd_d*.hip.  MASK: 0 none, 1 mask bits (a.mbits), 2
// key-padding bytes (a.mkeys).  KSPLIT: 8 waves on 128 rows, the two groups
// of 4 splitting the key tiles.
template <int D, int WAVES, int MASK, bool KSPLIT, bool BF16>
void launch_fused(const FwdArgs& a, int batch, bool causal, Schedule schedule,
                  hipStream_t stream);
// Whether a call runs on key-split workgroups: policy 4 or 5, or AUTO for
// launches whose blocks (or, causal at head_dim 64, pairs of blocks) all
// get a CU at once and whose rows are long enough to pay for the merge, and
// for causal head_dim-128 launches whose time is set by their largest query
// block.
bool use_key_split(const FwdArgs& a, int batch, int head_dim, bool causal, int policy);
// Whether AUTO runs a call without key-padding bytes on 256-row workgroups
// of 8 waves (non-causal launches of more than one and at most two 128-row
// blocks per CU, and long rows; see fa_fwd.hip).
bool use_wide_workgroups(const FwdArgs& a, int batch, int head_dim, bool causal, int policy);
// Whether key-split workgroups take pairs of query blocks (causal head_dim
// 64: policy 5, or AUTO when the blocks outnumber the CUs but the pairs do
// not, in rows of at least 32 blocks).
bool use_pair_split(const FwdArgs& a, int batch, int head_dim, bool causal, int policy);
int fused_block_m();  // rows of the smallest workgroup (grid-size checks)

// Split-K path (fa_decode.hip): taken when heads_q / heads_kv * seq_len <=
// kDecodeMaxRows (KV-cache decode: all query rows of one K/V head fit one
// 32-column MFMA tile), and for small launches, whose 128-row prefill grid
// would hold at most kSmallLaunchItems workgroups: their query rows then go
// in blocks of 32, each block's keys split over several workgroups.
constexpr int kDecodeMaxRows = 32;
constexpr int kSmallLaunchItems = 64;
struct DecArgs {
  FwdArgs f;
  int rows;         // query columns per unit: min(32, group * n)
  int total_rows;   // query rows per (batch, KV head): group * n
  int row_blocks;   // units per (batch, KV head): ceil(total_rows / 32)
  int splits;       // key ranges per unit
  int chunk_tiles;  // 32-key tiles per split
  int tiles;        // 32-key tiles any row can see
  float* part_o;    // [units, splits, rows, D] unnormalised O (splits > 1)
  float* part_ml;   // [units, splits, rows, 2]: max (log2 units), sum
};
struct DecodePlan {
  int rows, total_rows, row_blocks, units, tiles, splits, chunk_tiles;
  int64_t workspace_bytes;  // 0 when splits == 1
};
bool decode_eligible(const FwdArgs& a, int batch);
// Splits for a workspace of `workspace_bytes` (one split if it is too small).
DecodePlan plan_decode(const FwdArgs& a, int batch, int head_dim, bool causal,
                       int64_t workspace_bytes);
int launch_decode_forward(const FwdArgs& a, const DecodePlan& plan, int head_dim, bool causal,
                          void* workspace, hipStream_t stream);

// ---- Backward (fa_bwd.hip, fa_bwd_kernel.h) --------------------------------
// Kernel arguments of the two backward kernels (passed by value).  The
// grid-plan fields carry the names block_work reads.
struct BwdArgs {
  const _Float16* q;
  const _Float16* k;
  const _Float16* v;
  const _Float16* o;
  const _Float16* dout;
  const float* lse;  // [B*Hq, N] natural-log row LSE of the forward
  _Float16* dq;
  _Float16* dk;
  _Float16* dv;
  int64_t qsb, qsh, qsn;
  int64_t ksb, ksh, ksn;
  int64_t vsb, vsh, vsn;
  int64_t osb, osh, osn;
  int64_t dosb, dosh, dosn;
  int64_t dqsb, dqsh, dqsn;
  int64_t dksb, dksh, dksn;
  int64_t dvsb, dvsh, dvsn;
  // Workspace: per (b, query head) and 64-row query tile, 64 floats
  // lse * log2(e) (+inf for rows past N and rows that see no key), then 64
  // floats -rowsum(dO * O) (0 past N); the dQ kernel writes it.
  float* stats;
  // With mask ranges: after the stats, per (b, query head) and 64-row query
  // tile, the union [first, one past last) of its rows' spans of visible
  // keys (an int32 pair), which the dQ kernel writes and the dK/dV kernel
  // scans in place of every row's pair; nullptr without mask ranges.
  int32_t* tspans;
  const uint64_t* mbits;   // explicit mask bits (fa_fwd_params layout) or nullptr
  int64_t msb, msh, msq;   // its strides in 64-bit words
  const int32_t* mranges;  // per mask row (first, one past last) visible key, or nullptr
  int64_t mrsb, mrsh, mrsq;  // its strides in pairs
  int mwords;              // ceil(nk / 64): words of one mask row
  int n;       // query rows
  int nk;      // key/value rows
  int diag;    // causal: key j visible to query i iff j <= i + diag
  int hq;      // query heads
  int group;   // heads_q / heads_kv
  int qtiles;  // ceil(n / 64)
  float c2;    // scale * log2(e), signed
  float scale;
  // grid plan (launcher)
  int num_qblocks;  // dQ kernel: ceil(n / 128)
  int units;        // batch * heads_kv
  int xcds;         // 8 when units divide evenly over the XCDs, else 1
  int items;        // dQ kernel work items
  int pair_half;    // always 0 (no CU pairing)
};
constexpr int kBwdStatsTile = 64;    // query rows per stats record
constexpr int kBwdBlockKeys = 128;   // keys per dK/dV workgroup
constexpr int kBwdBlockRows = 128;   // query rows per dQ workgroup
// Workspace bytes of a backward call: the statistics records, then the
// query tiles' key spans (BwdArgs::stats, tspans).
inline int64_t bwd_stats_bytes(int64_t batch, int64_t heads_q, int64_t seq_len) {
  return batch * heads_q * ((seq_len + kBwdStatsTile - 1) / kBwdStatsTile) *
         (2 * kBwdStatsTile) * (int64_t)sizeof(float);
}
inline int64_t bwd_workspace_bytes(int64_t batch, int64_t heads_q, int64_t seq_len) {
  return bwd_stats_bytes(batch, heads_q, seq_len) +
         batch * heads_q * ((seq_len + kBwdStatsTile - 1) / kBwdStatsTile) * 2 *
             (int64_t)sizeof(int32_t);
}
// Launches the dQ and dK/dV kernels; all arguments validated.
int launch_backward(const BwdArgs& a, int batch, int head_dim, bool causal, bool bf16,
                    hipStream_t stream);
template <int D, bool BF16, bool MASK>
void launch_bwd(const BwdArgs& a, int batch, bool causal, hipStream_t stream);

// Boolean mask -> bit rows (fa_mask.hip); ranges (or nullptr): each row's
// first visible key and one past the last ([cols, 0] for none), int32 pairs.
int launch_pack_mask(const uint8_t* mask, int64_t batch, int64_t heads, int64_t rows,
                     int64_t cols, int64_t sb, int64_t sh, int64_t sq, int64_t sk,
                     uint64_t* out, int32_t* ranges, hipStream_t stream);

// Three-kernel path through an fp32 [B*Hq, N, N] score workspace.
int launch_naive_forward(const FwdArgs& a, int batch, int head_dim, bool causal,
                         float scale, float* workspace, hipStream_t stream);

}  // namespace fa
