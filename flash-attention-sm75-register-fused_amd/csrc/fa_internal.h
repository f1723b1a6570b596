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
};

// Launches the fused MFMA kernel; all arguments already validated.
// policy: 0 = automatic and 1 = 128-row workgroups of 4 waves (two per CU),
// 2 = 256-row workgroups of 8 waves (one per CU, K/V triple-buffered).
int launch_fused_forward(const FwdArgs& a, int batch, int head_dim, bool causal,
                         int policy, hipStream_t stream);
int fused_block_m();  // rows of the smallest workgroup (grid-size checks)

// Split-K path for few query rows per K/V head (fa_decode.hip): taken when
// heads_q / heads_kv * seq_len <= kDecodeMaxRows.
constexpr int kDecodeMaxRows = 32;
struct DecArgs {
  FwdArgs f;
  int rows;         // query columns per unit: group * n
  int splits;       // key ranges per unit
  int chunk_tiles;  // 32-key tiles per split
  int tiles;        // 32-key tiles any row can see
  float* part_o;    // [units, splits, rows, D] unnormalised O (splits > 1)
  float* part_ml;   // [units, splits, rows, 2]: max (log2 units), sum
};
struct DecodePlan {
  int rows, units, tiles, splits, chunk_tiles;
  int64_t workspace_bytes;  // 0 when splits == 1
};
bool decode_eligible(const FwdArgs& a);
// Splits for a workspace of `workspace_bytes` (one split if it is too small).
DecodePlan plan_decode(const FwdArgs& a, int batch, int head_dim, bool causal,
                       int64_t workspace_bytes);
int launch_decode_forward(const FwdArgs& a, const DecodePlan& plan, int head_dim, bool causal,
                          void* workspace, hipStream_t stream);

// Boolean mask -> bit rows (fa_mask.hip).
int launch_pack_mask(const uint8_t* mask, int64_t batch, int64_t heads, int64_t rows,
                     int64_t cols, int64_t sb, int64_t sh, int64_t sq, int64_t sk,
                     uint64_t* out, hipStream_t stream);

// Three-kernel path through an fp32 [B*Hq, N, N] score workspace.
int launch_naive_forward(const FwdArgs& a, int batch, int head_dim, bool causal,
                         float scale, float* workspace, hipStream_t stream);

}  // namespace fa
