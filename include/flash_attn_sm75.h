/*
 * flash_attn_sm75.h -- C ABI of the MI355X (gfx950) fused attention forward.
 *
 * Plain pointers and sizes only: no torch, no HIP types in the signatures.
 * Every tensor is IEEE binary16 (`fa_half`, the bit pattern of CUDA's `half`)
 * laid out [batch, heads, seq_len, head_dim] with head_dim contiguous (K and V
 * may hold a different number of rows, seq_len_kv, in fa_sm75_forward, which
 * also takes bfloat16 tensors: fa_fwd_params.dtype).
 *
 * Two groups of entry points:
 *
 *  1. The four launchers the reference's PyTorch binding declares
 *     (reference src/bindings/pytorch_extension.cpp:4-19), with the same
 *     argument order and meaning.  Like the reference launchers they run on
 *     the default stream and return only after the device is idle; an
 *     unsupported head_dim prints a message to stderr and returns with O
 *     untouched (reference src/kernels/flash_attention_forward.cu:812-816).
 *
 *  2. The stream-ordered, status-returning entry `fa_sm75_forward`, which
 *     the Python binding uses.  It adds grouped-query attention (heads_kv
 *     divides heads_q: query head h reads KV head h / (heads_q / heads_kv),
 *     the mapping the reference builds with repeat_interleave at
 *     src/flash_attention_sm75/ops.py:24-26), element strides, an optional
 *     fp32 row log-sum-exp output, and an explicit hipStream_t.  It
 *     validates every argument before touching the device and never blocks
 *     the host.
 */
#ifndef FLASH_ATTN_SM75_H
#define FLASH_ATTN_SM75_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One 16-bit value (bit pattern): binary16, or bfloat16 where
 * fa_fwd_params.dtype says so.  Only ever passed by pointer. */
typedef uint16_t fa_half;

/* Values of fa_fwd_params.dtype: the element type of Q, K, V and O.  No
 * reference counterpart (the reference is binary16 only).  With bfloat16 the
 * probabilities are rounded to bfloat16 before the P V product, as the
 * binary16 path rounds them to binary16. */
enum fa_dtype { FA_DTYPE_FP16 = 0, FA_DTYPE_BF16 = 1 };

/* Status codes returned by fa_sm75_forward / fa_sm75_naive_forward. */
enum fa_status {
  FA_OK = 0,
  FA_ERR_INVALID_ARGUMENT = 1,   /* null pointer, negative size, bad stride */
  FA_ERR_UNSUPPORTED_HEAD_DIM = 2, /* head_dim not in {64, 128} */
  FA_ERR_HEADS_NOT_DIVISIBLE = 3,  /* heads_q % heads_kv != 0 */
  FA_ERR_MISALIGNED = 4,           /* base/row stride not 16-byte aligned */
  FA_ERR_TOO_LARGE = 5,            /* a grid dimension would overflow */
  FA_ERR_HIP = 6                   /* HIP runtime error (see message) */
};

/* Values of fa_fwd_params.causal. */
enum fa_causal {
  FA_CAUSAL_NONE = 0,
  FA_CAUSAL_TOP_LEFT = 1,     /* key j visible to query i iff j <= i (the reference's
                                 causal flag; torch SDPA's is_causal) */
  FA_CAUSAL_BOTTOM_RIGHT = 2  /* iff j <= i + seq_len_kv - seq_len (queries are the
                                 last seq_len positions of the keys' sequence) */
};

/* Arguments of one forward call.  Strides are in elements; the last
 * (head_dim) dimension must be contiguous.  N = seq_len query rows,
 * Nk = seq_len_kv key rows (0 selects Nk = N). */
typedef struct fa_fwd_params {
  const fa_half* q;  /* [B, Hq,  N,  D] */
  const fa_half* k;  /* [B, Hkv, Nk, D] */
  const fa_half* v;  /* [B, Hkv, Nk, D] */
  fa_half* o;        /* [B, Hq,  N,  D] output */
  float* lse;        /* optional [B, Hq, N] fp32 natural-log row LSE, or NULL;
                        -inf for a row that sees no key (its O row is 0) */
  int64_t batch;
  int64_t heads_q;
  int64_t heads_kv;
  int64_t seq_len;
  int64_t head_dim;
  int64_t q_stride_b, q_stride_h, q_stride_n;
  int64_t k_stride_b, k_stride_h, k_stride_n;
  int64_t v_stride_b, v_stride_h, v_stride_n;
  int64_t o_stride_b, o_stride_h, o_stride_n;
  float scale;       /* softmax scale applied to Q.K (reference default 1/sqrt(D)) */
  int causal;        /* an fa_causal value */
  void* stream;      /* hipStream_t; NULL selects the default stream */
  int64_t seq_len_kv; /* key/value rows Nk; 0 means Nk = seq_len */
  void* workspace;    /* optional device scratch, or NULL: the split-K path's
                         partials (few query rows per K/V head, e.g. KV-cache
                         decode), or the fused kernel's ticket counters (its
                         dynamic, XCD-balanced schedule).  Contents on entry
                         do not matter; calls that share one race */
  int64_t workspace_bytes; /* its size; fa_sm75_workspace_size() gives the
                         amount for full parallelism.  With less, the call
                         still runs (fewer workgroups, or the static schedule)
                         and allocates nothing */
  /* Optional explicit mask (torch SDPA's boolean attn_mask), or NULL: bit k
   * of word w of row (b, h, i) set <=> key 64w + k is visible to query i of
   * query head h in batch b; fa_sm75_pack_mask builds it.  Strides are in
   * 64-bit words (0 broadcasts a dimension); a nonzero row stride must be
   * at least ceil(seq_len_kv / 64) words.  Combines (AND) with `causal`.  A row that
   * sees no key gets O = 0 and LSE = -inf. */
  const uint64_t* mask_bits;
  int64_t mask_stride_b, mask_stride_h, mask_stride_q;
  int dtype;          /* an fa_dtype (0, binary16, in a zeroed struct); the
                         naive path and the reference launchers are binary16 */
  /* Optional key-padding mask read in place, or NULL: byte (b, j) at
   * mask_keys + b * mask_keys_stride_b + j * mask_keys_stride_k, nonzero
   * <=> key j is visible to every query row of every head of batch b (torch
   * SDPA's boolean attn_mask of shape [B, 1, 1, Nk], [1, Nk] or [Nk], as
   * transformers builds it for padded batches).  The kernels read one byte
   * per key and form the words of mask_bits themselves, so a call needs no
   * fa_sm75_pack_mask launch.  Strides in bytes, non-negative (0 broadcasts
   * the batch).  Exclusive with mask_bits; combines (AND) with `causal`.
   * No reference counterpart (the reference takes no mask). */
  const uint8_t* mask_keys;
  int64_t mask_keys_stride_b, mask_keys_stride_k;
  /* Optional, with mask_bits: for each mask row, the first visible key and
   * one past the last one (an int32 pair; [seq_len_kv, 0] for a row that
   * sees no key), as fa_sm75_pack_mask_ranges writes them; bit 31 of the
   * first entry set means every key between the two is visible (the row
   * sees exactly that interval: causal, padding and sliding-window rows).
   * Strides in pairs, one per mask dimension (0 broadcasts).  The fused
   * kernel then skips the key tiles outside the span of its rows, and reads
   * no mask word for a tile inside the interval of every row of a wave whose
   * rows all carry the bit: a causal mask given as bits (what transformers
   * builds for a padded prefill, with is_causal false) costs about what the
   * causal flag does, and padding is not computed.  Pairs that claim less
   * than the bits show, or the bit for a row with a hidden key inside its
   * interval, would change the result: they must come from the same mask.
   * No reference counterpart. */
  const int32_t* mask_ranges;
  int64_t mask_ranges_stride_b, mask_ranges_stride_h, mask_ranges_stride_q;
} fa_fwd_params;

/* Fills strides for contiguous [B,H,N,D] Q/O and [B,Hkv,Nk,D] K/V tensors. */
void fa_sm75_set_contiguous_strides(fa_fwd_params* p);

/* Fused MFMA forward.  Replaces the launch in reference
 * src/kernels/flash_attention_forward.cu:795-817 (and the GQA expansion of
 * src/flash_attention_sm75/ops.py:6-27).  Asynchronous on p->stream.
 * Calls with (heads_q / heads_kv) * seq_len <= 32 take the split-K path,
 * which uses p->workspace when it is large enough.
 * Returns FA_OK or an fa_status; fa_sm75_last_error() holds the message. */
int fa_sm75_forward(const fa_fwd_params* p);

/* Workspace bytes fa_sm75_forward can use for this call (0: none); 0 also
 * for invalid parameters, which fa_sm75_forward reports.  No reference
 * counterpart (the reference has no decode path). */
int64_t fa_sm75_workspace_size(const fa_fwd_params* p);

/* Bytes of device scratch fa_sm75_forward_noalloc holds per GPU: the largest
 * workspace fa_sm75_workspace_size() can ask for (split-K partials of at most
 * 510 workgroups x 32 query rows x (128 + 2) floats, 8486400 bytes), rounded
 * up to 8.5 MiB. */
#define FA_SM75_NOALLOC_SCRATCH_BYTES (17u << 19)

/* fa_sm75_forward without a caller workspace and without any allocation: the
 * split-K partials or the dynamic schedule's counters live in one static
 * device array of FA_SM75_NOALLOC_SCRATCH_BYTES per GPU, which the library
 * holds until the process ends.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  p->workspace must
 * be NULL and p->workspace_bytes 0; a call whose fa_sm75_workspace_size()
 * exceeds the scratch returns FA_ERR_TOO_LARGE.  Every call on one GPU shares
 * that GPU's array, so calls that overlap on one GPU (different streams, or
 * threads) race; calls ordered on one stream do not.  Results are bitwise
 * those of fa_sm75_forward with a workspace of fa_sm75_workspace_size(p)
 * bytes.  Returns FA_OK or an fa_status. */
int fa_sm75_forward_noalloc(const fa_fwd_params* p);

/* Packs a boolean mask (one byte per element, nonzero = visible) of shape
 * [batch, heads, rows, cols] with element strides (any, 0 included) into the
 * bit layout of fa_fwd_params.mask_bits: out is [batch, heads, rows, words]
 * contiguous, words = ceil(cols / 64), bits past cols clear.  Asynchronous
 * on `stream`.  No reference counterpart (the reference takes no mask). */
int fa_sm75_pack_mask(const uint8_t* mask, int64_t batch, int64_t heads, int64_t rows,
                      int64_t cols, int64_t stride_b, int64_t stride_h, int64_t stride_q,
                      int64_t stride_k, uint64_t* out, void* stream);

/* fa_sm75_pack_mask that also writes, for each row, the first visible key
 * and one past the last one into ranges ([batch, heads, rows, 2] int32
 * contiguous; [cols, 0] for a row with no visible key), bit 31 of the first
 * set when every key between them is visible, for
 * fa_fwd_params.mask_ranges.  No reference counterpart. */
int fa_sm75_pack_mask_ranges(const uint8_t* mask, int64_t batch, int64_t heads, int64_t rows,
                             int64_t cols, int64_t stride_b, int64_t stride_h,
                             int64_t stride_q, int64_t stride_k, uint64_t* out,
                             int32_t* ranges, void* stream);

/* Three-pass reference-style path (QK^T -> row softmax -> PV) through an fp32
 * score workspace of batch*heads_q*seq_len*seq_len floats.  Replaces reference
 * src/kernels/naive_attention.cu:115-164.  Any head_dim that is a multiple of 8
 * (1..256) is accepted; seq_len_kv must be 0 or seq_len.  Asynchronous on
 * p->stream. */
int fa_sm75_naive_forward(const fa_fwd_params* p, float* workspace);

/* Message of the last failing call on this host thread ("" if none). */
const char* fa_sm75_last_error(void);

/* Human-readable name of a status code. */
const char* fa_sm75_status_string(int status);

/* ABI version of this header (bumped on incompatible changes). */
int fa_sm75_abi_version(void);

/* Fused-kernel selection, process-wide (no reference counterpart: a tuning
 * and testing control).  AUTO picks by problem size: the split-K path for
 * few query rows per K/V head; key-split workgroups for launches whose
 * query blocks all get a CU at once (where the rows are long enough:
 * non-causal from 16 key tiles at head_dim 64 and 24 at 128 or with at most
 * a quarter of the CUs busy, causal at head_dim 128, causal head_dim 64 from
 * 64) and for causal head_dim-128 launches small enough that their largest query block sets their time; paired
 * key-split workgroups for causal head_dim-64 launches whose pairs of query
 * blocks all get a CU at once (rows of at least 32 blocks); for calls
 * without key-padding bytes, 256-row workgroups of 8 waves for non-causal
 * launches of more than one and at most two 128-row blocks per CU and for
 * rows of at least
 * 4096 queries and keys (causal or with mask bits at head_dim 64;
 * non-causal at 128, causal from 8192) that the dynamic schedule would not
 * run; else 128-row workgroups, with the dynamic
 * XCD-balanced schedule for long launches when p->workspace holds its
 * counters.  NARROW forces 128-row workgroups of 4 waves (two per CU) on
 * the static schedule (one workgroup per query block); WIDE forces 256-row
 * workgroups of 8 waves (one per CU; K/V tiles triple-buffered at
 * head_dim 64, double-buffered at 128); DYNAMIC
 * forces 128-row workgroups on the dynamic schedule whenever the workspace
 * holds its counters; SPLIT forces 128-row workgroups of 8 waves, two
 * groups of 4 each taking half of the block's key tiles (one per CU);
 * SPLIT_PAIRS forces, for causal head_dim-64 calls (else as SPLIT),
 * workgroups of 8 waves on query blocks i and nqb-1-i of one head, their key
 * tiles dealt evenly to the two groups.  All compute the same function (the
 * two schedules bitwise so). */
enum fa_kernel_policy {
  FA_POLICY_AUTO = 0,
  FA_POLICY_NARROW = 1,
  FA_POLICY_WIDE = 2,
  FA_POLICY_DYNAMIC = 3,
  FA_POLICY_SPLIT = 4,
  FA_POLICY_SPLIT_PAIRS = 5
};
int fa_sm75_set_kernel_policy(int policy); /* FA_OK or FA_ERR_INVALID_ARGUMENT */
int fa_sm75_get_kernel_policy(void);

/* ---- Backward ------------------------------------------------------------
 * Gradients dQ, dK, dV of O = softmax(scale * Q K^T + causal mask) V from
 * dO = dL/dO, the forward's O and its fp32 row LSE (fa_fwd_params.lse).  No
 * reference counterpart: the reference's autograd Function raises
 * NotImplementedError in backward (src/flash_attention_sm75/ops.py:47-52);
 * this is the pass the reference names as future work (reference
 * DESIGN.md:155-163).
 * Shapes and strides as in fa_fwd_params (head_dim contiguous; strides
 * multiples of 8 elements); dQ, dO and O are [B, Hq, N, D], dK and dV
 * [B, Hkv, Nk, D] (for grouped heads each KV head's gradient sums over its
 * query heads).  P and dS are rounded to the element type before the
 * products that take them; sums are fp32.  Deterministic: the same inputs
 * give bitwise the same gradients. */
typedef struct fa_bwd_params {
  const fa_half* q;     /* [B, Hq,  N,  D] */
  const fa_half* k;     /* [B, Hkv, Nk, D] */
  const fa_half* v;     /* [B, Hkv, Nk, D] */
  const fa_half* o;     /* [B, Hq,  N,  D] forward output */
  const fa_half* dout;  /* [B, Hq,  N,  D] dL/dO */
  const float* lse;     /* [B, Hq, N] contiguous fp32 natural-log row LSE of
                           the forward (-inf: the row sees no key) */
  fa_half* dq;          /* [B, Hq,  N,  D] output */
  fa_half* dk;          /* [B, Hkv, Nk, D] output */
  fa_half* dv;          /* [B, Hkv, Nk, D] output */
  int64_t batch;
  int64_t heads_q;
  int64_t heads_kv;
  int64_t seq_len;      /* N */
  int64_t seq_len_kv;   /* Nk; 0 means Nk = seq_len */
  int64_t head_dim;     /* 64 or 128 */
  int64_t q_stride_b, q_stride_h, q_stride_n;
  int64_t k_stride_b, k_stride_h, k_stride_n;
  int64_t v_stride_b, v_stride_h, v_stride_n;
  int64_t o_stride_b, o_stride_h, o_stride_n;
  int64_t do_stride_b, do_stride_h, do_stride_n;
  int64_t dq_stride_b, dq_stride_h, dq_stride_n;
  int64_t dk_stride_b, dk_stride_h, dk_stride_n;
  int64_t dv_stride_b, dv_stride_h, dv_stride_n;
  float scale;          /* the forward's softmax scale */
  int causal;           /* an fa_causal value (the forward's) */
  int dtype;            /* an fa_dtype */
  void* stream;         /* hipStream_t; NULL selects the default stream */
  void* workspace;      /* device scratch of at least
                           fa_sm75_backward_workspace_size() bytes, 16-byte
                           aligned (required); calls that share one race */
  int64_t workspace_bytes;
  /* Optional explicit mask, or NULL: the forward's (fa_fwd_params.mask_bits,
   * same bit layout and word strides, 0 broadcasts a dimension); combines
   * (AND) with `causal`.  The LSE must come from a forward with this mask. */
  const uint64_t* mask_bits;
  int64_t mask_stride_b, mask_stride_h, mask_stride_q;
  /* Optional, with mask_bits: each mask row's span of visible keys, as in
   * fa_fwd_params.mask_ranges.  The dQ kernel then skips the key tiles no
   * row of its block sees, the dK/dV kernel the query tiles with no row that
   * sees a key of its block. */
  const int32_t* mask_ranges;
  int64_t mask_ranges_stride_b, mask_ranges_stride_h, mask_ranges_stride_q;
} fa_bwd_params;

/* Fills contiguous strides for every tensor of *p from its sizes. */
void fa_sm75_set_contiguous_bwd_strides(fa_bwd_params* p);

/* Backward: two kernels on p->stream (dQ, which also writes per-row
 * statistics into the workspace, then dK/dV).  Asynchronous; validates every argument
 * before touching the device.  Returns FA_OK or an fa_status. */
int fa_sm75_backward(const fa_bwd_params* p);

/* Workspace bytes fa_sm75_backward needs: 520 per (batch, query head, 64
 * query rows) -- that tile's row statistics, then its span of visible keys
 * when mask_ranges is given -- from batch, heads_q and seq_len alone (0 if
 * one is negative or p is NULL). */
int64_t fa_sm75_backward_workspace_size(const fa_bwd_params* p);

#define FA_SM75_ABI_VERSION 7

/* ---- Reference launcher signatures ------------------------------------ */

/* reference src/bindings/pytorch_extension.cpp:8-11,
 * src/kernels/flash_attention_forward.cu:795-817 */
void launch_flash_attention_forward(const fa_half* Q, const fa_half* K,
                                    const fa_half* V, fa_half* O, int batch,
                                    int heads, int seq_len, int head_dim,
                                    float scale, bool causal);

/* reference src/bindings/pytorch_extension.cpp:12-15,
 * src/kernels/flash_attention_forward.cu:820-833 (head_dim 64 only) */
void launch_flash_attention_forward_scalar(const fa_half* Q, const fa_half* K,
                                           const fa_half* V, fa_half* O,
                                           int batch, int heads, int seq_len,
                                           int head_dim, float scale,
                                           bool causal);

/* reference src/bindings/pytorch_extension.cpp:16-19,
 * src/kernels/flash_attention_forward.cu:836-849 (head_dim 64 only) */
void launch_flash_attention_forward_wmma_qk(const fa_half* Q, const fa_half* K,
                                            const fa_half* V, fa_half* O,
                                            int batch, int heads, int seq_len,
                                            int head_dim, float scale,
                                            bool causal);

/* reference src/bindings/pytorch_extension.cpp:4-7,
 * src/kernels/naive_attention.cu:115-164; workspace holds
 * batch*heads*seq_len*seq_len floats. */
void launch_naive_attention(const fa_half* Q, const fa_half* K,
                            const fa_half* V, fa_half* O, int batch, int heads,
                            int seq_len, int head_dim, float scale, bool causal,
                            float* workspace);

#ifdef __cplusplus
}
#endif

#endif /* FLASH_ATTN_SM75_H */
