// Fused attention forward kernel for gfx950 (MI355X / CDNA4), included by the
// instance files fa_fwd_d*.hip (one head dimension, workgroup shape and
// element type each, compiled in parallel); fa_fwd.hip dispatches between
// them.
//
// O = softmax(scale * Q K^T + mask) V with fp16 inputs, fp32 accumulation and
// an fp16 output, in one kernel (the hot path that reference
// src/kernels/flash_attention_forward.cu:345-791 implements for SM75); the
// BF16 instances take bfloat16 Q/K/V/O (bf16 MFMAs, P rounded to bf16).
//
// Work decomposition
//   A 1-D grid of batch * heads_q * ceil(N / kBlockM) workgroups, kBlockM =
//   128 query rows each, ordered so the workgroups reading one K/V pair share
//   an XCD (block_work in fa_kernel_common.h).
//   One workgroup = 4 waves; wave w owns query rows [q0 + 32w, q0 + 32w + 32).
//   Key/value rows stream through LDS in tiles of kBlockN = 64 keys.  Tiles
//   go straight from HBM to LDS (buffer_load ... lds: lane l's 16 bytes land
//   at M0 + 16 l), through buffer windows that end at the last key, so rows
//   past the sequence arrive as zeros.
//
// MFMA formulation (v_mfma_f32_32x32x16_f16, operand layouts verified on the
// device):
//   A[m][k]: lane l holds m = l%32, k = 8*(l/32) + j  (8 halves)
//   B[k][n]: lane l holds n = l%32, k = 8*(l/32) + j  (8 halves)
//   C[m][n]: lane l holds n = l%32, m = 8*(i/4) + 4*(l/32) + i%4 (16 floats)
//   * S^T = K Q^T: keys are the M side, queries the N side, so every lane owns
//     a single query (l%32) and 16 of its 32 keys per 32-key sub-tile.  The
//     row max over keys is an in-register reduction plus one lane swap
//     between the two wave halves; the row sum stays lane-local until the end.
//   * O^T = V^T P^T: the probabilities stay in the registers the S^T
//     accumulator produced, reinterpreted as the B operand.  The key order
//     inside each 16-key MFMA step is a permutation shared by P and V (the
//     contraction is order-free).  V^T operands come straight out of a
//     row-major LDS tile with ds_read_b64_tr_b16 (transposing LDS read).
//   * The O^T accumulator keeps, per lane, one query and D/2 of its
//     dimensions, so the online-softmax rescale is a per-lane scalar.
//
// Scheduling.  On this hardware a wave's VALU work overlaps its *own* MFMAs
// (issued between them) but hardly overlaps MFMAs of another wave on the
// same SIMD.  So the main loop is software pipelined and hand ordered:
// iteration j issues the MFMAs of S_{j+1} and P_j V_j one "slot" at a time,
// and each slot also carries the LDS reads needed a few slots later and a
// share of the softmax of S_j (exp, fp16 pack, row sum).
//
// Softmax numerics follow reference src/kernels/flash_attention_forward.cu:
// running max starts at -inf and the first rescale factor is 0 (:386,:483),
// masked keys contribute exactly 0 (:470-479), probabilities are rounded to
// fp16 before the PV product (:495), the final row factor is 1/l (:562).
// exp is evaluated as 2^(x * log2 e) with the log2 e folded into the scale.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "fa_internal.h"

#include "fa_kernel_common.h"

namespace fa {
namespace {

// Software-pipelined main loop: step j computes S^T_{j+1} = K_{j+1} Q^T while
// the VALU turns S^T_j into probabilities, then accumulates P_j V_j.  One
// barrier per step.  Two shapes (WAVES):
//   * 4 waves, 128 query rows, two workgroups per CU, K/V tiles double
//     buffered (STAGES = 2): step j loads K_{j+2} and V_{j+1} into the
//     buffers step j-1 freed, and they must land by the end of step j;
//   * 8 waves, 256 query rows, one workgroup per CU: every K/V tile serves
//     256 query rows, and each wave issues half as many direct loads (waves
//     0-3 load K, 4-7 load V).  At head_dim 64 triple buffered (STAGES = 3):
//     step j loads K_{j+3} and V_{j+2}, which have until the end of step j+1
//     to land.  At head_dim 128 double buffered like the 4-wave kernel: the
//     third stage's code (its unrolled rest steps) needs more than the 256
//     VGPRs of two waves per SIMD and spilled 101 of them, whose scratch
//     (about 39 MB for the resident waves) goes out to HBM; double buffered
//     it spills none and runs 1.004-1.018x faster (C4 1.018x, B=2 Hq=32
//     Hkv=8 N=8192 causal 1.018x, B=1 Hq=32 Hkv=8 N=4096 full 1.004x);
//   * KSPLIT: 8 waves, 128 query rows, one workgroup per CU: waves w and w+4
//     own the same 32 rows, and each group of 4 waves runs the 4-wave
//     pipeline over its half of the block's key tiles in its own half of the
//     LDS buffers; at the end group 1 hands its (O, max, sum) to group 0
//     through LDS, which merges and stores.  This halves the longest chain
//     of steps in launches whose time is set by their largest causal block.
// KV_SAME_STRIDE: K and V rows have the same stride, so the direct-load
// offsets are shared (saves registers).  MASK_MODE 1: an explicit mask (one
// 64-bit word per query row and tile, loaded a step ahead) hides keys too;
// MASK_MODE 2: a key-padding mask read as bytes (one per lane and tile, loaded
// a step ahead; a ballot over the wave forms the same word).
// ROWSUM: the row sums of P come from the matrix pipe, as one more 32-row
// output tile of O^T whose A operand is a row of ones (4 more MFMAs and 16
// fewer VALU instructions per tile).  Launched for head_dim-64 causal
// launches that hold every block at once: there a CU's large block runs its
// last tiles alone, one wave per SIMD, and its step latency is the launch's
// tail (measured: C3 +3.4%, B=1 Hq=14 Hkv=2 N=4096 +4.8%; launches that keep
// two waves per SIMD busy throughout lose 1-2%, the extra matrix work costing
// clock).
// DYN: the instance carries the dynamic schedule's item loop (4-wave launches
// that run it).  Static launches take instances without it: the loop's
// claim, prefetch and hand-off state costs registers all through the steps
// (the ROWSUM instance: 106 SGPRs spilled to VGPR lanes and 232 VGPRs with
// it, 15 and 222 without; C3 1.033-1.040x, results bitwise unchanged).
// LDS through which group 1 of a key split hands its share of a block to
// group 0: per row wave, MT * 1024 floats of O (four consecutive floats of a
// lane's accumulator per 16-byte slot), then 64 running maxima and 64 lane
// partial sums.  Allocated by the head_dim-64 key-split instances, whose
// dense tiles are smaller than that (the head_dim-128 ones hand over through
// a padded tile array, which the main loop no longer reads).
template <bool P, int MT>
__device__ __forceinline__ float* pair_exchange() {
  if constexpr (P) {
    __shared__ __attribute__((aligned(16))) float xo[4 * (MT * 1024 + 128)];
    return xo;
  } else {
    return nullptr;
  }
}

template <int D, bool CAUSAL, bool KV_SAME_STRIDE, int WAVES, int MASK_MODE, bool KSPLIT, bool BF16,
          bool ROWSUM, bool DYN>
__global__ void __launch_bounds__(64 * WAVES, 2) fa_fwd_kernel(const FwdArgs a) {
  static_assert(!DYN || (WAVES == 4 && !ROWSUM), "the dynamic schedule runs on 4-wave instances");
  constexpr bool MASK = MASK_MODE != 0;        // an explicit mask: bits or key bytes
  constexpr bool KEY_BYTES = MASK_MODE == 2;   // key-padding bytes (a.mkeys)
  // LDS tile layout: dense (no row padding, 8 direct loads per tile instead
  // of 12; interleaved A/B on head_dim-64 launches 1.013-1.031x, results
  // bitwise unchanged) at head_dim 64, padded at head_dim 128 (whose dense
  // swizzle would take more per-lane bases than its registers hold).
  constexpr bool DENSE = D == 64;
  using L = std::conditional_t<DENSE, LdsDense<D>, Lds<D>>;
  using E = Elem<BF16>;
  constexpr int KK = D / 16;       // 16-wide contraction steps of S^T
  constexpr int MT = D / 32;       // 32-row output tiles of O^T
  constexpr int MTX = MT + (ROWSUM ? 1 : 0);  // P V output tiles, the row-sum tile last
  constexpr int NS = 2 * KK;       // S^T MFMAs per tile
  constexpr int NPV = 4 * MTX;     // P V MFMAs per tile
  constexpr int PFK = 3;           // K operand reads run this many MFMAs ahead
  constexpr int PFV = 2;           // V operand reads run this many MFMAs ahead
  constexpr int ROW_WAVES = KSPLIT ? 4 : WAVES;  // waves owning distinct rows
  constexpr int BLOCK_M = 32 * ROW_WAVES;
  constexpr int STAGES = WAVES == 8 && !KSPLIT && D == 64 ? 3 : 2;  // K/V buffers per tile kind
  constexpr int SEGQ = L::Segs / 4;               // segments of one tile per wave quarter
  constexpr int LPW = 2 * L::Segs / ROW_WAVES;    // direct loads per wave per step
  constexpr bool SPLIT_ROLES = WAVES == 8 && !KSPLIT;  // a wave loads K or V, not both
  // The paired key split (a.pair_split) runs on the head_dim-64 causal
  // key-split instances (the head_dim-128 ones fill the LDS already).
  constexpr bool PAIRS = KSPLIT && D == 64 && CAUSAL;
  static_assert(WAVES == 4 || WAVES == 8, "4 or 8 waves");
  static_assert(!KSPLIT || (WAVES == 8 && !MASK), "key split: 8 waves, no mask");
  static_assert(L::Segs % 4 == 0, "tile segments must split over 4 waves");

  // STAGES K buffers and STAGES V buffers, distinct objects (not one array):
  // the loop is unrolled by STAGES, so every access names its buffer at
  // compile time and the compiler can see that the in-flight direct loads
  // never alias the tiles being read (it would otherwise drain vmcnt before
  // each LDS read).
  // With KSPLIT each array holds one tile per key group (group g at g Tile).
  constexpr int GROUP_TILES = KSPLIT ? 2 : 1;
  __shared__ __attribute__((aligned(1024))) _Float16 k_lds0[GROUP_TILES * L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 k_lds1[GROUP_TILES * L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 k_lds2[STAGES == 3 ? GROUP_TILES * L::Tile : 1];
  __shared__ __attribute__((aligned(1024))) _Float16 v_lds0[GROUP_TILES * L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 v_lds1[GROUP_TILES * L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 v_lds2[STAGES == 3 ? GROUP_TILES * L::Tile : 1];

  // Wave index: scalar (the direct loads' LDS destinations, M0, derive from
  // it) and the only thread coordinate kept across work items.
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int rw = KSPLIT ? wave & 3 : wave;     // row wave: rows q0 + 32 rw ..
  const int kgrp = KSPLIT ? wave >> 2 : 0;     // key group (KSPLIT)
  const int gofs = kgrp * L::Tile;             // its LDS tiles' offset

  // Work items.  Static schedule (a.ctr == nullptr): workgroup wg does item
  // wg.  Dynamic schedule (the 4-wave kernel's DYN instances, a.ctr set,
  // grid = resident workgroups): the items form a.xcds queues, queue x holding the items the
  // static schedule gives XCD x, one (batch, KV head) unit after the other
  // and largest first within each (block_work's unit_major order).  A
  // workgroup takes items from the head of its own XCD's queue; once that is
  // empty it takes from the tail (the smallest items) of the others, so XCDs
  // running at a higher clock take over the end of slower XCDs' work
  // without starting a long item late.  Each queue is one 64-bit counter,
  // head count in the low word, tail count in the high word: an atomic add
  // of 1 (head) or 2^32 (tail) claims head index h or tail index P-1-t of
  // the counts (h, t) it returns, if h + t < P (P items per queue).  Every
  // claim raises h + t by one, so no item is claimed twice.
  // Thread 0 (wave 0, lane 0) claims the items (the head claim for the next
  // item is issued at the start of the item's last step) and passes the item
  // and the set of queues it found empty to every wave through LDS: the
  // buffer of V_{STAGES-1}, which no direct load writes between an item's
  // last step and the next item's step 0 (the prologue fills the others).
  const bool dynamic = DYN && a.ctr != nullptr;
  const int nq = a.xcds;
  const int per_queue = a.items / nq;
  const int own_q = (int)(__builtin_amdgcn_s_getreg(kHwRegXccId) & 15u) % nq;
  int* const ticket_slot = (int*)(STAGES == 3 ? v_lds2 : v_lds1);
  auto lane_id = [] {
    return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  };
  auto claim = [&](int q, bool tail) -> uint64_t {
    return __hip_atomic_fetch_add(a.ctr + q * kCtrStride, tail ? (1ull << 32) : 1ull,
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  // Item of a claim's returned counts (h, t), or -1 if the queue was empty.
  auto claimed_item = [&](int q, bool tail, uint64_t ht) -> int {
    const int h = (int)(uint32_t)ht, t = (int)(ht >> 32);
    if (h + t >= per_queue) return -1;
    return (tail ? per_queue - 1 - t : h) * nq + q;
  };
  // Thread 0: the next item (-1: none left), from the prefetched head claim
  // of the own queue if there is one, else from the queues not yet empty.
  auto take_item = [&](bool prefetched, uint64_t ht, unsigned& empty) -> int {
    if (prefetched) {
      const int it = claimed_item(own_q, false, ht);
      if (it >= 0) return it;
      empty |= 1u << own_q;
    }
    for (int i = 0; i < nq; ++i) {
      const int qi = own_q + i < nq ? own_q + i : own_q + i - nq;
      if ((empty >> qi) & 1u) continue;
      const int it = claimed_item(qi, i != 0, claim(qi, i != 0));
      if (it >= 0) return it;
      empty |= 1u << qi;
    }
    return -1;
  };
  auto publish_item = [&](bool prefetched, uint64_t ht, unsigned empty) {
    if (wave == 0 && lane_id() == 0) {
      ticket_slot[0] = take_item(prefetched, ht, empty);
      ticket_slot[1] = (int)empty;
    }
  };
  int item = (int)blockIdx.x;
  unsigned empty_q = 0;  // queues found exhausted (scalar, same in every wave)
  if (dynamic) {
    publish_item(false, 0ull, 0u);
    __syncthreads();
    item = __builtin_amdgcn_readfirstlane(ticket_slot[0]);
    empty_q = (unsigned)__builtin_amdgcn_readfirstlane(ticket_slot[1]);
  }
  while (item >= 0) {
    // Lane-dependent values are derived per item from an opaque lane index,
    // so none of them is hoisted out of the item loop and kept live in VGPRs
    // between items (the main loop needs every register).
    int lane = lane_id();
    asm volatile("" : "+v"(lane));
    const int tid = wave * 64 + lane;
    const int wq = wave & 3;    // quarter of the direct-load segments
    const bool v_role = SPLIT_ROLES && wave >= 4;

    const int hi = lane >> 5;   // which half of the wave
    const int ql = lane & 31;   // query column owned by this lane
    const int grp = lane >> 4;  // 16-lane group (transposing reads)
    const int gi = lane & 15;
    // Thread 0: the head claim on the own queue for the next item, issued at
    // the start of this item's last step.
    const bool prefetch = dynamic && !((empty_q >> own_q) & 1u);
    uint64_t next_claim = 0ull;

    // Paired key split (KSPLIT at head_dim 64 with a.pair_split): the work
    // item is a pair of query blocks of one (batch, head), A = block nqb-1-i
    // and B = block i (none when the two coincide, the middle block of an odd
    // count), so under causal masking A is the larger.  Their T_A + T_B key
    // tiles are dealt evenly to the two key groups: group 0 runs tiles
    // [0, h) of A and group 1 the rest of A, then all of B, h = ceil((T_A +
    // T_B) / 2), both h steps.  Group 1 hands its share of A (unnormalised O,
    // running max, partial sums) to group 0 through LDS when it moves on to B;
    // group 0 merges it at the end and stores A, group 1 stores B.  Tile
    // indices in the step loop are then virtual (group 1 counts on from h):
    // tile_of maps them to key tiles, and seg_b tells B's from A's.
    const bool pairs = PAIRS && a.pair_split != 0;
    // Mask ranges make the blocks' work uneven like a causal launch's (a
    // causal mask given as bits): the same largest-first order then.
    const bool big_first = CAUSAL || (MASK && !KEY_BYTES && a.mranges != nullptr);
    const Work w = block_work(a, item, big_first && !pairs, dynamic);
    const int b = w.b, hq = w.hq, hkv = w.hkv;
    const int N = a.n;    // query rows
    const int NK = a.nk;  // key rows
    const int nqb = (N + BLOCK_M - 1) / BLOCK_M;
    const int qb = pairs ? nqb - 1 - w.qb : w.qb;
    const int qb_b = pairs && w.qb < nqb - 1 - w.qb ? w.qb : -1;  // block B, or -1
    const int bh = b * a.hq + hq;
    const int q0 = qb * BLOCK_M;
    const int qw = q0 + rw * 32;
    const int qrow = qw + ql;
    // Causal: the last key tile any row of this wave sees (floor division).
    const int wave_last_tile = (qw + 31 + a.diag) >> 6;
    const int qw_b = qb_b * BLOCK_M + rw * 32;  // (pairs with a block B)
    const int qrow_b = qw_b + ql;
    const bool g1b = pairs && kgrp == 1 && qb_b >= 0;  // this group moves on to B

    const _Float16* Qp = a.q + b * a.qsb + hq * a.qsh;
    // Mask bits of this lane's query row (rows past N read row N - 1), or
    // (key-padding bytes, a.mkeys) batch b's key row: lane l reads key
    // 64 j + l of tile j and a ballot forms the tile's word.
    const uint64_t* mrow =
        MASK && !KEY_BYTES
            ? a.mbits + b * a.msb + hq * a.msh + (int64_t)min(qrow, N - 1) * a.msq
            : nullptr;
    const uint8_t* krow = KEY_BYTES ? a.mkeys + b * a.mksb : nullptr;
    // What a step loads ahead for tile j: the lane's mask word, or its key
    // byte (lanes past the last key read the last key's byte, an
    // unconditional load; those keys are hidden by the sequence-end mask
    // whatever their bit says).
    auto mask_ahead = [&](int j) -> uint64_t {
      if constexpr (KEY_BYTES) return krow[(int64_t)min(j * kBlockN + lane, NK - 1) * a.mksk];
      else return mrow[j];
    };
    const _Float16* Kp = a.k + b * a.ksb + hkv * a.ksh;
    const _Float16* Vp = a.v + b * a.vsb + hkv * a.vsh;

    // Q^T fragments (B operand of S^T = K Q^T), resident for the whole kernel
    // (in pair mode group 1 also holds B's, which replace A's when it moves on).
    auto load_q = [&](int row, half8 (&qd)[KK]) {
      if (row < N) {
        const _Float16* qp = Qp + (int64_t)row * a.qsn + 8 * hi;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) qd[kk] = *(const half8*)(qp + 16 * kk);
      } else {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) qd[kk] = (half8)(_Float16)0;
      }
      if (a.negate_q) {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) qd[kk] = negate16(qd[kk]);
      }
    };
    half8 qf[KK];
    half8 qf_b[PAIRS ? KK : 1];
    load_q(qrow, qf);
    if constexpr (PAIRS) {
      if (g1b) load_q(qrow_b, qf_b);
    }

    // Mask ranges (mask bits with a.mranges): the span of keys some row of
    // the block sees, [span_lo, span_hi); the tiles outside it hide every
    // key from every row, so skipping them changes no result.  Each lane
    // reads its row's pair (rows past N read row N - 1), the wave and then
    // the workgroup (through the buffer of V_{STAGES-1}, which no load writes
    // before step 0, whose loads follow a barrier) take the union.
    // Dense waves: when every row of the wave sees exactly the interval of
    // its pair (bit 31 of the first entry), the keys [in_lo, in_hi) are
    // visible to all of them, and a tile inside that span needs no mask word
    // (it would be all ones; the sequence end and the causal diagonal are
    // masked as without a mask).  in_hi <= in_lo: no such tile.
    int span_lo = 0, span_hi = NK;
    int in_lo = 0, in_hi = 0;
    if constexpr (MASK && !KEY_BYTES) {
      if (a.mranges != nullptr) {
        const int32_t* rr =
            a.mranges + 2 * (b * a.mrsb + hq * a.mrsh + (int64_t)min(qrow, N - 1) * a.mrsq);
        const int32_t first = rr[0];
        span_lo = range_first_key(first);
        span_hi = rr[1];
        int lo_max = span_lo, hi_min = span_hi;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          lo_max = max(lo_max, __shfl_xor(lo_max, d));
          hi_min = min(hi_min, __shfl_xor(hi_min, d));
        }
        if (__builtin_amdgcn_ballot_w64(!range_is_dense(first)) == 0) {
          in_lo = __builtin_amdgcn_readfirstlane(lo_max);
          in_hi = __builtin_amdgcn_readfirstlane(hi_min);
        }
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          span_lo = min(span_lo, __shfl_xor(span_lo, d));
          span_hi = max(span_hi, __shfl_xor(span_hi, d));
        }
        int* const xs = (int*)(STAGES == 3 ? v_lds2 : v_lds1) + 16;
        if (lane == 0) {
          xs[2 * wave] = span_lo;
          xs[2 * wave + 1] = span_hi;
        }
        __syncthreads();
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
          span_lo = min(span_lo, xs[2 * w]);
          span_hi = max(span_hi, xs[2 * w + 1]);
        }
        span_lo = __builtin_amdgcn_readfirstlane(span_lo);
        span_hi = __builtin_amdgcn_readfirstlane(span_hi);
      }
    }
    // The mask word (or key byte) prepare takes for tile j: none to load for
    // a tile every row of a dense wave sees in full.
    auto mask_word = [&](int j) -> uint64_t {
      if (j * kBlockN >= in_lo && j * kBlockN + kBlockN <= in_hi) return ~0ull;
      return mask_ahead(j);
    };
    // Keys this block can see (none for a block entirely before the diagonal).
    const int kv_len = min(CAUSAL ? max(0, min(NK, q0 + BLOCK_M + a.diag)) : NK, span_hi);
    const int block_tiles = (kv_len + kBlockN - 1) / kBlockN;
    // Key tiles of block B (pair mode; 0 without one).
    const int kv_len_b =
        qb_b >= 0 ? (CAUSAL ? max(0, min(NK, qb_b * BLOCK_M + BLOCK_M + a.diag)) : NK) : 0;
    const int tiles_b = (kv_len_b + kBlockN - 1) / kBlockN;
    const int first_tile = span_lo < span_hi ? span_lo / kBlockN : 0;
    // Tiles [tile0, tile0 + ntiles) of this wave's key group.  KSPLIT: both
    // groups run ceil((block_tiles + tiles_b) / 2) steps (so their barriers
    // pair up); a tile past the block's keys is fully masked and adds
    // exactly nothing.
    const int ntiles =
        KSPLIT ? (block_tiles + tiles_b + 1) / 2 : max(0, block_tiles - first_tile);
    const int tile0 = KSPLIT ? kgrp * ntiles : first_tile;
    const int tile_end = tile0 + ntiles;
    // Virtual tile j (pair mode): B's tile j - T_A once j reaches T_A.
    auto seg_b = [&](int j) { return PAIRS && qb_b >= 0 && j >= block_tiles; };
    auto tile_of = [&](int j) { return seg_b(j) ? j - block_tiles : j; };
    // Group 1 starting directly in B holds B's Q from the start.
    if constexpr (PAIRS) {
      if (g1b && tile0 >= block_tiles) {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) qf[kk] = qf_b[kk];
      }
    }

    // Direct-load map: wave quarter wq fills 1 KB segments wq, wq + 4, ... of a
    // tile; lane l of a segment covers tile bytes [1024 seg + 16 l, +16).  The
    // global byte offset inside a tile of each segment (padding lanes: past
    // the end).  goff_a: K (4 waves) or this wave's tile kind (8 waves);
    // goff_b: V with its own stride (4 waves, different strides only).
    constexpr bool OWN_B = !SPLIT_ROLES && !KV_SAME_STRIDE;
    int goff_a[SEGQ], goff_b_own[OWN_B ? SEGQ : 1];
    int* goff_b = OWN_B ? goff_b_own : goff_a;
    const int64_t a_stride = v_role ? a.vsn : a.ksn;
#pragma unroll
    for (int s = 0; s < SEGQ; ++s) {
      const int pos = (wq + 4 * s) * 1024 + 16 * lane;  // bytes into the tile
      const int row = pos / (2 * L::Pitch);
      const int within = pos - row * (2 * L::Pitch);
      if constexpr (DENSE) {  // 8 rows of 128 bytes per segment, no padding
        const int c = (within >> 4) ^ dense_swizzle(row);
        goff_a[s] = (int)(row * a_stride * 2) + 16 * c;
        if (OWN_B) goff_b[s] = (int)(row * a.vsn * 2) + 16 * c;
      } else if (within < 2 * D) {
        const int c = (within >> 4) ^ ((row >> 2) & 3);
        goff_a[s] = (int)(row * a_stride * 2) + 16 * c;
        if (OWN_B) goff_b[s] = (int)(row * a.vsn * 2) + 16 * c;
      } else {
        goff_a[s] = -16;  // 0xfffffff0: beyond any window -> writes zeros
        if (OWN_B) goff_b[s] = -16;
      }
    }
    const int k_tile_bytes = (int)(kBlockN * a.ksn * 2);
    const int v_tile_bytes = (int)(kBlockN * a.vsn * 2);
    const int k_all_bytes = (int)(NK * a.ksn * 2);
    const int v_all_bytes = (int)(NK * a.vsn * 2);

    // Buffer selection by compile-time stage index (and the key group).
    auto kbuf = [&](auto st) -> _Float16* {
      constexpr int S = decltype(st)::value % STAGES;
      if constexpr (S == 0) return k_lds0 + gofs;
      else if constexpr (S == 1) return k_lds1 + gofs;
      else return k_lds2 + gofs;
    };
    auto vbuf = [&](auto st) -> _Float16* {
      constexpr int S = decltype(st)::value % STAGES;
      if constexpr (S == 0) return v_lds0 + gofs;
      else if constexpr (S == 1) return v_lds1 + gofs;
      else return v_lds2 + gofs;
    };
    // The offset is recomputed at each load (an opaque SGPR): hoisted, the
    // 4 x SEGQ segment addresses would live in SGPRs across the loop and be
    // spilled to VGPR lanes, each reload a v_readlane in the MFMA slots.
    auto lds_seg = [&](_Float16* tile, int s) -> lds_void* {
      int off = (wq + 4 * s) * 512;
      asm volatile("" : "+s"(off));
      return (lds_void*)(tile + off);
    };
    // Buffer windows of (virtual) tile jv (empty past the last tile: every
    // lane reads 0).
    auto k_window = [&](int jv) {
      const int j = tile_of(jv);
      const int bytes = k_all_bytes - j * k_tile_bytes;
      return make_rsrc(Kp + (int64_t)j * kBlockN * a.ksn, bytes > 0 ? bytes : 0);
    };
    auto v_window = [&](int jv) {
      const int j = tile_of(jv);
      const int bytes = v_all_bytes - j * v_tile_bytes;
      return make_rsrc(Vp + (int64_t)j * kBlockN * a.vsn, bytes > 0 ? bytes : 0);
    };
    // This wave's segments of K tile j (into kdst) or V tile j (into vdst).
    auto load_tile = [&](bool is_v, int j, _Float16* dst) {
      const __amdgpu_buffer_rsrc_t r = is_v ? v_window(j) : k_window(j);
#pragma unroll
      for (int s = 0; s < SEGQ; ++s)
        direct_load16(r, lds_seg(dst, s), (is_v && OWN_B) ? goff_b[s] : goff_a[s]);
    };

    // Per-lane LDS bases of the operand reads (see Lds, LdsDense): K rows ql
    // (+32t), chunk 2kk + hi; V rows 16ks + 4hi + gi/4 (+8), dims 32mt +
    // 16(grp&1) + 4(gi&3).  Padded: the swizzle touches the low two chunk bits,
    // so two K bases (kk even, odd) and two V bases (rows +0, +8) with
    // immediates for the rest; dense: one K base per kk and two V bases per
    // 64-dim half (mt).
    const int sK = (ql >> 2) & 3;
    const int k_base_even = ql * L::Pitch + 8 * (hi ^ sK);
    const int k_base_odd = ql * L::Pitch + 8 * ((2 + hi) ^ sK);
    const int v_row = 4 * hi + (gi >> 2);
    const int v_c = 2 * (grp & 1) + ((gi & 3) >> 1);
    const int v_base0 = v_row * L::Pitch + 8 * (v_c ^ hi) + 4 * (gi & 1);
    const int v_base1 = (v_row + 8) * L::Pitch + 8 * (v_c ^ (hi + 2)) + 4 * (gi & 1);
    int kd_base[DENSE ? KK : 1], vd_base0[DENSE ? MT : 1], vd_base1[DENSE ? MT : 1];
    if constexpr (DENSE) {
      const int sw = dense_swizzle(ql);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) kd_base[kk] = ql * L::Pitch + 8 * ((2 * kk + hi) ^ sw);
      const int sw0 = dense_swizzle(v_row), sw1 = dense_swizzle(v_row + 8);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        vd_base0[mt] = v_row * L::Pitch + 8 * ((v_c + 4 * mt) ^ sw0) + 4 * (gi & 1);
        vd_base1[mt] = (v_row + 8) * L::Pitch + 8 * ((v_c + 4 * mt) ^ sw1) + 4 * (gi & 1);
      }
    }

    // K operand i (sub-tile t = i / KK, step kk = i % KK) of one K buffer.
    auto read_k = [&](const _Float16* Ks, int i) -> half8 {
      const int t = i / KK, kk = i % KK;
      if constexpr (DENSE) return *(const half8*)(Ks + kd_base[kk] + 32 * t * L::Pitch);
      const int off = ((kk & 1) ? k_base_odd : k_base_even) + 32 * t * L::Pitch + 32 * (kk >> 1);
      return *(const half8*)(Ks + off);
    };
    // A operand of the row-sum tile (ROWSUM): row 0 all ones (lanes 0 and 32
    // hold its two 8-key halves), rows 1-31 zero.  Row 0 of that tile's
    // accumulator, lane c's register 0, is query c's sum of P; lanes 32-63
    // hold row 4 there, which stays zero, so halves_sum of register 0 gives
    // the sum in both lanes of the query.
    const half8 ones_a = ql == 0 ? (half8)E::round(1.0f) : (half8)(_Float16)0;
    // V^T operand v (16-key step ks = v / MTX, output tile mt = v % MTX; the
    // row-sum tile mt = MT takes the constant operand).
    auto read_v = [&](const _Float16* Vs, int v) -> half8 {
      const int ks = v / MTX, mt = v % MTX;
      if (ROWSUM && mt == MT) return ones_a;
      if constexpr (DENSE) {
        const int imm = 16 * ks * L::Pitch;
        const half4 lo = ds_read_tr16(Vs + vd_base0[mt] + imm);
        const half4 hi4 = ds_read_tr16(Vs + vd_base1[mt] + imm);
        return __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
      }
      const int imm = 16 * ks * L::Pitch + 32 * mt;
      const half4 lo = ds_read_tr16(Vs + v_base0 + imm);
      const half4 hi4 = ds_read_tr16(Vs + v_base1 + imm);
      return __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
    };

    float16v oacc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) oacc[mt] = (float16v)0.0f;
    float16v lacc = (float16v)0.0f;  // row-sum tile (ROWSUM)
    float m_run = -__builtin_inff();
    float l_run = 0.0f;              // the lane's part of its row sum (VALU row sums)
    const float c2 = a.c;  // |scale| * log2(e)

    // S^T of two tiles in flight, ping-pong by the parity of the step's
    // position in the unrolled loop: step u reads s_buf[u & 1] and fills the
    // other one (with three stages, one copy per three steps restores it).
    float16v s_buf[2][2];
    auto row_max = [](const float16v (&s)[2]) {
      float m0 = s[0][0], m1 = s[1][0];
#pragma unroll
      for (int i = 1; i < 16; ++i) {
        m0 = fmaxf(m0, s[0][i]);
        m1 = fmaxf(m1, s[1][i]);
      }
      return fmaxf(m0, m1);
    };
    float mc = 0.0f;  // running max of tile j's rows, times c2 (exp2 offset)
    // A row outgrew its running max by more than 2^kRescaleLog2 iff its max
    // score exceeds thr = m_run + kRescaleLog2 / c2 (-inf before any key).
    float thr = -__builtin_inff();

    // Pair mode, group 1: its share of block A (unnormalised O, running max,
    // lane partial sums) into the exchange area for group 0, and a fresh
    // state for block B.
    constexpr bool XAREA = KSPLIT && D == 64;  // the exchange area (pair_exchange)
    float* const pair_xo = pair_exchange<XAREA, MT>() + (XAREA ? rw * (MT * 1024 + 128) : 0);
    auto hand_off_a = [&]() {
      if constexpr (PAIRS) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *(float4*)(pair_xo + ((mt * 4 + g) * 64 + lane) * 4) =
                float4{oacc[mt][4 * g], oacc[mt][4 * g + 1], oacc[mt][4 * g + 2],
                       oacc[mt][4 * g + 3]};
        pair_xo[MT * 1024 + lane] = m_run;
        pair_xo[MT * 1024 + 64 + lane] = l_run;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) oacc[mt] = (float16v)0.0f;
        m_run = -__builtin_inff();
        l_run = 0.0f;
        mc = 0.0f;
        thr = -__builtin_inff();
      }
    };

    // Prepares tile j's scores for its softmax: masks them if tile j crosses
    // the sequence end or this wave's causal diagonal, or (MASK) hides a key
    // from some row of the wave (the unmasked max mx is then recomputed),
    // and raises the running max when some row outgrew it by more than
    // 2^kRescaleLog2 (rescaling O and l, and updating mc and thr).  mx: the
    // lane's max over its half of the row (the two wave halves hold the
    // row's other 16 keys of each 32-key sub-tile; the threshold test needs
    // no exchange between them, the rare rescale does).  mw: the lane's mask
    // word of tile j (bit k: key 64 j + k visible), or its key byte (key-padding
    // bytes), from which the wave's ballot forms that word.
    auto prepare = [&](int jv, float16v (&s)[2], float mx, uint64_t mw) {
      if constexpr (KEY_BYTES) mw = __builtin_amdgcn_ballot_w64(mw != 0);
      const int kstart = tile_of(jv) * kBlockN;
      const bool in_b = seg_b(jv);
      const int qw_j = in_b ? qw_b : qw;
      const int qrow_j = in_b ? qrow_b : qrow;
      bool need_mask =
          (kstart + kBlockN > NK) || (CAUSAL && kstart + kBlockN - 1 > qw_j + a.diag);
      if (MASK) need_mask = need_mask || __builtin_amdgcn_ballot_w64(~mw != 0) != 0;
      if (need_mask) {
        const uint64_t mws = mw >> (4 * hi);  // bit 32 t + 8 (i / 4) + i % 4: element (t, i)
        // Element (t, i) holds key kstart + 4 hi + off, off = 32 t + 8 (i / 4)
        // + i % 4 (a constant); it is visible iff off <= lim.
        const int last = CAUSAL ? min(NK - 1, qrow_j + a.diag) : NK - 1;
        const int lim = last - kstart - 4 * hi;
        // static_for: a loop the unroller leaves rolled would index s at run
        // time and move the score registers to scratch memory.
        static_for<32>([&](auto e_c) {
          constexpr int e = decltype(e_c)::value;
          constexpr int t = e >> 4, i = e & 15;
          constexpr int off = 32 * t + 8 * (i >> 2) + (i & 3);
          bool masked = off > lim;
          if (MASK) masked = masked || ((mws >> off) & 1) == 0;
          if (masked) s[t][i] = -__builtin_inff();
        });
        mx = row_max(s);
      }
      if (__builtin_amdgcn_ballot_w64(mx > thr) != 0) {
        const float m_new = fmaxf(m_run, halves_max(mx));
        const float m_use = (m_new == -__builtin_inff()) ? 0.0f : m_new;
        const float alpha =
            (m_run == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f((m_run - m_use) * c2);
        if constexpr (ROWSUM) lacc[0] *= alpha;  // its other entries stay 0
        else l_run *= alpha;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) oacc[mt] *= alpha;
        m_run = m_new;
        mc = m_use * c2;
        thr = m_new + kRescaleLog2 / c2;
      }
    };

    // One pipeline step for tile j, at position U of the unrolled loop (its
    // V tile is in buffer U % STAGES), whose scores are prepared.  HAS_NEXT:
    // tile j+1 exists, so S_{j+1} is computed (and prepared) here and the
    // loads of K_{j+STAGES} and V_{j+STAGES-1} are issued.
    auto step = [&](int j, auto has_next_t, auto u_t) {
      constexpr bool HAS_NEXT = decltype(has_next_t)::value;
      constexpr int U = decltype(u_t)::value;
      if constexpr (!HAS_NEXT) {
        if (prefetch && tid == 0) next_claim = claim(own_q, false);
      }
      constexpr int PAR = U & 1;
      constexpr int ns = HAS_NEXT ? NS : 0;     // S MFMAs this step
      const _Float16* Kn = kbuf(std::integral_constant<int, U + 1>{});
      const _Float16* Vc = vbuf(std::integral_constant<int, U>{});
      float16v (&s_cur)[2] = s_buf[PAR];
      float16v (&s_nxt)[2] = s_buf[1 - PAR];

      // Direct loads of K_{j+STAGES} (into the buffer K_j used) and
      // V_{j+STAGES-1} (into the buffer V_{j-1} used), one 1 KB segment after
      // each of the first MFMAs, so the address unit's queueing overlaps MFMA
      // execution.  Past the last tile the windows are empty.
      __amdgpu_buffer_rsrc_t rk_next, rv_next;
      uint64_t mw_next = ~0ull;
      if (HAS_NEXT) {
        rk_next = k_window(j + STAGES);
        rv_next = v_window(j + STAGES - 1);
        if (MASK) mw_next = mask_word(j + 1);  // consumed by prepare(j + 1) at the end
      }
      _Float16* k_dst = kbuf(std::integral_constant<int, U>{});
      _Float16* v_dst = vbuf(std::integral_constant<int, U + STAGES - 1>{});
      auto issue_load = [&](int q) {
        if constexpr (SPLIT_ROLES) {  // q < SEGQ: segment q of this wave's tile kind
          direct_load16(v_role ? rv_next : rk_next, lds_seg(v_role ? v_dst : k_dst, q), goff_a[q]);
        } else {  // q < SEGQ: K segment q, else V segment q - SEGQ
          if (q < SEGQ)
            direct_load16(rk_next, lds_seg(k_dst, q), goff_a[q]);
          else
            direct_load16(rv_next, lds_seg(v_dst, q - SEGQ), goff_b[q - SEGQ]);
        }
      };

      // ---- slots: S_{j+1} MFMAs, then P_j V_j --------------------------------
      // The softmax of S_j (16 pairs of scores) is spread over the slots.
      // Within a slot the MFMA is issued first, so the pairs of 16-key step ks
      // must sit in a slot before the first P V MFMA of step ks; pairs that
      // cannot (the last tile has no S MFMAs to hide them behind) go first.
      constexpr int NB = ns + NPV;                    // MFMA slots
      constexpr int PV_FIRST = ns;                    // slot of the first P V MFMA
      constexpr int PAIR_SLOTS = NB - MTX;            // slots available to pairs
      half8 kf[NS];
      // P operands as 32-bit lanes: each converted pair is written whole
      // (inserting its two halves one by one makes the compiler convert and
      // repack per element).
      uint4v pf[4];
      half8 vf[NPV];
      constexpr auto pair_slot = [](int p) constexpr {
        const int spread = (p * PAIR_SLOTS) / 16;
        const int last_ok = PV_FIRST + (p / 4) * MTX - 1;
        return spread < last_ok ? spread : last_ok;
      };
      // Row max of S_{j+1} over the lane's half of the row: element e
      // (sub-tile t = e / 16) is folded in at max_slot(e), a few slots after
      // the last MFMA into sub-tile t.
      constexpr auto max_slot = [](int e) constexpr {
        const int t = e >> 4, i = e & 15;
        const int first = (t + 1) * KK + 2;
        const int span = (t == 0 ? KK : NB - 1 - first);
        const int s = first + (i * span) / 16;
        return s < NB - 1 ? s : NB - 1;
      };
      constexpr auto last_max_slot = [max_slot]() constexpr {
        int m = 0;
        for (int e = 0; e < 32; ++e) m = max_slot(e) > m ? max_slot(e) : m;
        return m;
      };
      auto softmax_pair = [&](auto p_c) {
        constexpr int p = decltype(p_c)::value;
        constexpr int e = 2 * p;
        constexpr int t = e >> 4, i = e & 15;
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[t][i], c2, -mc));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[t][i + 1], c2, -mc));
        const half2v pr = E::pack(p0, p1);
        pf[2 * t + (i >> 3)][(i & 7) >> 1] = __builtin_bit_cast(unsigned, pr);
        if constexpr (!ROWSUM) {
          l_run = E::sum2(pr, l_run);
          // Keeps the row-sum update in this slot: left alone, the compiler
          // sinks all 16 of a step's (serially dependent) updates, with
          // repacks of their operands, to after the last MFMA, where nothing
          // hides their latency.
          asm volatile("" : "+v"(l_run));
        }
      };
      static_for<16>([&](auto p_c) {
        if constexpr (pair_slot(decltype(p_c)::value) < 0) softmax_pair(p_c);
      });
      // Head_dim 128: the wave issuing its MFMA slots outranks the other
      // workgroup's wave on the SIMD while that one runs prepare / waits at its
      // barrier (measured +1% on C4, +0.3% on C5; at head_dim 64, whose steps
      // are VALU-bound, -2%, so not there).
      // Pair mode, group 1: S_{j+1} is B's first tile.
      if constexpr (PAIRS) {
        if (HAS_NEXT && g1b && j + 1 == block_tiles) {
#pragma unroll
          for (int kk = 0; kk < KK; ++kk) qf[kk] = qf_b[kk];
        }
      }
      if constexpr (D == 128) __builtin_amdgcn_s_setprio(1);
      static_for<(PFK < ns ? PFK : ns)>([&](auto i_c) {
        kf[decltype(i_c)::value] = read_k(Kn, decltype(i_c)::value);
      });
      float mx_next = -__builtin_inff();
      static_for<NB>([&](auto slot_c) {
        constexpr int slot = decltype(slot_c)::value;
        // V operand reads, PFV MFMAs ahead of their use
        if constexpr (slot == (PV_FIRST >= PFV ? PV_FIRST - PFV : 0)) {
          static_for<PFV>([&](auto v_c) {
            vf[decltype(v_c)::value] = read_v(Vc, decltype(v_c)::value);
          });
        }
        if constexpr (slot >= PV_FIRST && slot - PV_FIRST + PFV < NPV) {
          vf[slot - PV_FIRST + PFV] = read_v(Vc, slot - PV_FIRST + PFV);
        }
        // the MFMA of this slot
        if constexpr (slot < PV_FIRST) {
          constexpr int i = slot;
          if constexpr (i + PFK < ns) kf[i + PFK] = read_k(Kn, i + PFK);
          constexpr int t = i / KK, kk = i % KK;
          s_nxt[t] = E::mfma(kf[i], qf[kk], kk == 0 ? (float16v)0.0f : s_nxt[t]);
        } else {
          constexpr int v = slot - PV_FIRST;
          constexpr int ks = v / MTX, mt = v % MTX;
          if constexpr (mt == MT)
            lacc = E::mfma(vf[v], __builtin_bit_cast(half8, pf[ks]), lacc);
          else
            oacc[mt] = E::mfma(vf[v], __builtin_bit_cast(half8, pf[ks]), oacc[mt]);
        }
        if constexpr (HAS_NEXT) {
          static_for<LPW>([&](auto q_c) {
            constexpr int q = decltype(q_c)::value;
            if constexpr ((q * (NB / 2)) / LPW == slot) issue_load(q);
          });
          static_for<32>([&](auto e_c) {
            constexpr int e = decltype(e_c)::value;
            if constexpr (max_slot(e) == slot) mx_next = fmaxf(mx_next, s_nxt[e >> 4][e & 15]);
          });
          // Pinned after its last update: otherwise the compiler sinks the whole
          // max chain into prepare's unmasked path, out of the MFMA slots.
          if constexpr (slot == last_max_slot()) asm volatile("" : "+v"(mx_next));
        }
        static_for<16>([&](auto p_c) {
          if constexpr (pair_slot(decltype(p_c)::value) == slot) softmax_pair(p_c);
        });
        fence_schedule();
      });

      if constexpr (D == 128) __builtin_amdgcn_s_setprio(0);
      // Pair mode, group 1: P_j V_j was A's last tile.
      if constexpr (PAIRS) {
        if (g1b && j + 1 == block_tiles) hand_off_a();
      }
      if (HAS_NEXT) {
        prepare(j + 1, s_nxt, mx_next, mw_next);
        // The loads of the previous step have landed (those of this step may
        // still be in flight with three stages), and every wave is done with
        // the buffers the next step's loads overwrite.
        barrier_after_loads<STAGES == 3 ? LPW : 0>();
      }
    };

    // Pair mode, group 1 with no tile of A: its (empty) share of A.
    if constexpr (PAIRS) {
      if (g1b && tile0 >= block_tiles) hand_off_a();
    }
    // ---- prologue: K_0..K_{STAGES-1} and V_0..V_{STAGES-2} into LDS; S_0 -----
    // (tile indices relative to tile0)
    if (ntiles > 0) {
      static_for<STAGES>([&](auto t_c) {
        if (!v_role) load_tile(false, tile0 + decltype(t_c)::value, kbuf(t_c));
      });
      static_for<STAGES - 1>([&](auto t_c) {
        if (!SPLIT_ROLES || v_role) load_tile(true, tile0 + decltype(t_c)::value, vbuf(t_c));
      });
    }
    // S_0 needs Q and K_0 only: the wave waits for its direct loads up to
    // those of K_0 (they complete in issue order; a split-role V wave loads
    // no K and waits for none), and the rest land while S_0 is computed.  Q
    // sits in registers, whose loads the compiler waits for itself.
    // Measured: 1.013x on B=4 H=12 N=1024 d=64, 1.006x on the causal
    // B=4 H=8 N=2048 d=64, 1.000-1.005x on longer launches; results bitwise
    // unchanged.
    if (ntiles > 0) {
      constexpr int AFTER_K0 = SPLIT_ROLES ? (STAGES - 1) * SEGQ : 2 * (STAGES - 1) * SEGQ;
      barrier_after_loads<AFTER_K0>();
    } else {
      barrier_after_loads<0>();
    }
    if (ntiles > 0) {
      const _Float16* k_first = kbuf(std::integral_constant<int, 0>{});
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        s_buf[0][t] = (float16v)0.0f;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          s_buf[0][t] = E::mfma(read_k(k_first, t * KK + kk), qf[kk], s_buf[0][t]);
      }
      prepare(tile0, s_buf[0], row_max(s_buf[0]), MASK ? mask_word(tile0) : ~0ull);
      // Step 0 loads K_STAGES into K_0's buffer: every wave must be done
      // reading it for S_0 first; and the prologue's other tiles must have
      // landed.
      barrier_after_loads<0>();
      using I0 = std::integral_constant<int, 0>;
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      int j = tile0;
      // Causal, head_dim 64: the wave computes the tiles up to the last one
      // its rows see (at least the first); the tiles after it lie wholly past
      // its diagonal, where its scores, probabilities and P V products are
      // exactly zero, so for those it only issues its share of the loads and
      // meets the barriers, leaving its SIMD to the waves that still see keys
      // (the upper waves of a block skip the last tiles of its diagonal; C3
      // 1.016x, B=1 Hq=32 N=4096 on 256-row workgroups 1.019x, results
      // bitwise unchanged).  Not at head_dim 128: the extra tail code costs
      // the 4-wave kernel registers it does not have (spills, 0.90-0.96x),
      // and the 256-row kernel measured no gain.
      constexpr bool TRIM = CAUSAL && !KSPLIT && D == 64;
      const int cend = TRIM ? min(tile_end, max(tile0 + 1, wave_last_tile + 1)) : tile_end;
      for (; j + STAGES < cend; j += STAGES) {  // every step has a next tile
        step(j, Flag<true>{}, I0{});
        step(j + 1, Flag<true>{}, I1{});
        if constexpr (STAGES == 3) {
          step(j + 2, Flag<true>{}, I2{});
          s_buf[0][0] = s_buf[1][0];
          s_buf[0][1] = s_buf[1][1];
        }
      }
      bool trimmed = false;
      if constexpr (TRIM) {
        if (cend < tile_end) {
          trimmed = true;
          // 1 .. STAGES computed steps left, each with a next tile (its loads)
          const int rest = cend - j;
          step(j, Flag<true>{}, I0{});
          if (rest >= 2) step(j + 1, Flag<true>{}, I1{});
          if constexpr (STAGES == 3) {
            if (rest == 3) step(j + 2, Flag<true>{}, I2{});
          }
          for (j += rest; j + 1 < tile_end; ++j) {
            // Loads of the step at position (j - tile0) % STAGES: K_{j+STAGES}
            // into K_j's buffer, V_{j+STAGES-1} into V_{j-1}'s.
            const int u = (j - tile0) % STAGES;
            _Float16* const k_dst =
                u == 0 ? kbuf(I0{}) : (u == 1 || STAGES == 2) ? kbuf(I1{}) : kbuf(I2{});
            const int uv = (u + STAGES - 1) % STAGES;
            _Float16* const v_dst =
                uv == 0 ? vbuf(I0{}) : (uv == 1 || STAGES == 2) ? vbuf(I1{}) : vbuf(I2{});
            const __amdgpu_buffer_rsrc_t rk = k_window(j + STAGES);
            const __amdgpu_buffer_rsrc_t rv = v_window(j + STAGES - 1);
            static_for<LPW>([&](auto q_c) {
              constexpr int q = decltype(q_c)::value;
              if constexpr (SPLIT_ROLES)
                direct_load16(v_role ? rv : rk, lds_seg(v_role ? v_dst : k_dst, q), goff_a[q]);
              else if constexpr (q < SEGQ)
                direct_load16(rk, lds_seg(k_dst, q), goff_a[q]);
              else
                direct_load16(rv, lds_seg(v_dst, q - SEGQ), goff_b[q - SEGQ]);
            });
            barrier_after_loads<STAGES == 3 ? LPW : 0>();
          }
          // The item's last step: the head claim for the next item.
          if (prefetch && tid == 0) next_claim = claim(own_q, false);
        }
      }
      if (!trimmed) {
        const int rest = tile_end - j;  // 1 .. STAGES steps left, the last one without a next tile
        if (rest == 1) {
          step(j, Flag<false>{}, I0{});
        } else if (STAGES == 2 || rest == 2) {
          step(j, Flag<true>{}, I0{});
          step(j + 1, Flag<false>{}, I1{});
        } else if constexpr (STAGES == 3) {
          step(j, Flag<true>{}, I0{});
          step(j + 1, Flag<true>{}, I1{});
          step(j + 2, Flag<false>{}, I2{});
        }
      }
    }
    // No direct load may land in LDS after the workgroup ends.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    // From here on l_run is the lane's part of its row sum either way (the
    // row-sum tile holds all of it in lanes 0-31, zero in lanes 32-63).
    if constexpr (ROWSUM) l_run = lacc[0];

    if constexpr (KSPLIT) {
      // Group 1 wave w+4 hands its O (unnormalised), running max and partial
      // sums to group 0 wave w (same rows, same lane layout) through the
      // exchange area (head_dim 64; in pair mode a group 1 that moved on to
      // block B filled it already) or the group-1 half of one LDS array,
      // which no wave reads any more (head_dim 128).
      __syncthreads();
      _Float16* const arr = rw == 0 ? k_lds0 : rw == 1 ? k_lds1 : rw == 2 ? v_lds0 : v_lds1;
      float* const xo = XAREA ? pair_xo : (float*)(arr + L::Tile);
      static_assert(XAREA || MT * 16 * 64 * 4 + 2 * 64 * 4 <= L::Tile * 2, "exchange fits a tile");
      if (kgrp == 1 && !g1b) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *(float4*)(xo + ((mt * 4 + g) * 64 + lane) * 4) =
                float4{oacc[mt][4 * g], oacc[mt][4 * g + 1], oacc[mt][4 * g + 2],
                       oacc[mt][4 * g + 3]};
        xo[MT * 1024 + lane] = m_run;
        xo[MT * 1024 + 64 + lane] = l_run;
      }
      __syncthreads();
      if (kgrp == 0) {
        const float m1 = xo[MT * 1024 + lane];
        const float l1 = xo[MT * 1024 + 64 + lane];
        const float m_new = fmaxf(m_run, m1);
        const float m_use = (m_new == -__builtin_inff()) ? 0.0f : m_new;
        const float a0 =
            (m_run == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f((m_run - m_use) * c2);
        const float a1 =
            (m1 == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f((m1 - m_use) * c2);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float4 o1 = *(const float4*)(xo + ((mt * 4 + g) * 64 + lane) * 4);
            oacc[mt][4 * g] = oacc[mt][4 * g] * a0 + o1.x * a1;
            oacc[mt][4 * g + 1] = oacc[mt][4 * g + 1] * a0 + o1.y * a1;
            oacc[mt][4 * g + 2] = oacc[mt][4 * g + 2] * a0 + o1.z * a1;
            oacc[mt][4 * g + 3] = oacc[mt][4 * g + 3] * a0 + o1.w * a1;
          }
        l_run = l_run * a0 + l1 * a1;
        m_run = m_new;
      }
    }

    // ---- epilogue: combine the two half-wave partial sums, normalise, store ---
    // (pair mode: group 0 stores block A, a group 1 that moved on stores B)
    const float l_tot = halves_sum(l_run);
    const float inv = (l_tot > 0.0f) ? (1.0f / l_tot) : 0.0f;
    const int srow = g1b ? qrow_b : qrow;
    if (srow < N && (kgrp == 0 || g1b)) {
      _Float16* op = a.o + b * a.osb + hq * a.osh + (int64_t)srow * a.osn;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          half4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = E::round(oacc[mt][4 * g + e] * inv);
          *(half4*)(op + 32 * mt + 8 * g + 4 * hi) = v;
        }
      }
      if (a.lse != nullptr && hi == 0) {
        const float m_use = (m_run == -__builtin_inff()) ? 0.0f : m_run;
        const float lse2 = m_use * c2 + __builtin_log2f(l_tot);
        a.lse[(int64_t)bh * N + srow] = lse2 * 0.69314718055994530942f;
      }
    }
    if (!dynamic) break;
    // Next item: every wave is past its last LDS read of this item's tiles.
    __syncthreads();
    publish_item(prefetch && ntiles > 0, next_claim, empty_q);
    __syncthreads();
    item = __builtin_amdgcn_readfirstlane(ticket_slot[0]);
    empty_q = (unsigned)__builtin_amdgcn_readfirstlane(ticket_slot[1]);
  }
}

}  // namespace

// Launches fa_fwd_kernel<D, ...> for one workgroup shape (WAVES, KSPLIT) and
// mask mode; the causal flag and K/V stride equality pick the instance.
// The dynamic schedule (use_dynamic_schedule) needs ticket counters in
// a.ctr; they are cleared first, and the grid is one workgroup per resident
// slot.
template <int D, int WAVES, int MASK, bool KSPLIT, bool BF16>
void launch_fused(const FwdArgs& a, int batch, bool causal, Schedule schedule,
                  hipStream_t stream) {
  const bool same = a.ksn == a.vsn;
  FwdArgs args = a;
  int64_t wgs = KSPLIT && D == 64 && causal && a.pair_split != 0
                    ? plan_pairs(args, batch)
                    : plan_grid(args, batch, KSPLIT ? 128 : 32 * WAVES);
  const int64_t slots = resident_fused_workgroups();
  const bool dyn =
      WAVES == 4 && args.ctr != nullptr && use_dynamic_schedule(args, batch, causal, schedule);
  if (dyn) {
    launch_clear_tickets(args.ctr, stream);
    wgs = std::min<int64_t>(wgs, slots);
  } else {
    args.ctr = nullptr;
    // Two 4-wave workgroups per CU, all blocks resident at once: pair large
    // and small causal blocks on each CU (block_work).
    if (WAVES == 4 && !KSPLIT && causal && wgs <= slots)
      args.pair_half = (int)(slots / 2 / args.xcds);
  }
  const dim3 grid((unsigned)wgs);
  const dim3 block(64 * WAVES);
#define FA_LAUNCH(C, S, R, Y)                                                                 \
  hipLaunchKernelGGL((fa_fwd_kernel<D, C, S, WAVES, MASK, KSPLIT, BF16, R, Y>), grid, block, 0,   \
                     stream, args)
  // Paired single-round launches at head_dim 64 take the ROWSUM instance
  // (always static: pair_half is only set without counters).
  if constexpr (D == 64 && WAVES == 4 && !MASK && !KSPLIT) {
    if (causal && args.pair_half > 0) {
      if (same) FA_LAUNCH(true, true, true, false); else FA_LAUNCH(true, false, true, false);
      return;
    }
  }
  if constexpr (WAVES == 4) {
    if (dyn) {
      if (causal) {
        if (same) FA_LAUNCH(true, true, false, true); else FA_LAUNCH(true, false, false, true);
      } else {
        if (same) FA_LAUNCH(false, true, false, true); else FA_LAUNCH(false, false, false, true);
      }
      return;
    }
  }
  if (causal) {
    if (same) FA_LAUNCH(true, true, false, false); else FA_LAUNCH(true, false, false, false);
  } else {
    if (same) FA_LAUNCH(false, true, false, false); else FA_LAUNCH(false, false, false, false);
  }
#undef FA_LAUNCH
}

}  // namespace fa
