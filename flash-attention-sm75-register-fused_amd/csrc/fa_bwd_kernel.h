// Fused attention backward kernels for gfx950 (MI355X / CDNA4), included by
// the instance files fa_bwd_d{64,128}{,_mask}.hip.
//
// Gradients of O = softmax(scale * Q K^T + mask) V, given dO = dL/dO, the
// forward's O and its row log-sum-exp (no reference counterpart: the
// reference's autograd backward raises, src/flash_attention_sm75/ops.py:47-52):
//   P = exp(scale * Q K^T - LSE)            (recomputed, never stored)
//   dV = P^T dO,  dP = dO V^T,  dS = P o (dP - rowsum(dO o O)),
//   dQ = scale * dS K,  dK = scale * dS^T Q.
// P and dS are rounded to the element type before the products that take
// them, as the forward rounds P; everything else accumulates in fp32.  The
// dK/dV kernel forms dS from the rounded P its dV product takes, the dQ
// kernel from the unrounded P (both within one rounding of each other).
//
// Two kernels, all deterministic (no atomics: every gradient element is
// summed by one wave in a fixed order), dQ launched first:
//   * fa_bwd_dq_kernel: one workgroup per (batch, query head, 128 rows), the
//     forward's shape: Q and dO rows resident, K and V tiles streamed through
//     double-buffered LDS; two workgroups per CU.  It also forms each row's
//     lse * log2(e) and -rowsum(dO o O) and writes them to the workspace in
//     64-row records (one direct load per tile for the next kernel).
//   * fa_bwd_dkdv_kernel: one workgroup of 8 waves per (batch, KV head, 128
//     keys); waves w and w+4 own keys k0 + 32w .. +32 and split the four
//     products (w: S, P, dV with the K rows resident; w+4: dP, dS, dK with
//     the V rows resident, P handed over through LDS).  It streams 64-row
//     tiles of Q and dO (and their stats and mask words) through triple-
//     buffered LDS for every query head of the group, so the GQA sum over
//     the group happens in the accumulators; one workgroup per CU, two waves
//     per SIMD.
// An explicit boolean mask (MASK instances) hides keys on top of the causal
// rule; rows that see no key have lse = -inf, so their P is 0.
// Tiles use the forward's LDS layout (Lds<D>: padded rows, 16-byte chunks
// XOR-swizzled), on which both operand reads below are conflict-free.
//
// MFMA layouts (v_mfma_f32_32x32x16, as in fa_fwd_kernel.h):
//   A[m][k]: lane l holds m = l%32, k = 8*(l/32) + j
//   B[k][n]: lane l holds n = l%32, k = 8*(l/32) + j
//   C[m][n]: lane l holds n = l%32, m = 8*(i/4) + 4*(l/32) + i%4
// dK/dV kernel: S = Q K^T and dP = dO V^T with queries on M and keys on N,
// so each lane owns one key; dV^T += dO^T P and dK^T += Q^T dS take P and dS
// straight from those accumulators as B operands (16-query steps in the row
// order C hands over), with dO^T and Q^T read transposed out of the tiles.
// dQ kernel: S^T = K Q^T and dP^T = V dO^T (lane = query, so LSE and the
// row sum are per-lane scalars), dQ^T += K^T dS^T.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa_internal.h"

#include "fa_kernel_common.h"

namespace fa {
namespace {

// Per-lane LDS addressing in one Lds<D> tile (64 rows):
//   row(t, kk): the 8 columns 16kk + 8(l/32) .. +8 of row 32t + l%32 (an A
//               or B operand whose m or n index is the tile row);
//   tr(ks, mt): the A operand X^T of the row-major tile X: column 32mt + l%32
//               of rows 16ks + {4(l/32) + 0..3, 8 + 4(l/32) + 0..3}, the
//               order in which an accumulator's 16 rows arrive as B (two
//               transposing ds_read_b64_tr_b16, 16 lanes = 4 rows x 16 columns).
template <int D>
struct TileReader {
  using L = Lds<D>;
  int row_even, row_odd, tr0, tr1;
  __device__ __forceinline__ explicit TileReader(int lane) {
    const int hi = lane >> 5, ql = lane & 31, grp = lane >> 4, gi = lane & 15;
    const int s = (ql >> 2) & 3;
    row_even = ql * L::Pitch + 8 * (hi ^ s);
    row_odd = ql * L::Pitch + 8 * ((2 + hi) ^ s);
    const int r = 4 * hi + (gi >> 2);
    const int c = 2 * (grp & 1) + ((gi & 3) >> 1);
    tr0 = r * L::Pitch + 8 * (c ^ hi) + 4 * (gi & 1);
    tr1 = (r + 8) * L::Pitch + 8 * (c ^ (hi + 2)) + 4 * (gi & 1);
  }
  __device__ __forceinline__ half8 row(const _Float16* tile, int t, int kk) const {
    const int off = ((kk & 1) ? row_odd : row_even) + 32 * t * L::Pitch + 32 * (kk >> 1);
    return *(const half8*)(tile + off);
  }
  __device__ __forceinline__ half8 tr(const _Float16* tile, int ks, int mt) const {
    const int imm = 16 * ks * L::Pitch + 32 * mt;
    const half4 lo = ds_read_tr16(tile + tr0 + imm);
    const half4 hi4 = ds_read_tr16(tile + tr1 + imm);
    return __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
  }
};

// Global byte offset of lane `lane`'s 16 bytes in 1 KB segment `seg` of an
// Lds<D> tile whose source rows are `stride` elements apart; -16 (past any
// buffer window, so the lane writes zeros) for bytes in the row padding.
template <int D>
__device__ __forceinline__ int seg_offset(int seg, int lane, int64_t stride) {
  using L = Lds<D>;
  const int pos = seg * 1024 + 16 * lane;
  const int row = pos / (2 * L::Pitch);
  const int within = pos - row * (2 * L::Pitch);
  if (within >= 2 * D) return -16;
  const int c = (within >> 4) ^ ((row >> 2) & 3);
  return (int)(row * stride * 2) + 16 * c;
}

// P or dS values of accumulator elements i, i+1 of 32-row sub-tile t as one
// packed 32-bit lane of the B operand of 16-row step 2t + (i >> 3).
template <class E, int NOPS>
__device__ __forceinline__ void put_pair(uint4v (&ops)[NOPS], int t, int i, float x, float y) {
  ops[2 * t + (i >> 3)][(i & 7) >> 1] = __builtin_bit_cast(unsigned, E::pack(x, y));
}

typedef float float4v __attribute__((ext_vector_type(4)));

// 4-byte direct load of one lane (lane l writes dst + 4 l).
__device__ __forceinline__ void direct_load4(__amdgpu_buffer_rsrc_t r, lds_void* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 4, voff, 0, 0, 0);
}

// ---- dK, dV with two waves per key group -----------------------------------
// One workgroup of 8 waves per (batch, KV head, 128 keys).  Waves w and w+4
// (w = 0..3) own keys k0 + 32w .. +32, one key per lane, and run on the same
// SIMD; they split each step's four products by role:
//   * P-wave (w): S = Q K^T, P = exp2(S c2 - lse2), dV^T += dO^T P;
//   * dS-wave (w+4): dP = dO V^T, dS = P o (dP - delta), dK^T += Q^T dS,
// taking P from the P-wave through LDS (the 16-bit values its dV product
// uses, 2 KB per 32-query sub-tile).  Each wave then holds one resident
// operand (K or V rows) and one accumulator (dV or dK): at most 256 registers,
// so two waves share each SIMD and cover each other's latencies, and every
// MFMA accumulates in VGPRs.
// Periods: in period p the P-waves work on step p and the dS-waves on step
// p - 1, whose P was written in period p - 1 (exchange buffers alternate by
// step parity).  Q/dO tiles (and their stats and mask words) are triple
// buffered: period p reads stages p and p - 1 and loads step p + 1 into the
// third; one barrier ends each period.
template <int D, bool CAUSAL, bool MASK, bool BF16>
__global__ void __launch_bounds__(512, 1) fa_bwd_dkdv_kernel(const BwdArgs a) {
  using L = Lds<D>;
  using E = Elem<BF16>;
  constexpr int KK = D / 16;
  constexpr int MT = D / 32;
  constexpr int SEGQ = L::Segs / 4;
  constexpr int PFR = 3;  // row-operand reads run this many MFMAs ahead
  constexpr int PFT = 3;  // transposing reads run this many MFMAs ahead
  __shared__ __attribute__((aligned(1024))) _Float16 q_lds0[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 q_lds1[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 q_lds2[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 d_lds0[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 d_lds1[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 d_lds2[L::Tile];
  __shared__ __attribute__((aligned(1024))) float s_lds0[256];
  __shared__ __attribute__((aligned(1024))) float s_lds1[256];
  __shared__ __attribute__((aligned(1024))) float s_lds2[256];
  __shared__ __attribute__((aligned(1024))) uint32_t m_lds0[MASK ? 256 : 1];
  __shared__ __attribute__((aligned(1024))) uint32_t m_lds1[MASK ? 256 : 1];
  __shared__ __attribute__((aligned(1024))) uint32_t m_lds2[MASK ? 256 : 1];
  // P exchange: [step parity][key group][sub-tile][16-query half][lane].
  __shared__ __attribute__((aligned(1024))) uint4v x_lds[2 * 4 * 2 * 2 * 64];

  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int role = wave >> 2;  // 0: P-wave, 1: dS-wave
  const int kq = wave & 3;     // key group
  const int lane = (int)threadIdx.x & 63;
  const int hi = lane >> 5, ql = lane & 31;

  // Work item: XCD x takes the units (b, hkv) [x U/8, (x+1) U/8) when
  // a.xcds == 8, key blocks in rank order (causal: block 0, which sees the
  // most queries, first).
  const int wg = (int)blockIdx.x;
  const int x = wg % a.xcds, p = wg / a.xcds;
  const int per = a.units / a.xcds;
  const int kb = p / per;
  const int u = x * per + (p - kb * per);
  const int hkv_count = a.hq / a.group;
  const int b = u / hkv_count, hkv = u - b * hkv_count;
  const int k0 = kb * kBwdBlockKeys;
  const int kw = k0 + 32 * kq;  // this wave's first key
  const int krow = kw + ql;     // this lane's key
  const int N = a.n, NK = a.nk;

  // The wave's resident B operand: K rows (P-wave) or V rows (dS-wave) of
  // the lane's key (n = key, k = dims).
  half8 of[KK];
  if (krow < NK) {
    const _Float16* src = role == 0
        ? a.k + b * a.ksb + hkv * a.ksh + (int64_t)krow * a.ksn + 8 * hi
        : a.v + b * a.vsb + hkv * a.vsh + (int64_t)krow * a.vsn + 8 * hi;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) of[kk] = *(const half8*)(src + 16 * kk);
  } else {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) of[kk] = (half8)(_Float16)0;
  }
  float16v acc[MT];  // dV^T (P-wave) or dK^T (dS-wave): m = dims, n = key
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = (float16v)0.0f;

  // Mask ranges (a.mranges): the query tiles whose span of visible keys
  // (the union of their rows' spans, a.tspans, which the dQ kernel wrote)
  // meets this block's keys [k0, k0 + 128), over the group's heads when the
  // mask has a head dimension; the other tiles have no row that sees a key
  // of the block, so skipping them changes no result (a tile kept because
  // only its union meets the block adds exact zeros).  Each thread scans a
  // share of the tiles, the wave and then the workgroup (through the P
  // exchange buffers, idle until the first period) take the union.
  int qt_lo = 0, qt_hi = a.qtiles;
  if constexpr (MASK) {
    if (a.mranges != nullptr) {
      int lo = a.qtiles, hi = 0;
      const int heads = a.mrsh != 0 ? a.group : 1;
      for (int e = (int)threadIdx.x; e < heads * a.qtiles; e += 512) {
        const int h = e / a.qtiles, qt = e - h * a.qtiles;
        const int32_t* ts =
            a.tspans + 2 * ((int64_t)(b * a.hq + hkv * a.group + h) * a.qtiles + qt);
        if (ts[0] < k0 + kBwdBlockKeys && ts[1] > k0) {
          lo = min(lo, qt);
          hi = max(hi, qt + 1);
        }
      }
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        lo = min(lo, __shfl_xor(lo, d));
        hi = max(hi, __shfl_xor(hi, d));
      }
      int* const xs = (int*)x_lds;
      if (lane == 0) {
        xs[2 * wave] = lo;
        xs[2 * wave + 1] = hi;
      }
      __syncthreads();
#pragma unroll
      for (int w2 = 0; w2 < 8; ++w2) {
        lo = min(lo, xs[2 * w2]);
        hi = max(hi, xs[2 * w2 + 1]);
      }
      __syncthreads();  // every wave has read the exchange before it is reused
      lo = __builtin_amdgcn_readfirstlane(lo);
      hi = __builtin_amdgcn_readfirstlane(hi);
      qt_lo = hi > lo ? lo : 0;
      qt_hi = hi > lo ? hi : 0;
    }
  }
  const int qt_begin =
      max(qt_lo, CAUSAL ? min(a.qtiles, max(0, k0 - a.diag) / kBwdStatsTile) : 0);
  const int qt_end = min(a.qtiles, qt_hi);
  const int per_head = max(0, qt_end - qt_begin);
  const int steps = a.group * per_head;

  // P-waves load the Q tile, dS-waves the dO tile (segments kq, kq+4, ..).
  int goff[SEGQ];
#pragma unroll
  for (int s = 0; s < SEGQ; ++s) goff[s] = seg_offset<D>(kq + 4 * s, lane, role == 0 ? a.qsn : a.dosn);
  auto qbuf = [&](auto st) -> _Float16* {
    constexpr int S = decltype(st)::value % 3;
    if constexpr (S == 0) return q_lds0;
    else if constexpr (S == 1) return q_lds1;
    else return q_lds2;
  };
  auto dbuf = [&](auto st) -> _Float16* {
    constexpr int S = decltype(st)::value % 3;
    if constexpr (S == 0) return d_lds0;
    else if constexpr (S == 1) return d_lds1;
    else return d_lds2;
  };
  auto sbuf = [&](auto st) -> float* {
    constexpr int S = decltype(st)::value % 3;
    if constexpr (S == 0) return s_lds0;
    else if constexpr (S == 1) return s_lds1;
    else return s_lds2;
  };
  auto mbuf = [&](auto st) -> uint32_t* {
    constexpr int S = decltype(st)::value % 3;
    if constexpr (S == 0) return m_lds0;
    else if constexpr (S == 1) return m_lds1;
    else return m_lds2;
  };
  // Steps go through the query tiles in descending order, every head of the
  // group at each tile: a cursor (qt, h) names query tile qt of query head
  // hkv * group + h.
  struct Cursor {
    int qt, h;
  };
  auto advance = [&](Cursor& c) {
    if (++c.h == a.group) {
      c.h = 0;
      --c.qt;
    }
  };
  auto issue = [&](const Cursor& c, auto st) {
    const int qt = c.qt;
    const int hq = hkv * a.group + c.h;
    const int q0 = qt * kBwdStatsTile;
    const int rows = N - q0;
    const __amdgpu_buffer_rsrc_t r = role == 0
        ? make_rsrc(a.q + b * a.qsb + hq * a.qsh + (int64_t)q0 * a.qsn, (int)(rows * a.qsn * 2))
        : make_rsrc(a.dout + b * a.dosb + hq * a.dosh + (int64_t)q0 * a.dosn,
                    (int)(rows * a.dosn * 2));
    _Float16* const dst = role == 0 ? qbuf(st) : dbuf(st);
#pragma unroll
    for (int s2 = 0; s2 < SEGQ; ++s2)
      direct_load16(r, (lds_void*)(dst + (kq + 4 * s2) * 512), goff[s2]);
    if (wave == 0) {
      const __amdgpu_buffer_rsrc_t rs = make_rsrc(
          a.stats + ((int64_t)(b * a.hq + hq) * a.qtiles + qt) * (2 * kBwdStatsTile),
          2 * kBwdStatsTile * 4);
      direct_load16(rs, (lds_void*)sbuf(st), 16 * lane);
    }
    if constexpr (MASK) {
      if (role == 0) {
        // Lane l: row q0 + l, 32-bit word 2 (k0 / 64) + kq of it; the window
        // ends after the last row's words (rows past it and words past the
        // keys read as 0).  Offsets of rows below N fit 32 bits (the C ABI
        // checks N * row stride); a lane past N whose offset wraps reads 0 or
        // some mask word inside the window, for a row that is never used.
        const uint64_t* mrow = a.mbits + b * a.msb + hq * a.msh + (int64_t)q0 * a.msq;
        const __amdgpu_buffer_rsrc_t rm =
            make_rsrc(mrow, (int)((((int64_t)rows - 1) * a.msq + a.mwords) * 8));
        direct_load4(rm, (lds_void*)(mbuf(st) + 64 * kq),
                     (int)(lane * a.msq * 8) + (k0 / 64) * 8 + 4 * kq);
      }
    }
  };

  const TileReader<D> rd(lane);
  const float c2 = a.c2 != 0.0f ? a.c2 : 1e-30f;
  const float mval = c2 > 0.0f ? -__builtin_inff() : __builtin_inff();
  // Scores of sub-tile t (element i: query q0 + 32t + 8(i/4) + 4hi + i%4)
  // whose key is past the query's causal diagonal or hidden by the mask -> mval.
  auto mask_scores = [&](float16v sv, int q0, int t, auto st) __attribute__((always_inline)) -> float16v {
    if constexpr (CAUSAL) {
      const int qs = q0 + 32 * t;
      if (kw + 31 > qs + a.diag) {
        static_for<16>([&](auto i_c) {
          constexpr int i = decltype(i_c)::value;
          if (krow > qs + 8 * (i >> 2) + 4 * hi + (i & 3) + a.diag) sv[i] = mval;
        });
      }
    }
    if constexpr (MASK) {
      const uint32_t* mw = mbuf(st) + 64 * kq + 32 * t + 4 * hi;
      static_for<4>([&](auto g_c) {
        constexpr int g = decltype(g_c)::value;
        const uint4v m4 = *(const uint4v*)(mw + 8 * g);
        static_for<4>([&](auto e_c) {
          constexpr int e = decltype(e_c)::value;
          if (((m4[e] >> ql) & 1u) == 0) sv[4 * g + e] = mval;
        });
      });
    }
    return sv;
  };
  auto xslot = [&](int par, int t, int h) -> uint4v* {
    return x_lds + (((par * 4 + kq) * 2 + t) * 2 + h) * 64 + lane;
  };

  // Slots of one step, for either role: S (or dP) of sub-tile 0 in slots
  // [0, KK), of sub-tile 1 in [KK, 2KK), then dV (or dK) of sub-tile 0 in
  // [2KK, 2KK + 2MT) and of sub-tile 1 after.  The element work of sub-tile
  // t (P, or dS) sits in the slots of the products before its consumer:
  // sub-tile 0 in [KK, 2KK), sub-tile 1 in [2KK, 2KK + 2MT).
  constexpr int NS = 2 * KK;
  constexpr int NG = 2 * MT;
  constexpr int NSLOT = NS + 2 * NG;
  // pair pr (0..7) of sub-tile t goes to this slot.
  constexpr auto pair_slot = [](int t, int pr) constexpr {
    return t == 0 ? KK + (pr * KK) / 8 : NS + (pr * NG) / 8;
  };

  // P-wave, step s on stage ST, exchange parity par.
  auto work_p = [&](const Cursor& c, auto st, int par) {
    const _Float16* qc = qbuf(st);
    const _Float16* dc = dbuf(st);
    const float* sc = sbuf(st);
    const int q0 = c.qt * kBwdStatsTile;
    float16v sv[2];
    float4v l4[2][4];
    uint4v pp[2][2];
    half8 rf[NS], tf[NG * 2];
    auto read_row = [&](int i) -> half8 { return rd.row(qc, i / KK, i % KK); };
    // Transposed operand v of the dV products: sub-tile v / NG, 16-query step
    // (v % NG) / MT, output tile v % MT.
    auto read_tr = [&](int v) -> half8 {
      const int t = v / NG, w = v % NG;
      return rd.tr(dc, 2 * t + w / MT, w % MT);
    };
    auto pair = [&](int t, int pr) {
      const int i = 2 * pr, g = i >> 2, e = i & 3;
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[t][i], c2, -l4[t][g][e]));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[t][i + 1], c2, -l4[t][g][e + 1]));
      unsigned w = __builtin_bit_cast(unsigned, E::pack(p0, p1));
      asm volatile("" : "+v"(w));  // keeps the pair in its slot (not sunk to its use)
      pp[t][i >> 3][(i & 7) >> 1] = w;
    };
    static_for<4>([&](auto g_c) {
      constexpr int g = decltype(g_c)::value;
      l4[0][g] = *(const float4v*)(sc + 8 * g + 4 * hi);
    });
    static_for<PFR>([&](auto i_c) { rf[decltype(i_c)::value] = read_row(decltype(i_c)::value); });
    static_for<NSLOT>([&](auto slot_c) {
      constexpr int slot = decltype(slot_c)::value;
      if constexpr (slot == NS - PFT) {
        static_for<PFT>([&](auto v_c) { tf[decltype(v_c)::value] = read_tr(decltype(v_c)::value); });
      }
      if constexpr (slot >= NS && slot - NS + PFT < 2 * NG) tf[slot - NS + PFT] = read_tr(slot - NS + PFT);
      if constexpr (slot < NS) {
        constexpr int t = slot / KK, kk = slot % KK;
        if constexpr (slot + PFR < NS) rf[slot + PFR] = read_row(slot + PFR);
        sv[t] = E::mfma(rf[slot], of[kk], kk == 0 ? (float16v)0.0f : sv[t]);
      } else {
        constexpr int v = slot - NS, t = v / NG, w = v % NG, h2 = w / MT, mt = w % MT;
        acc[mt] = E::mfma(tf[v], __builtin_bit_cast(half8, pp[t][h2]), acc[mt]);
      }
      fence_schedule();  // the slot's MFMA issues before its element work
      if constexpr (slot == KK) {
        static_for<4>([&](auto g_c) {
          constexpr int g = decltype(g_c)::value;
          l4[1][g] = *(const float4v*)(sc + 32 + 8 * g + 4 * hi);
        });
        sv[0] = mask_scores(sv[0], q0, 0, st);
      }
      if constexpr (slot == NS) sv[1] = mask_scores(sv[1], q0, 1, st);
      static_for<8>([&](auto p_c) {
        constexpr int pr = decltype(p_c)::value;
        if constexpr (pair_slot(0, pr) == slot) pair(0, pr);
        if constexpr (pair_slot(1, pr) == slot) pair(1, pr);
      });
      if constexpr (slot == NS) {
        *xslot(par, 0, 0) = pp[0][0];
        *xslot(par, 0, 1) = pp[0][1];
      }
      if constexpr (slot == NS + NG) {
        *xslot(par, 1, 0) = pp[1][0];
        *xslot(par, 1, 1) = pp[1][1];
      }
      fence_schedule();
    });
  };

  // dS-wave, one step on stage ST with exchange parity par.  The dP products
  // accumulate onto -delta (the stats record holds -rowsum(dO o O)), so
  // dS = P (dP - delta) is one multiply per element.
  auto work_ds = [&](auto st, int par) {
    const _Float16* qc = qbuf(st);
    const _Float16* dc = dbuf(st);
    const float* sc = sbuf(st);
    float16v dp[2];
    float16v nd[2];
    uint4v pr2[2][2], pd[2][2];
    half8 rf[NS], tf[NG * 2];
    auto read_row = [&](int i) -> half8 { return rd.row(dc, i / KK, i % KK); };
    auto read_tr = [&](int v) -> half8 {
      const int t = v / NG, w = v % NG;
      return rd.tr(qc, 2 * t + w / MT, w % MT);
    };
    auto read_nd = [&](int t) {
      static_for<4>([&](auto g_c) {
        constexpr int g = decltype(g_c)::value;
        const float4v v = *(const float4v*)(sc + kBwdStatsTile + 32 * t + 8 * g + 4 * hi);
        nd[t][4 * g + 0] = v[0];
        nd[t][4 * g + 1] = v[1];
        nd[t][4 * g + 2] = v[2];
        nd[t][4 * g + 3] = v[3];
      });
    };
    auto pair = [&](int t, int pr) {
      const int i = 2 * pr;
      const unsigned w = pr2[t][i >> 3][(i & 7) >> 1];
      unsigned w2 = __builtin_bit_cast(unsigned, E::pack(E::mul_lo(w, dp[t][i]), E::mul_hi(w, dp[t][i + 1])));
      asm volatile("" : "+v"(w2));  // keeps the pair in its slot
      pd[t][i >> 3][(i & 7) >> 1] = w2;
    };
    read_nd(0);
    static_for<PFR>([&](auto i_c) { rf[decltype(i_c)::value] = read_row(decltype(i_c)::value); });
    static_for<NSLOT>([&](auto slot_c) {
      constexpr int slot = decltype(slot_c)::value;
      if constexpr (slot == NS - PFT) {
        static_for<PFT>([&](auto v_c) { tf[decltype(v_c)::value] = read_tr(decltype(v_c)::value); });
      }
      if constexpr (slot >= NS && slot - NS + PFT < 2 * NG) tf[slot - NS + PFT] = read_tr(slot - NS + PFT);
      if constexpr (slot < NS) {
        constexpr int t = slot / KK, kk = slot % KK;
        if constexpr (slot + PFR < NS) rf[slot + PFR] = read_row(slot + PFR);
        dp[t] = E::mfma(rf[slot], of[kk], kk == 0 ? nd[t] : dp[t]);
      } else {
        constexpr int v = slot - NS, t = v / NG, w = v % NG, h2 = w / MT, mt = w % MT;
        acc[mt] = E::mfma(tf[v], __builtin_bit_cast(half8, pd[t][h2]), acc[mt]);
      }
      fence_schedule();
      if constexpr (slot == 1) {
        pr2[0][0] = *xslot(par, 0, 0);
        pr2[0][1] = *xslot(par, 0, 1);
      }
      if constexpr (slot == 2) read_nd(1);
      if constexpr (slot == KK) {
        pr2[1][0] = *xslot(par, 1, 0);
        pr2[1][1] = *xslot(par, 1, 1);
      }
      static_for<8>([&](auto p_c) {
        constexpr int pr = decltype(p_c)::value;
        if constexpr (pair_slot(0, pr) == slot) pair(0, pr);
        if constexpr (pair_slot(1, pr) == slot) pair(1, pr);
      });
      fence_schedule();
    });
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  // Period p loads step p + 1 into stage (p + 1) % 3 and ends with the barrier
  // that publishes it (and the P of step p); the roles run separate loops
  // with the same number of barriers.
  if (steps > 0) {
    Cursor ic{qt_end - 1, 0};  // next step to load
    Cursor wc{qt_end - 1, 0};  // step to work on
    issue(ic, I0{});
    advance(ic);
    barrier_after_loads<0>();
    if (role == 0) {
      // Period p: step p.  Unrolled by three (the stage is p % 3).
      auto body = [&](int p, auto st_c) {
        constexpr int ST = decltype(st_c)::value;
        if (p + 1 < steps) {
          issue(ic, std::integral_constant<int, ST + 1>{});
          advance(ic);
        }
        work_p(wc, st_c, p & 1);
        advance(wc);
        barrier_after_loads<0>();
      };
      int p = 0;
      for (; p + 3 <= steps; p += 3) {
        body(p, I0{});
        body(p + 1, I1{});
        body(p + 2, I2{});
      }
      if (p < steps) body(p, I0{});
      if (p + 1 < steps) body(p + 1, I1{});
    } else {
      // Period p: step p - 1 (stage (p - 1) % 3); period `steps` has no
      // barrier after it.  Unrolled by three from period 1.
      if (1 < steps) {
        issue(ic, I1{});
        advance(ic);
      }
      barrier_after_loads<0>();
      auto body = [&](int p, auto st_c) {
        constexpr int ST = decltype(st_c)::value;
        if (p + 1 < steps) {
          issue(ic, std::integral_constant<int, ST + 2>{});
          advance(ic);
        }
        work_ds(st_c, (p - 1) & 1);
        if (p < steps) barrier_after_loads<0>();
      };
      int p = 1;
      for (; p + 2 <= steps; p += 3) {
        body(p, I0{});
        body(p + 1, I1{});
        body(p + 2, I2{});
      }
      if (p <= steps) body(p, I0{});
      if (p + 1 <= steps) body(p + 1, I1{});
    }
  }

  if (krow < NK) {
    _Float16* dst = role == 0 ? a.dv + b * a.dvsb + hkv * a.dvsh + (int64_t)krow * a.dvsn
                              : a.dk + b * a.dksb + hkv * a.dksh + (int64_t)krow * a.dksn;
    const float f = role == 0 ? 1.0f : a.scale;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        half4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = E::round(acc[mt][4 * g + e] * f);
        *(half4*)(dst + 32 * mt + 8 * g + 4 * hi) = v;
      }
    }
  }
}

// ---- dQ ----------------------------------------------------------------------
// The forward's work decomposition (block_work; causal: largest block
// first): wave w owns query rows q0 + 32w .. +32 and walks the 64-key tiles
// its block can see, K and V tiles double buffered through LDS.  Two
// workgroups per CU (at most 256 VGPRs, 80 KiB of LDS each): measured 26%
// faster than one on the C4 training shape; with a mask at head_dim 128 one
// (its mask words do not fit those registers).  The tiles no row of the
// block masks run in a loop of their own, free of mask code.
template <int D, bool CAUSAL, bool MASK, bool BF16>
__global__ void __launch_bounds__(256, MASK && D == 128 ? 1 : 2) fa_bwd_dq_kernel(const BwdArgs a) {
  using L = Lds<D>;
  using E = Elem<BF16>;
  constexpr int KK = D / 16;
  constexpr int MT = D / 32;
  constexpr int SEGQ = L::Segs / 4;
  __shared__ __attribute__((aligned(1024))) _Float16 k_lds0[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 k_lds1[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 v_lds0[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 v_lds1[L::Tile];

  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = (int)threadIdx.x & 63;
  const int hi = lane >> 5, ql = lane & 31;
  const Work w = block_work(a, (int)blockIdx.x, CAUSAL);
  const int b = w.b, hq = w.hq, hkv = w.hkv;
  const int bh = b * a.hq + hq;
  const int q0 = w.qb * kBwdBlockRows;
  const int qw = q0 + 32 * wave;
  const int qrow = qw + ql;
  const int N = a.n, NK = a.nk;

  // Q and dO rows of the lane's query as B operands (n = query, k = dims),
  // and the row's statistics: lse2 = lse * log2(e) (+inf for a row that sees
  // no key) and ndelta = -rowsum(dO o O), each half-wave summing the dims
  // it holds (O is read once, here).
  half8 qf[KK], df[KK];
  float lse2 = __builtin_inff(), dot = 0.0f;
  if (qrow < N) {
    const _Float16* qp = a.q + b * a.qsb + hq * a.qsh + (int64_t)qrow * a.qsn + 8 * hi;
    const _Float16* dp = a.dout + b * a.dosb + hq * a.dosh + (int64_t)qrow * a.dosn + 8 * hi;
    const _Float16* op = a.o + b * a.osb + hq * a.osh + (int64_t)qrow * a.osn + 8 * hi;
    half8 of[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      qf[kk] = *(const half8*)(qp + 16 * kk);
      df[kk] = *(const half8*)(dp + 16 * kk);
      of[kk] = __builtin_nontemporal_load((const half8*)(op + 16 * kk));
    }
    const float l = a.lse[(int64_t)bh * N + qrow];
    lse2 = (l == -__builtin_inff()) ? __builtin_inff() : l * 1.4426950408889634f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        dot = __builtin_fmaf(E::to_f32(of[kk][e]), E::to_f32(df[kk][e]), dot);
    }
  } else {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qf[kk] = df[kk] = (half8)(_Float16)0;
  }
  dot += __shfl_xor(dot, 32);
  const float ndelta = qrow < N ? -dot : 0.0f;
  // The dK/dV kernel, launched after this one, reads them from the workspace:
  // one record per (b, query head, 64-row tile), rows past N as (+inf, 0).
  if (hi == 0 && qrow / kBwdStatsTile < a.qtiles) {
    float* const st =
        a.stats + ((int64_t)bh * a.qtiles + qrow / kBwdStatsTile) * (2 * kBwdStatsTile);
    st[qrow % kBwdStatsTile] = lse2;
    st[kBwdStatsTile + qrow % kBwdStatsTile] = ndelta;
  }
  float16v dq[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) dq[mt] = (float16v)0.0f;

  // dP accumulates onto -delta (every element of a lane is the lane's query).
  const float16v ndv = (float16v)ndelta;
  // Mask ranges (a.mranges): the span of keys some row of the block sees;
  // the tiles outside it hide every key from every row (as in the forward).
  int span_lo = 0, span_hi = NK;
  if constexpr (MASK) {
    if (a.mranges != nullptr) {
      const int32_t* rr =
          a.mranges + 2 * (b * a.mrsb + hq * a.mrsh + (int64_t)min(qrow, N - 1) * a.mrsq);
      span_lo = range_first_key(rr[0]);
      span_hi = rr[1];
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        span_lo = min(span_lo, __shfl_xor(span_lo, d));
        span_hi = max(span_hi, __shfl_xor(span_hi, d));
      }
      int* const xs = (int*)k_lds1;
      if (lane == 0) {
        xs[2 * wave] = span_lo;
        xs[2 * wave + 1] = span_hi;
      }
      __syncthreads();
      // The span of each 64-row query tile of the block (waves 2t and 2t+1)
      // for the dK/dV kernel, which runs after this one (rows past N carry
      // row N - 1's pair: a superset, which skips less and changes nothing).
      if ((wave & 1) == 0 && lane == 0) {
        const int qt = (q0 + 32 * wave) / kBwdStatsTile;
        if (qt < a.qtiles) {
          int32_t* const ts = a.tspans + 2 * ((int64_t)bh * a.qtiles + qt);
          ts[0] = min(xs[2 * wave], xs[2 * wave + 2]);
          ts[1] = max(xs[2 * wave + 1], xs[2 * wave + 3]);
        }
      }
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) {
        span_lo = min(span_lo, xs[2 * w2]);
        span_hi = max(span_hi, xs[2 * w2 + 1]);
      }
      __syncthreads();  // every wave has read the exchange before a tile lands there
      span_lo = __builtin_amdgcn_readfirstlane(span_lo);
      span_hi = __builtin_amdgcn_readfirstlane(span_hi);
    }
  }
  const int kv_len = min(CAUSAL ? max(0, min(NK, q0 + kBwdBlockRows + a.diag)) : NK, span_hi);
  const int ntiles = (kv_len + kBlockN - 1) / kBlockN;
  const int j_begin = span_lo < span_hi ? min(span_lo / kBlockN, ntiles) : ntiles;
  // MASK: the lane's mask row (rows past N read row N - 1; not stored).
  const uint64_t* mrow =
      MASK ? a.mbits + b * a.msb + hq * a.msh + (int64_t)min(qrow, N - 1) * a.msq : nullptr;

  int goff_k[SEGQ], goff_v[SEGQ];
#pragma unroll
  for (int s = 0; s < SEGQ; ++s) {
    goff_k[s] = seg_offset<D>(wave + 4 * s, lane, a.ksn);
    goff_v[s] = seg_offset<D>(wave + 4 * s, lane, a.vsn);
  }
  const _Float16* Kp = a.k + b * a.ksb + hkv * a.ksh;
  const _Float16* Vp = a.v + b * a.vsb + hkv * a.vsh;
  auto issue = [&](int j, _Float16* kdst, _Float16* vdst) {
    const int rows = NK - j * kBlockN;
    const __amdgpu_buffer_rsrc_t rk =
        make_rsrc(Kp + (int64_t)j * kBlockN * a.ksn, (int)(rows * a.ksn * 2));
    const __amdgpu_buffer_rsrc_t rv =
        make_rsrc(Vp + (int64_t)j * kBlockN * a.vsn, (int)(rows * a.vsn * 2));
#pragma unroll
    for (int s2 = 0; s2 < SEGQ; ++s2) {
      direct_load16(rk, (lds_void*)(kdst + (wave + 4 * s2) * 512), goff_k[s2]);
      direct_load16(rv, (lds_void*)(vdst + (wave + 4 * s2) * 512), goff_v[s2]);
    }
  };

  const TileReader<D> rd(lane);
  const float c2 = a.c2;

  // One key tile j on buffer parity PAR.  MASKED: the tile may need the
  // per-element mask (tested per pair, on this wave's need_mask); the
  // unmasked tiles run without any mask code, so the compiler interleaves
  // their exps with the MFMAs (a branch per pair splits the tile into blocks).
  auto step = [&](int j, auto par_t, auto masked_t) {
    constexpr int PAR = decltype(par_t)::value;
    constexpr bool MASKED = decltype(masked_t)::value;
    const _Float16* kc = PAR ? k_lds1 : k_lds0;
    const _Float16* vc = PAR ? v_lds1 : v_lds0;
    if (j + 1 < ntiles) issue(j + 1, PAR ? k_lds0 : k_lds1, PAR ? v_lds0 : v_lds1);
    const int kstart = j * kBlockN;
    // MASK: bit k of mw = key kstart + k visible to this lane's query.
    const uint64_t mw = MASK ? mrow[j] : ~0ull;
    bool need_mask = kstart + kBlockN > NK || (CAUSAL && kstart + kBlockN - 1 > qw + a.diag);
    if (MASK) need_mask = need_mask || __builtin_amdgcn_ballot_w64(~mw != 0) != 0;
    uint4v pd[4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float16v sa = (float16v)0.0f, dpa = ndv;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) sa = E::mfma(rd.row(kc, t, kk), qf[kk], sa);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) dpa = E::mfma(rd.row(vc, t, kk), df[kk], dpa);
      // Element i: key kstart + 32t + 8(i/4) + 4hi + i%4, query qrow.
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sa[i], c2, -lse2));
        float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sa[i + 1], c2, -lse2));
        if (MASKED && need_mask) {
          const int kt = 32 * t + 8 * (i >> 2) + 4 * hi + (i & 3);  // key within the tile
          const int key = kstart + kt;
          if (key >= NK || (CAUSAL && key > qrow + a.diag) || ((mw >> kt) & 1) == 0) p0 = 0.0f;
          if (key + 1 >= NK || (CAUSAL && key + 1 > qrow + a.diag) || ((mw >> (kt + 1)) & 1) == 0)
            p1 = 0.0f;
        }
        put_pair<E>(pd, t, i, p0 * dpa[i], p1 * dpa[i + 1]);
      }
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        dq[mt] = E::mfma(rd.tr(kc, ks, mt), __builtin_bit_cast(half8, pd[ks]), dq[mt]);
    }
    barrier_after_loads<0>();
  };

  // Tiles [0, j_split) need no mask for any wave of the workgroup (wave 0,
  // whose rows come first, is the first to meet its diagonal; every tile
  // lies inside the keys); the rest run the masked step.  With a boolean mask
  // any tile may need it.
  int j_split = 0;
  if (!MASK) {
    j_split = min(ntiles, NK / kBlockN);
    if (CAUSAL) j_split = min(j_split, max(0, q0 + a.diag + 1) / kBlockN);
  }
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  // Tile j sits in the buffers of parity j & 1.
  if (ntiles > j_begin)
    issue(j_begin, (j_begin & 1) ? k_lds1 : k_lds0, (j_begin & 1) ? v_lds1 : v_lds0);
  barrier_after_loads<0>();
  int j = j_begin;
  for (; j + 1 < j_split; j += 2) {
    step(j, P0{}, Flag<false>{});
    step(j + 1, P1{}, Flag<false>{});
  }
  if (j < j_split) step(j++, P0{}, Flag<false>{});
  for (; j < ntiles; ++j) {
    if (j & 1) step(j, P1{}, Flag<true>{});
    else step(j, P0{}, Flag<true>{});
  }

  if (qrow < N) {
    _Float16* op = a.dq + b * a.dqsb + hq * a.dqsh + (int64_t)qrow * a.dqsn;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        half4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = E::round(dq[mt][4 * g + e] * a.scale);
        *(half4*)(op + 32 * mt + 8 * g + 4 * hi) = v;
      }
    }
  }
}

}  // namespace

// Launches the two backward kernels for head dimension D (the launcher in
// fa_bwd.hip has planned the grids).
template <int D, bool BF16, bool MASK>
void launch_bwd(const BwdArgs& a, int batch, bool causal, hipStream_t stream) {
  const int dkdv_wgs = a.units * ((a.nk + kBwdBlockKeys - 1) / kBwdBlockKeys);
  const int dq_wgs = a.items;
  // dQ first: it writes the row statistics the dK/dV kernel reads (its grid
  // covers every query row, a.items = batch * heads * ceil(n / 128)).
  if (causal) {
    if (dq_wgs > 0)
      hipLaunchKernelGGL((fa_bwd_dq_kernel<D, true, MASK, BF16>), dim3(dq_wgs), dim3(256), 0, stream,
                         a);
    if (dkdv_wgs > 0)
      hipLaunchKernelGGL((fa_bwd_dkdv_kernel<D, true, MASK, BF16>), dim3(dkdv_wgs), dim3(512), 0,
                         stream, a);
  } else {
    if (dq_wgs > 0)
      hipLaunchKernelGGL((fa_bwd_dq_kernel<D, false, MASK, BF16>), dim3(dq_wgs), dim3(256), 0, stream,
                         a);
    if (dkdv_wgs > 0)
      hipLaunchKernelGGL((fa_bwd_dkdv_kernel<D, false, MASK, BF16>), dim3(dkdv_wgs), dim3(512), 0,
                         stream, a);
  }
}

}  // namespace fa
