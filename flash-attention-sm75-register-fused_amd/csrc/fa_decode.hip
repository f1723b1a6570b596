// Split-K forward for few query rows per K/V head (KV-cache decode).
//
// When heads_q / heads_kv * seq_len <= 32, all query rows that read one
// (batch, KV head) -- the "unit" -- fit the 32 query columns of one MFMA
// tile, and the work is streaming K and V once from HBM: the path is
// HBM-bound (2 * Nk * D * 2 bytes per unit against 4 * rows * Nk * D FLOP).
// The 128-row prefill kernel would read K/V once per query head and leave
// most of its rows empty, so this path reorganises the work:
//
//   * grid = units x splits: split s of a unit takes key tiles
//     [s * chunk, (s + 1) * chunk) of 32 keys; the four waves of a workgroup
//     take every fourth tile of the chunk and run independently (no
//     workgroup barrier inside the loop): K straight from HBM into VGPRs as
//     the MFMA A operand, V through a per-wave, double-buffered LDS tile
//     (direct-to-LDS loads, read back transposed with ds_read_b64_tr_b16);
//   * the four waves' (max, sum, O) merge through LDS at the end;
//   * with one split the workgroup writes O (and LSE) directly; otherwise it
//     writes an fp32 partial (unnormalised O, running max in log2 units, sum)
//     to the caller's workspace and fa_decode_combine (for many splits,
//     fa_decode_combine_wide) merges the splits.
//
// Small launches (a 128-row prefill grid of at most kSmallLaunchItems
// workgroups, e.g. one head of 512 rows) take the same path with the query
// rows of each (batch, KV head) in blocks of 32: a unit is then one such
// block, and its keys are split over workgroups like a decode unit's, so the
// launch spreads over many CUs instead of running a few long key chains.
//
// The MFMA formulation, the LDS tile layout, the online-softmax numerics and
// the lazy rescale are those of the prefill kernel (fa_fwd.hip): S^T = K Q^T
// with one query per lane, P kept in registers as the B operand of
// O^T = V^T P^T.  Query column c of unit (b, hkv, row block rb) is row
// r = 32 rb + c of the (batch, KV head): query head hkv * group + r / Nq,
// query index r % Nq.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "fa_internal.h"

#include "fa_kernel_common.h"

namespace fa {
namespace {

constexpr int kDecTile = 32;       // keys per wave tile
constexpr int kDecMinTiles = 8;    // fewest tiles a split is given (decode)
constexpr int kSmallMinTiles = 4;  // small launches: one tile per wave
// Small launches with at most this many 32-key tiles run one split per unit:
// the four waves of the workgroup (16 tiles each at most) are then the whole
// key split, and the launch needs neither a workspace nor the combine kernel
// (whose launch costs more than it saves on such short key ranges; measured
// on MI355X: one head of 512 rows 6.3 against 8.9 us, of 2048 rows even).
constexpr int kSmallNoSplitTiles = 64;
constexpr int kDecTargetWgs = 256; // one workgroup per CU (measured best)

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// Per-wave V tile: 32 rows of D halves with no padding (a direct load costs
// its wave about the same per instruction whatever it moves, so padding
// lanes were a third of the loads at head_dim 64, a fifth at 128).  Only the
// transposing V reads touch this tile, and each reads the same 64 bytes of
// rows 4k..4k+3 (and 4k+8..): chunk c of row r is stored at c ^ swz(r) so
// that those four rows land in four disjoint 64-byte windows of the 256-byte
// bank sweep -- at head_dim 64 (128-byte rows) rows 4k and 4k+2 differ in
// chunk bit 2 (dense_swizzle, as the prefill kernel's dense tiles), at 128
// (256-byte rows, one sweep each) chunk bits 2-3 take the row's position in
// its group of four.  swz(r + 16) = swz(r), so the two 16-key halves share a
// base; the XOR reaches chunk bit 2, so each 32-dim output tile has its own.
template <int D>
struct DecLds {
  static constexpr int Pitch = D;                      // halves per row
  static constexpr int Tile = kDecTile * Pitch;        // halves per V tile
  static constexpr int Segs = Tile * 2 / 1024;         // 1 KB direct-load segments
  static_assert(Tile * 2 % 1024 == 0, "V tile must be whole segments");
  static __device__ __forceinline__ int swz(int r) {
    if constexpr (D == 64) return dense_swizzle(r);
    else return (r & 3) << 2;
  }
};

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] and
// vmcnt[5:4] at bits 15:14, expcnt 7, lgkmcnt 15), followed by a compiler
// memory barrier: the waitcnt intrinsic does not touch memory as far as the
// compiler knows, so without it the LDS reads that depend on the wait could
// be hoisted above it.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  asm volatile("" ::: "memory");
}

// MASK_MODE: 0 no explicit mask, 1 mask bits (one 32-bit word per row and
// tile), 2 key-padding bytes (fa_fwd_params.mask_keys: one byte per key, the
// same for every row of the batch; a ballot over the tile's 32 bytes forms
// the word).
template <int D, bool CAUSAL, int MASK_MODE, bool BF16>
__global__ void __launch_bounds__(kThreads, 2) fa_decode_kernel(const DecArgs d) {
  constexpr bool MASK = MASK_MODE != 0;
  constexpr bool KEY_BYTES = MASK_MODE == 2;
  const FwdArgs& a = d.f;
  using L = DecLds<D>;
  using E = Elem<BF16>;
  constexpr int KK = D / 16;   // 16-wide contraction steps of S^T
  constexpr int MT = D / 32;   // 32-row output tiles of O^T
  constexpr int NPV = 2 * MT;  // P V MFMAs per 32-key tile
  constexpr int SEGS = L::Segs;

  // Per-wave V tiles: wave w uses [w * Tile, (w + 1) * Tile) of each array.
  __shared__ __attribute__((aligned(1024))) _Float16 v_lds0[kWaves * L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 v_lds1[kWaves * L::Tile];
  // Each wave's running max and row sums for the final merge (its O goes to
  // its two V tiles, which it fills exactly: MT 32 x 32 float tiles).
  __shared__ float ml_lds[kWaves * 128];
  static_assert(MT / 2 * 16 * 64 * 4 <= L::Tile * 2, "O of a wave fits its V tiles");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wave-uniform (in a scalar register): the per-wave buffer windows and LDS
  // destinations derived from it must be scalar, or every direct load would
  // become a loop over the distinct values of the wave.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hi = lane >> 5;
  const int ql = lane & 31;
  const int grp = lane >> 4;
  const int gi = lane & 15;

  const int unit = (int)blockIdx.x / d.splits;
  const int split = (int)blockIdx.x - unit * d.splits;
  const int hkv_count = a.hq / a.group;
  const int bh = unit / d.row_blocks;  // (batch, KV head)
  const int rb = unit - bh * d.row_blocks;
  const int b = bh / hkv_count;
  const int hkv = bh - b * hkv_count;
  const int nq = a.n;
  const int NK = a.nk;

  // This lane's query column: row r of the (batch, KV head).
  const int r = rb * kDecodeMaxRows + ql;
  const bool row_ok = ql < d.rows && r < d.total_rows;
  const int g = r / nq;
  const int qi = r - g * nq;
  const int hq = hkv * a.group + g;
  // Smallest query index of the block's rows (wave-uniform): causal tiles
  // past it + diag need the per-element mask.
  const int r0 = rb * kDecodeMaxRows;
  const int r_last = min(d.total_rows, r0 + kDecodeMaxRows) - 1;
  const bool one_head = r0 / nq == r_last / nq;
  const int qi_lo = one_head ? r0 % nq : 0;
  // Largest query index of the block's rows: under causal masking no row of
  // the unit sees a key past qi_hi + diag, so tiles past it are skipped.
  const int qi_hi = one_head ? r_last % nq : nq - 1;
  const int unit_tiles =
      CAUSAL ? min(d.tiles, max(0, (qi_hi + a.diag + kDecTile) / kDecTile)) : d.tiles;

  half8 qf[KK];
  if (row_ok) {
    const _Float16* qp = a.q + b * a.qsb + hq * a.qsh + (int64_t)qi * a.qsn + 8 * hi;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qf[kk] = *(const half8*)(qp + 16 * kk);
  } else {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qf[kk] = (half8)(_Float16)0;
  }
  if (a.negate_q) {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qf[kk] = negate16(qf[kk]);
  }

  // Tiles of this split, and this wave's share (every fourth one).
  const int t_begin = split * d.chunk_tiles;
  const int t_end = min(t_begin + d.chunk_tiles, unit_tiles);
  const int nt_w = t_end - t_begin > wave ? (t_end - t_begin - wave + kWaves - 1) / kWaves : 0;
  const int key0 = t_begin * kDecTile;
  const _Float16* Kp = a.k + b * a.ksb + hkv * a.ksh;
  const _Float16* Vp = a.v + b * a.vsb + hkv * a.vsh;

  // Loads of tile it are issued whether or not the tile exists (`valid`);
  // a missing tile reads through an empty window (zeros, no memory traffic),
  // so every iteration has the same loads in flight and one vmcnt value
  // serves all of them (a conditional load would make the compiler wait
  // for the worst case and serialise the prefetch).
  // K operand of tile it: key row (tile key base + ql), dims 16 kk + 8 hi;
  // rows past the last key read as zeros.
  const int k_rows_left = NK - key0;
  const int k_bytes = k_rows_left > 0 ? k_rows_left * (int)a.ksn * 2 : 0;
  auto load_k = [&](int it, half8 (&kf)[KK], bool valid) {
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(Kp + (int64_t)key0 * a.ksn, valid ? k_bytes : 0);
    const int key = (wave + kWaves * it) * kDecTile + ql;
    const int voff = key * (int)a.ksn * 2 + 16 * hi;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      kf[kk] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(rk, voff + 32 * kk, 0, 0));
  };

  // V direct loads: segment s, lane l covers tile bytes [1024 s + 16 l, +16).
  int goff_v[SEGS];
#pragma unroll
  for (int s = 0; s < SEGS; ++s) {
    const int pos = s * 1024 + 16 * lane;
    const int row = pos / (2 * L::Pitch);
    const int within = pos - row * (2 * L::Pitch);
    const int c = (within >> 4) ^ L::swz(row);
    goff_v[s] = (int)(row * a.vsn * 2) + 16 * c;
  }
  auto load_v = [&](int it, _Float16* tile, bool valid) {
    const int kb = key0 + (wave + kWaves * it) * kDecTile;
    const int rows_left = valid ? NK - kb : 0;
    const __amdgpu_buffer_rsrc_t rv =
        make_rsrc(Vp + (int64_t)kb * a.vsn, rows_left > 0 ? rows_left * (int)a.vsn * 2 : 0);
    // Non-temporal: every V row is read once (measured +13-17% on the
    // long-context shapes; the K loads, 32 rows x 32 bytes per instruction,
    // stay cached so that the other half of each line hits).
#pragma unroll
    for (int s = 0; s < SEGS; ++s) direct_load16_nt(rv, (lds_void*)(tile + s * 512), goff_v[s]);
  };
  _Float16* const my_v0 = v_lds0 + wave * L::Tile;
  _Float16* const my_v1 = v_lds1 + wave * L::Tile;

  // MASK: this lane's mask row read as 32-bit words (word t: keys of 32-key
  // tile t), through a buffer window over batch b's rows so the load is the
  // same kind as the K and V loads (their completion order is then the
  // issue order, which the vmcnt wait below relies on).  KEY_BYTES: byte
  // (tile * 32 + ql) of batch b's key row instead, one load per step too,
  // through a window that ends at the last key (keys past it read as 0).
  __amdgpu_buffer_rsrc_t rmask;
  int m_voff = 0;
  if (KEY_BYTES) {
    const int64_t span = NK > 0 ? (int64_t)(NK - 1) * a.mksk + 1 : 0;
    rmask = make_rsrc(a.mkeys + b * a.mksb, (int)min(span, (int64_t)INT32_MAX));
    m_voff = ql * (int)a.mksk;
  } else if (MASK) {
    const int hq_c = row_ok ? hq : hkv * a.group;
    const int qi_c = row_ok ? qi : 0;
    const int64_t words = (NK + 63) / 64;
    const int64_t span =
        ((int64_t)(hkv * a.group + a.group - 1) * a.msh + (int64_t)(nq - 1) * a.msq + words) * 8;
    rmask = make_rsrc(a.mbits + b * a.msb, (int)min(span, (int64_t)INT32_MAX));
    m_voff = (int)((hq_c * a.msh + qi_c * a.msq) * 8);
  }
  auto load_mask = [&](int it, bool valid) -> uint32_t {
    const int tile = valid ? t_begin + wave + kWaves * it : t_begin;
    if constexpr (KEY_BYTES)
      return __builtin_amdgcn_raw_buffer_load_b8(rmask, m_voff + tile * kDecTile * (int)a.mksk,
                                                 0, 0);
    return __builtin_amdgcn_raw_buffer_load_b32(rmask, m_voff + 4 * tile, 0, 0);
  };

  // Per-lane bases of the transposing V reads: rows 16ks + 4hi + gi/4
  // (+8), dims 32mt + 16(grp&1) + 4(gi&3), one pair of bases per mt.
  const int v_row = 4 * hi + (gi >> 2);
  const int v_c = 2 * (grp & 1) + ((gi & 3) >> 1);
  int v_base0[MT], v_base1[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    v_base0[mt] = v_row * L::Pitch + 8 * ((v_c + 4 * mt) ^ L::swz(v_row)) + 4 * (gi & 1);
    v_base1[mt] = (v_row + 8) * L::Pitch + 8 * ((v_c + 4 * mt) ^ L::swz(v_row + 8)) + 4 * (gi & 1);
  }
  auto read_v = [&](const _Float16* Vs, int v) -> half8 {
    const int ks = v / MT, mt = v % MT;
    const int imm = 16 * ks * L::Pitch;
    const half4 lo = ds_read_tr16(Vs + v_base0[mt] + imm);
    const half4 hi4 = ds_read_tr16(Vs + v_base1[mt] + imm);
    return __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
  };

  float16v oacc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) oacc[mt] = (float16v)0.0f;
  float m_run = -__builtin_inff();
  float l_run = 0.0f;
  const float c2 = a.c;
  const int diag_row = qi + a.diag;  // causal: keys <= diag_row are visible

  half8 kA[KK], kB[KK];

  // The word of a tile from what load_mask returned (bit k: key 32 t + k
  // visible): key bytes (lanes l and l + 32 hold key 32 t + l) give it as the
  // low half of a ballot; mask bits are the lane's word itself.
  auto word_of = [&](uint32_t raw) -> uint32_t {
    if constexpr (KEY_BYTES) return (uint32_t)__builtin_amdgcn_ballot_w64(raw != 0);
    else return raw;
  };
  // Whether no lane (query row) sees a key of a tile: its K and V are then
  // not read (an empty window: zeros, no memory traffic) and its scores are
  // all masked, so it adds exactly nothing.  Padded batches skip their
  // padding this way.
  auto hidden = [&](uint32_t w) -> bool { return __builtin_amdgcn_ballot_w64(w != 0) == 0; };

  // One tile: S, softmax, P V.  The loads of the next tile are issued first.
  // MASK: mw and w_next are the words of tiles it and it + 1; raw2 is what
  // load_mask returned for tile it + 2 (issued a step ago), and tile it + 3's
  // mask load goes to raw3.  Returns tile it + 2's word, formed after this
  // step's V wait, when raw2 has landed: every mask load is issued two steps
  // before its tile's K and V loads, so deciding whether they are needed
  // never waits.
  auto step = [&](int it, half8 (&kc)[KK], half8 (&kn)[KK], _Float16* vc, _Float16* vn,
                  uint32_t mw, uint32_t w_next, uint32_t raw2, uint32_t& raw3) -> uint32_t {
    const bool has_next = it + 1 < nt_w;
    const bool skip_next = MASK && hidden(w_next);
    if (MASK) raw3 = load_mask(it + 3, it + 3 < nt_w);
    load_k(it + 1, kn, has_next && !skip_next);
    load_v(it + 1, vn, has_next && !skip_next);
    float16v s = (float16v)0.0f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      s = E::mfma(kc[kk], qf[kk], s);

    const int kstart = key0 + (wave + kWaves * it) * kDecTile;
    bool need_mask =
        (kstart + kDecTile > NK) || (CAUSAL && kstart + kDecTile - 1 > qi_lo + a.diag);
    if (MASK) need_mask = need_mask || __builtin_amdgcn_ballot_w64(~mw != 0) != 0;
    if (need_mask) {
      const uint32_t mws = mw >> (4 * hi);  // bit 8 (i / 4) + i % 4: element i
      static_for<16>([&](auto i_c) {
        constexpr int i = decltype(i_c)::value;
        const int key = kstart + 8 * (i >> 2) + 4 * hi + (i & 3);
        bool masked = key >= NK || (CAUSAL && key > diag_row);
        if (MASK) masked = masked || ((mws >> (8 * (i >> 2) + (i & 3))) & 1) == 0;
        if (masked) s[i] = -__builtin_inff();
      });
    }
    float mx = s[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[i]);
    mx = halves_max(mx);
    const bool grow = (mx - m_run) * c2 > kRescaleLog2;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      const float m_new = fmaxf(m_run, mx);
      const float m_use = (m_new == -__builtin_inff()) ? 0.0f : m_new;
      const float alpha =
          (m_run == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f((m_run - m_use) * c2);
      l_run *= alpha;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) oacc[mt] *= alpha;
      m_run = m_new;
    }
    const float mc = ((m_run == -__builtin_inff()) ? 0.0f : m_run) * c2;
    uint4v pf[2];  // P operands as 32-bit lanes (pairs written whole)
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], c2, -mc));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i + 1], c2, -mc));
      const half2v pr = E::pack(p0, p1);
      pf[i >> 3][(i & 7) >> 1] = __builtin_bit_cast(unsigned, pr);
      l_run = E::sum2(pr, l_run);
    }
    // V of this tile has landed once only the next tile's loads are pending
    // (loads complete in order).
    wait_vmcnt<KK + SEGS + (MASK ? 1 : 0)>();
    const uint32_t w_next2 = MASK ? word_of(raw2) : ~0u;
    half8 vf[NPV];
#pragma unroll
    for (int v = 0; v < NPV; ++v) vf[v] = read_v(vc, v);
#pragma unroll
    for (int v = 0; v < NPV; ++v) {
      const int ks = v / MT, mt = v % MT;
      oacc[mt] = E::mfma(vf[v], __builtin_bit_cast(half8, pf[ks]), oacc[mt]);
    }
    return w_next2;
  };

  if (nt_w > 0) {
    // Every step issues one mask load (MASK), then K and V of its next tile;
    // the prologue issues the masks of tiles 0, 1 and 2, then K and V of tile
    // 0 (read whether hidden or not: deciding would wait for its mask first).
    uint32_t raw0 = 0u, raw1 = 0u, rawA = 0u, rawB = 0u, wc = ~0u, wn = ~0u;
    if (MASK) {
      raw0 = load_mask(0, true);
      raw1 = load_mask(1, 1 < nt_w);
      rawB = load_mask(2, 2 < nt_w);
    }
    load_k(0, kA, true);
    load_v(0, my_v0, true);
    if (MASK) {
      wc = word_of(raw0);
      wn = word_of(raw1);
    }
    int it = 0;
    for (; it + 1 < nt_w; it += 2) {
      uint32_t w2 = step(it, kA, kB, my_v0, my_v1, wc, wn, rawB, rawA);
      wc = wn;
      wn = w2;
      w2 = step(it + 1, kB, kA, my_v1, my_v0, wc, wn, rawA, rawB);
      wc = wn;
      wn = w2;
    }
    if (it < nt_w) step(it, kA, kB, my_v0, my_v1, wc, wn, rawB, rawA);
  }

  // ---- merge the four waves through LDS (the V tiles are free now) --------
  // The last step's loads of a tile that does not exist are still in flight:
  // drain them, or their zeros could land in LDS after the merge writes.
  wait_vmcnt<0>();
  const float l_tot = halves_sum(l_run);
  __syncthreads();
  {
    float* o_lo = (float*)(v_lds0 + wave * L::Tile);
    float* o_hi = (float*)(v_lds1 + wave * L::Tile);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float* dst = (mt < MT / 2 ? o_lo : o_hi) + (mt % (MT / 2)) * 16 * 64;
#pragma unroll
      for (int i = 0; i < 16; ++i) dst[i * 64 + lane] = oacc[mt][i];
    }
    float* ml = ml_lds + wave * 128;
    ml[lane] = m_run;
    ml[64 + lane] = l_tot;
  }
  __syncthreads();
  if (wave >= MT) return;
  const int mt = wave;  // this wave merges output tile mt
  float m_w[kWaves], M = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < kWaves; ++u) {
    const float* ml = ml_lds + u * 128;
    m_w[u] = ml[lane];
    M = fmaxf(M, m_w[u]);
  }
  float Ltot = 0.0f;
  float o[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = 0.0f;
#pragma unroll
  for (int u = 0; u < kWaves; ++u) {
    const float f = (m_w[u] == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f((m_w[u] - M) * c2);
    const float* base = (const float*)((mt < MT / 2 ? v_lds0 : v_lds1) + u * L::Tile) +
                        (mt % (MT / 2)) * 16 * 64;
    const float* ml = ml_lds + u * 128;
    Ltot += f * ml[64 + lane];
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] += f * base[i * 64 + lane];
  }
  if (!row_ok) return;
  if (d.splits == 1) {
    const float inv = (Ltot > 0.0f) ? (1.0f / Ltot) : 0.0f;
    _Float16* op = a.o + b * a.osb + hq * a.osh + (int64_t)qi * a.osn + 32 * mt + 4 * hi;
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      half4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = E::round(o[4 * g4 + e] * inv);
      *(half4*)(op + 8 * g4) = v;
    }
    if (a.lse != nullptr && mt == 0 && hi == 0) {
      const float m_use = (M == -__builtin_inff()) ? 0.0f : M;
      a.lse[((int64_t)b * a.hq + hq) * nq + qi] =
          (m_use * c2 + __builtin_log2f(Ltot)) * 0.69314718055994530942f;
    }
  } else {
    const int64_t p = ((int64_t)unit * d.splits + split) * d.rows + ql;
    float* po = d.part_o + p * D + 32 * mt + 4 * hi;
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      float4 v = {o[4 * g4], o[4 * g4 + 1], o[4 * g4 + 2], o[4 * g4 + 3]};
      *(float4*)(po + 8 * g4) = v;
    }
    if (mt == 0 && hi == 0) {
      d.part_ml[2 * p] = (M == -__builtin_inff()) ? -__builtin_inff() : M * c2;
      d.part_ml[2 * p + 1] = Ltot;
    }
  }
}

// Merges the splits of one (unit, query column) with 256 threads:
// O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s, M = max_s m_s.
// Thread (grp, dim) of the 256 / D groups of D threads takes every
// (256 / D)-th split from grp: it loads the (max, sum) records and its
// dimension of the partial O of four splits at a time, all independent of
// each other, and folds them into its own running (max, sum, O) as the
// prefill kernel folds key tiles; the groups' states merge once through
// LDS.  One round trip to memory per four splits and one barrier: the
// partials come from other XCDs' caches or HBM, so a merge that waits for
// the maxima before it asks for the sums and the O values pays that latency
// three times.
constexpr int kCombineThreads = 256;
constexpr int kMaxSplits = 1024;  // splits per unit (the plan's bound)

template <int D, bool BF16>
__global__ void __launch_bounds__(kCombineThreads) fa_decode_combine(const DecArgs d) {
  const FwdArgs& a = d.f;
  constexpr int GROUPS = kCombineThreads / D;
  __shared__ float m_grp[GROUPS], l_grp[GROUPS];
  __shared__ float o_grp[GROUPS][D];
  const int tid = threadIdx.x;
  const int unit = (int)blockIdx.x / d.rows;
  const int c = (int)blockIdx.x - unit * d.rows;  // query column of the unit
  const int hkv_count = a.hq / a.group;
  const int bh = unit / d.row_blocks;
  const int rb = unit - bh * d.row_blocks;
  const int b = bh / hkv_count;
  const int hkv = bh - b * hkv_count;
  const int r = rb * kDecodeMaxRows + c;
  if (r >= d.total_rows) return;  // whole workgroup: columns past the last row
  const int g = r / a.n;
  const int qi = r - g * a.n;
  const int hq = hkv * a.group + g;
  const int64_t p0 = (int64_t)unit * d.splits * d.rows + c;  // split s: p0 + s * rows
  const int S = d.splits;

  const int dim = tid % D;
  const int grp = tid / D;
  constexpr float kNegInf = -__builtin_inff();
  // Running state of this thread's splits: max (log2 units), sum, O[dim]
  // relative to that max.  A split that saw no key has max -inf and adds
  // nothing (2^-inf = 0); while every split so far is such, the state stays
  // (-inf, 0, 0).
  float m_run = kNegInf, l_run = 0.0f, o_run = 0.0f;
  auto fold = [&](int n, const float* ms, const float* ls, const float* os) {
    float m_new = m_run;
    for (int u = 0; u < n; ++u) m_new = fmaxf(m_new, ms[u]);
    if (m_new == kNegInf) return;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
    o_run *= alpha;
    for (int u = 0; u < n; ++u) {
      const float w = __builtin_amdgcn_exp2f(ms[u] - m_new);
      l_run += w * ls[u];
      o_run += w * os[u];
    }
    m_run = m_new;
  };
  int s = grp;
  for (; s + 3 * GROUPS < S; s += 4 * GROUPS) {
    float ms[4], ls[4], os[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t p = p0 + (int64_t)(s + u * GROUPS) * d.rows;
      ms[u] = d.part_ml[2 * p];
      ls[u] = d.part_ml[2 * p + 1];
      os[u] = d.part_o[p * D + dim];
    }
    fold(4, ms, ls, os);
  }
  for (; s < S; s += GROUPS) {
    const int64_t p = p0 + (int64_t)s * d.rows;
    const float ms = d.part_ml[2 * p], ls = d.part_ml[2 * p + 1], os = d.part_o[p * D + dim];
    fold(1, &ms, &ls, &os);
  }
  if (dim == 0) {
    m_grp[grp] = m_run;
    l_grp[grp] = l_run;
  }
  o_grp[grp][dim] = o_run;
  __syncthreads();
  if (grp != 0) return;
  float M = m_grp[0];
#pragma unroll
  for (int q = 1; q < GROUPS; ++q) M = fmaxf(M, m_grp[q]);
  float o = 0.0f, Ltot = 0.0f;
  if (M != kNegInf) {
#pragma unroll
    for (int q = 0; q < GROUPS; ++q) {
      const float w = __builtin_amdgcn_exp2f(m_grp[q] - M);
      o += w * o_grp[q][dim];
      Ltot += w * l_grp[q];
    }
  }
  const float inv = (Ltot > 0.0f) ? (1.0f / Ltot) : 0.0f;
  a.o[b * a.osb + hq * a.osh + (int64_t)qi * a.osn + dim] = Elem<BF16>::round(o * inv);
  if (a.lse != nullptr && dim == 0) {
    const float m_use = (M == -__builtin_inff()) ? 0.0f : M;
    a.lse[((int64_t)b * a.hq + hq) * a.n + qi] =
        (m_use + __builtin_log2f(Ltot)) * 0.69314718055994530942f;
  }
}

// Launches whose threads would each walk more than a few batches of splits
// in fa_decode_combine (split count times head_dim at least
// kWideCombineMin; e.g. one KV head of 65536 keys at 256 splits, whose
// combine took 23 us that way) take this variant: one workgroup per (unit,
// query column, 32 dimensions), 256 threads = 32 split groups x 8 lanes, lane
// i taking dimensions 4i..4i+3 of the chunk (a float4 of each split's
// partial O) and group g the splits g, g + 32, ... with up to 8 loads in
// flight per thread; the groups' states merge once through LDS.  For few
// splits its many small workgroups cost more than they save (a 16-column
// GQA decode with 4 splits: 14% slower), hence the threshold.
constexpr int kWideLanes = 8;                              // float4 lanes: 32 dims
constexpr int kWideGroups = kCombineThreads / kWideLanes;  // split groups
constexpr int kWideBatch = 8;                              // splits in flight per thread
constexpr int kWideCombineMin = 4096;                      // splits * head_dim

template <int D, bool BF16>
__global__ void __launch_bounds__(kCombineThreads) fa_decode_combine_wide(const DecArgs d) {
  const FwdArgs& a = d.f;
  constexpr int CHUNKS = D / (4 * kWideLanes);
  __shared__ float m_grp[kWideGroups], l_grp[kWideGroups];
  __shared__ float4 o_grp[kWideGroups][kWideLanes];
  const int tid = threadIdx.x;
  const int chunk = (int)blockIdx.x % CHUNKS;
  const int uc = (int)blockIdx.x / CHUNKS;
  const int unit = uc / d.rows;
  const int c = uc - unit * d.rows;  // query column of the unit
  const int hkv_count = a.hq / a.group;
  const int bh = unit / d.row_blocks;
  const int rb = unit - bh * d.row_blocks;
  const int b = bh / hkv_count;
  const int hkv = bh - b * hkv_count;
  const int r = rb * kDecodeMaxRows + c;
  if (r >= d.total_rows) return;  // whole workgroup: columns past the last row
  const int g = r / a.n;
  const int qi = r - g * a.n;
  const int hq = hkv * a.group + g;
  const int64_t p0 = (int64_t)unit * d.splits * d.rows + c;  // split s: p0 + s * rows
  const int S = d.splits;

  const int lane = tid % kWideLanes;
  const int grp = tid / kWideLanes;
  const int dim0 = 4 * (chunk * kWideLanes + lane);
  constexpr float kNegInf = -__builtin_inff();
  // Running state as in fa_decode_combine, for 4 dimensions.
  float m_run = kNegInf, l_run = 0.0f;
  float o_run[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s = grp; s < S; s += kWideBatch * kWideGroups) {
    float ms[kWideBatch], ls[kWideBatch];
    float4 os[kWideBatch];
    int n = 0;  // splits of this batch (a prefix of the 8)
#pragma unroll
    for (int u = 0; u < kWideBatch; ++u) {
      const int su = s + u * kWideGroups;
      if (su < S) {
        const int64_t p = p0 + (int64_t)su * d.rows;
        const float2 ml = *(const float2*)(d.part_ml + 2 * p);
        ms[u] = ml.x;
        ls[u] = ml.y;
        os[u] = *(const float4*)(d.part_o + p * D + dim0);
        n = u + 1;
      }
    }
    float m_new = m_run;
#pragma unroll
    for (int u = 0; u < kWideBatch; ++u)
      if (u < n) m_new = fmaxf(m_new, ms[u]);
    if (m_new == kNegInf) continue;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int e = 0; e < 4; ++e) o_run[e] *= alpha;
#pragma unroll
    for (int u = 0; u < kWideBatch; ++u) {
      if (u < n) {
        const float w = __builtin_amdgcn_exp2f(ms[u] - m_new);
        l_run += w * ls[u];
        o_run[0] += w * os[u].x;
        o_run[1] += w * os[u].y;
        o_run[2] += w * os[u].z;
        o_run[3] += w * os[u].w;
      }
    }
    m_run = m_new;
  }
  if (lane == 0) {
    m_grp[grp] = m_run;
    l_grp[grp] = l_run;
  }
  o_grp[grp][lane] = float4{o_run[0], o_run[1], o_run[2], o_run[3]};
  __syncthreads();
  if (grp != 0) return;
  float M = m_grp[0];
#pragma unroll
  for (int q = 1; q < kWideGroups; ++q) M = fmaxf(M, m_grp[q]);
  float o[4] = {0.0f, 0.0f, 0.0f, 0.0f}, Ltot = 0.0f;
  if (M != kNegInf) {
#pragma unroll 8
    for (int q = 0; q < kWideGroups; ++q) {
      const float w = __builtin_amdgcn_exp2f(m_grp[q] - M);
      const float4 oq = o_grp[q][lane];
      o[0] += w * oq.x;
      o[1] += w * oq.y;
      o[2] += w * oq.z;
      o[3] += w * oq.w;
      Ltot += w * l_grp[q];
    }
  }
  const float inv = (Ltot > 0.0f) ? (1.0f / Ltot) : 0.0f;
  half4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = Elem<BF16>::round(o[e] * inv);
  *(half4*)(a.o + b * a.osb + hq * a.osh + (int64_t)qi * a.osn + dim0) = v;
  if (a.lse != nullptr && chunk == 0 && lane == 0) {
    const float m_use = (M == kNegInf) ? 0.0f : M;
    a.lse[((int64_t)b * a.hq + hq) * a.n + qi] =
        (m_use + __builtin_log2f(Ltot)) * 0.69314718055994530942f;
  }
}

template <bool BF16>
void launch_decode_typed(const DecArgs& d, const DecodePlan& pl, int head_dim, bool causal,
                         hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)pl.units * pl.splits));
#define FA_DEC(DD, C, M) \
  hipLaunchKernelGGL((fa_decode_kernel<DD, C, M, BF16>), grid, dim3(kThreads), 0, stream, d)
#define FA_DEC_M(DD, C)                            \
  if (d.f.mkeys != nullptr) FA_DEC(DD, C, 2);      \
  else if (d.f.mbits != nullptr) FA_DEC(DD, C, 1); \
  else FA_DEC(DD, C, 0)
  if (head_dim == 128) {
    if (causal) { FA_DEC_M(128, true); } else { FA_DEC_M(128, false); }
  } else {
    if (causal) { FA_DEC_M(64, true); } else { FA_DEC_M(64, false); }
  }
#undef FA_DEC_M
#undef FA_DEC
  if (pl.splits > 1) {
    const bool wide = pl.splits * head_dim >= kWideCombineMin;
    const dim3 cgrid((unsigned)((int64_t)pl.units * pl.rows * (wide ? head_dim / 32 : 1)));
#define FA_CMB(DD)                                                                          \
  if (wide)                                                                                 \
    hipLaunchKernelGGL((fa_decode_combine_wide<DD, BF16>), cgrid, dim3(kCombineThreads), 0, \
                       stream, d);                                                          \
  else                                                                                      \
    hipLaunchKernelGGL((fa_decode_combine<DD, BF16>), cgrid, dim3(kCombineThreads), 0, stream, d)
    if (head_dim == 128) { FA_CMB(128); } else { FA_CMB(64); }
#undef FA_CMB
  }

}

}  // namespace

bool decode_eligible(const FwdArgs& a, int batch) {
  const bool decode = (int64_t)a.group * a.n <= kDecodeMaxRows;
  const int64_t prefill_items = (int64_t)batch * a.hq * ((a.n + 127) / 128);
  if (!decode && prefill_items > kSmallLaunchItems) return false;
  if (a.mbits != nullptr) {
    // The split-K kernel reads one batch's mask rows through a single 32-bit
    // buffer window (byte offsets up to this span); a call whose mask strides
    // span more runs on the prefill kernel, which reads the words through
    // 64-bit addresses.
    const int64_t words = ((int64_t)a.nk + 63) / 64;
    const int64_t span =
        ((int64_t)(a.hq - 1) * a.msh + (int64_t)(a.n - 1) * a.msq + words) * 8;
    if (span > (int64_t)INT32_MAX) return false;
  }
  // Key bytes: 32-bit offsets up to one tile past the last key.
  if (a.mkeys != nullptr && ((int64_t)a.nk + 64) * a.mksk > (int64_t)INT32_MAX) return false;
  return true;
}

DecodePlan plan_decode(const FwdArgs& a, int batch, int head_dim, bool causal,
                       int64_t workspace_bytes) {
  DecodePlan pl;
  pl.total_rows = a.group * a.n;
  pl.rows = std::min(pl.total_rows, kDecodeMaxRows);
  pl.row_blocks = (pl.total_rows + kDecodeMaxRows - 1) / kDecodeMaxRows;
  pl.units = batch * (a.hq / a.group) * pl.row_blocks;
  // Keys any query row can see.
  int64_t nk_eff = a.nk;
  if (causal) nk_eff = std::min<int64_t>(a.nk, std::max<int64_t>(0, (int64_t)a.n + a.diag));
  pl.tiles = (int)((nk_eff + kDecTile - 1) / kDecTile);
  int splits = std::min((kDecTargetWgs + pl.units - 1) / pl.units, kMaxSplits);
  splits = std::min(
      splits, std::max(1, pl.tiles / (pl.row_blocks > 1 ? kSmallMinTiles : kDecMinTiles)));
  splits = std::max(splits, 1);
  if (pl.row_blocks > 1 && pl.tiles <= kSmallNoSplitTiles) splits = 1;
  pl.chunk_tiles = std::max(1, (pl.tiles + splits - 1) / splits);
  pl.splits = std::max(1, (pl.tiles + pl.chunk_tiles - 1) / pl.chunk_tiles);
  pl.workspace_bytes =
      pl.splits > 1 ? (int64_t)pl.units * pl.splits * pl.rows * (head_dim + 2) * 4 : 0;
  if (pl.workspace_bytes > workspace_bytes) {  // not enough room: one split
    pl.splits = 1;
    pl.chunk_tiles = std::max(1, pl.tiles);
    pl.workspace_bytes = 0;
  }
  return pl;
}

int launch_decode_forward(const FwdArgs& a, const DecodePlan& pl, int head_dim, bool causal,
                          void* workspace, hipStream_t stream) {
  DecArgs d;
  d.f = a;
  d.rows = pl.rows;
  d.total_rows = pl.total_rows;
  d.row_blocks = pl.row_blocks;
  d.splits = pl.splits;
  d.chunk_tiles = pl.chunk_tiles;
  d.tiles = pl.tiles;
  d.part_o = static_cast<float*>(workspace);
  d.part_ml = pl.splits > 1
                  ? d.part_o + (int64_t)pl.units * pl.splits * pl.rows * head_dim
                  : nullptr;
  if (a.bf16)
    launch_decode_typed<true>(d, pl, head_dim, causal, stream);
  else
    launch_decode_typed<false>(d, pl, head_dim, causal, stream);
  return 0;
}

}  // namespace fa
