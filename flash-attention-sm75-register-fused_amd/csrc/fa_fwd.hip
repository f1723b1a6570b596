// Fused attention forward for gfx950 (MI355X / CDNA4).
//
// O = softmax(scale * Q K^T + mask) V with fp16 inputs, fp32 accumulation and
// an fp16 output, in one kernel (the hot path that reference
// src/kernels/flash_attention_forward.cu:345-791 implements for SM75).
//
// Work decomposition
//   grid.x = batch * heads_q, grid.y = query blocks of kBlockM = 128 rows.
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
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa_internal.h"

namespace fa {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBlockM = 32 * kWaves;  // queries per workgroup
constexpr int kBlockN = 64;           // keys per LDS tile
// Online-softmax rescale threshold (log2 units): the running max used for
// the exponent is only raised when a row's tile max exceeds it by more than
// this, so P stays <= 2^8 and the O/l rescale is skipped for most tiles.
// The result is mathematically unchanged (l and O use the same stale max).
constexpr float kRescaleLog2 = 8.0f;

// LDS tile layout: row r of a K or V tile starts at r * Pitch halves, with
// Pitch = D + 32 (64 bytes of padding per row), and its 16-byte chunk c is
// stored at chunk position c ^ ((r >> 2) & 3).  The padding shifts each row
// by 64 bytes modulo the 256-byte bank sweep, the XOR spreads the 4 rows of
// each aligned group over the 4 chunks of a 64-byte block.  Together:
//  * K operand reads (ds_read_b128, 16 lanes = 16 consecutive rows, one
//    chunk) hit 16 distinct 16-byte bank groups;
//  * transposing V reads (ds_read_b64_tr_b16, 32 lanes = 4 rows x two
//    32-byte chunk pairs) hit 8 distinct pair slots;
//  * the XOR only touches the low two chunk bits, so every address is a
//    per-lane base plus a compile-time immediate.
// A tile is written by whole-wave direct loads of 1 KB segments; lanes whose
// 16 bytes fall in the padding load from past the buffer window (zeros).
template <int D>
struct Lds {
  static constexpr int Pitch = D + 32;           // halves per row
  static constexpr int Tile = kBlockN * Pitch;   // halves per K (or V) tile
  static constexpr int Segs = Tile * 2 / 1024;   // 1 KB direct-load segments
  static constexpr int SegsPerWave = Segs / kWaves;
  static_assert(Segs % kWaves == 0, "segments must split over the waves");
};

__device__ __forceinline__ half4 ds_read_tr16(const _Float16* p) {
  short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) short4v*)(p));
  return __builtin_bit_cast(half4, r);
}

// Combines the two half-wave copies of a per-query value (lanes l and l^32):
// v_permlane32_swap(x, x) yields [x_lo, x_lo] and [x_hi, x_hi].
__device__ __forceinline__ float halves_max(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}

// Raw buffer resource over [base, base + bytes): loads past the end return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes,
                                           0x00020000);
}

// 16 bytes per lane from a buffer window straight into LDS (lane l writes
// dst + 16 l).  Kept out of line of the kernel template so the host pass
// still emits the kernel's launch stub.
__device__ __forceinline__ void direct_load16(__amdgpu_buffer_rsrc_t r, lds_void* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, 0, 0, 0);
}

// Freezes the instruction order at this point (nothing is moved across).
__device__ __forceinline__ void fence_schedule() { __builtin_amdgcn_sched_barrier(0); }

// Workgroup barrier that also publishes this wave's direct-to-LDS loads:
// they are counted by vmcnt, which the compiler does not drain before
// s_barrier on its own.  0x0F70 = vmcnt(0) expcnt(7) lgkmcnt(15) (gfx9).
__device__ __forceinline__ void barrier_after_direct_loads() {
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();
}

template <bool B>
struct Flag {
  static constexpr bool value = B;
};

// Software-pipelined main loop: iteration j computes S^T_{j+1} = K_{j+1} Q^T
// while the VALU turns S^T_j into probabilities, then accumulates P_j V_j.
// LDS holds two K and two V tiles; the direct loads of K_{j+2} and V_{j+1}
// issued during iteration j land in the buffers iteration j-1 freed, so one
// barrier per iteration suffices.  KV_SAME_STRIDE: K and V rows have the
// same stride, so V's direct-load offsets are K's (saves registers).
template <int D, bool CAUSAL, bool KV_SAME_STRIDE>
__global__ void __launch_bounds__(kThreads, 2) fa_fwd_kernel(const FwdArgs a) {
  using L = Lds<D>;
  constexpr int KK = D / 16;       // 16-wide contraction steps of S^T
  constexpr int MT = D / 32;       // 32-row output tiles of O^T
  constexpr int NS = 2 * KK;       // S^T MFMAs per tile
  constexpr int NPV = 4 * MT;      // P V MFMAs per tile
  constexpr int NSA = 4;           // S^T MFMAs issued while the row max is formed
  constexpr int PFK = 3;           // K operand reads run this many MFMAs ahead
  constexpr int PFV = 2;           // V operand reads run this many MFMAs ahead
  constexpr int SEGW = L::SegsPerWave;

  // [K buffer 0 | K buffer 1 | V buffer 0 | V buffer 1]
  // Four distinct objects (not one array): the loop is unrolled by two, so
  // every access names its buffer at compile time and the compiler can see
  // that the in-flight direct loads never alias the tiles being read (it
  // would otherwise drain vmcnt before each LDS read).
  __shared__ __attribute__((aligned(1024))) _Float16 k_lds0[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 k_lds1[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 v_lds0[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 v_lds1[L::Tile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hi = lane >> 5;   // which half of the wave
  const int ql = lane & 31;   // query column owned by this lane
  const int grp = lane >> 4;  // 16-lane group (transposing reads)
  const int gi = lane & 15;

  const int bh = blockIdx.x;
  const int b = bh / a.hq;
  const int hq = bh - b * a.hq;
  const int hkv = hq / a.group;
  const int qb = CAUSAL ? (a.num_qblocks - 1 - (int)blockIdx.y) : (int)blockIdx.y;
  const int q0 = qb * kBlockM;
  const int qw = q0 + wave * 32;
  const int qrow = qw + ql;
  const int N = a.n;

  const _Float16* Qp = a.q + b * a.qsb + hq * a.qsh;
  const _Float16* Kp = a.k + b * a.ksb + hkv * a.ksh;
  const _Float16* Vp = a.v + b * a.vsb + hkv * a.vsh;

  // Q^T fragments (B operand of S^T = K Q^T), resident for the whole kernel.
  half8 qf[KK];
  if (qrow < N) {
    const _Float16* qp = Qp + (int64_t)qrow * a.qsn + 8 * hi;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qf[kk] = *(const half8*)(qp + 16 * kk);
  } else {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qf[kk] = (half8)(_Float16)0;
  }
  if (a.negate_q) {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qf[kk] = -qf[kk];
  }

  const int kv_len = CAUSAL ? min(N, q0 + kBlockM) : N;
  const int ntiles = (kv_len + kBlockN - 1) / kBlockN;

  // Direct-load map: wave w fills 1 KB segments w, w + 4, ...; lane l of a
  // segment covers tile bytes [1024 seg + 16 l, +16).  Precompute the global
  // byte offset inside a tile for each segment (padding lanes: past the end).
  int goff_k[SEGW], goff_v_own[KV_SAME_STRIDE ? 1 : SEGW];
  int* goff_v = KV_SAME_STRIDE ? goff_k : goff_v_own;
#pragma unroll
  for (int s = 0; s < SEGW; ++s) {
    const int pos = (wave + kWaves * s) * 1024 + 16 * lane;  // bytes into the tile
    const int row = pos / (2 * L::Pitch);
    const int within = pos - row * (2 * L::Pitch);
    if (within < 2 * D) {
      const int c = (within >> 4) ^ ((row >> 2) & 3);
      goff_k[s] = (int)(row * a.ksn * 2) + 16 * c;
      if (!KV_SAME_STRIDE) goff_v[s] = (int)(row * a.vsn * 2) + 16 * c;
    } else {
      goff_k[s] = -16;  // 0xfffffff0: beyond any window -> writes zeros
      if (!KV_SAME_STRIDE) goff_v[s] = -16;
    }
  }
  const int k_tile_bytes = (int)(kBlockN * a.ksn * 2);
  const int v_tile_bytes = (int)(kBlockN * a.vsn * 2);
  const int k_all_bytes = (int)(N * a.ksn * 2);
  const int v_all_bytes = (int)(N * a.vsn * 2);

  // Buffer selection by compile-time parity.
  auto kbuf = [&](auto par) -> _Float16* {
    if constexpr (decltype(par)::value) return k_lds1; else return k_lds0;
  };
  auto vbuf = [&](auto par) -> _Float16* {
    if constexpr (decltype(par)::value) return v_lds1; else return v_lds0;
  };
  auto lds_seg = [&](_Float16* tile, int s) -> lds_void* {
    return (lds_void*)(tile + (wave + kWaves * s) * 512);
  };
  // Buffer windows of tile j (empty past the last tile: every lane reads 0).
  auto k_window = [&](int j) {
    const int bytes = k_all_bytes - j * k_tile_bytes;
    return make_rsrc(Kp + (int64_t)j * kBlockN * a.ksn, bytes > 0 ? bytes : 0);
  };
  auto v_window = [&](int j) {
    const int bytes = v_all_bytes - j * v_tile_bytes;
    return make_rsrc(Vp + (int64_t)j * kBlockN * a.vsn, bytes > 0 ? bytes : 0);
  };
  auto load_k = [&](int j, _Float16* dst) {
    const __amdgpu_buffer_rsrc_t r =
        make_rsrc(Kp + (int64_t)j * kBlockN * a.ksn, k_all_bytes - j * k_tile_bytes);
#pragma unroll
    for (int s = 0; s < SEGW; ++s)
      direct_load16(r, lds_seg(dst, s), goff_k[s]);
  };
  auto load_v = [&](int j, _Float16* dst) {
    const __amdgpu_buffer_rsrc_t r =
        make_rsrc(Vp + (int64_t)j * kBlockN * a.vsn, v_all_bytes - j * v_tile_bytes);
#pragma unroll
    for (int s = 0; s < SEGW; ++s)
      direct_load16(r, lds_seg(dst, s), goff_v[s]);
  };

  // Per-lane LDS bases of the operand reads (see Lds): K rows ql (+32t),
  // chunk 2kk + hi; V rows 16ks + 4hi + gi/4 (+8), dims 32mt + 16(grp&1) + 4(gi&3).
  const int sK = (ql >> 2) & 3;
  const int k_base_even = ql * L::Pitch + 8 * (hi ^ sK);
  const int k_base_odd = ql * L::Pitch + 8 * ((2 + hi) ^ sK);
  const int v_row = 4 * hi + (gi >> 2);
  const int v_c = 2 * (grp & 1) + ((gi & 3) >> 1);
  const int v_base0 = v_row * L::Pitch + 8 * (v_c ^ hi) + 4 * (gi & 1);
  const int v_base1 = (v_row + 8) * L::Pitch + 8 * (v_c ^ (hi + 2)) + 4 * (gi & 1);

  // K operand i (sub-tile t = i / KK, step kk = i % KK) of one K buffer.
  auto read_k = [&](const _Float16* Ks, int i) -> half8 {
    const int t = i / KK, kk = i % KK;
    const int off = ((kk & 1) ? k_base_odd : k_base_even) + 32 * t * L::Pitch + 32 * (kk >> 1);
    return *(const half8*)(Ks + off);
  };
  // V^T operand v (16-key step ks = v / MT, output tile mt = v % MT).
  auto read_v = [&](const _Float16* Vs, int v) -> half8 {
    const int ks = v / MT, mt = v % MT;
    const int imm = 16 * ks * L::Pitch + 32 * mt;
    const half4 lo = ds_read_tr16(Vs + v_base0 + imm);
    const half4 hi4 = ds_read_tr16(Vs + v_base1 + imm);
    return __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
  };

  float16v oacc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) oacc[mt] = (float16v)0.0f;
  float m_run = -__builtin_inff();
  float l_run = 0.0f;
  const float c2 = a.c;  // |scale| * log2(e)
  const half2v ones = {(_Float16)1.0f, (_Float16)1.0f};

  float16v s_cur[2], s_nxt[2];

  // One pipeline step for tile j (PAR = j & 1).  HAS_NEXT: tile j+1 exists,
  // so S_{j+1} is computed here and the loads of V_{j+1} (and K_{j+2}) are
  // issued.
  auto step = [&](int j, auto has_next_t, auto par_t) {
    constexpr bool HAS_NEXT = decltype(has_next_t)::value;
    constexpr bool PAR = decltype(par_t)::value;
    constexpr int ns = HAS_NEXT ? NS : 0;     // S MFMAs this step
    constexpr int nsa = HAS_NEXT ? NSA : 0;   // ... of which in the max block
    const _Float16* Kn = kbuf(Flag<!PAR>{});
    const _Float16* Vc = vbuf(Flag<PAR>{});

    // Direct loads of K_{j+2} (empty window past the end) and V_{j+1}; one
    // 1 KB segment is issued after each of the first MFMAs of block B, so
    // the address unit's queueing overlaps MFMA execution.
    __amdgpu_buffer_rsrc_t rk_next, rv_next;
    if (HAS_NEXT) {
      rk_next = k_window(j + 2);
      rv_next = v_window(j + 1);
    }
    _Float16* k_dst = kbuf(Flag<PAR>{});
    _Float16* v_dst = vbuf(Flag<!PAR>{});
    auto issue_load = [&](int q) {  // q < SEGW: K segment q, else V segment q - SEGW
      if (q < SEGW)
        direct_load16(rk_next, lds_seg(k_dst, q), goff_k[q]);
      else
        direct_load16(rv_next, lds_seg(v_dst, q - SEGW), goff_v[q - SEGW]);
    };

    // ---- mask (sequence tail, causal diagonal) --------------------------
    const int kstart = j * kBlockN;
    const bool need_mask = (kstart + kBlockN > N) || (CAUSAL && kstart + kBlockN - 1 > qw);
    if (need_mask) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = kstart + 32 * t + 8 * (i >> 2) + 4 * hi + (i & 3);
          const bool masked = (key >= N) || (CAUSAL && key > qrow);
          if (masked) s_cur[t][i] = -__builtin_inff();
        }
      }
    }

    // ---- block A: first S_{j+1} MFMAs while the row max is formed --------
    half8 kf[NS > 0 ? NS : 1];
#pragma unroll
    for (int i = 0; i < PFK && i < ns; ++i) kf[i] = read_k(Kn, i);
    float mx = -__builtin_inff();
    constexpr int MAXA = nsa > 0 ? nsa : 1;   // slots the max is spread over
#pragma unroll
    for (int slot = 0; slot < MAXA; ++slot) {
      if (slot < nsa) {
        const int i = slot;
        if (i + PFK < ns) kf[i + PFK] = read_k(Kn, i + PFK);
        const int t = i / KK, kk = i % KK;
        s_nxt[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
            kf[i], qf[kk], kk == 0 ? (float16v)0.0f : s_nxt[t], 0, 0, 0);
      }
#pragma unroll
      for (int e = slot * 32 / MAXA; e < (slot + 1) * 32 / MAXA; ++e)
        mx = fmaxf(mx, s_cur[e >> 4][e & 15]);
      fence_schedule();
    }
    mx = halves_max(mx);

    // ---- raise the running max only when some row outgrew it by 2^8 -----
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

    // ---- block B: remaining S_{j+1} MFMAs, then P_j V_j; the softmax of --
    // S_j (16 pairs of scores) is spread over the slots.  Within a slot the
    // MFMA is issued first, so the pairs of 16-key step ks must sit in a
    // slot before the first P V MFMA of step ks; pairs that cannot (the
    // last tile has no S MFMAs to hide them behind) go before the loop.
    constexpr int NB = (ns - nsa) + NPV;            // MFMA slots in block B
    constexpr int PV_FIRST = ns - nsa;              // slot of the first P V MFMA
    constexpr int PAIR_SLOTS = NB - MT;             // slots available to pairs
    half8 pf[4];
    half8 vf[NPV];
    auto pair_slot = [&](int p) {
      const int spread = (p * PAIR_SLOTS) / 16;
      const int last_ok = PV_FIRST + (p / 4) * MT - 1;
      return spread < last_ok ? spread : last_ok;
    };
    auto softmax_pair = [&](int p) {
      const int e = 2 * p;
      const int t = e >> 4, i = e & 15;
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[t][i], c2, -mc));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[t][i + 1], c2, -mc));
      const half2v pr = {(_Float16)p0, (_Float16)p1};
      pf[2 * t + (i >> 3)][i & 7] = pr[0];
      pf[2 * t + (i >> 3)][(i & 7) + 1] = pr[1];
      l_run = __builtin_amdgcn_fdot2(pr, ones, l_run, false);
    };
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      if (pair_slot(p) < 0) softmax_pair(p);
    }
#pragma unroll
    for (int slot = 0; slot < NB; ++slot) {
      const int pv_first = PV_FIRST;
      // V operand reads, PFV MFMAs ahead of their use
      if (slot == (pv_first >= PFV ? pv_first - PFV : 0)) {
#pragma unroll
        for (int v = 0; v < PFV; ++v) vf[v] = read_v(Vc, v);
      }
      if (slot >= pv_first) {
        const int v = slot - pv_first + PFV;
        if (v < NPV) vf[v] = read_v(Vc, v);
      }
      // the MFMA of this slot
      if (slot < pv_first) {
        const int i = nsa + slot;
        if (i + PFK < ns) kf[i + PFK] = read_k(Kn, i + PFK);
        const int t = i / KK, kk = i % KK;
        s_nxt[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
            kf[i], qf[kk], kk == 0 ? (float16v)0.0f : s_nxt[t], 0, 0, 0);
      } else {
        const int v = slot - pv_first;
        const int ks = v / MT, mt = v % MT;
        oacc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[v], pf[ks], oacc[mt], 0, 0, 0);
      }
      // direct loads spread over the first half of block B
      if (HAS_NEXT) {
#pragma unroll
        for (int q = 0; q < 2 * SEGW; ++q) {
          if ((q * (NB / 2)) / (2 * SEGW) == slot) issue_load(q);
        }
      }
      // softmax pairs assigned to this slot
#pragma unroll
      for (int p = 0; p < 16; ++p) {
        if (pair_slot(p) == slot) softmax_pair(p);
      }
      fence_schedule();
    }

    if (HAS_NEXT) {
      barrier_after_direct_loads();  // V_{j+1}, K_{j+2} landed; V_j, K_{j+1} reads done
#pragma unroll
      for (int t = 0; t < 2; ++t) s_cur[t] = s_nxt[t];
    }
  };

  // ---- prologue: K_0, V_0, K_1 into LDS; S_0 -------------------------------
  if (ntiles > 0) {
    load_k(0, k_lds0);
    load_v(0, v_lds0);
    if (ntiles > 1) load_k(1, k_lds1);
  }
  barrier_after_direct_loads();
  if (ntiles > 0) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      s_cur[t] = (float16v)0.0f;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        s_cur[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(read_k(k_lds0, t * KK + kk), qf[kk],
                                                          s_cur[t], 0, 0, 0);
    }
    int j = 0;
    for (; j + 2 < ntiles; j += 2) {
      step(j, Flag<true>{}, Flag<false>{});
      step(j + 1, Flag<true>{}, Flag<true>{});
    }
    if (j + 1 < ntiles) {
      step(j, Flag<true>{}, Flag<false>{});
      step(j + 1, Flag<false>{}, Flag<true>{});
    } else {
      step(j, Flag<false>{}, Flag<false>{});
    }
  }

  // ---- epilogue: combine the two half-wave partial sums, normalise, store ---
  const float l_tot = halves_sum(l_run);
  const float inv = (l_tot > 0.0f) ? (1.0f / l_tot) : 0.0f;
  if (qrow < N) {
    _Float16* op = a.o + b * a.osb + hq * a.osh + (int64_t)qrow * a.osn;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        half4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (_Float16)(oacc[mt][4 * g + e] * inv);
        *(half4*)(op + 32 * mt + 8 * g + 4 * hi) = v;
      }
    }
    if (a.lse != nullptr && hi == 0) {
      const float m_use = (m_run == -__builtin_inff()) ? 0.0f : m_run;
      const float lse2 = m_use * c2 + __builtin_log2f(l_tot);
      a.lse[(int64_t)bh * N + qrow] = lse2 * 0.69314718055994530942f;
    }
  }
}

}  // namespace

int launch_fused_forward(const FwdArgs& a, int batch, int head_dim, bool causal,
                         hipStream_t stream) {
  const int64_t nblocks = ((int64_t)a.n + kBlockM - 1) / kBlockM;
  FwdArgs args = a;
  args.num_qblocks = (int)nblocks;
  const dim3 grid((unsigned)(batch * a.hq), (unsigned)nblocks);
  const dim3 block(kThreads);
  const bool same = a.ksn == a.vsn;
#define FA_LAUNCH(D, C, S) \
  hipLaunchKernelGGL((fa_fwd_kernel<D, C, S>), grid, block, 0, stream, args)
  if (head_dim == 128) {
    if (causal) {
      if (same) FA_LAUNCH(128, true, true); else FA_LAUNCH(128, true, false);
    } else {
      if (same) FA_LAUNCH(128, false, true); else FA_LAUNCH(128, false, false);
    }
  } else {
    if (causal) {
      if (same) FA_LAUNCH(64, true, true); else FA_LAUNCH(64, true, false);
    } else {
      if (same) FA_LAUNCH(64, false, true); else FA_LAUNCH(64, false, false);
    }
  }
#undef FA_LAUNCH
  return 0;
}

int fused_block_m() { return kBlockM; }

}  // namespace fa
