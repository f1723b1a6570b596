// Fused attention forward, 256-row workgroups (gfx950, head_dim 128).
//
// Same math, MFMA formulation (S^T = K Q^T, O^T = V^T P^T), LDS tile layout
// and slot-by-slot instruction schedule as the 128-row kernel in fa_fwd.hip;
// the differences:
//  * one wave per SIMD, 64 query rows per wave as two 32-row column blocks
//    (c = 0, 1), so every K, Q and V operand read from LDS feeds two MFMAs,
//    and the fixed per-tile costs (row max, branches, barrier, load issue)
//    are paid once per 64 rows;
//  * Q lives in LDS (read per 16-wide step, not held in registers): the wave
//    needs S_j, S_{j+1}, O and P at once, and Q in registers would overflow
//    the 512 VGPR+AGPR per lane;
//  * LDS: K and V double buffers (80 KB) + the workgroup's Q rows (80 KB).
// Used for large problems (enough workgroups for every CU); a scale < 0 goes
// to the 128-row kernel.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa_internal.h"

#include "fa_kernel_common.h"

namespace fa {
namespace {

constexpr int kRowsPerWaveWide = kBlockMWide / kWaves;  // 64
static_assert(kRowsPerWaveWide == 64, "two 32-row column blocks per wave");

template <int D, bool CAUSAL, bool KV_SAME_STRIDE>
__global__ void __launch_bounds__(kThreads, 1) fa_fwd_wide_kernel(const FwdArgs a) {
  using L = Lds<D>;
  constexpr int KK = D / 16;       // 16-wide contraction steps of S^T
  constexpr int MT = D / 32;       // 32-row output tiles of O^T
  constexpr int NVF = 4 * MT;      // V operand fragments per tile (ks, mt)
  constexpr int NS = 4 * KK;       // S^T MFMAs per tile: (kk, c, t)
  constexpr int NPV = 2 * NVF;     // P V MFMAs per tile: (f, c)
  constexpr int NSA = 8;           // S^T MFMAs issued while the row maxima are formed
  constexpr int PFR = 4;           // K/Q operand reads run one 16-wide step ahead
  constexpr int PFV = 2;           // V fragments read this many fragments ahead
  constexpr int SEGW = L::SegsPerWave;
  constexpr int QSEGS = kRowsPerWaveWide * L::Pitch * 2 / 1024;  // per wave
  constexpr int QTILE = kRowsPerWaveWide * L::Pitch;            // halves per wave

  __shared__ __attribute__((aligned(1024))) _Float16 k_lds0[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 k_lds1[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 v_lds0[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 v_lds1[L::Tile];
  __shared__ __attribute__((aligned(1024))) _Float16 q_lds[kWaves * QTILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hi = lane >> 5;
  const int ql = lane & 31;
  const int grp = lane >> 4;
  const int gi = lane & 15;

  const Work w = block_work(a, (int)blockIdx.x, CAUSAL);
  const int b = w.b, hq = w.hq, hkv = w.hkv, qb = w.qb;
  const int bh = b * a.hq + hq;
  const int q0 = qb * kBlockMWide;
  const int qw = q0 + wave * kRowsPerWaveWide;
  const int N = a.n;    // query rows
  const int NK = a.nk;  // key rows
  int qrow[2];
  qrow[0] = qw + ql;
  qrow[1] = qw + 32 + ql;

  const _Float16* Qp = a.q + b * a.qsb + hq * a.qsh;
  const _Float16* Kp = a.k + b * a.ksb + hkv * a.ksh;
  const _Float16* Vp = a.v + b * a.vsb + hkv * a.vsh;
  _Float16* q_mine = q_lds + wave * QTILE;

  const int kv_len = CAUSAL ? max(0, min(NK, q0 + kBlockMWide + a.diag)) : NK;
  const int ntiles = (kv_len + kBlockN - 1) / kBlockN;

  // ---- direct-load maps (see Lds): tiles are filled by 1 KB segments ------
  auto tile_offset = [&](int pos, int64_t row_stride) {  // pos: bytes into an LDS tile
    const int row = pos / (2 * L::Pitch);
    const int within = pos - row * (2 * L::Pitch);
    if (within >= 2 * D) return -16;  // padding: past any window -> zeros
    const int c = (within >> 4) ^ ((row >> 2) & 3);
    return (int)(row * row_stride * 2) + 16 * c;
  };
  int goff_k[SEGW], goff_v_own[KV_SAME_STRIDE ? 1 : SEGW];
  int* goff_v = KV_SAME_STRIDE ? goff_k : goff_v_own;
#pragma unroll
  for (int s = 0; s < SEGW; ++s) {
    const int pos = (wave + kWaves * s) * 1024 + 16 * lane;
    goff_k[s] = tile_offset(pos, a.ksn);
    if (!KV_SAME_STRIDE) goff_v[s] = tile_offset(pos, a.vsn);
  }
  const int k_tile_bytes = (int)(kBlockN * a.ksn * 2);
  const int v_tile_bytes = (int)(kBlockN * a.vsn * 2);
  const int k_all_bytes = (int)(NK * a.ksn * 2);
  const int v_all_bytes = (int)(NK * a.vsn * 2);

  auto kbuf = [&](auto par) -> _Float16* {
    if constexpr (decltype(par)::value) return k_lds1; else return k_lds0;
  };
  auto vbuf = [&](auto par) -> _Float16* {
    if constexpr (decltype(par)::value) return v_lds1; else return v_lds0;
  };
  auto lds_seg = [&](_Float16* tile, int s) -> lds_void* {
    return (lds_void*)(tile + (wave + kWaves * s) * 512);
  };
  auto k_window = [&](int j) {
    const int bytes = k_all_bytes - j * k_tile_bytes;
    return make_rsrc(Kp + (int64_t)j * kBlockN * a.ksn, bytes > 0 ? bytes : 0);
  };
  auto v_window = [&](int j) {
    const int bytes = v_all_bytes - j * v_tile_bytes;
    return make_rsrc(Vp + (int64_t)j * kBlockN * a.vsn, bytes > 0 ? bytes : 0);
  };

  // ---- operand reads -------------------------------------------------------
  const int sK = (ql >> 2) & 3;
  const int k_base_even = ql * L::Pitch + 8 * (hi ^ sK);
  const int k_base_odd = ql * L::Pitch + 8 * ((2 + hi) ^ sK);
  const int v_row = 4 * hi + (gi >> 2);
  const int v_c = 2 * (grp & 1) + ((gi & 3) >> 1);
  const int v_base0 = v_row * L::Pitch + 8 * (v_c ^ hi) + 4 * (gi & 1);
  const int v_base1 = (v_row + 8) * L::Pitch + 8 * (v_c ^ (hi + 2)) + 4 * (gi & 1);

  // A operand of S^T (K rows 32t + ql) or B operand (Q rows 32c + ql): both
  // tiles share the layout, rows 32x + ql, chunk 2kk + hi.
  auto read_rows = [&](const _Float16* tile, int x, int kk) -> half8 {
    const int off = ((kk & 1) ? k_base_odd : k_base_even) + 32 * x * L::Pitch + 32 * (kk >> 1);
    return *(const half8*)(tile + off);
  };
  auto read_v = [&](const _Float16* Vs, int f) -> half8 {
    const int ks = f / MT, mt = f % MT;
    const int imm = 16 * ks * L::Pitch + 32 * mt;
    const half4 lo = ds_read_tr16(Vs + v_base0 + imm);
    const half4 hi4 = ds_read_tr16(Vs + v_base1 + imm);
    return __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
  };

  float16v oacc[2][MT];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) oacc[c][mt] = (float16v)0.0f;
  }
  float m_run[2] = {-__builtin_inff(), -__builtin_inff()};
  float l_run[2] = {0.0f, 0.0f};
  const float c2 = a.c;
  const half2v ones = {(_Float16)1.0f, (_Float16)1.0f};

  float16v s_cur[2][2], s_nxt[2][2];  // [column block][32-key sub-tile]

  // S^T MFMA m of a tile: kk = m / 4, c = (m / 2) % 2, t = m % 2, with
  // A = K(t, kk), B = Q(c, kk).  Operand read r (kk = r / 4): K(0,kk),
  // K(1,kk), Q(0,kk), Q(1,kk); read r is issued before MFMA r - PFR.
  half8 kfr[2][KK], qfr[2][KK];
  auto issue_read = [&](const _Float16* Ks, int r) {
    const int kk = r >> 2, type = r & 3;
    if (type < 2)
      kfr[type][kk] = read_rows(Ks, type, kk);
    else
      qfr[type - 2][kk] = read_rows(q_mine, type - 2, kk);
  };
  auto s_mfma = [&](float16v (&s)[2][2], int m) {
    const int kk = m >> 2, c = (m >> 1) & 1, t = m & 1;
    s[c][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kfr[t][kk], qfr[c][kk],
                                                     kk == 0 ? (float16v)0.0f : s[c][t], 0, 0, 0);
  };

  auto step = [&](int j, auto has_next_t, auto par_t) {
    constexpr bool HAS_NEXT = decltype(has_next_t)::value;
    constexpr bool PAR = decltype(par_t)::value;
    constexpr int ns = HAS_NEXT ? NS : 0;
    constexpr int nsa = HAS_NEXT ? NSA : 0;
    const _Float16* Kn = kbuf(Flag<!PAR>{});
    const _Float16* Vc = vbuf(Flag<PAR>{});

    __amdgpu_buffer_rsrc_t rk_next, rv_next;
    if (HAS_NEXT) {
      rk_next = k_window(j + 2);
      rv_next = v_window(j + 1);
    }
    _Float16* k_dst = kbuf(Flag<PAR>{});
    _Float16* v_dst = vbuf(Flag<!PAR>{});
    auto issue_load = [&](int q) {
      if (q < SEGW)
        direct_load16(rk_next, lds_seg(k_dst, q), goff_k[q]);
      else
        direct_load16(rv_next, lds_seg(v_dst, q - SEGW), goff_v[q - SEGW]);
    };

    // ---- mask (sequence tail, causal diagonal), per column block --------
    const int kstart = j * kBlockN;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const bool need_mask =
          (kstart + kBlockN > NK) || (CAUSAL && kstart + kBlockN - 1 > qw + 32 * c + a.diag);
      if (need_mask) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = kstart + 32 * t + 8 * (i >> 2) + 4 * hi + (i & 3);
            const bool masked = (key >= NK) || (CAUSAL && key > qrow[c] + a.diag);
            if (masked) s_cur[c][t][i] = -__builtin_inff();
          }
        }
      }
    }

    // ---- block A: first S_{j+1} MFMAs while both row maxima are formed ---
    if constexpr (HAS_NEXT) {
      static_for<PFR>([&](auto r_c) { issue_read(Kn, decltype(r_c)::value); });
    }
    float mx[2] = {-__builtin_inff(), -__builtin_inff()};
    constexpr int MAXA = nsa > 0 ? nsa : 1;
    static_for<MAXA>([&](auto slot_c) {
      constexpr int slot = decltype(slot_c)::value;
      if constexpr (slot < nsa) {
        if constexpr (slot + PFR < ns) issue_read(Kn, slot + PFR);
        s_mfma(s_nxt, slot);
      }
#pragma unroll
      for (int e = slot * 32 / MAXA; e < (slot + 1) * 32 / MAXA; ++e) {
        mx[0] = fmaxf(mx[0], s_cur[0][e >> 4][e & 15]);
        mx[1] = fmaxf(mx[1], s_cur[1][e >> 4][e & 15]);
      }
      fence_schedule();
    });
    mx[0] = halves_max(mx[0]);
    mx[1] = halves_max(mx[1]);

    const bool grow = (mx[0] - m_run[0]) * c2 > kRescaleLog2 ||
                      (mx[1] - m_run[1]) * c2 > kRescaleLog2;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const float m_new = fmaxf(m_run[c], mx[c]);
        const float m_use = (m_new == -__builtin_inff()) ? 0.0f : m_new;
        const float alpha = (m_run[c] == -__builtin_inff())
                                ? 0.0f
                                : __builtin_amdgcn_exp2f((m_run[c] - m_use) * c2);
        l_run[c] *= alpha;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) oacc[c][mt] *= alpha;
        m_run[c] = m_new;
      }
    }
    float mc[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) mc[c] = ((m_run[c] == -__builtin_inff()) ? 0.0f : m_run[c]) * c2;

    // ---- block B ----------------------------------------------------------
    // Slots: the remaining S_{j+1} MFMAs, then P_j V_j with V fragment f
    // feeding column blocks 0 and 1 in consecutive slots.  The 32 softmax
    // pairs (q = 2p + c) are spread so that pf[c][ks] is complete before the
    // first P V MFMA of step ks; within a slot the MFMA is issued first.
    constexpr int NB = (ns - nsa) + NPV;
    constexpr int PV_FIRST = ns - nsa;
    constexpr int PAIR_SLOTS = NB - 2 * MT;
    constexpr auto pair_slot = [](int q) constexpr {
      const int p = q >> 1;
      const int spread = (q * PAIR_SLOTS) / 32;
      const int last_ok = PV_FIRST + 2 * MT * (p / 4) - 1;
      return spread < last_ok ? spread : last_ok;
    };
    constexpr auto read_slot = [](int f) constexpr {
      const int s = PV_FIRST + 2 * (f - PFV);
      return s > 0 ? s : 0;
    };
    half8 pf[2][4];
    half8 vf[NVF];
    auto softmax_pair = [&](auto q_c) {
      constexpr int q = decltype(q_c)::value;
      constexpr int p = q >> 1, c = q & 1;
      constexpr int e = 2 * p;
      constexpr int t = e >> 4, i = e & 15;
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[c][t][i], c2, -mc[c]));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[c][t][i + 1], c2, -mc[c]));
      const half2v pr = {(_Float16)p0, (_Float16)p1};
      pf[c][2 * t + (i >> 3)][i & 7] = pr[0];
      pf[c][2 * t + (i >> 3)][(i & 7) + 1] = pr[1];
      l_run[c] = __builtin_amdgcn_fdot2(pr, ones, l_run[c], false);
    };
    static_for<32>([&](auto q_c) {
      if constexpr (pair_slot(decltype(q_c)::value) < 0) softmax_pair(q_c);
    });
    static_for<NB>([&](auto slot_c) {
      constexpr int slot = decltype(slot_c)::value;
      static_for<NVF>([&](auto f_c) {
        constexpr int f = decltype(f_c)::value;
        if constexpr (read_slot(f) == slot) vf[f] = read_v(Vc, f);
      });
      if constexpr (slot < PV_FIRST) {
        constexpr int m = nsa + slot;
        if constexpr (m + PFR < ns) issue_read(Kn, m + PFR);
        s_mfma(s_nxt, m);
      } else {
        constexpr int m = slot - PV_FIRST;
        constexpr int f = m >> 1, c = m & 1;
        constexpr int ks = f / MT, mt = f % MT;
        oacc[c][mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[f], pf[c][ks], oacc[c][mt], 0, 0, 0);
      }
      if constexpr (HAS_NEXT) {
        static_for<2 * SEGW>([&](auto q_c) {
          constexpr int q = decltype(q_c)::value;
          if constexpr ((q * (NB / 2)) / (2 * SEGW) == slot) issue_load(q);
        });
      }
      static_for<32>([&](auto q_c) {
        if constexpr (pair_slot(decltype(q_c)::value) == slot) softmax_pair(q_c);
      });
      fence_schedule();
    });

    if (HAS_NEXT) {
      barrier_after_direct_loads();
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int t = 0; t < 2; ++t) s_cur[c][t] = s_nxt[c][t];
      }
    }
  };

  // ---- prologue: this wave's Q rows, K_0, V_0, K_1 into LDS; S_0 -----------
  {
    const int qbytes = (N - qw) * (int)a.qsn * 2;
    const __amdgpu_buffer_rsrc_t rq =
        make_rsrc(Qp + (int64_t)qw * a.qsn, qbytes > 0 ? qbytes : 0);
#pragma unroll
    for (int s = 0; s < QSEGS; ++s)
      direct_load16(rq, (lds_void*)(q_mine + s * 512), tile_offset(s * 1024 + 16 * lane, a.qsn));
  }
  if (ntiles > 0) {
    const __amdgpu_buffer_rsrc_t rk0 = k_window(0), rv0 = v_window(0);
#pragma unroll
    for (int s = 0; s < SEGW; ++s) {
      direct_load16(rk0, lds_seg(k_lds0, s), goff_k[s]);
      direct_load16(rv0, lds_seg(v_lds0, s), goff_v[s]);
    }
    if (ntiles > 1) {
      const __amdgpu_buffer_rsrc_t rk1 = k_window(1);
#pragma unroll
      for (int s = 0; s < SEGW; ++s) direct_load16(rk1, lds_seg(k_lds1, s), goff_k[s]);
    }
  }
  barrier_after_direct_loads();
  if (ntiles > 0) {
    static_for<NS>([&](auto r_c) { issue_read(k_lds0, decltype(r_c)::value); });
    static_for<NS>([&](auto m_c) { s_mfma(s_cur, decltype(m_c)::value); });
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

  // ---- epilogue ---------------------------------------------------------------
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const float l_tot = halves_sum(l_run[c]);
    const float inv = (l_tot > 0.0f) ? (1.0f / l_tot) : 0.0f;
    if (qrow[c] < N) {
      _Float16* op = a.o + b * a.osb + hq * a.osh + (int64_t)qrow[c] * a.osn;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          half4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (_Float16)(oacc[c][mt][4 * g + e] * inv);
          *(half4*)(op + 32 * mt + 8 * g + 4 * hi) = v;
        }
      }
      if (a.lse != nullptr && hi == 0) {
        const float m_use = (m_run[c] == -__builtin_inff()) ? 0.0f : m_run[c];
        const float lse2 = m_use * c2 + __builtin_log2f(l_tot);
        a.lse[(int64_t)bh * N + qrow[c]] = lse2 * 0.69314718055994530942f;
      }
    }
  }
}

}  // namespace

int launch_fused_forward_wide(const FwdArgs& a, int batch, bool causal, hipStream_t stream) {
  FwdArgs args = a;
  const dim3 grid((unsigned)plan_grid(args, batch, kBlockMWide));
  const dim3 block(kThreads);
  const bool same = a.ksn == a.vsn;
#define FA_LAUNCH_WIDE(C, S) \
  hipLaunchKernelGGL((fa_fwd_wide_kernel<128, C, S>), grid, block, 0, stream, args)
  if (causal) {
    if (same) FA_LAUNCH_WIDE(true, true); else FA_LAUNCH_WIDE(true, false);
  } else {
    if (same) FA_LAUNCH_WIDE(false, true); else FA_LAUNCH_WIDE(false, false);
  }
#undef FA_LAUNCH_WIDE
  return 0;
}

}  // namespace fa
