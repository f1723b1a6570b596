// Fused attention forward for gfx950 (MI355X / CDNA4).
//
// O = softmax(scale * Q K^T + mask) V with fp16 inputs, fp32 accumulation and
// an fp16 output, in one kernel (the hot path that reference
// src/kernels/flash_attention_forward.cu:345-791 implements for SM75).
//
// Work decomposition
//   grid.x = batch * heads_q, grid.y = query blocks of kBlockM = 128 rows.
//   One workgroup = 4 waves; wave w owns query rows [q0 + 32w, q0 + 32w + 32).
//   Key/value rows stream through LDS in tiles of kBlockN = 64 keys, double
//   buffered (global -> VGPR staging -> LDS), one barrier per tile.
//
// MFMA formulation (v_mfma_f32_32x32x16_f16, operand layouts verified on the
// device):
//   A[m][k]: lane l holds m = l%32, k = 8*(l/32) + j  (8 halves)
//   B[k][n]: lane l holds n = l%32, k = 8*(l/32) + j  (8 halves)
//   C[m][n]: lane l holds n = l%32, m = 8*(i/4) + 4*(l/32) + i%4 (16 floats)
//   * S^T = K Q^T: keys are the M side, queries the N side, so every lane owns
//     a single query (l%32) and 16 of its 32 keys per 32-key sub-tile.  The
//     row max over keys is an in-register reduction plus one exchange with
//     lane l^32; the row sum never needs an exchange until the very end.
//   * O^T = V^T P^T: the probabilities stay in the registers the S^T
//     accumulator produced, reinterpreted as the B operand.  The key order
//     inside each 16-key MFMA step is a permutation shared by P and V (the
//     contraction is order-free).  V^T operands come straight out of a
//     row-major LDS tile with ds_read_b64_tr_b16 (transposing LDS read).
//   * The O^T accumulator keeps, per lane, one query and D/2 of its
//     dimensions, so the online-softmax rescale is a per-lane scalar.
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
typedef short short4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBlockM = 32 * kWaves;  // queries per workgroup
constexpr int kBlockN = 64;           // keys per LDS tile

// XOR swizzle of the 16-byte chunk index inside an LDS row, as a function of
// the row.  For D = 128 (16 chunks / 256 B per row) it makes
//  * the K-operand reads (32 rows x one 16 B chunk) hit 16 distinct chunk
//    slots per 16 lanes, and
//  * the transposing V reads (4 consecutive rows x one 32 B chunk pair per
//    16 lanes) hit 4 distinct pair slots.
// For D = 64 (8 chunks / 128 B per row, two rows per 256 B bank sweep) the
// same two properties hold with the rows' parity taken into account.
template <int D>
__device__ __forceinline__ int chunk_swizzle(int row) {
  if constexpr (D == 128) {
    return ((row & 7) << 1) | ((row >> 3) & 1);
  } else {
    return (((row >> 1) & 3) << 1) | ((row >> 3) & 1);
  }
}

template <int D>
__device__ __forceinline__ int lds_offset(int row, int chunk) {
  return row * D + 8 * (chunk ^ chunk_swizzle<D>(row));
}

__device__ __forceinline__ half4 ds_read_tr16(const _Float16* p) {
  short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) short4v*)(p));
  return __builtin_bit_cast(half4, r);
}

__device__ __forceinline__ float xor32(float x) {
  const int lane = __lane_id();
  int r = __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, x));
  return __builtin_bit_cast(float, r);
}

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(kThreads, 2) fa_fwd_kernel(const FwdArgs a) {
  constexpr int KK = D / 16;      // 16-wide contraction steps of S^T
  constexpr int MT = D / 32;      // 32-row output tiles of O^T
  constexpr int CPR = D / 8;      // 16-byte chunks per K/V row
  constexpr int TILE = kBlockN * D;
  constexpr int LOADS = kBlockN * CPR / kThreads;  // chunks per thread per tile
  static_assert(LOADS * kThreads == kBlockN * CPR, "tile must split evenly");

  __shared__ __attribute__((aligned(16))) _Float16 smem[4 * TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hi = lane >> 5;   // which half of the wave
  const int ql = lane & 31;   // query column owned by this lane

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

  u32x4 kst[LOADS], vst[LOADS];
  auto load_tile = [&](int j) {
#pragma unroll
    for (int p = 0; p < LOADS; ++p) {
      const int g = p * kThreads + tid;
      const int row = g / CPR;
      const int c = g % CPR;
      const int key = j * kBlockN + row;
      if (key < N) {
        kst[p] = *(const u32x4*)(Kp + (int64_t)key * a.ksn + 8 * c);
        vst[p] = *(const u32x4*)(Vp + (int64_t)key * a.vsn + 8 * c);
      } else {
        kst[p] = (u32x4)0u;
        vst[p] = (u32x4)0u;
      }
    }
  };
  auto store_tile = [&](int buf) {
    _Float16* Ks = smem + buf * 2 * TILE;
    _Float16* Vs = Ks + TILE;
#pragma unroll
    for (int p = 0; p < LOADS; ++p) {
      const int g = p * kThreads + tid;
      const int row = g / CPR;
      const int c = g % CPR;
      const int off = lds_offset<D>(row, c);
      *(u32x4*)(Ks + off) = kst[p];
      *(u32x4*)(Vs + off) = vst[p];
    }
  };

  float16v oacc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) oacc[mt] = (float16v)0.0f;
  float m_run = -__builtin_inff();
  float l_run = 0.0f;
  const float c2 = a.c;  // |scale| * log2(e)

  if (ntiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int j = 0; j < ntiles; ++j) {
    const int buf = j & 1;
    const bool has_next = (j + 1) < ntiles;
    if (has_next) load_tile(j + 1);

    const int kstart = j * kBlockN;
    const bool active = !CAUSAL || (kstart <= qw + 31);
    if (active) {
      const _Float16* Ks = smem + buf * 2 * TILE;
      const _Float16* Vs = Ks + TILE;

      // ---- S^T = K Q^T : two 32-key sub-tiles -------------------------------
      float16v s[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        s[t] = (float16v)0.0f;
        const int row = 32 * t + ql;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          const half8 kf = *(const half8*)(Ks + lds_offset<D>(row, 2 * kk + hi));
          s[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[kk], s[t], 0, 0, 0);
        }
      }

      // ---- mask (sequence tail, causal diagonal) ----------------------------
      const bool need_mask = (kstart + kBlockN > N) || (CAUSAL && kstart + kBlockN - 1 > qw);
      if (need_mask) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = kstart + 32 * t + 8 * (i >> 2) + 4 * hi + (i & 3);
            const bool masked = (key >= N) || (CAUSAL && key > qrow);
            if (masked) s[t][i] = -__builtin_inff();
          }
        }
      }

      // ---- online softmax on the accumulator layout -------------------------
      float mx = s[0][0];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[t][i]);
      }
      mx = fmaxf(mx, xor32(mx));
      const float m_new = fmaxf(m_run, mx);
      const float m_use = (m_new == -__builtin_inff()) ? 0.0f : m_new;
      const float alpha =
          (m_run == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f((m_run - m_use) * c2);
      const float mc = m_use * c2;

      half8 pf[4];
      float lsum = 0.0f;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[t][i], c2, -mc));
          lsum += p;
          pf[2 * t + (i >> 3)][i & 7] = (_Float16)p;
        }
      }
      l_run = l_run * alpha + lsum;
      m_run = m_new;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) oacc[mt] *= alpha;

      // ---- O^T += V^T P^T ---------------------------------------------------
      // Key order of 16-key step ks (sub-tile t = ks/2, half s = ks%2):
      // element e of the lane's 8 = key 32t + 16s + 8(e/4) + 4*hi + e%4.
      const int grp = lane >> 4;   // 16-lane group
      const int gi = lane & 15;    // index inside the group
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int rbase = 16 * ks + 4 * hi + (gi >> 2);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int d = 32 * mt + 16 * (grp & 1) + 4 * (gi & 3);
          const int chunk = d >> 3;
          const int sub = d & 7;
          const half4 lo = ds_read_tr16(Vs + lds_offset<D>(rbase, chunk) + sub);
          const half4 hi4 = ds_read_tr16(Vs + lds_offset<D>(rbase + 8, chunk) + sub);
          const half8 vf = __builtin_shufflevector(lo, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
          oacc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[ks], oacc[mt], 0, 0, 0);
        }
      }
    }

    if (has_next) store_tile(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: combine the two half-wave partial sums, normalise, store ---
  const float l_tot = l_run + xor32(l_run);
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
  if (head_dim == 128) {
    if (causal)
      hipLaunchKernelGGL((fa_fwd_kernel<128, true>), grid, block, 0, stream, args);
    else
      hipLaunchKernelGGL((fa_fwd_kernel<128, false>), grid, block, 0, stream, args);
  } else {
    if (causal)
      hipLaunchKernelGGL((fa_fwd_kernel<64, true>), grid, block, 0, stream, args);
    else
      hipLaunchKernelGGL((fa_fwd_kernel<64, false>), grid, block, 0, stream, args);
  }
  return 0;
}

int fused_block_m() { return kBlockM; }

}  // namespace fa
