// Three-pass attention through an fp32 score workspace: the compatibility
// path behind `naive_attention_forward` (reference
// src/kernels/naive_attention.cu:17-164).  Not a performance path: it
// materialises [B*Hq, N, N] scores and exists so callers of that op keep
// working.  The masked score value is -inf (the reference writes -1e9, which
// yields the same exact-zero probability).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa_internal.h"

namespace fa {
namespace {

// S[bh][i][j] = scale * <Q[i], K[j]>, masked entries -inf.
// grid (ceil(N/16), ceil(N/16), B*Hq), block (16, 16): x = key, y = query.
__global__ void naive_scores(const FwdArgs a, float* __restrict__ S, int D,
                             float scale, int causal) {
  const int j = blockIdx.x * 16 + threadIdx.x;
  const int i = blockIdx.y * 16 + threadIdx.y;
  const int bh = blockIdx.z;
  const int N = a.n;
  if (i >= N || j >= N) return;
  const int b = bh / a.hq;
  const int hq = bh - b * a.hq;
  const int hkv = hq / a.group;
  float* out = S + ((int64_t)bh * N + i) * N + j;
  if (causal && j > i) {
    *out = -__builtin_inff();
    return;
  }
  const _Float16* q = a.q + b * a.qsb + hq * a.qsh + (int64_t)i * a.qsn;
  const _Float16* k = a.k + b * a.ksb + hkv * a.ksh + (int64_t)j * a.ksn;
  float acc = 0.0f;
  for (int d = 0; d < D; ++d) acc += (float)q[d] * (float)k[d];
  *out = acc * scale;
}

// Row softmax in place; one 64-lane wave per row.
// grid (N, B*Hq), block 64.
__global__ void naive_softmax(float* __restrict__ S, int N) {
  const int i = blockIdx.x;
  const int bh = blockIdx.y;
  float* row = S + ((int64_t)bh * N + i) * N;
  float m = -__builtin_inff();
  for (int j = threadIdx.x; j < N; j += 64) m = fmaxf(m, row[j]);
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  float s = 0.0f;
  for (int j = threadIdx.x; j < N; j += 64) {
    const float e = (row[j] == -__builtin_inff()) ? 0.0f : expf(row[j] - m);
    row[j] = e;
    s += e;
  }
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
  const float inv = (s > 0.0f) ? 1.0f / s : 0.0f;
  for (int j = threadIdx.x; j < N; j += 64) row[j] *= inv;
}

// O[i][d] = sum_j P[i][j] V[j][d]; grid (N, B*Hq), block D (one lane per dim).
__global__ void naive_pv(const FwdArgs a, const float* __restrict__ P, int D) {
  const int i = blockIdx.x;
  const int bh = blockIdx.y;
  const int d = threadIdx.x;
  const int N = a.n;
  if (d >= D) return;
  const int b = bh / a.hq;
  const int hq = bh - b * a.hq;
  const int hkv = hq / a.group;
  const float* prow = P + ((int64_t)bh * N + i) * N;
  const _Float16* v = a.v + b * a.vsb + hkv * a.vsh + d;
  float acc = 0.0f;
  for (int j = 0; j < N; ++j) acc += prow[j] * (float)v[(int64_t)j * a.vsn];
  a.o[b * a.osb + hq * a.osh + (int64_t)i * a.osn + d] = (_Float16)acc;
}

}  // namespace

int launch_naive_forward(const FwdArgs& a, int batch, int head_dim, bool causal,
                         float scale, float* workspace, hipStream_t stream) {
  const unsigned bh = (unsigned)(batch * a.hq);
  const unsigned nt = (unsigned)((a.n + 15) / 16);
  hipLaunchKernelGGL(naive_scores, dim3(nt, nt, bh), dim3(16, 16), 0, stream, a,
                     workspace, head_dim, scale, causal ? 1 : 0);
  hipLaunchKernelGGL(naive_softmax, dim3((unsigned)a.n, bh), dim3(64), 0, stream,
                     workspace, a.n);
  hipLaunchKernelGGL(naive_pv, dim3((unsigned)a.n, bh), dim3((unsigned)head_dim), 0,
                     stream, a, (const float*)workspace, head_dim);
  return 0;
}

}  // namespace fa
