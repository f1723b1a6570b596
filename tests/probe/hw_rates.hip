// Throughput probes of the gfx950 units the attention kernels share:
// matrix (MFMA), vector (VALU) and LDS pipes, and the gap between
// back-to-back kernel launches on one stream.  Measurement infrastructure:
// built by __graft_entry__.build() into tests/probe/libhw_rates.so and run by
// tests/probe/hw_rates.py; nothing in the product loads it.
//
// Every probe launches one workgroup per CU (256 on MI355X, each of
// 4 * waves_per_simd waves, so every SIMD holds waves_per_simd waves), times
// one launch with HIP events and returns the rate, or a negative value on a
// HIP error.  Each wave works on its own registers or its own LDS
// addresses; every LDS address stays inside the 64 KiB buffer the kernel
// declares, and no probe touches global memory except its one-value result
// per thread.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));

constexpr int kCus = 256;

__device__ __forceinline__ void fence() { __builtin_amdgcn_sched_barrier(0); }

// 16 v_mfma_f32_32x32x16_f16 per iteration in four accumulator chains, with
// NV VALU instructions (alternately an FMA and an exp2) spread evenly
// between them (NV = 0: MFMA only).
template <int NV>
__global__ void mix_kernel(float* out, int iters) {
  const int lane = (int)threadIdx.x & 63;
  half8 a = (half8)(_Float16)(0.001f * lane);
  half8 b = (half8)(_Float16)0.002f;
  float16v c0 = (float16v)0.0f, c1 = c0, c2 = c0, c3 = c0;
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = 0.5f + 0.01f * i + lane * 1e-4f;
  asm volatile("" : "+v"(a), "+v"(b));
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      if ((m & 3) == 0) c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
      if ((m & 3) == 1) c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
      if ((m & 3) == 2) c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
      if ((m & 3) == 3) c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
#pragma unroll
      for (int k = 0; k < NV / 16; ++k) {
        const int i = (m * (NV / 16) + k) & 15;
        if (k & 1) v[i] = __builtin_amdgcn_exp2f(v[i]);
        else v[i] = __builtin_fmaf(v[i], 0.999f, -0.001f);
      }
      fence();
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += v[i] + c0[i] + c1[i] + c2[i] + c3[i];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// 16 VALU instructions per iteration, one kind: 0 v_fma_f32, 1 v_exp_f32,
// 2 v_max3_f32, 3 v_cvt_pk_f16_f32 + v_dot2c_f32_f16 (a pair).
template <int OP>
__global__ void valu_kernel(float* out, int iters) {
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = 0.5f + 0.001f * i - 0.0001f * (int)threadIdx.x;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (OP == 0) v[i] = __builtin_fmaf(v[i], 0.999f, -0.001f);
      if (OP == 1) v[i] = __builtin_amdgcn_exp2f(v[i]);
      if (OP == 2) v[i] = fmaxf(fmaxf(v[i], v[(i + 1) & 15]), v[(i + 5) & 15]);
      if (OP == 3) {
        const half2v p = half2v{(_Float16)v[i], (_Float16)v[(i + 3) & 15]};
        v[i] = __builtin_amdgcn_fdot2(p, half2v{(_Float16)1.0f, (_Float16)1.0f}, v[i], false);
      }
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += v[i];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// 16 LDS reads per iteration: OP 0 ds_read_b128 (1 KiB per wave), OP 1
// ds_read_b64_tr_b16 (512 bytes per wave); offsets below 64 KiB.
template <int OP>
__global__ void lds_kernel(float* out, int iters) {
  __shared__ __attribute__((aligned(16))) char buf[65536];
  const int lane = (int)threadIdx.x & 63;
  for (int i = (int)threadIdx.x; i < 65536 / 4; i += (int)blockDim.x) ((float*)buf)[i] = i * 0.5f;
  __syncthreads();
  float4v acc = (float4v)0.0f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if (OP == 0) {
        const int off = ((it & 3) << 14) + r * 1024 + 16 * lane;  // < 65536
        acc += *(const float4v*)(buf + off);
      } else {
        const int off = ((it & 3) << 14) + r * 512 + 8 * lane;  // < 65536
        const short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) short4v*)(buf + off));
        acc[0] += (float)v[0];
        acc[1] += (float)v[1];
      }
    }
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = acc[0] + acc[1] + acc[2] + acc[3];
}

// Runs `clocks` shader clocks (s_memtime) and returns.
__global__ void spin_kernel(long long clocks) {
  const long long t0 = clock64();
  while (clock64() - t0 < clocks) {
  }
}

float* g_out = nullptr;

// Milliseconds of one launch of f() (after one untimed warm-up launch).
template <class F>
double time_ms(F f) {
  if (g_out == nullptr && hipMalloc(&g_out, sizeof(float) * kCus * 1024) != hipSuccess) return -1.0;
  f(10);
  if (hipDeviceSynchronize() != hipSuccess) return -1.0;
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.0;
  (void)hipEventRecord(e0, nullptr);
  f(-1);
  (void)hipEventRecord(e1, nullptr);
  if (hipEventSynchronize(e1) != hipSuccess) return -1.0;
  float ms = 0.0f;
  (void)hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return hipGetLastError() == hipSuccess ? ms : -1.0;
}

bool valid_waves(int w) { return w >= 1 && w <= 4; }

}  // namespace

extern "C" {

// ns per iteration of 16 MFMAs interleaved with nvalu VALU instructions
// (nvalu in {0, 64, 112, 160}), per wave, with waves_per_simd waves on every
// SIMD (the SIMD's rate: iteration time / waves_per_simd).
double fa_rate_mix(int nvalu, int waves_per_simd, int iters) {
  if (!valid_waves(waves_per_simd) || iters <= 0) return -1.0;
  const dim3 grid(kCus), block(256 * waves_per_simd);
  auto go = [&](auto kern) {
    return time_ms([&](int n) {
      hipLaunchKernelGGL(kern, grid, block, 0, nullptr, g_out, n > 0 ? n : iters);
    });
  };
  double ms;
  switch (nvalu) {
    case 0: ms = go(mix_kernel<0>); break;
    case 64: ms = go(mix_kernel<64>); break;
    case 112: ms = go(mix_kernel<112>); break;
    case 160: ms = go(mix_kernel<160>); break;
    default: return -1.0;
  }
  return ms < 0 ? ms : ms * 1e6 / iters / waves_per_simd;
}

// ns per wave-instruction on one SIMD for VALU kind op (see valu_kernel).
double fa_rate_valu(int op, int waves_per_simd, int iters) {
  if (!valid_waves(waves_per_simd) || iters <= 0) return -1.0;
  const dim3 grid(kCus), block(256 * waves_per_simd);
  auto go = [&](auto kern) {
    return time_ms([&](int n) {
      hipLaunchKernelGGL(kern, grid, block, 0, nullptr, g_out, n > 0 ? n : iters);
    });
  };
  double ms;
  switch (op) {
    case 0: ms = go(valu_kernel<0>); break;
    case 1: ms = go(valu_kernel<1>); break;
    case 2: ms = go(valu_kernel<2>); break;
    case 3: ms = go(valu_kernel<3>); break;
    default: return -1.0;
  }
  const double insts = (double)iters * 16 * waves_per_simd * (op == 3 ? 2 : 1);
  return ms < 0 ? ms : ms * 1e6 / insts;
}

// LDS bytes read per ns per CU (op 0 ds_read_b128, 1 ds_read_b64_tr_b16).
double fa_rate_lds(int op, int waves_per_simd, int iters) {
  if (!valid_waves(waves_per_simd) || iters <= 0 || op < 0 || op > 1) return -1.0;
  const dim3 grid(kCus), block(256 * waves_per_simd);
  auto go = [&](auto kern) {
    return time_ms([&](int n) {
      hipLaunchKernelGGL(kern, grid, block, 0, nullptr, g_out, n > 0 ? n : iters);
    });
  };
  const double ms = op == 0 ? go(lds_kernel<0>) : go(lds_kernel<1>);
  const double bytes = (double)iters * 16 * (op == 0 ? 1024 : 512) * 4 * waves_per_simd;
  return ms < 0 ? ms : bytes / (ms * 1e6);
}

// Microseconds per launch of `launches` back-to-back launches of a kernel
// that spins `clocks` shader clocks in each of 256 workgroups.
double fa_rate_launch(long long clocks, int launches) {
  if (clocks < 0 || launches <= 0 || launches > 100000) return -1.0;
  hipEvent_t e0, e1;
  hipLaunchKernelGGL(spin_kernel, dim3(kCus), dim3(256), 0, nullptr, clocks);
  if (hipDeviceSynchronize() != hipSuccess) return -1.0;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.0;
  (void)hipEventRecord(e0, nullptr);
  for (int i = 0; i < launches; ++i)
    hipLaunchKernelGGL(spin_kernel, dim3(kCus), dim3(256), 0, nullptr, clocks);
  (void)hipEventRecord(e1, nullptr);
  if (hipEventSynchronize(e1) != hipSuccess) return -1.0;
  float ms = 0.0f;
  (void)hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return hipGetLastError() == hipSuccess ? ms * 1e3 / launches : -1.0;
}

}  // extern "C"
