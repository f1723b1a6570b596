// Device-side building blocks shared by the fused attention kernels
// (fa_fwd.hip: prefill, fa_decode.hip: split-K decode).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace fa {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short short8v __attribute__((ext_vector_type(8)));
typedef unsigned uint4v __attribute__((ext_vector_type(4)));

typedef __attribute__((address_space(3))) void lds_void;

// Element type of Q, K, V, O and P.  Every 16-bit value moves as a _Float16
// container (global and direct loads, LDS, transposing reads); only the
// MFMAs, the fp32 -> 16-bit roundings (round to nearest even) and the pair
// sums of P interpret the bits.
template <bool BF16>
struct Elem;
template <>
struct Elem<false> {  // binary16
  static __device__ __forceinline__ float16v mfma(half8 a, half8 b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ half2v pack(float x, float y) {
    return half2v{(_Float16)x, (_Float16)y};
  }
  // acc + x + y of a packed pair (one v_dot2 against (1, 1)).
  static __device__ __forceinline__ float sum2(half2v p, float acc) {
    const half2v ones = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(p, ones, acc, false);
  }
  static __device__ __forceinline__ _Float16 round(float x) { return (_Float16)x; }
  static __device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }
  // The low and high value of a packed pair, exactly.
  static __device__ __forceinline__ float lo_f32(unsigned w) {
    return (float)__builtin_bit_cast(half2v, w)[0];
  }
  static __device__ __forceinline__ float hi_f32(unsigned w) {
    return (float)__builtin_bit_cast(half2v, w)[1];
  }
  // x times the low (high) value of a packed pair, one rounding (an fma with
  // a zero addend: one v_fma_mix_f32 that reads the 16-bit half in place).
  static __device__ __forceinline__ float mul_lo(unsigned w, float x) {
    return __builtin_fmaf(lo_f32(w), x, 0.0f);
  }
  static __device__ __forceinline__ float mul_hi(unsigned w, float x) {
    return __builtin_fmaf(hi_f32(w), x, 0.0f);
  }
};
template <>
struct Elem<true> {  // bfloat16
  static __device__ __forceinline__ float16v mfma(half8 a, half8 b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ half2v pack(float x, float y) {
    return __builtin_bit_cast(half2v, bf16x2{(__bf16)x, (__bf16)y});
  }
  static __device__ __forceinline__ float sum2(half2v p, float acc) {
    const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p), ones, acc, false);
  }
  static __device__ __forceinline__ _Float16 round(float x) {
    return __builtin_bit_cast(_Float16, (__bf16)x);
  }
  static __device__ __forceinline__ float to_f32(_Float16 x) {
    return __builtin_bit_cast(float, (unsigned)__builtin_bit_cast(unsigned short, x) << 16);
  }
  static __device__ __forceinline__ float lo_f32(unsigned w) { return __builtin_bit_cast(float, w << 16); }
  static __device__ __forceinline__ float hi_f32(unsigned w) {
    return __builtin_bit_cast(float, w & 0xffff0000u);
  }
  static __device__ __forceinline__ float mul_lo(unsigned w, float x) { return lo_f32(w) * x; }
  static __device__ __forceinline__ float mul_hi(unsigned w, float x) { return hi_f32(w) * x; }
};

// -x of every element (sign flip; exact in either element type).
__device__ __forceinline__ half8 negate16(half8 x) {
  return __builtin_bit_cast(half8, __builtin_bit_cast(short8v, x) ^ (short8v)(short)0x8000);
}

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
  static_assert(Segs % 4 == 0, "segments must split over 4 waves");
};

// Dense LDS tile layout (the 4-wave forward kernel at head_dim 64): rows of
// D halves with no padding, so a 64-key tile is 8 KB and arrives in 8 direct
// loads of 1 KB where the padded one takes 12.  Chunk c of row r is stored
// at chunk c ^ dense_swizzle(r), a 3-bit value of (r >> 1) & 7 whose bits are
// reordered so that rows r and r + 2 differ in bit 2:
//  * K operand ds_read_b128 (16 lanes = 16 consecutive rows, one chunk): the
//    8 even rows take 8 distinct chunks of the first 128 bytes of the bank
//    sweep, the 8 odd rows 8 distinct chunks of the second;
//  * transposing V reads (32 lanes = rows 4k..4k+3, the same 64 bytes of
//    each): rows 4k and 4k+2 (likewise 4k+1 and 4k+3) land in opposite
//    64-byte halves of their 128 bytes.
// dense_swizzle(r + 16) = dense_swizzle(r), so the rows of one operand read
// 16 or 32 apart share a per-lane base; chunk bit 2 is swizzled, so each
// 64-dim half of a row (chunks 0-3 or 4-7) takes a base of its own.
template <int D>
struct LdsDense {
  static_assert(D == 64, "dense layout: head_dim 64");
  static constexpr int Pitch = D;               // halves per row
  static constexpr int Tile = kBlockN * Pitch;  // halves per K (or V) tile
  static constexpr int Segs = Tile * 2 / 1024;  // 1 KB direct-load segments
};
__device__ __forceinline__ int dense_swizzle(int r) {
  const int m = (r >> 1) & 7;
  return ((m & 1) << 2) | (m >> 1);
}

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

// First entry of a mask range pair (fa_mask.hip): the row's first visible
// key, with bit 31 set when every key up to the pair's second entry is
// visible too (the row sees exactly that interval).
__device__ __forceinline__ int range_first_key(int32_t v) { return v & 0x7fffffff; }
__device__ __forceinline__ bool range_is_dense(int32_t v) { return v < 0; }

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
// The same with the non-temporal policy (the "nt" bit: streamed data that no
// other workgroup reads again, e.g. a KV cache in decode).
__device__ __forceinline__ void direct_load16_nt(__amdgpu_buffer_rsrc_t r, lds_void* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, voff, 0, 0, 2);
}

// Freezes the instruction order at this point (nothing is moved across).
__device__ __forceinline__ void fence_schedule() { __builtin_amdgcn_sched_barrier(0); }

// Workgroup barrier after which all but this wave's last N direct-to-LDS
// loads have landed (vmcnt counts them, and they complete in order), so the
// tiles they wrote are visible to every wave, and every wave's LDS reads and
// writes before it are done (lgkmcnt 0).  The compiler does not wait for
// direct loads before s_barrier on its own.  __syncthreads() is not used: its
// workgroup fence counts direct loads as LDS writes and so adds a full
// vmcnt(0), which would drain the loads a multi-stage pipeline keeps in
// flight.  The empty asm statements with a memory clobber keep the compiler
// from moving memory accesses across the barrier, which the fence did.
template <int N>
__device__ __forceinline__ void barrier_after_loads() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <bool B>
struct Flag {
  static constexpr bool value = B;
};

// Compile-time loop: f(std::integral_constant<int, I>{}) for I = 0..N-1.
// Used for the long slot schedules, which must expand completely (a rolled
// loop would force the register arrays it indexes into scratch memory) and
// are too large for the loop unroller's pragma threshold.
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Work item of workgroup `wg` of the 1-D grid: batch b, query head hq, KV
// head hkv and query block qb.  The grid holds units * group * num_qblocks
// workgroups, a unit being one (batch, KV head).
//  * Workgroup wg runs on XCD wg % 8.  With a.xcds == 8 (units divisible by
//    8) XCD x takes the units [x*U/8, (x+1)*U/8), so all query heads of a
//    group, and all query blocks, that read one K/V pair share an L2.  With
//    a.xcds == 1 the whole grid is one sequence.
//  * Within a sequence, workgroups go rank-major: rank r of every head before
//    rank r+1.  Under causal masking rank 0 is the last (most expensive)
//    query block, so the cheap blocks fill the tail of the launch.
//  * a.pair_half > 0 (a causal launch that fits the GPU in one round): an
//    XCD hands its first 2 * CUs workgroups out so that sequence positions p
//    and p + pair_half share a CU (pair_half = CUs per XCD, times 8 with one
//    sequence).  Positions from pair_half on then hold the ranks in reverse,
//    so each CU gets a large and a small block: C3's CUs hold 34 key tiles
//    each instead of 20..48.
struct Work {
  int b, hq, hkv, qb;
};
// Args: FwdArgs, or BwdArgs for the backward's dQ kernel (same field names).
//  * unit_major (the dynamic schedule's queues): a sequence holds all blocks
//    of its first unit (rank-major within it) before the next unit's, so the
//    workgroups an XCD runs at once stream one K/V pair through its L2
//    (measured on C5: FETCH_SIZE 4.15 -> 2.14 GB per launch, same results).
template <class Args>
__device__ __forceinline__ Work block_work(const Args& a, int wg, bool causal,
                                           bool unit_major = false) {
  const int x = wg % a.xcds;
  int p = wg / a.xcds;
  if (a.pair_half > 0 && p >= a.pair_half) p = a.items / a.xcds - 1 + a.pair_half - p;
  const int per = a.units / a.xcds;   // units of this sequence
  const int row = per * a.group;      // workgroups per rank
  int rank, rest;
  if (unit_major) {
    const int per_unit = a.group * a.num_qblocks;
    const int uu = p / per_unit;
    const int pu = p - uu * per_unit;
    rank = pu / a.group;
    rest = uu * a.group + (pu - rank * a.group);
  } else {
    rank = p / row;
    rest = p - rank * row;
  }
  const int ul = rest / a.group;
  const int u = x * per + ul;
  const int hkv_count = a.hq / a.group;
  Work w;
  w.b = u / hkv_count;
  w.hkv = u - w.b * hkv_count;
  w.hq = w.hkv * a.group + (rest - ul * a.group);
  w.qb = causal ? a.num_qblocks - 1 - rank : rank;
  return w;
}

// s_getreg operand for the XCC_ID hardware register (id 20, bits [31:0]):
// its low bits name the XCD the wave runs on.
constexpr int kHwRegXccId = 20 | (31 << 11);

}  // namespace
}  // namespace fa
