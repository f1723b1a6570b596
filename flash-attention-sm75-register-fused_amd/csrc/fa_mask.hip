// Boolean attention mask -> packed bit rows.
//
// The fused kernels read an explicit mask as bits: word w of row (b, h, i)
// holds keys [64 w, 64 w + 64), bit k set <=> key 64 w + k is visible.  A
// 64-key prefill tile is then one 8-byte load per lane (its query row), and a
// 32-key decode tile half of one, instead of 64 (or 32) byte loads.
//
// Rows of consecutive bytes (key stride 1, what torch's bool tensors are):
// one wave packs two consecutive 1024-byte chunks of a row per pass (one for
// rows of at most 1024 keys), 16 words each.  Each lane loads 16 bytes at
// once (a 16-byte load at any alignment; the target runs in unaligned access
// mode, and a load never reaches past the row's last key) and turns them
// into 16 bits; the four lanes of a word combine theirs through cross-lane
// reads.  A row's last partial 16 bytes are read one by one.  Measured on
// MI355X: a [4, 1, 4096, 4096] mask (64 MiB, what transformers builds for a
// padded prefill of 4 x 4096 tokens, packed again in every layer) in 18.5 us
// instead of 191 us with one byte per lane and load; [8, 1, 1024, 1024] in
// 4.8 instead of 24.2 us.
//
// Other key strides: one wave builds one word per iteration, lane k reading
// element 64 w + k of the row, and a ballot over the wave is the word.
//
// Ranges (fa_sm75_pack_mask_ranges): each row's first visible key and one
// past its last, with bit 31 of the first set when every key between them
// is visible (the row's visible keys are exactly that interval: a causal,
// padding or sliding-window row).  The forward kernel then knows, without
// reading a mask word, that a tile inside the interval of every row of a
// wave hides nothing.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "fa_internal.h"

namespace fa {
namespace {

constexpr int kPackWaves = 4;
constexpr int kRowChunk = 1024;  // bytes of one row per wave and load (16 per lane)

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Bit e set <=> byte e of x is nonzero (e < 4): bit 7 of each byte of
// (x & 0x7f..) + 0x7f.. is set iff its low seven bits are not all zero (no
// carry leaves a byte), and x's own bit 7 covers the rest.
__device__ __forceinline__ uint32_t nonzero_bytes4(uint32_t x) {
  const uint32_t t = (((x & 0x7f7f7f7fu) + 0x7f7f7f7fu) | x) & 0x80808080u;
  return ((t >> 7) & 1u) | ((t >> 14) & 2u) | ((t >> 21) & 4u) | ((t >> 28) & 8u);
}

// Span of a row's visible keys, lane-wise: lo = the first, hi = one past the
// last, from 16 bits for keys k0 .. k0 + 15.
__device__ __forceinline__ void add_span(int& lo, int& hi, int k0, uint32_t bits16) {
  if (bits16 != 0) {
    lo = min(lo, k0 + __builtin_ctz(bits16));
    hi = max(hi, k0 + 32 - __builtin_clz(bits16));
  }
}

// The wave's span and count of visible keys (every lane gets them).
__device__ __forceinline__ void reduce_span(int& lo, int& hi, int& cnt) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    lo = min(lo, __shfl_xor(lo, d));
    hi = max(hi, __shfl_xor(hi, d));
    cnt += __shfl_xor(cnt, d);
  }
}

// The first entry of a row's range pair: its first visible key, bit 31 set
// when all keys of [lo, hi) are visible.
__device__ __forceinline__ int32_t range_first(int lo, int hi, int cnt, int64_t cols) {
  if (hi <= 0) return (int32_t)cols;  // no visible key
  return cnt == hi - lo ? (int32_t)((uint32_t)lo | 0x80000000u) : lo;
}

// Packs chunks c .. c + PASS - 1 (1024 bytes each) of the row at rp into out
// (the row's words), all loads issued before any is used (more bytes in
// flight per wave, in one stretch of the row); RANGES: widens the lane's span.
template <int PASS, bool RANGES>
__device__ __forceinline__ void pack_chunks(const uint8_t* rp, int64_t c, int64_t cols,
                                            int64_t words, uint64_t* row_out, int lane, int& lo,
                                            int& hi, int& cnt) {
  u32x4 v[PASS];
  bool whole[PASS];
#pragma unroll
  for (int u = 0; u < PASS; ++u) {
    const int64_t k0 = (c + u) * kRowChunk + 16 * lane;  // this lane's first key
    whole[u] = k0 + 16 <= cols;
    if (whole[u]) __builtin_memcpy(&v[u], rp + k0, 16);
  }
#pragma unroll
  for (int u = 0; u < PASS; ++u) {
    const int64_t k0 = (c + u) * kRowChunk + 16 * lane;
    uint32_t bits = 0;
    if (whole[u]) {
      bits = nonzero_bytes4(v[u].x) | (nonzero_bytes4(v[u].y) << 4) |
             (nonzero_bytes4(v[u].z) << 8) | (nonzero_bytes4(v[u].w) << 12);
    } else {
      for (int e = 0; e < 16; ++e)
        if (k0 + e < cols && rp[k0 + e] != 0) bits |= 1u << e;
    }
    if constexpr (RANGES) {
      add_span(lo, hi, (int)k0, bits);
      cnt += __builtin_popcount(bits);
    }
    // Word j of this chunk: the 16-bit groups of lanes 4j .. 4j + 3.
    const uint64_t g0 = (uint32_t)__shfl((int)bits, 4 * lane);
    const uint64_t g1 = (uint32_t)__shfl((int)bits, 4 * lane + 1);
    const uint64_t g2 = (uint32_t)__shfl((int)bits, 4 * lane + 2);
    const uint64_t g3 = (uint32_t)__shfl((int)bits, 4 * lane + 3);
    const int64_t w = (c + u) * (kRowChunk / 64) + lane;
    if (lane < kRowChunk / 64 && w < words) row_out[w] = g0 | (g1 << 16) | (g2 << 32) | (g3 << 48);
  }
}

// Rows of consecutive bytes.  Without ranges a work item is PASS chunks of a
// row; with ranges it is a whole row (its span is then one wave's), written
// to ranges[2 row], ranges[2 row + 1].
template <int PASS, bool RANGES>
__global__ void __launch_bounds__(64 * kPackWaves) fa_pack_mask_rows_kernel(
    const uint8_t* __restrict__ mask, int64_t heads, int64_t rows, int64_t cols, int64_t sb,
    int64_t sh, int64_t sq, int64_t words, int64_t spans, int64_t total,
    uint64_t* __restrict__ out, int32_t* __restrict__ ranges) {
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t)blockIdx.x * kPackWaves + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * kPackWaves;
  for (int64_t it = wave0; it < total; it += nwaves) {  // wave-uniform
    const int64_t row = RANGES ? it : it / spans;  // (b, h, i) flattened
    const int64_t i = row % rows;
    const int64_t bh = row / rows;
    const uint8_t* rp = mask + (bh / heads) * sb + (bh % heads) * sh + i * sq;
    int lo = (int)cols, hi = 0, cnt = 0;
    if constexpr (RANGES) {
      for (int64_t sp = 0; sp < spans; ++sp)
        pack_chunks<PASS, true>(rp, sp * PASS, cols, words, out + row * words, lane, lo, hi, cnt);
      reduce_span(lo, hi, cnt);
      if (lane == 0) {
        ranges[2 * row] = range_first(lo, hi, cnt, cols);
        ranges[2 * row + 1] = hi;
      }
    } else {
      pack_chunks<PASS, false>(rp, (it - row * spans) * PASS, cols, words, out + row * words,
                               lane, lo, hi, cnt);
    }
  }
}

// Other key strides: one wave per word (or, with ranges, per row), lane k
// reading element 64 w + k of the row, a ballot is the word.
template <bool RANGES>
__global__ void __launch_bounds__(64 * kPackWaves) fa_pack_mask_kernel(
    const uint8_t* __restrict__ mask, int64_t heads, int64_t rows, int64_t cols, int64_t sb,
    int64_t sh, int64_t sq, int64_t sk, int64_t words, int64_t total, uint64_t* __restrict__ out,
    int32_t* __restrict__ ranges) {
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t)blockIdx.x * kPackWaves + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * kPackWaves;
  for (int64_t it = wave0; it < total; it += nwaves) {
    const int64_t row = RANGES ? it : it / words;  // (b, h, i) flattened
    const int64_t i = row % rows;
    const int64_t bh = row / rows;
    const uint8_t* rp = mask + (bh / heads) * sb + (bh % heads) * sh + i * sq;
    const int64_t w0 = RANGES ? 0 : it - row * words;
    const int64_t w1 = RANGES ? words : w0 + 1;
    int lo = (int)cols, hi = 0, cnt = 0;  // wave-uniform (from ballots)
    for (int64_t w = w0; w < w1; ++w) {
      const int64_t key = 64 * w + lane;
      const bool visible = key < cols && rp[key * sk] != 0;
      const uint64_t bits = __builtin_amdgcn_ballot_w64(visible);
      if (lane == 0) out[row * words + w] = bits;
      if (RANGES && bits != 0) {
        lo = min(lo, (int)(64 * w) + (int)__builtin_ctzll(bits));
        hi = max(hi, (int)(64 * w) + 64 - (int)__builtin_clzll(bits));
        cnt += __builtin_popcountll(bits);
      }
    }
    if (RANGES && lane == 0) {
      ranges[2 * row] = range_first(lo, hi, cnt, cols);
      ranges[2 * row + 1] = hi;
    }
  }
}

}  // namespace

int launch_pack_mask(const uint8_t* mask, int64_t batch, int64_t heads, int64_t rows,
                     int64_t cols, int64_t sb, int64_t sh, int64_t sq, int64_t sk,
                     uint64_t* out, int32_t* ranges, hipStream_t stream) {
  const int64_t words = (cols + 63) / 64;
  const int64_t nrows = batch * heads * rows;
  if (nrows == 0 || words == 0) return 0;
  auto grid_of = [](int64_t items) {
    const int64_t blocks = (items + kPackWaves - 1) / kPackWaves;
    return dim3((unsigned)(blocks > 4096 ? 4096 : blocks));  // the waves stride over the rest
  };
  const dim3 block(64 * kPackWaves);
  if (sk == 1) {
    // Chunks per pass: two when the row fills them (four measured no faster).
    auto run = [&](auto pass_c) {
      constexpr int PASS = decltype(pass_c)::value;
      const int64_t spans = (cols + kRowChunk * PASS - 1) / (kRowChunk * PASS);
      if (ranges != nullptr)
        hipLaunchKernelGGL((fa_pack_mask_rows_kernel<PASS, true>), grid_of(nrows), block, 0,
                           stream, mask, heads, rows, cols, sb, sh, sq, words, spans, nrows, out,
                           ranges);
      else
        hipLaunchKernelGGL((fa_pack_mask_rows_kernel<PASS, false>), grid_of(nrows * spans), block,
                           0, stream, mask, heads, rows, cols, sb, sh, sq, words, spans,
                           nrows * spans, out, ranges);
    };
    if (cols > kRowChunk) run(std::integral_constant<int, 2>{});
    else run(std::integral_constant<int, 1>{});
    return 0;
  }
  if (ranges != nullptr)
    hipLaunchKernelGGL((fa_pack_mask_kernel<true>), grid_of(nrows), block, 0, stream, mask, heads,
                       rows, cols, sb, sh, sq, sk, words, nrows, out, ranges);
  else
    hipLaunchKernelGGL((fa_pack_mask_kernel<false>), grid_of(nrows * words), block, 0, stream,
                       mask, heads, rows, cols, sb, sh, sq, sk, words, nrows * words, out, ranges);
  return 0;
}

}  // namespace fa
