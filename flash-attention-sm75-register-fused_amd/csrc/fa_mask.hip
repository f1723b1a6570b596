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

// PASS consecutive 1024-byte chunks of one row per wave and pass, all loads
// issued before any is used (more bytes in flight per wave, in one stretch of
// the row).
template <int PASS>
__global__ void __launch_bounds__(64 * kPackWaves) fa_pack_mask_rows_kernel(
    const uint8_t* __restrict__ mask, int64_t heads, int64_t rows, int64_t cols, int64_t sb,
    int64_t sh, int64_t sq, int64_t words, int64_t spans, int64_t total,
    uint64_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t)blockIdx.x * kPackWaves + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * kPackWaves;
  for (int64_t it = wave0; it < total; it += nwaves) {  // wave-uniform
    const int64_t row = it / spans;  // (b, h, i) flattened
    const int64_t c = (it - row * spans) * PASS;
    const int64_t i = row % rows;
    const int64_t bh = row / rows;
    const uint8_t* rp = mask + (bh / heads) * sb + (bh % heads) * sh + i * sq;
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
      // Word j of this chunk: the 16-bit groups of lanes 4j .. 4j + 3.
      const uint64_t g0 = (uint32_t)__shfl((int)bits, 4 * lane);
      const uint64_t g1 = (uint32_t)__shfl((int)bits, 4 * lane + 1);
      const uint64_t g2 = (uint32_t)__shfl((int)bits, 4 * lane + 2);
      const uint64_t g3 = (uint32_t)__shfl((int)bits, 4 * lane + 3);
      const int64_t w = (c + u) * (kRowChunk / 64) + lane;
      if (lane < kRowChunk / 64 && w < words)
        out[row * words + w] = g0 | (g1 << 16) | (g2 << 32) | (g3 << 48);
    }
  }
}

__global__ void __launch_bounds__(64 * kPackWaves) fa_pack_mask_kernel(
    const uint8_t* __restrict__ mask, int64_t heads, int64_t rows, int64_t cols, int64_t sb,
    int64_t sh, int64_t sq, int64_t sk, int64_t words, int64_t total, uint64_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t)blockIdx.x * kPackWaves + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * kPackWaves;
  for (int64_t wi = wave0; wi < total; wi += nwaves) {
    const int64_t row = wi / words;       // (b, h, i) flattened
    const int64_t w = wi - row * words;
    const int64_t i = row % rows;
    const int64_t bh = row / rows;
    const int64_t h = bh % heads;
    const int64_t b = bh / heads;
    const int64_t key = 64 * w + lane;
    bool visible = false;
    if (key < cols) visible = mask[b * sb + h * sh + i * sq + key * sk] != 0;
    const uint64_t bits = __builtin_amdgcn_ballot_w64(visible);
    if (lane == 0) out[wi] = bits;
  }
}

}  // namespace

int launch_pack_mask(const uint8_t* mask, int64_t batch, int64_t heads, int64_t rows,
                     int64_t cols, int64_t sb, int64_t sh, int64_t sq, int64_t sk,
                     uint64_t* out, hipStream_t stream) {
  const int64_t words = (cols + 63) / 64;
  const int64_t nrows = batch * heads * rows;
  if (nrows == 0 || words == 0) return 0;
  if (sk == 1) {
    // Chunks per pass: two when the row fills them (four measured no faster).
    auto run = [&](auto pass_c) {
      constexpr int PASS = decltype(pass_c)::value;
      const int64_t spans = (cols + kRowChunk * PASS - 1) / (kRowChunk * PASS);
      const int64_t total = nrows * spans;
      int64_t blocks = (total + kPackWaves - 1) / kPackWaves;
      if (blocks > 4096) blocks = 4096;  // the waves stride over the rest
      hipLaunchKernelGGL(fa_pack_mask_rows_kernel<PASS>, dim3((unsigned)blocks),
                         dim3(64 * kPackWaves), 0, stream, mask, heads, rows, cols, sb, sh, sq,
                         words, spans, total, out);
    };
    if (cols > kRowChunk) run(std::integral_constant<int, 2>{});
    else run(std::integral_constant<int, 1>{});
    return 0;
  }
  const int64_t total = nrows * words;
  int64_t blocks = (total + kPackWaves - 1) / kPackWaves;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fa_pack_mask_kernel, dim3((unsigned)blocks), dim3(64 * kPackWaves), 0,
                     stream, mask, heads, rows, cols, sb, sh, sq, sk, words, total, out);
  return 0;
}

}  // namespace fa
