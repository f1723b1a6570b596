// Boolean attention mask -> packed bit rows.
//
// The fused kernels read an explicit mask as bits: word w of row (b, h, i)
// holds keys [64 w, 64 w + 64), bit k set <=> key 64 w + k is visible.  A
// 64-key prefill tile is then one 8-byte load per lane (its query row), and a
// 32-key decode tile half of one, instead of 64 (or 32) byte loads.
//
// One wave builds one word per iteration: lane k reads element 64 w + k of
// the row (64 consecutive bytes when the key stride is 1) and a ballot over
// the wave is the word.  The waves stride over all words of the output.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa_internal.h"

namespace fa {
namespace {

constexpr int kPackWaves = 4;

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
  const int64_t total = batch * heads * rows * words;
  if (total == 0) return 0;
  int64_t blocks = (total + kPackWaves - 1) / kPackWaves;
  if (blocks > 4096) blocks = 4096;  // the waves stride over the rest
  hipLaunchKernelGGL(fa_pack_mask_kernel, dim3((unsigned)blocks), dim3(64 * kPackWaves), 0,
                     stream, mask, heads, rows, cols, sb, sh, sq, sk, words, total, out);
  return 0;
}

}  // namespace fa
