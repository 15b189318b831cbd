// quantW packing on the device (load time).
//
// Reference: src/core/weights/quantPack.ts:12-28 (packQuantW), layout
// src/core/kernels/quantCommon.ts:8-31. Input: E experts, each a row-major
// output-first [n, k] matrix of signed values (torch's Linear layout, as a
// checkpoint stores it), experts back to back. Output: the experts' quantW
// words concatenated expert-major, i.e. the words of the logical [E·k, n]
// weight the expert ops take.
//
// One thread per output word. A tile (4 columns × 4 rows of one expert)
// holds 16·bits bits; for int8 word c of the tile is column c's 4 rows, for
// int4 word j holds columns 2j and 2j+1. Each thread reads its columns' 4
// consecutive row bytes (one 32-bit load per column: k is a multiple of 4).
#include "moe_internal.h"

namespace {

__global__ void k_pack_quantw(const int8_t *__restrict__ ints, int64_t E, int k, int n, int bits,
                              uint32_t *__restrict__ words) {
  const int words_per_tile = bits / 2;  // 16·bits / 32
  const int64_t tiles = E * (int64_t)(n / 4) * (k / 4);
  const int64_t total = tiles * words_per_tile;
  for (int64_t w = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; w < total;
       w += (int64_t)gridDim.x * blockDim.x) {
    const int64_t tile = w / words_per_tile;
    const int j = (int)(w - tile * words_per_tile);
    const int k4 = (int)(tile % (k / 4));
    const int64_t eu = tile / (k / 4);  // e·(n/4) + unit
    const int unit = (int)(eu % (n / 4));
    const int64_t e = eu / (n / 4);
    const int8_t *src = ints + e * (int64_t)n * k;
    uint32_t out;
    if (bits == 8) {
      const int c = unit * 4 + j;
      out = *(const uint32_t *)(src + (int64_t)c * k + k4 * 4);  // rows r at byte r
    } else {
      out = 0;
      for (int h = 0; h < 2; h++) {
        const int c = unit * 4 + 2 * j + h;
        const uint32_t v = *(const uint32_t *)(src + (int64_t)c * k + k4 * 4);
        for (int r = 0; r < 4; r++) out |= ((v >> (8 * r)) & 0xfu) << (4 * (4 * h + r));
      }
    }
    words[w] = out;
  }
}

}  // namespace

int launch_pack_quantw(const int8_t *ints, int E, int k, int n, int bits, uint32_t *words,
                       hipStream_t s) {
  MOE_NONNULL(ints);
  MOE_NONNULL(words);
  const int64_t total = (int64_t)E * (n / 4) * (k / 4) * (bits / 2);
  if (total == 0) return 0;
  const int64_t want = (total + 255) / 256;
  const int blocks = (int)(want < 65536 ? want : 65536);
  hipLaunchKernelGGL(k_pack_quantw, dim3(blocks), dim3(256), 0, s, ints, (int64_t)E, k, n, bits,
                     words);
  return 0;
}
