// The neuron-major permutation of the 4-bit down projections, on the device.
//
// hsd/layout.py:34-50 expands every nibble to a uint32, swaps axes and repacks (an 8x
// transient, done 16 experts at a time). Here a permutation is a pure 8x8 nibble-block
// transpose: the 8 words w[8*wo + n, cw] (n = 0..7) hold exactly the nibbles that the 8
// words out[8*cw + j, wo] (j = 0..7) hold, transposed. One thread transposes such a
// block in registers with three block-swap stages (4x4, 2x2, 1x1 nibble blocks); a
// workgroup stages a 32x32 tile of blocks through LDS so that both the reads (rows of
// the input) and the writes (rows of the output) are 128-byte coalesced. No transient
// memory at all; out-of-place; self-inverse.
#include "hsd_common.h"

namespace hsd {

namespace {

constexpr int kTile = 32;      // blocks per tile side: 32 input words x 32 output words
constexpr int kThreads = 256;

// In-register transpose of the 8x8 nibble matrix M[n][j] = nibble j of v[n].
__device__ __forceinline__ void transpose8x8_nibbles(uint32_t v[8]) {
#pragma unroll
  for (int n = 0; n < 4; ++n) {  // swap the off-diagonal 4x4 blocks
    const uint32_t a = v[n], b = v[n + 4];
    v[n] = (a & 0x0000FFFFu) | (b << 16);
    v[n + 4] = (a >> 16) | (b & 0xFFFF0000u);
  }
#pragma unroll
  for (int base = 0; base < 8; base += 4) {  // 2x2 blocks inside each 4x4 half
#pragma unroll
    for (int n = base; n < base + 2; ++n) {
      const uint32_t a = v[n], b = v[n + 2];
      v[n] = (a & 0x00FF00FFu) | ((b << 8) & 0xFF00FF00u);
      v[n + 2] = ((a >> 8) & 0x00FF00FFu) | (b & 0xFF00FF00u);
    }
  }
#pragma unroll
  for (int n = 0; n < 8; n += 2) {  // single nibbles inside each 2x2
    const uint32_t a = v[n], b = v[n + 1];
    v[n] = (a & 0x0F0F0F0Fu) | ((b << 4) & 0xF0F0F0F0u);
    v[n + 1] = ((a >> 4) & 0x0F0F0F0Fu) | (b & 0xF0F0F0F0u);
  }
}

// w [batch, R, CW] -> out [batch, 8*CW, R/8]
__global__ __launch_bounds__(kThreads) void k_permute_nibbles(const uint32_t* __restrict__ w,
                                                              uint32_t* __restrict__ out,
                                                              int64_t R, int64_t CW,
                                                              int tiles_cw) {
  __shared__ uint32_t tileT[8 * kTile * kTile];  // [8*cw_l + j][wo_l ^ cw_l]
  const int64_t RW = R / 8;
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t cw0 = (int64_t)(blockIdx.x % tiles_cw) * kTile;
  const int64_t wo0 = (int64_t)(blockIdx.x / tiles_cw) * kTile;
  const uint32_t* src = w + b * R * CW;
  uint32_t* dst = out + b * (8 * CW) * RW;

#pragma unroll
  for (int i = 0; i < (kTile * kTile) / kThreads; ++i) {
    const int bi = tid + kThreads * i;
    const int cw_l = bi & (kTile - 1), wo_l = bi / kTile;
    const int64_t cw = cw0 + cw_l, wo = wo0 + wo_l;
    uint32_t v[8];
    if (cw < CW && wo < RW) {
#pragma unroll
      for (int n = 0; n < 8; ++n) v[n] = src[(8 * wo + n) * CW + cw];
      transpose8x8_nibbles(v);
#pragma unroll
      for (int j = 0; j < 8; ++j) tileT[(8 * cw_l + j) * kTile + (wo_l ^ cw_l)] = v[j];
    }
  }
  __syncthreads();
  const int wo_l = tid & (kTile - 1);
#pragma unroll 4
  for (int row = tid / kTile; row < 8 * kTile; row += kThreads / kTile) {
    const int cw_l = row >> 3;
    const int64_t orow = 8 * cw0 + row, wo = wo0 + wo_l;
    if (cw0 + cw_l < CW && wo < RW) dst[orow * RW + wo] = tileT[row * kTile + (wo_l ^ cw_l)];
  }
}

constexpr int kT16 = 64;
// in [batch, R, C] -> out [batch, C, R], 16-bit elements.
__global__ __launch_bounds__(kThreads) void k_transpose_u16(const uint16_t* __restrict__ in,
                                                            uint16_t* __restrict__ out, int64_t R,
                                                            int64_t C, int tiles_c) {
  __shared__ uint32_t tile[kT16][kT16 + 1];
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t c0 = (int64_t)(blockIdx.x % tiles_c) * kT16;
  const int64_t r0 = (int64_t)(blockIdx.x / tiles_c) * kT16;
  const uint16_t* src = in + b * R * C;
  uint16_t* dst = out + b * R * C;
  const int lc = tid & (kT16 - 1);
  for (int lr = tid / kT16; lr < kT16; lr += kThreads / kT16) {
    const int64_t r = r0 + lr, c = c0 + lc;
    if (r < R && c < C) tile[lr][lc] = src[r * C + c];
  }
  __syncthreads();
  for (int lr = tid / kT16; lr < kT16; lr += kThreads / kT16) {
    const int64_t c = c0 + lr, r = r0 + lc;  // output row c, column r
    if (r < R && c < C) dst[c * R + r] = (uint16_t)tile[lc][lr];
  }
}

}  // namespace
}  // namespace hsd

using namespace hsd;

extern "C" int hsd_permute_nibbles(const uint32_t* w, uint32_t* out, int64_t batch, int64_t rows,
                                   int64_t words, void* stream) {
  if (!w || !out) return set_error(HSD_ERR_ARG, "hsd_permute_nibbles: null pointer");
  if (batch < 0 || rows < 0 || words < 0 || rows % 8)
    return set_error(HSD_ERR_SHAPE, "hsd_permute_nibbles: rows (%lld) must be a multiple of 8",
                     (long long)rows);
  if (batch > 65535) return set_error(HSD_ERR_SHAPE, "hsd_permute_nibbles: batch > 65535");
  if (batch == 0 || rows == 0 || words == 0) return HSD_OK;
  const int64_t tcw = (words + kTile - 1) / kTile, two = (rows / 8 + kTile - 1) / kTile;
  if (tcw * two > 0x7FFFFFFF) return set_error(HSD_ERR_SHAPE, "hsd_permute_nibbles: too large");
  dim3 grid((unsigned)(tcw * two), (unsigned)batch);
  hipLaunchKernelGGL(k_permute_nibbles, grid, dim3(kThreads), 0, as_stream(stream), w, out, rows,
                     words, (int)tcw);
  return check_launch("hsd_permute_nibbles");
}

extern "C" int hsd_transpose_u16(const uint16_t* in, uint16_t* out, int64_t batch, int64_t rows,
                                 int64_t cols, void* stream) {
  if (!in || !out) return set_error(HSD_ERR_ARG, "hsd_transpose_u16: null pointer");
  if (batch < 0 || rows < 0 || cols < 0) return set_error(HSD_ERR_SHAPE, "hsd_transpose_u16: negative size");
  if (batch > 65535) return set_error(HSD_ERR_SHAPE, "hsd_transpose_u16: batch > 65535");
  if (batch == 0 || rows == 0 || cols == 0) return HSD_OK;
  const int64_t tc = (cols + kT16 - 1) / kT16, tr = (rows + kT16 - 1) / kT16;
  if (tc * tr > 0x7FFFFFFF) return set_error(HSD_ERR_SHAPE, "hsd_transpose_u16: too large");
  dim3 grid((unsigned)(tc * tr), (unsigned)batch);
  hipLaunchKernelGGL(k_transpose_u16, grid, dim3(kThreads), 0, as_stream(stream), in, out, rows,
                     cols, (int)tc);
  return check_launch("hsd_transpose_u16");
}
