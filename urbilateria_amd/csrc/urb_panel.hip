// urb_panel.hip -- conversion of row-major packed weights (the checkpoint layout) into the
// panel layout the projection kernels stream (urb_kernels.hpp).  Bytes are moved, never
// re-encoded: a panel-layout matrix holds exactly the bytes of the row-major one.
#include "urb_panel.hpp"

#include <algorithm>

namespace urb {

// One thread per 16-byte unit of the panel-layout matrix.  `rb` = bytes per row; a panel holds
// 16 rows = rb units.
__global__ void pack_data_kernel(int fmt, const uint4* __restrict__ src, uint4* __restrict__ dst,
                                 size_t rb, size_t units) {
  for (size_t u = blockIdx.x * (size_t)blockDim.x + threadIdx.x; u < units;
       u += (size_t)gridDim.x * blockDim.x) {
    const size_t p = u / rb;
    const size_t v = u - p * rb;
    const size_t t = v >> 6;  // slab within the panel
    const int l = (int)(v & 63), ln = l & 15, lq = l >> 4;
    // byte offset of the unit within its row
    const size_t off = fmt == kFmtMXFP8 ? (t >> 1) * 128 + (size_t)lq * 32 + (t & 1) * 16
                                        : t * 64 + (size_t)lq * 16;
    dst[u] = src[((p * 16 + ln) * rb + off) >> 4];
  }
}

// One thread per scale byte.  `nb` = MX blocks per row; a panel holds 16 nb scales.
__global__ void pack_scales_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                   size_t nb, size_t n) {
  for (size_t b = blockIdx.x * (size_t)blockDim.x + threadIdx.x; b < n;
       b += (size_t)gridDim.x * blockDim.x) {
    const size_t p = b / (16 * nb);
    const size_t v = b - p * 16 * nb;
    const size_t s = v >> 6;
    const int l = (int)(v & 63), ln = l & 15, lq = l >> 4;
    dst[b] = src[(p * 16 + ln) * nb + 4 * s + lq];
  }
}

void launch_pack(int fmt, const uint8_t* data, const uint8_t* scales, int rows, int cols,
                 uint8_t* packed, uint8_t* packed_scales, hipStream_t s) {
  const size_t rb = fmt == kFmtBF16 ? (size_t)cols * 2
                                    : (fmt == kFmtMXFP4 ? (size_t)cols / 2 : (size_t)cols);
  const size_t units = (size_t)rows * rb / 16;
  const int blocks = (int)std::min<size_t>((units + 255) / 256, 8192);
  pack_data_kernel<<<blocks, 256, 0, s>>>(fmt, reinterpret_cast<const uint4*>(data),
                                          reinterpret_cast<uint4*>(packed), rb, units);
  if (fmt != kFmtBF16) {
    const size_t nb = (size_t)cols / 32, n = (size_t)rows * nb;
    const int sblocks = (int)std::min<size_t>((n + 255) / 256, 8192);
    pack_scales_kernel<<<sblocks, 256, 0, s>>>(scales, packed_scales, nb, n);
  }
}

}  // namespace urb
