// urb_panel.hpp -- device-side access to panel-layout weights (layout in urb_kernels.hpp).
#pragma once

#include "urb_device.hpp"
#include "urb_kernels.hpp"

namespace urb {

enum { kFmtBF16 = 0, kFmtMXFP4 = 1, kFmtMXFP8 = 2 };

template <int FMT>
__host__ __device__ constexpr size_t panel_row_bytes(size_t K) {
  return FMT == kFmtBF16 ? K * 2 : (FMT == kFmtMXFP4 ? K / 2 : K);
}

// Raw B operands of one lane for one K step.
template <int FMT>
struct BRaw;
template <>
struct BRaw<kFmtBF16> { uint4 q[4]; };
template <>
struct BRaw<kFmtMXFP4> { uint4 q; uint32_t s; };
template <>
struct BRaw<kFmtMXFP8> { uint4 q[2]; uint32_t s; };

// pd = panel data + 16 * lane, ps = panel scales + lane (see the layout in urb_kernels.hpp).
template <int FMT>
__device__ __forceinline__ void load_b(BRaw<FMT>& r, const uint8_t* __restrict__ pd,
                                       const uint8_t* __restrict__ ps, int step) {
  if constexpr (FMT == kFmtBF16) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      r.q[j] = *reinterpret_cast<const uint4*>(pd + (size_t)(4 * step + j) * 1024);
  } else if constexpr (FMT == kFmtMXFP4) {
    r.q = *reinterpret_cast<const uint4*>(pd + (size_t)step * 1024);
    r.s = ps[(size_t)step * 64];
  } else {
    r.q[0] = *reinterpret_cast<const uint4*>(pd + (size_t)(2 * step) * 1024);
    r.q[1] = *reinterpret_cast<const uint4*>(pd + (size_t)(2 * step + 1) * 1024);
    r.s = ps[(size_t)step * 64];
  }
}

}  // namespace urb
