// MLX affine 8-bit dequantisation in registers (quantization.rs:1-8, 147-155).
//
// Weight row n holds one u8 code per byte along the input dimension (four
// codes per little-endian u32, lowest byte first). Element k dequantises to
//   W[n][k] = s[n][k/64] * q + b[n][k/64]
// with s, b already cast to the layer dtype's precision. The fp32 product of
// an f16/bf16 scale and an 8-bit code is exact, so the fma below rounds once
// and gives the same fp32 value as a separate multiply and add; the result
// is then stored in the compute dtype (RNE for bf16).
#pragma once

#include "common.hpp"

namespace mhsa {

template <typename T>
__device__ __forceinline__ void dequant16(const u32x4 w, const float s, const float b, T* out) {
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float q = (float)((words[i] >> (8 * j)) & 0xFFu);
      out[4 * i + j] = from_float<T>(__builtin_fmaf(s, q, b));
    }
  }
}

}  // namespace mhsa
