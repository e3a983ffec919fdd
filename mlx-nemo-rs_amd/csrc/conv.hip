// The memory-bound middle of the Conformer ConvolutionModule
// (conformer.rs:2197-2291, 2305-2378): GLU over pointwise_conv1's output,
// padding frames zeroed, the depthwise conv over a causal (left) or
// symmetric window whose left context comes from zeros or the streaming
// conv cache, its bias, and -- for BatchNorm -- the inference-mode norm and
// SiLU, all in one pass. pointwise_conv1/2 run on the projection GEMMs.
//
// One workgroup covers kFrames output frames x kChannels channels of one
// batch item. It stages the GLU values of its kFrames + K - 1 window frames
// in LDS (each computed once from the two halves of pointwise_conv1's row,
// 4 channels per lane, several rows' loads in flight at once), then each
// wave convolves 16 frames from LDS. The block that holds the last frame
// tile also writes the new conv cache, the last K - 1 frames of
// [cache; GLU(x)] (conformer.rs:2341-2355), from the same LDS window.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace mhsa {
namespace {

constexpr int kChannels = 64;  // channels per workgroup
constexpr int kFrames = 64;    // output frames per workgroup
constexpr int kUnroll = 4;     // window row groups whose loads are in flight together

// Four consecutive channels of a row, widened to float.
template <typename T>
__device__ __forceinline__ floatx4 load4(const T* p);
template <>
__device__ __forceinline__ floatx4 load4<float>(const float* p) {
  return *reinterpret_cast<const floatx4*>(p);
}
template <>
__device__ __forceinline__ floatx4 load4<bf16>(const bf16* p) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return floatx4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
template <typename T>
__device__ __forceinline__ void store4(T* p, const floatx4& v);
template <>
__device__ __forceinline__ void store4<float>(float* p, const floatx4& v) {
  *reinterpret_cast<floatx4*>(p) = v;
}
template <>
__device__ __forceinline__ void store4<bf16>(bf16* p, const floatx4& v) {
  *reinterpret_cast<bf16x4*>(p) = bf16x4{(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
}

// TIn: pointwise_conv1 output dtype (the GLU is evaluated in it).
// ConvBF16: the depthwise conv and everything after it store bf16 (else f32).
// Lane l of a wave owns channels c0 + 4 (l % 16) + [0, 4) of window row /
// output frame group l / 16, so every access moves 4 channels (8 or 16 bytes)
// and 16 lanes cover a row's 64 channels contiguously.
template <typename TIn, bool ConvBF16>
__global__ __launch_bounds__(256) void conv_glu_dw_kernel(ConvParams p) {
#pragma clang fp contract(off)
  using TC = typename std::conditional<ConvBF16, bf16, float>::type;
  extern __shared__ floatx4 win[];  // [kFrames + K - 1][kChannels / 4]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane & 15, sub = lane >> 4;  // 4-channel group, row / frame within a group of 4
  const int c0 = blockIdx.x * kChannels, c = c0 + 4 * q;
  const int t0 = blockIdx.y * kFrames;
  const int b = blockIdx.z;
  const int T = p.T, D = p.D, K = p.K, C = K - 1;
  const int W = kFrames + K - 1;
  const int len = p.len[b];
  const TIn* g = static_cast<const TIn*>(p.g) + (int64_t)b * T * 2 * D;
  const float* cache = p.cache_in ? p.cache_in + ((int64_t)b * D + c) * C : nullptr;  // channel c, c+1.. at +C

  // GLU of every window frame (conformer.rs:2221-2231, 2319-2336): a *
  // sigmoid(b) with both results stored in TIn; padding frames (>= len) and
  // frames past T are zero; frames before 0 read the cache or are zero.
  // Rows 16 i + 4 wave + sub; kUnroll row groups load before any is used.
  for (int r0 = 0; r0 < W; r0 += 16 * kUnroll) {
    floatx4 av[kUnroll], gv[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int s = t0 - p.left + r0 + 16 * u + 4 * wave + sub;
      av[u] = floatx4{0.f, 0.f, 0.f, 0.f};
      gv[u] = floatx4{0.f, 0.f, 0.f, 0.f};
      if (s >= 0 && s < T && s < len) {
        const TIn* row = g + (int64_t)s * 2 * D;
        av[u] = load4(row + c);
        gv[u] = load4(row + D + c);
      } else if (s < 0 && cache && s >= -C) {
        av[u] = floatx4{cache[C + s], cache[C + C + s], cache[2 * C + C + s], cache[3 * C + C + s]};
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int r = r0 + 16 * u + 4 * wave + sub;
      const int s = t0 - p.left + r;
      if (r < W) {
        floatx4 v = av[u];  // the cached value itself, or zero
        if (s >= 0 && s < T && s < len) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = round_to<TIn>(av[u][e] * sigmoid_value<TIn>(gv[u][e]));
        }
        win[r * (kChannels / 4) + q] = v;
      }
    }
  }
  __syncthreads();

  // Depthwise conv (cross-correlation, weights [K, D] channel-fastest) for
  // frames wave * 16 + 4 i + sub, stored in the conv dtype, then the bias
  // add stored.
  floatx4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int f0 = 16 * wave + sub;
  for (int k = 0; k < K; ++k) {
    const floatx4 wk = *reinterpret_cast<const floatx4*>(p.w + (int64_t)k * D + c);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const floatx4 x = win[(f0 + 4 * i + k) * (kChannels / 4) + q];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][e] = __builtin_fmaf(wk[e], x[e], acc[i][e]);
    }
  }
  const floatx4 bias = p.bias ? *reinterpret_cast<const floatx4*>(p.bias + c) : floatx4{0.f, 0.f, 0.f, 0.f};
  floatx4 mean{}, inv{}, gw{}, gb{};
  if (p.bn) {
    mean = *reinterpret_cast<const floatx4*>(p.bn + c);
    inv = *reinterpret_cast<const floatx4*>(p.bn + D + c);
    gw = *reinterpret_cast<const floatx4*>(p.bn + 2 * D + c);
    gb = *reinterpret_cast<const floatx4*>(p.bn + 3 * D + c);
  }
  TC* y = static_cast<TC*>(p.y) + (int64_t)b * T * D;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = t0 + f0 + 4 * i;
    if (t >= T) break;
    floatx4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float x = round_to<TC>(acc[i][e]);
      if (p.bias) x = round_to<TC>(x + bias[e]);
      if (p.bn) {
        // BatchNorm in inference mode (conformer.rs:2157-2163): (x - mean) *
        // rsqrt(var + eps), then weight * x + bias, each op stored; the
        // per-channel rsqrt term is precomputed in the parameter dtype.
        x = round_to<TC>(x - mean[e]);
        x = round_to<TC>(x * inv[e]);
        x = round_to<TC>(gw[e] * x);
        x = round_to<TC>(x + gb[e]);
        x = silu_value<TC>(x);  // conformer.rs:2269
      }
      v[e] = x;
    }
    store4(y + (int64_t)t * D + c, v);
  }

  // New conv cache: frames T - C .. T - 1 of the [cache; GLU] sequence, held
  // in this (the last) frame tile's window at rows T - t0 + j.
  if (p.cache_out && t0 + kFrames >= T) {
    float* out = p.cache_out + ((int64_t)b * D + c) * C;
    for (int j = 4 * wave + sub; j < C; j += 16) {
      const floatx4 v = win[(T - t0 + j) * (kChannels / 4) + q];
#pragma unroll
      for (int e = 0; e < 4; ++e) out[e * C + j] = v[e];
    }
  }
}

template <typename TIn, bool ConvBF16>
hipError_t conv_launch(const ConvParams& p, int nb, hipStream_t s) {
  const size_t lds = (size_t)(kFrames + p.K - 1) * kChannels * sizeof(float);  // 48 KB at K = 129
  dim3 grid(p.D / kChannels, (p.T + kFrames - 1) / kFrames, nb);
  hipLaunchKernelGGL((conv_glu_dw_kernel<TIn, ConvBF16>), grid, dim3(256), lds, s, p);
  return hipGetLastError();
}

}  // namespace

hipError_t conv_glu_depthwise(DType glu_dt, DType conv_dt, const ConvParams& p, int nbatch, hipStream_t s) {
  if (nbatch <= 0 || p.T <= 0) return hipSuccess;
  if (nbatch > kMaxBatch || p.D <= 0 || p.D % kChannels || p.K < 1 || p.K > kMaxConvKernel || p.left < 0 ||
      p.left > p.K - 1 || !p.g || !p.y || !p.w)
    return hipErrorInvalidValue;
  // the cache supplies exactly the K - 1 frames before frame 0 (causal window)
  if ((p.cache_in || p.cache_out) && p.left != p.K - 1) return hipErrorInvalidValue;
  if (glu_dt == kF32 && conv_dt == kF32) return conv_launch<float, false>(p, nbatch, s);
  if (glu_dt == kBF16 && conv_dt == kBF16) return conv_launch<bf16, true>(p, nbatch, s);
  if (glu_dt == kBF16 && conv_dt == kF32) return conv_launch<bf16, false>(p, nbatch, s);
  return hipErrorInvalidValue;  // f32 GLU never feeds a bf16 conv
}

int conv_frame_tile() { return kFrames; }

}  // namespace mhsa
