// The memory-bound middle of the Conformer ConvolutionModule
// (conformer.rs:2197-2291, 2305-2378): GLU over pointwise_conv1's output,
// padding frames zeroed, the depthwise conv over a causal (left) or
// symmetric window whose left context comes from zeros or the streaming
// conv cache, its bias, and -- for BatchNorm -- the inference-mode norm and
// SiLU, all in one pass. pointwise_conv1/2 run on the projection GEMMs.
//
// One workgroup covers kFrames output frames x kChannels channels of one
// batch item. It stages the GLU values of its kFrames + K - 1 window frames
// in LDS (each computed once from the two halves of pointwise_conv1's row),
// then each wave convolves 16 frames per channel lane from LDS. The block
// that holds the last frame tile also writes the new conv cache, the last
// K - 1 frames of [cache; GLU(x)] (conformer.rs:2341-2355), from the same
// LDS window.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace mhsa {
namespace {

constexpr int kChannels = 64;               // channels per workgroup (one per lane)
constexpr int kFramesPerWave = 16;
constexpr int kFrames = 4 * kFramesPerWave;  // output frames per workgroup

template <typename TIn>
__device__ __forceinline__ float load_val(const TIn* p) {
  return (float)*p;
}

// TIn: pointwise_conv1 output dtype (the GLU is evaluated in it).
// ConvBF16: the depthwise conv and everything after it store bf16 (else f32).
template <typename TIn, bool ConvBF16>
__global__ __launch_bounds__(256) void conv_glu_dw_kernel(ConvParams p) {
#pragma clang fp contract(off)
  using TOut = typename std::conditional<ConvBF16, bf16, float>::type;
  using TC = typename std::conditional<ConvBF16, bf16, float>::type;
  extern __shared__ float win[];  // [kFrames + K - 1][kChannels]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c0 = blockIdx.x * kChannels, c = c0 + lane;
  const int t0 = blockIdx.y * kFrames;
  const int b = blockIdx.z;
  const int T = p.T, D = p.D, K = p.K, C = K - 1;
  const int W = kFrames + K - 1;
  const int len = p.len[b];
  const TIn* g = static_cast<const TIn*>(p.g) + (int64_t)b * T * 2 * D;
  const float* cache_row = p.cache_in ? p.cache_in + ((int64_t)b * D + c) * C : nullptr;

  // GLU of every window frame (conformer.rs:2221-2231, 2319-2336): a *
  // sigmoid(b) with both results stored in TIn; padding frames (>= len) and
  // frames past T are zero; frames before 0 read the cache or are zero.
  for (int r = wave; r < W; r += 4) {
    const int s = t0 - p.left + r;
    float v = 0.f;
    if (s >= 0 && s < T) {
      if (s < len) {
        const TIn* row = g + (int64_t)s * 2 * D;
        const float a = load_val(row + c), gate = load_val(row + D + c);
        v = round_to<TIn>(a * sigmoid_value<TIn>(gate));
      }
    } else if (s < 0 && cache_row && s >= -C) {
      v = cache_row[C + s];
    }
    win[r * kChannels + lane] = v;
  }
  __syncthreads();

  // Depthwise conv (cross-correlation, weights [K, D] channel-fastest),
  // stored in the conv dtype, then the bias add stored.
  float acc[kFramesPerWave];
#pragma unroll
  for (int i = 0; i < kFramesPerWave; ++i) acc[i] = 0.f;
  const int f0 = wave * kFramesPerWave;
  for (int k = 0; k < K; ++k) {
    const float wk = p.w[(int64_t)k * D + c];
#pragma unroll
    for (int i = 0; i < kFramesPerWave; ++i) acc[i] = __builtin_fmaf(wk, win[(f0 + i + k) * kChannels + lane], acc[i]);
  }
  const float bias = p.bias ? p.bias[c] : 0.f;
  float mean = 0.f, inv = 1.f, gw = 1.f, gb = 0.f;
  if (p.bn) {
    mean = p.bn[c];
    inv = p.bn[D + c];
    gw = p.bn[2 * D + c];
    gb = p.bn[3 * D + c];
  }
  TOut* y = static_cast<TOut*>(p.y) + (int64_t)b * T * D;
#pragma unroll
  for (int i = 0; i < kFramesPerWave; ++i) {
    const int t = t0 + f0 + i;
    if (t >= T) break;
    float v = round_to<TC>(acc[i]);
    if (p.bias) v = round_to<TC>(v + bias);
    if (p.bn) {
      // BatchNorm in inference mode (conformer.rs:2157-2163): (x - mean) *
      // rsqrt(var + eps), then weight * x + bias, each op stored; the
      // per-channel rsqrt term is precomputed in the parameter dtype.
      v = round_to<TC>(v - mean);
      v = round_to<TC>(v * inv);
      v = round_to<TC>(gw * v);
      v = round_to<TC>(v + gb);
      v = silu_value<TC>(v);  // conformer.rs:2269
    }
    y[(int64_t)t * D + c] = from_float<TOut>(v);
  }

  // New conv cache: frames T - C .. T - 1 of the [cache; GLU] sequence, held
  // in this (the last) frame tile's window at rows T - t0 + j.
  if (p.cache_out && t0 + kFrames >= T) {
    float* out_row = p.cache_out + ((int64_t)b * D + c) * C;
    for (int j = wave; j < C; j += 4) out_row[j] = win[(T - t0 + j) * kChannels + lane];
  }
}

template <typename TIn, bool ConvBF16>
hipError_t conv_launch(const ConvParams& p, int nb, hipStream_t s) {
  const size_t lds = (size_t)(kFrames + p.K - 1) * kChannels * sizeof(float);
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
