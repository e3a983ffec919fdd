// Small kernels around the attention path: the pre-LayerNorm of the MHSA
// sublayer (conformer.rs:1749), the streaming cache ring copies
// (attention.rs:650, 670-684; conformer.rs:983-1016) and the dequantised
// weight export used by the bit-exact checks.
#include <algorithm>

#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"
#include "quant.hpp"

namespace mhsa {
namespace {

// One wave per row; two-pass statistics in fp32 from registers.
template <typename T, int VPL>
__global__ __launch_bounds__(256) void ln_kernel(const T* x, T* y, const float* gamma, const float* beta,
                                                 float eps, int rows, int D, int act) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const T* xr = x + (int64_t)row * D;
  float v[VPL];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + 64 * i;
    v[i] = c < D ? (float)xr[c] : 0.f;
    s += v[i];
  }
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  const float mean = s / (float)D;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + 64 * i;
    const float d = c < D ? v[i] - mean : 0.f;
    q += d * d;
  }
  for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o, 64);
  const float rstd = rsqrtf(q / (float)D + eps);
  T* yr = y + (int64_t)row * D;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = lane + 64 * i;
    if (c < D) {
      float t = (v[i] - mean) * rstd;
      if (gamma) t *= gamma[c];
      if (beta) t += beta[c];
      if (act == kActSilu) t = silu_value<T>(round_to<T>(t));
      yr[c] = from_float<T>(t);
    }
  }
}

// The same with 16-byte accesses: lane l holds chunks l + 64 j of the row
// (D a multiple of 64 chunks), gamma and beta read as float4.
template <typename T, int NCH, bool GAMMA, bool BETA>
__global__ __launch_bounds__(256) void ln_vec_kernel(const T* x, T* y, const float* gamma, const float* beta,
                                                     float eps, int rows, int D, int act) {
  constexpr int E = 16 / sizeof(T);  // elements per chunk
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const T* xr = x + (int64_t)row * D;
  // The row's chunks, then gamma and beta of the same columns (they do not
  // depend on the row), all issued before the first wait so that their
  // latencies overlap; one instantiation per affine form keeps the loads
  // free of branches, which would split them into separate waits.
  u32x4 raw[NCH];
#pragma unroll
  for (int j = 0; j < NCH; ++j) raw[j] = *reinterpret_cast<const u32x4*>(xr + (lane + 64 * j) * E);
  floatx4 g4[NCH][E / 4], b4[NCH][E / 4];
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int e4 = 0; e4 < E / 4; ++e4) {
      const int c0 = (lane + 64 * j) * E + 4 * e4;
      g4[j][e4] = GAMMA ? *reinterpret_cast<const floatx4*>(gamma + c0) : floatx4{1.f, 1.f, 1.f, 1.f};
      b4[j][e4] = BETA ? *reinterpret_cast<const floatx4*>(beta + c0) : floatx4{0.f, 0.f, 0.f, 0.f};
    }
  __builtin_amdgcn_sched_barrier(0);
  float v[NCH][E];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const T* t = reinterpret_cast<const T*>(&raw[j]);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      v[j][e] = (float)t[e];
      s += v[j][e];
    }
  }
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  const float mean = s / (float)D;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float d = v[j][e] - mean;
      q += d * d;
    }
  for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o, 64);
  const float rstd = rsqrtf(q / (float)D + eps);
  T* yr = y + (int64_t)row * D;
  // (the activation test taken once, outside the element loops)
  auto emit = [&](auto silu) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c0 = (lane + 64 * j) * E;
      T out[E];
#pragma unroll
      for (int e4 = 0; e4 < E; e4 += 4) {
        const floatx4 g = g4[j][e4 / 4], b = b4[j][e4 / 4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float t = (v[j][e4 + e] - mean) * rstd;
          if (GAMMA) t *= g[e];
          if (BETA) t += b[e];
          if constexpr (decltype(silu)::value) t = silu_value<T>(round_to<T>(t));
          out[e4 + e] = from_float<T>(t);
        }
      }
      *reinterpret_cast<u32x4*>(yr + c0) = *reinterpret_cast<const u32x4*>(out);
    }
  };
  if (act == kActSilu) emit(std::true_type{});
  else emit(std::false_type{});
}

template <typename T, int NCH>
hipError_t ln_vec_launch(dim3 grid, const T* x, T* y, const float* g, const float* b, float eps, int rows, int D,
                         int act, hipStream_t s) {
  if (g && b) hipLaunchKernelGGL((ln_vec_kernel<T, NCH, true, true>), grid, dim3(256), 0, s, x, y, g, b, eps, rows, D, act);
  else if (g) hipLaunchKernelGGL((ln_vec_kernel<T, NCH, true, false>), grid, dim3(256), 0, s, x, y, g, b, eps, rows, D, act);
  else if (b) hipLaunchKernelGGL((ln_vec_kernel<T, NCH, false, true>), grid, dim3(256), 0, s, x, y, g, b, eps, rows, D, act);
  else hipLaunchKernelGGL((ln_vec_kernel<T, NCH, false, false>), grid, dim3(256), 0, s, x, y, g, b, eps, rows, D, act);
  return hipGetLastError();
}

template <typename T>
hipError_t ln_launch(const void* x, void* y, const float* g, const float* b, float eps, int rows, int D, int act,
                     hipStream_t s) {
  dim3 grid((rows + 3) / 4);
  constexpr int E = 16 / sizeof(T);
  const bool aligned = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y) |
                         reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(b)) & 15) == 0;
  if (aligned && D % (64 * E) == 0) {
    switch (D / (64 * E)) {
      case 1:
        return ln_vec_launch<T, 1>(grid, (const T*)x, (T*)y, g, b, eps, rows, D, act, s);
      case 2:
        return ln_vec_launch<T, 2>(grid, (const T*)x, (T*)y, g, b, eps, rows, D, act, s);
      case 4:
        return ln_vec_launch<T, 4>(grid, (const T*)x, (T*)y, g, b, eps, rows, D, act, s);
      default:
        break;
    }
  }
  if (D <= 512)
    hipLaunchKernelGGL((ln_kernel<T, 8>), grid, dim3(256), 0, s, (const T*)x, (T*)y, g, b, eps, rows, D, act);
  else if (D <= 1024)
    hipLaunchKernelGGL((ln_kernel<T, 16>), grid, dim3(256), 0, s, (const T*)x, (T*)y, g, b, eps, rows, D, act);
  else
    hipLaunchKernelGGL((ln_kernel<T, 32>), grid, dim3(256), 0, s, (const T*)x, (T*)y, g, b, eps, rows, D, act);
  return hipGetLastError();
}

// 16-byte chunks; `to_ring` selects the copy direction.
__global__ void ring_copy_kernel(const char* src, char* dst, int B, int n, int row_bytes, int R, int64_t ld_bytes,
                                 int off, bool to_ring) {
  const int cpr = row_bytes / 16;
  const int64_t total = (int64_t)B * n * cpr;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(e % cpr);
    const int64_t bt = e / cpr;
    const int t = (int)(bt % n), b = (int)(bt / n);
    const int64_t lin = ((int64_t)b * n + t) * row_bytes + c * 16;
    const int64_t ring = ((int64_t)b * R + (off + t) % R) * ld_bytes + c * 16;
    if (to_ring)
      *reinterpret_cast<u32x4*>(dst + ring) = *reinterpret_cast<const u32x4*>(src + lin);
    else
      *reinterpret_cast<u32x4*>(dst + lin) = *reinterpret_cast<const u32x4*>(src + ring);
  }
}

template <typename T>
__global__ void dequant_kernel(const uint32_t* w, const float* sb, float* out, int N, int K) {
  const int chunks = K / 16;
  const int64_t total = (int64_t)N * chunks;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int n = (int)(e / chunks), k = (int)(e % chunks) * 16;
    const u32x4 q = *reinterpret_cast<const u32x4*>(reinterpret_cast<const unsigned char*>(w) + (int64_t)n * K + k);
    const floatx2 s = *reinterpret_cast<const floatx2*>(sb + 2 * ((int64_t)n * (K / 64) + k / 64));
    T vals[16];
    dequant16<T>(q, s.x, s.y, vals);
#pragma unroll
    for (int i = 0; i < 16; ++i) out[(int64_t)n * K + k + i] = (float)vals[i];
  }
}

unsigned grid_for(int64_t n) { return (unsigned)std::min<int64_t>(std::max<int64_t>((n + 255) / 256, 1), 8192); }

__global__ void zero_kernel(u32x4* p, int64_t n16, uint8_t* tail, int ntail) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = u32x4{0u, 0u, 0u, 0u};
  if (blockIdx.x == 0 && (int)threadIdx.x < ntail) tail[threadIdx.x] = 0;
}

__global__ void widen_kernel(const bf16x8* src, floatx4* dst, int64_t n8) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n8; i += (int64_t)gridDim.x * blockDim.x) {
    const bf16x8 v = src[i];
    dst[2 * i] = floatx4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
    dst[2 * i + 1] = floatx4{(float)v[4], (float)v[5], (float)v[6], (float)v[7]};
  }
}

}  // namespace

hipError_t widen_bf16(const void* src, float* dst, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  if (!src || !dst || n % 8 || ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15))
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(widen_kernel, dim3(grid_for(n / 8)), dim3(256), 0, s, static_cast<const bf16x8*>(src),
                     reinterpret_cast<floatx4*>(dst), n / 8);
  return hipGetLastError();
}

hipError_t fill_zero(void* ptr, size_t bytes, hipStream_t s) {
  if (!bytes) return hipSuccess;
  if (!ptr || (reinterpret_cast<uintptr_t>(ptr) & 15)) return hipErrorInvalidValue;
  const int64_t n16 = (int64_t)(bytes / 16);
  const int ntail = (int)(bytes % 16);
  const int64_t blocks = std::min<int64_t>((n16 + 255) / 256 + 1, 4096);
  hipLaunchKernelGGL(zero_kernel, dim3((unsigned)blocks), dim3(256), 0, s, static_cast<u32x4*>(ptr), n16,
                     static_cast<uint8_t*>(ptr) + n16 * 16, ntail);
  return hipGetLastError();
}

hipError_t layer_norm(DType dt, const void* x, void* y, const float* gamma, const float* beta, float eps, int rows,
                      int D, hipStream_t s, int act) {
  if (rows <= 0) return hipSuccess;
  if (!x || !y || D <= 0 || D > kMaxLayerNormDim) return hipErrorInvalidValue;
  return dt == kF32 ? ln_launch<float>(x, y, gamma, beta, eps, rows, D, act, s)
                    : ln_launch<bf16>(x, y, gamma, beta, eps, rows, D, act, s);
}

static hipError_t ring_copy(DType dt, const void* src, void* dst, int B, int n, int D, int R, int64_t ld, int off,
                            bool to_ring, hipStream_t s) {
  if (B <= 0 || n <= 0) return hipSuccess;
  const int es = dtype_size(dt);
  if (!src || !dst || R <= 0 || off < 0 || (D * es) % 16 || (ld * es) % 16 || ld < D) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) return hipErrorInvalidValue;
  const int64_t total = (int64_t)B * n * (D * es / 16);
  hipLaunchKernelGGL(ring_copy_kernel, dim3(grid_for(total)), dim3(256), 0, s, (const char*)src, (char*)dst, B, n,
                     D * es, R, ld * es, off, to_ring);
  return hipGetLastError();
}

hipError_t ring_write(DType dt, const void* src, void* ring, int B, int n, int D, int R, int64_t ld, int off,
                      hipStream_t s) {
  return ring_copy(dt, src, ring, B, n, D, R, ld, off, true, s);
}

hipError_t ring_read(DType dt, const void* ring, void* dst, int B, int n, int D, int R, int64_t ld, int off,
                     hipStream_t s) {
  return ring_copy(dt, ring, dst, B, n, D, R, ld, off, false, s);
}

hipError_t dequant_export(DType dt, const uint32_t* w, const float* sb, float* out, int N, int K, hipStream_t s) {
  if (N <= 0 || K <= 0) return hipSuccess;
  if (!w || !sb || !out || K % 64) return hipErrorInvalidValue;
  const int64_t total = (int64_t)N * (K / 16);
  if (dt == kF32)
    hipLaunchKernelGGL(dequant_kernel<float>, dim3(grid_for(total)), dim3(256), 0, s, w, sb, out, N, K);
  else
    hipLaunchKernelGGL(dequant_kernel<bf16>, dim3(grid_for(total)), dim3(256), 0, s, w, sb, out, N, K);
  return hipGetLastError();
}

}  // namespace mhsa
