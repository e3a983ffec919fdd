// Projection GEMMs for the rel-pos MHSA sublayer (linear_q/k/v/out/pos).
//
// Replaces `LinearLayer::forward` (quantization.rs:126-162): y = x W^T + b for
// standard weights and MLX `quantized_matmul(transpose=true, group 64, 8 bit)`
// + b for affine-u8 weights, where the u8 codes are dequantised in registers
// on their way into LDS and feed the same MFMA tiles as dense weights.
//
// Tiling (gfx950): 128x128 output tile per 256-thread workgroup, 2x2 waves of
// 64x64, each wave a 4x4 grid of 16x16 MFMA tiles. One K step moves 128
// bytes per row (64 bf16 or 32 fp32), double-buffered in LDS with a 16-byte
// row pad; the next step's global loads are in flight while the MFMAs of the
// current step run.
#include "common.hpp"
#include "kernels.hpp"
#include "quant.hpp"

namespace mhsa {
namespace {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int NT = 256;
constexpr int ROWB = 128;        // bytes of one tile row per K step
constexpr int PITCH = ROWB + 16; // LDS row pitch (bytes)
constexpr int TILE_BYTES = BM * PITCH;

template <typename T, bool QUANT>
struct BLoad;

// Dense weights: the B tile is loaded exactly like the A tile.
template <typename T>
struct BLoad<T, false> {
  uint4 r[4];
  __device__ void load(const GemmParams& p, int n0, int k0, int tid) {
    const char* W = reinterpret_cast<const char*>(p.W);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + NT * i;
      const int row = c >> 3, cb = (c & 7) * 16;
      r[i] = *reinterpret_cast<const uint4*>(W + ((int64_t)(n0 + row) * p.K + k0) * sizeof(T) + cb);
    }
  }
  __device__ void store(char* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + NT * i;
      const int row = c >> 3, cb = (c & 7) * 16;
      *reinterpret_cast<uint4*>(lds + row * PITCH + cb) = r[i];
    }
  }
};

// Affine u8 weights: ROWB/sizeof(T) codes per row per K step, 16 codes per
// 16-byte load, each load inside one group of 64.
template <typename T>
struct BLoad<T, true> {
  static constexpr int CODES = ROWB / sizeof(T);  // codes per row per step
  static constexpr int CPR = CODES / 16;          // 16-byte chunks per row
  static constexpr int NCH = BN * CPR / NT;       // chunks per thread
  uint4 r[NCH];
  float2 sbv[NCH];
  __device__ void load(const GemmParams& p, int n0, int k0, int tid) {
    const unsigned char* W = reinterpret_cast<const unsigned char*>(p.W);
    const int groups = p.K / 64;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = tid + NT * i;
      const int row = c / CPR, kc = (c % CPR) * 16;
      const int n = n0 + row, k = k0 + kc;
      r[i] = *reinterpret_cast<const uint4*>(W + (int64_t)n * p.K + k);
      sbv[i] = *reinterpret_cast<const float2*>(p.sb + 2 * ((int64_t)n * groups + k / 64));
    }
  }
  __device__ void store(char* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = tid + NT * i;
      const int row = c / CPR, kc = (c % CPR) * 16;
      T vals[16];
      dequant16<T>(r[i], sbv[i].x, sbv[i].y, vals);
      uint4* dst = reinterpret_cast<uint4*>(lds + row * PITCH + kc * (int)sizeof(T));
      const uint4* src = reinterpret_cast<const uint4*>(vals);
#pragma unroll
      for (int j = 0; j < (int)(16 * sizeof(T) / 16); ++j) dst[j] = src[j];
    }
  }
};

template <typename T, bool QUANT>
__global__ __launch_bounds__(NT) void gemm_kernel(const GemmParams p) {
  using F = Frag<T>;
  using frag_t = typename F::type;
  constexpr int BK = ROWB / sizeof(T);
  __shared__ __attribute__((aligned(16))) char smem[2][2][TILE_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int n0 = blockIdx.x * BN;
  const int m0 = blockIdx.y * BM;
  const char* A = reinterpret_cast<const char*>(p.A);

  uint4 ra[4];
  auto load_a = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + NT * i;
      const int row = c >> 3, cb = (c & 7) * 16;
      const bool ok = m0 + row < p.M;
      ra[i] = load16<uint4>(A + ((int64_t)(ok ? m0 + row : 0) * p.lda + k0) * sizeof(T) + cb, ok);
    }
  };
  auto store_a = [&](char* lds) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + NT * i;
      const int row = c >> 3, cb = (c & 7) * 16;
      *reinterpret_cast<uint4*>(lds + row * PITCH + cb) = ra[i];
    }
  };
  BLoad<T, QUANT> rb;

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int nk = p.K / BK;
  load_a(0);
  rb.load(p, n0, 0, tid);
  store_a(smem[0][0]);
  rb.store(smem[0][1], tid);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      load_a((kt + 1) * BK);
      rb.load(p, n0, (kt + 1) * BK, tid);
    }
    const char* la = smem[cur][0];
    const char* lb = smem[cur][1];
#pragma unroll
    for (int kf = 0; kf < BK / F::KSTEP; ++kf) {
      frag_t af[4], bfr[4];
      const int cb = kf * 64 + (lane >> 4) * 16;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        af[t] = *reinterpret_cast<const frag_t*>(la + (wm * 64 + t * 16 + (lane & 15)) * PITCH + cb);
        bfr[t] = *reinterpret_cast<const frag_t*>(lb + (wn * 64 + t * 16 + (lane & 15)) * PITCH + cb);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mma16(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < nk) {
      store_a(smem[cur ^ 1][0]);
      rb.store(smem[cur ^ 1][1], tid);
    }
    __syncthreads();
  }

  // Epilogue, in the reference's op order: round the product, add the bias,
  // round, add the residual, round.
  T* C = reinterpret_cast<T*>(p.C);
  const T* R = reinterpret_cast<const T*>(p.R);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
      if (row >= p.M) continue;
      const int orow = (row / p.seg_rows) * p.seg_stride + (p.ring_off + row % p.seg_rows) % p.ring_len;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = n0 + wn * 64 + j * 16 + (lane & 15);
        float v = round_to<T>(acc[i][j][r]);
        if (p.bias) v = round_to<T>(v + p.bias[col]);
        if (R) v = round_to<T>((float)R[(int64_t)row * p.ldr + col] + v);
        C[(int64_t)orow * p.ldc + col] = from_float<T>(v);
      }
    }
  }
}

template <typename T, bool QUANT>
hipError_t launch(const GemmParams& p, hipStream_t s) {
  dim3 grid(p.N / BN, (p.M + BM - 1) / BM);
  hipLaunchKernelGGL((gemm_kernel<T, QUANT>), grid, dim3(NT), 0, s, p);
  return hipGetLastError();
}

}  // namespace

hipError_t gemm(DType dt, bool quantized, const GemmParams& p, hipStream_t s) {
  const int bk = ROWB / dtype_size(dt);
  if (p.M <= 0) return hipSuccess;
  if (p.N <= 0 || p.N % BN || p.K <= 0 || p.K % bk || (quantized && p.K % 64)) return hipErrorInvalidValue;
  if (!p.A || !p.W || !p.C || (quantized && !p.sb)) return hipErrorInvalidValue;
  if (p.seg_rows <= 0 || p.ring_len <= 0) return hipErrorInvalidValue;
  if (p.lda < p.K || p.ldc < p.N || (p.R && p.ldr < p.N)) return hipErrorInvalidValue;
  if (dt == kF32) return quantized ? launch<float, true>(p, s) : launch<float, false>(p, s);
  return quantized ? launch<bf16, true>(p, s) : launch<bf16, false>(p, s);
}

}  // namespace mhsa
