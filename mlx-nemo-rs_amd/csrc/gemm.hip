// Projection GEMMs for the rel-pos MHSA sublayer (linear_q/k/v/out/pos).
//
// Replaces `LinearLayer::forward` (quantization.rs:126-162): y = x W^T + b for
// standard weights and MLX `quantized_matmul(transpose=true, group 64, 8 bit)`
// + b for affine-u8 weights, where the u8 codes are dequantised in registers
// on their way into LDS and feed the same MFMA tiles as dense weights.
//
// Tiling (gfx950): a BM x BN output tile per workgroup of NWM x NWN waves. One
// K step moves 128 bytes per row (64 bf16 or 32 fp32), double-buffered in LDS
// with a 16-byte row pad (no pad costs 1.7x in bank conflicts); the next
// step's global loads are in flight while the MFMAs of the current one run.
// bf16 uses 32x32x16 MFMAs (one 16-byte A and B fragment per 32x32x16 step),
// fp32 four 16x16x4 MFMAs per 16-byte fragment pair. Tile shapes by size:
// 256x256 with 8 waves for large problems, 128x128 with 4 waves otherwise, and
// 64x64 tiles with a deterministic split over K when even those cannot fill
// 256 CUs (short sequences, streaming chunks, the position table): each split
// writes fp32 partials and a second kernel sums them in split order.
//
// With seg_T > 0 the M tiles are laid out per utterance (rows b*seg_T ..
// (b+1)*seg_T, never straddling two), so the V projection can be written
// transposed ([D][B*Tpad], tokens contiguous) through LDS with 16-byte stores.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"
#include "quant.hpp"

namespace mhsa {
namespace {

constexpr int ROWB = 128;         // bytes of one tile row per K step
constexpr int PITCH = ROWB + 16;  // LDS row pitch (bytes)

template <typename T, bool QUANT, int BN, int NT>
struct BLoad;

// Dense weights: the B tile is loaded exactly like the A tile.
template <typename T, int BN, int NT>
struct BLoad<T, false, BN, NT> {
  static constexpr int NCH = BN * (ROWB / 16) / NT;
  u32x4 r[NCH];
  __device__ __forceinline__ void load(const GemmParams& p, int n0, int k0, int tid) {
    const char* W = reinterpret_cast<const char*>(p.W);
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = tid + NT * i;
      const int row = c >> 3, cb = (c & 7) * 16;
      r[i] = *reinterpret_cast<const u32x4*>(W + ((int64_t)(n0 + row) * p.K + k0) * sizeof(T) + cb);
    }
  }
  __device__ __forceinline__ void store(char* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = tid + NT * i;
      const int row = c >> 3, cb = (c & 7) * 16;
      *reinterpret_cast<u32x4*>(lds + row * PITCH + cb) = r[i];
    }
  }
};

// Affine u8 weights: ROWB/sizeof(T) codes per row per K step, 16 codes per
// 16-byte load, each load inside one group of 64.
template <typename T, int BN, int NT>
struct BLoad<T, true, BN, NT> {
  static constexpr int CODES = ROWB / sizeof(T);  // codes per row per step
  static constexpr int CPR = CODES / 16;          // 16-byte chunks per row
  static constexpr int TOTAL = BN * CPR;
  static constexpr int NCH = (TOTAL + NT - 1) / NT;
  u32x4 r[NCH];
  floatx2 sbv[NCH];
  __device__ __forceinline__ void load(const GemmParams& p, int n0, int k0, int tid) {
    const unsigned char* W = reinterpret_cast<const unsigned char*>(p.W);
    const int groups = p.K / 64;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = tid + NT * i;
      if (TOTAL % NT && c >= TOTAL) break;
      const int row = c / CPR, kc = (c % CPR) * 16;
      const int n = n0 + row, k = k0 + kc;
      r[i] = *reinterpret_cast<const u32x4*>(W + (int64_t)n * p.K + k);
      sbv[i] = *reinterpret_cast<const floatx2*>(p.sb + 2 * ((int64_t)n * groups + k / 64));
    }
  }
  __device__ __forceinline__ void store(char* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int c = tid + NT * i;
      if (TOTAL % NT && c >= TOTAL) break;
      const int row = c / CPR, kc = (c % CPR) * 16;
      T vals[16];
      dequant16<T>(r[i], sbv[i].x, sbv[i].y, vals);
      u32x4* dst = reinterpret_cast<u32x4*>(lds + row * PITCH + kc * (int)sizeof(T));
      const u32x4* src = reinterpret_cast<const u32x4*>(vals);
#pragma unroll
      for (int j = 0; j < (int)(16 * sizeof(T) / 16); ++j) dst[j] = src[j];
    }
  }
};

// C offset of one output row (computed once per row).
__device__ __forceinline__ int64_t row_offset(const GemmParams& p, int row) {
  int orow = row;
  if (p.seg_rows < p.M || p.ring_off)
    orow = (row / p.seg_rows) * p.seg_stride + (p.ring_off + row % p.seg_rows) % p.ring_len;
  return (int64_t)orow * p.ldc;
}

// The reference's op order: round the product, add the bias, round, add the
// residual, round.
template <typename T>
__device__ __forceinline__ float epilogue_value(const GemmParams& p, int row, int col, float acc) {
  float v = round_to<T>(acc);
  if (p.bias) v = round_to<T>(v + p.bias[col]);
  if (p.R) v = round_to<T>((float)reinterpret_cast<const T*>(p.R)[(int64_t)row * p.ldr + col] + v);
  return v;
}

// Tile origin: flat M tiles, or per-utterance tiles when seg_T > 0.
template <int BM>
__device__ __forceinline__ void tile_rows(const GemmParams& p, int by, int& m0, int& m_end, int& seg) {
  if (p.seg_T > 0) {
    const int per = (p.seg_T + BM - 1) / BM;
    seg = by / per;
    m0 = seg * p.seg_T + (by % per) * BM;
    m_end = min(min(m0 + BM, (seg + 1) * p.seg_T), p.M);
  } else {
    seg = 0;
    m0 = by * BM;
    m_end = min(m0 + BM, p.M);
  }
}

// blockIdx.z = K split. With gridDim.z > 1 the raw fp32 sums go to
// p.partial[z][M][N] and gemm_reduce applies the epilogue.
template <typename T, bool QUANT, int BM, int BN, int NWM, int NWN>
__global__ __launch_bounds__(64 * NWM * NWN) void gemm_kernel(const GemmParams p) {
  constexpr int NT = 64 * NWM * NWN;
  constexpr bool BF = sizeof(T) == 2;
  constexpr int BK = ROWB / sizeof(T);
  constexpr int MS = BF ? 32 : 16;            // MFMA tile edge
  constexpr int WM = BM / NWM, WN = BN / NWN;  // per-wave tile
  constexpr int TM = WM / MS, TN = WN / MS;    // MFMA tiles per wave
  constexpr int ACH = BM * (ROWB / 16) / NT;   // A chunks per thread
  using acc_t = typename std::conditional<BF, floatx16, floatx4>::type;
  using frag_t = typename Frag<T>::type;
  __shared__ __attribute__((aligned(16))) char smem[2][(BM + BN) * PITCH];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int wm = w / NWN, wn = w % NWN;
  const int n0 = blockIdx.x * BN;
  int m0, m_end, seg;
  tile_rows<BM>(p, blockIdx.y, m0, m_end, seg);
  const int ksplit = p.K / gridDim.z;
  const int kbeg = blockIdx.z * ksplit;
  const char* A = reinterpret_cast<const char*>(p.A);

  // A rows past the tile's end are clamped into the matrix; their products
  // are never stored (or land in the padding columns of V^T).
  u32x4 ra[ACH];
  auto load_a = [&](int k0) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + NT * i;
      const int row = min(m0 + (c >> 3), p.M - 1), cb = (c & 7) * 16;
      ra[i] = *reinterpret_cast<const u32x4*>(A + ((int64_t)row * p.lda + k0) * sizeof(T) + cb);
    }
  };
  auto store_a = [&](char* lds) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + NT * i;
      *reinterpret_cast<u32x4*>(lds + (c >> 3) * PITCH + (c & 7) * 16) = ra[i];
    }
  };
  BLoad<T, QUANT, BN, NT> rb;

  acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = acc_t{};

  const int nk = ksplit / BK;
  load_a(kbeg);
  rb.load(p, n0, kbeg, tid);
  store_a(smem[0]);
  rb.store(smem[0] + BM * PITCH, tid);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      load_a(kbeg + (kt + 1) * BK);
      rb.load(p, n0, kbeg + (kt + 1) * BK, tid);
    }
    const char* la = smem[cur];
    const char* lb = smem[cur] + BM * PITCH;
    if constexpr (BF) {
#pragma unroll
      for (int kf = 0; kf < 4; ++kf) {  // 16 k per 32x32x16 step
        frag_t af[TM], bfr[TN];
        const int cb = kf * 32 + (lane >> 5) * 16;
#pragma unroll
        for (int t = 0; t < TM; ++t)
          af[t] = *reinterpret_cast<const frag_t*>(la + (wm * WM + t * 32 + (lane & 31)) * PITCH + cb);
#pragma unroll
        for (int t = 0; t < TN; ++t)
          bfr[t] = *reinterpret_cast<const frag_t*>(lb + (wn * WN + t * 32 + (lane & 31)) * PITCH + cb);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mma32(af[i], bfr[j], acc[i][j]);
      }
    } else {
#pragma unroll
      for (int kf = 0; kf < 2; ++kf) {  // 16 k per four 16x16x4 steps
        frag_t af[TM], bfr[TN];
        const int cb = kf * 64 + (lane >> 4) * 16;
#pragma unroll
        for (int t = 0; t < TM; ++t)
          af[t] = *reinterpret_cast<const frag_t*>(la + (wm * WM + t * 16 + (lane & 15)) * PITCH + cb);
#pragma unroll
        for (int t = 0; t < TN; ++t)
          bfr[t] = *reinterpret_cast<const frag_t*>(lb + (wn * WN + t * 16 + (lane & 15)) * PITCH + cb);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) acc[i][j] = mma16(af[i], bfr[j], acc[i][j]);
      }
    }
    if (kt + 1 < nk) {
      store_a(smem[cur ^ 1]);
      rb.store(smem[cur ^ 1] + BM * PITCH, tid);
    }
    __syncthreads();
  }

  // Accumulator element (i, j, r) of this lane -> tile-local (row, col).
  auto elem_row = [&](int i, int r) {
    if constexpr (BF) return wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    else return wm * WM + i * 16 + 4 * (lane >> 4) + r;
  };
  auto elem_col = [&](int j) {
    if constexpr (BF) return wn * WN + j * 32 + (lane & 31);
    else return wn * WN + j * 16 + (lane & 15);
  };
  constexpr int RPL = BF ? 16 : 4;  // accumulator values per lane per tile

  if (gridDim.z > 1) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < RPL; ++r) {
        const int row = m0 + elem_row(i, r);
        if (row >= m_end) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j)
          p.partial[((int64_t)blockIdx.z * p.M + row) * p.N + n0 + elem_col(j)] = acc[i][j][r];
      }
    return;
  }

  if (p.vt && n0 >= p.vt_col0) {
    // V tile: stage transposed in LDS ([col][row], the loop's buffers are
    // free after the last barrier), then write runs of 8 tokens per store.
    constexpr int TP = BM * 2 + 16;  // bytes per staged column
    static_assert(BN * TP <= 2 * (BM + BN) * PITCH, "V^T staging must fit the tile buffers");
    char* st = &smem[0][0];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < RPL; ++r) {
        const int lr = elem_row(i, r);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int lc = elem_col(j);
          const float v = epilogue_value<T>(p, min(m0 + lr, p.M - 1), n0 + lc, acc[i][j][r]);
          *reinterpret_cast<T*>(st + lc * TP + lr * 2) = from_float<T>(v);
        }
      }
    __syncthreads();
    T* VT = reinterpret_cast<T*>(p.vt);
    const int64_t tok0 = (int64_t)seg * p.vt_Tpad + (m0 - seg * p.seg_T);
    for (int c = tid; c < BN * (BM / 8); c += NT) {
      const int lc = c / (BM / 8), ch = c % (BM / 8);
      const u32x4 v = *reinterpret_cast<const u32x4*>(st + lc * TP + ch * 16);
      *reinterpret_cast<u32x4*>(VT + (int64_t)(n0 + lc - p.vt_col0) * p.vt_ld + tok0 + ch * 8) = v;
    }
    return;
  }

#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
      const int row = m0 + elem_row(i, r);
      if (row >= m_end) continue;
      const int64_t off = row_offset(p, row);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = n0 + elem_col(j);
        reinterpret_cast<T*>(p.C)[off + col] = from_float<T>(epilogue_value<T>(p, row, col, acc[i][j][r]));
      }
    }
}

// Sum the K-split partials in split order, then the epilogue.
template <typename T>
__global__ __launch_bounds__(256) void gemm_reduce(const GemmParams p, int splits) {
  const int64_t total = (int64_t)p.M * p.N;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int z = 0; z < splits; ++z) s += p.partial[z * total + e];
    const int row = (int)(e / p.N), col = (int)(e % p.N);
    reinterpret_cast<T*>(p.C)[row_offset(p, row) + col] = from_float<T>(epilogue_value<T>(p, row, col, s));
  }
}

template <int BM>
int64_t m_tiles(const GemmParams& p) {
  if (p.seg_T > 0) return (int64_t)(p.M / p.seg_T) * ((p.seg_T + BM - 1) / BM);
  return (p.M + BM - 1) / BM;
}

template <typename T, bool QUANT, int BM, int BN, int NWM, int NWN>
hipError_t launch(const GemmParams& p, int splits, hipStream_t s) {
  dim3 grid(p.N / BN, (unsigned)m_tiles<BM>(p), splits);
  hipLaunchKernelGGL((gemm_kernel<T, QUANT, BM, BN, NWM, NWN>), grid, dim3(64 * NWM * NWN), 0, s, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  const int64_t total = (int64_t)p.M * p.N;
  const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 4096);
  hipLaunchKernelGGL(gemm_reduce<T>, dim3(blocks), dim3(256), 0, s, p, splits);
  return hipGetLastError();
}

template <typename T, bool QUANT>
hipError_t dispatch(const GemmParams& p, hipStream_t s) {
  const int bk = ROWB / (int)sizeof(T);
  // 256x256 (8 waves) when it still fills the GPU about twice over: it
  // halves the LDS and L2 traffic per flop of 128x128 (measured 1.15x on
  // M = 15000, N = 3072); bf16 only (fp32 accumulators would not fit).
  if (sizeof(T) == 2 && p.N % 256 == 0 && m_tiles<256>(p) * (p.N / 256) >= 512 &&
      (!p.vt || (p.vt_Tpad % 256 == 0 && p.vt_col0 % 256 == 0)))
    return launch<T, QUANT, 256, 256, 4, 2>(p, 1, s);
  if (m_tiles<128>(p) * (p.N / 128) >= 384 && p.N % 128 == 0) return launch<T, QUANT, 128, 128, 2, 2>(p, 1, s);
  if (p.vt) return launch<T, QUANT, 128, 128, 2, 2>(p, 1, s);  // V^T epilogue needs whole 128-row tiles
  // Small problem: 64x64 tiles, and K splits until ~512 workgroups.
  const int64_t tiles = m_tiles<64>(p) * (p.N / 64);
  int splits = 1;
  while (p.partial && tiles * splits * 2 <= 512 && p.K % (splits * 2 * bk) == 0 && p.K / (splits * 2) >= 2 * bk &&
         (int64_t)splits * 2 * p.M * p.N <= p.partial_elems)
    splits *= 2;
  return launch<T, QUANT, 64, 64, 2, 2>(p, splits, s);
}

}  // namespace

hipError_t gemm(DType dt, bool quantized, const GemmParams& p, hipStream_t s) {
  const int bk = ROWB / dtype_size(dt);
  if (p.M <= 0) return hipSuccess;
  if (p.N <= 0 || p.N % 64 || p.K <= 0 || p.K % bk || (quantized && p.K % 64)) return hipErrorInvalidValue;
  if (!p.A || !p.W || !p.C || (quantized && !p.sb)) return hipErrorInvalidValue;
  if (p.seg_rows <= 0 || p.ring_len <= 0) return hipErrorInvalidValue;
  if (p.lda < p.K || p.ldc < p.N || (p.R && p.ldr < p.N)) return hipErrorInvalidValue;
  if (p.seg_T < 0 || (p.seg_T > 0 && p.M % p.seg_T)) return hipErrorInvalidValue;
  if (p.vt) {
    // V^T: per-utterance tiles, whole 16-byte token runs inside each padded row
    if (dt != kBF16 || p.seg_T <= 0 || p.vt_col0 % 128 || p.vt_Tpad % 128 || p.vt_Tpad < p.seg_T ||
        p.vt_ld < (int64_t)(p.M / p.seg_T) * p.vt_Tpad || p.vt_ld % 8 || (reinterpret_cast<uintptr_t>(p.vt) & 15))
      return hipErrorInvalidValue;
  }
  if (dt == kF32) return quantized ? dispatch<float, true>(p, s) : dispatch<float, false>(p, s);
  return quantized ? dispatch<bf16, true>(p, s) : dispatch<bf16, false>(p, s);
}

}  // namespace mhsa
