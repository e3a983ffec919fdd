// Projection GEMMs for the rel-pos MHSA sublayer (linear_q/k/v/out/pos).
//
// Replaces `LinearLayer::forward` (quantization.rs:126-162): y = x W^T + b for
// standard weights and MLX `quantized_matmul(transpose=true, group 64, 8 bit)`
// + b for affine-u8 weights, where the u8 codes are dequantised in registers
// on their way to the MFMAs and no dequantised weight reaches HBM.
//
// Kernels, by problem (gfx950, 256 CUs):
//  * gemm_tile_kernel: bf16 projections with enough rows to fill the GPU
//    (128x128, 192x128, 192x192, 192x256 or 256x256 tiles on 4 waves, direct-to-LDS operand
//    streams, LDS-staged epilogue; described at its definition).
//  * gemm_kpar_kernel: fp32 projections of few rows (the streaming chunk,
//    one short utterance): persistent workgroups over 32 x 32 tiles, each
//    tile's contraction split over the K / 64 waves of a workgroup and summed
//    in LDS.
//  * gemm_split_kernel + gemm_reduce: bf16 projections of few rows (the
//    position table of a short utterance): K split over workgroups, the
//    partial sums added in split order by a second kernel.
//  * gemm_kernel: everything else (large fp32 problems; bf16 shapes the tile
//    kernel does not take): BM x BN tiles on NWM x NWN waves, one 128-byte
//    K step per LDS stage, double-buffered with a 16-byte row pad; an
//    optional deterministic K split with gemm_reduce.
//
// With seg_T > 0 the M tiles are laid out per utterance (rows b*seg_T ..
// (b+1)*seg_T, never straddling two), so the V projection can be written
// transposed ([D][B*Tpad], tokens contiguous) with 16-byte stores.
#include <atomic>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"
#include "quant.hpp"

namespace mhsa {
namespace {

constexpr int ROWB = 128;         // bytes of one tile row per K step
constexpr int PITCH = ROWB + 16;  // LDS row pitch (bytes)

#include "gemm_tile.hpp"

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


// The reference's op order: round the product, add the bias, round, (SiLU,)
// add the (scaled) residual, round.
template <typename T>
__device__ __forceinline__ float epilogue_value(const GemmParams& p, int row, int col, float acc) {
  float v = round_to<T>(acc);
  if (p.bias) v = round_to<T>(v + p.bias[col]);
  if (p.act == kActSilu) v = silu_value<T>(v);
  if (p.R) v = round_to<T>((float)reinterpret_cast<const T*>(p.R)[(int64_t)row * p.ldr + col] + p.res_scale * v);
  return v;
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


template <int BM, int BN, bool QUANT, int NS>
__global__ __launch_bounds__(256, 1) void gemm_tile_kernel(const GemmParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[TileCfg<BM, BN, QUANT, NS>::LDS];
  gemm_tile_body<BM, BN, QUANT, NS>(p, (int)blockIdx.x, smem);
}

// Two independent tile GEMMs in one launch: p1's tiles in workgroups [0, n1)
// (n1 a multiple of 8), p2's in the workgroups after them. Workgroups are
// dispatched in index order, so p2's tiles take the CUs p1's tiles free as
// they end, instead of waiting for p1's last tile.
template <int BM1, int BN1, int NS1, int BM2, int BN2, int NS2, bool QUANT>
__global__ __launch_bounds__(256, 1) void gemm_pair_kernel(const GemmParams p1, int n1, const GemmParams p2) {
  constexpr int L1 = TileCfg<BM1, BN1, QUANT, NS1>::LDS, L2 = TileCfg<BM2, BN2, QUANT, NS2>::LDS;
  __shared__ __attribute__((aligned(1024))) char smem[L1 > L2 ? L1 : L2];
  const int block = (int)blockIdx.x;
  if (block < n1) gemm_tile_body<BM1, BN1, QUANT, NS1>(p1, block, smem);
  else gemm_tile_body<BM2, BN2, QUANT, NS2>(p2, block - n1, smem);
}

// ---------------------------------------------------------------------------
// Split-K kernel for projections with few rows (streaming chunks, short
// utterances, the position table): too few output tiles to fill 256 CUs, so
// the contraction is split. Workgroup (tile, z) takes a 64 x 64 output tile
// over k-columns [z KS, (z + 1) KS), with KS the k-columns of one 512-byte LDS
// row (128 fp32 or 256 bf16):
//  * its whole A and B slices (64 rows x 512 bytes each) go to LDS in one
//    burst of direct-to-LDS loads (quantized B: codes to registers,
//    dequantised, written), so the workgroup waits on memory once;
//  * 4 waves of 32 x 32 each, 16x16 MFMAs (fp32 16x16x4 or bf16 16x16x32),
//    one 16-byte fragment per lane and operand per step; 16-byte chunk c of
//    LDS row r sits at c ^ (r % 16), which spreads a fragment read's 16 rows
//    over all 64 banks;
//  * the raw fp32 sums go to partial[z][M][N], and gemm_reduce sums the
//    splits in order z = 0, 1, ... and applies the epilogue. (Reducing in the
//    last workgroup to arrive instead needs agent-scope fences, which on this
//    chip write back and invalidate the whole L2 per workgroup: measured
//    20x slower.)
template <typename T, bool QUANT>
__global__ __launch_bounds__(256) void gemm_split_kernel(const GemmParams p, int splits) {
  constexpr int ES = sizeof(T);
  constexpr int KS = 512 / ES;  // k-columns per workgroup
  __shared__ __attribute__((aligned(1024))) char smem[2 * 64 * 512];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 1, wn = w & 1;
  const int tile = (int)blockIdx.x / splits, z = (int)blockIdx.x % splits;
  const int tilesN = p.N / 64;
  const int m0 = tile / tilesN * 64, n0 = tile % tilesN * 64, k0 = z * KS;

  // A rows [m0, M): 8 loads per wave of 64 x 16 bytes (rows past M read zero)
  const char* Ab = reinterpret_cast<const char*>(p.A) + ((int64_t)m0 * p.lda + k0) * ES;
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)Ab, (short)0, (int)(((int64_t)(p.M - m0) * p.lda - k0) * ES), kRawBuffer);
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    const int pos = (w * 8 + g) * 64 + lane, row = pos >> 5;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void*)(smem + (w * 8 + g) * 1024), 16,
                                             (int)(row * p.lda * ES + 16 * ((pos & 31) ^ (row & 15))), 0, 0, 0);
  }
  char* Bs = smem + 64 * 512;
  if constexpr (!QUANT) {
    const char* Bb = reinterpret_cast<const char*>(p.W) + ((int64_t)n0 * p.K + k0) * ES;
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void*)Bb, (short)0, (int)(((int64_t)64 * p.K - k0) * ES), kRawBuffer);
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const int pos = (w * 8 + g) * 64 + lane, row = pos >> 5;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void*)(Bs + (w * 8 + g) * 1024), 16,
                                               (int)(row * p.K * ES + 16 * ((pos & 31) ^ (row & 15))), 0, 0, 0);
    }
  } else {
    // 16 codes -> 16 values = ES 16-byte LDS chunks; KS / 16 code chunks per row
    constexpr int CPR = KS / 16, QN = 64 * CPR / 256;
    const unsigned char* Wq = reinterpret_cast<const unsigned char*>(p.W);
    const int groups = p.K / 64;
    u32x4 qr[QN];
    floatx2 qs[QN];
#pragma unroll
    for (int i = 0; i < QN; ++i) {
      const int q = tid + 256 * i, r = q / CPR, k = k0 + (q % CPR) * 16;
      qr[i] = *reinterpret_cast<const u32x4*>(Wq + (int64_t)(n0 + r) * p.K + k);
      qs[i] = *reinterpret_cast<const floatx2*>(p.sb + 2 * ((int64_t)(n0 + r) * groups + k / 64));
    }
#pragma unroll
    for (int i = 0; i < QN; ++i) {
      const int q = tid + 256 * i, r = q / CPR, cc = q % CPR;
      T v[16];
      dequant16<T>(qr[i], qs[i].x, qs[i].y, v);
#pragma unroll
      for (int e = 0; e < ES; ++e)
        *reinterpret_cast<u32x4*>(Bs + r * 512 + 16 * ((cc * ES + e) ^ (r & 15))) = reinterpret_cast<const u32x4*>(v)[e];
    }
  }
  __syncthreads();  // (waits for this wave's loads first)

  // wave (wm, wn): rows 32 wm + 16 i + lane % 16 of A, 32 wn + 16 j + lane % 16
  // of B; step s reads logical chunk 4 s + lane / 16 of each row
  using F = typename Frag<T>::type;
  floatx4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{};
  const char* Ar = smem + (wm * 32 + (lane & 15)) * 512;
  const char* Br = Bs + (wn * 32 + (lane & 15)) * 512;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const int off = 16 * ((4 * s + (lane >> 4)) ^ (lane & 15));
    F a[2], b[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      a[t] = *reinterpret_cast<const F*>(Ar + t * 16 * 512 + off);
      b[t] = *reinterpret_cast<const F*>(Br + t * 16 * 512 + off);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mma16(a[i], b[j], acc[i][j]);
  }

  // raw fp32 sums to partial[z][M][N]; gemm_reduce sums the splits in order
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + e;
      if (row >= p.M) continue;
#pragma unroll
      for (int j = 0; j < 2; ++j)
        p.partial[((int64_t)z * p.M + row) * p.N + n0 + wn * 32 + j * 16 + (lane & 15)] = acc[i][j][e];
    }
}

// ---------------------------------------------------------------------------
// fp32 projections with few rows (the streaming chunk's 224 rows, one short
// utterance, the position table of a short one): too few 32 x 32 output
// tiles to give every CU several, so each tile's contraction is split over
// the waves of one workgroup, and the workgroups are persistent. Workgroup g
// of G (at most one per CU) takes tiles [g T / G, (g + 1) T / G) of the T
// tiles in row-tile-major order; wave w of NW = K / 64 owns k-columns
// [64 w, 64 w + 64), one quantization group:
//  * the A fragments of the current row tile stay in registers across its
//    column tiles, and the next tile's W loads are in flight while the
//    current tile's MFMAs run (always issued: the last tile reloads itself,
//    so no load sits on a conditional path and no wait is widened);
//  * dense rows load with four consecutive lanes on one 64 B run (lane l:
//    row l / 4, 16 B chunk l % 4 of each 64 B step), which the address unit
//    serves in a quarter of the cycles that MFMA-layout loads (16 rows per 16
//    lanes) take, measured 5.8 against 1.7 us for 256 KB on one CU; each
//    1 KB load reaches MFMA layout through 1 KB of the wave's own LDS, stored
//    as 16 rows x 64 B with chunk j of row r at 16 (j ^ (r / 4 % 4)), which is
//    conflict-free for the contiguous write and the 16-row read;
//  * quantized W loads its codes in MFMA layout (a quarter of the bytes)
//    with its group's {scale, bias} and dequantises in registers;
//  * the waves' 32 x 32 partial tiles meet in LDS (two buffers by tile
//    parity: one barrier per tile) and thread t sums element t over the
//    waves in order w = 0, 1, ..., then applies the epilogue.
// fp32 16x16x4 MFMA: lane l holds row l % 16 and k 4 (l / 16) + e of each
// 16-wide step, e = 0..3. Operands are addressed through buffer descriptors
// (one VGPR offset each, the tile and step in SGPRs); A rows past M read as
// zero and are not stored.
__device__ __forceinline__ void kpar_xpose(char* slot, int wr, int rd, floatx4& v) {
  *reinterpret_cast<floatx4*>(slot + wr) = v;
  v = *reinterpret_cast<const floatx4*>(slot + rd);
}

__device__ __forceinline__ floatx4 kpar_load(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

template <bool QUANT, int TR>
__global__ __launch_bounds__(1024) void gemm_kpar_kernel(const GemmParams p) {
  // TR x TR blocks of 16x16 per tile: 32x32 tiles (TR = 2), or 16x16 tiles
  // (TR = 1) for problems with too few 32x32 tiles to give each CU one
  constexpr int TS = 16 * TR, EPW = 64 * 4 * TR * TR;  // tile side; partial sums per wave
  __shared__ __attribute__((aligned(16))) float red[2][16][EPW];  // [tile parity][wave][element]
  __shared__ __attribute__((aligned(16))) char xsm[16][1024 * TR];  // TR 1 KB transpose slots per wave
  const int tid = threadIdx.x, lane = tid & 63, nt_threads = (int)blockDim.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), nw = nt_threads >> 6;
  const int tilesN = p.N / TS, T = (p.M + TS - 1) / TS * tilesN, G = (int)gridDim.x;
  const int v0 = (int)((int64_t)blockIdx.x * T / G), v1 = (int)((int64_t)(blockIdx.x + 1) * T / G);
  if (v0 >= v1) return;  // (whole workgroup)
  const int kq = w * 64 + 4 * (lane & 3);   // quad-run chunk of the wave's k-columns
  const int kf = w * 64 + 4 * (lane >> 4);  // MFMA-layout chunk
  char* xs = xsm[w];
  const int xw = (lane >> 2) * 64 + 16 * ((lane & 3) ^ ((lane >> 4) & 3));
  const int xr = (lane & 15) * 64 + 16 * ((lane >> 4) ^ ((lane >> 2) & 3));
  // (A rows are addressed from the row tile's first row in the range-checked
  // VGPR offset, so rows past M read as zero)
  const int voa = ((lane >> 2) * (int)p.lda + kq) * 4;
  const int groups = p.K / 64;

  floatx4 a[TR][4];
  auto loadA = [&](int mt) {
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void*)(reinterpret_cast<const float*>(p.A) + (int64_t)mt * TS * p.lda),
                                          (short)0, (int)((int64_t)(p.M - mt * TS) * p.lda * 4), kRawBuffer);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < TR; ++t) a[t][s] = kpar_load(ra, voa + t * 16 * (int)p.lda * 4 + 64 * s, 0);
    if (p.acopy && mt * tilesN >= v0 && mt * tilesN < v1) {
      // the workgroup holding the row tile's first column tile copies its
      // rows (each element once)
#pragma unroll
      for (int t = 0; t < TR; ++t) {
        const int row = mt * TS + 16 * t + (lane >> 2);
        if (row < p.M) {
          float* dst = reinterpret_cast<float*>(p.acopy) + mapped_row(p, row) * p.acopy_ld + kq;
#pragma unroll
          for (int s = 0; s < 4; ++s) *reinterpret_cast<floatx4*>(dst + 16 * s) = a[t][s];
        }
      }
    }
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < TR; ++t) kpar_xpose(xs + 1024 * t, xw, xr, a[t][s]);
  };

  // W chunk (u, s) of the tile being computed (dense: quad-run layout; quant:
  // the codes), replaced by the next tile's chunk as soon as step s has taken
  // it, so the next tile's loads overlap this tile's MFMAs
  floatx4 wd[TR][4];
  uint32_t wq[TR][4];
  floatx2 wsb[TR], wsb_next[TR];
  __amdgpu_buffer_rsrc_t rw, rs;
  int vow = 0, vos = 0;
  if constexpr (!QUANT) {
    rw = __builtin_amdgcn_make_buffer_rsrc((void*)p.W, (short)0, (int)((int64_t)p.N * p.K * 4), kRawBuffer);
    vow = ((lane >> 2) * p.K + kq) * 4;
  } else {
    rw = __builtin_amdgcn_make_buffer_rsrc((void*)p.W, (short)0, (int)((int64_t)p.N * p.K), kRawBuffer);
    rs = __builtin_amdgcn_make_buffer_rsrc((void*)p.sb, (short)0, (int)((int64_t)p.N * groups * 8), kRawBuffer);
    vow = (lane & 15) * p.K + kf;
    vos = ((lane & 15) * groups + w) * 8;
  }
  auto loadW = [&](int nt, int u, int s) {
    if constexpr (!QUANT)
      wd[u][s] = kpar_load(rw, vow, (nt * TS + 16 * u) * p.K * 4 + 64 * s);
    else
      wq[u][s] = __builtin_amdgcn_raw_buffer_load_b32(rw, vow, (nt * TS + 16 * u) * p.K + 16 * s, 0);
  };
  auto loadSB = [&](int nt, floatx2 (&d)[TR]) {
    if constexpr (QUANT) {
#pragma unroll
      for (int u = 0; u < TR; ++u)
        d[u] = __builtin_bit_cast(floatx2, __builtin_amdgcn_raw_buffer_load_b64(rs, vos, (nt * TS + 16 * u) * groups * 8, 0));
    }
  };

  int mt_cur = v0 / tilesN;
  loadA(mt_cur);
#pragma unroll
  for (int u = 0; u < TR; ++u)
#pragma unroll
    for (int s = 0; s < 4; ++s) loadW(v0 % tilesN, u, s);
  loadSB(v0 % tilesN, wsb);
  for (int v = v0; v < v1; ++v) {
    const int mt = v / tilesN, nt = v % tilesN;
    const int nn = min(v + 1, v1 - 1) % tilesN;  // the next tile's columns (the last tile reloads its own)
    loadSB(nn, wsb_next);
    floatx4 acc[TR][TR];
#pragma unroll
    for (int t = 0; t < TR; ++t)
#pragma unroll
      for (int u = 0; u < TR; ++u) acc[t][u] = floatx4{};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      floatx4 bf[TR];
#pragma unroll
      for (int u = 0; u < TR; ++u) {
        if constexpr (!QUANT) {
          kpar_xpose(xs + 1024 * u, xw, xr, wd[u][s]);
          bf[u] = wd[u][s];
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            bf[u][e] = __builtin_fmaf(wsb[u].x, (float)((wq[u][s] >> (8 * e)) & 0xFFu), wsb[u].y);
        }
        loadW(nn, u, s);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int t = 0; t < TR; ++t)
#pragma unroll
          for (int u = 0; u < TR; ++u)
            acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][s][j], bf[u][j], acc[t][u], 0, 0, 0);
    }
    if constexpr (QUANT) {
#pragma unroll
      for (int u = 0; u < TR; ++u) wsb[u] = wsb_next[u];
    }
    // element 256 (TR t + u) + 4 l + e of lane l: row 16 t + 4 (l / 16) + e,
    // column 16 u + l % 16 (each 16-byte store of a wave covers 1 KB of
    // consecutive words: no bank conflicts)
    float (&rb)[16][EPW] = red[v & 1];
#pragma unroll
    for (int t = 0; t < TR; ++t)
#pragma unroll
      for (int u = 0; u < TR; ++u) *reinterpret_cast<floatx4*>(&rb[w][256 * (TR * t + u) + 4 * lane]) = acc[t][u];
    __syncthreads();
    // (this buffer is written again two tiles on, after the next tile's
    // barrier, which every thread reaches only after its sums here)
    for (int idx = tid; idx < EPW; idx += nt_threads) {
      float sum = 0.f;
      for (int ww = 0; ww < nw; ++ww) sum += rb[ww][idx];
      const int tu = idx >> 8, l = (idx >> 2) & 63, e = idx & 3;
      const int row = mt * TS + 16 * (tu / TR) + 4 * (l >> 4) + e, col = nt * TS + 16 * (tu % TR) + (l & 15);
      if (row >= p.M) continue;
      const float y = epilogue_value<float>(p, row, col, sum);
      if (!p.C2)
        reinterpret_cast<float*>(p.C)[row_offset(p, row) + col] = y;
      else if (col < p.c2_col0)
        reinterpret_cast<float*>(p.C)[(int64_t)row * p.ldc + col] = y;
      else
        reinterpret_cast<float*>(p.C2)[mapped_row(p, row) * p.ldc2 + col - p.c2_col0] = y;
    }
    if (v + 1 < v1 && (v + 1) / tilesN != mt_cur) loadA(mt_cur = (v + 1) / tilesN);
  }
}

// Tile side of the K-parallel kernel: 16x16 tiles when 32x32 tiles would
// occupy at most half the CUs (the workgroup's chain of loads, MFMAs and
// reduction is then the whole kernel, and a quarter-size tile shortens it:
// measured 8.9 -> 6.6 us at 125 x 512 x 512 and 9.1 -> 7.9 us at 249 rows;
// at 224 x 1024 x 1024, 224 tiles of 32x32, 16x16 tiles were slower, 12.3
// against 13.5 us).
int kpar_tile_rows(const GemmParams& p) {
  return (int64_t)((p.M + 31) / 32) * (p.N / 32) <= 128 ? 1 : 2;
}

// Workgroups of the K-parallel kernel: as many tiles each as the tiles over
// the CUs need, spread so that no workgroup has more.
int kpar_grid(const GemmParams& p, int tr) {
  const int cus = device_cus();
  const int ts = 16 * tr;
  const int T = (p.M + ts - 1) / ts * (p.N / ts);
  const int per = (T + cus - 1) / cus;
  return (T + per - 1) / per;
}

template <bool QUANT>
hipError_t launch_kpar(const GemmParams& p, hipStream_t s) {
  if (kpar_tile_rows(p) == 1)
    hipLaunchKernelGGL((gemm_kpar_kernel<QUANT, 1>), dim3(kpar_grid(p, 1)), dim3(p.K), 0, s, p);
  else
    hipLaunchKernelGGL((gemm_kpar_kernel<QUANT, 2>), dim3(kpar_grid(p, 2)), dim3(p.K), 0, s, p);
  return hipGetLastError();
}

// The K-parallel kernel applies to fp32, K = 64 .. 1024, 16-byte operand
// rows, operands addressable by 32-bit buffer offsets and at most 4096 tiles
// (beyond that the other kernels fill the GPU).
template <typename T>
bool kpar_ok(const GemmParams& p) {
  return sizeof(T) == 4 && p.K % 64 == 0 && p.K <= 1024 && p.N % 32 == 0 && !p.vt && p.lda % 4 == 0 &&
         ((reinterpret_cast<uintptr_t>(p.A) | reinterpret_cast<uintptr_t>(p.W)) & 15) == 0 &&
         (int64_t)p.M * p.lda * 4 < ((int64_t)1 << 31) && (int64_t)p.N * p.K * 4 < ((int64_t)1 << 31) &&
         (int64_t)((p.M + 31) / 32) * (p.N / 32) <= 4096;
}

// The split kernel applies when the scratch holds every split's sums and its
// operand rows can be loaded as 16-byte chunks.
template <typename T>
int split_count(const GemmParams& p) {
  constexpr int KS = 512 / (int)sizeof(T);
  if (!p.partial || p.vt || p.K % KS || p.N % 64) return 0;
  if ((p.lda * (int64_t)sizeof(T)) % 16 || (p.K * (int64_t)sizeof(T)) % 16) return 0;
  if ((reinterpret_cast<uintptr_t>(p.A) | reinterpret_cast<uintptr_t>(p.W)) & 15) return 0;
  if ((int64_t)p.M * p.lda * (int64_t)sizeof(T) >= ((int64_t)1 << 31) ||
      (int64_t)p.N * p.K * (int64_t)sizeof(T) >= ((int64_t)1 << 31))
    return 0;
  const int splits = p.K / KS;
  if ((int64_t)splits * p.M * p.N > p.partial_elems) return 0;
  return splits;
}

// Estimated duration of one launch of the tile kernel, in units of one
// 192 x 192 tile pass at K = 1024 with every CU busy (measured: a 256 x 256
// pass 1.45; 128 x 128 0.5 alone on a CU with four stages, 0.75 for a pass of
// two per CU with two stages; 192 x 128 taken as 0.7, two thirds of the
// MFMAs of a 192 x 192 pass plus its fixed prologue and epilogue; 192 x 256
// taken as 1.3: a third more MFMAs than 192 x 192 at fewer LDS bytes each).
template <int BM, int BN>
double tile_cost(const GemmParams& p) {
  const int64_t tiles = m_tiles<BM>(p) * (p.N / BN);
  double c;
  if (BM == 128 && BN == 128) c = tiles <= 256 ? 0.5 : (double)((tiles + 511) / 512) * 0.75;
  else if (BM == 192 && BN == 128) c = (double)((tiles + 255) / 256) * 0.7;
  else if (BM == 192 && BN == 256) c = (double)((tiles + 255) / 256) * 1.3;
  else c = (double)((tiles + 255) / 256) * (BM * BN == 256 * 256 ? 1.45 : 1.0);
  return c * p.K / 1024.0;
}

template <int BM, int BN, bool QUANT, int NS>
hipError_t launch_tile(const GemmParams& p, hipStream_t s) {
  const int64_t tiles = m_tiles<BM>(p) * (p.N / BN);
  const unsigned grid = (unsigned)((tiles + 7) / 8 * 8);
  hipLaunchKernelGGL((gemm_tile_kernel<BM, BN, QUANT, NS>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

// The tile kernel's shape requirements: 16-byte runs in every operand and
// output row, and V^T runs of 8 tokens inside each utterance's span.
bool tile_ok(const GemmParams& p) {
  if (p.K % 64 || p.lda % 8 || p.ldc % 8 || (p.R && p.ldr % 8) || (p.vt && p.R)) return false;
  if ((reinterpret_cast<uintptr_t>(p.A) | reinterpret_cast<uintptr_t>(p.C) | reinterpret_cast<uintptr_t>(p.W)) & 15)
    return false;
  if (p.R && (reinterpret_cast<uintptr_t>(p.R) & 15)) return false;
  if (p.bias && (reinterpret_cast<uintptr_t>(p.bias) & 15)) return false;
  if (p.vt && (p.vt_col0 % 8 || p.vt_Tpad % 8)) return false;
  if ((int64_t)p.M * p.lda * 2 >= ((int64_t)1 << 31) || (int64_t)p.N * p.K * 2 >= ((int64_t)1 << 31)) return false;
  return true;
}

// bf16 projections go to the tile kernel: with at least ~100 tiles of
// 128 x 128 at the tile shape with the lowest estimated time, below that
// (short inputs, a short position table) as 64 x 64 tiles with four stages
// (749 x 1024 x 1024: 6.6 us against 12 us for split-K and its reduce).
// Stages: three (loads two ahead) for 192 x 192, 192 x 128 and the u8
// 192 x 256; four for a 128 x 128 tile that has its CU to itself, two when
// two share one; 256 x 256 and the dense 192 x 256 fit two. Returns false
// when p does not take the tile kernel.
bool tile_form(const GemmParams& p, TileForm& f) {
  if (!tile_ok(p) || p.N % 64) return false;
  if (p.N % 128 || m_tiles<128>(p) * (p.N / 128) < 96) {
    if (m_tiles<64>(p) * (p.N / 64) < 16) return false;
    f = TileForm{64, 64, 4};
    return true;
  }
  double best = tile_cost<128, 128>(p);
  f = m_tiles<128>(p) * (p.N / 128) <= 256 ? TileForm{128, 128, 4} : TileForm{128, 128, 2};
  if (p.N % 192 == 0 && tile_cost<192, 192>(p) < best) best = tile_cost<192, 192>(p), f = TileForm{192, 192, 3};
  if (p.N % 256 == 0 && tile_cost<256, 256>(p) < best) best = tile_cost<256, 256>(p), f = TileForm{256, 256, 2};
  if (tile_cost<192, 128>(p) < best) best = tile_cost<192, 128>(p), f = TileForm{192, 128, 3};
  if (p.N % 256 == 0 && tile_cost<192, 256>(p) < best) best = tile_cost<192, 256>(p), f = TileForm{192, 256, 2};
  return true;
}

template <bool QUANT>
bool dispatch_tile(const GemmParams& p, hipStream_t s, hipError_t& err) {
  TileForm f;
  if (!tile_form(p, f)) return false;
  if (f.bm == 64) err = launch_tile<64, 64, QUANT, 4>(p, s);
  else if (f.bm == 256) err = launch_tile<256, 256, QUANT, 2>(p, s);
  else if (f.bm == 192 && f.bn == 192) err = launch_tile<192, 192, QUANT, 3>(p, s);
  else if (f.bm == 192 && f.bn == 256) err = launch_tile<192, 256, QUANT, QUANT ? 3 : 2>(p, s);
  else if (f.bm == 192) err = launch_tile<192, 128, QUANT, 3>(p, s);
  else if (f.ns == 4) err = launch_tile<128, 128, QUANT, 4>(p, s);
  else err = launch_tile<128, 128, QUANT, 2>(p, s);
  return true;
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
  if constexpr (sizeof(T) == 4) {
    if (p.C2 || p.acopy) return launch_kpar<QUANT>(p, s);  // (validated by gemm())
  }
  if constexpr (sizeof(T) == 2) {
    hipError_t err;
    if (dispatch_tile<QUANT>(p, s, err)) return err;
  }
  // 256x256 (8 waves) when it still fills the GPU about twice over: it
  // halves the LDS and L2 traffic per flop of 128x128 (measured 1.15x on
  // M = 15000, N = 3072); bf16 only (fp32 accumulators would not fit).
  if (sizeof(T) == 2 && p.N % 256 == 0 && m_tiles<256>(p) * (p.N / 256) >= 512 &&
      (!p.vt || (p.vt_Tpad % 256 == 0 && p.vt_col0 % 256 == 0)))
    return launch<T, QUANT, 256, 256, 4, 2>(p, 1, s);
  if (m_tiles<128>(p) * (p.N / 128) >= 384 && p.N % 128 == 0) return launch<T, QUANT, 128, 128, 2, 2>(p, 1, s);
  if (p.vt) return launch<T, QUANT, 128, 128, 2, 2>(p, 1, s);  // V^T epilogue needs whole 128-row tiles
  // few rows of fp32: K-parallel workgroups, no second kernel (for bf16 the
  // position table of a short utterance measured the same as split-K: 13.4
  // against 12.6 us at 749 x 1024 x 1024, so bf16 keeps split-K); the split
  // output and row copy only exist there
  if constexpr (sizeof(T) == 4) {
    if (kpar_ok<T>(p)) return launch_kpar<QUANT>(p, s);
  }
  if (const int splits = split_count<T>(p)) {
    const int64_t tiles = (int64_t)((p.M + 63) / 64) * (p.N / 64);
    hipLaunchKernelGGL((gemm_split_kernel<T, QUANT>), dim3((unsigned)(tiles * splits)), dim3(256), 0, s, p, splits);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // (also for one split: the reduce kernel applies the epilogue)
    const int64_t total = (int64_t)p.M * p.N;
    const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 4096);
    hipLaunchKernelGGL(gemm_reduce<T>, dim3(blocks), dim3(256), 0, s, p, splits);
    return hipGetLastError();
  }
  // Small problem: 64x64 tiles, and K splits until ~512 workgroups.
  const int64_t tiles = m_tiles<64>(p) * (p.N / 64);
  int splits = 1;
  while (p.partial && tiles * splits * 2 <= 512 && p.K % (splits * 2 * bk) == 0 && p.K / (splits * 2) >= 2 * bk &&
         (int64_t)splits * 2 * p.M * p.N <= p.partial_elems)
    splits *= 2;
  return launch<T, QUANT, 64, 64, 2, 2>(p, splits, s);
}

}  // namespace

bool gemm_split_fused_ok(DType dt, const GemmParams& p) {
  if (dt != kF32 || p.vt || !kpar_ok<float>(p)) return false;
  if (p.C2 && (p.c2_col0 <= 0 || p.c2_col0 >= p.N || p.c2_col0 % 32 || p.ldc2 < p.N - p.c2_col0)) return false;
  if (p.acopy && (p.acopy_ld < p.K || (p.acopy_ld % 4) || (reinterpret_cast<uintptr_t>(p.acopy) & 15))) return false;
  return true;
}

hipError_t gemm_check(DType dt, bool quantized, const GemmParams& p) {
  const int bk = ROWB / dtype_size(dt);
  if ((p.C2 || p.acopy) && !gemm_split_fused_ok(dt, p)) return hipErrorInvalidValue;
  if (p.N <= 0 || p.N % 64 || p.K <= 0 || p.K % bk || (quantized && p.K % 64)) return hipErrorInvalidValue;
  if (!p.A || !p.W || !p.C || (quantized && !p.sb)) return hipErrorInvalidValue;
  if (p.seg_rows <= 0 || p.ring_len <= 0) return hipErrorInvalidValue;
  if (p.lda < p.K || p.ldc < (p.C2 ? p.c2_col0 : p.N) || (p.R && p.ldr < p.N)) return hipErrorInvalidValue;
  if (p.seg_T < 0 || (p.seg_T > 0 && p.M % p.seg_T)) return hipErrorInvalidValue;
  if (p.vt) {
    // V^T: per-utterance tiles, whole 16-byte token runs inside each padded row
    if (dt != kBF16 || p.seg_T <= 0 || p.vt_col0 % 128 || p.vt_Tpad % 128 || p.vt_Tpad < p.seg_T ||
        p.vt_ld < (int64_t)(p.M / p.seg_T) * p.vt_Tpad || p.vt_ld % 8 || (reinterpret_cast<uintptr_t>(p.vt) & 15))
      return hipErrorInvalidValue;
  }
  return hipSuccess;
}

bool gemm_tile_form(DType dt, bool quantized, const GemmParams& p, TileForm& f) {
  return dt == kBF16 && p.M > 0 && !p.C2 && !p.acopy && gemm_check(dt, quantized, p) == hipSuccess && tile_form(p, f);
}

namespace {
template <int BM1, int BN1, int NS1, bool QUANT>
hipError_t launch_pair(const GemmParams& p1, const GemmParams& p2, hipStream_t s) {
  const int64_t n1 = (m_tiles<BM1>(p1) * (p1.N / BN1) + 7) / 8 * 8, n2 = (m_tiles<64>(p2) * (p2.N / 64) + 7) / 8 * 8;
  hipLaunchKernelGGL((gemm_pair_kernel<BM1, BN1, NS1, 64, 64, 4, QUANT>), dim3((unsigned)(n1 + n2)), dim3(256), 0, s,
                     p1, (int)n1, p2);
  return hipGetLastError();
}

template <bool QUANT>
hipError_t dispatch_pair(const TileForm& f, const GemmParams& p1, const GemmParams& p2, hipStream_t s) {
  if (f.bm == 256) return launch_pair<256, 256, 2, QUANT>(p1, p2, s);
  if (f.bm == 192 && f.bn == 192) return launch_pair<192, 192, 3, QUANT>(p1, p2, s);
  if (f.bm == 192 && f.bn == 256) return launch_pair<192, 256, QUANT ? 3 : 2, QUANT>(p1, p2, s);
  if (f.bm == 192) return launch_pair<192, 128, 3, QUANT>(p1, p2, s);
  if (f.ns == 4) return launch_pair<128, 128, 4, QUANT>(p1, p2, s);
  return launch_pair<128, 128, 2, QUANT>(p1, p2, s);
}
}  // namespace

int device_cus() {
  constexpr int kDevices = 64;
  static std::atomic<int> cached[kDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < kDevices)
    if (const int n = cached[dev].load(std::memory_order_relaxed)) return n;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  if (dev >= 0 && dev < kDevices) cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Paired where p1's tiles take one round of CUs: the CUs its slowest tiles
// leave idle then run p2's tiles (measured: 3000 x 3072 Q/K/V tiles with
// 749 x 1024 position tiles, step 0.064 -> 0.061 ms). Past one round it
// measured no gain (15000 x 3072 with 257 rows: step 0.2174 against
// 0.2202 ms).
bool gemm_pair_ok(DType dt, bool quantized, const GemmParams& p1, const GemmParams& p2) {
  TileForm f1, f2;
  return p1.M > 0 && p2.M > 0 && gemm_tile_form(dt, quantized, p1, f1) && f1.bm != 64 &&
         gemm_tile_form(dt, quantized, p2, f2) && f2.bm == 64 &&
         (p1.seg_T > 0 ? (int64_t)(p1.M / p1.seg_T) * ((p1.seg_T + f1.bm - 1) / f1.bm) : (p1.M + f1.bm - 1) / f1.bm) *
                 (p1.N / f1.bn) <=
             device_cus();
}

hipError_t gemm_pair(DType dt, bool quantized, const GemmParams& p1, const GemmParams& p2, hipStream_t s) {
  if (!gemm_pair_ok(dt, quantized, p1, p2)) return hipErrorInvalidValue;
  TileForm f;
  tile_form(p1, f);
  return quantized ? dispatch_pair<true>(f, p1, p2, s) : dispatch_pair<false>(f, p1, p2, s);
}

hipError_t gemm(DType dt, bool quantized, const GemmParams& p, hipStream_t s) {
  if (p.M <= 0) return hipSuccess;
  if (hipError_t e = gemm_check(dt, quantized, p)) return e;
  if (dt == kF32) return quantized ? dispatch<float, true>(p, s) : dispatch<float, false>(p, s);
  return quantized ? dispatch<bf16, true>(p, s) : dispatch<bf16, false>(p, s);
}

}  // namespace mhsa
