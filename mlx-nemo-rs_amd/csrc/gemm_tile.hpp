// The bf16 tile GEMM's workgroup body and the helpers it shares with the
// other GEMM kernels, for every translation unit that launches it: the GEMM
// dispatcher, and the attention launch that runs a projection independent of
// the attention on the CUs the attention leaves idle.
// Included inside namespace mhsa { namespace { ... } } after common.hpp,
// kernels.hpp and quant.hpp.
#pragma once

// Output row of input row `row` under the seg/ring mapping.
__device__ __forceinline__ int64_t mapped_row(const GemmParams& p, int row) {
  int orow = row;
  if (p.seg_rows < p.M || p.ring_off)
    orow = (row / p.seg_rows) * p.seg_stride + (p.ring_off + row % p.seg_rows) % p.ring_len;
  return orow;
}

// C offset of one output row (computed once per row).
__device__ __forceinline__ int64_t row_offset(const GemmParams& p, int row) { return mapped_row(p, row) * p.ldc; }

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

template <int BM>
__host__ __device__ int64_t m_tiles(const GemmParams& p) {
  if (p.seg_T > 0) return (int64_t)(p.M / p.seg_T) * ((p.seg_T + BM - 1) / BM);
  return (p.M + BM - 1) / BM;
}

// ---------------------------------------------------------------------------
// bf16 tile kernel for the large projections (QKV, output and position
// projections of long inputs).
//
// One workgroup of 4 waves (2 x 2) computes a BM x BN tile; each wave holds a
// (BM/2) x (BN/2) block of fp32 accumulators (up to 128 x 128, in AGPRs) fed
// by 32x32x16 bf16 MFMAs, so every 16-byte operand fragment read from LDS
// serves BM/64 or BN/64 MFMAs. Operands stream through NS LDS stages of 64
// k-columns with direct-to-LDS buffer loads (no VGPR staging; rows past the
// matrix read as zero): A and dense B as 128-byte bf16 rows, quantized B as
// 64-byte rows of u8 codes, which each wave dequantises in registers after
// its fragment reads (below). A bf16 stage row's
// eight 16-byte chunks are stored XOR-permuted by (row / 2) % 8, which puts
// the 32 rows of one fragment read on all 64 banks. Within a stage the
// fragment reads of k-step s + 1 are issued before the MFMAs of step s
// (sched_barrier-pinned), and the first reads of the next stage are issued
// right after the stage barrier, ahead of the stage's last MFMAs.
//
// The MFMA takes the weight fragment as its first operand, so a lane's
// accumulators hold four consecutive output columns of one output row. The
// epilogue stages the bf16-rounded tile row-major in LDS and writes whole
// 16-byte runs: rows to C (bias, residual and the ring row remap applied per
// run), or, for columns at or past vt_col0, 8-token runs of V^T read down the
// staged columns.
template <int BM, int BN, bool QUANT, int NS_>
struct TileCfg {
  static constexpr int NS = NS_;                   // LDS stages; loads run NS - 1 stages ahead
  static constexpr int DIST = NS - 1;
  static constexpr int WM = BM / 2, WN = BN / 2;  // per-wave block
  static constexpr int TM = WM / 32, TN = WN / 32;
  // a stage holds 64 k-columns: A rows of 128 bytes (bf16), B rows of 128
  // bytes (bf16) or of 64 bytes (8-bit codes)
  static constexpr int BROW = QUANT ? 64 : 128;
  static constexpr int ABYTES = BM * 128, STAGE = BM * 128 + BN * BROW;
  static constexpr int NA = BM / 32;               // A loads per wave per stage (1 KB each)
  static constexpr int NB = BN * BROW / 4096;      // B loads per wave per stage (1 KB each)
  static constexpr int OP = WN * 2 + 16;           // staged output row pitch (bytes), row-major
  static constexpr int OPT = WM * 2 + 16;          // staged column pitch (bytes), transposed
  static constexpr int REG = WM * OP > WN * OPT ? WM * OP : WN * OPT;  // one wave's staging region
  // loads spread between MFMAs whenever a tile of at least 128 x 128 has a
  // CU to itself (a 64 x 64 tile has one MFMA per wave and k-step)
  static constexpr bool ILV = BM * BN >= 192 * 192 || (NS > 2 && BM * BN >= 128 * 128);
  // a wave block holding both C and V^T columns stages them twice (row-major
  // and transposed) where LDS allows: 8 staging regions
  static constexpr bool VMIX = 8 * REG <= 160 * 1024;
  static constexpr int STG = (VMIX ? 8 : 4) * REG;
  static constexpr int LDS = NS * STAGE > STG ? NS * STAGE : STG;
  static_assert(LDS <= 160 * 1024, "tile exceeds LDS");
};

typedef __attribute__((address_space(3))) void lds_void;
constexpr int kRawBuffer = 0x00020000;  // buffer descriptor dword 3: untyped 32-bit data

// The tile kernel's work as workgroup `block` of its grid, in `smem`
// (C::LDS bytes, 1024-byte aligned); run by threads 0-255.
template <int BM, int BN, bool QUANT, int NS>
__device__ __forceinline__ void gemm_tile_body(const GemmParams& p, int block, char* smem) {
  using C = TileCfg<BM, BN, QUANT, NS>;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 1, wn = w & 1;

  // Contiguous tile ranges per XCD (workgroup i runs on XCD i % 8), walked
  // 8 M tiles at a time so concurrently running tiles share A and B rows.
  const int tilesM = (int)m_tiles<BM>(p), tilesN = p.N / BN, nt = tilesM * tilesN;
  const int per = (nt + 7) / 8;
  const int W = (int)((unsigned)block % 8u) * per + (int)((unsigned)block / 8u);
  if (W >= nt) return;
  constexpr int GM = 8;
  const int gsz = GM * tilesN, first = W / gsz * GM, gm = min(tilesM - first, GM);
  const int tmi = first + (W % gsz) % gm, n0 = (W % gsz) / gm * BN;
  int m0, m_end, seg;
  tile_rows<BM>(p, tmi, m0, m_end, seg);

  const char* Ab = reinterpret_cast<const char*>(p.A) + (int64_t)m0 * p.lda * 2;
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc((void*)Ab, (short)0, (int)((int64_t)(p.M - m0) * p.lda * 2), kRawBuffer);
  // load g of wave w fills LDS chunks 64 (w NA + g) + [0, 64): row pos / 8,
  // stored chunk pos % 8, which holds k-chunk (pos % 8) ^ ((row / 2) % 8)
  int aoff[C::NA];
#pragma unroll
  for (int g = 0; g < C::NA; ++g) {
    const int pos = (w * C::NA + g) * 64 + lane, row = pos >> 3;
    aoff[g] = (int)(row * p.lda * 2 + 16 * ((pos & 7) ^ ((row >> 1) & 7)));
  }
  const char* Bb = reinterpret_cast<const char*>(p.W) + (int64_t)n0 * p.K * (QUANT ? 1 : 2);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc((void*)Bb, (short)0, (int)((int64_t)BN * p.K * (QUANT ? 1 : 2)), kRawBuffer);
  // dense B as A. Codes: load g of wave w fills LDS bytes 1024 (w NB + g) +
  // [0, 1024) of the B region, 16 rows of 64 codes: lane l stores row
  // l / 4, 16-byte chunk l % 4, which holds code chunk (l % 4) ^ ((row / 4) % 4)
  int boff[C::NB];
#pragma unroll
  for (int g = 0; g < C::NB; ++g) {
    if constexpr (QUANT) {
      const int row = (w * C::NB + g) * 16 + (lane >> 2);
      boff[g] = (int)(row * p.K + 16 * ((lane & 3) ^ ((row >> 2) & 3)));
    } else {
      const int pos = (w * C::NB + g) * 64 + lane, row = pos >> 3;
      boff[g] = (int)(row * p.K * 2 + 16 * ((pos & 7) ^ ((row >> 1) & 7)));
    }
  }
  constexpr int KB = QUANT ? 64 : 128;  // B bytes per row and stage
  auto issue = [&](int kt, int buf) {
    char* S = smem + buf * C::STAGE;
#pragma unroll
    for (int g = 0; g < C::NA; ++g)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void*)(S + (w * C::NA + g) * 1024), 16, (int)aoff[g],
                                               (int)(kt * 128), 0, 0);
#pragma unroll
    for (int g = 0; g < C::NB; ++g)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void*)(S + C::ABYTES + (w * C::NB + g) * 1024), 16,
                                               (int)boff[g], (int)(kt * KB), 0, 0);
  };
  auto issue1 = [&](int g, int kt, int buf) {  // load g of this wave's stage stream
    char* S = smem + buf * C::STAGE;
    if (g < C::NA)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void*)(S + (w * C::NA + g) * 1024), 16, (int)aoff[g],
                                               (int)(kt * 128), 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void*)(S + C::ABYTES + (w * C::NB + g - C::NA) * 1024), 16,
                                               (int)boff[g - C::NA], (int)(kt * KB), 0, 0);
  };
  // Quantized B is dequantised in registers, fragment by fragment, one
  // sub-step ahead of its MFMAs. Lane (row n, half h) reads the 32 codes
  // 32 h + [0, 32) of its row per stage as two 16-byte LDS reads (cq[0]:
  // sub-steps 0-1, cq[1]: 2-3); sub-step s takes codes 32 h + 8 s + [0, 8),
  // and the A fragments take the same k-columns (chunk 4 h + s). Scale and
  // bias of (row, group) for stage kt sit in register set kt % 2, loaded two
  // stages ahead.
  constexpr int TNQ = QUANT ? C::TN : 1;
  u32x4 cq[2][TNQ];
  floatx2 qsb[2][TNQ];
  const int groups = p.K / 64;
  const int qrow = wn * C::WN + (lane & 31);  // B row of fragment 0 within the tile
  auto sbload = [&](int kt, int set) {
#pragma unroll
    for (int j = 0; j < TNQ; ++j)
      qsb[set][j] = *reinterpret_cast<const floatx2*>(p.sb + 2 * ((int64_t)(n0 + qrow + 32 * j) * groups + kt));
  };
  // LDS offset of code chunk 2 (lane / 32) + u of fragment j's row
  int cqo[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) cqo[u] = C::ABYTES + qrow * 64 + 16 * ((2 * (lane >> 5) + u) ^ ((qrow >> 2) & 3));
  auto cread = [&](const char* S, int u) {
#pragma unroll
    for (int j = 0; j < TNQ; ++j) cq[u][j] = *reinterpret_cast<const u32x4*>(S + cqo[u] + j * 32 * 64);
  };

  // fragment (t, s): rows 32 t + lane % 32 of this wave's block, k-chunk
  // 2 s + lane / 32 of the stage (quantized B: 4 (lane / 32) + s, above)
  const int arow = (wm * C::WM + (lane & 31)) * 128;
  const int brow = C::ABYTES + (wn * C::WN + (lane & 31)) * 128;
  int so[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    so[s] = 16 * ((QUANT ? 4 * (lane >> 5) + s : 2 * s + (lane >> 5)) ^ ((lane >> 1) & 7));

  floatx16 acc[C::TN][C::TM];
#pragma unroll
  for (int j = 0; j < C::TN; ++j)
#pragma unroll
    for (int i = 0; i < C::TM; ++i) acc[j][i] = floatx16{};

  bf16x8 fa[2][C::TM], fb[2][C::TN];
  u32x4 fq[2][TNQ];  // dequantised B fragments, as packed bf16 pairs
  // half (e4) of fragment j for sub-step t: codes from cq, scale and bias
  // from set st (the same rounding as the dequantisation kernel); each pair
  // of values is one packed conversion
  auto deq4 = [&](int j, int t, int e4, int st) {
    if constexpr (QUANT) {
      const uint32_t c = cq[t >> 1][j][2 * (t & 1) + e4];
      float f[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) f[e] = __builtin_fmaf(qsb[st][j].x, (float)((c >> (8 * e)) & 0xFFu), qsb[st][j].y);
      const bf16x2 lo = {(bf16)f[0], (bf16)f[1]}, hi = {(bf16)f[2], (bf16)f[3]};
      fq[t & 1][j][2 * e4] = __builtin_bit_cast(uint32_t, lo);
      fq[t & 1][j][2 * e4 + 1] = __builtin_bit_cast(uint32_t, hi);
    }
  };
  auto bfr = [&](int b, int j) -> bf16x8 {
    if constexpr (QUANT) return __builtin_bit_cast(bf16x8, fq[b][j]);
    else return fb[b][j];
  };

  const int nk = p.K / 64;
  // The residual's 16-byte runs this lane adds in the epilogue (its stores
  // of 8 columns of C, below), loaded ahead of the operand stream: they are
  // in registers when the k-loop ends instead of being fetched after it
  // (an output GEMM with a residual measured 9% faster). They are the
  // oldest loads in flight, so only the wait for the first stages covers
  // them; every later wait count stays exact.
  constexpr int CPR = C::WN / 8, RIT = (C::WM * CPR + 63) / 64;
  constexpr bool RPRE = RIT <= 12;
  const int row0 = m0 + wm * C::WM, col0 = n0 + wn * C::WN;
  bf16x8 rpre[RPRE ? RIT : 1];
  // likewise the bias of this lane's columns, the same in each of its stores
  // when a row's runs divide the wave (64 lanes): FeedForward linear1 and
  // the pointwise convolutions measured 5-6% faster. (With 12 runs a row,
  // the 192x192 form, a lane meets three; loading those three measured
  // slower on the block's Q/K/V launch.)
  constexpr bool BPRE = 64 % CPR == 0;
  floatx4 bpre[2];
  if constexpr (BPRE) {
    if (p.bias) {
      const float* bc = p.bias + col0 + (lane % CPR) * 8;
      bpre[0] = *reinterpret_cast<const floatx4*>(bc);
      bpre[1] = *reinterpret_cast<const floatx4*>(bc + 4);
    }
  }
  if constexpr (RPRE) {
    if (p.R) {
#pragma unroll
      for (int it = 0; it < RIT; ++it) {
        const int id = it * 64 + lane, r = id / CPR, c = id % CPR;
        if (((C::WM * CPR) % 64 == 0 || id < C::WM * CPR) && row0 + r < m_end)
          rpre[it] = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const bf16*>(p.R) + (int64_t)(row0 + r) * p.ldr +
                                                       col0 + c * 8);
      }
    }
  }
  if constexpr (QUANT && C::DIST == 2) {
    // each stage's scale sets right after its codes, and a wait for stage 0
    // and its scales only: behind stage 1's codes then come set 1's scales
    // and stage 2's codes, the count every later wait assumes (a 192x192 u8
    // Q/K/V tile's prologue measured 3.1 us waiting for everything)
    // (the empty asm statements keep the issue order the counts rely on)
    issue(0, 0);
    asm volatile("" ::: "memory");
    sbload(0, 0);
    asm volatile("" ::: "memory");
    issue(min(1, nk - 1), 1);
    asm volatile("" ::: "memory");
    sbload(min(1, nk - 1), 1);
    asm volatile("" ::: "memory");
    constexpr int vm = C::NA + C::NB + C::TN;
    static_assert(vm < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((vm & 15) | ((vm >> 4) << 14) | (7 << 4));  // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
  } else if constexpr (QUANT) {
#pragma unroll
    for (int st = 0; st < C::DIST; ++st) issue(min(st, nk - 1), st);
    // with loads three or more stages ahead the loop's wait counts take the
    // two scale sets as the last loads issued here, so this wait is for all
    sbload(0, 0);
    sbload(min(1, nk - 1), 1);
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) lgkmcnt(0): stage 0 landed
    __syncthreads();
  } else {
#pragma unroll
    for (int st = 0; st < C::DIST; ++st) issue(min(st, nk - 1), st);
    // stage 0 landed; the later stages' loads may stay in flight (the
    // 8 x 375-frame bf16 offline step measured 2-3% faster than waiting for
    // all)
    constexpr int vm = (C::DIST - 1) * (C::NA + C::NB);
    static_assert(vm < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((vm & 15) | ((vm >> 4) << 14) | (7 << 4));  // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
  }

  auto rd = [&](const char* S, int s, int b) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i) fa[b][i] = *reinterpret_cast<const bf16x8*>(S + arow + i * 4096 + so[s]);
    if constexpr (!QUANT) {
#pragma unroll
      for (int j = 0; j < C::TN; ++j) fb[b][j] = *reinterpret_cast<const bf16x8*>(S + brow + j * 4096 + so[s]);
    }
  };
  // Stage kt (par = kt % 2, a literal at each call so register sets stay
  // static). Loads of the next stage go to the other buffer (free since the
  // last barrier); the last stage reloads itself, unused, so that every pass
  // has the same loads in flight and no wait count depends on a branch.
  auto stage = [&](int kt, int par) {
    const int cur = kt % C::NS, nb = (kt + 1) % C::NS;
    const char* S = smem + cur * C::STAGE;
    // stage kt + DIST streams into buffer (kt - 1) % NS, read last in stage kt - 1
    const int ktn = min(kt + C::DIST, nk - 1), nd = (kt + C::DIST) % C::NS;
    if constexpr (!C::ILV) issue(ktn, nd);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s < 3) {
        if (QUANT && s == 0) cread(S, 1);
        rd(S, s + 1, (s + 1) & 1);
      } else {
        // this wave's operand reads and its loads of stage kt + 1 are done
        // (the memory operations issued after stage kt + 1's loads, those of
        // DIST - 1 later stages and their scale loads, may still be in
        // flight); after the barrier every wave's are
        constexpr int vm = (C::DIST - 1) * (C::NA + C::NB + (QUANT ? C::TN : 0));
        static_assert(vm < 64, "vmcnt range");
        __builtin_amdgcn_s_waitcnt((vm & 15) | ((vm >> 4) << 14) | (7 << 4));  // lgkmcnt(0)
        asm volatile("s_barrier" ::: "memory");
        if constexpr (QUANT) cread(smem + nb * C::STAGE, 0);
        rd(smem + nb * C::STAGE, 0, 0);
        if constexpr (QUANT) sbload(min(kt + 2, nk - 1), par);  // set par: last used in sub-step 2
      }
      __builtin_amdgcn_sched_barrier(0);
      // fragments of sub-step s + 1 (sub-step 0 of stage kt + 1 in sub-step
      // 3) dequantised in 2 TN halves spread over this sub-step's MFMAs;
      // sub-step 3 leaves its first third to the code reads just issued
      constexpr int NM = C::TM * C::TN;
      auto qpart = [&](int m) {
        if constexpr (QUANT) {
          constexpr int P = 2 * C::TN;
          const int m0 = s == 3 ? NM / 3 : 0, span = NM - m0;
#pragma unroll
          for (int pc = 0; pc < P; ++pc)
            if (m0 + pc * span / P == m) deq4(pc >> 1, (s + 1) & 3, pc & 1, s == 3 ? par ^ 1 : par);
        }
      };
      if constexpr (C::ILV) {
        // one workgroup per CU: issuing a stage's loads in one burst stalls
        // the wave while the memory pipe takes them, so sub-steps 0-2 each
        // place a third of them between their MFMAs
        constexpr int ND = C::NA + C::NB, DQ = (ND + 2) / 3, EV = NM / DQ > 0 ? NM / DQ : 1;
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          const int j = m / C::TM, i = m % C::TM;
          acc[j][i] = mma32(bfr(s & 1, j), fa[s & 1][i], acc[j][i]);
          if (s < 3 && m % EV == EV - 1 && m / EV < DQ && s * DQ + m / EV < ND) issue1(s * DQ + m / EV, ktn, nd);
          qpart(m);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          const int j = m / C::TM, i = m % C::TM;
          acc[j][i] = mma32(bfr(s & 1, j), fa[s & 1][i], acc[j][i]);
          if constexpr (QUANT) {
            qpart(m);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  if constexpr (QUANT) {
    cread(smem, 0);
#pragma unroll
    for (int j = 0; j < C::TN; ++j) deq4(j, 0, 0, 0), deq4(j, 0, 1, 0);
  }
  rd(smem, 0, 0);
  int kt = 0;
  for (; kt + 1 < nk; kt += 2) {
    stage(kt, 0);
    stage(kt + 1, 1);
  }
  if (kt < nk) stage(kt, 0);

  // Stage T(acc): lane holds row 32 i + lane % 32 of the block and columns
  // 32 j + 8 q + 4 (lane / 32) + [0, 4). Blocks that only go to C are staged
  // row-major; blocks with V^T columns transposed (column n at n * OP, tokens
  // contiguous), so that a V^T run of 8 tokens is one 16-byte LDS read (read
  // from a row-major block, the run's rows 8 apart share two banks across the
  // wave: measured 6.2 against 2.5 us for the epilogue of a V block)
  __syncthreads();
  char* st = smem + w * C::REG;
  // columns [col0, col0 + ncn) go to C, the rest of the block to V^T
  const int ncn = p.vt ? min(max(p.vt_col0 - col0, 0), C::WN) : C::WN;
  const bool vtw = ncn < C::WN;
  const bool both = vtw && ncn > 0 && C::VMIX;  // C columns row-major in st, V^T columns transposed in stv
  char* stv = both ? smem + (4 + w) * C::REG : st;
  if (!vtw || both) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          bf16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (bf16)acc[j][i][4 * q + e];
          *reinterpret_cast<bf16x4*>(st + (i * 32 + (lane & 31)) * C::OP + (j * 32 + 8 * q + 4 * (lane >> 5)) * 2) = v;
        }
  }
  if (vtw) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            *reinterpret_cast<bf16*>(stv + (j * 32 + 8 * q + 4 * (lane >> 5) + e) * C::OPT + (i * 32 + (lane & 31)) * 2) =
                (bf16)acc[j][i][4 * q + e];
  }
  // 8 columns [col, col + 8) of block row r to C, with the bias and residual
  // (rv: the residual run, when prefetched)
  auto store_c = [&](int r, int col, bf16x8 v, const bf16x8* rvp = nullptr, const floatx4* bp = nullptr) {
    const int row = row0 + r;
    if (p.bias || p.R || p.act) {
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (float)v[e];
      if (p.bias) {
        const floatx4 b0 = bp ? bp[0] : *reinterpret_cast<const floatx4*>(p.bias + col);
        const floatx4 b1 = bp ? bp[1] : *reinterpret_cast<const floatx4*>(p.bias + col + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          f[e] = round_to<bf16>(f[e] + b0[e]);
          f[e + 4] = round_to<bf16>(f[e + 4] + b1[e]);
        }
      }
      if (p.act == kActSilu) {
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = silu_value<bf16>(f[e]);
      }
      if (p.R) {
        const bf16x8 rv =
            rvp ? *rvp : *reinterpret_cast<const bf16x8*>(reinterpret_cast<const bf16*>(p.R) + (int64_t)row * p.ldr + col);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = round_to<bf16>((float)rv[e] + p.res_scale * f[e]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (bf16)f[e];
    }
    *reinterpret_cast<bf16x8*>(reinterpret_cast<bf16*>(p.C) + row_offset(p, row) + col) = v;
  };
  if (!vtw || both) {
#pragma unroll
    for (int it = 0; it < (C::WM * CPR + 63) / 64; ++it) {
      const int id = it * 64 + lane;
      const int r = id / CPR, c = id % CPR;
      if ((C::WM * CPR) % 64 && id >= C::WM * CPR) break;
      if (c * 8 >= ncn || row0 + r >= m_end) continue;
      store_c(r, col0 + c * 8, *reinterpret_cast<const bf16x8*>(st + r * C::OP + c * 16),
              RPRE && p.R ? &rpre[RPRE ? it : 0] : nullptr, BPRE && p.bias ? bpre : nullptr);
    }
  } else if (ncn > 0) {
    // the C columns of a block staged only transposed: consecutive lanes on
    // consecutive rows, so each element read spans the banks
    for (int id = lane; id < C::WM * (ncn / 8); id += 64) {
      const int r = id % C::WM, c = id / C::WM;
      if (row0 + r >= m_end) continue;
      bf16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = *reinterpret_cast<const bf16*>(st + (c * 8 + e) * C::OPT + r * 2);
      store_c(r, col0 + c * 8, v);
    }
  }
  if (ncn < C::WN) {
    // V^T: 8-token runs down column n of the block (consecutive lanes on one
    // column's runs: contiguous stores); tokens at or past vt_Tpad belong to
    // the next utterance and are dropped
    constexpr int MCH = C::WM / 8;
    const int t0 = m0 - seg * p.seg_T + wm * C::WM;  // token of block row 0
    bf16* VT = reinterpret_cast<bf16*>(p.vt) + (int64_t)seg * p.vt_Tpad;
    const int nvt = (C::WN - ncn) * MCH;
    for (int id = lane; id < nvt; id += 64) {
      const int nl = ncn + id / MCH, mc = id % MCH;
      const int tok = t0 + mc * 8;
      if (tok >= p.vt_Tpad) continue;
      const int col = col0 + nl;
      bf16x8 v = *reinterpret_cast<const bf16x8*>(stv + nl * C::OPT + mc * 16);
      if (p.bias) {
        const float b = p.bias[col];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (bf16)((float)v[e] + b);
      }
      *reinterpret_cast<bf16x8*>(VT + (int64_t)(col - p.vt_col0) * p.vt_ld + tok) = v;
    }
  }
}

