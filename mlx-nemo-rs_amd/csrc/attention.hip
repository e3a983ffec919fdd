// Fused Transformer-XL relative-position attention for one head slice.
//
// Replaces, per query block, the reference's
//   q_u = q + pos_bias_u, q_v = q + pos_bias_v        (attention.rs:501-508)
//   bd = rel_shift(q_v P^T)[..., :L]                  (attention.rs:524-532, 818-855)
//   mask = context mask + key padding mask            (attention.rs:229-294, 536-543)
//   softmax(s q_u K^T + cast(s) bd + mask) V          (attention.rs:296-318)
// and the streaming bool-mask path where a fully hidden row yields zeros
// (attention.rs:774-790), with no [rows, 2L-1] score matrix in memory.
//
// Work split (gfx950, 64-wide waves): a workgroup owns QB = 16*NW queries of
// one (batch, head); each wave owns 16 queries. Keys advance in tiles of NK
// (64 for bf16, 32 for fp32) staged in LDS together with V^T and the band of
// QB+NK position rows the tile's (query, key) pairs can reach. Per tile and
// wave:
//   S^T  = K  . Qu^T   (NK x 16)       MFMA, K as the A operand
//   B'^T = P' . Qv^T   ((NK+16) x 16)  MFMA over the wave's position band
//   rel_shift: bd(j, i) = B'^T(j + 15 - i, i), an index remap through LDS
//   online fp32 softmax per query column, then O^T += V^T . Pr^T (MFMA)
// Scores stay in fp32 registers; probabilities are rounded to the compute
// dtype for the PV MFMA. Key tiles that no query of the block can see are
// skipped, so a +-w local window costs O(T w) instead of O(T^2).
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"
#include "quant.hpp"

namespace mhsa {
namespace {

#include "gemm_tile.hpp"

constexpr float kLog2e = 1.4426950408889634f;

std::atomic<int64_t> g_form_launches[kAttnForms];
void count_form(AttnForm f) { g_form_launches[f].fetch_add(1, std::memory_order_relaxed); }

// Every mask of the path hides keys outside one interval per query (i at
// absolute frame ia = qoff + i): the padding / unfilled-cache range
// [key_lo, key_hi) (attention.rs:280-294, conformer.rs:155-181); the regular
// context j - ia in [-left, right] (attention.rs:256-269); the chunked_limited
// context 0 <= ia/chunk - j/chunk <= left/chunk, i.e. whole chunks
// [(ia/chunk - left/chunk) * chunk, (ia/chunk + 1) * chunk)
// (attention.rs:241-255, conformer.rs:293-323). They intersect to [lo, hi),
// empty for rows past q_valid (conformer.rs:197-215).
__device__ __forceinline__ int2 query_interval(const AttnParams& p, int bl, int i) {
  int lo = max(p.key_lo[bl], 0), hi = min(p.key_hi[bl], p.L);
  if (i >= p.q_valid[bl] || i >= p.T) hi = lo;
  if (p.has_ctx) {
    const int ia = p.qoff + i;
    if (p.chunked && p.right >= 0) {
      const int chunk = p.right + 1;
      const int lc = p.left >= 0 ? p.left / chunk : 10000;
      const int qc = ia / chunk;
      lo = max(lo, (qc - lc) * chunk);
      hi = min(hi, (qc + 1) * chunk);
    } else {
      if (p.left >= 0) lo = max(lo, ia - p.left);
      if (!p.chunked && p.right >= 0) hi = min(hi, ia + p.right + 1);
    }
  }
  return make_int2(lo, max(hi, lo));
}

__device__ __forceinline__ bool in_interval(int j, int2 iv) {
  return (unsigned)(j - iv.x) < (unsigned)(iv.y - iv.x);
}

__device__ __forceinline__ int key_row(const AttnParams& p, int j) {
  return p.ring_len ? (p.ring_head + j) % p.ring_len : j;
}

// Keys [jbeg, jend) that can be visible to some query in [i0, i_end)
// (also evaluated on the host to size the bf16 kernel's position slack).
__host__ __device__ inline int imin(int a, int b) { return a < b ? a : b; }
__host__ __device__ inline int imax(int a, int b) { return a > b ? a : b; }
__host__ __device__ inline void key_range(const AttnParams& p, int bl, int i0, int i_end, int& jbeg, int& jend) {
  const int row_end = imin(i_end, p.q_valid[bl]);
  jbeg = imax(p.key_lo[bl], 0);
  jend = imin(p.key_hi[bl], p.L);
  if (row_end <= i0) {
    jend = jbeg;
    return;
  }
  if (!p.has_ctx) return;
  const int a0 = p.qoff + i0, a1 = p.qoff + row_end - 1;
  if (p.chunked && p.right >= 0) {
    const int chunk = p.right + 1;
    const int lc = p.left >= 0 ? p.left / chunk : 10000;
    const long lo = ((long)(a0 / chunk) - lc) * chunk;
    jbeg = imax(jbeg, (int)(lo > 0 ? lo : 0));
    jend = imin(jend, (a1 / chunk + 1) * chunk);
  } else {
    if (p.left >= 0) jbeg = imax(jbeg, a0 - p.left);
    if (!p.chunked && p.right >= 0) jend = imin(jend, a1 + p.right + 1);
  }
}

template <typename T, int DK, int NW, int NKO = 0>
struct Cfg {
  static constexpr int NT = 64 * NW;
  static constexpr int QB = 16 * NW;
  static constexpr int NK = NKO ? NKO : sizeof(T) == 2 ? 64 : 32;
  static constexpr int RB = DK * (int)sizeof(T);           // bytes per K/P row
  static constexpr int KP = RB + 16;                       // LDS pitch of K and P rows
  static constexpr int VP = NK * (int)sizeof(T) + 16;      // LDS pitch of V^T rows
  static constexpr int PR = QB + NK;                       // position rows staged per tile
  static constexpr int RMP = NK + 20;                      // remap row pitch (floats)
  static constexpr int K_OFF = 0;
  static constexpr int V_OFF = K_OFF + NK * KP;
  static constexpr int P_OFF = V_OFF + DK * VP;
  static constexpr int R_OFF = P_OFF + PR * KP;
  static constexpr int LDS = R_OFF + NW * 16 * RMP * 4;
  static constexpr int NKF = DK / Frag<T>::KSTEP;          // fragments along d_k
  static constexpr int NU = NK / 16;                       // 16-key sub-tiles
  static constexpr int NB = NU + 1;                        // 16-row band sub-tiles
};

// KS (key split, for inputs too short to give every CU a workgroup): the NW
// waves of a workgroup share its 16 queries and take the key tiles w,
// w + NW, ... each with LDS tiles of its own and no workgroup barrier in the
// loop; their softmax states (running maximum, sum, O) are merged at the end.
// In the split form each wave prefetches a whole key tile into registers
// (K, V and position rows: 16 KB per 16 keys at d_k = 128 in fp32), so fp32
// d_k = 128 takes 16-key tiles: with 32-key tiles the prefetch alone held 224
// of the 256 VGPRs and the kernel spilled to AGPRs and scratch.
template <typename T, int DK, bool KS>
constexpr int gen_tile_keys() { return KS && sizeof(T) == 4 && DK == 128 ? 16 : 0; }

template <typename T, int DK, int NW, bool DEBUG, bool KS = false>
__global__ __launch_bounds__(64 * NW) void attn_kernel(const AttnParams p) {
  // Forms: NW >= 4 waves of 16 queries sharing each key tile, or the key
  // split. A one-wave shared-tile form (16 queries, no split) is not built:
  // it gave wrong outputs whenever its per-key mask ran while spilling at
  // 256 VGPRs + 256 AGPRs, and the split form covers short query blocks.
  static_assert(KS || NW >= 4, "the shared-tile form needs at least 4 waves");
  using C = Cfg<T, DK, KS ? 1 : NW, gen_tile_keys<T, DK, KS>()>;  // (split: one wave's tile geometry, 16 queries)
  using F = Frag<T>;
  using frag_t = typename F::type;
  constexpr int NT = C::NT, QB = C::QB, NK = C::NK, EPL = F::EPL;
  __shared__ __attribute__((aligned(16))) char smem[KS ? NW * C::LDS : C::LDS];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, ql = lane & 15;
  const int tt = KS ? lane : tid;  // this thread's index among the threads that load a tile
  char* const tb = smem + (KS ? w * C::LDS : 0);
  char* Ks = tb + C::K_OFF;
  char* Vt = tb + C::V_OFF;
  char* Ps = tb + C::P_OFF;
  const int bl = blockIdx.z, b = p.b0 + bl, h = blockIdx.y;
  const int i0 = blockIdx.x * QB;
  const int wq = KS ? 0 : w;        // this wave's 16-query group in the block
  const int qi = i0 + 16 * wq + ql;  // this lane's query column
  float* Rm = reinterpret_cast<float*>(tb + C::R_OFF) + wq * 16 * C::RMP;

  // Queries with the position biases folded in, rounded like the reference's
  // bf16 adds; they are the B operand of both score products.
  frag_t qu[C::NKF], qv[C::NKF];
  {
    const T* qrow = reinterpret_cast<const T*>(p.q) + (int64_t)b * p.q_bs + (int64_t)qi * p.q_rs + h * DK;
    const bool ok = qi < p.T;
#pragma unroll
    for (int kf = 0; kf < C::NKF; ++kf) {
      const int d0 = kf * F::KSTEP + g * EPL;
      const frag_t raw = load16<frag_t>(qrow + d0, ok);
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float x = (float)raw[e];
        qu[kf][e] = from_float<T>(ok ? x + p.bias_u[h * DK + d0 + e] : 0.f);
        qv[kf][e] = from_float<T>(ok ? x + p.bias_v[h * DK + d0 + e] : 0.f);
      }
    }
  }

  floatx4 o[DK / 16];
#pragma unroll
  for (int d = 0; d < DK / 16; ++d) o[d] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  int jbeg, jend;
  key_range(p, bl, i0, min(i0 + QB, p.T), jbeg, jend);
  const int2 iv = query_interval(p, bl, qi);
  const float sc_qk = p.scale * kLog2e, sc_bd = p.scale_bd * kLog2e;
  const char* kbase = reinterpret_cast<const char*>(p.k) + ((int64_t)b * p.kv_bs + h * DK) * sizeof(T);
  const char* vbase = reinterpret_cast<const char*>(p.v) + ((int64_t)b * p.kv_bs + h * DK) * sizeof(T);
  const char* pbase = reinterpret_cast<const char*>(p.p) + (int64_t)h * DK * sizeof(T);

  // A key tile's K rows, V rows and position rows pmin .. pmin + PR - 1 are
  // loaded into registers one tile ahead (while the previous tile computes)
  // and stored to LDS at the top of their tile: rows past the last key or
  // outside the table read row 0 and are zeroed, so every load is issued
  // unconditionally.
  constexpr int CPR = C::RB / 16;                       // 16-byte chunks per row
  constexpr int NKV = (NK * CPR + NT - 1) / NT;         // K / V chunks per thread
  constexpr int NPC = (C::PR * CPR + NT - 1) / NT;      // position chunks per thread
  u32x4 kr[NKV], pr[NPC];
  frag_t vr[NKV];
  auto fetch = [&](int j0) {
#pragma unroll
    for (int i = 0; i < NKV; ++i) {
      const int c = tt + i * NT, row = min(c / CPR, NK - 1), cb = (c % CPR) * 16;
      const int j = j0 + row;
      const bool ok = c < NK * CPR && j < p.L;
      const int64_t off = (int64_t)(ok ? key_row(p, j) : 0) * p.kv_rs * sizeof(T) + cb;
      const u32x4 kv = *reinterpret_cast<const u32x4*>(kbase + off);
      const frag_t vv = *reinterpret_cast<const frag_t*>(vbase + off);
      kr[i] = ok ? kv : u32x4{0u, 0u, 0u, 0u};
      vr[i] = ok ? vv : frag_t{};
    }
    const int pmin = p.center - p.qoff - (i0 + QB - 1) + j0;
#pragma unroll
    for (int i = 0; i < NPC; ++i) {
      const int c = tt + i * NT, row = min(c / CPR, C::PR - 1), cb = (c % CPR) * 16;
      const int tp = pmin + row;
      const bool ok = c < C::PR * CPR && tp >= 0 && tp < p.p_rows;
      const u32x4 pv = *reinterpret_cast<const u32x4*>(pbase + (int64_t)(ok ? tp : 0) * p.p_rs * sizeof(T) + cb);
      pr[i] = ok ? pv : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < NKV; ++i) {
      const int c = tt + i * NT, row = c / CPR, cb = (c % CPR) * 16;
      if (c >= NK * CPR) break;
      *reinterpret_cast<u32x4*>(Ks + row * C::KP + cb) = kr[i];
      const int d0 = cb / (int)sizeof(T);  // V^T: transposed on the way in
      // (fp32: key k of V^T row d sits at k ^ 4 ((d / 16) % 4), which puts the
      // 4-byte stores of lanes 4 rows apart on distinct banks; reads of 4
      // consecutive keys stay one 16-byte read)
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const int kx = sizeof(T) == 4 ? row ^ (4 * (((d0 + e) >> 4) & 3)) : row;
        *reinterpret_cast<T*>(Vt + (d0 + e) * C::VP + kx * (int)sizeof(T)) = vr[i][e];
      }
    }
#pragma unroll
    for (int i = 0; i < NPC; ++i) {
      const int c = tt + i * NT, row = c / CPR, cb = (c % CPR) * 16;
      if (c >= C::PR * CPR) break;
      *reinterpret_cast<u32x4*>(Ps + row * C::KP + cb) = pr[i];
    }
  };
  // tiles of this wave (split) or of the workgroup: jfirst, jfirst + step, ...
  constexpr int step = KS ? NK * NW : NK;
  const int jfirst = (jbeg / NK) * NK + (KS ? NK * w : 0);
  const int jlast = jend > jfirst ? jfirst + (jend - 1 - jfirst) / step * step : jfirst;
  if (jfirst < jend) fetch(jfirst);
  for (int j0 = jfirst; j0 < jend; j0 += step) {
    // previous tile fully consumed (split: the wave's own tiles, whose LDS
    // operations run in order)
    if constexpr (!KS) __syncthreads();
    stash();
    fetch(min(j0 + step, jlast));  // (the last tile loads itself again, unused)
    if constexpr (!KS) __syncthreads();

    // S^T = K Qu^T and the wave's band B'^T = P' Qv^T.
    floatx4 s[C::NU], bd[C::NB];
#pragma unroll
    for (int u = 0; u < C::NU; ++u) s[u] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < C::NB; ++t) bd[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int band0 = QB - 16 - 16 * wq;  // first band row of this wave
#pragma unroll
    for (int kf = 0; kf < C::NKF; ++kf) {
      const int cb = kf * 64 + g * 16;
#pragma unroll
      for (int u = 0; u < C::NU; ++u) {
        const frag_t a = *reinterpret_cast<const frag_t*>(Ks + (16 * u + ql) * C::KP + cb);
        s[u] = mma16(a, qu[kf], s[u]);
      }
#pragma unroll
      for (int t = 0; t < C::NB; ++t) {
        const frag_t a = *reinterpret_cast<const frag_t*>(Ps + (band0 + 16 * t + ql) * C::KP + cb);
        bd[t] = mma16(a, qv[kf], bd[t]);
      }
    }

    // rel_shift as an LDS remap: band row n of query column ql holds the
    // pair (i = 16w + ql, j = n - 15 + ql).
#pragma unroll
    for (int t = 0; t < C::NB; ++t)
      *reinterpret_cast<floatx4*>(Rm + ql * C::RMP + 16 * t + 4 * g) = bd[t];
    __builtin_amdgcn_wave_barrier();

    float sc[C::NU][4];
    float tmax = -INFINITY;
    const bool full = __all(iv.x <= j0 && iv.y >= j0 + NK);  // no key of the tile hidden
#pragma unroll
    for (int u = 0; u < C::NU; ++u) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int jl = 16 * u + 4 * g + r;
        const int j = j0 + jl;
        const float bdv = Rm[ql * C::RMP + jl + 15 - ql];
        if (DEBUG && p.dbg_bd && qi < p.T && j < p.L)
          p.dbg_bd[(((int64_t)b * p.H + h) * p.T + qi) * p.L + j] = p.scale_bd * bdv;
        const float v = s[u][r] * sc_qk + bdv * sc_bd;
        sc[u][r] = full || in_interval(j, iv) ? v : -INFINITY;
        tmax = fmaxf(tmax, sc[u][r]);
      }
    }
    __builtin_amdgcn_wave_barrier();
    tmax = col_max(tmax);
    // Lazy rescale (wave-uniform branch; the MFMAs are outside it): O and l
    // move to a new maximum only when some column's maximum grew by more than
    // 8 in log2 units, so probabilities stay <= 2^8 and O / l is unchanged.
    // A column with nothing visible yet keeps zero O, l and probabilities.
    if (__any(tmax > m_run + 8.f)) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = __builtin_amdgcn_exp2f(m_run - (m_new == -INFINITY ? 0.f : m_new));
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < DK / 16; ++d) o[d] *= alpha;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float psum = 0.f;
#pragma unroll
    for (int u = 0; u < C::NU; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[u][r] = __builtin_amdgcn_exp2f(sc[u][r] - m_use);  // v_exp_f32; exp2(-inf) = 0
        psum += sc[u][r];
      }
    l_run += psum;

    // O^T += V^T Pr^T. The contraction slots of a fragment map to the keys
    // this lane already holds in S^T layout: keys 16u + 4g + r.
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int u = 0; u < C::NU; u += 2) {
        bf16x8 pb;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pb[r] = (bf16)sc[u][r];
          pb[4 + r] = (bf16)sc[u + 1][r];
        }
#pragma unroll
        for (int d = 0; d < DK / 16; ++d) {
          const char* vr = Vt + (16 * d + ql) * C::VP;
          const bf16x4 lo = *reinterpret_cast<const bf16x4*>(vr + (16 * u + 4 * g) * 2);
          const bf16x4 hi = *reinterpret_cast<const bf16x4*>(vr + (16 * (u + 1) + 4 * g) * 2);
          const bf16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[d] = mma16(a, pb, o[d]);
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < C::NU; ++u) {
        const floatx4 pb = {sc[u][0], sc[u][1], sc[u][2], sc[u][3]};
#pragma unroll
        for (int d = 0; d < DK / 16; ++d) {
          const floatx4 a = *reinterpret_cast<const floatx4*>(Vt + (16 * d + ql) * C::VP + ((16 * u + 4 * g) ^ (4 * (d & 3))) * 4);
          o[d] = mma16(a, pb, o[d]);
        }
      }
    }
  }

  if constexpr (KS) {
    // Merge the waves' states through LDS (each wave writes into its own
    // tile area): query column ql, d_k rows 16 d + 4 g + r of O at word
    // 64 (4 d + r) + lane (the lanes of one store on consecutive words: a
    // query-major layout put all 16 query columns on one bank); wave w then
    // finishes d_k rows 16 d + ... for d = w, w + NW, ...
    static_assert(C::LDS >= (DK * 16 + 32) * 4, "merge area");
    float* mo = reinterpret_cast<float*>(tb);
    const float l_w = col_sum(l_run);
    if (g == 0) {
      mo[DK * 16 + ql] = m_run;
      mo[DK * 16 + 16 + ql] = l_w;
    }
#pragma unroll
    for (int d = 0; d < DK / 16; ++d)
#pragma unroll
      for (int r = 0; r < 4; ++r) mo[64 * (4 * d + r) + lane] = o[d][r];
    __syncthreads();
    float mw[NW], m_all = -INFINITY;
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      mw[v] = reinterpret_cast<const float*>(smem + v * C::LDS)[DK * 16 + ql];
      m_all = fmaxf(m_all, mw[v]);
    }
    float l_all = 0.f, f[NW];
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      // a wave that saw nothing has m = -inf, l = 0 and O = 0
      f[v] = mw[v] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw[v] - m_all);
      l_all += f[v] * reinterpret_cast<const float*>(smem + v * C::LDS)[DK * 16 + 16 + ql];
    }
    const float inv = l_all > 0.f ? 1.f / l_all : 0.f;
    if (qi < p.T) {
      T* orow = reinterpret_cast<T*>(p.o) + (int64_t)b * p.o_bs + (int64_t)qi * p.o_rs + h * DK;
      for (int d = w; d < DK / 16; d += NW) {
        T vals[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float acc = 0.f;
#pragma unroll
          for (int v = 0; v < NW; ++v)
            acc += f[v] * reinterpret_cast<const float*>(smem + v * C::LDS)[64 * (4 * d + r) + lane];
          vals[r] = from_float<T>(acc * inv);
        }
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<u32x2*>(orow + 16 * d + 4 * g) = *reinterpret_cast<const u32x2*>(vals);
        } else {
          *reinterpret_cast<u32x4*>(orow + 16 * d + 4 * g) = *reinterpret_cast<const u32x4*>(vals);
        }
      }
    }
    return;
  }
  // Normalise; a query that saw no key outputs zeros.
  const float l_tot = col_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (qi < p.T) {
    T* orow = reinterpret_cast<T*>(p.o) + (int64_t)b * p.o_bs + (int64_t)qi * p.o_rs + h * DK;
#pragma unroll
    for (int d = 0; d < DK / 16; ++d) {
      T vals[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) vals[r] = from_float<T>(o[d][r] * inv);
      if constexpr (sizeof(T) == 2) {
        *reinterpret_cast<u32x2*>(orow + 16 * d + 4 * g) = *reinterpret_cast<const u32x2*>(vals);
      } else {
        *reinterpret_cast<u32x4*>(orow + 16 * d + 4 * g) = *reinterpret_cast<const u32x4*>(vals);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// bf16 path with 32x32x16 MFMAs: 32 queries per wave, NW waves per
// workgroup, NK-key tiles, in two forms: 4 waves over 64-key tiles (one wave
// per SIMD) and 8 waves over 32-key tiles (d_k = 128 only; two waves per
// SIMD, so one issues while the other waits on LDS or on an MFMA result).
// Every operand a tile needs is in LDS before the tile starts; the next
// tile's operands stream in meanwhile with direct-to-LDS loads
// (global_load_lds, 64 lanes per load, lane l at LDS base + l * size), so the
// loop waits on global memory only at its single barrier per tile.
//  * K rows and a V^T tile (written transposed by the projection GEMM) are
//    double-buffered and shared by the waves. K rows are staged in the order
//    key(m) = m with bits 2 and 3 swapped, so the score MFMA's output
//    registers hold, per lane, 8 consecutive keys of each 16-key step:
//    exactly the B operand layout of the PV MFMA, whose V^T operand is then
//    one 16-byte LDS read.
//  * Position rows live in a ring of QB + 2 NK rows. Wave w needs, for key
//    tile k, 32 (NU + 1) rows (NU = NK / 32) starting at
//    pb_w = center - qoff - (i_w + 31) + j0: NU + 1 band tiles of 32 rows
//    covering the pairs of its 32 queries and NK keys; the last band tile of
//    one key tile is the first of the next, so NU are computed per step.
//    Ring row rr holds position row R0 + rr with R0 the first row any wave
//    needs: tile k uses rr in [NK k, NK k + QB + NK) and loads
//    [NK k + QB + NK, NK k + QB + 2 NK) for tile k + 1.
//  * LDS rows are unpadded; 16-byte chunk j of a K or ring row r sits at
//    chunk j ^ (r % 16), so the 16 lanes an LDS read serves together hit 16
//    distinct bank groups; V^T rows are keyed by Cfg2::vkey.
//  * q_u = q + pos_bias_u and q_v = q + pos_bias_v are both held in
//    registers (bf16, as the reference adds them in the activation dtype,
//    attention.rs:501-508): q_u for the scores, q_v for the band.
//  * bd is rounded to bf16 in the remap strip, as the reference stores
//    matrix_bd in bf16 (attention.rs:530). The logits are
//    s * (q_u k) + bf16(bd * bf16(s)): the reference hands the position term
//    to the attention as the bf16 array matrix_bd * cast(s) (attention.rs:
//    308-311), one more bf16 rounding after the product. At the quantized
//    stack's logits (~1e3) that rounding moves a logit by several units, so
//    it is reproduced, not folded into one fp32 scale.
// ---------------------------------------------------------------------------
template <int DK, int NW>
struct Cfg2 {
  static constexpr int NT = 64 * NW;
  static constexpr int QB = 32 * NW;
  static constexpr int NK = NW == 8 ? 32 : 64;   // keys per tile
  static constexpr int NU = NK / 32;             // 32-key score blocks (and new band tiles) per tile
  static constexpr int RB = DK * 2;              // bytes per K / position row
  static constexpr int KCN = RB / 16;            // 16-byte chunks per K / position row
  static constexpr int VCN = NK * 2 / 16;        // 16-byte chunks per V^T row
  // XOR key of V^T row d's chunks. A 16-lane group of an LDS read takes 16
  // consecutive rows at one chunk index: with 128-byte rows (8 chunks) two
  // rows share each 16-byte bank group, keyed by d % 8; with 64-byte rows
  // (4 chunks) rows d, d + 4, d + 8, d + 12 share one quarter of the banks
  // and take distinct chunks by (d / 4) % 4.
  static __device__ __forceinline__ int vkey(int d) { return VCN == 4 ? (d >> 2) & 3 : d % VCN; }
  static constexpr int RING = QB + 2 * NK;       // position ring rows
  static constexpr int RMP = 32 * (NU + 1) + 4;  // remap row pitch (bf16 elements)
  static constexpr int KBUF = NK * RB;
  static constexpr int VBUF = DK * NK * 2;
  static constexpr int K_OFF = 0;                    // two K tiles
  static constexpr int V_OFF = 2 * KBUF;             // two V^T tiles
  static constexpr int P_OFF = V_OFF + 2 * VBUF;     // position ring
  static constexpr int R_OFF = P_OFF + RING * RB;    // remap strips
  static constexpr int LDS = R_OFF + NW * 32 * RMP * 2;
  static constexpr int NS = DK / 16;                 // 16-wide d_k steps
  static constexpr int KDMA = KBUF / 1024 / NW;      // 1 KB direct-to-LDS loads per wave and tile
  static constexpr int VDMA = VBUF / 1024 / NW;
  static constexpr int RPL = 1024 / RB;              // position rows per 1 KB load
  static constexpr int PDMA = NK / RPL / NW;         // position loads per wave for NK rows
  static_assert(KDMA * NW * 1024 == KBUF && VDMA * NW * 1024 == VBUF && PDMA * NW * RPL == NK, "tile split");
  static_assert(KDMA + VDMA <= NS && PDMA <= NS, "one load per band / score MFMA step");
  static_assert(LDS <= 160 * 1024, "LDS");
};

// bf16(v) (round to nearest even) as an fp32 value from one packed
// conversion: with 0 as its low input, the high half holds bf16(v) and the
// word is that value in fp32. (Written as the instruction: from the
// equivalent vector expression the compiler converts into the low half and
// then moves it up, two instructions.) v comes from a vector ALU result.
__device__ __forceinline__ float bf16_as_f32(float v) {
  bf16x2 r;
  asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(v));
  return __builtin_bit_cast(float, r);
}

// max and sum of v over lanes l and l ^ 32, with the halves of the wave
// exchanged by v_permlane32_swap (a vector ALU op; the equivalent shuffle is
// an LDS permute with its own address arithmetic). After the swap a holds
// v of lanes 0-31 in both halves and b v of lanes 32-63. (The compiler's
// builtin for the instruction returned one value for both operands here,
// so it is written as the instruction, with the wait states around it.)
__device__ __forceinline__ void halves(float v, float& a, float& b) {
  a = v;
  b = v;
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float max_xor32(float v) {
  float a, b;
  halves(v, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float sum_xor32(float v) {
  float a, b;
  halves(v, a, b);
  return a + b;
}

// Tile-local key held by LDS K row m (an involution on [0, 32) and [0, 64)).
__device__ __forceinline__ constexpr int swap23(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

typedef __attribute__((address_space(3))) void lds_void;
typedef __bf16 bf16x8_a2 __attribute__((ext_vector_type(8), aligned(2)));

// The kernel's work as workgroup `block` of `nblocks` (a multiple of 8), in
// `smem` (C::LDS bytes, 16-byte aligned), over the nb items p.order[ord0 ..
// ord0 + nb).
template <int DK, int NW, bool DEBUG, bool SKIP = false>
__device__ __forceinline__ void attn_bf16_body(const AttnParams& p, int nb, int block, int nblocks, char* smem,
                                               int ord0 = 0) {
  using C = Cfg2<DK, NW>;
  constexpr int QB = C::QB, NK = C::NK, NU = C::NU, NS = C::NS, RB = C::RB;
  constexpr int PF = 3;  // MFMA steps an LDS operand read is issued ahead

  // Work order for 8 XCDs: workgroup L runs on XCD L % 8, so each XCD gets a
  // contiguous range of (head, item, query block) work items and keeps those
  // heads' position rows and K/V in its own L2.
  const int nqb = (p.T + QB - 1) / QB;
  const int per = nblocks / 8;
  const int W = (int)((unsigned)block % 8u) * per + (int)((unsigned)block / 8u);
  if (W >= nqb * nb * p.H) return;
  const int tid = threadIdx.x, lane = tid & 63, hh = lane >> 5, c = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index (uniform)
  const int bl = p.order[ord0 + (W / nqb) % nb], b = p.b0 + bl, h = W / (nqb * nb);
  const int i0 = (W % nqb) * QB;
  const int iw = i0 + 32 * w;  // first query of this wave
  const int qi = iw + c;       // this lane's query column
  // Remap strip row of this query column: band value n at Rs[n], written 4
  // rows at a time (8-byte aligned), read 8 keys at a time at n = 31 - c + 8k
  // (2-byte aligned 16-byte reads, which the LDS serves unaligned).
  bf16* Rs = reinterpret_cast<bf16*>(smem + C::R_OFF) + (w * 32 + c) * C::RMP;

  // q_u fragments (B operand): lane holds d_k values 16s + 8hh + [0, 8).
  // Rows past T read the last row (finite; their keys are all masked).
  bf16x8 qu[NS], qv[NS];
  {
    const bf16* qrow =
        reinterpret_cast<const bf16*>(p.q) + (int64_t)b * p.q_bs + (int64_t)min(qi, p.T - 1) * p.q_rs + h * DK;
    const float* bu = p.bias_u + h * DK;
    const float* bv = p.bias_v + h * DK;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int d0 = 16 * s + 8 * hh;
      const bf16x8 raw = *reinterpret_cast<const bf16x8*>(qrow + d0);
      const floatx4 b0 = *reinterpret_cast<const floatx4*>(bu + d0);
      const floatx4 b1 = *reinterpret_cast<const floatx4*>(bu + d0 + 4);
      const floatx4 c0 = *reinterpret_cast<const floatx4*>(bv + d0);
      const floatx4 c1 = *reinterpret_cast<const floatx4*>(bv + d0 + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qu[s][e] = (bf16)((float)raw[e] + b0[e]);
        qu[s][e + 4] = (bf16)((float)raw[e + 4] + b1[e]);
        qv[s][e] = (bf16)((float)raw[e] + c0[e]);
        qv[s][e + 4] = (bf16)((float)raw[e + 4] + c1[e]);
      }
    }
  }

  floatx16 o[DK / 32];
  float l_run;

  int jbeg, jend;
  key_range(p, bl, i0, min(i0 + QB, p.T), jbeg, jend);
  const int2 iv = query_interval(p, bl, qi);
  // logits are formed already scaled (s q_u k + bf16(bd cast(s))), so the
  // exponent base change is the only factor left
  const float sc = kLog2e;
  const float lim = 100.f / sc;  // largest (logit - reference) kept without rescaling: 2^100
  // DEBUG: this lane's best visible key so far (lowest index on ties)
  float top_v = -INFINITY;
  int top_j = -1;
  const int jfirst = (jbeg / NK) * NK;
  // ring row rr holds position row R0 + rr
  const int R0 = p.center - p.qoff - (i0 + 31) + jfirst - 32 * (NW - 1);

  const char* kbase = reinterpret_cast<const char*>(p.k) + ((int64_t)b * p.kv_bs + h * DK) * 2;
  const char* vtbase = reinterpret_cast<const char*>(p.vt) + ((int64_t)h * DK * p.vt_ld + (int64_t)b * p.vt_bs) * 2;
  const char* pbase = reinterpret_cast<const char*>(p.p) + h * DK * 2;

  // Direct-to-LDS loads (buffer_load ... lds): each stream has a buffer
  // resource over its readable range, a uniform per-tile offset (soffset) and
  // a loop-invariant 32-bit offset per lane. Load g of this wave fills LDS
  // chunks 64g' + [0, 64) of its buffer, g' = w * (loads per wave) + g. Bytes
  // past a resource's range read as zero.
  constexpr int kRawBuffer = 0x00020000;  // descriptor dword 3: untyped 32-bit data
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
      (void*)kbase, (short)0, (int)((int64_t)(p.T + p.kv_pad) * p.kv_rs * 2 - h * DK * 2), kRawBuffer);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc((void*)vtbase, (short)0, (int)((int64_t)DK * p.vt_ld * 2), kRawBuffer);
  const char* pslack = pbase - (int64_t)p.p_pad * p.p_rs * 2;  // first readable position row
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      (void*)pslack, (short)0, (int)((int64_t)(p.p_rows + 2 * p.p_pad) * p.p_rs * 2 - h * DK * 2), kRawBuffer);
  // (passed to the builtins as (int) prvalues: an argument naming a variable
  // the lambda captured by reference makes the host compilation pass drop
  // the kernel's launch stub)
  int koff[C::KDMA], voff[C::VDMA], roff[C::PDMA];
#pragma unroll
  for (int g = 0; g < C::KDMA; ++g) {
    const int pos = (w * C::KDMA + g) * 64 + lane, m = pos / C::KCN;
    koff[g] = (int)(swap23(m) * p.kv_rs * 2 + 16 * ((pos % C::KCN) ^ (m % C::KCN)));
  }
#pragma unroll
  for (int g = 0; g < C::VDMA; ++g) {
    const int pos = (w * C::VDMA + g) * 64 + lane, d = pos / C::VCN;
    voff[g] = (int)(d * p.vt_ld * 2 + 16 * ((pos % C::VCN) ^ C::vkey(d)));
  }
#pragma unroll
  for (int g = 0; g < C::PDMA; ++g) {
    const int lr = (w * C::PDMA + g) * C::RPL + lane / C::KCN;  // ring row - rr0
    roff[g] = (int)(lr * p.p_rs * 2 + 16 * ((lane % C::KCN) ^ (lr % C::KCN)));
  }

  // Key tile j0 into buffer buf. Rows past the item's last key belong to the
  // next item or to the kv_pad slack after the last one: finite, and masked.
  auto load_tile = [&](int j0, int buf) {
    char* Ks = smem + C::K_OFF + buf * C::KBUF;
    char* Vt = smem + C::V_OFF + buf * C::VBUF;
    const int ks = j0 * (int)p.kv_rs * 2;
#pragma unroll
    for (int g = 0; g < C::KDMA; ++g)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(Ks + (w * C::KDMA + g) * 1024), 16, (int)koff[g], ks, 0, 0);
#pragma unroll
    for (int g = 0; g < C::VDMA; ++g)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(Vt + (w * C::VDMA + g) * 1024), 16, (int)voff[g], j0 * 2, 0,
                                               0);
  };
  // single loads of the same streams: load g of this wave's K and V^T share
  // of key tile jn into buffer bn; load g of its ring share
  auto dma_kv = [&](int g, int jn, int bn) {
    if (g < C::KDMA)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(smem + C::K_OFF + bn * C::KBUF + (w * C::KDMA + g) * 1024), 16,
                                               (int)koff[g], jn * (int)p.kv_rs * 2, 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(smem + C::V_OFF + bn * C::VBUF + (w * C::VDMA + g - C::KDMA) * 1024),
                                               16, (int)voff[g - C::KDMA], jn * 2, 0, 0);
  };
  auto dma_ring = [&](int g, int rr0) {
    const int n0 = R0 + rr0 + p.p_pad;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rp, (lds_void*)(smem + C::P_OFF + ((rr0 + (w * C::PDMA + g) * C::RPL) % C::RING) * RB), 16, (int)roff[g],
        n0 * (int)p.p_rs * 2, 0, 0);
  };
  // Ring rows [rr0, rr0 + NK) (rr0 a multiple of NK): this wave's share of
  // the position rows. Rows outside the table read the p_pad slack around it
  // (finite).
  // Every pair reading such a row lies outside its query's interval (past the
  // last key or query, or beyond a window the table was checked to cover), so
  // it is masked, and the values it reads cannot reach the output.
  auto load_ring = [&](int rr0) {
    char* ring = smem + C::P_OFF;
    const int n0 = R0 + rr0 + p.p_pad;  // row index from the first readable row
#pragma unroll
    for (int g = 0; g < C::PDMA; ++g)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rp, (lds_void*)(ring + ((rr0 + (w * C::PDMA + g) * C::RPL) % C::RING) * RB), 16, (int)roff[g],
          n0 * (int)p.p_rs * 2, 0, 0);
  };

  // This lane's byte offset of the 16-byte chunk 2st + hh of row c in a
  // K tile or ring block of 32 rows starting at a multiple of 32.
  int lo[NS];
#pragma unroll
  for (int st = 0; st < NS; ++st) lo[st] = c * RB + 16 * ((2 * st + hh) ^ (c % C::KCN));
  // Band tile of 32 ring rows from rr (a multiple of 32): initial accumulator
  // (row rr + 8a + 4hh + e in register 4a + e) and MFMAs.
  auto band_tile = [&](int rr) {
    floatx16 acc = floatx16{};
    const char* rb = smem + C::P_OFF + (rr % C::RING) * RB;
#pragma unroll
    for (int st = 0; st < NS; ++st) acc = mma32(*reinterpret_cast<const bf16x8*>(rb + lo[st]), qv[st], acc);
    return acc;
  };

  // Band tile t of the current key tile goes to remap strip columns
  // 32t + [0, 32), rounded to bf16 (this lane: rows 8a + 4hh + [0, 4)).
  auto pack = [&](const floatx16& bt) {
    bf16x16 v;
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = (bf16)bt[i];
    return v;
  };
  auto put = [&](const bf16x16& v, int t) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
      *reinterpret_cast<bf16x4*>(Rs + 32 * t + 8 * a + 4 * hh) = bf16x4{v[4 * a], v[4 * a + 1], v[4 * a + 2], v[4 * a + 3]};
  };

  // Softmax with a lazily moved reference per query: probabilities are
  // 2^((x - m_ref) s log2 e), with m_ref the first finite tile maximum of the
  // query (o and l are still zero until then). A later maximum above m_ref
  // makes probabilities larger than 1; up to 2^100 that stays far from fp32
  // and bf16 overflow for any key count, so o and l are only rescaled (to the
  // new tile maximum) when a tile maximum exceeds the reference by more than
  // that, which ordinary inputs never do. The final division by l removes the
  // reference.
  float m_ref = -INFINITY;
#pragma unroll
  for (int d = 0; d < DK / 32; ++d) o[d] = floatx16{};
  l_run = 0.f;
  // ring row of band tile 0 of this wave for key tile k: NK k + 32 (NW - 1 - w)
  int rrw = 32 * (NW - 1 - w);
  bf16x16 carry = bf16x16{};  // band tile 0 of the current key tile, as stored
  if (jfirst < jend) {
    load_tile(jfirst, 0);
#pragma unroll
    for (int rr = 0; rr < QB + NK; rr += NK) load_ring(rr);
  }
  __syncthreads();
  if (jfirst < jend) carry = pack(band_tile(rrw));

  bool have_carry = true;  // carry holds band tile 0 of the current key tile
  // Key tile j0 from LDS buffer BUF::value, a literal in each of the loop's
  // two calls below, so that the buffer's base folds into the immediate
  // offsets of the K and V^T fragment reads.
  auto key_tile = [&](int j0, auto BUF) {
    constexpr int buf = decltype(BUF)::value;
    const bool more = j0 + NK < jend;
    // the next key tile and its 64 new ring rows (last read before the
    // previous barrier; awaited at the next one), issued one load per MFMA
    // step of the band and score loops below: in one burst they stall the
    // wave while the memory pipe takes them. The last tile reloads itself,
    // unused, so that every iteration issues the same loads.
    const int jn = more ? j0 + NK : j0, rr0n = rrw - 32 * (NW - 1 - w) + QB + NK;

    // SKIP (8-wave form under a limited context): a wave none of whose
    // queries sees a key of this tile only issues its share of the loads.
    // The tile would add nothing (every probability 0; o, l and the
    // reference unchanged), and the other wave of its SIMD then has the SIMD
    // to itself. Under a window, a 256-query block's first and last tiles lie
    // outside most of its waves' windows. (In the 4-wave form each SIMD holds
    // one wave and the tile barrier waits for the slowest, so skipping there
    // measured slower; without a window no tile is skipped, and the check
    // alone measured 4% slower on 1500-frame items. The debug exports cover
    // every tile.)
    if constexpr (SKIP) {
      if (__all(iv.x >= iv.y || iv.y <= j0 || iv.x >= j0 + NK)) {
#pragma unroll
        for (int g = 0; g < C::KDMA + C::VDMA; ++g) dma_kv(g, jn, buf ^ 1);
#pragma unroll
        for (int g = 0; g < C::PDMA; ++g) dma_ring(g, rr0n);
        rrw += NK;
        have_carry = false;
        __syncthreads();
        return;
      }
    }
    // after a skipped tile, band tile 0 from its ring rows (present since
    // the last barrier)
    if (!have_carry) {
      carry = pack(band_tile(rrw));
      have_carry = true;
    }

    // Band tiles first, then the score MFMAs, and the band tiles are stored
    // to the remap strip (rel_shift: strip column n of query column c pairs
    // with key j0 + n - 31 + c) while the score chains finish: the band
    // chains' last results are ready by then, and the strip writes' latency
    // runs beside the score MFMAs (the 4 x 1500-frame attention of the u8
    // layer stack measured 3% faster than storing each band tile as soon as
    // its chain ends).
    put(carry, 0);
    floatx16 bt[NU];
    {
      // band tiles 1 .. NU as interleaved MFMA chains
      const char* rbt[NU];
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        bt[u] = floatx16{};
        rbt[u] = smem + C::P_OFF + ((rrw + 32 * (u + 1)) % C::RING) * RB;
      }
      // operand reads run PF steps ahead of the MFMAs; the sched_barriers pin
      // that order (the LDS latency is several MFMAs long)
      bf16x8 ab[PF][NU];
#pragma unroll
      for (int st = 0; st < PF; ++st)
#pragma unroll
        for (int u = 0; u < NU; ++u) ab[st][u] = *reinterpret_cast<const bf16x8*>(rbt[u] + lo[st]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int st = 0; st < NS; ++st) {
#pragma unroll
        for (int u = 0; u < NU; ++u) bt[u] = mma32(ab[st % PF][u], qv[st], bt[u]);
        if (st + PF < NS)
#pragma unroll
          for (int u = 0; u < NU; ++u) ab[st % PF][u] = *reinterpret_cast<const bf16x8*>(rbt[u] + lo[st + PF]);
        if (st < C::KDMA + C::VDMA) dma_kv(st, jn, buf ^ 1);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    rrw += NK;

    // S = K . q_u: output row m of block u is key 32u + swap23(m)
    const char* Ks = smem + C::K_OFF + buf * C::KBUF;
    floatx16 s[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) s[u] = floatx16{};
    {
      bf16x8 ka[PF][NU];
#pragma unroll
      for (int st = 0; st < PF; ++st)
#pragma unroll
        for (int u = 0; u < NU; ++u) ka[st][u] = *reinterpret_cast<const bf16x8*>(Ks + 32 * u * RB + lo[st]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int st = 0; st < NS; ++st) {
#pragma unroll
        for (int u = 0; u < NU; ++u) s[u] = mma32(ka[st % PF][u], qu[st], s[u]);
        if (st + PF < NS)
#pragma unroll
          for (int u = 0; u < NU; ++u)
            ka[st % PF][u] = *reinterpret_cast<const bf16x8*>(Ks + 32 * u * RB + lo[st + PF]);
        if (st < C::PDMA) dma_ring(st, rr0n);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // the band tiles to the strip, their chains done while the score MFMAs ran
#pragma unroll
    for (int u = 0; u + 1 < NU; ++u) put(pack(bt[u]), u + 1);
    carry = pack(bt[NU - 1]);
    put(carry, NU);
    __builtin_amdgcn_wave_barrier();

    // x = q_u k + bd for this lane's keys jl(u, r) = 32u + 16(r / 8) + 8hh + r % 8:
    // 8 consecutive keys per 16-byte read
    // Strip column 31 - c + jl holds key jl's value: an odd column for even c.
    // The 8 keys of a read come from 5 bf16 pairs read 4-byte aligned and
    // shifted by 0 or 16 bits per lane (unaligned 16-byte LDS reads cost the
    // strip phase about 600 cycles per tile).
    const int n0 = 31 - c + 8 * hh;
    const bf16x2* rd = reinterpret_cast<const bf16x2*>(Rs) + (n0 >> 1);
    const unsigned sh = 16u * (unsigned)(n0 & 1);
    float tmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        // (read as bf16 pairs, the element type the strip is written with, so
        // no type-based alias analysis can move it across those writes)
        const bf16x2* d = rd + 16 * u + 8 * g;
        uint32_t wv[5];
#pragma unroll
        for (int k = 0; k < 5; ++k) wv[k] = __builtin_bit_cast(uint32_t, d[k]);
        u32x4 al;
#pragma unroll
        for (int k = 0; k < 4; ++k) al[k] = __builtin_amdgcn_alignbit(wv[k + 1], wv[k], sh);
        const bf16x8 q8 = __builtin_bit_cast(bf16x8, al);
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            // the position term as the reference materialises it:
            // bf16(bf16(bd) * bf16(s)) (attention.rs:308-311)
            const float tb = bf16_as_f32((float)q8[e + k] * p.scale_bd);
            if (DEBUG && p.dbg_bd) {
              const int j = j0 + 32 * u + 16 * g + 8 * hh + e + k;
              if (qi < p.T && j < p.L) p.dbg_bd[(((int64_t)b * p.H + h) * p.T + qi) * p.L + j] = tb;
            }
            s[u][8 * g + e + k] = __builtin_fmaf(s[u][8 * g + e + k], p.scale, tb);
          }
        }
      }
    __builtin_amdgcn_wave_barrier();
    if (!__all(iv.x <= j0 && iv.y >= j0 + NK)) {  // some key of the tile is hidden from some query
      // key j = j0 + 8hh + jl(u, r) is visible iff j - lo < hi - lo (unsigned);
      // the opaque base keeps the 32 per-lane offsets from being hoisted out
      // of the loop into registers
      int jb = j0 + 8 * hh - iv.x;
      asm volatile("" : "+v"(jb));
      const unsigned span = (unsigned)(iv.y - iv.x);
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if ((unsigned)(jb + 32 * u + 16 * (r >> 3) + (r & 7)) >= span) s[u][r] = -INFINITY;
    }
    if (DEBUG && p.dbg_top) {
      // keys in increasing order within the lane; strict > keeps the lowest
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (s[u][r] > top_v) {
            top_v = s[u][r];
            top_j = j0 + 32 * u + 16 * (r >> 3) + 8 * hh + (r & 7);
          }
    }
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, s[u][r]);
    tmax = max_xor32(tmax);
    if (m_ref == -INFINITY) m_ref = tmax;
    if (__any(tmax > m_ref + lim)) {
      // (o holds only this lane's query: its column of O^T)
      const bool up = tmax > m_ref + lim;
      const float a = up ? __builtin_amdgcn_exp2f((m_ref - tmax) * sc) : 1.f;
      m_ref = up ? tmax : m_ref;
#pragma unroll
      for (int d = 0; d < DK / 32; ++d) o[d] *= a;
      l_run *= a;
    }
    const float msc = m_ref == -INFINITY ? 0.f : m_ref * sc;
    float psum = 0.f;
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[u][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u][r], sc, -msc));  // exp2(-inf) = 0
        psum += s[u][r];
      }
    l_run += psum;

    // O^T += V^T P^T over 16-key steps (u, jj): k-slot e of lane (c, hh) is
    // key 32u + 16jj + 8hh + e, register 8jj + e of block u.
    // (the V^T operands of the next 16-key step are read during this one)
    const char* Vrow = smem + C::V_OFF + buf * C::VBUF + c * (NK * 2);
    {
      bf16x8 vo[2][DK / 32];
      auto vread = [&](int step, bf16x8* dst) {
        const char* va = Vrow + 16 * ((2 * step + hh) ^ C::vkey(c));  // step = 2u + jj (row 32d + c: same key)
#pragma unroll
        for (int d = 0; d < DK / 32; ++d) dst[d] = *reinterpret_cast<const bf16x8*>(va + 32 * d * (NK * 2));
      };
      vread(0, vo[0]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int step = 0; step < NK / 16; ++step) {
        if (step + 1 < NK / 16) vread(step + 1, vo[(step + 1) & 1]);
        const int u = step >> 1, jj = step & 1;
        bf16x8 pb8;
#pragma unroll
        for (int e = 0; e < 8; ++e) pb8[e] = (bf16)s[u][8 * jj + e];
#pragma unroll
        for (int d = 0; d < DK / 32; ++d) o[d] = mma32(vo[step & 1][d], pb8, o[d]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }

    __syncthreads();  // waits for this wave's loads of the next tile first
  };
  for (int j0 = jfirst; j0 < jend; j0 += 2 * NK) {
    key_tile(j0, std::integral_constant<int, 0>{});
    if (j0 + NK < jend) key_tile(j0 + NK, std::integral_constant<int, 1>{});
  }

  const float l_tot = sum_xor32(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (DEBUG && p.dbg_top) {
    // merge with the lane holding the other 8-key halves of this query
    const float ov = __shfl_xor(top_v, 32, 64);
    const int oj = __shfl_xor(top_j, 32, 64);
    if (ov > top_v || (ov == top_v && oj >= 0 && (top_j < 0 || oj < top_j))) {
      top_v = ov;
      top_j = oj;
    }
    if (hh == 0 && qi < p.T) {
      const int64_t r = ((int64_t)b * p.H + h) * p.T + qi;
      p.dbg_top[r] = top_j;
      p.dbg_topv[r] = top_v;
    }
  }
  // The output goes through LDS: the accumulators hold one query per lane
  // (32 rows under a wave), the stores then write whole 16-byte runs of
  // each row. The position ring is free: the loop's last barrier is behind
  // every wave's last read of it.
  {
    constexpr int OP = DK * 2 + 16;  // staged row pitch (bytes)
    static_assert(C::NT / 64 * 32 * OP <= C::RING * RB, "output staging fits the ring");
    char* stg = smem + C::P_OFF + w * 32 * OP;
#pragma unroll
    for (int d = 0; d < DK / 32; ++d)
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        bf16x4 v4;
#pragma unroll
        for (int e = 0; e < 4; ++e) v4[e] = (bf16)(o[d][4 * a + e] * inv);
        *reinterpret_cast<bf16x4*>(stg + c * OP + (32 * d + 8 * a + 4 * hh) * 2) = v4;
      }
    asm volatile("" ::: "memory");  // (LDS serves one wave's accesses in order)
    constexpr int CPR = DK * 2 / 16, RPI = 64 / CPR;  // 16-byte chunks per row, rows per instruction
    const int ch = lane % CPR;
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int r = lane / CPR + RPI * i, q = iw + r;
      const u32x4 v = *reinterpret_cast<const u32x4*>(stg + r * OP + ch * 16);
      if (q < p.T)
        *reinterpret_cast<u32x4*>(reinterpret_cast<bf16*>(p.o) + (int64_t)b * p.o_bs + (int64_t)q * p.o_rs + h * DK +
                                  ch * 8) = v;
    }
  }
}

template <int DK, int NW, bool DEBUG, bool SKIP = false>
__global__ __launch_bounds__(64 * NW) void attn_bf16_kernel(const AttnParams p, int nb) {
  __shared__ __attribute__((aligned(16))) char smem[Cfg2<DK, NW>::LDS];
  attn_bf16_body<DK, NW, DEBUG, SKIP>(p, nb, (int)blockIdx.x, (int)gridDim.x, smem);
}

// The bf16 attention (d_k = 128) of p's items in both forms in one launch:
// items p.order[0, nb4) in the 4-wave form in workgroups [0, n4) (waves 4-7
// end at once), items p.order[nb4, nb) in the 8-wave form in workgroups
// [n4, n4 + n8), and, with GEMM, the tile GEMM `g` in the workgroups after
// them: a projection that does not depend on the attention (the next layer's
// position rows). Workgroups are dispatched in index order, so every
// attention workgroup has its CU before the first GEMM tile, and the tiles
// take the CUs the attention leaves idle. A GEMM workgroup runs the tile body
// on its first 4 waves.
template <bool GEMM, int GBM, int GBN, bool GQ, int GNS>
__global__ __launch_bounds__(512) void attn_bf16_mixed_kernel(const AttnParams p, int nb4, int n4, int nb, int n8,
                                                              const GemmParams g) {
  constexpr int L4 = Cfg2<128, 4>::LDS, L8 = Cfg2<128, 8>::LDS, LG = GEMM ? TileCfg<GBM, GBN, GQ, GNS>::LDS : 0;
  constexpr int LA = L4 > L8 ? L4 : L8;
  __shared__ __attribute__((aligned(1024))) char smem[LA > LG ? LA : LG];
  const int block = (int)blockIdx.x;
  if (block < n4) {
    if (threadIdx.x < 256) attn_bf16_body<128, 4, false>(p, nb4, block, n4, smem, 0);
  } else if (block < n4 + n8) {
    attn_bf16_body<128, 8, false>(p, nb - nb4, block - n4, n8, smem, nb4);
  } else if constexpr (GEMM) {
    if (threadIdx.x < 256) gemm_tile_body<GBM, GBN, GQ, GNS>(g, block - n4 - n8, smem);
  }
}

// Items in launch order, longest key range first, so that the work left for
// a second round of workgroups is the shortest; returns the workgroup count
// (a multiple of 8), or -1 when the grid would be too large.
template <int DK, int NW>
int64_t order_items(AttnParams& p, int nb) {
  using C = Cfg2<DK, NW>;
  const int64_t work = (int64_t)(p.T + C::QB - 1) / C::QB * p.H * nb;
  if (work > (1 << 30)) return -1;
  // items by descending work (query blocks x key tiles), ties in item order
  int64_t cost[kMaxBatch];
  for (int bl = 0; bl < nb; ++bl) {
    int jbeg, jend;
    key_range(p, bl, 0, p.T, jbeg, jend);
    const int rows = imin(p.q_valid[bl], p.T);
    cost[bl] = jend > jbeg && rows > 0 ? (int64_t)((rows + C::QB - 1) / C::QB) * ((jend - jbeg + C::NK - 1) / C::NK) : 0;
    p.order[bl] = bl;
  }
  std::stable_sort(p.order, p.order + nb, [&](int a, int b) { return cost[a] > cost[b]; });
  return (work + 7) / 8 * 8;
}

template <int DK, int NW, bool DEBUG, bool SKIP = false>
hipError_t launch2(AttnParams p, int nb, hipStream_t s) {
  const int64_t grid = order_items<DK, NW>(p, nb);
  if (grid < 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL((attn_bf16_kernel<DK, NW, DEBUG, SKIP>), dim3((unsigned)grid), dim3(Cfg2<DK, NW>::NT), 0, s,
                     p, nb);
  count_form(NW == 4 ? kFormBf16Wave4 : SKIP ? kFormBf16Wave8Skip : kFormBf16Wave8);
  return hipGetLastError();
}

// The 8-wave form (d_k = 128) where its 256-query blocks give at least
// kWide8 workgroups; otherwise the 4-wave form. (Under a limited context a
// 256-query block spans the key tiles of all its waves' windows, 512 keys
// on +-128-frame windows against 384 for a 128-query block; its waves pass
// over the tiles outside their own windows, and over 7500 frames the 8-wave
// form measured 6% faster than the 4-wave form.)
constexpr int kWide8 = 160;
// a window or chunk limits the keys some queries see
bool windowed(const AttnParams& p) { return p.has_ctx && (p.left >= 0 || p.right >= 0); }
template <int DK>
bool use_wide(const AttnParams& p, int nb) {
  if constexpr (DK != 128) return false;
  return (int64_t)(p.T + Cfg2<128, 8>::QB - 1) / Cfg2<128, 8>::QB * p.H * nb >= kWide8;
}

// Items of an 8-wave launch moved to the 4-wave form. The 8-wave form does
// more work per CU (measured ~4400 cycles per 32-key tile of a 256-query
// block against ~5450 per 64-key tile of a 128-query block); the 4-wave form
// spreads an item over twice the workgroups. When the 8-wave blocks take one
// round of workgroups with CUs left idle, the longest items, moved to the
// 4-wave form while the busy blocks still fit the CUs, finish sooner, and
// the launch ends with its slowest block.
struct FormSplit {
  int nb4 = 0;             // items p.order[0, nb4) in the 4-wave form
  int64_t n4 = 0, n8 = 0;  // workgroups of each form (multiples of 8)
};
constexpr int64_t kTile8 = 4400, kTile4 = 5450, kBlockFixed = 11000;  // cycles
FormSplit split_forms(AttnParams& p, int nb) {
  using C4 = Cfg2<128, 4>;
  using C8 = Cfg2<128, 8>;
  FormSplit f;
  int64_t c4[kMaxBatch], c8[kMaxBatch];
  int busy4[kMaxBatch], busy8[kMaxBatch];
  for (int bl = 0; bl < nb; ++bl) {
    int jbeg, jend;
    key_range(p, bl, 0, p.T, jbeg, jend);
    const int rows = imin(p.q_valid[bl], p.T), keys = jend > jbeg && rows > 0 ? jend - jbeg : 0;
    c8[bl] = keys ? kBlockFixed + kTile8 * ((keys + C8::NK - 1) / C8::NK) : 0;
    c4[bl] = keys ? kBlockFixed + kTile4 * ((keys + C4::NK - 1) / C4::NK) : 0;
    busy8[bl] = keys ? (rows + C8::QB - 1) / C8::QB * p.H : 0;
    busy4[bl] = keys ? (rows + C4::QB - 1) / C4::QB * p.H : 0;
    p.order[bl] = bl;
  }
  std::stable_sort(p.order, p.order + nb, [&](int a, int b) { return c8[a] > c8[b]; });
  int64_t busy = 0;
  for (int i = 0; i < nb; ++i) busy += busy8[p.order[i]];
  const int cus = device_cus();
  int best = 0;
  int64_t best_t = nb ? c8[p.order[0]] : 0, head4 = 0;
  for (int k = 1; k <= nb && busy <= cus; ++k) {
    const int it = p.order[k - 1];
    busy += busy4[it] - busy8[it];
    head4 = std::max(head4, c4[it]);
    const int64_t t = std::max(head4, k < nb ? c8[p.order[k]] : int64_t(0));
    // switch forms only for a clear gain (3%) over the model's error
    if (busy <= cus && t * 100 < best_t * 97) {
      best = k;
      best_t = t;
    }
  }
  if (best == 0) return f;
  f.nb4 = best;
  f.n4 = ((int64_t)(p.T + C4::QB - 1) / C4::QB * p.H * best + 7) / 8 * 8;
  f.n8 = ((int64_t)(p.T + C8::QB - 1) / C8::QB * p.H * (nb - best) + 7) / 8 * 8;
  return f;
}

template <bool GEMM, int GBM, int GBN, bool GQ, int GNS>
void launch_mixed(const AttnParams& p, int nb, const FormSplit& f, const GemmParams& g, int64_t gtiles,
                  hipStream_t s) {
  hipLaunchKernelGGL((attn_bf16_mixed_kernel<GEMM, GBM, GBN, GQ, GNS>), dim3((unsigned)(f.n4 + f.n8 + gtiles)),
                     dim3(512), 0, s, p, f.nb4, (int)f.n4, nb, (int)f.n8, g);
  count_form(GEMM ? kFormBf16MixedGemm : kFormBf16Mixed);
}

template <int DK>
hipError_t dispatch_bf16(const AttnParams& p, int nb, hipStream_t s) {
  const bool dbg = p.dbg_bd || p.dbg_top;
  if constexpr (DK == 128) {
    if (use_wide<DK>(p, nb)) {
      if (dbg) return launch2<DK, 8, true>(p, nb, s);
      if (windowed(p)) return launch2<DK, 8, false, true>(p, nb, s);
      if ((int64_t)p.T * p.H * nb <= (1 << 28)) {
        AttnParams a = p;
        const FormSplit f = split_forms(a, nb);
        if (f.nb4) {
          launch_mixed<false, 128, 128, false, 4>(a, nb, f, GemmParams(), 0, s);
          return hipGetLastError();
        }
      }
      return launch2<DK, 8, false>(p, nb, s);
    }
  }
  return dbg ? launch2<DK, 4, true>(p, nb, s) : launch2<DK, 4, false>(p, nb, s);
}

// One row per DK/8 lanes: each lane takes 8 d_k values, then a lane-group sum.
// ---------------------------------------------------------------------------
// fp32 chunk kernel for short query blocks (the cache-aware streaming step:
// T <= 16 queries against L <= 96 keys of the cache ring). One workgroup of
// eight waves per (item, head) stages the visible key rows and the position
// rows they reach in LDS once (eight waves, not four: a wave with some 60
// loads in flight waits about twice as long per byte as one with 20, measured
// 2.0 against 1.0 us for 152 KB on one CU), then:
//   S  = q_u K^T           (16 x keys)            fp32 16x16x4 MFMAs
//   B' = q_v P'^T          (16 x (keys + 15))      over the rows
//        P' = P[r0 + m], r0 = center - qoff - 15 + jbeg; rel_shift reads
//        bd(i, j) = B'[i][j - jbeg + 15 - i]
//   softmax per query row (fp32, exact max), probabilities in LDS
//   O  = probs . V         (16 x d_k), V^T staged over the consumed K rows
// The work items are few (items x heads), so every wave takes whole 16x16
// output tiles and nothing waits on another workgroup.
// ---------------------------------------------------------------------------
template <int DK>
struct CfgS {
  static constexpr int NT = 512, NW = NT / 64, NQ = 16, LMAX = 96, PMAX = LMAX + NQ - 1;
  static constexpr int RP = DK * 4 + 16;                                // K / V / position row pitch (bytes)
  static constexpr int K_OFF = 0;                                       // K rows, later V rows
  static constexpr int P_OFF = LMAX * RP;                               // position rows
  static constexpr int RPI = NT / (DK / 4);                             // rows per pass of the workgroup
  static constexpr int PROWS = (PMAX + RPI - 1) / RPI * RPI;            // (RPI is a multiple of 16)
  // score and band rows padded by 4 words: the MFMA result stores (rows
  // 4g + e of one column) and the PV operand reads (16 rows) then fall on
  // distinct banks
  static constexpr int SLD = LMAX + 4, BLD = PROWS + 4;
  static constexpr int S_OFF = P_OFF + PROWS * RP;                      // scores / probabilities [NQ][SLD]
  static constexpr int B_OFF = S_OFF + NQ * SLD * 4;                    // band products [NQ][BLD]
  static constexpr int Q_OFF = B_OFF + NQ * BLD * 4;                   // q + pos_bias_u, then q + pos_bias_v rows
  static constexpr int LDS = Q_OFF + 2 * NQ * RP;
  static constexpr int KCH = LMAX / RPI;                                // K / V chunks per thread
  static constexpr int PCH = PROWS / RPI;                               // position chunks per thread
  static_assert(KCH * RPI == LMAX && PCH * RPI == PROWS && RPI % 16 == 0, "row split");
  static_assert(LDS <= 160 * 1024, "LDS");
};

template <int DK>
__global__ __launch_bounds__(CfgS<DK>::NT) void attn_chunk_f32_kernel(const AttnParams p) {
  using C = CfgS<DK>;
  constexpr int NQ = C::NQ, LMAX = C::LMAX, NS = DK / 16, NW = C::NW;
  __shared__ __attribute__((aligned(16))) char smem[C::LDS];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int rl = lane & 15, g = lane >> 4;  // MFMA row / column in the tile, k group
  const int h = blockIdx.x, bl = blockIdx.y, b = p.b0 + bl;
  float* out = reinterpret_cast<float*>(p.o) + (int64_t)b * p.o_bs + h * DK;

  int jbeg, jend;
  key_range(p, bl, 0, p.T, jbeg, jend);
  const int nk = max(jend - jbeg, 0);  // visible keys (<= LMAX)
  if (nk == 0) {                       // no query of this item sees a key: zeros
    for (int e = tid; e < p.T * DK; e += C::NT) out[(int64_t)(e / DK) * p.o_rs + e % DK] = 0.f;
    return;
  }
  const int nkt = (nk + 15) / 16;   // 16-key tiles
  const int np = nk + NQ - 1;       // position rows
  const int npt = (np + 15) / 16;
  const int r0 = p.center - p.qoff - (NQ - 1) + jbeg;
  const float* kb = reinterpret_cast<const float*>(p.k) + (int64_t)b * p.kv_bs + h * DK;
  const float* vb = reinterpret_cast<const float*>(p.v) + (int64_t)b * p.kv_bs + h * DK;
  const float* pb = reinterpret_cast<const float*>(p.p) + h * DK;

  // This thread's rows (tid / (DK/4) + RPI i) and 16-byte column chunk, read
  // through buffer descriptors: rows past the last visible key and position
  // rows past the band get an offset beyond the descriptor's range, so they
  // read as zero without a memory access (their scores are masked and their
  // probabilities are zero); every load is issued before the first store.
  constexpr int kRawBuffer = 0x00020000;  // descriptor dword 3: untyped 32-bit data
  const int krows = p.ring_len ? p.ring_len : p.L;
  const int kbytes = ((krows - 1) * (int)p.kv_rs + DK) * 4, pbytes = ((p.p_rows - 1) * (int)p.p_rs + DK) * 4;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)kb, (short)0, kbytes, kRawBuffer);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)vb, (short)0, kbytes, kRawBuffer);
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc((void*)pb, (short)0, pbytes, kRawBuffer);
  const int row0 = tid / (DK / 4), cb = (tid % (DK / 4)) * 4;
  int koff[C::KCH];
  {
    int rr = key_row(p, jbeg + min(row0, nk - 1));
#pragma unroll
    for (int i = 0; i < C::KCH; ++i) {
      const int row = row0 + C::RPI * i;
      koff[i] = row < nk ? (rr * (int)p.kv_rs + cb) * 4 : kbytes;
      rr += C::RPI;  // the next row of this thread: key + RPI (ring: mod ring_len)
      if (p.ring_len && rr >= p.ring_len) rr -= p.ring_len;
    }
  }
  u32x4 kr[C::KCH], vr[C::KCH], pr[C::PCH];
#pragma unroll
  for (int i = 0; i < C::KCH; ++i) kr[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, koff[i], 0, 0);
#pragma unroll
  for (int i = 0; i < C::PCH; ++i) {
    // rows outside the table meet only masked pairs: clamped (finite)
    const int row = row0 + C::RPI * i;
    const int n = min(max(r0 + row, 0), p.p_rows - 1);
    pr[i] = __builtin_amdgcn_raw_buffer_load_b128(rp, row < np ? (n * (int)p.p_rs + cb) * 4 : pbytes, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < C::KCH; ++i) vr[i] = __builtin_amdgcn_raw_buffer_load_b128(rv, koff[i], 0, 0);
  // q rows with the two position biases added, staged in LDS with the same
  // row split as the keys (one 16-byte chunk per thread; rows past T read as
  // zero): loading the MFMA fragments straight from memory in every wave
  // would put 16 rows under each 16 lanes, which the address unit serves at
  // a quarter of the rate of whole 64-byte runs
  const int qrow = tid / (DK / 4);
  floatx4 qx, qbu, qbv;
  {
    const float* qbase = reinterpret_cast<const float*>(p.q) + (int64_t)b * p.q_bs + h * DK;
    const int qbytes = ((p.T - 1) * (int)p.q_rs + DK) * 4;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)qbase, (short)0, qbytes, kRawBuffer);
    qx = __builtin_bit_cast(floatx4,
                            __builtin_amdgcn_raw_buffer_load_b128(rq, qrow < p.T ? (qrow * (int)p.q_rs + cb) * 4 : qbytes, 0, 0));
    qbu = *reinterpret_cast<const floatx4*>(p.bias_u + h * DK + cb);
    qbv = *reinterpret_cast<const floatx4*>(p.bias_v + h * DK + cb);
  }
#pragma unroll
  for (int i = 0; i < C::KCH; ++i)
    *reinterpret_cast<u32x4*>(smem + C::K_OFF + (row0 + C::RPI * i) * C::RP + cb * 4) = kr[i];
#pragma unroll
  for (int i = 0; i < C::PCH; ++i)
    *reinterpret_cast<u32x4*>(smem + C::P_OFF + (row0 + C::RPI * i) * C::RP + cb * 4) = pr[i];
  if (qrow < NQ) {
    *reinterpret_cast<floatx4*>(smem + C::Q_OFF + qrow * C::RP + cb * 4) = qx + qbu;
    *reinterpret_cast<floatx4*>(smem + C::Q_OFF + (NQ + qrow) * C::RP + cb * 4) = qx + qbv;
  }
  __syncthreads();

  // q_u, q_v A fragments: row rl, d_k values 16s + 4g + [0, 4)
  floatx4 qu[NS], qv[NS];
#pragma unroll
  for (int st = 0; st < NS; ++st) {
    const int d = 16 * st + 4 * g;
    qu[st] = *reinterpret_cast<const floatx4*>(smem + C::Q_OFF + rl * C::RP + d * 4);
    qv[st] = *reinterpret_cast<const floatx4*>(smem + C::Q_OFF + (NQ + rl) * C::RP + d * 4);
  }

  // score tiles (keys) and band tiles (position rows), spread over the waves
  float* Sl = reinterpret_cast<float*>(smem + C::S_OFF);
  float* Bl = reinterpret_cast<float*>(smem + C::B_OFF);
  for (int t = w; t < nkt + npt; t += NW) {
    const bool is_s = t < nkt;
    const int tt = is_s ? t : t - nkt;
    const char* rows = smem + (is_s ? C::K_OFF : C::P_OFF) + (tt * 16 + rl) * C::RP + 16 * g;
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
    if (is_s) {
#pragma unroll
      for (int st = 0; st < NS; ++st) acc = mma16(qu[st], *reinterpret_cast<const floatx4*>(rows + 64 * st), acc);
    } else {
#pragma unroll
      for (int st = 0; st < NS; ++st) acc = mma16(qv[st], *reinterpret_cast<const floatx4*>(rows + 64 * st), acc);
    }
    // C layout: lane holds rows 4g + e of column rl
    float* dst = is_s ? Sl + 4 * g * C::SLD + tt * 16 + rl : Bl + 4 * g * C::BLD + tt * 16 + rl;
    const int ld = is_s ? C::SLD : C::BLD;
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[e * ld] = acc[e];
  }
  __syncthreads();

  // V rows over the K rows (all K reads are done)
#pragma unroll
  for (int i = 0; i < C::KCH; ++i)
    *reinterpret_cast<u32x4*>(smem + C::K_OFF + (row0 + C::RPI * i) * C::RP + cb * 4) = vr[i];

  // softmax per query row: wave w takes rows RW w + lane / RL, each row
  // split over RL lanes (keys jl = lane % RL + RL k), so the reductions stay
  // inside RL-lane groups
  {
    constexpr int RW = NQ / NW, RL = 64 / RW;
    static_assert(RW * NW == NQ && LMAX % RL == 0, "softmax rows");
    const int i = RW * w + lane / RL, q = lane % RL;
    const int2 iv = query_interval(p, bl, i);
    float x[LMAX / RL];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < LMAX / RL; ++k) {
      const int jl = q + RL * k;
      x[k] = -INFINITY;
      if (jl < nk && in_interval(jbeg + jl, iv))
        x[k] = Sl[i * C::SLD + jl] * p.scale + Bl[i * C::BLD + jl + NQ - 1 - i] * p.scale_bd;
      m = fmaxf(m, x[k]);
    }
#pragma unroll
    for (int o = RL / 2; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, RL));
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < LMAX / RL; ++k) {
      x[k] = m == -INFINITY ? 0.f : __expf(x[k] - m);
      sum += x[k];
    }
#pragma unroll
    for (int o = RL / 2; o > 0; o >>= 1) sum += __shfl_xor(sum, o, RL);
    const float inv = sum > 0.f ? 1.f / sum : 0.f;  // a row that sees no key gives 0
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < LMAX / RL; ++k) Sl[i * C::SLD + q + RL * k] = x[k] * inv;
  }
  __syncthreads();

  // O = probs . V: wave w takes d_k tiles w, w + NW, ...; the B operand is
  // V[key 16kt + 4g + s][16dt + rl], one float per MFMA
  const float* Vl = reinterpret_cast<const float*>(smem + C::K_OFF);
  for (int dt = w; dt < DK / 16; dt += NW) {
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int kt = 0; kt < nkt; ++kt) {
      const floatx4 a = *reinterpret_cast<const floatx4*>(Sl + rl * C::SLD + kt * 16 + 4 * g);
      floatx4 bv;
#pragma unroll
      for (int e = 0; e < 4; ++e) bv[e] = Vl[(kt * 16 + 4 * g + e) * (C::RP / 4) + dt * 16 + rl];
      acc = mma16(a, bv, acc);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 4 * g + e;
      if (i < p.T) out[(int64_t)i * p.o_rs + dt * 16 + rl] = acc[e];
    }
  }
}

template <typename T, int DK, int NW, bool DEBUG>
hipError_t launch(const AttnParams& p, int nb, hipStream_t s) {
  using C = Cfg<T, DK, NW>;
  dim3 grid((p.T + C::QB - 1) / C::QB, p.H, nb);
  hipLaunchKernelGGL((attn_kernel<T, DK, NW, DEBUG>), grid, dim3(C::NT), 0, s, p);
  count_form(kFormGeneric);
  return hipGetLastError();
}

// Key split: 16 queries per workgroup, NW waves over its key tiles.
template <typename T, int DK, int NW>
hipError_t launch_ks(const AttnParams& p, int nb, hipStream_t s) {
  dim3 grid((p.T + 15) / 16, p.H, nb);
  hipLaunchKernelGGL((attn_kernel<T, DK, NW, false, true>), grid, dim3(64 * NW), 0, s, p);
  count_form(kFormKeySplit);
  return hipGetLastError();
}

template <typename T, int DK>
hipError_t dispatch_nw(const AttnParams& p, int nb, hipStream_t s) {
  const bool dbg = p.dbg_bd != nullptr;
  // fp32 inputs too short to give the CUs a workgroup each (one utterance of
  // 125 frames: 16 workgroups of 64 queries) split their keys over the waves
  // Short query blocks (the streaming chunk against more keys than the chunk
  // kernel stages) take the key-split form too: a one-wave form of this
  // kernel (16 queries, no split) gave wrong outputs whenever its per-key
  // mask ran, while the key-split form of the same source is exact on those
  // shapes, so there is no one-wave form.
  if constexpr (sizeof(T) == 4) {
    if (!dbg && (p.T <= 16 || (int64_t)nb * p.H * ((p.T + 63) / 64) < 128))
      return launch_ks<T, DK, 4>(p, nb, s);  // (per-wave tiles: 34 / 37 KB of LDS)
  }
  return dbg ? launch<T, DK, 4, true>(p, nb, s) : launch<T, DK, 4, false>(p, nb, s);
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

__global__ void mask_kernel(const AttnParams p, uint8_t* out) {
  const int bl = blockIdx.y;
  const int64_t n = (int64_t)p.T * p.L;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int i = (int)(e / p.L), j = (int)(e % p.L);
    out[bl * n + e] = in_interval(j, query_interval(p, bl, i)) ? 1 : 0;
  }
}

__global__ void pos_index_kernel(int T, int L, int qoff, int center, int32_t* out) {
  const int64_t n = (int64_t)T * L;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
    const int i = (int)(e / L), j = (int)(e % L);
    // the same expression the attention kernel stages its position band with:
    // row pmin + (band0 + n) for n = (j - j0) + 15 - (i - i0 - 16w)
    out[e] = center - (qoff + i) + j;
  }
}

}  // namespace

template <int NW>
int pos_pad_for(const AttnParams& p, int nb) {
  // (query block and key tile of a form do not depend on d_k)
  constexpr int QB = Cfg2<128, NW>::QB, NK = Cfg2<128, NW>::NK;
  int need = 0;
  const int nqb = (p.T + QB - 1) / QB;
  for (int bl = 0; bl < nb; ++bl)
    for (int qb = 0; qb < nqb; ++qb) {
      const int i0 = qb * QB;
      int jbeg, jend;
      key_range(p, bl, i0, imin(i0 + QB, p.T), jbeg, jend);
      const int jfirst = jbeg / NK * NK;
      if (jfirst >= jend) continue;
      // the kernel reads ring rows rr in [0, NK * tiles + QB + NK): position rows R0 + rr
      const int64_t R0 = (int64_t)p.center - p.qoff - (i0 + 31) + jfirst - 32 * (NW - 1);
      const int64_t hi = R0 + (int64_t)(jend - jfirst + NK - 1) / NK * NK + QB + NK;
      need = (int)std::max<int64_t>(need, std::max<int64_t>(-R0, hi - p.p_rows));
    }
  return need;
}

// (the larger of both forms' needs: the form is chosen at launch)
int bf16_pos_pad(const AttnParams& p, int nb) { return std::max(pos_pad_for<4>(p, nb), pos_pad_for<8>(p, nb)); }

namespace {
// attention()'s argument checks for nb > 0 and T > 0.
hipError_t check_attention(DType dt, int head_dim, const AttnParams& p, int nb) {
  if (nb > kMaxBatch || p.L <= 0 || p.H <= 0 || p.p_rows <= 0) return hipErrorInvalidValue;
  if (!p.q || !p.k || !p.v || !p.p || !p.o || !p.bias_u || !p.bias_v) return hipErrorInvalidValue;
  if (!aligned16(p.q) || !aligned16(p.k) || !aligned16(p.v) || !aligned16(p.p) || !aligned16(p.o))
    return hipErrorInvalidValue;
  const int epv = 16 / dtype_size(dt);
  if (p.q_rs % epv || p.q_bs % epv || p.kv_rs % epv || p.kv_bs % epv || p.p_rs % epv || p.o_rs % epv ||
      p.o_bs % epv)
    return hipErrorInvalidValue;
  if (p.ring_len < 0 || (p.ring_len && p.ring_head < 0)) return hipErrorInvalidValue;
  // The bf16 and chunk kernels address one item's K/V rows, the V^T block
  // of one head and the position table through buffer descriptors with
  // 32-bit byte ranges and offsets: keep every such range below 2^31 bytes.
  {
    const int64_t es = dtype_size(dt), lim = (int64_t)1 << 31;
    const int64_t krows = (p.ring_len ? p.ring_len : p.L) + (int64_t)p.kv_pad;
    if (krows * p.kv_rs * es >= lim || (int64_t)(p.p_rows + 2 * (int64_t)p.p_pad) * p.p_rs * es >= lim ||
        (int64_t)p.T * p.q_rs * es >= lim || (p.vt && (int64_t)head_dim * p.vt_ld * es >= lim))
      return hipErrorInvalidValue;
  }
  if (p.vt) {
    // V^T columns of each batch are read in whole 64-key tiles
    if (dt != kBF16 || p.ring_len || !aligned16(p.vt) || p.vt_ld % 8 || p.vt_bs % 64 || p.vt_bs < p.T ||
        p.vt_ld < (int64_t)(p.b0 + nb) * p.vt_bs || p.L != p.T || p.kv_pad < 63 || p.p_pad < bf16_pos_pad(p, nb) ||
        (head_dim != 64 && head_dim != 128))
      return hipErrorInvalidValue;
  }
  return hipSuccess;
}
}  // namespace

hipError_t attention(DType dt, int head_dim, const AttnParams& p, int nb, hipStream_t s) {
  if (nb <= 0 || p.T <= 0) return hipSuccess;
  if (hipError_t e = check_attention(dt, head_dim, p, nb)) return e;
  if (p.vt) return head_dim == 64 ? dispatch_bf16<64>(p, nb, s) : dispatch_bf16<128>(p, nb, s);
  if (dt == kF32) {
    if (p.T <= CfgS<128>::NQ && p.L <= CfgS<128>::LMAX && !p.dbg_bd) {
      const dim3 grid(p.H, nb);
      if (head_dim == 64) hipLaunchKernelGGL(attn_chunk_f32_kernel<64>, grid, dim3(CfgS<64>::NT), 0, s, p);
      else if (head_dim == 128) hipLaunchKernelGGL(attn_chunk_f32_kernel<128>, grid, dim3(CfgS<128>::NT), 0, s, p);
      else return hipErrorInvalidValue;
      count_form(kFormChunkF32);
      return hipGetLastError();
    }
    if (head_dim == 64) return dispatch_nw<float, 64>(p, nb, s);
    if (head_dim == 128) return dispatch_nw<float, 128>(p, nb, s);
  } else {
    if (head_dim == 64) return dispatch_nw<bf16, 64>(p, nb, s);
    if (head_dim == 128) return dispatch_nw<bf16, 128>(p, nb, s);
  }
  return hipErrorInvalidValue;
}

int64_t attention_form_count(int form) {
  return form >= 0 && form < kAttnForms ? g_form_launches[form].load(std::memory_order_relaxed) : -1;
}

hipError_t attention_with_gemm(DType dt, int head_dim, const AttnParams& p, int nb, const GemmParams& g, bool gquant,
                               hipStream_t s) {
  if (nb <= 0 || p.T <= 0 || g.M <= 0) return hipErrorNotSupported;
  if (dt != kBF16 || head_dim != 128 || !p.vt || p.dbg_bd || p.dbg_top || !use_wide<128>(p, nb) || windowed(p))
    return hipErrorNotSupported;
  if (check_attention(dt, head_dim, p, nb) != hipSuccess) return hipErrorNotSupported;
  TileForm tf;
  if (!gemm_tile_form(dt, gquant, g, tf) || tf.bm != 128 || tf.bn != 128 || tf.ns != 4) return hipErrorNotSupported;
  AttnParams a = p;
  FormSplit f;
  if ((int64_t)p.T * p.H * nb <= (1 << 28)) f = split_forms(a, nb);
  if (!f.nb4) {
    f.n8 = order_items<128, 8>(a, nb);
    if (f.n8 < 0) return hipErrorNotSupported;
  }
  const int64_t tiles = (m_tiles<128>(g) * (g.N / 128) + 7) / 8 * 8;
  if (f.n4 + f.n8 + tiles > (1 << 30)) return hipErrorNotSupported;
  if (gquant) launch_mixed<true, 128, 128, true, 4>(a, nb, f, g, tiles, s);
  else launch_mixed<true, 128, 128, false, 4>(a, nb, f, g, tiles, s);
  return hipGetLastError();
}

hipError_t export_mask(const AttnParams& p, int nb, uint8_t* out, hipStream_t s) {
  if (nb <= 0 || p.T <= 0 || p.L <= 0) return hipSuccess;
  if (nb > kMaxBatch || !out) return hipErrorInvalidValue;
  const int64_t n = (int64_t)p.T * p.L;
  dim3 grid((unsigned)std::min<int64_t>((n + 255) / 256, 4096), nb);
  hipLaunchKernelGGL(mask_kernel, grid, dim3(256), 0, s, p, out);
  return hipGetLastError();
}

hipError_t export_pos_index(int T, int L, int qoff, int center, int32_t* out, hipStream_t s) {
  if (T <= 0 || L <= 0) return hipSuccess;
  if (!out) return hipErrorInvalidValue;
  const int64_t n = (int64_t)T * L;
  hipLaunchKernelGGL(pos_index_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 4096)), dim3(256), 0, s,
                     T, L, qoff, center, out);
  return hipGetLastError();
}

}  // namespace mhsa
