// CPU restatement of the reference rel-pos MHSA forward, fp32 + OpenMP.
//
// TEST INFRASTRUCTURE ONLY: the timed CPU baseline (bench.py's cpu_baseline
// leg) and a cross-check of the numpy oracle (tests/). The product never links
// or calls it.
//
// It follows the reference's op sequence as written
// (src/asr/modules/encoders/attention.rs:458-573), including its overcompute:
//   q, k, v = x W^T + b                         (478-480, quantization.rs:126-136)
//   p = linear_pos(pos_emb) over all 2T-1 rows  (493-499)
//   query blocks of query_block_size rows       (196-206, 517-519)
//   bd = (q + v_bias) P_slice^T over T+rows-1 columns, then rel_shift as
//        pad-left + reshape + drop-row + reshape, truncated to T (529-532, 832-855)
//   softmax(s (q + u_bias) k^T + cast(s) bd + mask) v over all T keys (299-318)
//   out = context W_out^T + b                   (558-565)
// The bf16 configurations are run on bf16-rounded inputs in fp32.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include <omp.h>

namespace {

// y[M, N] = x[M, K] w[N, K]^T (+ bias), cache-blocked dot products.
void linear(const float* x, const float* w, const float* bias, float* y, int M, int N, int K) {
  constexpr int MB = 16, NB = 64;
#pragma omp parallel for collapse(2) schedule(static)
  for (int m0 = 0; m0 < M; m0 += MB) {
    for (int n0 = 0; n0 < N; n0 += NB) {
      const int m1 = std::min(M, m0 + MB), n1 = std::min(N, n0 + NB);
      for (int m = m0; m < m1; ++m) {
        const float* xr = x + (int64_t)m * K;
        for (int n = n0; n < n1; ++n) {
          const float* wr = w + (int64_t)n * K;
          float acc = 0.f;
#pragma omp simd reduction(+ : acc)
          for (int k = 0; k < K; ++k) acc += xr[k] * wr[k];
          y[(int64_t)m * N + n] = acc + (bias ? bias[n] : 0.f);
        }
      }
    }
  }
}

int query_block_size(int64_t batch_heads, int seq_len, int64_t max_score) {
  const int64_t per_row = std::max<int64_t>(batch_heads * 2 * seq_len, 1);
  return (int)std::min<int64_t>(std::max<int64_t>(max_score / per_row, 1), std::max(seq_len, 1));
}

bool ctx_visible(int has, int left, int right, int chunked, int i, int j) {
  if (!has) return true;
  if (chunked && right >= 0) {
    const int chunk = right + 1;
    const int lc = left >= 0 ? left / chunk : 10000;
    const int d = i / chunk - j / chunk;
    return d >= 0 && d <= lc;
  }
  bool v = left < 0 || j - i >= -left;
  if (!chunked && right >= 0) v = v && j - i <= right;
  return v;
}

}  // namespace

extern "C" {

int cpu_mhsa_threads(void) { return omp_get_max_threads(); }

// All pointers are host fp32, row-major. lengths may be null (no padding);
// has_ctx = 0 means full attention. scale_bd is the scale applied to the
// position scores (1/sqrt(d_k) in fp32, its bf16 rounding in bf16 mode).
int cpu_mhsa_forward(int B, int T, int D, int H, const float* x, const float* pos_emb, const float* wq,
                     const float* bq, const float* wk, const float* bk, const float* wv, const float* bv,
                     const float* wo, const float* bo, const float* wpos, const float* pbu, const float* pbv,
                     int has_ctx, int left, int right, int chunked, const int* lengths, float scale_bd, float* out) {
  if (B <= 0 || T <= 0 || H <= 0 || D % H) return 22;
  const int dk = D / H, P = 2 * T - 1;
  const int64_t M = (int64_t)B * T;
  std::vector<float> q(M * D), k(M * D), v(M * D), p((int64_t)P * D), ctx(M * D);
  linear(x, wq, bq, q.data(), (int)M, D, D);
  linear(x, wk, bk, k.data(), (int)M, D, D);
  linear(x, wv, bv, v.data(), (int)M, D, D);
  linear(pos_emb, wpos, nullptr, p.data(), P, D, D);
  const float scale = 1.0f / std::sqrt((float)dk);
  const int block = query_block_size((int64_t)B * H, T, (int64_t)1 << 26);
  for (int s = 0; s < T; s += block) {
    const int e = std::min(T, s + block), rows = e - s, cols = T + rows - 1;
    const int c0 = T - e;  // first P row of the block's slice (attention.rs:529)
#pragma omp parallel
    {
      std::vector<float> bd((int64_t)rows * cols), padded((int64_t)rows * (cols + 1)), sc(T);
#pragma omp for collapse(2) schedule(static)
      for (int b = 0; b < B; ++b) {
        for (int h = 0; h < H; ++h) {
          // matrix_bd for the whole block (rows x cols)
          for (int r = 0; r < rows; ++r) {
            const float* qr = q.data() + ((int64_t)b * T + s + r) * D + h * dk;
            for (int c = 0; c < cols; ++c) {
              const float* pr = p.data() + (int64_t)(c0 + c) * D + h * dk;
              float acc = 0.f;
              for (int d = 0; d < dk; ++d) acc += (qr[d] + pbv[h * dk + d]) * pr[d];
              bd[(int64_t)r * cols + c] = acc;
            }
          }
          // rel_shift: pad one zero column on the left, view [cols+1, rows],
          // drop the first row, view back [rows, cols]
          for (int r = 0; r < rows; ++r) {
            padded[(int64_t)r * (cols + 1)] = 0.f;
            std::memcpy(&padded[(int64_t)r * (cols + 1) + 1], &bd[(int64_t)r * cols], sizeof(float) * cols);
          }
          const float* shifted = padded.data() + rows;
          for (int r = 0; r < rows; ++r) {
            const int i = s + r;
            const float* qr = q.data() + ((int64_t)b * T + i) * D + h * dk;
            const int len = lengths ? std::max(lengths[b], 1) : T;
            float mx = -INFINITY;
            for (int j = 0; j < T; ++j) {
              const float* kr = k.data() + ((int64_t)b * T + j) * D + h * dk;
              float acc = 0.f;
              for (int d = 0; d < dk; ++d) acc += (qr[d] + pbu[h * dk + d]) * kr[d];
              const bool vis = j < len && ctx_visible(has_ctx, left, right, chunked, i, j);
              sc[j] = vis ? scale * acc + scale_bd * shifted[(int64_t)r * cols + j] : -INFINITY;
              mx = std::max(mx, sc[j]);
            }
            float sum = 0.f;
            for (int j = 0; j < T; ++j) {
              sc[j] = mx == -INFINITY ? 0.f : std::exp(sc[j] - mx);
              sum += sc[j];
            }
            float* cr = ctx.data() + ((int64_t)b * T + i) * D + h * dk;
            for (int d = 0; d < dk; ++d) cr[d] = 0.f;
            for (int j = 0; j < T; ++j) {
              if (sc[j] == 0.f) continue;
              const float wj = sc[j] / sum;
              const float* vr = v.data() + ((int64_t)b * T + j) * D + h * dk;
              for (int d = 0; d < dk; ++d) cr[d] += wj * vr[d];
            }
          }
        }
      }
    }
  }
  linear(ctx.data(), wo, bo, out, (int)M, D, D);
  return 0;
}

}  // extern "C"
