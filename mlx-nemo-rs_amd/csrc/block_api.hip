// Host runtime of the rest of the Conformer block around the attention
// sublayer, on the same kernels: FeedForward (conformer.rs:2031-2088) and
// ConvolutionModule (conformer.rs:2105-2437).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <string>
#include <vector>

#include "host_common.hpp"
#include "kernels.hpp"
#include "sublayers.hpp"

using mhsa::DType;

// ---------------------------------------------------------------------------
// FeedForward (conformer.rs:2031-2088): linear2(silu(linear1(x))), each
// projection standard or MLX affine 8-bit, on the projection GEMMs with a
// SiLU epilogue; and the block's half-step sublayer x + 0.5 FF(LN(x))
// (conformer.rs:1703-1729, 1827-1851).
// ---------------------------------------------------------------------------

struct mhsa_ffn {
  int D = 0, F = 0;
  bool use_bias = false;
  DType dt = mhsa::kF32;
  HostLinear lin[2];  // linear1 [F, D], linear2 [D, F]
  bool dirty = true;
  DevBuf wbuf;
  DevLinear dev[2];
  DevLinear dev32[2];  // the same values in fp32 (for f32 activations)
  DevBuf act;      // [rows, F] silu(linear1(x))
  DevBuf hbuf;     // sublayer: LayerNorm output
  DevBuf ln_dev;
  std::vector<float> ln_host;
  DevBuf partial;  // split-K partials of small problems
  Profiler prof;
};

namespace {

int ffn_out(const mhsa_ffn* f, int i) { return i == 0 ? f->F : f->D; }
int ffn_in(const mhsa_ffn* f, int i) { return i == 0 ? f->D : f->F; }

int32_t prepare_ffn(mhsa_ffn* f) {
  if (!f->dirty) return MHSA_OK;
  const bool bf = f->dt == mhsa::kBF16;
  const size_t es = bf ? 2 : 4;
  auto rnd = [&](float v) { return bf ? round_bf16(v) : v; };
  size_t woff[2], sboff[2], boff[2], w32off[2], off = 0;
  for (int i = 0; i < 2; ++i) {
    const size_t n = (size_t)ffn_out(f, i) * ffn_in(f, i);
    woff[i] = off;
    off = align_up(off + (f->lin[i].quantized ? n : n * es), 256);
    sboff[i] = off;
    if (f->lin[i].quantized) off = align_up(off + (size_t)ffn_out(f, i) * (ffn_in(f, i) / 64) * 8, 256);
    boff[i] = off;
    off = align_up(off + (size_t)ffn_out(f, i) * 4, 256);
    w32off[i] = off;
    if (!f->lin[i].quantized && bf) off = align_up(off + n * 4, 256);
  }
  std::vector<char> host(off, 0);
  for (int i = 0; i < 2; ++i) {
    const HostLinear& h = f->lin[i];
    if (h.quantized) {
      std::memcpy(host.data() + woff[i], h.codes.data(), h.codes.size() * 4);
      float* sb = reinterpret_cast<float*>(host.data() + sboff[i]);
      for (size_t e = 0; e < h.qs.size(); ++e) {
        sb[2 * e] = rnd(h.qs[e]);
        sb[2 * e + 1] = rnd(h.qb[e]);
      }
    } else if (bf) {
      uint16_t* w = reinterpret_cast<uint16_t*>(host.data() + woff[i]);
      float* w32 = reinterpret_cast<float*>(host.data() + w32off[i]);
      for (size_t e = 0; e < h.w.size(); ++e) {
        w[e] = f32_to_bf16(h.w[e]);
        w32[e] = bf16_to_f32(w[e]);
      }
    } else {
      std::memcpy(host.data() + woff[i], h.w.data(), h.w.size() * 4);
    }
    float* b = reinterpret_cast<float*>(host.data() + boff[i]);
    for (size_t e = 0; e < h.bias.size(); ++e) b[e] = rnd(h.bias[e]);
  }
  if (f->wbuf.p) HIPCHK(hipDeviceSynchronize());  // earlier launches may still read the old values
  HIPCHK(f->wbuf.ensure(host.size()));
  HIPCHK(hipMemcpy(f->wbuf.p, host.data(), host.size(), hipMemcpyHostToDevice));
  const char* base = static_cast<const char*>(f->wbuf.p);
  for (int i = 0; i < 2; ++i) {
    f->dev[i].quantized = f->lin[i].quantized;
    f->dev[i].w = base + woff[i];
    f->dev[i].sb = f->lin[i].quantized ? reinterpret_cast<const float*>(base + sboff[i]) : nullptr;
    f->dev[i].bias = f->lin[i].bias.empty() ? nullptr : reinterpret_cast<const float*>(base + boff[i]);
    f->dev32[i] = f->dev[i];
    if (!f->lin[i].quantized && bf) f->dev32[i].w = base + w32off[i];
  }
  f->dirty = false;
  return MHSA_OK;
}

// Linear i of the FeedForward as a plain GEMM C[rows, out] = A[rows, in] W^T
// + b on activations of dtype `act` (prepare_ffn and the partial buffer
// come first).
mhsa::GemmParams ffn_gemm(mhsa_ffn* f, int i, DType act, const void* A, int rows, void* C) {
  const DevLinear& d = act == f->dt ? f->dev[i] : f->dev32[i];
  mhsa::GemmParams p;
  p.A = A;
  p.lda = ffn_in(f, i);
  p.W = d.w;
  p.sb = d.sb;
  p.bias = d.bias;
  p.C = C;
  p.ldc = ffn_out(f, i);
  p.M = rows;
  p.N = ffn_out(f, i);
  p.K = ffn_in(f, i);
  p.seg_rows = rows;
  p.ring_len = rows;
  p.partial = static_cast<float*>(f->partial.p);
  p.partial_elems = mhsa::kGemmPartialElems;
  return p;
}

// FeedForward on activations of dtype `act`: the module dtype, or f32 on the
// streaming path, where a bf16 module's ops meet f32 activations and MLX
// promotes them (its parameters keep their bf16 values).
int32_t ffn_impl(mhsa_ffn* f, const void* x, int rows, void* out, const void* residual, float res_scale, DType act,
                 hipStream_t s) {
  if (rows <= 0) return fail(MHSA_EINVAL, "rows must be positive (got %d)", rows);
  if (!x || !out) return fail(MHSA_EINVAL, "null tensor pointer");
  if (!aligned16(x) || !aligned16(out)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  int32_t rc = prepare_ffn(f);
  if (rc) return rc;
  const size_t es = mhsa::dtype_size(act);
  HIPCHK(f->act.ensure(align_up((int64_t)rows * f->F * es, 256)));
  HIPCHK(f->partial.ensure((size_t)mhsa::kGemmPartialElems * 4));
  for (int i = 0; i < 2; ++i) {
    mhsa::GemmParams p = ffn_gemm(f, i, act, i == 0 ? x : f->act.p, rows, i == 0 ? f->act.p : out);
    if (i == 0) p.act = mhsa::kActSilu;
    if (i == 1 && residual) {
      p.R = residual;
      p.ldr = f->D;
      p.res_scale = res_scale;
    }
    const char* tag = i == 0 ? "linear1" : "linear2";
    // (an in-place residual form is not repeated: each pass would add again)
    ProfScope ps(f->prof, tag, s, true, !(i == 1 && residual == out));
    for (int r = ps.reps(); r > 0; --r)
      HIPCHK(mhsa::gemm(act, f->lin[i].quantized, p, s));
  }
  return MHSA_OK;
}

int32_t ffn_sublayer(mhsa_ffn* f, void* x, int32_t rows, const float* gamma, const float* beta, float eps, DType act,
                     hipStream_t s) {
  if (!x || rows <= 0) return fail(MHSA_EINVAL, "bad sublayer arguments");
  if (!aligned16(x)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  if (f->D > mhsa::kMaxLayerNormDim)
    return fail(MHSA_ENOTSUP, "the sublayer's LayerNorm supports d_model <= %d (got %d)", mhsa::kMaxLayerNormDim, f->D);
  const int D = f->D;
  const float* gd = nullptr;
  const float* bd = nullptr;
  if (gamma || beta) {
    std::vector<float> tmp(2 * D);
    const bool bf = f->dt == mhsa::kBF16;
    for (int i = 0; i < D; ++i) {
      const float gv = gamma ? gamma[i] : 1.f, bv = beta ? beta[i] : 0.f;
      tmp[i] = bf ? round_bf16(gv) : gv;
      tmp[D + i] = bf ? round_bf16(bv) : bv;
    }
    if (tmp != f->ln_host) {
      if (f->ln_dev.p) HIPCHK(hipDeviceSynchronize());
      HIPCHK(f->ln_dev.ensure(tmp.size() * 4));
      HIPCHK(hipMemcpy(f->ln_dev.p, tmp.data(), tmp.size() * 4, hipMemcpyHostToDevice));
      f->ln_host = tmp;
    }
    gd = static_cast<const float*>(f->ln_dev.p);
    bd = gd + D;
  }
  HIPCHK(f->hbuf.ensure(align_up((int64_t)rows * D * mhsa::dtype_size(act), 256)));
  {
    ProfScope ps(f->prof, "layer_norm", s);
    for (int r = ps.reps(); r > 0; --r)
      HIPCHK(mhsa::layer_norm(act, x, f->hbuf.p, gd, bd, eps, rows, D, s));
  }
  // x + 0.5 * FF(LN(x)): the half step scales exactly (conformer.rs:1727-1729)
  return ffn_impl(f, f->hbuf.p, rows, x, x, 0.5f, act, s);
}

}  // namespace

extern "C" {

int32_t mhsa_ffn_create(int32_t d_model, int32_t ff_dim, int32_t use_bias, mhsa_ffn** out) {
  if (!out) return fail(MHSA_EINVAL, "null output pointer");
  *out = nullptr;
  if (d_model <= 0 || ff_dim <= 0 || d_model % 64 || ff_dim % 64)
    return fail(MHSA_EINVAL, "d_model %d and ff_dim %d must be positive multiples of 64", d_model, ff_dim);
  mhsa_ffn* f = new (std::nothrow) mhsa_ffn();
  if (!f) return fail(MHSA_ENOMEM, "out of host memory");
  f->D = d_model;
  f->F = ff_dim;
  f->use_bias = use_bias != 0;
  for (int i = 0; i < 2; ++i) {  // zero-initialised layers (conformer.rs:2046-2064)
    f->lin[i].w.assign((size_t)ffn_out(f, i) * ffn_in(f, i), 0.f);
    if (use_bias) f->lin[i].bias.assign(ffn_out(f, i), 0.f);
  }
  *out = f;
  return MHSA_OK;
}

void mhsa_ffn_destroy(mhsa_ffn* f) { delete f; }

int32_t mhsa_ffn_set_dtype(mhsa_ffn* f, int32_t dtype) {
  if (!f) return fail(MHSA_EINVAL, "null handle");
  if (dtype != MHSA_F32 && dtype != MHSA_BF16) return fail(MHSA_ENOTSUP, "dtype %d not supported (f32, bf16)", dtype);
  f->dt = dtype == MHSA_F32 ? mhsa::kF32 : mhsa::kBF16;
  f->dirty = true;
  return MHSA_OK;
}

int32_t mhsa_ffn_load_weights(mhsa_ffn* f, const mhsa_tensor* tensors, int32_t n, const char* prefix, int32_t strict,
                              int32_t quant_bits, int32_t quant_group) {
  if (!f) return fail(MHSA_EINVAL, "null handle");
  if ((n > 0 && !tensors) || !prefix) return fail(MHSA_EINVAL, "null tensor list or prefix");
  const TensorMap m{tensors, n};
  const int bits = quant_bits > 0 ? quant_bits : 8, group = quant_group > 0 ? quant_group : 64;
  const char* names[2] = {"linear1", "linear2"};
  HostLinear next[2] = {f->lin[0], f->lin[1]};
  for (int i = 0; i < 2; ++i) {  // FeedForward::load_weights via fetch_linear (conformer.rs:2074-2087)
    const std::string p = std::string(prefix) + "." + names[i];
    bool found = false;
    if (int32_t rc = load_linear(m, p, ffn_out(f, i), ffn_in(f, i), bits, group, next[i], &found)) return rc;
    if (!found && strict) return fail(MHSA_ENOENT, "missing weight `%s.weight`", p.c_str());
  }
  f->lin[0] = std::move(next[0]);
  f->lin[1] = std::move(next[1]);
  f->dirty = true;
  return MHSA_OK;
}

int32_t mhsa_ffn_forward(mhsa_ffn* f, const void* x, int32_t rows, void* out, void* hs) {
  if (!f) return fail(MHSA_EINVAL, "null handle");
  return ffn_impl(f, x, rows, out, nullptr, 1.f, f->dt, static_cast<hipStream_t>(hs));
}

int32_t mhsa_ffn_forward_f32(mhsa_ffn* f, const float* x, int32_t rows, float* out, void* hs) {
  if (!f) return fail(MHSA_EINVAL, "null handle");
  return ffn_impl(f, x, rows, out, nullptr, 1.f, mhsa::kF32, static_cast<hipStream_t>(hs));
}


int32_t mhsa_ffn_sublayer_forward(mhsa_ffn* f, void* x, int32_t rows, const float* gamma, const float* beta, float eps,
                                  void* hs) {
  if (!f) return fail(MHSA_EINVAL, "null handle");
  return ffn_sublayer(f, x, rows, gamma, beta, eps, f->dt, static_cast<hipStream_t>(hs));
}

int32_t mhsa_ffn_sublayer_forward_f32(mhsa_ffn* f, float* x, int32_t rows, const float* gamma, const float* beta,
                                      float eps, void* hs) {
  if (!f) return fail(MHSA_EINVAL, "null handle");
  return ffn_sublayer(f, x, rows, gamma, beta, eps, mhsa::kF32, static_cast<hipStream_t>(hs));
}

int32_t mhsa_ffn_profile_enable(mhsa_ffn* f, int32_t enable) {
  if (!f) return fail(MHSA_EINVAL, "null handle");
  return f->prof.enable(enable);
}
int32_t mhsa_ffn_profile_repeat(mhsa_ffn* f, const char* tag, int32_t n) {
  if (!f) return fail(MHSA_EINVAL, "null handle");
  return f->prof.set_repeat(tag, n);
}
int32_t mhsa_ffn_profile_reset(mhsa_ffn* f) {
  if (!f) return fail(MHSA_EINVAL, "null handle");
  return f->prof.reset();
}
int32_t mhsa_ffn_profile_count(mhsa_ffn* f) { return f ? f->prof.entries() : -1; }
int32_t mhsa_ffn_profile_entry(mhsa_ffn* f, int32_t idx, const char** name, double* total_ms, int32_t* launches) {
  if (!f) return fail(MHSA_EINVAL, "null handle");
  return f->prof.entry(idx, name, total_ms, launches);
}

int32_t mhsa_ffn_debug_linear(mhsa_ffn* f, int32_t which, int32_t f32_act, const void* x, int32_t rows, void* out,
                              void* hs) {
  if (!f) return fail(MHSA_EINVAL, "null handle");
  if (which < 0 || which > 1 || !x || !out || rows <= 0) return fail(MHSA_EINVAL, "bad arguments");
  if (!aligned16(x) || !aligned16(out)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  if (int32_t rc = prepare_ffn(f)) return rc;
  HIPCHK(f->partial.ensure((size_t)mhsa::kGemmPartialElems * 4));
  const DType act = f32_act ? mhsa::kF32 : f->dt;
  const mhsa::GemmParams p = ffn_gemm(f, which, act, x, rows, out);
  hipStream_t s = static_cast<hipStream_t>(hs);
  HIPCHK(mhsa::gemm(act, f->lin[which].quantized, p, s));
  HIPCHK(hipStreamSynchronize(s));
  return MHSA_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// ConvolutionModule (conformer.rs:2105-2437): pointwise_conv1 [2D, D] ->
// GLU -> padding frames zeroed -> depthwise conv (kernel K, causal or
// symmetric, streaming left context from the conv cache) -> BatchNorm or
// LayerNorm -> SiLU -> pointwise_conv2 [D, D]. The pointwise convs run on
// the projection GEMMs; the GLU, depthwise conv, BatchNorm and SiLU are one
// memory-bound kernel (LayerNorm, which needs whole rows, runs after it
// with SiLU fused).
//
// Dtypes follow MLX promotion as the reference writes the module: the
// causal left padding is an f32 zeros array (conformer.rs:2250-2256) and the
// streaming cache is f32 (streaming/core.rs:151), so the concatenation, and
// everything after it, is f32 even in a bf16 module; only a symmetric
// (non-causal) offline forward stays in the module dtype end to end. The
// parameters always hold their cast (dtype) values.
// ---------------------------------------------------------------------------

struct mhsa_conv {
  int D = 0, K = 0, norm = MHSA_CONV_BATCH_NORM;
  bool causal = false, use_bias = false;
  DType dt = mhsa::kF32;
  HostLinear lin[2];                // pointwise_conv1 [2D, D], pointwise_conv2 [D, D]
  std::vector<float> dw_w;          // depthwise weight [D, K] (MLX [D, K, 1])
  std::vector<float> dw_b;          // [D] or empty
  std::vector<float> nw, nb;        // norm weight / bias [D]
  std::vector<float> rmean, rvar;   // BatchNorm running statistics [D]
  bool dirty = true;
  DevBuf wbuf;
  DevLinear dev[2];    // weights in the module dtype
  DevLinear dev32[2];  // the same values in fp32 (for f32 activations)
  const float* taps = nullptr;      // [K, D]
  const float* taps_bias = nullptr; // [D] or null
  const float* norm_pack = nullptr; // BatchNorm [4, D] / LayerNorm [2, D]
  DevBuf gbuf;       // pointwise_conv1 output [rows, 2D]
  DevBuf ybuf;       // depthwise / norm / SiLU output [rows, D]
  DevBuf hbuf;       // sublayer LayerNorm output
  DevBuf cache_prev; // copy of a cache that several frame tiles read
  DevBuf ln_dev;
  std::vector<float> ln_host;
  DevBuf partial;
  Profiler prof;
};

namespace {

int conv_out(const mhsa_conv* m, int i) { return i == 0 ? 2 * m->D : m->D; }

int32_t prepare_conv(mhsa_conv* m) {
  if (!m->dirty) return MHSA_OK;
  const bool bf = m->dt == mhsa::kBF16;
  const int D = m->D, K = m->K;
  auto rnd = [&](float v) { return bf ? round_bf16(v) : v; };
  // layout: per linear {dtype weights | u32 codes, sb pairs, bias, fp32 weights}, taps, taps bias, norm pack
  size_t woff[2], sboff[2], boff[2], w32off[2], off = 0;
  for (int i = 0; i < 2; ++i) {
    const size_t n = (size_t)conv_out(m, i) * D;
    const bool q = m->lin[i].quantized;
    woff[i] = off;
    off = align_up(off + (q ? n : n * (bf ? 2 : 4)), 256);
    sboff[i] = off;
    if (q) off = align_up(off + (size_t)conv_out(m, i) * (D / 64) * 8, 256);
    boff[i] = off;
    off = align_up(off + (size_t)conv_out(m, i) * 4, 256);
    w32off[i] = off;
    if (!q && bf) off = align_up(off + n * 4, 256);
  }
  const size_t toff = off;
  off = align_up(off + (size_t)K * D * 4, 256);
  const size_t tboff = off;
  off = align_up(off + (size_t)D * 4, 256);
  const size_t noff = off;
  off = align_up(off + (size_t)4 * D * 4, 256);
  std::vector<char> host(off, 0);
  for (int i = 0; i < 2; ++i) {
    const HostLinear& h = m->lin[i];
    if (h.quantized) {
      std::memcpy(host.data() + woff[i], h.codes.data(), h.codes.size() * 4);
      float* sb = reinterpret_cast<float*>(host.data() + sboff[i]);
      for (size_t e = 0; e < h.qs.size(); ++e) {
        sb[2 * e] = rnd(h.qs[e]);
        sb[2 * e + 1] = rnd(h.qb[e]);
      }
    } else if (bf) {
      uint16_t* w = reinterpret_cast<uint16_t*>(host.data() + woff[i]);
      float* w32 = reinterpret_cast<float*>(host.data() + w32off[i]);
      for (size_t e = 0; e < h.w.size(); ++e) {
        w[e] = f32_to_bf16(h.w[e]);
        w32[e] = bf16_to_f32(w[e]);
      }
    } else {
      std::memcpy(host.data() + woff[i], h.w.data(), h.w.size() * 4);
    }
    float* b = reinterpret_cast<float*>(host.data() + boff[i]);
    for (size_t e = 0; e < h.bias.size(); ++e) b[e] = rnd(h.bias[e]);
  }
  float* taps = reinterpret_cast<float*>(host.data() + toff);
  for (int c = 0; c < D; ++c)
    for (int k = 0; k < K; ++k) taps[(size_t)k * D + c] = rnd(m->dw_w[(size_t)c * K + k]);
  float* tb = reinterpret_cast<float*>(host.data() + tboff);
  for (size_t c = 0; c < m->dw_b.size(); ++c) tb[c] = rnd(m->dw_b[c]);
  float* np = reinterpret_cast<float*>(host.data() + noff);
  if (m->norm == MHSA_CONV_BATCH_NORM) {
    // rsqrt(var + eps) is a parameter-only expression, evaluated in the
    // parameter dtype: eps is cast with the module (conformer.rs:2127-2130),
    // the sum and the rsqrt are stored in it.
    const float eps = rnd(1e-5f);
    for (int c = 0; c < D; ++c) {
      const float e = rnd(rnd(m->rvar[c]) + eps);
      np[c] = rnd(m->rmean[c]);
      np[D + c] = rnd((float)(1.0 / std::sqrt((double)e)));
      np[2 * D + c] = rnd(m->nw[c]);
      np[3 * D + c] = rnd(m->nb[c]);
    }
  } else {
    for (int c = 0; c < D; ++c) {
      np[c] = rnd(m->nw[c]);
      np[D + c] = rnd(m->nb[c]);
    }
  }
  if (m->wbuf.p) HIPCHK(hipDeviceSynchronize());  // earlier launches may still read the old values
  HIPCHK(m->wbuf.ensure(host.size()));
  HIPCHK(hipMemcpy(m->wbuf.p, host.data(), host.size(), hipMemcpyHostToDevice));
  const char* base = static_cast<const char*>(m->wbuf.p);
  for (int i = 0; i < 2; ++i) {
    DevLinear& d = m->dev[i];
    d.quantized = m->lin[i].quantized;
    d.w = base + woff[i];
    d.sb = d.quantized ? reinterpret_cast<const float*>(base + sboff[i]) : nullptr;
    d.bias = m->lin[i].bias.empty() ? nullptr : reinterpret_cast<const float*>(base + boff[i]);
    m->dev32[i] = d;
    if (!d.quantized && bf) m->dev32[i].w = base + w32off[i];
  }
  m->taps = reinterpret_cast<const float*>(base + toff);
  m->taps_bias = m->dw_b.empty() ? nullptr : reinterpret_cast<const float*>(base + tboff);
  m->norm_pack = reinterpret_cast<const float*>(base + noff);
  m->dirty = false;
  return MHSA_OK;
}

// One pointwise conv: C[rows, N] = A[rows, D] W^T + b (+ R) in `act` dtype.
int32_t conv_pointwise(mhsa_conv* m, int i, DType act, const void* A, int rows, void* C, const void* R,
                       hipStream_t s) {
  const DevLinear& d = act == m->dt ? m->dev[i] : m->dev32[i];
  mhsa::GemmParams p;
  p.A = A;
  p.lda = m->D;
  p.W = d.w;
  p.sb = d.sb;
  p.bias = d.bias;
  p.C = C;
  p.ldc = conv_out(m, i);
  p.M = rows;
  p.N = conv_out(m, i);
  p.K = m->D;
  p.seg_rows = rows;
  p.ring_len = rows;
  p.partial = static_cast<float*>(m->partial.p);
  p.partial_elems = mhsa::kGemmPartialElems;
  if (R) {
    p.R = R;
    p.ldr = m->D;
  }
  HIPCHK(mhsa::gemm(act, d.quantized, p, s));
  return MHSA_OK;
}

// The module's forward on activations of dtype `act` (the module dtype, or
// f32 on the streaming path). cache: [B, D, K-1] f32 device, updated in
// place, or null. Writes `out` [B, T, D] in conv_dtype(); with `residual`
// set, out = residual + module(x) (both in that dtype).
DType conv_dtype(const mhsa_conv* m, DType act, bool cache) { return cache || m->causal ? mhsa::kF32 : act; }

int32_t conv_impl(mhsa_conv* m, const void* x, int B, int T, DType act, const int32_t* lens, float* cache, void* out,
                  const void* residual, hipStream_t s) {
  if (B <= 0 || T <= 0) return fail(MHSA_EINVAL, "batch and seq_len must be positive (got %d, %d)", B, T);
  if (!x || !out) return fail(MHSA_EINVAL, "null tensor pointer");
  if (!aligned16(x) || !aligned16(out) || (cache && !aligned16(cache)))
    return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  if (cache && !m->causal)
    // a symmetric conv over [cache; x] yields T + K - 1 frames, which the
    // block's residual add rejects (conformer.rs:2364-2366, 1941)
    return fail(MHSA_EINVAL, "a conv cache needs a causal module");
  if (int32_t rc = prepare_conv(m)) return rc;
  const int D = m->D, K = m->K, C = K - 1;
  const int64_t rows = (int64_t)B * T;
  if (rows > INT32_MAX / 2) return fail(MHSA_EINVAL, "batch * seq_len too large");
  const DType cdt = conv_dtype(m, act, cache != nullptr);
  HIPCHK(m->gbuf.ensure(align_up(rows * 2 * D * mhsa::dtype_size(act), 256)));
  HIPCHK(m->ybuf.ensure(align_up(rows * D * mhsa::dtype_size(cdt), 256)));
  HIPCHK(m->partial.ensure((size_t)mhsa::kGemmPartialElems * 4));
  {
    ProfScope ps(m->prof, "pointwise_conv1", s);
    for (int r = ps.reps(); r > 0; --r)
      if (int32_t rc = conv_pointwise(m, 0, act, x, (int)rows, m->gbuf.p, nullptr, s)) return rc;
  }
  // several frame tiles of one item would read the cache while the last one
  // rewrites it: read a copy then
  const float* cache_in = cache;
  if (cache && C > 0 && T > mhsa::conv_frame_tile()) {
    const size_t bytes = (size_t)B * D * C * 4;
    HIPCHK(m->cache_prev.ensure(bytes));
    HIPCHK(hipMemcpyAsync(m->cache_prev.p, cache, bytes, hipMemcpyDeviceToDevice, s));
    cache_in = static_cast<const float*>(m->cache_prev.p);
  }
  // (a cache updated in place is not repeated: each pass would advance it)
  ProfScope ps(m->prof, "conv", s, true, !cache);
  for (int b0 = 0; b0 < B; b0 += mhsa::kMaxBatch) {
    const int nb = std::min(mhsa::kMaxBatch, B - b0);
    mhsa::ConvParams p;
    p.g = static_cast<const char*>(m->gbuf.p) + (size_t)b0 * T * 2 * D * mhsa::dtype_size(act);
    p.y = static_cast<char*>(m->ybuf.p) + (size_t)b0 * T * D * mhsa::dtype_size(cdt);
    if (cache && C > 0) {
      p.cache_in = cache_in + (size_t)b0 * D * C;
      p.cache_out = cache + (size_t)b0 * D * C;
    }
    p.w = m->taps;
    p.bias = m->taps_bias;
    p.bn = m->norm == MHSA_CONV_BATCH_NORM ? m->norm_pack : nullptr;
    p.T = T;
    p.D = D;
    p.K = K;
    p.left = m->causal ? C : C / 2;
    for (int b = 0; b < nb; ++b) p.len[b] = lens ? std::max(0, std::min(lens[b0 + b], T)) : T;
    for (int r = ps.reps(); r > 0; --r) HIPCHK(mhsa::conv_glu_depthwise(act, cdt, p, nb, s));
  }
  if (m->norm == MHSA_CONV_LAYER_NORM) {  // nn::LayerNorm (eps 1e-5) then SiLU, in place
    ps.next("layer_norm", false);  // in place
    HIPCHK(mhsa::layer_norm(cdt, m->ybuf.p, m->ybuf.p, m->norm_pack, m->norm_pack + D, 1e-5f, (int)rows, D, s,
                            mhsa::kActSilu));
  }
  // (an in-place residual form is not repeated: each pass would add again)
  ps.next("pointwise_conv2", residual != out);
  for (int r = ps.reps(); r > 0; --r)
    if (int32_t rc = conv_pointwise(m, 1, cdt, m->ybuf.p, (int)rows, out, residual, s)) return rc;
  return MHSA_OK;
}

int32_t check_conv(const mhsa_conv* m) { return m ? MHSA_OK : fail(MHSA_EINVAL, "null conv handle"); }

// conv_norm's affine parameters on the device (null when neither is given),
// rounded like the reference's cast of the norm to the module dtype and
// uploaded when they change.
int32_t conv_sublayer_norm(mhsa_conv* m, const float* gamma, const float* beta, const float** gd, const float** bd) {
  const int D = m->D;
  *gd = *bd = nullptr;
  if (!gamma && !beta) return MHSA_OK;
  std::vector<float> tmp(2 * D);
  const bool bf = m->dt == mhsa::kBF16;
  for (int i = 0; i < D; ++i) {
    const float gv = gamma ? gamma[i] : 1.f, bv = beta ? beta[i] : 0.f;
    tmp[i] = bf ? round_bf16(gv) : gv;
    tmp[D + i] = bf ? round_bf16(bv) : bv;
  }
  if (tmp != m->ln_host) {
    if (m->ln_dev.p) HIPCHK(hipDeviceSynchronize());  // earlier LayerNorm launches may still read them
    HIPCHK(m->ln_dev.ensure(tmp.size() * 4));
    HIPCHK(hipMemcpy(m->ln_dev.p, tmp.data(), tmp.size() * 4, hipMemcpyHostToDevice));
    m->ln_host = tmp;
  }
  *gd = static_cast<const float*>(m->ln_dev.p);
  *bd = *gd + D;
  return MHSA_OK;
}

}  // namespace

int32_t mhsa_conv_sublayer_to_f32(mhsa_conv* m, const void* x, DType x_dt, int B, int T, const int32_t* lens,
                                  const float* gamma, const float* beta, float eps, float* out, hipStream_t s) {
  if (int32_t rc = check_conv(m)) return rc;
  if (!x || !out || B <= 0 || T <= 0) return fail(MHSA_EINVAL, "bad sublayer arguments");
  if (!aligned16(x) || !aligned16(out)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  if (m->D > mhsa::kMaxLayerNormDim)
    return fail(MHSA_ENOTSUP, "the sublayer's LayerNorm supports d_model <= %d (got %d)", mhsa::kMaxLayerNormDim, m->D);
  if (x_dt != mhsa::kF32 && !(x_dt == m->dt && m->causal))
    return fail(MHSA_EINVAL, "only f32 activations, or a causal module's own-dtype ones, give an f32 sublayer");
  if (x_dt != mhsa::kF32 && x == out) return fail(MHSA_EINVAL, "the f32 output cannot overwrite bf16 input");
  const float* gd;
  const float* bd;
  if (int32_t rc = conv_sublayer_norm(m, gamma, beta, &gd, &bd)) return rc;
  const int D = m->D;
  const int64_t rows = (int64_t)B * T;
  HIPCHK(m->hbuf.ensure(align_up(rows * D * mhsa::dtype_size(x_dt), 256)));
  // conv_norm in the activations' dtype (conformer.rs:1793); the residual x
  // (conformer.rs:1814) then goes to out in f32, where the module adds to it
  HIPCHK(mhsa::layer_norm(x_dt, x, m->hbuf.p, gd, bd, eps, (int)rows, D, s));
  if (x_dt != mhsa::kF32) HIPCHK(mhsa::widen_bf16(x, out, rows * D, s));
  else if (x != out) HIPCHK(hipMemcpyAsync(out, x, (size_t)rows * D * 4, hipMemcpyDeviceToDevice, s));
  return conv_impl(m, m->hbuf.p, B, T, x_dt, lens, nullptr, out, out, s);
}

extern "C" {

int32_t mhsa_conv_create(int32_t d_model, int32_t kernel_size, int32_t norm_type, int32_t causal, int32_t use_bias,
                         mhsa_conv** out) {
  if (!out) return fail(MHSA_EINVAL, "null output pointer");
  *out = nullptr;
  if (d_model <= 0 || d_model % 64) return fail(MHSA_EINVAL, "d_model %d must be a positive multiple of 64", d_model);
  if (kernel_size < 1 || kernel_size > mhsa::kMaxConvKernel)
    return fail(MHSA_EINVAL, "kernel_size %d out of range [1, %d]", kernel_size, mhsa::kMaxConvKernel);
  // padding (K - 1) / 2 each side keeps T frames only for odd K (conformer.rs:2145-2152)
  if (!causal && kernel_size % 2 == 0)
    return fail(MHSA_EINVAL, "a symmetric (non-causal) conv needs an odd kernel_size (got %d)", kernel_size);
  if (norm_type != MHSA_CONV_BATCH_NORM && norm_type != MHSA_CONV_LAYER_NORM)
    return fail(MHSA_ENOTSUP, "conv norm type %d (only batch_norm and layer_norm are supported)", norm_type);
  if (norm_type == MHSA_CONV_LAYER_NORM && d_model > mhsa::kMaxLayerNormDim)
    return fail(MHSA_ENOTSUP, "the conv LayerNorm supports d_model <= %d (got %d)", mhsa::kMaxLayerNormDim, d_model);
  mhsa_conv* m = new (std::nothrow) mhsa_conv();
  if (!m) return fail(MHSA_ENOMEM, "out of host memory");
  m->D = d_model;
  m->K = kernel_size;
  m->norm = norm_type;
  m->causal = causal != 0;
  m->use_bias = use_bias != 0;
  // zero-initialised pointwise layers with zero biases (conformer.rs:2168-2172),
  // a zero depthwise kernel, and the norm's identity initialisation
  for (int i = 0; i < 2; ++i) {
    m->lin[i].w.assign((size_t)conv_out(m, i) * d_model, 0.f);
    m->lin[i].bias.assign(conv_out(m, i), 0.f);
  }
  m->dw_w.assign((size_t)d_model * kernel_size, 0.f);
  if (use_bias) m->dw_b.assign(d_model, 0.f);
  m->nw.assign(d_model, 1.f);
  m->nb.assign(d_model, 0.f);
  m->rmean.assign(d_model, 0.f);
  m->rvar.assign(d_model, 1.f);
  *out = m;
  return MHSA_OK;
}

void mhsa_conv_destroy(mhsa_conv* m) { delete m; }

int32_t mhsa_conv_set_dtype(mhsa_conv* m, int32_t dtype) {
  if (int32_t rc = check_conv(m)) return rc;
  if (dtype != MHSA_F32 && dtype != MHSA_BF16) return fail(MHSA_ENOTSUP, "dtype %d not supported (f32, bf16)", dtype);
  m->dt = dtype == MHSA_F32 ? mhsa::kF32 : mhsa::kBF16;
  m->dirty = true;
  return MHSA_OK;
}

int32_t mhsa_conv_cache_size(const mhsa_conv* m) { return m ? m->K - 1 : -1; }

int32_t mhsa_conv_profile_enable(mhsa_conv* m, int32_t enable) {
  if (int32_t rc = check_conv(m)) return rc;
  return m->prof.enable(enable);
}

int32_t mhsa_conv_profile_repeat(mhsa_conv* m, const char* tag, int32_t n) {
  if (int32_t rc = check_conv(m)) return rc;
  return m->prof.set_repeat(tag, n);
}

int32_t mhsa_conv_profile_reset(mhsa_conv* m) {
  if (int32_t rc = check_conv(m)) return rc;
  return m->prof.reset();
}

int32_t mhsa_conv_profile_count(mhsa_conv* m) { return m ? m->prof.entries() : -1; }

int32_t mhsa_conv_profile_entry(mhsa_conv* m, int32_t idx, const char** name, double* total_ms, int32_t* launches) {
  if (int32_t rc = check_conv(m)) return rc;
  return m->prof.entry(idx, name, total_ms, launches);
}

int32_t mhsa_conv_output_dtype(const mhsa_conv* m) {
  if (!m) return -1;
  return conv_dtype(m, m->dt, false) == mhsa::kF32 ? MHSA_F32 : MHSA_BF16;
}

int32_t mhsa_conv_debug_linear(mhsa_conv* m, int32_t which, int32_t f32_act, const void* x, int32_t rows, void* out,
                               void* hs) {
  if (int32_t rc = check_conv(m)) return rc;
  if (which < 0 || which > 1 || !x || !out || rows <= 0) return fail(MHSA_EINVAL, "bad arguments");
  if (!aligned16(x) || !aligned16(out)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  if (int32_t rc = prepare_conv(m)) return rc;
  HIPCHK(m->partial.ensure((size_t)mhsa::kGemmPartialElems * 4));
  hipStream_t s = static_cast<hipStream_t>(hs);
  if (int32_t rc = conv_pointwise(m, which, f32_act ? mhsa::kF32 : m->dt, x, rows, out, nullptr, s)) return rc;
  HIPCHK(hipStreamSynchronize(s));
  return MHSA_OK;
}

int32_t mhsa_conv_load_weights(mhsa_conv* m, const mhsa_tensor* tensors, int32_t n, const char* prefix, int32_t strict,
                               int32_t quant_bits, int32_t quant_group) {
  if (int32_t rc = check_conv(m)) return rc;
  if ((n > 0 && !tensors) || !prefix) return fail(MHSA_EINVAL, "null tensor list or prefix");
  const TensorMap tm{tensors, n};
  const int D = m->D, K = m->K;
  const int bits = quant_bits > 0 ? quant_bits : 8, group = quant_group > 0 ? quant_group : 64;
  const std::string pre(prefix);
  // everything is validated into copies first, so a failed load changes nothing
  HostLinear lin[2] = {m->lin[0], m->lin[1]};
  const char* lnames[2] = {"pointwise_conv1", "pointwise_conv2"};
  for (int i = 0; i < 2; ++i) {  // fetch_linear (conformer.rs:2396-2410)
    bool found = false;
    const std::string p = pre + "." + lnames[i];
    if (int32_t rc = load_linear(tm, p, conv_out(m, i), D, bits, group, lin[i], &found)) return rc;
    if (!found && strict) return fail(MHSA_ENOENT, "missing weight `%s.weight`", p.c_str());
  }
  // a float [D] vector at `key`, needed when strict (load_optional_param, loading.rs:192-200)
  auto vec = [&](const std::string& key, std::vector<float>& dst) -> int32_t {
    const mhsa_tensor* t = tm.find(key);
    if (!t) return strict ? fail(MHSA_ENOENT, "missing weight `%s`", key.c_str()) : MHSA_OK;
    if (!float_dtype(t->dtype) || numel(t) != D) return fail(MHSA_EINVAL, "`%s`: expected float [%d]", key.c_str(), D);
    dst.resize(D);
    for (int e = 0; e < D; ++e) dst[e] = load_host(t->dtype, t->data, e);
    return MHSA_OK;
  };
  // depthwise conv: weight in MLX layout [D, K, 1] (loading.rs:216-224); its
  // bias only when the module has one
  std::vector<float> dw_w = m->dw_w, dw_b = m->dw_b;
  const std::string dwp = pre + ".depthwise_conv";
  if (const mhsa_tensor* w = tm.find(dwp + ".weight")) {
    if (!float_dtype(w->dtype) || w->ndim != 3 || w->shape[0] != D || w->shape[1] != K || w->shape[2] != 1)
      return fail(MHSA_EINVAL, "`%s.weight`: expected float [%d, %d, 1]", dwp.c_str(), D, K);
    for (size_t e = 0; e < dw_w.size(); ++e) dw_w[e] = load_host(w->dtype, w->data, e);
  } else if (strict) {
    return fail(MHSA_ENOENT, "missing weight `%s.weight`", dwp.c_str());
  }
  if (m->use_bias)
    if (int32_t rc = vec(dwp + ".bias", dw_b)) return rc;
  // the norm's parameters sit under `batch_norm` for either type (conformer.rs:2419-2426)
  std::vector<float> nw = m->nw, nb = m->nb, rmean = m->rmean, rvar = m->rvar;
  const std::string np = pre + ".batch_norm";
  if (int32_t rc = vec(np + ".weight", nw)) return rc;
  if (int32_t rc = vec(np + ".bias", nb)) return rc;
  if (m->norm == MHSA_CONV_BATCH_NORM) {  // load_batch_norm (loading.rs:236-254)
    if (int32_t rc = vec(np + ".running_mean", rmean)) return rc;
    if (int32_t rc = vec(np + ".running_var", rvar)) return rc;
  }
  m->lin[0] = std::move(lin[0]);
  m->lin[1] = std::move(lin[1]);
  m->dw_w = std::move(dw_w);
  m->dw_b = std::move(dw_b);
  m->nw = std::move(nw);
  m->nb = std::move(nb);
  m->rmean = std::move(rmean);
  m->rvar = std::move(rvar);
  m->dirty = true;
  return MHSA_OK;
}

int32_t mhsa_conv_forward(mhsa_conv* m, const void* x, int32_t batch, int32_t seq_len, const int32_t* lengths,
                          void* out, void* hs) {
  if (int32_t rc = check_conv(m)) return rc;
  return conv_impl(m, x, batch, seq_len, m->dt, lengths, nullptr, out, nullptr, static_cast<hipStream_t>(hs));
}

int32_t mhsa_conv_forward_with_cache(mhsa_conv* m, const float* x, int32_t batch, int32_t seq_len, float* cache,
                                     const int32_t* lengths, float* out, void* hs) {
  if (int32_t rc = check_conv(m)) return rc;
  return conv_impl(m, x, batch, seq_len, mhsa::kF32, lengths, cache, out, nullptr, static_cast<hipStream_t>(hs));
}

int32_t mhsa_conv_sublayer_forward(mhsa_conv* m, void* x, int32_t batch, int32_t seq_len, float* cache,
                                   const int32_t* lengths, const float* gamma, const float* beta, float eps,
                                   void* hs) {
  if (int32_t rc = check_conv(m)) return rc;
  if (!x || batch <= 0 || seq_len <= 0) return fail(MHSA_EINVAL, "bad sublayer arguments");
  if (!aligned16(x)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  if (m->D > mhsa::kMaxLayerNormDim)
    return fail(MHSA_ENOTSUP, "the sublayer's LayerNorm supports d_model <= %d (got %d)", mhsa::kMaxLayerNormDim, m->D);
  // streaming activations are f32; offline ones are in the module dtype
  const DType act = cache ? mhsa::kF32 : m->dt;
  if (conv_dtype(m, act, cache != nullptr) != act)
    return fail(MHSA_ENOTSUP, "the causal bf16 module's output is f32 (MLX promotion), which the bf16 input "
                              "cannot hold in place: call mhsa_conv_forward and add the residual in f32");
  hipStream_t s = static_cast<hipStream_t>(hs);
  const int D = m->D;
  const float* gd;
  const float* bd;
  if (int32_t rc = conv_sublayer_norm(m, gamma, beta, &gd, &bd)) return rc;
  const int64_t rows = (int64_t)batch * seq_len;
  HIPCHK(m->hbuf.ensure(align_up(rows * D * mhsa::dtype_size(act), 256)));
  // conv_norm (conformer.rs:1793, 1939), then x + conv(.) (conformer.rs:1814, 1941)
  HIPCHK(mhsa::layer_norm(act, x, m->hbuf.p, gd, bd, eps, (int)rows, D, s));
  return conv_impl(m, m->hbuf.p, batch, seq_len, act, lengths, cache, x, x, s);
}

}  // extern "C"
