// Host runtime of the rel-pos MHSA library: the C ABI declared in
// include/relpos_mhsa.h, mirroring RelPositionMultiHeadAttention
// (attention.rs:328-893), LinearLayer (quantization.rs:36-162) and the
// encoder's streaming cache bookkeeping (conformer.rs:840-1047).
//
// A layer handle keeps fp32 master copies of its parameters and uploads them
// on first use after a change into kernel-native device layouts for its
// dtype: q/k/v rows stacked as one [3D, D] operand (one fused GEMM when all
// three have the same kind), dense weights in the compute dtype, affine u8
// codes as stored plus {scale, bias} float pairs, biases pre-rounded to the
// compute dtype.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/relpos_mhsa.h"
#include "host_common.hpp"
#include "kernels.hpp"
#include "sublayers.hpp"

using mhsa::DType;

namespace {

thread_local std::string g_err;


}  // namespace

int32_t mhsa::set_error(int32_t code, const char* msg) {
  g_err = msg ? msg : "";
  return code;
}

struct mhsa_layer {
  int D = 0, H = 0, dk = 0;
  bool use_bias = false;
  DType dt = mhsa::kF32;
  int cache_drop = 0;
  HostLinear lin[5];
  std::vector<float> pbu, pbv;
  bool dirty = true;
  // bumped by every upload of the parameters: streams compare it with the
  // version their cached K/V were projected with
  uint64_t version = 0;
  // device parameters
  DevBuf wbuf;
  DevLinear dev[5];
  bool qkv_fused = false;
  const float* d_pbu = nullptr;
  const float* d_pbv = nullptr;
  // scratch
  DevBuf ws;
  DevBuf gemm_partial;         // K-split partial sums of small GEMMs
  float* partial_override = nullptr;  // set for the duration of an allocation-free call
  DevBuf vtbuf;                // bf16: transposed V [D][B * Tpad]
  DevBuf hbuf;                 // sublayer: LayerNorm output
  const char* last_qkv = nullptr;  // where the last offline forward put [q|k|v] rows
  const char* last_pos = nullptr;  // and its projected position rows (debug export)
  DevBuf ln_dev;               // sublayer: LayerNorm gamma, beta
  std::vector<float> ln_host;  // values currently in ln_dev
  // Parameters the fp32 streaming kernels read (see prepare_stream): an
  // fp32 layer's own, or a bf16 layer's promoted to fp32
  DevLinear sdev[5];
  DevBuf wbuf32;               // bf16 layer: fp32 copies of its bf16 dense weights
  uint64_t stream_version = 0; // layer version sdev was built for
  // streaming position memo (attention.rs:749-761), fp32
  DevBuf pmemo;
  DevBuf pmemo_bf16;           // bf16 layer: the projection before widening
  int pmemo_len = -1;
  DevBuf uws;                  // workspace of the no-cache path
  Profiler prof;
};

namespace {
// ProfScope over a layer's profiler.
struct LayerProf : ProfScope {
  LayerProf(mhsa_layer* L, const char* tag, hipStream_t s_, bool enabled = true, bool repeatable = true)
      : ProfScope(L->prof, tag, s_, enabled, repeatable) {}
};
}  // namespace

struct mhsa_stream {
  mhsa_layer* layer = nullptr;
  int B = 0, C = 0, Tc = 0, R = 0;
  int head = 0;
  uint64_t kv_version = 0;  // layer version ring_kv was projected with (0 = never)
  std::vector<int32_t> fill;
  DevBuf ring_h;   // [B, R, D] fp32
  DevBuf ring_kv;  // [B, R, 2D] fp32 (K columns then V columns)
  DevBuf ws;
};

namespace {

DType dtype_of(const mhsa_layer* L) { return L->dt; }
size_t esz(const mhsa_layer* L) { return (size_t)mhsa::dtype_size(L->dt); }

// Upload the parameters in the layer's dtype (no-op when clean).
int32_t prepare(mhsa_layer* L) {
  if (!L->dirty) return MHSA_OK;
  const int D = L->D;
  const bool bf = L->dt == mhsa::kBF16;
  const size_t es = esz(L);
  auto rnd = [&](float v) { return bf ? round_bf16(v) : v; };
  const bool q0 = L->lin[0].quantized;
  L->qkv_fused = L->lin[1].quantized == q0 && L->lin[2].quantized == q0;

  // Layout: [qkv weights][out][pos] then sb blocks, biases, pos biases.
  const size_t dense_b = (size_t)D * D * es, codes_b = (size_t)D * D, sb_b = (size_t)D * (D / 64) * 2 * 4;
  std::vector<size_t> woff(5), sboff(5), boff(5);
  size_t off = 0;
  for (int i = 0; i < 5; ++i) {
    woff[i] = off;
    off += L->lin[i].quantized ? codes_b : dense_b;
  }
  for (int i = 0; i < 5; ++i) {
    off = align_up(off, 256);
    sboff[i] = off;
    if (L->lin[i].quantized) off += sb_b;
  }
  off = align_up(off, 256);
  const size_t bias_all = off;  // [3D] q/k/v bias block then out, pos
  for (int i = 0; i < 5; ++i) boff[i] = bias_all + (size_t)i * D * 4;
  off = bias_all + (size_t)5 * D * 4;
  off = align_up(off, 256);
  const size_t pb_off = off;
  off += (size_t)2 * D * 4;
  std::vector<char> host(off, 0);

  bool any_qkv_bias = false;
  for (int i = 0; i < 5; ++i) {
    const HostLinear& h = L->lin[i];
    if (h.quantized) {
      std::memcpy(host.data() + woff[i], h.codes.data(), codes_b);
      float* sb = reinterpret_cast<float*>(host.data() + sboff[i]);
      for (size_t e = 0; e < h.qs.size(); ++e) {
        sb[2 * e] = rnd(h.qs[e]);
        sb[2 * e + 1] = rnd(h.qb[e]);
      }
    } else if (bf) {
      uint16_t* w = reinterpret_cast<uint16_t*>(host.data() + woff[i]);
      for (size_t e = 0; e < h.w.size(); ++e) w[e] = f32_to_bf16(h.w[e]);
    } else {
      std::memcpy(host.data() + woff[i], h.w.data(), dense_b);
    }
    float* b = reinterpret_cast<float*>(host.data() + boff[i]);
    for (size_t e = 0; e < h.bias.size(); ++e) b[e] = rnd(h.bias[e]);
    if (i < 3 && !h.bias.empty()) any_qkv_bias = true;
  }
  float* pb = reinterpret_cast<float*>(host.data() + pb_off);
  for (int e = 0; e < D; ++e) {
    pb[e] = rnd(L->pbu[e]);
    pb[D + e] = rnd(L->pbv[e]);
  }
  // kernels of an earlier call (on any stream) may still read the old
  // parameters: let them finish before the buffer is reused or replaced
  if (L->wbuf.p) HIPCHK(hipDeviceSynchronize());
  HIPCHK(L->wbuf.ensure(host.size()));
  HIPCHK(hipMemcpy(L->wbuf.p, host.data(), host.size(), hipMemcpyHostToDevice));
  char* base = static_cast<char*>(L->wbuf.p);
  for (int i = 0; i < 5; ++i) {
    DevLinear& d = L->dev[i];
    d.quantized = L->lin[i].quantized;
    d.w = base + woff[i];
    d.sb = d.quantized ? reinterpret_cast<const float*>(base + sboff[i]) : nullptr;
    const bool has = !L->lin[i].bias.empty() || (i < 3 && L->qkv_fused && any_qkv_bias);
    d.bias = has ? reinterpret_cast<const float*>(base + boff[i]) : nullptr;
  }
  // With fused q/k/v the three operands must be contiguous rows of one
  // matrix: true for dense (woff stride D*D*es) and for codes (stride D*D).
  L->d_pbu = reinterpret_cast<const float*>(base + pb_off);
  L->d_pbv = L->d_pbu + D;
  L->dirty = false;
  L->pmemo_len = -1;
  ++L->version;
  return MHSA_OK;
}

// Transposed output of the V projection for the bf16 attention kernel.
struct VtOut {
  void* p = nullptr;
  int64_t ld = 0;  // row stride (elements) = B * Tpad
  int col0 = 0;    // first GEMM output column that belongs to V
  int T = 0, Tpad = 0;
};

// GEMM parameters of y = A W^T (+ bias) (+ R) for one of the layer's linears.
int32_t make_gemm(mhsa_layer* L, const DevLinear& lin, int n_rows_w, const void* A, int64_t lda, int M, void* C,
                  int64_t ldc, const void* R, int64_t ldr, mhsa::GemmParams& p, int seg_rows = 0, int seg_stride = 0,
                  int ring_off = 0, int ring_len = 0, const VtOut* vt = nullptr) {
  p = mhsa::GemmParams();
  p.A = A;
  p.lda = lda;
  p.W = lin.w;
  p.sb = lin.sb;
  p.bias = lin.bias;
  p.R = R;
  p.ldr = ldr;
  p.C = C;
  p.ldc = ldc;
  p.M = M;
  p.N = n_rows_w;
  p.K = L->D;
  p.seg_rows = seg_rows > 0 ? seg_rows : std::max(M, 1);
  p.seg_stride = seg_rows > 0 ? seg_stride : 0;
  p.ring_off = ring_off;
  p.ring_len = ring_len > 0 ? ring_len : std::max(M, 1);
  if (L->partial_override) {
    p.partial = L->partial_override;
  } else {
    HIPCHK(L->gemm_partial.ensure((size_t)mhsa::kGemmPartialElems * sizeof(float)));
    p.partial = static_cast<float*>(L->gemm_partial.p);
  }
  p.partial_elems = mhsa::kGemmPartialElems;
  if (vt) {
    p.vt = vt->p;
    p.vt_ld = vt->ld;
    p.vt_col0 = vt->col0;
    p.vt_Tpad = vt->Tpad;
    p.seg_T = vt->T;  // per-utterance M tiles
  }
  return MHSA_OK;
}

int32_t run_gemm(mhsa_layer* L, DType dt, const DevLinear& lin, int n_rows_w, const void* A, int64_t lda, int M,
                 void* C, int64_t ldc, const void* R, int64_t ldr, hipStream_t s, int seg_rows = 0,
                 int seg_stride = 0, int ring_off = 0, int ring_len = 0, const VtOut* vt = nullptr) {
  mhsa::GemmParams p;
  if (int32_t rc = make_gemm(L, lin, n_rows_w, A, lda, M, C, ldc, R, ldr, p, seg_rows, seg_stride, ring_off, ring_len,
                             vt))
    return rc;
  HIPCHK(mhsa::gemm(dt, lin.quantized, p, s));
  return MHSA_OK;
}

// q, k, v (and optionally only k, v) projections of `A` [M, D].
// With `vt`, V goes to the transposed buffer instead of columns [2D, 3D).
int32_t project_qkv(mhsa_layer* L, const void* A, int M, void* out, int64_t ldo, hipStream_t s,
                    const VtOut* vt = nullptr) {
  const size_t es = esz(L);
  if (L->qkv_fused) {
    VtOut v;
    if (vt) {
      v = *vt;
      v.col0 = 2 * L->D;
    }
    return run_gemm(L, L->dt, L->dev[0], 3 * L->D, A, L->D, M, out, ldo, nullptr, 0, s, 0, 0, 0, 0,
                    vt ? &v : nullptr);
  }
  for (int i = 0; i < 3; ++i) {
    VtOut v;
    if (vt && i == 2) {
      v = *vt;
      v.col0 = 0;
    }
    int32_t rc = run_gemm(L, L->dt, L->dev[i], L->D, A, L->D, M, static_cast<char*>(out) + (size_t)i * L->D * es, ldo,
                          nullptr, 0, s, 0, 0, 0, 0, (vt && i == 2) ? &v : nullptr);
    if (rc) return rc;
  }
  return MHSA_OK;
}

struct DistRange {
  int dmin, dmax;  // query-minus-key frame distances a visible pair can have
};

DistRange context_distances(const mhsa_context* ctx, int qoff, int T, int L) {
  // distances d = (qoff + i) - j over 0 <= i < T, 0 <= j < L
  DistRange r{qoff - (L - 1), qoff + T - 1};
  if (!ctx || (ctx->left < 0 && ctx->right < 0)) return r;
  if (ctx->chunked && ctx->right >= 0) {
    const int chunk = ctx->right + 1;
    const long lc = ctx->left >= 0 ? ctx->left / chunk : 10000;
    r.dmin = std::max(r.dmin, -(chunk - 1));
    r.dmax = (int)std::min<long>(r.dmax, (lc + 1) * chunk - 1);
  } else {
    if (ctx->left >= 0) r.dmax = std::min(r.dmax, ctx->left);
    if (!ctx->chunked && ctx->right >= 0) r.dmin = std::max(r.dmin, -ctx->right);
  }
  return r;
}

// Resolve the position table: full (2L-1 rows, centre L-1) or a centred band
// the context never reaches beyond. Returns the first table row to project,
// the row count, and the centre inside the projected rows.
int32_t plan_positions(int pos_len, int L, const DistRange& dr, int& row0, int& nrows, int& center) {
  if (pos_len <= 0 || pos_len % 2 == 0)
    return fail(MHSA_EINVAL, "pos_emb must have an odd number of rows (2*len-1 or a centred band), got %d", pos_len);
  if (dr.dmax < dr.dmin) {  // nothing visible: project a single row
    row0 = 0;
    nrows = 1;
    center = 0;
    return MHSA_OK;
  }
  const int c = (pos_len - 1) / 2;
  if (pos_len > 2 * L - 1)
    return fail(MHSA_EINVAL, "pos_emb has %d rows; expected %d (2*len-1) or fewer", pos_len, 2 * L - 1);
  if (pos_len < 2 * L - 1 && std::max(dr.dmax, -dr.dmin) > c)
    return fail(MHSA_EINVAL,
                "pos_emb band of %d rows covers distances +-%d but the attention context reaches %d..%d", pos_len,
                c, dr.dmin, dr.dmax);
  const int lo = std::max(dr.dmin, -c), hi = std::min(dr.dmax, c);
  row0 = c - hi;
  nrows = hi - lo + 1;
  center = hi;
  return MHSA_OK;
}

float scale_f32(int dk) { return 1.0f / std::sqrt((float)dk); }

void fill_attn_common(const mhsa_layer* L, mhsa::AttnParams& a) {
  a.H = L->H;
  a.scale = scale_f32(L->dk);
  a.scale_bd = L->dt == mhsa::kBF16 ? round_bf16(a.scale) : a.scale;  // attention.rs:308-311
  a.bias_u = L->d_pbu;
  a.bias_v = L->d_pbv;
}

void set_ctx(mhsa::AttnParams& a, const mhsa_context* ctx) {
  a.has_ctx = ctx && (ctx->left >= 0 || ctx->right >= 0);
  a.left = ctx ? ctx->left : -1;
  a.right = ctx ? ctx->right : -1;
  a.chunked = ctx ? ctx->chunked != 0 : 0;
}

// Launch attention in batch chunks of kMaxBatch; `per_batch` fills the
// per-item key range / valid rows.
template <typename Fn>
int32_t run_attention(const mhsa_layer* L, DType dt, mhsa::AttnParams a, int B, Fn per_batch, hipStream_t s) {
  for (int b0 = 0; b0 < B; b0 += mhsa::kMaxBatch) {
    const int nb = std::min(mhsa::kMaxBatch, B - b0);
    a.b0 = b0;
    for (int i = 0; i < nb; ++i) per_batch(b0 + i, a.key_lo[i], a.key_hi[i], a.q_valid[i]);
    HIPCHK(mhsa::attention(dt, L->dk, a, nb, s));
  }
  return MHSA_OK;
}

int32_t check_layer(const mhsa_layer* L) {
  if (!L) return fail(MHSA_EINVAL, "null layer handle");
  return MHSA_OK;
}


// Offline forward shared by mhsa_forward, the sublayer and the debug export.
// Debug outputs of the attention kernel (all null in the product path).
struct AttnDebug {
  float* bd = nullptr;     // scaled position scores [B, H, T, T]
  int* top = nullptr;      // bf16 kernel: top visible key per query row [B, H, T]
  float* topv = nullptr;   // and its logit
  bool any() const { return bd || top; }
};

// Fixed device memory an allocation-free call works in: [workspace | V^T]
// carved from `base`, `cap` bytes (the GEMMs' split-K partials are given
// separately through the layer's partial_override).
struct Arena {
  char* base = nullptr;
  size_t cap = 0;
};

// Key range and valid rows of item b of an offline call (attention.rs:281-285).
void offline_key_bounds(const int32_t* lens, int T, int b, int& lo, int& hi, int& qv) {
  lo = 0;
  hi = lens ? std::min(std::max(lens[b], 1), T) : T;
  qv = T;
}

// What an offline forward derives before its launches: the position rows it
// projects and where its workspace puts [q|k|v], the position rows, the
// attention output and (bf16) V^T.
struct OfflineLayout {
  int row0 = 0, nrows = 0, center = 0, pad = 0, kv_pad = 0;
  int64_t M = 0;
  bool use_vt = false;
  char* qkv = nullptr;
  char* P = nullptr;   // table rows [0, nrows) after `pad` slack rows
  char* cx = nullptr;
  VtOut vt;
};

int32_t offline_layout(mhsa_layer* L, int B, int T, int pos_len, const mhsa_context* ctx, const int32_t* lens,
                       hipStream_t s, const Arena* arena, OfflineLayout& o) {
  const int D = L->D;
  const size_t es = esz(L);
  const DistRange dr = context_distances(ctx, 0, T, T);
  int32_t rc;
  if ((rc = plan_positions(pos_len, T, dr, o.row0, o.nrows, o.center))) return rc;
  o.M = (int64_t)B * T;
  o.use_vt = L->dt == mhsa::kBF16;
  // bf16: position rows the kernel may read on either side of the table
  // (they only meet masked pairs) and key rows past the last item, kept as
  // finite slack in the workspace
  o.pad = 0;
  o.kv_pad = o.use_vt ? 64 : 0;
  if (o.use_vt) {
    mhsa::AttnParams a;
    fill_attn_common(L, a);
    a.T = T;
    a.L = T;
    a.qoff = 0;
    a.p_rows = o.nrows;
    a.center = o.center;
    set_ctx(a, ctx);
    for (int b0 = 0; b0 < B; b0 += mhsa::kMaxBatch) {
      const int nb = std::min(mhsa::kMaxBatch, B - b0);
      for (int i = 0; i < nb; ++i) offline_key_bounds(lens, T, b0 + i, a.key_lo[i], a.key_hi[i], a.q_valid[i]);
      o.pad = std::max(o.pad, mhsa::bf16_pos_pad(a, nb));
    }
  }
  o.pad = (int)align_up(o.pad, 8);
  const int64_t prow_n = o.nrows + 2 * (int64_t)o.pad;
  const size_t qkv_b = align_up((o.M + o.kv_pad) * 3 * D * es, 256), p_b = align_up(prow_n * D * es, 256),
               ctx_b = align_up(o.M * D * es, 256);
  // bf16: V also transposed per batch, [D][B * Tpad], for the MFMA PV operand.
  // The QKV GEMM writes every column the attention kernel reads (whole tiles
  // of tokens: projections of the next utterance's rows, or of zero rows past
  // the last one), so it needs no clearing.
  size_t vt_b = 0;
  if (o.use_vt) {
    o.vt.T = T;
    o.vt.Tpad = (int)align_up(T, 256);  // whole GEMM tiles of tokens per utterance
    o.vt.ld = (int64_t)B * o.vt.Tpad;
    vt_b = align_up((int64_t)D * o.vt.ld * 2, 256);
  }
  if (arena) {
    if (qkv_b + p_b + ctx_b + vt_b > arena->cap)
      return fail(MHSA_EINVAL, "batch %d x seq_len %d needs %zu bytes of workspace; the allocation-free forward "
                  "has %zu", B, T, qkv_b + p_b + ctx_b + vt_b, arena->cap);
    o.qkv = arena->base;
    if (o.use_vt) o.vt.p = arena->base + qkv_b + p_b + ctx_b;
    // the slack rows the bf16 kernel may read (key rows past the last item,
    // position rows around the table) hold the previous call's values: clear them
    if (o.kv_pad) HIPCHK(mhsa::fill_zero(o.qkv + (size_t)o.M * 3 * D * es, (size_t)o.kv_pad * 3 * D * es, s));
    if (o.pad) {
      HIPCHK(mhsa::fill_zero(o.qkv + qkv_b, (size_t)o.pad * D * es, s));
      HIPCHK(mhsa::fill_zero(o.qkv + qkv_b + (size_t)(o.pad + o.nrows) * D * es, (size_t)o.pad * D * es, s));
    }
  } else {
    const size_t ws_before = L->ws.n;
    HIPCHK(L->ws.ensure(qkv_b + p_b + ctx_b));
    if (L->ws.n != ws_before) HIPCHK(mhsa::fill_zero(L->ws.p, L->ws.n, s));  // slack rows start finite
    o.qkv = static_cast<char*>(L->ws.p);
    if (o.use_vt) {
      const size_t before = L->vtbuf.n;
      HIPCHK(L->vtbuf.ensure(vt_b));
      if (L->vtbuf.n != before) HIPCHK(mhsa::fill_zero(L->vtbuf.p, L->vtbuf.n, s));
      o.vt.p = L->vtbuf.p;
    }
  }
  o.P = o.qkv + qkv_b + (size_t)o.pad * D * es;
  o.cx = o.qkv + qkv_b + p_b;
  return MHSA_OK;
}

// The position projection P = pos_emb[row0 : row0 + nrows] W_pos^T of a layout.
int32_t pos_gemm(mhsa_layer* L, const OfflineLayout& o, const void* pos_emb, mhsa::GemmParams& g) {
  return make_gemm(L, L->dev[4], L->D, static_cast<const char*>(pos_emb) + (size_t)o.row0 * L->D * esz(L), L->D,
                   o.nrows, o.P, L->D, nullptr, 0, g);
}

// A projection to launch together with this call's attention (the next
// stacked layer's position rows), or none.
struct FusedNext {
  mhsa::GemmParams g;
  bool quant = false;
  DType dt = mhsa::kBF16;
};

// With `pos_ready` the layout's position rows are already projected. With
// `next`, that projection runs in the attention's launch where a fused form
// exists, else right after it.
int32_t forward_impl(mhsa_layer* L, const void* x, int B, int T, const void* pos_emb, int pos_len,
                     const mhsa_context* ctx, const int32_t* lens, void* out, const void* residual,
                     const AttnDebug& dbg, hipStream_t s, const Arena* arena = nullptr,
                     const OfflineLayout* ready = nullptr, const FusedNext* next = nullptr) {
  if (B <= 0 || T <= 0) return fail(MHSA_EINVAL, "batch and seq_len must be positive (got %d, %d)", B, T);
  if (!x || !pos_emb || (!out && !dbg.any())) return fail(MHSA_EINVAL, "null tensor pointer");
  if (!aligned16(x) || !aligned16(pos_emb) || (out && !aligned16(out)))
    return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  int32_t rc;
  if (arena) {
    if (L->dirty)
      return fail(MHSA_EINVAL, "the layer's parameters changed since their last upload, and uploading allocates: "
                               "run mhsa_forward once after loading weights or changing the dtype");
  } else if ((rc = prepare(L))) {
    return rc;
  }
  const bool prof = !arena;  // (event pairs are created on first use)
  const int D = L->D;
  const size_t es = esz(L);
  OfflineLayout o;
  if (ready) o = *ready;
  else if ((rc = offline_layout(L, B, T, pos_len, ctx, lens, s, arena, o))) return rc;
  L->last_qkv = o.qkv;
  L->last_pos = o.P;

  // The Q/K/V and position projections in one launch where both take tile
  // forms that pair (the position tiles take the CUs the Q/K/V tiles free as
  // they end), else one after the other.
  mhsa::GemmParams gq, gp;
  bool paired = false;
  if (!ready && L->qkv_fused && L->dev[0].quantized == L->dev[4].quantized) {
    VtOut v;
    if (o.use_vt) {
      v = o.vt;
      v.col0 = 2 * D;
    }
    if ((rc = make_gemm(L, L->dev[0], 3 * D, x, D, (int)o.M, o.qkv, 3 * D, nullptr, 0, gq, 0, 0, 0, 0,
                        o.use_vt ? &v : nullptr)) ||
        (rc = pos_gemm(L, o, pos_emb, gp)))
      return rc;
    paired = mhsa::gemm_pair_ok(L->dt, L->dev[0].quantized, gq, gp);
  }
  if (paired) {
    LayerProf ps(L, "gemm_qkv_pos", s, prof);
    for (int r = ps.reps(); r > 0; --r)
      HIPCHK(mhsa::gemm_pair(L->dt, L->dev[0].quantized, gq, gp, s));
  } else {
    {
      LayerProf ps(L, "gemm_qkv", s, prof);
      for (int r = ps.reps(); r > 0; --r)
        if ((rc = project_qkv(L, x, (int)o.M, o.qkv, 3 * D, s, o.use_vt ? &o.vt : nullptr))) return rc;
    }
    if (!ready) {
      LayerProf ps(L, "gemm_pos", s, prof);
      mhsa::GemmParams g;
      if ((rc = pos_gemm(L, o, pos_emb, g))) return rc;
      for (int r = ps.reps(); r > 0; --r)
        HIPCHK(mhsa::gemm(L->dt, L->dev[4].quantized, g, s));
    }
  }

  mhsa::AttnParams a;
  fill_attn_common(L, a);
  a.T = T;
  a.L = T;
  a.qoff = 0;
  a.p_rows = o.nrows;
  a.center = o.center;
  set_ctx(a, ctx);
  a.q = o.qkv;
  a.k = o.qkv + (size_t)D * es;
  a.v = o.qkv + (size_t)2 * D * es;
  a.q_bs = a.kv_bs = (int64_t)T * 3 * D;
  a.q_rs = a.kv_rs = 3 * D;
  a.p = o.P;
  a.p_rs = D;
  a.p_pad = o.pad;
  a.kv_pad = o.kv_pad;
  a.o = o.cx;
  a.o_bs = (int64_t)T * D;
  a.o_rs = D;
  a.dbg_bd = dbg.bd;
  a.dbg_top = dbg.top;
  a.dbg_topv = dbg.topv;
  if (o.use_vt) {
    a.vt = o.vt.p;
    a.vt_ld = o.vt.ld;
    a.vt_bs = o.vt.Tpad;
  }
  auto key_bounds = [&](int b, int& lo, int& hi, int& qv) { offline_key_bounds(lens, T, b, lo, hi, qv); };
  {
    LayerProf ps(L, "attention", s, prof);
    for (int r = ps.reps(); r > 0 && !rc; --r) {
      bool fused = false;
      if (next && B <= mhsa::kMaxBatch) {
        mhsa::AttnParams af = a;
        af.b0 = 0;
        for (int i = 0; i < B; ++i) key_bounds(i, af.key_lo[i], af.key_hi[i], af.q_valid[i]);
        const hipError_t e = mhsa::attention_with_gemm(L->dt, L->dk, af, B, next->g, next->quant, s);
        if (e != hipErrorNotSupported) {
          HIPCHK(e);
          fused = true;
        }
      }
      if (!fused) {
        rc = run_attention(L, L->dt, a, B, key_bounds, s);
        if (!rc && next) HIPCHK(mhsa::gemm(next->dt, next->quant, next->g, s));
      }
    }
  }
  if (rc) return rc;
  if (!out) return MHSA_OK;
  // (an in-place residual form is not repeated: each pass would add again)
  LayerProf ps(L, "gemm_out", s, prof, residual != out);
  for (int r = ps.reps(); r > 0 && !rc; --r)
    rc = run_gemm(L, L->dt, L->dev[3], D, o.cx, D, (int)o.M, out, D, residual, D, s);
  return rc;
}

// ---- allocation-free forward ---------------------------------------------
// mhsa_forward_noalloc works in this array: the GEMMs' split-K partials
// (kGemmPartialElems floats, as the allocating path uses, so both paths make
// the same kernel choices and give the same bits) followed by the offline
// workspace ([q|k|v] rows, position rows, attention output, bf16 V^T).
// Each GPU the library runs on holds its own copy until the process ends.
constexpr size_t kNoAllocScratchBytes = (size_t)128 << 20;
constexpr size_t kNoAllocPartialBytes = (size_t)mhsa::kGemmPartialElems * sizeof(float);
static_assert(kNoAllocPartialBytes % 256 == 0 && kNoAllocPartialBytes < kNoAllocScratchBytes, "scratch split");
}  // namespace

static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {
// Device address of `scratch` per device: host code never uses the array's
// name as an address (on the host it is only a stand-in for the symbol).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_dev[kMaxDevices] = {};

int32_t scratch_for_current_device(char** out) {
  int dev = -1;
  HIPCHK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail(MHSA_EINVAL, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    HIPCHK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(MHSA_EHIP, "hipGetSymbolAddress returned a null address");
    g_scratch_dev[dev] = static_cast<char*>(p);
  }
  *out = g_scratch_dev[dev];
  return MHSA_OK;
}

// K and V of every ring row from the cached inputs h (the reference
// re-projects [cache; x] on every step, attention.rs:721-722): run when the
// stream's projections are older than the layer's parameters, i.e. on the
// first step of a new stream (h = 0 gives K = b_k, V = b_v) and after any
// weight or dtype change.
int32_t reproject_ring(mhsa_layer* L, mhsa_stream* S, hipStream_t s) {
  const int D = L->D, M = S->B * S->R;
  char* kv = static_cast<char*>(S->ring_kv.p);
  int32_t rc;
  if (L->qkv_fused) {
    rc = run_gemm(L, mhsa::kF32, L->sdev[1], 2 * D, S->ring_h.p, D, M, kv, 2 * D, nullptr, 0, s);
  } else {
    rc = run_gemm(L, mhsa::kF32, L->sdev[1], D, S->ring_h.p, D, M, kv, 2 * D, nullptr, 0, s);
    if (!rc)
      rc = run_gemm(L, mhsa::kF32, L->sdev[2], D, S->ring_h.p, D, M, kv + (size_t)D * 4, 2 * D, nullptr, 0, s);
  }
  if (rc) return rc;
  S->kv_version = L->version;
  return MHSA_OK;
}

// The streaming path computes in fp32 for both layer dtypes. The reference
// keeps the streaming caches in f32 (conformer.rs:422-434) and never casts
// the streamed features to the layer dtype (conformer.rs:845-849), so in a
// bf16 model [cache; x] and every activation derived from it are f32: MLX
// promotes the bf16 parameters to f32 in each op, and a quantized
// projection dequantises in f32 from its bf16-cast scales and biases. Only
// the position rows are computed in bf16 (a bf16 table through bf16 weights,
// attention.rs:749-761). So for a bf16 layer the fp32 kernels read: dense
// weights as fp32 copies of their bf16 values, quantized ones as uploaded
// (codes + bf16-rounded scale/bias pairs, dequantised in fp32 by the GEMM),
// biases and pos biases as uploaded (bf16-rounded floats).
int32_t prepare_stream(mhsa_layer* L) {
  int32_t rc = prepare(L);
  if (rc) return rc;
  if (L->stream_version == L->version) return MHSA_OK;
  for (int i = 0; i < 5; ++i) L->sdev[i] = L->dev[i];
  if (L->dt == mhsa::kBF16) {
    const size_t n = (size_t)L->D * L->D;
    std::vector<float> host(5 * n, 0.f);
    bool any_dense = false;
    for (int i = 0; i < 5; ++i)
      if (!L->lin[i].quantized) {
        any_dense = true;
        for (size_t e = 0; e < n; ++e) host[i * n + e] = round_bf16(L->lin[i].w[e]);
      }
    if (any_dense) {
      if (L->wbuf32.p) HIPCHK(hipDeviceSynchronize());  // an earlier step may still read them
      HIPCHK(L->wbuf32.ensure(host.size() * 4));
      HIPCHK(hipMemcpy(L->wbuf32.p, host.data(), host.size() * 4, hipMemcpyHostToDevice));
      for (int i = 0; i < 5; ++i)
        if (!L->lin[i].quantized) L->sdev[i].w = static_cast<const float*>(L->wbuf32.p) + i * n;
    }
  }
  L->stream_version = L->version;
  return MHSA_OK;
}

// The sublayer's LayerNorm: its affine parameters on the device, uploaded
// when they change (rounded like the reference's cast of the norm to the
// layer dtype), and the output buffer for `rows` rows.
int32_t sublayer_norm(mhsa_layer* L, const float* gamma, const float* beta, int64_t rows, const float** gd,
                      const float** bd) {
  const int D = L->D;
  if (D > mhsa::kMaxLayerNormDim)
    return fail(MHSA_ENOTSUP, "the sublayer's LayerNorm supports d_model <= %d (got %d)", mhsa::kMaxLayerNormDim, D);
  *gd = *bd = nullptr;
  if (gamma || beta) {
    std::vector<float> tmp(2 * D);
    const bool bf = L->dt == mhsa::kBF16;
    for (int i = 0; i < D; ++i) {
      const float gv = gamma ? gamma[i] : 1.f, bv = beta ? beta[i] : 0.f;
      tmp[i] = bf ? round_bf16(gv) : gv;
      tmp[D + i] = bf ? round_bf16(bv) : bv;
    }
    if (tmp != L->ln_host) {
      if (L->ln_dev.p) HIPCHK(hipDeviceSynchronize());  // earlier LayerNorm launches may still read them
      HIPCHK(L->ln_dev.ensure(tmp.size() * 4));
      HIPCHK(hipMemcpy(L->ln_dev.p, tmp.data(), tmp.size() * 4, hipMemcpyHostToDevice));
      L->ln_host = tmp;
    }
    *gd = static_cast<const float*>(L->ln_dev.p);
    *bd = *gd + D;
  }
  HIPCHK(L->hbuf.ensure(align_up(rows * D * esz(L), 256)));
  return MHSA_OK;
}

}  // namespace

extern "C" {

const char* mhsa_last_error(void) { return g_err.c_str(); }
int32_t mhsa_version(void) { return 100; }

int32_t mhsa_create(int32_t d_model, int32_t n_heads, int32_t use_bias, mhsa_layer** out) {
  if (!out) return fail(MHSA_EINVAL, "null output pointer");
  *out = nullptr;
  if (d_model <= 0 || n_heads <= 0 || d_model % n_heads)
    return fail(MHSA_EINVAL, "d_model %d must be a positive multiple of n_heads %d", d_model, n_heads);
  const int dk = d_model / n_heads;
  if (dk != 64 && dk != 128) return fail(MHSA_ENOTSUP, "head_dim %d not supported (64 or 128)", dk);
  if (d_model % 128) return fail(MHSA_ENOTSUP, "d_model %d must be a multiple of 128", d_model);
  mhsa_layer* L = new (std::nothrow) mhsa_layer();
  if (!L) return fail(MHSA_ENOMEM, "out of host memory");
  L->D = d_model;
  L->H = n_heads;
  L->dk = dk;
  L->use_bias = use_bias != 0;
  for (int i = 0; i < 5; ++i) {
    L->lin[i].w.assign((size_t)d_model * d_model, 0.f);
    if (use_bias && i != MHSA_LINEAR_POS) L->lin[i].bias.assign(d_model, 0.f);
  }
  L->pbu.assign(d_model, 0.f);
  L->pbv.assign(d_model, 0.f);
  *out = L;
  return MHSA_OK;
}

void mhsa_destroy(mhsa_layer* layer) { delete layer; }

int32_t mhsa_set_dtype(mhsa_layer* L, int32_t dtype) {
  if (int32_t rc = check_layer(L)) return rc;
  if (dtype != MHSA_F32 && dtype != MHSA_BF16) return fail(MHSA_ENOTSUP, "dtype %d not supported (f32, bf16)", dtype);
  L->dt = dtype == MHSA_F32 ? mhsa::kF32 : mhsa::kBF16;
  L->dirty = true;
  L->pmemo_len = -1;
  return MHSA_OK;
}
int32_t mhsa_get_dtype(const mhsa_layer* L) { return L ? (L->dt == mhsa::kF32 ? MHSA_F32 : MHSA_BF16) : -1; }
int32_t mhsa_head_dim(const mhsa_layer* L) { return L ? L->dk : -1; }
int32_t mhsa_n_heads(const mhsa_layer* L) { return L ? L->H : -1; }
int32_t mhsa_d_model(const mhsa_layer* L) { return L ? L->D : -1; }
int32_t mhsa_set_cache_drop_size(mhsa_layer* L, int32_t n) {
  if (int32_t rc = check_layer(L)) return rc;
  if (n < 0) return fail(MHSA_EINVAL, "cache_drop_size must be >= 0");
  L->cache_drop = n;
  return MHSA_OK;
}

int32_t mhsa_load_linear_standard(mhsa_layer* L, int32_t which, int32_t dtype, const void* weight, const void* bias) {
  if (int32_t rc = check_layer(L)) return rc;
  if (which < 0 || which > 4) return fail(MHSA_EINVAL, "unknown projection %d", which);
  if (!weight || !float_dtype(dtype)) return fail(MHSA_EINVAL, "weight must be f32/bf16/f16 host data");
  HostLinear& h = L->lin[which];
  const size_t n = (size_t)L->D * L->D;
  h.quantized = false;
  h.codes.clear();
  h.qs.clear();
  h.qb.clear();
  h.w.resize(n);
  for (size_t i = 0; i < n; ++i) h.w[i] = load_host(dtype, weight, i);
  h.bias.clear();
  if (bias) {
    h.bias.resize(L->D);
    for (int i = 0; i < L->D; ++i) h.bias[i] = load_host(dtype, bias, i);
  }
  L->dirty = true;
  return MHSA_OK;
}

int32_t mhsa_load_linear_quantized(mhsa_layer* L, int32_t which, const uint32_t* weight, const uint16_t* scales,
                                   const uint16_t* biases, const uint16_t* bias, int32_t bits, int32_t group) {
  if (int32_t rc = check_layer(L)) return rc;
  if (which < 0 || which > 4) return fail(MHSA_EINVAL, "unknown projection %d", which);
  if (bits != 8 || group != 64)
    return fail(MHSA_ENOTSUP, "quantization bits=%d group_size=%d not supported (8, 64)", bits, group);
  if (!weight || !scales || !biases) return fail(MHSA_EINVAL, "null quantized tensor");
  HostLinear& h = L->lin[which];
  const int D = L->D, G = D / 64;
  h.quantized = true;
  h.w.clear();
  h.codes.assign(weight, weight + (size_t)D * D / 4);
  h.qs.resize((size_t)D * G);
  h.qb.resize((size_t)D * G);
  for (size_t i = 0; i < h.qs.size(); ++i) {
    h.qs[i] = f16_to_f32(scales[i]);
    h.qb[i] = f16_to_f32(biases[i]);
  }
  h.bias.clear();
  if (bias) {
    h.bias.resize(D);
    for (int i = 0; i < D; ++i) h.bias[i] = f16_to_f32(bias[i]);
  }
  L->dirty = true;
  return MHSA_OK;
}

int32_t mhsa_load_pos_bias(mhsa_layer* L, int32_t dtype, const void* u, const void* v) {
  if (int32_t rc = check_layer(L)) return rc;
  if (!u || !v || !float_dtype(dtype)) return fail(MHSA_EINVAL, "pos biases must be f32/bf16/f16 host data");
  for (int i = 0; i < L->D; ++i) {
    L->pbu[i] = load_host(dtype, u, i);
    L->pbv[i] = load_host(dtype, v, i);
  }
  L->dirty = true;
  return MHSA_OK;
}

int32_t mhsa_load_weights(mhsa_layer* L, const mhsa_tensor* tensors, int32_t n, const char* prefix, int32_t strict,
                          int32_t quant_bits, int32_t quant_group) {
  if (int32_t rc = check_layer(L)) return rc;
  if ((n > 0 && !tensors) || !prefix) return fail(MHSA_EINVAL, "null tensor list or prefix");
  auto find = [&](const std::string& key) -> const mhsa_tensor* {
    for (int i = 0; i < n; ++i)
      if (tensors[i].name && key == tensors[i].name) return &tensors[i];
    return nullptr;
  };
  auto numel = [](const mhsa_tensor* t) {
    int64_t e = 1;
    for (int i = 0; i < t->ndim; ++i) e *= t->shape[i];
    return e;
  };
  const int D = L->D;
  const char* names[5] = {"linear_q", "linear_k", "linear_v", "linear_out", "linear_pos"};
  const int bits = quant_bits > 0 ? quant_bits : 8, group = quant_group > 0 ? quant_group : 64;
  for (int i = 0; i < 5; ++i) {
    const std::string p = std::string(prefix) + "." + names[i];
    const mhsa_tensor* w = find(p + ".weight");
    const mhsa_tensor* sc = find(p + ".scales");
    const mhsa_tensor* qb = find(p + ".biases");
    const mhsa_tensor* b = find(p + ".bias");
    if (w && sc && qb) {  // quantization.rs:299-304
      if (bits != 8 || group != 64)
        return fail(MHSA_ENOTSUP, "`%s`: quantization bits=%d group_size=%d not supported (8, 64)", p.c_str(), bits,
                    group);
      if (w->dtype != MHSA_U32 || sc->dtype != MHSA_F16 || qb->dtype != MHSA_F16)
        return fail(MHSA_EINVAL, "`%s`: quantized tensors must be u32 weight and f16 scales/biases", p.c_str());
      if (numel(w) != (int64_t)D * D * bits / 32 || numel(sc) != (int64_t)D * D / group || numel(qb) != numel(sc))
        return fail(MHSA_EINVAL, "`%s`: quantized shapes do not match d_model %d", p.c_str(), D);
      if (b && (b->dtype != MHSA_F16 || numel(b) != D))
        return fail(MHSA_EINVAL, "`%s.bias`: expected f16 [%d]", p.c_str(), D);
      int32_t rc = mhsa_load_linear_quantized(L, i, static_cast<const uint32_t*>(w->data),
                                              static_cast<const uint16_t*>(sc->data),
                                              static_cast<const uint16_t*>(qb->data),
                                              b ? static_cast<const uint16_t*>(b->data) : nullptr, bits, group);
      if (rc) return rc;
    } else if (w) {
      // [O, I] or a pointwise-conv [O, 1, I] (quantization.rs:330-335)
      const bool shape_ok = (w->ndim == 2 && w->shape[0] == D && w->shape[1] == D) ||
                            (w->ndim == 3 && w->shape[0] == D && w->shape[1] == 1 && w->shape[2] == D);
      if (!shape_ok || !float_dtype(w->dtype))
        return fail(MHSA_EINVAL, "`%s.weight`: expected float [%d, %d]", p.c_str(), D, D);
      if (b && (!float_dtype(b->dtype) || numel(b) != D))
        return fail(MHSA_EINVAL, "`%s.bias`: expected float [%d]", p.c_str(), D);
      if (b && b->dtype != w->dtype) {
        std::vector<float> bb(D);
        for (int k = 0; k < D; ++k) bb[k] = load_host(b->dtype, b->data, k);
        int32_t rc = mhsa_load_linear_standard(L, i, w->dtype, w->data, nullptr);
        if (rc) return rc;
        L->lin[i].bias = bb;
      } else {
        int32_t rc = mhsa_load_linear_standard(L, i, w->dtype, w->data, b ? b->data : nullptr);
        if (rc) return rc;
      }
    } else if (strict) {
      return fail(MHSA_ENOENT, "missing weight `%s.weight`", p.c_str());  // loading.rs:107-116
    }
  }
  const mhsa_tensor* tu = find(std::string(prefix) + ".pos_bias_u");
  const mhsa_tensor* tv = find(std::string(prefix) + ".pos_bias_v");
  for (const mhsa_tensor* t : {tu, tv}) {
    if (t && (!float_dtype(t->dtype) || numel(t) != D))
      return fail(MHSA_EINVAL, "`%s`: expected float [%d, %d]", t->name, L->H, L->dk);
  }
  if (strict && (!tu || !tv))
    return fail(MHSA_ENOENT, "missing weight `%s.%s`", prefix, tu ? "pos_bias_v" : "pos_bias_u");
  if (tu)
    for (int k = 0; k < D; ++k) L->pbu[k] = load_host(tu->dtype, tu->data, k);
  if (tv)
    for (int k = 0; k < D; ++k) L->pbv[k] = load_host(tv->dtype, tv->data, k);
  L->dirty = true;
  return MHSA_OK;
}

int32_t mhsa_forward(mhsa_layer* L, const void* x, int32_t batch, int32_t seq_len, const void* pos_emb,
                     int32_t pos_len, const mhsa_context* ctx, const int32_t* lens, void* out, void* hs) {
  if (int32_t rc = check_layer(L)) return rc;
  if (!out) return fail(MHSA_EINVAL, "null output pointer");
  return forward_impl(L, x, batch, seq_len, pos_emb, pos_len, ctx, lens, out, nullptr, AttnDebug(),
                      static_cast<hipStream_t>(hs));
}

int32_t mhsa_forward_noalloc(mhsa_layer* L, const void* x, int32_t batch, int32_t seq_len, const void* pos_emb,
                             int32_t pos_len, const mhsa_context* ctx, const int32_t* lens, void* out, void* hs) {
  if (int32_t rc = check_layer(L)) return rc;
  if (!out) return fail(MHSA_EINVAL, "null output pointer");
  char* base = nullptr;
  if (int32_t rc = scratch_for_current_device(&base)) return rc;
  Arena arena;
  arena.base = base + kNoAllocPartialBytes;
  arena.cap = kNoAllocScratchBytes - kNoAllocPartialBytes;
  L->partial_override = reinterpret_cast<float*>(base);
  const int32_t rc = forward_impl(L, x, batch, seq_len, pos_emb, pos_len, ctx, lens, out, nullptr, AttnDebug(),
                                  static_cast<hipStream_t>(hs), &arena);
  L->partial_override = nullptr;
  return rc;
}

int32_t mhsa_sublayer_forward(mhsa_layer* L, void* x, int32_t batch, int32_t seq_len, const float* gamma,
                              const float* beta, float eps, const void* pos_emb, int32_t pos_len,
                              const mhsa_context* ctx, const int32_t* lens, void* hs) {
  if (int32_t rc = check_layer(L)) return rc;
  if (!x || batch <= 0 || seq_len <= 0) return fail(MHSA_EINVAL, "bad sublayer arguments");
  if (!aligned16(x)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(hs);
  const float* gd = nullptr;
  const float* bd = nullptr;
  if (int32_t rc = sublayer_norm(L, gamma, beta, (int64_t)batch * seq_len, &gd, &bd)) return rc;
  {
    LayerProf ps(L, "layer_norm", s);
    for (int r = ps.reps(); r > 0; --r)
      HIPCHK(mhsa::layer_norm(dtype_of(L), x, L->hbuf.p, gd, bd, eps, (int)((int64_t)batch * seq_len), L->D, s));
  }
  return forward_impl(L, L->hbuf.p, batch, seq_len, pos_emb, pos_len, ctx, lens, x, x, AttnDebug(), s);
}

int32_t mhsa_stack_sublayer_forward(mhsa_layer* const* layers, int32_t n_layers, void* x, int32_t batch,
                                    int32_t seq_len, const float* gammas, const float* betas, float eps,
                                    const void* pos_emb, int32_t pos_len, const mhsa_context* ctx,
                                    const int32_t* lens, void* hs) {
  if (!layers || n_layers <= 0) return fail(MHSA_EINVAL, "the stack needs at least one layer");
  for (int l = 0; l < n_layers; ++l) {
    if (int32_t rc = check_layer(layers[l])) return rc;
    if (layers[l]->D != layers[0]->D || layers[l]->dt != layers[0]->dt)
      return fail(MHSA_EINVAL, "layer %d has d_model %d / dtype %d, layer 0 has %d / %d", l, layers[l]->D,
                  (int)layers[l]->dt, layers[0]->D, (int)layers[0]->dt);
  }
  if (!x || batch <= 0 || seq_len <= 0) return fail(MHSA_EINVAL, "bad sublayer arguments");
  if (!pos_emb) return fail(MHSA_EINVAL, "null tensor pointer");
  if (!aligned16(x) || !aligned16(pos_emb)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(hs);
  const int64_t M = (int64_t)batch * seq_len;
  // every layer's parameters, norm and workspace before the first launch:
  // layer l + 1's position rows are projected while layer l runs
  std::vector<OfflineLayout> lay(n_layers);
  std::vector<const float*> gd(n_layers), bd(n_layers);
  for (int l = 0; l < n_layers; ++l) {
    mhsa_layer* L = layers[l];
    if (int32_t rc = prepare(L)) return rc;
    const size_t off = (size_t)l * L->D;
    if (int32_t rc = sublayer_norm(L, gammas ? gammas + off : nullptr, betas ? betas + off : nullptr, M, &gd[l], &bd[l]))
      return rc;
    if (int32_t rc = offline_layout(L, batch, seq_len, pos_len, ctx, lens, s, nullptr, lay[l])) return rc;
  }
  {
    mhsa_layer* L = layers[0];
    LayerProf ps(L, "gemm_pos", s);
    mhsa::GemmParams g;
    if (int32_t rc = pos_gemm(L, lay[0], pos_emb, g)) return rc;
    for (int r = ps.reps(); r > 0; --r) HIPCHK(mhsa::gemm(L->dt, L->dev[4].quantized, g, s));
  }
  for (int l = 0; l < n_layers; ++l) {
    mhsa_layer* L = layers[l];
    {
      LayerProf ps(L, "layer_norm", s);
      for (int r = ps.reps(); r > 0; --r)
        HIPCHK(mhsa::layer_norm(dtype_of(L), x, L->hbuf.p, gd[l], bd[l], eps, (int)M, L->D, s));
    }
    FusedNext nx;
    if (l + 1 < n_layers) {
      mhsa_layer* N = layers[l + 1];
      if (int32_t rc = pos_gemm(N, lay[l + 1], pos_emb, nx.g)) return rc;
      nx.quant = N->dev[4].quantized;
      nx.dt = N->dt;
    }
    if (int32_t rc = forward_impl(L, L->hbuf.p, batch, seq_len, pos_emb, pos_len, ctx, lens, x, x, AttnDebug(), s,
                                  nullptr, &lay[l], l + 1 < n_layers ? &nx : nullptr))
      return rc;
  }
  return MHSA_OK;
}

int32_t mhsa_stream_create(mhsa_layer* L, int32_t batch, int32_t cache_size, int32_t chunk_len, mhsa_stream** out) {
  if (int32_t rc = check_layer(L)) return rc;
  if (!out) return fail(MHSA_EINVAL, "null output pointer");
  *out = nullptr;
  if (batch <= 0 || cache_size < 0 || chunk_len <= 0)
    return fail(MHSA_EINVAL, "bad stream shape (batch %d, cache %d, chunk %d)", batch, cache_size, chunk_len);
  mhsa_stream* S = new (std::nothrow) mhsa_stream();
  if (!S) return fail(MHSA_ENOMEM, "out of host memory");
  S->layer = L;
  S->B = batch;
  S->C = cache_size;
  S->Tc = chunk_len;
  S->R = cache_size + chunk_len;
  S->fill.assign(batch, 0);
  const int D = L->D;
  const size_t hb = (size_t)batch * S->R * D * 4, kvb = 2 * hb;
  hipError_t e = S->ring_h.ensure(hb);
  if (e == hipSuccess) e = S->ring_kv.ensure(kvb);
  if (e == hipSuccess) e = hipMemset(S->ring_h.p, 0, hb);
  if (e == hipSuccess) e = hipMemset(S->ring_kv.p, 0, kvb);
  if (e != hipSuccess) {
    delete S;
    return fail(MHSA_EHIP, "stream allocation: %s", hipGetErrorString(e));
  }
  *out = S;
  return MHSA_OK;
}

void mhsa_stream_destroy(mhsa_stream* S) { delete S; }

int32_t mhsa_stream_fill(const mhsa_stream* S, int32_t* out) {
  if (!S || !out) return fail(MHSA_EINVAL, "null argument");
  std::copy(S->fill.begin(), S->fill.end(), out);
  return MHSA_OK;
}

int32_t mhsa_stream_load_cache(mhsa_stream* S, const void* cache, const int32_t* filled, void* hs) {
  if (!S || !cache) return fail(MHSA_EINVAL, "null argument");
  mhsa_layer* L = S->layer;
  if (!aligned16(cache)) return fail(MHSA_EINVAL, "cache must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(hs);
  int32_t rc = prepare_stream(L);
  if (rc) return rc;
  const int D = L->D;
  S->head = 0;
  for (int b = 0; b < S->B; ++b) S->fill[b] = filled ? std::min(std::max(filled[b], 0), S->C) : 0;
  if (S->C > 0) HIPCHK(mhsa::ring_write(mhsa::kF32, cache, S->ring_h.p, S->B, S->C, D, S->R, D, 0, s));
  return reproject_ring(L, S, s);
}

int32_t mhsa_stream_read_cache(const mhsa_stream* S, void* out, void* hs) {
  if (!S || !out) return fail(MHSA_EINVAL, "null argument");
  if (!aligned16(out)) return fail(MHSA_EINVAL, "cache_out must be 16-byte aligned");
  HIPCHK(mhsa::ring_read(mhsa::kF32, S->ring_h.p, out, S->B, S->C, S->layer->D, S->R, S->layer->D, S->head,
                         static_cast<hipStream_t>(hs)));
  return MHSA_OK;
}

}  // extern "C"

namespace {

// One cache-aware step (S != null: the chunk against the stream's ring) or
// the no-cache form (S == null: keys and values from x alone,
// attention.rs:687-700), both in fp32 (prepare_stream says why).
// lens (no cache only): the offline key padding, keys past lens[b] (clamped
// to >= 1) hidden as offline_key_bounds hides them.
int32_t stream_step(mhsa_layer* L, mhsa_stream* S, const void* x, int B, int T, const void* pos_emb, int pos_len,
                    const mhsa_stream_mask* mask, void* out, hipStream_t s, const void* residual = nullptr,
                    const int32_t* lens = nullptr) {
  if (!x || !pos_emb || !out) return fail(MHSA_EINVAL, "null tensor pointer");
  if (!aligned16(x) || !aligned16(pos_emb) || !aligned16(out))
    return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  if (B <= 0 || T <= 0) return fail(MHSA_EINVAL, "batch and seq_len must be positive (got %d, %d)", B, T);
  int32_t rc = prepare_stream(L);
  if (rc) return rc;
  const int D = L->D, C = S ? S->C : 0, R = S ? S->R : 0, Lk = C + T;
  const bool masked = mask && mask->present;
  const mhsa_context* ctx = masked ? &mask->ctx : nullptr;
  const DistRange dr = context_distances(ctx, C, T, Lk);
  int row0, nrows, center;
  if ((rc = plan_positions(pos_len, Lk, dr, row0, nrows, center))) return rc;

  // memoised position projection, keyed by pos_len (attention.rs:749-761);
  // a bf16 layer projects its bf16 table in bf16 and widens the result
  if (L->pmemo_len != pos_len) {
    HIPCHK(L->pmemo.ensure(align_up((int64_t)pos_len * D * 4, 256)));
    LayerProf ps(L, "gemm_pos", s, true, false);
    if (L->dt == mhsa::kBF16) {
      HIPCHK(L->pmemo_bf16.ensure(align_up((int64_t)pos_len * D * 2, 256)));
      if ((rc = run_gemm(L, mhsa::kBF16, L->dev[4], D, pos_emb, D, pos_len, L->pmemo_bf16.p, D, nullptr, 0, s)))
        return rc;
      HIPCHK(mhsa::widen_bf16(L->pmemo_bf16.p, static_cast<float*>(L->pmemo.p), (int64_t)pos_len * D, s));
    } else if ((rc = run_gemm(L, mhsa::kF32, L->sdev[4], D, pos_emb, D, pos_len, L->pmemo.p, D, nullptr, 0, s))) {
      return rc;
    }
    L->pmemo_len = pos_len;
  }
  if (S && S->kv_version != L->version && (rc = reproject_ring(L, S, s))) return rc;
  const int64_t M = (int64_t)B * T;
  const size_t qb = align_up(M * D * 4, 256);
  DevBuf& ws = S ? S->ws : L->uws;
  HIPCHK(ws.ensure((S ? 2 : 4) * qb));
  char* q = static_cast<char*>(ws.p);  // [M, D] (cached) or [M, 3D] q|k|v rows (no cache)
  char* cx = q + (S ? 1 : 3) * qb;
  const int slot = S ? (S->head + C) % R : 0;  // ring rows of this chunk
  char* kv = S ? static_cast<char*>(S->ring_kv.p) : q + (size_t)D * 4;

  // (the fused chunk launch's parameters; used when the shape allows it)
  mhsa::GemmParams fp;
  if (S && L->qkv_fused) {
    fp.A = x;
    fp.lda = D;
    fp.W = L->sdev[0].w;
    fp.sb = L->sdev[0].sb;
    fp.bias = L->sdev[0].bias;
    fp.C = q;
    fp.ldc = D;
    fp.C2 = kv;
    fp.ldc2 = 2 * D;
    fp.c2_col0 = D;
    fp.acopy = S->ring_h.p;
    fp.acopy_ld = D;
    fp.M = (int)M;
    fp.N = 3 * D;
    fp.K = D;
    fp.seg_rows = T;
    fp.seg_stride = R;
    fp.ring_off = slot;
    fp.ring_len = R;
  }
  const bool one_launch = !S || (L->qkv_fused && mhsa::gemm_split_fused_ok(mhsa::kF32, fp));
  // (only the one-launch ring form is repeated: it rewrites the same rows)
  LayerProf ps_kv(L, one_launch ? "gemm_qkv" : "gemm_q", s, true, S && one_launch);
  if (!S) {
    if (L->qkv_fused) {
      if ((rc = run_gemm(L, mhsa::kF32, L->sdev[0], 3 * D, x, D, (int)M, q, 3 * D, nullptr, 0, s))) return rc;
    } else {
      for (int i = 0; i < 3; ++i)
        if ((rc = run_gemm(L, mhsa::kF32, L->sdev[i], D, x, D, (int)M, q + (size_t)i * D * 4, 3 * D, nullptr, 0, s)))
          return rc;
    }
  } else {
    // One launch when the layer holds the stacked [3D, D] weight: Q to `q`,
    // K|V to the cache ring's rows of this chunk, and the chunk's input rows
    // copied into the input ring by the workgroups of the first column tile.
    if (one_launch) {
      for (int r = ps_kv.reps(); r > 0; --r) HIPCHK(mhsa::gemm(mhsa::kF32, L->sdev[0].quantized, fp, s));
    } else {
      if ((rc = run_gemm(L, mhsa::kF32, L->sdev[0], D, x, D, (int)M, q, D, nullptr, 0, s))) return rc;
      ps_kv.next("gemm_kv", false);
      if (L->qkv_fused) {
        if ((rc = run_gemm(L, mhsa::kF32, L->sdev[1], 2 * D, x, D, (int)M, kv, 2 * D, nullptr, 0, s, T, R, slot, R)))
          return rc;
      } else {
        if ((rc = run_gemm(L, mhsa::kF32, L->sdev[1], D, x, D, (int)M, kv, 2 * D, nullptr, 0, s, T, R, slot, R)))
          return rc;
        if ((rc = run_gemm(L, mhsa::kF32, L->sdev[2], D, x, D, (int)M, kv + (size_t)D * 4, 2 * D, nullptr, 0, s, T,
                           R, slot, R)))
          return rc;
      }
      ps_kv.next("ring_write", false);
      HIPCHK(mhsa::ring_write(mhsa::kF32, x, S->ring_h.p, B, T, D, R, D, slot, s));
    }
  }
  ps_kv.next("attention");

  std::vector<int32_t> used(B);
  for (int b = 0; b < B; ++b)
    used[b] = std::min(std::max(masked && mask->filled_host ? mask->filled_host[b] : (S ? S->fill[b] : 0), 0), C);
  mhsa::AttnParams a;
  fill_attn_common(L, a);
  a.scale_bd = a.scale;  // bd is an f32 array on this path: cast(s) is s (attention.rs:308-311)
  a.q = q;
  a.q_bs = (int64_t)T * (S ? D : 3 * D);
  a.q_rs = S ? D : 3 * D;
  a.k = kv;
  a.v = kv + (size_t)D * 4;
  a.kv_bs = S ? (int64_t)R * 2 * D : (int64_t)T * 3 * D;
  a.kv_rs = S ? 2 * D : 3 * D;
  a.ring_head = S ? S->head : 0;
  a.ring_len = R;
  a.p = static_cast<char*>(L->pmemo.p) + (size_t)row0 * D * 4;
  a.p_rs = D;
  a.p_rows = nrows;
  a.center = center;
  a.o = cx;
  a.o_bs = (int64_t)T * D;
  a.o_rs = D;
  a.T = T;
  a.L = Lk;
  a.qoff = C;
  set_ctx(a, ctx);
  for (int r = ps_kv.reps(); r > 0 && !rc; --r)
    rc = run_attention(
        L, mhsa::kF32, a, B,
        [&](int b, int& lo, int& hi, int& qv) {
          lo = masked ? C - used[b] : 0;  // unfilled cache rows (conformer.rs:155-181)
          hi = lens && !S ? std::min(std::max(lens[b], 1), T) : Lk;
          qv = masked && mask->valid_host ? std::min(std::max(mask->valid_host[b], 0), T) : T;
        },
        s);
  if (rc) return rc;
  ps_kv.next("gemm_out", residual != out);
  for (int r = ps_kv.reps(); r > 0 && !rc; --r)
    rc = run_gemm(L, mhsa::kF32, L->sdev[3], D, cx, D, (int)M, out, D, residual, D, s);
  if (rc) return rc;
  if (S) {
    const int keep = std::max(T - L->cache_drop, 0);  // attention.rs:665
    S->head = (S->head + keep) % R;
    for (int b = 0; b < B; ++b) S->fill[b] = std::min(used[b] + keep, C);  // conformer.rs:1025-1036
  }
  return MHSA_OK;
}

}  // namespace

extern "C" {

int32_t mhsa_forward_with_cache(mhsa_layer* L, mhsa_stream* S, const void* x, const void* pos_emb, int32_t pos_len,
                                const mhsa_stream_mask* mask, void* out, void* hs) {
  if (int32_t rc = check_layer(L)) return rc;
  if (!S || S->layer != L) return fail(MHSA_EINVAL, "stream does not belong to this layer");
  return stream_step(L, S, x, S->B, S->Tc, pos_emb, pos_len, mask, out, static_cast<hipStream_t>(hs));
}

int32_t mhsa_forward_uncached(mhsa_layer* L, const void* x, int32_t batch, int32_t seq_len, const void* pos_emb,
                              int32_t pos_len, const mhsa_stream_mask* mask, void* out, void* hs) {
  if (int32_t rc = check_layer(L)) return rc;
  return stream_step(L, nullptr, x, batch, seq_len, pos_emb, pos_len, mask, out, static_cast<hipStream_t>(hs));
}

}  // extern "C"

int32_t mhsa_sublayer_forward_act32(mhsa_layer* L, float* x, int B, int T, const float* gamma, const float* beta,
                                    float eps, const void* pos_emb, int pos_len, const mhsa_context* ctx,
                                    const int32_t* lens, hipStream_t s) {
  if (int32_t rc = check_layer(L)) return rc;
  if (!x || B <= 0 || T <= 0) return fail(MHSA_EINVAL, "bad sublayer arguments");
  if (!aligned16(x)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  const int64_t rows = (int64_t)B * T;
  const float* gd = nullptr;
  const float* bd = nullptr;
  if (int32_t rc = sublayer_norm(L, gamma, beta, rows, &gd, &bd)) return rc;
  HIPCHK(L->hbuf.ensure(align_up(rows * L->D * 4, 256)));  // the f32 LayerNorm output
  {
    LayerProf ps(L, "layer_norm", s);
    for (int r = ps.reps(); r > 0; --r)
      HIPCHK(mhsa::layer_norm(mhsa::kF32, x, L->hbuf.p, gd, bd, eps, (int)rows, L->D, s));
  }
  // forward projects its position rows on every call (attention.rs:511),
  // so the streaming path's memo is not reused across calls
  L->pmemo_len = -1;
  mhsa_stream_mask m{};
  if (ctx) {
    m.present = 1;
    m.ctx = *ctx;
  }
  return stream_step(L, nullptr, L->hbuf.p, B, T, pos_emb, pos_len, ctx ? &m : nullptr, x, s, x, lens);
}

struct mhsa_stack {
  std::vector<mhsa_layer*> layers;
  std::vector<mhsa_stream*> streams;
  int B = 0, C = 0, T = 0, D = 0;
  DevBuf h;       // [B, T, D] fp32: LayerNorm output of the current layer
  DevBuf ln;      // [layers, 2, D] fp32 gamma | beta as uploaded
  std::vector<float> ln_host;
  ~mhsa_stack() {
    for (mhsa_stream* st : streams) mhsa_stream_destroy(st);
  }
};

extern "C" {

int32_t mhsa_stack_create(mhsa_layer* const* layers, int32_t n_layers, int32_t batch, int32_t cache_size,
                          int32_t chunk_len, mhsa_stack** out) {
  if (!out || !layers || n_layers <= 0) return fail(MHSA_EINVAL, "null or empty layer list");
  *out = nullptr;
  std::unique_ptr<mhsa_stack> K(new (std::nothrow) mhsa_stack());
  if (!K) return fail(MHSA_ENOMEM, "out of host memory");
  for (int i = 0; i < n_layers; ++i) {
    if (!layers[i]) return fail(MHSA_EINVAL, "layer %d is null", i);
    if (layers[i]->D != layers[0]->D) return fail(MHSA_EINVAL, "layer %d has d_model %d, layer 0 %d", i, layers[i]->D,
                                                  layers[0]->D);
    if (layers[i]->D > mhsa::kMaxLayerNormDim)
      return fail(MHSA_ENOTSUP, "the sublayer's LayerNorm supports d_model <= %d", mhsa::kMaxLayerNormDim);
    for (int j = 0; j < i; ++j)
      if (layers[j] == layers[i]) return fail(MHSA_EINVAL, "layer %d appears twice", i);
    mhsa_stream* st = nullptr;
    if (int32_t rc = mhsa_stream_create(layers[i], batch, cache_size, chunk_len, &st)) return rc;
    K->layers.push_back(layers[i]);
    K->streams.push_back(st);
  }
  K->B = batch;
  K->C = cache_size;
  K->T = chunk_len;
  K->D = layers[0]->D;
  HIPCHK(K->h.ensure(align_up((int64_t)batch * chunk_len * K->D * 4, 256)));
  *out = K.release();
  return MHSA_OK;
}

void mhsa_stack_destroy(mhsa_stack* K) { delete K; }

int32_t mhsa_stack_load_cache(mhsa_stack* K, const void* cache, const int32_t* filled, void* hs) {
  if (!K || !cache) return fail(MHSA_EINVAL, "null argument");
  const size_t per = (size_t)K->B * K->C * K->D * 4;
  for (size_t l = 0; l < K->streams.size(); ++l)
    if (int32_t rc = mhsa_stream_load_cache(K->streams[l], static_cast<const char*>(cache) + l * per, filled, hs))
      return rc;
  return MHSA_OK;
}

int32_t mhsa_stack_read_cache(const mhsa_stack* K, void* out, void* hs) {
  if (!K || !out) return fail(MHSA_EINVAL, "null argument");
  const size_t per = (size_t)K->B * K->C * K->D * 4;
  for (size_t l = 0; l < K->streams.size(); ++l)
    if (int32_t rc = mhsa_stream_read_cache(K->streams[l], static_cast<char*>(out) + l * per, hs)) return rc;
  return MHSA_OK;
}

int32_t mhsa_stack_fill(const mhsa_stack* K, int32_t* out) {
  if (!K) return fail(MHSA_EINVAL, "null argument");
  return mhsa_stream_fill(K->streams[0], out);
}

int32_t mhsa_stack_step(mhsa_stack* K, void* x, const float* gamma, const float* beta, float eps, const void* pos_emb,
                        int32_t pos_len, const mhsa_stream_mask* mask, void* hs) {
  if (!K || !x) return fail(MHSA_EINVAL, "null argument");
  if (!aligned16(x)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(hs);
  const int D = K->D, n = (int)K->layers.size();
  const int64_t M = (int64_t)K->B * K->T;
  // per-layer LayerNorm gamma/beta ([layers, D] host arrays), held at each
  // layer's parameter precision (conformer.rs:422-434 casts the norms too)
  const float* g = nullptr;
  if (gamma || beta) {
    std::vector<float> tmp((size_t)2 * n * D);
    for (int l = 0; l < n; ++l) {
      const bool bf = K->layers[l]->dt == mhsa::kBF16;
      for (int i = 0; i < D; ++i) {
        const float gv = gamma ? gamma[(size_t)l * D + i] : 1.f, bv = beta ? beta[(size_t)l * D + i] : 0.f;
        tmp[(size_t)2 * l * D + i] = bf ? round_bf16(gv) : gv;
        tmp[(size_t)(2 * l + 1) * D + i] = bf ? round_bf16(bv) : bv;
      }
    }
    if (tmp != K->ln_host) {
      if (K->ln.p) HIPCHK(hipDeviceSynchronize());  // an earlier step may still read them
      HIPCHK(K->ln.ensure(tmp.size() * 4));
      HIPCHK(hipMemcpy(K->ln.p, tmp.data(), tmp.size() * 4, hipMemcpyHostToDevice));
      K->ln_host = tmp;
    }
    g = static_cast<const float*>(K->ln.p);
  }
  // every layer reads the fills of the step's start; each stream then moves
  // its own copy the same way (conformer.rs:1025-1036)
  std::vector<int32_t> fills(K->B);
  if (int32_t rc = mhsa_stream_fill(K->streams[0], fills.data())) return rc;
  mhsa_stream_mask m;
  if (mask && mask->present) {
    m = *mask;
    if (!m.filled_host) m.filled_host = fills.data();
    mask = &m;
  }
  for (int l = 0; l < n; ++l) {
    mhsa_layer* L = K->layers[l];
    {
      LayerProf ps(L, "layer_norm", s, true, false);
      HIPCHK(mhsa::layer_norm(mhsa::kF32, x, K->h.p, g ? g + (size_t)2 * l * D : nullptr,
                              g ? g + (size_t)(2 * l + 1) * D : nullptr, eps, (int)M, D, s));
    }
    if (int32_t rc = stream_step(L, K->streams[l], K->h.p, K->B, K->T, pos_emb, pos_len, mask, x, s, x)) return rc;
  }
  return MHSA_OK;
}

int32_t mhsa_pos_encoding(int32_t d_model, int32_t max_len, int32_t seq_len, float* out) {
  if (!out) return fail(MHSA_EINVAL, "null output pointer");
  if (seq_len <= 0) return fail(MHSA_EINVAL, "positional encoding requested for an empty sequence");
  if (d_model <= 0 || d_model % 2 || max_len <= 0) return fail(MHSA_EINVAL, "bad d_model / max_len");
  // Rows of a table of any max_len >= seq_len agree for the same distance,
  // so the slice (attention.rs:158-174) and the regenerated table
  // (attention.rs:137-145) are both the distances seq_len-1 .. -(seq_len-1).
  const float step = std::log(10000.0f) / (float)d_model;
  std::vector<float> div(d_model / 2);
  for (int k = 0; k < d_model / 2; ++k) div[k] = std::exp(-(float)(2 * k) * step);
  for (int r = 0; r < 2 * seq_len - 1; ++r) {
    const float pos = (float)(seq_len - 1 - r);
    for (int k = 0; k < d_model / 2; ++k) {
      const float ang = pos * div[k];
      out[(size_t)r * d_model + 2 * k] = (float)std::sin((double)ang);
      out[(size_t)r * d_model + 2 * k + 1] = (float)std::cos((double)ang);
    }
  }
  return MHSA_OK;
}

int32_t mhsa_profile_enable(mhsa_layer* L, int32_t enable) {
  if (int32_t rc = check_layer(L)) return rc;
  return L->prof.enable(enable);
}

int32_t mhsa_profile_repeat(mhsa_layer* L, const char* tag, int32_t n) {
  if (int32_t rc = check_layer(L)) return rc;
  return L->prof.set_repeat(tag, n);
}

int32_t mhsa_profile_reset(mhsa_layer* L) {
  if (int32_t rc = check_layer(L)) return rc;
  return L->prof.reset();
}

int32_t mhsa_profile_count(mhsa_layer* L) { return L ? L->prof.entries() : -1; }

int32_t mhsa_profile_entry(mhsa_layer* L, int32_t idx, const char** name, double* total_ms, int32_t* launches) {
  if (int32_t rc = check_layer(L)) return rc;
  return L->prof.entry(idx, name, total_ms, launches);
}

int32_t mhsa_debug_dequantize(mhsa_layer* L, int32_t which, float* out, void* hs) {
  if (int32_t rc = check_layer(L)) return rc;
  if (which < 0 || which > 4 || !out) return fail(MHSA_EINVAL, "bad arguments");
  if (!L->lin[which].quantized) return fail(MHSA_EINVAL, "projection %d is not quantized", which);
  int32_t rc = prepare(L);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(hs);
  HIPCHK(mhsa::dequant_export(dtype_of(L), static_cast<const uint32_t*>(L->dev[which].w), L->dev[which].sb, out, L->D,
                              L->D, s));
  HIPCHK(hipStreamSynchronize(s));
  return MHSA_OK;
}

int32_t mhsa_debug_linear(mhsa_layer* L, int32_t which, const void* x, int32_t rows, void* out, void* hs) {
  if (int32_t rc = check_layer(L)) return rc;
  if (which < 0 || which > 4 || !x || !out || rows < 0) return fail(MHSA_EINVAL, "bad arguments");
  if (!aligned16(x) || !aligned16(out)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  int32_t rc = prepare(L);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(hs);
  if ((rc = run_gemm(L, L->dt, L->dev[which], L->D, x, L->D, rows, out, L->D, nullptr, 0, s))) return rc;
  HIPCHK(hipStreamSynchronize(s));
  return MHSA_OK;
}

int32_t mhsa_debug_attention_forms(int64_t* counts, int32_t n) {
  if (!counts || n < 0) return fail(MHSA_EINVAL, "bad arguments");
  for (int f = 0; f < n && f < mhsa::kAttnForms; ++f) counts[f] = mhsa::attention_form_count(f);
  return mhsa::kAttnForms;
}

int32_t mhsa_debug_layer_norm(mhsa_layer* L, const void* x, int32_t rows, const float* gamma, const float* beta,
                              float eps, void* out, void* hs) {
  if (int32_t rc = check_layer(L)) return rc;
  if (!x || !out || rows <= 0) return fail(MHSA_EINVAL, "bad arguments");
  if (!aligned16(x) || !aligned16(out)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  const float* gd = nullptr;
  const float* bd = nullptr;
  if (int32_t rc = sublayer_norm(L, gamma, beta, rows, &gd, &bd)) return rc;
  hipStream_t s = static_cast<hipStream_t>(hs);
  HIPCHK(mhsa::layer_norm(dtype_of(L), x, out, gd, bd, eps, rows, L->D, s));
  HIPCHK(hipStreamSynchronize(s));
  return MHSA_OK;
}

int32_t mhsa_debug_linear_f32(mhsa_layer* L, int32_t which, const float* x, int32_t rows, float* out, void* hs) {
  if (int32_t rc = check_layer(L)) return rc;
  if (which < 0 || which > 4 || !x || !out || rows < 0) return fail(MHSA_EINVAL, "bad arguments");
  if (!aligned16(x) || !aligned16(out)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  int32_t rc = prepare_stream(L);
  if (rc) return rc;
  hipStream_t s = static_cast<hipStream_t>(hs);
  if ((rc = run_gemm(L, mhsa::kF32, L->sdev[which], L->D, x, L->D, rows, out, L->D, nullptr, 0, s))) return rc;
  HIPCHK(hipStreamSynchronize(s));
  return MHSA_OK;
}

int32_t mhsa_debug_offline_mask(int32_t B, int32_t T, const mhsa_context* ctx, const int32_t* lens, uint8_t* out,
                                void* hs) {
  if (B <= 0 || T <= 0 || !out) return fail(MHSA_EINVAL, "bad arguments");
  hipStream_t s = static_cast<hipStream_t>(hs);
  mhsa::AttnParams a;
  a.T = a.L = T;
  set_ctx(a, ctx);
  for (int b0 = 0; b0 < B; b0 += mhsa::kMaxBatch) {
    const int nb = std::min(mhsa::kMaxBatch, B - b0);
    for (int i = 0; i < nb; ++i) {
      a.key_lo[i] = 0;
      a.key_hi[i] = lens ? std::min(std::max(lens[b0 + i], 1), T) : T;
      a.q_valid[i] = T;
    }
    HIPCHK(mhsa::export_mask(a, nb, out + (size_t)b0 * T * T, s));
  }
  HIPCHK(hipStreamSynchronize(s));
  return MHSA_OK;
}

int32_t mhsa_debug_stream_mask(int32_t B, int32_t C, int32_t T, const mhsa_stream_mask* mask, uint8_t* out,
                               void* hs) {
  if (B <= 0 || C < 0 || T <= 0 || !out || !mask) return fail(MHSA_EINVAL, "bad arguments");
  if (mask->present && !mask->filled_host) return fail(MHSA_EINVAL, "filled_host is required");
  hipStream_t s = static_cast<hipStream_t>(hs);
  mhsa::AttnParams a;
  a.T = T;
  a.L = C + T;
  a.qoff = C;
  set_ctx(a, mask->present ? &mask->ctx : nullptr);
  for (int b0 = 0; b0 < B; b0 += mhsa::kMaxBatch) {
    const int nb = std::min(mhsa::kMaxBatch, B - b0);
    for (int i = 0; i < nb; ++i) {
      const int f = mask->present ? std::min(std::max(mask->filled_host[b0 + i], 0), C) : C;
      a.key_lo[i] = mask->present ? C - f : 0;
      a.key_hi[i] = C + T;
      a.q_valid[i] = mask->present && mask->valid_host ? std::min(std::max(mask->valid_host[b0 + i], 0), T) : T;
    }
    HIPCHK(mhsa::export_mask(a, nb, out + (size_t)b0 * T * (C + T), s));
  }
  HIPCHK(hipStreamSynchronize(s));
  return MHSA_OK;
}

int32_t mhsa_debug_rel_shift_index(int32_t rows, int32_t total_len, int32_t* out, void* hs) {
  if (rows <= 0 || total_len < rows || !out) return fail(MHSA_EINVAL, "bad arguments");
  hipStream_t s = static_cast<hipStream_t>(hs);
  // bd column = table row: centre total_len - 1, query i at frame total_len - rows + i
  HIPCHK(mhsa::export_pos_index(rows, total_len, total_len - rows, total_len - 1, out, s));
  HIPCHK(hipStreamSynchronize(s));
  return MHSA_OK;
}

int32_t mhsa_debug_position_scores(mhsa_layer* L, const void* x, int32_t B, int32_t T, const void* pos_emb,
                                   int32_t pos_len, float* out, void* q_out, void* p_out, void* hs) {
  if (int32_t rc = check_layer(L)) return rc;
  if (!out) return fail(MHSA_EINVAL, "null output pointer");
  hipStream_t s = static_cast<hipStream_t>(hs);
  AttnDebug dbg;
  dbg.bd = out;
  int32_t rc = forward_impl(L, x, B, T, pos_emb, pos_len, nullptr, nullptr, nullptr, nullptr, dbg, s);
  if (rc) return rc;
  // the workspace still holds [q | k | v] rows and, after them, the projected
  // position table (all pos_len rows: full attention projects every row)
  const size_t es = esz(L);
  const int64_t M = (int64_t)B * T;
  if (q_out)
    HIPCHK(hipMemcpy2DAsync(q_out, (size_t)L->D * es, L->last_qkv, (size_t)3 * L->D * es, (size_t)L->D * es,
                            (size_t)M, hipMemcpyDeviceToDevice, s));
  if (p_out)
    HIPCHK(hipMemcpyAsync(p_out, L->last_pos, (size_t)pos_len * L->D * es, hipMemcpyDeviceToDevice, s));
  HIPCHK(hipStreamSynchronize(s));
  return MHSA_OK;
}

int32_t mhsa_debug_top_keys(mhsa_layer* L, const void* x, int32_t B, int32_t T, const void* pos_emb, int32_t pos_len,
                            const mhsa_context* ctx, const int32_t* lens, int32_t* top_dev, float* logit_dev,
                            void* q_out, void* k_out, void* p_out, void* hs) {
  if (int32_t rc = check_layer(L)) return rc;
  if (!top_dev || !logit_dev) return fail(MHSA_EINVAL, "null output pointer");
  if (L->dt != mhsa::kBF16) return fail(MHSA_ENOTSUP, "top-key export is a bf16-kernel debug output");
  if (p_out && ctx && (ctx->left >= 0 || ctx->right >= 0))
    return fail(MHSA_EINVAL, "position rows are exported for full attention only");
  hipStream_t s = static_cast<hipStream_t>(hs);
  AttnDebug dbg;
  dbg.top = top_dev;
  dbg.topv = logit_dev;
  int32_t rc = forward_impl(L, x, B, T, pos_emb, pos_len, ctx, lens, nullptr, nullptr, dbg, s);
  if (rc) return rc;
  // the workspace holds [q | k | v] rows (bf16: v went to the transposed
  // buffer) and the projected position rows the kernel read
  const size_t es = esz(L), row = (size_t)L->D * es;
  const int64_t M = (int64_t)B * T;
  if (q_out) HIPCHK(hipMemcpy2DAsync(q_out, row, L->last_qkv, 3 * row, row, (size_t)M, hipMemcpyDeviceToDevice, s));
  if (k_out)
    HIPCHK(hipMemcpy2DAsync(k_out, row, L->last_qkv + row, 3 * row, row, (size_t)M, hipMemcpyDeviceToDevice, s));
  if (p_out) HIPCHK(hipMemcpyAsync(p_out, L->last_pos, (size_t)pos_len * row, hipMemcpyDeviceToDevice, s));
  HIPCHK(hipStreamSynchronize(s));
  return MHSA_OK;
}

}  // extern "C"
