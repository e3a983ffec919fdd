// Host runtime of the whole Conformer block and of the encoder's layer loops
// over blocks, composed from the sublayer entry points: ConformerBlock
// (conformer.rs:1613-2028) and the layer loops of ConformerEncoder::forward
// (conformer.rs:542-550) and ::forward_streaming (conformer.rs:949-1047).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <memory>
#include <string>
#include <vector>

#include "host_common.hpp"
#include "kernels.hpp"
#include "sublayers.hpp"

using mhsa::DType;

namespace {
constexpr float kNormEps = 1e-5f;  // nn::LayerNorm's default (conformer.rs:1684-1689)
constexpr int kNorms = 5;          // ff1, self_attn, conv, ff2, out
const char* const kNormNames[kNorms] = {"norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2",
                                        "norm_out"};
}  // namespace

struct mhsa_block {
  int D = 0, H = 0, F = 0, K = 0;
  bool causal = false;
  DType dt = mhsa::kF32;
  mhsa_ffn* ff1 = nullptr;
  mhsa_ffn* ff2 = nullptr;
  mhsa_layer* attn = nullptr;
  mhsa_conv* conv = nullptr;
  std::vector<float> nw[kNorms], nb[kNorms];  // LayerNorm weight / bias as loaded (fp32)
  DevBuf out_norm;                            // norm_out weight, bias in the block dtype's values
  std::vector<float> out_norm_host;           // what out_norm holds
  DevBuf work;                                // bf16 activations before a causal conv promotes them
  ~mhsa_block() {
    mhsa_ffn_destroy(ff1);
    mhsa_ffn_destroy(ff2);
    mhsa_destroy(attn);
    mhsa_conv_destroy(conv);
  }
};

struct mhsa_encoder {
  std::vector<mhsa_block*> blocks;        // not owned
  std::vector<mhsa_stack*> att;           // one attention ring per layer
  int B = 0, C = 0, T = 0, D = 0, KC = 0;  // KC: conv cache frames (K - 1)
  DevBuf conv_cache;                      // [layers, B, D, KC] fp32
  ~mhsa_encoder() {
    for (mhsa_stack* s : att) mhsa_stack_destroy(s);
  }
};

namespace {

int32_t check_block(const mhsa_block* k) { return k ? MHSA_OK : fail(MHSA_EINVAL, "null block handle"); }

// norm_out's parameters on the device, held at the block's parameter
// precision (set_dtype casts the norms, conformer.rs:1643-1660).
int32_t upload_out_norm(mhsa_block* k, const float** gd, const float** bd) {
  const bool bf = k->dt == mhsa::kBF16;
  std::vector<float> tmp(2 * k->D);
  for (int i = 0; i < k->D; ++i) {
    tmp[i] = bf ? round_bf16(k->nw[4][i]) : k->nw[4][i];
    tmp[k->D + i] = bf ? round_bf16(k->nb[4][i]) : k->nb[4][i];
  }
  if (tmp != k->out_norm_host) {
    if (k->out_norm.p) HIPCHK(hipDeviceSynchronize());  // an earlier launch may still read them
    HIPCHK(k->out_norm.ensure(tmp.size() * 4));
    HIPCHK(hipMemcpy(k->out_norm.p, tmp.data(), tmp.size() * 4, hipMemcpyHostToDevice));
    k->out_norm_host = tmp;
  }
  *gd = static_cast<const float*>(k->out_norm.p);
  *bd = *gd + k->D;
  return MHSA_OK;
}

// {prefix}.weight / .bias of one LayerNorm, each optional
// (load_layer_norm, loading.rs:203-214).
int32_t load_norm(const TensorMap& m, const std::string& prefix, int D, std::vector<float>& w,
                  std::vector<float>& b) {
  std::vector<float> nw = w, nb = b;
  for (int part = 0; part < 2; ++part) {
    const std::string key = prefix + (part ? ".bias" : ".weight");
    const mhsa_tensor* t = m.find(key);
    if (!t) continue;
    if (!float_dtype(t->dtype) || numel(t) != D) return fail(MHSA_EINVAL, "`%s`: expected float [%d]", key.c_str(), D);
    std::vector<float>& dst = part ? nb : nw;
    for (int i = 0; i < D; ++i) dst[i] = load_host(t->dtype, t->data, i);
  }
  w = std::move(nw);
  b = std::move(nb);
  return MHSA_OK;
}

int32_t block_forward(mhsa_block* k, void* x, int B, int T, const void* pos_emb, int pos_len,
                      const mhsa_context* ctx, const int32_t* lens, hipStream_t s) {
  if (!x || !pos_emb || B <= 0 || T <= 0) return fail(MHSA_EINVAL, "bad block arguments");
  if (k->causal && k->dt == mhsa::kBF16)
    return fail(MHSA_ENOTSUP, "a causal conv makes the rest of a bf16 block f32 (MLX promotion), which the bf16 "
                              "input cannot hold in place: call mhsa_block_forward_to");
  const int rows = B * T;
  // conformer.rs:1703-1729, 1747-1780, 1790-1814, 1827-1851, 1862
  if (int32_t rc = mhsa_ffn_sublayer_forward(k->ff1, x, rows, k->nw[0].data(), k->nb[0].data(), kNormEps, s))
    return rc;
  if (int32_t rc = mhsa_sublayer_forward(k->attn, x, B, T, k->nw[1].data(), k->nb[1].data(), kNormEps, pos_emb,
                                         pos_len, ctx, lens, s))
    return rc;
  if (int32_t rc = mhsa_conv_sublayer_forward(k->conv, x, B, T, nullptr, lens, k->nw[2].data(), k->nb[2].data(),
                                              kNormEps, s))
    return rc;
  if (int32_t rc = mhsa_ffn_sublayer_forward(k->ff2, x, rows, k->nw[3].data(), k->nb[3].data(), kNormEps, s))
    return rc;
  const float* gd;
  const float* bd;
  if (int32_t rc = upload_out_norm(k, &gd, &bd)) return rc;
  HIPCHK(mhsa::layer_norm(k->dt, x, x, gd, bd, kNormEps, rows, k->D, s));
  return MHSA_OK;
}

// The block's output dtype for activations stored in xdt: f32 once they are
// f32 or the conv is causal (its f32 zero padding, conformer.rs:2250-2256,
// promotes the depthwise conv and everything after it), else the block's.
DType block_out_dtype(const mhsa_block* k, DType xdt) {
  return xdt == mhsa::kF32 || k->causal ? mhsa::kF32 : k->dt;
}

// The block on activations made f32 before it (a bf16 block's ops then all
// run in f32 on the parameters' bf16 values), in place on x:
// conformer.rs:1703-1729, 1747-1780, 1790-1814, 1827-1851, 1862 as MLX
// promotes them.
int32_t block_forward_act32(mhsa_block* k, float* x, int B, int T, const void* pos_emb, int pos_len,
                            const mhsa_context* ctx, const int32_t* lens, hipStream_t s) {
  const int rows = B * T;
  if (int32_t rc = mhsa_ffn_sublayer_forward_f32(k->ff1, x, rows, k->nw[0].data(), k->nb[0].data(), kNormEps, s))
    return rc;
  if (int32_t rc = mhsa_sublayer_forward_act32(k->attn, x, B, T, k->nw[1].data(), k->nb[1].data(), kNormEps,
                                               pos_emb, pos_len, ctx, lens, s))
    return rc;
  if (int32_t rc = mhsa_conv_sublayer_to_f32(k->conv, x, mhsa::kF32, B, T, lens, k->nw[2].data(), k->nb[2].data(),
                                             kNormEps, x, s))
    return rc;
  if (int32_t rc = mhsa_ffn_sublayer_forward_f32(k->ff2, x, rows, k->nw[3].data(), k->nb[3].data(), kNormEps, s))
    return rc;
  const float* gd;
  const float* bd;
  if (int32_t rc = upload_out_norm(k, &gd, &bd)) return rc;
  HIPCHK(mhsa::layer_norm(mhsa::kF32, x, x, gd, bd, kNormEps, rows, k->D, s));
  return MHSA_OK;
}

// forward from x (stored in xdt) to out (in block_out_dtype): in place where
// the dtype holds, else through the block's bf16 copy of x up to the conv,
// whose sublayer writes the f32 sum to out.
int32_t block_forward_to(mhsa_block* k, const void* x, DType xdt, int B, int T, const void* pos_emb, int pos_len,
                         const mhsa_context* ctx, const int32_t* lens, void* out, hipStream_t s) {
  if (!x || !out || !pos_emb || B <= 0 || T <= 0) return fail(MHSA_EINVAL, "bad block arguments");
  if (!aligned16(x) || !aligned16(out)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  if (xdt != k->dt && xdt != mhsa::kF32)
    return fail(MHSA_EINVAL, "activations in dtype %d for a block of dtype %d", (int)xdt, (int)k->dt);
  const DType odt = block_out_dtype(k, xdt);
  const size_t in_bytes = (size_t)B * T * k->D * mhsa::dtype_size(xdt);
  const size_t out_bytes = (size_t)B * T * k->D * mhsa::dtype_size(odt);
  const char* xb = static_cast<const char*>(x);
  const char* ob = static_cast<const char*>(out);
  if (out != x && xb < ob + out_bytes && ob < xb + in_bytes)
    return fail(MHSA_EINVAL, "x and out must be the same buffer or not overlap");
  if (odt == xdt) {
    if (out != x) HIPCHK(hipMemcpyAsync(out, x, in_bytes, hipMemcpyDeviceToDevice, s));
    if (xdt == k->dt) return block_forward(k, out, B, T, pos_emb, pos_len, ctx, lens, s);
    return block_forward_act32(k, static_cast<float*>(out), B, T, pos_emb, pos_len, ctx, lens, s);
  }
  // bf16 activations into a causal bf16 block: bf16 up to the conv's padding
  if (out == x) return fail(MHSA_EINVAL, "the f32 output cannot overwrite its bf16 input (x and out must not overlap)");
  if (x != k->work.p) {  // (the encoder loop may have put them there)
    HIPCHK(k->work.ensure(align_up((int64_t)in_bytes, 256)));
    HIPCHK(hipMemcpyAsync(k->work.p, x, in_bytes, hipMemcpyDeviceToDevice, s));
  }
  const int rows = B * T;
  if (int32_t rc = mhsa_ffn_sublayer_forward(k->ff1, k->work.p, rows, k->nw[0].data(), k->nb[0].data(), kNormEps, s))
    return rc;
  if (int32_t rc = mhsa_sublayer_forward(k->attn, k->work.p, B, T, k->nw[1].data(), k->nb[1].data(), kNormEps,
                                         pos_emb, pos_len, ctx, lens, s))
    return rc;
  float* o = static_cast<float*>(out);
  if (int32_t rc = mhsa_conv_sublayer_to_f32(k->conv, k->work.p, xdt, B, T, lens, k->nw[2].data(), k->nb[2].data(),
                                             kNormEps, o, s))
    return rc;
  if (int32_t rc = mhsa_ffn_sublayer_forward_f32(k->ff2, o, rows, k->nw[3].data(), k->nb[3].data(), kNormEps, s))
    return rc;
  const float* gd;
  const float* bd;
  if (int32_t rc = upload_out_norm(k, &gd, &bd)) return rc;
  HIPCHK(mhsa::layer_norm(mhsa::kF32, o, o, gd, bd, kNormEps, rows, k->D, s));
  return MHSA_OK;
}

int32_t dtype_code(int32_t d, DType* out) {
  if (d == MHSA_F32) *out = mhsa::kF32;
  else if (d == MHSA_BF16) *out = mhsa::kBF16;
  else return fail(MHSA_EINVAL, "dtype %d is not f32 or bf16", d);
  return MHSA_OK;
}

}  // namespace

extern "C" {

int32_t mhsa_block_create(int32_t d_model, int32_t n_heads, int32_t ff_dim, int32_t conv_kernel, int32_t conv_norm,
                          int32_t causal, int32_t use_bias, mhsa_block** out) {
  if (!out) return fail(MHSA_EINVAL, "null output pointer");
  *out = nullptr;
  if (d_model > mhsa::kMaxLayerNormDim)
    return fail(MHSA_ENOTSUP, "the block's LayerNorms support d_model <= %d (got %d)", mhsa::kMaxLayerNormDim,
                d_model);
  std::unique_ptr<mhsa_block> k(new (std::nothrow) mhsa_block());
  if (!k) return fail(MHSA_ENOMEM, "out of host memory");
  if (int32_t rc = mhsa_ffn_create(d_model, ff_dim, use_bias, &k->ff1)) return rc;
  if (int32_t rc = mhsa_ffn_create(d_model, ff_dim, use_bias, &k->ff2)) return rc;
  if (int32_t rc = mhsa_create(d_model, n_heads, use_bias, &k->attn)) return rc;
  if (int32_t rc = mhsa_conv_create(d_model, conv_kernel, conv_norm, causal, use_bias, &k->conv)) return rc;
  k->D = d_model;
  k->H = n_heads;
  k->F = ff_dim;
  k->K = conv_kernel;
  k->causal = causal != 0;
  for (int i = 0; i < kNorms; ++i) {  // nn::LayerNorm::new: weight 1, bias 0
    k->nw[i].assign(d_model, 1.f);
    k->nb[i].assign(d_model, 0.f);
  }
  *out = k.release();
  return MHSA_OK;
}

void mhsa_block_destroy(mhsa_block* k) { delete k; }

int32_t mhsa_block_set_dtype(mhsa_block* k, int32_t dtype) {
  if (int32_t rc = check_block(k)) return rc;
  if (dtype != MHSA_F32 && dtype != MHSA_BF16) return fail(MHSA_ENOTSUP, "dtype %d not supported (f32, bf16)", dtype);
  for (int32_t rc : {mhsa_ffn_set_dtype(k->ff1, dtype), mhsa_ffn_set_dtype(k->ff2, dtype),
                     mhsa_set_dtype(k->attn, dtype), mhsa_conv_set_dtype(k->conv, dtype)})
    if (rc) return rc;
  k->dt = dtype == MHSA_F32 ? mhsa::kF32 : mhsa::kBF16;
  return MHSA_OK;
}

int32_t mhsa_block_load_weights(mhsa_block* k, const mhsa_tensor* tensors, int32_t n, const char* prefix,
                                int32_t strict, int32_t quant_bits, int32_t quant_group) {
  if (int32_t rc = check_block(k)) return rc;
  if ((n > 0 && !tensors) || !prefix) return fail(MHSA_EINVAL, "null tensor list or prefix");
  const std::string p(prefix);
  // The norms are parsed first and stored last; a failure in a module
  // leaves the modules before it loaded, as the reference's sequential
  // load_weights does.
  std::vector<float> nw[kNorms], nb[kNorms];
  const TensorMap m{tensors, n};
  for (int i = 0; i < kNorms; ++i) {
    nw[i] = k->nw[i];
    nb[i] = k->nb[i];
    if (int32_t rc = load_norm(m, p + "." + kNormNames[i], k->D, nw[i], nb[i])) return rc;
  }
  // ConformerBlock::load_weights (conformer.rs:1977-2028)
  if (int32_t rc = mhsa_ffn_load_weights(k->ff1, tensors, n, (p + ".feed_forward1").c_str(), strict, quant_bits,
                                         quant_group))
    return rc;
  if (int32_t rc = mhsa_load_weights(k->attn, tensors, n, (p + ".self_attn").c_str(), strict, quant_bits,
                                     quant_group))
    return rc;
  if (int32_t rc = mhsa_conv_load_weights(k->conv, tensors, n, (p + ".conv").c_str(), strict, quant_bits,
                                          quant_group))
    return rc;
  if (int32_t rc = mhsa_ffn_load_weights(k->ff2, tensors, n, (p + ".feed_forward2").c_str(), strict, quant_bits,
                                         quant_group))
    return rc;
  for (int i = 0; i < kNorms; ++i) {
    k->nw[i] = std::move(nw[i]);
    k->nb[i] = std::move(nb[i]);
  }
  return MHSA_OK;
}

mhsa_layer* mhsa_block_attention(mhsa_block* k) { return k ? k->attn : nullptr; }
mhsa_ffn* mhsa_block_feed_forward(mhsa_block* k, int32_t which) {
  return k && (which == 1 || which == 2) ? (which == 1 ? k->ff1 : k->ff2) : nullptr;
}
mhsa_conv* mhsa_block_conv(mhsa_block* k) { return k ? k->conv : nullptr; }

int32_t mhsa_block_forward(mhsa_block* k, void* x, int32_t batch, int32_t seq_len, const void* pos_emb,
                           int32_t pos_len, const mhsa_context* ctx, const int32_t* lengths, void* hs) {
  if (int32_t rc = check_block(k)) return rc;
  return block_forward(k, x, batch, seq_len, pos_emb, pos_len, ctx, lengths, static_cast<hipStream_t>(hs));
}

int32_t mhsa_encoder_forward(mhsa_block* const* blocks, int32_t n_layers, void* x, int32_t batch, int32_t seq_len,
                             const void* pos_emb, int32_t pos_len, const mhsa_context* ctx, const int32_t* lengths,
                             void* hs) {
  if (!blocks || n_layers <= 0) return fail(MHSA_EINVAL, "null or empty block list");
  for (int l = 0; l < n_layers; ++l) {
    if (!blocks[l]) return fail(MHSA_EINVAL, "block %d is null", l);
    if (blocks[l]->D != blocks[0]->D || blocks[l]->dt != blocks[0]->dt)
      return fail(MHSA_EINVAL, "block %d differs from block 0 in d_model or dtype", l);
  }
  // one pos_emb, context and padding for every layer (conformer.rs:542-550)
  for (int l = 0; l < n_layers; ++l)
    if (int32_t rc = block_forward(blocks[l], x, batch, seq_len, pos_emb, pos_len, ctx, lengths,
                                   static_cast<hipStream_t>(hs)))
      return rc;
  return MHSA_OK;
}

int32_t mhsa_block_output_dtype(const mhsa_block* k, int32_t x_dtype) {
  DType xdt;
  if (!k || (x_dtype != MHSA_F32 && x_dtype != MHSA_BF16)) return -1;
  xdt = x_dtype == MHSA_F32 ? mhsa::kF32 : mhsa::kBF16;
  if (xdt != k->dt && xdt != mhsa::kF32) return -1;
  return block_out_dtype(k, xdt) == mhsa::kF32 ? MHSA_F32 : MHSA_BF16;
}

int32_t mhsa_block_forward_to(mhsa_block* k, const void* x, int32_t x_dtype, int32_t batch, int32_t seq_len,
                              const void* pos_emb, int32_t pos_len, const mhsa_context* ctx, const int32_t* lengths,
                              void* out, void* hs) {
  if (int32_t rc = check_block(k)) return rc;
  DType xdt;
  if (int32_t rc = dtype_code(x_dtype, &xdt)) return rc;
  return block_forward_to(k, x, xdt, batch, seq_len, pos_emb, pos_len, ctx, lengths, out,
                          static_cast<hipStream_t>(hs));
}

int32_t mhsa_encoder_forward_to(mhsa_block* const* blocks, int32_t n_layers, const void* x, int32_t x_dtype,
                                int32_t batch, int32_t seq_len, const void* pos_emb, int32_t pos_len,
                                const mhsa_context* ctx, const int32_t* lengths, void* out, void* hs) {
  if (!blocks || n_layers <= 0) return fail(MHSA_EINVAL, "null or empty block list");
  DType xdt;
  if (int32_t rc = dtype_code(x_dtype, &xdt)) return rc;
  // every block checked, and the activations' dtype followed through the
  // stack, before the first launch
  DType dt = xdt;
  for (int l = 0; l < n_layers; ++l) {
    if (!blocks[l]) return fail(MHSA_EINVAL, "block %d is null", l);
    if (blocks[l]->D != blocks[0]->D || blocks[l]->dt != blocks[0]->dt)
      return fail(MHSA_EINVAL, "block %d differs from block 0 in d_model or dtype", l);
    if (dt != blocks[l]->dt && dt != mhsa::kF32)
      return fail(MHSA_EINVAL, "activations in dtype %d for a block of dtype %d", (int)dt, (int)blocks[l]->dt);
    dt = block_out_dtype(blocks[l], dt);
  }
  // one pos_emb, context and padding for every layer (conformer.rs:542-550):
  // the first block moves x to out, the others run on out
  hipStream_t s = static_cast<hipStream_t>(hs);
  if (int32_t rc = block_forward_to(blocks[0], x, xdt, batch, seq_len, pos_emb, pos_len, ctx, lengths, out, s))
    return rc;
  dt = block_out_dtype(blocks[0], xdt);
  for (int l = 1; l < n_layers; ++l) {
    const DType odt = block_out_dtype(blocks[l], dt);
    if (odt != dt) {
      // bf16 activations turning f32 here: out cannot hold both, so they
      // move to the block's own bf16 copy (block_forward_to copies them)
      // and the f32 result lands in out
      const size_t bytes = (size_t)batch * seq_len * blocks[l]->D * 2;
      HIPCHK(blocks[l]->work.ensure(align_up((int64_t)bytes, 256)));
      HIPCHK(hipMemcpyAsync(blocks[l]->work.p, out, bytes, hipMemcpyDeviceToDevice, s));
      if (int32_t rc = block_forward_to(blocks[l], blocks[l]->work.p, dt, batch, seq_len, pos_emb, pos_len, ctx,
                                        lengths, out, s))
        return rc;
    } else if (int32_t rc = block_forward_to(blocks[l], out, dt, batch, seq_len, pos_emb, pos_len, ctx, lengths,
                                             out, s)) {
      return rc;
    }
    dt = odt;
  }
  return MHSA_OK;
}

int32_t mhsa_encoder_create(mhsa_block* const* blocks, int32_t n_layers, int32_t batch, int32_t cache_size,
                            int32_t chunk_len, mhsa_encoder** out) {
  if (!out) return fail(MHSA_EINVAL, "null output pointer");
  *out = nullptr;
  if (!blocks || n_layers <= 0) return fail(MHSA_EINVAL, "null or empty block list");
  // every block checked before anything is allocated
  for (int l = 0; l < n_layers; ++l) {
    mhsa_block* k = blocks[l];
    if (!k) return fail(MHSA_EINVAL, "block %d is null", l);  // (block 0 first)
    if (k->D != blocks[0]->D || k->K != blocks[0]->K)
      return fail(MHSA_EINVAL, "block %d differs from block 0 in d_model or conv kernel size", l);
    if (!k->causal || k->K < 2)
      return fail(MHSA_EINVAL, "block %d: the streaming conv cache needs a causal convolution of kernel size >= 2", l);
    for (int j = 0; j < l; ++j)
      if (blocks[j] == k) return fail(MHSA_EINVAL, "block %d appears twice", l);
  }
  if (batch <= 0 || cache_size < 0 || chunk_len <= 0)
    return fail(MHSA_EINVAL, "bad encoder shape: batch %d, cache_size %d, chunk_len %d", batch, cache_size, chunk_len);
  std::unique_ptr<mhsa_encoder> e(new (std::nothrow) mhsa_encoder());
  if (!e) return fail(MHSA_ENOMEM, "out of host memory");
  for (int l = 0; l < n_layers; ++l) {
    mhsa_block* k = blocks[l];
    mhsa_stack* st = nullptr;
    if (int32_t rc = mhsa_stack_create(&k->attn, 1, batch, cache_size, chunk_len, &st)) return rc;
    e->att.push_back(st);
    e->blocks.push_back(k);
  }
  e->B = batch;
  e->C = cache_size;
  e->T = chunk_len;
  e->D = blocks[0]->D;
  e->KC = blocks[0]->K - 1;
  // cache_last_time starts at zeros (streaming/core.rs:151-157)
  const size_t bytes = (size_t)n_layers * batch * e->D * e->KC * 4;
  {
    HIPCHK(e->conv_cache.ensure(bytes));
    HIPCHK(mhsa::fill_zero(e->conv_cache.p, bytes, nullptr));
    HIPCHK(hipStreamSynchronize(nullptr));
  }
  *out = e.release();
  return MHSA_OK;
}

void mhsa_encoder_destroy(mhsa_encoder* e) { delete e; }

int32_t mhsa_encoder_load_cache(mhsa_encoder* e, const float* channel, const float* time, const int32_t* filled,
                                void* hs) {
  if (!e || !channel) return fail(MHSA_EINVAL, "null argument");
  const size_t per = (size_t)e->B * e->C * e->D;
  for (size_t l = 0; l < e->att.size(); ++l)
    if (int32_t rc = mhsa_stack_load_cache(e->att[l], channel + l * per, filled, hs)) return rc;
  const size_t bytes = e->att.size() * (size_t)e->B * e->D * e->KC * 4;
  {
    hipStream_t s = static_cast<hipStream_t>(hs);
    if (time) HIPCHK(hipMemcpyAsync(e->conv_cache.p, time, bytes, hipMemcpyDeviceToDevice, s));
    else HIPCHK(mhsa::fill_zero(e->conv_cache.p, bytes, s));
  }
  return MHSA_OK;
}

int32_t mhsa_encoder_read_cache(const mhsa_encoder* e, float* channel, float* time, void* hs) {
  if (!e || !channel) return fail(MHSA_EINVAL, "null argument");
  const size_t per = (size_t)e->B * e->C * e->D;
  for (size_t l = 0; l < e->att.size(); ++l)
    if (int32_t rc = mhsa_stack_read_cache(e->att[l], channel + l * per, hs)) return rc;
  const size_t bytes = e->att.size() * (size_t)e->B * e->D * e->KC * 4;
  if (time) {
    hipStream_t s = static_cast<hipStream_t>(hs);
    HIPCHK(hipMemcpyAsync(time, e->conv_cache.p, bytes, hipMemcpyDeviceToDevice, s));
    HIPCHK(hipStreamSynchronize(s));
  }
  return MHSA_OK;
}

int32_t mhsa_encoder_fill(const mhsa_encoder* e, int32_t* filled) {
  if (!e || !filled) return fail(MHSA_EINVAL, "null argument");
  return mhsa_stack_fill(e->att[0], filled);
}

int32_t mhsa_encoder_step(mhsa_encoder* e, float* x, const void* pos_emb, int32_t pos_len,
                          const mhsa_stream_mask* mask, const int32_t* valid, void* hs) {
  if (!e || !x || !pos_emb) return fail(MHSA_EINVAL, "null argument");
  if (!aligned16(x)) return fail(MHSA_EINVAL, "device tensors must be 16-byte aligned");
  const int rows = e->B * e->T;
  // every layer reads the fills of the step's start (conformer.rs:883-887
  // reads them once per chunk); each layer's ring then moves its own copy
  std::vector<int32_t> fills(e->B);
  if (int32_t rc = mhsa_stack_fill(e->att[0], fills.data())) return rc;
  mhsa_stream_mask m;
  if (mask && mask->present) {
    m = *mask;
    if (!m.filled_host) m.filled_host = fills.data();
    mask = &m;
  }
  for (size_t l = 0; l < e->blocks.size(); ++l) {
    mhsa_block* k = e->blocks[l];
    float* cache = static_cast<float*>(e->conv_cache.p) + l * (size_t)e->B * e->D * e->KC;
    // ConformerBlock::forward_with_cache (conformer.rs:1893-1971) on the f32
    // streaming activations
    if (int32_t rc = mhsa_ffn_sublayer_forward_f32(k->ff1, x, rows, k->nw[0].data(), k->nb[0].data(), kNormEps, hs))
      return rc;
    if (int32_t rc = mhsa_stack_step(e->att[l], x, k->nw[1].data(), k->nb[1].data(), kNormEps, pos_emb, pos_len,
                                     mask, hs))
      return rc;
    if (int32_t rc = mhsa_conv_sublayer_forward(k->conv, x, e->B, e->T, cache, valid, k->nw[2].data(),
                                                k->nb[2].data(), kNormEps, hs))
      return rc;
    if (int32_t rc = mhsa_ffn_sublayer_forward_f32(k->ff2, x, rows, k->nw[3].data(), k->nb[3].data(), kNormEps, hs))
      return rc;
    const float* gd;
    const float* bd;
    if (int32_t rc = upload_out_norm(k, &gd, &bd)) return rc;
    HIPCHK(mhsa::layer_norm(mhsa::kF32, x, x, gd, bd, kNormEps, rows, e->D, static_cast<hipStream_t>(hs)));
  }
  return MHSA_OK;
}

}  // extern "C"
