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
                              "input cannot hold in place");
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
