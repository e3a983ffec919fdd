/*
 * relpos_mhsa.h - C ABI of the MI355X (gfx950) FastConformer rel-pos MHSA path.
 *
 * Drop-in boundary for the attention sublayer of animaslabs/mlx-nemo-rs
 * (crate mlx-voice 0.3.0). Each entry point names the reference interface it
 * replaces (paths relative to the reference repository):
 *
 *   RelPositionMultiHeadAttention   src/asr/modules/encoders/attention.rs:328-893
 *   RelPositionalEncoding           src/asr/modules/encoders/attention.rs:19-194
 *   AttentionContext                src/asr/modules/encoders/attention.rs:208-273
 *   key_padding_mask                src/asr/modules/encoders/attention.rs:275-294
 *   LinearLayer / QuantizationConfig src/core/quantization.rs:17-162, 289-349
 *   streaming mask + cache          src/asr/modules/encoders/conformer.rs:97-323, 840-1047
 *   MHSA sublayer (pre-LN+residual) src/asr/modules/encoders/conformer.rs:1747-1780
 *
 * Conventions
 *  - Plain C types only. Activations, caches and outputs are DEVICE pointers
 *    owned by the caller, in the layer's dtype (fp32 or bf16), row-major,
 *    16-byte aligned. Weights are passed as HOST pointers and uploaded into a
 *    kernel-native layout owned by the layer handle.
 *  - Lengths and fill levels are HOST arrays, as in the reference
 *    (conformer.rs:852-857), so no call waits on the GPU.
 *  - Calls are asynchronous on the given HIP stream (hipStream_t passed as
 *    void*; NULL = the null stream). Weight uploads and debug exports are
 *    synchronous.
 *  - A handle is not reentrant (the reference takes &mut self,
 *    attention.rs:446, 606); different handles may be used from different
 *    threads.
 *  - Every function returns a status; on failure mhsa_last_error() gives a
 *    thread-local message. No exceptions or aborts cross the ABI.
 */
#ifndef RELPOS_MHSA_H
#define RELPOS_MHSA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes (reference: Result<T, Error>, src/core/error.rs:7-12) */
#define MHSA_OK 0
#define MHSA_ENOMEM 12
#define MHSA_EINVAL 22       /* bad shape / argument (Error::Model, MLX shape errors) */
#define MHSA_ENOTSUP 95      /* unsupported mode (e.g. bits != 8, group != 64) */
#define MHSA_ENOENT 2        /* strict load: a tensor is missing (loading.rs:107-116) */
#define MHSA_EHIP 1000       /* HIP runtime error; the message names it */

/* dtypes (mlx_rs::Dtype subset) */
#define MHSA_F32 0
#define MHSA_BF16 1
#define MHSA_F16 2
#define MHSA_U32 3

/* projections of one layer (attention.rs:333-342) */
#define MHSA_LINEAR_Q 0
#define MHSA_LINEAR_K 1
#define MHSA_LINEAR_V 2
#define MHSA_LINEAR_OUT 3
#define MHSA_LINEAR_POS 4

typedef struct mhsa_layer mhsa_layer;
typedef struct mhsa_stream mhsa_stream;

/* AttentionContext (attention.rs:211-227): left/right context in frames,
 * -1 = unlimited; chunked = 1 for the "chunked_limited" style. A context with
 * left < 0 and right < 0 means full attention (AttentionContext::new -> None). */
typedef struct {
  int32_t left;
  int32_t right;
  int32_t chunked;
} mhsa_context;

/* Streaming attention mask, built in-kernel from the parameters
 * create_attention_mask takes (conformer.rs:97-221):
 *  present      0 = the encoder has no att_context_size: no mask at all
 *  ctx          att_context_size and style
 *  filled_host  [B] cache fill per session (NULL = the stream's own count);
 *               the reference uses session 0's fill for every session
 *               (conformer.rs:883-887), this is the per-session superset
 *  valid_host   [B] valid query rows per session (NULL = all); rows past it
 *               see no key and yield zeros, as the reference's bool path */
typedef struct {
  int32_t present;
  mhsa_context ctx;
  const int32_t* filled_host;
  const int32_t* valid_host;
} mhsa_stream_mask;

/* Named host tensor for mhsa_load_weights (the Weights map, loading.rs:81). */
typedef struct {
  const char* name;
  int32_t dtype;     /* MHSA_F32 / MHSA_BF16 / MHSA_F16 / MHSA_U32 */
  int32_t ndim;
  int64_t shape[4];
  const void* data;  /* host pointer, row-major */
} mhsa_tensor;

/* ---- errors / library -------------------------------------------------- */

/* Thread-local message of the last failing call (error.rs Display). */
const char* mhsa_last_error(void);
/* ABI version (major * 100 + minor). */
int32_t mhsa_version(void);

/* ---- layer lifecycle ---------------------------------------------------- */

/* RelPositionMultiHeadAttention::new(d_model, n_heads, use_bias)
 * (attention.rs:367-406). Weights start at zero, dtype fp32. Kernels support
 * head_dim 64 or 128 and d_model a multiple of 128. */
int32_t mhsa_create(int32_t d_model, int32_t n_heads, int32_t use_bias, mhsa_layer** out);
void mhsa_destroy(mhsa_layer* layer);
/* set_dtype (attention.rs:409-423): MHSA_F32 or MHSA_BF16. Drops the
 * streaming position memo, as the reference does (attention.rs:421). */
int32_t mhsa_set_dtype(mhsa_layer* layer, int32_t dtype);
int32_t mhsa_get_dtype(const mhsa_layer* layer);
/* head_dim(), n_heads() (attention.rs:426-433) */
int32_t mhsa_head_dim(const mhsa_layer* layer);
int32_t mhsa_n_heads(const mhsa_layer* layer);
int32_t mhsa_d_model(const mhsa_layer* layer);
/* pub cache_drop_size (attention.rs:349-350), set by setup_streaming
 * (conformer.rs:812-817) */
int32_t mhsa_set_cache_drop_size(mhsa_layer* layer, int32_t cache_drop_size);

/* ---- weights ------------------------------------------------------------ */

/* LinearLayer::standard(weight [out,in], bias [out] | NULL)
 * (quantization.rs:62-65). data_dtype: MHSA_F32 / MHSA_BF16 / MHSA_F16.
 * linear_pos never takes a bias (attention.rs:385). */
int32_t mhsa_load_linear_standard(mhsa_layer* layer, int32_t which, int32_t data_dtype, const void* weight,
                                  const void* bias);
/* LinearLayer::quantized (quantization.rs:67-82): MLX affine layout
 * weight u32 [out, in*bits/32], scales and biases f16 [out, in/group],
 * bias f16 [out] | NULL. Only bits = 8, group_size = 64 are supported
 * (the reference's default, quantization.rs:307). */
int32_t mhsa_load_linear_quantized(mhsa_layer* layer, int32_t which, const uint32_t* weight,
                                   const uint16_t* scales_f16, const uint16_t* biases_f16,
                                   const uint16_t* bias_f16, int32_t bits, int32_t group_size);
/* pos_bias_u / pos_bias_v [n_heads, head_dim] (attention.rs:344-347, 388-389). */
int32_t mhsa_load_pos_bias(mhsa_layer* layer, int32_t data_dtype, const void* pos_bias_u, const void* pos_bias_v);
/* load_weights(weights, prefix, quant) (attention.rs:863-893): resolves
 * {prefix}.linear_{q,k,v,out,pos}.{weight,bias,scales,biases} and
 * {prefix}.pos_bias_{u,v}; a layer is quantized iff .scales and .biases exist
 * (quantization.rs:299-304), with (quant_bits, quant_group) or (8, 64) when
 * quant_bits <= 0 (quantization.rs:307). strict != 0 fails with MHSA_ENOENT on
 * the first missing tensor (loading.rs:107-116); otherwise missing tensors
 * keep their values. */
int32_t mhsa_load_weights(mhsa_layer* layer, const mhsa_tensor* tensors, int32_t n_tensors, const char* prefix,
                          int32_t strict, int32_t quant_bits, int32_t quant_group);

/* ---- checkpoints ---------------------------------------------------------- */

/* CheckpointLoader (checkpoint.rs:480-760) over an MLX safetensors file:
 * `path` is the .safetensors file or a directory holding model.safetensors,
 * weights.safetensors, model_weights.safetensors or weights/model.safetensors
 * (checkpoint.rs:694-731). The quantization comes from the directory's
 * config.yaml / model_config.yaml / config.json / model_config.json, else
 * config.json ("quantization": {"bits", "group_size"}, defaults 8 and 64,
 * checkpoint.rs:535-572, 613-621); for a file path, from config.json beside
 * it. The file is memory-mapped; tensors of dtype F32, F16, BF16 and U32 are
 * listed (the dtypes the path reads), others are skipped. */
typedef struct mhsa_checkpoint mhsa_checkpoint;
int32_t mhsa_checkpoint_open(const char* path, mhsa_checkpoint** out);
void mhsa_checkpoint_close(mhsa_checkpoint* ckpt);
/* quantization() (checkpoint.rs:682-690): bits and group size, 0 and 0 when
 * the checkpoint is not quantized. */
int32_t mhsa_checkpoint_quantization(const mhsa_checkpoint* ckpt, int32_t* bits, int32_t* group_size);
/* The tensor map (Array::load_safetensors, weights.rs:207-237): count, and
 * entry idx with its name, dtype, shape and a host pointer into the mapping
 * (valid until mhsa_checkpoint_close). */
int32_t mhsa_checkpoint_count(const mhsa_checkpoint* ckpt);
int32_t mhsa_checkpoint_tensor(const mhsa_checkpoint* ckpt, int32_t idx, mhsa_tensor* out);
/* __metadata__ value for `key` (NULL when absent), e.g. "format" = "mlx"
 * (WeightFormat::from_safetensors_metadata, weights.rs:27-35). */
int32_t mhsa_checkpoint_metadata(const mhsa_checkpoint* ckpt, const char* key, const char** value);
/* load_weights(&weights, prefix, quant) (attention.rs:863-893) from the
 * checkpoint's tensors with its quantization: mhsa_load_weights over the
 * mapped tensors. */
int32_t mhsa_load_weights_from_checkpoint(mhsa_layer* layer, const mhsa_checkpoint* ckpt, const char* prefix,
                                          int32_t strict);

/* ---- offline forward ---------------------------------------------------- */

/* forward(x, pos_emb, context, key_mask) (attention.rs:446-573).
 *  x        [batch, seq_len, d_model] device, layer dtype
 *  pos_emb  [pos_len, d_model] device, layer dtype: the table
 *           get_encoding(seq_len) gives (pos_len = 2*seq_len-1), or a centred
 *           band of 2W+1 rows (distances W..-W) when `context` hides every
 *           pair farther apart than W (a local window)
 *  ctx      NULL = full attention
 *  key_lengths_host [batch] valid frames per item (key_padding_mask,
 *           attention.rs:280-294; values clamped to >= 1), NULL = no padding
 *  out      [batch, seq_len, d_model] device, layer dtype
 * Only the position rows the context can reach are projected. */
int32_t mhsa_forward(mhsa_layer* layer, const void* x, int32_t batch, int32_t seq_len, const void* pos_emb,
                     int32_t pos_len, const mhsa_context* ctx, const int32_t* key_lengths_host, void* out,
                     void* hip_stream);

/* No counterpart in the reference. mhsa_forward for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): same arguments and results, but every
 * intermediate lives in a fixed 128 MiB device array of the library (16 MiB
 * of split-K partials, 112 MiB of workspace), one per GPU, held until the
 * process ends; it calls no hipMalloc or hipFree. Inputs needing more
 * workspace fail with MHSA_EINVAL (the message gives the bytes needed: about
 * 10 * d_model bytes per frame (batch * seq_len) plus 4 * d_model per position
 * row in bf16, 16 and 8 in fp32; at the 0.6B shape, batch 8 x 375 frames
 * needs 33 MB and batch 4 x 1500 needs 67 MB). The layer's parameters must
 * already be on the device (uploading allocates): after loading weights or
 * changing the dtype, run mhsa_forward once. All calls on one GPU share the
 * array, so calls that overlap on one GPU (different streams or threads)
 * race; serialise them. */
int32_t mhsa_forward_noalloc(mhsa_layer* layer, const void* x, int32_t batch, int32_t seq_len, const void* pos_emb,
                             int32_t pos_len, const mhsa_context* ctx, const int32_t* key_lengths_host, void* out,
                             void* hip_stream);

/* x <- x + forward(LayerNorm(x)) : the MHSA sublayer of ConformerBlock
 * (conformer.rs:1747-1780). ln_gamma / ln_beta [d_model] HOST fp32 arrays
 * (NULL = 1 / 0), eps as nn::LayerNorm (1e-5); d_model <= 2048. */
int32_t mhsa_sublayer_forward(mhsa_layer* layer, void* x_inout, int32_t batch, int32_t seq_len,
                              const float* ln_gamma_host, const float* ln_beta_host, float eps,
                              const void* pos_emb, int32_t pos_len, const mhsa_context* ctx,
                              const int32_t* key_lengths_host, void* hip_stream);

/* The offline encoder's layer loop over the MHSA sublayers
 * (conformer.rs:542-550: one pos_emb, context and padding mask for every
 * layer): x <- x + forward_l(LayerNorm_l(x)) for l = 0 .. n_layers - 1, with
 * the results of n_layers mhsa_sublayer_forward calls in order, bit for bit.
 * ln_gamma_host / ln_beta_host: HOST fp32 [n_layers, d_model] (NULL = 1 / 0),
 * as mhsa_stack_step takes them. Every layer has the same d_model and dtype.
 * Layer l + 1's position projection does not depend on layer l, so where the
 * bf16 attention leaves CUs idle it runs in the same launch as layer l's
 * attention. */
int32_t mhsa_stack_sublayer_forward(mhsa_layer* const* layers, int32_t n_layers, void* x_inout, int32_t batch,
                                    int32_t seq_len, const float* ln_gamma_host, const float* ln_beta_host,
                                    float eps, const void* pos_emb,
                                    int32_t pos_len, const mhsa_context* ctx, const int32_t* key_lengths_host,
                                    void* hip_stream);

/* ---- cache-aware streaming ---------------------------------------------- */

/* Streaming state of one layer for `batch` sessions: the attention cache of
 * `cache_size` frames (EncoderCache::last_channel slice, streaming/core.rs:
 * 117-166) kept as an HBM ring of C + chunk_len rows holding the cached
 * normalised inputs h and their projected K and V, plus each session's
 * fill. Zero-filled at creation, like EncoderCache::new. The cache is fp32
 * for both layer dtypes, as the reference keeps it (conformer.rs:422-434). */
int32_t mhsa_stream_create(mhsa_layer* layer, int32_t batch, int32_t cache_size, int32_t chunk_len,
                           mhsa_stream** out);
void mhsa_stream_destroy(mhsa_stream* stream);
/* Replace the cache with `cache` [batch, cache_size, d_model] (device, fp32,
 * oldest frame first) and set the fill levels (filled_host [batch], NULL = 0).
 * K/V of the cached rows are projected here. */
int32_t mhsa_stream_load_cache(mhsa_stream* stream, const void* cache, const int32_t* filled_host,
                               void* hip_stream);
/* Copy the cache out in the reference layout [batch, cache_size, d_model]. */
int32_t mhsa_stream_read_cache(const mhsa_stream* stream, void* cache_out, void* hip_stream);
/* Current fill level of each session [batch] (host). */
int32_t mhsa_stream_fill(const mhsa_stream* stream, int32_t* filled_out_host);

/* forward_with_cache(x, pos_emb, cache, _, att_mask) (attention.rs:606-816)
 * followed by the encoder's cache pad/truncate and fill update
 * (conformer.rs:983-999, 1025-1036).
 *  x       [batch, chunk_len, d_model] device fp32 (the normalised input h)
 *  pos_emb [2*(cache_size+chunk_len)-1, d_model] device, layer dtype; its
 *          projection is memoised per pos_len as the reference does
 *          (attention.rs:749-761)
 *  mask    NULL = no mask (att_context_size absent)
 *  out     [batch, chunk_len, d_model] device fp32
 * Activations are fp32 for both layer dtypes: with an f32 cache the
 * reference's [cache; x] and everything derived from it are f32 (MLX
 * promotes the bf16 parameters), and the streamed features are never cast to
 * the layer dtype (conformer.rs:845-849); a bf16 layer contributes its bf16
 * parameter values and bf16 position rows.
 * Afterwards the cache holds [cache[q_keep:]; x[:q_keep]] (q_keep =
 * chunk_len - cache_drop_size) and fill = min(fill + q_keep, cache_size). */
int32_t mhsa_forward_with_cache(mhsa_layer* layer, mhsa_stream* stream, const void* x, const void* pos_emb,
                                int32_t pos_len, const mhsa_stream_mask* mask, void* out, void* hip_stream);
/* forward_with_cache(x, pos_emb, None, _, att_mask): the no-cache path
 * (attention.rs:687-700), keys and values from x alone (total_len =
 * seq_len). Same dtypes as mhsa_forward_with_cache; pos_emb has
 * 2*seq_len-1 rows; the mask's fill levels do not apply (there is no cache).
 * The reference's returned cache is x[:, :seq_len - cache_drop_size], a slice
 * of the caller's own input. */
int32_t mhsa_forward_uncached(mhsa_layer* layer, const void* x, int32_t batch, int32_t seq_len, const void* pos_emb,
                              int32_t pos_len, const mhsa_stream_mask* mask, void* out, void* hip_stream);

/* ---- FeedForward (the rest of the Conformer block's GEMM work) ------------- */

/* FeedForward (conformer.rs:2031-2088): out = linear2(silu(linear1(x))),
 * linear1 [ff_dim, d_model], linear2 [d_model, ff_dim], each standard or MLX
 * affine 8-bit (group 64), with biases when use_bias. The projections run
 * on the same GEMM kernels as the attention projections (fused in-register
 * dequantisation), linear1 with a SiLU epilogue that stores sigmoid and the
 * product in the dtype as nn::silu does. d_model, ff_dim multiples of 64. */
typedef struct mhsa_ffn mhsa_ffn;
int32_t mhsa_ffn_create(int32_t d_model, int32_t ff_dim, int32_t use_bias, mhsa_ffn** out);
void mhsa_ffn_destroy(mhsa_ffn* ffn);
/* set_dtype (conformer.rs:2040-2043): MHSA_F32 or MHSA_BF16. */
int32_t mhsa_ffn_set_dtype(mhsa_ffn* ffn, int32_t dtype);
/* load_weights (conformer.rs:2074-2087): {prefix}.linear1 / .linear2 with
 * .weight, .bias, .scales, .biases as mhsa_load_weights resolves them
 * (prefix e.g. "encoder.layers.0.feed_forward1"). */
int32_t mhsa_ffn_load_weights(mhsa_ffn* ffn, const mhsa_tensor* tensors, int32_t n_tensors, const char* prefix,
                              int32_t strict, int32_t quant_bits, int32_t quant_group);
/* forward (conformer.rs:2066-2072): x, out [rows, d_model] device, dtype. */
int32_t mhsa_ffn_forward(mhsa_ffn* ffn, const void* x, int32_t rows, void* out, void* hip_stream);
/* The block's half-step sublayer x <- x + 0.5 * forward(LayerNorm(x))
 * (conformer.rs:1703-1729, 1827-1851); gamma/beta [d_model] host fp32 or
 * NULL, eps as nn::LayerNorm; the residual is fused into linear2's epilogue. */
int32_t mhsa_ffn_sublayer_forward(mhsa_ffn* ffn, void* x_inout, int32_t rows, const float* ln_gamma_host,
                                  const float* ln_beta_host, float eps, void* hip_stream);
/* The same two on f32 activations with the module's parameters (the streaming
 * path's form: its activations derive from the f32 caches, so in a bf16
 * model MLX promotes every op they meet to f32, conformer.rs:1914-1919,
 * 1956-1960; quantized weights dequantise in f32 from their cast scales).
 * x, out, x_inout f32. */
int32_t mhsa_ffn_forward_f32(mhsa_ffn* ffn, const float* x, int32_t rows, float* out, void* hip_stream);
int32_t mhsa_ffn_sublayer_forward_f32(mhsa_ffn* ffn, float* x_inout, int32_t rows, const float* ln_gamma_host,
                                      const float* ln_beta_host, float eps, void* hip_stream);
/* Per-kernel HIP-event timing of the module's launches, as mhsa_profile_*
 * does for a layer (tags linear1, linear2, layer_norm; the residual form of
 * linear2 is not repeated). No reference counterpart. */
int32_t mhsa_ffn_profile_enable(mhsa_ffn* ffn, int32_t enable);
int32_t mhsa_ffn_profile_repeat(mhsa_ffn* ffn, const char* tag, int32_t n);
int32_t mhsa_ffn_profile_reset(mhsa_ffn* ffn);
int32_t mhsa_ffn_profile_count(mhsa_ffn* ffn);
int32_t mhsa_ffn_profile_entry(mhsa_ffn* ffn, int32_t idx, const char** name, double* total_ms, int32_t* launches);
/* Debug: linear `which` (0 = linear1, 1 = linear2) alone, as the plain
 * LinearLayer::forward (quantization.rs:126-162) through the GEMM kernels the
 * module runs, without its SiLU or residual epilogue: out [rows, out_dim] =
 * x [rows, in_dim] W^T + b, device; in the module dtype, or f32 (the
 * promoted streaming form) when f32_act. */
int32_t mhsa_ffn_debug_linear(mhsa_ffn* ffn, int32_t which, int32_t f32_act, const void* x, int32_t rows, void* out,
                              void* hip_stream);

/* ---- ConvolutionModule (the Conformer block's convolution sublayer) ------- */

/* ConvolutionModule (conformer.rs:2105-2437): pointwise_conv1 [2D, D] ->
 * GLU (x1 * sigmoid(x2)) -> padding frames zeroed -> depthwise Conv1d
 * (kernel_size K, groups = D; causal: K - 1 frames of left context, else
 * (K - 1) / 2 zeros each side) -> BatchNorm (inference, running statistics)
 * or LayerNorm -> SiLU -> pointwise_conv2 [D, D]. The pointwise convs are
 * standard or MLX affine 8-bit linears (group 64) on the projection GEMMs;
 * GLU, depthwise conv, BatchNorm and SiLU are one fused kernel.
 * d_model a multiple of 64, K <= 129 (odd when not causal); LayerNorm needs
 * d_model <= 2048. Dtypes follow MLX promotion as the reference writes it:
 * a causal module pads with f32 zeros (conformer.rs:2250-2256) and the
 * streaming cache is f32, so everything after the GLU is f32 unless the
 * module is symmetric and runs offline (mhsa_conv_output_dtype). */
#define MHSA_CONV_BATCH_NORM 0 /* ConvNormType::BatchNorm (asr/config.rs:119-128) */
#define MHSA_CONV_LAYER_NORM 1 /* ConvNormType::LayerNorm */
typedef struct mhsa_conv mhsa_conv;
/* ConvolutionModule::new (conformer.rs:2138-2193): zero pointwise layers
 * with zero biases, a zero depthwise kernel (bias when use_bias), the norm
 * at its identity (weight 1, bias 0, running mean 0, variance 1). */
int32_t mhsa_conv_create(int32_t d_model, int32_t kernel_size, int32_t norm_type, int32_t causal, int32_t use_bias,
                         mhsa_conv** out);
void mhsa_conv_destroy(mhsa_conv* conv);
/* set_dtype (conformer.rs:2122-2136): MHSA_F32 or MHSA_BF16; BatchNorm's
 * eps (1e-5) is cast with the parameters. */
int32_t mhsa_conv_set_dtype(mhsa_conv* conv, int32_t dtype);
/* load_weights (conformer.rs:2389-2427): {prefix}.pointwise_conv1 /
 * .pointwise_conv2 as linears (.weight [O, I] or [O, 1, I], .bias, or
 * .weight/.scales/.biases), {prefix}.depthwise_conv.weight [D, K, 1] (MLX
 * layout) and .bias when use_bias, {prefix}.batch_norm.weight / .bias and,
 * for BatchNorm, .running_mean / .running_var (prefix e.g.
 * "encoder.layers.0.conv"). Strict: any missing tensor is MHSA_ENOENT. */
int32_t mhsa_conv_load_weights(mhsa_conv* conv, const mhsa_tensor* tensors, int32_t n_tensors, const char* prefix,
                               int32_t strict, int32_t quant_bits, int32_t quant_group);
/* cache_size (conformer.rs:2384-2386): K - 1. */
int32_t mhsa_conv_cache_size(const mhsa_conv* conv);
/* The dtype mhsa_conv_forward writes: the module dtype for a symmetric
 * module, MHSA_F32 for a causal one. */
int32_t mhsa_conv_output_dtype(const mhsa_conv* conv);
/* Debug: pointwise_conv{1,2} (which 0, 1) alone, as LinearLayer::forward
 * through the module's GEMM kernels: out [rows, 2D or D] = x [rows, D] W^T +
 * b, device, in the module dtype or f32 when f32_act. */
int32_t mhsa_conv_debug_linear(mhsa_conv* conv, int32_t which, int32_t f32_act, const void* x, int32_t rows,
                               void* out, void* hip_stream);
/* forward (conformer.rs:2197-2291): x [batch, seq_len, d_model] device, in
 * the module dtype; lengths [batch] host (frames >= lengths[b] are padding,
 * zeroed after the GLU; NULL = none); out [batch, seq_len, d_model] device
 * in mhsa_conv_output_dtype. */
int32_t mhsa_conv_forward(mhsa_conv* conv, const void* x, int32_t batch, int32_t seq_len, const int32_t* lengths,
                          void* out, void* hip_stream);
/* forward_with_cache (conformer.rs:2305-2378) on the streaming path's f32
 * activations: x, out [batch, seq_len, d_model] f32 device; cache [batch,
 * d_model, K - 1] f32 device (channel-major, as the reference's
 * cache_last_time slice), the left context of the causal conv, replaced in
 * place by the last K - 1 frames of [cache; GLU(x)]; NULL runs the no-cache
 * path (zero left padding). lengths as in mhsa_conv_forward (the
 * reference's pad_mask). A cache needs a causal module (MHSA_EINVAL). */
int32_t mhsa_conv_forward_with_cache(mhsa_conv* conv, const float* x, int32_t batch, int32_t seq_len, float* cache,
                                     const int32_t* lengths, float* out, void* hip_stream);
/* The block's convolution sublayer x <- x + conv(LayerNorm(x))
 * (conformer.rs:1790-1814; with cache 1936-1941), the residual fused into
 * pointwise_conv2's epilogue. cache NULL: offline, x in the module dtype
 * (MHSA_ENOTSUP for a causal bf16 module, whose f32 result x cannot hold);
 * cache set: streaming, x f32. gamma/beta [d_model] host fp32 or NULL. */
int32_t mhsa_conv_sublayer_forward(mhsa_conv* conv, void* x_inout, int32_t batch, int32_t seq_len, float* cache,
                                   const int32_t* lengths, const float* ln_gamma_host, const float* ln_beta_host,
                                   float eps, void* hip_stream);

/* Per-kernel HIP-event timing of the module's launches, as mhsa_profile_*
 * does for a layer (tags pointwise_conv1, conv, layer_norm, pointwise_conv2;
 * repeats skip launches whose repetition would change state: the in-place
 * cache update and the residual form). No reference counterpart. */
int32_t mhsa_conv_profile_enable(mhsa_conv* conv, int32_t enable);
int32_t mhsa_conv_profile_repeat(mhsa_conv* conv, const char* tag, int32_t n);
int32_t mhsa_conv_profile_reset(mhsa_conv* conv);
int32_t mhsa_conv_profile_count(mhsa_conv* conv);
int32_t mhsa_conv_profile_entry(mhsa_conv* conv, int32_t idx, const char** name, double* total_ms,
                                int32_t* launches);

/* ---- the whole Conformer block and the encoder's layer loops ---------------- */

/* ConformerBlock (conformer.rs:1613-2028): the half-step FeedForward, the
 * MHSA sublayer, the convolution sublayer, the second half-step FeedForward
 * and norm_out, each sublayer pre-LayerNorm + residual. The block owns one
 * handle of each module (mhsa_block_attention etc. give them out for
 * profiling; their lifetime is the block's). */
typedef struct mhsa_block mhsa_block;
/* ConformerBlock::new (conformer.rs:1662-1690): two FeedForward(d_model,
 * ff_dim), RelPositionMultiHeadAttention(d_model, n_heads, use_bias),
 * ConvolutionModule(d_model, conv_kernel, conv_norm, causal, use_bias) and
 * five LayerNorms at their init (weight 1, bias 0). */
int32_t mhsa_block_create(int32_t d_model, int32_t n_heads, int32_t ff_dim, int32_t conv_kernel, int32_t conv_norm,
                          int32_t causal, int32_t use_bias, mhsa_block** out);
void mhsa_block_destroy(mhsa_block* block);
/* set_dtype (conformer.rs:1643-1660): every module and norm. */
int32_t mhsa_block_set_dtype(mhsa_block* block, int32_t dtype);
/* load_weights (conformer.rs:1977-2028): {prefix}.feed_forward1,
 * .self_attn, .conv, .feed_forward2 as the modules' loaders take them, and
 * the optional LayerNorm tensors {prefix}.norm_feed_forward1, .norm_self_att,
 * .norm_conv, .norm_feed_forward2, .norm_out (.weight, .bias)
 * (prefix e.g. "encoder.layers.0"). */
int32_t mhsa_block_load_weights(mhsa_block* block, const mhsa_tensor* tensors, int32_t n_tensors, const char* prefix,
                                int32_t strict, int32_t quant_bits, int32_t quant_group);
mhsa_layer* mhsa_block_attention(mhsa_block* block);
mhsa_ffn* mhsa_block_feed_forward(mhsa_block* block, int32_t which /* 1 or 2 */);
mhsa_conv* mhsa_block_conv(mhsa_block* block);
/* forward (conformer.rs:1693-1875) in place: x_inout [batch, seq_len,
 * d_model] device in the block dtype; pos_emb, pos_len, ctx as for
 * mhsa_forward; lengths [batch] host or NULL (PaddingMask,
 * conformer.rs:1594-1615: keys past a length hidden from the attention,
 * clamped to >= 1; frames past it zeroed in the conv). MHSA_ENOTSUP for a
 * causal conv in a bf16 block (its f32 result promotes the rest of the
 * block: mhsa_block_forward_to takes that case). */
int32_t mhsa_block_forward(mhsa_block* block, void* x_inout, int32_t batch, int32_t seq_len, const void* pos_emb,
                           int32_t pos_len, const mhsa_context* ctx, const int32_t* lengths, void* hip_stream);
/* The offline encoder's layer loop (conformer.rs:542-550): every block in
 * order on x_inout with one pos_emb, context and padding. */
int32_t mhsa_encoder_forward(mhsa_block* const* blocks, int32_t n_layers, void* x_inout, int32_t batch,
                             int32_t seq_len, const void* pos_emb, int32_t pos_len, const mhsa_context* ctx,
                             const int32_t* lengths, void* hip_stream);
/* Dtype of forward's result on activations stored in x_dtype (MHSA_F32 or
 * the block dtype): MHSA_F32 once they are f32 or the conv is causal, whose
 * zero padding is an f32 array (conformer.rs:2250-2256), so that in a bf16
 * block MLX promotes the depthwise conv and every later op to f32; else the
 * block dtype. -1 for a null block or a dtype it cannot take. */
int32_t mhsa_block_output_dtype(const mhsa_block* block, int32_t x_dtype);
/* forward (conformer.rs:1693-1875) as the returned array of the reference's
 * ConformerBlock::forward, whose dtype may differ from its input's: x
 * [batch, seq_len, d_model] device in x_dtype, which is the block dtype or,
 * in a bf16 block, MHSA_F32 (activations an earlier causal conv promoted:
 * every op then runs in f32 on the parameters' bf16 values); out in
 * mhsa_block_output_dtype(block, x_dtype). out may be x when the two dtypes
 * agree, else they must not overlap; x is otherwise left unchanged. Other
 * arguments as mhsa_block_forward. */
int32_t mhsa_block_forward_to(mhsa_block* block, const void* x, int32_t x_dtype, int32_t batch, int32_t seq_len,
                              const void* pos_emb, int32_t pos_len, const mhsa_context* ctx, const int32_t* lengths,
                              void* out, void* hip_stream);
/* The offline encoder's layer loop (conformer.rs:542-550) over
 * mhsa_block_forward_to: block 0 reads x (x_dtype), the others run on out,
 * which ends in the dtype mhsa_block_output_dtype gives when chained over
 * the blocks (f32 after the first causal conv of a bf16 stack); x and out
 * must not overlap unless no block changes the dtype. */
int32_t mhsa_encoder_forward_to(mhsa_block* const* blocks, int32_t n_layers, const void* x, int32_t x_dtype,
                                int32_t batch, int32_t seq_len, const void* pos_emb, int32_t pos_len,
                                const mhsa_context* ctx, const int32_t* lengths, void* out, void* hip_stream);

/* The streaming encoder's per-chunk loop over n_layers blocks
 * (ConformerEncoder::forward_streaming, conformer.rs:840-1047, with
 * ConformerBlock::forward_with_cache, conformer.rs:1893-1971): per layer an
 * HBM ring of cache_size attention frames and the conv cache [batch,
 * d_model, K - 1] (cache_last_time, zeros at creation), one fill per
 * session. Blocks need causal convs of one kernel size >= 2; they are not
 * owned and must not serve another encoder at the same time. */
typedef struct mhsa_encoder mhsa_encoder;
int32_t mhsa_encoder_create(mhsa_block* const* blocks, int32_t n_layers, int32_t batch, int32_t cache_size,
                            int32_t chunk_len, mhsa_encoder** out);
void mhsa_encoder_destroy(mhsa_encoder* enc);
/* channel [n_layers, batch, cache_size, d_model] and time [n_layers, batch,
 * d_model, K - 1] device fp32 (time NULL = zeros); filled_host [batch] (NULL
 * = 0). */
int32_t mhsa_encoder_load_cache(mhsa_encoder* enc, const float* channel_cache, const float* time_cache,
                                const int32_t* filled_host, void* hip_stream);
int32_t mhsa_encoder_read_cache(const mhsa_encoder* enc, float* channel_cache_out, float* time_cache_out,
                                void* hip_stream);
int32_t mhsa_encoder_fill(const mhsa_encoder* enc, int32_t* filled_out_host);
/* One chunk through every block: x_inout [batch, chunk_len, d_model] device
 * fp32 (the streaming activations stay f32, conformer.rs:845-849), updated in
 * place; pos_emb [2*(cache_size+chunk_len)-1, d_model] device in the block
 * dtype; mask as for mhsa_stack_step; valid_host [batch] or NULL: the conv's
 * pad_mask (frames past valid zeroed after the GLU, conformer.rs:929-941). */
int32_t mhsa_encoder_step(mhsa_encoder* enc, float* x_inout, const void* pos_emb, int32_t pos_len,
                          const mhsa_stream_mask* mask, const int32_t* valid_host, void* hip_stream);

/* ---- encoder-level streaming ---------------------------------------------- */

/* The per-chunk layer loop of ConformerEncoder::forward_streaming
 * (conformer.rs:840-1047) over the attention sublayers of n_layers layers
 * (same d_model), with the EncoderCache (streaming/core.rs:117-166) kept as
 * one HBM ring per layer instead of the reference's slice, pad/truncate and
 * restack of [layers, batch, C, D] (conformer.rs:958-1023), and one fill per
 * session (the reference uses session 0's for every session,
 * conformer.rs:883-887). The layers must not be used by another stack or
 * stream at the same time. */
typedef struct mhsa_stack mhsa_stack;
int32_t mhsa_stack_create(mhsa_layer* const* layers, int32_t n_layers, int32_t batch, int32_t cache_size,
                          int32_t chunk_len, mhsa_stack** out);
void mhsa_stack_destroy(mhsa_stack* stack);
/* cache [n_layers, batch, cache_size, d_model] device fp32 (last_channel);
 * filled_host [batch] (last_channel_len; NULL = 0). */
int32_t mhsa_stack_load_cache(mhsa_stack* stack, const void* cache, const int32_t* filled_host, void* hip_stream);
int32_t mhsa_stack_read_cache(const mhsa_stack* stack, void* cache_out, void* hip_stream);
int32_t mhsa_stack_fill(const mhsa_stack* stack, int32_t* filled_out_host);
/* One chunk through every layer: x <- x + MHSA_l(LayerNorm_l(x)) with each
 * layer's cache (the attention part of ConformerBlock::forward_with_cache,
 * conformer.rs:1924-1934), then the fill update min(fill + q_keep, C)
 * (conformer.rs:1025-1036) with q_keep from each layer's cache_drop_size.
 *  x_inout  [batch, chunk_len, d_model] device fp32, updated in place
 *  ln_gamma_host / ln_beta_host  [n_layers, d_model] host fp32 (NULL = 1 / 0),
 *           held at each layer's parameter precision; eps as nn::LayerNorm
 *  pos_emb  [2*(cache_size+chunk_len)-1, d_model] device, layer dtype
 *  mask     as for mhsa_forward_with_cache; a NULL filled_host means every
 *           layer reads the fills the stack had at the start of the step. */
int32_t mhsa_stack_step(mhsa_stack* stack, void* x_inout, const float* ln_gamma_host, const float* ln_beta_host,
                        float eps, const void* pos_emb, int32_t pos_len, const mhsa_stream_mask* mask,
                        void* hip_stream);

/* ---- helpers ------------------------------------------------------------ */

/* RelPositionalEncoding::new(d_model, max_len).get_encoding(seq_len)
 * (attention.rs:59-103, 131-177) into a HOST fp32 buffer
 * [2*seq_len-1, d_model]; seq_len > max_len regenerates the table. */
int32_t mhsa_pos_encoding(int32_t d_model, int32_t max_len, int32_t seq_len, float* out_host);

/* ---- per-kernel timing --------------------------------------------------- */

/* No counterpart in the reference (it times whole calls with wall clocks,
 * examples/eval.rs:181-183, 289-295). When enabled, every kernel the layer
 * launches is bracketed by HIP events on the launch stream; totals accumulate
 * per kernel tag (gemm_qkv, gemm_pos, gemm_qkv_pos where the offline Q/K/V
 * and position projections run in one launch, attention, gemm_out,
 * layer_norm, gemm_q, gemm_kv, ring_write). Reading waits for the recorded
 * events. */
int32_t mhsa_profile_enable(mhsa_layer* layer, int32_t enable);
/* While profiling is enabled, issue every launch tagged `tag` n times inside
 * its event pair (it then counts as n launches), so the event overhead is
 * spread over n back-to-back launches. For timing only: an in-place output
 * (the sublayer's residual add) is applied n times. n = 1 turns it off. */
int32_t mhsa_profile_repeat(mhsa_layer* layer, const char* tag, int32_t n);
int32_t mhsa_profile_reset(mhsa_layer* layer);
/* Number of distinct tags recorded so far (flushes pending events). */
int32_t mhsa_profile_count(mhsa_layer* layer);
/* Entry idx: tag name (valid until the next reset), total ms and launches. */
int32_t mhsa_profile_entry(mhsa_layer* layer, int32_t idx, const char** name, double* total_ms, int32_t* launches);

/* ---- debug exports (bit-exact checks) ----------------------------------- */

/* Dequantised weight [out, in] of a quantized projection, as the GEMM loader
 * produces it in the current dtype, widened to fp32 (device output). */
int32_t mhsa_debug_dequantize(mhsa_layer* layer, int32_t which, float* out_dev, void* hip_stream);
/* One projection alone, LinearLayer::forward (quantization.rs:126-162):
 * out [rows, d_model] = x [rows, d_model] W^T (+ bias), device, layer dtype,
 * through the same GEMM kernels the forward pass uses. */
int32_t mhsa_debug_linear(mhsa_layer* layer, int32_t which, const void* x, int32_t rows, void* out_dev,
                          void* hip_stream);
/* The same projection as the streaming path runs it: f32 activations x,
 * out_dev [rows, d_model], fp32 kernels; a bf16 layer's parameters keep
 * their bf16 values (MLX promotes the op to f32, conformer.rs:845-849). */
int32_t mhsa_debug_linear_f32(mhsa_layer* layer, int32_t which, const float* x, int32_t rows, float* out_dev,
                              void* hip_stream);
/* Launches of each attention kernel form since the library was loaded
 * (process-wide; no reference counterpart): counts[f] for f < n, in the
 * order 0 bf16 4-wave, 1 bf16 8-wave, 2 bf16 8-wave with tile skipping,
 * 3 both bf16 forms in one launch, 4 both bf16 forms with a projection GEMM
 * in the launch, 5 fp32 streaming chunk, 6 generic, 7 generic key split.
 * Returns the number of forms (8). */
int32_t mhsa_debug_attention_forms(int64_t* counts, int32_t n);
/* The sublayer's LayerNorm alone (nn::LayerNorm, conformer.rs:1749), as
 * mhsa_sublayer_forward and mhsa_stack_sublayer_forward run it: out_dev
 * [rows, d_model] = LayerNorm(x) in the layer dtype (device); gamma/beta
 * host fp32 or NULL. */
int32_t mhsa_debug_layer_norm(mhsa_layer* layer, const void* x, int32_t rows, const float* ln_gamma_host,
                              const float* ln_beta_host, float eps, void* out_dev, void* hip_stream);
/* Visibility map [batch, seq_len, seq_len] (1 = visible) the offline kernel
 * applies for (ctx, key lengths) (device output). */
int32_t mhsa_debug_offline_mask(int32_t batch, int32_t seq_len, const mhsa_context* ctx,
                                const int32_t* key_lengths_host, uint8_t* out_dev, void* hip_stream);
/* Visibility map [batch, chunk_len, cache_size + chunk_len] the streaming
 * kernel applies (device output); filled_host must be given. */
int32_t mhsa_debug_stream_mask(int32_t batch, int32_t cache_size, int32_t chunk_len, const mhsa_stream_mask* mask,
                               uint8_t* out_dev, void* hip_stream);
/* Position-table row read for every (query i, key j) pair [rows, total_len]
 * (device output): the closed form of rel_shift + truncation
 * (attention.rs:831-855) as the kernel evaluates it. */
int32_t mhsa_debug_rel_shift_index(int32_t rows, int32_t total_len, int32_t* out_dev, void* hip_stream);
/* Scaled position scores cast(s) * rel_shift(q_v P^T)[..., :seq_len]
 * [batch, n_heads, seq_len, seq_len] fp32 (device), computed by the fused
 * kernel's MFMA + LDS remap path, for a full-attention offline call.
 * q_out_dev [batch, seq_len, d_model] and p_out_dev [pos_len, d_model]
 * (layer dtype, device, each may be NULL) receive the projected queries and
 * position rows the kernel consumed. */
int32_t mhsa_debug_position_scores(mhsa_layer* layer, const void* x, int32_t batch, int32_t seq_len,
                                   const void* pos_emb, int32_t pos_len, float* out_dev, void* q_out_dev,
                                   void* p_out_dev, void* hip_stream);
/* For a bf16 layer: the offline forward's attention logits
 * s*(q_u k) + cast(s)*bd + mask (attention.rs:299-318) reduced per query row
 * by the production kernel to the visible key with the largest logit (lowest
 * index on ties, -1 when the row sees no key): top_dev [batch, n_heads,
 * seq_len] int32 and logit_dev [batch, n_heads, seq_len] fp32 (device). The
 * arguments are those of mhsa_forward; no output is written. q_out_dev and
 * k_out_dev [batch, seq_len, d_model] and, for full attention, p_out_dev
 * [pos_len, d_model] (bf16, device, each may be NULL) receive the projected
 * queries, keys and position rows the kernel consumed. */
int32_t mhsa_debug_top_keys(mhsa_layer* layer, const void* x, int32_t batch, int32_t seq_len, const void* pos_emb,
                            int32_t pos_len, const mhsa_context* ctx, const int32_t* key_lengths_host,
                            int32_t* top_dev, float* logit_dev, void* q_out_dev, void* k_out_dev, void* p_out_dev,
                            void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* RELPOS_MHSA_H */
