// Launch interface between the host runtime (mhsa_api.hip) and the gfx950
// kernels (gemm.hip, attention.hip, misc.hip). Every launcher checks the shape
// assumptions its kernel relies on and returns a hipError_t (or
// hipErrorInvalidValue when a shape does not fit the kernel).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mhsa {

enum DType : int { kF32 = 0, kBF16 = 1 };

inline int dtype_size(DType d) { return d == kF32 ? 4 : 2; }

// C[out_row(r), n] = epilogue( sum_k A[r, k] * W[n, k] )
//   dense W: [N, K] in the compute dtype; quantized W: uint32 [N, K/4] holding
//   one u8 code per byte, with `sb` = [N, K/64] {scale, bias} float pairs.
//   out_row(r) = (r / seg_rows) * seg_stride + (ring_off + r % seg_rows) % ring_len
// Epilogue (reference order): y = T(acc); y = T(y + bias[n]); y = T(R[r, n] + y).
struct GemmParams {
  const void* A = nullptr;
  int64_t lda = 0;
  const void* W = nullptr;
  const float* sb = nullptr;
  const float* bias = nullptr;
  const void* R = nullptr;
  int64_t ldr = 0;
  void* C = nullptr;
  int64_t ldc = 0;
  int M = 0, N = 0, K = 0;
  int seg_rows = 0, seg_stride = 0, ring_off = 0, ring_len = 0;
  // fp32 scratch for K-split partial sums (small problems); null = no split
  float* partial = nullptr;
  int64_t partial_elems = 0;
  // Optional transposed copy of output columns [vt_col0, N) (the V
  // projection): VT[col - vt_col0][(row / seg_T) * vt_Tpad + row % seg_T],
  // row stride vt_ld; those columns are then not written to C. Columns past
  // each utterance's seg_T tokens receive finite filler.
  void* vt = nullptr;
  int64_t vt_ld = 0;
  int vt_col0 = 0, vt_Tpad = 0;
  // > 0: M tiles per utterance of seg_T rows (M a multiple of seg_T);
  // required with vt, where utterance b's tokens start at column b * vt_Tpad
  int seg_T = 0;
  // Optional split output (the streaming chunk's fused Q|K|V projection):
  // columns [c2_col0, N) go to C2 (leading dimension ldc2) at the rows the
  // seg/ring fields map to, columns below c2_col0 to C at rows as they are.
  // With acopy, A's rows are also copied to acopy (leading dimension
  // acopy_ld) at the mapped rows. Only gemm_split_fused_ok() shapes take them.
  void* C2 = nullptr;
  int64_t ldc2 = 0;
  int c2_col0 = 0;
  void* acopy = nullptr;
  int64_t acopy_ld = 0;
  // FeedForward epilogues (conformer.rs:1727-1729, 2066-2072): act = kActSilu
  // applies SiLU after the bias as the reference materialises nn::silu,
  // T(y * T(sigmoid(y))); res_scale multiplies y before the residual add (the
  // half-step residual R + 0.5 y; exact in either dtype)
  int act = 0;
  float res_scale = 1.f;
};
constexpr int kActSilu = 1;
// Scratch the K-split path can use: 64x64 tiles x splits stays <= ~512
// workgroups, so M*N*splits <= kGemmPartialElems.
constexpr int64_t kGemmPartialElems = (int64_t)1 << 22;
hipError_t gemm(DType dt, bool quantized, const GemmParams& p, hipStream_t s);
// gemm()'s argument checks alone (p.M > 0 assumed).
hipError_t gemm_check(DType dt, bool quantized, const GemmParams& p);
// The tile GEMM form (tile rows, tile columns, LDS stages) gemm() launches
// for a valid bf16 problem; false when it takes another kernel.
struct TileForm {
  int bm = 0, bn = 0, ns = 0;
};
bool gemm_tile_form(DType dt, bool quantized, const GemmParams& p, TileForm& f);
// Two independent GEMMs of one dtype and weight form in one launch: p2's
// tiles take the CUs p1's tiles free as they end. For a p1 that gemm() runs
// in one round of tiles of a form larger than 64x64 and a p2 it runs in the
// 64x64 form (gemm_pair_ok); the same results as gemm() on each. Otherwise
// hipErrorInvalidValue and nothing is launched.
bool gemm_pair_ok(DType dt, bool quantized, const GemmParams& p1, const GemmParams& p2);
hipError_t gemm_pair(DType dt, bool quantized, const GemmParams& p1, const GemmParams& p2, hipStream_t s);
// Whether gemm() takes this problem with C2 / acopy set (fp32, few rows).
bool gemm_split_fused_ok(DType dt, const GemmParams& p);
// Compute units of the current device (256 if the query fails), read once
// per device.
int device_cus();

constexpr int kMaxBatch = 64;

// Fused rel-pos attention over one head slice per (query tile, head, batch).
// Query i of batch b sits at absolute frame qoff + i; key j at frame j and is
// stored at row (ring_head + j) % ring_len (row j when ring_len == 0). The
// position row of pair (i, j) is center - (qoff + i) + j (the closed form of
// the Transformer-XL rel_shift). Key j is visible to query i iff
// key_lo[b] <= j < key_hi[b], i < q_valid[b], and the context rule holds.
struct AttnParams {
  const void* q = nullptr;
  int64_t q_bs = 0, q_rs = 0;
  const void* k = nullptr;
  const void* v = nullptr;
  int64_t kv_bs = 0, kv_rs = 0;
  int ring_head = 0, ring_len = 0;
  const void* p = nullptr;
  int64_t p_rs = 0;
  int p_rows = 0, center = 0;
  const float* bias_u = nullptr;  // [H, dk], values in the compute dtype
  const float* bias_v = nullptr;
  void* o = nullptr;
  int64_t o_bs = 0, o_rs = 0;
  float* dbg_bd = nullptr;  // debug: scaled position scores [B, H, T, L]
  // debug (bf16 kernel): per query row [B, H, T], the visible key with the
  // largest logit (lowest index on ties; -1 when none is visible) and that logit
  int* dbg_top = nullptr;
  float* dbg_topv = nullptr;
  // bf16 path: V^T [H*dk][B*Tpad] (key j of batch b at column b*vt_bs + j,
  // zeros or finite values past T); null selects the row-major V path.
  const void* vt = nullptr;
  int64_t vt_ld = 0, vt_bs = 0;
  // bf16 path: rows readable (finite) around the position table, p_pad
  // before row 0 and after row p_rows - 1 (at least bf16_pos_pad), and past
  // the last key row of the last item (at least 63)
  int p_pad = 0, kv_pad = 0;
  int T = 0, L = 0, qoff = 0, H = 0;
  float scale = 0.f, scale_bd = 0.f;
  int has_ctx = 0, left = -1, right = -1, chunked = 0;
  int b0 = 0;
  // bf16 (V^T) kernel: items in launch order, longest key range first, so
  // that the work left for a second round of workgroups is the shortest
  // (a permutation of [0, nbatch); filled by the launcher)
  int order[kMaxBatch];
  int key_lo[kMaxBatch];
  int key_hi[kMaxBatch];
  int q_valid[kMaxBatch];
};
hipError_t attention(DType dt, int head_dim, const AttnParams& p, int nbatch, hipStream_t s);
// attention() and, in the same launch, the tile GEMM `g`: a projection that
// does not depend on the attention (nor the attention on it), whose tiles
// take the CUs the attention leaves idle. Only for the bf16 8-wave form
// without a window or chunk limit and a GEMM of 128 x 128 tiles; otherwise
// hipErrorNotSupported and nothing is
// launched (the caller launches the two apart). Same results as apart.
hipError_t attention_with_gemm(DType dt, int head_dim, const AttnParams& p, int nbatch, const GemmParams& g,
                               bool gquant, hipStream_t s);
// Attention kernel forms, counted per launch (process-wide) so that tests
// can tell which form a dispatch took.
enum AttnForm {
  kFormBf16Wave4 = 0,  // bf16, 4 waves of 32 queries, 64-key tiles
  kFormBf16Wave8,      // bf16, 8 waves of 32 queries, 32-key tiles
  kFormBf16Wave8Skip,  // the 8-wave form with per-wave tile skipping (windows)
  kFormBf16Mixed,      // both bf16 forms in one launch
  kFormBf16MixedGemm,  // both bf16 forms and a projection GEMM in one launch
  kFormChunkF32,       // fp32 streaming chunk kernel
  kFormGeneric,        // generic kernel (fp32, or bf16 without V^T)
  kFormKeySplit,       // generic kernel, keys split over the waves
  kAttnForms
};
int64_t attention_form_count(int form);
// Position rows the bf16 kernel reads beyond the table on either side for
// these items' key ranges (key_lo / key_hi / q_valid, context, T, center).
int bf16_pos_pad(const AttnParams& p, int nbatch);

// Visibility map [nbatch, T, L] (1 = visible) from the same predicate the
// attention kernel applies.
hipError_t export_mask(const AttnParams& p, int nbatch, uint8_t* out, hipStream_t s);
// Position-row index of every (i, j) pair [T, L], as the attention kernel computes it.
hipError_t export_pos_index(int T, int L, int qoff, int center, int32_t* out, hipStream_t s);

// y = T(LayerNorm(x) * gamma + beta), statistics in fp32; gamma/beta may be null.
// act = kActSilu then applies nn::silu to the stored result (the conv
// module's norm -> SiLU). Rows are held in registers, one wave per row:
// D <= kMaxLayerNormDim; y may alias x.
constexpr int kMaxLayerNormDim = 2048;
hipError_t layer_norm(DType dt, const void* x, void* y, const float* gamma, const float* beta,
                      float eps, int rows, int D, hipStream_t s, int act = 0);

// ConvolutionModule middle (conformer.rs:2197-2291, 2305-2378) for a batch
// chunk: y[b, t, c] = post(sum_k w[k, c] * u[b, t - left + k, c] (+ bias[c]))
// where u = GLU(g) = g[.., :D] * sigmoid(g[.., D:]) in the GLU dtype, zero
// at frames >= len[b] and past T; frames before 0 come from cache_in
// [b, c, K-1+s] (f32, channel-major) or are zero. post = BatchNorm (bn =
// [4, D]: mean, rsqrt(var + eps), weight, bias) then SiLU when bn is set,
// else nothing (LayerNorm runs afterwards). cache_out (may equal cache_in
// only when one frame tile covers T) receives the last K - 1 frames of
// [cache; u]. g [B, T, 2D], y [B, T, D]; D % 64 == 0, K <= kMaxConvKernel.
constexpr int kMaxConvKernel = 129;
struct ConvParams {
  const void* g = nullptr;
  void* y = nullptr;
  const float* cache_in = nullptr;
  float* cache_out = nullptr;
  const float* w = nullptr;     // [K, D]
  const float* bias = nullptr;  // [D] or null
  const float* bn = nullptr;    // [4, D] or null
  int T = 0, D = 0, K = 0, left = 0;
  int len[kMaxBatch] = {};
};
hipError_t conv_glu_depthwise(DType glu_dt, DType conv_dt, const ConvParams& p, int nbatch, hipStream_t s);
// Output frames one workgroup covers (a cache updated in place needs T <= this).
int conv_frame_tile();

// Ring copies between a contiguous [B, n, D] block and a ring [B, R, ld]
// (row t of batch b <-> ring row (off + t) % R, columns [0, D)).
hipError_t ring_write(DType dt, const void* src, void* ring, int B, int n, int D, int R, int64_t ld,
                      int off, hipStream_t s);
hipError_t ring_read(DType dt, const void* ring, void* dst, int B, int n, int D, int R, int64_t ld,
                     int off, hipStream_t s);

// dst[i] = float(src[i]) for n bf16 values (16-byte aligned, n % 8 == 0).
hipError_t widen_bf16(const void* src, float* dst, int64_t n, hipStream_t s);

// Zero-fill of device memory by a kernel (no memset node under graph capture).
hipError_t fill_zero(void* ptr, size_t bytes, hipStream_t s);

// Dequantised weight [N, K] as the GEMM's loader produces it, widened to fp32.
hipError_t dequant_export(DType dt, const uint32_t* w, const float* sb, float* out, int N, int K,
                          hipStream_t s);

}  // namespace mhsa
