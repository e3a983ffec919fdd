// Sublayer forms that the block runtime (encoder_api.hip) composes from the
// modules of other translation units, for a bf16 block whose activations a
// causal conv has made f32: its zero padding is an f32 array
// (conformer.rs:2250-2256), so MLX promotes the depthwise conv and every
// later op of the block, and of every later block, to f32 on the
// parameters' bf16 values.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/relpos_mhsa.h"
#include "kernels.hpp"

// x <- x + MHSA(LayerNorm(x)) offline on f32 activations x [B, T, D]
// (conformer.rs:1747-1780, attention.rs:446-573), a layer of either dtype:
// the projections in fp32 on the layer's parameter values, matrix_bd in
// fp32, the position rows a table in the layer dtype through its weights;
// ctx and lens as mhsa_sublayer_forward takes them. (mhsa_api.hip)
int32_t mhsa_sublayer_forward_act32(mhsa_layer* L, float* x, int B, int T, const float* gamma, const float* beta,
                                    float eps, const void* pos_emb, int pos_len, const mhsa_context* ctx,
                                    const int32_t* lens, hipStream_t s);

// out = x + conv(LayerNorm(x)) offline in f32 (conformer.rs:1790-1814): x
// [B, T, D] in x_dt, either f32 activations or, for a causal module, bf16
// ones in a bf16 module, whose LayerNorm, pointwise_conv1 and GLU stay bf16
// before the f32 padding; out f32, equal to x or not overlapping it; lens as
// mhsa_conv_sublayer_forward takes them. (block_api.hip)
int32_t mhsa_conv_sublayer_to_f32(mhsa_conv* m, const void* x, mhsa::DType x_dt, int B, int T,
                                  const int32_t* lens, const float* gamma, const float* beta, float eps, float* out,
                                  hipStream_t s);
