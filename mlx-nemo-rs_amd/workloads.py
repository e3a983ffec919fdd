"""Synthetic workloads for the rel-pos MHSA path (host-side numpy generators).

Six configurations of the FastConformer attention sublayer:

* ``large_f32``       D=512, H=8, B=1, T=125, fp32, no padding, full context
                      (FastConformer-large, 10 s of audio), seed 0
* ``xl_offline_bf16`` D=1024, H=8, B=8, T=375, bf16, key padding with valid
                      lengths U{188..375}, seed 1
* ``xl_stream_f32``   D=1024, H=8, 16 sessions, 14-frame chunks against a
                      70-frame cache, [70, 13] chunked_limited context, fills
                      U{0..70}, 50 steps, fp32, seed 2
* ``xl_local_bf16``   D=1024, H=8, B=2, T=7500, bf16, regular (128, 128)
                      window with a 257-row banded position table, seed 3
* ``xl_stream_f32_24l`` the same streaming step through 24 distinct layers
                      (own weights and cache each, ~680 MB, beyond the 256 MB
                      Infinity Cache), seed 2
* ``xl_stack_u8``     24 sublayers x <- x + MHSA(LN(x)) with affine u8
                      projections (group 64, f16 scales U(0.002, 0.02), f16
                      biases N(0, 0.01), codes U{0..255}), B=4, T=1500, bf16,
                      valid lengths U{1000..1500}, seed 4

two of the block's ConvolutionModule (conformer.rs:2105-2437):

* ``conv_offline_bf16`` D=1024, K=9, BatchNorm, symmetric, B=8, T=375, bf16,
                      valid lengths U{188..375}, seed 5
* ``conv_stream_f32``  D=1024, K=9, LayerNorm, causal, 16 sessions, 14-frame
                      chunks through the [16, 1024, 8] f32 conv cache, 50
                      steps, fp32, seed 6

and two of the whole ConformerBlock (conformer.rs:1613-2028: FF1 half step,
MHSA, conv, FF2 half step, norm_out) at the 0.6B shape (ff_dim 4096, conv
kernel 9):

* ``block_offline_bf16`` B=8, T=375, bf16, symmetric conv with BatchNorm,
                      valid lengths U{188..375}, seed 7
* ``block_stream_f32`` 16 sessions, 14-frame chunks against a 70-frame
                      attention cache under [70, 13] chunked_limited, causal
                      conv with LayerNorm and its [16, 1024, 8] cache, fills
                      U{0..70}, 50 steps, fp32, seed 8

Weights are Xavier-uniform U(+-sqrt(6 / 2D)), pos_bias_u/v ~ N(0, 0.02^2),
inputs x ~ N(0, 1); every array comes from numpy's PCG64 with the stated
seed, so the same bytes reach the GPU and the oracle.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np


@dataclass
class Workload:
    name: str
    d_model: int
    n_heads: int
    batch: int
    seq_len: int
    dtype: str  # "float32" | "bfloat16"
    seed: int
    use_bias: bool = False
    lengths: Optional[List[int]] = None
    context: Optional[Tuple[int, int, str]] = None  # (left, right, style)
    pos_band: Optional[int] = None  # rows of a centred banded table (2W+1)
    quantized: bool = False
    layers: int = 1
    # streaming
    cache_size: int = 0
    steps: int = 0
    fills: Optional[List[int]] = None
    # "mhsa" (the attention sublayer), "conv" (ConvolutionModule) or
    # "block" (the whole ConformerBlock)
    module: str = "mhsa"
    conv_kernel: int = 0
    conv_norm: str = "batch_norm"
    causal: bool = False
    ff_dim: int = 0  # "block": FeedForward width

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads


def xavier(rng, d_out, d_in):
    bound = np.sqrt(6.0 / (d_in + d_out))
    return rng.uniform(-bound, bound, size=(d_out, d_in)).astype(np.float32)


def pack_u8(codes: np.ndarray) -> np.ndarray:
    """MLX 8-bit packing: four codes per u32 along the input dim, lowest byte first."""
    c = codes.astype(np.uint32)
    return (c[:, 0::4] | (c[:, 1::4] << 8) | (c[:, 2::4] << 16) | (c[:, 3::4] << 24)).astype(np.uint32)


def make_layer_weights(rng, d_model: int, n_heads: int, use_bias: bool, quantized: bool,
                       centred: bool = False) -> Dict[str, np.ndarray]:
    """Weights of one layer keyed like a checkpoint (`{name}.weight`, ...)."""
    d = d_model
    w: Dict[str, np.ndarray] = {}
    for name in ("linear_q", "linear_k", "linear_v", "linear_out", "linear_pos"):
        if quantized:
            codes = rng.integers(0, 256, size=(d, d))
            scales = rng.uniform(0.002, 0.02, size=(d, d // 64)).astype(np.float16)
            qb = rng.normal(0.0, 0.01, size=(d, d // 64))
            if centred:
                qb = qb - 128.0 * scales.astype(np.float64)
            w[f"{name}.weight"] = pack_u8(codes)
            w[f"{name}.scales"] = scales
            w[f"{name}.biases"] = qb.astype(np.float16)
        else:
            w[f"{name}.weight"] = xavier(rng, d, d)
        if use_bias and name != "linear_pos":
            w[f"{name}.bias"] = np.zeros(d, dtype=np.float16 if quantized else np.float32)
    dk = d // n_heads
    w["pos_bias_u"] = rng.normal(0.0, 0.02, size=(n_heads, dk)).astype(np.float32)
    w["pos_bias_v"] = rng.normal(0.0, 0.02, size=(n_heads, dk)).astype(np.float32)
    return w


def prefixed(weights: Dict[str, np.ndarray], prefix: str) -> Dict[str, np.ndarray]:
    return {f"{prefix}.{k}": v for k, v in weights.items()}


CONFIGS: Dict[str, Workload] = {
    "large_f32": Workload("large_f32", 512, 8, 1, 125, "float32", seed=0, use_bias=True),
    "xl_offline_bf16": Workload("xl_offline_bf16", 1024, 8, 8, 375, "bfloat16", seed=1),
    "xl_stream_f32": Workload("xl_stream_f32", 1024, 8, 16, 14, "float32", seed=2,
                              context=(70, 13, "chunked_limited"), cache_size=70, steps=50),
    "xl_stream_f32_24l": Workload("xl_stream_f32_24l", 1024, 8, 16, 14, "float32", seed=2,
                                  context=(70, 13, "chunked_limited"), cache_size=70, steps=50, layers=24),
    "xl_local_bf16": Workload("xl_local_bf16", 1024, 8, 2, 7500, "bfloat16", seed=3,
                              context=(128, 128, "regular"), pos_band=257),
    "xl_stack_u8": Workload("xl_stack_u8", 1024, 8, 4, 1500, "bfloat16", seed=4, quantized=True, layers=24),
    "conv_offline_bf16": Workload("conv_offline_bf16", 1024, 8, 8, 375, "bfloat16", seed=5, use_bias=True,
                                  module="conv", conv_kernel=9, conv_norm="batch_norm"),
    "conv_stream_f32": Workload("conv_stream_f32", 1024, 8, 16, 14, "float32", seed=6, use_bias=True, steps=50,
                                module="conv", conv_kernel=9, conv_norm="layer_norm", causal=True),
    "block_offline_bf16": Workload("block_offline_bf16", 1024, 8, 8, 375, "bfloat16", seed=7, use_bias=True,
                                   module="block", conv_kernel=9, conv_norm="batch_norm", ff_dim=4096),
    "block_stream_f32": Workload("block_stream_f32", 1024, 8, 16, 14, "float32", seed=8, use_bias=True,
                                 cache_size=70, steps=50, context=(70, 13, "chunked_limited"), module="block",
                                 conv_kernel=9, conv_norm="layer_norm", causal=True, ff_dim=4096),
}

BLOCK_NORMS = ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out")


def make_block_weights(rng, d: int, h: int, f: int, k: int, norm: str = "batch_norm", prefix: str = "blk"):
    """One ConformerBlock's tensors keyed like a checkpoint (conformer.rs:1977-2028):
    feed_forward1/2 Xavier-uniform with biases N(0, 0.02), self_attn as
    make_layer_weights with zero biases, conv as make_conv_weights, the five
    LayerNorms weight U(0.8, 1.2), bias N(0, 0.05)."""
    w: Dict[str, np.ndarray] = {}
    for ff in ("feed_forward1", "feed_forward2"):
        for name, (o, i) in (("linear1", (f, d)), ("linear2", (d, f))):
            w[f"{prefix}.{ff}.{name}.weight"] = xavier(rng, o, i)
            w[f"{prefix}.{ff}.{name}.bias"] = rng.normal(0, 0.02, o).astype(np.float32)
    w.update(prefixed(make_layer_weights(rng, d, h, True, False), f"{prefix}.self_attn"))
    w.update(make_conv_weights(rng, d, k, norm, False, True, f"{prefix}.conv"))
    for n in BLOCK_NORMS:
        w[f"{prefix}.{n}.weight"] = rng.uniform(0.8, 1.2, d).astype(np.float32)
        w[f"{prefix}.{n}.bias"] = rng.normal(0, 0.05, d).astype(np.float32)
    return w


def make_conv_weights(rng, d: int, k: int, norm: str = "batch_norm", quantized: bool = False,
                      use_bias: bool = True, prefix: str = "conv") -> Dict[str, np.ndarray]:
    """ConvolutionModule tensors keyed like a checkpoint (conformer.rs:2389-2427):
    pointwise convs Xavier-uniform (or affine u8 with zero-mean weights:
    scales U(2e-4, 1e-3), biases -128 s + N(0, 1e-3)), biases N(0, 0.1),
    depthwise [D, K, 1] ~ N(0, 1/K), norm weight U(0.5, 1.5) and bias
    N(0, 0.1), running mean N(0, 0.1) and variance U(0.5, 2)."""
    w: Dict[str, np.ndarray] = {}
    for name, o in (("pointwise_conv1", 2 * d), ("pointwise_conv2", d)):
        if quantized:
            codes = rng.integers(0, 256, size=(o, d))
            sc = rng.uniform(2e-4, 1e-3, size=(o, d // 64)).astype(np.float16)
            w[f"{prefix}.{name}.weight"] = pack_u8(codes)
            w[f"{prefix}.{name}.scales"] = sc
            w[f"{prefix}.{name}.biases"] = (-128.0 * sc.astype(np.float64)
                                            + rng.normal(0, 1e-3, sc.shape)).astype(np.float16)
            if use_bias:
                w[f"{prefix}.{name}.bias"] = rng.normal(0, 0.1, o).astype(np.float16)
        else:
            w[f"{prefix}.{name}.weight"] = xavier(rng, o, d)
            if use_bias:
                w[f"{prefix}.{name}.bias"] = rng.normal(0, 0.1, o).astype(np.float32)
    w[f"{prefix}.depthwise_conv.weight"] = (rng.standard_normal((d, k, 1)) / np.sqrt(k)).astype(np.float32)
    if use_bias:
        w[f"{prefix}.depthwise_conv.bias"] = rng.normal(0, 0.1, d).astype(np.float32)
    w[f"{prefix}.batch_norm.weight"] = rng.uniform(0.5, 1.5, d).astype(np.float32)
    w[f"{prefix}.batch_norm.bias"] = rng.normal(0, 0.1, d).astype(np.float32)
    if norm == "batch_norm":
        w[f"{prefix}.batch_norm.running_mean"] = rng.normal(0, 0.1, d).astype(np.float32)
        w[f"{prefix}.batch_norm.running_var"] = rng.uniform(0.5, 2.0, d).astype(np.float32)
    return w


def instantiate(cfg: Workload, centred: bool = False):
    """Draw the workload's weights and inputs. Returns (layers, x, extras):
    layers: list of per-layer weight dicts; x: float32 [B, T, D] (or the first
    chunk for streaming); extras: lengths / fills / per-step chunks."""
    rng = np.random.default_rng(cfg.seed)
    if cfg.module == "block":
        w = make_block_weights(rng, cfg.d_model, cfg.n_heads, cfg.ff_dim, cfg.conv_kernel, cfg.conv_norm)
        extras = {}
        if cfg.cache_size:
            B, C, D = cfg.batch, cfg.cache_size, cfg.d_model
            extras["fills"] = [int(v) for v in rng.integers(0, C + 1, size=B)]
            cache = rng.standard_normal((1, B, C, D)).astype(np.float32)
            for b, fl in enumerate(extras["fills"]):
                cache[:, b, : C - fl] = 0.0
            extras["cache"] = cache
            extras["conv_cache"] = np.zeros((1, B, D, cfg.conv_kernel - 1), dtype=np.float32)
            extras["chunks"] = rng.standard_normal((cfg.steps, B, cfg.seq_len, D)).astype(np.float32)
            return [w], extras["chunks"][0], extras
        extras["lengths"] = [int(v) for v in rng.integers(cfg.seq_len // 2, cfg.seq_len + 1, size=cfg.batch)]
        return [w], rng.standard_normal((cfg.batch, cfg.seq_len, cfg.d_model)).astype(np.float32), extras
    if cfg.module == "conv":
        w = make_conv_weights(rng, cfg.d_model, cfg.conv_kernel, cfg.conv_norm, cfg.quantized, cfg.use_bias)
        extras = {}
        if cfg.steps:  # streaming chunks through the conv cache
            extras["chunks"] = rng.standard_normal((cfg.steps, cfg.batch, cfg.seq_len, cfg.d_model)).astype(np.float32)
            extras["cache"] = np.zeros((cfg.batch, cfg.d_model, cfg.conv_kernel - 1), dtype=np.float32)
            return [w], extras["chunks"][0], extras
        extras["lengths"] = [int(v) for v in rng.integers(cfg.seq_len // 2, cfg.seq_len + 1, size=cfg.batch)]
        return [w], rng.standard_normal((cfg.batch, cfg.seq_len, cfg.d_model)).astype(np.float32), extras
    layers = [make_layer_weights(rng, cfg.d_model, cfg.n_heads, cfg.use_bias, cfg.quantized, centred)
              for _ in range(cfg.layers)]
    extras = {}
    if cfg.cache_size:
        extras["fills"] = [int(v) for v in rng.integers(0, cfg.cache_size + 1, size=cfg.batch)]
        cache = rng.standard_normal((cfg.batch, cfg.cache_size, cfg.d_model)).astype(np.float32)
        for b, f in enumerate(extras["fills"]):
            cache[b, : cfg.cache_size - f] = 0.0  # unfilled rows are zeros, as EncoderCache::new
        extras["cache"] = cache
        extras["chunks"] = rng.standard_normal((cfg.steps, cfg.batch, cfg.seq_len, cfg.d_model)).astype(np.float32)
        return layers, extras["chunks"][0], extras
    if cfg.name == "xl_offline_bf16":
        extras["lengths"] = [int(v) for v in rng.integers(188, 376, size=cfg.batch)]
    elif cfg.name == "xl_stack_u8":
        extras["lengths"] = [int(v) for v in rng.integers(1000, 1501, size=cfg.batch)]
    x = rng.standard_normal((cfg.batch, cfg.seq_len, cfg.d_model)).astype(np.float32)
    return layers, x, extras


def algorithmic_flops(cfg: Workload, lengths=None, fills=None) -> float:
    """Useful MFMA work of one pass: the projections plus 2*D FLOPs per
    (query, visible key) pair for each of QK^T, the surviving part of QP^T
    and PV. Padded queries count, padded keys and masked pairs do not.
    Streaming: one step with projected K/V cached, `fills` the per-session
    cache fill levels that step reads."""
    D, T, B = cfg.d_model, cfg.seq_len, cfg.batch
    if cfg.cache_size:
        pairs = sum(T * (T + f) for f in (fills or [cfg.cache_size] * B))
        return cfg.layers * (2.0 * D * D * (4 * B * T) + 6.0 * D * pairs)
    lens = lengths or [T] * B
    if cfg.context is not None and cfg.context[2] == "regular":
        left, right = cfg.context[0], cfg.context[1]
        pairs = 0
        for ln in lens:
            i = np.arange(T)
            lo = np.maximum(i - left, 0)
            hi = np.minimum(i + right, ln - 1)
            pairs += int(np.maximum(hi - lo + 1, 0).sum())
        pos_rows = cfg.pos_band or (2 * T - 1)
    else:
        pairs = sum(T * ln for ln in lens)
        pos_rows = 2 * T - 1
    return cfg.layers * (2.0 * D * D * (4 * B * T + pos_rows) + 6.0 * D * pairs)


def conv_work(cfg: Workload, tag: str):
    """Algorithmic work of one launch of a ConvolutionModule kernel:
    (amount, "TFLOP/s" | "GB/s", "mfma" | "hbm"). The fused conv kernel
    reads pointwise_conv1's output [rows, 2D], writes [rows, D] and, in
    streaming, reads and rewrites the [B, D, K-1] f32 cache; parameters
    (K + 5) D floats."""
    D, rows, K = cfg.d_model, cfg.batch * cfg.seq_len, cfg.conv_kernel
    es_in = 2 if cfg.dtype == "bfloat16" and not cfg.steps else 4
    es_out = 2 if es_in == 2 and not cfg.causal else 4
    if tag == "pointwise_conv1":
        return 2.0 * rows * 2 * D * D, "TFLOP/s", "mfma"
    if tag == "pointwise_conv2":
        return 2.0 * rows * D * D, "TFLOP/s", "mfma"
    if tag == "conv":
        cache = 2 * 4 * cfg.batch * D * (K - 1) if cfg.steps else 0
        return float(rows * D * (2 * es_in + es_out) + (K + 5) * D * 4 + cache), "GB/s", "hbm"
    if tag == "layer_norm":
        return float(2 * rows * D * es_out), "GB/s", "hbm"
    return None


def conv_flops(cfg: Workload) -> float:
    """Useful work of one ConvolutionModule pass: both pointwise convs and
    the depthwise conv (2 K FLOPs per output element)."""
    D, rows = cfg.d_model, cfg.batch * cfg.seq_len
    return 2.0 * rows * D * (3 * D + cfg.conv_kernel)


def chunk_attention_bytes(cfg: Workload, fills) -> float:
    """Algorithmic HBM bytes of one streaming chunk-attention launch (fp32):
    the chunk's q, the visible cached and new K/V rows, the position rows the
    step reaches and the output."""
    D, T, B, C = cfg.d_model, cfg.seq_len, cfg.batch, cfg.cache_size
    band = 2 * (C + T) - 1
    vis = sum(T + f for f in fills)
    return 4.0 * (2 * B * T * D + 2 * vis * D + band * D)


def algorithmic_bytes(cfg: Workload) -> float:
    """One compulsory read of every input and weight and one write of every output."""
    D, T, B = cfg.d_model, cfg.seq_len, cfg.batch
    es = 2 if cfg.dtype == "bfloat16" else 4
    if cfg.quantized:
        w = 5 * (D * D + 2 * 2 * D * (D // 64))
    else:
        w = 5 * D * D * es
    pos_rows = cfg.pos_band or (2 * T - 1)
    return cfg.layers * (w + 2 * B * T * D * es + pos_rows * D * es)


def block_flops(cfg: Workload, lengths=None, fills=None) -> float:
    """Useful MFMA work of one ConformerBlock pass: both FeedForwards
    (2 x 2 x 2 rows D F), the attention sublayer as algorithmic_flops counts
    it (streaming: K/V of the cache already projected), and the conv module
    as conv_flops counts it."""
    rows = cfg.batch * cfg.seq_len
    return 8.0 * rows * cfg.d_model * cfg.ff_dim + algorithmic_flops(cfg, lengths, fills) + conv_flops(cfg)

