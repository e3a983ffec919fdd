"""The CPU baseline: the reference's rel-pos MHSA op sequence in float32 numpy.

TEST INFRASTRUCTURE ONLY: timed by the `cpu_baseline` leg of `bench.py`; the
product never imports it. (The float64 oracle in `relpos_oracle.py` is what
parity is checked against; this module is the same algorithm run for speed.)

The reference's CPU path is MLX's CPU backend (unavailable offline), where
every matmul is a BLAS sgemm and the rest are elementwise kernels. This
restatement does the same with numpy's OpenBLAS sgemm (all its threads) and
numpy elementwise ops, following the reference as written, overcompute
included:

* `forward` (attention.rs:458-573): q/k/v projections, `linear_pos` over all
  2T-1 table rows, query blocks of `query_block_size` rows (196-206), per
  block bd = (q + v_bias) P_slice^T over T + rows - 1 columns (529-530), the
  pad + reshape `rel_shift` truncated to T (531-532, 832-855), the context
  and padding masks (533-543), softmax(s (q + u_bias) K^T + cast(s) bd +
  mask) V over all T keys (296-318), `linear_out` (558-565);
* `forward_with_cache` (attention.rs:606-816): K/V re-projected over
  [cache; x] (650, 721-722) every step, the projected position rows memoised
  per pos_len (749-761), bd over all 2L-1 columns;
* `sublayer` (conformer.rs:1747-1780): x + MHSA(LayerNorm(x)).

Quantized projections are dequantised once per layer and then run as sgemm
(MLX dequantises inside every quantized matmul), which can only make this
baseline faster than the reference's.
"""
from __future__ import annotations

import math

import numpy as np

MAX_SCORE_ELEMENTS = 1 << 26  # attention.rs:196-197
LINEARS = ("linear_q", "linear_k", "linear_v", "linear_out", "linear_pos")


def threads() -> int:
    """BLAS threads numpy's OpenBLAS runs with."""
    try:
        from threadpoolctl import threadpool_info
        n = [i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"]
        return int(max(n)) if n else 1
    except Exception:
        return 1


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def layer_params(weights, dtype_bf16: bool = False):
    """float32 parameter arrays of one layer from a checkpoint-style dict
    (`linear_q.weight`, ... , `pos_bias_u`); quantized projections dequantised
    (W = s q + b per group of 64, quantization.rs:1-8) and, like every weight
    of a bf16 model, held at their bf16 values when `dtype_bf16`."""
    def bf(a):
        if not dtype_bf16:
            return a
        u = a.view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)

    out = {}
    for name in LINEARS:
        if f"{name}.scales" in weights:
            w = np.asarray(weights[f"{name}.weight"], dtype=np.uint32)
            codes = np.stack([(w >> (8 * i)) & 0xFF for i in range(4)], axis=-1).reshape(w.shape[0], -1)
            s = bf(_f32(weights[f"{name}.scales"]))
            b = bf(_f32(weights[f"{name}.biases"]))
            wt = codes.astype(np.float32) * np.repeat(s, 64, axis=1) + np.repeat(b, 64, axis=1)
        else:
            wt = _f32(weights[f"{name}.weight"])
        out[f"{name}.weight"] = bf(_f32(wt))
        bias = weights.get(f"{name}.bias")
        out[f"{name}.bias"] = None if bias is None else bf(_f32(bias))
    out["pos_bias_u"] = bf(_f32(weights["pos_bias_u"]).reshape(-1))
    out["pos_bias_v"] = bf(_f32(weights["pos_bias_v"]).reshape(-1))
    return out


def _linear(x, w, b):
    y = x @ w.T
    return y + b if b is not None else y


def _heads(t, h):
    b, n, d = t.shape
    return t.reshape(b, n, h, d // h).transpose(0, 2, 1, 3)


def _rel_shift(x):
    """Pad one zero column left, view [P+1, rows], drop row 0 (attention.rs:832-855)."""
    *lead, rows, pos_len = x.shape
    xp = np.concatenate([np.zeros(tuple(lead) + (rows, 1), np.float32), x], axis=-1)
    return xp.reshape(tuple(lead) + (pos_len + 1, rows))[..., 1:, :].reshape(tuple(lead) + (rows, pos_len))


def _softmax_v(scores, v):
    m = scores.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, np.float32(0.0))
    e = np.exp(scores - m)
    return (e / e.sum(axis=-1, keepdims=True)) @ v


def _context_mask(ctx, start, end, seq_len):
    """attention.rs:229-272 (ctx = (left, right, chunked))."""
    if ctx is None:
        return None
    left, right, chunked = ctx
    i = np.arange(start, end).reshape(-1, 1)
    j = np.arange(seq_len).reshape(1, -1)
    if chunked and right >= 0:
        chunk = right + 1
        lc = left // chunk if left >= 0 else 10000
        d = i // chunk - j // chunk
        vis = (d >= 0) & (d <= lc)
    else:
        vis = (j - i >= -max(left, 0)) if left >= 0 else np.ones((end - start, seq_len), bool)
        if not chunked and right >= 0:
            vis &= j - i <= right
    return np.where(vis, np.float32(0.0), np.float32(-np.inf))


def forward(P, n_heads, x, pos_emb, ctx=None, lengths=None, scale_bd=None):
    """attention.rs:446-573 as written. x [B,T,D] f32, pos_emb [2T-1, D]."""
    x = _f32(x)
    B, T, D = x.shape
    h, dk = n_heads, D // n_heads
    scale = np.float32(1.0) / np.sqrt(np.float32(dk))
    sbd = np.float32(scale if scale_bd is None else scale_bd)
    q = _heads(_linear(x, P["linear_q.weight"], P["linear_q.bias"]), h)
    k = _heads(_linear(x, P["linear_k.weight"], P["linear_k.bias"]), h)
    v = _heads(_linear(x, P["linear_v.weight"], P["linear_v.bias"]), h)
    pp = _heads(_linear(_f32(pos_emb).reshape(1, -1, D), P["linear_pos.weight"], None), h)
    q_u = q + P["pos_bias_u"].reshape(1, h, 1, dk)
    q_v = q + P["pos_bias_v"].reshape(1, h, 1, dk)
    p_t = np.swapaxes(pp, -1, -2)
    kt = np.swapaxes(k, -1, -2)
    kmask = None
    if lengths is not None and not all(int(n) >= T for n in lengths):
        lens = np.array([max(int(n), 1) for n in lengths]).reshape(-1, 1, 1, 1)
        kmask = np.where(np.arange(T).reshape(1, 1, 1, T) < lens, np.float32(0.0), np.float32(-np.inf))
    block = int(min(max(MAX_SCORE_ELEMENTS // max(B * h * 2 * T, 1), 1), T))  # 196-206
    outs = []
    for start in range(0, T, block):
        end = min(start + block, T)
        bd = q_v[:, :, start:end] @ p_t[..., T - end:2 * T - 1 - start]
        bd = _rel_shift(bd)[..., :T]
        mask = bd * sbd
        cm = _context_mask(ctx, start, end, T)
        if cm is not None:
            mask = mask + cm
        if kmask is not None:
            mask = mask + kmask
        outs.append(_softmax_v(scale * (q_u[:, :, start:end] @ kt) + mask, v))
    o = np.concatenate(outs, axis=2).transpose(0, 2, 1, 3).reshape(B, T, D)
    return _linear(o, P["linear_out.weight"], P["linear_out.bias"])


def layer_norm(x, eps=1e-5):
    mu = x.mean(axis=-1, keepdims=True)
    d = x - mu
    return d / np.sqrt((d * d).mean(axis=-1, keepdims=True) + np.float32(eps))


def sublayer(P, n_heads, x, pos_emb, ctx=None, lengths=None, scale_bd=None):
    """x + MHSA(LayerNorm(x)) (conformer.rs:1747-1780), gamma = 1, beta = 0."""
    return x + forward(P, n_heads, layer_norm(x), pos_emb, ctx, lengths, scale_bd)


class Streamer:
    """forward_with_cache (attention.rs:606-816) for a batch of sessions with
    one additive mask per step (the reference builds it from session 0's fill,
    conformer.rs:883-927); keeps the cache [B, C, D] and the position memo."""

    def __init__(self, P, n_heads, cache, pos_emb, ctx):
        self.P, self.h = P, n_heads
        self.cache = _f32(cache)
        self.pos = _f32(pos_emb)
        self.ctx = ctx
        self.memo = None  # attention.rs:749-761

    def step(self, x, filled):
        P, h = self.P, self.h
        x = _f32(x)
        B, T, D = x.shape
        C = self.cache.shape[1]
        L = C + T
        dk = D // h
        scale = np.float32(1.0) / np.sqrt(np.float32(dk))
        kv_in = np.concatenate([self.cache, x], axis=1)  # 650
        q = _heads(_linear(x, P["linear_q.weight"], P["linear_q.bias"]), h)
        k = _heads(_linear(kv_in, P["linear_k.weight"], P["linear_k.bias"]), h)  # 721
        v = _heads(_linear(kv_in, P["linear_v.weight"], P["linear_v.bias"]), h)  # 722
        if self.memo is None:
            self.memo = np.swapaxes(_heads(_linear(self.pos.reshape(1, -1, D), P["linear_pos.weight"], None), h), -1, -2)
        q_u = q + P["pos_bias_u"].reshape(1, h, 1, dk)
        q_v = q + P["pos_bias_v"].reshape(1, h, 1, dk)
        bd = _rel_shift(q_v @ self.memo)[..., :L]  # 770-772
        mask = bd * scale
        cm = _context_mask(self.ctx, C, L, L)
        if cm is not None:
            mask = mask + cm
        if filled < C:  # the unfilled cache offset (conformer.rs:155-181)
            mask = mask + np.where(np.arange(L) >= C - filled, np.float32(0.0), np.float32(-np.inf))
        o = _softmax_v(scale * (q_u @ np.swapaxes(k, -1, -2)) + mask, v)
        out = _linear(o.transpose(0, 2, 1, 3).reshape(B, T, D), P["linear_out.weight"], P["linear_out.bias"])
        self.cache = np.concatenate([self.cache[:, T:], x], axis=1)  # 670-676 (cache_drop_size 0)
        return out


# ---------------------------------------------------------------------------
# ConvolutionModule (conformer.rs:2105-2437)
# ---------------------------------------------------------------------------

def conv_params(weights, dtype_bf16: bool = False, prefix: str = "conv"):
    """float32 parameters of a ConvolutionModule from checkpoint-style tensors,
    at bf16 values for a bf16 model, as f32 activations meet them: quantized
    pointwise convs dequantised in f32 from the cast scales and biases; the
    BatchNorm rsqrt(var + eps) term precomputed in the parameter dtype."""
    def bf(a):
        a = _f32(a)
        if not dtype_bf16:
            return a
        u = a.view(np.uint32).astype(np.uint64)
        return ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)

    out = {}
    for name in ("pointwise_conv1", "pointwise_conv2"):
        k = f"{prefix}.{name}"
        if f"{k}.scales" in weights:
            w = np.asarray(weights[f"{k}.weight"], dtype=np.uint32)
            codes = np.stack([(w >> (8 * i)) & 0xFF for i in range(4)], axis=-1).reshape(w.shape[0], -1)
            s, b = bf(weights[f"{k}.scales"]), bf(weights[f"{k}.biases"])
            # dequantised in f32 from the cast scales and biases (the promoted path)
            out[f"{name}.weight"] = codes.astype(np.float32) * np.repeat(s, 64, axis=1) + np.repeat(b, 64, axis=1)
        else:
            out[f"{name}.weight"] = bf(weights[f"{k}.weight"])
        bias = weights.get(f"{k}.bias")
        out[f"{name}.bias"] = None if bias is None else bf(bias)
    out["taps"] = bf(np.asarray(weights[f"{prefix}.depthwise_conv.weight"])[:, :, 0].T)  # [K, D]
    dwb = weights.get(f"{prefix}.depthwise_conv.bias")
    out["taps_bias"] = None if dwb is None else bf(dwb)
    out["norm_weight"] = bf(weights[f"{prefix}.batch_norm.weight"])
    out["norm_bias"] = bf(weights[f"{prefix}.batch_norm.bias"])
    if f"{prefix}.batch_norm.running_var" in weights:
        out["mean"] = bf(weights[f"{prefix}.batch_norm.running_mean"])
        out["inv"] = bf(1.0 / np.sqrt(bf(bf(weights[f"{prefix}.batch_norm.running_var"]) + bf(np.float32(1e-5)))))
    return out


def conv_module(P, x, lengths=None, cache=None, causal=False):
    """ConvolutionModule::forward / forward_with_cache (conformer.rs:2197-2291,
    2305-2378): pointwise_conv1 (sgemm), GLU, padding frames zeroed, the
    depthwise conv as K shifted multiply-adds over the zero- or cache-padded
    sequence, BatchNorm or LayerNorm, SiLU, pointwise_conv2. cache [B, D, K-1]
    is returned updated."""
    b_, t_, d_ = x.shape
    k = P["taps"].shape[0]
    h = _linear(x, P["pointwise_conv1.weight"], P["pointwise_conv1.bias"])
    u = h[..., :d_] * (np.float32(1.0) / (np.float32(1.0) + np.exp(-h[..., d_:])))
    if lengths is not None:
        u = u * (np.arange(t_)[None, :, None] < np.asarray(lengths)[:, None, None])
    new_cache = None
    if cache is not None:
        seq = np.concatenate([cache.transpose(0, 2, 1), u], axis=1)
        new_cache = np.ascontiguousarray(seq[:, seq.shape[1] - (k - 1):].transpose(0, 2, 1))
    elif causal:
        seq = np.concatenate([np.zeros((b_, k - 1, d_), np.float32), u], axis=1)
    else:
        p = (k - 1) // 2
        seq = np.concatenate([np.zeros((b_, p, d_), np.float32), u, np.zeros((b_, p, d_), np.float32)], axis=1)
    y = seq[:, 0:t_] * P["taps"][0]
    for j in range(1, k):
        y += seq[:, j:j + t_] * P["taps"][j]
    if P["taps_bias"] is not None:
        y += P["taps_bias"]
    if "inv" in P:
        y = ((y - P["mean"]) * P["inv"]) * P["norm_weight"] + P["norm_bias"]
    else:
        y = layer_norm(y) * P["norm_weight"] + P["norm_bias"]
    y = y * (np.float32(1.0) / (np.float32(1.0) + np.exp(-y)))
    return _linear(y, P["pointwise_conv2.weight"], P["pointwise_conv2.bias"]), new_cache


# ---------------------------------------------------------------------------
# ConformerBlock (conformer.rs:1693-1971)
# ---------------------------------------------------------------------------

def _bf16_values(a):
    u = _f32(a).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)


def block_params(weights, prefix: str = "blk", dtype_bf16: bool = False):
    """float32 parameters of a ConformerBlock from checkpoint-style tensors
    (at bf16 values for a bf16 model): both FeedForwards, the attention layer
    (layer_params), the conv module (conv_params) and the five LayerNorms."""
    bf = _bf16_values if dtype_bf16 else _f32
    out = {}
    for ff in ("feed_forward1", "feed_forward2"):
        out[ff] = {n: (bf(weights[f"{prefix}.{ff}.{n}.weight"]), bf(weights[f"{prefix}.{ff}.{n}.bias"]))
                   for n in ("linear1", "linear2")}
    att = {k[len(prefix) + len(".self_attn."):]: v for k, v in weights.items() if k.startswith(f"{prefix}.self_attn.")}
    out["attn"] = layer_params(att, dtype_bf16)
    out["conv"] = conv_params(weights, dtype_bf16, f"{prefix}.conv")
    out["norms"] = [(bf(weights[f"{prefix}.{n}.weight"]), bf(weights[f"{prefix}.{n}.bias"]))
                    for n in ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out")]
    return out


def ffn(P, x):
    """FeedForward::forward (conformer.rs:2066-2072): linear2(silu(linear1(x)))."""
    h = _linear(x, *P["linear1"])
    return _linear(h * (np.float32(1.0) / (np.float32(1.0) + np.exp(-h))), *P["linear2"])


def _ln(x, nw):
    return layer_norm(x) * nw[0] + nw[1]


def block(P, n_heads, x, pos_emb, ctx=None, lengths=None, causal=False):
    """ConformerBlock::forward (conformer.rs:1693-1875)."""
    half = np.float32(0.5)
    n = P["norms"]
    x = x + half * ffn(P["feed_forward1"], _ln(x, n[0]))
    x = x + forward(P["attn"], n_heads, _ln(x, n[1]), pos_emb, ctx, lengths)
    x = x + conv_module(P["conv"], _ln(x, n[2]), lengths, None, causal)[0]
    x = x + half * ffn(P["feed_forward2"], _ln(x, n[3]))
    return _ln(x, n[4])


class BlockStreamer:
    """ConformerBlock::forward_with_cache (conformer.rs:1893-1971) for a batch
    of sessions: the attention as Streamer (K/V re-projected over [cache; x]
    every step) and the conv cache [B, D, K-1]."""

    def __init__(self, P, n_heads, att_cache, conv_cache, pos_emb, ctx):
        self.P = P
        self.att = Streamer(P["attn"], n_heads, att_cache, pos_emb, ctx)
        self.conv_cache = _f32(conv_cache)

    def step(self, x, filled):
        half = np.float32(0.5)
        n = self.P["norms"]
        x = x + half * ffn(self.P["feed_forward1"], _ln(x, n[0]))
        x = x + self.att.step(_ln(x, n[1]), filled)
        y, self.conv_cache = conv_module(self.P["conv"], _ln(x, n[2]), None, self.conv_cache, True)
        x = x + y
        x = x + half * ffn(self.P["feed_forward2"], _ln(x, n[3]))
        return _ln(x, n[4])
