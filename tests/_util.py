"""Helpers shared by the test modules (not a test module itself)."""
from __future__ import annotations

import numpy as np

import relpos_oracle as O

LINEARS = ("linear_q", "linear_k", "linear_v", "linear_out", "linear_pos")


def oracle_params(weights, d_model, n_heads, cache_drop_size=0) -> O.MhsaParams:
    """Oracle view of a workload weight dict (keys `linear_q.weight`, ...)."""
    lin = {}
    for name in LINEARS:
        if f"{name}.scales" in weights:
            lin[name] = O.LinearLayer(weights[f"{name}.weight"], weights.get(f"{name}.bias"),
                                      weights[f"{name}.scales"], weights[f"{name}.biases"])
        else:
            lin[name] = O.LinearLayer(np.asarray(weights[f"{name}.weight"], dtype=np.float64),
                                      weights.get(f"{name}.bias"))
    return O.MhsaParams(d_model, n_heads, lin["linear_q"], lin["linear_k"], lin["linear_v"], lin["linear_out"],
                        lin["linear_pos"], np.asarray(weights["pos_bias_u"], dtype=np.float64),
                        np.asarray(weights["pos_bias_v"], dtype=np.float64), cache_drop_size)


def rel_err(got, ref, mask=None) -> float:
    """max |got - ref| / max |ref| over the selected rows."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if mask is not None:
        got, ref = got[mask], ref[mask]
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))


def row_rel_err(got, ref, mask=None) -> float:
    """max over rows (last axis) of max |got - ref| / max |ref| within the row:
    the relative error of each output row, read separately."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if mask is not None:
        got, ref = got[mask], ref[mask]
    d = np.max(np.abs(got - ref), axis=-1)
    r = np.max(np.abs(ref), axis=-1)
    return float(np.max(d / np.maximum(r, 1e-30)))


def abs_err(got, ref, mask=None) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if mask is not None:
        got, ref = got[mask], ref[mask]
    return float(np.max(np.abs(got - ref)))


def bf16_abs_excess(got, ref, tol) -> tuple[float, int]:
    """The bf16 absolute bound read on the bf16 grid: each output within
    max(tol, one bf16 ulp of its reference value) (above |x| = 4 one ulp is
    0.03125, so a value there either equals the reference or lies at least
    one ulp away). Returns (max of |got - ref| / that bound, number of outputs
    farther than tol)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    _, e = np.frexp(np.abs(ref))
    bound = np.maximum(tol, np.ldexp(1.0, e - 8))
    d = np.abs(got - ref)
    return float(np.max(d / bound)), int(np.sum(d > tol))


def random_weights(rng, d_model, n_heads, use_bias=True, scale=None, quantized=False):
    """Random layer weights (Xavier-like unless `scale`), keyed like a checkpoint."""
    import workloads as W
    w = W.make_layer_weights(rng, d_model, n_heads, use_bias, quantized)
    if use_bias and not quantized:
        for name in LINEARS[:4]:
            w[f"{name}.bias"] = (rng.standard_normal(d_model) * 0.1).astype(np.float32)
    if scale is not None and not quantized:
        for name in LINEARS:
            w[f"{name}.weight"] = (rng.standard_normal((d_model, d_model)) * scale).astype(np.float32)
    w["pos_bias_u"] = (rng.standard_normal(w["pos_bias_u"].shape) * 0.3).astype(np.float32)
    w["pos_bias_v"] = (rng.standard_normal(w["pos_bias_v"].shape) * 0.3).astype(np.float32)
    return w


def conv_weights(rng, d, k, norm="batch_norm", quant=False, use_bias=True, prefix="conv"):
    """ConvolutionModule tensors keyed like a checkpoint (the workloads' generator)."""
    import workloads as W
    return W.make_conv_weights(rng, d, k, norm, quant, use_bias, prefix)


def conv_oracle(w, norm="batch_norm", causal=False, prefix="conv") -> O.ConvModuleParams:
    """Oracle view of `conv_weights` tensors."""
    lin = []
    for name in ("pointwise_conv1", "pointwise_conv2"):
        k = f"{prefix}.{name}"
        if f"{k}.scales" in w:
            lin.append(O.LinearLayer(w[f"{k}.weight"], w.get(f"{k}.bias"), w[f"{k}.scales"], w[f"{k}.biases"]))
        else:
            lin.append(O.LinearLayer(np.asarray(w[f"{k}.weight"], np.float64), w.get(f"{k}.bias")))
    g = lambda n: w.get(f"{prefix}.{n}")
    return O.ConvModuleParams(lin[0], np.asarray(g("depthwise_conv.weight"), np.float64), g("depthwise_conv.bias"),
                              lin[1], norm, g("batch_norm.weight"), g("batch_norm.bias"),
                              g("batch_norm.running_mean"), g("batch_norm.running_var"), causal)


def ffn_weights(rng, d, f, quant, prefix="ff", use_bias=True):
    """FeedForward linear1 [f, d], linear2 [d, f] keyed like a checkpoint:
    dense Xavier, or affine u8 with zero-mean weights (scales U(1e-4, 1e-3))
    so activations stay O(1); biases N(0, 0.1)."""
    import workloads as W
    w = {}
    for name, (o, i) in (("linear1", (f, d)), ("linear2", (d, f))):
        if quant:
            codes = rng.integers(0, 256, size=(o, i))
            sc = rng.uniform(1e-4, 1e-3, size=(o, i // 64)).astype(np.float16)
            w[f"{prefix}.{name}.weight"] = W.pack_u8(codes)
            w[f"{prefix}.{name}.scales"] = sc
            w[f"{prefix}.{name}.biases"] = (-128.0 * sc.astype(np.float64)
                                            + rng.normal(0, 1e-3, sc.shape)).astype(np.float16)
            if use_bias:
                w[f"{prefix}.{name}.bias"] = rng.normal(0, 0.1, o).astype(np.float16)
        else:
            w[f"{prefix}.{name}.weight"] = W.xavier(rng, o, i)
            if use_bias:
                w[f"{prefix}.{name}.bias"] = rng.normal(0, 0.1, o).astype(np.float32)
    return w


def ffn_oracle(w, prefix="ff"):
    lin = []
    for name in ("linear1", "linear2"):
        k = f"{prefix}.{name}"
        if f"{k}.scales" in w:
            lin.append(O.LinearLayer(w[f"{k}.weight"], w.get(f"{k}.bias"), w[f"{k}.scales"], w[f"{k}.biases"]))
        else:
            lin.append(O.LinearLayer(np.asarray(w[f"{k}.weight"], np.float64), w.get(f"{k}.bias")))
    return O.FeedForwardParams(*lin)


BLOCK_NORMS = ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out")


def block_weights(rng, d, h, f, k, norm="batch_norm", quant=False, prefix="blk"):
    """One ConformerBlock's tensors keyed like a checkpoint
    (conformer.rs:1977-2028): feed_forward1/2, self_attn (quantized ones
    zero-mean, so the attention stays well conditioned), conv and the five
    LayerNorms (weight 1 + N(0, 0.1), bias N(0, 0.1))."""
    import workloads as W
    w = {}
    w.update(ffn_weights(rng, d, f, quant, f"{prefix}.feed_forward1"))
    att = W.make_layer_weights(rng, d, h, True, quant)
    if quant:  # zero-mean codes: scales U(1e-4, 1e-3), biases -128 s + N(0, 1e-3)
        for name in LINEARS:
            sc = rng.uniform(1e-4, 1e-3, size=att[f"{name}.scales"].shape).astype(np.float16)
            att[f"{name}.scales"] = sc
            att[f"{name}.biases"] = (-128.0 * sc.astype(np.float64) + rng.normal(0, 1e-3, sc.shape)).astype(np.float16)
    else:
        for name in LINEARS[:4]:
            att[f"{name}.bias"] = (rng.standard_normal(d) * 0.1).astype(np.float32)
    w.update(W.prefixed(att, f"{prefix}.self_attn"))
    w.update(conv_weights(rng, d, k, norm, quant, True, f"{prefix}.conv"))
    w.update(ffn_weights(rng, d, f, quant, f"{prefix}.feed_forward2"))
    for n in BLOCK_NORMS:
        w[f"{prefix}.{n}.weight"] = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
        w[f"{prefix}.{n}.bias"] = (0.1 * rng.standard_normal(d)).astype(np.float32)
    return w


def block_oracle(w, d, h, norm="batch_norm", causal=False, prefix="blk") -> O.ConformerBlockParams:
    """Oracle view of `block_weights` tensors."""
    att = {k[len(prefix) + len(".self_attn."):]: v for k, v in w.items() if k.startswith(f"{prefix}.self_attn.")}
    nrm = lambda n: (np.asarray(w[f"{prefix}.{n}.weight"], np.float64), np.asarray(w[f"{prefix}.{n}.bias"], np.float64))
    return O.ConformerBlockParams(ffn_oracle(w, f"{prefix}.feed_forward1"), nrm(BLOCK_NORMS[0]), oracle_params(att, d, h),
                                  nrm(BLOCK_NORMS[1]), conv_oracle(w, norm, causal, f"{prefix}.conv"),
                                  nrm(BLOCK_NORMS[2]), ffn_oracle(w, f"{prefix}.feed_forward2"), nrm(BLOCK_NORMS[3]),
                                  nrm(BLOCK_NORMS[4]))

