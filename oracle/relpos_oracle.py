"""CPU oracle for the FastConformer rel-pos multi-head self-attention path.

TEST INFRASTRUCTURE ONLY. This module is the oracle: it may be imported by
`tests/`, by `__graft_entry__.smoke()` and by the `cpu_baseline` leg of
`bench.py`, and by nothing else. The product (the HIP library under
`mlx-nemo-rs_amd/`) never calls it and has no CPU fallback.

It restates, in float64 numpy, the reference algorithm *as written* in
animaslabs/mlx-nemo-rs (crate `mlx-voice` 0.3.0):

* `src/asr/modules/encoders/attention.rs` (rel-pos table, query-blocked
  offline attention, cache-aware streaming attention, context and padding
  masks, `rel_shift` as pad + reshape + slice),
* `src/core/quantization.rs` (standard and MLX affine 8-bit linear layers),
* `src/asr/modules/encoders/conformer.rs` (streaming mask builder, cache
  pad/truncate, fill bookkeeping, the pre-LN + residual MHSA sublayer).

Each function cites the reference lines it follows. Two dtype modes:

* ``"float32"``: every op is evaluated in float64 with no intermediate
  rounding (the f32 reference differs from it by f32 rounding only).
* ``"bfloat16"``: values are rounded to bfloat16 (round-to-nearest-even) at
  every point where the reference materialises a bf16 MLX array (linear
  outputs, bias adds, `matrix_bd`, the scaled mask, attention context). The
  softmax itself is float64: MLX's internal SDPA precision is not observable
  without MLX, so it is parity-unpinned at ULP level (pinned only through the
  invariants the reference's own tests assert).

Which parts are pinned, and by what, is listed in the header of each test
module under `tests/` (test_oracle_*.py).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np

F32 = "float32"
BF16 = "bfloat16"
NEG_INF = float("-inf")

# attention.rs:196-197
MAX_SCORE_ELEMENTS = 1 << 26


# ---------------------------------------------------------------------------
# dtype emulation
# ---------------------------------------------------------------------------

def bf16_round(x) -> np.ndarray:
    """Round to bfloat16 (RNE) and return the value as float64.

    Goes through float32 first, as MLX does when an f32 result is stored into
    a bf16 array. Infinities pass through; the path produces no NaNs.
    """
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = r.astype(np.uint32).view(np.float32).astype(np.float64)
    inf = np.isinf(a)
    if inf.any():
        out[inf] = a[inf]
    return out


def to_dtype(x, dtype: str) -> np.ndarray:
    """Value of `x` after a cast to the reference dtype (`as_dtype`)."""
    if dtype == BF16:
        return bf16_round(x)
    return np.asarray(x, dtype=np.float64)


def bf16_bits(x) -> np.ndarray:
    """uint16 bit patterns of bf16(x) (RNE), for uploading bf16 tensors."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    return r.astype(np.uint16)


def _rnd(x, dtype):
    """Round an op result the way the reference stores it in `dtype`."""
    return bf16_round(x) if dtype == BF16 else x


# ---------------------------------------------------------------------------
# a1: sinusoidal relative positional encoding (attention.rs:19-194)
# ---------------------------------------------------------------------------

def create_pe(d_model: int, max_len: int) -> np.ndarray:
    """NeMo rel-pos table [1, 2*max_len-1, d_model] as float32.

    attention.rs:59-103: positions max_len-1 .. -(max_len-1) (63-67); div_term
    exp(-(i) * ln(10000)/d) evaluated in host f32 (70-74); angles as an f32
    broadcast multiply (77-79); pe[:, 0::2] = sin, pe[:, 1::2] = cos (82-89).
    sin/cos are evaluated in float64 on the f32 angle and rounded to f32.
    """
    pe_len = 2 * max_len - 1
    positions = np.arange(max_len - 1, -max_len, -1, dtype=np.float32).reshape(pe_len, 1)
    ln = np.float32(np.log(np.float32(10000.0)))
    step = np.float32(ln / np.float32(d_model))
    i = np.arange(0, d_model, 2, dtype=np.float32)
    div = np.exp((-i * step).astype(np.float32)).astype(np.float32).reshape(1, d_model // 2)
    angles = (positions * div).astype(np.float32)
    a64 = angles.astype(np.float64)
    pe = np.empty((pe_len, d_model), dtype=np.float32)
    pe[:, 0::2] = np.sin(a64).astype(np.float32)
    pe[:, 1::2] = np.cos(a64).astype(np.float32)
    return pe.reshape(1, pe_len, d_model)


class RelPositionalEncoding:
    """attention.rs:19-194 (`new` 35-51, `get_encoding` 131-177)."""

    def __init__(self, d_model: int, max_len: int, xscaling: bool):
        self.d_model = d_model
        self.max_len = max_len
        # attention.rs:36-40
        self.xscale = float(np.sqrt(np.float32(d_model))) if xscaling else 1.0
        self.pe = create_pe(d_model, max_len)

    def get_encoding(self, seq_len: int) -> np.ndarray:
        if seq_len == 0:  # attention.rs:132-136
            raise ValueError("positional encoding requested for an empty sequence")
        if seq_len > self.max_len:  # attention.rs:137-145: regenerate
            return create_pe(self.d_model, seq_len)
        start = self.max_len - seq_len  # attention.rs:158-174
        end = self.max_len + seq_len - 1
        return self.pe[:, start:end, :]


# ---------------------------------------------------------------------------
# a6, a8, a9: blocking and masks
# ---------------------------------------------------------------------------

def query_block_size(batch_heads: int, seq_len: int, max_score_elements: int) -> int:
    """attention.rs:200-206."""
    per_row = batch_heads * 2 * seq_len
    return int(min(max(max_score_elements // max(per_row, 1), 1), max(seq_len, 1)))


@dataclass(frozen=True)
class AttentionContext:
    """attention.rs:208-273 (NeMo `_create_masks` for offline attention)."""

    left: int
    right: int
    chunked: bool

    @staticmethod
    def new(size: Tuple[int, int], style: str) -> Optional["AttentionContext"]:
        left, right = size
        if left >= 0 or right >= 0:  # attention.rs:220-227
            return AttentionContext(left, right, style == "chunked_limited")
        return None

    def block_visible(self, start: int, end: int, seq_len: int) -> np.ndarray:
        """Boolean visibility [rows, seq_len] (attention.rs:238-269)."""
        rows = np.arange(start, end, dtype=np.int64).reshape(end - start, 1)
        cols = np.arange(0, seq_len, dtype=np.int64).reshape(1, seq_len)
        if self.chunked and self.right >= 0:
            chunk = self.right + 1
            left_chunks = self.left // chunk if self.left >= 0 else 10000
            diff = rows // chunk - cols // chunk
            return (diff >= 0) & (diff <= left_chunks)
        offset = cols - rows
        visible = offset >= -max(self.left, 0)
        if self.left < 0:
            visible = np.ones_like(visible)
        if not self.chunked and self.right >= 0:
            visible = visible & (offset <= self.right)
        return visible

    def block_mask(self, start: int, end: int, seq_len: int) -> np.ndarray:
        """Additive 0 / -inf mask [rows, seq_len] (attention.rs:229-272)."""
        return np.where(self.block_visible(start, end, seq_len), 0.0, NEG_INF)


def key_padding_mask(lengths, seq_len: int) -> Optional[np.ndarray]:
    """[B,1,1,seq_len] additive mask, None if nothing is padding (attention.rs:280-294)."""
    lengths = [int(v) for v in lengths]
    if all(v >= seq_len for v in lengths):
        return None
    lens = np.array([max(v, 1) for v in lengths], dtype=np.int64).reshape(-1, 1, 1, 1)
    frames = np.arange(seq_len, dtype=np.int64).reshape(1, 1, 1, seq_len)
    return np.where(frames < lens, 0.0, NEG_INF)


# ---------------------------------------------------------------------------
# a7: Transformer-XL rel_shift (attention.rs:818-855)
# ---------------------------------------------------------------------------

def rel_shift(x: np.ndarray) -> np.ndarray:
    """Pad one zero column on the left, view as [pos_len+1, rows], drop the
    first row, view back as [rows, pos_len] (attention.rs:832-855)."""
    *lead, rows, pos_len = x.shape
    pad = np.zeros(tuple(lead) + (rows, 1), dtype=x.dtype)
    xp = np.concatenate([pad, x], axis=-1)
    xr = xp.reshape(tuple(lead) + (pos_len + 1, rows))
    xs = xr[..., 1:, :]
    return np.ascontiguousarray(xs).reshape(tuple(lead) + (rows, pos_len))


# ---------------------------------------------------------------------------
# a2, a3: linear layers (quantization.rs:36-162)
# ---------------------------------------------------------------------------

def unpack_codes(w_u32: np.ndarray, bits: int = 8) -> np.ndarray:
    """MLX packing: element k of a row sits in word k // (32/bits) at bit
    offset (k % (32/bits)) * bits, lowest bits first (quantization.rs:1-8)."""
    per = 32 // bits
    mask = (1 << bits) - 1
    w = w_u32.astype(np.uint64)
    parts = [(w >> (bits * p)) & mask for p in range(per)]
    codes = np.stack(parts, axis=-1)  # [N, K/per, per]
    return codes.reshape(w_u32.shape[0], w_u32.shape[1] * per).astype(np.int64)


def dequantize(w_u32, scales, biases, bits: int = 8, group_size: int = 64,
               dtype: str = F32, store: Optional[str] = None) -> np.ndarray:
    """Affine dequantisation W[n,k] = s[n,k/g] * q[n,k] + b[n,k/g].

    quantization.rs:1-8 (layout), 100-111 (`cast`: in bf16 mode the f16
    scales and biases are cast to bf16 first), 147-155 (`quantized_matmul`).
    Evaluated in f32: the f32 product of an f16/bf16 scale and an 8-bit code is
    exact, so the f32 sum has a single rounding and is unique with or without
    an fma. In bf16 mode the weight is then stored as bf16 (RNE), unless
    `store` is F32 (an f32 input promotes the op to f32, below).
    """
    codes = unpack_codes(np.asarray(w_u32, dtype=np.uint32), bits).astype(np.float32)
    s = np.asarray(scales, dtype=np.float32)
    b = np.asarray(biases, dtype=np.float32)
    if dtype == BF16:
        s = bf16_round(s).astype(np.float32)
        b = bf16_round(b).astype(np.float32)
    s_full = np.repeat(s, group_size, axis=1)
    b_full = np.repeat(b, group_size, axis=1)
    w = (s_full * codes).astype(np.float32) + b_full  # f32 product (exact), f32 sum
    w = w.astype(np.float32)
    if (store or dtype) == BF16:
        return bf16_round(w)
    return w.astype(np.float64)


@dataclass
class LinearLayer:
    """quantization.rs:36-59. Standard: weight [out,in] (+ bias). Quantized:
    packed u32 weight [out, in*bits/32], f16 scales/biases [out, in/group]."""

    weight: np.ndarray
    bias: Optional[np.ndarray] = None
    scales: Optional[np.ndarray] = None
    biases: Optional[np.ndarray] = None
    bits: int = 8
    group_size: int = 64

    @property
    def is_quantized(self) -> bool:
        return self.scales is not None

    def dense_weight(self, dtype: str) -> np.ndarray:
        """Weight values the matmul consumes after `cast(dtype)` (quantization.rs:92-114)."""
        if self.is_quantized:
            return dequantize(self.weight, self.scales, self.biases, self.bits,
                              self.group_size, dtype)
        return to_dtype(self.weight, dtype)

    def forward(self, x: np.ndarray, dtype: str = F32) -> np.ndarray:
        """quantization.rs:126-162: y = x W^T (+ bias); each MLX op's bf16 result is rounded."""
        w = self.dense_weight(dtype)
        y = _rnd(np.matmul(x, w.T), dtype)
        if self.bias is not None:
            y = _rnd(y + to_dtype(self.bias, dtype), dtype)
        return y

    def promoted_weight(self, dtype: str) -> np.ndarray:
        """The weight an f32 input meets after `cast(dtype)`: MLX promotes the
        op to f32, so a dense weight is its `dtype` value and a quantized one
        s*q + b evaluated in f32 from the cast scales and biases, not rounded
        to bf16 afterwards (quantization.rs:92-114, 147-155)."""
        if self.is_quantized:
            return dequantize(self.weight, self.scales, self.biases, self.bits, self.group_size, dtype, store=F32)
        return to_dtype(self.weight, dtype)

    def forward_promoted(self, x: np.ndarray, dtype: str = F32) -> np.ndarray:
        """quantization.rs:126-162 on an f32 input with the parameters cast to
        `dtype`: matmul and bias add promote to f32, so nothing is rounded to
        bf16. Equal to `forward` when dtype is F32."""
        y = np.matmul(x, self.promoted_weight(dtype).T)
        if self.bias is not None:
            y = y + to_dtype(self.bias, dtype)
        return y


# ---------------------------------------------------------------------------
# a10: attend (attention.rs:296-318)
# ---------------------------------------------------------------------------

def f32_scale(head_dim: int) -> float:
    """1/sqrt(d_k) computed in f32 (attention.rs:307)."""
    return float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))


def _softmax(scores: np.ndarray) -> np.ndarray:
    m = np.max(scores, axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    e = np.exp(scores - m)
    return e / np.sum(e, axis=-1, keepdims=True)


def position_term(matrix_bd, additive_mask, head_dim: int, dtype: str):
    """The additive mask `attend` hands to the attention: bd * cast(s), stored
    in the bd dtype, plus the context/padding mask, stored again
    (attention.rs:307-314)."""
    scale = f32_scale(head_dim)
    mask = _rnd(matrix_bd * to_dtype(scale, dtype), dtype)
    if additive_mask is not None:
        mask = _rnd(mask + additive_mask, dtype)
    return mask


def attend_logits(q_u, k, matrix_bd, additive_mask, head_dim: int, dtype: str):
    """The logits softmax sees inside `attend`: s * q_u k^T + position_term
    (attention.rs:299-318; SDPA scales the content term by the f32 scale)."""
    scale = f32_scale(head_dim)
    return scale * np.matmul(q_u, np.swapaxes(k, -1, -2)) + position_term(matrix_bd, additive_mask, head_dim, dtype)


def attend(q_u, k, v, matrix_bd, additive_mask, head_dim: int, dtype: str):
    """softmax(s * q_u k^T + bd * cast(s) + mask) v (attention.rs:299-318).

    `fast::scaled_dot_product_attention` is evaluated in float64 (MLX
    internal precision unpinned); its output is stored in `dtype`.
    """
    probs = _softmax(attend_logits(q_u, k, matrix_bd, additive_mask, head_dim, dtype))
    return _rnd(np.matmul(probs, v), dtype)


# ---------------------------------------------------------------------------
# The attention module (attention.rs:320-893)
# ---------------------------------------------------------------------------

@dataclass
class MhsaParams:
    """Weights of one `RelPositionMultiHeadAttention` (attention.rs:328-361)."""

    d_model: int
    n_heads: int
    linear_q: LinearLayer
    linear_k: LinearLayer
    linear_v: LinearLayer
    linear_out: LinearLayer
    linear_pos: LinearLayer
    pos_bias_u: np.ndarray  # [H, d_k]
    pos_bias_v: np.ndarray  # [H, d_k]
    cache_drop_size: int = 0

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads


def _split_heads(t: np.ndarray, n_heads: int) -> np.ndarray:
    b, n, d = t.shape
    return t.reshape(b, n, n_heads, d // n_heads).transpose(0, 2, 1, 3)


def _merge_heads(t: np.ndarray) -> np.ndarray:
    b, h, n, dk = t.shape
    return t.transpose(0, 2, 1, 3).reshape(b, n, h * dk)


def project(p: MhsaParams, x: np.ndarray, pos_emb: np.ndarray, dtype: str = F32):
    """The offline forward's projections (attention.rs:478-499), heads split:
    q, k, v [B,H,T,dk] and the projected position rows pp [1,H,P,dk]."""
    x = np.asarray(x, dtype=np.float64)
    pos_emb = np.asarray(pos_emb, dtype=np.float64)
    h = p.n_heads
    q = _split_heads(p.linear_q.forward(x, dtype), h)  # 478-490
    k = _split_heads(p.linear_k.forward(x, dtype), h)
    v = _split_heads(p.linear_v.forward(x, dtype), h)
    pp = _split_heads(p.linear_pos.forward(pos_emb, dtype), h)  # 493-499: [1,H,P,dk]
    return q, k, v, pp


def biased_queries(p: MhsaParams, q: np.ndarray, dtype: str):
    """q_u = q + pos_bias_u, q_v = q + pos_bias_v in the activation dtype (attention.rs:501-508)."""
    h, dk = p.n_heads, p.head_dim
    bu = to_dtype(p.pos_bias_u, dtype).reshape(1, h, 1, dk)
    bv = to_dtype(p.pos_bias_v, dtype).reshape(1, h, 1, dk)
    return _rnd(q + bu, dtype), _rnd(q + bv, dtype)


def _offline_mask(context, key_mask, start: int, end: int, seq_len: int):
    """Context mask of query rows [start, end) plus the key padding mask (attention.rs:533-543)."""
    cmask = context.block_mask(start, end, seq_len) if context is not None else None
    if cmask is not None and key_mask is not None:
        return cmask + key_mask
    return cmask if cmask is not None else key_mask


def attention_logits(p: MhsaParams, q: np.ndarray, k: np.ndarray, pp: np.ndarray,
                     context: Optional[AttentionContext] = None,
                     key_mask: Optional[np.ndarray] = None, dtype: str = F32) -> np.ndarray:
    """Logits [B,H,T,T] the offline forward's softmax sees, from projected
    q, k [B,H,T,dk] and position rows pp [1,H,2T-1,dk]: the whole query range
    as one block (blocking does not change any element, attention.rs:1066-1104)."""
    seq_len = q.shape[2]
    q_u, q_v = biased_queries(p, q, dtype)
    bd = _rnd(np.matmul(q_v, np.swapaxes(pp, -1, -2)), dtype)  # 530
    bd = rel_shift(bd)[..., :seq_len]
    return attend_logits(q_u, k, bd, _offline_mask(context, key_mask, 0, seq_len, seq_len), p.head_dim, dtype)


def mhsa_forward(p: MhsaParams, x: np.ndarray, pos_emb: np.ndarray,
                 context: Optional[AttentionContext] = None,
                 key_mask: Optional[np.ndarray] = None, dtype: str = F32,
                 max_score_elements: int = MAX_SCORE_ELEMENTS) -> np.ndarray:
    """Offline forward, `forward` / `forward_blocked` (attention.rs:446-573).

    x [B,T,D] and pos_emb [1,2T-1,D] hold values already in `dtype`.
    """
    bsz, seq_len, _ = np.shape(x)
    h, dk = p.n_heads, p.head_dim
    q, k, v, pp = project(p, x, pos_emb, dtype)
    q_u, q_v = biased_queries(p, q, dtype)
    p_t = np.swapaxes(pp, -1, -2)  # 510
    block = query_block_size(bsz * h, seq_len, max_score_elements)  # 517
    outs = []
    for start in range(0, seq_len, block):  # 519-551
        end = min(start + block, seq_len)
        qu_b = q_u[:, :, start:end, :]
        qv_b = q_v[:, :, start:end, :]
        p_slice = p_t[..., (seq_len - end):(2 * seq_len - 1 - start)]  # 529
        bd = _rnd(np.matmul(qv_b, p_slice), dtype)  # 530
        bd = rel_shift(bd)[..., :seq_len]  # 531-532
        mask = _offline_mask(context, key_mask, start, end, seq_len)  # 533-543
        outs.append(attend(qu_b, k, v, bd, mask, dk, dtype))  # 544
    ctx = np.concatenate(outs, axis=2) if len(outs) > 1 else outs[0]
    return p.linear_out.forward(_merge_heads(ctx), dtype)  # 558-565


def cache_update(cache: np.ndarray, x: np.ndarray, cache_drop_size: int) -> np.ndarray:
    """New attention cache after one chunk (attention.rs:661-686, padded or
    truncated to the cache size as the encoder does in conformer.rs:983-999)."""
    cache_size = cache.shape[1]
    seq_len = x.shape[1]
    q_keep = max(seq_len - cache_drop_size, 0)  # 665
    if q_keep > 0:
        nc = np.concatenate([cache[:, q_keep:, :], x[:, :q_keep, :]], axis=1)  # 670-676
    else:
        nc = cache.copy()
    n = nc.shape[1]
    if n < cache_size:  # conformer.rs:986-993
        nc = np.concatenate([np.zeros((nc.shape[0], cache_size - n, nc.shape[2])), nc], axis=1)
    elif n > cache_size:  # conformer.rs:994-997
        nc = nc[:, n - cache_size:, :]
    return nc


def mhsa_forward_with_cache(p: MhsaParams, x: np.ndarray, pos_emb: np.ndarray,
                            cache: Optional[np.ndarray], att_mask=None,
                            dtype: str = F32, pos_rows: Optional[np.ndarray] = None):
    """Cache-aware streaming forward (attention.rs:606-816).

    `att_mask` is None, a bool array [B|1, T, L] (True = visible, the
    unfused path of 777-790 where a fully hidden row yields 0), or an additive
    float array (fused SDPA path, 791-792). Returns (out, new_cache).

    x and the cache are f32 arrays, as the encoder streams them: its caches
    stay f32 after `set_dtype` (conformer.rs:422-434) and the streamed
    features are never cast (conformer.rs:845-849). With `dtype` = bf16 the
    parameters are the bf16-cast ones, but every op that meets an f32
    activation promotes to f32 (MLX type promotion), so only the position
    rows -- a bf16 table through bf16 weights -- are rounded to bf16.

    `pos_rows` [P, D], when given, replaces linear_pos(pos_emb): a test can
    then feed a kernel's own projected rows, pinned separately.
    """
    x = np.asarray(x, dtype=np.float64)
    pos_emb = np.asarray(pos_emb, dtype=np.float64)
    bsz, seq_len, _ = x.shape
    h, dk = p.n_heads, p.head_dim
    if cache is not None:
        kv_in = np.concatenate([cache, x], axis=1)  # 650
        total = cache.shape[1] + seq_len
        new_cache = cache_update(cache, x, p.cache_drop_size)
    else:  # 687-700
        kv_in = x
        total = seq_len
        q_keep = max(seq_len - p.cache_drop_size, 0)
        new_cache = x[:, :q_keep, :]
    q = _split_heads(p.linear_q.forward_promoted(x, dtype), h)  # 718
    k = _split_heads(p.linear_k.forward_promoted(kv_in, dtype), h)  # 721
    v = _split_heads(p.linear_v.forward_promoted(kv_in, dtype), h)  # 722
    pe = p.linear_pos.forward(pos_emb, dtype) if pos_rows is None else np.asarray(pos_rows, np.float64)[None]
    pp = _split_heads(pe, h)  # 749-761: the table is in `dtype`
    p_t = np.swapaxes(pp, -1, -2)
    bu = to_dtype(p.pos_bias_u, dtype).reshape(1, h, 1, dk)
    bv = to_dtype(p.pos_bias_v, dtype).reshape(1, h, 1, dk)
    q_u = q + bu  # f32
    q_v = q + bv
    bd = np.matmul(q_v, p_t)  # 770, f32
    bd = rel_shift(bd)[..., :total]  # 771-772
    if att_mask is not None:
        att_mask = np.asarray(att_mask)
        m4 = att_mask.reshape(att_mask.shape[0], 1, seq_len, total)  # 776
    if att_mask is not None and att_mask.dtype == np.bool_:  # 783-789
        # divides by the f32 sqrt(d_k) rather than multiplying by 1/sqrt (784)
        scores = (np.matmul(q_u, np.swapaxes(k, -1, -2)) + bd) / float(np.sqrt(np.float32(dk)))
        scores = np.where(m4, scores, NEG_INF)
        w = _softmax(scores)
        w = np.where(m4, w, 0.0)
        ctx = np.matmul(w, v)
    elif att_mask is not None:
        ctx = attend(q_u, k, v, bd, m4, dk, F32)  # cast(s) to bd's dtype, f32
    else:
        ctx = attend(q_u, k, v, bd, None, dk, F32)
    out = p.linear_out.forward_promoted(_merge_heads(ctx), dtype)  # 795-807
    return out, new_cache


# ---------------------------------------------------------------------------
# a13: streaming attention mask (conformer.rs:97-323, 883-927)
# ---------------------------------------------------------------------------

def _triu(mask: np.ndarray, diagonal: int) -> np.ndarray:
    """conformer.rs:227-251: keep col - row >= diagonal."""
    rows, cols = mask.shape[1], mask.shape[2]
    diff = np.arange(cols).reshape(1, cols) - np.arange(rows).reshape(rows, 1)
    return mask & (diff >= diagonal)[None]


def _tril(mask: np.ndarray, diagonal: int) -> np.ndarray:
    """conformer.rs:253-277: keep col - row <= diagonal."""
    rows, cols = mask.shape[1], mask.shape[2]
    diff = np.arange(cols).reshape(1, cols) - np.arange(rows).reshape(rows, 1)
    return mask & (diff <= diagonal)[None]


def _chunked_limited(max_len: int, chunk: int, left_chunks: int) -> np.ndarray:
    """conformer.rs:293-323."""
    idx = np.arange(max_len) // chunk
    diff = idx.reshape(-1, 1) - idx.reshape(1, -1)
    return ((diff >= 0) & (diff <= left_chunks)).reshape(1, max_len, max_len)


def create_attention_mask(att_context_size: Tuple[int, int], style: str,
                          max_audio_length: int, cache_len: int,
                          filled_cache_len: int, tensor_seq_len: int,
                          valid_seq_len: int) -> np.ndarray:
    """Bool mask [1, T, C+T], True = visible (conformer.rs:97-221)."""
    m = np.ones((1, max_audio_length, max_audio_length), dtype=bool)
    left, right = att_context_size
    if style == "chunked_limited":  # 124-142
        if right == -1:
            if left >= 0:
                m = _triu(m, -left)
        else:
            chunk = right + 1
            lc = left // chunk if left >= 0 else 10000
            m = _chunked_limited(max_audio_length, chunk, lc)
    else:  # 143-151
        if left >= 0:
            m = _triu(m, -left)
        if right >= 0:
            m = _tril(m, right)
    offset = cache_len - filled_cache_len  # 155-181
    if offset > 0:
        valid = (np.arange(max_audio_length) >= offset).reshape(1, 1, max_audio_length)
        m = m & valid
    m = m[:, cache_len:, :]  # 191
    if valid_seq_len < tensor_seq_len:  # 197-215
        rows = (np.arange(tensor_seq_len) < valid_seq_len).reshape(1, tensor_seq_len, 1)
        m = m & rows
    return m


def streaming_mask(att_context_size, style, cache_size, filled, seq_len, valid_seq_len):
    """The mask `forward_streaming` hands to each layer (conformer.rs:894-927):
    None when every key is visible, the bool mask when a row can be blank
    (valid < T), otherwise the additive 0/-inf form."""
    if att_context_size is None:
        return None
    m = create_attention_mask(att_context_size, style, cache_size + seq_len, cache_size,
                              filled, seq_len, valid_seq_len)
    if m.all():
        return None
    if valid_seq_len < seq_len:
        return m
    return np.where(m, 0.0, NEG_INF)


def next_fill(filled: int, seq_len: int, cache_drop_size: int, cache_size: int) -> int:
    """conformer.rs:1025-1036: min(f + (T - drop), C)."""
    keep = max(seq_len - cache_drop_size, 0)
    return min(filled + keep, cache_size)


# ---------------------------------------------------------------------------
# a16: pre-LN + residual sublayer (conformer.rs:1747-1780)
# ---------------------------------------------------------------------------

def layer_norm(x: np.ndarray, gamma=None, beta=None, eps: float = 1e-5,
               dtype: str = F32) -> np.ndarray:
    """mlx nn::LayerNorm(D) (eps 1e-5, affine), statistics in float64, output in dtype."""
    x = np.asarray(x, dtype=np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps)
    if gamma is not None:
        y = y * to_dtype(gamma, dtype)
    if beta is not None:
        y = y + to_dtype(beta, dtype)
    return _rnd(y, dtype)


def mhsa_sublayer(p: MhsaParams, x, pos_emb, context=None, key_mask=None,
                  gamma=None, beta=None, dtype: str = F32, eps: float = 1e-5):
    """x + MHSA(LayerNorm(x)) (conformer.rs:1747-1780); the norm parameters
    hold their `dtype` values (set_dtype casts the norms, conformer.rs:1656)."""
    gamma = None if gamma is None else to_dtype(gamma, dtype)
    beta = None if beta is None else to_dtype(beta, dtype)
    h = layer_norm(x, gamma, beta, eps, dtype)
    a = mhsa_forward(p, h, pos_emb, context, key_mask, dtype)
    return _rnd(np.asarray(x, dtype=np.float64) + a, dtype)


# ---------------------------------------------------------------------------
# FeedForward (conformer.rs:2031-2088) and its half-step sublayer
# ---------------------------------------------------------------------------

def silu(x: np.ndarray, dtype: str = F32) -> np.ndarray:
    """mlx nn::silu = x * sigmoid(x) as two ops, each result stored in `dtype`
    (conformer.rs:2069); evaluated in float64."""
    x = np.asarray(x, dtype=np.float64)
    sig = _rnd(1.0 / (1.0 + np.exp(-x)), dtype)
    return _rnd(x * sig, dtype)


def _pointwise(layer: LinearLayer, x, act: str, dtype: str):
    """A pointwise conv on activations stored in `act`: in the module dtype
    (`forward`) or f32 with the cast parameters promoted (`forward_promoted`)."""
    if act == dtype:
        return layer.forward(x, dtype)
    return layer.forward_promoted(x, dtype)


@dataclass
class FeedForwardParams:
    """linear1 [ff_dim, d_model], linear2 [d_model, ff_dim] (conformer.rs:2031-2064)."""

    linear1: LinearLayer
    linear2: LinearLayer


def feed_forward(p: FeedForwardParams, x: np.ndarray, dtype: str = F32, act: Optional[str] = None) -> np.ndarray:
    """FeedForward::forward (conformer.rs:2066-2072): linear2(silu(linear1(x))).
    `act` is the dtype x is stored in (default `dtype`): f32 activations in a
    bf16 module (the streaming path) promote every op to f32 over the
    parameters' bf16 values."""
    act = act or dtype
    x = np.asarray(x, dtype=np.float64)
    return _pointwise(p.linear2, silu(_pointwise(p.linear1, x, act, dtype), act), act, dtype)


def feed_forward_sublayer(p: FeedForwardParams, x, gamma=None, beta=None, dtype: str = F32, eps: float = 1e-5,
                          act: Optional[str] = None):
    """x + 0.5 * FeedForward(LayerNorm(x)) (conformer.rs:1703-1729, 1914-1919):
    the half is cast to the output's dtype, the scaled output and the sum
    stored; the LayerNorm parameters hold their `dtype` values, its output is
    stored in `act`."""
    act = act or dtype
    g = None if gamma is None else to_dtype(gamma, dtype)
    b = None if beta is None else to_dtype(beta, dtype)
    y = feed_forward(p, layer_norm(x, g, b, eps, act), dtype, act)
    return _rnd(np.asarray(x, dtype=np.float64) + _rnd(to_dtype(0.5, act) * y, act), act)


# ---------------------------------------------------------------------------
# ConvolutionModule (conformer.rs:2105-2437) and its sublayer
# ---------------------------------------------------------------------------

@dataclass
class ConvModuleParams:
    """ConvolutionModule (conformer.rs:2105-2193). depthwise_weight is in the
    MLX Conv1d layout [D, K, 1] (loading.rs:216-224); norm is "batch_norm"
    (weight, bias, running_mean, running_var) or "layer_norm" (weight, bias),
    both loaded from `{prefix}.batch_norm` (conformer.rs:2419-2426)."""

    pointwise_conv1: LinearLayer
    depthwise_weight: np.ndarray
    depthwise_bias: Optional[np.ndarray]
    pointwise_conv2: LinearLayer
    norm: str
    norm_weight: np.ndarray
    norm_bias: np.ndarray
    running_mean: Optional[np.ndarray] = None
    running_var: Optional[np.ndarray] = None
    causal: bool = False

    @property
    def kernel_size(self) -> int:
        return int(self.depthwise_weight.shape[1])


def sigmoid(x: np.ndarray, dtype: str = F32) -> np.ndarray:
    """mlx sigmoid, the result stored in `dtype` (float64 inside)."""
    return _rnd(1.0 / (1.0 + np.exp(-np.asarray(x, dtype=np.float64))), dtype)


def glu(h: np.ndarray, d_model: int, dtype: str) -> np.ndarray:
    """conformer.rs:2221-2226: x1 * sigmoid(x2) over the two channel halves,
    the sigmoid and the product each stored in `dtype`."""
    return _rnd(h[..., :d_model] * sigmoid(h[..., d_model:], dtype), dtype)


def depthwise_conv1d(u: np.ndarray, weight, bias, pad_left: int, pad_right: int,
                     dtype: str, param_dtype: str) -> np.ndarray:
    """nn::Conv1d with groups = channels on [B, L, D] (cross-correlation:
    y[t, c] = sum_k w[c, k] * u_pad[t + k, c]), the conv result stored in
    `dtype`, then the bias add stored (mlx Conv1d forward). Weights carry
    their `param_dtype` values; zero padding on each side."""
    w = to_dtype(np.asarray(weight, dtype=np.float64)[:, :, 0], param_dtype)  # [D, K]
    k = w.shape[1]
    u = np.asarray(u, dtype=np.float64)
    b_, l_, d_ = u.shape
    up = np.zeros((b_, pad_left + l_ + pad_right, d_))
    up[:, pad_left:pad_left + l_] = u
    t_out = up.shape[1] - k + 1
    y = np.zeros((b_, t_out, d_))
    for j in range(k):
        y += up[:, j:j + t_out, :] * w[:, j]
    y = _rnd(y, dtype)
    if bias is not None:
        y = _rnd(y + to_dtype(bias, param_dtype), dtype)
    return y


def batch_norm_inference(x, mean, var, weight, bias, dtype: str, param_dtype: str,
                         eps: float = 1e-5) -> np.ndarray:
    """mlx-rs 0.32 nn::BatchNorm with training = false (conformer.rs:2155-2163,
    loading.rs:236-254): (x - running_mean) * rsqrt(running_var + eps), then
    weight * x + bias, each op stored in its result dtype. The parameters and
    eps hold their `param_dtype` values (eps cast in set_dtype,
    conformer.rs:2127-2130), so rsqrt(var + eps) involves parameters only and
    is stored in `param_dtype`; the ops with x are stored in `dtype`."""
    e = _rnd(to_dtype(var, param_dtype) + to_dtype(eps, param_dtype), param_dtype)
    inv = _rnd(1.0 / np.sqrt(e), param_dtype)
    y = _rnd(np.asarray(x, dtype=np.float64) - to_dtype(mean, param_dtype), dtype)
    y = _rnd(y * inv, dtype)
    y = _rnd(to_dtype(weight, param_dtype) * y, dtype)
    return _rnd(y + to_dtype(bias, param_dtype), dtype)


def conv_module(p: ConvModuleParams, x, dtype: str = F32, act: Optional[str] = None,
                lengths=None, cache=None):
    """ConvolutionModule::forward (conformer.rs:2197-2291) and
    ::forward_with_cache (conformer.rs:2305-2378) on x [B, T, D].

    `dtype` is the module dtype (set_dtype), `act` the dtype x is stored in
    (default `dtype`; the streaming path feeds f32). `lengths` [B]: frames
    t >= lengths[b] are zeroed after the GLU (PaddingMask.valid / pad_mask).
    `cache` [B, D, K-1] (f32) is the conv cache: the conv then runs over
    [cache; GLU(x)] and the new cache is its last K-1 frames; without it a
    causal module pads K-1 zero frames on the left, a symmetric one (K-1)/2
    on each side. The causal padding and the cache are f32 arrays, so in a
    bf16 module MLX promotes the concatenation and everything after it to
    f32 (conformer.rs:2250-2256, 2328-2336). Returns (out, new_cache)."""
    act = act or dtype
    x = np.asarray(x, dtype=np.float64)
    b_, t_, d_ = x.shape
    k = p.kernel_size
    u = glu(_pointwise(p.pointwise_conv1, x, act, dtype), d_, act)
    if lengths is not None:
        valid = np.arange(t_)[None, :] < np.asarray(lengths)[:, None]
        u = np.where(valid[:, :, None], u, 0.0)
    new_cache = None
    if cache is not None:
        if not p.causal:
            raise ValueError("a conv cache needs a causal module")
        seq = np.concatenate([np.transpose(np.asarray(cache, dtype=np.float64), (0, 2, 1)), u], axis=1)
        new_cache = np.transpose(seq[:, seq.shape[1] - (k - 1):, :], (0, 2, 1)).copy()
        conv_dt, pad_l, pad_r = F32, 0, 0
        u = seq
    elif p.causal:
        conv_dt, pad_l, pad_r = F32, k - 1, 0
    else:
        conv_dt, pad_l, pad_r = act, (k - 1) // 2, (k - 1) // 2
    y = depthwise_conv1d(u, p.depthwise_weight, p.depthwise_bias, pad_l, pad_r, conv_dt, dtype)
    if p.norm == "batch_norm":
        y = batch_norm_inference(y, p.running_mean, p.running_var, p.norm_weight, p.norm_bias,
                                 conv_dt, dtype)
    else:
        y = layer_norm(y, to_dtype(p.norm_weight, dtype), to_dtype(p.norm_bias, dtype), 1e-5, conv_dt)
    y = silu(y, conv_dt)
    return _pointwise(p.pointwise_conv2, y, conv_dt, dtype), new_cache


def conv_sublayer(p: ConvModuleParams, x, gamma=None, beta=None, dtype: str = F32,
                  act: Optional[str] = None, lengths=None, cache=None, eps: float = 1e-5):
    """x + conv(LayerNorm(x)) (conformer.rs:1790-1814; with the cache
    1936-1941); the conv_norm parameters hold their `dtype` values and the
    LayerNorm output is stored in `act`. Returns (out, new_cache)."""
    act = act or dtype
    g = None if gamma is None else to_dtype(gamma, dtype)
    b = None if beta is None else to_dtype(beta, dtype)
    h = layer_norm(x, g, b, eps, act)
    y, new_cache = conv_module(p, h, dtype, act, lengths, cache)
    out_dt = F32 if (cache is not None or p.causal) else act
    return _rnd(np.asarray(x, dtype=np.float64) + y, out_dt), new_cache


# ---------------------------------------------------------------------------
# ConformerBlock (conformer.rs:1613-2028): FF1 half-step, MHSA, conv, FF2
# half-step, norm_out
# ---------------------------------------------------------------------------

@dataclass
class ConformerBlockParams:
    """One ConformerBlock (conformer.rs:1613-1641, new 1662-1690): each norm a
    (weight, bias) pair, None meaning the identity init (load_layer_norm
    leaves a missing tensor at its init, loading.rs:203-214)."""

    ff1: FeedForwardParams
    ff1_norm: Tuple
    attn: MhsaParams
    attn_norm: Tuple
    conv: ConvModuleParams
    conv_norm: Tuple
    ff2: FeedForwardParams
    ff2_norm: Tuple
    out_norm: Tuple


def conformer_block(p: ConformerBlockParams, x, pos_emb, context: Optional[AttentionContext] = None,
                    lengths=None, dtype: str = F32, act: Optional[str] = None, pos_rows=None):
    """ConformerBlock::forward (conformer.rs:1693-1875) on x [B, T, D] in
    `dtype`: x + 0.5 FF1(LN(x)) (1703-1729), x + MHSA(LN(x)) with the key
    padding mask of `lengths` (1747-1780), x + conv(LN(x)) with frames past
    `lengths` zeroed (1790-1814), x + 0.5 FF2(LN(x)) (1827-1851), then
    norm_out (1862). `lengths` builds PaddingMask (conformer.rs:1594-1615):
    None when no frame is padding. A causal conv in a bf16 block promotes
    the rest of the block to f32 (the conv's f32 padding), as MLX does.

    `act` is the dtype x is stored in (default `dtype`): F32 in a bf16 block
    means activations an earlier block's causal conv promoted, so that every
    op of this block runs in f32 on the bf16 parameter values -- the
    attention as `forward` (attention.rs:446-573) computes it from an f32 x:
    f32 projections, matrix_bd = q_v (f32) . linear_pos(pos_emb) (bf16) in
    f32, the scale cast to f32 and the additive mask; the arithmetic of
    mhsa_forward_with_cache without a cache, whose `pos_rows` it passes on
    (a test can feed a kernel's own bf16 position rows)."""
    x = np.asarray(x, dtype=np.float64)
    t_ = x.shape[1]
    if lengths is not None and all(int(v) >= t_ for v in lengths):
        lengths = None  # PaddingMask::new gives None
    key_mask = key_padding_mask(lengths, t_) if lengths is not None else None
    if (act or dtype) != dtype:
        if act != F32:
            raise ValueError("activations other than the block dtype are f32")
        return _conformer_block_f32_activations(p, x, pos_emb, context, key_mask, lengths, dtype, pos_rows)
    x = feed_forward_sublayer(p.ff1, x, *p.ff1_norm, dtype=dtype)
    x = mhsa_sublayer(p.attn, x, pos_emb, context, key_mask, *p.attn_norm, dtype=dtype)
    x, _ = conv_sublayer(p.conv, x, *p.conv_norm, dtype=dtype, lengths=lengths)
    act = F32 if p.conv.causal else dtype
    x = feed_forward_sublayer(p.ff2, x, *p.ff2_norm, dtype=dtype, act=act)
    g, b = p.out_norm
    return layer_norm(x, None if g is None else to_dtype(g, dtype), None if b is None else to_dtype(b, dtype),
                      1e-5, act)


def _conformer_block_f32_activations(p: ConformerBlockParams, x, pos_emb, context, key_mask, lengths, dtype,
                                     pos_rows=None):
    """conformer_block on activations stored in f32 in a `dtype` block: each
    sublayer as in the f32-activation forms above, the attention as
    mhsa_forward_with_cache without a cache and with the offline additive
    mask (attention.rs:533-543) over the whole query range."""
    t_ = x.shape[1]

    def norm(pair):
        g, b = pair
        return None if g is None else to_dtype(g, dtype), None if b is None else to_dtype(b, dtype)

    x = feed_forward_sublayer(p.ff1, x, *p.ff1_norm, dtype=dtype, act=F32)  # 1703-1729
    h = layer_norm(x, *norm(p.attn_norm), 1e-5, F32)
    mask = _offline_mask(context, key_mask, 0, t_, t_)
    if mask is not None:  # [B|1, T, T] as mhsa_forward_with_cache takes it
        mask = np.broadcast_to(mask, np.broadcast_shapes(mask.shape, (1, 1, t_, t_)))
        mask = mask.reshape(mask.shape[0], t_, t_)
    a, _ = mhsa_forward_with_cache(p.attn, h, pos_emb, None, mask, dtype, pos_rows=pos_rows)  # 1747-1780
    x = _rnd(x + a, F32)
    x, _ = conv_sublayer(p.conv, x, *p.conv_norm, dtype=dtype, act=F32, lengths=lengths)  # 1790-1814
    x = feed_forward_sublayer(p.ff2, x, *p.ff2_norm, dtype=dtype, act=F32)  # 1827-1851
    return layer_norm(x, *norm(p.out_norm), 1e-5, F32)  # 1862


def conformer_encoder(blocks, x, pos_emb, context: Optional[AttentionContext] = None, lengths=None,
                      dtype: str = F32, pos_rows=None):
    """The offline encoder's layer loop (conformer.rs:542-550): every block on
    one pos_emb, context and padding, the activations turning f32 at the first
    causal conv of a bf16 stack; `pos_rows` [blocks] as conformer_block takes
    them. Returns (x, the dtype x ends in)."""
    act = dtype
    for i, p in enumerate(blocks):
        x = conformer_block(p, x, pos_emb, context, lengths, dtype, act, None if pos_rows is None else pos_rows[i])
        if p.conv.causal:
            act = F32
    return x, act


def conformer_block_with_cache(p: ConformerBlockParams, x, pos_emb, att_cache, conv_cache, att_mask=None,
                               pad_lengths=None, dtype: str = F32, pos_rows=None):
    """ConformerBlock::forward_with_cache (conformer.rs:1893-1971) on the
    streaming path's f32 activations x [B, T, D]: every op that meets them is
    f32 (the parameters hold their `dtype` values). The attention caches
    its LayerNorm output h (attention.rs:579-586); `att_mask` and `pos_rows`
    as mhsa_forward_with_cache takes them; `pad_lengths` [B] zero the conv's
    frames past them (pad_mask, conformer.rs:929-941). Returns (x,
    new_att_cache, new_conv_cache)."""
    x = np.asarray(x, dtype=np.float64)
    x = feed_forward_sublayer(p.ff1, x, *p.ff1_norm, dtype=dtype, act=F32)  # 1914-1919
    g, b = p.attn_norm
    h = layer_norm(x, None if g is None else to_dtype(g, dtype), None if b is None else to_dtype(b, dtype), 1e-5, F32)
    a, new_att = mhsa_forward_with_cache(p.attn, h, pos_emb, att_cache, att_mask, dtype, pos_rows=pos_rows)  # 1924-1933
    x = x + a
    x, new_conv = conv_sublayer(p.conv, x, *p.conv_norm, dtype=dtype, act=F32, lengths=pad_lengths,
                                cache=conv_cache)  # 1936-1941
    x = feed_forward_sublayer(p.ff2, x, *p.ff2_norm, dtype=dtype, act=F32)  # 1950-1955
    g, b = p.out_norm
    x = layer_norm(x, None if g is None else to_dtype(g, dtype), None if b is None else to_dtype(b, dtype), 1e-5,
                   F32)  # 1960
    return x, new_att, new_conv


# ---------------------------------------------------------------------------
# Index maps exported for bit-exact checks
# ---------------------------------------------------------------------------

def rel_shift_index(rows: int, total_len: int, pos_len: int) -> np.ndarray:
    """Flat source index (row * pos_len + column) of the `matrix_bd` entry that
    lands at (i, j) after rel_shift + truncation to `total_len` keys, found by
    running `rel_shift` on a unique ramp (the construction of
    attention.rs:1248-1282). -1 marks a padding zero."""
    ramp = (np.arange(rows * pos_len, dtype=np.float64) + 1.0).reshape(rows, pos_len)
    return rel_shift(ramp)[:, :total_len].astype(np.int64) - 1
