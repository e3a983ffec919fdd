"""Pins for the CPU oracle (`oracle/relpos_oracle.py`), run without a GPU.

Every oracle function is checked against something that does not restate
its own formula:

* the reference's known-answer and invariant tests (`attention.rs:896-1358`,
  `quantization.rs:413-430`), re-expressed on numpy inputs;
* the mathematical definition of Transformer-XL relative attention, evaluated
  with an explicit relative-position index per (query, key) pair instead of
  the oracle's pad + reshape `rel_shift` and query blocking;
* exact arithmetic (dequantisation in float64, bf16 rounding against torch's
  own float32 -> bfloat16 conversion, LayerNorm against torch);
* hand-derived known answers for the streaming mask and the cache slide.

The reference has no numeric golden tensors for this path (its randomized
tests draw from `mlx::random`, which is unavailable here), so only their
invariants carry over.
"""
import math

import numpy as np
import pytest
import torch

import relpos_oracle as O


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------

def random_params(d_model, n_heads, seed, use_bias=True, scale=0.3):
    """Random weights in the style of `random_attention` (attention.rs:1000-1016)."""
    rng = np.random.default_rng(seed)
    d = d_model
    w = lambda: rng.standard_normal((d, d)) * scale
    b = lambda: rng.standard_normal(d) * scale
    dk = d // n_heads
    return O.MhsaParams(
        d_model, n_heads,
        O.LinearLayer(w(), b() if use_bias else None),
        O.LinearLayer(w(), b() if use_bias else None),
        O.LinearLayer(w(), b() if use_bias else None),
        O.LinearLayer(w(), None),
        O.LinearLayer(w(), None),
        rng.standard_normal((n_heads, dk)) * scale,
        rng.standard_normal((n_heads, dk)) * scale,
    )


def direct_attention(p, x_q, kv_in, pos_emb, cache_len, visible, scale=None, scale_bd=None, P=None):
    """Rel-pos attention from its definition, one (query, key) pair at a time.

    Query row i sits at absolute frame cache_len + i; key j at frame j. The
    table row for relative distance r = (cache_len + i) - j is (L - 1) - r,
    since the table lists distances L-1 down to -(L-1). `visible` is a bool
    array [B, T, L]; a row with no visible key yields 0 (attention.rs:788).
    """
    h, dk = p.n_heads, p.head_dim
    L = kv_in.shape[1]
    q = p.linear_q.forward(x_q)
    k = p.linear_k.forward(kv_in)
    v = p.linear_v.forward(kv_in)
    P = p.linear_pos.forward(pos_emb[0]) if P is None else P
    s = O.f32_scale(dk) if scale is None else scale
    sb = s if scale_bd is None else scale_bd
    B, T, _ = x_q.shape
    ctx = np.zeros((B, T, h * dk))
    for b in range(B):
        for hh in range(h):
            sl = slice(hh * dk, (hh + 1) * dk)
            for i in range(T):
                qu = q[b, i, sl] + p.pos_bias_u[hh]
                qv = q[b, i, sl] + p.pos_bias_v[hh]
                scores = np.full(L, -np.inf)
                for j in range(L):
                    if not visible[b, i, j]:
                        continue
                    row = (L - 1) - ((cache_len + i) - j)
                    scores[j] = s * (qu @ k[b, j, sl]) + sb * (qv @ P[row, sl])
                if np.isfinite(scores).any():
                    e = np.exp(scores - scores.max())
                    ctx[b, i, sl] = (e / e.sum()) @ v[b, :, sl]
    return p.linear_out.forward(ctx)


def nemo_visible(size, style, i, j):
    """Brute-force port of NeMo `_create_masks` (attention.rs:1108-1119)."""
    left, right = size
    if style == "chunked_limited" and right >= 0:
        chunk = right + 1
        lc = left // chunk if left >= 0 else 10000
        diff = i // chunk - j // chunk
        return 0 <= diff <= lc
    right_ok = style == "chunked_limited" or right < 0 or j - i <= right
    return (left < 0 or j - i >= -left) and right_ok


# ---------------------------------------------------------------------------
# a1: positional encoding (attention.rs:902-915, 1150-1246, 1337-1357)
# ---------------------------------------------------------------------------

def test_rel_positional_encoding_creation():
    pe = O.RelPositionalEncoding(512, 100, True)
    assert abs(pe.xscale - math.sqrt(512.0)) < 1e-5


def test_rel_positional_encoding_shape():
    pe = O.RelPositionalEncoding(512, 100, False)
    assert pe.get_encoding(50).shape == (1, 99, 512)


def test_rel_positional_encoding_empty_is_error():
    with pytest.raises(ValueError):
        O.RelPositionalEncoding(16, 10, False).get_encoding(0)


def test_rel_positional_encoding_values():
    enc = O.RelPositionalEncoding(4, 3, False).get_encoding(3)
    assert enc.shape == (1, 5, 4)
    data = enc.reshape(-1)
    d1 = math.exp(-2.0 * math.log(10000.0) / 4.0)
    exp_row0 = [math.sin(2.0), math.cos(2.0), math.sin(2.0 * d1), math.cos(2.0 * d1)]
    for c in range(4):
        assert abs(data[c] - exp_row0[c]) < 1e-5
    assert abs(data[8] - 0.0) < 1e-5 and abs(data[9] - 1.0) < 1e-5
    # the last row is distance -2: sin is odd, cos even
    assert abs(data[16] + math.sin(2.0)) < 1e-5 and abs(data[17] - math.cos(2.0)) < 1e-5


def test_rel_positional_encoding_extends_past_max_len():
    a = O.RelPositionalEncoding(16, 10, False).get_encoding(25)
    b = O.RelPositionalEncoding(16, 40, False).get_encoding(25)
    assert a.shape == (1, 49, 16)
    assert np.max(np.abs(a - b)) < 1e-6


def test_rel_positional_encoding_streaming_dimensions():
    pe = O.RelPositionalEncoding(512, 5000, False)
    assert pe.get_encoding(84).shape == (1, 167, 512)


def test_positional_table_against_float64_sinusoid():
    # every entry is sin/cos of distance * 10000^(-2k/d), to f32 accuracy
    d, L = 64, 50
    enc = O.RelPositionalEncoding(d, 60, False).get_encoding(L)[0].astype(np.float64)
    dist = np.arange(L - 1, -L, -1, dtype=np.float64).reshape(-1, 1)
    freq = 10000.0 ** (-np.arange(0, d, 2, dtype=np.float64) / d)
    ang = dist * freq
    assert np.max(np.abs(enc[:, 0::2] - np.sin(ang))) < 5e-5
    assert np.max(np.abs(enc[:, 1::2] - np.cos(ang))) < 5e-5


# ---------------------------------------------------------------------------
# a7: rel_shift (attention.rs:917-998, 1248-1335)
# ---------------------------------------------------------------------------

def test_rel_shift_shape():
    assert O.rel_shift(np.ones((1, 1, 4, 7))).shape == (1, 1, 4, 7)


def test_rel_shift_correctness():
    x = np.arange(15, dtype=np.float64).reshape(1, 1, 3, 5)
    s = O.rel_shift(x).reshape(-1)
    assert list(s[0:3]) == [2.0, 3.0, 4.0]
    assert list(s[5:8]) == [6.0, 7.0, 8.0]
    assert list(s[10:13]) == [10.0, 11.0, 12.0]


def _verify_rel_shift(seq_len, pos_len, num_keys):
    x = np.arange(seq_len * pos_len, dtype=np.float64).reshape(1, 1, seq_len, pos_len)
    s = O.rel_shift(x).reshape(seq_len, pos_len)
    for i in range(seq_len):
        for j in range(num_keys):
            assert s[i, j] == i * pos_len + (seq_len - 1 - i + j)


def test_rel_shift_property_standard():
    for seq_len in range(1, 9):
        _verify_rel_shift(seq_len, 2 * seq_len - 1, seq_len)


def test_rel_shift_property_streaming():
    for seq_len in range(1, 7):
        for cache_len in range(1, 7):
            total = seq_len + cache_len
            _verify_rel_shift(seq_len, 2 * total - 1, total)


def test_rel_shift_no_padding_zeros_in_output():
    seq_len, total = 4, 7
    pos_len = 2 * total - 1
    x = 100.0 + np.arange(seq_len * pos_len, dtype=np.float64).reshape(1, 1, seq_len, pos_len)
    s = O.rel_shift(x).reshape(seq_len, pos_len)
    assert (s[:, :total] >= 100.0).all()


def test_rel_shift_index_map_closed_form():
    for rows, total in [(1, 1), (5, 5), (14, 84), (13, 13), (7, 30)]:
        pos_len = 2 * total - 1
        idx = O.rel_shift_index(rows, total, pos_len)
        i = np.arange(rows).reshape(-1, 1)
        j = np.arange(total).reshape(1, -1)
        assert (idx == i * pos_len + (rows - 1 - i + j)).all()


# ---------------------------------------------------------------------------
# a8, a9: masks and blocking (attention.rs:1106-1148, 196-206)
# ---------------------------------------------------------------------------

def test_attention_context_mask_matches_nemo():
    seq_len = 23
    cases = [((56, 3), "chunked_limited"), ((5, 1), "chunked_limited"),
             ((-1, 2), "chunked_limited"), ((4, -1), "chunked_limited"),
             ((3, 2), "regular"), ((-1, 0), "regular")]
    for size, style in cases:
        ctx = O.AttentionContext.new(size, style)
        m = ctx.block_mask(7, 19, seq_len)
        assert m.shape == (12, seq_len)
        for i in range(7, 19):
            for j in range(seq_len):
                assert (m[i - 7, j] == 0.0) == nemo_visible(size, style, i, j), (size, style, i, j)
    assert O.AttentionContext.new((-1, -1), "chunked_limited") is None


def test_key_padding_mask():
    assert O.key_padding_mask([13, 13], 13) is None
    m = O.key_padding_mask([13, 9, 0], 13)
    assert m.shape == (3, 1, 1, 13)
    assert (m[0] == 0).all()
    assert (m[1, 0, 0, :9] == 0).all() and np.isneginf(m[1, 0, 0, 9:]).all()
    # length clamped to at least one key (attention.rs:285)
    assert m[2, 0, 0, 0] == 0 and np.isneginf(m[2, 0, 0, 1:]).all()


def test_query_block_size():
    assert O.query_block_size(4, 13, 2 * 2 * 2 * 13 * 5) == 5
    assert O.query_block_size(4, 13, 1 << 62) == 13
    assert O.query_block_size(4, 13, 1) == 1
    # configuration shapes quoted in the survey of the reference path
    assert O.query_block_size(2 * 8, 7500, O.MAX_SCORE_ELEMENTS) == 279
    assert O.query_block_size(4 * 8, 1500, O.MAX_SCORE_ELEMENTS) == 699


# ---------------------------------------------------------------------------
# a2, a3: linear layers and dequantisation
# ---------------------------------------------------------------------------

def test_standard_linear_forward():
    # quantization.rs:413-430
    layer = O.LinearLayer(np.array([[1.0, 2, 3], [4, 5, 6]]), np.array([0.1, 0.2]))
    y = layer.forward(np.ones((1, 3)))
    assert abs(y[0, 0] - 6.1) < 1e-5 and abs(y[0, 1] - 15.2) < 1e-5


def test_unpack_codes_known_word():
    w = np.array([[0x04030201, 0xFFEE0080]], dtype=np.uint32)
    assert list(O.unpack_codes(w, 8)[0]) == [1, 2, 3, 4, 0x80, 0x00, 0xEE, 0xFF]


def test_dequantize_known_values():
    # one row, one group of 64: s = 0.5, b = 0.25 (both exact in f16 and bf16)
    codes = np.arange(64, dtype=np.uint32)
    w = (codes[0::4] | (codes[1::4] << 8) | (codes[2::4] << 16) | (codes[3::4] << 24)).reshape(1, 16)
    s = np.array([[0.5]], dtype=np.float16)
    b = np.array([[0.25]], dtype=np.float16)
    for dt in (O.F32, O.BF16):
        deq = O.dequantize(w, s, b, 8, 64, dt)
        assert (deq[0] == 0.5 * np.arange(64) + 0.25).all()


def test_dequantize_exact_in_float64():
    # f32(s) * q is exact, so the f32 result equals float64 s*q + b rounded once
    rng = np.random.default_rng(5)
    n, k = 32, 256
    w = rng.integers(0, 2 ** 32, size=(n, k // 4), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(0.002, 0.02, size=(n, k // 64)).astype(np.float16)
    b = (rng.standard_normal((n, k // 64)) * 0.01).astype(np.float16)
    codes = np.stack([(w.astype(np.uint64) >> (8 * p)) & 255 for p in range(4)], -1).reshape(n, k)
    exact = np.repeat(s.astype(np.float64), 64, 1) * codes + np.repeat(b.astype(np.float64), 64, 1)
    got = O.dequantize(w, s, b, 8, 64, O.F32)
    assert (got == exact.astype(np.float32).astype(np.float64)).all()
    # bf16 mode: scales and biases cast to bf16 first, weight stored as bf16
    sb = torch.from_numpy(s.astype(np.float32)).to(torch.bfloat16).double().numpy()
    bb = torch.from_numpy(b.astype(np.float32)).to(torch.bfloat16).double().numpy()
    exact_b = np.repeat(sb, 64, 1) * codes + np.repeat(bb, 64, 1)
    ref_b = torch.from_numpy(exact_b.astype(np.float32)).to(torch.bfloat16).double().numpy()
    assert (O.dequantize(w, s, b, 8, 64, O.BF16) == ref_b).all()


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(10000) * 10.0 ** rng.integers(-8, 8, 10000),
                        [1 + 2 ** -8, 1 + 3 * 2 ** -8, -1 - 2 ** -8, 0.0, 65504.0]])
    ref = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).double().numpy()
    assert (O.bf16_round(x) == ref).all()
    bits = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (O.bf16_bits(x) == bits).all()


def test_layer_norm_matches_torch():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 7, 64)) * 3 + 1
    g, b = rng.standard_normal(64), rng.standard_normal(64)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(x), (64,), torch.from_numpy(g),
                                         torch.from_numpy(b), 1e-5).numpy()
    assert np.max(np.abs(O.layer_norm(x, g, b, 1e-5) - ref)) < 1e-12


# ---------------------------------------------------------------------------
# a10/a15 offline attention against the definition (attention.rs:446-573)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("ctx", [None, ((4, 1), "chunked_limited"), ((3, 2), "regular"),
                                 ((-1, 2), "chunked_limited"), ((2, -1), "regular")])
def test_offline_forward_matches_definition(ctx):
    d, h, T = 16, 2, 13
    p = random_params(d, h, seed=1)
    rng = np.random.default_rng(11)
    x = rng.standard_normal((2, T, d))
    lengths = [T, 9]
    pos = O.RelPositionalEncoding(d, 64, False).get_encoding(T)
    context = O.AttentionContext.new(*ctx) if ctx else None
    out = O.mhsa_forward(p, x, pos, context, O.key_padding_mask(lengths, T))
    vis = np.ones((2, T, T), dtype=bool)
    for b in range(2):
        for i in range(T):
            for j in range(T):
                ok = j < lengths[b]
                if context is not None:
                    ok = ok and nemo_visible(ctx[0], ctx[1], i, j)
                vis[b, i, j] = ok
    ref = direct_attention(p, x, x, pos, 0, vis)
    # compare rows that see at least one key (others are unspecified in the reference)
    rows = vis.any(axis=2)
    assert np.max(np.abs(out - ref)[rows]) < 1e-10


def test_blocked_attention_matches_full():
    d, h, T = 16, 2, 13
    p = random_params(d, h, seed=2)
    x = np.random.default_rng(11).standard_normal((2, T, d))
    pos = O.RelPositionalEncoding(d, 64, False).get_encoding(T)
    for ctx in [None, O.AttentionContext.new((4, 1), "chunked_limited"),
                O.AttentionContext.new((3, 2), "regular")]:
        full = O.mhsa_forward(p, x, pos, ctx, None, max_score_elements=1 << 62)
        blocked = O.mhsa_forward(p, x, pos, ctx, None, max_score_elements=2 * 2 * 2 * 13 * 5)
        assert np.max(np.abs(full - blocked)) < 1e-12
        for dt in (O.BF16,):
            fb = O.mhsa_forward(p, O.bf16_round(x), O.bf16_round(pos), ctx, None, dt, 1 << 62)
            bb = O.mhsa_forward(p, O.bf16_round(x), O.bf16_round(pos), ctx, None, dt, 2 * 2 * 2 * 13 * 5)
            assert np.max(np.abs(fb - bb)) == 0.0


def test_padded_keys_are_ignored():
    d, h, T, valid = 16, 2, 13, 9
    p = random_params(d, h, seed=3)
    x = np.random.default_rng(12).standard_normal((2, T, d))
    x[1, valid:, :] = 50.0
    pe = O.RelPositionalEncoding(d, 64, False)
    km = O.key_padding_mask([T, valid], T)
    assert km is not None and O.key_padding_mask([T, T], T) is None
    for ctx in [None, O.AttentionContext.new((3, 2), "regular")]:
        masked = O.mhsa_forward(p, x, pe.get_encoding(T), ctx, km)
        full_row = O.mhsa_forward(p, x[:1], pe.get_encoding(T), ctx, None)
        short_row = O.mhsa_forward(p, x[1:2, :valid], pe.get_encoding(valid), ctx, None)
        assert np.max(np.abs(masked[:1] - full_row)) < 1e-10
        assert np.max(np.abs(masked[1:2, :valid] - short_row)) < 1e-10


def test_bf16_mode_rounds_only_at_op_boundaries():
    # with bf16-exact inputs the bf16 oracle stays within bf16 noise of float64
    d, h, T = 32, 2, 11
    p = random_params(d, h, seed=4, scale=0.15)
    x = O.bf16_round(np.random.default_rng(1).standard_normal((1, T, d)))
    pos = O.bf16_round(O.RelPositionalEncoding(d, 64, False).get_encoding(T))
    for lin in (p.linear_q, p.linear_k, p.linear_v, p.linear_out, p.linear_pos):
        lin.weight = O.bf16_round(lin.weight)
        if lin.bias is not None:
            lin.bias = O.bf16_round(lin.bias)
    p.pos_bias_u, p.pos_bias_v = O.bf16_round(p.pos_bias_u), O.bf16_round(p.pos_bias_v)
    f = O.mhsa_forward(p, x, pos)
    b = O.mhsa_forward(p, x, pos, dtype=O.BF16)
    assert (O.bf16_round(b) == b).all()
    assert 0 < np.max(np.abs(f - b)) < 0.05 * np.max(np.abs(f))


def _torch_bf16_forward(p, x, pos):
    """The reference's offline bf16 forward with every array a torch bfloat16
    tensor, so each op result is stored in bf16 because of its dtype, not
    because of an explicit rounding call (torch's CPU bf16 matmul accumulates
    in fp32 and rounds once, as MLX's does):

    linear outputs and bias adds (quantization.rs:126-136), q + pos_bias_u/v
    (attention.rs:501-508), matrix_bd (530), bd * cast(scale) (308-311), the
    attention output (315-317). The softmax itself runs in float64 (MLX's SDPA
    precision is unpinned). rel_shift is taken from its closed form
    out[i][j] = bd[i][T-1-i+j] (attention.rs:1248-1282) with a gather.
    """
    bf = torch.bfloat16
    t = lambda a: torch.tensor(np.asarray(a, dtype=np.float32)).to(bf)
    B, T, D = x.shape
    h, dk = p.n_heads, p.head_dim

    def linear(lin, a):
        y = a @ t(lin.weight).T
        return y + t(lin.bias) if lin.bias is not None else y

    split = lambda y, n: y.reshape(y.shape[0], n, h, dk).transpose(1, 2)
    X, PE = t(x), t(pos[0])
    q = split(linear(p.linear_q, X), T)
    k = split(linear(p.linear_k, X), T)
    v = split(linear(p.linear_v, X), T)
    P = split(linear(p.linear_pos, PE)[None], 2 * T - 1)
    q_u = q + t(p.pos_bias_u).reshape(1, h, 1, dk)
    q_v = q + t(p.pos_bias_v).reshape(1, h, 1, dk)
    bd = q_v @ P.transpose(-1, -2)  # [B, h, T, 2T-1], bf16
    i = torch.arange(T).reshape(T, 1)
    j = torch.arange(T).reshape(1, T)
    idx = ((T - 1) - i + j).expand(B, h, T, T)
    bd = torch.gather(bd, 3, idx)
    scale = torch.tensor(1.0, dtype=torch.float32) / torch.sqrt(torch.tensor(float(dk), dtype=torch.float32))
    pos_term = bd * scale.to(bf)  # bf16 * bf16 -> bf16
    logits = scale.double() * (q_u.double() @ k.double().transpose(-1, -2)) + pos_term.double()
    ctx = (torch.softmax(logits, dim=-1) @ v.double()).to(bf)
    ctx = ctx.transpose(1, 2).reshape(B, T, D)
    return linear(p.linear_out, ctx).double().numpy()


def _bf16_case():
    """A small case whose every bf16 rounding changes the output: bf16-exact
    inputs and weights with full 8-bit significands, so each matmul and add
    produces more bits than bf16 keeps, and d_k = 8, whose 1/sqrt(d_k) is not
    a bf16 number (bf16(1/sqrt 8) = 0.353515625)."""
    d, h, T = 16, 2, 5
    p = random_params(d, h, seed=11, scale=0.6)
    rng = np.random.default_rng(12)
    x = O.bf16_round(rng.standard_normal((2, T, d)))
    pos = O.bf16_round(O.RelPositionalEncoding(d, 64, False).get_encoding(T))
    return p, x, pos


def test_bf16_oracle_equals_native_bf16_restatement():
    """Pins where the bf16 oracle rounds: it must equal, bit for bit, the
    reference's op sequence run on native bfloat16 tensors."""
    p, x, pos = _bf16_case()
    got = O.mhsa_forward(p, x, pos, dtype=O.BF16)
    ref = _torch_bf16_forward(p, x, pos)
    assert np.array_equal(got, ref), np.max(np.abs(got - ref))


def test_bf16_oracle_every_rounding_is_load_bearing(monkeypatch):
    """Dropping any single one of the oracle's bf16 roundings (op results via
    `_rnd`, weight and bias casts via `to_dtype`) changes the output of the
    case above, so together with the bit-exact match to the native-bf16
    restatement a dropped or an added rounding fails."""
    p, x, pos = _bf16_case()
    base = O.mhsa_forward(p, x, pos, dtype=O.BF16)
    for fname in ("_rnd", "to_dtype"):
        orig = getattr(O, fname)
        calls = {"n": 0, "skip": -1}

        def patched(a, dtype, _orig=orig):
            calls["n"] += 1
            if calls["n"] - 1 == calls["skip"]:
                return np.asarray(a, dtype=np.float64)
            return _orig(a, dtype)

        monkeypatch.setattr(O, fname, patched)
        O.mhsa_forward(p, x, pos, dtype=O.BF16)
        n = calls["n"]
        assert n == (13 if fname == "_rnd" else 11), (fname, n)
        for k in range(n):
            calls["n"], calls["skip"] = 0, k
            out = O.mhsa_forward(p, x, pos, dtype=O.BF16)
            assert not np.array_equal(out, base), f"dropping {fname} call {k} of {n} leaves the output unchanged"
        monkeypatch.setattr(O, fname, orig)


# ---------------------------------------------------------------------------
# a11-a14: streaming (attention.rs:606-816, conformer.rs:97-323, 883-1036)
# ---------------------------------------------------------------------------

def test_streaming_mask_c3_shape_only_offset():
    # [70,13] chunked_limited, 14-frame chunks: query chunk (70+i)//14 = 5 and
    # key chunks 0..5, 70/14 = 5 left chunks -> only the unfilled-cache offset hides keys
    for f in (0, 1, 13, 56, 69, 70):
        m = O.create_attention_mask((70, 13), "chunked_limited", 84, 70, f, 14, 14)
        assert m.shape == (1, 14, 84)
        expect = np.broadcast_to(np.arange(84) >= 70 - f, (14, 84))
        assert (m[0] == expect).all()


def test_streaming_mask_regular_known_answer():
    # regular (2, 1), cache 3 (filled 2), chunk 3: query i at frame 3+i sees
    # frames 3+i-2 .. 3+i+1, and frame 0 is unfilled
    m = O.create_attention_mask((2, 1), "regular", 6, 3, 2, 3, 3)[0].astype(int)
    expect = np.array([[0, 1, 1, 1, 1, 0],
                       [0, 0, 1, 1, 1, 1],
                       [0, 0, 0, 1, 1, 1]])
    assert (m == expect).all()
    # valid length 2: the last query row sees nothing
    m2 = O.create_attention_mask((2, 1), "regular", 6, 3, 2, 3, 2)[0].astype(int)
    assert (m2[:2] == expect[:2]).all() and (m2[2] == 0).all()


def test_streaming_mask_chunked_known_answer():
    # chunked_limited (2, 1): chunk 2, 1 left chunk; cache 4 (full), 2 queries at frames 4, 5
    m = O.create_attention_mask((2, 1), "chunked_limited", 6, 4, 4, 2, 2)[0].astype(int)
    expect = np.array([[0, 0, 1, 1, 1, 1],
                       [0, 0, 1, 1, 1, 1]])
    assert (m == expect).all()
    # unlimited right context: only triu(-left) (conformer.rs:126-130)
    m = O.create_attention_mask((1, -1), "chunked_limited", 5, 3, 3, 2, 2)[0].astype(int)
    assert (m == np.array([[0, 0, 1, 1, 1], [0, 0, 0, 1, 1]])).all()


def test_streaming_mask_kinds():
    assert O.streaming_mask(None, "regular", 4, 0, 2, 2) is None
    assert O.streaming_mask((70, 13), "chunked_limited", 70, 70, 14, 14) is None
    add = O.streaming_mask((70, 13), "chunked_limited", 70, 10, 14, 14)
    assert add.dtype == np.float64 and np.isneginf(add).any()
    bm = O.streaming_mask((70, 13), "chunked_limited", 70, 10, 14, 12)
    assert bm.dtype == np.bool_ and not bm[0, 13].any()


def test_cache_update_known_answer():
    cache = np.arange(1, 6, dtype=np.float64).reshape(1, 5, 1)  # rows 1..5
    x = np.arange(10, 13, dtype=np.float64).reshape(1, 3, 1)  # rows 10..12
    assert list(O.cache_update(cache, x, 0)[0, :, 0]) == [4, 5, 10, 11, 12]
    assert list(O.cache_update(cache, x, 1)[0, :, 0]) == [3, 4, 5, 10, 11]
    assert list(O.cache_update(cache, x, 3)[0, :, 0]) == [1, 2, 3, 4, 5]
    small = np.arange(1, 3, dtype=np.float64).reshape(1, 2, 1)
    # more kept frames than the cache holds: newest rows win (conformer.rs:994-997)
    assert list(O.cache_update(small, x, 0)[0, :, 0]) == [11, 12]
    assert O.next_fill(60, 14, 0, 70) == 70 and O.next_fill(0, 14, 0, 70) == 14
    assert O.next_fill(5, 14, 20, 70) == 5


@pytest.mark.parametrize("kind", ["none", "additive", "bool"])
def test_streaming_forward_matches_definition(kind):
    d, h, C, T = 16, 2, 6, 3
    p = random_params(d, h, seed=7)
    rng = np.random.default_rng(8)
    x = rng.standard_normal((2, T, d))
    filled, valid = (6, T) if kind == "none" else ((4, T) if kind == "additive" else (4, 2))
    cache = rng.standard_normal((2, C, d))
    cache[:, : C - filled, :] = 0.0
    pos = O.RelPositionalEncoding(d, 64, False).get_encoding(C + T)
    mask = O.streaming_mask((4, 1), "regular", C, filled, T, valid)
    if kind == "none":
        mask = O.streaming_mask(None, "regular", C, filled, T, valid)
        assert mask is None
    else:
        assert (mask.dtype == np.bool_) == (kind == "bool")
    out, nc = O.mhsa_forward_with_cache(p, x, pos, cache, mask)
    vis = np.ones((2, T, C + T), dtype=bool)
    if kind != "none":
        for i in range(T):
            for j in range(C + T):
                fi = C + i
                vis[:, i, j] = (j - fi >= -4) and (j - fi <= 1) and j >= C - filled and i < valid
    # the unfused bool path divides by the f32 sqrt(d_k) (attention.rs:784)
    scale = 1.0 / float(np.sqrt(np.float32(p.head_dim))) if kind == "bool" else None
    ref = direct_attention(p, x, np.concatenate([cache, x], 1), pos, C, vis, scale=scale)
    assert np.max(np.abs(out - ref)) < 1e-10
    assert (nc == np.concatenate([cache[:, T:], x], 1)).all()


@pytest.mark.parametrize("quantized", [False, True])
def test_streaming_bf16_is_f32_math_on_bf16_parameters(quantized):
    """bf16 streaming (f32 cache and chunk, attention.rs:606-816 under MLX
    promotion): equals the definition evaluated in float64 on the cast
    parameters -- dense weights, biases and pos biases rounded to bf16,
    quantized weights dequantised in f32 from bf16-rounded scales and biases
    (the already pinned f32 dequantisation of pre-rounded inputs) -- with the
    position rows the bf16 projection of the bf16 table (pinned by the
    native-bf16 restatement), and the position term scaled by the f32 scale."""
    d, h, C, T = 128, 2, 6, 3
    rng = np.random.default_rng(21)
    if quantized:
        import workloads as W
        from _util import oracle_params
        w = W.make_layer_weights(rng, d, h, True, True)
        for name in ("linear_q", "linear_k", "linear_v", "linear_out"):
            w[f"{name}.bias"] = rng.normal(0, 0.1, d).astype(np.float16)
        p = oracle_params(w, d, h)
    else:
        p = random_params(d, h, seed=22, scale=0.1)
    x = rng.standard_normal((2, T, d)).astype(np.float32).astype(np.float64)
    cache = rng.standard_normal((2, C, d)).astype(np.float32).astype(np.float64)
    pos = O.bf16_round(O.RelPositionalEncoding(d, 64, False).get_encoding(C + T))
    out, _ = O.mhsa_forward_with_cache(p, x, pos, cache, None, dtype=O.BF16)

    def cast(lin):
        if lin.is_quantized:
            s16 = O.bf16_round(np.asarray(lin.scales, dtype=np.float32))
            b16 = O.bf16_round(np.asarray(lin.biases, dtype=np.float32))
            wt = O.dequantize(lin.weight, s16, b16, lin.bits, lin.group_size, O.F32)
        else:
            wt = O.bf16_round(lin.weight)
        return O.LinearLayer(wt, None if lin.bias is None else O.bf16_round(lin.bias))

    pc = O.MhsaParams(d, h, cast(p.linear_q), cast(p.linear_k), cast(p.linear_v), cast(p.linear_out),
                      cast(p.linear_pos), O.bf16_round(p.pos_bias_u), O.bf16_round(p.pos_bias_v))
    P = p.linear_pos.forward(pos[0], O.BF16)
    vis = np.ones((2, T, C + T), dtype=bool)
    ref = direct_attention(pc, x, np.concatenate([cache, x], 1), pos, C, vis, P=P)
    assert np.max(np.abs(out - ref)) < 1e-9 * np.max(np.abs(ref))
    # and it is not the all-bf16 arithmetic of the offline bf16 forward
    rounded = O.bf16_round(ref)
    assert np.max(np.abs(out - rounded)) > 0


def test_streaming_chunk_equals_offline_rows():
    # A full cache holding the previous frames and no mask: the chunk's outputs
    # equal the last T rows of offline attention over cache + chunk.
    d, h, C, T = 16, 2, 5, 4
    p = random_params(d, h, seed=9)
    rng = np.random.default_rng(10)
    seq = rng.standard_normal((1, C + T, d))
    pos = O.RelPositionalEncoding(d, 64, False).get_encoding(C + T)
    out, _ = O.mhsa_forward_with_cache(p, seq[:, C:], pos, seq[:, :C], None)
    # offline over all C+T frames, keeping only the last T query rows
    full = O.mhsa_forward(p, seq, pos)
    assert np.max(np.abs(out - full[:, C:])) < 1e-10


# ---------------------------------------------------------------------------
# FeedForward (conformer.rs:2031-2088) and the half-step sublayer
# ---------------------------------------------------------------------------

def _ffn_params(d, f, seed, scale=0.5):
    rng = np.random.default_rng(seed)
    return O.FeedForwardParams(O.LinearLayer(rng.standard_normal((f, d)) * scale, rng.standard_normal(f) * scale),
                               O.LinearLayer(rng.standard_normal((d, f)) * scale, rng.standard_normal(d) * scale))


def test_feed_forward_f32_matches_torch():
    p = _ffn_params(16, 64, 31, scale=0.3)
    x = np.random.default_rng(32).standard_normal((5, 16))
    xt = torch.tensor(x, dtype=torch.float64)
    h = torch.nn.functional.silu(torch.nn.functional.linear(xt, torch.tensor(p.linear1.weight),
                                                              torch.tensor(p.linear1.bias)))
    ref = torch.nn.functional.linear(h, torch.tensor(p.linear2.weight), torch.tensor(p.linear2.bias)).numpy()
    assert np.max(np.abs(O.feed_forward(p, x) - ref)) < 1e-12


def test_feed_forward_bf16_equals_native_bf16_restatement():
    """bf16 tensors round every op result: linear (matmul, bias add),
    sigmoid, the product (nn::silu as two ops), linear2; then the half-step
    residual 0.5 * y + x."""
    p = _ffn_params(16, 64, 33)
    x = O.bf16_round(np.random.default_rng(34).standard_normal((7, 16)))
    bf = torch.bfloat16
    t = lambda a: torch.tensor(np.asarray(a, dtype=np.float32)).to(bf)
    X = t(x)
    h = X @ t(p.linear1.weight).T + t(p.linear1.bias)
    h = h * torch.sigmoid(h)
    y = h @ t(p.linear2.weight).T + t(p.linear2.bias)
    assert np.array_equal(O.feed_forward(p, x, O.BF16), y.double().numpy())
    half = torch.tensor(0.5, dtype=bf)
    s = (X + half * y).double().numpy()
    yo = O.feed_forward(p, x, O.BF16)
    assert np.array_equal(O.bf16_round(x + O.bf16_round(0.5 * yo)), s)
    # the sublayer on an input whose LayerNorm is the identity-free case
    sub = O.feed_forward_sublayer(p, x, dtype=O.BF16)
    assert np.array_equal(sub, O.bf16_round(x + 0.5 * O.feed_forward(p, O.layer_norm(x, dtype=O.BF16), O.BF16)))


# ---------------------------------------------------------------------------
# ConvolutionModule (conformer.rs:2105-2437)
# ---------------------------------------------------------------------------

def _conv_params(d, k, norm, causal, seed, use_bias=True):
    from _util import conv_oracle, conv_weights
    return conv_oracle(conv_weights(np.random.default_rng(seed), d, k, norm, False, use_bias), norm, causal)


def _torch_conv_module(p, x, lengths=None, left=None):
    """The module from torch library routines in float64: linear, F.glu,
    F.conv1d (groups = channels), F.batch_norm (inference) or F.layer_norm,
    F.silu, linear."""
    F = torch.nn.functional
    T_ = lambda a: None if a is None else torch.tensor(np.asarray(a, dtype=np.float64))
    xt = T_(x)
    d = xt.shape[-1]
    h = F.linear(xt, T_(p.pointwise_conv1.weight), T_(p.pointwise_conv1.bias))
    u = F.glu(h, dim=-1)
    if lengths is not None:
        valid = torch.arange(u.shape[1])[None, :] < torch.tensor(lengths)[:, None]
        u = u * valid[:, :, None]
    k = p.kernel_size
    ut = u.transpose(1, 2)  # [B, D, T]
    if p.causal:
        ut = F.pad(ut, (k - 1, 0))
        pad = 0
    else:
        pad = (k - 1) // 2
    w = T_(p.depthwise_weight).permute(0, 2, 1)  # [D, 1, K]
    y = F.conv1d(ut, w, T_(p.depthwise_bias), padding=pad, groups=d).transpose(1, 2)
    if p.norm == "batch_norm":
        y = F.batch_norm(y.transpose(1, 2), T_(p.running_mean), T_(p.running_var), T_(p.norm_weight),
                         T_(p.norm_bias), training=False, eps=1e-5).transpose(1, 2)
    else:
        y = F.layer_norm(y, (d,), T_(p.norm_weight), T_(p.norm_bias), eps=1e-5)
    y = F.silu(y)
    return F.linear(y, T_(p.pointwise_conv2.weight), T_(p.pointwise_conv2.bias)).numpy()


@pytest.mark.parametrize("norm,causal,k,lengths", [("batch_norm", False, 9, None), ("batch_norm", True, 9, [11, 6]),
                                                   ("layer_norm", True, 4, None), ("layer_norm", False, 31, [3, 11]),
                                                   ("batch_norm", False, 1, [11, 0])])
def test_conv_module_f32_matches_torch(norm, causal, k, lengths):
    """Structure and order of the module (GLU halves, padding zeroed before
    the conv, cross-correlation over the causal / symmetric window, the
    norm, SiLU) against torch's own conv1d / batch_norm / layer_norm / glu."""
    p = _conv_params(16, k, norm, causal, 40 + k)
    x = np.random.default_rng(41).standard_normal((2, 11, 16))
    got, cache = O.conv_module(p, x, O.F32, lengths=lengths)
    assert cache is None
    ref = _torch_conv_module(p, x, lengths)
    assert np.max(np.abs(got - ref)) < 1e-12


@pytest.mark.parametrize("chunk", [5, 3, 13])
def test_conv_cache_chunks_equal_offline_causal(chunk):
    """Streaming a causal module chunk by chunk through its [B, D, K-1]
    cache, starting from zeros, reproduces the offline forward of the whole
    sequence (the left zero padding is the initial cache), whatever the
    chunk size relative to K-1 = 8; the cache after each chunk holds the
    last K-1 GLU frames of everything seen (or zeros before them)."""
    d, k, T = 16, 9, 27
    p = _conv_params(d, k, "layer_norm", True, 42)
    x = np.random.default_rng(43).standard_normal((2, T, d))
    whole, _ = O.conv_module(p, x, O.F32)
    cache = np.zeros((2, d, k - 1))
    outs = []
    for t0 in range(0, T, chunk):
        y, cache = O.conv_module(p, x[:, t0:t0 + chunk], O.F32, cache=cache)
        outs.append(y)
        seen = O.glu(O.LinearLayer.forward(p.pointwise_conv1, x[:, :t0 + y.shape[1]]), d, O.F32)
        want = np.concatenate([np.zeros((2, k - 1, d)), seen], axis=1)[:, -(k - 1):]
        assert np.max(np.abs(cache - np.transpose(want, (0, 2, 1)))) < 1e-12
    assert np.max(np.abs(np.concatenate(outs, axis=1) - whole)) < 1e-12
    with pytest.raises(ValueError):
        O.conv_module(_conv_params(d, k, "layer_norm", False, 42), x, O.F32, cache=cache)


def _bf16_rsqrt(s):
    """rsqrt of a bf16 tensor, correctly rounded to bf16 (torch's CPU bf16
    rsqrt is off by 1-2 ulps on some inputs; the value is a float64 sqrt and
    division, rounded once through f32)."""
    return (1.0 / torch.sqrt(s.double())).float().to(torch.bfloat16)


def test_conv_module_bf16_symmetric_equals_native_bf16_restatement():
    """A symmetric bf16 module stays bf16: every op result is rounded --
    pointwise matmul and bias add, sigmoid, GLU product, depthwise conv and
    its bias add, (x - mean), rsqrt(var + eps) with eps cast to bf16, the
    product, weight * x, + bias, sigmoid, SiLU product, pointwise_conv2."""
    d, k = 16, 5
    p = _conv_params(d, k, "batch_norm", False, 44)
    x = O.bf16_round(np.random.default_rng(45).standard_normal((2, 9, d)))
    bf = torch.bfloat16
    t = lambda a: torch.tensor(np.asarray(a, dtype=np.float32)).to(bf)
    h = t(x) @ t(p.pointwise_conv1.weight).T + t(p.pointwise_conv1.bias)
    u = h[..., :d] * torch.sigmoid(h[..., d:])
    up = torch.nn.functional.pad(u.double(), (0, 0, 2, 2))
    w = t(p.depthwise_weight[:, :, 0]).double()  # [D, K]
    y = sum(up[:, j:j + 9, :] * w[:, j] for j in range(k)).to(bf) + t(p.depthwise_bias)
    y = (y - t(p.running_mean)) * _bf16_rsqrt(t(p.running_var) + torch.tensor(1e-5).to(bf))
    y = t(p.norm_weight) * y + t(p.norm_bias)
    y = y * torch.sigmoid(y)
    ref = y @ t(p.pointwise_conv2.weight).T + t(p.pointwise_conv2.bias)
    got, _ = O.conv_module(p, x, O.BF16)
    assert np.array_equal(got, ref.double().numpy())


def test_conv_module_bf16_causal_promotes_to_f32():
    """A causal bf16 module: pointwise_conv1 and the GLU in bf16, then the
    f32 zero padding promotes the conv, norm, SiLU and pointwise_conv2 to f32
    with bf16-valued parameters -- except rsqrt(var + eps), which involves
    bf16 parameters only and stays bf16. torch applies the same promotion
    rules; its f32 ops round to f32, the oracle does not (1e-6 apart)."""
    d, k = 16, 4
    p = _conv_params(d, k, "batch_norm", True, 46)
    x = O.bf16_round(np.random.default_rng(47).standard_normal((2, 9, d)))
    bf = torch.bfloat16
    t = lambda a: torch.tensor(np.asarray(a, dtype=np.float32)).to(bf)
    h = t(x) @ t(p.pointwise_conv1.weight).T + t(p.pointwise_conv1.bias)
    u = h[..., :d] * torch.sigmoid(h[..., d:])
    up = torch.cat([torch.zeros(2, k - 1, d, dtype=torch.float32), u], dim=1)  # f32 zeros promote
    assert up.dtype == torch.float32
    w = t(p.depthwise_weight[:, :, 0])
    y = sum(up[:, j:j + 9, :] * w[:, j] for j in range(k)) + t(p.depthwise_bias)
    assert y.dtype == torch.float32
    s = t(p.running_var) + torch.tensor(1e-5).to(bf)
    assert s.dtype == bf

    def tail(inv):
        z = (y - t(p.running_mean)) * inv
        z = t(p.norm_weight) * z + t(p.norm_bias)
        z = z * torch.sigmoid(z)
        return (z @ t(p.pointwise_conv2.weight).float().T + t(p.pointwise_conv2.bias)).double().numpy()

    ref = tail(_bf16_rsqrt(s))
    got, _ = O.conv_module(p, x, O.BF16)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 1e-6
    # the bf16 rounding of the rsqrt term is load-bearing: an f32 one moves the result
    alt = tail(torch.rsqrt(s.float()))
    assert np.max(np.abs(alt - got)) / np.max(np.abs(ref)) > 1e-4


def test_feed_forward_promoted_matches_torch_promotion():
    """f32 activations through a bf16 FeedForward: torch's own type
    promotion of an f32 tensor against bf16 parameters gives the oracle's
    promoted form (f32 ops on bf16-valued weights, no bf16 rounding), within
    torch's f32 rounding; the bf16-rounded module form differs by far more."""
    p = _ffn_params(16, 64, 35)
    x = np.random.default_rng(36).standard_normal((5, 16)).astype(np.float32)
    bf = torch.bfloat16
    t = lambda a: torch.tensor(np.asarray(a, dtype=np.float32)).to(bf)
    X = torch.tensor(x)
    h = X @ t(p.linear1.weight).float().T + t(p.linear1.bias)
    assert h.dtype == torch.float32
    h = h * torch.sigmoid(h)
    y = (h @ t(p.linear2.weight).float().T + t(p.linear2.bias)).double().numpy()
    got = O.feed_forward(p, x, O.BF16, act=O.F32)
    assert np.max(np.abs(got - y)) / np.max(np.abs(y)) < 1e-6
    assert np.max(np.abs(O.feed_forward(p, O.bf16_round(x), O.BF16) - got)) / np.max(np.abs(y)) > 1e-3


# ---------------------------------------------------------------------------
# ConformerBlock (conformer.rs:1693-1971)
# ---------------------------------------------------------------------------

def _block_params(d, h, f, k, seed, causal=True, zero=()):
    """A block with random modules and norms; modules named in `zero` output
    exactly 0 (FeedForward: linear2 zero; attention: linear_out zero;
    conv: pointwise_conv2 zero)."""
    rng = np.random.default_rng(seed)
    ff1, ff2 = _ffn_params(d, f, seed + 1, 0.3), _ffn_params(d, f, seed + 2, 0.3)
    attn = random_params(d, h, seed + 3, scale=0.3)
    conv = _conv_params(d, k, "layer_norm", causal, seed + 4)
    zl = lambda lin: O.LinearLayer(np.zeros_like(lin.weight), None if lin.bias is None else np.zeros_like(lin.bias))
    if "ff1" in zero:
        ff1 = O.FeedForwardParams(ff1.linear1, zl(ff1.linear2))
    if "ff2" in zero:
        ff2 = O.FeedForwardParams(ff2.linear1, zl(ff2.linear2))
    if "attn" in zero:
        attn.linear_out = zl(attn.linear_out)
    if "conv" in zero:
        conv.pointwise_conv2 = zl(conv.pointwise_conv2)
    norm = lambda: (1.0 + 0.2 * rng.standard_normal(d), 0.2 * rng.standard_normal(d))
    return O.ConformerBlockParams(ff1, norm(), attn, norm(), conv, norm(), ff2, norm(), norm())


def _torch_ln(x, nw):
    F = torch.nn.functional
    return F.layer_norm(torch.tensor(x), (x.shape[-1],), torch.tensor(nw[0]), torch.tensor(nw[1]), eps=1e-5).numpy()


def _torch_ffn(p, x):
    F = torch.nn.functional
    xt = torch.tensor(x)
    hh = F.silu(F.linear(xt, torch.tensor(p.linear1.weight), torch.tensor(p.linear1.bias)))
    return F.linear(hh, torch.tensor(p.linear2.weight), torch.tensor(p.linear2.bias)).numpy()


@pytest.mark.parametrize("live", [("ff1",), ("attn",), ("conv",), ("ff2",), ("ff1", "attn"), ("attn", "conv"),
                                  ("conv", "ff2"), ("ff1", "attn", "conv", "ff2")])
def test_conformer_block_sublayer_order(live):
    """The block from library routines and the definition-based attention
    (torch layer_norm / linear / silu / conv1d, `direct_attention`), in the
    order conformer.rs:1693-1875 runs them: x += 0.5 FF1(LN1 x); x +=
    MHSA(LN2 x); x += conv(LN3 x); x += 0.5 FF2(LN4 x); norm_out. Modules not
    in `live` output zero; with two or more live, a swapped order changes the
    result (checked), so the comparison pins the order, the half steps and
    each residual."""
    d, h, f, k, T = 16, 2, 32, 5, 9
    p = _block_params(d, h, f, k, 50, zero=tuple(m for m in ("ff1", "attn", "conv", "ff2") if m not in live))
    x = np.random.default_rng(51).standard_normal((2, T, d))
    pos = O.RelPositionalEncoding(d, 64, False).get_encoding(T)
    vis = np.ones((2, T, T), dtype=bool)
    steps = {
        "ff1": lambda y: y + 0.5 * _torch_ffn(p.ff1, _torch_ln(y, p.ff1_norm)),
        "attn": lambda y: y + direct_attention(p.attn, _torch_ln(y, p.attn_norm), _torch_ln(y, p.attn_norm), pos, 0,
                                               vis),
        "conv": lambda y: y + _torch_conv_module(p.conv, _torch_ln(y, p.conv_norm)),
        "ff2": lambda y: y + 0.5 * _torch_ffn(p.ff2, _torch_ln(y, p.ff2_norm)),
    }
    order = ["ff1", "attn", "conv", "ff2"]
    y = x
    for m in order:
        y = steps[m](y)
    ref = _torch_ln(y, p.out_norm)
    got = O.conformer_block(p, x, pos, None, None, O.F32)
    assert np.max(np.abs(got - ref)) < 1e-10
    if len(live) > 1:
        y = x
        for m in reversed(order):
            y = steps[m](y)
        assert np.max(np.abs(_torch_ln(y, p.out_norm) - ref)) > 1e-3


def test_conformer_block_key_padding_and_conv_padding():
    """Padding from lengths (PaddingMask, conformer.rs:1594-1615): keys past
    each length are hidden from attention (length 0 keeps key 0, the
    reference's clamp) and the conv zeroes those frames after its GLU; with
    every length >= T there is no mask at all."""
    d, h, f, k, T = 16, 2, 32, 5, 9
    p = _block_params(d, h, f, k, 52, causal=False)
    x = np.random.default_rng(53).standard_normal((3, T, d))
    pos = O.RelPositionalEncoding(d, 64, False).get_encoding(T)
    lengths = [T, 4, 0]
    got = O.conformer_block(p, x, pos, None, lengths, O.F32)
    vis = np.zeros((3, T, T), dtype=bool)
    for b, ln in enumerate(lengths):
        vis[b, :, :max(ln, 1)] = True
    y = x + 0.5 * _torch_ffn(p.ff1, _torch_ln(x, p.ff1_norm))
    hn = _torch_ln(y, p.attn_norm)
    y = y + direct_attention(p.attn, hn, hn, pos, 0, vis)
    y = y + _torch_conv_module(p.conv, _torch_ln(y, p.conv_norm), lengths)
    y = y + 0.5 * _torch_ffn(p.ff2, _torch_ln(y, p.ff2_norm))
    assert np.max(np.abs(got - _torch_ln(y, p.out_norm))) < 1e-10
    assert np.array_equal(O.conformer_block(p, x, pos, None, [T, T + 3, T], O.F32),
                          O.conformer_block(p, x, pos, None, None, O.F32))


def test_conformer_block_streaming_equals_offline_chunked():
    """The cache-aware block over consecutive chunks, from empty caches
    (attention fill 0, conv cache zeros), equals the offline block over the
    whole sequence under the same chunked_limited context with a causal
    conv: rows are row-wise through FF / LayerNorm, the attention cache holds
    the normalised inputs h that offline attention reads as keys, the
    streaming mask hides exactly the keys outside the chunk window, and the
    conv cache is the causal left context."""
    d, h, f, k = 16, 2, 32, 5
    C, T, n = 8, 4, 4
    p = _block_params(d, h, f, k, 54, causal=True)
    seq = np.random.default_rng(55).standard_normal((1, n * T, d))
    ctx = ((C, T - 1), "chunked_limited")
    whole = O.conformer_block(p, seq, O.RelPositionalEncoding(d, 64, False).get_encoding(n * T),
                              O.AttentionContext.new(*ctx), None, O.F32)
    att, conv, fill = np.zeros((1, C, d)), np.zeros((1, d, k - 1)), 0
    pos = O.RelPositionalEncoding(d, 64, False).get_encoding(C + T)
    for c in range(n):
        m = O.streaming_mask(ctx[0], ctx[1], C, fill, T, T)
        y, att, conv = O.conformer_block_with_cache(p, seq[:, c * T:(c + 1) * T], pos, att, conv, m, None, O.F32)
        assert np.max(np.abs(y - whole[:, c * T:(c + 1) * T])) < 1e-10, c
        fill = O.next_fill(fill, T, 0, C)


def _bf16_cast_block(p):
    """The block's parameters as set_dtype(bf16) leaves them: every dense
    weight, bias and norm parameter rounded to bf16 (the block's own dtype
    stays f32 here)."""
    r = lambda a: None if a is None else O.bf16_round(np.asarray(a, dtype=np.float64))
    lin = lambda l: O.LinearLayer(r(l.weight), r(l.bias))
    ffn = lambda f: O.FeedForwardParams(lin(f.linear1), lin(f.linear2))
    a = p.attn
    attn = O.MhsaParams(a.d_model, a.n_heads, lin(a.linear_q), lin(a.linear_k), lin(a.linear_v), lin(a.linear_out),
                        lin(a.linear_pos), r(a.pos_bias_u), r(a.pos_bias_v))
    c = p.conv
    conv = O.ConvModuleParams(lin(c.pointwise_conv1), r(c.depthwise_weight), r(c.depthwise_bias),
                              lin(c.pointwise_conv2), c.norm, r(c.norm_weight), r(c.norm_bias), r(c.running_mean),
                              r(c.running_var), c.causal)
    nrm = lambda pair: (r(pair[0]), r(pair[1]))
    return O.ConformerBlockParams(ffn(p.ff1), nrm(p.ff1_norm), attn, nrm(p.attn_norm), conv, nrm(p.conv_norm),
                                  ffn(p.ff2), nrm(p.ff2_norm), nrm(p.out_norm))


@pytest.mark.parametrize("causal,ctx,lengths", [(True, None, [9, 6]), (False, ((3, 2), "regular"), None),
                                                (True, ((8, 1), "chunked_limited"), [9, 1])])
def test_conformer_block_f32_activations_is_the_f32_block_on_bf16_parameters(causal, ctx, lengths):
    """A bf16 block on activations an earlier causal conv made f32 runs every
    op in f32 on the bf16 parameter values (MLX promotion). With the conv's
    norm a LayerNorm (BatchNorm's rsqrt term stays bf16) and linear_pos the
    identity over a bf16 table (so its rows are exact in either dtype), that
    is the f32 block on bf16-rounded parameters, equal in every output (the
    two store the same f32 roundings), while the all-bf16 block is 1e-2
    off. (The contexts keep key
    0 in every row's window: a row that sees no key is NaN in the
    reference.)"""
    d, h, f, k, T = 16, 2, 32, 5, 9
    p = _block_params(d, h, f, k, 56, causal=causal)
    p.attn.linear_pos = O.LinearLayer(np.eye(d), None)
    x = np.random.default_rng(57).standard_normal((2, T, d)).astype(np.float32).astype(np.float64)
    pos = O.bf16_round(O.RelPositionalEncoding(d, 64, False).get_encoding(T))
    context = O.AttentionContext.new(*ctx) if ctx else None
    got = O.conformer_block(p, x, pos, context, lengths, O.BF16, act=O.F32)
    ref = O.conformer_block(_bf16_cast_block(p), x, pos, context, lengths, O.F32)
    scale = np.max(np.abs(ref))
    assert np.array_equal(got, ref)
    assert np.max(np.abs(O.conformer_block(p, O.bf16_round(x), pos, context, lengths, O.BF16) - got)) / scale > 1e-3


def test_conformer_encoder_promotes_after_the_first_causal_conv():
    """conformer_encoder: a bf16 stack keeps bf16 activations through
    symmetric blocks and turns f32 at the first causal one; every later
    block then takes f32 activations (conformer.rs:542-550 calls each block
    on the previous block's returned array)."""
    d, h, f, k, T = 16, 2, 32, 5, 7
    ps = [_block_params(d, h, f, k, 60 + 5 * i, causal=c) for i, c in enumerate((False, True, True))]
    x = O.bf16_round(np.random.default_rng(61).standard_normal((1, T, d)))
    pos = O.bf16_round(O.RelPositionalEncoding(d, 64, False).get_encoding(T))
    out, act = O.conformer_encoder(ps, x, pos, None, None, O.BF16)
    assert act == O.F32
    y0 = O.conformer_block(ps[0], x, pos, None, None, O.BF16)
    assert np.array_equal(y0, O.bf16_round(y0))  # still bf16 after the symmetric block
    y1 = O.conformer_block(ps[1], y0, pos, None, None, O.BF16)
    assert not np.array_equal(y1, O.bf16_round(y1))  # f32 after the causal one
    y2 = O.conformer_block(ps[2], y1, pos, None, None, O.BF16, act=O.F32)
    assert np.array_equal(out, y2)
    # an f32 stack never changes dtype
    assert O.conformer_encoder(ps, x, pos, None, None, O.F32)[1] == O.F32
