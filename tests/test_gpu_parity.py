"""GPU parity of the HIP rel-pos MHSA path against the CPU oracle.

Tolerances (stated by the path's contract):
* fp32: per output row, max |gpu - oracle| / max |oracle| <= 1e-4 ("max
  relative error", read row by row),
* bf16: max |gpu - oracle| <= 2e-2 (absolute),
* dequantised int8 weights, masks and rel_shift index maps: bit-exact.

Rows whose queries see no key at all are excluded from offline comparisons
(the reference leaves them unspecified, conformer.rs:1590-1593); streaming
rows past the valid length must be exactly the output bias, as the
reference's bool-mask path gives.
"""
import numpy as np
import pytest
import torch

import relpos_oracle as O
import relpos_mhsa as M
import workloads as W
from _util import abs_err, oracle_params, random_weights, rel_err, row_rel_err

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4
BF16_TOL = 2e-2


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    M.library()
    yield
    torch.cuda.synchronize()


def dev(a, dtype):
    t = torch.from_numpy(np.ascontiguousarray(np.asarray(a, dtype=np.float32)))
    return t.to("cuda").to(torch.float32 if dtype == O.F32 else torch.bfloat16).contiguous()


def host(t):
    return t.float().cpu().numpy().astype(np.float64)


def gpu_layer(weights, d_model, n_heads, use_bias, dtype, prefix="layer"):
    layer = M.RelPositionMultiHeadAttention(d_model, n_heads, use_bias)
    layer.load_weights(W.prefixed(weights, prefix), prefix)
    layer.set_dtype(dtype)
    return layer


def visible_rows(B, T, ctx, lengths):
    """[B, T] True where the query sees at least one key."""
    vis = np.ones((B, T), dtype=bool)
    if ctx is None and lengths is None:
        return vis
    for b in range(B):
        m = ctx.block_visible(0, T, T) if ctx is not None else np.ones((T, T), dtype=bool)
        if lengths is not None:
            m = m & (np.arange(T)[None, :] < max(lengths[b], 1))
        vis[b] = m.any(axis=1)
    return vis


# ---------------------------------------------------------------------------
# bit-exact index maps, masks and dequantisation
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("rows,total", [(1, 1), (3, 3), (5, 5), (13, 13), (14, 84), (7, 30), (125, 125)])
def test_rel_shift_index_bitexact(rows, total):
    pos_len = 2 * total - 1
    got = M.debug_rel_shift_index(rows, total).cpu().numpy()
    flat = O.rel_shift_index(rows, total, pos_len)
    assert (flat >= 0).all()
    assert (flat // pos_len == np.arange(rows)[:, None]).all()  # never crosses rows
    assert np.array_equal(got, flat % pos_len)


CONTEXTS = [None, ((56, 3), "chunked_limited"), ((5, 1), "chunked_limited"), ((-1, 2), "chunked_limited"),
            ((4, -1), "chunked_limited"), ((3, 2), "regular"), ((-1, 0), "regular"), ((128, 128), "regular")]


@pytest.mark.parametrize("ctx", CONTEXTS)
def test_offline_mask_bitexact(ctx):
    T, lengths = 23, [23, 9, 1, 0, 40]
    context = M.AttentionContext.new(*ctx) if ctx else None
    octx = O.AttentionContext.new(*ctx) if ctx else None
    got = M.debug_offline_mask(len(lengths), T, context, lengths).cpu().numpy().astype(bool)
    for b, ln in enumerate(lengths):
        ref = octx.block_visible(0, T, T) if octx else np.ones((T, T), dtype=bool)
        km = O.key_padding_mask(lengths, T)
        if km is not None:
            ref = ref & (km[b, 0, 0] == 0.0)[None, :]
        assert np.array_equal(got[b], ref), (ctx, b)


@pytest.mark.parametrize("ctx,C,T", [((70, 13), 70, 14), ((2, 1), 3, 3), ((2, 1), 4, 2), ((1, -1), 3, 2),
                                     ((5, 2), 6, 3)])
@pytest.mark.parametrize("style", ["chunked_limited", "regular"])
def test_stream_mask_bitexact(ctx, C, T, style):
    fills = [0, C // 2, C, 1 if C else 0]
    valid = [T, T - 1, 0, T]
    mask = M.StreamingMask(ctx, style, fills, valid)
    got = M.debug_stream_mask(len(fills), C, T, mask).cpu().numpy().astype(bool)
    for b in range(len(fills)):
        ref = O.create_attention_mask(ctx, style, C + T, C, fills[b], T, valid[b])[0]
        assert np.array_equal(got[b], ref), (b, fills[b], valid[b])


@pytest.mark.parametrize("dtype", [O.F32, O.BF16])
def test_dequantize_bitexact(dtype):
    rng = np.random.default_rng(21)
    w = W.make_layer_weights(rng, 256, 2, False, True)
    layer = gpu_layer(w, 256, 2, False, dtype)
    for name in ("linear_q", "linear_pos"):
        got = layer.debug_dequantize(name).cpu().numpy().astype(np.float64)
        ref = O.dequantize(w[f"{name}.weight"], w[f"{name}.scales"], w[f"{name}.biases"], 8, 64, dtype)
        assert np.array_equal(got, ref), name


# ---------------------------------------------------------------------------
# the fused kernel's position scores (MFMA band + LDS rel_shift remap)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("d_model,n_heads,T", [(128, 2, 37), (256, 2, 70), (256, 2, 16)])
def test_position_scores_match_rel_shift(d_model, n_heads, T):
    rng = np.random.default_rng(3)
    w = random_weights(rng, d_model, n_heads)
    p = oracle_params(w, d_model, n_heads)
    x = rng.standard_normal((2, T, d_model)).astype(np.float32)
    pos = O.RelPositionalEncoding(d_model, 5000, False).get_encoding(T)
    layer = gpu_layer(w, d_model, n_heads, True, O.F32)
    got = host(layer.debug_position_scores(dev(x, O.F32), dev(pos, O.F32)))
    # oracle: scale * rel_shift((q + v) P^T)[..., :T] as attention.rs:503-532 writes it
    h, dk = n_heads, d_model // n_heads
    q = p.linear_q.forward(x.astype(np.float64)).reshape(2, T, h, dk).transpose(0, 2, 1, 3)
    P = p.linear_pos.forward(pos[0].astype(np.float64)).reshape(2 * T - 1, h, dk).transpose(1, 0, 2)
    bd = np.matmul(q + p.pos_bias_v.reshape(1, h, 1, dk), np.swapaxes(P, -1, -2)[None])
    ref = O.f32_scale(dk) * O.rel_shift(bd)[..., :T]
    assert row_rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("d_model,n_heads,B,T", [(256, 2, 2, 37), (256, 2, 2, 100), (256, 2, 2, 300),
                                                 (2048, 16, 5, 520)])
def test_position_scores_bf16_match_rel_shift(d_model, n_heads, B, T):
    """bf16 path (32x32 MFMA band with carried band tile, bf16 remap strip;
    the last shape gives 240 blocks of 256 queries, which take the 8-wave
    form with 32-key tiles, the others the 4-wave form with 64-key tiles):
    bd is stored in bf16 as the reference stores matrix_bd (attention.rs:530),
    from q_v = bf16(q + v) as the reference forms it (attention.rs:501-508),
    and the exported term is bf16(bd * bf16(s)) as `attend` materialises it
    (attention.rs:308-311). Starting from the kernel's own bf16 q and P (the
    projections are pinned separately), each term is bf16-representable and
    lies between bf16(bf16(x) * bf16(s)) at x = rel_shift(q_v P^T) -/+ the
    fp32 accumulation bound of its d_k products (the three roundings are
    monotone): the exact term's value, except where the kernel's fp32 band
    sum sits within accumulation noise of a bf16 rounding boundary of bd (the
    neighbouring value) or cancels to far below its products."""
    rng = np.random.default_rng(4)
    w = random_weights(rng, d_model, n_heads)
    p = oracle_params(w, d_model, n_heads)
    x = O.bf16_round(rng.standard_normal((B, T, d_model)))
    pos = O.bf16_round(O.RelPositionalEncoding(d_model, 5000, False).get_encoding(T))
    layer = gpu_layer(w, d_model, n_heads, True, O.BF16)
    xd, pd = dev(x, O.BF16), dev(pos, O.BF16)
    got, qd, Pd = layer.debug_position_scores(xd, pd, with_inputs=True)
    got = host(got)
    h, dk = n_heads, d_model // n_heads
    q = host(qd).reshape(B, T, h, dk).transpose(0, 2, 1, 3)
    P = host(Pd).reshape(2 * T - 1, h, dk).transpose(1, 0, 2)
    v = O.bf16_round(p.pos_bias_v).reshape(1, h, 1, dk)
    qv = O.bf16_round(q + v)
    Pt = np.swapaxes(P, -1, -2)[None]
    exact = O.rel_shift(np.matmul(qv, Pt))[..., :T]
    # fp32 accumulation error of a d_k = 128 term dot product: at most
    # 128 * 2^-24 = 2^-17 of sum |q_v||p|
    acc = O.rel_shift(np.matmul(np.abs(qv), np.abs(Pt)))[..., :T] * 2.0 ** -17
    sbd = float(np.asarray(O.bf16_round(np.float32(O.f32_scale(dk)))).reshape(-1)[0])
    ref = O.bf16_round(O.bf16_round(exact) * sbd)
    assert np.array_equal(O.bf16_round(got), got), "the position term is not stored in bf16"
    lo = O.bf16_round(O.bf16_round(exact - acc) * sbd)
    hi = O.bf16_round(O.bf16_round(exact + acc) * sbd)
    d = np.abs(got - ref)
    bad = (got < lo) | (got > hi)
    print(f"T={T}: {int(np.sum(d > 0))} of {d.size} terms at another bf16 value than the exact term's, "
          f"{int(np.sum(lo != hi))} with more than one value in reach")
    assert not bad.any(), (f"{int(bad.sum())} of {bad.size} terms differ; worst {float(np.max(d[bad])):.3g} "
                           f"at {np.argwhere(bad)[:3].tolist()}")


@pytest.mark.parametrize("d_model,rows", [(128, 40000), (256, 40000)])
def test_dense_projection_unit_rows_return_the_weights(d_model, rows):
    """Unit rows (row r = e_{r mod K}) through the dense bf16 projections
    return the bf16 weights exactly: each output is one product 1 * w. At
    d_model 128 and 40000 rows the GEMM takes 192-row tiles with two k-stages
    (three LDS stages), whose prologue waits for stage 0 only with stage 1's
    loads in flight; at 256 it takes 192x256 tiles with four."""
    rng = np.random.default_rng(d_model + rows)
    w = W.make_layer_weights(rng, d_model, 2, False, False)
    layer = gpu_layer(w, d_model, 2, False, O.BF16)
    x = torch.zeros((rows, d_model), dtype=torch.bfloat16, device="cuda")
    idx = torch.arange(rows, device="cuda")
    x[idx, idx % d_model] = 1
    for name in ("linear_q", "linear_k", "linear_v", "linear_out", "linear_pos"):
        wb = torch.from_numpy(np.ascontiguousarray(w[f"{name}.weight"], dtype=np.float32)).bfloat16().float().numpy()
        ref = wb.T[np.arange(rows) % d_model]
        got = layer.debug_linear(name, x).float().cpu().numpy().reshape(ref.shape)
        bad = got != ref
        assert not bad.any(), f"{name}: {int(bad.sum())} of {bad.size} outputs differ, first at {np.argwhere(bad)[0]}"


@pytest.mark.parametrize("quantized", [False, True])
def test_paired_projections_equal_separate_launches(quantized):
    """At the xl_offline_bf16 shape (D=1024, B=8, T=375) the forward runs the
    fused Q/K/V projection (3000 x 3072, 192x192 tiles) and the position
    projection (749 rows, 64x64 tiles) in one launch, the position tiles
    after the Q/K/V tiles. The q rows and position rows it leaves equal those
    of the q and position linears run alone (`mhsa_debug_linear`, separate
    launches and, for q, another tile form), bit for bit: every tile form
    sums a dot product in the same 32x32x16 MFMA steps along K. For dense and
    affine-u8 weights."""
    cfg = W.CONFIGS["xl_offline_bf16"]
    D, H, T, B = cfg.d_model, cfg.n_heads, cfg.seq_len, cfg.batch
    rng = np.random.default_rng(61)
    w = W.make_layer_weights(rng, D, H, not quantized, quantized)
    layer = gpu_layer(w, D, H, not quantized, O.BF16)
    xd = dev(rng.standard_normal((B, T, D)), O.BF16)
    pd = dev(O.RelPositionalEncoding(D, 5000, True).get_encoding(T), O.BF16)
    _, qd, Pd = layer.debug_position_scores(xd, pd, with_inputs=True)
    q_alone = layer.debug_linear("linear_q", xd)
    P_alone = layer.debug_linear("linear_pos", pd)
    torch.cuda.synchronize()
    assert torch.isfinite(qd.float()).all() and torch.isfinite(Pd.float()).all()
    assert torch.equal(Pd.reshape(P_alone.shape), P_alone), \
        f"position rows differ by up to {float((Pd.float() - P_alone.float()).abs().max()):.3g}"
    assert torch.equal(qd, q_alone), f"q rows differ by up to {float((qd.float() - q_alone.float()).abs().max()):.3g}"


# ---------------------------------------------------------------------------
# offline forward
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("d_model,n_heads", [(128, 2), (256, 2)])
@pytest.mark.parametrize("ctx", [None, ((4, 1), "chunked_limited"), ((3, 2), "regular"), ((-1, 2), "chunked_limited"),
                                 ((2, -1), "regular"), ((30, 30), "regular")])
def test_forward_f32_contexts_and_padding(d_model, n_heads, ctx):
    rng = np.random.default_rng(5)
    w = random_weights(rng, d_model, n_heads, scale=0.08)
    p = oracle_params(w, d_model, n_heads)
    B, T, lengths = 3, 45, [45, 30, 1]
    x = rng.standard_normal((B, T, d_model)).astype(np.float32)
    pos = O.RelPositionalEncoding(d_model, 5000, False).get_encoding(T)
    octx = O.AttentionContext.new(*ctx) if ctx else None
    ref = O.mhsa_forward(p, x, pos, octx, O.key_padding_mask(lengths, T))
    layer = gpu_layer(w, d_model, n_heads, True, O.F32)
    got = host(layer.forward(dev(x, O.F32), dev(pos, O.F32), M.AttentionContext.new(*ctx) if ctx else None,
                             M.key_padding_mask(lengths, T)))
    rows = visible_rows(B, T, octx, lengths)
    assert row_rel_err(got, ref, rows) < F32_TOL


def test_forward_f32_many_query_blocks():
    """fp32 at a size with enough query blocks for the whole-workgroup form of
    the generic kernel (4 x 8 heads x 5 blocks of 64 queries = 160 workgroups;
    short inputs take the key-split form): key padding and a chunked context,
    against the float64 oracle."""
    rng = np.random.default_rng(12)
    d_model, n_heads, B, T = 512, 8, 4, 300
    w = random_weights(rng, d_model, n_heads, scale=0.05)
    p = oracle_params(w, d_model, n_heads)
    lengths = [300, 257, 130, 64]
    x = rng.standard_normal((B, T, d_model)).astype(np.float32)
    pos = O.RelPositionalEncoding(d_model, 5000, False).get_encoding(T)
    layer = gpu_layer(w, d_model, n_heads, True, O.F32)
    for ctx in (None, ((64, 15), "chunked_limited")):
        octx = O.AttentionContext.new(*ctx) if ctx else None
        ref = O.mhsa_forward(p, x, pos, octx, O.key_padding_mask(lengths, T))
        got = host(layer.forward(dev(x, O.F32), dev(pos, O.F32), M.AttentionContext.new(*ctx) if ctx else None,
                                 M.key_padding_mask(lengths, T)))
        assert row_rel_err(got, ref, visible_rows(B, T, octx, lengths)) < F32_TOL, ctx


def test_forward_large_f32():
    """FastConformer-large layer, fp32, B=1, T=125 (10 s of audio)."""
    cfg = W.CONFIGS["large_f32"]
    layers, x, _ = W.instantiate(cfg)
    p = oracle_params(layers[0], cfg.d_model, cfg.n_heads)
    pos = O.RelPositionalEncoding(cfg.d_model, 5000, True).get_encoding(cfg.seq_len)
    ref = O.mhsa_forward(p, x, pos)
    layer = gpu_layer(layers[0], cfg.d_model, cfg.n_heads, cfg.use_bias, O.F32)
    got = host(layer.forward(dev(x, O.F32), dev(pos, O.F32)))
    err = row_rel_err(got, ref)
    print(f"large_f32 max relative error {err:.3e}")
    assert err < F32_TOL


def test_forward_xl_offline_bf16():
    """0.6B-shape layer, bf16, B=8, T=375 with key padding."""
    cfg = W.CONFIGS["xl_offline_bf16"]
    layers, x, ex = W.instantiate(cfg)
    lengths = ex["lengths"]
    p = oracle_params(layers[0], cfg.d_model, cfg.n_heads)
    pos = O.RelPositionalEncoding(cfg.d_model, 5000, True).get_encoding(cfg.seq_len)
    xb, pb = O.bf16_round(x), O.bf16_round(pos)
    ref = O.mhsa_forward(p, xb, pb, None, O.key_padding_mask(lengths, cfg.seq_len), dtype=O.BF16)
    layer = gpu_layer(layers[0], cfg.d_model, cfg.n_heads, cfg.use_bias, O.BF16)
    got = host(layer.forward(dev(x, O.BF16), dev(pos, O.BF16), None, M.key_padding_mask(lengths, cfg.seq_len)))
    err = abs_err(got, ref)
    n_far = int(np.sum(np.abs(got - ref) > BF16_TOL))
    print(f"xl_offline_bf16 max abs error {err:.3e} (max |ref| {np.max(np.abs(ref)):.2f}), "
          f"{n_far} of {ref.size} outputs beyond {BF16_TOL}")
    assert err < BF16_TOL


def _biased_weights(seed, d_model, n_heads, sigma):
    rng = np.random.default_rng(seed)
    w = W.make_layer_weights(rng, d_model, n_heads, True, False)
    for name in ("linear_q", "linear_k", "linear_v", "linear_out"):
        w[f"{name}.bias"] = rng.normal(0.0, sigma, size=d_model).astype(np.float32)
    return w, rng


@pytest.mark.parametrize("rows", [3000, 1537, 6000])
def test_linear_bf16_bias_large(rows):
    """y = T(T(x W^T) + b) (quantization.rs:126-162) on row counts that take
    the tiled bf16 GEMM (6000 rows: 192 x 128 tiles), including a ragged last
    tile. The fp32 sum may round
    T(x W^T) one ulp away from the float64 product before the bias add, so each
    output is within one ulp of the pre-bias value, one ulp of the result and
    one fp32 rounding unit of sum |x||w| of the oracle."""
    D, H = 1024, 8
    w, rng = _biased_weights(21, D, H, 0.5)
    p = oracle_params(w, D, H)
    layer = gpu_layer(w, D, H, True, O.BF16)
    x = O.bf16_round(rng.normal(size=(rows, D)))
    for name in ("linear_q", "linear_out"):
        got = host(layer.debug_linear(name, dev(x, O.BF16)))
        lin = getattr(p, name)
        ref = lin.forward(x, O.BF16)
        wd = lin.dense_weight(O.BF16)
        pre = x @ wd.T

        def ulp(a):
            return np.ldexp(1.0, np.frexp(np.abs(a))[1] - 8)

        bound = ulp(pre) + ulp(ref) + np.abs(x) @ np.abs(wd).T * 2.0 ** -24
        d = np.abs(got - ref)
        print(f"{name} rows={rows}: worst |d|/bound {np.max(d / bound):.3f}")
        assert np.all(d <= bound), name


@pytest.mark.parametrize("rows,quant", [(700, False), (700, True), (125, False), (33, True)])
def test_linear_f32_persistent_tiles(rows, quant):
    """fp32 y = x W^T + b on row counts that take the K-parallel kernel with
    persistent workgroups: 700 rows are 22 x 32 tiles of 32 x 32, three per
    workgroup, so ranges cross from one row tile into the next (the A rows
    are reloaded mid-range) and the last row tile is ragged; 125 and 33 rows
    give one tile per workgroup. Dense and u8 weights, with biases, within
    1e-5 of the float64 oracle."""
    D, H = 1024, 8
    rng = np.random.default_rng(61)
    w = W.make_layer_weights(rng, D, H, True, quant, centred=True)
    for name in ("linear_q", "linear_out"):
        if quant:
            s = rng.uniform(1e-4, 1e-3, size=w[f"{name}.scales"].shape)
            w[f"{name}.scales"] = s.astype(np.float16)
            b = -128.0 * w[f"{name}.scales"].astype(np.float64) + rng.normal(0, 1e-3, size=s.shape)
            w[f"{name}.biases"] = b.astype(np.float16)
        w[f"{name}.bias"] = rng.normal(0, 0.1, D).astype(w[f"{name}.bias"].dtype)
    p = oracle_params(w, D, H)
    layer = gpu_layer(w, D, H, True, O.F32)
    x = rng.standard_normal((rows, D)).astype(np.float32)
    for name in ("linear_q", "linear_out"):
        got = host(layer.debug_linear(name, dev(x, O.F32)))
        ref = getattr(p, name).forward(x.astype(np.float64), O.F32)
        assert row_rel_err(got, ref) < 1e-5, name


def test_forward_bf16_with_biases():
    """The offline bf16 layer with non-zero linear biases (the V bias enters
    through the transposed V epilogue), B=2, T=375, key padding; biases of
    scale 0.1 keep the outputs at the magnitude the bf16 bound is stated for."""
    D, H, T = 1024, 8, 375
    w, rng = _biased_weights(22, D, H, 0.1)
    x = rng.normal(size=(2, T, D))
    lengths = [T, 301]
    p = oracle_params(w, D, H)
    pos = O.RelPositionalEncoding(D, 5000, True).get_encoding(T)
    ref = O.mhsa_forward(p, O.bf16_round(x), O.bf16_round(pos), None, O.key_padding_mask(lengths, T), dtype=O.BF16)
    layer = gpu_layer(w, D, H, True, O.BF16)
    got = host(layer.forward(dev(x, O.BF16), dev(pos, O.BF16), None, M.key_padding_mask(lengths, T)))
    err = abs_err(got, ref)
    print(f"bf16 with biases: max abs error {err:.3e} (max |ref| {np.max(np.abs(ref)):.2f})")
    assert err < BF16_TOL


def test_forward_bf16_more_blocks_than_cus():
    """The offline bf16 layer on a shape with more query blocks than CUs
    (8 items of 1000-1100 valid frames, T = 1100, 4 heads: about 270 blocks
    of 128 queries, so workgroups run in two rounds), 9 key tiles per block
    and key padding, against the oracle within the bf16 tolerance."""
    D, H, T, B = 512, 4, 1100, 8
    w, rng = _biased_weights(81, D, H, 0.1)
    x = rng.normal(size=(B, T, D))
    lengths = [int(v) for v in rng.integers(1000, T + 1, size=B)]
    lengths[0] = T
    p = oracle_params(w, D, H)
    pos = O.RelPositionalEncoding(D, 5000, True).get_encoding(T)
    ref = O.mhsa_forward(p, O.bf16_round(x), O.bf16_round(pos), None, O.key_padding_mask(lengths, T), dtype=O.BF16)
    layer = gpu_layer(w, D, H, True, O.BF16)
    got = host(layer.forward(dev(x, O.BF16), dev(pos, O.BF16), None, M.key_padding_mask(lengths, T)))
    err = abs_err(got, ref)
    print(f"bf16 two rounds: max abs error {err:.3e} (max |ref| {np.max(np.abs(ref)):.2f})")
    assert err < BF16_TOL


def test_forward_bf16_4000_rows():
    """The 0.6B-shape offline bf16 layer at B=4, T=1000 (4000 rows): its
    Q/K/V projection runs as 192 x 128 tiles whose blocks hold both K and V^T
    columns, and its 8 query blocks per item over 16 key tiles; key padding,
    against the oracle within the bf16 tolerance."""
    D, H, T, B = 1024, 8, 1000, 4
    w, rng = _biased_weights(83, D, H, 0.1)
    x = rng.normal(size=(B, T, D))
    lengths = [int(v) for v in rng.integers(700, T + 1, size=B)]
    lengths[1] = T
    p = oracle_params(w, D, H)
    pos = O.RelPositionalEncoding(D, 5000, True).get_encoding(T)
    ref = O.mhsa_forward(p, O.bf16_round(x), O.bf16_round(pos), None, O.key_padding_mask(lengths, T), dtype=O.BF16)
    layer = gpu_layer(w, D, H, True, O.BF16)
    got = host(layer.forward(dev(x, O.BF16), dev(pos, O.BF16), None, M.key_padding_mask(lengths, T)))
    err = abs_err(got, ref)
    print(f"bf16 4000 rows: max abs error {err:.3e} (max |ref| {np.max(np.abs(ref)):.2f})")
    assert err < BF16_TOL


@pytest.mark.parametrize("padded", [False, True], ids=["eight_wave", "mixed_forms"])
def test_forward_bf16_eight_wave_blocks(padded):
    """The 0.6B-shape offline bf16 layer at B=5, T=1100: 5 blocks of 256
    queries per (item, head), 200 workgroups, so the attention takes the
    8-wave form with 32-key tiles; the last block is ragged (76 queries).
    Unpadded, every item takes that form. With key padding (lengths 921,
    1015, 1100, 989, 1028, ending inside key tiles) the longest item takes
    the 4-wave form in the same launch: 72 workgroups of 128 queries with 18
    tiles of 64 keys, beside 160 8-wave workgroups whose longest has 33 tiles
    of 32 keys (35 for the moved item). Against the oracle within the bf16
    tolerance."""
    D, H, T, B = 1024, 8, 1100, 5
    w, rng = _biased_weights(85, D, H, 0.1)
    x = rng.normal(size=(B, T, D))
    lengths = [int(v) for v in rng.integers(600, T + 1, size=B)]
    lengths[2] = T
    mask = O.key_padding_mask(lengths, T) if padded else None
    p = oracle_params(w, D, H)
    pos = O.RelPositionalEncoding(D, 5000, True).get_encoding(T)
    ref = O.mhsa_forward(p, O.bf16_round(x), O.bf16_round(pos), None, mask, dtype=O.BF16)
    layer = gpu_layer(w, D, H, True, O.BF16)
    before = M.debug_attention_forms()
    got = host(layer.forward(dev(x, O.BF16), dev(pos, O.BF16), None,
                             M.key_padding_mask(lengths, T) if padded else None))
    after = M.debug_attention_forms()
    ran = {k for k in after if after[k] > before[k]}
    assert ran == ({"bf16_mixed"} if padded else {"bf16_wave8"}), ran
    err = abs_err(got, ref)
    print(f"bf16 eight-wave blocks (padded {padded}): max abs error {err:.3e} (max |ref| {np.max(np.abs(ref)):.2f})")
    assert err < BF16_TOL


def test_bf16_scores_growing_far_past_first_tile():
    """Scores that grow along the keys by thousands (x_t = g(t) z + noise with
    g rising to 31, so q_i . k_j scales with g(i) g(j)) exceed the first key
    tile's maximum by far more than 2^100 in exp2 units; the kernel then moves
    its softmax reference and rescales its sums mid-row. The output matches the
    oracle's exact softmax to bf16 precision of the output scale."""
    D, H, T = 1024, 8, 375
    rng = np.random.default_rng(23)
    w = W.make_layer_weights(rng, D, H, False, False)
    z = rng.normal(size=D)
    g = 1.0 + 30.0 * np.arange(T) / T
    x = (g[:, None] * z[None, :] + 0.1 * rng.normal(size=(T, D)))[None]
    p = oracle_params(w, D, H)
    pos = O.RelPositionalEncoding(D, 5000, True).get_encoding(T)
    ref = O.mhsa_forward(p, O.bf16_round(x), O.bf16_round(pos), None, None, dtype=O.BF16)
    layer = gpu_layer(w, D, H, False, O.BF16)
    got = host(layer.forward(dev(x, O.BF16), dev(pos, O.BF16), None))
    rel = abs_err(got, ref) / np.max(np.abs(ref))
    print(f"growing scores: max abs error / max|ref| {rel:.3e} (max |ref| {np.max(np.abs(ref)):.1f})")
    assert rel < 1e-2


def test_padded_keys_are_ignored_gpu():
    """attention.rs:1025-1064 on the GPU: a padded row attends like the row unpadded."""
    cfg = W.CONFIGS["xl_offline_bf16"]
    layers, x, _ = W.instantiate(cfg)
    T, valid = cfg.seq_len, 200
    x = x[:2].copy()
    x[1, valid:] = 50.0
    pe = M.RelPositionalEncoding(cfg.d_model, 5000, True)
    layer = gpu_layer(layers[0], cfg.d_model, cfg.n_heads, False, O.F32)
    for ctx in (None, M.AttentionContext.new((3, 2), "regular")):
        masked = host(layer.forward(dev(x, O.F32), dev(pe.get_encoding(T), O.F32), ctx, M.key_padding_mask([T, valid], T)))
        full = host(layer.forward(dev(x[:1], O.F32), dev(pe.get_encoding(T), O.F32), ctx))
        short = host(layer.forward(dev(x[1:2, :valid], O.F32), dev(pe.get_encoding(valid), O.F32), ctx))
        # the reference's own bounds (attention.rs:1060-1061); the GEMM's K
        # split depends on the row count, so batch 1 and 2 sum in other orders
        assert row_rel_err(masked[:1], full) < 1e-5
        assert row_rel_err(masked[1:2, :valid], short) < 1e-5


def test_local_window_bf16_against_oracle():
    """+-128 regular window with the 257-row banded table, checked against the
    reference algorithm on the full 2T-1 table at a size the oracle finishes quickly."""
    cfg = W.CONFIGS["xl_local_bf16"]
    layers, _, _ = W.instantiate(cfg)
    T = 700
    x = np.random.default_rng(30).standard_normal((1, T, cfg.d_model)).astype(np.float32)
    p = oracle_params(layers[0], cfg.d_model, cfg.n_heads)
    pe = O.RelPositionalEncoding(cfg.d_model, 5000, True)
    full, band = pe.get_encoding(T), pe.get_encoding(129)
    ref = O.mhsa_forward(p, O.bf16_round(x), O.bf16_round(full), O.AttentionContext.new((128, 128), "regular"),
                         None, dtype=O.BF16)
    layer = gpu_layer(layers[0], cfg.d_model, cfg.n_heads, False, O.BF16)
    got = host(layer.forward(dev(x, O.BF16), dev(band, O.BF16), M.AttentionContext.new((128, 128), "regular")))
    err = abs_err(got, ref)
    print(f"local window T={T} max abs error {err:.3e}")
    assert err < BF16_TOL


@pytest.mark.parametrize("ctx", [((128, 128), "regular"), ((40, 7), "regular"), ((-1, 16), "regular"),
                                 ((64, -1), "regular"), ((70, 13), "chunked_limited"), ((-1, 31), "chunked_limited")])
def test_forward_bf16_contexts_against_oracle(ctx):
    """The bf16 kernel under each kind of context (attention.rs:208-273): two-
    and one-sided regular windows and chunked_limited chunks, with key
    padding (lengths 600, 451, 257 of T = 600), on the full 2T-1 table, against
    the oracle within the bf16 tolerance on the rows that see a key. Windows
    leave a block's first or last key tiles outside some waves' queries, which
    those waves pass over."""
    D, H, T, lengths = 256, 2, 600, [600, 451, 257]
    rng = np.random.default_rng(73)
    w = random_weights(rng, D, H)
    p = oracle_params(w, D, H)
    x = O.bf16_round(rng.standard_normal((len(lengths), T, D)))
    pos = O.bf16_round(O.RelPositionalEncoding(D, 5000, True).get_encoding(T))
    octx = O.AttentionContext.new(*ctx)
    ref = O.mhsa_forward(p, x, pos, octx, O.key_padding_mask(lengths, T), dtype=O.BF16)
    layer = gpu_layer(w, D, H, True, O.BF16)
    got = host(layer.forward(dev(x, O.BF16), dev(pos, O.BF16), M.AttentionContext.new(*ctx),
                             M.key_padding_mask(lengths, T)))
    rows = visible_rows(len(lengths), T, octx, lengths)
    err = abs_err(got[rows], ref[rows])
    print(f"bf16 context {ctx}: max abs error {err:.3e}")
    assert err < BF16_TOL


@pytest.mark.parametrize("ctx", [((70, 13), "chunked_limited"), ((64, -1), "regular")])
def test_forward_bf16_contexts_eight_wave(ctx):
    """The same at the 0.6B shape with B=4, T=1100 (lengths 1100, 987, 800,
    1033): 5 blocks of 256 queries per item and head, 160 workgroups, so the
    8-wave form runs, whose waves pass over the key tiles outside their
    queries' windows or chunks."""
    D, H, T, lengths = 1024, 8, 1100, [1100, 987, 800, 1033]
    rng = np.random.default_rng(74)
    w = random_weights(rng, D, H)
    p = oracle_params(w, D, H)
    x = O.bf16_round(rng.standard_normal((len(lengths), T, D)))
    pos = O.bf16_round(O.RelPositionalEncoding(D, 5000, True).get_encoding(T))
    octx = O.AttentionContext.new(*ctx)
    ref = O.mhsa_forward(p, x, pos, octx, O.key_padding_mask(lengths, T), dtype=O.BF16)
    layer = gpu_layer(w, D, H, True, O.BF16)
    got = host(layer.forward(dev(x, O.BF16), dev(pos, O.BF16), M.AttentionContext.new(*ctx),
                             M.key_padding_mask(lengths, T)))
    rows = visible_rows(len(lengths), T, octx, lengths)
    err = abs_err(got[rows], ref[rows])
    print(f"bf16 context {ctx}, 8-wave form: max abs error {err:.3e}")
    assert err < BF16_TOL


def test_local_window_full_size_band_equals_full_table():
    """At B=2, T=7500 the banded table and the full 2T-1 table must give
    bit-identical outputs (the band holds every row the window reads)."""
    cfg = W.CONFIGS["xl_local_bf16"]
    layers, x, _ = W.instantiate(cfg)
    pe = M.RelPositionalEncoding(cfg.d_model, 5000, True)
    layer = gpu_layer(layers[0], cfg.d_model, cfg.n_heads, False, O.BF16)
    ctx = M.AttentionContext.new((128, 128), "regular")
    xd = dev(x, O.BF16)
    a = layer.forward(xd, dev(pe.get_encoding(129), O.BF16), ctx)
    b = layer.forward(xd, dev(pe.get_encoding(cfg.seq_len), O.BF16), ctx)
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b)
    with pytest.raises(M.MhsaError):  # a band narrower than the window is rejected
        layer.forward(xd, dev(pe.get_encoding(100), O.BF16), ctx)


# ---------------------------------------------------------------------------
# streaming
# ---------------------------------------------------------------------------

def test_streaming_xl_50_steps():
    """16 sessions, 14-frame chunks, 70-frame cache, [70,13] chunked_limited,
    per-session fills, 50 steps carrying the cache. The oracle runs each
    session as its own B=1 reference step (the reference's mask uses one fill
    for the whole batch, conformer.rs:883-887)."""
    cfg = W.CONFIGS["xl_stream_f32"]
    layers, _, ex = W.instantiate(cfg)
    B, C, T, D = cfg.batch, cfg.cache_size, cfg.seq_len, cfg.d_model
    p = oracle_params(layers[0], D, cfg.n_heads)
    pos = O.RelPositionalEncoding(D, 5000, True).get_encoding(C + T)
    layer = gpu_layer(layers[0], D, cfg.n_heads, False, O.F32)
    st = layer.stream(B, C, T)
    st.load_cache(dev(ex["cache"], O.F32), ex["fills"])
    pos_d = dev(pos, O.F32)
    caches = [ex["cache"][b:b + 1].astype(np.float64) for b in range(B)]
    fills = list(ex["fills"])
    check_steps = {0, 1, 2, 4, 5, 10, 25, 49}
    worst = 0.0
    for step in range(cfg.steps):
        x = ex["chunks"][step]
        got = st.step(dev(x, O.F32), pos_d, M.StreamingMask((70, 13), "chunked_limited"))
        assert st.fill() == [min(f + T, C) for f in fills]
        if step in check_steps:
            g = host(got)
            for b in range(B):
                mask = O.streaming_mask((70, 13), "chunked_limited", C, fills[b], T, T)
                ref, _ = O.mhsa_forward_with_cache(p, x[b:b + 1], pos, caches[b], mask)
                e = row_rel_err(g[b:b + 1], ref)
                worst = max(worst, e)
                assert e < F32_TOL, (step, b, fills[b], e)
        for b in range(B):
            caches[b] = O.cache_update(caches[b], x[b:b + 1].astype(np.float64), 0)
            fills[b] = O.next_fill(fills[b], T, 0, C)
    print(f"streaming worst relative error {worst:.3e}")
    cache_gpu = st.read_cache().cpu().numpy()
    assert np.array_equal(cache_gpu, np.concatenate(caches, 0).astype(np.float32))


def test_streaming_new_stream_with_biases_no_mask():
    """A stream that never saw load_cache starts from the reference's zero
    cache (EncoderCache::new): its unfilled rows are h = 0, so their keys and
    values are the projection biases (attention.rs:650, 721-722), visible
    when no mask is given. Three steps with q/k/v/out biases against the
    oracle carrying a zero-initialised cache."""
    rng = np.random.default_rng(14)
    w = random_weights(rng, 256, 2, use_bias=True, scale=0.05)
    p = oracle_params(w, 256, 2)
    B, C, T = 2, 20, 6
    pos = O.RelPositionalEncoding(256, 5000, False).get_encoding(C + T)
    layer = gpu_layer(w, 256, 2, True, O.F32)
    st = layer.stream(B, C, T)
    cache = np.zeros((B, C, 256))
    for step in range(3):
        x = rng.standard_normal((B, T, 256)).astype(np.float32)
        got = host(st.step(dev(x, O.F32), dev(pos, O.F32)))
        ref, cache = O.mhsa_forward_with_cache(p, x, pos, cache, None)
        assert row_rel_err(got, ref) < F32_TOL, step
    assert np.array_equal(st.read_cache().cpu().numpy(), cache.astype(np.float32))


def test_streaming_weights_changed_mid_stream():
    """The reference re-projects the cached h with the current weights on
    every step; reloading weights between steps must do the same."""
    rng = np.random.default_rng(15)
    w1 = random_weights(rng, 256, 2, use_bias=True, scale=0.05)
    w2 = random_weights(rng, 256, 2, use_bias=True, scale=0.05)
    B, C, T = 2, 20, 6
    pos = O.RelPositionalEncoding(256, 5000, False).get_encoding(C + T)
    layer = gpu_layer(w1, 256, 2, True, O.F32)
    st = layer.stream(B, C, T)
    cache = rng.standard_normal((B, C, 256))
    st.load_cache(dev(cache, O.F32), [C, C])
    x = rng.standard_normal((B, T, 256)).astype(np.float32)
    st.step(dev(x, O.F32), dev(pos, O.F32))
    _, cache = O.mhsa_forward_with_cache(oracle_params(w1, 256, 2), x, pos, cache.astype(np.float32), None)
    layer.load_weights(W.prefixed(w2, "layer"), "layer")
    x = rng.standard_normal((B, T, 256)).astype(np.float32)
    got = host(st.step(dev(x, O.F32), dev(pos, O.F32)))
    ref, _ = O.mhsa_forward_with_cache(oracle_params(w2, 256, 2), x, pos, cache, None)
    assert row_rel_err(got, ref) < F32_TOL


@pytest.mark.parametrize("B,C,T,ctx", [(3, 140, 27, ((140, 26), "chunked_limited")),
                                       (32, 140, 27, ((100, 8), "regular")),
                                       (2, 100, 14, ((70, 13), "chunked_limited"))])
def test_streaming_long_context_ring_wraps(B, C, T, ctx):
    """Streaming shapes past the chunk kernel's limits (T > 16 or more than 96
    keys), so the generic fp32 kernel reads the ring: key-split form (few
    workgroups), four-wave form (B = 32) and one-wave form (T = 14, 114 keys).
    Nine steps wrap the ring head past its end; every step is checked
    against the oracle and the cache read back bit-equal."""
    rng = np.random.default_rng(16)
    d, h = 512, 4
    w = random_weights(rng, d, h, use_bias=True, scale=0.04)
    p = oracle_params(w, d, h)
    pos = O.RelPositionalEncoding(d, 5000, False).get_encoding(C + T)
    layer = gpu_layer(w, d, h, True, O.F32)
    st = layer.stream(B, C, T)
    cache = rng.standard_normal((B, C, d)).astype(np.float32)
    fills = [int(v) for v in rng.integers(0, C + 1, size=B)]
    for b in range(B):
        cache[b, :C - fills[b]] = 0.0
    st.load_cache(dev(cache, O.F32), fills)
    caches = [cache[b:b + 1].astype(np.float64) for b in range(B)]
    pos_d = dev(pos, O.F32)
    (left, right), style = ctx
    for step in range(9):
        x = rng.standard_normal((B, T, d)).astype(np.float32)
        got = host(st.step(dev(x, O.F32), pos_d, M.StreamingMask((left, right), style)))
        for b in range(B):
            mask = O.streaming_mask((left, right), style, C, fills[b], T, T)
            ref, caches[b] = O.mhsa_forward_with_cache(p, x[b:b + 1], pos, caches[b], mask)
            assert row_rel_err(got[b:b + 1], ref) < F32_TOL, (step, b)
            fills[b] = O.next_fill(fills[b], T, 0, C)
        assert st.fill() == fills
    assert np.array_equal(st.read_cache().cpu().numpy(), np.concatenate(caches, 0).astype(np.float32))


@pytest.mark.parametrize("keys", [97, 98, 112, 114, 129])
@pytest.mark.parametrize("d,h", [(512, 4), (512, 8)], ids=["dk128", "dk64"])
def test_streaming_key_split_partial_tiles(keys, d, h):
    """14-frame chunks against caches of keys - 14 rows, key counts that end
    inside a key tile (past the chunk kernel's 96 keys, so the generic fp32
    kernel's key-split form runs, with its per-key mask on the last tile and on
    the unfilled-cache offset). Per-session fills, with and without a chunked
    context; one step against the oracle."""
    rng = np.random.default_rng(keys + h)
    T = 14
    C = keys - T
    B = 3
    w = random_weights(rng, d, h, use_bias=True, scale=0.04)
    p = oracle_params(w, d, h)
    pos = O.RelPositionalEncoding(d, 5000, False).get_encoding(C + T)
    layer = gpu_layer(w, d, h, True, O.F32)
    for ctx in (None, ((C, T - 1), "chunked_limited")):
        st = layer.stream(B, C, T)
        cache = rng.standard_normal((B, C, d)).astype(np.float32)
        fills = [C, C // 2, 3]
        for b in range(B):
            cache[b, :C - fills[b]] = 0.0
        st.load_cache(dev(cache, O.F32), fills)
        x = rng.standard_normal((B, T, d)).astype(np.float32)
        before = M.debug_attention_forms()
        mask = M.StreamingMask(*ctx, fills, [T] * B) if ctx else None
        got = host(st.step(dev(x, O.F32), dev(pos, O.F32), mask))
        after = M.debug_attention_forms()
        assert {k for k in after if after[k] > before[k]} == {"generic_key_split"}
        for b in range(B):
            m = O.streaming_mask(ctx[0], ctx[1], C, fills[b], T, T) if ctx else None
            ref, _ = O.mhsa_forward_with_cache(p, x[b:b + 1], pos, cache[b:b + 1].astype(np.float64), m)
            assert row_rel_err(got[b:b + 1], ref) < F32_TOL, (ctx, b)


def test_streaming_bf16_layer_xl_shape():
    """A bf16 layer streamed as the encoder streams it: f32 cache and chunk,
    so the arithmetic is f32 on the bf16-cast parameters, with bf16 position
    rows (conformer.rs:422-434, 845-849). 16 sessions, 14-frame chunks
    against the 70-frame cache, [70,13] chunked_limited, per-session fills,
    12 steps against the oracle's bf16 streaming (fp32 bound) and the cache
    read back bit-equal.

    The position rows are a bf16 matmul: the GPU rounds its fp32 sum, the
    oracle the exact one, so an element whose exact value lies within fp32
    accumulation noise of a bf16 rounding boundary may land on the other
    neighbour. They are checked for exactly that, and the oracle then runs on
    the GPU's rows, which keeps the comparison at the fp32 bound."""
    cfg = W.CONFIGS["xl_stream_f32"]
    layers, _, ex = W.instantiate(cfg)
    B, C, T, D = cfg.batch, cfg.cache_size, cfg.seq_len, cfg.d_model
    w = dict(layers[0])
    rng = np.random.default_rng(17)
    for name in ("linear_q", "linear_k", "linear_v", "linear_out"):
        w[f"{name}.bias"] = rng.normal(0, 0.1, D).astype(np.float32)
    p = oracle_params(w, D, cfg.n_heads)
    pos = O.bf16_round(O.RelPositionalEncoding(D, 5000, True).get_encoding(C + T))
    layer = gpu_layer(w, D, cfg.n_heads, True, O.BF16)
    st = layer.stream(B, C, T)
    st.load_cache(dev(ex["cache"], O.F32), ex["fills"])
    pos_d = dev(pos, O.BF16)
    P_gpu = host(layer.debug_linear("linear_pos", pos_d))[0]
    exact = pos[0] @ p.linear_pos.dense_weight(O.BF16).T
    acc = np.abs(pos[0]) @ np.abs(p.linear_pos.dense_weight(O.BF16)).T * 2.0 ** -20
    _, e = np.frexp(np.abs(exact))
    near = np.abs(np.abs(exact) - np.abs(O.bf16_round(exact))) >= np.ldexp(0.5, e - 8) - acc
    d = P_gpu != O.bf16_round(exact)
    assert not (d & ~near).any()
    _, eg = np.frexp(np.maximum(np.abs(P_gpu), np.abs(exact)))
    assert np.all(np.abs(P_gpu - exact) <= np.ldexp(1.0, eg - 8) + acc)  # one ulp + fp32 accumulation
    caches = [ex["cache"][b:b + 1].astype(np.float64) for b in range(B)]
    fills = list(ex["fills"])
    worst = 0.0
    for step in range(12):
        x = ex["chunks"][step]
        got = host(st.step(dev(x, O.F32), pos_d, M.StreamingMask((70, 13), "chunked_limited")))
        for b in range(B):
            mask = O.streaming_mask((70, 13), "chunked_limited", C, fills[b], T, T)
            ref, caches[b] = O.mhsa_forward_with_cache(p, x[b:b + 1], pos, caches[b], mask, dtype=O.BF16,
                                                       pos_rows=P_gpu)
            e = row_rel_err(got[b:b + 1], ref)
            worst = max(worst, e)
            assert e < F32_TOL, (step, b, e)
            fills[b] = O.next_fill(fills[b], T, 0, C)
    print(f"bf16 streaming worst per-row relative error {worst:.3e}")
    assert np.array_equal(st.read_cache().cpu().numpy(), np.concatenate(caches, 0).astype(np.float32))


@pytest.mark.parametrize("dtype", [O.F32, O.BF16])
@pytest.mark.parametrize("quant", [False, True])
def test_forward_without_cache(dtype, quant):
    """forward_with_cache with no cache (attention.rs:687-700): keys and
    values from the chunk alone, under a chunked_limited mask whose rows past
    the valid length are blank (the bool path: they give the output bias),
    in both layer dtypes and both projection kinds. The functional form also
    returns the reference's new cache x[:, :T - cache_drop_size]."""
    rng = np.random.default_rng(18)
    d, h, B, T = 256, 2, 3, 37
    if quant:
        w = W.make_layer_weights(rng, d, h, True, True, centred=True)
        for name in ("linear_q", "linear_k", "linear_v", "linear_out", "linear_pos"):
            sc = rng.uniform(1e-4, 1e-3, size=w[f"{name}.scales"].shape)
            w[f"{name}.scales"] = sc.astype(np.float16)
            w[f"{name}.biases"] = (-128.0 * w[f"{name}.scales"].astype(np.float64)).astype(np.float16)
            if name != "linear_pos":
                w[f"{name}.bias"] = rng.normal(0, 0.1, d).astype(np.float16)
    else:
        w = random_weights(rng, d, h, use_bias=True, scale=0.05)
    p = oracle_params(w, d, h, cache_drop_size=2)
    layer = gpu_layer(w, d, h, True, dtype)
    layer.cache_drop_size = 2
    x = rng.standard_normal((B, T, d)).astype(np.float32)
    pos = O.RelPositionalEncoding(d, 5000, False).get_encoding(T)
    pos = pos if dtype == O.F32 else O.bf16_round(pos)
    valid = 30
    out, nc = layer.forward_with_cache(dev(x, O.F32), dev(pos, dtype), None, 0,
                                       M.StreamingMask((12, 5), "chunked_limited", [0] * B, [valid] * B))
    mask = O.streaming_mask((12, 5), "chunked_limited", 0, 0, T, valid)
    assert mask.dtype == np.bool_
    ref, ref_nc = O.mhsa_forward_with_cache(p, x, pos, None, mask, dtype=dtype)
    got = host(out)
    assert row_rel_err(got, ref) < F32_TOL
    bias = O.to_dtype(np.asarray(w["linear_out.bias"], dtype=np.float64), dtype)
    assert np.allclose(got[:, valid:], bias[None, None, :], atol=1e-6)
    assert np.array_equal(host(nc), ref_nc)


def test_streaming_rows_past_valid_give_output_bias():
    rng = np.random.default_rng(8)
    w = random_weights(rng, 128, 2, use_bias=True, scale=0.08)
    p = oracle_params(w, 128, 2)
    C, T = 6, 5
    x = rng.standard_normal((2, T, 128)).astype(np.float32)
    cache = rng.standard_normal((2, C, 128)).astype(np.float32)
    pos = O.RelPositionalEncoding(128, 64, False).get_encoding(C + T)
    layer = gpu_layer(w, 128, 2, True, O.F32)
    st = layer.stream(2, C, T)
    st.load_cache(dev(cache, O.F32), [4, 4])
    got = host(st.step(dev(x, O.F32), dev(pos, O.F32), M.StreamingMask((4, 1), "regular", [4, 4], [3, 3])))
    for b in range(2):
        mask = O.streaming_mask((4, 1), "regular", C, 4, T, 3)
        assert mask.dtype == np.bool_
        ref, _ = O.mhsa_forward_with_cache(p, x[b:b + 1], pos, cache[b:b + 1].astype(np.float64), mask)
        assert row_rel_err(got[b:b + 1], ref) < F32_TOL
        assert np.allclose(got[b, 3:], w["linear_out.bias"][None, :], atol=1e-6)


def test_streaming_functional_form_and_cache_drop():
    """forward_with_cache(x, pos, cache) -> (out, new_cache) like the reference,
    with cache_drop_size > 0 (regular style)."""
    rng = np.random.default_rng(9)
    w = random_weights(rng, 128, 2, use_bias=True, scale=0.08)
    p = oracle_params(w, 128, 2, cache_drop_size=2)
    C, T = 7, 5
    x = rng.standard_normal((3, T, 128)).astype(np.float32)
    cache = rng.standard_normal((3, C, 128)).astype(np.float32)
    pos = O.RelPositionalEncoding(128, 64, False).get_encoding(C + T)
    layer = gpu_layer(w, 128, 2, True, O.F32)
    layer.cache_drop_size = 2
    out, nc = layer.forward_with_cache(dev(x, O.F32), dev(pos, O.F32), dev(cache, O.F32), C, None)
    ref, ref_nc = O.mhsa_forward_with_cache(p, x, pos, cache.astype(np.float64), None)
    assert row_rel_err(host(out), ref) < F32_TOL
    assert np.array_equal(nc.cpu().numpy(), ref_nc.astype(np.float32))


def test_streaming_equals_offline_last_rows():
    """A full cache of the previous frames and no mask: the chunk output equals
    the last T rows of offline attention over cache + chunk (GPU vs GPU)."""
    rng = np.random.default_rng(10)
    w = random_weights(rng, 256, 2, use_bias=False, scale=0.05)
    C, T = 70, 14
    seq = rng.standard_normal((2, C + T, 256)).astype(np.float32)
    pos = O.RelPositionalEncoding(256, 5000, False).get_encoding(C + T)
    layer = gpu_layer(w, 256, 2, False, O.F32)
    st = layer.stream(2, C, T)
    st.load_cache(dev(seq[:, :C], O.F32), [C, C])
    got = host(st.step(dev(seq[:, C:], O.F32), dev(pos, O.F32)))
    full = host(layer.forward(dev(seq, O.F32), dev(pos, O.F32)))
    assert row_rel_err(got, full[:, C:]) < 1e-5


@pytest.mark.parametrize("dtype", [O.F32, O.BF16])
@pytest.mark.parametrize("d_model,n_heads,kind", [(256, 4, "u8"), (256, 4, "mixed"), (1280, 10, "u8"),
                                                  (512, 8, "dense")])
def test_streaming_projection_kinds_with_biases(d_model, n_heads, kind, dtype):
    """Cache-aware steps with q/k/v/out biases and u8, dense or mixed q/k/v.
    Same-kind q/k/v with D <= 1024 take one launch for the chunk's Q, its K|V
    rows of the cache ring and its copy into the input ring; mixed kinds and
    D = 1280 take separate launches. Four steps against the oracle (fp32
    bound) and the exported cache bit-equal to the oracle's."""
    rng = np.random.default_rng(51)
    quant = kind != "dense"
    w = W.make_layer_weights(rng, d_model, n_heads, True, quant, centred=True)
    for name in ("linear_q", "linear_k", "linear_v", "linear_out", "linear_pos"):
        if quant:  # |W| ~ 0.04: scores stay O(1)
            s = rng.uniform(1e-4, 1e-3, size=w[f"{name}.scales"].shape)
            w[f"{name}.scales"] = s.astype(np.float16)
            b = -128.0 * w[f"{name}.scales"].astype(np.float64) + rng.normal(0, 1e-3, size=s.shape)
            w[f"{name}.biases"] = b.astype(np.float16)
        if name != "linear_pos":
            w[f"{name}.bias"] = rng.normal(0, 0.1, d_model).astype(w[f"{name}.bias"].dtype)
    if kind == "mixed":  # dense V beside u8 Q and K
        del w["linear_v.scales"], w["linear_v.biases"]
        w["linear_v.weight"] = W.xavier(rng, d_model, d_model)
        w["linear_v.bias"] = w["linear_v.bias"].astype(np.float32)
    p = oracle_params(w, d_model, n_heads)
    B, C, T = 3, 70, 14
    cache = rng.standard_normal((B, C, d_model)).astype(np.float32)
    pos = O.RelPositionalEncoding(d_model, 5000, False).get_encoding(C + T)
    pos = pos if dtype == O.F32 else O.bf16_round(pos)
    layer = gpu_layer(w, d_model, n_heads, True, dtype)
    st = layer.stream(B, C, T)
    fills = [70, 23, 0]
    st.load_cache(dev(cache, O.F32), fills)
    pos_d = dev(pos, dtype)
    caches = [cache[b:b + 1].astype(np.float64) for b in range(B)]
    for step in range(4):
        x = rng.standard_normal((B, T, d_model)).astype(np.float32)
        got = host(st.step(dev(x, O.F32), pos_d, M.StreamingMask((70, 13), "chunked_limited")))
        for b in range(B):
            mask = O.streaming_mask((70, 13), "chunked_limited", C, fills[b], T, T)
            ref, _ = O.mhsa_forward_with_cache(p, x[b:b + 1], pos, caches[b], mask, dtype=dtype)
            assert row_rel_err(got[b:b + 1], ref) < F32_TOL, (step, b)
            caches[b] = O.cache_update(caches[b], x[b:b + 1].astype(np.float64), 0)
            fills[b] = O.next_fill(fills[b], T, 0, C)
        assert st.fill() == fills
    assert np.array_equal(st.read_cache().cpu().numpy(), np.concatenate(caches, 0).astype(np.float32))


@pytest.mark.parametrize("d_model,n_heads", [(128, 2), (256, 2)])
@pytest.mark.parametrize("T,lengths", [(12, [12, 7, 1]), (16, [16, 16, 9]), (1, [1, 1, 1])])
@pytest.mark.parametrize("ctx", [None, ((4, 1), "chunked_limited"), ((3, 2), "regular")])
def test_forward_f32_short_utterances(d_model, n_heads, T, lengths, ctx):
    """Offline fp32 utterances of at most 16 frames take the chunk kernel
    (one workgroup per item and head, keys = the utterance); with key
    padding, one-frame items and contexts, against the oracle within the
    fp32 bound on the rows that see a key."""
    rng = np.random.default_rng(91)
    w = random_weights(rng, d_model, n_heads, scale=0.08)
    p = oracle_params(w, d_model, n_heads)
    B = len(lengths)
    x = rng.standard_normal((B, T, d_model)).astype(np.float32)
    pos = O.RelPositionalEncoding(d_model, 5000, False).get_encoding(T)
    octx = O.AttentionContext.new(*ctx) if ctx else None
    ref = O.mhsa_forward(p, x, pos, octx, O.key_padding_mask(lengths, T))
    layer = gpu_layer(w, d_model, n_heads, True, O.F32)
    got = host(layer.forward(dev(x, O.F32), dev(pos, O.F32), M.AttentionContext.new(*ctx) if ctx else None,
                             M.key_padding_mask(lengths, T)))
    rows = visible_rows(B, T, octx, lengths)
    assert row_rel_err(got, ref, rows) < F32_TOL


@pytest.mark.parametrize("d_model,n_heads,T", [(256, 2, 50), (1024, 8, 40), (1280, 10, 30)])
def test_sublayer_f32_against_oracle(d_model, n_heads, T):
    """x + MHSA(LayerNorm(x)) (conformer.rs:1747-1780) in fp32 with LayerNorm
    gamma/beta and key padding: the LayerNorm kernel's statistics and affine,
    the attention and the residual-fused output GEMM, within the fp32 bound."""
    rng = np.random.default_rng(31)
    w = random_weights(rng, d_model, n_heads)
    p = oracle_params(w, d_model, n_heads)
    x = rng.normal(size=(2, T, d_model)) * 3.0 + 0.5
    gamma = rng.uniform(0.5, 1.5, d_model).astype(np.float32)
    beta = rng.normal(0, 0.1, d_model).astype(np.float32)
    lengths = [T, T - 7]
    pos = O.RelPositionalEncoding(d_model, 5000, False).get_encoding(T)
    ref = O.mhsa_sublayer(p, x, pos, None, O.key_padding_mask(lengths, T), gamma=gamma, beta=beta, dtype=O.F32)
    layer = gpu_layer(w, d_model, n_heads, True, O.F32)
    xd = dev(x, O.F32)
    layer.sublayer_forward_(xd, dev(pos, O.F32), None, M.key_padding_mask(lengths, T), gamma=gamma, beta=beta)
    got = host(xd)
    vis = visible_rows(2, T, None, lengths)
    assert row_rel_err(got[vis], ref[vis]) < F32_TOL


# ---------------------------------------------------------------------------
# quantized 24-layer stack
# ---------------------------------------------------------------------------

def _stack_oracle(layers, cfg, x, lengths, pos, T):
    out = O.bf16_round(x)
    for wts in layers:
        p = oracle_params(wts, cfg.d_model, cfg.n_heads)
        out = O.mhsa_sublayer(p, out, O.bf16_round(pos), None, O.key_padding_mask(lengths, T), dtype=O.BF16)
    return out


def _stack_gpu(layers, cfg, x, lengths, pos):
    gl = [gpu_layer(wts, cfg.d_model, cfg.n_heads, False, O.BF16) for wts in layers]
    xd = dev(x, O.BF16)
    pd = dev(pos, O.BF16)
    for layer in gl:
        layer.sublayer_forward_(xd, pd, None, M.key_padding_mask(lengths, x.shape[1]))
    return xd


@pytest.mark.parametrize("dtype", [O.BF16, O.F32])
def test_quantized_linear_full_shape(dtype):
    """The fused dequant-GEMM at the stack's shape (M = 4 x 1500 rows) with
    the specified code/scale/bias distribution. In bf16 every output is within
    one bf16 ulp of the oracle (float64 dot product of the bf16-dequantised
    weights, rounded once) plus one fp32 rounding unit of sum |x||w| -- the
    fp32 accumulation noise, which dominates only for outputs near zero
    (|y| < 2e-3 against terms of ~1.5). In fp32: within 1e-5 relative."""
    cfg = W.CONFIGS["xl_stack_u8"]
    layers, x, _ = W.instantiate(cfg)
    w = layers[0]
    p = oracle_params(w, cfg.d_model, cfg.n_heads)
    layer = gpu_layer(w, cfg.d_model, cfg.n_heads, False, dtype)
    xin = (O.bf16_round(x) if dtype == O.BF16 else x.astype(np.float64)).reshape(-1, cfg.d_model)
    xd = dev(x, dtype)
    for name in ("linear_q", "linear_pos"):
        got = host(layer.debug_linear(name, xd)).reshape(-1, cfg.d_model)
        lin = getattr(p, name)
        ref = lin.forward(xin, dtype)
        if dtype == O.BF16:
            _, e = np.frexp(ref)
            ulp = np.ldexp(1.0, e - 8)
            acc = np.abs(xin) @ np.abs(lin.dense_weight(dtype)).T * 2.0 ** -24
            d = np.abs(got - ref)
            print(f"{name}: {int(np.sum(d > ulp))} of {d.size} outputs beyond 1 ulp, worst excess "
                  f"{np.max((d - ulp) / acc):.3f} fp32 units of sum|x||w|")
            assert np.all(d <= ulp + acc), name
        else:
            assert row_rel_err(got, ref) < 1e-5, name


@pytest.mark.parametrize("d_model,n_heads,rows", [(384, 6, 1537), (768, 6, 3000)])
def test_quantized_linear_bf16_tile_shapes(d_model, n_heads, rows):
    """The bf16 dequant-GEMM on shapes that take the other tile paths: d_model
    384 with 1537 rows gives 64x64 tiles over six k-stages and a ragged last
    row tile; 768 with 3000 rows gives larger tiles over 12 stages. Codes, scales and biases as the stack specifies; every output
    within one bf16 ulp of the oracle plus one fp32 rounding unit of
    sum |x||w|, as in the full-shape test."""
    rng = np.random.default_rng(71)
    w = W.make_layer_weights(rng, d_model, n_heads, False, True)
    p = oracle_params(w, d_model, n_heads)
    layer = gpu_layer(w, d_model, n_heads, False, O.BF16)
    x = O.bf16_round(rng.normal(size=(rows, d_model)))
    xd = dev(x, O.BF16)
    for name in ("linear_q", "linear_out"):
        got = host(layer.debug_linear(name, xd))
        lin = getattr(p, name)
        ref = lin.forward(x, O.BF16)
        _, e = np.frexp(ref)
        ulp = np.ldexp(1.0, e - 8)
        acc = np.abs(x) @ np.abs(lin.dense_weight(O.BF16)).T * 2.0 ** -24
        d = np.abs(got - ref)
        print(f"{name} d_model={d_model}: {int(np.sum(d > ulp))} of {d.size} beyond 1 ulp")
        assert np.all(d <= ulp + acc), name


def test_stack_u8_well_conditioned_against_oracle():
    """Two quantized sublayers (pre-LN, residual) at B=2, T=300 with codes
    U{0..255}, scales U(1e-4, 1e-3) and biases -128 s + N(0, 1e-3), so weights
    are zero-mean with |W| ~ 0.1 and the softmax is not argmax-degenerate.
    The residual stream reaches |x| ~ 5 where one bf16 ulp is 0.03, so the
    bound is 2e-2 of max |ref|."""
    cfg = W.CONFIGS["xl_stack_u8"]
    rng = np.random.default_rng(41)
    layers = []
    for _ in range(2):
        wts = W.make_layer_weights(rng, cfg.d_model, cfg.n_heads, False, True)
        for name in ("linear_q", "linear_k", "linear_v", "linear_out", "linear_pos"):
            s = rng.uniform(1e-4, 1e-3, size=wts[f"{name}.scales"].shape)
            wts[f"{name}.scales"] = s.astype(np.float16)
            b = -128.0 * wts[f"{name}.scales"].astype(np.float64) + rng.normal(0, 1e-3, size=s.shape)
            wts[f"{name}.biases"] = b.astype(np.float16)
        layers.append(wts)
    T, lengths = 300, [300, 217]
    x = rng.standard_normal((2, T, cfg.d_model)).astype(np.float32)
    pos = O.RelPositionalEncoding(cfg.d_model, 5000, True).get_encoding(T)
    ref = _stack_oracle(layers, cfg, x, lengths, pos, T)
    got = host(_stack_gpu(layers, cfg, x, lengths, pos))
    err = rel_err(got, ref)
    n_far = int(np.sum(np.abs(got - ref) > 2e-2))
    print(f"well-conditioned u8 stack: max abs error {abs_err(got, ref):.3e}, / max|ref| {err:.3e}, "
          f"{n_far} of {ref.size} outputs beyond 2e-2 absolute")
    assert err < 2e-2


@pytest.mark.parametrize("kind", ["u8_8wave_fused", "u8_mixed_fused", "bf16_4wave", "f32"])
def test_stack_sublayer_forward_equals_layer_loop(kind):
    """mhsa_stack_sublayer_forward gives the results of mhsa_sublayer_forward
    called layer by layer, bit for bit: at the quantized stack's shape (B=4,
    T=1500, key padding: each next layer's position projection runs in the
    same launch as the attention), on a bf16 shape of the 4-wave form and in
    fp32 (projections run apart), with per-layer LayerNorm parameters. At the
    stack's shape, lengths 1014, 1438, 1303, 1396 keep every item in the
    8-wave form; with lengths 1000, 1364, 1295, 1227 (the stack workload's)
    the longest item takes the 4-wave form in the same launch."""
    if kind.startswith("u8_"):
        cfg = W.CONFIGS["xl_stack_u8"]
        D, H, T, B, n = cfg.d_model, cfg.n_heads, cfg.seq_len, cfg.batch, 3
        rng = np.random.default_rng(47)
        wts = [W.make_layer_weights(rng, D, H, False, True) for _ in range(n)]
        lengths = [int(v) for v in rng.integers(1000, T + 1, size=B)]
        if kind == "u8_mixed_fused":
            lengths = [1000, 1364, 1295, 1227]
        dtype = O.BF16
    else:
        D, H, T, B, n = 256, 2, 300, 3, 3
        rng = np.random.default_rng(48)
        wts = [W.make_layer_weights(rng, D, H, True, False) for _ in range(n)]
        lengths = [300, 211, 97]
        dtype = O.BF16 if kind == "bf16_4wave" else O.F32
    layers = [gpu_layer(w, D, H, not kind.startswith("u8_"), dtype) for w in wts]
    gamma = 1.0 + 0.1 * rng.standard_normal((n, D))
    beta = 0.1 * rng.standard_normal((n, D))
    x = rng.standard_normal((B, T, D))
    pos = O.RelPositionalEncoding(D, 5000, True).get_encoding(T)
    kmask = M.key_padding_mask(lengths, T)
    xa, pd = dev(x, dtype), dev(pos, dtype)
    xb = xa.clone()
    for i, layer in enumerate(layers):
        layer.sublayer_forward_(xa, pd, None, kmask, gamma[i], beta[i])
    before = M.debug_attention_forms()
    M.stack_sublayer_forward_(layers, xb, pd, None, kmask, gamma, beta)
    torch.cuda.synchronize()
    after = M.debug_attention_forms()
    ran = {k: after[k] - before[k] for k in after if after[k] > before[k]}
    want = {"u8_8wave_fused": {"bf16_mixed_gemm": n - 1, "bf16_wave8": 1},
            "u8_mixed_fused": {"bf16_mixed_gemm": n - 1, "bf16_mixed": 1},
            "bf16_4wave": {"bf16_wave4": n}, "f32": {"generic_key_split": n}}[kind]
    assert ran == want, ran
    assert torch.isfinite(xb.float()).all()
    assert torch.equal(xa, xb), f"{kind}: max difference {float((xa.float() - xb.float()).abs().max()):.3g}"


def test_stack_u8_full_size_deterministic():
    cfg = W.CONFIGS["xl_stack_u8"]
    layers, x, ex = W.instantiate(cfg)
    pos = M.RelPositionalEncoding(cfg.d_model, 5000, True).get_encoding(cfg.seq_len).numpy()
    a = _stack_gpu(layers, cfg, x, ex["lengths"], pos)
    b = _stack_gpu(layers, cfg, x, ex["lengths"], pos)
    assert torch.isfinite(a.float()).all()
    assert torch.equal(a, b)


# ---------------------------------------------------------------------------
# on-disk checkpoints
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("quantized", [True, False])
def test_layer_from_safetensors_checkpoint(tmp_path, quantized):
    """A layer loaded from an MLX safetensors checkpoint (written by the
    safetensors package, quantization in config.json) computes exactly what
    the same weights loaded from memory compute, in bf16."""
    import json
    from safetensors.numpy import save_file
    rng = np.random.default_rng(72)
    d, h, T = 256, 2, 90
    w = W.make_layer_weights(rng, d, h, True, quantized, centred=True)
    prefix = "encoder.layers.3.self_attn"
    save_file({f"{prefix}.{k}": np.ascontiguousarray(v) for k, v in w.items()}, str(tmp_path / "model.safetensors"),
              metadata={"format": "mlx"})
    if quantized:
        (tmp_path / "config.json").write_text(json.dumps({"quantization": {"bits": 8, "group_size": 64}}))
    a = M.RelPositionMultiHeadAttention(d, h, True)
    a.load_checkpoint(M.Checkpoint(str(tmp_path)), prefix)
    a.set_dtype(O.BF16)
    b = gpu_layer(w, d, h, True, O.BF16)
    x = dev(rng.standard_normal((2, T, d)), O.BF16)
    pos = dev(O.RelPositionalEncoding(d, 5000, True).get_encoding(T), O.BF16)
    assert torch.equal(a.forward(x, pos, None, [T, 51]), b.forward(x, pos, None, [T, 51]))


# ---------------------------------------------------------------------------
# encoder-level streaming: the stack of attention sublayers
# ---------------------------------------------------------------------------

def _stack_oracle_step(params, gammas, betas, xb, caches_b, pos, fill, T, C, dtype):
    """One chunk of one session through the layers, as the reference's
    ConformerBlock::forward_with_cache attention part (conformer.rs:1924-1934)
    with the session's own fill."""
    mask = O.streaming_mask((70, 13), "chunked_limited", C, fill, T, T)
    for l, p in enumerate(params):
        h = O.layer_norm(xb, O.to_dtype(gammas[l], dtype), O.to_dtype(betas[l], dtype), 1e-5, O.F32)
        y, caches_b[l] = O.mhsa_forward_with_cache(p, h, pos, caches_b[l], mask, dtype=dtype)
        xb = xb + y
    return xb


@pytest.mark.parametrize("dtype,quant,n_layers,B,steps", [(O.F32, False, 24, 4, 50), (O.BF16, True, 4, 3, 8)])
def test_streaming_stack_against_per_session_oracle(dtype, quant, n_layers, B, steps):
    """n_layers attention sublayers streamed together for `steps` chunks:
    14-frame chunks, a 70-frame cache per layer, [70,13] chunked_limited,
    per-session fills and LayerNorm parameters per layer. The oracle runs
    every session as its own B=1 reference stream through every layer; each
    step's output is checked (fp32 bound), and so are the caches of all
    layers read back at the end (they hold each layer's LayerNorm output,
    computed in fp32 here and in float64 by the oracle, so not bit-equal)."""
    rng = np.random.default_rng(81)
    d, h, C, T = 256, 4, 70, 14
    ws = []
    for _ in range(n_layers):
        if quant:
            w = W.make_layer_weights(rng, d, h, True, True, centred=True)
            for name in ("linear_q", "linear_k", "linear_v", "linear_out", "linear_pos"):
                sc = rng.uniform(1e-4, 1e-3, size=w[f"{name}.scales"].shape)
                w[f"{name}.scales"] = sc.astype(np.float16)
                w[f"{name}.biases"] = (-128.0 * w[f"{name}.scales"].astype(np.float64)).astype(np.float16)
                if name != "linear_pos":
                    w[f"{name}.bias"] = rng.normal(0, 0.1, d).astype(np.float16)
        else:
            w = random_weights(rng, d, h, use_bias=True, scale=0.05)
        ws.append(w)
    params = [oracle_params(w, d, h) for w in ws]
    gammas = rng.uniform(0.5, 1.5, (n_layers, d)).astype(np.float32)
    betas = rng.normal(0, 0.1, (n_layers, d)).astype(np.float32)
    layers = [gpu_layer(w, d, h, True, dtype, prefix=f"l{i}") for i, w in enumerate(ws)]
    stack = M.StreamingStack(layers, B, C, T)
    cache = rng.standard_normal((n_layers, B, C, d)).astype(np.float32)
    fills = [int(v) for v in rng.integers(0, C + 1, size=B)]
    for b in range(B):
        cache[:, b, :C - fills[b]] = 0.0
    stack.load_cache(dev(cache, O.F32), fills)
    caches = [[cache[l, b:b + 1].astype(np.float64) for l in range(n_layers)] for b in range(B)]
    pos = O.RelPositionalEncoding(d, 5000, True).get_encoding(C + T)
    pos = pos if dtype == O.F32 else O.bf16_round(pos)
    pos_d = dev(pos, dtype)
    worst = 0.0
    for step in range(steps):
        x = rng.standard_normal((B, T, d)).astype(np.float32)
        xd = dev(x, O.F32)
        stack.step_(xd, pos_d, M.StreamingMask((70, 13), "chunked_limited"), gammas, betas)
        got = host(xd)
        for b in range(B):
            ref = _stack_oracle_step(params, gammas, betas, x[b:b + 1].astype(np.float64), caches[b], pos, fills[b],
                                     T, C, dtype)
            e = row_rel_err(got[b:b + 1], ref)
            worst = max(worst, e)
            assert e < F32_TOL, (step, b, e)
            fills[b] = O.next_fill(fills[b], T, 0, C)
        assert stack.fill() == fills
    print(f"stack of {n_layers} layers, {steps} steps: worst per-row relative error {worst:.3e}")
    got_cache = stack.read_cache().cpu().numpy()
    ref_cache = np.stack([np.concatenate([caches[b][l] for b in range(B)], 0) for l in range(n_layers)])
    live = np.abs(ref_cache).max(axis=-1) > 0  # unfilled rows are zeros on both sides
    assert np.array_equal(got_cache[~live], ref_cache[~live].astype(np.float32))
    assert row_rel_err(got_cache[live], ref_cache[live]) < 1e-5


# ---------------------------------------------------------------------------
# FeedForward (conformer.rs:2031-2088)
# ---------------------------------------------------------------------------

def _ffn_weights(rng, d, f, quant, prefix="ff"):
    """linear1 [f, d], linear2 [d, f] with biases: dense Xavier, or affine u8
    with zero-mean weights (scales U(1e-4, 1e-3)) so activations stay O(1)."""
    w = {}
    for name, (o, i) in (("linear1", (f, d)), ("linear2", (d, f))):
        if quant:
            codes = rng.integers(0, 256, size=(o, i))
            sc = rng.uniform(1e-4, 1e-3, size=(o, i // 64)).astype(np.float16)
            w[f"{prefix}.{name}.weight"] = W.pack_u8(codes)
            w[f"{prefix}.{name}.scales"] = sc
            w[f"{prefix}.{name}.biases"] = (-128.0 * sc.astype(np.float64) + rng.normal(0, 1e-3, sc.shape)).astype(np.float16)
            w[f"{prefix}.{name}.bias"] = rng.normal(0, 0.1, o).astype(np.float16)
        else:
            w[f"{prefix}.{name}.weight"] = W.xavier(rng, o, i)
            w[f"{prefix}.{name}.bias"] = rng.normal(0, 0.1, o).astype(np.float32)
    return w


def _ffn_oracle(w, prefix="ff"):
    lin = []
    for name in ("linear1", "linear2"):
        k = f"{prefix}.{name}"
        if f"{k}.scales" in w:
            lin.append(O.LinearLayer(w[f"{k}.weight"], w[f"{k}.bias"], w[f"{k}.scales"], w[f"{k}.biases"]))
        else:
            lin.append(O.LinearLayer(np.asarray(w[f"{k}.weight"], np.float64), w[f"{k}.bias"]))
    return O.FeedForwardParams(*lin)


@pytest.mark.parametrize("dtype,quant,rows", [(O.BF16, True, 6000), (O.BF16, False, 6000), (O.F32, True, 500),
                                              (O.F32, False, 37)])
def test_feed_forward_against_oracle(dtype, quant, rows):
    """FeedForward at the 0.6B shape (d_model 1024, ff_dim 4096; 6000 rows is
    the stack's B=4 x T=1500): linear1 with the SiLU epilogue, linear2, on the
    same dequant-GEMMs as the attention projections; then the half-step
    sublayer x + 0.5 FF(LN(x)) with the residual in linear2's epilogue.
    Outputs reach ~15, where one bf16 ulp is 0.0625, so bf16 is bounded per
    row (2e-2 of the row's max), fp32 within 1e-4 per row."""
    rng = np.random.default_rng(91)
    d, f = 1024, 4096
    w = _ffn_weights(rng, d, f, quant)
    p = _ffn_oracle(w)
    ff = M.FeedForward(d, f, True)
    ff.load_weights(w, "ff")
    ff.set_dtype(dtype)
    x = rng.standard_normal((rows, d))
    x = O.bf16_round(x) if dtype == O.BF16 else x.astype(np.float32).astype(np.float64)
    got = host(ff.forward(dev(x, dtype)))
    ref = O.feed_forward(p, x, dtype)
    err = row_rel_err(got, ref)
    print(f"feed_forward {dtype} quant={quant} rows={rows}: per-row error {err:.3e}, max abs "
          f"{abs_err(got, ref):.3e} (max |ref| {np.max(np.abs(ref)):.2f})")
    assert err < (BF16_TOL if dtype == O.BF16 else F32_TOL)
    gamma = rng.uniform(0.5, 1.5, d).astype(np.float32)
    beta = rng.normal(0, 0.1, d).astype(np.float32)
    xd = dev(x, dtype)
    ff.sublayer_forward_(xd, gamma, beta)
    ref = O.feed_forward_sublayer(p, x, gamma, beta, dtype)
    err = row_rel_err(host(xd), ref)
    print(f"  sublayer: per-row error / row max {err:.3e}")
    assert err < (BF16_TOL if dtype == O.BF16 else F32_TOL)


@pytest.mark.parametrize("quant", [False, True])
def test_feed_forward_f32_activations_in_bf16_module(quant):
    """The streaming path's FeedForward: f32 activations meet a bf16 module,
    so every op promotes to f32 over the parameters' bf16 values (quantized
    weights dequantised in f32 from their bf16-cast scales), and nothing is
    rounded to bf16; forward and the half-step sublayer, within the fp32
    bound, 224 rows (16 sessions x 14 frames)."""
    rng = np.random.default_rng(93)
    d, f = 1024, 4096
    w = _ffn_weights(rng, d, f, quant)
    p = _ffn_oracle(w)
    ff = M.FeedForward(d, f, True)
    ff.load_weights(w, "ff")
    ff.set_dtype(O.BF16)
    x = rng.standard_normal((224, d)).astype(np.float32).astype(np.float64)
    got = host(ff.forward(dev(x, O.F32)))
    ref = O.feed_forward(p, x, O.BF16, act=O.F32)
    err = row_rel_err(got, ref)
    print(f"feed_forward bf16 module, f32 activations, quant={quant}: per-row error {err:.3e}")
    assert err < F32_TOL
    gamma = rng.uniform(0.5, 1.5, d).astype(np.float32)
    beta = rng.normal(0, 0.1, d).astype(np.float32)
    xd = dev(x, O.F32)
    ff.sublayer_forward_(xd, gamma, beta)
    ref = O.feed_forward_sublayer(p, x, gamma, beta, O.BF16, act=O.F32)
    err = row_rel_err(host(xd), ref)
    print(f"  sublayer: per-row error {err:.3e}")
    assert err < F32_TOL
