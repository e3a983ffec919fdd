"""GPU parity of the whole Conformer block and the encoder's layer loops
against the oracle's composed block (conformer.rs:1693-1971).

Tolerances: fp32 per output row max |gpu - oracle| / max |oracle| <= 1e-4.
bf16: per output row max |gpu - oracle| <= 2e-2 of the row's max |oracle|.
Five bf16-rounded sublayers run in sequence (each checked on its own at
2e-2 absolute elsewhere): a one-ulp difference of an intermediate that the
GPU's fp32 sums and the oracle's exact ones round to different neighbours
moves the later sublayers' sums, so a few outputs of |x| ~ 2-5 end two or
three ulps (0.03-0.05) from the oracle's; measured 265 (dense) and 1082 (u8)
of 614400 outputs past 2e-2 absolute, largest 0.047 at row maxima ~4, and
the check also bounds that count at 1%.
"""
import ctypes

import numpy as np
import pytest
import torch

import relpos_oracle as O
import relpos_mhsa as M
from _util import block_oracle, block_weights, row_rel_err

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


def gpu_block(w, d, h, f, k, norm, causal, dtype, prefix="blk"):
    blk = M.ConformerBlock(d, h, f, k, norm, causal, True)
    blk.load_weights(w, prefix)
    blk.set_dtype(dtype)
    return blk


@pytest.mark.parametrize("dtype,quant,norm,causal", [(O.BF16, False, "batch_norm", False),
                                                     (O.BF16, True, "batch_norm", False),
                                                     (O.F32, False, "layer_norm", True),
                                                     (O.F32, True, "batch_norm", False)])
def test_block_offline_against_oracle(dtype, quant, norm, causal):
    """One 0.6B-shape block (d_model 1024, 8 heads, ff 4096, conv kernel 9)
    at B=3, T=200 with key/frame padding (lengths 200, 131, 57), dense or
    affine u8 projections, against conformer_block."""
    d, h, f, k, B, T = 1024, 8, 4096, 9, 3, 200
    rng = np.random.default_rng(70 + quant)
    w = block_weights(rng, d, h, f, k, norm, quant)
    p = block_oracle(w, d, h, norm, causal)
    lengths = [200, 131, 57]
    x = O.to_dtype(rng.standard_normal((B, T, d)), dtype)
    pos = O.to_dtype(O.RelPositionalEncoding(d, 5000, True).get_encoding(T), dtype)
    blk = gpu_block(w, d, h, f, k, norm, causal, dtype)
    xd = dev(x, dtype)
    blk.forward_(xd, dev(pos, dtype), None, lengths)
    got = host(xd)
    ref = O.conformer_block(p, x, pos, None, lengths, dtype)
    if dtype == O.F32:
        err = row_rel_err(got, ref)
        print(f"block f32 quant={quant}: max per-row error / row max {err:.3e}")
        assert err < F32_TOL
    else:
        err = row_rel_err(got, ref)
        n_far = int(np.sum(np.abs(got - ref) > BF16_TOL))
        print(f"block bf16 quant={quant}: max |err| {np.max(np.abs(got - ref)):.3e}, per-row error / row max "
              f"{err:.3e}, {n_far} of {got.size} outputs beyond {BF16_TOL} (max |ref| {np.max(np.abs(ref)):.2f})")
        assert err < BF16_TOL
        assert n_far <= 1e-2 * got.size


@pytest.mark.parametrize("dtype,quant", [(O.BF16, False), (O.F32, True)])
def test_block_offline_large_shape_against_oracle(dtype, quant):
    """The FastConformer large shape (d_model 512, 8 heads of 64, ff 2048,
    conv kernel 9): the d_k = 64 attention forms, the GEMMs at 512 and 2048
    columns and the 512-wide LayerNorms inside one block, at B=4, T=250 with
    key/frame padding (lengths 250, 199, 120, 33), against conformer_block."""
    d, h, f, k, B, T = 512, 8, 2048, 9, 4, 250
    rng = np.random.default_rng(512 + quant)
    w = block_weights(rng, d, h, f, k, "batch_norm", quant)
    p = block_oracle(w, d, h, "batch_norm", False)
    lengths = [250, 199, 120, 33]
    x = O.to_dtype(rng.standard_normal((B, T, d)), dtype)
    pos = O.to_dtype(O.RelPositionalEncoding(d, 5000, True).get_encoding(T), dtype)
    blk = gpu_block(w, d, h, f, k, "batch_norm", False, dtype)
    xd = dev(x, dtype)
    blk.forward_(xd, dev(pos, dtype), None, lengths)
    got = host(xd)
    ref = O.conformer_block(p, x, pos, None, lengths, dtype)
    err = row_rel_err(got, ref)
    if dtype == O.F32:
        print(f"large block f32 quant={quant}: max per-row error / row max {err:.3e}")
        assert err < F32_TOL
    else:
        n_far = int(np.sum(np.abs(got - ref) > BF16_TOL))
        print(f"large block bf16: per-row error / row max {err:.3e}, {n_far} of {got.size} outputs beyond {BF16_TOL}")
        assert err < BF16_TOL
        assert n_far <= 1e-2 * got.size


def test_block_bf16_causal_conv_is_refused():
    d, h, f, k = 256, 2, 512, 4
    rng = np.random.default_rng(72)
    w = block_weights(rng, d, h, f, k, "layer_norm", False)
    blk = gpu_block(w, d, h, f, k, "layer_norm", True, O.BF16)
    x = dev(rng.standard_normal((1, 10, d)), O.BF16)
    pos = dev(O.RelPositionalEncoding(d, 5000, True).get_encoding(10), O.BF16)
    with pytest.raises(M.MhsaError) as e:
        blk.forward_(x, pos)
    assert e.value.code == M.MHSA_ENOTSUP


@pytest.mark.parametrize("quant", [False, True])
def test_block_forward_to_bf16_causal_against_oracle(quant):
    """A bf16 block with a causal conv (kernel 9, LayerNorm) on bf16 input:
    FF1 and the MHSA sublayer in bf16, then the conv's f32 zero padding
    promotes the depthwise conv and everything after it (conformer.rs:
    2250-2256), so the block returns f32 (mhsa_block_forward_to). 0.6B
    shape at B=3, T=200 with lengths (200, 131, 57), dense or affine u8
    projections, against conformer_block; the bf16 sublayers' roundings
    carry into the f32 result, so the bound is the bf16 block's. x is left
    as it was."""
    d, h, f, k, B, T = 1024, 8, 4096, 9, 3, 200
    rng = np.random.default_rng(80 + quant)
    w = block_weights(rng, d, h, f, k, "layer_norm", quant)
    p = block_oracle(w, d, h, "layer_norm", True)
    lengths = [200, 131, 57]
    x = O.to_dtype(rng.standard_normal((B, T, d)), O.BF16)
    pos = O.to_dtype(O.RelPositionalEncoding(d, 5000, True).get_encoding(T), O.BF16)
    blk = gpu_block(w, d, h, f, k, "layer_norm", True, O.BF16)
    assert blk.output_dtype(torch.bfloat16) == torch.float32
    xd = dev(x, O.BF16)
    x0 = xd.clone()
    out = blk.forward(xd, dev(pos, O.BF16), None, lengths)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and torch.equal(xd, x0)
    got = host(out)
    ref = O.conformer_block(p, x, pos, None, lengths, O.BF16)
    assert not np.array_equal(ref, O.bf16_round(ref))  # the oracle's result is f32 too
    err = row_rel_err(got, ref)
    n_far = int(np.sum(np.abs(got - ref) > BF16_TOL))
    print(f"bf16 causal block quant={quant}: max |err| {np.max(np.abs(got - ref)):.3e}, per-row error / row max "
          f"{err:.3e}, {n_far} of {got.size} outputs beyond {BF16_TOL}")
    assert err < BF16_TOL
    assert n_far <= 1e-2 * got.size


@pytest.mark.parametrize("ctx,quant", [(None, False), (((100, 8), "regular"), True),
                                       (((160, 15), "chunked_limited"), False)])
def test_block_forward_to_f32_activations_against_oracle(ctx, quant):
    """A bf16 block on f32 activations (what every block after the first
    causal conv of a bf16 encoder receives): every op in f32 on the bf16
    parameter values, the attention as the offline forward computes it from
    an f32 x -- key padding (lengths 180, 97), the context, matrix_bd in
    f32 over the layer's bf16 position rows (handed to the oracle, as in the
    streaming tests) -- against conformer_block(act=f32) at the f32 bound.
    In place (out = x). (Each window reaches key 0 from every row: a row
    that sees no key is NaN in the reference.)"""
    d, h, f, k, B, T = 512, 4, 2048, 9, 2, 180
    rng = np.random.default_rng(83 + quant)
    w = block_weights(rng, d, h, f, k, "layer_norm", quant)
    p = block_oracle(w, d, h, "layer_norm", True)
    lengths = [180, 97]
    context = M.AttentionContext.new(*ctx) if ctx else None
    octx = O.AttentionContext.new(*ctx) if ctx else None
    x = rng.standard_normal((B, T, d)).astype(np.float32).astype(np.float64)
    pos = O.to_dtype(O.RelPositionalEncoding(d, 5000, True).get_encoding(T), O.BF16)
    blk = gpu_block(w, d, h, f, k, "layer_norm", True, O.BF16)
    pos_d = dev(pos, O.BF16)
    xd = dev(x, O.F32)
    assert blk.output_dtype(torch.float32) == torch.float32
    lib = M.library()
    M._check(lib.mhsa_block_forward_to(blk._h, M._dptr(xd), M.F32, B, T, M._dptr(pos_d), pos_d.shape[1],
                                       ctypes.byref(context.c()) if context else None, M._int_array(lengths),
                                       M._dptr(xd), M._stream_ptr()))
    got = host(xd)
    ref = O.conformer_block(p, x, pos, octx, lengths, O.BF16, act=O.F32, pos_rows=_layer_pos_rows(blk, pos_d))
    err = row_rel_err(got, ref)
    print(f"bf16 block on f32 activations ctx={ctx} quant={quant}: per-row error / row max {err:.3e}")
    assert err < F32_TOL


def test_encoder_forward_to_promotes_like_the_block_loop():
    """mhsa_encoder_forward_to over bf16 blocks (symmetric, causal, causal):
    bf16 activations through the first, f32 from the second's conv on (the
    loop moves them out of the output buffer before the promotion), equal
    bit for bit to chaining ConformerBlock.forward, and against the oracle's
    conformer_encoder with each layer's bf16 position rows."""
    d, h, f, k, B, T = 512, 4, 2048, 9, 2, 150
    rng = np.random.default_rng(86)
    kinds = [("batch_norm", False), ("layer_norm", True), ("layer_norm", True)]
    ws = [block_weights(rng, d, h, f, k, nrm, False, prefix=f"l{i}") for i, (nrm, _) in enumerate(kinds)]
    ps = [block_oracle(w, d, h, nrm, c, prefix=f"l{i}") for i, (w, (nrm, c)) in enumerate(zip(ws, kinds))]
    blks = [gpu_block(w, d, h, f, k, nrm, c, O.BF16, prefix=f"l{i}") for i, (w, (nrm, c)) in enumerate(zip(ws, kinds))]
    x = O.to_dtype(rng.standard_normal((B, T, d)), O.BF16)
    pos = O.to_dtype(O.RelPositionalEncoding(d, 5000, True).get_encoding(T), O.BF16)
    xd, pos_d = dev(x, O.BF16), dev(pos, O.BF16)
    lengths = [150, 97]
    y = xd
    for blk in blks:
        y = blk.forward(y, pos_d, None, lengths)
    out = M.encoder_forward(blks, xd, pos_d, None, lengths)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and torch.equal(out, y)
    rows = [_layer_pos_rows(blk, pos_d) for blk in blks]
    ref, act = O.conformer_encoder(ps, x, pos, None, lengths, O.BF16, pos_rows=rows)
    assert act == O.F32
    err = row_rel_err(host(out), ref)
    print(f"encoder (bf16: symmetric, causal, causal): per-row error / row max {err:.3e}")
    assert err < BF16_TOL


def test_encoder_forward_equals_block_loop():
    """The offline encoder loop over 3 bf16 blocks equals calling each block
    in turn, bit for bit."""
    d, h, f, k, B, T = 512, 4, 2048, 9, 2, 150
    rng = np.random.default_rng(73)
    ws = [block_weights(rng, d, h, f, k, "batch_norm", False, prefix=f"l{i}") for i in range(3)]
    blks = [gpu_block(w, d, h, f, k, "batch_norm", False, O.BF16, prefix=f"l{i}") for i, w in enumerate(ws)]
    x = dev(rng.standard_normal((B, T, d)), O.BF16)
    pos = dev(O.RelPositionalEncoding(d, 5000, True).get_encoding(T), O.BF16)
    a, b = x.clone(), x.clone()
    for blk in blks:
        blk.forward_(a, pos, None, [150, 97])
    M.encoder_forward_(blks, b, pos, None, [150, 97])
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("tag", ["linear1", "linear2", "pointwise_conv2", "gemm_out"])
def test_profiler_repeat_issues_in_place_launches_once(tag):
    """The event profiler issues the launches of its repeat tag n times per
    event pair. The residual forms that update x in place (FeedForward
    linear2, pointwise_conv2, the attention's output projection) are issued
    once whatever the tag, and credited with one launch; others (linear1)
    with n. Either way the block's output equals the unprofiled one."""
    d, h, f, k, B, T, n, calls = 512, 4, 2048, 9, 2, 150, 4, 3
    rng = np.random.default_rng(75)
    w = block_weights(rng, d, h, f, k, "batch_norm", False)
    blk = gpu_block(w, d, h, f, k, "batch_norm", False, O.BF16)
    x = dev(rng.standard_normal((B, T, d)), O.BF16)
    pos = dev(O.RelPositionalEncoding(d, 5000, True).get_encoding(T), O.BF16)
    a, b = x.clone(), x.clone()
    for _ in range(calls):
        blk.forward_(a, pos, None, [150, 97])
    parts = blk.parts()
    for pt in parts:
        pt.profile_reset()
        pt.profile_repeat(tag, n)
        pt.profile(True)
    for _ in range(calls):
        blk.forward_(b, pos, None, [150, 97])
    torch.cuda.synchronize()
    counts = [pt.profile_read() for pt in parts]
    for pt in parts:
        pt.profile(False)
        pt.profile_repeat(None, 1)
    assert torch.equal(a, b), tag
    got = sum(c[tag][1] for c in counts if tag in c)
    owners = sum(1 for c in counts if tag in c)  # FeedForward tags: both FeedForwards
    expect = owners * calls * (n if tag == "linear1" else 1)
    assert got == expect, (tag, got, expect)


def _layer_pos_rows(blk, pos_d):
    """The bf16 position rows the block's attention layer projects (its
    streaming memo), through the layer's own GEMM."""
    lib = M.library()
    h = lib.mhsa_block_attention(blk._h)
    rows = pos_d.numel() // pos_d.shape[-1]
    out = torch.empty_like(pos_d)
    M._check(lib.mhsa_debug_linear(h, M.LINEARS.index("linear_pos"), M._dptr(pos_d), rows, M._dptr(out),
                                   M._stream_ptr()))
    return host(out)[0]


@pytest.mark.timeout(900)
@pytest.mark.parametrize("dtype,steps", [(O.F32, 24), (O.BF16, 8)])
def test_streaming_encoder_24_steps_against_oracle(dtype, steps):
    """Two cache-aware blocks (causal conv kernel 9 with LayerNorm, d_model
    512, 4 heads, ff 2048) streamed chunks of 14 frames for 3 sessions with
    per-session fills (0, 33, 70) against a 70-frame cache under the
    [70, 13] chunked_limited context: every step's output against the
    oracle's conformer_block_with_cache run per session on its own state
    (end to end), and both caches read back at the end. fp32 blocks for 24
    steps; bf16 blocks for 8, where the streamed activations stay f32 and
    every op is f32 on the bf16 parameter values (conformer.rs:845-849), and
    the bf16 position rows the layer projects are handed to the oracle (the
    GPU rounds its fp32 sum, the oracle the exact one: an element within
    accumulation noise of a rounding boundary may differ by one ulp, which
    test_streaming_bf16_layer_xl_shape checks on its own)."""
    d, h, f, k = 512, 4, 2048, 9
    B, C, T = 3, 70, 14
    ctx = ((70, 13), "chunked_limited")
    rng = np.random.default_rng(74)
    ws = [block_weights(rng, d, h, f, k, "layer_norm", False, prefix=f"l{i}") for i in range(2)]
    ps = [block_oracle(w, d, h, "layer_norm", True, prefix=f"l{i}") for i, w in enumerate(ws)]
    blks = [gpu_block(w, d, h, f, k, "layer_norm", True, dtype, prefix=f"l{i}") for i, w in enumerate(ws)]
    enc = M.StreamingEncoder(blks, B, C, T)
    fills = [0, 33, 70]
    att = rng.standard_normal((2, B, C, d)) * 0.5
    for b in range(B):
        att[:, b, :C - fills[b]] = 0.0
    conv = rng.standard_normal((2, B, d, k - 1)) * 0.5
    enc.load_cache(dev(att, O.F32), dev(conv, O.F32), fills)
    state = [[(att[l, b:b + 1], conv[l, b:b + 1]) for l in range(2)] for b in range(B)]
    pos = O.to_dtype(O.RelPositionalEncoding(d, 5000, True).get_encoding(C + T), dtype)
    pos_d = dev(pos, dtype)
    rows = [_layer_pos_rows(blk, pos_d) if dtype == O.BF16 else None for blk in blks]
    worst = 0.0
    for step in range(steps):
        x = rng.standard_normal((B, T, d))
        xd = dev(x, O.F32)
        enc.step_(xd, pos_d, M.StreamingMask(*ctx, None, [T] * B))
        got = host(xd)
        for b in range(B):
            m = O.streaming_mask(ctx[0], ctx[1], C, fills[b], T, T)
            y = x[b:b + 1].astype(np.float32).astype(np.float64)
            for l in range(2):
                a_c, c_c = state[b][l]
                y, a_c, c_c = O.conformer_block_with_cache(ps[l], y, pos, a_c, c_c, m, None, dtype, rows[l])
                state[b][l] = (a_c, c_c)
            e = row_rel_err(got[b:b + 1], y)
            worst = max(worst, e)
            assert e < F32_TOL, (step, b, e)
            fills[b] = O.next_fill(fills[b], T, 0, C)
        assert enc.fill() == fills
    ch, tm = enc.read_cache()
    ch, tm = host(ch), host(tm)
    for b in range(B):
        for l in range(2):
            assert row_rel_err(ch[l, b:b + 1], state[b][l][0]) < F32_TOL
            assert row_rel_err(np.swapaxes(tm[l, b:b + 1], 1, 2), np.swapaxes(state[b][l][1], 1, 2)) < F32_TOL
    print(f"streaming encoder ({dtype}), 2 blocks x {steps} steps x {B} sessions: worst per-row error / row max "
          f"{worst:.3e}")


def test_streaming_encoder_valid_frames_against_oracle():
    """Chunks whose sessions end early: per step and session a valid frame
    count below the chunk (the last chunk of an utterance). The attention
    hides every key from rows at or past it (the bool mask: those rows give 0
    before linear_out, attention.rs:774-790) and the conv zeroes the GLU
    frames past it (pad_mask, conformer.rs:929-941), per session here where
    the reference uses session 0's count for all. Two fp32 blocks, 6 steps,
    against the oracle per session."""
    d, h, f, k = 512, 4, 2048, 9
    B, C, T = 3, 70, 14
    ctx = ((70, 13), "chunked_limited")
    valids = [[14, 9, 1], [14, 14, 5], [7, 14, 14], [0, 3, 14], [14, 13, 2], [11, 14, 14]]
    rng = np.random.default_rng(76)
    ws = [block_weights(rng, d, h, f, k, "layer_norm", False, prefix=f"l{i}") for i in range(2)]
    ps = [block_oracle(w, d, h, "layer_norm", True, prefix=f"l{i}") for i, w in enumerate(ws)]
    blks = [gpu_block(w, d, h, f, k, "layer_norm", True, O.F32, prefix=f"l{i}") for i, w in enumerate(ws)]
    enc = M.StreamingEncoder(blks, B, C, T)
    fills = [0, 33, 70]
    att = rng.standard_normal((2, B, C, d)) * 0.5
    for b in range(B):
        att[:, b, :C - fills[b]] = 0.0
    conv = rng.standard_normal((2, B, d, k - 1)) * 0.5
    enc.load_cache(dev(att, O.F32), dev(conv, O.F32), fills)
    state = [[(att[l, b:b + 1], conv[l, b:b + 1]) for l in range(2)] for b in range(B)]
    pos = O.RelPositionalEncoding(d, 5000, True).get_encoding(C + T)
    pos_d = dev(pos, O.F32)
    worst = 0.0
    for step, valid in enumerate(valids):
        x = rng.standard_normal((B, T, d))
        xd = dev(x, O.F32)
        enc.step_(xd, pos_d, M.StreamingMask(*ctx, None, valid), valid)
        got = host(xd)
        for b in range(B):
            m = O.streaming_mask(ctx[0], ctx[1], C, fills[b], T, valid[b])
            y = x[b:b + 1].astype(np.float32).astype(np.float64)
            for l in range(2):
                a_c, c_c = state[b][l]
                y, a_c, c_c = O.conformer_block_with_cache(ps[l], y, pos, a_c, c_c, m, [valid[b]], O.F32)
                state[b][l] = (a_c, c_c)
            e = row_rel_err(got[b:b + 1], y)
            worst = max(worst, e)
            assert e < F32_TOL, (step, b, valid[b], e)
            fills[b] = O.next_fill(fills[b], T, 0, C)
        assert enc.fill() == fills
    print(f"streaming encoder with valid frame counts: worst per-row error / row max {worst:.3e}")
