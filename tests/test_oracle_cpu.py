"""The fp32 C++ restatement (the bench's CPU baseline) agrees with the numpy
oracle on small shapes with contexts and padding, so the timed baseline
computes the same function as the reference algorithm."""
import numpy as np
import pytest

import cpu_ref
import relpos_oracle as O
from _util import oracle_params, random_weights, rel_err


@pytest.mark.parametrize("ctx", [None, (4, 1, True), (3, 2, False), (-1, 2, True)])
def test_cpu_restatement_matches_oracle(ctx):
    rng = np.random.default_rng(2)
    d, h, B, T = 64, 2, 3, 29
    w = random_weights(rng, d, h, scale=0.15)
    x = rng.standard_normal((B, T, d)).astype(np.float32)
    pos = O.RelPositionalEncoding(d, 100, False).get_encoding(T)
    lengths = [29, 17, 3]
    got = cpu_ref.forward(w, h, x, pos, ctx, lengths)
    octx = None if ctx is None else O.AttentionContext.new((ctx[0], ctx[1]), "chunked_limited" if ctx[2] else "regular")
    ref = O.mhsa_forward(oracle_params(w, d, h), x, pos, octx, O.key_padding_mask(lengths, T))
    rows = np.ones((B, T), dtype=bool)
    for b in range(B):
        m = octx.block_visible(0, T, T) if octx else np.ones((T, T), dtype=bool)
        rows[b] = (m & (np.arange(T)[None, :] < lengths[b])).any(axis=1)
    assert rel_err(got, ref, rows) < 1e-5


def test_cpu_restatement_blocks_like_the_reference():
    # T large enough that query_block_size splits the queries into blocks
    rng = np.random.default_rng(3)
    d, h, B, T = 64, 4, 2, 2100
    assert O.query_block_size(B * h, T, O.MAX_SCORE_ELEMENTS) < T
    w = random_weights(rng, d, h, scale=0.1)
    x = rng.standard_normal((B, T, d)).astype(np.float32)
    pos = O.RelPositionalEncoding(d, 5000, False).get_encoding(T)
    got = cpu_ref.forward(w, h, x, pos, (16, 16, False))
    ref = O.mhsa_forward(oracle_params(w, d, h), x, pos, O.AttentionContext.new((16, 16), "regular"))
    assert rel_err(got, ref) < 1e-5


# ---------------------------------------------------------------------------
# the BLAS-backed float32 restatement the bench times (oracle/cpu_blas.py)
# ---------------------------------------------------------------------------

import cpu_blas  # noqa: E402
import workloads as W  # noqa: E402


@pytest.mark.parametrize("ctx", [None, (4, 1, True), (3, 2, False)])
def test_cpu_blas_forward_matches_oracle(ctx):
    rng = np.random.default_rng(4)
    d, h, B, T = 64, 2, 3, 29
    w = random_weights(rng, d, h, scale=0.15)
    x = rng.standard_normal((B, T, d)).astype(np.float32)
    pos = O.RelPositionalEncoding(d, 100, False).get_encoding(T)
    lengths = [29, 17, 3]
    got = cpu_blas.forward(cpu_blas.layer_params(w), h, x, pos[0], ctx, lengths)
    octx = None if ctx is None else O.AttentionContext.new((ctx[0], ctx[1]), "chunked_limited" if ctx[2] else "regular")
    ref = O.mhsa_forward(oracle_params(w, d, h), x, pos, octx, O.key_padding_mask(lengths, T))
    rows = np.ones((B, T), dtype=bool)
    for b in range(B):
        m = octx.block_visible(0, T, T) if octx else np.ones((T, T), dtype=bool)
        rows[b] = (m & (np.arange(T)[None, :] < lengths[b])).any(axis=1)
    assert rel_err(got, ref, rows) < 1e-5


def test_cpu_blas_quantized_sublayer_blocks_match_oracle():
    rng = np.random.default_rng(5)
    d, h, B, T = 128, 8, 2, 1500
    assert O.query_block_size(B * h, T, O.MAX_SCORE_ELEMENTS) < T
    w = W.make_layer_weights(rng, d, h, False, True, centred=True)
    x = rng.standard_normal((B, T, d)).astype(np.float32)
    pos = O.RelPositionalEncoding(d, 5000, False).get_encoding(T)
    got = cpu_blas.sublayer(cpu_blas.layer_params(w), h, x, pos[0], None, [T, 1200])
    ref = O.mhsa_sublayer(oracle_params(w, d, h), x, pos, None, O.key_padding_mask([T, 1200], T))
    assert rel_err(got, ref) < 1e-4


def test_cpu_blas_streaming_matches_oracle():
    rng = np.random.default_rng(6)
    d, h, B, C, T = 128, 2, 2, 20, 6
    w = random_weights(rng, d, h, scale=0.1)
    p = oracle_params(w, d, h)
    cache = rng.standard_normal((B, C, d)).astype(np.float32)
    filled = 11
    cache[:, :C - filled] = 0.0
    pos = O.RelPositionalEncoding(d, 5000, False).get_encoding(C + T)
    st = cpu_blas.Streamer(cpu_blas.layer_params(w), h, cache, pos[0], (12, 5, True))
    caches = cache.astype(np.float64)
    for step in range(3):
        x = rng.standard_normal((B, T, d)).astype(np.float32)
        got = st.step(x, filled)
        mask = O.streaming_mask((12, 5), "chunked_limited", C, filled, T, T)
        ref, caches = O.mhsa_forward_with_cache(p, x, pos, caches, mask)
        assert rel_err(got, ref) < 1e-5, step
        filled = O.next_fill(filled, T, 0, C)


@pytest.mark.parametrize("norm,causal,stream,quant,bf", [("batch_norm", False, False, False, False),
                                                         ("batch_norm", False, False, True, True),
                                                         ("layer_norm", True, True, False, False),
                                                         ("layer_norm", True, False, True, True)])
def test_cpu_blas_conv_module_matches_oracle(norm, causal, stream, quant, bf):
    """The baseline's ConvolutionModule against the float64 oracle: f32
    activations on the module's (bf16-valued when bf) parameters, offline
    with ragged lengths and streaming over two chunks through the cache."""
    from _util import conv_oracle
    rng = np.random.default_rng(77)
    d, k = 128, 9
    w = W.make_conv_weights(rng, d, k, norm, quant)
    p = conv_oracle(w, norm, causal)
    P = cpu_blas.conv_params(w, bf)
    dt = O.BF16 if bf else O.F32
    x = rng.standard_normal((3, 20, d)).astype(np.float32)
    lens = [20, 13, 2]
    if stream:
        c_ref = np.zeros((3, d, k - 1))
        c = c_ref.astype(np.float32)
        for _ in range(2):
            got, c = cpu_blas.conv_module(P, x, lens, c, causal)
            ref, c_ref = O.conv_module(p, x, dt, act=O.F32, lengths=lens, cache=c_ref)
            assert rel_err(got, ref) < 1e-4 and rel_err(c, c_ref) < 1e-4
    else:
        got, _ = cpu_blas.conv_module(P, x, lens, None, causal)
        ref, _ = O.conv_module(p, x, dt, act=O.F32, lengths=lens)
        assert rel_err(got, ref) < 1e-4
