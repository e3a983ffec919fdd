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
