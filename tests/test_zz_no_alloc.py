"""The allocation-free forward (mhsa_forward_noalloc) against mhsa_forward.

Both run the same kernels with the same tile and split choices, so their
outputs must be identical bit for bit. Each case makes two calls in a row,
the second on a smaller input (the fixed scratch keeps the first call's
contents, which must not leak into the second), and checks that an input
needing more workspace than the scratch holds, or a layer whose weights
have not been uploaded yet, is rejected with an error.
"""
import numpy as np
import pytest
import torch

import relpos_oracle as O
import relpos_mhsa as M
import workloads as W
from _util import random_weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    M.library()
    yield
    torch.cuda.synchronize()


def _case(layer, rng, B, T, D, tdt, ctx, lengths):
    x = torch.from_numpy(rng.standard_normal((B, T, D)).astype(np.float32)).cuda().to(tdt)
    pos = M.RelPositionalEncoding(D, 5000, True).get_encoding(T).cuda().to(tdt).contiguous()
    km = M.key_padding_mask(lengths, T) if lengths else None
    ref = layer.forward(x, pos, ctx, km)
    out = torch.full_like(x, float("nan"))
    layer.forward_noalloc(x, pos, out, ctx, km)
    torch.cuda.synchronize()
    return ref, out


@pytest.mark.parametrize("dtype", [O.BF16, O.F32])
def test_noalloc_forward_equals_forward_two_calls(dtype):
    rng = np.random.default_rng(61)
    D, H = 1024, 8
    w = random_weights(rng, D, H, use_bias=True, scale=0.03)
    layer = M.RelPositionMultiHeadAttention(D, H, True)
    layer.load_weights(W.prefixed(w, "l"), "l")
    layer.set_dtype(dtype)
    tdt = torch.bfloat16 if dtype == O.BF16 else torch.float32
    # the 0.6B offline shape with key padding, then a smaller windowed input
    B, T = (8, 375) if dtype == O.BF16 else (1, 125)
    lens = [int(v) for v in rng.integers(T // 2, T + 1, size=B)]
    ref, out = _case(layer, rng, B, T, D, tdt, None, lens)
    assert torch.equal(ref, out)
    ref, out = _case(layer, rng, 2, 61, D, tdt, M.AttentionContext.new((8, 2), "regular"), [61, 40])
    assert torch.equal(ref, out)


def test_noalloc_rejects_oversized_input_and_stale_weights():
    rng = np.random.default_rng(62)
    D, H = 1024, 8
    w = random_weights(rng, D, H, use_bias=False, scale=0.03)
    layer = M.RelPositionMultiHeadAttention(D, H, False)
    layer.load_weights(W.prefixed(w, "l"), "l")
    layer.set_dtype(torch.bfloat16)
    x = torch.zeros((1, 16, D), dtype=torch.bfloat16, device="cuda")
    pos = M.RelPositionalEncoding(D, 5000, True).get_encoding(16).cuda().to(torch.bfloat16).contiguous()
    out = torch.empty_like(x)
    with pytest.raises(M.MhsaError) as e:  # parameters not uploaded yet
        layer.forward_noalloc(x, pos, out)
    assert e.value.code == M.MHSA_EINVAL
    layer.forward(x, pos)  # uploads
    layer.forward_noalloc(x, pos, out)
    T = 16000  # ~4 * 1024 * 16000 * 2 bytes of workspace: more than the scratch holds
    xl = torch.zeros((1, T, D), dtype=torch.bfloat16, device="cuda")
    pl = torch.zeros((2 * T - 1, D), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(M.MhsaError) as e:
        layer.forward_noalloc(xl, pl, torch.empty_like(xl))
    assert e.value.code == M.MHSA_EINVAL and "workspace" in str(e.value)
