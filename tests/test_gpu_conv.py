"""GPU parity of the ConvolutionModule (conformer.rs:2105-2437) against the
oracle: the pointwise convs on the projection GEMMs and the fused GLU /
depthwise / BatchNorm / SiLU kernel (LayerNorm after it), offline and with
the streaming conv cache.

Tolerances: per output row, max |gpu - oracle| / max |oracle| <= 1e-4 where
the activations are f32 (f32 modules, and every streaming call, whose
activations are f32 in a bf16 module too); <= 2e-2 where pointwise_conv1 and
the GLU run in bf16 (a bf16 module offline): their results are rounded to
bf16 and a GEMM summed in another order flips an occasional ulp (0.4%). The
new conv cache is compared within the same f32 bound per entry.
"""
import numpy as np
import pytest
import torch

import relpos_oracle as O
import relpos_mhsa as M
from _util import conv_oracle, conv_weights, row_rel_err

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
    t = torch.from_numpy(np.ascontiguousarray(np.asarray(a, dtype=np.float32))).to("cuda")
    return t if dtype == O.F32 else t.to(torch.bfloat16).contiguous()


def host(t):
    return t.float().cpu().numpy().astype(np.float64)


def _module(w, d, k, norm, causal, dtype):
    m = M.ConvolutionModule(d, k, norm, causal=causal)
    m.load_weights(w, "conv")
    m.set_dtype(dtype)
    return m


def _input(rng, shape, dtype):
    x = rng.standard_normal(shape)
    return O.bf16_round(x) if dtype == O.BF16 else x.astype(np.float32).astype(np.float64)


@pytest.mark.parametrize("dtype,norm,causal,k,quant,B,T,d,lengths", [
    (O.F32, "batch_norm", False, 31, False, 2, 150, 256, [150, 97]),
    (O.BF16, "batch_norm", False, 31, True, 4, 375, 1024, None),
    (O.BF16, "layer_norm", True, 9, False, 2, 70, 512, [70, 33]),
    (O.F32, "layer_norm", True, 9, True, 3, 17, 512, None),
    (O.F32, "batch_norm", False, 1, False, 1, 5, 64, [3]),
    (O.F32, "batch_norm", False, 3, False, 70, 4, 64, list(range(70))),
])
def test_conv_forward_against_oracle(dtype, norm, causal, k, quant, B, T, d, lengths):
    """Offline forward: symmetric and causal windows, frames past the lengths
    zeroed after the GLU, several frame tiles per item (T > 64), K = 1, more
    items than one launch's batch chunk (70 > 64), u8 pointwise convs. A
    causal bf16 module returns f32 (MLX promotion at the f32 padding)."""
    rng = np.random.default_rng(1000 + k + T)
    w = conv_weights(rng, d, k, norm, quant)
    p = conv_oracle(w, norm, causal)
    m = _module(w, d, k, norm, causal, dtype)
    x = _input(rng, (B, T, d), dtype)
    print(f"conv forward {dtype} {norm} causal={causal} K={k} quant={quant} B={B} T={T} D={d}", flush=True)
    out = m.forward(dev(x, dtype), lengths)
    assert out.dtype == (torch.float32 if causal or dtype == O.F32 else torch.bfloat16)
    ref, _ = O.conv_module(p, x, dtype, lengths=lengths)
    err = row_rel_err(host(out), ref)
    print(f"  per-row error {err:.3e} (max |ref| {np.max(np.abs(ref)):.2f})")
    assert err < (BF16_TOL if dtype == O.BF16 else F32_TOL)


@pytest.mark.parametrize("dtype,norm,quant,B,chunk,d", [
    (O.BF16, "layer_norm", True, 16, 14, 1024),
    (O.F32, "batch_norm", False, 4, 5, 256),
    (O.BF16, "batch_norm", False, 2, 100, 512),
    (O.F32, "layer_norm", False, 70, 3, 128),
])
def test_conv_streaming_cache_against_oracle(dtype, norm, quant, B, chunk, d):
    """forward_with_cache over consecutive chunks (K = 9, cache [B, D, 8]
    f32, updated in place): each chunk's output and the cache after it match
    the oracle; the last chunk has ragged lengths (padding frames zeroed
    before they reach the cache). Chunks of 14 (the streaming shape) and 5
    (< K - 1, so part of the old cache stays) update in place from one frame
    tile; 100 frames span two tiles and read a copy of the cache; 70 sessions
    take two launches' batch chunks, each with its own cache slice."""
    rng = np.random.default_rng(2000 + chunk)
    k = 9
    w = conv_weights(rng, d, k, norm, quant)
    p = conv_oracle(w, norm, True)
    m = _module(w, d, k, norm, True, dtype)
    cache_ref = np.zeros((B, d, k - 1))
    cache = torch.zeros((B, d, k - 1), dtype=torch.float32, device="cuda")
    for step in range(4):
        lengths = None if step < 3 else [chunk - (b % 3) for b in range(B)]
        x = rng.standard_normal((B, chunk, d)).astype(np.float32).astype(np.float64)
        print(f"conv stream {dtype} {norm} quant={quant} B={B} chunk={chunk} step={step}", flush=True)
        out, _ = m.forward_with_cache(dev(x, O.F32), cache, lengths)
        ref, cache_ref = O.conv_module(p, x, dtype, act=O.F32, lengths=lengths, cache=cache_ref)
        err = row_rel_err(host(out), ref)
        cerr = np.max(np.abs(host(cache) - cache_ref)) / max(np.max(np.abs(cache_ref)), 1e-30)
        print(f"  per-row error {err:.3e}, cache error {cerr:.3e}")
        assert err < F32_TOL and cerr < F32_TOL
    # the no-cache path of forward_with_cache: zero left padding, f32
    x = rng.standard_normal((B, chunk, d)).astype(np.float32).astype(np.float64)
    out, _ = m.forward_with_cache(dev(x, O.F32), None)
    ref, _ = O.conv_module(p, x, dtype, act=O.F32)
    assert row_rel_err(host(out), ref) < F32_TOL


@pytest.mark.parametrize("dtype,causal,stream", [(O.F32, False, False), (O.BF16, False, False),
                                                 (O.BF16, True, True)])
def test_conv_sublayer_against_oracle(dtype, causal, stream):
    """The block's convolution sublayer x + conv(LayerNorm(x)), residual fused
    into pointwise_conv2: offline in the module dtype, or streaming (f32 x
    with the cache). A causal bf16 module cannot run it offline in place (its
    f32 result does not fit the bf16 input): MHSA_ENOTSUP."""
    rng = np.random.default_rng(3000)
    d, k, B, T = 512, 9 if causal else 15, 3, 40
    w = conv_weights(rng, d, k, "batch_norm", False)
    p = conv_oracle(w, "batch_norm", causal)
    m = _module(w, d, k, "batch_norm", causal, dtype)
    gamma = rng.uniform(0.5, 1.5, d).astype(np.float32)
    beta = rng.normal(0, 0.1, d).astype(np.float32)
    act = O.F32 if stream else dtype
    x = _input(rng, (B, T, d), act)
    lengths = [T, T - 7, 1]
    if stream:
        c0 = rng.normal(0, 0.5, (B, d, k - 1)).astype(np.float32)
        cache = torch.from_numpy(c0).cuda()
        xd = dev(x, O.F32)
        m.sublayer_forward_(xd, gamma, beta, cache=cache, lengths=lengths)
        ref, cref = O.conv_sublayer(p, x, gamma, beta, dtype, act=O.F32, lengths=lengths,
                                    cache=c0.astype(np.float64))
        assert np.max(np.abs(host(cache) - cref)) / np.max(np.abs(cref)) < F32_TOL
        with pytest.raises(M.MhsaError) as e:
            m.sublayer_forward_(dev(x, dtype), gamma, beta)
        assert e.value.code == M.MHSA_ENOTSUP
    else:
        xd = dev(x, dtype)
        m.sublayer_forward_(xd, gamma, beta, lengths=lengths)
        ref, _ = O.conv_sublayer(p, x, gamma, beta, dtype, lengths=lengths)
    err = row_rel_err(host(xd), ref)
    print(f"conv sublayer {dtype} causal={causal} stream={stream}: per-row error {err:.3e}")
    assert err < (BF16_TOL if act == O.BF16 else F32_TOL)


def test_conv_cache_needs_causal_module():
    rng = np.random.default_rng(4000)
    w = conv_weights(rng, 128, 9, "batch_norm", False)
    m = _module(w, 128, 9, "batch_norm", False, O.F32)
    x = dev(rng.standard_normal((2, 14, 128)), O.F32)
    cache = torch.zeros((2, 128, 8), device="cuda")
    with pytest.raises(M.MhsaError) as e:
        m.forward_with_cache(x, cache)
    assert e.value.code == M.MHSA_EINVAL
