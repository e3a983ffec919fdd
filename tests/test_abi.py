"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/relpos_mhsa.h declares, and its host-side logic (argument checks,
strict/lenient weight loading as loading.rs:107-116, the position table of
attention.rs:59-177) behaves like the reference. No kernel is launched here.
"""
import ctypes
import os
import re

import numpy as np
import pytest

import relpos_oracle as O
import relpos_mhsa as M
import workloads as W


@pytest.fixture(scope="module")
def lib():
    return M.library()


def declared_functions(repo_root):
    text = open(os.path.join(repo_root, "include", "relpos_mhsa.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mhsa_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported(lib, repo_root):
    names = declared_functions(repo_root)
    assert len(names) >= 25
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(M.EXPORTS) == names


def test_version_and_error_message(lib):
    assert lib.mhsa_version() == 100
    h = ctypes.c_void_p()
    assert lib.mhsa_create(100, 8, 1, ctypes.byref(h)) == M.MHSA_EINVAL
    assert b"multiple of n_heads" in lib.mhsa_last_error()
    assert lib.mhsa_create(512, 16, 1, ctypes.byref(h)) == M.MHSA_ENOTSUP  # head_dim 32
    assert lib.mhsa_create(512, 8, 1, None) == M.MHSA_EINVAL


def test_layer_accessors_and_dtype(lib):
    layer = M.RelPositionMultiHeadAttention(1024, 8, False)
    assert layer.head_dim() == 128 and layer.n_heads() == 8
    layer.set_dtype("bfloat16")
    import torch
    assert layer.dtype == torch.bfloat16
    with pytest.raises(M.MhsaError) as e:
        layer.set_dtype("float16")
    assert e.value.code == M.MHSA_ENOTSUP
    layer.cache_drop_size = 3
    assert layer.cache_drop_size == 3


def test_stack_sublayer_forward_argument_checks(lib):
    """The offline stack rejects an empty layer list and layers of different
    d_model before touching any tensor."""
    a = M.RelPositionMultiHeadAttention(512, 8, False)
    b = M.RelPositionMultiHeadAttention(1024, 8, False)
    arr = (ctypes.c_void_p * 2)(a._h.value, b._h.value)
    assert lib.mhsa_stack_sublayer_forward(arr, 0, None, 1, 1, None, None, 1e-5, None, 1, None, None, None) == \
        M.MHSA_EINVAL
    assert lib.mhsa_stack_sublayer_forward(arr, 2, None, 1, 1, None, None, 1e-5, None, 1, None, None, None) == \
        M.MHSA_EINVAL
    assert b"layer 1 has d_model 1024" in lib.mhsa_last_error()
    with pytest.raises(M.MhsaError):
        M.stack_sublayer_forward_([], np.zeros((1, 1, 512), np.float32), np.zeros((1, 512), np.float32))


def test_load_weights_strict_and_lenient():
    rng = np.random.default_rng(0)
    w = W.make_layer_weights(rng, 128, 2, True, False)
    full = W.prefixed(w, "encoder.layers.0.self_attn")
    layer = M.RelPositionMultiHeadAttention(128, 2, True)
    layer.load_weights(full, "encoder.layers.0.self_attn")
    partial = {k: v for k, v in full.items() if "linear_v" not in k}
    with pytest.raises(M.MhsaError) as e:
        layer.load_weights(partial, "encoder.layers.0.self_attn")
    assert e.value.code == M.MHSA_ENOENT and "linear_v.weight" in str(e.value)
    layer.load_weights(partial, "encoder.layers.0.self_attn", strict=False)
    bad = dict(full)
    bad["encoder.layers.0.self_attn.linear_q.weight"] = np.zeros((128, 64), np.float32)
    with pytest.raises(M.MhsaError) as e:
        layer.load_weights(bad, "encoder.layers.0.self_attn")
    assert e.value.code == M.MHSA_EINVAL


def test_load_weights_detects_quantization():
    rng = np.random.default_rng(1)
    w = W.make_layer_weights(rng, 128, 2, False, True)
    layer = M.RelPositionMultiHeadAttention(128, 2, False)
    layer.load_weights(W.prefixed(w, "p"), "p")
    with pytest.raises(M.MhsaError) as e:
        layer.load_weights(W.prefixed(w, "p"), "p", quant=M.QuantizationConfig(4, 64))
    assert e.value.code == M.MHSA_ENOTSUP  # only 8-bit, group-64 layers have kernels
    q = {k: v for k, v in W.prefixed(w, "p").items()}
    ql = M.LinearLayer.quantized(q["p.linear_q.weight"], q["p.linear_q.scales"], q["p.linear_q.biases"], bits=4)
    with pytest.raises(M.MhsaError) as e:
        layer.set_linear("linear_q", ql)
    assert e.value.code == M.MHSA_ENOTSUP


def test_pos_encoding_matches_oracle():
    pe = M.RelPositionalEncoding(512, 5000, True)
    assert abs(pe.xscale() - np.sqrt(512.0)) < 1e-5
    for L in (1, 3, 84, 125):
        got = pe.get_encoding(L).numpy()
        ref = O.RelPositionalEncoding(512, 5000, True).get_encoding(L)
        assert got.shape == (1, 2 * L - 1, 512)
        # host f32 exp may differ by an ulp between libm builds; the
        # reference's own value test allows 1e-5 (attention.rs:1169-1246)
        assert np.max(np.abs(got - ref)) < 1e-5
    small = M.RelPositionalEncoding(4, 3, False).get_encoding(3).numpy().reshape(-1)
    d1 = np.exp(-2.0 * np.log(10000.0) / 4.0)
    assert abs(small[0] - np.sin(2.0)) < 1e-6 and abs(small[3] - np.cos(2 * d1)) < 1e-6
    assert abs(small[8]) < 1e-7 and abs(small[9] - 1.0) < 1e-7
    # past max_len: regenerated table equals a larger precomputed one (attention.rs:1150-1167)
    a = M.RelPositionalEncoding(16, 10, False).get_encoding(25).numpy()
    b = M.RelPositionalEncoding(16, 40, False).get_encoding(25).numpy()
    assert np.array_equal(a, b)
    with pytest.raises(M.MhsaError):
        pe.get_encoding(0)


def test_key_padding_and_context_helpers():
    assert M.key_padding_mask([13, 13], 13) is None
    assert M.key_padding_mask([13, 9, 0], 13) == (13, 9, 1)
    assert M.AttentionContext.new((-1, -1), "chunked_limited") is None
    c = M.AttentionContext.new((70, 13), "chunked_limited")
    assert c.chunked and (c.left, c.right) == (70, 13)
