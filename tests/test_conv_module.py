"""Host logic of the ConvolutionModule C ABI (mhsa_conv_*), no GPU needed:
construction limits, dtype rules and weight loading as ConvolutionModule
::new / ::load_weights define them (conformer.rs:2138-2193, 2389-2427,
loading.rs:192-254). Numerics are the GPU tests' job."""
import numpy as np
import pytest

import relpos_mhsa as M
from _util import conv_weights


def test_create_limits_and_dtypes():
    for args, code in (((100, 9, "batch_norm", False), M.MHSA_EINVAL),   # d_model % 64
                       ((128, 8, "batch_norm", False), M.MHSA_EINVAL),   # even K, symmetric
                       ((128, 0, "batch_norm", True), M.MHSA_EINVAL),
                       ((128, 131, "batch_norm", True), M.MHSA_EINVAL),  # K > 129
                       ((4096, 9, "layer_norm", True), M.MHSA_ENOTSUP),  # LayerNorm d_model > 2048
                       ((128, 9, "group_norm", True), M.MHSA_ENOTSUP)):
        with pytest.raises(M.MhsaError) as e:
            M.ConvolutionModule(*args)
        assert e.value.code == code, args
    import torch
    sym = M.ConvolutionModule(128, 31, "batch_norm", causal=False)
    cau = M.ConvolutionModule(128, 8, "layer_norm", causal=True)  # even K is fine causally
    assert (sym.cache_size(), cau.cache_size()) == (30, 7)
    for dt in ("float32", "bfloat16"):
        sym.set_dtype(dt)
        cau.set_dtype(dt)
        assert sym.output_dtype() == (torch.float32 if dt == "float32" else torch.bfloat16)
        assert cau.output_dtype() == torch.float32  # f32 causal padding promotes


def test_load_weights_keys_shapes_and_strictness():
    rng = np.random.default_rng(0)
    w = conv_weights(rng, 128, 9, "batch_norm", quant=False)
    conv = M.ConvolutionModule(128, 9, "batch_norm", causal=True)
    conv.load_weights(w, "conv")
    conv.load_weights(conv_weights(rng, 128, 9, "batch_norm", quant=True), "conv")  # u8 pointwise convs
    for key in ("conv.depthwise_conv.weight", "conv.batch_norm.running_var", "conv.pointwise_conv2.weight",
                "conv.depthwise_conv.bias"):
        part = {k: v for k, v in w.items() if k != key}
        with pytest.raises(M.MhsaError) as e:
            conv.load_weights(part, "conv")
        assert e.value.code == M.MHSA_ENOENT and key in str(e.value), key
        conv.load_weights(part, "conv", strict=False)  # lenient: the old value stays
    # a module without bias neither needs nor reads the depthwise bias
    nob = M.ConvolutionModule(128, 9, "batch_norm", causal=True, use_bias=False)
    nob.load_weights({k: v for k, v in w.items() if k != "conv.depthwise_conv.bias"}, "conv")
    # LayerNorm reads weight and bias under `batch_norm` and no running statistics
    ln = M.ConvolutionModule(128, 9, "layer_norm", causal=True)
    ln.load_weights({k: v for k, v in w.items() if "running" not in k}, "conv")
    for key, bad in (("conv.depthwise_conv.weight", np.zeros((128, 1, 9), np.float32)),  # PyTorch layout
                     ("conv.pointwise_conv1.weight", np.zeros((128, 128), np.float32)),
                     ("conv.batch_norm.weight", np.zeros(64, np.float32))):
        with pytest.raises(M.MhsaError) as e:
            conv.load_weights({**w, key: bad}, "conv")
        assert e.value.code == M.MHSA_EINVAL, key
    q = conv_weights(rng, 128, 9, "batch_norm", quant=True)
    with pytest.raises(M.MhsaError) as e:
        conv.load_weights(q, "conv", quant=M.QuantizationConfig(4, 64))
    assert e.value.code == M.MHSA_ENOTSUP
