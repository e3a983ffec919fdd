"""Host logic of the ConformerBlock and streaming-encoder C ABI
(mhsa_block_*, mhsa_encoder_*), no GPU needed: construction limits, weight
loading as ConformerBlock::load_weights defines it (conformer.rs:1977-2028:
the four modules under their names, the five LayerNorms optional), and the
encoder's checks of its blocks (conformer.rs:840-1047 streams causal convs
only). Numerics are the GPU tests' job."""
import ctypes

import numpy as np
import pytest

import relpos_mhsa as M
import workloads as W

D, H, F, K = 128, 2, 256, 9


def block_weights(rng, norm="batch_norm", prefix="blk"):
    return W.make_block_weights(rng, D, H, F, K, norm, prefix)


def test_create_limits():
    for args, code in (((100, 2, F, K), M.MHSA_EINVAL),      # d_model % n_heads / head_dim
                       ((128, 2, F, 0), M.MHSA_EINVAL),      # conv kernel 0
                       ((128, 2, F, 8), M.MHSA_EINVAL),      # even symmetric conv kernel
                       ((4096, 8, F, K), M.MHSA_ENOTSUP)):   # LayerNorms up to d_model 2048
        with pytest.raises(M.MhsaError) as e:
            M.ConformerBlock(*args)
        assert e.value.code == code, args
    lib = M.library()
    assert lib.mhsa_block_create(D, H, F, K, M.CONV_BATCH_NORM, 0, 1, None) == M.MHSA_EINVAL
    blk = M.ConformerBlock(D, H, F, K)
    for which in (0, 3):
        assert not lib.mhsa_block_feed_forward(blk._h, which)
    assert lib.mhsa_block_feed_forward(blk._h, 1) and lib.mhsa_block_feed_forward(blk._h, 2)
    assert lib.mhsa_block_attention(blk._h) and lib.mhsa_block_conv(blk._h)
    assert not lib.mhsa_block_attention(None)
    with pytest.raises(M.MhsaError) as e:
        blk.set_dtype("float16")
    assert e.value.code == M.MHSA_ENOTSUP
    blk.set_dtype("bfloat16")


def test_load_weights_modules_and_norms():
    rng = np.random.default_rng(0)
    w = block_weights(rng)
    blk = M.ConformerBlock(D, H, F, K)
    blk.load_weights(w, "blk")
    # the LayerNorms are optional (each defaults to weight 1, bias 0)
    no_norms = {k: v for k, v in w.items() if ".norm_" not in k}
    blk.load_weights(no_norms, "blk")
    # a module weight is not: strict loading names the missing key
    for key in ("blk.feed_forward1.linear1.weight", "blk.self_attn.linear_q.weight",
                "blk.conv.depthwise_conv.weight", "blk.feed_forward2.linear2.weight"):
        part = dict(w)
        del part[key]
        with pytest.raises(M.MhsaError) as e:
            blk.load_weights(part, "blk")
        assert key in str(e.value)
    # a linear's bias is optional, as the reference's loader reads it
    # (quantization.rs:296-306: `weights.get(bias_key)`)
    part = dict(w)
    del part["blk.feed_forward2.linear2.bias"]
    blk.load_weights(part, "blk")
    # a norm of the wrong length is rejected
    bad = dict(w)
    bad["blk.norm_out.weight"] = np.ones(D + 1, np.float32)
    with pytest.raises(M.MhsaError):
        blk.load_weights(bad, "blk")
    # another prefix finds nothing
    with pytest.raises(M.MhsaError):
        blk.load_weights(w, "encoder.layers.0")


def test_encoder_checks_its_blocks():
    lib = M.library()
    causal = M.ConformerBlock(D, H, F, K, "layer_norm", causal=True)
    causal2 = M.ConformerBlock(D, H, F, K, "layer_norm", causal=True)
    symmetric = M.ConformerBlock(D, H, F, K, "batch_norm", causal=False)
    other_k = M.ConformerBlock(D, H, F, 5, "layer_norm", causal=True)
    other_d = M.ConformerBlock(2 * D, H, F, K, "layer_norm", causal=True)

    def create(blocks, batch=2, cache=8, chunk=4):
        arr = (ctypes.c_void_p * max(len(blocks), 1))(*[b._h.value if b else None for b in blocks])
        h = ctypes.c_void_p()
        return lib.mhsa_encoder_create(arr, len(blocks), batch, cache, chunk, ctypes.byref(h))

    assert create([]) == M.MHSA_EINVAL
    assert create([symmetric]) == M.MHSA_EINVAL
    assert b"causal convolution" in lib.mhsa_last_error()
    assert create([causal, symmetric]) == M.MHSA_EINVAL
    assert create([causal, other_k]) == M.MHSA_EINVAL
    assert b"differs from block 0" in lib.mhsa_last_error()
    assert create([causal, other_d]) == M.MHSA_EINVAL
    assert create([causal, causal2, causal]) == M.MHSA_EINVAL
    assert b"appears twice" in lib.mhsa_last_error()
    assert create([causal, None]) == M.MHSA_EINVAL
    assert b"block 1 is null" in lib.mhsa_last_error()
    for shape in ((0, 8, 4), (2, -1, 4), (2, 8, 0)):
        assert create([causal, causal2], *shape) == M.MHSA_EINVAL, shape
        assert b"bad encoder shape" in lib.mhsa_last_error()
    h = ctypes.c_void_p()
    assert lib.mhsa_encoder_create(None, 1, 2, 8, 4, ctypes.byref(h)) == M.MHSA_EINVAL
    arr = (ctypes.c_void_p * 1)(causal._h.value)
    assert lib.mhsa_encoder_create(arr, 1, 2, 8, 4, None) == M.MHSA_EINVAL


def test_forward_to_dtypes_and_argument_checks():
    """mhsa_block_output_dtype: f32 once the activations are f32 or the conv
    is causal (its f32 zero padding promotes a bf16 block,
    conformer.rs:2250-2256), else the block dtype; bf16 activations into an
    f32 block are not a case. mhsa_block_forward_to and
    mhsa_encoder_forward_to reject bad arguments before any device work
    (the addresses below are never dereferenced)."""
    lib = M.library()
    sym = M.ConformerBlock(D, H, F, K, "batch_norm", causal=False)
    cau = M.ConformerBlock(D, H, F, K, "layer_norm", causal=True)
    for blk in (sym, cau):
        assert lib.mhsa_block_output_dtype(blk._h, M.F32) == M.F32
        assert lib.mhsa_block_output_dtype(blk._h, M.BF16) == -1
    sym.set_dtype("bfloat16")
    cau.set_dtype("bfloat16")
    assert lib.mhsa_block_output_dtype(sym._h, M.BF16) == M.BF16
    assert lib.mhsa_block_output_dtype(cau._h, M.BF16) == M.F32
    assert lib.mhsa_block_output_dtype(sym._h, M.F32) == M.F32
    assert lib.mhsa_block_output_dtype(cau._h, M.F32) == M.F32
    assert lib.mhsa_block_output_dtype(None, M.F32) == -1
    assert lib.mhsa_block_output_dtype(sym._h, 7) == -1
    import torch
    assert cau.output_dtype(torch.bfloat16) == torch.float32 and sym.output_dtype("bfloat16") == torch.bfloat16

    x, o, pe = ctypes.c_void_p(1 << 20), ctypes.c_void_p(2 << 20), ctypes.c_void_p(3 << 20)

    def fwd(blk, xp, dt, out, b=2, t=8):
        return lib.mhsa_block_forward_to(blk._h, xp, dt, b, t, pe, 2 * t - 1, None, None, out, None)

    f32blk = M.ConformerBlock(D, H, F, K)
    assert fwd(sym, x, 7, o) == M.MHSA_EINVAL  # not a dtype
    assert fwd(f32blk, x, M.BF16, o) == M.MHSA_EINVAL  # bf16 activations in an f32 block
    assert fwd(cau, x, M.BF16, x) == M.MHSA_EINVAL  # the f32 result over its bf16 input
    assert b"overlap" in lib.mhsa_last_error()
    assert fwd(cau, x, M.BF16, ctypes.c_void_p((1 << 20) + 2 * 8 * D)) == M.MHSA_EINVAL  # partly overlapping
    assert fwd(sym, x, M.BF16, ctypes.c_void_p((1 << 20) + 2 * 8 * D)) == M.MHSA_EINVAL  # the same, one dtype
    assert fwd(cau, ctypes.c_void_p((1 << 20) + 8), M.BF16, o) == M.MHSA_EINVAL  # misaligned
    assert fwd(sym, x, M.BF16, o, b=0) == M.MHSA_EINVAL
    assert lib.mhsa_block_forward_to(None, x, M.F32, 2, 8, pe, 15, None, None, o, None) == M.MHSA_EINVAL
    # the encoder checks its blocks and follows the dtype through them first
    enc = lambda blocks, dt: lib.mhsa_encoder_forward_to((ctypes.c_void_p * len(blocks))(*[k._h.value for k in blocks]),
                                                       len(blocks), x, dt, 2, 8, pe, 15, None, None, o, None)
    assert enc([f32blk, cau], M.F32) == M.MHSA_EINVAL  # dtypes differ
    assert b"differs from block 0" in lib.mhsa_last_error()
    assert enc([cau, sym], 7) == M.MHSA_EINVAL
    assert lib.mhsa_encoder_forward_to(None, 1, x, M.BF16, 2, 8, pe, 15, None, None, o, None) == M.MHSA_EINVAL
