"""The MLX safetensors checkpoint reader (mhsa_checkpoint_*), no GPU needed.

Fixtures are written here by the `safetensors` package (numpy and torch
writers, the latter for bf16) in the MLX 8-bit layout the reference loads
(u32-packed codes, f16 scales and biases, quantization.rs:1-8, 289-349) and
with the config files CheckpointLoader reads its quantization from
(checkpoint.rs:535-572, 613-621). The reader must return every tensor's
name, dtype, shape and bytes as written, find the weights and config in a
model directory (checkpoint.rs:694-753), reject malformed files, and load a
layer as mhsa_load_weights does.
"""
import ctypes
import json
import os
import struct

import numpy as np
import pytest

import relpos_mhsa as M
import workloads as W

PREFIX = "encoder.layers.0.self_attn"


def _layer_tensors(quantized, d=128, h=2, seed=0):
    rng = np.random.default_rng(seed)
    w = W.make_layer_weights(rng, d, h, True, quantized)
    for name in ("linear_q", "linear_k", "linear_v", "linear_out"):
        w[f"{name}.bias"] = rng.normal(0, 0.1, d).astype(np.float16 if quantized else np.float32)
    return {f"{PREFIX}.{k}": np.ascontiguousarray(v) for k, v in w.items()}


def _save(path, tensors, metadata=None):
    from safetensors.numpy import save_file
    save_file(tensors, str(path), metadata=metadata)


def test_reads_every_tensor_as_written(tmp_path):
    t = _layer_tensors(True)
    t["encoder.pre_encode.counter"] = np.arange(3, dtype=np.int64)  # a dtype the path never reads
    _save(tmp_path / "model.safetensors", t, {"format": "mlx"})
    ck = M.Checkpoint(str(tmp_path / "model.safetensors"))
    got = ck.tensors()
    assert set(got) == set(t) - {"encoder.pre_encode.counter"}
    for k, v in got.items():
        assert v.dtype == t[k].dtype and v.shape == t[k].shape and np.array_equal(v, t[k]), k
    assert ck.metadata("format") == "mlx" and ck.metadata("absent") is None
    assert ck.quantization() is None  # no config beside the file


def test_bf16_tensors(tmp_path):
    import torch
    from safetensors.torch import save_file
    w = torch.randn(8, 16).to(torch.bfloat16)
    save_file({"x.weight": w}, str(tmp_path / "w.safetensors"))
    got = M.Checkpoint(str(tmp_path / "w.safetensors")).tensors()["x.weight"]
    assert np.array_equal(got, w.view(torch.int16).numpy().view(np.uint16))


@pytest.mark.parametrize("config", ["config.json", "config.yaml", "model_config.yaml+config.json", "none"])
def test_directory_discovery_and_quantization(tmp_path, config):
    _save(tmp_path / "weights.safetensors", _layer_tensors(True))
    if config == "config.json":
        (tmp_path / "config.json").write_text(json.dumps({"model_type": "x", "quantization": {"bits": 8, "group_size": 64}}))
    elif config == "config.yaml":
        (tmp_path / "config.yaml").write_text("model: conformer\nquantization:\n  bits: 8\n  group_size: 64\nd_model: 128\n")
    elif config == "model_config.yaml+config.json":
        # the main config has none; MLX keeps it in config.json (checkpoint.rs:613-621)
        (tmp_path / "model_config.yaml").write_text("d_model: 128\n")
        (tmp_path / "config.json").write_text(json.dumps({"quantization": {"group_size": 64, "bits": 4}}))
    ck = M.Checkpoint(str(tmp_path))
    q = ck.quantization()
    if config == "none":
        assert q is None
    else:
        assert (q.bits, q.group_size) == ((4, 64) if "model_config" in config else (8, 64))
    assert len(ck.tensors()) == len(_layer_tensors(True))


def test_quantization_defaults_and_flow_yaml(tmp_path):
    _save(tmp_path / "model.safetensors", _layer_tensors(True))
    (tmp_path / "config.yaml").write_text("quantization: {group_size: 32}\n")
    q = M.Checkpoint(str(tmp_path)).quantization()
    assert (q.bits, q.group_size) == (8, 32)


def test_load_layer_from_checkpoint(tmp_path):
    """A quantized layer loads with the checkpoint's (8, 64); a config naming
    4 bits is rejected as the reference's 8-bit-only kernels would be; strict
    loading of a prefix that is not there fails with ENOENT."""
    _save(tmp_path / "model.safetensors", _layer_tensors(True))
    (tmp_path / "config.json").write_text(json.dumps({"quantization": {"bits": 8, "group_size": 64}}))
    ck = M.Checkpoint(str(tmp_path))
    layer = M.RelPositionMultiHeadAttention(128, 2, True)
    layer.load_checkpoint(ck, PREFIX)
    with pytest.raises(M.MhsaError) as e:
        layer.load_checkpoint(ck, "encoder.layers.7.self_attn")
    assert e.value.code == M.MHSA_ENOENT
    layer.load_checkpoint(ck, "encoder.layers.7.self_attn", strict=False)  # lenient: nothing to load
    (tmp_path / "config.json").write_text(json.dumps({"quantization": {"bits": 4, "group_size": 64}}))
    with pytest.raises(M.MhsaError) as e:
        M.RelPositionMultiHeadAttention(128, 2, True).load_checkpoint(M.Checkpoint(str(tmp_path)), PREFIX)
    assert e.value.code == M.MHSA_ENOTSUP


def _raw_file(path, entries, data, header_len=None, pad=b""):
    hdr = json.dumps(entries).encode() + pad
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hdr) if header_len is None else header_len))
        f.write(hdr)
        f.write(data)


def test_misaligned_tensor_and_malformed_files(tmp_path):
    # an f32 tensor at an odd byte offset (written by hand) reads back exactly
    a = np.arange(3, dtype=np.float16)
    b = np.linspace(-1, 1, 5).astype(np.float32)
    ents = {"a": {"dtype": "F16", "shape": [3], "data_offsets": [0, 6]},
            "b": {"dtype": "F32", "shape": [5], "data_offsets": [7, 27]}}
    data = a.tobytes() + b"\x00" + b.tobytes()
    _raw_file(tmp_path / "odd.safetensors", ents, data, pad=b"  ")
    got = M.Checkpoint(str(tmp_path / "odd.safetensors")).tensors()
    assert np.array_equal(got["a"], a) and np.array_equal(got["b"], b)
    # header length past the end of the file
    _raw_file(tmp_path / "bad1.safetensors", ents, data, header_len=1 << 20)
    # offsets that disagree with the shape
    bad = dict(ents, b={"dtype": "F32", "shape": [6], "data_offsets": [7, 27]})
    _raw_file(tmp_path / "bad2.safetensors", bad, data)
    # not JSON
    with open(tmp_path / "bad3.safetensors", "wb") as f:
        f.write(struct.pack("<Q", 5) + b"{nope" + data)
    # a shape whose byte size wraps 64 bits to the empty range it names
    # (2^40 * 2^40 * 4 = 2^82 = 0 mod 2^64), a negative and a fractional
    # dimension, a negative offset
    wrap = dict(ents, b={"dtype": "F32", "shape": [2 ** 40, 2 ** 40], "data_offsets": [7, 7]})
    _raw_file(tmp_path / "bad4.safetensors", wrap, data)
    _raw_file(tmp_path / "bad5.safetensors", dict(ents, b={"dtype": "F32", "shape": [-5], "data_offsets": [7, 27]}),
              data)
    _raw_file(tmp_path / "bad6.safetensors", dict(ents, b={"dtype": "F32", "shape": [2.5, 2], "data_offsets": [7, 27]}),
              data)
    _raw_file(tmp_path / "bad7.safetensors", dict(ents, a={"dtype": "F16", "shape": [3], "data_offsets": [-6, 0]}),
              data)
    for n in ("bad1", "bad2", "bad3", "bad4", "bad5", "bad6", "bad7"):
        with pytest.raises(M.MhsaError) as e:
            M.Checkpoint(str(tmp_path / f"{n}.safetensors"))
        assert e.value.code == M.MHSA_EINVAL, n
    with pytest.raises(M.MhsaError) as e:
        M.Checkpoint(str(tmp_path / "missing.safetensors"))
    assert e.value.code == M.MHSA_ENOENT
