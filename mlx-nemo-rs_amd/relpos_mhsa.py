"""Python mirror of the reference's rel-pos MHSA API over the HIP C ABI.

The classes follow animaslabs/mlx-nemo-rs (crate mlx-voice 0.3.0) so tests and
callers read like the reference:

* `RelPositionMultiHeadAttention`  src/asr/modules/encoders/attention.rs:328-893
* `RelPositionalEncoding`          attention.rs:19-194
* `AttentionContext`, `key_padding_mask`  attention.rs:208-294
* `LinearLayer`, `QuantizationConfig`     src/core/quantization.rs:17-162

Device tensors are torch tensors on the GPU (torch supplies memory and the
current HIP stream); all arithmetic runs in `libmhsa_hip.so`. There is no CPU
fallback: constructing a layer without the built library raises.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Dict, Optional, Sequence, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmhsa_hip.so")

MHSA_OK, MHSA_ENOENT, MHSA_ENOMEM, MHSA_EINVAL, MHSA_ENOTSUP, MHSA_EHIP = 0, 2, 12, 22, 95, 1000
F32, BF16, F16, U32 = 0, 1, 2, 3
LINEARS = ("linear_q", "linear_k", "linear_v", "linear_out", "linear_pos")

# Every symbol include/relpos_mhsa.h declares.
EXPORTS = (
    "mhsa_last_error", "mhsa_version", "mhsa_create", "mhsa_destroy", "mhsa_set_dtype", "mhsa_get_dtype",
    "mhsa_head_dim", "mhsa_n_heads", "mhsa_d_model", "mhsa_set_cache_drop_size", "mhsa_load_linear_standard",
    "mhsa_load_linear_quantized", "mhsa_load_pos_bias", "mhsa_load_weights", "mhsa_checkpoint_open",
    "mhsa_checkpoint_close", "mhsa_checkpoint_quantization", "mhsa_checkpoint_count", "mhsa_checkpoint_tensor",
    "mhsa_checkpoint_metadata", "mhsa_load_weights_from_checkpoint", "mhsa_forward", "mhsa_forward_noalloc",
    "mhsa_sublayer_forward", "mhsa_stack_sublayer_forward", "mhsa_stream_create", "mhsa_stream_destroy", "mhsa_stream_load_cache",
    "mhsa_stream_read_cache", "mhsa_stream_fill", "mhsa_forward_with_cache", "mhsa_forward_uncached",
    "mhsa_stack_create", "mhsa_stack_destroy", "mhsa_stack_load_cache", "mhsa_stack_read_cache", "mhsa_stack_fill",
    "mhsa_stack_step", "mhsa_ffn_create", "mhsa_ffn_destroy", "mhsa_ffn_set_dtype", "mhsa_ffn_load_weights",
    "mhsa_ffn_forward", "mhsa_ffn_sublayer_forward", "mhsa_ffn_forward_f32", "mhsa_ffn_sublayer_forward_f32",
    "mhsa_conv_create", "mhsa_conv_destroy", "mhsa_conv_set_dtype",
    "mhsa_conv_load_weights", "mhsa_conv_cache_size", "mhsa_conv_output_dtype", "mhsa_conv_forward",
    "mhsa_conv_forward_with_cache", "mhsa_conv_sublayer_forward", "mhsa_conv_profile_enable",
    "mhsa_conv_profile_repeat", "mhsa_conv_profile_reset", "mhsa_conv_profile_count", "mhsa_conv_profile_entry",
    "mhsa_pos_encoding",
    "mhsa_block_create", "mhsa_block_destroy", "mhsa_block_set_dtype", "mhsa_block_load_weights",
    "mhsa_block_attention", "mhsa_block_feed_forward", "mhsa_block_conv", "mhsa_block_forward",
    "mhsa_encoder_forward", "mhsa_block_output_dtype", "mhsa_block_forward_to", "mhsa_encoder_forward_to",
    "mhsa_encoder_create", "mhsa_encoder_destroy", "mhsa_encoder_load_cache",
    "mhsa_encoder_read_cache", "mhsa_encoder_fill", "mhsa_encoder_step",
    "mhsa_ffn_profile_enable", "mhsa_ffn_profile_repeat", "mhsa_ffn_profile_reset", "mhsa_ffn_profile_count",
    "mhsa_ffn_profile_entry", "mhsa_ffn_debug_linear", "mhsa_conv_debug_linear",
    "mhsa_debug_dequantize", "mhsa_debug_linear", "mhsa_debug_linear_f32", "mhsa_debug_layer_norm",
    "mhsa_debug_attention_forms", "mhsa_debug_offline_mask", "mhsa_debug_stream_mask", "mhsa_debug_rel_shift_index",
    "mhsa_debug_position_scores", "mhsa_debug_top_keys", "mhsa_profile_enable", "mhsa_profile_repeat",
    "mhsa_profile_reset", "mhsa_profile_count",
    "mhsa_profile_entry",
)


class MhsaError(RuntimeError):
    """A failing C-ABI call (the reference's `Error`, src/core/error.rs:7-12)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class Context(ctypes.Structure):
    _fields_ = [("left", ctypes.c_int32), ("right", ctypes.c_int32), ("chunked", ctypes.c_int32)]


class StreamMask(ctypes.Structure):
    _fields_ = [("present", ctypes.c_int32), ("ctx", Context),
                ("filled_host", ctypes.POINTER(ctypes.c_int32)),
                ("valid_host", ctypes.POINTER(ctypes.c_int32))]


class Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("shape", ctypes.c_int64 * 4), ("data", ctypes.c_void_p)]


_LIB = None


def library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the HIP library once; raises if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise MhsaError(MHSA_ENOENT, f"{path} is missing: build it with mlx-nemo-rs_amd/build.py")
    lib = ctypes.CDLL(path)
    P, I, F, VP = ctypes.POINTER, ctypes.c_int32, ctypes.c_float, ctypes.c_void_p
    PI = P(ctypes.c_int32)
    sig = {
        "mhsa_last_error": (ctypes.c_char_p, []),
        "mhsa_version": (I, []),
        "mhsa_create": (I, [I, I, I, P(VP)]),
        "mhsa_destroy": (None, [VP]),
        "mhsa_set_dtype": (I, [VP, I]),
        "mhsa_get_dtype": (I, [VP]),
        "mhsa_head_dim": (I, [VP]),
        "mhsa_n_heads": (I, [VP]),
        "mhsa_d_model": (I, [VP]),
        "mhsa_set_cache_drop_size": (I, [VP, I]),
        "mhsa_load_linear_standard": (I, [VP, I, I, VP, VP]),
        "mhsa_load_linear_quantized": (I, [VP, I, VP, VP, VP, VP, I, I]),
        "mhsa_load_pos_bias": (I, [VP, I, VP, VP]),
        "mhsa_load_weights": (I, [VP, P(Tensor), I, ctypes.c_char_p, I, I, I]),
        "mhsa_checkpoint_open": (I, [ctypes.c_char_p, P(VP)]),
        "mhsa_checkpoint_close": (None, [VP]),
        "mhsa_checkpoint_quantization": (I, [VP, PI, PI]),
        "mhsa_checkpoint_count": (I, [VP]),
        "mhsa_checkpoint_tensor": (I, [VP, I, P(Tensor)]),
        "mhsa_checkpoint_metadata": (I, [VP, ctypes.c_char_p, P(ctypes.c_char_p)]),
        "mhsa_load_weights_from_checkpoint": (I, [VP, VP, ctypes.c_char_p, I]),
        "mhsa_forward": (I, [VP, VP, I, I, VP, I, P(Context), PI, VP, VP]),
        "mhsa_forward_noalloc": (I, [VP, VP, I, I, VP, I, P(Context), PI, VP, VP]),
        "mhsa_sublayer_forward": (I, [VP, VP, I, I, P(ctypes.c_float), P(ctypes.c_float), F, VP, I, P(Context), PI,
                                      VP]),
        "mhsa_stack_sublayer_forward": (I, [P(VP), I, VP, I, I, P(ctypes.c_float), P(ctypes.c_float), F, VP, I,
                                            P(Context), PI, VP]),
        "mhsa_stream_create": (I, [VP, I, I, I, P(VP)]),
        "mhsa_stream_destroy": (None, [VP]),
        "mhsa_stream_load_cache": (I, [VP, VP, PI, VP]),
        "mhsa_stream_read_cache": (I, [VP, VP, VP]),
        "mhsa_stream_fill": (I, [VP, PI]),
        "mhsa_forward_with_cache": (I, [VP, VP, VP, VP, I, P(StreamMask), VP, VP]),
        "mhsa_forward_uncached": (I, [VP, VP, I, I, VP, I, P(StreamMask), VP, VP]),
        "mhsa_stack_create": (I, [P(VP), I, I, I, I, P(VP)]),
        "mhsa_stack_destroy": (None, [VP]),
        "mhsa_stack_load_cache": (I, [VP, VP, PI, VP]),
        "mhsa_stack_read_cache": (I, [VP, VP, VP]),
        "mhsa_stack_fill": (I, [VP, PI]),
        "mhsa_stack_step": (I, [VP, VP, P(ctypes.c_float), P(ctypes.c_float), F, VP, I, P(StreamMask), VP]),
        "mhsa_ffn_create": (I, [I, I, I, P(VP)]),
        "mhsa_ffn_destroy": (None, [VP]),
        "mhsa_ffn_set_dtype": (I, [VP, I]),
        "mhsa_ffn_load_weights": (I, [VP, P(Tensor), I, ctypes.c_char_p, I, I, I]),
        "mhsa_ffn_forward": (I, [VP, VP, I, VP, VP]),
        "mhsa_ffn_sublayer_forward": (I, [VP, VP, I, P(ctypes.c_float), P(ctypes.c_float), F, VP]),
        "mhsa_ffn_forward_f32": (I, [VP, VP, I, VP, VP]),
        "mhsa_ffn_sublayer_forward_f32": (I, [VP, VP, I, P(ctypes.c_float), P(ctypes.c_float), F, VP]),
        "mhsa_conv_create": (I, [I, I, I, I, I, P(VP)]),
        "mhsa_conv_destroy": (None, [VP]),
        "mhsa_conv_set_dtype": (I, [VP, I]),
        "mhsa_conv_load_weights": (I, [VP, P(Tensor), I, ctypes.c_char_p, I, I, I]),
        "mhsa_conv_cache_size": (I, [VP]),
        "mhsa_conv_output_dtype": (I, [VP]),
        "mhsa_conv_forward": (I, [VP, VP, I, I, PI, VP, VP]),
        "mhsa_conv_forward_with_cache": (I, [VP, VP, I, I, VP, PI, VP, VP]),
        "mhsa_conv_sublayer_forward": (I, [VP, VP, I, I, VP, PI, P(ctypes.c_float), P(ctypes.c_float), F, VP]),
        "mhsa_conv_profile_enable": (I, [VP, I]),
        "mhsa_conv_profile_repeat": (I, [VP, ctypes.c_char_p, I]),
        "mhsa_conv_profile_reset": (I, [VP]),
        "mhsa_conv_profile_count": (I, [VP]),
        "mhsa_conv_profile_entry": (I, [VP, I, P(ctypes.c_char_p), P(ctypes.c_double), PI]),
        "mhsa_pos_encoding": (I, [I, I, I, P(ctypes.c_float)]),
        "mhsa_block_create": (I, [I, I, I, I, I, I, I, P(VP)]),
        "mhsa_block_destroy": (None, [VP]),
        "mhsa_block_set_dtype": (I, [VP, I]),
        "mhsa_block_load_weights": (I, [VP, P(Tensor), I, ctypes.c_char_p, I, I, I]),
        "mhsa_block_attention": (VP, [VP]),
        "mhsa_block_feed_forward": (VP, [VP, I]),
        "mhsa_block_conv": (VP, [VP]),
        "mhsa_block_forward": (I, [VP, VP, I, I, VP, I, P(Context), PI, VP]),
        "mhsa_encoder_forward": (I, [P(VP), I, VP, I, I, VP, I, P(Context), PI, VP]),
        "mhsa_block_output_dtype": (I, [VP, I]),
        "mhsa_block_forward_to": (I, [VP, VP, I, I, I, VP, I, P(Context), PI, VP, VP]),
        "mhsa_encoder_forward_to": (I, [P(VP), I, VP, I, I, I, VP, I, P(Context), PI, VP, VP]),
        "mhsa_encoder_create": (I, [P(VP), I, I, I, I, P(VP)]),
        "mhsa_encoder_destroy": (None, [VP]),
        "mhsa_encoder_load_cache": (I, [VP, VP, VP, PI, VP]),
        "mhsa_encoder_read_cache": (I, [VP, VP, VP, VP]),
        "mhsa_encoder_fill": (I, [VP, PI]),
        "mhsa_encoder_step": (I, [VP, VP, VP, I, P(StreamMask), PI, VP]),
        "mhsa_debug_dequantize": (I, [VP, I, VP, VP]),
        "mhsa_debug_linear": (I, [VP, I, VP, I, VP, VP]),
        "mhsa_debug_linear_f32": (I, [VP, I, VP, I, VP, VP]),
        "mhsa_debug_attention_forms": (I, [P(ctypes.c_int64), I]),
        "mhsa_debug_layer_norm": (I, [VP, VP, I, P(ctypes.c_float), P(ctypes.c_float), F, VP, VP]),
        "mhsa_ffn_debug_linear": (I, [VP, I, I, VP, I, VP, VP]),
        "mhsa_ffn_profile_enable": (I, [VP, I]),
        "mhsa_ffn_profile_repeat": (I, [VP, ctypes.c_char_p, I]),
        "mhsa_ffn_profile_reset": (I, [VP]),
        "mhsa_ffn_profile_count": (I, [VP]),
        "mhsa_ffn_profile_entry": (I, [VP, I, P(ctypes.c_char_p), P(ctypes.c_double), PI]),
        "mhsa_conv_debug_linear": (I, [VP, I, I, VP, I, VP, VP]),
        "mhsa_debug_offline_mask": (I, [I, I, P(Context), PI, VP, VP]),
        "mhsa_debug_stream_mask": (I, [I, I, I, P(StreamMask), VP, VP]),
        "mhsa_debug_rel_shift_index": (I, [I, I, VP, VP]),
        "mhsa_debug_position_scores": (I, [VP, VP, I, I, VP, I, VP, VP, VP, VP]),
        "mhsa_debug_top_keys": (I, [VP, VP, I, I, VP, I, P(Context), PI, VP, VP, VP, VP, VP, VP]),
        "mhsa_profile_enable": (I, [VP, I]),
        "mhsa_profile_repeat": (I, [VP, ctypes.c_char_p, I]),
        "mhsa_profile_reset": (I, [VP]),
        "mhsa_profile_count": (I, [VP]),
        "mhsa_profile_entry": (I, [VP, I, P(ctypes.c_char_p), P(ctypes.c_double), PI]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def _check(rc: int):
    if rc != MHSA_OK:
        raise MhsaError(rc, library().mhsa_last_error().decode())


def _stream_ptr():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _int_array(vals) -> Optional[ctypes.Array]:
    if vals is None:
        return None
    return (ctypes.c_int32 * len(vals))(*[int(v) for v in vals])


def _host_f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _torch_dtype(dtype):
    import torch
    return torch.float32 if dtype == F32 else torch.bfloat16


def _dtype_code(dtype) -> int:
    import torch
    if dtype in (F32, "float32", "f32", torch.float32):
        return F32
    if dtype in (BF16, "bfloat16", "bf16", torch.bfloat16):
        return BF16
    raise MhsaError(MHSA_ENOTSUP, f"dtype {dtype!r} not supported (float32, bfloat16)")


# ---------------------------------------------------------------------------
# reference helper types
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class QuantizationConfig:
    """quantization.rs:17-32."""

    bits: int = 8
    group_size: int = 64


class _Profiled:
    """Per-kernel HIP-event timing of a handle's launches (the C ABI's
    <prefix>profile_* calls)."""

    _PROFILE = "mhsa_profile_"

    def _pf(self, name):
        return getattr(self._lib, self._PROFILE + name)

    def profile(self, enable: bool = True) -> None:
        _check(self._pf("enable")(self._h, 1 if enable else 0))

    def profile_repeat(self, tag: Optional[str], n: int = 1) -> None:
        """Issue launches tagged `tag` n times per event pair while profiling."""
        _check(self._pf("repeat")(self._h, tag.encode() if tag else None, int(n)))

    def profile_reset(self) -> None:
        _check(self._pf("reset")(self._h))

    def profile_read(self) -> Dict[str, Tuple[float, int]]:
        """{kernel tag: (total ms, launches)} accumulated since the last reset."""
        out = {}
        for i in range(self._pf("count")(self._h)):
            name, ms, n = ctypes.c_char_p(), ctypes.c_double(), ctypes.c_int32()
            _check(self._pf("entry")(self._h, i, ctypes.byref(name), ctypes.byref(ms), ctypes.byref(n)))
            out[name.value.decode()] = (ms.value, n.value)
        return out


@dataclass
class LinearLayer:
    """quantization.rs:36-59: standard (weight [out,in] + bias) or MLX affine
    quantized (u32 weight, f16 scales/biases, optional f16 bias)."""

    weight: np.ndarray
    bias: Optional[np.ndarray] = None
    scales: Optional[np.ndarray] = None
    biases: Optional[np.ndarray] = None
    bits: int = 8
    group_size: int = 64

    @staticmethod
    def standard(weight, bias=None) -> "LinearLayer":
        return LinearLayer(np.asarray(weight), None if bias is None else np.asarray(bias))

    @staticmethod
    def quantized(weight, scales, biases, bias=None, bits=8, group_size=64) -> "LinearLayer":
        return LinearLayer(np.asarray(weight, dtype=np.uint32), None if bias is None else np.asarray(bias),
                           np.asarray(scales, dtype=np.float16), np.asarray(biases, dtype=np.float16), bits,
                           group_size)

    def is_quantized(self) -> bool:
        return self.scales is not None


@dataclass(frozen=True)
class AttentionContext:
    """attention.rs:208-227; `new` returns None for full attention."""

    left: int
    right: int
    chunked: bool

    @staticmethod
    def new(size: Tuple[int, int], style: str) -> Optional["AttentionContext"]:
        left, right = size
        if left >= 0 or right >= 0:
            return AttentionContext(int(left), int(right), style == "chunked_limited")
        return None

    def c(self) -> Context:
        return Context(self.left, self.right, 1 if self.chunked else 0)


def key_padding_mask(lengths: Sequence[int], seq_len: int) -> Optional[Tuple[int, ...]]:
    """attention.rs:280-294: None when no frame is padding, otherwise the
    per-item valid lengths (clamped to >= 1) the kernel masks keys with."""
    if all(int(v) >= seq_len for v in lengths):
        return None
    return tuple(max(int(v), 1) for v in lengths)


class RelPositionalEncoding:
    """attention.rs:19-194. `get_encoding` returns a host float32 tensor
    [1, 2*seq_len-1, d_model]; move it to the device in the layer dtype."""

    def __init__(self, d_model: int, max_len: int, xscaling: bool):
        self._d_model = d_model
        self.max_len = max_len
        self._xscale = float(np.sqrt(np.float32(d_model))) if xscaling else 1.0

    def get_encoding(self, seq_len: int):
        import torch
        out = np.empty((2 * seq_len - 1, self._d_model) if seq_len > 0 else (0,), dtype=np.float32)
        _check(library().mhsa_pos_encoding(self._d_model, self.max_len, seq_len,
                                           out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        return torch.from_numpy(out).reshape(1, 2 * seq_len - 1, self._d_model)

    def xscale(self) -> float:
        return self._xscale

    def d_model(self) -> int:
        return self._d_model


@dataclass
class StreamingMask:
    """The parameters `create_attention_mask` takes (conformer.rs:97-221);
    `filled`/`valid` are per session (the reference uses session 0's)."""

    att_context_size: Optional[Tuple[int, int]]
    style: str = "chunked_limited"
    filled: Optional[Sequence[int]] = None
    valid: Optional[Sequence[int]] = None

    def c(self):
        keep = []
        if self.att_context_size is None:
            return StreamMask(0, Context(-1, -1, 0), None, None), keep
        left, right = self.att_context_size
        f = _int_array(self.filled)
        v = _int_array(self.valid)
        keep += [f, v]
        m = StreamMask(1, Context(int(left), int(right), 1 if self.style == "chunked_limited" else 0),
                       ctypes.cast(f, ctypes.POINTER(ctypes.c_int32)) if f is not None else None,
                       ctypes.cast(v, ctypes.POINTER(ctypes.c_int32)) if v is not None else None)
        return m, keep


def _tensor_list(weights: Dict[str, np.ndarray]):
    """A Weights map as the C ABI's tensor list (arrays kept alive by the caller)."""
    arrays, tensors = [], []
    for name, arr in weights.items():
        a = np.ascontiguousarray(arr)
        code = {np.dtype(np.float32): F32, np.dtype(np.float16): F16, np.dtype(np.uint32): U32}.get(a.dtype)
        if code is None:
            a = np.ascontiguousarray(a, dtype=np.float32)
            code = F32
        arrays.append(a)
        shape = (ctypes.c_int64 * 4)(*(list(a.shape) + [0] * (4 - a.ndim)))
        tensors.append(Tensor(name.encode(), code, a.ndim, shape, a.ctypes.data))
    return (Tensor * max(len(tensors), 1))(*tensors), len(tensors), arrays


class FeedForward(_Profiled):
    """FeedForward (conformer.rs:2031-2088) backed by the HIP library."""

    _PROFILE = "mhsa_ffn_profile_"

    def __init__(self, d_model: int, ff_dim: int, use_bias: bool):
        lib = library()
        h = ctypes.c_void_p()
        _check(lib.mhsa_ffn_create(d_model, ff_dim, 1 if use_bias else 0, ctypes.byref(h)))
        self._h, self._lib = h, lib
        self.d_model, self.ff_dim = d_model, ff_dim
        self._dtype = F32

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.mhsa_ffn_destroy(h)
            self._h = None

    def set_dtype(self, dtype) -> None:
        self._dtype = _dtype_code(dtype)
        _check(self._lib.mhsa_ffn_set_dtype(self._h, self._dtype))

    def load_weights(self, weights: Dict[str, np.ndarray], prefix: str,
                     quant: Optional[QuantizationConfig] = None, strict: bool = True) -> None:
        arr_t, n, keep = _tensor_list(weights)
        bits, group = (quant.bits, quant.group_size) if quant else (0, 0)
        _check(self._lib.mhsa_ffn_load_weights(self._h, arr_t, n, prefix.encode(), 1 if strict else 0, bits, group))

    def _check(self, x):
        """x in the module dtype, or f32 (the streaming path's promoted form)."""
        import torch
        want = _torch_dtype(self._dtype)
        if (not x.is_cuda or x.dtype not in (want, torch.float32) or not x.is_contiguous()
                or x.shape[-1] != self.d_model):
            raise MhsaError(MHSA_EINVAL, f"expected a contiguous {want} or float32 GPU tensor [..., {self.d_model}]")
        return x.dtype == torch.float32 and want != torch.float32

    def forward(self, x):
        """forward (conformer.rs:2066-2072); an f32 x in a bf16 module runs
        the promoted form (mhsa_ffn_forward_f32)."""
        import torch
        promoted = self._check(x)
        out = torch.empty_like(x)
        fn = self._lib.mhsa_ffn_forward_f32 if promoted else self._lib.mhsa_ffn_forward
        _check(fn(self._h, _dptr(x), x.numel() // self.d_model, _dptr(out), _stream_ptr()))
        return out

    def sublayer_forward_(self, x, gamma=None, beta=None, eps=1e-5):
        """In place x <- x + 0.5 * forward(LayerNorm(x)) (conformer.rs:1703-1729)."""
        promoted = self._check(x)
        g = None if gamma is None else _host_f32(gamma)
        b = None if beta is None else _host_f32(beta)
        fp = ctypes.POINTER(ctypes.c_float)
        fn = self._lib.mhsa_ffn_sublayer_forward_f32 if promoted else self._lib.mhsa_ffn_sublayer_forward
        _check(fn(self._h, _dptr(x), x.numel() // self.d_model, None if g is None else g.ctypes.data_as(fp),
                  None if b is None else b.ctypes.data_as(fp), float(eps), _stream_ptr()))
        return x

    def debug_linear(self, which: int, x):
        """linear1 (0) or linear2 (1) alone, without its epilogue, through the
        module's GEMM kernels; an f32 x in a bf16 module runs the promoted form."""
        import torch
        promoted = self._check(x) if which == 0 else None
        if which == 1:
            want = _torch_dtype(self._dtype)
            if not x.is_cuda or x.dtype not in (want, torch.float32) or x.shape[-1] != self.ff_dim:
                raise MhsaError(MHSA_EINVAL, f"expected a {want} or float32 GPU tensor [..., {self.ff_dim}]")
            promoted = x.dtype == torch.float32 and want != torch.float32
        rows = x.numel() // x.shape[-1]
        n = self.ff_dim if which == 0 else self.d_model
        out = torch.empty((rows, n), dtype=x.dtype, device=x.device)
        _check(self._lib.mhsa_ffn_debug_linear(self._h, which, 1 if promoted else 0, _dptr(x.contiguous()), rows,
                                               _dptr(out), _stream_ptr()))
        return out


CONV_BATCH_NORM, CONV_LAYER_NORM = 0, 1


class ConvolutionModule(_Profiled):
    """ConvolutionModule (conformer.rs:2105-2437) backed by the HIP library.

    norm: "batch_norm" or "layer_norm" (ConvNormType, asr/config.rs:119-128).
    A causal module's output is f32 whatever its dtype (the f32 causal
    padding and conv cache promote, conformer.rs:2250-2256, 2328-2336)."""

    _PROFILE = "mhsa_conv_profile_"

    def __init__(self, d_model: int, kernel_size: int, norm: str = "batch_norm", causal: bool = False,
                 use_bias: bool = True):
        codes = {"batch_norm": CONV_BATCH_NORM, "layer_norm": CONV_LAYER_NORM}
        if norm not in codes:
            raise MhsaError(MHSA_ENOTSUP, f"conv_norm_type `{norm}` (only batch_norm and layer_norm are supported)")
        lib = library()
        h = ctypes.c_void_p()
        _check(lib.mhsa_conv_create(d_model, kernel_size, codes[norm], 1 if causal else 0, 1 if use_bias else 0,
                                    ctypes.byref(h)))
        self._h, self._lib = h, lib
        self.d_model, self.kernel_size, self.causal = d_model, kernel_size, causal
        self._dtype = F32

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.mhsa_conv_destroy(h)
            self._h = None

    def set_dtype(self, dtype) -> None:
        self._dtype = _dtype_code(dtype)
        _check(self._lib.mhsa_conv_set_dtype(self._h, self._dtype))

    def cache_size(self) -> int:
        return self._lib.mhsa_conv_cache_size(self._h)

    def output_dtype(self):
        return _torch_dtype(self._lib.mhsa_conv_output_dtype(self._h))

    def load_weights(self, weights: Dict[str, np.ndarray], prefix: str,
                     quant: Optional[QuantizationConfig] = None, strict: bool = True) -> None:
        arr_t, n, keep = _tensor_list(weights)
        bits, group = (quant.bits, quant.group_size) if quant else (0, 0)
        _check(self._lib.mhsa_conv_load_weights(self._h, arr_t, n, prefix.encode(), 1 if strict else 0, bits, group))

    def _check_x(self, x, dtype):
        if not x.is_cuda or x.dtype != dtype or not x.is_contiguous() or x.dim() != 3 or x.shape[-1] != self.d_model:
            raise MhsaError(MHSA_EINVAL, f"expected a contiguous {dtype} GPU tensor [B, T, {self.d_model}]")

    def _lens(self, lengths, batch):
        if lengths is None:
            return None
        lens = _int_array(lengths)
        if len(lens) != batch:
            raise MhsaError(MHSA_EINVAL, f"lengths must have {batch} entries")
        return lens

    def _check_cache(self, cache, x):
        import torch
        want = (x.shape[0], self.d_model, self.cache_size())
        if (not cache.is_cuda or cache.dtype != torch.float32 or not cache.is_contiguous()
                or tuple(cache.shape) != want or cache.device != x.device):
            raise MhsaError(MHSA_EINVAL, f"cache must be a contiguous float32 GPU tensor {list(want)} on x's device")

    def debug_linear(self, which: int, x, f32_act: bool = False):
        """pointwise_conv1 (0) or pointwise_conv2 (1) alone through the
        module's GEMM kernels: x [rows, D] in the module dtype, or f32 with
        `f32_act` (the promoted form)."""
        import torch
        want = torch.float32 if f32_act else _torch_dtype(self._dtype)
        if not x.is_cuda or x.dtype != want or not x.is_contiguous() or x.shape[-1] != self.d_model:
            raise MhsaError(MHSA_EINVAL, f"expected a contiguous {want} GPU tensor [..., {self.d_model}]")
        rows = x.numel() // self.d_model
        out = torch.empty((rows, (2 if which == 0 else 1) * self.d_model), dtype=want, device=x.device)
        _check(self._lib.mhsa_conv_debug_linear(self._h, which, 1 if f32_act else 0, _dptr(x), rows, _dptr(out),
                                                _stream_ptr()))
        return out

    def forward(self, x, lengths=None):
        """forward (conformer.rs:2197-2291); lengths [B] (frames past them are padding)."""
        import torch
        self._check_x(x, _torch_dtype(self._dtype))
        out = torch.empty(x.shape, dtype=self.output_dtype(), device=x.device)
        _check(self._lib.mhsa_conv_forward(self._h, _dptr(x), x.shape[0], x.shape[1],
                                           self._lens(lengths, x.shape[0]), _dptr(out), _stream_ptr()))
        return out

    def forward_with_cache(self, x, cache=None, lengths=None):
        """forward_with_cache (conformer.rs:2305-2378) on f32 x; `cache`
        [B, D, K-1] f32 is updated in place (the returned new cache)."""
        import torch
        self._check_x(x, torch.float32)
        if cache is not None:
            self._check_cache(cache, x)
        out = torch.empty_like(x)
        _check(self._lib.mhsa_conv_forward_with_cache(self._h, _dptr(x), x.shape[0], x.shape[1],
                                                      None if cache is None else _dptr(cache),
                                                      self._lens(lengths, x.shape[0]), _dptr(out), _stream_ptr()))
        return out, cache

    def sublayer_forward_(self, x, gamma=None, beta=None, eps=1e-5, cache=None, lengths=None):
        """In place x <- x + forward(LayerNorm(x)) (conformer.rs:1790-1814),
        or with the cache on f32 x (conformer.rs:1936-1941)."""
        import torch
        self._check_x(x, torch.float32 if cache is not None else _torch_dtype(self._dtype))
        if cache is not None:
            self._check_cache(cache, x)
        g = None if gamma is None else _host_f32(gamma)
        b = None if beta is None else _host_f32(beta)
        fp = ctypes.POINTER(ctypes.c_float)
        _check(self._lib.mhsa_conv_sublayer_forward(self._h, _dptr(x), x.shape[0], x.shape[1],
                                                    None if cache is None else _dptr(cache),
                                                    self._lens(lengths, x.shape[0]),
                                                    None if g is None else g.ctypes.data_as(fp),
                                                    None if b is None else b.ctypes.data_as(fp), float(eps),
                                                    _stream_ptr()))
        return x


class Checkpoint:
    """CheckpointLoader (checkpoint.rs:480-760) over an MLX safetensors file or
    model directory: the memory-mapped tensor map and the quantization
    settings from the model's config."""

    _NP = {F32: np.float32, F16: np.float16, U32: np.uint32}

    def __init__(self, path: str):
        lib = library()
        h = ctypes.c_void_p()
        _check(lib.mhsa_checkpoint_open(os.fsencode(path), ctypes.byref(h)))
        self._h, self._lib = h, lib

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.mhsa_checkpoint_close(h)
            self._h = None

    def quantization(self) -> Optional[QuantizationConfig]:
        bits, group = ctypes.c_int32(), ctypes.c_int32()
        _check(self._lib.mhsa_checkpoint_quantization(self._h, ctypes.byref(bits), ctypes.byref(group)))
        return QuantizationConfig(bits.value, group.value) if bits.value else None

    def metadata(self, key: str) -> Optional[str]:
        v = ctypes.c_char_p()
        _check(self._lib.mhsa_checkpoint_metadata(self._h, key.encode(), ctypes.byref(v)))
        return None if v.value is None else v.value.decode()

    def tensors(self) -> Dict[str, np.ndarray]:
        """name -> host array (a copy; bf16 entries as their uint16 bit patterns)."""
        out = {}
        for i in range(self._lib.mhsa_checkpoint_count(self._h)):
            t = Tensor()
            _check(self._lib.mhsa_checkpoint_tensor(self._h, i, ctypes.byref(t)))
            shape = tuple(t.shape[k] for k in range(t.ndim))
            dt = self._NP.get(t.dtype, np.uint16)
            n = int(np.prod(shape)) if shape else 1
            buf = (ctypes.c_char * (n * np.dtype(dt).itemsize)).from_address(t.data)
            out[t.name.decode()] = np.frombuffer(bytes(buf), dtype=dt).reshape(shape)
        return out


# ---------------------------------------------------------------------------
# the attention module
# ---------------------------------------------------------------------------

class RelPositionMultiHeadAttention(_Profiled):
    """RelPositionMultiHeadAttention (attention.rs:328-893) backed by the HIP library."""

    def __init__(self, d_model: int, n_heads: int, use_bias: bool):
        lib = library()
        h = ctypes.c_void_p()
        _check(lib.mhsa_create(d_model, n_heads, 1 if use_bias else 0, ctypes.byref(h)))
        self._h = h
        self._lib = lib
        self.d_model = d_model
        self._cache_drop_size = 0

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.mhsa_destroy(h)
            self._h = None

    # attention.rs:409-433
    def set_dtype(self, dtype) -> None:
        _check(self._lib.mhsa_set_dtype(self._h, _dtype_code(dtype)))

    @property
    def dtype(self):
        return _torch_dtype(self._lib.mhsa_get_dtype(self._h))

    def head_dim(self) -> int:
        return self._lib.mhsa_head_dim(self._h)

    def n_heads(self) -> int:
        return self._lib.mhsa_n_heads(self._h)

    @property
    def cache_drop_size(self) -> int:
        return self._cache_drop_size

    @cache_drop_size.setter
    def cache_drop_size(self, n: int) -> None:
        _check(self._lib.mhsa_set_cache_drop_size(self._h, int(n)))
        self._cache_drop_size = int(n)

    # weights (attention.rs:863-893, quantization.rs:62-82)
    def set_linear(self, name: str, layer: LinearLayer) -> None:
        which = LINEARS.index(name)
        if layer.is_quantized():
            w = np.ascontiguousarray(layer.weight, dtype=np.uint32)
            s = np.ascontiguousarray(layer.scales, dtype=np.float16)
            b = np.ascontiguousarray(layer.biases, dtype=np.float16)
            bias = None if layer.bias is None else np.ascontiguousarray(layer.bias, dtype=np.float16)
            _check(self._lib.mhsa_load_linear_quantized(
                self._h, which, w.ctypes.data, s.ctypes.data, b.ctypes.data,
                None if bias is None else bias.ctypes.data, layer.bits, layer.group_size))
        else:
            w = _host_f32(layer.weight)
            bias = None if layer.bias is None else _host_f32(layer.bias)
            _check(self._lib.mhsa_load_linear_standard(self._h, which, F32, w.ctypes.data,
                                                       None if bias is None else bias.ctypes.data))

    def set_pos_bias(self, u, v) -> None:
        u, v = _host_f32(u), _host_f32(v)
        _check(self._lib.mhsa_load_pos_bias(self._h, F32, u.ctypes.data, v.ctypes.data))

    def load_weights(self, weights: Dict[str, np.ndarray], prefix: str,
                     quant: Optional[QuantizationConfig] = None, strict: bool = True) -> None:
        arr_t, n, keep = _tensor_list(weights)
        bits, group = (quant.bits, quant.group_size) if quant else (0, 0)
        _check(self._lib.mhsa_load_weights(self._h, arr_t, n, prefix.encode(), 1 if strict else 0, bits, group))

    def load_checkpoint(self, ckpt: "Checkpoint", prefix: str, strict: bool = True) -> None:
        """load_weights from an on-disk checkpoint with its quantization."""
        _check(self._lib.mhsa_load_weights_from_checkpoint(self._h, ckpt._h, prefix.encode(), 1 if strict else 0))

    # attention.rs:446-573
    def forward(self, x, pos_emb, context: Optional[AttentionContext] = None,
                key_mask: Optional[Sequence[int]] = None):
        import torch
        b, t, d = x.shape
        pe = pos_emb.reshape(-1, d)
        self._check_dev(x, pe)
        out = torch.empty_like(x)
        ctx = context.c() if context is not None else None
        lens = _int_array(key_mask)
        _check(self._lib.mhsa_forward(self._h, _dptr(x), b, t, _dptr(pe), pe.shape[0],
                                      ctypes.byref(ctx) if ctx is not None else None, lens, _dptr(out),
                                      _stream_ptr()))
        return out

    def forward_noalloc(self, x, pos_emb, out, context: Optional[AttentionContext] = None,
                        key_mask: Optional[Sequence[int]] = None):
        """`forward` into a caller-given `out`, with every intermediate in the
        library's fixed per-GPU scratch (no device allocation; no counterpart
        in the reference). The parameters must already be uploaded: run
        `forward` once after loading weights or changing the dtype."""
        b, t, d = x.shape
        pe = pos_emb.reshape(-1, d)
        self._check_dev(x, pe, out)
        ctx = context.c() if context is not None else None
        _check(self._lib.mhsa_forward_noalloc(self._h, _dptr(x), b, t, _dptr(pe), pe.shape[0],
                                              ctypes.byref(ctx) if ctx is not None else None, _int_array(key_mask),
                                              _dptr(out), _stream_ptr()))
        return out

    def sublayer_forward_(self, x, pos_emb, context=None, key_mask=None, gamma=None, beta=None, eps=1e-5):
        """In place x <- x + forward(LayerNorm(x)) (conformer.rs:1747-1780)."""
        b, t, d = x.shape
        pe = pos_emb.reshape(-1, d)
        self._check_dev(x, pe)
        ctx = context.c() if context is not None else None
        g = None if gamma is None else _host_f32(gamma)
        bb = None if beta is None else _host_f32(beta)
        fp = ctypes.POINTER(ctypes.c_float)
        _check(self._lib.mhsa_sublayer_forward(
            self._h, _dptr(x), b, t, None if g is None else g.ctypes.data_as(fp),
            None if bb is None else bb.ctypes.data_as(fp), float(eps), _dptr(pe), pe.shape[0],
            ctypes.byref(ctx) if ctx is not None else None, _int_array(key_mask), _stream_ptr()))
        return x

    # attention.rs:606-816, functional form: cache in, cache out
    def forward_with_cache(self, x, pos_emb, cache, cache_filled_len=0, att_mask: Optional[StreamingMask] = None):
        """Returns (output, new_cache) like the reference; the cache is [B, C, D]
        or None (the no-cache path, attention.rs:687-700). x, the cache and the
        output are fp32 for both layer dtypes; pos_emb is in the layer dtype.
        `att_mask` describes the mask (None = no mask); its `filled` defaults
        to `cache_filled_len` for every session."""
        import torch
        b, t, d = x.shape
        if cache is None:
            pe = pos_emb.reshape(-1, d)
            self._check_stream_dev(x, pe)
            out = torch.empty_like(x)
            m, keep = (att_mask.c() if att_mask is not None else (None, []))
            _check(self._lib.mhsa_forward_uncached(self._h, _dptr(x), b, t, _dptr(pe), pe.shape[0],
                                                   ctypes.byref(m) if m is not None else None, _dptr(out),
                                                   _stream_ptr()))
            return out, x[:, :max(t - self._cache_drop_size, 0)].clone()
        c = cache.shape[1]
        st = self.stream(b, c, t)
        if att_mask is not None and att_mask.att_context_size is not None and att_mask.filled is None:
            att_mask = StreamingMask(att_mask.att_context_size, att_mask.style, [cache_filled_len] * b,
                                     att_mask.valid)
        st.load_cache(cache, [cache_filled_len] * b)
        out = st.step(x, pos_emb, att_mask)
        return out, st.read_cache()

    def stream(self, batch: int, cache_size: int, chunk_len: int) -> "StreamState":
        return StreamState(self, batch, cache_size, chunk_len)

    def debug_dequantize(self, name: str):
        import torch
        out = torch.empty((self.d_model, self.d_model), dtype=torch.float32, device="cuda")
        _check(self._lib.mhsa_debug_dequantize(self._h, LINEARS.index(name), _dptr(out), _stream_ptr()))
        return out

    # per-kernel HIP-event timing (no counterpart in the reference)
    def debug_linear(self, name: str, x):
        """One projection alone through the forward pass's GEMM kernels."""
        import torch
        rows = x.numel() // self.d_model
        self._check_dev(x)
        out = torch.empty_like(x)
        _check(self._lib.mhsa_debug_linear(self._h, LINEARS.index(name), _dptr(x), rows, _dptr(out),
                                           _stream_ptr()))
        return out

    def debug_linear_f32(self, name: str, x):
        """The projection as the streaming path runs it: f32 x and output,
        fp32 kernels (a bf16 layer's parameters keep their bf16 values)."""
        import torch
        if not x.is_cuda or x.dtype != torch.float32 or not x.is_contiguous():
            raise MhsaError(MHSA_EINVAL, "expected a contiguous float32 GPU tensor")
        rows = x.numel() // self.d_model
        out = torch.empty_like(x)
        _check(self._lib.mhsa_debug_linear_f32(self._h, LINEARS.index(name), _dptr(x), rows, _dptr(out),
                                               _stream_ptr()))
        return out

    def debug_layer_norm(self, x, gamma=None, beta=None, eps=1e-5):
        """The sublayer's LayerNorm alone, as the (stack) sublayer forward runs it."""
        import torch
        self._check_dev(x)
        out = torch.empty_like(x)
        g = None if gamma is None else _host_f32(gamma)
        b = None if beta is None else _host_f32(beta)
        fp = ctypes.POINTER(ctypes.c_float)
        _check(self._lib.mhsa_debug_layer_norm(self._h, _dptr(x), x.numel() // self.d_model,
                                               None if g is None else g.ctypes.data_as(fp),
                                               None if b is None else b.ctypes.data_as(fp), float(eps), _dptr(out),
                                               _stream_ptr()))
        return out

    def debug_position_scores(self, x, pos_emb, with_inputs: bool = False):
        """Scaled rel-shifted position scores [B, H, T, T] (fp32); with
        `with_inputs`, also the projected q [B, T, D] and position rows the
        kernel consumed."""
        import torch
        b, t, d = x.shape
        pe = pos_emb.reshape(-1, d)
        self._check_dev(x, pe)
        out = torch.empty((b, self.n_heads(), t, t), dtype=torch.float32, device=x.device)
        q = torch.empty_like(x) if with_inputs else None
        p = torch.empty_like(pe) if with_inputs else None
        _check(self._lib.mhsa_debug_position_scores(self._h, _dptr(x), b, t, _dptr(pe), pe.shape[0], _dptr(out),
                                                    _dptr(q) if q is not None else None,
                                                    _dptr(p) if p is not None else None, _stream_ptr()))
        return (out, q, p) if with_inputs else out

    def debug_top_keys(self, x, pos_emb, context: Optional[AttentionContext] = None,
                       key_mask: Optional[Sequence[int]] = None, with_inputs: bool = False):
        """bf16 layers: per query row, the visible key with the largest
        attention logit as the production kernel forms it, and that logit:
        ([B, H, T] int32, [B, H, T] float32); -1 where a row sees no key.
        With `with_inputs` (full attention), also the projected q, k [B, T, D]
        and position rows [P, D] the kernel consumed."""
        import torch
        b, t, d = x.shape
        pe = pos_emb.reshape(-1, d)
        self._check_dev(x, pe)
        top = torch.empty((b, self.n_heads(), t), dtype=torch.int32, device=x.device)
        val = torch.empty((b, self.n_heads(), t), dtype=torch.float32, device=x.device)
        q = torch.empty_like(x) if with_inputs else None
        k = torch.empty_like(x) if with_inputs else None
        p = torch.empty_like(pe) if with_inputs else None
        ctx = context.c() if context is not None else None
        opt = lambda a: _dptr(a) if a is not None else None
        _check(self._lib.mhsa_debug_top_keys(self._h, _dptr(x), b, t, _dptr(pe), pe.shape[0],
                                             ctypes.byref(ctx) if ctx is not None else None, _int_array(key_mask),
                                             _dptr(top), _dptr(val), opt(q), opt(k), opt(p), _stream_ptr()))
        return (top, val, q, k, p) if with_inputs else (top, val)

    def _check_stream_dev(self, x, pe, *more):
        """Streaming tensors: x, caches and outputs fp32, pos_emb in the layer dtype."""
        import torch
        for t in (x,) + more:
            if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous():
                raise MhsaError(MHSA_EINVAL, f"streaming activations are contiguous float32 GPU tensors, got "
                                             f"{t.dtype} on {t.device}")
        self._check_dev(pe)

    def _check_dev(self, *ts):
        want = self.dtype
        for t in ts:
            if not t.is_cuda or t.dtype != want or not t.is_contiguous():
                raise MhsaError(MHSA_EINVAL, f"expected a contiguous {want} GPU tensor, got {t.dtype} "
                                             f"on {t.device}")


class StreamState:
    """Per-layer streaming state: the attention cache as an HBM ring
    (EncoderCache::last_channel slice, streaming/core.rs:117-166)."""

    def __init__(self, layer: RelPositionMultiHeadAttention, batch: int, cache_size: int, chunk_len: int):
        self.layer = layer
        self.batch, self.cache_size, self.chunk_len = batch, cache_size, chunk_len
        h = ctypes.c_void_p()
        _check(layer._lib.mhsa_stream_create(layer._h, batch, cache_size, chunk_len, ctypes.byref(h)))
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self.layer._lib.mhsa_stream_destroy(h)
            self._h = None

    def load_cache(self, cache, filled: Optional[Sequence[int]] = None) -> None:
        import torch
        if not cache.is_cuda or cache.dtype != torch.float32 or not cache.is_contiguous():
            raise MhsaError(MHSA_EINVAL, "the cache is a contiguous float32 GPU tensor")
        _check(self.layer._lib.mhsa_stream_load_cache(self._h, _dptr(cache), _int_array(filled), _stream_ptr()))

    def read_cache(self):
        import torch
        out = torch.empty((self.batch, self.cache_size, self.layer.d_model), dtype=torch.float32, device="cuda")
        _check(self.layer._lib.mhsa_stream_read_cache(self._h, _dptr(out), _stream_ptr()))
        return out

    def fill(self):
        arr = (ctypes.c_int32 * self.batch)()
        _check(self.layer._lib.mhsa_stream_fill(self._h, arr))
        return list(arr)

    def step(self, x, pos_emb, mask: Optional[StreamingMask] = None, out=None):
        import torch
        b, t, d = x.shape
        pe = pos_emb.reshape(-1, d)
        if out is None:
            out = torch.empty_like(x)
        self.layer._check_stream_dev(x, pe, out)
        m, keep = (mask.c() if mask is not None else (None, []))
        _check(self.layer._lib.mhsa_forward_with_cache(self.layer._h, self._h, _dptr(x), _dptr(pe), pe.shape[0],
                                                       ctypes.byref(m) if m is not None else None, _dptr(out),
                                                       _stream_ptr()))
        return out


def stack_sublayer_forward_(layers: Sequence["RelPositionMultiHeadAttention"], x, pos_emb, context=None,
                            key_mask=None, gamma=None, beta=None, eps=1e-5):
    """The offline encoder's layer loop over the attention sublayers
    (conformer.rs:542-550): in place x <- x + MHSA_l(LN_l(x)) for every layer,
    with the results of calling `sublayer_forward_` layer by layer;
    gamma/beta [layers, d_model] (None = 1 / 0)."""
    layers = list(layers)
    if not layers:
        raise MhsaError(MHSA_EINVAL, "the stack needs at least one layer")
    b, t, d = x.shape
    pe = pos_emb.reshape(-1, d)
    layers[0]._check_dev(x, pe)
    ctx = context.c() if context is not None else None
    g = None if gamma is None else _host_f32(gamma)
    bb = None if beta is None else _host_f32(beta)
    fp = ctypes.POINTER(ctypes.c_float)
    arr = (ctypes.c_void_p * len(layers))(*[l._h.value for l in layers])
    lib = layers[0]._lib
    _check(lib.mhsa_stack_sublayer_forward(
        arr, len(layers), _dptr(x), b, t, None if g is None else g.ctypes.data_as(fp),
        None if bb is None else bb.ctypes.data_as(fp), float(eps), _dptr(pe), pe.shape[0],
        ctypes.byref(ctx) if ctx is not None else None, _int_array(key_mask), _stream_ptr()))
    return x


class StreamingStack:
    """The encoder's streaming layer loop over the attention sublayers
    (ConformerEncoder::forward_streaming, conformer.rs:840-1047): one cache
    ring per layer, one fill per session."""

    def __init__(self, layers: Sequence[RelPositionMultiHeadAttention], batch: int, cache_size: int,
                 chunk_len: int):
        self.layers = list(layers)
        self.batch, self.cache_size, self.chunk_len = batch, cache_size, chunk_len
        self._lib = library()
        arr = (ctypes.c_void_p * len(self.layers))(*[l._h.value for l in self.layers])
        h = ctypes.c_void_p()
        _check(self._lib.mhsa_stack_create(arr, len(self.layers), batch, cache_size, chunk_len, ctypes.byref(h)))
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.mhsa_stack_destroy(h)
            self._h = None

    def load_cache(self, cache, filled: Optional[Sequence[int]] = None) -> None:
        """cache: [layers, batch, cache_size, d_model] float32 GPU tensor."""
        _check(self._lib.mhsa_stack_load_cache(self._h, _dptr(cache.contiguous()), _int_array(filled), _stream_ptr()))

    def read_cache(self):
        import torch
        out = torch.empty((len(self.layers), self.batch, self.cache_size, self.layers[0].d_model),
                          dtype=torch.float32, device="cuda")
        _check(self._lib.mhsa_stack_read_cache(self._h, _dptr(out), _stream_ptr()))
        return out

    def fill(self):
        arr = (ctypes.c_int32 * self.batch)()
        _check(self._lib.mhsa_stack_fill(self._h, arr))
        return list(arr)

    def step_(self, x, pos_emb, mask: Optional[StreamingMask] = None, gamma=None, beta=None, eps=1e-5):
        """In place x <- x + MHSA_l(LN_l(x)) for every layer; gamma/beta [layers, d_model]."""
        import torch
        if not x.is_cuda or x.dtype != torch.float32 or not x.is_contiguous():
            raise MhsaError(MHSA_EINVAL, "the stack streams contiguous float32 GPU activations")
        pe = pos_emb.reshape(-1, x.shape[-1])
        self.layers[0]._check_dev(pe)
        g = None if gamma is None else _host_f32(gamma)
        b = None if beta is None else _host_f32(beta)
        fp = ctypes.POINTER(ctypes.c_float)
        m, keep = (mask.c() if mask is not None else (None, []))
        _check(self._lib.mhsa_stack_step(self._h, _dptr(x), None if g is None else g.ctypes.data_as(fp),
                                         None if b is None else b.ctypes.data_as(fp), float(eps), _dptr(pe),
                                         pe.shape[0], ctypes.byref(m) if m is not None else None, _stream_ptr()))
        return x


# ---------------------------------------------------------------------------
# debug exports
# ---------------------------------------------------------------------------

ATTENTION_FORMS = ("bf16_wave4", "bf16_wave8", "bf16_wave8_skip", "bf16_mixed", "bf16_mixed_gemm", "chunk_f32",
                   "generic", "generic_key_split")


def debug_attention_forms() -> Dict[str, int]:
    """Launches of each attention kernel form since the library was loaded."""
    lib = library()
    arr = (ctypes.c_int64 * len(ATTENTION_FORMS))()
    n = lib.mhsa_debug_attention_forms(arr, len(ATTENTION_FORMS))
    if n < 0:
        _check(n)
    return {name: int(arr[i]) for i, name in enumerate(ATTENTION_FORMS)}


def debug_offline_mask(batch: int, seq_len: int, context: Optional[AttentionContext],
                       key_lengths: Optional[Sequence[int]]):
    import torch
    out = torch.empty((batch, seq_len, seq_len), dtype=torch.uint8, device="cuda")
    ctx = context.c() if context is not None else None
    _check(library().mhsa_debug_offline_mask(batch, seq_len, ctypes.byref(ctx) if ctx is not None else None,
                                             _int_array(key_lengths), _dptr(out), _stream_ptr()))
    return out


def debug_stream_mask(batch: int, cache_size: int, chunk_len: int, mask: StreamingMask):
    import torch
    out = torch.empty((batch, chunk_len, cache_size + chunk_len), dtype=torch.uint8, device="cuda")
    m, keep = mask.c()
    _check(library().mhsa_debug_stream_mask(batch, cache_size, chunk_len, ctypes.byref(m), _dptr(out),
                                            _stream_ptr()))
    return out


def debug_rel_shift_index(rows: int, total_len: int):
    import torch
    out = torch.empty((rows, total_len), dtype=torch.int32, device="cuda")
    _check(library().mhsa_debug_rel_shift_index(rows, total_len, _dptr(out), _stream_ptr()))
    return out


class _View(_Profiled):
    """A module handle owned by a ConformerBlock: its profiler only."""

    def __init__(self, lib, handle, prefix: str):
        self._lib, self._h, self._PROFILE = lib, ctypes.c_void_p(handle), prefix


class ConformerBlock:
    """ConformerBlock (conformer.rs:1613-2028) backed by the HIP library:
    FF1 half-step, MHSA, convolution, FF2 half-step, norm_out."""

    def __init__(self, d_model: int, n_heads: int, ff_dim: int, conv_kernel: int, conv_norm: str = "batch_norm",
                 causal: bool = False, use_bias: bool = True):
        lib = library()
        h = ctypes.c_void_p()
        norm = CONV_BATCH_NORM if conv_norm == "batch_norm" else CONV_LAYER_NORM
        _check(lib.mhsa_block_create(d_model, n_heads, ff_dim, conv_kernel, norm, 1 if causal else 0,
                                     1 if use_bias else 0, ctypes.byref(h)))
        self._h, self._lib = h, lib
        self.d_model, self.n_heads, self.ff_dim, self.conv_kernel = d_model, n_heads, ff_dim, conv_kernel
        self.causal = causal
        self._dtype = F32

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.mhsa_block_destroy(h)
            self._h = None

    def set_dtype(self, dtype) -> None:
        self._dtype = _dtype_code(dtype)
        _check(self._lib.mhsa_block_set_dtype(self._h, self._dtype))

    @property
    def dtype(self):
        return _torch_dtype(self._dtype)

    def load_weights(self, weights: Dict[str, np.ndarray], prefix: str,
                     quant: Optional[QuantizationConfig] = None, strict: bool = True) -> None:
        arr_t, n, keep = _tensor_list(weights)
        bits, group = (quant.bits, quant.group_size) if quant else (0, 0)
        _check(self._lib.mhsa_block_load_weights(self._h, arr_t, n, prefix.encode(), 1 if strict else 0, bits, group))

    def parts(self):
        """Profiled views of the block's attention layer, conv module and both
        FeedForwards (owned by the block)."""
        lib = self._lib
        return [_View(lib, lib.mhsa_block_attention(self._h), "mhsa_profile_"),
                _View(lib, lib.mhsa_block_conv(self._h), "mhsa_conv_profile_"),
                _View(lib, lib.mhsa_block_feed_forward(self._h, 1), "mhsa_ffn_profile_"),
                _View(lib, lib.mhsa_block_feed_forward(self._h, 2), "mhsa_ffn_profile_")]

    def forward_(self, x, pos_emb, context: Optional[AttentionContext] = None, lengths: Optional[Sequence[int]] = None):
        """In place x <- block(x) (conformer.rs:1693-1875); lengths [B] build the
        padding masks (PaddingMask, conformer.rs:1594-1615)."""
        b, t, d = x.shape
        pe = pos_emb.reshape(-1, d)
        want = _torch_dtype(self._dtype)
        for a in (x, pe):
            if not a.is_cuda or a.dtype != want or not a.is_contiguous():
                raise MhsaError(MHSA_EINVAL, f"expected contiguous {want} GPU tensors")
        ctx = context.c() if context is not None else None
        if lengths is not None and len(lengths) != b:
            raise MhsaError(MHSA_EINVAL, f"lengths must have {b} entries")
        _check(self._lib.mhsa_block_forward(self._h, _dptr(x), b, t, _dptr(pe), pe.shape[0],
                                            ctypes.byref(ctx) if ctx is not None else None, _int_array(lengths),
                                            _stream_ptr()))
        return x

    def output_dtype(self, x_dtype):
        """Dtype of forward's result on activations in x_dtype: f32 once they
        are f32 or the conv is causal (its f32 zero padding promotes a bf16
        block, conformer.rs:2250-2256), else the block dtype."""
        code = self._lib.mhsa_block_output_dtype(self._h, _dtype_code(x_dtype))
        if code < 0:
            raise MhsaError(MHSA_EINVAL, f"a {self.dtype} block cannot take {x_dtype} activations")
        return _torch_dtype(code)

    def forward(self, x, pos_emb, context: Optional[AttentionContext] = None,
                lengths: Optional[Sequence[int]] = None):
        """block(x) as a new tensor (conformer.rs:1693-1875) in
        output_dtype(x.dtype): x in the block dtype or, in a bf16 block, f32
        activations an earlier causal conv promoted."""
        import torch
        b, t, d = x.shape
        pe = pos_emb.reshape(-1, d)
        if not x.is_cuda or not x.is_contiguous() or not pe.is_cuda or not pe.is_contiguous():
            raise MhsaError(MHSA_EINVAL, "expected contiguous GPU tensors")
        if pe.dtype != _torch_dtype(self._dtype):
            raise MhsaError(MHSA_EINVAL, f"pos_emb must be {self.dtype}")
        if lengths is not None and len(lengths) != b:
            raise MhsaError(MHSA_EINVAL, f"lengths must have {b} entries")
        out = torch.empty((b, t, d), dtype=self.output_dtype(x.dtype), device=x.device)
        ctx = context.c() if context is not None else None
        _check(self._lib.mhsa_block_forward_to(self._h, _dptr(x), _dtype_code(x.dtype), b, t, _dptr(pe),
                                               pe.shape[0], ctypes.byref(ctx) if ctx is not None else None,
                                               _int_array(lengths), _dptr(out), _stream_ptr()))
        return out


def encoder_forward_(blocks: Sequence[ConformerBlock], x, pos_emb, context=None, lengths=None):
    """The offline encoder's layer loop over blocks (conformer.rs:542-550), in place."""
    blocks = list(blocks)
    if not blocks:
        raise MhsaError(MHSA_EINVAL, "the encoder needs at least one block")
    b, t, d = x.shape
    pe = pos_emb.reshape(-1, d)
    ctx = context.c() if context is not None else None
    arr = (ctypes.c_void_p * len(blocks))(*[k._h.value for k in blocks])
    _check(blocks[0]._lib.mhsa_encoder_forward(arr, len(blocks), _dptr(x), b, t, _dptr(pe), pe.shape[0],
                                               ctypes.byref(ctx) if ctx is not None else None,
                                               _int_array(lengths), _stream_ptr()))
    return x


def encoder_forward(blocks: Sequence[ConformerBlock], x, pos_emb, context=None, lengths=None):
    """The offline encoder's layer loop over blocks (conformer.rs:542-550) as
    a new tensor, whose dtype follows the blocks' output_dtype (f32 after the
    first causal conv of a bf16 stack)."""
    import torch
    blocks = list(blocks)
    if not blocks:
        raise MhsaError(MHSA_EINVAL, "the encoder needs at least one block")
    b, t, d = x.shape
    pe = pos_emb.reshape(-1, d)
    if not x.is_cuda or not x.is_contiguous() or not pe.is_cuda or not pe.is_contiguous():
        raise MhsaError(MHSA_EINVAL, "expected contiguous GPU tensors")
    dt = x.dtype
    for k in blocks:
        dt = k.output_dtype(dt)
    out = torch.empty((b, t, d), dtype=dt, device=x.device)
    ctx = context.c() if context is not None else None
    arr = (ctypes.c_void_p * len(blocks))(*[k._h.value for k in blocks])
    _check(blocks[0]._lib.mhsa_encoder_forward_to(arr, len(blocks), _dptr(x), _dtype_code(x.dtype), b, t, _dptr(pe),
                                                  pe.shape[0], ctypes.byref(ctx) if ctx is not None else None,
                                                  _int_array(lengths), _dptr(out), _stream_ptr()))
    return out


class StreamingEncoder:
    """The streaming encoder's per-chunk loop over blocks with causal convs
    (ConformerEncoder::forward_streaming, conformer.rs:840-1047): per layer an
    attention ring and the conv cache; one fill per session."""

    def __init__(self, blocks: Sequence[ConformerBlock], batch: int, cache_size: int, chunk_len: int):
        self.blocks = list(blocks)
        lib = self.blocks[0]._lib
        arr = (ctypes.c_void_p * len(self.blocks))(*[k._h.value for k in self.blocks])
        h = ctypes.c_void_p()
        _check(lib.mhsa_encoder_create(arr, len(self.blocks), batch, cache_size, chunk_len, ctypes.byref(h)))
        self._h, self._lib = h, lib
        self.batch, self.cache_size, self.chunk_len = batch, cache_size, chunk_len
        self.d_model = self.blocks[0].d_model

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.mhsa_encoder_destroy(h)
            self._h = None

    def load_cache(self, channel, time=None, filled: Optional[Sequence[int]] = None) -> None:
        _check(self._lib.mhsa_encoder_load_cache(self._h, _dptr(channel), _dptr(time) if time is not None else None,
                                                 _int_array(filled), _stream_ptr()))

    def read_cache(self):
        import torch
        n = len(self.blocks)
        ch = torch.empty((n, self.batch, self.cache_size, self.d_model), dtype=torch.float32, device="cuda")
        tm = torch.empty((n, self.batch, self.d_model, self.blocks[0].conv_kernel - 1), dtype=torch.float32,
                         device="cuda")
        _check(self._lib.mhsa_encoder_read_cache(self._h, _dptr(ch), _dptr(tm), _stream_ptr()))
        return ch, tm

    def fill(self):
        arr = (ctypes.c_int32 * self.batch)()
        _check(self._lib.mhsa_encoder_fill(self._h, arr))
        return list(arr)

    def step_(self, x, pos_emb, mask: Optional[StreamingMask] = None, valid: Optional[Sequence[int]] = None):
        """One chunk through every block, in place (x fp32 [B, T, D])."""
        import torch
        d = self.d_model
        if not x.is_cuda or x.dtype != torch.float32 or not x.is_contiguous():
            raise MhsaError(MHSA_EINVAL, "streaming activations are contiguous float32 GPU tensors")
        pe = pos_emb.reshape(-1, d)
        m, keep = (mask.c() if mask is not None else (None, []))
        _check(self._lib.mhsa_encoder_step(self._h, _dptr(x), _dptr(pe), pe.shape[0],
                                           ctypes.byref(m) if m is not None else None, _int_array(valid),
                                           _stream_ptr()))
        return x
