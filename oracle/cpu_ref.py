"""ctypes wrapper of the fp32 CPU restatement (oracle/cpu_ref.cpp).

TEST INFRASTRUCTURE ONLY: used by tests/ to cross-check the numpy oracle.
The timed CPU baseline of bench.py is the numpy + OpenBLAS restatement in
oracle/cpu_blas.py, not this file.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libmhsa_cpu.so")
_lib = None


def build():
    subprocess.run(["make", "-B", "-C", HERE], check=True, capture_output=True)
    return LIB


def library():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = ctypes.CDLL(LIB)
        _lib.cpu_mhsa_forward.restype = ctypes.c_int
        _lib.cpu_mhsa_threads.restype = ctypes.c_int
    return _lib


def threads() -> int:
    return library().cpu_mhsa_threads()


def _f(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def forward(weights, n_heads, x, pos_emb, context=None, lengths=None, scale_bd=None):
    """Reference algorithm as written, fp32. weights: dict with
    `linear_{q,k,v,out,pos}.weight` [D,D], optional `.bias`, `pos_bias_u/v`.
    context: (left, right, chunked) or None. Returns [B, T, D] float32."""
    x = _f(x)
    B, T, D = x.shape
    dk = D // n_heads
    if scale_bd is None:
        scale_bd = float(np.float32(1.0) / np.sqrt(np.float32(dk)))
    arrs = {}
    for name in ("linear_q", "linear_k", "linear_v", "linear_out", "linear_pos"):
        arrs[name + ".weight"] = _f(weights[name + ".weight"])
        b = weights.get(name + ".bias")
        arrs[name + ".bias"] = None if b is None else _f(b)
    pbu, pbv = _f(weights["pos_bias_u"]).reshape(-1), _f(weights["pos_bias_v"]).reshape(-1)
    pe = _f(pos_emb).reshape(2 * T - 1, D)
    out = np.empty_like(x)
    P = lambda a: None if a is None else a.ctypes.data_as(ctypes.c_void_p)
    has, left, right, chunked = (0, -1, -1, 0) if context is None else (1, context[0], context[1], int(context[2]))
    lens = None if lengths is None else (ctypes.c_int * B)(*[int(v) for v in lengths])
    rc = library().cpu_mhsa_forward(
        B, T, D, n_heads, P(x), P(pe),
        P(arrs["linear_q.weight"]), P(arrs["linear_q.bias"]), P(arrs["linear_k.weight"]), P(arrs["linear_k.bias"]),
        P(arrs["linear_v.weight"]), P(arrs["linear_v.bias"]), P(arrs["linear_out.weight"]),
        P(arrs["linear_out.bias"]), P(arrs["linear_pos.weight"]), P(pbu), P(pbv), has, left, right, chunked, lens,
        ctypes.c_float(scale_bd), P(out))
    if rc != 0:
        raise RuntimeError(f"cpu_mhsa_forward failed: {rc}")
    return out
