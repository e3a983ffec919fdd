"""Bit-exact int8 dequantisation on the production GEMM paths.

The quantized projections never materialise a dequantised weight: each GEMM
unpacks the u8 codes and applies W = s * q + b in registers, one form per
kernel (the bf16 tile kernel in all its tile shapes, the paired Q/K/V +
position launch, the fp32 K-parallel, tile and split kernels). Feeding unit
rows through a kernel reads those weights back: with row r of the input equal
to e_{r mod K}, output row r is column r mod K of W (one product 1 * w, the
other terms exactly 0), so every output element is one dequantised weight
as the kernel formed it. It must equal the oracle's dequantisation
(quantization.rs:1-8 layout, 100-111 bf16 cast of scales and biases,
147-155 quantized_matmul): f32(s) * q is exact, so the f32 sum has one
rounding and the value is unique; in bf16 mode it is then stored as bf16.

Scales and biases here span a wide range of f16 exponents (both signs,
subnormal scales included), so a dropped rounding, a double rounding
(product and sum rounded apart with a bf16 scale) or a wrong group index
changes some weight.
"""
import numpy as np
import pytest
import torch

import relpos_oracle as O
import relpos_mhsa as M
import workloads as W

pytestmark = pytest.mark.gpu

LINEARS = ("linear_q", "linear_k", "linear_v", "linear_out", "linear_pos")


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    M.library()
    yield
    torch.cuda.synchronize()


def wide_u8(rng, o, i):
    """Packed u8 codes (every value 0..255 occurs), f16 scales of random sign
    with exponents over [-18, 1] (subnormals below -14) and f16 biases over
    [-16, 4]."""
    codes = rng.integers(0, 256, size=(o, i))
    codes.reshape(-1)[:256] = np.arange(256)
    g = i // 64
    sc = (rng.choice([-1.0, 1.0], size=(o, g)) * np.exp2(rng.uniform(-18, 1, size=(o, g)))).astype(np.float16)
    bi = (rng.choice([-1.0, 1.0], size=(o, g)) * np.exp2(rng.uniform(-16, 4, size=(o, g)))).astype(np.float16)
    return W.pack_u8(codes), sc, bi


def unit_rows(rows, k, dtype):
    """[rows, k] with row r = e_{r mod k}, on the GPU in `dtype`."""
    x = torch.zeros((rows, k), dtype=dtype, device="cuda")
    x[torch.arange(rows, device="cuda"), torch.arange(rows, device="cuda") % k] = 1
    return x


def expect(wdeq, rows):
    """Output of unit rows through W: row r is W[:, r mod K]."""
    return wdeq.T[np.arange(rows) % wdeq.shape[1]]


def exact(got, ref, what):
    got = got.float().cpu().numpy().reshape(ref.shape)
    bad = got != ref.astype(np.float32)
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} weights differ, first at {np.argwhere(bad)[0]}"


def quant_layer(rng, d=1024, h=8):
    w = W.make_layer_weights(rng, d, h, False, True)
    for name in LINEARS:
        w[f"{name}.weight"], w[f"{name}.scales"], w[f"{name}.biases"] = wide_u8(rng, d, d)
    return w


def deq(w, name, dtype, store=None):
    return O.dequantize(w[f"{name}.weight"], w[f"{name}.scales"], w[f"{name}.biases"], 8, 64, dtype, store)


def gpu_layer(w, d, h, dtype):
    layer = M.RelPositionMultiHeadAttention(d, h, False)
    layer.load_weights(W.prefixed(w, "l"), "l")
    layer.set_dtype(dtype)
    return layer


# bf16 tile kernel forms at N = K = 1024: 64x64 (1024 rows), 128x128 with four
# stages (2048), 192x128 (6000), 128x128 with two stages (6200), 256x256 (15000)
@pytest.mark.parametrize("rows", [1024, 2048, 6000, 6200, 15000])
def test_projection_dequant_bf16_tile_forms(rows):
    rng = np.random.default_rng(rows)
    w = quant_layer(rng)
    layer = gpu_layer(w, 1024, 8, O.BF16)
    x = unit_rows(rows, 1024, torch.bfloat16)
    for name in LINEARS:
        exact(layer.debug_linear(name, x), expect(deq(w, name, O.BF16), rows), f"{name} rows={rows}")


# fp32 kernels: K-parallel with 16x16 (100 rows) and 32x32 tiles (1024), the
# 128x128 tile kernel (6200)
@pytest.mark.parametrize("rows", [100, 1024, 6200])
def test_projection_dequant_f32_kernels(rows):
    rng = np.random.default_rng(100 + rows)
    w = quant_layer(rng)
    layer = gpu_layer(w, 1024, 8, O.F32)
    x = unit_rows(rows, 1024, torch.float32)
    for name in LINEARS:
        exact(layer.debug_linear(name, x), expect(deq(w, name, O.F32), rows), f"{name} rows={rows}")


@pytest.mark.parametrize("rows", [100, 224, 1024])
def test_projection_dequant_streaming_form_of_bf16_layer(rows):
    """The streaming path of a bf16 layer: f32 activations, so the fp32 GEMM
    dequantises with the bf16-cast scales and keeps the f32 weight (MLX
    promotion, conformer.rs:845-849)."""
    rng = np.random.default_rng(200 + rows)
    w = quant_layer(rng)
    layer = gpu_layer(w, 1024, 8, O.BF16)
    x = unit_rows(rows, 1024, torch.float32)
    for name in LINEARS:
        exact(layer.debug_linear_f32(name, x), expect(deq(w, name, O.BF16, O.F32), rows), f"{name} rows={rows}")


@pytest.mark.parametrize("batch,seq", [(8, 375), (2, 7500)])
def test_forward_projections_dequant(batch, seq):
    """The offline forward's own projection launches: at 8 x 375 the fused
    Q/K/V GEMM (192x192 tiles) and the position GEMM (64x64) run as one paired
    launch; at 2 x 7500 the Q/K/V GEMM takes 256x256 tiles. The projected q, k
    and position rows the attention consumed are read back."""
    rng = np.random.default_rng(batch * seq)
    w = quant_layer(rng)
    layer = gpu_layer(w, 1024, 8, O.BF16)
    rows = batch * seq
    x = unit_rows(rows, 1024, torch.bfloat16).reshape(batch, seq, 1024)
    pos = unit_rows(2 * seq - 1, 1024, torch.bfloat16).reshape(1, 2 * seq - 1, 1024)
    _, _, q, k, p = layer.debug_top_keys(x, pos, None, None, with_inputs=True)
    exact(q, expect(deq(w, "linear_q", O.BF16), rows), "q")
    exact(k, expect(deq(w, "linear_k", O.BF16), rows), "k")
    exact(p, expect(deq(w, "linear_pos", O.BF16), 2 * seq - 1), "position rows")


def ffn_u8(rng, d, f):
    w = {}
    for name, (o, i) in (("linear1", (f, d)), ("linear2", (d, f))):
        w[f"ff.{name}.weight"], w[f"ff.{name}.scales"], w[f"ff.{name}.biases"] = wide_u8(rng, o, i)
    return w


@pytest.mark.parametrize("dtype,f32_act,rows", [(O.BF16, False, 3000), (O.BF16, False, 4096), (O.BF16, False, 6000),
                                                (O.BF16, True, 224), (O.F32, False, 4096)])
def test_feed_forward_dequant(dtype, f32_act, rows):
    """FeedForward's linear1 [4096, 1024] and linear2 [1024, 4096] (64 groups
    per row) through the module's GEMMs, without their epilogues (linear1 at
    3000 and 6000 rows takes 192x256 tiles, at 4096 192x128)."""
    d, f = 1024, 4096
    rng = np.random.default_rng(300 + rows)
    w = ffn_u8(rng, d, f)
    ff = M.FeedForward(d, f, False)
    ff.load_weights(w, "ff")
    ff.set_dtype(dtype)
    tdt = torch.float32 if (f32_act or dtype == O.F32) else torch.bfloat16
    store = O.F32 if f32_act else None
    for which, (name, k) in enumerate((("linear1", d), ("linear2", f))):
        ref = O.dequantize(w[f"ff.{name}.weight"], w[f"ff.{name}.scales"], w[f"ff.{name}.biases"], 8, 64, dtype,
                           store)
        exact(ff.debug_linear(which, unit_rows(rows, k, tdt)), expect(ref, rows), f"{name} rows={rows}")


def test_projection_dequant_u8_two_stages():
    """A 192-row u8 tile with only two k-stages: d_model 128 at 40000 rows
    takes 192x128 tiles (three LDS stages, loads two ahead), whose prologue
    waits for stage 0 and its scales with stage 1's codes and scales still in
    flight; the loop's first wait must then cover them."""
    d, rows = 128, 40000
    rng = np.random.default_rng(128)
    w = quant_layer(rng, d, 2)
    layer = gpu_layer(w, d, 2, O.BF16)
    x = unit_rows(rows, d, torch.bfloat16)
    for name in LINEARS:
        exact(layer.debug_linear(name, x), expect(deq(w, name, O.BF16), rows), f"{name} d_model={d} rows={rows}")


def test_feed_forward_dequant_u8_one_stage():
    """linear1 of a d_model-64 FeedForward (K = 64: one k-stage, so every
    later load is a reload of it) at 40000 rows: 192x256 u8 tiles, three
    stages."""
    d, f, rows = 64, 256, 40000
    rng = np.random.default_rng(64)
    w = ffn_u8(rng, d, f)
    ff = M.FeedForward(d, f, False)
    ff.load_weights(w, "ff")
    ff.set_dtype(O.BF16)
    ref = O.dequantize(w["ff.linear1.weight"], w["ff.linear1.scales"], w["ff.linear1.biases"], 8, 64, O.BF16)
    exact(ff.debug_linear(0, unit_rows(rows, d, torch.bfloat16)), expect(ref, rows), f"linear1 d_model={d} rows={rows}")


@pytest.mark.parametrize("dtype,f32_act,rows", [(O.BF16, False, 3000), (O.BF16, True, 224), (O.F32, False, 1024)])
def test_conv_pointwise_dequant(dtype, f32_act, rows):
    """ConvolutionModule's pointwise_conv1 [2048, 1024] and pointwise_conv2
    [1024, 1024] through the module's GEMMs."""
    d = 1024
    rng = np.random.default_rng(400 + rows)
    w = W.make_conv_weights(rng, d, 9, "batch_norm", True, False, "conv")
    for name, o in (("pointwise_conv1", 2 * d), ("pointwise_conv2", d)):
        w[f"conv.{name}.weight"], w[f"conv.{name}.scales"], w[f"conv.{name}.biases"] = wide_u8(rng, o, d)
    conv = M.ConvolutionModule(d, 9, "batch_norm", False, False)
    conv.load_weights(w, "conv")
    conv.set_dtype(dtype)
    tdt = torch.float32 if (f32_act or dtype == O.F32) else torch.bfloat16
    store = O.F32 if f32_act else None
    x = unit_rows(rows, d, tdt)
    for which, name in enumerate(("pointwise_conv1", "pointwise_conv2")):
        ref = O.dequantize(w[f"conv.{name}.weight"], w[f"conv.{name}.scales"], w[f"conv.{name}.biases"], 8, 64,
                           dtype, store)
        exact(conv.debug_linear(which, x, f32_act), expect(ref, rows), f"{name} rows={rows}")
