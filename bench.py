#!/usr/bin/env python3
"""Benchmark of the MI355X rel-pos MHSA path (one GPU).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME] [--no-cpu]

A step is one pass of the path over one batch of synthetic input already
resident in HBM:
  xl_offline_bf16 (default)  one sublayer forward, D=1024, H=8, B=8, T=375, bf16,
                             key padding (valid lengths U{188..375})
  large_f32                  one forward, D=512, H=8, B=1, T=125, fp32
  xl_local_bf16              one forward, B=2, T=7500, +-128 window, 257-row table
  xl_stack_u8                24 quantized pre-LN sublayers, B=4, T=1500, bf16
  xl_stream_f32              one 14-frame chunk for 16 sessions against the
                             70-frame cache ring, fp32 (frames = 16 * 14)
Prints one JSON line: whole-step throughput in encoder frames/s, the dominant
kernel's roofline (its average launch time from HIP events recorded on the
launch stream by the library's profiler) and the CPU baseline (the fp32 C++
restatement of the reference algorithm, timed on the host's cores).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mlx-nemo-rs_amd"))

METRIC = "rel-pos MHSA encoder frames/sec (0.6B shape, bf16); % of MFMA/HBM roofline"
PEAK = {"bf16": 2500.0, "f32": 157.3}  # dense MFMA TFLOP/s (MI355X)
HBM_PEAK = 8000.0  # GB/s


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="xl_offline_bf16")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run a plain device copy of BYTES (calibrates rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def copy_probe(nbytes: int):
    """A plain copy kernel of known size: FETCH_SIZE / WRITE_SIZE for it should
    read nbytes / 1024 KiB per dispatch; the ratio scales the path's counters."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": nbytes, "dispatches": 5}))


def kernel_work(cfg, tag, lengths, fills):
    """Algorithmic work of one launch of kernel `tag`: (amount, unit, bound)."""
    D, T, B = cfg.d_model, cfg.seq_len, cfg.batch
    if cfg.cache_size:  # streaming chunk
        C = cfg.cache_size
        if tag == "attention":  # bytes: Q + visible K/V + position band + O (fp32)
            band = 2 * (C + T) - 1
            vis = sum(T + f for f in fills)
            return (4.0 * (2 * B * T * D + 2 * vis * D + band * D), "GB/s", "hbm")
        rows = {"gemm_qkv": 3, "gemm_q": 1, "gemm_kv": 2, "gemm_out": 1}.get(tag)
        if rows:
            return (2.0 * B * T * D * D * rows, "TFLOP/s", "mfma")
        return None
    lens = lengths or [T] * B
    if tag == "gemm_qkv":
        return (2.0 * B * T * 3 * D * D, "TFLOP/s", "mfma")
    if tag == "gemm_out":
        return (2.0 * B * T * D * D, "TFLOP/s", "mfma")
    if tag == "gemm_pos":
        rows = cfg.pos_band or (2 * T - 1)
        return (2.0 * rows * D * D, "TFLOP/s", "mfma")
    if tag == "attention":
        import workloads as W
        total = W.algorithmic_flops(cfg, lengths) / cfg.layers
        proj = 2.0 * D * D * (4 * B * T + (cfg.pos_band or (2 * T - 1)))
        return (total - proj, "TFLOP/s", "mfma")
    if tag == "layer_norm":
        es = 2 if cfg.dtype == "bfloat16" else 4
        return (2.0 * B * T * D * es, "GB/s", "hbm")
    return None


def measured_traffic(workload, kernel):
    """HBM bytes per launch of `kernel`, from the rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary committed for this workload (each counter scaled by what it reads for a
    plain copy of known size). None when no summary covers the kernel."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{workload}.txt")
    if not os.path.exists(path):
        return None
    ff = wf = None
    for line in open(path):
        kv = dict(t.split("=", 1) for t in line.split()[1:] if "=" in t)
        if line.startswith("calibration"):
            ff, wf = float(kv["fetch_factor"]), float(kv["write_factor"])
        elif line.startswith("traffic") and kv.get("kernel") == kernel and ff is not None:
            return round((float(kv["fetch_kib"]) * ff + float(kv["write_kib"]) * wf) * 1024.0)
    return None


def cpu_baseline(cfg, layer_w, x, pos, lengths, budget_s):
    """Time the fp32 CPU restatement of the reference algorithm on the host."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import cpu_ref
    import subprocess

    xin, pin = x, pos
    scale_bd = None
    if cfg.dtype == "bfloat16":
        import torch
        xin = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
        pin = torch.from_numpy(pos).to(torch.bfloat16).float().numpy()
        dk = cfg.d_model // cfg.n_heads
        scale_bd = float(torch.tensor(1.0 / np.sqrt(np.float32(dk)), dtype=torch.float32).to(torch.bfloat16).float())
    ctx = None
    if cfg.context is not None:
        ctx = (cfg.context[0], cfg.context[1], cfg.context[2] == "chunked_limited")
    passes, t0 = 0, time.perf_counter()
    while True:
        cpu_ref.forward(layer_w, cfg.n_heads, xin, pin, ctx, lengths, scale_bd)
        passes += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    el = time.perf_counter() - t0
    try:
        model = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        model = next((l.split(":", 1)[1].strip() for l in model.splitlines() if l.startswith("Model name")), "")
    except Exception:
        model = ""
    return {"value": round(passes * cfg.batch * cfg.seq_len / el, 2), "unit": "frames/s", "cores": cpu_ref.threads(),
            "kind": "port",
            "sample": f"{passes} full pass(es) of the workload (B={cfg.batch}, T={cfg.seq_len}) in {el:.1f} s; "
                      f"fp32 C++ restatement of the reference algorithm as written (all 2T-1 position rows, "
                      f"pad-reshape rel_shift, full-key masked softmax), OpenMP; CPU: {model}"}


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import relpos_mhsa as M
    import workloads as W

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        sys.exit(1)
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    M.library()  # fails loudly if the HIP library is missing
    cfg = W.CONFIGS[args.config]
    layers_w, x, ex = W.instantiate(cfg)
    dt = torch.bfloat16 if cfg.dtype == "bfloat16" else torch.float32
    D, T, B = cfg.d_model, cfg.seq_len, cfg.batch
    lengths = ex.get("lengths")
    fills = ex.get("fills")

    layers = []
    for i, w in enumerate(layers_w):
        layer = M.RelPositionMultiHeadAttention(D, cfg.n_heads, cfg.use_bias)
        layer.load_weights(W.prefixed(w, f"encoder.layers.{i}.self_attn"), f"encoder.layers.{i}.self_attn")
        layer.set_dtype(dt)
        layers.append(layer)
    pe = M.RelPositionalEncoding(D, 5000, True)
    ctx = M.AttentionContext.new((cfg.context[0], cfg.context[1]), cfg.context[2]) if cfg.context else None
    kmask = M.key_padding_mask(lengths, T) if lengths else None

    if cfg.cache_size:
        C = cfg.cache_size
        pos_np = pe.get_encoding(C + T).numpy()
        pos = torch.from_numpy(pos_np).cuda().to(dt).contiguous()
        chunks = torch.from_numpy(ex["chunks"]).cuda().to(dt).contiguous()
        st = layers[0].stream(B, C, T)
        st.load_cache(torch.from_numpy(ex["cache"]).cuda().contiguous(), fills)
        mask = M.StreamingMask((cfg.context[0], cfg.context[1]), cfg.context[2])
        out = torch.empty_like(chunks[0])
        state = {"i": 0}

        def step():
            st.step(chunks[state["i"] % cfg.steps], pos, mask, out)
            state["i"] += 1
        frames_per_step = B * T
    else:
        pos_rows = cfg.pos_band if cfg.pos_band else T
        pos_np = pe.get_encoding((pos_rows + 1) // 2 if cfg.pos_band else T).numpy()
        pos = torch.from_numpy(pos_np).cuda().to(dt).contiguous()
        xd = torch.from_numpy(x).cuda().to(dt).contiguous()
        if cfg.layers > 1:
            xs = xd.clone()

            def step():
                xs.copy_(xd)
                for layer in layers:
                    layer.sublayer_forward_(xs, pos, ctx, kmask)
        else:
            out = torch.empty_like(xd)
            layer = layers[0]

            def step():
                M._check(layer._lib.mhsa_forward(layer._h, M._dptr(xd), B, T, M._dptr(pos), pos.shape[1],
                                                 M.ctypes.byref(ctx.c()) if ctx else None, M._int_array(kmask),
                                                 M._dptr(out), M._stream_ptr()))
        frames_per_step = B * T

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    ms_per_step = wall * 1e3 / args.steps
    value = frames_per_step * args.steps / wall

    # per-kernel averages from the library's event profiler (separate pass)
    for layer in layers:
        layer.profile_reset()
        layer.profile(True)
    prof_steps = min(args.steps, 50)
    for _ in range(prof_steps):
        step()
    torch.cuda.synchronize()
    kernels = {}
    for layer in layers:
        for tag, (ms, n) in layer.profile_read().items():
            tot, cnt = kernels.get(tag, (0.0, 0))
            kernels[tag] = (tot + ms, cnt + n)
        layer.profile(False)
    dom = max(kernels, key=lambda k: kernels[k][0])
    avg_ms = kernels[dom][0] / kernels[dom][1]
    work = kernel_work(cfg, dom, lengths, fills)
    dtag = "bf16" if cfg.dtype == "bfloat16" else "f32"
    roof = None
    if work:
        amount, unit, bound = work
        if unit == "TFLOP/s":
            ach, peak = amount / (avg_ms * 1e-3) / 1e12, PEAK[dtag]
        else:
            ach, peak = amount / (avg_ms * 1e-3) / 1e9, HBM_PEAK
        roof = {"bound": bound, "kernel": dom, "achieved": round(ach, 2), "peak": peak, "unit": unit,
                "frac": round(ach / peak, 4), "traffic": measured_traffic(cfg.name, dom), "avg_launch_us": round(avg_ms * 1e3, 2),
                "algorithmic_per_launch": amount}

    total_flops = W.algorithmic_flops(cfg, lengths, fills)
    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "frames/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dtag, "data": "synthetic (seeded numpy PCG64; Xavier-uniform weights)",
        "config": {"workload": cfg.name, "d_model": D, "n_heads": cfg.n_heads, "batch": B, "seq_len": T,
                   "layers": cfg.layers, "quantized_u8": cfg.quantized,
                   "key_padding": bool(lengths), "context": cfg.context, "cache_size": cfg.cache_size or None},
        "gpu_ms_per_step": round(gpu_ms / args.steps, 4),
        "step_tflops": round(total_flops / (ms_per_step * 1e-3) / 1e12, 2),
        "roofline": roof,
        "kernels_avg_us": {k: round(v[0] / v[1] * 1e3, 2) for k, v in sorted(kernels.items())},
    }
    if not args.no_cpu and cfg.name in ("xl_offline_bf16", "large_f32"):
        result["cpu_baseline"] = cpu_baseline(cfg, layers_w[0], x, pos_np, lengths, args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result))


if __name__ == "__main__":
    main()
