"""Benchmark: one DINOv3 token-correction pass on one MI355X.

Workload (BASELINE.json metric "ms per correction pass + corrected tokens/s, ViT-L/16 512px, 25%
keep"): ViT-L/16 at 512 px, B=16 (1029 tokens per image), 24 blocks, bf16, random-init weights, top
25% of the 1024 patches per image (k=256) selected by importance = ||delta_p||_2 with
delta ~ Laplace(0,1). One step = one full correction pass through the executor API
(`DINOv3ClassifierExecutor.correct_forward`, i.e. `run_dinov3_correct_block` for every layer):
the importance reduction, the top-k plan (recomputed every pass) and all 24 correction blocks. The K/V and
blocks_out_sum caches come from an untimed approximate pass over the base tokens.

Output: one JSON line on stdout. `value` = corrected tokens/s = B*k / pass time; `ms_per_step` =
ms per correction pass. By default the step is recorded once into a HIP graph and the timed steps
are replays (every kernel of the pass runs each step; `config.eager_ms_per_step` is the same K steps
launched one kernel at a time, `--graph 0` reports that instead). `roofline` is for the dominant
kernel, timed live with HIP events around each of its launches in the eager steps; `cpu_baseline`
times the CPU oracle (the reference's eager op sequence on bf16 CPU tensors) on a bounded sample of
the same workload.

Only one GPU is used: `--gpus N` with N > 1 exits with an explanation.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "ms per correction pass + corrected tokens/s, ViT-L/16 512px, 25% keep"
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E

SHAPES = {  # name: (backbone, embed, heads, mlp, depth, img)
    "vits16_224": ("vits16", 384, 6, 1536, 12, 224),
    "vitb16_512": ("vitb16", 768, 12, 3072, 12, 512),
    "vitl16_512": ("vitl16", 1024, 16, 4096, 24, 512),
}


def _roctx():
    """roctxProfilerResume/Pause (rocprofiler-sdk's roctx), used to bracket the timed steps for
    `rocprofv3 --selected-regions`; no-ops when no profiler is attached."""
    for cand in ("librocprofiler-sdk-roctx.so.1", "/opt/rocm/lib/librocprofiler-sdk-roctx.so"):
        try:
            lib = ctypes.CDLL(cand)
        except OSError:
            continue
        if hasattr(lib, "roctxProfilerResume") and hasattr(lib, "roctxProfilerPause"):
            lib.roctxProfilerResume.argtypes = [ctypes.c_uint64]
            lib.roctxProfilerPause.argtypes = [ctypes.c_uint64]
            return lib
    return None


def kernel_work(tag: str, B: int, T: int, N: int, C: int, H: int, mlp: int):
    """Algorithmic work of one launch at a site: (amount, unit, bound)."""
    M = B * T
    if tag == "gemm0":   # qkv
        return 2.0 * M * C * 3 * C / 1e12, "TFLOP/s", "mfma"
    if tag == "gemm1":   # fc1 + GELU
        return 2.0 * M * C * mlp / 1e12, "TFLOP/s", "mfma"
    if tag == "gemm2":   # proj + LayerScale + residual
        return 2.0 * M * C * C / 1e12, "TFLOP/s", "mfma"
    if tag == "gemm3":   # fc2 + LayerScale
        return 2.0 * M * mlp * C / 1e12, "TFLOP/s", "mfma"
    if tag == "attention":
        return 4.0 * B * H * T * N * (C // H) / 1e12, "TFLOP/s", "mfma"
    if tag == "reconstruct":  # fused minimum: 3 B N C + 2 M C bf16 elements + row map
        return (3.0 * B * N * C * 2 + 2.0 * M * C * 2 + 4.0 * B * N) / 1e9, "GB/s", "hbm"
    if tag == "packed_residual":  # read x_act, x_attn, mlp; write x_new, blocks_out_sum rows; row ids
        return (5.0 * M * C * 2 + 16.0 * M) / 1e9, "GB/s", "hbm"
    if tag == "gather_rows":
        return (2.0 * M * C * 2 + 16.0 * M) / 1e9, "GB/s", "hbm"
    if tag == "qkv_post":  # read qkv rows, write q packed + k,v cache rows
        return (2.0 * M * 3 * C * 2 + 16.0 * M) / 1e9, "GB/s", "hbm"
    if tag == "layernorm":
        return (2.0 * M * C * 2) / 1e9, "GB/s", "hbm"
    raise ValueError(tag)


def probe_kernel_name(tag: str, B: int, T: int, C: int, mlp: int):
    """Kernel a GEMM launch site runs in this build (None for other sites)."""
    from appcorr_amd import _lib
    from appcorr_amd import kernels as K

    M = B * T
    shapes = {"gemm0": (M, 3 * C, C, 5), "gemm1": (M, mlp, C, _lib.EPI_BIAS_GELU),
              "gemm2": (M, C, C, _lib.EPI_BIAS_LS_RESID), "gemm3": (M, C, mlp, _lib.EPI_BIAS_LS)}
    if tag not in shapes:
        return None
    return K.linear_kernel_name(*shapes[tag])


def cpu_baseline(name: str, B: int, keep: float, budget_s: float):
    """Oracle (reference eager op order, bf16 CPU tensors) on a bounded sample: one correction block
    of the same shape, repeated until ~budget_s; scaled to a full pass (plan + depth x block)."""
    import torch

    from oracle import model as OM
    from oracle import plan as OP

    nthreads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    torch.set_num_threads(nthreads)
    cfg = OM.CONFIGS[name]
    w = OM.make_block_weights(cfg, 0, depth=1)[0]
    g = torch.Generator().manual_seed(7)
    N, C, H, D = cfg.num_tokens, cfg.dim, cfg.heads, cfg.head_dim
    x = torch.randn(B, N, C, generator=g).to(torch.bfloat16)
    imp = torch.rand(B, cfg.num_patches, generator=g)
    cache = {"layer0_kv": torch.randn(B, N, 2, H, D, generator=g).to(torch.bfloat16),
             "layer0_blocks_out_sum": (torch.randn(B, N, C, generator=g) * 0.01).to(torch.bfloat16)}
    rope = OM.rope_tables(cfg)
    k = OP.keep_count(cfg.num_patches, keep)
    dind = OM.full_dindice(cfg, B).numpy()
    t0 = time.perf_counter()
    plan = OP.build_plan(imp.numpy(), k, dind, cfg.num_pretokens, N)
    t_plan = time.perf_counter() - t0
    times = []
    with torch.no_grad():
        OM.correct_block(cfg, w, x, plan, rope, cache, "layer0", mode="bf16")  # warm-up
        start = time.perf_counter()
        while len(times) < 10 and (time.perf_counter() - start < budget_s or len(times) < 2):
            t0 = time.perf_counter()
            OM.correct_block(cfg, w, x, plan, rope, cache, "layer0", mode="bf16")
            times.append(time.perf_counter() - t0)
    blk = statistics.median(times)
    pass_s = t_plan + cfg.depth * blk
    return {
        "value": B * k / pass_s,
        "unit": "corrected tokens/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"1 of {cfg.depth} blocks ({name}, B={B}, k={k}, bf16 torch CPU eager ops), median of "
                   f"{len(times)} runs = {blk * 1e3:.1f} ms/block, plus the top-k plan ({t_plan * 1e3:.1f} ms); "
                   f"scaled to a {cfg.depth}-block pass = {pass_s * 1e3:.0f} ms"),
        "ms_per_pass": pass_s * 1e3,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="vitl16_512", choices=sorted(SHAPES))
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--keep", type=float, default=0.25)
    ap.add_argument("--probe", default="gemm1", help="launch site timed for the roofline (gemm0..3, attention, ...)")
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU-baseline sampling (0 = skip)")
    ap.add_argument("--cache", default="approx", choices=("approx", "random"),
                    help="fill the K/V + residual caches with the approximate pass (default) or random values")
    ap.add_argument("--graph", type=int, default=1,
                    help="1: record the step into a HIP graph and time its replays (the eager time is reported "
                         "alongside); 0: time eager launches only")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="before the timed steps, copy this many MiB device-to-device once (a plain copy of known "
                         "size that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one MI355X; the correction path shards over images "
              "(data parallel, no exchange) and multi-GPU runs are not part of it. Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from appcorr_amd import _lib
    from appcorr_amd import kernels as K
    from appcorr_amd.dinov3.layers import SelfAttentionBlock
    from appcorr_amd.server.dinov3_classifier import DINOv3ClassifierExecutor, make_group_plan
    from appcorr_amd.server.protocol import ExperimentConfig

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _lib.verify_runtime(0)
    bb, C, H, mlp, depth, img = SHAPES[args.config]
    B = args.batch
    grid = img // 16
    P = grid * grid
    N = 5 + P
    k = min(int(P * args.keep), P)
    T = 5 + k

    config = ExperimentConfig(model_name=f"dinov3_classifier_{bb}", batch_size=B, image_shape=(img, img, 3),
                              backbone=bb, appcorr_kwargs={
                                  "method": "partial_token", "token_keep_ratio": args.keep,
                                  "mobile_pscore": "residual_energy", "mobile_pscore_weight": 1.0,
                                  "server_pscore_weight": 0.0, "pscore_fusion": "add"})
    ex = DINOv3ClassifierExecutor(dev)
    ex.load_model(config.model_name, config)

    # Synthetic tokens: base ~ N(0,1); full-res = base + delta on patch rows, delta ~ Laplace(0,1).
    g = torch.Generator(device=dev).manual_seed(1)
    x_base = torch.randn(B, N, C, generator=g, device=dev)
    # u uniform on the open interval (-1, 1) as torch.distributions.Laplace samples it: u = rand - 0.5
    # with log1p(-2|u|) gives -inf whenever rand returns exactly 0 (about once per 2^24 draws, i.e.
    # about once in this 16.7M-element tensor), which turns a whole image into NaN downstream.
    eps = torch.finfo(torch.float32).eps
    u = torch.rand(B, P, C, generator=g, device=dev) * (2.0 - eps) + (eps - 1.0)
    delta = -torch.sign(u) * torch.log1p(-u.abs())
    if not bool(torch.isfinite(delta).all()):
        raise RuntimeError("bench: non-finite synthetic residual")
    x_full = x_base.clone()
    x_full[:, 5:] += delta
    context = {"input_tokens": x_base.to(torch.bfloat16).contiguous(),
               "rope_sincos": ex.model.rope_embed(H=grid, W=grid)}
    dind = torch.arange(N, device=dev).unsqueeze(0).expand(B, -1).contiguous()
    context["group_plans"] = {1: make_group_plan(dind, 5)}
    with torch.no_grad():
        if args.cache == "approx":
            ex.approx_forward({"layers": (0, depth)}, context, config)  # fills the K/V + residual caches
        else:
            # Random caches of the same shapes: the correction does the same work on any values. Used
            # for profiles, so that the only HIP kernels in the trace are the correction pass's.
            Dh = C // H
            context["cache_feature"] = {}
            for i in range(depth):
                context["cache_feature"][f"layer{i}_kv"] = torch.randn(B, N, 2, H, Dh, generator=g, device=dev).to(
                    torch.bfloat16)
                context["cache_feature"][f"layer{i}_blocks_out_sum"] = (
                    torch.randn(B, N, C, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    context["input_tokens"] = x_full.to(torch.bfloat16).contiguous()
    params = {"layers": (0, depth), "group_id": 1}

    def step():
        SelfAttentionBlock._invalidate_partial_token_derived_caches(context["cache_feature"])
        context["mobile_pscore_hint_map"] = K.patch_importance(delta)
        ex.correct_forward(params, context, config)

    with torch.no_grad():
        for _ in range(args.warmup):
            step()
        if args.calib_copy_mib > 0:
            # A plain copy of known size through the library's own row-copy kernel (16-byte lanes,
            # like the GEMM's operand loads): N MiB of 4 KiB rows. A 512 MiB fill in between evicts
            # the source from L2 and the MALL so every source byte comes from HBM.
            rows = (args.calib_copy_mib << 20) // 4096
            src = torch.ones(1, rows, 2048, device=dev, dtype=torch.bfloat16)
            torch.zeros(128 << 20, device=dev, dtype=torch.float32)
            K.gather_rows(src, torch.zeros(rows, device=dev, dtype=torch.long), torch.arange(rows, device=dev))
            torch.cuda.synchronize()
            del src
        torch.cuda.synchronize()
        roctx = _roctx()
        if roctx is not None:
            roctx.roctxProfilerResume(0)
        s = torch.cuda.current_stream()

        def timed(fn):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            w0 = time.perf_counter()
            a.record(s)
            for _ in range(args.steps):
                fn()
            b.record(s)
            torch.cuda.synchronize()
            return a.elapsed_time(b) / args.steps, time.perf_counter() - w0

        # Eager launches, with the probe on the roofline launch site.
        K.set_probe(args.probe)
        ms_eager, wall_eager = timed(step)
        events = K.probe_events()
        K.set_probe(None)
        ms, wall = ms_eager, wall_eager
        if args.graph:
            from appcorr_amd.graphs import capture

            replay = capture(step, dev, warmup=1)
            ms, wall = timed(replay)
        if roctx is not None:
            roctx.roctxProfilerPause(0)
        # The corrected tokens of the last timed pass must be finite (outside the timed region).
        out = context["current_feature"]
        if not bool(torch.isfinite(out.float()).all()):
            raise RuntimeError("bench: the correction pass produced non-finite tokens")
    value = B * k / (ms / 1e3)

    roof = None
    if events:
        durs = [a.elapsed_time(b) for a, b in events]
        avg_ms = sum(durs) / len(durs)
        amount, unit, bound = kernel_work(args.probe, B, T, N, C, H, mlp)
        achieved = amount / (avg_ms / 1e3)
        peak = PEAK_BF16_TFLOPS if bound == "mfma" else PEAK_HBM_GBS
        roof = {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                "frac": round(achieved / peak, 4), "traffic": None, "kernel": args.probe,
                "launches": len(durs), "avg_us": round(avg_ms * 1e3, 2)}
        # HBM bytes per launch of this kernel at this workload, from the committed rocprofv3
        # FETCH_SIZE / WRITE_SIZE summary (appcorr_amd.profiling traffic), when one exists.
        tkey = f"{args.probe}@{args.config}/b{B}/k{k}"
        tpath = os.path.join(ROOT, "profiles", "traffic.json")
        if os.path.exists(tpath):
            rec = json.load(open(tpath)).get(tkey)
            running = probe_kernel_name(args.probe, B, T, C, mlp)
            if rec and (running is None or rec["kernel"] == running):
                roof["traffic"] = rec["traffic_bytes"]
                roof["traffic_source"] = f"profiles/traffic.json[{tkey}] ({rec['kernel']})"
            elif rec:
                roof["traffic_source"] = (f"profiles/traffic.json[{tkey}] was measured on {rec['kernel']}, "
                                          f"this build runs {running}: not used")

    cpu = None
    if args.cpu_budget > 0:
        cpu = cpu_baseline(args.config, B, args.keep, args.cpu_budget)
    flops = depth * (2 * B * T * C * (3 * C + C + 2 * mlp) + 4 * B * H * T * N * (C // H))
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "corrected tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"dinov3_{args.config}_correction", "batch": B, "tokens_per_image": N,
                   "keep_ratio": args.keep, "k": k, "selected_rows": B * T, "blocks": depth,
                   "pass_tflop": round(flops / 1e12, 4), "pass_tflops_achieved": round(flops / (ms / 1e3) / 1e12, 1),
                   "wall_ms_per_step": round(wall * 1e3 / args.steps, 4),
                   "launch": "hip_graph" if args.graph else "eager",
                   "eager_ms_per_step": round(ms_eager, 4)},
        "roofline": roof, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
