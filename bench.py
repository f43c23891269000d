"""Benchmark: one DINOv3 token-correction pass on one MI355X.

Default workload (BASELINE.json metric "ms per correction pass + corrected tokens/s, ViT-L/16 512px, 25%
keep"): ViT-L/16 at 512 px, B=16 (1029 tokens per image), 24 blocks, bf16, random-init weights, top
25% of the 1024 patches per image (k=256) selected by importance = ||delta_p||_2 with
delta ~ Laplace(0,1). `--config` selects the other BASELINE shapes (ViT-S, ViT-B, ViT-7B at B=4, keep
10%) and `--keep` the sweep points. One step = one full correction pass through the executor API
(`DINOv3ClassifierExecutor.correct_forward`, i.e. `run_dinov3_correct_block` for every layer): the
importance reduction, the top-k plan (recomputed every pass) and all correction blocks. The K/V and
blocks_out_sum caches come from an untimed approximate pass over the base tokens.

Output: one JSON line on stdout. `value` = corrected tokens/s = B*k / pass time; `ms_per_step` = ms
per correction pass. The step is recorded once into a HIP graph and the timed steps are replays (every
kernel of the pass runs each step; `config.eager_ms_per_step` is the same K steps launched one kernel
at a time, `--graph 0` reports that instead).

`roofline` is for the dominant kernel: every MFMA launch site of the pass (qkv, proj, the MLP GEMMs,
attention) is timed with HIP events around each launch in separate eager steps, and the site with the
largest share of the pass is reported, with all sites under `roofline.sites`. `cpu_baseline` times the
CPU oracle (the reference's eager op sequence on bf16 CPU tensors) on the same inputs, weights and
caches as the GPU run, with one torch thread per CPU this process may run on.

Only one GPU is used: `--gpus N` with N > 1 exits with an explanation.
"""

from __future__ import annotations

import argparse
import ctypes
import json
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

# name: (backbone, embed, heads, ffn hidden, depth, img, ffn kind, default batch, default keep)
SHAPES = {
    "vits16_224": ("vits16", 384, 6, 1536, 12, 224, "mlp", 1, 0.5),
    "vitb16_512": ("vitb16", 768, 12, 3072, 12, 512, "mlp", 8, 0.25),
    "vitl16_512": ("vitl16", 1024, 16, 4096, 24, 512, "mlp", 16, 0.25),
    "vit7b16_1024": ("vit7b16", 4096, 32, 8192, 40, 1024, "swiglu", 4, 0.1),
}
MFMA_SITES = {"mlp": ("qkv", "proj", "fc1", "fc2", "attention"),
              "swiglu": ("qkv", "proj", "w1", "w2", "w3", "attention")}


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


def site_work(site: str, B: int, T: int, N: int, C: int, H: int, hid: int):
    """Algorithmic work of one launch at a site: (amount in TFLOP or GB, unit, bound)."""
    M = B * T
    flops = {"qkv": 2.0 * M * C * 3 * C, "proj": 2.0 * M * C * C, "fc1": 2.0 * M * C * hid,
             "fc2": 2.0 * M * hid * C, "w1": 2.0 * M * C * hid, "w2": 2.0 * M * C * hid,
             "w3": 2.0 * M * hid * C, "attention": 4.0 * B * H * T * N * (C // H)}
    if site in flops:
        return flops[site] / 1e12, "TFLOP/s", "mfma"
    if site == "packed_residual":  # read x_act, x_attn, mlp; write x_new, blocks_out_sum rows; row ids
        return (5.0 * M * C * 2 + 16.0 * M) / 1e9, "GB/s", "hbm"
    if site == "gather_rows":
        return (2.0 * M * C * 2 + 16.0 * M) / 1e9, "GB/s", "hbm"
    if site == "layernorm":
        return (2.0 * M * C * 2) / 1e9, "GB/s", "hbm"
    raise ValueError(site)


def site_kernel_name(site: str, B: int, T: int, C: int, hid: int):
    """Kernel a GEMM launch site runs in this build (None for other sites)."""
    from appcorr_amd import _lib
    from appcorr_amd import kernels as K

    M = B * T
    shapes = {"qkv": (M, 3 * C, C, 5), "proj": (M, C, C, _lib.EPI_BIAS_LS_RESID),
              "fc1": (M, hid, C, _lib.EPI_BIAS_GELU), "fc2": (M, C, hid, _lib.EPI_BIAS_LS),
              "w1": (M, hid, C, _lib.EPI_BIAS_SILU_MUL), "w2": (M, hid, C, _lib.EPI_BIAS),
              "w3": (M, C, hid, _lib.EPI_BIAS_LS)}
    if site not in shapes:
        return None
    return K.linear_kernel_name(*shapes[site])


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(name: str, blocks, x_full, caches, hint, k: int, budget_s: float):
    """The oracle (the reference's eager op sequence on bf16 CPU tensors, with the top-k plan) on the
    GPU run's own weights, layer-0 tokens, K/V + blocks_out_sum caches and importance scores, one torch
    thread per CPU this process may run on (nproc). 3 warm-up and 10 timed passes, median; when 13
    passes would exceed `budget_s`, the same over the first n blocks, scaled to the full depth."""
    import torch

    from oracle import model as OM
    from oracle import plan as OP

    nproc = len(os.sched_getaffinity(0))
    torch.set_num_threads(nproc)
    cfg = OM.CONFIGS[name]
    B, N = x_full.shape[0], x_full.shape[1]
    dind = OM.full_dindice(cfg, B).numpy()
    depth = len(blocks)

    rope = OM.rope_tables(cfg)

    def run(n_blk):
        cache = dict(caches)
        t0 = time.perf_counter()
        plan = OP.build_plan(hint.numpy(), k, dind, cfg.num_pretokens, N)
        x = x_full
        with torch.no_grad():
            for i in range(n_blk):
                x, cache = OM.correct_block(cfg, blocks[i], x, plan, rope, cache, f"layer{i}", mode="bf16")
        return time.perf_counter() - t0

    run(1)  # one block: warm-up (first-call costs of the CPU kernels)
    t1 = run(1)
    n_blk = depth if 13 * t1 * depth <= budget_s else max(1, int(budget_s / (13 * t1)))
    n_blk = min(n_blk, depth)
    for _ in range(3):
        run(n_blk)
    times = [run(n_blk) for _ in range(10)]
    med = statistics.median(times)
    pass_s = med * depth / n_blk
    what = "full passes" if n_blk == depth else f"the first {n_blk} of {depth} blocks (+ the plan), scaled x{depth / n_blk:g}"
    return {
        "value": B * k / pass_s,
        "unit": "corrected tokens/s",
        "cores": nproc,
        "kind": "port",
        "sample": (f"{name} B={B} k={k}, the GPU run's weights, tokens, caches and importance; bf16 torch CPU eager "
                   f"ops ({what}), 3 warm-up + 10 timed, median {med * 1e3:.1f} ms -> {pass_s * 1e3:.0f} ms per pass"),
        "ms_per_pass": round(pass_s * 1e3, 2),
        "cpu_model": _cpu_model(),
        "os_cpu_count": os.cpu_count(),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="vitl16_512", choices=sorted(SHAPES))
    ap.add_argument("--batch", type=int, default=None, help="images per pass (default: the config's)")
    ap.add_argument("--keep", type=float, default=None, help="token keep ratio (default: the config's)")
    ap.add_argument("--precision", default="bf16", help="correct_precision of the executor")
    ap.add_argument("--cpu-budget", type=float, default=45.0,
                    help="seconds of CPU-baseline sampling (0 = skip); full passes whenever 13 of them fit")
    ap.add_argument("--cache", default="approx", choices=("approx", "random"),
                    help="fill the K/V + residual caches with the approximate pass (default) or random values")
    ap.add_argument("--graph", type=int, default=1,
                    help="1: record the step into a HIP graph and time its replays (the eager time is reported "
                         "alongside); 0: time eager launches only")
    ap.add_argument("--probe", type=int, default=1, help="1: time every MFMA launch site in extra eager steps")
    ap.add_argument("--approx-steps", type=int, default=0,
                    help="after the correction timing, time this many approximate passes (the cache producer, "
                         "eager launches) with --approx-pscore as the server score; reported under approx_pass")
    ap.add_argument("--approx-pscore", default="patch_attn_prob_layermean",
                    help="server_pscore of the timed approximate passes (weight 1)")
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
    bb, C, H, hid, depth, img, ffn, b_dflt, keep_dflt = SHAPES[args.config]
    B = args.batch or b_dflt
    keep = keep_dflt if args.keep is None else args.keep
    grid = img // 16
    P = grid * grid
    N = 5 + P
    k = min(int(P * keep), P)
    T = 5 + k

    config = ExperimentConfig(model_name=f"dinov3_classifier_{bb}", batch_size=B, image_shape=(img, img, 3),
                              backbone=bb, correct_precision=args.precision, appcorr_kwargs={
                                  "method": "partial_token", "token_keep_ratio": keep,
                                  "mobile_pscore": "residual_energy", "mobile_pscore_weight": 1.0,
                                  "server_pscore_weight": 0.0, "pscore_fusion": "add"})
    ex = DINOv3ClassifierExecutor(dev)
    ex.load_model(config.model_name, config)

    # Synthetic tokens: base ~ N(0,1); full-res = base + delta on patch rows, delta ~ Laplace(0,1).
    g = torch.Generator(device=dev).manual_seed(1)
    x_base = torch.randn(B, N, C, generator=g, device=dev)
    # u uniform on the open interval (-1, 1) as torch.distributions.Laplace samples it: u = rand - 0.5
    # with log1p(-2|u|) gives -inf whenever rand returns exactly 0 (about once per 2^24 draws, i.e.
    # about once in a 16.7M-element tensor), which turns a whole image into NaN downstream.
    eps = torch.finfo(torch.float32).eps
    u = torch.rand(B, P, C, generator=g, device=dev) * (2.0 - eps) + (eps - 1.0)
    delta = -torch.sign(u) * torch.log1p(-u.abs())
    del u
    if not bool(torch.isfinite(delta).all()):
        raise RuntimeError("bench: non-finite synthetic residual")
    x_full = x_base.clone()
    x_full[:, 5:] += delta
    context = {"input_tokens": x_base.to(torch.bfloat16).contiguous(),
               "rope_sincos": ex.model.rope_embed(H=grid, W=grid)}
    del x_base
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
    del x_full
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

        def timed(fn, steps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            w0 = time.perf_counter()
            a.record(s)
            for _ in range(steps):
                fn()
            b.record(s)
            torch.cuda.synchronize()
            return a.elapsed_time(b) / steps, time.perf_counter() - w0

        ms_eager, wall_eager = timed(step, args.steps)
        ms, wall = ms_eager, wall_eager
        if args.graph:
            from appcorr_amd.graphs import capture

            replay = capture(step, dev, warmup=1)
            ms, wall = timed(replay, args.steps)
        if roctx is not None:
            roctx.roctxProfilerPause(0)
        # Per-site launch times, in eager steps of their own (the events do not touch the timed steps).
        events = {}
        if args.probe:
            K.set_probe(MFMA_SITES[ffn])
            timed(step, max(3, args.steps // 4))
            events = K.probe_events()
            K.set_probe(None)
        # The corrected tokens of the last pass must be finite (outside the timed region).
        out = context["current_feature"]
        if not bool(torch.isfinite(out.float()).all()):
            raise RuntimeError("bench: the correction pass produced non-finite tokens")
        # The approximate pass (every token through every block, caching K/V, the residual sums and the
        # server score), timed on its own context so the correction's caches stay as they are.
        approx = None
        if args.approx_steps > 0:
            akw = dict(config.appcorr_kwargs)
            akw.update(server_pscore=args.approx_pscore, server_pscore_weight=1.0)
            aconfig = ExperimentConfig(model_name=config.model_name, batch_size=B, image_shape=config.image_shape,
                                       backbone=bb, correct_precision=args.precision, appcorr_kwargs=akw)
            actx = {"input_tokens": context["input_tokens"], "rope_sincos": context["rope_sincos"],
                    "group_plans": context["group_plans"]}

            def astep():
                ex.approx_forward({"layers": (0, depth)}, actx, aconfig)

            astep()
            ams, _ = timed(astep, args.approx_steps)
            approx = {"ms_per_pass": round(ams, 4), "server_pscore": args.approx_pscore, "steps": args.approx_steps,
                      "launch": "eager", "tokens_per_s": round(B * N / (ams / 1e3), 1)}
            del actx
    value = B * k / (ms / 1e3)

    roof = None
    if events:
        sites = {}
        probe_steps = max(3, args.steps // 4)
        for site, evs in events.items():
            durs = [a.elapsed_time(b) for a, b in evs]
            avg_ms = sum(durs) / len(durs)
            amount, unit, bound = site_work(site, B, T, N, C, H, hid)
            achieved = amount / (avg_ms / 1e3)
            peak = PEAK_BF16_TFLOPS if bound == "mfma" else PEAK_HBM_GBS
            per_pass = len(durs) / probe_steps
            sites[site] = {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                           "frac": round(achieved / peak, 4), "avg_us": round(avg_ms * 1e3, 2),
                           "launches_per_pass": per_pass,
                           "share_of_pass": round(avg_ms * per_pass / ms, 4)}
        dom = max(sites, key=lambda x: sites[x]["avg_us"] * sites[x]["launches_per_pass"])
        roof = dict(sites[dom])
        roof.update({"kernel": dom, "traffic": None})
        # HBM bytes per launch of this kernel at this workload, from the committed rocprofv3
        # FETCH_SIZE / WRITE_SIZE summary (appcorr_amd.profiling traffic), when one exists.
        tkey = f"{dom}@{args.config}/b{B}/k{k}"
        tpath = os.path.join(ROOT, "profiles", "traffic.json")
        if os.path.exists(tpath):
            rec = json.load(open(tpath)).get(tkey)
            running = site_kernel_name(dom, B, T, C, hid)
            if rec and (running is None or rec["kernel"] == running):
                roof["traffic"] = rec["traffic_bytes"]
                roof["traffic_source"] = f"profiles/traffic.json[{tkey}] ({rec['kernel']})"
            elif rec:
                roof["traffic_source"] = (f"profiles/traffic.json[{tkey}] was measured on {rec['kernel']}, "
                                          f"this build runs {running}: not used")
        roof["sites"] = {kk: {f: v[f] for f in ("achieved", "frac", "avg_us", "launches_per_pass", "share_of_pass")}
                         for kk, v in sites.items()}
        roof["timing"] = ("HIP events recorded on the launch stream around every launch of each site, in eager "
                          "probe steps after the timed replays; avg_us is the mean bracket, a few us above the "
                          "kernel's own duration (rocprofv3 kernel trace)")

    cpu = None
    if args.cpu_budget > 0:
        from oracle.model import CONFIGS

        cfg_name = next(n for n in CONFIGS if n == args.config)
        blocks = []
        for blk in ex.model.blocks:
            blocks.append({kk: v.detach().to("cpu") for kk, v in blk.state_dict().items()})
        caches = {kk: v.to("cpu") for kk, v in context["cache_feature"].items()
                  if isinstance(v, torch.Tensor) and (kk.endswith("_kv") or kk.endswith("_blocks_out_sum"))}
        cpu = cpu_baseline(cfg_name, blocks, context["input_tokens"].cpu(), caches,
                           context["mobile_pscore_hint_map"].cpu(), k, args.cpu_budget)
    attn_flops = 4 * B * H * T * N * (C // H)
    gemm_flops = 2 * B * T * C * (4 * C + (2 if ffn == "mlp" else 3) * hid)
    flops = depth * (gemm_flops + attn_flops)
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "corrected tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"dinov3_{args.config}_correction", "batch": B, "tokens_per_image": N,
                   "keep_ratio": keep, "k": k, "selected_rows": B * T, "blocks": depth,
                   "correct_precision": args.precision,
                   "pass_tflop": round(flops / 1e12, 4), "pass_tflops_achieved": round(flops / (ms / 1e3) / 1e12, 1),
                   "wall_ms_per_step": round(wall * 1e3 / args.steps, 4),
                   "launch": "hip_graph" if args.graph else "eager",
                   "eager_ms_per_step": round(ms_eager, 4)},
        "roofline": roof, "cpu_baseline": cpu,
    }
    if approx is not None:
        line["approx_pass"] = approx
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
