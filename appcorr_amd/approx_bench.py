"""Timing of the approximate pass alone (the cache producer of the correction pass).

    python -m appcorr_amd.approx_bench [--config vitl16_512] [--passes 3] [--warmup 1]
                                       [--pscore cls_attn_prob] [--batch B] [--img PIXELS]

`DINOv3ClassifierExecutor.approx_forward` over all blocks (dinov3_classifier.py:547-589): every token
through every block, caching each block's K/V (after RoPE), its residual sum and the server score
named by --pscore (weight 1). Random-init weights of the named backbone, synthetic N(0, 1) tokens,
eager launches. Prints one JSON line: ms per pass (HIP events around the timed passes) and tokens/s.
Only approximate passes run on the GPU after set-up, so `rocprofv3 --kernel-trace --stats` of this
command gives the pass's kernel time (`python -m appcorr_amd.profiling kernel-stats` with
--warmup + --passes passes).
"""

from __future__ import annotations

import argparse
import json

import torch

from . import _lib
from .server.dinov3_classifier import DINOv3ClassifierExecutor, make_group_plan
from .server.protocol import ExperimentConfig

# backbone, image size, default batch: the BASELINE configurations
CONFIGS = {
    "vits16_224": ("vits16", 224, 1),
    "vitb16_512": ("vitb16", 512, 8),
    "vitl16_512": ("vitl16", 512, 16),
    "vit7b16_1024": ("vit7b16", 1024, 4),
}


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="vitl16_512", choices=sorted(CONFIGS))
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--img", type=int, default=None, help="image size in pixels (default: the config's)")
    ap.add_argument("--passes", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--pscore", default="cls_attn_prob", help="server_pscore cached by every block (weight 1)")
    args = ap.parse_args(argv)

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _lib.verify_runtime(0)
    bb, img, b_dflt = CONFIGS[args.config]
    img = args.img or img
    B = args.batch or b_dflt
    grid = img // 16
    config = ExperimentConfig(model_name=f"dinov3_classifier_{bb}", batch_size=B, image_shape=(img, img, 3),
                              backbone=bb, correct_precision="bf16", appcorr_kwargs={
                                  "method": "partial_token", "server_pscore": args.pscore,
                                  "server_pscore_weight": 1.0})
    ex = DINOv3ClassifierExecutor(dev)
    ex.load_model(config.model_name, config)
    C = ex.model.blocks[0].norm1.weight.numel()
    depth = len(ex.model.blocks)
    N = 5 + grid * grid
    g = torch.Generator(device=dev).manual_seed(1)
    ctx = {"input_tokens": torch.randn(B, N, C, generator=g, device=dev).to(torch.bfloat16),
           "rope_sincos": ex.model.rope_embed(H=grid, W=grid)}
    dind = torch.arange(N, device=dev).unsqueeze(0).expand(B, -1).contiguous()
    ctx["group_plans"] = {1: make_group_plan(dind, 5)}
    params = {"layers": (0, depth)}

    with torch.no_grad():
        for _ in range(args.warmup):
            ex.approx_forward(params, ctx, config)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(args.passes):
            ex.approx_forward(params, ctx, config)
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / args.passes
    key = f"layer{depth - 1}_server_pscore"
    score = ctx["cache_feature"].get(key)
    if score is None or not bool(torch.isfinite(score.float()).all()):
        raise RuntimeError("approx_bench: the pass did not cache a finite server score")
    print(json.dumps({"workload": f"dinov3_{bb}_{img}_approx", "batch": B, "tokens_per_image": N,
                      "blocks": depth, "server_pscore": args.pscore, "passes": args.passes,
                      "warmup": args.warmup, "ms_per_pass": round(ms, 4),
                      "tokens_per_s": round(B * N / (ms / 1e3), 1), "launch": "eager"}), flush=True)


if __name__ == "__main__":
    main()
