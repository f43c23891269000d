"""Standalone timings of the HBM-bound kernels of the correction path at the BASELINE shapes.

    python -m appcorr_amd.kernel_bench [--iters N] [--only name,name]
    python -m appcorr_amd.kernel_bench --gemm      (the pass GEMM shapes, this build vs torch F.linear)

One JSON line per kernel and shape: microseconds per launch (a HIP graph of back-to-back launches
replayed between two events, inputs resident in HBM and rotated over copies that together exceed
twice the 256 MB last-level cache), algorithmic bytes per launch, achieved GB/s and the fraction of
MI355X's 8 TB/s HBM peak. Rows (the standalone parts of the hot path):
  * nvfp4_quantize / nvfp4_dequantize at [16464, 1024] and [16464, 4096] bf16 (
    N(0, 1) with 1 % of the entries scaled by 50; tensor scale amax / (448 * 6) as the reference's
    test takes it, tests/test_nvfp4_fused_quantize.py:48);
  * gather_rows: the selected rows of x [16, 1029, 1024] (M = 4176, k = 256), once per pass;
  * scatter_rows: the K/V rewrite of 4176 rows of 2 * 16 * 64 into the [16, 1029, 2, 16, 64] cache
    (the unfused form; the headline pass writes K/V from the QKV GEMM's epilogue).
The corrected-token throughput of the whole pass is bench.py's; this module only times kernels.
"""

from __future__ import annotations

import argparse
import json
import statistics

import torch

from . import _lib
from . import kernels as K

PEAK_HBM_GBS = 8000.0


ROTATE_BYTES = 640 << 20  # > 2x the 256 MB last-level cache: every launch reads data no cache holds


def _copies(nbytes: int) -> int:
    """Input copies to rotate over so that one pass over them exceeds ROTATE_BYTES."""
    return max(2, -(-ROTATE_BYTES // max(1, nbytes)))


def _time(fns, iters: int) -> float:
    """Microseconds of one launch: one launch per input copy (`fns`, rotating over copies whose total
    size exceeds twice the last-level cache, so inputs come from HBM) recorded into a HIP graph, the
    graph replayed `iters` times between two events (no host launch gaps), median over five runs."""
    fns = list(fns)
    for fn in fns:
        fn()
    torch.cuda.synchronize()
    per_graph = len(fns)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for fn in fns:
            fn()
    g.replay()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    runs = []
    for _ in range(5):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(s)
        for _ in range(iters):
            g.replay()
        b.record(s)
        torch.cuda.synchronize()
        runs.append(a.elapsed_time(b) * 1e3 / (iters * per_graph))
    return statistics.median(runs)


def _line(name: str, shape, us: float, nbytes: float, extra=None) -> dict:
    gbs = nbytes / (us * 1e-6) / 1e9
    d = {"kernel": name, "shape": list(shape), "us": round(us, 2), "bytes": int(nbytes), "GB_per_s": round(gbs, 1),
         "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)}
    if extra:
        d.update(extra)
    return d


def nvfp4_input(M: int, Kd: int, device, seed: int = 0) -> torch.Tensor:
    """N(0, 1) bf16 with 1 % of the entries (random positions) scaled by 50."""
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(M, Kd, generator=g, device=device)
    mask = torch.rand(M, Kd, generator=g, device=device) < 0.01
    x = torch.where(mask, x * 50.0, x)
    return x.to(torch.bfloat16).contiguous()


def run(iters: int = 10, only=None) -> list[dict]:
    dev = torch.device("cuda", 0)
    out = []
    want = (lambda n: only is None or n in only)
    for (M, Kd) in ((16464, 1024), (16464, 4096)):
        x = nvfp4_input(M, Kd, dev)
        ts = (x.float().abs().amax() / (448.0 * 6.0)).reshape(1).to(torch.float32)
        nsc = K.nvfp4_scale_numel(M, Kd)
        nbytes = M * Kd * 2 + M * Kd // 2 + nsc + 4
        xs = [x] + [x.clone() for _ in range(_copies(nbytes) - 1)]
        if want("nvfp4_quantize"):
            us = _time([(lambda xi=xi: K.quantize_nvfp4_swizzled(xi, ts)) for xi in xs], iters)
            out.append(_line("nvfp4_quantize", (M, Kd), us, nbytes, {"copies": len(xs)}))
        if want("nvfp4_dequantize"):
            qs = [K.quantize_nvfp4_swizzled(xi, ts) for xi in xs]
            us = _time([(lambda q=q, sc=sc: K.dequantize_nvfp4(q, sc, ts)) for q, sc in qs], iters)
            out.append(_line("nvfp4_dequantize", (M, Kd), us, nbytes, {"copies": len(qs)}))
            del qs
        del x, xs
    if want("copy_reference") or want("write_reference") or want("read_reference"):
        # The practical streaming ceiling: torch's device copy of 512 MiB (read + write), same timing.
        nb = 512 << 20
        srcs = [torch.empty(nb // 2, device=dev, dtype=torch.bfloat16).fill_(1.0) for _ in range(2)]
        dsts = [torch.empty_like(srcs[0]) for _ in range(2)]
        us = _time([(lambda a=a, b=b: b.copy_(a)) for a, b in zip(srcs, dsts)], max(2, iters // 4))
        out.append(_line("copy_reference", (nb,), us, 2 * nb, {"note": "torch device copy, 512 MiB"}))
        us = _time([(lambda b=b: b.fill_(2.0)) for b in dsts], max(2, iters // 4))
        out.append(_line("write_reference", (nb,), us, nb, {"note": "torch fill, 512 MiB"}))
        sums = torch.empty(2, device=dev, dtype=torch.float32)
        us = _time([(lambda a=a, i=i: torch.sum(a, dim=(0,), dtype=torch.float32, out=sums[i])) for i, a in enumerate(srcs)],
                   max(2, iters // 4))
        out.append(_line("read_reference", (nb,), us, nb, {"note": "torch sum, 512 MiB"}))
        del srcs, dsts, sums
    for (M, Kd) in ((1656, 4096),):  # the ViT-7B fp4 pass's activation quantize-dequantize (x-hat only)
        if not want("nvfp4_qdq"):
            break
        x = nvfp4_input(M, Kd, dev)
        ts = (x.float().abs().amax() / (448.0 * 6.0)).reshape(1).to(torch.float32)
        nbytes = 2 * M * Kd * 2
        xs = [x] + [x.clone() for _ in range(_copies(nbytes) - 1)]
        us = _time([(lambda xi=xi: K.nvfp4_quantize_dequantize(xi, ts)) for xi in xs], iters)
        out.append(_line("nvfp4_qdq", (M, Kd), us, nbytes, {"copies": len(xs)}))
        del x, xs
    for (M, C) in ((4176, 1024), (1656, 4096)):  # norm2 of the ViT-L / ViT-7B passes
        if not want("layernorm_rows"):
            break
        nbytes = 2 * M * C * 2
        xs = [torch.randn(M, C, device=dev).to(torch.bfloat16) for _ in range(_copies(nbytes))]
        w = torch.randn(C, device=dev).to(torch.bfloat16)
        b = torch.randn(C, device=dev).to(torch.bfloat16)
        outs = [torch.empty(M, C, device=dev, dtype=torch.bfloat16) for _ in range(2)]
        us = _time([(lambda xi=xi, i=i: K.layer_norm(xi, w, b, 1e-6, out=outs[i % 2])) for i, xi in enumerate(xs)],
                   iters)
        out.append(_line("layernorm_rows", (M, C), us, nbytes, {"copies": len(xs)}))
        del xs, outs
    B, N, C, H, Dh, k = 16, 1029, 1024, 16, 64, 256
    T = 5 + k
    g = torch.Generator(device=dev).manual_seed(1)
    bi = torch.arange(B, device=dev).repeat_interleave(T)
    ti = torch.stack([torch.cat([torch.arange(5, device=dev),
                                 5 + torch.randperm(N - 5, generator=g, device=dev)[:k].sort().values])
                      for _ in range(B)]).reshape(-1)
    n = bi.numel()
    if want("gather_rows"):
        nbytes = 2 * n * C * 2 + 16 * n
        src = [torch.randn(B, N, C, generator=g, device=dev).to(torch.bfloat16) for _ in range(_copies(B * N * C * 2))]
        us = _time([(lambda s_=s_: K.gather_rows(s_, bi, ti)) for s_ in src], iters)
        out.append(_line("gather_rows", (n, C), us, nbytes, {"copies": len(src)}))
        del src
    if want("scatter_rows"):
        nbytes = 2 * n * 2 * H * Dh * 2 + 16 * n
        kvs = [torch.randn(B, N, 2, H, Dh, generator=g, device=dev).to(torch.bfloat16)
               for _ in range(_copies(B * N * 2 * H * Dh * 2))]
        rows = torch.randn(n, 2, H, Dh, generator=g, device=dev).to(torch.bfloat16)
        us = _time([(lambda kv=kv: K.scatter_rows(kv, bi, ti, rows)) for kv in kvs], iters)
        out.append(_line("scatter_rows", (n, 2 * H * Dh), us, nbytes, {"copies": len(kvs)}))
        del kvs
    return out


# The GEMMs of the correction pass: (site, M, N, K, epilogue of the pass) -- ViT-L/16 512 px, B = 16,
# keep 25 % (M = 4176) and ViT-7B at 1024 px, B = 4, keep 10 % (M = 1656; w1 / w2 as one 16384-wide
# product are two 8192-wide products here, as the pass runs them).
GEMM_SHAPES = (
    ("vitl16 qkv", 4176, 3072, 1024, _lib.EPI_BIAS),
    ("vitl16 proj", 4176, 1024, 1024, _lib.EPI_BIAS_LS_RESID),
    ("vitl16 fc1", 4176, 4096, 1024, _lib.EPI_BIAS_GELU),
    ("vitl16 fc2", 4176, 1024, 4096, _lib.EPI_BIAS_LS),
    ("vit7b16 qkv", 1656, 12288, 4096, _lib.EPI_BIAS),
    ("vit7b16 proj", 1656, 4096, 4096, _lib.EPI_BIAS_LS_RESID),
    ("vit7b16 w1", 1656, 8192, 4096, _lib.EPI_BIAS),
    ("vit7b16 w3", 1656, 4096, 8192, _lib.EPI_BIAS_LS),
)


def run_gemms(iters: int = 10) -> list[dict]:
    """Each pass GEMM shape with this build's kernel (the pass's epilogue) and with torch's
    F.linear (hipBLASLt / rocBLAS, bias epilogue only) on the same bf16 operands, same timing."""
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(3)
    out = []
    for name, M, N, Kd, epi in GEMM_SHAPES:
        a = torch.randn(M, Kd, generator=g, device=dev).to(torch.bfloat16)
        w = (torch.randn(N, Kd, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        bias = (torch.randn(N, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        gamma = torch.full((N,), 0.5, device=dev, dtype=torch.bfloat16)
        resid = torch.randn(M, N, generator=g, device=dev).to(torch.bfloat16) if epi == _lib.EPI_BIAS_LS_RESID else None
        c = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
        ours = _time([lambda: K.linear(a, w, bias, epilogue=epi, gamma=gamma, resid=resid, out=c)], iters)
        lib = _time([lambda: torch.nn.functional.linear(a, w, bias)], iters)
        flop = 2.0 * M * N * Kd
        out.append({"kernel": "gemm", "site": name, "M": M, "N": N, "K": Kd, "epilogue": epi,
                    "ours_us": round(ours, 2), "library_us": round(lib, 2),
                    "ours_tflops": round(flop / ours / 1e6, 1), "library_tflops": round(flop / lib / 1e6, 1)})
        del a, w, bias, gamma, resid, c
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--iters", type=int, default=10, help="graph replays per timing run")
    ap.add_argument("--only", default=None, help="comma-separated kernel names")
    ap.add_argument("--gemm", action="store_true",
                    help="time the pass GEMM shapes against torch's F.linear (hipBLASLt) instead")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="end with a plain copy of this many MiB through gather_rows (4 KiB rows, source "
                         "evicted from the caches first): the calibration dispatch for HBM byte counters")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("kernel_bench needs a GPU")
    _lib.verify_runtime(0)
    only = set(args.only.split(",")) if args.only else None
    with torch.no_grad():
        for d in (run_gemms(args.iters) if args.gemm else run(args.iters, only)):
            print(json.dumps(d), flush=True)
        if args.calib_copy_mib > 0:
            dev = torch.device("cuda", 0)
            rows = (args.calib_copy_mib << 20) // 4096
            src = torch.ones(1, rows, 2048, device=dev, dtype=torch.bfloat16)
            torch.zeros(128 << 20, device=dev, dtype=torch.float32)  # 512 MiB: evicts src from L2 and the MALL
            K.gather_rows(src, torch.zeros(rows, device=dev, dtype=torch.long), torch.arange(rows, device=dev))
            torch.cuda.synchronize()


if __name__ == "__main__":
    main()
