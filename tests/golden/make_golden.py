"""Writes the committed golden fixtures under tests/golden/ from the CPU oracle.

The reference ships no tensor fixtures for this path and cannot run here (it needs a CUDA Triton
runtime, nvtx and torchao), so these vectors come from the oracle, whose functions are pinned in
tests/test_oracle_*.py. The fixtures freeze those pinned outputs: the GPU tests compare the HIP
library against them directly, and tests/test_golden.py checks that the oracle still reproduces them.

    python tests/golden/make_golden.py        # rewrites the .npz files (deterministic)
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import model as OM  # noqa: E402
from oracle import nvfp4 as Q  # noqa: E402
from oracle import plan as OP  # noqa: E402
from oracle import rows as OR  # noqa: E402
from oracle.bf16 import f32_to_bf16_bits, torch_bf16_to_bits  # noqa: E402

# ------------------------------------------------------------------------------------------------
# Top-k plan: ties, -inf candidates, NaN, k in {0, 1, P/4, P-1, P}, a candidate subset
# ------------------------------------------------------------------------------------------------


def topk_cases():
    rng = np.random.default_rng(10)
    cases = []
    B, P, pre = 3, 200, 5
    s = rng.standard_normal((B, P)).astype(np.float32)
    s[0, 10:30] = 0.5          # a run of ties
    s[1, ::7] = -np.inf        # masked candidates (block.py:1033-1037)
    s[2, 3] = np.nan
    s[2, 50:60] = -0.0
    s[2, 60:70] = 0.0
    dind = np.tile(np.arange(pre + P), (B, 1)).astype(np.int64)
    for k in (0, 1, 50, 199, 200):
        cases.append((f"full_k{k}", s, dind, pre, pre + P, k))
    # candidate subset: a group holding every third patch token of a 600-patch image
    P2 = 160
    s2 = np.round(rng.standard_normal((2, P2)) * 4).astype(np.float32) / 4  # heavy ties
    toks = pre + 3 * np.arange(P2)
    dind2 = np.tile(np.concatenate([np.arange(pre), toks]), (2, 1)).astype(np.int64)
    cases.append(("subset_k40", s2, dind2, pre, pre + 600, 40))
    return cases


def make_topk():
    out = {}
    for name, s, dind, pre, N, k in topk_cases():
        p = OP.build_plan(s, k, dind, pre, N)
        out[f"{name}/scores"] = s
        out[f"{name}/dindice"] = dind
        out[f"{name}/meta"] = np.array([pre, N, k], dtype=np.int64)
        for f in ("update_indice", "active_batch_idx", "active_pos_idx", "active_token_idx", "active_patch_mask",
                  "active_rope_idx", "keep_mask", "row_slot"):
            out[f"{name}/{f}"] = getattr(p, f)
    np.savez_compressed(os.path.join(HERE, "topk_plan.npz"), **out)


# ------------------------------------------------------------------------------------------------
# Rows: gather, scatter, reconstruct + scatter + persist (bf16 bit patterns)
# ------------------------------------------------------------------------------------------------


def make_rows():
    rng = np.random.default_rng(11)
    B, N, C, T = 3, 77, 192, 21
    x = f32_to_bf16_bits(rng.standard_normal((B, N, C)).astype(np.float32))
    bos = f32_to_bf16_bits((rng.standard_normal((B, N, C)) * 0.1).astype(np.float32))
    b = np.repeat(np.arange(B), T).astype(np.int64)
    t = np.concatenate([np.sort(rng.choice(N, T, replace=False)) for _ in range(B)]).astype(np.int64)
    x_act = OR.gather_rows(x, b, t)
    x_attn = f32_to_bf16_bits(rng.standard_normal((B * T, C)).astype(np.float32))
    mlp = f32_to_bf16_bits((rng.standard_normal((B * T, C)) * 0.3).astype(np.float32))
    x_out, bos_new = OR.reconstruct_scatter_persist(x, bos, b, t, x_act, x_attn, mlp)
    kv = f32_to_bf16_bits(rng.standard_normal((B, N, 2, 3, 64)).astype(np.float32))
    kv_rows = f32_to_bf16_bits(rng.standard_normal((B * T, 2, 3, 64)).astype(np.float32))
    kv_new = OR.scatter_rows(kv, b, t, kv_rows)
    row_slot = np.full((B, N), -1, dtype=np.int32)
    row_slot[b, t] = np.arange(B * T, dtype=np.int32)
    np.savez_compressed(os.path.join(HERE, "rows.npz"), x=x, bos=bos, b=b, t=t, row_slot=row_slot, x_act=x_act,
                        x_attn=x_attn, mlp=mlp, x_out=x_out, bos_new=bos_new, kv=kv, kv_rows=kv_rows, kv_new=kv_new)


# ------------------------------------------------------------------------------------------------
# NVFP4: grid- and midpoint-valued blocks, a constant block, signed zeros, a masked tail
# ------------------------------------------------------------------------------------------------


def make_nvfp4():
    rng = np.random.default_rng(12)
    M, K = 200, 192  # 2 x 3 tiles, 72 padding rows in the last tile row
    x = rng.standard_normal((M, K)).astype(np.float32) * np.exp(rng.uniform(-3, 3, (M, 1))).astype(np.float32)
    grid = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], dtype=np.float32)
    x[0, :16] = np.concatenate([grid, -grid])                           # e2m1 grid values and their negatives
    x[1, :16] = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5, 6] * 2, dtype=np.float32)  # every e2m1 midpoint
    x[2, :16] = 3.0                                                      # constant block
    x[3, :16] = np.array([-0.0] * 15 + [6.0], dtype=np.float32)          # signed zeros
    xb = f32_to_bf16_bits(x)
    from oracle.bf16 import bf16_bits_to_f32

    xf = bf16_bits_to_f32(xb)
    ts = Q.per_tensor_amax_to_scale(float(np.abs(xf).max()))
    qdata, scales = Q.quantize(xf, ts)
    deq = f32_to_bf16_bits(Q.dequantize(qdata, scales, ts, M, K))
    np.savez_compressed(os.path.join(HERE, "nvfp4.npz"), x=xb, ts=np.array([ts], dtype=np.float32), qdata=qdata,
                        scales=scales, deq=deq)


# ------------------------------------------------------------------------------------------------
# One ViT-S correction block (B=1, 224 px, keep 50 %), stress weights: inputs from seeds, outputs stored
# ------------------------------------------------------------------------------------------------

VITS_SEED = 0


def vits_block_weights():
    cfg = OM.CONFIGS["vits16_224"]
    return cfg, OM.make_block_weights(cfg, VITS_SEED, gamma=1.0, bias_std=0.05, ln_std=0.1, depth=1)


def vits_block_inputs():
    cfg, weights = vits_block_weights()
    x_base, x_full, _, imp = OM.make_inputs(cfg, 1, VITS_SEED + 1)
    rope = OM.rope_tables(cfg)
    _, cache = OM.approx_pass(cfg, weights, x_base, rope)
    k = OP.keep_count(cfg.num_patches, 0.5)
    plan = OP.build_plan(imp.numpy(), k, OM.full_dindice(cfg, 1).numpy(), cfg.num_pretokens, cfg.num_tokens)
    return cfg, weights, x_full, imp, rope, cache, plan


def make_vits_block():
    cfg, weights, x_full, imp, rope, cache, plan = vits_block_inputs()
    cache_in = {k_: v.clone() for k_, v in cache.items()}
    x_out, cache_out = OM.correct_block(cfg, weights[0], x_full, plan, rope, cache_in, "layer0")
    np.savez_compressed(os.path.join(HERE, "vits_block.npz"),
                        x_in=torch_bf16_to_bits(x_full), kv_in=torch_bf16_to_bits(cache["layer0_kv"]),
                        bos_in=torch_bf16_to_bits(cache["layer0_blocks_out_sum"]),
                        importance=imp.numpy(), update_indice=plan.update_indice,
                        x_out=torch_bf16_to_bits(x_out), kv_out=torch_bf16_to_bits(cache_out["layer0_kv"]),
                        bos_out=torch_bf16_to_bits(cache_out["layer0_blocks_out_sum"]))


if __name__ == "__main__":
    make_topk()
    make_rows()
    make_nvfp4()
    make_vits_block()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
