"""The oracle reproduces the committed golden fixtures (tests/golden/*.npz) bit-for-bit (CPU).

The fixtures freeze the oracle's pinned outputs; this test fails if a change to the oracle moves any
of them, and the GPU tests in test_gpu_golden.py compare the HIP library against the same files.
"""

import os
import sys

import numpy as np

from oracle import model as OM
from oracle import nvfp4 as Q
from oracle import plan as OP
from oracle import rows as OR
from oracle.bf16 import bf16_bits_to_f32, bits_to_torch_bf16, f32_to_bf16_bits, torch_bf16_to_bits

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_golden  # noqa: E402


def load(name):
    return np.load(os.path.join(GOLDEN, name))


def test_topk_plan_fixture():
    z = load("topk_plan.npz")
    names = sorted({k.split("/")[0] for k in z.files})
    assert len(names) == 6
    for name in names:
        pre, N, k = z[f"{name}/meta"].tolist()
        p = OP.build_plan(z[f"{name}/scores"], k, z[f"{name}/dindice"], pre, N)
        for f in ("update_indice", "active_batch_idx", "active_pos_idx", "active_token_idx", "active_patch_mask",
                  "active_rope_idx", "keep_mask", "row_slot"):
            np.testing.assert_array_equal(getattr(p, f), z[f"{name}/{f}"], err_msg=f"{name}/{f}")


def test_rows_fixture():
    z = load("rows.npz")
    b, t = z["b"], z["t"]
    np.testing.assert_array_equal(OR.gather_rows(z["x"], b, t), z["x_act"])
    xo, nb = OR.reconstruct_scatter_persist(z["x"], z["bos"], b, t, z["x_act"], z["x_attn"], z["mlp"])
    np.testing.assert_array_equal(xo, z["x_out"])
    np.testing.assert_array_equal(nb, z["bos_new"])
    np.testing.assert_array_equal(OR.scatter_rows(z["kv"], b, t, z["kv_rows"]), z["kv_new"])


def test_nvfp4_fixture():
    z = load("nvfp4.npz")
    x = bf16_bits_to_f32(z["x"])
    ts = float(z["ts"][0])
    q, s = Q.quantize(x, ts)
    np.testing.assert_array_equal(q, z["qdata"])
    np.testing.assert_array_equal(s, z["scales"])
    M, K = x.shape
    np.testing.assert_array_equal(f32_to_bf16_bits(Q.dequantize(q, s, ts, M, K)), z["deq"])


def test_vits_block_fixture():
    z = load("vits_block.npz")
    cfg, weights, x_full, imp, rope, cache, plan = make_golden.vits_block_inputs()
    np.testing.assert_array_equal(torch_bf16_to_bits(x_full), z["x_in"])
    np.testing.assert_array_equal(torch_bf16_to_bits(cache["layer0_kv"]), z["kv_in"])
    np.testing.assert_array_equal(imp.numpy(), z["importance"])
    cache_in = {"layer0_kv": bits_to_torch_bf16(z["kv_in"]), "layer0_blocks_out_sum": bits_to_torch_bf16(z["bos_in"])}
    x_out, c = OM.correct_block(cfg, weights[0], bits_to_torch_bf16(z["x_in"]), plan, rope, cache_in, "layer0")
    np.testing.assert_array_equal(torch_bf16_to_bits(x_out), z["x_out"])
    np.testing.assert_array_equal(torch_bf16_to_bits(c["layer0_kv"]), z["kv_out"])
    np.testing.assert_array_equal(torch_bf16_to_bits(c["layer0_blocks_out_sum"]), z["bos_out"])
