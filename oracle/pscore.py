"""Server patch scores of the approximate pass, restated on the CPU. Test infrastructure only.

Reference: SelfAttention.compute_attention_partial_token
(appcorr/models/dinov3/layers/attention.py:215-278) and the fused key-side kernel
(appcorr/models/dinov3/layers/triton_kernels/attention_pscore.py:20-98, 172-241). The reference
evaluates the scores with eager torch ops on bf16 tensors (under the server's bf16 model), so every
op's output is rounded to bf16; the points are, for one query q and the keys K of one head:

    s   = bf16(q . K^T)                 bf16 matmul: fp32 accumulate, one rounding   (:267)
    s   = bf16(fp32(s) * fp32(scale))   bf16 tensor times a Python float             (:267)
    p   = bf16(e_n / sum_n e_n),        e_n = exp(s_n - max s), fp32                 (softmax, :268)
    m   = bf16(fp32(sum_h p) * fl(1/H)) mean over heads: fp32 accumulate, x factor   (:268)

(torch's mean multiplies the fp32 sum by the float factor num_outputs / numel = fl(1/H).)

Here every fp32 accumulation is evaluated exactly (float64, then one rounding to fp32) and exp is
evaluated in float64 and rounded to fp32: the correctly rounded value of each step. A GPU kernel
whose fp32 accumulations differ in order can differ from this only where a value lies within an
fp32 ulp of a bf16 rounding boundary; the HIP kernels of this build accumulate in float64 as well
and agree bit for bit. Parity unpinned against the reference's own device (cuBLAS accumulation
order, CUDA's expf, the block-reduction order of torch's softmax and mean), which cannot run here.

Functions
  query_attention_prob   one query per (image, head): cls_attn_prob (q = the cls token, :267-271)
                         and patch_pseudo_attn_prob (q = the pseudo query, :255-261)
  pseudo_query           the pseudo query of patch_pseudo_attn_prob (:254-259)
  patch_attn_prob        mean over heads, then over queries, of the full softmax (:251-253)
  patch_attn_prob_fused  the fused kernel's score for 32 x 128 heads: fp32 probabilities from the
                         row log-sum-exp, summed over queries and heads, x 1/(H N), one rounding
                         (attention_pscore.py:20-98, 172-212)
"""

from __future__ import annotations

import numpy as np

from .bf16 import round_bf16

BF16_EPS = np.float32(2.0 ** -7)  # torch.finfo(torch.bfloat16).eps (attention.py:257)


def _f32(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float64).astype(np.float32)


def _bf(a) -> np.ndarray:
    """fp32 array -> bf16 values (round to nearest even), as fp32."""
    return round_bf16(np.asarray(a, dtype=np.float32))


def _bf_from_exact(a) -> np.ndarray:
    """An exact (float64) accumulation -> fp32 -> bf16: the bf16 output of an fp32-accumulating op."""
    return _bf(_f32(a))


def _softmax_bf16(s: np.ndarray) -> np.ndarray:
    """torch softmax over the last axis of a bf16 tensor: fp32 max, e = exp(s - max), fp32 sum,
    bf16(e / sum)."""
    s = s.astype(np.float32)
    d = s - s.max(axis=-1, keepdims=True)                        # fp32 subtraction
    e = _f32(np.exp(d.astype(np.float64)))
    tot = _f32(e.astype(np.float64).sum(axis=-1, keepdims=True))
    return _bf(e / tot)                                           # fp32 IEEE division


def _mean_bf16(p: np.ndarray, axis: int) -> np.ndarray:
    """torch .mean(axis) of a bf16 tensor: fp32 accumulate, x fl(1/n), bf16."""
    n = p.shape[axis]
    factor = np.float32(1.0) / np.float32(n)
    return _bf(_f32(p.astype(np.float64).sum(axis=axis)) * factor)


def _scores(q: np.ndarray, k: np.ndarray, scale: float) -> np.ndarray:
    """s = bf16(bf16(q . K^T) * scale) for q [B, H, T, D] and k [B, N, H, D] (bf16 values, fp32)."""
    raw = np.matmul(q.astype(np.float64), k.astype(np.float64).transpose(0, 2, 3, 1))   # [B, H, T, N]
    return _bf(_bf_from_exact(raw) * np.float32(scale))


def query_attention_prob(q: np.ndarray, k: np.ndarray, scale: float) -> np.ndarray:
    """softmax(q . K^T * scale) for one query per (image, head), mean over heads, as fp32.

    q [B, H, D] (bf16 values), k [B, N, H, D] (the K cache after RoPE) -> [B, N] fp32 holding bf16
    values: cls_attn_prob's `.softmax(-1).mean(dim=1).squeeze(1).to(float32)` (attention.py:267-271)
    and, with the pseudo query, patch_pseudo_attn_prob's `.mean(dim=1).mean(dim=1)` (:260-261; the
    second mean is over one query and leaves the bf16 value unchanged).
    """
    p = _softmax_bf16(_scores(q[:, :, None, :], k, scale))      # [B, H, 1, N]
    return _mean_bf16(p[:, :, 0, :], axis=1)


def pseudo_query(q_patch: np.ndarray) -> np.ndarray:
    """The pseudo query of patch_pseudo_attn_prob (attention.py:254-259) for q_patch [B, H, P, D]
    (bf16 values, the patch queries after RoPE) -> [B, H, D] bf16 values:

        q_mean = bf16(fl(sum_p q) * fl(1/P))
        qmn    = max(bf16(sqrt(fl(sum_d q_mean^2))), eps_bf16)         (norm: fp32 accumulate, sqrt)
        target = bf16(fl(sum_p bf16(sqrt(fl(sum_d q^2)))) * fl(1/P))
        q_ps   = bf16(q_mean * bf16(target / qmn))
    """
    q = q_patch.astype(np.float32)
    P = q.shape[2]
    fp = np.float32(1.0) / np.float32(P)
    q_mean = _bf(_f32(q.astype(np.float64).sum(axis=2)) * fp)                                  # [B, H, D]
    qmn = _bf(np.sqrt(_f32((q_mean.astype(np.float64) ** 2).sum(axis=-1))))                     # [B, H]
    qmn = np.maximum(qmn, BF16_EPS)
    norms = _bf(np.sqrt(_f32((q.astype(np.float64) ** 2).sum(axis=-1))))                        # [B, H, P]
    target = _bf(_f32(norms.astype(np.float64).sum(axis=-1)) * fp)                              # [B, H]
    ratio = _bf(target / qmn)
    return _bf(q_mean * ratio[..., None])


def patch_attn_prob(q: np.ndarray, k: np.ndarray, scale: float) -> np.ndarray:
    """Dense patch_attn_prob(_layermean) (attention.py:251-253): q [B, H, N, D], k [B, N, H, D] ->
    [B, N] bf16 values = mean over queries of (mean over heads of the bf16 softmax)."""
    p = _softmax_bf16(_scores(q, k, scale))                       # [B, H, N, N]
    ph = _mean_bf16(p, axis=1)                                    # [B, N, N]
    return _mean_bf16(ph, axis=1)                                 # [B, N]


def _scaled_scores(q: np.ndarray, k: np.ndarray, scale: float) -> np.ndarray:
    """q [B, H, T, D], k [B, N, H, D] -> q . k * scale [B, H, T, N] in float64."""
    return np.matmul(q.astype(np.float64), k.astype(np.float64).transpose(0, 2, 3, 1)) * float(scale)


def row_logsumexp(q: np.ndarray, k: np.ndarray, scale: float) -> np.ndarray:
    """The row log-sum-exp SDPA returns beside its output (attention_pscore.py:136-168, cuDNN's LSE):
    lse[b, h, t] = ln sum_n exp(q[b, h, t] . k[b, n, h] * scale), natural log, exact (float64) evaluation
    with the max taken out. q [B, H, T, D], k [B, N, H, D] -> [B, H, T]."""
    s = _scaled_scores(q, k, scale)
    mx = s.max(axis=-1, keepdims=True)
    return (mx + np.log(np.exp(s - mx).sum(axis=-1, keepdims=True)))[..., 0]


def patch_attn_prob_fused(q: np.ndarray, k: np.ndarray, scale: float) -> np.ndarray:
    """Fused key-side score (attention_pscore.py:20-98): p = exp(q.k * scale - lse) in fp32 from
    the row log-sum-exp of SDPA, summed over all queries and heads, times 1/(H N), rounded to bf16
    once. Exact (float64) evaluation; the reference's own fp32 kernel sums with atomics in no fixed
    order, so a device result agrees within fp32 rounding before the final bf16 rounding."""
    B, H, T, D = q.shape
    s = _scaled_scores(q, k, scale)
    lse = row_logsumexp(q, k, scale)[..., None]
    p = np.exp(s - lse)
    col = p.sum(axis=(1, 2)) * (1.0 / float(H * T))
    return _bf(_f32(col))
