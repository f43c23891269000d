"""DINOv3 classifier executor: the reference caller of the correction path.

Follows offload/server/model/dinov3_classifier.py: group correction plans (:12-37, :231-281),
preprocess (:330-527), prepare_tokens (:529-545), approx_forward (:547-589) and correct_forward
(:591-663), which drives `run_dinov3_correct_block` once per layer with the same kwargs. Weights
are random-initialised at the requested hub shape (there is no checkpoint loading here); the linear
classification head is plumbing around the backbone.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict

import numpy as np
import torch

from ..dinov3.backbone import dinov3_backbone
from .base import ModelExecutor
from .protocol import Task, normalize_appcorr_kwargs


@dataclass
class QueryState:
    query_pos_idx: torch.Tensor
    query_valid_mask: torch.Tensor
    active_batch_idx: torch.Tensor
    active_pos_idx: torch.Tensor
    active_token_idx: torch.Tensor
    active_query_pos: torch.Tensor
    active_query_pos_padded: torch.Tensor
    active_query_mask: torch.Tensor
    all_valid: bool


@dataclass
class GroupCorrectionPlan:
    num_pretokens: int
    prefix_dindice: torch.Tensor
    group_patch_dindice: torch.Tensor
    group_patch_keep_local_idx: torch.Tensor
    full_dindice: torch.Tensor
    pruned_dindice: torch.Tensor
    query_state: QueryState | None
    kept_patch_count: torch.Tensor
    full_patch_count: torch.Tensor
    kept_residual_mass: torch.Tensor
    full_residual_mass: torch.Tensor


def make_group_plan(dindice: torch.Tensor, num_pretokens: int) -> GroupCorrectionPlan:
    """A correction group over the candidate tokens `dindice` [B, pre + P] (no image-residual pruning)."""
    B = dindice.shape[0]
    P = dindice.shape[1] - num_pretokens
    dev = dindice.device
    count = torch.full((B,), P, device=dev, dtype=torch.int32)
    zeros = torch.zeros((B,), device=dev, dtype=torch.float32)
    return GroupCorrectionPlan(
        num_pretokens=num_pretokens, prefix_dindice=dindice[:, :num_pretokens],
        group_patch_dindice=dindice[:, num_pretokens:],
        group_patch_keep_local_idx=torch.arange(P, device=dev, dtype=torch.long).unsqueeze(0).expand(B, -1),
        full_dindice=dindice, pruned_dindice=dindice, query_state=None, kept_patch_count=count,
        full_patch_count=count.clone(), kept_residual_mass=zeros, full_residual_mass=zeros.clone())


def _patch_count_sums(plan: GroupCorrectionPlan) -> torch.Tensor:
    """fp32 [2] = (0 + kept_patch_count.sum(), 0 + full_patch_count.sum()), computed once per pair
    of count tensors (a plan whose count tensors are replaced gets new sums)."""
    cached = getattr(plan, "_count_sums", None)
    if cached is None or cached[0] is not plan.kept_patch_count or cached[1] is not plan.full_patch_count:
        sums = torch.stack([plan.kept_patch_count.sum(dtype=torch.float32),
                            plan.full_patch_count.sum(dtype=torch.float32)]) + 0.0
        cached = (plan.kept_patch_count, plan.full_patch_count, sums)
        plan._count_sums = cached
    return cached[2]


class DINOv3ClassifierExecutor(ModelExecutor):
    def __init__(self, device: torch.device):
        super().__init__(device)
        self.norm_mean = torch.tensor([0.485, 0.456, 0.406], device=device).view(1, 3, 1, 1)
        self.norm_std = torch.tensor([0.229, 0.224, 0.225], device=device).view(1, 3, 1, 1)
        self.head = None
        # Keep the selected rows packed across a correction run when the plan is shared by all layers.
        self.packed_correction = True

    @staticmethod
    def _get_group_plans(context: Dict[str, Any]) -> Dict[int, GroupCorrectionPlan]:
        return context.setdefault("group_plans", {})

    def load_model(self, model_name: str, config: Any):
        name = getattr(config, "backbone", None) or "vitl16"
        for cand in ("vit7b16", "vitl16", "vitb16", "vits16"):
            if cand in model_name:
                name = cand
        self.model = dinov3_backbone(name, device=self.device).eval()
        C = self.model.embed_dim
        g = torch.Generator().manual_seed(1)
        self.head = (torch.randn(getattr(config, "num_classes", 1000), 2 * C, generator=g) * 0.02).to(
            device=self.device, dtype=torch.bfloat16)
        self.configure_dinov3_approx_precision(self.model, config)
        self.configure_dinov3_correct_precision(self.model, config)

    def preprocess(self, batch_data: Any, task: Task, context: Dict[str, Any], config: Any):
        t = batch_data if isinstance(batch_data, torch.Tensor) else torch.from_numpy(np.asarray(batch_data))
        t = t.to(self.device, non_blocking=True)
        if t.ndim != 4:
            raise ValueError(f"Expected 4D tensor input, got {tuple(t.shape)}")
        if t.shape[1] != 3 and t.shape[-1] == 3:
            t = t.permute(0, 3, 1, 2)
        is_u8 = t.dtype == torch.uint8
        t = t.float()
        if is_u8:
            t = t / 255.0
        context["input_tensor"] = (t - self.norm_mean) / self.norm_std
        H, W = config.image_shape[:2]
        ph = pw = config.patch_size if isinstance(config.patch_size, int) else config.patch_size[0]
        num_patches = (H // ph) * (W // pw)
        B = t.shape[0]
        if "group_map" not in context:
            context["group_map"] = torch.full((B, num_patches), -1, device=self.device, dtype=torch.long)
        gm = context["group_map"]
        hint = torch.zeros((B, num_patches), device=self.device, dtype=torch.float32)
        if task is not None and task.payload:
            b = torch.tensor([p.image_idx for p in task.payload], device=self.device)
            s = torch.tensor([p.spatial_idx for p in task.payload], device=self.device)
            g = torch.tensor([p.group_id for p in task.payload], device=self.device)
            h = torch.tensor([float(p.pscore_hint) for p in task.payload], device=self.device)
            gm[b, s] = g
            hint[b, s] = h
        context["mobile_pscore_hint_map"] = self._normalize_patch_score_map(hint)
        num_pre = self.model.num_pretokens
        plans = self._get_group_plans(context)
        plans.clear()
        pre = torch.arange(num_pre, device=self.device).unsqueeze(0).expand(B, -1)
        for gid in sorted(set(int(v) for v in gm.unique().tolist()) - {-1}):
            try:
                spatial = torch.where(gm == gid)[1].view(B, -1)
            except RuntimeError:
                continue  # non-uniform group size across images (reference skips these too)
            plans[gid] = make_group_plan(torch.cat([pre, spatial + num_pre], dim=1), num_pre)

    def prepare_tokens(self, task: Task, context: Dict[str, Any], config: Any):
        if "input_tensor" not in context:
            return
        with torch.no_grad():
            tokens, (H, W) = self.model.prepare_tokens(context["input_tensor"])
        context["input_tokens"] = tokens.to(torch.bfloat16).contiguous()
        context["hw_tuple"] = (H, W)
        context.setdefault("current_feature", context["input_tokens"])
        if "rope_sincos" not in context:
            context["rope_sincos"] = self.model.rope_embed(H=H, W=W)

    def approx_forward(self, params: Dict[str, Any], context: Dict[str, Any], config: Any):
        layers = params.get("layers", (0, len(self.model.blocks)))
        opts = normalize_appcorr_kwargs(config.appcorr_kwargs, config.transmission_kwargs)
        start, end = layers[0], layers[1]
        x = context["input_tokens"] if start == 0 else context.get("current_feature", context.get("input_tokens"))
        cache = context.get("cache_feature", {})
        rope = context.get("rope_sincos")
        self.begin_dinov3_approx_event()
        for lidx in range(start, end):
            x, cache = self.run_dinov3_approx_block(lidx, x, rope, cache, tag=f"layer{lidx}",
                                                    appcorr_method=opts["method"],
                                                    server_pscore=opts["server_pscore"],
                                                    server_pscore_weight=opts["server_pscore_weight"])
        context["current_feature"] = x
        context["cache_feature"] = cache
        return self.dinov3_approx_event_metadata()

    def correct_forward(self, params: Dict[str, Any], context: Dict[str, Any], config: Any):
        layers = params.get("layers", (0, len(self.model.blocks)))
        group_id = params.get("group_id", 1)
        start, end = layers[0], layers[1]
        plan = self._get_group_plans(context).get(group_id)
        if plan is None:
            print(f"!!! [Executor] Missing group correction plan for group {group_id}.")
            return
        dindice = plan.pruned_dindice.to(device=self.device, non_blocking=True)
        plan.pruned_dindice = dindice
        cache = context.get("cache_feature", {})
        rope = context.get("rope_sincos")
        x = context.get("input_tokens")
        opts = normalize_appcorr_kwargs(config.appcorr_kwargs, config.transmission_kwargs)
        hint = context.get("mobile_pscore_hint_map")
        # total = total + count.sum() for the two counters (dinov3_classifier.py:618-634), with the
        # group plan's sums computed once and both additions in one launch.
        keys = ("_token_prune_kept_patch_total", "_token_prune_full_patch_total")
        sums = _patch_count_sums(plan)
        prev = [cache.get(k) for k in keys]
        if prev[0] is None and prev[1] is None:
            cache[keys[0]], cache[keys[1]] = sums[0], sums[1]
        else:
            prev = [x.new_zeros((), dtype=torch.float32) if p is None else p for p in prev]
            for k, t in zip(keys, torch._foreach_add(prev, [sums[0], sums[1]])):
                cache[k] = t
        self.begin_dinov3_correct_event()
        block_kwargs = dict(
            appcorr_method=opts["method"], token_keep_ratio=opts["token_keep_ratio"],
            token_keep_thres=opts["token_keep_thres"], mobile_pscore=opts["mobile_pscore"],
            mobile_pscore_weight=opts["mobile_pscore_weight"], mobile_pscore_hint=hint,
            server_pscore=opts["server_pscore"], server_pscore_weight=opts["server_pscore_weight"],
            pscore_fusion=opts["pscore_fusion"], sdpa_query_bucket_size=opts["sdpa_query_bucket_size"],
            attn_col_alive_ratio=opts["attn_col_alive_ratio"], fixed_query_state=plan.query_state,
            group_plan=plan, attn_cache_key=group_id, debug=False)
        # With a query plan shared by every layer the selected rows stay packed across the whole run
        # (bit-identical to the per-block loop below, one gather and one full-tensor write in total).
        res = None
        if self.packed_correction and self._dinov3_correct_precision is not None and end > start:
            res = self._dinov3_correct_precision.run_blocks_packed(range(start, end), x, dindice, rope, cache,
                                                                   **block_kwargs)
        if res is not None:
            x, cache = res
        else:
            for lidx in range(start, end):
                x, cache = self.run_dinov3_correct_block(lidx, x, dindice, rope, cache, f"layer{lidx}",
                                                         source_key=f"layer{lidx}", **block_kwargs)
        context["current_feature"] = x
        context["cache_feature"] = cache
        return self.dinov3_correct_event_metadata()

    def capture_correct_forward(self, params: Dict[str, Any], context: Dict[str, Any], config: Any,
                                warmup: int = 2):
        """Record one correction pass into a HIP graph and return its replay function.

        The query-plan cache is cleared before recording, so the recorded work includes building the
        plan: every replay rebuilds it from the current scores and runs every block, on the tensors
        the recording used (context["input_tokens"], context["mobile_pscore_hint_map"], the cache
        dict's K/V and blocks_out_sum tensors, the group plan); refresh their contents in place
        between replays.
        context["current_feature"] after a replay holds that replay's output. Outputs equal an eager
        correct_forward bit for bit; the running statistics in the cache hold one pass's values.
        """
        from appcorr_amd.dinov3.layers import SelfAttentionBlock
        from appcorr_amd.graphs import capture

        stat_keys = ("_token_pscore_kept_mass_total", "_token_pscore_full_mass_total", "_partial_token_kept_patch_total",
                     "_partial_token_full_patch_total", "_partial_token_sample_total",
                     "_token_prune_kept_patch_total", "_token_prune_full_patch_total")

        def run():
            cache = context.setdefault("cache_feature", {})
            SelfAttentionBlock._invalidate_partial_token_derived_caches(cache)
            for k in stat_keys:  # recorded from zero: each replay leaves one pass's statistics
                cache.pop(k, None)
            self.correct_forward(params, context, config)

        with torch.no_grad():
            return capture(run, self.device, warmup)

    def head_inference(self, task: Task, context: Dict[str, Any], config: Any) -> Dict[str, Any]:
        feat = context.get("current_feature")
        xn = self.model.final_norm(feat)
        lin = torch.cat([xn[:, 0], xn[:, self.model.num_pretokens:].float().mean(dim=1).to(xn.dtype)], dim=1)
        logits = (lin.float() @ self.head.float().T)
        context["output"] = logits
        probs = torch.softmax(logits, dim=1)
        entropy = -(probs * torch.log(probs + 1e-10)).sum(dim=1)
        top5_p, top5_i = torch.topk(probs, k=min(5, probs.shape[1]), dim=1)
        return {"entropy": entropy.cpu().tolist(), "top5_probs": top5_p.cpu().tolist(),
                "top5_indices": top5_i.cpu().tolist()}

    def full_inference(self, task: Task, context: Dict[str, Any], config: Any):
        self.prepare_tokens(task, context, config)
        x = context["input_tokens"]
        cache: Dict[str, Any] = {}
        with torch.no_grad():
            for i, blk in enumerate(self.model.blocks):
                x, cache = blk.approx(x, context["rope_sincos"], cache, f"full{i}", server_pscore_weight=0.0)
        context["current_feature"] = x
        return self.head_inference(task, context, config)

    def decide_exit(self, task: Task, context: Dict[str, Any], config: Any) -> Dict[str, Any]:
        return {}

    def get_final_results(self, task: Task, context: Dict[str, Any], config: Any) -> Dict[int, Any]:
        out = context.get("output")
        if out is None:
            return {}
        pred = out.argmax(dim=1).cpu().tolist()
        return {i: {"class": int(c)} for i, c in enumerate(pred)}
