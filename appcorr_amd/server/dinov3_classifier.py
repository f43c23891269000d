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

from .. import _lib
from .. import kernels as K
from ..dinov3.backbone import dinov3_backbone
from ..tracing import trace_range
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
    """A correction group over the candidate tokens `dindice` [B, pre + P] without image-residual pruning
    (dinov3_classifier.py:231-281 with token_prune_enabled False)."""
    B = dindice.shape[0]
    P = dindice.shape[1] - num_pretokens
    dev = dindice.device
    count = torch.full((B,), P, device=dev, dtype=torch.int32)
    zeros = torch.zeros((B,), device=dev, dtype=torch.float32)
    # every query position valid: the query state of dinov3_classifier.py:199-229, built without a
    # host read
    q = dindice.shape[1]
    pos = torch.arange(q, device=dev, dtype=torch.long)
    qs = QueryState(query_pos_idx=pos.unsqueeze(0).expand(B, -1), query_valid_mask=torch.ones((B, q), device=dev,
                                                                                             dtype=torch.bool),
                    active_batch_idx=torch.arange(B, device=dev, dtype=torch.long).repeat_interleave(q),
                    active_pos_idx=pos.repeat(B), active_token_idx=dindice.reshape(-1), active_query_pos=pos.repeat(B),
                    active_query_pos_padded=pos.unsqueeze(0).expand(B, -1),
                    active_query_mask=torch.ones((B, q), device=dev, dtype=torch.bool), all_valid=True)
    return GroupCorrectionPlan(
        num_pretokens=num_pretokens, prefix_dindice=dindice[:, :num_pretokens],
        group_patch_dindice=dindice[:, num_pretokens:],
        group_patch_keep_local_idx=torch.arange(P, device=dev, dtype=torch.long).unsqueeze(0).expand(B, -1),
        full_dindice=dindice, pruned_dindice=dindice, query_state=qs, kept_patch_count=count,
        full_patch_count=count.clone(), kept_residual_mass=zeros, full_residual_mass=zeros.clone())


def _plan_sums(plan: GroupCorrectionPlan) -> torch.Tensor:
    """fp32 [4] = 0 + (kept_patch_count.sum(), full_patch_count.sum(), kept_residual_mass.sum(),
    full_residual_mass.sum()), computed once per set of plan tensors (a plan whose tensors are
    replaced gets new sums)."""
    src = (plan.kept_patch_count, plan.full_patch_count, plan.kept_residual_mass, plan.full_residual_mass)
    cached = getattr(plan, "_sums", None)
    if cached is None or any(a is not b for a, b in zip(cached[0], src)):
        sums = torch.stack([t.sum(dtype=torch.float32) for t in src]) + 0.0
        cached = (src, sums)
        plan._sums = cached
    return cached[1]


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

    @staticmethod
    def _patch_grid(config: Any) -> tuple[int, int, int, int]:
        H, W = config.image_shape[:2]
        ph, pw = (config.patch_size, config.patch_size) if isinstance(config.patch_size, int) else config.patch_size
        return H // ph, W // pw, ph, pw

    def _get_active_batch_indices(self, context: Dict[str, Any], full_batch_size: int) -> torch.Tensor:
        """dinov3_classifier.py:48-51."""
        if "active_indices" in context and len(context["active_indices"]) < full_batch_size:
            return context["active_indices"].to(device=self.device, dtype=torch.long)
        return torch.arange(full_batch_size, device=self.device, dtype=torch.long)

    def _build_mobile_pscore_hint_map(self, task: Task, context: Dict[str, Any], config: Any, batch_size: int,
                                      num_patches: int) -> torch.Tensor:
        """dinov3_classifier.py:53-89: the payload's per-patch pscore_hint at the finest transmitted
        level, scattered into [B, P] (active images only) and row-normalised."""
        hint_map = torch.zeros((batch_size, num_patches), device=self.device, dtype=torch.float32)
        target = min(config.transmission_kwargs.get("pyramid_levels", [0]))
        payload = task.payload if task is not None else []
        if "active_indices" in context and len(context["active_indices"]) < config.batch_size:
            idx_map = {orig: local for local, orig in enumerate(context["active_indices"].tolist())}
            valid = [p for p in payload
                     if p.image_idx in idx_map and p.res_level == target and 0 <= p.spatial_idx < num_patches]
            b_list = [idx_map[p.image_idx] for p in valid]
        else:
            valid = [p for p in payload if p.res_level == target and 0 <= p.spatial_idx < num_patches]
            b_list = [p.image_idx for p in valid]
        if not valid:
            return hint_map
        b_t = torch.tensor(b_list, device=self.device, dtype=torch.long)
        s_t = torch.tensor([p.spatial_idx for p in valid], device=self.device, dtype=torch.long)
        h_t = torch.tensor([float(getattr(p, "pscore_hint", 0.0)) for p in valid], device=self.device,
                           dtype=torch.float32)
        hint_map[b_t, s_t] = h_t
        return self._normalize_patch_score_map(hint_map)

    def _compute_patch_residual_rms(self, context: Dict[str, Any], config: Any,
                                    active_indices: torch.Tensor) -> torch.Tensor | None:
        """dinov3_classifier.py:91-122: per-patch RMS of the decoded frame minus the previous one
        ([B_active, gh * gw] fp32), in one HIP kernel on the uint8 frames."""
        curr_np, prev_np = context.get("input_hr_np"), context.get("prev_input_hr_np")
        if curr_np is None or prev_np is None:
            return None
        curr = torch.as_tensor(np.ascontiguousarray(curr_np)).to(self.device, non_blocking=True)
        prev = torch.as_tensor(np.ascontiguousarray(prev_np)).to(self.device, non_blocking=True)
        if curr.ndim != 4 or prev.ndim != 4:
            return None
        if curr.dtype not in (torch.uint8, torch.int16, torch.float32):
            curr, prev = curr.float(), prev.float()
        gh, gw, ph, pw = self._patch_grid(config)
        if tuple(curr.shape[1:3]) != (gh * ph, gw * pw):
            raise ValueError(f"decoded frames {tuple(curr.shape)} do not tile into {gh}x{gw} patches of {ph}x{pw}")
        return K.patch_residual_score(curr.contiguous(), prev.contiguous(), (ph, pw), _lib.IMPORTANCE_RMS,
                                      image_idx=active_indices.contiguous())

    def _apply_image_residual_token_pruning(self, dindice: torch.Tensor, spatial_indices: torch.Tensor,
                                            patch_residual_rms: torch.Tensor | None, threshold: float, min_keep: int):
        """dinov3_classifier.py:124-197: keep the candidates whose residual RMS reaches the threshold or
        that are among the min_keep largest, then compact them (one host read of the largest count, as
        the reference's .item())."""
        B, P = spatial_indices.shape
        num_pre = dindice.shape[1] - P
        dev = dindice.device
        full_count = torch.full((B,), P, device=dev, dtype=torch.int32)
        zeros = torch.zeros((B,), device=dev, dtype=torch.float32)
        full_idx = torch.arange(P, device=dev, dtype=torch.long).unsqueeze(0).expand(B, -1)
        if patch_residual_rms is None or P == 0:
            return dindice, full_count.clone(), full_count, zeros, zeros.clone(), full_idx
        spatial = spatial_indices.contiguous()
        pk = K.residual_prune_keep(patch_residual_rms.contiguous(), spatial, threshold, min_keep)
        width = int(pk.kept_count.max().item()) if B > 0 else 0
        if width == P:
            return dindice, pk.kept_count, full_count, pk.kept_mass, pk.full_mass, full_idx
        pruned, local = K.residual_prune_compact(pk.keep, spatial, dindice.contiguous(), num_pre, width)
        return pruned, pk.kept_count, full_count, pk.kept_mass, pk.full_mass, local

    @staticmethod
    def _build_fixed_query_state(dindice: torch.Tensor, kept_patch_count: torch.Tensor, num_pretokens: int) -> QueryState:
        """dinov3_classifier.py:199-229 (the group plan's query metadata; the blocks build their own plan)."""
        B, q = dindice.shape
        dev = dindice.device
        pos = torch.arange(q, device=dev, dtype=torch.long).unsqueeze(0).expand(B, -1)
        lengths = kept_patch_count.to(device=dev, dtype=torch.long) + num_pretokens
        valid = pos < lengths.unsqueeze(1)
        bi, pi = valid.nonzero(as_tuple=True)
        max_active = int(lengths.max().item()) if lengths.numel() > 0 else 0
        if max_active > 0:
            padded = torch.arange(max_active, device=dev, dtype=torch.long).unsqueeze(0).expand(B, -1)
            amask = padded < lengths.unsqueeze(1)
        else:
            padded = torch.empty((B, 0), device=dev, dtype=torch.long)
            amask = torch.empty((B, 0), device=dev, dtype=torch.bool)
        return QueryState(query_pos_idx=pos, query_valid_mask=valid, active_batch_idx=bi, active_pos_idx=pi,
                          active_token_idx=dindice[bi, pi], active_query_pos=pi, active_query_pos_padded=padded,
                          active_query_mask=amask,
                          all_valid=bool(torch.all(lengths == q).item()) if lengths.numel() > 0 else True)

    def _build_group_plan(self, dindice: torch.Tensor, spatial_indices: torch.Tensor,
                          patch_residual_rms: torch.Tensor | None, num_pretokens: int, token_prune_enabled: bool,
                          token_prune_threshold: float, token_prune_min_keep: int) -> GroupCorrectionPlan:
        """dinov3_classifier.py:231-281."""
        plan = make_group_plan(dindice, num_pretokens)
        pruned = dindice
        if token_prune_enabled:
            (pruned, plan.kept_patch_count, plan.full_patch_count, plan.kept_residual_mass, plan.full_residual_mass,
             plan.group_patch_keep_local_idx) = self._apply_image_residual_token_pruning(
                dindice, spatial_indices, patch_residual_rms, token_prune_threshold, token_prune_min_keep)
        if pruned is not dindice or token_prune_enabled:
            plan.query_state = self._build_fixed_query_state(pruned, plan.kept_patch_count, num_pretokens)
        plan.pruned_dindice = pruned
        return plan

    def preprocess(self, batch_data: Any, task: Task, context: Dict[str, Any], config: Any):
        """dinov3_classifier.py:330-527: normalised input, the request's patch -> group map, the mobile
        hint map, and one correction plan per transmitted group (image-residual pruning optional)."""
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
        t = (t - self.norm_mean) / self.norm_std
        sliced = "active_indices" in context and len(context["active_indices"]) < config.batch_size
        if sliced:
            t = t[context["active_indices"]]
        context["input_tensor"] = t
        gh, gw, _, _ = self._patch_grid(config)
        num_patches = gh * gw
        if "group_map" not in context:
            context["group_map"] = torch.full((t.shape[0], num_patches), -1, device=self.device, dtype=torch.long)
        gm = context["group_map"]
        payload = task.payload if task is not None else []
        if sliced:
            idx_map = {orig: local for local, orig in enumerate(context["active_indices"].tolist())}
            payload = [p for p in payload if p.image_idx in idx_map]
            b_list = [idx_map[p.image_idx] for p in payload]
        else:
            b_list = [p.image_idx for p in payload]
        s_list = [p.spatial_idx for p in payload]
        g_list = [p.group_id for p in payload]
        if b_list:
            b_t = torch.tensor(b_list, device=self.device, dtype=torch.long)
            s_t = torch.tensor(s_list, device=self.device, dtype=torch.long)
            g_t = torch.tensor(g_list, device=self.device, dtype=torch.long)
            gm[b_t, s_t] = g_t
        context["mobile_pscore_hint_map"] = self._build_mobile_pscore_hint_map(task, context, config, t.shape[0],
                                                                               num_patches)
        num_pre = self.model.num_pretokens
        B = gm.shape[0]
        opts = normalize_appcorr_kwargs(config.appcorr_kwargs, config.transmission_kwargs)
        active = self._get_active_batch_indices(context, config.batch_size)
        rms = self._compute_patch_residual_rms(context, config, active)
        plans = self._get_group_plans(context)
        plans.clear()
        if not b_list:
            return
        pre = torch.arange(num_pre, device=self.device).unsqueeze(0).expand(B, -1)
        for gid in sorted(set(g_list)):
            try:
                spatial = s_t[g_t == gid].view(B, -1)
            except RuntimeError:
                print(f"!!! [Executor] Non-uniform group {gid} size detected. Fallback skip.")
                continue
            plans[gid] = self._build_group_plan(torch.cat([pre, spatial + num_pre], dim=1), spatial, rms, num_pre,
                                                opts["token_prune_enabled"], opts["token_prune_threshold"],
                                                opts["token_prune_min_keep"])

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
        with trace_range(f"approx_forward|layers={start}-{end}"):
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
        # total = total + value.sum() for the four pruning counters (dinov3_classifier.py:618-634), with
        # the group plan's sums computed once and the additions in one launch.
        if plan.query_state is not None:
            keys = ("_token_prune_kept_patch_total", "_token_prune_full_patch_total",
                    "_token_prune_kept_residual_mass_total", "_token_prune_full_residual_mass_total")
            sums = _plan_sums(plan)
            prev = [cache.get(k) for k in keys]
            if all(p is None for p in prev):
                for k, v in zip(keys, sums.unbind(0)):
                    cache[k] = v
            else:
                prev = [x.new_zeros((), dtype=torch.float32) if p is None else p for p in prev]
                for k, t in zip(keys, torch._foreach_add(prev, list(sums.unbind(0)))):
                    cache[k] = t
        self.begin_dinov3_correct_event()
        with trace_range(f"correct_forward|group={group_id}|layers={start}-{end}"):
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
        correct_forward bit for bit. The running statistics (`_token_pscore_*_total`, ...) continue
        from the values the cache held before recording: the graph writes one pass's statistics, and
        each replay adds them into the running totals (one small launch after the graph), which the
        cache then holds. With a plan shared by the layers (one addition per pass) the totals equal
        those of eager passes bit for bit; with per-layer plans a pass's layer values are summed
        before they are added (the fp32 association differs). The warm-up and recording passes are
        not counted.
        """
        from appcorr_amd.dinov3.layers import SelfAttentionBlock
        from appcorr_amd.graphs import capture

        stat_keys = ("_token_pscore_kept_mass_total", "_token_pscore_full_mass_total", "_partial_token_kept_patch_total",
                     "_partial_token_full_patch_total", "_partial_token_sample_total",
                     "_token_prune_kept_patch_total", "_token_prune_full_patch_total",
                     "_token_prune_kept_residual_mass_total", "_token_prune_full_residual_mass_total")

        def run():
            cache = context.setdefault("cache_feature", {})
            SelfAttentionBlock._invalidate_partial_token_derived_caches(cache)
            for k in stat_keys:  # recorded from zero: each replay leaves one pass's statistics
                cache.pop(k, None)
            self.correct_forward(params, context, config)

        cache0 = context.setdefault("cache_feature", {})
        base = {k: cache0[k].clone() for k in stat_keys if torch.is_tensor(cache0.get(k))}
        with torch.no_grad():
            replay = capture(run, self.device, warmup)
        cache = context["cache_feature"]
        per_pass = {k: cache[k] for k in stat_keys if torch.is_tensor(cache.get(k))}  # written by every replay
        totals = {k: base[k] if k in base else torch.zeros_like(v) for k, v in per_pass.items()}
        keys = list(per_pass)

        def replay_and_accumulate() -> None:
            replay()
            if keys:
                torch._foreach_add_([totals[k] for k in keys], [per_pass[k] for k in keys])
                cache.update(totals)

        replay_and_accumulate.graph = replay.graph
        replay_and_accumulate.replay = replay
        if keys:
            cache.update(totals)
        return replay_and_accumulate

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
