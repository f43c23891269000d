"""Instruction protocol and correction settings, as consumed by the executor API.

Same names, fields and option semantics as the reference's offload/common/protocol.py
(default_appcorr_kwargs :6-35, normalize_appcorr_kwargs :62-181, OpType / Instruction / Task
:368-394, InferenceResult :396-415). The scheduler, transport and codec fields that only the control
plane uses are accepted and passed through but play no part here.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum, auto
from typing import Any, Dict, List


def default_appcorr_kwargs() -> Dict[str, Any]:
    return {
        "enabled": False, "generated_from_client": False, "global_source_mode": "global_first", "update_attn": False,
        "pyramid_levels": [0], "token_res": [1.0], "plan": [], "num_groups": 1, "group_strategy": "uniform",
        "token_keep_ratio": 0.2, "token_keep_thres": None, "token_keep_cap": 0, "attn_col_alive_ratio": 1.0,
        "mobile_pscore": "none", "mobile_pscore_weight": 0.0, "server_pscore": "cls_attn_prob",
        "server_pscore_weight": 1.0, "pscore_fusion": "add", "sdpa_query_bucket_size": 0, "sdpa_warmup": True,
        "sdpa_warmup_runs": 2, "correct_warmup_runs": 1, "token_prune_enabled": False, "token_prune_threshold": 0.0,
        "token_prune_min_keep": 1, "method": "partial_token", "debug": False,
    }


_MOBILE_ALIASES = {
    "residual_rms": "residual_rms", "patch_residual_rms": "residual_rms", "residual_l2": "residual_energy",
    "residual_l2_energy": "residual_energy", "residual_energy": "residual_energy",
    "patch_residual_l2": "residual_energy", "patch_residual_energy": "residual_energy",
}
_SERVER_ALIASES = {
    "pseudo_patch_attn_prob": "patch_pseudo_attn_prob",
    "pseudo_patch_attn_prob_layermean": "patch_pseudo_attn_prob_layermean",
}


def normalize_appcorr_kwargs(appcorr_kwargs: Dict[str, Any] | None = None,
                             transmission_kwargs: Dict[str, Any] | None = None) -> Dict[str, Any]:
    """Defaults, aliases and validation of the correction options (reference protocol.py:62-181)."""
    from ..dinov3.layers import SelfAttentionBlock

    raw = dict(appcorr_kwargs or {})
    explicit_enabled = raw.pop("enabled", None)
    enabled_from_appcorr = bool(raw)
    if transmission_kwargs:
        if "pyramid_levels" in transmission_kwargs:
            levels = list(transmission_kwargs["pyramid_levels"])
            if "pyramid_levels" in raw and list(raw["pyramid_levels"]) != levels:
                raise ValueError("appcorr_kwargs.pyramid_levels must match transmission_kwargs.pyramid_levels")
            raw["pyramid_levels"] = levels
        if "num_groups" in transmission_kwargs:
            ng = max(int(transmission_kwargs["num_groups"]), 1)
            if "num_groups" in raw and max(int(raw["num_groups"]), 1) != ng:
                raise ValueError("appcorr_kwargs.num_groups must match transmission_kwargs.num_groups")
            raw["num_groups"] = ng
    if "persist_correction_residual" in raw:
        raise ValueError("appcorr_kwargs.persist_correction_residual no longer exists; the corrected increment is "
                         "always persisted.")
    d = default_appcorr_kwargs()
    o = default_appcorr_kwargs()
    o.update(raw)
    o["enabled"] = enabled_from_appcorr if explicit_enabled is None else bool(explicit_enabled)
    o["generated_from_client"] = bool(o["generated_from_client"])
    if o["global_source_mode"] not in ("global_first", "final_correct", "approx"):
        o["global_source_mode"] = d["global_source_mode"]
    o["update_attn"] = bool(o["update_attn"])
    for key in ("pyramid_levels", "token_res", "plan"):
        o[key] = list(o[key])
    o["num_groups"] = max(int(o["num_groups"]), 1)
    o["group_strategy"] = str(o["group_strategy"])
    ratio = o["token_keep_ratio"]
    if "token_keep_ratio" not in raw and "cls_alive_ratio" in raw:
        ratio = raw["cls_alive_ratio"]
    o["token_keep_ratio"] = float(ratio)
    thres = o["token_keep_thres"]
    o["token_keep_thres"] = None if thres in (None, "", "null", "None") else float(thres)
    o["token_keep_cap"] = max(0, int(o.get("token_keep_cap", 0) or 0))
    o["attn_col_alive_ratio"] = float(o["attn_col_alive_ratio"])
    mp = str(o["mobile_pscore"])
    if mp in ("", "null", "None"):
        mp = d["mobile_pscore"]
    o["mobile_pscore"] = _MOBILE_ALIASES.get(mp, mp)
    o["mobile_pscore_weight"] = float(o["mobile_pscore_weight"])
    sp = str(o["server_pscore"])
    legacy = raw.get("token_prune_score")
    if legacy is not None and "server_pscore" not in raw:
        sp = str(legacy)
    if bool(raw.get("patch_attn_prune", False)) and "server_pscore" not in raw and legacy is None:
        sp = "patch_attn_prob"
    if sp == "patch_attn_prune":
        sp = "patch_attn_prob"
    sp = _SERVER_ALIASES.get(sp, sp)
    fusion_legacy = str(raw.get("server_pscore_layer_fusion", "")).lower()
    if fusion_legacy in ("mean", "avg", "all_layer_mean", "layer_mean", "mean_all_layers"):
        sp = {"patch_attn_prob": "patch_attn_prob_layermean",
              "patch_pseudo_attn_prob": "patch_pseudo_attn_prob_layermean",
              "cls_attn_prob": "cls_attn_prob_layermean"}.get(sp, sp)
    if sp not in SelfAttentionBlock._VALID_SERVER_PSCORES:
        raise ValueError(f"Unknown server_pscore '{sp}'. Available values: "
                         f"{sorted(SelfAttentionBlock._VALID_SERVER_PSCORES)}")
    o["server_pscore"] = sp
    o["server_pscore_weight"] = float(o["server_pscore_weight"])
    fu = str(o["pscore_fusion"]).lower()
    fu = {"mul": "multiply", "product": "multiply", "geomean": "geo_mean", "geometric_mean": "geo_mean"}.get(fu, fu)
    o["pscore_fusion"] = fu if fu in ("add", "multiply", "geo_mean") else d["pscore_fusion"]
    o["sdpa_query_bucket_size"] = max(int(o["sdpa_query_bucket_size"] or 0), 0)
    o["sdpa_warmup"] = bool(o["sdpa_warmup"])
    o["sdpa_warmup_runs"] = max(int(o["sdpa_warmup_runs"] or 0), 0)
    o["correct_warmup_runs"] = max(int(o["correct_warmup_runs"] or 0), 0)
    o["token_prune_enabled"] = bool(o["token_prune_enabled"])
    o["token_prune_threshold"] = float(o["token_prune_threshold"])
    o["token_prune_min_keep"] = max(int(o["token_prune_min_keep"]), 1)
    o["method"] = str(o["method"])
    o["debug"] = bool(o["debug"])
    return o


@dataclass
class ExperimentConfig:
    """The subset of the reference ExperimentConfig (protocol.py:184-259) the executor reads."""
    model_name: str = "dinov3_classifier"
    batch_size: int = 1
    image_shape: tuple = (512, 512, 3)
    patch_size: Any = 16
    appcorr_kwargs: Dict[str, Any] = field(default_factory=dict)
    transmission_kwargs: Dict[str, Any] = field(default_factory=dict)
    correct_precision: str = "bf16"
    correct_compile: bool = False
    correct_fp4_calib_events: int = 1
    correct_fp4_proj_precision: str = "fp8"
    correct_bucket_rows: int = 0
    backbone: str = "vitl16"
    num_classes: int = 1000


class OpType(Enum):
    FULL_INFERENCE = auto()
    APPROX_FORWARD = auto()
    CORRECT_FORWARD = auto()
    HEAD_INFERENCE = auto()
    LOAD_INPUT = auto()
    PREPARE_TOKENS = auto()
    SEND_RESPONSE = auto()
    FREE_SESSION = auto()
    TIME_SYNC = auto()
    DECIDE_EXIT = auto()
    EXIT_ALL = auto()


@dataclass
class Instruction:
    op_type: OpType
    params: Dict[str, Any] = field(default_factory=dict)


@dataclass
class Patch:
    image_idx: int
    spatial_idx: int
    res_level: int = 0
    group_id: int = 1
    pscore_hint: float = 0.0


@dataclass
class Task:
    task_id: int
    request_id: int
    payload: List[Patch]
    instructions: List[Instruction]


@dataclass
class InferenceResult:
    task_id: int
    timestamp: float
    output: Any
    server_events: List[Dict[str, Any]] = field(default_factory=list)
    cache_size_bytes: int = 0
    cache_breakdown_bytes: Dict[str, int] = field(default_factory=dict)
    token_pscore_kept_mass: float = 0.0
    token_pscore_full_mass: float = 0.0
    partial_token_kept_patch: float = 0.0
    partial_token_full_patch: float = 0.0
    partial_token_sample_count: float = 0.0
