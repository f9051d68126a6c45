"""Environment switches of the FP8 / INT4 weight paths.

The variable names, defaults, accepted spellings and errors are the
reference's (fastdms/layers/linear.py:17-361, 1051-1073 and
fastdms/layers/embed_head.py:28-85), so a deployment configured for the
reference selects the same kernels here.  Every reader is evaluated at call
time, as in the reference.
"""
from __future__ import annotations

import os
import re

_TRUE = {"1", "true", "yes", "on"}
_OFF = {"", "0", "false", "no", "off"}
_QUANTIZED = {"1", "true", "yes", "on", "quant", "quantized", "fp8"}


def env_bool(name: str, default: bool) -> bool:
    """linear.py:39-43: unset or blank -> default."""
    raw = os.environ.get(name)
    if raw is None or raw.strip() == "":
        return default
    return raw.strip().lower() in _TRUE


def _env_choice(name: str, default: int, allowed: set[int]) -> int:
    """linear.py:176-184."""
    raw = os.environ.get(name)
    if raw is None or raw.strip() == "":
        return default
    value = int(raw)
    if value not in allowed:
        raise ValueError(f"{name} must be one of {', '.join(str(v) for v in sorted(allowed))}; got {value}")
    return value


def _min_rows(name: str, default: int) -> int:
    raw = os.environ.get(name)
    if raw is None or raw.strip() == "":
        return default
    return max(1, int(raw))


def _keep_explicit() -> bool:
    raw = os.environ.get("FASTDMS_FP8_KEEP_BF16_WEIGHTS")
    return raw is not None and raw.strip() != ""


# --- FP8 weights (linear.py:17-91) -------------------------------------------

def fp8_weights_enabled() -> bool:
    return os.environ.get("FASTDMS_FP8_WEIGHTS", "0").strip().lower() in _TRUE


def fp8_weight_scope() -> str:
    return os.environ.get("FASTDMS_FP8_WEIGHT_SCOPE", "mlp").strip().lower()


def fp8_keep_bf16_weights() -> bool:
    return os.environ.get("FASTDMS_FP8_KEEP_BF16_WEIGHTS", "1").strip().lower() in _TRUE


def _keep_for(name: str) -> bool:
    return env_bool(name, fp8_keep_bf16_weights() if _keep_explicit() else False)


def fp8_min_rows() -> int:
    return max(1, int(os.environ.get("FASTDMS_FP8_MIN_ROWS", "2")))


def fp8_module_min_rows(module_name: str | None = None) -> int:
    """linear.py:364-371."""
    if module_name and module_name.endswith(".gate_up_proj"):
        return _min_rows("FASTDMS_FP8_GATE_UP_MIN_ROWS", fp8_min_rows())
    if module_name and module_name.endswith(".down_proj"):
        return _min_rows("FASTDMS_FP8_DOWN_MIN_ROWS", fp8_min_rows())
    return fp8_min_rows()


def fp8_module_keep_bf16_weight(module_name: str | None = None) -> bool:
    """linear.py:374-383."""
    if module_name is None:
        return fp8_keep_bf16_weights()
    if ".self_attn." in module_name:
        return _keep_for("FASTDMS_FP8_KEEP_BF16_ATTENTION")
    if module_name.endswith(".gate_up_proj"):
        return _keep_for("FASTDMS_FP8_KEEP_BF16_GATE_UP")
    if module_name.endswith(".down_proj"):
        return _keep_for("FASTDMS_FP8_KEEP_BF16_DOWN")
    return fp8_keep_bf16_weights()


def _row1_mode(name: str, default: str) -> str:
    raw = os.environ.get(name, default).strip().lower()
    if raw in _OFF:
        return "off"
    if raw in _QUANTIZED:
        return "quantized"
    if raw == "raw_unsafe":
        return "raw"
    raise ValueError(f"{name} must be off, quantized, or raw_unsafe")


def fp8_down_row1_mode() -> str:
    return _row1_mode("FASTDMS_FP8_DOWN_ROW1_TRITON", "quantized")


def fp8_gate_up_row1_mode() -> str:
    return _row1_mode("FASTDMS_FP8_GATE_UP_ROW1_TRITON", "quantized")


def fp8_attention_row1_shadow_enabled() -> bool:
    return env_bool("FASTDMS_FP8_ATTENTION_ROW1_SHADOW", True)


def fp8_attention_full_enabled() -> bool:
    return env_bool("FASTDMS_FP8_ATTENTION_FULL", True)


def fp8_attention_row1_mode() -> str:
    shadow_or_full = fp8_attention_row1_shadow_enabled() or fp8_attention_full_enabled()
    return _row1_mode("FASTDMS_FP8_ATTENTION_ROW1_TRITON", "quantized" if shadow_or_full else "0")


def fp8_row1_mode() -> str:
    return _row1_mode("FASTDMS_FP8_ROW1_TRITON", "0")


def fp8_small_m_enabled() -> bool:
    return env_bool("FASTDMS_FP8_SMALL_M_TRITON", True)


def fp8_small_m_max_rows() -> int:
    return _env_choice("FASTDMS_FP8_SMALL_M_TRITON_MAX_ROWS", 8, {2, 4, 8, 16})


_SCOPE_ERR = ("FASTDMS_FP8_WEIGHT_SCOPE must be one of all, mlp, attention, "
              "qkv, attn_out, mlp_gate_up, mlp_down, lm_head, mlp_lm_head; got {!r}")


def _name_in_scope(scope: str, name: str) -> bool | None:
    """Module-name test shared by the FP8 and INT4 scopes (linear.py:1051-1073,
    271-290); None for an unknown scope."""
    if scope in {"all", "transformer"}:
        return True
    if scope in {"lm_head", "head"}:
        return False
    if scope in {"mlp_lm_head", "mlp+lm_head", "mlp_head", "mlp+head", "mlp", "ffn"}:
        return ".mlp." in name
    if scope in {"attention", "attn"}:
        return ".self_attn." in name
    if scope == "qkv":
        return name.endswith(".qkv_proj")
    if scope in {"attn_out", "o_proj"}:
        return name.endswith(".o_proj")
    if scope in {"mlp_gate_up", "gate_up"}:
        return name.endswith(".gate_up_proj")
    if scope in {"mlp_down", "down"}:
        return name.endswith(".down_proj")
    return None


def fp8_module_in_scope(name: str, scope: str) -> bool:
    hit = _name_in_scope(scope, name)
    if hit is None:
        raise ValueError(_SCOPE_ERR.format(scope))
    return hit


# --- INT4 row-1 weights (linear.py:203-361) ----------------------------------

def int4_weights_enabled() -> bool:
    return env_bool("FASTDMS_INT4_ROW1_WEIGHTS", False)


def int4_scope_parts() -> list[str]:
    scope = os.environ.get("FASTDMS_INT4_ROW1_SCOPE", "all").strip().lower()
    parts = [p.strip() for p in scope.replace(",", "+").split("+") if p.strip()]
    return parts or ["none"]


def _layer_id(module_name: str | None) -> int | None:
    if not module_name:
        return None
    m = re.search(r"(?:^|\.)layers\.(\d+)(?:\.|$)", module_name)
    return None if m is None else int(m.group(1))


def _layer_filter_allows(filt: str | None, module_name: str | None) -> bool:
    """``scope@layers`` filters (linear.py:221-257): all / * / even / odd / a-b
    ranges / single ids, joined with '|'."""
    if not filt:
        return True
    value = filt.strip().lower()
    if value in {"all", "*"}:
        return True
    lid = _layer_id(module_name)
    if lid is None:
        return False
    for item in (i.strip() for i in value.split("|")):
        if not item:
            continue
        if item in ("even", "odd"):
            if lid % 2 == (0 if item == "even" else 1):
                return True
        elif "-" in item:
            lo, hi = item.split("-", 1)
            if int(lo) <= lid <= int(hi):
                return True
        elif lid == int(item):
            return True
    return False


def _split_filter(scope: str) -> tuple[str, str | None]:
    if "@" not in scope:
        return scope, None
    base, filt = scope.split("@", 1)
    if not base or not filt:
        raise ValueError(f"FASTDMS_INT4_ROW1_SCOPE layer filters must use scope@layers, got {scope!r}")
    return base, filt


_INT4_SCOPE_ERR = ("FASTDMS_INT4_ROW1_SCOPE must be one or more of all, transformer, mlp, attention, "
                   "qkv, attn_out, mlp_gate_up, mlp_down, lm_head, mlp_lm_head, none; got {!r}")


def int4_module_in_scope(module_name: str | None) -> bool:
    """linear.py:271-297."""
    for part in int4_scope_parts():
        scope, filt = _split_filter(part)
        if not _layer_filter_allows(filt, module_name):
            continue
        if scope in {"none", "off", "0", "false"}:
            continue
        hit = _name_in_scope(scope, module_name or "")
        if hit is None:
            raise ValueError(_INT4_SCOPE_ERR.format(scope))
        if hit:
            return True
    return False


def int4_lm_head_enabled() -> bool:
    """linear.py:300-331: a filter-free all / lm_head / mlp_lm_head part."""
    if not int4_weights_enabled():
        return False
    for part in int4_scope_parts():
        scope, filt = _split_filter(part)
        if filt is not None:
            continue
        if scope in {"all", "lm_head", "head", "mlp_lm_head", "mlp_head"}:
            return True
        if _name_in_scope(scope, "") is None and scope not in {"none", "off", "0", "false"}:
            raise ValueError(_INT4_SCOPE_ERR.format(scope))
    return False


def int4_group_size() -> int:
    return _env_choice("FASTDMS_INT4_ROW1_GROUP_SIZE", 256, {32, 64, 128, 256})


def int4_quant_mode() -> str:
    raw = os.environ.get("FASTDMS_INT4_ROW1_QUANT_MODE", "symmetric").strip().lower()
    if raw in {"", "sym", "symmetric"}:
        return "symmetric"
    if raw in {"asym", "asymmetric", "affine"}:
        return "asymmetric"
    raise ValueError("FASTDMS_INT4_ROW1_QUANT_MODE must be symmetric or asymmetric")


def int4_max_rows() -> int:
    return _env_choice("FASTDMS_INT4_ROW1_MAX_ROWS", 1, {1, 2, 4, 8, 16})


# --- LM head (embed_head.py:28-85) -------------------------------------------

def fp8_lm_head_enabled() -> bool:
    explicit = os.environ.get("FASTDMS_FP8_LM_HEAD")
    if explicit is not None:
        return explicit.strip().lower() in _TRUE
    return fp8_weight_scope() in {"lm_head", "head", "mlp_lm_head", "mlp+lm_head", "mlp_head", "mlp+head"}


def fp8_lm_head_min_rows() -> int:
    return _min_rows("FASTDMS_FP8_LM_HEAD_MIN_ROWS", fp8_min_rows())


def fp8_keep_bf16_lm_head_weight() -> bool:
    return env_bool("FASTDMS_FP8_KEEP_BF16_LM_HEAD", fp8_keep_bf16_weights())


def fp8_lm_head_row1_enabled() -> bool:
    return env_bool("FASTDMS_FP8_LM_HEAD_ROW1_TRITON", True)


def greedy_fused_argmax_enabled() -> bool:
    return env_bool("FASTDMS_GREEDY_FUSED_ARGMAX", True)


def int4_lm_head_rerank_topk() -> int:
    raw = os.environ.get("FASTDMS_INT4_ROW1_LM_HEAD_RERANK_TOPK")
    if raw is None or raw.strip() == "" or raw.strip().lower() in {"0", "false", "no", "off"}:
        return 0
    value = int(raw)
    if value not in {2, 4, 8, 16, 32}:
        raise ValueError("FASTDMS_INT4_ROW1_LM_HEAD_RERANK_TOPK must be one of 0, 2, 4, 8, 16, 32")
    return value
