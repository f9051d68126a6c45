"""Host logic of the FP8 / INT4 weight paths: the environment switches
(linear.py:17-361, embed_head.py:28-85) and the dispatch order of
LinearBase._linear (linear.py:855-926) and the LM head (embed_head.py:491-598).
No kernels run: the modules get their flags set directly."""
import pytest
import torch

from fastdms_amd.layers import quant_env as qe
from fastdms_amd.layers.embed_head import ParallelLMHead
from fastdms_amd.layers.linear import QX_DIVIDE, QX_NONE, QX_TORCH, LinearBase

_ENV = [k for k in __import__("os").environ if k.startswith("FASTDMS_")]


@pytest.fixture(autouse=True)
def _clean_env(monkeypatch):
    for k in _ENV:
        monkeypatch.delenv(k, raising=False)


def _lin(name, *, keep=True, row1_only=False, int4=False, k=2048, n=2048):
    m = LinearBase(k, n)
    m._fp8_weight_enabled = True
    m._fp8_module_name = name
    m._fp8_row1_only = row1_only
    m._fp8_min_rows = qe.fp8_module_min_rows(name)
    m._int4_enabled = int4
    if not keep:
        m._drop_bf16_weight()
    return m


def test_defaults_follow_reference():
    assert not qe.fp8_weights_enabled() and qe.fp8_weight_scope() == "mlp"
    assert qe.fp8_keep_bf16_weights() and qe.fp8_min_rows() == 2
    assert qe.fp8_down_row1_mode() == "quantized" and qe.fp8_gate_up_row1_mode() == "quantized"
    assert qe.fp8_attention_row1_mode() == "quantized" and qe.fp8_row1_mode() == "off"
    assert qe.fp8_small_m_enabled() and qe.fp8_small_m_max_rows() == 8
    assert qe.int4_group_size() == 256 and qe.int4_quant_mode() == "symmetric" and qe.int4_max_rows() == 1
    assert qe.int4_lm_head_rerank_topk() == 0 and qe.greedy_fused_argmax_enabled()
    # gate_up / down / attention drop their bf16 weight unless the global switch is set explicitly
    assert not qe.fp8_module_keep_bf16_weight("model.layers.0.mlp.gate_up_proj")
    assert qe.fp8_module_keep_bf16_weight("model.layers.0.other")


def test_env_parsing_errors(monkeypatch):
    monkeypatch.setenv("FASTDMS_FP8_DOWN_ROW1_TRITON", "maybe")
    with pytest.raises(ValueError):
        qe.fp8_down_row1_mode()
    monkeypatch.setenv("FASTDMS_INT4_ROW1_GROUP_SIZE", "48")
    with pytest.raises(ValueError):
        qe.int4_group_size()
    monkeypatch.setenv("FASTDMS_INT4_ROW1_LM_HEAD_RERANK_TOPK", "3")
    with pytest.raises(ValueError):
        qe.int4_lm_head_rerank_topk()
    with pytest.raises(ValueError):
        qe.fp8_module_in_scope("x", "bogus")


def test_int4_scope_and_layer_filters(monkeypatch):
    monkeypatch.setenv("FASTDMS_INT4_ROW1_WEIGHTS", "1")
    monkeypatch.setenv("FASTDMS_INT4_ROW1_SCOPE", "mlp_down@even|5-6+qkv@1")
    assert qe.int4_module_in_scope("model.layers.2.mlp.down_proj")
    assert qe.int4_module_in_scope("model.layers.5.mlp.down_proj")
    assert not qe.int4_module_in_scope("model.layers.7.mlp.down_proj")
    assert not qe.int4_module_in_scope("model.layers.2.mlp.gate_up_proj")
    assert qe.int4_module_in_scope("model.layers.1.self_attn.qkv_proj")
    assert not qe.int4_lm_head_enabled()          # every part carries a layer filter
    monkeypatch.setenv("FASTDMS_INT4_ROW1_SCOPE", "mlp+lm_head")
    assert qe.int4_lm_head_enabled() and not qe.int4_module_in_scope("model.layers.0.self_attn.o_proj")
    monkeypatch.setenv("FASTDMS_INT4_ROW1_SCOPE", "none")
    assert not qe.int4_module_in_scope("model.layers.0.mlp.down_proj") and not qe.int4_lm_head_enabled()
    monkeypatch.setenv("FASTDMS_INT4_ROW1_SCOPE", "mlp@")
    with pytest.raises(ValueError):
        qe.int4_module_in_scope("model.layers.0.mlp.down_proj")


def test_linear_dispatch_order(monkeypatch):
    gu = _lin("model.layers.0.mlp.gate_up_proj", keep=False)
    assert gu.route(1) == ("fp8", QX_DIVIDE)             # row-1 kernel, quantised activation
    assert gu.route(4) == ("fp8", QX_DIVIDE)             # small-M kernel
    assert gu.route(8) == ("fp8", QX_DIVIDE)
    assert gu.route(9) == ("fp8", QX_TORCH)              # _fp8_linear (scaled_mm)
    # down with its bf16 weight kept: the row-1 mode is off, one row is below the FP8 minimum
    down = _lin("model.layers.0.mlp.down_proj", keep=True)
    assert down.route(1) == ("bf16", QX_NONE)
    assert down.route(2) == ("fp8", QX_DIVIDE)
    # raw row-1 mode: unquantised activation
    monkeypatch.setenv("FASTDMS_FP8_GATE_UP_ROW1_TRITON", "raw_unsafe")
    assert gu.route(1) == ("fp8", QX_NONE)
    # row-1-only attention shadow: bf16 beyond one row
    attn = _lin("model.layers.0.self_attn.qkv_proj", row1_only=True)
    assert attn.route(1) == ("fp8", QX_DIVIDE) and attn.route(4) == ("bf16", QX_NONE)
    # INT4 shadow first while the row-1 mode is on
    i4 = _lin("model.layers.0.mlp.gate_up_proj", keep=False, int4=True)
    monkeypatch.delenv("FASTDMS_FP8_GATE_UP_ROW1_TRITON")
    assert i4.route(1) == ("int4", QX_NONE) and i4.route(2) == ("fp8", QX_DIVIDE)
    monkeypatch.setenv("FASTDMS_INT4_ROW1_MAX_ROWS", "4")
    assert i4.route(4) == ("int4", QX_NONE) and i4.route(5) == ("fp8", QX_DIVIDE)
    monkeypatch.setenv("FASTDMS_FP8_GATE_UP_ROW1_TRITON", "0")
    assert i4.route(1) == ("fp8", QX_TORCH)              # INT4 needs the row-1 mode; weight dropped -> FP8
    # small-M switched off, dequant implementation
    monkeypatch.setenv("FASTDMS_FP8_SMALL_M_TRITON", "0")
    monkeypatch.setenv("FASTDMS_FP8_LINEAR_IMPL", "dequant")
    assert gu.route(4) == ("fp8_dequant", QX_NONE)
    assert LinearBase(256, 256).route(1) == ("bf16", QX_NONE)


def test_lm_head_dispatch(monkeypatch):
    h = ParallelLMHead(4096, 2048)
    assert h.route(1) == ("bf16", 0) and h.greedy_route(8) == ("bf16", 0, True)
    h._fp8_weight_enabled = True
    h._fp8_min_rows = qe.fp8_lm_head_min_rows()
    # bf16 weight kept, one row: below the FP8 minimum (2) -> bf16
    assert h.route(1) == ("bf16", 0)
    assert h.route(2) == ("fp8", QX_TORCH) and h.greedy_route(2) == ("fp8", QX_TORCH, True)
    h._drop_bf16_weight()
    assert h.route(1) == ("fp8", QX_DIVIDE)
    assert h.greedy_route(1) == ("fp8", QX_DIVIDE, False)   # row-1 argmax: fp32 scores
    h._int4_enabled = True
    assert h.route(1) == ("int4", 0) and h.greedy_route(1) == ("int4", 0, True)
    monkeypatch.setenv("FASTDMS_INT4_ROW1_LM_HEAD_RERANK_TOPK", "8")
    assert h.route(1) == ("fp8", QX_DIVIDE) and h.greedy_route(1)[0] == "int4_rerank"
    assert h.greedy_route(3) == ("fp8", QX_TORCH, True)
    monkeypatch.setenv("FASTDMS_FP8_LM_HEAD_ROW1_TRITON", "0")
    assert h.route(1) == ("fp8", QX_TORCH)


def test_convert_linear_modules_scope(monkeypatch):
    """linear.py:1076-1095 scope selection, with quantisation itself stubbed."""
    from torch import nn
    from fastdms_amd.layers import linear as L
    calls = []
    monkeypatch.setattr(L.LinearBase, "quantize_weight_to_fp8",
                        lambda self, **kw: calls.append((kw["module_name"], kw["keep_bf16_weight"], kw["row1_only"])))
    root = nn.Module()
    root.layers = nn.ModuleList([nn.Module()])
    blk = root.layers[0]
    blk.self_attn, blk.mlp = nn.Module(), nn.Module()
    blk.self_attn.qkv_proj = L.LinearBase(256, 256)
    blk.mlp.gate_up_proj = L.LinearBase(256, 512)
    blk.mlp.down_proj = L.LinearBase(256, 256)
    assert L.convert_linear_modules_to_fp8(root) == 3    # mlp scope + attention (full by default)
    assert ("layers.0.self_attn.qkv_proj", False, False) in calls
    calls.clear()
    monkeypatch.setenv("FASTDMS_FP8_ATTENTION_FULL", "0")
    assert L.convert_linear_modules_to_fp8(root) == 3
    assert ("layers.0.self_attn.qkv_proj", True, True) in calls   # row-1-only shadow keeps bf16
    calls.clear()
    monkeypatch.setenv("FASTDMS_FP8_ATTENTION_ROW1_SHADOW", "0")
    monkeypatch.setenv("FASTDMS_FP8_WEIGHT_SCOPE", "mlp_down")
    assert L.convert_linear_modules_to_fp8(root) == 1 and calls[0][0] == "layers.0.mlp.down_proj"


def test_norm_stats_buffers_must_match_the_strips():
    """The split RMSNorm's statistics buffer is exactly [rows, N / 16]: the
    producer writes row * strips + strip and the consumer sums every column
    of its row into the norm, so a wider buffer is rejected before any launch
    (CPU tensors: the shape checks come first)."""
    from fastdms_amd.layers.linear import EPI_SILU_MUL, linear_norm_stats, linear_residual_stats
    rows, k, n = 8, 2048, 4096
    x = torch.zeros(rows, k, dtype=torch.bfloat16)
    w = torch.zeros(n, k, dtype=torch.bfloat16)
    res = torch.zeros(rows, n, dtype=torch.bfloat16)
    f = torch.zeros(rows, n)
    with pytest.raises(ValueError, match="ssq_out"):
        linear_residual_stats(x, w, res, f, torch.zeros(rows, n // 16 + 16))
    with pytest.raises(ValueError, match="ssq_out"):
        linear_residual_stats(x, w, res, f, torch.zeros(rows * n // 16 + 64))
    nw = torch.ones(n, dtype=torch.bfloat16)
    w2 = torch.zeros(2 * 1024, n, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ssq must be"):
        linear_norm_stats(f, torch.zeros(rows, n // 16 + 1), nw, 1e-5, w2, epilogue=EPI_SILU_MUL)
    with pytest.raises(ValueError, match="ssq must be"):
        linear_norm_stats(f, torch.zeros(rows, n // 32), nw, 1e-5, w2, epilogue=EPI_SILU_MUL)
