"""The CPU model oracle for an engine's model (test helper): its weights, and
for converted linears their FP8 / INT4 weights plus the module's own routing
decision per row count, so the oracle follows the engine's dispatch."""
from __future__ import annotations

import torch


def int4_weights(module):
    """Dequantised INT4 shadow of a linear: bf16((q - 8) * scale + zero)."""
    packed = module.weight_int4.cpu()
    q = torch.stack([packed & 0xF, packed >> 4], dim=-1).reshape(packed.shape[0], -1).float()
    g = module._int4_group_size
    sz = module.weight_int4_scale_zeros.float().cpu()  # [K/group, N, 2] (the reference's layout)
    s = sz[:, :, 0].t().repeat_interleave(g, dim=1)
    z = sz[:, :, 1].t().repeat_interleave(g, dim=1)
    return ((q - 8.0) * s + z).to(torch.bfloat16).float()


def oracle_for(runner, config, *, quant: bool, dms: dict, capacity_tokens: int | None = None):
    """The CPU model oracle holding ``runner``'s weights; with ``quant`` the
    FP8 / INT4 weights of the converted linears and the modules' own route
    decisions, so it computes what the engine's dispatch computes.
    ``capacity_tokens``: the oracle's span arena per layer (default the
    engine's)."""
    from oracle.model import OracleModel, weights_from_model
    model = runner.model
    kw = {}
    if quant:
        fp8, int4 = {}, {}
        for name, mod in model.named_modules():
            if getattr(mod, "_fp8_weight_enabled", False) and name != "lm_head":
                fp8[name] = (mod.weight_fp8.t().contiguous().view(torch.uint8).cpu().numpy(),
                             mod.weight_scale_inv.float().cpu().numpy())
                if getattr(mod, "_int4_enabled", False):
                    int4[name] = int4_weights(mod)
        emb = model.model.embed_tokens
        if emb._fp8_embedding_enabled:
            kw["embed_fp8"] = (emb._fp8_embedding_weight.view(torch.uint8).cpu().numpy(),
                               emb._fp8_embedding_scale_inv.float().cpu().numpy().reshape(-1))
        mods = dict(model.named_modules())
        from fastdms_amd.layers.linear import QX_NONE, QX_TORCH

        def route(name, rows):
            # the module's own dispatch decision (linear.py:855-926, pinned on
            # the CPU by tests/test_linear_dispatch.py)
            mod = mods.get(name)
            if mod is None or not getattr(mod, "_fp8_weight_enabled", False):
                return "bf16"
            path, qx = mod.route(rows)
            if path == "fp8":
                assert qx != QX_NONE, "unquantised FP8 activations are not modelled by the oracle"
                return "fp8_torch" if qx == QX_TORCH else "fp8"
            assert path in ("int4", "bf16"), path
            return path

        kw.update(fp8_linear=fp8, int4_linear=int4, route=route)
    weights = weights_from_model(model)
    return OracleModel(weights, config.hf_config, window_size=dms["dms_window_size"],
                       alpha_scale=dms["dms_alpha_scale"], alpha_offset=dms["dms_alpha_offset"],
                       capacity_tokens=capacity_tokens or runner.compact_kv_manager.capacity_tokens,
                       max_model_len=config.max_model_len, **kw)
