"""Per-(layer, kv head) FP8 KV scales on the GPU (no reference counterpart: the
reference stores K/V with a bare cast, compact_kv.py:243-252, and dequantises
with one, compact_attention.py:387, 399).  A scale s stores x * fp32(1 / s)
as e4m3 and dequantises fp8 * s in the attention kernel's registers.

* scale 1 everywhere gives bit-identical results to the unscaled calls (the
  parity mode);
* the stored FP8 rows (prefill pack, decode append) are bit-exact against the
  oracle's scaled quantisation;
* attention over scaled storage is within 2e-2 (max-abs-relative) of the
  oracle's float64 attention over the same scaled storage, on BASELINE
  configs[0]-style inputs (B=1, 32 / 8 heads, D=64, 2048 tokens: the last 256
  kept, older ones kept with probability 1/8), flat and paged (16-token pages
  under a random permutation);
* the engine in "calibrate" mode follows the oracle model in the same mode.
"""
import numpy as np
import pytest
import torch

from helpers import from_values, require_gpu, storage_of, values_of
from oracle import attention as oatt
from oracle import compact_kv as ock
from oracle import numerics

pytestmark = pytest.mark.gpu


def _rel(got, ref):
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def _scales(rng, h, lo=0.02, hi=4.0):
    return np.exp(rng.uniform(np.log(lo), np.log(hi), h)).astype(np.float32)


@pytest.mark.parametrize("unit", [False, True])
def test_pack_with_scales_bit_exact(unit):
    """Ragged two-sequence prefill pack with per-head scales: FP8 rows equal
    the oracle's scaled quantisation; unit scales equal the unscaled pack."""
    require_gpu()
    from fastdms_amd.engine.compact_kv import _streaming_pack_rank_scatter_hip
    rng = np.random.default_rng(3 + unit)
    T, H, D, W = 700, 8, 64, 64
    k = numerics.cast(rng.standard_normal((T, H, D)).astype(np.float32) * 6, numerics.DT_BF16)
    v = numerics.cast(rng.standard_normal((T, H, D)).astype(np.float32) * 0.05, numerics.DT_BF16)
    evict = rng.random((T, H)) < 0.8
    ks = np.ones(H, np.float32) if unit else _scales(rng, H)
    vs = np.ones(H, np.float32) if unit else _scales(rng, H, 1e-3, 0.1)
    cap = T
    base = (np.arange(H) * cap).astype(np.int32)
    live, offs = ock.streaming_pack_fused_rank_prepare(evict, T, W)
    outs = []
    for scaled in (True, False):
        ck = torch.zeros((H * cap, D), dtype=torch.uint8, device="cuda").view(torch.float8_e4m3fn)
        cv = torch.zeros_like(ck)
        pos = torch.full((H, cap), -1, dtype=torch.int32, device="cuda")
        em = torch.zeros((H, cap), dtype=torch.bool, device="cuda")
        kw = dict(k_scale=torch.from_numpy(ks).cuda(), v_scale=torch.from_numpy(vs).cuda()) if scaled else {}
        _streaming_pack_rank_scatter_hip(k=from_values(k, numerics.DT_BF16), v=from_values(v, numerics.DT_BF16),
                                         seq_evict=torch.from_numpy(evict).cuda(),
                                         block_offsets=torch.from_numpy(np.ascontiguousarray(offs)).cuda(),
                                         compact_k=ck, compact_v=cv, token_positions=pos, evict_mask=em,
                                         base_offsets=torch.from_numpy(base).cuda(), start=0, seq_len=T,
                                         window_size=W, **kw)
        torch.cuda.synchronize()
        outs.append((storage_of(ck), storage_of(cv)))
    ck_o = np.zeros((H * cap, D), np.uint8)
    cv_o = np.zeros_like(ck_o)
    ock.streaming_pack_rank_scatter(k=k, v=v, seq_evict=evict, compact_k=ck_o, compact_v=cv_o,
                                    token_positions=np.full((H, cap), -1, np.int32),
                                    evict_mask=np.zeros((H, cap), bool), base_offsets=base, start=0, seq_len=T,
                                    window_size=W, dtype_code=numerics.DT_FP8, k_scale=ks, v_scale=vs)
    assert np.array_equal(outs[0][0], ck_o) and np.array_equal(outs[0][1], cv_o)
    if unit:
        assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])


def _config0(rng, ctx=2048, window=256, hkv=8, g=4, d=64):
    keep = rng.random((hkv, ctx)) < 1.0 / 8
    keep[:, ctx - window:] = True
    return keep


@pytest.mark.parametrize("paged", [False, True])
def test_attention_with_scales_matches_oracle(paged):
    """configs[0]-style single-layer decode attention over scaled FP8
    storage; unit scales give the unscaled kernel's output bit for bit."""
    require_gpu()
    from fastdms_amd.layers.compact_attention import compact_decode_attention, compact_decode_attention_paged
    rng = np.random.default_rng(11 + paged)
    hkv, g, d, page = 8, 4, 64, 16
    keep = _config0(rng)
    live = keep.sum(-1).astype(np.int32).reshape(1, hkv)
    # K / V far from the unit range (large K, small V): the scales bring them into it
    kt = rng.standard_normal((hkv, 2048, d)).astype(np.float32) * 900.0
    vt = rng.standard_normal((hkv, 2048, d)).astype(np.float32) * 2e-3
    ks = (np.abs(kt).max(axis=(1, 2)) / 224.0).astype(np.float32)
    vs = (np.abs(vt).max(axis=(1, 2)) / 224.0).astype(np.float32)
    cap = int(live.max())
    rows = np.zeros((hkv * cap, d), np.float32), np.zeros((hkv * cap, d), np.float32)
    base = (np.arange(hkv) * cap).astype(np.int32).reshape(1, hkv)
    for h in range(hkv):
        sel = np.nonzero(keep[h])[0]
        rows[0][h * cap:h * cap + len(sel)] = kt[h, sel] * (np.float32(1) / ks[h])
        rows[1][h * cap:h * cap + len(sel)] = vt[h, sel] * (np.float32(1) / vs[h])
    ck = numerics.to_storage(rows[0], numerics.DT_FP8)
    cv = numerics.to_storage(rows[1], numerics.DT_FP8)
    q = numerics.cast(rng.standard_normal((1, hkv * g, d)).astype(np.float32) * 0.01, numerics.DT_BF16)
    ref = oatt.compact_decode_attention(q, numerics.from_storage(ck, numerics.DT_FP8),
                                        numerics.from_storage(cv, numerics.DT_FP8), base, live, k_scale=ks,
                                        v_scale=vs)
    qd = from_values(q, numerics.DT_BF16)
    ksd, vsd = torch.from_numpy(ks).cuda(), torch.from_numpy(vs).cuda()
    if paged:
        npg = -(-cap // page)
        perm = rng.permutation(hkv * npg).astype(np.int32)
        table = perm.reshape(1, hkv, npg)
        ckp, cvp = np.zeros((hkv * npg * page, d), np.uint8), np.zeros((hkv * npg * page, d), np.uint8)
        for h in range(hkv):
            for pg in range(npg):
                n = min(page, cap - pg * page)
                src = slice(h * cap + pg * page, h * cap + pg * page + n)
                dst = slice(int(table[0, h, pg]) * page, int(table[0, h, pg]) * page + n)
                ckp[dst], cvp[dst] = ck[src], cv[src]
        ckd = torch.from_numpy(ckp).cuda().view(torch.float8_e4m3fn)
        cvd = torch.from_numpy(cvp).cuda().view(torch.float8_e4m3fn)
        run = lambda **kw: compact_decode_attention_paged(qd, ckd, cvd, torch.from_numpy(table).cuda(),
                                                          torch.from_numpy(live).cuda(), page_size=page, **kw)
    else:
        ckd = torch.from_numpy(ck).cuda().view(torch.float8_e4m3fn)
        cvd = torch.from_numpy(cv).cuda().view(torch.float8_e4m3fn)
        run = lambda **kw: compact_decode_attention(qd, ckd, cvd, torch.from_numpy(base).cuda(),
                                                    torch.from_numpy(live).cuda(), **kw)
    out = run(k_scale=ksd, v_scale=vsd)
    ones = torch.ones(hkv, device="cuda")
    out1, out0 = run(k_scale=ones, v_scale=ones), run()
    torch.cuda.synchronize()
    assert _rel(values_of(out), ref) <= 2e-2
    assert torch.equal(out1, out0)


def test_fused_decode_with_scales_matches_oracle():
    """The fused decision / RoPE / scaled FP8 append / attention launch: the
    appended rows bit-exact against the oracle's scaled store, the output
    within 2e-2 of the oracle's attention over the scaled span."""
    require_gpu()
    import fastdms_amd.layers.compact_attention as ca
    rng = np.random.default_rng(5)
    b, hq, hkv, d, cap = 4, 32, 8, 64, 1200
    g = hq // hkv
    live_prev = rng.integers(100, 1100, (b, hkv)).astype(np.int32)
    base = (np.arange(b * hkv).reshape(b, hkv) * cap).astype(np.int32)
    slot = base + live_prev
    live = live_prev + 1
    ks, vs = _scales(rng, hkv, 0.5, 8.0), _scales(rng, hkv, 0.01, 0.2)
    qkv = numerics.cast(rng.standard_normal((b, (hq + 2 * hkv) * d)).astype(np.float32) * 3, numerics.DT_BF16)
    q = qkv[:, :hq * d].reshape(b, hq, d).copy()
    k = qkv[:, hq * d:(hq + hkv) * d].reshape(b, hkv, d).copy()
    v = qkv[:, (hq + hkv) * d:].reshape(b, hkv, d).copy()
    positions = rng.integers(2000, 8000, b)
    cache = oatt.rope_cos_sin_cache(d, 8192, 500000.0)
    ck = numerics.to_storage(rng.standard_normal((b * hkv * cap, d)).astype(np.float32), numerics.DT_FP8)
    cv = numerics.to_storage(rng.standard_normal((b * hkv * cap, d)).astype(np.float32), numerics.DT_FP8)
    qo, cko, cvo = q.copy(), ck.copy(), cv.copy()
    ev = oatt.fused_dms_rope_store_compact_decode(q=qo, k=k.copy(), v=v, cos_sin_cache=cache, compact_k=cko,
                                                  compact_v=cvo, slot_mapping=slot, positions=positions,
                                                  num_kv_heads=hkv, alpha_scale=10.0, alpha_offset=5.0,
                                                  q_dtype_code=numerics.DT_BF16, k_dtype_code=numerics.DT_BF16,
                                                  compact_dtype_code=numerics.DT_FP8, store_q=True,
                                                  store_transient_k=False, k_scale=ks, v_scale=vs)
    ref = oatt.compact_decode_attention(qo, numerics.from_storage(cko, numerics.DT_FP8),
                                        numerics.from_storage(cvo, numerics.DT_FP8), base, live, k_scale=ks,
                                        v_scale=vs)
    qkv_d = from_values(qkv, numerics.DT_BF16)
    ckd = torch.from_numpy(ck).cuda().view(torch.float8_e4m3fn)
    cvd = torch.from_numpy(cv).cuda().view(torch.float8_e4m3fn)
    evd = torch.empty((b, hkv), device="cuda", dtype=torch.bool)
    out = ca.fused_dms_rope_store_compact_decode_attention(
        qkv_d[:, :hq * d].view(b, hq, d), qkv_d[:, hq * d:(hq + hkv) * d].view(b, hkv, d),
        qkv_d[:, (hq + hkv) * d:].view(b, hkv, d), torch.from_numpy(cache).cuda(), ckd, cvd,
        torch.from_numpy(slot).cuda(), evd, torch.from_numpy(positions).cuda(), torch.from_numpy(base).cuda(),
        torch.from_numpy(live).cuda(), num_kv_heads=hkv, alpha_scale=10.0, alpha_offset=5.0, max_live_count=cap,
        k_scale=torch.from_numpy(ks).cuda(), v_scale=torch.from_numpy(vs).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(evd.cpu().numpy(), ev)
    assert np.array_equal(storage_of(ckd), cko) and np.array_equal(storage_of(cvd), cvo)
    assert _rel(values_of(out), ref) <= 2e-2


def test_engine_calibrated_scales_follow_the_oracle():
    """The engine with compact_kv_fp8_scales="calibrate" (scales from each
    layer's first prefill): the scale tables equal the oracle model's, and
    each decode step's logits (oracle on the GPU's compact state) stay within
    the tolerance of the unscaled engine test."""
    require_gpu()
    import test_gpu_engine as tge
    from oracle.model import OracleModel, weights_from_model
    from fastdms_amd import LLM, SamplingParams
    rng = np.random.default_rng(9)
    prompts = [rng.integers(0, 512, n).tolist() for n in (300, 517, 800, 64)]
    llm = LLM("tiny-llama", max_model_len=2048, max_num_seqs=8, max_num_batched_tokens=16384,
              fused_greedy_head=False, compact_kv_fp8_scales="calibrate", **tge.DMS)
    runner = llm.model_runner
    saved = torch.nn.functional.linear
    torch.nn.functional.linear = tge._fp32_linear
    try:
        orc = OracleModel(weights_from_model(runner.model), llm.config.hf_config, window_size=32, alpha_scale=10.0,
                          alpha_offset=5.0, capacity_tokens=runner.compact_kv_manager.capacity_tokens,
                          max_model_len=llm.config.max_model_len, fp8_scales="calibrate")
        sp = SamplingParams(temperature=0.0, max_tokens=12, ignore_eos=True)
        seqs = [llm.add_request(p, sp) for p in prompts]
        llm.step()
        orc.prefill([(s.seq_id, s.prompt_token_ids, 12) for s in seqs])
        mgr = runner.compact_kv_manager
        got_scales = mgr.kv_scales.cpu().numpy()
        # the same amax / 224 of the layer's packed rows (a bf16 ulp apart at
        # most, where GEMM order moved the largest element)
        assert np.allclose(got_scales, orc.kv_scales, rtol=1e-2), "calibrated scales differ"
        assert not np.allclose(got_scales, 1.0)
        orc.kv_scales[:] = got_scales  # decode from the GPU's tables, as from its compact state
        worst = 0.0
        for _ in range(11):
            torch.cuda.synchronize()
            tge._sync_oracle_state(orc, mgr, seqs)
            orc.decode([s.seq_id for s in seqs], [s.last_token for s in seqs], [len(s) - 1 for s in seqs])
            llm.step()
            got = runner.model.lm_head.last_logits.float().cpu()
            want = orc.last_logits
            worst = max(worst, float((got - want).pow(2).mean().sqrt() / want.pow(2).mean().sqrt()))
        llm.exit()
    finally:
        torch.nn.functional.linear = saved
    assert worst <= 1e-2, worst
