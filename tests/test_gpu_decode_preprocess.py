"""A9/A10/B8: fused decode DMS + RoPE + append, unfused append and prefill
RoPE on the GPU vs the oracle (bit-exact: RoPE is computed with separately
rounded fp32 products and sums on both sides)."""
import numpy as np
import pytest
import torch

from helpers import TORCH_DTYPE, from_values, require_gpu, storage_of, values_of
from oracle import attention as oatt
from oracle import numerics

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("q_code,cc,store_q,store_k", [
    (numerics.DT_F32, numerics.DT_F32, True, True),     # the reference test's dtypes
    (numerics.DT_F32, numerics.DT_F32, True, False),
    (numerics.DT_F32, numerics.DT_F32, False, True),
    (numerics.DT_BF16, numerics.DT_FP8, True, False),   # engine dtypes
])
def test_fused_preprocess_small_case(q_code, cc, store_q, store_k):
    """B=3, Hkv=2, G=2, D=32 with hand-set decision values (test_compact_kv.py:973-1120)."""
    require_gpu()
    from fastdms_amd.layers.compact_attention import fused_dms_rope_store_compact_decode
    rng = np.random.default_rng(19)
    b, hkv, g, d = 3, 2, 2, 32
    q = numerics.cast(rng.standard_normal((b, hkv * g, d)).astype(np.float32), q_code)
    k = numerics.cast(rng.standard_normal((b, hkv, d)).astype(np.float32), q_code)
    v = numerics.cast(rng.standard_normal((b, hkv, d)).astype(np.float32), q_code)
    q[:, 0::g, -1] = numerics.cast(np.array([[0.01, 0.06], [0.05, 0.08], [0.10, -0.01]], np.float32), q_code)
    positions = np.array([0, 3, 7])
    slot = np.array([[0, 3], [6, 9], [12, 15]], np.int32)
    cache = oatt.rope_cos_sin_cache(d, 16, 10000.0)
    sd = numerics.storage_dtype(cc)
    ck, cv = np.zeros((18, d), sd), np.zeros((18, d), sd)
    qo, ko = q.copy(), k.copy()
    ev = oatt.fused_dms_rope_store_compact_decode(q=qo, k=ko, v=v, cos_sin_cache=cache, compact_k=ck, compact_v=cv,
                                                  slot_mapping=slot, positions=positions, num_kv_heads=hkv,
                                                  alpha_scale=100.0, alpha_offset=5.0, q_dtype_code=q_code,
                                                  k_dtype_code=q_code, compact_dtype_code=cc, store_q=store_q,
                                                  store_transient_k=store_k)
    qd, kd, vd = from_values(q, q_code), from_values(k, q_code), from_values(v, q_code)
    ckd = torch.zeros((18, d), device="cuda", dtype=TORCH_DTYPE[cc])
    cvd = torch.zeros_like(ckd)
    evd = torch.empty((b, hkv), device="cuda", dtype=torch.bool)
    fused_dms_rope_store_compact_decode(qd, kd, vd, torch.from_numpy(cache).cuda(), ckd, cvd,
                                        torch.from_numpy(slot).cuda(), evd, torch.from_numpy(positions).cuda(),
                                        num_kv_heads=hkv, alpha_scale=100.0, alpha_offset=5.0, store_q=store_q,
                                        store_transient_k=store_k)
    torch.cuda.synchronize()
    assert np.array_equal(evd.cpu().numpy(), ev)
    assert np.array_equal(values_of(qd), qo)
    assert np.array_equal(values_of(kd), ko)
    assert np.array_equal(storage_of(ckd), ck) and np.array_equal(storage_of(cvd), cv)


def test_fused_preprocess_llama_shape_strided_views():
    """Llama-3.2-1B decode shape: q/k/v are views of one qkv row (llama.py:92-96), bf16 -> FP8 arena,
    slot -1 skips the append (compact_attention.py:190)."""
    require_gpu()
    from fastdms_amd.layers.compact_attention import fused_dms_rope_store_compact_decode
    rng = np.random.default_rng(5)
    b, hq, hkv, d = 8, 32, 8, 64
    qkv = numerics.cast(rng.standard_normal((b, (hq + 2 * hkv) * d)).astype(np.float32), numerics.DT_BF16)
    q = qkv[:, :hq * d].reshape(b, hq, d).copy()
    k = qkv[:, hq * d:(hq + hkv) * d].reshape(b, hkv, d).copy()
    v = qkv[:, (hq + hkv) * d:].reshape(b, hkv, d).copy()
    positions = rng.integers(0, 8192, b)
    slot = rng.permutation(4 * b * hkv)[:b * hkv].reshape(b, hkv).astype(np.int32)
    slot[2, 3] = -1
    cache = oatt.rope_cos_sin_cache(d, 8192, 500000.0)
    ck = np.zeros((4 * b * hkv, d), np.uint8)
    cv = np.zeros_like(ck)
    qo, ko = q.copy(), k.copy()
    ev = oatt.fused_dms_rope_store_compact_decode(q=qo, k=ko, v=v, cos_sin_cache=cache, compact_k=ck, compact_v=cv,
                                                  slot_mapping=slot, positions=positions, num_kv_heads=hkv,
                                                  alpha_scale=10.0, alpha_offset=5.0, q_dtype_code=numerics.DT_BF16,
                                                  k_dtype_code=numerics.DT_BF16, compact_dtype_code=numerics.DT_FP8,
                                                  store_q=True, store_transient_k=False)
    qkv_d = from_values(qkv, numerics.DT_BF16)
    qd = qkv_d[:, :hq * d].view(b, hq, d)
    kd = qkv_d[:, hq * d:(hq + hkv) * d].view(b, hkv, d)
    vd = qkv_d[:, (hq + hkv) * d:].view(b, hkv, d)
    ckd = torch.zeros((4 * b * hkv, d), device="cuda", dtype=torch.float8_e4m3fn)
    cvd = torch.zeros_like(ckd)
    evd = torch.empty((b, hkv), device="cuda", dtype=torch.bool)
    fused_dms_rope_store_compact_decode(qd, kd, vd, torch.from_numpy(cache).cuda(), ckd, cvd,
                                        torch.from_numpy(slot).cuda(), evd, torch.from_numpy(positions).cuda(),
                                        num_kv_heads=hkv, alpha_scale=10.0, alpha_offset=5.0, store_q=True,
                                        store_transient_k=False)
    torch.cuda.synchronize()
    assert np.array_equal(evd.cpu().numpy(), ev)
    assert np.array_equal(values_of(qd), qo)
    assert np.array_equal(values_of(kd), k)  # transient k not stored
    assert np.array_equal(storage_of(ckd), ck) and np.array_equal(storage_of(cvd), cv)


def test_store_compact_kvcache_matches_oracle():
    require_gpu()
    from fastdms_amd.layers.compact_attention import store_compact_kvcache
    rng = np.random.default_rng(6)
    b, hkv, d = 4, 3, 16
    key = numerics.cast(rng.standard_normal((b, hkv, d)).astype(np.float32), numerics.DT_BF16)
    val = numerics.cast(rng.standard_normal((b, hkv, d)).astype(np.float32), numerics.DT_BF16)
    slot = rng.permutation(40)[:b * hkv].reshape(b, hkv).astype(np.int32)
    slot[0, 0] = -1
    ck = np.zeros((40, d), np.uint8)
    cv = np.zeros_like(ck)
    oatt.store_compact_kvcache(key, val, ck, cv, slot, numerics.DT_FP8)
    ckd = torch.zeros((40, d), device="cuda", dtype=torch.float8_e4m3fn)
    cvd = torch.zeros_like(ckd)
    store_compact_kvcache(from_values(key, numerics.DT_BF16), from_values(val, numerics.DT_BF16), ckd, cvd,
                          torch.from_numpy(slot).cuda())
    torch.cuda.synchronize()
    assert np.array_equal(storage_of(ckd), ck) and np.array_equal(storage_of(cvd), cv)


def test_prefill_rope_matches_apply_rotary_emb():
    require_gpu()
    from fastdms_amd.layers.rotary_embedding import get_rope
    rng = np.random.default_rng(8)
    t, hq, hkv, d = 300, 32, 8, 64
    rope = get_rope(d, d, 8192, 500000.0, {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                                          "high_freq_factor": 4.0, "original_max_position_embeddings": 8192})
    cache = rope.cos_sin_cache.numpy()
    pos = rng.integers(0, 8192, t)
    q = numerics.cast(rng.standard_normal((t, hq, d)).astype(np.float32), numerics.DT_BF16)
    k = numerics.cast(rng.standard_normal((t, hkv, d)).astype(np.float32), numerics.DT_BF16)
    cs = cache[pos]
    cos, sin = cs[..., :d // 2], cs[..., d // 2:]
    qe = oatt.apply_rotary_emb(q, cos, sin, numerics.DT_BF16)
    ke = oatt.apply_rotary_emb(k, cos, sin, numerics.DT_BF16)
    qd, kd = from_values(q, numerics.DT_BF16), from_values(k, numerics.DT_BF16)
    dev_cache = rope.cos_sin_cache.cuda()
    from fastdms_amd.layers.rotary_embedding import rope_inplace
    rope_inplace(qd, torch.from_numpy(pos).cuda(), dev_cache)
    rope_inplace(kd, torch.from_numpy(pos).cuda(), dev_cache)
    torch.cuda.synchronize()
    assert np.array_equal(values_of(qd), qe) and np.array_equal(values_of(kd), ke)


@pytest.mark.parametrize("d,split_rows,qk_norm", [(64, None, False), (128, None, False), (64, 256, False),
                                                  (64, None, True), (128, None, True)])
def test_fused_decode_attention_matches_oracle(monkeypatch, d, split_rows, qk_norm):
    """One-launch decode preprocess + attention (fdms_fused_decode_attention) on
    Llama / Qwen3 head shapes with q/k/v as views of one qkv row: the decision
    and the appended FP8 rows bit-exact vs the oracle's preprocess (store_q off),
    q / k untouched, the output within 2e-2 of the oracle's attention over the
    span incl. the appended token; split_rows=256 splits long spans so the
    appended token lands in the last split.  qk_norm: Qwen3's per-head
    RMSNorm of q and k done in the kernel from the raw rows, vs the oracle
    fed the normalised rows (the per-head sums of squares add up in another
    order, so at most two appended FP8 bytes may differ)."""
    require_gpu()
    import fastdms_amd.layers.compact_attention as ca
    if split_rows is not None:
        monkeypatch.setattr(ca, "attention_split_plan", lambda device, pairs, max_live, mfma, **kw: (8, split_rows))
    rng = np.random.default_rng(d + (split_rows or 0))
    b, hq, hkv = 8, 32, 8
    g = hq // hkv
    cap = 1600
    live_prev = rng.integers(0, 1500, (b, hkv)).astype(np.int32)
    live_prev[0, 0] = 0
    live_prev[1, 2] = 63
    live_prev[2, 5] = 255
    base = (np.arange(b * hkv).reshape(b, hkv) * cap).astype(np.int32)
    slot = base + live_prev
    live_prev[3, 1] = 700
    slot[3, 1] = -1  # no append for this pair: its span is read as is
    live = live_prev + (slot >= 0)
    qkv = numerics.cast(rng.standard_normal((b, (hq + 2 * hkv) * d)).astype(np.float32), numerics.DT_BF16)
    q = qkv[:, :hq * d].reshape(b, hq, d).copy()
    k = qkv[:, hq * d:(hq + hkv) * d].reshape(b, hkv, d).copy()
    v = qkv[:, (hq + hkv) * d:].reshape(b, hkv, d).copy()
    positions = rng.integers(2000, 8192, b)
    cache = oatt.rope_cos_sin_cache(d, 8192, 500000.0)
    ck = numerics.to_storage(rng.standard_normal((b * hkv * cap, d)).astype(np.float32), numerics.DT_FP8)
    cv = numerics.to_storage(rng.standard_normal((b * hkv * cap, d)).astype(np.float32), numerics.DT_FP8)
    qn_w = kn_w = None
    qo, ko, cko, cvo = q.copy(), k.copy(), ck.copy(), cv.copy()
    if qk_norm:
        qn_w = numerics.cast((1.0 + 0.25 * rng.standard_normal(d)).astype(np.float32), numerics.DT_BF16)
        kn_w = numerics.cast((1.0 + 0.25 * rng.standard_normal(d)).astype(np.float32), numerics.DT_BF16)
        eps = 1e-6

        def head_norm(x, w):  # layernorm.py:19-40 on each head
            xt = torch.from_numpy(x.astype(np.float32))
            inv = torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + eps)
            xn = (xt * inv).to(torch.bfloat16).float()
            return (xn * torch.from_numpy(w.astype(np.float32))).to(torch.bfloat16).float().numpy()
        qo, ko = head_norm(q, qn_w), head_norm(k, kn_w)
    ev = oatt.fused_dms_rope_store_compact_decode(q=qo, k=ko, v=v, cos_sin_cache=cache, compact_k=cko, compact_v=cvo,
                                                  slot_mapping=slot, positions=positions, num_kv_heads=hkv,
                                                  alpha_scale=10.0, alpha_offset=5.0, q_dtype_code=numerics.DT_BF16,
                                                  k_dtype_code=numerics.DT_BF16, compact_dtype_code=numerics.DT_FP8,
                                                  store_q=True, store_transient_k=False)
    ref = oatt.compact_decode_attention(qo, numerics.from_storage(cko, numerics.DT_FP8),
                                        numerics.from_storage(cvo, numerics.DT_FP8), base, live)
    qkv_d = from_values(qkv, numerics.DT_BF16)
    qd = qkv_d[:, :hq * d].view(b, hq, d)
    kd = qkv_d[:, hq * d:(hq + hkv) * d].view(b, hkv, d)
    vd = qkv_d[:, (hq + hkv) * d:].view(b, hkv, d)
    ckd = torch.from_numpy(ck).cuda().view(torch.float8_e4m3fn)
    cvd = torch.from_numpy(cv).cuda().view(torch.float8_e4m3fn)
    evd = torch.empty((b, hkv), device="cuda", dtype=torch.bool)
    assert ca.fused_decode_attention_supported(qd, kd, vd, ckd)
    out = ca.fused_dms_rope_store_compact_decode_attention(
        qd, kd, vd, torch.from_numpy(cache).cuda(), ckd, cvd, torch.from_numpy(slot).cuda(), evd,
        torch.from_numpy(positions).cuda(), torch.from_numpy(base).cuda(), torch.from_numpy(live).cuda(),
        num_kv_heads=hkv, alpha_scale=10.0, alpha_offset=5.0, max_live_count=cap,
        q_norm_weight=None if qn_w is None else from_values(qn_w, numerics.DT_BF16),
        k_norm_weight=None if kn_w is None else from_values(kn_w, numerics.DT_BF16), norm_eps=1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(evd.cpu().numpy(), ev)
    if qk_norm:
        assert int((storage_of(ckd) != cko).sum()) <= 2 and np.array_equal(storage_of(cvd), cvo)
    else:
        assert np.array_equal(storage_of(ckd), cko) and np.array_equal(storage_of(cvd), cvo)
    assert np.array_equal(values_of(qd), q) and np.array_equal(values_of(kd), k)
    got = values_of(out)
    assert float(np.abs(got - ref).max() / np.abs(ref).max()) <= 2e-2
    assert g == 4

    # The same step on 16-row pages in a shuffled pool (the paged entry point,
    # whose page ids of each split's first rows are read with the live
    # count): the decisions, the appended rows (at their page) and the output
    # equal the span launch's bit for bit.
    npg = b * hkv * cap // 16
    perm = rng.permutation(npg)
    ckp, cvp = np.empty_like(ck), np.empty_like(cv)
    ckp.reshape(npg, 16, d)[perm] = ck.reshape(npg, 16, d)
    cvp.reshape(npg, 16, d)[perm] = cv.reshape(npg, 16, d)
    table = perm[(base // 16)[..., None] + np.arange(cap // 16)].astype(np.int32)
    lp = np.minimum(live_prev, cap - 1)
    pslot = np.where(slot >= 0, np.take_along_axis(table, (lp // 16)[..., None], 2)[..., 0] * 16 + lp % 16,
                     -1).astype(np.int32)
    ckpd = torch.from_numpy(ckp).cuda().view(torch.float8_e4m3fn)
    cvpd = torch.from_numpy(cvp).cuda().view(torch.float8_e4m3fn)
    evpd = torch.empty((b, hkv), device="cuda", dtype=torch.bool)
    outp = ca.fused_dms_rope_store_compact_decode_attention(
        qd, kd, vd, torch.from_numpy(cache).cuda(), ckpd, cvpd, torch.from_numpy(pslot).cuda(), evpd,
        torch.from_numpy(positions).cuda(), torch.from_numpy(base).cuda(), torch.from_numpy(live).cuda(),
        num_kv_heads=hkv, alpha_scale=10.0, alpha_offset=5.0, max_live_count=cap,
        block_tables=torch.from_numpy(table).cuda(), page_size=16,
        q_norm_weight=None if qn_w is None else from_values(qn_w, numerics.DT_BF16),
        k_norm_weight=None if kn_w is None else from_values(kn_w, numerics.DT_BF16), norm_eps=1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(evpd.cpu().numpy(), evd.cpu().numpy())
    assert np.array_equal(storage_of(ckpd).reshape(npg, 16, d)[perm], storage_of(ckd).reshape(npg, 16, d))
    assert np.array_equal(storage_of(cvpd).reshape(npg, 16, d)[perm], storage_of(cvd).reshape(npg, 16, d))
    assert np.array_equal(values_of(outp), got)
