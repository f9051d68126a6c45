"""Pin the attention-side oracle: softmax attention against torch's library
routines, paged addressing against flat spans, RoPE against the reference
formula, and the fused decode preprocess against its unfused composition."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import numerics
from oracle.dms import extract_dms_eviction_decisions


def test_compact_decode_attention_matches_torch_sdpa():
    rng = np.random.default_rng(0)
    b, hkv, g, d = 2, 3, 4, 16
    live = rng.integers(1, 30, (b, hkv))
    base = np.zeros((b, hkv), np.int32)
    cur = 0
    for bi in range(b):
        for h in range(hkv):
            base[bi, h] = cur
            cur += live[bi, h] + 3
    ck = rng.standard_normal((cur, d)).astype(np.float32)
    cv = rng.standard_normal((cur, d)).astype(np.float32)
    q = rng.standard_normal((b, hkv * g, d)).astype(np.float32)
    out = oatt.compact_decode_attention(q, ck, cv, base, live)
    for bi in range(b):
        for qh in range(hkv * g):
            h = qh // g
            kk = torch.from_numpy(ck[base[bi, h]:base[bi, h] + live[bi, h]]).double()
            vv = torch.from_numpy(cv[base[bi, h]:base[bi, h] + live[bi, h]]).double()
            ref = torch.nn.functional.scaled_dot_product_attention(
                torch.from_numpy(q[bi, qh]).double()[None, None, None], kk[None, None], vv[None, None])
            np.testing.assert_allclose(out[bi, qh], ref[0, 0, 0].numpy(), rtol=1e-10, atol=1e-12)


def test_paged_attention_equals_span_attention_under_page_permutation():
    rng = np.random.default_rng(1)
    b, hkv, g, d, page = 1, 8, 4, 64, 16
    live = rng.integers(100, 500, (b, hkv))
    max_pages = int(-(-live.max() // page))
    total_pages = b * hkv * max_pages
    perm = rng.permutation(total_pages)
    bt = perm.reshape(b, hkv, max_pages).astype(np.int32)
    kv_k = rng.standard_normal((total_pages * page, d)).astype(np.float32)
    kv_v = rng.standard_normal((total_pages * page, d)).astype(np.float32)
    q = rng.standard_normal((b, hkv * g, d)).astype(np.float32)
    out_p = oatt.compact_decode_attention_paged(q, kv_k, kv_v, bt, live, page)
    # gather to a flat span layout and compare
    spans_k, spans_v, base = [], [], np.zeros((b, hkv), np.int32)
    cur = 0
    for bi in range(b):
        for h in range(hkv):
            rows = oatt.paged_rows(bt[bi, h], live[bi, h], page)
            base[bi, h] = cur
            spans_k.append(kv_k[rows])
            spans_v.append(kv_v[rows])
            cur += live[bi, h]
    out_s = oatt.compact_decode_attention(q, np.concatenate(spans_k), np.concatenate(spans_v), base, live)
    np.testing.assert_allclose(out_p, out_s, rtol=0, atol=0)


def test_causal_prefill_matches_torch_sdpa():
    rng = np.random.default_rng(2)
    cu = [0, 5, 17, 40]
    hq, hkv, d = 8, 2, 16
    q = rng.standard_normal((40, hq, d)).astype(np.float32)
    k = rng.standard_normal((40, hkv, d)).astype(np.float32)
    v = rng.standard_normal((40, hkv, d)).astype(np.float32)
    out = oatt.causal_prefill_attention(q, k, v, cu)
    for i in range(3):
        s0, s1 = cu[i], cu[i + 1]
        qq = torch.from_numpy(q[s0:s1]).double().transpose(0, 1)
        kk = torch.from_numpy(k[s0:s1]).double().transpose(0, 1).repeat_interleave(hq // hkv, 0)
        vv = torch.from_numpy(v[s0:s1]).double().transpose(0, 1).repeat_interleave(hq // hkv, 0)
        ref = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, is_causal=True).transpose(0, 1)
        np.testing.assert_allclose(out[s0:s1], ref.numpy(), rtol=1e-10, atol=1e-12)


def test_chunked_prefill_rows_equal_the_full_prompt_rows():
    """A chunk's queries aligned to the end of their keys (the retained
    earlier chunks + the chunk) give the same rows as the unchunked causal
    attention over the whole prompt; a wrong alignment offset fails."""
    rng = np.random.default_rng(3)
    lens = [23, 40, 9]
    hq, hkv, d = 4, 2, 16
    cu = np.concatenate([[0], np.cumsum(lens)])
    q = rng.standard_normal((cu[-1], hq, d))
    k = rng.standard_normal((cu[-1], hkv, d))
    v = rng.standard_normal((cu[-1], hkv, d))
    full = oatt.causal_prefill_attention(q, k, v, cu)
    for cut in ([10, 17, 0], [22, 1, 8], [0, 39, 3]):
        rows = [np.arange(cu[i] + cut[i], cu[i + 1]) for i in range(3)]
        cq = np.concatenate([[0], np.cumsum([len(r) for r in rows])])
        out = oatt.causal_prefill_attention(q[np.concatenate(rows)], k, v, cq, cu_seqlens_k=cu)
        np.testing.assert_allclose(out, full[np.concatenate(rows)], rtol=1e-12, atol=1e-12)
        # queries aligned to the start of the keys instead see too few keys
        assert not np.allclose(out[:3], oatt.causal_prefill_attention(q[np.concatenate(rows)][:3], k[:3], v[:3],
                                                                       [0, 3])) or cut[0] == 0


def test_rope_table_and_rotation_match_reference_formula():
    cache = oatt.rope_cos_sin_cache(64, 32, 500000.0)
    inv = 1.0 / (500000.0 ** (torch.arange(0, 64, 2, dtype=torch.float) / 64))
    t = torch.arange(32, dtype=torch.float)
    freqs = torch.outer(t, inv)
    assert np.array_equal(cache[:, 0, :32], freqs.cos().numpy())
    assert np.array_equal(cache[:, 0, 32:], freqs.sin().numpy())
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 3, 64)).astype(np.float32)
    pos = np.array([0, 1, 7, 19, 31])
    cs = cache[pos]
    cos, sin = cs[..., :32], cs[..., 32:]
    y = oatt.apply_rotary_emb(x, cos, sin, numerics.DT_F32)
    xt = torch.from_numpy(x)
    x1, x2 = xt[..., :32], xt[..., 32:]
    ct, st = torch.from_numpy(cos), torch.from_numpy(sin)
    ref = torch.cat([x1 * ct - x2 * st, x2 * ct + x1 * st], dim=-1)
    assert np.array_equal(y, ref.numpy())
    # position 0 is the identity rotation
    assert np.array_equal(y[0], x[0])


def test_llama3_rope_scaling_leaves_high_freqs_and_scales_low_freqs():
    sc = {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}
    base = oatt.rope_inv_freq(64, 500000.0)
    scaled = oatt.rope_inv_freq(64, 500000.0, sc)
    wl = 2 * np.pi / base
    assert np.array_equal(scaled[wl < 8192 / 4], base[wl < 8192 / 4])
    np.testing.assert_allclose(scaled[wl > 8192], base[wl > 8192] / 32.0, rtol=1e-6)


@pytest.mark.parametrize("q_code,cc", [(numerics.DT_F32, numerics.DT_F32), (numerics.DT_BF16, numerics.DT_FP8)])
def test_fused_decode_preprocess_equals_unfused_composition(q_code, cc):
    """The reference checks fused == extract -> RoPE -> store (test_compact_kv.py:973-1040)."""
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
    ck = np.zeros((18, d), sd)
    cv = np.zeros((18, d), sd)
    qf, kf = q.copy(), k.copy()
    ev = oatt.fused_dms_rope_store_compact_decode(q=qf, k=kf, v=v, cos_sin_cache=cache, compact_k=ck, compact_v=cv,
                                                  slot_mapping=slot, positions=positions, num_kv_heads=hkv,
                                                  alpha_scale=100.0, alpha_offset=5.0, q_dtype_code=q_code,
                                                  k_dtype_code=q_code, compact_dtype_code=cc)
    q_ref, ev_ref = extract_dms_eviction_decisions(q, num_kv_heads=hkv, num_qo_heads=hkv * g, head_dim=d,
                                                   alpha_scale=100.0, alpha_offset=5.0)
    cs = cache[positions][:, None, 0]
    cos, sin = cs[..., :d // 2], cs[..., d // 2:]
    q_ref = oatt.apply_rotary_emb(q_ref, cos, sin, q_code)
    assert np.array_equal(ev, ev_ref)
    if q_code == numerics.DT_F32:  # the reference test's hand-set decision values
        assert ev.tolist() == [[False, True], [False, True], [True, False]]
    assert np.array_equal(qf, q_ref)
    # the arena receives RoPE(k) straight from fp32 (no rounding to k's dtype first)
    half = d // 2
    k1, k2 = k[..., :half], k[..., half:]
    y1, y2 = oatt.rotate(k1, k2, cos, sin)
    krot = np.concatenate([y1, y2], -1)
    for bi in range(b):
        for h in range(hkv):
            assert np.array_equal(ck[slot[bi, h]], numerics.to_storage(krot[bi, h], cc))
            assert np.array_equal(cv[slot[bi, h]], numerics.to_storage(v[bi, h], cc))
    assert np.array_equal(kf, numerics.cast(krot, q_code))


def test_storage_attention_equals_value_attention():
    rng = np.random.default_rng(9)
    b, hkv, g, d = 2, 2, 4, 16
    live = np.array([[5, 17], [1, 30]])
    base = np.array([[0, 40], [80, 120]])
    ck = numerics.e4m3fn_encode(rng.standard_normal((160, d)).astype(np.float32))
    cv = numerics.e4m3fn_encode(rng.standard_normal((160, d)).astype(np.float32))
    q = rng.standard_normal((b, hkv * g, d)).astype(np.float32)
    a = oatt.compact_decode_attention_storage(q, ck, cv, numerics.DT_FP8, base, live)
    ref = oatt.compact_decode_attention(q, numerics.e4m3fn_decode(ck), numerics.e4m3fn_decode(cv), base, live)
    np.testing.assert_allclose(a, ref, rtol=1e-12, atol=1e-12)
