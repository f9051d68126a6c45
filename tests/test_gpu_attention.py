"""B2-B7: compact decode attention on the GPU vs the float64 oracle.

Tolerance: max|out - ref| / max|ref| <= 2e-2 for bf16 q with FP8/bf16 K/V
(the north-star bound); <= 1e-5 when q and K/V are fp32.
"""
import numpy as np
import pytest
import torch

from helpers import TORCH_DTYPE, from_values, require_gpu, values_of
from oracle import attention as oatt
from oracle import numerics

pytestmark = pytest.mark.gpu
TOL_LOWP = 2e-2
TOL_F32 = 1e-5


def _rel_err(got, ref):
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def _force_splits(monkeypatch, n):
    import fastdms_amd.layers.compact_attention as ca
    monkeypatch.setattr(ca, "attention_split_plan", lambda device, pairs, max_live, mfma, **kw: (n, 0))


@pytest.mark.parametrize("splits", [None, 1, 2, 3, 20])
def test_reference_splitk_case(monkeypatch, splits):
    """q [2,8,16], spans at [[0,24],[48,72]] with live [[17,13],[19,11]] (test_compact_kv.py:1244-1280)."""
    require_gpu()
    from fastdms_amd.layers.compact_attention import compact_decode_attention
    if splits is not None:
        _force_splits(monkeypatch, splits)
    rng = np.random.default_rng(17)
    q = rng.standard_normal((2, 8, 16)).astype(np.float32)
    ck = rng.standard_normal((96, 16)).astype(np.float32)
    cv = rng.standard_normal((96, 16)).astype(np.float32)
    base = np.array([[0, 24], [48, 72]], np.int32)
    live = np.array([[17, 13], [19, 11]], np.int32)
    ref = oatt.compact_decode_attention(q, ck, cv, base, live)
    out = compact_decode_attention(torch.from_numpy(q).cuda(), torch.from_numpy(ck).cuda(),
                                   torch.from_numpy(cv).cuda(), torch.from_numpy(base).cuda(),
                                   torch.from_numpy(live).cuda(), max_live_count=20, block_n=16)
    torch.cuda.synchronize()
    assert _rel_err(values_of(out), ref) <= TOL_F32


def _config1_case(rng, b=1, hkv=8, g=4, d=64, ctx=2048, window=256, page=16):
    """keep = last 256 tokens | Bernoulli(1/8); pages of 16 with a random permutation."""
    keep = rng.random((b, hkv, ctx)) < 1.0 / 8
    keep[..., ctx - window:] = True
    live = keep.sum(-1).astype(np.int32)
    max_pages = int(-(-live.max() // page))
    total_pages = b * hkv * max_pages
    bt = rng.permutation(total_pages).reshape(b, hkv, max_pages).astype(np.int32)
    kd = numerics.cast(rng.standard_normal((total_pages * page, d)).astype(np.float32), numerics.DT_FP8)
    vd = numerics.cast(rng.standard_normal((total_pages * page, d)).astype(np.float32), numerics.DT_FP8)
    q = numerics.cast(rng.standard_normal((b, hkv * g, d)).astype(np.float32), numerics.DT_BF16)
    return q, kd, vd, bt, live, page


@pytest.mark.parametrize("seed", [0, 1])
def test_config1_paged_fp8_matches_oracle(seed):
    require_gpu()
    from fastdms_amd.layers.compact_attention import compact_decode_attention_paged
    rng = np.random.default_rng(seed)
    q, kd, vd, bt, live, page = _config1_case(rng)
    ref = oatt.compact_decode_attention_paged(q, kd, vd, bt, live, page)
    out = compact_decode_attention_paged(from_values(q, numerics.DT_BF16), from_values(kd, numerics.DT_FP8),
                                         from_values(vd, numerics.DT_FP8), torch.from_numpy(bt).cuda(),
                                         torch.from_numpy(live).cuda(), page, max_live_count=int(live.max()))
    torch.cuda.synchronize()
    assert _rel_err(values_of(out), ref) <= TOL_LOWP


def test_paged_is_invariant_to_page_permutation():
    require_gpu()
    from fastdms_amd.layers.compact_attention import compact_decode_attention_paged
    rng = np.random.default_rng(3)
    q, kd, vd, bt, live, page = _config1_case(rng)
    # move every page to a new physical location, keeping contents
    total = bt.size
    perm = rng.permutation(total)
    kd2 = np.zeros_like(kd)
    vd2 = np.zeros_like(vd)
    for old in range(total):
        kd2[perm[old] * page:(perm[old] + 1) * page] = kd[old * page:(old + 1) * page]
        vd2[perm[old] * page:(perm[old] + 1) * page] = vd[old * page:(old + 1) * page]
    bt2 = perm[bt].astype(np.int32)
    args = dict(page_size=page, max_live_count=int(live.max()))
    o1 = compact_decode_attention_paged(from_values(q, numerics.DT_BF16), from_values(kd, numerics.DT_FP8),
                                        from_values(vd, numerics.DT_FP8), torch.from_numpy(bt).cuda(),
                                        torch.from_numpy(live).cuda(), **args)
    o2 = compact_decode_attention_paged(from_values(q, numerics.DT_BF16), from_values(kd2, numerics.DT_FP8),
                                        from_values(vd2, numerics.DT_FP8), torch.from_numpy(bt2).cuda(),
                                        torch.from_numpy(live).cuda(), **args)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


@pytest.mark.parametrize("d,kv_code", [(64, numerics.DT_FP8), (128, numerics.DT_FP8), (64, numerics.DT_BF16),
                                       (128, numerics.DT_F32)])
def test_ragged_batch_spans_match_oracle(d, kv_code):
    """c=8 ragged live counts in flat spans with gaps between them (reference layout)."""
    require_gpu()
    from fastdms_amd.layers.compact_attention import compact_decode_attention
    rng = np.random.default_rng(d + kv_code)
    b, hkv, g = 8, 8, 4
    live = rng.integers(1, 1400, (b, hkv)).astype(np.int32)
    live[0, 0] = 1
    base = np.zeros((b, hkv), np.int32)
    cur = 0
    for bi in range(b):
        for h in range(hkv):
            base[bi, h] = cur
            cur += int(live[bi, h]) + int(rng.integers(0, 40))
    ck = numerics.cast(rng.standard_normal((cur, d)).astype(np.float32), kv_code)
    cv = numerics.cast(rng.standard_normal((cur, d)).astype(np.float32), kv_code)
    q = numerics.cast(rng.standard_normal((b, hkv * g, d)).astype(np.float32), numerics.DT_BF16)
    ref = oatt.compact_decode_attention(q, ck, cv, base, live)
    out = compact_decode_attention(from_values(q, numerics.DT_BF16), from_values(ck, kv_code),
                                   from_values(cv, kv_code), torch.from_numpy(base).cuda(),
                                   torch.from_numpy(live).cuda(), max_live_count=8320)
    torch.cuda.synchronize()
    assert _rel_err(values_of(out), ref) <= TOL_LOWP


@pytest.mark.parametrize("d,paged", [(64, False), (128, False), (64, True)])
def test_matrix_core_per_pair_splits(monkeypatch, d, paged):
    """Matrix-core kernel with split_rows > 0: pairs of one launch take 1, 2 or
    3 splits from their own live counts (workgroups past a pair's count exit,
    one-split pairs skip the merge), twice in a row so the counters are reused."""
    require_gpu()
    import fastdms_amd.layers.compact_attention as ca
    rng = np.random.default_rng(d + paged)
    b, hkv, g, page = 4, 4, 4, 16
    live = np.array([[1, 64, 65, 511], [512, 513, 1024, 1025], [1535, 1536, 7, 900], [130, 1200, 2, 333]], np.int32)
    span = 1600
    base = (np.arange(b * hkv).reshape(b, hkv) * span).astype(np.int32)
    ck = numerics.cast(rng.standard_normal((b * hkv * span, d)).astype(np.float32), numerics.DT_FP8)
    cv = numerics.cast(rng.standard_normal((b * hkv * span, d)).astype(np.float32), numerics.DT_FP8)
    q = numerics.cast(rng.standard_normal((b, hkv * g, d)).astype(np.float32), numerics.DT_BF16)
    ref = oatt.compact_decode_attention(q, ck, cv, base, live)
    monkeypatch.setattr(ca, "attention_split_plan", lambda device, pairs, max_live, mfma, **kw: (4, 512))
    qd, ckd, cvd = from_values(q, numerics.DT_BF16), from_values(ck, numerics.DT_FP8), from_values(cv, numerics.DT_FP8)
    assert ca.mfma_attention_path(qd, ckd, g)
    if paged:
        # page p of span (b, h) is physical page perm[...]: same rows, permuted pages
        npg = span // page
        perm = rng.permutation(b * hkv * npg).astype(np.int32)
        table = perm.reshape(b, hkv, npg)
        ckp, cvp = np.empty_like(ck), np.empty_like(cv)
        for bi in range(b):
            for h in range(hkv):
                for pg in range(npg):
                    src = slice(int(base[bi, h]) + pg * page, int(base[bi, h]) + (pg + 1) * page)
                    dst = slice(int(table[bi, h, pg]) * page, (int(table[bi, h, pg]) + 1) * page)
                    ckp[dst], cvp[dst] = ck[src], cv[src]
        outs = [ca.compact_decode_attention_paged(qd, from_values(ckp, numerics.DT_FP8),
                                                  from_values(cvp, numerics.DT_FP8), torch.from_numpy(table).cuda(),
                                                  torch.from_numpy(live).cuda(), page_size=page, max_live_count=1600)
                for _ in range(2)]
    else:
        outs = [ca.compact_decode_attention(qd, ckd, cvd, torch.from_numpy(base).cuda(), torch.from_numpy(live).cuda(),
                                            max_live_count=1600) for _ in range(2)]
    torch.cuda.synchronize()
    for out in outs:
        assert _rel_err(values_of(out), ref) <= TOL_LOWP


def test_split_count_does_not_change_fp32_result(monkeypatch):
    require_gpu()
    from fastdms_amd.layers.compact_attention import compact_decode_attention
    rng = np.random.default_rng(11)
    b, hkv, g, d = 2, 4, 2, 32
    live = np.array([[700, 1, 33, 256], [5, 999, 1000, 64]], np.int32)
    base = (np.arange(b * hkv).reshape(b, hkv) * 1024).astype(np.int32)
    ck = rng.standard_normal((b * hkv * 1024, d)).astype(np.float32)
    cv = rng.standard_normal((b * hkv * 1024, d)).astype(np.float32)
    q = rng.standard_normal((b, hkv * g, d)).astype(np.float32)
    ref = oatt.compact_decode_attention(q, ck, cv, base, live)
    args = [torch.from_numpy(x).cuda() for x in (q, ck, cv, base, live)]
    for s in (1, 2, 7, 64, 300):
        _force_splits(monkeypatch, s)
        out = compact_decode_attention(*args, max_live_count=1000)
        torch.cuda.synchronize()
        assert _rel_err(values_of(out), ref) <= TOL_F32, s


def test_inline_q_rope_equals_prerotated_q():
    """B4: rotate q inside attention (decision lane zeroed) == fused preprocess with store_q."""
    require_gpu()
    from fastdms_amd.layers.compact_attention import compact_decode_attention
    rng = np.random.default_rng(12)
    b, hkv, g, d = 1, 8, 4, 64
    q = numerics.cast(rng.standard_normal((b, hkv * g, d)).astype(np.float32), numerics.DT_BF16)
    live = rng.integers(10, 500, (b, hkv)).astype(np.int32)
    base = (np.arange(hkv) * 512).reshape(1, hkv).astype(np.int32)
    ck = numerics.cast(rng.standard_normal((hkv * 512, d)).astype(np.float32), numerics.DT_FP8)
    cv = numerics.cast(rng.standard_normal((hkv * 512, d)).astype(np.float32), numerics.DT_FP8)
    cache = oatt.rope_cos_sin_cache(d, 4096, 500000.0)
    pos = np.array([3000])
    # oracle: zero the decision lane, rotate in fp32 (not rounded to bf16), attend
    qr = q.astype(np.float32).copy()
    half = d // 2
    cs = cache[pos[0], 0]
    for hh in range(hkv * g):
        x2 = qr[0, hh, half:].copy()
        if hh % g == 0:
            x2[half - 1] = 0.0
        y1, y2 = oatt.rotate(qr[0, hh, :half], x2, cs[:half], cs[half:])
        qr[0, hh] = np.concatenate([y1, y2])
    ref = oatt.compact_decode_attention(qr, ck, cv, base, live)
    out = compact_decode_attention(from_values(q, numerics.DT_BF16), from_values(ck, numerics.DT_FP8),
                                   from_values(cv, numerics.DT_FP8), torch.from_numpy(base).cuda(),
                                   torch.from_numpy(live).cuda(), max_live_count=512,
                                   q_rope_positions=torch.from_numpy(pos).cuda(),
                                   q_rope_cos_sin_cache=torch.from_numpy(cache).cuda())
    torch.cuda.synchronize()
    assert _rel_err(values_of(out), ref) <= TOL_LOWP


def test_argument_errors():
    require_gpu()
    from fastdms_amd.layers.compact_attention import compact_decode_attention
    q = torch.zeros((1, 8, 16), device="cuda")
    kv = torch.zeros((4, 16), device="cuda")
    meta = torch.zeros((1, 2), device="cuda", dtype=torch.int32)
    with pytest.raises(ValueError):
        compact_decode_attention(q, kv, kv, meta, meta, max_live_count=0)
    with pytest.raises(ValueError):
        compact_decode_attention(q, kv, torch.zeros((4, 8), device="cuda"), meta, meta, max_live_count=1)
    with pytest.raises(ValueError):
        compact_decode_attention(q, kv, kv, meta, meta[:, :1].expand(1, 3), max_live_count=1)


def test_fp8_hardware_decode_is_e4m3fn():
    """v_cvt_pk_f32_fp8 (used by the tiled kernel) decodes OCP e4m3fn: all 256
    codes in each byte position of a dword, NaN codes included."""
    require_gpu()
    from fastdms_amd import _native as nat
    codes = np.arange(256, dtype=np.uint8)
    data = np.stack([np.roll(codes, s) for s in range(4)], axis=1).reshape(-1)  # every code at every byte lane
    src = torch.from_numpy(data).cuda()
    out = torch.empty(data.size, device="cuda", dtype=torch.float32)
    nat.call("fdms_fp8_decode_hw", src.data_ptr(), out.data_ptr(), data.size, nat.stream())
    torch.cuda.synchronize()
    want = numerics.e4m3fn_decode(data)
    got = out.cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))  # bit-exact, signed zeros too


def _span_case(rng, lives, hkv, g, d, kv_code, gap=5):
    """Ragged spans laid out back to back with gaps in one arena."""
    b = len(lives) // hkv
    live = np.asarray(lives, np.int32).reshape(b, hkv)
    base = np.zeros((b, hkv), np.int32)
    cur = 3
    for i in range(b):
        for h in range(hkv):
            base[i, h] = cur
            cur += int(live[i, h]) + gap
    ck = numerics.cast(rng.standard_normal((cur + 2, d)).astype(np.float32) * 2, kv_code)
    cv = numerics.cast(rng.standard_normal((cur + 2, d)).astype(np.float32), kv_code)
    q = numerics.cast(rng.standard_normal((b, hkv * g, d)).astype(np.float32), numerics.DT_BF16)
    return q, ck, cv, base, live


@pytest.mark.parametrize("d,g,kv_code", [(64, 4, numerics.DT_FP8), (128, 4, numerics.DT_FP8),
                                         (64, 1, numerics.DT_FP8), (64, 2, numerics.DT_FP8),
                                         (64, 8, numerics.DT_FP8), (128, 8, numerics.DT_FP8),
                                         (128, 1, numerics.DT_FP8), (64, 4, numerics.DT_BF16),
                                         (128, 4, numerics.DT_BF16), (128, 8, numerics.DT_BF16)])
@pytest.mark.parametrize("splits", [None, 1, 7])
def test_tiled_kernel_spans(monkeypatch, d, g, kv_code, splits):
    """The tiled fast path (bf16 q, D 64/128, G 1-8) against the float64 oracle:
    live counts from 1 to several tiles, ragged over (b, h)."""
    require_gpu()
    from fastdms_amd.layers.compact_attention import compact_decode_attention
    if splits is not None:
        _force_splits(monkeypatch, splits)
    rng = np.random.default_rng(d * 100 + g + kv_code)
    hkv = 2
    lives = [1, 2, 63, 64, 65, 255, 256, 257, 1000, 1300]
    q, ck, cv, base, live = _span_case(rng, lives, hkv, g, d, kv_code)
    ref = oatt.compact_decode_attention(q, ck, cv, base, live)
    out = compact_decode_attention(from_values(q, numerics.DT_BF16), from_values(ck, kv_code),
                                   from_values(cv, kv_code), torch.from_numpy(base).cuda(),
                                   torch.from_numpy(live).cuda(), max_live_count=int(live.max()))
    torch.cuda.synchronize()
    assert _rel_err(values_of(out), ref) <= TOL_LOWP
    # per (b, head) too: a short span must not hide behind a long one's scale
    got = values_of(out)
    for i in range(got.shape[0]):
        for hh in range(got.shape[1]):
            e = np.abs(got[i, hh] - ref[i, hh]).max() / max(np.abs(ref[i, hh]).max(), 1e-30)
            assert e <= TOL_LOWP, (i, hh, e)


def test_tiled_and_generic_kernels_agree(monkeypatch):
    """Same inputs through both kernels (FASTDMS_AMD_ATTN_GENERIC=1 selects the
    generic one): both within bf16 rounding of each other."""
    require_gpu()
    from fastdms_amd.layers.compact_attention import compact_decode_attention
    rng = np.random.default_rng(5)
    q, ck, cv, base, live = _span_case(rng, [700, 33, 1, 1200, 400, 90, 256, 512], 8, 4, 64, numerics.DT_FP8)
    args = (from_values(q, numerics.DT_BF16), from_values(ck, numerics.DT_FP8), from_values(cv, numerics.DT_FP8),
            torch.from_numpy(base).cuda(), torch.from_numpy(live).cuda())
    tiled = values_of(compact_decode_attention(*args, max_live_count=1200))
    monkeypatch.setenv("FASTDMS_AMD_ATTN_GENERIC", "1")
    generic = values_of(compact_decode_attention(*args, max_live_count=1200))
    torch.cuda.synchronize()
    assert _rel_err(tiled, generic) <= 1e-2


@pytest.mark.parametrize("d", [64, 128])
def test_tiled_paged_and_inline_rope(d):
    """Paged addressing and inline q RoPE through the tiled kernel."""
    require_gpu()
    from fastdms_amd.layers.compact_attention import compact_decode_attention, compact_decode_attention_paged
    rng = np.random.default_rng(d)
    q, kd, vd, bt, live, page = _config1_case(rng, b=2, hkv=4, g=4, d=d, ctx=1500)
    ref = oatt.compact_decode_attention_paged(q, kd, vd, bt, live, page)
    out = compact_decode_attention_paged(from_values(q, numerics.DT_BF16), from_values(kd, numerics.DT_FP8),
                                         from_values(vd, numerics.DT_FP8), torch.from_numpy(bt).cuda(),
                                         torch.from_numpy(live).cuda(), page)
    torch.cuda.synchronize()
    assert _rel_err(values_of(out), ref) <= TOL_LOWP
    # inline RoPE (B = 1)
    q1 = q[:1]
    cache = oatt.rope_cos_sin_cache(d, 4096, 500000.0)
    pos = np.array([2999])
    qr = q1.astype(np.float32).copy()
    half = d // 2
    cs = cache[pos[0], 0]
    for hh in range(q1.shape[1]):
        x2 = qr[0, hh, half:].copy()
        if hh % 4 == 0:
            x2[half - 1] = 0.0
        y1, y2 = oatt.rotate(qr[0, hh, :half], x2, cs[:half], cs[half:])
        qr[0, hh] = np.concatenate([y1, y2])
    base = np.arange(4, dtype=np.int32).reshape(1, 4) * 2000
    live1 = np.array([[700, 1, 1999, 300]], np.int32)
    ck = numerics.cast(rng.standard_normal((8000, d)).astype(np.float32), numerics.DT_FP8)
    cv = numerics.cast(rng.standard_normal((8000, d)).astype(np.float32), numerics.DT_FP8)
    ref = oatt.compact_decode_attention(qr, ck, cv, base, live1)
    out = compact_decode_attention(from_values(q1, numerics.DT_BF16), from_values(ck, numerics.DT_FP8),
                                   from_values(cv, numerics.DT_FP8), torch.from_numpy(base).cuda(),
                                   torch.from_numpy(live1).cuda(), max_live_count=2000,
                                   q_rope_positions=torch.from_numpy(pos).cuda(),
                                   q_rope_cos_sin_cache=torch.from_numpy(cache).cuda())
    torch.cuda.synchronize()
    assert _rel_err(values_of(out), ref) <= TOL_LOWP


@pytest.mark.parametrize("b,fused", [(80, False), (80, True), (3, False)])
def test_matrix_core_heavy_tail_splits(monkeypatch, b, fused):
    """The matrix-core kernel's per-pair splits over a heavy-tailed batch
    (live counts from 1 to 6000, a few pairs holding most rows) at several
    split bounds with the default rows per split: 640 pairs at b = 80, a tiny
    batch at b = 3, twice in a row (the tickets are reused), vs the float64
    oracle."""
    require_gpu()
    import fastdms_amd.layers.compact_attention as ca
    rng = np.random.default_rng(b * 7 + fused)
    hkv, g, d = 8, 4, 64
    live = np.minimum(rng.pareto(1.2, (b, hkv)) * 120 + 1, 6000).astype(np.int32)
    live[0, 0] = 6000
    live[-1, -1] = 1
    cap = int(live.max()) + 1
    base = (np.arange(b * hkv).reshape(b, hkv) * cap).astype(np.int32)
    rows = b * hkv * cap
    ck = numerics.to_storage(rng.standard_normal((rows, d)).astype(np.float32), numerics.DT_FP8)
    cv = numerics.to_storage(rng.standard_normal((rows, d)).astype(np.float32), numerics.DT_FP8)
    q = numerics.cast(rng.standard_normal((b, hkv * g, d)).astype(np.float32), numerics.DT_BF16)
    qd = from_values(q, numerics.DT_BF16)
    ckd = torch.from_numpy(ck).cuda().view(torch.float8_e4m3fn)
    cvd = torch.from_numpy(cv).cuda().view(torch.float8_e4m3fn)
    base_d, live_d = torch.from_numpy(base).cuda(), torch.from_numpy(live).cuda()
    qr = q.copy()
    if fused:  # position 0: RoPE is the identity, only the decision lane is zeroed
        qr.reshape(b, hkv, g, d)[:, :, 0, d - 1] = 0.0
    ref = oatt.compact_decode_attention(qr, numerics.from_storage(ck, numerics.DT_FP8),
                                        numerics.from_storage(cv, numerics.DT_FP8), base, live)
    for target in (1, 8, 24):
        monkeypatch.setattr(ca, "attention_split_plan", lambda device, pairs, max_live, mfma, t=target, **kw: (t, 0))
        if fused:
            # no append (slot -1): the fused kernel attends over the stored span
            kq = qd[:, :hkv].contiguous()
            pos = torch.zeros(b, dtype=torch.int64, device="cuda")
            cache = torch.from_numpy(oatt.rope_cos_sin_cache(d, 16, 500000.0)).cuda()
            slot = torch.full((b, hkv), -1, dtype=torch.int32, device="cuda")
            ev = torch.empty((b, hkv), dtype=torch.bool, device="cuda")
            outs = [ca.fused_dms_rope_store_compact_decode_attention(
                qd, kq, kq, cache, ckd, cvd, slot, ev, pos, base_d, live_d, num_kv_heads=hkv, alpha_scale=10.0,
                alpha_offset=5.0, max_live_count=cap) for _ in range(2)]
        else:
            outs = [ca.compact_decode_attention(qd, ckd, cvd, base_d, live_d, max_live_count=cap) for _ in range(2)]
        torch.cuda.synchronize()
        for out in outs:
            assert _rel_err(values_of(out), ref) <= TOL_LOWP, target
