"""The decode step's attention work plan on the GPU (no reference counterpart:
the reference partitions inside its split-K kernels, compact_attention.py:
334-603, 1116-1336).

* fdms_paged_prepare_decode_plan against its CPU restatement (the emulator's
  paged_prepare_decode_plan, tests/native_emulator.py) on random paged
  states, including spans whose pages are full (a page pop per append) and a
  pool too short for every pop: live counts, append rows, block tables, pages
  held, stack top, overflow flag and every item slot, bit for bit.
* fdms_fused_decode_attention_planned on that plan against the unplanned
  launch (fdms_fused_decode_attention_paged) on the same state: DMS decisions
  and appended FP8 rows bit for bit, outputs bit for bit at head_dim 64 (the
  same partition) and within a bf16 rounding at head_dim 128 (the plan
  splits pairs into 512-rank pieces there, so the fp32 summation order
  differs), and both against the oracle's attention over the spans gathered
  through the tables (2e-2 max-abs-relative).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import require_gpu

pytestmark = pytest.mark.gpu

PAGE = 16


def _state(rng, L, B, H, max_live, spare_pages, full_every=5):
    """live [L, B, H] (every full_every-th span a multiple of 16: its append
    pops a page), held = ceil(live / 16), tables through a random page
    permutation, the rest of the pool on the stacks."""
    live = rng.integers(0, max_live, (L, B, H)).astype(np.int32)
    flat = live.reshape(-1)
    flat[::full_every] = (flat[::full_every] // PAGE) * PAGE
    held = -(-live // PAGE)
    max_pages = -(-(max_live + 1) // PAGE)
    pool = int(held.sum(axis=(1, 2)).max()) + spare_pages
    bt = np.full((L, B, H, max_pages), -1, np.int32)
    stack = np.zeros((L, pool), np.int32)
    top = np.zeros(L, np.int32)
    for l in range(L):
        perm = rng.permutation(pool).astype(np.int32)
        used = 0
        for b in range(B):
            for h in range(H):
                n = int(held[l, b, h])
                bt[l, b, h, :n] = perm[used:used + n]
                used += n
        top[l] = pool - used
        stack[l, :top[l]] = perm[used:]
    return live, held.astype(np.int32), bt, stack, top, pool, max_pages


def _run_plan(call, t, L, B, H, max_pages, part):
    rows, heavy, splits = part
    call("fdms_paged_prepare_decode_plan", t["live"].data_ptr(), *t["live"].stride(), t["slot"].data_ptr(),
         *t["slot"].stride(), t["bt"].data_ptr(), *t["bt"].stride()[:3], t["held"].data_ptr(), *t["held"].stride(),
         t["stack"].data_ptr(), t["stack"].stride(0), t["top"].data_ptr(), max_pages, t["overflow"].data_ptr(),
         t["pos"].data_ptr(), t["plan"].data_ptr(), t["plan"].stride(0), rows, heavy, splits, L, B, H, 0)


def _tensors(live, held, bt, stack, top, pos, L, B, H, items, device):
    mk = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    return dict(live=mk(live), held=mk(held), bt=mk(bt), stack=mk(stack), top=mk(top), pos=mk(pos),
                slot=torch.full((L, B, H), -7, dtype=torch.int32, device=device),
                overflow=torch.zeros(1, dtype=torch.int32, device=device),
                plan=torch.full((L, 4 + items * 72), -9, dtype=torch.int32, device=device))


@pytest.mark.parametrize("L,B,H,max_live,spare,seed,part", [
    (3, 8, 8, 2900, 64, 0, (1024, 512)), (2, 3, 8, 600, 40, 1, (1024, 512)), (2, 40, 8, 1500, 500, 2, (1024, 1024)),
    (2, 8, 8, 1200, 3, 3, (512, 512)), (1, 1, 2, 40, 8, 4, (1024, 512)), (2, 8, 8, 3000, 64, 5, (256, 128))])
def test_plan_kernel_equals_its_restatement(L, B, H, max_live, spare, seed, part):
    require_gpu()
    from fastdms_amd import _native as nat
    from native_emulator import Emulator
    rng = np.random.default_rng(seed)
    live, held, bt, stack, top, pool, max_pages = _state(rng, L, B, H, max_live, spare)
    pos = rng.integers(max_live, 8000, B).astype(np.int64)
    splits = min(64, -(-(max_live + 1) // part[1]))
    items = splits * B * H
    dev = _tensors(live, held, bt, stack, top, pos, L, B, H, items, "cuda")
    _run_plan(lambda name, *a: nat.call(name, *a[:-1], nat.stream()), dev, L, B, H, max_pages, (*part, splits))
    torch.cuda.synchronize()
    cpu = _tensors(live, held, bt, stack, top, pos, L, B, H, items, "cpu")
    emu = Emulator()
    _run_plan(lambda name, *a: emu(name, *a), cpu, L, B, H, max_pages, (*part, splits))
    for key in ("live", "slot", "bt", "held", "top", "overflow", "plan"):
        assert torch.equal(dev[key].cpu(), cpu[key]), key
    short = int(dev["overflow"].item())
    further = cpu["plan"][:, 3].tolist()
    print(f"L{L} B{B} H{H} part {part}: {B * H} first + {further} further splits per layer (grid {items}), "
          f"overflow {short}, pool {pool}", flush=True)
    if spare == 3:
        assert short == 1, "the short pool case must run out of pages"


@pytest.mark.parametrize("d,qk_norm,scales", [(64, False, False), (64, False, True), (128, True, False)])
def test_planned_attention_equals_the_unplanned_launch(d, qk_norm, scales):
    require_gpu()
    from fastdms_amd import _native as nat
    from fastdms_amd.layers import compact_attention as ca
    from oracle import attention as oatt
    from oracle import numerics
    rng = np.random.default_rng(d + qk_norm + 2 * scales)
    L, B, H, hq = 1, 8, 8, 32
    max_live = 2900
    live, held, bt, stack, top, pool, max_pages = _state(rng, L, B, H, max_live, 64)
    pos = rng.integers(max_live, 8000, B).astype(np.int64)
    plan = ca.DecodePlan("cuda", L, B * H, max_live + 1, d)
    dev = _tensors(live, held, bt, stack, top, pos, L, B, H, (plan.items.shape[1] - 4) // 72, "cuda")
    dev["plan"] = plan.items
    _run_plan(lambda name, *a: nat.call(name, *a[:-1], nat.stream()), dev, L, B, H, max_pages,
              plan.partition(B * H))
    assert int(dev["overflow"].item()) == 0
    rows = pool * PAGE
    ck = torch.from_numpy(numerics.to_storage(rng.standard_normal((rows, d)).astype(np.float32) * 2,
                                              numerics.DT_FP8)).cuda().view(torch.float8_e4m3fn)
    cv = torch.from_numpy(numerics.to_storage(rng.standard_normal((rows, d)).astype(np.float32),
                                              numerics.DT_FP8)).cuda().view(torch.float8_e4m3fn)
    qkv = torch.from_numpy(numerics.cast(rng.standard_normal((B, (hq + 2 * H) * d)).astype(np.float32) * 3,
                                         numerics.DT_BF16)).cuda().to(torch.bfloat16)
    q, k, v = qkv[:, :hq * d].view(B, hq, d), qkv[:, hq * d:(hq + H) * d].view(B, H, d), qkv[:, (hq + H) * d:].view(B, H, d)
    cache = torch.from_numpy(oatt.rope_cos_sin_cache(d, 8192, 500000.0)).cuda()
    norms = {}
    if qk_norm:
        w = lambda: torch.from_numpy(numerics.cast((1 + 0.2 * rng.standard_normal(d)).astype(np.float32),  # noqa: E731
                                                   numerics.DT_BF16)).cuda().to(torch.bfloat16)
        norms = dict(q_norm_weight=w(), k_norm_weight=w(), norm_eps=1e-6)
    ks = vs = None
    if scales:
        ks = torch.from_numpy((0.5 + rng.random(H)).astype(np.float32)).cuda()
        vs = torch.from_numpy((0.5 + rng.random(H)).astype(np.float32)).cuda()
    ck2, cv2 = ck.clone(), cv.clone()
    ev_p = torch.empty((B, H), dtype=torch.bool, device="cuda")
    out_p = ca.fused_decode_attention_planned(q, k, v, cache, ck, cv, ev_p, dev["pos"], plan, 0, num_kv_heads=H,
                                              alpha_scale=10.0, alpha_offset=5.0, k_scale=ks, v_scale=vs, **norms)
    ev_u = torch.empty((B, H), dtype=torch.bool, device="cuda")
    out_u = ca.fused_dms_rope_store_compact_decode_attention(
        q, k, v, cache, ck2, cv2, dev["slot"][0], ev_u, dev["pos"], None, dev["live"][0], num_kv_heads=H,
        alpha_scale=10.0, alpha_offset=5.0, max_live_count=max_live + 1, k_scale=ks, v_scale=vs,
        block_tables=dev["bt"][0], page_size=PAGE, **norms)
    torch.cuda.synchronize()
    assert torch.equal(ev_p, ev_u), "DMS decisions"
    assert torch.equal(ck.view(torch.uint8), ck2.view(torch.uint8)) and torch.equal(cv.view(torch.uint8),
                                                                                      cv2.view(torch.uint8))
    a, u = out_p.float().cpu().numpy(), out_u.float().cpu().numpy()
    rel = float(np.abs(a - u).max() / np.abs(u).max())
    if d == 64:  # the same partition: the same bits
        assert torch.equal(out_p.view(torch.int16), out_u.view(torch.int16)), f"planned vs unplanned {rel:.3e}"
    assert rel <= 8e-3, f"planned vs unplanned max-abs-rel {rel:.3e}"
    # both against the oracle over the spans gathered through the tables
    lv = dev["live"][0].cpu().numpy()
    tb = dev["bt"][0].cpu().numpy()
    kf = numerics.from_storage(ck.view(torch.uint8).cpu().numpy(), numerics.DT_FP8)
    vf = numerics.from_storage(cv.view(torch.uint8).cpu().numpy(), numerics.DT_FP8)
    cap = int(lv.max())
    base = (np.arange(B * H).reshape(B, H) * cap).astype(np.int32)
    kspan = np.zeros((B * H * cap, d), np.float64)
    vspan = np.zeros_like(kspan)
    for b in range(B):
        for h in range(H):
            r = np.arange(lv[b, h])
            rows_ = tb[b, h, r // PAGE].astype(np.int64) * PAGE + r % PAGE
            kspan[base[b, h]:base[b, h] + lv[b, h]] = kf[rows_]
            vspan[base[b, h]:base[b, h] + lv[b, h]] = vf[rows_]
    qf = q.float().cpu().numpy()
    if qk_norm:
        qt = torch.from_numpy(qf)
        qt = (qt * torch.rsqrt(qt.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16).float()
        qf = (qt * norms["q_norm_weight"].float().cpu()).to(torch.bfloat16).float().numpy()
    cs = oatt.rope_cos_sin_cache(d, 8192, 500000.0)
    qr = qf.copy()
    qr[:, ::hq // H, d - 1] = 0.0
    qr = oatt.apply_rotary_emb(qr, cs[pos][:, None, 0, :d // 2], cs[pos][:, None, 0, d // 2:], numerics.DT_BF16)
    ref = oatt.compact_decode_attention(qr, kspan, vspan, base, lv,
                                        k_scale=None if ks is None else ks.cpu().numpy(),
                                        v_scale=None if vs is None else vs.cpu().numpy())
    for name, o in (("planned", a), ("unplanned", u)):
        err = float(np.abs(o - ref).max() / np.abs(ref).max())
        assert err <= 2e-2, f"{name} vs oracle {err:.3e}"
    print(f"d={d} qk_norm={qk_norm} scales={scales}: planned vs unplanned {rel:.2e}, partition "
          f"{plan.partition(B * H)}", flush=True)
