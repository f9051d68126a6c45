"""fdms_fused_decode_attention_noalloc (the allocation-free variant of the fused
decode attention, whose split partials and tickets live in the library's own
device array) against fdms_fused_decode_attention with a caller workspace,
through the C-ABI: decisions, appended FP8 rows and outputs bit-identical, on
two calls in a row, the second with a smaller batch (the array keeps the
first call's contents), with and without per-head FP8 scales."""
import numpy as np
import pytest
import torch

from helpers import from_values, require_gpu
from oracle import attention as oatt
from oracle import numerics

pytestmark = pytest.mark.gpu


def _case(rng, b, hkv=8, g=4, d=64, cap=1600):
    hq = hkv * g
    live_prev = rng.integers(1, cap - 1, (b, hkv)).astype(np.int32)
    base = (np.arange(b * hkv).reshape(b, hkv) * cap).astype(np.int32)
    slot = base + live_prev
    slot[0, 1] = -1  # a pair without an append
    live = live_prev + (slot >= 0)
    qkv = numerics.cast(rng.standard_normal((b, (hq + 2 * hkv) * d)).astype(np.float32), numerics.DT_BF16)
    ck = numerics.to_storage(rng.standard_normal((b * hkv * cap, d)).astype(np.float32), numerics.DT_FP8)
    cv = numerics.to_storage(rng.standard_normal((b * hkv * cap, d)).astype(np.float32), numerics.DT_FP8)
    pos = rng.integers(2000, 8000, b).astype(np.int64)
    return qkv, ck, cv, base, slot, live, pos, cap


def _run(noalloc, case, hkv, g, d, scales, splits, split_rows):
    from fastdms_amd import _native as nat
    from fastdms_amd.engine.dms import dms_threshold_args
    from fastdms_amd.layers.compact_attention import attention_workspace
    qkv, ck, cv, base, slot, live, pos, cap = case
    b, hq = qkv.shape[0], hkv * g
    qkv_d = from_values(qkv, numerics.DT_BF16)
    q = qkv_d[:, :hq * d].view(b, hq, d)
    k = qkv_d[:, hq * d:(hq + hkv) * d].view(b, hkv, d)
    v = qkv_d[:, (hq + hkv) * d:].view(b, hkv, d)
    ckd = torch.from_numpy(ck.copy()).cuda()
    cvd = torch.from_numpy(cv.copy()).cuda()
    cache = torch.from_numpy(oatt.rope_cos_sin_cache(d, 8192, 500000.0)).cuda()
    posd, slotd = torch.from_numpy(pos).cuda(), torch.from_numpy(slot).cuda()
    based, lived = torch.from_numpy(base).cuda(), torch.from_numpy(live).cuda()
    ev = torch.full((b, hkv), 7, dtype=torch.uint8, device="cuda")
    out = torch.full((b, hq, d), float("nan"), dtype=torch.bfloat16, device="cuda")
    ks, vs = (None, None) if scales is None else (torch.from_numpy(scales[0]).cuda(),
                                                  torch.from_numpy(scales[1]).cuda())
    s_, off, thr, positive = dms_threshold_args(10.0, 5.0)
    head = [q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0),
            v.stride(1), cache.data_ptr(), cache.stride(0), cache.stride(2), posd.data_ptr(), slotd.data_ptr(),
            slotd.stride(0), slotd.stride(1), ev.data_ptr(), ev.stride(0), ev.stride(1), s_, off, thr, positive,
            ckd.data_ptr(), cvd.data_ptr(), d, based.data_ptr(), based.stride(0), based.stride(1), lived.data_ptr(),
            lived.stride(0), lived.stride(1), out.data_ptr(), out.stride(0), out.stride(1)]
    tail = [b, hkv, g, d, splits, split_rows, d ** -0.5, nat.ptr(ks), nat.ptr(vs), None, None, 0.0, nat.stream()]
    if noalloc:
        nat.call("fdms_fused_decode_attention_noalloc", *head, *tail)
    else:
        ws, cnt = attention_workspace(q.device, b * hkv * splits * g * (d + 2), b * hkv)
        nat.call("fdms_fused_decode_attention", *head, ws.data_ptr(), cnt.data_ptr(), *tail)
    torch.cuda.synchronize()
    return ev.cpu(), out.cpu(), ckd.cpu(), cvd.cpu()


@pytest.mark.parametrize("scaled", [False, True])
def test_noalloc_equals_workspace_entry_point(scaled):
    require_gpu()
    rng = np.random.default_rng(21 + scaled)
    hkv, g, d = 8, 4, 64
    # first call: 8 sequences, long spans split 7 ways; second: 3 sequences
    for b, splits, rows in ((8, 7, 256), (3, 4, 512)):
        case = _case(rng, b, hkv, g, d)
        scales = None
        if scaled:
            scales = (np.exp(rng.uniform(-1, 1, hkv)).astype(np.float32),
                      np.exp(rng.uniform(-1, 1, hkv)).astype(np.float32))
        want = _run(False, case, hkv, g, d, scales, splits, rows)
        got = _run(True, case, hkv, g, d, scales, splits, rows)
        for w, x in zip(want, got):
            assert torch.equal(w.view(torch.uint8) if w.dtype != torch.uint8 else w,
                               x.view(torch.uint8) if x.dtype != torch.uint8 else x)
        assert not torch.isnan(got[1].float()).any()


def test_noalloc_rejects_sizes_beyond_its_scratch():
    """pairs * splits * group * (head_dim + 2) above 2^21 floats is refused
    before anything is launched."""
    require_gpu()
    from fastdms_amd import _native as nat
    lib = nat.lib()
    fn = lib.fdms_fused_decode_attention_noalloc
    args = [None, 0, 0, None, 0, 0, None, 0, 0, None, 0, 0, None, None, 0, 0, None, 0, 0, 1.0, 1.0, 1.0, 1,
            None, None, 64, None, 0, 0, None, 0, 0, None, 0, 0]
    # 512 sequences x 8 heads x 64 splits x 4 x 66 floats > 2^21
    rc = fn(*args, 512, 8, 4, 64, 64, 256, 0.125, None, None, None, None, 0.0, None)
    assert rc == 1  # hipErrorInvalidValue


def _first_call_under_capture() -> None:
    """Child process body: the process's first fdms_fused_decode_attention_noalloc
    call is made under HIP graph capture (so the library's ticket-zeroing
    kernel is captured, not run: the tickets rely on the device array being
    zero at module load); three replays, with eager work and synchronizations
    between them, each equal to the workspace entry point's eager result."""
    rng = np.random.default_rng(5)
    hkv, g, d = 8, 4, 64
    case = _case(rng, 6, hkv, g, d)
    want = _run(False, case, hkv, g, d, None, 7, 256)
    from fastdms_amd import _native as nat
    from fastdms_amd.engine.dms import dms_threshold_args
    qkv, ck, cv, base, slot, live, pos, cap = case
    b, hq = qkv.shape[0], hkv * g
    qkv_d = from_values(qkv, numerics.DT_BF16)
    q, k, v = (qkv_d[:, :hq * d].view(b, hq, d), qkv_d[:, hq * d:(hq + hkv) * d].view(b, hkv, d),
               qkv_d[:, (hq + hkv) * d:].view(b, hkv, d))
    ckd, cvd = torch.from_numpy(ck.copy()).cuda(), torch.from_numpy(cv.copy()).cuda()
    cache = torch.from_numpy(oatt.rope_cos_sin_cache(d, 8192, 500000.0)).cuda()
    posd, slotd = torch.from_numpy(pos).cuda(), torch.from_numpy(slot).cuda()
    based, lived = torch.from_numpy(base).cuda(), torch.from_numpy(live).cuda()
    ev = torch.zeros((b, hkv), dtype=torch.uint8, device="cuda")
    out = torch.zeros((b, hq, d), dtype=torch.bfloat16, device="cuda")
    s_, off, thr, positive = dms_threshold_args(10.0, 5.0)
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream), torch.cuda.graph(graph, stream=stream):
        nat.call("fdms_fused_decode_attention_noalloc", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
                 k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), cache.data_ptr(),
                 cache.stride(0), cache.stride(2), posd.data_ptr(), slotd.data_ptr(), slotd.stride(0),
                 slotd.stride(1), ev.data_ptr(), ev.stride(0), ev.stride(1), s_, off, thr, positive, ckd.data_ptr(),
                 cvd.data_ptr(), d, based.data_ptr(), based.stride(0), based.stride(1), lived.data_ptr(),
                 lived.stride(0), lived.stride(1), out.data_ptr(), out.stride(0), out.stride(1), b, hkv, g, d, 7,
                 256, d ** -0.5, None, None, None, None, 0.0, nat.stream())
    for replay in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        noise = torch.randn(1 << 20, device="cuda").sum()  # eager work between the replays
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        got = (ev.cpu(), out.cpu(), ckd.cpu(), cvd.cpu())
        for w, x in zip(want, got):
            assert torch.equal(w.view(torch.uint8) if w.dtype != torch.uint8 else w,
                               x.view(torch.uint8) if x.dtype != torch.uint8 else x), f"replay {replay}"
    print("first call under capture: 3 replays equal", flush=True)


def test_first_call_on_a_device_under_graph_capture():
    """In a fresh process (the library keeps its per-device set-up for the
    process's lifetime) the first allocation-free call is captured."""
    require_gpu()
    import os
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    code = ("import sys; sys.path[:0] = [%r, %r]; import test_zz_no_alloc as t; t._first_call_under_capture()"
            % (str(root), str(root / "tests")))
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300,
                         env=dict(os.environ))
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0 and "3 replays equal" in res.stdout
