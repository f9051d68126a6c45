"""A11-A15: decode expiry (exact / full / incremental / skip policy), append
slots and decision recording on the GPU vs the stateful oracle (bit-exact)."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import TORCH_DTYPE, require_gpu, storage_of, to_torch
from oracle import compact_kv as ock
from oracle import numerics

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def _mk(layer_major, code, L=2, H=2, d=4, cap_tokens=128, mml=9, max_tokens=5, prompt=4, n_seqs=1):
    from fastdms_amd.engine.compact_kv import CompactKVManager
    from fastdms_amd.engine.sequence import Sequence
    from fastdms_amd.sampling_params import SamplingParams
    prod = CompactKVManager(num_layers=L, num_kv_heads=H, capacity_tokens=cap_tokens, max_model_len=mml,
                            device="cuda", head_dim=d, compact_dtype=TORCH_DTYPE[code], per_layer_storage=True,
                            layer_major_metadata=layer_major, max_active_seqs=max(2, n_seqs))
    orc = ock.OracleCompactKVManager(L, H, cap_tokens, mml, head_dim=d, dtype_code=code)
    seqs = [Sequence(list(range(prompt)), SamplingParams(max_tokens=max_tokens)) for _ in range(n_seqs)]
    for s in seqs:
        prod.allocate(s)
        orc.allocate(s.seq_id, prompt, max_tokens)
    return prod, orc, seqs


def _load_state(prod, orc, seqs, live_per_lh, positions_fn, evict_fn, value_fn, code):
    """Write the same spans into both managers (like _build_cuda_expiry_case, test_compact_kv.py:365-402)."""
    L, H, d = prod.num_layers, prod.num_kv_heads, prod.head_dim
    for layer in range(L):
        high = 64
        for s in seqs:
            live = [live_per_lh(s, layer, h) for h in range(H)]
            prod._allocate_layer_ranges_for_seq(prod.seq_states[s.seq_id], layer, live)
            orc.allocate_layer_ranges_for_seq(orc.seq_states[s.seq_id], layer, live)
            os_ = orc.seq_states[s.seq_id]
            high = max(high, int((os_.base_offsets[layer] + os_.range_capacity[layer]).max()))
        prod._ensure_layer_storage(layer, high)
        orc._ensure_layer_storage(layer, high)
        prod.compact_k_per_layer[layer].zero_()
        prod.compact_v_per_layer[layer].zero_()
    for s in seqs:
        ps, os_ = prod.seq_states[s.seq_id], orc.seq_states[s.seq_id]
        for layer in range(L):
            ck_o, cv_o = orc.compact_k_per_layer[layer], orc.compact_v_per_layer[layer]
            for h in range(H):
                n = live_per_lh(s, layer, h)
                pos = positions_fn(s, layer, h, n)
                ev = evict_fn(s, layer, h, pos)
                os_.live_counts[layer, h] = n
                os_.token_positions[layer, h, :n] = pos
                os_.evict_mask[layer, h, :n] = ev
                b0 = int(os_.base_offsets[layer, h])
                vals = value_fn(s, layer, h, pos)
                ck_o[b0:b0 + n] = numerics.to_storage(vals, code)
                cv_o[b0:b0 + n] = numerics.to_storage(vals + 0.5, code)
        ps.live_counts.copy_(torch.from_numpy(os_.live_counts).cuda())
        ps.token_positions.copy_(torch.from_numpy(os_.token_positions).cuda())
        ps.evict_mask.copy_(torch.from_numpy(os_.evict_mask).cuda())
    for layer in range(L):
        prod.compact_k_per_layer[layer].copy_(to_torch(orc.compact_k_per_layer[layer], code))
        prod.compact_v_per_layer[layer].copy_(to_torch(orc.compact_v_per_layer[layer], code))


def _append(prod, orc, seqs, position, value_fn, evict_fn, code):
    """_append_cuda_expiry_token (test_compact_kv.py:405-421) on both managers."""
    for s in seqs:
        ps, os_ = prod.seq_states[s.seq_id], orc.seq_states[s.seq_id]
        for layer in range(prod.num_layers):
            for h in range(prod.num_kv_heads):
                idx = int(os_.live_counts[layer, h])
                b0 = int(os_.base_offsets[layer, h])
                ev = evict_fn(s, layer, h, np.array([position]))[0]
                os_.token_positions[layer, h, idx] = position
                os_.evict_mask[layer, h, idx] = ev
                val = value_fn(s, layer, h, np.array([position]))
                orc.compact_k_per_layer[layer][b0 + idx] = numerics.to_storage(val, code)[0]
                orc.compact_v_per_layer[layer][b0 + idx] = numerics.to_storage(val + 0.5, code)[0]
                os_.live_counts[layer, h] += 1
        ps.live_counts.copy_(torch.from_numpy(os_.live_counts).cuda())
        ps.token_positions.copy_(torch.from_numpy(os_.token_positions).cuda())
        ps.evict_mask.copy_(torch.from_numpy(os_.evict_mask).cuda())
    for layer in range(prod.num_layers):
        prod.compact_k_per_layer[layer].copy_(to_torch(orc.compact_k_per_layer[layer], code))
        prod.compact_v_per_layer[layer].copy_(to_torch(orc.compact_v_per_layer[layer], code))


def _assert_equal(prod, orc, seqs):
    torch.cuda.synchronize()
    for s in seqs:
        ps, os_ = prod.seq_states[s.seq_id], orc.seq_states[s.seq_id]
        assert np.array_equal(ps.live_counts.cpu().numpy(), os_.live_counts)
        assert np.array_equal(ps.token_positions.cpu().numpy(), os_.token_positions)
        assert np.array_equal(ps.evict_mask.cpu().numpy(), os_.evict_mask)
        for layer in range(prod.num_layers):
            ckp = storage_of(prod.compact_k_per_layer[layer])
            cvp = storage_of(prod.compact_v_per_layer[layer])
            for h in range(prod.num_kv_heads):
                b0, n = int(os_.base_offsets[layer, h]), int(os_.live_counts[layer, h])
                assert np.array_equal(ckp[b0:b0 + n], orc.compact_k_per_layer[layer][b0:b0 + n])
                assert np.array_equal(cvp[b0:b0 + n], orc.compact_v_per_layer[layer][b0:b0 + n])


@pytest.mark.parametrize("code", [numerics.DT_F32, numerics.DT_FP8])
@pytest.mark.parametrize("layer_major", [False, True])
def test_reference_expiry_sequence(monkeypatch, code, layer_major):
    """test_compact_kv.py:1283-1329: capacity 9 (not a power of two), window 3,
    exact at cur=8, then forced incremental at 9 and 10 with appends between."""
    require_gpu()
    prod, orc, seqs = _mk(layer_major, code)
    live_fn = lambda s, l, h: [6, 7][h]
    pos_fn = lambda s, l, h, n: np.arange(n, dtype=np.int32)
    ev_fn = lambda s, l, h, pos: (pos % 2) == 0
    val_fn = lambda s, l, h, pos: (np.float32(l * 10.0 + h) + pos.astype(np.float32) * np.float32(0.01))[:, None] \
        .repeat(prod.head_dim, 1).astype(np.float32)
    _load_state(prod, orc, seqs, live_fn, pos_fn, ev_fn, val_fn, code)
    monkeypatch.setenv("FASTDMS_DMS_EXPIRY_TRITON", "0")
    st_p = prod.apply_dms_evictions(seqs, [8], window_size=3)
    act, st_o = orc.apply_dms_evictions([s.seq_id for s in seqs], [8], window_size=3, triton_mode="0")
    assert act == "exact" and st_p == st_o
    _assert_equal(prod, orc, seqs)
    for cur in (9, 10):
        _append(prod, orc, seqs, cur - 1, val_fn, ev_fn, code)
        monkeypatch.setenv("FASTDMS_DMS_EXPIRY_TRITON", "1")
        monkeypatch.setenv("FASTDMS_DMS_EXPIRY_INTERVAL", "1")
        prod.apply_dms_evictions(seqs, [cur], window_size=3)
        act, _ = orc.apply_dms_evictions([s.seq_id for s in seqs], [cur], window_size=3, triton_mode="1",
                                         interval_env="1")
        assert act == "incremental"
        _assert_equal(prod, orc, seqs)


@pytest.mark.parametrize("layer_major", [True, False])
def test_large_batched_expiry_policy_run(monkeypatch, layer_major):
    """4 sequences x 3 layers x 8 heads, FP8 rows of 64 B, ~1-2k live slots;
    auto policy: exact, skips, a full expiry at a window multiple, then forced incremental."""
    require_gpu()
    code = numerics.DT_FP8
    rng = np.random.default_rng(2)
    prod, orc, seqs = _mk(layer_major, code, L=3, H=8, d=64, cap_tokens=80000, mml=4096, max_tokens=300,
                          prompt=2000, n_seqs=4)
    lives = {(s.seq_id, l, h): int(rng.integers(200, 1800)) for s in seqs for l in range(3) for h in range(8)}
    live_fn = lambda s, l, h: lives[(s.seq_id, l, h)]
    pos_fn = lambda s, l, h, n: np.sort(rng.choice(2000, n, replace=False)).astype(np.int32)
    flags = {}

    def ev_fn(s, l, h, pos):
        return np.array([flags.setdefault((s.seq_id, l, h, int(p)), bool(rng.random() < 0.7)) for p in pos])

    val_fn = lambda s, l, h, pos: (rng.standard_normal((len(pos), 64)) * 2).astype(np.float32)
    _load_state(prod, orc, seqs, live_fn, pos_fn, ev_fn, val_fn, code)
    monkeypatch.delenv("FASTDMS_DMS_EXPIRY_TRITON", raising=False)
    monkeypatch.delenv("FASTDMS_DMS_EXPIRY_INTERVAL", raising=False)
    ids = [s.seq_id for s in seqs]
    cur = 2040
    seen = []
    for step in range(30):
        pos = [cur + step] * 4
        if step >= 20:
            monkeypatch.setenv("FASTDMS_DMS_EXPIRY_TRITON", "1")
            monkeypatch.setenv("FASTDMS_DMS_EXPIRY_INTERVAL", "1")
            mode, interval = "1", "1"
        else:
            mode, interval = "auto", None
        act = prod.expiry_action(seqs, pos, 256)
        st_p = prod.apply_dms_evictions(seqs, pos, window_size=256)
        act_o, st_o = orc.apply_dms_evictions(ids, pos, window_size=256, triton_mode=mode, interval_env=interval)
        assert act == act_o
        assert st_p == st_o
        seen.append(act)
        _assert_equal(prod, orc, seqs)
        _append(prod, orc, seqs, cur + step, val_fn, ev_fn, code)
    assert {"exact", "skip", "full", "incremental"} <= set(seen)


def test_record_and_prepare_golden_on_gpu():
    require_gpu()
    from fastdms_amd.engine.compact_kv import CompactKVManager
    from fastdms_amd.engine.sequence import Sequence
    from fastdms_amd.sampling_params import SamplingParams
    g = GOLDEN["record_decisions_layer_major"]
    m = CompactKVManager(num_layers=g["num_layers"], num_kv_heads=g["num_kv_heads"],
                         capacity_tokens=g["capacity_tokens"], max_model_len=g["max_model_len"], device="cuda",
                         layer_major_metadata=True, max_active_seqs=g["max_active_seqs"])
    seqs = [Sequence([10, 11], SamplingParams(max_tokens=4)), Sequence([20, 21], SamplingParams(max_tokens=4))]
    for s in seqs:
        m.allocate(s).live_counts.fill_(g["initial_live"])
    ev = torch.tensor(g["evictions"], device="cuda", dtype=torch.bool)
    for positions in (g["positions"], torch.tensor(g["positions"], device="cuda", dtype=torch.int64)):
        stats = m.record_appended_dms_decisions(seqs, positions, ev)
        torch.cuda.synchronize()
        assert stats == g["expected_stats"]
        assert m.layer_major_token_positions[:, 0, :, 0].cpu().tolist() == g["expected_positions_slot0"]
        assert m.layer_major_token_positions[:, 1, :, 0].cpu().tolist() == g["expected_positions_slot1"]
        assert torch.equal(m.layer_major_evict_mask[:, :2, :, 0].cpu(), ev.cpu())

    p = GOLDEN["prepare_decode_metadata"]
    for layer_major in (False, True):
        m = CompactKVManager(num_layers=p["num_layers"], num_kv_heads=p["num_kv_heads"],
                             capacity_tokens=p["capacity_tokens"], max_model_len=p["max_model_len"], device="cuda",
                             layer_major_metadata=layer_major, max_active_seqs=2)
        seq = Sequence([10, 11], SamplingParams(max_tokens=p["max_tokens"]))
        st = m.allocate(seq)
        for layer in range(p["num_layers"]):
            m._allocate_layer_ranges_for_seq(st, layer, torch.full((p["num_kv_heads"],), 2, dtype=torch.int32))
        m.mark_all_heads_live(seq.seq_id, p["live_per_head"])
        base, live, slot, mx = m.prepare_decode_metadata([seq])
        torch.cuda.synchronize()
        assert base.cpu().tolist() == p["expected_base_offsets"]
        assert slot.cpu().tolist() == p["expected_slot_mapping"]
        assert live.cpu().tolist() == p["expected_live_counts"]
        assert st.live_counts.cpu().tolist() == p["expected_state_live_counts"]
        assert mx == st.max_capacity_per_lh
