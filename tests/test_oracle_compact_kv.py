"""Pin the compact-KV oracle on the reference's literal vectors, brute force
and set-formula invariants; check the product manager's host-only
bookkeeping (allocator, views) on the same vectors."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import compact_kv as ock
from oracle import numerics

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def test_pack_compact_kv_golden():
    g = GOLDEN["pack_compact_kv"]
    k = np.arange(40, dtype=np.float32).reshape(g["k_shape"])
    v = k + 100
    ck, cv, base, live, pos = ock.pack_compact_kv(k, v, np.array(g["live_mask"]))
    assert list(ck.shape) == g["expected_compact_shape"]
    assert base.tolist() == g["expected_base_offsets"]
    assert live.tolist() == g["expected_live_counts"]
    assert pos.tolist() == g["expected_token_positions"]
    assert np.array_equal(cv, ck + 100)


def test_emulated_stride_mask_golden():
    g = GOLDEN["emulated_stride_mask"]
    m = ock.build_emulated_dms_live_mask(num_layers=g["num_layers"], num_kv_heads=g["num_kv_heads"],
                                         num_tokens=g["num_tokens"], mode="dms_stride", stride=g["stride"],
                                         recent_tokens=g["recent_tokens"])
    assert m.tolist() == g["expected"]


@pytest.mark.parametrize("impl", ["oracle", "product"])
def test_allocator_alloc_free_golden(impl):
    g = GOLDEN["allocator_alloc_free"]
    if impl == "oracle":
        m = ock.OracleCompactKVManager(g["num_layers"], g["num_kv_heads"], g["capacity_tokens"], g["max_model_len"])
        st = m.allocate(0, g["prompt_tokens"], g["max_tokens"])
        assert m.allocate(0, g["prompt_tokens"], g["max_tokens"]) is st
        base, rcap = st.base_offsets.tolist(), st.range_capacity.tolist()
        sid = 0
    else:
        from fastdms_amd.engine.compact_kv import CompactKVManager
        from fastdms_amd.engine.sequence import Sequence
        from fastdms_amd.sampling_params import SamplingParams
        m = CompactKVManager(num_layers=g["num_layers"], num_kv_heads=g["num_kv_heads"],
                             capacity_tokens=g["capacity_tokens"], max_model_len=g["max_model_len"], device="cpu")
        seq = Sequence(list(range(g["prompt_tokens"])), SamplingParams(max_tokens=g["max_tokens"]))
        st = m.allocate(seq)
        assert m.allocate(seq) is st
        base, rcap = st.base_offsets.tolist(), st.range_capacity.tolist()
        sid = seq.seq_id
    assert st.max_capacity_per_lh == g["expected_max_capacity_per_lh"]
    assert base == g["expected_base_offsets"]
    assert rcap == g["expected_range_capacity"]
    assert m.free_tokens == g["expected_free_tokens"]
    m.free(sid)
    assert m.free_tokens == g["expected_free_tokens"]
    assert [[list(r) for r in layer] for layer in m.free_ranges_per_layer] == g["expected_free_ranges_after_free"]


def test_product_layer_major_active_slots_golden():
    from fastdms_amd.engine.compact_kv import CompactKVManager
    from fastdms_amd.engine.sequence import Sequence
    from fastdms_amd.sampling_params import SamplingParams
    g = GOLDEN["layer_major_active_slots"]
    m = CompactKVManager(num_layers=g["num_layers"], num_kv_heads=g["num_kv_heads"],
                         capacity_tokens=g["capacity_tokens"], max_model_len=g["max_model_len"], device="cpu",
                         layer_major_metadata=True, max_active_seqs=g["max_active_seqs"])
    seqs = [Sequence(list(range(n)), SamplingParams(max_tokens=mt)) for n, mt in g["seqs"]]
    states = [m.allocate(s) for s in seqs]
    assert [s.active_slot for s in states] == g["expected_active_slots"]
    states[0].live_counts[0, 1] = 7
    states[0].token_positions[0, 1, 0] = 11
    states[0].evict_mask[0, 1, 0] = True
    assert m.layer_major_live_counts[0, 0, 1].item() == 7
    assert m.layer_major_token_positions[0, 0, 1, 0].item() == 11
    assert m.layer_major_evict_mask[0, 0, 1, 0].item() is True
    assert m._contiguous_active_slot_start(states) == g["expected_contiguous_start_in_order"]
    assert m._contiguous_active_slot_start(states[::-1]) == g["expected_contiguous_start_reversed"]
    m.free(seqs[0].seq_id)
    n, mt = g["third_seq"]
    st2 = m.allocate(Sequence(list(range(n)), SamplingParams(max_tokens=mt)))
    assert st2.active_slot == g["expected_third_slot_after_free_first"]
    assert st2.live_counts.sum().item() == 0
    assert st2.token_positions.max().item() == -1


@pytest.mark.parametrize("impl", ["oracle", "product"])
def test_prepare_decode_metadata_golden(impl):
    g = GOLDEN["prepare_decode_metadata"]
    live = [g["live_per_head"]] * g["num_kv_heads"]
    if impl == "oracle":
        m = ock.OracleCompactKVManager(g["num_layers"], g["num_kv_heads"], g["capacity_tokens"], g["max_model_len"])
        st = m.allocate(0, g["prompt_tokens"], g["max_tokens"])
        for l in range(g["num_layers"]):
            m.allocate_layer_ranges_for_seq(st, l, live)
        st.live_counts[:] = g["live_per_head"]
        base, lc, slot, mx = m.prepare_decode_metadata([0])
        state_live = st.live_counts.tolist()
    else:
        from fastdms_amd.engine.compact_kv import CompactKVManager
        from fastdms_amd.engine.sequence import Sequence
        from fastdms_amd.sampling_params import SamplingParams
        m = CompactKVManager(num_layers=g["num_layers"], num_kv_heads=g["num_kv_heads"],
                             capacity_tokens=g["capacity_tokens"], max_model_len=g["max_model_len"], device="cpu")
        seq = Sequence(list(range(g["prompt_tokens"])), SamplingParams(max_tokens=g["max_tokens"]))
        st = m.allocate(seq)
        for l in range(g["num_layers"]):
            m._allocate_layer_ranges_for_seq(st, l, torch.full((g["num_kv_heads"],), 2, dtype=torch.int32))
        m.mark_all_heads_live(seq.seq_id, g["live_per_head"])
        base, lc, slot, mx = m.prepare_decode_metadata([seq])
        state_live = st.live_counts.tolist()
    assert np.asarray(base).tolist() == g["expected_base_offsets"]
    assert np.asarray(slot).tolist() == g["expected_slot_mapping"]
    assert np.asarray(lc).tolist() == g["expected_live_counts"]
    assert state_live == g["expected_state_live_counts"]
    assert mx == st.max_capacity_per_lh == g["expected_max_live_count_is_max_capacity"]


def test_product_layer_head_live_counts_golden():
    from fastdms_amd.engine.compact_kv import CompactKVManager
    from fastdms_amd.engine.sequence import Sequence
    from fastdms_amd.sampling_params import SamplingParams
    g = GOLDEN["layer_head_live_counts"]
    m = CompactKVManager(num_layers=g["num_layers"], num_kv_heads=g["num_kv_heads"],
                         capacity_tokens=g["capacity_tokens"], max_model_len=g["max_model_len"], device="cpu")
    seq = Sequence(list(range(g["prompt_tokens"])), SamplingParams(max_tokens=g["max_tokens"]))
    st = m.allocate(seq)
    live = torch.tensor(g["live_counts"], dtype=torch.int32)
    for l in range(g["num_layers"]):
        m._allocate_layer_ranges_for_seq(st, l, live[l])
    m.mark_live_counts(seq.seq_id, live)
    assert st.live_counts.tolist() == g["live_counts"]
    with pytest.raises(RuntimeError):
        m.mark_live_counts(seq.seq_id, live + 100)


def test_record_decisions_oracle_golden():
    g = GOLDEN["record_decisions_layer_major"]
    m = ock.OracleCompactKVManager(g["num_layers"], g["num_kv_heads"], g["capacity_tokens"], g["max_model_len"])
    for sid in (0, 1):
        st = m.allocate(sid, 2, 4)
        st.live_counts[:] = g["initial_live"]
    stats = m.record_appended_dms_decisions([0, 1], g["positions"], np.array(g["evictions"]))
    assert stats == g["expected_stats"]
    assert m.seq_states[0].token_positions[:, :, 0].tolist() == g["expected_positions_slot0"]
    assert m.seq_states[1].token_positions[:, :, 0].tolist() == g["expected_positions_slot1"]
    ev = np.array(g["evictions"])
    assert np.array_equal(np.stack([m.seq_states[s].evict_mask[:, :, 0] for s in (0, 1)], axis=1), ev)


def test_allocator_rollback_and_exhaustion():
    m = ock.OracleCompactKVManager(1, 2, 10, 100)
    st = m.allocate(0, 6, 0)
    with pytest.raises(RuntimeError):
        m.allocate_layer_ranges_for_seq(st, 0, [6, 6])  # 6 + 6 > 10: second head fails
    assert m.free_ranges_per_layer[0] == [(0, 10)]  # first head rolled back


def test_free_list_coalesces():
    m = ock.OracleCompactKVManager(1, 1, 100, 100)
    a = m._alloc_range(0, 10)
    b = m._alloc_range(0, 20)
    c = m._alloc_range(0, 30)
    m._free_range(0, b, 20)
    assert m.free_ranges_per_layer[0] == [(10, 20), (60, 40)]
    m._free_range(0, a, 10)
    m._free_range(0, c, 30)
    assert m.free_ranges_per_layer[0] == [(0, 100)]


# --- brute force / set-formula pins of the pack and expiry restatements ----

def _brute_pack(seq_evict, seq_len, window):
    kept = {h: [t for t in range(seq_len)
                if (not seq_evict[t, h]) or t >= max(0, seq_len - 1 - window)]
            for h in range(seq_evict.shape[1])}
    return kept


@pytest.mark.parametrize("seq_len,window", [(1, 0), (37, 5), (541, 31), (1000, 256), (300, 1000)])
def test_prefill_rank_is_stable_order_of_kept_tokens(seq_len, window):
    rng = np.random.default_rng(seq_len)
    h, d = 3, 4
    ev = rng.random((seq_len, h)) > 0.4
    k = rng.standard_normal((seq_len, h, d)).astype(np.float32)
    v = rng.standard_normal((seq_len, h, d)).astype(np.float32)
    cap = seq_len + 8
    base = np.array([0, cap, 2 * cap], dtype=np.int32)
    ck = np.zeros((3 * cap, d), np.float32)
    cv = np.zeros((3 * cap, d), np.float32)
    pos = np.full((h, cap), -1, np.int32)
    evm = np.zeros((h, cap), bool)
    live = ock.streaming_pack_rank_scatter(k=k, v=v, seq_evict=ev, compact_k=ck, compact_v=cv, token_positions=pos,
                                           evict_mask=evm, base_offsets=base, start=0, seq_len=seq_len,
                                           window_size=window, dtype_code=numerics.DT_F32)
    kept = _brute_pack(ev, seq_len, window)
    lv, offs = ock.streaming_pack_fused_rank_prepare(ev, seq_len, window)
    assert lv.tolist() == live.tolist() == [len(kept[hh]) for hh in range(h)]
    for hh in range(h):
        ts = kept[hh]
        assert pos[hh, :len(ts)].tolist() == ts
        assert (pos[hh, len(ts):] == -1).all()
        assert evm[hh, :len(ts)].tolist() == ev[ts, hh].tolist()
        assert np.array_equal(ck[base[hh]:base[hh] + len(ts)], k[ts, hh])
        assert np.array_equal(cv[base[hh]:base[hh] + len(ts)], v[ts, hh])
        # chunk offsets are the kept counts of earlier 256-token chunks
        for c in range(offs.shape[1]):
            assert offs[hh, c] == sum(1 for t in ts if t < 256 * c)


def test_expiry_exact_matches_set_formula():
    rng = np.random.default_rng(5)
    cap, live, d, cur, w = 40, 33, 4, 70, 8
    pos = np.full(cap, -1, np.int32)
    pos[:live] = np.sort(rng.choice(70, live, replace=False))
    ev = np.zeros(cap, bool)
    ev[:live] = rng.random(live) > 0.5
    ck = rng.standard_normal((cap + 5, d)).astype(np.float32)
    cv = rng.standard_normal((cap + 5, d)).astype(np.float32)
    base = 5
    keep_idx = [s for s in range(live) if (not ev[s]) or (cur - pos[s]) <= w]
    exp_pos = pos[keep_idx].copy()
    exp_ev = ev[keep_idx].copy()
    exp_k = ck[base + np.array(keep_idx)].copy()
    new_live = ock.expiry_exact(positions=pos, evict=ev, live=live, base=base, compact_k=ck, compact_v=cv,
                                current_position=cur, window_size=w)
    assert new_live == len(keep_idx)
    assert np.array_equal(pos[:new_live], exp_pos) and (pos[new_live:] == -1).all()
    assert np.array_equal(ev[:new_live], exp_ev) and not ev[new_live:].any()
    assert np.array_equal(ck[base:base + new_live], exp_k)


def test_incremental_expiry_reaches_exact_when_one_token_ages_out_per_step():
    # tokens at positions 0..49, every other one evicted; advancing cur by 1
    # per step ages out at most one evicted token per step, so repeated
    # incremental expiry equals one exact expiry at the final position.
    cap, live, w = 64, 50, 10
    base_pos = np.full(cap, -1, np.int32)
    base_pos[:live] = np.arange(live)
    base_ev = np.zeros(cap, bool)
    base_ev[:live] = np.arange(live) % 2 == 0
    rows = np.arange(cap, dtype=np.float32)[:, None].repeat(2, 1)
    p1, e1, k1, v1 = base_pos.copy(), base_ev.copy(), rows.copy(), rows.copy() + 1000
    n = live
    for cur in range(w + 1, 60):
        n = ock.expiry_incremental(positions=p1, evict=e1, live=n, base=0, compact_k=k1, compact_v=v1,
                                   current_position=cur, window_size=w)
    p2, e2, k2, v2 = base_pos.copy(), base_ev.copy(), rows.copy(), rows.copy() + 1000
    n2 = ock.expiry_exact(positions=p2, evict=e2, live=live, base=0, compact_k=k2, compact_v=v2,
                          current_position=59, window_size=w)
    assert n == n2
    assert np.array_equal(p1, p2) and np.array_equal(e1, e2)
    assert np.array_equal(k1[:n], k2[:n]) and np.array_equal(v1[:n], v2[:n])


def test_expiry_policy_branches():
    m = ock.OracleCompactKVManager(1, 1, 64, 64, head_dim=4)
    for sid in range(4):
        m.allocate(sid, 4, 4)
    ids4 = [0, 1, 2, 3]
    assert m.expiry_action(ids4, [10, 10, 10, 10], 256) == "exact"  # first step
    for sid in ids4:
        m.seq_states[sid].dms_initial_expiry_done = True
        m.seq_states[sid].last_dms_expiry_position = 9
    assert m.expiry_action(ids4, [10, 10, 10, 10], 256) == "skip"
    m.seq_states[1].last_dms_expiry_position = 255
    assert m.expiry_action(ids4, [10, 256, 10, 10], 256) == "full"  # one sequence crosses a window multiple
    m.seq_states[1].last_dms_expiry_position = 9
    assert m.expiry_action(ids4, [10, 10, 10, 10], 256, triton_mode="1") == "incremental"
    assert m.expiry_action(ids4, [10, 10, 10, 10], 256, triton_mode="1", interval_env="16") == "skip"
    assert m.expiry_action([0, 1], [10, 10], 256) == "exact"  # B in {2, 3}
    assert m.expiry_action(ids4, [10, 10, 10, 10], 256, triton_mode="0") == "exact"
    assert m.expiry_action(ids4, [11, 10, 10, 10], 256) == "exact"  # not sequential


def test_spans_from_pages_inverts_a_random_paging():
    """oracle.compact_kv.spans_from_pages: spans of random lengths scattered
    into 16-row pages under a random page permutation, then gathered back,
    are the original spans, rank for rank (and rows past live stay zero)."""
    rng = np.random.default_rng(3)
    L, S, H, P, W = 2, 3, 2, 16, 8
    live = rng.integers(0, 70, (L, S, H))
    pages_needed = (live + P - 1) // P
    npages = int(pages_needed.sum(axis=(1, 2)).max()) + 3
    bt = np.full((L, S, H, 5), -1, np.int32)
    spans = {}
    arenas_k = [np.zeros((npages * P, W), np.uint8) for _ in range(L)]
    arenas_v = [np.zeros((npages * P, W), np.uint8) for _ in range(L)]
    for l in range(L):
        ids = rng.permutation(npages)
        at = 0
        for s in range(S):
            for h in range(H):
                n, npg = int(live[l, s, h]), int(pages_needed[l, s, h])
                bt[l, s, h, :npg] = ids[at:at + npg]
                at += npg
                vals = rng.integers(1, 255, (n, W)).astype(np.uint8)
                spans[l, s, h] = vals
                for r in range(n):
                    row = bt[l, s, h, r // P] * P + r % P
                    arenas_k[l][row] = vals[r]
                    arenas_v[l][row] = 255 - vals[r]
    slots, caps = [2, 0], [80, 75]
    new_k, new_v, bases = ock.spans_from_pages(arenas_k, arenas_v, bt, live, slots, caps, P)
    for i, (s, cap) in enumerate(zip(slots, caps)):
        for l in range(L):
            for h in range(H):
                b, n = int(bases[i][l, h]), int(live[l, s, h])
                assert np.array_equal(new_k[l][b:b + n], spans[l, s, h])
                assert np.array_equal(new_v[l][b:b + n], 255 - spans[l, s, h])
                assert not new_k[l][b + n:b + cap].any()
    assert bases[1][0, 0] == caps[0] * H
