"""Paged compact KV on the GPU (16-row FP8 pages, device page pool) against the
span oracle (oracle/compact_kv.py).

The reference has no pages, so parity is defined on ranks: for every (layer,
seq, kv head) the live count, the token position and evict flag at rank r,
and the K / V bytes at rank r gathered through the block table must equal the
oracle's span element r (bit-exact) -- after the prefill pack, after every
decode step (expiry policy, append, decision recording) and after frees.  The
block tables themselves are pinned by invariants (tests/paged_invariants.py):
ceil(live / 16) pages per span, no page twice, held + free = the whole pool,
freed pages back on the stack.  Attention must not see the layout: the paged
kernel over the pages equals the span kernel over the oracle's spans, and a
random relabelling of the pages leaves it bit-identical.
"""
import os

import numpy as np
import pytest
import torch

from helpers import from_values, require_gpu, storage_of, to_torch
from oracle import attention as oatt
from oracle import compact_kv as ock
from oracle import numerics
from paged_invariants import PAGE, check_page_invariants, gather_span_rows

pytestmark = pytest.mark.gpu

FP8 = numerics.DT_FP8


def _setup(lens, *, L=2, hkv=4, d=64, max_tokens=48, pool_tokens=1 << 14, mml=2048, seed=7):
    from fastdms_amd.engine.paged_kv import PagedCompactKVManager
    from fastdms_amd.engine.sequence import Sequence
    from fastdms_amd.sampling_params import SamplingParams
    prod = PagedCompactKVManager(num_layers=L, num_kv_heads=hkv, capacity_tokens=pool_tokens, max_model_len=mml,
                                 device="cuda", head_dim=d, compact_dtype=torch.float8_e4m3fn,
                                 max_active_seqs=len(lens) + 2)
    orc = ock.OracleCompactKVManager(L, hkv, 1 << 17, mml, head_dim=d, dtype_code=FP8)
    seqs = [Sequence(list(range(n)), SamplingParams(max_tokens=max_tokens)) for n in lens]
    return prod, orc, seqs, np.random.default_rng(seed)


def _prefill(prod, orc, seqs, rng, *, hq=8, window=31, evict_p=0.8):
    L, hkv, d = prod.num_layers, prod.num_kv_heads, prod.head_dim
    for s in seqs:
        prod.allocate(s)
        orc.allocate(s.seq_id, s.num_prompt_tokens, s.max_tokens)
    prod.begin_prefill()
    lens = [s.num_prompt_tokens for s in seqs]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cu_d = torch.from_numpy(cu).cuda()
    ids = [s.seq_id for s in seqs]
    for layer in range(L):
        t = int(cu[-1])
        k = numerics.cast(rng.standard_normal((t, hkv, d)).astype(np.float32) * 2, numerics.DT_BF16)
        v = numerics.cast(rng.standard_normal((t, hkv, d)).astype(np.float32) * 2, numerics.DT_BF16)
        ev = rng.random((t, hkv)) < evict_p
        prod.streaming_pack_layer(layer_id=layer, k=from_values(k, numerics.DT_BF16),
                                  v=from_values(v, numerics.DT_BF16), evict_mask=torch.from_numpy(ev).cuda(),
                                  cu_seqlens_q=cu_d, seq_ids=ids, window_size=window, cu_seqlens_host=cu.tolist())
        orc.streaming_pack_layer(layer_id=layer, k=k, v=v, evict_mask=ev, cu_seqlens_q=cu, seq_ids=ids,
                                 window_size=window)
    prod.stage_prefill_check(ids)
    torch.cuda.synchronize()
    prod.finish_prefill_check()


def _compare(prod, orc, seqs, what):
    """Rank-level parity of every span plus the pool invariants."""
    torch.cuda.synchronize()
    check_page_invariants(prod)
    arenas = [(storage_of(prod.compact_k_per_layer[l]), storage_of(prod.compact_v_per_layer[l]))
              for l in range(prod.num_layers)]
    for s in seqs:
        ps, os_ = prod.seq_states[s.seq_id], orc.seq_states[s.seq_id]
        live = ps.live_counts.cpu().numpy()
        assert np.array_equal(live, os_.live_counts), f"{what}: live counts of seq {s.seq_id}"
        pos, ev = ps.token_positions.cpu().numpy(), ps.evict_mask.cpu().numpy()
        for l in range(prod.num_layers):
            for h in range(prod.num_kv_heads):
                n = int(live[l, h])
                assert np.array_equal(pos[l, h, :n], os_.token_positions[l, h, :n]), f"{what}: positions {l, h}"
                assert np.array_equal(ev[l, h, :n], os_.evict_mask[l, h, :n]), f"{what}: evict flags {l, h}"
                b0 = int(os_.base_offsets[l, h])
                for arena, oarena in zip(arenas[l], (orc.compact_k_per_layer[l], orc.compact_v_per_layer[l])):
                    got = gather_span_rows(prod, l, ps.active_slot, h, arena)
                    assert np.array_equal(got, oarena[b0:b0 + n]), f"{what}: K/V bytes of span {l, s.seq_id, h}"


def test_paged_prefill_pack_matches_the_span_oracle():
    """Ragged batch incl. a 1-token prompt and a 1024-token prompt (4 chunks):
    live counts, positions, evict flags and page contents bit-exact, pages
    popped on the device with no host sync in the layer loop."""
    require_gpu()
    prod, orc, seqs, rng = _setup([300, 1, 541, 1024, 257])
    syncs = prod.page_syncs
    _prefill(prod, orc, seqs, rng)
    assert prod.page_syncs == syncs
    _compare(prod, orc, seqs, "prefill")
    used = check_page_invariants(prod)["pages_used"]
    want = [sum(-(-int(n) // PAGE) for st in orc.seq_states.values() for n in st.live_counts[l])
            for l in range(prod.num_layers)]
    assert used == want


@pytest.mark.parametrize("interval", [None, "1"])
def test_paged_decode_steps_match_the_span_oracle(monkeypatch, interval):
    """40 decode steps of 5 sequences: the expiry policy (first-step exact
    pass, then skip / windowed full passes, or incremental every step), the
    page-popping append, decision recording; the spans, metadata and pool
    after every step equal the oracle's."""
    require_gpu()
    from fastdms_amd.layers.compact_attention import store_compact_kvcache
    if interval is not None:
        monkeypatch.setenv("FASTDMS_DMS_EXPIRY_TRITON", "1")
        monkeypatch.setenv("FASTDMS_DMS_EXPIRY_INTERVAL", interval)
    window = 31
    prod, orc, seqs, rng = _setup([300, 40, 541, 700, 257], seed=11)
    _prefill(prod, orc, seqs, rng, window=window)
    L, H, d = prod.num_layers, prod.num_kv_heads, prod.head_dim
    ids = [s.seq_id for s in seqs]
    mode = os.environ.get("FASTDMS_DMS_EXPIRY_TRITON", "auto")
    for step in range(40):
        cur = [s.num_prompt_tokens + step for s in seqs]
        prod.pack_active_slots([prod.seq_states[i] for i in ids])
        prod.apply_dms_evictions(seqs, cur, window_size=window, sync_stats=False)
        orc.apply_dms_evictions(ids, cur, window_size=window, triton_mode=mode, interval_env=interval)
        bt, live, slot, _ = prod.prepare_decode_metadata(seqs)
        _, _, oslot, _ = orc.prepare_decode_metadata(ids)
        key = numerics.cast(rng.standard_normal((L, len(seqs), H, d)).astype(np.float32) * 2, numerics.DT_BF16)
        val = numerics.cast(rng.standard_normal((L, len(seqs), H, d)).astype(np.float32) * 2, numerics.DT_BF16)
        for l in range(L):
            store_compact_kvcache(from_values(key[l], numerics.DT_BF16), from_values(val[l], numerics.DT_BF16),
                                  prod.compact_k_per_layer[l], prod.compact_v_per_layer[l], slot[l])
            oatt.store_compact_kvcache(key[l], val[l], orc.compact_k_per_layer[l], orc.compact_v_per_layer[l],
                                       oslot[l], FP8)
        evict = rng.random((L, len(seqs), H)) < 0.6
        prod.record_appended_dms_decisions(seqs, cur, torch.from_numpy(evict).cuda(), sync_stats=False)
        orc.record_appended_dms_decisions(ids, cur, evict)
        _compare(prod, orc, seqs, f"decode step {step}")
    prod.check_overflow()


def test_paged_attention_sees_ranks_not_pages():
    """The paged attention kernel over the pool equals the span kernel over
    the oracle's spans (same inputs in the same rank order), and relabelling
    the pages with a random permutation (rows moved, tables rewritten) leaves
    the output bit-identical."""
    require_gpu()
    from fastdms_amd.layers.compact_attention import compact_decode_attention, compact_decode_attention_paged
    prod, orc, seqs, rng = _setup([300, 77, 541, 1024, 257], seed=5)
    _prefill(prod, orc, seqs, rng)
    torch.cuda.synchronize()
    B, hq, d = len(seqs), 8, prod.head_dim
    slots = [prod.seq_states[s.seq_id].active_slot for s in seqs]
    q = from_values(numerics.cast(rng.standard_normal((B, hq, d)).astype(np.float32), numerics.DT_BF16),
                    numerics.DT_BF16)
    for l in range(prod.num_layers):
        bt = prod.block_tables[l, slots].contiguous()
        live = prod.layer_major_live_counts[l, slots].contiguous()
        max_live = int(live.max())
        ck, cv = prod.compact_k_per_layer[l], prod.compact_v_per_layer[l]
        out = compact_decode_attention_paged(q, ck, cv, bt, live, PAGE, max_live_count=max_live)
        base = torch.from_numpy(np.stack([orc.seq_states[s.seq_id].base_offsets[l] for s in seqs])).cuda()
        span = compact_decode_attention(q, to_torch(orc.compact_k_per_layer[l], FP8),
                                        to_torch(orc.compact_v_per_layer[l], FP8), base, live,
                                        max_live_count=max_live)
        assert torch.equal(out, span), f"layer {l}: paged attention differs from the span kernel"
        perm = torch.from_numpy(rng.permutation(prod.num_pages).astype(np.int64)).cuda()
        rows = (perm[:, None] * PAGE + torch.arange(PAGE, device="cuda")[None, :]).reshape(-1)
        ck2, cv2 = torch.empty_like(ck), torch.empty_like(cv)
        ck2[rows] = ck[:prod.num_pages * PAGE]
        cv2[rows] = cv[:prod.num_pages * PAGE]
        bt2 = torch.where(bt >= 0, perm[bt.clamp(min=0).long()].to(torch.int32), bt)
        out2 = compact_decode_attention_paged(q, ck2, cv2, bt2, live, PAGE, max_live_count=max_live)
        assert torch.equal(out, out2), f"layer {l}: a page relabelling changed the attention output"


def test_freed_pages_return_to_the_pool():
    """Freeing sequences pushes every page back (no sync); the freed pages
    are reused by the next admission; the whole pool is free at the end."""
    require_gpu()
    prod, orc, seqs, rng = _setup([300, 1, 541, 1024, 257])
    _prefill(prod, orc, seqs, rng)
    torch.cuda.synchronize()
    before = check_page_invariants(prod)["pages_used"]
    prod.free(seqs[2].seq_id)
    prod.free(seqs[0].seq_id)
    after = check_page_invariants(prod)["pages_used"]
    freed = [sum(-(-int(n) // PAGE) for n in orc.seq_states[s.seq_id].live_counts[l]) for l in range(2)
             for s in (seqs[0], seqs[2])]
    assert [b - a for b, a in zip(before, after)] == [freed[0] + freed[1], freed[2] + freed[3]]
    from fastdms_amd.engine.sequence import Sequence
    from fastdms_amd.sampling_params import SamplingParams
    again = [Sequence(list(range(900)), SamplingParams(max_tokens=8))]
    orc2 = ock.OracleCompactKVManager(2, prod.num_kv_heads, 1 << 17, 2048, head_dim=prod.head_dim, dtype_code=FP8)
    _prefill(prod, orc2, again, rng)
    _compare(prod, orc2, again, "after reuse")
    for s in [seqs[1], seqs[3], seqs[4], again[0]]:
        prod.free(s.seq_id)
    torch.cuda.synchronize()
    check_page_invariants(prod)
    assert prod.page_top.tolist() == [prod.num_pages] * prod.num_layers
    assert not prod.seq_states and prod.pages_bound() == 0


def test_a_prefill_that_does_not_fit_is_refused_and_leaves_the_pool_whole():
    """A pool too small for the batch: the pack kernels take no page beyond
    the budget, the failed spans are left empty, the host raises
    CompactCapacityExhausted after the step, and freeing the batch restores
    the whole pool (the engine then defers or preempts)."""
    require_gpu()
    from fastdms_amd.engine.compact_kv import CompactCapacityExhausted
    prod, orc, seqs, rng = _setup([1024, 900, 800], pool_tokens=60 * PAGE, max_tokens=8)
    with pytest.raises(CompactCapacityExhausted):
        _prefill(prod, orc, seqs, rng, evict_p=0.2)
    torch.cuda.synchronize()
    check_page_invariants(prod)
    for s in seqs:
        prod.free(s.seq_id)
    torch.cuda.synchronize()
    assert prod.page_top.tolist() == [prod.num_pages] * prod.num_layers
    assert int(prod.overflow.item()) == 0
