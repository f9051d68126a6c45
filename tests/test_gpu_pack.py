"""A4/A5/A6/A7: streaming prefill pack on the GPU vs the oracle (bit-exact
ranks, positions, evict flags, live counts, base offsets and arena bytes)."""
import numpy as np
import pytest
import torch

from helpers import TORCH_DTYPE, from_values, require_gpu, storage_of, to_torch
from oracle import compact_kv as ock
from oracle import numerics

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("in_code,out_code", [(numerics.DT_F32, numerics.DT_F32), (numerics.DT_FP8, numerics.DT_FP8),
                                              (numerics.DT_BF16, numerics.DT_FP8), (numerics.DT_F32, numerics.DT_FP8),
                                              (numerics.DT_BF16, numerics.DT_BF16)])
def test_fused_rank_pack_matches_oracle(in_code, out_code):
    """The reference's fused-rank case (test_compact_kv.py:1180-1241): 541 tokens, W=31."""
    require_gpu()
    from fastdms_amd.engine.compact_kv import _streaming_pack_fused_rank_prepare, _streaming_pack_rank_scatter_hip
    rng = np.random.default_rng(29)
    seq_len, window, h, d = 541, 31, 3, 16
    k = numerics.cast(rng.standard_normal((seq_len, h, d)).astype(np.float32) * 3, in_code)
    v = numerics.cast(rng.standard_normal((seq_len, h, d)).astype(np.float32) * 3, in_code)
    ev = rng.random((seq_len, h)) > 0.5
    base = np.array([0, 640, 1280], dtype=np.int32)
    sd = numerics.storage_dtype(out_code)
    ck = np.zeros((1920, d), sd)
    cv = np.zeros((1920, d), sd)
    pos = np.full((h, 700), -1, np.int32)
    evm = np.zeros((h, 700), bool)
    live = ock.streaming_pack_rank_scatter(k=k, v=v, seq_evict=ev, compact_k=ck, compact_v=cv, token_positions=pos,
                                           evict_mask=evm, base_offsets=base, start=0, seq_len=seq_len,
                                           window_size=window, dtype_code=out_code)
    _, offs = ock.streaming_pack_fused_rank_prepare(ev, seq_len, window)

    kd, vd = from_values(k, in_code), from_values(v, in_code)
    evd = torch.from_numpy(ev).cuda()
    live_d, offs_d = _streaming_pack_fused_rank_prepare(seq_evict=evd, seq_len=seq_len, window_size=window)
    ckd = torch.zeros((1920, d), device="cuda", dtype=TORCH_DTYPE[out_code])
    cvd = torch.zeros_like(ckd)
    posd = torch.full((h, 700), -1, device="cuda", dtype=torch.int32)
    evmd = torch.zeros((h, 700), device="cuda", dtype=torch.bool)
    _streaming_pack_rank_scatter_hip(k=kd, v=vd, seq_evict=evd, block_offsets=offs_d, compact_k=ckd, compact_v=cvd,
                                     token_positions=posd, evict_mask=evmd,
                                     base_offsets=torch.from_numpy(base).cuda(), start=0, seq_len=seq_len,
                                     window_size=window)
    torch.cuda.synchronize()
    assert live_d.cpu().tolist() == live.tolist()
    assert np.array_equal(offs_d.cpu().numpy(), offs)
    assert np.array_equal(storage_of(ckd), ck)
    assert np.array_equal(storage_of(cvd), cv)
    assert np.array_equal(posd.cpu().numpy(), pos)
    assert np.array_equal(evmd.cpu().numpy(), evm)


@pytest.mark.parametrize("code", [numerics.DT_F32, numerics.DT_FP8])
def test_precomputed_rank_scatter_matches_oracle(code):
    """The reference's scatter case (test_compact_kv.py:1123-1177): 37 tokens."""
    require_gpu()
    from fastdms_amd.engine.compact_kv import _streaming_pack_scatter_hip
    rng = np.random.default_rng(23)
    seq_len, h, d = 37, 3, 16
    k = numerics.cast(rng.standard_normal((seq_len, h, d)).astype(np.float32), code)
    v = numerics.cast(rng.standard_normal((seq_len, h, d)).astype(np.float32), code)
    keep = rng.random((seq_len, h)) > 0.35
    keep[-1] = True
    rank = np.cumsum(keep, axis=0) - 1
    ev = rng.random((seq_len, h)) > 0.5
    base = np.array([0, 48, 96], dtype=np.int32)
    sd = numerics.storage_dtype(code)
    ck = np.zeros((144, d), sd)
    cv = np.zeros((144, d), sd)
    pos = np.full((h, 64), -1, np.int32)
    evm = np.zeros((h, 64), bool)
    ock.streaming_pack_scatter(k=k, v=v, keep=keep, rank=rank, seq_evict=ev, compact_k=ck, compact_v=cv,
                               token_positions=pos, evict_mask=evm, base_offsets=base, start=0, seq_len=seq_len,
                               dtype_code=code)
    ckd = torch.zeros((144, d), device="cuda", dtype=TORCH_DTYPE[code])
    cvd = torch.zeros_like(ckd)
    posd = torch.full((h, 64), -1, device="cuda", dtype=torch.int32)
    evmd = torch.zeros((h, 64), device="cuda", dtype=torch.bool)
    _streaming_pack_scatter_hip(k=from_values(k, code), v=from_values(v, code), keep=torch.from_numpy(keep).cuda(),
                                rank=torch.from_numpy(rank.astype(np.int32)).cuda(),
                                seq_evict=torch.from_numpy(ev).cuda(), compact_k=ckd, compact_v=cvd,
                                token_positions=posd, evict_mask=evmd, base_offsets=torch.from_numpy(base).cuda(),
                                start=0, seq_len=seq_len)
    torch.cuda.synchronize()
    assert np.array_equal(storage_of(ckd), ck) and np.array_equal(storage_of(cvd), cv)
    assert np.array_equal(posd.cpu().numpy(), pos) and np.array_equal(evmd.cpu().numpy(), evm)


def _make_batch(rng, lens, hq, hkv, d, evict_p):
    t = sum(lens)
    qkv = numerics.cast(rng.standard_normal((t, (hq + 2 * hkv) * d)).astype(np.float32), numerics.DT_BF16)
    ev = rng.random((t, hkv)) < evict_p
    return qkv, ev


@pytest.mark.parametrize("layer_major", [True, False])
def test_manager_streaming_pack_ragged_batch_matches_oracle(layer_major):
    require_gpu()
    from fastdms_amd.engine.compact_kv import CompactKVManager
    from fastdms_amd.engine.sequence import Sequence
    from fastdms_amd.sampling_params import SamplingParams
    rng = np.random.default_rng(7)
    L, hq, hkv, d, window = 2, 8, 4, 64, 31
    lens = [300, 1, 541, 1024, 257]
    max_tokens = 16
    cap = 4096
    prod = CompactKVManager(num_layers=L, num_kv_heads=hkv, capacity_tokens=cap, max_model_len=2048, device="cuda",
                            head_dim=d, compact_dtype=torch.float8_e4m3fn, per_layer_storage=True,
                            layer_major_metadata=layer_major, max_active_seqs=8)
    orc = ock.OracleCompactKVManager(L, hkv, cap, 2048, head_dim=d, dtype_code=numerics.DT_FP8)
    seqs = [Sequence(list(range(n)), SamplingParams(max_tokens=max_tokens)) for n in lens]
    for s in seqs:
        prod.allocate(s)
        orc.allocate(s.seq_id, s.num_prompt_tokens, s.max_tokens)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    cu_d = torch.from_numpy(cu).cuda()
    ids = [s.seq_id for s in seqs]
    for layer in range(L):
        qkv, ev = _make_batch(rng, lens, hq, hkv, d, 0.8)
        qkv_d = from_values(qkv, numerics.DT_BF16)
        k_d = qkv_d[:, hq * d:(hq + hkv) * d].view(-1, hkv, d)
        v_d = qkv_d[:, (hq + hkv) * d:].view(-1, hkv, d)
        prod.streaming_pack_layer(layer_id=layer, k=k_d, v=v_d, evict_mask=torch.from_numpy(ev).cuda(),
                                  cu_seqlens_q=cu_d, seq_ids=ids, window_size=window)
        k = qkv[:, hq * d:(hq + hkv) * d].reshape(-1, hkv, d)
        v = qkv[:, (hq + hkv) * d:].reshape(-1, hkv, d)
        orc.streaming_pack_layer(layer_id=layer, k=k, v=v, evict_mask=ev, cu_seqlens_q=cu, seq_ids=ids,
                                 window_size=window)
    torch.cuda.synchronize()
    assert prod.free_ranges_per_layer == orc.free_ranges_per_layer
    for s in seqs:
        ps, os_ = prod.seq_states[s.seq_id], orc.seq_states[s.seq_id]
        assert np.array_equal(ps.live_counts.cpu().numpy(), os_.live_counts)
        assert np.array_equal(ps.base_offsets.cpu().numpy(), os_.base_offsets)
        assert np.array_equal(ps.range_capacity.cpu().numpy(), os_.range_capacity)
        assert np.array_equal(ps.token_positions.cpu().numpy(), os_.token_positions)
        assert np.array_equal(ps.evict_mask.cpu().numpy(), os_.evict_mask)
        for layer in range(L):
            ckp = storage_of(prod.compact_k_per_layer[layer])
            cvp = storage_of(prod.compact_v_per_layer[layer])
            for h in range(hkv):
                b0, n = int(os_.base_offsets[layer, h]), int(os_.live_counts[layer, h])
                assert np.array_equal(ckp[b0:b0 + n], orc.compact_k_per_layer[layer][b0:b0 + n])
                assert np.array_equal(cvp[b0:b0 + n], orc.compact_v_per_layer[layer][b0:b0 + n])
    # arenas grew to a 256-multiple high-water mark like the reference
    for layer in range(L):
        assert prod.compact_k_per_layer[layer].shape[0] == orc.compact_k_per_layer[layer].shape[0]
