"""Host-side launch plan of the matrix-core decode attention (CPU only): the
Python mirror of the kernel's launch shape must give a split bound that
covers every pair, since the kernel clamps a pair's split count to it.  The
kernel's rule (fdms_compact_decode_attention / fdms_fused_decode_attention*):
a pair of at most split_rows live rows is one workgroup; a longer one takes
ceil(live / h) splits, h = split_rows / 2 at head_dim 64 with at most 128
(seq, kv head) pairs, else split_rows."""
import pytest
import torch

from fastdms_amd.layers import compact_attention as ca


def _kernel_splits(live, split_rows, head_dim, pairs):
    rows = -(-split_rows // 64) * 64
    h = max(64, -(-((rows // 2) if head_dim == 64 and pairs <= 128 else rows) // 64) * 64)
    return 1 if live <= rows else -(-live // h)


@pytest.mark.parametrize("head_dim,fused", [(64, True), (64, False), (128, True), (128, False)])
@pytest.mark.parametrize("pairs", [8, 16, 17, 64, 128, 129, 1024])
def test_split_bound_covers_every_pair(monkeypatch, head_dim, fused, pairs):
    for var in ("FASTDMS_AMD_ATTN_WAVES", "FASTDMS_AMD_ATTN_SPLIT_DIV", "FASTDMS_AMD_ATTN_SPLIT_ROWS"):
        monkeypatch.delenv(var, raising=False)
    waves = ca.attention_waves(head_dim, fused, pairs)
    assert waves == (8 if fused and (head_dim == 128 or 16 < pairs <= 128) else 4)
    for max_live in (1, 63, 64, 512, 1024, 1025, 2700, 8448, 65536):
        splits, rows = ca.attention_split_plan(torch.device("cpu"), pairs, max_live, True, waves=waves,
                                               head_dim=head_dim)
        assert 1 <= splits <= 64
        needed = max(_kernel_splits(live, rows, head_dim, pairs) for live in range(max(1, max_live - 130),
                                                                                max_live + 1))
        # the bound covers every pair up to max_live unless the 64-split cap binds
        assert splits >= min(needed, 64), (max_live, splits, needed, rows)


def test_tuning_switches_are_mirrored(monkeypatch):
    monkeypatch.setenv("FASTDMS_AMD_ATTN_WAVES", "4")
    assert ca.attention_waves(64, True, 64) == 4
    assert ca.attention_waves(128, True, 64) == 8  # the fused preprocess needs 2.5 * head_dim threads
    monkeypatch.setenv("FASTDMS_AMD_ATTN_SPLIT_DIV", "1")
    assert ca.mfma_heavy_rows(1024, 64, 64) == 1024
    monkeypatch.setenv("FASTDMS_AMD_ATTN_SPLIT_DIV", "4")
    assert ca.mfma_heavy_rows(1024, 64, 64) == 256
    monkeypatch.delenv("FASTDMS_AMD_ATTN_SPLIT_DIV")
    assert ca.mfma_heavy_rows(1024, 64, 64) == 512 and ca.mfma_heavy_rows(1024, 128, 64) == 1024
    assert ca.mfma_heavy_rows(1024, 64, 129) == 1024
