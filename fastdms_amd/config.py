"""Engine configuration (mirror of fastdms/config.py:42-107).

``model`` names a synthetic preset ("llama-3.2-1b", "qwen3-8b", "tiny-llama",
"tiny-qwen3"), a ``ModelConfig`` or a dict of its fields: this build has no
checkpoint loader, so weights are seeded random values (``seed``).  The DMS /
compact-KV fields keep the reference's names and meaning; the compact-DMS path
is the only KV mode here (``compact_kv_retention_mode == "dms"``).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .layers.quant_env import env_bool as _env_flag

_KV_CACHE_DTYPES = {"auto": None, "float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32,
                    "float8_e4m3fn": torch.float8_e4m3fn}


@dataclass(slots=True)
class Config:
    model: object = "llama-3.2-1b"
    max_num_batched_tokens: int = 16384
    max_num_seqs: int = 512
    max_model_len: int = 4096
    gpu_memory_utilization: float = 0.9
    tensor_parallel_size: int = 1
    enforce_eager: bool = False
    hf_config: object = None
    eos: int = -1
    kvcache_block_size: int = 256
    kv_cache_dtype: str = "float8_e4m3fn"
    num_kvcache_blocks: int = 0
    compact_kv_enabled: bool = True
    compact_kv_capacity_tokens: int = 0
    compact_kv_retention_mode: str = "dms"
    compact_kv_retention_stride: int = 1
    compact_kv_retention_recent_tokens: int = 0
    dms_metadata_path: str | None = None
    dms_window_size: int | None = None
    dms_alpha_scale: float | None = None
    dms_alpha_offset: float | None = None
    num_page_override: int | None = None
    token_pool_tokens: int | None = None
    compact_kv_budget_bytes: int | None = None
    compact_kv_target_live_tokens_per_seq: int | None = None
    compact_kv_layer_major_metadata: bool = True
    # Where the compact K/V rows live (no reference counterpart; the reference
    # stores flat spans from a host first-fit allocator, compact_kv.py:697-857):
    # "paged" = 16-row pages from a device-resident free-page pool (pack,
    # decode append, expiry and free allocate on the device, no host sync per
    # prefill layer); "span" = the reference's flat spans
    compact_kv_layout: str = "paged"
    seed: int = 0
    dms_survive_fraction: float = 0.125
    compact_decode_cudagraph: bool = True
    # Per-(layer, kv head) FP8 KV scales (no reference counterpart; the
    # reference stores K/V with a bare cast): "unit" = none (the reference's
    # numerics), "calibrate" = set from each layer's first prefill (amax / 224)
    compact_kv_fp8_scales: str = "unit"
    # What happens when a prefill's compact spans do not fit (the reference
    # raises from the allocator, compact_kv.py:715-718): "defer" puts the
    # prefill back at the head of the queue until a running sequence finishes;
    # "preempt" frees the most recently admitted running sequences (re-admitted
    # later by re-prefilling their tokens) until it fits.
    compact_admission: str = "defer"
    # Decode rows reserved per compact span after the pack.  None reserves
    # max_tokens (the reference's sizing: decode never runs out); a smaller
    # number overcommits the KV memory: a full span grows during decode and,
    # when no range is free, the youngest running sequence is preempted.
    compact_decode_reserve_tokens: int | None = None
    # LM-head GEMV fused with the greedy argmax (no logits materialised);
    # FASTDMS_GREEDY_FUSED_ARGMAX, default on (embed_head.py:62-63)
    fused_greedy_head: bool = field(default_factory=lambda: _env_flag("FASTDMS_GREEDY_FUSED_ARGMAX", True))

    def __post_init__(self):
        from .models.synthetic import model_config
        assert self.kvcache_block_size % 256 == 0
        if self.compact_kv_layout not in ("paged", "span"):
            raise ValueError(f"compact_kv_layout must be 'paged' or 'span', got {self.compact_kv_layout!r}")
        if self.compact_admission not in ("defer", "preempt"):
            raise ValueError(f"compact_admission must be 'defer' or 'preempt', got {self.compact_admission!r}")
        if self.compact_decode_reserve_tokens is not None and (
                self.compact_admission != "preempt" or self.compact_decode_reserve_tokens < 1):
            raise ValueError("compact_decode_reserve_tokens needs compact_admission='preempt' and a positive value")
        if self.tensor_parallel_size != 1:
            raise ValueError("this build runs on one GPU (tensor_parallel_size must be 1)")
        assert self.kv_cache_dtype in _KV_CACHE_DTYPES, f"kv_cache_dtype must be one of {sorted(_KV_CACHE_DTYPES)}"
        if not self.compact_kv_enabled or self.compact_kv_retention_mode != "dms":
            raise ValueError("this build implements the compact-DMS KV path only "
                             "(compact_kv_enabled=True, compact_kv_retention_mode='dms')")
        if self.dms_window_size is not None:
            assert self.dms_window_size >= 0
        if self.dms_alpha_scale is not None:
            assert self.dms_alpha_scale != 0.0
        self.hf_config = model_config(self.model)
        self.max_model_len = min(self.max_model_len, self.hf_config.max_position_embeddings)

    def resolve_kv_cache_dtype(self) -> torch.dtype:
        dtype = _KV_CACHE_DTYPES[self.kv_cache_dtype]
        return torch.bfloat16 if dtype is None else dtype
