"""Model runner for the compact-DMS path (mirror of fastdms/engine/model_runner.py,
single GPU).

Prefill (eager): token batch -> per layer DMS capture, RoPE, streaming pack of
the prompt into compact FP8 spans, dense causal attention -> greedy token of
each sequence's last position.

Decode: the host decides the expiry action (the reference's policy, which
depends only on positions the host knows) and launches it; the rest of the
step — append-slot preparation, the whole forward, LM head + argmax and
recording of the appended tokens' DMS decisions — is captured once per batch
composition as a HIP graph and replayed, so a step costs one graph launch
and one device->host copy of the token ids.
"""
from __future__ import annotations

import os

import torch

from .. import _native as nat
from ..config import Config
from ..layers.compact_attention import DecodePlan, decode_plan_enabled, reserve_attention_workspace
from ..layers import quant_env as qe
from ..layers.linear import convert_linear_modules_to_fp8, reserve_linear_workspace
from ..models.synthetic import build_synthetic_model
from ..utils.context import get_context, reset_context, set_context
from .chunked_prefill import ChunkPlan, PromptStage
from .compact_kv import CompactKVManager
from .paged_kv import PagedCompactKVManager
from .dms import DMSMetadata, load_dms_metadata
from .sequence import Sequence, SequenceStatus


def decode_lookahead_enabled() -> bool:
    """FASTDMS_AMD_DECODE_LOOKAHEAD (default on): launch a certain next decode
    step before reading back the current one's ids."""
    return os.environ.get("FASTDMS_AMD_DECODE_LOOKAHEAD", "1").strip().lower() not in ("0", "false", "no", "off")


def compact_greedy_fast_loop_enabled() -> bool:
    """FASTDMS_COMPACT_GREEDY_FAST_LOOP (default on), model_runner.py:30-32."""
    return os.environ.get("FASTDMS_COMPACT_GREEDY_FAST_LOOP", "1").strip().lower() not in ("0", "false", "no", "off")


def convert_model_weights(model) -> tuple[int, bool, bool]:
    """FP8 / INT4 weights from the environment, as model_runner.py:72-113:
    FASTDMS_FP8_WEIGHTS converts the linear layers in scope, FASTDMS_FP8_LM_HEAD
    (or a head scope) the LM head, and then FASTDMS_FP8_EMBEDDING the token
    table (shared with the head's FP8 rows under
    FASTDMS_FP8_EMBEDDING_SHARE_LM_HEAD).  Returns (converted linears, FP8
    head, FP8 embedding)."""
    if not qe.fp8_weights_enabled():
        return 0, False, False
    converted = convert_linear_modules_to_fp8(model)
    lm_head = model.lm_head
    embed = model.model.embed_tokens
    fp8_embedding = qe.env_bool("FASTDMS_FP8_EMBEDDING", True)
    fp8_head = False
    if qe.fp8_lm_head_enabled():
        tied = (fp8_embedding and embed.weight.untyped_storage().data_ptr()
                == lm_head.weight.untyped_storage().data_ptr())
        keep = qe.fp8_keep_bf16_lm_head_weight()
        if tied and not qe.env_bool("FASTDMS_FP8_KEEP_BF16_EMBEDDING", False):
            keep = False
        lm_head.quantize_weight_to_fp8(keep_bf16_weight=keep)
        fp8_head = True
    if fp8_embedding:
        keep_embed = qe.env_bool("FASTDMS_FP8_KEEP_BF16_EMBEDDING", False)
        if qe.env_bool("FASTDMS_FP8_EMBEDDING_SHARE_LM_HEAD", False) and fp8_head:
            embed.enable_fp8_embedding_from_lm_head(lm_head, keep_bf16_weight=keep_embed)
        else:
            embed.quantize_embedding_to_fp8(keep_bf16_weight=keep_embed)
    return converted, fp8_head, fp8_embedding


class ModelRunner:

    def __init__(self, config: Config, device: str | torch.device = "cuda"):
        self.config = config
        hf = config.hf_config
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("ModelRunner needs a HIP device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        torch.cuda.set_device(self.device)
        self.model = build_synthetic_model(hf, seed=config.seed, device=self.device,
                                           survive_fraction=config.dms_survive_fraction)
        self.fp8_weight_modules, self.fp8_lm_head, self.fp8_embedding = convert_model_weights(self.model)
        self.dms_metadata = self._dms_metadata()
        self.num_layers = hf.num_hidden_layers
        self.num_kv_heads = hf.num_key_value_heads
        self.head_dim = hf.head_dim
        self.kv_dtype = config.resolve_kv_cache_dtype()
        self.max_num_seqs = config.max_num_seqs
        self.allocate_kv_cache()
        reserve_attention_workspace(self.device, self.max_num_seqs * self.num_kv_heads,
                                    hf.num_attention_heads // hf.num_key_value_heads, hf.head_dim)
        reserve_linear_workspace(self.device, max(hf.vocab_size, 2 * hf.intermediate_size,
                                                  (hf.num_attention_heads + 2 * hf.num_key_value_heads) * hf.head_dim))
        self.evict_buffer = torch.zeros((self.num_layers, self.max_num_seqs, self.num_kv_heads),
                                        device=self.device, dtype=torch.bool)
        self.static_positions = torch.zeros(self.max_num_seqs, device=self.device, dtype=torch.int64)
        self.static_slot = torch.zeros((self.num_layers, self.max_num_seqs, self.num_kv_heads), device=self.device,
                                       dtype=torch.int32)
        # a decode step's input ids and, at its end, its greedy ids (the next
        # step's input when the device feeds it); one more int64 after them
        # holds the page pool's overflow flag, so one copy reads both back
        self._readback = torch.zeros(self.max_num_seqs + 1, device=self.device, dtype=torch.int64)
        self.static_tokens = self._readback[:self.max_num_seqs]
        if self.compact_kv_manager.paged:
            self.compact_kv_manager.bind_overflow(self._readback[self.max_num_seqs:].view(torch.int32)[:1])
        # the paged decode step's attention work plan (static: captured graphs keep its address)
        self.decode_plan = (DecodePlan(self.device, self.num_layers, self.max_num_seqs * self.num_kv_heads,
                                       config.max_model_len + 1, hf.head_dim)
                            if self.compact_kv_manager.paged and decode_plan_enabled(hf.head_dim) else None)
        self.prompt_stages: dict[int, PromptStage] = {}  # long prompts between their chunks
        self.pinned_ids = torch.zeros(self.max_num_seqs, dtype=torch.int64, pin_memory=True)
        self.pinned_pos = torch.zeros(self.max_num_seqs, dtype=torch.int64, pin_memory=True)
        # decode lookahead (run_decode): two pinned sets each for the sampled
        # ids read back and the positions sent, alternating per staged step
        self._tok_ring = [torch.zeros(self.max_num_seqs + 1, dtype=torch.int64, pin_memory=True) for _ in range(2)]
        self._pos_ring = [torch.zeros(self.max_num_seqs, dtype=torch.int64, pin_memory=True) for _ in range(2)]
        self._ring = 0
        self._lookahead: dict | None = None  # the decode step in flight ahead of the host
        self.graphs: dict[tuple, tuple] = {}
        self.graph_pool = None
        self._warm: set = set()
        self.last_compact_prefill_stats: dict = {}
        self.last_dms_decode_stats: list = []
        self.last_decode_seq_ids: list[int] = []
        self.compact_live_tokens_peak = 0
        fp8 = getattr(torch, "float8_e4m3fn", None)
        group = hf.num_attention_heads // hf.num_key_value_heads
        self._static_attention_bound = (
            os.environ.get("FASTDMS_AMD_ATTN_MFMA", "1").strip() != "0"
            and os.environ.get("FASTDMS_AMD_ATTN_GENERIC", "0").strip() != "1"
            and self.kv_dtype == fp8 and group <= 4 and hf.head_dim in (64, 128))

    # -- setup -----------------------------------------------------------------
    def _dms_metadata(self) -> DMSMetadata:
        """Config overrides on top of the loaded/default metadata (model_runner.py:133-146)."""
        c = self.config
        if c.dms_metadata_path:
            base = load_dms_metadata(".", c.dms_metadata_path)
        else:
            base = DMSMetadata(model_path=str(c.model), source_path="", source_kind="synthetic_defaults",
                               packaged_metadata_found=False, window_size=256, alpha_scale=100.0, alpha_offset=5.0)
        return DMSMetadata(model_path=base.model_path, source_path=base.source_path, source_kind=base.source_kind,
                           packaged_metadata_found=base.packaged_metadata_found,
                           window_size=c.dms_window_size if c.dms_window_size is not None else base.window_size,
                           alpha_scale=c.dms_alpha_scale if c.dms_alpha_scale is not None else base.alpha_scale,
                           alpha_offset=c.dms_alpha_offset if c.dms_alpha_offset is not None else base.alpha_offset,
                           target_cr=base.target_cr, context_len=base.context_len,
                           compression_mode=base.compression_mode)

    def allocate_kv_cache(self) -> None:
        """Per-layer compact arenas, allocated up front so their addresses never
        change (captured decode graphs stay valid).  Capacity per layer:
        compact_kv_capacity_tokens, else compact_kv_budget_bytes, else the
        worst case max_num_seqs * kv_heads * max_model_len."""
        c = self.config
        itemsize = torch.empty((), dtype=self.kv_dtype).element_size()
        if c.compact_kv_capacity_tokens > 0:
            cap = int(c.compact_kv_capacity_tokens)
        elif c.compact_kv_budget_bytes is not None:
            cap = int(c.compact_kv_budget_bytes) // (2 * self.num_layers * self.head_dim * itemsize)
        else:
            cap = self.max_num_seqs * self.num_kv_heads * c.max_model_len
        if cap <= 0:
            raise ValueError("compact KV capacity must be positive")
        if c.compact_kv_layout == "paged":
            self.compact_kv_manager = PagedCompactKVManager(
                num_layers=self.num_layers, num_kv_heads=self.num_kv_heads, capacity_tokens=cap,
                max_model_len=c.max_model_len, device=self.device, head_dim=self.head_dim,
                compact_dtype=self.kv_dtype, max_active_seqs=self.max_num_seqs,
                decode_reserve_tokens=c.compact_decode_reserve_tokens, fp8_scales=c.compact_kv_fp8_scales)
        else:
            self.compact_kv_manager = CompactKVManager(
                num_layers=self.num_layers, num_kv_heads=self.num_kv_heads, capacity_tokens=cap,
                max_model_len=c.max_model_len, device=self.device,
                target_live_tokens_per_seq=c.compact_kv_target_live_tokens_per_seq, head_dim=self.head_dim,
                compact_dtype=self.kv_dtype, per_layer_storage=True, layer_major_metadata=True,
                max_active_seqs=self.max_num_seqs, preallocate=True,
                decode_reserve_tokens=c.compact_decode_reserve_tokens, fp8_scales=c.compact_kv_fp8_scales)
        attn_modules = []
        for layer_id, layer in enumerate(self.model.model.layers):
            layer.self_attn.attn.layer_id = layer_id
            attn_modules.append(layer.self_attn.attn)
        self.compact_kv_manager.attach_attention_modules(attn_modules)

    # -- prefill -----------------------------------------------------------------
    def prepare_prefill(self, seqs: list[Sequence]):
        input_ids, positions, cu = [], [], [0]
        max_q = 0
        for seq in seqs:
            n = len(seq)
            start = min(seq.num_cached_tokens, n - 1)
            nq = seq.num_scheduled_tokens
            input_ids.extend(seq[start:start + nq])
            positions.extend(range(start, start + nq))
            cu.append(cu[-1] + nq)
            max_q = max(max_q, nq)
        ids_t = torch.tensor(input_ids, dtype=torch.int64, pin_memory=True).to(self.device, non_blocking=True)
        pos_t = torch.tensor(positions, dtype=torch.int64, pin_memory=True).to(self.device, non_blocking=True)
        cu_t = torch.tensor(cu, dtype=torch.int32, pin_memory=True).to(self.device, non_blocking=True)
        pack_ids = []
        chunk = None
        for i, seq in enumerate(seqs):
            # a re-prefill after preemption stops one token short: the next
            # decode step appends the last token
            target = seq.num_tokens - 1 if seq.reprefill else seq.num_tokens
            start = seq.num_cached_tokens
            done = min(start + seq.num_scheduled_tokens, target)
            if start > 0 or done < target:  # a chunk of a prompt longer than the step's budget
                if i != 0:
                    raise RuntimeError("only the first sequence of a prefill batch may be chunked")
                chunk = self._plan_chunk(seq, start, seq.num_scheduled_tokens, target)
                if chunk.final:
                    self.compact_kv_manager.allocate(seq)
                continue
            self.compact_kv_manager.allocate(seq)
            pack_ids.append(seq.seq_id)
        if chunk is not None:
            rest = cu[1:]
            chunk.rest_ids = pack_ids
            chunk.cu_rest_host = [c - chunk.rows for c in rest]
            chunk.max_rest = max((rest[j + 1] - rest[j] for j in range(len(rest) - 1)), default=0)
            chunk.cu_rest = (torch.tensor(chunk.cu_rest_host, dtype=torch.int32, pin_memory=True)
                             .to(self.device, non_blocking=True)) if pack_ids else None
            pack_ids = pack_ids + ([chunk.seq_id] if chunk.final else [])
        if self.compact_kv_manager.paged:
            self.compact_kv_manager.begin_prefill()
        md = self.dms_metadata
        set_context(True, cu_t, cu_t, max_q, max_q, dms_capture_enabled=True, dms_alpha_scale=md.alpha_scale,
                    dms_alpha_offset=md.alpha_offset, dms_layer_evictions={},
                    streaming_pack_manager=self.compact_kv_manager, streaming_pack_seq_ids=pack_ids,
                    streaming_pack_window_size=md.window_size, cu_seqlens_q_host=cu, prefill_chunk=chunk)
        return ids_t, pos_t

    def _plan_chunk(self, seq: Sequence, start: int, rows: int, target: int) -> ChunkPlan:
        """The stage and launch metadata of one chunk of a long prompt: the
        prompt's dense stage is made at its first chunk (a restarted prompt,
        e.g. a re-prefill, starts a new one) and must hold exactly the chunks
        before this one."""
        stage = self.prompt_stages.get(seq.seq_id)
        if start == 0 or stage is None or stage.total != target:
            stage = PromptStage(self.num_layers, target, self.num_kv_heads, self.head_dim, self.device)
            self.prompt_stages[seq.seq_id] = stage
        if stage.filled != start or start + rows > target:
            raise RuntimeError(f"prompt chunk {start}..{start + rows} of seq {seq.seq_id} does not follow the "
                               f"{stage.filled} staged tokens")
        end = start + rows
        dev = lambda v: torch.tensor(v, dtype=torch.int32, pin_memory=True).to(self.device, non_blocking=True)
        return ChunkPlan(seq.seq_id, stage, start, rows, end == target, dev([0, rows]), dev([0, end]), [], None,
                         None, 0)

    def _no_step_in_flight(self, what: str) -> None:
        if self._lookahead is not None:
            raise RuntimeError(f"{what} while a decode step launched ahead is in flight (LLMEngine.drain() first)")

    @torch.inference_mode()
    def run_prefill(self, seqs: list[Sequence]) -> list[int]:
        self._no_step_in_flight("prefill")
        ids, pos = self.prepare_prefill(seqs)
        try:
            hidden = self.model(ids, pos)
        except BaseException:
            reset_context()  # e.g. CompactCapacityExhausted from a layer's pack: the engine frees and retries
            raise
        head = self.model.lm_head
        if self.config.fused_greedy_head:
            tokens = self.model.compute_greedy_token_ids(hidden)
            head.last_logits = None
        else:
            logits = self.model.compute_logits(hidden)
            head.last_logits = logits
            tokens = torch.empty(logits.shape[0], device=logits.device, dtype=torch.int64)
            nat.call("fdms_argmax_rows", logits.data_ptr(), nat.dtype_code(logits.dtype), logits.stride(0),
                     logits.shape[0], logits.shape[1], tokens.data_ptr(), nat.stream())
        ctx = get_context()
        total = sum(e.numel() for e in ctx.dms_layer_evictions.values())
        true = sum(e.sum() for e in ctx.dms_layer_evictions.values())
        chunk = ctx.prefill_chunk
        packed = list(ctx.streaming_pack_seq_ids or [])
        reset_context()
        mgr = self.compact_kv_manager
        if mgr.paged:
            mgr.stage_prefill_check(packed)
        out = tokens.tolist()
        if mgr.paged:
            mgr.finish_prefill_check()  # CompactCapacityExhausted when the batch's pages did not fit
        if chunk is not None:  # the chunk is staged; a completed prompt is packed and its stage dropped
            chunk.stage.filled = chunk.end
            if chunk.final:
                self.prompt_stages.pop(chunk.seq_id, None)
        self.last_compact_prefill_stats = {"eviction_decisions_total": total,
                                           "eviction_decisions_true": int(true) if total else 0}
        return out

    # -- decode ------------------------------------------------------------------
    def _decode_body(self, start: int, batch: int, max_live_hint: int) -> torch.Tensor:
        """One decode step on static buffers; captured into a graph.  Returns the
        logits tensor (graph-owned under capture: each replay refreshes it)."""
        mgr = self.compact_kv_manager
        L, H = self.num_layers, self.num_kv_heads
        slot = self.static_slot[:, :batch]
        plan = self.decode_plan if mgr.paged else None
        if mgr.paged:
            bt, live = mgr.paged_prepare_decode(start, batch, slot, plan=plan, positions=self.static_positions)
            base = None
        else:
            bt = None
            base = mgr.layer_major_base_offsets[:, start:start + batch]
            live = mgr.layer_major_live_counts[:, start:start + batch]
            nat.call("fdms_prepare_decode_metadata", base.data_ptr(), base.stride(0), base.stride(1),
                     base.stride(2), live.data_ptr(), live.stride(0), live.stride(1), live.stride(2),
                     slot.data_ptr(), slot.stride(0), slot.stride(1), slot.stride(2), L, batch, H, nat.stream())
        md = self.dms_metadata
        evict = self.evict_buffer[:, :batch]
        set_context(False, block_tables=bt, compact_kv_enabled=True, compact_base_offsets=base,
                    compact_live_counts=live, compact_slot_mapping=slot, compact_max_live_count=max_live_hint,
                    dms_capture_enabled=True, dms_alpha_scale=md.alpha_scale, dms_alpha_offset=md.alpha_offset,
                    dms_layer_evictions_buffer=evict, compact_plan=plan)
        ids = self.static_tokens[:batch]  # read before the step's own ids overwrite them
        pos = self.static_positions[:batch]
        logits = None
        if self.model.decode_fused_supported(batch):
            if self.config.fused_greedy_head:
                self.model.forward_decode_fused(ids, pos, greedy_out=self.static_tokens[:batch])
            else:
                logits = self.model.forward_decode_fused(ids, pos)
        else:
            hidden = self.model(ids, pos)
            head = self.model.lm_head
            if self.config.fused_greedy_head:
                head.greedy_into(hidden.contiguous(), self.static_tokens[:batch])
            else:
                logits = head.logits(hidden.contiguous())
        if logits is not None:
            nat.call("fdms_argmax_rows", logits.data_ptr(), nat.dtype_code(logits.dtype), logits.stride(0), batch,
                     logits.shape[1], self.static_tokens.data_ptr(), nat.stream())
        p, e = mgr.layer_major_token_positions, mgr.layer_major_evict_mask.view(torch.uint8)
        ev = evict.view(torch.uint8)
        nat.call("fdms_record_dms_decisions", p.data_ptr(), p.stride(0), p.stride(1), p.stride(2), p.stride(3),
                 e.data_ptr(), e.stride(0), e.stride(1), e.stride(2), e.stride(3), mgr.layer_major_live_counts.data_ptr(),
                 *mgr.layer_major_live_counts.stride(), ev.data_ptr(), ev.stride(0), ev.stride(1), ev.stride(2),
                 pos.data_ptr(), 1, None, start, L, batch, H, nat.stream())
        reset_context()
        return logits

    def attention_hint(self, seqs: list[Sequence]) -> int:
        """Bound on the live count of every (layer, seq, kv head) of the batch,
        which sets the attention split count.  On the matrix-core path a pair's
        split count follows its own live count and the bound only caps it, so
        the static bound max_model_len serves every step (one decode graph per
        batch shape, never recaptured as the spans grow).  Other kernels split
        evenly by the bound: there it is the host's upper bound rounded up to
        the next 256-token bucket, so eager and graph-replayed steps use the
        same split count (bit-identical results) and one graph serves up to
        256 steps."""
        if self._static_attention_bound:
            return (self.config.max_model_len // 256 + 1) * 256
        return (self.compact_kv_manager.max_live_upper_bound(seqs) // 256 + 1) * 256

    @torch.inference_mode()
    def _begin_decode_step(self, seqs: list[Sequence], positions: list[int]) -> tuple[int, int]:
        """Host side of one decode step: the expiry launch the policy picks for
        these positions and the live bounds; returns (start slot, attention
        bound).  The batch occupies slots start .. start + len - 1."""
        mgr = self.compact_kv_manager
        stats = mgr.apply_dms_evictions(seqs, positions, window_size=self.dms_metadata.window_size, sync_stats=False)
        self.last_dms_decode_stats = [dict(stats, phase="expire")]
        states = [mgr.seq_states[s.seq_id] for s in seqs]
        start = mgr._contiguous_active_slot_start(states)
        if start is None:
            raise RuntimeError("decode batch must occupy contiguous active slots")
        mgr.note_decode_step(states)
        return start, self.attention_hint(seqs)

    def _replay_decode(self, start: int, batch: int, hint: int) -> None:
        """One decode step on the static buffers: the captured graph of this
        batch shape (captured on its second use; the first runs eagerly so the
        library GEMMs pick their kernels outside capture)."""
        mgr = self.compact_kv_manager
        use_graph = self.config.compact_decode_cudagraph and not self.config.enforce_eager
        key = (start, batch)
        if use_graph and key not in self._warm:
            self._warm.add(key)
            use_graph = False
        if use_graph:
            entry = self.graphs.get(key)
            if entry is not None and (entry[1] != mgr.storage_version or hint != entry[2]):
                entry = None
            if entry is None:
                graph = torch.cuda.CUDAGraph()
                torch.cuda.synchronize()
                with torch.cuda.graph(graph, pool=self.graph_pool):
                    logits = self._decode_body(start, batch, hint)
                self.graph_pool = graph.pool()
                entry = (graph, mgr.storage_version, hint, logits)
                self.graphs[key] = entry
            entry[0].replay()
            self.model.lm_head.last_logits = entry[3]
        else:
            self.model.lm_head.last_logits = self._decode_body(start, batch, hint)

    def lookahead_pending(self) -> bool:
        """True while a decode step launched ahead of the host is in flight:
        the engine's next step must be the decode of that same batch."""
        return self._lookahead is not None

    def _stage_tokens(self, batch: int):
        """Queue the copy of the step's sampled ids (and, paged, the page
        pool's overflow flag after them: one copy) to pinned memory; return
        (that buffer, event marking it done)."""
        buf = self._tok_ring[self._ring]
        self._ring ^= 1
        if self.compact_kv_manager.paged:
            buf.copy_(self._readback, non_blocking=True)
        else:
            buf[:batch].copy_(self.static_tokens[:batch], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        return buf, ev

    def _lookahead_ok(self, seqs: list[Sequence]) -> bool:
        """The step after the one just launched is certain: greedy ids on the
        device (fused head), ignore_eos sequences none of which finishes with
        this step, paged KV with room for two more appends."""
        mgr = self.compact_kv_manager
        if not (decode_lookahead_enabled() and self.config.fused_greedy_head and mgr.paged):
            return False
        if any(s.temperature > 1e-10 or not s.ignore_eos or s.num_completion_tokens + 2 > s.max_tokens
               for s in seqs):
            return False
        return mgr.decode_pages_fit(2)

    @torch.inference_mode()
    def run_decode(self, seqs: list[Sequence], lookahead: bool = False) -> list[int]:
        """One decode step of ``seqs``; returns its greedy / sampled ids.  With
        ``lookahead`` (the engine knows the next step decodes the same batch)
        the following step is launched before this one's ids are read back --
        its input ids come from the device -- so the host's per-step work
        overlaps the GPU; that step is then the one a later call returns."""
        mgr = self.compact_kv_manager
        batch = len(seqs)
        self.last_decode_seq_ids = [s.seq_id for s in seqs]  # the rows of this step's logits / ids
        la, self._lookahead = self._lookahead, None
        if la is not None:  # this step is already in flight
            if la["ids"] != [s.seq_id for s in seqs]:
                raise RuntimeError("the decode step in flight is for another batch")
            host, done = la["host"], la["event"]
        else:
            positions = [len(seq) - 1 for seq in seqs]
            # finished / preempted sequences leave holes in the layer-major slots:
            # move the batch's rows to slots 0 .. batch-1 (one launch per step)
            mgr.pack_active_slots([mgr.seq_states[s.seq_id] for s in seqs])
            start, hint = self._begin_decode_step(seqs, positions)
            for i, seq in enumerate(seqs):
                self.pinned_ids[i] = seq.last_token
                self.pinned_pos[i] = positions[i]
            self.static_tokens[:batch].copy_(self.pinned_ids[:batch], non_blocking=True)
            self.static_positions[:batch].copy_(self.pinned_pos[:batch], non_blocking=True)
            self._replay_decode(start, batch, hint)
            self.compact_live_tokens_peak = max(self.compact_live_tokens_peak, mgr.max_live_upper_bound(seqs))
            host, done = self._stage_tokens(batch)
        if lookahead and self._lookahead_ok(seqs):
            positions = [len(seq) for seq in seqs]  # one past the step in flight
            start, hint = self._begin_decode_step(seqs, positions)
            pos = self._pos_ring[self._ring]
            for i, p in enumerate(positions):
                pos[i] = p
            self.static_positions[:batch].copy_(pos[:batch], non_blocking=True)
            # its input ids are the step in flight's greedy ids, already in static_tokens
            self._replay_decode(start, batch, hint)
            self.compact_live_tokens_peak = max(self.compact_live_tokens_peak, mgr.max_live_upper_bound(seqs) + 1)
            nhost, nev = self._stage_tokens(batch)
            self._lookahead = {"ids": [s.seq_id for s in seqs], "host": nhost, "event": nev}
        done.synchronize()
        out = host[:batch].tolist()
        if mgr.paged:
            mgr.raise_if_overflow(int(host[self.max_num_seqs:].view(torch.int32)[0]))
        return out

    @torch.inference_mode()
    def run_compact_greedy_decode_loop(self, seqs: list[Sequence], max_steps: int):
        """Greedy decode of ``max_steps`` tokens for the batch with no host
        sync between steps (model_runner.py:971-1053, which does batch size 1):
        each step's sampled ids feed the next step on the device, positions come
        from a pinned host table filled up front, the expiry policy is decided
        on the host from the positions alone, and one copy of all the tokens
        ends the loop.  Requires the fused greedy head, ignore_eos sequences
        (no EOS check until the end) and the full span reservation.  Returns
        the tokens of a single sequence (the reference's form) or one list per
        sequence."""
        if max_steps <= 0:
            return [] if len(seqs) == 1 else [[] for _ in seqs]
        self._no_step_in_flight("the greedy fast loop")
        if not self.config.fused_greedy_head:
            raise RuntimeError("compact greedy fast loop requires the fused greedy argmax path")
        if self.config.compact_decode_reserve_tokens is not None:
            raise RuntimeError("compact greedy fast loop requires the full decode reservation")
        if any(not s.ignore_eos or s.temperature > 0 for s in seqs):
            raise RuntimeError("compact greedy fast loop requires greedy, ignore_eos sequences")
        if any(s.num_completion_tokens + max_steps > s.max_tokens for s in seqs):
            raise RuntimeError("compact greedy fast loop would run past max_tokens")
        mgr = self.compact_kv_manager
        batch = len(seqs)
        mgr.pack_active_slots([mgr.seq_states[s.seq_id] for s in seqs])
        if mgr.paged and not mgr.decode_pages_fit(max_steps):
            raise RuntimeError(f"compact greedy fast loop: {max_steps} appends do not fit the page pool")
        base_pos = [len(seq) - 1 for seq in seqs]
        pos_table = torch.tensor([[p + step for p in base_pos] for step in range(max_steps)], dtype=torch.int64,
                                 pin_memory=True)
        for i, seq in enumerate(seqs):
            self.pinned_ids[i] = seq.last_token
        self.static_tokens[:batch].copy_(self.pinned_ids[:batch], non_blocking=True)
        tokens = torch.empty((max_steps, batch), device=self.device, dtype=torch.int64)
        for step in range(max_steps):
            start, hint = self._begin_decode_step(seqs, pos_table[step].tolist())
            self.static_positions[:batch].copy_(pos_table[step], non_blocking=True)
            self._replay_decode(start, batch, hint)  # its input ids: the previous step's, in static_tokens
            tokens[step].copy_(self.static_tokens[:batch])
        if mgr.paged:
            mgr.stage_overflow_check()
        out = tokens.t().contiguous().cpu().tolist()  # the loop's one host sync
        if mgr.paged:
            mgr.check_overflow(sync=False)
        for seq, toks in zip(seqs, out):
            for t in toks:
                seq.append_token(t)
                seq.num_cached_tokens += 1
            seq.num_scheduled_tokens = 0
            if seq.num_completion_tokens >= seq.max_tokens:
                seq.status = SequenceStatus.FINISHED
        self.compact_live_tokens_peak = max(self.compact_live_tokens_peak, mgr.max_live_upper_bound(seqs))
        return out[0] if batch == 1 else out

    def run(self, seqs: list[Sequence], is_prefill: bool, lookahead: bool = False) -> list[int]:
        return self.run_prefill(seqs) if is_prefill else self.run_decode(seqs, lookahead)

    def free_compact(self, seq_ids: list[int]) -> None:
        self._no_step_in_flight("freeing compact KV")
        for sid in seq_ids:
            self.compact_kv_manager.free(sid)

    def exit(self) -> None:
        self.graphs.clear()
        self.graph_pool = None
