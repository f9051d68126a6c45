"""CPU emulator of libfastdms_amd's C-ABI — TEST INFRASTRUCTURE ONLY.

Lets the CPU test suite drive the real engine glue (fastdms_amd/engine,
layers, models) end to end without a GPU: ``nat.call(name, *args)`` is
replaced by a function that resolves every raw pointer to the torch storage
that owns it, builds strided views with exactly the strides and extents the
HIP kernel would use (``as_strided`` refuses any view that leaves its
storage, and data-dependent indices are range-checked explicitly), and applies
the entry point's documented semantics (include/fastdms_amd.h) with the
oracle's numerics.  An access a kernel would make outside the buffer it was
handed raises ``OutOfBounds`` naming the entry point and the argument.

This never stands in for the HIP library in the product: only tests install
it, and only over CPU tensors.
"""
from __future__ import annotations

import bisect
import gc
import warnings
from contextlib import contextmanager

import numpy as np
import torch

from oracle import numerics

DT_F32, DT_F16, DT_BF16, DT_FP8 = 0, 1, 2, 3
_TORCH = {DT_F32: torch.float32, DT_F16: torch.float16, DT_BF16: torch.bfloat16, DT_FP8: torch.uint8}
_ITEM = {DT_F32: 4, DT_F16: 2, DT_BF16: 2, DT_FP8: 1}


class OutOfBounds(RuntimeError):
    pass


class _Registry:
    """Maps raw addresses to the CPU storages that own them."""

    def __init__(self):
        self.bases: list[int] = []
        self.entries: list[tuple[int, int, torch.UntypedStorage]] = []

    def refresh(self, generation: int | None = None):
        """Scan the garbage collector's objects for CPU tensors: all of them
        (generation None: the cache is replaced, dropping freed storages), or
        only one gc generation (new tensors sit in generation 0 until a
        collection moves them on), whose storages are added to the cache."""
        seen = {}
        objs = gc.get_objects() if generation is None else gc.get_objects(generation)
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            for o in objs:
                if not isinstance(o, torch.Tensor):
                    continue
                try:
                    if o.device.type == "cpu":
                        s = o.untyped_storage()
                        seen[s.data_ptr()] = (s.data_ptr(), s.nbytes(), s)
                except Exception:  # noqa: BLE001 - fake/meta tensors
                    continue
        if generation is not None:
            for e in self.entries:
                seen.setdefault(e[0], e)
        self.entries = sorted(seen.values(), key=lambda e: e[0])
        self.bases = [e[0] for e in self.entries]

    def find(self, ptr: int):
        for attempt in (None, 0, 1, "all"):
            if attempt is not None:
                self.refresh(None if attempt == "all" else attempt)
            i = bisect.bisect_right(self.bases, ptr) - 1
            if i >= 0:
                base, nbytes, s = self.entries[i]
                if base <= ptr < base + max(nbytes, 1):
                    return base, nbytes, s
        return None


class Emulator:
    def __init__(self):
        self.reg = _Registry()
        self.calls: list[str] = []
        self.name = ""

    # -- views ---------------------------------------------------------------
    def _flat(self, ptr, dtype, what):
        if not ptr:
            raise OutOfBounds(f"{self.name}: NULL {what}")
        hit = self.reg.find(int(ptr))
        if hit is None:
            raise OutOfBounds(f"{self.name}: {what} pointer {ptr:#x} is not inside any live CPU tensor")
        base, nbytes, s = hit
        item = torch.empty((), dtype=dtype).element_size()
        off = int(ptr) - base
        if off % item:
            raise OutOfBounds(f"{self.name}: {what} pointer not aligned to {item} bytes")
        flat = torch.empty(0, dtype=dtype)
        flat.set_(s, 0, (nbytes // item,), (1,))
        return flat, off // item

    def view(self, ptr, dtype, size, stride, what):
        flat, off = self._flat(ptr, dtype, what)
        size = tuple(int(x) for x in size)
        stride = tuple(int(x) for x in stride)
        if any(x < 0 for x in stride):
            raise OutOfBounds(f"{self.name}: negative stride for {what}")
        if all(x > 0 for x in size):
            last = off + sum((n - 1) * st for n, st in zip(size, stride))
            if last >= flat.numel():
                raise OutOfBounds(f"{self.name}: {what} needs element {last} of a {flat.numel()}-element buffer "
                                  f"(size {size}, stride {stride}, offset {off})")
        return flat.as_strided(size, stride, off)

    def view_at(self, ptr, dtype, elem_offset, size, stride, what):
        """view() of the buffer starting elem_offset elements after ptr."""
        item = torch.empty((), dtype=dtype).element_size()
        return self.view(int(ptr) + int(elem_offset) * item, dtype, size, stride, what)

    def flat_at(self, ptr, dtype, what):
        """(flat storage view, element offset of ptr) for data-dependent indexing."""
        return self._flat(ptr, dtype, what)

    def gather_idx(self, flat, idx, what):
        idx = torch.as_tensor(idx, dtype=torch.int64)
        if idx.numel() and (int(idx.min()) < 0 or int(idx.max()) >= flat.numel()):
            raise OutOfBounds(f"{self.name}: {what} index range [{int(idx.min())}, {int(idx.max())}] outside "
                              f"[0, {flat.numel()})")
        return idx

    # -- value conversion ----------------------------------------------------
    @staticmethod
    def load(t: torch.Tensor, code: int) -> torch.Tensor:
        if code == DT_FP8:
            return torch.from_numpy(numerics.e4m3fn_decode(t.contiguous().numpy()))
        return t.to(torch.float32)

    @staticmethod
    def store(dst: torch.Tensor, vals: torch.Tensor, code: int) -> None:
        vals = vals.to(torch.float32)
        if code == DT_FP8:
            dst.copy_(torch.from_numpy(numerics.e4m3fn_encode(vals.contiguous().numpy())))
        else:
            dst.copy_(vals.to(_TORCH[code]))

    # -- dispatch --------------------------------------------------------------
    def __call__(self, name, *args):
        self.name = name
        self.calls.append(name)
        fn = getattr(self, name[len("fdms_"):], None)
        if fn is None:
            raise NotImplementedError(f"emulator has no {name}")
        rc = fn(*args)
        if rc:
            raise RuntimeError(f"{name} failed with HIP error {rc}")

    # -- entry points ------------------------------------------------------------
    def abi_version(self):
        return 0

    def copy_bytes(self, src, dst, n, blocks, stream):
        self.view(dst, torch.uint8, (n,), (1,), "dst").copy_(self.view(src, torch.uint8, (n,), (1,), "src"))

    def convert(self, src, sdt, dst, ddt, n, stream):
        v = self.load(self.view(src, _TORCH[sdt], (n,), (1,), "src"), sdt)
        self.store(self.view(dst, _TORCH[ddt], (n,), (1,), "dst"), v, ddt)

    @staticmethod
    def _decide(v, alpha_scale, alpha_offset, threshold, positive):
        if positive:
            return v > np.float32(threshold)
        return (v * np.float32(alpha_scale)) - np.float32(alpha_offset) > 0

    def extract_dms_decisions(self, q, qdt, qs_t, qs_h, qs_d, evict, es_t, es_h, T, H, G, D, a_s, a_o, thr, pos,
                              stream):
        if T < 0 or H <= 0 or G <= 0 or D <= 0:
            return 1
        if T == 0:
            return 0
        lane = self.view_at(q, _TORCH[qdt], (D - 1) * qs_d, (T, H), (qs_t, G * qs_h), "q decision lane")
        v = self.load(lane, qdt)
        e = self._decide(v, a_s, a_o, thr, pos)
        self.view(evict, torch.uint8, (T, H), (es_t, es_h), "evict").copy_(e.to(torch.uint8))
        lane.zero_()
        return 0

    def _inv_scales(self, scale, H, what):
        """fp32 1 / scale[h] per kv head (the kernels' IEEE division), ones without a table."""
        if not scale:
            return torch.ones(H, dtype=torch.float32)
        s = self.view(scale, torch.float32, (H,), (1,), what).clone()
        return (torch.ones(H, dtype=torch.float32) / s).float()

    def _scales(self, scale, H, what):
        if not scale:
            return torch.ones(H, dtype=torch.float32)
        return self.view(scale, torch.float32, (H,), (1,), what).clone()

    def _seq_spans(self, cu, single_start, single_len, num_seqs):
        if cu:
            c = self.view(cu, torch.int32, (num_seqs + 1,), (1,), "cu_seqlens").tolist()
            return [(c[b], c[b], c[b + 1] - c[b]) for b in range(num_seqs)]
        return [(single_start, 0, single_len)]

    def streaming_pack_prepare(self, evict, es_t, es_h, cu, single_len, num_seqs, window, H, max_chunks, live_out,
                               lo_b, lo_h, offsets, of_b, of_h, of_c, positions, evict_meta, meta_rows, tp_b, tp_h,
                               em_b, em_h, meta_cap, stream):
        if num_seqs <= 0 or H <= 0 or max_chunks < 0:
            return 1
        spans = self._seq_spans(cu, 0, single_len, num_seqs)
        live = self.view(live_out, torch.int32, (num_seqs, H), (lo_b, lo_h), "live_out")
        offs = self.view(offsets, torch.int32, (num_seqs, H, max_chunks), (of_b, of_h, of_c), "block_offsets") \
            if max_chunks > 0 else None
        rows = list(range(num_seqs))
        if meta_rows:
            rows = self.view(meta_rows, torch.int32, (num_seqs,), (1,), "meta_rows").tolist()
        for b, (tok0, ev0, n) in enumerate(spans):
            ev = self.view_at(evict, torch.uint8, ev0 * es_t, (n, H), (es_t, es_h), "evict")
            if positions:
                for h in range(H):
                    self.view_at(positions, torch.int32, rows[b] * tp_b + h * tp_h, (meta_cap,), (1,),
                                 "positions").fill_(-1)
                    self.view_at(evict_meta, torch.uint8, rows[b] * em_b + h * em_h, (meta_cap,), (1,),
                                 "evict_meta").zero_()
            nch = (n + 255) // 256
            thresh = max(0, n - 1 - window)
            for h in range(H):
                keep = torch.zeros(0, dtype=torch.bool)
                if n > 0:
                    t = torch.arange(n)
                    keep = (ev[:, h] == 0) | (t >= thresh)
                running = 0
                for c in range(max_chunks):
                    offs[b, h, c] = running
                    if c < nch:
                        running += int(keep[c * 256:(c + 1) * 256].sum())
                live[b, h] = running
        return 0

    def streaming_pack_rank_scatter(self, k, v, kvdt, ks_t, ks_h, vs_t, vs_h, evict, es_t, es_h, cu, single_start,
                                    single_len, num_seqs, bo, bo_b, bo_h, bo_c, base, bs_b, bs_h, ck, cv, cdt, cs_s,
                                    positions, evict_meta, meta_rows, tp_b, tp_h, tp_s, em_b, em_h, em_s, window, H,
                                    D, max_chunks, vec, k_scale, v_scale, stream, _table=None):
        if num_seqs <= 0 or H <= 0 or D <= 0 or max_chunks <= 0 or vec <= 0 or D % vec:
            return 1
        kinv, vinv = self._inv_scales(k_scale, H, "k_scale"), self._inv_scales(v_scale, H, "v_scale")
        spans = self._seq_spans(cu, single_start, single_len, num_seqs)
        rows = list(range(num_seqs))
        if meta_rows:
            rows = self.view(meta_rows, torch.int32, (num_seqs,), (1,), "meta_rows").tolist()
        offs = self.view(bo, torch.int32, (num_seqs, H, max_chunks), (bo_b, bo_h, bo_c), "block_offsets")
        bases = None if _table else self.view(base, torch.int32, (num_seqs, H), (bs_b, bs_h), "base")
        ckf, ck0 = self.flat_at(ck, _TORCH[cdt], "compact_k")
        cvf, cv0 = self.flat_at(cv, _TORCH[cdt], "compact_v")
        pflat, poff = self.flat_at(positions, torch.int32, "positions")
        eflat, eoff = self.flat_at(evict_meta, torch.uint8, "evict_meta")
        for b, (tok0, ev0, n) in enumerate(spans):
            if n <= 0:
                continue
            n_do = min(n, max_chunks * 256)  # the grid covers max_chunks chunks
            ev = self.view_at(evict, torch.uint8, ev0 * es_t, (n, H), (es_t, es_h), "evict")
            kview = self.view_at(k, _TORCH[kvdt], tok0 * ks_t, (n, H, D), (ks_t, ks_h, 1), "k")
            vview = self.view_at(v, _TORCH[kvdt], tok0 * vs_t, (n, H, D), (vs_t, vs_h, 1), "v")
            thresh = max(0, n - 1 - window)
            t = torch.arange(n_do)
            for h in range(H):
                e = ev[:n_do, h]
                keep = (e == 0) | (t >= thresh)
                local = torch.zeros(n_do, dtype=torch.int64)
                for c in range((n_do + 255) // 256):
                    kc = keep[c * 256:(c + 1) * 256]
                    local[c * 256:(c + 1) * 256] = torch.cumsum(kc.to(torch.int64), 0) - 1 + int(offs[b, h, c])
                src = torch.nonzero(keep).flatten()
                rank = local[src]
                pidx = self.gather_idx(pflat, poff + rows[b] * tp_b + h * tp_h + rank * tp_s, "positions")
                eidx = self.gather_idx(eflat, eoff + rows[b] * em_b + h * em_h + rank * em_s, "evict_meta")
                pflat[pidx] = src.to(torch.int32)
                eflat[eidx] = e[src]
                if _table:  # paged: rank r at row table[row, h, r >> 4] * 16 + (r & 15); no page -> not stored
                    bt, bt_b, bt_h = _table
                    btf, bt0 = self.flat_at(bt, torch.int32, "block_table")
                    pg = btf[self.gather_idx(btf, bt0 + rows[b] * bt_b + h * bt_h + rank // 16, "block_table")]
                    ok = pg >= 0
                    src, rank, pg = src[ok], rank[ok], pg[ok]
                    dst_rows = pg.to(torch.int64) * 16 + rank % 16
                else:
                    dst_rows = int(bases[b, h]) + rank
                didx = dst_rows[:, None] * cs_s + torch.arange(D)[None, :]
                self.gather_idx(ckf, ck0 + didx, "compact_k")
                self.gather_idx(cvf, cv0 + didx, "compact_v")
                kvals = self.load(kview[src, h], kvdt)
                vvals = self.load(vview[src, h], kvdt)
                if k_scale or v_scale:  # stored = x * (1 / scale), one fp32 rounding
                    kvals, vvals = (kvals * kinv[h]).float(), (vvals * vinv[h]).float()
                tmp = torch.empty(didx.shape, dtype=_TORCH[cdt])
                self.store(tmp, kvals, cdt)
                ckf[ck0 + didx] = tmp
                self.store(tmp, vvals, cdt)
                cvf[cv0 + didx] = tmp
        return 0

    def _rotate(self, x1, x2, c, s):
        return x1 * c - x2 * s, x2 * c + x1 * s

    def _cos_sin(self, cos_sin, cs_p, cs_d, pos, D):
        flat, off = self.flat_at(cos_sin, torch.float32, "cos_sin")
        half = D // 2
        pos = torch.as_tensor(pos, dtype=torch.int64)
        ci = off + pos[:, None] * cs_p + torch.arange(half)[None, :] * cs_d
        si = off + pos[:, None] * cs_p + (torch.arange(half)[None, :] + half) * cs_d
        self.gather_idx(flat, ci, "cos_sin")
        self.gather_idx(flat, si, "cos_sin")
        return flat[ci], flat[si]

    def rope_inplace(self, x, dt, xs_t, xs_h, T, NH, D, cos_sin, cs_p, cs_d, positions, stream):
        if T == 0:
            return 0
        xv = self.view(x, _TORCH[dt], (T, NH, D), (xs_t, xs_h, 1), "x")
        pos = self.view(positions, torch.int64, (T,), (1,), "positions")
        c, s = self._cos_sin(cos_sin, cs_p, cs_d, pos, D)
        f = self.load(xv, dt)
        half = D // 2
        y1, y2 = self._rotate(f[..., :half], f[..., half:], c[:, None, :], s[:, None, :])
        self.store(xv, torch.cat([y1, y2], -1), dt)
        return 0

    def dms_rope_store_compact_decode(self, q, qdt, qs_b, qs_h, k, v, kvdt, ks_b, ks_h, vs_b, vs_h, cos_sin, cs_p,
                                      cs_d, ck, cv, cdt, c_s, slot, sm_b, sm_h, ev_out, ev_b, ev_h, positions, B, H,
                                      G, D, a_s, a_o, thr, pos_scale, store_q, store_tk, k_scale, v_scale, stream):
        if B == 0:
            return 0
        kinv, vinv = self._inv_scales(k_scale, H, "k_scale"), self._inv_scales(v_scale, H, "v_scale")
        qv = self.view(q, _TORCH[qdt], (B, H * G, D), (qs_b, qs_h, 1), "q")
        kv_ = self.view(k, _TORCH[kvdt], (B, H, D), (ks_b, ks_h, 1), "k")
        vv = self.view(v, _TORCH[kvdt], (B, H, D), (vs_b, vs_h, 1), "v")
        sl = self.view(slot, torch.int32, (B, H), (sm_b, sm_h), "slot_mapping")
        ev = self.view(ev_out, torch.uint8, (B, H), (ev_b, ev_h), "evict_out")
        pos = self.view(positions, torch.int64, (B,), (1,), "positions")
        c, s = self._cos_sin(cos_sin, cs_p, cs_d, pos, D)
        half = D // 2
        qf = self.load(qv, qdt)
        dec = qf[:, ::G, D - 1]
        ev.copy_(self._decide(dec, a_s, a_o, thr, pos_scale).to(torch.uint8))
        if store_q:
            q2 = qf.clone()
            q2[:, ::G, D - 1] = 0.0
            y1, y2 = self._rotate(q2[..., :half], q2[..., half:], c[:, None, :], s[:, None, :])
            self.store(qv, torch.cat([y1, y2], -1), qdt)
        kf = self.load(kv_, kvdt)
        y1, y2 = self._rotate(kf[..., :half], kf[..., half:], c[:, None, :], s[:, None, :])
        krot = torch.cat([y1, y2], -1)
        if store_tk:
            self.store(kv_, krot, kvdt)
        vf = self.load(vv, kvdt)
        ckf, ck0 = self.flat_at(ck, _TORCH[cdt], "compact_k")
        cvf, cv0 = self.flat_at(cv, _TORCH[cdt], "compact_v")
        for b in range(B):
            for h in range(H):
                r = int(sl[b, h])
                if r < 0:
                    continue
                idx = self.gather_idx(ckf, ck0 + r * c_s + torch.arange(D), "compact_k slot")
                self.gather_idx(cvf, cv0 + r * c_s + torch.arange(D), "compact_v slot")
                tmp = torch.empty(D, dtype=_TORCH[cdt])
                self.store(tmp, (krot[b, h] * kinv[h]).float(), cdt)
                ckf[idx] = tmp
                self.store(tmp, (vf[b, h] * vinv[h]).float() if v_scale else vf[b, h], cdt)
                cvf[cv0 + r * c_s + torch.arange(D)] = tmp
        return 0

    def _qk_norm(self, q, qs_b, qs_h, k, ks_b, ks_h, B, H, G, D, q_norm, k_norm, eps):
        """Qwen3's per-head QK-norm of the fused entry points, as the RMSNorm
        entry point computes it: (q, qs_b, qs_h, k, ks_b, ks_h) of normalised
        copies (the caller keeps self._keep alive for the call)."""
        def norm(ptr, sb, sh, heads, wptr, what):
            x = self.view(ptr, torch.bfloat16, (B, heads, D), (sb, sh, 1), what).float()
            w = self.view(wptr, torch.bfloat16, (D,), (1,), what + "_norm").float()
            inv = torch.rsqrt((x * x).sum(-1, keepdim=True) / D + eps)
            o = ((x * inv).to(torch.bfloat16).float() * w).to(torch.bfloat16).contiguous()
            self._keep.append(o)
            return o.data_ptr(), heads * D, D
        if q_norm:
            q, qs_b, qs_h = norm(q, qs_b, qs_h, H * G, q_norm, "q")
        if k_norm:
            k, ks_b, ks_h = norm(k, ks_b, ks_h, H, k_norm, "k")
        return q, qs_b, qs_h, k, ks_b, ks_h

    def fused_decode_attention(self, q, qs_b, qs_h, k, ks_b, ks_h, v, vs_b, vs_h, cos_sin, cs_p, cs_d, positions,
                               slot, sm_b, sm_h, ev_out, ev_b, ev_h, a_s, a_o, thr, pos_scale, ck, cv, c_s, base,
                               bo_b, bo_h, live, lc_b, lc_h, out, os_b, os_h, ws, counters, B, H, G, D, splits,
                               split_rows, scale, k_scale, v_scale, q_norm, k_norm, eps, stream):
        """The documented composition: (QK-norm,) preprocess (store_q =
        store_transient_k = 0) then attention with in-kernel q RoPE over the
        span incl. the append."""
        if B == 0:
            return 0
        if G > 4 or D not in (64, 128):
            return 1
        self._keep = []
        q, qs_b, qs_h, k, ks_b, ks_h = self._qk_norm(q, qs_b, qs_h, k, ks_b, ks_h, B, H, G, D, q_norm, k_norm, eps)
        self.dms_rope_store_compact_decode(q, DT_BF16, qs_b, qs_h, k, v, DT_BF16, ks_b, ks_h, vs_b, vs_h, cos_sin,
                                           cs_p, cs_d, ck, cv, DT_FP8, c_s, slot, sm_b, sm_h, ev_out, ev_b, ev_h,
                                           positions, B, H, G, D, a_s, a_o, thr, pos_scale, 0, 0, k_scale, v_scale,
                                           stream)
        return self.compact_decode_attention(q, DT_BF16, qs_b, qs_h, ck, cv, DT_FP8, c_s, base, bo_b, bo_h, None, 0,
                                             0, 0, live, lc_b, lc_h, out, os_b, os_h, ws, counters, B, H, G, D,
                                             splits, split_rows, scale, cos_sin, cs_p, cs_d, positions, k_scale,
                                             v_scale, stream)

    def store_compact_kvcache(self, key, value, kvdt, ks_b, ks_h, vs_b, vs_h, ck, cv, cdt, c_s, slot, sm_b, sm_h,
                              B, H, D, k_scale, v_scale, stream):
        if B == 0:
            return 0
        kinv, vinv = self._inv_scales(k_scale, H, "k_scale"), self._inv_scales(v_scale, H, "v_scale")
        kv_ = self.load(self.view(key, _TORCH[kvdt], (B, H, D), (ks_b, ks_h, 1), "key"), kvdt)
        vv = self.load(self.view(value, _TORCH[kvdt], (B, H, D), (vs_b, vs_h, 1), "value"), kvdt)
        sl = self.view(slot, torch.int32, (B, H), (sm_b, sm_h), "slot_mapping")
        ckf, ck0 = self.flat_at(ck, _TORCH[cdt], "compact_k")
        cvf, cv0 = self.flat_at(cv, _TORCH[cdt], "compact_v")
        for b in range(B):
            for h in range(H):
                r = int(sl[b, h])
                if r < 0:
                    continue
                idx = self.gather_idx(ckf, ck0 + r * c_s + torch.arange(D), "compact_k slot")
                self.gather_idx(cvf, cv0 + r * c_s + torch.arange(D), "compact_v slot")
                tmp = torch.empty(D, dtype=_TORCH[cdt])
                self.store(tmp, (kv_[b, h] * kinv[h]).float() if k_scale or v_scale else kv_[b, h], cdt)
                ckf[idx] = tmp
                self.store(tmp, (vv[b, h] * vinv[h]).float() if k_scale or v_scale else vv[b, h], cdt)
                cvf[cv0 + r * c_s + torch.arange(D)] = tmp
        return 0

    def compact_decode_attention(self, q, qdt, qs_b, qs_h, ck, cv, kvdt, c_s, base, bo_b, bo_h, bt, bt_b, bt_h,
                                 page_size, live, lc_b, lc_h, out, os_b, os_h, ws, counters, B, H, G, D, splits,
                                 split_rows, scale, rope_cs, rcs_p, rcs_d, rope_pos, k_scale, v_scale, stream):
        if B == 0:
            return 0
        ksc, vsc = self._scales(k_scale, H, "k_scale"), self._scales(v_scale, H, "v_scale")
        if splits > 1:
            self.view(ws, torch.float32, (B * H * splits * G * (D + 2),), (1,), "workspace")
            cnt = self.view(counters, torch.int32, (B * H,), (1,), "counters")
            if bool((cnt != 0).any()):
                raise OutOfBounds(f"{self.name}: split counters are not zero before the launch")
        qv = self.view(q, _TORCH[qdt], (B, H * G, D), (qs_b, qs_h, 1), "q")
        ov = self.view(out, _TORCH[qdt], (B, H * G, D), (os_b, os_h, 1), "out")
        lv = self.view(live, torch.int32, (B, H), (lc_b, lc_h), "live_counts")
        qf = self.load(qv, qdt)
        if rope_pos:
            pos = self.view(rope_pos, torch.int64, (B,), (1,), "rope_positions")
            c, s = self._cos_sin(rope_cs, rcs_p, rcs_d, pos, D)
            half = D // 2
            q2 = qf.clone()
            q2[:, ::G, D - 1] = 0.0
            y1, y2 = self._rotate(q2[..., :half], q2[..., half:], c[:, None, :], s[:, None, :])
            qf = self.load(torch.cat([y1, y2], -1).to(_TORCH[qdt]) if qdt != DT_FP8 else torch.cat([y1, y2], -1),
                           qdt if qdt != DT_FP8 else DT_F32)
        ckf, ck0 = self.flat_at(ck, _TORCH[kvdt], "compact_k")
        cvf, cv0 = self.flat_at(cv, _TORCH[kvdt], "compact_v")
        res = torch.empty((B, H * G, D), dtype=torch.float32)
        for b in range(B):
            for h in range(H):
                n = int(lv[b, h])
                if n <= 0:
                    raise OutOfBounds(f"{self.name}: live count {n} at (b={b}, h={h})")
                r = torch.arange(n)
                if bt:
                    btf, bt0 = self.flat_at(bt, torch.int32, "block_tables")
                    pidx = self.gather_idx(btf, bt0 + b * bt_b + h * bt_h + r // page_size, "block_tables")
                    rows = btf[pidx].to(torch.int64) * page_size + r % page_size
                else:
                    bv = self.view(base, torch.int32, (B, H), (bo_b, bo_h), "base_offsets")
                    rows = int(bv[b, h]) + r
                idx = rows[:, None] * c_s + torch.arange(D)[None, :]
                kk = self.load(ckf[self.gather_idx(ckf, ck0 + idx, "compact_k span")], kvdt).double()
                vv = self.load(cvf[self.gather_idx(cvf, cv0 + idx, "compact_v span")], kvdt).double()
                qq = qf[b, h * G:(h + 1) * G].double()
                sc = qq @ (kk * float(ksc[h])).T * scale  # dequant: fp8 value * scale
                p = torch.softmax(sc, dim=-1)
                res[b, h * G:(h + 1) * G] = (p @ (vv * float(vsc[h]))).float()
        self.store(ov, res, qdt)
        return 0

    def dms_expiry(self, incremental, positions, ps_l, ps_s, ps_h, evict, es_l, es_s, es_h, live, lc_l, lc_s, lc_h,
                   base, bo_l, bo_s, bo_h, ck, cv, layer_k, layer_v, row_bytes, c_s_bytes, cur, L, S, H, window,
                   stream, _paged=None):
        from oracle import compact_kv as ock
        if S == 0:
            return 0
        lv = self.view(live, torch.int32, (L, S, H), (lc_l, lc_s, lc_h), "live_counts")
        bv = None if _paged else self.view(base, torch.int32, (L, S, H), (bo_l, bo_s, bo_h), "base_offsets")
        cp = self.view(cur, torch.int64, (S,), (1,), "current_positions")
        pflat, poff = self.flat_at(positions, torch.int32, "positions")
        eflat, eoff = self.flat_at(evict, torch.uint8, "evict")
        if layer_k:
            lk = self.view(layer_k, torch.int64, (L,), (1,), "layer_k").tolist()
            lvv = self.view(layer_v, torch.int64, (L,), (1,), "layer_v").tolist()
        for l in range(L):
            ka = lk[l] if layer_k else ck
            va = lvv[l] if layer_k else cv
            kf, k0 = self.flat_at(ka, torch.uint8, "compact_k arena")
            vf, v0 = self.flat_at(va, torch.uint8, "compact_v arena")
            for s_ in range(S):
                for h in range(H):
                    n = int(lv[l, s_, h])
                    if n == 0:
                        continue
                    pi = self.gather_idx(pflat, poff + l * ps_l + s_ * ps_s + h * ps_h + torch.arange(n), "positions")
                    ei = self.gather_idx(eflat, eoff + l * es_l + s_ * es_s + h * es_h + torch.arange(n), "evict")
                    if _paged:
                        span_rows = self._page_rows(_paged, l, s_, h, n)
                    else:
                        span_rows = int(bv[l, s_, h]) + torch.arange(n)
                    rows_b = span_rows[:, None] * c_s_bytes + torch.arange(row_bytes)[None, :]
                    self.gather_idx(kf, k0 + rows_b, "compact_k rows")
                    self.gather_idx(vf, v0 + rows_b, "compact_v rows")
                    pos_row = pflat[pi].numpy().copy()
                    ev_row = (eflat[ei].numpy() != 0)
                    krows = kf[k0 + rows_b].numpy().copy()
                    vrows = vf[v0 + rows_b].numpy().copy()
                    fn = ock.expiry_incremental if incremental else ock.expiry_exact
                    new_live = fn(positions=pos_row, evict=ev_row, live=n, base=0, compact_k=krows,
                                  compact_v=vrows, current_position=int(cp[s_]), window_size=int(window))
                    pflat[pi] = torch.from_numpy(pos_row.astype(np.int32))
                    eflat[ei] = torch.from_numpy(ev_row.astype(np.uint8))
                    kf[k0 + rows_b] = torch.from_numpy(krows)
                    vf[v0 + rows_b] = torch.from_numpy(vrows)
                    lv[l, s_, h] = new_live
                    if _paged:
                        self._release_pages(_paged, l, s_, h, new_live)
        return 0

    # -- paged layout --------------------------------------------------------------
    def _page_rows(self, pg, l, s_, h, n):
        """Physical rows of ranks 0 .. n-1 of span (l, s, h) through its table."""
        btf, bt0 = self.flat_at(pg["bt"], torch.int32, "block_table")
        r = torch.arange(n)
        idx = self.gather_idx(btf, bt0 + l * pg["bt_l"] + s_ * pg["bt_s"] + h * pg["bt_h"] + r // 16,
                              "block_table")
        pages = btf[idx].to(torch.int64)
        if n and int(pages.min()) < 0:
            raise OutOfBounds(f"{self.name}: span (l={l}, s={s_}, h={h}) reads a rank without a page")
        return pages * 16 + r % 16

    def _push_pages(self, stack, stack_stride, top, l, pages):
        tf, t0 = self.flat_at(top, torch.int32, "page_top")
        ti = self.gather_idx(tf, [t0 + l], "page_top")
        at = int(tf[ti][0])
        sf, s0 = self.flat_at(stack, torch.int32, "page_stack")
        si = self.gather_idx(sf, s0 + l * stack_stride + at + torch.arange(len(pages)), "page_stack")
        sf[si] = torch.as_tensor(pages, dtype=torch.int32)
        tf[ti] = at + len(pages)

    def _pop_pages(self, stack, stack_stride, top, l, n):
        """n page ids off layer l's stack, or None (pool short, nothing taken)."""
        tf, t0 = self.flat_at(top, torch.int32, "page_top")
        ti = self.gather_idx(tf, [t0 + l], "page_top")
        at = int(tf[ti][0])
        if n > at:
            return None
        sf, s0 = self.flat_at(stack, torch.int32, "page_stack")
        si = self.gather_idx(sf, s0 + l * stack_stride + at - n + torch.arange(n), "page_stack")
        tf[ti] = at - n
        return sf[si].clone()

    def _release_pages(self, pg, l, s_, h, live_after):
        keep = (live_after + 15) // 16
        hf, h0 = self.flat_at(pg["held"], torch.int32, "pages_held")
        hi = self.gather_idx(hf, [h0 + l * pg["hd_l"] + s_ * pg["hd_s"] + h * pg["hd_h"]], "pages_held")
        n = int(hf[hi][0])
        if n <= keep:
            return
        btf, bt0 = self.flat_at(pg["bt"], torch.int32, "block_table")
        idx = self.gather_idx(btf, bt0 + l * pg["bt_l"] + s_ * pg["bt_s"] + h * pg["bt_h"] + torch.arange(keep, n),
                              "block_table")
        self._push_pages(pg["stack"], pg["stack_stride"], pg["top"], l, btf[idx].clone())
        btf[idx] = -1
        hf[hi] = keep

    def paged_pack_prepare(self, evict, es_t, es_h, cu, num_seqs, window, H, max_chunks, live_out, lo_b, lo_h,
                           offsets, of_b, of_h, of_c, positions, evict_meta, meta_rows, tp_b, tp_h, em_b, em_h,
                           meta_cap, page_stack, page_top, page_budget, bt, bt_b, bt_h, held, hd_b, hd_h, max_pages,
                           overflow, stream):
        if num_seqs <= 0 or H <= 0 or max_chunks <= 0 or max_pages <= 0 or not page_budget:
            return 1
        rc = self.streaming_pack_prepare(evict, es_t, es_h, cu, 0, num_seqs, window, H, max_chunks, live_out, lo_b,
                                         lo_h, offsets, of_b, of_h, of_c, positions, evict_meta, meta_rows, tp_b,
                                         tp_h, em_b, em_h, meta_cap, stream)
        if rc:
            return rc
        live = self.view(live_out, torch.int32, (num_seqs, H), (lo_b, lo_h), "live_out")
        rows = list(range(num_seqs))
        if meta_rows:
            rows = self.view(meta_rows, torch.int32, (num_seqs,), (1,), "meta_rows").tolist()
        ov = self.view(overflow, torch.int32, (1,), (1,), "overflow")
        for b in range(num_seqs):
            for h in range(H):
                n = (int(live[b, h]) + 15) // 16
                got, flag = None, 1
                if 0 < n <= max_pages:
                    budget = self.view(page_budget, torch.int32, (1,), (1,), "page_budget")
                    if int(budget[0]) >= n:  # the debit fits; the stack must then hold the pages
                        budget[0] -= n
                        got, flag = self._pop_pages(page_stack, 0, page_top, 0, n), 2
                if got is None and n > 0:
                    ov[0] = max(int(ov[0]), flag)
                    live[b, h] = 0
                table = self.view_at(bt, torch.int32, rows[b] * bt_b + h * bt_h, (max_pages,), (1,), "block_table")
                table.fill_(-1)
                if got is not None:
                    table[:n] = got
                self.view_at(held, torch.int32, rows[b] * hd_b + h * hd_h, (1,), (1,), "pages_held")[0] = \
                    n if got is not None else 0
        return 0

    def paged_pack_scatter(self, k, v, kvdt, ks_t, ks_h, vs_t, vs_h, evict, es_t, es_h, cu, num_seqs, bo, bo_b,
                           bo_h, bo_c, ck, cv, cdt, cs_s, positions, evict_meta, meta_rows, tp_b, tp_h, tp_s, em_b,
                           em_h, em_s, bt, bt_b, bt_h, window, H, D, max_chunks, vec, k_scale, v_scale, stream):
        if not bo or not cu or not bt:
            return 1
        return self.streaming_pack_rank_scatter(k, v, kvdt, ks_t, ks_h, vs_t, vs_h, evict, es_t, es_h, cu, 0, 0,
                                                num_seqs, bo, bo_b, bo_h, bo_c, None, 0, 0, ck, cv, cdt, cs_s,
                                                positions, evict_meta, meta_rows, tp_b, tp_h, tp_s, em_b, em_h, em_s,
                                                window, H, D, max_chunks, vec, k_scale, v_scale, stream,
                                                _table=(bt, bt_b, bt_h))

    def paged_prepare_decode(self, live, l_l, l_b, l_h, slot, s_l, s_b, s_h, bt, bt_l, bt_b, bt_h, held, hd_l, hd_b,
                             hd_h, stack, stack_stride, top, max_pages, overflow, L, B, H, stream):
        if L <= 0 or B < 0 or H <= 0 or max_pages <= 0:
            return 1
        if B == 0:
            return 0
        lv = self.view(live, torch.int32, (L, B, H), (l_l, l_b, l_h), "live")
        sv = self.view(slot, torch.int32, (L, B, H), (s_l, s_b, s_h), "slot_out")
        hv = self.view(held, torch.int32, (L, B, H), (hd_l, hd_b, hd_h), "pages_held")
        ov = self.view(overflow, torch.int32, (1,), (1,), "overflow")
        for l in range(L):
            for b in range(B):
                for h in range(H):
                    n, np_ = int(lv[l, b, h]), int(hv[l, b, h])
                    table = self.view_at(bt, torch.int32, l * bt_l + b * bt_b + h * bt_h, (max_pages,), (1,),
                                         "block_table")
                    if n >= 16 * np_:
                        got = self._pop_pages(stack, stack_stride, top, l, 1) if np_ < max_pages else None
                        if got is None:
                            ov[0] = 1
                            sv[l, b, h] = -1
                            continue
                        table[np_] = got[0]
                        np_ += 1
                        hv[l, b, h] = np_
                    sv[l, b, h] = int(table[n // 16]) * 16 + n % 16
                    lv[l, b, h] = n + 1
        return 0

    @staticmethod
    def _plan_splits(n, rows, heavy, splits):
        return 1 if n <= rows else min(splits, -(-n // heavy))

    def paged_prepare_decode_plan(self, live, l_l, l_b, l_h, slot, s_l, s_b, s_h, bt, bt_l, bt_b, bt_h, held, hd_l,
                                  hd_b, hd_h, stack, stack_stride, top, max_pages, overflow, positions, plan, plan_l,
                                  split_rows, heavy_rows, num_splits, L, B, H, stream):
        """The slot assignment above (its sequential pops take the stack from
        the top in (layer, seq, head) order, as the kernel's block prefix
        does), then each layer's work items: the unplanned launch's partition
        of each span, the appended rank left out of the rows and flagged, the
        page id of every 16-rank quarter; split 0 of pair p at item p, the
        further splits packed after the pairs, their number in the int
        before the layer's items."""
        if (num_splits <= 0 or B * H > 8192 or not positions or not plan or split_rows % 64 or heavy_rows % 64
                or not 64 <= heavy_rows <= split_rows <= 1024):
            return 1
        rc = self.paged_prepare_decode(live, l_l, l_b, l_h, slot, s_l, s_b, s_h, bt, bt_l, bt_b, bt_h, held, hd_l,
                                       hd_b, hd_h, stack, stack_stride, top, max_pages, overflow, L, B, H, stream)
        if rc or B == 0:
            return rc
        pairs = B * H
        lv = self.view(live, torch.int32, (L, B, H), (l_l, l_b, l_h), "live")
        sv = self.view(slot, torch.int32, (L, B, H), (s_l, s_b, s_h), "slot_out")
        pos = self.view(positions, torch.int64, (B,), (1,), "positions")
        for l in range(L):
            block = self.view_at(plan, torch.int32, l * plan_l, (4 + num_splits * pairs * 72,), (1,), "plan")
            items = block[4:].view(num_splits * pairs, 72)
            extra = 0
            for b in range(B):
                for h in range(H):
                    p = b * H + h
                    n, app = int(lv[l, b, h]), int(sv[l, b, h])
                    ns = self._plan_splits(n, split_rows, heavy_rows, num_splits) if n > 0 else 1
                    per = (-(-n // ns) + 63) // 64 * 64
                    table = self.view_at(bt, torch.int32, l * bt_l + b * bt_b + h * bt_h, (max_pages,), (1,),
                                         "block_table")
                    for sp in range(ns):
                        it = items[p if sp == 0 else pairs + extra + sp - 1]
                        r0 = min(n, sp * per)
                        r1 = min(n, r0 + per)
                        flags = 0
                        if app >= 0 and r0 < n and r1 == n:
                            flags, r1 = 1, n - 1
                        last = max(r1 - 1, r0)
                        used = (r1 - r0 + 63) // 64 * 4 if r1 > r0 else 0
                        pages = [int(table[min(r0 + 16 * j, last) // 16]) for j in range(used)]
                        it[:8 + used] = torch.tensor([p, r0, r1, sp | (ns << 16), n, app, int(pos[b]), flags] + pages,
                                                     dtype=torch.int32)
                    extra += ns - 1
            block[3] = extra
        return 0

    def fused_decode_attention_planned(self, q, qs_b, qs_h, k, ks_b, ks_h, v, vs_b, vs_h, cos_sin, cs_p, cs_d,
                                       positions, plan, ev_out, ev_b, ev_h, a_s, a_o, thr, pos_scale, ck, cv, c_s,
                                       out, os_b, os_h, ws, counters, B, H, G, D, splits, scale, k_scale, v_scale,
                                       q_norm, k_norm, eps, stream):
        """Check the layer's plan (every pair's live items cover its ranks
        once, in split order, with consistent split counts, live count, append
        row and position; the items past its count name its pair and count),
        rebuild each span's rows from the items' page ids alone, and run the
        unplanned composition on them."""
        if B == 0:
            return 0
        if splits <= 0 or G > 4 or D not in (64, 128) or not positions:
            return 1
        pairs = B * H
        extra = int(self.view_at(plan, torch.int32, -1, (1,), (1,), "plan count")[0])
        if not 0 <= extra <= pairs * (splits - 1):
            raise OutOfBounds(f"{self.name}: {extra} further splits for a grid of {pairs * splits}")
        items = self.view(plan, torch.int32, (pairs + extra, 72), (72, 1), "plan").clone().tolist()
        pos_in = self.view(positions, torch.int64, (B,), (1,), "positions")
        live = torch.zeros((B, H), dtype=torch.int32)
        slot = torch.full((B, H), -1, dtype=torch.int32)
        maxp = 1
        its_of = {p: [items[p]] for p in range(pairs)}
        for it in items[pairs:]:
            if not 0 <= it[0] < pairs:
                raise OutOfBounds(f"{self.name}: item of pair {it[0]}")
            its_of[it[0]].append(it)
        for p, its in its_of.items():
            ns = its[0][3] >> 16
            if len(its) != ns or any(it[0] != p or (it[3] & 0xFFFF) != sp or it[3] >> 16 != ns
                                     for sp, it in enumerate(its)) or not 1 <= ns <= splits:
                raise OutOfBounds(f"{self.name}: inconsistent items of pair {p}")
            maxp = max(maxp, -(-its[0][4] // 16))
        table = torch.full((B, H, maxp), -1, dtype=torch.int32)
        for p, its in its_of.items():
            b, h = divmod(p, H)
            lv, app, ps = its[0][4], its[0][5], its[0][6]
            if any((it[4], it[5], it[6]) != (lv, app, ps) for it in its) or ps != int(pos_in[b]):
                raise OutOfBounds(f"{self.name}: inconsistent items of pair {p}")
            covered = 0
            for i, it in enumerate(its):
                r0, r1, flags = it[1], it[2], it[7]
                if r0 != covered or r0 % 64 or r1 < r0 or r1 - r0 > 1024:
                    raise OutOfBounds(f"{self.name}: item ranks [{r0}, {r1}) of pair {p} after {covered}")
                for r in range(r0, r1):
                    page = it[8 + (r - r0) // 16]
                    if table[b, h, r // 16] not in (-1, page):
                        raise OutOfBounds(f"{self.name}: pair {p} rank {r} on two pages")
                    table[b, h, r // 16] = page
                covered = r1
                if flags & 1:
                    if app < 0 or r1 != lv - 1 or i != len(its) - 1:
                        raise OutOfBounds(f"{self.name}: appended rank of pair {p} misplaced")
                    covered = lv
            if covered != lv:
                raise OutOfBounds(f"{self.name}: pair {p} covers {covered} of {lv} ranks")
            if app >= 0:  # the appended rank's page: the one holding the append row
                table[b, h, (lv - 1) // 16] = app // 16
            live[b, h], slot[b, h] = lv, app
        self._plan_keep = (live, slot, table)
        return self.fused_decode_attention_paged(q, qs_b, qs_h, k, ks_b, ks_h, v, vs_b, vs_h, cos_sin, cs_p, cs_d,
                                                 positions, slot.data_ptr(), H, 1, ev_out, ev_b, ev_h, a_s, a_o,
                                                 thr, pos_scale, ck, cv, c_s, table.data_ptr(), H * maxp, maxp, 16,
                                                 live.data_ptr(), H, 1, out, os_b, os_h, ws, counters, B, H, G, D,
                                                 splits, 0, scale, k_scale, v_scale, q_norm, k_norm, eps, stream)

    def paged_free(self, rows, num_rows, bt, bt_l, bt_b, bt_h, held, hd_l, hd_b, hd_h, live, l_l, l_b, l_h, stack,
                   stack_stride, top, L, H, stream):
        if L <= 0 or num_rows < 0 or H <= 0:
            return 1
        if num_rows == 0:
            return 0
        rv = self.view(rows, torch.int32, (num_rows,), (1,), "rows").tolist()
        for l in range(L):
            for r in rv:
                for h in range(H):
                    hp = self.view_at(held, torch.int32, l * hd_l + r * hd_b + h * hd_h, (1,), (1,), "pages_held")
                    n = int(hp[0])
                    if n > 0:
                        table = self.view_at(bt, torch.int32, l * bt_l + r * bt_b + h * bt_h, (n,), (1,),
                                             "block_table")
                        self._push_pages(stack, stack_stride, top, l, table.clone())
                        table.fill_(-1)
                    hp[0] = 0
                    self.view_at(live, torch.int32, l * l_l + r * l_b + h * l_h, (1,), (1,), "live")[0] = 0
        return 0

    def paged_expiry(self, incremental, positions, ps_l, ps_s, ps_h, evict, es_l, es_s, es_h, live, lc_l, lc_s, lc_h,
                     bt, bt_l, bt_s, bt_h, held, hd_l, hd_s, hd_h, stack, stack_stride, top, layer_k, layer_v,
                     row_bytes, c_s_bytes, cur, L, S, H, window, stream):
        if not bt or not layer_k or not layer_v:
            return 1
        pg = dict(bt=bt, bt_l=bt_l, bt_s=bt_s, bt_h=bt_h, held=held, hd_l=hd_l, hd_s=hd_s, hd_h=hd_h, stack=stack,
                  stack_stride=stack_stride, top=top)
        return self.dms_expiry(incremental, positions, ps_l, ps_s, ps_h, evict, es_l, es_s, es_h, live, lc_l, lc_s,
                               lc_h, None, 0, 0, 0, None, None, layer_k, layer_v, row_bytes, c_s_bytes, cur, L, S, H,
                               window, stream, _paged=pg)

    def fused_decode_attention_paged(self, q, qs_b, qs_h, k, ks_b, ks_h, v, vs_b, vs_h, cos_sin, cs_p, cs_d,
                                     positions, slot, sm_b, sm_h, ev_out, ev_b, ev_h, a_s, a_o, thr, pos_scale, ck, cv,
                                     c_s, bt, bt_b, bt_h, page_size, live, lc_b, lc_h, out, os_b, os_h, ws, counters,
                                     B, H, G, D, splits, split_rows, scale, k_scale, v_scale, q_norm, k_norm, eps,
                                     stream):
        if B == 0:
            return 0
        if G > 4 or D not in (64, 128) or not bt:
            return 1
        self._keep = []
        q, qs_b, qs_h, k, ks_b, ks_h = self._qk_norm(q, qs_b, qs_h, k, ks_b, ks_h, B, H, G, D, q_norm, k_norm, eps)
        self.dms_rope_store_compact_decode(q, DT_BF16, qs_b, qs_h, k, v, DT_BF16, ks_b, ks_h, vs_b, vs_h, cos_sin,
                                           cs_p, cs_d, ck, cv, DT_FP8, c_s, slot, sm_b, sm_h, ev_out, ev_b, ev_h,
                                           positions, B, H, G, D, a_s, a_o, thr, pos_scale, 0, 0, k_scale, v_scale,
                                           stream)
        return self.compact_decode_attention(q, DT_BF16, qs_b, qs_h, ck, cv, DT_FP8, c_s, None, 0, 0, bt, bt_b, bt_h,
                                             page_size, live, lc_b, lc_h, out, os_b, os_h, ws, counters, B, H, G, D,
                                             splits, split_rows, scale, cos_sin, cs_p, cs_d, positions, k_scale,
                                             v_scale, stream)

    def prepare_decode_metadata(self, base, b_l, b_b, b_h, live, l_l, l_b, l_h, slot, s_l, s_b, s_h, L, B, H,
                                stream):
        if L <= 0 or B < 0 or H <= 0:
            return 1
        if B == 0:
            return 0
        bv = self.view(base, torch.int32, (L, B, H), (b_l, b_b, b_h), "base")
        lv = self.view(live, torch.int32, (L, B, H), (l_l, l_b, l_h), "live")
        sv = self.view(slot, torch.int32, (L, B, H), (s_l, s_b, s_h), "slot_out")
        sv.copy_(bv + lv)
        lv.add_(1)
        return 0

    def record_dms_decisions(self, positions, p_l, p_s, p_h, p_c, evict, e_l, e_s, e_h, e_c, live, l_l, l_s, l_h,
                             evict_all, a_l, a_b, a_h, cur, pos64, meta_rows, row_start, L, B, H, stream):
        if L <= 0 or B < 0 or H <= 0:
            return 1
        if B == 0:
            return 0
        rows = list(range(row_start, row_start + B))
        if meta_rows:
            rows = self.view(meta_rows, torch.int32, (B,), (1,), "meta_rows").tolist()
        cp = self.view(cur, torch.int64 if pos64 else torch.int32, (B,), (1,), "cur_positions")
        av = self.view(evict_all, torch.uint8, (L, B, H), (a_l, a_b, a_h), "evict_all")
        pflat, poff = self.flat_at(positions, torch.int32, "positions")
        eflat, eoff = self.flat_at(evict, torch.uint8, "evict")
        lflat, loff = self.flat_at(live, torch.int32, "live")
        for l in range(L):
            for b in range(B):
                for h in range(H):
                    li = self.gather_idx(lflat, [loff + l * l_l + rows[b] * l_s + h * l_h], "live")
                    idx = int(lflat[li][0]) - 1
                    if idx < 0:
                        raise OutOfBounds(f"{self.name}: live count 0 at (l={l}, row={rows[b]}, h={h})")
                    pi = self.gather_idx(pflat, [poff + l * p_l + rows[b] * p_s + h * p_h + idx * p_c], "positions")
                    ei = self.gather_idx(eflat, [eoff + l * e_l + rows[b] * e_s + h * e_h + idx * e_c], "evict")
                    pflat[pi] = int(cp[b])
                    eflat[ei] = int(av[l, b, h])
        return 0

    def argmax_rows(self, x, dt, stride, rows, n, out, stream):
        if rows == 0:
            return 0
        xv = self.load(self.view(x, _TORCH[dt], (rows, n), (stride, 1), "x"), dt)
        m = xv.max(dim=1, keepdim=True).values  # NaN if the row holds one (torch.argmax semantics)
        hit = torch.where(torch.isnan(m), torch.isnan(xv), xv == m)
        first = torch.where(hit, torch.arange(n)[None, :], n).min(dim=1).values
        self.view(out, torch.int64, (rows,), (1,), "out").copy_(first)
        return 0

    def _store_row_amax(self, amax_out, out_rows, q_out=0, q_stride=0, q_mode=0):
        """amax_out[r] = max |out[r]|; q_out = e4m3fn(out * 448/amax) (oracle/linear.py's row quantisation)."""
        from oracle import linear as olin
        rows, hidden = out_rows.shape
        if q_out and (not amax_out or q_mode not in (1, 2) or q_stride < hidden):
            raise OutOfBounds(f"{self.name}: bad q_out arguments")
        if amax_out:
            am = out_rows.float().abs().amax(dim=1)
            self.view(amax_out, torch.float32, (rows,), (1,), "amax_out").copy_(am)
            if q_out:
                xs = olin.amax_to_scale(am.numpy(), torch_form=q_mode == 2)
                codes = numerics.e4m3fn_encode((out_rows.float().numpy() * xs[:, None]).astype(np.float32))
                self.view(q_out, torch.uint8, (rows, hidden), (q_stride, 1), "q_out").copy_(torch.from_numpy(codes))

    def rmsnorm(self, x, in_stride, in_head_stride, heads, residual, weight, out, out_stride, residual_out, rows,
                hidden, eps, amax_out, q_out, q_stride, q_mode, stream):
        if rows < 0 or hidden <= 0 or hidden % 8 or hidden > 8192 or heads <= 0:
            return 1
        if rows == 0:
            return 0
        tokens = rows // heads
        xv = self.view(x, torch.bfloat16, (tokens, heads, hidden), (in_stride, in_head_stride, 1), "in")
        f = xv.float().reshape(rows, hidden)
        if residual:
            f = f + self.view(residual, torch.bfloat16, (rows, hidden), (hidden, 1), "residual").float()
        if residual_out:
            self.view(residual_out, torch.bfloat16, (rows, hidden), (hidden, 1), "residual_out").copy_(
                f.to(torch.bfloat16))
        w = self.view(weight, torch.bfloat16, (hidden,), (1,), "weight").float()
        inv = torch.rsqrt((f * f).sum(-1, keepdim=True) / hidden + eps)
        xn = (f * inv).to(torch.bfloat16).float()
        o = (xn * w).to(torch.bfloat16)
        if out:
            self.view(out, torch.bfloat16, (rows, hidden), (out_stride, 1), "out").copy_(o)
        elif not q_out:
            return 1
        self._store_row_amax(amax_out, o, q_out, q_stride, q_mode)
        return 0

    def rmsnorm_partials(self, partials, k_splits, split_stride, residual, weight, out, out_stride, residual_out,
                         rows, hidden, eps, row_scale, col_scale, amax_out, q_out, q_stride, q_mode, stream):
        if rows < 0 or hidden <= 0 or hidden % 8 or hidden > 8192 or k_splits < 1 or split_stride < rows * hidden:
            return 1
        if rows == 0:
            return 0
        part = self.view(partials, torch.float32, (k_splits, rows, hidden), (split_stride, hidden, 1), "partials")
        acc = torch.zeros((rows, hidden), dtype=torch.float32)
        for s in range(k_splits):
            acc = acc + part[s]
        if row_scale:
            acc = acc * self.view(row_scale, torch.float32, (rows,), (1,), "row_scale")[:, None]
        if col_scale:
            acc = acc * self.view(col_scale, torch.float32, (hidden,), (1,), "col_scale")[None, :]
        f = acc.to(torch.bfloat16).float()
        if residual:
            f = f + self.view(residual, torch.bfloat16, (rows, hidden), (hidden, 1), "residual").float()
        if residual_out:
            self.view(residual_out, torch.bfloat16, (rows, hidden), (hidden, 1), "residual_out").copy_(
                f.to(torch.bfloat16))
        w = self.view(weight, torch.bfloat16, (hidden,), (1,), "weight").float()
        inv = torch.rsqrt((f * f).sum(-1, keepdim=True) / hidden + eps)
        xn = (f * inv).to(torch.bfloat16).float()
        o = (xn * w).to(torch.bfloat16)
        if out:
            self.view(out, torch.bfloat16, (rows, hidden), (out_stride, 1), "out").copy_(o)
        elif not q_out:
            return 1
        self._store_row_amax(amax_out, o, q_out, q_stride, q_mode)
        return 0

    def embedding_rmsnorm(self, ids, n, table, t_s, vocab, weight, eps, out, o_s, rows_out, r_s, hidden, stream):
        """rows_out = table[ids] (NaN rows for ids outside the table), out = their RMSNorm."""
        if n < 0 or hidden <= 0 or hidden % 8 or vocab <= 0 or r_s != hidden or t_s < hidden or o_s < hidden:
            return 1
        if n == 0:
            return 0
        idv = self.view(ids, torch.int64, (n,), (1,), "ids")
        ok = (idv >= 0) & (idv < vocab)
        tab = self.view(table, torch.bfloat16, (vocab, hidden), (t_s, 1), "table")
        f = tab[torch.where(ok, idv, torch.zeros_like(idv))].float()
        f[~ok] = float("nan")
        self.view(rows_out, torch.bfloat16, (n, hidden), (r_s, 1), "rows_out").copy_(f.to(torch.bfloat16))
        w = self.view(weight, torch.bfloat16, (hidden,), (1,), "weight").float()
        inv = torch.rsqrt((f * f).sum(-1, keepdim=True) / hidden + eps)
        o = ((f * inv).to(torch.bfloat16).float() * w).to(torch.bfloat16)
        self.view(out, torch.bfloat16, (n, hidden), (o_s, 1), "out").copy_(o)
        return 0

    def embedding_fp8(self, ids, n, table, t_s, scale_inv, vocab, out, o_s, dim, stream):
        """bf16(bf16(e4m3fn row) * bf16(scale_inv)), NaN rows for ids outside [0, vocab)."""
        if n < 0 or dim <= 0 or dim % 8 or vocab <= 0 or t_s < dim or o_s < dim:
            return 1
        if n == 0:
            return 0
        idv = self.view(ids, torch.int64, (n,), (1,), "ids")
        ok = (idv >= 0) & (idv < vocab)
        safe = torch.where(ok, idv, torch.zeros_like(idv))
        tab = self.view(table, torch.uint8, (vocab, dim), (t_s, 1), "table")
        rows = torch.from_numpy(numerics.e4m3fn_decode(tab[safe].numpy()).astype(np.float32))
        s = self.view(scale_inv, torch.float32, (vocab,), (1,), "scale_inv")[safe]
        s = s.to(torch.bfloat16).float().reshape(-1, 1)
        y = (rows * s).to(torch.bfloat16)
        y[~ok] = float("nan")
        self.view(out, torch.bfloat16, (n, dim), (o_s, 1), "out").copy_(y)
        return 0

    def silu_mul(self, x, out, rows, f, stream):
        if rows == 0:
            return 0
        xv = self.view(x, torch.bfloat16, (rows, 2 * f), (2 * f, 1), "x").float()
        g, u = xv[:, :f], xv[:, f:]
        self.view(out, torch.bfloat16, (rows, f), (f, 1), "out").copy_((torch.nn.functional.silu(g) * u)
                                                                         .to(torch.bfloat16))
        return 0

    def quantize_fp8_rows(self, x, dt, x_s, rows, k, out, out_s, scale_inv, torch_form, stream):
        from oracle import linear as olin
        if rows == 0:
            return 0
        xv = self.load(self.view(x, _TORCH[dt], (rows, k), (x_s, 1), "in"), dt).numpy()
        q, xs = olin.quantize_rows_fp8(xv, torch_form=bool(torch_form))
        self.view(out, torch.uint8, (rows, k), (out_s, 1), "out").copy_(torch.from_numpy(q))
        sinv = (np.float32(1.0) / xs).astype(np.float32)
        self.view(scale_inv, torch.float32, (rows,), (1,), "scale_inv").copy_(torch.from_numpy(sinv))
        return 0

    def fp8_gemm(self, x, x_s, x_inv, w, w_s, w_inv, bias, y, y_s, M, N, K, stream):
        """y = bf16((xq . w8) * x_inv * w_inv) (+ bias in bf16), fp32 products."""
        if M < 0 or N <= 0 or K <= 0 or K % 16 or x_s % 16 or w_s % 16:
            return 1
        if M == 0:
            return 0
        xq = torch.from_numpy(numerics.e4m3fn_decode(self.view(x, torch.uint8, (M, K), (x_s, 1), "x").numpy()))
        wq = torch.from_numpy(numerics.e4m3fn_decode(self.view(w, torch.uint8, (N, K), (w_s, 1), "w").numpy()))
        xi = self.view(x_inv, torch.float32, (M,), (1,), "x_inv")
        wi = self.view(w_inv, torch.float32, (N,), (1,), "w_inv")
        acc = (xq.float() @ wq.float().T) * xi.reshape(-1, 1) * wi.reshape(1, -1)
        out = acc.to(torch.bfloat16)
        if bias:
            out = (out.float() + self.view(bias, torch.bfloat16, (N,), (1,), "bias").float()).to(torch.bfloat16)
        self.view(y, torch.bfloat16, (M, N), (y_s, 1), "y").copy_(out)
        return 0

    def linear_small_m(self, x, x_s, m, k, w, w_dtype, w_s, wsi, bias, n, prologue, norm_w, eps, res, res_s,
                       res_out, ro_s, qx, epilogue, k_splits, ws, counters, y, y_s, x_amax, x_amax_n, x_amax_s,
                       amax_out, row_scale_out, x_dtype, stream):
        """Same expressions as oracle/model.py (rmsnorm, mlp, linear) and oracle/linear.py.
        A producer's x_amax must equal x's own row amax (the kernel's contract);
        x_dtype FP8: x holds the e4m3fn codes its producer quantised with that amax.
        Prologue 2: x holds fp32 rows f and x_amax the per-strip sums of f^2 of an
        epilogue-4 producer; epilogue 4: f = bf16 result + residual to y (fp32),
        bf16(f) to residual_out, per-strip sums of f^2 to amax_out."""
        from oracle import linear as olin
        if m == 0 or n == 0:
            return 0
        n_out = n // 2 if epilogue == 1 else n
        if m > 16 or (k // max(k_splits, 1)) % 256 or n_out % 16 or prologue not in (0, 1, 2) or epilogue == 2:
            return 1
        stats_in, stats_out = prologue == 2, epilogue == 4
        if stats_in and (x_dtype != DT_F32 or qx or not x_amax or x_amax_n != k // 16 or k % 16 or epilogue > 1):
            return 1
        if stats_out and (prologue or qx or not res or not res_out or not amax_out):
            return 1
        if x_amax and not stats_in and (prologue or not qx or x_amax_n < 1 or (m > 1 and x_amax_s < x_amax_n)):
            return 1
        if (amax_out and epilogue > 1 and not stats_out) or (row_scale_out and epilogue != 3):
            return 1
        xq_in = x_dtype == DT_FP8
        if (x_dtype not in (DT_BF16, DT_FP8) and not stats_in) or (xq_in and (w_dtype != DT_FP8 or not qx or not x_amax)):
            return 1
        am = None
        if x_amax and not stats_in:
            self.calls.append("fdms_linear_small_m:x_amax" + (":fp8_x" if xq_in else ""))
            am = self.view(x_amax, torch.float32, (m, x_amax_n), (x_amax_s, 1), "x_amax").amax(dim=1)
            if not xq_in:
                want = self.view(x, torch.bfloat16, (m, k), (x_s, 1), "x").float().abs().amax(dim=1)
                if not torch.equal(am, want):
                    raise AssertionError(f"{self.name}: x_amax {am.tolist()} is not x's row amax {want.tolist()}")

        def quantised_x():
            """(activation values after the FP8 row quantisation, 1 / x_s) as float64."""
            if xq_in:
                codes = self.view(x, torch.uint8, (m, k), (x_s, 1), "x").numpy()
                xs = olin.amax_to_scale(am.numpy(), torch_form=qx == 2)
                return numerics.e4m3fn_decode(codes).astype(np.float64), (np.float32(1.0) / xs).astype(np.float64)
            xq, xs = olin.quantize_rows_fp8(self.view(x, torch.bfloat16, (m, k), (x_s, 1), "x").float().numpy(),
                                            torch_form=qx == 2)
            return numerics.e4m3fn_decode(xq).astype(np.float64), (np.float32(1.0) / xs).astype(np.float64)

        if epilogue == 3:  # split partials: all of the fp32 sum in split 0, zeros in the others
            if prologue or bias or not ws:
                return 1
            part = self.view(ws, torch.float32, (k_splits, m, n), (m * n, n, 1), "partials")
            if w_dtype == DT_FP8:
                wv = numerics.e4m3fn_decode(self.view(w, torch.uint8, (n, k), (w_s, 1), "weight").numpy())
            else:
                wv = self.view(w, torch.bfloat16, (n, k), (w_s, 1), "weight").float().numpy()
            if qx:
                xv, inv = quantised_x()
            else:
                xv = self.view(x, torch.bfloat16, (m, k), (x_s, 1), "x").float().numpy()
                inv = np.ones(m)
            part.zero_()
            part[0].copy_(torch.from_numpy((xv.astype(np.float64) @ wv.astype(np.float64).T).astype(np.float32)))
            if row_scale_out:
                self.view(row_scale_out, torch.float32, (m,), (1,), "row_scale_out").copy_(
                    torch.from_numpy(inv.astype(np.float32)))
            if w_dtype == DT_FP8:
                self.calls.append("fdms_linear_small_m:fp8_partials")
            return 0
        if k_splits > 1:
            strips = n_out // 16
            self.view(ws, torch.float32, (strips * k_splits * 256 * (2 if epilogue else 1),), (1,), "workspace")
            cnt = self.view(counters, torch.int32, (strips,), (1,), "counters")
            if bool((cnt != 0).any()):
                raise OutOfBounds(f"{self.name}: split-K counters are not zero before the launch")
        bv = self.view(bias, torch.bfloat16, (n,), (1,), "bias").float() if bias else None
        if xq_in:
            a = None
        elif stats_in:
            self.calls.append("fdms_linear_small_m:norm_stats")
            f = self.view(x, torch.float32, (m, k), (x_s, 1), "x")
            ss = self.view(x_amax, torch.float32, (m, x_amax_n), (x_amax_s, 1), "x_amax").sum(dim=1, keepdim=True)
            a = (f * torch.rsqrt(ss / k + eps)).to(torch.bfloat16).float()
            nw = self.view(norm_w, torch.bfloat16, (k,), (1,), "norm_weight").float()
            a = (a * nw).to(torch.bfloat16).float()
        elif prologue == 1:
            xv = self.view(x, torch.bfloat16, (m, k), (x_s, 1), "x").float()
            f = xv + (self.view(res, torch.bfloat16, (m, k), (res_s, 1), "residual").float() if res else 0.0)
            if res_out:
                self.view(res_out, torch.bfloat16, (m, k), (ro_s, 1), "residual_out").copy_(f.to(torch.bfloat16))
            var = (f * f).mean(dim=-1, keepdim=True)
            a = (f * torch.rsqrt(var + eps)).to(torch.bfloat16).float()
            nw = self.view(norm_w, torch.bfloat16, (k,), (1,), "norm_weight").float()
            a = (a * nw).to(torch.bfloat16).float()
        else:
            a = self.view(x, torch.bfloat16, (m, k), (x_s, 1), "x").float()
        if w_dtype == DT_FP8:
            w8 = self.view(w, torch.uint8, (n, k), (w_s, 1), "weight").numpy()
            si = self.view(wsi, torch.float32, (n,), (1,), "scale_inv").numpy()
            if xq_in:
                xv, inv = quantised_x()
                acc = (xv @ numerics.e4m3fn_decode(w8).astype(np.float64).T) * inv[:, None] * \
                    si.astype(np.float64)[None, :]
            else:
                acc = olin.fp8_linear(a.numpy(), w8.T, si, quantize_x=bool(qx), torch_form=qx == 2)
            out = torch.from_numpy(acc.astype(np.float32)).to(torch.bfloat16).float()
            if bv is not None:
                out = (out + bv).to(torch.bfloat16).float()
        else:
            wv = self.view(w, torch.bfloat16, (n, k), (w_s, 1), "weight").float()
            out = a @ wv.T
            if bv is not None:
                out = out + bv
            out = out.to(torch.bfloat16).float()
        if epilogue == 1:  # gate_up -> SiluAndMul, the oracle model's mlp expression
            g, u = out[:, :n_out], out[:, n_out:]
            out = torch.nn.functional.silu(g) * u
        if stats_out:
            self.calls.append("fdms_linear_small_m:residual_stats")
            rv = self.view(res, torch.bfloat16, (m, n), (res_s, 1), "residual").float()
            f = out + rv
            self.view(res_out, torch.bfloat16, (m, n), (ro_s, 1), "residual_out").copy_(f.to(torch.bfloat16))
            self.view(y, torch.float32, (m, n), (y_s, 1), "y").copy_(f)
            self.view(amax_out, torch.float32, (m, n // 16), (n // 16, 1), "amax_out").copy_(
                (f * f).reshape(m, n // 16, 16).sum(dim=2))
            return 0
        yb = out.to(torch.bfloat16)
        self.view(y, torch.bfloat16, (m, n_out), (y_s, 1), "y").copy_(yb)
        if amax_out:
            strips = n_out // 16
            self.view(amax_out, torch.float32, (m, strips), (strips, 1), "amax_out").copy_(
                yb.float().abs().reshape(m, strips, 16).amax(dim=2))
        return 0

    def linear_argmax_small_m(self, x, x_s, m, k, w, w_dtype, w_s, wsi, bias, n, qx, bf16_scores, k_splits, ws,
                              counters, part_val, part_idx, out, stream):
        """Greedy head: scores as the oracle model's lm_head (bf16 logits) or
        oracle/linear.py's FP8 scores (fp32, or bf16 logits), torch.argmax order."""
        from oracle import linear as olin
        if m == 0:
            return 0
        strips = n // 16
        self.view(part_val, torch.float32, (m, strips), (strips, 1), "part_val")
        self.view(part_idx, torch.int32, (m, strips), (strips, 1), "part_idx")
        a = self.view(x, torch.bfloat16, (m, k), (x_s, 1), "x").float()
        bv = self.view(bias, torch.bfloat16, (n,), (1,), "bias").float() if bias else None
        if w_dtype == DT_FP8:
            w8 = self.view(w, torch.uint8, (n, k), (w_s, 1), "weight").numpy()
            si = self.view(wsi, torch.float32, (n,), (1,), "scale_inv").numpy()
            sc = torch.from_numpy(olin.fp8_linear(a.numpy(), w8.T, si, quantize_x=bool(qx),
                                                  torch_form=qx == 2).astype(np.float32))
            if bf16_scores:
                sc = sc.to(torch.bfloat16).float()
                if bv is not None:
                    sc = (sc + bv).to(torch.bfloat16).float()
            elif bv is not None:
                sc = sc + bv
        else:
            wv = self.view(w, torch.bfloat16, (n, k), (w_s, 1), "weight").float()
            sc = a @ wv.T
            if bv is not None:
                sc = sc + bv
            sc = sc.to(torch.bfloat16).float()
        mx = sc.max(dim=1, keepdim=True).values
        hit = torch.where(torch.isnan(mx), torch.isnan(sc), sc == mx)
        tok = torch.where(hit, torch.arange(n)[None, :], n).min(dim=1).values
        self.view(out, torch.int64, (m,), (1,), "out_tokens").copy_(tok)
        return 0

    def fp8_rerank_topk(self, x, x_s, rows, k, w, w_s, sinv, n, cand, topk, out, stream):
        from oracle import linear as olin
        if rows == 0:
            return 0
        a = self.view(x, torch.bfloat16, (rows, k), (x_s, 1), "x").float().numpy()
        c = self.view(cand, torch.int64, (rows, topk), (topk, 1), "candidates").numpy()
        w8 = self.view(w, torch.uint8, (n, k), (w_s, 1), "weight").numpy()
        si = self.view(sinv, torch.float32, (n,), (1,), "scale_inv").numpy()
        toks = [olin.fp8_rerank_topk(a[r], c[r], w8.T, si) for r in range(rows)]
        self.view(out, torch.int64, (rows,), (1,), "out").copy_(torch.tensor(toks, dtype=torch.int64))
        return 0

    def quantize_int4_groups(self, w, w_dtype, w_s, rows, k, group, asym, out, out_s, scale_zeros, sz_s, stream):
        from oracle import linear as olin
        if rows < 0 or k <= 0 or group < 2 or group % 2 or k % group or sz_s < rows:
            return 1
        if rows == 0:
            return 0
        wv = self.load(self.view(w, _TORCH[w_dtype], (rows, k), (w_s, 1), "weight"), w_dtype).numpy()
        q, sc, z = olin.quantize_weight_int4(wv, group, "asymmetric" if asym else "symmetric")
        packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
        self.view(out, torch.uint8, (rows, k // 2), (out_s, 1), "packed").copy_(torch.from_numpy(packed))
        # the reference's scale_zeros [groups, N, 2] (sz_s pairs between groups)
        sz = self.view(scale_zeros, torch.bfloat16, (k // group, rows, 2), (2 * sz_s, 2, 1), "scale_zeros")
        sz[:, :, 0].copy_(torch.from_numpy(sc).to(torch.bfloat16).t())
        sz[:, :, 1].copy_(torch.from_numpy(z).to(torch.bfloat16).t())
        return 0

    def linear_int4_small_m(self, x, x_s, m, k, w, w_s, scale_zeros, group, sz_s, bias, n, epilogue, k_splits, ws,
                            counters, part_val, part_idx, out_tokens, y, y_s, stream):
        """W4A16 with each weight dequantised to bf16 ((q - 8) * s + z), fp32
        accumulation, the bf16 linear's bias / epilogue / greedy semantics;
        epilogue 3 writes the fp32 product as split partials (all of it in
        split 0) for the next RMSNorm to sum."""
        from oracle import linear as olin
        from oracle import numerics
        if m == 0 or n == 0:
            return 0
        n_out = n // 2 if epilogue == 1 else n
        if (m > 16 or (k // max(k_splits, 1)) % 256 or n_out % 16 or k % group or epilogue not in (0, 1, 2, 3)
                or sz_s < n or (epilogue == 3 and (bias or not ws))):
            return 1
        p = self.view(w, torch.uint8, (n, k // 2), (w_s, 1), "packed").numpy()
        q = np.empty((n, k), np.uint8)
        q[:, 0::2], q[:, 1::2] = p & 0xF, p >> 4
        sz = self.view(scale_zeros, torch.bfloat16, (k // group, n, 2), (2 * sz_s, 2, 1), "scale_zeros").float()
        sc, z = sz[:, :, 0].t().contiguous().numpy(), sz[:, :, 1].t().contiguous().numpy()
        deq = torch.from_numpy(numerics.bf16_round(olin.int4_dequant(q, sc, z, group).astype(np.float32)))
        a = self.view(x, torch.bfloat16, (m, k), (x_s, 1), "x").float()
        if epilogue == 3:
            part = self.view(ws, torch.float32, (k_splits, m, n), (m * n, n, 1), "partials")
            part.zero_()
            part[0].copy_((a.double() @ deq.double().T).float())
            self.calls.append("fdms_linear_int4_small_m:partials")
            return 0
        out = (a @ deq.T).to(torch.bfloat16).float()
        if bias:  # linear.py:475-477: bias added to the bf16 matmul result
            out = (out + self.view(bias, torch.bfloat16, (n,), (1,), "bias").float()).to(torch.bfloat16).float()
        if epilogue == 2:
            strips = n // 16
            self.view(part_val, torch.float32, (m, strips), (strips, 1), "part_val")
            self.view(part_idx, torch.int32, (m, strips), (strips, 1), "part_idx")
            mx = out.max(dim=1, keepdim=True).values
            hit = torch.where(torch.isnan(mx), torch.isnan(out), out == mx)
            tok = torch.where(hit, torch.arange(n)[None, :], n).min(dim=1).values
            self.view(out_tokens, torch.int64, (m,), (1,), "out_tokens").copy_(tok)
            return 0
        if epilogue == 1:
            g, u = out[:, :n_out], out[:, n_out:]
            out = torch.nn.functional.silu(g) * u
        self.view(y, torch.bfloat16, (m, n_out), (y_s, 1), "y").copy_(out.to(torch.bfloat16))
        return 0

    def prefill_attention(self, q, qs_t, qs_h, k, ks_t, ks_h, v, vs_t, vs_h, out, os_t, os_h, cu, num_seqs,
                          max_seqlen, hq, hkv, d, scale, stream):
        return self.prefill_attention_varlen(q, qs_t, qs_h, k, ks_t, ks_h, v, vs_t, vs_h, out, os_t, os_h, cu, cu,
                                             num_seqs, max_seqlen, hq, hkv, d, scale, stream)

    def prefill_attention_varlen(self, q, qs_t, qs_h, k, ks_t, ks_h, v, vs_t, vs_h, out, os_t, os_h, cu, cuk,
                                 num_seqs, max_seqlen, hq, hkv, d, scale, stream):
        """Causal softmax in float64, queries aligned to the end of their keys."""
        if num_seqs == 0 or max_seqlen <= 0:
            return 0
        c = self.view(cu, torch.int32, (num_seqs + 1,), (1,), "cu_seqlens_q").tolist()
        ck = self.view(cuk, torch.int32, (num_seqs + 1,), (1,), "cu_seqlens_k").tolist()
        t, tk = c[-1], ck[-1]
        if max(c[i + 1] - c[i] for i in range(num_seqs)) > max_seqlen:
            raise OutOfBounds(f"{self.name}: a sequence is longer than max_seqlen (rows would be skipped)")
        if any(ck[i + 1] - ck[i] < c[i + 1] - c[i] for i in range(num_seqs)):
            raise OutOfBounds(f"{self.name}: a sequence has fewer keys than queries")
        qv = self.view(q, torch.bfloat16, (t, hq, d), (qs_t, qs_h, 1), "q").float()
        kv_ = self.view(k, torch.bfloat16, (tk, hkv, d), (ks_t, ks_h, 1), "k").float()
        vv = self.view(v, torch.bfloat16, (tk, hkv, d), (vs_t, vs_h, 1), "v").float()
        ov = self.view(out, torch.bfloat16, (t, hq, d), (os_t, os_h, 1), "out")
        g = hq // hkv
        res = torch.empty((t, hq, d), dtype=torch.float32)
        for i in range(num_seqs):
            s0, s1, k0, k1 = c[i], c[i + 1], ck[i], ck[i + 1]
            n, nk = s1 - s0, k1 - k0
            mask = torch.ones(n, nk, dtype=torch.bool).tril(nk - n)
            for h in range(hq):
                sc = (qv[s0:s1, h].double() @ kv_[k0:k1, h // g].double().T) * scale
                sc = sc.masked_fill(~mask, float("-inf"))
                res[s0:s1, h] = (torch.softmax(sc, -1) @ vv[k0:k1, h // g].double()).float()
        ov.copy_(res.to(torch.bfloat16))
        return 0


class _HostEvent:
    """torch.cuda.Event for the emulator, whose copies complete when issued."""

    def __init__(self, *a, **k):
        pass

    def record(self, *a, **k):
        pass

    def synchronize(self):
        pass

    def query(self):
        return True


@contextmanager
def cpu_engine():
    """Run fastdms_amd's engine on CPU tensors through the emulator.

    Patches device placement (every "cuda" tensor lands on the CPU), the few
    torch.cuda calls the engine makes, and ``_native.call``; restores all of
    them on exit.  Graph capture is unavailable: use enforce_eager=True."""
    import fastdms_amd._native as nat
    import fastdms_amd.engine.model_runner as mr
    import fastdms_amd.layers.compact_attention as ca

    emu = Emulator()
    saved = []

    def patch(obj, name, value):
        saved.append((obj, name, getattr(obj, name)))
        setattr(obj, name, value)

    def strip(fn):
        def wrapped(*a, **k):
            k.pop("device", None)
            k.pop("pin_memory", None)
            return fn(*a, **k)
        return wrapped

    for fname in ("zeros", "full", "tensor", "ones", "arange", "randn", "zeros_like", "full_like", "ones_like",
                  "as_tensor"):
        patch(torch, fname, strip(getattr(torch, fname)))

    def poisoned(fn):
        """torch.empty* whose memory reads as NaN / -1 until written, so a kernel
        that consumes memory nobody wrote shows up in the results."""
        def wrapped(*a, **k):
            k.pop("device", None)
            k.pop("pin_memory", None)
            t = fn(*a, **k)
            if t.dtype != torch.bool and t.numel():
                t.view(-1).view(torch.uint8).fill_(0xFF) if t.is_contiguous() else t.fill_(float("nan"))
            return t
        return wrapped

    patch(torch, "empty", poisoned(torch.empty))
    patch(torch, "empty_like", poisoned(torch.empty_like))
    orig_to = torch.Tensor.to

    def to(self, *a, **k):
        a = tuple(x for x in a if not (isinstance(x, torch.device) or (isinstance(x, str))))
        k.pop("device", None)
        k.pop("non_blocking", None)
        return orig_to(self, *a, **k) if (a or k) else self

    patch(torch.Tensor, "to", to)
    orig_copy = torch.Tensor.copy_
    patch(torch.Tensor, "copy_", lambda self, src, non_blocking=False: orig_copy(self, src))
    def linear(x, w, b=None):  # fp32 accumulation then one bf16 rounding, as the oracle model computes
        y = x.float() @ w.float().T
        if b is not None:
            y = y + b.float()
        return y.to(x.dtype)

    patch(torch.nn.functional, "linear", linear)
    patch(torch.cuda, "set_device", lambda d: None)
    patch(torch.cuda, "current_device", lambda: 0)
    patch(torch.cuda, "synchronize", lambda *a, **k: None)
    patch(torch.cuda, "is_available", lambda: True)
    patch(torch.cuda, "Event", _HostEvent)
    patch(nat, "call", emu)
    patch(nat, "stream", lambda: 0)
    patch(nat, "require_cuda", lambda *a, **k: None)
    patch(ca, "_num_cus", lambda device: 256)
    import fastdms_amd.layers.linear as lin
    patch(lin, "_num_cus", lambda device: 256)
    orig_build = mr.build_synthetic_model
    patch(mr, "build_synthetic_model", lambda cfg, **k: orig_build(cfg, **{**k, "device": "cpu"}))
    # prefill FP8 GEMMs on this library's kernel (emulated): hipBLASLt's scaled
    # GEMM is a GPU library call, covered by the GPU tests
    patch(lin, "fp8_gemm_impl", lambda: "fdms")
    try:
        yield emu
    finally:
        for obj, name, value in reversed(saved):
            setattr(obj, name, value)
