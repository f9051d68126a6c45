"""Kernels around the DMS path that the model runs every layer: MFMA operand
layout, RMSNorm (+ residual, + per-head strided rows), SiLU*up, the FP8
embedding gather, row argmax, dense causal prefill attention and the strided
decode-slot preparation."""
import numpy as np
import pytest
import torch

from helpers import require_gpu
from oracle import attention as oatt

pytestmark = pytest.mark.gpu


def _bf16(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16)


def test_mfma_operand_layout():
    """v_mfma_f32_16x16x32_bf16 with the lane layout the prefill kernel assumes.
    Small integers keep every product and sum exact, so the check is exact."""
    require_gpu()
    from fastdms_amd import _native as nat
    rng = np.random.default_rng(0)
    a = rng.integers(-3, 4, (16, 32)).astype(np.float32)
    b = rng.integers(-3, 4, (32, 16)).astype(np.float32)
    ad, bd = _bf16(a).cuda(), _bf16(b).cuda()
    c = torch.empty((16, 16), device="cuda", dtype=torch.float32)
    nat.call("fdms_mfma_probe", ad.data_ptr(), bd.data_ptr(), c.data_ptr(), nat.stream())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(c.cpu().numpy(), a @ b)


def _rms_ref(x, w, eps, residual=None):
    """layernorm.py:19-40 in fp32 on the CPU; returns (out, residual_out)."""
    x = x.float()
    res_out = None
    if residual is not None:
        x = x + residual.float()
        res_out = x.to(torch.bfloat16)
    inv = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return (x * inv).to(torch.bfloat16).float().mul(w.float()).to(torch.bfloat16), res_out


def _ulp_close(got: torch.Tensor, want: torch.Tensor, what: str):
    """bf16 results may differ by one unit in the last place (fp32 reduction order)."""
    g, w = got.float().cpu(), want.float().cpu()
    tol = w.abs() * 2.0 ** -7 + 1e-6
    bad = (g - w).abs() > tol
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} elements beyond 1 bf16 ulp"


@pytest.mark.parametrize("rows,hidden", [(1, 2048), (37, 256), (9, 4096), (3, 8192), (100, 64), (513, 128)])
def test_rmsnorm(rows, hidden):
    require_gpu()
    from fastdms_amd.layers.layernorm import rms_norm
    g = torch.Generator().manual_seed(rows * 7 + hidden)
    x = torch.randn(rows, hidden, generator=g).to(torch.bfloat16)
    r = torch.randn(rows, hidden, generator=g).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16)
    out = rms_norm(x.cuda(), w.cuda(), 1e-5)
    want, _ = _rms_ref(x, w, 1e-5)
    _ulp_close(out, want, "rmsnorm")
    out, res = rms_norm(x.cuda(), w.cuda(), 1e-5, residual=r.cuda())
    want, want_res = _rms_ref(x, w, 1e-5, residual=r)
    torch.cuda.synchronize()
    assert torch.equal(res.cpu(), want_res), "residual_out must be bf16(x + residual) exactly"
    _ulp_close(out, want, "rmsnorm+residual")


def test_rmsnorm_per_head_strided_view():
    """Qwen3 q_norm / k_norm: RMSNorm of every head of a [T, H, D] view that
    lives inside the fused qkv rows (qwen3.py:82-197)."""
    require_gpu()
    from fastdms_amd.layers.layernorm import rms_norm
    t, hq, hkv, d = 13, 8, 2, 128
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(t, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    qkv_d = qkv.cuda()
    k_view = qkv_d[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    out = rms_norm(k_view, w.cuda(), 1e-6)
    want, _ = _rms_ref(qkv[:, hq * d:(hq + hkv) * d].reshape(t * hkv, d), w, 1e-6)
    _ulp_close(out.reshape(t * hkv, d), want, "per-head rmsnorm")
    torch.cuda.synchronize()
    assert torch.equal(qkv_d.cpu(), qkv), "the input view must not be modified"


@pytest.mark.parametrize("rows,f", [(1, 8192), (29, 512), (8, 12288)])
def test_silu_mul(rows, f):
    require_gpu()
    from fastdms_amd.layers.activation import silu_and_mul
    g = torch.Generator().manual_seed(rows + f)
    x = (3 * torch.randn(rows, 2 * f, generator=g)).to(torch.bfloat16)
    out = silu_and_mul(x.cuda())
    xf = x.float()
    want = (torch.nn.functional.silu(xf[:, :f]) * xf[:, f:]).to(torch.bfloat16)
    _ulp_close(out, want, "silu_mul")


@pytest.mark.parametrize("vocab,dim,n", [(128256, 2048, 8), (1000, 4096, 3000), (512, 264, 17)])
def test_fp8_embedding_gather_matches_the_oracle(vocab, dim, n):
    """(f)2: the FP8 embedding gather equals the oracle's rows bit for bit
    (bf16(bf16(e4m3fn row) * bf16(scale_inv)), embed_head.py:422-432; the
    table quantised by quantize_fp8_rows as the reference's FP8 table), for
    repeated ids, the first and last rows and the LM-head-sized table; an id
    outside the table gives a NaN row without touching memory outside it."""
    require_gpu()
    from fastdms_amd.layers.embed_head import VocabParallelEmbedding
    from oracle import linear as olin
    from oracle import numerics
    g = torch.Generator().manual_seed(vocab + dim)
    w = (torch.randn(vocab, dim, generator=g) * 0.05).to(torch.bfloat16)
    emb = VocabParallelEmbedding(vocab, dim)
    emb.weight.data = w.cuda()
    emb.quantize_embedding_to_fp8()
    ids = torch.randint(0, vocab, (n,), generator=g)
    ids[0], ids[-1] = 0, vocab - 1
    if n > 4:
        ids[2] = ids[1]
    got = emb(ids.cuda()).cpu()
    codes, sinv = olin.quantize_weight_to_fp8(w.float().numpy())   # W8^T [dim, vocab], [1, vocab]
    rows = numerics.e4m3fn_decode(codes.T[ids.numpy()]).astype(np.float32)
    s = torch.from_numpy(sinv.reshape(-1)[ids.numpy()]).to(torch.bfloat16).float().reshape(-1, 1)
    want = (torch.from_numpy(rows).to(torch.bfloat16).float() * s).to(torch.bfloat16)
    assert torch.equal(got, want)
    bad = torch.tensor([3, -1, vocab, 1], device="cuda")
    y = emb(bad).cpu()
    assert torch.isnan(y[1].float()).all() and torch.isnan(y[2].float()).all()
    assert torch.equal(y[0], emb(torch.tensor([3], device="cuda")).cpu()[0])


@pytest.mark.parametrize("vocab,hidden,n", [(128256, 2048, 8), (151936, 4096, 8), (1000, 264, 37)])
def test_embedding_rms_norm_equals_gather_then_rmsnorm(vocab, hidden, n):
    """fdms_embedding_rmsnorm (the decode step's bf16 gather + first
    input_layernorm in one launch): the gathered rows equal F.embedding bit for
    bit, the normalised rows equal fdms_rmsnorm of them bit for bit (the same
    kernel) and the oracle's RMSNorm (layernorm.py:16-28) within one bf16 ulp;
    ids outside the table give NaN rows in both outputs."""
    require_gpu()
    from fastdms_amd.layers.embed_head import embedding_rms_norm
    from fastdms_amd.layers.layernorm import rms_norm
    g = torch.Generator().manual_seed(vocab + n)
    table = (torch.randn((vocab, hidden), generator=g) * 0.5).to(torch.bfloat16).cuda()
    w = (1.0 + 0.2 * torch.randn(hidden, generator=g)).to(torch.bfloat16).cuda()
    ids = torch.randint(0, vocab, (n,), generator=g).cuda()
    h, rows = embedding_rms_norm(ids, table, w, 1e-5)
    want_rows = torch.nn.functional.embedding(ids, table)
    want_h = rms_norm(want_rows, w, 1e-5)
    torch.cuda.synchronize()
    assert torch.equal(rows, want_rows)
    assert torch.equal(h, want_h)
    ref, _ = _rms_ref(want_rows.cpu(), w.cpu(), 1e-5)
    _ulp_close(h, ref, "embedding rmsnorm")
    bad = ids.clone()
    bad[0], bad[-1] = -1, vocab
    h2, rows2 = embedding_rms_norm(bad, table, w, 1e-5)
    torch.cuda.synchronize()
    for t in (h2, rows2):
        assert torch.isnan(t[0].float()).all() and torch.isnan(t[-1].float()).all()
        assert torch.equal(t[1:-1], (h if t is h2 else rows)[1:-1])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_argmax_rows_matches_torch(dtype):
    """Lowest index on ties; NaN wins (torch.argmax semantics), so the id is
    always a valid token."""
    require_gpu()
    from fastdms_amd import _native as nat
    g = torch.Generator().manual_seed(11)
    n = 128256
    x = torch.randn(7, n, generator=g).to(dtype)
    x[1, 5000] = x[1, 90000] = 50.0           # tie: lowest index
    x[2, :] = -float("inf")                  # all -inf: index 0
    x[3, 77] = float("nan")                  # NaN beats every number
    x[4, 1000] = x[4, 600] = float("nan")    # lowest NaN
    x[5, n - 1] = 99.0                       # last element
    x[6, :] = float("nan")
    xd = x.cuda()
    out = torch.empty(7, device="cuda", dtype=torch.int64)
    nat.call("fdms_argmax_rows", xd.data_ptr(), nat.dtype_code(dtype), xd.stride(0), 7, n, out.data_ptr(),
             nat.stream())
    torch.cuda.synchronize()
    assert out.cpu().tolist() == [int(torch.argmax(x[i].float())) for i in range(7)]
    assert out.cpu().tolist()[1:7] == [5000, 0, 77, 600, n - 1, 0]


@pytest.mark.parametrize("d,lens,hq,hkv,ramp", [
    (64, [1, 63, 64, 65, 200, 517], 8, 2, 0.0),
    (128, [129, 700, 2], 8, 2, 0.0),
    (64, [31, 160, 1500], 4, 4, 0.0),      # G = 1 (packed kernel, 128 positions per workgroup)
    (128, [95, 300], 8, 4, 0.0),           # G = 2
    (64, [77, 400], 6, 2, 0.0),            # G = 3 (per-head kernel)
    (64, [2100, 130], 8, 2, 3.0),          # keys scaled up along the sequence: the running max keeps growing
    (128, [900], 8, 2, 3.0),
])
def test_prefill_attention_vs_oracle(d, lens, hq, hkv, ramp):
    """Causal varlen attention (flash_attn_varlen_func semantics, attention.py:85-92)
    on q/k/v that are strided views of fused qkv rows, GQA hq/hkv.  ramp > 0
    scales key t of each sequence by 1 + ramp * t / len, so later blocks raise
    the softmax max (the kernel's rescale path)."""
    require_gpu()
    from fastdms_amd.layers.attention import prefill_attention
    t = sum(lens)
    rng = np.random.default_rng(d + 7 * hq + hkv)
    qkv = rng.standard_normal((t, (hq + 2 * hkv) * d)).astype(np.float32)
    if ramp:
        pos = np.concatenate([np.arange(n) / n for n in lens]).astype(np.float32)
        qkv[:, hq * d:(hq + hkv) * d] *= (1.0 + ramp * pos)[:, None]
    qkv_b = _bf16(qkv)
    qkv_v = qkv_b.float().numpy()
    q = qkv_v[:, :hq * d].reshape(t, hq, d)
    k = qkv_v[:, hq * d:(hq + hkv) * d].reshape(t, hkv, d)
    v = qkv_v[:, (hq + hkv) * d:].reshape(t, hkv, d)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    want = oatt.causal_prefill_attention(q, k, v, cu)
    dq = qkv_b.cuda()
    qd = dq[:, :hq * d].view(t, hq, d)
    kd = dq[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    vd = dq[:, (hq + hkv) * d:].view(t, hkv, d)
    out = prefill_attention(qd, kd, vd, torch.from_numpy(cu).cuda(), max(lens), d ** -0.5)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err <= 2e-2, f"max-abs-rel error {err:.3g}"
    # bf16 output: most elements are within a couple of bf16 ulps of the exact value
    assert np.mean(np.abs(got - want) <= 2 ** -7 * np.abs(want) + 4e-3) > 0.99


@pytest.mark.parametrize("hq,hkv", [(8, 2), (8, 4), (4, 4)])
def test_prefill_attention_query_tiles_agree(hq, hkv, monkeypatch):
    """The packed kernel with two or four 16-row query tiles per wave (four
    is selectable at head_dim 64): each row's arithmetic is the same, only a
    workgroup's span of positions differs, so the outputs are bit-identical,
    and both match the oracle.  Keys grow along the sequence, so the lazy
    rescale runs after the first block."""
    require_gpu()
    from fastdms_amd.layers.attention import prefill_attention
    d, lens = 64, [1, 700, 1500, 64, 129]
    t = sum(lens)
    rng = np.random.default_rng(hq * 10 + hkv)
    qkv = rng.standard_normal((t, (hq + 2 * hkv) * d)).astype(np.float32)
    pos = np.concatenate([np.arange(n) / n for n in lens]).astype(np.float32)
    qkv[:, hq * d:(hq + hkv) * d] *= (1.0 + 3.0 * pos)[:, None]
    qkv_b = _bf16(qkv)
    qkv_v = qkv_b.float().numpy()
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    want = oatt.causal_prefill_attention(qkv_v[:, :hq * d].reshape(t, hq, d),
                                         qkv_v[:, hq * d:(hq + hkv) * d].reshape(t, hkv, d),
                                         qkv_v[:, (hq + hkv) * d:].reshape(t, hkv, d), cu)
    dq = qkv_b.cuda()
    qd = dq[:, :hq * d].view(t, hq, d)
    kd = dq[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    vd = dq[:, (hq + hkv) * d:].view(t, hkv, d)
    outs = {}
    for qt in ("2", "4"):
        monkeypatch.setenv("FASTDMS_AMD_PREFILL_QT", qt)
        outs[qt] = prefill_attention(qd, kd, vd, torch.from_numpy(cu).cuda(), max(lens), d ** -0.5)
        torch.cuda.synchronize()
    assert torch.equal(outs["2"], outs["4"])
    got = outs["4"].float().cpu().numpy()
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err <= 2e-2, f"max-abs-rel error {err:.3g}"
    assert np.mean(np.abs(got - want) <= 2 ** -7 * np.abs(want) + 4e-3) > 0.99


@pytest.mark.parametrize("d,lens,cuts,hq,hkv", [
    (64, [300, 517, 64], [128, 100, 0], 8, 2),     # G = 4, prefix a multiple of 64 / not / none
    (128, [700, 129], [511, 128], 8, 2),
    (64, [1500, 90], [1499, 37], 4, 4),           # G = 1, a one-row chunk
    (128, [400], [3], 8, 4),                      # G = 2
    (64, [333, 200], [200, 1], 6, 2),             # G = 3 (per-head kernel)
])
def test_prefill_attention_chunk_over_retained_prefix(d, lens, cuts, hq, hkv):
    """A prompt chunk attending to the retained earlier chunks plus itself
    (flash_attn_varlen_func with cu_seqlens_k, queries aligned to the end of
    the keys): equal to the oracle's varlen form, and to the same rows of the
    unchunked prefill to bf16 rounding."""
    require_gpu()
    from fastdms_amd.layers.attention import prefill_attention
    rng = np.random.default_rng(d + hq + sum(cuts))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    t = int(cu[-1])
    q = _bf16(rng.standard_normal((t, hq, d)).astype(np.float32))
    k = _bf16(rng.standard_normal((t, hkv, d)).astype(np.float32))
    v = _bf16(rng.standard_normal((t, hkv, d)).astype(np.float32))
    rows = np.concatenate([np.arange(cu[i] + cuts[i], cu[i + 1]) for i in range(len(lens))])
    cq = np.concatenate([[0], np.cumsum([n - c for n, c in zip(lens, cuts)])]).astype(np.int32)
    qc = q[torch.from_numpy(rows)].contiguous()
    want = oatt.causal_prefill_attention(qc.float().numpy(), k.float().numpy(), v.float().numpy(), cq,
                                         cu_seqlens_k=cu)
    out = prefill_attention(qc.cuda(), k.cuda(), v.cuda(), torch.from_numpy(cq).cuda(),
                            int(max(n - c for n, c in zip(lens, cuts))), d ** -0.5,
                            cu_seqlens_k=torch.from_numpy(cu).cuda())
    full = prefill_attention(q.cuda(), k.cuda(), v.cuda(), torch.from_numpy(cu).cuda(), max(lens), d ** -0.5)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err <= 2e-2, f"max-abs-rel error {err:.3g}"
    assert np.mean(np.abs(got - want) <= 2 ** -7 * np.abs(want) + 4e-3) > 0.99
    same = np.abs(got - full.float().cpu().numpy()[rows])
    assert np.mean(same <= 2 ** -7 * np.abs(want) + 4e-3) > 0.99


def test_prepare_decode_metadata_strided_slot_output():
    """slot_out as a [:, :B] view of a wider [L, max_seqs, H] buffer (the decode
    graph's static buffer): only the view's elements are written."""
    require_gpu()
    from fastdms_amd import _native as nat
    L, S, H, B, start = 3, 8, 2, 3, 2
    g = torch.Generator().manual_seed(2)
    base = torch.randint(0, 10000, (L, S, H), generator=g, dtype=torch.int32)
    live = torch.randint(1, 500, (L, S, H), generator=g, dtype=torch.int32)
    slot_buf = torch.full((L, S, H), -7, dtype=torch.int32)
    bd, ld, sd = base.cuda(), live.cuda(), slot_buf.cuda()
    bv, lv, sv = bd[:, start:start + B], ld[:, start:start + B], sd[:, :B]
    nat.call("fdms_prepare_decode_metadata", bv.data_ptr(), *bv.stride(), lv.data_ptr(), *lv.stride(), sv.data_ptr(),
             *sv.stride(), L, B, H, nat.stream())
    torch.cuda.synchronize()
    want_slot = slot_buf.clone()
    want_slot[:, :B] = base[:, start:start + B] + live[:, start:start + B]
    want_live = live.clone()
    want_live[:, start:start + B] += 1
    assert torch.equal(sd.cpu(), want_slot)
    assert torch.equal(ld.cpu(), want_live)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,stride", [(1001, 1003), (77, 80), (4104, 4104), (151936, 151936), (3, 8)])
def test_argmax_rows_tails_and_unaligned_rows(dtype, n, stride):
    """Vector path with a scalar tail, and the scalar path for rows that are
    not 16-byte aligned; values drawn from a few levels so ties are common."""
    require_gpu()
    from fastdms_amd import _native as nat
    g = torch.Generator().manual_seed(n)
    rows = 5
    buf = torch.randint(0, 7, (rows, stride), generator=g).to(dtype)
    x = buf[:, :n]
    xd = buf.cuda()[:, :n]
    out = torch.empty(rows, device="cuda", dtype=torch.int64)
    nat.call("fdms_argmax_rows", xd.data_ptr(), nat.dtype_code(dtype), xd.stride(0), rows, n, out.data_ptr(),
             nat.stream())
    torch.cuda.synchronize()
    assert out.cpu().tolist() == [int(torch.argmax(x[i].float())) for i in range(rows)]
