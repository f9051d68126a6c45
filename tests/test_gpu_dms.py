"""A1: extract_dms_eviction_decisions on the GPU vs the oracle (bit-exact)."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import from_values, require_gpu, values_of
from oracle import dms as odms
from oracle import numerics

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def test_threshold_edges_golden_and_out_param():
    require_gpu()
    from fastdms_amd.engine.dms import extract_dms_eviction_decisions
    g = GOLDEN["dms_threshold_edges"]
    vals = np.array(g["decision_values_f32_bits"], dtype=np.int32).view(np.float32)
    rng = np.random.default_rng(0)
    q = rng.standard_normal((11, 32, 64)).astype(np.float32)
    q[:, 0::4, -1] = vals[:, None]
    qd = torch.from_numpy(q).cuda()
    q_clean, evict = extract_dms_eviction_decisions(qd.clone(), num_kv_heads=8, num_qo_heads=32, head_dim=64,
                                                    alpha_scale=g["alpha_scale"], alpha_offset=g["alpha_offset"],
                                                    inplace=True)
    out = torch.empty((11, 8), device="cuda", dtype=torch.bool)
    q2, ev2 = extract_dms_eviction_decisions(qd.clone(), num_kv_heads=8, num_qo_heads=32, head_dim=64,
                                             alpha_scale=g["alpha_scale"], alpha_offset=g["alpha_offset"],
                                             inplace=True, out=out)
    torch.cuda.synchronize()
    exp_q, exp_ev = odms.extract_dms_eviction_decisions(q, num_kv_heads=8, num_qo_heads=32, head_dim=64,
                                                        alpha_scale=g["alpha_scale"], alpha_offset=g["alpha_offset"])
    assert evict.cpu().numpy()[:, 0].tolist() == g["expected_evict"]
    assert np.array_equal(evict.cpu().numpy(), exp_ev)
    assert np.array_equal(q_clean.cpu().numpy(), exp_q)
    assert ev2.data_ptr() == out.data_ptr()
    assert np.array_equal(ev2.cpu().numpy(), exp_ev) and np.array_equal(q2.cpu().numpy(), exp_q)


@pytest.mark.parametrize("scale,offset", [(10.0, 5.0), (100.0, 5.0), (-100.0, 5.0)])
def test_bf16_strided_qkv_view_matches_oracle(scale, offset):
    require_gpu()
    from fastdms_amd.engine.dms import extract_dms_eviction_decisions
    rng = np.random.default_rng(1)
    t, hq, hkv, d = 1000, 32, 8, 64
    qkv = numerics.cast(rng.standard_normal((t, (hq + 2 * hkv) * d)).astype(np.float32) * 0.7, numerics.DT_BF16)
    dev = from_values(qkv, numerics.DT_BF16)
    q_view = dev[:, :hq * d]  # strided view, like qkv.split (llama.py:93)
    q_clean, evict = extract_dms_eviction_decisions(q_view, num_kv_heads=hkv, num_qo_heads=hq, head_dim=d,
                                                    alpha_scale=scale, alpha_offset=offset, inplace=True)
    torch.cuda.synchronize()
    exp_q, exp_ev = odms.extract_dms_eviction_decisions(qkv[:, :hq * d], num_kv_heads=hkv, num_qo_heads=hq,
                                                        head_dim=d, alpha_scale=scale, alpha_offset=offset)
    assert np.array_equal(evict.cpu().numpy(), exp_ev)
    assert np.array_equal(values_of(q_clean), exp_q)
    assert np.array_equal(values_of(dev[:, hq * d:]), qkv[:, hq * d:])  # k/v untouched


def test_empty_and_cpu_inputs():
    require_gpu()
    from fastdms_amd.engine.dms import extract_dms_eviction_decisions
    q = torch.empty((0, 32, 64), device="cuda", dtype=torch.bfloat16)
    _, ev = extract_dms_eviction_decisions(q, num_kv_heads=8, num_qo_heads=32, head_dim=64, alpha_scale=10.0,
                                           alpha_offset=5.0)
    assert ev.shape == (0, 8)
    with pytest.raises(RuntimeError):
        extract_dms_eviction_decisions(torch.zeros((2, 32, 64)), num_kv_heads=8, num_qo_heads=32, head_dim=64,
                                       alpha_scale=10.0, alpha_offset=5.0)
    with pytest.raises(ValueError):
        extract_dms_eviction_decisions(q, num_kv_heads=7, num_qo_heads=32, head_dim=64, alpha_scale=10.0,
                                       alpha_offset=5.0)
