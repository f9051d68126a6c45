"""Pin the DMS decision oracle on the reference's literal vectors; test the
host-side metadata loader of the product (pure host logic)."""
import json
from pathlib import Path

import numpy as np

from oracle import dms as odms

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def test_threshold_edges_match_golden():
    g = GOLDEN["dms_threshold_edges"]
    vals = np.array(g["decision_values_f32_bits"], dtype=np.int32).view(np.float32)
    got = odms.dms_decide(vals, g["alpha_scale"], g["alpha_offset"])
    assert got.tolist() == g["expected_evict"]
    # the three hand-picked edge tokens: ==0.05 keeps, nextafter up evicts, down keeps
    assert got[:3].tolist() == [False, True, False]


def test_negative_scale_branch_is_affine_threshold():
    v = np.array([-1.0, -0.05, 0.0, 0.05, 1.0], dtype=np.float32)
    got = odms.dms_decide(v, -100.0, 5.0)  # v * -100 - 5 > 0  <=>  v < -0.05
    assert got.tolist() == [True, False, False, False, False]


def test_dms_interface_checks():
    g = GOLDEN["dms_interface"]
    t, hkv, gq, d = g["tokens"], g["num_kv_heads"], g["q_per_kv"], g["head_dim"]
    thr = g["alpha_offset"] / g["alpha_scale"]
    q = np.zeros((t, hkv, gq, d), dtype=np.float32)
    for tok, head, delta in g["set"]:
        q[tok, head, 0, -1] = thr + delta
    q_clean, evict = odms.extract_dms_eviction_decisions(q.reshape(t, hkv * gq, d), num_kv_heads=hkv,
                                                         num_qo_heads=hkv * gq, head_dim=d,
                                                         alpha_scale=g["alpha_scale"], alpha_offset=g["alpha_offset"])
    live = odms.build_dms_live_mask(evict.T[None], current_position=t - 1, window_size=g["window_size"])
    borrowed = q_clean.reshape(t, hkv, gq, d)[:, :, 0, -1]
    checks = {
        "evict_true_token0_head0": bool(evict[0, 0]),
        "evict_false_token1_head0": not bool(evict[1, 0]),
        "evict_true_token2_head3": bool(evict[2, 3]),
        "borrowed_neuron_zeroed": float(np.abs(borrowed).max()) == 0.0,
        "old_evicted_token_not_live": not bool(live[0, 0, 0]),
        "old_non_evicted_token_live": bool(live[0, 0, 1]),
        "recent_evicted_token_live": bool(live[0, 3, 2]),
    }
    assert checks == g["expected"]


def test_extract_zeroes_only_the_borrowed_channel():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((7, 32, 64)).astype(np.float32)
    qc, ev = odms.extract_dms_eviction_decisions(q, num_kv_heads=8, num_qo_heads=32, head_dim=64,
                                                 alpha_scale=10.0, alpha_offset=5.0)
    mask = np.ones_like(q, dtype=bool)
    mask[:, 0::4, 63] = False
    assert np.array_equal(qc[mask], q[mask])
    assert (qc[:, 0::4, 63] == 0).all()
    assert np.array_equal(ev, q[:, 0::4, 63] > np.float32(0.5))


def test_product_metadata_loader_resolves_hf_aliases(tmp_path):
    from fastdms_amd.engine.dms import load_dms_metadata
    g = GOLDEN["dms_metadata_hf_aliases"]
    d = tmp_path / "qwen3-dms"
    d.mkdir()
    (d / "config.json").write_text(json.dumps(g["config"]))
    m = load_dms_metadata(d)
    got = {k: getattr(m, k) for k in g["expected"]}
    assert got == g["expected"]
    assert m.source_path.endswith("config.json")


def test_product_metadata_loader_defaults_and_precedence(tmp_path):
    from fastdms_amd.engine.dms import load_dms_metadata
    g = GOLDEN["dms_metadata_defaults"]
    model = tmp_path / "run" / "final"
    model.mkdir(parents=True)
    (tmp_path / "run" / "training_log.json").write_text(json.dumps({"config": {}}))
    m = load_dms_metadata(model)
    assert (m.window_size, m.alpha_scale, m.alpha_offset) == (g["window_size"], g["alpha_scale"], g["alpha_offset"])
    assert m.source_kind == "parent_training_log"
    (model / "dms_metadata.json").write_text(json.dumps({"config": {"window_size": 7}}))
    m2 = load_dms_metadata(model)
    assert m2.source_kind == "packaged_metadata" and m2.window_size == 7 and m2.packaged_metadata_found
