"""Write tests/golden/reference_vectors.json.

The fixture holds the literal inputs and expected outputs that the
reference's own tests and checks assert (shisa-ai/FastDMS
tests/test_compact_kv.py and benchmarks/check_dms_interface.py), transcribed
as data with the file:line each case comes from.  Nothing here imports or
runs the reference.  The DMS threshold edge case is completed with torch's
own CPU float32 comparison (the reference's CPU branch, dms.py:222-227, is a
plain torch comparison), so its expected flags come from the library routine
the reference itself calls.

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
from pathlib import Path

import torch

OUT = Path(__file__).with_name("reference_vectors.json")


def dms_threshold_edges():
    # test_compact_kv.py:441-483 — 11 tokens, q[:, 0::4, -1] = linspace(-0.1, 0.2),
    # token 0 exactly 0.05, token 1 nextafter(0.05, 1), token 2 nextafter(0.05, 0).
    vals = torch.linspace(-0.1, 0.2, 11, dtype=torch.float32)
    vals[0] = 0.05
    vals[1] = torch.nextafter(torch.tensor(0.05), torch.tensor(1.0))
    vals[2] = torch.nextafter(torch.tensor(0.05), torch.tensor(0.0))
    evict = (vals > (5.0 / 100.0)).tolist()
    return {
        "source": "tests/test_compact_kv.py:441-483; expected via torch CPU fp32 compare (dms.py:224-225)",
        "alpha_scale": 100.0,
        "alpha_offset": 5.0,
        "decision_values_f32_bits": [int(x) for x in vals.view(torch.int32).tolist()],
        "expected_evict": evict,
    }


def main():
    data = {
        "pack_compact_kv": {
            "source": "tests/test_compact_kv.py:60-81",
            "k_shape": [1, 5, 2, 4],
            "k": "arange(40) reshaped; v = k + 100",
            "live_mask": [[[True, False, True, False, True], [False, True, True, False, False]]],
            "expected_compact_shape": [5, 4],
            "expected_base_offsets": [[0, 3]],
            "expected_live_counts": [[3, 2]],
            "expected_token_positions": [0, 2, 4, 1, 2],
        },
        "allocator_alloc_free": {
            "source": "tests/test_compact_kv.py:162-187",
            "num_layers": 3, "num_kv_heads": 2, "capacity_tokens": 64, "max_model_len": 32,
            "prompt_tokens": 3, "max_tokens": 5,
            "expected_max_capacity_per_lh": 8,
            "expected_base_offsets": [[-1, -1], [-1, -1], [-1, -1]],
            "expected_range_capacity": [[0, 0], [0, 0], [0, 0]],
            "expected_free_tokens": 192,
            "expected_free_ranges_after_free": [[[0, 64]], [[0, 64]], [[0, 64]]],
        },
        "layer_major_active_slots": {
            "source": "tests/test_compact_kv.py:189-222",
            "num_layers": 2, "num_kv_heads": 2, "capacity_tokens": 32, "max_model_len": 16, "max_active_seqs": 2,
            "seqs": [[3, 4], [2, 4]],
            "expected_active_slots": [0, 1],
            "expected_contiguous_start_in_order": 0,
            "expected_contiguous_start_reversed": None,
            "third_seq": [1, 4],
            "expected_third_slot_after_free_first": 0,
        },
        "prepare_decode_metadata": {
            "source": "tests/test_compact_kv.py:225-249",
            "num_layers": 2, "num_kv_heads": 2, "capacity_tokens": 32, "max_model_len": 16,
            "prompt_tokens": 2, "max_tokens": 4, "live_per_head": 2,
            "expected_base_offsets": [[[0, 6]], [[0, 6]]],
            "expected_slot_mapping": [[[2, 8]], [[2, 8]]],
            "expected_live_counts": [[[3, 3]], [[3, 3]]],
            "expected_state_live_counts": [[3, 3], [3, 3]],
            "expected_max_live_count_is_max_capacity": 6,
        },
        "record_decisions_layer_major": {
            "source": "tests/test_compact_kv.py:252-282",
            "num_layers": 2, "num_kv_heads": 2, "capacity_tokens": 32, "max_model_len": 16, "max_active_seqs": 2,
            "initial_live": 1,
            "evictions": [[[True, False], [False, True]], [[False, False], [True, True]]],
            "positions": [10, 20],
            "expected_stats": {"eviction_decisions_true": 4, "eviction_decisions_total": 8},
            "expected_positions_slot0": [[10, 10], [10, 10]],
            "expected_positions_slot1": [[20, 20], [20, 20]],
        },
        "layer_head_live_counts": {
            "source": "tests/test_compact_kv.py:323-339",
            "num_layers": 2, "num_kv_heads": 2, "capacity_tokens": 32, "max_model_len": 16,
            "prompt_tokens": 3, "max_tokens": 5,
            "live_counts": [[2, 3], [4, 5]],
        },
        "emulated_stride_mask": {
            "source": "tests/test_compact_kv.py:342-362",
            "num_layers": 2, "num_kv_heads": 2, "num_tokens": 8, "stride": 3, "recent_tokens": 2,
            "expected": [[[p >= 6 or (p + l + h) % 3 == 0 or p == 7 for p in range(8)] for h in range(2)]
                         for l in range(2)],
        },
        "dms_interface": {
            "source": "benchmarks/check_dms_interface.py:28-67",
            "tokens": 4, "num_kv_heads": 8, "q_per_kv": 4, "head_dim": 64,
            "alpha_scale": 100.0, "alpha_offset": 5.0, "window_size": 1,
            "set": [[0, 0, 0.01], [1, 0, -0.01], [2, 3, 0.01]],
            "expected": {"evict_true_token0_head0": True, "evict_false_token1_head0": True,
                         "evict_true_token2_head3": True, "borrowed_neuron_zeroed": True,
                         "old_evicted_token_not_live": True, "old_non_evicted_token_live": True,
                         "recent_evicted_token_live": True},
        },
        "dms_metadata_hf_aliases": {
            "source": "tests/test_compact_kv.py:116-143",
            "config": {"model_type": "qwen3", "dms_window_size": 512, "dms_alpha_scale": 100.0,
                       "dms_initial_alpha_offset": 5.0, "dms_cr": 8, "max_position_embeddings": 40960},
            "expected": {"source_kind": "hf_config_dms", "packaged_metadata_found": False, "window_size": 512,
                         "alpha_scale": 100.0, "alpha_offset": 5.0, "target_cr": 8, "context_len": 40960},
        },
        "dms_threshold_edges": dms_threshold_edges(),
        "dms_metadata_defaults": {
            "source": "fastdms/engine/dms.py:70-75",
            "window_size": 256, "alpha_scale": 100.0, "alpha_offset": 5.0,
        },
    }
    OUT.write_text(json.dumps(data, indent=1, sort_keys=True) + "\n", encoding="utf-8")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
