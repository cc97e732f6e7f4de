"""Writes reference_kats.json: the known-answer vectors held by the reference's
own tests, transcribed as data (inputs and expected outputs), with the
reference file:line each one comes from.  Run: python tests/golden/make_fixtures.py
"""
import json
from pathlib import Path

values = [2., -1., 2., 0., -0., 3., -3., 1., 1., 2., -1., 0., 4., 4., -4., 0.]
ids = [115, 102, 108, 101, 109, 103, 114, 100, 113, 104, 112, 105, 111, 106, 110, 107]

KATS = {
    "sort_stable_signed_zero": {
        "source": "sglang/srt/layers/attention/v1_native/test_fused_grouping_small.py:88-99",
        "values": ["-0.0" if (v == 0 and str(v).startswith("-")) else v for v in values],
        "ids": ids,
        "expected": [ids[i] for i in sorted(range(16), key=lambda i: (-values[i], i))],
    },
    "sort_split_chain": {
        "source": "sglang/srt/layers/attention/v1_native/test_fused_grouping_small.py:101-115",
        "perm": list(range(100, 116)),
        "unit0": [1, -1] * 8,
        "anchor": [101, 100],
        "expected": list(range(100, 116, 2)) + list(range(101, 116, 2)),
    },
    "sort_special_pattern": {
        "source": "experiments/v1_kernel_opt_20261022/test_sort_cub.py:12-13",
        "pattern": ["0.0", "-0.0", "1.0", "1.0", "-1.0", "-inf", "inf", "0.0"],
        "repeat": 512,
    },
    "gather_small": {
        "source": "sglang/srt/layers/attention/v1_native/test_gather_slots_small.py:12-43",
        "req": [5, 1, 7, 0, 6, 2],
        "ids": [[0, 2, -1], [4, 1, 4]],
        "physical": [[5, 7, -1], [6, 1, 6]],
        "pool_slots": 8, "heads": 2, "dim": 128,
        "k_rule": "arange(8*2*128).reshape(8,2,128) as bf16",
        "v_rule": "(-arange(8*2*128)-16).reshape(8,2,128) as bf16",
    },
    "gather_workspace": {
        "source": "sglang/srt/layers/attention/v1_native/test_gather_slots_small.py:45-61",
        "ids_rule": "(arange(4096) % 6).reshape(2, 2048); second call flips columns, head 1",
    },
    "page_lifecycle": {
        "source": "sglang/srt/layers/attention/v1_deepseek/test_page_management_and_tail_small.py:14-57",
        "capacity": 16,
        "tmp_rule": "page p: 8448 bytes equal to p",
        "mapping_rule": "arange(1024).reshape(16, 64)",
        "first_table": list(range(15, -1, -1)),
        "count_after_first": 0,
        "refs_after_first": 1,
        "refs_after_second": 2,
        "refs_after_release_a": 1,
        "count_after_release_b": 16,
        "centers_rule": "2 x 8448 bytes: first 8192 = 7, scales = 1.25",
    },
    "fingerprint_hand": {
        "source": "experiments/fine_pool_shared_20261021/MLA_INDEX_KERNELS_INPUT_OUTPUT.md:231",
        "bytes_head": [1, 2], "members_head": [10, 20], "hash": [3141875, 26276919],
    },
    "fingerprint_words": {
        "source": "experiments/v1_kernel_opt_20261022/KERNEL_IMPLEMENTATION_DETAILS.md:308-321",
        "word_bytes": [1, 2, 3, 4], "weighted": 30,
    },
    "page_match_modes": {
        "source": "experiments/v1_kernel_opt_20261022/bench_pages.py:20-28",
        "miss": "all -1",
        "hit": "live pages 1..16 hold the temp pages -> match = 1..16",
        "collision": "page 0 has equal hashes and members but one byte flipped -> still 1..16",
    },
    "shared_tail": {
        "source": "sglang/srt/layers/attention/v1_deepseek/test_page_management_and_tail_small.py:59-88",
        "rows": 4, "np": 18, "cap": 1, "scratch": 3,
        "lens": [1100, 1100, 1101, 1101], "owners": [0, 0, 2, 2],
        "native_rule": "page p: fp8 bytes encode p+1 (e4m3fn), scales arange(64)+1",
        "nt_rule": "arange(17, -1, -1) for every row",
        "fill": 255,
        "fine_table": [[1, 2, 3], [1, 2, 3], [7, 8, 9], [7, 8, 9]],
    },
    "route_example": {
        "source": "sglang/srt/layers/attention/v1_deepseek/example_v1_query_single_head.py:11-41; "
                  "README_QUERY_SINGLE_HEAD_EXAMPLE.md:23",
        "B": 1024, "P": 128, "CAP": 128, "TAKE": 40, "N": 4097, "TOP": 2048, "WINDOW": 64, "seed": 19,
        "first_selected": [48, 49, 50, 51, 52, 53, 54, 55],
        "fine_candidates": 2688,
    },
}


def example_permutations():
    """The example's two page permutations: the first two draws of a CPU
    torch.Generator seeded 19 (native table over P pages, then the reordered
    pool over CAP pages), stored as data so the tests need no RNG replay."""
    import torch
    gen = torch.Generator().manual_seed(KATS["route_example"]["seed"])
    native = torch.randperm(KATS["route_example"]["P"], generator=gen).tolist()
    reorder = torch.randperm(KATS["route_example"]["CAP"], generator=gen).tolist()
    return native, reorder


KATS["route_example"]["native_pages"], KATS["route_example"]["reorder_pages"] = example_permutations()

if __name__ == "__main__":
    out = Path(__file__).with_name("reference_kats.json")
    out.write_text(json.dumps(KATS, indent=1) + "\n")
    print(out)
