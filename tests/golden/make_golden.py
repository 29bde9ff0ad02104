"""Write tests/golden/reference_known_answers.json.

The fixtures are the literal inputs and expected outputs that light-vllm's own
tests assert (transcribed data, cited file:line relative to the light-vllm
tree).  No reference code is imported or run; nothing here reads the reference
at run time.  Re-run with ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import json
from pathlib import Path

OUT = Path(__file__).with_name("reference_known_answers.json")


def known_answers() -> dict:
    query_keys = [[[20 + 8 * t + 4 * h + d for d in range(4)] for h in range(2)] for t in range(5)]
    prefix_keys = [[[8 * t + 4 * h + d for d in range(4)] for h in range(2)] for t in range(2)]
    return {
        "slot_mapping": [
            {
                "source": "tests/test_paged_attention.py:121-130",
                "block_tables": [[2, 0], [1, 3]],
                "num_computed_tokens": [0, 1],
                "query_lengths": [3, 2],
                "reserved": [3, 2],
                "block_size": 2,
                "expected": [4, 5, 0, 3, 6],
            },
            {
                "source": "tests/test_paged_attention.py:448-462 (unused lookahead is reserved, not written)",
                "block_tables": [[0, 1, 2]],
                "num_computed_tokens": [0],
                "query_lengths": [1],
                "reserved": [3],
                "block_size": 1,
                "num_blocks": 3,
                "expected": [0],
            },
            {
                "source": "docs/diagrams/light-vllm-paged-attention-token-path.html (worked example)",
                "block_tables": [[7, 2]],
                "num_computed_tokens": [5],
                "query_lengths": [2],
                "reserved": [2],
                "block_size": 4,
                "expected": [9, 10],
            },
        ],
        "linear_detection": {
            "source": "tests/test_paged_attention.py:133-146",
            "linear": [[-1, 0, 1]],
            "tree": [[-1, 0, 0]],
        },
        "visibility_packing": {
            "source": "tests/test_paged_attention.py:149-175",
            "layouts": [[-1, 0, 0], [-1, 0]],
            "block_tables": [[0, 1], [2]],
            "num_computed_tokens": [0, 0],
            "query_start_loc": [0, 3, 5],
            "request_indices": [0, 0, 0, 1, 1],
            "visibility_start": [0, 9, 13],
            "visibility": [True, False, False, True, True, False, True, False, True, True, False, True, True],
        },
        "query_layout": {
            "source": "tests/test_query_layout.py:28-45",
            "parents": [-1, 0, 0, 2],
            "prefix_length": 5,
            "positions": [5, 6, 6, 7],
            "visibility": [
                [True, False, False, False],
                [True, True, False, False],
                [True, False, True, False],
                [True, False, True, True],
            ],
            "append_draft": {"num_inputs": 2, "draft_parents": [-1, 0, 0], "expected": [-1, 0, 1, 2, 2]},
        },
        "visible_positions": {
            "source": "tests/test_paged_attention.py:84-118 (visible_indices of the tree test)",
            "parents": [-1, 0, 0, 2],
            "num_computed_tokens": 0,
            "expected": [[0], [0, 1], [0, 2], [0, 2, 3]],
        },
        "compact": {
            "source": "tests/test_paged_attention.py:178-228",
            "num_blocks": 4,
            "block_size": 2,
            "num_kv_heads": 2,
            "head_size": 4,
            "prefix_keys": prefix_keys,
            "prefix_value_offset": 100,
            "prefix_slots": [2, 3],
            "parents": [-1, 0, 0, 2, 3],
            "block_table": [1, 3, 0, 2],
            "num_computed_tokens": 2,
            "num_readonly_prefix_blocks": 1,
            "query_keys": query_keys,
            "query_value_offset": 100,
            "retained": [0, 2, 4],
            "destination_slots": [6, 7, 0],
            "expected_moved": 2,
        },
        "contiguous_compact": {
            "source": "tests/test_kv_cache.py:553-573",
            "history": [1, 2, 10, 30, 50],
            "sequence": [1, 2, 10, 20, 30, 40, 50],
            "num_computed_tokens": 2,
            "retained": [0, 2, 4],
            "expected": [1, 2, 10, 30, 50],
        },
        "validation_errors": [
            {
                "source": "tests/test_paged_attention.py:312-320",
                "block_tables": [[0]], "num_computed_tokens": [1], "query_lengths": [2],
                "num_blocks": 4, "block_size": 2, "match": "block table does not cover",
            },
            {
                "source": "tests/test_paged_attention.py:323-339",
                "block_tables": [[4, 0]], "num_computed_tokens": [2], "query_lengths": [1],
                "num_blocks": 4, "block_size": 2, "match": "out-of-range physical block",
            },
            {
                "source": "tests/test_paged_attention.py:342-357",
                "block_tables": [[0, 0]], "num_computed_tokens": [2], "query_lengths": [1],
                "num_blocks": 4, "block_size": 2, "match": "aliases a physical block within one request",
            },
            {
                "source": "tests/test_paged_attention.py:360-376",
                "block_tables": [[0], [0]], "num_computed_tokens": [0, 1], "query_lengths": [1, 1],
                "num_blocks": 4, "block_size": 2, "match": "alias a physical block across requests",
            },
            {
                "source": "tests/test_paged_attention.py:412-433 (one-sided sharing)",
                "block_tables": [[0, 1], [0, 2]], "num_computed_tokens": [2, 2], "query_lengths": [1, 1],
                "readonly": [1, 0], "num_blocks": 5, "block_size": 2,
                "match": "alias a physical block across requests",
            },
            {
                "source": "tests/test_paged_attention.py:412-433 (misaligned sharing)",
                "block_tables": [[0, 1, 2], [3, 0, 4]], "num_computed_tokens": [4, 4], "query_lengths": [1, 1],
                "readonly": [1, 2], "num_blocks": 5, "block_size": 2,
                "match": "alias a physical block across requests",
            },
            {
                "source": "tests/test_paged_attention.py:436-445",
                "block_tables": [[0]], "num_computed_tokens": [1], "query_lengths": [1],
                "readonly": [1], "num_blocks": 2, "block_size": 2,
                "match": "exceed the computed prefix",
            },
            {
                "source": "tests/test_paged_attention.py:465-491 (case 1)",
                "block_tables": [[0, 0]], "num_computed_tokens": [0], "query_lengths": [1],
                "num_blocks": 4, "block_size": 2, "match": "unused physical blocks",
            },
            {
                "source": "tests/test_paged_attention.py:465-491 (case 2)",
                "block_tables": [[0], [1, 0]], "num_computed_tokens": [0, 0], "query_lengths": [1, 1],
                "num_blocks": 4, "block_size": 2, "match": "unused physical blocks",
            },
        ],
        "valid_shared_prefix": {
            "source": "tests/test_paged_attention.py:379-409",
            "block_tables": [[0, 1], [0, 2]], "num_computed_tokens": [2, 2], "query_lengths": [1, 1],
            "readonly": [1, 1], "num_blocks": 4, "block_size": 2,
        },
        "speculative_compact_contract": {
            "source": "tests/test_speculative.py:185-236",
            "note": "retained = formal inputs + accepted path; compact returns the moved-token count",
            "cases": [
                {"inputs": 2, "accepted": [0, 1], "retained": [0, 1, 2, 3]},
                {"inputs": 2, "accepted": [0], "retained": [0, 1, 2]},
                {"inputs": 2, "accepted": [], "retained": [0, 1]},
            ],
        },
    }


def main() -> None:
    OUT.write_text(json.dumps(known_answers(), indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
