"""Writes reference_test_expectations.json: inputs and expected outputs that
the reference's own tests assert for the slot-table host logic.  Nothing is
imported from the reference; the literals are transcribed from its tests
(file:line in each entry), and the down-column case applies the slicing
rule those tests assert (tests/test_down_proj_col_cache.py:131-146) to a
small deterministic byte pattern."""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def down_columns_case():
    # tests/test_down_proj_col_cache.py:21-29 use H_OUT=64, I_IN=256, BLOCK_SIZE=8,
    # QBS=16; a smaller instance of the same geometry keeps the fixture short.
    h_out, i_in, bs, qbs = 4, 32, 8, 16
    bytes_per_row, bytes_per_cblk, absmax_per_row = i_in // 2, bs // 2, i_in // qbs
    packed = [(o * 37 + c * 11 + 5) % 256 for o in range(h_out) for c in range(bytes_per_row)]
    absmax = [0.25 * (o * absmax_per_row + a + 1) for o in range(h_out) for a in range(absmax_per_row)]
    blocks = [0, 3, 1]
    exp_packed = [[[packed[o * bytes_per_row + b * bytes_per_cblk + j] for j in range(bytes_per_cblk)]
                   for b in blocks] for o in range(h_out)]
    exp_absmax = [[absmax[o * absmax_per_row + (b * bs) // qbs] for b in blocks] for o in range(h_out)]
    return {
        "source": "tests/test_down_proj_col_cache.py:114-146 (shapes [H_OUT, n, BLOCK_SIZE/2], [H_OUT, n]; "
                  "packed = raw_2d[:, b*BLOCK_SIZE/2 : +BLOCK_SIZE/2], absmax = absmax_2d[:, (b*BLOCK_SIZE)//QBS])",
        "h_out": h_out, "in_features": i_in, "block_size": bs, "qbs": qbs, "blocks": blocks,
        "packed": packed, "absmax": absmax, "expected_packed": exp_packed, "expected_absmax": exp_absmax,
    }


def main():
    doc = {
        "plan_fixed_capacity_bank_update": {
            "source": "tests/test_throughput_contract.py:308-321",
            "existing_block_ids": [10, 11, -1], "existing_scores": [5.0, 1.0, 0.0], "active_count": 2,
            "capacity": 3, "novel_blocks": [20, 21],
            "expected_active_count": 3, "expected_slots": [2, 1], "expected_block_ids": [10, 21, 20],
            "expected_scores_above": {"1": 5.0, "2": 5.0},
        },
        "calibration_recency": {
            "source": "tests/test_throughput_contract.py:261-287",
            "num_blocks": 8, "recency_power": 2.0, "active_blocks": [[1, 1], [2, 2], [3, 3]],
            "expected_order_desc": [3, 2, 1],
        },
        "down_column_gather": down_columns_case(),
        "hot_cold_partition": {
            "source": "tests/test_prewarm_col_cache.py:66-72, 133-139, 169-190, 227-240 (hot iff lookup >= 0)",
            "cases": [
                {"hot_blocks": [0, 1, 2], "total_blocks": 8, "routing": [0, 1, 2, 3, 4, 5], "expected_cold": [3, 4, 5]},
                {"hot_blocks": [], "total_blocks": 8, "routing": [0, 1, 2, 3, 4, 5],
                 "expected_cold": [0, 1, 2, 3, 4, 5]},
                {"hot_blocks": [0, 1, 2], "total_blocks": 8, "routing": [0, 1, 2], "expected_cold": []},
            ],
        },
    }
    with open(os.path.join(HERE, "reference_test_expectations.json"), "w") as f:
        json.dump(doc, f, indent=1)


if __name__ == "__main__":
    main()
