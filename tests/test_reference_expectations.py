"""The oracle and the package's host-side layout logic against the
expectations the reference's own tests assert (tests/golden fixture).  The
device slot plan and the hot/cold rule are checked against the same fixture
in tests/test_gpu_cache.py."""
import json
import os

import numpy as np
import torch

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_test_expectations.json")


def _fix():
    with open(FIX) as f:
        return json.load(f)


def _check_plan(case, slots, ids, scores, active):
    assert int(active) == case["expected_active_count"]
    assert [int(v) for v in slots] == case["expected_slots"]
    assert [int(v) for v in ids] == case["expected_block_ids"]
    for i, lo in case["expected_scores_above"].items():
        assert float(scores[int(i)]) > lo


def test_fixed_capacity_plan_oracle(orc):
    c = _fix()["plan_fixed_capacity_bank_update"]
    _check_plan(c, *orc.plan_fixed_capacity_bank_update(c["existing_block_ids"], c["existing_scores"],
                                                        c["active_count"], c["capacity"], c["novel_blocks"]))


def test_down_column_gather_oracle(orc):
    c = _fix()["down_column_gather"]
    p, a = orc.gather_down_columns(np.array(c["packed"], dtype=np.uint8), np.array(c["absmax"], dtype=np.float32),
                                   c["blocks"], c["h_out"], c["in_features"], c["qbs"], block_size=c["block_size"])
    assert p.shape == (c["h_out"], len(c["blocks"]), c["block_size"] // 2) and p.dtype == np.uint8
    assert a.shape == (c["h_out"], len(c["blocks"])) and a.dtype == np.float32
    assert p.tolist() == c["expected_packed"]
    assert a.tolist() == c["expected_absmax"]


def test_active_layout_oracle_and_package(orc):
    """Ordered blocks are the ascending unique in-range ids (CPU unique,
    RT:4873); active_local inverts them; each flat_mask row has 32 ones per
    own valid block (RT:4883-4901); neurons are the blocks' 32-row ranges."""
    from next_step_ai_amd.layout import build_sparse_active_layout

    rng = np.random.default_rng(7)
    for rows, k, nb in [(1, 9, 40), (3, 6, 20), (4, 5, 12)]:
        ab = rng.integers(-2, nb + 3, size=(rows, k))
        ordered, local, mask, neurons = orc.active_layout(ab, nb)
        valid = ab[(ab >= 0) & (ab < nb)]
        assert ordered.tolist() == sorted(set(valid.tolist()))
        for t in range(rows):
            for i in range(k):
                b = ab[t, i]
                if 0 <= b < nb:
                    assert ordered[local[t, i]] == b
                else:
                    assert local[t, i] == -1
            own = set(ab[t][(ab[t] >= 0) & (ab[t] < nb)].tolist())
            assert mask[t].sum() == 32 * len(own)
        assert neurons.tolist() == [32 * b + r for b in ordered.tolist() for r in range(32)]
        po, pl, pm, _ = build_sparse_active_layout(active_blocks=torch.from_numpy(ab), rows=rows, block_size=32,
                                                   max_valid_blocks=nb, dtype=torch.float32,
                                                   device=torch.device("cpu"))
        assert po.tolist() == ordered.tolist()
        assert pl.numpy().tolist() == local.tolist()
        assert np.array_equal(pm.numpy(), mask)


def test_hot_cold_partition_oracle(orc):
    """The oracle's hot/cold split against the reference tests' cases: hot iff
    the lookup is >= 0 (slot 0 is hot: a `> 0` rule fails the first case)."""
    for case in _fix()["hot_cold_partition"]["cases"]:
        lookup = -np.ones(case["total_blocks"], dtype=np.int64)
        for slot, b in enumerate(case["hot_blocks"]):
            lookup[b] = slot
        pos, slots, cold, cold_mask = orc.partition_by_lookup(lookup, case["routing"])
        assert cold.tolist() == case["expected_cold"]
        assert [int(case["routing"][p]) for p in pos] == [b for b in case["routing"] if b not in case["expected_cold"]]
        assert [int(s) for s in slots] == [int(lookup[case["routing"][p]]) for p in pos]
        assert int(cold_mask.sum()) == len(case["expected_cold"])
