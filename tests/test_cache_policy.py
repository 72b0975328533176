"""Hot-block cache policy on the CPU: the oracle's promotion and calibration
restatements against the reference tests' expectations and closed forms,
and the package's recency weights."""
import json
import os

import numpy as np
import torch

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_test_expectations.json")


def _fix():
    with open(FIX) as f:
        return json.load(f)


def test_calibration_recency_order(orc):
    c = _fix()["calibration_recency"]
    counts = orc.calibration_counts(np.zeros(c["num_blocks"], np.float32), c["active_blocks"], c["num_blocks"],
                                    c["recency_power"])
    order = c["expected_order_desc"]
    for hi, lo in zip(order, order[1:]):
        assert counts[hi] > counts[lo]
    # closed form: row r holds its block twice, weight ((r + 1) / 3) ** 2
    for r, b in enumerate([1, 2, 3]):
        w = np.float32(np.float32(r + 1) / np.float32(3)) ** np.float32(2)
        assert counts[b] == np.float32(w + w)
    assert counts[0] == 0 and counts[4:].sum() == 0


def test_recency_weights_package_match_oracle(orc):
    from next_step_ai_amd.slot_table import recency_weights

    for rows, power in ((1, 1.0), (3, 2.0), (17, 0.5), (256, 1.5)):
        w = recency_weights(rows, power).numpy()
        pos = np.arange(1, rows + 1, dtype=np.float32)
        ref = np.power(pos / np.float32(rows), np.float32(power)).astype(np.float32)
        assert w.dtype == np.float32
        np.testing.assert_allclose(w, ref, rtol=2e-7, atol=0)
        assert w[-1] == 1.0


def _argmin_plan(ids, scores, active, cap, novel):
    """The plan by the reference's one-at-a-time loop (RT:2576-2617), here as
    plain Python, for checking the oracle's restatement on many cases."""
    ids, scores = list(ids), [np.float32(v) for v in scores]
    active = max(0, min(active, len(ids), cap))
    novel = list(novel)[:cap]
    base = float(max(scores[:active])) + 1.0 if active > 0 else 1.0
    nxt, slots = active, []
    for i, b in enumerate(novel):
        if nxt < cap:
            s, nxt = nxt, nxt + 1
            active = max(active, s + 1)
        else:
            m = min(scores[:cap])
            s = scores.index(m)
        ids[s] = b
        scores[s] = np.float32(base + float(i + 1) * 1e-3)
        slots.append(s)
    return slots, ids, scores, active


def test_plan_oracle_matches_argmin_loop(orc):
    rng = np.random.default_rng(5)
    for _ in range(300):
        cap = int(rng.integers(1, 12))
        ids = rng.integers(0, 40, size=cap).tolist()
        scores = rng.integers(0, 4, size=cap).astype(np.float32).tolist()  # many ties
        active = int(rng.integers(0, cap + 1))
        novel = rng.choice(np.arange(40, 80), size=int(rng.integers(0, 2 * cap + 2)), replace=False).tolist()
        a = orc.plan_fixed_capacity_bank_update(ids, scores, active, cap, novel)
        b = _argmin_plan(ids, scores, active, cap, novel)
        assert a[0].tolist() == b[0] and a[1].tolist() == b[1] and a[3] == b[3]
        assert [np.float32(v) for v in a[2]] == b[2]


def test_promote_oracle_invariants(orc):
    rng = np.random.default_rng(6)
    NB, cap = 64, 20
    lookup = np.full(NB, -1)
    res = rng.choice(NB, size=cap - 4, replace=False)
    lookup[res] = np.arange(res.size)
    slot_block = np.concatenate([res, -np.ones(4, np.int64)])
    scores = np.zeros(cap, np.float32)
    active = res.size
    for step in range(40):
        sel = np.sort(rng.choice(NB, size=12, replace=False))
        old_max = scores[:active].max() if active else None
        novel = sel[lookup[sel] < 0]
        lookup, slot_block, scores, active, per = orc.promote_blocks(lookup, slot_block, scores, active, sel)
        # every novel block took a slot (12 <= capacity); a hit of the same
        # token may be evicted, as in the reference
        assert set(sel[per >= 0].tolist()) == set(novel.tolist())
        for e, b in enumerate(sel):
            assert per[e] == -1 or lookup[b] == per[e]
        # the lookup and the slots agree
        for s in range(active):
            assert lookup[slot_block[s]] == s
        assert (lookup >= 0).sum() == active
        if old_max is not None:
            for s in per[per >= 0]:
                assert scores[s] > old_max
