"""Pins the oracle router (RT:4209-4238, RT:4311-4352 restated with the exact
precision contract) by brute force with exact rationals, and compares it
with torch's fp16 CPU ops (informative: same values wherever no score sits
on an fp16 rounding boundary)."""
from fractions import Fraction

import numpy as np
import torch


def _f(h):
    return Fraction(float(np.uint16(h).view(np.float16)))


def _round16(fr: Fraction) -> int:
    """Exact rational -> fp16 bits via an independent path: numpy's correctly
    rounded float64 -> float16 when the value is exactly a double, else a
    bracket search over fp16 values."""
    d = float(fr)
    if Fraction(d) == fr:
        with np.errstate(over="ignore"):
            return int(np.float64(d).astype(np.float16).view(np.uint16))
    # not a double: find neighbours lo < fr < hi among fp16 values, pick the nearer (ties impossible here)
    cand = np.float64(d).astype(np.float16)
    lo = np.nextafter(cand, np.float16(-np.inf))
    hi = np.nextafter(cand, np.float16(np.inf))
    best = min((lo, cand, hi), key=lambda v: abs(Fraction(float(v)) - fr))
    return int(np.float16(best).view(np.uint16))


def _brute_route(x, enc_w, enc_b, sw, sb, k, btk=None, dbn=None, legacy=False):
    R, H = enc_w.shape
    lat = []
    for r in range(R):
        s = sum((_f(x[c]) * _f(enc_w[r, c]) for c in range(H)), Fraction(0)) + (_f(enc_b[r]) if enc_b is not None else 0)
        lat.append(_round16(s))
    lat = np.array(lat, dtype=np.uint16)
    if btk is not None and btk < R:
        mags = [abs(float(np.uint16(v).view(np.float16))) for v in lat]
        order = sorted(range(R), key=lambda i: (-mags[i], i))
        keep = set(order[:btk])
        lat = np.array([v if i in keep else (v & 0x8000) for i, v in enumerate(lat)], dtype=np.uint16)
    NB = sw.shape[0]
    scores = []
    for j in range(NB):
        la = [(_f(v & 0x7FFF) if legacy else _f(v)) for v in lat]
        s = sum((la[r] * _f(sw[j, r]) for r in range(R)), Fraction(0))
        if not legacy and sb is not None:
            s += _f(sb[j])
        h = _round16(s)
        if not legacy and (h & 0x8000):
            h = 0
        if dbn is not None:
            d16 = np.float32(dbn[j]).astype(np.float16)
            h = int((np.float32(np.uint16(h).view(np.float16)) * np.float32(d16)).astype(np.float16).view(np.uint16))
        scores.append(h)
    scores = np.array(scores, dtype=np.uint16)
    vals = scores.view(np.float16).astype(np.float64)
    sel = sorted(range(NB), key=lambda j: (-vals[j], j))[:k]
    return lat, scores, np.array(sel, dtype=np.int32)


def _r16(rng, shape, std):
    return (rng.standard_normal(shape) * std).astype(np.float16).view(np.uint16)


def test_route_matches_brute_force(orc):
    rng = np.random.default_rng(0)
    for trial, (H, R, NB, k, btk) in enumerate([(24, 4, 17, 5, None), (40, 6, 23, 23, 3), (16, 3, 9, 1, None)]):
        x = _r16(rng, H, 1.0)
        ew, eb = _r16(rng, (R, H), 0.3), _r16(rng, R, 0.1)
        sw, sb = _r16(rng, (NB, R), 0.3), _r16(rng, NB, 0.1)
        want = _brute_route(x, ew, eb, sw, sb, k, btk=btk)
        got = orc.route(x, ew, eb, sw, sb, k, basis_top_k=btk)
        for w, g in zip(want, got):
            assert np.array_equal(w, g), trial


def test_route_legacy_and_norm_match_brute_force(orc):
    rng = np.random.default_rng(1)
    H, R, NB, k = 20, 5, 15, 4
    x = _r16(rng, H, 1.0)
    ew, eb = _r16(rng, (R, H), 0.3), _r16(rng, R, 0.1)
    sw = _r16(rng, (NB, R), 0.3) & 0x7FFF
    dbn = (rng.random(NB) * 3).astype(np.float32)
    want = _brute_route(x, ew, eb, sw, None, k, dbn=dbn, legacy=True)
    got = orc.route(x, ew, eb, sw, None, k, down_block_norm=dbn, legacy_abs=True)
    for w, g in zip(want, got):
        assert np.array_equal(w, g)


def test_ties_resolve_to_lowest_index(orc):
    H, R, NB = 8, 2, 12
    x = np.zeros(H, dtype=np.uint16)
    ew = np.zeros((R, H), dtype=np.uint16)
    sw = np.zeros((NB, R), dtype=np.uint16)
    sb = np.array([1, 3, 3, 2, 3, 1, 2, 3, 0, 3, 2, 1], dtype=np.float16).view(np.uint16)
    _, _, sel = orc.route(x, ew, None, sw, sb, 7)
    assert sel.tolist() == [1, 2, 4, 7, 9, 3, 6]
    assert orc.topk_lowest_index(sb, 7).tolist() == sel.tolist()
    # clamp_min(0): negative scores tie at zero
    sbn = np.array([-1, -2, 0.5, -3, -0.0, 0], dtype=np.float16).view(np.uint16)
    _, sc, sel = orc.route(x, ew, None, np.zeros((6, R), np.uint16), sbn, 4)
    assert sc.view(np.float16).tolist() == [0, 0, 0.5, 0, 0, 0]
    assert sel.tolist() == [2, 0, 1, 3]


def test_informative_agreement_with_torch_fp16(orc):
    """torch's fp16 CPU linear accumulates differently and torch.topk breaks
    ties arbitrarily; the selected sets still agree almost always."""
    rng = np.random.default_rng(2)
    H, R, NB, k = 1024, 32, 256, 24
    agree_sets = 0
    trials = 8
    for _ in range(trials):
        x = _r16(rng, H, 1.0)
        ew, eb = _r16(rng, (R, H), 0.02), _r16(rng, R, 0.02)
        sw, sb = _r16(rng, (NB, R), 0.02), _r16(rng, NB, 0.02)
        lat_o, sc_o, sel_o = orc.route(x, ew, eb, sw, sb, k)
        t = lambda a: torch.from_numpy(a.view(np.float16).copy())  # noqa: E731
        lat_t = torch.nn.functional.linear(t(x).reshape(1, H), t(ew), t(eb))
        sc_t = torch.nn.functional.linear(lat_t, t(sw), t(sb)).clamp_min(0.0)
        sel_t = sc_t.topk(k, dim=-1).indices[0].numpy()
        lat_match = np.mean(lat_t[0].numpy().view(np.uint16) == lat_o)
        assert lat_match > 0.9
        agree_sets += set(sel_t.tolist()) == set(sel_o.tolist())
    assert agree_sets >= trials - 2
