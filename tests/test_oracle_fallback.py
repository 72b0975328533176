"""The oracle's dequant-fallback leg (``y_fallback`` of orc_sparse_mlp): the
reference's fp16 rounding points (RT:5439-5488, self.dtype = fp16):

  R1  Wg, Wu = fp16(code * absmax)              (bitsandbytes dequant into fp16)
  R2  g, u   = fp16(x . Wg), fp16(x . Wu)        (F.linear, fp16 output)
  R3  s      = fp16(silu(g))                     (F.silu on fp16)
  R4  a      = fp16(s * u)
  R5  Wd     = fp16(fp16(code) * fp16(absmax))   (code and absmax cast to fp16, mul_)
  R6  y      = fp16(a . Wd)                      (round to nearest even)

Pinned two ways.  Known answers: ternary codes (-1, 0, +1), absmax chosen so
that the products and sums are exact rationals, integer x; the expected y is
computed with exact rational arithmetic at those rounding points, and
dropping any one of R1-R5, or rounding y toward zero instead of to nearest,
changes it (so a missing, extra or misplaced rounding point fails).  Random
small shapes: a numpy restatement of the same points (fp64 sums, single
roundings to fp16) equals the oracle bit for bit."""
import math
from fractions import Fraction

import numpy as np

QBS = 64
CODES = {0: Fraction(-1), 7: Fraction(0), 15: Fraction(1)}  # NF4 indices of -1, 0, +1


def f16(v: Fraction, toward_zero: bool = False) -> Fraction:
    """v rounded to fp16 (nearest, ties to even; or toward zero), exactly."""
    if v == 0:
        return Fraction(0)
    sign, a = (-1 if v < 0 else 1), abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    q = max(e - 10, -24)  # exponent of the fp16 ulp at a
    m = a / Fraction(2) ** q
    n = m.numerator // m.denominator
    frac = m - n
    if not toward_zero and (frac > Fraction(1, 2) or (frac == Fraction(1, 2) and n % 2 == 1)):
        n += 1
    r = n * Fraction(2) ** q
    assert r <= 65504, "test values stay finite"
    return sign * r


def silu(g: Fraction) -> Fraction:
    x = float(g)
    return Fraction(x / (1.0 + math.exp(-x)))


def model(x, gn, ga, un, ua, dn, da, drop=None, y_toward_zero=False):
    """y per output row: x [H] ints; gn/un [32A, H] code indices, ga/ua
    [32A, H/QBS] absmax; dn [H, 32A] indices, da [H, A] absmax (Fractions)."""
    R, H = gn.shape
    r1 = (lambda v: v) if drop == "R1" else f16
    r2 = (lambda v: v) if drop == "R2" else f16
    r3 = (lambda v: v) if drop == "R3" else f16
    r4 = (lambda v: v) if drop == "R4" else f16
    a = []
    for r in range(R):
        g = r2(sum(r1(CODES[gn[r, c]] * ga[r][c // QBS]) * x[c] for c in range(H)))
        u = r2(sum(r1(CODES[un[r, c]] * ua[r][c // QBS]) * x[c] for c in range(H)))
        a.append(r4(r3(silu(g)) * u))
    y = []
    for o in range(H):
        acc = Fraction(0)
        for r in range(R):
            c, am = CODES[dn[o, r]], da[o][r // 32]
            wd = c * am if drop == "R5" else f16(f16(c) * f16(am))
            acc += wd * a[r]
        y.append(f16(acc, toward_zero=y_toward_zero))
    return y


def pack(idx):
    """[rows, cols] nibble indices -> row-major packed bytes (even element high)."""
    flat = idx.reshape(-1).astype(np.uint8)
    return ((flat[0::2] << 4) | flat[1::2]).astype(np.uint8)


def _case(seed):
    rng = np.random.default_rng(seed)
    H, A = 128, 2
    R = 32 * A
    tern = np.array([0, 7, 15])
    gn, un = tern[rng.integers(0, 3, (R, H))], tern[rng.integers(0, 3, (R, H))]
    dn = tern[rng.integers(0, 3, (H, R))]
    # absmax values: fp32-exact rationals, some not fp16-representable (1 + 2^-12
    # rounds to 1), some small (2^-12 puts low bits into g), some plain
    pool = [Fraction(1), Fraction(1) + Fraction(1, 4096), Fraction(1, 4096), Fraction(3, 2048), Fraction(3, 4),
            Fraction(5, 16), Fraction(1, 8) + Fraction(1, 2 ** 16)]
    ga = [[pool[i] for i in rng.integers(0, len(pool), H // QBS)] for _ in range(R)]
    ua = [[pool[i] for i in rng.integers(0, len(pool), H // QBS)] for _ in range(R)]
    da = [[pool[i] for i in rng.integers(0, len(pool), A)] for _ in range(H)]
    x = [int(v) for v in rng.integers(-3, 4, H)]
    return H, A, x, gn, ga, un, ua, dn, da


def _oracle_fallback(orc, H, A, x, gn, ga, un, ua, dn, da):
    f32 = lambda rows: np.array([[float(v) for v in r] for r in rows], dtype=np.float32)  # noqa: E731
    for rows in (ga, ua, da):
        assert all(Fraction(float(np.float32(float(v)))) == v for r in rows for v in r)  # exact in fp32
    x16 = np.array(x, dtype=np.float16).view(np.uint16).reshape(1, H)
    gp = pack(gn).reshape(A, 32 * H // 2)
    upk = pack(un).reshape(A, 32 * H // 2)
    # down [H, A, 16]: block b's 32 columns of row o
    dp = np.stack([pack(dn[:, 32 * b:32 * b + 32]).reshape(H, 16) for b in range(A)], axis=1)
    al = np.arange(A, dtype=np.int32).reshape(1, A)
    _, yf = orc.sparse_mlp(x16, al, gp, f32(ga).reshape(A, -1), upk, f32(ua).reshape(A, -1), dp, f32(da), qbs=QBS,
                           want_exact=False, want_fallback=True)
    return [Fraction(float(v)) for v in yf[0].view(np.float16).astype(np.float64)]


def test_fallback_known_answers_every_rounding_point(orc):
    for seed in range(40):
        case = _case(seed)
        H, A, x, gn, ga, un, ua, dn, da = case
        want = model(x, gn, ga, un, ua, dn, da)
        variants = {d: model(x, gn, ga, un, ua, dn, da, drop=d) for d in ("R1", "R2", "R3", "R4", "R5")}
        variants["R6 toward zero"] = model(x, gn, ga, un, ua, dn, da, y_toward_zero=True)
        if all(v != want for v in variants.values()):
            break
    else:
        raise AssertionError("no seed makes every rounding point visible")
    assert _oracle_fallback(orc, *case) == want, f"seed {seed}"


def test_fallback_matches_numpy_restatement(orc):
    """Random NF4 weights (all 16 codes), random absmax and x at small
    shapes: the numpy restatement (fp64 sums, single roundings to fp16 by
    numpy's direct conversions) equals the oracle bit for bit."""
    code32 = orc.nf4_code().astype(np.float32)
    code16 = code32.astype(np.float16)
    for seed, (H, A, qbs) in enumerate([(128, 3, 64), (256, 5, 64), (512, 2, 128)]):
        rng = np.random.default_rng(100 + seed)
        R = 32 * A
        gn, un = rng.integers(0, 16, (R, H)), rng.integers(0, 16, (R, H))
        dn = rng.integers(0, 16, (H, R))
        ga = (np.abs(rng.standard_normal((R, H // qbs))) * 0.05 + 1e-3).astype(np.float32)
        ua = (np.abs(rng.standard_normal((R, H // qbs))) * 0.05 + 1e-3).astype(np.float32)
        da = (np.abs(rng.standard_normal((H, A))) * 0.05 + 1e-3).astype(np.float32)
        x16 = rng.standard_normal(H).astype(np.float16)

        def deq16(n, am):  # R1: fp32 product, one rounding to fp16
            return (code32[n] * np.repeat(am, qbs, axis=1)).astype(np.float16)

        g16 = (deq16(gn, ga).astype(np.float64) @ x16.astype(np.float64)).astype(np.float16)  # R2
        u16 = (deq16(un, ua).astype(np.float64) @ x16.astype(np.float64)).astype(np.float16)
        gd = g16.astype(np.float64)
        s16 = (gd / (1.0 + np.exp(-gd))).astype(np.float16)  # R3
        a16 = (s16.astype(np.float32) * u16.astype(np.float32)).astype(np.float16)  # R4 (exact fp32 product)
        wd16 = (code16[dn].astype(np.float32)
                * np.repeat(da.astype(np.float16), 32, axis=1).astype(np.float32)).astype(np.float16)  # R5
        y16 = (wd16.astype(np.float64) @ a16.astype(np.float64)).astype(np.float16)  # R6

        dp = np.stack([pack(dn[:, 32 * b:32 * b + 32]).reshape(H, 16) for b in range(A)], axis=1)
        _, yf = orc.sparse_mlp(x16.view(np.uint16).reshape(1, H), np.arange(A, dtype=np.int32).reshape(1, A),
                               pack(gn).reshape(A, -1), ga.reshape(A, -1), pack(un).reshape(A, -1),
                               ua.reshape(A, -1), dp, da, qbs=qbs, want_exact=False, want_fallback=True)
        assert np.array_equal(yf[0], y16.view(np.uint16)), (H, A, qbs)
