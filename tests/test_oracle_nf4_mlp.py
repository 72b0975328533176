"""Pins the oracle's NF4 format, quantiser and MLP math.

NF4 quantisation itself (bitsandbytes==0.49.1 quantize_4bit / double quant)
cannot be run here: bitsandbytes is not installed, so its bit-exact outputs
are parity unpinned; the invariants below fix what the published algorithm
determines (code table, nearest-code rule, packing order, round trip).
"""
import numpy as np


def test_nf4_code_table_invariants(orc):
    c = orc.nf4_code()
    assert c.size == 16
    assert c[0] == -1.0 and c[7] == 0.0 and c[15] == 1.0
    assert np.all(np.diff(c) > 0)


def test_nf4_packing_order_and_nearest_code(orc):
    c = orc.nf4_code().astype(np.float64)
    # one quant block of 64 holding every code value exactly (absmax 1)
    w = np.tile(c, 4).astype(np.float32)
    pk, am = orc.nf4_quantize(w, 64)
    assert am.tolist() == [1.0]
    nib = np.empty(64, dtype=np.int64)
    nib[0::2] = pk >> 4   # even element -> high nibble
    nib[1::2] = pk & 0xF
    assert nib.tolist() == list(range(16)) * 4
    # random values: the code is the nearest one (ties only at exact midpoints)
    rng = np.random.default_rng(0)
    w = (rng.standard_normal(64 * 500) * 0.02).astype(np.float32)
    pk, am = orc.nf4_quantize(w, 64)
    nib = np.empty(w.size, dtype=np.int64)
    nib[0::2] = pk >> 4
    nib[1::2] = pk & 0xF
    v = (w.reshape(-1, 64) * (np.float32(1) / am[:, None])).reshape(-1).astype(np.float64)
    dist = np.abs(v[:, None] - c[None, :])
    best = np.argmin(dist, axis=1)
    near_tie = np.sort(dist, axis=1)[:, 1] - np.sort(dist, axis=1)[:, 0] < 1e-6
    assert np.all((best == nib) | near_tie)
    assert np.array_equal(am, np.abs(w.reshape(-1, 64)).max(axis=1))


def test_nf4_round_trip_error_bound(orc):
    rng = np.random.default_rng(1)
    w = (rng.standard_normal(1 << 16) * 0.02).astype(np.float32)
    pk, am = orc.nf4_quantize(w, 64)
    wd = orc.nf4_dequant(pk, am, w.size, 64)
    c = orc.nf4_code().astype(np.float64)
    half_gap = np.max(np.diff(c)) / 2
    err = np.abs(wd - w).reshape(-1, 64)
    assert np.all(err <= half_gap * am[:, None] * (1 + 1e-6))
    # dequant is code[nib] * absmax in fp32
    nib_hi = pk[0] >> 4
    assert wd[0] == np.float32(c[nib_hi]) * am[0]
    zero = orc.nf4_quantize(np.zeros(64, np.float32), 64)
    assert zero[1][0] == 0 and np.all(zero[0] == 0x77)


def test_dynamic_map_and_double_quant(orc):
    m = orc.dynamic_map_signed()
    assert m.size == 256 and np.all(np.diff(m) >= 0)
    assert m[-1] == 1.0 and 0.0 in m and m[0] < -0.9
    assert np.count_nonzero(m > 0) == 128 and np.count_nonzero(m < 0) == 127
    rng = np.random.default_rng(2)
    absmax = np.abs(rng.standard_normal(3000) * 0.05).astype(np.float32) + 0.01
    q, a2, off = orc.double_quant(absmax, m)
    assert q.dtype == np.uint8 and a2.size == (3000 + 255) // 256
    back = orc.double_dequant(q, a2, off, m)
    assert np.max(np.abs(back - absmax)) <= np.max(a2) * np.max(np.diff(m)) / 2 * 1.001 + 1e-7
    # the dequantised value is fl32(fl32(map[q] * absmax2) + offset)
    i = 1234
    assert back[i] == np.float32(np.float32(m[q[i]] * a2[i // 256]) + np.float32(off))


def _dense(orc, packed, absmax, rows, cols, qbs=64):
    """Dense fp64 weights decoded with numpy: element 2i is the high nibble
    of byte i, value code[nib] * absmax[e // qbs] (exact in fp64)."""
    packed = np.asarray(packed, dtype=np.uint8).reshape(-1)
    nib = np.empty(packed.size * 2, dtype=np.int64)
    nib[0::2] = packed >> 4
    nib[1::2] = packed & 0xF
    code = orc.nf4_code().astype(np.float64)
    scale = np.repeat(np.asarray(absmax, dtype=np.float64).reshape(-1), qbs)
    return (code[nib] * scale).reshape(rows, cols)


def test_sparse_mlp_all_blocks_equals_dense_llama_mlp(orc):
    """With every block selected the sparse MLP is the textbook
    down(silu(gate(x)) * up(x)) of the dequantised dense weights."""
    L = orc.synthetic_layer_cpu(H=256, I=1024, R=8, NB=32, seed=3)
    H, I = 256, 1024
    NB = I // 32
    blocks = np.arange(NB)
    gp, ga = orc.gather_rows_blocks(L["gate_packed"], L["gate_absmax"], blocks, H, 64)
    upk, ua = orc.gather_rows_blocks(L["up_packed"], L["up_absmax"], blocks, H, 64)
    dp, da = orc.gather_down_columns(L["down_packed"], L["down_absmax"], blocks, H, I, 64)
    ye, yf = orc.sparse_mlp(L["x16"].reshape(1, H), np.arange(NB, dtype=np.int32).reshape(1, NB), gp, ga, upk, ua,
                            dp, da)
    Wg = _dense(orc, L["gate_packed"], L["gate_absmax"], I, H)
    Wu = _dense(orc, L["up_packed"], L["up_absmax"], I, H)
    Wd = _dense(orc, L["down_packed"], L["down_absmax"], H, I)
    x = L["x16"].view(np.float16).astype(np.float64)
    g, u = Wg @ x, Wu @ x
    y = Wd @ (g / (1 + np.exp(-g)) * u)
    assert np.allclose(ye[0], y, rtol=1e-9, atol=1e-12)
    e_ref = orc.rel_l2(orc.f16_bits_to_f32(yf[0]), y)
    assert 1e-5 < e_ref < 2e-2  # the fp16 rounding points cost ~1e-3 relative


def test_sparse_mlp_subset_and_row_masks(orc):
    """A subset of blocks equals the dense MLP restricted to those
    intermediate neurons; with several rows each row only uses its own
    blocks (flat_mask semantics, RT:5453)."""
    L = orc.synthetic_layer_cpu(H=256, I=2048, R=8, NB=64, seed=4)
    H, I = 256, 2048
    Wg = _dense(orc, L["gate_packed"], L["gate_absmax"], I, H)
    Wu = _dense(orc, L["up_packed"], L["up_absmax"], I, H)
    Wd = _dense(orc, L["down_packed"], L["down_absmax"], H, I)
    ordered = np.array([2, 5, 9, 33, 60])
    gp, ga = orc.gather_rows_blocks(L["gate_packed"], L["gate_absmax"], ordered, H, 64)
    upk, ua = orc.gather_rows_blocks(L["up_packed"], L["up_absmax"], ordered, H, 64)
    dp, da = orc.gather_down_columns(L["down_packed"], L["down_absmax"], ordered, H, I, 64)
    rng = np.random.default_rng(5)
    x16 = (rng.standard_normal((2, H))).astype(np.float16)
    local = np.array([[0, 2, 4], [1, 3, -1]], dtype=np.int32)
    ye, _ = orc.sparse_mlp(x16.view(np.uint16), local, gp, ga, upk, ua, dp, da, want_fallback=False)
    for t in range(2):
        x = x16[t].astype(np.float64)
        neurons = np.concatenate([np.arange(32 * ordered[s], 32 * ordered[s] + 32) for s in local[t] if s >= 0])
        g, u = Wg[neurons] @ x, Wu[neurons] @ x
        y = Wd[:, neurons] @ (g / (1 + np.exp(-g)) * u)
        assert np.allclose(ye[t], y, rtol=1e-9, atol=1e-12)
