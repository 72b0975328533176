"""GPU router vs the oracle: selected blocks, latent and scores bit-exact."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _rand16(rng, shape, std):
    return (rng.standard_normal(shape) * std).astype(np.float16).view(np.uint16)


def _dev(a16, device):
    return torch.from_numpy(a16.view(np.int16).copy()).view(torch.float16).to(device)


def _route_gpu(device, x16, enc_w, enc_b, sw, sb, k, *, btk=None, dbn=None, legacy=False, sorted_by_score=True):
    from next_step_ai_amd import router

    routing = {"enc_w": _dev(enc_w, device), "enc_b": None if enc_b is None else _dev(enc_b, device)}
    if legacy:
        routing["dec_norm_t"] = _dev(sw, device).transpose(0, 1).contiguous()
    else:
        routing["route_score_weight"] = _dev(sw, device)
        routing["route_score_bias"] = None if sb is None else _dev(sb, device)
    if dbn is not None:
        routing["down_block_norm"] = torch.from_numpy(dbn)
    x = _dev(x16, device).reshape(-1, enc_w.shape[1])
    sel, lat, sc = router.route_tokens(x, routing, k, sorted_by_score=sorted_by_score, basis_top_k=btk,
                                       return_scores=True)
    torch.cuda.synchronize()
    return (sel.cpu().numpy(), lat.cpu().view(torch.int16).numpy().view(np.uint16),
            sc.cpu().view(torch.int16).numpy().view(np.uint16))


CASES = [
    # H, R, NB, k, btk, std_x
    (256, 8, 40, 5, None, 1.0),
    (512, 16, 64, 64, None, 1.0),
    (1000, 12, 97, 13, 5, 3.0),       # H not a multiple of 8 -> scalar path; basis_top_k mask
    (4096, 64, 448, 64, None, 1.0),   # 8B shape
    (16384, 64, 1664, 208, None, 1.0),  # 405B shape
]


@pytest.mark.parametrize("H,R,NB,k,btk,sx", CASES)
def test_route_matches_oracle(gpu, orc, H, R, NB, k, btk, sx):
    rng = np.random.default_rng(H + NB)
    x = _rand16(rng, H, sx)
    enc_w, enc_b = _rand16(rng, (R, H), 0.02), _rand16(rng, R, 0.02)
    sw, sb = _rand16(rng, (NB, R), 0.02), _rand16(rng, NB, 0.02)
    lat_o, sc_o, sel_o = orc.route(x, enc_w, enc_b, sw, sb, k, basis_top_k=btk)
    sel, lat, sc = _route_gpu(gpu, x, enc_w, enc_b, sw, sb, k, btk=btk)
    assert np.array_equal(lat[0], lat_o)
    assert np.array_equal(sc[0], sc_o)
    assert np.array_equal(sel[0], sel_o)
    sel_asc, _, _ = _route_gpu(gpu, x, enc_w, enc_b, sw, sb, k, btk=btk, sorted_by_score=False)
    assert np.array_equal(sel_asc[0], np.sort(sel_o))


def test_route_ties_lowest_index(gpu, orc):
    H, R, NB, k = 256, 4, 300, 37
    rng = np.random.default_rng(7)
    x = _rand16(rng, H, 1.0)
    enc_w, enc_b = _rand16(rng, (R, H), 0.02), _rand16(rng, R, 0.02)
    sw = np.zeros((NB, R), dtype=np.uint16)
    # three distinct bias levels, many equal scores at each level
    sb = np.array([0.5, 0.25, 0.5, 0.125] * (NB // 4), dtype=np.float16).view(np.uint16)
    _, sc_o, sel_o = orc.route(x, enc_w, enc_b, sw, sb, k)
    sel, _, sc = _route_gpu(gpu, x, enc_w, enc_b, sw, sb, k)
    assert np.array_equal(sel[0], sel_o)
    assert np.array_equal(sel[0], np.arange(0, 4 * k, 2)[:k])  # all 0.5's, lowest indices first


def test_route_all_blocks_and_one_block(gpu, orc):
    H, R, NB = 256, 8, 50
    rng = np.random.default_rng(11)
    x = _rand16(rng, H, 1.0)
    enc_w, enc_b = _rand16(rng, (R, H), 0.02), _rand16(rng, R, 0.02)
    sw, sb = _rand16(rng, (NB, R), 0.5), _rand16(rng, NB, 0.02)
    for k in (1, NB):
        _, _, sel_o = orc.route(x, enc_w, enc_b, sw, sb, k)
        sel, _, _ = _route_gpu(gpu, x, enc_w, enc_b, sw, sb, k)
        assert np.array_equal(sel[0], sel_o)


def test_route_legacy_abs_and_down_block_norm(gpu, orc):
    H, R, NB, k = 512, 16, 96, 9
    rng = np.random.default_rng(13)
    x = _rand16(rng, H, 1.0)
    enc_w, enc_b = _rand16(rng, (R, H), 0.02), _rand16(rng, R, 0.02)
    sw = _rand16(rng, (NB, R), 0.02)
    absw = (sw & 0x7FFF).astype(np.uint16)
    dbn = (rng.random(NB) * 2).astype(np.float32)
    lat_o, sc_o, sel_o = orc.route(x, enc_w, enc_b, absw, None, k, legacy_abs=True, down_block_norm=dbn)
    sel, lat, sc = _route_gpu(gpu, x, enc_w, enc_b, absw, None, k, legacy=True, dbn=dbn)
    assert np.array_equal(lat[0], lat_o)
    assert np.array_equal(sc[0], sc_o)
    assert np.array_equal(sel[0], sel_o)


def test_route_multi_row(gpu, orc):
    H, R, NB, k, N = 2048, 32, 256, 24, 5
    rng = np.random.default_rng(17)
    x = _rand16(rng, (N, H), 1.0)
    enc_w, enc_b = _rand16(rng, (R, H), 0.02), _rand16(rng, R, 0.02)
    sw, sb = _rand16(rng, (NB, R), 0.02), _rand16(rng, NB, 0.02)
    sel, _, _ = _route_gpu(gpu, x, enc_w, enc_b, sw, sb, k)
    for t in range(N):
        _, _, sel_o = orc.route(x[t], enc_w, enc_b, sw, sb, k)
        assert np.array_equal(sel[t], sel_o)


def test_route_sparse_mlp_dropin(gpu, orc):
    from next_step_ai_amd.router import route_sparse_mlp

    H, R, NB, k = 1024, 16, 128, 11
    rng = np.random.default_rng(19)
    x = _rand16(rng, (1, 3, H), 1.0)
    enc_w, enc_b = _rand16(rng, (R, H), 0.02), _rand16(rng, R, 0.02)
    sw, sb = _rand16(rng, (NB, R), 0.02), _rand16(rng, NB, 0.02)
    routing = {"enc_w": _dev(enc_w, gpu), "enc_b": _dev(enc_b, gpu), "route_score_weight": _dev(sw, gpu),
               "route_score_bias": _dev(sb, gpu), "down_block_norm": None, "top_k": k, "basis_top_k": R}
    out = route_sparse_mlp(_dev(x, gpu).reshape(1, 3, H), routing)
    assert out.dtype == torch.int64 and tuple(out.shape) == (3, k)
    for t in range(3):
        _, _, sel_o = orc.route(x[0, t], enc_w, enc_b, sw, sb, k)
        assert np.array_equal(out[t].cpu().numpy(), sel_o)
    assert route_sparse_mlp(_dev(x, gpu), None) is None


@pytest.mark.parametrize("H,R,N,sx,sw,btk,legacy", [
    (4096, 20, 37, 1.0, 0.02, None, False),   # ragged tiles: 20 latent rows, 37 tokens
    (16384, 64, 64, 3.0, 1.0, None, False),   # 405B hidden size, large products
    (2048, 64, 29, 1.0, 0.02, 17, False),     # basis_top_k mask on 8 tokens per scores workgroup
    (1024, 200, 19, 1.0, 0.02, 50, False),    # R > 128: one token per scores workgroup
    (2048, 32, 21, 1.0, 0.02, None, True),    # legacy |latent| scores with down_block_norm
])
def test_route_many_rows_tiled_latent(gpu, orc, H, R, N, sx, sw, btk, legacy):
    """From 8 tokens on the latent is computed in 8 x 8 tiles of latent rows
    and tokens (a split of the same exact sums) and the scores of 8 tokens
    share one workgroup: latent, scores and selection of every row bit-exact
    against the oracle."""
    NB, k = 97, 10
    rng = np.random.default_rng(H + N)
    x = _rand16(rng, (N, H), sx)
    enc_w, enc_b = _rand16(rng, (R, H), sw), _rand16(rng, R, 0.02)
    swt, sb = _rand16(rng, (NB, R), 0.02), _rand16(rng, NB, 0.02)
    dbn = None
    if legacy:
        swt = (swt & 0x7FFF).astype(np.uint16)
        sb = None
        dbn = (rng.random(NB) * 2).astype(np.float32)
    print(f"route many rows H={H} R={R} N={N} btk={btk} legacy={legacy}", flush=True)
    sel, lat, sc = _route_gpu(gpu, x, enc_w, enc_b, swt, sb, k, btk=btk, legacy=legacy, dbn=dbn)
    for t in range(N):
        lat_o, sc_o, sel_o = orc.route(x[t], enc_w, enc_b, swt, sb, k, basis_top_k=btk, legacy_abs=legacy,
                                       down_block_norm=dbn)
        assert np.array_equal(lat[t], lat_o), f"latent of row {t}"
        assert np.array_equal(sc[t], sc_o), f"scores of row {t}"
        assert np.array_equal(sel[t], sel_o), f"selection of row {t}"


def test_route_tiled_latent_large_terms_exact(gpu, orc):
    """Terms of 65504^2 that reach 2^42 before they cancel: the tiled latent
    must fall back to three-part sums (a two-part sum would round the small
    term 1 x (0.5 + 2^-11) added while the running sum is above 2^42)."""
    H, R, N, NB, k = 4096, 8, 8, 40, 5
    big = np.float16(65504.0)
    x = np.zeros((N, H), dtype=np.float16)
    w = np.zeros((R, H), dtype=np.float16)
    x[:, :1280] = big
    w[:, :1280] = big                      # waves 0-4 of the tile: +65504^2 each
    x[:, 1536:2816] = big
    w[:, 1536:2816] = -big                 # waves 6-10: the same terms with the other sign
    for t in range(N):
        x[t, 1280] = np.float16(1.0 + t / 8.0)
    for r in range(R):
        w[r, 1280] = np.float16(0.5 + 2.0 ** -11 + r * 2.0 ** -10)
    rng = np.random.default_rng(23)
    x16, w16 = x.view(np.uint16), w.view(np.uint16)
    enc_b = _rand16(rng, R, 0.02)
    swt, sb = _rand16(rng, (NB, R), 0.02), _rand16(rng, NB, 0.02)
    sel, lat, sc = _route_gpu(gpu, x16, w16, enc_b, swt, sb, k)
    for t in range(N):
        lat_o, sc_o, sel_o = orc.route(x16[t], w16, enc_b, swt, sb, k)
        assert np.array_equal(lat[t], lat_o), f"latent of row {t}"
        assert np.array_equal(sc[t], sc_o) and np.array_equal(sel[t], sel_o)


def test_route_tiled_latent_one_large_output_exact(gpu, orc):
    """Only one output of a tile (latent row 3, token 5: not the tile's first
    lane) has terms of 65504^2 that pass 2^42 before they cancel; every other
    output stays small.  The whole tile must take the three-part sums, so
    that output's latent equals the oracle's."""
    H, R, N, NB, k = 4096, 8, 8, 40, 5
    big = np.float16(65504.0)
    rng = np.random.default_rng(29)
    x = (rng.standard_normal((N, H)) * 0.5).astype(np.float16)
    w = (rng.standard_normal((R, H)) * 0.02).astype(np.float16)
    for cols in (slice(0, 1280), slice(1536, 2816)):  # only row 3 and token 5 meet the large values
        x[:, cols] = 0
        w[:, cols] = 0
    x[5, :1280] = big
    w[3, :1280] = big
    x[5, 1536:2816] = big
    w[3, 1536:2816] = -big
    # the rest of that output's sixth 256-column wave span is zero, so the
    # span's two-part sum is 0.5 + 2^-11 (an odd multiple of 2^-11), which a
    # running sum above 2^42 (spacing 2^-10) would round: 0.9697 instead of 0.97
    x[5, 1281:1536] = 0
    x[5, 1280] = np.float16(1.0)
    w[3, 1280] = np.float16(0.5 + 2.0 ** -11)
    x16, w16 = x.view(np.uint16), w.view(np.uint16)
    enc_b = np.zeros(R, dtype=np.uint16)
    swt, sb = _rand16(rng, (NB, R), 0.02), _rand16(rng, NB, 0.02)
    sel, lat, sc = _route_gpu(gpu, x16, w16, enc_b, swt, sb, k)
    for t in range(N):
        lat_o, sc_o, sel_o = orc.route(x16[t], w16, enc_b, swt, sb, k)
        assert np.array_equal(lat[t], lat_o), f"latent of row {t}"
        assert np.array_equal(sc[t], sc_o) and np.array_equal(sel[t], sel_o)


def test_route_tiled_latent_fp16_ties_exact(gpu, orc):
    """Outputs whose exact sum is an fp16 tie (1 + 2^-11, halfway between 1
    and 1 + 2^-10; -3 - 2^-10, halfway between -3 and -3 - 2^-9): the tiled
    latent's fast fp64 pass must leave them to the exact sums, which round
    ties to even (1 and -3).  Every other output is random."""
    H, R, N, NB, k = 2048, 16, 16, 40, 5
    rng = np.random.default_rng(37)
    x = (rng.standard_normal((N, H)) * 0.5).astype(np.float16)
    w = (rng.standard_normal((R, H)) * 0.02).astype(np.float16)
    # token 2 x latent row 5: 1 * 1 + 1 * 2^-11 (other terms zero)
    x[2, :] = 0
    w[5, :] = 0
    x[2, 0] = x[2, 1] = np.float16(1.0)
    w[5, 0], w[5, 1] = np.float16(1.0), np.float16(2.0 ** -11)
    # token 11 x latent row 9: -1 * 3 - 1 * 2^-10
    x[11, :] = 0
    w[9, :] = 0
    x[11, 0] = x[11, 1] = np.float16(-1.0)
    w[9, 0], w[9, 1] = np.float16(3.0), np.float16(2.0 ** -10)
    x16, w16 = x.view(np.uint16), w.view(np.uint16)
    enc_b = np.zeros(R, dtype=np.uint16)
    swt, sb = _rand16(rng, (NB, R), 0.02), _rand16(rng, NB, 0.02)
    sel, lat, sc = _route_gpu(gpu, x16, w16, enc_b, swt, sb, k)
    assert lat.view(np.float16)[2, 5] == np.float16(1.0)
    assert lat.view(np.float16)[11, 9] == np.float16(-3.0)
    for t in range(N):
        lat_o, sc_o, sel_o = orc.route(x16[t], w16, enc_b, swt, sb, k)
        assert np.array_equal(lat[t], lat_o), f"latent of row {t}"
        assert np.array_equal(sc[t], sc_o) and np.array_equal(sel[t], sel_o)


def test_route_many_rows_scores_ties_and_cancellation_exact(gpu, orc):
    """Scores of 8 tokens or more on the matrix cores: outputs that are exact
    fp16 ties (1 + 2^-11 -> 1, 3 + 2^-10 -> 3) and one whose terms of 65504^2
    cancel to 0.5 + 2^-11 must leave the fp64 pass to the exact sums.  The
    latent is x's first R columns exactly (enc_w is the identity, no bias),
    so the score terms are set directly."""
    H, R, N, NB, k = 256, 64, 16, 40, 5
    rng = np.random.default_rng(41)
    x = (rng.standard_normal((N, H)) * 0.5).astype(np.float16)
    enc_w = np.zeros((R, H), dtype=np.float16)
    enc_w[np.arange(R), np.arange(R)] = np.float16(1.0)
    sw = (rng.standard_normal((NB, R)) * 0.02).astype(np.float16)
    one, big = np.float16(1.0), np.float16(65504.0)
    x[3, :R] = 0                     # token 3 x block 7: 1 * 1 + 1 * 2^-11
    x[3, 0] = x[3, 1] = one
    sw[7, :] = 0
    sw[7, 0], sw[7, 1] = one, np.float16(2.0 ** -11)
    x[9, :R] = 0                     # token 9 x block 11: 1 * 3 + 1 * 2^-10
    x[9, 0] = x[9, 1] = one
    sw[11, :] = 0
    sw[11, 0], sw[11, 1] = np.float16(3.0), np.float16(2.0 ** -10)
    x[12, :R] = 0                    # token 12 x block 20: 65504^2 - 65504^2 + (0.5 + 2^-11)
    x[12, 0], x[12, 1], x[12, 2] = big, big, one
    sw[20, :] = 0
    sw[20, 0], sw[20, 1], sw[20, 2] = big, -big, np.float16(0.5 + 2.0 ** -11)
    x16, w16, s16 = x.view(np.uint16), enc_w.view(np.uint16), sw.view(np.uint16)
    enc_b = np.zeros(R, dtype=np.uint16)
    sb = np.zeros(NB, dtype=np.uint16)
    sel, lat, sc = _route_gpu(gpu, x16, w16, enc_b, s16, sb, k)
    scf = sc.view(np.float16)
    assert scf[3, 7] == one and scf[9, 11] == np.float16(3.0) and scf[12, 20] == np.float16(0.5 + 2.0 ** -11)
    for t in range(N):
        lat_o, sc_o, sel_o = orc.route(x16[t], w16, enc_b, s16, sb, k)
        assert np.array_equal(lat[t], lat_o), f"latent of row {t}"
        assert np.array_equal(sc[t], sc_o), f"scores of row {t}"
        assert np.array_equal(sel[t], sel_o), f"selection of row {t}"
