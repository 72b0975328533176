"""Dense-guard prefill MLP (nsmlp_dense_mlp_slots_f16; RT:5775-5831) on MFMA.

Bars:
  * against the oracle (every block selected for every token), the decode
    bars: relL2(gpu, exact) <= max(1e-3, e_ref) and relL2(gpu, fallback) <=
    2 e_ref + 1e-3, with e_ref = relL2(fallback restatement, exact);
  * against a float64 torch restatement with the dense guard's own rounding
    points (fp16 weights fp16(code * absmax), g, silu(g), u, act; y rounded
    once), where only the summation order differs: relL2 <= 1e-3 and every
    element within 4 fp16 ulps of it plus 1e-3 of the row's largest |y|;
  * double-quantised absmax bit-identical to the fp32 path, host-resident
    blocks bit-identical to HBM slots, fused residual add bit-identical to
    the separate fp16 add, and a second run bit-identical (deterministic).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().contiguous().numpy()


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _deq16(packed, absmax, rows, cols, qbs, code):
    """fp16(code[nibble] * absmax) of a row-major NF4 [rows, cols] weight."""
    p = packed.reshape(rows, cols // 2)
    idx = torch.stack([(p >> 4).long(), (p & 15).long()], dim=-1).reshape(rows, cols)
    return (code[idx] * absmax.reshape(rows, cols // qbs).repeat_interleave(qbs, dim=1)).half()


def _torch_dense_guard(L, x16, code):
    H, I, qbs = L.H, L.I, L.qbs
    wg = _deq16(L.gate_packed, L.gate_absmax, I, H, qbs, code).double()
    wu = _deq16(L.up_packed, L.up_absmax, I, H, qbs, code).double()
    wd = _deq16(L.down_packed, L.down_absmax, H, I, qbs, code).double()
    x = x16.double()
    g16 = (x @ wg.T).half()
    s16 = torch.nn.functional.silu(g16.double()).half()
    u16 = (x @ wu.T).half()
    a16 = (s16.double() * u16.double()).half()
    return (a16.double() @ wd.T)  # fp64 sums; the kernel rounds once


@pytest.mark.parametrize("M", [1, 100])
def test_dense_mlp_matches_oracle(gpu, orc, M):
    from next_step_ai_amd.synth import make_synthetic_layer, synth_normal_f16

    H, I, R = 2048, 4096, 16
    print(f"dense guard vs oracle H={H} I={I} M={M}", flush=True)
    L = make_synthetic_layer(H=H, I=I, R=R, seed=131, device=gpu)
    table = L.slot_table()
    x = synth_normal_f16(132, (M, H), 1.0, gpu)
    y = table.dense_mlp(x)
    torch.cuda.synchronize()
    blocks = np.arange(L.NB)
    gp, ga = orc.gather_rows_blocks(_np(L.gate_packed), _np(L.gate_absmax), blocks, H, L.qbs)
    upk, ua = orc.gather_rows_blocks(_np(L.up_packed), _np(L.up_absmax), blocks, H, L.qbs)
    dp, da = orc.gather_down_columns(_np(L.down_packed), _np(L.down_absmax), blocks, H, I, L.qbs)
    active = np.tile(np.arange(L.NB, dtype=np.int32), (M, 1))
    ye, yf = orc.sparse_mlp(_u16(x), active, gp, ga, upk, ua, dp, da, qbs=L.qbs)
    yfb = orc.f16_bits_to_f32(yf).astype(np.float64)
    got = _np(y).astype(np.float64)
    e_ref = orc.rel_l2(yfb, ye)
    e_gpu = orc.rel_l2(got, ye)
    e_gf = orc.rel_l2(got, yfb)
    print(f"  relL2(gpu,exact)={e_gpu:.3e} relL2(fallback,exact)={e_ref:.3e} relL2(gpu,fallback)={e_gf:.3e}",
          flush=True)
    assert e_gpu <= max(1e-3, e_ref)
    assert e_gf <= 2 * e_ref + 1e-3


def test_dense_mlp_matches_torch_restatement_two_token_tiles(gpu, orc):
    from next_step_ai_amd.synth import make_synthetic_layer, synth_normal_f16

    H, I, R, M = 4096, 14336, 64, 257  # 8B shape; the second 256-token tile holds one token
    print(f"dense guard vs torch H={H} I={I} M={M}", flush=True)
    L = make_synthetic_layer(H=H, I=I, R=R, seed=133, device=gpu)
    table = L.slot_table()
    x = synth_normal_f16(134, (M, H), 1.0, gpu)
    y = table.dense_mlp(x)
    y2 = table.dense_mlp(x)
    code = torch.tensor(orc.nf4_code(), device=gpu)
    ref = _torch_dense_guard(L, x, code)
    torch.cuda.synchronize()
    assert torch.equal(y, y2), "dense MLP is not deterministic"
    got = y.double()
    e = float(torch.linalg.norm(got - ref) / torch.linalg.norm(ref))
    ulp = torch.abs(ref.half().double()).clamp_min(2.0 ** -14) * 2.0 ** -10
    tol = 4 * ulp + 1e-3 * ref.abs().amax(dim=1, keepdim=True)
    worst = float(((got - ref).abs() / tol).max())
    print(f"  relL2(gpu, torch fp64 restatement)={e:.3e} worst |err|/tol={worst:.3f}", flush=True)
    assert e <= 1e-3
    assert worst <= 1.0


def test_dense_mlp_split_block_groups_and_batch_invariance(gpu, orc):
    """1664 blocks = 416 groups of 4: on 256 CUs, 256 groups run whole over K
    and the other 160 are split in K over all the CUs (their fp32 partial sums
    added in K order by a second kernel).  Three token tiles (600 tokens)
    against the float64 torch restatement, and each tile's rows bit-identical
    to a call over that tile alone: the split depends on the layer shape, not
    on how many tokens share the call."""
    from next_step_ai_amd.synth import make_synthetic_layer, synth_normal_f16

    H, I, R, M = 1024, 53248, 16, 600
    print(f"dense guard split groups H={H} I={I} M={M}", flush=True)
    L = make_synthetic_layer(H=H, I=I, R=R, seed=161, device=gpu)
    table = L.slot_table()
    x = synth_normal_f16(162, (M, H), 1.0, gpu)
    y = table.dense_mlp(x)
    tiles = ((0, 256), (256, 512), (512, 600))
    ys = [table.dense_mlp(x[a:b].contiguous()) for a, b in tiles]
    code = torch.tensor(orc.nf4_code(), device=gpu)
    ref = _torch_dense_guard(L, x, code)
    torch.cuda.synchronize()
    got = y.double()
    e = float(torch.linalg.norm(got - ref) / torch.linalg.norm(ref))
    ulp = torch.abs(ref.half().double()).clamp_min(2.0 ** -14) * 2.0 ** -10
    tol = 4 * ulp + 1e-3 * ref.abs().amax(dim=1, keepdim=True)
    worst = float(((got - ref).abs() / tol).max())
    print(f"  relL2(gpu, torch fp64 restatement)={e:.3e} worst |err|/tol={worst:.3f}", flush=True)
    assert e <= 1e-3
    assert worst <= 1.0
    for (a, b), yt in zip(tiles, ys):
        assert torch.equal(y[a:b], yt), f"tokens {a}..{b} differ from a call over them alone"


def test_dense_mlp_405b_shape_matches_torch_restatement(gpu, orc):
    """The dense-guard workload itself (hidden 16384, intermediate 53248, 256
    tokens): 256 block groups run whole and 160 are split in K over the CUs.
    Every output against the float64 torch restatement, and a second call
    bit-identical."""
    from next_step_ai_amd.synth import make_synthetic_layer, synth_normal_f16

    H, I, R, M = 16384, 53248, 64, 256
    print(f"dense guard 405B shape H={H} I={I} M={M}", flush=True)
    L = make_synthetic_layer(H=H, I=I, R=R, seed=171, device=gpu, double_quant=True)
    table = L.slot_table()
    x = synth_normal_f16(172, (M, H), 1.0, gpu)
    y = table.dense_mlp(x)
    y2 = table.dense_mlp(x)
    torch.cuda.synchronize()
    assert torch.equal(y, y2), "dense MLP is not deterministic"
    code = torch.tensor(orc.nf4_code(), device=gpu)
    ref = _torch_dense_guard(L, x, code)
    got = y.double()
    e = float(torch.linalg.norm(got - ref) / torch.linalg.norm(ref))
    ulp = torch.abs(ref.half().double()).clamp_min(2.0 ** -14) * 2.0 ** -10
    tol = 4 * ulp + 1e-3 * ref.abs().amax(dim=1, keepdim=True)
    worst = float(((got - ref).abs() / tol).max())
    print(f"  relL2(gpu, torch fp64 restatement)={e:.3e} worst |err|/tol={worst:.3f}", flush=True)
    assert e <= 1e-3
    assert worst <= 1.0


def test_dense_mlp_formats_residency_and_residual(gpu):
    from next_step_ai_amd.synth import make_synthetic_layer, synth_normal_f16

    H, I, R, M = 2048, 4096, 16, 64
    print(f"dense guard formats H={H} I={I} M={M}", flush=True)
    L = make_synthetic_layer(H=H, I=I, R=R, seed=135, device=gpu, double_quant=True)
    x = synth_normal_f16(136, (M, H), 1.0, gpu)
    y_f32 = L.slot_table(absmax="f32").dense_mlp(x)
    y_dq = L.slot_table(absmax="dq").dense_mlp(x)
    rng = np.random.default_rng(135)
    half = torch.from_numpy(rng.choice(L.NB, size=L.NB // 2, replace=False))
    y_host = L.slot_table(resident_blocks=half, host_copy=True).dense_mlp(x)
    res = synth_normal_f16(137, (M, H), 2.0, gpu)
    t = L.slot_table()
    y_res = t.dense_mlp(x, residual=res)
    inplace = res.clone()
    t.dense_mlp(x, out=inplace, residual=inplace)
    torch.cuda.synchronize()
    assert torch.equal(y_dq, y_f32), "double-quantised absmax differs from the resolved fp32 path"
    assert torch.equal(y_host, y_f32), "host-resident blocks differ from HBM slots"
    assert torch.equal(y_res, res + y_f32) and torch.equal(inplace, res + y_f32)


def test_dense_mlp_smallest_shape(gpu, orc):
    """One gate/up workgroup (4 blocks), one down row tile split in two block
    ranges, three tokens."""
    from next_step_ai_amd.synth import make_synthetic_layer, synth_normal_f16

    H, I, R, M = 256, 128, 8, 3
    print(f"dense guard smallest H={H} I={I} M={M}", flush=True)
    L = make_synthetic_layer(H=H, I=I, R=R, seed=139, device=gpu)
    x = synth_normal_f16(140, (M, H), 1.0, gpu)
    y = L.slot_table().dense_mlp(x)
    code = torch.tensor(orc.nf4_code(), device=gpu)
    ref = _torch_dense_guard(L, x, code)
    torch.cuda.synchronize()
    e = float(torch.linalg.norm(y.double() - ref) / torch.linalg.norm(ref))
    print(f"  relL2={e:.3e}", flush=True)
    assert e <= 1e-3


@pytest.mark.parametrize("M", [37, 64, 100, 128, 150, 300])
def test_dense_mlp_token_tiles_bit_identical(gpu, M):
    """Tokens past the last whole 256-token tile (all of a shorter prompt) run
    in a 64-, 128- or 192-token tile; every token's output equals the one a
    full 256-token tile gives it, bit for bit."""
    from next_step_ai_amd.synth import make_synthetic_layer, synth_normal_f16

    H, I, R = 4096, 14336, 64
    print(f"dense guard token tiles H={H} I={I} M={M}", flush=True)
    L = make_synthetic_layer(H=H, I=I, R=R, seed=141, device=gpu, double_quant=True)
    t = L.slot_table()
    x = synth_normal_f16(142, (300, H), 1.0, gpu)
    y_full = t.dense_mlp(x[:256].contiguous())        # one 256-token tile
    y = t.dense_mlp(x[:M].contiguous())
    res = synth_normal_f16(143, (M, H), 1.0, gpu)
    y_res = t.dense_mlp(x[:M].contiguous(), residual=res)
    if M > 256:
        y_tail = t.dense_mlp(x[M - 256:M].contiguous())  # the last M - 256 tokens inside a full tile
    torch.cuda.synchronize()
    assert torch.equal(y[:min(M, 256)], y_full[:min(M, 256)])
    if M > 256:
        assert torch.equal(y[256:], y_tail[512 - M:])
    assert torch.equal(y_res, res + y)


@pytest.mark.parametrize("qbs", [32, 128])
def test_dense_mlp_quant_block_sizes(gpu, orc, qbs):
    """Absmax blocks of 32 and 128 columns: a gate/up lane's 32 columns of a
    step are one absmax entry at qbs 32 and half of one at qbs 128, and the
    down's block columns likewise; against the float64 restatement, and the
    double-quantised path bit-identical to the fp32 path of the resolved
    absmax."""
    from next_step_ai_amd.synth import make_synthetic_layer, synth_normal_f16

    H, I, R, M = 1024, 2048, 16, 70
    print(f"dense guard qbs={qbs} H={H} I={I} M={M}", flush=True)
    L = make_synthetic_layer(H=H, I=I, R=R, seed=150 + qbs, device=gpu, qbs=qbs, double_quant=True)
    x = synth_normal_f16(151 + qbs, (M, H), 1.0, gpu)
    y_dq = L.slot_table().dense_mlp(x)
    y_f32 = L.slot_table(absmax="f32").dense_mlp(x)
    code = torch.tensor(orc.nf4_code(), device=gpu)
    ref = _torch_dense_guard(L, x, code)
    torch.cuda.synchronize()
    assert torch.equal(y_dq, y_f32), "double-quantised absmax differs from the resolved fp32 path"
    e = float(torch.linalg.norm(y_f32.double() - ref) / torch.linalg.norm(ref))
    print(f"  relL2={e:.3e}", flush=True)
    assert e <= 1e-3
