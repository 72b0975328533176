"""GPU double-quantised absmax (bitsandbytes nested state) vs the oracle.

Bar: the quantiser, the dequantiser and the u8 gathers are bit-exact against
the oracle; a decode over u8 absmax slots equals, bit for bit, the decode over
fp32 slots holding the resolved absmax (the values the reference computes
with, RT:4621-4625), which the fp32 decode tests pin against the oracle."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().contiguous().numpy()


@pytest.mark.parametrize("dq_block", [256, 64])
def test_quantize_and_resolve_match_oracle(gpu, orc, dq_block):
    from next_step_ai_amd.nested_absmax import NestedAbsmax

    rng = np.random.default_rng(dq_block)
    n = 37 * dq_block + 11
    absmax = (np.abs(rng.standard_normal(n)) * 0.03 + 0.002).astype(np.float32)
    absmax[dq_block: 2 * dq_block] = np.float32(0.0125)  # absmax2 = 0 block
    off = 0.0125
    print(f"nested absmax quantise n={n} dq_block={dq_block}", flush=True)
    nest = NestedAbsmax.quantize(torch.from_numpy(absmax).to(gpu), blocksize=dq_block, offset=off)
    res = nest.resolve()
    torch.cuda.synchronize()
    q_o, a2_o, _ = orc.double_quant(absmax, dq_block=dq_block, offset=off)
    assert np.array_equal(_np(nest.absmax2).view(np.uint32), a2_o.view(np.uint32))
    assert np.array_equal(_np(nest.q), q_o)
    back_o = orc.double_dequant(q_o, a2_o, off, dq_block=dq_block)
    assert np.array_equal(_np(res).view(np.uint32), back_o.view(np.uint32))
    if dq_block == 256:
        # the default offset (the mean, bitsandbytes' compress_statistics) and
        # the codes it leads to equal the oracle's defaults
        nest0 = NestedAbsmax.quantize(torch.from_numpy(absmax).to(gpu))
        torch.cuda.synchronize()
        q_d, a2_d, off_d = orc.double_quant(absmax)
        assert nest0.offset == off_d and off_d != 0.0
        assert np.array_equal(_np(nest0.q), q_d)
        assert np.array_equal(_np(nest0.absmax2).view(np.uint32), a2_d.view(np.uint32))


def test_q8_gathers_match_reference_slicing(gpu, orc):
    from next_step_ai_amd.slot_table import gather_down_columns, gather_row_blocks

    rng = np.random.default_rng(8)
    H, I, qbs = 512, 4096, 64
    NB = I // 32
    gp = rng.integers(0, 256, I * H // 2, dtype=np.uint8)
    gq = rng.integers(0, 256, I * H // qbs, dtype=np.uint8)
    dp = rng.integers(0, 256, H * I // 2, dtype=np.uint8)
    dq = rng.integers(0, 256, H * I // qbs, dtype=np.uint8)
    blocks = np.array([0, 9, 4, NB - 1, 63], dtype=np.int64)
    t = lambda a: torch.from_numpy(a).to(gpu)  # noqa: E731
    rp, rq = gather_row_blocks(t(gp), t(gq), t(blocks), H, qbs)
    dpk, dqk = gather_down_columns(t(dp), t(dq), t(blocks), H, I, qbs)
    torch.cuda.synchronize()
    gq2 = gq.reshape(NB, 32, H // qbs)[blocks]
    # slot layout: rows 2p and 2p+1 interleaved, [n, 16, H/qbs, 2]
    exp_q = np.stack([gq2[:, 0::2, :], gq2[:, 1::2, :]], axis=-1)
    assert rq.dtype == torch.uint8 and np.array_equal(_np(rq), exp_q)
    _, rq_only = gather_row_blocks(None, t(gq), t(blocks), H, qbs)
    assert torch.equal(rq_only, rq)
    assert np.array_equal(_np(rp), gp.reshape(NB, -1)[blocks])
    dq2 = dq.reshape(H, I // qbs)
    assert dqk.dtype == torch.uint8 and np.array_equal(_np(dqk), dq2[:, (blocks * 32) // qbs].T)
    dp2 = dp.reshape(H, I // 2)
    exp = np.stack([dp2[:, 16 * b: 16 * b + 16] for b in blocks])
    assert np.array_equal(_np(dpk), exp)


SHAPES = [
    # H, I, k: generic kernels (H not a multiple of 2048), then the streaming path
    (256, 2048, 16),
    (1024, 4096, 40),
    (2048, 8192, 48),
    (4096, 14336, 64),
    (16384, 53248, 208),
]


@pytest.mark.parametrize("H,I,k", SHAPES)
def test_decode_over_nested_absmax_equals_resolved_fp32(gpu, orc, H, I, k):
    from next_step_ai_amd.synth import make_synthetic_layer

    print(f"nested-absmax decode H={H} I={I} k={k}", flush=True)
    L = make_synthetic_layer(H=H, I=I, R=16, seed=900 + k, device=gpu, double_quant=True)
    out_dq, sel_dq = L.layer(k, absmax="dq").forward(L.x)
    out_f, sel_f = L.layer(k, absmax="f32").forward(L.x)
    torch.cuda.synchronize()
    assert torch.equal(sel_dq, sel_f)
    assert torch.equal(out_dq, out_f), "u8 absmax decode differs from the fp32 decode of the resolved absmax"
    # the resolved absmax are the oracle's dequantisation of the nested state
    for name, a in (("gate", L.gate_absmax), ("down", L.down_absmax)):
        n = L.nested[name]
        back = orc.double_dequant(_np(n.q), _np(n.absmax2), n.offset, _np(n.code2), dq_block=n.blocksize)
        assert np.array_equal(_np(a).reshape(-1).view(np.uint32), back.view(np.uint32))


def test_nested_absmax_with_host_misses(gpu, orc):
    from next_step_ai_amd.slot_table import SparseMlpLayer
    from next_step_ai_amd.synth import make_synthetic_layer

    H, I, k = 2048, 8192, 40
    L = make_synthetic_layer(H=H, I=I, R=16, seed=31, device=gpu, double_quant=True)
    full = L.layer(k, absmax="dq")
    out_full, sel = full.forward(L.x)
    sel_np = _np(sel).astype(np.int64)
    rng = np.random.default_rng(1)
    hit = sel_np[rng.permutation(k)[: int(k * 0.7)]]
    others = np.setdiff1d(np.arange(L.NB), sel_np)
    resident = np.concatenate([hit, rng.choice(others, size=L.NB // 2 - hit.size, replace=False)])
    table = L.slot_table(resident_blocks=torch.from_numpy(resident), host_copy=True, absmax="dq")
    part = SparseMlpLayer(L.router(), table, k)
    out_part, sel2 = part.forward(L.x)
    torch.cuda.synchronize()
    assert torch.equal(sel2, sel)
    assert torch.equal(out_part, out_full)
