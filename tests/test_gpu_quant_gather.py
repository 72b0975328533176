"""GPU NF4 quantiser, synthetic generator and slot-table gathers vs the oracle (bit-exact)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().contiguous().numpy()


@pytest.mark.parametrize("qbs", [64, 128, 32])
def test_nf4_quantize_matches_oracle(gpu, orc, qbs):
    from next_step_ai_amd import _lib
    from next_step_ai_amd._runtime import ptr, stream_handle

    rng = np.random.default_rng(qbs)
    n = 1 << 18
    w = (rng.standard_normal(n) * 0.02).astype(np.float32)
    w[:qbs] = 0.0  # an all-zero quant block
    w[qbs: 2 * qbs] = np.linspace(-1, 1, qbs, dtype=np.float32)  # values on code midpoints
    wt = torch.from_numpy(w).to(gpu)
    packed = torch.empty(n // 2, dtype=torch.uint8, device=gpu)
    absmax = torch.empty(n // qbs, dtype=torch.float32, device=gpu)
    _lib.call("nsmlp_nf4_quantize_f32", ptr(wt), n, qbs, ptr(packed), ptr(absmax), stream_handle(gpu))
    torch.cuda.synchronize()
    pk_o, am_o = orc.nf4_quantize(w, qbs)
    assert np.array_equal(_np(absmax).view(np.uint32), am_o.view(np.uint32))
    assert np.array_equal(_np(packed), pk_o)


def test_synth_nf4_equals_quantized_synth_normal(gpu, orc):
    from next_step_ai_amd import _lib
    from next_step_ai_amd._runtime import ptr, stream_handle
    from next_step_ai_amd.synth import synth_nf4, synth_normal_f32

    n, qbs, std = 1 << 16, 64, 0.02
    w = synth_normal_f32(1234, (n,), std, gpu)
    pk, am = synth_nf4(1234, n, qbs, std, gpu)
    torch.cuda.synchronize()
    pk_o, am_o = orc.nf4_quantize(_np(w), qbs)
    assert np.array_equal(_np(pk), pk_o)
    assert np.array_equal(_np(am).view(np.uint32), am_o.view(np.uint32))
    z = _np(w) / std
    assert abs(float(z.mean())) < 0.02 and abs(float(z.std()) - 1.0) < 0.02


def test_gather_rows_and_down_columns(gpu, orc):
    from next_step_ai_amd.slot_table import gather_down_columns, gather_row_blocks

    rng = np.random.default_rng(5)
    H, I, qbs = 512, 2048, 64
    NB = I // 32
    gp = rng.integers(0, 256, I * H // 2, dtype=np.uint8)
    ga = rng.standard_normal(I * H // qbs).astype(np.float32)
    dp = rng.integers(0, 256, H * I // 2, dtype=np.uint8)
    da = rng.standard_normal(H * I // qbs).astype(np.float32)
    blocks = np.array([0, 5, 3, NB - 1, 17], dtype=np.int64)
    t = lambda a: torch.from_numpy(a).to(gpu)  # noqa: E731
    p, a = gather_row_blocks(t(gp), t(ga), torch.from_numpy(blocks), H, qbs)
    po, ao = orc.gather_rows_blocks(gp, ga, blocks, H, qbs)
    assert np.array_equal(_np(p), po) and np.array_equal(_np(a), ao)
    for block_major in (False, True):
        p, a = gather_down_columns(t(dp), t(da), torch.from_numpy(blocks), H, I, qbs, block_major=block_major)
        po, ao = orc.gather_down_columns(dp, da, blocks, H, I, qbs)  # [H, n, 16], [H, n]
        if block_major:
            po, ao = po.transpose(1, 0, 2), ao.T
        assert np.array_equal(_np(p), po) and np.array_equal(_np(a), ao)
