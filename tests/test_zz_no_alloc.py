"""The no-allocation decode layer (nsmlp_decode_layer_noalloc_f16) against the
workspace entry points it varies (nsmlp_decode_layer_f16, _add_f16), through
the C ABI: selections and outputs bit-identical (same kernels), on calls in
a row where the later ones are smaller (the per-device scratch keeps the
last call's contents), with and without the fused residual add; the status
word handed over; shapes outside its scratch rejected with a message."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _p(t):
    return None if t is None else int(t.data_ptr())


def _noalloc(layer, x, residual=None, status=None):
    from next_step_ai_amd import _lib
    from next_step_ai_amd._runtime import stream_handle

    out = torch.empty(layer.table.H, dtype=torch.float16, device=layer.device)
    sel = torch.empty(layer.top_k, dtype=torch.int32, device=layer.device)
    _lib.call("nsmlp_decode_layer_noalloc_f16", ctypes.byref(layer._r), ctypes.byref(layer._t), _p(x), _p(residual),
              layer.top_k, _p(sel), _p(out), _p(status), stream_handle(layer.device))
    return out, sel


def test_noalloc_matches_layer_entry_points(gpu):
    from next_step_ai_amd.synth import make_synthetic_layer, synth_normal_f16

    print("[noalloc] 405B, 8B and small layers", flush=True)
    layers = [
        make_synthetic_layer(H=16384, I=53248, R=64, seed=2100, device=gpu, double_quant=True).layer(208),
        make_synthetic_layer(H=4096, I=14336, R=64, seed=2101, device=gpu, double_quant=True).layer(64),
        make_synthetic_layer(H=2048, I=8192, R=16, seed=2102, device=gpu).layer(40),
    ]
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    for i, layer in enumerate(layers):  # each call smaller than the one before
        H = layer.table.H
        x = synth_normal_f16(2200 + i, (H,), 1.0, gpu)
        res = synth_normal_f16(2300 + i, (H,), 1.0, gpu)
        ref_out, ref_sel = layer.forward(x)
        ref_add, _ = layer.forward(x, residual=res)
        out, sel = _noalloc(layer, x, status=status)
        out_add, sel_add = _noalloc(layer, x, residual=res)
        torch.cuda.synchronize()
        assert torch.equal(sel, ref_sel) and torch.equal(sel_add, ref_sel), f"layer {i}: selection"
        assert torch.equal(out, ref_out), f"layer {i}: output"
        assert torch.equal(out_add, ref_add), f"layer {i}: output with the residual add"
    assert int(status.item()) == 0
    # back to the largest layer after the smaller ones
    x = synth_normal_f16(2200, (16384,), 1.0, gpu)
    ref_out, ref_sel = layers[0].forward(x)
    out, sel = _noalloc(layers[0], x)
    torch.cuda.synchronize()
    assert torch.equal(sel, ref_sel) and torch.equal(out, ref_out)


def test_noalloc_reports_unavailable_blocks_and_rejects_large_shapes(gpu):
    import numpy as np

    from next_step_ai_amd import _lib
    from next_step_ai_amd.slot_table import SparseMlpLayer
    from next_step_ai_amd.synth import make_synthetic_layer

    L = make_synthetic_layer(H=2048, I=8192, R=16, seed=2103, device=gpu)
    full = L.layer(40)
    _, sel = full.forward(L.x)
    missing = int(sel[5])
    table = L.slot_table(resident_blocks=torch.from_numpy(np.setdiff1d(np.arange(L.NB), [missing])))
    layer = SparseMlpLayer(L.router(), table, 40)
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    _noalloc(layer, L.x, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == _lib.NSMLP_STATUS_BLOCK_UNAVAILABLE
    status.zero_()
    _noalloc(full, L.x, status=status)  # the scratch's word was cleared by the hand-over
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    # a bad call without status_out leaves its bit in the scratch; the next
    # call clears the word at its start, so it reports its own status only
    _noalloc(layer, L.x)
    _noalloc(full, L.x, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == 0
    big = make_synthetic_layer(H=2048, I=131072, R=16, seed=2104, device=gpu)  # 4096 blocks
    with pytest.raises(RuntimeError, match="per-device scratch holds 262144"):
        _noalloc(big.layer(2048), big.x)  # k = 2048 needs more than the scratch
    odd = make_synthetic_layer(H=1024, I=4096, R=16, seed=2105, device=gpu)
    with pytest.raises(RuntimeError, match="streaming kernels only"):
        _noalloc(odd.layer(16), odd.x)
