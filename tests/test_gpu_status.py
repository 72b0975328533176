"""The kernels' status word reaches the caller: a selected block that is
neither in an HBM slot nor host-copied (the reference's gather raises for
it, RT:4530-4578) and a grouped prefill down partial outside the
fixed-point range.  No test makes a kernel fault: such blocks are read
through zero-extent buffer descriptors (zeros) by design."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ptr(t):
    return int(t.data_ptr())


def test_layer_check_blocks_raises_for_unavailable_block(gpu):
    from next_step_ai_amd import _lib
    from next_step_ai_amd._runtime import stream_handle, workspace
    from next_step_ai_amd.slot_table import SparseMlpLayer
    from next_step_ai_amd.synth import make_synthetic_layer

    H, I, R, k = 2048, 8192, 16, 40
    L = make_synthetic_layer(H=H, I=I, R=R, seed=91, device=gpu)
    full = SparseMlpLayer(L.router(), L.slot_table(), k, check_blocks=True)
    y_full, sel = full.forward(L.x)
    full.check_status()  # every block resident: nothing to report
    sel_np = sel.cpu().numpy()
    missing = int(sel_np[3])
    resident = np.setdiff1d(np.arange(L.NB), [missing])
    table = L.slot_table(resident_blocks=torch.from_numpy(resident))  # no host copies
    layer = SparseMlpLayer(L.router(), table, k, check_blocks=True)
    y, sel2 = layer.forward(L.x)
    with pytest.raises(RuntimeError, match="neither in an HBM slot nor host-copied"):
        layer.check_status()
    layer.check_status()  # the report was consumed
    torch.cuda.synchronize()
    assert torch.equal(sel2, sel)
    assert not torch.equal(y, y_full)  # the missing block contributed zero
    # the next forward raises by itself once the earlier report has arrived
    layer.forward(L.x)
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="neither in an HBM slot"):
        layer.forward(L.x)

    # the C ABI hand-over: OR into dst, then the word is clear (an unchecked
    # decode on the same stream's workspace sets the word again)
    table.decode(L.x, sel)
    ws = workspace(int(_lib.lib().nsmlp_decode_workspace_bytes(H, k)), gpu)
    dst = torch.zeros(2, dtype=torch.int32, device=gpu)
    s = stream_handle(gpu)
    _lib.call("nsmlp_workspace_take_status", _ptr(ws), _ptr(dst), s)
    _lib.call("nsmlp_workspace_take_status", _ptr(ws), _ptr(dst) + 4, s)
    torch.cuda.synchronize()
    assert dst.tolist() == [_lib.NSMLP_STATUS_BLOCK_UNAVAILABLE, 0]


def test_decode_check_and_out_of_range_ids(gpu):
    from next_step_ai_amd.synth import make_synthetic_layer

    L = make_synthetic_layer(H=2048, I=4096, R=8, seed=93, device=gpu)
    t = L.slot_table()
    ok = torch.tensor([1, 5, 9], dtype=torch.int32)
    t.decode(L.x, ok, check=True)
    with pytest.raises(RuntimeError, match="out of range"):
        t.decode(L.x, torch.tensor([1, 5, L.NB + 7], dtype=torch.int32), check=True)


def test_prefill_fixed_point_range_is_reported(gpu):
    """Grouped down (M k < 2 NB): a block whose down absmax makes a partial
    exceed 2^23 sets the fixed-range bit, and the check raises."""
    from next_step_ai_amd.synth import make_synthetic_layer, synth_normal_f16

    H, I, R, k, M = 2048, 4096, 16, 8, 2
    L = make_synthetic_layer(H=H, I=I, R=R, seed=95, device=gpu)
    t = L.slot_table(absmax="f32")
    x = synth_normal_f16(96, (M, H), 1.0, gpu)
    sel = L.router().route(x, k)
    assert M * k < 2 * L.NB
    y = t.prefill(x, sel, check=True)  # ordinary weights: in range
    assert torch.isfinite(y.float()).all()
    b = int(sel[0, 0])
    t.down_absmax[b].fill_(1.0e7)  # block-major slots, identity lookup: slot b
    with pytest.raises(RuntimeError, match="fixed-point range"):
        t.prefill(x, sel, check=True)


def test_checked_call_reports_its_own_status_only(gpu):
    """An unchecked call that reads an unavailable block leaves its bit in the
    shared workspace's status word; a checked call after it (a good one) does
    not raise: the check clears the word before its call.  The same for a
    checked layer after an unchecked layer on the same stream."""
    from next_step_ai_amd.slot_table import SparseMlpLayer
    from next_step_ai_amd.synth import make_synthetic_layer

    H, I, R, k = 2048, 8192, 16, 40
    L = make_synthetic_layer(H=H, I=I, R=R, seed=97, device=gpu)
    full = L.slot_table()
    _, sel = L.layer(k).forward(L.x)
    missing = int(sel[2])
    bad = L.slot_table(resident_blocks=torch.from_numpy(np.setdiff1d(np.arange(L.NB), [missing])))
    bad.decode(L.x, sel)  # unchecked: leaves the bit
    full.decode(L.x, sel, check=True)  # must not raise
    bad.prefill(L.x.reshape(1, H).repeat(2, 1), sel.reshape(1, k).repeat(2, 1))
    full.prefill(L.x.reshape(1, H).repeat(2, 1), sel.reshape(1, k).repeat(2, 1), check=True)
    bad_layer = SparseMlpLayer(L.router(), bad, k)
    good_layer = SparseMlpLayer(L.router(), full, k, check_blocks=True)
    bad_layer.forward(L.x)
    good_layer.forward(L.x)
    good_layer.check_status()
    # and the bad call, checked, still raises
    with pytest.raises(RuntimeError, match="neither in an HBM slot"):
        bad.decode(L.x, sel, check=True)
