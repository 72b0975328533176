"""The reference runtime's failure branches driven through the drop-ins with
injected faults (nsmlp_fault_inject), on the GPU.

`_RuntimeDecode` restates the control flow of the runtime's Triton decode
(RT:5560-5685): the single-kernel entry point is tried while enabled, a
failure is counted and the path is turned off after three (RT:5626-5637); the
v1 entry point is tried next, and any exception there switches the runtime
to the dequant fallback (RT:5681-5685).  Faults fire before the device is
touched, so every kernel that does run exits normally."""
import numpy as np
import pytest
import torch

from test_fault_inject import _is_oom
from test_gpu_decode import _np, _oracle_for_layer

pytestmark = pytest.mark.gpu


class _RuntimeDecode:
    def __init__(self, single, v1):
        self.single, self.v1 = single, v1
        self.single_enabled = True
        self.single_fail_count = 0
        self.fused_enabled = True
        self.backend = None

    def __call__(self):
        if self.single_enabled:
            try:
                out = self.single()
                self.backend = "single_kernel_sparse_decode_sm75"
                return out
            except Exception:
                self.single_fail_count += 1
                if self.single_fail_count >= 3:
                    self.single_enabled = False
        try:
            out = self.v1()
            self.backend = "fused_sparse_decode_v1"
            return out
        except Exception:
            self.fused_enabled = False
            self.backend = "dequant_sparse_fallback"
            return None


def test_runtime_failure_branches_with_injected_faults(gpu, orc):
    from next_step_ai_amd import _lib
    from next_step_ai_amd.sparse_mlp import (
        triton_fused_sparse_mlp_decode_4bit,
        triton_sparse_mlp_decode_4bit_single_kernel_sm75,
    )
    from next_step_ai_amd.synth import make_synthetic_layer

    H, I, R, k = 2048, 8192, 32, 48
    L = make_synthetic_layer(H=H, I=I, R=R, seed=11, device=gpu)
    layer = L.layer(k)
    y_ref, sel = layer.forward(L.x)
    y_ref = y_ref.clone()
    _, _, (gp, ga, upk, ua, dp, da) = _oracle_for_layer(orc, L, _np(sel).astype(np.int64))
    code = torch.tensor(orc.nf4_code(), device=gpu)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    gp, ga, upk, ua, dp, da = (t(a) for a in (gp, ga, upk, ua, dp, da))

    def single():
        out = torch.empty((1, H), dtype=torch.float16, device=gpu)
        acc = torch.empty(H, dtype=torch.float32, device=gpu)
        return triton_sparse_mlp_decode_4bit_single_kernel_sm75(
            L.x.reshape(1, H), sel, gp, ga, code, upk, ua, code, dp, da, code, out, acc, H, 32, 64, k)

    def v1():
        return triton_fused_sparse_mlp_decode_4bit(
            L.x.reshape(1, H), torch.arange(k, dtype=torch.int32, device=gpu).reshape(1, k),
            torch.ones((1, k * 32), dtype=torch.float16, device=gpu),
            gate_packed_weight=gp.reshape(-1), gate_absmax=ga.reshape(-1), gate_code=code, gate_input_dim=H,
            gate_quant_block_size=64, gate_bias=None,
            up_packed_weight=upk.reshape(-1), up_absmax=ua.reshape(-1), up_code=code, up_input_dim=H,
            up_quant_block_size=64, up_bias=None,
            down_packed_weight=dp.reshape(-1), down_absmax=da.reshape(-1), down_code=code,
            down_out_features=H, down_in_features=k * 32, down_quant_block_size=32, down_bias=None, block_size=32)

    print("[fault inject] single kernel fails 3 times, v1 serves", flush=True)
    rt = _RuntimeDecode(single, v1)
    with _lib.injected_faults("single_kernel_decode_f16=hip:3"):
        for i in range(3):
            y = rt()
            torch.cuda.synchronize()
            assert rt.backend == "fused_sparse_decode_v1" and torch.equal(y.reshape(-1), y_ref), i
        assert rt.single_fail_count == 3 and not rt.single_enabled
        # the fault's count is used up: the single kernel works again, but the runtime keeps it off
        y = rt()
        torch.cuda.synchronize()
        assert rt.backend == "fused_sparse_decode_v1" and torch.equal(y.reshape(-1), y_ref)
    y = single()
    torch.cuda.synchronize()
    assert torch.equal(y.reshape(-1), y_ref), "a call after the injected failures differs"

    print("[fault inject] v1 fails: the runtime switches to the dequant fallback", flush=True)
    rt = _RuntimeDecode(single, v1)
    with _lib.injected_faults("single_kernel_decode_f16=oom,fused_decode_gathered_f16=hip:1"):
        assert rt() is None and rt.backend == "dequant_sparse_fallback" and not rt.fused_enabled
        assert rt.single_fail_count == 1
        with pytest.raises(RuntimeError) as ei:
            single()
        assert _is_oom(str(ei.value)), str(ei.value)

    print("[fault inject] the layer call: an injected OOM, then the same output", flush=True)
    with _lib.injected_faults("decode_layer_f16=oom:1"):
        with pytest.raises(RuntimeError) as ei:
            layer.forward(L.x)
        assert _is_oom(str(ei.value))
        y2, sel2 = layer.forward(L.x)
        torch.cuda.synchronize()
    assert torch.equal(y2, y_ref) and torch.equal(sel2, sel)
