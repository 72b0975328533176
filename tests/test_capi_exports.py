"""The C-ABI library loads on the host and exports every symbol include/nsmlp.h
declares (no compute calls: this runs without a GPU)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    with open(os.path.join(ROOT, "include", "nsmlp.h")) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nsmlp_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from next_step_ai_amd import _lib

    path = _lib.LIB_PATH
    if not os.path.exists(path):
        from next_step_ai_amd import build_lib

        build_lib.build()
    return ctypes.CDLL(path)


def test_header_declares_entry_points():
    names = _declared()
    for must in ("nsmlp_route_f16", "nsmlp_decode_slots_f16", "nsmlp_decode_layer_f16",
                 "nsmlp_single_kernel_decode_f16", "nsmlp_fused_decode_gathered_f16",
                 "nsmlp_output_linear_nf4_f16", "nsmlp_input_linear_nf4_f16"):
        assert must in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_header():
    from next_step_ai_amd import _lib

    assert set(_declared()) == set(_lib.SIGNATURES)


def test_host_only_calls(lib):
    from next_step_ai_amd import _lib

    L = _lib.lib()
    assert L.nsmlp_version() >= 100
    # workspace sizing is pure host arithmetic
    assert L.nsmlp_decode_workspace_bytes(16384, 208) > 16384 * 4
    assert L.nsmlp_layer_workspace_bytes(16384, 64, 1664, 208) >= L.nsmlp_decode_workspace_bytes(16384, 208)
    # argument validation runs before any device work and sets the error string
    rc = L.nsmlp_route_f16(None, 1, 100000, None, None, 64, 64, None, None, None, 1664, 0, 208, None, None, None,
                           None, 0, None)
    assert rc == -22 and b"hidden size" in L.nsmlp_last_error()
    rc = L.nsmlp_single_kernel_decode_f16(None, None, None, None, None, None, None, None, None, None, None, None,
                                          16384, 16, 64, 208, None, 0, None)
    assert rc == -22 and b"block_size" in L.nsmlp_last_error()


def test_no_cpu_fallback_without_gpu():
    import torch

    from next_step_ai_amd.sparse_mlp import triton_sparse_input_linear_4bit

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(RuntimeError, match="GPU tensor"):
        triton_sparse_input_linear_4bit(
            torch.zeros(1, 64, dtype=torch.float16), torch.zeros(1, 1, dtype=torch.int32),
            packed_weight=torch.zeros(64 * 16, dtype=torch.uint8), absmax=torch.ones(64),
            code=torch.zeros(16), out_features=32, in_features=64, quant_block_size=32, bias=None, block_size=32)


def test_host_validation_of_lm_head_dense_and_residual_entry_points(lib):
    """Argument checks of the LM-head, dense-guard and residual entry points
    run on the host before any device work (no GPU needed)."""
    import ctypes

    from next_step_ai_amd import _lib

    L = _lib.lib()
    assert L.nsmlp_version() >= 102
    assert L.nsmlp_dense_linear_nf4_f16(None, None, 1, None, None, None) == -22
    assert b"NULL matrix" in L.nsmlp_last_error()
    m = _lib.Nf4Matrix(out_features=10, in_features=20000, qbs=64)
    assert L.nsmlp_dense_linear_nf4_f16(ctypes.byref(m), None, 1, None, None, None) == -22
    assert b"in_features" in L.nsmlp_last_error()
    m = _lib.Nf4Matrix(out_features=10, in_features=4096, qbs=48)
    assert L.nsmlp_dense_linear_nf4_f16(ctypes.byref(m), None, 1, None, None, None) == -22
    assert b"quant block size" in L.nsmlp_last_error()
    m = _lib.Nf4Matrix(out_features=10, in_features=4096, qbs=64, dq_block=100)
    assert L.nsmlp_dense_linear_nf4_f16(ctypes.byref(m), None, 1, None, None, None) == -22
    assert b"dq_block" in L.nsmlp_last_error()
    m = _lib.Nf4Matrix(out_features=300000, in_features=16384, qbs=64)
    assert L.nsmlp_dense_linear_nf4_f16(ctypes.byref(m), None, 1, None, None, None) == -22
    assert b"2 GiB" in L.nsmlp_last_error()
    m = _lib.Nf4Matrix(out_features=10, in_features=4096, qbs=64)
    assert L.nsmlp_dense_linear_nf4_f16(ctypes.byref(m), None, 0, None, None, None) == 0  # no rows: nothing to do
    assert L.nsmlp_dense_linear_nf4_f16(ctypes.byref(m), None, 1, None, None, None) == -22
    assert b"NULL tensor" in L.nsmlp_last_error()
    # dense-guard MLP: shape rules and workspace sizing
    t = _lib.SlotTable(H=1000, I=4096, qbs=64, n_slots=128)
    assert L.nsmlp_dense_mlp_slots_f16(ctypes.byref(t), None, 4, None, None, None, 0, None) == -22
    t = _lib.SlotTable(H=2048, I=4096, qbs=64, n_slots=128)
    assert L.nsmlp_dense_mlp_workspace_bytes(2048, 4096, 256) > 256 * 4096 * 2 + 256 * 2048 * 4
    # the residual layer call needs a residual
    r = _lib.Router(R=16, basis_top_k=16, NB=128)
    assert L.nsmlp_decode_layer_add_f16(ctypes.byref(r), ctypes.byref(t), None, None, 16, None, None, None, 0,
                                        None) == -22
    assert b"residual" in L.nsmlp_last_error()
    # the input linear takes block sizes that are multiples of 32
    assert L.nsmlp_input_linear_nf4_f16(None, 1, 4096, None, 1, None, None, None, 64, 10, None, 48, None, None) == -22
    assert b"block_size" in L.nsmlp_last_error()
