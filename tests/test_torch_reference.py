"""The torch-CPU restatement of the reference's decode path (the benchmark's
CPU baseline, oracle/torch_reference.py) against the oracle.

Bars: the fp32 variant's MLP within 1e-5 (relative L2) of the oracle's
exact fp64 result over the same blocks; the fp16 variant (the reference's
compute dtype and rounding points) within the oracle fallback leg's own
error of the exact result (relL2 <= 2 e_ref + 1e-3, the decode bar), since
torch's fp16 CPU linear may round its sums differently from the oracle's
exact-then-round dots; the layout equals the oracle's; the routed block sets
agree with the oracle's exact route (torch's fp16 topk breaks ties in its own
order, which these seeded scores do not exercise)."""
import numpy as np
import torch

from oracle import torch_reference as tref


def _layer(orc, H, I, R, k, seed):
    L = orc.synthetic_layer_cpu(H, I, R, I // 32, seed)
    _, _, sel_o = orc.route(L["x16"], L["enc_w16"], L["enc_b16"], L["score_w16"], L["score_b16"], k)
    return L, np.sort(sel_o).astype(np.int64)


def _gathered(orc, L, sel):
    H, I, qbs = L["H"], L["I"], L["qbs"]
    gp, ga = orc.gather_rows_blocks(L["gate_packed"], L["gate_absmax"], sel, H, qbs)
    upk, ua = orc.gather_rows_blocks(L["up_packed"], L["up_absmax"], sel, H, qbs)
    dp, da = orc.gather_down_columns(L["down_packed"], L["down_absmax"], sel, H, I, qbs)
    return tuple(torch.from_numpy(np.ascontiguousarray(a)) for a in (gp, ga, upk, ua, dp, da))


def _f16(bits):
    return torch.from_numpy(np.asarray(bits, dtype=np.uint16).view(np.float16).copy())


def test_torch_reference_matches_oracle(orc):
    for H, I, R, k, seed in ((512, 4096, 16, 24, 1), (1024, 8192, 32, 40, 2)):
        L, sel = _layer(orc, H, I, R, k, seed)
        g = _gathered(orc, L, sel)
        code = torch.from_numpy(orc.nf4_code().astype(np.float32))
        args = (_f16(L["x16"]), _f16(L["enc_w16"]), _f16(L["enc_b16"]), _f16(L["score_w16"]), _f16(L["score_b16"]),
                k, g, code, L["qbs"])
        out32, ordered32 = tref.decode_layer(*args, dtype=torch.float32)
        out16, ordered16 = tref.decode_layer(*args, dtype=torch.float16)
        assert np.array_equal(ordered16.numpy(), sel), "fp16 torch route differs from the oracle's"
        ye, yf = orc.sparse_mlp(L["x16"].reshape(1, H), np.arange(k, dtype=np.int32).reshape(1, k),
                                *(t.numpy() for t in g), qbs=L["qbs"])
        e_ref = orc.rel_l2(orc.f16_bits_to_f32(yf[0]), ye[0])
        assert orc.rel_l2(out32.numpy().reshape(-1), ye[0]) <= 1e-5
        e16 = orc.rel_l2(out16.float().numpy().reshape(-1), ye[0])
        assert e16 <= 2 * e_ref + 1e-3, (e16, e_ref)


def test_torch_layout_matches_oracle(orc):
    rng = np.random.default_rng(3)
    blocks = rng.integers(-2, 60, size=(3, 7))
    ordered, local, mask, neurons = tref.active_layout(torch.from_numpy(blocks), 3, 50, torch.float16)
    o_ordered, o_local, o_mask, o_neurons = orc.active_layout(blocks, 50)
    assert np.array_equal(ordered.numpy(), np.asarray(o_ordered))
    assert np.array_equal(local.numpy(), np.asarray(o_local))
    assert np.array_equal(mask.float().numpy(), np.asarray(o_mask, dtype=np.float32))
    assert np.array_equal(neurons.numpy(), np.asarray(o_neurons))
