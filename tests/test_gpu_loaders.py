"""On-disk formats to the device: a layer written as bitsandbytes NF4
safetensors plus a routing artifact, read back into a slot table and a
router, routes and decodes bit-identically to the in-memory layer."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nested", [False, True])
def test_layer_from_disk_matches_in_memory(gpu, tmp_path, nested):
    from next_step_ai_amd._runtime import nf4_code
    from next_step_ai_amd.loaders import (Nf4Param, load_routing_artifact, router_from_routing,
                                          slot_table_from_safetensors, write_nf4_safetensors)
    from next_step_ai_amd.slot_table import SparseMlpLayer
    from next_step_ai_amd.synth import make_synthetic_layer

    H, I, R, k = 2048, 8192, 16, 40
    print(f"[loaders] nested={nested} H={H} I={I}", flush=True)
    L = make_synthetic_layer(H=H, I=I, R=R, seed=71, device=gpu, double_quant=nested)
    code = nf4_code(gpu)

    def param(packed, name, shape):
        am = L.nested[name] if nested else getattr(L, f"{name}_absmax")
        return Nf4Param(packed=packed, absmax=am, code=code, blocksize=L.qbs, shape=shape, dtype="float16")

    pre = "model.layers.3.mlp."
    write_nf4_safetensors(tmp_path / "model.safetensors", {
        f"{pre}gate_proj.weight": param(L.gate_packed, "gate", (I, H)),
        f"{pre}up_proj.weight": param(L.up_packed, "up", (I, H)),
        f"{pre}down_proj.weight": param(L.down_packed, "down", (H, I)),
    })
    torch.save({"config": {"artifact_target": "intermediate_block_scores", "block_domain": "intermediate",
                           "basis_rank": R, "basis_top_k": R, "block_size": 32, "num_blocks": I // 32,
                           "top_k_by_layer": {"3": k}},
                "layer_selection": [3],
                "layer_states": {"3": {"encoder_weight": L.enc_w.cpu(), "encoder_bias": L.enc_b.cpu(),
                                       "score_weight": L.score_w.cpu(), "score_bias": L.score_b.cpu(),
                                       "scale": torch.tensor(1.0)}},
                "stats": {}}, tmp_path / "basis.pt")

    ref = SparseMlpLayer(L.router(), L.slot_table(absmax="dq" if nested else "f32"), k)
    out_ref, sel_ref = ref.forward(L.x)
    routing = load_routing_artifact(tmp_path / "basis.pt", hidden_size=H, intermediate_size=I, device=gpu)
    assert routing[3]["top_k"] == k
    table = slot_table_from_safetensors(tmp_path, 3, device=gpu)
    assert (table.nested is not None) == nested
    layer = SparseMlpLayer(router_from_routing(routing[3], gpu), table, routing[3]["top_k"])
    out, sel = layer.forward(L.x)
    torch.cuda.synchronize()
    assert torch.equal(sel, sel_ref)
    assert torch.equal(out, out_ref)
    # a resident subset with host copies reads the same
    rng = np.random.default_rng(71)
    part = slot_table_from_safetensors(tmp_path, 3, device=gpu, host_copy=True,
                                       resident_blocks=torch.from_numpy(rng.choice(I // 32, 100, replace=False)))
    out2, _ = SparseMlpLayer(router_from_routing(routing[3], gpu), part, k).forward(L.x)
    torch.cuda.synchronize()
    assert torch.equal(out2, out_ref)


def _quantised(orc, rng, out_f, in_f, nested):
    """NF4 weight made on the CPU by the oracle's quantiser: (packed, the fp32
    absmax the MLP uses, the absmax state written to disk)."""
    from next_step_ai_amd.nested_absmax import NestedAbsmax

    w = (rng.standard_normal(out_f * in_f) * 0.02).astype(np.float32)
    packed, absmax = orc.nf4_quantize(w, qbs=64)
    if not nested:
        return packed, absmax, torch.from_numpy(absmax)
    q, a2, off = orc.double_quant(absmax)
    code2 = orc.dynamic_map_signed().astype(np.float32)
    resolved = orc.double_dequant(q, a2, off)  # the reference's resolution (RT:4621-4625)
    state = NestedAbsmax(q=torch.from_numpy(q), absmax2=torch.from_numpy(a2), code2=torch.from_numpy(code2),
                         offset=float(off), blocksize=256)
    return packed, resolved, state


def _write_hand_packed(path, params):
    """Every projection key by key in bitsandbytes' QuantState.as_dict(packed=True)
    form: the packed weight [n/2, 1] u8, absmax, quant_map, the nested state and
    one JSON blob tensor."""
    import json

    from safetensors.torch import save_file

    from next_step_ai_amd.nested_absmax import NestedAbsmax

    out = {}
    for name, (packed, state, code, shape) in params.items():
        meta = {"quant_type": "nf4", "blocksize": 64, "dtype": "float16", "shape": list(shape)}
        out[name] = torch.from_numpy(packed).reshape(-1, 1)
        out[f"{name}.quant_map"] = code.clone()
        if isinstance(state, NestedAbsmax):
            out[f"{name}.absmax"] = state.q
            out[f"{name}.nested_absmax"] = state.absmax2
            out[f"{name}.nested_quant_map"] = state.code2.clone()
            meta.update({"nested_blocksize": 256, "nested_dtype": "float32", "nested_offset": state.offset})
        else:
            out[f"{name}.absmax"] = state
        out[f"{name}.quant_state.bitsandbytes__nf4"] = torch.tensor(list(json.dumps(meta).encode("utf-8")),
                                                                    dtype=torch.uint8)
    save_file(out, str(path))


@pytest.mark.parametrize("nested,hand_packed", [(False, False), (True, False), (False, True), (True, True)])
def test_disk_loaded_layer_matches_oracle(gpu, orc, tmp_path, nested, hand_packed):
    """A layer whose weights and quant state the oracle made on the CPU, written
    to disk (by the package's writer, or key by key in bitsandbytes' packed
    quant-state form), read by slot_table_from_safetensors and
    load_routing_artifact: the routed blocks equal the oracle's route and the
    output is within the decode bars of the oracle MLP computed from the bytes
    and absmax that were written (runtime/safetensor_loader.py:391-472,
    RT:779-991)."""
    from test_gpu_decode import _check_tolerance

    from next_step_ai_amd.loaders import (Nf4Param, load_routing_artifact, router_from_routing,
                                          slot_table_from_safetensors, write_nf4_safetensors)
    from next_step_ai_amd.slot_table import SparseMlpLayer

    H, I, R, k, li = 2048, 8192, 16, 40, 5
    NB = I // 32
    print(f"[loaders vs oracle] nested={nested} hand_packed={hand_packed}", flush=True)
    rng = np.random.default_rng(100 + 2 * nested + hand_packed)
    gp, ga, gst = _quantised(orc, rng, I, H, nested)
    upk, ua, ust = _quantised(orc, rng, I, H, nested)
    dp, da, dst = _quantised(orc, rng, H, I, nested)
    code = torch.from_numpy(orc.nf4_code().astype(np.float32))
    pre = f"model.layers.{li}.mlp."
    projs = {f"{pre}gate_proj.weight": (gp, gst, (I, H)), f"{pre}up_proj.weight": (upk, ust, (I, H)),
             f"{pre}down_proj.weight": (dp, dst, (H, I))}
    if hand_packed:
        _write_hand_packed(tmp_path / "model.safetensors",
                           {n: (p, st, code, shape) for n, (p, st, shape) in projs.items()})
    else:
        write_nf4_safetensors(tmp_path / "model.safetensors", {
            n: Nf4Param(packed=torch.from_numpy(p), absmax=st, code=code, blocksize=64, shape=shape,
                        dtype="float16") for n, (p, st, shape) in projs.items()})

    def f16(shape, std):
        return (rng.standard_normal(shape) * std).astype(np.float16)

    enc_w, enc_b, score_w, score_b = f16((R, H), 0.02), f16((R,), 0.02), f16((NB, R), 0.02), f16((NB,), 0.02)
    torch.save({"config": {"artifact_target": "intermediate_block_scores", "block_domain": "intermediate",
                           "basis_rank": R, "basis_top_k": R, "block_size": 32, "num_blocks": NB,
                           "top_k_by_layer": {str(li): k}},
                "layer_selection": [li],
                "layer_states": {str(li): {"encoder_weight": torch.from_numpy(enc_w),
                                           "encoder_bias": torch.from_numpy(enc_b),
                                           "score_weight": torch.from_numpy(score_w),
                                           "score_bias": torch.from_numpy(score_b), "scale": torch.tensor(1.0)}},
                "stats": {}}, tmp_path / "basis.pt")
    x = f16((H,), 1.0)

    routing = load_routing_artifact(tmp_path / "basis.pt", hidden_size=H, intermediate_size=I, device=gpu)
    table = slot_table_from_safetensors(tmp_path, li, device=gpu)
    assert (table.nested is not None) == nested
    layer = SparseMlpLayer(router_from_routing(routing[li], gpu), table, routing[li]["top_k"])
    out, sel = layer.forward(torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()

    u16 = lambda a: a.view(np.uint16)  # noqa: E731
    _, _, sel_o = orc.route(u16(x), u16(enc_w), u16(enc_b), u16(score_w), u16(score_b), k)
    sel_np = sel.cpu().numpy().astype(np.int64)
    assert np.array_equal(sel_np, np.sort(sel_o)), "routed blocks differ from the oracle"
    g_p, g_a = orc.gather_rows_blocks(gp, ga, sel_np, H, 64)
    u_p, u_a = orc.gather_rows_blocks(upk, ua, sel_np, H, 64)
    d_p, d_a = orc.gather_down_columns(dp, da, sel_np, H, I, 64)
    ye, yf = orc.sparse_mlp(u16(x).reshape(1, H), np.arange(k, dtype=np.int32).reshape(1, k), g_p, g_a, u_p, u_a,
                            d_p, d_a, qbs=64)
    y = out.cpu().numpy().astype(np.float64)
    _check_tolerance(orc, y, ye[0], orc.f16_bits_to_f32(yf[0]).astype(np.float64),
                     f"disk-loaded layer nested={nested} hand_packed={hand_packed}")
