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
