"""The layer block bank (MlpBlockBankLayout and its projection check,
runtime/block_bank.py:7-101 in the reference) and where this build applies
it: the routing artifact's ``block_bank_layout`` (RT:906-912) and the slot
table's checkpoint shapes before a table is built (RT:5171-5172).  CPU only:
every check raises before any device work."""
import numpy as np
import pytest
import torch

from next_step_ai_amd.layout import (MlpBlockBankLayout, build_intermediate_mlp_block_bank_layout,
                                     validate_intermediate_mlp_block_bank_params)


def _layout(**kw):
    args = dict(layer_idx=2, hidden_size=64, intermediate_size=256, block_size=32, num_blocks=8)
    args.update(kw)
    return MlpBlockBankLayout(**args)


def test_layout_fields_bounds_and_dict():
    L = _layout()
    assert L.block_bounds(0) == (0, 32) and L.block_bounds(7) == (224, 256)
    assert L.as_dict() == {"layer_idx": 2, "hidden_size": 64, "intermediate_size": 256, "block_size": 32,
                           "num_blocks": 8}
    for b in (-1, 8):
        with pytest.raises(RuntimeError, match="no block"):
            L.block_bounds(b)
    with pytest.raises(Exception):
        L.num_blocks = 9  # frozen


@pytest.mark.parametrize("kw,msg", [
    ({"layer_idx": -1}, "negative"),
    ({"hidden_size": 0}, "hidden_size = 0"),
    ({"intermediate_size": 0}, "intermediate_size = 0"),
    ({"block_size": 0}, "block_size = 0"),
    ({"intermediate_size": 250}, "leave 26"),     # 250 = 7 * 32 + 26
    ({"num_blocks": 7}, "make 8 blocks"),
])
def test_layout_rules(kw, msg):
    with pytest.raises(RuntimeError, match=msg):
        _layout(**kw)


def test_build_layout_infers_or_checks_the_block_count():
    L = build_intermediate_mlp_block_bank_layout(layer_idx=0, hidden_size=16384, intermediate_size=53248,
                                                 block_size=32)
    assert L.num_blocks == 1664
    with pytest.raises(RuntimeError, match="make 1664 blocks"):
        build_intermediate_mlp_block_bank_layout(layer_idx=0, hidden_size=16384, intermediate_size=53248,
                                                 block_size=32, num_blocks=1665)


_GOOD = dict(gate_in_features=64, gate_out_features=256, up_in_features=64, up_out_features=256,
             down_in_features=256, down_out_features=64)


@pytest.mark.parametrize("field,value,name", [
    ("gate_in_features", 65, "gate"), ("up_in_features", 32, "up"),
    ("gate_out_features", 224, "gate"), ("up_out_features", 288, "up"),
    ("down_in_features", 64, "down"), ("down_out_features", 256, "down"),
])
def test_projection_rules(field, value, name):
    validate_intermediate_mlp_block_bank_params(layout=_layout(), **_GOOD)
    feats = dict(_GOOD, **{field: value})
    with pytest.raises(RuntimeError, match=f"layer 2: .*{name} maps"):
        validate_intermediate_mlp_block_bank_params(layout=_layout(), **feats)


def test_transposed_down_names_every_mismatch():
    feats = dict(_GOOD, down_in_features=64, down_out_features=256)
    with pytest.raises(RuntimeError) as e:
        validate_intermediate_mlp_block_bank_params(layout=_layout(), **feats)
    assert "down maps 64 -> 256" in str(e.value) and "needs 256 -> 64" in str(e.value)


def test_routing_artifact_carries_the_block_bank(tmp_path):
    from next_step_ai_amd.loaders import load_routing_artifact

    H, I, R, NB = 64, 256, 4, 8
    g = torch.Generator().manual_seed(0)
    state = {"encoder_weight": torch.randn(R, H, generator=g), "encoder_bias": torch.randn(R, generator=g),
             "score_weight": torch.randn(NB, R, generator=g), "score_bias": torch.randn(NB, generator=g),
             "block_domain": "intermediate"}
    torch.save({"config": {"block_size": 32, "artifact_target": "intermediate_block_scores"},
                "layer_states": {"5": state}}, tmp_path / "r.pt")
    r = load_routing_artifact(tmp_path / "r.pt", hidden_size=H, intermediate_size=I, sparse_top_k=3)
    L = r[5]["block_bank_layout"]
    assert isinstance(L, MlpBlockBankLayout)
    assert L.as_dict() == {"layer_idx": 5, "hidden_size": H, "intermediate_size": I, "block_size": 32,
                           "num_blocks": NB}


def _checkpoint(tmp_path, orc, shapes):
    from next_step_ai_amd.loaders import Nf4Param, write_nf4_safetensors

    params = {}
    rng = np.random.default_rng(3)
    for name, (o, i) in shapes.items():
        packed, absmax = orc.nf4_quantize((rng.standard_normal(o * i) * 0.02).astype(np.float32), qbs=64)
        params[f"model.layers.0.mlp.{name}_proj.weight"] = Nf4Param(
            packed=torch.from_numpy(packed), absmax=torch.from_numpy(absmax),
            code=torch.from_numpy(orc.nf4_code().astype(np.float32)), blocksize=64, shape=(o, i), dtype="float16")
    write_nf4_safetensors(tmp_path / "m.safetensors", params)


def test_checkpoint_shapes_checked_before_the_table(tmp_path, orc):
    """A down projection stored for another intermediate size, or a layout
    of another bank, is refused before anything reaches a device."""
    from next_step_ai_amd.loaders import slot_table_from_safetensors

    _checkpoint(tmp_path, orc, {"gate": (256, 64), "up": (256, 64), "down": (64, 288)})
    with pytest.raises(RuntimeError, match="down maps 288 -> 64 features, the bank needs 256 -> 64"):
        slot_table_from_safetensors(tmp_path, 0, device=torch.device("cpu"))
    _checkpoint(tmp_path, orc, {"gate": (256, 64), "up": (256, 64), "down": (64, 256)})
    other = build_intermediate_mlp_block_bank_layout(layer_idx=0, hidden_size=64, intermediate_size=512,
                                                     block_size=32)
    with pytest.raises(RuntimeError, match="gate maps 64 -> 256 features, the bank needs 64 -> 512"):
        slot_table_from_safetensors(tmp_path, 0, device=torch.device("cpu"), block_bank_layout=other)


def test_table_from_tensors_checks_the_bank():
    """from_reference checks the bank (features implied by the packed sizes)
    before it needs the device: a gate of the wrong size, or absmax of the
    wrong length, is refused."""
    from next_step_ai_amd.slot_table import _check_bank

    H, I, qbs = 64, 256, 64
    gp, up, dp = (torch.zeros(H * I // 2, dtype=torch.uint8) for _ in range(3))
    ga, ua, da = (torch.zeros(H * I // qbs) for _ in range(3))
    _check_bank(0, None, None, H, I, qbs, gp, ga, up, ua, dp, da)
    with pytest.raises(RuntimeError, match="gate maps 64 -> 224"):
        _check_bank(0, None, None, H, I, qbs, gp[: H * 224 // 2], ga, up, ua, dp, da)
    with pytest.raises(RuntimeError, match="up absmax has 255 entries, expected 256"):
        _check_bank(0, None, None, H, I, qbs, gp, ga, up, ua[:255], dp, da)
    with pytest.raises(RuntimeError, match="the block bank is 64 x 512"):
        _check_bank(0, build_intermediate_mlp_block_bank_layout(layer_idx=0, hidden_size=64,
                                                                intermediate_size=512, block_size=32),
                    None, H, I, qbs, gp, ga, up, ua, dp, da)
