"""GPU NF4 LM head (nsmlp_dense_linear_nf4_f16; runtime/lm_head.py:450-474)
against the oracle.

Bar:
  * known answers (codes -1/0/+1, power-of-two absmax, integer x): bit-exact,
    fp32 sums and fp16 logits (these values are exact in the fp16 code table
    and every partial sum is exact in fp32, in any order);
  * random weights: per logit |y - exact| <= (2^-11 + in 2^-24) sum_c |w x|
    (the kernel's fp16 code table moves each code by at most 2^-11 relative;
    fp32 accumulation of `in` terms), relL2 <= 1e-3, and the fp16 logits are
    the round-to-nearest of the kernel's own fp32 sums;
  * double-quantised absmax: bit-identical to the fp32 path over the
    resolved absmax (the kernel resolves each absmax to the same fp32 value);
  * one and two token rows per pass give bit-identical logits.
"""
import numpy as np
import pytest
import torch

from tests.test_oracle_lm_head import _known_case

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().contiguous().numpy()


def _run(gpu, x, packed, absmax, code, V, H, qbs, with_f32=True):
    from next_step_ai_amd.lm_head import dense_linear_nf4

    xt = torch.from_numpy(x).to(gpu)
    f32 = torch.empty((x.shape[0], V), dtype=torch.float32, device=gpu) if with_f32 else None
    out = dense_linear_nf4(xt, packed, absmax, code, V, H, qbs, out_f32=f32)
    torch.cuda.synchronize()
    return out, f32


@pytest.mark.parametrize("V,H,qbs,rows", [
    (5, 64, 32, 1),        # one split, lanes past the row load zeros
    (37, 96, 32, 3),       # ragged vocabulary, two rows then one
    (1001, 2048, 64, 2),   # one full split per wave (8 items per round)
    (403, 6144, 64, 3),    # three splits: two waves idle
    (517, 16384, 256, 2),  # eight splits (the 405B hidden size)
])
def test_dense_linear_known_answers_bit_exact(gpu, orc, V, H, qbs, rows):
    print(f"lm head known answer V={V} H={H} qbs={qbs} rows={rows}", flush=True)
    rng = np.random.default_rng(V + H)
    packed, absmax, x, ref = _known_case(rng, V, H, qbs, rows)
    x = np.clip(x, -2, 2).astype(np.float16)
    ref = orc.dense_linear_nf4(x.view(np.uint16), packed, absmax, V, H, qbs)
    code = torch.tensor(orc.nf4_code(), device=gpu)
    out, f32 = _run(gpu, x, torch.from_numpy(packed).to(gpu), torch.from_numpy(absmax).to(gpu), code, V, H, qbs)
    assert np.array_equal(_np(f32).astype(np.float64), ref)
    assert np.array_equal(_np(out).view(np.uint16), orc.f32_to_f16_bits(ref.astype(np.float32)))


def _random_case(gpu, orc, rng, V, H, qbs, rows):
    w = (rng.standard_normal((V, H)) * 0.02).astype(np.float32)
    packed, absmax = orc.nf4_quantize(w, qbs)
    x = rng.standard_normal((rows, H)).astype(np.float16)
    return packed, absmax, x


def _check_random(orc, x, packed, absmax, V, H, qbs, out, f32):
    exact = orc.dense_linear_nf4(x.view(np.uint16), packed, absmax, V, H, qbs)
    wd = orc.nf4_dequant(packed, absmax, V * H, qbs).reshape(V, H).astype(np.float64)
    mag = np.abs(x.astype(np.float64)) @ np.abs(wd).T
    got = _np(f32).astype(np.float64)
    bound = (2.0 ** -11 + H * 2.0 ** -24) * mag + 1e-30
    worst = float(np.max(np.abs(got - exact) / bound))
    e = orc.rel_l2(got, exact)
    print(f"  relL2(f32, exact)={e:.3e} worst |err|/bound={worst:.3f}", flush=True)
    assert worst <= 1.0
    assert e <= 1e-3
    assert np.array_equal(_np(out).view(np.uint16), orc.f32_to_f16_bits(_np(f32)))


@pytest.mark.parametrize("V,H,qbs,rows", [(300, 4096, 64, 1), (129, 8192, 64, 3), (64, 5120, 128, 2)])
def test_dense_linear_random_within_bound(gpu, orc, V, H, qbs, rows):
    print(f"lm head random V={V} H={H} qbs={qbs} rows={rows}", flush=True)
    rng = np.random.default_rng(3 * V + H)
    packed, absmax, x = _random_case(gpu, orc, rng, V, H, qbs, rows)
    code = torch.tensor(orc.nf4_code(), device=gpu)
    out, f32 = _run(gpu, x, torch.from_numpy(packed).to(gpu), torch.from_numpy(absmax).to(gpu), code, V, H, qbs)
    _check_random(orc, x, packed, absmax, V, H, qbs, out, f32)


def test_dense_linear_nested_absmax_bit_identical(gpu, orc):
    from next_step_ai_amd.nested_absmax import NestedAbsmax

    V, H, qbs, rows = 777, 4096, 64, 2
    print(f"lm head nested absmax V={V} H={H}", flush=True)
    rng = np.random.default_rng(11)
    packed, absmax, x = _random_case(gpu, orc, rng, V, H, qbs, rows)
    code = torch.tensor(orc.nf4_code(), device=gpu)
    pk = torch.from_numpy(packed).to(gpu)
    nested = NestedAbsmax.quantize(torch.from_numpy(absmax).to(gpu))
    resolved = nested.resolve()
    out_n, f32_n = _run(gpu, x, pk, nested, code, V, H, qbs)
    out_r, f32_r = _run(gpu, x, pk, resolved, code, V, H, qbs)
    assert torch.equal(f32_n, f32_r) and torch.equal(out_n, out_r)
    _check_random(orc, x, packed, _np(resolved), V, H, qbs, out_r, f32_r)


def test_lm_head_forward_matches_reference_call(gpu, orc):
    """lm_head_forward over the reference's meta dict equals the dense product,
    and a meta with a partial active_idx goes through the sparse input linear
    with 256-column blocks (the reference's own call, lm_head.py:461-473)."""
    from next_step_ai_amd.lm_head import dense_linear_nf4, lm_head_forward, lm_head_nf4_meta

    V, H, qbs = 500, 2048, 64
    rng = np.random.default_rng(5)
    packed, absmax, x = _random_case(gpu, orc, rng, V, H, qbs, 3)
    code = torch.tensor(orc.nf4_code(), device=gpu)
    meta = lm_head_nf4_meta(torch.from_numpy(packed).to(gpu), torch.from_numpy(absmax).to(gpu), code, V, H, qbs)
    assert meta["block_size"] == 256
    hidden = torch.from_numpy(x).to(gpu).view(1, 3, H)
    logits = lm_head_forward(hidden, meta)
    assert logits.shape == (1, 3, V) and logits.dtype == torch.float16
    direct = dense_linear_nf4(hidden.view(3, H), meta["packed_weight"], meta["absmax"], code, V, H, qbs)
    assert torch.equal(logits.view(3, V), direct)
    bf = lm_head_forward(hidden.to(torch.bfloat16), meta)
    assert bf.dtype == torch.bfloat16
    # partial selection: blocks 1, 3, 6 of 8 (256 columns each)
    sparse = dict(meta, active_idx=torch.tensor([[1, 3, 6]], dtype=torch.int32, device=gpu))
    got = _np(lm_head_forward(hidden, sparse)).reshape(3, V).astype(np.float64)
    wd = orc.nf4_dequant(packed, absmax, V * H, qbs).reshape(V, H).astype(np.float64)
    cols = np.concatenate([np.arange(b * 256, (b + 1) * 256) for b in (1, 3, 6)])
    ref = x.astype(np.float64)[:, cols] @ wd[:, cols].T
    assert orc.rel_l2(got, ref) < 2e-3


def test_lm_head_405b_vocab_sampled_rows(gpu, orc):
    """The full 405B head (vocabulary 128256 x hidden 16384, 1.05 GB packed):
    256 sampled logits per token against the oracle, and one- and two-row
    passes bit-identical."""
    from next_step_ai_amd.lm_head import dense_linear_nf4
    from next_step_ai_amd.synth import synth_nf4, synth_normal_f16

    V, H, qbs = 128256, 16384, 64
    print(f"lm head 405B V={V} H={H}", flush=True)
    packed, absmax = synth_nf4(61, V * H, qbs, 0.02, gpu)
    code = torch.tensor(orc.nf4_code(), device=gpu)
    x = synth_normal_f16(62, (2, H), 1.0, gpu)
    f32 = torch.empty((2, V), dtype=torch.float32, device=gpu)
    out2 = dense_linear_nf4(x, packed, absmax, code, V, H, qbs, out_f32=f32)
    out1 = dense_linear_nf4(x[:1], packed, absmax, code, V, H, qbs)
    torch.cuda.synchronize()
    assert torch.equal(out1[0], out2[0])
    rows = torch.from_numpy(np.sort(np.random.default_rng(9).choice(V, 256, replace=False))).to(gpu)
    pk_rows = _np(packed.view(V, H // 2).index_select(0, rows))
    am_rows = _np(absmax.view(V, H // qbs).index_select(0, rows))
    xs = _np(x)
    sub_out = out2.index_select(1, rows)
    sub_f32 = f32.index_select(1, rows).contiguous()
    _check_random(orc, xs, pk_rows, am_rows, 256, H, qbs, sub_out.contiguous(), sub_f32)
    del packed, absmax


@pytest.mark.parametrize("V,H,qbs,rows", [(1, 32, 32, 1), (3, 64, 32, 5), (6, 2080, 32, 2)])
def test_dense_linear_tiny_and_ragged_shapes(gpu, orc, V, H, qbs, rows):
    """Fewer rows than one 4-row item, one active lane, a split with a single
    32-column lane group past 2048 columns, five token rows (2 + 2 + 1)."""
    print(f"lm head tiny V={V} H={H} rows={rows}", flush=True)
    rng = np.random.default_rng(V * 7 + H)
    packed, absmax, x, ref = _known_case(rng, V, H, qbs, rows)
    x = np.clip(x, -2, 2).astype(np.float16)
    ref = orc.dense_linear_nf4(x.view(np.uint16), packed, absmax, V, H, qbs)
    code = torch.tensor(orc.nf4_code(), device=gpu)
    out, f32 = _run(gpu, x, torch.from_numpy(packed).to(gpu), torch.from_numpy(absmax).to(gpu), code, V, H, qbs)
    assert np.array_equal(_np(f32).astype(np.float64), ref)
    assert np.array_equal(_np(out).view(np.uint16), orc.f32_to_f16_bits(ref.astype(np.float32)))
