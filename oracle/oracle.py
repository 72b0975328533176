"""CPU oracle for the blockwise-sparse NF4 MLP decode path.

TEST INFRASTRUCTURE ONLY.  This module is the checker: ``tests/``,
``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` are the
only code that may import it.  The product (``next_step_ai_amd``) never imports
it and has no CPU fallback.

Heavy arithmetic lives in ``nsmlp_oracle.c`` (loaded through ctypes); the
host-side logic of the reference path is restated here in numpy.  Every
function cites the reference lines it follows (paths relative to the reference
repository; RT = llama3_neuroplastic/experiments/streaming_llama_runtime.py,
TSM = llama3_neuroplastic/triton_sparse_mlp.py).

Pinning status (what checks each function, see tests/test_oracle_*.py):
  f16 conversions        numpy float16 (IEEE RNE), exhaustive over fp16
  exact dot + rounding   Python Fraction brute force; numpy fp64 where exact
  route                  brute force on tiny NB; torch fp16 CPU (informative)
  active_layout          torch.unique / reference test expectations
  gather_* (slot/gather) reference tests test_down_proj_col_cache.py /
                         test_prewarm_col_cache.py expectations
  plan / promote_blocks  reference test test_throughput_contract.py:308-321
                         expectations; the argmin rule by brute force
  calibration_counts     reference test test_throughput_contract.py:261-287
                         (recency order) and a closed form per block
  nf4 quantize/dequant   closed-form invariants (round trip, nearest code);
                         bitsandbytes itself is absent: parity unpinned
  double quant           closed-form invariants; bitsandbytes absent: parity unpinned
  sparse_mlp             dense-MLP closed form (all blocks), numpy fp64
  dense_linear_nf4       hand-packed known answers (codes -1/0/+1, power-of-
                         two absmax, integer x: exact sums), ragged shapes
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libnsmlp_oracle.so")
_lib = None

BLOCK = 32


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        from . import build as _build  # type: ignore
        _build.build()
    lib = ctypes.CDLL(_LIB_PATH)
    P = ctypes.c_void_p
    L = ctypes.c_long
    I = ctypes.c_int
    lib.orc_f16_to_f32.restype = ctypes.c_float
    lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.orc_f32_to_f16.restype = ctypes.c_uint16
    lib.orc_f32_to_f16.argtypes = [ctypes.c_float]
    lib.orc_f64_to_f16.restype = ctypes.c_uint16
    lib.orc_f64_to_f16.argtypes = [ctypes.c_double]
    lib.orc_fix48_to_f16.restype = ctypes.c_uint16
    lib.orc_fix48_to_f16.argtypes = [ctypes.c_int64, ctypes.c_uint64]
    lib.orc_dot_exact_f16.restype = ctypes.c_uint16
    lib.orc_dot_exact_f16.argtypes = [P, P, L, P]
    lib.orc_dot_exact_fix48.restype = I
    lib.orc_dot_exact_fix48.argtypes = [P, P, L, P, P, P]
    lib.orc_route_f16.restype = I
    lib.orc_route_f16.argtypes = [P, I, P, P, I, I, P, P, P, I, I, I, P, P, P]
    lib.orc_nf4_code.restype = None
    lib.orc_nf4_code.argtypes = [P]
    lib.orc_nf4_quantize.restype = None
    lib.orc_nf4_quantize.argtypes = [P, L, I, P, P]
    lib.orc_nf4_dequant_f32.restype = None
    lib.orc_nf4_dequant_f32.argtypes = [P, P, L, I, P, P]
    lib.orc_dynamic_map_signed.restype = None
    lib.orc_dynamic_map_signed.argtypes = [P]
    lib.orc_double_quant.restype = None
    lib.orc_double_quant.argtypes = [P, L, P, P, P, P]
    lib.orc_double_dequant.restype = None
    lib.orc_double_dequant.argtypes = [P, P, ctypes.c_float, P, L, P]
    lib.orc_double_quant_ex.restype = None
    lib.orc_double_quant_ex.argtypes = [P, L, P, L, ctypes.c_float, P, P]
    lib.orc_double_dequant_ex.restype = None
    lib.orc_double_dequant_ex.argtypes = [P, P, ctypes.c_float, P, L, L, P]
    lib.orc_sparse_mlp.restype = I
    lib.orc_sparse_mlp.argtypes = [I, I, I, I, P, P, I, P, P, P, P, P, P, P, P, P, P]
    for name in ("orc_f32_to_f16_array", "orc_f16_to_f32_array", "orc_f64_to_f16_array"):
        getattr(lib, name).restype = None
        getattr(lib, name).argtypes = [P, L, P]
    lib.orc_num_threads.restype = I
    lib.orc_num_threads.argtypes = []
    lib.orc_set_num_threads.restype = None
    lib.orc_set_num_threads.argtypes = [I]
    _lib = lib
    return lib


def _p(a):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def set_num_threads(n: int) -> None:
    _load().orc_set_num_threads(int(n))


def num_threads() -> int:
    return int(_load().orc_num_threads())


# ----------------------------------------------------------------- fp16 ---

def f32_to_f16_bits(a) -> np.ndarray:
    a = _c(a, np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    _load().orc_f32_to_f16_array(_p(a), a.size, _p(out))
    return out


def f64_to_f16_bits(a) -> np.ndarray:
    a = _c(a, np.float64)
    out = np.empty(a.shape, dtype=np.uint16)
    _load().orc_f64_to_f16_array(_p(a), a.size, _p(out))
    return out


def f16_bits_to_f32(a) -> np.ndarray:
    a = _c(a, np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    _load().orc_f16_to_f32_array(_p(a), a.size, _p(out))
    return out


def fix48_to_f16_bits(v: int) -> int:
    """Round the exact value v * 2^-48 (v a Python int, |v| < 2^127) to fp16 bits."""
    v = int(v)
    lo = v & ((1 << 64) - 1)
    hi = (v >> 64)
    if hi >= (1 << 63):
        hi -= 1 << 64
    return int(_load().orc_fix48_to_f16(ctypes.c_int64(hi), ctypes.c_uint64(lo)))


def dot_exact_fix48(a16, b16, bias16=None) -> int:
    """Exact sum a.b (+bias) of fp16 bit arrays as an integer multiple of 2^-48."""
    a16 = _c(a16, np.uint16)
    b16 = _c(b16, np.uint16)
    bias = None if bias16 is None else _c(np.array([bias16]), np.uint16)
    hi = ctypes.c_int64()
    lo = ctypes.c_uint64()
    rc = _load().orc_dot_exact_fix48(_p(a16), _p(b16), a16.size, _p(bias), ctypes.byref(hi), ctypes.byref(lo))
    if rc != 0:
        raise ValueError("non-finite input")
    return (int(hi.value) << 64) | int(lo.value)


def dot_exact_f16(a16, b16, bias16=None) -> int:
    a16 = _c(a16, np.uint16)
    b16 = _c(b16, np.uint16)
    bias = None if bias16 is None else _c(np.array([bias16]), np.uint16)
    return int(_load().orc_dot_exact_f16(_p(a16), _p(b16), a16.size, _p(bias)))


# --------------------------------------------------------------- router ---

def route(x16, enc_w16, enc_b16, score_w16, score_b16, k, *, basis_top_k=None, down_block_norm=None,
          legacy_abs=False):
    """One-token router (RT:4209-4238 latent, RT:4311-4352 scores/top-k).

    All fp16 inputs are given as uint16 bit arrays.  Returns
    (latent16 [R], scores16 [NB], sel [k] int32 in (score desc, index asc) order).
    ``legacy_abs`` restates the path without ``route_score_weight``
    (RT:4332-4334): scores = |latent| @ dec_norm_t, with ``score_w16`` holding
    dec_norm_t transposed ([NB, R]) and no bias or clamp.
    """
    x16 = _c(x16, np.uint16).reshape(-1)
    enc_w16 = _c(enc_w16, np.uint16)
    R, H = enc_w16.shape
    assert x16.size == H
    enc_b = None if enc_b16 is None else _c(enc_b16, np.uint16).reshape(-1)
    score_w16 = _c(score_w16, np.uint16)
    NB = score_w16.shape[0]
    assert score_w16.shape[1] == R
    sb = None if score_b16 is None else _c(score_b16, np.uint16).reshape(-1)
    dbn = None if down_block_norm is None else _c(down_block_norm, np.float32).reshape(-1)
    btk = R if basis_top_k is None else int(basis_top_k)
    kk = max(1, min(int(k), NB))
    latent = np.empty(R, dtype=np.uint16)
    scores = np.empty(NB, dtype=np.uint16)
    sel = np.empty(kk, dtype=np.int32)
    rc = _load().orc_route_f16(_p(x16), H, _p(enc_w16), _p(enc_b), R, btk, _p(score_w16), _p(sb), _p(dbn), NB,
                               1 if legacy_abs else 0, kk, _p(latent), _p(scores), _p(sel))
    if rc != 0:
        raise ValueError("non-finite router input")
    return latent, scores, sel


def f16_order_key(h16) -> np.ndarray:
    """Monotone integer key of fp16 bit patterns (-0 maps to +0)."""
    h = _c(h16, np.uint16).astype(np.uint32)
    h = np.where(h == 0x8000, 0, h)
    return np.where(h & 0x8000, (~h) & 0xFFFF, h | 0x8000).astype(np.uint32)


def topk_lowest_index(scores16, k) -> np.ndarray:
    """Selection rule: the k largest, ties broken by the lowest index."""
    key = f16_order_key(scores16).astype(np.int64)
    idx = np.arange(key.size, dtype=np.int64)
    order = np.lexsort((idx, -key))
    return order[: max(1, min(int(k), key.size))].astype(np.int32)


# --------------------------------------------------------------- layout ---

def active_layout(active_blocks, max_valid_blocks, block_size=BLOCK):
    """Restates _build_sparse_active_layout (RT:4857-4908) without a hot-cache
    ordering: union (rows>1), range filter, ``unique`` (ascending on CPU),
    ``active_local`` = slot of each routed block in the ordered list (-1 when
    invalid), ``flat_mask`` = per-row 0/1 over ordered slots repeated 32x,
    ``active_neurons`` = intermediate neuron ids of the ordered blocks."""
    ab = np.asarray(active_blocks, dtype=np.int64)
    if ab.ndim == 1:
        ab = ab.reshape(1, -1)
    rows = ab.shape[0]
    u = ab.reshape(-1)
    u = u[(u >= 0) & (u < int(max_valid_blocks))]
    ordered = np.unique(u).astype(np.int64)
    A = ordered.size
    lookup = np.full(int(max_valid_blocks), -1, dtype=np.int32)
    lookup[ordered] = np.arange(A, dtype=np.int32)
    valid = (ab >= 0) & (ab < int(max_valid_blocks))
    active_local = np.full(ab.shape, -1, dtype=np.int32)
    active_local[valid] = lookup[ab[valid]]
    slot_mask = np.zeros((rows, A), dtype=np.float32)
    for t in range(rows):
        s = active_local[t][active_local[t] >= 0]
        slot_mask[t, s] = 1.0
    flat_mask = np.repeat(slot_mask, block_size, axis=1)
    neurons = (ordered[:, None] * block_size + np.arange(block_size)[None, :]).reshape(-1)
    return ordered, active_local, flat_mask, neurons


# ------------------------------------------------------- gather / slots ---

def gather_rows_blocks(packed_flat, absmax_flat, blocks, in_features, qbs, block_size=BLOCK):
    """Gate/up gather (RT:4627-4660, RT:4530-4578): block b is rows
    [32b, 32b+32) of the row-major [out, in] weight, i.e. the contiguous byte
    range [b*32*in/2, (b+1)*32*in/2) and absmax range [b*32*in/qbs, ...)."""
    packed_flat = np.asarray(packed_flat, dtype=np.uint8).reshape(-1)
    absmax_flat = np.asarray(absmax_flat, dtype=np.float32).reshape(-1)
    bpb = block_size * in_features // 2
    apb = block_size * in_features // qbs
    pb = packed_flat.reshape(-1, bpb)
    ab = absmax_flat.reshape(-1, apb)
    idx = np.asarray(blocks, dtype=np.int64)
    return pb[idx].copy(), ab[idx].copy()


def gather_down_columns(packed_flat, absmax_flat, blocks, out_features, in_features, qbs, block_size=BLOCK):
    """Down-proj column gather (RT:4479-4528 _load_down_proj_cold_cols): per
    block b the byte slice raw_2d[:, b*bs/2 : b*bs/2 + bs/2] and the absmax
    column absmax_2d[:, (b*bs)//qbs]; stacked on dim 1 -> [H, n, bs/2], [H, n]."""
    raw_2d = np.asarray(packed_flat, dtype=np.uint8).reshape(out_features, in_features // 2)
    abs_2d = np.asarray(absmax_flat, dtype=np.float32).reshape(out_features, in_features // qbs)
    bpc = block_size // 2
    idx = np.asarray(blocks, dtype=np.int64)
    cols = (idx[:, None] * bpc + np.arange(bpc)[None, :]).reshape(-1)
    packed = raw_2d[:, cols].reshape(out_features, idx.size, bpc).copy()
    absmax = abs_2d[:, (idx * block_size) // qbs].copy()
    return packed, absmax


def partition_by_lookup(lookup, selected):
    """The hot/cold split of a selection (RT:3588-3604): a selected block is hot
    when its slot lookup is >= 0.  Returns (positions of the hot entries in
    the selection, their slots, the cold block ids in selection order, the
    cold mask)."""
    lk = np.asarray(lookup, dtype=np.int64)
    sel = np.asarray(selected, dtype=np.int64)
    slot = lk[sel]
    hot = slot >= 0
    pos = np.flatnonzero(hot)
    return pos, slot[pos], sel[~hot], ~hot


def plan_fixed_capacity_bank_update(existing_block_ids, existing_scores, active_count, capacity, novel_blocks):
    """Restates _plan_fixed_capacity_bank_update (RT:2576-2617): fill free slots
    first, then replace the lowest-score slot; a new block's score is
    (max active score + 1) + (i+1)*1e-3."""
    cap = max(0, int(capacity))
    ids = np.array(existing_block_ids, dtype=np.int64).copy()
    scores = np.array(existing_scores, dtype=np.float32).copy()
    active = max(0, min(int(active_count), ids.size, cap))
    novel = np.asarray(novel_blocks, dtype=np.int64).reshape(-1)
    if cap <= 0 or novel.size == 0:
        return np.zeros(0, dtype=np.int64), ids, scores, active
    novel = novel[:cap]
    base = float(scores[:active].max()) + 1.0 if active > 0 else 1.0
    nxt = active
    slots = []
    for i, b in enumerate(novel.tolist()):
        if nxt < cap:
            s = nxt
            nxt += 1
            active = max(active, s + 1)
        else:
            s = int(np.argmin(scores[:cap]))
        ids[s] = b
        scores[s] = np.float32(base + float(i + 1) * 1e-3)
        slots.append(s)
    return np.array(slots, dtype=np.int64), ids, scores, active


def promote_blocks(lookup, slot_block, slot_score, active_count, blocks, *, grow_only=False):
    """One promotion of a token's selected ``blocks`` into a fixed-capacity
    bank, as the reference's down-bank promotion takes it (RT:2908-3018):
    the novel blocks are the valid ids not in ``lookup`` (first occurrence, in
    order), planned by ``plan_fixed_capacity_bank_update``; an evicted
    block's lookup entry becomes -1 and a promoted block's its slot.  With
    ``grow_only`` only the free slots are used (the gate/up hot cache, which
    grows and never evicts, RT:2809-2906).  Returns (lookup, slot_block,
    slot_score, active_count, slot per entry of blocks or -1)."""
    lookup = np.array(lookup, dtype=np.int64).copy()
    NB = lookup.size
    cap = len(slot_block)
    novel, seen = [], set()
    for b in [int(v) for v in np.asarray(blocks).reshape(-1)]:
        if 0 <= b < NB and lookup[b] < 0 and b not in seen:
            novel.append(b)
            seen.add(b)
    active = max(0, min(int(active_count), cap))
    if grow_only:
        novel = novel[:cap - active]
    slots, ids, scores, active_new = plan_fixed_capacity_bank_update(slot_block, slot_score, active, cap, novel)
    old_ids = np.array(slot_block, dtype=np.int64)
    for b, s in zip(novel, slots.tolist()):
        o = int(old_ids[s])
        if 0 <= o < NB and lookup[o] == s:
            lookup[o] = -1
        lookup[b] = s
    slot_of = {b: s for b, s in zip(novel, slots.tolist())}
    per_entry, given = [], set()
    for b in [int(v) for v in np.asarray(blocks).reshape(-1)]:
        if b in slot_of and b not in given:
            per_entry.append(slot_of[b])
            given.add(b)
        else:
            per_entry.append(-1)
    return lookup, ids, scores, active_new, np.array(per_entry, dtype=np.int64)


def calibration_counts(counts, active_blocks, num_blocks, recency_power):
    """Restates _record_hot_cache_calibration_blocks (RT:2205-2243): rows of
    active_blocks [N, k]; row r weighs ((r + 1) / N) ** power (fp32); every
    valid id of the row adds the weight to its count, row by row (fp32 adds
    in entry order, as index_add_ on the CPU)."""
    counts = np.array(counts, dtype=np.float32).copy()
    rows = np.asarray(active_blocks, dtype=np.int64)
    rows = rows.reshape(-1, rows.shape[-1] if rows.ndim > 0 else 1)
    n = rows.shape[0]
    # the weights as the reference computes them: torch.pow in fp32 on the CPU
    # (numpy's float32 power can differ from it in the last place)
    import torch

    pos = torch.arange(1, n + 1, dtype=torch.float32)
    w = torch.pow(pos / float(max(n, 1)), float(recency_power)).numpy()
    for r in range(n):
        for b in rows[r].tolist():
            if 0 <= b < num_blocks:
                counts[b] = np.float32(counts[b] + w[r])
    return counts


# ------------------------------------------------------------------ NF4 ---

def nf4_code() -> np.ndarray:
    out = np.empty(16, dtype=np.float32)
    _load().orc_nf4_code(_p(out))
    return out


def nf4_quantize(w, qbs=64):
    """Blockwise NF4 quantisation (restated bitsandbytes quantize_4bit, nf4)."""
    w = _c(w, np.float32).reshape(-1)
    n = w.size
    assert n % qbs == 0 and qbs % 2 == 0
    packed = np.empty(n // 2, dtype=np.uint8)
    absmax = np.empty(n // qbs, dtype=np.float32)
    _load().orc_nf4_quantize(_p(w), n, int(qbs), _p(packed), _p(absmax))
    return packed, absmax


def nf4_dequant(packed, absmax, n, qbs=64, code=None):
    packed = _c(packed, np.uint8).reshape(-1)
    absmax = _c(absmax, np.float32).reshape(-1)
    code = nf4_code() if code is None else _c(code, np.float32)
    out = np.empty(int(n), dtype=np.float32)
    _load().orc_nf4_dequant_f32(_p(packed), _p(absmax), int(n), int(qbs), _p(code), _p(out))
    return out


def dynamic_map_signed() -> np.ndarray:
    out = np.empty(256, dtype=np.float32)
    _load().orc_dynamic_map_signed(_p(out))
    return out


def double_quant(absmax, map256=None, *, dq_block=256, offset=None):
    """bitsandbytes double quantisation of an fp32 absmax vector (restated):
    returns (q u8, absmax2 f32, offset).  ``offset`` defaults to the mean."""
    absmax = _c(absmax, np.float32).reshape(-1)
    m = dynamic_map_signed() if map256 is None else _c(map256, np.float32)
    n = absmax.size
    q = np.empty(n, dtype=np.uint8)
    a2 = np.empty((n + dq_block - 1) // dq_block, dtype=np.float32)
    if offset is None:
        if dq_block != 256:
            raise ValueError("the mean offset is computed for dq_block=256 only; pass offset")
        off = np.empty(1, dtype=np.float32)
        _load().orc_double_quant(_p(absmax), n, _p(m), _p(q), _p(a2), _p(off))
        return q, a2, float(off[0])
    _load().orc_double_quant_ex(_p(absmax), n, _p(m), int(dq_block), ctypes.c_float(offset), _p(q), _p(a2))
    return q, a2, float(np.float32(offset))


def double_dequant(q, absmax2, offset, map256=None, *, dq_block=256):
    q = _c(q, np.uint8).reshape(-1)
    a2 = _c(absmax2, np.float32).reshape(-1)
    m = dynamic_map_signed() if map256 is None else _c(map256, np.float32)
    out = np.empty(q.size, dtype=np.float32)
    _load().orc_double_dequant_ex(_p(q), _p(a2), ctypes.c_float(offset), _p(m), q.size, int(dq_block), _p(out))
    return out


# ------------------------------------------------------------------ MLP ---

def sparse_mlp(x16, active_local, gate_packed, gate_absmax, up_packed, up_absmax, down_packed, down_absmax,
               code=None, qbs=64, want_exact=True, want_fallback=True):
    """Blockwise-sparse NF4 MLP over the reference's gathered layouts
    (RT:5433-5492 fallback; TSM:807-914 single-kernel layout contract).

    x16 [rows, H] uint16 (fp16 bits); active_local [rows, kk] int32;
    gate/up packed [A, 32, H/2], absmax [A, 32, H/qbs]; down packed [H, A, 16],
    absmax [H, A].  Returns (y_exact fp64 [rows, H] or None,
    y_fallback fp16 bits [rows, H] or None)."""
    x16 = _c(x16, np.uint16)
    if x16.ndim == 1:
        x16 = x16.reshape(1, -1)
    rows, H = x16.shape
    al = _c(active_local, np.int32)
    if al.ndim == 1:
        al = al.reshape(1, -1)
    kk = al.shape[1]
    gp = _c(gate_packed, np.uint8)
    A = gp.size // (BLOCK * H // 2)
    ga = _c(gate_absmax, np.float32)
    up = _c(up_packed, np.uint8)
    ua = _c(up_absmax, np.float32)
    dp = _c(down_packed, np.uint8)
    da = _c(down_absmax, np.float32)
    assert gp.size == A * BLOCK * H // 2 and up.size == gp.size
    assert ga.size == A * BLOCK * H // qbs and ua.size == ga.size
    assert dp.size == H * A * BLOCK // 2 and da.size == H * A
    code = nf4_code() if code is None else _c(code, np.float32)
    ye = np.empty((rows, H), dtype=np.float64) if want_exact else None
    yf = np.empty((rows, H), dtype=np.uint16) if want_fallback else None
    rc = _load().orc_sparse_mlp(rows, H, A, int(qbs), _p(x16), _p(al), kk, _p(gp), _p(ga), _p(up), _p(ua), _p(dp),
                                _p(da), _p(code), _p(ye), _p(yf), None)
    if rc != 0:
        raise ValueError("unsupported shape")
    return ye, yf


def dense_linear_nf4(x16, packed, absmax, out_features, in_features, qbs, code=None):
    """The NF4 LM head (runtime/lm_head.py:450-474: triton_sparse_input_linear_4bit
    with every block active over the row-major [V, H] weight):
    y[t][o] = sum_c fp32(code[nib(o, c)] * absmax[(o*H + c) // qbs]) * x[t][c],
    element o*H + c in the high nibble of its byte when even (TSM:499-507,
    with the row-major element index the LM-head meta holds, lm_head.py:221-241).
    x16: fp16 bits [rows, H].  Returns the fp64 sums [rows, V]."""
    x = f16_bits_to_f32(np.asarray(x16, dtype=np.uint16).reshape(-1, int(in_features))).astype(np.float64)
    w = nf4_dequant(packed, absmax, int(out_features) * int(in_features), int(qbs), code)
    w = w.reshape(int(out_features), int(in_features)).astype(np.float64)
    return x @ w.T


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64).reshape(-1)
    b = np.asarray(b, dtype=np.float64).reshape(-1)
    den = float(np.linalg.norm(b))
    return float(np.linalg.norm(a - b)) / (den if den > 0 else 1.0)


# ---------------------------------------------------- synthetic (small) ---

def synthetic_layer_cpu(H, I, R, NB, seed, qbs=64, std=0.02):
    """Seeded synthetic layer for CPU-only checks (numpy Generator): NF4
    gate/up [I, H] and down [H, I] from N(0, std), router fp16 ~ N(0, std),
    x fp16 ~ N(0, 1).  Returns a dict of numpy arrays in the reference layouts."""
    rng = np.random.default_rng(seed)
    gate_w = (rng.standard_normal((I, H), dtype=np.float32) * std).astype(np.float32)
    up_w = (rng.standard_normal((I, H), dtype=np.float32) * std).astype(np.float32)
    down_w = (rng.standard_normal((H, I), dtype=np.float32) * std).astype(np.float32)
    gp, ga = nf4_quantize(gate_w, qbs)
    upk, ua = nf4_quantize(up_w, qbs)
    dp, da = nf4_quantize(down_w, qbs)
    enc_w = rng.standard_normal((R, H), dtype=np.float32) * std
    enc_b = rng.standard_normal((R,), dtype=np.float32) * std
    sw = rng.standard_normal((NB, R), dtype=np.float32) * std
    sb = rng.standard_normal((NB,), dtype=np.float32) * std
    x = rng.standard_normal((H,), dtype=np.float32)
    return {
        "H": H, "I": I, "R": R, "NB": NB, "qbs": qbs,
        "gate_packed": gp, "gate_absmax": ga, "up_packed": upk, "up_absmax": ua,
        "down_packed": dp, "down_absmax": da,
        "enc_w16": f32_to_f16_bits(enc_w), "enc_b16": f32_to_f16_bits(enc_b),
        "score_w16": f32_to_f16_bits(sw), "score_b16": f32_to_f16_bits(sb),
        "x16": f32_to_f16_bits(x),
    }
