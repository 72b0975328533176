#!/usr/bin/env python3
"""Benchmark: blockwise-sparse NF4 MLP decode, one 405B-shaped layer per step.

A step is one decode token through one layer's hot path: the learned-basis
router (exact fp16 dots + top-k with lowest-index ties) and the fused NF4
sparse MLP over the selected blocks, read straight from the HBM slot table.
Steps rotate over --layers distinct seeded layers (default 8, ~12 GB) so that
the 256 MB Infinity Cache cannot serve a layer's 191 MB of selected blocks.

Reported (one JSON line):
  value         decode_tok_s = 1e6 / (126 * us_per_layer), MLP-only (router +
                sparse MLP per layer, 126 layers per token)
  ms_per_step   wall time per layer (router + MLP), inputs resident in HBM
  roofline      the sparse-MLP decode launch pair (k_gu_rep + k_down_rep),
                timed with one pair of HIP events on its launch stream around
                all steps: algorithmic bytes per launch (selected packed NF4 +
                their absmax in the stored format + x + out) / mean duration.  traffic: HBM bytes per launch from the rocprofv3
                FETCH_SIZE / WRITE_SIZE summary committed for this workload,
                scaled by the same counters on a plain copy (null without it)
  cpu_baseline  the oracle's restatement of the reference PyTorch path
                (router + dequant fallback with fp16 rounding points) on the
                host cores, on the same layer shape

The weights are NF4 with double-quantised absmax (bitsandbytes
compress_statistics: u8 codes, one fp32 scale per 256, an offset), the format
the workload names; --absmax f32 stores the resolved fp32 absmax instead (the
reference runtime's slot-table format, RT:4621-4625).

--config 3 measures the same layer with half of the blocks in HBM slots and
the selected blocks' misses (62 of 208) read from pinned host copies over
the host link; --config 5 decodes 64 tokens through a stack of 126 resident
layers (x <- x + mlp(x)) and reports the end-to-end decode_tok_s; --config 6
times the NF4 LM head (vocabulary 128256 x hidden 16384) for one token;
--graph replays each config-5 token as one captured HIP graph; --config 7 times the
dense-guard prefill MLP (256 tokens through every block) on MFMA.
Each prints the same JSON line shape with its own config.

--copy-calibration BYTES runs only a plain device copy of BYTES (the
reference kernel for the counter calibration) and prints its size.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "sparse-MLP µs/layer + HBM GB/s vs peak, 405B shape top-k 208; decode_tok_s"
PEAK_GBS = 8000.0
MODEL_LAYERS = 126
# config id -> (hidden, intermediate, basis rank, top-k)
CONFIGS = {1: (4096, 14336, 64, 64), 2: (16384, 53248, 64, 208), 3: (16384, 53248, 64, 208),
           4: (16384, 53248, 64, 208), 5: (16384, 53248, 64, 208), 6: (16384, 53248, 64, 208),
           7: (16384, 53248, 64, 1664)}
LM_VOCAB = 128256
PREFILL_TOKENS = 256
PEAK_F16_TFLOPS = 2500.0  # dense fp16 MFMA
WORKLOADS = {
    1: "8B-shaped MLP layer decode: hidden 4096, intermediate 14336, block 32 (448 blocks), top-k 64",
    2: "405B-shaped MLP layer decode: hidden 16384, intermediate 53248, block 32 (1664 blocks), top-k 208",
    3: "405B-shaped MLP layer decode with partial residency: hidden 16384, intermediate 53248, top-k 208; "
       "832 of 1664 blocks in HBM slots, 62 of the 208 selected blocks read from pinned host copies",
    4: "405B-shaped MLP chunked prefill: 256 tokens, per-token top-208 routing unioned into a block set, "
       "grouped fp16 MFMA gate/up/down with SiLU fused (hidden 16384, intermediate 53248, block 32)",
    5: "126-layer stack of 405B-shaped MLP layers (hidden 16384, intermediate 53248, top-k 208), all resident; "
       "64 decode tokens at batch 1, x <- x + mlp(x) per layer",
    6: "405B NF4 LM head decode: logits over vocabulary 128256 from hidden 16384 (dense NF4 GEMV, "
       "every input block active), one token",
    7: "405B-shaped dense-guard prefill MLP: 256 tokens through every block (hidden 16384, intermediate 53248), "
       "fp16 MFMA GEMMs over NF4 weights decoded in registers",
}
STACK_LAYERS = 126
STACK_TOKENS = 64
# gate/up weights of the stack: N(0, 0.002), so that x <- x + mlp(x) stays
# finite over 126 layers with no norm in between (the MLP's gain grows with
# |x|^2; at 0.02 the hidden state overflows within a few layers); down and
# router N(0, 0.02); the bytes moved are the same
STACK_GATE_UP_STD = 0.002
C3_RESIDENT, C3_MISSES = 832, 62
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_sparse_mlp_decode.json")


def algorithmic_bytes(H: int, I: int, k: int, qbs: int, absmax: str = "dq8", dq_block: int = 256) -> int:
    """Bytes the sparse MLP must move once per layer: the selected blocks'
    packed NF4 (gate, up: 32 x H/2; down: H x 16) and absmax (gate, up:
    32 x H/qbs; down: H, one per row and block; 4 bytes fp32, or 1 byte u8
    double-quantised plus the fp32 second-level scales they use: per gate/up
    block its rows' 32 H/qbs / dq_block (at least 1), and the down weight's
    whole H I/qbs / dq_block), plus x and out."""
    ab = 4 if absmax == "f32" else 1
    per_block = 2 * (32 * H // 2 + ab * 32 * H // qbs) + (16 * H + ab * H)
    total = k * per_block + 2 * H * 2
    if absmax != "f32":
        total += 2 * k * 4 * max(1, 32 * H // qbs // dq_block) + 4 * (H * I // qbs // dq_block)
    return total


def router_bytes(H: int, R: int, NB: int) -> int:
    return 2 * (R * H + R + NB * R + NB + H)


def host_threads() -> int:
    """Threads for the CPU baseline: the host's CPU share when the
    environment sets one (OMP_NUM_THREADS; the GPU boxes allot 16 cores per
    GPU), else every core this process may run on."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    share = os.environ.get("OMP_NUM_THREADS", "").strip()
    if share.isdigit() and int(share) > 0:
        n = min(n, int(share))
    return max(1, n)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_description() -> dict:
    """The host the CPU baseline ran on: lscpu's model, sockets and cores,
    os.cpu_count(), the affinity mask and torch's thread count."""
    import subprocess

    import torch

    info = {"model": cpu_model(), "os_cpu_count": os.cpu_count()}
    try:
        info["affinity_cpus"] = len(os.sched_getaffinity(0))
    except AttributeError:
        pass
    info["torch_num_threads"] = torch.get_num_threads()
    info["omp_num_threads_env"] = os.environ.get("OMP_NUM_THREADS")
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        fields = dict(line.split(":", 1) for line in out.splitlines() if ":" in line)
        for key, name in (("Model name", "lscpu_model"), ("Socket(s)", "sockets"),
                          ("Core(s) per socket", "cores_per_socket"), ("Thread(s) per core", "threads_per_core")):
            if key in fields:
                v = fields[key].strip()
                info[name] = int(v) if v.isdigit() else v
    except (OSError, subprocess.SubprocessError, ValueError):
        pass
    return info


def measured_traffic(config: int, absmax: str):
    """HBM bytes per sparse-MLP launch pair from the committed counter
    summary, or None when there is none for this workload."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    entry = t.get("configs", {}).get(f"{config}-{absmax}")
    if not entry:
        return None
    return int(entry["fetch_bytes"] + entry["write_bytes"])


def _median_us(fn, runs: int) -> tuple[float, int]:
    """Median wall time of fn() in µs over max(10, runs) runs after 3 warm-ups."""
    for _ in range(3):
        fn()
    times = []
    for _ in range(max(10, runs)):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times) * 1e6, len(times)


def cpu_baseline(layer, sel, runs: int, H: int, I: int, k: int, qbs: int, absmax: str) -> dict:
    """Time the reference PyTorch path on the host cores: the torch-CPU
    restatement of the router, the active layout and the dequant fallback
    (RT:4209-4352, RT:4857-4908, RT:5433-5492) in fp16, over the selected
    blocks already gathered; beside it, the oracle's C port of the same path
    (fp16 rounding points, fp64 sums, OpenMP)."""
    import numpy as np
    import torch

    from oracle import oracle as orc
    from oracle import torch_reference as tref

    threads = host_threads()
    orc.set_num_threads(threads)
    torch_threads = torch.get_num_threads()
    torch.set_num_threads(threads)

    def u16(t):
        return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)

    def npy(t):
        return t.detach().cpu().contiguous().numpy()

    sel_np = npy(sel).astype(np.int64)
    gp, ga = orc.gather_rows_blocks(npy(layer.gate_packed), npy(layer.gate_absmax), sel_np, H, qbs)
    upk, ua = orc.gather_rows_blocks(npy(layer.up_packed), npy(layer.up_absmax), sel_np, H, qbs)
    t = layer.table
    dp = npy(t.down_packed)[sel_np].transpose(1, 0, 2).copy()  # block-major -> the reference's [H, k, 16]
    if layer.nested is not None:
        # the reference computes with the resolved fp32 absmax (RT:4621-4625)
        da_full = npy(layer.nested["down"].resolve()).reshape(H, I // qbs)
        da = da_full[:, (sel_np * 32) // qbs].copy()
    else:
        da = npy(t.down_absmax)[sel_np].T.copy()
    x16, ew, eb, sw, sb = (u16(v) for v in (layer.x, layer.enc_w, layer.enc_b, layer.score_w, layer.score_b))
    al = np.arange(k, dtype=np.int32).reshape(1, k)
    abytes = algorithmic_bytes(H, I, k, qbs, absmax)

    def port():
        orc.route(x16, ew, eb, sw, sb, k)
        orc.sparse_mlp(x16.reshape(1, H), al, gp, ga, upk, ua, dp, da, qbs=qbs, want_exact=False, want_fallback=True)

    port_us, port_n = _median_us(port, runs)
    # the torch-CPU restatement of the reference path, fp16 as the runtime computes
    g = tuple(torch.from_numpy(np.ascontiguousarray(a)) for a in (gp, ga, upk, ua, dp, da))
    tx, tew, teb, tsw, tsb = (v.detach().cpu() for v in (layer.x, layer.enc_w, layer.enc_b, layer.score_w,
                                                         layer.score_b))
    code = torch.from_numpy(orc.nf4_code().astype(np.float32))
    ordered = None

    def torch_path():
        nonlocal ordered
        _, ordered = tref.decode_layer(tx, tew, teb, tsw, tsb, k, g, code, qbs, dtype=torch.float16)

    us, n = _median_us(torch_path, runs)
    torch.set_num_threads(torch_threads)
    same = ordered is not None and np.array_equal(ordered.numpy(), sel_np)
    return {
        "value": round(1e6 / (MODEL_LAYERS * us), 6),
        "unit": "tok/s",
        "us_per_layer": round(us, 1),
        "gbs": round(abytes / (us * 1e-6) / 1e9, 3),
        "cores": threads,
        "kind": "port",
        "cpu": cpu_model(),
        "host": host_description(),
        "sample": f"1 layer through the torch-CPU restatement of the reference's PyTorch path in fp16 (router "
                  f"F.linear + topk, active layout, bitsandbytes-style dequant fallback MLP over {k} pre-gathered "
                  f"blocks), median of {n} runs after 3 warm-ups, {threads} torch threads (the host's CPU share); "
                  f"its selection {'equals' if same else 'differs from'} the GPU's",
        "c_port": {
            "value": round(1e6 / (MODEL_LAYERS * port_us), 6),
            "unit": "tok/s",
            "us_per_layer": round(port_us, 1),
            "gbs": round(abytes / (port_us * 1e-6) / 1e9, 3),
            "cores": threads,
            "sample": f"the oracle's C port of the same path (exact router, fp16 rounding points, fp64 sums), "
                      f"median of {port_n} runs after 3 warm-ups, {threads} OpenMP threads",
        },
    }


def copy_calibration(nbytes: int) -> int:
    import torch

    dev = torch.device("cuda", 0)
    a = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    a.fill_(1)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": nbytes, "read_bytes": nbytes, "write_bytes": nbytes}), flush=True)
    return 0


def timed_loop_us(launch, steps: int) -> float:
    """Mean µs per step of `launch(i)` for i < steps: one pair of HIP events
    on the current stream (the stream the C ABI is given) brackets the whole
    loop, so no event marker sits between two steps' kernels."""
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(steps):
        launch(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / steps


def base_result(args, value: float, us_per_layer: float, H: int, I: int, R: int, k: int, qbs: int) -> dict:
    return {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_per_layer / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "nf4(u8)*f16->f32",
        "data": "synthetic",
        "config": {
            "workload": WORKLOADS[args.config] + f"; NF4 qbs {qbs} with "
                        + ("double-quantised absmax (u8, fp32 per 256, offset)" if args.absmax == "dq8"
                           else "fp32 absmax"),
            "hidden": H, "intermediate": I, "basis_rank": R, "top_k": k, "block": 32, "quant_block": qbs,
            "absmax": args.absmax,
        },
    }


def run_partial(args) -> int:
    """Config 3: half of the blocks resident, 62 of the 208 selected blocks
    not in HBM slots.  The layer has a hot-block cache: each token routes,
    promotes its misses into slots (the fixed-capacity plan, the blocks
    copied once from pinned host memory) and decodes every block from HBM.
    The cache state is restored before every step, so every step promotes the
    same 62 misses.  Also reported: the decode reading the misses zero-copy
    from the host copies with no promotion."""
    import numpy as np
    import torch

    from next_step_ai_amd._runtime import workspace
    from next_step_ai_amd.router import route_tokens
    from next_step_ai_amd.slot_table import HotBlockCache, SparseMlpLayer
    from next_step_ai_amd.synth import make_synthetic_layer

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    H, I, R, k = CONFIGS[3]
    qbs, NB = 64, I // 32
    n_layers = min(args.layers, 4)  # each keeps a pinned host copy of all its blocks
    layers = []
    for l in range(n_layers):
        L = make_synthetic_layer(H=H, I=I, R=R, seed=3000 + l, device=device, double_quant=args.absmax == "dq8",
                                 keep_f32_absmax=args.absmax == "f32")
        sel = route_tokens(L.x.reshape(1, H), L.routing_dict(k), k, sorted_by_score=False).reshape(-1)
        sel_np = sel.cpu().numpy().astype(np.int64)
        rng = np.random.default_rng(3000 + l)
        hit = sel_np[rng.permutation(k)[: k - C3_MISSES]]
        others = np.setdiff1d(np.arange(NB), sel_np)
        resident = np.concatenate([hit, rng.choice(others, size=C3_RESIDENT - hit.size, replace=False)])
        L.table = L.slot_table(resident_blocks=torch.from_numpy(resident), host_copy=True, drop_reference_down=True)
        L.mlp = SparseMlpLayer(L.router(), L.table, k)
        misses = int((L.table.lookup_cpu()[torch.from_numpy(sel_np)] < 0).sum())
        assert misses == C3_MISSES, misses
        # the slots of the token's hits score above the others (calibrated hot
        # blocks): the plan evicts non-selected blocks
        scores = torch.zeros(C3_RESIDENT)
        scores[: hit.size] = 1.0
        L.cache = HotBlockCache(L.table, scores=scores)
        L.cached = SparseMlpLayer(L.router(), L.table, k, cache=L.cache)
        c = L.cache
        L.saved = (L.table.lookup.clone(), c.slot_block.clone(), c.slot_score.clone(), c.active.clone())
        layers.append(L)
        print(f"[bench] config 3 layer {l}: {misses} of {k} selected blocks on the host", file=sys.stderr, flush=True)

    def restore(L):
        lk, sb, ss, ac = L.saved
        L.table.lookup.copy_(lk)
        L.cache.slot_block.copy_(sb)
        L.cache.slot_score.copy_(ss)
        L.cache.active.copy_(ac)

    outs = [torch.empty(H, dtype=torch.float16, device=device) for _ in layers]
    sels = [torch.empty(k, dtype=torch.int32, device=device) for _ in layers]
    ws = workspace(layers[0].mlp.workspace_bytes(), device)
    n = len(layers)
    # zero-copy decode: misses read from the pinned host copies, no promotion
    for i in range(args.warmup):
        layers[i % n].mlp.forward(layers[i % n].x, out=outs[i % n], sel_out=sels[i % n], ws=ws)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        layers[i % n].mlp.forward(layers[i % n].x, out=outs[i % n], sel_out=sels[i % n], ws=ws)
    torch.cuda.synchronize()
    zc_us = (time.perf_counter() - t0) / args.steps * 1e6
    y_zc = [o.clone() for o in outs]
    # promote-first decode, HIP events around each step (the restore of the
    # cache state between steps stays outside them; the blocks whose slots a
    # promotion took are not selected by the layer's token, so the restored
    # lookup still serves every selected block its own bytes)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for i in range(args.warmup):
        L = layers[i % n]
        restore(L)
        L.cached.forward(L.x, out=outs[i % n], sel_out=sels[i % n], ws=ws)
    torch.cuda.synchronize()
    for i in range(args.steps):
        L = layers[i % n]
        restore(L)
        evs[i][0].record()
        L.cached.forward(L.x, out=outs[i % n], sel_out=sels[i % n], ws=ws)
        evs[i][1].record()
    torch.cuda.synchronize()
    per = [a.elapsed_time(b) * 1e3 for a, b in evs]
    us = statistics.mean(per)
    for j in range(n):
        assert torch.equal(outs[j], y_zc[j]), "promote-first output differs from the zero-copy decode"
    per_block = algorithmic_bytes(H, I, 1, qbs, args.absmax) - algorithmic_bytes(H, I, 0, qbs, args.absmax)
    miss_bytes = C3_MISSES * per_block
    hit_bytes = algorithmic_bytes(H, I, k, qbs, args.absmax) - miss_bytes
    res = base_result(args, 1e6 / (MODEL_LAYERS * us), us, H, I, R, k, qbs)
    res["config"].update({"resident_blocks": C3_RESIDENT, "host_misses": C3_MISSES, "rotating_layers": n})
    res.update({
        "us_per_layer": round(us, 3),
        "us_per_layer_median": round(statistics.median(per), 3),
        "hbm_hit_bytes_per_layer": hit_bytes,
        "host_miss_bytes_per_layer": miss_bytes,
        # the misses cross the host link once, into their slots: their bytes
        # over the whole layer time is a lower bound of the link rate reached
        "host_link_gbs_lower_bound": round(miss_bytes / (us * 1e-6) / 1e9, 2),
        "zero_copy_us_per_layer": round(zc_us, 3),
        "zero_copy_host_link_gbs_lower_bound": round(miss_bytes / (zc_us * 1e-6) / 1e9, 2),
        "note": "a step = route + promotion of the 62 misses into slots (plan + copies from pinned host memory) + "
                "decode of all 208 blocks from HBM; host-link bound, so the HBM roofline does not apply to this "
                "config; zero_copy_* = the decode reading the misses from the host copies with no promotion "
                "(outputs bit-identical)",
    })
    print(json.dumps(res), flush=True)
    return 0


def run_prefill(args) -> int:
    """Config 4: 256-token chunked prefill through one layer: per-token routing
    plus the grouped MFMA MLP over the union of the selected blocks."""
    import torch

    from next_step_ai_amd.synth import make_synthetic_layer, sub_seed, synth_normal_f16

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    H, I, R, k = CONFIGS[4]
    qbs, NB, M = 64, I // 32, PREFILL_TOKENS
    n_layers = min(args.layers, 3)
    layers = []
    for l in range(n_layers):
        L = make_synthetic_layer(H=H, I=I, R=R, seed=4000 + l, device=device, double_quant=args.absmax == "dq8",
                                 keep_f32_absmax=args.absmax == "f32")
        L.table = L.slot_table(drop_reference_down=True)
        L.xs = synth_normal_f16(sub_seed(4000 + l, "x"), (M, H), 1.0, device)
        L.sel = L.router().route(L.xs, k)
        layers.append(L)
    routers = [L.router() for L in layers]
    outs = [torch.empty((M, H), dtype=torch.float16, device=device) for _ in layers]
    n = len(layers)
    steps = max(1, args.steps // 10)  # a prefill step is ~100x a decode step
    for i in range(max(1, args.warmup // 10)):
        L = layers[i % n]
        L.table.prefill(L.xs, routers[i % n].route(L.xs, k), out=outs[i % n])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        L = layers[i % n]
        L.table.prefill(L.xs, routers[i % n].route(L.xs, k), out=outs[i % n])
    torch.cuda.synchronize()
    step_us = (time.perf_counter() - t0) / steps * 1e6
    def mlp(i: int) -> None:
        L = layers[i % n]
        L.table.prefill(L.xs, L.sel, out=outs[i % n])

    mlp_us = timed_loop_us(mlp, steps)
    union = [int(torch.unique(L.sel).numel()) for L in layers]
    per_block = algorithmic_bytes(H, I, 1, qbs, args.absmax) - algorithmic_bytes(H, I, 0, qbs, args.absmax)
    ubytes = int(statistics.mean(union)) * per_block + 2 * 2 * M * H
    useful_flop = 2.0 * 3 * M * k * 32 * H
    res = base_result(args, M / (step_us * 1e-6), step_us, H, I, R, k, qbs)
    res["unit"] = "tok/s"
    res["steps"] = steps
    res["config"].update({"tokens": M, "union_blocks": union, "rotating_layers": n})
    res.update({
        "prefill_us_per_layer": round(step_us, 3),
        "prefill_mlp_us": round(mlp_us, 3),
        "route_us": round(max(0.0, step_us - mlp_us), 3),
        "prefill_tok_s_per_layer": round(M / (step_us * 1e-6), 1),
        "union_bytes": ubytes,
        "roofline": {"bound": "hbm", "achieved": round(ubytes / (mlp_us * 1e-6) / 1e9, 2), "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": round(ubytes / (mlp_us * 1e-6) / 1e9 / PEAK_GBS, 4), "traffic": None,
                     "kernels": "k_pf_mark + k_pf_scan + k_pf_list + k_pf_gu + k_dg_down + k_dg_fin (k_pf_down for small unions)"},
        "mfma": {"useful_tflops": round(useful_flop / (mlp_us * 1e-6) / 1e12, 2), "peak_tflops": PEAK_F16_TFLOPS,
                 "frac": round(useful_flop / (mlp_us * 1e-6) / 1e12 / PEAK_F16_TFLOPS, 4),
                 "useful_flop": useful_flop},
    })
    print(json.dumps(res), flush=True)
    return 0


def run_dense_guard(args) -> int:
    """Config 7: the dense-guard prefill MLP (every block for every token)."""
    import torch

    from next_step_ai_amd.synth import make_synthetic_layer, sub_seed, synth_normal_f16

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    H, I, R, _ = CONFIGS[7]
    qbs, M = 64, args.tokens
    n_layers = min(args.layers, 2)
    layers = []
    for l in range(n_layers):
        L = make_synthetic_layer(H=H, I=I, R=R, seed=7000 + l, device=device, double_quant=args.absmax == "dq8",
                                 keep_f32_absmax=args.absmax == "f32")
        L.table = L.slot_table(drop_reference_down=True)
        L.xs = synth_normal_f16(sub_seed(7000 + l, "x"), (M, H), 1.0, device)
        layers.append(L)
    outs = [torch.empty((M, H), dtype=torch.float16, device=device) for _ in layers]
    n = len(layers)
    steps = max(1, args.steps // 20)
    for i in range(max(1, args.warmup // 10)):
        layers[i % n].table.dense_mlp(layers[i % n].xs, out=outs[i % n])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    us = timed_loop_us(lambda i: layers[i % n].table.dense_mlp(layers[i % n].xs, out=outs[i % n]), steps)
    step_us = (time.perf_counter() - t0) / steps * 1e6
    flop = 2.0 * 3 * M * I * H
    res = base_result(args, M / (step_us * 1e-6), step_us, H, I, R, I // 32, qbs)
    res["metric"] = f"dense-guard prefill MLP tok/s per layer + MFMA TFLOP/s vs peak, 405B shape, {M} tokens"
    res["steps"] = steps
    res["config"].update({"tokens": M, "rotating_layers": n})
    res.update({
        "dense_mlp_us": round(us, 3),
        "roofline": {"bound": "mfma", "achieved": round(flop / (us * 1e-6) / 1e12, 2), "peak": PEAK_F16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(flop / (us * 1e-6) / 1e12 / PEAK_F16_TFLOPS, 4),
                     "traffic": None, "flop": flop, "kernels": "k_dg_gu2 + k_dg_gu_fix + k_dg_down + k_dg_fin"},
    })
    print(json.dumps(res), flush=True)
    return 0


def run_stack(args) -> int:
    """Config 5: 126 resident layers, 64 decode tokens through all of them."""
    import torch

    from next_step_ai_amd._runtime import workspace
    from next_step_ai_amd.slot_table import SparseMlpLayer
    from next_step_ai_amd.synth import make_synthetic_layer, sub_seed, synth_normal_f16

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    H, I, R, k = CONFIGS[5]
    qbs = 64
    t_gen = time.perf_counter()
    mlps = []
    for l in range(STACK_LAYERS):
        L = make_synthetic_layer(H=H, I=I, R=R, seed=5000 + l, device=device, double_quant=args.absmax == "dq8",
                                 keep_f32_absmax=args.absmax == "f32", gate_up_std=STACK_GATE_UP_STD)
        table = L.slot_table(drop_reference_down=True)
        mlps.append(SparseMlpLayer(L.router(), table, k))
        del L
        if (l + 1) % 16 == 0 or l + 1 == STACK_LAYERS:
            torch.cuda.synchronize()
            print(f"[bench] config 5: {l + 1}/{STACK_LAYERS} layers generated "
                  f"({torch.cuda.memory_allocated(device) / 2**30:.1f} GiB), {time.perf_counter() - t_gen:.0f}s",
                  file=sys.stderr, flush=True)
    tokens = [synth_normal_f16(sub_seed(5000 + t, "x"), (H,), 1.0, device) for t in range(STACK_TOKENS + args.warmup)]
    ws = workspace(mlps[0].workspace_bytes(), device)
    out = torch.empty(H, dtype=torch.float16, device=device)
    sel = torch.empty(k, dtype=torch.int32, device=device)
    xa = torch.empty(H, dtype=torch.float16, device=device)
    xb = torch.empty(H, dtype=torch.float16, device=device)

    def token(x0):
        xa.copy_(x0)
        x, y = xa, xb
        for m in mlps:
            if args.unfused_residual:
                m.forward(x, out=out, sel_out=sel, ws=ws)
                torch.add(x, out, out=y)  # the residual add of the decode loop
            else:  # the same add fused into the down kernel's output
                m.forward(x, out=y, sel_out=sel, ws=ws, residual=x)
            x, y = y, x
        return x

    if args.graph:  # the whole token as one captured graph
        from next_step_ai_amd.decode_graph import StackGraph

        g = StackGraph(mlps)
        token = g.run  # noqa: F811
    for t in range(args.warmup):
        token(tokens[STACK_TOKENS + t])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(STACK_TOKENS):
        last = token(tokens[t])
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    finite = bool(torch.isfinite(last.float()).all())
    tok_s = STACK_TOKENS / dt
    us_layer = dt / (STACK_TOKENS * STACK_LAYERS) * 1e6
    layer_bytes = algorithmic_bytes(H, I, k, qbs, args.absmax) + router_bytes(H, R, I // 32)
    res = base_result(args, tok_s, us_layer, H, I, R, k, qbs)
    res["steps"] = STACK_TOKENS
    res["config"].update({"layers": STACK_LAYERS, "tokens": STACK_TOKENS, "graph": bool(args.graph),
                          "residual": "separate add" if args.unfused_residual and not args.graph else "fused",
                          "resident_bytes": int(torch.cuda.memory_allocated(device))})
    res.update({
        "us_per_layer": round(us_layer, 3),
        "decode_tok_s_126_layers": round(tok_s, 3),
        "aggregate_hbm_gbs": round(layer_bytes * STACK_TOKENS * STACK_LAYERS / dt / 1e9, 2),
        "algorithmic_bytes_per_layer": layer_bytes,
        "generation_s": round(time.perf_counter() - t_gen - dt, 1),
        "final_hidden_finite": finite,
        "gate_up_std": STACK_GATE_UP_STD,
    })
    print(json.dumps(res), flush=True)
    return 0


def lm_head_bytes(V: int, H: int, qbs: int, absmax: str, dq_block: int = 256) -> int:
    """Bytes one LM-head pass must move: packed NF4 (V H / 2), absmax (fp32,
    or u8 codes plus one fp32 scale per dq_block codes and the 256-entry
    second-level table), x (fp16) and the fp16 logits."""
    n_abs = V * H // qbs
    ab = 4 * n_abs if absmax == "f32" else n_abs + 4 * ((n_abs + dq_block - 1) // dq_block) + 4 * 256
    return V * H // 2 + ab + 2 * H + 2 * V + 4 * 16


def run_lm_head(args) -> int:
    """Config 6: the 405B NF4 LM head for one decode token."""
    import numpy as np
    import torch

    from next_step_ai_amd.lm_head import dense_linear_nf4
    from next_step_ai_amd.nested_absmax import NestedAbsmax
    from next_step_ai_amd._runtime import nf4_code
    from next_step_ai_amd.synth import synth_nf4, synth_normal_f16

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    V, H, qbs = LM_VOCAB, 16384, 64
    packed, absmax = synth_nf4(6001, V * H, qbs, 0.02, device)
    if args.absmax == "dq8":
        absmax = NestedAbsmax.quantize(absmax)
    code = nf4_code(device)
    xs = [synth_normal_f16(6100 + t, (1, H), 1.0, device) for t in range(4)]
    for i in range(args.warmup):
        dense_linear_nf4(xs[i % 4], packed, absmax, code, V, H, qbs)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    us = timed_loop_us(lambda i: dense_linear_nf4(xs[i % 4], packed, absmax, code, V, H, qbs), args.steps)
    wall_us = (time.perf_counter() - t0) / args.steps * 1e6
    nbytes = lm_head_bytes(V, H, qbs, args.absmax)
    gbs = nbytes / (us * 1e-6) / 1e9
    res = base_result(args, 1e6 / wall_us, wall_us, H, 0, 0, 0, qbs)
    res["metric"] = "NF4 LM head µs/token + HBM GB/s vs peak, vocabulary 128256 x hidden 16384"
    res["config"] = {"workload": WORKLOADS[6] + f"; NF4 qbs {qbs} with "
                     + ("double-quantised absmax (u8, fp32 per 256, offset)" if args.absmax == "dq8"
                        else "fp32 absmax"),
                     "vocab": V, "hidden": H, "quant_block": qbs, "absmax": args.absmax, "rows": 1}
    res.update({
        "lm_head_us": round(us, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_GBS, 4), "traffic": None, "algorithmic_bytes": nbytes,
                     "kernel": "k_rows_rep"},
    })
    if not args.no_cpu_baseline:
        from oracle import oracle as orc

        sample = 2048
        pk = packed.view(V, H // 2)[:sample].cpu().numpy()
        am = (absmax.resolve() if isinstance(absmax, NestedAbsmax) else absmax).view(V, H // qbs)[:sample].cpu().numpy()
        xh = xs[0].cpu().view(torch.int16).numpy().view(np.uint16)
        orc.set_num_threads(host_threads())
        for _ in range(3):  # warm-ups
            orc.dense_linear_nf4(xh, pk, am, sample, H, qbs)
        times = []
        for _ in range(max(10, args.cpu_runs)):
            c0 = time.perf_counter()
            orc.dense_linear_nf4(xh, pk, am, sample, H, qbs)
            times.append(time.perf_counter() - c0)
        full_s = statistics.median(times) * V / sample
        res["cpu_baseline"] = {"value": round(1.0 / full_s, 4), "unit": "tok/s", "cores": host_threads(),
                               "kind": "port", "host": host_description(),
                               "sample": f"oracle NF4 dequant + fp64 GEMV over the first {sample} of {V} vocabulary "
                                         f"rows, median of {len(times)} runs after 3 warm-ups, scaled by "
                                         f"{V}/{sample}; {cpu_model()}",
                               "us_per_token": round(full_s * 1e6, 1)}
    print(json.dumps(res), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    ap.add_argument("--layers", type=int, default=8, help="distinct layers rotated over the steps")
    ap.add_argument("--cpu-runs", type=int, default=10, help="timed CPU-baseline runs (at least 10)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES")
    ap.add_argument("--unfused-residual", action="store_true",
                    help="config 5: the residual add as its own launch instead of in the down kernel")
    ap.add_argument("--graph", action="store_true",
                    help="config 5: replay each token as one captured graph instead of eager launches")
    ap.add_argument("--tokens", type=int, default=PREFILL_TOKENS,
                    help="prompt tokens of --config 7 (the dense guard; 256 by default)")
    ap.add_argument("--absmax", choices=("dq8", "f32"), default="dq8",
                    help="absmax storage: double-quantised u8 (default) or resolved fp32")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only; --gpus {args.gpus} is not supported: this decode path has no "
              "multi-GPU mode (one GPU holds a whole layer's slot table)", file=sys.stderr)
        return 2
    if args.copy_calibration > 0:
        return copy_calibration(args.copy_calibration)
    if args.config == 3:
        return run_partial(args)
    if args.config == 4:
        return run_prefill(args)
    if args.config == 5:
        return run_stack(args)
    if args.config == 6:
        return run_lm_head(args)
    if args.config == 7:
        return run_dense_guard(args)

    import torch

    from next_step_ai_amd._runtime import workspace
    from next_step_ai_amd.slot_table import SparseMlpLayer
    from next_step_ai_amd.synth import make_synthetic_layer

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    H, I, R, k = CONFIGS[args.config]
    qbs = 64
    t_gen = time.perf_counter()
    layers = []
    for l in range(args.layers):
        L = make_synthetic_layer(H=H, I=I, R=R, seed=1000 * args.config + l, device=device,
                                 double_quant=args.absmax == "dq8")
        L.table = L.slot_table(drop_reference_down=True)
        L.mlp = SparseMlpLayer(L.router(), L.table, k)
        layers.append(L)
    torch.cuda.synchronize()
    t_gen = time.perf_counter() - t_gen
    print(f"[bench] generated {args.layers} layers H={H} I={I} k={k} in {t_gen:.1f}s", file=sys.stderr, flush=True)

    outs = [torch.empty(H, dtype=torch.float16, device=device) for _ in layers]
    sels = [torch.empty(k, dtype=torch.int32, device=device) for _ in layers]
    ws = workspace(layers[0].mlp.workspace_bytes(), device)
    n = len(layers)
    for i in range(args.warmup):
        j = i % n
        layers[j].mlp.forward(layers[j].x, out=outs[j], sel_out=sels[j], ws=ws)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        j = i % n
        layers[j].mlp.forward(layers[j].x, out=outs[j], sel_out=sels[j], ws=ws)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    us_per_layer = (t1 - t0) / args.steps * 1e6
    print(f"[bench] {args.steps} steps: {us_per_layer:.2f} us/layer (router + MLP)", file=sys.stderr, flush=True)

    # Sparse-MLP decode launch pair alone, HIP events on its launch stream
    # (torch's current stream, the one the C ABI is given) around all steps.
    for j in range(n):
        layers[j].table.decode(layers[j].x, sels[j], out=outs[j])

    def pair(i: int) -> None:
        j = i % n
        layers[j].table.decode(layers[j].x, sels[j], out=outs[j])

    mlp_us = timed_loop_us(pair, args.steps)
    route_us = max(0.0, us_per_layer - mlp_us)

    abytes = algorithmic_bytes(H, I, k, qbs, args.absmax)
    achieved = abytes / (mlp_us * 1e-6) / 1e9
    result = {
        "metric": METRIC,
        "value": round(1e6 / (MODEL_LAYERS * us_per_layer), 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_per_layer / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "nf4(u8)*f16->f32",
        "data": "synthetic",
        "config": {
            "workload": WORKLOADS[args.config] + f"; NF4 qbs {qbs} with "
                        + ("double-quantised absmax (u8, fp32 per 256, offset)" if args.absmax == "dq8"
                           else "fp32 absmax") + f"; all blocks HBM-resident; "
                        f"{args.layers} rotating seeded layers; batch 1 fp16 token",
            "hidden": H, "intermediate": I, "basis_rank": R, "top_k": k, "block": 32, "quant_block": qbs,
            "absmax": args.absmax, "rotating_layers": args.layers,
        },
        "us_per_layer": round(us_per_layer, 3),
        "sparse_mlp_us": round(mlp_us, 3),
        "router_us": round(route_us, 3),
        "decode_tok_s_126_layers": round(1e6 / (MODEL_LAYERS * us_per_layer), 3),
        "algorithmic_bytes_per_layer": abytes,
        "router_bytes_per_layer": router_bytes(H, R, I // 32),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_GBS, 4),
            "traffic": measured_traffic(args.config, args.absmax),
            "kernels": "k_gu_rep + k_down_rep (the sparse-MLP decode launch pair)",
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(layers[0], sels[0], args.cpu_runs, H, I, k, qbs, args.absmax)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
