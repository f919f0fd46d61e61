#!/usr/bin/env python3
# SPDX-License-Identifier: Apache-2.0
"""Fused EXL3 decode GEMV throughput on one MI355X (the headline metric, on the 27B-class layer shapes).

A step is one decode token's pass of the EXL3 GEMV hot path at batch 1 through the layers of a 27B-class
model at K = 6 (6.0 bpw, 3INST codebook): per layer the four launches the reference's fused decode path makes
(sibling groups, kernels.py:263-299, linear.py:124-193): q/k/v (5120 -> 6144 + 1024 + 1024, one launch),
o (6144 -> 5120), gate/up (5120 -> 17408 + 17408, one launch), down (17408 -> 5120), over `--layers`
distinct layers (default 64, the model's depth: 16.4 GB of trellis), so the weights stream from HBM, not
from the 256 MB Infinity Cache. One step is one replay of a HIP graph holding all of them; exactly --steps
steps are timed (20 steps ~ 0.1 s). Inputs (rotated activations, trellis, svh) are resident in HBM before
timing starts.

  value          whole-job GB/s: algorithmic bytes of all timed steps / wall time of the timed region
                 (graph replays, so host launch cost is excluded)
  roofline       the GEMV kernel: algorithmic bytes per launch / its average launch duration = GPU time
                 between HIP events recorded on the replay stream around the timed replays, divided by
                 their launches; against the 8 TB/s HBM3E peak; traffic = HBM bytes per launch from
                 rocprofv3 FETCH_SIZE / WRITE_SIZE (profiles/), or null. per_shape: each shape's launches of
                 all layers in one graph, replayed, events around the replays / launches (as the headline)
  cpu_baseline   the NumPy oracle (reconstruct + fp32 matmul + Hadamard + svh) on the q projection
  mixed_k        config 3: the 27B projections with K drawn per tensor from {2,3,4,5,6,8}, rows 1 / 2 / 4 / 8,
                 whole layers replayed from a HIP graph with siblings grouped as the loader groups them (one
                 q/k/v and one gate/up launch whatever their K); split_by_K: the same tensors grouped the
                 reference's way (equal K only), with the GB/s of each K's launches
  prefill        config 4: M = 4608 through gate / up / down at K = 6, TFLOP/s against the fp16 MFMA peak
  decode_tok_s   end-to-end batch-1 greedy decode of the synthetic 27B-shape EXL3 decoder (config 5: 64
                 layers, hidden 5120, MLP 17408, GQA 48/8 x 128, head 5120 -> 151936, K = 6): a 512-token
                 random-id prompt, then 256 tokens, each decode step replayed from one captured HIP graph

    python bench.py [--gpus 1] [--steps 60] [--warmup 5] [--mode exact|fast] [--decoder-layers 64]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
METRIC = "fused EXL3 GEMV GB/s (% HBM peak) at 6 bpw; 27B-shape decode tok/s"

# (name, k, member output features)
LAYER = [("qkv", 5120, [6144, 1024, 1024]), ("o", 6144, [5120]), ("gate_up", 5120, [17408, 17408]),
         ("down", 17408, [5120])]


def _import_package():
    import importlib.util
    name = "omlx_exl3_amd"
    if name in sys.modules:
        return sys.modules[name]
    pkg_dir = os.path.join(ROOT, "omlx-exl3_amd")
    spec = importlib.util.spec_from_file_location(name, os.path.join(pkg_dir, "__init__.py"),
                                                  submodule_search_locations=[pkg_dir])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def algorithmic_bytes(k: int, ns: list[int], K: int, rows: int) -> int:
    """trellis + svh + rotated inputs (one per member) + output, per launch."""
    n = sum(ns)
    return sum(K * k * m // 8 for m in ns) + 2 * n + 2 * rows * k * len(ns) + 2 * rows * n


def read_traffic(path: str):
    """HBM bytes per GEMV launch from a committed rocprofv3 summary (lines 'key: value')."""
    if not os.path.exists(path):
        return None
    vals = {}
    for line in open(path):
        if ":" in line and not line.lstrip().startswith("#"):
            key, v = line.split(":", 1)
            vals[key.strip()] = v.strip()
    try:
        return float(vals["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def _cpu_reconstruct_cols(args):
    """Worker of cpu_baseline: the oracle's reconstruction of one column range of the trellis."""
    tr_cols, k, ncols, K = args
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    from oracle import exl3_oracle as O
    return O.reconstruct_inner(tr_cols, k, ncols, K, 0)


def cpu_baseline(seconds_budget: float = 30.0) -> dict:
    """NumPy oracle on the q projection (5120 -> 6144, K = 6): bit-exact reconstruct (column ranges in
    parallel worker processes, one per visible core), rotation, fp32 matmul, output Hadamard * svh. Median
    of 7 runs after one warm-up: about 1 s of wall time, 15-20 s of CPU work on 16 cores."""
    import concurrent.futures
    import multiprocessing

    import numpy as np

    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    from oracle import exl3_oracle as O

    k, n, K = 5120, 6144, 6
    rng = np.random.default_rng(7)
    tr = O.random_trellis(k, n, K, 7)
    su = np.where(rng.integers(0, 2, k) == 1, 1.0, -1.0).astype(np.float16)
    sv = np.where(rng.integers(0, 2, n) == 1, 1.0, -1.0).astype(np.float16)
    x = rng.standard_normal((1, k)).astype(np.float16)
    cores = len(os.sched_getaffinity(0))
    nt = n // 16
    bounds = [nt * i // cores for i in range(cores + 1)]
    chunks = [(np.ascontiguousarray(tr[:, a:b]), k, 16 * (b - a), K) for a, b in zip(bounds, bounds[1:]) if b > a]
    # fresh worker interpreters (the parent has initialised the GPU; the workers never touch it)
    pool = concurrent.futures.ProcessPoolExecutor(max_workers=len(chunks),
                                                  mp_context=multiprocessing.get_context("spawn"))

    def run():
        t0 = time.perf_counter()
        w = np.concatenate(list(pool.map(_cpu_reconstruct_cols, chunks)), axis=1).view(np.float16).astype(np.float32)
        t1 = time.perf_counter()
        xh = O.rot(x, su.reshape(1, k))[0].astype(np.float32)
        y = O.fwht128_f32(xh @ w) * O.HAD_SCALE * sv.astype(np.float32)
        t2 = time.perf_counter()
        return t1 - t0, t2 - t1, y

    t_start = time.perf_counter()
    run()
    recs, mats = [], []
    for _ in range(7):
        a, b, _y = run()
        recs.append(a)
        mats.append(b)
        if time.perf_counter() - t_start > seconds_budget:
            break
    pool.shutdown()
    w_check = np.concatenate([_cpu_reconstruct_cols(c) for c in chunks[:1]], axis=1)
    if not np.array_equal(w_check, O.reconstruct_inner(tr[:, :bounds[1]], k, 16 * bounds[1], K, 0)):
        raise RuntimeError("cpu_baseline: parallel reconstruct differs")
    rec, mat = statistics.median(recs), statistics.median(mats)
    trellis_bytes = K * k * n // 8
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    gbs = trellis_bytes / (rec + mat) / 1e9
    return {
        "value": round(gbs, 5), "unit": "GB/s", "cores": cores, "kind": "port",
        "sample": (f"q projection 5120->6144 K=6 (23.6 MB trellis), median of {len(recs)} runs: NumPy oracle "
                   f"reconstruct {rec:.3f} s ({len(chunks)} worker processes, column ranges) + rotation/fp32 "
                   f"matmul/Hadamard {mat * 1e3:.1f} ms (BLAS on {cores} visible cores); {cpu_model}"),
        "decode_tok_s_extrapolated": round(gbs * 1e9 / DECODE_BYTES_PER_TOKEN, 5),
    }


MFMA_F16_PEAK_TFLOPS = 2500.0
# each prefill form runs untimed for at least this long first: two passes leave the clocks short of their
# sustained MFMA state, and the first form timed read ~8% slow behind them
PREFILL_WARM_S = 0.6
# the decode GEMV's untimed eager passes run at least this long before its first timing
GEMV_WARM_S = 0.6
# weight bytes read per decode token of the 64-layer 27B-shape decoder at K = 6 (layers' trellis + head)
DECODE_BYTES_PER_TOKEN = 64 * 255_590_400 + 583_434_240
# 27B projections as separate tensors (their K drawn per tensor in the mixed-bitrate configuration)
PROJ = [("q", 5120, 6144), ("k", 5120, 1024), ("v", 5120, 1024), ("o", 6144, 5120), ("gate", 5120, 17408),
        ("up", 5120, 17408), ("down", 17408, 5120)]


def mixed_k_benchmark(pk, torch, dev, rows_list=(1, 2, 4, 8), n_layers=8, reps=10) -> dict:
    """Config 3: the 27B projections with K drawn per tensor from {2, 3, 4, 5, 6, 8} (seeded), at batch rows 1,
    2, 4, 8. Siblings are grouped as the loader groups them: q/k/v and gate/up are one launch each whatever
    their K (the mixed-width GEMV). For comparison the same tensors are also run grouped the reference's way
    (only siblings of equal K share a launch, loader.py:137-156), with GB/s per K from that form. Layers
    rotate over a working set beyond the Infinity Cache; GB/s = algorithmic bytes (at the drawn K) / time. A
    form's launches are replayed from one HIP graph (back to back, no host dispatch between them); per K,
    that K's launches are replayed from a graph of their own."""
    import random
    rnd = random.Random(3)
    g = torch.Generator(device=dev).manual_seed(77)
    shape = {name: (k, n) for name, k, n in PROJ}
    sibsets = (("q", "k", "v"), ("gate", "up"), ("o",), ("down",))
    layers, draws = [], []
    for _ in range(n_layers):
        Ks = {name: rnd.choice([2, 3, 4, 5, 6, 8]) for name, _, _ in PROJ}
        draws.append(Ks)
        tens = {}
        for name, (k, n) in shape.items():
            tens[name] = (torch.randint(-32768, 32768, (k // 16, n // 16, 16 * Ks[name]), dtype=torch.int16,
                                        device=dev, generator=g),
                          torch.where(torch.rand(n, device=dev, generator=g) < 0.5, -1.0, 1.0).half())
        layers.append((Ks, tens))
    out = {"draws": draws, "per_rows": {}}
    bpw = sum(K * k * n for Ks in draws for (name, k, n) in PROJ for K in [Ks[name]]) / \
        sum(k * n for _ in draws for (_, k, n) in PROJ)
    out["mean_bpw"] = round(bpw, 3)

    def launches(rows, by_k):
        """(plan, xh, trellises, out) per launch of every layer; by_k: the reference's grouping."""
        items, nbytes = [], 0
        for Ks, tens in layers:
            for sib in sibsets:
                subsets = {}
                for name in sib:
                    subsets.setdefault(Ks[name] if by_k else 0, []).append(name)
                for names in subsets.values():
                    k = shape[names[0]][0]
                    ns = [shape[nm][1] for nm in names]
                    mKs = [Ks[nm] for nm in names]
                    svh = torch.cat([tens[nm][1] for nm in names])
                    plan = pk.kernels.TrellisGemvPlan(k, ns, mKs, 0, svh, rows, torch.float16)
                    xh = torch.randn((len(ns), rows, k), device=dev, generator=g).half()
                    o = torch.empty((rows, sum(ns)), dtype=torch.float16, device=dev)
                    items.append((plan, xh, [tens[nm][0] for nm in names], o))
                    nbytes += sum(algorithmic_bytes(k, [n], K, rows) for n, K in zip(ns, mKs))
        return items, nbytes

    cap = torch.cuda.Stream(device=dev)

    def graph_of(sel):
        """The selected launches captured in one HIP graph (an eager pass on the capture stream first)."""
        cap.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(cap):
            for plan, xh, trs, o in sel:
                plan(xh, trs, out=o)
        torch.cuda.current_stream(dev).wait_stream(cap)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for plan, xh, trs, o in sel:
                plan(xh, trs, out=o)
        return gr

    def time_graph(gr):
        """ms per replay: HIP events on the replay stream around `reps` back-to-back replays."""
        for _ in range(2):
            gr.replay()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            gr.replay()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / reps

    def whole(items, nbytes):
        graph = graph_of(items)
        ms = statistics.median(time_graph(graph) for _ in range(3))
        del graph
        return {"launches_per_layer": round(len(items) / n_layers, 2), "us_per_layer": round(ms * 1e3 / n_layers, 1),
                "GB_s": round(nbytes / ms / 1e6, 1), "pct_hbm_peak": round(100 * nbytes / ms / 1e6 / HBM_PEAK_GBS, 1)}

    # warm-up: the first form's graph replayed ~100 times before any timing (the clocks settle under load;
    # without it the first form measured, rows 1, read up to 10% slow)
    items, _nb = launches(rows_list[0], by_k=False)
    gr = graph_of(items)
    for _ in range(100):
        gr.replay()
    torch.cuda.synchronize()
    del gr, items
    for rows in rows_list:
        items, nbytes = launches(rows, by_k=False)
        res = whole(items, nbytes)
        del items
        # the reference's grouping of the same tensors, and per K from it
        items, nbytes = launches(rows, by_k=True)
        split = whole(items, nbytes)
        per_k = {}
        for K in sorted({plan.K for plan, _x, _t, _o in items}):
            sel = [it for it in items if it[0].K == K]
            gr = graph_of(sel)
            ms_k = statistics.median(time_graph(gr) for _ in range(3))
            del gr
            nb = sum(algorithmic_bytes(p.k, p.ns, p.K, rows) for p, _x, _t, _o in sel)
            per_k[str(K)] = {"launches": len(sel), "GB_s": round(nb / ms_k / 1e6, 1),
                             "pct_hbm_peak": round(100 * nb / ms_k / 1e6 / HBM_PEAK_GBS, 1)}
        del items
        split["per_K"] = per_k
        res["split_by_K"] = split
        out["per_rows"][str(rows)] = res
    return out


# PyTorch TunableOp's table of the fastest hipBLASLt / rocBLAS solution of each 27B projection GEMM at 16..4608
# rows on MI355X (hipBLASLt's default heuristic does not pick it for these shapes); read by the platform-BLAS
# comparison leg of the prefill measurement only.
GEMM_TABLE = os.path.join(ROOT, "bench_gemm_table_mi355x.csv")


def blas_prefill(pk, torch, xh, tr, k, n, K, cb, svh, out, table_ok):
    """The reference's prefill structure on the platform BLAS, for comparison only (linear.py:97-105):
    reconstruct W_inner^T (exl3_reconstruct), an fp16 GEMM with fp32 accumulation by hipBLASLt through
    torch.matmul (TunableOp on with tuning off around the call, so a shape GEMM_TABLE lists runs its recorded
    solution), then the output rotation (exl3_prefill_out_rotate)."""
    wt = pk.kernels.decode_wt(tr, k, n, K, cb)
    if table_ok:
        tun = torch.cuda.tunable
        was_on, was_tuning = tun.is_enabled(), tun.tuning_is_enabled()
        tun.tuning_enable(False)
        tun.enable(True)
        try:
            g = torch.matmul(xh, wt.t())
        finally:
            tun.enable(was_on)
            tun.tuning_enable(was_tuning)
    else:
        g = torch.matmul(xh, wt.t())
    return pk.kernels.prefill_out_rotate(g, svh, None, out)


def prefill_benchmark(pk, torch, dev, rows=4608, reps=6) -> dict:
    """Config 4: M = 4608 rotated fp16 activations through gate / up (5120 -> 17408) and down (17408 -> 5120)
    at K = 6. Forms timed: "matmul" (W_inner^T reconstructed, then the hand-written MFMA GEMM with the output
    rotation in its epilogue: prefill_gemm's default), "fused" (trellis tiles reconstructed in LDS, MFMA, Hadamard
    epilogue, one launch), and for comparison "blas" (reconstruct, hipBLASLt fp16 GEMM with the tabled solution,
    output rotation: the reference's structure on the platform BLAS). Every form first runs over the three
    projections untimed, at least twice and for at least PREFILL_WARM_S seconds (warm clocks, allocator, plans);
    a form's figure is then the GPU time of `reps` back-to-back passes over gate, up and down (HIP events, the
    region starting behind one more untimed pass so the GPU is busy when it opens); per projection the same with
    that projection alone. TFLOP/s = 2 M k n / time, against the 2.5 PFLOP/s dense fp16 MFMA peak."""
    g = torch.Generator(device=dev).manual_seed(5)
    table_ok = False
    if os.path.exists(GEMM_TABLE):
        try:
            table_ok = bool(torch.cuda.tunable.read_file(GEMM_TABLE))   # False if its version lines differ
        except RuntimeError:
            table_ok = False
    paths = ("matmul", "fused", "blas")
    shapes = (("gate", 5120, 17408), ("up", 5120, 17408), ("down", 17408, 5120))
    data = {}
    for name, k, n in shapes:
        tr = torch.randint(-32768, 32768, (k // 16, n // 16, 96), dtype=torch.int16, device=dev, generator=g)
        svh = torch.where(torch.rand(n, device=dev, generator=g) < 0.5, -1.0, 1.0).half()
        xh = torch.randn((rows, k), device=dev, generator=g).half()
        out = torch.empty((rows, n), dtype=torch.float16, device=dev)
        data[name] = (k, n, tr, svh, xh, out)

    def call(name, path):
        k, n, tr, svh, xh, out = data[name]
        if path == "blas":
            blas_prefill(pk, torch, xh, tr, k, n, 6, 0, svh, out, table_ok)
        else:
            pk.kernels.prefill_gemm(xh, tr, k, n, 6, 0, svh, out=out, path=path)

    def timed(names, path):
        for nm in names:   # left running while the timed calls are queued
            call(nm, path)
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            for nm in names:
                call(nm, path)
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / reps

    flop = {name: 2.0 * rows * k * n for name, k, n in shapes}
    names = [sh[0] for sh in shapes]
    per, tot = {}, {}
    for path in paths:
        warm_until = time.perf_counter() + PREFILL_WARM_S
        passes = 0
        while passes < 2 or time.perf_counter() < warm_until:
            for nm in names:
                call(nm, path)
            torch.cuda.synchronize()
            passes += 1
        ms_all = timed(names, path)
        tot[path] = (sum(flop.values()), ms_all)
        per[path] = {}
        for nm in names:
            ms = timed([nm], path)
            per[path][nm] = {"ms": round(ms, 3), "TFLOP_s": round(flop[nm] / ms / 1e9, 1)}
    del data
    auto = "matmul"   # prefill_gemm's "auto" path for these shapes (k a multiple of 64)
    tf = {p: tot[p][0] / tot[p][1] / 1e9 for p in tot}
    return {"rows": rows, "path": auto, "per_proj": per[auto], "TFLOP_s": round(tf[auto], 1),
            "peak_TFLOP_s": MFMA_F16_PEAK_TFLOPS, "mfma_frac": round(tf[auto] / MFMA_F16_PEAK_TFLOPS, 4),
            "ms_total": round(tot[auto][1], 2), "blas_gemm_table": table_ok,
            "by_path": {p: {"TFLOP_s": round(tf[p], 1), "ms_total": round(tot[p][1], 2), "per_proj": per[p]}
                        for p in per}}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def decode_benchmark(pk, torch, dev, n_layers: int, prompt: int, gen: int) -> dict:
    """Config 5: build the synthetic decoder, prefill a random-id prompt, then time `gen` greedy decode
    steps replayed from one captured HIP graph (inputs, weights and KV cache resident in HBM)."""
    from omlx_exl3_amd.synthetic import DecoderConfig, SyntheticDecoder, greedy_step

    cfg = DecoderConfig(n_layers=n_layers, max_len=prompt + gen + 8)
    t0 = time.perf_counter()
    model = SyntheticDecoder(cfg, seed=2024, device=dev)
    torch.cuda.synchronize()
    t_build = time.perf_counter() - t0
    log(f"decoder built ({n_layers} layers) in {t_build:.1f} s")
    g = torch.Generator(device=dev).manual_seed(99)
    ids = torch.randint(0, cfg.vocab, (prompt,), generator=g, device=dev)
    pos = torch.arange(prompt, device=dev)
    model(ids, pos)                                      # warm-up prefill (plans, kernels)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits = model(ids, pos)
    torch.cuda.synchronize()
    t_prefill = time.perf_counter() - t0
    log(f"prefill of {prompt} tokens: {t_prefill * 1e3:.1f} ms")
    tok = torch.zeros(1, dtype=torch.int64, device=dev)
    cur = torch.full((1,), prompt, dtype=torch.int64, device=dev)
    tok.copy_(greedy_step.argmax(logits).view(1))
    start_tok, start_pos = tok.clone(), cur.clone()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        greedy_step(model, tok, cur)                     # eager warm-up step (plans for 1 row, buffers)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        greedy_step(model, tok, cur)
    tok.copy_(start_tok)
    cur.copy_(start_pos)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(gen):
        graph.replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    log(f"{gen} decode steps: {wall * 1e3:.1f} ms")
    finite = bool(torch.isfinite(model.last_logits).all().item())
    tok_s = gen / wall
    L_avg = prompt + gen / 2
    kv_bytes = n_layers * 2 * cfg.n_kv_heads * cfg.head_dim * 2 * L_avg
    weights = n_layers * cfg.layer_trellis_bytes() + cfg.head_trellis_bytes()
    bpt = weights + kv_bytes
    return {"tok_s": round(tok_s, 2), "ms_per_token": round(wall / gen * 1e3, 3), "layers": n_layers,
            "prompt": prompt, "gen_tokens": gen, "bytes_per_token": int(bpt),
            "GB_s": round(bpt * tok_s / 1e9, 1), "pct_hbm_peak": round(100 * bpt * tok_s / 1e9 / HBM_PEAK_GBS, 1),
            "prefill_tok_s": round(prompt / t_prefill, 1), "build_s": round(t_build, 1),
            "logits_finite": finite, "fused": model.fused, "sibling_groups": model.groups,
            "decode_path": "fusion.fuse_decode: DecodeStep + HeadNorm, prologue form (five launches per layer)"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=60, help="timed steps (one step = one decode token's GEMVs)")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--mode", choices=["exact", "fast"], default="exact")
    ap.add_argument("--table", action="store_true",
                    help="the table GEMV kernel (LDS codebook lookup for half of each run) instead of hashing")
    ap.add_argument("--layers", type=int, default=64, help="distinct 27B-shape layers per step")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--traffic-file", default=os.path.join(ROOT, "profiles", "gemv_27b_k6_traffic.txt"))
    ap.add_argument("--copy-probe", action="store_true",
                    help="run only a 1 GiB device copy (calibrates rocprofv3 FETCH/WRITE counters)")
    ap.add_argument("--decoder-layers", type=int, default=64, help="layers of the end-to-end decoder (0 = skip)")
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--no-configs", action="store_true", help="skip the mixed-K (config 3) and prefill (config 4) lines")
    ap.add_argument("--only", choices=["prefill", "mixed", "decode"],
                    help="run one measurement alone and print its JSON (for profiling)")
    ap.add_argument("--gen", type=int, default=256)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (the EXL3 linear would shard "
              "column-parallel, row-parallel with an all-reduce over RCCL); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    dev = torch.device("cuda:0")
    if args.copy_probe:
        a = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        a.fill_(1)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(10):
            b.copy_(a)
        e.record()
        torch.cuda.synchronize()
        ms = s.elapsed_time(e) / 10
        print(json.dumps({"copy_bytes": 1 << 30, "copy_ms": ms, "copy_GBps_read_plus_write": 2 * (1 << 30) / ms / 1e6}))
        return 0

    pk = _import_package()
    if args.only:
        if args.only == "prefill":
            print(json.dumps(prefill_benchmark(pk, torch, dev)))
        elif args.only == "mixed":
            print(json.dumps(mixed_k_benchmark(pk, torch, dev)))
        else:
            print(json.dumps(decode_benchmark(pk, torch, dev, args.decoder_layers, args.prompt, args.gen)))
        return 0
    K, cb, rows = 6, 0, 1
    fast = args.mode == "fast"
    g = torch.Generator(device=dev).manual_seed(1234)
    layers = []
    for _ in range(args.layers):
        items = []
        for name, k, ns in LAYER:
            trs = [torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, device=dev, generator=g)
                   for n in ns]
            svh = torch.where(torch.rand(sum(ns), device=dev, generator=g) < 0.5, -1.0, 1.0).half()
            xh = torch.randn((len(ns), rows, k), device=dev, generator=g).half()
            plan = pk.kernels.TrellisGemvPlan(k, ns, K, cb, svh, rows, torch.float16, fast=fast,
                                              table=args.table)
            out = torch.empty((rows, sum(ns)), dtype=torch.float16, device=dev)
            items.append((name, plan, xh, trs, out, algorithmic_bytes(k, ns, K, rows)))
        layers.append(items)
    step_bytes = sum(it[5] for it in layers[0])
    L = args.layers

    def run_layer(items):
        for _name, plan, xh, trs, out, _b in items:
            plan(xh, trs, out=out)

    # eager passes (plans, kernels), at least one and for at least GEMV_WARM_S seconds: the clocks settle under
    # load before the first timing
    warm_until = time.perf_counter() + GEMV_WARM_S
    passes = 0
    while passes < 1 or time.perf_counter() < warm_until:
        for items in layers:
            run_layer(items)
        torch.cuda.synchronize()
        passes += 1

    # ---- per-shape launch durations: one shape's launches of all layers (different weights each) captured in
    # one graph and replayed; HIP events on the replay stream around the timed replays, divided by the launches
    # (the way the kernels run in a decode step: back to back, no host gaps) ----
    cap = torch.cuda.Stream(device=dev)
    per_shape = {}
    for si, (name, _k, _ns) in enumerate(LAYER):
        cap.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(cap):
            for items in layers:
                _n, plan, xh, trs, out, _b = items[si]
                plan(xh, trs, out=out)
        torch.cuda.current_stream(dev).wait_stream(cap)
        torch.cuda.synchronize()
        g_shape = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_shape):
            for items in layers:
                _n, plan, xh, trs, out, _b = items[si]
                plan(xh, trs, out=out)
        for _ in range(3):
            g_shape.replay()
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 10
        torch.cuda.synchronize()
        s_ev.record()
        for _ in range(reps):
            g_shape.replay()
        e_ev.record()
        torch.cuda.synchronize()
        us = s_ev.elapsed_time(e_ev) * 1e3 / (reps * L)
        nb = layers[0][si][5]
        per_shape[name] = {"bytes": nb, "us_per_launch": round(us, 2), "GB_s": round(nb / us / 1e3, 1),
                           "pct_hbm_peak": round(100 * nb / us / 1e3 / HBM_PEAK_GBS, 1)}
        del g_shape

    # ---- whole-job throughput: one step = all layers' launches captured in one graph, replayed ----
    graph = torch.cuda.CUDAGraph()
    cap.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(cap):
        for items in layers:           # one eager pass on the capture stream before capture
            run_layer(items)
    torch.cuda.current_stream(dev).wait_stream(cap)
    torch.cuda.synchronize()
    ref_out = [it[4].clone() for it in layers[-1]]
    with torch.cuda.graph(graph):
        for items in layers:
            run_layer(items)
    graph.replay()
    torch.cuda.synchronize()
    for it, r in zip(layers[-1], ref_out):
        if not torch.equal(it[4], r):
            print("graph replay differs from the eager result", file=sys.stderr)
            return 1
    for _ in range(args.warmup):
        graph.replay()
    # HIP events on the replay stream bracket the timed replays: the GPU time of the timed region divided
    # by its launches is the average launch duration (back-to-back launches, as rocprofv3 sees them)
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    steps = args.steps
    value = step_bytes * L * steps / wall / 1e9

    traffic = read_traffic(args.traffic_file)
    n_launch = steps * L * len(layers[0])
    per_launch_bytes = step_bytes / len(layers[0])
    avg_launch_ms = ev0.elapsed_time(ev1) / n_launch
    kernel_gbs = per_launch_bytes / avg_launch_ms / 1e6
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / steps * 1e3, 4),
        "timed_s": round(wall, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": ("27B-class decode GEMVs, batch 1, K=6 (6.0 bpw) 3INST; a step = one token through "
                                f"{L} distinct layers of fused GEMV launches qkv 5120->6144+1024+1024, o 6144->5120, "
                                "gate_up 5120->17408+17408, down 17408->5120 "
                                f"({step_bytes * L / 1e9:.2f} GB of weights per step)"),
                   "global_batch": rows, "bpw": K, "codebook": "3inst", "gemv_mode": args.mode,
                   "gemv_kernel": "table" if (args.table and not fast) else "hash",
                   "parallelism": "none (1 GPU)"},
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
        "roofline": {"bound": "hbm", "achieved": round(kernel_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "algorithmic_bytes_per_launch": round(per_launch_bytes),
                     "avg_launch_us": round(avg_launch_ms * 1e3, 3)},
        "per_shape": per_shape,
        "decode_tok_s": None,
    }
    log(f"GEMV: {value:.1f} GB/s whole job, kernel {kernel_gbs:.1f} GB/s")
    del layers, graph
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    if not args.no_configs:
        result["mixed_k"] = mixed_k_benchmark(pk, torch, dev)
        log(f"mixed K: {result['mixed_k']['per_rows']}")
        torch.cuda.empty_cache()
        result["prefill"] = prefill_benchmark(pk, torch, dev)
        log(f"prefill: {result['prefill']['TFLOP_s']} TFLOP/s")
        torch.cuda.empty_cache()
    if args.decoder_layers > 0:
        dec = decode_benchmark(pk, torch, dev, args.decoder_layers, args.prompt, args.gen)
        result["decode_tok_s"] = dec["tok_s"]
        result["decode"] = dec
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
        log("cpu baseline done")
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
