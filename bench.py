#!/usr/bin/env python3
"""Benchmark of the ragged paged-attention path on one MI355X.

Headline (BASELINE.json ``metric``): Llama-3-8B-shape ragged paged decode --
256 sequences, lognormal context lengths (median 1024, sigma 1, clipped to
[16, 8192]), bf16, 32/8 heads, head_dim 128, block 16 -- one step being the
KV scatter of the 256 new tokens followed by paged decode attention. ``value``
is the step's algorithmic HBM bytes / step time (GB/s), inputs resident in HBM.

Also reported, one section per BASELINE config: C1 (Qwen2.5-0.5B-shape decode),
C3 (the mixed chunked-prefill + decode packed step, us/step and tokens/s), C4
(prefix-sharing decode), C5 (W4A16 linears), the page copies, fused RoPE +
scatter and RMSNorm / SwiGLU. Every GPU time is the median of three timed loops
(HIP events on the launch stream, device syncs around each loop). Each config
has a CPU-baseline leg: the reference's CPU path (oracle/reference_path.py) on
the whole workload, on the host threads this job may use, median of >= 3 runs.

``python bench.py [--steps K] [--warmup W]``; only ``--gpus 1`` is supported.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
METRIC = "paged-decode achieved HBM GB/s (% of peak) + packed-step µs, Llama-3-8B shape"
RUNS = 3  # timed loops per GPU measurement; the median is reported


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the host-side reference timing")
    ap.add_argument("--skip-extra", action="store_true", help="headline only (no packed / prefix lines)")
    ap.add_argument("--case", default=None,
                    help="with --only w4a16: name, name:m or :m (qkv / o / gate / down / gate_up); with --only "
                         "prefix: plain or cascade -- one workload's dispatches per run (a profiling aid)")
    ap.add_argument("--only", choices=["all", "decode", "c1", "packed", "prefix", "w4a16", "block_copy", "rope_cache",
                                       "norm_act", "copy"], default="all",
                    help="decode (C2 step) / c1 / packed (C3) / prefix (C4) / w4a16 (C5) / block_copy / rope_cache / "
                         "norm_act: that section alone, GPU only; copy: 1 GiB device copies of known size, the "
                         "calibration kernel for the FETCH_SIZE/WRITE_SIZE counters (profiling aids)")
    return ap.parse_args()


def time_runs(fn, steps: int, warmup: int, runs: int = RUNS):
    """ms per call: ``warmup`` untimed calls, then ``runs`` timed loops of exactly ``steps``
    calls, each bracketed by device syncs and HIP events recorded on torch's current
    stream (the stream the kernels run on). Returns (median ms, every run's ms, wall
    ms per call of the median run)."""
    import torch

    for _ in range(warmup):
        fn()
    res = []
    for _ in range(runs):
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record()
        for _ in range(steps):
            fn()
        end.record()
        torch.cuda.synchronize()
        res.append((start.elapsed_time(end) / steps, (time.perf_counter() - t0) * 1e3 / steps))
    med = sorted(res)[len(res) // 2]
    return med[0], [round(r[0], 5) for r in res], med[1]


def graph_time(fn, calls: int, replays: int, warmup: int = 3, runs: int = RUNS) -> float:
    """ms per call of ``fn`` with ``calls`` calls captured in one HIP graph, the graph
    replayed ``replays`` times between HIP events, median of ``runs`` such loops: host
    dispatch cost (Python, ctypes) is kept out of kernels that run for a few microseconds."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warmup):  # first calls allocate the output pool and workspace
            fn()
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(calls):
            fn()
    out = []
    with torch.cuda.stream(s):
        g.replay()
        s.synchronize()
        for _ in range(runs):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(s)
            for _ in range(replays):
                g.replay()
            end.record(s)
            end.synchronize()
            out.append(start.elapsed_time(end) / (replays * calls))
    del g
    return statistics.median(out)


def host_threads() -> dict:
    """Host threads for the CPU baseline: every core of this process's affinity mask,
    capped by OMP_NUM_THREADS when the job sets it (the GPU box's CPU share)."""
    aff = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    n = min(aff, int(omp)) if omp.isdigit() and int(omp) > 0 else aff
    return {"threads": n, "affinity_cores": aff, "omp_num_threads": omp or None}


def cpu_time(fn, budget_s: float = 4.0, min_runs: int = 3, max_runs: int = 200):
    """Median seconds of ``fn`` on the host over at least ``min_runs`` runs (more while
    the runs fit ``budget_s``), after one untimed run; returns (median, runs)."""
    fn()
    times = []
    while len(times) < min_runs or (sum(times) < budget_s and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def decode_bytes(b) -> dict:
    """Algorithmic HBM bytes of one decode step (every byte the math must move, once)."""
    elem = b.kv_cache.element_size()
    kv = sum(b.ctx_host) * 2 * b.n_kv * b.head_dim * elem
    q_out = 2 * b.total_tokens * b.n_q * b.head_dim * elem
    meta = sum(math.ceil(c / b.block_size) for c in b.ctx_host) * 4 + b.batch * 4
    attn = kv + q_out + meta
    scatter = 2 * 2 * b.total_tokens * b.n_kv * b.head_dim * elem + b.total_tokens * 8
    return {"kv": kv, "attention": attn, "scatter": scatter, "step": attn + scatter}


def prefill_flops(b) -> float:
    """Causal attention FLOPs of the prefill rows: 4 * n_q * D * sum(Tq*prior + Tq(Tq+1)/2)."""
    f = 0.0
    for ctx, ql in zip(b.ctx_host, b.query_lens):
        if ql > 1:
            prior = ctx - ql
            f += 4.0 * b.n_q * b.head_dim * (ql * prior + ql * (ql + 1) / 2)
    return f


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "paged_decode_c2_hbm_traffic.json")
# the sources the decode launch is built from: a traffic profile describes the kernel
# revision these hash to, and is attached to the roofline only at that revision
DECODE_SOURCES = ("paged_decode.hip", "paged_attention.hip", "attention_common.h", "ss_common.h")


def decode_source_hash() -> str:
    h = hashlib.sha256()
    for name in DECODE_SOURCES:
        with open(os.path.join(ROOT, "slipstream_amd", "csrc", name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic(bytes_per_launch: int):
    """HBM bytes per decode launch from the committed FETCH_SIZE / WRITE_SIZE passes
    (rocprofv3 --pmc, one counter per run, scaled by a copy kernel's readings), used
    only when they were taken on this exact workload (same algorithmic bytes) and at
    this kernel revision (same source hash). Returns (bytes or None, source, note)."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None, None, "no traffic profile committed"
    if rec.get("algorithmic_bytes_per_launch") != bytes_per_launch:
        return None, None, "traffic profile taken on another workload"
    if rec.get("decode_sources_sha16") != decode_source_hash():
        return None, None, "traffic profile taken at another kernel revision"
    return int(rec["hbm_bytes_per_launch"]), os.path.relpath(TRAFFIC_FILE, ROOT), None


# ---- CPU-baseline legs: the reference's CPU path (oracle/reference_path.py) on the
# whole workload, on the host threads this job may use, median of >= 3 runs.


def _cpu_setup() -> dict:
    import torch

    th = host_threads()
    torch.set_num_threads(th["threads"])
    return th


def _host_tables(tables_host: list[list[int]]):
    import torch

    width = max(1, max(len(t) for t in tables_host))
    t = torch.full((len(tables_host), width), -1, dtype=torch.int32)
    for i, row in enumerate(tables_host):
        if row:
            t[i, : len(row)] = torch.tensor(row, dtype=torch.int32)
    return t


def _cpu_record(seconds: float, runs: int, th: dict, what: str, **extra) -> dict:
    rec = {"us_per_step": round(seconds * 1e6, 1), "cores": th["threads"], "kind": "port",
           "sample": what + f", median of {runs} runs", "affinity_cores": th["affinity_cores"],
           "omp_num_threads": th["omp_num_threads"], "cpu_model": _cpu_model()}
    rec.update(extra)
    return rec


def cpu_decode_step(b, nbytes: dict) -> dict:
    """C2: the reference's decode step on the host -- index_put scatter of the new tokens,
    then per sequence a gather of its pages and eager attention in bf16 with an fp32
    softmax (attention_ref.py:21-89, attention.py:64-88) -- over all 256 sequences."""
    from oracle import reference_path as ref

    th = _cpu_setup()
    pool = b.kv_cache.cpu()
    tables = _host_tables(b.tables_host)
    lens, q = b.context_lens.cpu(), b.padded_q().cpu()
    k_new, v_new, slots = b.k_new.cpu(), b.v_new.cpu(), b.slot_mapping.cpu()

    def step():
        ref.scatter(k_new, v_new, pool, slots, 0, b.block_size)
        ref.paged_attention(q, pool, tables, lens, 0, b.scale, b.block_size)

    t, runs = cpu_time(step, budget_s=6.0)
    rec = _cpu_record(t, runs, th, f"reference CPU path on the whole C2 step ({b.batch} sequences, "
                                   f"{sum(b.ctx_host)} KV tokens: index_put scatter + per-sequence gather + eager "
                                   "bf16 attention)")
    rec.update({"value": round(nbytes["step"] / t / 1e9, 3), "unit": "GB/s"})
    return rec


def cpu_c1(b, gpu_out) -> dict:
    """C1 on the host (the config's own CPU path), and the distance of the GPU output
    from the float64 oracle and from that path -- computed here, in the CPU leg, as the
    checker."""
    import numpy as np

    from oracle import paged_attention as ora
    from oracle import reference_path as ref

    th = _cpu_setup()
    pool, tables = b.kv_cache.cpu(), _host_tables(b.tables_host)
    lens, q = b.context_lens.cpu(), b.padded_q().cpu()
    t, runs = cpu_time(lambda: ref.paged_attention(q, pool, tables, lens, 0, b.scale, b.block_size), budget_s=3.0)
    want = ref.paged_attention(q, pool, tables, lens, 0, b.scale, b.block_size).float().numpy().astype(np.float64)
    exact = ora.paged_attention(q.float().numpy().astype(np.float64), pool.float().numpy().astype(np.float64),
                                tables.numpy(), np.array(b.ctx_host), 0, b.scale, b.block_size)
    got = gpu_out.float().cpu().numpy().astype(np.float64)
    big = np.abs(exact) >= 0.2
    return {"cpu_baseline": _cpu_record(t, runs, th, f"reference CPU path on the whole C1 batch ({b.batch} "
                                                    "sequences, fp16: per-sequence gather + eager attention)"),
            "max_abs_err_vs_oracle": float(np.abs(got - exact).max()),
            "max_rel_err_vs_oracle": float((np.abs(got - exact)[big] / np.abs(exact[big])).max()) if big.any() else 0.0,
            "max_abs_err_vs_reference_dtype_path": float(np.abs(got - want).max()),
            "reference_dtype_path_max_abs_err_vs_oracle": float(np.abs(want - exact).max())}


def cpu_packed_step(m) -> dict:
    """C3 as the reference runs a mixed step (llm_engine.py:508-567): the scatter of all
    2240 new tokens, the 192 decodes as one B x 1 paged_attention_decode call, each
    512-token chunk as its own B = 1 prefill call -- every sequence, on the host."""
    import torch

    from oracle import reference_path as ref

    th = _cpu_setup()
    pool = m.kv_cache.cpu()
    tables = _host_tables(m.tables_host)
    lens = m.context_lens.cpu()
    q = m.q.cpu()
    k_new, v_new, slots = m.k_new.cpu(), m.v_new.cpu(), m.slot_mapping.cpu()
    cu = m.cu_seqlens.cpu().tolist()
    dec = [i for i, ql in enumerate(m.query_lens) if ql == 1]
    pre = [i for i, ql in enumerate(m.query_lens) if ql > 1]
    q_dec = torch.stack([q[cu[i]] for i in dec]).unsqueeze(2)  # [n_dec, n_q, 1, D]
    q_pre = [q[cu[i]:cu[i + 1]].transpose(0, 1).unsqueeze(0).contiguous() for i in pre]

    def step():
        ref.scatter(k_new, v_new, pool, slots, 0, m.block_size)
        ref.paged_attention(q_dec, pool, tables[dec], lens[dec], 0, m.scale, m.block_size)
        for i, qi in zip(pre, q_pre):
            ref.paged_attention(qi, pool, tables[i : i + 1], lens[i : i + 1], 0, m.scale, m.block_size)

    t, runs = cpu_time(step, budget_s=6.0)
    rec = _cpu_record(t, runs, th, f"reference CPU path on the whole C3 step ({len(dec)} decodes as one call, "
                                   f"{len(pre)} chunks as one call each, scatter of {m.total_tokens} tokens)")
    rec.update({"tokens_per_s": round(m.total_tokens / t, 1)})
    return rec


def cpu_prefix(p) -> dict:
    """C4 as the reference decodes it: every sequence gathers its pages, shared prefix
    included (paged_attention_ref over prefix-cache tables)."""
    from oracle import reference_path as ref

    th = _cpu_setup()
    pool, tables = p.kv_cache.cpu(), _host_tables(p.tables_host)
    lens, q = p.context_lens.cpu(), p.padded_q().cpu()
    t, runs = cpu_time(lambda: ref.paged_attention(q, pool, tables, lens, 0, p.scale, p.block_size), budget_s=4.0)
    return _cpu_record(t, runs, th, f"reference CPU path on the whole C4 batch ({p.batch} sequences, the shared "
                                    "prefix gathered per sequence)")


C5_SHAPES = [(4096, 6144, "qkv"), (4096, 4096, "o"), (4096, 14336, "gate"), (4096, 14336, "up"),
             (14336, 4096, "down")]
ROTATE_BYTES = 640 << 20  # distinct weight bytes cycled per case: > 2x the 256 MB MALL


def _case_filter(case: str | None):
    """``--case`` of the profiling aids: "name", "name:m" or ":m" selects W4A16 cases
    (name qkv / o / gate / down / gate_up), "plain" or "cascade" the C4 leg."""
    if not case or ":" not in case and case in ("plain", "cascade"):
        return lambda name, m: True
    want_name, _, want_m = case.partition(":")
    return lambda name, m: (not want_name or want_name == name) and (not want_m or int(want_m) == m)


def w4a16_section(dev, steps: int, warmup: int, cpu: bool = False, case: str | None = None) -> dict:
    """C5: W4A16 linears of one Llama-3-8B layer at M in {1, 16, 64, 256}.

    Each case cycles through enough weight copies that the MALL cannot serve
    them; bytes = the reference-format operands read once + activations + output.
    The calls of one cycle are captured in a HIP graph (see ``graph_time``).
    CPU leg: the reference's dequantise-then-matmul (quant_ref.py:119-133) on the
    same operands, per linear and M (gate_up is this build's stacked layout, which
    the reference does not have).
    """
    import torch

    from slipstream_amd import workloads
    from slipstream_amd.kernels import w4a16_gemm

    cases = []
    layer_us = {}
    fused_us = {}  # the quantized MLP's layout: gate and up as one 4096 x 28672 linear
    cpu_layer_us = {}
    dense_layer_us = {}  # the same layer with dense bf16 weights through torch (hipBLASLt)
    th = _cpu_setup() if cpu else None
    keep = _case_filter(case)
    for k, n, name in C5_SHAPES + [(4096, 2 * 14336, "gate_up")]:
        if name == "up":  # same shape as gate: timed once, counted twice in the layer total
            continue
        if not any(keep(name, m) for m in (1, 16, 64, 256)):
            continue
        base = workloads.w4a16_linear(k, n, 256, device=dev, seed=k + n)
        copies = max(2, min(64, -(-ROTATE_BYTES // base.weight_bytes())))
        qws = [base.qweight] + [base.qweight.clone() for _ in range(copies - 1)]
        scs = [base.scales] + [base.scales.clone() for _ in range(copies - 1)]
        qzs = [base.qzeros] + [base.qzeros.clone() for _ in range(copies - 1)]
        host = None
        if cpu and name != "gate_up":
            host = (base.x.cpu(), base.qweight.cpu(), base.scales.cpu(), base.qzeros.cpu())
        for m in (1, 16, 64, 256):
            if not keep(name, m):
                continue
            x = base.x[:m].contiguous()
            idx = [0]

            def call():
                i = idx[0] % copies
                idx[0] += 1
                return w4a16_gemm(x, qws[i], scs[i], qzs[i], base.group_size)

            ms = graph_time(call, copies, max(3, steps // copies))
            wbytes = n * k // 2 + n * (k // base.group_size) * (base.scales.element_size() + 4)
            nbytes = wbytes + 2 * m * k + 2 * m * n
            flops = 2.0 * m * n * k
            gbs = nbytes / (ms * 1e-3) / 1e9
            tfl = flops / (ms * 1e-3) / 1e12
            bound = "mfma" if flops / nbytes > 312 else "hbm"
            frac = tfl / BF16_PEAK_TFLOPS if bound == "mfma" else gbs / HBM_PEAK_GBS
            case = {"linear": name, "k": k, "n": n, "m": m, "us": round(ms * 1e3, 2), "GBps": round(gbs, 1),
                    "TFLOPs": round(tfl, 2), "bound": bound, "frac": round(frac, 4), "weight_copies": copies}
            if host is not None:
                from oracle import reference_path as ref

                xh = host[0][:m].contiguous()
                t, _ = cpu_time(lambda: ref.w4a16_gemm(xh, host[1], host[2], host[3], base.group_size),
                                budget_s=0.0)
                case["cpu_us"] = round(t * 1e6, 1)
                cpu_layer_us[m] = cpu_layer_us.get(m, 0.0) + t * 1e6 * (2 if name == "gate" else 1)
            cases.append(case)
            if name != "gate_up":
                layer_us[m] = layer_us.get(m, 0.0) + ms * 1e3 * (2 if name == "gate" else 1)
            if name != "gate":
                fused_us[m] = fused_us.get(m, 0.0) + ms * 1e3
        xs = base.x
        del qws, scs, qzs, base, host
        torch.cuda.empty_cache()
        # Reference point, not a baseline of this path: the same product with dense bf16
        # weights through torch (hipBLASLt), weights rotated past the MALL the same way
        dcopies = max(2, min(16, -(-ROTATE_BYTES // (n * k * 2))))
        dws = [torch.randn(n, k, device=dev, dtype=torch.bfloat16) for _ in range(dcopies)]
        for c in cases:
            if c["linear"] != name or "dense_bf16_us" in c:
                continue
            xd = xs[: c["m"]].contiguous()
            didx = [0]

            def dense_call():
                i = didx[0] % dcopies
                didx[0] += 1
                return torch.nn.functional.linear(xd, dws[i])

            c["dense_bf16_us"] = round(graph_time(dense_call, dcopies, max(3, steps // dcopies)) * 1e3, 2)
            if name != "gate_up":
                dense_layer_us[c["m"]] = dense_layer_us.get(c["m"], 0.0) + c["dense_bf16_us"] * (2 if name == "gate" else 1)
        del dws, xs
        torch.cuda.empty_cache()
    out = {"workload": "C5 W4A16 linears of one Llama-3-8B layer (qkv 4096x6144, o 4096x4096, gate/up "
                       "4096x14336, down 14336x4096), g=128, fp16 scales, zeros 8, bf16 x",
           "cases": cases, "layer_us_by_m": {str(m): round(v, 2) for m, v in layer_us.items()},
           "layer_fused_gate_up_us_by_m": {str(m): round(v, 2) for m, v in fused_us.items()},
           "dense_bf16_layer_us_by_m": {str(m): round(v, 2) for m, v in dense_layer_us.items()},
           "note": "layer = qkv + o + gate + up + down (the reference's linears); layer_fused_gate_up = "
                   "qkv + o + gate_up + down (W4A16MLP's layout: gate and up stacked in one launch); "
                   "dense_bf16_*: the same products with dense bf16 weights through torch.nn.functional.linear "
                   "(hipBLASLt), a reference point for the MFMA-bound cases, not part of this path"}
    if cpu:
        out["cpu_baseline"] = _cpu_record(0.0, 3, th, "reference CPU path (unpack, fp32 dequant, cast, dense "
                                                       "matmul) per linear and M; cases[].cpu_us")
        del out["cpu_baseline"]["us_per_step"]
        out["cpu_baseline"]["layer_us_by_m"] = {str(m): round(v, 1) for m, v in cpu_layer_us.items()}
    return out


def block_copy_section(dev, steps: int, warmup: int) -> dict:
    """Page copies: copy-on-write of 2048 random pages of the C2 pool
    (one layer: K and V planes, 32 KB pages) and swap out / in of 512 pages to a pinned
    host cache. Bytes: every copied page is read once and written once."""
    import numpy as np
    import torch

    from slipstream_amd import workloads
    from slipstream_amd.kernels import copy_blocks, swap_blocks

    b = workloads.llama_decode(device=dev, seed=1)
    kv = b.kv_cache
    nb = kv.shape[2]
    page = kv[0, 0, 0].numel() * kv.element_size()
    rng = np.random.default_rng(0)
    blocks = rng.permutation(nb)[:4096].tolist()
    cow = dict(zip(blocks[:2048], blocks[2048:]))
    cow_pairs = torch.tensor(list(cow.items()), dtype=torch.int64, device=dev)
    ms_cow, _, _ = time_runs(lambda: copy_blocks(kv, cow_pairs), steps, warmup)  # kernel: pairs on the device
    ms_cow_dict, _, _ = time_runs(lambda: copy_blocks(kv, cow), max(3, steps // 4), 2)  # with the host upload
    cow_bytes = 2 * len(cow) * 2 * page
    host = torch.empty((1, 2, 512) + tuple(kv.shape[3:]), dtype=kv.dtype).pin_memory()
    out_map = dict(zip(blocks[:512], range(512)))
    in_map = dict(zip(range(512), blocks[512:1024]))
    ms_out, _, _ = time_runs(lambda: swap_blocks(kv, host, out_map), max(3, steps // 4), 2)
    ms_in, _, _ = time_runs(lambda: swap_blocks(host, kv, in_map), max(3, steps // 4), 2)
    swap_bytes = 512 * 2 * page
    del b, kv, host
    torch.cuda.empty_cache()
    return {"workload": "2048 copy-on-write page pairs in the C2 pool (K and V, 32 KB pages); swap of 512 "
                        "pages to / from a pinned host cache",
            "cow_us": round(ms_cow * 1e3, 2), "cow_GBps": round(cow_bytes / (ms_cow * 1e-3) / 1e9, 1),
            "cow_dict_us": round(ms_cow_dict * 1e3, 2),
            "cow_frac_hbm": round(cow_bytes / (ms_cow * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "swap_out_us": round(ms_out * 1e3, 2), "swap_out_GBps": round(swap_bytes / (ms_out * 1e-3) / 1e9, 1),
            "swap_in_us": round(ms_in * 1e3, 2), "swap_in_GBps": round(swap_bytes / (ms_in * 1e-3) / 1e9, 1)}


def rope_cache_section(dev, steps: int, warmup: int) -> dict:
    """Rotary embedding + KV scatter, fused, against the unfused pair the attention layer
    runs (torch's apply_rotary_pos_emb arithmetic on Q and K, then the scatter), at the C2
    decode step (256 tokens) and the C3 packed step (2240 tokens), Llama-3-8B shape.
    Bytes of the fused op: Q, K, V, cos, sin read once; rotated Q, K and V written once."""
    import torch

    from slipstream_amd.kernels import reshape_and_cache, rope_and_cache

    out = {"workload": "fused RoPE + KV scatter vs unfused (torch RoPE on Q, K then the scatter), "
                       "Llama-3-8B shape, bf16, packed token stream"}
    g = torch.Generator(device=dev).manual_seed(0)
    n_q, n_kv, d = 32, 8, 128
    for name, n in (("c2_256_tokens", 256), ("c3_2240_tokens", 2240)):
        q = torch.randn(n, n_q, d, generator=g, device=dev).to(torch.bfloat16)
        k = torch.randn(n, n_kv, d, generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn(n, n_kv, d, generator=g, device=dev).to(torch.bfloat16)
        pos = torch.arange(n, device=dev, dtype=torch.float32)[:, None] * 0.01
        cos, sin = torch.cos(pos.expand(n, d)).to(torch.bfloat16), torch.sin(pos.expand(n, d)).to(torch.bfloat16)
        kv = torch.zeros(1, 2, (n + 15) // 16 + 8, 16, n_kv, d, dtype=torch.bfloat16, device=dev)
        slots = torch.randperm(kv.shape[2] * 16, generator=g, device=dev)[:n]

        def fused():
            return rope_and_cache(q, k, v, cos, sin, kv, slots, 0, 16)

        def unfused():
            c, s_ = cos[:, None], sin[:, None]
            rot = lambda x: torch.cat((-x[..., d // 2:], x[..., : d // 2]), dim=-1)  # noqa: E731
            qe = q * c + rot(q) * s_
            ke = k * c + rot(k) * s_
            reshape_and_cache(ke, v, kv, slots, 0, 16)
            return qe

        ms_f = graph_time(fused, 8, max(3, steps // 8))
        ms_u = graph_time(unfused, 8, max(3, steps // 8))
        nbytes = n * ((n_q + 2 * n_kv) * d * 2 * 2 + 2 * d * 2)
        out[name] = {"fused_us": round(ms_f * 1e3, 2), "unfused_us": round(ms_u * 1e3, 2),
                     "fused_GBps": round(nbytes / (ms_f * 1e-3) / 1e9, 1), "bytes": nbytes}
    return out


def norm_act_section(dev, steps: int, warmup: int) -> dict:
    """RMSNorm (with residual) and SwiGLU kernels against the reference's eager torch
    arithmetic at a 256-token decode step of Llama-3-8B (hidden 4096, intermediate 14336),
    bf16. Bytes: inputs read once, output written once."""
    import torch
    import torch.nn.functional as F

    from slipstream_amd.kernels import fused_rmsnorm, fused_swiglu

    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(256, 4096, generator=g, device=dev).to(torch.bfloat16)
    r = torch.randn(256, 4096, generator=g, device=dev).to(torch.bfloat16)
    w = torch.ones(4096, device=dev, dtype=torch.bfloat16)
    gate = torch.randn(256, 14336, generator=g, device=dev).to(torch.bfloat16)
    up = torch.randn(256, 14336, generator=g, device=dev).to(torch.bfloat16)

    def eager_norm():
        s = x + r
        s32 = s.float()
        return w * (s32 * torch.rsqrt(s32.pow(2).mean(-1, keepdim=True) + 1e-6)).to(s.dtype)

    ms_n = graph_time(lambda: fused_rmsnorm(x, w, r, 1e-6), 16, max(3, steps // 8))
    ms_ne = graph_time(eager_norm, 16, max(3, steps // 8))
    ms_s = graph_time(lambda: fused_swiglu(gate, up), 16, max(3, steps // 8))
    ms_se = graph_time(lambda: F.silu(gate) * up, 16, max(3, steps // 8))
    nb, sb = 3 * x.numel() * 2, 3 * gate.numel() * 2
    return {"workload": "256-token decode step, Llama-3-8B: RMSNorm(x + residual) [256, 4096], "
                        "SwiGLU [256, 14336], bf16",
            "rmsnorm_us": round(ms_n * 1e3, 2), "rmsnorm_eager_us": round(ms_ne * 1e3, 2),
            "rmsnorm_GBps": round(nb / (ms_n * 1e-3) / 1e9, 1),
            "swiglu_us": round(ms_s * 1e3, 2), "swiglu_eager_us": round(ms_se * 1e3, 2),
            "swiglu_GBps": round(sb / (ms_s * 1e-3) / 1e9, 1)}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def c2_section(args, dev) -> tuple[dict, object]:
    """The headline: C2 decode step (scatter + decode attention), and the roofline of
    the decode attention launch. Returns the result line and the batch."""
    from slipstream_amd import workloads
    from slipstream_amd.kernels import paged_attention_decode, reshape_and_cache

    b = workloads.llama_decode(device=dev, seed=args.seed)
    q = b.padded_q()
    nbytes = decode_bytes(b)

    def attn():
        return paged_attention_decode(q, b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)

    def step():
        reshape_and_cache(b.k_new, b.v_new, b.kv_cache, b.slot_mapping, 0, 16)
        return attn()

    ms_step, step_runs, wall_step = time_runs(step, args.steps, args.warmup)
    ms_attn, attn_runs, _ = time_runs(attn, args.steps, args.warmup)
    value = nbytes["step"] / (ms_step * 1e-3) / 1e9
    traffic, traffic_src, traffic_note = measured_traffic(nbytes["attention"])
    attn_gbs = nbytes["attention"] / (ms_attn * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)*0.5 K/V/Q, seeded lognormal lengths, random block permutation)",
        "config": {
            "workload": "C2 Llama-3-8B-shape ragged paged decode step: KV scatter of 256 new tokens + paged decode",
            "batch": b.batch,
            "n_q_heads": b.n_q,
            "n_kv_heads": b.n_kv,
            "head_dim": b.head_dim,
            "block_size": b.block_size,
            "context_lens": "lognormal(median 1024, sigma 1.0) clipped [16, 8192]",
            "kv_tokens": sum(b.ctx_host),
            "pool_blocks": int(b.kv_cache.shape[2]),
        },
        "runs": RUNS,
        "ms_per_step_runs": step_runs,
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "tokens_per_s": round(b.batch / (ms_step * 1e-3), 1),
        "step_bytes": nbytes["step"],
        "wall_ms_per_step": round(wall_step, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": "paged decode attention launch (split-K decode_kernel + decode_merge_kernel)",
            "achieved": round(attn_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "traffic_note": traffic_note,
            "decode_sources_sha16": decode_source_hash(),
            "bytes_per_launch": nbytes["attention"],
            "us_per_launch": round(ms_attn * 1e3, 2),
            "us_per_launch_runs": [round(r * 1e3, 2) for r in attn_runs],
        },
    }
    return result, b


def c1_section(args, dev, cpu: bool) -> dict:
    """C1: Qwen2.5-0.5B-shape decode attention (fp16, 14/2 heads, D 64, 8 sequences)."""
    import torch

    from slipstream_amd import workloads
    from slipstream_amd.kernels import paged_attention_decode

    b = workloads.qwen05_decode(device=dev, seed=args.seed)
    q = b.padded_q()

    def attn():
        return paged_attention_decode(q, b.kv_cache, b.block_tables, b.context_lens, 0, b.scale, 16)

    ms, _, _ = time_runs(attn, args.steps, args.warmup)
    ms_g = graph_time(attn, 16, max(3, args.steps // 16))
    out = {"workload": "C1 Qwen2.5-0.5B-shape paged decode: fp16, 14/2 heads, D 64, bs 16, 8 sequences ctx "
                       "U[32,512], 512-block pool",
           "us_per_launch": round(ms * 1e3, 2), "us_per_launch_graph": round(ms_g * 1e3, 2),
           "kv_tokens": sum(b.ctx_host)}
    if cpu:
        res = attn()
        torch.cuda.synchronize()
        c = cpu_c1(b, res)
        c["cpu_baseline"]["gpu_over_cpu"] = round(c["cpu_baseline"]["us_per_step"] / (ms_g * 1e3), 1)
        out.update(c)
    return out


def packed_section(args, dev, cpu: bool) -> dict:
    """C3: the mixed chunked-prefill + decode packed step."""
    import torch

    from slipstream_amd import workloads
    from slipstream_amd.kernels import packed_attention, paged_attention_varlen, reshape_and_cache
    from slipstream_amd.paged_cache import build_packed_step

    m = workloads.mixed_step(device=dev, seed=args.seed)
    mb = decode_bytes(m)

    def mixed():
        reshape_and_cache(m.k_new, m.v_new, m.kv_cache, m.slot_mapping, 0, 16)
        return paged_attention_varlen(m.q, m.kv_cache, m.block_tables, m.cu_seqlens, m.context_lens, 0,
                                      m.scale, 16, m.max_query_len)

    ms_mixed, mixed_runs, _ = time_runs(mixed, max(10, args.steps // 2), args.warmup)

    # the same step as one layer runs it with nothing built on the host: metadata on
    # the device, RoPE fused with the scatter, then the varlen attention
    ql_dev = torch.tensor(m.query_lens, dtype=torch.int32, device=dev)
    prior_dev = m.context_lens.to(torch.int32) - ql_dev
    pos = torch.arange(m.total_tokens, device=dev, dtype=torch.float32)[:, None] * 0.01
    cos_t = torch.cos(pos.expand(-1, m.head_dim)).to(torch.bfloat16)
    sin_t = torch.sin(pos.expand(-1, m.head_dim)).to(torch.bfloat16)

    def layer_step():
        meta = build_packed_step(m.block_tables, prior_dev, ql_dev, 16, m.total_tokens, m.max_query_len)
        return packed_attention(m.q, m.k_new, m.v_new, cos_t, sin_t, m.kv_cache, meta, 0, m.scale, 16)

    ms_layer, _, _ = time_runs(layer_step, max(10, args.steps // 2), args.warmup)
    ms_layer_graph = graph_time(layer_step, 4, max(3, args.steps // 8))
    dec_kv = sum(c for c, ql in zip(m.ctx_host, m.query_lens) if ql == 1) * 2 * m.n_kv * m.head_dim * 2
    pre_kv = sum(c for c, ql in zip(m.ctx_host, m.query_lens) if ql > 1) * 2 * m.n_kv * m.head_dim * 2
    flops = prefill_flops(m)
    roof_us = ((dec_kv + pre_kv + mb["scatter"]) / (HBM_PEAK_GBS * 1e9) + flops / (BF16_PEAK_TFLOPS * 1e12)) * 1e6
    out = {
        "workload": "C3 mixed step: 192 decodes (ctx U[128,4096]) + 4 x 512-token chunks (prior U[0,4096]), "
                    "2240 tokens, KV scatter of all 2240 + varlen attention",
        "us_per_step": round(ms_mixed * 1e3, 2),
        "us_per_step_runs": [round(r * 1e3, 2) for r in mixed_runs],
        "tokens_per_s": round(m.total_tokens / (ms_mixed * 1e-3), 1),
        "roofline_us": round(roof_us, 2),
        "roofline_frac": round(roof_us / (ms_mixed * 1e3), 4),
        "roofline": {"bound": "hbm (decode, scatter) + mfma (prefill)", "achieved_us": round(ms_mixed * 1e3, 2),
                     "roofline_us": round(roof_us, 2), "frac": round(roof_us / (ms_mixed * 1e3), 4)},
        "decode_kv_bytes": dec_kv,
        "prefill_flops": flops,
        "layer_step_us": round(ms_layer * 1e3, 2),
        "layer_step_graph_us": round(ms_layer_graph * 1e3, 2),
        "layer_step": "device-built metadata + fused RoPE/scatter + varlen attention (no host lists)",
    }
    if cpu:
        out["cpu_baseline"] = cpu_packed_step(m)
        out["cpu_baseline"]["gpu_over_cpu"] = round(out["cpu_baseline"]["us_per_step"] / (ms_mixed * 1e3), 1)
    return out


def prefix_section(args, dev, cpu: bool) -> dict:
    """C4: decode over prefix-cache tables (128 sequences sharing a 2048-token prefix).
    ``--case plain`` / ``cascade`` times one leg alone (a profiling aid)."""
    from slipstream_amd import workloads
    from slipstream_amd.kernels import paged_attention_decode, paged_attention_shared_prefix

    p = workloads.prefix_share(device=dev, seed=args.seed)
    pq = p.padded_q()

    def pref():
        return paged_attention_decode(pq, p.kv_cache, p.block_tables, p.context_lens, 0, p.scale, 16)

    def casc():
        return paged_attention_shared_prefix(pq, p.kv_cache, p.block_tables, p.context_lens, 0, p.scale, 16,
                                             p.shared_blocks)

    if args.case in ("plain", "cascade"):
        fn = pref if args.case == "plain" else casc
        ms, _, _ = time_runs(fn, args.steps, args.warmup)
        ms_g = graph_time(fn, 8, max(3, args.steps // 8))
        return {"leg": args.case, "us_per_launch": round(ms * 1e3, 2), "us_per_launch_graph": round(ms_g * 1e3, 2)}
    ms_pref, _, _ = time_runs(pref, args.steps, args.warmup)
    ms_casc, _, _ = time_runs(casc, args.steps, args.warmup)
    ms_pref_g = graph_time(pref, 8, max(3, args.steps // 8))
    ms_casc_g = graph_time(casc, 8, max(3, args.steps // 8))
    uniq = workloads.kv_bytes(p, unique=True)
    logical = workloads.kv_bytes(p, unique=False)
    best = min(ms_casc_g, ms_pref_g)
    out = {
        "workload": "C4 Qwen2.5-7B shape (28/4 heads) decode, 128 sequences sharing a 2048-token prefix "
                    "+ private U[64,512] suffix",
        "us_per_launch": round(ms_pref * 1e3, 2),
        "unique_GBps": round(uniq / (ms_pref * 1e-3) / 1e9, 1),
        "logical_GBps": round(logical / (ms_pref * 1e-3) / 1e9, 1),
        "us_per_launch_graph": round(ms_pref_g * 1e3, 2),
        "shared_prefix_us": round(ms_casc * 1e3, 2),
        "shared_prefix_us_graph": round(ms_casc_g * 1e3, 2),
        "shared_prefix_unique_GBps_graph": round(uniq / (ms_casc_g * 1e-3) / 1e9, 1),
        "unique_bytes": uniq,
        "logical_bytes": logical,
        "roofline": {"bound": "hbm", "kernel": "paged_attention_shared_prefix (graph-timed)",
                     "achieved": round(uniq / (ms_casc_g * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(uniq / (ms_casc_g * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "frac_plain_decode": round(uniq / (ms_pref_g * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "bytes": "unique K+V bytes (the shared prefix once)"},
        "note": "unique bytes fit the 256 MB MALL; both figures reported. shared_prefix_*: "
                "paged_attention_shared_prefix (prefix read once for the batch, suffix decode, "
                "log-sum-exp combine), same result as the plain decode within the attention tolerance",
    }
    if cpu:
        out["cpu_baseline"] = cpu_prefix(p)
        out["cpu_baseline"]["gpu_over_cpu"] = round(out["cpu_baseline"]["us_per_step"] / (best * 1e3), 1)
    return out


def main() -> int:
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "this build has no multi-GPU path", file=sys.stderr)
        return 2

    import torch

    from slipstream_amd import _ffi

    _ffi.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.only == "copy":  # counter calibration: a plain copy of known size
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        src.fill_(1)
        dst = torch.empty_like(src)
        ms, _, _ = time_runs(lambda: dst.copy_(src), 5, 1, runs=1)
        print(json.dumps({"copy_bytes_read": src.numel(), "copy_bytes_written": dst.numel(),
                          "us_per_copy": round(ms * 1e3, 1)}), flush=True)
        return 0
    sections = {  # profiling aids: one section alone, GPU only
        "c1": lambda: c1_section(args, dev, False),
        "packed": lambda: packed_section(args, dev, False),
        "prefix": lambda: prefix_section(args, dev, False),
        "w4a16": lambda: w4a16_section(dev, args.steps, args.warmup, case=args.case),
        "block_copy": lambda: block_copy_section(dev, args.steps, args.warmup),
        "norm_act": lambda: norm_act_section(dev, args.steps, args.warmup),
        "rope_cache": lambda: rope_cache_section(dev, args.steps, args.warmup),
    }
    if args.only in sections:
        print(json.dumps({args.only: sections[args.only]()}), flush=True)
        return 0

    cpu = not args.no_cpu_baseline
    # ---- C2: headline decode step ------------------------------------------------
    result, b = c2_section(args, dev)
    if cpu:
        result["cpu_baseline"] = cpu_decode_step(b, decode_bytes(b))
        result["cpu_baseline"]["gpu_over_cpu"] = round(result["value"] / max(result["cpu_baseline"]["value"], 1e-9), 1)
    del b
    torch.cuda.empty_cache()
    if args.only == "decode" or args.skip_extra:
        print(json.dumps(result), flush=True)
        return 0

    result["c1_decode"] = c1_section(args, dev, cpu)
    result["packed_step"] = packed_section(args, dev, cpu)
    torch.cuda.empty_cache()
    result["prefix_share"] = prefix_section(args, dev, cpu)
    torch.cuda.empty_cache()
    result["w4a16"] = w4a16_section(dev, args.steps, args.warmup, cpu)
    result["block_copy"] = block_copy_section(dev, args.steps, args.warmup)
    result["rope_cache"] = rope_cache_section(dev, args.steps, args.warmup)
    result["norm_act"] = norm_act_section(dev, args.steps, args.warmup)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
