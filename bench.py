"""Benchmark: decode attention over the int8ring_int4 tiered KV cache at a 262,144-token context, all 12 layers.

Workload (one "step" = one decode token through all 12 attention layers): 16 query / 2 KV heads, head_dim 256;
per layer an 8,192-slot INT8 ring (newest positions) + 253,952 older positions in 3,968 INT4-G32 pages of 64 tokens
at randomly permuted physical pages.  The cache is filled through the real write path (quantize-append, with the
oldest ring rows requantized INT8 -> INT4 on eviction).  Synthetic data: K ~ N(0,1) with 8 of 256 channels per
head x8 (seeded per layer), V ~ N(0,1), Q ~ N(0,1)/16, bf16.

Prints ONE JSON line: value = KV GB/s (algorithmic KV payload + scale bytes read per step / step time), with
us/token over all layers, the roofline of the decode kernel (live HIP-event timing of its launches) and the CPU
oracle timed on a bounded sample (one layer at the full context) as the baseline; its output also checks layer 0
of the timed path against the oracle ("parity").  The same line carries "configs": compact figures of the other
configurations (chunked prefill, quantize-append, decode with append, ragged decode, top-k sparse decode at 16 / 2
and 24 / 2 heads, dense decode over the slot-indexed pool, paged prefix-chunk attention at the reference's published
timing case), measured after the headline; --no-sub-configs leaves them out.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--impl mfma|ref]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HQ, H, D, LAYERS = 16, 2, 256, 12
CTX, RING = 262_144, 8192
PAGE = 64
PEAK_HBM = 8.0e12


def _headline_streams(layer: int, seed: int = 0):
    """The seeded input stream of one layer of the headline cache: a device generator (seed * 1000 + layer) and the
    x8 multiplier of the layer's 8 outlier K channels per head (drawn on the CPU from the same seed)."""
    g = torch.Generator(device="cuda").manual_seed(seed * 1000 + layer)
    gc = torch.Generator().manual_seed(seed * 1000 + layer)
    ch = torch.stack([torch.randperm(D, generator=gc)[:8] for _ in range(H)])
    mul = torch.ones(H, D)
    for h in range(H):
        mul[h, ch[h]] = 8.0
    return g, mul.to("cuda")


def _headline_chunk(g, mul):
    """The next RING tokens of a layer's stream: K ~ N(0, 1) with the outlier channels x8, V ~ N(0, 1), bf16."""
    k = (torch.randn(RING, H, D, device="cuda", generator=g) * mul).to(torch.bfloat16)
    v = torch.randn(RING, H, D, device="cuda", generator=g).to(torch.bfloat16)
    return k, v


def headline_inputs(layer: int, seed: int = 0):
    """All CTX tokens of one layer's K and V exactly as build_cache appended them (the same draws in the same
    order), on the device."""
    g, mul = _headline_streams(layer, seed)
    parts = [_headline_chunk(g, mul) for _ in range(0, CTX, RING)]
    return torch.cat([k for k, _ in parts]), torch.cat([v for _, v in parts])


def build_cache(seed: int = 0):
    """The headline cache: CTX positions x LAYERS layers appended through the write path in RING-token chunks (the
    oldest ring rows requantized into INT4 pages once the ring is full), pages from a permutation seeded with
    `seed`; and one seeded query per layer (N(0, 1) / 16, bf16)."""
    import kvtier  # noqa: F401
    from kvtier.kvt import PosTieredCache
    n_cold = CTX - RING
    n_pages = n_cold // PAGE
    cache = PosTieredCache(LAYERS, H, D, n_pages=n_pages, ring_total=RING, max_seqs=1, max_pages=n_pages + 1,
                           device="cuda", page_seed=seed)
    cache.add_seq(RING)
    streams = [_headline_streams(layer, seed) for layer in range(LAYERS)]
    for a in range(0, CTX, RING):
        plan = cache.plan_append([0], [RING])
        for layer in range(LAYERS):
            k, v = _headline_chunk(*streams[layer])
            cache.append(layer, plan, k, v)
        cache.commit(plan)
    torch.cuda.synchronize()
    gq = torch.Generator(device="cuda").manual_seed(seed + 77)
    q = (torch.randn(LAYERS, 1, HQ, D, device="cuda", generator=gq) / 16).to(torch.bfloat16)
    return cache, q


def cpu_baseline(cache, q, layer: int = 0):
    """The oracle (torch, CPU) on one layer at the full context: gather + dequant of every position, fp32 attention.
    Returns GB/s of KV bytes processed, the thread count and the sample description."""
    from oracle import ref
    torch.set_num_threads(os.cpu_count() or 1)
    st = ref.SeqState(0, RING, 0, cache.h_len[0], list(cache.h_pages[0]))
    oc = ref.PosTieredCache.__new__(ref.PosTieredCache)
    oc.H, oc.D, oc.group8 = H, D, cache.group8
    for name in ("k4", "v4", "ks4", "vs4", "rk", "rv", "rks", "rvs"):
        setattr(oc, name, getattr(cache, name)[layer].cpu())
    oc.seqs = [st]
    qc = q[layer, 0].cpu()
    t0 = time.perf_counter()
    kk, vv = oc.rows(0)
    exp = ref.attention_rows(qc, kk, vv, D ** -0.5)
    dt = time.perf_counter() - t0
    nbytes = cache.kv_bytes()
    return dict(value=round(nbytes / dt / 1e9, 3), unit="GB/s", cores=torch.get_num_threads(), kind="port",
                sample=f"oracle/ref.py dequant + fp32 attention of 1 of {LAYERS} layers at {CTX} tokens "
                       f"({nbytes} KV bytes, {dt:.2f} s)"), exp


def _cpu_threads() -> int:
    torch.set_num_threads(os.cpu_count() or 1)
    return torch.get_num_threads()


def cpu_baseline_append(n: int = RING, reps: int = 3) -> dict:
    """The reference's torch write arithmetic on the host cores (oracle/ref.py, vectorized over tokens): INT8-G64
    quantization of n new K and V rows and INT4-G32 requantization of n evicted ring rows; GB/s of the same
    algorithmic bytes as the GPU line."""
    from oracle import ref
    cores = _cpu_threads()
    g = torch.Generator().manual_seed(5)
    k = torch.randn(n, H, D, generator=g).to(torch.bfloat16)
    v = torch.randn(n, H, D, generator=g).to(torch.bfloat16)
    q8 = torch.randint(-127, 128, (n, H, D), dtype=torch.int8, generator=g)
    s8 = (0.002 + 0.02 * torch.rand(n, H, D // 64, generator=g)).half()
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        ref.quant8(k)
        ref.quant8(v)
        ref.requant8to4(q8, s8)
        ref.requant8to4(q8, s8)
        best = min(best, time.perf_counter() - t0)
    ring_row = H * 2 * (D + 2 * (D // 64))
    pool_row = H * 2 * (D // 2 + 2 * (D // 32))
    nbytes = n * (H * 2 * D * 2 + ring_row + 12) + n * (ring_row + pool_row)
    return dict(value=round(nbytes / best / 1e9, 3), unit="GB/s", cores=cores, kind="port",
                sample=f"oracle/ref.py quant8 of {n} K and V rows + requant8to4 of {n} evicted K and V ring rows, "
                       f"one layer ({best * 1e3:.1f} ms, best of {reps})")


def cpu_baseline_sparse(pool: dict, owner, r2t, idx, q, R: int, sm) -> dict:
    """The reference's CPU path for one layer of the top-k decode (oracle/ref.py): dequantize every request's
    selected slots as the gather writes them, then fp32 attention; us per layer."""
    from oracle import ref
    cores = _cpu_threads()
    cpu = {k: v.cpu() for k, v in pool.items()}
    own, rt, ix, qc, smc = owner.cpu(), r2t.cpu(), idx.cpu(), q.cpu(), sm.cpu()
    t0 = time.perf_counter()
    for b in range(ix.shape[0]):
        slots = rt[b, ix[b].long()]
        kk, vv = ref.dequant_slots_tiered(slots, cpu["k4"], cpu["v4"], cpu["ks4"], cpu["vs4"], cpu["rk"], cpu["rv"],
                                          cpu["rks"], cpu["rvs"], own, R - 1, smc, smc)
        ref.attention_rows(qc[b], kk, vv, D ** -0.5)
    dt = time.perf_counter() - t0
    return dict(value=round(dt * 1e6, 1), unit="us per layer", cores=cores, kind="port",
                sample=f"oracle/ref.py dequant_slots_tiered + attention_rows of {ix.shape[0]} requests x "
                       f"{ix.shape[1]} selected positions, one layer ({dt * 1e3:.1f} ms)")


def cpu_baseline_prefill(k_rows, v_rows, q_rows, a: int) -> dict:
    """The reference's CPU attention form (oracle/ref.py attention_rows) for a sample of prefill queries: query j of
    the sample sits at position a + j and attends to dequantized positions 0 .. a + j; TFLOP/s (causal flops)."""
    from oracle import ref
    cores = _cpu_threads()
    n = q_rows.shape[0]
    t0 = time.perf_counter()
    for j in range(n):
        ref.attention_rows(q_rows[j], k_rows[:a + j + 1], v_rows[:a + j + 1], D ** -0.5)
    dt = time.perf_counter() - t0
    flops = 4.0 * HQ * D * sum(a + j + 1 for j in range(n))
    return dict(value=round(flops / dt / 1e12, 4), unit="TFLOP/s", cores=cores, kind="port",
                sample=f"oracle/ref.py attention_rows of {n} queries at positions {a}..{a + n - 1} over the "
                       f"dequantized cache of one layer ({dt * 1e3:.1f} ms)")


CAL_BYTES = 256 * 1024 * 1024   # the calibration copy: 256 MiB read + 256 MiB written


def pmc_sample(impl: str) -> None:
    """The workload run under `rocprofv3 --pmc FETCH_SIZE` (then WRITE_SIZE): 12 eager decode layers (split-K +
    combine) after a warm-up, then one device copy of CAL_BYTES whose counter reading calibrates the counter."""
    import kvtier  # noqa: F401
    from kvtier.kvt import kvt_decode_attn, kvt_decode_plan
    cache, q = build_cache()
    ws = {}
    out = torch.empty(1, HQ, D, dtype=torch.float32, device="cuda")
    for _ in range(2):
        plan = kvt_decode_plan(cache, HQ, workspace=ws) if impl == "mfma" else None
        for layer in range(LAYERS):
            kvt_decode_attn(cache, layer, q[layer], out=out, impl=impl, workspace=ws, plan=plan, check_q=False)
        torch.cuda.synchronize()
    calibration_copy()
    print(json.dumps({"pmc_sample": impl, "kv_bytes_per_layer": cache.kv_bytes(), "cal_bytes": CAL_BYTES}))


def calibration_copy() -> None:
    """One device copy of CAL_BYTES, whose counter reading calibrates FETCH_SIZE / WRITE_SIZE."""
    src = torch.empty(CAL_BYTES // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()


DECODE_KERNELS = ("decode_rows_kernel", "decode_mfma_kernel", "decode_ref_kernel")


def traffic_summary(fetch_csv: str, write_csv: str, out_json: str, out_txt: str, impl: str,
                    kernels: str = "") -> None:
    """Average FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the decode kernel from two rocprofv3 --pmc counter
    CSVs, scaled by the ratio of the calibration copy's known bytes to its counter reading; also the median per
    dispatch of the cache build's append launches, scaled the same way.  `kernels` (comma-separated kernel-name
    parts) measures those kernels instead: the average per dispatch of each, and their sum as bytes per launch
    group (one layer of the top-k decode: split-K + combine)."""
    if kernels:
        return _traffic_of(fetch_csv, write_csv, out_json, out_txt, kernels.split(","))
    per_kernel = _pmc_per_kernel

    lines = []
    res = {"impl": impl}
    for counter, path, key in (("FETCH_SIZE", fetch_csv, "read"), ("WRITE_SIZE", write_csv, "write")):
        acc = per_kernel(path, counter)
        dec = [v for k, v in acc.items() if any(name in k for name in DECODE_KERNELS)]
        cal = [v for k, v in acc.items() if "copy" in k.lower() and max(v) * 1024 > CAL_BYTES / 4]
        assert dec and cal, (counter, list(acc))
        dec_v = [x for v in dec for x in v]
        cal_v = max(cal, key=max)
        cal_kib = max(cal_v)
        factor = CAL_BYTES / (cal_kib * 1024)
        dec_kib = sum(dec_v) / len(dec_v)
        res[key] = {"counter_kib_per_dispatch": round(dec_kib, 1), "calibration_copy_kib": round(cal_kib, 1),
                    "factor": round(factor, 4), "bytes_per_launch": round(dec_kib * 1024 * factor)}
        lines.append(f"{counter}: decode kernel {dec_kib:.1f} KiB/dispatch over {len(dec_v)} dispatches; copy of "
                     f"{CAL_BYTES} B {key}s {cal_kib:.1f} KiB -> factor {factor:.4f} -> {dec_kib * 1024 * factor:.0f} B")
    res["hbm_bytes_per_launch"] = res["read"]["bytes_per_launch"] + res["write"]["bytes_per_launch"]
    # the write path: the cache build's 384 append launches (8,192 tokens each; all but the first 12 evict)
    app = {}
    for counter, path, key in (("FETCH_SIZE", fetch_csv, "read"), ("WRITE_SIZE", write_csv, "write")):
        vals = sorted(x for k, v in per_kernel(path, counter).items() if "append_evict_kernel" in k for x in v)
        if vals:
            med = vals[len(vals) // 2]
            app[key] = round(med * 1024 * res[key]["factor"])
            lines.append(f"{counter}: append_evict median {med:.1f} KiB/dispatch over {len(vals)} dispatches -> "
                         f"{app[key]} B")
    if app:
        res["append_evict_bytes_per_launch"] = app
    with open(out_json, "w") as f:
        json.dump(res, f, indent=1)
    with open(out_txt, "a") as f:  # appended under the commands already written at the top of the file
        f.write("\n".join(lines) + "\n")
    print(json.dumps(res))


def _pmc_per_kernel(path: str, counter: str) -> dict:
    """Kernel name -> the counter's values per dispatch, from a rocprofv3 --pmc counter_collection CSV."""
    import csv
    acc = {}
    with open(path) as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") == counter:
                acc.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
    return acc


def _traffic_of(fetch_csv: str, write_csv: str, out_json: str, out_txt: str, names) -> None:
    res, lines = {"kernels": list(names)}, []
    for counter, path, key in (("FETCH_SIZE", fetch_csv, "read"), ("WRITE_SIZE", write_csv, "write")):
        acc = _pmc_per_kernel(path, counter)
        cal = [v for k, v in acc.items() if "copy" in k.lower() and max(v) * 1024 > CAL_BYTES / 4]
        assert cal, (counter, list(acc))
        cal_kib = max(max(cal, key=max))
        factor = CAL_BYTES / (cal_kib * 1024)
        per, total = {}, 0
        for name in names:
            vals = [x for k, v in acc.items() if name in k for x in v]
            assert vals, (counter, name, list(acc))
            kib = sum(vals) / len(vals)
            per[name] = round(kib * 1024 * factor)
            total += per[name]
            lines.append(f"{counter}: {name} {kib:.1f} KiB/dispatch over {len(vals)} dispatches; copy of {CAL_BYTES} "
                         f"B {key}s {cal_kib:.1f} KiB -> factor {factor:.4f} -> {per[name]} B")
        res[key] = {"factor": round(factor, 4), "bytes_per_dispatch": per, "bytes_per_launch": total}
    res["hbm_bytes_per_launch"] = res["read"]["bytes_per_launch"] + res["write"]["bytes_per_launch"]
    with open(out_json, "w") as f:
        json.dump(res, f, indent=1)
    with open(out_txt, "a") as f:
        f.write("\n".join(lines) + "\n")
    print(json.dumps(res))


def _measured_traffic(name: str):
    """HBM bytes per launch (group) from a committed profiles/<name>.json written by --traffic-summary, or None."""
    path = os.path.join(ROOT, "profiles", name + ".json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)["hbm_bytes_per_launch"]


def _layer_kv(n: int, layer: int, seed: int):
    """Seeded synthetic K (8 of 256 channels per head x8) and V for one layer, bf16 on the GPU."""
    gc = torch.Generator().manual_seed(seed * 1000 + layer)
    mul = torch.ones(H, D)
    for h in range(H):
        mul[h, torch.randperm(D, generator=gc)[:8]] = 8.0
    g = torch.Generator(device="cuda").manual_seed(seed * 1000 + layer)
    k = (torch.randn(n, H, D, device="cuda", generator=g) * mul.to("cuda")).to(torch.bfloat16)
    v = torch.randn(n, H, D, device="cuda", generator=g).to(torch.bfloat16)
    return k, v


def prefill_workload(args) -> dict:
    """Chunked prefill of a 10,001-token prompt, 12 layers, chunks of 2,048: per chunk the device-side append plan,
    the quantize-append of every layer (the ring's oldest rows requantized into INT4 pages once it is full), then
    causal prefill attention of every layer (the first chunk over its fresh bf16 K/V, later ones over the tiers).
    Timed: whole prompt; prefill kernels also timed alone (HIP events) for the matrix-core rate."""
    import kvtier  # noqa: F401
    from kvtier.kvt import PosTieredCache, kvt_prefill_attn
    N, CH = 10_001, 2048
    n_pages = (N - RING) // PAGE + 2
    kv = [_layer_kv(N, layer, seed=3) for layer in range(LAYERS)]
    gq = torch.Generator(device="cuda").manual_seed(303)
    qs = [(torch.randn(N, HQ, D, device="cuda", generator=gq) / 16).to(torch.bfloat16) for _ in range(LAYERS)]
    chunks = [(a, min(CH, N - a)) for a in range(0, N, CH)]
    cus = {n: torch.tensor([0, n], dtype=torch.int32, device="cuda") for _, n in chunks}
    outs = [torch.empty(CH, HQ, D, dtype=torch.bfloat16, device="cuda") for _ in range(LAYERS)]

    last = {}

    def run(events=None):
        cache = PosTieredCache(LAYERS, H, D, n_pages=n_pages, ring_total=RING, max_seqs=1, max_pages=n_pages + 1,
                               device="cuda", page_seed=0)
        last["cache"] = cache
        cache.add_seq(RING)
        # device-side append plans (positions, page pops, length updates in one launch; no host loop or copy per
        # chunk), one per chunk length, built before the timed region
        plans = {n: cache.plan_device([0], [n]) for n in sorted({n for _, n in chunks})}
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for a, n in chunks:
            plan = plans[n]
            cache.launch_plan(plan)
            for layer in range(LAYERS):
                cache.append(layer, plan, kv[layer][0][a:a + n], kv[layer][1][a:a + n])
            for layer in range(LAYERS):
                if events is not None:
                    e0 = torch.cuda.Event(enable_timing=True)
                    e0.record()
                src = dict(k_src=kv[layer][0][:n], v_src=kv[layer][1][:n]) if a == 0 else {}
                kvt_prefill_attn(cache, layer, qs[layer][a:a + n], cus[n], max_q=n, out=outs[layer][:n], **src)
                if events is not None:
                    e1 = torch.cuda.Event(enable_timing=True)
                    e1.record()
                    events.append((e0, e1))
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    for _ in range(args.warmup):
        run()
    times, evs = [], []
    for _ in range(args.steps):
        ev = []
        times.append(run(ev))
        evs.append(ev)
    torch.cuda.synchronize()
    t_prompt = min(times)
    # per prompt, the sum of its prefill launches' event intervals; the least over the timed prompts (as t_prompt),
    # since an interval also holds any wait for the host to issue the launch
    t_prefill = min(sum(a.elapsed_time(b) for a, b in ev) for ev in evs) / 1e3
    flops = 4.0 * HQ * D * (N * (N + 1) // 2) * LAYERS
    cpu = None
    if not args.no_cpu_baseline:   # the last 64 queries of layer 0 over its dequantized cache (oracle rows)
        from oracle import ref
        cache = last["cache"]
        oc = ref.PosTieredCache.__new__(ref.PosTieredCache)
        oc.H, oc.D, oc.group8 = H, D, cache.group8
        for name in ("k4", "v4", "ks4", "vs4", "rk", "rv", "rks", "rvs"):
            setattr(oc, name, getattr(cache, name)[0].cpu())
        oc.seqs = [ref.SeqState(0, RING, 0, cache.h_len[0], list(cache.h_pages[0]))]
        kk, vv = oc.rows(0)
        cpu = cpu_baseline_prefill(kk, vv, qs[0][N - 64:].cpu(), N - 64)
    return {
        "metric": "chunked prefill 10,001 tokens x 12 layers: ms per prompt (append + evict + causal prefill)",
        "value": round(t_prompt * 1e3, 3), "unit": "ms", "higher_is_better": False, "steps": args.steps,
        "warmup": args.warmup, "dtype": "bf16 QK / f16 PV mfma, f32", "data": "synthetic",
        "config": {"workload": "10,001-token prompt, chunks of 2048, 12 layers, 16 Q / 2 KV heads, D 256, ring 8192 "
                               "(1,809 positions evicted to INT4 pages in the last chunk)"},
        "roofline": {"bound": "mfma", "achieved": round(flops / t_prefill / 1e12, 2), "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(flops / t_prefill / 2.5e15, 4), "traffic": None,
                     "kernel": "prefill (causal, all chunks and layers)", "kernel_ms": round(t_prefill * 1e3, 3),
                     "flops": flops},
        "cpu_baseline": cpu,
    }


def append_workload(args) -> dict:
    """Steady-state quantize-append: 12 layers, 4 steps of 8,192-token appends into a full 8,192-row ring (every
    token evicts the oldest ring row into an INT4 page), fresh bf16 K/V per (step, layer).  The 48 launches are
    captured in one HIP graph so the timing is the device's (a Python launch costs more than a kernel); value = GB/s
    of the path's algorithmic HBM bytes."""
    import kvtier  # noqa: F401
    from kvtier.kvt import PosTieredCache
    S, N = 4, RING
    n_pages = (S + 1) * N // PAGE + 2
    cache = PosTieredCache(LAYERS, H, D, n_pages=n_pages, ring_total=RING, max_seqs=1, max_pages=n_pages + 1,
                           device="cuda", page_seed=1)
    cache.add_seq(RING)
    fill = cache.plan_append([0], [N])
    for layer in range(LAYERS):
        k, v = _layer_kv(N, layer, seed=20)
        cache.append(layer, fill, k, v)
    cache.commit(fill)
    plans = []
    for _ in range(S):
        plans.append(cache.plan_append([0], [N]))
        cache.commit(plans[-1])
    kv = [[_layer_kv(N, layer, seed=21 + s) for layer in range(LAYERS)] for s in range(S)]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for s in range(S):                                        # warm-up outside the capture
            for layer in range(LAYERS):
                cache.append(layer, plans[s], *kv[s][layer])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for s in range(S):
            for layer in range(LAYERS):
                cache.append(layer, plans[s], *kv[s][layer])
    _settle(g.replay)
    for _ in range(max(1, args.warmup)):
        g.replay()
    torch.cuda.synchronize()
    reps = max(1, args.steps)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    t_launch = e0.elapsed_time(e1) / 1e3 / (reps * S * LAYERS)
    nbytes = cache.append_bytes(N, N)
    gbps = nbytes / t_launch / 1e9
    cpu = None if args.no_cpu_baseline else cpu_baseline_append(N)
    traffic = None   # HBM bytes per launch measured by two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE)
    tfile = os.path.join(ROOT, "profiles", "decode_262k_traffic.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            ae = json.load(f).get("append_evict_bytes_per_launch")
        if ae:
            traffic = int(ae["read"]) + int(ae["write"])
    return {
        "metric": "quantize-append with ring eviction: GB/s of algorithmic HBM bytes (8,192 tokens per launch)",
        "value": round(gbps, 1), "unit": "GB/s", "higher_is_better": True, "steps": reps, "warmup": args.warmup,
        "us_per_launch": round(t_launch * 1e6, 2), "dtype": "f32 (bf16 in, INT8/INT4 out)", "data": "synthetic",
        "config": {"workload": "append 8,192 tokens x 12 layers into a full 8,192-row ring, 2 KV heads, D 256, "
                               "INT8-G64 ring, INT4-G32 pages; 4 steps per graph replay"},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                     "frac": round(gbps * 1e9 / PEAK_HBM, 4), "traffic": traffic, "kernel": "append_evict",
                     "bytes_per_launch": nbytes},
        "cpu_baseline": cpu,
    }


SETTLE_S = 0.2   # untimed replays before every timed region (seconds of wall time)


def _settle(replay, seconds: float = SETTLE_S) -> int:
    """Replays a graph, untimed, for `seconds` of wall time and returns how many times.  After an idle stretch (cache
    building, host work) the GPU's clocks take several milliseconds to come up: the first 20 replays of the 12-layer
    decode graph run about 10 % slower than every later batch of 20 (501 vs 451 us per step, measured on one box), so
    each timed region starts on a GPU that has been busy for a while.  Only replays whose repetition leaves the state
    unchanged are settled this way."""
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            replay()
        n += 8
        torch.cuda.synchronize()
    return n


def _graph_time(fn, warmup: int, reps: int) -> float:
    """Seconds per replay of a HIP graph of fn() (captured after one eager run on a side stream), timed after the
    graph has run for SETTLE_S seconds and then `warmup` more times."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        fn()
    _settle(gr.replay)
    for _ in range(max(1, warmup)):
        gr.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = max(1, reps)
    e0.record()
    for _ in range(reps):
        gr.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / reps


def gather_tier_ratio(args) -> dict:
    """The reference's tiered-vs-single-tier gather microbench (gemv/test_kv_tiers.py:561-605): 2,048 of a 4,000-token
    request's positions (sorted), batch 1, through the compact gather into the bf16 scratch -- the tiered pool with
    every row cold (owner -1) against the INT4 pool alone, and with every row hot (a ring as large as the pool whose
    rows are the INT8 pool, owner = identity) against the INT8 pool alone.  The reference's plan target is <= 1.10x
    each.  Device time per call: a HIP graph of 50 back-to-back calls.  Outputs checked bit for bit (all-cold ==
    INT4, all-hot == INT8), as the reference's bench asserts."""
    from kvtier import sparse_attn as sa
    slots, tk, L, reps = 4096, 2048, 4000, 50
    g = torch.Generator(device="cuda").manual_seed(43)
    gc = torch.Generator().manual_seed(43)
    cuda = dict(device="cuda")
    k4 = torch.randint(0, 256, (slots, H, D // 2), dtype=torch.uint8, generator=g, **cuda)
    v4 = torch.randint(0, 256, (slots, H, D // 2), dtype=torch.uint8, generator=g, **cuda)
    ks4 = (0.05 + 0.3 * torch.rand(slots, H, D // 32, generator=g, **cuda)).half()
    vs4 = (0.05 + 0.3 * torch.rand(slots, H, D // 32, generator=g, **cuda)).half()
    k8 = torch.randint(-127, 128, (slots, H, D), dtype=torch.int8, generator=g, **cuda)
    v8 = torch.randint(-127, 128, (slots, H, D), dtype=torch.int8, generator=g, **cuda)
    ks8 = (0.002 + 0.02 * torch.rand(slots, H, D // 64, generator=g, **cuda)).half()
    vs8 = (0.002 + 0.02 * torch.rand(slots, H, D // 64, generator=g, **cuda)).half()
    sm = torch.ones(H, D, dtype=torch.float16, **cuda)
    r2t = torch.randperm(slots, generator=gc).to(torch.int32)[None].to("cuda")
    ridx = torch.zeros(1, dtype=torch.int64, **cuda)
    idx = torch.randperm(L, generator=gc)[:tk].sort().values.to(torch.int32)[None].to("cuda")
    seq = torch.tensor([L], dtype=torch.int32, **cuda)
    cu = torch.tensor([0, tk], dtype=torch.int32, **cuda)
    ok = torch.empty(tk, H, D, dtype=torch.bfloat16, **cuda)
    ov = torch.empty_like(ok)
    ring = dict(ring_k=k8, ring_v=v8, ring_ks=ks8, ring_vs=vs8, ring_mask=slots - 1)
    kw4 = dict(k_scale=ks4, v_scale=vs4, sm_k=sm, sm_v=sm, kv_bits=4)
    cases = {"tiered_cold": (k4, v4, dict(kw4, owner=torch.full((slots,), -1, dtype=torch.int32, **cuda), **ring)),
             "int4": (k4, v4, kw4),
             "tiered_hot": (k4, v4, dict(kw4, owner=torch.arange(slots, dtype=torch.int32, **cuda), **ring)),
             "int8": (k8, v8, dict(k_scale=ks8, v_scale=vs8, sm_k=sm, sm_v=sm, kv_bits=8))}
    outs, us = {}, {}
    for name, (kk, vv, kw) in cases.items():
        sa.qwen_sparse_kv_extraction_compact_triton(kk, vv, r2t, ridx, idx, seq, cu, ok, ov, 1, tk, **kw)
        torch.cuda.synchronize()
        outs[name] = (ok.clone(), ov.clone())

        def calls(kk=kk, vv=vv, kw=kw):
            for _ in range(reps):
                sa.qwen_sparse_kv_extraction_compact_triton(kk, vv, r2t, ridx, idx, seq, cu, ok, ov, 1, tk, **kw)
        us[name] = _graph_time(calls, args.warmup, max(args.steps, 5)) / reps * 1e6
    same = lambda a, b: all(torch.equal(x, y) for x, y in zip(outs[a], outs[b]))
    return {"us_per_call": {k: round(v, 2) for k, v in us.items()},
            "cold_vs_int4": round(us["tiered_cold"] / us["int4"], 3),
            "hot_vs_int8": round(us["tiered_hot"] / us["int8"], 3),
            "bit_exact": same("tiered_cold", "int4") and same("tiered_hot", "int8"),
            "reference_target": 1.10}


def sparse_workload(args) -> dict:
    """Top-k sparse decode over the tiered (slot-indexed) pool: 8 requests of 65,536 tokens on randomly allocated
    slots, 12 layers, 2,051 selected positions per request (distinct, random), INT8-G64 ring of 8,192 rows whose
    owner table names one slot per row; args.hq query heads over 2 KV heads (16, or 24 as the served model).
    Times one HIP graph of the 12 layers' fused top-k decode (split-K + combine: 33 splits per request and KV
    head; the same with the splits merged inside the launch beside it, slower at this split count) and, for scale,
    one of the 12 layers' gathers into the bf16 scratch alone (the reference's unfused path runs an attention over
    that scratch on top).  Byte model per layer: each selected position's K and V rows of both KV heads from the tier
    that serves it (codes + fp16 scales), plus the index entry, its req_to_token slot and the ring owner probe (4 B
    each).  Synthetic random codes and scales."""
    hq = getattr(args, "hq", HQ)
    import kvtier  # noqa: F401
    from kvtier import sparse_attn as sa
    B, CTX, TOPK, R = 8, 65_536, 2051, 8192
    slots = B * CTX
    g = torch.Generator(device="cuda").manual_seed(41)
    gc = torch.Generator().manual_seed(41)

    def layer_pool():
        return dict(
            k4=torch.randint(0, 256, (slots, H, D // 2), dtype=torch.uint8, device="cuda", generator=g),
            v4=torch.randint(0, 256, (slots, H, D // 2), dtype=torch.uint8, device="cuda", generator=g),
            ks4=(0.05 + 0.3 * torch.rand(slots, H, D // 32, device="cuda", generator=g)).half(),
            vs4=(0.05 + 0.3 * torch.rand(slots, H, D // 32, device="cuda", generator=g)).half(),
            rk=torch.randint(-127, 128, (R, H, D), dtype=torch.int8, device="cuda", generator=g),
            rv=torch.randint(-127, 128, (R, H, D), dtype=torch.int8, device="cuda", generator=g),
            rks=(0.002 + 0.02 * torch.rand(R, H, D // 64, device="cuda", generator=g)).half(),
            rvs=(0.002 + 0.02 * torch.rand(R, H, D // 64, device="cuda", generator=g)).half())

    pools = [layer_pool() for _ in range(LAYERS)]
    owner = (torch.arange(R, dtype=torch.int64) + R * torch.randint(0, slots // R, (R,), generator=gc)).to(torch.int32)
    owner = owner.to("cuda")
    r2t = torch.randperm(slots, generator=gc).to(torch.int32).reshape(B, CTX).to("cuda")
    req_idx = torch.arange(B, dtype=torch.int64, device="cuda")
    idx = torch.stack([torch.randperm(CTX, generator=gc)[:TOPK] for _ in range(B)]).to(torch.int32).to("cuda")
    seq_lens = torch.full((B,), CTX, dtype=torch.int32, device="cuda")
    counts = torch.empty(B, dtype=torch.int32, device="cuda")
    cu_k = torch.empty(B + 1, dtype=torch.int32, device="cuda")
    sa.qwen_sparse_fa2_cu_seqlens_triton(seq_lens, idx, counts, cu_k, B, TOPK)
    sm = (0.5 + torch.rand(H, D, device="cuda", generator=g)).half()
    q = [(torch.randn(B, hq, D, device="cuda", generator=g) / 4).to(torch.bfloat16) for _ in range(LAYERS)]
    outs = [torch.empty(B, hq, D, dtype=torch.float32, device="cuda") for _ in range(LAYERS)]
    ws = [{} for _ in range(LAYERS)]
    scr_k = torch.empty(B * TOPK, H, D, dtype=torch.bfloat16, device="cuda")
    scr_v = torch.empty_like(scr_k)
    # gathered bytes per layer: each selected position's K and V rows of both heads from its tier
    sel = r2t.gather(1, idx.long()).long()
    hot = (owner.long()[sel & (R - 1)] == sel)
    n_hot = int(hot.sum())
    n_cold = hot.numel() - n_hot
    bytes_layer = H * 2 * (n_hot * (D + 2 * (D // 64)) + n_cold * (D // 2 + 2 * (D // 32))) + 3 * 4 * hot.numel()

    def fused(merge="auto"):
        for layer in range(LAYERS):
            pl = pools[layer]
            sa.qwen_sparse_decode_attn(q[layer], pl["k4"], pl["v4"], r2t, req_idx, idx, seq_lens, cu_k, B, TOPK,
                                       pl["ks4"], pl["vs4"], sm, sm, 4, pl["rk"], pl["rv"], pl["rks"], pl["rvs"],
                                       owner, R - 1, out=outs[layer], workspace=ws[layer], merge=merge)

    def gather():
        for layer in range(LAYERS):
            pl = pools[layer]
            sa.qwen_sparse_kv_extraction_compact_triton(pl["k4"], pl["v4"], r2t, req_idx, idx, seq_lens, cu_k, scr_k,
                                                        scr_v, B, TOPK, pl["ks4"], pl["vs4"], sm, sm, 4, pl["rk"],
                                                        pl["rv"], pl["rks"], pl["rvs"], owner, R - 1)

    def graph_time(fn):
        return _graph_time(fn, args.warmup, args.steps)

    if getattr(args, "pmc_sample", False):   # eager 12-layer steps under rocprofv3 --pmc, then the calibration copy
        for _ in range(3):
            fused()
        torch.cuda.synchronize()
        calibration_copy()
        print(json.dumps({"pmc_sample": "sparse", "kv_bytes_per_layer": bytes_layer, "cal_bytes": CAL_BYTES}))
        return None
    t_fused = graph_time(fused)
    t_in = graph_time(lambda: fused("launch"))
    t_gather = graph_time(gather)
    gbps = bytes_layer * LAYERS / t_fused / 1e9
    cpu = None if args.no_cpu_baseline else cpu_baseline_sparse(pools[0], owner, r2t, idx, q[0], R, sm)
    return {
        "metric": f"top-k sparse decode, fused (12 layers, batch 8, topk 2051, {hq} Q / 2 KV heads): us per step",
        "value": round(t_fused * 1e6, 1), "unit": "us", "higher_is_better": False, "steps": max(1, args.steps),
        "warmup": args.warmup, "dtype": "bf16-mfma/f32", "data": "synthetic",
        "config": {"workload": f"8 requests x 65,536 tokens on random slots, 12 layers, {hq} Q / 2 KV heads, D 256, "
                               "2,051 selected positions each, tiered pool (INT8-G64 ring of 8,192 rows + INT4-G32)",
                   "hot_fraction": round(n_hot / hot.numel(), 4)},
        "merged_in_launch_us_per_step": round(t_in * 1e6, 1),
        "gather_only_us_per_step": round(t_gather * 1e6, 1),
        "gather_tier_ratio": gather_tier_ratio(args),
        "kv_bytes_per_layer": bytes_layer,
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                     "frac": round(gbps * 1e9 / PEAK_HBM, 4),
                     "traffic": _measured_traffic(f"sparse_topk2051_{hq}q_traffic"),
                     "kernel": "sparse_decode + combine (per layer)"},
        "cpu_baseline": cpu,
    }


def slots_workload(args) -> dict:
    """Dense decode over the slot-indexed tiered pool (the layout the reference's backend reads): 4 requests of
    65,536 positions on randomly permuted slots, 1 layer, INT8-G64 ring of 8,192 rows whose owner table names one slot
    per row (3 % of the positions hot), every position attended.  Times one HIP graph of decode_attn_slots through the
    matrix cores (the fused sparse decode with every position selected, + the combine) and, for scale, the scalar
    reference-precision kernel.  Byte model per position and KV head: the K and V rows of its tier (INT8 256 B + 8 B
    of scales, or INT4 128 B + 16 B, per tensor) plus its req_to_token slot and owner probe.  Synthetic random codes
    and scales."""
    import kvtier  # noqa: F401
    from kvtier.kvt import decode_attn_slots
    B, CTX, R = 4, 65_536, 8192
    slots = B * CTX
    g = torch.Generator(device="cuda").manual_seed(51)
    gc = torch.Generator().manual_seed(51)
    k4 = torch.randint(0, 256, (slots, H, D // 2), dtype=torch.uint8, device="cuda", generator=g)
    v4 = torch.randint(0, 256, (slots, H, D // 2), dtype=torch.uint8, device="cuda", generator=g)
    ks4 = (0.05 + 0.3 * torch.rand(slots, H, D // 32, device="cuda", generator=g)).half()
    vs4 = (0.05 + 0.3 * torch.rand(slots, H, D // 32, device="cuda", generator=g)).half()
    rk = torch.randint(-127, 128, (R, H, D), dtype=torch.int8, device="cuda", generator=g)
    rv = torch.randint(-127, 128, (R, H, D), dtype=torch.int8, device="cuda", generator=g)
    rks = (0.002 + 0.02 * torch.rand(R, H, D // 64, device="cuda", generator=g)).half()
    rvs = (0.002 + 0.02 * torch.rand(R, H, D // 64, device="cuda", generator=g)).half()
    owner = (torch.arange(R, dtype=torch.int64) + R * torch.randint(0, slots // R, (R,), generator=gc)).to(torch.int32)
    r2t = torch.randperm(slots, generator=gc).to(torch.int32).reshape(B, CTX)
    hot = (owner.long()[r2t.long() & (R - 1)] == r2t.long())
    n_hot = int(hot.sum())
    n_cold = hot.numel() - n_hot
    owner, r2t = owner.to("cuda"), r2t.to("cuda")
    req_idx = torch.arange(B, dtype=torch.int64, device="cuda")
    seq = torch.full((B,), CTX, dtype=torch.int32, device="cuda")
    q = (torch.randn(B, HQ, D, device="cuda", generator=g) / 16).to(torch.bfloat16)
    bytes_step = H * (n_hot * 2 * (D + 2 * (D // 64)) + n_cold * 2 * (D // 2 + 2 * (D // 32))) + 8 * hot.numel()
    ws = {}
    outs = {}

    def run(impl):
        def fn():
            outs[impl] = decode_attn_slots(q, seq, r2t, req_idx, k4, v4, ks4, vs4, rk, rv, rks, rvs, owner, R - 1,
                                           impl=impl, max_len=CTX, workspace=ws if impl == "mfma" else None)
        return fn

    t_mfma = _graph_time(run("mfma"), args.warmup, args.steps)
    t_ref = _graph_time(run("ref"), 1, max(1, args.steps // 4))
    err = float((outs["mfma"] - outs["ref"]).abs().max())
    gbps = bytes_step / t_mfma / 1e9
    return {
        "metric": "dense decode over the slot-indexed tiered pool (4 x 65,536 positions, 1 layer): us per step",
        "value": round(t_mfma * 1e6, 1), "unit": "us", "higher_is_better": False, "steps": max(1, args.steps),
        "warmup": args.warmup, "dtype": "bf16-mfma/f32", "data": "synthetic",
        "config": {"workload": "4 requests x 65,536 positions on random slots, 1 layer, 16 Q / 2 KV heads, D 256, "
                               "tiered pool (INT8-G64 ring of 8,192 rows + INT4-G32)",
                   "hot_fraction": round(n_hot / hot.numel(), 4)},
        "scalar_kernel_us_per_step": round(t_ref * 1e6, 1),
        "max_abs_vs_scalar_kernel": err,
        "kv_bytes_per_step": bytes_step,
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                     "frac": round(gbps * 1e9 / PEAK_HBM, 4), "traffic": None,
                     "kernel": "sparse_decode over every position + combine"},
        "cpu_baseline": None,
    }


def _indexer_rows(q_len: int, prefix: int, topk: int, gen: torch.Generator) -> torch.Tensor:
    """Index rows shaped like the indexer's output for a chunk of q_len queries after `prefix` positions (the timing
    case of gemv/test_kv_paged_prefix.py:306-331): per query sorted distinct positions below its visible length,
    -1 padding; about 3 % of the rows empty, 3 % only current-chunk positions, 4 % one position (at most 8 each) and
    15 % a random shorter selection."""
    idx = torch.full((q_len, topk), -1, dtype=torch.int32)
    special = {"empty": 0, "chunk_only": 0, "single": 0}
    for j in range(q_len):
        visible = prefix + j + 1
        n = min(topk, visible)
        u = float(torch.rand(1, generator=gen))
        if u < 0.03 and special["empty"] < 8:
            special["empty"] += 1
            continue
        if u < 0.06 and prefix > 0 and special["chunk_only"] < 8:
            special["chunk_only"] += 1
            pos = torch.arange(prefix, visible)[:n]
        elif u < 0.10 and special["single"] < 8:
            special["single"] += 1
            pos = torch.randint(0, visible, (1,), generator=gen)
        else:
            if u < 0.25:
                n = int(torch.randint(0, n + 1, (1,), generator=gen))
            pos = torch.randperm(visible, generator=gen)[:n].sort().values
        idx[j, :pos.numel()] = pos.to(torch.int32)
    return idx


def paged_prefix_workload(args) -> dict:
    """The reference's published timing case of its paged prefix-chunk attention (gemv/test_kv_paged_prefix.py:539-611;
    figures in patches/kv_paged_prefix.py:42-45): one request with a 60,000-token prefix and a 1,024-query chunk,
    1 KV head x 12 q heads, D 256, tiered pool (INT8-G64 ring of 8,192 rows over INT4-G32; position p in slot p, so
    the newest 8,192 slots own the ring), topk 2,051 with the indexer-like rows of _indexer_rows.  Times
    sparse_gqa_fwd_interface_paged: device time per call (HIP graph of back-to-back calls) and, as the reference
    measures, the median host time of a synchronized call.  Byte model (the reference's): each valid selection's K
    and V rows from the tier that serves it + 12 B of index, slot and owner reads.  Synthetic random codes and
    scales; the CPU baseline (the oracle on 8 sampled queries) also gives the max-abs difference of those queries."""
    import kvtier  # noqa: F401
    from kvtier import sparse_attn as sa
    PREFIX, CHUNK, R, TOPK, QH = 60_000, 1024, 8192, 2051, 12
    ctx = PREFIX + CHUNK
    h1 = 1
    g = torch.Generator(device="cuda").manual_seed(51)
    gc = torch.Generator().manual_seed(51)
    pool = dict(
        k4=torch.randint(0, 256, (ctx, h1, D // 2), dtype=torch.uint8, device="cuda", generator=g),
        v4=torch.randint(0, 256, (ctx, h1, D // 2), dtype=torch.uint8, device="cuda", generator=g),
        ks4=(0.05 + 0.3 * torch.rand(ctx, h1, D // 32, device="cuda", generator=g)).half(),
        vs4=(0.05 + 0.3 * torch.rand(ctx, h1, D // 32, device="cuda", generator=g)).half(),
        rk=torch.randint(-127, 128, (R, h1, D), dtype=torch.int8, device="cuda", generator=g),
        rv=torch.randint(-127, 128, (R, h1, D), dtype=torch.int8, device="cuda", generator=g),
        rks=(0.002 + 0.02 * torch.rand(R, h1, D // 64, device="cuda", generator=g)).half(),
        rvs=(0.002 + 0.02 * torch.rand(R, h1, D // 64, device="cuda", generator=g)).half())
    rows = torch.arange(R, dtype=torch.int64)
    owner = torch.where(rows < ctx % R, rows + (ctx // R) * R, rows + (ctx // R - 1) * R).to(torch.int32).to("cuda")
    r2t = torch.arange(ctx, dtype=torch.int32, device="cuda").reshape(1, ctx)
    req_idx = torch.zeros(1, dtype=torch.int64, device="cuda")
    kv_lens = torch.tensor([ctx], dtype=torch.int32, device="cuda")
    cu_q = torch.tensor([0, CHUNK], dtype=torch.int64, device="cuda")
    idx_cpu = _indexer_rows(CHUNK, PREFIX, TOPK, gc)
    idx = idx_cpu.to("cuda")
    sm_k = (0.5 + torch.rand(h1, D, device="cuda", generator=g)).half()
    sm_v = (0.5 + torch.rand(h1, D, device="cuda", generator=g)).half()
    q = (torch.randn(CHUNK, QH, D, device="cuda", generator=g) / 4).to(torch.bfloat16)
    out = torch.empty(CHUNK, QH, D, dtype=torch.float32, device="cuda")

    def call():
        sa.sparse_gqa_fwd_interface_paged(q, idx, cu_q, kv_lens, r2t, req_idx, pool["k4"], pool["v4"], pool["ks4"],
                                          pool["vs4"], sm_k, sm_v, D ** -0.5, CHUNK, 4, pool["rk"], pool["rv"],
                                          pool["rks"], pool["rvs"], owner, R - 1, out=out)

    if getattr(args, "pmc_sample", False):   # eager calls under rocprofv3 --pmc, then the calibration copy
        for _ in range(5):
            call()
        torch.cuda.synchronize()
        calibration_copy()
        print(json.dumps({"pmc_sample": "paged_prefix", "cal_bytes": CAL_BYTES}))
        return None
    t_dev = _graph_time(call, args.warmup, max(args.steps, 10))
    host = []
    for _ in range(10):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        call()
        torch.cuda.synchronize()
        host.append(time.perf_counter() - t0)
    t_host = sorted(host)[len(host) // 2]
    sel = idx_cpu[idx_cpu >= 0].long()               # every entry is below its query's visible length here
    hot = owner.cpu().long()[sel & (R - 1)] == sel
    n_sel, n_hot = sel.numel(), int(hot.sum())
    row4, row8 = 2 * (D // 2 + 2 * (D // 32)), 2 * (D + 2 * (D // 64))
    kv_bytes = h1 * ((n_sel - n_hot) * row4 + n_hot * row8) + 12 * n_sel
    flops = 4.0 * D * QH * n_sel
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import ref
        cores = _cpu_threads()
        cp = {k: v.cpu() for k, v in pool.items()}
        own, qc, smk, smv, oc = owner.cpu(), q.cpu(), sm_k.cpu(), sm_v.cpu(), out.cpu()
        sample = [j for j in range(CHUNK - 1, -1, -127)][:8]
        err = 0.0
        t0 = time.perf_counter()
        for j in sample:
            slots = ref.prefill_selected_positions(idx_cpu[j], PREFIX + j + 1, ctx, TOPK)
            kk, vv = ref.dequant_slots_tiered(slots, cp["k4"], cp["v4"], cp["ks4"], cp["vs4"], cp["rk"], cp["rv"],
                                              cp["rks"], cp["rvs"], own, R - 1, smk, smv)
            o = ref.attention_rows(qc[j], kk, vv, D ** -0.5)
            err = max(err, float((o - oc[j]).abs().nan_to_num(0.0).max()))
        dt = time.perf_counter() - t0
        cpu = dict(value=round(dt / len(sample) * 1e3, 3), unit="ms per query", cores=cores, kind="port",
                   sample=f"oracle/ref.py prefill_selected_positions + dequant_slots_tiered + attention_rows of "
                          f"{len(sample)} queries of the chunk ({dt * 1e3:.1f} ms); max-abs vs the GPU rows {err:.2e}")
    return {
        "metric": "paged prefix-chunk attention over the tiered pool (prefix 60,000, chunk 1,024, 1 KV head x 12 "
                  "q heads, topk 2,051): ms per call",
        "value": round(t_dev * 1e3, 4), "unit": "ms", "higher_is_better": False, "steps": max(args.steps, 10),
        "warmup": args.warmup, "dtype": "bf16-mfma/f32", "data": "synthetic",
        "config": {"workload": "the reference's paged-prefix timing case: 1 request, prefix 60,000 + chunk 1,024 "
                               "queries, 1 KV head x 12 q heads, D 256, tiered pool (INT8-G64 ring 8,192 over "
                               "INT4-G32), topk 2,051, indexer-like rows",
                   "selected_rows": n_sel, "hot_fraction": round(n_hot / max(n_sel, 1), 4)},
        "host_median_ms_per_synchronized_call": round(t_host * 1e3, 4),
        "reference_published_ms": {"paged_tiered": 6.10, "paged_int8": 3.19, "paged_int4": 4.21,
                                   "materialised_gather_plus_kernel": 1.31,
                                   "hardware": "RTX PRO 4000 Blackwell (~0.5 TB/s)"},
        "kv_bytes_per_call": kv_bytes,
        "TFLOPs": round(flops / t_dev / 1e12, 2),
        "roofline": {"bound": "hbm", "achieved": round(kv_bytes / t_dev / 1e9, 1), "peak": PEAK_HBM / 1e9,
                     "unit": "GB/s", "frac": round(kv_bytes / t_dev / PEAK_HBM, 4),
                     "traffic": _measured_traffic("paged_prefix_60k_traffic"),
                     "kernel": "sparse_prefill (row requests; the 21.9 MB pool is re-read through the caches)"},
        "cpu_baseline": cpu,
    }


def lazy_workload(args) -> dict:
    """Lazy backing of the tiered slot pool on HIP virtual memory at the full context: 262,144 slots x 12 layers
    (2 KV heads, D 256; INT8 ring of 8,192 rows eagerly allocated).  Times, host wall with the device synchronized:
    the pool's construction (48 reservations + the 4,096-token floor), the growth from the floor to the full pool in
    2,048-token hand-outs of PagedTokenAllocator (each backs the next 2,048 slots of all 48 buffers and zeroes them,
    14.2 MB), and the release back to the floor once every slot is free.  Then two readers of the pool as 12-layer
    HIP graphs, over the lazily backed pool and over an eagerly allocated one of the same shape: the fused top-k
    decode (8 requests x 32,768 slots, 2,051 random positions each: random rows) and the whole-prefix
    gather-dequant (every slot, streaming).  Pool contents are the zeros of fresh backing (timing only)."""
    import kvtier  # noqa: F401
    from kvtier import sparse_attn as sa
    from kvtier.tiered_kv_pool import MHATokenToKVPoolTiered, PagedTokenAllocator
    SIZE, STEP, B, TOPK = 262_144, 2048, 8, 2051
    CTXB = SIZE // B

    def pool(lazy):
        return MHATokenToKVPoolTiered(SIZE, PAGE, torch.uint8, H, D, LAYERS, "cuda", lazy=lazy)

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    lz = pool(True)
    torch.cuda.synchronize()
    t_build = time.perf_counter() - t0
    alloc = PagedTokenAllocator(SIZE, PAGE, lz, device="cuda")
    step_s, chunks = [], []
    while alloc.available_size() >= STEP:
        t0 = time.perf_counter()
        idx = alloc.alloc(STEP)
        torch.cuda.synchronize()
        step_s.append(time.perf_counter() - t0)
        if idx is None:
            raise RuntimeError(f"lazy backing refused a hand-out at {len(chunks) * STEP} slots")
        chunks.append(idx)
    backed_full = lz.lazy_backed_tokens
    step_bytes = STEP * lz._lazy.bytes_per_token()
    eager = pool(False)
    gc = torch.Generator().manual_seed(43)
    g = torch.Generator(device="cuda").manual_seed(43)
    r2t = torch.cat(chunks).to(torch.int32).reshape(B, CTXB).contiguous()
    req_idx = torch.arange(B, dtype=torch.int64, device="cuda")
    idx = torch.stack([torch.randperm(CTXB, generator=gc)[:TOPK] for _ in range(B)]).to(torch.int32).to("cuda")
    seq_lens = torch.full((B,), CTXB, dtype=torch.int32, device="cuda")
    cu_k = torch.tensor([i * TOPK for i in range(B + 1)], dtype=torch.int32, device="cuda")
    cu_p = torch.tensor([i * CTXB for i in range(B + 1)], dtype=torch.int32, device="cuda")
    q = [(torch.randn(B, hq, D, device="cuda", generator=g) / 4).to(torch.bfloat16) for _ in range(LAYERS)]
    outs = [torch.empty(B, hq, D, dtype=torch.float32, device="cuda") for _ in range(LAYERS)]
    scr_k = torch.empty(SIZE, H, D, dtype=torch.bfloat16, device="cuda")
    scr_v = torch.empty_like(scr_k)

    def readers(p):
        ws = [{} for _ in range(LAYERS)]

        def fused():
            for layer in range(LAYERS):
                k, v = p.get_kv_buffer(layer)
                ks, vs = p.get_kv_scale_buffer(layer)
                sk, sv = p.get_kv_smooth_buffer(layer)
                rk, rv, rks, rvs = p.get_kv_ring_buffer(layer)
                sa.qwen_sparse_decode_attn(q[layer], k, v, r2t, req_idx, idx, seq_lens, cu_k, B, TOPK, ks, vs, sk, sv,
                                           4, rk, rv, rks, rvs, p.ring_owner, p.ring_mask, out=outs[layer],
                                           workspace=ws[layer])

        def prefix():
            for layer in range(LAYERS):
                k, v = p.get_kv_buffer(layer)
                ks, vs = p.get_kv_scale_buffer(layer)
                sk, sv = p.get_kv_smooth_buffer(layer)
                rk, rv, rks, rvs = p.get_kv_ring_buffer(layer)
                sa.qwen_sparse_prefix_gather_dequant_tiered(k, v, ks, vs, sk, sv, r2t, req_idx, seq_lens, cu_p, scr_k,
                                                            scr_v, B, CTXB, rk, rv, rks, rvs, p.ring_owner,
                                                            p.ring_mask)
        return (_graph_time(fused, args.warmup, args.steps), _graph_time(prefix, args.warmup, args.steps))

    t_fused_l, t_prefix_l = readers(lz)
    t_fused_e, t_prefix_e = readers(eager)
    del eager
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for c in chunks:
        alloc.free(c)
    t_release = time.perf_counter() - t0
    backed_after = lz.lazy_backed_tokens
    step_s.sort()
    med = step_s[len(step_s) // 2]
    fused_bytes = LAYERS * B * TOPK * H * 2 * (D // 2 + 2 * (D // 32))        # INT4 rows + scales of both heads
    prefix_bytes = LAYERS * SIZE * H * 2 * (D // 2 + 2 * (D // 32) + 2 * D)   # + the bf16 rows written
    gbps = fused_bytes / t_fused_l / 1e9
    return {
        "metric": "lazy KV backing (12-layer 262,144-slot tiered pool): us per 2,048-token commit step",
        "value": round(med * 1e6, 1), "unit": "us", "higher_is_better": False, "steps": max(1, args.steps),
        "warmup": args.warmup, "dtype": "u8/f16 (pool)", "data": "synthetic (zeros of fresh backing)",
        "config": {"workload": "262,144-slot tiered pool x 12 layers on HIP VMM (2 MiB granules), floor 4,096, "
                               "margin 2,048; readers: top-k decode 8 x 2,051 of 32,768, whole-prefix gather"},
        "commit_steps": len(step_s), "commit_bytes_per_step": step_bytes,
        "commit_us": {"median": round(med * 1e6, 1), "min": round(step_s[0] * 1e6, 1),
                      "max": round(step_s[-1] * 1e6, 1),
                      "mean": round(sum(step_s) / len(step_s) * 1e6, 1)},
        "commit_GBps_median": round(step_bytes / med / 1e9, 2),
        "build_ms": round(t_build * 1e3, 2), "release_ms": round(t_release * 1e3, 2),
        "backed_tokens": {"full": backed_full, "after_release": backed_after},
        "sparse_decode_us_per_step": {"lazy": round(t_fused_l * 1e6, 1), "eager": round(t_fused_e * 1e6, 1)},
        "prefix_gather_us_per_step": {"lazy": round(t_prefix_l * 1e6, 1), "eager": round(t_prefix_e * 1e6, 1)},
        "prefix_gather_GBps": {"lazy": round(prefix_bytes / t_prefix_l / 1e9, 1),
                               "eager": round(prefix_bytes / t_prefix_e / 1e9, 1)},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                     "frac": round(gbps * 1e9 / PEAK_HBM, 4), "traffic": None,
                     "kernel": "sparse_decode + combine over the lazily backed pool (per layer)"},
        "cpu_baseline": None,
    }


def decode_steps_workload(args, ragged: bool) -> dict:
    """ragged = False: one layer, 10,001-token context (ring 8192 + 1,809 paged positions), 1,000 steps of
    append-one-token + decode.  ragged = True: 8 sequences with log-uniform lengths in [1024, 65536] (seeded), 12
    layers, two sequences sharing a 4,096-token prefix in common pages, 256 iterations of one decode step per
    sequence (append + decode of every layer).  Reports us per step (wall, host planning included), the KV GB/s of
    the decode launches as timed by events around the eager calls, and the decode of the final state replayed as a
    HIP graph (the device's own rate)."""
    import kvtier  # noqa: F401
    from kvtier.kvt import PosTieredCache, kvt_decode_attn, kvt_decode_plan
    layers = LAYERS if ragged else 1
    # a decode plan is one more launch per step that the step's layers share: worth it from two layers on
    use_plan = args.impl == "mfma" and layers > 1
    if ragged:
        gl = torch.Generator().manual_seed(4)
        lens = [int(math.exp(math.log(1024) + (math.log(65536) - math.log(1024)) * float(u)))
                for u in torch.rand(8, generator=gl)]
        lens[0], lens[1] = max(lens[0], 4096 + 1024), max(lens[1], 4096 + 1024)   # the two prefix sharers
        steps = 256
    else:
        lens = [10_001]
        steps = 1000
    S = len(lens)
    rings = [min(RING, 1 << (max(1, L) - 1).bit_length()) for L in lens]
    shared = 4096 if ragged else 0
    n_host = min(100, steps // 4)              # host-planned eager steps, timed for reference
    extra = args.warmup + n_host + 4           # tokens appended besides the timed steps (warm-ups, capture)
    n_pages = sum(max(0, L + steps + extra - r) // PAGE + 2 for L, r in zip(lens, rings)) + shared // PAGE
    max_pages = max(lens) // PAGE + (steps + extra) // PAGE + 4
    cache = PosTieredCache(layers, H, D, n_pages=n_pages, ring_total=sum(rings), max_seqs=S, max_pages=max_pages,
                           device="cuda", page_seed=5)
    # the shared prefix: 64 pages taken from the allocator and written once with the INT4 writer (positions 0..4095),
    # then referenced by sequences 0 and 1 through their page tables (ring_start = 4096)
    seqs = []
    if shared:
        from kvtier import sparse_attn
        shared_pages = [cache.alloc.pop() for _ in range(shared // PAGE)]
        rows = (torch.tensor(shared_pages, device="cuda")[:, None] * PAGE
                + torch.arange(PAGE, device="cuda")[None, :]).reshape(-1)
        ones = torch.ones(H, D, dtype=torch.float16, device="cuda")
        for layer in range(layers):
            k, v = _layer_kv(shared, layer, seed=40)
            sparse_attn.quant_store_kv_int4(k, v, rows, cache.k4[layer], cache.v4[layer], cache.ks4[layer],
                                            cache.vs4[layer], ones, ones)
    for i, (L, r) in enumerate(zip(lens, rings)):
        if shared and i < 2:
            seqs.append(cache.add_seq(r, ring_start=shared, shared_pages=shared_pages))
        else:
            seqs.append(cache.add_seq(r))
    done = [shared if (shared and i < 2) else 0 for i in range(S)]
    while any(d < L for d, L in zip(done, lens)):
        act = [i for i in range(S) if done[i] < lens[i]]
        cnt = [min(rings[i], lens[i] - done[i]) for i in act]
        plan = cache.plan_append([seqs[i] for i in act], cnt)
        for layer in range(layers):
            k, v = _layer_kv(sum(cnt), layer, seed=7 + done[act[0]])
            cache.append(layer, plan, k, v)
        cache.commit(plan)
        for i, n in zip(act, cnt):
            done[i] += n
    n_all = cache.n_seqs
    gq = torch.Generator(device="cuda").manual_seed(9)
    q = (torch.randn(layers, n_all, HQ, D, device="cuda", generator=gq) / 16).to(torch.bfloat16)
    knew, vnew = _layer_kv(S, 0, seed=11)
    ws = {}
    out = torch.empty(n_all, HQ, D, dtype=torch.float32, device="cuda")

    # eager steps through the host planner (plan_append: a Python loop, page pops, host-to-device copies)
    def host_step():
        plan = cache.plan_append(seqs, [1] * S)
        for layer in range(layers):
            cache.append(layer, plan, knew, vnew)
        cache.commit(plan)
        dp = kvt_decode_plan(cache, HQ, workspace=ws) if use_plan else None
        for layer in range(layers):
            kvt_decode_attn(cache, layer, q[layer], out=out, impl=args.impl, workspace=ws, plan=dp, check_q=False)

    for _ in range(args.warmup):
        host_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n_host):
        host_step()
    torch.cuda.synchronize()
    wall_host = (time.perf_counter() - t0) / n_host

    # the timed steps: the device plan (positions, page pops, lengths on the device), every layer's append and decode
    # captured once as one HIP graph and replayed once per step -- no host work per step
    dplan = cache.plan_device(seqs, [1] * S)

    def dev_step():
        cache.launch_plan(dplan)
        for layer in range(layers):
            cache.append(layer, dplan, knew, vnew)
        dp = kvt_decode_plan(cache, HQ, workspace=ws) if use_plan else None
        for layer in range(layers):
            kvt_decode_attn(cache, layer, q[layer], out=out, impl=args.impl, workspace=ws, plan=dp, check_q=False)

    dev_step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dev_step()
    graph.replay()
    torch.cuda.synchronize()
    cache.sync_host()
    kv_first = cache.kv_bytes(seqs) * layers
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    g0.record()
    for _ in range(steps):
        graph.replay()
    g1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    dev_s = g0.elapsed_time(g1) / 1e3 / steps
    cache.sync_host()
    kv_last = cache.kv_bytes(seqs) * layers
    kv_avg = (kv_first + kv_last) / 2

    # decode alone over the final state (every layer, one graph): the device's decode rate
    def dec_only():
        dp = kvt_decode_plan(cache, HQ, workspace=ws) if use_plan else None
        for layer in range(layers):
            kvt_decode_attn(cache, layer, q[layer], out=out, impl=args.impl, workspace=ws, plan=dp, check_q=False)

    dec_only()   # (eagerly first: the split map of the final lengths)
    torch.cuda.synchronize()
    dgraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(dgraph):
        dec_only()
    dgraph.replay()
    torch.cuda.synchronize()
    _settle(dgraph.replay)
    d0, d1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    d0.record()
    for _ in range(20):
        dgraph.replay()
    d1.record()
    torch.cuda.synchronize()
    dec_graph = d0.elapsed_time(d1) / 1e3 / 20
    # the same decode 12 times in one graph (the 1-layer workload only): device time per decode without the cost of
    # launching a graph per decode
    dec_b2b = None
    if layers == 1:
        bgraph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(bgraph):
            for _ in range(12):
                dec_only()
        _settle(bgraph.replay)
        d0.record()
        for _ in range(20):
            bgraph.replay()
        d1.record()
        torch.cuda.synchronize()
        dec_b2b = d0.elapsed_time(d1) / 1e3 / (20 * 12)
    name = ("ragged decode: 8 sequences, 12 layers, shared 4,096-token prefix, 256 iterations" if ragged
            else "decode with append: 10,001-token context, 1 layer, 1,000 steps")
    return {
        "metric": name + ": us per step", "value": round(wall * 1e6, 1), "unit": "us", "higher_is_better": False,
        "steps": steps, "warmup": args.warmup, "dtype": "f16-mfma/f32", "data": "synthetic",
        "config": {"workload": name, "lens": lens, "rings": rings, "impl": args.impl,
                   "step": "device append plan + append of every layer + decode plan + decode of every layer, one "
                           "HIP graph per step"},
        "device_us_per_step": round(dev_s * 1e6, 1),
        "wall_over_device": round(wall / dev_s, 3),
        "host_planned_eager_us_per_step": round(wall_host * 1e6, 1),
        "kv_GBps_per_step": round(kv_avg / dev_s / 1e9, 1),
        "kv_bytes_per_step": int(kv_avg),
        "decode_graph_us_per_step": round(dec_graph * 1e6, 1),
        "decode_graph_kv_GBps": round(kv_last / dec_graph / 1e9, 1),
        "decode_back_to_back_us": None if dec_b2b is None else round(dec_b2b * 1e6, 1),
    }


def sub_configs(args) -> dict:
    """Compact figures of the other configurations, measured in the same process after the headline (whose cache
    is freed first): chunked prefill of a 10,001-token prompt, the 8,192-token quantize-append with eviction, decode
    with append at a 10,001-token context, ragged 8-sequence decode, the top-k sparse decode at 16 / 2 and 24 / 2
    heads, the dense decode over the slot-indexed pool and the paged prefix-chunk attention at the reference's published
    timing case.  Each runs without its CPU baseline; a failure is reported in place of its figures."""
    sub = argparse.Namespace(**vars(args))
    sub.no_cpu_baseline, sub.steps, sub.warmup = True, 5, 1
    res = {}

    def run(name, fn, pick):
        try:
            res[name] = pick(fn(sub))
        except Exception as e:  # noqa: BLE001 -- reported in the line, never hidden
            res[name] = {"error": f"{type(e).__name__}: {e}"}
        torch.cuda.synchronize()
        torch.cuda.empty_cache()

    def pick_steps(r):
        return {"us_per_step": r["value"], "device_us_per_step": r["device_us_per_step"],
                "kv_GBps": r["kv_GBps_per_step"], "decode_graph_us_per_step": r["decode_graph_us_per_step"],
                "decode_graph_kv_GBps": r["decode_graph_kv_GBps"],
                "decode_back_to_back_us": r["decode_back_to_back_us"]}

    def pick_sparse(r):
        return {"us_per_step": r["value"], "GBps": r["roofline"]["achieved"], "hbm_frac": r["roofline"]["frac"],
                "kv_bytes_per_layer": r["kv_bytes_per_layer"], "gather_only_us_per_step": r["gather_only_us_per_step"],
                "gather_tier_ratio": r["gather_tier_ratio"]}

    run("prefill10k", prefill_workload,
        lambda r: {"ms_per_prompt": r["value"], "kernel_ms": r["roofline"]["kernel_ms"],
                   "TFLOPs": r["roofline"]["achieved"], "mfma_frac": r["roofline"]["frac"]})
    run("append8192", append_workload,
        lambda r: {"GBps": r["value"], "hbm_frac": r["roofline"]["frac"], "us_per_launch": r["us_per_launch"]})
    run("decode10k_append", lambda a: decode_steps_workload(a, False), pick_steps)
    run("ragged8", lambda a: decode_steps_workload(a, True), pick_steps)
    for hq in (16, 24):
        run(f"sparse_topk2051_{hq}q", lambda a, hq=hq: sparse_workload(argparse.Namespace(**dict(vars(a), hq=hq))),
            pick_sparse)
    run("slots_dense_4x65k", slots_workload,
        lambda r: {"us_per_step": r["value"], "GBps": r["roofline"]["achieved"], "hbm_frac": r["roofline"]["frac"],
                   "scalar_kernel_us_per_step": r["scalar_kernel_us_per_step"]})
    run("paged_prefix_60k", paged_prefix_workload,
        lambda r: {"ms_per_call": r["value"], "host_ms": r["host_median_ms_per_synchronized_call"],
                   "TFLOPs": r["TFLOPs"], "row_GBps": r["roofline"]["achieved"],
                   "reference_published_ms": r["reference_published_ms"]["paged_tiered"]})
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--impl", default=os.environ.get("KVT_DECODE_IMPL", "mfma"))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--workload", default="decode262k", choices=["decode262k", "prefill10k", "decode10k", "ragged", "append", "sparse", "slots", "paged_prefix", "lazy"],
                    help="decode262k (default): the headline line; the others measure the remaining configurations")
    ap.add_argument("--hq", type=int, default=HQ, help="query heads of the sparse workload (2 KV heads)")
    ap.add_argument("--no-sub-configs", action="store_true",
                    help="headline only: skip the compact figures of the other configurations")
    ap.add_argument("--pmc-sample", action="store_true", help="run the rocprofv3 --pmc traffic sample and exit")
    ap.add_argument("--traffic-summary", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "OUT_JSON", "OUT_TXT"),
                    help="summarize two rocprofv3 --pmc counter CSVs into the traffic file and exit")
    ap.add_argument("--traffic-kernels", default="",
                    help="with --traffic-summary: comma-separated kernel-name parts to measure instead of the decode")
    args = ap.parse_args()
    if args.traffic_summary:
        traffic_summary(*args.traffic_summary, impl=args.impl, kernels=args.traffic_kernels)
        return
    if args.pmc_sample and args.workload in ("sparse", "paged_prefix"):
        (sparse_workload if args.workload == "sparse" else paged_prefix_workload)(args)
        return
    if args.pmc_sample:
        pmc_sample(args.impl)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); sharding across GPUs is a documented "
              "design, not a measured path", file=sys.stderr)
        sys.exit(2)
    if args.workload != "decode262k":
        fn = {"prefill10k": prefill_workload, "decode10k": lambda a: decode_steps_workload(a, False),
              "ragged": lambda a: decode_steps_workload(a, True), "append": append_workload,
              "sparse": sparse_workload, "slots": slots_workload, "paged_prefix": paged_prefix_workload,
              "lazy": lazy_workload}[args.workload]
        line = fn(args)
        line["n_gpus"] = 1
        print(json.dumps(line))
        return
    import kvtier  # noqa: F401
    from kvtier.kvt import kvt_decode_attn, kvt_decode_plan

    cache, q = build_cache()
    ws = {}
    outs = [torch.empty(1, HQ, D, dtype=torch.float32, device="cuda") for _ in range(LAYERS)]

    def step(events=None):
        # the step's decode plan (every block's ranges and first tile rows, shared by the 12 layers), then per layer
        # the split-K launch + the combine; the synthetic queries are in the fp16 range (no per-call host check)
        plan = kvt_decode_plan(cache, HQ, workspace=ws) if args.impl == "mfma" else None
        for layer in range(LAYERS):
            kvt_decode_attn(cache, layer, q[layer], out=outs[layer], impl=args.impl, workspace=ws, events=events,
                            plan=plan, check_q=False)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # the timed step: one HIP graph holding the 12 layers' split-K + combine launches (no host work per step)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    settle = _settle(graph.replay)
    for _ in range(args.warmup):
        graph.replay()
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record()
    for _ in range(args.steps):
        graph.replay()
    t_end.record()
    torch.cuda.synchronize()
    ms_step = t_start.elapsed_time(t_end) / args.steps
    # kernel timing: HIP events on the launch stream around K replays of a graph of the 12 split-K launches alone
    # (the step's plan built before), per launch = elapsed / (K x 12): the kernel's device time plus the boundary to
    # the next launch, no host gaps (events around eager launches also count the launch latency)
    kplan = kvt_decode_plan(cache, HQ, workspace=ws) if args.impl == "mfma" else None

    def splitk_only():
        for layer in range(LAYERS):
            kvt_decode_attn(cache, layer, q[layer], out=outs[layer], impl=args.impl, workspace=ws, plan=kplan,
                            check_q=False, partials_only=True)

    kgraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(kgraph):
        splitk_only()
    _settle(kgraph.replay)
    k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    k0.record()
    for _ in range(args.steps):
        kgraph.replay()
    k1.record()
    torch.cuda.synchronize()
    kern_avg_s = k0.elapsed_time(k1) / 1e3 / (args.steps * LAYERS)
    # the rest of a step per layer: the combine launch and its boundary (plus 1 / 12 of the plan launch)
    comb_avg_us = (ms_step / 1e3 / LAYERS - kern_avg_s) * 1e6
    graph.replay()   # the outputs of a full step again, for the parity check below
    torch.cuda.synchronize()
    bytes_layer = cache.kv_bytes()
    bytes_step = bytes_layer * LAYERS
    value = bytes_step / (ms_step / 1e3) / 1e9
    achieved = bytes_layer / kern_avg_s
    traffic = None
    tfile = os.path.join(ROOT, "profiles", "decode_262k_traffic.json")
    if os.path.exists(tfile):
        with open(tfile) as f:
            t = json.load(f)
        if t.get("impl") == args.impl:
            traffic = t.get("hbm_bytes_per_launch")
    cpu = parity = None
    if not args.no_cpu_baseline:
        # the CPU leg's oracle output doubles as a correctness check of the timed path at its own shape: layer 0's
        # output of the last graph replay against the oracle's fp32 attention over the cache's rows
        cpu, exp = cpu_baseline(cache, q)
        err = (outs[0][0].cpu() - exp).abs()
        parity = {"layer": 0, "max_abs": float(err.max()), "mean_abs": float(err.mean()),
                  "tolerance": [2e-3, 1e-3], "ok": bool(float(err.max()) <= 2e-3 and float(err.mean()) <= 1e-3)}
        if not parity["ok"]:
            print(f"bench.py: the measured decode differs from the oracle beyond tolerance ({parity}); the line is "
                  "invalid", file=sys.stderr)
    line = {
        "metric": "decode-attn KV GB/s and % HBM peak at 256k ctx; us/token all layers",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"seconds": SETTLE_S, "replays": settle},
        "ms_per_step": round(ms_step, 4),
        "us_per_token_all_layers": round(ms_step * 1e3, 1),
        "hbm_frac_of_step": round(value * 1e9 / PEAK_HBM, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16-mfma/f32" if args.impl == "mfma" else "f32",
        "data": "synthetic",
        "config": {
            "workload": "decode 262144-token context x 12 layers: 16 Q / 2 KV heads, D 256, INT8-G64 ring 8192 + "
                        "253952 tokens in 3968 INT4-G32 pages (permuted), batch 1",
            "impl": args.impl,
            "kernel": ("full-row split-K (both KV heads per wavefront) with the step's decode plan + combine"
                       if args.impl == "mfma" else "reference-precision split-K + combine"),
            "kv_bytes_per_layer": bytes_layer,
            "kv_bytes_per_step": bytes_step,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved / 1e9, 2),
            "peak": PEAK_HBM / 1e9,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM, 4),
            "traffic": traffic,
            "kernel": "decode split-K (per layer launch)",
            "kernel_avg_us": round(kern_avg_s * 1e6, 2),
            "kernel_timing": "graph of the 12 split-K launches alone, HIP events, per launch incl. the boundary",
            "rest_of_layer_us": round(comb_avg_us, 2),
        },
        "cpu_baseline": cpu,
        "parity": parity,
    }
    if parity is not None and not parity["ok"]:
        line["invalid"] = "decode output outside the oracle tolerance"
    if not args.no_sub_configs:
        del cache, q, outs, ws, graph
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        line["configs"] = sub_configs(args)
    print(json.dumps(line))
    if parity is not None and not parity["ok"]:
        sys.exit(1)


if __name__ == "__main__":
    main()
