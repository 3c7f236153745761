"""Benchmark of Inkling relative-bias flash attention on one MI355X.

Headline (the `value`): causal prefill over a batch of 8 sequences of 4096
tokens, Hq 8 / Hkv 2, head_dim 128, bf16, per-head bias table [8,128]
(rel_extent 128), one call of the prefill kernel per step.  Reported as
TFLOP/s of algorithmic work, FLOPs = 4 * head_dim * (visible query-key pairs),
with the reference's own 2*S^2*D*Hq*B count alongside.

Also measured in the same run: split-KV decode (batch 64, one query per
sequence, KV lengths U[1024,16384] seeded, non-causal so the whole cache is
streamed) as KV GB/s against the 8 TB/s HBM peak, also with the same keys in
a paged cache (blocks of 16 tokens, shuffled) and as an fp8 (e4m3) cache; the
other prefill sequence lengths {1024, 2048, 8192}; the headline shape with a
per-token bias (fp32 extent 128, bf16 extent 1024) and with the fused
RelLogitsProj; the sliding-window chunked prefill (batch 16, window 63) with
the KV tiles it visits; the reference's own benchmark config (batch 1,
Hq = Hkv = 4, per-token bf16 bias of extent 1024, S 64..4096) next to its
published latencies; and, as the CPU baseline, the fp32 CPU oracle over the
whole headline batch (median of up to 3 passes, at most ~30 s).

Usage:  python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu]
        [--only prefill|decode|all] [--seq 4096]
Prints ONE JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "inkling-fa4-relative-attention_amd"))
sys.path.insert(0, REPO)

MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16/fp16 MFMA
HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _ensure_built():
    pkg = os.path.join(REPO, "inkling-fa4-relative-attention_amd", "inkling_fa4")
    if not (os.path.exists(os.path.join(pkg, "libifa4.so")) and
            os.path.exists(os.path.join(pkg, "_ifa4_torch.so"))):
        import __graft_entry__

        __graft_entry__.build()


def settle(fn, seconds=0.5):
    """Run `fn` untimed for about `seconds` of wall time.  The GPU clock ramps
    up over a few hundred ms of load; ten warmup calls of a 0.3 ms kernel are
    not enough (the first timed window then runs ~12% slow)."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


def time_gpu(fn, steps, warmup, settle_s=0.5):
    """Average ms per call of `fn` over `steps` back-to-back calls, bracketed by
    HIP events on the current stream (where the operator launches).  The
    clocks are settled first (`settle_s` seconds), then `warmup` untimed calls
    run."""
    import torch

    settle(fn, settle_s)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def time_gpu_samples(fn, steps, warmup):
    """Per-call event timings (ms) for percentiles."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    for a, b in evs:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return sorted(a.elapsed_time(b) for a, b in evs)


def prefill_bench(seq_len, steps, warmup, batch=8, samples=True):
    import torch
    from inkling_fa4 import inkling_fa4_rel_attention, testing

    case = testing.long_prefill(seq_len, batch=batch)
    pairs = case.visible_pairs()
    d = case.q.shape[2]
    hq = case.q.shape[1]
    flops = 4.0 * d * pairs
    flops_ref_formula = 2.0 * seq_len * seq_len * d * hq * batch
    c = case.to("cuda")
    args = c.args()

    def step():
        return inkling_fa4_rel_attention(*args, causal=True, softmax_scale=c.scale)

    ms = time_gpu(step, steps, warmup)
    samples = time_gpu_samples(step, max(10, min(steps, 50)), 2) if samples else [ms]
    tflops = flops / (ms * 1e-3) / 1e12
    return {
        "seq_len": seq_len, "batch": batch, "ms": ms, "tflops": tflops,
        "tflops_ref_formula": flops_ref_formula / (ms * 1e-3) / 1e12,
        "flops": flops, "flops_ref_formula": flops_ref_formula,
        "p10_ms": samples[len(samples) // 10], "p50_ms": samples[len(samples) // 2],
        "p90_ms": samples[(9 * len(samples)) // 10],
        "frac_of_peak": tflops / MFMA_BF16_PEAK_TFLOPS,
    }, case


def prefill_bias_variants(steps, warmup, seq_len=4096, batch=8):
    """The headline shape with the bias from a per-token rel_logits [Tq, Hq, 128]
    fp32 (what the reference operator takes) and from the fused RelLogitsProj
    factors r [Tq, Hq, 16], W [16, R'] (no rel_logits in HBM): R' = 128 with
    fp32 r, and the serving model's global extent 1024 with fp32 and bf16 r,
    next to the products that would materialise the per-token path's
    rel_logits from the same factors: [Tq, Hq, 128] fp32 and [Tq, Hq, 1024]
    bf16 (the per-token path's end-to-end time is that plus the attention)."""
    import torch
    from inkling_fa4 import (inkling_fa4_rel_attention, inkling_fa4_rel_attention_rproj,
                             testing)

    case = testing.make_case("per_token", [seq_len] * batch, [seq_len] * batch, 8, 2, 128,
                             torch.bfloat16, seed=3, rel_table=False)
    c = case.to("cuda")
    args = c.args()
    res = {"per_token_rel_ms": time_gpu(lambda: inkling_fa4_rel_attention(
        *args, causal=True, softmax_scale=c.scale), steps, warmup)}
    del args
    g = torch.Generator().manual_seed(4)
    r = (0.3 * torch.randn(case.q.shape[0], 8, 16, generator=g)).to("cuda")
    for ext in (128, 1024):
        w = (0.3 * torch.randn(16, ext, generator=g)).to("cuda")
        for r_in, key in ((r, f"rproj_rel{ext}_ms"), (r.bfloat16(), f"rproj_rel{ext}_bf16r_ms")):
            if ext == 128 and r_in.dtype == torch.bfloat16:
                continue
            res[key] = time_gpu(lambda: inkling_fa4_rel_attention_rproj(
                c.q, c.k, c.v, r_in, w, c.cu_q, c.cu_k, c.max_q, c.max_k, ext, causal=True,
                softmax_scale=c.scale), steps, warmup)
        if ext == 128:  # fp32 [Tq * Hq, 16] @ [16, 128], as the per-token leg reads it
            res["materialise_rel128_ms"] = time_gpu(
                lambda: torch.matmul(r.view(-1, 16), w), steps, warmup)
        if ext == 1024:
            res["materialise_rel1024_ms"] = time_gpu(
                lambda: torch.einsum("thc,cd->thd", r, w).to(torch.bfloat16), steps, warmup)
    res["rproj_ms"] = res["rproj_rel128_ms"]
    return res


# The reference's published prefill latencies (RTX 3090, sm86, after tuning;
# README.md:9-14) for its benchmark config (benchmarks/benchmark_prefill.py:20-49):
# batch 1, Hq = Hkv = 4, head_dim 128, bf16, causal, per-token bf16 rel_logits of
# extent 1024, 10 warmup + 50 timed calls of the wrapper between two events.
REFERENCE_README_MS = {64: 0.103, 128: 0.102, 512: 0.104, 1024: 0.160, 2048: 0.359,
                       4096: 1.037}


def reference_config_bench(seq_lens=(64, 128, 256, 512, 1024, 2048, 4096)):
    """The reference's own benchmark config at each of its sequence lengths,
    timed like the reference times it (10 warmup calls, then 50 calls of the
    operator between two events), after the usual clock settling."""
    import torch
    from inkling_fa4 import inkling_fa4_rel_attention, testing

    rows = {}
    for s in seq_lens:
        case = testing.make_case("reference_config", [s], [s], 4, 4, 128, torch.bfloat16,
                                 seed=7, rel_extent=1024, rel_table=False,
                                 rel_dtype=torch.bfloat16, rel_std=1.0)
        c = case.to("cuda")
        args = c.args()
        ms = time_gpu(lambda: inkling_fa4_rel_attention(*args, causal=True), 50, 10,
                      settle_s=0.25)
        flops_ref = 2.0 * s * s * 128 * 4  # benchmark_prefill.py:47
        row = {"ms": round(ms, 5), "tflops_ref_formula": round(flops_ref / (ms * 1e-3) / 1e12, 3)}
        if s in REFERENCE_README_MS:
            row["reference_rtx3090_ms"] = REFERENCE_README_MS[s]
        rows[str(s)] = row
        log(f"reference config seq {s}: {ms:.4f} ms")
    return {"batch": 1, "n_heads": 4, "kv_heads": 4, "head_dim": 128, "rel_extent": 1024,
            "rel": "per-token bf16", "causal": True, "seq": rows}


def window_chunked_bench(steps, warmup):
    """Sliding-window chunked prefill: batch 16, 128 new tokens over a 384-key
    cache, window 63, causal; FLOPs of the visible pairs and the KV tiles the
    kernel visits against an unpruned kernel."""
    from inkling_fa4 import inkling_fa4_rel_attention, prefill_tile_counts, testing

    case = testing.window_chunked()
    flops = 4.0 * case.q.shape[2] * case.visible_pairs()
    visited, total = prefill_tile_counts(case.cu_q, case.cu_k, case.q.shape[1], causal=True,
                                         window_size=case.window_size)
    c = case.to("cuda")
    args = c.args()
    ms = time_gpu(lambda: inkling_fa4_rel_attention(*args, causal=True,
                                                    window_size=c.window_size), steps, warmup)
    return {"ms": round(ms, 5), "tflops": round(flops / (ms * 1e-3) / 1e12, 3),
            "flops": flops, "kv_tiles_visited": visited, "kv_tiles_total": total}


def per_token_bias_bench(steps, warmup, rel_extent, seq_len=4096, batch=8):
    """The headline shape with a per-token bf16 rel_logits [Tq, Hq, rel_extent]
    (the reference's benchmark and test layout)."""
    import torch
    from inkling_fa4 import inkling_fa4_rel_attention, testing

    case = testing.make_case("per_token_bf16", [seq_len] * batch, [seq_len] * batch, 8, 2, 128,
                             torch.bfloat16, seed=8, rel_extent=rel_extent, rel_table=False,
                             rel_dtype=torch.bfloat16)
    flops = 4.0 * 128 * case.visible_pairs()
    c = case.to("cuda")
    args = c.args()
    ms = time_gpu(lambda: inkling_fa4_rel_attention(*args, causal=True), steps, warmup)
    return {"rel_extent": rel_extent, "ms": round(ms, 5),
            "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
            "rel_bytes": case.rel.numel() * case.rel.element_size()}


def decode_small_bench(steps, warmup, shapes=((1, 8192), (1, 32768), (1, 131072), (4, 8192))):
    """Decode at serving batch sizes: `batch` sequences of `keys` cached keys each
    (Hq 8 / Hkv 2, d 128, bf16, non-causal: every key streamed); us per call and
    the KV rate."""
    import torch
    from inkling_fa4 import inkling_fa4_rel_attention_decode, testing

    rows = {}
    for batch, keys in shapes:
        case = testing.make_case("decode_small", [1] * batch, [keys] * batch, 8, 2, 128,
                                 torch.bfloat16, seed=23, causal=False)
        c = case.to("cuda")
        args = c.args()
        ms = time_gpu(lambda: inkling_fa4_rel_attention_decode(*args, causal=False), steps,
                      warmup)
        kv_bytes = batch * keys * 2 * 128 * 2 * 2
        rows[f"{batch}x{keys}"] = {"us": round(ms * 1e3, 2),
                                   "gbps": round(kv_bytes / (ms * 1e-3) / 1e9, 1)}
        log(f"decode {batch} x {keys} keys: {ms * 1e3:.1f} us")
        del c, args
    return rows


def decode_bottom_right_bench(steps, warmup, rel_extent=1024):
    """The 64-sequence decode batch in the serving convention: the query at key
    Lk - 1 (bottom-right, causal keeps every key) with a per-token bf16 bias
    of `rel_extent` (the serving model's global layers: 1024), so the last
    `rel_extent` keys of every cache carry bias; beside the same call top-left,
    where no key falls in the band."""
    import torch
    from inkling_fa4 import inkling_fa4_rel_attention_decode, testing

    g, lens = testing.decode_lengths()
    case = testing.make_case("decode_br", [1] * len(lens), lens, 8, 2, 128, torch.bfloat16,
                             seed=5, causal=True, rel_extent=rel_extent, rel_table=False,
                             rel_dtype=torch.bfloat16, gen=g)
    c = case.to("cuda")
    args = c.args()
    br = time_gpu(lambda: inkling_fa4_rel_attention_decode(
        *args, causal=True, softmax_scale=c.scale, bottom_right=True), steps, warmup)
    tl = time_gpu(lambda: inkling_fa4_rel_attention_decode(
        *args, causal=False, softmax_scale=c.scale), steps, warmup)
    return {"rel_extent": rel_extent, "bottom_right_us": br * 1e3, "top_left_us": tl * 1e3}


def decode_bench(steps, warmup, block_size=0, fp8=False):
    """Decode over the 64-sequence batch; block_size > 0: the same keys in a
    paged cache of that block size (blocks in a shuffled physical order);
    fp8: the keys and values stored as float8_e4m3fn with per-tensor scales."""
    import torch
    from inkling_fa4 import (inkling_fa4_rel_attention_decode,
                             inkling_fa4_rel_attention_decode_paged, testing)

    case = testing.decode(causal=False)
    lens_k = (case.cu_k[1:] - case.cu_k[:-1])
    sum_l = int(lens_k.sum())
    hkv, d = case.k.shape[1], case.k.shape[2]
    esize = 1 if fp8 else case.k.element_size()
    kv_bytes = sum_l * hkv * d * 2 * esize
    qo_bytes = 2 * case.q.numel() * case.q.element_size()
    table_bytes = 0
    c = case.to("cuda")
    args = c.args()
    kw = {}
    if fp8:
        k8, v8, ks, vs, _ = testing.fp8_kv(case)
        kw = {"k_scale": ks, "v_scale": vs}
    if block_size:
        src = testing.replace(case, k=k8, v=v8) if fp8 else case
        pk = testing.paginate(src, block_size=block_size, seed=0, spare_blocks=0,
                              fill=0.0).to("cuda")
        table_bytes = 4 * int(((lens_k + block_size - 1) // block_size).sum())

        def step():
            return inkling_fa4_rel_attention_decode_paged(
                c.q, pk.k_cache, pk.v_cache, c.rel, c.cu_q, pk.seqused_k, pk.block_table,
                c.max_q, c.max_k, c.rel_extent, causal=False, softmax_scale=c.scale, **kw)
    elif fp8:
        k8, v8 = k8.to("cuda"), v8.to("cuda")

        def step():
            return inkling_fa4_rel_attention_decode(
                c.q, k8, v8, c.rel, c.cu_q, c.cu_k, c.max_q, c.max_k, c.rel_extent,
                causal=False, softmax_scale=c.scale, **kw)
    else:
        def step():
            return inkling_fa4_rel_attention_decode(*args, causal=False, softmax_scale=c.scale)

    ms = time_gpu(step, steps, warmup)
    nbytes = kv_bytes + qo_bytes + table_bytes
    gbps = nbytes / (ms * 1e-3) / 1e9
    out = {"batch": case.q.shape[0], "sum_kv_len": sum_l, "bytes": nbytes,
           "us": ms * 1e3, "gbps": gbps, "frac_of_peak": gbps / HBM_PEAK_GBPS}
    if block_size:
        out["block_size"] = block_size
    if fp8:
        out["kv_dtype"] = "float8_e4m3fn"
    return out


def copy_bandwidth():
    """Device-to-device copy bandwidth (GB/s, read + write) of a 1 GiB buffer."""
    import torch

    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    ms = time_gpu(lambda: b.copy_(a), 10, 3, settle_s=0.05)
    return 2 * n / (ms * 1e-3) / 1e9


def physical_cores():
    """Distinct (package, core) pairs in /proc/cpuinfo; None where it is unreadable."""
    try:
        pairs, phys = set(), None
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key = key.strip()
                if key == "physical id":
                    phys = val.strip()
                elif key == "core id":
                    pairs.add((phys, val.strip()))
        return len(pairs) or None
    except OSError:
        return None


def cpu_baseline(case, repeats=3, budget_s=30.0):
    """fp32 CPU oracle over the headline batch (every sequence, all heads),
    timed `repeats` times (fewer if the budget is spent); the median is reported."""
    import torch
    from oracle import ref_rel_attn

    try:
        threads = len(os.sched_getaffinity(0))
    except AttributeError:
        threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    cq, ck = case.cu_q.tolist(), case.cu_k.tolist()
    flops = sum(4.0 * case.q.shape[2] * ((cq[b + 1] - cq[b]) * (cq[b + 1] - cq[b] + 1) // 2)
                * case.q.shape[1] for b in range(len(cq) - 1))
    times, t_start = [], time.perf_counter()
    for r in range(repeats):
        t0 = time.perf_counter()
        for b in range(len(cq) - 1):
            lq = cq[b + 1] - cq[b]
            cu = torch.tensor([0, lq], dtype=torch.int32)
            ref_rel_attn(case.q[cq[b]:cq[b + 1]], case.k[ck[b]:ck[b + 1]],
                         case.v[ck[b]:ck[b + 1]], case.rel[cq[b]:cq[b + 1]], cu, cu,
                         case.scale, case.rel_extent, causal=True)
        times.append(time.perf_counter() - t0)
        log(f"cpu baseline: pass {r} over the batch {times[-1]:.2f} s")
        if time.perf_counter() - t_start + times[-1] > budget_s:
            break
    dt = sorted(times)[len(times) // 2]
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port", "seconds": round(dt, 6), "passes_s": [round(t, 6) for t in times],
            "cpu_count": os.cpu_count(), "physical_cores": physical_cores(),
            "sample": f"median of {len(times)} passes over the whole headline batch "
                      f"({len(cq) - 1} sequences of {cq[1] - cq[0]} tokens, all "
                      f"{case.q.shape[1]} heads), fp32 oracle (dense scores per sequence "
                      "and head) on the host CPU"}


def traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE KiB per dispatch, each scaled by the
    factor the same counter reads for a device copy of known size)."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        k = t["kernels"][kernel]
        cal = t["copy_calibration"]
        return round(1024 * (k["fetch_kib"] * cal["fetch_factor"] +
                             k["write_kib"] * cal["write_factor"]))
    except (OSError, KeyError, ValueError):
        return None


def copy_loop(n_bytes=256 << 20, reps=5):
    """Device copies of a known size, for calibrating FETCH_SIZE/WRITE_SIZE."""
    import torch

    a = torch.ones(n_bytes, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    log(f"copied {reps} x {n_bytes} bytes")


def summarize(db_path, last=None):
    """Print per-kernel dispatch statistics and per-dispatch counter averages
    from a rocprofv3 output database (SQLite).  With `last`, each kernel's
    figures cover only its last `last` dispatches (by start time): the timed
    steps of a `--no-samples` run, without the clock-settling calls before
    them."""
    import sqlite3

    con = sqlite3.connect(db_path)
    print(f"profile: {db_path}" + (f" (last {last} dispatches of each kernel)" if last else ""))
    print("| kernel | calls | avg us | min us | max us | total us |")
    print("|---|---|---|---|---|---|")
    keep = {}  # kernel name -> dispatch ids summarised
    for (name,) in con.execute("select distinct name from kernels"):
        rows = list(con.execute("select dispatch_id, duration from kernels where name = ? "
                                "order by start", (name,)))
        if last:
            rows = rows[-last:]
        keep[name] = {r[0] for r in rows}
        d = [r[1] / 1e3 for r in rows]
        print(f"| {name} | {len(d)} | {sum(d) / len(d):.3f} | {min(d):.3f} | {max(d):.3f} "
              f"| {sum(d):.1f} |")
    per = {}  # (kernel, counter) -> {dispatch: value}
    for k, cn, did, v in con.execute("select kernel_name, counter_name, dispatch_id, value "
                                     "from counters_collection"):
        if last and did not in keep.get(k, ()):
            continue
        cell = per.setdefault((k, cn), {})
        cell[did] = cell.get(did, 0.0) + v
    if per:
        print()
        print("| kernel | counter | per-dispatch avg | dispatches |")
        print("|---|---|---|---|")
        for (k, cn), cell in sorted(per.items()):
            vals = list(cell.values())
            print(f"| {k} | {cn} | {sum(vals) / len(vals):.6g} | {len(vals)} |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--only", choices=["all", "prefill", "decode"], default="all")
    ap.add_argument("--seq", type=int, default=4096)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--summarize", metavar="DB",
                    help="print a rocprofv3 output database as markdown tables and exit")
    ap.add_argument("--last", type=int, default=None,
                    help="with --summarize: only each kernel's last N dispatches")
    ap.add_argument("--no-samples", action="store_true",
                    help="skip the per-call timing samples after the timed steps (profiling "
                         "runs: the timed steps are then each kernel's last dispatches)")
    ap.add_argument("--copy-only", action="store_true",
                    help="only run device copies of a known size (counter calibration)")
    args = ap.parse_args()
    if args.summarize:
        summarize(args.summarize, args.last)
        return 0
    if args.gpus != 1:
        print("bench.py measures one GPU: the library has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        return 2

    _ensure_built()
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev_name = torch.cuda.get_device_name(0)
    log(f"device {dev_name}")
    if args.copy_only:
        copy_loop()
        return 0

    result = {
        "metric": "prefill ms + TFLOPS @seq4096 Hq8/Hkv2 d128; decode KV GB/s; % roofline",
        "value": None, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v, N(0,0.5) bias table)",
        "config": {"workload": f"causal prefill, batch 8 x seq {args.seq}, Hq 8, Hkv 2, "
                               "head_dim 128, rel_extent 128, bf16",
                   "global_batch": 8, "seq_len": args.seq, "parallelism": "single GPU"},
    }
    case = None
    if args.only in ("all", "prefill"):
        log(f"prefill seq {args.seq}: {args.steps} steps")
        pre, case = prefill_bench(args.seq, args.steps, args.warmup,
                                  samples=not args.no_samples)
        log(f"prefill seq {args.seq}: {pre['ms']:.4f} ms  {pre['tflops']:.1f} TFLOP/s")
        result["value"] = round(pre["tflops"], 2)
        result["ms_per_step"] = round(pre["ms"], 5)
        result["prefill"] = pre
        result["roofline"] = {"bound": "mfma", "kernel": "prefill_fwd_kernel<128,bf16>",
                              "achieved": round(pre["tflops"], 2),
                              "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                              "frac": round(pre["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4),
                              "traffic": traffic("prefill_fwd_kernel")}
        if not args.no_sweep:
            sweep = {}
            for s in (1024, 2048, 8192):
                if s == args.seq:
                    continue
                st = max(5, args.steps // (4 if s == 8192 else 1))
                r, _ = prefill_bench(s, st, max(2, args.warmup // 2))
                log(f"prefill seq {s}: {r['ms']:.4f} ms  {r['tflops']:.1f} TFLOP/s")
                sweep[str(s)] = {"ms": round(r["ms"], 5), "tflops": round(r["tflops"], 2),
                                 "frac_of_peak": round(r["frac_of_peak"], 4)}
            result["prefill_sweep"] = sweep
            bv = prefill_bias_variants(max(5, args.steps // 2), max(2, args.warmup // 2), args.seq)
            log(f"prefill seq {args.seq}, per-token bias: {bv['per_token_rel_ms']:.4f} ms "
                f"(+ {bv['materialise_rel128_ms']:.4f} ms to materialise it); "
                f"fused RelLogitsProj: {bv['rproj_ms']:.4f} ms; at rel_extent 1024: "
                f"{bv['rproj_rel1024_ms']:.4f} ms (bf16 r {bv['rproj_rel1024_bf16r_ms']:.4f}), "
                f"materialising its rel_logits: {bv['materialise_rel1024_ms']:.4f} ms")
            result["prefill_bias_variants"] = {k: round(v, 5) for k, v in bv.items()}
            pt = per_token_bias_bench(max(5, args.steps // 2), max(2, args.warmup // 2), 1024,
                                      args.seq)
            log(f"prefill seq {args.seq}, per-token bf16 bias, rel_extent 1024: "
                f"{pt['ms']:.4f} ms  {pt['tflops']:.1f} TFLOP/s")
            result["prefill_bias_variants"]["per_token_bf16_rel1024"] = pt
            wc = window_chunked_bench(args.steps, args.warmup)
            log(f"window + chunked prefill (batch 16, 128 over 384 keys, window 63): "
                f"{wc['ms']:.4f} ms, KV tiles {wc['kv_tiles_visited']} of {wc['kv_tiles_total']}")
            result["window_chunked"] = wc
            result["reference_config"] = reference_config_bench()
    if args.only in ("all", "decode"):
        log(f"decode: {args.steps} steps")
        dec = decode_bench(args.steps, args.warmup)
        log(f"decode: {dec['us']:.1f} us  {dec['gbps']:.0f} GB/s")
        result["decode"] = {**dec, "roofline": {"bound": "hbm",
                                                "kernel": "decode_stream_kernel + decode_combine_kernel",
                                                "achieved": round(dec["gbps"], 1),
                                                "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                                                "frac": round(dec["frac_of_peak"], 4),
                                                "traffic": traffic("decode_stream_kernel")}}
        log(f"decode, paged cache (block 16): {args.steps} steps")
        dp = decode_bench(args.steps, args.warmup, block_size=16)
        log(f"decode paged: {dp['us']:.1f} us  {dp['gbps']:.0f} GB/s")
        result["decode_paged"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                  for k, v in dp.items()}
        log(f"decode, fp8 KV cache: {args.steps} steps")
        d8 = decode_bench(args.steps, args.warmup, fp8=True)
        log(f"decode fp8: {d8['us']:.1f} us  {d8['gbps']:.0f} GB/s")
        result["decode_fp8"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                for k, v in d8.items()}
        if not args.no_sweep:
            log(f"decode, paged fp8 cache (block 16): {args.steps} steps")
            dp8 = decode_bench(args.steps, args.warmup, block_size=16, fp8=True)
            log(f"decode paged fp8: {dp8['us']:.1f} us  {dp8['gbps']:.0f} GB/s")
            result["decode_paged_fp8"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                          for k, v in dp8.items()}
        if not args.no_sweep:  # (kept out of profiling runs: same kernel, other shapes)
            result["decode_small_batch"] = decode_small_bench(args.steps, args.warmup)
            dbr = decode_bottom_right_bench(args.steps, args.warmup)
            log(f"decode bottom-right, bf16 bias extent 1024: {dbr['bottom_right_us']:.1f} us "
                f"(top-left, no key in the band: {dbr['top_left_us']:.1f} us)")
            result["decode_bottom_right_bias"] = {k: (round(v, 2) if isinstance(v, float) else v)
                                                  for k, v in dbr.items()}
        if result["value"] is None:
            result["value"] = round(dec["gbps"], 1)
            result["unit"] = "GB/s"
            result["ms_per_step"] = round(dec["us"] / 1e3, 5)
            result["roofline"] = result["decode"]["roofline"]
    if args.only == "all":
        try:
            result["copy_gbps"] = round(copy_bandwidth(), 1)
            log(f"device copy bandwidth: {result['copy_gbps']} GB/s")
        except RuntimeError as e:  # out of memory on a busy device: report, continue
            result["copy_gbps"] = None
            log(f"copy bandwidth skipped: {e}")
    if not args.skip_cpu and case is not None:
        log("cpu baseline (fp32 oracle over the batch)")
        result["cpu_baseline"] = cpu_baseline(case)
        log(f"cpu baseline: {result['cpu_baseline']['value']:.4f} TFLOP/s "
            f"in {result['cpu_baseline']['seconds']:.1f} s")
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
