"""Tile sweep of the gfx950 kernels: build variants over compile-time knobs,
check each against the in-tree build, time it on the GPU, optionally with
rocprofv3 counters.

Replaces the reference's benchmarks/autotune.py:21-81, an exhaustive
BLOCK_Q/BLOCK_K/warps/stages timing loop whose launches pass out=None with zero
output strides (autotune.py:74,78), so its numbers cannot be trusted.

Two steps, so that variants are built where hipcc is and timed where the GPU is:

  python -m inkling_fa4.sweep build --dir DIR --grid IFA4_LOOK_K=2,4,6 --grid IFA4_PRIO=0,1
  python -m inkling_fa4.sweep run --dir DIR --workload prefill [--seq 4096] [--steps 30]
        (workloads: prefill = shared bias table; prefill_reference = the reference's own
        benchmark config (batch 1, 4 heads, per-token bf16 bias of extent 1024, split
        KV); decode_br1024 = the decode batch bottom-right with a per-token bf16 bias
        of extent 1024; prefill_token = per-token fp32 bias of
        extent 128; prefill_token1024 = per-token bf16 bias of extent 1024;
        prefill_table1024 = one shared bf16 bias row of extent 1024; rproj128 /
        rproj512 / rproj1024 = fused projection of that extent; decode, decode_fp8,
        decode_paged, decode_paged_fp8)
        [--counters SQ_VALU_MFMA_BUSY_CYCLES,GRBM_GUI_ACTIVE] [--out table.md]
  python -m inkling_fa4.sweep split [--shapes reference,headline] [--seqs 1024,4096]
        (split-KV prefill against the unsplit kernel, in-tree build)

`build` writes one sub-directory per grid point holding libifa4.so, a copy of the
torch binding (it loads the libifa4.so next to it), knobs.json and the digest of
the sources (one snapshot per call: edits during the build do not leak in).  `run` first
runs the in-tree build, then each variant in a child process with IFA4_LIB_DIR
pointing at its directory; a variant whose output on a small case differs from
the in-tree build's (atol 2e-2 on out, 1e-3 on lse) is reported and not timed.

Knobs (macros of the kernel sources):
  prefill_fwd.hip  IFA4_LOOK_K, IFA4_LOOK_V   LDS reads in flight ahead of the QK / PV MFMAs
                   IFA4_PRIO                  raised wave priority around MFMA blocks (0/1)
                   IFA4_SCHED                 scheduling groups (0/1)
                   IFA4_PV2                   key-block-major PV (0/1)
                   IFA4_BIAS_LDS              shared bias table in LDS (0/1)
                   IFA4_PREFILL_NQB           32-row blocks per wave (1/2)
                   IFA4_BLOCK_K               keys per KV tile (32/64)
                   IFA4_WPE                   waves per SIMD the register budget targets
                   IFA4_PREFILL_WAVES         waves per workgroup (4: 128 query rows, 8: 256)
                   IFA4_PROJ_SKIP             fused projection: skip distance blocks outside
                                              the band (0/1; workloads rproj128/512/1024)
                   IFA4_PROJ_EARLY            fused projection: key block 0's distances
                                              projected before the QK products (0/1)
                   IFA4_MERGE_BATCH           split-KV merge pass: chunks whose loads are in
                                              flight together (2/4/8)
                   IFA4_MERGE_PARTS           split-KV merge pass: workgroups per query tile
                                              (4/8/16)
  ifa4_device.hpp  IFA4_DMA_COVER_EACH        hazard cover on every LDS DMA (1) or one per
                                              batch of a tile's DMAs (0)
  decode_fwd.hip   IFA4_DECODE_WPE            waves per SIMD the stream pass's registers target
                   IFA4_COMBINE_SPLIT         combine of many-part segments over 2 or 4
                                              workgroups per (head, sequence) (0/1)
                   IFA4_DECODE_BAND_UNITS     stream-K weight of a bias-band step (4 units = a
                                              plain step; workload decode_br1024)
                   IFA4_DECODE_PAIR_OVERLAP   fp8 kv head pairs: next step's loads in flight
                                              while a step computes (0/1)
                   IFA4_DECODE_NBUF_PAIR      fp8 kv head pairs: step buffers per wave (2/3)
                   IFA4_DECODE_WPE_PAIR       fp8 kv head pairs: waves per SIMD of the budget
  tile_table.h     IFA4_DECODE_WAVES          persistent waves of the decode stream pass
                   IFA4_DECODE_MIN_STEPS      fewest 32-key steps per wave (small calls)
                   IFA4_DECODE_MAX_PARTS      most waves per (sequence, kv head) cache
                   IFA4_DECODE_WAVES_FP8      the same for an fp8 KV cache (workload decode_fp8)
                   IFA4_DECODE_WAVES_PAGED    the same for a paged cache (workload decode_paged)
                   IFA4_DECODE_FP8_PAIRS      fp8 caches of d 128 with adjacent kv heads stream
                                              kv head pairs (0/1; workload decode_fp8)
                   IFA4_DECODE_WAVES_FP8_PAIR waves of such a pair stream
                   IFA4_DECODE_WAVES_FP8_PAIR_PAGED  the same for a paged cache (workload
                                              decode_paged_fp8)
                   IFA4_PREFILL_SPLIT_MAX_GRID  largest prefill grid the table splits (split KV)
                   IFA4_PREFILL_CHUNK_PCT     split KV: chunk length, percent of the balanced share
                   IFA4_PREFILL_MIN_CHUNK     split KV: shortest chunk in KV tiles
                   IFA4_PREFILL_CHUNK_FIT     split KV: chunk lengthened until the chunks fit the
                                              resident slots (0/1)
                   IFA4_PREFILL_SPLIT_MIN_SAVED  split KV taken for chunks over half the longest
                                              KV range only if they shorten it by this many tiles
"""
import argparse
import hashlib
import itertools
import json
import os
import shutil
import sqlite3
import subprocess
import sys
import tempfile
import time

_HERE = os.path.dirname(os.path.abspath(__file__))
_PKG_ROOT = os.path.dirname(_HERE)  # inkling-fa4-relative-attention_amd/


def _grid_points(specs):
    """['A=1,2', 'B=x'] -> [{'A': '1', 'B': 'x'}, {'A': '2', 'B': 'x'}]"""
    names, values = [], []
    for spec in specs:
        name, _, vals = spec.partition("=")
        if not name or not vals:
            raise SystemExit(f"bad --grid {spec!r}: expected NAME=v1,v2,...")
        names.append(name)
        values.append(vals.split(","))
    return [dict(zip(names, combo)) for combo in itertools.product(*values)]


def _source_digest(csrc, include):
    h = hashlib.sha256()
    for d in (csrc, include):
        for name in sorted(os.listdir(d)):
            path = os.path.join(d, name)
            if os.path.isfile(path) and name.endswith((".hip", ".cpp", ".h", ".hpp")):
                h.update(name.encode())
                with open(path, "rb") as f:
                    h.update(f.read())
    return h.hexdigest()[:12]


def cmd_build(args):
    sys.path.insert(0, _PKG_ROOT)
    import build as b  # inkling-fa4-relative-attention_amd/build.py

    ext = os.path.join(_HERE, b.EXT_NAME)
    if not os.path.exists(ext):
        raise SystemExit(f"{ext} is missing: build the package first (build.py)")
    os.makedirs(args.dir, exist_ok=True)
    with tempfile.TemporaryDirectory() as snap:
        # every variant of this call is built from one copy of the sources, so
        # an edit while the grid builds cannot mix two versions in one library
        csrc = shutil.copytree(b.CSRC, os.path.join(snap, "csrc"))
        include = shutil.copytree(b.INCLUDE, os.path.join(snap, "include"))
        digest = _source_digest(csrc, include)
        for knobs in _grid_points(args.grid):
            name = "_".join(f"{k.replace('IFA4_', '').lower()}{v}" for k, v in knobs.items())
            out = os.path.join(args.dir, name)
            with tempfile.TemporaryDirectory() as tmp:
                b.build_library(args.jobs, out_dir=out,
                                defines=[f"{k}={v}" for k, v in knobs.items()], build_dir=tmp,
                                csrc=csrc, include=include)
            shutil.copy2(ext, os.path.join(out, b.EXT_NAME))
            with open(os.path.join(out, "knobs.json"), "w") as f:
                json.dump(knobs, f)
            with open(os.path.join(out, "source.txt"), "w") as f:
                f.write(digest + "\n")
            print(f"built {out}  {knobs}  sources {digest}", flush=True)
    return 0


def _case(workload, seq, batch=1, heads=4):
    import torch
    from inkling_fa4 import testing

    if workload == "prefill":
        # check case: ragged tails, bias-band tiles, a run of interior tiles (the
        # 700-token sequence), Lq > Lk and Lq < Lk; non-causal, so that no mask
        # hides a bias element (the timed case is causal)
        check = testing.make_case("sweep_check", [700, 64, 300], [700, 33, 500], 8, 2, 128,
                                  torch.bfloat16, seed=2, causal=False, rel_extent=400)
        return check, testing.long_prefill(seq, batch=8)
    if workload == "prefill_reference":
        # the reference's benchmark config (benchmarks/benchmark_prefill.py:20-49):
        # batch 1, Hq = Hkv = 4, d 128, causal, per-token bf16 bias of extent 1024;
        # the tile table splits its KV range (underfilled grid)
        # (--batch / --heads change the batch and the head count, Hq = Hkv)
        mk = lambda name, lens, h, seed: testing.make_case(  # noqa: E731
            name, lens, lens, h, h, 128, torch.bfloat16, seed=seed, rel_extent=1024,
            rel_table=False, rel_dtype=torch.bfloat16, rel_std=1.0)
        return mk("sweep_check", [1500], 4, 2), mk("reference_config", [seq] * batch, heads, 7)
    if workload.startswith("prefill_token") or workload.startswith("rproj"):
        # per-token rel_logits (extent 128 fp32, or 1024 bf16 for prefill_token1024),
        # or the fused projection (its factors are drawn in _call): batch 8,
        # Hq 8 / Hkv 2, d 128, causal
        ext = int(workload[5:]) if workload.startswith("rproj") else (
            1024 if workload == "prefill_token1024" else 128)
        rd = torch.bfloat16 if workload == "prefill_token1024" else torch.float32
        mk = lambda name, lens, seed: testing.make_case(  # noqa: E731
            name, lens, lens, 8, 2, 128, torch.bfloat16, seed=seed, rel_extent=ext,
            rel_table=False, rel_dtype=rd)
        return mk("sweep_check", [1300, 64, 33], 2), mk("per_token", [seq] * 8, 3)
    if workload == "prefill_table1024":
        # one bf16 bias row of extent 1024 shared by every token (token stride 0):
        # the shared-table path, or with IFA4_BIAS_LDS=0 the per-token gather
        # reading a bias that stays in cache -- what the gather costs besides
        # its HBM bytes
        mk = lambda name, lens, seed: testing.make_case(  # noqa: E731
            name, lens, lens, 8, 2, 128, torch.bfloat16, seed=seed, rel_extent=1024,
            rel_table=True, rel_dtype=torch.bfloat16)
        return mk("sweep_check", [1300, 64, 33], 2), mk("table1024", [seq] * 8, 3)
    if workload.startswith("decode_small"):
        # --batch sequences of --seq cached keys each (serving at small batch);
        # _fp8 / _paged: the same keys as an fp8 or a paged cache
        lens = [seq] * batch
        return (testing.make_case("sweep_check", [1] * 3, [300, 5000, 77], 8, 2, 128,
                                  torch.bfloat16, seed=21, causal=False),
                testing.make_case("decode_small", [1] * batch, lens, 8, 2, 128,
                                  torch.bfloat16, seed=22, causal=False))
    if workload == "decode_br1024":
        # the decode batch in the serving convention: bottom-right, causal, a
        # per-token bf16 bias of extent 1024 (the last 1024 keys of every cache)
        g, lens = testing.decode_lengths()
        mk = lambda name, lq, lk, seed, gen=None: testing.make_case(  # noqa: E731
            name, lq, lk, 8, 2, 128, torch.bfloat16, seed=seed, causal=True, rel_extent=1024,
            rel_table=False, rel_dtype=torch.bfloat16, gen=gen)
        return (mk("sweep_check", [1] * 3, [300, 5000, 1500], 21),
                mk("decode_br", [1] * len(lens), lens, 5, g))
    return testing.decode(batch=8, seed=21, causal=False), testing.decode(causal=False)


def _call(workload, case, return_lse):
    import torch
    from inkling_fa4 import (inkling_fa4_rel_attention, inkling_fa4_rel_attention_decode,
                             inkling_fa4_rel_attention_decode_paged,
                             inkling_fa4_rel_attention_rproj, testing)

    if workload.startswith("rproj"):  # r [Tq, 8, 16] fp32, W [16, R'] (std 0.3)
        g = torch.Generator().manual_seed(4)
        r = (0.3 * torch.randn(case.q.shape[0], case.q.shape[1], 16, generator=g)).to(
            case.q.device)
        w = (0.3 * torch.randn(16, case.rel_extent, generator=g)).to(case.q.device)
        return lambda: inkling_fa4_rel_attention_rproj(
            case.q, case.k, case.v, r, w, case.cu_q, case.cu_k, case.max_q, case.max_k,
            case.rel_extent, causal=case.causal, softmax_scale=case.scale,
            return_lse=return_lse)
    fn = (inkling_fa4_rel_attention if workload.startswith("prefill")
          else inkling_fa4_rel_attention_decode)
    args = case.args()
    kw = {}
    if workload in ("decode_paged", "decode_small_paged", "decode_paged_fp8"):
        # blocks of 16, shuffled (decode_paged_fp8: an fp8 cache, per-tensor scales)
        kw = {}
        src = case.to("cpu")
        if workload == "decode_paged_fp8":
            k8, v8, ks, vs, _ = testing.fp8_kv(src)
            src = testing.replace(src, k=k8, v=v8)
            kw = {"k_scale": ks, "v_scale": vs}
        pk = testing.paginate(src, block_size=16, seed=0, spare_blocks=0,
                              fill=0.0).to(case.q.device)
        return lambda: inkling_fa4_rel_attention_decode_paged(
            case.q, pk.k_cache, pk.v_cache, case.rel, case.cu_q, pk.seqused_k, pk.block_table,
            case.max_q, case.max_k, case.rel_extent, causal=case.causal,
            window_size=case.window_size, softmax_scale=case.scale, return_lse=return_lse, **kw)
    if workload in ("decode_fp8", "decode_small_fp8"):  # fp8 cache, per-tensor scales
        k8, v8, ks, vs, _ = testing.fp8_kv(case)
        args = (args[0], k8, v8) + args[3:]
        kw = {"k_scale": ks, "v_scale": vs}
    if workload == "decode_br1024":
        kw = {"bottom_right": True}
    return lambda: fn(*args, causal=case.causal, window_size=case.window_size,
                      softmax_scale=case.scale, return_lse=return_lse, **kw)


def cmd_measure(args):
    """Child process: small-case output to args.check_out, then the timing (JSON)."""
    import torch

    small, big = (c.to("cuda") for c in _case(args.workload, args.seq, args.batch, args.heads))
    if args.check_out:  # skipped under counters: only the timed workload's dispatches count
        out, lse = _call(args.workload, small, True)()
        torch.save({"out": out.cpu(), "lse": lse.cpu()}, args.check_out)
    fn = _call(args.workload, big, False)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < args.settle:  # settle the clocks
        for _ in range(8):
            fn()
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(args.steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    print(json.dumps({"ms": a.elapsed_time(b) / args.steps}))
    return 0


def _prefill_args(c, out, rel_dtype):
    """ifa4_args of a prefill call on case `c` (device tensors) writing `out`."""
    from inkling_fa4 import _abi

    q, k, v, rel = c.q, c.k, c.v, c.rel
    return _abi.make_args(
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), rel=rel.data_ptr(), out=out.data_ptr(),
        cu_seqlens_q=c.cu_q.data_ptr(), cu_seqlens_k=c.cu_k.data_ptr(), q_stride_t=q.stride(0),
        q_stride_h=q.stride(1), k_stride_t=k.stride(0), k_stride_h=k.stride(1),
        v_stride_t=v.stride(0), v_stride_h=v.stride(1), rel_stride_t=rel.stride(0),
        rel_stride_h=rel.stride(1), out_stride_t=out.stride(0), out_stride_h=out.stride(1),
        total_q=q.shape[0], total_k=k.shape[0], batch=c.cu_q.numel() - 1, n_heads=q.shape[1],
        kv_heads=k.shape[1], head_dim=q.shape[2], rel_extent=c.rel_extent,
        rel_width=rel.shape[2], max_seqlen_q=c.max_q, max_seqlen_k=c.max_k,
        causal=int(c.causal), softmax_scale=c.scale, qkv_dtype=_abi.IFA4_BF16,
        rel_dtype=rel_dtype)


def cmd_split(args):
    """Split-KV prefill against the unsplit kernel on the same inputs, through
    the C ABI: ifa4_prefill_fwd (never splits) vs ifa4_prefill_fwd_ws with the
    workspace the tile table asks for (splits when it decides to).  Shapes:
    the reference benchmark's (batch 1, Hq = Hkv = 4, per-token bf16 bias of
    extent 1024) and the headline's (batch 8, Hq 8 / Hkv 2, shared table)."""
    import ctypes

    import torch
    from inkling_fa4 import _abi, testing

    lib = _abi.lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rows = ["| shape | seq | workspace MiB | unsplit ms | split ms |", "|---|---|---|---|---|"]
    for shape in args.shapes.split(","):
        for seq in (int(x) for x in args.seqs.split(",")):
            if shape == "reference":
                case = testing.make_case("reference_config", [seq], [seq], 4, 4, 128,
                                         torch.bfloat16, seed=7, rel_extent=1024,
                                         rel_table=False, rel_dtype=torch.bfloat16, rel_std=1.0)
                rd = _abi.IFA4_BF16
            else:
                case = testing.long_prefill(seq, batch=8)
                rd = _abi.IFA4_FP32
            c = case.to("cuda")
            out = torch.empty_like(c.q)
            a = _prefill_args(c, out, rd)
            n = lib.ifa4_prefill_workspace_bytes(ctypes.byref(a))
            ws = torch.empty(max(n, 256), dtype=torch.uint8, device="cuda")
            times = []
            for fn in (lambda: lib.ifa4_prefill_fwd(ctypes.byref(a), stream),
                       lambda: lib.ifa4_prefill_fwd_ws(ctypes.byref(a),
                                                       ctypes.c_void_p(ws.data_ptr()), n,
                                                       stream)):
                t0 = time.perf_counter()
                while time.perf_counter() - t0 < args.settle:
                    for _ in range(8):
                        fn()
                    torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(args.steps):
                    fn()
                e1.record()
                torch.cuda.synchronize()
                times.append(e0.elapsed_time(e1) / args.steps)
            rows.append(f"| {shape} | {seq} | {n / 2**20:.1f} | {times[0]:.4f} | {times[1]:.4f} |")
            print(rows[-1], flush=True)
    if args.out:
        with open(args.out, "w") as f:
            f.write("\n".join(rows) + "\n")
    return 0


def _counters(db, kernel_prefix):
    con = sqlite3.connect(db)
    rows = con.execute("select kernel_name, counter_name, avg(value) from counters_collection "
                       "group by kernel_name, counter_name")
    return {cn: v for k, cn, v in rows if kernel_prefix in k}


def cmd_run(args):
    import torch

    variants = [("in-tree", None, {})]
    sources = set()
    for name in sorted(os.listdir(args.dir)):
        d = os.path.join(args.dir, name)
        if os.path.exists(os.path.join(d, "knobs.json")):
            with open(os.path.join(d, "knobs.json")) as f:
                variants.append((name, d, json.load(f)))
            src = os.path.join(d, "source.txt")
            sources.add(open(src).read().strip() if os.path.exists(src) else "?")
    if len(sources) > 1:
        print(f"warning: variants were built from different sources {sorted(sources)}",
              file=sys.stderr, flush=True)
    kernel = "decode_stream_kernel" if args.workload.startswith("decode") else "prefill_fwd_kernel"
    rows, ref = [], None
    with tempfile.TemporaryDirectory() as tmp:
        for name, d, knobs in variants:
            env = dict(os.environ)
            env.pop("IFA4_LIB_DIR", None)
            if d is not None:
                env["IFA4_LIB_DIR"] = os.path.abspath(d)
            check = os.path.join(tmp, f"{name}.pt")
            child = [sys.executable, "-m", "inkling_fa4.sweep", "measure", "--workload",
                     args.workload, "--seq", str(args.seq), "--batch", str(args.batch),
                     "--heads", str(args.heads), "--steps", str(args.steps),
                     "--warmup", str(args.warmup), "--settle", str(args.settle),
                     "--check-out", check]
            res = subprocess.run(child, env=env, cwd=_PKG_ROOT, capture_output=True, text=True,
                                 timeout=args.timeout)
            if res.returncode != 0:
                rows.append((name, knobs, None, "failed to run", {}))
                print(f"{name}: failed\n{res.stderr[-2000:]}", file=sys.stderr, flush=True)
                continue
            got = torch.load(check, weights_only=True)
            verdict = "reference"
            if ref is None:
                ref = got
            else:
                ok = (torch.allclose(got["out"].float(), ref["out"].float(), atol=2e-2, rtol=2e-2)
                      and torch.allclose(got["lse"], ref["lse"], atol=1e-3, rtol=0))
                verdict = "agrees" if ok else "DIFFERS (not timed)"
                if not ok:
                    rows.append((name, knobs, None, verdict, {}))
                    continue
            ms = json.loads(res.stdout.strip().splitlines()[-1])["ms"]
            cnt = {}
            if args.counters:
                pmc_dir = os.path.join(tmp, f"pmc_{name}")
                # counters on a short run: every dispatch is serialised under --pmc
                short = child[:child.index("--steps")] + [
                    "--steps", "3", "--warmup", "1", "--settle", "0", "--check-out", ""]
                prof = ["rocprofv3", "--pmc"] + args.counters.split(",") + \
                       ["-d", pmc_dir, "-o", "run", "--"] + short
                pr = subprocess.run(prof, env=env, cwd=_PKG_ROOT, capture_output=True, text=True,
                                    timeout=args.timeout)
                db = os.path.join(pmc_dir, "run_results.db")
                if pr.returncode == 0 and os.path.exists(db):
                    cnt = _counters(db, kernel)
            rows.append((name, knobs, ms, verdict, cnt))
            print(f"{name}: {ms:.4f} ms {verdict} {cnt}", flush=True)
    names = sorted({c for r in rows for c in r[4]})
    lines = [f"| variant | knobs | ms | check | " + " | ".join(names) + " |",
             "|---|---|---|---|" + "---|" * len(names)]
    for name, knobs, ms, verdict, cnt in rows:
        ms_s = f"{ms:.4f}" if ms is not None else "—"
        lines.append(f"| {name} | {json.dumps(knobs)} | {ms_s} | {verdict} | " +
                     " | ".join(f"{cnt[c]:.4g}" if c in cnt else "—" for c in names) + " |")
    table = "\n".join(lines)
    print(table)
    if args.out:
        with open(args.out, "w") as f:
            f.write(table + "\n")
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m inkling_fa4.sweep")
    sub = ap.add_subparsers(dest="cmd", required=True)
    b = sub.add_parser("build")
    b.add_argument("--dir", required=True)
    b.add_argument("--grid", action="append", required=True, help="NAME=v1,v2,...")
    b.add_argument("--jobs", type=int, default=4)
    for name in ("run", "measure"):
        r = sub.add_parser(name)
        r.add_argument("--workload", choices=["prefill", "prefill_reference", "prefill_token",
                                              "prefill_token1024", "prefill_table1024",
                                              "rproj128", "rproj512", "rproj1024", "decode",
                                              "decode_small", "decode_small_fp8",
                                              "decode_small_paged", "decode_fp8",
                                              "decode_paged", "decode_br1024",
                                              "decode_paged_fp8"],
                       default="prefill")
        r.add_argument("--seq", type=int, default=4096)
        r.add_argument("--batch", type=int, default=1,
                       help="prefill_reference / decode_small*: sequences of --seq tokens")
        r.add_argument("--heads", type=int, default=4, help="prefill_reference: Hq = Hkv")
        r.add_argument("--steps", type=int, default=30)
        r.add_argument("--warmup", type=int, default=5)
        r.add_argument("--settle", type=float, default=0.5, help="seconds of untimed calls first")
        if name == "run":
            r.add_argument("--dir", required=True)
            r.add_argument("--counters", default="")
            r.add_argument("--out", default="")
            r.add_argument("--timeout", type=int, default=300)
        else:
            r.add_argument("--check-out", default="",
                           help="file for the small-case output ('' = no check case)")
    sp = sub.add_parser("split")
    sp.add_argument("--shapes", default="reference,headline")
    sp.add_argument("--seqs", default="1024,2048,4096,8192")
    sp.add_argument("--steps", type=int, default=30)
    sp.add_argument("--settle", type=float, default=0.3)
    sp.add_argument("--out", default="")
    args = ap.parse_args(argv)
    return {"build": cmd_build, "run": cmd_run, "measure": cmd_measure,
            "split": cmd_split}[args.cmd](args)


if __name__ == "__main__":
    sys.exit(main())
