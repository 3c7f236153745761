"""Write golden input/output vectors for relative-bias attention.

Runs ONLY in the build container, where the reference checkout is mounted.
It loads `src/inkling_fa4/reference.py` of the reference by file path (so
the package `__init__`, which imports Triton, is never executed), feeds it
small seeded inputs and stores inputs + outputs as `.npz` fixtures next to
this script.  The fixtures are data; nothing of the reference travels with
them.

Why these cases: each one pins a convention of `ref_rel_attn`
(reference.py:19-40) that no closed form fixes by itself --
  * the sign of `offset = Lq - Lk` in the bias distance (reference.py:28-31),
  * top-left causal masking on local indices when Lq != Lk (reference.py:36),
  * zero (not clamped) bias outside [0, rel_extent) (reference.py:32-35),
  * a left-only window that also applies when causal=False (reference.py:37),
  * NaN rows when every key is masked (reference.py:38),
  * output rounded to q.dtype (reference.py:20,39),
  * the GQA head map h // (Hq // Hkv) (reference.py:20,26),
  * rel_logits with a last dim larger than rel_extent and a token stride of 0.

Usage:  python tests/golden/make_golden.py
"""
import importlib.util
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF_FILE = "/root/reference/src/inkling_fa4/reference.py"


def _load_reference():
    spec = importlib.util.spec_from_file_location("_ref_reference_py", REF_FILE)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.ref_rel_attn


_NP_OF = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


def _to_np(t):
    """Tensor -> (array, dtype tag); bf16 is stored as its uint16 bit pattern."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16), "bf16"
    if t.dtype == torch.float16:
        return t.numpy(), "f16"
    return t.numpy(), "f32"


def _cu(lens):
    c = [0]
    for n in lens:
        c.append(c[-1] + n)
    return torch.tensor(c, dtype=torch.int32)


def make_case(name, seed, lq, lk, hq, hkv, d, rel_extent, rel_width, dtype,
              rel_dtype, causal, window_left, scale, rel_table=False):
    g = torch.Generator().manual_seed(seed)
    tq, tk = sum(lq), sum(lk)
    q = torch.randn(tq, hq, d, generator=g).to(dtype)
    k = torch.randn(tk, hkv, d, generator=g).to(dtype)
    v = torch.randn(tk, hkv, d, generator=g).to(dtype)
    if rel_table:
        table = (0.5 * torch.randn(hq, rel_width, generator=g)).to(rel_dtype)
        rel = table.unsqueeze(0).expand(tq, hq, rel_width)
    else:
        rel = torch.randn(tq, hq, rel_width, generator=g).to(rel_dtype)
    cuq, cuk = _cu(lq), _cu(lk)
    return dict(name=name, q=q, k=k, v=v, rel=rel, cuq=cuq, cuk=cuk,
                scale=scale, rel_extent=rel_extent, causal=causal,
                window_left=window_left, rel_table=rel_table)


CASES = [
    # ragged GQA prefill, per-token bias, Lq == Lk per sequence
    dict(name="ragged_gqa", seed=1, lq=[13, 7, 20], lk=[13, 7, 20], hq=4, hkv=2,
         d=16, rel_extent=8, rel_width=8, dtype=torch.float32,
         rel_dtype=torch.float32, causal=True, window_left=None, scale=1 / 16),
    # chunked prefill: Lq < Lk, delta negative, top-left causal
    dict(name="chunked_causal", seed=2, lq=[5, 9], lk=[12, 21], hq=2, hkv=1,
         d=16, rel_extent=16, rel_width=16, dtype=torch.float32,
         rel_dtype=torch.float32, causal=True, window_left=None, scale=0.25),
    # Lq > Lk, non-causal: delta positive, bias d = i + (Lq-Lk) - j
    dict(name="lq_gt_lk_noncausal", seed=3, lq=[12], lk=[5], hq=2, hkv=2,
         d=8, rel_extent=10, rel_width=12, dtype=torch.float32,
         rel_dtype=torch.float32, causal=False, window_left=None, scale=0.3),
    # left window without causal: keys to the right stay visible
    dict(name="window_noncausal", seed=4, lq=[16], lk=[16], hq=2, hkv=1,
         d=8, rel_extent=6, rel_width=6, dtype=torch.float32,
         rel_dtype=torch.float32, causal=False, window_left=3, scale=0.35),
    # window + causal + chunked, two sequences
    dict(name="window_causal_chunked", seed=5, lq=[8, 6], lk=[20, 14], hq=4, hkv=1,
         d=16, rel_extent=12, rel_width=16, dtype=torch.float32,
         rel_dtype=torch.float32, causal=True, window_left=4, scale=1 / 16),
    # rows with no visible key -> NaN in the reference
    dict(name="empty_rows_nan", seed=6, lq=[6], lk=[3], hq=1, hkv=1,
         d=8, rel_extent=4, rel_width=4, dtype=torch.float32,
         rel_dtype=torch.float32, causal=True, window_left=1, scale=0.3),
    # bf16 inputs/outputs (output rounded to q.dtype), bf16 bias, stride-0 table
    dict(name="bf16_table", seed=7, lq=[24, 9], lk=[24, 9], hq=4, hkv=2,
         d=32, rel_extent=16, rel_width=16, dtype=torch.bfloat16,
         rel_dtype=torch.bfloat16, causal=True, window_left=None, scale=1 / 32,
         rel_table=True),
    # fp16 config of the 64-token single sequence prefill (D=64, scale 1/sqrt(64))
    dict(name="prefill_s64_fp16_d64", seed=8, lq=[64], lk=[64], hq=4, hkv=4,
         d=64, rel_extent=128, rel_width=128, dtype=torch.float16,
         rel_dtype=torch.float32, causal=True, window_left=None, scale=0.125,
         rel_table=True),
    # ragged GQA bf16 prefill, 3 sequences [64,33,17], Hq=8 Hkv=2 D=128, rel 128
    dict(name="ragged_114_bf16_d128", seed=9, lq=[64, 33, 17], lk=[64, 33, 17],
         hq=8, hkv=2, d=128, rel_extent=128, rel_width=128, dtype=torch.bfloat16,
         rel_dtype=torch.float32, causal=True, window_left=None, scale=1 / 128,
         rel_table=True),
    # decode: one query per sequence, causal and non-causal
    dict(name="decode_causal", seed=10, lq=[1, 1, 1], lk=[40, 17, 64], hq=4, hkv=2,
         d=16, rel_extent=8, rel_width=8, dtype=torch.float32,
         rel_dtype=torch.float32, causal=True, window_left=None, scale=0.25),
    dict(name="decode_noncausal", seed=11, lq=[1, 1, 1], lk=[40, 17, 64], hq=4, hkv=2,
         d=16, rel_extent=8, rel_width=8, dtype=torch.float32,
         rel_dtype=torch.float32, causal=False, window_left=None, scale=0.25),
    # decode with a short KV that keeps the bias alive (Lk < 2*Lq fails, bias at d>=0)
    dict(name="short_kv_bias_alive", seed=12, lq=[4], lk=[6], hq=2, hkv=1,
         d=8, rel_extent=8, rel_width=8, dtype=torch.float32,
         rel_dtype=torch.float32, causal=False, window_left=None, scale=0.5),
]


def main():
    ref_rel_attn = _load_reference()
    for spec in CASES:
        spec = dict(spec)
        c = make_case(**spec)
        with torch.no_grad():
            out = ref_rel_attn(c["q"], c["k"], c["v"], c["rel"], c["cuq"], c["cuk"],
                               c["scale"], c["rel_extent"], causal=c["causal"],
                               window_left=c["window_left"])
        arrs = {}
        for key in ("q", "k", "v", "out"):
            a, tag = _to_np(c[key] if key != "out" else out)
            arrs[key] = a
            arrs[key + "_dtype"] = np.array(tag)
        if c["rel_table"]:
            a, tag = _to_np(c["rel"][0])
            arrs["rel_table"] = a
            arrs["rel_tokens"] = np.array(c["q"].shape[0], dtype=np.int64)
        else:
            a, tag = _to_np(c["rel"])
            arrs["rel"] = a
        arrs["rel_dtype"] = np.array(tag)
        arrs["cu_seqlens_q"] = c["cuq"].numpy()
        arrs["cu_seqlens_k"] = c["cuk"].numpy()
        arrs["scale"] = np.array(c["scale"], dtype=np.float64)
        arrs["rel_extent"] = np.array(c["rel_extent"], dtype=np.int64)
        arrs["causal"] = np.array(bool(c["causal"]))
        arrs["window_left"] = np.array(-1 if c["window_left"] is None else c["window_left"],
                                       dtype=np.int64)
        path = os.path.join(HERE, f"{c['name']}.npz")
        np.savez_compressed(path, **arrs)
        nan_rows = int(torch.isnan(out.float()).any(dim=-1).sum())
        print(f"wrote {os.path.relpath(path)}  out{tuple(out.shape)} {out.dtype} nan_rows={nan_rows}")


if __name__ == "__main__":
    sys.exit(main())
