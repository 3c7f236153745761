"""Golden vectors of the reference oracle (see make_golden.py) and their loader."""
import glob
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _tensor(arr, tag):
    if tag == "bf16":
        return torch.from_numpy(arr.view(np.int16).copy()).view(torch.bfloat16)
    t = torch.from_numpy(arr.copy())
    return t.to(torch.float16) if tag == "f16" else t.to(torch.float32)


def names():
    return sorted(os.path.splitext(os.path.basename(p))[0]
                  for p in glob.glob(os.path.join(HERE, "*.npz")))


def load(name):
    """Return a dict with tensors q, k, v, rel, out, cu_seqlens_q/k and scalars."""
    z = np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False)
    d = {}
    for key in ("q", "k", "v", "out"):
        d[key] = _tensor(z[key], str(z[key + "_dtype"]))
    rel_tag = str(z["rel_dtype"])
    if "rel_table" in z.files:
        table = _tensor(z["rel_table"], rel_tag)
        n = int(z["rel_tokens"])
        d["rel"] = table.unsqueeze(0).expand(n, *table.shape)
    else:
        d["rel"] = _tensor(z["rel"], rel_tag)
    d["cu_seqlens_q"] = torch.from_numpy(z["cu_seqlens_q"].copy())
    d["cu_seqlens_k"] = torch.from_numpy(z["cu_seqlens_k"].copy())
    d["scale"] = float(z["scale"])
    d["rel_extent"] = int(z["rel_extent"])
    d["causal"] = bool(z["causal"])
    wl = int(z["window_left"])
    d["window_left"] = None if wl < 0 else wl
    d["name"] = name
    return d
