"""Loader of the torch binding (_ifa4_torch.so -> torch.ops.inkling_fa4).

There is no fallback: if the binding or libifa4.so is missing, or the tensors
are not on a GPU, the operators raise.
"""
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
# IFA4_LIB_DIR: load the native pair (_ifa4_torch.so, libifa4.so) from another
# directory, e.g. one variant build of a tile sweep (inkling_fa4.sweep).
LIB_DIR = os.environ.get("IFA4_LIB_DIR", _HERE)
EXT_PATH = os.path.join(LIB_DIR, "_ifa4_torch.so")
_loaded = False


def ops():
    """Return torch.ops.inkling_fa4, loading the binding on first use."""
    global _loaded
    if not _loaded:
        if not os.path.exists(EXT_PATH):
            raise ImportError(
                f"{EXT_PATH} is missing; build it with "
                "`python inkling-fa4-relative-attention_amd/build.py`")
        torch.ops.load_library(EXT_PATH)
        _loaded = True
    return torch.ops.inkling_fa4


def loaded_paths():
    """Native libraries this module loads (for provenance checks)."""
    return [EXT_PATH, os.path.join(LIB_DIR, "libifa4.so")]
