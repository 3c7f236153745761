"""Tile presets, gfx950 edition.

Same public surface as src/inkling_fa4/autotune_configs.py:17-85 (`PRESETS`,
`_detect_arch`, `get_preset`) so callers that print or pass presets keep
working.  On MI355X the tile shape is a property of the compiled HIP kernel;
the values are read from the library's tile table (ifa4_prefill_tile), and
`num_warps` counts 64-wide wavefronts.  The reference's sm86/sm90/sm100 rows
are not carried over: they tune Triton kernels that do not exist here.
"""
import functools

from . import _abi


@functools.lru_cache(maxsize=None)
def _gfx950_row(head_dim=128):
    t = _abi.prefill_tile(head_dim)
    return (t.block_q, t.block_k, t.waves, t.stages)


# Sequence lengths the shape was swept at (causal batch 8, Hq 8 / Hkv 2, d 128;
# timing plus SQ_VALU_MFMA_BUSY_CYCLES / GRBM_GUI_ACTIVE per variant): the same
# shape (64-key tiles, 4 waves x 32 rows) was fastest at each of them, so every
# bucket holds it; what changes with the length and the grid is the KV split
# (get_preset's KV_CHUNK).
SWEPT_SEQ_LENS = (1024, 2048, 4096, 8192)


def __getattr__(name):
    # PRESETS is built on first access (it queries libifa4.so), in the
    # reference's layout: (threshold, BLOCK_Q, BLOCK_K, num_warps, num_stages)
    # buckets, the last used above the largest threshold.
    if name == "PRESETS":
        bq, bk, w, st = _gfx950_row(128)
        return {"gfx950": {"default": (bq, bk, w, st),
                           "buckets": [(s, bq, bk, w, st) for s in SWEPT_SEQ_LENS]}}
    raise AttributeError(name)


def _detect_arch() -> str:
    """'gfx950' on MI355X; the GCN arch name of another AMD GPU; 'gfx950' when
    no GPU is visible (the library is built for gfx950 only)."""
    import torch

    if not torch.cuda.is_available():
        return "gfx950"
    name = getattr(torch.cuda.get_device_properties(0), "gcnArchName", "gfx950")
    return name.split(":")[0]


def get_preset(seq_len: int, arch: str | None = None, head_dim: int = 128, batch: int = 1,
               n_heads: int = 4, causal: bool = True) -> dict:
    """Tile config used for `seq_len` query tokens: BLOCK_Q, BLOCK_K,
    num_warps (wavefronts) and num_stages (LDS buffers), plus KV_CHUNK, the
    keys per KV chunk when the table splits a causal call of `batch` sequences
    over `n_heads` heads at that length (0: no split; the defaults are the
    reference benchmark's batch 1, 4 heads).  The shape is the same at every
    length (sequence-length buckets were swept and one shape won each); the
    split is what changes with the length and the grid.  `arch` is accepted
    for signature compatibility; every arch maps to the gfx950 table."""
    del arch
    t = _abi.prefill_tile(head_dim, batch=batch, n_heads=n_heads, seq_len=seq_len,
                          causal=causal)
    return {"BLOCK_Q": t.block_q, "BLOCK_K": t.block_k, "num_warps": t.waves,
            "num_stages": t.stages, "KV_CHUNK": t.kv_chunk}
