"""Inkling relative-position-bias flash attention, MI355X (gfx950) native.

Same export names as the reference package (src/inkling_fa4/__init__.py:1-11),
minus `ref_rel_attn`: the fp32 oracle is test infrastructure and lives in the
repository's `oracle/` package, outside the product.  Added: the paged-KV
decode entry point `inkling_fa4_rel_attention_decode_paged` and the fused
relative-logit projection `inkling_fa4_rel_attention_rproj`.
"""
from . import autotune_configs
from .ops import (
    inkling_fa4_rel_attention,
    inkling_fa4_rel_attention_decode,
    inkling_fa4_rel_attention_decode_paged,
    inkling_fa4_rel_attention_decode_triton,
    inkling_fa4_rel_attention_kv_pruned_triton,
    inkling_fa4_rel_attention_rproj,
    inkling_fa4_rel_attention_triton,
    prefill_tile_counts,
)

__all__ = [
    "inkling_fa4_rel_attention",
    "inkling_fa4_rel_attention_decode",
    "inkling_fa4_rel_attention_decode_paged",
    "inkling_fa4_rel_attention_triton",
    "inkling_fa4_rel_attention_decode_triton",
    "inkling_fa4_rel_attention_kv_pruned_triton",
    "inkling_fa4_rel_attention_rproj",
    "prefill_tile_counts",
    "autotune_configs",
]
