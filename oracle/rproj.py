"""Fused relative-logit projection (test oracle).

The serving backend computes the bias from low-rank factors
(outputs/architecture.md:24,52-54, RelLogitsProj: einsum(thd,de->the, r, W),
16 -> rel_extent) and hands the materialised rel_logits to the attention
kernel, whose semantics the reference oracle fixes
(src/inkling_fa4/reference.py:19-40).  Restated here: materialise with an fp32
einsum, then the oracle.  No kernel counterpart in the reference.

TEST INFRASTRUCTURE: imported only by tests.
Pinned by tests/test_oracle_rproj.py: the einsum against an explicit loop on a
tiny shape (index order r[t,h,c] * W[c,d]), and a rank-one W that reproduces a
given per-head table.
"""
import torch

from .reference import ref_rel_attn_with_lse


def rel_logits_from_proj(r, w):
    """[Tq, Hq, d] x [d, R'] -> [Tq, Hq, R'] fp32."""
    return torch.einsum("thc,cd->thd", r.float(), w.float())


@torch.no_grad()
def ref_rel_attn_rproj_with_lse(q, k, v, r, w, cu_seqlens_q, cu_seqlens_k, scale, rel_extent,
                                causal=True, window_left=None, bottom_right=False):
    return ref_rel_attn_with_lse(q, k, v, rel_logits_from_proj(r, w), cu_seqlens_q, cu_seqlens_k,
                                 scale, rel_extent, causal=causal, window_left=window_left,
                                 bottom_right=bottom_right)
