"""Paged KV cache -> contiguous varlen K/V (test oracle).

The reference kernels take contiguous varlen K/V only
(src/inkling_fa4/reference.py:19-23 slices k[ks:ke] per sequence); its
serving backend keeps the cache in blocks of 16 tokens
(outputs/architecture.md:117-120).  The paged semantics restated here: key j
of sequence b is row j % block_size of block block_table[b, j // block_size];
the sequence holds seqused_k[b] keys.  A table entry outside [0, num_blocks)
stands for a block of zeros (the library's memory-safe reading of a bad entry).

The attention itself is then the contiguous oracle (reference.py restatement)
on the gathered K/V.

TEST INFRASTRUCTURE: imported only by tests.
Pinned by tests/test_oracle_paged.py: identity tables reproduce the
contiguous cache; permuting the physical blocks (and the table with them) and
changing the block size leave the gather unchanged; rows outside a sequence
never reach it.
"""
import torch

from .reference import ref_rel_attn_with_lse


@torch.no_grad()
def gather_paged(k_cache, v_cache, block_table, seqused_k):
    """Return (k [sum L, Hkv, D], v, cu_seqlens_k int32 [batch+1])."""
    n_blocks, bs = k_cache.shape[0], k_cache.shape[1]
    ks, vs, cu = [], [], [0]
    for b, n in enumerate(int(x) for x in seqused_k.tolist()):
        j = torch.arange(n)
        ent = block_table[b, (j // bs)].long()
        ok = (ent >= 0) & (ent < n_blocks)
        blk = torch.where(ok, ent, torch.zeros_like(ent))
        rows = j % bs
        kb = k_cache[blk, rows]
        vb = v_cache[blk, rows]
        zero = torch.zeros((), dtype=k_cache.dtype)
        ks.append(torch.where(ok[:, None, None], kb, zero))
        vs.append(torch.where(ok[:, None, None], vb, zero))
        cu.append(cu[-1] + n)
    return torch.cat(ks), torch.cat(vs), torch.tensor(cu, dtype=torch.int32)


@torch.no_grad()
def ref_rel_attn_paged_with_lse(q, k_cache, v_cache, rel_logits, cu_seqlens_q, seqused_k,
                                block_table, scale, rel_extent, causal=True, window_left=None,
                                bottom_right=False):
    """Oracle over a paged cache: (out [Tq,Hq,D] in q.dtype, lse [Hq,Tq] fp32)."""
    k, v, cu_k = gather_paged(k_cache, v_cache, block_table, seqused_k)
    return ref_rel_attn_with_lse(q, k, v, rel_logits, cu_seqlens_q, cu_k, scale, rel_extent,
                                 causal=causal, window_left=window_left,
                                 bottom_right=bottom_right)
