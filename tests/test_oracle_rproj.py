"""Pins the oracle of the fused relative-logit projection (oracle/rproj.py):
the einsum's index order against an explicit loop, and a rank-one factorisation
that must reproduce a given per-head table (so the projected bias lands on the
same distances as a materialised rel_logits)."""
import torch

from inkling_fa4 import testing
from oracle import ref_rel_attn_rproj_with_lse, ref_rel_attn_with_lse, rel_logits_from_proj


def test_einsum_index_order():
    g = torch.Generator().manual_seed(0)
    r = torch.randn(5, 3, 16, generator=g)
    w = torch.randn(16, 7, generator=g)
    got = rel_logits_from_proj(r, w)
    for t in range(5):
        for h in range(3):
            for d in range(7):
                want = sum(float(r[t, h, c]) * float(w[c, d]) for c in range(16))
                assert abs(float(got[t, h, d]) - want) < 1e-4


def test_rank_one_factorisation_reproduces_a_table():
    """r[t,h,:] = e_h (one-hot head), W[h,:] = table[h,:]: the projection gives
    rel_logits[t,h,d] = table[h,d] for every token, i.e. the stride-0 table."""
    case = testing.ragged_varlen()
    hq = case.q.shape[1]
    table = case.rel[0].float()                    # [Hq, 128]
    tq = case.q.shape[0]
    r = torch.zeros(tq, hq, 16)
    r[:, torch.arange(hq), torch.arange(hq)] = 1.0
    w = torch.zeros(16, table.shape[1])
    w[:hq] = table
    a = ref_rel_attn_rproj_with_lse(case.q, case.k, case.v, r, w, case.cu_q, case.cu_k,
                                    case.scale, case.rel_extent, causal=True)
    b = ref_rel_attn_with_lse(case.q, case.k, case.v, case.rel, case.cu_q, case.cu_k,
                              case.scale, case.rel_extent, causal=True)
    assert torch.equal(a[0], b[0]) and torch.allclose(a[1], b[1], atol=1e-6, rtol=0)
