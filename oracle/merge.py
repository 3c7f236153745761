"""Closed-form merge of attention partials by log-sum-exp (test oracle).

No reference counterpart: the reference decode kernel
(src/inkling_fa4/triton_kernel_decode.py:66-118) walks the whole KV range
in one program.  A split-KV decode computes, for disjoint key ranges S_1..S_n
of one query row,

    lse_s = log sum_{j in S_s} exp(x_j),   o_s = sum_{j in S_s} e^{x_j - lse_s} v_j

and the exact full-range result is

    lse = log sum_s exp(lse_s),            o = sum_s e^{lse_s - lse} o_s .

An empty split has lse_s = -inf and contributes nothing.

TEST INFRASTRUCTURE ONLY.
"""
import math

import torch


def merge_partials(o_parts, lse_parts):
    """o_parts [n, ..., D] fp32 (normalised per split), lse_parts [n, ...].

    Returns (o [..., D], lse [...]).  All-empty rows give o = 0, lse = -inf.
    """
    lse_parts = lse_parts.float()
    m = lse_parts.max(dim=0).values
    m_safe = torch.where(torch.isinf(m), torch.zeros_like(m), m)
    w = torch.exp(lse_parts - m_safe.unsqueeze(0))
    total = w.sum(dim=0)
    lse = torch.where(total > 0, m_safe + torch.log(total), torch.full_like(m, -math.inf))
    coef = torch.where(total.unsqueeze(0) > 0, w / total.clamp_min(1e-38).unsqueeze(0),
                       torch.zeros_like(w))
    o = (coef.unsqueeze(-1) * o_parts.float()).sum(dim=0)
    return o, lse
