"""Large and strongly varying logits against the fp32 oracle.

Key norms ramp along each sequence, so the scores span tens of log2 units:
ramping up, the row max grows tile after tile and the deferred rescale of O
fires many times; ramping down, the first tiles dominate and the later ones
underflow.  For decode the long sequences are split across persistent waves,
so the combine step merges partial results whose maxima lie far apart.
Tolerances are the operator's (out atol/rtol 2e-2, lse atol 1e-3).
"""
from dataclasses import replace

import pytest
import torch

from inkling_fa4 import (inkling_fa4_rel_attention, inkling_fa4_rel_attention_decode,
                         inkling_fa4_rel_attention_decode_paged, testing)
from oracle import ref_rel_attn_paged_with_lse, ref_rel_attn_with_lse

pytestmark = pytest.mark.gpu

ATOL, RTOL, LSE_ATOL = 2e-2, 2e-2, 1e-3


def _ramp_keys(case, lo, hi):
    """Key j of each sequence scaled by a factor from lo (first key) to hi (last)."""
    cu = case.cu_k.tolist()
    f = torch.ones(case.k.shape[0])
    for b in range(len(cu) - 1):
        n = cu[b + 1] - cu[b]
        if n:
            f[cu[b]:cu[b + 1]] = torch.linspace(lo, hi, n)
    return replace(case, k=(case.k.float() * f[:, None, None]).to(case.k.dtype))


def _score_span_log2(case):
    """Largest spread (log2 units) of one row's scores, first sequence, head 0."""
    lq = int(case.cu_q[1])
    lk = int(case.cu_k[1])
    q = case.q[:lq, 0].float()
    k = case.k[:lk, 0].float()
    s = (q @ k.T) * case.scale * 1.4426950408889634
    return float((s.max(1).values - s.min(1).values).max())


def _compare(out, lse, want):
    want_out, want_lse = want
    assert not torch.isnan(want_out).any()
    torch.testing.assert_close(out.cpu().float(), want_out.float(), atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(lse.cpu(), want_lse, atol=LSE_ATOL, rtol=0)


@pytest.mark.parametrize("ramp", [(0.05, 5.0), (5.0, 0.05)], ids=["up", "down"])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_ramped_keys(cuda, ramp, causal):
    case = testing.make_case("ramp", [300, 700, 129], [300, 700, 129], 8, 2, 128, torch.bfloat16,
                             seed=11, causal=causal, scale=0.3)
    case = _ramp_keys(case, *ramp)
    assert _score_span_log2(case) > 40  # several times the rescale threshold of 8
    c = case.to(cuda)
    out, lse = inkling_fa4_rel_attention(*c.args(), causal=c.causal, softmax_scale=c.scale,
                                         return_lse=True)
    torch.cuda.synchronize()
    _compare(out, lse, ref_rel_attn_with_lse(case.q, case.k, case.v, case.rel, case.cu_q,
                                             case.cu_k, case.scale, case.rel_extent,
                                             causal=case.causal))


def test_prefill_ramped_keys_large_bias_fp16_d64(cuda):
    """Large per-token bias on top of ramped keys, fp16, head_dim 64, a window."""
    case = testing.make_case("ramp_bias", [200, 450], [260, 450], 6, 3, 64, torch.float16,
                             seed=12, causal=True, window_left=150, scale=0.25, rel_table=False,
                             rel_std=4.0, rel_extent=100)
    case = _ramp_keys(case, 0.1, 4.0)
    c = case.to(cuda)
    out, lse = inkling_fa4_rel_attention(*c.args(), causal=c.causal, window_size=c.window_size,
                                         softmax_scale=c.scale, return_lse=True)
    torch.cuda.synchronize()
    _compare(out, lse, ref_rel_attn_with_lse(case.q, case.k, case.v, case.rel, case.cu_q,
                                             case.cu_k, case.scale, case.rel_extent,
                                             causal=case.causal,
                                             window_left=case.window_or_none))


@pytest.mark.parametrize("ramp", [(0.05, 5.0), (5.0, 0.05)], ids=["up", "down"])
def test_decode_ramped_keys(cuda, ramp):
    lens_k = [3000, 1500, 700, 64, 9000]
    case = testing.make_case("ramp_dec", [1] * len(lens_k), lens_k, 8, 2, 128, torch.bfloat16,
                             seed=13, causal=False, scale=0.3)
    case = _ramp_keys(case, *ramp)
    c = case.to(cuda)
    out, lse = inkling_fa4_rel_attention_decode(*c.args(), causal=False, softmax_scale=c.scale,
                                                return_lse=True)
    torch.cuda.synchronize()
    _compare(out, lse, ref_rel_attn_with_lse(case.q, case.k, case.v, case.rel, case.cu_q,
                                             case.cu_k, case.scale, case.rel_extent,
                                             causal=False))


def test_decode_paged_ramped_keys(cuda):
    lens_k = [4000, 900, 33]
    case = testing.make_case("ramp_paged", [1] * len(lens_k), lens_k, 8, 1, 128, torch.bfloat16,
                             seed=14, causal=False, scale=0.3)
    case = _ramp_keys(case, 0.05, 5.0)
    pk = testing.paginate(case, block_size=16, seed=14)
    c, p = case.to(cuda), pk.to(cuda)
    out, lse = inkling_fa4_rel_attention_decode_paged(
        c.q, p.k_cache, p.v_cache, c.rel, c.cu_q, p.seqused_k, p.block_table, c.max_q, c.max_k,
        c.rel_extent, causal=False, softmax_scale=c.scale, return_lse=True)
    torch.cuda.synchronize()
    _compare(out, lse, ref_rel_attn_paged_with_lse(case.q, pk.k_cache, pk.v_cache, case.rel,
                                                   case.cu_q, pk.seqused_k, pk.block_table,
                                                   case.scale, case.rel_extent, causal=False))
