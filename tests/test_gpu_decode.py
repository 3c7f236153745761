"""GPU parity of the split-KV decode kernels against the fp32 oracle.

out within atol 2e-2 / rtol 2e-2 (bf16/fp16), lse within 1e-3 absolute.
"""
import math

import pytest
import torch

from inkling_fa4 import (inkling_fa4_rel_attention, inkling_fa4_rel_attention_decode,
                         inkling_fa4_rel_attention_decode_triton, testing)
from oracle import ref_rel_attn_with_lse

pytestmark = pytest.mark.gpu

ATOL, RTOL, LSE_ATOL = 2e-2, 2e-2, 1e-3


def _decode(case, dev, fn=inkling_fa4_rel_attention_decode):
    c = case.to(dev)
    out, lse = fn(*c.args(), causal=c.causal, window_size=c.window_size,
                  softmax_scale=c.scale, return_lse=True)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


def _oracle(case):
    return ref_rel_attn_with_lse(case.q, case.k, case.v, case.rel, case.cu_q, case.cu_k,
                                 case.scale, case.rel_extent, causal=case.causal,
                                 window_left=case.window_or_none)


def _check(got, want):
    torch.testing.assert_close(got[0].float(), want[0].float(), atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(got[1], want[1], atol=LSE_ATOL, rtol=0)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("scale", ["1/D", "1/sqrtD"])
def test_decode_batch64_full(cuda, causal, scale):
    case = testing.decode(causal=causal, scale=(1 / 128 if scale == "1/D" else 1 / math.sqrt(128)))
    _check(_decode(case, cuda), _oracle(case))


def test_decode_fp16(cuda):
    case = testing.decode(dtype=torch.float16, batch=16, seed=6)
    _check(_decode(case, cuda), _oracle(case))


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2), (12, 4), (8, 1), (16, 1), (6, 2)])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_decode_gqa_groups_and_head_dims(cuda, hq, hkv, head_dim):
    lens = [1, 2, 63, 64, 65, 200, 1000, 3000]
    case = testing.make_case("dec_gqa", [1] * len(lens), lens, hq, hkv, head_dim, torch.bfloat16,
                             seed=hq * 10 + hkv, causal=False, rel_table=False, scale=0.1)
    _check(_decode(case, cuda), _oracle(case))


def test_decode_live_bias_on_single_key(cuda):
    """Lk = 1: dist = 0 is inside the band, so the bias of distance 0 is added
    (the only decode case where the bias is alive)."""
    case = testing.make_case("dec_bias", [1, 1, 1], [1, 1, 5], 4, 2, 128, torch.bfloat16, seed=3,
                             causal=False, rel_table=False, rel_std=2.0)
    _check(_decode(case, cuda), _oracle(case))


def test_decode_window_is_inert(cuda):
    case = testing.make_case("dec_win", [1] * 4, [10, 500, 2000, 77], 8, 2, 128, torch.bfloat16,
                             seed=4, causal=False, window_left=5)
    _check(_decode(case, cuda), _oracle(case))


def test_decode_matches_prefill_kernel(cuda):
    """The two kernels agree on the same single-query batch."""
    case = testing.decode(batch=12, seed=9)
    a = _decode(case, cuda)
    b = _decode(case, cuda, fn=inkling_fa4_rel_attention)
    torch.testing.assert_close(a[0].float(), b[0].float(), atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(a[1], b[1], atol=1e-4, rtol=0)


def test_decode_alias_falls_back_to_prefill_for_multi_token_queries(cuda):
    case = testing.make_case("dec_multi", [3, 2], [40, 50], 8, 2, 128, torch.bfloat16, seed=5)
    got = _decode(case, cuda, fn=inkling_fa4_rel_attention_decode_triton)
    _check(got, _oracle(case))


def test_decode_empty_kv_rows(cuda):
    """A sequence with no keys gives out = 0 and lse = -inf."""
    case = testing.make_case("dec_empty", [1, 1], [0, 30], 4, 4, 128, torch.bfloat16, seed=6,
                             causal=False)
    out, lse = _decode(case, cuda)
    assert (out[0].float() == 0).all()
    assert torch.isneginf(lse[:, 0]).all()
    want = _oracle(case)
    torch.testing.assert_close(out[1].float(), want[0][1].float(), atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(lse[:, 1], want[1][:, 1], atol=LSE_ATOL, rtol=0)
