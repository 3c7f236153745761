"""GPU parity of the bottom-right alignment flag (upstream flash-attn
convention, outputs/architecture.md:72) against the oracle's bottom-right mode.

Prefill, decode (contiguous and paged).  With bottom-right alignment the bias is
alive in chunked prefill and in decode (the last rel_extent keys), which the
reference alignment never exercises.  out within atol / rtol 2e-2, lse within
1e-3; rows that see no key give out 0 and lse -inf (the oracle gives NaN).
"""
import pytest
import torch

from inkling_fa4 import (inkling_fa4_rel_attention, inkling_fa4_rel_attention_decode,
                         inkling_fa4_rel_attention_decode_paged, testing)
from inkling_fa4._abi import IFA4_FLAG_NO_PRUNE
from oracle import ref_rel_attn_paged_with_lse, ref_rel_attn_with_lse

pytestmark = pytest.mark.gpu

ATOL, RTOL, LSE_ATOL = 2e-2, 2e-2, 1e-3


def _prefill(case, dev, **kw):
    c = case.to(dev)
    print(f"bottom-right prefill {case.name}: lq {case.cu_q.diff().tolist()} "
          f"lk {case.cu_k.diff().tolist()}", flush=True)
    out, lse = inkling_fa4_rel_attention(*c.args(), causal=c.causal, window_size=c.window_size,
                                         softmax_scale=c.scale, return_lse=True, **kw)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


def _oracle(case, bottom_right=True):
    return ref_rel_attn_with_lse(case.q, case.k, case.v, case.rel, case.cu_q, case.cu_k,
                                 case.scale, case.rel_extent, causal=case.causal,
                                 window_left=case.window_or_none, bottom_right=bottom_right)


def _check(got, want):
    out, lse = got
    want_out, want_lse = want
    empty = torch.isnan(want_out.float()).any(-1)  # [Tq, Hq]: rows that see no key
    assert (out.float()[empty] == 0).all()
    assert torch.isneginf(lse.transpose(0, 1)[empty]).all()
    keep = ~empty
    torch.testing.assert_close(out.float()[keep], want_out.float()[keep], atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(lse.transpose(0, 1)[keep], want_lse.transpose(0, 1)[keep],
                               atol=LSE_ATOL, rtol=0)


def test_chunked_prefill_bias_alive(cuda):
    """128 new tokens over a 384-key cache, window 63: bottom-right rows see
    keys 256 + i - 63 .. 256 + i, all inside the bias band."""
    case = testing.window_chunked(batch=4)
    got = _prefill(case, cuda, bottom_right=True)
    want = _oracle(case)
    _check(got, want)
    assert not torch.allclose(want[1], _oracle(case, bottom_right=False)[1])


@pytest.mark.parametrize("causal,window", [(True, None), (True, 40), (False, 100), (False, None)])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_ragged_lq_below_and_above_lk(cuda, causal, window, head_dim):
    case = testing.make_case("br_ragged", [100, 300, 64, 7, 250], [400, 120, 64, 900, 250], 8, 2,
                             head_dim, torch.bfloat16, seed=21, causal=causal,
                             window_left=-1 if window is None else window, rel_table=False)
    _check(_prefill(case, cuda, bottom_right=True), _oracle(case))


def test_fp16_stride0_table(cuda):
    case = testing.make_case("br_fp16", [200, 33], [500, 33], 8, 2, 128, torch.float16, seed=22,
                             causal=True)
    _check(_prefill(case, cuda, bottom_right=True), _oracle(case))


def test_equal_lengths_flag_is_bit_identical(cuda):
    case = testing.ragged_varlen()
    a = _prefill(case, cuda)
    b = _prefill(case, cuda, bottom_right=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_pruning_is_bit_invariant_bottom_right(cuda):
    case = testing.make_case("br_prune", [300, 700], [900, 500], 8, 2, 128, torch.bfloat16,
                             seed=23, causal=True, window_left=150)
    a = _prefill(case, cuda, bottom_right=True)
    b = _prefill(case, cuda, bottom_right=True, _flags=IFA4_FLAG_NO_PRUNE)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def _decode(case, dev):
    c = case.to(dev)
    print(f"bottom-right decode {case.name}: batch {c.cu_q.numel() - 1}, causal {c.causal}, "
          f"window {c.window_left}", flush=True)
    out, lse = inkling_fa4_rel_attention_decode(*c.args(), causal=c.causal,
                                                window_size=c.window_size, softmax_scale=c.scale,
                                                return_lse=True, bottom_right=True)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


@pytest.mark.parametrize("causal,window", [(True, None), (False, None), (True, 100), (True, 0),
                                           (False, 37)])
def test_decode_bottom_right(cuda, causal, window):
    """Decode sees every key (causal), the last window_left + 1 keys (window),
    and the bias of the last rel_extent keys."""
    lens = [1, 2, 31, 32, 33, 100, 128, 129, 1000, 5000]
    case = testing.make_case("br_dec", [1] * len(lens), lens, 8, 2, 128, torch.bfloat16,
                             seed=24, causal=causal, window_left=-1 if window is None else window,
                             rel_table=False, rel_std=1.0)
    _check(_decode(case, cuda), _oracle(case))


def test_decode_bottom_right_batch64(cuda):
    case = testing.decode(batch=64, causal=True)
    _check(_decode(case, cuda), _oracle(case))


@pytest.mark.parametrize("window", [None, 45])
def test_paged_decode_bottom_right(cuda, window):
    lens = [5, 40, 300, 2049]
    case = testing.make_case("br_paged", [1] * len(lens), lens, 8, 2, 128, torch.bfloat16,
                             seed=25, causal=True, window_left=-1 if window is None else window,
                             rel_table=False)
    pk = testing.paginate(case, block_size=16, seed=7)
    c, p = case.to(cuda), pk.to(cuda)
    out, lse = inkling_fa4_rel_attention_decode_paged(
        c.q, p.k_cache, p.v_cache, c.rel, c.cu_q, p.seqused_k, p.block_table, c.max_q, c.max_k,
        c.rel_extent, causal=True, window_size=c.window_size, softmax_scale=c.scale,
        return_lse=True, bottom_right=True)
    torch.cuda.synchronize()
    want = ref_rel_attn_paged_with_lse(case.q, pk.k_cache, pk.v_cache, case.rel, case.cu_q,
                                       pk.seqused_k, pk.block_table, case.scale, case.rel_extent,
                                       causal=True, window_left=case.window_or_none,
                                       bottom_right=True)
    _check((out.cpu(), lse.cpu()), want)
    contiguous = _decode(case, cuda)  # same keys; the split merge may differ in order
    torch.testing.assert_close(out.cpu().float(), contiguous[0].float(), atol=1e-3, rtol=1e-2)
    torch.testing.assert_close(lse.cpu(), contiguous[1], atol=1e-5, rtol=0)
