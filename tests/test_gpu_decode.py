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


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2), (12, 4), (8, 1), (16, 1), (6, 2), (32, 1),
                                     (48, 2)])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_decode_gqa_groups_and_head_dims(cuda, hq, hkv, head_dim):
    """Groups above 16 (32, 24) run through the prefill kernel."""
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


# ---- stream-K partition: every cache laid end to end in 32-key steps, split
# evenly over min(2048, steps) persistent waves ---------------------------------------

@pytest.mark.parametrize("causal", [False, True])
def test_decode_stream_many_short_caches(cuda, causal):
    """150 sequences (three 64-sequence chunks of the device-side scan), empty and
    one-key caches mixed in: waves cross many cache boundaries, the cursor reloads
    sequence chunks, and empty caches own no steps."""
    g = torch.Generator().manual_seed(11)
    lens = torch.randint(0, 100, (150,), generator=g).tolist()
    lens[3] = 0
    lens[70] = 1
    lens[140] = 32
    case = testing.make_case("dec_short", [1] * 150, lens, 8, 2, 128, torch.bfloat16, seed=12,
                             causal=causal)
    out, lse = _decode(case, cuda)
    want = _oracle(case)
    live = torch.tensor([n > 0 for n in lens])
    torch.testing.assert_close(out[live].float(), want[0][live].float(), atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(lse[:, live], want[1][:, live], atol=LSE_ATOL, rtol=0)
    assert (out[~live].float() == 0).all() and torch.isneginf(lse[:, ~live]).all()


def test_decode_stream_one_cache_over_all_waves(cuda):
    """One 70,000-key cache per kv head: 2,188 steps each over 896 waves, so
    every wave holds a piece and the merge of a head sums ~449 partials (four
    combine workgroups per head, each over a quarter of the row)."""
    case = testing.make_case("dec_long", [1], [70000], 8, 2, 128, torch.bfloat16, seed=13,
                             causal=False)
    _check(_decode(case, cuda), _oracle(case))


@pytest.mark.parametrize("head_dim", [64, 128])
def test_decode_stream_step_boundaries(cuda, head_dim):
    """Cache lengths at and around multiples of the 32-key step, with more steps
    than waves so wave ranges start and stop inside caches."""
    lens = [31, 32, 33, 63, 64, 65, 95, 96, 97, 4096, 4097, 4127, 4128, 4129] * 5
    case = testing.make_case("dec_steps", [1] * len(lens), lens, 4, 4, head_dim, torch.bfloat16,
                             seed=14, causal=False)
    _check(_decode(case, cuda), _oracle(case))


@pytest.mark.parametrize("keys,head_dim", [(8192, 64), (8192, 128), (131072, 64), (131072, 128)])
def test_decode_one_sequence_split_combine(cuda, keys, head_dim):
    """One sequence spread over many waves: ~129 partials per (head, sequence)
    at 8K keys (256 waves), ~449 at 128K (896 waves).  The combine then splits
    each row's 16-byte chunks over 2 workgroups (8K keys, d 64) or 4 (the
    rest), each merging every partial for its slice; all splits must agree on
    the normalisation, and split 0 writes the LSE.  Reference semantics:
    src/inkling_fa4/reference.py:38-39."""
    case = testing.make_case("dec_split", [1], [keys], 8, 2, head_dim, torch.bfloat16,
                             seed=15, causal=False)
    print(f"one sequence of {keys} keys, d {head_dim}", flush=True)
    _check(_decode(case, cuda), _oracle(case))


@pytest.mark.parametrize("hq,hkv,head_dim", [(8, 2, 128), (8, 1, 64), (4, 4, 128), (16, 1, 128)])
@pytest.mark.parametrize("rel_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_decode_bottom_right_token_bias_views(cuda, rel_dtype, hq, hkv, head_dim):
    """Bottom-right decode (the query at key Lk - 1) with a per-token bias of
    extent 1024: the last 1024 keys of every cache carry bias, gathered per
    step as whole dwords from the sequence's bias row.  The bias is passed as
    a view one element into a wider buffer (a 16-bit row then starts 2 bytes
    into a dword) with an odd head stride (R' + 1), so the element's half of
    its dword alternates between heads; caches shorter and longer than the
    extent, and lengths on step and extent boundaries; GQA groups 1, 4, 8 and
    16 and d 64."""
    lens = [1, 5, 31, 300, 1023, 1024, 1025, 2049, 4000, 70]
    case = testing.make_case("dec_brbias", [1] * len(lens), lens, hq, hkv, head_dim,
                             torch.bfloat16, seed=16, causal=True, rel_extent=1024,
                             rel_table=False, rel_dtype=rel_dtype, rel_std=1.0)
    tq, hq, rw = case.rel.shape
    wide = torch.zeros(tq, hq, rw + 1, dtype=rel_dtype)
    wide[:, :, 1:] = case.rel
    c = case.to(cuda)
    rel_view = wide.to(cuda)[:, :, 1:]
    assert rel_view.stride() == (hq * (rw + 1), rw + 1, 1) and rel_view.storage_offset() == 1
    print(f"bottom-right token bias {rel_dtype}, Hq {hq} / Hkv {hkv}, d {head_dim}", flush=True)
    out, lse = inkling_fa4_rel_attention_decode(
        c.q, c.k, c.v, rel_view, c.cu_q, c.cu_k, c.max_q, c.max_k, c.rel_extent, causal=True,
        softmax_scale=c.scale, return_lse=True, bottom_right=True)
    torch.cuda.synchronize()
    want = ref_rel_attn_with_lse(case.q, case.k, case.v, case.rel, case.cu_q, case.cu_k,
                                 case.scale, case.rel_extent, causal=True, bottom_right=True)
    _check((out.cpu(), lse.cpu()), want)
