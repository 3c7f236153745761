"""GPU parity of decode over a paged KV cache (block tables).

Two bars: against the fp32 oracle over the gathered cache (out within atol /
rtol 2e-2, lse within 1e-3), and agreement with the contiguous decode kernel on
the same keys up to the order of the split merge (lse within 1e-5).
Every pool holds NaN in the rows no sequence owns and garbage table entries
past each sequence's blocks, so a read outside a sequence shows up as NaN.
"""
import pytest
import torch

from inkling_fa4 import (inkling_fa4_rel_attention_decode, inkling_fa4_rel_attention_decode_paged,
                         testing)
from oracle import ref_rel_attn_paged_with_lse

pytestmark = pytest.mark.gpu

ATOL, RTOL, LSE_ATOL = 2e-2, 2e-2, 1e-3


def _paged(case, pk, dev, max_k=None):
    c, p = case.to(dev), pk.to(dev)
    print(f"paged decode: batch {c.cu_q.numel() - 1}, block {pk.k_cache.shape[1]}, "
          f"heads {c.q.shape[1]}/{c.k.shape[1]}, D {c.q.shape[2]}, causal {c.causal}", flush=True)
    out, lse = inkling_fa4_rel_attention_decode_paged(
        c.q, p.k_cache, p.v_cache, c.rel, c.cu_q, p.seqused_k, p.block_table, c.max_q,
        c.max_k if max_k is None else max_k, c.rel_extent, causal=c.causal,
        window_size=c.window_size, softmax_scale=c.scale, return_lse=True)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


def _contiguous(case, dev):
    c = case.to(dev)
    out, lse = inkling_fa4_rel_attention_decode(*c.args(), causal=c.causal,
                                                window_size=c.window_size, softmax_scale=c.scale,
                                                return_lse=True)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


def _oracle(case, pk):
    return ref_rel_attn_paged_with_lse(case.q, pk.k_cache, pk.v_cache, case.rel, case.cu_q,
                                       pk.seqused_k, pk.block_table, case.scale, case.rel_extent,
                                       causal=case.causal, window_left=case.window_or_none)


def _check(got, want):
    torch.testing.assert_close(got[0].float(), want[0].float(), atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(got[1], want[1], atol=LSE_ATOL, rtol=0)


def _same(a, b):
    """Paged and contiguous decode read the same keys with the same per-step
    arithmetic; only the stream-K split differs (a paged cache streams with more
    waves), so results agree up to the order of the split merge: lse within
    1e-5, out within one 16-bit rounding step."""
    torch.testing.assert_close(a[0].float(), b[0].float(), atol=1e-3, rtol=1e-2)
    torch.testing.assert_close(a[1], b[1], atol=1e-5, rtol=0)


@pytest.mark.parametrize("block_size", [16, 8, 32, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_paged_decode_batch(cuda, block_size, causal):
    case = testing.decode(batch=24, seed=31, causal=causal, lo=1, hi=5000)
    pk = testing.paginate(case, block_size=block_size, seed=block_size)
    got = _paged(case, pk, cuda)
    _check(got, _oracle(case, pk))
    _same(got, _contiguous(case, cuda))


@pytest.mark.parametrize("hq,hkv", [(8, 2), (4, 4), (16, 1), (6, 2)])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_paged_gqa_and_head_dims(cuda, hq, hkv, head_dim):
    lens = [1, 7, 8, 16, 17, 31, 32, 33, 300, 1500]
    case = testing.make_case("paged_gqa", [1] * len(lens), lens, hq, hkv, head_dim,
                             torch.bfloat16, seed=hq + hkv, causal=False, rel_table=False,
                             scale=0.1)
    pk = testing.paginate(case, block_size=16, seed=head_dim)
    got = _paged(case, pk, cuda)
    _check(got, _oracle(case, pk))
    _same(got, _contiguous(case, cuda))


def test_paged_fp16_and_empty_sequences(cuda):
    lens = [0, 100, 0, 2049, 1]
    case = testing.make_case("paged_fp16", [1] * len(lens), lens, 8, 2, 128, torch.float16,
                             seed=5, causal=False)
    pk = testing.paginate(case, block_size=16, seed=1)
    got = _paged(case, pk, cuda)
    _same(got, _contiguous(case, cuda))
    assert torch.equal(got[0][[0, 2]], torch.zeros_like(got[0][[0, 2]]))
    assert torch.isneginf(got[1][:, [0, 2]]).all()
    live = [1, 3, 4]
    want = _oracle(case, pk)
    _check((got[0][live], got[1][:, live]), (want[0][live], want[1][:, live]))


def test_paged_many_sequences_and_wide_table(cuda):
    """150 sequences (three 64-sequence chunks of the device-side scan), a
    table slice wider than needed (row stride > row length)."""
    g, lens = testing.decode_lengths(batch=150, seed=40, lo=1, hi=900)
    case = testing.make_case("paged_many", [1] * 150, lens, 8, 2, 128, torch.bfloat16, seed=40,
                             causal=False, gen=g)
    pk = testing.paginate(case, block_size=16, seed=2, extra_columns=9)
    wide = torch.full((150, pk.block_table.shape[1] + 11), 1 << 30, dtype=torch.int32)
    wide[:, 3:3 + pk.block_table.shape[1]] = pk.block_table
    pk.block_table = wide[:, 3:3 + pk.block_table.shape[1]]  # stride(0) > size(1)
    assert pk.block_table.stride(0) > pk.block_table.shape[1]
    got = _paged(case, pk, cuda)
    _check(got, _oracle(case, pk))
    _same(got, _contiguous(case, cuda))


def test_paged_one_long_sequence(cuda):
    """One 70000-key cache (windows of 64 table entries are refilled 68 times)."""
    case = testing.make_case("paged_long", [1], [70000], 8, 2, 128, torch.bfloat16, seed=8,
                             causal=False)
    pk = testing.paginate(case, block_size=16, seed=3)
    got = _paged(case, pk, cuda)
    _check(got, _oracle(case, pk))
    _same(got, _contiguous(case, cuda))


def test_paged_entries_outside_the_pool_read_as_zero(cuda):
    """A bad table entry (past the pool, or negative) reads as zero keys and
    values: no fault, and the result matches the oracle's reading."""
    lens = [40, 100, 33]
    case = testing.make_case("paged_bad", [1] * 3, lens, 8, 2, 128, torch.bfloat16, seed=12,
                             causal=False)
    pk = testing.paginate(case, block_size=16, seed=4)
    pk.block_table[0, 1] = pk.k_cache.shape[0] + 3
    pk.block_table[1, 0] = -5
    got = _paged(case, pk, cuda)
    _check(got, _oracle(case, pk))


def test_paged_lengths_past_the_table_are_clamped(cuda):
    """seqused_k beyond what a table row addresses is clamped to
    max_blocks * block_size keys."""
    lens = [64, 20]
    case = testing.make_case("paged_clamp", [1] * 2, lens, 4, 2, 64, torch.bfloat16, seed=13,
                             causal=False)
    pk = testing.paginate(case, block_size=16, seed=5)  # table rows of 4 blocks
    pk.seqused_k = torch.tensor([1000, 20], dtype=torch.int32)
    got = _paged(case, pk, cuda, max_k=64)
    want = _oracle(case, testing.PagedKV(pk.k_cache, pk.v_cache, pk.block_table,
                                         torch.tensor([64, 20], dtype=torch.int32)))
    _check(got, want)


def test_paged_rejects_bad_block_size(cuda):
    case = testing.make_case("paged_bs", [1], [40], 4, 2, 64, torch.bfloat16, seed=1,
                             causal=False)
    pk = testing.paginate(case, block_size=16, seed=0)
    pk.k_cache = torch.zeros(8, 12, 2, 64, dtype=torch.bfloat16)  # 12: not a power of two
    pk.v_cache = torch.zeros_like(pk.k_cache)
    with pytest.raises(RuntimeError, match="IFA4_EINVAL"):
        _paged(case, pk, cuda)
