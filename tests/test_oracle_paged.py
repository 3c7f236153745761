"""Pins the paged-cache oracle (oracle/paged.py) and the test helper that
builds paged caches (inkling_fa4.testing.paginate).

The gather is fixed by properties a plausible indexing mistake breaks:
an identity table over a block-reshaped contiguous cache reproduces it;
permuting the physical blocks (and the table with them) changes nothing;
the block size changes nothing; rows no sequence owns (NaN) never reach the
result; an entry outside the pool reads as zeros."""
import math

import pytest
import torch

from inkling_fa4 import testing
from oracle import gather_paged, ref_rel_attn_paged_with_lse, ref_rel_attn_with_lse


def _identity_pool(k, v, cu, bs):
    """Each sequence's rows padded to whole blocks, blocks numbered in order."""
    kb, vb, rows, nxt = [], [], [], 0
    cu = [int(x) for x in cu]
    width = max([1] + [math.ceil((cu[b + 1] - cu[b]) / bs) for b in range(len(cu) - 1)])
    for b in range(len(cu) - 1):
        n = cu[b + 1] - cu[b]
        nb = math.ceil(n / bs)
        pad = nb * bs - n
        kb.append(torch.cat([k[cu[b]:cu[b + 1]], torch.zeros(pad, *k.shape[1:], dtype=k.dtype)]))
        vb.append(torch.cat([v[cu[b]:cu[b + 1]], torch.zeros(pad, *v.shape[1:], dtype=v.dtype)]))
        rows.append(list(range(nxt, nxt + nb)) + [0] * (width - nb))
        nxt += nb
    kc = torch.cat(kb).view(-1, bs, *k.shape[1:])
    vc = torch.cat(vb).view(-1, bs, *v.shape[1:])
    lens = torch.tensor([cu[b + 1] - cu[b] for b in range(len(cu) - 1)], dtype=torch.int32)
    return kc, vc, torch.tensor(rows, dtype=torch.int32), lens


def _case(seed=0, lens=(37, 0, 64, 129, 5)):
    return testing.make_case("paged", [1] * len(lens), list(lens), 8, 2, 64, torch.bfloat16,
                             seed=seed, causal=False)


@pytest.mark.parametrize("bs", [8, 16, 32])
def test_identity_table_reproduces_the_contiguous_cache(bs):
    c = _case()
    kc, vc, table, lens = _identity_pool(c.k, c.v, c.cu_k.tolist(), bs)
    k, v, cu = gather_paged(kc, vc, table, lens)
    assert torch.equal(cu, c.cu_k)
    assert torch.equal(k, c.k) and torch.equal(v, c.v)


def test_block_permutation_and_block_size_invariance():
    c = _case(seed=1)
    kc, vc, table, lens = _identity_pool(c.k, c.v, c.cu_k.tolist(), 16)
    perm = torch.randperm(kc.shape[0], generator=torch.Generator().manual_seed(3))
    kc2 = torch.empty_like(kc)
    vc2 = torch.empty_like(vc)
    kc2[perm] = kc
    vc2[perm] = vc
    k1, v1, _ = gather_paged(kc2, vc2, perm[table.long()].int(), lens)
    k8, v8, _ = gather_paged(*_identity_pool(c.k, c.v, c.cu_k.tolist(), 8))
    assert torch.equal(k1, c.k) and torch.equal(v1, c.v)
    assert torch.equal(k8, k1) and torch.equal(v8, v1)
    # a wrong row index (j // bs for j % bs) or a transposed table would differ
    assert not torch.equal(gather_paged(kc2, vc2, table, lens)[0], c.k)


@pytest.mark.parametrize("bs", [8, 16, 64])
def test_paginate_helper_round_trips(bs):
    c = _case(seed=2)
    pk = testing.paginate(c, block_size=bs, seed=bs, extra_columns=2)
    assert pk.k_cache.isnan().any()  # spare blocks and tails are NaN
    k, v, cu = gather_paged(pk.k_cache, pk.v_cache, pk.block_table, pk.seqused_k)
    assert torch.equal(k, c.k) and torch.equal(v, c.v) and torch.equal(cu, c.cu_k)
    # table entries past a sequence's blocks are garbage, outside the pool
    assert (pk.block_table >= pk.k_cache.shape[0]).any()


def test_entry_outside_the_pool_reads_as_zero():
    c = _case(seed=3, lens=(40,))
    pk = testing.paginate(c, block_size=16, seed=0)
    table = pk.block_table.clone()
    table[0, 1] = pk.k_cache.shape[0] + 7
    k, v, _ = gather_paged(pk.k_cache, pk.v_cache, table, pk.seqused_k)
    assert torch.equal(k[16:32], torch.zeros_like(k[16:32]))
    assert torch.equal(k[:16], c.k[:16]) and torch.equal(v[32:], c.v[32:])
    table[0, 0] = -1
    k, _, _ = gather_paged(pk.k_cache, pk.v_cache, table, pk.seqused_k)
    assert torch.equal(k[:16], torch.zeros_like(k[:16]))


@pytest.mark.parametrize("causal", [False, True])
def test_paged_oracle_equals_contiguous_oracle(causal):
    c = _case(seed=4)
    pk = testing.paginate(c, block_size=16, seed=9)
    out_p, lse_p = ref_rel_attn_paged_with_lse(c.q, pk.k_cache, pk.v_cache, c.rel, c.cu_q,
                                               pk.seqused_k, pk.block_table, c.scale,
                                               c.rel_extent, causal=causal)
    out_c, lse_c = ref_rel_attn_with_lse(c.q, c.k, c.v, c.rel, c.cu_q, c.cu_k, c.scale,
                                         c.rel_extent, causal=causal)
    assert torch.equal(out_p, out_c) and torch.equal(lse_p, lse_c)
    assert not out_p[c.cu_k[1:] - c.cu_k[:-1] > 0].isnan().any()
