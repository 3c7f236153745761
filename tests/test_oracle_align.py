"""Pins the oracle's bottom-right alignment (upstream flash-attn convention,
outputs/architecture.md:72; no counterpart in the reference's own oracle).

It is tied to the golden-pinned top-left oracle and to an independent
attention core by exact identities:
  * Lq == Lk: the two alignments coincide;
  * Lk >= Lq: bottom-right rows equal the last Lq rows of a top-left call whose
    queries are prefixed with Lk - Lq extra rows (query i then sits at key
    position i + Lk - Lq in both);
  * Lq > Lk: the last Lk rows equal a call on those rows alone (Lq' = Lk), the
    first Lq - Lk rows see no key under causal masking;
  * zero bias: torch SDPA with the bottom-right boolean mask.
A dropped offset, a flipped sign or a top-left mask fails one of these."""
import math

import pytest
import torch

from inkling_fa4 import testing
from oracle import ref_rel_attn_with_lse


def _one(lq, lk, seed, causal=True, window=None, rel_std=0.5, hq=4, hkv=2, d=64):
    c = testing.make_case("align", [lq], [lk], hq, hkv, d, torch.bfloat16, seed=seed,
                          rel_table=False, rel_std=rel_std, causal=causal,
                          window_left=-1 if window is None else window)
    return c


def _run(c, bottom_right, causal=None, window=None, q=None, rel=None, cu_q=None):
    return ref_rel_attn_with_lse(c.q if q is None else q, c.k, c.v, c.rel if rel is None else rel,
                                 c.cu_q if cu_q is None else cu_q, c.cu_k, c.scale, c.rel_extent,
                                 causal=c.causal if causal is None else causal,
                                 window_left=c.window_or_none if window is None else window,
                                 bottom_right=bottom_right)


@pytest.mark.parametrize("causal,window", [(True, None), (False, 7), (True, 20), (False, None)])
def test_equal_lengths_align_the_same(causal, window):
    c = _one(90, 90, seed=1, causal=causal, window=window)
    a, b = _run(c, False), _run(c, True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


@pytest.mark.parametrize("lq,lk,causal,window", [(40, 300, True, None), (64, 200, True, 63),
                                                 (17, 150, False, 30), (1, 500, True, 100)])
def test_prefix_padding_identity(lq, lk, causal, window):
    c = _one(lq, lk, seed=2, causal=causal, window=window)
    pad = lk - lq
    g = torch.Generator().manual_seed(9)
    qp = torch.cat([torch.randn(pad, *c.q.shape[1:], generator=g).to(c.q.dtype), c.q])
    relp = torch.cat([torch.randn(pad, *c.rel.shape[1:], generator=g), c.rel])
    cu = torch.tensor([0, lk], dtype=torch.int32)
    top = _run(c, False, q=qp, rel=relp, cu_q=cu)         # reference semantics, Lq' = Lk
    bot = _run(c, True)
    assert torch.equal(bot[0], top[0][pad:]) and torch.equal(bot[1], top[1][:, pad:])
    # and it is not the reference alignment on the unpadded call
    ref = _run(c, False)
    assert not torch.equal(bot[1], ref[1])


def test_more_queries_than_keys():
    lq, lk = 100, 40
    c = _one(lq, lk, seed=3, causal=True)
    bot = _run(c, True)
    assert torch.isneginf(bot[1][:, :lq - lk]).all()
    tail_q, tail_rel = c.q[lq - lk:], c.rel[lq - lk:]
    cu = torch.tensor([0, lk], dtype=torch.int32)
    alone = _run(c, True, q=tail_q, rel=tail_rel, cu_q=cu)
    assert torch.equal(bot[0][lq - lk:], alone[0]) and torch.equal(bot[1][:, lq - lk:], alone[1])


@pytest.mark.parametrize("lq,lk,window", [(30, 70, None), (50, 50, 10), (20, 90, 5)])
def test_bias_free_case_matches_sdpa(lq, lk, window):
    c = _one(lq, lk, seed=4, causal=True, window=window, rel_std=0.0)
    out, _ = _run(c, True)
    i = torch.arange(lq).unsqueeze(1) + (lk - lq)
    j = torch.arange(lk).unsqueeze(0)
    mask = j <= i
    if window is not None:
        mask &= (i - j) <= window
    group = c.q.shape[1] // c.k.shape[1]
    q = c.q.float().transpose(0, 1)                                   # [H, lq, d]
    k = c.k.float().repeat_interleave(group, 1).transpose(0, 1)
    v = c.v.float().repeat_interleave(group, 1).transpose(0, 1)
    want = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask,
                                                            scale=c.scale)
    torch.testing.assert_close(out.float(), want.transpose(0, 1).to(out.dtype).float(),
                               atol=1e-2, rtol=0)


def test_decode_bottom_right_bias_is_alive():
    """Lq = 1 over Lk keys: the last rel_extent keys carry the bias (dist =
    Lk - 1 - j), unlike the reference alignment where decode never sees it."""
    c = _one(1, 300, seed=5, causal=True)
    zero = c.rel.clone().zero_()
    with_bias = _run(c, True)
    without = _run(c, True, rel=zero)
    assert not torch.equal(with_bias[1], without[1])
    ref_a, ref_b = _run(c, False), _run(c, False, rel=zero)
    assert torch.equal(ref_a[1], ref_b[1])
    assert math.isfinite(float(with_bias[1].min()))
