"""The oracle against what the mathematics fixes, independently of its code:
torch SDPA (an independent attention core), the Toeplitz structure of a
stride-0 bias table read back through one-hot values, closed-form LSEs,
packing invariance and the split-merge identity.  The oracle computes in fp32
(as the reference does), so float64 comparisons use fp32-level tolerances;
every planted mistake these tests guard against moves results by O(0.1)."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from scipy.special import logsumexp

from oracle import merge_partials, ref_rel_attn, ref_rel_attn_with_lse


def _cu(lens):
    return torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)


def _inputs(lq, lk, hq, hkv, d, r, seed, table=False, width=None):
    g = torch.Generator().manual_seed(seed)
    tq, tk = sum(lq), sum(lk)
    q = torch.randn(tq, hq, d, generator=g, dtype=torch.float64)
    k = torch.randn(tk, hkv, d, generator=g, dtype=torch.float64)
    v = torch.randn(tk, hkv, d, generator=g, dtype=torch.float64)
    w = width or r
    if table:
        t = torch.randn(hq, w, generator=g, dtype=torch.float64)
        rel = t.unsqueeze(0).expand(tq, hq, w)
    else:
        rel = torch.randn(tq, hq, w, generator=g, dtype=torch.float64)
    return q, k, v, rel


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2), (6, 3)])
def test_bias_dead_chunk_equals_sdpa_top_left_causal(hq, hkv):
    """Lk >= 2 Lq: no visible pair has dist >= 0, so the op is plain causal
    attention with top-left alignment, which is what SDPA's is_causal does."""
    lq, lk, d = 9, 23, 16
    q, k, v, rel = _inputs([lq], [lk], hq, hkv, d, 32, seed=11)
    scale = 0.3
    out = ref_rel_attn(q, k, v, rel, _cu([lq]), _cu([lk]), scale, 32, causal=True)
    rep = hq // hkv
    kk = k.repeat_interleave(rep, dim=1).transpose(0, 1)
    vv = v.repeat_interleave(rep, dim=1).transpose(0, 1)
    want = F.scaled_dot_product_attention(q.transpose(0, 1), kk, vv, is_causal=True, scale=scale)
    torch.testing.assert_close(out, want.transpose(0, 1), atol=2e-6, rtol=0)


def test_noncausal_bias_dead_equals_sdpa_and_lse_closed_form():
    lq, lk, d = 3, 40, 8
    q, k, v, rel = _inputs([lq], [lk], 2, 1, d, 4, seed=12)
    out, lse = ref_rel_attn_with_lse(q, k, v, rel, _cu([lq]), _cu([lk]), 0.5, 4, causal=False)
    kk = k.expand(lk, 2, d).transpose(0, 1)
    vv = v.expand(lk, 2, d).transpose(0, 1)
    want = F.scaled_dot_product_attention(q.transpose(0, 1), kk, vv, scale=0.5)
    torch.testing.assert_close(out, want.transpose(0, 1), atol=2e-6, rtol=0)
    s = np.einsum("qhd,kd->hqk", q.numpy(), k[:, 0].numpy()) * 0.5
    np.testing.assert_allclose(lse.numpy(), logsumexp(s, axis=-1), rtol=0, atol=1e-5)


@pytest.mark.parametrize("causal,window", [(True, None), (False, None), (True, 5), (False, 3)])
def test_stride0_table_is_toeplitz_bias(causal, window):
    """q = 0 makes the logits equal the bias; one-hot values read the
    probabilities back.  For Lq = Lk a per-head table T gives
    log p[i,j] - log p[i,i] = T[i-j]·[0 <= i-j < R] - T[0] on visible pairs."""
    L, r = 14, 6
    g = torch.Generator().manual_seed(13)
    table = torch.randn(1, r, generator=g, dtype=torch.float64)
    rel = table.unsqueeze(0).expand(L, 1, r)
    q = torch.zeros(L, 1, L, dtype=torch.float64)
    k = torch.zeros(L, 1, L, dtype=torch.float64)
    v = torch.eye(L, dtype=torch.float64).unsqueeze(1)
    p, lse = ref_rel_attn_with_lse(q, k, v, rel, _cu([L]), _cu([L]), 1.0, r, causal=causal,
                                   window_left=window)
    p = p[:, 0]
    T = table[0].numpy()
    for i in range(L):
        row_vals = []
        for j in range(L):
            vis = (not causal or i >= j) and (window is None or i - j <= window)
            if not vis:
                assert p[i, j] == 0.0
                continue
            b = T[i - j] if 0 <= i - j < r else 0.0
            row_vals.append(b)
            assert math.isclose(math.log(p[i, j]) - math.log(p[i, i]), b - T[0], abs_tol=2e-6)
        assert math.isclose(lse[0, i].item(), float(logsumexp(row_vals)), abs_tol=2e-6)


def test_bias_distance_offset_for_chunked_query():
    """Lq < Lk with a non-causal query block and zero logits: the bias read by
    query i at key j is rel[i, i + (Lq - Lk) - j] inside the band."""
    lq, lk, r = 4, 6, 8
    g = torch.Generator().manual_seed(14)
    rel = torch.randn(lq, 1, r, generator=g, dtype=torch.float64)
    q = torch.zeros(lq, 1, lk, dtype=torch.float64)
    k = torch.zeros(lk, 1, lk, dtype=torch.float64)
    v = torch.eye(lk, dtype=torch.float64).unsqueeze(1)
    p = ref_rel_attn(q, k, v, rel, _cu([lq]), _cu([lk]), 1.0, r, causal=False)[:, 0]
    for i in range(lq):
        logits = []
        for j in range(lk):
            dist = i + (lq - lk) - j
            logits.append(rel[i, 0, dist].item() if 0 <= dist < r else 0.0)
        want = np.exp(np.array(logits) - logsumexp(logits))
        np.testing.assert_allclose(p[i].numpy(), want, atol=2e-7)


def test_float64_loop_restatement_tiny():
    """Element-by-element float64 loop on tiny ragged GQA shapes."""
    lq, lk = [5, 3, 7], [5, 6, 2]
    hq, hkv, d, r = 4, 2, 4, 3
    q, k, v, rel = _inputs(lq, lk, hq, hkv, d, r, seed=15, width=5)
    cq, ck = _cu(lq), _cu(lk)
    for causal in (True, False):
        for window in (None, 1):
            out = ref_rel_attn(q, k, v, rel, cq, ck, 0.7, r, causal=causal, window_left=window)
            for b in range(3):
                for h in range(hq):
                    kh = h // (hq // hkv)
                    for i in range(lq[b]):
                        logits, vals = [], []
                        for j in range(lk[b]):
                            if causal and j > i:
                                continue
                            if window is not None and i - j > window:
                                continue
                            x = 0.7 * float(q[cq[b] + i, h] @ k[ck[b] + j, kh])
                            dist = i + lq[b] - lk[b] - j
                            if 0 <= dist < r:
                                x += float(rel[cq[b] + i, h, dist])
                            logits.append(x)
                            vals.append(v[ck[b] + j, kh].numpy())
                        got = out[cq[b] + i, h].numpy()
                        if not logits:
                            assert np.isnan(got).all()
                            continue
                        w = np.exp(np.array(logits) - logsumexp(logits))
                        np.testing.assert_allclose(got, w @ np.array(vals), atol=2e-6)


def test_packing_invariance():
    """A packed varlen batch equals each sequence computed on its own."""
    lq, lk = [7, 1, 12], [9, 5, 12]
    q, k, v, rel = _inputs(lq, lk, 4, 2, 8, 6, seed=16)
    out, lse = ref_rel_attn_with_lse(q, k, v, rel, _cu(lq), _cu(lk), 0.4, 6, causal=True,
                                     window_left=4)
    cq, ck = _cu(lq).tolist(), _cu(lk).tolist()
    for b in range(3):
        o_b, l_b = ref_rel_attn_with_lse(q[cq[b]:cq[b + 1]], k[ck[b]:ck[b + 1]],
                                         v[ck[b]:ck[b + 1]], rel[cq[b]:cq[b + 1]],
                                         _cu([lq[b]]), _cu([lk[b]]), 0.4, 6, causal=True,
                                         window_left=4)
        assert torch.equal(out[cq[b]:cq[b + 1]].nan_to_num(), o_b.nan_to_num())
        assert torch.equal(lse[:, cq[b]:cq[b + 1]], l_b)


@pytest.mark.parametrize("n_splits", [1, 2, 7, 37])
def test_merge_partials_split_invariance(n_splits):
    """Splitting one query row's keys and merging (o_s, lse_s) by LSE equals
    the unsplit softmax-weighted sum (closed form, float64)."""
    g = torch.Generator().manual_seed(17)
    L, D = 37, 8
    x = torch.randn(3, L, generator=g, dtype=torch.float64) * 3
    vals = torch.randn(L, D, generator=g, dtype=torch.float64)
    full_lse = torch.logsumexp(x, -1)
    full_o = torch.softmax(x, -1) @ vals
    bounds = np.linspace(0, L, n_splits + 1).round().astype(int)
    o_parts, l_parts = [], []
    for s in range(n_splits):
        a, b = bounds[s], bounds[s + 1]
        if a == b:
            o_parts.append(torch.zeros(3, D, dtype=torch.float64))
            l_parts.append(torch.full((3,), -math.inf, dtype=torch.float64))
            continue
        l_parts.append(torch.logsumexp(x[:, a:b], -1))
        o_parts.append(torch.softmax(x[:, a:b], -1) @ vals[a:b])
    o, lse = merge_partials(torch.stack(o_parts), torch.stack(l_parts))
    torch.testing.assert_close(lse, full_lse.float(), atol=1e-5, rtol=0)
    torch.testing.assert_close(o, full_o.float(), atol=1e-5, rtol=0)


def test_merge_partials_all_empty():
    o, lse = merge_partials(torch.zeros(3, 2, 4), torch.full((3, 2), -math.inf))
    assert torch.equal(o, torch.zeros(2, 4))
    assert torch.isinf(lse).all() and (lse < 0).all()
