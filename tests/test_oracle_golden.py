"""The fp32 oracle against golden vectors written by the reference's own
reference.py (tests/golden/make_golden.py), and proof that those vectors pin
each convention: every planted mistake below makes at least one fixture fail.
"""
import math

import pytest
import torch

import golden
from oracle import ref_rel_attn, ref_rel_attn_with_lse

NAMES = golden.names()


def _run(oracle_fn, d):
    return oracle_fn(d["q"], d["k"], d["v"], d["rel"], d["cu_seqlens_q"], d["cu_seqlens_k"],
                     d["scale"], d["rel_extent"], causal=d["causal"],
                     window_left=d["window_left"])


def _matches(got, want):
    """Equal NaN pattern; values equal up to one rounding step of the dtype."""
    if got.dtype != want.dtype or got.shape != want.shape:
        return False
    g, w = got.float(), want.float()
    if not torch.equal(torch.isnan(g), torch.isnan(w)):
        return False
    ok = ~torch.isnan(w)
    eps = {torch.float32: 2e-6, torch.bfloat16: 2 ** -7, torch.float16: 2 ** -10}[want.dtype]
    return bool(((g[ok] - w[ok]).abs() <= eps * w[ok].abs() + 1e-6).all())


def test_fixture_set_present():
    assert len(NAMES) >= 12, NAMES


@pytest.mark.parametrize("name", NAMES)
def test_oracle_matches_reference_golden(name):
    d = golden.load(name)
    out = _run(ref_rel_attn, d)
    assert _matches(out, d["out"]), name


@pytest.mark.parametrize("name", NAMES)
def test_oracle_lse_is_consistent_with_out(name):
    """out = sum_j exp(s_ij - lse_i) v_j: with V replaced by one-hot rows the
    output is the probability matrix, whose rows must sum to 1 exactly where
    lse is finite (and the row must be NaN/empty where lse = -inf)."""
    d = golden.load(name)
    q, k = d["q"].float(), d["k"].float()
    cu_k = d["cu_seqlens_k"].tolist()
    lk_max = max(cu_k[b + 1] - cu_k[b] for b in range(len(cu_k) - 1))
    # one-hot values v[j] = e_{local j}; q and k zero-padded to the same width
    # (the output takes q's shape), which leaves every dot product unchanged
    width = max(q.shape[-1], lk_max)
    q = torch.nn.functional.pad(q, (0, width - q.shape[-1]))
    k = torch.nn.functional.pad(k, (0, width - k.shape[-1]))
    eye = torch.zeros(k.shape[0], k.shape[1], width)
    for b in range(len(cu_k) - 1):
        for j in range(cu_k[b + 1] - cu_k[b]):
            eye[cu_k[b] + j, :, j] = 1.0
    probs, lse = ref_rel_attn_with_lse(q, k, eye, d["rel"], d["cu_seqlens_q"],
                                       d["cu_seqlens_k"], d["scale"], d["rel_extent"],
                                       causal=d["causal"], window_left=d["window_left"])
    rows = probs.sum(-1)  # [Tq, Hq]
    finite = torch.isfinite(lse.transpose(0, 1))
    assert torch.allclose(rows[finite], torch.ones_like(rows[finite]), atol=1e-5)
    assert torch.isnan(rows[~finite]).all()


# ---- planted mistakes: a mutant oracle with one convention changed ------------------------

def _mutant(q, k, v, rel, cu_q, cu_k, scale, rel_extent, causal=True, window_left=None,
            mutation=None):
    """Dense oracle with one deliberately wrong convention (CPU only)."""
    n_q, hq, _ = q.shape
    hkv = k.shape[1]
    group = hq // hkv
    out = torch.zeros_like(q)
    cq, ck = cu_q.tolist(), cu_k.tolist()
    for b in range(len(cq) - 1):
        q0, q1, k0, k1 = cq[b], cq[b + 1], ck[b], ck[b + 1]
        lq, lk = q1 - q0, k1 - k0
        i = torch.arange(lq).unsqueeze(1)
        j = torch.arange(lk).unsqueeze(0)
        delta = (lk - lq) if mutation == "delta_sign" else (lq - lk)
        dist = i + delta - j
        if mutation == "bias_index_reversed":
            dist = j - i - delta
        band = (dist >= 0) & (dist < rel_extent)
        idx = dist.clamp(0, rel_extent - 1)
        if causal:
            vis = (i + (lk - lq) >= j) if mutation == "bottom_right_causal" else (i >= j)
        else:
            vis = torch.ones(lq, lk, dtype=torch.bool)
        if window_left is not None:
            if not (mutation == "window_only_with_causal" and not causal):
                vis = vis & ((i - j) <= window_left)
        for h in range(hq):
            kh = (h % hkv) if mutation == "gqa_modulo" else (h // group)
            s = q[q0:q1, h].float() @ k[k0:k1, kh].float().T * scale
            bias = torch.gather(rel[q0:q1, h].float(), 1, idx)
            if mutation != "bias_clamped":
                bias = torch.where(band, bias, torch.zeros_like(bias))
            s = s + bias
            s = s.masked_fill(~vis, -math.inf)
            p = torch.softmax(s, -1)
            if mutation == "empty_rows_zero":
                p = torch.nan_to_num(p, nan=0.0)
            o = p @ v[k0:k1, kh].float()
            out[q0:q1, h] = o if mutation == "no_output_rounding" else o.to(out.dtype)
    if mutation == "no_output_rounding":
        return out.float()
    return out


MUTATIONS = ["delta_sign", "bias_index_reversed", "bottom_right_causal",
             "window_only_with_causal", "gqa_modulo", "bias_clamped", "empty_rows_zero",
             "no_output_rounding"]


def test_unmutated_twin_matches_golden():
    for name in NAMES:
        d = golden.load(name)
        out = _run(lambda *a, **kw: _mutant(*a, **kw, mutation=None), d)
        assert _matches(out, d["out"]), name


@pytest.mark.parametrize("mutation", MUTATIONS)
def test_golden_vectors_catch_planted_mistake(mutation):
    failed = []
    for name in NAMES:
        d = golden.load(name)
        out = _run(lambda *a, **kw: _mutant(*a, **kw, mutation=mutation), d)
        if not _matches(out, d["out"]):
            failed.append(name)
    assert failed, f"no golden case detects mutation {mutation!r}"
