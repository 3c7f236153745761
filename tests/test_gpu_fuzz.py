"""Seeded random sweep of the prefill and decode entry points against the oracle.

Each case draws its own shapes and options (ragged lengths with Lk >= Lq and
Lk < Lq, GQA ratios, head_dim 64/128, bf16/fp16, causal or not, left windows,
rel_extent from 1 to 200, per-token and shared bias, bf16/fp32 bias, top-left
and bottom-right alignment; for decode also paged caches of several block
sizes and fp8 caches; for prefill also the fused relative-logit projection),
runs the HIP path and compares every row with the fp32 oracle at the
operator's tolerances (out atol/rtol 2e-2, lse atol 1e-3).
"""
import random

import pytest
import torch

from inkling_fa4 import (inkling_fa4_rel_attention, inkling_fa4_rel_attention_decode,
                         inkling_fa4_rel_attention_decode_paged, inkling_fa4_rel_attention_rproj,
                         testing)
from oracle import ref_rel_attn_paged_with_lse, ref_rel_attn_rproj_with_lse, ref_rel_attn_with_lse

pytestmark = pytest.mark.gpu

ATOL, RTOL, LSE_ATOL = 2e-2, 2e-2, 1e-3
HEADS = [(4, 4), (8, 2), (6, 3), (8, 1), (2, 1), (16, 4)]


def _draw(seed, decode):
    r = random.Random(seed)
    batch = r.randint(1, 6)
    if decode:
        lens_q = [1] * batch
        lens_k = [r.choice([0, 1, r.randint(1, 64), r.randint(64, 1500)]) for _ in range(batch)]
    else:
        lens_q = [r.choice([1, r.randint(1, 64), r.randint(64, 300)]) for _ in range(batch)]
        lens_k = [max(0, lq + r.choice([0, r.randint(0, 300), -r.randint(0, lq)])) for lq in lens_q]
    hq, hkv = r.choice(HEADS)
    head_dim = r.choice([64, 128])
    dtype = r.choice([torch.bfloat16, torch.float16])
    rel_extent = r.choice([1, 16, 100, 128, 200])
    opts = dict(
        causal=r.random() < 0.6,
        window_left=r.choice([-1, -1, 0, r.randint(1, 200)]),
        rel_table=r.random() < 0.6,
        rel_dtype=r.choice([torch.float32, torch.bfloat16]),
        rel_extent=rel_extent,
        rel_width=rel_extent + r.choice([0, 0, 7]),
        scale=r.choice([None, 0.3]),
    )
    bottom_right = r.random() < 0.3
    return lens_q, lens_k, hq, hkv, head_dim, dtype, opts, bottom_right


def _check(case, out, lse, bottom_right, want=None):
    """Rows that see no key are NaN in the oracle (the reference's softmax over
    nothing); the operator writes out = 0 and lse = -inf there."""
    if want is None:
        want = ref_rel_attn_with_lse(
            case.q, case.k, case.v, case.rel, case.cu_q, case.cu_k, case.scale, case.rel_extent,
            causal=case.causal, window_left=case.window_or_none, bottom_right=bottom_right)
    want_out, want_lse = want
    out, lse = out.cpu().float(), lse.cpu().transpose(0, 1)  # lse as [Tq, Hq]
    want_lse = want_lse.transpose(0, 1)
    empty = torch.isnan(want_out.float()).any(-1) | torch.isneginf(want_lse)  # [Tq, Hq]
    assert (out[empty] == 0).all()
    assert torch.isneginf(lse[empty]).all()
    keep = ~empty
    torch.testing.assert_close(out[keep], want_out.float()[keep], atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(lse[keep], want_lse[keep], atol=LSE_ATOL, rtol=0)


@pytest.mark.parametrize("seed", range(24))
def test_prefill_random_configs(cuda, seed):
    lens_q, lens_k, hq, hkv, d, dtype, opts, br = _draw(1000 + seed, decode=False)
    case = testing.make_case(f"fuzz{seed}", lens_q, lens_k, hq, hkv, d, dtype, seed=seed, **opts)
    c = case.to(cuda)
    out, lse = inkling_fa4_rel_attention(*c.args(), causal=c.causal, window_size=c.window_size,
                                         softmax_scale=c.scale, return_lse=True, bottom_right=br)
    torch.cuda.synchronize()
    _check(case, out, lse, br)


@pytest.mark.parametrize("seed", range(16))
def test_decode_random_configs(cuda, seed):
    lens_q, lens_k, hq, hkv, d, dtype, opts, br = _draw(2000 + seed, decode=True)
    case = testing.make_case(f"fuzzd{seed}", lens_q, lens_k, hq, hkv, d, dtype, seed=seed, **opts)
    c = case.to(cuda)
    out, lse = inkling_fa4_rel_attention_decode(*c.args(), causal=c.causal,
                                                window_size=c.window_size, softmax_scale=c.scale,
                                                return_lse=True, bottom_right=br)
    torch.cuda.synchronize()
    _check(case, out, lse, br)


@pytest.mark.parametrize("seed", range(12))
def test_decode_paged_random_configs(cuda, seed):
    lens_q, lens_k, hq, hkv, d, dtype, opts, br = _draw(3000 + seed, decode=True)
    case = testing.make_case(f"fuzzp{seed}", lens_q, lens_k, hq, hkv, d, dtype, seed=seed, **opts)
    block = random.Random(seed).choice([8, 16, 32, 64, 256])
    pk = testing.paginate(case, block_size=block, seed=seed)
    c, p = case.to(cuda), pk.to(cuda)
    out, lse = inkling_fa4_rel_attention_decode_paged(
        c.q, p.k_cache, p.v_cache, c.rel, c.cu_q, p.seqused_k, p.block_table, c.max_q, c.max_k,
        c.rel_extent, causal=c.causal, window_size=c.window_size, softmax_scale=c.scale,
        return_lse=True, bottom_right=br)
    torch.cuda.synchronize()
    want = ref_rel_attn_paged_with_lse(case.q, pk.k_cache, pk.v_cache, case.rel, case.cu_q,
                                       pk.seqused_k, pk.block_table, case.scale, case.rel_extent,
                                       causal=case.causal, window_left=case.window_or_none,
                                       bottom_right=br)
    _check(case, out, lse, br, want)


@pytest.mark.parametrize("seed", range(12))
def test_decode_fp8_random_configs(cuda, seed):
    lens_q, lens_k, hq, hkv, d, dtype, opts, br = _draw(4000 + seed, decode=True)
    if hq // hkv > 8:
        hq = hkv * 8
    if sum(lens_k) == 0:  # the per-tensor fp8 scale needs at least one key
        lens_k[0] = 5
    case = testing.make_case(f"fuzz8{seed}", lens_q, lens_k, hq, hkv, d, dtype, seed=seed, **opts)
    k8, v8, ks, vs, deq = testing.fp8_kv(case)
    c = case.to(cuda)
    out, lse = inkling_fa4_rel_attention_decode(
        c.q, k8.to(cuda), v8.to(cuda), c.rel, c.cu_q, c.cu_k, c.max_q, c.max_k, c.rel_extent,
        causal=c.causal, window_size=c.window_size, softmax_scale=c.scale, return_lse=True,
        bottom_right=br, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    _check(deq, out, lse, br)


@pytest.mark.parametrize("seed", range(8))
def test_decode_fp8_pair_random_configs(cuda, seed):
    """Random configs held to the fp8 caches whose adjacent kv heads stream in
    pairs (d 128, an even number of kv heads, at most 4 query heads each)."""
    lens_q, lens_k, _, _, _, dtype, opts, br = _draw(4500 + seed, decode=True)
    r = random.Random(seed)
    hkv = r.choice([2, 4, 6])
    hq = hkv * r.choice([1, 2, 3, 4])
    if sum(lens_k) == 0:
        lens_k[0] = 5
    case = testing.make_case(f"fuzzp{seed}", lens_q, lens_k, hq, hkv, 128, dtype, seed=seed,
                             **opts)
    k8, v8, ks, vs, deq = testing.fp8_kv(case)
    c = case.to(cuda)
    out, lse = inkling_fa4_rel_attention_decode(
        c.q, k8.to(cuda), v8.to(cuda), c.rel, c.cu_q, c.cu_k, c.max_q, c.max_k, c.rel_extent,
        causal=c.causal, window_size=c.window_size, softmax_scale=c.scale, return_lse=True,
        bottom_right=br, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    _check(deq, out, lse, br)


@pytest.mark.parametrize("seed", range(12))
def test_rproj_random_configs(cuda, seed):
    lens_q, lens_k, hq, hkv, d, dtype, opts, br = _draw(5000 + seed, decode=False)
    r = random.Random(seed)
    opts["rel_extent"] = r.choice([1, 16, 64, 100, 128, 300, 512, 1024])
    width = opts["rel_extent"] + r.choice([0, 9])
    opts["rel_width"] = width
    case = testing.make_case(f"fuzzr{seed}", lens_q, lens_k, hq, hkv, d, dtype, seed=seed, **opts)
    g = torch.Generator().manual_seed(seed)
    rr = (0.3 * torch.randn(case.q.shape[0], hq, 16, generator=g)).to(
        r.choice([torch.float32, torch.bfloat16]))
    w = 0.3 * torch.randn(16, width, generator=g)
    c = case.to(cuda)
    out, lse = inkling_fa4_rel_attention_rproj(
        c.q, c.k, c.v, rr.to(cuda), w.to(cuda), c.cu_q, c.cu_k, c.max_q, c.max_k, c.rel_extent,
        causal=c.causal, window_size=c.window_size, softmax_scale=c.scale, return_lse=True,
        bottom_right=br)
    torch.cuda.synchronize()
    want = ref_rel_attn_rproj_with_lse(case.q, case.k, case.v, rr, w, case.cu_q, case.cu_k,
                                       case.scale, case.rel_extent, causal=case.causal,
                                       window_left=case.window_or_none, bottom_right=br)
    _check(case, out, lse, br, want)
