"""GPU parity of prefill with the fused relative-logit projection
(inkling_fa4_rel_attention_rproj): the bias is computed in the kernel from
r [Tq, Hq, 16] and W [16, R'] instead of a materialised rel_logits, on the
matrix cores, for any rel_extent (128 and below, and the serving model's 512
and 1024).

Against the oracle on the einsum-materialised rel_logits: out within atol /
rtol 2e-2, lse within 1e-3.  A rank-one factorisation that reproduces a
per-head table must give the table path's result.
"""
import pytest
import torch

from inkling_fa4 import inkling_fa4_rel_attention, inkling_fa4_rel_attention_rproj, testing
from oracle import ref_rel_attn_rproj_with_lse

pytestmark = pytest.mark.gpu

ATOL, RTOL, LSE_ATOL = 2e-2, 2e-2, 1e-3


def _factors(case, width, seed, r_dtype=torch.float32, std=0.3):
    g = torch.Generator().manual_seed(seed)
    r = (std * torch.randn(case.q.shape[0], case.q.shape[1], 16, generator=g)).to(r_dtype)
    w = std * torch.randn(16, width, generator=g)
    return r, w


def _run(case, r, w, dev, bottom_right=False):
    c = case.to(dev)
    print(f"rproj {case.name}: lq {case.cu_q.diff().tolist()[:4]} rel_extent {case.rel_extent} "
          f"W {tuple(w.shape)} r {r.dtype}", flush=True)
    out, lse = inkling_fa4_rel_attention_rproj(
        c.q, c.k, c.v, r.to(dev), w.to(dev), c.cu_q, c.cu_k, c.max_q, c.max_k, c.rel_extent,
        causal=c.causal, window_size=c.window_size, softmax_scale=c.scale, return_lse=True,
        bottom_right=bottom_right)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


def _check(got, want):
    out, lse = got
    want_out, want_lse = want
    empty = torch.isnan(want_out.float()).any(-1)
    keep = ~empty
    torch.testing.assert_close(out.float()[keep], want_out.float()[keep], atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(lse.transpose(0, 1)[keep], want_lse.transpose(0, 1)[keep],
                               atol=LSE_ATOL, rtol=0)


def _oracle(case, r, w, bottom_right=False):
    return ref_rel_attn_rproj_with_lse(case.q, case.k, case.v, r, w, case.cu_q, case.cu_k,
                                       case.scale, case.rel_extent, causal=case.causal,
                                       window_left=case.window_or_none, bottom_right=bottom_right)


@pytest.mark.parametrize("r_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rel_extent,width", [(128, 128), (64, 200), (100, 128)])
def test_rproj_ragged_gqa(cuda, r_dtype, rel_extent, width):
    case = testing.make_case("rproj_ragged", [300, 64, 33, 700], [300, 64, 33, 700], 8, 2, 128,
                             torch.bfloat16, seed=41, rel_extent=rel_extent, rel_width=width)
    r, w = _factors(case, width, seed=rel_extent, r_dtype=r_dtype)
    _check(_run(case, r, w, cuda), _oracle(case, r, w))


@pytest.mark.parametrize("head_dim,dtype", [(64, torch.float16), (128, torch.float16),
                                            (64, torch.bfloat16)])
def test_rproj_head_dims_dtypes(cuda, head_dim, dtype):
    case = testing.make_case("rproj_dims", [130, 257], [130, 257], 4, 4, head_dim, dtype, seed=42)
    r, w = _factors(case, 128, seed=3)
    _check(_run(case, r, w, cuda), _oracle(case, r, w))


@pytest.mark.parametrize("causal,window", [(True, 63), (False, None)])
def test_rproj_bottom_right_chunked(cuda, causal, window):
    """128 new tokens over 384 keys, bottom-right: the bias band is live."""
    case = testing.make_case("rproj_chunk", [128] * 4, [384] * 4, 8, 2, 128, torch.bfloat16,
                             seed=43, causal=causal, window_left=-1 if window is None else window)
    r, w = _factors(case, 128, seed=4)
    _check(_run(case, r, w, cuda, bottom_right=True), _oracle(case, r, w, bottom_right=True))


def test_rproj_rank_one_equals_table_path(cuda):
    case = testing.long_prefill(1024, batch=2)
    hq, tq = case.q.shape[1], case.q.shape[0]
    table = case.rel[0].float()
    r = torch.zeros(tq, hq, 16)
    r[:, torch.arange(hq), torch.arange(hq)] = 1.0
    w = torch.zeros(16, table.shape[1])
    w[:hq] = table
    got = _run(case, r, w, cuda)
    c = case.to(cuda)
    out, lse = inkling_fa4_rel_attention(*c.args(), causal=True, softmax_scale=c.scale,
                                         return_lse=True)
    torch.cuda.synchronize()
    torch.testing.assert_close(got[0].float(), out.cpu().float(), atol=1e-2, rtol=1e-2)
    torch.testing.assert_close(got[1], lse.cpu(), atol=1e-5, rtol=0)


@pytest.mark.parametrize("r_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rel_extent", [512, 1024])
def test_rproj_serving_extents(cuda, r_dtype, rel_extent):
    """The serving model's local (512) and global (1024) extents
    (outputs/architecture.md:57-58): sequences shorter than the band, across
    it and longer than it; 256-row query tiles with ragged tails."""
    lens = [1500, 700, 64, 1100, 2100]
    case = testing.make_case("rproj_serving", lens, lens, 8, 2, 128, torch.bfloat16, seed=44,
                             rel_extent=rel_extent, rel_width=rel_extent + 16)
    r, w = _factors(case, rel_extent + 16, seed=rel_extent, r_dtype=r_dtype)
    _check(_run(case, r, w, cuda), _oracle(case, r, w))


@pytest.mark.parametrize("causal,window,bottom_right", [(True, 700, False), (False, -1, True),
                                                        (True, -1, True)])
def test_rproj_long_extent_masks(cuda, causal, window, bottom_right):
    """rel_extent 1024 with a window, bottom-right chunked prefill (300 new
    tokens over 1800 keys) and lq > lk."""
    case = testing.make_case("rproj_masks", [300, 1200, 900], [1800, 1200, 600], 6, 3, 64,
                             torch.float16, seed=45, causal=causal, window_left=window,
                             rel_extent=1024, rel_width=1024)
    r, w = _factors(case, 1024, seed=5)
    _check(_run(case, r, w, cuda, bottom_right), _oracle(case, r, w, bottom_right))


def test_rproj_large_bias_lse(cuda):
    """Bias values of several units (r, W std 1): the hi + lo split keeps the
    projected bias to ~2^-16 relative, so the LSE stays within 1e-3."""
    lens = [1024, 513]
    case = testing.make_case("rproj_big", lens, lens, 4, 4, 128, torch.bfloat16, seed=46,
                             rel_extent=1024, rel_width=1024)
    r, w = _factors(case, 1024, seed=6, std=1.0)
    _check(_run(case, r, w, cuda), _oracle(case, r, w))
