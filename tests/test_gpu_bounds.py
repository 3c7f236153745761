"""Prefill reads nothing outside a sequence's K/V rows.

K and V are views into larger NaN-filled allocations: the rows of a sequence
that holds keys but no queries are NaN, and so are the rows past the end of the
tensors (past cu_seqlens_k[-1]).  Sequence lengths are not multiples of the
64-key KV tile, so every sequence with queries ends in a partial tile whose
rows past its last key lie in NaN memory.  Those rows must read as zero (the
tile DMA's range check), so that masked keys contribute exactly nothing: any
read of them would turn the output into NaN through 0 * NaN in the P.V
product.  The outputs of the sequences with queries are compared with the
oracle (out atol / rtol 2e-2, lse 1e-3), for unsplit and split-KV calls, at
head_dim 64 and 128, causal and not, and for the fused projection.
"""
import pytest
import torch

from inkling_fa4 import _abi, inkling_fa4_rel_attention, inkling_fa4_rel_attention_rproj, testing
from oracle import ref_rel_attn_rproj_with_lse, ref_rel_attn_with_lse

pytestmark = pytest.mark.gpu

ATOL, RTOL, LSE_ATOL = 2e-2, 2e-2, 1e-3
PAD_ROWS = 128  # NaN rows after the tensors' last row

# sequences 1 and 3 hold keys and no queries: their rows are NaN
LENS_Q = [100, 0, 37, 0, 171]
LENS_K = [100, 70, 37, 45, 171]


def _nan_views(t, dev):
    """t on the device as the leading rows of a NaN-filled allocation, with the
    rows of the query-less sequences set to NaN too."""
    big = torch.full((t.shape[0] + PAD_ROWS,) + tuple(t.shape[1:]), float("nan"),
                     dtype=t.dtype, device=dev)
    big[:t.shape[0]] = t.to(dev)
    view = big[:t.shape[0]]
    starts = [0]
    for n in LENS_K:
        starts.append(starts[-1] + n)
    for b, lq in enumerate(LENS_Q):
        if lq == 0:
            view[starts[b]:starts[b + 1]] = float("nan")
    return view


def _case(head_dim, causal, dtype, seed):
    case = testing.make_case("nan_pad", LENS_Q, LENS_K, 8, 2, head_dim, dtype, seed=seed,
                             causal=causal, rel_table=False, rel_dtype=torch.bfloat16,
                             rel_std=1.0, rel_extent=96)
    # the oracle sees the same NaN rows (they belong to sequences without queries)
    starts = case.cu_k.tolist()
    for b, lq in enumerate(LENS_Q):
        if lq == 0:
            case.k[starts[b]:starts[b + 1]] = float("nan")
            case.v[starts[b]:starts[b + 1]] = float("nan")
    return case


def _check(case, out, lse, want_out, want_lse):
    rows = torch.zeros(case.q.shape[0], dtype=torch.bool)
    cq = case.cu_q.tolist()
    for b, lq in enumerate(LENS_Q):
        rows[cq[b]:cq[b] + lq] = True
    assert torch.isfinite(out.float()).all(), "a read outside the sequence reached the output"
    torch.testing.assert_close(out.float()[rows], want_out.float()[rows], atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(lse[:, rows], want_lse[:, rows], atol=LSE_ATOL, rtol=0)


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("head_dim,dtype", [(128, torch.bfloat16), (64, torch.float16)])
def test_prefill_nan_outside_sequences(cuda, split, causal, head_dim, dtype):
    case = _case(head_dim, causal, dtype, seed=91)
    print(f"nan-padded K/V: d {head_dim} {dtype} causal {causal} split {split}", flush=True)
    k, v = _nan_views(case.k, cuda), _nan_views(case.v, cuda)
    flags = _abi.IFA4_FLAG_SPLIT_KV_2 if split else 0
    out, lse = inkling_fa4_rel_attention(
        case.q.to(cuda), k, v, case.rel.to(cuda), case.cu_q.to(cuda), case.cu_k.to(cuda),
        case.max_q, case.max_k, case.rel_extent, causal=causal, softmax_scale=case.scale,
        return_lse=True, _flags=flags)
    torch.cuda.synchronize()
    want_out, want_lse = ref_rel_attn_with_lse(case.q, case.k, case.v, case.rel, case.cu_q,
                                               case.cu_k, case.scale, case.rel_extent,
                                               causal=causal)
    _check(case, out.cpu(), lse.cpu(), want_out, want_lse)


@pytest.mark.parametrize("causal", [True, False])
def test_rproj_nan_outside_sequences(cuda, causal):
    case = _case(128, causal, torch.bfloat16, seed=92)
    print(f"nan-padded K/V, fused projection: causal {causal}", flush=True)
    g = torch.Generator().manual_seed(93)
    r = 0.3 * torch.randn(case.q.shape[0], case.q.shape[1], 16, generator=g)
    w = 0.3 * torch.randn(16, case.rel_extent, generator=g)
    k, v = _nan_views(case.k, cuda), _nan_views(case.v, cuda)
    out, lse = inkling_fa4_rel_attention_rproj(
        case.q.to(cuda), k, v, r.to(cuda), w.to(cuda), case.cu_q.to(cuda), case.cu_k.to(cuda),
        case.max_q, case.max_k, case.rel_extent, causal=causal, softmax_scale=case.scale,
        return_lse=True)
    torch.cuda.synchronize()
    want_out, want_lse = ref_rel_attn_rproj_with_lse(case.q, case.k, case.v, r, w, case.cu_q,
                                                     case.cu_k, case.scale, case.rel_extent,
                                                     causal=causal)
    _check(case, out.cpu(), lse.cpu(), want_out, want_lse)
