"""GPU parity of the prefill kernel against the fp32 oracle.

Tolerances (from the operator's contract): out within atol 2e-2 (rtol 2e-2,
as the reference's own tests) for bf16/fp16; lse within 1e-3 absolute.
Inputs are seeded and identical bit for bit on both sides (the oracle upcasts
the device-dtype values).  Large workloads are checked on a subset of
(sequence, head) pairs against the oracle and, everywhere, through
size-independent properties.
"""
import math

import pytest
import torch

import golden
from inkling_fa4 import (inkling_fa4_rel_attention, inkling_fa4_rel_attention_kv_pruned_triton,
                         inkling_fa4_rel_attention_triton, testing)
from inkling_fa4._abi import IFA4_FLAG_NO_PRUNE
from oracle import ref_rel_attn, ref_rel_attn_with_lse

pytestmark = pytest.mark.gpu

ATOL, RTOL, LSE_ATOL = 2e-2, 2e-2, 1e-3


def _run(case, dev, **kw):
    c = case.to(dev)
    out, lse = inkling_fa4_rel_attention(*c.args(), causal=c.causal, window_size=c.window_size,
                                         softmax_scale=c.scale, return_lse=True, **kw)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


def _oracle(case):
    return ref_rel_attn_with_lse(case.q, case.k, case.v, case.rel, case.cu_q, case.cu_k,
                                 case.scale, case.rel_extent, causal=case.causal,
                                 window_left=case.window_or_none)


def _check(out, lse, want_out, want_lse, rows=None):
    if rows is not None:
        out, want_out = out[rows], want_out[rows]
        lse, want_lse = lse[:, rows], want_lse[:, rows]
    torch.testing.assert_close(out.float(), want_out.float(), atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(lse, want_lse, atol=LSE_ATOL, rtol=0)


def test_prefill_s64_fp16_d64(cuda):
    case = testing.prefill_s64()
    out, lse = _run(case, cuda)
    _check(out, lse, *_oracle(case))


@pytest.mark.parametrize("scale", ["1/D", "1/sqrtD"])
def test_ragged_varlen_gqa(cuda, scale):
    case = testing.ragged_varlen(scale=(1 / 128 if scale == "1/D" else 1 / math.sqrt(128)))
    out, lse = _run(case, cuda)
    _check(out, lse, *_oracle(case))


@pytest.mark.parametrize("scale", ["1/D", "1/sqrtD"])
def test_window_chunked(cuda, scale):
    case = testing.window_chunked(scale=(1 / 128 if scale == "1/D" else 1 / math.sqrt(128)))
    out, lse = _run(case, cuda)
    _check(out, lse, *_oracle(case))


def test_long_prefill_s1024_full(cuda):
    case = testing.long_prefill(1024)
    out, lse = _run(case, cuda)
    _check(out, lse, *_oracle(case))


def _sub_case(case, b, heads=None):
    """Sequence b of a packed case as its own one-sequence case; with `heads`
    = (first, last) only q heads first/last and their kv heads are kept."""
    cq, ck = case.cu_q.tolist(), case.cu_k.tolist()
    q0, q1, k0, k1 = cq[b], cq[b + 1], ck[b], ck[b + 1]
    q, k, v, rel = case.q[q0:q1], case.k[k0:k1], case.v[k0:k1], case.rel[q0:q1]
    if heads is not None:
        group = q.shape[1] // k.shape[1]
        hs = list(heads)
        q, rel = q[:, hs], rel[:, hs]
        k, v = k[:, [h // group for h in hs]], v[:, [h // group for h in hs]]
    return testing.Case(name=f"{case.name}[{b}]", q=q, k=k, v=v, rel=rel,
                        cu_q=torch.tensor([0, q1 - q0], dtype=torch.int32),
                        cu_k=torch.tensor([0, k1 - k0], dtype=torch.int32),
                        max_q=q1 - q0, max_k=k1 - k0, rel_extent=case.rel_extent,
                        causal=case.causal, window_left=case.window_left, scale=case.scale)


@pytest.mark.parametrize("seq_len", [2048, 4096])
def test_long_prefill_full_batch(cuda, seq_len):
    """The headline workload (batch 8, Hq 8 / Hkv 2, d 128, rel 128, causal) in
    full: every (sequence, head) pair of out and lse against the oracle."""
    case = testing.long_prefill(seq_len)
    out, lse = _run(case, cuda)
    _check(out, lse, *_oracle(case))


def test_long_prefill_s8192_sampled_sequences(cuda):
    """S 8192: full batch on the GPU; the first and last head of sequence 7 (one
    of each kv head) re-computed by the oracle, the rest checked finite."""
    case = testing.long_prefill(8192)
    out, lse = _run(case, cuda)
    assert torch.isfinite(out.float()).all()
    assert torch.isfinite(lse).all()
    cq = case.cu_q.tolist()
    hq = case.q.shape[1]
    heads = (0, hq - 1)
    b = 7
    sub = _sub_case(case, b, heads)
    want_out, want_lse = _oracle(sub)
    rows = slice(cq[b], cq[b + 1])
    torch.testing.assert_close(out[rows][:, list(heads)].float(), want_out.float(),
                               atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(lse[list(heads)][:, rows], want_lse, atol=LSE_ATOL, rtol=0)


# ---- the reference's 14 test cases (tests/test_correctness.py:22-75), seeded -------------

HEAD_CONFIGS = [(4, 4), (8, 2)]


def _ref_case(lens_q, lens_k, hq, hkv, rel_ext, seed, window=-1):
    # rel_logits per token [Tq, Hq, R] ~ N(0,1) bf16, as make_case
    # (tests/test_correctness.py:11-20); scale 1/HEAD_DIM
    return testing.make_case("ref", lens_q, lens_k, hq, hkv, 128, torch.bfloat16, seed=seed,
                             rel_extent=rel_ext, rel_table=False, rel_dtype=torch.bfloat16,
                             rel_std=1.0, window_left=window, scale=1 / 128)


def _ref_check(case, dev):
    c = case.to(dev)
    got = inkling_fa4_rel_attention_triton(*c.args(), window_size=c.window_size)
    want = ref_rel_attn(case.q, case.k, case.v, case.rel, case.cu_q, case.cu_k, 1.0 / 128,
                        case.rel_extent, window_left=case.window_or_none)
    torch.testing.assert_close(got.float().cpu(), want.float(), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("hq,hkv", HEAD_CONFIGS)
@pytest.mark.parametrize("seq_len", [64, 128])
def test_ref_prefill_basic(cuda, hq, hkv, seq_len):
    _ref_check(_ref_case([seq_len], [seq_len], hq, hkv, 1024, seed=100 + seq_len), cuda)


@pytest.mark.parametrize("hq,hkv", HEAD_CONFIGS)
def test_ref_ragged(cuda, hq, hkv):
    _ref_check(_ref_case([64, 33, 17], [64, 33, 17], hq, hkv, 1024, seed=101), cuda)


@pytest.mark.parametrize("hq,hkv", HEAD_CONFIGS)
def test_ref_long_ctx(cuda, hq, hkv):
    _ref_check(_ref_case([512], [512], hq, hkv, 128, seed=102), cuda)


@pytest.mark.parametrize("hq,hkv", HEAD_CONFIGS)
def test_ref_sliding_window(cuda, hq, hkv):
    _ref_check(_ref_case([128], [128], hq, hkv, 64, seed=103, window=63), cuda)


@pytest.mark.parametrize("hq,hkv", HEAD_CONFIGS)
def test_ref_chunked(cuda, hq, hkv):
    _ref_check(_ref_case([128], [256], hq, hkv, 1024, seed=104), cuda)


@pytest.mark.parametrize("hq,hkv", HEAD_CONFIGS)
def test_ref_decode_through_prefill(cuda, hq, hkv):
    _ref_check(_ref_case([1], [128], hq, hkv, 1024, seed=105), cuda)


# ---- golden vectors of the reference oracle, on the GPU ----------------------------------

@pytest.mark.parametrize("name", ["prefill_s64_fp16_d64", "ragged_114_bf16_d128"])
def test_golden_vectors_on_gpu(cuda, name):
    d = golden.load(name)
    dev = cuda
    rel = d["rel"]
    rel = rel[0].to(dev).unsqueeze(0).expand(rel.shape) if rel.stride(0) == 0 else rel.to(dev)
    cq, ck = d["cu_seqlens_q"], d["cu_seqlens_k"]
    lens_q = (cq[1:] - cq[:-1]).tolist()
    lens_k = (ck[1:] - ck[:-1]).tolist()
    out = inkling_fa4_rel_attention(d["q"].to(dev), d["k"].to(dev), d["v"].to(dev), rel,
                                    cq.to(dev), ck.to(dev), max(lens_q), max(lens_k),
                                    d["rel_extent"], causal=d["causal"],
                                    window_size=(d["window_left"] if d["window_left"] is not None
                                                 else -1, 0),
                                    softmax_scale=d["scale"])
    torch.testing.assert_close(out.float().cpu(), d["out"].float(), atol=ATOL, rtol=RTOL)


# ---- semantics corners -------------------------------------------------------------------

@pytest.mark.parametrize("causal,window", [(False, -1), (False, 40), (True, 17), (True, 0)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_masks_and_dtypes(cuda, causal, window, dtype):
    case = testing.make_case("corners", [200, 77, 1, 129], [200, 300, 64, 129], 6, 2, 128, dtype,
                             seed=7, rel_extent=96, rel_width=100, causal=causal,
                             window_left=window, rel_table=False, scale=0.09)
    out, lse = _run(case, cuda)
    want_out, want_lse = _oracle(case)
    _check(out, lse, want_out, want_lse)


@pytest.mark.parametrize("head_dim", [64, 128])
def test_lq_greater_than_lk_and_empty_rows(cuda, head_dim):
    """Lq > Lk with a window: some rows see no key.  The kernel writes out = 0
    and lse = -inf there (the oracle gives NaN); other rows match."""
    case = testing.make_case("empty_rows", [150, 40], [70, 40], 4, 4, head_dim, torch.bfloat16,
                             seed=8, rel_extent=128, causal=True, window_left=3, rel_table=False)
    out, lse = _run(case, cuda)
    want_out, want_lse = _oracle(case)
    empty = torch.isnan(want_out.float()).any(-1)  # [Tq, Hq]
    assert empty.any()
    assert (out.float()[empty] == 0).all()
    assert torch.isneginf(lse.transpose(0, 1)[empty]).all()
    keep = ~empty
    torch.testing.assert_close(out.float()[keep], want_out.float()[keep], atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(lse.transpose(0, 1)[keep], want_lse.transpose(0, 1)[keep],
                               atol=LSE_ATOL, rtol=0)


def test_pruning_is_bit_invariant(cuda):
    """Skipping fully-masked KV tiles changes nothing, bit for bit."""
    case = testing.make_case("prune", [700, 333], [700, 900], 8, 2, 128, torch.bfloat16, seed=9,
                             causal=True, window_left=150)
    a = _run(case, cuda)
    b = _run(case, cuda, _flags=IFA4_FLAG_NO_PRUNE)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_stride0_table_equals_materialised(cuda):
    case = testing.ragged_varlen()
    a = _run(case, cuda)
    mat = testing.Case(**{**case.__dict__, "rel": case.rel.contiguous()})
    b = _run(mat, cuda)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_strided_views_and_kv_pruned_alias(cuda):
    """q/k/v as head-sliced views of wider buffers; the kv_pruned name runs
    the same kernel."""
    case = testing.ragged_varlen(seed=21)
    dev = cuda
    qw = torch.zeros(case.q.shape[0], 10, 128, dtype=case.q.dtype)
    qw[:, 1:9] = case.q
    kw = torch.zeros(case.k.shape[0], 5, 128, dtype=case.k.dtype)
    kw[:, 2:4] = case.k
    vw = torch.zeros_like(kw)
    vw[:, 3:5] = case.v
    c = case.to(dev)
    got = inkling_fa4_rel_attention_kv_pruned_triton(
        qw.to(dev)[:, 1:9], kw.to(dev)[:, 2:4], vw.to(dev)[:, 3:5], c.rel, c.cu_q, c.cu_k,
        c.max_q, c.max_k, c.rel_extent, softmax_scale=c.scale)
    want = inkling_fa4_rel_attention(*c.args(), softmax_scale=c.scale)
    assert torch.equal(got.cpu(), want.cpu())


def test_rejects_bad_arguments(cuda):
    case = testing.ragged_varlen().to(cuda)
    with pytest.raises(ValueError):
        inkling_fa4_rel_attention(*case.args(), head_dim=64)
    with pytest.raises(RuntimeError):
        inkling_fa4_rel_attention(case.q.float(), case.k.float(), case.v.float(), *case.args()[3:])
    with pytest.raises(RuntimeError):  # rel narrower than rel_extent
        inkling_fa4_rel_attention(*case.args()[:8], 512)


def test_repeat_runs_are_deterministic(cuda):
    case = testing.window_chunked(seed=31)
    a = _run(case, cuda)
    b = _run(case, cuda)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
