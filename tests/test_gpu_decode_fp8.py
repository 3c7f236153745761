"""GPU parity of decode over an FP8 (OCP e4m3) KV cache with per-tensor scales.

The oracle runs on the dequantised keys and values (k8 * k_scale, v8 *
v_scale in fp32, exactly what the kernel converts), so the bar is the usual
one: out within atol / rtol 2e-2, lse within 1e-3.  Paged fp8 must equal
contiguous fp8 bit for bit.
"""
import pytest
import torch

from inkling_fa4 import (inkling_fa4_rel_attention_decode, inkling_fa4_rel_attention_decode_paged,
                         testing)
from oracle import ref_rel_attn_with_lse

pytestmark = pytest.mark.gpu

ATOL, RTOL, LSE_ATOL = 2e-2, 2e-2, 1e-3


def _fp8_decode(case, dev, bottom_right=False):
    k8, v8, ks, vs, deq = testing.fp8_kv(case)
    c = case.to(dev)
    print(f"fp8 decode {case.name}: batch {c.cu_q.numel() - 1}, heads {c.q.shape[1]}/"
          f"{c.k.shape[1]}, D {c.q.shape[2]}, causal {c.causal}", flush=True)
    out, lse = inkling_fa4_rel_attention_decode(
        c.q, k8.to(dev), v8.to(dev), c.rel, c.cu_q, c.cu_k, c.max_q, c.max_k, c.rel_extent,
        causal=c.causal, window_size=c.window_size, softmax_scale=c.scale, return_lse=True,
        bottom_right=bottom_right, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    return (out.cpu(), lse.cpu()), deq


def _oracle(deq, bottom_right=False):
    return ref_rel_attn_with_lse(deq.q, deq.k, deq.v, deq.rel, deq.cu_q, deq.cu_k, deq.scale,
                                 deq.rel_extent, causal=deq.causal,
                                 window_left=deq.window_or_none, bottom_right=bottom_right)


def _check(got, want):
    torch.testing.assert_close(got[0].float(), want[0].float(), atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(got[1], want[1], atol=LSE_ATOL, rtol=0)


@pytest.mark.parametrize("causal", [False, True])
def test_fp8_decode_batch64(cuda, causal):
    case = testing.decode(causal=causal)
    got, deq = _fp8_decode(case, cuda)
    _check(got, _oracle(deq))


@pytest.mark.parametrize("hq,hkv", [(8, 2), (4, 4), (8, 1), (6, 2)])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp8_gqa_head_dims_dtypes(cuda, hq, hkv, head_dim, dtype):
    lens = [1, 2, 31, 32, 33, 100, 1000, 3000]
    case = testing.make_case("fp8_gqa", [1] * len(lens), lens, hq, hkv, head_dim, dtype,
                             seed=hq * 7 + hkv, causal=False, rel_table=False, scale=0.1)
    got, deq = _fp8_decode(case, cuda)
    _check(got, _oracle(deq))


def test_fp8_bottom_right_bias_and_window(cuda):
    lens = [5, 130, 700, 2000]
    case = testing.make_case("fp8_br", [1] * len(lens), lens, 8, 2, 128, torch.bfloat16, seed=31,
                             causal=True, window_left=300, rel_table=False, rel_std=1.0)
    got, deq = _fp8_decode(case, cuda, bottom_right=True)
    _check(got, _oracle(deq, bottom_right=True))


@pytest.mark.parametrize("block_size,head_dim", [(16, 128), (8, 128), (16, 64), (64, 64)])
def test_fp8_paged_equals_contiguous(cuda, block_size, head_dim):
    lens = [1, 17, 300, 1025, 4000]
    case = testing.make_case("fp8_paged", [1] * len(lens), lens, 8, 2, head_dim, torch.bfloat16,
                             seed=32, causal=False)
    k8, v8, ks, vs, deq = testing.fp8_kv(case)
    pk = testing.paginate(testing.replace(case, k=k8, v=v8), block_size=block_size, seed=3,
                          fill=0.0)
    c, p = case.to(cuda), pk.to(cuda)
    out, lse = inkling_fa4_rel_attention_decode_paged(
        c.q, p.k_cache, p.v_cache, c.rel, c.cu_q, p.seqused_k, p.block_table, c.max_q, c.max_k,
        c.rel_extent, causal=False, softmax_scale=c.scale, return_lse=True, k_scale=ks,
        v_scale=vs)
    torch.cuda.synchronize()
    got = (out.cpu(), lse.cpu())
    contiguous, _ = _fp8_decode(case, cuda)
    assert torch.equal(got[0], contiguous[0]) and torch.equal(got[1], contiguous[1])
    _check(got, _oracle(deq))


@pytest.mark.parametrize("head_dim", [64, 128])
def test_fp8_gqa_group_16(cuda, head_dim):
    lens = [40, 50, 1000, 4100]
    case = testing.make_case("fp8_g16", [1] * len(lens), lens, 16, 1, head_dim, torch.bfloat16,
                             seed=1, causal=False, scale=0.1)
    got, deq = _fp8_decode(case, cuda)
    _check(got, _oracle(deq))


def test_fp8_rejects_what_it_does_not_serve(cuda):
    case = testing.make_case("fp8_g32", [1, 1], [40, 50], 32, 1, 128, torch.bfloat16, seed=1,
                             causal=False)
    with pytest.raises(ValueError):
        _fp8_decode(case, cuda)
    case = testing.make_case("fp8_prefill", [4], [40], 8, 2, 128, torch.bfloat16, seed=1,
                             causal=False)
    with pytest.raises(ValueError):
        _fp8_decode(case, cuda)


@pytest.mark.parametrize("keys", [32768, 131072])
def test_fp8_one_sequence_split_combine(cuda, keys):
    """One sequence of an fp8 cache over 2048 waves: ~1,025 partials per
    (head, sequence) at 32K keys and 128K, merged by four combine workgroups
    per (head, sequence), each over a quarter of the row, in several rounds of
    loads.  Against the oracle on the dequantised K/V."""
    case = testing.make_case("fp8_split", [1], [keys], 8, 2, 128, torch.bfloat16, seed=33,
                             causal=False)
    print(f"fp8 one sequence of {keys} keys", flush=True)
    got, deq = _fp8_decode(case, cuda)
    _check(got, _oracle(deq))
