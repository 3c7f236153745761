"""GPU parity of decode over an FP8 (OCP e4m3) KV cache with per-tensor scales.

The oracle runs on the dequantised keys and values (k8 * k_scale, v8 *
v_scale in fp32, exactly what the kernel converts), so the bar is the usual
one: out within atol / rtol 2e-2, lse within 1e-3.  Paged fp8 must match
contiguous fp8 up to the order of the split merge (the same per-step arithmetic,
kv head pairs at d 128, one kv head per wave at d 64; a paged cache streams with
more waves): lse within 1e-5, out within one 16-bit rounding step.
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


def _same(a, b):
    """Paged against contiguous: the same keys and per-step arithmetic, another
    stream-K split."""
    torch.testing.assert_close(a[0].float(), b[0].float(), atol=1e-3, rtol=1e-2)
    torch.testing.assert_close(a[1], b[1], atol=1e-5, rtol=0)


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


@pytest.mark.parametrize("hq,hkv,rel_dtype", [(8, 2, torch.float32), (8, 2, torch.bfloat16),
                                              (4, 4, torch.float16), (6, 2, torch.bfloat16)])
def test_fp8_bottom_right_bias_and_window(cuda, hq, hkv, rel_dtype):
    """Bottom-right fp8 decode with a per-token bias and a left window (kv head
    pairs: the bias gather follows the pair mode's key order)."""
    lens = [5, 130, 700, 2000, 1025]
    case = testing.make_case("fp8_br", [1] * len(lens), lens, hq, hkv, 128, torch.bfloat16,
                             seed=31, causal=True, window_left=300, rel_table=False,
                             rel_std=1.0, rel_dtype=rel_dtype)
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
    _same(got, contiguous)
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


def _fp8_decode_views(case, dev, pad):
    """fp8 decode with K and V passed as views whose head stride is D + pad
    (pad 0: the contiguous cache, whose adjacent kv heads stream in pairs
    when the kv heads are even, D is 128 and a pair holds at most 8 query
    heads; pad 16: every kv head alone)."""
    k8, v8, ks, vs, deq = testing.fp8_kv(case)
    t, hkv, d = k8.shape

    def widen(x):
        if pad == 0:
            return x.to(dev)
        w = torch.zeros(t, hkv, d + pad, dtype=torch.uint8)
        w[:, :, :d] = x.view(torch.uint8)
        return w.view(x.dtype).to(dev)[:, :, :d]

    kk, vv = widen(k8), widen(v8)
    assert kk.stride(1) == d + pad and vv.stride(1) == d + pad
    c = case.to(dev)
    print(f"fp8 decode {case.name}: heads {c.q.shape[1]}/{hkv}, D {d}, head stride {d + pad}",
          flush=True)
    out, lse = inkling_fa4_rel_attention_decode(
        c.q, kk, vv, c.rel, c.cu_q, c.cu_k, c.max_q, c.max_k, c.rel_extent, causal=c.causal,
        window_size=c.window_size, softmax_scale=c.scale, return_lse=True, k_scale=ks,
        v_scale=vs)
    torch.cuda.synchronize()
    return (out.cpu(), lse.cpu()), deq


@pytest.mark.parametrize("hq,hkv", [(4, 2), (8, 2), (6, 2), (16, 4), (8, 8), (16, 2)])
def test_fp8_kv_head_pairs_and_single_heads(cuda, hq, hkv):
    """Adjacent kv heads of a d-128 fp8 cache stream in pairs (a wave reads
    whole rows of both heads; the pair's query heads share the 16 S^T
    columns, each keeping the logits of its own kv head, and PV adds each
    head's Vᵀ times P with the other head's columns zeroed).  Pairs of 2, 4,
    6 and 8 query heads; several pairs (Hkv 4, 8); a group of 8 per kv head
    (16 per pair: streamed one kv head at a time).  The same cache through
    views with a padded head stride streams one kv head per wave; both
    against the oracle on the dequantised K/V."""
    lens = [1, 2, 31, 32, 33, 100, 1000, 3000, 4097]
    case = testing.make_case("fp8_pairs", [1] * len(lens), lens, hq, hkv, 128, torch.bfloat16,
                             seed=hq * 5 + hkv, causal=False, rel_table=False, rel_extent=64,
                             scale=0.1)
    for pad in (0, 16):
        got, deq = _fp8_decode_views(case, cuda, pad)
        _check(got, _oracle(deq))


def test_fp8_pairs_many_short_caches(cuda):
    """150 sequences of 0..99 keys (empty and one-key caches among them) in
    kv head pairs: waves cross many pair segments, the cursor reloads sequence
    chunks, and empty caches own no steps."""
    g = torch.Generator().manual_seed(17)
    lens = torch.randint(0, 100, (150,), generator=g).tolist()
    lens[3] = 0
    lens[70] = 1
    lens[140] = 32
    case = testing.make_case("fp8_short", [1] * 150, lens, 8, 2, 128, torch.bfloat16, seed=18,
                             causal=False)
    got, deq = _fp8_decode(case, cuda)
    live = torch.tensor([n > 0 for n in lens])
    want = _oracle(deq)
    torch.testing.assert_close(got[0][live].float(), want[0][live].float(), atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(got[1][:, live], want[1][:, live], atol=LSE_ATOL, rtol=0)
    assert (got[0][~live].float() == 0).all() and torch.isneginf(got[1][:, ~live]).all()


@pytest.mark.parametrize("block_size", [8, 32])
def test_fp8_paged_pairs_bottom_right_bias(cuda, block_size):
    """kv head pairs of a paged fp8 cache, bottom-right with a per-token bf16 bias
    and a left window: the contiguous pair stream's results up to the merge
    order, and both held to the oracle."""
    lens = [5, 130, 700, 2000, 1025, 33]
    case = testing.make_case("fp8_pbr", [1] * len(lens), lens, 8, 2, 128, torch.bfloat16,
                             seed=34, causal=True, window_left=300, rel_table=False,
                             rel_std=1.0, rel_dtype=torch.bfloat16, rel_extent=512)
    k8, v8, ks, vs, deq = testing.fp8_kv(case)
    pk = testing.paginate(testing.replace(case, k=k8, v=v8), block_size=block_size, seed=5,
                          fill=0.0)
    c, p = case.to(cuda), pk.to(cuda)
    out, lse = inkling_fa4_rel_attention_decode_paged(
        c.q, p.k_cache, p.v_cache, c.rel, c.cu_q, p.seqused_k, p.block_table, c.max_q, c.max_k,
        c.rel_extent, causal=True, window_size=c.window_size, softmax_scale=c.scale,
        return_lse=True, bottom_right=True, k_scale=ks, v_scale=vs)
    torch.cuda.synchronize()
    got = (out.cpu(), lse.cpu())
    contiguous, _ = _fp8_decode(case, cuda, bottom_right=True)
    _same(got, contiguous)
    want = _oracle(deq, bottom_right=True)
    _check(got, want)
    _check(contiguous, want)
