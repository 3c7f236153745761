"""In-wave online-softmax rescale of the decode stream, on every cache format.

A decode wave streams an equal contiguous range of P = ceil(T / W) 32-key
steps over the (sequence, kv head) caches laid end to end (T steps, W waves).
Inside its range a wave keeps one running max per query head and rescales
its accumulator O whenever that max grows by more than 8 log2 units after
the wave's first step of a cache.  The keys here carry a sawtooth gain along
each sequence (0.05 -> 5 over every 64 keys), so every odd 32-key step of a
cache lies tens of log2 units above the even step before it: a wave whose
range holds an even step and the next odd step of one cache rescales O.

Before each GPU call the test rebuilds the wave partition on the host for
the wave count the tile table uses (896 for a contiguous 16-bit cache, 2048
for a paged or fp8 one, 1024 / 1536 for a contiguous / paged fp8 cache of d 128
whose adjacent kv heads stream in pairs, a pair's two caches then being one
segment) and
asserts that P >= 2 and that some wave's range grows one head's max by more
than 8 log2 units after its first step of a cache.  The results are then compared with the oracle (fp8: on the
dequantised K/V): out within atol/rtol 2e-2, lse within 1e-3.  Reference
semantics: src/inkling_fa4/reference.py:38-39 (softmax over all keys, then PV).
"""
import math
from dataclasses import replace

import pytest
import torch

from inkling_fa4 import (inkling_fa4_rel_attention_decode,
                         inkling_fa4_rel_attention_decode_paged, testing)
from oracle import ref_rel_attn_paged_with_lse, ref_rel_attn_with_lse

ATOL, RTOL, LSE_ATOL = 2e-2, 2e-2, 1e-3
STEP = 32
RESCALE_LOG2 = 8.0


def _view(fmt, head_dim):
    """(waves, kv heads streamed in pairs) of a cache format, as the tile table
    streams the 8 / 2-head cases here."""
    if fmt == "bf16":
        return 896, False
    if fmt == "fp8" and head_dim == 128:
        return 1024, True
    if fmt == "fp8_paged" and head_dim == 128:
        return 1536, True
    return 2048, False


FORMATS = ("bf16", "paged", "fp8", "fp8_paged")
# the table's small-call caps: steps per wave; waves per cache (or one per
# PART_STEPS steps of a longer cache)
MIN_STEPS, MAX_PARTS, PART_STEPS = 2, 128, 2
LENS_K = [30000, 1, 7000, 16384, 33, 12000, 64, 20000, 9001, 5000, 31000, 2500]


def _sawtooth(case, period=64, lo=0.05, hi=5.0):
    """Key j of each sequence scaled by lo + (hi - lo) * (j % period) / (period - 1)."""
    cu = case.cu_k.tolist()
    f = torch.ones(case.k.shape[0])
    ramp = torch.linspace(lo, hi, period)
    for b in range(len(cu) - 1):
        n = cu[b + 1] - cu[b]
        j = torch.arange(n)
        f[cu[b]:cu[b + 1]] = ramp[j % period]
    return replace(case, k=(case.k.float() * f[:, None, None]).to(case.k.dtype))


def _step_maxima(case, pair=False):
    """Per segment, (sequence, kv head) or with `pair` (sequence, pair of kv
    heads): [steps, query heads] maxima of the logits (log2 units) of each
    32-key step, non-causal top-left decode (every key visible)."""
    cq, ck = case.cu_q.tolist(), case.cu_k.tolist()
    hq, hkv = case.q.shape[1], case.k.shape[1]
    g = hq // hkv
    per = 2 if pair else 1
    out = []
    for b in range(len(ck) - 1):
        q = case.q[cq[b]].float()  # [Hq, D]
        k = case.k[ck[b]:ck[b + 1]].float()  # [L, Hkv, D]
        n = k.shape[0]
        for kp in range(hkv // per):
            if n == 0:
                out.append(torch.zeros(0, per * g))
                continue
            s = torch.cat([(k[:, kh] @ q[kh * g:(kh + 1) * g].T)
                           for kh in range(per * kp, per * kp + per)], 1)
            s = s * case.scale * math.log2(math.e)
            steps = (n + STEP - 1) // STEP
            pad = torch.full((steps * STEP - n, per * g), -math.inf)
            out.append(torch.cat([s, pad]).view(steps, STEP, per * g).amax(1))
    return out


def _rescale_waves(maxima, waves, max_k, batch, hkv):
    """(P, number of waves whose range raises one head's max by more than the
    threshold after the wave's first step of a cache) for a stream of `waves`
    persistent waves, capped as the library caps them: at least MIN_STEPS steps
    of the call's step bound per wave, at most max(MAX_PARTS, steps of the
    longest cache / PART_STEPS) waves per cache."""
    seg_steps = [m.shape[0] for m in maxima]
    total = sum(seg_steps)
    per_seg = (max_k + STEP - 1) // STEP
    bound = batch * hkv * per_seg
    w = min(waves, -(-bound // MIN_STEPS),
            batch * hkv * max(MAX_PARTS, -(-per_seg // PART_STEPS)))
    p = (total + w - 1) // w
    starts, acc = [], 0
    for n in seg_steps:
        starts.append(acc)
        acc += n
    hits = 0
    for wave in range(w):
        g0, g1 = wave * p, min(wave * p + p, total)
        hit = False
        for seg, n in enumerate(seg_steps):
            a, e = max(g0, starts[seg]), min(g1, starts[seg] + n)
            if e - a < 2:
                continue
            m = maxima[seg][a - starts[seg]:e - starts[seg]]
            if bool(((m[1:].cummax(0).values - m[0]) > RESCALE_LOG2).any()):
                hit = True
                break
        hits += hit
    return p, hits


def _case(head_dim, seed):
    case = testing.make_case("rescale", [1] * len(LENS_K), LENS_K, 8, 2, head_dim,
                             torch.bfloat16, seed=seed, causal=False, scale=0.3)
    return _sawtooth(case)


def _assert_drives_rescale(case, fmt, head_dim):
    w, pair = _view(fmt, head_dim)
    maxima = _step_maxima(case, pair)
    segs_per_seq = case.k.shape[1] // (2 if pair else 1)
    p, hits = _rescale_waves(maxima, w, case.max_k, len(LENS_K), segs_per_seq)
    print(f"{fmt} d{head_dim}, waves {w}: {p} steps per wave, {hits} waves rescale inside "
          f"their range", flush=True)
    assert p >= 2 and hits > 0


def _compare(out, lse, want):
    want_out, want_lse = want
    assert not torch.isnan(want_out).any()
    torch.testing.assert_close(out.cpu().float(), want_out.float(), atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(lse.cpu(), want_lse, atol=LSE_ATOL, rtol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("head_dim", [128, 64])
def test_decode_in_wave_rescale(cuda, fmt, head_dim):
    case = _case(head_dim, seed=40 + head_dim)
    fp8 = fmt.startswith("fp8")
    if fp8:
        k8, v8, ks, vs, deq = testing.fp8_kv(case)
        _assert_drives_rescale(deq, fmt, head_dim)
        want = ref_rel_attn_with_lse(deq.q, deq.k, deq.v, deq.rel, deq.cu_q, deq.cu_k,
                                     deq.scale, deq.rel_extent, causal=False)
        kk, vv, kw = k8, v8, dict(k_scale=ks, v_scale=vs)
    else:
        _assert_drives_rescale(case, fmt, head_dim)
        want = None
        kk, vv, kw = case.k, case.v, {}
    c = case.to(cuda)
    print(f"decode rescale {fmt} d{head_dim}: {len(LENS_K)} caches, "
          f"{sum(LENS_K)} keys", flush=True)
    if fmt.endswith("paged"):
        pk = testing.paginate(replace(case, k=kk, v=vv), block_size=16, seed=head_dim,
                              fill=0.0)
        p = pk.to(cuda)
        out, lse = inkling_fa4_rel_attention_decode_paged(
            c.q, p.k_cache, p.v_cache, c.rel, c.cu_q, p.seqused_k, p.block_table, c.max_q,
            c.max_k, c.rel_extent, causal=False, softmax_scale=c.scale, return_lse=True, **kw)
        if want is None:
            want = ref_rel_attn_paged_with_lse(case.q, pk.k_cache, pk.v_cache, case.rel,
                                               case.cu_q, pk.seqused_k, pk.block_table,
                                               case.scale, case.rel_extent, causal=False)
    else:
        out, lse = inkling_fa4_rel_attention_decode(
            c.q, kk.to(cuda), vv.to(cuda), c.rel, c.cu_q, c.cu_k, c.max_q, c.max_k,
            c.rel_extent, causal=False, softmax_scale=c.scale, return_lse=True, **kw)
        if want is None:
            want = ref_rel_attn_with_lse(case.q, case.k, case.v, case.rel, case.cu_q, case.cu_k,
                                         case.scale, case.rel_extent, causal=False)
    torch.cuda.synchronize()
    _compare(out, lse, want)


@pytest.mark.parametrize("head_dim", [128, 64])
def test_sawtooth_case_drives_rescale_on_host(head_dim):
    """CPU side of the GPU test: the case and its fp8 copy drive the rescale."""
    case = _case(head_dim, seed=40 + head_dim)
    deq = testing.fp8_kv(case)[4]
    for fmt in FORMATS:
        _assert_drives_rescale(deq if fmt.startswith("fp8") else case, fmt, head_dim)


def test_partition_model_detects_planted_flat_keys():
    """The host partition check itself: with no sawtooth (plain N(0,1) keys at
    a small scale) no wave sees its max grow by 8 log2 units, so the check
    would fail a case that does not drive the rescale."""
    case = testing.make_case("flat", [1] * len(LENS_K), LENS_K, 8, 2, 64, torch.bfloat16,
                             seed=3, causal=False, scale=1.0 / 64)
    p, hits = _rescale_waves(_step_maxima(case), 2048, case.max_k, len(LENS_K), 2)
    assert p >= 2 and hits == 0
