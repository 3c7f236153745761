"""fp32 CPU restatement of Inkling relative-bias attention (test oracle).

Follows the reference's dense per-(sequence, head) algorithm in
src/inkling_fa4/reference.py:19-40:

  for each sequence b (reference.py:21-23) and query head h (:25):
    kv head  kh = h // (Hq // Hkv)                              (:20, :26)
    s[i,j]   = scale * <q_i, k_j>  in fp32                       (:24, :27)
    dist     = i + (Lq - Lk) - j       (local indices)           (:28-31)
    s[i,j]  += rel[qs+i, h, dist]  if 0 <= dist < rel_extent     (:32-35)
               (0 outside the band, NOT clamped)
    mask     causal: keep i >= j  (top-left, local indices)      (:36)
             window: keep i - j <= window_left (left only)       (:37)
    p        = softmax_j(s) in fp32 (all-masked row -> NaN)      (:38)
    out      = p @ v, rounded to q.dtype                         (:39)

The log-sum-exp (natural log, fp32, layout [Hq, total_q]) is an addition:
the reference returns no LSE.  Rows with no visible key get lse = -inf.

TEST INFRASTRUCTURE: imported only by tests, smoke() and the bench's CPU
baseline.  Runs on whatever device its inputs live on (CPU in practice).
"""
import math

import torch


def _lengths(cu):
    c = [int(x) for x in cu.detach().cpu().tolist()]
    return [(c[b], c[b + 1]) for b in range(len(c) - 1)]


@torch.no_grad()
def ref_rel_attn_with_lse(q, k, v, rel_logits, cu_seqlens_q, cu_seqlens_k, scale,
                          rel_extent, causal=True, window_left=None, bottom_right=False):
    """Return (out [Tq,Hq,D] in q.dtype, lse [Hq,Tq] fp32).

    bottom_right=True is an addition with no counterpart in the reference: the
    upstream flash-attn alignment of its serving backend
    (outputs/architecture.md:72, d = (i + sk - sq) - j).  Query i sits at key
    position i + (Lk - Lq) for the bias distance, the causal mask and the
    window.  It equals the reference semantics when Lq == Lk.
    """
    n_q, hq, _ = q.shape
    hkv = k.shape[1]
    if hq % hkv:
        raise ValueError("n_heads must be a multiple of kv_heads")
    group = hq // hkv
    out = torch.zeros_like(q)
    lse = torch.full((hq, n_q), -math.inf, dtype=torch.float32, device=q.device)
    for (q0, q1), (k0, k1) in zip(_lengths(cu_seqlens_q), _lengths(cu_seqlens_k)):
        lq, lk = q1 - q0, k1 - k0
        if lq <= 0:
            continue
        rows = torch.arange(lq, device=q.device).unsqueeze(1)
        cols = torch.arange(lk, device=q.device).unsqueeze(0)
        if bottom_right:
            pos = rows + (lk - lq)          # key position of query i
            dist = pos - cols
        else:
            pos = rows                      # reference.py:36-37 (top-left)
            dist = rows - cols + (lq - lk)  # reference.py:28-31
        band = (dist >= 0) & (dist < rel_extent)
        gather_idx = dist.clamp(min=0, max=rel_extent - 1)
        visible = torch.ones(lq, lk, dtype=torch.bool, device=q.device)
        if causal:
            visible &= pos >= cols
        if window_left is not None:
            visible &= (pos - cols) <= window_left
        for h in range(hq):
            kh = h // group
            qf = q[q0:q1, h].float()
            kf = k[k0:k1, kh].float()
            vf = v[k0:k1, kh].float()
            scores = torch.matmul(qf, kf.transpose(0, 1)) * scale
            table = rel_logits[q0:q1, h].float()
            bias = torch.gather(table, 1, gather_idx) if lk > 0 else scores
            scores = scores + torch.where(band, bias, torch.zeros_like(scores))
            scores = scores.masked_fill(~visible, -math.inf)
            probs = torch.softmax(scores, dim=-1)
            out[q0:q1, h] = torch.matmul(probs, vf).to(out.dtype)
            if lk > 0:
                lse[h, q0:q1] = torch.logsumexp(scores, dim=-1)
    return out, lse


def ref_rel_attn(q, k, v, rel_logits, cu_seqlens_q, cu_seqlens_k, scale, rel_extent,
                 causal=True, window_left=None):
    """Same signature and result as the reference's `ref_rel_attn`
    (src/inkling_fa4/reference.py:4): returns `out` only."""
    return ref_rel_attn_with_lse(q, k, v, rel_logits, cu_seqlens_q, cu_seqlens_k, scale,
                                 rel_extent, causal=causal, window_left=window_left)[0]
