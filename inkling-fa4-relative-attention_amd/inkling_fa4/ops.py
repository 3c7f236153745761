"""Python operator API of Inkling relative-bias flash attention on MI355X.

Drop-in for the reference's Triton wrappers, same names and positional
signatures:

  inkling_fa4_rel_attention_triton            src/inkling_fa4/triton_kernel.py:84-107
  inkling_fa4_rel_attention_kv_pruned_triton  src/inkling_fa4/triton_kernel_kv_pruned.py:210-279
  inkling_fa4_rel_attention_decode_triton     src/inkling_fa4/triton_kernel_decode.py:127-170

plus the same entry points under names without the `_triton` suffix, and
`inkling_fa4_rel_attention_decode_paged` for a paged KV cache (block tables),
the format of the serving caller (outputs/architecture.md:117-120), and
`inkling_fa4_rel_attention_rproj` with the bias computed in the kernel from the
RelLogitsProj factors (outputs/architecture.md:24,52-54).

Differences from the reference wrappers (all deliberate):
  * one kernel launch for the whole batch and no host synchronisation (the
    reference reads every cu_seqlens entry to the host, triton_kernel.py:95);
    `max_seqlen_q/k` must therefore bound every sequence length;
  * keyword-only `softmax_scale` (default 1/head_dim, what the reference
    prefill kernel hard-codes at triton_kernel.py:55) and `return_lse`
    (returns (out, lse) with lse [n_heads, total_q] fp32, natural log);
  * `head_dim`, `n_heads`, `kv_heads` default to the tensor shapes; an explicit
    value that disagrees with the shapes raises (the reference reads out of
    bounds, triton_kernel.py:33-37);
  * `window_size[1]` is accepted and ignored, as in the reference
    (triton_kernel.py:105 passes only window_size[0]);
  * `arch` is accepted and ignored: gfx950 has one tile table;
  * a row with no visible key yields out = 0 and lse = -inf;
  * shapes, dtypes, strides and sizes are validated on the host and errors
    raise; the contents of cu_seqlens stay on the device and are not checked
    there against the contract (non-decreasing, from 0, ending within the
    tensors), but each sequence's range is clamped to the tensors' rows, so a
    malformed array yields unspecified results for its sequences, never an
    access outside the tensors.  Decode additionally needs cu_seqlens_q =
    arange(batch + 1): rows of a sequence with another query count get
    out = 0 and lse = -inf.
The decode entry point uses the same default scale as prefill (1/head_dim);
the reference decode kernel uses 1/sqrt(head_dim)
(triton_kernel_decode.py:57), inconsistent with its prefill kernel.
"""
import math

import torch

from . import _abi
from ._native import ops as _ops


def _resolve(q, k, n_heads, kv_heads, head_dim, softmax_scale):
    if q.dim() != 3 or k.dim() != 3:
        raise ValueError("q and k must be [tokens, heads, head_dim]")
    hq, d = q.shape[1], q.shape[2]
    hkv = k.shape[1]
    if n_heads is not None and n_heads != hq:
        raise ValueError(f"n_heads={n_heads} disagrees with q.shape[1]={hq}")
    if kv_heads is not None and kv_heads != hkv:
        raise ValueError(f"kv_heads={kv_heads} disagrees with k.shape[1]={hkv}")
    if head_dim is not None and head_dim != d:
        raise ValueError(f"head_dim={head_dim} disagrees with q.shape[-1]={d}")
    if hq % hkv:
        raise ValueError(f"n_heads={hq} is not a multiple of kv_heads={hkv}")
    scale = (1.0 / d) if softmax_scale is None else float(softmax_scale)
    return scale


_FLAG_BOTTOM_RIGHT = 0x2  # IFA4_FLAG_BOTTOM_RIGHT


def _flag_bits(bottom_right, extra=0):
    return int(extra) | (_FLAG_BOTTOM_RIGHT if bottom_right else 0)


def _window_left(window_size):
    if window_size is None:
        return -1
    left = int(window_size[0])
    return left if left >= 0 else -1


@torch.no_grad()
def inkling_fa4_rel_attention(q, k, v, rel_logits, cu_seqlens_q, cu_seqlens_k,
                              max_seqlen_q, max_seqlen_k, rel_extent, causal=True,
                              window_size=(-1, -1), n_heads=None, kv_heads=None,
                              head_dim=None, arch=None, *, softmax_scale=None,
                              return_lse=False, bottom_right=False, _flags=0):
    """Varlen / GQA / chunked / sliding-window prefill forward.

    q [total_q, Hq, D], k/v [total_k, Hkv, D] (bf16 or fp16, last dim contiguous),
    rel_logits [total_q, Hq, R' >= rel_extent] (bf16/fp16/fp32, any token stride
    including 0), cu_seqlens_q/k int32 [batch+1] on the same GPU.
    Returns out [total_q, Hq, D] in q.dtype, or (out, lse) with return_lse.
    bottom_right=True: upstream flash-attn alignment (query i at key position
    i + Lk - Lq for the bias distance, causal mask and window); the default is
    the reference's top-left alignment.
    """
    scale = _resolve(q, k, n_heads, kv_heads, head_dim, softmax_scale)
    out, lse = _ops().fwd(q, k, v, rel_logits, cu_seqlens_q, cu_seqlens_k, int(max_seqlen_q),
                          int(max_seqlen_k), int(rel_extent), bool(causal),
                          _window_left(window_size), scale, bool(return_lse),
                          _flag_bits(bottom_right, _flags))
    return (out, lse) if return_lse else out


@torch.no_grad()
def inkling_fa4_rel_attention_decode(q, k, v, rel_logits, cu_seqlens_q, cu_seqlens_k,
                                     max_seqlen_q, max_seqlen_k, rel_extent, causal=True,
                                     window_size=(-1, -1), n_heads=None, kv_heads=None,
                                     head_dim=None, arch=None, *, softmax_scale=None,
                                     return_lse=False, bottom_right=False, k_scale=1.0,
                                     v_scale=1.0):
    """Decode forward: exactly one query token per sequence
    (cu_seqlens_q == arange(batch + 1)), KV split across workgroups and merged
    by log-sum-exp.  Falls through to the prefill kernel when q holds more
    tokens than there are sequences, or for GQA groups above 16.

    k / v may be torch.float8_e4m3fn (an FP8 KV cache, GQA groups up to 16):
    the keys and values are k * k_scale and v * v_scale.
    """
    scale = _resolve(q, k, n_heads, kv_heads, head_dim, softmax_scale)
    batch = cu_seqlens_q.shape[0] - 1
    group = q.shape[1] // k.shape[1]
    if q.shape[0] != batch or group > 16:
        if k.dtype == torch.float8_e4m3fn:
            raise ValueError("fp8 K/V needs one query per sequence and GQA groups up to 16")
        return inkling_fa4_rel_attention(q, k, v, rel_logits, cu_seqlens_q, cu_seqlens_k,
                                         max_seqlen_q, max_seqlen_k, rel_extent, causal,
                                         window_size, softmax_scale=scale,
                                         return_lse=return_lse, bottom_right=bottom_right)
    out, lse = _ops().decode(q, k, v, rel_logits, cu_seqlens_q, cu_seqlens_k,
                             int(max_seqlen_q), int(max_seqlen_k), int(rel_extent), bool(causal),
                             _window_left(window_size), scale, bool(return_lse),
                             _flag_bits(bottom_right), float(k_scale), float(v_scale))
    return (out, lse) if return_lse else out


@torch.no_grad()
def inkling_fa4_rel_attention_decode_paged(q, k_cache, v_cache, rel_logits, cu_seqlens_q,
                                           seqused_k, block_table, max_seqlen_q, max_seqlen_k,
                                           rel_extent, causal=True, window_size=(-1, -1), *,
                                           softmax_scale=None, return_lse=False,
                                           bottom_right=False, k_scale=1.0, v_scale=1.0):
    """Decode over a paged KV cache (the serving backend's format,
    outputs/architecture.md:117-120: blocks of 16 tokens).

    k_cache / v_cache [num_blocks, block_size, Hkv, D] (block_size a power of
    two >= 8, last dim contiguous), block_table int32 [batch, max_blocks]
    (sequence b's key j sits in block block_table[b, j // block_size] at row
    j % block_size), seqused_k int32 [batch] keys per sequence; one query per
    sequence (cu_seqlens_q == arange(batch + 1)), GQA groups up to 16.
    Results equal inkling_fa4_rel_attention_decode on the same keys stored
    contiguously, up to the order in which the KV splits are merged.  max_seqlen_k must bound seqused_k.  An fp8
    cache (torch.float8_e4m3fn, with k_scale / v_scale) needs blocks of at
    least 16 tokens when head_dim is 64.
    """
    if k_cache.dim() != 4:
        raise ValueError("k_cache must be [num_blocks, block_size, kv_heads, head_dim]")
    scale = _resolve(q, k_cache[0], None, None, None, softmax_scale)
    out, lse = _ops().decode_paged(q, k_cache, v_cache, rel_logits, cu_seqlens_q, seqused_k,
                                   block_table, int(max_seqlen_q), int(max_seqlen_k),
                                   int(rel_extent), bool(causal), _window_left(window_size),
                                   scale, bool(return_lse), _flag_bits(bottom_right),
                                   float(k_scale), float(v_scale))
    return (out, lse) if return_lse else out


@torch.no_grad()
def inkling_fa4_rel_attention_rproj(q, k, v, rel_r, rel_w, cu_seqlens_q, cu_seqlens_k,
                                    max_seqlen_q, max_seqlen_k, rel_extent, causal=True,
                                    window_size=(-1, -1), *, softmax_scale=None,
                                    return_lse=False, bottom_right=False):
    """Prefill with the relative bias computed in the kernel from the low-rank
    factors of the serving backend's RelLogitsProj (outputs/architecture.md:24,
    52-54): rel_logits = einsum('thd,de->the', rel_r, rel_w) is never
    materialised.

    rel_r [total_q, Hq, 16] (bf16 or fp32, last dim contiguous), rel_w [16, R']
    with R' >= rel_extent; any rel_extent (the serving model's 512 local and
    1024 global included).  The band is projected on the matrix cores with
    r and W split into bf16 hi + lo parts (about 16 significant bits).
    Otherwise as inkling_fa4_rel_attention.
    """
    scale = _resolve(q, k, None, None, None, softmax_scale)
    if rel_w.dim() != 2 or rel_w.shape[0] != rel_r.shape[-1]:
        raise ValueError("rel_w must be [d_rel, R'] with d_rel = rel_r.shape[-1]")
    wt = rel_w.t().to(torch.float32).contiguous()  # W^T [R', 16], 64 bytes per distance
    out, lse = _ops().fwd_rproj(q, k, v, rel_r, wt, cu_seqlens_q, cu_seqlens_k,
                                int(max_seqlen_q), int(max_seqlen_k), int(rel_extent),
                                bool(causal), _window_left(window_size), scale, bool(return_lse),
                                _flag_bits(bottom_right))
    return (out, lse) if return_lse else out


def inkling_fa4_rel_attention_triton(q, k, v, rel_logits, cu_seqlens_q, cu_seqlens_k,
                                     max_seqlen_q, max_seqlen_k, rel_extent, causal=True,
                                     window_size=(-1, -1), n_heads=None, kv_heads=None,
                                     head_dim=None, arch=None, **kw):
    """Name kept from src/inkling_fa4/triton_kernel.py:85; runs the HIP kernel."""
    return inkling_fa4_rel_attention(q, k, v, rel_logits, cu_seqlens_q, cu_seqlens_k,
                                     max_seqlen_q, max_seqlen_k, rel_extent, causal,
                                     window_size, n_heads, kv_heads, head_dim, arch, **kw)


def inkling_fa4_rel_attention_kv_pruned_triton(q, k, v, rel_logits, cu_seqlens_q,
                                               cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                                               rel_extent, causal=True, window_size=(-1, -1),
                                               n_heads=None, kv_heads=None, head_dim=None,
                                               arch=None, **kw):
    """Name kept from src/inkling_fa4/triton_kernel_kv_pruned.py:210; the HIP
    prefill kernel always prunes fully-masked KV tiles."""
    return inkling_fa4_rel_attention(q, k, v, rel_logits, cu_seqlens_q, cu_seqlens_k,
                                     max_seqlen_q, max_seqlen_k, rel_extent, causal,
                                     window_size, n_heads, kv_heads, head_dim, arch, **kw)


def inkling_fa4_rel_attention_decode_triton(q, k, v, rel_logits, cu_seqlens_q, cu_seqlens_k,
                                            max_seqlen_q, max_seqlen_k, rel_extent, causal=True,
                                            window_size=(-1, -1), n_heads=None, kv_heads=None,
                                            head_dim=None, arch=None, **kw):
    """Name kept from src/inkling_fa4/triton_kernel_decode.py:128."""
    return inkling_fa4_rel_attention_decode(q, k, v, rel_logits, cu_seqlens_q, cu_seqlens_k,
                                            max_seqlen_q, max_seqlen_k, rel_extent, causal,
                                            window_size, n_heads, kv_heads, head_dim, arch, **kw)


def prefill_tile_counts(cu_seqlens_q, cu_seqlens_k, n_heads, causal=True, window_size=(-1, -1),
                        head_dim=128, bottom_right=False):
    """(visited, total) KV tiles of a prefill call: tiles the kernel loads after
    causal/window pruning vs tiles an unpruned kernel would load."""
    cq = [int(x) for x in torch.as_tensor(cu_seqlens_q).cpu().tolist()]
    ck = [int(x) for x in torch.as_tensor(cu_seqlens_k).cpu().tolist()]
    return _abi.count_tiles(cq, ck, n_heads, causal=causal,
                            window_left=_window_left(window_size), head_dim=head_dim,
                            bottom_right=bottom_right)


def default_scale(head_dim):
    """Default softmax scale of the drop-in API (1/head_dim)."""
    return 1.0 / head_dim


def sdpa_scale(head_dim):
    """The conventional 1/sqrt(head_dim) scale."""
    return 1.0 / math.sqrt(head_dim)
