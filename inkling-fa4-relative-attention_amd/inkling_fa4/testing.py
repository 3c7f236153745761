"""Seeded synthetic inputs for the operator's reference workloads.

Inputs are drawn on the CPU from `torch.Generator().manual_seed(seed)` in a
fixed order (lengths, q, k, v, bias), q/k/v ~ N(0, 1) rounded to the device
dtype, the bias table ~ N(0, 0.5) fp32.  A GPU run and the fp32 CPU oracle see
exactly the same bits (the oracle upcasts the rounded values).

Workloads (all varlen-packed [tokens, heads, head_dim]):
  prefill_s64      batch 1, S 64, Hq=Hkv=4, D 64, fp16, causal, per-head bias
                   table [4,128], scale 1/sqrt(64)
  ragged_varlen    3 sequences [64,33,17], Hq 8, Hkv 2, D 128, bf16, causal
  long_prefill     batch 8, S in {1024,2048,4096,8192}, Hq 8, Hkv 2, D 128,
                   bf16, causal (the throughput workload)
  window_chunked   batch 16, 128 new tokens over a 384-key cache (256 prefix +
                   128 chunk), window_left 63, causal, Hq 8, Hkv 2, D 128, bf16
  decode           batch 64, one query per sequence, KV lengths U[1024,16384],
                   Hq 8, Hkv 2, D 128, bf16
Every bias table is [Hq, 128] passed as a token-stride-0 view [total_q, Hq, 128],
rel_extent 128.
"""
from dataclasses import dataclass, replace

import torch


@dataclass
class Case:
    name: str
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    rel: torch.Tensor
    cu_q: torch.Tensor
    cu_k: torch.Tensor
    max_q: int
    max_k: int
    rel_extent: int
    causal: bool
    window_left: int  # -1: none
    scale: float

    def to(self, device):
        rel = self.rel
        if rel.stride(0) == 0:  # keep the table a stride-0 view on the device
            rel = rel[0].to(device).unsqueeze(0).expand(rel.shape)
        else:
            rel = rel.to(device)
        return replace(self, q=self.q.to(device), k=self.k.to(device), v=self.v.to(device),
                       rel=rel, cu_q=self.cu_q.to(device), cu_k=self.cu_k.to(device))

    @property
    def window_size(self):
        return (self.window_left, 0) if self.window_left >= 0 else (-1, -1)

    @property
    def window_or_none(self):
        return self.window_left if self.window_left >= 0 else None

    def args(self):
        """Positional arguments of the operator API."""
        return (self.q, self.k, self.v, self.rel, self.cu_q, self.cu_k, self.max_q, self.max_k,
                self.rel_extent)

    def visible_pairs(self):
        """Number of visible (query, key) pairs summed over sequences and heads."""
        cq = self.cu_q.cpu().tolist()
        ck = self.cu_k.cpu().tolist()
        total = 0
        for b in range(len(cq) - 1):
            lq, lk = cq[b + 1] - cq[b], ck[b + 1] - ck[b]
            i = torch.arange(lq).unsqueeze(1)
            j = torch.arange(lk).unsqueeze(0)
            vis = torch.ones(lq, lk, dtype=torch.bool)
            if self.causal:
                vis &= i >= j
            if self.window_left >= 0:
                vis &= (i - j) <= self.window_left
            total += int(vis.sum())
        return total * self.q.shape[1]


def _cu(lengths):
    c = [0]
    for n in lengths:
        c.append(c[-1] + int(n))
    return torch.tensor(c, dtype=torch.int32)


def make_case(name, lens_q, lens_k, n_heads, kv_heads, head_dim, dtype, *, seed, rel_extent=128,
              rel_width=None, causal=True, window_left=-1, scale=None, rel_table=True,
              rel_dtype=torch.float32, rel_std=0.5, gen=None):
    g = gen if gen is not None else torch.Generator().manual_seed(seed)
    tq, tk = int(sum(lens_q)), int(sum(lens_k))
    rel_width = rel_extent if rel_width is None else rel_width
    q = torch.randn(tq, n_heads, head_dim, generator=g).to(dtype)
    k = torch.randn(tk, kv_heads, head_dim, generator=g).to(dtype)
    v = torch.randn(tk, kv_heads, head_dim, generator=g).to(dtype)
    if rel_table:
        table = (rel_std * torch.randn(n_heads, rel_width, generator=g)).to(rel_dtype)
        rel = table.unsqueeze(0).expand(tq, n_heads, rel_width)
    else:
        rel = (rel_std * torch.randn(tq, n_heads, rel_width, generator=g)).to(rel_dtype)
    return Case(name=name, q=q, k=k, v=v, rel=rel, cu_q=_cu(lens_q), cu_k=_cu(lens_k),
                max_q=max(lens_q) if len(lens_q) else 0,
                max_k=max(lens_k) if len(lens_k) else 0, rel_extent=rel_extent,
                causal=causal, window_left=window_left,
                scale=(1.0 / head_dim) if scale is None else scale)


def prefill_s64(seed=1, dtype=torch.float16):
    return make_case("prefill_s64", [64], [64], 4, 4, 64, dtype, seed=seed, scale=0.125)


def ragged_varlen(seed=2, dtype=torch.bfloat16, scale=None):
    return make_case("ragged_varlen", [64, 33, 17], [64, 33, 17], 8, 2, 128, dtype, seed=seed,
                     scale=scale)


def long_prefill(seq_len=4096, batch=8, seed=3, dtype=torch.bfloat16, scale=None):
    return make_case(f"long_prefill_s{seq_len}", [seq_len] * batch, [seq_len] * batch, 8, 2, 128,
                     dtype, seed=seed, scale=scale)


def window_chunked(seed=4, dtype=torch.bfloat16, scale=None, batch=16):
    return make_case("window_chunked", [128] * batch, [384] * batch, 8, 2, 128, dtype, seed=seed,
                     window_left=63, scale=scale)


def decode_lengths(batch=64, seed=5, lo=1024, hi=16384):
    g = torch.Generator().manual_seed(seed)
    return g, [int(x) for x in torch.randint(lo, hi + 1, (batch,), generator=g).tolist()]


def decode(seed=5, batch=64, dtype=torch.bfloat16, causal=False, scale=None, lo=1024, hi=16384):
    g, lens = decode_lengths(batch, seed, lo, hi)
    return make_case("decode", [1] * batch, lens, 8, 2, 128, dtype, seed=seed, causal=causal,
                     scale=scale, gen=g)


@dataclass
class PagedKV:
    """A paged copy of a case's K/V: k_cache / v_cache [num_blocks, block_size,
    Hkv, D], block_table int32 [batch, max_blocks], seqused_k int32 [batch]."""
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    block_table: torch.Tensor
    seqused_k: torch.Tensor

    def to(self, device):
        return PagedKV(*(t.to(device) for t in (self.k_cache, self.v_cache, self.block_table,
                                                 self.seqused_k)))


def paginate(case, block_size=16, seed=0, spare_blocks=5, fill=float("nan"),
             unused_entry=1 << 30, extra_columns=0):
    """Store the case's K/V in a block pool: the sequences' blocks in a seeded
    random physical order, `spare_blocks` unreferenced blocks, and every row no
    sequence owns (spare blocks, rows past a sequence's end) set to `fill`.
    Table entries past a sequence's last block hold `unused_entry`;
    `extra_columns` widens the table beyond what the longest sequence needs."""
    g = torch.Generator().manual_seed(seed)
    cu = [int(x) for x in case.cu_k.tolist()]
    lens = [cu[b + 1] - cu[b] for b in range(len(cu) - 1)]
    nblk = [(n + block_size - 1) // block_size for n in lens]
    max_blocks = max([1] + nblk) + extra_columns
    total = sum(nblk) + spare_blocks
    phys = torch.randperm(max(total, 1), generator=g).tolist()
    hkv, d = case.k.shape[1], case.k.shape[2]
    kc = torch.full((max(total, 1), block_size, hkv, d), fill, dtype=case.k.dtype)
    vc = torch.full_like(kc, fill)
    table = torch.full((len(lens), max_blocks), unused_entry, dtype=torch.int32)
    nxt = 0
    for b, n in enumerate(lens):
        for j in range(nblk[b]):
            blk = phys[nxt]
            nxt += 1
            table[b, j] = blk
            rows = min(block_size, n - j * block_size)
            src = cu[b] + j * block_size
            kc[blk, :rows] = case.k[src:src + rows]
            vc[blk, :rows] = case.v[src:src + rows]
    return PagedKV(kc, vc, table, torch.tensor(lens, dtype=torch.int32))


def fp8_kv(case, k_scale=None, v_scale=None):
    """FP8 (OCP e4m3, torch.float8_e4m3fn) copy of a case's K/V with one scale
    per tensor (default: the tensor's max magnitude maps to 448).  Returns
    (k8, v8, k_scale, v_scale, dequantised case); the dequantised case holds
    k8 * k_scale and v8 * v_scale in fp32, the exact values the kernel sees."""
    def scale_of(t):
        m = float(t.float().abs().max())
        return (m / 448.0) if m > 0 else 1.0
    ks = scale_of(case.k) if k_scale is None else float(k_scale)
    vs = scale_of(case.v) if v_scale is None else float(v_scale)
    k8 = (case.k.float() / ks).to(torch.float8_e4m3fn)
    v8 = (case.v.float() / vs).to(torch.float8_e4m3fn)
    deq = replace(case, k=k8.float() * ks, v=v8.float() * vs)
    return k8, v8, ks, vs, deq
