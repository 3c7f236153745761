// Prefill forward of relative-bias flash attention for gfx950 (MI355X).
//
// Replaces _fa4_rel_attn_prefill_kernel (src/inkling_fa4/triton_kernel.py:6-82)
// and its KV-pruned variant (src/inkling_fa4/triton_kernel_kv_pruned.py:25-207),
// with one launch over every (query tile, head, sequence) instead of one launch
// per sequence (triton_kernel.py:94-106).
//
// Work decomposition.  A workgroup of 4 waves owns BLOCK_Q = 128 query rows of
// one (sequence, head); wave w owns rows 32w .. 32w+31.  K/V tiles of BLOCK_K =
// 64 keys are staged in LDS (double buffered, register prefetch of the next
// tile while the current one is computed).  Two workgroups share a CU (two
// waves per SIMD), so one wave's softmax overlaps the other's matrix products.
//
// Score layout.  Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16:
// A = K rows from LDS, B = Q held in registers for the whole KV loop.  In the
// C layout a lane then owns ONE query (column l % 32) and 16 keys of every
// 32-key block, so the row max/sum of the softmax are in-lane reductions plus
// one exchange with lane l ^ 32, and P leaves the accumulator already in the
// B-operand layout of the next product O^T = V^T P^T (no LDS round trip for P).
// V is written to LDS transposed (V^T[d][key]) with the key order inside each
// 16-key group permuted (bits 2 and 3 swapped) so every A operand of the PV
// product is one 16-byte LDS read.
//
// Memory access.  Q/K/V rows and bias values are read with buffer loads over
// per-(sequence, head) resources: rows past the sequence end fall outside the
// resource and read as zero, so ragged tails need no branches and offsets are
// 32-bit.
//
// Softmax.  exp2 with softmax_scale*log2(e) folded into one FMA; the bias is
// pre-multiplied by log2(e).  The running max is only raised when it grows by
// more than 2^8 (deferred rescale), which keeps the result exact and skips the
// O rescale on most tiles.  Row sums accumulate the fp32 P (summing the
// rounded 16-bit P instead would cost the LSE up to 2^-9 relative on short rows).
//
// Workgroup order.  Workgroup i runs on XCD i % 8; when the (sequence, kv
// head) pairs divide evenly, XCD x gets pairs x, x+8, ... so each pair's K/V
// is served from one XCD's L2 (measured: 72 instead of 337 MiB fetched from
// the fabric per call on the 8 x 4096 workload).  Heaviest q tiles go first.
//
// Tile classes per (wave, KV tile): fully masked -> skipped (causal: keys after
// the wave's last row; window: keys left of the window); edge (diagonal, window
// boundary, KV tail, or within the relative-bias band 0 <= dist < rel_extent)
// -> per-element key-range mask + bias gather; interior -> plain flash attention.
#include "ifa4_device.hpp"
#include "ifa4_kernels.h"

#ifndef IFA4_PRIO
#define IFA4_PRIO 0
#endif

namespace ifa4 {
namespace {

constexpr int kWaves = 4;
constexpr int kBlockQ = 32 * kWaves;  // 128
constexpr int kBlockK = 64;
constexpr int kThreads = 64 * kWaves;

template <int D>
struct PrefillLds {
  static constexpr int kPitch = D + 8;           // K row pitch (elements)
  static constexpr int vPitch = kBlockK + 8;     // V^T row pitch (elements)
  static constexpr int kElems = kBlockK * kPitch;
  static constexpr int vElems = D * vPitch;
  static constexpr int stage = kElems + vElems;  // 16-bit elements per stage
};

// LDS position of key `kk` inside a V^T row: bits 2 and 3 swapped, so the 8
// keys one lane needs for a 16-key PV step are contiguous.
__device__ __forceinline__ int vt_pos(int kk) {
  return (kk & ~12) | ((kk & 4) << 1) | ((kk & 8) >> 1);
}

// Bytes a resource over `rows` rows of `stride` elements (row length d) spans.
__device__ __forceinline__ uint32_t span_bytes(int rows, int64_t stride, int d, int esize) {
  return rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * stride + d) * esize) : 0u;
}

template <int D, typename Tag, typename Rel>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_fwd_kernel(PrefillParams p) {
  using E = Elem<Tag>;
  using L = PrefillLds<D>;
  constexpr int kKChunks = D / 8;                         // 16-byte chunks per K row
  constexpr int kKItems = kBlockK * kKChunks / kThreads;  // K chunks per thread
  constexpr int kVItems = (kBlockK / 4) * (D / 8);        // (4-key group, d-chunk) items
  constexpr int kDBlocks = D / 32;
  constexpr int kKSteps = D / 16;

  __shared__ __align__(16) uint16_t lds[2 * L::stage];

  // ---- which (q tile, head, sequence): heaviest (last) q tiles first --------
  int qtile, head, seq;
  if (p.xcd_pairs) {
    // Workgroup i runs on XCD i % 8.  Give XCD x the (sequence, kv head) pairs
    // x, x+8, ... so their K/V stay in that XCD's L2; heaviest q tiles first.
    const int x = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int per_xcd = p.xcd_pairs;  // pairs per XCD
    const int per_tile = per_xcd * p.group;
    qtile = p.n_qtiles - 1 - slot / per_tile;
    const int rem = slot % per_tile;
    const int pair = x + 8 * (rem / p.group);
    const int kv_heads = p.n_heads / p.group;
    seq = pair / kv_heads;
    head = (pair % kv_heads) * p.group + rem % p.group;
  } else {
    const int per_tile = p.n_heads * p.batch;
    const int lin = blockIdx.x;
    qtile = p.n_qtiles - 1 - lin / per_tile;
    const int rem = lin % per_tile;
    head = rem % p.n_heads;
    seq = rem / p.n_heads;
  }

  const int qs = p.cu_q[seq];
  const int lq = p.cu_q[seq + 1] - qs;
  const int ks = p.cu_k[seq];
  const int lk = p.cu_k[seq + 1] - ks;
  const int q0 = qtile * kBlockQ;
  if (q0 >= lq) return;
  const int kvh = head / p.group;
  const int delta = lq - lk;
  const int wl = p.window_left;
  const int rext = p.rel_extent;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 31;   // query column of this lane
  const int half = lane >> 5;  // 0 / 1

  // ---- per-(sequence, head) buffer resources --------------------------------------
  const uint16_t* q_base = static_cast<const uint16_t*>(p.q) + (int64_t)qs * p.q_st +
                           (int64_t)head * p.q_sh;
  const uint16_t* k_base = static_cast<const uint16_t*>(p.k) + (int64_t)ks * p.k_st +
                           (int64_t)kvh * p.k_sh;
  const uint16_t* v_base = static_cast<const uint16_t*>(p.v) + (int64_t)ks * p.v_st +
                           (int64_t)kvh * p.v_sh;
  const rsrc_t rq = make_rsrc(q_base, span_bytes(lq, p.q_st, D, 2));
  const rsrc_t rk = make_rsrc(k_base, span_bytes(lk, p.k_st, D, 2));
  const rsrc_t rv = make_rsrc(v_base, span_bytes(lk, p.v_st, D, 2));
  const uint32_t k_row = (uint32_t)p.k_st * 2, v_row = (uint32_t)p.v_st * 2;

  // ---- key range of the workgroup (tile pruning) ---------------------------
  const int q_hi = min(q0 + kBlockQ, lq);  // exclusive
  int kend = lk, kbeg = 0;
  if (!p.no_prune) {
    if (p.causal) kend = min(kend, q_hi);
    if (wl >= 0) kbeg = max(0, q0 - wl);
  }
  const int kt_beg = kbeg / kBlockK;
  const int kt_end = kend > kbeg ? (kend + kBlockK - 1) / kBlockK : kt_beg;

  // ---- per-wave rows ---------------------------------------------------------
  const int qa = q0 + 32 * wave;               // first row of the wave (local)
  const int wrows = max(0, min(32, lq - qa));  // valid rows of the wave
  const int qi = qa + col;                     // this lane's query (local)
  const bool row_ok = qi < lq;
  int wkend = lk, wkbeg = 0;
  if (!p.no_prune) {
    if (p.causal) wkend = min(lk, qa + wrows);
    if (wl >= 0) wkbeg = max(0, qa - wl);
  }

  // ---- Q fragment (B operand), kept for the whole loop -----------------------
  u32x4_t qf[kKSteps];
#pragma unroll
  for (int kk = 0; kk < kKSteps; ++kk)
    qf[kk] = buf_load_16(rq, (uint32_t)(qi * p.q_st + 16 * kk + 8 * half) * 2);

  const float c2 = p.scale_log2;  // softmax_scale * log2(e)
  float m_run = -INFINITY;         // running max (log2 domain), same in both halves
  float l_run = 0.f;               // partial row sum over this half's keys
  f32x16_t o[kDBlocks];
#pragma unroll
  for (int db = 0; db < kDBlocks; ++db) o[db] = f32x16_t{};

  // ---- K/V tile loader (global -> registers -> LDS) ---------------------------
  u32x4_t kreg[kKItems];
  u32x4_t vreg[4];
  const bool v_loader = tid < kVItems;
  const int v_kg = tid % (kBlockK / 4);  // 4-key group
  const int v_dc = tid / (kBlockK / 4);  // 8-wide d chunk

  auto load_tile = [&](int kt) {
    const int kb = kt * kBlockK;
#pragma unroll
    for (int r = 0; r < kKItems; ++r) {
      const int item = tid + r * kThreads;
      const int row = item / kKChunks;
      const int ch = item % kKChunks;
      kreg[r] = buf_load_16(rk, (uint32_t)(kb + row) * k_row + 16 * ch);
    }
    if (v_loader) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        vreg[r] = buf_load_16(rv, (uint32_t)(kb + 4 * v_kg + r) * v_row + 16 * v_dc);
    }
  };
  auto store_tile = [&](int buf) {
    uint16_t* kl = lds + buf * L::stage;
    uint16_t* vl = kl + L::kElems;
#pragma unroll
    for (int r = 0; r < kKItems; ++r) {
      const int item = tid + r * kThreads;
      const int row = item / kKChunks;
      const int ch = item % kKChunks;
      *reinterpret_cast<u32x4_t*>(kl + row * L::kPitch + 8 * ch) = kreg[r];
    }
    if (v_loader) {
      // vreg[r] holds V[key 4*kg + r][d 8*dc .. 8*dc+7]; write V^T rows d with
      // the 4 keys side by side (8 bytes) at the permuted key position.
      const int pos = vt_pos(4 * v_kg);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t lo01 = __builtin_amdgcn_perm(vreg[1][w], vreg[0][w], 0x05040100u);
        const uint32_t lo23 = __builtin_amdgcn_perm(vreg[3][w], vreg[2][w], 0x05040100u);
        const uint32_t hi01 = __builtin_amdgcn_perm(vreg[1][w], vreg[0][w], 0x07060302u);
        const uint32_t hi23 = __builtin_amdgcn_perm(vreg[3][w], vreg[2][w], 0x07060302u);
        const int d0 = 8 * v_dc + 2 * w;
        *reinterpret_cast<u32x2_t*>(vl + d0 * L::vPitch + pos) = u32x2_t{lo01, lo23};
        *reinterpret_cast<u32x2_t*>(vl + (d0 + 1) * L::vPitch + pos) = u32x2_t{hi01, hi23};
      }
    }
  };

  // Bias resource: the (sequence, head) rows of the bias; this lane reads its row.
  const rsrc_t rrel = make_rsrc(
      static_cast<const char*>(p.rel) + ((int64_t)qs * p.rel_st + (int64_t)head * p.rel_sh) *
                                            Rel::kBytes,
      span_bytes(lq, p.rel_st, p.rel_width, Rel::kBytes));
  const uint32_t rel_row_off = (uint32_t)(qi * p.rel_st) * Rel::kBytes;

  if (kt_beg < kt_end) load_tile(kt_beg);
  for (int kt = kt_beg; kt < kt_end; ++kt) {
    const int buf = (kt - kt_beg) & 1;
    store_tile(buf);
    __syncthreads();
    if (kt + 1 < kt_end) load_tile(kt + 1);

    const int kb = kt * kBlockK;
    // Wave-uniform activity / class of this tile.
    const bool active = wrows > 0 && kb < wkend && kb + kBlockK > wkbeg;
    if (!active) continue;
    const int imin = qa, imax = qa + wrows - 1;
    const int jmin = kb, jmax = kb + kBlockK - 1;
    const bool need_mask = jmax >= lk || (p.causal && jmax > imin) ||
                           (wl >= 0 && imax - jmin > wl);
    const bool has_bias =
        rext > 0 && (imax + delta - jmin >= 0) && (imin + delta - jmax <= rext - 1);

    const uint16_t* kl = lds + buf * L::stage;
    const uint16_t* vl = kl + L::kElems;

    // ---- S^T = K Q^T -----------------------------------------------------------
    f32x16_t s[kBlockK / 32];
#if IFA4_PRIO
    __builtin_amdgcn_s_setprio(1);
#endif
#pragma unroll
    for (int blk = 0; blk < kBlockK / 32; ++blk) {
      s[blk] = f32x16_t{};
      const uint16_t* krow = kl + (32 * blk + col) * L::kPitch + 8 * half;
#pragma unroll
      for (int kk = 0; kk < kKSteps; ++kk) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t*>(krow + 16 * kk);
        s[blk] = E::mfma32(a, qf[kk], s[blk]);
      }
    }

#if IFA4_PRIO
    __builtin_amdgcn_s_setprio(0);
#endif
    // ---- logits (log2 domain) and tile max ---------------------------------------
    // Element (blk, e) of this lane is tile-local key 32*blk + 8*(e>>2) + (e&3)
    // + 4*half; `kc` below drops the lane term, which is folded into the bounds.
    float sc;  // factor applied inside the exponent FMA
    float mx = -INFINITY;
    if (need_mask || has_bias) {
      sc = 1.f;
      int hi = lk - 1 - kb;
      if (p.causal) hi = min(hi, qi - kb);
      if (!row_ok) hi = -1;
      const int lo = wl >= 0 ? qi - wl - kb : -1;
      const int hi_h = hi - 4 * half, lo_h = lo - 4 * half;
      const int dbase = qi + delta - kb - 4 * half;  // dist = dbase - kc
      float bias[kBlockK / 2];
      if (has_bias) {
#pragma unroll
        for (int blk = 0; blk < kBlockK / 32; ++blk)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int kc = 32 * blk + 8 * (e >> 2) + (e & 3);
            const int dist = dbase - kc;
            const uint32_t off = (uint32_t)dist < (uint32_t)rext
                                     ? rel_row_off + (uint32_t)dist * Rel::kBytes
                                     : kOutOfRange;
            bias[16 * blk + e] = Rel::load(rrel, off);
          }
      }
#pragma unroll
      for (int blk = 0; blk < kBlockK / 32; ++blk) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kc = 32 * blk + 8 * (e >> 2) + (e & 3);
          float x = s[blk][e] * c2;
          if (has_bias) x = fmaf(bias[16 * blk + e], kLog2e, x);
          x = (kc >= lo_h && kc <= hi_h) ? x : -INFINITY;
          s[blk][e] = x;
          mx = fmaxf(mx, x);
        }
      }
    } else {
      sc = c2;
#pragma unroll
      for (int blk = 0; blk < kBlockK / 32; ++blk)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[blk][e]);
      mx *= c2;
    }
    mx = max_xor32(mx);

    // ---- deferred rescale ----------------------------------------------------------
    const float m_cand = fmaxf(m_run, mx);
    const bool grow = m_cand > m_run + kRescaleThreshold;
    if (wave_any(grow)) {
      const float m_upd = grow ? m_cand : m_run;
      const float alpha = grow ? fast_exp2(m_run - m_upd) : 1.f;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[db][e] *= alpha;
      m_run = m_upd;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;

    // ---- P = exp2(x - m), packed to the PV B operand, row sum ----------------------
    u32x4_t pb[kBlockK / 16];
#pragma unroll
    for (int t = 0; t < kBlockK / 16; ++t) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pv[e] = fast_exp2(fmaf(s[t >> 1][8 * (t & 1) + e], sc, -m_use));
        l_run += pv[e];
      }
      pb[t] = u32x4_t{E::pack2(pv[0], pv[1]), E::pack2(pv[2], pv[3]), E::pack2(pv[4], pv[5]),
                      E::pack2(pv[6], pv[7])};
    }

    // ---- O^T += V^T P^T ----------------------------------------------------------
#if IFA4_PRIO
    __builtin_amdgcn_s_setprio(1);
#endif
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) {
      const uint16_t* vrow = vl + (32 * db + col) * L::vPitch + 8 * half;
#pragma unroll
      for (int t = 0; t < kBlockK / 16; ++t) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t*>(vrow + 16 * t);
        o[db] = E::mfma32(a, pb[t], o[db]);
      }
    }
#if IFA4_PRIO
    __builtin_amdgcn_s_setprio(0);
#endif
  }

  // ---- epilogue: normalise, store O and LSE ------------------------------------------
  const float l_tot = add_xor32(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (row_ok) {
    uint16_t* obase = static_cast<uint16_t*>(p.out) + (int64_t)(qs + qi) * p.o_st +
                      (int64_t)head * p.o_sh;
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 32 * db + 8 * i + 4 * half;
        const u32x2_t w = {E::pack2(o[db][4 * i] * inv, o[db][4 * i + 1] * inv),
                           E::pack2(o[db][4 * i + 2] * inv, o[db][4 * i + 3] * inv)};
        *reinterpret_cast<u32x2_t*>(obase + d) = w;
      }
    }
    if (p.lse != nullptr && half == 0) {
      const float lse = l_tot > 0.f ? (m_run + __log2f(l_tot)) * kLn2 : -INFINITY;
      p.lse[(int64_t)head * p.lse_sh + qs + qi] = lse;
    }
  }
}

template <int D, typename Tag, typename Rel>
hipError_t launch_prefill_t(const PrefillParams& p_in, hipStream_t stream) {
  PrefillParams p = p_in;
  const int per_tile = p.n_heads * p.batch;
  const int64_t blocks = (int64_t)p.n_qtiles * per_tile;
  const int pairs = p.batch * (p.n_heads / p.group);
  p.xcd_pairs = pairs % 8 == 0 ? pairs / 8 : 0;
  if (blocks <= 0) return hipSuccess;
  hipLaunchKernelGGL((prefill_fwd_kernel<D, Tag, Rel>), dim3((unsigned)blocks), dim3(kThreads),
                     0, stream, p);
  return hipGetLastError();
}

template <int D, typename Tag>
hipError_t launch_prefill_rel(const PrefillParams& p, hipStream_t stream) {
  switch (p.rel_dtype) {
    case 0: return launch_prefill_t<D, Tag, RelBf16>(p, stream);
    case 1: return launch_prefill_t<D, Tag, RelF16>(p, stream);
    default: return launch_prefill_t<D, Tag, RelF32>(p, stream);
  }
}

}  // namespace

int prefill_block_q() { return kBlockQ; }
int prefill_block_k() { return kBlockK; }
int prefill_waves() { return kWaves; }

hipError_t launch_prefill(const PrefillParams& p, int head_dim, int qkv_dtype,
                          hipStream_t stream) {
  if (head_dim == 128) {
    return qkv_dtype == 0 ? launch_prefill_rel<128, Bf16Tag>(p, stream)
                          : launch_prefill_rel<128, F16Tag>(p, stream);
  }
  return qkv_dtype == 0 ? launch_prefill_rel<64, Bf16Tag>(p, stream)
                        : launch_prefill_rel<64, F16Tag>(p, stream);
}

}  // namespace ifa4
