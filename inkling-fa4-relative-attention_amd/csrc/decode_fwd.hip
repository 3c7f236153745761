// Split-KV decode of relative-bias attention for gfx950 (MI355X).
//
// Replaces _fa4_rel_attn_decode_kernel and its per-sequence launch loop
// (src/inkling_fa4/triton_kernel_decode.py:22-124,127-170).  Semantics follow
// the reference oracle (src/inkling_fa4/reference.py:19-40) for Lq = 1:
// query local index i = 0, dist = (1 - Lk) - j, causal keeps j <= 0 only, and
// the left window never masks (i - j <= 0).
//
// Pass 1 (decode_split_kernel): one wave per (kv head, KV split, sequence),
// kv head fastest so the two halves of a token row are read back to back.  The
// wave serves all G = n_heads / kv_heads query heads of its kv head, so every
// K/V byte is read from HBM once.  Per 32-key step:
//   * K and V rows are read with coalesced 16-byte buffer loads (each wave
//     load covers whole rows), one step ahead of the compute (register double
//     buffering), rows past the split end read as zero;
//   * K goes through a small padded LDS tile into the A operand of
//     S^T = K Q^T on v_mfma_f32_16x16x32 (B = the G query rows, zero padded to
//     16 columns);
//   * online softmax per head (exp2, deferred rescale);
//   * O += P V on the VALU: a lane holds one 16-byte chunk of a V row and reads
//     that key's G probabilities from LDS (broadcast).
// It writes the normalised partial o and its log2-sum-exp to the workspace.
//
// Pass 2 (decode_combine_kernel): per (head, sequence) merge of the valid
// splits by log-sum-exp (four waves share the splits, wave-parallel max/sum);
// writes out (q dtype) and lse (natural log).
#include "ifa4_device.hpp"
#include "ifa4_kernels.h"

namespace ifa4 {
namespace {

constexpr int kStep = 32;  // keys per pipeline step of a decode wave

// Lane layouts of a decode wave (D = head_dim):
//   row layout (loads, PV):  r = lane / (D/8) is the row within a wave load,
//                            c = lane % (D/8) the 16-byte d chunk;
//   S^T layout (QK):         n = lane % 16 the query head, g = lane / 16.
template <int D>
struct DecodeShape {
  static constexpr int kLpr = D / 8;           // lanes per K/V row
  static constexpr int kRpi = 64 / kLpr;       // rows per wave load
  static constexpr int kLoads = kStep / kRpi;  // wave loads per tensor per step
  static constexpr int kPitch = D + 8;         // LDS K row pitch (elements)
  static constexpr int kKSteps = D / 32;       // 16x16x32 MFMAs per 16 keys
};

template <int D, typename Tag, int G>
__global__ __launch_bounds__(64) void decode_split_kernel(DecodeParams p) {
  using E = Elem<Tag>;
  using S = DecodeShape<D>;

  __shared__ __align__(16) uint16_t k_lds[kStep * S::kPitch];
  __shared__ float p_lds[kStep * G];
  __shared__ float a_lds[G];
  __shared__ float l_lds[G];

  const int kvh = blockIdx.x;
  const int split = blockIdx.y;
  const int seq = blockIdx.z;
  const int qs = p.cu_q[seq];
  const int lq = p.cu_q[seq + 1] - qs;
  const int ks = p.cu_k[seq];
  const int lk = p.cu_k[seq + 1] - ks;
  if (lq != 1) return;
  const int kend = p.causal ? min(lk, 1) : lk;
  const int c0 = split * p.chunk;
  if (c0 >= kend) return;
  const int c1 = min(c0 + p.chunk, kend);
  const int delta = lq - lk;
  const int g_act = p.group;

  const int lane = threadIdx.x;
  const int r = lane / S::kLpr;  // row layout
  const int c = lane % S::kLpr;
  const int n = lane & 15;       // S^T layout
  const int g = lane >> 4;

  // Q (B operand): column n = head kvh*G + n, k-slots = d 32*kk + 8*g .. +7.
  const uint16_t* qbase = static_cast<const uint16_t*>(p.q) + (int64_t)qs * p.q_st;
  u32x4_t qf[S::kKSteps];
#pragma unroll
  for (int kk = 0; kk < S::kKSteps; ++kk) {
    qf[kk] = (n < g_act) ? ld_global_16(qbase + (int64_t)(kvh * g_act + n) * p.q_sh + 32 * kk +
                                        8 * g)
                         : u32x4_t{0, 0, 0, 0};
  }
  // K/V rows [0, c1) of this (sequence, kv head); rows at or past c1 read as 0.
  const uint16_t* kbase = static_cast<const uint16_t*>(p.k) + (int64_t)ks * p.k_st +
                          (int64_t)kvh * p.k_sh;
  const uint16_t* vbase = static_cast<const uint16_t*>(p.v) + (int64_t)ks * p.v_st +
                          (int64_t)kvh * p.v_sh;
  const rsrc_t rk = make_rsrc(kbase, (uint32_t)(((int64_t)(c1 - 1) * p.k_st + D) * 2));
  const rsrc_t rv = make_rsrc(vbase, (uint32_t)(((int64_t)(c1 - 1) * p.v_st + D) * 2));
  const uint32_t k_row = (uint32_t)p.k_st * 2, v_row = (uint32_t)p.v_st * 2;

  const float c2 = p.scale_log2;
  float m_run = -INFINITY;  // per head n (S^T lanes), identical over g
  float l_run = 0.f;        // partial sum over this lane's keys
  float o[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] = 0.f;

  auto load = [&](u32x4_t* kr, u32x4_t* vr, int k0) {
#pragma unroll
    for (int i = 0; i < S::kLoads; ++i) {
      const uint32_t row = (uint32_t)(k0 + S::kRpi * i + r);
      kr[i] = buf_load_16(rk, row * k_row + 16 * c);
      vr[i] = buf_load_16(rv, row * v_row + 16 * c);
    }
  };

  auto step = [&](const u32x4_t* kr, const u32x4_t* vr, int k0) {
    // K rows -> LDS (row-major, padded rows: conflict-free A-operand reads)
#pragma unroll
    for (int i = 0; i < S::kLoads; ++i)
      *reinterpret_cast<u32x4_t*>(k_lds + (S::kRpi * i + r) * S::kPitch + 8 * c) = kr[i];
    __syncthreads();

    // S^T = K Q^T: lane (n, g) gets keys 16*blk + 4*g + j of head n
    f32x4_t acc[kStep / 16];
#pragma unroll
    for (int blk = 0; blk < kStep / 16; ++blk) {
      acc[blk] = f32x4_t{};
      const uint16_t* krow = k_lds + (16 * blk + n) * S::kPitch + 8 * g;
#pragma unroll
      for (int kk = 0; kk < S::kKSteps; ++kk)
        acc[blk] = E::mfma16(*reinterpret_cast<const u32x4_t*>(krow + 32 * kk), qf[kk], acc[blk]);
    }

    const bool tail = k0 + kStep > c1;
    const bool bias = delta - k0 >= 0;  // some key of the step has dist >= 0
    float mx = -INFINITY;
#pragma unroll
    for (int blk = 0; blk < kStep / 16; ++blk) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float x = acc[blk][j] * c2;
        if (tail || bias) {
          const int key = k0 + 16 * blk + 4 * g + j;
          const int dist = delta - key;  // i = 0
          if (bias && n < g_act && key < c1 && dist >= 0 && dist < p.rel_extent) {
            x += load_rel(p.rel, (int64_t)qs * p.rel_st + (int64_t)(kvh * g_act + n) * p.rel_sh +
                                     dist, p.rel_dtype) * kLog2e;
          }
          if (key >= c1) x = -INFINITY;
        }
        acc[blk][j] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));

    const float m_cand = fmaxf(m_run, mx);
    const bool grow = m_cand > m_run + kRescaleThreshold;
    const bool any_grow = wave_any(grow);
    if (any_grow) {
      const float m_upd = grow ? m_cand : m_run;
      const float alpha = grow ? fast_exp2(m_run - m_upd) : 1.f;
      l_run *= alpha;
      m_run = m_upd;
      if (g == 0 && n < G) a_lds[n] = alpha;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
#pragma unroll
    for (int blk = 0; blk < kStep / 16; ++blk) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float pv = fast_exp2(acc[blk][j] - m_use);
        l_run += pv;
        if (n < G) p_lds[(16 * blk + 4 * g + j) * G + n] = pv;
      }
    }
    __syncthreads();

    if (any_grow) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float a = a_lds[h];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] *= a;
      }
    }
    // O += P V (VALU): row layout, key S::kRpi*i + r of the step
#pragma unroll
    for (int i = 0; i < S::kLoads; ++i) {
      const int kl = S::kRpi * i + r;
      float vv[8];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        vv[2 * w] = E::lo(vr[i][w]);
        vv[2 * w + 1] = E::hi(vr[i][w]);
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float ph = p_lds[kl * G + h];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] = fmaf(ph, vv[e], o[h][e]);
      }
    }
  };

  // Two register buffers; the loads of the next step are in flight while the
  // current one is computed.
  u32x4_t ka[S::kLoads], va[S::kLoads], kb[S::kLoads], vb[S::kLoads];
  int k0 = c0;
  load(ka, va, k0);
  while (true) {
    const int k1 = k0 + kStep;
    if (k1 < c1) load(kb, vb, k1);
    step(ka, va, k0);
    if (k1 >= c1) break;
    const int k2 = k1 + kStep;
    if (k2 < c1) load(ka, va, k2);
    step(kb, vb, k1);
    if (k2 >= c1) break;
    k0 = k2;
  }

  // -- finalise the split: reduce over lanes, normalise, write the partial --
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  if (g == 0 && n < G) l_lds[n] = l_run;
#pragma unroll
  for (int h = 0; h < G; ++h) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = o[h][e];
#pragma unroll
      for (int off = S::kLpr; off < 64; off <<= 1) v += __shfl_xor(v, off);
      o[h][e] = v;
    }
  }
  __syncthreads();

  const int n_splits = p.n_splits;
  if (r == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      if (h < g_act) {
        const float lt = l_lds[h];
        const float inv = lt > 0.f ? 1.f / lt : 0.f;
        float* dst = p.ws_o + (((int64_t)seq * p.n_heads + kvh * g_act + h) * n_splits + split) * D +
                     8 * c;
        *reinterpret_cast<f32x4_t*>(dst) = f32x4_t{o[h][0] * inv, o[h][1] * inv, o[h][2] * inv,
                                                   o[h][3] * inv};
        *reinterpret_cast<f32x4_t*>(dst + 4) = f32x4_t{o[h][4] * inv, o[h][5] * inv,
                                                       o[h][6] * inv, o[h][7] * inv};
      }
    }
  }
  if (g == 0 && n < g_act) {
    const float lse2 = l_run > 0.f ? m_run + __log2f(l_run) : -INFINITY;
    p.ws_lse[((int64_t)seq * p.n_heads + kvh * g_act + n) * n_splits + split] = lse2;
  }
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

constexpr int kCombineWaves = 4;

// One workgroup per (head, sequence); wave w merges splits w, w+4, ... with
// independent loads in flight, the four partial sums meet in LDS.
template <int D, typename Tag>
__global__ __launch_bounds__(64 * kCombineWaves) void decode_combine_kernel(DecodeParams p) {
  using E = Elem<Tag>;
  constexpr int kPer = D / 64;  // d values per lane
  __shared__ float part[kCombineWaves - 1][64 * kPer];
  const int head = blockIdx.x;
  const int seq = blockIdx.y;
  const int qs = p.cu_q[seq];
  const int lq = p.cu_q[seq + 1] - qs;
  const int lk = p.cu_k[seq + 1] - p.cu_k[seq];
  if (lq != 1) return;
  const int kend = p.causal ? min(lk, 1) : lk;
  // Splits pass 1 wrote for this sequence (never more than were launched, even
  // if a length exceeds the max_seqlen_k the grid was sized with).
  const int ns = min(kend > 0 ? (kend + p.chunk - 1) / p.chunk : 0, p.n_splits);
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)seq * p.n_heads + head;
  const float* lse_s = p.ws_lse + row * p.n_splits;
  const float* o_s = p.ws_o + row * p.n_splits * D + kPer * lane;

  // Every wave computes the max and the weight sum over all splits.
  float m = -INFINITY;
  for (int s = lane; s < ns; s += 64) m = fmaxf(m, lse_s[s]);
  m = wave_max(m);
  const float m_use = m == -INFINITY ? 0.f : m;
  float wpart = 0.f;
  for (int s = lane; s < ns; s += 64) wpart += fast_exp2(lse_s[s] - m_use);
  const float wsum = wave_sum(wpart);

  float acc[kPer];
#pragma unroll
  for (int e = 0; e < kPer; ++e) acc[e] = 0.f;
#pragma unroll 8
  for (int s = wave; s < ns; s += kCombineWaves) {
    const float wu = fast_exp2(lse_s[s] - m_use);
#pragma unroll
    for (int e = 0; e < kPer; ++e) acc[e] = fmaf(wu, o_s[(int64_t)s * D + e], acc[e]);
  }
  if (wave > 0) {
#pragma unroll
    for (int e = 0; e < kPer; ++e) part[wave - 1][kPer * lane + e] = acc[e];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < kCombineWaves - 1; ++w)
#pragma unroll
    for (int e = 0; e < kPer; ++e) acc[e] += part[w][kPer * lane + e];

  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  uint16_t* dst = static_cast<uint16_t*>(p.out) + (int64_t)qs * p.o_st + (int64_t)head * p.o_sh +
                  kPer * lane;
  if constexpr (kPer == 2) {
    *reinterpret_cast<uint32_t*>(dst) = E::pack2(acc[0] * inv, acc[1] * inv);
  } else {
    const uint32_t w = E::pack2(acc[0] * inv, 0.f);
    *dst = (uint16_t)(w & 0xffffu);
  }
  if (p.lse != nullptr && lane == 0) {
    p.lse[(int64_t)head * p.lse_sh + qs] = wsum > 0.f ? (m_use + __log2f(wsum)) * kLn2 : -INFINITY;
  }
}

template <int D, typename Tag, int G>
hipError_t launch_decode_g(const DecodeParams& p, hipStream_t stream) {
  hipLaunchKernelGGL((decode_split_kernel<D, Tag, G>), dim3(p.kv_heads, p.n_splits, p.batch),
                     dim3(64), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((decode_combine_kernel<D, Tag>), dim3(p.n_heads, p.batch),
                     dim3(64 * kCombineWaves), 0, stream, p);
  return hipGetLastError();
}

template <int D, typename Tag>
hipError_t launch_decode_d(const DecodeParams& p, hipStream_t stream) {
  if (p.group <= 1) return launch_decode_g<D, Tag, 1>(p, stream);
  if (p.group <= 2) return launch_decode_g<D, Tag, 2>(p, stream);
  if (p.group <= 4) return launch_decode_g<D, Tag, 4>(p, stream);
  if (p.group <= 8) return launch_decode_g<D, Tag, 8>(p, stream);
  return launch_decode_g<D, Tag, 16>(p, stream);
}

}  // namespace

int decode_max_group() { return 16; }

hipError_t launch_decode(const DecodeParams& p, int head_dim, int qkv_dtype, hipStream_t stream) {
  if (p.batch <= 0 || p.n_splits <= 0) return hipSuccess;
  if (head_dim == 128) {
    return qkv_dtype == 0 ? launch_decode_d<128, Bf16Tag>(p, stream)
                          : launch_decode_d<128, F16Tag>(p, stream);
  }
  return qkv_dtype == 0 ? launch_decode_d<64, Bf16Tag>(p, stream)
                        : launch_decode_d<64, F16Tag>(p, stream);
}

}  // namespace ifa4
