// Prefill forward of relative-bias flash attention for gfx950 (MI355X).
//
// Replaces _fa4_rel_attn_prefill_kernel (src/inkling_fa4/triton_kernel.py:6-82)
// and its KV-pruned variant (src/inkling_fa4/triton_kernel_kv_pruned.py:25-207),
// with one launch over every (query tile, head, sequence) instead of one launch
// per sequence (triton_kernel.py:94-106).
//
// Work decomposition.  A workgroup owns BLOCK_Q = 128 query rows of one
// (sequence, head).  Each wave owns NQB blocks of 32 rows.  K/V tiles of
// BLOCK_K = 64 keys go from HBM straight into LDS with buffer_load ... lds
// (no registers, no LDS store instructions); two LDS stages, the DMA of the
// next tile is in flight while the current one is computed.  Two shapes (the
// library builds NQB = 1; NQB = 2 is the sweep knob IFA4_PREFILL_NQB):
//   NQB = 2: 2 waves x 64 rows, 1 wave per SIMD with up to 512 registers;
//            every K / V^T fragment read from LDS feeds two MFMAs, and the two
//            independent row blocks let one block's softmax overlap the other
//            block's matrix products inside the wave;
//   NQB = 1: 4 waves x 32 rows, 2 waves per SIMD (<= 256 registers); the two
//            workgroups on a CU interleave instead.
//
// Score layout.  Each wave computes S^T = K Q^T with v_mfma_f32_32x32x16:
// A = K rows from LDS, B = Q held in registers for the whole KV loop.  In the
// C layout a lane then owns ONE query (column l % 32) and 16 keys of every
// 32-key block, so the row max/sum of the softmax are in-lane reductions plus
// one exchange with lane l ^ 32, and P leaves the accumulator already in the
// B-operand layout of the next product O^T = V^T P^T (no LDS round trip for P).
// V stays row-major in LDS; the A operand of the PV product (V^T, 8 keys per
// lane) is two ds_read_b64_tr_b16 transposing reads: within a 16-lane group,
// source lane j pointing at V[k0 + j/4][d0 + 4(j%4)] returns to lane i the
// four values V[k0 .. k0+3][d0 + i], which is exactly the key order of P.
// LDS rows are stored with their 16-byte chunks XOR-swizzled (swz below: at
// d 128, f(row) = 4(row & 3) | ((row >> 2) & 1) | 2((row >> 4) & 1)), so the K
// reads (rows {0..7, 16..23} or {8..15, 24..31} of a 32-key block per pass)
// and the 4-row transposing V reads each hit distinct banks.
//
// Memory access.  Q/K/V rows and bias values are read with buffer loads over
// per-(sequence, head) resources: rows past the sequence end fall outside the
// resource and read as zero, so ragged tails need no branches and offsets are
// 32-bit.
//
// Softmax.  exp2 with softmax_scale*log2(e) folded into one FMA; the bias is
// added in score units (bias / softmax_scale), so every tile shares one
// exponent form.  The running max is only raised when it grows by
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
#define IFA4_PRIO 1
#endif
#ifndef IFA4_PREFILL_NQB
#define IFA4_PREFILL_NQB 1
#endif
#ifndef IFA4_BIAS_LDS
#define IFA4_BIAS_LDS 1
#endif
#ifndef IFA4_SCHED
#define IFA4_SCHED 1
#endif
#ifndef IFA4_PV2
#define IFA4_PV2 1
#endif
#ifndef IFA4_ONEBAR
#define IFA4_ONEBAR 1
#endif
#ifndef IFA4_PVALU
#define IFA4_PVALU 7
#endif
#ifndef IFA4_DMA2
#define IFA4_DMA2 1
#endif
#ifndef IFA4_BIAS_EARLY
#define IFA4_BIAS_EARLY 1
#endif
#ifndef IFA4_PROJ_SKIP
#define IFA4_PROJ_SKIP 1
#endif
#ifndef IFA4_PROJ_EARLY
#define IFA4_PROJ_EARLY 1
#endif
#ifndef IFA4_MERGE_BATCH
#define IFA4_MERGE_BATCH 4
#endif
#ifndef IFA4_MERGE_PARTS
#define IFA4_MERGE_PARTS 8
#endif
#ifndef IFA4_MERGE_THREADS
#define IFA4_MERGE_THREADS 256
#endif

namespace ifa4 {
namespace {

// Tile shape of one instantiation of the kernel.
template <int NQB, int BK, int WPE, int WAVES>
struct PrefillShape {
  static constexpr int kNqb = NQB;                    // 32-row query blocks per wave
  static constexpr int kWaves = WAVES;                // waves per workgroup
  static constexpr int kBlockQ = 32 * NQB * kWaves;   // 128
  static constexpr int kBlockK = BK;                  // keys per KV tile (32 or 64)
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kWavesPerSimd = WPE;           // occupancy the register budget targets
  // Bias table in LDS, for the layout where every token of the sequence shares
  // one per-head table (token stride 0): rel[dist] at index
  // kBiasTop - dist (descending, so that a lane's 16 keys, whose distances
  // fall, read ascending addresses), zeros for dist outside [0, rel_extent),
  // dist from -kBiasPad to kBiasLdsMax + kBiasPad - 1.  A wave's tile
  // that has bias sees dist (over all 32 * NQB lanes' rows, valid or not, and
  // the BK keys) in an interval of 32 * NQB + BK - 1 values that meets
  // [0, rel_extent), so a padding of 32 * NQB + BK - 2 on both sides covers
  // every read: no range checks.
  static constexpr int kBiasPad = (32 * NQB + BK - 2 + 31) / 32 * 32;
  static_assert(kBiasPad >= 32 * NQB + BK - 2, "bias table padding covers a tile's band");
};

#ifndef IFA4_BLOCK_K
#define IFA4_BLOCK_K 64
#endif
#ifndef IFA4_WPE
#define IFA4_WPE (IFA4_PREFILL_NQB == 1 ? 2 : 1)
#endif
#ifndef IFA4_PREFILL_WAVES
#define IFA4_PREFILL_WAVES (IFA4_PREFILL_NQB == 1 ? 4 : 2)
#endif
// The shape the library is built with (sweep knobs IFA4_PREFILL_NQB,
// IFA4_BLOCK_K, IFA4_WPE, IFA4_PREFILL_WAVES).
using Shape = PrefillShape<IFA4_PREFILL_NQB, IFA4_BLOCK_K, IFA4_WPE, IFA4_PREFILL_WAVES>;
#ifndef IFA4_LOOK_K
#define IFA4_LOOK_K 4
#endif
#ifndef IFA4_LOOK_V
#define IFA4_LOOK_V 4
#endif
[[maybe_unused]] constexpr int kLookK = IFA4_LOOK_K;  // K fragment reads in flight ahead of the QK MFMAs
[[maybe_unused]] constexpr int kLookV = IFA4_LOOK_V;  // V^T operand pairs in flight ahead of the PV MFMAs (PV2 off)

// One LDS stage: K tile then V tile, each [kBlockK][D] row-major, swizzled.
template <typename Sh, int D>
struct PrefillStage {
  static constexpr int kTile = Sh::kBlockK * D;          // 16-bit elements per tensor
  static constexpr int kElems = 2 * kTile;
  static constexpr int kChunks = D / 8;                  // 16-byte chunks per row
  static constexpr int kRowsPerDma = 1024 / (2 * D);     // rows one wave DMA covers
  static constexpr int kDmaPerTensor = Sh::kBlockK / kRowsPerDma;
  static constexpr int kDmaPerWave = 2 * kDmaPerTensor / Sh::kWaves;
};

// Keys of a 32-key block in the S^T tile: MFMA row r of S^T = K Q^T reads K
// row perm32(r), so that lane half h, which holds rows 8i + 4h + j (i, j in
// 0..3) of the 32x32 C layout, holds keys 16h + 4i + j: sixteen consecutive
// keys, whose relative-bias distances are consecutive too.
__device__ __forceinline__ int perm32(int r) {
  return (((r >> 2) & 1) << 4) | ((r >> 3) << 2) | (r & 3);
}

// 16-byte chunk swizzle of an LDS row, kChunks = chunks per row (16 or 8).
// Chunk c of tile row `row` sits at chunk c ^ swz(row).  The QK A-operand reads
// (ds_read_b128, 16 lanes per pass) cover rows {0..7, 16..23} or {8..15,
// 24..31} of a 32-key block at one chunk; the transposing V reads of PV cover
// four consecutive rows and four chunks per half wave: both are conflict-free
// (every bank once per pass) for 16 chunks per row (d 128, one row per 256-byte
// bank line) and 8 (d 64, two rows per line).
template <int kChunks>
__device__ __forceinline__ int swz(int row) {
  if constexpr (kChunks == 16)
    return ((row & 3) << 2) | ((row >> 2) & 1) | (((row >> 4) & 1) << 1);
  else
    return (((row >> 1) & 1) << 2) | ((row >> 2) & 1) | (((row >> 4) & 1) << 1);
}

// s_waitcnt immediates: at most n vector-memory operations of this wave
// outstanding (LDS/export counters unconstrained); all LDS operations done.
constexpr int vmcnt_imm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }
constexpr int kLgkm0 = 15 | (7 << 4) | (0 << 8) | (3 << 14);

constexpr int kBiasLdsMax = 1024;  // longest shared bias table staged in LDS

// Fused relative-logit projection (kProj): bias(i, dist) = sum_c r[i, c] *
// W[c, dist] with r [Tq, Hq, kProjDim] and W^T [R', kProjDim] fp32, any
// rel_extent.  For a wave's 32 rows qa .. qa+31 and a 64-key tile at kb the
// distances fall in T0 .. T0 + 94, T0 = qa + delta - kb - 63: three blocks of 32
// distances.  Block T is one MFMA product M^T = W^T[T0 + 32T + m, :] r^T (A =
// 32 distances x 16 channels, B = 16 channels x 32 rows) in bf16 split into
// hi + lo parts (W_hi r_hi + W_lo r_hi + W_hi r_lo: ~16 mantissa bits, the lo
// x lo term is below fp32 rounding of the sum).  The C layout gives lane (u,
// g) the distances 8i + 4g + j of row u; two blocks go to the wave's tile in
// LDS (row u, pitch kProjPitch floats), from which the lane holding keys
// 16h .. 16h+15 of a 32-key block reads its row's 16 distances along a
// diagonal.  Pitch 68: the 16-byte writes (16 rows per pass) and the diagonal
// reads (32 rows per pass, row u at u*69 + const) hit distinct banks.  W^T rows
// of the next tile are fetched with the next tile's DMA.
constexpr int kProjDim = 16;
constexpr int kProjPitch = 68;
// The projection's shape: 8 waves x 32 rows, so that the eight 8.5 KiB
// projection tiles and the two K/V stages (132 KiB at head_dim 128) give two
// waves per SIMD from one workgroup per CU.
using ProjShape = PrefillShape<1, 64, 2, 8>;

// Eight fp32 values -> packed bf16 pairs hi = x truncated (exact in fp32) and
// lo = bf16(x - hi) (round to nearest even): hi + lo carries 16 significant bits.
__device__ __forceinline__ void split_bf16x8(const float* x, u32x4_t& hi, u32x4_t& lo) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t a = __float_as_uint(x[2 * k]) & 0xffff0000u;
    const uint32_t b = __float_as_uint(x[2 * k + 1]) & 0xffff0000u;
    hi[k] = (a >> 16) | b;
    lo[k] = Elem<Bf16Tag>::pack2(x[2 * k] - __uint_as_float(a), x[2 * k + 1] - __uint_as_float(b));
  }
}

// Bytes a resource over `rows` rows of `stride` elements (row length d) spans.
__device__ __forceinline__ uint32_t span_bytes(int rows, int64_t stride, int d, int esize) {
  return rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * stride + d) * esize) : 0u;
}

// KV tiles [kt_beg, kt_end) a query tile visits (tile pruning): causal keeps
// keys below the tile's last row (+ qpos), the window keys from its first row
// (+ qpos) minus window_left; the prefill kernel and the merge of split-KV
// partials both derive a tile's range (and so its chunk count) from this.
struct TileRange {
  int beg, end;
};
template <typename Sh>
__device__ __forceinline__ TileRange tile_range(const PrefillParams& p, int q0, int lq, int lk,
                                                int qpos) {
  const int q_hi = min(q0 + Sh::kBlockQ, lq);  // exclusive
  int kend = lk, kbeg = 0;
  if (!p.no_prune) {
    if (p.causal) kend = min(kend, q_hi + qpos);
    if (p.window_left >= 0) kbeg = max(0, q0 + qpos - p.window_left);
  }
  const int beg = kbeg / Sh::kBlockK;
  return TileRange{beg, kend > kbeg ? (kend + Sh::kBlockK - 1) / Sh::kBlockK : beg};
}

// Split KV: chunk c of the key axis holds KV tiles [c, c + 1) * chunk_tiles;
// a query tile's k-th chunk is the k-th chunk its range meets, so the same
// tiles fall in the same chunks whatever the pruning.  Chunks a query tile
// spans: at least one (which also writes the rows of a tile with no visible
// key), at most the n_chunks slots the grid and the workspace hold.
__device__ __forceinline__ int tile_chunks(const PrefillParams& p, const TileRange& r) {
  if (p.chunk_tiles <= 0) return 1;
  const int n = r.end > r.beg ? (r.end + p.chunk_tiles - 1) / p.chunk_tiles -
                                    r.beg / p.chunk_tiles
                              : 1;
  return min(max(n, 1), p.n_chunks);
}

template <typename Sh, int D, typename Tag, typename Rel, bool kProj, bool kTab>
__global__ __launch_bounds__(Sh::kThreads) __attribute__((amdgpu_waves_per_eu(
    Sh::kWavesPerSimd, Sh::kWavesPerSimd))) void prefill_fwd_kernel(PrefillParams p) {
  using E = Elem<Tag>;
  using St = PrefillStage<Sh, D>;
  constexpr int kNqb = Sh::kNqb, kBlockQ = Sh::kBlockQ;
  constexpr int kBlockK = Sh::kBlockK, kThreads = Sh::kThreads, kBiasPad = Sh::kBiasPad;
  constexpr int kBiasLdsFloats = 2 * kBiasPad + kBiasLdsMax;
  constexpr int kBiasTop = kBiasLdsMax + kBiasPad - 1;  // table index of dist 0
  constexpr int kDBlocks = D / 32;
  constexpr int kKSteps = D / 16;

  // Both stages in one array: a read of stage 1 is the stage-0 address plus a
  // constant, which folds into the instruction's offset (one address register
  // per fragment instead of one per fragment and stage).
  __shared__ __align__(1024) uint16_t stages[2 * St::kElems];
  // bias table (shared-table layout); with kProj, one projection tile per wave
  constexpr bool kTable = kTab && !kProj;  // the shared bias table, staged in LDS
  __shared__ __align__(16) float bias_lds[kTable ? kBiasLdsFloats : 4];
  __shared__ __align__(16) float mproj[kProj ? Sh::kWaves * 32 * kProjPitch : 4];
  static_assert(!kProj || (kNqb == 1 && kBlockK == 64), "projection tiles: 32 rows x 64 keys");
  uint16_t* const stage0 = stages;
  uint16_t* const stage1 = stages + St::kElems;

  // ---- which (q tile, KV chunk, head, sequence): heaviest (last) q tiles first --
  // A q tile's chunks (split KV; one when not splitting) are consecutive, so
  // a chunk that ends early is followed by the next q tile's work.
  int qtile, chunk, head, seq;
  if (p.xcd_pairs) {
    // Workgroup i runs on XCD i % 8.  Give XCD x the (sequence, kv head) pairs
    // x, x+8, ... so their K/V stay in that XCD's L2; heaviest q tiles first.
    const int x = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int per_xcd = p.xcd_pairs;  // pairs per XCD
    const int per_tile = per_xcd * p.group;
    const int qc = slot / per_tile;
    qtile = p.n_qtiles - 1 - qc / p.n_chunks;
    chunk = qc % p.n_chunks;
    const int rem = slot % per_tile;
    const int pair = x + 8 * (rem / p.group);
    const int kv_heads = p.n_heads / p.group;
    seq = pair / kv_heads;
    head = (pair % kv_heads) * p.group + rem % p.group;
  } else {
    const int per_tile = p.n_heads * p.batch;
    const int lin = blockIdx.x;
    const int qc = lin / per_tile;
    qtile = p.n_qtiles - 1 - qc / p.n_chunks;
    chunk = qc % p.n_chunks;
    const int rem = lin % per_tile;
    head = rem % p.n_heads;
    seq = rem / p.n_heads;
  }

  const SeqBounds bq = seq_bounds(p.cu_q, seq, p.total_q);
  const SeqBounds bk = seq_bounds(p.cu_k, seq, p.total_k);
  const int qs = bq.start, lq = bq.len;
  const int ks = bk.start, lk = bk.len;
  const int q0 = qtile * kBlockQ;
  if (q0 >= lq) return;
  const int kvh = head / p.group;
  // Query i sits at key position i + qpos for the causal and window masks;
  // the bias distance is dist = i + delta - j.  Top-left (the reference
  // oracle, src/inkling_fa4/reference.py:28-37): qpos = 0, delta = lq - lk.
  // Bottom-right (upstream flash-attn): qpos = delta = lk - lq.
  const int qpos = p.bottom_right ? lk - lq : 0;
  const int delta = p.bottom_right ? lk - lq : lq - lk;
  const int wl = p.window_left;
  const int rext = p.rel_extent;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int lane = tid & 63;
  const int col = lane & 31;   // query column of this lane (per row block)
  const int half = lane >> 5;  // 0 / 1

  // ---- per-(sequence, head) buffer resources --------------------------------------
  const uint16_t* q_base = static_cast<const uint16_t*>(p.q) + (int64_t)qs * p.q_st +
                           (int64_t)head * p.q_sh;
  const uint16_t* k_base = static_cast<const uint16_t*>(p.k) + (int64_t)ks * p.k_st +
                           (int64_t)kvh * p.k_sh;
  const uint16_t* v_base = static_cast<const uint16_t*>(p.v) + (int64_t)ks * p.v_st +
                           (int64_t)kvh * p.v_sh;
  const rsrc_t rq = make_rsrc(q_base, span_bytes(lq, p.q_st, D, 2));
  [[maybe_unused]] const rsrc_t rk = make_rsrc(k_base, span_bytes(lk, p.k_st, D, 2));
  [[maybe_unused]] const rsrc_t rv = make_rsrc(v_base, span_bytes(lk, p.v_st, D, 2));
  const uint32_t k_row = (uint32_t)p.k_st * 2, v_row = (uint32_t)p.v_st * 2;

  // ---- key range of the workgroup (tile pruning, then this KV chunk) ---------
  const TileRange tr = tile_range<Sh>(p, q0, lq, lk, qpos);
  const int nch = tile_chunks(p, tr);
  if (chunk >= nch) return;
  int kt_beg = tr.beg, kt_end = tr.end;
  if (nch > 1) {
    const int c0 = (tr.beg / p.chunk_tiles + chunk) * p.chunk_tiles;
    kt_beg = max(tr.beg, c0);
    kt_end = min(tr.end, c0 + p.chunk_tiles);
  }

  // ---- per-wave rows ---------------------------------------------------------
  const int qa = q0 + 32 * kNqb * wave;                  // first row of the wave (local)
  const int wrows = max(0, min(32 * kNqb, lq - qa));     // valid rows of the wave
  int wkend = lk, wkbeg = 0;
  if (!p.no_prune) {
    if (p.causal) wkend = min(lk, qa + wrows + qpos);
    if (wl >= 0) wkbeg = max(0, qa + qpos - wl);
  }
  int qi[kNqb];        // this lane's query (local) in each row block
  bool row_ok[kNqb];
#pragma unroll
  for (int qb = 0; qb < kNqb; ++qb) {
    qi[qb] = qa + 32 * qb + col;
    row_ok[qb] = qi[qb] < lq;
  }

  // ---- Q fragments (B operand), kept for the whole loop ----------------------
  u32x4_t qf[kNqb][kKSteps];
#pragma unroll
  for (int qb = 0; qb < kNqb; ++qb)
#pragma unroll
    for (int kk = 0; kk < kKSteps; ++kk)
      qf[qb][kk] = buf_load_16(rq, (uint32_t)(qi[qb] * p.q_st + 16 * kk + 8 * half) * 2);

  const float c2 = p.scale_log2;  // softmax_scale * log2(e)
  const float inv_scale = kLog2e / c2;  // bias -> score units (1 / softmax_scale)
  float m_run[kNqb];               // running max (log2 domain), same in both halves
  float l_run[kNqb];               // partial row sum over this half's keys
  f32x16_t o[kNqb][kDBlocks];
#pragma unroll
  for (int qb = 0; qb < kNqb; ++qb) {
    m_run[qb] = -INFINITY;
    l_run[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) o[qb][db] = f32x16_t{};
  }

  // ---- K/V tile DMA: HBM -> LDS, rows past the sequence end read as zero -----------
  // A wave DMA writes 64 x 16 contiguous bytes = kRowsPerDma rows; lane L fills
  // slot L % kChunks of row L / kChunks with the chunk that swizzles to it.
  const int dma_row = lane / St::kChunks;
  const int dma_slot = lane % St::kChunks;
#if IFA4_DMA2
  // Each wave DMAs rows of one tensor (K for the first half of the waves, V for
  // the second).  A lane's offset within a DMA is relative to the tile's first
  // row: one register per DMA of the wave (its tile row's offset and swizzled
  // chunk), set once.  The tile's start goes into the base of a resource built
  // per tile (scalar arithmetic), whose size ends with the sequence's last row,
  // so rows of a partial last tile past the sequence end read as zero.
  static_assert(St::kDmaPerWave <= St::kDmaPerTensor && St::kDmaPerTensor % St::kDmaPerWave == 0,
                "a wave's DMAs stay within one tensor");
  const bool dma_v = wave * St::kDmaPerWave >= St::kDmaPerTensor;
  const uint32_t dma_rowb = dma_v ? v_row : k_row;
  const char* const dma_base = reinterpret_cast<const char*>(dma_v ? v_base : k_base);
  const uint32_t dma_span = span_bytes(lk, dma_v ? p.v_st : p.k_st, D, 2);
  uint32_t dma_voff[St::kDmaPerWave];
#pragma unroll
  for (int u = 0; u < St::kDmaPerWave; ++u) {
    const int id = wave * St::kDmaPerWave + u;
    const int blk = dma_v ? id - St::kDmaPerTensor : id;
    const int row = blk * St::kRowsPerDma + dma_row;  // tile row
    dma_voff[u] = (uint32_t)row * dma_rowb + 16u * (uint32_t)(dma_slot ^ swz<St::kChunks>(row));
  }
  const uint32_t lds_stages = lds_addr(stages);
  auto dma_tile = [&](int kt, uint16_t* stage) {
    const int kb = kt * kBlockK;
    const uint32_t stage_lds = lds_stages + (uint32_t)((stage - stages) * 2);
    const uint32_t skip = (uint32_t)kb * dma_rowb;  // bytes before the tile's first row
    const rsrc_t r = make_rsrc_uniform(dma_base + skip, dma_span > skip ? dma_span - skip : 0u);
    if (!IFA4_DMA_COVER_EACH) hazard_nop5();  // batch cover (sweep knob)
#pragma unroll
    for (int u = 0; u < St::kDmaPerWave; ++u) {
      const int id = wave * St::kDmaPerWave + u;
      const int blk = dma_v ? id - St::kDmaPerTensor : id;
      const uint32_t dst = stage_lds + (uint32_t)(((dma_v ? St::kTile : 0) + blk * 512) * 2);
      dma_16_tile(r, dma_voff[u], dst);
    }
  };
#else
  auto dma_tile = [&](int kt, uint16_t* stage) {
    const int kb = kt * kBlockK;
#pragma unroll
    for (int u = 0; u < St::kDmaPerWave; ++u) {
      const int id = wave * St::kDmaPerWave + u;  // 0 .. 2*kDmaPerTensor-1
      const bool is_v = id >= St::kDmaPerTensor;
      const int blk = is_v ? id - St::kDmaPerTensor : id;
      const int row = blk * St::kRowsPerDma + dma_row;
      const int chunk = dma_slot ^ swz<St::kChunks>(row);
      uint16_t* dst = stage + (is_v ? St::kTile : 0) + blk * 512;
      const uint32_t off = (uint32_t)(kb + row) * (is_v ? v_row : k_row) + 16 * chunk;
      dma_16(is_v ? rv : rk, off, dst);
    }
  };
#endif

  // Bias resource: the (sequence, head) rows of the bias (with kProj: of r,
  // 16 values per row); each lane reads its rows.
  const rsrc_t rrel = make_rsrc(
      static_cast<const char*>(p.rel) + ((int64_t)qs * p.rel_st + (int64_t)head * p.rel_sh) *
                                            Rel::kBytes,
      span_bytes(lq, p.rel_st, kProj ? kProjDim : p.rel_width, Rel::kBytes));
  // Shared-table layout with a table short enough to stage in LDS (the host
  // launches the kTab instantiation for it: token stride 0, rel_extent <=
  // kBiasLdsMax); the other instantiation reads per-token rows.
  const bool bias_in_lds = kTable && rext > 0;
  // Fused projection.  W^T [rel_width, 16] fp32 (64-byte rows) stays in L2;
  // rows outside [0, rel_extent) read as zero, so the projected bias is zero
  // there with no further test.  The B operand (this lane's row of r, channels
  // 8g .. 8g+7 in bf16 hi + lo) is set once; the A operands of a tile (its
  // three distance blocks) are fetched one tile ahead.
  using EB = Elem<Bf16Tag>;
  const rsrc_t rwt = make_rsrc(p.wt, kProj ? (uint32_t)((int64_t)p.rel_width * kProjDim * 4) : 0u);
  u32x4_t r_hi{}, r_lo{};
  u32x4_t w_raw[3][2];
  // wave-uniform: the tile at kb is visited by this wave and meets the band
  auto proj_tile = [&](int kb) {
    return rext > 0 && wrows > 0 && kb < wkend && kb + kBlockK > wkbeg &&
           qa + wrows - 1 + delta - kb >= 0 && qa + delta - (kb + kBlockK - 1) <= rext - 1;
  };
  // distance block t of the tile at kb meets [0, rext) (wave-uniform); blocks
  // that do not are zero and skip their fetch and products
  auto proj_live = [&](int kb, int t) {
    const int lo = qa + delta - kb - (kBlockK - 1) + 32 * t;
    return !IFA4_PROJ_SKIP || (lo + 31 >= 0 && lo < rext);
  };
  auto proj_fetch = [&](int kt) {
    if (!proj_tile(kt * kBlockK)) return;
    const int d0 = qa + delta - kt * kBlockK - (kBlockK - 1) + col;  // block 0, row col
#pragma unroll
    for (int t = 0; t < 3; ++t) {
      if (!proj_live(kt * kBlockK, t)) continue;
      const int dist = d0 + 32 * t;
      const uint32_t off =
          (uint32_t)dist < (uint32_t)rext ? (uint32_t)dist * 64u + 32u * half : kOutOfRange;
      w_raw[t][0] = buf_load_16(rwt, off);
      w_raw[t][1] = buf_load_16(rwt, off + 16);
    }
  };
  float* const mp = mproj + (kProj ? wave * 32 * kProjPitch : 0);  // this wave's tile
  // distance block t of the current tile (its W^T rows split just before use)
  auto proj_block = [&](int kb, int t) -> f32x16_t {
    if (!proj_live(kb, t)) return f32x16_t{};
    float w[8];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      w[c] = __uint_as_float(w_raw[t][0][c]);
      w[4 + c] = __uint_as_float(w_raw[t][1][c]);
    }
    u32x4_t w_hi, w_lo;
    split_bf16x8(w, w_hi, w_lo);
    f32x16_t acc = EB::mfma32(w_hi, r_hi, f32x16_t{});
    acc = EB::mfma32(w_lo, r_hi, acc);
    if constexpr (Rel::kBytes == 4) acc = EB::mfma32(w_hi, r_lo, acc);  // bf16 r: no lo part
    return acc;
  };
  auto proj_put = [&](const f32x16_t& acc, int slot) {
    float* dst = mp + col * kProjPitch + 32 * slot + 4 * half;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<f32x4_t*>(dst + 8 * i) =
          f32x4_t{acc[4 * i], acc[4 * i + 1], acc[4 * i + 2], acc[4 * i + 3]};
  };
  // bias of this lane's 16 keys in key block blk: block blk sees
  // distance blocks 1 - blk (slot 0) and 2 - blk (slot 1); element e sits at
  // position col + 31 - 16 * half - e of the lane's row.  Block 1 serves both
  // key blocks and is projected twice: one accumulator live at a time.
  auto proj_fill = [&](int kb, int blk) {
    proj_put(proj_block(kb, 1 - blk), 0);
    __builtin_amdgcn_sched_barrier(0);
    proj_put(proj_block(kb, 2 - blk), 1);
  };
  // Key block 0's distances are projected before the QK products of the tile
  // (the LDS writes land while the MFMAs run), key block 1's after its reads.
  constexpr bool kProjEarly = IFA4_PROJ_EARLY;
  auto proj_bias = [&](int kb, int blk, float* bias) {
    if (!(kProjEarly && blk == 0)) proj_fill(kb, blk);
    const float* src = mp + col * (kProjPitch + 1) + 31 - 16 * half;
#pragma unroll
    for (int e = 0; e < 16; ++e) bias[e] = src[-e];
  };

  // Per-token bias of the 16 consecutive keys a lane holds in a 32-key block,
  // at distances dtop - e (e = 0..15) of its row (element offset rel_row in the
  // bias resource), times log2(e), zero outside [0, rel_extent).  The 16
  // values are contiguous in memory: fp32 in four 16-byte loads, 16-bit types
  // in nine dwords from the even element at or below the lowest (two 16-byte
  // loads and one 4-byte load), shifted into place.  A wave with a valid row
  // whose span would start before the resource (the first row of a sequence,
  // or a token stride of 0) or end past it (the last row) falls back to one
  // load per element, so no vector load straddles either end.
  const int rel_par = Rel::kBytes == 2 ? (int)((reinterpret_cast<uintptr_t>(p.rel) +
                                                ((int64_t)qs * p.rel_st + (int64_t)head * p.rel_sh) *
                                                    Rel::kBytes) >> 1) & 1
                                       : 0;  // element parity of the resource base
  const int rel_span = lq > 0 ? (lq - 1) * (int)p.rel_st + p.rel_width : 0;  // elements
  auto token_bias = [&](int rel_row, int dtop, bool valid, float* bias) {
    constexpr int kSpan = Rel::kBytes == 2 ? 18 : 16;  // elements the vector loads cover
    const int lo = rel_row + dtop - 15;               // element of the lowest distance
    const int start = Rel::kBytes == 2 ? lo - ((lo + rel_par) & 1) : lo;  // dword-aligned
    if (wave_any(valid && (start < 0 || start + kSpan > rel_span))) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int dist = dtop - e;
        const uint32_t off = (uint32_t)dist < (uint32_t)rext
                                 ? (uint32_t)(rel_row + dist) * Rel::kBytes
                                 : kOutOfRange;
        bias[e] = Rel::load(rrel, off);
      }
      return;
    }
    const uint32_t boff = valid ? (uint32_t)start * Rel::kBytes : kOutOfRange;
    if constexpr (Rel::kBytes == 4) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4_t w = buf_load_16(rrel, boff + 16 * c);
#pragma unroll
        for (int j = 0; j < 4; ++j) bias[15 - (4 * c + j)] = __uint_as_float(w[j]);  // dist lo + 4c + j
      }
    } else {
      const u32x4_t w0 = buf_load_16(rrel, boff);
      const u32x4_t w1 = buf_load_16(rrel, boff + 16);
      const uint32_t w2 = buf_load_4(rrel, boff + 32);
      const uint32_t w[9] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3], w2};
      const uint32_t sh = 16u * (uint32_t)(lo - start);  // 0 or 16 bits
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t pr = __builtin_amdgcn_alignbit(w[k + 1], w[k], sh);  // dist lo+2k, lo+2k+1
        bias[15 - 2 * k] = Rel::lo(pr);
        bias[14 - 2 * k] = Rel::hi(pr);
      }
    }
    const bool in_band = dtop - 15 >= 0 && dtop < rext;
    if (!wave_all(in_band)) {
#pragma unroll
      for (int e = 0; e < 16; ++e) bias[e] = (uint32_t)(dtop - e) < (uint32_t)rext ? bias[e] : 0.f;
    }
  };
  // The same in two halves, so that the vector loads are issued before a tile's
  // QK products and their latency hides behind them: tok_issue loads the raw
  // dwords (nothing on the per-element path, which runs whole in tok_finish),
  // tok_finish unpacks, scales and masks.  Used for 16-bit bias types
  // (kTokEarly): measured on 8 x 4096 with a bf16 bias of extent 1024, 0.424 ->
  // 0.376 ms, and 3-6% on batch 1 x 4 heads at S 1024 / 4096.
  struct TokRaw {
    uint32_t w[Rel::kBytes == 4 ? 16 : 9];
    bool slow;  // wave-uniform: one load per element
  };
  constexpr bool kTokEarly = IFA4_BIAS_EARLY && !kProj && !kTable && Rel::kBytes == 2;
  auto tok_issue = [&](int rel_row, int dtop, bool valid, TokRaw& t) {
    constexpr int kSpan = Rel::kBytes == 2 ? 18 : 16;
    const int lo = rel_row + dtop - 15;
    const int start = Rel::kBytes == 2 ? lo - ((lo + rel_par) & 1) : lo;
    t.slow = wave_any(valid && (start < 0 || start + kSpan > rel_span));
    if (t.slow) return;
    const uint32_t boff = valid ? (uint32_t)start * Rel::kBytes : kOutOfRange;
    if constexpr (Rel::kBytes == 4) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4_t w = buf_load_16(rrel, boff + 16 * c);
#pragma unroll
        for (int j = 0; j < 4; ++j) t.w[4 * c + j] = w[j];
      }
    } else {
      const u32x4_t w0 = buf_load_16(rrel, boff);
      const u32x4_t w1 = buf_load_16(rrel, boff + 16);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        t.w[j] = w0[j];
        t.w[4 + j] = w1[j];
      }
      t.w[8] = buf_load_4(rrel, boff + 32);
    }
  };
  auto tok_finish = [&](int rel_row, int dtop, bool valid, const TokRaw& t, float* bias) {
    if (t.slow) {
      token_bias(rel_row, dtop, valid, bias);  // takes the per-element path again
      return;
    }
    if constexpr (Rel::kBytes == 4) {
#pragma unroll
      for (int k = 0; k < 16; ++k) bias[15 - k] = __uint_as_float(t.w[k]);  // dist lo + k
    } else {
      const int lo = rel_row + dtop - 15;
      const int start = lo - ((lo + rel_par) & 1);
      const uint32_t sh = 16u * (uint32_t)(lo - start);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t pr = __builtin_amdgcn_alignbit(t.w[k + 1], t.w[k], sh);
        bias[15 - 2 * k] = Rel::lo(pr);
        bias[14 - 2 * k] = Rel::hi(pr);
      }
    }
    const bool in_band = dtop - 15 >= 0 && dtop < rext;
    if (!wave_all(in_band)) {
#pragma unroll
      for (int e = 0; e < 16; ++e) bias[e] = (uint32_t)(dtop - e) < (uint32_t)rext ? bias[e] : 0.f;
    }
  };

  // 16-bit per-token bias with a 1 / softmax_scale that the bias type holds
  // exactly (any power of two: the reference's 1 / head_dim): each element is
  // added to its score as one v_dot2 of its (realigned) packed pair with
  // (1 / softmax_scale, 0) or (0, 1 / softmax_scale), no unpacking.
  uint32_t dsel_lo = 0, dsel_hi = 0;
  bool dot_ok = false;
  if constexpr (kTokEarly) {
    dsel_lo = Rel::pack_lo(inv_scale);
    dsel_hi = dsel_lo << 16;
    dot_ok = Rel::unpack_lo(dsel_lo) == inv_scale;
  }
  // s[e] += bias / softmax_scale for the 16 keys of block blk, one dot product
  // per element, on a block whose 16 distances are all in the band; false (and
  // nothing added) otherwise
  auto tok_dot = [&](int rel_row, int dtop, const TokRaw& t, f32x16_t& sv) {
    const bool in_band = dtop - 15 >= 0 && dtop < rext;
    if (!dot_ok || t.slow || !wave_all(in_band)) return false;
    if constexpr (Rel::kBytes == 2) {
      const int lo = rel_row + dtop - 15;
      const int start = lo - ((lo + rel_par) & 1);
      const uint32_t sh = 16u * (uint32_t)(lo - start);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t pr = __builtin_amdgcn_alignbit(t.w[k + 1], t.w[k], sh);
        sv[15 - 2 * k] = Rel::dot2(pr, dsel_lo, sv[15 - 2 * k]);
        sv[14 - 2 * k] = Rel::dot2(pr, dsel_hi, sv[14 - 2 * k]);
      }
    }
    return true;
  };

  // Lane constants of the LDS fragment reads.
  // K (A operand of QK): row 32*blk + perm32(col), chunk 2*kk + half.
  // V^T (A operand of PV, two transposing reads): 16-lane group gq = lane / 16,
  // lane i = lane % 16 of the group addresses V[k0 + i/4][d0 + 4*(i%4)] with
  // d0 = 32*db + 16*(gq % 2) and k0 = 32*(t/2) + 16*half + 8*(t%2) (+ 4 for the
  // second read): the keys P holds for key block t (elements 8*(t%2) .. +7 of
  // the S^T block t/2) in the same order.
  const int tr_i = lane & 15;
  const int tr_row = tr_i >> 2;                         // + k0
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (tr_i & 3);  // + 32*db

  auto compute = [&](int kt, const uint16_t* stage) {
    const int kb = kt * kBlockK;
    // Wave-uniform activity / class of this tile.
    const bool active = wrows > 0 && kb < wkend && kb + kBlockK > wkbeg;
    // W^T rows of the next tile (fused projection): fetched once this tile's
    // are consumed, so that only one tile's operands are live at a time
    auto fetch_next = [&] {
      if constexpr (kProj)
        if (kt + 1 < kt_end) proj_fetch(kt + 1);
    };
    if (!active) {
      fetch_next();
      return;
    }
    const int imin = qa, imax = qa + wrows - 1;
    const int jmin = kb, jmax = kb + kBlockK - 1;
    const bool need_mask = jmax >= lk || (p.causal && jmax > imin + qpos) ||
                           (wl >= 0 && imax + qpos - jmin > wl);
    const bool has_bias =
        rext > 0 && (imax + delta - jmin >= 0) && (imin + delta - jmax <= rext - 1);
    const uint16_t* kl = stage;
    const uint16_t* vl = stage + St::kTile;
    if constexpr (kProj && kProjEarly) {
      if (has_bias) proj_fill(kb, 0);
    }
    // 16-bit per-token bias of both key blocks: loads issued ahead of the QK
    // products (fp32 bias keeps them after: its 32 raw registers cost the
    // instantiation that also serves the shared table 2.5%)
    TokRaw traw[kTokEarly ? kNqb : 1][kTokEarly ? kBlockK / 32 : 1];
    if constexpr (kTokEarly) {
      if (has_bias && !bias_in_lds) {
#pragma unroll
        for (int qb = 0; qb < kNqb; ++qb)
#pragma unroll
          for (int blk = 0; blk < kBlockK / 32; ++blk)
            tok_issue(qi[qb] * (int)p.rel_st, qi[qb] + delta - kb - 16 * half - 32 * blk,
                      row_ok[qb], traw[qb][blk]);
        asm volatile("" ::: "memory");  // keep them ahead of the products
      }
    }

    // ---- S^T = K Q^T (each K fragment feeds every row block) ---------------------
    f32x16_t s[kNqb][kBlockK / 32];
#if IFA4_PRIO
    __builtin_amdgcn_s_setprio(1);
#endif
#pragma unroll
    for (int blk = 0; blk < kBlockK / 32; ++blk) {
#pragma unroll
      for (int qb = 0; qb < kNqb; ++qb) s[qb][blk] = f32x16_t{};
      const int row = 32 * blk + perm32(col);
      const uint16_t* krow = kl + row * D;
      const int sw = swz<St::kChunks>(row);
#pragma unroll
      for (int kk = 0; kk < kKSteps; ++kk) {
        const u32x4_t a =
            *reinterpret_cast<const u32x4_t*>(krow + 8 * ((2 * kk + half) ^ sw));
#pragma unroll
        for (int qb = 0; qb < kNqb; ++qb) s[qb][blk] = E::mfma32(a, qf[qb][kk], s[qb][blk]);
      }
    }
#if IFA4_SCHED
    // Keep kLookK fragment reads in flight ahead of the MFMAs (the default
    // schedule waits for each LDS read right before its MFMA).
    {
      constexpr int kReads = (kBlockK / 32) * kKSteps;
      __builtin_amdgcn_sched_group_barrier(0x100, kLookK, 0);
#pragma unroll
      for (int i = 0; i < kReads - kLookK; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, kNqb, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, kNqb * kLookK, 0);
    }
#endif
#if IFA4_PRIO
    __builtin_amdgcn_s_setprio(0);
#endif

#if IFA4_PV2
    // V^T operand of key block t for d block db: two transposing reads.
    auto read_vt = [&](int db, int t) -> u32x4_t {
      u32x2_t part[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int row = 32 * (t >> 1) + 16 * half + 8 * (t & 1) + 4 * r + tr_row;
        const int c = 32 * db + tr_col;  // element column, multiple of 4
        const uint16_t* src = vl + row * D + 8 * ((c >> 3) ^ swz<St::kChunks>(row)) + (c & 7);
        part[r] = __builtin_bit_cast(
            u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                         (__attribute__((address_space(3))) s16x4_t*)src));
      }
      return u32x4_t{part[0][0], part[0][1], part[1][0], part[1][1]};
    };
    // Key block 0's V^T fragments are read now; their latency hides behind the
    // softmax below.  Not on bias tiles of the fused projection, whose bias
    // computation needs the registers (it is long enough to hide them anyway).
    u32x4_t vfr[kDBlocks];
    const bool vfr_early = !(kProj && has_bias);
    if (vfr_early) {
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) vfr[db] = read_vt(db, 0);
    }
#endif

    // ---- logits (log2 domain) and tile max ---------------------------------------
    // Element (blk, e) of a lane is tile-local key 32*blk + 16*half + e; `kc`
    // below drops the lane term, which is folded into the bounds.
    // bias of this lane's 16 keys in key block blk (element e at
    // dist = dbase - 32 blk - e); only on tiles that meet the band
    auto tile_bias = [&](int qb, int blk, float* bias) {
      const int dbase = qi[qb] + delta - kb - 16 * half;  // dist = dbase - kc
      if constexpr (kTable) {
        // element e at dist = dbase - kc: a constant offset from one base
        int j0 = kBiasTop - dbase;  // table index of the lane's key 0
        asm("" : "+v"(j0));          // one base address, the keys as read offsets
        const float* tb = bias_lds + j0;
#pragma unroll
        for (int e = 0; e < 16; ++e) bias[e] = tb[32 * blk + e];
      } else if constexpr (kProj) {
        proj_bias(kb, blk, bias);
      } else {
        const int rel_row = qi[qb] * (int)p.rel_st;  // element offset of the row
        if constexpr (kTokEarly)
          tok_finish(rel_row, dbase - 32 * blk, row_ok[qb], traw[qb][blk], bias);
        else
          token_bias(rel_row, dbase - 32 * blk, row_ok[qb], bias);
      }
    };
    // key-range mask as an additive -inf: visible iff lo <= 16 half + kc <= hi,
    // one unsigned compare per element (an empty range maps to a start no key
    // reaches)
    auto mask_bias = [&](int qb, int blk, float* bias) {
      int hi = lk - 1 - kb;
      if (p.causal) hi = min(hi, qi[qb] + qpos - kb);
      if (!row_ok[qb]) hi = -1;
      const int lo = wl >= 0 ? qi[qb] + qpos - wl - kb : -1;
      const bool none = hi < lo;
      const uint32_t lo_h = none ? 0x80000000u : (uint32_t)(lo - 16 * half);
      const uint32_t span = none ? 0u : (uint32_t)(hi - lo);
#pragma unroll
      for (int e = 0; e < 16; ++e)
        bias[e] = (uint32_t)(32 * blk + e) - lo_h <= span ? bias[e] : -INFINITY;
    };
    float sc = c2;  // factor applied inside the exponent FMA
    float mx[kNqb];
    if constexpr (!kProj) {
      // Scores stay in score units on every tile (the exponent FMA applies
      // softmax_scale * log2(e) to all of them).  Tiles in the bias band and
      // masked tiles (diagonal, window edge, KV tail) add bias / softmax_scale
      // in place, one FMA per element, with -inf as the bias of a masked key
      // (finite scores then give -inf); interior tiles keep the products.
      if constexpr (kTable) {
        // shared table: read on every masked tile too (off the band, the
        // index is clamped into the table's zero padding)
        if (need_mask || has_bias) {
#pragma unroll
          for (int qb = 0; qb < kNqb; ++qb) {
            const int dbase = qi[qb] + delta - kb - 16 * half;  // dist = dbase - kc
            int j0 = min(max(kBiasTop - dbase, 0), kBiasLdsFloats - kBlockK);
            asm("" : "+v"(j0));  // one base address, the keys as read offsets
            const float* tb = bias_lds + j0;
#pragma unroll
            for (int blk = 0; blk < kBlockK / 32; ++blk) {
              float bias[16];
#pragma unroll
              for (int e = 0; e < 16; ++e) bias[e] = tb[32 * blk + e];
              if (need_mask) mask_bias(qb, blk, bias);
#pragma unroll
              for (int e = 0; e < 16; ++e)
                s[qb][blk][e] = fmaf(bias[e], inv_scale, s[qb][blk][e]);
            }
          }
        }
      } else if (has_bias) {
#pragma unroll
        for (int qb = 0; qb < kNqb; ++qb) {
#pragma unroll
          for (int blk = 0; blk < kBlockK / 32; ++blk) {
            bool done = false;
            if constexpr (kTokEarly) {
              const int dtop = qi[qb] + delta - kb - 16 * half - 32 * blk;
              done = tok_dot(qi[qb] * (int)p.rel_st, dtop, traw[qb][blk], s[qb][blk]);
            }
            if (done) {
              if (need_mask) {
                float keep[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) keep[e] = 0.f;
                mask_bias(qb, blk, keep);
#pragma unroll
                for (int e = 0; e < 16; ++e) s[qb][blk][e] += keep[e];
              }
            } else {
              float bias[16];
              tile_bias(qb, blk, bias);
              if (need_mask) mask_bias(qb, blk, bias);
#pragma unroll
              for (int e = 0; e < 16; ++e)
                s[qb][blk][e] = fmaf(bias[e], inv_scale, s[qb][blk][e]);
            }
          }
        }
      } else if (need_mask) {  // masked tile off the band: the mask alone, in place
#pragma unroll
        for (int qb = 0; qb < kNqb; ++qb) {
#pragma unroll
          for (int blk = 0; blk < kBlockK / 32; ++blk) {
            float keep[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) keep[e] = 0.f;
            mask_bias(qb, blk, keep);
#pragma unroll
            for (int e = 0; e < 16; ++e) s[qb][blk][e] += keep[e];
          }
        }
      }
#pragma unroll
      for (int qb = 0; qb < kNqb; ++qb) {
        float m = -INFINITY;
#pragma unroll
        for (int blk = 0; blk < kBlockK / 32; ++blk)
#pragma unroll
          for (int e = 0; e < 16; ++e) m = fmaxf(m, s[qb][blk][e]);
        mx[qb] = m * c2;
      }
    } else if (need_mask || has_bias) {
      // fused projection: logits in log2 units on bias and masked tiles (the
      // per-element form keeps fewer registers live beside the projection)
      sc = 1.f;
#pragma unroll
      for (int qb = 0; qb < kNqb; ++qb) {
        int hi = lk - 1 - kb;
        if (p.causal) hi = min(hi, qi[qb] + qpos - kb);
        if (!row_ok[qb]) hi = -1;
        const int lo = wl >= 0 ? qi[qb] + qpos - wl - kb : -1;
        const int hi_h = hi - 16 * half, lo_h = lo - 16 * half;
        float m = -INFINITY;
#pragma unroll
        for (int blk = 0; blk < kBlockK / 32; ++blk) {
          float bias[16];
          if (has_bias) tile_bias(qb, blk, bias);
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int kc = 32 * blk + e;
            float x = s[qb][blk][e] * c2;
            if (has_bias) x = fmaf(bias[e], kLog2e, x);
            if (need_mask) x = (kc >= lo_h && kc <= hi_h) ? x : -INFINITY;
            s[qb][blk][e] = x;
            m = fmaxf(m, x);
          }
        }
        mx[qb] = m;
      }
    } else {
#pragma unroll
      for (int qb = 0; qb < kNqb; ++qb) {
        float m = -INFINITY;
#pragma unroll
        for (int blk = 0; blk < kBlockK / 32; ++blk)
#pragma unroll
          for (int e = 0; e < 16; ++e) m = fmaxf(m, s[qb][blk][e]);
        mx[qb] = m * c2;
      }
    }

    fetch_next();

#if IFA4_PV2
    if (!vfr_early) {
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) vfr[db] = read_vt(db, 0);
    }
#endif

    // ---- deferred rescale ----------------------------------------------------------
    bool grow[kNqb];
    bool any_grow = false;
#pragma unroll
    for (int qb = 0; qb < kNqb; ++qb) {
      mx[qb] = max_xor32(mx[qb]);
      const float m_cand = fmaxf(m_run[qb], mx[qb]);
      grow[qb] = m_cand > m_run[qb] + kRescaleThreshold;
      mx[qb] = m_cand;
      any_grow |= grow[qb];
    }
    if (wave_any(any_grow)) {
#pragma unroll
      for (int qb = 0; qb < kNqb; ++qb) {
        const float m_upd = grow[qb] ? mx[qb] : m_run[qb];
        const float alpha = grow[qb] ? fast_exp2(m_run[qb] - m_upd) : 1.f;
        l_run[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < kDBlocks; ++db)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[qb][db][e] *= alpha;
        m_run[qb] = m_upd;
      }
    }

#if IFA4_PV2
    // ---- P = exp2(x - m) per 16-key block t, then O^T += V^T P^T -------------------
    // Key-block-major: the MFMAs of block t run while block t+1's exponentials
    // are computed and its V^T fragments are read.
    float m_use[kNqb];
#pragma unroll
    for (int qb = 0; qb < kNqb; ++qb) m_use[qb] = m_run[qb] == -INFINITY ? 0.f : m_run[qb];
    auto make_p = [&](int qb, int t) -> u32x4_t {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pv[e] = fast_exp2(fmaf(s[qb][t >> 1][8 * (t & 1) + e], sc, -m_use[qb]));
        l_run[qb] += pv[e];
      }
      return u32x4_t{E::pack2(pv[0], pv[1]), E::pack2(pv[2], pv[3]), E::pack2(pv[4], pv[5]),
                     E::pack2(pv[6], pv[7])};
    };
    u32x4_t pcur[kNqb];
#pragma unroll
    for (int qb = 0; qb < kNqb; ++qb) pcur[qb] = make_p(qb, 0);
#if IFA4_PRIO
    __builtin_amdgcn_s_setprio(1);
#endif
#pragma unroll
    for (int t = 0; t < kBlockK / 16; ++t) {
      u32x4_t pnext[kNqb];
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
        for (int qb = 0; qb < kNqb; ++qb) o[qb][db] = E::mfma32(vfr[db], pcur[qb], o[qb][db]);
        if (t + 1 < kBlockK / 16) vfr[db] = read_vt(db, t + 1);
      }
      if (t + 1 < kBlockK / 16) {
#pragma unroll
        for (int qb = 0; qb < kNqb; ++qb) pnext[qb] = make_p(qb, t + 1);
#pragma unroll
        for (int qb = 0; qb < kNqb; ++qb) pcur[qb] = pnext[qb];
      }
    }
#if IFA4_SCHED
    // Per key block t < 3: each MFMA followed by the two reads of the next
    // block's fragment and a share of the next block's exponentials.
    {
      constexpr int kT = kBlockK / 16;
      constexpr int kPValu = IFA4_PVALU;  // ~28 VALU/TRANS per block of P over 4 MFMAs
#pragma unroll
      for (int t = 0; t < kT - 1; ++t) {
#pragma unroll
        for (int db = 0; db < kDBlocks; ++db) {
          __builtin_amdgcn_sched_group_barrier(0x008, kNqb, 1);
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
          __builtin_amdgcn_sched_group_barrier(0x402, kPValu * kNqb, 1);
        }
      }
      __builtin_amdgcn_sched_group_barrier(0x008, kNqb * kDBlocks, 1);
    }
#endif
#if IFA4_PRIO
    __builtin_amdgcn_s_setprio(0);
#endif
  };
#else
    // ---- P = exp2(x - m), packed to the PV B operand, row sum ----------------------
    u32x4_t pb[kNqb][kBlockK / 16];
#pragma unroll
    for (int qb = 0; qb < kNqb; ++qb) {
      const float m_use = m_run[qb] == -INFINITY ? 0.f : m_run[qb];
#pragma unroll
      for (int t = 0; t < kBlockK / 16; ++t) {
        float pv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pv[e] = fast_exp2(fmaf(s[qb][t >> 1][8 * (t & 1) + e], sc, -m_use));
          l_run[qb] += pv[e];
        }
        pb[qb][t] = u32x4_t{E::pack2(pv[0], pv[1]), E::pack2(pv[2], pv[3]),
                            E::pack2(pv[4], pv[5]), E::pack2(pv[6], pv[7])};
      }
    }

    // ---- O^T += V^T P^T (each V^T fragment feeds every row block) -------------------
#if IFA4_PRIO
    __builtin_amdgcn_s_setprio(1);
#endif
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
      for (int t = 0; t < kBlockK / 16; ++t) {
        u32x2_t part[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int row = 32 * (t >> 1) + 16 * half + 8 * (t & 1) + 4 * r + tr_row;
          const int c = 32 * db + tr_col;  // element column, multiple of 4
          const uint16_t* src = vl + row * D + 8 * ((c >> 3) ^ swz<St::kChunks>(row)) + (c & 7);
          part[r] = __builtin_bit_cast(
              u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                           (__attribute__((address_space(3))) s16x4_t*)src));
        }
        const u32x4_t a = {part[0][0], part[0][1], part[1][0], part[1][1]};
#pragma unroll
        for (int qb = 0; qb < kNqb; ++qb) o[qb][db] = E::mfma32(a, pb[qb][t], o[qb][db]);
      }
    }
#if IFA4_SCHED
    // Same for the PV product: kLookV operand pairs (two transposing reads
    // each) in flight ahead of the MFMAs.
    {
      constexpr int kGroups = kDBlocks * (kBlockK / 16);
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * kLookV, 1);
#pragma unroll
      for (int i = 0; i < kGroups - kLookV; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, kNqb, 1);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, kNqb * kLookV, 1);
    }
#endif
#if IFA4_PRIO
    __builtin_amdgcn_s_setprio(0);
#endif
  };
#endif

  // ---- pipeline: DMA of tile kt+1 in flight while tile kt is computed -------------
  // The DMA is invisible to the compiler (dma_16), so these waits and barriers are
  // the only ordering between a stage's DMA and its reads.
#if IFA4_ONEBAR
  // One barrier per tile: wait for this wave's part of tile kt (its DMA was
  // issued a step earlier), barrier (every part landed, and every wave is done
  // with tile kt-1, whose stage tile kt+1 now overwrites), then issue tile
  // kt+1's DMA and compute tile kt.
  auto step = [&](int kt, uint16_t* cur, uint16_t* nxt) {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + 1 < kt_end) dma_tile(kt + 1, nxt);
    compute(kt, cur);
  };
#else
  // Two barriers per tile: issue tile kt+1's DMA; wait until only it is
  // outstanding for this wave; barrier (every wave's part of tile kt landed);
  // compute; barrier (the stage may be overwritten next).  1.4% slower.
  static_assert(!kProj, "the projection fetches W^T rows with the one-barrier pipeline");
  auto step = [&](int kt, uint16_t* cur, uint16_t* nxt) {
    if (kt + 1 < kt_end) {
      dma_tile(kt + 1, nxt);
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(St::kDmaPerWave));
    } else {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    compute(kt, cur);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
#endif
  // The bias table (shared-table layout) is read with the Q fragments and the
  // first tile; one wait for all three, then it goes to LDS.  The first tile's
  // barrier publishes it.
  constexpr int kBiasPer = (2 * kBiasPad + kBiasLdsMax + kThreads - 1) / kThreads;
  float tab[kBiasPer];
  if (bias_in_lds) {
#pragma unroll
    for (int i = 0; i < kBiasPer; ++i) {
      const int idx = tid + i * kThreads;  // table index
      const int dist = kBiasTop - idx;
      const uint32_t off = (uint32_t)dist < (uint32_t)rext ? (uint32_t)dist * Rel::kBytes
                                                            : kOutOfRange;
      tab[i] = Rel::load(rrel, off);
    }
  }
  // Fused projection: this lane's row of r (channels 8 * half .. +7) as the B
  // operand, and the first tile's W^T rows.
  if constexpr (kProj) {
    float rv[8];
    const uint32_t roff = (uint32_t)((qa + col) * (int)p.rel_st + 8 * half) * Rel::kBytes;
#pragma unroll
    for (int c = 0; c < 8; ++c) rv[c] = Rel::load(rrel, roff + c * Rel::kBytes);
    split_bf16x8(rv, r_hi, r_lo);
    if (kt_beg < kt_end) proj_fetch(kt_beg);
  }
  if (kt_beg < kt_end) dma_tile(kt_beg, stage0);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  if (bias_in_lds) {
#pragma unroll
    for (int i = 0; i < kBiasPer; ++i) {
      const int idx = tid + i * kThreads;
      if (idx < 2 * kBiasPad + kBiasLdsMax) bias_lds[idx] = tab[i];
    }
    __builtin_amdgcn_s_waitcnt(kLgkm0);
  }
  for (int kt = kt_beg; kt < kt_end; kt += 2) {
    step(kt, stage0, stage1);
    if (kt + 1 < kt_end) step(kt + 1, stage1, stage0);
  }

  // ---- epilogue: normalise, store O and LSE (split KV: this chunk's partial) -----
  // The lane's row and half are derived again from the lane id (v_mbcnt), so
  // that no register has to carry them across the KV loop.
  const int lane_e = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int half_e = lane_e >> 5;
#pragma unroll
  for (int qb = 0; qb < kNqb; ++qb) {
    const float l_tot = add_xor32(l_run[qb]);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const int qi_e = qa + 32 * qb + (lane_e & 31);
    const bool ok_e = qi_e < lq;
    if (ok_e && nch > 1) {
      // normalised O of the chunk (fp32) and its LSE in log2 units
      const int64_t prow = ((int64_t)chunk * p.n_heads + head) * p.total_q + qs + qi_e;
      float* pbase = p.part_o + prow * D;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          *reinterpret_cast<f32x4_t*>(pbase + 32 * db + 8 * i + 4 * half_e) =
              f32x4_t{o[qb][db][4 * i] * inv, o[qb][db][4 * i + 1] * inv,
                      o[qb][db][4 * i + 2] * inv, o[qb][db][4 * i + 3] * inv};
      if (half_e == 0) p.part_lse[prow] = l_tot > 0.f ? m_run[qb] + __log2f(l_tot) : -INFINITY;
    } else if (ok_e) {
      uint16_t* obase = static_cast<uint16_t*>(p.out) + (int64_t)(qs + qi_e) * p.o_st +
                        (int64_t)head * p.o_sh;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 32 * db + 8 * i + 4 * half_e;
          const u32x2_t w = {E::pack2(o[qb][db][4 * i] * inv, o[qb][db][4 * i + 1] * inv),
                             E::pack2(o[qb][db][4 * i + 2] * inv, o[qb][db][4 * i + 3] * inv)};
          *reinterpret_cast<u32x2_t*>(obase + d) = w;
        }
      }
      if (p.lse != nullptr && half_e == 0) {
        const float lse = l_tot > 0.f ? (m_run[qb] + __log2f(l_tot)) * kLn2 : -INFINITY;
        p.lse[(int64_t)head * p.lse_sh + qs + qi_e] = lse;
      }
    }
  }
}

// Merge of split-KV partials (second pass after a split launch): kMergeParts
// workgroups per (q tile, head, sequence), each an eighth of the tile's rows
// (against a quarter: 1.3% faster on one sequence of 4096 over 4 heads, 3% at
// 2048, within 1% elsewhere; sixteenths no better); a
// tile whose range did not split was written by the prefill kernel itself and
// is skipped.  32 threads share a row (head_dim / 32 consecutive d values each)
// and a thread holds kRows rows; chunks go in rounds of kChunkBatch whose loads
// (rows x chunks) are all in flight at once, merged online (running max over
// the chunks' LSEs).
constexpr int kMergeThreads = IFA4_MERGE_THREADS;
constexpr int kMergeParts = IFA4_MERGE_PARTS;
template <typename Sh, int D, typename Tag>
__global__ __launch_bounds__(kMergeThreads) void prefill_merge_kernel(PrefillParams p) {
  using E = Elem<Tag>;
  constexpr int kTpr = 32;                          // threads per row
  constexpr int kPer = D / kTpr;                    // d values per thread
  constexpr int kStride = kMergeThreads / kTpr;     // rows per pass of the workgroup
  constexpr int kRows = Sh::kBlockQ / kMergeParts / kStride;  // rows per thread
  static_assert(kRows >= 1 && kRows * kStride * kMergeParts == Sh::kBlockQ,
                "merge workgroups cover the query tile's rows exactly");
  const int qtile = blockIdx.x / kMergeParts, part = blockIdx.x % kMergeParts;
  const int head = blockIdx.y, seq = blockIdx.z;
  const SeqBounds bq = seq_bounds(p.cu_q, seq, p.total_q);
  const SeqBounds bk = seq_bounds(p.cu_k, seq, p.total_k);
  const int q0 = qtile * Sh::kBlockQ;
  if (q0 >= bq.len) return;
  const int qpos = p.bottom_right ? bk.len - bq.len : 0;
  const TileRange tr = tile_range<Sh>(p, q0, bq.len, bk.len, qpos);
  const int nch = tile_chunks(p, tr);
  if (nch <= 1) return;
  const int r0 = q0 + part * (Sh::kBlockQ / kMergeParts) + (int)threadIdx.x / kTpr;
  const int d0 = ((int)threadIdx.x % kTpr) * kPer;
  const int64_t chunk_rows = (int64_t)p.n_heads * p.total_q;
  const int64_t row0 = (int64_t)head * p.total_q + bq.start;
  float m[kRows], l[kRows], acc[kRows][kPer];
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
#pragma unroll
    for (int e = 0; e < kPer; ++e) acc[i][e] = 0.f;
  }
  // kChunkBatch chunks per round: every load of a round (its rows x chunks)
  // is issued before the first is used
  constexpr int kChunkBatch = IFA4_MERGE_BATCH;
  // Rounds start at absolute chunk indices that are multiples of kChunkBatch
  // (slot k of this query tile is absolute chunk tr.beg / chunk_tiles + k), so
  // the chunks meet in the same rounds whatever the pruning: chunks a pruned
  // range drops hold no key (LSE -inf) and leave the running sums bit-unchanged.
  const int lead = (tr.beg / p.chunk_tiles) % kChunkBatch;
  for (int c0 = -lead; c0 < nch; c0 += kChunkBatch) {
    float ls[kChunkBatch][kRows];
    float os[kChunkBatch][kRows][kPer];
#pragma unroll
    for (int cb = 0; cb < kChunkBatch; ++cb) {
#pragma unroll
      for (int i = 0; i < kRows; ++i) {
        const int row = r0 + kStride * i;
        const bool ok = row < bq.len && c0 + cb >= 0 && c0 + cb < nch;
        const int64_t prow = (ok ? c0 + cb : 0) * chunk_rows + row0 + row;
        ls[cb][i] = ok ? p.part_lse[prow] : -INFINITY;
        if constexpr (kPer == 4) {
          const f32x4_t v =
              ok ? *reinterpret_cast<const f32x4_t*>(p.part_o + prow * D + d0) : f32x4_t{};
#pragma unroll
          for (int e = 0; e < 4; ++e) os[cb][i][e] = v[e];
        } else {
#pragma unroll
          for (int e = 0; e < kPer; ++e) os[cb][i][e] = ok ? p.part_o[prow * D + d0 + e] : 0.f;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      float mn = m[i];
#pragma unroll
      for (int cb = 0; cb < kChunkBatch; ++cb) mn = fmaxf(mn, ls[cb][i]);
      const float mu = mn == -INFINITY ? 0.f : mn;
      const float a_old = fast_exp2(m[i] - mu);
      l[i] *= a_old;
#pragma unroll
      for (int e = 0; e < kPer; ++e) acc[i][e] *= a_old;
#pragma unroll
      for (int cb = 0; cb < kChunkBatch; ++cb) {
        const float a_new = fast_exp2(ls[cb][i] - mu);
        l[i] += a_new;
#pragma unroll
        for (int e = 0; e < kPer; ++e) acc[i][e] += a_new * os[cb][i][e];
      }
      m[i] = mn;
    }
  }
#pragma unroll
  for (int i = 0; i < kRows; ++i) {
    const int row = r0 + kStride * i;
    if (row >= bq.len) continue;
    const float inv = l[i] > 0.f ? 1.f / l[i] : 0.f;
    uint16_t* dst = static_cast<uint16_t*>(p.out) + (int64_t)(bq.start + row) * p.o_st +
                    (int64_t)head * p.o_sh + d0;
    if constexpr (kPer == 4) {
      *reinterpret_cast<u32x2_t*>(dst) = u32x2_t{E::pack2(acc[i][0] * inv, acc[i][1] * inv),
                                                 E::pack2(acc[i][2] * inv, acc[i][3] * inv)};
    } else {
      *reinterpret_cast<uint32_t*>(dst) = E::pack2(acc[i][0] * inv, acc[i][1] * inv);
    }
    if (p.lse != nullptr && d0 == 0)
      p.lse[(int64_t)head * p.lse_sh + bq.start + row] =
          l[i] > 0.f ? (m[i] + __log2f(l[i])) * kLn2 : -INFINITY;
  }
}

template <typename Sh, int D, typename Tag, typename Rel, bool kProj, bool kTab = false>
hipError_t launch_prefill_t(const PrefillParams& p_in, hipStream_t stream) {
  PrefillParams p = p_in;
  if (p.n_chunks < 1) p.n_chunks = 1;
  const int per_tile = p.n_heads * p.batch;
  const int64_t blocks = (int64_t)p.n_qtiles * p.n_chunks * per_tile;
  const int pairs = p.batch * (p.n_heads / p.group);
  p.xcd_pairs = pairs % 8 == 0 ? pairs / 8 : 0;
  if (blocks <= 0) return hipSuccess;
  hipLaunchKernelGGL((prefill_fwd_kernel<Sh, D, Tag, Rel, kProj, kTab>), dim3((unsigned)blocks),
                     dim3(Sh::kThreads), 0, stream, p);
  if constexpr (!kProj) {  // the fused projection never splits
    if (p.chunk_tiles > 0) {
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL((prefill_merge_kernel<Sh, D, Tag>),
                         dim3(p.n_qtiles * kMergeParts, p.n_heads, p.batch), dim3(kMergeThreads),
                         0, stream, p);
    }
  }
  return hipGetLastError();
}

template <int D, typename Tag>
hipError_t launch_prefill_rel(const PrefillParams& p, hipStream_t stream) {
  if (p.wt != nullptr) {  // fused projection: r in bf16 or fp32
    return p.rel_dtype == 2 ? launch_prefill_t<ProjShape, D, Tag, RelF32, true>(p, stream)
                            : launch_prefill_t<ProjShape, D, Tag, RelBf16, true>(p, stream);
  }
  // one per-head table shared by every token (token stride 0), short enough
  // for LDS: the table instantiation; per-token rows (or no bias): the other
  const bool tab =
      IFA4_BIAS_LDS && p.rel_st == 0 && p.rel_extent > 0 && p.rel_extent <= kBiasLdsMax;
  if (tab) {
    switch (p.rel_dtype) {
      case 0: return launch_prefill_t<Shape, D, Tag, RelBf16, false, true>(p, stream);
      case 1: return launch_prefill_t<Shape, D, Tag, RelF16, false, true>(p, stream);
      default: return launch_prefill_t<Shape, D, Tag, RelF32, false, true>(p, stream);
    }
  }
  switch (p.rel_dtype) {
    case 0: return launch_prefill_t<Shape, D, Tag, RelBf16, false>(p, stream);
    case 1: return launch_prefill_t<Shape, D, Tag, RelF16, false>(p, stream);
    default: return launch_prefill_t<Shape, D, Tag, RelF32, false>(p, stream);
  }
}

}  // namespace

int prefill_block_q() { return Shape::kBlockQ; }
int prefill_proj_block_q() { return ProjShape::kBlockQ; }
int prefill_block_k() { return Shape::kBlockK; }
int prefill_waves() { return Shape::kWaves; }

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
