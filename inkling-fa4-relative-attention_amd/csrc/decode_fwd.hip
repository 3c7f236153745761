// Split-KV decode of relative-bias attention for gfx950 (MI355X), stream-K.
//
// Replaces _fa4_rel_attn_decode_kernel and its per-sequence launch loop
// (src/inkling_fa4/triton_kernel_decode.py:22-124,127-170).  Semantics follow
// the reference oracle (src/inkling_fa4/reference.py:19-40) for Lq = 1:
// query local index i = 0, dist = (1 - Lk) - j, causal keeps j <= 0 only, and
// the left window never masks (i - j <= 0).  With bottom-right alignment
// (IFA4_FLAG_BOTTOM_RIGHT) the query sits at key Lk - 1: dist = (Lk - 1) - j,
// causal keeps every key, the window keeps j >= Lk - 1 - window_left.
//
// Work decomposition.  A "segment" is one (sequence, kv head); it holds the
// 32-key steps of its visible keys (decode_keys).  All segments' steps are laid
// end to end (sequence-major, kv head minor), weighted in units (kUnits per
// step, kBandUnits per step with bias), and W persistent waves (about one
// resident round on the chip) each take an equal contiguous range of P =
// ceil(T / W) units, computing the steps that start in it.  A wave therefore
// streams K/V without gaps across segment
// boundaries; where its range leaves a segment it writes one (o, lse) partial
// and carries on (no wave ends after each split, which would hold its slot
// until its stores drain: measured 11.8 us of 117 on the benchmark batch).
// Every wave derives the same T, P and its own start from cu_seqlens, so the
// split needs no host synchronisation and no atomics.
//
// Pass 1 (decode_stream_kernel), per 32-key step of a segment:
//   * K and V rows arrive with coalesced, non-temporal 16-byte buffer loads
//     kNbuf - 1 steps ahead of the compute (a ring of register buffers), rows
//     past the segment end read as zero; the next segment's Q (all G query
//     heads of the kv head) arrives ahead of it by LDS DMA into a ring of kNbuf
//     slots;
//   * K goes through a small padded LDS tile into the A operand of
//     S^T = K Q^T on v_mfma_f32_16x16x32 (B = the G query rows, zero padded to
//     16 columns); an fp8 cache converts to the 16-bit type on the way;
//   * online softmax per head (exp2, deferred rescale);
//   * O^T += V^T P^T on v_mfma_f32_16x16x32: V through a swizzled LDS tile read
//     with transposing ds_read_b64_tr_b16, P^T straight from the S^T layout.
// Partial of (segment s, wave w) -> workspace slot s + w (slots increase with
// w, so the map is one-to-one); the wave holding a segment's first step also
// records the range of waves that cover the segment.
//
// Pair mode (kPair: an fp8 cache, d 128, contiguous or paged, whose kv heads
// 2m and 2m + 1 sit side by side in every row).  A segment is (sequence, kv head pair) and a wave
// loads whole 256-byte rows of both heads, so each step reads two contiguous
// 8 KiB runs (one kv head per wave would read 128-byte halves of 256-byte
// rows).  K and V stay fp8 in LDS (both tiles 8 KiB, so two waves per SIMD
// still fit) and convert to the 16-bit type at the MFMA operand: K rows by
// 8-byte reads, Vᵀ by transposing 8-bit reads (ds_read_b64_tr_b8).  The query
// heads of both kv heads share the 16 S^T columns: QK runs each head's
// half of the row against the same Q registers into two accumulators and a
// column keeps the one of its own kv head; PV adds each head's Vᵀ times P with
// the other head's columns zeroed.
//
// Pass 2 (decode_combine_kernel): per (head, sequence) merge of the segment's
// partials by log-sum-exp (16 part groups of a workgroup each merge online,
// then meet in LDS); writes out (q dtype) and lse (natural log).
#include "ifa4_device.hpp"
#include "ifa4_kernels.h"

#ifndef IFA4_DECODE_NT
#define IFA4_DECODE_NT 1
#endif
#ifndef IFA4_FP8_CVT2
#define IFA4_FP8_CVT2 1
#endif
// Split the combine of segments with many parts over several workgroups
// (sweep knob; 0: one workgroup per (head, sequence)).
#ifndef IFA4_COMBINE_SPLIT
#define IFA4_COMBINE_SPLIT 1
#endif
// Register budget of the stream pass: at least this many waves per SIMD
// (2: at most 256 VGPRs, so that 2048 persistent waves fit in one round).
#ifndef IFA4_DECODE_WPE
#define IFA4_DECODE_WPE 2
#endif
// Register buffers of K/V steps in flight per wave for an fp8 cache (the wave
// computes one step while the loads of the next kNbuf - 1 are outstanding);
// 16-bit caches use 2 (a third buffer of their twice-larger steps does not fit
// the register budget).
#ifndef IFA4_DECODE_NBUF_FP8
#define IFA4_DECODE_NBUF_FP8 2
#endif
#ifndef IFA4_DECODE_PAIR_OVERLAP
#define IFA4_DECODE_PAIR_OVERLAP 1
#endif
// Pair mode: step buffers per wave and the register budget (waves per SIMD).
#ifndef IFA4_DECODE_NBUF_PAIR
#define IFA4_DECODE_NBUF_PAIR 2
#endif
#ifndef IFA4_DECODE_WPE_PAIR
#define IFA4_DECODE_WPE_PAIR 2
#endif

namespace ifa4 {
namespace {

constexpr int kStep = 32;  // keys per pipeline step of a decode wave
// Stream-K weights: a step counts kUnits units of work, a step with keys in a
// bottom-right bias band kBandUnits (its bias loads and adds), and the waves
// take equal ranges of units, so the waves holding caches' ends (where the
// band is) get fewer steps.
#ifndef IFA4_DECODE_BAND_UNITS
#define IFA4_DECODE_BAND_UNITS 7
#endif
constexpr int kUnits = 4;
constexpr int kBandUnits = IFA4_DECODE_BAND_UNITS;
static_assert(kBandUnits >= kUnits && kBandUnits <= 2 * kUnits, "band step weight");

// K/V stream loads.  Each cache byte is read once per call, so the loads are
// marked non-temporal: a streaming-read probe over the 580 MB benchmark cache
// measured 6.2-6.6 TB/s with non-temporal loads against 5.7 TB/s without.
__device__ __forceinline__ u32x4_t kv_load(rsrc_t r, uint32_t byte_off) {
#if IFA4_DECODE_NT
  return buf_load_16_nt(r, byte_off);
#else
  return buf_load_16(r, byte_off);
#endif
}
constexpr int kDecodeFp8MaxGroup = 16;

// Lane layouts of a decode wave (D = head_dim, Eb = bytes per K/V element):
//   row layout (loads, PV):  r = lane / kLpr is the row within a wave load,
//                            c = lane % kLpr the 16-byte chunk (16/Eb elements);
//   S^T layout (QK):         n = lane % 16 the query head, g = lane / 16.
template <int D, int Eb>
struct DecodeShape {
  static constexpr int kLpr = D * Eb / 16;     // lanes per K/V row
  static constexpr int kEpl = 16 / Eb;         // elements of a row per lane
  static constexpr int kRpi = 64 / kLpr;       // rows per wave load
  static constexpr int kLoads = kStep / kRpi;  // wave loads per tensor per step
  static constexpr int kGroupRows = kRpi > 8 ? kRpi : 8;  // paged: rows per resource
  static constexpr int kPitch = D + 8;         // LDS K row pitch (elements)
  static constexpr int kKSteps = D / 32;       // 16x16x32 MFMAs per 16 keys
  static constexpr int kChunks = D / 8;        // 16-byte chunks of a 16-bit row
  static constexpr int kDBlocks = D / 16;      // 16-row blocks of O^T (PV MFMAs per step)
};

// V tile of one step in LDS: [kStep][D] 16-bit, row-major, unpadded; chunk c of
// row r sits at chunk c ^ vswz(r).  A transposing read of the PV A operand
// covers four consecutive rows and one chunk pair per 16-lane group, eight
// consecutive rows per half wave: the swizzle gives those rows distinct chunk
// pairs (and, with two rows per 256-byte bank line at D = 64, distinct halves).
template <int D>
__device__ __forceinline__ int vswz(int row) {
  constexpr int kRowsPerLine = 128 / D;
  return 2 * ((row / kRowsPerLine) & (D / 16 - 1));
}

// Pair mode tiles in LDS: fp8 rows of both heads (2 D = 256 bytes) at a pitch
// of 272 bytes, so that 16 rows read at one column hit 16 distinct bank
// quads.  The keys of a step are permuted: S^T row 4g + j of key block blk is
// key 8g + 4 blk + j (pair_key), so a 16-lane group's eight P k-slots are the
// eight consecutive keys 8g..8g+7.  K holds one key block at a time (16 rows:
// wave load 2t + blk to tile rows 4t..4t+3), V the whole step.  Vᵀ is read by
// ds_read_b64_tr_b8: in each 16-lane group, lane 2j (2j + 1) points at bytes
// 0..7 (8..15) of a 16-byte column block of row j, and lane i receives byte i
// of the block from rows j = 0..7 (measured on gfx950).
constexpr int kPairPitch = 272;
// First key (from the step's first) of S^T rows 4g..4g+3 of key block blk.
template <bool kPair>
__device__ __forceinline__ int pair_key(int blk, int g) {
  return kPair ? 8 * g + 4 * blk : 16 * blk + 4 * g;
}

// 8 fp8 bytes -> the 16-bit MFMA operand (exact).
template <typename E>
__device__ __forceinline__ u32x4_t fp8x8_operand(u32x2_t w) {
  return u32x4_t{E::template fp8x2<false>(w[0]), E::template fp8x2<true>(w[0]),
                 E::template fp8x2<false>(w[1]), E::template fp8x2<true>(w[1])};
}

// 8 fp8 (OCP e4m3) values in two dwords (byte i = element i) -> fp32, exactly;
// every e4m3 value is also exact in bf16 and fp16.
__device__ __forceinline__ void fp8x8_to_f32(uint32_t w0, uint32_t w1, float* f) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w0, false);
  const f32x2_t b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w0, true);
  const f32x2_t c = __builtin_amdgcn_cvt_pk_f32_fp8((int)w1, false);
  const f32x2_t d = __builtin_amdgcn_cvt_pk_f32_fp8((int)w1, true);
  f[0] = a[0]; f[1] = a[1]; f[2] = b[0]; f[3] = b[1];
  f[4] = c[0]; f[5] = c[1]; f[6] = d[0]; f[7] = d[1];
}

// One Q slot in LDS: the G heads of a kv head, [G][D], in whole 1 KiB DMAs.
template <int D, int G>
struct DecodeQ {
  static constexpr int kDma = (G * D + 511) / 512;
  static constexpr int kElems = 512 * kDma;
};

// Visible keys [kbeg, kend) of the single query of a sequence with lk keys.
// Top-left (the reference oracle): causal keeps key 0 only, the left window
// never masks (i - j <= 0).  Bottom-right: query 0 sits at key lk - 1, so
// causal keeps every key and the window keeps keys >= lk - 1 - window_left.
// Steps start at the 32-key boundary kfirst <= kbeg (keys below kbeg are
// masked), so a step never straddles a 32-key boundary of the sequence.
struct KeyRange {
  int kbeg, kfirst, kend;
};
__device__ __forceinline__ KeyRange decode_keys(const DecodeParams& p, int lk) {
  KeyRange r;
  if (p.bottom_right) {
    r.kend = lk;
    r.kbeg = p.window_left >= 0 ? max(0, lk - 1 - p.window_left) : 0;
  } else {
    r.kend = p.causal ? min(lk, 1) : lk;
    r.kbeg = 0;
  }
  r.kfirst = r.kbeg & ~(kStep - 1);
  return r;
}

// Steps of a sequence: 32-key steps over [kfirst, kend), 0 when it does not
// hold exactly one query.
__device__ __forceinline__ int seq_steps(int lq, const KeyRange& r) {
  const int n = r.kend - r.kfirst;
  return (lq == 1 && n > 0) ? (n + kStep - 1) / kStep : 0;
}

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int x, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(x, off);
    if (lane >= off) x += t;
  }
  return x;
}

// Per-lane view of 64 consecutive sequences (lane i <-> sequence base + i).
// Work is counted in units (kUnits per step, kBandUnits per band step); each
// of a sequence's kv heads is a segment of `units` units.
struct SeqChunk {
  int base;        // first sequence of the chunk (wave-uniform)
  int total_incl;  // units of all sequences up to the end of the chunk (uniform)
  int steps, excl, qs, ks, kbeg, kend, lk;  // this lane's sequence
};

// Steps of a segment before its first bias-band step (bottom-right alignment
// puts the last rel_extent keys in the band; top-left decode has no band).
__device__ __forceinline__ int band_start(const DecodeParams& p, int kbeg, int kend, int lk,
                                          int steps) {
  if (!p.bottom_right || p.rel_extent <= 0 || steps <= 0) return steps;
  const int band0 = max(kbeg, lk - p.rel_extent);  // first key with bias
  return band0 < kend ? min(steps, (band0 - (kbeg & ~(kStep - 1))) / kStep) : steps;
}
// Units of a segment of `steps` steps, nb of them before the band.
__device__ __forceinline__ int seg_units(int steps, int nb) {
  return kUnits * nb + kBandUnits * (steps - nb);
}

// Keys of sequence `seq` in a paged cache: seqused_k clamped to what the
// table row can address.
__device__ __forceinline__ int paged_len(const DecodeParams& p, int seq) {
  const int cap = p.max_blocks << p.block_shift;
  return min(max(p.seqused_k[seq], 0), cap);
}

template <bool kPaged>
__device__ __forceinline__ SeqChunk load_chunk(const DecodeParams& p, int base, int excl0,
                                               int lane) {
  SeqChunk c;
  c.base = base;
  const int seq = base + lane;
  c.steps = 0;
  c.qs = c.ks = c.kbeg = c.kend = c.lk = 0;
  if (seq < p.batch) {
    const SeqBounds bq = seq_bounds(p.cu_q, seq, p.total_q);
    c.qs = bq.start;
    const int lq = bq.len;
    if constexpr (kPaged) {
      c.lk = paged_len(p, seq);
    } else {
      const SeqBounds bk = seq_bounds(p.cu_k, seq, p.total_k);
      c.ks = bk.start;
      c.lk = bk.len;
    }
    const KeyRange kr = decode_keys(p, c.lk);
    c.kbeg = kr.kbeg;
    c.kend = kr.kend;
    c.steps = seq_steps(lq, kr);
  }
  const int units = seg_units(c.steps, band_start(p, c.kbeg, c.kend, c.lk, c.steps));
  const int incl = wave_incl_scan(units, lane);
  c.excl = excl0 + incl - units;
  c.total_incl = excl0 + __builtin_amdgcn_readlane(incl, 63);
  return c;
}

// Where a step lives: wave-uniform description of it and its segment.
struct Cursor {
  int seq, kvh, step, steps;  // step within the segment, steps of the segment
  int nb, units;              // steps before the band, units of the segment
  int seg;                    // seq * kv_heads + kvh
  int seg_u0;                 // global unit of the segment's first step
  int qs, ks, kbeg, kend, lk;  // keys [kbeg, kend) visible; steps from kbeg & ~31
  int slot;                   // Q slot of the segment (0 / 1)
  bool first;                 // first step of the segment in this wave
};

// Unit (from the segment's start) where step s of the cursor's segment starts.
__device__ __forceinline__ int step_unit(const Cursor& cu, int s) {
  return s < cu.nb ? kUnits * s : kUnits * cu.nb + kBandUnits * (s - cu.nb);
}
// First step of the segment that starts at unit u or later (steps if none).
__device__ __forceinline__ int unit_step(const Cursor& cu, int u) {
  const int ub = kUnits * cu.nb;
  const int s = u <= ub ? (u + kUnits - 1) / kUnits : cu.nb + (u - ub + kBandUnits - 1) / kBandUnits;
  return min(s, cu.steps);
}

// First key of the cursor's step (a multiple of 32).
__device__ __forceinline__ int step_key0(const Cursor& cu) {
  return (cu.kbeg & ~(kStep - 1)) + cu.step * kStep;
}

template <int D, typename Tag, int G, bool kPaged, int Eb, bool kPair>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(kPair ? IFA4_DECODE_WPE_PAIR : IFA4_DECODE_WPE, 8))) void decode_stream_kernel(DecodeParams p) {
  using E = Elem<Tag>;
  using S = DecodeShape<D, Eb>;
  static_assert(!kPair || (Eb == 1 && D == 128 && G >= 2 && G <= 8), "pair mode: fp8, d 128");
  constexpr int kRowE = kPair ? 2 * D : D;  // elements of the K / V row a wave loads
  using L = DecodeShape<kRowE, Eb>;         // load layout

  // 16-bit tiles (K padded rows, V swizzled), or in pair mode the fp8 tiles
  // (K: 16 rows, V: kStep rows, kPairPitch bytes each)
  __shared__ __align__(16) uint16_t k_lds[kPair ? 16 * kPairPitch / 2 : kStep * S::kPitch];
  __shared__ __align__(16) uint16_t v_lds[kPair ? kStep * kPairPitch / 2 : kStep * D];
  using Q = DecodeQ<D, G>;
  constexpr int kNbuf = kPair ? IFA4_DECODE_NBUF_PAIR : Eb == 1 ? IFA4_DECODE_NBUF_FP8 : 2;
  // Loads of the next step in flight while a step computes (pair mode).  The
  // other formats issue them only while the wave's range lasts; the compiler
  // then merges the two paths' counts and its wait before a step's LDS writes
  // also covers the next step's loads, so each wave computes with no loads in
  // flight -- measured faster for them at their wave counts.
  constexpr bool kOverlap = kPair && IFA4_DECODE_PAIR_OVERLAP;
  static_assert(kNbuf >= 2 && kNbuf <= 3, "two or three step buffers");
  // One Q slot per step buffer: the segments of the steps in flight hold
  // distinct slots, so a slot is rewritten only after its segment's Q was read.
  __shared__ __align__(1024) uint16_t q_lds[kNbuf][Q::kElems];

  const int w = blockIdx.x;
  const int W = p.n_waves;
  const int lane = threadIdx.x;
  const int r = lane / L::kLpr;  // row layout
  const int c = lane % L::kLpr;
  const int n = lane & 15;       // S^T layout
  const int g = lane >> 4;
  const int hkv = p.kv_heads;
  const int g_act = p.group;

  // ---- total units T (every wave derives the same), this wave's range ----------
  // A wave computes the steps that start inside its range of units.
  SeqChunk ch = load_chunk<kPaged>(p, 0, 0, lane);
  int total = ch.total_incl;
  for (int b = 64; b < p.batch; b += 64) total = load_chunk<kPaged>(p, b, total, lane).total_incl;
  const int T = hkv * total;
  if (T == 0) return;
  const int P = (T + W - 1) / W;
  const int g0 = w * P;
  const int g1 = min(g0 + P, T);
  if (g0 >= g1) return;
  if (p.batch > 64) ch = load_chunk<kPaged>(p, 0, 0, lane);

  // Cursor of the first step that starts at global unit gu or later (gu only
  // moves forward; the chunk follows it).  Returns steps == 0 if there is none
  // (gu past the last step start; the bound keeps the search finite whatever
  // cu_seqlens holds).
  auto locate = [&](int gu) -> Cursor {
    while (true) {
      const int nb_l = band_start(p, ch.kbeg, ch.kend, ch.lk, ch.steps);
      const int units_l = seg_units(ch.steps, nb_l);
      const bool hit = units_l > 0 && hkv * (ch.excl + units_l) > gu;
      const uint64_t m = __builtin_amdgcn_ballot_w64(hit);
      if (m != 0) {
        const int L = __builtin_ctzll(m);
        Cursor cu;
        cu.seq = ch.base + L;
        cu.steps = __builtin_amdgcn_readlane(ch.steps, L);
        cu.nb = __builtin_amdgcn_readlane(nb_l, L);
        cu.units = __builtin_amdgcn_readlane(units_l, L);
        const int excl = __builtin_amdgcn_readlane(ch.excl, L);
        const int local = gu - hkv * excl;
        cu.kvh = local / cu.units;
        cu.seg = cu.seq * hkv + cu.kvh;
        cu.seg_u0 = hkv * excl + cu.kvh * cu.units;
        cu.step = unit_step(cu, local - cu.kvh * cu.units);
        if (cu.step == cu.steps) {  // no step of this segment starts at gu or later
          gu = cu.seg_u0 + cu.units;
          continue;
        }
        cu.qs = __builtin_amdgcn_readlane(ch.qs, L);
        cu.ks = __builtin_amdgcn_readlane(ch.ks, L);
        cu.kbeg = __builtin_amdgcn_readlane(ch.kbeg, L);
        cu.kend = __builtin_amdgcn_readlane(ch.kend, L);
        cu.lk = __builtin_amdgcn_readlane(ch.lk, L);
        cu.slot = 0;
        cu.first = false;
        return cu;
      }
      if (ch.base + 64 >= p.batch) {
        Cursor none{};
        none.steps = 0;
        return none;
      }
      ch = load_chunk<kPaged>(p, ch.base + 64, ch.total_incl, lane);
    }
  };

  // ---- loads of one step, Q of a segment ---------------------------------------------
  const uint32_t k_row = (uint32_t)p.k_st * Eb, v_row = (uint32_t)p.v_st * Eb;
  const char* const k_bytes0 = static_cast<const char*>(p.k);
  const char* const v_bytes0 = static_cast<const char*>(p.v);
  // Paged cache: lane L holds table entry tw_base + L of sequence tw_seq (a
  // window of 64 blocks; a 32-key step never straddles two windows).  A step
  // reads its row groups (8 keys, or the rows of one wave load when larger)
  // through one buffer resource per block, so rows past the sequence end and
  // entries outside the pool read as zero.
  int tw = -1, tw_seq = -1, tw_base = 0;
  const int bmask = (1 << p.block_shift) - 1;
  auto load_paged = [&](u32x4_t* kr, u32x4_t* vr, const Cursor& cu, bool on) {
    const int k0 = step_key0(cu);
    const int blk0 = k0 >> p.block_shift;
    if (on && (cu.seq != tw_seq || blk0 < tw_base || blk0 >= tw_base + 64)) {
      tw_seq = cu.seq;
      tw_base = blk0 & ~63;
      const int nblk = (cu.lk + bmask) >> p.block_shift;
      const int e = tw_base + lane;
      tw = e < nblk ? p.block_table[(int64_t)cu.seq * p.bt_stride + e] : -1;
    }
    const uint32_t k_bytes = (uint32_t)(((int64_t)bmask * p.k_st + kRowE) * Eb);
    const uint32_t v_bytes = (uint32_t)(((int64_t)bmask * p.v_st + kRowE) * Eb);
    constexpr int kGroups = kStep / L::kGroupRows;
    rsrc_t rk[kGroups], rv[kGroups];
#pragma unroll
    for (int grp = 0; grp < kGroups; ++grp) {
      const int ent = __builtin_amdgcn_readlane(
          tw, ((k0 + L::kGroupRows * grp) >> p.block_shift) - tw_base);
      const bool ok = on && (unsigned)ent < (unsigned)p.num_blocks;
      const int64_t eb = ok ? (int64_t)ent : 0;
      rk[grp] = make_rsrc_uniform(k_bytes0 + (eb * p.k_sblk + (int64_t)cu.kvh * p.k_sh) * Eb,
                                  ok ? k_bytes : 0u);
      rv[grp] = make_rsrc_uniform(v_bytes0 + (eb * p.v_sblk + (int64_t)cu.kvh * p.v_sh) * Eb,
                                  ok ? v_bytes : 0u);
    }
#pragma unroll
    for (int i = 0; i < L::kLoads; ++i) {
      const int key = k0 + L::kRpi * i + r;
      const uint32_t row = (uint32_t)(key & bmask);
      const bool valid = key < cu.kend;
      const int grp = (L::kRpi * i) / L::kGroupRows;
      kr[i] = kv_load(rk[grp], valid ? row * k_row + 16 * c : kOutOfRange);
      vr[i] = kv_load(rv[grp], valid ? row * v_row + 16 * c : kOutOfRange);
    }
  };
  // on = false: the same loads through empty resources, which read zeros and
  // touch no memory
  auto load = [&](u32x4_t* kr, u32x4_t* vr, const Cursor& cu, bool on) {
    if constexpr (kPaged) {
      load_paged(kr, vr, cu, on);
    } else {
      const char* kbase = k_bytes0 + ((int64_t)cu.ks * p.k_st + (int64_t)cu.kvh * p.k_sh) * Eb;
      const char* vbase = v_bytes0 + ((int64_t)cu.ks * p.v_st + (int64_t)cu.kvh * p.v_sh) * Eb;
      const rsrc_t rk = make_rsrc_uniform(
          kbase, on ? (uint32_t)(((int64_t)(cu.kend - 1) * p.k_st + kRowE) * Eb) : 0u);
      const rsrc_t rv = make_rsrc_uniform(
          vbase, on ? (uint32_t)(((int64_t)(cu.kend - 1) * p.v_st + kRowE) * Eb) : 0u);
      const int k0 = step_key0(cu);
#pragma unroll
      for (int i = 0; i < L::kLoads; ++i) {
        const uint32_t row = (uint32_t)(k0 + L::kRpi * i + r);
        kr[i] = kv_load(rk, row * k_row + 16 * c);
        vr[i] = kv_load(rv, row * v_row + 16 * c);
      }
    }
  };
  // Q rows of the segment's heads -> q_lds[slot] as [head][D]; heads past the
  // group read as zero.  Issued before the loads of the segment's first step, so those
  // loads completing (which the compute waits for) implies this DMA has landed.
  auto load_q = [&](const Cursor& cu) {
    const uint16_t* qbase = static_cast<const uint16_t*>(p.q) + (int64_t)cu.qs * p.q_st +
                            (int64_t)cu.kvh * g_act * p.q_sh;
    const rsrc_t rq =
        make_rsrc_uniform(qbase, (uint32_t)(((int64_t)(g_act - 1) * p.q_sh + D) * 2));
#pragma unroll
    for (int u = 0; u < Q::kDma; ++u) {
      const int e = u * 512 + 8 * lane;  // element of the [G][D] slot
      const int h = e / D, d = e % D;
      const uint32_t off = h < g_act ? (uint32_t)(h * p.q_sh + d) * 2 : kOutOfRange;
      dma_16(rq, off, q_lds[cu.slot] + u * 512);
    }
  };

  const float c2 = p.scale_log2;
  float m_run = -INFINITY;  // per head n (S^T lanes), identical over g
  float l_run = 0.f;        // partial sum over this lane's keys
  // O^T = V^T P^T in the 16x16 C layout: lane (n, g) holds d = 16 db + 4 g + j
  // of head n (columns n >= group are padding and never stored).
  f32x4_t o[S::kDBlocks];
  u32x4_t qf[S::kKSteps];

  const int rel_esz = p.rel_dtype == 2 ? 4 : 2;  // bytes per bias element
  // (o * inv, lse2) of head n -> workspace slot; the lane's head and d offset
  // are derived again from the lane id (v_mbcnt), so that no register carries
  // the slot addresses across the stream loop
  auto put_partial = [&](int slot, float inv, float lse2) {
    int ln = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    asm volatile("" : "+v"(ln));  // computed here, not hoisted out of the loop
    const int hn = ln & 15, hg = ln >> 4;
    if (hn < g_act) {
      float* dst = p.ws_o + ((int64_t)slot * g_act + hn) * D + 4 * hg;
#pragma unroll
      for (int db = 0; db < S::kDBlocks; ++db)
        *reinterpret_cast<f32x4_t*>(dst + 16 * db) = o[db] * inv;
      if (hg == 0) p.ws_lse[(int64_t)slot * g_act + hn] = lse2;
    }
  };
  struct StepBias {
    u32x4_t bw[kStep / 16];
    uint32_t rel_skew;
    bool bias, run_form;
  };
  // The bias loads of a step (see below); issued before the step's K/V wait.
  auto bias_loads = [&](const Cursor& cu) -> StepBias {
    StepBias sb;
    const int k0 = step_key0(cu);
    const int delta = p.bottom_right ? cu.lk - 1 : 1 - cu.lk;  // dist = delta - key (i = 0)
    // some key of the step lies in the bias band 0 <= dist < rel_extent (the
    // step's distances run from delta - k0 down to delta - k0 - 31)
    const bool bias = p.rel_extent > 0 && delta - k0 >= 0 && delta - k0 - (kStep - 1) < p.rel_extent;
    sb.bias = bias;
    // Per-token bias of the step.  Lane (n, g) holds keys k0 + pair_key(blk, g)
    // + j of head n: per blk a run of four keys whose distances dt - j (dt =
    // delta - k0 - pair_key(blk, g)) are four consecutive elements of the
    // head's bias row, lowest address at j = 3.  One 16-byte load per run (fp32: exactly the
    // run; 16-bit: the dword-aligned 16 bytes around it, realigned with
    // v_alignbit), issued before the K/V wait below so that it lands with the
    // K/V rows, through one buffer resource over the sequence's bias rows (all
    // heads; base aligned down to 4 bytes, `rel_skew` the bytes it moved):
    // addresses outside it read as zero, and no 16-byte window straddles its
    // ends (such a step loads one dword per element instead).  Elements outside
    // the band are zeroed after the load (only on the steps at its edges).
    u32x4_t* bw = sb.bw;
    uint32_t rel_skew = 0;
    bool run_form = false;
    if (bias) {
      const uint64_t row = reinterpret_cast<uint64_t>(p.rel) +
                           (uint64_t)((int64_t)cu.qs * p.rel_st * rel_esz);
      rel_skew = (uint32_t)(row & 3u);
      const uint32_t bytes =
          (rel_skew +
           (uint32_t)(((int64_t)(p.n_heads - 1) * p.rel_sh + p.rel_extent) * rel_esz) + 3u) &
          ~3u;
      const rsrc_t rr = make_rsrc_uniform(reinterpret_cast<const void*>(row - rel_skew), bytes);
      // element offsets stay below 2^30 (validation bounds the heads' span)
      const int hoff = (cu.kvh * g_act + n) * (int)p.rel_sh;
      // 16-byte loads on a step whose distances are all >= 3 (so no run starts
      // before the rows) and whose windows all end inside the resource
      // (block 0 holds the lane's highest addresses)
      const int dt0 = delta - k0 - pair_key<kPair>(0, g);
      const uint32_t b30 = rel_skew + (uint32_t)(hoff + dt0 - 3) * (uint32_t)rel_esz;
      const bool straddle = n < g_act && dt0 - 3 < p.rel_extent && (b30 & ~3u) + 16u > bytes;
      run_form = delta - k0 - (kStep - 1) >= 3 && !wave_any(straddle);
#pragma unroll
      for (int blk = 0; blk < kStep / 16; ++blk) {
        const int dt = delta - k0 - pair_key<kPair>(blk, g);
        const int e3 = hoff + dt - 3;  // element of j = 3
        const uint32_t b3 = rel_skew + (uint32_t)e3 * (uint32_t)rel_esz;
        const bool any = n < g_act && dt >= 0 && dt - 3 < p.rel_extent;
        if (!run_form) {
          // the step holding distances 0..2 (a run of head 0 could start before
          // the rows) or a window past the rows' end: one dword per element
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bool ok = n < g_act && dt - j >= 0 && dt - j < p.rel_extent;
            const uint32_t off = rel_skew + (uint32_t)(hoff + dt - j) * (uint32_t)rel_esz;
            bw[blk][j] = buf_load_4(rr, ok ? (off & ~3u) : kOutOfRange);
          }
        } else {
          bw[blk] = buf_load_16(rr, any ? (b3 & ~3u) : kOutOfRange);
        }
      }
    }
    sb.rel_skew = rel_skew;
    sb.run_form = run_form;
    return sb;
  };
  auto step = [&](const u32x4_t* kr, const u32x4_t* vr, const Cursor& cu, const StepBias& sb,
                  bool last) {
    const int k0 = step_key0(cu);
    const int c1 = cu.kend;
    const int delta = p.bottom_right ? cu.lk - 1 : 1 - cu.lk;  // dist = delta - key (i = 0)
    const bool tail = k0 + kStep > c1 || k0 < cu.kbeg;
    const bool bias = sb.bias;
    const u32x4_t* bw = sb.bw;
    const uint32_t rel_skew = sb.rel_skew;
    const bool run_form = sb.run_form;
    if (cu.first) {
      m_run = -INFINITY;
      l_run = 0.f;
#pragma unroll
      for (int db = 0; db < S::kDBlocks; ++db) o[db] = f32x4_t{};
      if (cu.step == 0 && lane == 0) {
        // this wave holds the segment's first step: record the covering waves
        p.ws_meta[2 * cu.seg] = w;
        p.ws_meta[2 * cu.seg + 1] = (cu.seg_u0 + step_unit(cu, cu.steps - 1)) / P;
      }
    }
    // K rows -> LDS (row-major, padded rows: conflict-free A-operand reads of
    // QK), V rows -> LDS (swizzled: conflict-free transposing reads of PV).
    // fp8 converts to the MFMA type on the way (exact); the K scale is folded
    // into the logit scale, the V scale into the partial's normalisation.
    // Waiting for these loads also completes the (earlier) Q DMA of the segment.
    // Pair mode stores the fp8 bytes as they are: V rows, and K rows of key
    // block 0 (block 1 follows once QK has read block 0).
    auto put_k_pair = [&](int blk) {
#pragma unroll
      for (int t = 0; t < L::kLoads / 2; ++t)
        *reinterpret_cast<u32x4_t*>(reinterpret_cast<uint8_t*>(k_lds) +
                                    (4 * t + r) * kPairPitch + 16 * c) = kr[2 * t + blk];
    };
    if constexpr (kPair) put_k_pair(0);
#pragma unroll
    for (int i = 0; i < L::kLoads; ++i) {
      const int row = L::kRpi * i + r;
      uint16_t* kdst = k_lds + row * S::kPitch + S::kEpl * c;
      if constexpr (kPair) {
        *reinterpret_cast<u32x4_t*>(reinterpret_cast<uint8_t*>(v_lds) + row * kPairPitch +
                                    16 * c) = vr[i];
      } else if constexpr (Eb == 2) {
        *reinterpret_cast<u32x4_t*>(kdst) = kr[i];
        *reinterpret_cast<u32x4_t*>(v_lds + row * D + 8 * (c ^ vswz<D>(row))) = vr[i];
      } else {
#pragma unroll
        for (int hlf = 0; hlf < 2; ++hlf) {
#if IFA4_FP8_CVT2
          // one conversion per pair, straight to the 16-bit type
          const uint32_t w0 = kr[i][2 * hlf], w1 = kr[i][2 * hlf + 1];
          *reinterpret_cast<u32x4_t*>(kdst + 8 * hlf) =
              u32x4_t{E::template fp8x2<false>(w0), E::template fp8x2<true>(w0),
                      E::template fp8x2<false>(w1), E::template fp8x2<true>(w1)};
#else
          float f[8];
          fp8x8_to_f32(kr[i][2 * hlf], kr[i][2 * hlf + 1], f);
          *reinterpret_cast<u32x4_t*>(kdst + 8 * hlf) =
              u32x4_t{E::pack2(f[0], f[1]), E::pack2(f[2], f[3]), E::pack2(f[4], f[5]),
                      E::pack2(f[6], f[7])};
#endif
          const uint32_t x0 = vr[i][2 * hlf], x1 = vr[i][2 * hlf + 1];
          *reinterpret_cast<u32x4_t*>(v_lds + row * D + 8 * ((2 * c + hlf) ^ vswz<D>(row))) =
              u32x4_t{E::template fp8x2<false>(x0), E::template fp8x2<true>(x0),
                      E::template fp8x2<false>(x1), E::template fp8x2<true>(x1)};
        }
      }
    }
    wave_lds_sync();
    if (cu.first) {
      // Q (B operand): column n = head n of the kv head, k-slots = d 32*kk + 8*g .. +7.
#pragma unroll
      for (int kk = 0; kk < S::kKSteps; ++kk)
        qf[kk] = n < g_act
                     ? *reinterpret_cast<const u32x4_t*>(q_lds[cu.slot] + n * D + 32 * kk + 8 * g)
                     : u32x4_t{0, 0, 0, 0};
    }

    // S^T = K Q^T: lane (n, g) gets keys pair_key(blk, g) + j of head n
    f32x4_t acc[kStep / 16];
    // pair mode: column n holds a query head of the pair's second kv head
    const bool hi_head = kPair && n >= (g_act >> 1);
#pragma unroll
    for (int blk = 0; blk < kStep / 16; ++blk) {
      acc[blk] = f32x4_t{};
      if constexpr (kPair) {
        if (blk == 1) {  // block 0 has been read: K rows of block 1 replace it
          wave_lds_sync();
          put_k_pair(1);
          wave_lds_sync();
        }
        // A = 8 fp8 bytes of tile row n (key pair_key), k-slots 8g..8g+7 of d
        // block kk of kv head h (byte 128 h + 32 kk + 8 g), converted
        const uint8_t* krow = reinterpret_cast<const uint8_t*>(k_lds) + n * kPairPitch + 8 * g;
        f32x4_t acc1{};
#pragma unroll
        for (int kk = 0; kk < S::kKSteps; ++kk) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const u32x4_t a = fp8x8_operand<E>(
                *reinterpret_cast<const u32x2_t*>(krow + 128 * h + 32 * kk));
            if (h == 0)
              acc[blk] = E::mfma16(a, qf[kk], acc[blk]);
            else
              acc1 = E::mfma16(a, qf[kk], acc1);
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[blk][j] = hi_head ? acc1[j] : acc[blk][j];
      } else {
        const uint16_t* krow = k_lds + (16 * blk + n) * S::kPitch + 8 * g;
#pragma unroll
        for (int kk = 0; kk < S::kKSteps; ++kk)
          acc[blk] =
              E::mfma16(*reinterpret_cast<const u32x4_t*>(krow + 32 * kk), qf[kk], acc[blk]);
      }
    }

    float mx = -INFINITY;
#pragma unroll
    for (int blk = 0; blk < kStep / 16; ++blk) {
      // raw bias of the lane's 4 keys of this block (zero off the band)
      float bv[4] = {0.f, 0.f, 0.f, 0.f};
      if (bias) {
        const int dt = delta - k0 - pair_key<kPair>(blk, g);
        const int hoff = (cu.kvh * g_act + n) * (int)p.rel_sh;
        if (!run_form) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            // the element's half of its dword (16-bit types): by its byte offset
            const uint32_t off = rel_skew + (uint32_t)(hoff + dt - j) * (uint32_t)rel_esz;
            const uint32_t hv = (bw[blk][j] >> (8 * (off & 2u))) & 0xffffu;
            bv[j] = rel_esz == 4      ? __uint_as_float(bw[blk][j])
                    : p.rel_dtype == 0 ? __uint_as_float(hv << 16)
                                       : (float)__builtin_bit_cast(_Float16, (uint16_t)hv);
          }
        } else if (rel_esz == 4) {
#pragma unroll
          for (int j = 0; j < 4; ++j) bv[j] = __uint_as_float(bw[blk][3 - j]);
        } else {
          // 16-bit: the run starts 0 or 2 bytes into bw[blk][0]
          const uint32_t sh = 8u * ((rel_skew + 2u * (uint32_t)(hoff + dt - 3)) & 2u);
          const uint32_t p0 = __builtin_amdgcn_alignbit(bw[blk][1], bw[blk][0], sh);  // j = 3, 2
          const uint32_t p1 = __builtin_amdgcn_alignbit(bw[blk][2], bw[blk][1], sh);  // j = 1, 0
          const uint32_t h[4] = {p1 >> 16, p1 & 0xffffu, p0 >> 16, p0 & 0xffffu};  // j = 0..3
#pragma unroll
          for (int j = 0; j < 4; ++j)
            bv[j] = p.rel_dtype == 0 ? __uint_as_float(h[j] << 16)
                                     : (float)__builtin_bit_cast(_Float16, (uint16_t)h[j]);
        }
        if (!wave_all(n >= g_act || (dt - 3 >= 0 && dt < p.rel_extent))) {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            bv[j] = (uint32_t)(dt - j) < (uint32_t)p.rel_extent ? bv[j] : 0.f;
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float x = acc[blk][j] * c2;
        if (tail || bias) {
          const int key = k0 + pair_key<kPair>(blk, g) + j;
          if (bias) x = fmaf(bv[j], kLog2e, x);
          if (key >= c1 || key < cu.kbeg) x = -INFINITY;
        }
        acc[blk][j] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = max_xor16(mx);
    mx = max_xor32(mx);

    const float m_cand = fmaxf(m_run, mx);
    const bool grow = m_cand > m_run + kRescaleThreshold;
    const bool any_grow = wave_any(grow);
    float alpha = 1.f;
    if (any_grow) {
      const float m_upd = grow ? m_cand : m_run;
      alpha = grow ? fast_exp2(m_run - m_upd) : 1.f;
      l_run *= alpha;
      m_run = m_upd;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    // P^T as the B operand of O^T += V^T P^T: column n = head, k-slots 0..3 =
    // keys 4g..4g+3, 4..7 = keys 16+4g..16+4g+3 (where the S^T layout left them;
    // pair mode: keys 8g..8g+7)
    float pv[kStep / 16][4];
#pragma unroll
    for (int blk = 0; blk < kStep / 16; ++blk) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pv[blk][j] = fast_exp2(acc[blk][j] - m_use);
        l_run += pv[blk][j];
      }
    }
    const u32x4_t pb = {E::pack2(pv[0][0], pv[0][1]), E::pack2(pv[0][2], pv[0][3]),
                        E::pack2(pv[1][0], pv[1][1]), E::pack2(pv[1][2], pv[1][3])};
    if (any_grow) {
      // lane (n, g) holds rows of head n, whose factor it computed itself
#pragma unroll
      for (int db = 0; db < S::kDBlocks; ++db) o[db] *= alpha;
    }

    // O^T += V^T P^T on v_mfma_f32_16x16x32: A = V^T (row d, the same key
    // k-slots as P), two transposing reads: 16-lane group g, lane i points at
    // V[k0 + i/4][16 db + 4 (i % 4)] and receives V[k0 .. k0+3][16 db + i].
    // Pair mode: one 8-bit transposing read per (kv head, d block): lane i
    // points at bytes 8 (i & 1) .. +7 of the block in key row 8g + i/2 and
    // receives its d = 16 db + i at keys 8g..8g+7 (the P k-slots); each head's
    // product sees P with the other head's columns zeroed.
    if constexpr (kPair) {
      const u32x4_t pz{0u, 0u, 0u, 0u};
      const u32x4_t pbh[2] = {hi_head ? pz : pb, hi_head ? pb : pz};
      const uint8_t* vsrc =
          reinterpret_cast<const uint8_t*>(v_lds) + (8 * g + (n >> 1)) * kPairPitch + 8 * (n & 1);
#pragma unroll
      for (int db = 0; db < S::kDBlocks; ++db) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint8_t* src = vsrc + 128 * h + 16 * db;
          typedef int i32x2_t __attribute__((ext_vector_type(2)));
          const u32x2_t w = __builtin_bit_cast(
              u32x2_t, __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                           (__attribute__((address_space(3))) i32x2_t*)src));
          o[db] = E::mfma16(fp8x8_operand<E>(w), pbh[h], o[db]);
        }
      }
    }
#pragma unroll
    for (int db = 0; db < (kPair ? 0 : S::kDBlocks); ++db) {
      u32x2_t part[2];
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        const int row = 16 * blk + 4 * g + (n >> 2);
        const int chunk = 2 * db + ((n & 3) >> 1);
        const uint16_t* src = v_lds + row * D + 8 * (chunk ^ vswz<D>(row)) + 4 * (n & 1);
        part[blk] = __builtin_bit_cast(
            u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                         (__attribute__((address_space(3))) s16x4_t*)src));
      }
      o[db] = E::mfma16(u32x4_t{part[0][0], part[0][1], part[1][0], part[1][1]}, pb, o[db]);
    }
    wave_lds_sync();  // k_lds / v_lds are rewritten by the next step

    if (!last) return;
    // ---- partial of (segment, wave): normalise, store ------------------------------
    const float l_tot = add_xor32(add_xor16(l_run));  // per head n, all g
    const float inv = l_tot > 0.f ? p.v_scale / l_tot : 0.f;  // V scale (1 for 16-bit V)
    const float lse2 = l_tot > 0.f ? m_run + __log2f(l_tot) : -INFINITY;
    put_partial(cu.seg + w, inv, lse2);
  };

  // ---- stream: loads of the next kNbuf - 1 steps in flight while a step is computed --
  // Buffer j of the ring holds step gs + ((j - j0) mod kNbuf); live[j] says it
  // holds a step of this wave's range.  Cursors and buffers are indexed by
  // compile-time constants only (the inner loop is unrolled).
  Cursor cur[kNbuf];
  bool live[kNbuf];
  u32x4_t kbuf[kNbuf][L::kLoads], vbuf[kNbuf][L::kLoads];
  cur[0] = locate(g0);
  if (cur[0].steps == 0) return;
  if (cur[0].seg_u0 + step_unit(cur[0], cur[0].step) >= g1) {
    // No step starts in this wave's range.  If the range lies inside the
    // segment (between two of its steps' starts), the segment's partials run
    // over this wave's slot too: an empty one (nothing seen) goes there.
    if (g0 >= cur[0].seg_u0) {
#pragma unroll
      for (int db = 0; db < S::kDBlocks; ++db) o[db] = f32x4_t{};
      put_partial(cur[0].seg + w, 0.f, -INFINITY);
    }
    return;
  }
  cur[0].first = true;
  load_q(cur[0]);
  load(kbuf[0], vbuf[0], cur[0], true);
  live[0] = true;
  // Next cursor after `cu`, with its Q slot (a new segment takes the next slot,
  // whose earlier segment's Q was read into registers kNbuf - 1 steps before).
  auto next = [&](const Cursor& cu) -> Cursor {
    if (cu.step + 1 < cu.steps) {
      Cursor nx = cu;
      nx.step = cu.step + 1;
      nx.first = false;
      return nx;
    }
    Cursor nx = locate(cu.seg_u0 + cu.units);
    nx.slot = cu.slot + 1 == kNbuf ? 0 : cu.slot + 1;
    nx.first = true;
    return nx;
  };
  // issue the loads of the step after the one in buffer jp into buffer j
  auto issue = [&](int j, int jp) {
    live[j] = live[jp];
    if (live[j]) {
      cur[j] = next(cur[jp]);
      live[j] = cur[j].steps > 0 && cur[j].seg_u0 + step_unit(cur[j], cur[j].step) < g1;
    }
    if constexpr (kOverlap) {
      // every path issues the step's loads (past the range through empty
      // resources), so the wait for a step's rows leaves the next step's in flight
      if (live[j] && cur[j].first) load_q(cur[j]);
      load(kbuf[j], vbuf[j], cur[j], live[j]);
    } else if (live[j]) {
      if (cur[j].first) load_q(cur[j]);
      load(kbuf[j], vbuf[j], cur[j], true);
    }
  };
#pragma unroll
  for (int j = 1; j < kNbuf - 1; ++j) issue(j, j - 1);
  bool more = true;
  while (more) {
#pragma unroll
    for (int j = 0; j < kNbuf; ++j) {
      if (more) {
        const int jn = (j + kNbuf - 1) % kNbuf;  // buffer of the step kNbuf - 1 ahead
        const int jp = (j + kNbuf - 2) % kNbuf;  // buffer of the step before it
        StepBias sb;
        // with loads in flight across steps, the step's bias loads go out
        // before the next step's K/V loads, so that waiting for them leaves those
        // in flight (loads complete in order)
        if constexpr (kOverlap) sb = bias_loads(cur[j]);
        issue(jn, jp);
        if constexpr (!kOverlap) sb = bias_loads(cur[j]);
        const int j1 = (j + 1) % kNbuf;          // buffer of the next step
        step(kbuf[j], vbuf[j], cur[j], sb, !live[j1] || cur[j1].first);
        more = live[j1];
      }
    }
  }
}

constexpr int kCombineWaves = 8;

// SPLIT workgroups per (head, sequence), workgroup z over the 16-byte chunks
// [z, z + 1) * D / (4 SPLIT) of the row.  Two dependent memory rounds: the
// sequence bounds and the segment's wave range (independent loads), then the
// parts themselves.  Thread (g, c) holds chunk c and merges parts g, g +
// kGroups, ... online (running max, rescaled sums, four parts' loads in
// flight); the kGroups results of a chunk meet in LDS.  With 8 waves that is
// 16 groups per split at D = 128 (32 at D = 64), so a segment of up to 64
// (128) parts per split merges in one round of loads.  The host takes more
// splits for segments of many parts (a few long caches spread over many
// waves: one sequence of 128K keys over 1024 waves has ~512 parts per cache).
// Every split merges the same parts in the same order, so the running max and
// sum, and with them the normalisation, are the same bits in all of them; split
// 0 writes the LSE.
template <int D, typename Tag, int SPLIT>
__global__ __launch_bounds__(64 * kCombineWaves) void decode_combine_kernel(DecodeParams p) {
  using E = Elem<Tag>;
  constexpr int kThreads = 64 * kCombineWaves;
  constexpr int kChunks = D / 4 / SPLIT;        // 16-byte chunks of this split
  constexpr int kGroups = kThreads / kChunks;   // part groups
  __shared__ f32x4_t part_o[kGroups][kChunks];
  __shared__ float part_m[kGroups];
  __shared__ float part_l[kGroups];
  const int head = blockIdx.x;
  const int seq = blockIdx.y;
  const int split = blockIdx.z;
  const int tid = threadIdx.x;
  const int c = tid % kChunks, grp = tid / kChunks;
  const int cc = split * kChunks + c;  // chunk of the row
  const int ga = p.group;
  const int kvh = head / ga, h = head % ga;
  const int seg = seq * p.kv_heads + kvh;
  const SeqBounds bq = seq_bounds(p.cu_q, seq, p.total_q);
  const int qs = bq.start, lq = bq.len;
  const int lk = p.block_table != nullptr ? paged_len(p, seq) : seq_bounds(p.cu_k, seq, p.total_k).len;
  const int meta_first = p.ws_meta[2 * seg];  // read before knowing it is needed
  const int meta_last = p.ws_meta[2 * seg + 1];
  if (lq != 1) {
    // Not one query token (cu_seqlens_q is not arange): the pass above streamed
    // nothing for this sequence; its query rows, if any, get out = 0, lse = -inf.
    for (int row = grp; row < lq; row += kGroups) {
      uint16_t* dst = static_cast<uint16_t*>(p.out) + (int64_t)(qs + row) * p.o_st +
                      (int64_t)head * p.o_sh + 4 * cc;
      *reinterpret_cast<u32x2_t*>(dst) = u32x2_t{0u, 0u};
      if (p.lse != nullptr && cc == 0) p.lse[(int64_t)head * p.lse_sh + qs + row] = -INFINITY;
    }
    return;
  }
  int w_first = 0, parts = 0;
  if (seq_steps(lq, decode_keys(p, lk)) > 0 && p.n_waves > 0) {
    // clamped so that a slot index can never leave the workspace
    w_first = min(max(meta_first, 0), p.n_waves - 1);
    parts = min(max(meta_last, w_first), p.n_waves - 1) - w_first + 1;
  }
  // part i of the segment lives in slot seg + w_first + i
  const float* lse_s = p.ws_lse + (int64_t)(seg + w_first) * ga + h;
  const float* o_s = p.ws_o + ((int64_t)(seg + w_first) * ga + h) * D + 4 * cc;
  const int64_t o_stride = (int64_t)ga * D;

  float m = -INFINITY, l = 0.f;
  f32x4_t acc{};
#pragma unroll 4
  for (int s = grp; s < parts; s += kGroups) {
    const float ls = lse_s[(int64_t)s * ga];
    const f32x4_t os = *reinterpret_cast<const f32x4_t*>(o_s + s * o_stride);
    const float mn = fmaxf(m, ls);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float a_old = fast_exp2(m - mu), a_new = fast_exp2(ls - mu);
    l = l * a_old + a_new;
    acc = acc * a_old + a_new * os;
    m = mn;
  }
  part_o[grp][c] = acc;
  if (c == 0) {  // every thread of a group has merged the same parts: one m, l
    part_m[grp] = m;
    part_l[grp] = l;
  }
  __syncthreads();
  if (grp != 0) return;
  float mt = part_m[0];
#pragma unroll
  for (int g = 1; g < kGroups; ++g) mt = fmaxf(mt, part_m[g]);
  const float mu = mt == -INFINITY ? 0.f : mt;
  float lt = 0.f;
  f32x4_t out{};
#pragma unroll
  for (int g = 0; g < kGroups; ++g) {
    const float a = fast_exp2(part_m[g] - mu);
    lt += a * part_l[g];
    out += a * part_o[g][c];
  }
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  uint16_t* dst = static_cast<uint16_t*>(p.out) + (int64_t)qs * p.o_st + (int64_t)head * p.o_sh +
                  4 * cc;
  *reinterpret_cast<u32x2_t*>(dst) =
      u32x2_t{E::pack2(out[0] * inv, out[1] * inv), E::pack2(out[2] * inv, out[3] * inv)};
  if (p.lse != nullptr && cc == 0) {
    p.lse[(int64_t)head * p.lse_sh + qs] = lt > 0.f ? (mu + __log2f(lt)) * kLn2 : -INFINITY;
  }
}

template <int D, typename Tag, int G>
hipError_t launch_decode_g(const DecodeParams& p, hipStream_t stream) {
  if (p.n_waves > 0) {
    const dim3 grid(p.n_waves), block(64);
    if (p.kv_pair) {
      // the host pairs kv heads only for fp8 caches of d 128 whose pairs hold
      // 2..8 query heads
      if constexpr (D == 128 && G >= 2 && G <= 8) {
        if (!p.kv_fp8) return hipErrorInvalidValue;
        if (p.block_table != nullptr)
          hipLaunchKernelGGL((decode_stream_kernel<D, Tag, G, true, 1, true>), grid, block, 0,
                             stream, p);
        else
          hipLaunchKernelGGL((decode_stream_kernel<D, Tag, G, false, 1, true>), grid, block, 0,
                             stream, p);
      } else {
        return hipErrorInvalidValue;
      }
    } else if (p.kv_fp8) {
      if (p.block_table != nullptr)
        hipLaunchKernelGGL((decode_stream_kernel<D, Tag, G, true, 1, false>), grid, block, 0,
                           stream, p);
      else
        hipLaunchKernelGGL((decode_stream_kernel<D, Tag, G, false, 1, false>), grid, block, 0,
                           stream, p);
    } else {
      if (p.block_table != nullptr)
        hipLaunchKernelGGL((decode_stream_kernel<D, Tag, G, true, 2, false>), grid, block, 0,
                           stream, p);
      else
        hipLaunchKernelGGL((decode_stream_kernel<D, Tag, G, false, 2, false>), grid, block, 0,
                           stream, p);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  // Splits of the combine: enough part groups that the parts of a segment
  // (about waves / segments + 1 when the caches are of similar length) merge in
  // one round of four loads per thread, at most 4.
  const int64_t segs = (int64_t)p.batch * p.kv_heads;
  const int64_t parts = segs > 0 ? (int64_t)p.n_waves / segs + 1 : 1;
  constexpr int64_t kRound = 4 * (64 * kCombineWaves) / (D / 4);  // parts per round, 1 split
  const dim3 block(64 * kCombineWaves);
  if (IFA4_COMBINE_SPLIT && parts > 2 * kRound)
    hipLaunchKernelGGL((decode_combine_kernel<D, Tag, 4>), dim3(p.n_heads, p.batch, 4), block, 0,
                       stream, p);
  else if (IFA4_COMBINE_SPLIT && parts > kRound)
    hipLaunchKernelGGL((decode_combine_kernel<D, Tag, 2>), dim3(p.n_heads, p.batch, 2), block, 0,
                       stream, p);
  else
    hipLaunchKernelGGL((decode_combine_kernel<D, Tag, 1>), dim3(p.n_heads, p.batch), block, 0,
                       stream, p);
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
int decode_fp8_max_group() { return kDecodeFp8MaxGroup; }

hipError_t launch_decode(const DecodeParams& p, int head_dim, int qkv_dtype, hipStream_t stream) {
  if (p.batch <= 0) return hipSuccess;
  if (head_dim == 128) {
    return qkv_dtype == 0 ? launch_decode_d<128, Bf16Tag>(p, stream)
                          : launch_decode_d<128, F16Tag>(p, stream);
  }
  return qkv_dtype == 0 ? launch_decode_d<64, Bf16Tag>(p, stream)
                        : launch_decode_d<64, F16Tag>(p, stream);
}

}  // namespace ifa4
