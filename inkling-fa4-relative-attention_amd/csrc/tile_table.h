// gfx950 tile table.  Replaces the per-arch Triton presets of
// src/inkling_fa4/autotune_configs.py:17-50 (seq-length buckets of
// BLOCK_Q/BLOCK_K/num_warps/num_stages for sm86/sm90/sm100).
//
// Prefill: one shape for every sequence length, and a sequence-length (grid)
// dependent split of the KV range (prefill_split_for, below).  The kernel is
// written for 4 waves x 32 query rows (BLOCK_Q 128) and 64-key KV tiles in two
// LDS stages (64 KiB of LDS at head_dim 128, so two workgroups fit in the 160
// KiB of a CU; 236 VGPRs, two waves per SIMD); the shape is a compile-time
// property of the kernel, listed here so the host reports what runs.  Swept on
// causal batch 8, Hq 8 / Hkv 2, d 128 at S 1024 / 2048 / 4096 / 8192
// (profiles/sweep_prefill_shapes_b8.md): BLOCK_K 64 x 4 waves 0.0314 / 0.0771 /
// 0.2646 / 0.9865 ms; 256-row workgroups of 8 waves +13 / +4.5 / +1.4 / +1.5%;
// 32-key tiles +9 / +6 / +6 / +6%; 64 rows per wave at one wave per SIMD
// (PREFILL_NQB 2) +79% at S 4096 (profiles/sweep_prefill_knobs_b8_s4096.md).
// SQ_VALU_MFMA_BUSY_CYCLES is the same for every variant and GRBM_GUI_ACTIVE
// follows the time: the shape sets how much of the MFMA work overlaps the
// softmax, not how much MFMA work there is.
//
// Decode: persistent waves of the stream-K pass (at most one per 32-key step).
#pragma once

#include <stdint.h>

namespace ifa4 {

struct PrefillTileEntry {
  int32_t head_dim;
  int32_t block_q;
  int32_t block_k;
  int32_t waves;
  int32_t stages;
};

constexpr PrefillTileEntry kPrefillTiles[] = {
    {64, 128, 64, 4, 2},
    {128, 128, 64, 4, 2},
};

// Persistent waves of the decode stream pass (at most; never more than the
// steps), from the sweep on the 64-sequence batch (KV 1K-16K, non-causal;
// profiles/sweep_decode_waves_b64.md, before the K/V loads were non-temporal;
// with them, profiles/sweep_decode_nt_b64.md: contiguous 896 waves 0.097 ms,
// 1536 0.103; paged 0.105 either way):
//   contiguous bf16: 896 waves 0.112 ms, 1024 0.112, 768 0.113, 2048 0.116,
//                    512 0.151 (too few bytes in flight);
//   paged (blocks of 16): 2048 0.120, 1024 0.121, 896 0.133, 768 0.149 -- a
//                    table-window refill stalls the wave, more waves hide it;
//   fp8 K/V: 2048 0.065, 3072 0.074, 1536 0.078, 1024 0.084 (half the bytes
//                    per step: more waves for the same bytes in flight).
#ifndef IFA4_DECODE_WAVES
#define IFA4_DECODE_WAVES 896
#endif
#ifndef IFA4_DECODE_WAVES_PAGED
#define IFA4_DECODE_WAVES_PAGED 2048
#endif
#ifndef IFA4_DECODE_WAVES_FP8
#define IFA4_DECODE_WAVES_FP8 2048
#endif
constexpr int64_t kDecodeWaves = IFA4_DECODE_WAVES;
constexpr int64_t kDecodeWavesPaged = IFA4_DECODE_WAVES_PAGED;
constexpr int64_t kDecodeWavesFp8 = IFA4_DECODE_WAVES_FP8;
constexpr int32_t kDecodeStep = 32;  // keys per step of a decode wave

// Upper bound of the 32-key steps of a decode call: every (sequence, kv head)
// at max_seqlen_k keys (one key when causal: top-left alignment, Lq = 1).
// key0_only: top-left causal decode, which sees key 0 only.
inline int64_t decode_max_steps(int64_t batch, int64_t kv_heads, int64_t max_seqlen_k,
                                bool key0_only) {
  const int64_t keys = key0_only ? (max_seqlen_k > 0 ? 1 : 0) : max_seqlen_k;
  return batch * kv_heads * ((keys + kDecodeStep - 1) / kDecodeStep);
}

// Small calls (few caches, or few steps): at least kDecodeMinSteps 32-key
// steps per wave, and at most kDecodeMaxParts waves per (sequence, kv head)
// cache -- or, for caches longer than kDecodeMaxParts * kDecodePartSteps
// steps, one wave per kDecodePartSteps steps.  With the combine split over
// several workgroups for many-part segments, a part of 2 steps (the same as the
// floor per wave, which then is the binding cap) measured fastest: one
// sequence of 16K / 32K / 64K keys 14.8 / 21.2 / 23.6 -> 12.9 / 15.8 / 21.3 us
// (8 steps per part before), fp8 cache 32K 21.9 -> 15.0, paged 32K 30.0 -> 18.6;
// 8K, 128K and the 64-sequence batch unchanged.  Same-session sweeps, Hq 8 /
// Hkv 2, d 128, non-causal (profiles/sweep_decode_small.md).
#ifndef IFA4_DECODE_MIN_STEPS
#define IFA4_DECODE_MIN_STEPS 2
#endif
#ifndef IFA4_DECODE_MAX_PARTS
#define IFA4_DECODE_MAX_PARTS 128
#endif
#ifndef IFA4_DECODE_PART_STEPS
#define IFA4_DECODE_PART_STEPS 2
#endif
constexpr int64_t kDecodeMinSteps = IFA4_DECODE_MIN_STEPS;
constexpr int64_t kDecodeMaxParts = IFA4_DECODE_MAX_PARTS;
constexpr int64_t kDecodePartSteps = IFA4_DECODE_PART_STEPS;

// fp8 caches of d 128 (contiguous or paged) whose kv heads sit side by side in
// every row (head stride = head_dim) stream their kv heads in pairs, one wave
// over whole rows of both (a pair holds at most 8 query heads); the kernel
// then sees half the kv heads, twice the group and 32-key steps of twice the
// bytes.
#ifndef IFA4_DECODE_FP8_PAIRS
#define IFA4_DECODE_FP8_PAIRS 1
#endif
#ifndef IFA4_DECODE_WAVES_FP8_PAIR
#define IFA4_DECODE_WAVES_FP8_PAIR 1024
#endif
constexpr int64_t kDecodeWavesFp8Pair = IFA4_DECODE_WAVES_FP8_PAIR;
// (paged: 1536, as for one kv head per wave more waves hide the block-table
// window refills; batch 64 at blocks of 16, one box: 64.5 us at 1024, 59.6 at
// 1536, 60.4-60.9 at 2048, against 66.0 streaming one kv head per wave)
#ifndef IFA4_DECODE_WAVES_FP8_PAIR_PAGED
#define IFA4_DECODE_WAVES_FP8_PAIR_PAGED 1536
#endif
constexpr int64_t kDecodeWavesFp8PairPaged = IFA4_DECODE_WAVES_FP8_PAIR_PAGED;
inline bool decode_pairs(bool fp8, int64_t head_dim, int64_t kv_heads, int64_t group,
                         int64_t k_stride_h, int64_t v_stride_h) {
  return IFA4_DECODE_FP8_PAIRS && fp8 && head_dim == 128 && kv_heads % 2 == 0 &&
         2 * group <= 8 && k_stride_h == head_dim && v_stride_h == head_dim;
}

// kv_heads: as the kernel sees them (pairs when pair is set).
inline int32_t decode_waves_for(int64_t batch, int64_t kv_heads, int64_t max_seqlen_k,
                                bool key0_only, bool fp8, bool paged, bool pair = false) {
  const int64_t t = decode_max_steps(batch, kv_heads, max_seqlen_k, key0_only);
  int64_t w = kDecodeWaves;
  if (paged && kDecodeWavesPaged > w) w = kDecodeWavesPaged;
  if (fp8 && kDecodeWavesFp8 > w) w = kDecodeWavesFp8;
  if (pair) w = paged ? kDecodeWavesFp8PairPaged : kDecodeWavesFp8Pair;
  const int64_t by_steps = (t + kDecodeMinSteps - 1) / kDecodeMinSteps;
  const int64_t seg_steps = batch * kv_heads > 0 ? t / (batch * kv_heads) : 0;
  const int64_t long_parts = (seg_steps + kDecodePartSteps - 1) / kDecodePartSteps;
  const int64_t by_parts =
      batch * kv_heads * (long_parts > kDecodeMaxParts ? long_parts : kDecodeMaxParts);
  if (by_steps < w) w = by_steps;
  if (by_parts < w) w = by_parts;
  return (int32_t)w;
}

// Split KV for prefill calls whose grid leaves the chip underfilled (few
// sequences or heads, short sequences): the longest query tile's KV range is
// the critical path, so when it exceeds the work one slot would get with
// perfect balance, every query tile's range is cut into chunks of that many
// tiles (at least kPrefillMinChunk), one workgroup per chunk, and a second pass
// merges the chunks' partials by log-sum-exp.  The chunk is then lengthened
// until the chunks with work fit the resident slots at once: with the balanced
// share, a query tile's last chunk is short and the count overshoots the slots
// a little (528 for one sequence of 4096 over 4 heads), and the few left over
// ran as a second round.  Fitted, against the balanced share (same session):
// one sequence over 4 heads, S 4096 / 8192: 61.6 -> 48.6, 141.6 -> 109.5 us;
// 8 x 1024: 39.5 -> 36.2; 4 x 2048: 59.5 -> 50.0; 2 x 4096 over 4 heads and
// 1 x 4096 over 8: 90.7 -> 74.2 (S 1024 / 2048 fit already: unchanged).
// Where splitting pays (same-session sweeps with the balanced share, per-token
// bf16 bias of extent 1024, Hq = Hkv, causal):
//   * grids of at most a quarter of the resident slots always: one sequence
//     over 4 heads, S 1024 / 2048 / 4096: 45.4 -> 22.2, 71.9 -> 31.3,
//     104.9 -> 65.8 us;
//   * grids of up to half of them when the longest range is at least
//     kPrefillSplitWideMinTiles: batch 8 x 1024 over 4 heads (256 workgroups,
//     16 tiles) 53.4 -> 43.3 us, 4 x 2048 73.1 -> 63.7, 1 x 8192 172.5 -> 147.7;
//     with 8-tile ranges the merge costs more than it saves (16 x 512: 30.6 ->
//     31.9 us; the shared-table 8 x 512 over 8 heads: 18.0 -> 28.8);
//   * with fitted chunks, grids below the slots too, when the chunk is at most
//     half of the longest range or shortens it by kPrefillSplitMinSaved tiles
//     (against no split, same session): 3 x 4096 over 4 heads (384 workgroups,
//     chunk 44 of 64 tiles) 112.3 -> 104.8 us, 5 x 2048 (16 of 32) 71.4 ->
//     61.5, 1 x 8192 over 6 (86 of 128) 185.5 -> 170.3, 5 x 1024 over 8 (8 of
//     16) 48.2 -> 41.5; at 22 of 32 (6 x 2048, 3 x 2048 over 8) equal, at 12 of
//     16 (12 x 1024) 1% slower, at 14 of 16 (7 x 1024 over 8) 12% slower;
//   * never at the slots and above: every grid of 512 workgroups measured lost
//     (8 x 1024 over 8 heads 32.0 -> 45.6 us, 1 x 16384 over 4 heads 373 -> 447,
//     2 x 8192 206 -> 225), and no chunk fits the slots there.
// The estimate assumes every sequence holds max_seqlen_q queries over
// max_seqlen_k keys (top-left); it only steers performance, any chunk size
// gives the same results up to rounding.  kPrefillSlots: resident workgroups
// of the prefill kernel on MI355X (256 CUs x 2).
constexpr int64_t kPrefillSlots = 512;
// Shortest chunk: 2 tiles (against 4, one sequence over 4 heads, same session:
// S 384 / 512 / 1024 18.6 -> 14.3, 18.5 -> 14.7, 20.4 -> 18.8 us; 3 tiles in
// between).
#ifndef IFA4_PREFILL_MIN_CHUNK
#define IFA4_PREFILL_MIN_CHUNK 2
#endif
constexpr int32_t kPrefillMinChunk = IFA4_PREFILL_MIN_CHUNK;
#ifndef IFA4_PREFILL_SPLIT_MAX_GRID
#define IFA4_PREFILL_SPLIT_MAX_GRID 511
#endif
constexpr int64_t kPrefillSplitMaxGrid = IFA4_PREFILL_SPLIT_MAX_GRID;  // below kPrefillSlots
// A split is taken when its chunk is at most half of the longest KV range, or
// shortens that range by at least this many tiles.
#ifndef IFA4_PREFILL_SPLIT_MIN_SAVED
#define IFA4_PREFILL_SPLIT_MIN_SAVED 16
#endif
constexpr int64_t kPrefillSplitMinSaved = IFA4_PREFILL_SPLIT_MIN_SAVED;
constexpr int64_t kPrefillSplitSmallGrid = 128;                        // kPrefillSlots / 4
// Chunk length as a percentage of the balanced share (sweep knob).
#ifndef IFA4_PREFILL_CHUNK_PCT
#define IFA4_PREFILL_CHUNK_PCT 100
#endif
constexpr int64_t kPrefillChunkPct = IFA4_PREFILL_CHUNK_PCT;
// Lengthen the chunk until every chunk with work is resident at once (1), or
// keep the balanced share (0; sweep knob).
#ifndef IFA4_PREFILL_CHUNK_FIT
#define IFA4_PREFILL_CHUNK_FIT 1
#endif
constexpr int64_t kPrefillSplitWideMinTiles = 16;

struct PrefillSplit {
  int32_t chunk_tiles;  // 0: no split
  int32_t n_chunks;     // chunk slots per query tile in the grid
};

// Tiles of the longest query tile and of all query tiles of one (sequence,
// head), for a sequence of lq queries over lk keys with top-left masks.
inline void prefill_tile_work(int64_t lq, int64_t lk, bool causal, int64_t window_left,
                              int32_t block_q, int32_t block_k, int64_t* tmax, int64_t* total) {
  *tmax = 0;
  *total = 0;
  for (int64_t q0 = 0; q0 < lq; q0 += block_q) {
    const int64_t q_hi = q0 + block_q < lq ? q0 + block_q : lq;
    const int64_t kend = causal ? (q_hi < lk ? q_hi : lk) : lk;
    const int64_t kbeg = window_left >= 0 ? (q0 - window_left > 0 ? q0 - window_left : 0) : 0;
    const int64_t t = kend > kbeg ? (kend + block_k - 1) / block_k - kbeg / block_k : 0;
    if (t > *tmax) *tmax = t;
    *total += t;
  }
}

// Chunks with work of one (sequence, head) when the KV range of every query
// tile is cut at multiples of `chunk` key tiles (the kernel's alignment).
inline int64_t prefill_chunk_count(int64_t lq, int64_t lk, bool causal, int64_t window_left,
                                   int32_t block_q, int32_t block_k, int64_t chunk) {
  int64_t n = 0;
  for (int64_t q0 = 0; q0 < lq; q0 += block_q) {
    const int64_t q_hi = q0 + block_q < lq ? q0 + block_q : lq;
    const int64_t kend = causal ? (q_hi < lk ? q_hi : lk) : lk;
    const int64_t kbeg = window_left >= 0 ? (q0 - window_left > 0 ? q0 - window_left : 0) : 0;
    if (kend <= kbeg) continue;
    n += ((kend + block_k - 1) / block_k - 1) / chunk - (kbeg / block_k) / chunk + 1;
  }
  return n;
}

// forced_chunk > 0: split every query tile into chunks of that many tiles.
inline PrefillSplit prefill_split_for(int64_t batch, int64_t n_heads, int64_t max_q,
                                      int64_t max_k, bool causal, int64_t window_left,
                                      int32_t block_q, int32_t block_k, int32_t forced_chunk) {
  PrefillSplit s{0, 1};
  if (batch <= 0 || max_q <= 0 || max_k <= 0) return s;
  int64_t tmax = 0, total = 0;
  prefill_tile_work(max_q, max_k, causal, window_left, block_q, block_k, &tmax, &total);
  int64_t chunk = forced_chunk;
  if (chunk <= 0) {
    const int64_t grid = (max_q + block_q - 1) / block_q * n_heads * batch;
    if (grid > kPrefillSplitMaxGrid) return s;
    if (grid > kPrefillSplitSmallGrid && tmax < kPrefillSplitWideMinTiles) return s;
    const int64_t balanced =
        ((total * batch * n_heads + kPrefillSlots - 1) / kPrefillSlots * kPrefillChunkPct + 99) /
        100;
    chunk = balanced > kPrefillMinChunk ? balanced : kPrefillMinChunk;
    if (IFA4_PREFILL_CHUNK_FIT && chunk < tmax) {
      // Chunks of the balanced share can number a little more than the slots
      // (each query tile's last chunk is short): the few left over then run as
      // a second round.  Take the shortest chunk whose workgroups all fit
      // (binary search; the count falls as the chunk grows).
      auto fits = [&](int64_t c) {
        return prefill_chunk_count(max_q, max_k, causal, window_left, block_q, block_k, c) *
                   batch * n_heads <=
               kPrefillSlots;
      };
      if (!fits(chunk)) {
        // hi = tmax: one chunk per query tile whose range starts at key 0, which
        // the grid (below the slots) fits; otherwise the search ends there and
        // the call is not split
        int64_t lo = chunk, hi = tmax;
        while (hi - lo > 1) {
          const int64_t mid = lo + (hi - lo) / 2;
          if (fits(mid)) hi = mid; else lo = mid;
        }
        chunk = hi;
      }
    }
    // A split that shortens the longest range by little does not repay the
    // chunks' partials and the merge pass.
    if (tmax <= chunk || (2 * chunk > tmax && tmax - chunk < kPrefillSplitMinSaved)) return s;
  }
  // chunk slots: enough for a query tile that meets every key tile (chunks are
  // aligned to multiples of `chunk` tiles on the key axis), so the grid and the
  // workspace cover whatever the masks, lengths and alignment of a sequence
  const int64_t key_tiles = (max_k + block_k - 1) / block_k;
  s.chunk_tiles = (int32_t)chunk;
  s.n_chunks = (int32_t)((key_tiles + chunk - 1) / chunk);
  if (s.n_chunks < 1) s.n_chunks = 1;
  return s;
}

}  // namespace ifa4
