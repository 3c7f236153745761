// gfx950 tile table.  Replaces the per-arch Triton presets of
// src/inkling_fa4/autotune_configs.py:17-50 (seq-length buckets of
// BLOCK_Q/BLOCK_K/num_warps/num_stages for sm86/sm90/sm100).
//
// Prefill: one shape for every sequence length.  The kernel is written for
// 4 waves x 32 query rows (BLOCK_Q 128) and 64-key KV tiles in two LDS stages
// (64 KiB of LDS at head_dim 128, so two workgroups fit in the 160 KiB of a
// CU); the shape is a compile-time property of the kernel, listed here so the
// host reports what runs.
//
// Decode: keys per KV split.  The split count is ceil(max_seqlen_k / chunk);
// the chunk is the largest power-of-two multiple of 64 that still gives at
// least kDecodeTargetWaves split waves, so short caches are split finer.
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

#ifndef IFA4_DECODE_TARGET_WAVES
#define IFA4_DECODE_TARGET_WAVES 8192
#endif
constexpr int32_t kDecodeChunks[] = {1024, 512, 256, 128, 64};
constexpr int64_t kDecodeTargetWaves = IFA4_DECODE_TARGET_WAVES;

inline int32_t decode_chunk_for(int64_t batch, int64_t kv_heads, int64_t max_seqlen_k) {
  for (int32_t c : kDecodeChunks) {
    const int64_t splits = (max_seqlen_k + c - 1) / c;
    if (batch * kv_heads * splits >= kDecodeTargetWaves) return c;
  }
  return kDecodeChunks[sizeof(kDecodeChunks) / sizeof(kDecodeChunks[0]) - 1];
}

}  // namespace ifa4
