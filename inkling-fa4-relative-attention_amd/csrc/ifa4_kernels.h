// Internal interface between the C ABI layer (ifa4_api.cpp) and the HIP
// kernels.  Not installed; the public interface is include/ifa4.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

struct ifa4_args;

namespace ifa4 {

struct PrefillParams {
  const void* q;
  const void* k;
  const void* v;
  const void* rel;
  void* out;
  float* lse;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, rel_st, rel_sh, o_st, o_sh, lse_sh;
  int32_t total_q;      // rows of q / out (cu_seqlens_q is clamped to it)
  int32_t total_k;      // rows of k / v (cu_seqlens_k is clamped to it)
  int32_t batch;
  int32_t n_heads;
  int32_t group;        // n_heads / kv_heads
  int32_t rel_extent;
  int32_t rel_width;    // last dim of rel (>= rel_extent)
  int32_t window_left;  // -1: none
  int32_t causal;
  int32_t bottom_right; // 1: query i sits at key position i + (lk - lq) (IFA4_FLAG_BOTTOM_RIGHT)
  int32_t no_prune;
  int32_t rel_dtype;    // 0 bf16, 1 fp16, 2 fp32
  int32_t n_qtiles;     // ceil(max_seqlen_q / block_q)
  int32_t xcd_pairs;    // (sequence, kv head) pairs per XCD in the XCD-aware order, or 0
  float scale_log2;     // softmax_scale * log2(e)
  // Split KV (chunk_tiles > 0): each q tile's KV tile range is cut into chunks
  // of chunk_tiles tiles, one workgroup each (n_chunks chunk slots per q tile in
  // the grid); a tile with more than one chunk writes normalised partials
  // part_o [n_chunks][n_heads][total_q][head_dim] fp32 and their LSE (log2
  // units) part_lse [n_chunks][n_heads][total_q], merged by a second pass.
  int32_t chunk_tiles;
  int32_t n_chunks;
  float* part_o;
  float* part_lse;
  // Fused relative-logit projection (wt != nullptr): rel / rel_st / rel_sh /
  // rel_dtype describe r [Tq, Hq, 16]; wt is W^T [rel_width, 16] fp32, rows
  // contiguous; bias(i, dist) = sum_c r[i, c] * wt[dist, c].
  const float* wt;
};

struct DecodeParams {
  const void* q;
  const void* k;
  const void* v;
  const void* rel;
  void* out;
  float* lse;
  const int32_t* cu_q;
  const int32_t* cu_k;
  float* ws_o;        // [batch * kv_heads + n_waves][group][head_dim] partials
  float* ws_lse;      // [batch * kv_heads + n_waves][group] (log2 domain)
  int32_t* ws_meta;   // [batch * kv_heads][2]: first and last wave of a segment
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, rel_st, rel_sh, o_st, o_sh, lse_sh;
  int32_t total_q;   // rows of q / out (cu_seqlens_q is clamped to it)
  int32_t total_k;   // rows of k / v (cu_seqlens_k is clamped to it; unused when paged)
  int32_t batch;
  int32_t n_heads;
  int32_t kv_heads;
  int32_t group;
  int32_t rel_extent;
  int32_t causal;
  int32_t bottom_right;  // see PrefillParams
  int32_t window_left;   // -1: none (only matters with bottom_right: top-left decode never masks)
  int32_t rel_dtype;
  int32_t n_waves;   // persistent waves of pass 1 (0: nothing to stream)
  int32_t kv_fp8;    // 1: K and V are fp8 (OCP e4m3), K scale folded into scale_log2
  // 1: each kv head of these params is a pair of adjacent fp8 kv heads (k_sh,
  // v_sh = 2 * head_dim, group = both heads' query heads), streamed as whole rows
  int32_t kv_pair;
  float scale_log2;
  float v_scale;     // multiplies the output (1 for 16-bit V)
  // Paged KV cache (block_table != nullptr): k/v are block pools, key j of
  // sequence b is row j & (2^block_shift - 1) of block
  // block_table[b * bt_stride + (j >> block_shift)]; lengths from seqused_k.
  const int32_t* block_table;
  const int32_t* seqused_k;
  int64_t bt_stride, k_sblk, v_sblk;
  int32_t block_shift;
  int32_t num_blocks;
  int32_t max_blocks;  // table entries per sequence
};

int prefill_block_q();
int prefill_proj_block_q();  // query rows per workgroup of the fused-projection kernel
int prefill_block_k();
int prefill_waves();
hipError_t launch_prefill(const PrefillParams& p, int head_dim, int qkv_dtype, hipStream_t stream);

int decode_max_group();
int decode_fp8_max_group();
hipError_t launch_decode(const DecodeParams& p, int head_dim, int qkv_dtype, hipStream_t stream);

// Common body of the contiguous 16-bit decode entry points (ifa4_api.cpp): the
// host checks with the workspace bytes the call needs, and the call itself on
// a caller-provided workspace.
int32_t decode_workspace_need(const ifa4_args* args, size_t* bytes);
int32_t decode_run(const ifa4_args* args, void* workspace, size_t workspace_bytes, void* stream);

}  // namespace ifa4
