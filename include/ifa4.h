/*
 * ifa4.h -- C ABI of the MI355X (gfx950) relative-bias flash attention library.
 *
 * The library (libifa4.so) holds hand-written HIP kernels for the forward pass
 * of Inkling relative-position-bias attention.  It has no torch dependency: every
 * argument is a plain pointer, size, stride or enum.  The caller owns every
 * buffer; the library never allocates, frees or synchronises, and launches only
 * on the stream it is given.  All entry points are re-entrant (the tile table is
 * const) and return an ifa4_status; nothing throws or aborts across the ABI.
 *
 * Semantics are those of the reference oracle `ref_rel_attn`
 * (src/inkling_fa4/reference.py:19-40):
 *   for sequence b, local query i in [0,Lq), local key j in [0,Lk),
 *   kv head kh = h / (n_heads / kv_heads),
 *     s    = softmax_scale * <q[qs+i,h], k[ks+j,kh]>
 *     dist = i + (Lq - Lk) - j;  s += rel[qs+i, h, dist]  iff 0 <= dist < rel_extent
 *     visible iff (!causal || i >= j) && (window_left < 0 || i - j <= window_left)
 *     out[qs+i,h] = softmax_j(s) @ v[ks+j,kh]           (written in the q dtype)
 *     lse[h, qs+i] = ln sum_j exp(s)  over visible j     (fp32, optional)
 * A row with no visible key gets out = 0 and lse = -inf (the reference oracle
 * yields NaN there; the reference Triton kernels yield 0).
 */
#ifndef IFA4_H_
#define IFA4_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IFA4_ABI_VERSION 1

typedef enum ifa4_status {
  IFA4_OK = 0,
  IFA4_EINVAL = 1,        /* malformed argument: null pointer, bad size or stride */
  IFA4_EUNSUPPORTED = 2,  /* well-formed but not implemented (head_dim, dtype mix) */
  IFA4_EWORKSPACE = 3,    /* decode workspace missing or too small */
  IFA4_ELAUNCH = 4        /* the HIP runtime reported an error at launch */
} ifa4_status;

typedef enum ifa4_dtype {
  IFA4_BF16 = 0,
  IFA4_FP16 = 1,
  IFA4_FP32 = 2,
  IFA4_FP8_E4M3 = 3   /* OCP e4m3 (float8_e4m3fn); K/V of ifa4_decode_quant_fwd only */
} ifa4_dtype;

/* Flags (ifa4_args.flags). */
#define IFA4_FLAG_NO_PRUNE 0x1u  /* debug: visit every KV tile (pruning-invariance tests) */
/*
 * Bottom-right alignment, the convention of upstream flash-attn and of the
 * serving backend's score_mod (outputs/architecture.md:72, d = (i + sk - sq) - j):
 * query i sits at key position i + (Lk - Lq), so
 *   dist = i + (Lk - Lq) - j,  causal keeps j <= i + (Lk - Lq),
 *   the window keeps i + (Lk - Lq) - j <= window_left.
 * Without the flag the semantics are the reference oracle's (top-left, above).
 * The two agree when Lq == Lk.
 */
#define IFA4_FLAG_BOTTOM_RIGHT 0x2u
/* test: ifa4_prefill_fwd_ws splits every query tile's KV range into chunks of
 * two KV tiles (exercises the split-KV merge on small inputs) */
#define IFA4_FLAG_SPLIT_KV_2 0x4u

/*
 * Arguments of one forward call.  Layouts (element strides, last dim contiguous):
 *   q   [total_q, n_heads,  head_dim]   qkv_dtype
 *   k,v [total_k, kv_heads, head_dim]   qkv_dtype
 *   rel [total_q, n_heads,  rel_width]  rel_dtype, rel_width >= rel_extent;
 *        rel_stride_t may be 0 (one per-head table shared by every token)
 *   out [total_q, n_heads,  head_dim]   qkv_dtype
 *   lse [n_heads, total_q] fp32 with head stride lse_stride_h (may be NULL)
 *   cu_seqlens_q/k: device int32 [batch+1], non-decreasing, cu[0] = 0,
 *        cu_q[batch] <= total_q, cu_k[batch] <= total_k.  Read only on the device,
 *        where each sequence's [cu[b], cu[b+1]) is clamped to [0, total]: offsets
 *        outside that range, or decreasing, give shorter or empty sequences
 *        (results for them are unspecified) but never reads or writes outside
 *        the tensors.
 * max_seqlen_q/k must bound every sequence length; they size the grid (query
 * rows past max_seqlen_q are not written).
 * q and out may be NULL when total_q == 0, k and v when total_k == 0 (contiguous
 * K/V): nothing is read from or written to them then.
 * Mirrors the argument list of inkling_fa4_rel_attention_triton
 * (src/inkling_fa4/triton_kernel.py:85-89,99-105) plus softmax_scale and lse.
 */
typedef struct ifa4_args {
  uint32_t struct_size;   /* sizeof(ifa4_args), checked by ifa4_validate */
  uint32_t flags;         /* IFA4_FLAG_* */
  const void* q;
  const void* k;
  const void* v;
  const void* rel;
  void* out;
  float* lse;
  const int32_t* cu_seqlens_q;
  const int32_t* cu_seqlens_k;
  int64_t q_stride_t, q_stride_h;
  int64_t k_stride_t, k_stride_h;
  int64_t v_stride_t, v_stride_h;
  int64_t rel_stride_t, rel_stride_h;
  int64_t out_stride_t, out_stride_h;
  int64_t lse_stride_h;
  int64_t total_q, total_k;
  int32_t batch;
  int32_t n_heads;
  int32_t kv_heads;
  int32_t head_dim;
  int32_t rel_extent;
  int32_t rel_width;
  int32_t max_seqlen_q;
  int32_t max_seqlen_k;
  int32_t window_left;    /* -1: no window */
  int32_t causal;         /* 0 or 1; top-left aligned on local indices */
  float softmax_scale;    /* > 0 */
  int32_t qkv_dtype;      /* ifa4_dtype: IFA4_BF16 or IFA4_FP16 */
  int32_t rel_dtype;      /* ifa4_dtype */
} ifa4_args;

/*
 * Fused relative-logit projection (prefill): instead of a materialised
 * rel_logits [total_q, n_heads, rel_width], the bias is computed in the kernel
 * from the low-rank factors of the serving backend's RelLogitsProj
 * (outputs/architecture.md:24,52-54, einsum(thd,de->the, r, W)):
 *   bias(token t, head h, dist) = sum_c r[t, h, c] * W[c, dist],  c < d_rel = 16,
 * applied for 0 <= dist < rel_extent as usual.  r has args.rel_dtype (bf16 or
 * fp32) and the element strides below (last dim contiguous); W is passed
 * transposed, wt = W^T [args.rel_width, 16] fp32, rows contiguous.  args.rel and
 * args.rel_stride_t/h are not read.  Any rel_extent <= rel_width: the band is
 * projected on the matrix cores (bf16 hi + lo split of r and W^T, ~16
 * significant bits) one 32-row x 64-key tile at a time; W^T rows are read
 * from L2 (rel_width x 64 bytes).
 */
typedef struct ifa4_rel_proj {
  uint32_t struct_size;   /* sizeof(ifa4_rel_proj) */
  int32_t d_rel;          /* 16 */
  const void* r;          /* [total_q, n_heads, d_rel] */
  int64_t r_stride_t, r_stride_h;
  const float* wt;        /* [rel_width, d_rel] fp32, 16-byte aligned */
} ifa4_rel_proj;

/* Tile shape chosen for a call (the gfx950 tile table). */
typedef struct ifa4_tile {
  int32_t block_q;        /* query rows per workgroup */
  int32_t block_k;        /* keys per KV tile */
  int32_t waves;          /* wavefronts per workgroup */
  int32_t stages;         /* LDS buffers for K/V */
  int32_t kv_chunk;       /* decode: most keys one wave streams; prefill: keys per KV
                             chunk when ifa4_prefill_fwd_ws splits the call, else 0 */
} ifa4_tile;

/* Human-readable name of a status code; never NULL. */
const char* ifa4_status_str(int32_t status);

/* ABI version the library was built with (IFA4_ABI_VERSION). */
int32_t ifa4_abi_version(void);

/* Pure host-side argument check; touches no device memory. */
int32_t ifa4_validate(const ifa4_args* args);

/*
 * Prefill / varlen / chunked / sliding-window forward, one launch over every
 * (query tile, head, sequence).  Replaces the per-sequence launch loop of
 * inkling_fa4_rel_attention_triton (src/inkling_fa4/triton_kernel.py:84-107)
 * and inkling_fa4_rel_attention_kv_pruned_triton
 * (src/inkling_fa4/triton_kernel_kv_pruned.py:210-279).  stream: hipStream_t
 * (NULL = the null stream).
 */
int32_t ifa4_prefill_fwd(const ifa4_args* args, void* stream);

/*
 * Prefill with a workspace, for calls whose grid would leave the chip
 * underfilled or unbalanced (few sequences or heads, short sequences): the
 * tile table then cuts each query tile's KV range into chunks processed by
 * separate workgroups (split KV), and a second pass merges the chunks' partial
 * outputs by log-sum-exp.  ifa4_prefill_workspace_bytes gives the workspace
 * the call needs, 0 when the table does not split it (ifa4_prefill_fwd_ws then
 * runs exactly ifa4_prefill_fwd and the workspace may be NULL).  The workspace
 * (256-byte aligned, contents on entry irrelevant) is scratch for one call;
 * calls that share one must not overlap.  Results equal ifa4_prefill_fwd's up
 * to the rounding of the merge.  Replaces the same launch loop as
 * ifa4_prefill_fwd (src/inkling_fa4/triton_kernel.py:94-106), whose grid of
 * (heads, query tiles) per sequence has the same underfill at small batch.
 */
size_t ifa4_prefill_workspace_bytes(const ifa4_args* args);
int32_t ifa4_prefill_fwd_ws(const ifa4_args* args, void* workspace, size_t workspace_bytes,
                            void* stream);

/* Prefill with the fused relative-logit projection (ifa4_rel_proj). */
int32_t ifa4_prefill_rproj_fwd(const ifa4_args* args, const ifa4_rel_proj* proj, void* stream);

/* Tile shape ifa4_prefill_fwd uses for these arguments, and the KV split of
 * ifa4_prefill_fwd_ws (kv_chunk). */
int32_t ifa4_prefill_tile(const ifa4_args* args, ifa4_tile* tile);

/*
 * Host-side count of the KV tiles the prefill kernel visits, using the same
 * pruning rule as the device code, from host copies of cu_seqlens.  total =
 * tiles an unpruned kernel would visit.  For reports and tests.
 */
int32_t ifa4_prefill_count_tiles(const ifa4_args* args, const int32_t* host_cu_seqlens_q,
                                 const int32_t* host_cu_seqlens_k, int64_t* visited,
                                 int64_t* total);

/*
 * Decode: exactly one query token per sequence (total_q == batch, and
 * cu_seqlens_q = arange(batch + 1), which only the device reads: the rows of a
 * sequence with another query count get out = 0 and lse = -inf).  Split-KV,
 * stream-K: pass 1 runs up to W persistent waves (W from the tile table: 896
 * for a contiguous 16-bit cache, 2048 for a paged one; for an fp8 cache 1024
 * when adjacent kv heads stream in pairs, 1536 paged, else 2048; fewer for
 * small calls) over all (sequence, kv head) caches laid end to end in 32-key
 * steps, each wave an equal range of work (a step whose keys carry bias
 * counts 7/4 of a plain one; ifa4_decode_tile reports the keys per wave of a
 * contiguous 16-bit cache); it writes one (o, lse) partial per (cache, wave)
 * it touches into the workspace.  Pass 2 merges each cache's partials by log-sum-exp and
 * writes out/lse.  The workspace (ifa4_decode_workspace_bytes, 256-byte
 * aligned, contents on entry irrelevant) is scratch for one call; calls that
 * share a workspace must not overlap.  Replaces
 * inkling_fa4_rel_attention_decode_triton
 * (src/inkling_fa4/triton_kernel_decode.py:127-170).
 */
size_t ifa4_decode_workspace_bytes(const ifa4_args* args);
int32_t ifa4_decode_tile(const ifa4_args* args, ifa4_tile* tile);
int32_t ifa4_decode_fwd(const ifa4_args* args, void* workspace, size_t workspace_bytes,
                        void* stream);

/*
 * Paged KV cache, the serving caller's format (the reference's serving backend
 * keeps KV in blocks of 16 tokens, outputs/architecture.md:117-120; the
 * reference kernels themselves take contiguous varlen K/V only).  The cache is
 * a pool of fixed-size blocks
 *   k_cache, v_cache [num_blocks, block_size, kv_heads, head_dim]  (qkv_dtype)
 * addressed as  base + blk * k_stride_block + row * args.k_stride_t
 *                    + kv_head * args.k_stride_h  (elements; same for v).
 * Sequence b holds seqused_k[b] keys; its key j sits in block
 *   block_table[b * block_table_stride + j / block_size]  at row j % block_size.
 * With a paged cache, args.k / args.v are the pool bases, args.cu_seqlens_k is
 * not read (may be NULL), args.total_k is ignored, and args.max_seqlen_k must
 * bound every seqused_k[b].  Keys are read only below seqused_k[b] (clamped to
 * [0, max_blocks_per_seq * block_size]); a table entry outside [0, num_blocks)
 * reads as zero keys and values instead of leaving the pool.
 */
typedef struct ifa4_paged_kv {
  uint32_t struct_size;         /* sizeof(ifa4_paged_kv) */
  int32_t block_size;           /* tokens per block: a power of two, 8 .. 65536 */
  const int32_t* block_table;   /* device int32 [batch, block_table_stride] */
  const int32_t* seqused_k;     /* device int32 [batch]: keys held by each sequence */
  int64_t block_table_stride;   /* elements between the table rows of two sequences */
  int64_t k_stride_block;       /* elements between two blocks of k_cache */
  int64_t v_stride_block;       /* elements between two blocks of v_cache */
  int32_t num_blocks;           /* blocks in the pool */
  int32_t max_blocks_per_seq;   /* table entries per sequence, >= ceil(max_seqlen_k / block_size) */
} ifa4_paged_kv;

/*
 * Decode over a paged KV cache: the same two passes as ifa4_decode_fwd with
 * the same workspace layout (more partial slots: a paged cache streams with up
 * to 2048 waves), results equal to ifa4_decode_fwd on the same keys stored
 * contiguously up to the order of the split merge.  Replaces the KV-cache read of the serving
 * backend's flash_attn_varlen_func call (block_table / seqused_k arguments),
 * outputs/architecture.md:117-120.
 */
size_t ifa4_decode_paged_workspace_bytes(const ifa4_args* args, const ifa4_paged_kv* kv);
int32_t ifa4_decode_paged_fwd(const ifa4_args* args, const ifa4_paged_kv* kv, void* workspace,
                              size_t workspace_bytes, void* stream);

/*
 * Quantised KV cache for decode: K and V stored as fp8 (OCP e4m3), one scale
 * per tensor (k = k_stored * k_scale, v = v_stored * v_scale), the serving
 * backend's FP8 KV cache (outputs/architecture.md:127, "Dtype: BF16 / FP8").
 * q, out and rel keep args.qkv_dtype / rel_dtype; K/V strides are in fp8
 * elements (bytes) and must be multiples of 16.  It halves the bytes decode
 * streams.  The result is that of ifa4_decode_fwd on the dequantised K/V
 * (computed in fp32 from the exact fp8 values).
 */
typedef struct ifa4_kv_quant {
  uint32_t struct_size;   /* sizeof(ifa4_kv_quant) */
  int32_t kv_dtype;       /* IFA4_FP8_E4M3 */
  float k_scale;          /* > 0, finite */
  float v_scale;          /* > 0, finite */
} ifa4_kv_quant;

/* kv: NULL for contiguous K/V (args.cu_seqlens_k), else a paged cache. */
size_t ifa4_decode_quant_workspace_bytes(const ifa4_args* args, const ifa4_paged_kv* kv,
                                         const ifa4_kv_quant* quant);
int32_t ifa4_decode_quant_fwd(const ifa4_args* args, const ifa4_paged_kv* kv,
                              const ifa4_kv_quant* quant, void* workspace,
                              size_t workspace_bytes, void* stream);

/*
 * Allocation-free decode: ifa4_decode_fwd with the library's own workspace
 * instead of a workspace argument.  No counterpart in the reference; it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The workspace is a
 * device array of IFA4_DECODE_SCRATCH_BYTES that each GPU holds from the
 * library's first use there until the process ends; a call that needs more
 * (ifa4_decode_workspace_bytes) returns IFA4_EWORKSPACE before touching the
 * device.  The call allocates and frees nothing.  Every call on one GPU shares
 * that GPU's array, so calls that overlap in time on one GPU (other streams or
 * host threads) race.  `stream` must belong to the current device (else
 * IFA4_EINVAL).  Results are those of ifa4_decode_fwd on the same arguments.
 * The array's device address is looked up on the first call on each device and
 * kept for the rest of the process: after hipDeviceReset on a device (or an
 * unload of the library) the kept address is stale, so the entry point must not
 * be called there again.
 */
#define IFA4_DECODE_SCRATCH_BYTES (32u << 20)
int32_t ifa4_decode_fwd_noalloc(const ifa4_args* args, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* IFA4_H_ */
