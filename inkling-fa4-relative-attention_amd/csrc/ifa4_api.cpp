// C ABI of the gfx950 relative-bias attention library: argument validation,
// tile selection and kernel dispatch.  Declared in include/ifa4.h.
//
// The reference has no validation at all (src/inkling_fa4/triton_kernel.py:84-107:
// bad shapes surface as Triton errors or silent out-of-bounds reads); here every
// entry point checks its arguments on the host before anything is launched and
// reports a status code.
#include "ifa4.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "ifa4_kernels.h"
#include "tile_table.h"

namespace {

constexpr float kLog2eHost = 1.4426950408889634f;

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Row counts as the kernels take them (cu_seqlens are clamped to these on the
// device); a row index past INT32_MAX is not addressable there anyway.
int32_t clamp_rows(int64_t n) { return n < INT32_MAX ? (int32_t)n : INT32_MAX; }

// kv != nullptr: K/V are a paged cache described by *kv (checked by
// check_paged); cu_seqlens_k is then not read and may be NULL.
// kv_esize: bytes per K/V element (2, or 1 for an fp8 cache).
int32_t check_args(const ifa4_args* a, const ifa4_paged_kv* kv = nullptr, int kv_esize = 2) {
  if (a == nullptr) return IFA4_EINVAL;
  if (a->struct_size != sizeof(ifa4_args)) return IFA4_EINVAL;
  if (a->batch < 0 || a->n_heads < 1 || a->kv_heads < 1) return IFA4_EINVAL;
  if (a->n_heads % a->kv_heads != 0) return IFA4_EINVAL;
  if (a->total_q < 0 || a->total_k < 0) return IFA4_EINVAL;
  if (a->max_seqlen_q < 0 || a->max_seqlen_k < 0) return IFA4_EINVAL;
  if (a->rel_extent < 0 || a->rel_width < a->rel_extent) return IFA4_EINVAL;
  if (a->window_left < -1) return IFA4_EINVAL;
  if (a->causal != 0 && a->causal != 1) return IFA4_EINVAL;
  if (a->qkv_dtype < IFA4_BF16 || a->qkv_dtype > IFA4_FP32) return IFA4_EINVAL;
  if (a->rel_dtype < IFA4_BF16 || a->rel_dtype > IFA4_FP32) return IFA4_EINVAL;
  if (a->head_dim < 1) return IFA4_EINVAL;
  if (a->q_stride_t < 0 || a->q_stride_h < 0 || a->k_stride_t < 0 || a->k_stride_h < 0 ||
      a->v_stride_t < 0 || a->v_stride_h < 0 || a->rel_stride_t < 0 || a->rel_stride_h < 0 ||
      a->out_stride_t < 0 || a->out_stride_h < 0 || a->lse_stride_h < 0)
    return IFA4_EINVAL;
  if (!(std::isfinite(a->softmax_scale))) return IFA4_EINVAL;
  if (a->batch == 0) return IFA4_OK;  // nothing to read or write
  if (a->cu_seqlens_q == nullptr || (kv == nullptr && a->cu_seqlens_k == nullptr))
    return IFA4_EINVAL;
  // Empty query or key sets may come with null data pointers (an empty tensor's
  // storage); the kernels then read nothing from them.
  if ((a->q == nullptr || a->out == nullptr) && a->total_q > 0) return IFA4_EINVAL;
  if ((a->k == nullptr || a->v == nullptr) && (kv != nullptr || a->total_k > 0))
    return IFA4_EINVAL;
  if (a->rel_extent > 0 && a->rel == nullptr) return IFA4_EINVAL;
  if (a->lse != nullptr) {
    if (!aligned(a->lse, 4)) return IFA4_EINVAL;
    if (a->n_heads > 1 && a->lse_stride_h < a->total_q) return IFA4_EINVAL;
  }
  // Supported, not just well-formed.
  if (a->head_dim != 64 && a->head_dim != 128) return IFA4_EUNSUPPORTED;
  if (a->qkv_dtype == IFA4_FP32) return IFA4_EUNSUPPORTED;
  if (!(a->softmax_scale > 0.f)) return IFA4_EUNSUPPORTED;
  // 16-byte vector loads of q/k/v rows, 8-byte stores of out rows.
  if (!aligned(a->q, 16) || !aligned(a->k, 16) || !aligned(a->v, 16) || !aligned(a->out, 16))
    return IFA4_EUNSUPPORTED;
  if ((a->q_stride_t | a->q_stride_h | a->out_stride_t | a->out_stride_h) % 8 != 0)
    return IFA4_EUNSUPPORTED;
  if ((a->k_stride_t | a->k_stride_h | a->v_stride_t | a->v_stride_h) % (16 / kv_esize) != 0)
    return IFA4_EUNSUPPORTED;
  if (a->rel != nullptr && !aligned(a->rel, a->rel_dtype == IFA4_FP32 ? 4 : 2))
    return IFA4_EINVAL;
  // Kernels address one sequence of one head through a buffer resource with
  // 32-bit offsets and read rows past the sequence end as zero: token rows
  // must not overlap, and a sequence's rows must span less than 2 GiB.
  if (a->q_stride_t < a->head_dim || a->k_stride_t < a->head_dim ||
      a->v_stride_t < a->head_dim)
    return IFA4_EUNSUPPORTED;
  if (a->rel_stride_t != 0 && a->rel_stride_t < a->rel_width) return IFA4_EUNSUPPORTED;
  const int64_t rel_esize = a->rel_dtype == IFA4_FP32 ? 4 : 2;
  const int64_t kLimit = int64_t(1) << 31;
  const int64_t kpad = 128;  // rows a tile may read past the end
  // a paged cache is addressed one block at a time (check_paged)
  const int64_t k_rows = kv == nullptr ? a->max_seqlen_k + kpad : 0;
  if ((a->max_seqlen_q + kpad) * a->q_stride_t * 2 >= kLimit ||
      k_rows * a->k_stride_t * kv_esize >= kLimit || k_rows * a->v_stride_t * kv_esize >= kLimit ||
      ((a->max_seqlen_q + kpad) * a->rel_stride_t + a->rel_width) * rel_esize >= kLimit)
    return IFA4_EUNSUPPORTED;
  return IFA4_OK;
}

// Decode reads the query heads of a GQA group, and the bias of every head of a
// token, through one buffer resource each: their spans over the heads must stay
// below 2 GiB too.  Prefill addresses each head from its own 64-bit base and
// has no such limit.
int32_t check_head_spans(const ifa4_args* a) {
  const int64_t kLimit = int64_t(1) << 31;
  const int64_t rel_esize = a->rel_dtype == IFA4_FP32 ? 4 : 2;
  if ((int64_t)(a->n_heads - 1) * a->q_stride_h * 2 + (int64_t)a->head_dim * 2 >= kLimit ||
      (a->rel_extent > 0 &&
       ((int64_t)(a->n_heads - 1) * a->rel_stride_h + a->rel_width) * rel_esize >= kLimit))
    return IFA4_EUNSUPPORTED;
  return IFA4_OK;
}

// Paged KV cache description (include/ifa4.h, ifa4_paged_kv).
int32_t check_paged(const ifa4_args* a, const ifa4_paged_kv* kv, int kv_esize = 2) {
  if (kv == nullptr || kv->struct_size != sizeof(ifa4_paged_kv)) return IFA4_EINVAL;
  const int32_t bs = kv->block_size;
  if (bs < 8 || bs > 65536 || (bs & (bs - 1)) != 0) return IFA4_EINVAL;
  // one wave load covers 1024 / (head_dim * esize) rows, all within one block
  if (a->head_dim > 0 && bs < 1024 / (a->head_dim * kv_esize)) return IFA4_EUNSUPPORTED;
  if (kv->block_table_stride < 0 || kv->k_stride_block < 0 || kv->v_stride_block < 0 ||
      kv->num_blocks < 0 || kv->max_blocks_per_seq < 0)
    return IFA4_EINVAL;
  if (a->batch == 0) return IFA4_OK;
  if (kv->block_table == nullptr || kv->seqused_k == nullptr || !aligned(kv->block_table, 4) ||
      !aligned(kv->seqused_k, 4))
    return IFA4_EINVAL;
  if (kv->num_blocks < 1 || kv->max_blocks_per_seq < 1) return IFA4_EINVAL;
  // the table row must address max_seqlen_k keys; key indices stay in int32
  if ((int64_t)kv->max_blocks_per_seq * bs < a->max_seqlen_k) return IFA4_EINVAL;
  if ((int64_t)kv->max_blocks_per_seq * bs > (int64_t(1) << 30)) return IFA4_EUNSUPPORTED;
  // 16-byte loads from every block; one block of one kv head spans < 2 GiB
  if ((kv->k_stride_block | kv->v_stride_block) % (16 / kv_esize) != 0) return IFA4_EUNSUPPORTED;
  const int64_t kLimit = int64_t(1) << 31;
  if (((int64_t)(bs - 1) * a->k_stride_t + a->head_dim) * kv_esize >= kLimit ||
      ((int64_t)(bs - 1) * a->v_stride_t + a->head_dim) * kv_esize >= kLimit)
    return IFA4_EUNSUPPORTED;
  return IFA4_OK;
}

ifa4::PrefillParams make_prefill_params(const ifa4_args* a) {
  ifa4::PrefillParams p{};
  p.q = a->q;
  p.k = a->k;
  p.v = a->v;
  p.rel = a->rel;
  p.out = a->out;
  p.lse = a->lse;
  p.cu_q = a->cu_seqlens_q;
  p.cu_k = a->cu_seqlens_k;
  p.q_st = a->q_stride_t;
  p.q_sh = a->q_stride_h;
  p.k_st = a->k_stride_t;
  p.k_sh = a->k_stride_h;
  p.v_st = a->v_stride_t;
  p.v_sh = a->v_stride_h;
  p.rel_st = a->rel_stride_t;
  p.rel_sh = a->rel_stride_h;
  p.o_st = a->out_stride_t;
  p.o_sh = a->out_stride_h;
  p.lse_sh = a->lse_stride_h;
  p.total_q = clamp_rows(a->total_q);
  p.total_k = clamp_rows(a->total_k);
  p.batch = a->batch;
  p.n_heads = a->n_heads;
  p.group = a->n_heads / a->kv_heads;
  p.rel_extent = a->rel_extent;
  p.rel_width = a->rel_width;
  // any window of 2^30 keys or more covers every sequence (rows stay below 2^31
  // bytes / 256-byte rows): clamped so that index arithmetic on it stays in int32
  p.window_left = a->window_left < (1 << 30) ? a->window_left : (1 << 30);
  p.causal = a->causal;
  p.bottom_right = (a->flags & IFA4_FLAG_BOTTOM_RIGHT) ? 1 : 0;
  p.no_prune = (a->flags & IFA4_FLAG_NO_PRUNE) ? 1 : 0;
  p.rel_dtype = a->rel_dtype;
  const int bq = ifa4::prefill_block_q();
  p.n_qtiles = (a->max_seqlen_q + bq - 1) / bq;
  p.scale_log2 = a->softmax_scale * kLog2eHost;
  p.chunk_tiles = 0;
  p.n_chunks = 1;
  return p;
}

// Split-KV plan of a prefill call and the workspace it needs: partial O
// [n_chunks][n_heads][total_q][head_dim] fp32, then their LSEs, 256-byte aligned.
struct PrefillWorkspace {
  ifa4::PrefillSplit split;
  int64_t o_bytes, lse_bytes;
  int64_t total() const { return split.chunk_tiles > 0 ? o_bytes + lse_bytes : 0; }
};
PrefillWorkspace prefill_workspace(const ifa4_args* a) {
  PrefillWorkspace w;
  const bool bottom_right = (a->flags & IFA4_FLAG_BOTTOM_RIGHT) != 0;
  // bottom-right masks see the last max_seqlen_q keys' positions: estimate with
  // the full key range visible (causal off), which only shifts the heuristic
  w.split = ifa4::prefill_split_for(a->batch, a->n_heads, a->max_seqlen_q, a->max_seqlen_k,
                                    a->causal != 0 && !bottom_right,
                                    bottom_right ? -1 : a->window_left, ifa4::prefill_block_q(),
                                    ifa4::prefill_block_k(),
                                    (a->flags & IFA4_FLAG_SPLIT_KV_2) ? 2 : 0);
  const int64_t rows = (int64_t)w.split.n_chunks * a->n_heads * a->total_q;
  w.o_bytes = (rows * a->head_dim * 4 + 255) / 256 * 256;
  w.lse_bytes = (rows * 4 + 255) / 256 * 256;
  return w;
}

// Top-left causal decode (Lq = 1) sees key 0 only.
bool key0_only(const ifa4_args* a) {
  return a->causal != 0 && (a->flags & IFA4_FLAG_BOTTOM_RIGHT) == 0;
}

// The kv heads and group the decode kernels see: the call's own, or pairs of
// adjacent kv heads of an fp8 cache (ifa4::decode_pairs).
struct DecodeView {
  int64_t kv_heads, group;
  bool pair;
};
DecodeView decode_view(const ifa4_args* a, bool fp8) {
  DecodeView v{a->kv_heads, a->n_heads / a->kv_heads, false};
  if (ifa4::decode_pairs(fp8, a->head_dim, v.kv_heads, v.group, a->k_stride_h, a->v_stride_h)) {
    v.kv_heads /= 2;
    v.group *= 2;
    v.pair = true;
  }
  return v;
}

int32_t decode_waves(const ifa4_args* a, bool fp8 = false, bool paged = false) {
  const DecodeView v = decode_view(a, fp8);
  return ifa4::decode_waves_for(a->batch, v.kv_heads, a->max_seqlen_k, key0_only(a), fp8, paged,
                                v.pair);
}

// Decode workspace: partial (o, lse) slots, one per (segment, wave) pair that
// can exist (batch * kv_heads + waves, in the kernels' view of the kv heads),
// then the per-segment wave ranges.
struct DecodeLayout {
  int64_t slots, o_bytes, lse_bytes, meta_bytes;
  int64_t total() const { return o_bytes + lse_bytes + meta_bytes; }
};
DecodeLayout decode_layout(const ifa4_args* a, bool fp8 = false, bool paged = false) {
  DecodeLayout l;
  const DecodeView v = decode_view(a, fp8);
  const int64_t segs = (int64_t)a->batch * v.kv_heads;
  const int64_t group = v.group;
  l.slots = segs + decode_waves(a, fp8, paged);
  l.o_bytes = (l.slots * group * a->head_dim * 4 + 255) / 256 * 256;
  l.lse_bytes = (l.slots * group * 4 + 255) / 256 * 256;
  l.meta_bytes = segs * 2 * 4;
  return l;
}

// Quantised K/V description (include/ifa4.h, ifa4_kv_quant).
int32_t check_quant(const ifa4_kv_quant* qt) {
  if (qt->struct_size != sizeof(ifa4_kv_quant)) return IFA4_EINVAL;
  if (qt->kv_dtype != IFA4_FP8_E4M3) return IFA4_EUNSUPPORTED;
  if (!std::isfinite(qt->k_scale) || !std::isfinite(qt->v_scale) || !(qt->k_scale > 0.f) ||
      !(qt->v_scale > 0.f))
    return IFA4_EINVAL;
  return IFA4_OK;
}

int32_t check_decode(const ifa4_args* a, const ifa4_paged_kv* kv = nullptr,
                     const ifa4_kv_quant* qt = nullptr) {
  int32_t st = IFA4_OK;
  if (qt != nullptr && (st = check_quant(qt)) != IFA4_OK) return st;
  const int esize = qt != nullptr ? 1 : 2;
  if ((st = check_args(a, kv, esize)) != IFA4_OK) return st;
  if ((st = check_head_spans(a)) != IFA4_OK) return st;
  if (kv != nullptr && (st = check_paged(a, kv, esize)) != IFA4_OK) return st;
  if (qt != nullptr && a->n_heads / a->kv_heads > ifa4::decode_fp8_max_group())
    return IFA4_EUNSUPPORTED;
  if (a->batch > 0 && a->total_q != a->batch) return IFA4_EINVAL;  // one query per sequence
  if (a->n_heads / a->kv_heads > ifa4::decode_max_group()) return IFA4_EUNSUPPORTED;
  return IFA4_OK;
}

int32_t run_decode(const ifa4_args* args, const ifa4_paged_kv* kv, const ifa4_kv_quant* qt,
                   void* workspace, size_t workspace_bytes, void* stream) {
  const int32_t st = check_decode(args, kv, qt);
  if (st != IFA4_OK) return st;
  if (args->batch == 0) return IFA4_OK;
  const DecodeLayout lay = decode_layout(args, qt != nullptr, kv != nullptr);
  if (workspace == nullptr || workspace_bytes < (size_t)lay.total() || !aligned(workspace, 256))
    return IFA4_EWORKSPACE;

  ifa4::DecodeParams p{};
  p.q = args->q;
  p.k = args->k;
  p.v = args->v;
  p.rel = args->rel;
  p.out = args->out;
  p.lse = args->lse;
  p.cu_q = args->cu_seqlens_q;
  p.cu_k = kv == nullptr ? args->cu_seqlens_k : nullptr;
  p.ws_o = static_cast<float*>(workspace);
  p.ws_lse = reinterpret_cast<float*>(static_cast<char*>(workspace) + lay.o_bytes);
  p.ws_meta = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + lay.o_bytes +
                                         lay.lse_bytes);
  p.q_st = args->q_stride_t;
  p.q_sh = args->q_stride_h;
  const DecodeView view = decode_view(args, qt != nullptr);
  p.k_st = args->k_stride_t;
  p.k_sh = args->k_stride_h * (view.pair ? 2 : 1);
  p.v_st = args->v_stride_t;
  p.v_sh = args->v_stride_h * (view.pair ? 2 : 1);
  p.rel_st = args->rel_stride_t;
  p.rel_sh = args->rel_stride_h;
  p.o_st = args->out_stride_t;
  p.o_sh = args->out_stride_h;
  p.lse_sh = args->lse_stride_h;
  p.total_q = clamp_rows(args->total_q);
  p.total_k = clamp_rows(args->total_k);
  p.batch = args->batch;
  p.n_heads = args->n_heads;
  p.kv_heads = (int32_t)view.kv_heads;
  p.group = (int32_t)view.group;
  p.kv_pair = view.pair ? 1 : 0;
  p.rel_extent = args->rel_extent;
  p.causal = args->causal;
  p.bottom_right = (args->flags & IFA4_FLAG_BOTTOM_RIGHT) ? 1 : 0;
  p.window_left = args->window_left < (1 << 30) ? args->window_left : (1 << 30);
  p.rel_dtype = args->rel_dtype;
  p.n_waves = decode_waves(args, qt != nullptr, kv != nullptr);
  p.kv_fp8 = qt != nullptr ? 1 : 0;
  p.scale_log2 = args->softmax_scale * (qt != nullptr ? qt->k_scale : 1.f) * kLog2eHost;
  p.v_scale = qt != nullptr ? qt->v_scale : 1.f;
  if (kv != nullptr) {
    p.block_table = kv->block_table;
    p.seqused_k = kv->seqused_k;
    p.bt_stride = kv->block_table_stride;
    p.k_sblk = kv->k_stride_block;
    p.v_sblk = kv->v_stride_block;
    p.block_shift = __builtin_ctz((unsigned)kv->block_size);
    p.num_blocks = kv->num_blocks;
    p.max_blocks = kv->max_blocks_per_seq;
  }
  const hipError_t e = ifa4::launch_decode(p, args->head_dim, args->qkv_dtype,
                                           static_cast<hipStream_t>(stream));
  return e == hipSuccess ? IFA4_OK : IFA4_ELAUNCH;
}

}  // namespace

namespace ifa4 {

int32_t decode_workspace_need(const ifa4_args* args, size_t* bytes) {
  const int32_t st = check_decode(args);
  *bytes = st == IFA4_OK && args->batch > 0 ? (size_t)decode_layout(args).total() : 0;
  return st;
}

int32_t decode_run(const ifa4_args* args, void* workspace, size_t workspace_bytes, void* stream) {
  return run_decode(args, nullptr, nullptr, workspace, workspace_bytes, stream);
}

}  // namespace ifa4

extern "C" {

const char* ifa4_status_str(int32_t status) {
  switch (status) {
    case IFA4_OK: return "IFA4_OK";
    case IFA4_EINVAL: return "IFA4_EINVAL: invalid argument";
    case IFA4_EUNSUPPORTED: return "IFA4_EUNSUPPORTED: argument combination not supported";
    case IFA4_EWORKSPACE: return "IFA4_EWORKSPACE: workspace missing or too small";
    case IFA4_ELAUNCH: return "IFA4_ELAUNCH: kernel launch failed";
    default: return "IFA4: unknown status";
  }
}

int32_t ifa4_abi_version(void) { return IFA4_ABI_VERSION; }

int32_t ifa4_validate(const ifa4_args* args) { return check_args(args); }

int32_t ifa4_prefill_tile(const ifa4_args* args, ifa4_tile* tile) {
  if (args == nullptr || tile == nullptr) return IFA4_EINVAL;
  for (const auto& e : ifa4::kPrefillTiles) {
    if (e.head_dim == args->head_dim) {
      tile->block_q = e.block_q;
      tile->block_k = e.block_k;
      tile->waves = e.waves;
      tile->stages = e.stages;
      // split KV (ifa4_prefill_fwd_ws): keys per chunk, 0 when the call does not split
      const ifa4::PrefillSplit sp = ifa4::prefill_split_for(
          args->batch, args->n_heads, args->max_seqlen_q, args->max_seqlen_k,
          args->causal != 0 && (args->flags & IFA4_FLAG_BOTTOM_RIGHT) == 0,
          (args->flags & IFA4_FLAG_BOTTOM_RIGHT) ? -1 : args->window_left, e.block_q, e.block_k,
          (args->flags & IFA4_FLAG_SPLIT_KV_2) ? 2 : 0);
      tile->kv_chunk = sp.chunk_tiles * e.block_k;
      return IFA4_OK;
    }
  }
  return IFA4_EUNSUPPORTED;
}

int32_t ifa4_prefill_fwd(const ifa4_args* args, void* stream) {
  const int32_t st = check_args(args);
  if (st != IFA4_OK) return st;
  if (args->batch == 0 || args->max_seqlen_q == 0) return IFA4_OK;
  const ifa4::PrefillParams p = make_prefill_params(args);
  const hipError_t e = ifa4::launch_prefill(p, args->head_dim, args->qkv_dtype,
                                            static_cast<hipStream_t>(stream));
  return e == hipSuccess ? IFA4_OK : IFA4_ELAUNCH;
}

size_t ifa4_prefill_workspace_bytes(const ifa4_args* args) {
  if (check_args(args) != IFA4_OK || args->batch == 0 || args->max_seqlen_q == 0) return 0;
  return (size_t)prefill_workspace(args).total();
}

int32_t ifa4_prefill_fwd_ws(const ifa4_args* args, void* workspace, size_t workspace_bytes,
                            void* stream) {
  const int32_t st = check_args(args);
  if (st != IFA4_OK) return st;
  if (args->batch == 0 || args->max_seqlen_q == 0) return IFA4_OK;
  ifa4::PrefillParams p = make_prefill_params(args);
  const PrefillWorkspace w = prefill_workspace(args);
  if (w.total() > 0) {
    if (workspace == nullptr || workspace_bytes < (size_t)w.total() || !aligned(workspace, 256))
      return IFA4_EWORKSPACE;
    p.chunk_tiles = w.split.chunk_tiles;
    p.n_chunks = w.split.n_chunks;
    p.part_o = static_cast<float*>(workspace);
    p.part_lse = reinterpret_cast<float*>(static_cast<char*>(workspace) + w.o_bytes);
  }
  const hipError_t e = ifa4::launch_prefill(p, args->head_dim, args->qkv_dtype,
                                            static_cast<hipStream_t>(stream));
  return e == hipSuccess ? IFA4_OK : IFA4_ELAUNCH;
}

int32_t ifa4_prefill_rproj_fwd(const ifa4_args* args, const ifa4_rel_proj* pr, void* stream) {
  if (args == nullptr || pr == nullptr || pr->struct_size != sizeof(ifa4_rel_proj))
    return IFA4_EINVAL;
  if (pr->d_rel != 16) return IFA4_EUNSUPPORTED;
  if (args->rel_dtype != IFA4_BF16 && args->rel_dtype != IFA4_FP32) return IFA4_EUNSUPPORTED;
  if (pr->r_stride_t < 0 || pr->r_stride_h < 0) return IFA4_EINVAL;
  // The rel arguments of ifa4_args describe r here: checked below, not by check_args.
  ifa4_args b = *args;
  b.rel = pr->r;
  b.rel_stride_t = 0;
  b.rel_stride_h = 0;
  const int32_t st = check_args(&b);
  if (st != IFA4_OK) return st;
  if (args->batch == 0 || args->max_seqlen_q == 0) return IFA4_OK;
  if (args->rel_extent > 0) {
    const int64_t esize = args->rel_dtype == IFA4_FP32 ? 4 : 2;
    if (pr->r == nullptr || pr->wt == nullptr || !aligned(pr->r, esize) || !aligned(pr->wt, 16))
      return IFA4_EINVAL;
    if (pr->r_stride_t != 0 && pr->r_stride_t < 16) return IFA4_EUNSUPPORTED;
    if (((int64_t)args->max_seqlen_q + ifa4::prefill_proj_block_q()) * pr->r_stride_t * esize >=
            (int64_t(1) << 31) ||
        (int64_t)args->rel_width * 64 >= (int64_t(1) << 31))
      return IFA4_EUNSUPPORTED;
  }
  ifa4::PrefillParams p = make_prefill_params(&b);
  p.rel = pr->r;
  p.rel_st = pr->r_stride_t;
  p.rel_sh = pr->r_stride_h;
  p.wt = args->rel_extent > 0 ? pr->wt : nullptr;  // no bias at all: the plain kernel
  if (p.wt != nullptr) {
    const int bq = ifa4::prefill_proj_block_q();
    p.n_qtiles = (args->max_seqlen_q + bq - 1) / bq;
  }
  const hipError_t e = ifa4::launch_prefill(p, args->head_dim, args->qkv_dtype,
                                            static_cast<hipStream_t>(stream));
  return e == hipSuccess ? IFA4_OK : IFA4_ELAUNCH;
}

int32_t ifa4_prefill_count_tiles(const ifa4_args* args, const int32_t* cu_q, const int32_t* cu_k,
                                 int64_t* visited, int64_t* total) {
  if (args == nullptr || cu_q == nullptr || cu_k == nullptr || visited == nullptr ||
      total == nullptr)
    return IFA4_EINVAL;
  if (args->batch < 0 || args->n_heads < 1) return IFA4_EINVAL;
  const int bq = ifa4::prefill_block_q();
  const int bk = ifa4::prefill_block_k();
  const bool no_prune = (args->flags & IFA4_FLAG_NO_PRUNE) != 0;
  const bool bottom_right = (args->flags & IFA4_FLAG_BOTTOM_RIGHT) != 0;
  int64_t vis = 0, tot = 0;
  for (int b = 0; b < args->batch; ++b) {
    const int lq = cu_q[b + 1] - cu_q[b];
    const int lk = cu_k[b + 1] - cu_k[b];
    if (lq < 0 || lk < 0) return IFA4_EINVAL;
    const int qpos = bottom_right ? lk - lq : 0;  // key position of query 0
    for (int q0 = 0; q0 < lq; q0 += bq) {
      const int q_hi = q0 + bq < lq ? q0 + bq : lq;
      int kend = lk, kbeg = 0;
      if (!no_prune) {
        if (args->causal) kend = kend < q_hi + qpos ? kend : q_hi + qpos;
        if (args->window_left >= 0) {
          const int lo = q0 + qpos - args->window_left;
          kbeg = lo > 0 ? lo : 0;
        }
      }
      const int kt_beg = kbeg / bk;
      const int kt_end = kend > kbeg ? (kend + bk - 1) / bk : kt_beg;
      vis += (int64_t)(kt_end - kt_beg) * args->n_heads;
      tot += (int64_t)((lk + bk - 1) / bk) * args->n_heads;
    }
  }
  *visited = vis;
  *total = tot;
  return IFA4_OK;
}

size_t ifa4_decode_workspace_bytes(const ifa4_args* args) {
  if (check_decode(args) != IFA4_OK) return 0;
  return (size_t)decode_layout(args).total();
}

int32_t ifa4_decode_tile(const ifa4_args* args, ifa4_tile* tile) {
  if (tile == nullptr) return IFA4_EINVAL;
  const int32_t st = check_decode(args);
  if (st != IFA4_OK) return st;
  // One wave per workgroup, 32-key steps, two register stages; kv_chunk = the
  // most keys one persistent wave streams (ceil(steps / waves) steps).
  tile->block_q = 1;
  tile->block_k = ifa4::kDecodeStep;
  tile->waves = 1;
  tile->stages = 2;
  const int64_t steps = ifa4::decode_max_steps(args->batch, args->kv_heads, args->max_seqlen_k,
                                               key0_only(args));
  const int32_t w = decode_waves(args);
  tile->kv_chunk = w > 0 ? (int32_t)(((steps + w - 1) / w) * ifa4::kDecodeStep) : 0;
  return IFA4_OK;
}

int32_t ifa4_decode_fwd(const ifa4_args* args, void* workspace, size_t workspace_bytes,
                        void* stream) {
  return run_decode(args, nullptr, nullptr, workspace, workspace_bytes, stream);
}

size_t ifa4_decode_paged_workspace_bytes(const ifa4_args* args, const ifa4_paged_kv* kv) {
  if (check_decode(args, kv) != IFA4_OK) return 0;
  return (size_t)decode_layout(args, false, true).total();
}

int32_t ifa4_decode_paged_fwd(const ifa4_args* args, const ifa4_paged_kv* kv, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (kv == nullptr) return IFA4_EINVAL;
  return run_decode(args, kv, nullptr, workspace, workspace_bytes, stream);
}

size_t ifa4_decode_quant_workspace_bytes(const ifa4_args* args, const ifa4_paged_kv* kv,
                                         const ifa4_kv_quant* quant) {
  if (quant == nullptr || check_decode(args, kv, quant) != IFA4_OK) return 0;
  return (size_t)decode_layout(args, true, kv != nullptr).total();
}

int32_t ifa4_decode_quant_fwd(const ifa4_args* args, const ifa4_paged_kv* kv,
                              const ifa4_kv_quant* quant, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (quant == nullptr) return IFA4_EINVAL;
  return run_decode(args, kv, quant, workspace, workspace_bytes, stream);
}

}  // extern "C"
