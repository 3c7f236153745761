// Thin PyTorch-ROCm binding over the C ABI (include/ifa4.h).
//
// Registers torch.ops.inkling_fa4.fwd / .fwd_rproj / .decode / .decode_paged.  The binding checks tensor
// devices, dtypes and shapes, allocates out / lse / the decode workspace from
// torch's caching allocator, fills an ifa4_args and calls the library on the
// current HIP stream.  No math happens here, and there is no fallback: a
// status other than IFA4_OK raises.
//
// Mirrors the wrapper signature of inkling_fa4_rel_attention_triton
// (src/inkling_fa4/triton_kernel.py:84-107); the Python layer (inkling_fa4.ops)
// keeps the positional API and adds softmax_scale / return_lse.
#include <ATen/ATen.h>
#include <torch/library.h>
#include <c10/hip/HIPStream.h>

#include <tuple>

#include "ifa4.h"

namespace {

int32_t dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kBFloat16: return IFA4_BF16;
    case at::kHalf: return IFA4_FP16;
    case at::kFloat: return IFA4_FP32;
    default: return -1;
  }
}

void check_status(int32_t st, const char* what) {
  TORCH_CHECK(st == IFA4_OK, "inkling_fa4.", what, ": ", ifa4_status_str(st));
}

ifa4_args make_args(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                    const at::Tensor& rel, const at::Tensor& cu_q, const at::Tensor& cu_k,
                    int64_t max_q, int64_t max_k, int64_t rel_extent, bool causal,
                    int64_t window_left, double softmax_scale, int64_t flags) {
  TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda() && rel.is_cuda() && cu_q.is_cuda() &&
                  cu_k.is_cuda(),
              "inkling_fa4: every tensor must be on the GPU");
  const auto dev = q.device();
  TORCH_CHECK(k.device() == dev && v.device() == dev && rel.device() == dev &&
                  cu_q.device() == dev && cu_k.device() == dev,
              "inkling_fa4: tensors must be on one device");
  TORCH_CHECK(q.dim() == 3 && k.dim() == 3 && v.dim() == 3 && rel.dim() == 3,
              "inkling_fa4: q, k, v, rel_logits must be 3-D [tokens, heads, dim]");
  TORCH_CHECK(k.sizes() == v.sizes(), "inkling_fa4: k and v shapes differ");
  TORCH_CHECK(q.size(2) == k.size(2), "inkling_fa4: q and k head_dim differ");
  TORCH_CHECK(rel.size(0) == q.size(0) && rel.size(1) == q.size(1),
              "inkling_fa4: rel_logits must be [total_q, n_heads, >= rel_extent]");
  const bool kv_fp8 = k.scalar_type() == at::kFloat8_e4m3fn;
  TORCH_CHECK(k.scalar_type() == v.scalar_type() && (kv_fp8 || q.scalar_type() == k.scalar_type()),
              "inkling_fa4: q, k, v dtypes differ (k/v may both be float8_e4m3fn in decode)");
  TORCH_CHECK(q.stride(2) == 1 && k.stride(2) == 1 && v.stride(2) == 1 && rel.stride(2) == 1,
              "inkling_fa4: the last dim of q, k, v, rel_logits must be contiguous");
  TORCH_CHECK(cu_q.scalar_type() == at::kInt && cu_k.scalar_type() == at::kInt,
              "inkling_fa4: cu_seqlens must be int32");
  TORCH_CHECK(cu_q.dim() == 1 && cu_k.dim() == 1 && cu_q.numel() == cu_k.numel() &&
                  cu_q.numel() >= 1,
              "inkling_fa4: cu_seqlens_q/k must be 1-D of equal length batch+1");
  TORCH_CHECK(cu_q.is_contiguous() && cu_k.is_contiguous(),
              "inkling_fa4: cu_seqlens must be contiguous");
  const int32_t qd = dtype_code(q.scalar_type());
  const int32_t rd = dtype_code(rel.scalar_type());
  TORCH_CHECK(qd == IFA4_BF16 || qd == IFA4_FP16, "inkling_fa4: q/k/v must be bf16 or fp16");
  TORCH_CHECK(rd >= 0, "inkling_fa4: rel_logits must be bf16, fp16 or fp32");

  ifa4_args a{};
  a.struct_size = sizeof(ifa4_args);
  a.flags = static_cast<uint32_t>(flags);
  a.q = q.data_ptr();
  a.k = k.data_ptr();
  a.v = v.data_ptr();
  a.rel = rel.data_ptr();
  a.cu_seqlens_q = cu_q.data_ptr<int32_t>();
  a.cu_seqlens_k = cu_k.data_ptr<int32_t>();
  a.q_stride_t = q.stride(0);
  a.q_stride_h = q.stride(1);
  a.k_stride_t = k.stride(0);
  a.k_stride_h = k.stride(1);
  a.v_stride_t = v.stride(0);
  a.v_stride_h = v.stride(1);
  a.rel_stride_t = rel.stride(0);
  a.rel_stride_h = rel.stride(1);
  a.total_q = q.size(0);
  a.total_k = k.size(0);
  a.batch = static_cast<int32_t>(cu_q.numel() - 1);
  a.n_heads = static_cast<int32_t>(q.size(1));
  a.kv_heads = static_cast<int32_t>(k.size(1));
  a.head_dim = static_cast<int32_t>(q.size(2));
  a.rel_extent = static_cast<int32_t>(rel_extent);
  a.rel_width = static_cast<int32_t>(rel.size(2));
  a.max_seqlen_q = static_cast<int32_t>(max_q);
  a.max_seqlen_k = static_cast<int32_t>(max_k);
  a.window_left = window_left < 0 ? -1 : static_cast<int32_t>(window_left);
  a.causal = causal ? 1 : 0;
  a.softmax_scale = static_cast<float>(softmax_scale);
  a.qkv_dtype = qd;
  a.rel_dtype = rd;
  return a;
}

// fp8 K/V (decode only): the per-tensor scales as an ifa4_kv_quant.
ifa4_kv_quant kv_quant(double k_scale, double v_scale) {
  ifa4_kv_quant qt{};
  qt.struct_size = sizeof(ifa4_kv_quant);
  qt.kv_dtype = IFA4_FP8_E4M3;
  qt.k_scale = static_cast<float>(k_scale);
  qt.v_scale = static_cast<float>(v_scale);
  return qt;
}

std::tuple<at::Tensor, at::Tensor> fwd(const at::Tensor& q, const at::Tensor& k,
                                       const at::Tensor& v, const at::Tensor& rel,
                                       const at::Tensor& cu_q, const at::Tensor& cu_k,
                                       int64_t max_q, int64_t max_k, int64_t rel_extent,
                                       bool causal, int64_t window_left, double softmax_scale,
                                       bool return_lse, int64_t flags) {
  TORCH_CHECK(k.scalar_type() != at::kFloat8_e4m3fn,
              "inkling_fa4.fwd: fp8 K/V is supported by decode only");
  ifa4_args a = make_args(q, k, v, rel, cu_q, cu_k, max_q, max_k, rel_extent, causal,
                          window_left, softmax_scale, flags);
  at::Tensor out = at::empty_like(q, q.options().memory_format(at::MemoryFormat::Contiguous));
  at::Tensor lse = return_lse ? at::empty({q.size(1), q.size(0)}, q.options().dtype(at::kFloat))
                              : at::empty({0}, q.options().dtype(at::kFloat));
  a.out = out.data_ptr();
  a.out_stride_t = out.stride(0);
  a.out_stride_h = out.stride(1);
  if (return_lse) {
    a.lse = lse.data_ptr<float>();
    a.lse_stride_h = lse.stride(0);
  }
  check_status(ifa4_validate(&a), "fwd");
  const hipStream_t stream = c10::hip::getCurrentHIPStream(q.device().index()).stream();
  // split-KV workspace when the tile table splits this call (0 bytes otherwise)
  const size_t ws_bytes = ifa4_prefill_workspace_bytes(&a);
  at::Tensor ws = ws_bytes > 0 ? at::empty({(int64_t)ws_bytes}, q.options().dtype(at::kByte))
                               : at::Tensor();
  check_status(ifa4_prefill_fwd_ws(&a, ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes, stream),
               "fwd");
  return {out, lse};
}

// Prefill with the fused relative-logit projection: r [Tq, Hq, 16] (bf16 or
// fp32), wt = W^T [R', 16] fp32 contiguous.
std::tuple<at::Tensor, at::Tensor> fwd_rproj(const at::Tensor& q, const at::Tensor& k,
                                             const at::Tensor& v, const at::Tensor& r,
                                             const at::Tensor& wt, const at::Tensor& cu_q,
                                             const at::Tensor& cu_k, int64_t max_q, int64_t max_k,
                                             int64_t rel_extent, bool causal, int64_t window_left,
                                             double softmax_scale, bool return_lse,
                                             int64_t flags) {
  TORCH_CHECK(r.dim() == 3 && r.size(0) == q.size(0) && r.size(1) == q.size(1) &&
                  r.size(2) == 16 && r.stride(2) == 1,
              "inkling_fa4.fwd_rproj: r must be [total_q, n_heads, 16] with a contiguous last dim");
  TORCH_CHECK(wt.dim() == 2 && wt.size(1) == 16 && wt.is_contiguous() &&
                  wt.scalar_type() == at::kFloat,
              "inkling_fa4.fwd_rproj: wt must be W^T [R', 16] fp32, contiguous");
  TORCH_CHECK(r.scalar_type() == at::kFloat || r.scalar_type() == at::kBFloat16,
              "inkling_fa4.fwd_rproj: r must be fp32 or bf16");
  TORCH_CHECK(wt.is_cuda() && wt.device() == q.device(), "inkling_fa4.fwd_rproj: wt on q's GPU");
  // make_args checks r in the rel slot: a [total_q, n_heads, 16] view passes
  ifa4_args a = make_args(q, k, v, r, cu_q, cu_k, max_q, max_k, rel_extent, causal, window_left,
                          softmax_scale, flags);
  a.rel_width = static_cast<int32_t>(wt.size(0));
  ifa4_rel_proj pr{};
  pr.struct_size = sizeof(ifa4_rel_proj);
  pr.d_rel = 16;
  pr.r = r.data_ptr();
  pr.r_stride_t = r.stride(0);
  pr.r_stride_h = r.stride(1);
  pr.wt = wt.data_ptr<float>();
  at::Tensor out = at::empty_like(q, q.options().memory_format(at::MemoryFormat::Contiguous));
  at::Tensor lse = return_lse ? at::empty({q.size(1), q.size(0)}, q.options().dtype(at::kFloat))
                              : at::empty({0}, q.options().dtype(at::kFloat));
  a.out = out.data_ptr();
  a.out_stride_t = out.stride(0);
  a.out_stride_h = out.stride(1);
  if (return_lse) {
    a.lse = lse.data_ptr<float>();
    a.lse_stride_h = lse.stride(0);
  }
  const hipStream_t stream = c10::hip::getCurrentHIPStream(q.device().index()).stream();
  check_status(ifa4_prefill_rproj_fwd(&a, &pr, stream), "fwd_rproj");
  return {out, lse};
}

std::tuple<at::Tensor, at::Tensor> decode(const at::Tensor& q, const at::Tensor& k,
                                          const at::Tensor& v, const at::Tensor& rel,
                                          const at::Tensor& cu_q, const at::Tensor& cu_k,
                                          int64_t max_q, int64_t max_k, int64_t rel_extent,
                                          bool causal, int64_t window_left,
                                          double softmax_scale, bool return_lse,
                                          int64_t flags, double k_scale, double v_scale) {
  ifa4_args a = make_args(q, k, v, rel, cu_q, cu_k, max_q, max_k, rel_extent, causal,
                          window_left, softmax_scale, flags);
  at::Tensor out = at::empty_like(q, q.options().memory_format(at::MemoryFormat::Contiguous));
  at::Tensor lse = return_lse ? at::empty({q.size(1), q.size(0)}, q.options().dtype(at::kFloat))
                              : at::empty({0}, q.options().dtype(at::kFloat));
  a.out = out.data_ptr();
  a.out_stride_t = out.stride(0);
  a.out_stride_h = out.stride(1);
  if (return_lse) {
    a.lse = lse.data_ptr<float>();
    a.lse_stride_h = lse.stride(0);
  }
  const bool kv_fp8 = k.scalar_type() == at::kFloat8_e4m3fn;
  const ifa4_kv_quant qt = kv_quant(k_scale, v_scale);
  if (!kv_fp8) check_status(ifa4_validate(&a), "decode");
  const size_t ws_bytes = kv_fp8 ? ifa4_decode_quant_workspace_bytes(&a, nullptr, &qt)
                                 : ifa4_decode_workspace_bytes(&a);
  if (ws_bytes == 0 && a.batch > 0)  // invalid arguments: the call reports which status
    check_status(kv_fp8 ? ifa4_decode_quant_fwd(&a, nullptr, &qt, nullptr, 0, nullptr)
                        : ifa4_decode_fwd(&a, nullptr, 0, nullptr),
                 "decode");
  at::Tensor ws = at::empty({static_cast<int64_t>(ws_bytes) + 256}, q.options().dtype(at::kByte));
  const uintptr_t base = reinterpret_cast<uintptr_t>(ws.data_ptr());
  void* aligned_ws = reinterpret_cast<void*>((base + 255) / 256 * 256);
  const hipStream_t stream = c10::hip::getCurrentHIPStream(q.device().index()).stream();
  check_status(kv_fp8 ? ifa4_decode_quant_fwd(&a, nullptr, &qt, aligned_ws, ws_bytes, stream)
                      : ifa4_decode_fwd(&a, aligned_ws, ws_bytes, stream),
               "decode");
  return {out, lse};
}

// Decode over a paged KV cache: k_cache / v_cache [num_blocks, block_size,
// kv_heads, head_dim], block_table int32 [batch, max_blocks_per_seq],
// seqused_k int32 [batch].  Same outputs as decode().
std::tuple<at::Tensor, at::Tensor> decode_paged(
    const at::Tensor& q, const at::Tensor& k_cache, const at::Tensor& v_cache,
    const at::Tensor& rel, const at::Tensor& cu_q, const at::Tensor& seqused_k,
    const at::Tensor& block_table, int64_t max_q, int64_t max_k, int64_t rel_extent, bool causal,
    int64_t window_left, double softmax_scale, bool return_lse, int64_t flags, double k_scale,
    double v_scale) {
  TORCH_CHECK(k_cache.dim() == 4 && v_cache.dim() == 4,
              "inkling_fa4.decode_paged: k_cache / v_cache must be "
              "[num_blocks, block_size, kv_heads, head_dim]");
  TORCH_CHECK(k_cache.sizes() == v_cache.sizes(),
              "inkling_fa4.decode_paged: k_cache and v_cache shapes differ");
  TORCH_CHECK(block_table.is_cuda() && seqused_k.is_cuda() &&
                  block_table.device() == q.device() && seqused_k.device() == q.device(),
              "inkling_fa4.decode_paged: block_table / seqused_k must be on q's GPU");
  TORCH_CHECK(block_table.scalar_type() == at::kInt && seqused_k.scalar_type() == at::kInt,
              "inkling_fa4.decode_paged: block_table and seqused_k must be int32");
  TORCH_CHECK(block_table.dim() == 2 && block_table.stride(1) == 1,
              "inkling_fa4.decode_paged: block_table must be 2-D with contiguous rows");
  TORCH_CHECK(seqused_k.dim() == 1 && seqused_k.is_contiguous(),
              "inkling_fa4.decode_paged: seqused_k must be 1-D contiguous");
  TORCH_CHECK(block_table.size(0) == cu_q.numel() - 1 && seqused_k.numel() == cu_q.numel() - 1,
              "inkling_fa4.decode_paged: block_table / seqused_k need one row per sequence");
  // The per-token view [blocks * block_size, kv_heads, head_dim] of the first
  // block carries the row / head strides; block strides travel separately.
  const at::Tensor k_rows = k_cache.select(0, 0);
  const at::Tensor v_rows = v_cache.select(0, 0);
  ifa4_args a = make_args(q, k_rows, v_rows, rel, cu_q, cu_q, max_q, max_k, rel_extent, causal,
                          window_left, softmax_scale, flags);
  a.k = k_cache.data_ptr();
  a.v = v_cache.data_ptr();
  a.cu_seqlens_k = nullptr;
  a.total_k = 0;
  ifa4_paged_kv kv{};
  kv.struct_size = sizeof(ifa4_paged_kv);
  kv.block_size = static_cast<int32_t>(k_cache.size(1));
  kv.block_table = block_table.data_ptr<int32_t>();
  kv.seqused_k = seqused_k.data_ptr<int32_t>();
  kv.block_table_stride = block_table.stride(0);
  kv.k_stride_block = k_cache.stride(0);
  kv.v_stride_block = v_cache.stride(0);
  kv.num_blocks = static_cast<int32_t>(k_cache.size(0));
  kv.max_blocks_per_seq = static_cast<int32_t>(block_table.size(1));

  at::Tensor out = at::empty_like(q, q.options().memory_format(at::MemoryFormat::Contiguous));
  at::Tensor lse = return_lse ? at::empty({q.size(1), q.size(0)}, q.options().dtype(at::kFloat))
                              : at::empty({0}, q.options().dtype(at::kFloat));
  a.out = out.data_ptr();
  a.out_stride_t = out.stride(0);
  a.out_stride_h = out.stride(1);
  if (return_lse) {
    a.lse = lse.data_ptr<float>();
    a.lse_stride_h = lse.stride(0);
  }
  const bool kv_fp8 = k_cache.scalar_type() == at::kFloat8_e4m3fn;
  const ifa4_kv_quant qt = kv_quant(k_scale, v_scale);
  const size_t ws_bytes = kv_fp8 ? ifa4_decode_quant_workspace_bytes(&a, &kv, &qt)
                                 : ifa4_decode_paged_workspace_bytes(&a, &kv);
  if (ws_bytes == 0 && a.batch > 0)  // invalid arguments: the call reports which status
    check_status(kv_fp8 ? ifa4_decode_quant_fwd(&a, &kv, &qt, nullptr, 0, nullptr)
                        : ifa4_decode_paged_fwd(&a, &kv, nullptr, 0, nullptr),
                 "decode_paged");
  at::Tensor ws = at::empty({static_cast<int64_t>(ws_bytes) + 256}, q.options().dtype(at::kByte));
  const uintptr_t base = reinterpret_cast<uintptr_t>(ws.data_ptr());
  void* aligned_ws = reinterpret_cast<void*>((base + 255) / 256 * 256);
  const hipStream_t stream = c10::hip::getCurrentHIPStream(q.device().index()).stream();
  check_status(kv_fp8 ? ifa4_decode_quant_fwd(&a, &kv, &qt, aligned_ws, ws_bytes, stream)
                      : ifa4_decode_paged_fwd(&a, &kv, aligned_ws, ws_bytes, stream),
               "decode_paged");
  return {out, lse};
}

}  // namespace

TORCH_LIBRARY(inkling_fa4, m) {
  m.def(
      "fwd(Tensor q, Tensor k, Tensor v, Tensor rel_logits, Tensor cu_seqlens_q, "
      "Tensor cu_seqlens_k, int max_seqlen_q, int max_seqlen_k, int rel_extent, bool causal, "
      "int window_left, float softmax_scale, bool return_lse, int flags) -> (Tensor, Tensor)");
  m.def(
      "fwd_rproj(Tensor q, Tensor k, Tensor v, Tensor r, Tensor wt, Tensor cu_seqlens_q, "
      "Tensor cu_seqlens_k, int max_seqlen_q, int max_seqlen_k, int rel_extent, bool causal, "
      "int window_left, float softmax_scale, bool return_lse, int flags) -> (Tensor, Tensor)");
  m.def(
      "decode(Tensor q, Tensor k, Tensor v, Tensor rel_logits, Tensor cu_seqlens_q, "
      "Tensor cu_seqlens_k, int max_seqlen_q, int max_seqlen_k, int rel_extent, bool causal, "
      "int window_left, float softmax_scale, bool return_lse, int flags, float k_scale, "
      "float v_scale) -> (Tensor, Tensor)");
  m.def(
      "decode_paged(Tensor q, Tensor k_cache, Tensor v_cache, Tensor rel_logits, "
      "Tensor cu_seqlens_q, Tensor seqused_k, Tensor block_table, int max_seqlen_q, "
      "int max_seqlen_k, int rel_extent, bool causal, int window_left, float softmax_scale, "
      "bool return_lse, int flags, float k_scale, float v_scale) -> (Tensor, Tensor)");
}

TORCH_LIBRARY_IMPL(inkling_fa4, CUDA, m) {
  m.impl("fwd", &fwd);
  m.impl("fwd_rproj", &fwd_rproj);
  m.impl("decode", &decode);
  m.impl("decode_paged", &decode_paged);
}
