// Torch extension over the C ABI of libpkv_decode.so: the reference's own
// binding (scripts/evaluate_flashattn_submission.py:24-86, BINDING_CPP:
// `run_kernel` taking tensors and the 15 reference arguments), and a
// stream-aware decode in the shape of flash_attn_with_kvcache's core
// (eval:232-247): it allocates `out` and the workspace from torch's caching
// allocator and runs on torch's current stream.  Errors raise instead of
// being dropped.  Built in-tree by pagedkv.build.build_torch_binding().

#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <cmath>
#include <cstdint>

#include "pkv_decode.h"

namespace {

void check_status(int st, const char* what) {
    TORCH_CHECK(st == PKV_OK, what, ": ", pkv_strerror(st), " (status ", st, ")");
}

// The reference binding's run_kernel_torch: same arguments, same meaning
// (bf16 tensors, scale 1/sqrt(headdim), heuristic splits, null stream).
void run_kernel_torch(torch::Tensor q, torch::Tensor k_cache_paged, torch::Tensor v_cache_paged,
                      torch::Tensor output, torch::Tensor cache_seqlens, torch::Tensor block_table,
                      int64_t batch_size, int64_t seqlen_k, int64_t seqlen_q, int64_t num_heads,
                      int64_t num_heads_k, int64_t headdim, int64_t page_block_size, int64_t num_blocks,
                      int64_t causal) {
    TORCH_CHECK(cache_seqlens.scalar_type() == torch::kInt32 && block_table.scalar_type() == torch::kInt32,
                "run_kernel: cache_seqlens and block_table must be int32");
    run_kernel(q.data_ptr(), k_cache_paged.data_ptr(), v_cache_paged.data_ptr(), output.data_ptr(),
               cache_seqlens.data_ptr<int32_t>(), block_table.data_ptr<int32_t>(), batch_size, seqlen_k, seqlen_q,
               num_heads, num_heads_k, headdim, page_block_size, num_blocks, causal);
    check_status(pkv_last_status(), "run_kernel");
}

// out = decode attention of q [B, M, H, D] over the paged caches
// [num_pages, P, Hk, D] (fp16 / bf16 like q), block_table int32 [B, stride],
// cache_seqlens int32 [B]; causal = flash-attn's bottom-right mask for M > 1.
torch::Tensor decode(torch::Tensor q, torch::Tensor k_cache, torch::Tensor v_cache, torch::Tensor cache_seqlens,
                     torch::Tensor block_table, double softmax_scale, int64_t num_splits, bool causal,
                     int64_t max_seqlen) {
    TORCH_CHECK(q.is_cuda() && k_cache.is_cuda() && v_cache.is_cuda() && cache_seqlens.is_cuda() &&
                    block_table.is_cuda(),
                "decode: all tensors must be on the GPU");
    TORCH_CHECK(q.dim() == 4 && k_cache.dim() == 4 && v_cache.dim() == 4, "decode: q [B, M, H, D], caches [N, P, Hk, D]");
    TORCH_CHECK(q.is_contiguous() && k_cache.is_contiguous() && v_cache.is_contiguous() &&
                    cache_seqlens.is_contiguous() && block_table.is_contiguous(),
                "decode: tensors must be contiguous");
    TORCH_CHECK(q.scalar_type() == torch::kBFloat16 || q.scalar_type() == torch::kFloat16,
                "decode: q must be bf16 or fp16");
    TORCH_CHECK(k_cache.scalar_type() == q.scalar_type() && v_cache.scalar_type() == q.scalar_type(),
                "decode: caches must have q's dtype");
    TORCH_CHECK(k_cache.sizes() == v_cache.sizes(), "decode: k_cache and v_cache shapes differ");
    TORCH_CHECK(cache_seqlens.scalar_type() == torch::kInt32 && block_table.scalar_type() == torch::kInt32,
                "decode: cache_seqlens and block_table must be int32");
    TORCH_CHECK(block_table.dim() == 2 && cache_seqlens.dim() == 1, "decode: block_table [B, stride], cache_seqlens [B]");
    TORCH_CHECK(q.size(3) == k_cache.size(3), "decode: q and caches disagree on head_dim");
    TORCH_CHECK(block_table.size(0) == q.size(0) && cache_seqlens.size(0) == q.size(0),
                "decode: batch sizes disagree");

    const c10::DeviceGuard guard(q.device());
    pkv_decode_desc d{};
    d.batch = q.size(0);
    d.seqlen_q = q.size(1);
    d.num_heads = q.size(2);
    d.head_dim = q.size(3);
    d.num_pages = k_cache.size(0);
    d.page_size = k_cache.size(1);
    d.num_heads_k = k_cache.size(2);
    d.block_table_stride = block_table.size(1);
    d.max_seqlen = max_seqlen;
    d.dtype = q.scalar_type() == torch::kBFloat16 ? PKV_DTYPE_BF16 : PKV_DTYPE_F16;
    d.path = PKV_PATH_AUTO;
    d.mask = causal ? PKV_MASK_CAUSAL : 0;
    const int splits = static_cast<int>(num_splits);
    const size_t ws_bytes = pkv_decode_workspace_size(&d, splits);
    torch::Tensor ws;
    if (ws_bytes > 0) {
        ws = torch::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(torch::kUInt8));
        d.workspace = ws.data_ptr();
        d.workspace_bytes = ws_bytes;
    }
    torch::Tensor out = torch::empty_like(q);
    const float scale = softmax_scale > 0 ? static_cast<float>(softmax_scale)
                                          : 1.0f / std::sqrt(static_cast<float>(d.head_dim));
    hipStream_t stream = c10::hip::getCurrentHIPStream(q.device().index()).stream();
    check_status(pkv_decode(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr<int32_t>(),
                            cache_seqlens.data_ptr<int32_t>(), scale, splits, out.data_ptr(), &d, stream),
                 "pkv_decode");
    return out;
}

} // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("run_kernel", &run_kernel_torch, "the reference's 15-argument run_kernel over libpkv_decode.so");
    m.def("decode", &decode, "paged-KV decode attention on torch's current stream", py::arg("q"),
          py::arg("k_cache"), py::arg("v_cache"), py::arg("cache_seqlens"), py::arg("block_table"),
          py::arg("softmax_scale") = 0.0, py::arg("num_splits") = 0, py::arg("causal") = false,
          py::arg("max_seqlen") = 0);
}
