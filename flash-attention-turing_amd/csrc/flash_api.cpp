// Host layer: the `flash_attn_turing` Python extension over the C ABI of
// libfa_mi355x.so (include/fa_mi355x.h).
//
// Mirrors the reference's pybind module (csrc/flash_attn/flash_api.cpp:717-724):
// the same five bindings (fwd, bwd, varlen_fwd, varlen_bwd, fwd_kvcache), the
// same argument order, the same TORCH_CHECK conditions and messages, and the
// same [b, h, seqlen_q] / [b, h, max_seqlen_q] LSE layout.  Differences, all
// deliberate:
//   * every kernel runs on the current HIP stream under a device guard (the
//     reference launched fwd/bwd on the legacy default stream);
//   * outputs are allocated with `empty` where the kernels write every element
//     (the reference zero-filled them because early-exit CTAs wrote nothing);
//   * the GQA dK/dV sum is done inside the dK/dV kernel (no expanded
//     per-q-head buffers, no torch::sum_out);
//   * the KV append is one device kernel for contiguous, remapped and paged
//     caches (no host loop over the batch), and the chunked KV path reads the
//     cache through cache_batch_idx in-kernel (no index_select copy);
//   * inputs must be float16 on the GPU; tensors whose strides or base address
//     are not 16-byte aligned are made contiguous before the launch.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <optional>
#include <vector>

#include "fa_mi355x.h"

namespace {

inline void check_supported_head_dim(const int64_t head_size) {
    TORCH_CHECK(head_size == 64 || head_size == 128, "Turing FlashAttention supports head_dim 64 or 128");
}

inline void check_fp16_cuda(const at::Tensor &t, const char *name) {
    TORCH_CHECK(t.is_cuda(), name, " must be a CUDA (HIP) tensor");
    TORCH_CHECK(t.scalar_type() == at::kHalf, name, " must be a float16 tensor");
}

// 16-byte aligned base and strides (in elements, multiple of 8), last dim contiguous.
inline bool is_aligned(const at::Tensor &t) {
    bool ok = t.stride(-1) == 1 && (reinterpret_cast<uintptr_t>(t.data_ptr()) & 15u) == 0;
    for (int64_t i = 0; ok && i + 1 < t.dim(); ++i) ok = (t.stride(i) % 8) == 0 || t.size(i) == 1;
    return ok;
}
// A fresh contiguous copy when not (contiguous() alone would keep a misaligned base).
inline at::Tensor aligned(const at::Tensor &t) { return is_aligned(t) ? t : t.clone(at::MemoryFormat::Contiguous); }

// A gradient output: the caller's tensor (for instance one slice of a packed
// dqkv) when it is given, written in place if its layout suits the kernels and
// through a temporary copied into it otherwise; a new tensor when absent.
// zero: rows no sequence covers (varlen padding) read 0 in a new tensor.
struct GradOut {
    at::Tensor dst, buf;
    void finish() {
        if (!buf.is_same(dst)) dst.copy_(buf);
    }
};
inline GradOut grad_out(const std::optional<at::Tensor> &given, const at::Tensor &like, bool zero,
                        const char *name) {
    auto fresh = [&] { return zero ? at::zeros(like.sizes(), like.options()) : at::empty(like.sizes(), like.options()); };
    if (!given.has_value()) {
        at::Tensor t = fresh();
        return {t, t};
    }
    const at::Tensor &g = *given;
    check_fp16_cuda(g, name);
    TORCH_CHECK(g.device() == like.device(), name, " must be on the device of its input");
    TORCH_CHECK(g.sizes() == like.sizes(), name, " must have the shape of its input");
    return {g, is_aligned(g) ? g : fresh()};
}

inline fa_tensor desc4(const at::Tensor &t) {  // [batch][row][head][d]
    return fa_tensor{t.data_ptr(), t.stride(0), t.stride(1), t.stride(2)};
}
inline fa_tensor desc3(const at::Tensor &t) {  // packed [total][head][d]
    return fa_tensor{t.data_ptr(), 0, t.stride(0), t.stride(1)};
}

// Sizes go to the kernels as int32 (their index math is 64-bit where products can overflow).
inline int32_t i32(int64_t v, const char *what) {
    TORCH_CHECK(v >= 0 && v <= INT32_MAX, what, " must be below 2^31");
    return int32_t(v);
}

inline hipStream_t current_stream() { return c10::hip::getCurrentHIPStream().stream(); }

inline void check_rc(int rc, const char *what) {
    TORCH_CHECK(rc == FA_OK, what, " failed: ", fa_error_string(rc));
}

int num_cus(int device) {
    static int cached[64] = {0};
    if (device >= 0 && device < 64 && cached[device]) return cached[device];
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n <= 0) n = 256;
    if (device >= 0 && device < 64) cached[device] = n;
    return n;
}

}  // namespace

std::vector<at::Tensor> mha_fwd(at::Tensor q, at::Tensor k, at::Tensor v, const float softmax_scale, bool is_causal) {
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "q, k, v must be rank-4 tensors");
    const int64_t batch_size = q.size(0), seqlen_q = q.size(1), num_heads = q.size(2), head_size = q.size(3);
    const int64_t seqlen_k = k.size(1), num_heads_k = k.size(2);
    TORCH_CHECK(k.size(0) == batch_size && v.size(0) == batch_size, "k/v batch size must match q");
    TORCH_CHECK(v.size(1) == seqlen_k, "k and v seqlen_k must match");
    TORCH_CHECK(v.size(2) == num_heads_k, "k and v num_heads must match");
    TORCH_CHECK(k.size(3) == head_size && v.size(3) == head_size, "q/k/v head_dim must match");
    TORCH_CHECK(num_heads % num_heads_k == 0, "num_heads_q must be divisible by num_heads_k for GQA/MQA");
    check_supported_head_dim(head_size);
    check_fp16_cuda(q, "q");
    check_fp16_cuda(k, "k");
    check_fp16_cuda(v, "v");
    c10::DeviceGuard guard(q.device());
    q = aligned(q);
    k = aligned(k);
    v = aligned(v);

    at::Tensor o = at::empty(q.sizes(), q.options());
    at::Tensor l = at::empty({batch_size, num_heads, seqlen_q}, q.options().dtype(at::kFloat));

    fa_fwd_args a{};
    a.q = desc4(q);
    a.k = desc4(k);
    a.v = desc4(v);
    a.o = desc4(o);
    a.lse = l.data_ptr<float>();
    a.batch = i32(batch_size, "batch_size");
    a.seqlen_q = i32(seqlen_q, "seqlen_q");
    a.seqlen_k = i32(seqlen_k, "seqlen_k");
    a.nheads = i32(num_heads, "num_heads");
    a.nheads_k = i32(num_heads_k, "num_heads_k");
    a.head_dim = int32_t(head_size);
    a.lse_seqlen = i32(seqlen_q, "seqlen_q");
    a.softmax_scale = softmax_scale;
    a.causal = is_causal ? 1 : 0;
    check_rc(fa_fwd(&a, current_stream()), "fa_fwd");
    return {o, l};
}

std::vector<at::Tensor> mha_bwd(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor out, at::Tensor l,
                                at::Tensor dout, const float softmax_scale, bool is_causal,
                                std::optional<at::Tensor> dq_, std::optional<at::Tensor> dk_,
                                std::optional<at::Tensor> dv_) {
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "q, k, v must be rank-4 tensors");
    TORCH_CHECK(out.dim() == 4 && dout.dim() == 4, "out and dout must be rank-4 tensors");
    const int64_t batch_size = q.size(0), seqlen_q = q.size(1), num_heads = q.size(2), head_size = q.size(3);
    const int64_t seqlen_k = k.size(1), num_heads_k = k.size(2);
    TORCH_CHECK(k.size(0) == batch_size && v.size(0) == batch_size, "k/v batch size must match q");
    TORCH_CHECK(v.size(1) == seqlen_k, "k and v seqlen_k must match");
    TORCH_CHECK(v.size(2) == num_heads_k, "k and v num_heads must match");
    TORCH_CHECK(k.size(3) == head_size && v.size(3) == head_size, "q/k/v head_dim must match");
    TORCH_CHECK(out.sizes() == q.sizes() && dout.sizes() == q.sizes(), "out and dout must match q shape");
    TORCH_CHECK(num_heads % num_heads_k == 0, "num_heads_q must be divisible by num_heads_k for GQA/MQA");
    check_supported_head_dim(head_size);
    for (auto *t : {&q, &k, &v, &out, &dout}) check_fp16_cuda(*t, "q, k, v, out and dout");
    TORCH_CHECK(l.is_cuda() && l.scalar_type() == at::kFloat && l.dim() == 3 && l.size(0) == batch_size &&
                    l.size(1) == num_heads && l.size(2) == seqlen_q && l.is_contiguous(),
                "l must be a contiguous float32 tensor of shape [batch_size, nheads_q, seqlen_q]");
    c10::DeviceGuard guard(q.device());
    q = aligned(q);
    k = aligned(k);
    v = aligned(v);
    out = aligned(out);
    dout = aligned(dout);

    GradOut dq = grad_out(dq_, q, false, "dq"), dk = grad_out(dk_, k, false, "dk"), dv = grad_out(dv_, v, false, "dv");
    at::Tensor dsum = at::empty({2, l.numel()}, l.options());  // -D, then LSE*log2(e)

    fa_bwd_args a{};
    a.q = desc4(q);
    a.k = desc4(k);
    a.v = desc4(v);
    a.o = desc4(out);
    a.dout = desc4(dout);
    a.dq = desc4(dq.buf);
    a.dk = desc4(dk.buf);
    a.dv = desc4(dv.buf);
    a.lse = l.data_ptr<float>();
    a.dsum = dsum.data_ptr<float>();
    a.batch = i32(batch_size, "batch_size");
    a.seqlen_q = i32(seqlen_q, "seqlen_q");
    a.seqlen_k = i32(seqlen_k, "seqlen_k");
    a.nheads = i32(num_heads, "num_heads");
    a.nheads_k = i32(num_heads_k, "num_heads_k");
    a.head_dim = int32_t(head_size);
    a.lse_seqlen = i32(seqlen_q, "seqlen_q");
    a.softmax_scale = softmax_scale;
    a.causal = is_causal ? 1 : 0;
    check_rc(fa_bwd(&a, current_stream()), "fa_bwd");
    for (auto *g : {&dq, &dk, &dv}) g->finish();
    return {dq.dst, dk.dst, dv.dst};
}

static void check_cu_seqlens(const at::Tensor &cu_seqlens_q, const at::Tensor &cu_seqlens_k) {
    TORCH_CHECK(cu_seqlens_q.is_cuda() && cu_seqlens_k.is_cuda(), "cu_seqlens_q/cu_seqlens_k must be CUDA tensors");
    TORCH_CHECK(cu_seqlens_q.scalar_type() == at::kInt && cu_seqlens_k.scalar_type() == at::kInt,
                "cu_seqlens_q/cu_seqlens_k must be int32 tensors");
    TORCH_CHECK(cu_seqlens_q.is_contiguous() && cu_seqlens_k.is_contiguous(),
                "cu_seqlens_q/cu_seqlens_k must be contiguous");
    TORCH_CHECK(cu_seqlens_q.dim() == 1 && cu_seqlens_k.dim() == 1, "cu_seqlens_q/cu_seqlens_k must be rank-1");
    TORCH_CHECK(cu_seqlens_q.numel() >= 2 && cu_seqlens_k.numel() >= 2,
                "cu_seqlens_q/cu_seqlens_k must have at least 2 elements");
    TORCH_CHECK(cu_seqlens_k.numel() == cu_seqlens_q.numel(),
                "cu_seqlens_k must have shape [batch_size + 1] with cumulative offsets");
}

static void check_varlen_qkv(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v) {
    TORCH_CHECK(k.size(0) == v.size(0), "k and v total tokens must match");
    TORCH_CHECK(k.size(1) == v.size(1), "k and v num_heads must match");
    TORCH_CHECK(k.size(2) == v.size(2), "k and v head_dim must match");
    TORCH_CHECK(q.size(2) == k.size(2), "q/k/v head_dim must match");
    TORCH_CHECK(q.size(1) % k.size(1) == 0, "num_heads_q must be divisible by num_heads_k for GQA/MQA");
}

std::vector<at::Tensor> mha_varlen_fwd(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor &cu_seqlens_q,
                                       at::Tensor &cu_seqlens_k, const int max_seqlen_q, const int max_seqlen_k,
                                       const float softmax_scale, bool is_causal) {
    TORCH_CHECK(q.dim() == 3 && k.dim() == 3 && v.dim() == 3, "q, k, v must be rank-3 packed tensors");
    check_cu_seqlens(cu_seqlens_q, cu_seqlens_k);
    const int64_t batch_size = cu_seqlens_q.numel() - 1;
    check_varlen_qkv(q, k, v);
    const int64_t num_heads = q.size(1), num_heads_k = k.size(1), head_size = q.size(2);
    check_supported_head_dim(head_size);
    TORCH_CHECK(max_seqlen_q >= 0 && max_seqlen_k >= 0, "max_seqlen_q/max_seqlen_k must be non-negative");
    check_fp16_cuda(q, "q");
    check_fp16_cuda(k, "k");
    check_fp16_cuda(v, "v");
    c10::DeviceGuard guard(q.device());
    q = aligned(q);
    k = aligned(k);
    v = aligned(v);

    // Packed rows past cu_seqlens_q[-1] belong to no sequence and stay 0.
    at::Tensor out = at::zeros(q.sizes(), q.options());
    at::Tensor l = at::empty({batch_size, num_heads, max_seqlen_q}, q.options().dtype(at::kFloat));

    fa_fwd_args a{};
    a.q = desc3(q);
    a.k = desc3(k);
    a.v = desc3(v);
    a.o = desc3(out);
    a.lse = l.data_ptr<float>();
    a.cu_seqlens_q = cu_seqlens_q.data_ptr<int32_t>();
    a.cu_seqlens_k = cu_seqlens_k.data_ptr<int32_t>();
    a.batch = i32(batch_size, "batch_size");
    a.seqlen_q = max_seqlen_q;
    a.seqlen_k = max_seqlen_k;
    a.nheads = i32(num_heads, "num_heads");
    a.nheads_k = i32(num_heads_k, "num_heads_k");
    a.head_dim = int32_t(head_size);
    a.lse_seqlen = max_seqlen_q;
    a.softmax_scale = softmax_scale;
    a.causal = is_causal ? 1 : 0;
    // Query blocks ordered most work first on the device (sequences of mixed lengths).
    at::Tensor work_order = at::empty({int64_t(std::max<size_t>(fa_fwd_order_len(&a), 1))}, cu_seqlens_q.options());
    a.work_order = work_order.data_ptr<int32_t>();
    check_rc(fa_fwd(&a, current_stream()), "fa_fwd (varlen)");
    return {out, l};
}

std::vector<at::Tensor> mha_varlen_bwd(at::Tensor q, at::Tensor k, at::Tensor v, at::Tensor out, at::Tensor l,
                                       at::Tensor dout, at::Tensor cu_seqlens_q, at::Tensor cu_seqlens_k,
                                       const int max_seqlen_q, const int max_seqlen_k, const float softmax_scale,
                                       bool is_causal, std::optional<at::Tensor> dq_, std::optional<at::Tensor> dk_,
                                       std::optional<at::Tensor> dv_) {
    TORCH_CHECK(q.dim() == 3 && k.dim() == 3 && v.dim() == 3, "q, k, v must be rank-3 packed tensors");
    check_cu_seqlens(cu_seqlens_q, cu_seqlens_k);
    const int64_t batch_size = cu_seqlens_q.numel() - 1;
    check_varlen_qkv(q, k, v);
    TORCH_CHECK(out.sizes() == q.sizes(), "out must match q shape");
    TORCH_CHECK(dout.sizes() == q.sizes(), "dout must match q shape");
    TORCH_CHECK(l.dim() == 3, "l must be rank-3 for varlen_bwd");
    const int64_t num_heads = q.size(1), num_heads_k = k.size(1), head_size = q.size(2);
    check_supported_head_dim(head_size);
    TORCH_CHECK(l.size(0) == batch_size && l.size(1) == num_heads && l.size(2) == max_seqlen_q,
                "l must have shape [batch_size, nheads_q, max_seqlen_q]");
    for (auto *t : {&q, &k, &v, &out, &dout}) check_fp16_cuda(*t, "q, k, v, out and dout");
    TORCH_CHECK(l.is_cuda() && l.scalar_type() == at::kFloat && l.is_contiguous(),
                "l must be a contiguous float32 CUDA tensor");
    c10::DeviceGuard guard(q.device());
    q = aligned(q);
    k = aligned(k);
    v = aligned(v);
    out = aligned(out);
    dout = aligned(dout);

    // Packed rows past the last sequence belong to no sequence: 0 in a new
    // gradient tensor, left as they are in a caller's.
    GradOut dq = grad_out(dq_, q, true, "dq"), dk = grad_out(dk_, k, true, "dk"), dv = grad_out(dv_, v, true, "dv");
    at::Tensor dsum = at::empty({2, l.numel()}, l.options());  // -D, then LSE*log2(e)

    fa_bwd_args a{};
    a.q = desc3(q);
    a.k = desc3(k);
    a.v = desc3(v);
    a.o = desc3(out);
    a.dout = desc3(dout);
    a.dq = desc3(dq.buf);
    a.dk = desc3(dk.buf);
    a.dv = desc3(dv.buf);
    a.lse = l.data_ptr<float>();
    a.dsum = dsum.data_ptr<float>();
    a.cu_seqlens_q = cu_seqlens_q.data_ptr<int32_t>();
    a.cu_seqlens_k = cu_seqlens_k.data_ptr<int32_t>();
    a.batch = i32(batch_size, "batch_size");
    a.seqlen_q = max_seqlen_q;
    a.seqlen_k = max_seqlen_k;
    a.nheads = i32(num_heads, "num_heads");
    a.nheads_k = i32(num_heads_k, "num_heads_k");
    a.head_dim = int32_t(head_size);
    a.lse_seqlen = max_seqlen_q;
    a.softmax_scale = softmax_scale;
    a.causal = is_causal ? 1 : 0;
    // dQ and dK/dV work items ordered longest first on the device (sequences of mixed lengths).
    at::Tensor work_order = at::empty({int64_t(std::max<size_t>(fa_bwd_order_len(&a), 1))}, cu_seqlens_k.options());
    a.work_order = work_order.data_ptr<int32_t>();
    check_rc(fa_bwd(&a, current_stream()), "fa_bwd (varlen)");
    for (auto *g : {&dq, &dk, &dv}) g->finish();
    return {dq.dst, dk.dst, dv.dst};
}

std::vector<at::Tensor> mha_fwd_kvcache(at::Tensor q, at::Tensor k_cache, at::Tensor v_cache,
                                        std::optional<at::Tensor> k_opt, std::optional<at::Tensor> v_opt,
                                        at::Tensor cache_seqlens, std::optional<at::Tensor> rotary_cos,
                                        std::optional<at::Tensor> rotary_sin,
                                        std::optional<at::Tensor> cache_batch_idx_opt,
                                        std::optional<at::Tensor> cache_leftpad,
                                        std::optional<at::Tensor> block_table_opt,
                                        std::optional<at::Tensor> alibi_slopes, std::optional<at::Tensor> out_opt,
                                        const float softmax_scale, bool is_causal, int window_size_left,
                                        int window_size_right, const float softcap, bool rotary_interleaved,
                                        int num_splits, std::optional<at::Tensor> status_opt) {
    // Order and texts follow flash_api.cpp:530-628.  status (optional, after
    // the reference's arguments): an int32 device word; when given, the cache
    // capacity and cache_batch_idx bounds are checked on the device instead of
    // by host reads (no synchronisation, so the call can be graph-captured):
    // 1 (capacity) / 2 (cache row) are ORed into it for the caller to report.
    TORCH_CHECK(!out_opt.has_value(), "Turing KV-cache does not support a preallocated output tensor yet");
    // Rotary embeddings, local windows, softcap, ALiBi and cache_leftpad
    // (rejected by the reference, flash_api.cpp:530-539) take upstream
    // FlashAttention's semantics; attention with them runs in the split kernel.
    TORCH_CHECK(std::isfinite(softcap), "softcap must be finite");
    TORCH_CHECK(num_splits >= 0, "num_splits must be non-negative");

    TORCH_CHECK(q.is_cuda() && k_cache.is_cuda() && v_cache.is_cuda(), "q, k_cache, v_cache must be CUDA tensors");
    TORCH_CHECK(q.scalar_type() == at::kHalf && k_cache.scalar_type() == at::kHalf &&
                    v_cache.scalar_type() == at::kHalf,
                "q, k_cache, v_cache must be float16 tensors");
    TORCH_CHECK(q.dim() == 4 && k_cache.dim() == 4 && v_cache.dim() == 4, "q, k_cache, v_cache must be rank-4 tensors");
    TORCH_CHECK(k_cache.size(1) == v_cache.size(1), "k_cache and v_cache seqlen must match");
    TORCH_CHECK(k_cache.size(2) == v_cache.size(2), "k_cache and v_cache num_heads must match");
    TORCH_CHECK(q.size(3) == k_cache.size(3) && q.size(3) == v_cache.size(3), "q, k_cache, v_cache head_dim must match");
    TORCH_CHECK(q.size(2) % k_cache.size(2) == 0, "num_heads_q must be divisible by num_heads_k for GQA/MQA");
    check_supported_head_dim(q.size(3));
    TORCH_CHECK(q.stride(-1) == 1 && k_cache.stride(-1) == 1 && v_cache.stride(-1) == 1,
                "q, k_cache, v_cache must have contiguous last dimension");
    TORCH_CHECK(cache_seqlens.is_cuda(), "cache_seqlens must be a CUDA tensor");
    TORCH_CHECK(cache_seqlens.scalar_type() == at::kInt, "cache_seqlens must be an int32 tensor");
    TORCH_CHECK(cache_seqlens.is_contiguous(), "cache_seqlens must be contiguous");
    TORCH_CHECK(cache_seqlens.dim() == 1 && cache_seqlens.numel() == q.size(0),
                "cache_seqlens must have shape [batch_size]");

    const int64_t batch_size = q.size(0), seqlen_q = q.size(1), num_heads = q.size(2), head_size = q.size(3);
    const int64_t num_heads_k = k_cache.size(2);
    const bool has_block_table = block_table_opt.has_value();
    at::Tensor block_table;
    int64_t page_block_size = 0;
    int64_t seqlen_cache = k_cache.size(1);
    int64_t batch_size_cache = k_cache.size(0);
    if (has_block_table) {
        block_table = *block_table_opt;
        TORCH_CHECK(block_table.is_cuda(), "block_table must be a CUDA tensor");
        TORCH_CHECK(block_table.scalar_type() == at::kInt, "block_table must be an int32 tensor");
        TORCH_CHECK(block_table.stride(-1) == 1, "block_table must have contiguous last dimension");
        TORCH_CHECK(block_table.dim() == 2 && block_table.size(0) == batch_size,
                    "block_table must have shape [batch_size, max_num_blocks_per_seq]");
        page_block_size = k_cache.size(1);
        TORCH_CHECK(page_block_size % 256 == 0, "Paged KV cache block size must be divisible by 256");
        seqlen_cache = block_table.size(1) * page_block_size;
        batch_size_cache = batch_size;
    }
    TORCH_CHECK(seqlen_cache <= INT32_MAX, "KV cache capacity must be below 2^31 tokens per sequence");

    at::Tensor cache_batch_idx;
    const bool has_cache_batch_idx = cache_batch_idx_opt.has_value();
    if (has_cache_batch_idx) {
        TORCH_CHECK(!has_block_table, "Paged KV cache does not support cache_batch_idx");
        cache_batch_idx = *cache_batch_idx_opt;
        TORCH_CHECK(cache_batch_idx.is_cuda(), "cache_batch_idx must be a CUDA tensor");
        TORCH_CHECK(cache_batch_idx.scalar_type() == at::kInt, "cache_batch_idx must be an int32 tensor");
        TORCH_CHECK(cache_batch_idx.is_contiguous(), "cache_batch_idx must be contiguous");
        TORCH_CHECK(cache_batch_idx.dim() == 1 && cache_batch_idx.numel() == batch_size,
                    "cache_batch_idx must have shape [batch_size]");
    } else {
        TORCH_CHECK(batch_size == batch_size_cache,
                    "q and cache batch size must match when cache_batch_idx is not provided");
    }

    at::Tensor k, v;
    const bool has_k = k_opt.has_value(), has_v = v_opt.has_value();
    TORCH_CHECK(has_k == has_v, "k and v must either both be provided or both be None");
    int64_t seqlen_new = 0;
    if (has_k) {
        k = *k_opt;
        v = *v_opt;
        TORCH_CHECK(k.is_cuda() && v.is_cuda(), "k and v must be CUDA tensors");
        TORCH_CHECK(k.scalar_type() == at::kHalf && v.scalar_type() == at::kHalf, "k and v must be float16 tensors");
        TORCH_CHECK(k.dim() == 4 && v.dim() == 4, "k and v must be rank-4 tensors");
        TORCH_CHECK(k.size(0) == batch_size && v.size(0) == batch_size, "k/v batch size must match q");
        TORCH_CHECK(k.size(1) == v.size(1), "k and v seqlen must match");
        TORCH_CHECK(k.size(2) == num_heads_k && v.size(2) == num_heads_k, "k/v num_heads must match the cache num_heads");
        TORCH_CHECK(k.size(3) == head_size && v.size(3) == head_size, "k/v head_dim must match q");
        TORCH_CHECK(k.stride(-1) == 1 && v.stride(-1) == 1, "k and v must have contiguous last dimension");
        seqlen_new = k.size(1);
    }

    c10::DeviceGuard guard(q.device());
    int32_t *status = nullptr;
    if (status_opt.has_value()) {
        const at::Tensor &st = *status_opt;
        TORCH_CHECK(st.is_cuda() && st.device() == q.device() && st.scalar_type() == at::kInt && st.numel() >= 1 &&
                        st.is_contiguous(),
                    "status must be a contiguous int32 tensor on the device of q");
        status = st.data_ptr<int32_t>();
    }
    // Without a status word, the reference's host-visible checks (two
    // device-to-host reads); the kernels bound every access either way.
    if (!status && batch_size > 0) {
        const int64_t max_end = cache_seqlens.max().item<int>() + seqlen_new;
        TORCH_CHECK(max_end <= seqlen_cache, "cache capacity is insufficient for the requested append length");
    }
    if (!status && has_cache_batch_idx && batch_size > 0) {
        at::Tensor idx_cpu = cache_batch_idx.to(at::kCPU);
        const int32_t *p = idx_cpu.data_ptr<int32_t>();
        for (int64_t i = 0; i < batch_size; ++i)
            TORCH_CHECK(p[i] >= 0 && p[i] < batch_size_cache, "cache_batch_idx entries must be within cache batch bounds");
    }

    q = aligned(q);
    TORCH_CHECK(((reinterpret_cast<uintptr_t>(k_cache.data_ptr()) | reinterpret_cast<uintptr_t>(v_cache.data_ptr())) &
                 15u) == 0 &&
                    k_cache.stride(0) % 8 == 0 && k_cache.stride(1) % 8 == 0 && k_cache.stride(2) % 8 == 0 &&
                    v_cache.stride(0) % 8 == 0 && v_cache.stride(1) % 8 == 0 && v_cache.stride(2) % 8 == 0,
                "k_cache and v_cache must be 16-byte aligned with strides that are multiples of 8 elements");
    if (has_k) {
        k = aligned(k);
        v = aligned(v);
    }

    at::Tensor out = at::empty(q.sizes(), q.options());
    at::Tensor lse = at::empty({batch_size, num_heads, seqlen_q}, q.options().dtype(at::kFloat));
    hipStream_t stream = current_stream();

    fa_kvcache_args a{};
    a.q = desc4(q);
    a.k_cache = desc4(k_cache);
    a.v_cache = desc4(v_cache);
    if (has_k) {
        a.k_new = desc4(k);
        a.v_new = desc4(v);
    }
    a.o = desc4(out);
    a.lse = lse.data_ptr<float>();
    a.cache_seqlens = cache_seqlens.data_ptr<int32_t>();
    a.cache_batch_idx = has_cache_batch_idx ? cache_batch_idx.data_ptr<int32_t>() : nullptr;
    a.block_table = has_block_table ? block_table.data_ptr<int32_t>() : nullptr;
    a.block_table_stride = has_block_table ? block_table.stride(0) : 0;
    a.batch = i32(batch_size, "batch_size");
    a.seqlen_q = i32(seqlen_q, "seqlen_q");
    a.nheads = i32(num_heads, "num_heads");
    a.nheads_k = i32(num_heads_k, "num_heads_k");
    a.head_dim = int32_t(head_size);
    a.seqlen_new = i32(seqlen_new, "seqlen_new");
    a.page_block_size = int32_t(page_block_size);
    a.softmax_scale = softmax_scale;
    a.causal = is_causal ? 1 : 0;
    a.num_splits = 1;
    a.cache_capacity = int32_t(seqlen_cache);
    a.cache_batch = has_block_table ? 0 : i32(batch_size_cache, "cache batch size");
    a.status = status;
    // Upstream's normalisation: a bound at least the cache capacity is no bound.
    if (window_size_left >= seqlen_cache) window_size_left = -1;
    if (window_size_right >= seqlen_cache) window_size_right = -1;
    a.local_window = (window_size_left >= 0 || window_size_right >= 0) ? 1 : 0;
    a.window_left = window_size_left;
    a.window_right = window_size_right;
    a.softcap = softcap > 0.f ? softcap : 0.f;
    if (cache_leftpad.has_value()) {
        const at::Tensor &lp = *cache_leftpad;
        TORCH_CHECK(lp.is_cuda() && lp.device() == q.device(), "cache_leftpad must be a CUDA tensor on the device of q");
        TORCH_CHECK(lp.scalar_type() == at::kInt, "cache_leftpad must have dtype int32");
        TORCH_CHECK(lp.dim() == 1 && lp.size(0) == batch_size && lp.is_contiguous(),
                    "cache_leftpad must be a contiguous tensor of shape [batch_size]");
        a.cache_leftpad = lp.data_ptr<int32_t>();
    }
    if (alibi_slopes.has_value()) {
        const at::Tensor &al = *alibi_slopes;
        TORCH_CHECK(al.is_cuda() && al.device() == q.device(), "alibi_slopes must be a CUDA tensor on the device of q");
        TORCH_CHECK(al.scalar_type() == at::kFloat, "ALiBi slopes must have dtype fp32");
        TORCH_CHECK(al.stride(-1) == 1, "ALiBi slopes tensor must have contiguous last dimension");
        TORCH_CHECK((al.dim() == 1 && al.size(0) == num_heads) ||
                        (al.dim() == 2 && al.size(0) == batch_size && al.size(1) == num_heads),
                    "ALiBi slopes must have shape (num_heads) or (batch_size, num_heads)");
        a.alibi_slopes = al.data_ptr<float>();
        a.alibi_batch_stride = al.dim() == 2 ? al.stride(0) : 0;
    }
    at::Tensor cos_t, sin_t;
    if (rotary_cos.has_value() || rotary_sin.has_value()) {
        // Upstream's checks for the rotary tables.
        TORCH_CHECK(has_k, "If rotary cos/sin are provided, new key / value to be appended to KV cache must also be provided");
        TORCH_CHECK(rotary_cos.has_value() && rotary_sin.has_value(),
                    "If rotary cos is provided, rotary sin must also be provided");
        cos_t = *rotary_cos;
        sin_t = *rotary_sin;
        TORCH_CHECK(cos_t.is_cuda() && cos_t.device() == q.device() && sin_t.is_cuda() && sin_t.device() == q.device(),
                    "rotary_cos / rotary_sin must be CUDA tensors on the device of q");
        TORCH_CHECK(cos_t.scalar_type() == at::kHalf && sin_t.scalar_type() == at::kHalf,
                    "rotary_cos / rotary_sin must have the same dtype as query");
        TORCH_CHECK(cos_t.dim() == 2, "rotary_cos must have shape (seqlen_ro, rotary_dim / 2)");
        const int64_t rotary_dim = 2 * cos_t.size(1), seqlen_ro = cos_t.size(0);
        TORCH_CHECK(rotary_dim <= head_size, "rotary_dim must be <= headdim");
        TORCH_CHECK(rotary_dim % 16 == 0, "Only rotary dimensions divisible by 16 are currently supported");
        TORCH_CHECK(sin_t.dim() == 2 && sin_t.size(0) == seqlen_ro && sin_t.size(1) == rotary_dim / 2,
                    "rotary_sin must have the shape of rotary_cos");
        TORCH_CHECK(seqlen_ro >= 1 && seqlen_ro <= INT32_MAX, "rotary_cos must have at least one row");
        if (has_block_table)
            TORCH_CHECK(seqlen_ro >= seqlen_cache, "cos/sin seqlen must be at least the seqlen of KV cache");
        // The kernels read angle row p at p * rotary_dim / 2 (packed rows): a
        // view with any other row stride (a column slice of a wider table) is
        // copied first.
        cos_t = aligned(cos_t.contiguous());
        sin_t = aligned(sin_t.contiguous());
        a.rotary_cos = cos_t.data_ptr();
        a.rotary_sin = sin_t.data_ptr();
        a.rotary_dim = int32_t(rotary_dim);
        a.rotary_seqlen = int32_t(seqlen_ro);
        a.rotary_interleaved = rotary_interleaved ? 1 : 0;
    }
    const bool options =
        a.local_window || a.softcap > 0.f || a.cache_leftpad || a.alibi_slopes || a.rotary_dim > 0;

    // Routing of flash_api.cpp:668: paged, explicit splits > 1 or single-token decode
    // take the split-KV kernel; a contiguous multi-token chunk takes the tiled
    // forward kernel with per-batch key counts and the batch remap.
    const bool use_split_kernel = has_block_table || num_splits > 1 || seqlen_q == 1 || options;
    if (use_split_kernel) {
        a.num_splits = fa_kv_num_splits(num_splits, int(seqlen_cache), int(head_size), int(seqlen_q),
                                        int(batch_size), int(num_heads), int(num_heads_k),
                                        num_cus(q.get_device()));
        // Workspace: split accumulators (num_splits > 1), then the longest-first
        // sequence order the split kernel schedules by and its work counter, then
        // the split counts with which it combines the partials itself.  Append,
        // split and combine are then two launches.
        const int64_t rows = batch_size * num_heads * seqlen_q;
        const int64_t acc_floats = a.num_splits > 1 ? a.num_splits * rows * (head_size + 1) : 0;
        const int64_t counts = int64_t(fa_kv_split_count_len(&a));
        at::Tensor ws = at::empty({acc_floats + batch_size + 1 + counts}, q.options().dtype(at::kFloat));
        if (a.num_splits > 1) {
            a.out_accum = ws.data_ptr<float>();
            a.lse_accum = a.out_accum + a.num_splits * rows * head_size;
        }
        a.batch_order = reinterpret_cast<int32_t *>(ws.data_ptr<float>() + acc_floats);
        a.split_count = counts > 0 ? a.batch_order + batch_size + 1 : nullptr;
        check_rc(fa_fwd_kvcache(&a, stream), "fa_fwd_kvcache");
        return {out, lse};
    }

    check_rc(fa_kv_append(&a, stream), "fa_kv_append");

    fa_fwd_args f{};
    f.q = desc4(q);
    f.k = desc4(k_cache);
    f.v = desc4(v_cache);
    f.o = desc4(out);
    f.lse = lse.data_ptr<float>();
    f.seqused_k = cache_seqlens.data_ptr<int32_t>();
    f.seqused_k_add = int32_t(seqlen_new);
    f.k_batch_idx = a.cache_batch_idx;
    f.batch = i32(batch_size, "batch_size");
    f.seqlen_q = i32(seqlen_q, "seqlen_q");
    f.seqlen_k = int32_t(seqlen_cache);
    f.nheads = i32(num_heads, "num_heads");
    f.nheads_k = i32(num_heads_k, "num_heads_k");
    f.head_dim = int32_t(head_size);
    f.lse_seqlen = i32(seqlen_q, "seqlen_q");
    f.softmax_scale = softmax_scale;
    f.causal = is_causal ? 1 : 0;
    f.k_batch = i32(batch_size_cache, "cache batch size");
    f.status = status;
    check_rc(fa_fwd(&f, stream), "fa_fwd (kv-cache chunk)");
    return {out, lse};
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    // The library found at load time must have the struct layouts this module was compiled with.
    TORCH_CHECK(fa_abi_version() == FA_ABI_VERSION, "libfa_mi355x.so has argument-struct layout version ",
                fa_abi_version(), ", flash_attn_turing was built against version ", FA_ABI_VERSION, ": rebuild both");
    m.def("fwd", &mha_fwd, "Forward pass");
    // dq / dk / dv (optional, after the reference's arguments): tensors the
    // gradients are written into, such as the slices of a packed dqkv.
    m.def("bwd", &mha_bwd, "Backward pass", py::arg("q"), py::arg("k"), py::arg("v"), py::arg("out"), py::arg("l"),
          py::arg("dout"), py::arg("softmax_scale"), py::arg("is_causal"), py::arg("dq") = py::none(),
          py::arg("dk") = py::none(), py::arg("dv") = py::none());
    m.def("varlen_fwd", &mha_varlen_fwd, "Varlen forward pass");
    m.def("varlen_bwd", &mha_varlen_bwd, "Varlen backward pass", py::arg("q"), py::arg("k"), py::arg("v"),
          py::arg("out"), py::arg("l"), py::arg("dout"), py::arg("cu_seqlens_q"), py::arg("cu_seqlens_k"),
          py::arg("max_seqlen_q"), py::arg("max_seqlen_k"), py::arg("softmax_scale"), py::arg("is_causal"),
          py::arg("dq") = py::none(), py::arg("dk") = py::none(), py::arg("dv") = py::none());
    m.def("fwd_kvcache", &mha_fwd_kvcache, "KV-cache forward pass", py::arg("q"), py::arg("k_cache"),
          py::arg("v_cache"), py::arg("k"), py::arg("v"), py::arg("cache_seqlens"), py::arg("rotary_cos"),
          py::arg("rotary_sin"), py::arg("cache_batch_idx"), py::arg("cache_leftpad"), py::arg("block_table"),
          py::arg("alibi_slopes"), py::arg("out"), py::arg("softmax_scale"), py::arg("is_causal"),
          py::arg("window_size_left"), py::arg("window_size_right"), py::arg("softcap"),
          py::arg("rotary_interleaved"), py::arg("num_splits"), py::arg("status") = py::none());
}
