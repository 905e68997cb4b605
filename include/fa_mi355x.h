/*
 * fa_mi355x.h - C ABI of the MI355X (gfx950) FlashAttention kernels.
 *
 * This is the boundary between the host layer (the `flash_attn_turing`
 * PyTorch extension, or any FFI: ctypes, cgo, JNI) and the hand-written HIP
 * kernels in libfa_mi355x.so.  Every entry point takes plain device pointers,
 * sizes and strides (in elements, 64-bit), never allocates, launches on the
 * given HIP stream (a `hipStream_t` passed as `void *`, NULL = default
 * stream) and returns FA_OK or an error code (see fa_error_string).
 *
 * Tensor convention (reference: flash_attention_interface.py:457-462, 530-539;
 * flash_api.cpp:188-256): q/o [batch][seqlen][heads][head_dim] fp16 with the
 * last dimension contiguous; k/v [batch][seqlen_k][heads_k][head_dim].  For
 * packed varlen tensors ([total][heads][head_dim]) batch_stride is ignored and
 * the row offset of batch b is cu_seqlens[b].  LSE is fp32
 * [batch][heads][lse_seqlen].  head_dim is 64 or 128 (flash_api.cpp:10-14).
 * Rows, heads and the base pointer must be 16-byte aligned (strides multiple
 * of 8 elements).
 */
#ifndef FA_MI355X_H
#define FA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    FA_OK = 0,
    FA_ERR_INVALID_ARG = -1,   /* shape / pointer / alignment check failed   */
    FA_ERR_UNSUPPORTED = -2,   /* head_dim not in {64, 128} and similar      */
    FA_ERR_WORKSPACE = -3,     /* missing or too small workspace             */
    FA_ERR_SCRATCH = -4        /* request beyond fa_fwd_kvcache_noalloc's static scratch */
    /* positive values are hipError_t codes from the launch                  */
};

/* A strided fp16 tensor [batch][row][head][head_dim]; strides in elements. */
typedef struct fa_tensor {
    void *ptr;
    int64_t batch_stride;
    int64_t row_stride;
    int64_t head_stride;
} fa_tensor;

/*
 * Forward attention.  Replaces the reference's run_mha_fwd(Flash_fwd_params&)
 * (flash_api.cpp:174-179, params from set_params_fprop :39-106) used by
 * mha_fwd (:188-256), mha_varlen_fwd (:353-416) and the KV-cache chunk path
 * (:686-714).
 */
typedef struct fa_fwd_args {
    fa_tensor q, k, v, o;           /* fp16; o is written for every valid row   */
    float *lse;                     /* fp32 [batch][nheads][lse_seqlen]          */
    const int32_t *cu_seqlens_q;    /* [batch+1] or NULL (dense)                 */
    const int32_t *cu_seqlens_k;    /* [batch+1] or NULL (dense)                 */
    const int32_t *seqused_k;       /* [batch] keys used per batch, or NULL      */
    const int32_t *k_batch_idx;     /* [batch] k/v batch read by q batch b, or NULL */
    int32_t seqused_k_add;          /* added to seqused_k[b] (appended tokens)   */
    int32_t batch, seqlen_q, seqlen_k, nheads, nheads_k, head_dim;
    int32_t lse_seqlen;             /* seqlen_q, or max_seqlen_q for varlen      */
    float softmax_scale;
    int32_t causal;                 /* bottom-right aligned (mask.h:52)          */
    /* KV-cache chunk checks, done on the device (no host read; replaces the
     * reference's host-side checks flash_api.cpp:627, 634-641): with seqused_k,
     * a batch whose key count is negative or above seqlen_k, or whose
     * k_batch_idx is outside [0, k_batch), is given no keys (O = 0, LSE = 0)
     * and, when status is set, ORs 1 (capacity) or 2 (cache row) into *status. */
    int32_t k_batch;                /* batches of k/v bounding k_batch_idx, 0 = unchecked */
    int32_t *status;                /* device int32 error word, or NULL          */
    /* Optional workspace for varlen calls (cu_seqlens_q set), fa_fwd_order_len(args)
     * int32s: fa_fwd then first lists the (sequence, query block) work items on
     * the device, most work first, and launches the workgroups in that order;
     * NULL keeps the natural order.  Results are the same either way. */
    int32_t *work_order;
} fa_fwd_args;

/* Length in int32s of fa_fwd's work_order workspace: batch * ceil(lse_seqlen / 32).
 * No counterpart in the reference (its grid is in natural order). */
size_t fa_fwd_order_len(const fa_fwd_args *args);
int fa_fwd(const fa_fwd_args *args, void *stream);

/*
 * Backward attention.  Replaces run_mha_bwd(Flash_bwd_params&) (flash_api.cpp:181-186)
 * and run_flash_bwd's three launches (flash_bwd_launch_template.h:69-146), plus
 * the GQA dK/dV reduction done with torch::sum_out (flash_api.cpp:338-348,
 * 493-503): dk/dv are written per KV head, the group is summed in-kernel.
 */
typedef struct fa_bwd_args {
    fa_tensor q, k, v, o, dout;     /* fp16 inputs                               */
    fa_tensor dq, dk, dv;           /* fp16 outputs, every valid row written     */
    const float *lse;               /* fp32 [batch][nheads][lse_seqlen]          */
    float *dsum;                    /* workspace fp32 [2][batch][nheads][lse_seqlen]: -rowsum(dO*O),
                                       then LSE*log2(e) (written by fa_bwd_dq / fa_bwd_preprocess) */
    const int32_t *cu_seqlens_q;
    const int32_t *cu_seqlens_k;
    int32_t batch, seqlen_q, seqlen_k, nheads, nheads_k, head_dim;
    int32_t lse_seqlen;
    float softmax_scale;
    int32_t causal;
    /* Optional workspace for varlen calls, fa_bwd_order_len(args) int32s:
     * fa_bwd_dkdv (cu_seqlens_k set) first lists the (sequence, key block)
     * work items on the device, most query rows first, and launches the dK/dV
     * workgroups in that order, and fa_bwd_dq (cu_seqlens_q set) does the same
     * for its (sequence, query block) items, most keys first, in the second
     * part of the workspace; NULL keeps the natural order, which is longest
     * first only when every sequence has the same length.  Results are the same
     * either way (each item is computed independently). */
    int32_t *work_order;
} fa_bwd_args;

/* Length in int32s of the work_order workspace: batch * (ceil(seqlen_k / 128) +
 * ceil(lse_seqlen / 32)).  No counterpart in the reference (its grids are in
 * natural order). */
size_t fa_bwd_order_len(const fa_bwd_args *args);
/* D = rowsum(dO * O) (flash_bwd_preprocess_kernel.h:23-96), stored negated in dsum plane 0. */
int fa_bwd_preprocess(const fa_bwd_args *args, void *stream);
/* dQ kernel (flash_bwd_kernel.h:25-609); computes and stores the dsum workspace itself. */
int fa_bwd_dq(const fa_bwd_args *args, void *stream);
/* dK/dV kernel with in-kernel GQA accumulation (flash_bwd_kernel.h:613-1344); reads the
 * dsum workspace written by fa_bwd_dq or fa_bwd_preprocess. */
int fa_bwd_dkdv(const fa_bwd_args *args, void *stream);
/* dQ (with the dsum workspace) then dK/dV, in stream order. */
int fa_bwd(const fa_bwd_args *args, void *stream);

/*
 * KV-cache attention.  Replaces run_kvcache_paged_append (kvcache_native.cu:956-993),
 * the contiguous append loop (flash_api.cpp:643-654) and run_mha_fwd_kvcache_native
 * (kvcache_native.cu:995-1218) called from mha_fwd_kvcache (flash_api.cpp:508-715).
 * Attention runs over L_b = cache_seqlens[b] + seqlen_new keys.
 */
typedef struct fa_kvcache_args {
    fa_tensor q;                    /* [batch][seqlen_q][nheads][head_dim]       */
    fa_tensor k_cache, v_cache;     /* contiguous [batch_cache][capacity][nheads_k][d]
                                       or paged [num_blocks][page_block_size][nheads_k][d] */
    fa_tensor k_new, v_new;         /* [batch][seqlen_new][nheads_k][d]; ptr NULL = no append */
    fa_tensor o;                    /* [batch][seqlen_q][nheads][head_dim]       */
    float *lse;                     /* [batch][nheads][seqlen_q]                 */
    const int32_t *cache_seqlens;   /* [batch] tokens in the cache before append */
    const int32_t *cache_batch_idx; /* [batch] cache row of batch b, or NULL     */
    const int32_t *block_table;     /* [batch][block_table_stride], or NULL      */
    int64_t block_table_stride;
    int32_t batch, seqlen_q, nheads, nheads_k, head_dim;
    int32_t seqlen_new;             /* tokens appended per sequence (0 = none)   */
    int32_t page_block_size;        /* paged: multiple of 256; contiguous: 0     */
    int32_t num_splits;             /* >= 1, as resolved by fa_kv_num_splits     */
    float softmax_scale;
    int32_t causal;
    float *out_accum;               /* workspace [num_splits][batch*nheads*seqlen_q][d] fp32, 8-byte aligned */
    float *lse_accum;               /* workspace [num_splits][batch*nheads*seqlen_q] fp32    */
    int32_t *batch_order;           /* workspace [batch + 1]: sequences longest first and a work
                                       counter (both filled by fa_kv_splitkv or fa_fwd_kvcache),
                                       or NULL for the natural order                           */
    /* Device-side input checks (replace the host reads of flash_api.cpp:627,
     * 634-641 and interface.py:855, so a decode step needs no host sync): a
     * sequence with cache_seqlens[b] < 0, cache_seqlens[b] + seqlen_new >
     * cache_capacity, or cache_batch_idx[b] outside [0, cache_batch) is not
     * appended to and is attended over no keys (O = 0, LSE = 0); with status
     * set, 1 (capacity) or 2 (cache row) is ORed into *status.  0 = unchecked. */
    int32_t cache_capacity;         /* tokens one sequence's cache holds (paged: pages * page size) */
    int32_t cache_batch;            /* rows of a contiguous cache (bounds cache_batch_idx)         */
    int32_t *status;                /* device int32 error word, or NULL                            */
    /* Upstream FlashAttention options the reference's signature takes but rejects
     * (flash_attention_interface.py:617-634), with upstream's semantics: query i
     * (at key position p = i + L - seqlen_q) sees keys [p - window_left, p + window_right]
     * (a negative bound is unbounded; causal also caps the right side at p), and
     * softcap > 0 replaces the scaled score x by softcap * tanh(x / softcap),
     * ALiBi adds -slope[h] * |p - j| to the score of key j, and key j < cache_leftpad[b]
     * does not exist for sequence b (positions unchanged).  Zero-initialised, all are off. */
    int32_t local_window;           /* 1: apply window_left / window_right; 0: no window */
    int32_t window_left, window_right;
    float softcap;                  /* > 0: softcapping on                                          */
    const int32_t *cache_leftpad;   /* [batch] first valid key of each sequence, or NULL            */
    const float *alibi_slopes;      /* fp32 [nheads] (batch stride 0) or [batch][nheads], or NULL   */
    int64_t alibi_batch_stride;
    /* Rotary embedding on append (upstream FlashAttention's, also rejected by the
     * reference): with rotary_dim > 0 (a multiple of 16, at most head_dim; k_new
     * required), channels [0, rotary_dim) of appended key t of sequence b are
     * rotated at position cache_seqlens[b] + t before the store, and those of
     * query row i at cache_seqlens[b] + i when causal or local_window, else at
     * cache_seqlens[b]; position p's angles are row p of rotary_cos / rotary_sin
     * (fp16 [rotary_seqlen][rotary_dim / 2], contiguous, 16-byte aligned; a
     * position past the last row takes the last row).  Interleaved rotates
     * channel pairs (2j, 2j + 1) by angle j, otherwise (j, j + rotary_dim / 2). */
    const void *rotary_cos, *rotary_sin;
    int32_t rotary_dim;             /* 0: no rotary embedding                                       */
    int32_t rotary_seqlen;
    int32_t rotary_interleaved;
    /* Workspace of fa_kv_split_count_len(args) int32s, or NULL.  With it, batch_order
     * and num_splits > 1, the split kernel combines the partials itself: the last of
     * the num_splits items of each (batch, kv head, 32-row tile) to finish reads them
     * and writes o and lse, so fa_kv_combine has nothing left to do (it returns at
     * once) and fa_fwd_kvcache runs two kernels (append with ordering, split) instead
     * of four.  The ordering kernel zeroes these counts on every call. */
    int32_t *split_count;
} fa_kvcache_args;

/* Split count for a request (kvcache_native.cu:913-952 choose_num_splits);
 * requested > 0 is returned unchanged. */
int fa_kv_num_splits(int requested, int seqlen_k_capacity, int head_dim, int seqlen_q,
                     int batch, int nheads, int nheads_k, int num_cus);
/* Bytes of the split accumulators for args->num_splits (0 when num_splits == 1);
 * batch_order, when used, needs (batch + 1) * 4 more. */
size_t fa_kv_workspace_bytes(const fa_kvcache_args *args);
/* int32s of the split_count workspace: batch * nheads_k * ceil(nheads / nheads_k *
 * seqlen_q / 32) when num_splits > 1, else 0. */
size_t fa_kv_split_count_len(const fa_kvcache_args *args);
/* In-place append of k_new/v_new at cache_seqlens (contiguous, remapped or paged). */
int fa_kv_append(const fa_kvcache_args *args, void *stream);
/* Split-KV partial attention; writes o/lse directly when num_splits == 1, or with
 * batch_order and split_count. */
int fa_kv_splitkv(const fa_kvcache_args *args, void *stream);
/* Log-sum-exp combine of the split partials into o/lse (kvcache_native.cu:676-729);
 * nothing to do when fa_kv_splitkv combined them (batch_order and split_count set). */
int fa_kv_combine(const fa_kvcache_args *args, void *stream);
/* append + split-KV + combine in stream order (with batch_order the append and the
 * ordering share one launch). */
int fa_fwd_kvcache(const fa_kvcache_args *args, void *stream);

/*
 * Allocation-free variant of fa_fwd_kvcache.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  The
 * same kernels run; out_accum, lse_accum, batch_order and split_count in args
 * are ignored and taken instead from a static device array of
 * FA_NOALLOC_SCRATCH_BYTES per device, held until the process ends (the calling
 * thread's current device must be the stream's).  A request needing more than
 * that, i.e. fa_kv_workspace_bytes(args) + 4 * (batch + 1 +
 * fa_kv_split_count_len(args)) bytes, returns FA_ERR_SCRATCH.
 * No allocation or free happens in the call.  Calls on one device share its
 * array: calls that overlap on one device (on different streams) race.
 */
#define FA_NOALLOC_SCRATCH_BYTES (16u << 20)
int fa_fwd_kvcache_noalloc(const fa_kvcache_args *args, void *stream);

/* Human-readable text for a return code (FA_* or hipError_t). */
const char *fa_error_string(int code);

/*
 * Version of the argument-struct layouts above.  It changes whenever a struct
 * gains, loses or moves a field (3: fa_fwd_args.work_order, fa_bwd_args.work_order
 * and fa_kvcache_args.split_count appended).  A caller compiled against this
 * header checks fa_abi_version() == FA_ABI_VERSION once after loading the
 * library and refuses a mismatch: the entry points themselves cannot tell a
 * shorter struct from an older caller.  No counterpart in the reference (its
 * bindings are compiled together with its kernels).
 */
#define FA_ABI_VERSION 3
int fa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FA_MI355X_H */
