// KV-cache attention for gfx950 (MI355X): in-place append, split-KV partial
// attention over contiguous / remapped / paged caches, log-sum-exp combine.
//
// Replaces csrc/flash_attn/src/kvcache_native.cu: paged_append_kernel
// (:782-871), the contiguous append loop of flash_api.cpp:643-654, the split
// kernels (:148-674) and kvcache_combine_kernel (:676-729).  Semantics kept:
// attention over L = cache_seqlens[b] + seqlen_new keys; split s of S covers
// [L*s/S, L*(s+1)/S) (:191-192); causal keeps key j for query row i iff
// j <= i + L - seqlen_q (:347); GQA kv_head = head / (h/hk) (:341); an empty
// split has LSE -inf and output 0 (:355-372); the combine weights are
// exp(lse_s - lse_total) and a row with no key gets O = 0, LSE = 0 (:697-727);
// probabilities stay fp32 through the PV product (:599, :636-672).
//
// Design: one workgroup per (batch, group of HPI adjacent KV heads, split,
// 32-row tile) where the rows are the q-heads of the GQA group times the query
// positions, so every K/V byte of the split is read once.  The keys of the
// split are walked in 32-key tiles aligned to absolute positions (a tile never
// straddles a page: pages are multiples of 256 tokens); wave w serves head
// w % HPI of the group and its tiles t with t % (4 / HPI) == w / HPI (HPI = 1:
// one head, tile t to wave t % 4).  Each wave
// streams its tiles through a private LDS slot with direct global -> LDS
// copies (global_load_lds): it reads a tile's MFMA operands into registers,
// issues the next tile's copy into the same slot and then computes, so the
// copy is in flight during the compute, with no register staging of the copy
// and no workgroup barrier in the loop.  K stays natural (MFMA A operand
// rows), V natural and read transposed with ds_read_b64_tr_b16.  Each wave
// keeps its own online softmax state; the waves of each head merge their
// partial states through LDS at the end.  Paged, remapped and contiguous
// caches with the same head stride take the same tile order and the same
// arithmetic, so their results are bit-identical for the same logical cache.
// Work items are ordered with the sequence rank slowest: when the caller
// passes a batch_order workspace, one
// workgroup of the append launch first ranks the sequences by key count
// (longest first) and a resident grid of two workgroups per CU deals the items
// out from a device counter in that order, so the longest sequences start
// first, the short ones fill the end, and no workgroup is relaunched between
// items.  With split counts as well, the last split item of each row tile to
// finish combines the tile's partials, so a decode call is two launches.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "fa_common.h"

// The split kernel's fused combine publishes partials with relaxed agent-scope
// atomics and relies on gfx950's write-through of agent-scope stores (see
// kv_splitkv_kernel); this file is built for gfx950 only.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "fa_kvcache.hip targets gfx950: its fused combine relies on gfx950's agent-scope store visibility"
#endif

namespace fa {

constexpr int kKvThreads = 256;
constexpr int kKvWaves = 4;
constexpr int kTile = 32;  // keys per wave tile

__device__ __forceinline__ const f16 *kv_row_ptr(const fa_tensor &t, const fa_kvcache_args &a, int b, int cache_row,
                                                 int hk, int pos) {
    // Element pointer of token `pos` (logical) of sequence b, head hk.
    int64_t off;
    if (a.block_table) {
        const int page = a.page_block_size;
        const int blk = a.block_table[int64_t(b) * a.block_table_stride + pos / page];
        off = int64_t(blk) * t.batch_stride + int64_t(pos % page) * t.row_stride;
    } else {
        off = int64_t(cache_row) * t.batch_stride + int64_t(pos) * t.row_stride;
    }
    return (const f16 *)t.ptr + off + int64_t(hk) * t.head_stride;
}

// Cache length and cache row of sequence b, checked against the cache: a
// negative length, more tokens than the cache holds after the append, or a
// row outside a remapped cache makes the sequence invalid (err bit 1:
// capacity, bit 2: row).  An invalid sequence is not appended to and is
// attended over no keys, so no access leaves the cache whatever the lengths
// and indices hold; the host learns of it from the status word.
struct KvSeq {
    int L0;   // tokens in the cache before the append (0 when invalid)
    int row;  // cache row (contiguous cache)
    int err;
};
__device__ __forceinline__ KvSeq kv_seq(const fa_kvcache_args &a, int b) {
    KvSeq s;
    s.L0 = a.cache_seqlens[b];
    s.row = a.cache_batch_idx ? a.cache_batch_idx[b] : b;
    s.err = (s.L0 < 0 || (a.cache_capacity > 0 && int64_t(s.L0) + a.seqlen_new > a.cache_capacity) ? 1 : 0) |
            (a.cache_batch_idx && a.cache_batch > 0 && (s.row < 0 || s.row >= a.cache_batch) ? 2 : 0);
    if (s.err) {
        s.L0 = 0;
        s.row = 0;
    }
    return s;
}

// Rotary embedding of the 8 channels [c0, c0 + 8) of one row (c0 a multiple of
// 8 below rotary_dim) at position pos: x holds them, row points at channel 0
// of the row (the non-interleaved form reads the partner channels there).
// Each output is x_a * cos - x_b * sin or x_a * sin + x_b * cos in fp32; the
// products of fp16 values are exact in fp32, so it is the exact rotation of
// the fp16 inputs rounded once to fp32, then to fp16.
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 rotary8(const fa_kvcache_args &a, const u32x4 x, const f16 *row, int c0, int pos) {
    // Opaque to the optimiser: keeps the per-channel table addresses from being
    // hoisted out of the split kernel's item loop, where they would stay live
    // (in spilled registers) through it.
    asm volatile("" : "+v"(c0));
    const int half = a.rotary_dim / 2;
    const int64_t base = int64_t(min(max(pos, 0), a.rotary_seqlen - 1)) * half;
    const f16 *cs = (const f16 *)a.rotary_cos + base;
    const f16 *sn = (const f16 *)a.rotary_sin + base;
    const f16x8 xv = as_h8(x);
    f16x8 r;
    if (a.rotary_interleaved) {
        const f16x4 c = *reinterpret_cast<const f16x4 *>(cs + c0 / 2);
        const f16x4 s = *reinterpret_cast<const f16x4 *>(sn + c0 / 2);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float x0 = float(xv[2 * e]), x1 = float(xv[2 * e + 1]);
            const float ce = float(c[e]), se = float(s[e]);
            r[2 * e] = f16(x0 * ce - x1 * se);
            r[2 * e + 1] = f16(x0 * se + x1 * ce);
        }
    } else {
        const bool first = c0 < half;
        const int j0 = first ? c0 : c0 - half;
        const f16x8 pv = as_h8(ldg16(row + (first ? c0 + half : j0)));
        const f16x8 c = as_h8(ldg16(cs + j0));
        const f16x8 s = as_h8(ldg16(sn + j0));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float xe = float(xv[e]), pe = float(pv[e]), ce = float(c[e]), se = float(s[e]);
            r[e] = f16(first ? xe * ce - pe * se : xe * ce + pe * se);
        }
    }
    return __builtin_bit_cast(u32x4, r);
}

// ---------------------------------------------------------------------------
// Append of 16-byte chunk idx of k_new / v_new, one per thread (with
// rotary_dim > 0, the key chunks below rotary_dim are rotated at their
// position first).
template <int HD>
__device__ __forceinline__ void append_chunk(const fa_kvcache_args &a, const int64_t idx) {
    constexpr int KCH = HD / 8;
    const int64_t total = int64_t(a.batch) * a.seqlen_new * a.nheads_k * KCH;
    if (idx >= total) return;
    const int c = int(idx % KCH);
    int64_t rest = idx / KCH;
    const int hk = int(rest % a.nheads_k);
    rest /= a.nheads_k;
    const int t = int(rest % a.seqlen_new);
    const int b = int(rest / a.seqlen_new);
    const KvSeq sq = kv_seq(a, b);
    if (sq.err) {
        if (a.status && idx % (int64_t(a.seqlen_new) * a.nheads_k * KCH) == 0) atomicOr(a.status, sq.err);
        return;
    }
    const int pos = sq.L0 + t;
    const int cache_row = sq.row;
    const f16 *ks = (const f16 *)a.k_new.ptr + int64_t(b) * a.k_new.batch_stride + int64_t(t) * a.k_new.row_stride +
                    int64_t(hk) * a.k_new.head_stride + 8 * c;
    const f16 *vs = (const f16 *)a.v_new.ptr + int64_t(b) * a.v_new.batch_stride + int64_t(t) * a.v_new.row_stride +
                    int64_t(hk) * a.v_new.head_stride + 8 * c;
    f16 *kd = const_cast<f16 *>(kv_row_ptr(a.k_cache, a, b, cache_row, hk, pos)) + 8 * c;
    f16 *vd = const_cast<f16 *>(kv_row_ptr(a.v_cache, a, b, cache_row, hk, pos)) + 8 * c;
    u32x4 kx = ldg16(ks);
    if (8 * c < a.rotary_dim) kx = rotary8(a, kx, ks - 8 * c, 8 * c, pos);
    *reinterpret_cast<u32x4 *>(kd) = kx;
    *reinterpret_cast<u32x4 *>(vd) = ldg16(vs);
}

// ---------------------------------------------------------------------------
// Append and ordering in one launch of kOrderThreads-thread workgroups.  The
// first order_wgs workgroups (0 or 1) rank the sequences: batch_order[r] = the
// sequence with the r-th most keys, by a counting sort over key-count buckets
// (exact below 32 keys, then 32 buckets per power of two: about 3 % apart;
// order within a bucket is arbitrary, which changes no result), and zero the
// split kernel's work counter batch_order[batch] and its n_count split counts.
// The other workgroups append one 16-byte chunk per thread.  The two parts
// touch disjoint memory (the ranking reads cache_seqlens only).
__device__ __forceinline__ int kv_len_bucket(int n) {
    if (n < 32) return n;
    const int msb = 31 - __clz(n);
    return (msb - 4) * 32 + ((n >> (msb - 5)) & 31);
}
template <int HD>
__global__ __launch_bounds__(kOrderThreads) void kv_prep_kernel(const fa_kvcache_args a, const int order_wgs,
                                                                int32_t *const count, const int n_count) {
    if (int(blockIdx.x) < order_wgs) {
        if (threadIdx.x == 0) a.batch_order[a.batch] = 0;
        for (int i = threadIdx.x; i < n_count; i += kOrderThreads) count[i] = 0;
        order_items(
            a.batch,
            [&](int b) {
                const KvSeq sq = kv_seq(a, b);
                return kv_len_bucket(sq.err ? 0 : sq.L0 + a.seqlen_new);
            },
            a.batch_order, true);
        return;
    }
    append_chunk<HD>(a, int64_t(blockIdx.x - order_wgs) * kOrderThreads + threadIdx.x);
}

// ---------------------------------------------------------------------------
// Combine of one output row r (of batch * nheads * seqlen_q) by one wave.  Lane
// s reads split s's LSE (further rounds past 64 splits) while the partial
// outputs of the first kPreSplits splits are loaded at the same time; the
// maximum and the weight sum are wave reductions, and each lane sums HD / 64
// output elements over the splits with the weight exp(lse_s - lse_total)
// taken from lane s.  Run by the combine kernel, or inside the split kernel by
// the last split item of a row tile.
constexpr int kPreSplits = 16;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

// Split partials as the combine reads them.  Inside the split kernel
// (COHERENT) they are device-scope atomic loads, which see what device-scope
// stores of other workgroups left whatever this XCD's L2 holds (the partials
// are stored that way); the combine kernel, launched after the split kernel,
// reads them plainly.
template <bool COHERENT>
__device__ __forceinline__ float load_part(const float *p) {
    if constexpr (COHERENT)
        return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        return *p;
}
template <bool COHERENT, int DPL>
__device__ __forceinline__ float __attribute__((ext_vector_type(DPL))) load_part_vec(const float *p) {
    typedef float fdpl __attribute__((ext_vector_type(DPL)));
    if constexpr (!COHERENT) {
        return *reinterpret_cast<const fdpl *>(p);
    } else if constexpr (DPL == 1) {
        fdpl v;
        v[0] = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return v;
    } else {
        static_assert(DPL == 2, "one 64-bit load per lane");
        const uint64_t u =
            __hip_atomic_load(reinterpret_cast<const uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return __builtin_bit_cast(fdpl, u);
    }
}

template <int HD, bool COHERENT>
__device__ __forceinline__ void combine_row(const fa_kvcache_args &a, const int r, int lane) {
    // Opaque to the optimiser: keeps the addresses below from being hoisted out
    // of the split kernel's item loop into registers live through its tile loop.
    asm volatile("" : "+v"(lane));
    constexpr int DPL = HD / 64;  // output elements per lane
    typedef float fdpl __attribute__((ext_vector_type(DPL)));
    const int nrow = a.batch * a.nheads * a.seqlen_q;
    const int S = a.num_splits;
    auto part = [&](int s) {
        return load_part_vec<COHERENT, DPL>(a.out_accum + (int64_t(s) * nrow + r) * HD + DPL * lane);
    };
    auto lse_of = [&](int s) { return load_part<COHERENT>(a.lse_accum + int64_t(s) * nrow + r); };
    // Splits past S re-read split S - 1 (finite) and get weight 0 below.
    fdpl pre[kPreSplits];
#pragma unroll
    for (int s = 0; s < kPreSplits; ++s) pre[s] = part(min(s, S - 1));
    const float lse0 = lane < S ? lse_of(lane) : -INFINITY;
    float lmax = lse0;
    for (int s0 = 64; s0 < S; s0 += 64)
        if (s0 + lane < S) lmax = fmaxf(lmax, lse_of(s0 + lane));
    lmax = wave_max(lmax);
    float psum = 0.f;
    if (lmax != -INFINITY) {
        if (lane < S) psum = expf(lse0 - lmax);
        for (int s0 = 64; s0 < S; s0 += 64)
            if (s0 + lane < S) psum += expf(lse_of(s0 + lane) - lmax);
    }
    const float wsum = wave_sum(psum);
    const bool live = lmax != -INFINITY && wsum > 0.f;
    const float ltot = live ? lmax + logf(wsum) : -INFINITY;
    fdpl acc;
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
    if (live) {
        const float w0 = lane < S ? expf(lse0 - ltot) : 0.f;
        auto weight = [](float w, int s) {
            return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), s));
        };
#pragma unroll
        for (int s = 0; s < kPreSplits; ++s) acc += weight(w0, s) * pre[s];  // lane s >= S holds w0 = 0
        for (int s0 = 0; s0 < S; s0 += 64) {
            const float w = s0 == 0 ? w0 : (s0 + lane < S ? expf(lse_of(s0 + lane) - ltot) : 0.f);
            const int n = min(64, S - s0);
#pragma unroll 1
            for (int s = s0 == 0 ? kPreSplits : 0; s < n; ++s) acc += weight(w, s) * part(s0 + s);
        }
    }
    const int qp = r % a.seqlen_q;
    const int bh = r / a.seqlen_q;
    const int h = bh % a.nheads, b = bh / a.nheads;
    f16 *op = (f16 *)a.o.ptr + int64_t(b) * a.o.batch_stride + int64_t(qp) * a.o.row_stride +
              int64_t(h) * a.o.head_stride + DPL * lane;
#pragma unroll
    for (int i = 0; i < DPL; ++i) op[i] = (f16)acc[i];
    if (lane == 0) a.lse[r] = live ? ltot : 0.f;
}

// ---------------------------------------------------------------------------
// Split-KV partial attention.
template <int HD>
struct KvCfg {
    static constexpr int KCH = HD / 8;
    static constexpr int TILE = kTile * HD * 2;         // one K or V tile, natural layout
    static constexpr int STAGE = 2 * TILE;              // K tile, then V tile
    // Ring stages per wave.  A tile's operands are read into registers and the
    // stage is refilled before the tile is computed, so one stage keeps a tile
    // in flight; at head_dim 64 a second stage (more bytes in flight, +1 % on a
    // long-context decode) still lets two workgroups share a CU, at 128 it
    // would not (one's start-up and merge overlap the other's streaming).
    static constexpr int NST = HD == 64 ? 2 : 1;
    static constexpr int WAVE_LDS = NST * STAGE;        // also holds HD x 32 fp32 at the merge
    static constexpr int CPW = kTile * KCH / 64;        // copies per lane per tile (K or V)
    static constexpr int MAX_PAGES = 1024;              // page ids of one split staged in LDS
};

// The running maximum m that a row's probabilities P = exp2(S*c - m) are taken
// against is raised (and O, l rescaled) only when some row of the wave finds a
// score more than this many doublings above it; P stays below 2^8, and its hi +
// lo fp16 halves still carry about 22 bits.
constexpr float kKvRescaleSlack = 8.f;

// tanh x = 1 - 2 / (e^(2x) + 1): exactly +-1 at the ends, an absolute error of a
// few fp32 ulps of 1 in between (what a softcapped score needs).
__device__ __forceinline__ float tanh_fast(float x) {
    const float e = exp2_fast(x * (2.f * kLog2e));
    return 1.f - 2.f * __builtin_amdgcn_rcpf(e + 1.f);
}

// Work items are (sequence rank, split, kv head, row tile), rank slowest: with
// batch_order the longest sequences' items come first (longest-job-first keeps
// the last items short).  With DYN the grid is resident (two workgroups per
// CU) and each workgroup, after its first item blockIdx.x, takes the next
// unclaimed item from a device counter, so no workgroup is relaunched and
// the items are dealt out greedily in that order.  The counter
// (batch_order[batch]) is zeroed by kv_prep_kernel on the same stream.
// With count (num_splits > 1, DYN) the split kernel also combines: count[(b *
// nheads_k + hk) * row_tiles + rt] (zeroed by kv_prep_kernel) counts the
// finished splits of that row tile, and the item that finishes last combines
// the tile's rows with combine_row, as the combine kernel would.
// EXT switches on the local window, softcap, ALiBi, cache_leftpad and rotary options
// (a separate instance, so the plain kernel carries none of their work).
// HPI (1, 2 or 4) KV heads per item: wave w serves head hk0 + w % HPI and
// takes every (4 / HPI)-th tile of it, so at one key position the waves of a
// workgroup read HPI adjacent heads' rows, HPI * head_dim * 2 contiguous bytes
// of a head-interleaved cache row, where one head alone reads 128 or 256.
template <int HD, bool DYN, bool EXT, int HPI>
__global__ __launch_bounds__(256, 2) void kv_splitkv_kernel(const fa_kvcache_args a, const int row_tiles,
                                                            const int n_items, int32_t *const count) {
    using C = KvCfg<HD>;
    static_assert(HPI == 1 || HPI == 2 || HPI == 4, "heads per item");
    constexpr int WPH = kKvWaves / HPI;  // waves per head
    __shared__ __attribute__((aligned(16))) char smem[kKvWaves * C::WAVE_LDS + kKvWaves * 2 * 32 * 4];
    __shared__ int pages[C::MAX_PAGES];
    __shared__ int next_item, last_item;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar loop control
    const int col = lane & 31, hh = lane >> 5;
    const int n_groups = a.nheads_k / HPI;
    for (int item = blockIdx.x; item < n_items;) {
        int rest = item;
        const int rt = rest % row_tiles;
        rest /= row_tiles;
        const int hk0 = (rest % n_groups) * HPI;  // the item's first KV head
        const int hk = hk0 + wave % HPI;          // this wave's
        rest /= n_groups;
        const int split = rest % a.num_splits;
        const int rank = rest / a.num_splits;
        const int b = a.batch_order ? a.batch_order[rank] : rank;
        const int G = a.nheads / a.nheads_k;
        const int R = G * a.seqlen_q;  // rows of this (batch, kv head): row = qpos * G + g

        const KvSeq sq = kv_seq(a, b);
        if (sq.err && a.status && tid == 0) atomicOr(a.status, sq.err);
        const int L = sq.err ? 0 : sq.L0 + a.seqlen_new;
        const int S = a.num_splits;
        // Valid keys [kstart, L): cache_leftpad moves the start, positions stay.
        const int kstart = EXT && a.cache_leftpad ? min(max(a.cache_leftpad[b], 0), L) : 0;
        const int s0 = kstart + int((int64_t(L - kstart) * split) / S);
        const int s1 = kstart + int((int64_t(L - kstart) * (split + 1)) / S);
        const int cache_row = sq.row;

        // This lane's query row.
        const int row = rt * 32 + col;
        const bool row_ok = row < R;
        const int qpos = row_ok ? row / G : 0;
        const int hq = hk * G + (row_ok ? row % G : 0);
        int lim = a.causal ? qpos + L - a.seqlen_q : L - 1;  // last visible key
        int w_lo = 0;                                          // first visible key
        // Keys whose tiles this item walks: the split, narrowed to the union of
        // its rows' windows.
        int k_lo = s0, k_hi = s1;
        // Wave-uniform bounds of the keys every row of the tile sees: tiles in
        // [max(s0, wlo_max), min(s1, lim_min + 1)) need no mask.
        const int p_first = (rt * 32) / G + L - a.seqlen_q;  // smallest query position of the tile
        int lim_min = a.causal ? p_first : L - 1;
        int wlo_max = 0;
        if constexpr (EXT) {
            if (a.local_window) {
                const int p_last = (min(R, rt * 32 + 32) - 1) / G + L - a.seqlen_q;
                if (a.window_right >= 0) lim_min = min(lim_min, p_first + a.window_right);
                if (a.window_left >= 0) wlo_max = p_last - a.window_left;
            }
        }
        if constexpr (EXT) {
            if (a.local_window) {
                const int pos = qpos + L - a.seqlen_q;  // the query's own key position
                if (a.window_right >= 0) lim = min(lim, pos + a.window_right);
                if (a.window_left >= 0) w_lo = pos - a.window_left;
                const int p_lo = (rt * 32) / G + L - a.seqlen_q;
                const int p_hi = (min(R, rt * 32 + 32) - 1) / G + L - a.seqlen_q;
                int hi = a.causal ? p_hi : L - 1;
                if (a.window_right >= 0) hi = min(hi, p_hi + a.window_right);
                if (a.window_left >= 0) k_lo = max(k_lo, p_lo - a.window_left);
                k_hi = max(k_lo, min(k_hi, hi + 1));
            }
        }

        const bool neg = a.softmax_scale < 0.f;
        const bool capped = EXT && a.softcap > 0.f;
        const bool alibi = EXT && a.alibi_slopes != nullptr;
        // Softcapped or biased scores are formed in natural units (scaled), so
        // the exponent multiplier is log2(e) for them and scale * log2(e)
        // otherwise; cap_in = scale / softcap.
        const bool natural = capped || alibi;
        const float cscale = natural ? kLog2e : fabsf(a.softmax_scale) * kLog2e;
        const float cap_in = capped ? fabsf(a.softmax_scale) / a.softcap : 0.f;
        const float slope = alibi ? a.alibi_slopes[int64_t(b) * a.alibi_batch_stride + hq] : 0.f;
        const int qkey = qpos + L - a.seqlen_q;  // the query's own key position (ALiBi distance origin)
        // Rotary position of the query: its own (cache_seqlens + i) when causal
        // or windowed, else cache_seqlens for every row.
        const int rpos = sq.L0 + (a.causal || a.local_window ? qpos : 0);
        f16x8 qB[HD / 16];
        {
            const f16 *qp = (const f16 *)a.q.ptr + int64_t(b) * a.q.batch_stride + int64_t(qpos) * a.q.row_stride +
                            int64_t(hq) * a.q.head_stride;
    #pragma unroll
            for (int g = 0; g < HD / 16; ++g) {
                u32x4 v = row_ok ? ldg16(qp + 16 * g + 8 * hh) : zero_u4();
                if (EXT && row_ok && 16 * g + 8 * hh < a.rotary_dim) v = rotary8(a, v, qp, 16 * g + 8 * hh, rpos);
                if (neg) v = neg_h8(v);
                qB[g] = as_h8(v);
            }
        }

        f32x16 o[HD / 32];
    #pragma unroll
        for (int i = 0; i < HD / 32; ++i) o[i] = zero16();
        float m_t = -INFINITY, l_p = 0.f;

        const int t_first = k_lo / kTile;
        const int t_last = k_hi > k_lo ? (k_hi - 1) / kTile : t_first - 1;
        const int my_first = t_first + wave / HPI;
        const int n_my = my_first <= t_last ? (t_last - my_first) / WPH + 1 : 0;

        // Page ids of the split, staged in LDS so the ring never waits on a table read.
        const int page = a.page_block_size;
        const int pg_first = a.block_table ? (t_first * kTile) / page : 0;
        const int n_pages = a.block_table && k_hi > k_lo ? (t_last * kTile) / page - pg_first + 1 : 0;
        const bool pages_in_lds = n_pages <= C::MAX_PAGES;
        if (a.block_table && pages_in_lds) {
            const int32_t *bt = a.block_table + int64_t(b) * a.block_table_stride + pg_first;
            // Opaque start index: keeps this loop's per-lane addresses from being
            // hoisted out of the item loop (and spilled in the options instance).
            int i0 = tid;
            asm volatile("" : "+v"(i0));
            for (int i = i0; i < n_pages; i += kKvThreads) pages[i] = bt[i];
        }
        __syncthreads();

        const int64_t krs = a.k_cache.row_stride, vrs = a.v_cache.row_stride;

        // The tile loop, instantiated twice: with the split's page ids in LDS (and
        // no other vector-memory load while copies are in flight), and a fallback
        // that reads the block table per tile for splits spanning more pages.
        auto run = [&](auto lds_pages_tag) {
        constexpr bool LDS_PAGES = decltype(lds_pages_tag)::value;
        // Copy tile t into ring stage st of this wave.  Rows past L re-read key L - 1
        // of the same tile (finite values; masked below).
        auto issue = [&](int t, int st) {
            const int p0 = t * kTile;
            int64_t koff, voff;
            if (a.block_table) {
                const int pi = p0 / page;
                int blk;
                if constexpr (LDS_PAGES)
                    blk = pages[pi - pg_first];
                else
                    blk = a.block_table[int64_t(b) * a.block_table_stride + pi];
                const int in_page = p0 - pi * page;
                koff = int64_t(blk) * a.k_cache.batch_stride + int64_t(in_page) * krs;
                voff = int64_t(blk) * a.v_cache.batch_stride + int64_t(in_page) * vrs;
            } else {
                koff = int64_t(cache_row) * a.k_cache.batch_stride + int64_t(p0) * krs;
                voff = int64_t(cache_row) * a.v_cache.batch_stride + int64_t(p0) * vrs;
            }
            const f16 *kb = (const f16 *)a.k_cache.ptr + koff + int64_t(hk) * a.k_cache.head_stride;
            const f16 *vb = (const f16 *)a.v_cache.ptr + voff + int64_t(hk) * a.v_cache.head_stride;
            char *ks = smem + (wave * C::NST + st) * C::STAGE;
            char *vs = ks + C::TILE;
            dma_tile<HD, kTile, 64>(ks, kb, krs, 0, L - 1 - p0, 0, lane);
            dma_tile<HD, kTile, 64>(vs, vb, vrs, 0, L - 1 - p0, 0, lane);
        };

        TileReader<HD> rd;
        rd.init(lane);
        if (n_my > 0) issue(my_first, 0);
        if (C::NST > 1 && n_my > 1) issue(my_first + WPH, 1);
        for (int k = 0; k < n_my; ++k) {
            const int st = k % C::NST;
            if (k + 1 < n_my)
                wait_vmem_n<(C::NST - 1) * 2 * C::CPW>();  // newer tiles may stay in flight
            else
                wait_vmem();
            const char *ks = smem + (wave * C::NST + st) * C::STAGE;
            const char *vs = ks + C::TILE;
            const int p0 = (my_first + k * WPH) * kTile;
            // All operands of the tile into registers first, then refill the stage
            // right away: two tiles stay in flight while this one is computed.
            f16x8 ka[HD / 16], va[HD / 32][2];
    #pragma unroll
            for (int g = 0; g < HD / 16; ++g) ka[g] = rd.a_operand(ks, 0, g);
    #pragma unroll
            for (int dt = 0; dt < HD / 32; ++dt)
    #pragma unroll
                for (int gg = 0; gg < 2; ++gg) va[dt][gg] = rd.tr_operand(vs, 16 * gg, dt);
            wait_lds();
            if (k + C::NST < n_my) issue(my_first + (k + C::NST) * WPH, st);
            f32x16 s = mfma32(ka[0], qB[0], zero16());
    #pragma unroll
            for (int g = 1; g < HD / 16; ++g) s = mfma32(ka[g], qB[g], s);
            if constexpr (EXT) {
                if (natural) {
                    const float sc = fabsf(a.softmax_scale);
    #pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        float x = capped ? a.softcap * tanh_fast(s[r] * cap_in) : s[r] * sc;
                        if (alibi) x -= slope * float(abs(qkey - (p0 + acc_lrow(r, hh))));
                        s[r] = x;
                    }
                }
            }
            float mx = -INFINITY;
            const bool interior = p0 >= s0 && p0 + kTile <= s1 && p0 + kTile - 1 <= lim_min && p0 >= wlo_max;
            if (interior) {
    #pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
            } else {
    #pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = p0 + acc_lrow(r, hh);
                    if (key < s0 || key >= s1 || key > lim || (EXT && key < w_lo)) s[r] = -INFINITY;
                    mx = fmaxf(mx, s[r]);
                }
            }
            mx = max_xor32(mx);
            const float mx_t = mx == -INFINITY ? -INFINITY : mx * cscale;
            if (__builtin_amdgcn_ballot_w64(mx_t > m_t + kKvRescaleSlack) != 0) {
                const float m_new = fmaxf(m_t, mx_t);
                const float alpha = m_new == -INFINITY ? 1.f : exp2_fast(m_t - m_new);
                l_p *= alpha;
    #pragma unroll
                for (int dt = 0; dt < HD / 32; ++dt)
    #pragma unroll
                    for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
                m_t = m_new;
            }
            const float m_use = m_t == -INFINITY ? 0.f : m_t;
            // A masked score is -inf after every transform, and exp2(-inf) = 0.
            float rs = 0.f;
    #pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = exp2_fast(fmaf(s[r], cscale, -m_use));
                s[r] = p;
                rs += p;
            }
            l_p += rs;
            // P stays fp32-accurate through the product: P = hi + lo with both halves fp16.
            f16x8 ph[2], pl[2];
    #pragma unroll
            for (int gg = 0; gg < 2; ++gg)
    #pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const float p = s[8 * gg + u];
                    const f16 hi = (f16)p;
                    ph[gg][u] = hi;
                    pl[gg][u] = (f16)(p - float(hi));
                }
    #pragma unroll
            for (int dt = 0; dt < HD / 32; ++dt) {
    #pragma unroll
                for (int gg = 0; gg < 2; ++gg) {
                    o[dt] = mfma32(va[dt][gg], ph[gg], o[dt]);
                    o[dt] = mfma32(va[dt][gg], pl[gg], o[dt]);
                }
            }
        }
        };
        if (pages_in_lds)
            run(std::true_type{});
        else
            run(std::false_type{});

        // Merge the waves of each head (waves j, j + HPI, ...): each publishes
        // (m, l) per row and its O^T tile.
        const float l_w = sum_xor32(l_p);
        float *mrow = reinterpret_cast<float *>(smem + kKvWaves * C::WAVE_LDS);
        float *lrow = mrow + kKvWaves * 32;
        __syncthreads();  // every wave is done with its ring
        float *ow = reinterpret_cast<float *>(smem + wave * C::WAVE_LDS);  // [HD][32] fp32
    #pragma unroll
        for (int dt = 0; dt < HD / 32; ++dt)
    #pragma unroll
            for (int r = 0; r < 16; ++r) ow[(dt * 32 + acc_row(r, hh)) * 32 + col] = o[dt][r];
        if (hh == 0) {
            mrow[wave * 32 + col] = m_t;
            lrow[wave * 32 + col] = l_w;
        }
        __syncthreads();

        const int rows_here = min(32, R - rt * 32);
        const int nrow_all = a.batch * a.nheads * a.seqlen_q;
        for (int e = tid; e < HPI * rows_here * HD; e += kKvThreads) {
            const int j = e / (rows_here * HD), c = (e / HD) % rows_here, d = e % HD;
            float mstar = -INFINITY;
    #pragma unroll
            for (int i = 0; i < WPH; ++i) mstar = fmaxf(mstar, mrow[(j + HPI * i) * 32 + c]);
            float lsum = 0.f, acc = 0.f;
            if (mstar != -INFINITY) {
    #pragma unroll
                for (int i = 0; i < WPH; ++i) {
                    const int w = j + HPI * i;
                    const float mw = mrow[w * 32 + c];
                    const float sc = mw == -INFINITY ? 0.f : exp2_fast(mw - mstar);
                    lsum += lrow[w * 32 + c] * sc;
                    acc += reinterpret_cast<const float *>(smem + w * C::WAVE_LDS)[d * 32 + c] * sc;
                }
            }
            const bool live = lsum > 0.f;
            const float outv = live ? acc / lsum : 0.f;
            const float lse = live ? (mstar + log2_fast(lsum)) * kLn2 : -INFINITY;
            const int r = rt * 32 + c;
            const int qp = r / G, h = (hk0 + j) * G + r % G;
            const int64_t orow = (int64_t(b) * a.nheads + h) * a.seqlen_q + qp;  // (batch, head, qpos)
            if (S == 1) {
                f16 *op = (f16 *)a.o.ptr + int64_t(b) * a.o.batch_stride + int64_t(qp) * a.o.row_stride +
                          int64_t(h) * a.o.head_stride;
                op[d] = (f16)outv;
                if (d == 0) a.lse[orow] = live ? lse : 0.f;
            } else {
                // Device-scope stores: the last split item of the tile may combine
                // them on another XCD in this same launch.
                __hip_atomic_store(a.out_accum + (int64_t(split) * nrow_all + orow) * HD + d, outv, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                if (d == 0)
                    __hip_atomic_store(a.lse_accum + int64_t(split) * nrow_all + orow, lse, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        if (DYN && S > 1 && count) {
            // The item counts itself done once every wave's partial stores have
            // completed (vmcnt 0: written at device scope); the item that brings
            // the count to S has seen all S items' stores complete and reads the
            // partials with device-scope loads.  No cache-wide write-back or
            // invalidate is needed (both would stall this XCD's L2 once per item).
            // This rests on gfx950's agent-scope accesses, not on the HIP memory
            // model (the atomics are relaxed): an agent-scope store is written
            // past the XCD's L2 before its vmcnt completes, and an agent-scope
            // load does not hit another XCD's stale L2 copy; the #error at the
            // top of this file keeps other targets from building it.  The count
            // of a row tile of a head group sits at its first head's slot.
            wait_vmem();
            __syncthreads();
            if (tid == 0)
                last_item = __hip_atomic_fetch_add(count + (int64_t(b) * a.nheads_k + hk0) * row_tiles + rt, 1,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
            __syncthreads();
            if (last_item) {
                for (int c = wave; c < HPI * rows_here; c += kKvWaves) {
                    const int j = c / rows_here, r = rt * 32 + c % rows_here;
                    combine_row<HD, true>(a, (b * a.nheads + (hk0 + j) * G + r % G) * a.seqlen_q + r / G, lane);
                }
            }
        }
        if constexpr (!DYN) break;
        __syncthreads();  // every thread is done with this item's LDS
        if (tid == 0) next_item = atomicAdd(a.batch_order + a.batch, 1) + int(gridDim.x);
        __syncthreads();
        item = next_item;
    }
}

// ---------------------------------------------------------------------------
// Combine kernel: one wave per (batch, head, qpos) row.
template <int HD>
__global__ __launch_bounds__(256) void kv_combine_kernel(const fa_kvcache_args a) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= a.batch * a.nheads * a.seqlen_q) return;
    combine_row<HD, false>(a, r, threadIdx.x & 63);
}

static int check_kv(const fa_kvcache_args *p) {
    if (!p) return FA_ERR_INVALID_ARG;
    const fa_kvcache_args &a = *p;
    if (a.head_dim != 64 && a.head_dim != 128) return FA_ERR_UNSUPPORTED;
    if (a.batch < 0 || a.seqlen_q < 0 || a.nheads <= 0 || a.nheads_k <= 0 || a.nheads % a.nheads_k != 0 ||
        a.seqlen_new < 0 || a.num_splits < 1 || !a.cache_seqlens || !a.lse)
        return FA_ERR_INVALID_ARG;
    if (a.block_table && (a.page_block_size <= 0 || a.page_block_size % kTile != 0)) return FA_ERR_INVALID_ARG;
    if (a.block_table && a.cache_batch_idx) return FA_ERR_INVALID_ARG;
    if (!(a.softcap >= 0.f) || a.softcap == INFINITY) return FA_ERR_INVALID_ARG;  // NaN fails too
    if (a.rotary_dim != 0 &&
        (a.rotary_dim < 0 || a.rotary_dim % 16 != 0 || a.rotary_dim > a.head_dim || a.rotary_seqlen < 1 ||
         !a.rotary_cos || !a.rotary_sin || !a.k_new.ptr ||
         ((reinterpret_cast<uintptr_t>(a.rotary_cos) | reinterpret_cast<uintptr_t>(a.rotary_sin)) & 15u)))
        return FA_ERR_INVALID_ARG;
    return FA_OK;
}

}  // namespace fa

extern "C" int fa_kv_num_splits(int requested, int seqlen_k_capacity, int head_dim, int seqlen_q, int batch,
                                int nheads, int nheads_k, int num_cus) {
    // An explicit request is honoured (kvcache_native.cu:922-924).  Otherwise
    // (measured on MI355X over paged and contiguous decode shapes) a work item
    // streams best with about 8192 cache positions: fewer and the per-item
    // start-up and the combine weigh in, more and the longest-first deal
    // balances worse.  Enough splits are also taken for one item per compute
    // unit, and a split keeps at least 512 positions, or, for a cache of 512
    // positions or more cut into at most 16 splits, at least 64 (a short cache
    // on few sequences: one sequence of 1024 positions, 32 / 8 heads, takes
    // 15.5 us per call in 16 splits against 20.3 in 2).  Only the capacity is
    // known on the host (the live lengths are on the device).
    (void)head_dim;
    if (requested > 0) return requested;
    if (batch <= 0 || nheads_k <= 0 || nheads <= 0 || seqlen_k_capacity <= 0) return 1;
    const int rows = (nheads / nheads_k) * seqlen_q;
    const int64_t wgs = int64_t(batch) * nheads_k * ((rows + 31) / 32);
    const int64_t by_len = (int64_t(seqlen_k_capacity) + 4096) / 8192;
    const int64_t by_fill = (int64_t(std::max(num_cus, 1)) + wgs - 1) / std::max<int64_t>(wgs, 1);
    int64_t max_by_len = seqlen_k_capacity / 512;
    if (seqlen_k_capacity >= 512) max_by_len = std::max<int64_t>(max_by_len, std::min(16, seqlen_k_capacity / 64));
    max_by_len = std::max<int64_t>(1, max_by_len);
    return int(std::max<int64_t>(1, std::min<int64_t>({std::max(by_len, by_fill), max_by_len, 128})));
}

extern "C" size_t fa_kv_workspace_bytes(const fa_kvcache_args *a) {
    if (!a || a->num_splits <= 1) return 0;
    const size_t rows = size_t(a->batch) * a->nheads * a->seqlen_q;
    return size_t(a->num_splits) * rows * (size_t(a->head_dim) + 1) * sizeof(float);
}

extern "C" size_t fa_kv_split_count_len(const fa_kvcache_args *a) {
    if (!a || a->num_splits <= 1 || a->batch <= 0 || a->nheads_k <= 0 || a->nheads <= 0 || a->seqlen_q <= 0)
        return 0;
    const int64_t rows = int64_t(a->nheads / a->nheads_k) * a->seqlen_q;
    return size_t(int64_t(a->batch) * a->nheads_k * ((rows + 31) / 32));
}

namespace fa {
namespace {

bool has_append(const fa_kvcache_args &a) { return a.k_new.ptr && a.seqlen_new > 0 && a.batch > 0; }

int check_append(const fa_kvcache_args &a) {
    if (!has_append(a)) return FA_OK;
    if (!a.v_new.ptr || fa::check_tensor(a.k_new, true) || fa::check_tensor(a.v_new, true) ||
        fa::check_tensor(a.k_cache, true) || fa::check_tensor(a.v_cache, true))
        return FA_ERR_INVALID_ARG;
    return FA_OK;
}

// Work items of the split kernel: (batch, kv head, split, 32-row tile).
int64_t split_items(const fa_kvcache_args &a) {
    const int R = (a.nheads / a.nheads_k) * a.seqlen_q;
    return int64_t(a.batch) * a.nheads_k * ((R + 31) / 32) * a.num_splits;
}

int check_split(const fa_kvcache_args &a) {
    if (fa::check_tensor(a.q, true) || fa::check_tensor(a.o, true) || fa::check_tensor(a.k_cache, true) ||
        fa::check_tensor(a.v_cache, true))
        return FA_ERR_INVALID_ARG;
    if (a.num_splits > 1 && (!a.out_accum || !a.lse_accum)) return FA_ERR_WORKSPACE;
    // The combine reads head_dim 128 partials as 64-bit (atomic) loads.
    if (a.num_splits > 1 && (reinterpret_cast<uintptr_t>(a.out_accum) & 7u)) return FA_ERR_INVALID_ARG;
    if (split_items(a) > 0x7fffffff) return FA_ERR_INVALID_ARG;
    return FA_OK;
}

// The split kernel combines its partials itself: a resident grid (batch_order)
// with split counts and more than one split.
bool fused_combine(const fa_kvcache_args &a) { return a.batch_order && a.split_count && a.num_splits > 1; }

// kv_prep_kernel over the append's chunks (append) after one ordering workgroup (order).
int launch_prep(const fa_kvcache_args &a, bool append, bool order, hipStream_t s) {
    const int64_t chunks = append ? int64_t(a.batch) * a.seqlen_new * a.nheads_k * (a.head_dim / 8) : 0;
    const int order_wgs = order ? 1 : 0;
    const int64_t blocks = order_wgs + (chunks + kOrderThreads - 1) / kOrderThreads;
    if (blocks == 0) return FA_OK;
    if (blocks > 0x7fffffff) return FA_ERR_INVALID_ARG;
    int32_t *count = order && fused_combine(a) ? a.split_count : nullptr;
    const int n_count = count ? int(fa_kv_split_count_len(&a)) : 0;
    if (a.head_dim == 128)
        hipLaunchKernelGGL(kv_prep_kernel<128>, dim3(unsigned(blocks)), dim3(kOrderThreads), 0, s, a, order_wgs, count,
                           n_count);
    else
        hipLaunchKernelGGL(kv_prep_kernel<64>, dim3(unsigned(blocks)), dim3(kOrderThreads), 0, s, a, order_wgs, count,
                           n_count);
    return int(hipGetLastError());
}

// KV heads per work item of the resident split kernel without options: in a
// head-interleaved cache (head stride = head_dim) enough adjacent heads that
// one key position's rows of an item are 512 contiguous bytes (HBM reads of
// 128-byte pieces at a 2 KB stride run about 10 % below 512-byte ones on
// MI355X), while every resident workgroup still gets at least four items:
// with fewer, the items of the longest sequences (their splits are the
// largest) decide the call's time.
int kv_heads_per_item(const fa_kvcache_args &a) {
    const bool interleaved = a.k_cache.head_stride == a.head_dim && a.v_cache.head_stride == a.head_dim;
    const bool ext = a.local_window || a.softcap > 0.f || a.cache_leftpad || a.alibi_slopes || a.rotary_dim > 0;
    if (!a.batch_order || ext || !interleaved) return 1;
    const int64_t items = split_items(a), slots = 2 * int64_t(device_cus());
    int hpi = 1;
    while (hpi < 4 && int64_t(a.head_dim) * 2 * (2 * hpi) <= 512 && a.nheads_k % (2 * hpi) == 0 &&
           items / (2 * hpi) >= 4 * slots)
        hpi *= 2;
    return hpi;
}

// The split kernel.  With batch_order (ranked and its counter reset by
// launch_prep on the same stream): a resident grid of two workgroups per CU
// that deals the items out in that order.  Without it: one workgroup per item.
int launch_split(const fa_kvcache_args &a, hipStream_t s) {
    const int hpi = kv_heads_per_item(a);
    const int64_t gx = split_items(a) / hpi;
    if (gx == 0) return FA_OK;
    const int row_tiles = ((a.nheads / a.nheads_k) * a.seqlen_q + 31) / 32;
    const int n_items = int(gx);
    const bool dyn = a.batch_order != nullptr;
    const unsigned grid = unsigned(dyn ? std::min<int64_t>(gx, 2 * int64_t(device_cus())) : gx);
    int32_t *count = fused_combine(a) ? a.split_count : nullptr;
    const bool ext = a.local_window || a.softcap > 0.f || a.cache_leftpad || a.alibi_slopes || a.rotary_dim > 0;
    auto go = [&](auto hd_tag, auto dyn_tag, auto ext_tag, auto hpi_tag) {
        constexpr int HD = decltype(hd_tag)::value, HPI = decltype(hpi_tag)::value;
        constexpr bool DYN = decltype(dyn_tag)::value, EXT = decltype(ext_tag)::value;
        hipLaunchKernelGGL((kv_splitkv_kernel<HD, DYN, EXT, HPI>), dim3(grid), dim3(kKvThreads), 0, s, a, row_tiles,
                           n_items, count);
    };
    using H128 = std::integral_constant<int, 128>;
    using H64 = std::integral_constant<int, 64>;
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    using P4 = std::integral_constant<int, 4>;
    using T = std::true_type;
    using F = std::false_type;
    if (a.head_dim == 128) {
        if (dyn && !ext) hpi == 2 ? go(H128{}, T{}, F{}, P2{}) : go(H128{}, T{}, F{}, P1{});
        else if (dyn) go(H128{}, T{}, T{}, P1{});
        else ext ? go(H128{}, F{}, T{}, P1{}) : go(H128{}, F{}, F{}, P1{});
    } else {
        if (dyn && !ext) hpi == 4 ? go(H64{}, T{}, F{}, P4{}) : hpi == 2 ? go(H64{}, T{}, F{}, P2{}) : go(H64{}, T{}, F{}, P1{});
        else if (dyn) go(H64{}, T{}, T{}, P1{});
        else ext ? go(H64{}, F{}, T{}, P1{}) : go(H64{}, F{}, F{}, P1{});
    }
    return int(hipGetLastError());
}

// The combine kernel, unless there is one split or the split kernel combined.
int launch_combine(const fa_kvcache_args &a, hipStream_t s) {
    if (a.num_splits <= 1 || fused_combine(a)) return FA_OK;
    const int64_t nrow = int64_t(a.batch) * a.nheads * a.seqlen_q;
    if (nrow == 0) return FA_OK;
    const int64_t blocks = (nrow + 3) / 4;
    if (a.head_dim == 128)
        hipLaunchKernelGGL(kv_combine_kernel<128>, dim3(unsigned(blocks)), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(kv_combine_kernel<64>, dim3(unsigned(blocks)), dim3(256), 0, s, a);
    return int(hipGetLastError());
}

}  // namespace
}  // namespace fa

extern "C" int fa_kv_append(const fa_kvcache_args *args, void *stream) {
    int rc = fa::check_kv(args);
    if (rc || (rc = fa::check_append(*args))) return rc;
    if (!fa::has_append(*args)) return FA_OK;
    return fa::launch_prep(*args, true, false, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int fa_kv_splitkv(const fa_kvcache_args *args, void *stream) {
    int rc = fa::check_kv(args);
    if (rc || (rc = fa::check_split(*args))) return rc;
    const fa_kvcache_args &a = *args;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (fa::split_items(a) == 0) return FA_OK;
    if (a.batch_order && (rc = fa::launch_prep(a, false, true, s))) return rc;
    return fa::launch_split(a, s);
}

extern "C" int fa_kv_combine(const fa_kvcache_args *args, void *stream) {
    int rc = fa::check_kv(args);
    if (rc) return rc;
    const fa_kvcache_args &a = *args;
    if (a.num_splits <= 1 || fa::fused_combine(a)) return FA_OK;
    if (!a.out_accum || !a.lse_accum) return FA_ERR_WORKSPACE;
    return fa::launch_combine(a, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int fa_fwd_kvcache(const fa_kvcache_args *args, void *stream) {
    int rc = fa::check_kv(args);
    if (rc || (rc = fa::check_append(*args)) || (rc = fa::check_split(*args))) return rc;
    const fa_kvcache_args &a = *args;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    // One launch appends and ranks (the ranking reads cache_seqlens only).
    const bool order = a.batch_order && fa::split_items(a) > 0;
    if ((rc = fa::launch_prep(a, fa::has_append(a), order, s))) return rc;
    if ((rc = fa::launch_split(a, s))) return rc;
    return fa::launch_combine(a, s);
}

// ---------------------------------------------------------------------------
// Allocation-free decode: fa_fwd_kvcache with its split workspace (out_accum,
// lse_accum, batch_order, split_count) carved from a static device array
// instead of caller memory, for callers that cannot allocate (code under HIP
// graph capture, serving loops, harnesses that forbid hipMalloc).  The array
// is FA_NOALLOC_SCRATCH_BYTES per device for the life of the process; its
// device address is looked up once per device (hipGetSymbolAddress) and only
// that address is handed to the kernels.  Nothing in it needs clearing between
// calls: the split kernel writes every partial it later combines, and the
// ordering workgroup resets the work counter and the split counts.  Calls on
// one device share the array, so calls that overlap on a device (different
// streams) race.
static __device__ __align__(256) char scratch[FA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch[kMaxDevices] = {};

// Device address of this device's scratch array (looked up on the device's first call).
int scratch_address(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return int(e);
    if (dev < 0 || dev >= kMaxDevices) return FA_ERR_INVALID_ARG;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        // The first call on a device may come from inside a stream capture whose
        // mode forbids runtime calls that are not stream work (the lookup can
        // load the code object on the device): relax this thread's mode for the
        // lookup only; it enqueues nothing.
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        e = hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) return int(e);
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        const hipError_t e2 = hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess) return int(e);
        if (e2 != hipSuccess) return int(e2);
        if (!p) return FA_ERR_SCRATCH;
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return FA_OK;
}

// Scratch bytes a call needs: the split accumulators, then batch + 1 int32s of
// order and counter, then the split counts.
size_t noalloc_bytes(const fa_kvcache_args *a) {
    return fa_kv_workspace_bytes(a) +
           (size_t(a->batch > 0 ? a->batch : 0) + 1 + size_t(fa_kv_split_count_len(a))) * sizeof(int32_t);
}

}  // namespace

extern "C" int fa_fwd_kvcache_noalloc(const fa_kvcache_args *args, void *stream) {
    int rc = fa::check_kv(args);
    if (rc) return rc;
    if (noalloc_bytes(args) > FA_NOALLOC_SCRATCH_BYTES) return FA_ERR_SCRATCH;
    void *base = nullptr;
    if ((rc = scratch_address(&base))) return rc;
    fa_kvcache_args a = *args;
    const size_t acc = fa_kv_workspace_bytes(&a);
    float *f = static_cast<float *>(base);
    if (a.num_splits > 1) {
        a.out_accum = f;
        a.lse_accum = f + size_t(a.num_splits) * a.batch * a.nheads * a.seqlen_q * a.head_dim;
    } else {
        a.out_accum = a.lse_accum = nullptr;
    }
    a.batch_order = reinterpret_cast<int32_t *>(static_cast<char *>(base) + acc);
    a.split_count = fa_kv_split_count_len(&a) > 0 ? a.batch_order + (a.batch > 0 ? a.batch : 0) + 1 : nullptr;
    return fa_fwd_kvcache(&a, stream);
}
