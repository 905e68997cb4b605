// Forward attention for gfx950 (MI355X).
//
// Replaces the reference forward (csrc/flash_attn/src/flash_fwd_kernel.h:23-711,
// flash_fwd_launch_template.h:9-118).  Semantics kept: fp16 Q/K/V, fp32
// accumulation, scale applied to the fp32 scores, bottom-right causal mask
// (mask.h:52-104), GQA head mapping (fwd_kernel.h:76), varlen offsets and
// seqused_k (block_info.h:4-36), P rounded to fp16 before the PV product
// (fwd_kernel.h:415), O = 0 and LSE = 0 for a row with no visible key
// (fwd_kernel.h:616-662).
//
// Each wave owns 32 queries of one (batch, head) and walks 64-key blocks.  It
// computes S^T = K Q^T (keys on the MFMA M dimension) so each lane holds one
// query column and 32 keys of a block: the row max needs one cross-half
// exchange and the row sum none.  Q^T stays in registers as the B operand.  K
// and V tiles go from HBM straight into LDS with global_load_lds (no register
// staging), two stages; V keeps its natural layout and is read transposed
// with ds_read_b64_tr_b16.  P^T feeds the O^T += V^T P^T MFMAs directly from
// the accumulators (see fa_common.h).
//
// Two kernels share that per-wave arithmetic (so their results are the same
// bit for bit) and differ in how the waves of a SIMD take turns:
//   * fwd_pp_kernel (head_dim 128, grids of at least two workgroups per CU):
//     8 waves, two per SIMD, in two groups that alternate a matrix phase (the
//     PV product of block j - 1 and the S product of block j: all the LDS
//     operand reads and MFMAs) and a softmax phase (block j's exponentials),
//     separated by workgroup barriers, so one group's softmax runs on the
//     VALU while the other group's MFMAs run on the matrix cores;
//   * fwd_kernel (head_dim 64 and small grids): 4 waves, two (head_dim 128)
//     or three (head_dim 64) independent workgroups per CU.
#include <type_traits>

#include "fa_common.h"

namespace fa {

constexpr int kFwdBN = 64;  // keys per block

template <int HD, int NT>
struct FwdCfg {
    static constexpr int BM = 32 * (NT / 64);     // queries per workgroup (32 per wave)
    static constexpr int BN = kFwdBN;
    static constexpr int TILE = BN * HD * 2;      // one K or V tile
    static constexpr int STAGE = 2 * TILE;        // a K tile and a V tile
};

// Each row's probabilities P = exp2(S*c - m) are taken against its exact
// running maximum m, as in the reference's online softmax: the block that
// raises some row's maximum rescales O and the row sums of the wave (by 1 for
// the rows whose maximum stands), so a row's largest score gives P = 1 exactly
// and no P exceeds 1.  (Raising m only when a score outgrows it by 2^8 skips
// most rescales but rounds the dominant keys' P to fp16 at up to 2^8, which
// doubles the output error of rows dominated by a few keys.)  As in the
// reference, the PV product takes P rounded to fp16 and both O and the LSE
// are normalised by the fp32 sum of the unrounded P.

// Per-workgroup extents and base pointers of one (batch, query heads, block of
// query positions).  A workgroup covers gp = 2^lg query heads of one GQA group
// (gp divides the group, so the heads share their K / V) at P = BM / gp
// positions from m0: its K / V tiles serve all of them.  Each wave takes 32
// rows of one head (fwd_wave narrows the pointers to it).
struct FwdWork {
    int b, h, hk, sq, sk, m0, P, causal_off, n_blocks;
    const f16 *qp, *kp, *vp;
    f16 *op;
    float *lse_row;
    float cscale;
    bool neg;
};

// Fills w for workgroup blockIdx.x; false when the block has no query rows
// (its LSE padding is then written here).
template <int BM, bool CAUSAL>
__device__ __forceinline__ bool fwd_work(const fa_fwd_args &a, int num_m_blocks, int lg, FwdWork &w) {
    int mb;
    const int gp = 1 << lg;
    const int packs = a.nheads >> lg;  // head packs per batch
    if (a.work_order && a.cu_seqlens_q) {
        // Item of the device-built order (head packs fastest), longest first.
        const int it = a.work_order[blockIdx.x / packs];
        w.b = __builtin_amdgcn_readfirstlane(it / num_m_blocks);
        mb = __builtin_amdgcn_readfirstlane(it - w.b * num_m_blocks);
        w.h = (blockIdx.x % packs) * gp;
    } else {
        const int bp_count = a.batch * packs;
        const int bp = blockIdx.x % bp_count;
        mb = blockIdx.x / bp_count;
        if (CAUSAL) mb = num_m_blocks - 1 - mb;  // causal blocks are issued heaviest first
        w.b = bp / packs;
        w.h = (bp - w.b * packs) * gp;
    }
    w.P = BM >> lg;
    w.hk = w.h / (a.nheads / a.nheads_k);
    const bool packed_q = a.cu_seqlens_q != nullptr, packed_k = a.cu_seqlens_k != nullptr;
    const SeqInfo si = seq_info(w.b, a.seqlen_q, a.seqlen_k, a.cu_seqlens_q, a.cu_seqlens_k, a.seqused_k,
                                a.seqused_k_add);
    w.sq = si.sq;
    w.sk = si.sk;
    int kb = a.k_batch_idx ? a.k_batch_idx[w.b] : w.b;
    if (a.seqused_k) {
        // KV-cache chunk: a key count past the cache or a cache row outside it
        // leaves the batch with no keys, and the error goes to the status word.
        const int used = a.seqused_k[w.b];
        const int err = (used < 0 || int64_t(used) + a.seqused_k_add > a.seqlen_k ? 1 : 0) |
                        (a.k_batch_idx && a.k_batch > 0 && (kb < 0 || kb >= a.k_batch) ? 2 : 0);
        if (err) {
            w.sk = 0;
            kb = 0;
            if (a.status && threadIdx.x == 0) atomicOr(a.status, err);
        }
    }
    w.m0 = mb * w.P;
    w.lse_row = a.lse + (int64_t(w.b) * a.nheads + w.h) * a.lse_seqlen;
    if (w.m0 >= w.sq) {
        // Rows past this sequence's length: LSE padding is 0 (flash_api.cpp:388).
        for (int i = threadIdx.x; i < gp * w.P; i += blockDim.x) {
            const int row = w.m0 + i % w.P;
            if (row < a.lse_seqlen) w.lse_row[int64_t(i / w.P) * a.lse_seqlen + row] = 0.f;
        }
        return false;
    }
    w.qp = (const f16 *)a.q.ptr + base_off(a.q, packed_q, w.b, si.q_start, w.h);
    w.kp = (const f16 *)a.k.ptr + base_off(a.k, packed_k, kb, si.k_start, w.hk);
    w.vp = (const f16 *)a.v.ptr + base_off(a.v, packed_k, kb, si.k_start, w.hk);
    w.op = (f16 *)a.o.ptr + base_off(a.o, packed_q, w.b, si.q_start, w.h);
    w.causal_off = w.sk - w.sq;  // key j visible to query i iff j <= i + causal_off
    int n_end = w.sk;
    if (CAUSAL) n_end = max(0, min(w.sk, w.m0 + w.P + w.causal_off));
    w.n_blocks = (n_end + kFwdBN - 1) / kFwdBN;
    // Negative scales are folded into Q's sign so that the exp argument uses |scale|.
    w.neg = a.softmax_scale < 0.f;
    w.cscale = fabsf(a.softmax_scale) * kLog2e;
    return true;
}

// Narrows w to the rows of 32-row tile t of the workgroup: tile t is head
// w.h + t / (P / 32), positions m0 + 32 (t % (P / 32)) .. + 31.  Returns the
// tile's first position.
__device__ __forceinline__ int fwd_wave(const fa_fwd_args &a, FwdWork &w, int t) {
    const int tiles = w.P >> 5;  // position tiles per head (a power of two)
    const int hp = t >> (31 - __builtin_clz(tiles));
    w.h += hp;
    w.qp += int64_t(hp) * a.q.head_stride;
    w.op += int64_t(hp) * a.o.head_stride;
    w.lse_row += int64_t(hp) * a.lse_seqlen;
    return w.m0 + 32 * (t & (tiles - 1));
}

// Q^T of query qi as B operands: lane (query col, half hh), K step g covers d = 16g + 8hh + 0..7.
template <int HD>
__device__ __forceinline__ void load_q(const fa_fwd_args &a, const FwdWork &w, int qi, int hh, f16x8 (&qB)[HD / 16]) {
#pragma unroll
    for (int g = 0; g < HD / 16; ++g) {
        u32x4 v = zero_u4();
        if (qi < w.sq) v = ldg16(w.qp + int64_t(qi) * a.q.row_stride + 16 * g + 8 * hh);
        if (w.neg) v = neg_h8(v);
        qB[g] = as_h8(v);
    }
}

// Online-softmax state of a wave's 32 queries (this lane's query column).
struct SoftmaxRow {
    float m_t = -INFINITY;  // reference max of scale*log2(e)*S for this lane's query
    float l_p = 0.f;        // partial row sum over this lane half's keys (fp32 P)
};

// One 64-key block of S^T (two 32 x 32 accumulator tiles) -> P^T operands:
// mask (MASK: keys past lim, relative to the block start), running maximum,
// rescale of O, exponentials, row sums.
template <int HD, bool MASK>
__device__ __forceinline__ void softmax_block(f32x16 (&s)[2], f16x8 (&pB)[4], f32x16 (&o)[HD / 32], SoftmaxRow &r,
                                              float cscale, int lim, int hh) {
    if constexpr (MASK) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                if (kt * 32 + acc_lrow(e, hh) > lim) s[kt][e] = -INFINITY;
    }
    float mx = s[0][0];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kt][e]);
    mx = max_xor32(mx);
    const float mx_t = MASK && mx == -INFINITY ? -INFINITY : mx * cscale;
    if (__builtin_amdgcn_ballot_w64(mx_t > r.m_t) != 0) {
        const float m_new = fmaxf(r.m_t, mx_t);
        const float alpha = m_new == -INFINITY ? 1.f : exp2_fast(r.m_t - m_new);
        r.l_p *= alpha;
#pragma unroll
        for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
            for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;
        r.m_t = m_new;
    }
    const float m_use = r.m_t == -INFINITY ? 0.f : r.m_t;
    float rs = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float x = s[kt][e];
            float p = exp2_fast(fmaf(x, cscale, -m_use));
            if constexpr (MASK) p = x == -INFINITY ? 0.f : p;
            s[kt][e] = p;
            rs += p;
        }
    r.l_p += rs;
#pragma unroll
    for (int gg = 0; gg < 4; ++gg) {
        pB[gg] = pack8(s[gg >> 1], 8 * (gg & 1));
    }
}

// Epilogue: O / l in fp16, LSE = ln(sum exp(scale*S)); empty rows give 0 / 0.
template <int HD>
__device__ __forceinline__ void store_row(const fa_fwd_args &a, const FwdWork &w, int qi, int hh,
                                          const f32x16 (&o)[HD / 32], const SoftmaxRow &r) {
    const float l_tot = sum_xor32(r.l_p);
    if (qi < w.sq) {
        const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
        f16 *orow = w.op + int64_t(qi) * a.o.row_stride;
#pragma unroll
        for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                f16x4 v;
#pragma unroll
                for (int t = 0; t < 4; ++t) v[t] = (f16)(o[dt][4 * a4 + t] * inv);
                *reinterpret_cast<f16x4 *>(orow + dt * 32 + 8 * a4 + 4 * hh) = v;
            }
        if (hh == 0) w.lse_row[qi] = l_tot > 0.f ? (r.m_t + log2_fast(l_tot)) * kLn2 : 0.f;
    } else if (hh == 0 && qi < a.lse_seqlen) {
        w.lse_row[qi] = 0.f;
    }
}

// Copies of K / V block nb into an LDS tile by all NT threads.  A block that
// runs past the sequence re-reads its last key for the missing rows (masked).
template <int HD, int NT>
struct KvLoader {
    TileCopier<HD, kFwdBN, NT> kcp, vcp;
    __device__ __forceinline__ void init(const fa_fwd_args &a, int wave, int lane) {
        kcp.init(a.k.row_stride, wave, lane);
        vcp.init(a.v.row_stride, wave, lane);
    }
    __device__ __forceinline__ void k(const fa_fwd_args &a, const FwdWork &w, char *smem, uint32_t off, int nb,
                                      int wave, int lane) const {
        const int n0 = nb * kFwdBN;
        if (n0 + kFwdBN <= w.sk)
            kcp.copy_to(lds_addr(smem) + off, w.kp + int64_t(n0) * a.k.row_stride, a.k.row_stride);
        else
            dma_tile<HD, kFwdBN, NT>(smem + off, w.kp, a.k.row_stride, n0, w.sk - 1, wave, lane);
    }
    __device__ __forceinline__ void v(const fa_fwd_args &a, const FwdWork &w, char *smem, uint32_t off, int nb,
                                      int wave, int lane) const {
        const int n0 = nb * kFwdBN;
        if (n0 + kFwdBN <= w.sk)
            vcp.copy_to(lds_addr(smem) + off, w.vp + int64_t(n0) * a.v.row_stride, a.v.row_stride);
        else
            dma_tile<HD, kFwdBN, NT>(smem + off, w.vp, a.v.row_stride, n0, w.sk - 1, wave, lane);
    }
};

// ---------------------------------------------------------------------------
// 4-wave kernel: each wave runs S, softmax and PV of a block in turn; two
// workgroups per CU at head_dim 128 (64 KB LDS, 246 registers), three at
// head_dim 64 (32 KB LDS, at most 168 registers), overlap one wave's softmax
// with the others' MFMAs on each SIMD.  QT = 2 (head_dim 64): each wave takes
// two 32-query tiles of one head and each K / V operand it reads from LDS
// feeds both tiles' MFMAs, which halves the LDS reads per MFMA (at head_dim 64
// a score costs half the MFMA work of head_dim 128 for the same reads of V;
// measured 3-6 % faster at seqlen 8192); two workgroups of 256 queries per
// CU.  The per-tile arithmetic is the same, so the results are the same bits.
template <int HD, bool CAUSAL, int QT>
__global__ __launch_bounds__(256, QT == 2 || HD == 128 ? 2 : 3) void fwd_kernel(const fa_fwd_args a,
                                                                                const int num_m_blocks, const int lg) {
    constexpr int NT = 256;
    using C = FwdCfg<HD, NT>;
    constexpr int BM = C::BM * QT, BN = C::BN;
    __shared__ __attribute__((aligned(16))) char smem[2 * C::STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int hh = lane >> 5;
    FwdWork w;
    if (!fwd_work<BM, CAUSAL>(a, num_m_blocks, lg, w)) return;

    // The wave's tiles QT * wave + t: one head (the launcher packs at most BM / 64 heads when QT = 2,
    // so a head spans at least 64 positions).
    const int q_lo = fwd_wave(a, w, QT * wave);
    int qi[QT];
    f16x8 qB[QT][HD / 16];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        qi[t] = q_lo + 32 * t + (lane & 31);
        load_q<HD>(a, w, qi[t], hh, qB[t]);
    }
    wait_vmem();  // only the tile copies are in flight inside the loop

    f32x16 o[QT][HD / 32];
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
        for (int i = 0; i < HD / 32; ++i) o[t][i] = zero16();
    SoftmaxRow row[QT];

    TileReader<HD> rd;
    rd.init(lane);
    KvLoader<HD, NT> ld;
    ld.init(a, wave, lane);
    auto issue = [&](int nb, int st) FA_INLINE {
        ld.k(a, w, smem, st * C::STAGE, nb, wave, lane);
        ld.v(a, w, smem, st * C::STAGE + C::TILE, nb, wave, lane);
    };

    // One key block: S^T = K Q^T, online softmax, O^T += V^T P^T.  MASK is a
    // compile-time switch so the blocks away from the causal diagonal and
    // the sequence end carry no masking work at all.  A tile with no visible
    // key in a block it shares with the wave's other tile gets P = 0 there
    // (its O, sums and maximum unchanged).
    auto block = [&](int nb, auto mask_tag) FA_INLINE {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int buf = nb & 1;
        wait_vmem();
        __syncthreads();  // block nb is in LDS; every wave is done with stage buf ^ 1
        if (nb + 1 < w.n_blocks) issue(nb + 1, buf ^ 1);
        const int n0 = nb * BN;
        if (CAUSAL && MASK && n0 > q_lo + 32 * QT - 1 + w.causal_off) return;  // no visible key for this wave
        if (q_lo >= w.sq) return;                                               // no query row of the sequence
        const char *ks = smem + buf * C::STAGE;
        const char *vs = ks + C::TILE;
        f32x16 s[QT][2];
        f16x8 pB[QT][4];
        auto softmax = [&]() FA_INLINE {
#pragma unroll
            for (int t = 0; t < QT; ++t) {
                const int lim = (CAUSAL ? min(w.sk - 1, qi[t] + w.causal_off) : w.sk - 1) - n0;
                softmax_block<HD, MASK>(s[t], pB[t], o[t], row[t], w.cscale, lim, hh);
            }
        };
        if constexpr (QT == 1) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                s[0][kt] = mfma32(rd.a_operand(ks, 32 * kt, 0), qB[0][0], zero16());
#pragma unroll
                for (int g = 1; g < HD / 16; ++g) s[0][kt] = mfma32(rd.a_operand(ks, 32 * kt, g), qB[0][g], s[0][kt]);
            }
            softmax();
#pragma unroll
            for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
                for (int gg = 0; gg < 4; ++gg) o[0][dt] = mfma32(rd.tr_operand(vs, 16 * gg, dt), pB[0][gg], o[0][dt]);
        } else {
            // Each operand feeds both tiles' MFMAs.  The reads run PIPE steps
            // ahead behind scheduling fences (all of them hoisted to the top
            // would not fit the registers of two waves per SIMD), from the
            // lane's base offsets with this block's stage added once (opaque:
            // hoisted out of the loop, the per-read addresses would hold
            // registers for the whole kernel); each read is one XOR and an
            // immediate (TileReader::a_operand_at).
            constexpr int PIPE = 3, NS = 2 * (HD / 16), NPV = 4 * (HD / 32);
            const int soff = buf * C::STAGE;
            static_assert(C::STAGE % 512 == 0, "stage offsets must be multiples of 512 bytes");
            int ab = rd.a_base + soff, tb0 = rd.tr_base[0] + soff, tb1 = rd.tr_base[1] + soff;
            asm volatile("" : "+v"(ab), "+v"(tb0), "+v"(tb1));
            f16x8 op[PIPE];
            auto rd_k = [&](int u) FA_INLINE {
                op[u % PIPE] = rd.a_operand_at(smem + 32 * (u / (HD / 16)) * (HD * 2), ab, u % (HD / 16));
            };
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < PIPE - 1; ++u) rd_k(u);
#pragma unroll
            for (int u = 0; u < NS; ++u) {
                if (u + PIPE - 1 < NS) rd_k(u + PIPE - 1);
                const int kt = u / (HD / 16), g = u % (HD / 16);
#pragma unroll
                for (int t = 0; t < QT; ++t) s[t][kt] = mfma32(op[u % PIPE], qB[t][g], g == 0 ? zero16() : s[t][kt]);
                __builtin_amdgcn_sched_barrier(0);
            }
            softmax();
            auto rd_v = [&](int u) FA_INLINE {
                op[u % PIPE] = rd.tr_operand_at(smem + C::TILE + 16 * (u & 3) * (HD * 2), tb0, tb1, u >> 2);
            };
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < PIPE - 1; ++u) rd_v(u);
#pragma unroll
            for (int u = 0; u < NPV; ++u) {
                if (u + PIPE - 1 < NPV) rd_v(u + PIPE - 1);
#pragma unroll
                for (int t = 0; t < QT; ++t) o[t][u >> 2] = mfma32(op[u % PIPE], pB[t][u & 3], o[t][u >> 2]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    // Blocks [0, n_full) need no mask for any wave of the workgroup: every key
    // is below the sequence end and at or below the diagonal of the first query.
    int n_full = min(w.n_blocks, w.sk / BN);
    if (CAUSAL) n_full = min(n_full, max(0, (w.m0 + w.causal_off + 1) / BN));
    if (w.n_blocks > 0) issue(0, 0);
    for (int nb = 0; nb < n_full; ++nb) block(nb, std::false_type{});
    for (int nb = n_full; nb < w.n_blocks; ++nb) block(nb, std::true_type{});
#pragma unroll
    for (int t = 0; t < QT; ++t) store_row<HD>(a, w, qi[t], hh, o[t], row[t]);
}

// ---------------------------------------------------------------------------
// Ping-pong kernel: 8 waves over 256 queries.  Waves w and w + 4 share a SIMD
// (waves go to the SIMDs in order, 0..3 then again 0..3); group g = w / 4
// holds 32-query tile 2 (w % 4) + g, so both groups span the workgroup's rows
// and reach the causal diagonal together.  Iteration j (two barriers):
//   group 0: matrix phase [PV of block j - 1, S of block j] | softmax of j
//   group 1: softmax of j - 1 | matrix phase [PV of j - 1, S of j]
// Stage j & 1 holds K_j and V_{j - 1}; the next stage's copies (K_{j + 1},
// V_j) go out at the start of iteration j.  Matrix-phase operands are read
// PIPE steps ahead of their MFMAs with a scheduling fence per step.
constexpr int kPpPipe = 8;

template <int HD, bool CAUSAL>
__global__ __launch_bounds__(512, 1) void fwd_pp_kernel(const fa_fwd_args a, const int num_m_blocks, const int lg) {
    constexpr int NT = 512;
    using C = FwdCfg<HD, NT>;
    constexpr int BM = C::BM, BN = C::BN;
    __shared__ __attribute__((aligned(16))) char smem[2 * C::STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int grp = wave >> 2;                                  // 0: matrix phase first
    const int hh = lane >> 5;
    FwdWork w;
    if (!fwd_work<BM, CAUSAL>(a, num_m_blocks, lg, w)) return;

    const int q_lo = fwd_wave(a, w, 2 * (wave & 3) + grp);
    const int qi = q_lo + (lane & 31);
    f16x8 qB[HD / 16];
    load_q<HD>(a, w, qi, hh, qB);
    wait_vmem();  // only the tile copies are in flight inside the loop

    f32x16 o[HD / 32];
#pragma unroll
    for (int i = 0; i < HD / 32; ++i) o[i] = zero16();
    SoftmaxRow row;

    TileReader<HD> rd;
    rd.init(lane);
    KvLoader<HD, NT> ld;
    ld.init(a, wave, lane);

    // Last key this wave sees; blocks [0, nbw) hold its keys, and blocks
    // [0, n_full) need no mask for any of its queries.
    const int wave_last_key = CAUSAL ? min(w.sk - 1, q_lo + 31 + w.causal_off) : w.sk - 1;
    const int nbw = q_lo < w.sq ? max(0, min(w.n_blocks, (wave_last_key + BN) / BN)) : 0;
    int n_full = min(w.n_blocks, w.sk / BN);
    if (CAUSAL) n_full = min(n_full, max(0, (q_lo + w.causal_off + 1) / BN));

    f32x16 s[2];
    f16x8 pB[4];
    // Matrix phase of iteration j: O^T += V_{j-1}^T P_{j-1}^T (DO_PV), then
    // S_j^T = K_j Q^T (DO_S); step t < NPV is a PV MFMA, the rest S MFMAs.
    constexpr int NPV = 4 * (HD / 32), NS = 2 * (HD / 16);
    auto matrix = [&](int j, auto pv_tag, auto s_tag) FA_INLINE {
        constexpr bool DO_PV = decltype(pv_tag)::value, DO_S = decltype(s_tag)::value;
        constexpr int T0 = DO_PV ? 0 : NPV, T1 = DO_S ? NPV + NS : NPV;
        // The lane's read bases with stage j & 1 added once (opaque: hoisted out
        // of the loop, the per-read addresses would hold registers for the
        // whole kernel); each read is then one XOR and an immediate
        // (TileReader::a_operand_at).
        const int soff = (j & 1) * C::STAGE;
        static_assert(C::STAGE % 512 == 0, "stage offsets must be multiples of 512 bytes");
        int ab = rd.a_base + soff, tb0 = rd.tr_base[0] + soff, tb1 = rd.tr_base[1] + soff;
        asm volatile("" : "+v"(ab), "+v"(tb0), "+v"(tb1));
        f16x8 opnd[kPpPipe];
        auto read = [&](int t) FA_INLINE {
            if (t < NPV)
                opnd[t % kPpPipe] = rd.tr_operand_at(smem + C::TILE + 16 * (t & 3) * (HD * 2), tb0, tb1, t >> 2);
            else
                opnd[t % kPpPipe] =
                    rd.a_operand_at(smem + 32 * ((t - NPV) / (HD / 16)) * (HD * 2), ab, (t - NPV) % (HD / 16));
        };
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = T0; t < T0 + kPpPipe - 1 && t < T1; ++t) read(t);
#pragma unroll
        for (int t = T0; t < T1; ++t) {
            if (t + kPpPipe - 1 < T1) read(t + kPpPipe - 1);
            if (t < NPV) {
                o[t >> 2] = mfma32(opnd[t % kPpPipe], pB[t & 3], o[t >> 2]);
            } else {
                const int u = t - NPV, kt = u / (HD / 16), g = u % (HD / 16);
                s[kt] = mfma32(opnd[t % kPpPipe], qB[g], g == 0 ? zero16() : s[kt]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto softmax = [&](int j, auto mask_tag) FA_INLINE {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int lim = (CAUSAL ? min(w.sk - 1, qi + w.causal_off) : w.sk - 1) - j * BN;
        softmax_block<HD, MASK>(s, pB, o, row, w.cscale, lim, hh);
    };
    auto softmax_any = [&](int j) FA_INLINE {
        if (j < n_full)
            softmax(j, std::false_type{});
        else
            softmax(j, std::true_type{});
    };
    // Start of iteration j: K_j and V_{j-1} are in stage j & 1 (every wave's
    // copies have landed) and stage (j + 1) & 1 is free: the next copies go out.
    auto top = [&](int j) FA_INLINE {
        wait_vmem();
        __syncthreads();
        if (j < w.n_blocks) {
            if (j + 1 < w.n_blocks) ld.k(a, w, smem, ((j + 1) & 1) * C::STAGE, j + 1, wave, lane);
            ld.v(a, w, smem, ((j + 1) & 1) * C::STAGE + C::TILE, j, wave, lane);
        }
    };
    auto mid = []() FA_INLINE { __builtin_amdgcn_s_barrier(); };
    using T = std::true_type;
    using F = std::false_type;

    // Every wave runs iterations 0..n_blocks (two barriers each); a wave does
    // S for blocks j < nbw and PV for 1 <= j <= nbw.
    if (w.n_blocks > 0) ld.k(a, w, smem, 0, 0, wave, lane);
    int j = 1;
    if (grp == 0) {
        top(0);
        if (nbw > 0) matrix(0, F{}, T{});
        mid();
        if (nbw > 0) softmax_any(0);
        for (; j < min(nbw, n_full); ++j) {
            top(j);
            matrix(j, T{}, T{});
            mid();
            softmax(j, F{});
        }
        for (; j < nbw; ++j) {
            top(j);
            matrix(j, T{}, T{});
            mid();
            softmax(j, T{});
        }
        if (nbw > 0) {
            top(nbw);
            matrix(nbw, T{}, F{});
            mid();
            j = nbw + 1;
        }
    } else {
        top(0);
        mid();
        if (nbw > 0) matrix(0, F{}, T{});
        for (; j < min(nbw, n_full + 1); ++j) {
            top(j);
            softmax(j - 1, F{});
            mid();
            matrix(j, T{}, T{});
        }
        for (; j < nbw; ++j) {
            top(j);
            softmax(j - 1, T{});
            mid();
            matrix(j, T{}, T{});
        }
        if (nbw > 0) {
            top(nbw);
            softmax_any(nbw - 1);
            mid();
            matrix(nbw, T{}, F{});
            j = nbw + 1;
        }
    }
    for (; j <= w.n_blocks; ++j) {
        top(j);
        mid();
    }
    store_row<HD>(a, w, qi, hh, o, row);
}

// Varlen work order (order_items in fa_common.h): item it = b * nmb + mb is
// block mb of P query positions of sequence b, its work about positions x
// keys seen by the block's last position, in buckets of P x 64; blocks past a
// sequence's end come last (they still write LSE padding).
__global__ __launch_bounds__(kOrderThreads) void fwd_order_kernel(const fa_fwd_args a, const int nmb, const int P) {
    order_items(a.batch * nmb, [&](int it) {
        const int b = it / nmb, mb = it - b * nmb;
        const int sq = a.cu_seqlens_q[b + 1] - a.cu_seqlens_q[b];
        const int sk = a.cu_seqlens_k ? a.cu_seqlens_k[b + 1] - a.cu_seqlens_k[b] : a.seqlen_k;
        const int m0 = mb * P;
        if (m0 >= sq) return -1;
        const int64_t rows = min(P, sq - m0);
        const int64_t keys = a.causal ? max(0, min(sk, m0 + P + sk - sq)) : max(sk, 0);
        return int(min<int64_t>(rows * keys / (int64_t(P) * 64), kOrderBuckets - 1));
    }, a.work_order, true);
}

static int launch_order(const fa_fwd_args &a, int nmb, int P, hipStream_t stream) {
    if (!a.work_order || !a.cu_seqlens_q) return FA_OK;
    hipLaunchKernelGGL(fwd_order_kernel, dim3(1), dim3(kOrderThreads), 0, stream, a, nmb, P);
    return int(hipGetLastError());
}

// log2 of the query heads per workgroup for a BM-row kernel: the largest
// power of two that divides the GQA group (those heads read the same K / V)
// and leaves whole 32-row tiles per head.  The K / V tiles a workgroup loads
// then serve gp heads instead of one, and the workgroup spans BM / gp
// positions, so a causal block wastes less on the diagonal.
static int fwd_pack_log2(const fa_fwd_args &a, int BM) {
    const int group = a.nheads / a.nheads_k;
    int lg = 0;
    while ((64 << lg) <= BM && group % (2 << lg) == 0) ++lg;
    return lg;
}

template <int HD, bool CAUSAL>
static int launch_fwd(const fa_fwd_args &a, hipStream_t stream) {
    // The ping-pong kernel when its grid fills the chip at least twice over
    // and sequences reach 2048 rows; the 4-wave kernel otherwise (and at
    // head_dim 64, where it measured faster).  Below 2048 rows the 128-row
    // blocks waste less on causal diagonals and ragged sequence ends and deal
    // out more evenly (measured varlen causal, 32 / 8 heads: 64 x 1024 rows
    // +3 %, 64 x U[64, 1024] +14 %; 32 x 2048 even; 16 x 4096 -5 %).  Both
    // give the same bits.
    if constexpr (HD == 128) {
        constexpr int BM = FwdCfg<HD, 512>::BM;
        const int lg = fwd_pack_log2(a, BM), P = BM >> lg;
        const int64_t pp_m_blocks = (a.lse_seqlen + P - 1) / P;
        const int64_t pp_grid = pp_m_blocks * a.batch * (a.nheads >> lg);
        if (pp_grid >= 2 * int64_t(device_cus()) && a.lse_seqlen >= 2048) {
            if (pp_grid > 0x7fffffff) return FA_ERR_INVALID_ARG;
            const int rc = launch_order(a, int(pp_m_blocks), P, stream);
            if (rc) return rc;
            hipLaunchKernelGGL((fwd_pp_kernel<HD, CAUSAL>), dim3(unsigned(pp_grid)), dim3(512), 0, stream, a,
                               int(pp_m_blocks), lg);
            return int(hipGetLastError());
        }
    }
    // Head_dim 64: two query tiles per wave when that grid still fills the chip
    // twice over.  A wave's two tiles must be one head's, so at most 4 heads
    // share a workgroup (64 positions each).
    if constexpr (HD == 64) {
        constexpr int BM2 = 2 * FwdCfg<HD, 256>::BM;
        const int lg = min(fwd_pack_log2(a, BM2), 2), P = BM2 >> lg;
        const int64_t m_blocks = (a.lse_seqlen + P - 1) / P;
        const int64_t grid = m_blocks * a.batch * (a.nheads >> lg);
        if (grid >= 2 * int64_t(device_cus())) {
            if (grid > 0x7fffffff) return FA_ERR_INVALID_ARG;
            const int rc = launch_order(a, int(m_blocks), P, stream);
            if (rc) return rc;
            hipLaunchKernelGGL((fwd_kernel<HD, CAUSAL, 2>), dim3(unsigned(grid)), dim3(256), 0, stream, a,
                               int(m_blocks), lg);
            return int(hipGetLastError());
        }
    }
    constexpr int BM = FwdCfg<HD, 256>::BM;
    const int lg = fwd_pack_log2(a, BM), P = BM >> lg;
    const int num_m_blocks = (a.lse_seqlen + P - 1) / P;
    const int64_t grid = int64_t(num_m_blocks) * a.batch * (a.nheads >> lg);
    if (grid == 0) return FA_OK;
    if (grid > 0x7fffffff) return FA_ERR_INVALID_ARG;
    const int rc = launch_order(a, num_m_blocks, P, stream);
    if (rc) return rc;
    hipLaunchKernelGGL((fwd_kernel<HD, CAUSAL, 1>), dim3(unsigned(grid)), dim3(256), 0, stream, a, num_m_blocks, lg);
    return int(hipGetLastError());
}

}  // namespace fa

extern "C" int fa_fwd(const fa_fwd_args *args, void *stream) {
    if (!args) return FA_ERR_INVALID_ARG;
    const fa_fwd_args &a = *args;
    if (a.head_dim != 64 && a.head_dim != 128) return FA_ERR_UNSUPPORTED;
    if (a.batch < 0 || a.seqlen_q < 0 || a.seqlen_k < 0 || a.nheads <= 0 || a.nheads_k <= 0 ||
        a.nheads % a.nheads_k != 0 || !a.lse || a.lse_seqlen < a.seqlen_q)
        return FA_ERR_INVALID_ARG;
    if (fa::check_tensor(a.q, true) || fa::check_tensor(a.k, true) || fa::check_tensor(a.v, true) ||
        fa::check_tensor(a.o, true))
        return FA_ERR_INVALID_ARG;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (a.head_dim == 128)
        return a.causal ? fa::launch_fwd<128, true>(a, s) : fa::launch_fwd<128, false>(a, s);
    return a.causal ? fa::launch_fwd<64, true>(a, s) : fa::launch_fwd<64, false>(a, s);
}

extern "C" size_t fa_fwd_order_len(const fa_fwd_args *a) {
    if (!a || a->batch <= 0 || a->lse_seqlen <= 0) return 0;
    return size_t(a->batch) * size_t((a->lse_seqlen + 31) / 32);  // blocks of 32 positions at the least
}
