// Backward attention for gfx950 (MI355X).
//
// Replaces flash_bwd_preprocess_kernel.h:23-96 (D = rowsum(dO * O)),
// flash_bwd_kernel.h:25-609 (dQ, one workgroup per query block) and
// :613-1344 (dK/dV, one workgroup per key block), launched by
// flash_bwd_launch_template.h:69-146, and the GQA reduction that
// flash_api.cpp:297-307, 338-348 does with expanded per-q-head buffers and
// torch::sum_out: here the dK/dV workgroup loops over the q-heads of its KV
// head and accumulates the group in fp32 registers.
//
// Math (flash_bwd_kernel.h:417-436, 585-588, 1066-1143, 1317-1319):
//   P  = exp(scale*S - LSE)     (0 where masked)
//   dS = P * (dP - D)           with dP = dO V^T, rounded to fp16
//   dV = P^T dO (P rounded to fp16), dQ = scale * dS K, dK = scale * dS^T Q.
//
// dQ kernel: 4 waves x 32 queries; S^T = K Q^T and dP^T = V dO^T put keys on
// the MFMA M dimension so each lane owns one query (one LSE, one D); dS^T
// feeds dQ^T += K^T dS^T straight from the accumulators.
// dK/dV kernel: 4 waves x 32 keys; S = Q K^T and dP = dO V^T put queries on
// M so P and dS feed dV^T += dO^T P and dK^T += Q^T dS.
#include <algorithm>
#include <type_traits>

#include "fa_common.h"

namespace fa {

constexpr int kBwdThreads = 256;
// MFMA steps by which the dQ kernel's LDS operand reads run ahead (head_dim
// 128; 3 at head_dim 64, whose registers then allow three workgroups per CU).
constexpr int kDqPipe = 4;

// ---------------------------------------------------------------------------
// Preprocess: dsum[b][h][i] = -sum_d fp32(O) * fp32(dO) (stored negated, the
// initial value of the dK/dV kernel's dP accumulators); padding rows get 0.
// One group of KCH threads per row; consecutive groups take consecutive rows of
// one head so the row sums are written contiguously.  fa_bwd computes the same
// sums inside the dQ kernel; this standalone kernel serves fa_bwd_preprocess.
template <int HD>
__global__ __launch_bounds__(256) void bwd_preprocess_kernel(const fa_bwd_args a) {
    constexpr int KCH = HD / 8;
    constexpr int ROWS = kBwdThreads / KCH;  // rows per workgroup
    const int b = blockIdx.z, h = blockIdx.y;
    const bool packed = a.cu_seqlens_q != nullptr;
    const SeqInfo si = seq_info(b, a.seqlen_q, a.seqlen_k, a.cu_seqlens_q, a.cu_seqlens_k, nullptr, 0);
    const int i = blockIdx.x * ROWS + threadIdx.x / KCH;
    const int c = threadIdx.x % KCH;
    if (i >= a.lse_seqlen) return;
    float acc = 0.f;
    if (i < si.sq) {
        const f16 *op = (const f16 *)a.o.ptr + base_off(a.o, packed, b, si.q_start, h) + int64_t(i) * a.o.row_stride;
        const f16 *dp =
            (const f16 *)a.dout.ptr + base_off(a.dout, packed, b, si.q_start, h) + int64_t(i) * a.dout.row_stride;
        const f16x8 ov = as_h8(ldg16(op + 8 * c)), dv = as_h8(ldg16(dp + 8 * c));
#pragma unroll
        for (int j = 0; j < 8; ++j) acc += float(ov[j]) * float(dv[j]);
    }
#pragma unroll
    for (int off = KCH / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, KCH);
    if (c == 0) {
        const int64_t idx = (int64_t(b) * a.nheads + h) * a.lse_seqlen + i;
        const int64_t plane = int64_t(a.batch) * a.nheads * a.lse_seqlen;
        a.dsum[idx] = -acc;
        a.dsum[plane + idx] = i < si.sq ? a.lse[idx] * kLog2e : 0.f;
    }
}

// ---------------------------------------------------------------------------
// dQ kernel: 4 waves x 32 queries; 64-key blocks of K and V copied HBM -> LDS
// (two stages, global_load_lds); S^T = K Q^T and dP^T = V dO^T read K, V as
// natural A operands, dQ^T += K^T dS^T reads K transposed
// (ds_read_b64_tr_b16).  A workgroup holds gp = 2^lg query heads of one GQA
// group (gp divides the group, so they share K / V) at P = 128 / gp positions
// from m0: wave w takes head h + w / (P / 32), positions m0 + 32 (w % (P / 32))
// onward, and the K / V tiles serve all gp heads.  The prologue computes
// D = rowsum(dO * O) for the wave's rows and stores -D for the dK/dV kernel.
template <int HD>
struct DqCfg {
    static constexpr int BM = 128, BN = 64, NT = kBwdThreads;
    static constexpr int TILE = BN * HD * 2;  // K or V tile, natural layout
    static constexpr int STAGE = 2 * TILE;
};

template <int HD, bool CAUSAL>
__global__ __launch_bounds__(256, HD == 64 ? 3 : 2) void bwd_dq_kernel(const fa_bwd_args a, const int num_m_blocks,
                                                                       const int lg) {
    using C = DqCfg<HD>;
    constexpr int DQP = HD == 64 ? 3 : kDqPipe;
    constexpr int BM = C::BM, BN = C::BN, NT = C::NT;
    __shared__ __attribute__((aligned(16))) char smem[2 * C::STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int col = lane & 31, hh = lane >> 5;
    const int packs = a.nheads >> lg;  // head packs per batch
    int b, h, mb;
    if (a.work_order && a.cu_seqlens_q) {
        // Item of the device-built order (head packs fastest); -1: no query rows.
        const int nnb = (a.seqlen_k + 127) / 128;
        const int it = a.work_order[int64_t(a.batch) * nnb + blockIdx.x / packs];
        if (it < 0) return;
        b = __builtin_amdgcn_readfirstlane(it / num_m_blocks);
        mb = __builtin_amdgcn_readfirstlane(it - b * num_m_blocks);
        h = (blockIdx.x % packs) << lg;
    } else {
        const int bp_count = a.batch * packs;
        const int bp = blockIdx.x % bp_count;
        mb = blockIdx.x / bp_count;
        if (CAUSAL) mb = num_m_blocks - 1 - mb;
        b = bp / packs;
        h = (bp - b * packs) << lg;
    }
    const int hk = h / (a.nheads / a.nheads_k);
    const bool packed_q = a.cu_seqlens_q != nullptr, packed_k = a.cu_seqlens_k != nullptr;
    const SeqInfo si = seq_info(b, a.seqlen_q, a.seqlen_k, a.cu_seqlens_q, a.cu_seqlens_k, nullptr, 0);
    const int sq = si.sq, sk = si.sk;
    const int P = BM >> lg;  // positions per head
    const int m0 = mb * P;
    if (m0 >= sq) return;
    h += wave >> (2 - lg);  // this wave's head: P / 32 = 2^(2 - lg) waves per head

    const f16 *qp = (const f16 *)a.q.ptr + base_off(a.q, packed_q, b, si.q_start, h);
    const f16 *dop = (const f16 *)a.dout.ptr + base_off(a.dout, packed_q, b, si.q_start, h);
    const f16 *opp = (const f16 *)a.o.ptr + base_off(a.o, packed_q, b, si.q_start, h);
    const f16 *kp = (const f16 *)a.k.ptr + base_off(a.k, packed_k, b, si.k_start, hk);
    const f16 *vp = (const f16 *)a.v.ptr + base_off(a.v, packed_k, b, si.k_start, hk);
    f16 *dqp = (f16 *)a.dq.ptr + base_off(a.dq, packed_q, b, si.q_start, h);
    const int64_t lrow = (int64_t(b) * a.nheads + h) * a.lse_seqlen;
    const int64_t krs = a.k.row_stride, vrs = a.v.row_stride;

    const int causal_off = sk - sq;
    int n_end = sk;
    if (CAUSAL) n_end = max(0, min(sk, m0 + P + causal_off));
    const int n_blocks = (n_end + BN - 1) / BN;
    const float cs = a.softmax_scale * kLog2e;

    TileCopier<HD, BN, NT> kcp, vcp;
    kcp.init(krs, wave, lane);
    vcp.init(vrs, wave, lane);
    auto issue = [&](int nb, int st) {
        char *ks = smem + st * C::STAGE;
        const int n0 = nb * BN;
        if (n0 + BN <= sk) {
            // Addresses formed per call: hoisted, they were spilled at head_dim 128.
            kcp.template copy_to<true>(lds_addr(smem) + st * C::STAGE, kp + int64_t(n0) * krs, krs);
            vcp.template copy_to<true>(lds_addr(smem) + st * C::STAGE + C::TILE, vp + int64_t(n0) * vrs, vrs);
        } else {
            dma_tile<HD, BN, NT>(ks, kp, krs, n0, sk - 1, wave, lane);
            dma_tile<HD, BN, NT>(ks + C::TILE, vp, vrs, n0, sk - 1, wave, lane);
        }
    };
    // Block 0's copies go out before the row loads below, so the two
    // latencies overlap; the first block's wait covers both.
    if (n_blocks > 0) issue(0, 0);

    // Q^T, dO^T as B operands (lane: query col, d = 16g + 8hh + 0..7) and this
    // lane's half of D = sum_d O * dO.
    const int q_lo = m0 + 32 * (wave & ((P >> 5) - 1));
    const int qi = q_lo + col;
    const bool qv = qi < sq;
    f16x8 qB[HD / 16], doB[HD / 16];
    float dpart = 0.f;
#pragma unroll
    for (int g = 0; g < HD / 16; ++g) {
        qB[g] = as_h8(qv ? ldg16(qp + int64_t(qi) * a.q.row_stride + 16 * g + 8 * hh) : zero_u4());
        doB[g] = as_h8(qv ? ldg16(dop + int64_t(qi) * a.dout.row_stride + 16 * g + 8 * hh) : zero_u4());
        const f16x8 ov = as_h8(qv ? ldg16(opp + int64_t(qi) * a.o.row_stride + 16 * g + 8 * hh) : zero_u4());
#pragma unroll
        for (int t = 0; t < 8; ++t) dpart += float(ov[t]) * float(doB[g][t]);
    }
    const float dsum = sum_xor32(dpart);
    const float lse2 = qv ? a.lse[lrow + qi] * kLog2e : 0.f;
    if (qv && hh == 0) {
        a.dsum[lrow + qi] = -dsum;  // -D: the dK/dV kernel seeds its dP accumulators with it
        a.dsum[int64_t(a.batch) * a.nheads * a.lse_seqlen + lrow + qi] = lse2;  // for the dK/dV kernel
    }

    f32x16 dq[HD / 32];
#pragma unroll
    for (int i = 0; i < HD / 32; ++i) dq[i] = zero16();
    // The dP^T accumulators start from -D (one value per lane: the lane's
    // query), so dP - D comes out of the MFMAs.  Each block fills that seed
    // tile just before its dP chains (16 moves instead of 32 subtractions);
    // held for the whole kernel its 16 registers would not fit at head_dim
    // 128, nor three workgroups per CU at 64.

    TileReader<HD> rd;
    rd.init(lane);

    auto block = [&](int nb, auto mask_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int buf = nb & 1;
        wait_vmem();
        __syncthreads();  // block nb is in LDS; every wave is done with stage buf ^ 1
        if (nb + 1 < n_blocks) issue(nb + 1, buf ^ 1);
        const int n0 = nb * BN;
        if (CAUSAL && MASK && n0 > q_lo + 31 + causal_off) return;  // no visible key for this wave
        if (q_lo >= sq) return;                                      // no query row of the sequence
        // Operand reads run DQP - 1 MFMA steps ahead through a ring of
        // registers, with a scheduling fence per step, so an MFMA does not
        // wait for the LDS read issued just before it.  The lane's read bases
        // get this block's stage added once (opaque, so the per-read
        // addresses are not hoisted to hold registers for the whole kernel);
        // each read is then one XOR and an immediate (TileReader::a_operand_at).
        const int soff = buf * C::STAGE;
        static_assert(C::STAGE % 512 == 0, "stage offsets must be multiples of 512 bytes");
        int ab = rd.a_base + soff, tb0 = rd.tr_base[0] + soff, tb1 = rd.tr_base[1] + soff;
        asm volatile("" : "+v"(ab), "+v"(tb0), "+v"(tb1));
        f16x8 opnd[DQP];
        // S / dP step t: chain c = t % 4 (s[0], dp[0], s[1], dp[1]) at K step
        // g = t / 4, so consecutive MFMAs feed four independent accumulators
        // and each chain still sums g = 0, 1, ... in order.
        constexpr int NSD = 4 * (HD / 16), NDQ = 4 * (HD / 32), NDT = HD / 32;
        auto read_sd = [&](int t) FA_INLINE {
            const int c = t & 3;
            opnd[t % DQP] = rd.a_operand_at(smem + (c & 1) * C::TILE + 32 * (c >> 1) * (HD * 2), ab, t >> 2);
        };
        // dQ step u: accumulator dt = u % NDT at key step gg = u / NDT.
        auto read_dq = [&](int u) FA_INLINE {
            opnd[u % DQP] = rd.tr_operand_at(smem + 16 * (u / NDT) * (HD * 2), tb0, tb1, u % NDT);
        };
        f32x16 s[2], dp[2];
        f32x16 seed;
        {
            float nd = -dsum;
            asm volatile("" : "+v"(nd));  // per block: not hoisted into 16 live registers
#pragma unroll
            for (int i = 0; i < 16; ++i) seed[i] = nd;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < DQP - 1; ++t) read_sd(t);
#pragma unroll
        for (int t = 0; t < NSD; ++t) {
            if (t + DQP - 1 < NSD) read_sd(t + DQP - 1);
            const int c = t & 3, g = t >> 2;
            if (c & 1)
                dp[c >> 1] = mfma32(opnd[t % DQP], doB[g], g == 0 ? seed : dp[c >> 1]);
            else
                s[c >> 1] = mfma32(opnd[t % DQP], qB[g], g == 0 ? zero16() : s[c >> 1]);
            __builtin_amdgcn_sched_barrier(0);
        }
        // The first K^T reads of the dQ product do not depend on dS: they go
        // out before the softmax, which hides their latency.
#pragma unroll
        for (int u = 0; u < DQP - 1; ++u) read_dq(u);
        const int lim = (CAUSAL ? min(sk - 1, qi + causal_off) : sk - 1) - n0;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float p = exp2_fast(fmaf(s[t][r], cs, -lse2));
                if constexpr (MASK) p = t * 32 + acc_lrow(r, hh) > lim ? 0.f : p;
                s[t][r] = p * dp[t][r];
            }
        f16x8 dsB[4];
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) dsB[gg] = pack8(s[gg >> 1], 8 * (gg & 1));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < NDQ; ++u) {
            if (u + DQP - 1 < NDQ) read_dq(u + DQP - 1);
            dq[u % NDT] = mfma32(opnd[u % DQP], dsB[u / NDT], dq[u % NDT]);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Blocks [0, n_full) are fully visible to every row of the workgroup.
    int n_full = min(n_blocks, sk / BN);
    if (CAUSAL) n_full = min(n_full, max(0, (m0 + causal_off + 1) / BN));
    for (int nb = 0; nb < n_full; ++nb) block(nb, std::false_type{});
    for (int nb = n_full; nb < n_blocks; ++nb) block(nb, std::true_type{});

    if (qv) {
        // Opaque to the optimiser: keeps the output address from being computed
        // before the block loops and held (spilled) through them.
        int qo = qi;
        asm volatile("" : "+v"(qo));
        f16 *row = dqp + int64_t(qo) * a.dq.row_stride;
#pragma unroll
        for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                f16x4 v;
#pragma unroll
                for (int t = 0; t < 4; ++t) v[t] = (f16)(dq[dt][4 * a4 + t] * a.softmax_scale);
                *reinterpret_cast<f16x4 *>(row + dt * 32 + 8 * a4 + 4 * hh) = v;
            }
    }
}

// ---------------------------------------------------------------------------
// dK/dV kernel: 4 waves over 128 keys of one (batch, KV head), two workgroups
// per CU.  Wave w owns keys 32 w .. +31 and every query of every 32-query
// block, so the register file holds one 32 x 32 S / dP tile per wave next to
// its dK/dV accumulators, and each SIMD runs one wave of each of two
// independent workgroups: one workgroup's block barriers, prologue and
// epilogue overlap the other's blocks.  K goes HBM -> registers as the S B
// operands; V stays in LDS for the whole kernel as the dP B operands.  For
// every q-head of the GQA group and every query block that sees these keys,
// Q, dO, LSE and D are copied HBM -> LDS (two stages); S = Q K^T and
// dP = dO V^T read Q, dO as natural A operands, dV^T += dO^T P and
// dK^T += Q^T dS read them transposed.  The group's contributions accumulate
// in fp32 registers (no per-q-head dK/dV buffers) and each wave stores its
// keys' rows.  Needs D and LSE*log2(e) (the dsum workspace) from the dQ or
// the preprocess kernel.
constexpr int kDkvThreads = 256;

template <int HD>
struct DkvCfg {
    static constexpr int BN = 128, NT = kDkvThreads;
    static constexpr int BM = 32;                             // queries per block
    static constexpr int QTILE = BM * HD * 2;                 // Q or dO tile, natural layout
    static constexpr int LROWS = 64;                          // LSE / D slots: one 4-byte DMA per lane
    static constexpr int STAGE = 2 * QTILE + 2 * LROWS * 4;   // Q, dO, LSE, D
    static constexpr int VTILE = BN * HD * 2;                 // the workgroup's V rows
    static constexpr int LDS = 2 * STAGE + VTILE;
    static_assert(2 * LDS <= 160 * 1024, "two workgroups per CU");
};

// Varlen work orders (order_items in fa_common.h).  dK/dV: item it = b * nnb
// + nb is key block nb of sequence b, its work the number of query rows that
// see the block (causal: min(sq, sk - 128 nb), else sq), in 64-row buckets;
// dQ: item it = b * nmb + mb is block mb of P query positions, its work the
// keys the block's last position sees (causal: min(sk, P (mb + 1) + sk - sq),
// else sk), in 64-key buckets.  The list of the dK/dV items comes first in
// work_order, that of the dQ items after it (fa_bwd_order_len).
__global__ __launch_bounds__(kOrderThreads) void bwd_order_kernel(const fa_bwd_args a, const int nnb) {
    order_items(a.batch * nnb, [&](int it) {
        const int b = it / nnb, nb = it - b * nnb;
        const int sk = a.cu_seqlens_k[b + 1] - a.cu_seqlens_k[b];
        const int sq = a.cu_seqlens_q ? a.cu_seqlens_q[b + 1] - a.cu_seqlens_q[b] : a.seqlen_q;
        const int k0 = nb * 128;
        if (k0 >= sk) return -1;
        const int rows = a.causal ? max(0, min(sq, sk - k0)) : max(sq, 0);
        return min(rows >> 6, kOrderBuckets - 1);
    }, a.work_order, false);
}

__global__ __launch_bounds__(kOrderThreads) void dq_order_kernel(const fa_bwd_args a, const int nnb, const int nmb,
                                                                 const int P) {
    order_items(a.batch * nmb, [&](int it) {
        const int b = it / nmb, mb = it - b * nmb;
        const int sq = a.cu_seqlens_q[b + 1] - a.cu_seqlens_q[b];
        const int sk = a.cu_seqlens_k ? a.cu_seqlens_k[b + 1] - a.cu_seqlens_k[b] : a.seqlen_k;
        const int m0 = mb * P;
        if (m0 >= sq) return -1;
        const int keys = a.causal ? max(0, min(sk, m0 + P + sk - sq)) : sk;
        return min(keys >> 6, kOrderBuckets - 1);
    }, a.work_order + int64_t(a.batch) * nnb, false);
}

template <int HD, bool CAUSAL>
__global__ __launch_bounds__(kDkvThreads, 2) void bwd_dkdv_kernel(const fa_bwd_args a, const int nnb) {
    using C = DkvCfg<HD>;
    constexpr int BN = C::BN, BM = C::BM, NT = C::NT, LROWS = C::LROWS;
    __shared__ __attribute__((aligned(16))) char smem[C::LDS];

    const int tid = threadIdx.x, lane = tid & 63;
    const int kg = __builtin_amdgcn_readfirstlane(tid >> 6);  // the wave's key group (wave-uniform)
    const int wave = kg;
    const int col = lane & 31, hh = lane >> 5;
    int b, hk, nb;
    if (a.work_order && a.cu_seqlens_k) {
        // Item of the device-built order (kv head fastest); -1: no keys.
        const int it = a.work_order[blockIdx.x / a.nheads_k];
        if (it < 0) return;
        b = __builtin_amdgcn_readfirstlane(it / nnb);
        nb = __builtin_amdgcn_readfirstlane(it - b * nnb);
        hk = blockIdx.x % a.nheads_k;
    } else {
        const int bh_count = a.batch * a.nheads_k;
        const int bhk = blockIdx.x % bh_count;
        nb = blockIdx.x / bh_count;  // smallest key blocks (most queries) first
        b = bhk / a.nheads_k;
        hk = bhk - b * a.nheads_k;
    }
    const int G = a.nheads / a.nheads_k;
    const bool packed_q = a.cu_seqlens_q != nullptr, packed_k = a.cu_seqlens_k != nullptr;
    const SeqInfo si = seq_info(b, a.seqlen_q, a.seqlen_k, a.cu_seqlens_q, a.cu_seqlens_k, nullptr, 0);
    const int sq = si.sq, sk = si.sk;
    const int k0 = nb * BN;
    if (k0 >= sk) return;

    const f16 *kp = (const f16 *)a.k.ptr + base_off(a.k, packed_k, b, si.k_start, hk);
    const f16 *vp = (const f16 *)a.v.ptr + base_off(a.v, packed_k, b, si.k_start, hk);
    const int causal_off = sk - sq;
    const float cs = a.softmax_scale * kLog2e;
    const int64_t qrs = a.q.row_stride, dors = a.dout.row_stride;

    const int kw0 = k0 + kg * 32;
    const int key = kw0 + col;
    const bool kv_ok = key < sk;
    TileReader<HD> rd0;
    rd0.init(lane);
    // V rows of the workgroup as MFMA B operands (lane: key col,
    // d = 16g + 8hh + 0..7).  Row r of each 32-row group is stored at position
    // sigma(r), so the B-operand read of key col is the conflict-free A-operand
    // pattern.
    char *vs_lds = smem + 2 * C::STAGE;
    auto load_rows = [&](char *tile, const f16 *src, int64_t rs) {
        constexpr int KCH = HD / 8;
#pragma unroll
        for (int i = 0; i < BN * KCH / NT; ++i) {
            const int base = (i * (NT / 64) + wave) * 64;
            const int p = base + lane, pos = p / KCH, cs = p % KCH;
            const int row = (pos & ~31) | sigma(pos & 31);
            const int64_t r = min(k0 + row, sk - 1);
            g2l16(src + r * rs + 8 * (cs ^ swz<KCH>(pos)), tile + base * 16);
        }
    };
    load_rows(vs_lds, vp, a.v.row_stride);
    // The wave's K rows stay in registers as the S B operands for the whole
    // kernel, loaded straight from HBM (lane: key col, d = 16g + 8hh + 0..7;
    // keys past the sequence re-read its last row, their columns never stored).
    // Issued after the V copies and waited for with them at the first block.
    f16x8 kreg[HD / 16];
    {
        const f16 *kr = kp + int64_t(min(key, sk - 1)) * a.k.row_stride + 8 * hh;
#pragma unroll
        for (int g = 0; g < HD / 16; ++g) kreg[g] = *reinterpret_cast<const f16x8 *>(kr + 16 * g);
    }
    f32x16 dk[HD / 32], dv[HD / 32];
#pragma unroll
    for (int i = 0; i < HD / 32; ++i) {
        dk[i] = zero16();
        dv[i] = zero16();
    }

    // Query blocks that can see this key block, repeated for each q-head of the group.
    const int m_first = CAUSAL ? max(0, k0 - causal_off) / BM : 0;
    const int n_qb = max(0, (sq + BM - 1) / BM - m_first);

    TileCopier<HD, BM, NT> qcp, ocp;
    qcp.init(qrs, wave, lane);
    ocp.init(dors, wave, lane);
    // Copies of the next (q-head, query block): running pointers to its first Q / dO row and
    // its LSE / D entries, advanced by one block per step (and moved to the
    // next q-head of the group after the last block of a head), so a step's
    // address work is a few scalar adds.  Rows past the sequence re-read its
    // last row (finite values; their P and dS are zeroed below).
    const int64_t lse_plane = int64_t(a.batch) * a.nheads * a.lse_seqlen;
    const f16 *nq = (const f16 *)a.q.ptr + base_off(a.q, packed_q, b, si.q_start, hk * G);
    const f16 *ndo = (const f16 *)a.dout.ptr + base_off(a.dout, packed_q, b, si.q_start, hk * G);
    const float *nd = a.dsum + (int64_t(b) * a.nheads + hk * G) * a.lse_seqlen;
    int nh = 0, ni = 0;  // q-head (within the group) and block of the next copy
    const uint32_t smem_l = lds_addr(smem);
    const int64_t q_step = int64_t(BM) * qrs, do_step = int64_t(BM) * dors;
    const f16 *nq_row = nq + int64_t(m_first) * q_step, *ndo_row = ndo + int64_t(m_first) * do_step;
    auto issue_next = [&](int st) {
        const int q0 = (m_first + ni) * BM;
        const uint32_t qt_l = smem_l + st * C::STAGE, ot_l = qt_l + C::QTILE, lf_l = ot_l + C::QTILE;
        if (q0 + BM <= sq) {
            qcp.copy_to(qt_l, nq_row, qrs);
            ocp.copy_to(ot_l, ndo_row, dors);
        } else {
            char *qt = smem + st * C::STAGE;
            dma_tile<HD, BM, NT>(qt, nq, qrs, q0, sq - 1, wave, lane);
            dma_tile<HD, BM, NT>(qt + C::QTILE, ndo, dors, q0, sq - 1, wave, lane);
        }
        // LSE*log2(e) (second plane of the dsum workspace) and D per query row
        // (64 lanes each; the block reads the first BM).
        const int r = min(q0 + lane, sq - 1);
        if (wave == 0) g2l4_to(nd + lse_plane + r, lf_l);
        if (wave == 1) g2l4_to(nd + r, lf_l + LROWS * 4);
        nq_row += q_step;
        ndo_row += do_step;
        if (++ni == n_qb) {
            ni = 0;
            ++nh;
            nq += a.q.head_stride;
            ndo += a.dout.head_stride;
            nd += a.lse_seqlen;
            nq_row = nq + int64_t(m_first) * q_step;
            ndo_row = ndo + int64_t(m_first) * do_step;
        }
    };

    // The wave's V rows do not move, so their HD / 16 operand addresses are
    // formed once and held (the lane's A-operand base plus the rows' LDS
    // offset, a multiple of 512 bytes, XOR the step: TileReader::a_operand_at).
    const int vb0 = rd0.a_base + 2 * C::STAGE + 32 * kg * (HD * 2);
    int vaddr[HD / 16];
#pragma unroll
    for (int g = 0; g < HD / 16; ++g) vaddr[g] = vb0 ^ (g << 5);
    static_assert(C::STAGE % 512 == 0 && C::QTILE % 512 == 0 && (32 * HD * 2) % 512 == 0,
                  "tile offsets must be multiples of 512 bytes");

    // Block j (queries qh0 ..): S = Q K^T and dP = dO V^T, P, dS, then
    // dV^T += dO^T P and dK^T += Q^T dS.
    auto block = [&](int j, int qh0, auto mask_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int soff = (j & 1) * C::STAGE;
        const float *lf = reinterpret_cast<const float *>(smem + soff + 2 * C::QTILE);
        // The lane's read bases with this block's stage added (once per block:
        // opaque, so the per-read addresses are not hoisted out of the loop,
        // where they would hold dozens of registers for the whole kernel); each
        // read is then one XOR (TileReader::a_operand_at / tr_operand_at) and
        // an immediate: Q at 0, dO at QTILE, rows 16.. of a tile at 16 rows.
        int qb = rd0.a_base + soff, tb0 = rd0.tr_base[0] + soff, tb1 = rd0.tr_base[1] + soff;
        asm volatile("" : "+v"(qb), "+v"(tb0), "+v"(tb1));
        // Operand reads run PIPE steps ahead of the MFMAs that use them, and a
        // scheduling fence after each step keeps that order, so the dK/dV
        // accumulators, the S/dP tiles and the operands in flight fit the
        // 256 registers of a two-waves-per-SIMD wave.
        constexpr int PIPE = 2, NG = HD / 16;
        f16x8 qa[PIPE], oa[PIPE], va[PIPE];
        auto ld = [&](int g) {
            qa[g % PIPE] = rd0.a_operand_at(smem, qb, g);
            oa[g % PIPE] = rd0.a_operand_at(smem + C::QTILE, qb, g);
            va[g % PIPE] = lds_ld16(smem, vaddr[g]);
        };
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < PIPE - 1; ++g) ld(g);
        // dP starts from -D of its rows (the workspace holds -D), so the
        // product comes out as dP - D.
        f32x16 s = zero16(), dp;
#pragma unroll
        for (int r8 = 0; r8 < 2; ++r8) {
            const int ql0 = 16 * r8 + 8 * hh;  // rows ql0 + 0..7 for accumulators 8*r8 + 0..7
            const f32x4 d_a = *reinterpret_cast<const f32x4 *>(lf + LROWS + ql0);
            const f32x4 d_b = *reinterpret_cast<const f32x4 *>(lf + LROWS + ql0 + 4);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                dp[8 * r8 + u] = d_a[u];
                dp[8 * r8 + 4 + u] = d_b[u];
            }
        }
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            if (g + PIPE - 1 < NG) ld(g + PIPE - 1);
            s = mfma32(qa[g % PIPE], kreg[g], s);
            dp = mfma32(oa[g % PIPE], va[g % PIPE], dp);
            __builtin_amdgcn_sched_barrier(0);
        }
        // Masked blocks: accumulator 8 r8 + u holds query qh0 + 8 hh + c with
        // c = 16 r8 + u, live for m_lo <= c < m_hi (the key at or below the
        // query's diagonal, the query inside the sequence): two compares with
        // a constant per element.
        const int mbase = qh0 + 8 * hh;
        const int m_lo = CAUSAL ? key - causal_off - mbase : -(1 << 30), m_hi = sq - mbase;
#pragma unroll
        for (int r8 = 0; r8 < 2; ++r8) {
            const int ql0 = 16 * r8 + 8 * hh;  // rows ql0 + 0..7 for accumulators 8*r8 + 0..7
            const f32x4 l_a = *reinterpret_cast<const f32x4 *>(lf + ql0);
            const f32x4 l_b = *reinterpret_cast<const f32x4 *>(lf + ql0 + 4);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int r = 8 * r8 + u;
                const float l2 = u < 4 ? l_a[u] : l_b[u - 4];
                float p = exp2_fast(fmaf(s[r], cs, -l2));
                if constexpr (MASK) {
                    const int c = 16 * r8 + u;
                    p = (c < m_lo || c >= m_hi) ? 0.f : p;
                }
                s[r] = p;
                dp[r] = p * dp[r];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        f16x8 pB[2], dsB[2];
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
            pB[gg] = pack8(s, 8 * gg);
            dsB[gg] = pack8(dp, 8 * gg);
        }
        // Step t = (dt, gg): dV^T[dt] += dO^T P and dK^T[dt] += Q^T dS, the
        // transposed operands read PIPE steps ahead.
        constexpr int NT2 = 2 * (HD / 32);
        f16x8 ta[PIPE], tq[PIPE];
        auto ldt = [&](int t) {
            ta[t % PIPE] = rd0.tr_operand_at(smem + C::QTILE + 16 * (t & 1) * (HD * 2), tb0, tb1, t >> 1);
            tq[t % PIPE] = rd0.tr_operand_at(smem + 16 * (t & 1) * (HD * 2), tb0, tb1, t >> 1);
        };
#pragma unroll
        for (int t = 0; t < PIPE - 1; ++t) ldt(t);
#pragma unroll
        for (int t = 0; t < NT2; ++t) {
            if (t + PIPE - 1 < NT2) ldt(t + PIPE - 1);
            dv[t >> 1] = mfma32(ta[t % PIPE], pB[t & 1], dv[t >> 1]);
            dk[t >> 1] = mfma32(tq[t % PIPE], dsB[t & 1], dk[t >> 1]);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Each wave walks the same sequence of blocks (one barrier per block) in
    // four straight loops per q-head: blocks that see none of the wave's keys
    // (skipped), diagonal blocks (masked), full blocks, and a ragged last
    // block (masked).  Straight loops keep the dK/dV accumulators in place;
    // branching per block would copy them at every join.  Keys past the
    // sequence need no mask: their columns are never stored.
    int j = 0;  // running block index (stage j & 1)
    auto step = [&](int i, auto mask_tag, bool compute) {
        wait_vmem();
        __syncthreads();  // block j is in LDS; every wave is done with stage (j & 1) ^ 1
        if (nh < G) issue_next((j & 1) ^ 1);
        if (compute) block(j, (m_first + i) * BM, mask_tag);
        ++j;
    };
    auto clampi = [](int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); };
    // Smallest block index i whose start (m_first + i) * BM reaches x.
    auto first_at = [&](int x) { return ((x + BM - 1) >> 5) - m_first; };
    static_assert(BM == 32, "first_at divides by 32");
    const int i1 = CAUSAL ? clampi(first_at(kw0 - 31 - causal_off), 0, n_qb) : 0;
    const int i2 = CAUSAL ? clampi(first_at(kw0 + 31 - causal_off), i1, n_qb) : 0;
    const int i3 = clampi(first_at(sq - 31), i2, n_qb);
    // The first block's copies go out with the V rows and the K loads; the
    // first step's wait and barrier cover all of them.  With no block to walk,
    // the V copies still land before the wave ends.
    if (n_qb > 0)
        issue_next(0);
    else
        wait_vmem();
    for (int hidx = 0; hidx < G && n_qb > 0; ++hidx) {
        for (int i = 0; i < i1; ++i) step(i, std::true_type{}, false);
        for (int i = i1; i < i2; ++i) step(i, std::true_type{}, true);
        for (int i = i2; i < i3; ++i) step(i, std::false_type{}, true);
        for (int i = i3; i < n_qb; ++i) step(i, std::true_type{}, true);
    }

    // Lane (col, hh) holds d = 32 dt + 8 a4 + 4 hh + t (accumulator 4 a4 + t)
    // of key `key`: four consecutive fp16 per store.
    if (!kv_ok) return;
    f16 *dkrow = (f16 *)a.dk.ptr + base_off(a.dk, packed_k, b, si.k_start, hk) + int64_t(key) * a.dk.row_stride;
    f16 *dvrow = (f16 *)a.dv.ptr + base_off(a.dv, packed_k, b, si.k_start, hk) + int64_t(key) * a.dv.row_stride;
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
            f16x4 k4, v4;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                k4[t] = (f16)(dk[dt][4 * a4 + t] * a.softmax_scale);
                v4[t] = (f16)dv[dt][4 * a4 + t];
            }
            *reinterpret_cast<f16x4 *>(dkrow + dt * 32 + 8 * a4 + 4 * hh) = k4;
            *reinterpret_cast<f16x4 *>(dvrow + dt * 32 + 8 * a4 + 4 * hh) = v4;
        }
}

// ---------------------------------------------------------------------------
// Launchers.

static int check_bwd(const fa_bwd_args *p) {
    if (!p) return FA_ERR_INVALID_ARG;
    const fa_bwd_args &a = *p;
    if (a.head_dim != 64 && a.head_dim != 128) return FA_ERR_UNSUPPORTED;
    if (a.batch < 0 || a.seqlen_q < 0 || a.seqlen_k < 0 || a.nheads <= 0 || a.nheads_k <= 0 ||
        a.nheads % a.nheads_k != 0 || !a.lse || a.lse_seqlen < a.seqlen_q)
        return FA_ERR_INVALID_ARG;
    if (!a.dsum) return FA_ERR_WORKSPACE;
    return FA_OK;
}

template <int HD>
static int launch_preprocess(const fa_bwd_args &a, hipStream_t s) {
    constexpr int ROWS = kBwdThreads / (HD / 8);
    const int64_t gx = (int64_t(a.lse_seqlen) + ROWS - 1) / ROWS;
    if (gx == 0 || a.batch == 0) return FA_OK;
    if (a.nheads > 65535 || a.batch > 65535) return FA_ERR_INVALID_ARG;
    hipLaunchKernelGGL(bwd_preprocess_kernel<HD>, dim3(unsigned(gx), unsigned(a.nheads), unsigned(a.batch)),
                       dim3(kBwdThreads), 0, s, a);
    return int(hipGetLastError());
}

template <int HD, bool CAUSAL>
static int launch_dq(const fa_bwd_args &a, hipStream_t s) {
    // Query heads per workgroup: the largest power of two dividing the GQA
    // group, up to one per wave (they share the K / V tiles).
    static_assert(DqCfg<HD>::BM == 128, "the dQ kernel packs at most 4 heads of 32 rows");
    const int group = a.nheads / a.nheads_k;
    int lg = 0;
    while (lg < 2 && group % (2 << lg) == 0) ++lg;
    const int P = DqCfg<HD>::BM >> lg;
    const int nmb = (a.lse_seqlen + P - 1) / P;
    const int64_t grid = int64_t(nmb) * a.batch * (a.nheads >> lg);
    if (grid == 0) return FA_OK;
    if (grid > 0x7fffffff) return FA_ERR_INVALID_ARG;
    if (a.work_order && a.cu_seqlens_q) {
        const int nnb = (a.seqlen_k + 127) / 128;
        hipLaunchKernelGGL(dq_order_kernel, dim3(1), dim3(kOrderThreads), 0, s, a, nnb, nmb, P);
        const int rc = int(hipGetLastError());
        if (rc) return rc;
    }
    hipLaunchKernelGGL((bwd_dq_kernel<HD, CAUSAL>), dim3(unsigned(grid)), dim3(kBwdThreads), 0, s, a, nmb, lg);
    return int(hipGetLastError());
}

template <int HD, bool CAUSAL>
static int launch_dkdv(const fa_bwd_args &a, hipStream_t s) {
    // seqlen_k bounds every sequence's key count (max_seqlen_k for varlen).
    static_assert(DkvCfg<HD>::BN == 128, "bwd_order_kernel and fa_bwd_order_len assume 128-key blocks");
    const int nnb = (a.seqlen_k + DkvCfg<HD>::BN - 1) / DkvCfg<HD>::BN;
    const int64_t grid = int64_t(nnb) * a.batch * a.nheads_k;
    if (grid == 0) return FA_OK;
    if (grid > 0x7fffffff) return FA_ERR_INVALID_ARG;
    if (a.work_order && a.cu_seqlens_k) {
        hipLaunchKernelGGL(bwd_order_kernel, dim3(1), dim3(kOrderThreads), 0, s, a, nnb);
        const int rc = int(hipGetLastError());
        if (rc) return rc;
    }
    hipLaunchKernelGGL((bwd_dkdv_kernel<HD, CAUSAL>), dim3(unsigned(grid)), dim3(kDkvThreads), 0, s, a, nnb);
    return int(hipGetLastError());
}

}  // namespace fa

static int check_bwd_tensors(const fa_bwd_args *a) {
    const fa_tensor *ts[] = {&a->q, &a->k, &a->v, &a->o, &a->dout, &a->dq, &a->dk, &a->dv};
    for (const fa_tensor *t : ts)
        if (fa::check_tensor(*t, true)) return FA_ERR_INVALID_ARG;
    return FA_OK;
}

extern "C" int fa_bwd_preprocess(const fa_bwd_args *args, void *stream) {
    int rc = fa::check_bwd(args);
    if (rc) return rc;
    if ((rc = check_bwd_tensors(args))) return rc;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    return args->head_dim == 128 ? fa::launch_preprocess<128>(*args, s) : fa::launch_preprocess<64>(*args, s);
}

extern "C" int fa_bwd_dq(const fa_bwd_args *args, void *stream) {
    int rc = fa::check_bwd(args);
    if (rc) return rc;
    if ((rc = check_bwd_tensors(args))) return rc;
    const fa_bwd_args &a = *args;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (a.head_dim == 128) return a.causal ? fa::launch_dq<128, true>(a, s) : fa::launch_dq<128, false>(a, s);
    return a.causal ? fa::launch_dq<64, true>(a, s) : fa::launch_dq<64, false>(a, s);
}

extern "C" int fa_bwd_dkdv(const fa_bwd_args *args, void *stream) {
    int rc = fa::check_bwd(args);
    if (rc) return rc;
    if ((rc = check_bwd_tensors(args))) return rc;
    const fa_bwd_args &a = *args;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (a.head_dim == 128) return a.causal ? fa::launch_dkdv<128, true>(a, s) : fa::launch_dkdv<128, false>(a, s);
    return a.causal ? fa::launch_dkdv<64, true>(a, s) : fa::launch_dkdv<64, false>(a, s);
}

extern "C" size_t fa_bwd_order_len(const fa_bwd_args *a) {
    if (!a || a->batch <= 0) return 0;
    const size_t nnb = size_t((std::max(a->seqlen_k, 0) + 127) / 128);
    const size_t nmb = size_t((std::max(a->lse_seqlen, 0) + 31) / 32);  // dQ blocks of 32 positions at the least
    return size_t(a->batch) * (nnb + nmb);
}

extern "C" int fa_bwd(const fa_bwd_args *args, void *stream) {
    // The dQ kernel also writes -D = -rowsum(dO * O) for the dK/dV kernel.
    int rc = fa_bwd_dq(args, stream);
    if (rc) return rc;
    return fa_bwd_dkdv(args, stream);
}
