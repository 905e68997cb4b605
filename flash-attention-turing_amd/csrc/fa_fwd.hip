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
// Design: one workgroup = 4 waves = 128 queries of one (batch, head); each
// wave owns 32 queries.  The wave computes S^T = K Q^T (keys on the MFMA M
// dimension) so each lane holds one query column and 32 keys of a 64-key
// block: the row max needs one cross-half exchange and the row sum none.
// Q^T stays in registers as the B operand.  K and V tiles go from HBM
// straight into LDS with global_load_lds (no register staging), two stages,
// the next block's copy in flight while the current block is computed; V is
// kept in its natural layout and read transposed with ds_read_b64_tr_b16.
// P^T feeds the O^T += V^T P^T MFMAs directly from the accumulators (see
// fa_common.h).  Two workgroups share a CU (64 KB LDS each at head_dim 128),
// so one wave's softmax overlaps the other's MFMAs on each SIMD.
#include <type_traits>

#include "fa_common.h"

namespace fa {

template <int HD>
struct FwdCfg {
    static constexpr int NT = 256;                // threads
    static constexpr int OCC = 2;                 // workgroups per CU
    static constexpr int BM = 32 * (NT / 64);     // queries per workgroup (32 per wave)
    static constexpr int BN = 64;                 // keys per block
    static constexpr int KCH = HD / 8;            // 16-byte chunks per row
    static constexpr int TILE = BN * HD * 2;      // one K or V tile
    static constexpr int STAGE = 2 * TILE;        // K tile, then V tile
};

// The running maximum m a row's probabilities P = exp2(S*c - m) are taken
// against is raised (and O, l rescaled) only in the blocks where some row of
// the wave finds a score more than kRescaleSlack above it, so most blocks skip
// the rescale; P then stays below 2^kRescaleSlack, well inside fp16.  O is
// normalised by the sum of the fp16-rounded P that the PV product used
// (l_o), so O = sum P V / l_o is built from consistent weights: a row
// dominated by one key returns that key's V exactly whatever the stale
// maximum, as it does with P = 1 in the reference.  The LSE uses the fp32 sum
// of the unrounded P (l_p), as the reference does.
constexpr float kRescaleSlack = 8.f;

// Sum of the eight fp16 values of an MFMA operand, accumulated in fp32.
__device__ __forceinline__ float sum8(const f16x8 &v, float acc) {
    typedef f16 f16x2 __attribute__((ext_vector_type(2)));
    const f16x2 one = {f16(1), f16(1)};
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(v, v, 0, 1), one, acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(v, v, 2, 3), one, acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(v, v, 4, 5), one, acc, false);
    return __builtin_amdgcn_fdot2(__builtin_shufflevector(v, v, 6, 7), one, acc, false);
}

template <int HD, bool CAUSAL>
__global__ __launch_bounds__(FwdCfg<HD>::NT, FwdCfg<HD>::OCC) void fwd_kernel(const fa_fwd_args a, const int num_m_blocks) {
    using C = FwdCfg<HD>;
    constexpr int BM = C::BM, BN = C::BN, NT = C::NT;
    __shared__ __attribute__((aligned(16))) char smem[2 * C::STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int col = lane & 31, hh = lane >> 5;

    // Causal blocks are issued heaviest (largest m block) first.
    const int bh_count = a.batch * a.nheads;
    const int bh = blockIdx.x % bh_count;
    int mb = blockIdx.x / bh_count;
    if (CAUSAL) mb = num_m_blocks - 1 - mb;
    const int b = bh / a.nheads, h = bh - b * a.nheads;
    const int hk = h / (a.nheads / a.nheads_k);

    const bool packed_q = a.cu_seqlens_q != nullptr, packed_k = a.cu_seqlens_k != nullptr;
    const SeqInfo si = seq_info(b, a.seqlen_q, a.seqlen_k, a.cu_seqlens_q, a.cu_seqlens_k, a.seqused_k,
                                a.seqused_k_add);
    const int sq = si.sq;
    int sk = si.sk;
    int kb = a.k_batch_idx ? a.k_batch_idx[b] : b;
    if (a.seqused_k) {
        // KV-cache chunk: a key count past the cache or a cache row outside it
        // leaves the batch with no keys, and the error goes to the status word.
        const int used = a.seqused_k[b];
        const int err = (used < 0 || int64_t(used) + a.seqused_k_add > a.seqlen_k ? 1 : 0) |
                        (a.k_batch_idx && a.k_batch > 0 && (kb < 0 || kb >= a.k_batch) ? 2 : 0);
        if (err) {
            sk = 0;
            kb = 0;
            if (a.status && tid == 0) atomicOr(a.status, err);
        }
    }
    const int m0 = mb * BM;
    float *lse_row = a.lse + (int64_t(b) * a.nheads + h) * a.lse_seqlen;
    if (m0 >= sq) {
        // Rows past this sequence's length: LSE padding is 0 (flash_api.cpp:388).
        for (int i = m0 + tid; i < m0 + BM && i < a.lse_seqlen; i += NT) lse_row[i] = 0.f;
        return;
    }
    const f16 *qp = (const f16 *)a.q.ptr + base_off(a.q, packed_q, b, si.q_start, h);
    const f16 *kp = (const f16 *)a.k.ptr + base_off(a.k, packed_k, kb, si.k_start, hk);
    const f16 *vp = (const f16 *)a.v.ptr + base_off(a.v, packed_k, kb, si.k_start, hk);
    f16 *op = (f16 *)a.o.ptr + base_off(a.o, packed_q, b, si.q_start, h);
    const int64_t qrs = a.q.row_stride, krs = a.k.row_stride, vrs = a.v.row_stride, ors = a.o.row_stride;

    const int causal_off = sk - sq;  // key j visible to query i iff j <= i + causal_off
    int n_end = sk;
    if (CAUSAL) n_end = max(0, min(sk, m0 + BM + causal_off));
    const int n_blocks = (n_end + BN - 1) / BN;

    // Negative scales are folded into Q's sign so that the exp argument uses |scale|.
    const bool neg = a.softmax_scale < 0.f;
    const float cscale = fabsf(a.softmax_scale) * kLog2e;

    // Q^T as the B operand: lane (query col, half hh), K step g covers d = 16g + 8hh + 0..7.
    const int qi = m0 + wave * 32 + col;
    f16x8 qB[HD / 16];
#pragma unroll
    for (int g = 0; g < HD / 16; ++g) {
        u32x4 v = zero_u4();
        if (qi < sq) v = ldg16(qp + int64_t(qi) * qrs + 16 * g + 8 * hh);
        if (neg) v = neg_h8(v);
        qB[g] = as_h8(v);
    }
    wait_vmem();  // only the tile copies are in flight inside the loop

    f32x16 o[HD / 32];
#pragma unroll
    for (int i = 0; i < HD / 32; ++i) o[i] = zero16();
    float m_t = -INFINITY;  // reference max of scale*log2(e)*S for this lane's query
    float l_p = 0.f;        // partial row sum over this lane half's keys (fp32 P, for the LSE)
    float l_o = 0.f;        // the same over the fp16-rounded P (normalises O)

    TileReader<HD> rd;
    rd.init(lane);
    TileCopier<HD, BN, NT> kcp, vcp;
    kcp.init(krs, wave, lane);
    vcp.init(vrs, wave, lane);
    // Copy of key block nb into stage st.  A block that runs past the
    // sequence re-reads its last key for the missing rows (masked below).
    const uint32_t smem_l = lds_addr(smem);
    auto issue = [&](int nb, int st) {
        char *ks = smem + st * C::STAGE;
        const int n0 = nb * BN;
        if (n0 + BN <= sk) {
            kcp.copy_to(smem_l + st * C::STAGE, kp + int64_t(n0) * krs, krs);
            vcp.copy_to(smem_l + st * C::STAGE + C::TILE, vp + int64_t(n0) * vrs, vrs);
        } else {
            dma_tile<HD, BN, NT>(ks, kp, krs, n0, sk - 1, wave, lane);
            dma_tile<HD, BN, NT>(ks + C::TILE, vp, vrs, n0, sk - 1, wave, lane);
        }
    };

    const int q_lo = m0 + wave * 32;
    // One key block: S^T = K Q^T, online softmax, O^T += V^T P^T.  MASK is a
    // compile-time switch so the blocks away from the causal diagonal and
    // the sequence end carry no masking work at all.
    auto block = [&](int nb, auto mask_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int buf = nb & 1;
        wait_vmem();
        __syncthreads();  // block nb is in LDS; every wave is done with stage buf ^ 1
        if (nb + 1 < n_blocks) issue(nb + 1, buf ^ 1);
        const int n0 = nb * BN;
        if (CAUSAL && MASK && n0 > q_lo + 31 + causal_off) return;  // no visible key for this wave
        const char *ks = smem + buf * C::STAGE;
        const char *vs = ks + C::TILE;
        f32x16 s[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            s[kt] = mfma32(rd.a_operand(ks, 32 * kt, 0), qB[0], zero16());
#pragma unroll
            for (int g = 1; g < HD / 16; ++g) s[kt] = mfma32(rd.a_operand(ks, 32 * kt, g), qB[g], s[kt]);
        }
        if constexpr (MASK) {
            const int lim = (CAUSAL ? min(sk - 1, qi + causal_off) : sk - 1) - n0;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (kt * 32 + acc_lrow(r, hh) > lim) s[kt][r] = -INFINITY;
        }
        float mx = s[0][0];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kt][r]);
        mx = max_xor32(mx);
        const float mx_t = MASK && mx == -INFINITY ? -INFINITY : mx * cscale;
        if (__builtin_amdgcn_ballot_w64(mx_t > m_t + kRescaleSlack) != 0) {
            const float m_new = fmaxf(m_t, mx_t);
            const float alpha = m_new == -INFINITY ? 1.f : exp2_fast(m_t - m_new);
            l_p *= alpha;
            l_o *= alpha;
#pragma unroll
            for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
            m_t = m_new;
        }
        const float m_use = m_t == -INFINITY ? 0.f : m_t;
        float rs = 0.f;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float x = s[kt][r];
                float p = exp2_fast(fmaf(x, cscale, -m_use));
                if constexpr (MASK) p = x == -INFINITY ? 0.f : p;
                s[kt][r] = p;
                rs += p;
            }
        l_p += rs;
        f16x8 pB[4];
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
            pB[gg] = pack8(s[gg >> 1], 8 * (gg & 1));
            l_o = sum8(pB[gg], l_o);
        }
#pragma unroll
        for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
            for (int gg = 0; gg < 4; ++gg) o[dt] = mfma32(rd.tr_operand(vs, 16 * gg, dt), pB[gg], o[dt]);
    };

    // Blocks [0, n_full) need no mask for any wave of the workgroup: every key
    // is below the sequence end and at or below the diagonal of the first query.
    int n_full = min(n_blocks, sk / BN);
    if (CAUSAL) n_full = min(n_full, max(0, (m0 + causal_off + 1) / BN));
    if (n_blocks > 0) issue(0, 0);
    for (int nb = 0; nb < n_full; ++nb) block(nb, std::false_type{});
    for (int nb = n_full; nb < n_blocks; ++nb) block(nb, std::true_type{});

    // Epilogue: O / l in fp16, LSE = ln(sum exp(scale*S)); empty rows give 0 / 0.
    const float l_tot = sum_xor32(l_p);
    const float lo_tot = sum_xor32(l_o);
    if (qi < sq) {
        const float inv = lo_tot > 0.f ? 1.f / lo_tot : 0.f;
        f16 *orow = op + int64_t(qi) * ors;
#pragma unroll
        for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                f16x4 v;
#pragma unroll
                for (int t = 0; t < 4; ++t) v[t] = (f16)(o[dt][4 * a4 + t] * inv);
                *reinterpret_cast<f16x4 *>(orow + dt * 32 + 8 * a4 + 4 * hh) = v;
            }
        if (hh == 0) lse_row[qi] = l_tot > 0.f ? (m_t + log2_fast(l_tot)) * kLn2 : 0.f;
    } else if (hh == 0 && qi < a.lse_seqlen) {
        lse_row[qi] = 0.f;
    }
}

template <int HD, bool CAUSAL>
static int launch_fwd(const fa_fwd_args &a, hipStream_t stream) {
    const int num_m_blocks = (a.lse_seqlen + FwdCfg<HD>::BM - 1) / FwdCfg<HD>::BM;
    const int64_t grid = int64_t(num_m_blocks) * a.batch * a.nheads;
    if (grid == 0) return FA_OK;
    if (grid > 0x7fffffff) return FA_ERR_INVALID_ARG;
    hipLaunchKernelGGL((fwd_kernel<HD, CAUSAL>), dim3(unsigned(grid)), dim3(FwdCfg<HD>::NT), 0, stream, a,
                       num_m_blocks);
    return int(hipGetLastError());
}

}  // namespace fa

extern "C" int fa_check_tensor(const fa_tensor &t, bool required);

extern "C" int fa_fwd(const fa_fwd_args *args, void *stream) {
    if (!args) return FA_ERR_INVALID_ARG;
    const fa_fwd_args &a = *args;
    if (a.head_dim != 64 && a.head_dim != 128) return FA_ERR_UNSUPPORTED;
    if (a.batch < 0 || a.seqlen_q < 0 || a.seqlen_k < 0 || a.nheads <= 0 || a.nheads_k <= 0 ||
        a.nheads % a.nheads_k != 0 || !a.lse || a.lse_seqlen < a.seqlen_q)
        return FA_ERR_INVALID_ARG;
    if (fa_check_tensor(a.q, true) || fa_check_tensor(a.k, true) || fa_check_tensor(a.v, true) ||
        fa_check_tensor(a.o, true))
        return FA_ERR_INVALID_ARG;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (a.head_dim == 128)
        return a.causal ? fa::launch_fwd<128, true>(a, s) : fa::launch_fwd<128, false>(a, s);
    return a.causal ? fa::launch_fwd<64, true>(a, s) : fa::launch_fwd<64, false>(a, s);
}
