// Device helpers shared by the gfx950 attention kernels.
//
// MFMA conventions (v_mfma_f32_32x32x16_f16, wave64):
//   A operand (32 x 16): lane l supplies row l%32, K slots 8*(l/32)+0..7
//   B operand (16 x 32): lane l supplies column l%32, K slots 8*(l/32)+0..7
//   C/D (32 x 32, 16 fp32 per lane): lane l holds column l%32 and rows
//       8*(r/4) + 4*(l/32) + r%4 for accumulator r = 0..15.
//
// Chaining an accumulator tile into the K dimension of the next MFMA:
// the rows of a C tile live in a lane in two runs (r = 0..7, r = 8..15).  If
// the first GEMM's operand that supplies those rows is loaded with the row
// permutation sigma (swap bits 2 and 3 of the row index), accumulator
// r of lane half h holds logical row 16*(r/8) + 8*h + r%8.  Accumulators
// 8g..8g+7 of a lane are then exactly the 8 consecutive logical rows that
// lane supplies in K step g of a following MFMA, so S^T / P^T / dS^T tiles
// feed the PV, dV, dK and dQ products with no data movement (a C tile is
// the B operand of the same matrix, and the A operand of its transpose).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fa_mi355x.h"

namespace fa {

// Compute units of the current device (host; fa_abi.hip).
int device_cus();
// FA_OK when t is usable by the kernels: a 16-byte aligned base and strides that
// keep every row and head 16-byte aligned; a null pointer is an error only when
// required (host; fa_abi.hip).
int check_tensor(const fa_tensor &t, bool required);

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Forces a lambda used inside a kernel's hot loop to be inlined.
#define FA_INLINE __attribute__((always_inline))

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ f32x16 mfma32(const f16x8 a, const f16x8 b, const f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.f;
    return z;
}

// Row permutation applied when loading rows that a later MFMA consumes along K.
__device__ __forceinline__ int sigma(int i) {
    return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1);
}
// Logical row (0..31) of accumulator r in lane half h for a sigma-loaded tile.
__device__ __forceinline__ int acc_lrow(int r, int h) { return 16 * (r >> 3) + 8 * h + (r & 7); }
// Natural row of accumulator r in lane half h (no permutation at load).
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// Maximum / sum of x over lanes l and l ^ 32, in every lane.  v_permlane32_swap
// of x with itself leaves x[l % 32] in one result and x[l % 32 + 32] in the
// other, so this is one VALU op instead of an LDS round trip (ds_bpermute);
// both halves compute lo + hi in the same order, so the sum is the same bits
// in all lanes.
__device__ __forceinline__ float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float log2_fast(float x) { return __builtin_amdgcn_logf(x); }

// ---------------------------------------------------------------------------
// LDS tiles are addressed in 16-byte chunks with an XOR swizzle of the chunk
// index (swz below), so MFMA operand reads and transposed reads are
// bank-conflict free.

__device__ __forceinline__ f16x8 lds_ld16(const char *base, int off) {
    return *reinterpret_cast<const f16x8 *>(base + off);
}

// ---------------------------------------------------------------------------
// gfx950 direct global -> LDS copies and LDS transpose reads.

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4_t;

// global_load_lds_dwordx4: lane l's 16 bytes at `g` land at lds_base + 16*l.
// lds_base must be the same for the whole wave.  Issued from inline assembly
// (M0 saved and restored around it) so that the compiler does not treat the
// copy as a pending write to all of LDS: its automatic waits would otherwise
// stall every transposed LDS read until the prefetched tile has landed.  The
// compiler therefore does not count these copies either: wait for them
// explicitly (wait_vmem / wait_vmem_n) before a barrier that publishes the
// tile, and issue no other vector-memory loads while copies are in flight
// (the compiler's own waits for those would then also cover the copies).
// An SALU write of M0 needs one wait state before an LDS-DMA load reads it
// (the CDNA manually-inserted wait states; the compiler inserts none inside
// inline assembly), hence the s_nop after each M0 write below.
__device__ __forceinline__ void g2l16(const void *g, char *lds_base) {
    const uint32_t l =
        __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)lds_base);
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(g), "s"(l)
        : "memory");
}
// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const char *p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char *)p;
}
// N (1, 2 or 4) global_load_lds_dwordx4 copies with one M0 save / restore:
// copy i moves lane l's 16 bytes at g[i] to LDS byte l[i] + 16*l, where l[i]
// are wave-uniform LDS addresses.  Same waiting rules as g2l16.
template <int N>
__device__ __forceinline__ void g2l16_batch(const void *const (&g)[N], const uint32_t (&l)[N]) {
    uint32_t saved;
    if constexpr (N == 1) {
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %2\n\t"
            "s_nop 0\n\t"
            "global_load_lds_dwordx4 %1, off\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "v"(g[0]), "s"(l[0])
            : "memory");
    } else if constexpr (N == 2) {
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %3\n\t"
            "s_nop 0\n\t"
            "global_load_lds_dwordx4 %1, off\n\t"
            "s_mov_b32 m0, %4\n\t"
            "s_nop 0\n\t"
            "global_load_lds_dwordx4 %2, off\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "v"(g[0]), "v"(g[1]), "s"(l[0]), "s"(l[1])
            : "memory");
    } else {
        static_assert(N == 4, "batches of 1, 2 or 4 copies");
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %5\n\t"
            "s_nop 0\n\t"
            "global_load_lds_dwordx4 %1, off\n\t"
            "s_mov_b32 m0, %6\n\t"
            "s_nop 0\n\t"
            "global_load_lds_dwordx4 %2, off\n\t"
            "s_mov_b32 m0, %7\n\t"
            "s_nop 0\n\t"
            "global_load_lds_dwordx4 %3, off\n\t"
            "s_mov_b32 m0, %8\n\t"
            "s_nop 0\n\t"
            "global_load_lds_dwordx4 %4, off\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "v"(g[0]), "v"(g[1]), "v"(g[2]), "v"(g[3]), "s"(l[0]), "s"(l[1]), "s"(l[2]), "s"(l[3])
            : "memory");
    }
}
// global_load_lds_dword to a wave-uniform LDS byte address l: lane l's 4 bytes land at l + 4*lane.
__device__ __forceinline__ void g2l4_to(const void *g, uint32_t l) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dword %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(g), "s"(__builtin_amdgcn_readfirstlane(l))
        : "memory");
}
// s_waitcnt vmcnt(0) (expcnt / lgkmcnt left at their maxima).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// s_waitcnt lgkmcnt(0): every LDS read issued so far has returned its data.
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// s_waitcnt vmcnt(N), N < 64.
template <int N>
__device__ __forceinline__ void wait_vmem_n() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// ds_read_b64_tr_b16.  Within each group of 16 lanes, lane i receives element
// j (j = 0..3) = the 16-bit word at (address of group lane 4*j + i/4) + 2*(i%4)
// bytes.  Pointing group lane s = 4*j + q at row r0 + j, column c0 + 4*q of a
// row-major fp16 tile therefore hands lane i the 4 words (r0 + j, c0 + i):
// a 4-row x 16-column block transposed across the 16 lanes.
__device__ __forceinline__ f16x4 lds_tr4(const char *base, int off) {
    return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t *)(base + off)));
}

// Placement of a natural [rows][KCH 16-byte chunks] fp16 tile in LDS: chunk c
// of row r sits at chunk c ^ swz(r).  The XOR masks are chosen so that both
// read patterns the kernels use are bank-conflict free with 64 four-byte
// banks (16 lanes per ds_read_b128 phase, 32 per ds_read_b64 phase):
//   * MFMA A-operand rows: lanes read rows sigma(0..31) at one chunk pair;
//   * lds_tr4 transposed reads: 8 rows x 64 bytes per instruction.
// At head_dim 64 two rows share a 256-byte bank window, so the 8 rows of
// each parity in a 16-lane phase need 8 distinct chunks: the mask uses row
// bits 1, 2 and 3 (an exhaustive search over XOR masks of the row bits for
// both read patterns).  Both masks repeat every 16 rows, as TileCopier needs.
template <int KCH>
__device__ __forceinline__ int swz(int row) {
    if constexpr (KCH == 16)
        return ((row & 1) ? 4 : 0) ^ ((row & 2) ? 10 : 0) ^ ((row & 4) ? 2 : 0) ^ ((row & 8) ? 1 : 0);
    else
        return ((row & 2) ? 4 : 0) ^ ((row & 4) ? 1 : 0) ^ ((row & 8) ? 2 : 0);
}

// Copy rows [row0, row0 + ROWS) of a [rows][HD] fp16 source (row stride rs,
// rows clamped to <= last_row) into a swizzled natural tile with DMA: the NT
// threads of the workgroup each move ROWS*HD/8/NT chunks.  General form (any
// row0, clamping per row); TileCopier below is the fast path.
template <int HD, int ROWS, int NT>
__device__ __forceinline__ void dma_tile(char *tile, const f16 *src, int64_t rs, int row0, int last_row, int wave,
                                         int lane) {
    constexpr int KCH = HD / 8, CPT = ROWS * KCH / NT, WAVES = NT / 64;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int base = (i * WAVES + wave) * 64;
        const int p = base + lane, row = p / KCH, cs = p % KCH;
        const int64_t r = min(row0 + row, last_row);
        g2l16(src + r * rs + 8 * (cs ^ swz<KCH>(row)), tile + base * 16);
    }
}

// Unclamped tile copy with the per-lane source offsets computed once: copy i
// of a lane moves chunk cs of row row_l + i * (NT / KCH); NT / KCH is a
// multiple of 16, so the swizzle of every copy equals that of row_l.
template <int HD, int ROWS, int NT>
struct TileCopier {
    static constexpr int KCH = HD / 8, CPT = ROWS * KCH / NT, WAVES = NT / 64, RSTEP = NT / KCH;
    static_assert(RSTEP % 16 == 0, "row step must keep the swizzle");
    int64_t goff;  // elements from row 0 of the tile to this lane's chunk of copy 0
    int lds0;      // byte offset of copy 0's wave chunk block in the tile
    __device__ __forceinline__ void init(int64_t rs, int wave, int lane) {
        const int p = wave * 64 + lane, row = p / KCH, cs = p % KCH;
        goff = int64_t(row) * rs + 8 * (cs ^ swz<KCH>(row));
        lds0 = wave * 64 * 16;
    }
    // src_row0: element pointer of the tile's first row (wave-uniform).  The
    // copies go out as one batch (one M0 save / restore, LDS addresses as
    // scalar offsets of the tile's base).
    __device__ __forceinline__ void copy(char *tile, const f16 *src_row0, int64_t rs) const {
        copy_to(lds_addr(tile), src_row0, rs);
    }
    // The same with the tile given as its LDS byte address (no pointer cast in the loop).
    // FRESH: the per-copy lane addresses are formed on every call (one 64-bit add
    // each; the offset is opaque to the optimiser) instead of being hoisted out
    // of the caller's loop as CPT loop-invariant pointers held in registers.
    template <bool FRESH = false>
    __device__ __forceinline__ void copy_to(uint32_t tile_l, const f16 *src_row0, int64_t rs) const {
        const uint32_t l0 = __builtin_amdgcn_readfirstlane(tile_l + lds0);
        int64_t go = goff;
        if constexpr (FRESH) asm volatile("" : "+v"(go));
        if constexpr (CPT == 1 || CPT == 2 || CPT == 4) {
            const void *g[CPT];
            uint32_t l[CPT];
#pragma unroll
            for (int i = 0; i < CPT; ++i) {
                g[i] = src_row0 + go + int64_t(i) * RSTEP * rs;
                l[i] = l0 + i * WAVES * 1024;
            }
            g2l16_batch<CPT>(g, l);
        } else {
            static_assert(CPT == 1 || CPT == 2 || CPT == 4, "copies per lane");
        }
    }
};

// Per-lane LDS byte offsets of the MFMA operand reads from swizzled natural
// tiles, computed once per kernel.  A chunk index c = 2g + h (or 4dt + x) XOR
// a per-lane swizzle equals the g = 0 (dt = 0) chunk XOR (g << 1) (dt << 2),
// so every read is one v_xor plus a ds_read with an immediate row offset.
template <int HD>
struct TileReader {
    int a_base;      // A operand: row sigma(col), chunk hh (g = 0)
    int tr_base[2];  // transposed operand: rows 8h + j and 8h + j + 4, column block of dt = 0
    __device__ __forceinline__ void init(int lane) {
        constexpr int KCH = HD / 8;
        const int col = lane & 31, h = lane >> 5;
        const int row = sigma(col);
        a_base = row * (HD * 2) + (((h ^ swz<KCH>(row)) & (KCH - 1)) << 4);
        const int j = (lane & 15) >> 2, q = lane & 3, db = (lane >> 4) & 1;
        const int x = 2 * db + (q >> 1), byte = (q & 1) * 8;
#pragma unroll
        for (int hs = 0; hs < 2; ++hs) {
            const int r = 8 * h + j + 4 * hs;
            tr_base[hs] = r * (HD * 2) + (((x ^ swz<KCH>(r)) & (KCH - 1)) << 4) + byte;
        }
    }
    // A operand (32 x 16): lane (m, h) gets chunk 2g + h of row r0 + sigma(m); r0 % 32 == 0.
    __device__ __forceinline__ f16x8 a_operand(const char *tile, int r0, int g) const {
        return lds_ld16(tile + r0 * (HD * 2), a_base ^ (g << 5));
    }
    // Transposed A operand: lane (m, h) gets column 32*dt + m of rows r0 + 8h + 0..7; r0 % 16 == 0.
    __device__ __forceinline__ f16x8 tr_operand(const char *tile, int r0, int dt) const {
        const char *t = tile + r0 * (HD * 2);
        const f16x4 lo = lds_tr4(t, tr_base[0] ^ (dt << 6));
        const f16x4 hi = lds_tr4(t, tr_base[1] ^ (dt << 6));
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
    // The same reads from lane bases that already include a tile offset t, a
    // multiple of 512 bytes: the step XOR (g << 5, dt << 6: bits 5-7) and the
    // add of t (bits 9 and up, no carry out of the low bits) commute, so
    // (base + t) ^ m == (base ^ m) + t.  A caller forms base + t once per tile
    // and each read is then one XOR, the rest of the address an immediate.
    __device__ __forceinline__ f16x8 a_operand_at(const char *lds0, int base_t, int g) const {
        return lds_ld16(lds0, base_t ^ (g << 5));
    }
    __device__ __forceinline__ f16x8 tr_operand_at(const char *lds0, int b0_t, int b1_t, int dt) const {
        const f16x4 lo = lds_tr4(lds0, b0_t ^ (dt << 6));
        const f16x4 hi = lds_tr4(lds0, b1_t ^ (dt << 6));
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
};

// ---------------------------------------------------------------------------
// Global memory.

__device__ __forceinline__ u32x4 ldg16(const f16 *p) { return *reinterpret_cast<const u32x4 *>(p); }
__device__ __forceinline__ u32x4 zero_u4() {
    u32x4 z;
    z[0] = z[1] = z[2] = z[3] = 0u;
    return z;
}
__device__ __forceinline__ f16x8 as_h8(const u32x4 v) { return __builtin_bit_cast(f16x8, v); }
__device__ __forceinline__ u32x4 neg_h8(const u32x4 v) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = v[i] ^ 0x80008000u;
    return r;
}

// 8 fp32 accumulators -> one fp16x8 MFMA operand (round to nearest even).
__device__ __forceinline__ f16x8 pack8(const f32x16 &acc, int base) {
    f16x8 r;
#pragma unroll
    for (int t = 0; t < 8; ++t) r[t] = (f16)acc[base + t];
    return r;
}

// ---------------------------------------------------------------------------
// Longest-first work lists for varlen grids.  One workgroup of kOrderThreads
// counting-sorts items [0, n_items) by bucket(it) (0 .. kOrderBuckets - 1,
// larger = more work; -1 = no work): a histogram, a scan over the buckets in
// descending order, then a scatter through per-bucket cursors.  out[] gets the
// items largest bucket first, then the empty items (their ids when keep_empty,
// for kernels that still have padding to write, else -1).  Order within a
// bucket follows the LDS atomics; every item is computed independently, so
// results do not depend on it.
constexpr int kOrderThreads = 1024, kOrderBuckets = 1024;

template <class Bucket>
__device__ __forceinline__ void order_items(int n_items, Bucket bucket, int32_t *out, bool keep_empty) {
    static_assert(kOrderThreads == kOrderBuckets, "one histogram bucket and one scan slot per thread");
    __shared__ int hist[kOrderBuckets];
    __shared__ int scan[kOrderBuckets];
    __shared__ int n_empty;
    const int tid = threadIdx.x;
    hist[tid] = 0;
    if (tid == 0) n_empty = 0;
    __syncthreads();
    for (int it = tid; it < n_items; it += kOrderThreads) {
        const int k = bucket(it);
        if (k >= 0) atomicAdd(&hist[k], 1);
    }
    __syncthreads();
    // Inclusive scan of the counts in descending bucket order (slot t = bucket kOrderBuckets - 1 - t).
    const int c = hist[kOrderBuckets - 1 - tid];
    scan[tid] = c;
    __syncthreads();
    for (int d = 1; d < kOrderBuckets; d <<= 1) {
        const int v = tid >= d ? scan[tid - d] : 0;
        __syncthreads();
        scan[tid] += v;
        __syncthreads();
    }
    hist[kOrderBuckets - 1 - tid] = scan[tid] - c;  // first slot of the bucket
    const int total = scan[kOrderBuckets - 1];
    __syncthreads();
    for (int it = tid; it < n_items; it += kOrderThreads) {
        const int k = bucket(it);
        if (k >= 0)
            out[atomicAdd(&hist[k], 1)] = it;
        else if (keep_empty)
            out[total + atomicAdd(&n_empty, 1)] = it;
    }
    if (!keep_empty)
        for (int i = total + tid; i < n_items; i += kOrderThreads) out[i] = -1;
}

// Per-batch extents of a dense or packed (varlen) batch.
struct SeqInfo {
    int q_start, sq, k_start, sk;
};

__device__ __forceinline__ SeqInfo seq_info(int b, int seqlen_q, int seqlen_k, const int32_t *cu_q,
                                            const int32_t *cu_k, const int32_t *seqused_k, int seqused_add) {
    SeqInfo s;
    s.q_start = 0;
    s.sq = seqlen_q;
    s.k_start = 0;
    s.sk = seqlen_k;
    if (cu_q) {
        s.q_start = cu_q[b];
        s.sq = cu_q[b + 1] - s.q_start;
    }
    if (cu_k) {
        s.k_start = cu_k[b];
        s.sk = cu_k[b + 1] - s.k_start;
    } else if (seqused_k) {
        s.sk = seqused_k[b] + seqused_add;
    }
    return s;
}

// Element offset of (batch b / packed row start, head) in a strided tensor.
__device__ __forceinline__ int64_t base_off(const fa_tensor &t, bool packed, int b, int row_start, int head) {
    return (packed ? int64_t(row_start) * t.row_stride : int64_t(b) * t.batch_stride) +
           int64_t(head) * t.head_stride;
}

}  // namespace fa
