// Hardware ceilings of one MI355X (gfx950) for the attention kernels' rooflines:
//   * v_mfma_f32_32x32x16_f16 throughput and the shader clock it runs at, with
//     operands in registers and in the forward's matrix-phase pattern (K as
//     ds_read_b128 A operands, V^T either as ds_read_b64_tr_b16 transposed
//     reads or as ds_read_b128 from a transposed tile), one or two waves per
//     SIMD, and with 64 queries per wave (each operand read feeds two MFMAs);
//   * LDS instruction costs per CU with many reads / writes in flight:
//     ds_read_b128, ds_read_b64_tr_b16, ds_write_b128, ds_write_b64;
//   * VALU issue costs: v_exp_f32 alone, v_fma_f32 alone, the two interleaved,
//     and v_exp_f32 beside MFMAs of the same wave (the softmax's mix);
//   * HBM read bandwidth: contiguous, and in 128 / 256 / 512-byte pieces at a
//     2 KB stride (one / two / four heads of a head-interleaved KV cache row).
// Timing only.  Every LDS address stays inside the workgroup's buffer and every
// global address inside the allocation; every loop is bounded.  The on-chip probes
// time their loops from inside: each wave stamps s_memrealtime (100 MHz) and
// s_memtime (shader cycles) around its loop, and a rate is taken over the span from
// the first wave's start to the last wave's end, at the clock those stamps give.
// (Event time over the whole launch also counts the operand set-up before the
// loops, which in an earlier form of this file was most of a millisecond.)
//
// Build: build.py compiles it to probes/ceiling_probe.  Run: ceiling_probe [iters].
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#define CHECK(x)                                                                              \
    do {                                                                                      \
        hipError_t e_ = (x);                                                                  \
        if (e_ != hipSuccess) {                                                               \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);        \
            std::exit(1);                                                                     \
        }                                                                                     \
    } while (0)

namespace {

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x16 mfma(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f16x4 tr4(const char *p) {
    return __builtin_bit_cast(
        f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4 *)(p)));
}

constexpr int kLdsUsed = 64 * 1024;   // the probes address the first 64 KB
constexpr int kLdsAlloc = 96 * 1024;  // more than half the CU's 160 KB: one workgroup per CU
constexpr int kPipe = 8;              // operand reads run this many MFMA steps ahead

enum Mode {
    kMfmaRegs,      // 32 MFMAs per step on register operands, 6 accumulator chains
    kMatrixTr,      // forward matrix phase: 16 PV MFMAs (V^T by 2 transposed reads) + 16 S MFMAs (K b128)
    kMatrixVt,      // the same with V^T as a transposed tile read by ds_read_b128
    kMatrix64q,     // 64 queries per wave: each of the 32 operand reads feeds two MFMAs
    kReadB128,      // 16 ds_read_b128 in flight per step
    kReadTr,        // 32 ds_read_b64_tr_b16 in flight per step
    kWriteB128,     // 16 ds_write_b128 per step
    kWriteB64,      // 16 ds_write_b64 per step
    kExp,           // 32 v_exp_f32 per step, 8 independent chains
    kFma,           // 32 v_fma_f32 per step, 8 independent chains
    kExpFma,        // 32 v_exp_f32 and 32 v_fma_f32 per step, interleaved
    kMfmaExp,       // 16 MFMAs (register operands) and 32 v_exp_f32 per step in the same wave
    kMfmaFma,       // 16 MFMAs and 64 v_fma_f32 per step in the same wave (4 between MFMAs)
    kMfmaSoft,      // 16 MFMAs, 32 v_exp_f32 and 96 v_fma_f32 per step in the same wave (a softmax's mix)
    kSplitFma,      // two waves per SIMD: one issues MFMAs (32 per step), the other v_fma_f32 (384 per step)
    kSplitExp,      // the same with v_exp_f32 (112 per step) in the second wave
};

struct Stamp {
    long long cycles, t0, t1;  // s_memtime span and s_memrealtime start / end of one wave's loop
};

template <int MODE, int NT>
__global__ __launch_bounds__(NT, 1) void probe_kernel(float *sink, Stamp *stamp, int iters) {
    __shared__ __attribute__((aligned(16))) char smem[kLdsAlloc];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Pseudo-random fp16 in [-1, 1]: the matrix cores' power (and so the clock) depends on the data.
    for (int i = tid; i < kLdsUsed / 2; i += NT) {
        const unsigned h = (unsigned(i) * 2654435761u) ^ (unsigned(i) >> 7);
        reinterpret_cast<f16 *>(smem)[i] = f16(float(int(h % 2001u) - 1000) * 0.001f);
    }
    // Operands with constant indices only (fully unrolled), so they live in registers.
    f16x8 q[8], p[4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) q[i][e] = f16(0.01f * float(((lane * 37 + i * 11 + e * 7) % 201) - 100));
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) p[i][e] = f16(0.01f * float(((lane * 53 + i * 13 + e * 5) % 199) - 99));
    f32x16 o[4], s[2], o2[4], s2[2];
    float ex[8], fx[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) ex[c] = fx[c] = 0.25f + 0.01f * float(c + (lane & 7));
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[i][e] = o2[i][e] = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[i][e] = s2[i][e] = 0.f;
    __syncthreads();
    const long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    // Tiles swizzled as the kernels' are: 16-byte chunk c of row r at c ^ (r & 15) (256-byte rows),
    // or c ^ ((r >> 1) & 7) for the 128-byte rows of a transposed V tile.
    const int arow = lane & 31;
    const int abase = arow * 256 + (((lane >> 5) ^ (arow & 15)) << 4);
    const int tx = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1), tbyte = (lane & 1) * 8;
    const int tr0 = 8 * (lane >> 5) + ((lane & 15) >> 2), tr1 = tr0 + 4;
    const int trb0 = tr0 * 256 + ((tx ^ (tr0 & 15)) << 4) + tbyte;
    const int trb1 = tr1 * 256 + ((tx ^ (tr1 & 15)) << 4) + tbyte;
    for (int it = 0; it < iters; ++it) {
        const char *ks = smem + ((it + wave) & 1) * 32768;  // a 16 KB K tile, then a 16 KB V tile
        const char *vs = ks + 16384;
        if constexpr (MODE == kMfmaRegs) {
#pragma unroll
            for (int t = 0; t < 32; ++t) {
                if (t < 16)
                    o[t & 3] = mfma(q[t & 7], p[t & 3], o[t & 3]);
                else
                    s[t & 1] = mfma(q[t & 7], p[t & 3], s[t & 1]);
            }
        } else if constexpr (MODE == kMatrixTr || MODE == kMatrixVt || MODE == kMatrix64q) {
            f16x8 opnd[kPipe];
            auto read = [&](int t) {
                if (t < 16 && MODE == kMatrixVt) {
                    const int d = 32 * (t & 3) + (lane & 31), kc = 2 * (t >> 2) + (lane >> 5);
                    opnd[t % kPipe] = *reinterpret_cast<const f16x8 *>(vs + d * 128 + ((kc ^ ((d >> 1) & 7)) << 4));
                } else if (t < 16) {
                    const char *b = vs + 16 * (t & 3) * 256;
                    const f16x4 lo = tr4(b + (trb0 ^ ((t >> 2) << 6))), hi = tr4(b + (trb1 ^ ((t >> 2) << 6)));
                    opnd[t % kPipe] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                } else {
                    const int u = t - 16;
                    opnd[t % kPipe] = *reinterpret_cast<const f16x8 *>(ks + (u >> 3) * 8192 + (abase ^ ((u & 7) << 5)));
                }
            };
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < kPipe - 1; ++t) read(t);
#pragma unroll
            for (int t = 0; t < 32; ++t) {
                if (t + kPipe - 1 < 32) read(t + kPipe - 1);
                if (t < 16) {
                    o[t >> 2] = mfma(opnd[t % kPipe], p[t & 3], o[t >> 2]);
                    if constexpr (MODE == kMatrix64q) o2[t >> 2] = mfma(opnd[t % kPipe], p[(t + 1) & 3], o2[t >> 2]);
                } else {
                    const int u = t - 16;
                    s[u >> 3] = mfma(opnd[t % kPipe], q[u & 7], s[u >> 3]);
                    if constexpr (MODE == kMatrix64q) s2[u >> 3] = mfma(opnd[t % kPipe], q[(u + 1) & 7], s2[u >> 3]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i][0] = f16(s[i >> 1][i] + (MODE == kMatrix64q ? s2[i >> 1][i] : 0.f));
        } else if constexpr (MODE == kReadB128) {
            f16x8 r[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) r[u] = *reinterpret_cast<const f16x8 *>(ks + (u >> 3) * 8192 + (abase ^ ((u & 7) << 5)));
#pragma unroll
            for (int u = 0; u < 16; ++u) asm volatile("" : "+v"(r[u]));
#pragma unroll
            for (int u = 0; u < 16; ++u) p[u & 3] += r[u];
        } else if constexpr (MODE == kReadTr) {
            f16x4 r[32];
#pragma unroll
            for (int t = 0; t < 32; ++t)
                r[t] = tr4(vs + 16 * (t & 3) * 256 + ((t & 16 ? trb1 : trb0) ^ (((t >> 2) & 3) << 6)));
#pragma unroll
            for (int t = 0; t < 32; ++t) asm volatile("" : "+v"(r[t]));
#pragma unroll
            for (int t = 0; t < 32; ++t) p[t & 3] += __builtin_shufflevector(r[t], r[t], 0, 1, 2, 3, 0, 1, 2, 3);
        } else if constexpr (MODE == kWriteB128) {
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                f16x8 v = p[t & 3];
                asm volatile("" : "+v"(v));
                *reinterpret_cast<f16x8 *>(const_cast<char *>(vs) + (t >> 3) * 8192 + (abase ^ ((t & 7) << 5))) = v;
            }
            asm volatile("" ::: "memory");
        } else if constexpr (MODE == kExp || MODE == kFma || MODE == kExpFma) {
            // exp2(-x) converges to ~0.64 and x * 0.999 + 0.001 to 1: the values stay finite.
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    if constexpr (MODE != kFma) ex[c] = __builtin_amdgcn_exp2f(-ex[c]);
                    if constexpr (MODE != kExp) fx[c] = __builtin_fmaf(fx[c], 0.999f, 0.001f);
                }
        } else if constexpr (MODE == kMfmaFma || MODE == kMfmaSoft) {
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                o[t & 3] = mfma(q[t & 7], p[t & 3], o[t & 3]);
#pragma unroll
                for (int u = 0; u < (MODE == kMfmaFma ? 4 : 6); ++u)
                    fx[(4 * t + u) & 7] = __builtin_fmaf(fx[(4 * t + u) & 7], 0.999f, 0.001f);
                if constexpr (MODE == kMfmaSoft) {
                    ex[(2 * t) & 7] = __builtin_amdgcn_exp2f(-ex[(2 * t) & 7]);
                    ex[(2 * t + 1) & 7] = __builtin_amdgcn_exp2f(-ex[(2 * t + 1) & 7]);
                }
            }
        } else if constexpr (MODE == kSplitFma || MODE == kSplitExp) {
            if (wave < NT / 128) {
#pragma unroll
                for (int t = 0; t < 32; ++t) o[t & 3] = mfma(q[t & 7], p[t & 3], o[t & 3]);
            } else if constexpr (MODE == kSplitFma) {
#pragma unroll
                for (int t = 0; t < 48; ++t)
#pragma unroll
                    for (int c = 0; c < 8; ++c) fx[c] = __builtin_fmaf(fx[c], 0.999f, 0.001f);
            } else {
#pragma unroll
                for (int t = 0; t < 14; ++t)
#pragma unroll
                    for (int c = 0; c < 8; ++c) ex[c] = __builtin_amdgcn_exp2f(-ex[c]);
            }
        } else if constexpr (MODE == kMfmaExp) {
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                o[t & 3] = mfma(q[t & 7], p[t & 3], o[t & 3]);
                ex[(2 * t) & 7] = __builtin_amdgcn_exp2f(-ex[(2 * t) & 7]);
                ex[(2 * t + 1) & 7] = __builtin_amdgcn_exp2f(-ex[(2 * t + 1) & 7]);
            }
        } else {
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                f16x4 v = __builtin_shufflevector(p[t & 3], p[t & 3], 0, 1, 2, 3);
                asm volatile("" : "+v"(v));
                *reinterpret_cast<f16x4 *>(const_cast<char *>(vs) + 16 * (t & 3) * 256 + (trb0 ^ (((t >> 2) & 1) << 6))) = v;
            }
            asm volatile("" ::: "memory");
        }
    }
    {
        const long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
        if (lane == 0) stamp[blockIdx.x * (NT / 64) + (tid >> 6)] = Stamp{c1 - c0, r0, r1};
    }
    float acc = 0.f;
    for (int i = 0; i < 4; ++i)
        for (int e = 0; e < 16; ++e) acc += o[i][e] + o2[i][e];
    for (int i = 0; i < 2; ++i)
        for (int e = 0; e < 16; ++e) acc += s[i][e] + s2[i][e];
    for (int i = 0; i < 4; ++i)
        for (int e = 0; e < 8; ++e) acc += float(p[i][e]);
    for (int c = 0; c < 8; ++c) acc += ex[c] + fx[c];
    // Read the tiles back so the write probes' stores stay live.
    __syncthreads();
    for (int i = tid; i < kLdsUsed / 2; i += NT) acc += float(reinterpret_cast<const f16 *>(smem)[i]);
    sink[blockIdx.x * NT + tid] = acc;
}

struct Timing {
    double ms;   // first wave's loop start to last wave's loop end
    double ghz;  // shader clock over the loops (all waves)
};

// Loop span of the waves w with lo <= w % per_wg < hi (per_wg waves per workgroup).
Timing span_of(const std::vector<Stamp> &st, int per_wg, int lo, int hi) {
    long long t0 = -1, t1 = -1;
    double cyc = 0, ticks = 0;
    for (size_t i = 0; i < st.size(); ++i) {
        const int w = int(i) % per_wg;
        if (w < lo || w >= hi) continue;
        const Stamp &s = st[i];
        cyc += double(s.cycles);
        ticks += double(s.t1 - s.t0);
        t0 = t0 < 0 || s.t0 < t0 ? s.t0 : t0;
        t1 = t1 < 0 || s.t1 > t1 ? s.t1 : t1;
    }
    Timing t{};
    t.ms = double(t1 - t0) * 1e-5;
    t.ghz = ticks > 0 ? cyc / ticks * 0.1 : 0.0;
    return t;
}

template <typename F>
Timing time_launch(F launch, Stamp *stamp, int nwaves, std::vector<Stamp> *keep = nullptr) {
    launch();
    CHECK(hipDeviceSynchronize());
    launch();
    CHECK(hipDeviceSynchronize());
    std::vector<Stamp> st(nwaves);
    CHECK(hipMemcpy(st.data(), stamp, nwaves * sizeof(Stamp), hipMemcpyDeviceToHost));
    if (keep) *keep = st;
    long long t0 = st[0].t0, t1 = st[0].t1;
    double cyc = 0, ticks = 0;
    for (const Stamp &s : st) {
        cyc += double(s.cycles);
        ticks += double(s.t1 - s.t0);
        t0 = s.t0 < t0 ? s.t0 : t0;
        t1 = s.t1 > t1 ? s.t1 : t1;
    }
    Timing t{};
    t.ms = double(t1 - t0) * 1e-5;
    t.ghz = ticks > 0 ? cyc / ticks * 0.1 : 0.0;
    return t;
}

// One workgroup per CU; NT / 256 waves per SIMD.  MFMA modes: TFLOP/s and the matrix
// cores' busy fraction (MFMA count x 32 cycles over the run's cycles at its clock).
// LDS modes: bytes and instructions per CU per cycle.  VALU modes: SIMD cycles per
// wave64 instruction (the step's cycles over its VALU instructions, all waves of a SIMD).
template <int MODE, int NT>
void run_probe(const char *name, int ncu, int iters, float *sink, Stamp *stamp) {
    std::vector<Stamp> st;
    const Timing t = time_launch(
        [&] { hipLaunchKernelGGL((probe_kernel<MODE, NT>), dim3(ncu), dim3(NT), 0, 0, sink, stamp, iters); }, stamp,
        ncu * NT / 64, &st);
    if (MODE == kSplitFma || MODE == kSplitExp) {
        // Waves 0..3 (one per SIMD) issue MFMAs, waves 4..7 VALU, each about 1024 cycles per step
        // alone; each group's own loop span.  Full overlap keeps both at their lone rates.
        const Timing tm = span_of(st, NT / 64, 0, NT / 128), tv = span_of(st, NT / 64, NT / 128, NT / 64);
        const double mcyc = tm.ms * 1e-3 * tm.ghz * 1e9, vcyc = tv.ms * 1e-3 * tv.ghz * 1e9;
        const double nvalu = (MODE == kSplitFma ? 384.0 : 112.0) * iters;
        std::printf("| %-44s | 1 + 1 | MFMA busy %.2f over its loop | %.2f GHz | %.2f clk per VALU instruction |\n",
                    name, 32.0 * iters * 32.0 / mcyc, tm.ghz, vcyc / nvalu);
        return;
    }
    const double waves_per_cu = NT / 64.0, cycles = t.ms * 1e-3 * t.ghz * 1e9;
    if (MODE <= kMatrix64q) {
        const double mfma_per_wave = (MODE == kMatrix64q ? 64.0 : 32.0) * iters;
        const double tf = mfma_per_wave * waves_per_cu * ncu * 32768.0 / (t.ms * 1e-3) / 1e12;
        const double busy = mfma_per_wave * (waves_per_cu / 4.0) * 32.0 / cycles;
        std::printf("| %-44s | %d | %8.1f TFLOP/s | %.2f GHz | MFMA busy %.2f |\n", name, NT / 256, tf, t.ghz, busy);
    } else if (MODE >= kExp) {
        const double per = MODE == kExpFma || MODE == kMfmaFma ? 64.0 : MODE == kMfmaSoft ? 128.0 : 32.0;
        const double valu = per * iters * (waves_per_cu / 4.0);
        const bool mf = MODE == kMfmaExp || MODE == kMfmaFma || MODE == kMfmaSoft;
        const double busy = mf ? 16.0 * iters * (waves_per_cu / 4.0) * 32.0 / cycles : 0.0;
        std::printf("| %-44s | %d | %8.2f clk per VALU instruction | %.2f GHz | MFMA busy %.2f |\n", name, NT / 256,
                    cycles / valu, t.ghz, busy);
    } else {
        const double instr = (MODE == kReadTr ? 32.0 : 16.0) * iters * waves_per_cu;
        const double bytes_per = MODE == kReadB128 || MODE == kWriteB128 ? 1024.0 : 512.0;
        std::printf("| %-44s | %d | %8.1f B/clk/CU | %.2f GHz | %.2f clk per instruction |\n", name, NT / 256,
                    instr * bytes_per / cycles, t.ghz, cycles / instr);
    }
}

// HBM reads.  Contiguous: workgroup w reads 16-byte chunks w * 1024 + ..., grid-strided.
__global__ __launch_bounds__(256) void read_contig(const u32x4 *p, size_t n16, unsigned *sink) {
    u32x4 acc = {0, 0, 0, 0};
    constexpr int U = 4;
    for (size_t base = size_t(blockIdx.x) * 256 * U; base < n16; base += size_t(gridDim.x) * 256 * U) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t i = base + u * 256 + threadIdx.x;
            v[u] = i < n16 ? p[i] : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u];
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x12345678u) sink[0] = 1;
}

// Pieces: the buffer as [rows][2048 / SEG][SEG bytes]; workgroup w reads column w % (2048 / SEG).
template <int SEG>
__global__ __launch_bounds__(256) void read_pieces(const char *p, size_t rows, unsigned *sink) {
    constexpr int H = 2048 / SEG, LPR = SEG / 16, RPI = 256 / LPR, U = 4;
    const int h = blockIdx.x % H, r_in = threadIdx.x / LPR, c = threadIdx.x % LPR;
    const size_t per_h = gridDim.x / H, wi = blockIdx.x / H;
    u32x4 acc = {0, 0, 0, 0};
    for (size_t r0 = wi * RPI * U; r0 < rows; r0 += per_h * RPI * U) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t r = r0 + u * RPI + r_in;
            v[u] = r < rows ? *reinterpret_cast<const u32x4 *>(p + r * 2048 + h * SEG + c * 16) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u];
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x12345678u) sink[0] = 1;
}

template <typename F>
void run_read(const char *name, size_t bytes, F launch) {
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    launch();
    CHECK(hipDeviceSynchronize());
    float best = 1e30f;
    for (int r = 0; r < 5; ++r) {
        CHECK(hipEventRecord(e0));
        launch();
        CHECK(hipEventRecord(e1));
        CHECK(hipEventSynchronize(e1));
        float ms;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        best = ms < best ? ms : best;
    }
    std::printf("| %-44s | %.4f ms | %.2f TB/s |\n", name, best, double(bytes) / (best * 1e-3) / 1e12);
    CHECK(hipEventDestroy(e0));
    CHECK(hipEventDestroy(e1));
}

}  // namespace

int main(int argc, char **argv) {
    const int iters = argc > 1 ? std::atoi(argv[1]) : 2000;
    if (iters < 1 || iters > 100000) {
        std::printf("iters must be in [1, 100000]\n");
        return 2;
    }
    int dev = 0, ncu = 0;
    CHECK(hipGetDevice(&dev));
    CHECK(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
    float *sink;
    Stamp *stamp;
    CHECK(hipMalloc(&sink, size_t(ncu) * 1024 * sizeof(float)));
    CHECK(hipMalloc(&stamp, size_t(ncu) * 16 * sizeof(Stamp)));
    std::printf("%d CUs, one workgroup per CU, %d steps per wave\n\n", ncu, iters);
    std::printf("| probe | waves/SIMD | rate | clock | |\n|---|---|---|---|---|\n");
    run_probe<kMfmaRegs, 256>("MFMA, register operands", ncu, iters, sink, stamp);
    run_probe<kMfmaRegs, 512>("MFMA, register operands", ncu, iters, sink, stamp);
    run_probe<kMatrixTr, 256>("matrix phase, V^T by transposed reads", ncu, iters, sink, stamp);
    run_probe<kMatrixTr, 512>("matrix phase, V^T by transposed reads", ncu, iters, sink, stamp);
    run_probe<kMatrixVt, 256>("matrix phase, V^T tile read by ds_read_b128", ncu, iters, sink, stamp);
    run_probe<kMatrixVt, 512>("matrix phase, V^T tile read by ds_read_b128", ncu, iters, sink, stamp);
    run_probe<kMatrix64q, 256>("matrix phase, 64 queries per wave", ncu, iters, sink, stamp);
    run_probe<kReadB128, 1024>("ds_read_b128, 16 in flight", ncu, iters, sink, stamp);
    run_probe<kReadTr, 1024>("ds_read_b64_tr_b16, 32 in flight", ncu, iters, sink, stamp);
    run_probe<kWriteB128, 1024>("ds_write_b128", ncu, iters, sink, stamp);
    run_probe<kWriteB64, 1024>("ds_write_b64", ncu, iters, sink, stamp);
    run_probe<kExp, 512>("v_exp_f32", ncu, iters, sink, stamp);
    run_probe<kExp, 1024>("v_exp_f32", ncu, iters, sink, stamp);
    run_probe<kFma, 512>("v_fma_f32", ncu, iters, sink, stamp);
    run_probe<kFma, 1024>("v_fma_f32", ncu, iters, sink, stamp);
    run_probe<kExpFma, 512>("v_exp_f32 + v_fma_f32 interleaved", ncu, iters, sink, stamp);
    run_probe<kExpFma, 1024>("v_exp_f32 + v_fma_f32 interleaved", ncu, iters, sink, stamp);
    run_probe<kMfmaExp, 256>("16 MFMAs + 32 v_exp_f32, one wave", ncu, iters, sink, stamp);
    run_probe<kMfmaExp, 512>("16 MFMAs + 32 v_exp_f32, one wave", ncu, iters, sink, stamp);
    run_probe<kMfmaFma, 256>("16 MFMAs + 64 v_fma_f32, one wave", ncu, iters, sink, stamp);
    run_probe<kMfmaSoft, 256>("16 MFMAs + 32 exp + 96 fma, one wave", ncu, iters, sink, stamp);
    run_probe<kMfmaSoft, 512>("16 MFMAs + 32 exp + 96 fma, one wave", ncu, iters, sink, stamp);
    run_probe<kSplitFma, 512>("MFMA wave beside a v_fma_f32 wave", ncu, iters, sink, stamp);
    run_probe<kSplitExp, 512>("MFMA wave beside a v_exp_f32 wave", ncu, iters, sink, stamp);

    const size_t bytes = size_t(1536) << 20;
    char *buf;
    unsigned *rsink;
    CHECK(hipMalloc(&buf, bytes));
    CHECK(hipMalloc(&rsink, sizeof(unsigned)));
    CHECK(hipMemset(buf, 1, bytes));
    const unsigned grid = unsigned((8 * ncu + 15) / 16 * 16);  // a multiple of every piece count per row
    std::printf("\n| HBM read, 1.5 GiB, %u workgroups | best of 5 | rate |\n|---|---|---|\n", grid);
    run_read("contiguous", bytes, [&] {
        hipLaunchKernelGGL(read_contig, dim3(grid), dim3(256), 0, 0, (const u32x4 *)buf, bytes / 16, rsink);
    });
    run_read("512-byte pieces at a 2 KB stride", bytes, [&] {
        hipLaunchKernelGGL((read_pieces<512>), dim3(grid), dim3(256), 0, 0, buf, bytes / 2048, rsink);
    });
    run_read("256-byte pieces at a 2 KB stride", bytes, [&] {
        hipLaunchKernelGGL((read_pieces<256>), dim3(grid), dim3(256), 0, 0, buf, bytes / 2048, rsink);
    });
    run_read("128-byte pieces at a 2 KB stride", bytes, [&] {
        hipLaunchKernelGGL((read_pieces<128>), dim3(grid), dim3(256), 0, 0, buf, bytes / 2048, rsink);
    });
    CHECK(hipFree(buf));
    CHECK(hipFree(rsink));
    CHECK(hipFree(sink));
    CHECK(hipFree(stamp));
    return 0;
}
