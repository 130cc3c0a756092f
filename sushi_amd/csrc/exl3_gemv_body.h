// (Kernel body shared by the per-family translation units exl3_gemv_<family>.hip.)
// Trellis GEMV for 1..16 rows: the decode arm of the dense linear (linear.linear, beamivalice/sushi
// src/exl3/linear.zig:317-336, Metal ROWS_SOURCE/ROWS_FINISH_SOURCE in src/exl3/project_rows.zig:145-249, :345-362)
// and of the routed MoE chain (PAIR_GEMV_SOURCE :2082-2241, DOWN_FUSED_SOURCE :1820-2023 in
// src/exl3/expert_exl3_kernels.zig).
//
// MI355X layout.  A workgroup (GEMV_WAVES = 8 waves, one workgroup per CU at C1) owns one output group of 8 tiles
// (128 outputs, one Hadamard block) of one (bank, x-block) pair over one k split of at most 32 k-tiles (whole
// 128-blocks).  Per k-tile row a wave streams the group's 8 tiles, which lie contiguous in the pack order
// [IT][OT][n] (8*n*2 bytes, 1 KiB at K4): lane = 8*o + j reads chunk j of tile o, the words carrying codewords
// 32j..32j+31 = output columns j and j+8 over all 16 k rows (tensorCorePerm).  Every lane owns two output columns
// outright and decodes its 32 weights into registers as packed f16 pairs (t, t+1) = rows (r, r+1) of one column.
// Those pairs are, as they stand, B columns of v_mfma_f32_4x4x4_16b_f16, whose A rows are batch rows of the
// prepared input in LDS: the matrix cores take the dot products, four batch rows per instruction set, and the VALU
// keeps the decode.  No cross-lane reduction happens inside a wave; the waves meet once in LDS.
//
// Latency: a wave issues the loads of all its tiles (<= 4) before the prologue, so HBM latency overlaps the input
// preparation (x * suh, FWHT-128, f16 -- or the MoE SwiGLU mid).  The finish (FWHT-128, * svh) runs in the same
// launch: with one split directly; otherwise each split folds its transformed partial into exact fixed-point
// accumulators with one returning atomic per output and the split that completes an output stores it (fold_finish),
// or, past the fold's limits, the last workgroup of an output group to arrive sums the partial planes.
#pragma once
#include "exl3_kernels.h"
#include "exl3_tables.h"
#include "exl3_lane_decode.h"

namespace exl3 {

constexpr int GEMV_THREADS = 64 * GEMV_WAVES;
constexpr int MAX_KSPAN = 2048;
// LDS pitch (halves) of a prepared input row: 16 bytes past MAX_KSPAN, so the rows that the four lane groups of a
// matrix instruction read at one k fall in different LDS banks.
constexpr int XS_PITCH = MAX_KSPAN + 8;

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

// v_mfma_f32_4x4x4_16b_f16: sixteen independent 4x4x4 products, block b on lanes 4b..4b+3.  Lane 4b+i holds row i of
// the block's A (4 k values) and column i of its B (the same 4 k), and receives column i of the block's D (rows 0..3).
__device__ __forceinline__ f4_t mfma4(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, f4_t c) {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(h4_t, u2_t{a0, a1}),
                                              __builtin_bit_cast(h4_t, u2_t{b0, b1}), c, 0, 0, 0);
}

// Batch rows are served four at a time (one set of matrix instructions per group of four).
template <int RT>
struct RowGroups {
    static constexpr int G = (RT + 3) / 4;
};

__device__ __forceinline__ float load_x(const void *x, int dt, size_t i) {
    if (dt == DT_F16) return load_act<DT_F16>(x, i);
    if (dt == DT_BF16) return load_act<DT_BF16>(x, i);
    return load_act<DT_F32>(x, i);
}

__device__ __forceinline__ void store_y(void *y, int dt, size_t i, float v) {
    if (dt == DT_F16) store_act<DT_F16>(y, i, v);
    else if (dt == DT_BF16) store_act<DT_BF16>(y, i, v);
    else store_act<DT_F32>(y, i, v);
}

__device__ __forceinline__ float load_y(const void *y, int dt, size_t i) {
    if (dt == DT_F16) return load_act<DT_F16>(y, i);
    if (dt == DT_BF16) return load_act<DT_BF16>(y, i);
    return load_act<DT_F32>(y, i);
}

// v rounded to y's dtype and back (the routed sum's rounding before a shared expert is added).
__device__ __forceinline__ float round_y(int dt, float v) {
    if (dt == DT_F16) return __half2float(__float2half_rn(v));
    if (dt == DT_BF16) return __bfloat162float(__float2bfloat16(v));
    return v;
}

// v rounded to y's 16-bit dtype (f16 or bf16), as its bit pattern, and back.
__device__ __forceinline__ uint32_t y_bits16(int dt, float v) {
    if (dt == DT_F16) return __half_as_ushort(__float2half_rn(v));
    return __bfloat16_as_ushort(__float2bfloat16(v));
}
__device__ __forceinline__ float y_from_bits16(int dt, uint32_t b) {
    if (dt == DT_F16) return __half2float(__ushort_as_half((unsigned short)b));
    return __uint_as_float(b << 16);
}

struct GemvCtx {
    int g, proj, bank, og, sp, S, KS, kt0, IT, OT, G, x_dtype;
    int gy;                     // the group's index in the grid (shared groups first): the fused chain's counters
    uint32_t x_div_m;           // slots per x row, as a div_magic constant
    int rows;                   // rows of this group (a window's own count in the sorted MoE arm)
    int xg;                     // x row of the group's row 0 (per-slot and dense arms, a shared expert's rows)
    int slot0;                  // MoE slot of the group's row 0 (a shared expert's rows: virtual slots past the routed)
    const uint32_t *wslots;     // the window's slots, or null (group = slot, or plain rows)
    const void *x;
    const uint16_t *suh, *svh;  // this projection's banks (selected once: an indexed kernel-argument read would be
    float *part;                // a dependent scalar load)
    float sv0, sv1;             // svh of this lane's two outputs, fetched at entry for the finish
};

// Output FWHT + svh for one row of a 128-output block held as (v0 = col lane, v1 = col lane + 64).
__device__ __forceinline__ void finish_block(const GemvArgs &a, const GemvCtx &c, int rho, float v0, float v1,
                                             int lane) {
    fwht128_wave(v0, v1, lane);
    const size_t yrow = a.y_rows_major ? (size_t)rho * a.groups + c.g : (size_t)c.g * a.rows + rho;
    const size_t yo = yrow * a.out + (size_t)c.og * 128;
    store_y(a.y, a.y_dtype, yo + lane, v0 * HAD_SCALE * c.sv0);
    store_y(a.y, a.y_dtype, yo + lane + 64, v1 * HAD_SCALE * c.sv1);
}

// Row r of this group: its input row, its partial plane (elements into [.][S][.][out]) and, for the MoE mid, its slot.
// WIN: the group is an expert window (the sorted MoE arm), a compile-time choice so the dense kernels carry none of it.
template <bool WIN>
__device__ __forceinline__ size_t x_row(const GemvArgs &a, const GemvCtx &c, int r) {
    if constexpr (WIN) return (size_t)div_by_magic(c.wslots[r], c.x_div_m);
    else return (size_t)c.xg + r;
}
// SH: a shared expert's rows keep one plane per row (slot slot0 + r), as the per-slot rows do.
template <bool WIN, bool SH>
__device__ __forceinline__ size_t part_row(const GemvArgs &a, const GemvCtx &c, int r) {
    if constexpr (WIN) return ((size_t)c.wslots[r] * c.S + c.sp) * a.out;
    else if constexpr (SH) return ((size_t)(c.slot0 + r) * c.S + c.sp) * a.out;
    else return (((size_t)c.g * c.S + c.sp) * a.rows + r) * a.out;
}
template <bool WIN>
__device__ __forceinline__ int slot_of(const GemvCtx &c, int r) {
    if constexpr (WIN) return (int)c.wslots[r];
    else return c.slot0 + r;  // per-slot groups hold one row
}

// A lane's prepared input for one k-tile (its A rows at k 0..15 of the tile): read before the tile's decode, so the
// LDS latency hides behind it.
struct XFrag {
    uint4 X, Y;
};
__device__ __forceinline__ XFrag read_xfrag(const uint16_t (*xs)[XS_PITCH], int row, int kk) {
    const uint16_t *xg = &xs[row][kk * 16];
    return XFrag{*reinterpret_cast<const uint4 *>(xg), *reinterpret_cast<const uint4 *>(xg + 8)};
}
// The lane's 16 decoded pairs (w, as decoded: hash / pair values over 4096) against every batch row of k-tile kk; f0 is
// row group 0's fragment, the others are read here.
template <int RT>
__device__ __forceinline__ void mfma_dot(const uint32_t (&w)[16], const uint16_t (*xs)[XS_PITCH], int kk, int rows,
                                         f4_t (&accA)[RowGroups<RT>::G], f4_t (&accB)[RowGroups<RT>::G], int i4,
                                         const XFrag &f0) {
#pragma unroll
    for (int g = 0; g < RowGroups<RT>::G; g++) {
        if (g > 0 && 4 * g >= rows) break;
        const XFrag f = g == 0 ? f0 : read_xfrag(xs, min(4 * g + i4, RT - 1), kk);
        const uint4 X = f.X, Y = f.Y;
        accA[g] = mfma4(X.x, X.y, w[0], w[4], accA[g]);
        accB[g] = mfma4(X.x, X.y, w[2], w[6], accB[g]);
        accA[g] = mfma4(X.z, X.w, w[8], w[12], accA[g]);
        accB[g] = mfma4(X.z, X.w, w[10], w[14], accB[g]);
        accA[g] = mfma4(Y.x, Y.y, w[1], w[5], accA[g]);
        accB[g] = mfma4(Y.x, Y.y, w[3], w[7], accB[g]);
        accA[g] = mfma4(Y.z, Y.w, w[9], w[13], accA[g]);
        accB[g] = mfma4(Y.z, Y.w, w[11], w[15], accB[g]);
    }
}

// The 32 weights of one tile chunk (lane-owned columns j and j+8) against every batch row, on the matrix cores.
// Lane 8o + j is lane 4b + i of block b = 2o + j/4 with i = j % 4: its decoded pairs of column j over k rows 4s..4s+3
// (pairs (0, 4), (8, 12), (1, 5), (9, 13) for s = 0..3; column j + 8: (2, 6), (10, 14), (3, 7), (11, 15)) are the B
// column i of that block as they stand, and its A row is batch row 4g + i of the prepared input at the same k, so
// accA[g] / accB[g] collect rows 4g..4g+3 of columns j / j + 8.  Rows past RT read row RT - 1 (their results are
// never used); rows at or past `rows` (wave-uniform) hold zeros in LDS, and whole groups past it are skipped.
template <int FAM, int N, int RT, bool MASKED>
__device__ __forceinline__ void decode_tile(const uint32_t (&A)[LaneBits<N>::AW], const uint16_t (*xs)[XS_PITCH],
                                            int kk, int rows, const DecodeK &k, f4_t (&accA)[RowGroups<RT>::G],
                                            f4_t (&accB)[RowGroups<RT>::G], int i4) {
    const XFrag f0 = read_xfrag(xs, min(i4, RT - 1), kk);
    uint32_t w[16];
    decode_weights<FAM, N, MASKED>(A, k, w);
    mfma_dot<RT>(w, xs, kk, rows, accA, accB, i4, f0);
}

// The same for a lane of a per-tile-rate bank, at its own tile's rate (k: the lane's constants).
template <int FAM, int RT, bool MASKED>
__device__ __forceinline__ void decode_tile_tiled(const uint32_t (&A)[3], bool k1, const uint16_t (*xs)[XS_PITCH],
                                                  int kk, int rows, const DecodeK &k, f4_t (&accA)[RowGroups<RT>::G],
                                                  f4_t (&accB)[RowGroups<RT>::G], int i4) {
    const XFrag f0 = read_xfrag(xs, min(i4, RT - 1), kk);
    uint32_t w[16];
    decode_weights_tiled<FAM, MASKED>(A, k1, k, w);
    mfma_dot<RT>(w, xs, kk, rows, accA, accB, i4, f0);
}

// x[i] as f32 from an f16 / bf16 / f32 array without branching on the dtype: one 32-bit load of the aligned word
// that holds the element, then bit-mask selects.  (A branch per dtype joins through a register copy, and that copy
// makes the load wait for its data right there.)  The array starts 4-byte aligned (the C ABI checks it) and rows
// are multiples of 128 elements, so the word never leaves the array.  The load is addressed as global memory: a flat
// load would also count against lgkmcnt and be waited for with the scalar loads.
__device__ __forceinline__ float load_x_nb(const void *x, int dt, size_t i) {
    const bool wide = dt == DT_F32;
    const size_t byte = wide ? i * 4 : i * 2;
    typedef __attribute__((address_space(1))) const uint32_t global_u32;
    const uint32_t w = *(global_u32 *)(static_cast<const char *>(x) + (byte & ~(size_t)3));
    const uint32_t h = __builtin_amdgcn_alignbit(w, w, (uint32_t)(byte & 2) * 8u) & 0xFFFFu;
    const uint32_t f16b = __float_as_uint(h2f((uint16_t)h)), bf16b = h << 16;
    const uint32_t m_wide = 0u - (uint32_t)wide, m_f16 = 0u - (uint32_t)(dt == DT_F16);
    return __uint_as_float((w & m_wide) | (~m_wide & ((f16b & m_f16) | (bf16b & ~m_f16))));
}

// The prologue's input loads for a wave's first jobs, issued ahead of the tile loads (loads retire in order, so an
// input load issued behind 16 KiB of tile loads would hold the prologue back until all of them had landed).  Loads
// are unconditional (a job past the end re-reads job 0 and is then discarded): no branch, so no early wait.
template <int RT, bool WIN>
struct PrologueRegs {
    // jobs per wave when a split spans at most TPW * GEMV_WAVES k-tiles (TPW * GEMV_WAVES / 8 blocks per row), at
    // most 4 held in registers (past that the prologue loads as it goes: 16 rows would otherwise spill); the sorted
    // MoE arm's splits span up to two such batches, so its windows hold 4
    static constexpr int JOBS = WIN ? 4 : (RT * TPW / 8) < 1 ? 1 : (RT * TPW / 8) > 4 ? 4 : (RT * TPW / 8);
    float x0[JOBS], x1[JOBS], s0[JOBS], s1[JOBS];
};

template <int PRO, int RT, bool WIN>
__device__ __forceinline__ void prologue_fetch(const GemvArgs &a, const GemvCtx &c, int wave, int lane,
                                               PrologueRegs<RT, WIN> &pr) {
    if constexpr (PRO == PRO_X) {
        const int nblk = c.KS >> 3;
#pragma unroll
        for (int i = 0; i < PrologueRegs<RT, WIN>::JOBS; i++) {
            int job = wave + GEMV_WAVES * i;
            int rho = 0, b = job;  // one row: no division
            if constexpr (RT > 1) {
                rho = job / nblk;
                b = job - rho * nblk;
            }
            if (!(job < nblk * RT && rho < c.rows)) rho = b = 0;
            const int kb = c.kt0 * 16 + b * 128;
            const size_t in = (size_t)c.IT << 4;
            const size_t si = (size_t)c.bank * in + kb;
            const size_t xi = x_row<WIN>(a, c, rho) * in + kb;
            pr.x0[i] = load_x_nb(c.x, c.x_dtype, xi + lane);
            pr.x1[i] = load_x_nb(c.x, c.x_dtype, xi + lane + 64);
            pr.s0[i] = h2f(c.suh[si + lane]);
            pr.s1[i] = h2f(c.suh[si + lane + 64]);
        }
    }
}

// Sums the gate and up planes of one 128-block over the previous launch's k splits, issuing a chunk of loads before
// any add (a loop that adds as it loads would wait out one memory round trip per split).
// BYPASS (the fused chain): the planes were written through to memory by workgroups that may sit on other XCDs in
// the same launch, so they are read with system-scope loads, past this XCD's L2 (which may hold an earlier call's).
constexpr int MID_CHUNK = 8;
template <bool BYPASS = false>
__device__ __forceinline__ void mid_planes(const GemvArgs &a, int slot, int kb, int lane, float (&w)[2][2]) {
    w[0][0] = w[0][1] = w[1][0] = w[1][1] = 0.f;
    for (int s0 = 0; s0 < a.mid_splits; s0 += MID_CHUNK) {
        float t[2][2][MID_CHUNK];
#pragma unroll
        for (int pj = 0; pj < 2; pj++) {
#pragma unroll
            for (int q = 0; q < MID_CHUNK; q++) {
                const int s2 = min(s0 + q, a.mid_splits - 1);
                const float *pp = a.mid_part[pj] + ((size_t)slot * a.mid_splits + s2) * a.in + kb;
                if constexpr (BYPASS) {
                    t[pj][0][q] = __hip_atomic_load(pp + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    t[pj][1][q] = __hip_atomic_load(pp + lane + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                } else {
                    t[pj][0][q] = pp[lane];
                    t[pj][1][q] = pp[lane + 64];
                }
            }
        }
#pragma unroll
        for (int pj = 0; pj < 2; pj++) {
#pragma unroll
            for (int q = 0; q < MID_CHUNK; q++) {
                const bool in = s0 + q < a.mid_splits;
                w[pj][0] += in ? t[pj][0][q] : 0.f;
                w[pj][1] += in ? t[pj][1][q] : 0.f;
            }
        }
    }
}

template <int PRO, int RT, bool WIN, bool SH, int CH = 0>
__device__ __forceinline__ void prologue(const GemvArgs &a, const GemvCtx &c, uint16_t (*xs)[XS_PITCH], int wave,
                                         int lane, const PrologueRegs<RT, WIN> &pr) {
    const int nblk = c.KS >> 3;
    for (int job = wave; job < nblk * RT; job += GEMV_WAVES) {
        const int rho = RT > 1 ? job / nblk : 0, b = job - rho * nblk;
        const int kb = c.kt0 * 16 + b * 128;
        const int i = (job - wave) / GEMV_WAVES;
        float v0 = 0.f, v1 = 0.f;
        if (rho < c.rows) {
            const size_t si = (size_t)c.bank * a.in + kb;
            if constexpr (PRO == PRO_X) {  // prepareInput (expert_exl3.zig:490-501)
                if (i < PrologueRegs<RT, WIN>::JOBS) {
                    v0 = f16r(pr.x0[i]) * pr.s0[i];
                    v1 = f16r(pr.x1[i]) * pr.s1[i];
                } else {
                    const size_t xi = x_row<WIN>(a, c, rho) * a.in + kb;
                    v0 = f16r(load_x_nb(c.x, a.x_dtype, xi + lane)) * h2f(c.suh[si + lane]);
                    v1 = f16r(load_x_nb(c.x, a.x_dtype, xi + lane + 64)) * h2f(c.suh[si + lane + 64]);
                }
            } else {  // the SwiGLU mid of the decode chain (DOWN_FUSED_SOURCE prologue, :1838-1920)
                // The gate / up svh and suh_down depend on the expert only: their loads go out with the planes',
                // so the job waits out one memory round trip, not three.
                float msv_v[2][2];
#pragma unroll
                for (int pj = 0; pj < 2; pj++) {
                    const uint16_t *msv = SH ? a.sh_mid_svh[pj] : a.mid_svh[pj];
                    msv_v[pj][0] = h2f(msv[si + lane]);
                    msv_v[pj][1] = h2f(msv[si + lane + 64]);
                }
                const float su0 = h2f(c.suh[si + lane]), su1 = h2f(c.suh[si + lane + 64]);
                float w[2][2];
                mid_planes<CH == 2>(a, slot_of<WIN>(c, rho), kb, lane, w);
                float gv[2], uv[2];
#pragma unroll
                for (int pj = 0; pj < 2; pj++) {
                    float w0 = w[pj][0], w1 = w[pj][1];
                    fwht128_wave(w0, w1, lane);
                    w0 *= HAD_SCALE * msv_v[pj][0];
                    w1 *= HAD_SCALE * msv_v[pj][1];
                    if (pj == 0) {
                        gv[0] = w0;
                        gv[1] = w1;
                    } else {
                        uv[0] = w0;
                        uv[1] = w1;
                    }
                }
                if (a.clamp_limit > 0.f) {
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        gv[i] = fminf(gv[i], a.clamp_limit);
                        uv[i] = fminf(fmaxf(uv[i], -a.clamp_limit), a.clamp_limit);
                    }
                }
                v0 = silu(gv[0]) * uv[0] * su0;
                v1 = silu(gv[1]) * uv[1] * su1;
            }
            fwht128_wave(v0, v1, lane);
            v0 *= HAD_SCALE;
            v1 *= HAD_SCALE;
        }
        xs[rho][b * 128 + lane] = __half_as_ushort(__float2half_rn(v0));
        xs[rho][b * 128 + lane + 64] = __half_as_ushort(__float2half_rn(v1));
    }
}

// One output's fixed-point term: the arrival count plus either the biased 24-bit-fraction value or, for a value that
// is not finite or not below 2^21 in magnitude, a mark in the out-of-range field (the value itself then goes to the
// overflow word, fold_overflow).  v * 2^24 is exact in f32 and below 2^45, and rintf rounds it to the nearest integer.
__device__ __forceinline__ bool fold_in_range(float v) { return fabsf(v) < 2097152.0f; }  // NaN fails the compare too

__device__ __forceinline__ unsigned long long fold_term(float v) {
    const unsigned long long one = 1ull << FOLD_COUNT_SHIFT;
    if (!fold_in_range(v)) return one | (1ull << FOLD_BAD_SHIFT);
    const long long q = (long long)rintf(v * 16777216.0f);
    return one + (unsigned long long)(q + FOLD_BIAS);
}

// The contributions of this lane's two outputs that fall outside the fixed-point range go, in f64, to their overflow
// words before the arrivals are counted: a release fence (only in a wave that had one) orders them ahead of the fold
// adds, so the arrival that completes an output sees them.  f64 keeps inf and NaN as they are (inf + -inf is NaN).
__device__ __forceinline__ void fold_overflow(unsigned long long *w0, unsigned long long *w1, float v0, float v1) {
    const bool o0 = !fold_in_range(v0), o1 = !fold_in_range(v1);
    if (o0) __hip_atomic_fetch_add(reinterpret_cast<double *>(w0 + FOLD_WORDS), (double)v0, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    if (o1) __hip_atomic_fetch_add(reinterpret_cast<double *>(w1 + FOLD_WORDS), (double)v1, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    if (__ballot(o0 || o1)) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
}

// The output value of word `w` once its last word value `t` holds all S arrivals: the exact sum of the in-range
// terms, plus, when any contribution was out of range, the overflow word's f64 sum (read and cleared here, after an
// acquire fence that pairs with the contributors' release).
__device__ __forceinline__ float fold_value(unsigned long long t, int S, unsigned long long *w) {
    const int bad = (int)((t >> FOLD_BAD_SHIFT) & 63u);
    const long long sum = (long long)(t & ((1ull << FOLD_BAD_SHIFT) - 1)) - (long long)(S - bad) * FOLD_BIAS;
    double v = (double)sum * (1.0 / 16777216.0);
    if (bad) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        v += __hip_atomic_exchange(reinterpret_cast<double *>(w + FOLD_WORDS), 0.0, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    return (float)v;
}

// Fused split-k finish by exact accumulation.  The output transform (FWHT-128, then * svh) is linear, so each split
// applies it to its own partial and the sum of the transformed partials is the transformed sum.  Each split adds
// its 24-bit-fraction fixed-point terms, together with an arrival count, into one 64-bit word per output with a
// single atomic that returns the previous word; the split whose add completes the count holds the whole sum, stores
// y and clears the word for the next call.  Integer addition makes the result independent of arrival order, and
// neither partial planes nor a second round trip (store acknowledgement, then counter) sit on the path.  Wave w
// finishes rows w, w + GEMV_WAVES, ...
// The MoE down projection folds the same way across slots: slot s adds its score-weighted output into row
// s / topk (the score-weighted reduce of REDUCE_SOURCE / REDUCE_SHARED_SOURCE, expert_exl3_kernels.zig:2338-2406),
// and the completing arrival rounds the routed sum to y's dtype before adding the shared expert.  MOE (the down
// projection's PRO_MID kernels) is a compile-time choice: the dense kernels carry none of the slot, score and
// shared-expert handling.
template <int RT, bool WIN, bool MOE, bool SH>
__device__ __forceinline__ void fold_finish(const GemvArgs &a, const GemvCtx &c, float (*red)[RT][128], int wave,
                                            int lane) {
    for (int r = wave; r < c.rows; r += GEMV_WAVES) {
        float v0 = 0.f, v1 = 0.f;
#pragma unroll
        for (int w = 0; w < GEMV_WAVES; w++) {
            v0 += red[w][r][lane];
            v1 += red[w][r][lane + 64];
        }
        v0 *= a.out_scale;
        v1 *= a.out_scale;
        fwht128_wave(v0, v1, lane);
        size_t yrow;
        float sc = 1.0f;
        bool shared = false;
        if constexpr (MOE) {
            const int slot = slot_of<WIN>(c, r);
            shared = SH;
            if (shared) {  // the shared expert's own row, score 1, into its own words
                yrow = (size_t)(slot - a.sh_from);
            } else {
                yrow = (size_t)(slot / a.fold_topk);
                sc = load_any(a.fold_scores, a.score_dtype, slot);
            }
        } else {
            yrow = a.y_rows_major ? (size_t)r * a.groups + c.g : (size_t)c.g * a.rows + r;
        }
        const int arrivals = shared ? c.S : a.fold_arrivals;
        const float f0 = (v0 * HAD_SCALE * c.sv0) * sc, f1 = (v1 * HAD_SCALE * c.sv1) * sc;
        const unsigned long long t0 = fold_term(f0), t1 = fold_term(f1);
        const size_t yo = yrow * a.out + (size_t)c.og * 128;
        unsigned long long *w0 = (shared ? a.sh_fold : a.fold) + yo + lane, *w1 = w0 + 64;
        fold_overflow(w0, w1, f0, f1);
        const unsigned long long o0 = __hip_atomic_fetch_add(w0, t0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned long long o1 = __hip_atomic_fetch_add(w1, t1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // Both adds go out before either result is examined: one memory round trip for the pair, not two.
        __builtin_amdgcn_sched_barrier(0);
        const unsigned long long last = (unsigned long long)(arrivals - 1);
        if constexpr (!MOE) {
            // Both outcomes are settled before either store, so no store waits on the other output's check.
            const bool d0 = (o0 >> FOLD_COUNT_SHIFT) == last, d1 = (o1 >> FOLD_COUNT_SHIFT) == last;
            const float y0 = d0 ? fold_value(o0 + t0, arrivals, w0) : 0.f;
            const float y1 = d1 ? fold_value(o1 + t1, arrivals, w1) : 0.f;
            if (d0) {
                store_y(a.y, a.y_dtype, yo + lane, y0);
                *w0 = 0ull;  // no split of this launch touches it again; the next launch reads it after the boundary
            }
            if (d1) {
                store_y(a.y, a.y_dtype, yo + lane + 64, y1);
                *w1 = 0ull;
            }
            continue;
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const unsigned long long o = h ? o1 : o0, t = h ? t1 : t0;
            if ((o >> FOLD_COUNT_SHIFT) != last) continue;
            const size_t i = yo + lane + 64 * h;
            float v = fold_value(o + t, arrivals, h ? w1 : w0);
            if (a.fold_comb) {
                // The routed sum and the shared expert's, each rounded to y's 16-bit dtype, meet in one word: each
                // adds its bit pattern into its own half-word with a flag; whichever arrives second holds both and
                // stores T(T(routed) + T(shared)), the rounding moeWithShared keeps (REDUCE_SHARED_SOURCE,
                // expert_exl3_kernels.zig:2391-2406).
                const uint32_t b = y_bits16(a.y_dtype, v);
                const unsigned long long term = shared ? (1ull << 62) | b : (1ull << 63) | ((unsigned long long)b << 16);
                unsigned long long *cw = a.fold_comb + i;
                const unsigned long long old = __hip_atomic_fetch_add(cw, term, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (old != 0) {
                    const uint32_t rb = shared ? (uint32_t)(old >> 16) & 0xFFFFu : b;
                    const uint32_t hb = shared ? b : (uint32_t)old & 0xFFFFu;
                    store_y(a.y, a.y_dtype, i, y_from_bits16(a.y_dtype, rb) + y_from_bits16(a.y_dtype, hb));
                    *cw = 0ull;
                }
            } else {
                if (a.fold_shared) {
                    const float sh = load_y(a.fold_shared, a.y_dtype, i);
                    v = round_y(a.y_dtype, v) +
                        (a.fold_gate ? gated_shared(a.y_dtype, load_y(a.fold_gate, a.y_dtype, yrow), sh) : sh);
                }
                store_y(a.y, a.y_dtype, i, v);
            }
            // No split of this launch touches the word again, and the next launch reads it after the kernel boundary:
            // a plain store suffices (a device-scope store would be written through and hold up the kernel's end).
            *(h ? w1 : w0) = 0ull;
        }
    }
}

// svh of this lane's two outputs, for the finish.
// PIN (dense launches): the offset passes through an empty asm, so the address arithmetic (and with it the wait for
// the argument load that supplies the bank pointer) cannot be hoisted above the caller's tile loads.
template <bool PIN = false>
__device__ __forceinline__ void fetch_svh(GemvCtx &c, int lane) {
    uint32_t sv = (uint32_t)c.bank * ((uint32_t)c.OT << 4) + (uint32_t)c.og * 128u;
    if constexpr (PIN) asm volatile("" : "+s"(sv));
    c.sv0 = h2f(c.svh[(size_t)sv + lane]);
    c.sv1 = h2f(c.svh[(size_t)sv + lane + 64]);
}

// A per-tile-rate projection as a workgroup reads it (N == N_TILED): its segment tables and the constants at both
// rates.
struct TiledSrc {
    const uint32_t *seg_off;
    const uint8_t *seg_k1;
    DecodeK ka, kb;
};

// Everything a workgroup does once its rate is known: loads, prologue, decode + dot, reduction, finish.
// N == N_TILED: each tile at its own rate (ts), tb the projection's whole trellis.
// PIN: a uniform-rate launch's body (see fetch_svh).
// The fused chain's down workgroup: wave 0 waits until its group's gate/up workgroups have all arrived (their planes
// written through to memory first), at most CHAIN_SPIN_TICKS, so the wait always ends; a workgroup barrier then
// releases the other waves (one poller per workgroup keeps the polls off the counters' memory channel).
__device__ __forceinline__ void chain_wait(const GemvArgs &a, const GemvCtx &c, int wave) {
    if (wave == 0) {
        const uint32_t *ctr = a.chain_ctr + (size_t)(2 * c.gy) * COUNTER_STRIDE;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (uint32_t)a.chain_need) {
            __builtin_amdgcn_s_sleep(8);
            if (__builtin_amdgcn_s_memrealtime() - t0 > CHAIN_SPIN_TICKS) break;
        }
    }
    __syncthreads();
}

// CH: the fused chain's role (0 none; 1 gate/up: planes written through, then the group's arrival counted; 2 down:
// tile loads, then the wait, then the mid from the planes past the L2).
template <int FAM, int N, int RT, int PRO, bool WIN, bool SH, bool PIN = false, int CH = 0>
__device__ __forceinline__ void gemv_body(const GemvArgs &a, GemvCtx &c, const uint16_t *__restrict__ tb,
                                          int n, const DecodeK &k, uint16_t (*xs)[XS_PITCH], float (*red)[RT][128],
                                          const TiledSrc &ts = TiledSrc{}) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it stay scalar
    const int o = lane >> 3, j = lane & 7;
    constexpr int RG = RowGroups<RT>::G;
    f4_t accA[RG], accB[RG];
#pragma unroll
    for (int g = 0; g < RG; g++) accA[g] = accB[g] = f4_t{0.f, 0.f, 0.f, 0.f};

    if constexpr (N != 0) {
        constexpr bool TILED = N == N_TILED;
        constexpr int AW = TILED ? 3 : LaneBits<(TILED ? TILED_NB : N)>::AW;
        // This wave's k-tiles are wave, wave + GEMV_WAVES, ...; a split spans whole 128-blocks (8 k-tiles), so every
        // wave has at least one.  The first TPW loads are issued unconditionally (a wave with fewer tiles re-reads its
        // last one), so the compiler counts them and each tile's decode waits only for that tile's own loads.
        const int ntiles = (c.KS - wave + GEMV_WAVES - 1) / GEMV_WAVES;
        PrologueRegs<RT, WIN> pr;
        prologue_fetch<PRO, RT, WIN>(a, c, wave, lane, pr);
        __builtin_amdgcn_sched_barrier(0);  // the input loads stay ahead of the tile loads (vmcnt retires in order)
        uint32_t Aw[TPW][AW];
        bool k1s[TPW];  // N_TILED: the lane's tile in slot t is at TILED_NA
        // tile (tk, og * 8 + o): the uniform start of k-tile row tk of the group plus the lane's tile offset
        const uint32_t lane_words = TILED ? 0u : (uint32_t)(o * N) >> 1;
        auto row_of = [&](int tk) __attribute__((always_inline)) {
            return reinterpret_cast<const uint32_t *>(tb + ((size_t)tk * c.OT + c.og * 8) * N);
        };
        auto load_slot = [&](int t, int tk) __attribute__((always_inline)) {
            if constexpr (TILED) {  // segment (bank, tk, og): its start and mask are wave-uniform
                const size_t seg = ((size_t)c.bank * c.IT + tk) * (size_t)(c.OT >> 3) + c.og;
                const uint32_t m = seg_mask(ts.seg_k1, seg);
                const uint32_t *row = reinterpret_cast<const uint32_t *>(tb) + ts.seg_off[seg];
                const bool k1 = ((m >> o) & 1u) != 0;
                const uint32_t lw = 16u * (uint32_t)o - 8u * (uint32_t)__builtin_popcount(m & ((1u << o) - 1u));
                load_lane_words_tiled(row, lw, j, k1, Aw[t]);
                k1s[t] = k1;
            } else {
                load_lane_words_u<N>(row_of(tk), lane_words, j, Aw[t]);
            }
        };
#pragma unroll
        for (int t = 0; t < TPW; t++) load_slot(t, c.kt0 + wave + GEMV_WAVES * min(t, ntiles - 1));
        __builtin_amdgcn_sched_barrier(0);  // svh's address comes from an argument load: its wait stays behind
        fetch_svh<PIN>(c, lane);
        if constexpr (CH == 2) chain_wait(a, c, wave);
        prologue<PRO, RT, WIN, SH, CH>(a, c, xs, wave, lane, pr);
        __syncthreads();
        if constexpr (CH == 2) {
            // every wave of this workgroup is past its wait: count it; the group's last clears both counters (no
            // workgroup of the group reads them again in this launch, and the next launch reads them after it)
            if (wave == 0 && lane == 0) {
                uint32_t *ctr = a.chain_ctr + (size_t)(2 * c.gy) * COUNTER_STRIDE;
                const uint32_t old = __hip_atomic_fetch_add(ctr + COUNTER_STRIDE, 1u, __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT);
                if (old == (uint32_t)a.chain_need2 - 1u) {
                    __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(ctr + COUNTER_STRIDE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
        const bool masked = k.wmask != 0xFFFFu;
        auto decode_at = [&](int t, int tt) __attribute__((always_inline)) {  // slot t holds the wave's tile tt
            const int kk = wave + GEMV_WAVES * tt;
            if constexpr (TILED) {
                const DecodeK kl = tiled_constants(k1s[t], ts.ka, ts.kb);
                if (masked) decode_tile_tiled<FAM, RT, true>(Aw[t], k1s[t], xs, kk, c.rows, kl, accA, accB, lane & 3);
                else decode_tile_tiled<FAM, RT, false>(Aw[t], k1s[t], xs, kk, c.rows, kl, accA, accB, lane & 3);
            } else {
                if (masked) decode_tile<FAM, N, RT, true>(Aw[t], xs, kk, c.rows, k, accA, accB, lane & 3);
                else decode_tile<FAM, N, RT, false>(Aw[t], xs, kk, c.rows, k, accA, accB, lane & 3);
            }
        };
        int t0 = 0;
        // Splits longer than TPW tiles per wave: every batch but the last refills each slot with the same slot of the
        // next batch as soon as it is decoded, so the next batch's words are in flight while this batch's remaining
        // tiles decode (a slot past the end re-reads the wave's last tile).
        for (; t0 + TPW < ntiles; t0 += TPW) {
#pragma unroll
            for (int t = 0; t < TPW; t++) {
                decode_at(t, t0 + t);
                load_slot(t, c.kt0 + wave + GEMV_WAVES * min(t0 + TPW + t, ntiles - 1));
            }
        }
#pragma unroll
        for (int t = 0; t < TPW; t++)
            if (t0 + t < ntiles) decode_at(t, t0 + t);

    } else {  // any other rate: the generic reader (runtime funnel per codeword)
        fetch_svh(c, lane);
        PrologueRegs<RT, WIN> pr;
        prologue_fetch<PRO, RT, WIN>(a, c, wave, lane, pr);
        prologue<PRO, RT, WIN, SH>(a, c, xs, wave, lane, pr);
        __syncthreads();
        for (int kk = wave; kk < c.KS; kk += GEMV_WAVES) {
            const int tk = c.kt0 + kk;
            const uint32_t *words = reinterpret_cast<const uint32_t *>(tb + ((size_t)tk * c.OT + c.og * 8 + o) * n);
            uint32_t w[16];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int t = 32 * j + 2 * i;
                w[i] = decode_pair_h2<FAM>(codeword_at(words, n, t), codeword_at(words, n, t + 1), k);
            }
            mfma_dot<RT>(w, xs, kk, c.rows, accA, accB, lane & 3, read_xfrag(xs, min(lane & 3, RT - 1), kk));
        }
    }
    // the matrix cores take the hash / pair weights as decoded, the codebook's values over 4096 (f16 subnormals
    // among them, which they multiply exactly); out_scale applies the 4096 to every arm alike
    float acc0[RT], acc1[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) {
        acc0[r] = accA[r >> 2][r & 3];
        acc1[r] = accB[r >> 2][r & 3];
    }

    // ---- cross-wave reduction
#pragma unroll
    for (int r = 0; r < RT; r++) {
        red[wave][r][o * 16 + j] = acc0[r];
        red[wave][r][o * 16 + j + 8] = acc1[r];
    }
    __syncthreads();
    if (a.fold) {  // the host enables the fold only for split dense launches and the MoE down projection
        fold_finish<RT, WIN, PRO == PRO_MID, SH>(a, c, red, wave, lane);
        return;
    }
    const bool direct = c.S == 1 && !a.partial_only;
    if (direct) {
        for (int idx = tid; idx < RT * 128; idx += GEMV_THREADS) {
            const int r = idx >> 7, col = idx & 127;
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < GEMV_WAVES; w++) s += red[w][r][col];
            red[0][r][col] = s * a.out_scale;
        }
        __syncthreads();
        for (int r = wave; r < c.rows; r += GEMV_WAVES) finish_block(a, c, r, red[0][r][lane], red[0][r][lane + 64], lane);
        return;
    }

    // Split k: wave 0 alone sums the workgroup's partial, stores it, arrives at the output group's counter and, if it
    // is the last split to arrive, finishes the group.  Its own stores are then the only ones the arrival has to
    // follow, so no workgroup barrier sits between the stores, the arrival and the finish.
    if (wave != 0) return;
    // An output group's splits share one XCD (and so one L2) when the workgroup remap applies (G % 8 == 0): its
    // partials then meet in that L2.  Otherwise they are written through to memory.
    const bool xcd_local = (c.G & 7) == 0;
    float *part = c.part;
    for (int r = 0; r < c.rows; r++) {
        float *dst = part + part_row<WIN, SH>(a, c, r) + (size_t)c.og * 128;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int col = lane + 64 * h;
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < GEMV_WAVES; w++) s += red[w][r][col];
            s *= a.out_scale;
            if (CH == 0 && (a.partial_only || xcd_local)) dst[col] = s;  // L1 writes through to the XCD's L2
            else __hip_atomic_store(dst + col, s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);  // through to memory
        }
    }
    if constexpr (CH == 1) {
        // the fused chain's gate/up: the stores are acknowledged, then this workgroup's arrival is counted for its
        // group (the down workgroups wait for all of them)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (lane == 0)
            __hip_atomic_fetch_add(a.chain_ctr + (size_t)(2 * c.gy) * COUNTER_STRIDE, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (a.partial_only || !a.fused_finish) return;

    // ---- single-launch finish.  The partial stores are acknowledged (s_waitcnt vmcnt(0)) before lane 0 bumps the
    // counter, so they are in the L2 / memory before any later arriver can see the count.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    uint32_t *ctr = &a.counters[(((size_t)c.proj * a.groups + c.g) * c.G + c.og) * COUNTER_STRIDE];
    uint32_t old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old != (uint32_t)(c.S - 1)) return;
    if (xcd_local) {
        // This CU's L1 may hold lines of these partials from an earlier call: drop them, then read the XCD's L2.
        asm volatile("buffer_inv sc0" ::: "memory");
        for (int r = 0; r < c.rows; r++) {
            float v0, v1;
            sum_planes<false>(part + (((size_t)c.g * c.S) * a.rows + r) * a.out + (size_t)c.og * 128,
                              (size_t)a.rows * a.out, c.S, lane, v0, v1);
            finish_block(a, c, r, v0, v1, lane);
        }
    } else {
        for (int r = 0; r < c.rows; r++) {
            float v0, v1;
            sum_planes<true>(part + (((size_t)c.g * c.S) * a.rows + r) * a.out + (size_t)c.og * 128,
                             (size_t)a.rows * a.out, c.S, lane, v0, v1);
            finish_block(a, c, r, v0, v1, lane);
        }
    }
    if (lane == 0) *ctr = 0u;  // every split has arrived: the next launch reads it after the kernel boundary
}

// Per-rate decode constants for a ragged bank (hash rows and pair rows differ by rate; the window mask does not).
template <int FAM>
__device__ __forceinline__ DecodeK rate_constants(const GemvArgs &a, int n) {
    DecodeK k = a.k;
    if constexpr (FAM == FAM_HASH || FAM == FAM_PAIR) table_row(a.table, n, k.mult, k.mask0, k.mask1, k.rot);
    return k;
}

// One workgroup's work for group g.  SH: g is a fused shared expert's group of token rows (compiled into the
// per-slot kernels only; the other groups run the SH = false copy, whose set-up is that of a launch without a
// shared expert).
// L: the workgroup's index within the group's (output group, split) grid; gy: the group's index in the grid (the
// fused chain's counters); proj: the projection.  CH: the fused chain's role (gemv_body).
template <int FAM, int N, int RT, int PRO, bool WIN, bool SH, int CH = 0>
__device__ __forceinline__ void gemv_group(int g, const void *x, const uint16_t *tr0, const uint16_t *suh0,
                                           const uint32_t *bank_of, const GemvGeo &geo, int rows, int x_dtype,
                                           const GemvArgs &a, uint16_t (*xs)[XS_PITCH], float (*red)[RT][128], int L,
                                           int gy, int proj) {
    GemvCtx c;
    c.x = x;
    c.x_div_m = geo.xdiv_m;
    c.x_dtype = x_dtype;
    c.IT = (int)(geo.tiles & 0xFFFFu);
    c.OT = (int)(geo.tiles >> 16);
    c.G = c.OT >> 3;
    c.S = (int)(geo.sks & 0xFFFFu);
    c.gy = gy;
    // keep an output group's splits on one XCD when G % 8 == 0 (workgroups go round-robin over the 8 XCDs)
    const bool remap = (c.G & 7) == 0;
    const unsigned q = remap ? (unsigned)L >> 3 : (unsigned)L, qs = div_by_magic(q, geo.s_m);
    c.og = remap ? (int)qs * 8 + (L & 7) : (int)qs;
    c.sp = (int)(q - qs * (unsigned)c.S);
    c.g = g;
    c.proj = proj;
    const bool p1 = c.proj != 0;
    const uint16_t *trellis;
    c.part = p1 ? a.partial[1] : a.partial[0];
    c.rows = rows;
    c.wslots = nullptr;
    if constexpr (SH) {  // the shared expert: expert 0 of the one-expert bank, token rows RT g .. RT g + RT - 1
        c.suh = a.sh_suh[c.proj];
        c.svh = a.sh_svh[c.proj];
        trellis = a.sh_trellis[c.proj];
        c.bank = 0;
        c.xg = RT * g;
        c.rows = min(RT, a.sh_rows - c.xg);
        c.slot0 = a.sh_from + c.xg;
    } else {
        // Projection 0's suh and trellis are preloaded arguments, so a dense launch's first loads issue without an
        // argument load ahead of them.  Projection 1 (grid z = 1) reads its pointers from `a` under a real branch:
        // the index is opaque to the compiler, so those loads cannot be hoisted into a select, and the empty asm
        // uses them inside the branch, so their wait stays there too (a wait for any scalar load waits for all).
        int pz = c.proj;
        asm volatile("" : "+s"(pz));
        c.suh = suh0;
        trellis = tr0;
        if (pz != 0) {
            c.suh = a.suh[pz];
            trellis = a.trellis[pz];
            asm volatile("" ::"s"(c.suh), "s"(trellis));
        }
        c.svh = p1 ? a.svh[1] : a.svh[0];
        c.xg = 0;
        c.slot0 = 0;
        if constexpr (WIN) {  // sorted MoE arm: this group is an expert window (windows past the count do nothing)
            if ((uint32_t)c.g >= *a.win_count) return;
            c.bank = (int)min(a.win_expert[c.g], (uint32_t)(a.bank_limit - 1));
            c.rows = (int)min(a.win_rows[c.g], (uint32_t)MOE_WINDOW_ROWS);
            c.wslots = a.win_slots + (size_t)c.g * MOE_WINDOW_ROWS;
        } else {
            c.xg = (int)div_by_magic((uint32_t)c.g, geo.xdiv_m) * rows;
            if (a.rows_total) c.rows = min(rows, a.rows_total - c.xg);  // row groups: the last holds the rest
            c.slot0 = c.g;
            c.bank = bank_of ? (int)min(bank_of[c.g], (uint32_t)(a.bank_limit - 1)) : min(c.g, a.bank_limit - 1);
        }
    }
    c.KS = (int)(geo.sks >> 16);
    c.kt0 = c.sp * c.KS;
    c.sv0 = c.sv1 = 0.f;  // fetched by gemv_body once the tile loads are out

    if constexpr (N >= 0) {
        const int n = N ? N : a.n;
        const uint16_t *tb = trellis + (size_t)c.bank * c.IT * c.OT * n;
        gemv_body<FAM, N, RT, PRO, WIN, SH, (N > 0 && !WIN && !SH && CH == 0), CH>(a, c, tb, n, a.k, xs, red);
    } else if constexpr (N == N_TILED) {
        // Per-tile-rate bank: every tile at TILED_NA or TILED_NB, read through the projection's segment tables (a
        // fused shared expert keeps its own uniform rate, a lane-reader rate the host checked).
        if constexpr (SH) {
            const int n = a.sh_n;
            const DecodeK k = rate_constants<FAM>(a, n);
            switch (n) {
            case 16: gemv_body<FAM, 16, RT, PRO, WIN, SH>(a, c, trellis, n, k, xs, red); break;
            case 24: gemv_body<FAM, 24, RT, PRO, WIN, SH>(a, c, trellis, n, k, xs, red); break;
            case 32: gemv_body<FAM, 32, RT, PRO, WIN, SH>(a, c, trellis, n, k, xs, red); break;
            case 40: gemv_body<FAM, 40, RT, PRO, WIN, SH>(a, c, trellis, n, k, xs, red); break;
            case 48: gemv_body<FAM, 48, RT, PRO, WIN, SH>(a, c, trellis, n, k, xs, red); break;
            case 64: gemv_body<FAM, 64, RT, PRO, WIN, SH>(a, c, trellis, n, k, xs, red); break;
            default: break;
            }
        } else {
            TiledSrc ts;
            ts.seg_off = p1 ? a.seg_off[1] : a.seg_off[0];
            ts.seg_k1 = p1 ? a.seg_k1[1] : a.seg_k1[0];
            ts.ka = rate_constants<FAM>(a, TILED_NA);
            ts.kb = rate_constants<FAM>(a, TILED_NB);
            gemv_body<FAM, N_TILED, RT, PRO, WIN, SH>(a, c, trellis, 0, a.k, xs, red, ts);
        }
    } else {
        // Ragged bank: the rate comes from the expert's meta row (a shared expert has its own uniform rate).
        // N == -1 serves the rates with a lane reader and skips the rest; N == -2 (a second launch over the same
        // grid) serves only the rest, with the generic reader (kept out of the first kernel, whose registers it
        // would otherwise set).
        int n;
        const uint16_t *tb;
        if constexpr (SH) {
            n = a.sh_n;
            tb = trellis;
        } else {
            const int col = p1 ? a.meta_col[1] : a.meta_col[0];
            const uint32_t *m = a.meta + (size_t)c.bank * 8;
            n = (int)m[col];
            tb = trellis + 2 * (size_t)m[4 + col];
        }
        const DecodeK k = rate_constants<FAM>(a, n);
        const bool lane_rate = n == 16 || n == 24 || n == 32 || n == 40 || n == 48 || n == 64;
        if constexpr (N == -1) {
            switch (n) {
            case 16: gemv_body<FAM, 16, RT, PRO, WIN, SH>(a, c, tb, n, k, xs, red); break;
            case 24: gemv_body<FAM, 24, RT, PRO, WIN, SH>(a, c, tb, n, k, xs, red); break;
            case 32: gemv_body<FAM, 32, RT, PRO, WIN, SH>(a, c, tb, n, k, xs, red); break;
            case 40: gemv_body<FAM, 40, RT, PRO, WIN, SH>(a, c, tb, n, k, xs, red); break;
            case 48: gemv_body<FAM, 48, RT, PRO, WIN, SH>(a, c, tb, n, k, xs, red); break;
            case 64: gemv_body<FAM, 64, RT, PRO, WIN, SH>(a, c, tb, n, k, xs, red); break;
            default: break;
            }
        } else {
            if (!lane_rate) gemv_body<FAM, 0, RT, PRO, WIN, SH>(a, c, tb, n, k, xs, red);
        }
    }
}

// N > 0: one rate for the launch; N == 0: the generic reader; N == -1 / -2: per-expert rate from the ragged meta table
// (lane-reader rates / the other rates), dispatched per workgroup; N == N_TILED: per-tile rates.
// SHP: the launch carries a fused shared expert's rows (either MoE arm): a separate instantiation, so launches
// without them keep a kernel whose registers hold none of it.
template <int FAM, int N, int RT, int PRO, bool WIN, bool SHP>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_kernel(const void *x, const uint16_t *tr0, const uint16_t *suh0,
                                                            const uint32_t *bank_of, uint32_t tiles, uint32_t sks,
                                                            uint32_t s_m, uint32_t xdiv_m, int rows_dt, int sh_groups,
                                                            GemvArgs a) {
    // The leading scalar arguments are the ones the first loads need (the input and suh of the prologue, the tile
    // words, the block-to-tile map and whether this group is a fused shared expert's): the build preloads them into
    // SGPRs (14 dwords, rows and x's dtype sharing one), so those loads issue without waiting for an argument load
    // and the map takes no division.  The struct `a` holds everything for the rest of the kernel.
    const int rows = rows_dt & 0xFFFF, x_dtype = rows_dt >> 16;
    const GemvGeo geo{tiles, sks, s_m, xdiv_m};
    // A shared expert's groups hold SH_ROWS token rows each, so its weights are decoded once per SH_ROWS rows.
    constexpr int RX = (SHP && RT < SH_ROWS) ? SH_ROWS : RT;
    __shared__ __align__(16) uint16_t xs[RX][XS_PITCH];
    __shared__ float red[GEMV_WAVES * RX * 128];
    int g = blockIdx.y;
    if constexpr (SHP && RT == 1 && !WIN) {
        // The per-slot MoE arm with a shared expert: its groups come first (they carry SH_ROWS rows each, the
        // heaviest workgroups, so they start in the first round), then the routed slots.
        if (g < sh_groups) {
            gemv_group<FAM, N, SH_ROWS, PRO, WIN, true>(g, x, tr0, suh0, bank_of, geo, rows, x_dtype, a, xs,
                                                        reinterpret_cast<float (*)[SH_ROWS][128]>(red), blockIdx.x,
                                                        g, blockIdx.z);
            return;
        }
        g -= sh_groups;
    }
    if constexpr (SHP && WIN) {
        // The sorted MoE arm with a shared expert: its groups of SH_ROWS (= MOE_WINDOW_ROWS) token rows come first,
        // then the expert windows.
        static_assert(RT == SH_ROWS, "a window holds as many rows as a shared group");
        if (g < sh_groups) {
            gemv_group<FAM, N, SH_ROWS, PRO, false, true>(g, x, tr0, suh0, bank_of, geo, rows, x_dtype, a, xs,
                                                          reinterpret_cast<float (*)[SH_ROWS][128]>(red), blockIdx.x,
                                                          g, blockIdx.z);
            return;
        }
        g -= sh_groups;
    }
    gemv_group<FAM, N, RT, PRO, WIN, false>(g, x, tr0, suh0, bank_of, geo, rows, x_dtype, a, xs,
                                            reinterpret_cast<float (*)[RT][128]>(red), blockIdx.x, blockIdx.y,
                                            blockIdx.z);
}

// The per-slot decode chain in one launch (run_moe_chain): a 1D grid of w1 gate/up workgroups (a1, PRO_X, grid
// order x = (output group, split), then group, then projection, as gemv_kernel's) and then the down workgroups (a2,
// PRO_MID).  Workgroups start in index order on each XCD, so when a down workgroup starts every gate/up workgroup
// before it on that XCD has started, and the ones on other XCDs only wait behind gate/up work: the waits end.  A
// shared expert's groups (SHP) come first in both halves.
// One half of the fused chain (CH 1: gate/up with PRO_X, CH 2: down with PRO_MID) for workgroup b of that half.
template <int FAM, int N, bool SHP, int CH>
__device__ __forceinline__ void chain_half(const GemvArgs &a, const GemvGeo &geo, int b, uint16_t (*xs)[XS_PITCH],
                                           float *red) {
    constexpr int PRO = CH == 1 ? PRO_X : PRO_MID;
    const int X = (int)(geo.tiles >> 19) * (int)(geo.sks & 0xFFFFu);  // output groups (out / 16 / 8) x splits
    const int q = b / X;
    const int gy = q % a.groups, proj = q / a.groups, L = b - q * X;
    const void *x = CH == 1 ? a.x : nullptr;
    if (SHP && gy < a.sh_groups) {
        gemv_group<FAM, N, SH_ROWS, PRO, false, true, CH>(gy, x, a.trellis[0], a.suh[0], a.bank_of, geo, a.rows,
                                                          a.x_dtype, a, xs,
                                                          reinterpret_cast<float (*)[SH_ROWS][128]>(red), L, gy, proj);
        return;
    }
    gemv_group<FAM, N, 1, PRO, false, false, CH>(gy - (SHP ? a.sh_groups : 0), x, a.trellis[0], a.suh[0], a.bank_of,
                                                 geo, a.rows, a.x_dtype, a, xs,
                                                 reinterpret_cast<float (*)[1][128]>(red), L, gy, proj);
}

// The per-slot decode chain in one launch (run_moe_chain): a 1D grid of w1 gate/up workgroups (a1, PRO_X, grid
// order x = (output group, split), then group, then projection, as gemv_kernel's) and then the down workgroups (a2,
// PRO_MID).  Workgroups start in index order on each XCD, so when a down workgroup starts every gate/up workgroup
// before it on that XCD has started, and the ones on other XCDs only wait behind gate/up work: the waits end.  A
// shared expert's groups (SHP) come first in both halves.
template <int FAM, int N, bool SHP>
__global__ __launch_bounds__(GEMV_THREADS) void moe_chain_kernel(GemvArgs a1, GemvArgs a2, GemvGeo geo1, GemvGeo geo2,
                                                                 int w1) {
    constexpr int RX = SHP ? SH_ROWS : 1;
    __shared__ __align__(16) uint16_t xs[RX][XS_PITCH];
    __shared__ float red[GEMV_WAVES * RX * 128];
    const int b = (int)blockIdx.x;
    if (b < w1) chain_half<FAM, N, SHP, 1>(a1, geo1, b, xs, red);
    else chain_half<FAM, N, SHP, 2>(a2, geo2, b - w1, xs, red);
}

// Separate finish: one wave per (output group, row, group, projection).
template <int FAM>
__global__ __launch_bounds__(64) void gemv_finish_kernel(GemvArgs a) {
    GemvCtx c;
    c.og = blockIdx.x;
    const int r = blockIdx.y % a.rows;
    c.g = blockIdx.y / a.rows;
    if (a.rows_total && c.g * a.rows + r >= a.rows_total) return;  // the last row group's rows past the rest
    c.proj = blockIdx.z;
    const bool p1 = c.proj != 0;
    c.svh = p1 ? a.svh[1] : a.svh[0];
    const float *part = p1 ? a.partial[1] : a.partial[0];
    c.bank = a.bank_of ? (int)min(a.bank_of[c.g], (uint32_t)(a.bank_limit - 1)) : min(c.g, a.bank_limit - 1);
    const int lane = threadIdx.x;
    const size_t sv = (size_t)c.bank * a.out + (size_t)c.og * 128;
    c.sv0 = h2f(c.svh[sv + lane]);
    c.sv1 = h2f(c.svh[sv + lane + 64]);
    float v0, v1;
    sum_planes<false>(part + (((size_t)c.g * a.splits) * a.rows + r) * a.out + (size_t)c.og * 128,
                      (size_t)a.rows * a.out, a.splits, lane, v0, v1);
    finish_block(a, c, r, v0, v1, lane);
}

template <int FAM, int N, int RT, int PRO, bool WIN, bool SHP = false>
static void launch_one(const GemvArgs &a, dim3 grid, hipStream_t s) {
    const GemvGeo geo = gemv_geo(a);
    hipLaunchKernelGGL((gemv_kernel<FAM, N, RT, PRO, WIN, SHP>), grid, dim3(GEMV_THREADS), 0, s, a.x, a.trellis[0],
                       a.suh[0], a.bank_of, geo.tiles, geo.sks, geo.s_m, geo.xdiv_m, a.rows | (a.x_dtype << 16),
                       a.sh_groups, a);
}

template <int FAM, int N, int PRO>
static void launch_slot(const GemvArgs &a, dim3 grid, hipStream_t s) {  // one row per group; shared rows or not
    if (a.sh_groups > 0) launch_one<FAM, N, 1, PRO, false, true>(a, grid, s);
    else launch_one<FAM, N, 1, PRO, false, false>(a, grid, s);
}

template <int FAM, int N, int PRO>
static hipError_t launch_gemv_n(const GemvArgs &a, hipStream_t s) {
    const int G = a.out / 128;
    // the block-to-tile map's packed fields (gemv_geo) and its divisions' exactness
    if (a.in / 16 > 0xFFFF || a.out / 16 > 0xFFFF || a.splits < 1 || (a.in / 16) % a.splits || a.x_div < 1 ||
        a.x_div > 255 || (unsigned long long)G * a.splits * (unsigned)a.splits >= (1ull << 32))
        return hipErrorInvalidValue;  // x rows are found as slot / x_div for up to 2^24 slots
    dim3 grid((unsigned)(G * a.splits), (unsigned)a.groups, (unsigned)a.nproj);
    if (a.win_count) {  // the sorted MoE arm: expert windows of MOE_WINDOW_ROWS rows, f32 planes or the fold out
        if (a.rows != MOE_WINDOW_ROWS || !(a.partial_only || a.fold)) return hipErrorInvalidValue;
        if (a.sh_groups > 0) launch_one<FAM, N, MOE_WINDOW_ROWS, PRO, true, true>(a, grid, s);
        else launch_one<FAM, N, MOE_WINDOW_ROWS, PRO, true, false>(a, grid, s);
    } else if constexpr (PRO == PRO_X && N >= 0) {
        if (a.rows <= 1) launch_slot<FAM, N, PRO>(a, grid, s);
        else if (a.rows <= 2) launch_one<FAM, N, 2, PRO, false>(a, grid, s);
        else if (a.rows <= 4) launch_one<FAM, N, 4, PRO, false>(a, grid, s);
        else if (a.rows <= 8) launch_one<FAM, N, 8, PRO, false>(a, grid, s);
        else launch_one<FAM, N, 16, PRO, false>(a, grid, s);
    } else {  // the MoE decode chain: one row per (slot, bank) pair
        if (a.rows != 1) return hipErrorInvalidValue;
        launch_slot<FAM, N, PRO>(a, grid, s);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (!a.partial_only && a.splits > 1 && !a.fused_finish) {
        hipLaunchKernelGGL(gemv_finish_kernel<FAM>, dim3((unsigned)G, (unsigned)(a.rows * a.groups), (unsigned)a.nproj),
                           dim3(64), 0, s, a);
        e = hipGetLastError();
    }
    return e;
}

template <int FAM, int N>
static void launch_chain_n(const GemvArgs &a1, const GemvArgs &a2, unsigned w1, unsigned w2, hipStream_t s) {
    const GemvGeo g1 = gemv_geo(a1), g2 = gemv_geo(a2);
    if (a1.sh_groups > 0)
        hipLaunchKernelGGL((moe_chain_kernel<FAM, N, true>), dim3(w1 + w2), dim3(GEMV_THREADS), 0, s, a1, a2, g1, g2,
                           (int)w1);
    else
        hipLaunchKernelGGL((moe_chain_kernel<FAM, N, false>), dim3(w1 + w2), dim3(GEMV_THREADS), 0, s, a1, a2, g1, g2,
                           (int)w1);
}

template <int FAM>
static hipError_t launch_moe_chain(const GemvArgs &a1, const GemvArgs &a2, hipStream_t s) {
    // the block-to-tile maps' packed fields and divisions (as launch_gemv_n checks them), one row per group, the
    // same rate and groups in both halves, gate/up writing planes and down folding
    for (const GemvArgs *a : {&a1, &a2}) {
        if (a->in / 16 > 0xFFFF || a->out / 16 > 0xFFFF || a->splits < 1 || (a->in / 16) % a->splits ||
            a->x_div < 1 || a->x_div > 255 || a->rows != 1 || !a->chain_ctr)
            return hipErrorInvalidValue;
    }
    if (a1.n != a2.n || a1.groups != a2.groups || a1.sh_groups != a2.sh_groups || a1.nproj != 2 || a2.nproj != 1 ||
        !a1.partial_only || !a2.fold || a1.win_count || a2.win_count || a1.meta || a1.seg_off[0])
        return hipErrorInvalidValue;
    const unsigned w1 = (unsigned)(a1.out / 128 * a1.splits) * (unsigned)a1.groups * 2u;
    const unsigned w2 = (unsigned)(a2.out / 128 * a2.splits) * (unsigned)a2.groups;
    if ((unsigned)a1.chain_need != w1 / (unsigned)a1.groups || (unsigned)a2.chain_need2 != w2 / (unsigned)a2.groups)
        return hipErrorInvalidValue;
    switch (a1.n) {
    case 16: launch_chain_n<FAM, 16>(a1, a2, w1, w2, s); break;
    case 24: launch_chain_n<FAM, 24>(a1, a2, w1, w2, s); break;
    case 32: launch_chain_n<FAM, 32>(a1, a2, w1, w2, s); break;
    case 40: launch_chain_n<FAM, 40>(a1, a2, w1, w2, s); break;
    case 48: launch_chain_n<FAM, 48>(a1, a2, w1, w2, s); break;
    case 64: launch_chain_n<FAM, 64>(a1, a2, w1, w2, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int FAM, int PRO>
static hipError_t launch_gemv_fam(const GemvArgs &a, hipStream_t s) {
    if (a.seg_off[0]) {  // per-tile rates: the hash-product families only (the host refuses the others)
        if constexpr (FAM == FAM_PAIR || FAM == FAM_MUL1) return hipErrorInvalidValue;
        else return launch_gemv_n<FAM, N_TILED, PRO>(a, s);
    }
    if (a.meta) {  // ragged: the lane-reader rates, then any other rate (unless the host ruled them out)
        hipError_t e = launch_gemv_n<FAM, -1, PRO>(a, s);
        return e != hipSuccess || a.meta_lane_only ? e : launch_gemv_n<FAM, -2, PRO>(a, s);
    }
    switch (a.n) {
    case 16: return launch_gemv_n<FAM, 16, PRO>(a, s);
    case 24: return launch_gemv_n<FAM, 24, PRO>(a, s);
    case 32: return launch_gemv_n<FAM, 32, PRO>(a, s);
    case 40: return launch_gemv_n<FAM, 40, PRO>(a, s);
    case 48: return launch_gemv_n<FAM, 48, PRO>(a, s);
    case 64: return launch_gemv_n<FAM, 64, PRO>(a, s);
    default: return launch_gemv_n<FAM, 0, PRO>(a, s);
    }
}

#ifdef EXL3_GEMV_FAM
// One translation unit per codebook family (compiled in parallel): exl3_gemv_<family>.hip defines EXL3_GEMV_FAM.
#define EXL3_CAT2(a, b) a##b
#define EXL3_CAT(a, b) EXL3_CAT2(a, b)
hipError_t EXL3_CAT(run_gemv_fam_, EXL3_GEMV_FAM)(int prologue, const GemvArgs &a, hipStream_t s) {
    return prologue == PRO_MID ? launch_gemv_fam<EXL3_GEMV_FAM, PRO_MID>(a, s)
                               : launch_gemv_fam<EXL3_GEMV_FAM, PRO_X>(a, s);
}

hipError_t EXL3_CAT(run_moe_chain_fam_, EXL3_GEMV_FAM)(const GemvArgs &a1, const GemvArgs &a2, hipStream_t s) {
    return launch_moe_chain<EXL3_GEMV_FAM>(a1, a2, s);
}
#endif

}  // namespace exl3
