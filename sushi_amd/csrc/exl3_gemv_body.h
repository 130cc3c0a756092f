// (Kernel body shared by the per-family translation units exl3_gemv_<family>.hip.)
// Trellis GEMV for 1..8 rows: the decode arm of the dense linear (linear.linear, beamivalice/sushi
// src/exl3/linear.zig:317-336, Metal ROWS_SOURCE/ROWS_FINISH_SOURCE in src/exl3/project_rows.zig:145-249, :345-362)
// and of the routed MoE chain (PAIR_GEMV_SOURCE :2082-2241, DOWN_FUSED_SOURCE :1820-2023 in
// src/exl3/expert_exl3_kernels.zig).
//
// MI355X layout.  A workgroup (4 waves) owns one output group of 8 tiles (128 outputs, one Hadamard block) of one
// (bank, x-block) pair over one k split (whole 128-blocks).  Per k-tile row a wave streams the group's 8 tiles,
// which lie contiguous in the pack order [IT][OT][n] (8*n*2 bytes, 1 KiB at K4): lane = 8*o + j reads chunk j of
// tile o, the words carrying codewords 32j..32j+31 = fragment threads 4j..4j+3 of tensorCorePerm = output columns
// j and j+8 over all 16 k rows.  Every lane owns two output columns outright, decodes its 32 weights into registers
// as packed f16 pairs (t, t+1) = rows (r, r+1) of one column and feeds v_dot2_f32_f16 against the prepared input
// held in LDS.  No cross-lane reduction happens inside a wave; the 4 waves (different k-tiles) meet once in LDS.
// The prologue prepares the split's k range (x * suh, FWHT-128, f16) or, for the MoE down projection, builds the
// SwiGLU mid from the gate/up planes.  The finish (FWHT-128, * svh) runs in the same launch when there is one
// split, in the last workgroup of an output group to arrive (fused finish), or in a small second kernel.
#pragma once
#include "exl3_kernels.h"
#include "exl3_tables.h"

namespace exl3 {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t w, uint32_t x, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, w), __builtin_bit_cast(h2_t, x), acc, false);
}

constexpr int GEMV_WAVES = 4;
constexpr int GEMV_THREADS = 64 * GEMV_WAVES;
constexpr int MAX_KSPAN = 2048;

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

__device__ __forceinline__ float silu(float g) {
    // g * sigmoid(g), evaluated on exp(-|g|) so neither branch overflows (the reference's mid uses the same split)
    const float e = __expf(-fabsf(g));
    const float s = g >= 0.f ? 1.f / (1.f + e) : e / (1.f + e);
    return g * s;
}

struct GemvCtx {
    int g, proj, bank, og, sp, S, KS, kt0, IT, OT, G;
};

// Output FWHT + svh for one row of a 128-output block held as (v0 = col lane, v1 = col lane + 64).
__device__ __forceinline__ void finish_block(const GemvArgs &a, const GemvCtx &c, int rho, float v0, float v1,
                                             int lane) {
    fwht128_wave(v0, v1, lane);
    const size_t sv = (size_t)c.bank * a.out + (size_t)c.og * 128;
    const size_t yo = ((size_t)c.g * a.rows + rho) * a.out + (size_t)c.og * 128;
    store_y(a.y, a.y_dtype, yo + lane, v0 * HAD_SCALE * h2f(a.svh[c.proj][sv + lane]));
    store_y(a.y, a.y_dtype, yo + lane + 64, v1 * HAD_SCALE * h2f(a.svh[c.proj][sv + lane + 64]));
}

template <int FAM, int N, int RT>
__device__ __forceinline__ void gemv_main(const GemvArgs &a, const GemvCtx &c, const uint16_t *__restrict__ tb,
                                          int n, const DecodeK &k, const uint16_t (*xs)[MAX_KSPAN], int wave, int lane,
                                          float (&acc0)[RT], float (&acc1)[RT]) {
    const int o = lane >> 3, j = lane & 7;
    for (int kk = wave; kk < c.KS; kk += GEMV_WAVES) {
        const int tk = c.kt0 + kk;
        const uint32_t *words = reinterpret_cast<const uint32_t *>(tb + ((size_t)tk * c.OT + c.og * 8 + o) * n);
        uint4 X[RT], Y[RT];
#pragma unroll
        for (int r = 0; r < RT; r++) {
            X[r] = *reinterpret_cast<const uint4 *>(&xs[r][kk * 16]);
            Y[r] = *reinterpret_cast<const uint4 *>(&xs[r][kk * 16 + 8]);
        }
        if constexpr (N != 0) {
            uint32_t A[LaneBits<N>::AW];
            load_lane_words<N>(words, j, A);
#pragma unroll
            for (int q = 0; q < 4; q++) {
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const int u = 8 * q + 2 * p;
                    const uint32_t h = decode_pair_h2<FAM>(lane_codeword<N>(A, u), lane_codeword<N>(A, u + 1), k);
#pragma unroll
                    for (int r = 0; r < RT; r++) {
                        const uint4 &V = (p & 1) ? Y[r] : X[r];
                        const uint32_t xv = q == 0 ? V.x : q == 1 ? V.y : q == 2 ? V.z : V.w;
                        if (p < 2) acc0[r] = dot2(h, xv, acc0[r]);
                        else acc1[r] = dot2(h, xv, acc1[r]);
                    }
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) {
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    const int t = 32 * j + 8 * q + 2 * p;
                    const uint32_t h = decode_pair_h2<FAM>(codeword_at(words, n, t), codeword_at(words, n, t + 1), k);
#pragma unroll
                    for (int r = 0; r < RT; r++) {
                        const uint4 &V = (p & 1) ? Y[r] : X[r];
                        const uint32_t xv = q == 0 ? V.x : q == 1 ? V.y : q == 2 ? V.z : V.w;
                        if (p < 2) acc0[r] = dot2(h, xv, acc0[r]);
                        else acc1[r] = dot2(h, xv, acc1[r]);
                    }
                }
            }
        }
    }
}

// Per-rate decode constants for a ragged bank (hash rows and pair rows differ by rate; the window mask does not).
template <int FAM>
__device__ __forceinline__ DecodeK rate_constants(const GemvArgs &a, int n) {
    DecodeK k = a.k;
    if constexpr (FAM == FAM_HASH || FAM == FAM_PAIR) {
        table_row(a.table, n, k.mult, k.mask0, k.mask1, k.rot);
    }
    return k;
}

// N > 0: one rate for the launch; N < 0: per-expert rate from the ragged meta table, dispatched per workgroup.
template <int FAM, int N, int RT, int PRO>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_kernel(GemvArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    GemvCtx c;
    c.IT = a.in >> 4;
    c.OT = a.out >> 4;
    c.G = c.OT >> 3;
    c.S = a.splits;
    const int L = blockIdx.x;
    if ((c.G & 7) == 0) {  // keep an output group's splits on one XCD (workgroups go round-robin over 8 XCDs)
        const int xcd = L & 7, r = L >> 3;
        c.og = (r / c.S) * 8 + xcd;
        c.sp = r % c.S;
    } else {
        c.og = L / c.S;
        c.sp = L % c.S;
    }
    c.g = blockIdx.y;
    c.proj = blockIdx.z;
    c.bank = a.bank_of ? (int)min(a.bank_of[c.g], (uint32_t)(a.bank_limit - 1)) : c.g;
    c.KS = c.IT / c.S;
    c.kt0 = c.sp * c.KS;

    __shared__ __align__(16) uint16_t xs[RT][MAX_KSPAN];
    __shared__ float red[GEMV_WAVES][RT][128];
    __shared__ int last_flag;

    // ---- prologue over this split's k range
    const int nblk = c.KS >> 3;
    for (int job = wave; job < nblk * RT; job += GEMV_WAVES) {
        const int rho = job / nblk, b = job - rho * nblk;
        const int kb = c.kt0 * 16 + b * 128;
        float v0 = 0.f, v1 = 0.f;
        if (rho < a.rows) {
            const size_t si = (size_t)c.bank * a.in + kb;
            if constexpr (PRO == PRO_X) {  // prepareInput (expert_exl3.zig:490-501)
                const size_t xi = ((size_t)(c.g / a.x_div) * a.rows + rho) * a.in + kb;
                v0 = f16r(load_x(a.x, a.x_dtype, xi + lane));
                v1 = f16r(load_x(a.x, a.x_dtype, xi + lane + 64));
            } else {  // the SwiGLU mid of the decode chain (DOWN_FUSED_SOURCE prologue, :1838-1920)
                float gv[2], uv[2];
#pragma unroll
                for (int pj = 0; pj < 2; pj++) {
                    float w0 = 0.f, w1 = 0.f;
                    for (int s2 = 0; s2 < a.mid_splits; s2++) {
                        const float *pp = a.mid_part[pj] + ((size_t)c.g * a.mid_splits + s2) * a.in + kb;
                        w0 += pp[lane];
                        w1 += pp[lane + 64];
                    }
                    fwht128_wave(w0, w1, lane);
                    w0 *= HAD_SCALE * h2f(a.mid_svh[pj][si + lane]);
                    w1 *= HAD_SCALE * h2f(a.mid_svh[pj][si + lane + 64]);
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
                v0 = silu(gv[0]) * uv[0];
                v1 = silu(gv[1]) * uv[1];
            }
            v0 *= h2f(a.suh[c.proj][si + lane]);
            v1 *= h2f(a.suh[c.proj][si + lane + 64]);
            fwht128_wave(v0, v1, lane);
            v0 *= HAD_SCALE;
            v1 *= HAD_SCALE;
        }
        xs[rho][b * 128 + lane] = __half_as_ushort(__float2half_rn(v0));
        xs[rho][b * 128 + lane + 64] = __half_as_ushort(__float2half_rn(v1));
    }
    __syncthreads();

    // ---- decode + dot
    float acc0[RT], acc1[RT];
#pragma unroll
    for (int r = 0; r < RT; r++) acc0[r] = acc1[r] = 0.f;
    if constexpr (N >= 0) {
        const int n = N ? N : a.n;
        const uint16_t *tb = a.trellis[c.proj] + (size_t)c.bank * c.IT * c.OT * n;
        gemv_main<FAM, N, RT>(a, c, tb, n, a.k, xs, wave, lane, acc0, acc1);
    } else {
        const uint32_t *m = a.meta + (size_t)c.bank * 8;
        const int n = (int)m[a.meta_col[c.proj]];
        const uint16_t *tb = a.trellis[c.proj] + 2 * (size_t)m[4 + a.meta_col[c.proj]];
        const DecodeK k = rate_constants<FAM>(a, n);
        switch (n) {
        case 16: gemv_main<FAM, 16, RT>(a, c, tb, n, k, xs, wave, lane, acc0, acc1); break;
        case 24: gemv_main<FAM, 24, RT>(a, c, tb, n, k, xs, wave, lane, acc0, acc1); break;
        case 32: gemv_main<FAM, 32, RT>(a, c, tb, n, k, xs, wave, lane, acc0, acc1); break;
        case 48: gemv_main<FAM, 48, RT>(a, c, tb, n, k, xs, wave, lane, acc0, acc1); break;
        case 64: gemv_main<FAM, 64, RT>(a, c, tb, n, k, xs, wave, lane, acc0, acc1); break;
        default: gemv_main<FAM, 0, RT>(a, c, tb, n, k, xs, wave, lane, acc0, acc1); break;
        }
    }

    // ---- cross-wave reduction
    {
        const int o = lane >> 3, j = lane & 7;
#pragma unroll
        for (int r = 0; r < RT; r++) {
            red[wave][r][o * 16 + j] = acc0[r];
            red[wave][r][o * 16 + j + 8] = acc1[r];
        }
    }
    __syncthreads();
    const bool direct = c.S == 1 && !a.partial_only;
    float *part = a.partial[c.proj];
    for (int idx = tid; idx < RT * 128; idx += GEMV_THREADS) {
        const int r = idx >> 7, col = idx & 127;
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < GEMV_WAVES; w++) s += red[w][r][col];
        s *= a.out_scale;
        if (direct) red[0][r][col] = s;
        else if (r < a.rows) part[(((size_t)c.g * c.S + c.sp) * a.rows + r) * a.out + (size_t)c.og * 128 + col] = s;
    }
    if (direct) {
        __syncthreads();
        for (int r = wave; r < a.rows; r += GEMV_WAVES) finish_block(a, c, r, red[0][r][lane], red[0][r][lane + 64], lane);
        return;
    }
    if (a.partial_only || !a.fused_finish) return;

    // ---- fused finish: the last split of this output group to arrive sums the partials and finishes.
    __threadfence();
    __syncthreads();
    uint32_t *ctr = &a.counters[((size_t)c.proj * a.groups + c.g) * c.G + c.og];
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last_flag = old == (uint32_t)(c.S - 1);
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    for (int r = wave; r < a.rows; r += GEMV_WAVES) {
        float v0 = 0.f, v1 = 0.f;
        for (int s2 = 0; s2 < c.S; s2++) {
            const float *pp = part + (((size_t)c.g * c.S + s2) * a.rows + r) * a.out + (size_t)c.og * 128;
            v0 += __builtin_nontemporal_load(pp + lane);
            v1 += __builtin_nontemporal_load(pp + lane + 64);
        }
        finish_block(a, c, r, v0, v1, lane);
    }
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Separate finish: one wave per (output group, row, group, projection).
template <int FAM>
__global__ __launch_bounds__(64) void gemv_finish_kernel(GemvArgs a) {
    GemvCtx c;
    c.og = blockIdx.x;
    const int r = blockIdx.y % a.rows;
    c.g = blockIdx.y / a.rows;
    c.proj = blockIdx.z;
    c.bank = a.bank_of ? (int)min(a.bank_of[c.g], (uint32_t)(a.bank_limit - 1)) : c.g;
    const int lane = threadIdx.x;
    float v0 = 0.f, v1 = 0.f;
    for (int s = 0; s < a.splits; s++) {
        const float *pp = a.partial[c.proj] + (((size_t)c.g * a.splits + s) * a.rows + r) * a.out + (size_t)c.og * 128;
        v0 += pp[lane];
        v1 += pp[lane + 64];
    }
    finish_block(a, c, r, v0, v1, lane);
}

template <int FAM, int N, int PRO>
static hipError_t launch_gemv_n(const GemvArgs &a, hipStream_t s) {
    const int G = a.out / 128;
    dim3 grid((unsigned)(G * a.splits), (unsigned)a.groups, (unsigned)a.nproj);
    if constexpr (PRO == PRO_X && N >= 0) {
        if (a.rows <= 1) hipLaunchKernelGGL((gemv_kernel<FAM, N, 1, PRO>), grid, dim3(GEMV_THREADS), 0, s, a);
        else if (a.rows <= 2) hipLaunchKernelGGL((gemv_kernel<FAM, N, 2, PRO>), grid, dim3(GEMV_THREADS), 0, s, a);
        else if (a.rows <= 4) hipLaunchKernelGGL((gemv_kernel<FAM, N, 4, PRO>), grid, dim3(GEMV_THREADS), 0, s, a);
        else hipLaunchKernelGGL((gemv_kernel<FAM, N, 8, PRO>), grid, dim3(GEMV_THREADS), 0, s, a);
    } else {  // the MoE stages run one row per (slot, bank) pair
        if (a.rows != 1) return hipErrorInvalidValue;
        hipLaunchKernelGGL((gemv_kernel<FAM, N, 1, PRO>), grid, dim3(GEMV_THREADS), 0, s, a);
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

template <int FAM, int PRO>
static hipError_t launch_gemv_fam(const GemvArgs &a, hipStream_t s) {
    if (a.meta) return launch_gemv_n<FAM, -1, PRO>(a, s);
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
    return prologue == PRO_MID ? launch_gemv_fam<EXL3_GEMV_FAM, PRO_MID>(a, s) : launch_gemv_fam<EXL3_GEMV_FAM, PRO_X>(a, s);
}
#endif

}  // namespace exl3
