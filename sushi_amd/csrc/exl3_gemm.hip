// Dense trellis GEMM for wide row counts (the prefill arm of linear.linear: prepareIndexed +
// innerGemmSortedTable + finishIndexedAs, beamivalice/sushi src/exl3/linear.zig:322-335 and
// src/exl3/expert_exl3_kernels.zig:1341-1620).
//
// MI355X layout.  A workgroup of 2 waves owns a 128-row x 128-column output tile (one Hadamard block wide, so
// the output FWHT + svh finish runs in its epilogue) over the whole k range, in k-steps of 32 (two trellis
// k-tiles).  The prepared input rows are staged through LDS; each wave owns 64 output columns (4 trellis tiles)
// and decodes its weights straight into v_mfma_f32_16x16x32_f16 B fragments: lane l = 16h + c needs column c of a
// 16-column block at k = 8h..8h+7, which is the codeword set {8q + 2p + e} (q = 0..3, e = 0..1) of chunk j = c % 8
// with p = 2*(c / 8) + h % 2 (tensorCorePerm), i.e. eight codewords from one 2n-bit run of the tile stream.
// Integer rates (n = 16K) use this reader; other rates are first decoded to a transposed f16 copy in workspace.
#include "exl3_kernels.h"
#include "exl3_lane_decode.h"
#include "exl3_tables.h"

namespace exl3 {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int GM_WAVES = 2;
constexpr int GM_THREADS = 64 * GM_WAVES;
constexpr int GM_MT = 128;    // rows per workgroup
constexpr int GM_XP = 40;     // LDS pitch (halves) of a staged x row: 32 + 8 pad

// ---- prepare: xp[g][r][:] = f16(H128(f16(x) * suh) / sqrt(128))  (prepareIndexed / PREPARE_SOURCE :852-885)
__global__ __launch_bounds__(64) void gemm_prepare_kernel(GemmArgs a) {
    const int b = blockIdx.x, r = blockIdx.y, g = blockIdx.z, lane = threadIdx.x;
    const size_t xi = ((size_t)g * a.rows + r) * a.in + (size_t)b * 128;
    const size_t si = (size_t)g * a.in + (size_t)b * 128;
    float v0, v1;
    if (a.x_dtype == DT_F16) {
        v0 = load_act<DT_F16>(a.x, xi + lane);
        v1 = load_act<DT_F16>(a.x, xi + lane + 64);
    } else if (a.x_dtype == DT_BF16) {
        v0 = f16r(load_act<DT_BF16>(a.x, xi + lane));
        v1 = f16r(load_act<DT_BF16>(a.x, xi + lane + 64));
    } else {
        v0 = f16r(load_act<DT_F32>(a.x, xi + lane));
        v1 = f16r(load_act<DT_F32>(a.x, xi + lane + 64));
    }
    v0 *= h2f(a.suh[si + lane]);
    v1 *= h2f(a.suh[si + lane + 64]);
    fwht128_wave(v0, v1, lane);
    a.xp[xi + lane] = __half_as_ushort(__float2half_rn(v0 * HAD_SCALE));
    a.xp[xi + lane + 64] = __half_as_ushort(__float2half_rn(v1 * HAD_SCALE));
}

// ---- prepare into MFMA A-fragment order: for 16-row tile rt and 32-k block kb of group g, the 1 KiB at
// xp[((g * RT + rt) * (in / 32) + kb) * 512] holds lane l = 16h + c's fragment (row 16 rt + c, k = 32 kb + 8h .. +7)
// at l * 8 halves, so one MFMA wave's load of a fragment is one contiguous 1 KiB.  RT = ceil(rows / 16); rows past
// the end of the last tile are zeros.  A workgroup (4 waves) prepares 16 rows x NB 128-blocks (two where they pair
// up): each wave loads its 4 rows of every block at once and runs their FWHTs together into an LDS tile, then every
// thread writes one 16-byte fragment per block.
template <int DT, int NB>
__global__ __launch_bounds__(256) void gemm_prepare_frag_kernel(GemmArgs a) {
    const int b0 = blockIdx.x * NB, rt = blockIdx.y, g = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int RT = (a.rows + 15) / 16;
    __shared__ __align__(16) uint16_t t[NB][16][128 + 8];
    const int m0 = rt * 16 + wave * 4;
    // every load in bounds (a row past the end reads the last row and is zeroed after), so a wave's four rows of
    // every block go out together with suh, with no branch to wait at
    float v0[NB][4], v1[NB][4], u0[NB], u1[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        const size_t si = (size_t)g * a.in + (size_t)(b0 + nb) * 128;
        u0[nb] = h2f(a.suh[si + lane]);
        u1[nb] = h2f(a.suh[si + lane + 64]);
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            const size_t xi = ((size_t)g * a.rows + min(m0 + rr, a.rows - 1)) * a.in + (size_t)(b0 + nb) * 128;
            v0[nb][rr] = load_act<DT>(a.x, xi + lane);
            v1[nb][rr] = load_act<DT>(a.x, xi + lane + 64);
        }
    }
    const float sc = fwht_relaid_sign(lane) * HAD_SCALE;
    const int c0 = fwht_relaid_col(lane, 0), c1 = fwht_relaid_col(lane, 1);
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            const bool live = m0 + rr < a.rows;
            v0[nb][rr] = live ? f16r(v0[nb][rr]) * u0[nb] : 0.f;
            v1[nb][rr] = live ? f16r(v1[nb][rr]) * u1[nb] : 0.f;
        }
        fwht128_wave_rows_relaid<4>(v0[nb], v1[nb], lane);
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            const int r = wave * 4 + rr;
            t[nb][r][c0] = __half_as_ushort(__float2half_rn(v0[nb][rr] * sc));
            t[nb][r][c1] = __half_as_ushort(__float2half_rn(v1[nb][rr] * sc));
        }
    }
    __syncthreads();
    const int kq = tid >> 6, c = lane & 15, h = lane >> 4;  // 32-k block kq of a 128-block, fragment lane (c, h)
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        const uint4 v = *reinterpret_cast<const uint4 *>(&t[nb][c][kq * 32 + 8 * h]);
        const size_t kb = (size_t)(b0 + nb) * 4 + kq;
        *reinterpret_cast<uint4 *>(a.xp + (((size_t)g * RT + rt) * (a.in / 32) + kb) * 512 + (size_t)lane * 8) = v;
    }
}

template <int DT>
static void launch_gemm_prepare_frag(const GemmArgs &a, hipStream_t s) {
    const int blocks = a.in / 128;
    const dim3 grid2((unsigned)(blocks / 2), (unsigned)((a.rows + 15) / 16), (unsigned)a.groups);
    const dim3 grid1((unsigned)blocks, (unsigned)((a.rows + 15) / 16), (unsigned)a.groups);
    if (blocks % 2 == 0) hipLaunchKernelGGL((gemm_prepare_frag_kernel<DT, 2>), grid2, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((gemm_prepare_frag_kernel<DT, 1>), grid1, dim3(256), 0, s, a);
}

// ---- dense fallback: tiles decoded to wt[g][out][in] f16 (transposed, so a B fragment is 16 contiguous bytes)
template <int FAM>
__global__ void gemm_decode_transposed_kernel(GemmArgs a, uint16_t *__restrict__ wt) {
    const int IT = a.in >> 4, OT = a.out >> 4;
    const int tile = blockIdx.x, g = blockIdx.y;
    const int tk = tile / OT, tn = tile % OT;
    const uint32_t *words =
        reinterpret_cast<const uint32_t *>(a.trellis + ((size_t)g * IT * OT + (size_t)tile) * a.n);
    const int t = 2 * threadIdx.x;
    uint32_t h = decode_pair_h2<FAM>(codeword_at(words, a.n, t), codeword_at(words, a.n, t + 1), a.k);
    const int T = t >> 3, i = t & 7, q = T & 3, j = T >> 2;
    const int row = 2 * q + ((i & 2) ? 8 : 0);
    const int col = j + ((i & 4) ? 8 : 0);
    uint32_t *dst = reinterpret_cast<uint32_t *>(wt + ((size_t)g * a.out + (size_t)tn * 16 + col) * a.in +
                                                 (size_t)tk * 16 + row);
    *dst = h;  // rows (row, row+1) of one column are adjacent in the transposed copy
}

template <int FAM, int N>
__global__ __launch_bounds__(GM_THREADS) void gemm_kernel(GemmArgs a, const uint16_t *__restrict__ wt) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int IT = a.in >> 4, OT = a.out >> 4;
    const int og = blockIdx.x, mb = blockIdx.y, g = blockIdx.z;
    const int m0 = mb * GM_MT;

    __shared__ __align__(16) uint16_t xs[GM_MT * GM_XP];
    __shared__ float outs[32][129];

    const int c = lane & 15, h = lane >> 4;
    const int kt_off = h >> 1, half = h & 1, j = c & 7, p = 2 * (c >> 3) + half;
    const DecodeK k = a.k;
    const uint16_t *tb = a.trellis + (size_t)g * IT * OT * a.n;

    f4_t acc[8][4];
#pragma unroll
    for (int rb = 0; rb < 8; rb++)
#pragma unroll
        for (int cb = 0; cb < 4; cb++) acc[rb][cb] = f4_t{0.f, 0.f, 0.f, 0.f};

    // Per-lane bit base of its eight codewords inside a tile: codeword (q, e) ends 32 + (e+1)K + q*n/2 bits past it.
    constexpr int K = N ? N / 16 : 1;
    constexpr int NW = N ? N / 2 : 1;
    constexpr int AW = N ? (32 + 2 * K + 3 * (N / 2) + 16 + 31) / 32 + 1 : 1;  // words covering the span, +1 to funnel
    const int span = 16 * (N ? N : 16);
    const int base = ((2 * j * (N ? N : 16) - 32 + 2 * p * K) % span + span) % span;
    const int wb = base >> 5, sb = base & 31;

    const int nks = IT / 2;
    for (int ks = 0; ks < nks; ks++) {
        // stage 128 rows x 32 k of the prepared input
        __syncthreads();
        {
            const int row = tid;  // GM_THREADS == GM_MT
            const int m = m0 + row;
            uint4 v0 = {0, 0, 0, 0}, v1 = v0, v2 = v0, v3 = v0;
            if (m < a.rows) {
                const uint4 *src = reinterpret_cast<const uint4 *>(a.xp + ((size_t)g * a.rows + m) * a.in + ks * 32);
                v0 = src[0];
                v1 = src[1];
                v2 = src[2];
                v3 = src[3];
            }
            uint4 *dst = reinterpret_cast<uint4 *>(&xs[row * GM_XP]);
            dst[0] = v0;
            dst[1] = v1;
            dst[2] = v2;
            dst[3] = v3;
        }
        // B fragments for this wave's 4 column blocks
        uint32_t B[4][4];
        const int tk = 2 * ks + kt_off;
#pragma unroll
        for (int cb = 0; cb < 4; cb++) {
            const int o = og * 8 + wave * 4 + cb;
            if constexpr (N != 0) {
                const uint32_t *words = reinterpret_cast<const uint32_t *>(tb + ((size_t)tk * OT + o) * N);
                uint32_t R[AW];
#pragma unroll
                for (int i = 0; i < AW; i++) R[i] = words[(wb + i) % NW];
                uint32_t A[AW - 1];
#pragma unroll
                for (int i = 0; i < AW - 1; i++) A[i] = sb ? __builtin_amdgcn_alignbit(R[i], R[i + 1], 32 - sb) : R[i];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    uint32_t cw[2];
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const int end = 32 + (e + 1) * K + q * (N / 2);
                        const int aw = (end - 1) >> 5;
                        const int sh = 32 * (aw + 1) - end;
                        cw[e] = aw == 0 ? (A[0] >> sh) : __builtin_amdgcn_alignbit(A[aw - 1], A[aw], sh);
                    }
                    B[cb][q] = decode_pair_h2<FAM>(cw[0], cw[1], k);
                }
            } else {
                const uint4 v = *reinterpret_cast<const uint4 *>(
                    wt + ((size_t)g * a.out + (size_t)o * 16 + c) * a.in + (size_t)tk * 16 + 8 * half);
                B[cb][0] = v.x;
                B[cb][1] = v.y;
                B[cb][2] = v.z;
                B[cb][3] = v.w;
            }
        }
        __syncthreads();
#pragma unroll
        for (int rb = 0; rb < 8; rb++) {
            const uint4 av = *reinterpret_cast<const uint4 *>(&xs[(rb * 16 + c) * GM_XP + 8 * h]);
            const h8_t A8 = __builtin_bit_cast(h8_t, av);
#pragma unroll
            for (int cb = 0; cb < 4; cb++) {
                const uint4 bv = {B[cb][0], B[cb][1], B[cb][2], B[cb][3]};
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A8, __builtin_bit_cast(h8_t, bv), acc[rb][cb], 0,
                                                                     0, 0);
            }
        }
    }

    // ---- epilogue: 32-row chunks through LDS, then FWHT-128 + svh per row
    const size_t sv = (size_t)g * a.out + (size_t)og * 128;
#pragma unroll
    for (int ch = 0; ch < 4; ch++) {
        __syncthreads();
#pragma unroll
        for (int rr = 0; rr < 2; rr++) {
            const int rb = ch * 2 + rr;
#pragma unroll
            for (int cb = 0; cb < 4; cb++)
#pragma unroll
                for (int i = 0; i < 4; i++) outs[rr * 16 + 4 * h + i][wave * 64 + cb * 16 + c] = acc[rb][cb][i];
        }
        __syncthreads();
        for (int r = wave; r < 32; r += GM_WAVES) {
            const int m = m0 + ch * 32 + r;
            if (m >= a.rows) break;
            float v0 = outs[r][lane], v1 = outs[r][lane + 64];
            fwht128_wave(v0, v1, lane);
            const size_t yo = ((size_t)g * a.rows + m) * a.out + (size_t)og * 128;
            const float y0 = v0 * codebook_scale<FAM>() * HAD_SCALE * h2f(a.svh[sv + lane]);
            const float y1 = v1 * codebook_scale<FAM>() * HAD_SCALE * h2f(a.svh[sv + lane + 64]);
            if (a.y_dtype == DT_F16) {
                store_act<DT_F16>(a.y, yo + lane, y0);
                store_act<DT_F16>(a.y, yo + lane + 64, y1);
            } else if (a.y_dtype == DT_BF16) {
                store_act<DT_BF16>(a.y, yo + lane, y0);
                store_act<DT_BF16>(a.y, yo + lane + 64, y1);
            } else {
                store_act<DT_F32>(a.y, yo + lane, y0);
                store_act<DT_F32>(a.y, yo + lane + 64, y1);
            }
        }
    }
}

// ---- the decode-once GEMM (integer and half-integer rates with a lane reader: n = 16, 24, 32, 40, 48, 64)
//
// A workgroup owns a 256-row x 128-column output tile (one Hadamard block wide, so the FWHT + svh finish runs in its
// epilogue) over all of k, in super-steps of 128 k (eight trellis k-tile rows), with the decode and the MFMAs on
// different waves.  The decoders (lane 8o + j: codewords 32j..32j+31 of tile o = columns j and j+8 over 16 k rows,
// the GEMV's lane decoder) fill a double-buffered LDS slab held column-major (B[col][k]), their tile words loaded a
// super-step ahead: waves 8-11, wave 8 + d decoding k-tile rows d and d + 4 of every super-step; when the live rows
// fit in 128 (MFMA waves 4-7 would have no rows), waves 4-7 decode too and each of the eight decoders takes one row
// (wave 8 + d row d, wave 4 + d row 4 + d), so a short window -- the common MoE window -- decodes on two waves per
// SIMD.  Waves 0-7 run the MFMAs: wave w owns rows 64 (w >> 1) .. + 63 and columns 64 (w & 1) .. + 63 as 4 x 4
// v_mfma_f32_16x16x32_f16 tiles per 32 k, with A fragments read from the prepared input in fragment order (one
// contiguous 1 KiB per load, a 64-k step ahead) and each 64-k step's B fragments read from the slab before its first
// MFMA.  One workgroup barrier per super-step hands the slab over: after barrier S + 1 the MFMA waves have finished
// reading slab S & 1 and the decoders have finished writing slab (S + 1) & 1.  Every weight is decoded once per
// 256-row tile.  Row groups wholly past the live rows leave before the first barrier.
constexpr int G2_MT = 256;   // rows per workgroup
constexpr int G2_BP = 72;    // LDS pitch (halves) of one ping-pong slab column: 64 k + 8 pad (16-byte aligned rows)
constexpr int G4_BP = 136;   // LDS pitch (halves) of one decode-wave-tile slab column: 128 k + 8 pad
constexpr int G4_HELP_ROWS = 128;  // live rows up to which MFMA waves 4-7 decode
constexpr int G2_EP = 129;   // epilogue staging pitch (floats)
constexpr int G4_WAVES = 12;
constexpr int G4_THREADS = 64 * G4_WAVES;

// Outputs at columns i and i + 64 of one row, in y's dtype.
__device__ __forceinline__ void store_y4(void *y, int dt, size_t i, float y0, float y1) {
    if (dt == DT_F16) {
        store_act<DT_F16>(y, i, y0);
        store_act<DT_F16>(y, i + 64, y1);
    } else if (dt == DT_BF16) {
        store_act<DT_BF16>(y, i, y0);
        store_act<DT_BF16>(y, i + 64, y1);
    } else {
        store_act<DT_F32>(y, i, y0);
        store_act<DT_F32>(y, i + 64, y1);
    }
}

// The MFMA waves' main loop of the decode-wave tile over the first NRB of the wave's four 16-row blocks (the rest of
// acc stays zero): instantiated per live-block count, so a short row group (a window of 65-85 rows leaves its second
// one or two) neither loads A nor issues MFMAs for its empty blocks, without a branch in the loop.  nks 64-k steps,
// two per super-step: 1 + nks / 2 barriers, as the decoders meet.
template <int NRB>
__device__ __forceinline__ void gemm4_mfma_loop(const uint16_t *const (&xfrag)[4], int nks, int cb0, int c, int h,
                                                uint16_t (*Bs)[128 * G4_BP], f4_t (&acc)[4][4]) {
    // A fragments in two register sets, a full step apart: set X serves even steps and set Y odd ones; each set is
    // refilled for the step after next as soon as its MFMAs have issued, so a fragment has a whole step to arrive.
    uint4 AX[4][2], AY[4][2];
    auto load_a = [&](int ks, uint4 (&A)[4][2]) __attribute__((always_inline)) {
        const int kk = min(ks, nks - 1);
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int rb = 0; rb < NRB; rb++)
                A[rb][kb] = *reinterpret_cast<const uint4 *>(xfrag[rb] + (size_t)(kk * 2 + kb) * 512);
    };
    load_a(0, AX);
    load_a(1, AY);
    __syncthreads();  // barrier 0
    auto mstep = [&](int ks, uint4 (&A)[4][2]) __attribute__((always_inline)) {
        const uint16_t *slab = Bs[(ks >> 1) & 1] + (ks & 1) * 64;  // super-step ks / 2, its k half ks & 1
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            uint4 bv[4];  // this half-step's B fragments (the A sets hold the registers a whole step of B would take)
#pragma unroll
            for (int cb = 0; cb < 4; cb++)
                bv[cb] = *reinterpret_cast<const uint4 *>(slab + ((cb0 + cb) * 16 + c) * G4_BP + kb * 32 + 8 * h);
#pragma unroll
            for (int cb = 0; cb < 4; cb++) {
                const h8_t B8 = __builtin_bit_cast(h8_t, bv[cb]);
#pragma unroll
                for (int rb = 0; rb < NRB; rb++)
                    acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, A[rb][kb]), B8,
                                                                         acc[rb][cb], 0, 0, 0);
            }
        }
        load_a(ks + 2, A);
    };
    for (int ks = 0; ks < nks; ks += 2) {  // nks is even: one super-step
        mstep(ks, AX);
        mstep(ks + 1, AY);
        __syncthreads();
    }
}

// ---- the decoders' readers: where a decoder finds k-tile row rs * i + r of its output group in its i-th load (the
// group's 8 tiles, lane 8 o + j reading chunk j of tile o; rs = 4 or 8 rows apart), and how a lane's chunk decodes.
// load(i) is called for i = 0, 1, 2, ... in order (past the last, nks - 1, it re-reads the last).
// One rate N for the bank: the row lies `kstep` halves further each load.
template <int FAM, int N>
struct RateReader {
    static constexpr int AW = LaneBits<N>::AW;
    const uint16_t *tb;  // the row in k-step 0
    size_t kstep;
    uint32_t lane_words;
    int j, nks;
    DecodeK k;
    __device__ __forceinline__ RateReader(const uint16_t *bank, int r, int rs, int OT, int og, int nks_, int lane,
                                          const DecodeK &k_)
        : tb(bank + ((size_t)r * OT + og * 8) * N), kstep((size_t)rs * OT * N),
          lane_words((uint32_t)((lane >> 3) * N) >> 1), j(lane & 7), nks(nks_), k(k_) {}
    __device__ __forceinline__ void load(int ks, uint32_t (&W)[AW]) {
        load_lane_words_u<N>(reinterpret_cast<const uint32_t *>(tb + (size_t)min(ks, nks - 1) * kstep), lane_words,
                             j, W);
    }
    __device__ __forceinline__ void decode(const uint32_t (&W)[AW], uint32_t (&w)[16]) const {
        if (k.wmask != 0xFFFFu) decode_weights<FAM, N, true>(W, k, w);
        else decode_weights<FAM, N, false>(W, k, w);
    }
};

// A per-tile-rate projection (configs[4]'s K1 / K2 mix): the row of load i is segment seg0 + i * seg_step, at the
// word offset and with the rate mask of the segment tables; lane 8 o + j's tile starts 16 o - 8 popcount(mask below o)
// words in, at TILED_NA when bit o is set.  The segment's offset and mask (scalar loads) are fetched two loads ahead,
// so a tile's vector loads never wait on them, also where a decoder issues two loads back to back.
template <int FAM>
struct TiledReader {
    static constexpr int AW = 4;  // the lane's three words and its tile's rate flag
    const uint32_t *words;        // the projection's whole trellis
    const uint32_t *seg_off;
    const uint8_t *seg_k1;
    size_t seg0, seg_step;
    int o, j, nks;
    DecodeK ka, kb;
    uint32_t n_off, n_m, f_off, f_m;  // offset and mask of the next load and of the one after it
    __device__ __forceinline__ TiledReader(const uint16_t *trellis, const uint32_t *off, const uint8_t *k1, int e,
                                           int r, int rs, int IT, int OT, int og, int nks_, int lane,
                                           const DecodeK &ka_, const DecodeK &kb_)
        : words(reinterpret_cast<const uint32_t *>(trellis)), seg_off(off), seg_k1(k1),
          seg0(((size_t)e * IT + r) * (size_t)(OT >> 3) + og), seg_step((size_t)rs * (OT >> 3)), o(lane >> 3),
          j(lane & 7), nks(nks_), ka(ka_), kb(kb_) {
        fetch(0, n_off, n_m);
        fetch(1, f_off, f_m);
    }
    __device__ __forceinline__ void fetch(int ks, uint32_t &off, uint32_t &m) const {
        const size_t seg = seg0 + (size_t)min(ks, nks - 1) * seg_step;
        m = seg_mask(seg_k1, seg);
        off = seg_off[seg];
    }
    __device__ __forceinline__ void load(int ks, uint32_t (&W)[AW]) {
        const uint32_t m = n_m, off = n_off;
        const bool k1 = ((m >> o) & 1u) != 0;
        const uint32_t lw = 16u * (uint32_t)o - 8u * (uint32_t)__builtin_popcount(m & ((1u << o) - 1u));
        uint32_t A[3];
        load_lane_words_tiled(words + off, lw, j, k1, A);
        W[0] = A[0];
        W[1] = A[1];
        W[2] = A[2];
        W[3] = k1 ? 1u : 0u;
        n_off = f_off;
        n_m = f_m;
        fetch(ks + 2, f_off, f_m);
    }
    __device__ __forceinline__ void decode(const uint32_t (&W)[AW], uint32_t (&w)[16]) const {
        const uint32_t A[3] = {W[0], W[1], W[2]};
        const bool k1 = W[3] != 0;
        const DecodeK kl = tiled_constants(k1, ka, kb);
        if (kb.wmask != 0xFFFFu) decode_weights_tiled<FAM, true>(A, k1, kl, w);
        else decode_weights_tiled<FAM, false>(A, k1, kl, w);
    }
};

// The decoders of the decode-wave tile, D of them (4: waves 8-11; 8: waves 8-11 and 4-7), decoder d decoding rows
// d + 4 t (t < 8 / D) of each super-step into the slab the MFMA waves read after the super-step's barrier, the words
// of the next super-step in flight.  The reader takes row d every 8 / D loads apart (4 rows apart for D = 4, 8 for
// D = 8), nsup * 8 / D loads in all.  1 + nsup barriers.
template <int FAM, int D, class R>
__device__ __forceinline__ void gemm4_decode_waves(R &rd, int nsup, int d, int lane, uint16_t (*Bs)[128 * G4_BP]) {
    static_assert(D == 4 || D == 8, "four or eight decoders");
    constexpr int T = 8 / D;  // rows per decoder per super-step
    const int o = lane >> 3, j = lane & 7;
    auto decode_store = [&](const uint32_t (&W)[R::AW], uint16_t *slab, int row) __attribute__((always_inline)) {
        uint32_t w[16];
        rd.decode(W, w);
        uint16_t *cj = slab + (o * 16 + j) * G4_BP + row * 16;
        uint16_t *cj8 = cj + 8 * G4_BP;
        *reinterpret_cast<uint4 *>(cj) = uint4{w[0], w[4], w[8], w[12]};
        *reinterpret_cast<uint4 *>(cj + 8) = uint4{w[1], w[5], w[9], w[13]};
        *reinterpret_cast<uint4 *>(cj8) = uint4{w[2], w[6], w[10], w[14]};
        *reinterpret_cast<uint4 *>(cj8 + 8) = uint4{w[3], w[7], w[11], w[15]};
    };
    uint32_t P[T][R::AW], Q[T][R::AW];
#pragma unroll
    for (int t = 0; t < T; t++) rd.load(t, P[t]);
#pragma unroll
    for (int t = 0; t < T; t++) rd.load(T + t, Q[t]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < T; t++) decode_store(P[t], Bs[0], d + 4 * t);
    __syncthreads();  // barrier 0: slab 0 is ready
    // super-step S: the words of S + 2 into the set just decoded, S + 1's rows into slab (S + 1) & 1
    auto sstep = [&](int S, const uint32_t (&C)[T][R::AW], uint32_t (&Nx)[T][R::AW]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < T; t++) rd.load(T * (S + 2) + t, Nx[t]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < T; t++) decode_store(C[t], Bs[(S + 1) & 1], d + 4 * t);
        __syncthreads();
    };
    int S = 0;
    for (; S + 1 < nsup; S += 2) {
        sstep(S, Q, P);
        sstep(S + 1, P, Q);
    }
    if (S < nsup) sstep(S, Q, P);
}

// The MFMA waves (waves 0-7) of one workgroup's 256-row x 128-column output tile: prepared rows in fragment tiles from
// xfrag0 (row tile rt at xfrag0 + rt * (in / 32) * 512), of which the first `rows` (<= 256) are live.  The epilogue
// hands the raw inner products of rows m .. m + 3 to emit(m, live, v0[4], v1[4], lane, rid) (columns lane and
// lane + 64 of the group, m the row within the tile, the first `live` of them live); the caller applies the output
// transform (four rows at a time) or stores the raw values.  With row_ids, lane l of rid holds row_ids[m0 + l] for the
// wave's row group m0 .. m0 + 63 (loaded before the main loop, so the epilogue finds each row's id with a lane read
// instead of a memory round trip per row); without, rid is 0.
template <class Emit>
__device__ __forceinline__ void gemm4_mfma_waves(int in, const uint16_t *__restrict__ xfrag0, int rows,
                                                 const uint32_t *__restrict__ row_ids, uint16_t (*Bs)[128 * G4_BP],
                                                 Emit emit) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nks = (in >> 4) / 4;  // even: in is a multiple of 128
    // A row group wholly past the live rows (a short window or row tail) has nothing to compute and leaves at once;
    // like the decode waves' exit, an ended wave no longer counts at the barriers.
    const int m0 = (wave >> 1) * 64, cb0 = (wave & 1) * 4;
    if (m0 >= rows) return;
    const uint32_t rid = row_ids ? row_ids[min(m0 + lane, rows - 1)] : 0u;
    const int c = lane & 15, h = lane >> 4;
    const int RT = (rows + 15) / 16;
    const uint16_t *xfrag[4];
#pragma unroll
    for (int rb = 0; rb < 4; rb++) {
        const int rt = min(m0 / 16 + rb, RT - 1);
        xfrag[rb] = xfrag0 + (size_t)rt * (size_t)(in / 32) * 512 + (size_t)lane * 8;
    }
    f4_t acc[4][4];
#pragma unroll
    for (int rb = 0; rb < 4; rb++)
#pragma unroll
        for (int cb = 0; cb < 4; cb++) acc[rb][cb] = f4_t{0.f, 0.f, 0.f, 0.f};
    switch (min(4, RT - m0 / 16)) {  // the wave's live 16-row blocks
    case 1: gemm4_mfma_loop<1>(xfrag, nks, cb0, c, h, Bs, acc); break;
    case 2: gemm4_mfma_loop<2>(xfrag, nks, cb0, c, h, Bs, acc); break;
    case 3: gemm4_mfma_loop<3>(xfrag, nks, cb0, c, h, Bs, acc); break;
    default: gemm4_mfma_loop<4>(xfrag, nks, cb0, c, h, Bs, acc); break;
    }

    // ---- epilogue (the decode waves have left, so the barriers below join the live MFMA waves): per 16-row block, the
    // two waves of a row group stage their column halves side by side in LDS, then each hands 8 of the rows on.
    float *ep = reinterpret_cast<float *>(&Bs[0][0]) + (wave >> 1) * 16 * G2_EP;
#pragma unroll
    for (int rb = 0; rb < 4; rb++) {
#pragma unroll
        for (int cb = 0; cb < 4; cb++)
#pragma unroll
            for (int i = 0; i < 4; i++) ep[(4 * h + i) * G2_EP + (cb0 + cb) * 16 + c] = acc[rb][cb][i];
        __syncthreads();
#pragma unroll
        for (int r4 = 0; r4 < 8; r4 += 4) {
            const int r = (wave & 1) * 8 + r4, m = m0 + rb * 16 + r;
            if (m >= rows) break;
            float v0[4], v1[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v0[i] = ep[(r + i) * G2_EP + lane];
                v1[i] = ep[(r + i) * G2_EP + lane + 64];
            }
            emit(m, min(4, rows - m), v0, v1, lane, rid);
        }
        __syncthreads();
    }
}

// This wave's decoder index in the decode-wave tile, or -1 for an MFMA wave: waves 8-11 are decoders 0-3; with the
// live rows within G4_HELP_ROWS, waves 4-7 (whose row groups are empty) are decoders 4-7.
__device__ __forceinline__ int gemm4_decoder(int wave, int rows) {
    if (wave >= 8) return wave - 8;
    return (rows <= G4_HELP_ROWS && wave >= 4) ? wave : -1;
}

// Decoder d over the reader mk(r, rs, loads) makes (row r, rows rs apart, `loads` loads): eight decoders when `help`
// (the live rows within G4_HELP_ROWS), else four.
template <int FAM, class MakeReader>
__device__ __forceinline__ void gemm4_decode_role(bool help, int d, int nsup, int lane, uint16_t (*Bs)[128 * G4_BP],
                                                  MakeReader mk) {
    if (help) {
        auto rd = mk(d, 8, nsup);
        gemm4_decode_waves<FAM, 8>(rd, nsup, d, lane, Bs);
    } else {
        auto rd = mk(d, 4, 2 * nsup);
        gemm4_decode_waves<FAM, 4>(rd, nsup, d, lane, Bs);
    }
}

// One workgroup's 256-row x 128-column output tile of output group og of a bank at one rate N whose tiles start at
// `bank` ([in/16][out/16][N]): the decoders (gemm4_decoder) decode, the other waves multiply (gemm4_mfma_waves, whose
// `emit` receives the raw inner products).
template <int FAM, int N, class Emit>
__device__ __forceinline__ void gemm4_tile(int in, int out, int og, const uint16_t *__restrict__ bank,
                                           const uint16_t *__restrict__ xfrag0, int rows, const uint32_t *row_ids,
                                           const DecodeK &k, uint16_t (*Bs)[128 * G4_BP], Emit emit) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int d = gemm4_decoder(wave, rows);
    if (d >= 0) {
        gemm4_decode_role<FAM>(rows <= G4_HELP_ROWS, d, in >> 7, lane, Bs, [&](int r, int rs, int loads) {
            return RateReader<FAM, N>(bank, r, rs, out >> 4, og, loads, lane, k);
        });
        return;
    }
    gemm4_mfma_waves(in, xfrag0, rows, row_ids, Bs, emit);
}

template <int FAM, int N>
__global__ __launch_bounds__(G4_THREADS) void gemm4_kernel(GemmArgs a) {
    const int IT = a.in >> 4, OT = a.out >> 4;
    const int nog = a.out / 128, nm = (a.rows + G2_MT - 1) / G2_MT;
    const int L = blockIdx.x;
    int og, mt;
    if (nm <= 8 && 8 % nm == 0 && nog % (8 / nm) == 0) {
        const int xcd = L & 7, per = 8 / nm;
        mt = xcd / per;
        og = (L >> 3) * per + xcd % per;
    } else {
        og = L % nog;
        mt = L / nog;
    }
    const int g = blockIdx.z;
    __shared__ __align__(16) uint16_t Bs[2][128 * G4_BP];
    const int RT = (a.rows + 15) / 16;
    const uint16_t *xfrag0 = a.xp + ((size_t)g * RT + (size_t)mt * (G2_MT / 16)) * (size_t)(a.in / 32) * 512;
    const size_t sv = (size_t)g * a.out + (size_t)og * 128;
    const int lane = threadIdx.x & 63;
    const float s0 = h2f(a.svh[sv + lane]), s1 = h2f(a.svh[sv + lane + 64]);
    gemm4_tile<FAM, N>(a.in, a.out, og, a.trellis + (size_t)g * IT * OT * N, xfrag0, min(G2_MT, a.rows - mt * G2_MT),
                       nullptr, a.k, Bs,
                       [&](int m, int live, float (&v0)[4], float (&v1)[4], int ln, uint32_t)
                           __attribute__((always_inline)) {
                           fwht128_wave_rows<4>(v0, v1, ln);
                           for (int i = 0; i < live; i++) {
                               const size_t yo = ((size_t)g * a.rows + mt * G2_MT + m + i) * a.out + (size_t)og * 128;
                               store_y4(a.y, a.y_dtype, yo + ln, v0[i] * codebook_scale<FAM>() * HAD_SCALE * s0,
                                        v1[i] * codebook_scale<FAM>() * HAD_SCALE * s1);
                           }
                       });
}

// ---- the ping-pong GEMM (hash-product families at the lane-reader rates)
//
// A workgroup of 8 waves owns an MT-row x 128-column output tile (MT = 256 or 512; one Hadamard block wide, so the
// FWHT + svh finish runs in its epilogue) over all of k, in k-steps of 64 (four trellis k-tiles).  Every wave owns
// RW = MT / 8 rows x all 128 columns (RW / 16 x 8 v_mfma_f32_16x16x32_f16 tiles) with its A fragments in registers, so
// each prepared row is loaded once per workgroup, and every wave also decodes: waves r and r + 4 decode the two column
// halves of k-tile row r of step s + 2 (the GEMV's lane decoder, half a chunk each) into a triple-buffered LDS slab.
// Waves r and r + 4 share a SIMD: wave r runs its step's MFMAs first and then decodes, wave r + 4 decodes first, so
// on every SIMD one wave feeds the matrix core while the other decodes on the VALU (a decode wave beside MFMA waves
// leaves their rate untouched).  One barrier per step: the slab read in step s was written in step s - 2 and the one
// written in step s was last read in step s - 1, each on the other side of a barrier.  The trellis words are loaded
// a step before their decode, the A fragments of step s + 1 as soon as step s's MFMAs of that half have issued.
// Every weight is decoded once per MT rows (twice per 1024 rows at MT = 512, against four times for the 256-row tile).
//
// KS = 2 splits k in halves over twice the workgroups (a grid of few 512-row tiles then fills the chip and still
// decodes every weight once per 512 rows).  Each half finishes half of every wave's rows: it writes the raw
// accumulators of the other half's rows through to memory, arrives at the tile's counter, adds the other half's
// partial of its own rows (a sum of two, so independent of which came first) and runs their epilogue.  The first to
// arrive waits, bounded, for the second; past the wait it hands the whole tile over.
constexpr int G5_WAVES = 8;
constexpr int G5_THREADS = 64 * G5_WAVES;
constexpr int G5_SLAB = 128 * G2_BP;                                        // halves per slab
constexpr int G5_SP = 144;  // epilogue stage pitch (halves): the four 16-lane groups' rows land 8 banks apart
constexpr int G5_LDS = (3 * G5_SLAB * 2 > G5_WAVES * 16 * G5_SP * 2) ? 3 * G5_SLAB * 2 : G5_WAVES * 16 * G5_SP * 2;

template <int FAM, int N, int MT, int KS>
__global__ __launch_bounds__(G5_THREADS, 1) void gemm5_kernel(GemmArgs a) {
    static_assert(FAM != FAM_PAIR && FAM != FAM_MUL1, "hash-product families");
    static_assert(KS == 1 || KS == 2, "whole k or halves");
    constexpr int RW = MT / G5_WAVES;  // rows per wave
    constexpr int RB = RW / 16;        // row blocks per wave
    constexpr int AW = LaneBits<N>::AW;
    const int IT = a.in >> 4, OT = a.out >> 4;
    const int nog = a.out / 128, nm = (a.rows + MT - 1) / MT;
    // split ks of a tile: the grid's second half (its tile index repeats the first half's, so the same XCD map)
    const int ks = KS == 1 ? 0 : (int)blockIdx.x / (nm * nog);
    const int L = KS == 1 ? (int)blockIdx.x : (int)blockIdx.x - ks * nm * nog;
    int og, mt;
    if (nm <= 8 && 8 % nm == 0 && nog % (8 / nm) == 0) {  // a row tile's workgroups share an XCD (its A rows in one L2)
        const int xcd = L & 7, per = 8 / nm;
        mt = xcd / per;
        og = (L >> 3) * per + xcd % per;
    } else {
        og = L % nog;
        mt = L / nog;
    }
    const int g = blockIdx.z;
    __shared__ __align__(16) uint8_t lds[G5_LDS];
    uint16_t *slabs = reinterpret_cast<uint16_t *>(lds);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 15, h = lane >> 4;
    const int RT = (a.rows + 15) / 16;
    const int nks = IT / 4 / KS;   // this split's k-steps (IT is a multiple of 8: whole 128-blocks)
    const int s0g = ks * nks;      // its first k-step
    const DecodeK k = a.k;
    const bool masked = k.wmask != 0xFFFFu;

    // ---- decode role: column half H of k-tile row r of each step
    const int r = wave & 3, H = wave >> 2;
    const int o = lane >> 3, j = lane & 7;
    const size_t kstep = (size_t)4 * OT * N;  // halves from one k-step's row r to the next
    const uint16_t *tb = a.trellis + (size_t)g * IT * OT * N + ((size_t)r * OT + og * 8) * N + (size_t)s0g * kstep;
    const uint32_t lane_words = (uint32_t)(o * N) >> 1;
    auto load_words = [&](int s, uint32_t (&W)[AW]) __attribute__((always_inline)) {
        load_lane_words_u<N>(reinterpret_cast<const uint32_t *>(tb + (size_t)min(s, nks - 1) * kstep), lane_words, j,
                             W);
    };
    // the slab column this lane writes (rows r * 16 .. + 15 of the step's 64 k)
    const int col = o * 16 + j + 8 * H;
    auto decode_into = [&](int s, const uint32_t (&W)[AW]) __attribute__((always_inline)) {
        uint32_t w[8];
        if (H) {
            if (masked) decode_weights_half<FAM, N, true, 1>(W, k, w);
            else decode_weights_half<FAM, N, false, 1>(W, k, w);
        } else {
            if (masked) decode_weights_half<FAM, N, true, 0>(W, k, w);
            else decode_weights_half<FAM, N, false, 0>(W, k, w);
        }
        uint16_t *dst = slabs + (size_t)(s % 3) * G5_SLAB + col * G2_BP + r * 16;
        *reinterpret_cast<uint4 *>(dst) = uint4{w[0], w[2], w[4], w[6]};
        *reinterpret_cast<uint4 *>(dst + 8) = uint4{w[1], w[3], w[5], w[7]};
    };

    // ---- MFMA role: rows m0 .. m0 + RW - 1 of the tile, all 128 columns
    const int m0 = mt * MT + wave * RW;
    // fragment (row tile rt, 32-k block kk) of group g: bytes ((rt in/32 + kk) 1024 + 16 lane) of the group's
    // prepared rows, read through a buffer resource (uniform base and offset in scalar registers, one lane offset)
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    const size_t xp_group = (size_t)RT * (size_t)(a.in / 32) * 512;  // halves per group
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(a.xp + (size_t)g * xp_group), (short)0, (int)(xp_group * 2), 0x00020000);
    const uint32_t a_lane = (uint32_t)lane * 16u;
    f4_t acc[RB][8];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int cb = 0; cb < 8; cb++) acc[rb][cb] = f4_t{0.f, 0.f, 0.f, 0.f};
    uint4 A[2][RB];
    auto load_a = [&](int s, int kb) __attribute__((always_inline)) {
        const int kk = (s0g + min(s, nks - 1)) * 2 + kb;
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            const int rt = min(m0 / 16 + rb, RT - 1);
            const int soff = (rt * (a.in / 32) + kk) * 1024;
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(xrs, a_lane, soff, 0);
            A[kb][rb] = uint4{v.x, v.y, v.z, v.w};
        }
    };
    // B fragment f = kb * 8 + cb of step s; the first PD of a step are read before it starts (at the end of the
    // wave's previous decode phase), the rest PD fragments ahead of their MFMAs
    constexpr int PD = 3;
    auto frag = [&](int s, int f) __attribute__((always_inline)) {
        const uint16_t *bp = slabs + (size_t)(s % 3) * G5_SLAB + c * G2_BP + 8 * h;
        return *reinterpret_cast<const uint4 *>(bp + (f & 7) * 16 * G2_BP + (f >> 3) * 32);
    };
    uint4 bpre[PD];
    auto read_first = [&](int s) __attribute__((always_inline)) {
#pragma unroll
        for (int f = 0; f < PD; f++) bpre[f] = frag(s, f);
    };
    auto mfma_phase = [&](int s) __attribute__((always_inline)) {
        uint4 bq[16];
#pragma unroll
        for (int f = 0; f < PD; f++) bq[f] = bpre[f];
#pragma unroll
        for (int f = 0; f < 16; f++) {
            if (f + PD < 16) bq[f + PD] = frag(s, f + PD);
            const int kb = f >> 3, cb = f & 7;
            const h8_t B8 = __builtin_bit_cast(h8_t, bq[f]);
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, A[kb][rb]), B8,
                                                                     acc[rb][cb], 0, 0, 0);
            if (f == 7) load_a(s + 1, 0);
            if (f == 15) load_a(s + 1, 1);
            if (f & 1) __builtin_amdgcn_sched_barrier(0);  // keep the B reads a few fragments ahead, not all at once
        }
    };

    // ---- the step loop.  Every wave runs the same order -- step s's MFMAs, then a decode -- and waves differ only in
    // where their barrier falls: waves 0-3 (H = 0) decode step s + 2 before barrier s, waves 4-7 (H = 1) decode step
    // s + 3 after it.  So between two barriers a SIMD's H = 0 wave runs its MFMAs and then decodes while its H = 1
    // wave decodes and then runs its MFMAs.  Slab t % 3 is read in step t after barrier t - 1; its H = 0 half is
    // written before barrier t - 2, its H = 1 half after barrier t - 3; both after the reads of step t - 3, which end
    // before barrier t - 3.  The words of step s + 2 + H sit in ring slot s % 3, loaded in the step before.
    uint32_t W0[AW], W1[AW], W2[AW];
    load_a(0, 0);
    load_a(0, 1);
    {
        uint32_t P0[AW], P1[AW];
        load_words(0, P0);
        load_words(1, P1);
        load_words(2, W2);
        load_words(2 + H, W0);
        decode_into(0, P0);
        decode_into(1, P1);
        if (H) decode_into(2, W2);
    }
    __syncthreads();
    read_first(0);
    auto step = [&](int s, const uint32_t (&Wd)[AW], uint32_t (&Wl)[AW]) __attribute__((always_inline)) {
        mfma_phase(s);
        __builtin_amdgcn_sched_barrier(0);
        if (H) __syncthreads();
        if (s + 2 + H < nks) decode_into(s + 2 + H, Wd);
        if (s + 3 + H < nks) load_words(s + 3 + H, Wl);
        if (s + 1 < nks) read_first(s + 1);  // slab s + 1 was complete before barrier s - 1
        __builtin_amdgcn_sched_barrier(0);
        if (!H) __syncthreads();
    };
    for (int s = 0; s < nks; s += 3) {
        step(s, W0, W1);
        if (s + 1 < nks) step(s + 1, W1, W2);
        if (s + 2 < nks) step(s + 2, W2, W0);
    }
    __syncthreads();  // the H = 1 waves' last decode (none: s + 3 >= nks) and every slab read are behind this

    // Row blocks this workgroup finishes: all of them, or with k in halves the half's own (set below).
    bool fin_lo = true, fin_hi = true;  // row blocks 0 .. RB/2 - 1 and RB/2 .. RB - 1 of every wave
    if constexpr (KS == 2) {
        // partial of split ks: [tile][ks][wave][rb][cb] blocks of 64 lanes x 4 floats, one 1 KiB store each.  Half ks
        // finishes row blocks RB/2 ks .. RB/2 ks + RB/2 - 1 of every wave: it writes the partner's row blocks of its
        // partial, arrives, and adds the partner's partial of its own.  The first to arrive waits (at most a.kwait
        // ticks) for the second; past the wait it writes its own row blocks too and hands the whole tile over, and
        // the second finishes every row.  Each output is the same sum of two either way.
        static_assert(RB % 2 == 0, "halves of the row blocks");
        constexpr int RH = RB / 2;
        const size_t tile = ((size_t)g * nm + mt) * nog + og;
        const size_t wave_f = (size_t)RB * 8 * 256;  // floats per wave
        float *mine = a.kpart + ((tile * 2 + ks) * G5_WAVES + wave) * wave_f;
        const float *other = a.kpart + ((tile * 2 + (ks ^ 1)) * G5_WAVES + wave) * wave_f;
        const __amdgpu_buffer_rsrc_t mr = __builtin_amdgcn_make_buffer_rsrc(mine, (short)0, (int)(wave_f * 4), 0x00020000);
        const __amdgpu_buffer_rsrc_t orr =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(other), (short)0, (int)(wave_f * 4), 0x00020000);
        // sc0 sc1: the stores go through to memory and the loads bypass the caches (the halves may sit on two XCDs)
        constexpr int SYS = 1 | 16;
        auto store_rows = [&](int half) __attribute__((always_inline)) {
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
                if (rb / RH == half) {
#pragma unroll
                    for (int cb = 0; cb < 8; cb++)
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, acc[rb][cb]), mr, a_lane,
                                                               (rb * 8 + cb) * 1024, SYS);
                }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // acknowledged before the counter moves
        };
        constexpr uint32_t HANDED = 0x40000000u;  // the first half gave its whole tile to the second
        store_rows(ks ^ 1);
        __syncthreads();
        __shared__ uint32_t arrived;
        uint32_t *ctr = a.kctr + tile * COUNTER_STRIDE;
        if (tid == 0) arrived = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const uint32_t st = arrived;
        __syncthreads();  // every wave has read `arrived` before wave 0 reuses it
        bool all = false;
        if (st == 0) {
            // first: wave 0 polls for the second's arrival, at most kwait ticks, so the wait always ends
            if (tid == 0) {
                const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                uint32_t v = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                while (v < 2u && __builtin_amdgcn_s_memrealtime() - t0 < (uint64_t)a.kwait) {
                    __builtin_amdgcn_s_sleep(2);
                    v = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                arrived = v;
            }
            __syncthreads();
            if (arrived < 2u) {
                // the second has not arrived: write this half's own row blocks, then hand the tile over unless the
                // second arrived meanwhile (then it has written this half's rows and finishes its own as usual)
                store_rows(ks);
                __syncthreads();
                if (tid == 0) {
                    uint32_t expect = 1u;
                    __hip_atomic_compare_exchange_strong(ctr, &expect, HANDED, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
                    arrived = expect;  // 1: handed over; 2: the second arrived first
                }
                __syncthreads();
                if (arrived == 1u) return;
            }
            if (tid == 0) *ctr = 0u;  // both arrived and the second never reads it again; the next launch reads it
                                      // after the kernel boundary
        } else if (st >= HANDED) {
            all = true;  // the first handed over the whole tile
            if (tid == 0) *ctr = 0u;
        }
        fin_lo = all || ks == 0;
        fin_hi = all || ks == 1;
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
            if (rb < RH ? fin_lo : fin_hi) {
#pragma unroll
                for (int cb = 0; cb < 8; cb++) {
                    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(orr, a_lane, (rb * 8 + cb) * 1024, SYS);
                    acc[rb][cb] += __builtin_bit_cast(f4_t, v);
                }
            }
    }

    // ---- epilogue: the output transform straight from the accumulators.  Column cb * 16 + c of the tile sits in
    // acc[.][cb] of lane c + 16 h (rows 4 h .. 4 h + 3), and H128 = H8 (over cb) x H16 (over c): the stages of bits
    // 6, 5, 4 are butterflies between a lane's own registers, those of bits 3 .. 0 the DPP stages within each 16-lane
    // row.  These are fwht128_wave's stages in its order with its sums, so the outputs equal the row-wise transform's
    // bit for bit, without staging rows through LDS or running one transform per row.
    const size_t sv = (size_t)g * a.out + (size_t)og * 128;
    float svc[8];
#pragma unroll
    for (int cb = 0; cb < 8; cb++) svc[cb] = h2f(a.svh[sv + cb * 16 + c]);
    const float sg8 = lane_sign<8>(lane), sg4 = lane_sign<4>(lane), sg2 = lane_sign<2>(lane), sg1 = lane_sign<1>(lane);
    // 16-bit outputs go out through a per-wave LDS stage of 16 rows (the slab ring is free past the last barrier):
    // one 16-byte store covers four rows' eighths, against a 2-byte store per lane from the lane layout
    // (and so does any y not 16-byte aligned: then every output goes out straight from the lane layout)
    const bool wide = a.y_dtype == DT_F32 || (reinterpret_cast<uintptr_t>(a.y) & 15) != 0, bf16 = a.y_dtype == DT_BF16;
    uint16_t *stage = reinterpret_cast<uint16_t *>(lds) + wave * 16 * G5_SP;
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        if (!(rb < RB / 2 ? fin_lo : fin_hi)) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float v[8];
#pragma unroll
            for (int cb = 0; cb < 8; cb++) v[cb] = acc[rb][cb][i];
#pragma unroll
            for (int hb = 4; hb >= 1; hb >>= 1)
#pragma unroll
                for (int cb = 0; cb < 8; cb++)
                    if (!(cb & hb)) {
                        const float lo = v[cb], hi = v[cb | hb];
                        v[cb] = lo + hi;
                        v[cb | hb] = lo - hi;
                    }
#pragma unroll
            for (int cb = 0; cb < 8; cb += 2) fwht_stage<8>(v[cb], v[cb + 1], sg8);
#pragma unroll
            for (int cb = 0; cb < 8; cb += 2) fwht_stage<4>(v[cb], v[cb + 1], sg4);
#pragma unroll
            for (int cb = 0; cb < 8; cb += 2) fwht_stage<2>(v[cb], v[cb + 1], sg2);
#pragma unroll
            for (int cb = 0; cb < 8; cb += 2) fwht_stage<1>(v[cb], v[cb + 1], sg1);
            if (wide) {
                const int m = m0 + rb * 16 + 4 * h + i;
                if (m < a.rows) {
                    const size_t yo = ((size_t)g * a.rows + m) * a.out + (size_t)og * 128 + c;
#pragma unroll
                    for (int cb = 0; cb < 8; cb++) {
                        const float y = v[cb] * codebook_scale<FAM>() * HAD_SCALE * svc[cb];
                        if (a.y_dtype == DT_F16) store_act<DT_F16>(a.y, yo + cb * 16, y);
                        else if (bf16) store_act<DT_BF16>(a.y, yo + cb * 16, y);
                        else store_act<DT_F32>(a.y, yo + cb * 16, y);
                    }
                }
            } else {
#pragma unroll
                for (int cb = 0; cb < 8; cb++) {
                    // y is rounded to f32 first, as every other output path rounds it (the empty asm keeps the
                    // product from fusing into the 16-bit conversion, which would round once and differ at ties)
                    float y = v[cb] * codebook_scale<FAM>() * HAD_SCALE * svc[cb];
                    asm("" : "+v"(y));
                    stage[(4 * h + i) * G5_SP + cb * 16 + c] =
                        bf16 ? __bfloat16_as_ushort(__float2bfloat16(y)) : __half_as_ushort(__float2half_rn(y));
                }
            }
        }
        if (!wide) {  // the wave's 16 rows, row-major in its LDS region: four rows per 16-byte store
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int rr = 4 * q + (lane >> 4), m = m0 + rb * 16 + rr;
                const uint4 val = *reinterpret_cast<const uint4 *>(stage + rr * G5_SP + (lane & 15) * 8);
                if (m < a.rows)
                    *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(a.y) + ((size_t)g * a.rows + m) * a.out +
                                               (size_t)og * 128 + (lane & 15) * 8) = val;
            }
        }
    }
}

// Expert index of a window (routed ones clamped below `experts`; with a shared expert, `experts` is it) and the token
// row of a slot (routed slot s is token s / topk, shared slot nslots + r is token r).
__device__ __forceinline__ int moe_expert(const MoeGemmArgs &a, uint32_t e) {
    return (int)min(e, (uint32_t)(a.experts - 1 + a.sh));
}
__device__ __forceinline__ uint32_t moe_token(const MoeGemmArgs &a, uint32_t slot) {
    return slot < (uint32_t)a.nslots ? slot / (uint32_t)a.topk : slot - (uint32_t)a.nslots;
}

// ---- the routed GEMM arm: workgroup (og, window w, projection p) runs the tile of window w's rows against its
// expert's bank and writes the raw inner products to planes[p][slot][out] (the mid / the reduce applies the output
// transform).  Windows past the count exit before any barrier.  Workgroups go out to the XCDs in turn (L & 7), so
// the out / 128 column groups of one window are numbered to land on one XCD one after another: they read the same
// prepared rows, which then come from that XCD's L2 after the first (numbered by the window, each group would pull
// them through its own XCD's L2).
// N > 0: a uniform bank at rate N.  N == -1: a ragged bank (`rate_groups.moePrefill`, rate_groups.zig:2039-2075):
// each workgroup reads its expert's rate and tile offset from the meta table and its decode waves take that rate's
// reader (one launch for every rate group; the MFMA waves are the same for all).  N == N_TILED: a per-tile-rate bank,
// the decode waves reading each k-step's segment offset and rate mask.  Either way a fused shared expert (expert
// `experts`) decodes at its own uniform rate sh_n.
template <int FAM>
__device__ __forceinline__ DecodeK rate_decode(const DecodeK &base, int table, int n) {
    DecodeK k = base;
    if constexpr (FAM == FAM_HASH || FAM == FAM_PAIR) table_row(table, n, k.mult, k.mask0, k.mask1, k.rot);
    return k;
}

// Decoder d at a rate known only at run time (a lane-reader rate; any other leaves the slab undecoded, which the
// host rules out).
template <int FAM>
__device__ __forceinline__ void gemm4_decode_waves_at(int n, const uint16_t *bank, int OT, int og, int nsup, int d,
                                                      bool help, int lane, const DecodeK &k,
                                                      uint16_t (*Bs)[128 * G4_BP]) {
    switch (n) {
#define EXL3_RATE_CASE(NN)                                                                                             \
    case NN:                                                                                                           \
        gemm4_decode_role<FAM>(help, d, nsup, lane, Bs, [&](int r, int rs, int loads) {                                \
            return RateReader<FAM, NN>(bank, r, rs, OT, og, loads, lane, k);                                           \
        });                                                                                                            \
        break;
        EXL3_RATE_CASE(16)
        EXL3_RATE_CASE(24)
        EXL3_RATE_CASE(32)
        EXL3_RATE_CASE(40)
        EXL3_RATE_CASE(48)
        EXL3_RATE_CASE(64)
#undef EXL3_RATE_CASE
    default: break;
    }
}

template <int FAM, int N>
__global__ __launch_bounds__(G4_THREADS) void moe_gemm4_kernel(MoeGemmArgs a) {
    const int nog = a.out / 128, L = blockIdx.x, q = L >> 3;
    const int og = q % nog, w = (q / nog) * 8 + (L & 7), p = blockIdx.y;
    if ((uint32_t)w >= *a.win.win_count) return;
    const int IT = a.in >> 4, OT = a.out >> 4;
    const int e = moe_expert(a, a.win.win_expert[w]);
    const int rows = (int)min(a.win.win_rows[w], (uint32_t)G2_MT);
    const uint32_t *slots = a.win.sorted + a.win.win_start[w];
    __shared__ __align__(16) uint16_t Bs[2][128 * G4_BP];
    const uint16_t *xfrag0 = a.xp[p] + (size_t)a.win.win_tile0[w] * (size_t)(a.in / 32) * 512;
    float *planes = a.planes[p];
    auto emit = [&](int m, int live, float (&v0)[4], float (&v1)[4], int ln, uint32_t rid)
                    __attribute__((always_inline)) {
        for (int i = 0; i < live; i++) {  // rid: the slot of row (m & ~63) + lane
            const uint32_t slot = (uint32_t)__builtin_amdgcn_readlane((int)rid, (m & 63) + i);
            float *row = planes + (size_t)slot * a.out + (size_t)og * 128;
            row[ln] = v0[i] * codebook_scale<FAM>();
            row[ln + 64] = v1[i] * codebook_scale<FAM>();
        }
    };
    if constexpr (N > 0) {
        const uint16_t *bank = e < a.experts ? a.trellis[p] + (size_t)e * IT * OT * N : a.sh_trellis[p];
        gemm4_tile<FAM, N>(a.in, a.out, og, bank, xfrag0, rows, slots, a.k, Bs, emit);
    } else {
        const int lane = threadIdx.x & 63;
        const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        const int d = gemm4_decoder(wave, rows);
        if (d < 0) {
            gemm4_mfma_waves(a.in, xfrag0, rows, slots, Bs, emit);
            return;
        }
        const int nsup = IT / 8;
        const bool help = rows <= G4_HELP_ROWS;
        if (e >= a.experts) {  // the shared expert: its own uniform bank
            gemm4_decode_waves_at<FAM>(a.sh_n, a.sh_trellis[p], OT, og, nsup, d, help, lane,
                                       rate_decode<FAM>(a.k, a.table, a.sh_n), Bs);
            return;
        }
        if constexpr (N == N_TILED) {
            const DecodeK ka = rate_decode<FAM>(a.k, a.table, TILED_NA), kb = rate_decode<FAM>(a.k, a.table, TILED_NB);
            gemm4_decode_role<FAM>(help, d, nsup, lane, Bs, [&](int r, int rs, int loads) {
                return TiledReader<FAM>(a.trellis[p], a.seg_off[p], a.seg_k1[p], e, r, rs, IT, OT, og, loads, lane, ka,
                                        kb);
            });
        } else {
            const uint32_t *m = a.meta + (size_t)e * 8;
            const int col = a.meta_col[p];
            const int n = (int)m[col];
            gemm4_decode_waves_at<FAM>(n, a.trellis[p] + 2 * (size_t)m[4 + col], OT, og, nsup, d, help, lane,
                                       rate_decode<FAM>(a.k, a.table, n), Bs);
        }
    }
}

// ---- the routed GEMM arm's inputs.  Tile t (16 sorted rows of one window, the window's tiles contiguous from
// win_tile0) is prepared into fragment order at xp + t * (in / 32) * 512, as gemm_prepare_frag_kernel does for dense
// rows; rows past the window's end are zeros.  Tiles past the count exit at once.
struct TileRows {
    bool live;
    int rows;             // live rows of the tile (16 unless the window's last)
    int e;                // the window's expert
    const uint32_t *slots;
};

__device__ __forceinline__ TileRows tile_rows(const MoeGemmArgs &a, int t) {
    TileRows r;
    const uint4 ti = a.win.tile_info[t];  // t < max_tiles (the grid); read beside the count, used only if live
    r.live = (uint32_t)t < *a.win.tile_count;
    if (!r.live) return r;
    r.rows = (int)ti.y;
    r.e = moe_expert(a, ti.x);
    r.slots = a.win.sorted + ti.z;
    return r;
}

// The 16 x 128 f16 tile in LDS to fragment order (one 16-byte store per thread).
__device__ __forceinline__ void tile_to_frag(const uint16_t (*tl)[128 + 8], uint16_t *xp, int t, int b, int in,
                                             int tid) {
    const int lane = tid & 63, kq = tid >> 6, c = lane & 15, h = lane >> 4;
    const uint4 v = *reinterpret_cast<const uint4 *>(&tl[c][kq * 32 + 8 * h]);
    *reinterpret_cast<uint4 *>(xp + ((size_t)t * (in / 32) + (size_t)b * 4 + kq) * 512 + (size_t)lane * 8) = v;
}

// prepareInput (expert_exl3.zig:490-501) of each row's token with its expert's suh, for gate and up from one load of
// the rows, over NB consecutive 128-column blocks of one tile.  Every load is in bounds (a row past the tile's end
// reads the tile's last live row and is zeroed after), so a wave's four rows of every block go out together with the
// suh loads, behind only the tile's table and slot reads; the transforms then run for both projections at once.
// (A workgroup per projection gathered each token row from memory once per projection: 95 us at 2048 tokens.)
template <int NB, int DT>
__global__ __launch_bounds__(256) void moe_gemm_prepare_kernel(MoeGemmArgs a) {
    const int b0 = blockIdx.x * NB, t = blockIdx.y;
    const TileRows tr = tile_rows(a, t);
    if (!tr.live) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ __align__(16) uint16_t tl[NB][2][16][128 + 8];
    const bool shx = tr.e >= a.experts;
    const size_t se = shx ? 0 : (size_t)tr.e * a.in;
    uint32_t sl[4];
#pragma unroll
    for (int rr = 0; rr < 4; rr++) sl[rr] = tr.slots[min(wave * 4 + rr, max(tr.rows - 1, 0))];
    size_t xr[4];
#pragma unroll
    for (int rr = 0; rr < 4; rr++) xr[rr] = (size_t)moe_token(a, __builtin_amdgcn_readfirstlane(sl[rr])) * a.in;
    float x0[NB][4], x1[NB][4], u0[NB][2], u1[NB][2];
#pragma unroll
    for (int rr = 0; rr < 4; rr++)
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            const size_t xi = xr[rr] + (size_t)(b0 + nb) * 128;
            x0[nb][rr] = load_act<DT>(a.x, xi + lane);
            x1[nb][rr] = load_act<DT>(a.x, xi + lane + 64);
        }
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const uint16_t *su = shx ? a.sh_suh[q] : a.suh[q];
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            const size_t si = se + (size_t)(b0 + nb) * 128;
            u0[nb][q] = h2f(su[si + lane]);
            u1[nb][q] = h2f(su[si + lane + 64]);
        }
    }
    const float sc = fwht_relaid_sign(lane) * HAD_SCALE;
    const int c0 = fwht_relaid_col(lane, 0), c1 = fwht_relaid_col(lane, 1);
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        float v0[8], v1[8];  // [projection][row]; rows past the end are zeros
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            const bool live = wave * 4 + rr < tr.rows;
            const float y0 = live ? f16r(x0[nb][rr]) : 0.f, y1 = live ? f16r(x1[nb][rr]) : 0.f;
#pragma unroll
            for (int q = 0; q < 2; q++) {
                v0[q * 4 + rr] = y0 * u0[nb][q];
                v1[q * 4 + rr] = y1 * u1[nb][q];
            }
        }
        fwht128_wave_rows_relaid<8>(v0, v1, lane);
#pragma unroll
        for (int q = 0; q < 2; q++)
#pragma unroll
            for (int rr = 0; rr < 4; rr++) {
                const int r = wave * 4 + rr;
                tl[nb][q][r][c0] = __half_as_ushort(__float2half_rn(v0[q * 4 + rr] * sc));
                tl[nb][q][r][c1] = __half_as_ushort(__float2half_rn(v1[q * 4 + rr] * sc));
            }
    }
    __syncthreads();
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
        for (int q = 0; q < 2; q++) tile_to_frag(tl[nb][q], a.xp[q], t, b0 + nb, a.in, tid);
}

// The SwiGLU mid of the routed GEMM arm (DOWN_FUSED_SOURCE's prologue, expert_exl3_kernels.zig:1838-1925; the
// decode chain's PRO_MID with one plane): gate and up = svh * H(raw inner), the clamps, SiLU(gate) * up * suh_down,
// H, f16 -- the down projection's prepared input, in fragment order at xp[0] (a.in = inter).
__global__ __launch_bounds__(256) void moe_gemm_mid_kernel(MoeGemmArgs a) {
    const int b = blockIdx.x, t = blockIdx.y;
    const TileRows tr = tile_rows(a, t);
    if (!tr.live) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ __align__(16) uint16_t tl[16][128 + 8];
    const bool shx = tr.e >= a.experts;  // the shared expert's rows: its own scales
    const size_t si = (shx ? 0 : (size_t)tr.e * a.in) + (size_t)b * 128;
    const uint16_t *svg = shx ? a.sh_mid_svh[0] : a.mid_svh[0], *svu = shx ? a.sh_mid_svh[1] : a.mid_svh[1];
    const uint16_t *sud = shx ? a.sh_down_suh : a.down_suh;
    // the gate / up transforms leave column fwht_relaid_col(lane, s) in slot s, so the scales are read there
    const int c0 = fwht_relaid_col(lane, 0), c1 = fwht_relaid_col(lane, 1);
    const float sg0 = h2f(svg[si + c0]), sg1 = h2f(svg[si + c1]);
    const float su0 = h2f(svu[si + c0]), su1 = h2f(svu[si + c1]);
    const float sd0 = h2f(sud[si + c0]), sd1 = h2f(sud[si + c1]);
    // the wave's four rows, both planes, all loads in bounds and out together (a row past the tile's end reads the
    // last live row and is zeroed after)
    uint32_t sl[4];
#pragma unroll
    for (int rr = 0; rr < 4; rr++) sl[rr] = tr.slots[min(wave * 4 + rr, max(tr.rows - 1, 0))];
    float w0[8], w1[8];  // [gate rows 0..3, up rows 0..3]
#pragma unroll
    for (int rr = 0; rr < 4; rr++) {
        const size_t pi = (size_t)__builtin_amdgcn_readfirstlane(sl[rr]) * a.in + (size_t)b * 128;
        w0[rr] = a.mid_planes[0][pi + lane];
        w1[rr] = a.mid_planes[0][pi + lane + 64];
        w0[4 + rr] = a.mid_planes[1][pi + lane];
        w1[4 + rr] = a.mid_planes[1][pi + lane + 64];
    }
#pragma unroll
    for (int rr = 0; rr < 4; rr++)
        if (wave * 4 + rr >= tr.rows) w0[rr] = w1[rr] = w0[4 + rr] = w1[4 + rr] = 0.f;
    fwht128_wave_rows_relaid<8>(w0, w1, lane);
    // the transforms' sign folded into the scales (exact: both factors change sign)
    const float sgn = fwht_relaid_sign(lane);
    const float kg0 = sgn * (HAD_SCALE * sg0), kg1 = sgn * (HAD_SCALE * sg1);
    const float ku0 = sgn * (HAD_SCALE * su0), ku1 = sgn * (HAD_SCALE * su1);
    float v0[4], v1[4];
#pragma unroll
    for (int rr = 0; rr < 4; rr++) {
        float a0 = w0[rr] * kg0, a1 = w1[rr] * kg1;
        float b0 = w0[4 + rr] * ku0, b1 = w1[4 + rr] * ku1;
        if (a.clamp_limit > 0.f) {
            a0 = fminf(a0, a.clamp_limit);
            a1 = fminf(a1, a.clamp_limit);
            b0 = fminf(fmaxf(b0, -a.clamp_limit), a.clamp_limit);
            b1 = fminf(fmaxf(b1, -a.clamp_limit), a.clamp_limit);
        }
        v0[rr] = silu(a0) * b0 * sd0;
        v1[rr] = silu(a1) * b1 * sd1;
    }
    fwht128_wave_rows_relaid<4, true>(v0, v1, lane);  // rows past the end: silu(0) * 0 = 0, zeros stay zeros
    const float sc = sgn * HAD_SCALE;
    const int d0 = fwht_relaid2_col(lane, 0), d1 = fwht_relaid2_col(lane, 1);
#pragma unroll
    for (int rr = 0; rr < 4; rr++) {
        const int r = wave * 4 + rr;
        tl[r][d0] = __half_as_ushort(__float2half_rn(v0[rr] * sc));
        tl[r][d1] = __half_as_ushort(__float2half_rn(v1[rr] * sc));
    }
    __syncthreads();
    tile_to_frag(tl, a.xp[0], t, b, a.in, tid);
}

template <int DT>
static void launch_moe_gemm_prepare(const MoeGemmArgs &a, hipStream_t s) {
    // two 128-column blocks a workgroup where they pair up (measured at 2048 tokens of configs[3]: 85 -> 79 us; four
    // blocks took 110)
    const int blocks = a.in / 128;
    if (blocks % 2 == 0)
        hipLaunchKernelGGL((moe_gemm_prepare_kernel<2, DT>), dim3((unsigned)(blocks / 2), (unsigned)a.max_tiles),
                           dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((moe_gemm_prepare_kernel<1, DT>), dim3((unsigned)blocks, (unsigned)a.max_tiles), dim3(256),
                           0, s, a);
}

hipError_t run_moe_gemm_prepare(const MoeGemmArgs &a, int nproj, hipStream_t s) {
    if (nproj != 2) return hipErrorInvalidValue;  // gate and up together
    if (a.x_dtype == DT_F16) launch_moe_gemm_prepare<DT_F16>(a, s);
    else if (a.x_dtype == DT_BF16) launch_moe_gemm_prepare<DT_BF16>(a, s);
    else launch_moe_gemm_prepare<DT_F32>(a, s);
    return hipGetLastError();
}

hipError_t run_moe_gemm_mid(const MoeGemmArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(moe_gemm_mid_kernel, dim3((unsigned)(a.in / 128), (unsigned)a.max_tiles), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int FAM>
static hipError_t launch_moe_gemm_fam(const MoeGemmArgs &a, int nproj, hipStream_t s) {
    // x: column group and window, the windows rounded up to whole rounds of the 8 XCDs (the extra ones exit)
    const dim3 grid((unsigned)(a.out / 128) * (unsigned)((a.max_windows + 7) / 8 * 8), (unsigned)nproj);
    if (a.seg_off[0]) {  // per-tile rates: the hash-product families
        if constexpr (FAM == FAM_PAIR || FAM == FAM_MUL1) return hipErrorInvalidValue;
        else hipLaunchKernelGGL((moe_gemm4_kernel<FAM, N_TILED>), grid, dim3(G4_THREADS), 0, s, a);
        return hipGetLastError();
    }
    if (a.meta) {
        hipLaunchKernelGGL((moe_gemm4_kernel<FAM, -1>), grid, dim3(G4_THREADS), 0, s, a);
        return hipGetLastError();
    }
    switch (a.n) {
    case 16: hipLaunchKernelGGL((moe_gemm4_kernel<FAM, 16>), grid, dim3(G4_THREADS), 0, s, a); break;
    case 24: hipLaunchKernelGGL((moe_gemm4_kernel<FAM, 24>), grid, dim3(G4_THREADS), 0, s, a); break;
    case 32: hipLaunchKernelGGL((moe_gemm4_kernel<FAM, 32>), grid, dim3(G4_THREADS), 0, s, a); break;
    case 40: hipLaunchKernelGGL((moe_gemm4_kernel<FAM, 40>), grid, dim3(G4_THREADS), 0, s, a); break;
    case 48: hipLaunchKernelGGL((moe_gemm4_kernel<FAM, 48>), grid, dim3(G4_THREADS), 0, s, a); break;
    case 64: hipLaunchKernelGGL((moe_gemm4_kernel<FAM, 64>), grid, dim3(G4_THREADS), 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t run_moe_gemm(int fam, const MoeGemmArgs &a, int nproj, hipStream_t s) {
    switch (fam) {
    case FAM_MCG: return launch_moe_gemm_fam<FAM_MCG>(a, nproj, s);
    case FAM_MUL1: return launch_moe_gemm_fam<FAM_MUL1>(a, nproj, s);
    case FAM_HASH: return launch_moe_gemm_fam<FAM_HASH>(a, nproj, s);
    case FAM_PAIR: return launch_moe_gemm_fam<FAM_PAIR>(a, nproj, s);
    default: return launch_moe_gemm_fam<FAM_3INST>(a, nproj, s);
    }
}

template <int FAM, int N>
static hipError_t launch_gemm_lane_n(const GemmArgs &a, hipStream_t s) {
    if (a.x_dtype == DT_F16) launch_gemm_prepare_frag<DT_F16>(a, s);
    else if (a.x_dtype == DT_BF16) launch_gemm_prepare_frag<DT_BF16>(a, s);
    else launch_gemm_prepare_frag<DT_F32>(a, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // The ping-pong body once its 512-row tiles still give most CUs a workgroup (measured at C3's 4096 x 14336: 768 to
    // 4096 rows 13-24% faster than the 256-row decode-wave tile; at 512 rows, 112 workgroups, 18% slower, and with k in
    // halves, 224 workgroups, 3% faster).
    int arm = a.arm ? a.arm : gemm_default_arm(a.groups, a.rows, a.out);
    if constexpr (FAM == FAM_PAIR || FAM == FAM_MUL1) arm = 4;  // the ping-pong body serves the hash-product families
    // n = 40's unaligned lane reader does not fit the 512-row tile's registers (it would spill): the 256-row one
    if constexpr (N == 40) arm = arm == 5 ? (a.arm ? 6 : 4) : arm;
    if (arm == 7 && (N == 40 || !a.kpart)) arm = 4;  // the split needs its partial region (the host sizes it)
    if (arm == 5 || arm == 6 || arm == 7) {
        const int mt = arm == 6 ? 256 : 512;
        dim3 grid((unsigned)((a.out / 128) * ((a.rows + mt - 1) / mt) * (arm == 7 ? 2 : 1)), 1, (unsigned)a.groups);
        if constexpr (FAM != FAM_PAIR && FAM != FAM_MUL1) {
            if constexpr (N != 40) {
                if (arm == 5) hipLaunchKernelGGL((gemm5_kernel<FAM, N, 512, 1>), grid, dim3(G5_THREADS), 0, s, a);
                if (arm == 7) hipLaunchKernelGGL((gemm5_kernel<FAM, N, 512, 2>), grid, dim3(G5_THREADS), 0, s, a);
            }
            if (arm == 6) hipLaunchKernelGGL((gemm5_kernel<FAM, N, 256, 1>), grid, dim3(G5_THREADS), 0, s, a);
        }
        return hipGetLastError();
    }
    dim3 grid((unsigned)((a.out / 128) * ((a.rows + G2_MT - 1) / G2_MT)), 1, (unsigned)a.groups);
    hipLaunchKernelGGL((gemm4_kernel<FAM, N>), grid, dim3(G4_THREADS), 0, s, a);
    return hipGetLastError();
}

template <int FAM, int N>
static hipError_t launch_gemm_n(const GemmArgs &a, const uint16_t *wt, hipStream_t s) {
    dim3 grid((unsigned)(a.out / 128), (unsigned)((a.rows + GM_MT - 1) / GM_MT), (unsigned)a.groups);
    hipLaunchKernelGGL((gemm_kernel<FAM, N>), grid, dim3(GM_THREADS), 0, s, a, wt);
    return hipGetLastError();
}

template <int FAM>
static hipError_t launch_gemm_fam(const GemmArgs &a, hipStream_t s) {
    switch (a.n) {
    case 16: return launch_gemm_lane_n<FAM, 16>(a, s);
    case 24: return launch_gemm_lane_n<FAM, 24>(a, s);
    case 32: return launch_gemm_lane_n<FAM, 32>(a, s);
    case 40: return launch_gemm_lane_n<FAM, 40>(a, s);
    case 48: return launch_gemm_lane_n<FAM, 48>(a, s);
    case 64: return launch_gemm_lane_n<FAM, 64>(a, s);
    default: break;
    }
    hipLaunchKernelGGL(gemm_prepare_kernel, dim3((unsigned)(a.in / 128), (unsigned)a.rows, (unsigned)a.groups),
                       dim3(64), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // Any other rate: decode to a transposed f16 copy in workspace (held after xp), then the same MFMA body.
    uint16_t *wt = a.wt;
    hipLaunchKernelGGL(gemm_decode_transposed_kernel<FAM>,
                       dim3((unsigned)((a.in / 16) * (a.out / 16)), (unsigned)a.groups), dim3(128), 0, s, a, wt);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_gemm_n<FAM, 0>(a, wt, s);
}

hipError_t run_gemm(int fam, const GemmArgs &a, hipStream_t s) {
    switch (fam) {
    case FAM_MCG: return launch_gemm_fam<FAM_MCG>(a, s);
    case FAM_MUL1: return launch_gemm_fam<FAM_MUL1>(a, s);
    case FAM_HASH: return launch_gemm_fam<FAM_HASH>(a, s);
    case FAM_PAIR: return launch_gemm_fam<FAM_PAIR>(a, s);
    default: return launch_gemm_fam<FAM_3INST>(a, s);
    }
}

}  // namespace exl3
