// The lane decoder shared by the GEMV and the GEMM: one lane's 32 codewords of a 16x16 trellis tile, from its
// aligned stream words, to 16 packed f16 weight pairs (t, t+1).  Lane chunk j of a tile holds codewords 32j..32j+31,
// the weights of output columns j and j+8 over all 16 k rows (tensorCorePerm, beamivalice/sushi
// src/exl3/expert_exl3.zig:379-398): pair i = 4qq + p covers rows 2qq + 8(p & 1) + {0, 1} of column j (p < 2) or
// j + 8 (p >= 2).
#pragma once
#include "exl3_common.cuh"

namespace exl3 {

// Codeword v of the lane as (window index, high half?): for K = 1, 2, 4 the window ending at codeword v + 16/K
// carries codeword v in its high half, so half the windows serve two codewords.
template <int N>
struct Pairing {
    static constexpr bool ON = N == 16 || N == 32 || N == 64;
    static constexpr int STEP = ON ? 256 / N : 32;
    __device__ static constexpr bool hi(int v) { return ON && ((v / STEP) % 2 == 0); }
    __device__ static constexpr int win(int v) { return hi(v) ? v + STEP : v; }
};

// A scheduling fence: nothing moves across it, so each phase below stays one batch of independent instructions.
__device__ __forceinline__ void phase_fence() { __builtin_amdgcn_sched_barrier(0); }

// A pair of hash / pair family weights times 2^12 (exact: they are the codebook values over 4096), as the
// reconstruction returns them.  The matrix cores take them unscaled (codebook_scale).
__device__ __forceinline__ uint32_t scale_h2_4096(uint32_t v) {
    __half2 h = __builtin_bit_cast(__half2, v);
    h = __hmul2(h, __half2(__float2half(4096.0f), __float2half(4096.0f)));
    return __builtin_bit_cast(uint32_t, h);
}

// The weights of the lane's chunk, unscaled for the hash / pair families (the x4096 is applied by the caller).
// Written in fenced phases (windows, product step 1, step 2, masks, low sums, high sums): within a phase no
// instruction depends on another, so no result is read by the instruction right after it and the hazard recognizer
// inserts no wait states (gfx950 needs one between a 16-bit-lane or SDWA write and its reader).
template <int FAM, int N, bool MASKED>
__device__ __forceinline__ void decode_weights(const uint32_t (&A)[LaneBits<N>::AW], const DecodeK &k,
                                               uint32_t (&w)[16]) {
    using P = Pairing<N>;
    if constexpr (FAM == FAM_PAIR || FAM == FAM_MUL1) {
        uint32_t win[32];
#pragma unroll
        for (int v = 0; v < 32; v++) {
            if (P::win(v) == v) {
                win[v] = lane_codeword<N>(A, v);
                if constexpr (MASKED) win[v] &= k.wmask | (k.wmask << 16);
            }
        }
        if constexpr (FAM == FAM_PAIR) {
            // both weights of a pair decode from the odd codeword (decodePair, expert_exl3.zig:298-301)
            uint32_t pr[16];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int v = 2 * i + 1;
                pr[i] = P::hi(v) ? mul16x32<true>(win[P::win(v)], k.mult >> 16, k.mult & 0xFFFFu)
                                 : mul16x32<false>(win[P::win(v)], k.mult >> 16, k.mult & 0xFFFFu);
            }
            uint32_t h0[16], h1[16];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                h0[i] = pr[i] & k.mask0;
                h1[i] = __builtin_amdgcn_alignbit(pr[i], pr[i], 32u - k.rot) & k.mask1;
            }
            // the sums in two fenced phases, as the hash-product families write theirs below: each is an SDWA write
            // in inline asm, whose readers need wait states the compiler does not count for asm (an MFMA reading
            // one two instructions later read stale weights); phased, a sum is read no sooner than the next phase
            phase_fence();
#pragma unroll
            for (int i = 0; i < 16; i++)
                asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1"
                    : "=v"(w[i]) : "v"(h0[i]));
            phase_fence();
#pragma unroll
            for (int i = 0; i < 16; i++)
                asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
                    : "+v"(w[i]) : "v"(h1[i]));
            phase_fence();
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t x0 = win[P::win(2 * i)], x1 = win[P::win(2 * i + 1)];
                const uint32_t c0 = P::hi(2 * i) ? x0 >> 16 : x0, c1 = P::hi(2 * i + 1) ? x1 >> 16 : x1;
                w[i] = pack_h2(decode1<FAM_MUL1>(c0, k), decode1<FAM_MUL1>(c1, k));
            }
        }
    } else {
        // Rates without pairing (one window per codeword) run the phases over two halves of the chunk, so only half
        // the windows and products are live at once; paired windows serve codewords up to 16 apart, so paired rates
        // run all 32 together.
        constexpr int H = P::ON ? 1 : 2;
        constexpr int V = 32 / H;
#pragma unroll
        for (int hh = 0; hh < H; hh++) {
            const int v0 = hh * V;
            uint32_t win[V], h[V];
#pragma unroll
            for (int v = 0; v < V; v++) {
                if (P::win(v0 + v) == v0 + v) {
                    win[v] = lane_codeword<N>(A, v0 + v);
                    if constexpr (MASKED) win[v] &= k.wmask | (k.wmask << 16);
                }
            }
            phase_fence();
#pragma unroll
            for (int v = 0; v < V; v++) {
                const int wv = P::win(v0 + v) - v0;
                h[v] = P::hi(v0 + v) ? hash_step1<FAM, true>(win[wv], k) : hash_step1<FAM, false>(win[wv], k);
            }
            phase_fence();
#pragma unroll
            for (int v = 0; v < V; v++) {
                const int wv = P::win(v0 + v) - v0;
                if (P::hi(v0 + v)) hash_step2<FAM, true>(win[wv], k, h[v]);
                else hash_step2<FAM, false>(win[wv], k, h[v]);
            }
            phase_fence();
#pragma unroll
            for (int v = 0; v < V; v++) h[v] = hash_halves<FAM>(h[v], k);
            phase_fence();
#pragma unroll
            for (int i = 0; i < V / 2; i++)
                asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1"
                    : "=v"(w[v0 / 2 + i]) : "v"(h[2 * i]));
            phase_fence();
#pragma unroll
            for (int i = 0; i < V / 2; i++)
                asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
                    : "+v"(w[v0 / 2 + i]) : "v"(h[2 * i + 1]));
            phase_fence();
        }
    }
}

// Half of the lane's chunk, for the hash-product families (MCG, 3INST, hash rows): the 8 weight pairs of column
// j + 8 H (pairs i with (i & 2) == 2 H, in the order 2H, 2H+1, 2H+4, 2H+5, ..., 2H+13), so two waves can share one
// chunk's decode.  Output pair q holds rows 2 (q >> 1) + 8 (q & 1) + {0, 1} of that column; unscaled.  The phases run
// over two groups of 8 codewords, so few registers are live beside a caller's accumulators.
template <int FAM, int N, bool MASKED, int H>
__device__ __forceinline__ void decode_weights_half(const uint32_t (&A)[LaneBits<N>::AW], const DecodeK &k,
                                                    uint32_t (&w)[8]) {
    static_assert(FAM != FAM_PAIR && FAM != FAM_MUL1, "the half decoder serves the hash-product families");
    using P = Pairing<N>;
    // codeword u (0..15) of this half: pair 2H + (u >> 1 & 1) + 4 (u >> 2), element u & 1
    auto cw_of = [](int u) constexpr { return 2 * (2 * H + ((u >> 1) & 1) + 4 * (u >> 2)) + (u & 1); };
#pragma unroll
    for (int gq = 0; gq < 2; gq++) {
        uint32_t win[8], h[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            win[i] = lane_codeword<N>(A, P::win(cw_of(8 * gq + i)));
            if constexpr (MASKED) win[i] &= k.wmask | (k.wmask << 16);
        }
        phase_fence();
#pragma unroll
        for (int i = 0; i < 8; i++)
            h[i] = P::hi(cw_of(8 * gq + i)) ? hash_step1<FAM, true>(win[i], k) : hash_step1<FAM, false>(win[i], k);
        phase_fence();
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (P::hi(cw_of(8 * gq + i))) hash_step2<FAM, true>(win[i], k, h[i]);
            else hash_step2<FAM, false>(win[i], k, h[i]);
        }
        phase_fence();
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = hash_halves<FAM>(h[i], k);
        phase_fence();
#pragma unroll
        for (int q = 0; q < 4; q++)
            asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1"
                : "=v"(w[4 * gq + q]) : "v"(h[2 * q]));
        phase_fence();
#pragma unroll
        for (int q = 0; q < 4; q++)
            asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
                : "+v"(w[4 * gq + q]) : "v"(h[2 * q + 1]));
        phase_fence();
    }
}

// ------------------------------------------------------------------------------------------------------------
// Per-tile rates (configs[4]'s seeded K1 / K2 tile mix, a layout extension: the reference fixes a rate per tensor or
// per expert group, src/exl3/layout.zig:56-62, and decodes every tile at its own n with decodeTile,
// src/exl3/expert_exl3.zig:338-357).  A segment is the 8 tiles (k-tile row tk, output group s) one wave reads; they
// lie contiguous from the segment's word offset, tile o at TILED_NA halfwords when bit o of the segment's mask is set,
// else TILED_NB, so tile o starts 16 o - 8 popcount(mask below o) words in.  Each lane decodes its chunk at its own
// tile's rate.
// The lane's words of its tile: A[0..1] as load_lane_words<16> reads them (k1), else A[0..2] as load_lane_words<32>.
// `row` is the segment's wave-uniform start and lane_words its tile's offset (words); loads take the scalar-base form.
__device__ __forceinline__ void load_lane_words_tiled(const uint32_t *__restrict__ row, uint32_t lane_words, int j,
                                                      bool k1, uint32_t (&A)[3]) {
    typedef __attribute__((address_space(1))) const uint32_t global_u32;
    const char *base = reinterpret_cast<const char *>(row);
    auto at = [&](uint32_t w) __attribute__((always_inline)) {
        return *(global_u32 *)(base + (uint32_t)((lane_words + w) * 4u));
    };
    const uint32_t i0 = k1 ? (uint32_t)((j + 7) & 7) : (uint32_t)((2 * j + 15) & 15);
    const uint32_t i1 = k1 ? (uint32_t)j : (uint32_t)(2 * j);
    const uint32_t i2 = k1 ? (uint32_t)j : (uint32_t)(2 * j + 1);  // unused at n = 16 (a repeat of A[1])
    A[0] = at(i0);
    A[1] = at(i1);
    A[2] = at(i2);
}

// The lane's 16 weight pairs at its own rate.  Both rates pair codewords in 32-bit windows (Pairing<16>: window s
// ending at codeword 16 + s carries codeword s in its high half; Pairing<32>: the windows ending at codewords 8 + s
// and 16 + s (s >= 8) carry s and 8 + s), so only the window extraction depends on the rate; the products, masks and
// sums run once over 16 windows in the n = 32 arrangement (codewords 0-7 = high halves 0-7, 8-15 = low 0-7, 16-23 =
// high 8-15, 24-31 = low 8-15).  At n = 16 the middle two groups of that arrangement hold codewords 16-23 and 8-15,
// so a k1 lane swaps pairs 4-7 with 8-11 at the end.  k: the lane's rate constants.
template <int FAM, bool MASKED>
__device__ __forceinline__ void decode_weights_tiled(const uint32_t (&A)[3], bool k1, const DecodeK &k,
                                                     uint32_t (&w)[16]) {
    static_assert(FAM != FAM_PAIR && FAM != FAM_MUL1, "per-tile rates serve the hash-product families");
    const uint32_t A16[2] = {A[0], A[1]};
    uint32_t win[16], hl[16], hh[16];
#pragma unroll
    for (int s = 0; s < 16; s++) {
        const uint32_t c16 = lane_codeword<16>(A16, 16 + s);
        const uint32_t c32 = lane_codeword<32>(A, s < 8 ? 8 + s : 16 + s);
        win[s] = k1 ? c16 : c32;
        if constexpr (MASKED) win[s] &= k.wmask | (k.wmask << 16);
    }
    phase_fence();
#pragma unroll
    for (int s = 0; s < 16; s++) {
        hl[s] = hash_step1<FAM, false>(win[s], k);
        hh[s] = hash_step1<FAM, true>(win[s], k);
    }
    phase_fence();
#pragma unroll
    for (int s = 0; s < 16; s++) {
        hash_step2<FAM, false>(win[s], k, hl[s]);
        hash_step2<FAM, true>(win[s], k, hh[s]);
    }
    phase_fence();
#pragma unroll
    for (int s = 0; s < 16; s++) {
        hl[s] = hash_halves<FAM>(hl[s], k);
        hh[s] = hash_halves<FAM>(hh[s], k);
    }
    phase_fence();
    // codeword v of the n = 32 arrangement
    auto h_of = [&](int v) __attribute__((always_inline)) {
        return v < 8 ? hh[v] : v < 16 ? hl[v - 8] : v < 24 ? hh[v - 8] : hl[v - 16];
    };
#pragma unroll
    for (int i = 0; i < 16; i++)
        asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1"
            : "=v"(w[i]) : "v"(h_of(2 * i)));
    phase_fence();
#pragma unroll
    for (int i = 0; i < 16; i++)
        asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
            : "+v"(w[i]) : "v"(h_of(2 * i + 1)));
    phase_fence();
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint32_t a = w[4 + q], b = w[8 + q];
        w[4 + q] = k1 ? b : a;
        w[8 + q] = k1 ? a : b;
    }
}

// The mask of segment `seg` (8 bits, one per tile), read through its aligned 32-bit word so the load stays a scalar
// one (the host checks that the table is 4-byte aligned; its length, a multiple of 8, keeps the word inside it).
__device__ __forceinline__ uint32_t seg_mask(const uint8_t *k1, size_t seg) {
    const uint32_t w = reinterpret_cast<const uint32_t *>(k1)[seg >> 2];
    return (w >> (8u * (uint32_t)(seg & 3))) & 0xFFu;
}

// A lane's rate constants in a per-tile-rate bank: the hash rows differ by rate (mult, mask); the window mask and the
// fixed families' constants do not.
__device__ __forceinline__ DecodeK tiled_constants(bool k1, const DecodeK &ka, const DecodeK &kb) {
    DecodeK k = kb;
    k.mult = k1 ? ka.mult : kb.mult;
    k.mask0 = k1 ? ka.mask0 : kb.mask0;
    return k;
}

}  // namespace exl3
