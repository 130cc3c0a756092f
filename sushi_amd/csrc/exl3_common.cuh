// Shared device code for the EXL3/STQ trellis kernels on gfx950 (CDNA4, wave64).
//
// Format facts the kernels rely on (beamivalice/sushi src/exl3/expert_exl3.zig):
//  * A 16x16 tile of one projection is n u16 = n/2 u32 words, word i = hw[2i] | hw[2i+1] << 16, read as one
//    MSB-first circular bitstream of 16n bits (unpackTile, :313-336).
//  * Weight t (0..255) of a tile is the 16-bit window ending at bit floor((t+1)n/16) (Rate.bitEnd, :202-205),
//    masked to the pack's window width (Window.mask, :124-126), decoded by the codebook (:267-311), and lands at
//    row-major tile position tensorCorePerm[t] (:379-398): t = 8T + i, T = 4j + q, row = {2q, 2q+1, 2q+8, 2q+9}[i % 4],
//    col = j + 8 * (i >= 4).  Row is the input (k) index, col the output index.
//  * Tiles of one projection lie [E][in/16][out/16][n] (pack order).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

namespace exl3 {

enum Codebook : int { CB_MUL1 = 0, CB_MCG = 1, CB_SPEC1 = 2, CB_PAIR1 = 3, CB_STD1 = 4, CB_3INST = 5 };
// Kernel-side decode families: SPEC1 and STD1 share the hash-mask body with a per-rate (mult, mask) row.
enum Family : int { FAM_MCG = 0, FAM_MUL1 = 1, FAM_HASH = 2, FAM_PAIR = 3, FAM_3INST = 4 };

// Per-tile-rate banks (configs[4]'s K1 / K2 tile mix): every tile at one of these two rates, and the kernels' rate
// parameter for such a bank.
constexpr int TILED_NA = 16, TILED_NB = 32;
constexpr int N_TILED = -3;

// Runtime decode constants for one (codebook, window, table, rate): filled on the host.
struct DecodeK {
    uint32_t wmask;  // codeword window mask (w16: 0xFFFF)
    uint32_t mult;   // hash / pair multiplier
    uint32_t mask0;  // hash mask / pair mask0
    uint32_t mask1;  // pair mask1
    uint32_t rot;    // pair rotate
};

__device__ __forceinline__ uint32_t pack_h2(__half lo, __half hi) {
    return (uint32_t)__half_as_ushort(lo) | ((uint32_t)__half_as_ushort(hi) << 16);
}

// Sum of the two f16 halves of `h`, rounded to f16 (the reference's f32 add then f16 round; exact-sum arguments
// make the two equal: for MCG/3INST both halves lie in [2^-3, 2), for hash masks both are < 2^-11).
__device__ __forceinline__ __half half_sum(uint32_t h) {
    return __hadd(__ushort_as_half((unsigned short)(h & 0xFFFFu)), __ushort_as_half((unsigned short)(h >> 16)));
}

// c * M mod 2^32 for a 16-bit codeword c (upper bits of c already clear).
__device__ __forceinline__ uint32_t hash_mul(uint32_t c, uint32_t m) { return c * m; }

// One weight from a 16-bit codeword for the scalar families, as f16 bits.  `c` holds the codeword in its low 16
// bits; its high bits are ignored.
template <int FAM>
__device__ __forceinline__ __half decode1(uint32_t c, const DecodeK &k) {
    c &= k.wmask;
    if constexpr (FAM == FAM_MCG) {
        uint32_t p = hash_mul(c, 0xCBAC1FEDu);
        return half_sum((p & 0x8FFF8FFFu) ^ 0x3B603B60u);
    } else if constexpr (FAM == FAM_3INST) {
        uint32_t p = c * 89226354u + 64248484u;
        return half_sum((p & 0x8FFF8FFFu) ^ 0x3B603B60u);
    } else if constexpr (FAM == FAM_MUL1) {
        uint32_t p = hash_mul(c, 0x83DCD12Du);
        uint32_t s = (p & 0x00FF00FFu) + ((p >> 8) & 0x00FF00FFu);
        uint32_t bsum = 0x6400u + (s & 0xFFFFu) + (s >> 16);
        float h = __half2float(__ushort_as_half((unsigned short)bsum));
        float r = __builtin_fmaf(h, __half2float(__ushort_as_half((unsigned short)0x1EEEu)),
                                 __half2float(__ushort_as_half((unsigned short)0xC931u)));
        return __float2half_rn(r);
    } else {  // FAM_HASH: unscaled half sum; the x4096 scale is applied by the caller
        uint32_t p = hash_mul(c, k.mult);
        return half_sum(p & k.mask0);
    }
}

// PAIR1: both weights of a pair from the odd weight's codeword (decodePair, expert_exl3.zig:298-301), unscaled.
__device__ __forceinline__ uint32_t decode_pair_unscaled(uint32_t c, const DecodeK &k) {
    c &= k.wmask;
    uint32_t p = c * k.mult;
    uint32_t r = (p << k.rot) | (p >> ((32u - k.rot) & 31u));
    return pack_h2(half_sum(p & k.mask0), half_sum(r & k.mask1));
}

// Whether a family's decoded half is the weight over 4096 (hash masks and PAIR1 store unscaled sums; the scale
// is a power of two, so applying it to the f32 result or to the f16 weight gives the same bytes).
template <int FAM>
__device__ __forceinline__ constexpr bool family_scaled() {
    return FAM == FAM_HASH || FAM == FAM_PAIR;
}
// The factor from a family's decoded values to its weights.  The matrix cores take the decoded values as they are
// (f16 subnormals included: v_mfma_f32_4x4x4_16b_f16 and v_mfma_f32_16x16x32_f16 multiply them exactly, checked
// against exact sums on gfx950), and the finish applies this power of two to the f32 sums, exactly.
template <int FAM>
__device__ __forceinline__ constexpr float codebook_scale() {
    return family_scaled<FAM>() ? 4096.0f : 1.0f;
}

// Weights (t, t+1) of a tile as packed f16 (lo = t, hi = t+1), from their codewords (c0 for t, c1 for t+1, t even).
// Unscaled for hash/pair families.
template <int FAM>
__device__ __forceinline__ uint32_t decode_pair_h2(uint32_t c0, uint32_t c1, const DecodeK &k) {
    if constexpr (FAM == FAM_PAIR) {
        return decode_pair_unscaled(c1, k);
    } else {
        return pack_h2(decode1<FAM>(c0, k), decode1<FAM>(c1, k));
    }
}

// ------------------------------------------------------------------------------------------------------------
// Hand-scheduled gfx950 decode primitives for the GEMV's hot loop.  A 32-bit funnel window `x` holds one codeword
// in its low half and (for rates K = 1, 2, 4) the codeword 16/K positions earlier in its high half; HI selects it.
// Every op here is full rate: the 32-bit hash multiply c*M (a quarter-rate v_mul_lo_u32) becomes
//   t = lo16(c * hi16(M)) << 16        v_mul_lo_u16 (SDWA: reads the 16-bit half, writes the high half)
//   p = c * lo16(M) + t                v_mad_u32_u16 (op_sel picks the half)
// which equals c*M mod 2^32 because c < 2^16.

template <bool HI>
__device__ __forceinline__ uint32_t mul16x32(uint32_t x, uint32_t mh, uint32_t ml) {
    uint32_t t, p;
    if constexpr (HI) {
        asm("v_mul_lo_u16_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:WORD_0"
            : "=v"(t) : "v"(x), "v"(mh));
        asm("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[1,0,0,0]" : "=v"(p) : "v"(x), "v"(ml), "v"(t));
    } else {
        asm("v_mul_lo_u16_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_0"
            : "=v"(t) : "v"(x), "v"(mh));
        asm("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(p) : "v"(x), "v"(ml), "v"(t));
    }
    return p;
}

// The hash products of the GEMV hot loop as two full-rate steps, so a tile's codewords can run each step as one
// batch (no instruction then reads the result of the one just before it, and the hazard recognizer inserts no wait
// states):
//   MCG / hash rows: step 1  t = lo16(c * hi16(M)) << 16       v_mul_lo_u16 (SDWA, high half written, low cleared)
//                    step 2  t = c * lo16(M) + t               v_mad_u32_u16, in place     -> c*M mod 2^32
//   3INST (LCG):     step 1  p = c * lo16(A) + B               v_mad_u32_u16
//                    step 2  p.hi = lo16(c * hi16(A) + p.hi)   v_mad_u16 op_sel (high half written, low kept)
//                                                              -> c*A + B mod 2^32
constexpr uint32_t LCG_A = 89226354u, LCG_B = 64248484u;

template <int FAM>
__device__ __forceinline__ uint32_t hash_mult(const DecodeK &k) {
    return FAM == FAM_MCG ? 0xCBAC1FEDu : FAM == FAM_3INST ? LCG_A : k.mult;
}

template <int FAM, bool HI>
__device__ __forceinline__ uint32_t hash_step1(uint32_t x, const DecodeK &k) {
    const uint32_t m = hash_mult<FAM>(k);
    uint32_t p;
    if constexpr (FAM == FAM_3INST) {
        if constexpr (HI)
            asm("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[1,0,0,0]" : "=v"(p) : "v"(x), "v"(m & 0xFFFFu), "v"(LCG_B));
        else
            asm("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(p) : "v"(x), "v"(m & 0xFFFFu), "v"(LCG_B));
    } else {
        if constexpr (HI)
            asm("v_mul_lo_u16_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:WORD_0"
                : "=v"(p) : "v"(x), "v"(m >> 16));
        else
            asm("v_mul_lo_u16_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_0"
                : "=v"(p) : "v"(x), "v"(m >> 16));
    }
    return p;
}

template <int FAM, bool HI>
__device__ __forceinline__ void hash_step2(uint32_t x, const DecodeK &k, uint32_t &p) {
    const uint32_t m = hash_mult<FAM>(k);
    if constexpr (FAM == FAM_3INST) {
        if constexpr (HI) asm("v_mad_u16 %0, %1, %2, %0 op_sel:[1,0,1,1]" : "+v"(p) : "v"(x), "v"(m >> 16));
        else asm("v_mad_u16 %0, %1, %2, %0 op_sel:[0,0,1,1]" : "+v"(p) : "v"(x), "v"(m >> 16));
    } else {
        if constexpr (HI) asm("v_mad_u32_u16 %0, %1, %2, %0 op_sel:[1,0,0,0]" : "+v"(p) : "v"(x), "v"(m & 0xFFFFu));
        else asm("v_mad_u32_u16 %0, %1, %2, %0" : "+v"(p) : "v"(x), "v"(m & 0xFFFFu));
    }
}

// The masked product: the f16 pair whose sum is the weight (unscaled for hash rows).
template <int FAM>
__device__ __forceinline__ uint32_t hash_halves(uint32_t p, const DecodeK &k) {
    if constexpr (FAM == FAM_HASH) return p & k.mask0;
    else return (p & 0x8FFF8FFFu) ^ 0x3B603B60u;
}

// ------------------------------------------------------------------------------------------------------------
// Bit windows.  A lane that owns codewords 32j..32j+31 of a tile (the 8 weights of fragment threads 4j..4j+3)
// reads stream bits [2jn - 32, 2jn + 2n): codeword u (0..31) ends at 32 + floor((u+1) n / 16) in that range.

template <int N>
struct LaneBits {
    static constexpr int NW = N / 2;                                 // words per tile
    static constexpr bool ALIGNED = (N % 16) == 0;                   // 2jn is word aligned for every lane
    static constexpr int AW = (2 * N + 32 + 31) / 32;                // aligned words the lane's range spans
    __device__ static constexpr int end_of(int u) { return 32 + ((u + 1) * N) / 16; }
};

// Load the lane's aligned 32-bit words A[0..AW) for tile `words` (u32 view) and chunk j (0..7).  A[i] holds stream
// bits [2jn - 32 + 32i, +32) of the circular tile stream.
template <int N>
__device__ __forceinline__ void load_lane_words(const uint32_t *__restrict__ words, int j, uint32_t (&A)[LaneBits<N>::AW]) {
    constexpr int NW = LaneBits<N>::NW;
    constexpr int AW = LaneBits<N>::AW;
    if constexpr (LaneBits<N>::ALIGNED) {
        const int w0 = j * (N / 16);  // first word of the lane's own chunk
        A[0] = words[(w0 + NW - 1) % NW];
#pragma unroll
        for (int i = 1; i < AW; i++) A[i] = words[w0 + i - 1];
    } else {
        const int base = 2 * j * N - 32 + 32 * NW;  // offset by one lap to stay non-negative
        const int wb = base >> 5;
        const int s = base & 31;
        uint32_t R[AW + 1];
#pragma unroll
        for (int i = 0; i < AW + 1; i++) R[i] = words[(wb + i) % NW];
#pragma unroll
        for (int i = 0; i < AW; i++) {
            uint64_t two = ((uint64_t)R[i] << 32) | R[i + 1];
            A[i] = (uint32_t)(two >> (32 - s));
        }
    }
}

// The same words for a tile at `row` (wave-uniform: the group's first tile of a k-tile row) plus the lane's own tile
// offset `lane_words` (u32 words, per lane).  For the rates whose chunks start on a word (N % 16 == 0), each load is
// addressed as the uniform base plus a 32-bit byte offset, so it takes the scalar-base form and a tile costs no 64-bit
// vector address arithmetic; the other rates keep the per-lane pointer, whose contiguous words load as one wide access.
template <int N>
__device__ __forceinline__ void load_lane_words_u(const uint32_t *__restrict__ row, uint32_t lane_words, int j,
                                                  uint32_t (&A)[LaneBits<N>::AW]) {
    if constexpr (LaneBits<N>::ALIGNED) {
        constexpr int NW = LaneBits<N>::NW;
        constexpr int AW = LaneBits<N>::AW;
        typedef __attribute__((address_space(1))) const uint32_t global_u32;
        const char *base = reinterpret_cast<const char *>(row);
        auto at = [&](uint32_t w) __attribute__((always_inline)) {
            return *(global_u32 *)(base + (uint32_t)((lane_words + w) * 4u));
        };
        const int w0 = j * (N / 16);
        A[0] = at((uint32_t)((w0 + NW - 1) % NW));
#pragma unroll
        for (int i = 1; i < AW; i++) A[i] = at((uint32_t)(w0 + i - 1));
    } else {
        load_lane_words<N>(row + lane_words, j, A);
    }
}

// Codeword u (0..31) of the lane from its aligned words (low 16 bits valid).
template <int N>
__device__ __forceinline__ uint32_t lane_codeword(const uint32_t (&A)[LaneBits<N>::AW], int u) {
    const int e = LaneBits<N>::end_of(u);  // exclusive end bit within A
    const int a = (e - 1) >> 5;            // word holding the last bit
    const int sh = 32 * (a + 1) - e;       // bits of word a after the window
    if (a == 0) return A[0] >> sh;
    return __builtin_amdgcn_alignbit(A[a - 1], A[a], sh);
}

// Codeword t of a tile at a runtime rate n: the 16 stream bits ending at floor((t+1)n/16), circular
// (the generic reader for rates without a specialised kernel).
__device__ __forceinline__ uint32_t codeword_at(const uint32_t *__restrict__ words, int n, int t) {
    const int nw = n >> 1;
    const int total = 16 * n;
    const int end = ((t + 1) * n) >> 4;
    const int last = (end + total - 1) % total;
    const int wl = last >> 5;
    const int wp = (wl + nw - 1) % nw;
    return __builtin_amdgcn_alignbit(words[wp], words[wl], 31 - (last & 31)) & 0xFFFFu;
}

// ------------------------------------------------------------------------------------------------------------
// Wave64 128-point Walsh-Hadamard: lane l holds v0 = x[l], v1 = x[l + 64].  Unnormalised (the caller scales by
// 1/sqrt(128)).  Matches hadamard128 (expert_exl3.zig:400-414) up to f32 summation order.

// Every lane exchange stays in the VALU (no LDS round trip): DPP for H = 1..8, the gfx950 row swaps for 16 and 32.
// A butterfly stage gives lane l the sum x[l] + x[l ^ H] where bit H of l is clear and x[l ^ H] - x[l] where it is
// set, each one rounding, as fmaf(other, +-1, first) with the lane's sign.

// +1.0 where bit H of the lane is clear, -1.0 where it is set.
template <int H>
__device__ __forceinline__ float lane_sign(int lane) {
    constexpr int SH = H == 1 ? 31 : H == 2 ? 30 : H == 4 ? 29 : H == 8 ? 28 : H == 16 ? 27 : 26;
    return __builtin_bit_cast(float, 0x3F800000u | (((uint32_t)lane & H) << SH));
}

// The value of lane (lane ^ H) within a 16-lane row: quad permutes for H = 1, 2, a half-row mirror then a quad
// reversal for 4 (7 - (l ^ 3) = l ^ 4 within 8 lanes), a row rotate by 8 for 8.
template <int H>
__device__ __forceinline__ float xor_lane_row(float v) {
    const int b = __builtin_bit_cast(int, v);
    int r;
    if constexpr (H == 1) r = __builtin_amdgcn_mov_dpp(b, 0xB1, 0xF, 0xF, false);       // quad_perm [1,0,3,2]
    else if constexpr (H == 2) r = __builtin_amdgcn_mov_dpp(b, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    else if constexpr (H == 4)
        r = __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(b, 0x141, 0xF, 0xF, false), 0x1B, 0xF, 0xF, false);
    else r = __builtin_amdgcn_mov_dpp(b, 0x128, 0xF, 0xF, false);                        // row_ror:8
    return __builtin_bit_cast(float, r);
}

template <int H>
__device__ __forceinline__ void fwht_stage(float &v0, float &v1, float sign) {
    if constexpr (H >= 16) {
        // v_permlane{16,32}_swap exchanges the odd rows (of 16 or 32 lanes) of its first operand with the even rows
        // of its second: with both holding v, the first then holds the lower lane's value of each pair (lo) and the
        // second the upper's (hi), and the stage is lo + sign * hi.  Written in asm: the compiler's two-result form
        // of the builtin lost the second result when both inputs were one value.  The s_nops cover the VALU write
        // -> swap read and swap write -> VALU read hazards.
        // Volatile: left free to move, the swaps were scheduled into the GEMV's decode (C1 6.57 -> 6.83 us).
        float lo0 = v0, hi0 = v0, lo1 = v1, hi1 = v1;
        if constexpr (H == 16)
            asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\tv_permlane16_swap_b32 %2, %3\n\ts_nop 1"
                         : "+v"(lo0), "+v"(hi0), "+v"(lo1), "+v"(hi1));
        else
            asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\tv_permlane32_swap_b32 %2, %3\n\ts_nop 1"
                         : "+v"(lo0), "+v"(hi0), "+v"(lo1), "+v"(hi1));
        v0 = __builtin_fmaf(hi0, sign, lo0);
        v1 = __builtin_fmaf(hi1, sign, lo1);
    } else {
        v0 = __builtin_fmaf(v0, sign, xor_lane_row<H>(v0));
        v1 = __builtin_fmaf(v1, sign, xor_lane_row<H>(v1));
    }
}

__device__ __forceinline__ void fwht128_wave(float &v0, float &v1, int lane) {
    {
        float a = v0, b = v1;
        v0 = a + b;
        v1 = a - b;
    }
    fwht_stage<32>(v0, v1, lane_sign<32>(lane));
    fwht_stage<16>(v0, v1, lane_sign<16>(lane));
    fwht_stage<8>(v0, v1, lane_sign<8>(lane));
    fwht_stage<4>(v0, v1, lane_sign<4>(lane));
    fwht_stage<2>(v0, v1, lane_sign<2>(lane));
    fwht_stage<1>(v0, v1, lane_sign<1>(lane));
}

// R independent 128-point transforms (one per row), each stage over every row before the next stage: the rows'
// exchanges of one stage go out together instead of each transform waiting out its own chain.  Each row's result
// equals fwht128_wave's.
template <int R>
__device__ __forceinline__ void fwht128_wave_rows(float (&v0)[R], float (&v1)[R], int lane) {
#pragma unroll
    for (int i = 0; i < R; i++) {
        const float a = v0[i], b = v1[i];
        v0[i] = a + b;
        v1[i] = a - b;
    }
    const float s32 = lane_sign<32>(lane), s16 = lane_sign<16>(lane), s8 = lane_sign<8>(lane), s4 = lane_sign<4>(lane),
                s2 = lane_sign<2>(lane), s1 = lane_sign<1>(lane);
#pragma unroll
    for (int i = 0; i < R; i++) fwht_stage<32>(v0[i], v1[i], s32);
#pragma unroll
    for (int i = 0; i < R; i++) fwht_stage<16>(v0[i], v1[i], s16);
#pragma unroll
    for (int i = 0; i < R; i++) fwht_stage<8>(v0[i], v1[i], s8);
#pragma unroll
    for (int i = 0; i < R; i++) fwht_stage<4>(v0[i], v1[i], s4);
#pragma unroll
    for (int i = 0; i < R; i++) fwht_stage<2>(v0[i], v1[i], s2);
#pragma unroll
    for (int i = 0; i < R; i++) fwht_stage<1>(v0[i], v1[i], s1);
}

// ---- fwht128_wave_rows in about half the VALU instructions, each result bit-identical (the same butterfly pairs,
// stage order and roundings), left at another place in the wave and possibly negated.
// * Bits 5 and 4: one v_permlane{32,16}_swap of (v0, v1) puts both values of each pair in one lane, lower first,
//   and the stage is v0 + v1, v0 - v1 in place (instead of two copies, two swaps and two FMAs per row).  The slot
//   then stands for the bit just done.
// * Bits 3..0: the partner comes through DPP inside the FMA, own + sign * partner (v_fmac_f32_dpp; the mov_dpp and
//   the FMA do not fuse when the compiler is left to it).  On the lane whose bit is set that is own - partner, the
//   butterfly's result negated; rounding to nearest is odd-symmetric, so the value is exact up to that sign, and the
//   partners of every later stage carry the same sign (they agree on all bits done before).
// On return lane l's slot s holds fwht_relaid_sign(l) * y[fwht_relaid_col(l, s)].  Needs the whole wave active.
__device__ __forceinline__ int fwht_relaid_col(int lane, int slot) {
    return (lane & 15) | (slot << 4) | ((lane & 48) << 1);
}
__device__ __forceinline__ float fwht_relaid_sign(int lane) {
    return (__builtin_popcount(lane & 15) & 1) ? -1.f : 1.f;
}

template <int H>
__device__ __forceinline__ void permlane_swap_pair(float &a, float &b) {
    const unsigned ua = __builtin_bit_cast(unsigned, a), ub = __builtin_bit_cast(unsigned, b);
    if constexpr (H == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(ua, ub, false, false);
        a = __builtin_bit_cast(float, (unsigned)r[0]);
        b = __builtin_bit_cast(float, (unsigned)r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(ua, ub, false, false);
        a = __builtin_bit_cast(float, (unsigned)r[0]);
        b = __builtin_bit_cast(float, (unsigned)r[1]);
    }
}

// a..d += sign * (their value on lane ^ H), H in {1, 2, 4, 8} (the stage of fwht_stage<H> with own and partner
// exchanged).  The leading s_nop covers the VALU write -> DPP read hazard of the first instruction; the others read
// registers written at least two instructions earlier.  H = 4 is a half-row mirror into temporaries, then a quad
// reversal inside the FMA (7 - (l ^ 3) = l ^ 4 within 8 lanes).
#define EXL3_FMAC_DPP(d, s, g, ctl) "v_fmac_f32_dpp %" #d ", %" #s ", %" #g " " ctl " row_mask:0xf bank_mask:0xf\n\t"
#define EXL3_FMAC_DPP4(ctl)                                                                                     \
    "s_nop 1\n\t" EXL3_FMAC_DPP(0, 0, 4, ctl) EXL3_FMAC_DPP(1, 1, 4, ctl) EXL3_FMAC_DPP(2, 2, 4, ctl)             \
        EXL3_FMAC_DPP(3, 3, 4, ctl)
template <int H>
__device__ __forceinline__ void fmac_dpp4(float &a, float &b, float &c, float &d, float sign) {
    if constexpr (H == 4) {
        float t0, t1, t2, t3;
        asm("s_nop 1\n\t"
            "v_mov_b32_dpp %4, %0 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
            "v_mov_b32_dpp %5, %1 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
            "v_mov_b32_dpp %6, %2 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
            "v_mov_b32_dpp %7, %3 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
            EXL3_FMAC_DPP(0, 4, 8, "quad_perm:[3,2,1,0]") EXL3_FMAC_DPP(1, 5, 8, "quad_perm:[3,2,1,0]")
            EXL3_FMAC_DPP(2, 6, 8, "quad_perm:[3,2,1,0]") EXL3_FMAC_DPP(3, 7, 8, "quad_perm:[3,2,1,0]")
            : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3)
            : "v"(sign));
    } else if constexpr (H == 1) {
        asm(EXL3_FMAC_DPP4("quad_perm:[1,0,3,2]") : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "v"(sign));
    } else if constexpr (H == 2) {
        asm(EXL3_FMAC_DPP4("quad_perm:[2,3,0,1]") : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "v"(sign));
    } else {
        static_assert(H == 8, "a lane bit of a 16-lane row");
        asm(EXL3_FMAC_DPP4("row_ror:8") : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "v"(sign));
    }
}
#undef EXL3_FMAC_DPP4
#undef EXL3_FMAC_DPP

// IN_RELAID: the input already stands where fwht_relaid_col puts a result (an elementwise function of an earlier
// relaid transform); a third swap keeps the stage order 6, 5, 4, and the results land at fwht_relaid2_col instead.
template <int R, bool IN_RELAID = false>
__device__ __forceinline__ void fwht128_wave_rows_relaid(float (&v0)[R], float (&v1)[R], int lane) {
    static_assert(R % 2 == 0, "rows in pairs");
    auto butterfly = [&](int i) {
        const float a = v0[i], b = v1[i];
        v0[i] = a + b;
        v1[i] = a - b;
    };
    if constexpr (IN_RELAID) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            permlane_swap_pair<32>(v0[i], v1[i]);
            butterfly(i);
        }
    } else {
#pragma unroll
        for (int i = 0; i < R; i++) butterfly(i);
    }
#pragma unroll
    for (int i = 0; i < R; i++) {
        permlane_swap_pair<IN_RELAID ? 16 : 32>(v0[i], v1[i]);
        butterfly(i);
    }
#pragma unroll
    for (int i = 0; i < R; i++) {
        permlane_swap_pair<IN_RELAID ? 32 : 16>(v0[i], v1[i]);
        butterfly(i);
    }
    const float s8 = lane_sign<8>(lane), s4 = lane_sign<4>(lane), s2 = lane_sign<2>(lane), s1 = lane_sign<1>(lane);
#pragma unroll
    for (int i = 0; i < R; i += 2) fmac_dpp4<8>(v0[i], v1[i], v0[i + 1], v1[i + 1], s8);
#pragma unroll
    for (int i = 0; i < R; i += 2) fmac_dpp4<4>(v0[i], v1[i], v0[i + 1], v1[i + 1], s4);
#pragma unroll
    for (int i = 0; i < R; i += 2) fmac_dpp4<2>(v0[i], v1[i], v0[i + 1], v1[i + 1], s2);
#pragma unroll
    for (int i = 0; i < R; i += 2) fmac_dpp4<1>(v0[i], v1[i], v0[i + 1], v1[i + 1], s1);
}

// Where fwht128_wave_rows_relaid<R, true> leaves y[j]: slot for bit 4, lane bit 5 for bit 5, lane bit 4 for bit 6.
__device__ __forceinline__ int fwht_relaid2_col(int lane, int slot) {
    return (lane & 15) | (slot << 4) | (lane & 32) | ((lane & 16) << 2);
}

constexpr float HAD_SCALE = 0.08838834764831845f;

// Sum over s = 0..S-1 (in that order) of the f32 planes p + s * stride at (lane, lane + 64).  Loads go out eight
// planes at a time before any add: a loop that adds as it loads waits out one memory round trip per plane.
// BYPASS reads with system-scope atomic loads (data another workgroup wrote through to memory).
template <bool BYPASS>
__device__ __forceinline__ void sum_planes(const float *p, size_t stride, int S, int lane, float &v0, float &v1) {
    constexpr int CH = 8;
    v0 = v1 = 0.f;
    for (int s0 = 0; s0 < S; s0 += CH) {
        float t0[CH], t1[CH];
#pragma unroll
        for (int q = 0; q < CH; q++) {
            const float *pp = p + (size_t)min(s0 + q, S - 1) * stride;
            if constexpr (BYPASS) {
                t0[q] = __hip_atomic_load(pp + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                t1[q] = __hip_atomic_load(pp + lane + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            } else {
                t0[q] = pp[lane];
                t1[q] = pp[lane + 64];
            }
        }
#pragma unroll
        for (int q = 0; q < CH; q++) {
            const bool in = s0 + q < S;
            v0 += in ? t0[q] : 0.f;
            v1 += in ? t1[q] : 0.f;
        }
    }
}

// ------------------------------------------------------------------------------------------------------------
// Activation dtypes at the boundary.
enum DType : int { DT_F16 = 0, DT_BF16 = 1, DT_F32 = 2 };

template <int DT>
__device__ __forceinline__ float load_act(const void *p, size_t i) {
    if constexpr (DT == DT_F16) return __half2float(reinterpret_cast<const __half *>(p)[i]);
    else if constexpr (DT == DT_BF16) return __bfloat162float(reinterpret_cast<const __hip_bfloat16 *>(p)[i]);
    else return reinterpret_cast<const float *>(p)[i];
}

template <int DT>
__device__ __forceinline__ void store_act(void *p, size_t i, float v) {
    if constexpr (DT == DT_F16) reinterpret_cast<__half *>(p)[i] = __float2half_rn(v);
    else if constexpr (DT == DT_BF16) reinterpret_cast<__hip_bfloat16 *>(p)[i] = __float2bfloat16(v);
    else reinterpret_cast<float *>(p)[i] = v;
}

__device__ __forceinline__ float f16r(float v) { return __half2float(__float2half_rn(v)); }

// v rounded to an activation dtype and back.
__device__ __forceinline__ float round_act(int dt, float v) {
    if (dt == DT_F16) return __half2float(__float2half_rn(v));
    if (dt == DT_BF16) return __bfloat162float(__float2bfloat16(v));
    return v;
}

// Element i of an f16 / bf16 / f32 array as f32.
__device__ __forceinline__ float load_any(const void *p, int dt, size_t i) {
    if (dt == DT_F16) return load_act<DT_F16>(p, i);
    if (dt == DT_BF16) return load_act<DT_BF16>(p, i);
    return load_act<DT_F32>(p, i);
}

// SiLU of the routed chain's mid: g * sigmoid(g), evaluated on exp(-|g|) so neither branch overflows (the
// reference's mid uses the same split, DOWN_FUSED_SOURCE, src/exl3/expert_exl3_kernels.zig:1838-1925).
__device__ __forceinline__ float silu(float g) {
    const float e = __expf(-fabsf(g));
    const float s = g >= 0.f ? 1.f / (1.f + e) : e / (1.f + e);
    return g * s;
}

// The gated shared expert's term T(sigmoid(gate) * shared) in dtype T = dt, rounding where MLX's Sigmoid and
// Multiply round in T (REDUCE_GATED_SHARED_SOURCE, beamivalice/sushi src/exl3/expert_exl3_kernels.zig:2410-2431):
// ex = T(exp|g|), rc = T(1 / T(1 + ex)), sig = g < 0 ? rc : T(1 - rc).  exp runs in f64 and is rounded to f32 first.
__device__ __forceinline__ float gated_shared(int dt, float g, float shared) {
    const float ex = round_act(dt, (float)exp((double)fabsf(g)));
    const float rc = round_act(dt, 1.0f / round_act(dt, 1.0f + ex));
    const float sig = g < 0.0f ? rc : round_act(dt, 1.0f - rc);
    return round_act(dt, sig * shared);
}

__device__ __forceinline__ float h2f(uint16_t b) { return __half2float(__ushort_as_half(b)); }

}  // namespace exl3
