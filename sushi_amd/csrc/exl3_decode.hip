// Trellis decode kernels: a codeword list (the exhaustive 65,536-codeword check) and the dense reconstruction
// of one projection's inner matrix ("dequantized fp16 weights", bit-exact with reconstructInner,
// beamivalice/sushi src/exl3/expert_exl3.zig:416-438).  The reconstruction runs the decoder the GEMV and the GEMM
// multiply with: the lane reader and lane decoder at the rates they serve (16, 24, 32, 40, 48, 64), the generic
// per-codeword reader at every other rate, so the weights it returns are the hot path's own; a per-tile-rate bank
// through the tiled reader and decoder.
#include "exl3_kernels.h"
#include "exl3_lane_decode.h"

namespace exl3 {

template <int FAM>
__global__ void decode_codewords_kernel(const uint16_t *__restrict__ cw, int64_t count, DecodeK k,
                                        uint16_t *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const uint32_t c = cw[i];
    if constexpr (FAM == FAM_PAIR) {
        uint32_t h = decode_pair_unscaled(c, k);
        __half w0 = __hmul(__ushort_as_half((unsigned short)(h & 0xFFFFu)), __float2half(4096.0f));
        __half w1 = __hmul(__ushort_as_half((unsigned short)(h >> 16)), __float2half(4096.0f));
        out[2 * i] = __half_as_ushort(w0);
        out[2 * i + 1] = __half_as_ushort(w1);
    } else {
        __half w = decode1<FAM>(c, k);
        if constexpr (family_scaled<FAM>()) w = __hmul(w, __float2half(4096.0f));
        out[i] = __half_as_ushort(w);
    }
}

// One thread per weight pair (t, t+1), t even; 128 threads per tile.  grid.x = tiles.
template <int FAM>
__global__ void reconstruct_inner_kernel(const uint16_t *__restrict__ trellis, int it, int ot, int n, DecodeK k,
                                         uint16_t *__restrict__ out) {
    const int tile = blockIdx.x;
    const int tk = tile / ot, tn = tile % ot;
    const uint32_t *words = reinterpret_cast<const uint32_t *>(trellis + (size_t)tile * n);
    const int p = threadIdx.x;  // pair index 0..127
    const int t = 2 * p;
    const uint32_t c0 = codeword_at(words, n, t);
    const uint32_t c1 = codeword_at(words, n, t + 1);
    uint32_t h = decode_pair_h2<FAM>(c0, c1, k);
    __half w0 = __ushort_as_half((unsigned short)(h & 0xFFFFu));
    __half w1 = __ushort_as_half((unsigned short)(h >> 16));
    if constexpr (family_scaled<FAM>()) {
        w0 = __hmul(w0, __float2half(4096.0f));
        w1 = __hmul(w1, __float2half(4096.0f));
    }
    // tensorCorePerm: t = 8T + i, T = 4j + q; rows {2q, 2q+1, 2q+8, 2q+9}[i%4], col j + 8*(i>=4).
    const int T = t >> 3, i = t & 7, q = T & 3, j = T >> 2;
    const int row = 2 * q + ((i & 2) ? 8 : 0) + (i & 1);
    const int col = j + ((i & 4) ? 8 : 0);
    const size_t of = (size_t)ot * 16;
    const size_t base = ((size_t)tk * 16 + row) * of + (size_t)tn * 16 + col;
    out[base] = __half_as_ushort(w0);
    out[base + of] = __half_as_ushort(w1);  // weight t+1 is the next row (i odd), same column
}

// Lane-reader rates: one wave per 8 consecutive tiles of the pack order, lane 8o + j reading chunk j of tile o with
// load_lane_words_u (the wave-uniform start of the 8 tiles plus the lane's tile offset, as the GEMV and the GEMM
// address a k-tile row of an output group) and decoding it with decode_weights, hash / pair values then times 4096
// (the weights themselves; the matrix cores take the values unscaled and their finishes apply the 4096).  Pair
// i = 4qq + p of the lane holds rows 2qq + 8(p & 1) + {0, 1} of column j (p < 2) or j + 8 (p >= 2).  A tail wave's
// lanes past the last tile re-read it and store nothing.
constexpr int RL_WAVES = 4;
template <int FAM, int N, bool MASKED>
__global__ __launch_bounds__(64 * RL_WAVES) void reconstruct_lane_kernel(const uint16_t *__restrict__ trellis,
                                                                         int tiles, int ot, DecodeK k,
                                                                         uint16_t *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int wv = blockIdx.x * RL_WAVES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t0 = wv * 8;
    if (t0 >= tiles) return;
    const int o = lane >> 3, j = lane & 7;
    const int t = min(t0 + o, tiles - 1);
    uint32_t A[LaneBits<N>::AW];
    load_lane_words_u<N>(reinterpret_cast<const uint32_t *>(trellis + (size_t)t0 * N), (uint32_t)((t - t0) * N) >> 1,
                         j, A);
    uint32_t w[16];
    decode_weights<FAM, N, MASKED>(A, k, w);
    if constexpr (family_scaled<FAM>()) {
#pragma unroll
        for (int i = 0; i < 16; i++) w[i] = scale_h2_4096(w[i]);
    }
    if (t0 + o >= tiles) return;
    const int tk = t / ot, tn = t - tk * ot;
    const size_t of = (size_t)ot * 16;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int qq = i >> 2, p = i & 3;
        const size_t at = ((size_t)tk * 16 + 2 * qq + 8 * (p & 1)) * of + (size_t)tn * 16 + j + 8 * (p >> 1);
        out[at] = (uint16_t)(w[i] & 0xFFFFu);
        out[at + of] = (uint16_t)(w[i] >> 16);
    }
}

template <int FAM, int N>
static hipError_t launch_reconstruct_lane(const uint16_t *trellis, int tiles, int ot, const DecodeK &k, uint16_t *out,
                                          hipStream_t s) {
    const int waves = (tiles + 7) / 8;
    const dim3 grid((unsigned)((waves + RL_WAVES - 1) / RL_WAVES));
    if (k.wmask != 0xFFFFu)
        hipLaunchKernelGGL((reconstruct_lane_kernel<FAM, N, true>), grid, dim3(64 * RL_WAVES), 0, s, trellis, tiles, ot,
                           k, out);
    else
        hipLaunchKernelGGL((reconstruct_lane_kernel<FAM, N, false>), grid, dim3(64 * RL_WAVES), 0, s, trellis, tiles,
                           ot, k, out);
    return hipGetLastError();
}

// One expert of a per-tile-rate bank: one wave per segment (8 tiles of one k-tile row), lane 8o + j decoding chunk j
// of tile o at that tile's own rate with the GEMV's tiled reader and decoder.
template <int FAM, bool MASKED>
__global__ __launch_bounds__(64 * RL_WAVES) void reconstruct_tiled_kernel(const uint16_t *__restrict__ trellis,
                                                                          const uint32_t *__restrict__ seg_off,
                                                                          const uint8_t *__restrict__ seg_k1,
                                                                          int expert, int it, int ot, DecodeK ka,
                                                                          DecodeK kb, uint16_t *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int sg = blockIdx.x * RL_WAVES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // segment of the expert
    const int segs = ot / 8;
    if (sg >= it * segs) return;
    const int o = lane >> 3, j = lane & 7;
    const int tk = sg / segs, s8 = sg - tk * segs;
    const size_t seg = ((size_t)expert * it + tk) * segs + s8;
    const uint32_t m = seg_k1[seg];
    const bool k1 = ((m >> o) & 1u) != 0;
    const uint32_t lw = 16u * (uint32_t)o - 8u * (uint32_t)__builtin_popcount(m & ((1u << o) - 1u));
    uint32_t A[3];
    load_lane_words_tiled(reinterpret_cast<const uint32_t *>(trellis) + seg_off[seg], lw, j, k1, A);
    uint32_t w[16];
    decode_weights_tiled<FAM, MASKED>(A, k1, tiled_constants(k1, ka, kb), w);
    if constexpr (family_scaled<FAM>()) {
#pragma unroll
        for (int i = 0; i < 16; i++) w[i] = scale_h2_4096(w[i]);
    }
    const int tn = s8 * 8 + o;
    const size_t of = (size_t)ot * 16;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int qq = i >> 2, p = i & 3;
        const size_t at = ((size_t)tk * 16 + 2 * qq + 8 * (p & 1)) * of + (size_t)tn * 16 + j + 8 * (p >> 1);
        out[at] = (uint16_t)(w[i] & 0xFFFFu);
        out[at + of] = (uint16_t)(w[i] >> 16);
    }
}

template <int FAM>
static hipError_t launch_reconstruct_tiled(const uint16_t *trellis, const uint32_t *seg_off, const uint8_t *seg_k1,
                                           int expert, int it, int ot, const DecodeK &ka, const DecodeK &kb,
                                           uint16_t *out, hipStream_t s) {
    const int waves = it * (ot / 8);
    const dim3 grid((unsigned)((waves + RL_WAVES - 1) / RL_WAVES));
    if (kb.wmask != 0xFFFFu)
        hipLaunchKernelGGL((reconstruct_tiled_kernel<FAM, true>), grid, dim3(64 * RL_WAVES), 0, s, trellis, seg_off,
                           seg_k1, expert, it, ot, ka, kb, out);
    else
        hipLaunchKernelGGL((reconstruct_tiled_kernel<FAM, false>), grid, dim3(64 * RL_WAVES), 0, s, trellis, seg_off,
                           seg_k1, expert, it, ot, ka, kb, out);
    return hipGetLastError();
}

hipError_t run_reconstruct_tiled(int fam, const uint16_t *trellis, const uint32_t *seg_off, const uint8_t *seg_k1,
                                 int expert, int it, int ot, const DecodeK &ka, const DecodeK &kb, uint16_t *out,
                                 hipStream_t s) {
    if (it * ot == 0) return hipSuccess;
    switch (fam) {
    case FAM_MCG: return launch_reconstruct_tiled<FAM_MCG>(trellis, seg_off, seg_k1, expert, it, ot, ka, kb, out, s);
    case FAM_HASH: return launch_reconstruct_tiled<FAM_HASH>(trellis, seg_off, seg_k1, expert, it, ot, ka, kb, out, s);
    case FAM_3INST: return launch_reconstruct_tiled<FAM_3INST>(trellis, seg_off, seg_k1, expert, it, ot, ka, kb, out, s);
    default: return hipErrorInvalidValue;
    }
}

template <int FAM>
static hipError_t launch_decode_codewords(const uint16_t *cw, int64_t count, const DecodeK &k, uint16_t *out,
                                          hipStream_t s) {
    const int bs = 256;
    const int64_t grid = (count + bs - 1) / bs;
    hipLaunchKernelGGL(decode_codewords_kernel<FAM>, dim3((unsigned)grid), dim3(bs), 0, s, cw, count, k, out);
    return hipGetLastError();
}

hipError_t run_decode_codewords(int fam, const uint16_t *cw, int64_t count, const DecodeK &k, uint16_t *out,
                                hipStream_t s) {
    if (count <= 0) return hipSuccess;
    switch (fam) {
    case FAM_MCG: return launch_decode_codewords<FAM_MCG>(cw, count, k, out, s);
    case FAM_MUL1: return launch_decode_codewords<FAM_MUL1>(cw, count, k, out, s);
    case FAM_HASH: return launch_decode_codewords<FAM_HASH>(cw, count, k, out, s);
    case FAM_PAIR: return launch_decode_codewords<FAM_PAIR>(cw, count, k, out, s);
    default: return launch_decode_codewords<FAM_3INST>(cw, count, k, out, s);
    }
}

template <int FAM>
static hipError_t launch_reconstruct(const uint16_t *trellis, int it, int ot, int n, const DecodeK &k, uint16_t *out,
                                     hipStream_t s) {
    switch (n) {
    case 16: return launch_reconstruct_lane<FAM, 16>(trellis, it * ot, ot, k, out, s);
    case 24: return launch_reconstruct_lane<FAM, 24>(trellis, it * ot, ot, k, out, s);
    case 32: return launch_reconstruct_lane<FAM, 32>(trellis, it * ot, ot, k, out, s);
    case 40: return launch_reconstruct_lane<FAM, 40>(trellis, it * ot, ot, k, out, s);
    case 48: return launch_reconstruct_lane<FAM, 48>(trellis, it * ot, ot, k, out, s);
    case 64: return launch_reconstruct_lane<FAM, 64>(trellis, it * ot, ot, k, out, s);
    default: break;
    }
    hipLaunchKernelGGL(reconstruct_inner_kernel<FAM>, dim3((unsigned)(it * ot)), dim3(128), 0, s, trellis, it, ot, n,
                       k, out);
    return hipGetLastError();
}

hipError_t run_reconstruct_inner(int fam, const uint16_t *trellis, int it, int ot, int n, const DecodeK &k,
                                 uint16_t *out, hipStream_t s) {
    if (it * ot == 0) return hipSuccess;
    switch (fam) {
    case FAM_MCG: return launch_reconstruct<FAM_MCG>(trellis, it, ot, n, k, out, s);
    case FAM_MUL1: return launch_reconstruct<FAM_MUL1>(trellis, it, ot, n, k, out, s);
    case FAM_HASH: return launch_reconstruct<FAM_HASH>(trellis, it, ot, n, k, out, s);
    case FAM_PAIR: return launch_reconstruct<FAM_PAIR>(trellis, it, ot, n, k, out, s);
    default: return launch_reconstruct<FAM_3INST>(trellis, it, ot, n, k, out, s);
    }
}

}  // namespace exl3
