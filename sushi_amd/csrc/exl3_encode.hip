// Trellis encoder search on the GPU: the two-pass tail-biting Viterbi of src/encoder/encode.zig:170-309
// (`Encoder.encodeTile` / `packStates`), one 16x16 tile per search, T tiles per workgroup.
//
// Per step the search scores every codeword of the window once per tile: cw = (fresh << kr) | e over the
// 2^(w - k_next) edges e (the bits the next codeword keeps) and the 2^k_next fresh high bits, error
// fma(value(cw) - x, value(cw) - x, cost[cw >> k]) in f32 against the f16 path cost of its predecessor, and keeps per
// edge the first minimum as an f16 cost and a one-byte backpointer.  The arithmetic is the reference's, so the codes
// are the same: f32 squared error fused with the predecessor's cost, f16 path costs clamped at 65504, first minimum.
//
// Layout: the workgroup's threads own edges; each thread decodes a codeword once and scores it for all T tiles of the
// workgroup, so the decode is shared.  The two cost rows of every tile live in LDS (T x 2 x 2^(w - kmin) halves); the
// backpointers (256 x 2^(w - kmin) bytes per tile) go to the caller's workspace, one slot per workgroup, and are
// walked back by one lane per tile.  Codeword values are decoded on the fly (decode1), bit-exact with the engine's.
#include "exl3_kernels.h"

// The f64 squared error is summed term by term as the reference does; no multiply-add contraction in this file
// (the path costs' fused multiply-add is written out as fmaf).
#pragma clang fp contract(off)

namespace exl3 {

namespace {

constexpr int ENC_THREADS = 512;
constexpr float H_INF = 65504.0f;

__device__ __forceinline__ int fresh_bits(int n, int t) {
    return (((t + 1) * n) >> 4) - ((t * n) >> 4);
}

// tensorCorePerm (src/exl3/expert_exl3.zig:379-398): trellis index i -> row-major tile position.
__device__ __forceinline__ int tensor_core_perm(int i) {
    const int lane = i >> 3, j = i & 7;
    const int r0 = (lane & 3) * 2, c0 = lane >> 2;
    const int r = r0 + (j & 1) + ((j & 2) ? 8 : 0);
    return r * 16 + c0 + (j >= 4 ? 8 : 0);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) { return __half_as_ushort(__float2half_rn(v)); }
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// One step of the search for all T tiles: scores every codeword, writes each edge's minimum and backpointer.
template <int FAM, int T>
__device__ __forceinline__ void search_step(int step, int ri, int n, int w, const DecodeK &dk, const float *xs,
                                            const uint16_t *prev, uint16_t *curr, uint8_t *back, size_t back_tile,
                                            int stride, bool pinned, const int *pin) {
    const int k = fresh_bits(n, ri);
    const int k_next = fresh_bits(n, (ri + 1) & 255);
    const int kr = w - k_next;
    const int edges = 1 << kr;
    const int kk = 1 << k_next;
    float target[T];
#pragma unroll
    for (int t = 0; t < T; t++) target[t] = xs[t * 256 + ri];
    uint8_t *row = back + (size_t)ri * stride;
    for (int e = threadIdx.x; e < edges; e += ENC_THREADS) {
        float best[T];
        int bf[T];
#pragma unroll
        for (int t = 0; t < T; t++) { best[t] = H_INF; bf[t] = 0; }
        for (int fresh = 0; fresh < kk; fresh++) {
            const uint32_t cw = ((uint32_t)fresh << kr) | (uint32_t)e;
            const uint32_t pred = cw >> k;
            const float v = __half2float(decode1<FAM>(cw, dk));
#pragma unroll
            for (int t = 0; t < T; t++) {
                const float dh = v - target[t];
                float err;
                if (step == 0) {
                    if (pinned && (int)pred != pin[t]) {
                        err = H_INF;
                    } else {
                        const float sq = dh * dh;
                        err = sq < H_INF ? sq : H_INF;
                    }
                } else {
                    err = __builtin_fmaf(dh, dh, f16_bits_to_f32(prev[t * 2 * stride + pred]));
                }
                if (err < best[t]) { best[t] = err; bf[t] = fresh; }
            }
        }
#pragma unroll
        for (int t = 0; t < T; t++) {
            curr[t * 2 * stride + e] = f32_to_f16_bits(best[t]);
            row[t * back_tile + e] = (uint8_t)bf[t];
        }
    }
}

template <int FAM, int T>
__global__ __launch_bounds__(ENC_THREADS) void encode_search_kernel(const float *__restrict__ tiles, int64_t count,
                                                                    int n, int w, DecodeK dk,
                                                                    uint16_t *__restrict__ packed,
                                                                    double *__restrict__ sse,
                                                                    float *__restrict__ recon,
                                                                    uint8_t *__restrict__ back_ws, int stride) {
    extern __shared__ __align__(16) unsigned char enc_lds[];
    // LDS: cost rows [T][2][stride] u16, then x [T][256] f32, paths [T][256] u16, packed words [T][64] u32,
    // the final-edge reduction [ENC_THREADS / 64][T] u32 and the pins [T].
    uint16_t *costs = reinterpret_cast<uint16_t *>(enc_lds);
    float *xs = reinterpret_cast<float *>(enc_lds + (size_t)T * 2 * stride * 2);
    uint16_t *path = reinterpret_cast<uint16_t *>(xs + T * 256);
    uint32_t *words = reinterpret_cast<uint32_t *>(path + T * 256);
    uint32_t *red = words + T * 64;
    int *pin = reinterpret_cast<int *>(red + (ENC_THREADS / 64) * T);

    const size_t back_tile = (size_t)256 * stride;
    uint8_t *back = back_ws + (size_t)blockIdx.x * T * back_tile;
    const int64_t batches = (count + T - 1) / T;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    for (int64_t b = blockIdx.x; b < batches; b += gridDim.x) {
        const int64_t tile0 = b * T;
        // Inputs, permuted into trellis order (tensorCorePerm): x[i] = tile[perm[i]].
        for (int i = tid; i < T * 256; i += ENC_THREADS) {
            const int t = i >> 8, j = i & 255;
            const int64_t tile = tile0 + t < count ? tile0 + t : count - 1;
            xs[i] = tiles[tile * 256 + tensor_core_perm(j)];
        }
        __syncthreads();
        for (int pass = 0; pass < 2; pass++) {
            const int roll = pass == 0 ? 128 : 0;
            int cur = 0;
            for (int step = 0; step < 256; step++) {
                const int ri = (step + roll) & 255;
                search_step<FAM, T>(step, ri, n, w, dk, xs, costs + cur * stride, costs + (cur ^ 1) * stride, back,
                                    back_tile, stride, pass == 1, pin);
                cur ^= 1;
                __syncthreads();
            }
            // The edge the traceback starts from: pass 0 the first cheapest final edge (an f16 cost is >= 0, so its
            // bits order as the values do and (bits << 16 | edge) orders by cost, then edge); pass 1 the pin.
            if (pass == 0) {
                const int final_edges = 1 << (w - fresh_bits(n, 0));
#pragma unroll
                for (int t = 0; t < T; t++) {
                    uint32_t key = 0xFFFFFFFFu;
                    for (int e = tid; e < final_edges; e += ENC_THREADS) {
                        const uint32_t c = costs[t * 2 * stride + cur * stride + e];
                        const uint32_t kv = (c << 16) | (uint32_t)e;
                        key = kv < key ? kv : key;
                    }
                    for (int off = 32; off > 0; off >>= 1) {
                        const uint32_t o = (uint32_t)__shfl_xor((int)key, off);
                        key = o < key ? o : key;
                    }
                    if (lane == 0) red[wave * T + t] = key;
                }
                __syncthreads();
                if (tid < T) {
                    uint32_t key = 0xFFFFFFFFu;
                    for (int v = 0; v < ENC_THREADS / 64; v++) key = red[v * T + tid] < key ? red[v * T + tid] : key;
                    pin[tid] = (int)(key & 0xFFFFu);
                }
                __syncthreads();
            }
            // Traceback, one lane per tile.
            if (tid < T) {
                const int t = tid;
                int edge = pin[t];
                const uint8_t *bt = back + (size_t)t * back_tile;
                for (int step_i = 255; step_i >= 0; step_i--) {
                    const int ri = (step_i + roll) & 255;
                    const int k = fresh_bits(n, ri);
                    const int kr = w - fresh_bits(n, (ri + 1) & 255);
                    const int state = ((int)bt[(size_t)ri * stride + edge] << kr) | edge;
                    edge = state >> k;
                    if (pass == 1) {
                        path[t * 256 + ri] = (uint16_t)state;
                    } else if (ri == 0) {
                        break;
                    }
                }
                pin[t] = edge;
            }
            __syncthreads();
        }
        // packStates: step t's fresh k bits (the state's low bits), MSB first, end at bitEnd(t) of a stream read as
        // 32-bit words whose bit 31 comes first; stored little-endian, a word is the halfword pair (lo, hi).
        for (int i = tid; i < T * 64; i += ENC_THREADS) words[i] = 0u;
        __syncthreads();
        for (int i = tid; i < T * 256; i += ENC_THREADS) {
            const int t = i >> 8, s = i & 255;
            const int k = fresh_bits(n, s);
            const int end = ((s + 1) * n) >> 4;
            const uint32_t field = (uint32_t)path[i] & ((1u << k) - 1u);
            const int p0 = end - k;
            const int j0 = p0 >> 5, o0 = p0 & 31;
            if (o0 + k <= 32) {
                atomicOr(&words[t * 64 + j0], field << (32 - o0 - k));
            } else {
                const int hi = 32 - o0;  // bits in the first word
                atomicOr(&words[t * 64 + j0], field >> (k - hi));
                atomicOr(&words[t * 64 + j0 + 1], field << (32 - (k - hi)));
            }
        }
        __syncthreads();
        for (int i = tid; i < T * (n / 2); i += ENC_THREADS) {
            const int t = i / (n / 2), j = i % (n / 2);
            if (tile0 + t < count) {
                const uint32_t v = words[t * 64 + j];
                packed[(tile0 + t) * n + 2 * j] = (uint16_t)(v & 0xFFFFu);
                packed[(tile0 + t) * n + 2 * j + 1] = (uint16_t)(v >> 16);
            }
        }
        // The values the decoder will produce, back in row-major tile order.
        if (recon != nullptr)
            for (int i = tid; i < T * 256; i += ENC_THREADS) {
                const int t = i >> 8, j = i & 255;
                if (tile0 + t < count)
                    recon[(tile0 + t) * 256 + tensor_core_perm(j)] = __half2float(decode1<FAM>(path[i], dk));
            }
        // The path's squared error in f64, summed in trellis order as the reference does.
        if (sse != nullptr && tid < T && tile0 + tid < count) {
            double acc = 0.0;
            for (int i = 0; i < 256; i++) {
                const double d = (double)xs[tid * 256 + i] - (double)__half2float(decode1<FAM>(path[tid * 256 + i], dk));
                acc += d * d;
            }
            sse[tile0 + tid] = acc;
        }
        __syncthreads();
    }
}

template <int FAM, int T>
hipError_t launch_encode(const EncodeArgs &a, hipStream_t s) {
    const size_t lds = encode_lds_bytes(T, a.stride);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&encode_search_kernel<FAM, T>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((encode_search_kernel<FAM, T>), dim3((unsigned)a.grid), dim3(ENC_THREADS), lds, s, a.tiles,
                       a.count, a.n, a.w, a.k, a.packed, a.sse, a.recon, a.back, a.stride);
    return hipGetLastError();
}

template <int FAM>
hipError_t launch_encode_t(const EncodeArgs &a, hipStream_t s) {
    switch (a.tiles_per_wg) {
    case 16: return launch_encode<FAM, 16>(a, s);
    case 8: return launch_encode<FAM, 8>(a, s);
    case 4: return launch_encode<FAM, 4>(a, s);
    case 2: return launch_encode<FAM, 2>(a, s);
    default: return launch_encode<FAM, 1>(a, s);
    }
}

}  // namespace

size_t encode_lds_bytes(int tiles_per_wg, int stride) {
    const size_t t = (size_t)tiles_per_wg;
    return t * 2 * stride * 2 + t * 256 * 4 + t * 256 * 2 + t * 64 * 4 + (ENC_THREADS / 64) * t * 4 + t * 4;
}

hipError_t run_encode(int fam, const EncodeArgs &a, hipStream_t s) {
    if (a.count == 0) return hipSuccess;
    switch (fam) {
    case FAM_MCG: return launch_encode_t<FAM_MCG>(a, s);
    case FAM_MUL1: return launch_encode_t<FAM_MUL1>(a, s);
    default: return launch_encode_t<FAM_3INST>(a, s);
    }
}

}  // namespace exl3
