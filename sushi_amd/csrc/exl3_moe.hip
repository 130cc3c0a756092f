// MoE chain tail, routing and layout kernels, plus the GEMV family dispatcher.
//
//  * moe_reduce_kernel: the decode chain's score-weighted reduce (REDUCE_SOURCE / REDUCE_SHARED_SOURCE,
//    beamivalice/sushi src/exl3/expert_exl3_kernels.zig:2338-2406): per (row, 128-block), each routed slot's down
//    plane is summed over its k splits, FWHT-128'd and scaled by svh, then weighted by its score; the routed sum is
//    rounded to the output dtype before a shared expert is added, as the reference does.
//  * route_topk_kernel: moeRoutingChainOn (src/moe_router.zig:22-62).
//  * tile_major_kernel: layout.tileMajor / tileMajorInverse (src/exl3/layout.zig:139-158).
#include "exl3_kernels.h"

namespace exl3 {

hipError_t run_gemv(int fam, int prologue, const GemvArgs &a, hipStream_t s) {
    switch (fam) {
    case FAM_MCG: return run_gemv_fam_FAM_MCG(prologue, a, s);
    case FAM_MUL1: return run_gemv_fam_FAM_MUL1(prologue, a, s);
    case FAM_HASH: return run_gemv_fam_FAM_HASH(prologue, a, s);
    case FAM_PAIR: return run_gemv_fam_FAM_PAIR(prologue, a, s);
    default: return run_gemv_fam_FAM_3INST(prologue, a, s);
    }
}

hipError_t run_moe_chain(int fam, const GemvArgs &a1, const GemvArgs &a2, hipStream_t s) {
    switch (fam) {
    case FAM_MCG: return run_moe_chain_fam_FAM_MCG(a1, a2, s);
    case FAM_MUL1: return run_moe_chain_fam_FAM_MUL1(a1, a2, s);
    case FAM_HASH: return run_moe_chain_fam_FAM_HASH(a1, a2, s);
    case FAM_PAIR: return run_moe_chain_fam_FAM_PAIR(a1, a2, s);
    default: return run_moe_chain_fam_FAM_3INST(a1, a2, s);
    }
}

int gemv_default_splits(int in, int out, int rows, int groups_times_proj, int max_batches, int target_wgs) {
    // Splits cut k on whole Hadamard blocks.  A split of at most TPW * GEMV_WAVES k-tiles lets every wave issue all
    // of its tile loads before the prologue; up to max_batches such batches per wave are allowed where the grid is
    // large (each workgroup then pays its start-up latency once for more work, the later batches' loads overlapping
    // the decode).  Past that, more splits only add partial traffic unless the grid is still short of one workgroup
    // per CU.
    // With 8 or more rows a workgroup carries enough work per tile that half the workgroup target fills the chip, and
    // every split it saves is one fewer fold arrival per output.
    const int blocks = in / 128;
    const int it = in / 16;
    const long G = (long)(out / 128) * groups_times_proj;
    const long base = target_wgs > 0 ? target_wgs : GEMV_TARGET_WGS;
    const long target = rows >= 8 ? base / 2 : base;
    int best = blocks;
    for (int s = 1; s <= blocks; s++) {
        if (blocks % s) continue;
        if (it / s > TPW * GEMV_WAVES * max_batches) continue;
        best = s;
        if (G * s >= target) break;
    }
    if (target_wgs > 0) return best;
    // A grid that leaves part of its last round of CUs idle (448 workgroups are 1.75 per CU) gives way to the next
    // split count if that fills its rounds better and still leaves every wave two tiles or more: 14336x4096 takes
    // 16 splits (512 workgroups) rather than 14, and 16 rows at 4096x4096 take 256 workgroups rather than 128.
    auto fill = [](long w) { return (double)w / (double)(((w + 255) / 256) * 256); };
    for (int s = best + 1; s <= blocks; s++) {
        if (blocks % s) continue;
        if (it / s < 2 * GEMV_WAVES) break;
        if (fill(G * s) > fill(G * best) + 0.05) best = s;
        break;
    }
    return best;
}

__device__ __forceinline__ void store_out(void *y, int dt, size_t i, float v) {
    if (dt == DT_F16) store_act<DT_F16>(y, i, v);
    else if (dt == DT_BF16) store_act<DT_BF16>(y, i, v);
    else store_act<DT_F32>(y, i, v);
}

__device__ __forceinline__ float round_to(int dt, float v) {
    if (dt == DT_F16) return __half2float(__float2half_rn(v));
    if (dt == DT_BF16) return __bfloat162float(__float2bfloat16(v));
    return v;
}

// One workgroup per (row, RB consecutive 128-blocks): wave w handles items w, w + RW, ... (the slots, and a shared
// expert's term: sum of the slot's k splits, FWHT, svh, score) for all its blocks into LDS, the blocks' loads first
// and their transforms together; then every thread adds the slots of its columns in slot order (the reference's
// order) and finishes.  (One block per workgroup ran 82 us for 2048 rows x 8 slots x 2048 columns: 32768 workgroups
// each reading 4 KiB; a ninth wave for a shared expert's term ran slower than eight waves taking nine items.)  RB = 4
// where that still leaves at least 1024 workgroups, else 1 (a decode batch of 32 rows would get 128).
constexpr int RW = 8;
template <int RB, int SDT>
__global__ __launch_bounds__(64 * RW) void moe_reduce_kernel(ReduceArgs a) {
    const int row = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = min(RB, a.hidden / 128 - (int)blockIdx.x * RB);  // this workgroup's blocks
    const size_t base = (size_t)blockIdx.x * RB * 128;
    extern __shared__ float contrib[];  // [topk (+ 1: a shared expert's term)][RB * 128]
    // RB even: the relaid transform (fewer instructions, same roundings), so svh is read and each result stored at the
    // column the lane then holds; its sign folds into the scale (exact)
    constexpr bool RELAID = RB % 2 == 0;
    const int c0 = RELAID ? fwht_relaid_col(lane, 0) : lane, c1 = RELAID ? fwht_relaid_col(lane, 1) : lane + 64;
    const float hs = RELAID ? fwht_relaid_sign(lane) * HAD_SCALE : HAD_SCALE;
    // The shared expert's term (a one-expert layer's slot: score 1, its own planes of one split): block b on wave
    // (topk + b) % RW, continuing the slots' round robin (as a whole ninth item it doubled one wave's work: 78 us at
    // 2048 rows), so at most one block per wave.  Its loads go out ahead of the slots' (a wave without a block reads
    // an in-bounds address it then ignores): loaded after its wave's slot item, it cost a second memory round trip.
    static_assert(RB <= RW, "one shared block per wave");
    const int bsh = ((wave - a.topk) % RW + RW) % RW;
    const bool has_sh = a.sh_part != nullptr && bsh < nb;
    const float *shp = has_sh ? a.sh_part + (size_t)row * a.hidden + base + bsh * 128 : a.part;
    const uint16_t *shv = has_sh ? a.sh_svh + base + bsh * 128 : a.svh;
    const float sh0 = 0.f + shp[lane], sh1 = 0.f + shp[lane + 64];
    const float shs0 = h2f(shv[lane]), shs1 = h2f(shv[lane + 64]);
    // one slot item per wave when topk <= RW, peeled off the loop: the loop's back edge made the first item's plane
    // loads wait for every load before them, the shared term's included
    auto item = [&](int kk) __attribute__((always_inline)) {
        const int slot = row * a.topk + kk;
        const float *pl = a.part + (size_t)slot * a.splits * a.hidden + base;
        // every load in bounds (a block past this workgroup's last reads its last); the planes first, as they need
        // only the slot: the svh loads wait on the slot's expert id and are needed only after the transform
        float v0[RB], v1[RB], s0[RB], s1[RB];
#pragma unroll
        for (int b = 0; b < RB; b++) {
            const int bb = min(b, nb - 1);
            if (a.splits == 1) {  // sum_planes' sum of one plane (0 + x), without its eight-split batch of loads
                v0[b] = 0.f + pl[bb * 128 + lane];
                v1[b] = 0.f + pl[bb * 128 + lane + 64];
            } else {
                sum_planes<false>(pl + bb * 128, a.hidden, a.splits, lane, v0[b], v1[b]);
            }
        }
        const int e = (int)min(a.slots[slot], (uint32_t)(a.bank_limit - 1));
        const float sc = load_act<SDT>(a.scores, slot);  // one load, no dtype branch to wait at
        const uint16_t *sv = a.svh + (size_t)e * a.hidden + base;
#pragma unroll
        for (int b = 0; b < RB; b++) {
            const int bb = min(b, nb - 1);
            s0[b] = h2f(sv[bb * 128 + c0]);
            s1[b] = h2f(sv[bb * 128 + c1]);
        }
        if constexpr (RELAID) fwht128_wave_rows_relaid<RB>(v0, v1, lane);
        else fwht128_wave_rows<RB>(v0, v1, lane);
#pragma unroll
        for (int b = 0; b < RB; b++)
            if (b < nb) {
                contrib[kk * RB * 128 + b * 128 + c0] = (v0[b] * hs * s0[b]) * sc;
                contrib[kk * RB * 128 + b * 128 + c1] = (v1[b] * hs * s1[b]) * sc;
            }
    };
    if (wave < a.topk) item(wave);
    for (int kk = wave + RW; kk < a.topk; kk += RW) item(kk);
    if (has_sh) {
        float v0 = sh0, v1 = sh1;
        fwht128_wave(v0, v1, lane);
        contrib[a.topk * RB * 128 + bsh * 128 + lane] = (v0 * HAD_SCALE * shs0) * 1.0f;
        contrib[a.topk * RB * 128 + bsh * 128 + lane + 64] = (v1 * HAD_SCALE * shs1) * 1.0f;
    }
    __syncthreads();
    const float g = a.shared && a.gate ? load_any(a.gate, a.y_dtype, row) : 0.f;
    for (int col = threadIdx.x; col < nb * 128; col += 64 * RW) {
        float y = 0.f;
        for (int kk = 0; kk < a.topk; kk++) y += contrib[kk * RB * 128 + col];
        const size_t yo = (size_t)row * a.hidden + base + col;
        if (a.shared) {
            float sh = load_any(a.shared, a.y_dtype, yo);
            if (a.gate) sh = gated_shared(a.y_dtype, g, sh);  // sigmoid(gate) * shared in y's dtype
            y = round_to(a.y_dtype, y) + sh;
        } else if (a.sh_part) {  // as the one-expert layer rounds its output, then as `shared` above
            const float sh = round_to(a.y_dtype, 0.f + contrib[a.topk * RB * 128 + col]);
            y = round_to(a.y_dtype, y) + sh;
        }
        store_out(a.y, a.y_dtype, yo, y);
    }
}

template <int RB>
static void launch_moe_reduce(const ReduceArgs &a, dim3 grid, size_t lds, hipStream_t s) {
    const dim3 block(64 * RW);
    if (a.score_dtype == DT_F16) hipLaunchKernelGGL((moe_reduce_kernel<RB, DT_F16>), grid, block, lds, s, a);
    else if (a.score_dtype == DT_BF16) hipLaunchKernelGGL((moe_reduce_kernel<RB, DT_BF16>), grid, block, lds, s, a);
    else hipLaunchKernelGGL((moe_reduce_kernel<RB, DT_F32>), grid, block, lds, s, a);
}

hipError_t run_moe_reduce(const ReduceArgs &a, hipStream_t s) {
    if (a.topk > kMoeReduceMaxTopk) return hipErrorInvalidValue;
    const int items = a.topk + (a.sh_part ? 1 : 0), blocks = a.hidden / 128;
    if ((long)a.rows * ((blocks + 3) / 4) >= 1024)
        launch_moe_reduce<4>(a, dim3((unsigned)((blocks + 3) / 4), (unsigned)a.rows),
                             (size_t)items * 4 * 128 * sizeof(float), s);
    else
        launch_moe_reduce<1>(a, dim3((unsigned)blocks, (unsigned)a.rows), (size_t)items * 128 * sizeof(float), s);
    return hipGetLastError();
}

// Expert windows for the sorted MoE arm (the grouping moePrefill's sort does, expert_exl3_kernels.zig:2861-2931 with
// sorted_windows.zig:10-165): slot s (expert e = inds[s], clamped below `experts`) gets rank r = the number of slots
// before it with the same expert, and lands in window wbase[e] + r / MOE_WINDOW_ROWS at row r % MOE_WINDOW_ROWS, where
// wbase is the exclusive scan of ceil(count[e] / MOE_WINDOW_ROWS) over experts.  Ranks come from one wave walking the
// slots in order, 64 at a time: a slot's rank is its expert's running count plus the lanes before it in the same
// round with the same expert (found by one ballot per bit of the expert id), so the result does not depend on thread
// timing.
constexpr int WIN_THREADS = 1024;
__global__ __launch_bounds__(WIN_THREADS) void moe_windows_kernel(const uint32_t *__restrict__ inds, int nslots,
                                                                  int experts, uint32_t *__restrict__ win_count,
                                                                  uint32_t *__restrict__ win_expert,
                                                                  uint32_t *__restrict__ win_rows,
                                                                  uint32_t *__restrict__ win_slots) {
    __shared__ uint16_t ex[kMoeWindowMaxSlots];
    __shared__ uint32_t cnt[kMoeWindowMaxExperts];
    __shared__ uint32_t wbase[kMoeWindowMaxExperts];
    __shared__ uint32_t part[WIN_THREADS];
    __shared__ uint32_t fill[kMoeWindowMaxExperts];
    const int tid = threadIdx.x;
    for (int e = tid; e < experts; e += WIN_THREADS) cnt[e] = fill[e] = 0;
    for (int s = tid; s < nslots; s += WIN_THREADS) ex[s] = (uint16_t)min(inds[s], (uint32_t)(experts - 1));
    __syncthreads();
    for (int s = tid; s < nslots; s += WIN_THREADS) atomicAdd(&cnt[ex[s]], 1u);
    __syncthreads();
    // exclusive scan of windows per expert: each thread sums a contiguous run of experts, then a scan of the runs
    const int per = (experts + WIN_THREADS - 1) / WIN_THREADS;
    const int e0 = min(tid * per, experts), e1 = min(e0 + per, experts);
    uint32_t local = 0;
    for (int e = e0; e < e1; e++) local += (cnt[e] + MOE_WINDOW_ROWS - 1) / MOE_WINDOW_ROWS;
    part[tid] = local;
    __syncthreads();
    for (int off = 1; off < WIN_THREADS; off <<= 1) {
        const uint32_t v = tid >= off ? part[tid - off] : 0u;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    uint32_t run = part[tid] - local;
    for (int e = e0; e < e1; e++) {
        wbase[e] = run;
        run += (cnt[e] + MOE_WINDOW_ROWS - 1) / MOE_WINDOW_ROWS;
    }
    if (tid == WIN_THREADS - 1) *win_count = part[tid];
    __syncthreads();
    if (tid < 64) {  // wave 0 ranks the slots in order
        const int lane = tid;
        const int id_bits = experts > 1 ? 32 - __clz(experts - 1) : 0;
        for (int base = 0; base < nslots; base += 64) {
            const int s = base + lane;
            const bool live = s < nslots;
            const int e = live ? (int)ex[s] : 0;
            // The lanes holding this lane's expert: one ballot per bit of the expert id, and the live lanes.
            unsigned long long same = __ballot(live);
            for (int b = 0; b < id_bits; b++) {
                const unsigned long long set = __ballot((e >> b) & 1);
                same &= ((e >> b) & 1) ? set : ~set;
            }
            const unsigned long long below = (1ull << lane) - 1ull;
            const uint32_t before = (uint32_t)__popcll(same & below);
            const bool last = live && (same & ~below & ~(1ull << lane)) == 0ull;
            if (live) {
                const uint32_t rank = fill[e] + before;
                const uint32_t w = wbase[e] + rank / MOE_WINDOW_ROWS, r = rank % MOE_WINDOW_ROWS;
                win_slots[(size_t)w * MOE_WINDOW_ROWS + r] = (uint32_t)s;
                if (r == 0) {
                    win_expert[w] = (uint32_t)e;
                    win_rows[w] = min(cnt[e] - rank, (uint32_t)MOE_WINDOW_ROWS);
                }
                if (last) fill[e] = rank + 1;  // the expert's last slot this round carries its count forward
            }
        }
    }
}

hipError_t run_moe_windows(const uint32_t *inds, int nslots, int experts, uint32_t *win_count, uint32_t *win_expert,
                           uint32_t *win_rows, uint32_t *win_slots, hipStream_t s) {
    if (nslots <= 0 || nslots > kMoeWindowMaxSlots || experts <= 0 || experts > kMoeWindowMaxExperts)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(moe_windows_kernel, dim3(1), dim3(WIN_THREADS), 0, s, inds, nslots, experts, win_count,
                       win_expert, win_rows, win_slots);
    return hipGetLastError();
}

// Expert windows for the routed GEMM arm (the sort and window table of moePrefill, expert_exl3_kernels.zig:
// 2861-2931 with sorted_windows.zig:10-165), in compact form: the slots sorted by expert (stable: ascending slot within
// an expert) into `sorted`, expert e's run starting at sbase[e] = the exclusive scan of the per-expert counts; each
// run cut into windows of up to MOE_GEMM_WINDOW_ROWS rows (window i of expert e is wbase[e] + i, starting at sorted
// position sbase[e] + i * W); and the 16-row fragment tiles of the prepared inputs numbered so that expert e's rows
// occupy tiles tbase[e] .. tbase[e] + ceil(count / 16) - 1 (a window's tiles are contiguous, from win_tile0).
// tile_info[t] holds tile t's expert, live rows and first sorted position (one load for the kernels that walk tiles).
// A shared expert's rows (sh_rows > 0) are slots nslots .. ns - 1 of expert `experts`.
//
// Two launches over contiguous chunks of the slots, one workgroup per chunk.  The first ranks each slot among the
// chunk's earlier slots of its expert and writes the chunk's per-expert counts; the second sums the counts of the
// chunks before its own (the slot's rank among all earlier slots is that plus its rank in the chunk), scans the
// experts' slots, tiles and windows, and places its chunk.  Every rank is a count of earlier slots, so the result does
// not depend on thread timing.
constexpr int GR_THREADS = 512;   // ranking workgroup: one slot per thread per pass
constexpr int GP_THREADS = 1024;  // placing workgroup: one thread per expert
static_assert(GP_THREADS >= kMoeGemmMaxExperts, "the placing workgroup scans one expert per thread");

__device__ __forceinline__ uint32_t gemm_expert_of(const uint32_t *inds, int nslots, int experts, int s) {
    return s < nslots ? min(inds[s], (uint32_t)(experts - 1)) : (uint32_t)experts;
}

__global__ __launch_bounds__(GR_THREADS) void moe_gemm_rank_kernel(const uint32_t *__restrict__ inds, int nslots,
                                                                   int experts, int sh_rows, int chunk,
                                                                   MoeGemmWindows t) {
    constexpr int NW = GR_THREADS / 64;
    __shared__ uint32_t wc[NW][kMoeGemmMaxExperts];  // this pass: each wave's count per expert
    __shared__ uint32_t run[kMoeGemmMaxExperts];     // the chunk's earlier passes
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ns = nslots + sh_rows, ne = experts + (sh_rows > 0 ? 1 : 0);
    const int id_bits = ne > 1 ? 32 - __clz(ne - 1) : 0;
    const int c0 = blockIdx.x * chunk, c1 = min(c0 + chunk, ns);
    for (int e = tid; e < ne; e += GR_THREADS) run[e] = 0;
    for (int base = c0; base < c1; base += GR_THREADS) {
        const int s = base + tid;
        const bool live = s < c1;
        const int e = live ? (int)gemm_expert_of(inds, nslots, experts, s) : 0;  // in flight while wc is cleared
        for (int e2 = tid; e2 < ne; e2 += GR_THREADS)
#pragma unroll
            for (int w = 0; w < NW; w++) wc[w][e2] = 0;
        __syncthreads();
        // the lanes of this wave holding this lane's expert: one ballot per bit of the expert id, and the live lanes
        unsigned long long same = __ballot(live);
        for (int b = 0; b < id_bits; b++) {
            const unsigned long long set = __ballot((e >> b) & 1);
            same &= ((e >> b) & 1) ? set : ~set;
        }
        const unsigned long long below = (1ull << lane) - 1ull;
        const uint32_t before = (uint32_t)__popcll(same & below);
        if (live && (same & ~below & ~(1ull << lane)) == 0ull) wc[wave][e] = before + 1;  // the wave's last of e
        __syncthreads();
        if (live) {
            uint32_t r = run[e] + before;
            for (int w = 0; w < wave; w++) r += wc[w][e];
            t.ranks[s] = r;
        }
        __syncthreads();
        for (int e2 = tid; e2 < ne; e2 += GR_THREADS) {
            uint32_t v = 0;
#pragma unroll
            for (int w = 0; w < NW; w++) v += wc[w][e2];
            run[e2] += v;
        }
        __syncthreads();
    }
    for (int e = tid; e < ne; e += GR_THREADS) t.chunk_counts[(size_t)e * kMoeGemmMaxChunks + blockIdx.x] = run[e];
}

// Inclusive prefix sum over the wave's lanes.
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t u = __shfl_up(v, off, 64);
        v += lane >= off ? u : 0u;
    }
    return v;
}

__global__ __launch_bounds__(GP_THREADS) void moe_gemm_place_kernel(const uint32_t *__restrict__ inds, int nslots,
                                                                    int experts, int sh_rows, int chunk, int nchunks,
                                                                    MoeGemmWindows t) {
    constexpr int NW = GP_THREADS / 64;
    __shared__ uint32_t cnt[kMoeGemmMaxExperts];
    __shared__ uint32_t pre[kMoeGemmMaxExperts];  // the expert's slots in the chunks before this one
    __shared__ uint32_t sb[kMoeGemmMaxExperts];
    __shared__ uint32_t tb[kMoeGemmMaxExperts];
    __shared__ uint32_t wb[kMoeGemmMaxExperts];
    __shared__ uint32_t wsum[3][NW];
    constexpr uint32_t W = MOE_GEMM_WINDOW_ROWS;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = blockIdx.x;
    const int ns = nslots + sh_rows, ne = experts + (sh_rows > 0 ? 1 : 0);
    // Thread v takes the v-th expert of the scan order (a shared expert first, so its windows -- full ones of 256
    // rows, the GEMMs' heaviest workgroups -- are numbered and dispatched first instead of trailing the grid): its
    // row of chunk counts in one round of loads (entries past nchunks are ignored), its total and the part before
    // this chunk.
    const int c0 = c * chunk, c1 = min(c0 + chunk, ns);
    // this thread's first slot of the chunk: its expert and its rank in the chunk, in flight under the scans
    uint32_t x0 = 0, r0 = 0;
    if (c0 + tid < c1) {
        x0 = gemm_expert_of(inds, nslots, experts, c0 + tid);
        r0 = t.ranks[c0 + tid];
    }
    const int v = tid;
    const int e = v < ne ? (sh_rows > 0 ? (v == 0 ? experts : v - 1) : v) : 0;
    uint32_t total = 0, p = 0;
    if (v < ne) {
        const uint4 *row = reinterpret_cast<const uint4 *>(t.chunk_counts + (size_t)e * kMoeGemmMaxChunks);
        uint4 q4[kMoeGemmMaxChunks / 4];
#pragma unroll
        for (int q = 0; q < kMoeGemmMaxChunks / 4; q++) q4[q] = row[q];
#pragma unroll
        for (int q = 0; q < kMoeGemmMaxChunks / 4; q++) {
            const uint32_t u[4] = {q4[q].x, q4[q].y, q4[q].z, q4[q].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int cc = 4 * q + i;
                total += cc < nchunks ? u[i] : 0u;
                p += cc < c ? u[i] : 0u;
            }
        }
        cnt[e] = total;
        pre[e] = p;
    }
    // three exclusive scans in scan order (slots, 16-row tiles, windows): within each wave, then over the waves
    const uint32_t ls = total, lt = (total + 15) / 16, lw = (total + W - 1) / W;
    const uint32_t is = wave_inclusive_sum(ls, lane), it = wave_inclusive_sum(lt, lane),
                   iw = wave_inclusive_sum(lw, lane);
    if (lane == 63) {
        wsum[0][wave] = is;
        wsum[1][wave] = it;
        wsum[2][wave] = iw;
    }
    __syncthreads();
    uint32_t os = 0, ot = 0, ow = 0, at = 0, aw = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) {
        os += w < wave ? wsum[0][w] : 0u;
        ot += w < wave ? wsum[1][w] : 0u;
        ow += w < wave ? wsum[2][w] : 0u;
        at += wsum[1][w];
        aw += wsum[2][w];
    }
    if (v < ne) {
        sb[e] = os + is - ls;
        tb[e] = ot + it - lt;
        wb[e] = ow + iw - lw;
    }
    if (c == 0 && tid == 0) {
        *t.win_count = aw;
        *t.tile_count = at;
    }
    __syncthreads();
    for (int s = c0 + tid; s < c1; s += GP_THREADS) {
        const bool first = s == c0 + tid;
        const uint32_t x = first ? x0 : gemm_expert_of(inds, nslots, experts, s);
        const uint32_t rank = pre[x] + (first ? r0 : t.ranks[s]);
        t.sorted[sb[x] + rank] = (uint32_t)s;
        if (rank % W == 0) {  // the first slot of a window writes its row
            const uint32_t w = wb[x] + rank / W, rows = min(cnt[x] - rank, W);
            const uint32_t tile0 = tb[x] + rank / 16;
            t.win_expert[w] = x;
            t.win_rows[w] = rows;
            t.win_start[w] = sb[x] + rank;
            t.win_tile0[w] = tile0;
            for (uint32_t i = 0; i < (rows + 15) / 16; i++)
                t.tile_info[tile0 + i] = uint4{x, min(16u, rows - 16 * i), sb[x] + rank + 16 * i, 0u};
        }
    }
}

// Slots per chunk: whole ranking passes, at most kMoeGemmMaxChunks chunks.
int moe_gemm_chunk(int ns) {
    const int per = (ns + kMoeGemmMaxChunks - 1) / kMoeGemmMaxChunks;
    return std::max(GR_THREADS, (per + GR_THREADS - 1) / GR_THREADS * GR_THREADS);
}

hipError_t run_moe_gemm_windows(const uint32_t *inds, int nslots, int experts, int sh_rows, const MoeGemmWindows &t,
                                hipStream_t s) {
    if (nslots <= 0 || experts <= 0 || sh_rows < 0 || experts + (sh_rows > 0 ? 1 : 0) > kMoeGemmMaxExperts)
        return hipErrorInvalidValue;
    const int ns = nslots + sh_rows, chunk = moe_gemm_chunk(ns), nchunks = (ns + chunk - 1) / chunk;
    hipLaunchKernelGGL(moe_gemm_rank_kernel, dim3(nchunks), dim3(GR_THREADS), 0, s, inds, nslots, experts, sh_rows,
                       chunk, t);
    hipLaunchKernelGGL(moe_gemm_place_kernel, dim3(nchunks), dim3(GP_THREADS), 0, s, inds, nslots, experts, sh_rows,
                       chunk, nchunks, t);
    return hipGetLastError();
}

// One wave per row (four rows a workgroup): lane l holds experts l, l + 64, ... in registers (experts <= 1024, so at
// most 16 each); k rounds of a wave-wide argmax (ties to the lower index), then the softmax mass of the picks over the
// full row, renormalised.  Selection keys are the logits with NaN read as -inf, and a per-lane mask keeps each expert
// from being picked twice: every round starts from "no candidate" and takes any unpicked expert over it, so with
// k <= experts (checked by the host) each pick is a distinct index in [0, experts) whatever the logits hold.  A NaN
// logit still reaches the softmax, so such a row's scores come out NaN, as the chain's do.  The argmax order is total,
// so the picks do not depend on the reduction's order; the sums (the denominator, the renormalisation) are taken
// across the wave.  (A 256-thread workgroup per row, with two barriers a round, took 24.9 us for 2048 rows x 256.)
__device__ __forceinline__ float route_key(float v) { return v != v ? -INFINITY : v; }

// (value, index) pair order of the argmax: larger key first, then the lower index.
__device__ __forceinline__ bool route_better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

constexpr int ROUTE_PER_LANE = 16;  // experts per lane at most: 1024 / 64

// One step of a wave reduction towards lane 63 (the gfx9 DPP scan: row shifts by 1, 2, 4, 8 within each 16-lane row,
// then lane 15 into rows 1 and 3 and lane 31 into rows 2 and 3): each lane combines its value with the one DPP brings
// it, or with `none` where the source lane is outside its row or the lane is masked off.  After the last step lane
// 63 holds the whole wave's reduction.
template <int CTRL, int ROWS, int BANKS>
__device__ __forceinline__ int dpp_from(int v, int none) {
    return __builtin_amdgcn_update_dpp(none, v, CTRL, ROWS, BANKS, false);
}
#define EXL3_DPP_SCAN(STEP)                                                                                           \
    STEP(0x111, 0xF, 0xF) STEP(0x112, 0xF, 0xF) STEP(0x114, 0xF, 0xF) STEP(0x118, 0xF, 0xF) STEP(0x142, 0xA, 0xF)    \
    STEP(0x143, 0xC, 0xF)

__device__ __forceinline__ float wave_max(float v) {
#define EXL3_MAX_STEP(C, R, B)                                                                                        \
    v = fmaxf(v, __builtin_bit_cast(float, dpp_from<C, R, B>(__builtin_bit_cast(int, v),                             \
                                                                __builtin_bit_cast(int, -INFINITY))));
    EXL3_DPP_SCAN(EXL3_MAX_STEP)
#undef EXL3_MAX_STEP
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_sum(float v) {
#define EXL3_SUM_STEP(C, R, B) v += __builtin_bit_cast(float, dpp_from<C, R, B>(__builtin_bit_cast(int, v), 0));
    EXL3_DPP_SCAN(EXL3_SUM_STEP)
#undef EXL3_SUM_STEP
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// The wave's best (key, index) under route_better; index `none` is "no candidate" and loses to any other.
__device__ __forceinline__ void wave_argmax(float &bv, int &bi, int none) {
#define EXL3_ARG_STEP(C, R, B)                                                                                        \
    {                                                                                                                 \
        const float ov = __builtin_bit_cast(float, dpp_from<C, R, B>(__builtin_bit_cast(int, bv),                     \
                                                                     __builtin_bit_cast(int, -INFINITY)));           \
        const int oi = dpp_from<C, R, B>(bi, none);                                                                   \
        const bool take = oi != none && (bi == none || route_better(ov, oi, bv, bi));                                 \
        bv = take ? ov : bv;                                                                                          \
        bi = take ? oi : bi;                                                                                          \
    }
    EXL3_DPP_SCAN(EXL3_ARG_STEP)
#undef EXL3_ARG_STEP
    bv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bv), 63));
    bi = __builtin_amdgcn_readlane(bi, 63);
}
#undef EXL3_DPP_SCAN

// PER: experts per lane, the smallest power of two with 64 PER >= experts.
template <int PER>
__global__ __launch_bounds__(256) void route_topk_kernel(const float *__restrict__ logits, int rows, int experts,
                                                         int k, uint32_t *__restrict__ inds,
                                                         float *__restrict__ scores) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (row >= rows) return;  // wave-uniform: the wave's row
    const float *l = logits + (size_t)row * experts;
    float v[PER];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; i++) {  // every load in bounds; experts past the row are left out below
        const int e = lane + 64 * i;
        v[i] = l[min(e, experts - 1)];
        mx = e < experts ? fmaxf(mx, v[i]) : mx;
    }
    mx = wave_max(mx);
    float den = 0.f;
#pragma unroll
    for (int i = 0; i < PER; i++) den += lane + 64 * i < experts ? __expf(v[i] - mx) : 0.f;
    den = wave_sum(den);
    uint32_t taken = 0;  // bit i: expert lane + 64 i picked
    int mine = 0;        // lane j < k: the j-th pick
    for (int j = 0; j < k; j++) {
        // bi = experts marks "no candidate yet": any unpicked expert beats it (its key is at least -inf).
        float bv = -INFINITY;
        int bi = experts;
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int e = lane + 64 * i;
            const float kv = route_key(v[i]);
            const bool take = e < experts && !((taken >> i) & 1u) && (bi == experts || route_better(kv, e, bv, bi));
            bv = take ? kv : bv;
            bi = take ? e : bi;
        }
        wave_argmax(bv, bi, experts);
        // every lane holds the same (bv, bi); k <= experts leaves an unpicked expert every round, so bi < experts
        taken |= (bi & 63) == lane ? 1u << (bi >> 6) : 0u;
        mine = lane == j ? bi : mine;
    }
    const float p = lane < k ? __expf(l[mine] - mx) / den : 0.f;
    const float sum = wave_sum(p);
    if (lane < k) {
        inds[(size_t)row * k + lane] = (uint32_t)mine;
        scores[(size_t)row * k + lane] = p / sum;
    }
}

hipError_t run_route_topk(const float *logits, int rows, int experts, int k, uint32_t *inds, float *scores,
                          hipStream_t s) {
    if (rows == 0) return hipSuccess;
    if (experts > 64 * ROUTE_PER_LANE || k > 64) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, grid, block, 0, s, logits, rows, experts, k, inds, scores); };
    if (experts <= 64) go(route_topk_kernel<1>);
    else if (experts <= 128) go(route_topk_kernel<2>);
    else if (experts <= 256) go(route_topk_kernel<4>);
    else if (experts <= 512) go(route_topk_kernel<8>);
    else go(route_topk_kernel<16>);
    return hipGetLastError();
}

// One workgroup per (expert, tile) of the source; n halfwords copied by the first n threads.
__global__ void tile_major_kernel(const uint16_t *__restrict__ src, uint16_t *__restrict__ dst, int it, int ot, int n,
                                  int inverse) {
    const int e = blockIdx.y;
    const int t = blockIdx.x;  // index in the pack order: tk * ot + tn
    const int tk = t / ot, tn = t % ot;
    const int pair = tn >> 1, o = tn & 1;
    const size_t pack = ((size_t)tk * ot + tn) * n;
    const size_t pm = (((size_t)pair * it + tk) * 2 + o) * n;
    const size_t eb = (size_t)e * it * ot * n;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        if (!inverse) dst[eb + pm + i] = src[eb + pack + i];
        else dst[eb + pack + i] = src[eb + pm + i];
    }
}

hipError_t run_tile_major(const uint16_t *src, uint16_t *dst, int experts, int it, int ot, int n, int inverse,
                          hipStream_t s) {
    if (experts == 0 || it * ot == 0) return hipSuccess;
    hipLaunchKernelGGL(tile_major_kernel, dim3((unsigned)(it * ot), (unsigned)experts), dim3(64), 0, s, src, dst, it,
                       ot, n, inverse);
    return hipGetLastError();
}

__global__ void fill_zero_kernel(uint32_t *__restrict__ p, size_t words) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < words; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

hipError_t run_fill_zero(void *p, size_t bytes, hipStream_t s) {
    const size_t words = bytes / 4;
    if (words == 0) return hipSuccess;
    size_t blocks = (words + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, s, reinterpret_cast<uint32_t *>(p),
                       words);
    return hipGetLastError();
}

// ---- moeGroups (src/exl3/root.zig:646-703): each group's routing and the f32 sum of the group outputs

// Slot s of expert e in [lo, lo + count): local id e - lo with its score; any other slot: local id 0, score 0 (the
// reference's where(mask, inds - lo, 0) and where(mask, scores, 0)).  Scores widen exactly to f32.
__global__ void moe_group_routing_kernel(const uint32_t *__restrict__ inds, const void *__restrict__ scores, int dt,
                                         int nslots, uint32_t lo, uint32_t count, uint32_t *__restrict__ local,
                                         float *__restrict__ weight) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nslots) return;
    const uint32_t e = inds[s];
    const bool in = e >= lo && e - lo < count;
    local[s] = in ? e - lo : 0u;
    weight[s] = in ? load_any(scores, dt, (size_t)s) : 0.0f;
}

hipError_t run_moe_group_routing(const uint32_t *inds, const void *scores, int score_dtype, int nslots, uint32_t lo,
                                 uint32_t count, uint32_t *local, float *weight, hipStream_t s) {
    if (nslots <= 0) return hipSuccess;
    hipLaunchKernelGGL(moe_group_routing_kernel, dim3((unsigned)((nslots + 255) / 256)), dim3(256), 0, s, inds, scores,
                       score_dtype, nslots, lo, count, local, weight);
    return hipGetLastError();
}

__global__ void add_f32_kernel(float *__restrict__ acc, const float *__restrict__ part, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        acc[i] += part[i];
}

__global__ void cast_f32_kernel(const float *__restrict__ src, void *__restrict__ y, int dt, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        store_out(y, dt, i, src[i]);
}

static unsigned elementwise_blocks(size_t n) {
    const size_t b = (n + 255) / 256;
    return (unsigned)(b > 4096 ? 4096 : b);
}

hipError_t run_add_f32(float *acc, const float *part, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(add_f32_kernel, dim3(elementwise_blocks(n)), dim3(256), 0, s, acc, part, n);
    return hipGetLastError();
}

hipError_t run_cast_f32(const float *src, void *y, int y_dtype, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(cast_f32_kernel, dim3(elementwise_blocks(n)), dim3(256), 0, s, src, y, y_dtype, n);
    return hipGetLastError();
}

}  // namespace exl3
