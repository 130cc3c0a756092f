// Internal launch interface between the C-ABI layer (exl3_capi.hip) and the kernel translation units.
#pragma once

#include <string>

#include "exl3_common.cuh"

namespace exl3 {

hipError_t run_decode_codewords(int fam, const uint16_t *cw, int64_t count, const DecodeK &k, uint16_t *out,
                                hipStream_t s);
hipError_t run_reconstruct_inner(int fam, const uint16_t *trellis, int it, int ot, int n, const DecodeK &k,
                                 uint16_t *out, hipStream_t s);
// One expert of a per-tile-rate bank (segment tables as GemvArgs::seg_off / seg_k1 describe them); ka / kb are the
// constants at TILED_NA / TILED_NB.
hipError_t run_reconstruct_tiled(int fam, const uint16_t *trellis, const uint32_t *seg_off, const uint8_t *seg_k1,
                                 int expert, int it, int ot, const DecodeK &ka, const DecodeK &kb, uint16_t *out,
                                 hipStream_t s);

enum Prologue : int { PRO_X = 0, PRO_MID = 1 };

// Fused-finish arrival counters sit one per 128-byte line (32 words) in the workspace's counter region.
constexpr int COUNTER_STRIDE = 32;

// Fixed-point fused finish (the fold): one 64-bit word per output holds the arrival count in bits 63..58 (so at
// most FOLD_MAX_SPLITS splits), the count of contributions outside the fixed-point range in bits 57..52, and in bits
// 51..0 the sum of the splits' biased terms q + FOLD_BIAS, q = round(v * 2^FOLD_FRAC) for |v| < 2^21.  A contribution
// outside that range (or not finite) is added in f64 to the output's overflow word, FOLD_WORDS words past its fold
// word, before its arrival is counted; the arrival that completes the output adds the overflow word to the exact sum
// when the out-of-range count says it is in use, and clears it.  The region of fold words and the region of overflow
// words each hold FOLD_WORDS words.
constexpr int FOLD_MAX_SPLITS = 63;
constexpr int FOLD_COUNT_SHIFT = 58;
constexpr int FOLD_BAD_SHIFT = 52;
constexpr int FOLD_FRAC = 24;
constexpr long long FOLD_BIAS = 1LL << 45;
constexpr size_t FOLD_WORDS = (size_t(4) << 20) / sizeof(unsigned long long);

// GEMV workgroup shape: GEMV_WAVES waves, each loading up to TPW k-tiles of the output group before its prologue
// and refilling each slot as it is decoded.  Two slots rather than four: with fewer requests in flight at the start,
// the first tiles (and the input of the prologue) come back sooner, and two waves per SIMD keep the VALU busy.
// One workgroup per CU (256 CUs) is the target grid.
constexpr int GEMV_WAVES = 8;
constexpr int TPW = 2;
constexpr int GEMV_TARGET_WGS = 256;

// Division by a launch constant d >= 1 as one multiply-high: m = 0 stands for d = 1, else m = ceil(2^32 / d), and
// floor(q m / 2^32) = q / d whenever q (d - 1) < 2^32 (with m d = 2^32 + r, r < d, and q = k d + j: the excess
// q r / 2^32 stays below 1 <= d - j).  The GEMV's block-to-tile map divides by its split count and its x row
// divisor this way, ahead of its first loads (a general 32-bit division is some 20 dependent instructions).
__host__ __device__ inline uint32_t div_magic(uint32_t d) {
    return d <= 1 ? 0u : (uint32_t)((0x100000000ull + d - 1) / d);
}
__device__ __forceinline__ uint32_t div_by_magic(uint32_t q, uint32_t m) { return m ? __umulhi(q, m) : q; }

// Trellis GEMV over `groups` independent (bank, x-block) pairs, 1..8 rows each.
//  * dense linear: groups = 1 (or G for linearGrouped), bank_of = null, x_div = 1;
//  * MoE pair GEMV: groups = slots, bank_of = expert id per slot, x_div = topk, two projections (gate, up) on
//    grid.z, partial_only (f32 planes for the mid);
//  * MoE down GEMV: PRO_MID prologue builds its input from the gate/up planes (sum splits, FWHT, svh, clamp,
//    SwiGLU, * suh_down, FWHT, f16) and writes f32 planes for the reduce.
struct GemvArgs {
    const void *x;
    int x_dtype;
    int rows;
    int in;
    int out;
    int x_div;
    // PRO_MID inputs: gate/up planes [groups][mid_splits][in] f32 and the gate/up svh banks ([E][in])
    const float *mid_part[2];
    int mid_splits;
    const uint16_t *mid_svh[2];
    float clamp_limit;  // 0 = none
    // banks, one per projection (grid.z)
    const uint16_t *trellis[2];
    const uint16_t *suh[2];
    const uint16_t *svh[2];
    int n;                   // uniform rate; 0 with `meta` = per-expert rates
    const uint32_t *bank_of; // [groups] expert id, or null (bank = group)
    const uint32_t *meta;    // ragged meta [E][8]: n at col pi, word offset at col 4 + pi
    int meta_lane_only;      // every ragged rate is a lane-reader rate: no launch for the other rates
    int meta_col[2];
    // per-tile-rate bank (N_TILED): per projection, the segment tables [E][in/16][out/128] (word offset of each
    // segment of 8 tiles, and its mask: bit o set = tile o at TILED_NA, else TILED_NB); null = not tiled
    const uint32_t *seg_off[2];
    const uint8_t *seg_k1[2];
    int table;               // codebook table for per-rate rows (ragged hash / pair families)
    int bank_limit;          // expert count: ids are clamped below it (memory safety on bad routing)
    DecodeK k;
    float out_scale;
    float *partial[2];       // [groups][splits][rows][out] f32
    uint32_t *counters;      // [groups][out/128], zero between calls
    unsigned long long *fold; // fixed-point fused finish: one word per output, zero between calls; null = off
    int fold_arrivals;        // contributions per output word (the dense GEMV's splits; topk * splits for the MoE down)
    int fold_topk;            // > 0: MoE down -- slot s folds into output row s / fold_topk, scaled by fold_scores[s]
    const void *fold_scores;  // [slots] in score_dtype (f32, bf16 or f16)
    int score_dtype;
    const void *fold_shared;  // MoE: [rows][out] in y's dtype, added after the routed sum's rounding; null = none
    const void *fold_gate;    // MoE: [rows] gate logits in y's dtype: fold_shared is added as sigmoid(gate) * shared
    // A fused shared expert's own fold words [rows][out] and the words where the rounded routed and shared sums
    // meet (see sh_from below); beside the fold's other fields, which the finish reads together.
    unsigned long long *sh_fold;
    unsigned long long *fold_comb;
    void *y;
    int y_dtype;
    int y_rows_major;  // dense: group g's row r is output row r * groups + g ([rows][groups * out]), else g * rows + r
    int rows_total;    // dense row groups of one bank: the rows of all groups (the last group holds the rest), or 0
    int splits;
    int groups;
    int nproj;
    int fused_finish;
    int partial_only;
    // Expert windows (the sorted MoE arm): group g is window g, whose win_rows[g] (<= MOE_WINDOW_ROWS) rows are the
    // slots win_slots[g][r] of expert win_expert[g]; windows past *win_count exit at once.  Null: group g is slot g.
    const uint32_t *win_count;
    const uint32_t *win_expert;
    const uint32_t *win_rows;
    const uint32_t *win_slots;
    // A shared expert fused into the routed launches (per-slot arm): the first sh_groups groups of the grid are the
    // shared expert's token rows, SH_ROWS per group, decoded from the one-expert bank sh_* at rate sh_n with score 1
    // (the routed slots follow); their planes and slots are sh_from + row, past the routed slots (sh_from = their
    // count).  The down projection folds them into their own words (sh_fold); the rounded routed and shared sums then
    // meet in fold_comb, whose second arrival stores T(T(routed) + T(shared)).  sh_groups = 0: no shared expert (the
    // kernel takes it as a preloaded leading argument).
    int sh_groups;
    int sh_from;
    int sh_rows;   // token rows (the shared groups hold SH_ROWS of them each)
    int sh_n;
    const uint16_t *sh_trellis[2];
    const uint16_t *sh_suh[2];
    const uint16_t *sh_svh[2];
    const uint16_t *sh_mid_svh[2];  // PRO_MID: the shared expert's gate / up svh
    // The fused decode chain (one launch for gate/up and down, run_moe_chain): group y of the grid (shared groups
    // first, then the slots) has a pair of counters 128 bytes apart in the zeroed region, chain_ctr[2 y] (arrivals of
    // its gate/up workgroups, chain_need of them) and chain_ctr[2 y + 1] (down workgroups past their wait,
    // chain_need2 of them; the last clears both).
    uint32_t *chain_ctr;
    int chain_need;
    int chain_need2;
};

// The fused chain's counters sit at the top of the zeroed region's overflow half (its low entries serve the fold
// words in use), CHAIN_CTR_BYTES of them.
constexpr size_t CHAIN_CTR_BYTES = size_t(128) << 10;
// A down workgroup waits for its group's gate/up planes at most this many s_memrealtime ticks (100 MHz: 0.2 s), so
// every wave leaves its wait whatever happens to the workgroups it waits for.
constexpr uint64_t CHAIN_SPIN_TICKS = 20000000ull;

// The GEMV's block-to-tile map, preloaded as leading kernel arguments: k-tiles and output tiles (in / 16 | out / 16
// << 16), splits and k-tiles per split (S | (in / 16 / S) << 16), and the div_magic constants of S and x_div.
struct GemvGeo {
    uint32_t tiles, sks, s_m, xdiv_m;
};
inline GemvGeo gemv_geo(const GemvArgs &a) {
    const uint32_t it = (uint32_t)a.in / 16, ot = (uint32_t)a.out / 16, s = (uint32_t)a.splits;
    return GemvGeo{it | ot << 16, s | (it / s) << 16, div_magic(s), div_magic((uint32_t)a.x_div)};
}

// Rows per expert window in the sorted MoE arm.
constexpr int MOE_WINDOW_ROWS = 4;

// Token rows per group of a fused shared expert (its weights are decoded once per group).
constexpr int SH_ROWS = 4;

hipError_t run_gemv(int fam, int prologue, const GemvArgs &a, hipStream_t s);
hipError_t run_gemv_fam_FAM_MCG(int prologue, const GemvArgs &a, hipStream_t s);
hipError_t run_gemv_fam_FAM_MUL1(int prologue, const GemvArgs &a, hipStream_t s);
hipError_t run_gemv_fam_FAM_HASH(int prologue, const GemvArgs &a, hipStream_t s);
hipError_t run_gemv_fam_FAM_PAIR(int prologue, const GemvArgs &a, hipStream_t s);
hipError_t run_gemv_fam_FAM_3INST(int prologue, const GemvArgs &a, hipStream_t s);
// The per-slot MoE decode chain in one launch: gate/up (a1, PRO_X, f32 planes written through to memory, then its
// group's arrival counted) and the SwiGLU mid + down (a2, PRO_MID, folded into y) as one grid, the down workgroups
// after the gate/up ones; a down workgroup issues its tile loads, then waits for its group's gate/up arrivals.  Uniform
// banks at one lane-reader rate (a1.n == a2.n), one row per group.
hipError_t run_moe_chain(int fam, const GemvArgs &a1, const GemvArgs &a2, hipStream_t s);
hipError_t run_moe_chain_fam_FAM_MCG(const GemvArgs &a1, const GemvArgs &a2, hipStream_t s);
hipError_t run_moe_chain_fam_FAM_MUL1(const GemvArgs &a1, const GemvArgs &a2, hipStream_t s);
hipError_t run_moe_chain_fam_FAM_HASH(const GemvArgs &a1, const GemvArgs &a2, hipStream_t s);
hipError_t run_moe_chain_fam_FAM_PAIR(const GemvArgs &a1, const GemvArgs &a2, hipStream_t s);
hipError_t run_moe_chain_fam_FAM_3INST(const GemvArgs &a1, const GemvArgs &a2, hipStream_t s);
int gemv_default_splits(int in, int out, int rows, int groups_times_proj, int max_batches = 1, int target_wgs = 0);

// Top-k the MoE reduce holds per row (REDUCE_MAX_TOPK, src/exl3/expert_exl3_kernels.zig:2562).
constexpr int kMoeReduceMaxTopk = 32;

// MoE finish: y[row] = sum_k score * (FWHT(sum_s down_part) * svh_down[e]) (+ shared), REDUCE_SOURCE.
struct ReduceArgs {
    const float *part;  // [slots][splits][hidden]
    int splits;
    int hidden;
    int topk;
    int rows;
    const uint32_t *slots;
    int bank_limit;
    const void *scores;   // [slots] in score_dtype
    int score_dtype;
    const uint16_t *svh;  // [E][hidden]
    const void *shared;   // [rows][hidden] in y dtype, or null
    const void *gate;     // [rows] in y dtype: shared is added as sigmoid(gate) * shared; null = plain add
    // or a shared expert's raw down planes [rows][hidden] and svh (shared null): its score-1 term, rounded to y's
    // dtype as a one-expert layer's output, is added as `shared` would be
    const float *sh_part;
    const uint16_t *sh_svh;
    void *y;
    int y_dtype;
    float out_scale;
};
hipError_t run_moe_reduce(const ReduceArgs &a, hipStream_t s);

// moeGroups (src/exl3/root.zig:646-703): one group's routing -- slots of experts [lo, lo + count) as local ids with
// their scores, every other slot as local expert 0 with score 0 (f32) -- and the f32 group sums: acc += part, then
// y = T(acc).
hipError_t run_moe_group_routing(const uint32_t *inds, const void *scores, int score_dtype, int nslots, uint32_t lo,
                                 uint32_t count, uint32_t *local, float *weight, hipStream_t s);
hipError_t run_add_f32(float *acc, const float *part, size_t n, hipStream_t s);
hipError_t run_cast_f32(const float *src, void *y, int y_dtype, size_t n, hipStream_t s);

// Groups the slots of a routing by expert into windows of up to MOE_WINDOW_ROWS rows, slots in ascending order
// within an expert (a stable counting sort): one workgroup; slots <= kMoeWindowMaxSlots, experts <= kMoeWindowMaxExperts.
constexpr int kMoeWindowMaxSlots = 8192;
constexpr int kMoeWindowMaxExperts = 4096;
hipError_t run_moe_windows(const uint32_t *inds, int nslots, int experts, uint32_t *win_count, uint32_t *win_expert,
                           uint32_t *win_rows, uint32_t *win_slots, hipStream_t s);

// The routed GEMM arm's expert windows (moe_gemm_rank_kernel + moe_gemm_place_kernel): slots sorted by expert,
// windows of up to MOE_GEMM_WINDOW_ROWS rows of one expert, and the 16-row fragment tiles of their prepared inputs.
constexpr int MOE_GEMM_WINDOW_ROWS = 256;
constexpr int kMoeGemmMaxExperts = 1024;
struct MoeGemmWindows {
    uint32_t *win_count;    // [1] windows
    uint32_t *tile_count;   // [1] 16-row tiles over all windows
    uint32_t *sorted;       // [slots] slot ids by expert, ascending within an expert
    uint32_t *win_expert;   // [windows]
    uint32_t *win_rows;     // [windows] rows (<= MOE_GEMM_WINDOW_ROWS)
    uint32_t *win_start;    // [windows] first sorted position
    uint32_t *win_tile0;    // [windows] first fragment tile
    uint4 *tile_info;       // [tiles] each tile's window expert, live rows (<= 16) and first sorted position
    uint32_t *chunk_counts; // [experts (+ 1 shared)][kMoeGemmMaxChunks] scratch: each expert's count per chunk
    uint32_t *ranks;        // [slots] scratch: each slot's rank among its chunk's earlier slots of its expert
};
constexpr int kMoeGemmMaxChunks = 64;
// sh_rows > 0 adds a shared expert as expert `experts`: slots nslots .. nslots + sh_rows - 1, one per token row.
hipError_t run_moe_gemm_windows(const uint32_t *inds, int nslots, int experts, int sh_rows, const MoeGemmWindows &t,
                                hipStream_t s);

// The routed GEMM arm (a prefill-width layer: every expert's rows in windows of up to 256, each weight decoded once
// per window on the matrix cores).  Projection p of grid z: x prepared per window row with that expert's suh into
// xp[p] (fragment order, tile t at xp + t * (in / 32) * 512), the raw inner products written to planes[p]
// [slot][out] (f32, no output transform: the mid / the reduce applies it).  With sh = 1 a shared expert is expert
// `experts`, its banks in the sh_ pointers and its rows the slots from nslots on (slot nslots + r is token row r).
struct MoeGemmArgs {
    MoeGemmWindows win;
    const void *x;          // [tokens][hidden] (gate/up) -- the token of routed slot s is s / topk
    int x_dtype;
    int topk;
    int in, out;
    int experts;
    int nslots;             // routed slots
    int sh;                 // 1: a shared expert follows the routed ones
    const uint16_t *trellis[2];
    const uint16_t *suh[2];
    const uint16_t *sh_trellis[2];
    const uint16_t *sh_suh[2];
    int n;                  // uniform rate; 0 with `meta` (ragged) or `seg_off` (per-tile rates)
    int sh_n;               // the shared expert's rate (a lane-reader rate)
    DecodeK k;              // the decode at n (uniform), else the codebook's base constants
    int table;              // codebook table of the per-rate rows (hash / pair families)
    // ragged bank (rate_groups.zig:22-140): meta [E][8], projection p's rate at column meta_col[p] and its tiles' u32
    // word offset at column 4 + meta_col[p]; every rate a lane-reader rate (the host checks)
    const uint32_t *meta;
    int meta_col[2];
    // per-tile-rate bank: projection p's segment tables [E][in/16][out/128] (word offset, TILED_NA mask)
    const uint32_t *seg_off[2];
    const uint8_t *seg_k1[2];
    uint16_t *xp[2];        // prepared inputs, fragment order
    float *planes[2];       // raw inner [slots][out]
    // the mid (down input): gate / up planes [slots][inter] -> xp_down, with the gate / up svh and the down suh
    const float *mid_planes[2];
    const uint16_t *mid_svh[2];
    const uint16_t *down_suh;
    const uint16_t *sh_mid_svh[2];
    const uint16_t *sh_down_suh;
    float clamp_limit;
    int max_tiles;          // grid bound: tiles over all windows
    int max_windows;        // grid bound: windows
};
hipError_t run_moe_gemm_prepare(const MoeGemmArgs &a, int nproj, hipStream_t s);
hipError_t run_moe_gemm_mid(const MoeGemmArgs &a, hipStream_t s);
hipError_t run_moe_gemm(int fam, const MoeGemmArgs &a, int nproj, hipStream_t s);

// Dense GEMM arm (prefill, rows > 8): prepare x -> xp f16, decode tiles to MFMA fragments, finish in the epilogue.
struct GemmArgs {
    const void *x;
    int x_dtype;
    int rows;
    int in;
    int out;
    const uint16_t *trellis;
    int n;
    const uint16_t *suh;
    const uint16_t *svh;
    DecodeK k;
    uint16_t *xp;     // workspace: prepared input, f16 -- [groups][rows][in], or in MFMA A-fragment order (see gemm)
    uint16_t *wt;     // workspace [groups][out][in] f16 (rates without a direct reader)
    void *y;
    int y_dtype;
    int groups;
    int arm;          // GEMM body: 0 = the row-count policy, 4 = 256-row tile (decode waves), 5 / 6 = ping-pong 512 / 256,
                      // 7 = ping-pong 512 with k in halves
    float *kpart;     // arm 7: workspace for the halves' partials (gemm_kpart_bytes), or null
    uint32_t *kctr;   // arm 7: one zeroed counter per tile (COUNTER_STRIDE words apart), left at zero
    uint32_t kwait;   // arm 7: 100 MHz ticks the first half to arrive waits for the other before handing it the tile
};
// The row-count policy for arm 0 (the C-ABI layer applies it and sizes arm 7's region accordingly).
inline int gemm_default_arm(int groups, int rows, int out) {
    const long wg5 = (long)((rows + 511) / 512) * (out / 128) * groups;
    if (rows > 512 && wg5 >= 192) return 5;
    if (rows > 256 && rows <= 512 && wg5 < 192 && 2 * wg5 >= 160) return 7;
    return 4;
}
// arm 7's partial region: two halves of every 512-row x 128-column tile, f32
inline size_t gemm_kpart_bytes(int groups, int rows, int out) {
    return (size_t)groups * ((rows + 511) / 512) * (out / 128) * 2 * 512 * 128 * sizeof(float);
}
hipError_t run_gemm(int fam, const GemmArgs &a, hipStream_t s);

hipError_t run_route_topk(const float *logits, int rows, int experts, int k, uint32_t *inds, float *scores,
                          hipStream_t s);
hipError_t run_tile_major(const uint16_t *src, uint16_t *dst, int experts, int it, int ot, int n, int inverse,
                          hipStream_t s);
hipError_t run_fill_zero(void *p, size_t bytes, hipStream_t s);

// Trellis encoder search (src/encoder/encode.zig:170-309): `count` row-major 16x16 f32 tiles -> packed codes [count][n]
// and, when `sse` is set, each path's f64 squared error.  `tiles_per_wg` tiles share a workgroup; `back` holds
// grid x tiles_per_wg x 256 x stride backpointer bytes (stride = 2^(w - kmin)).
struct EncodeArgs {
    const float *tiles;
    int64_t count;
    int n;
    int w;
    DecodeK k;
    uint16_t *packed;
    double *sse;
    float *recon;   // optional: the decoded values of each tile's path, row-major [count][256]
    uint8_t *back;
    int stride;
    int tiles_per_wg;
    int grid;
};
size_t encode_lds_bytes(int tiles_per_wg, int stride);
hipError_t run_encode(int fam, const EncodeArgs &a, hipStream_t s);

// A search launch's shape for a tile count: backpointer stride, tiles per workgroup, the grid that fills the GPU
// (grid_cap) and the backpointer bytes of one workgroup.
struct EncodeTuning {
    int stride;
    int tiles_per_wg;
    int grid_cap;
    size_t per_wg;
};

// Whole-tensor quantizer (src/encoder/quantize.zig:600-626): host pointers in and out, a device workspace.
enum QuantStatus : int { QUANT_OK = 0, QUANT_LAUNCH = 1, QUANT_WORKSPACE = 2, QUANT_HESSIAN = 3 };
struct QuantArgs {
    const float *w;         // [in][out]
    const float *h;         // [in][in]
    const float *sign_in;   // [in]
    const float *sign_out;  // [out]
    int in, out, n, w_bits, mode, fam;
    DecodeK k;
    EncodeTuning tune_g;     // the global scale's sample tiles (up to 128)
    EncodeTuning tune_rows;  // one 16-row group's out/16 tiles
    uint16_t *packed;        // [in/16][out/16][n]
    uint16_t *suh;           // [in] f16 bits
    uint16_t *svh;           // [out] f16 bits
    float *g;
    void *workspace;
    size_t workspace_bytes;
    hipStream_t stream;
};
size_t quantize_workspace_bytes(int in, int out, const EncodeTuning &tune_g, const EncodeTuning &tune_rows);
int quantize_tensor(const QuantArgs &q, std::string *msg);

}  // namespace exl3
