/*
 * sushi_exl3_hip -- MI355X (gfx950) HIP implementation of beamivalice/sushi's EXL3/STQ trellis-quantized
 * linear-layer hot path, behind a plain C ABI.
 *
 * This is the cut the reference's host would bind instead of its `sushi_exl3` Zig module
 * (src/exl3/root.zig, src/exl3/linear.zig, src/exl3/expert_exl3_kernels.zig).  Conventions:
 *   - every pointer is a device pointer unless stated; the caller owns all memory (inputs, outputs, workspace);
 *   - nothing here allocates device memory: a call that needs scratch takes a caller workspace whose size the
 *     matching *_workspace_size() reports (the reference allocates per call through MLX; this ABI does not);
 *   - launches are asynchronous on the caller's stream; no entry point synchronises the host
 *     (the reference never reads back on the decode path either, docs/mlx-serve-integration.md:186-191);
 *   - every refusal happens before any launch and returns a negative status; exl3_last_error() describes it
 *     (thread-local, valid until the next call on the same thread);
 *   - not thread-safe per stream: call from the thread that owns the stream, as the reference requires
 *     (docs/mlx-serve-integration.md:151-169).  The decode parameters travel with every call (no process-global
 *     codebook, unlike kernels.setDecodeParams, src/exl3/expert_exl3_kernels.zig:937-944).
 *
 * Layouts (the reference's, src/exl3/root.zig:28-39):
 *   trellis  u16 [E][in/16][out/16][n]   n = 16*K halfwords per 16x16 tile, even, 16..128
 *   suh      f16 [E][in]                 input sign/scale vector
 *   svh      f16 [E][out]                output sign/scale vector
 *   x        [rows][in]  f16 | bf16 | f32  (exl3_dtype), 4-byte aligned
 *   y        [rows][out] same dtype set
 */
#ifndef SUSHI_EXL3_HIP_H
#define SUSHI_EXL3_HIP_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EXL3_ABI_VERSION 5

/* Codebook: the reference's `Codebook` enum values (src/exl3/expert_exl3.zig:54-61), plus 3INST as an
 * extension (QTIP's LCG codebook, not in the reference). */
typedef enum {
    EXL3_CB_MUL1 = 0,
    EXL3_CB_MCG = 1,
    EXL3_CB_SPEC1 = 2,
    EXL3_CB_PAIR1 = 3,
    EXL3_CB_STD1 = 4,
    EXL3_CB_3INST = 5
} exl3_codebook;

/* Codebook tables, in the order of codebook_tables.zig `shipped` (:101-106). */
typedef enum {
    EXL3_TABLE_NONE = -1,
    EXL3_TABLE_PAIR1_W16_V1 = 0,
    EXL3_TABLE_SPEC1_W15 = 1,
    EXL3_TABLE_SPEC1_W16 = 2,
    EXL3_TABLE_STD1 = 3
} exl3_table;

/* `Decode` (src/exl3/expert_exl3.zig:141-174): codebook, codeword window width (8..16) and table. */
typedef struct {
    int32_t codebook;
    int32_t window_bits;
    int32_t table;
} exl3_decode_t;

typedef enum { EXL3_DT_F16 = 0, EXL3_DT_BF16 = 1, EXL3_DT_F32 = 2 } exl3_dtype;

/* Status codes.  The reference's named Zig errors map one to one (src/exl3/root.zig:104-133, :421-423;
 * src/exl3/expert_exl3_kernels.zig:2569, :1475); DECLINED is the reference's `null` = "take the fallback"
 * (src/exl3/linear.zig:56-60, src/moe_gqmv.zig:574-577). */
typedef enum {
    EXL3_OK = 0,
    EXL3_DECLINED = 1,
    EXL3_ERR_BAD_SHAPE = -1,                 /* BadExl3Shape */
    EXL3_ERR_BAD_DTYPE = -2,                 /* BadExl3Dtype */
    EXL3_ERR_TABLE_UNKNOWN = -3,             /* Exl3CodebookTableUnknown */
    EXL3_ERR_TOPK_EXCEEDS_REDUCE = -4,       /* Exl3TopKExceedsReduceBank */
    EXL3_ERR_TOPK_UNSUPPORTED = -5,          /* Exl3TopkUnsupported */
    EXL3_ERR_INVALID_CLAMP = -6,             /* InvalidExl3Clamp */
    EXL3_ERR_SHARED_NEEDS_DECODE_ROWS = -7,  /* Exl3SharedNeedsDecodeRows */
    EXL3_ERR_LAUNCH = -8,                    /* Exl3GemmLaunchFailed / a HIP launch error */
    EXL3_ERR_WORKSPACE = -9,                 /* caller workspace too small or misaligned */
    EXL3_ERR_RATE_MISSING = -10,             /* Exl3CodebookTableRateMissing */
    EXL3_ERR_WINDOW = -11,                   /* Exl3WindowUnsupported; the encoder's WindowUnsupported */
    EXL3_ERR_CODEBOOK_UNSUPPORTED = -12,     /* encoder: CodebookUnsupported (src/encoder/encode.zig:7) */
    EXL3_ERR_RATE_UNSUPPORTED = -13,         /* encoder: RateUnsupported */
    EXL3_ERR_WINDOW_TOO_NARROW = -14,        /* encoder: WindowTooNarrow */
    EXL3_ERR_HESSIAN = -15,                  /* quantizer: HessianNotPositiveDefinite (src/encoder/quantize.zig:351) */
    EXL3_ERR_GROUP_MISSING = -16             /* Exl3GroupMissing (src/exl3/root.zig:647) */
} exl3_status;

/* One projection's bank (`Proj`, src/exl3/root.zig:28-30). */
typedef struct {
    const uint16_t *trellis;
    const uint16_t *suh;
    const uint16_t *svh;
    int32_t n;
} exl3_proj_t;

/* `Bank` (src/exl3/root.zig:39). */
typedef struct {
    exl3_proj_t gate, up, down;
} exl3_bank_t;

/* `Ragged` (src/exl3/rate_groups.zig:22-60): one ragged trellis per projection (experts' tiles contiguous, each
 * at its own rate), scales concatenated over experts, and the per-expert meta table of META_WORDS = 8 u32:
 * {n_gate, n_up, n_down, group, off_gate, off_up, off_down, local}, offsets in u32 words. */
typedef struct {
    const uint16_t *trellis[3];
    const uint16_t *suh[3];
    const uint16_t *svh[3];
    const uint32_t *meta; /* device [experts][8] */
    int32_t experts;
    /* Nonzero promises that every rate in `meta` is one of 16, 24, 32, 40, 48, 64 (the host builder knows the
     * rates, `rate_groups.zig` groups them); the library then skips the launch that serves any other rate.
     * Zero (the default of a zeroed struct) is always correct. */
    int32_t lane_rates_only;
} exl3_ragged_t;

/* A per-tile-rate bank (configs[4]'s seeded K1 / K2 tile mix).  No counterpart in the reference, which fixes a rate
 * per tensor (src/exl3/layout.zig:56-62) or per expert group (src/exl3/rate_groups.zig:22-140); each tile still
 * decodes at its own n as decodeTile does (src/exl3/expert_exl3.zig:338-357), so this is a layout extension.  A
 * segment is the 8 tiles (k-tile row tk, output tiles 8s .. 8s + 7) of one expert's projection: segment index
 * (e * in/16 + tk) * out/128 + s lies contiguous from u32 word seg_off[index] of the projection's trellis, tiles in
 * column order, tile o at n_a halfwords when bit o of seg_k1[index] is set, else at n_b.  n_a = 16, n_b = 32 (K1 and
 * K2); codebooks MCG, 3INST and the SPEC1 / STD1 hash rows whose table has both rates (spec1-w15).  Segments may lie
 * in any order; laying a column group's k-tile rows one after another ((e, s, tk) order, as sushi_amd's packer does)
 * keeps each 128-byte line of the stream in the one workgroup that reads its segments.  seg_k1 must be
 * 4-byte aligned.  Word offsets are u32, so one projection's trellis spans at most 16 GiB. */
typedef struct {
    const uint16_t *trellis[3]; /* gate, up, down */
    const uint32_t *seg_off[3]; /* device [experts][in/16][out/128] */
    const uint8_t *seg_k1[3];   /* device, same shape */
    const uint16_t *suh[3];     /* [experts][in] */
    const uint16_t *svh[3];     /* [experts][out] */
    int32_t experts;
    int32_t n_a, n_b;
} exl3_tiled_t;

int32_t exl3_abi_version(void);
const char *exl3_last_error(void);

/* Arm overrides for tests and tuning sweeps: no counterpart in the reference, whose arms are fixed per build, and
 * nothing a production caller needs.  Every knob starts unset (the library's own choice); exl3_set_override(knob,
 * value, 1) pins it and (knob, 0, 0) unsets it.  Process-wide, read at each call; change them only while no call
 * is being issued.  Nothing in the environment changes an arm. */
typedef enum {
    EXL3_KNOB_GEMV_SPLITS = 0,          /* k splits of the dense decode GEMV (must divide in/128; else ignored) */
    EXL3_KNOB_GEMV_SEPARATE_FINISH = 1, /* 1: split GEMVs finish in a second kernel */
    EXL3_KNOB_GEMV_FOLD = 2,            /* 0: split GEMVs finish through arrival counters + partial planes */
    EXL3_KNOB_MOE_DECODE_ROWS_MAX = 3,  /* rows up to which a routed layer takes the per-slot arm */
    EXL3_KNOB_MOE_SPLITS1 = 4,          /* k splits of the routed gate/up GEMV */
    EXL3_KNOB_MOE_SPLITS2 = 5,          /* k splits of the routed down GEMV */
    EXL3_KNOB_MOE_WINDOWS = 6,          /* 0: no sorted (expert-window) arm */
    EXL3_KNOB_MOE_FOLD = 7,             /* 0: the down projection writes planes and a reduce kernel finishes */
    EXL3_KNOB_MOE_GEMM = 8,             /* 1: a routed layer takes the GEMM arm where it can, 0: never */
    EXL3_KNOB_GEMM_ARM = 9,             /* dense GEMM body: 4 = decode-wave tile, 5 / 6 = ping-pong 512 / 256 rows,
                                           7 = ping-pong 512 rows with k in two halves */
    EXL3_KNOB_MOE_CHAIN = 10,           /* per-slot decode chain: 1 = gate/up and down in one launch where it
                                           serves, 0 = two launches (default: one launch for 2..8 rows with a fused
                                           shared bank) */
    EXL3_KNOB_GEMV_ROWS_PER_GROUP = 11, /* dense decode GEMV of 2..16 rows: rows per group of workgroups (the
                                           groups share the one bank and each decodes it; the last holds the rest;
                                           default: two groups from 5 rows on banks of <= 2048 x 2048, else whole) */
    EXL3_KNOB_GEMM_SPLIT_WAIT = 12,     /* the GEMM tile with k in halves: 100 MHz ticks the first half to finish
                                           waits for the second before handing it the whole tile (0: never waits;
                                           default: 20 us where both halves of every tile fit on the CUs at once,
                                           else 0) */
    EXL3_KNOB_COUNT = 13
} exl3_knob;
int32_t exl3_set_override(int32_t knob, int32_t value, int32_t enable);

/* Decodes `count` codewords (low `window_bits` kept) at rate n to f16 bits; PAIR1 writes two weights per codeword
 * (both weights of a pair come from the odd weight's codeword).  Replaces the Metal exhaustive-codeword test kernels
 * (src/exl3/kernel_source.zig:409-517) and the host `decodeCodeword`/`decodeHashMask`/`decodePair`
 * (src/exl3/expert_exl3.zig:267-311). */
int32_t exl3_decode_codewords(const uint16_t *codewords, int64_t count, int32_t n, exl3_decode_t dec, uint16_t *out,
                              hipStream_t stream);

/* `reconstructInner` (src/exl3/expert_exl3.zig:416-438): the dequantized f16 inner matrix [in][out] of one bank,
 * bit-exact with the reference decoder. */
int32_t exl3_reconstruct_inner(const uint16_t *trellis, int32_t in_features, int32_t out_features, int32_t n,
                               exl3_decode_t dec, uint16_t *out, hipStream_t stream);

/* `linear.linear` / `linearWith` (src/exl3/linear.zig:27-34) and `trunk.matmul` (src/exl3/trunk.zig:53-92):
 * y[rows][out] = finish(inner(prepare(x))) for one bank (trellis [1][in/16][out/16][n]).  Rows <= 16 take the
 * decode GEMV (projectRows, src/exl3/project_rows.zig:456-459, whose 8-row limit is raised to 16 here), wider the
 * MFMA GEMM (`run`, src/exl3/linear.zig:317-336).  in and out must be multiples of 128. */
size_t exl3_linear_workspace_size(int32_t rows, int32_t in_features, int32_t out_features, int32_t n);
int32_t exl3_linear(const void *x, int32_t x_dtype, int32_t rows, int32_t in_features, int32_t out_features,
                    const uint16_t *trellis, int32_t n, const uint16_t *suh, const uint16_t *svh, exl3_decode_t dec,
                    void *y, int32_t y_dtype, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* `linear.linearGrouped` (src/exl3/linear.zig:37-53): x [G][rows][in] through the G-bank projection
 * (trellis [G][in/16][out/16][n], suh [G][in], svh [G][out]), bank g serving x[g] -> y [G][rows][out]. */
size_t exl3_linear_grouped_workspace_size(int32_t groups, int32_t rows, int32_t in_features, int32_t out_features,
                                          int32_t n);
int32_t exl3_linear_grouped(const void *x, int32_t x_dtype, int32_t groups, int32_t rows, int32_t in_features,
                            int32_t out_features, const uint16_t *trellis, int32_t n, const uint16_t *suh,
                            const uint16_t *svh, exl3_decode_t dec, void *y, int32_t y_dtype, void *workspace,
                            size_t workspace_bytes, hipStream_t stream);

/* `linear.linear` without a workspace, for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference, which allocates
 * per call through MLX.  The same arms and results as exl3_linear; the scratch is a static device array of
 * EXL3_NOALLOC_SCRATCH_BYTES that each GPU holds until the process ends, so the call itself allocates nothing.
 * The first call on a device sets that scratch up (its address, and its zeroed region cleared by a fill kernel on
 * `stream`) and must run outside a stream capture; calls after it may be captured.  Every call on one GPU shares
 * that GPU's scratch: calls that overlap in time on one GPU (two streams, two threads) race, so issue them in
 * order.  A call whose scratch (exl3_linear_workspace_size) exceeds the limit returns EXL3_ERR_WORKSPACE before
 * any launch: the decode GEMV fits at every shape the reference serves; the GEMM arm fits while its prepared input
 * (rows rounded up to 16, x in f16) stays within the 24 MiB past the zeroed region. */
#define EXL3_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int32_t exl3_linear_noalloc(const void *x, int32_t x_dtype, int32_t rows, int32_t in_features, int32_t out_features,
                            const uint16_t *trellis, int32_t n, const uint16_t *suh, const uint16_t *svh,
                            exl3_decode_t dec, void *y, int32_t y_dtype, hipStream_t stream);

/* `linear.linearPair` (src/exl3/linear.zig:60-95): x [groups][rows][in] through the G-bank projection a (trellis
 * [G][in/16][mid/16][a_n], suh [G][in], svh [G][mid]), that result read as [rows][G * mid] through the one-bank
 * projection b (trellis [1][G*mid/16][out/16][b_n]) -> y [rows][out]: linearGrouped, the transpose and linear, bit
 * for bit, without the transpose (a's finish writes its rows as b reads them) and in two launches.  The intermediate
 * is in x's dtype, as the reference's is.  Returns EXL3_DECLINED (nothing launched) past one decode launch's 16 rows,
 * as the reference returns null past its multi-row launch; the caller then makes the three calls. */
size_t exl3_linear_pair_workspace_size(int32_t groups, int32_t rows, int32_t in_features, int32_t mid_features,
                                       int32_t out_features);
int32_t exl3_linear_pair(const void *x, int32_t x_dtype, int32_t groups, int32_t rows, int32_t in_features,
                         int32_t mid_features, int32_t out_features, const uint16_t *a_trellis, int32_t a_n,
                         const uint16_t *a_suh, const uint16_t *a_svh, exl3_decode_t a_dec,
                         const uint16_t *b_trellis, int32_t b_n, const uint16_t *b_suh, const uint16_t *b_svh,
                         exl3_decode_t b_dec, void *y, int32_t y_dtype, void *workspace, size_t workspace_bytes,
                         hipStream_t stream);

/* Clears a workspace once after allocation.  Every workspace begins with an 8 MiB region of fused-finish arrival
 * counters, accumulators and their overflow words that must start at zero; the calls that use them always leave them
 * at zero again, and no other call writes there, so one init per allocation suffices.  Calls that share a workspace
 * must not overlap in time (they would race on its scratch).  A small fill kernel, never hipMemsetAsync. */
int32_t exl3_workspace_init(void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Routed SwiGLU experts: `moe` (src/exl3/root.zig:51-53), `moeWithShared` (:56-67, `shared` [rows][hidden] in y's
 * dtype, added after the routed output's rounding as REDUCE_SHARED_SOURCE does,
 * src/exl3/expert_exl3_kernels.zig:2391-2406), `moeClamped` (:98-124, clamp_limit in 1..128, 0 = none).
 * x [rows][hidden]; inds [rows][topk] u32 (i32 accepted: same bits); scores [rows][topk] in scores_dtype (f32, bf16
 * or f16, as root.zig:114 admits).  Banks: gate/up trellis [E][hidden/16][inter/16][n], down
 * [E][inter/16][hidden/16][n]; each projection at its own rate (gate and up at different rates take one launch each,
 * as moeMixedDecode does, root.zig:705-722).  Arms: up to 8 rows the per-slot decode chain (pair GEMV -> fused
 * SwiGLU mid + down GEMV -> score-weighted fold or reduce); wider batches the same chain over expert windows of up to
 * 4 rows; prefill widths (from 4 slots per expert on average, every projection at one of the rates 16, 24, 32, 40,
 * 48, 64) the routed GEMM arm on the matrix cores (`moePrefill`, expert_exl3_kernels.zig:2861-2931).
 * verify_rows != 0 marks speculative-verify rows: as the reference does (root.zig:169, `rows <= DECODE_ROWS_MAX or
 * verify_rows`), they never take the GEMM arm, so they round as decode rows do at every width. */
size_t exl3_moe_workspace_size(int32_t rows, int32_t topk, int32_t hidden, int32_t inter);
int32_t exl3_moe(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter, int32_t experts,
                 const exl3_bank_t *bank, const uint32_t *inds, const void *scores, int32_t scores_dtype, int32_t topk,
                 exl3_decode_t dec, int32_t verify_rows, int32_t clamp_limit, const void *shared, void *y,
                 int32_t y_dtype, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* `moeWithGatedShared` (src/exl3/root.zig:71-90): y = routed + sigmoid(gate) * shared_down, with shared_down the shared
 * expert's output [rows][hidden] and shared_gate its gate logit [rows] (one per row), both in y's dtype T.  The terms
 * round in T where MLX's Sigmoid, Multiply and Add do (REDUCE_GATED_SHARED_SOURCE,
 * src/exl3/expert_exl3_kernels.zig:2410-2431): T(T(routed) + T(sig * shared)), sig = g < 0 ? rc : T(1 - rc),
 * rc = T(1 / T(1 + T(exp|g|))).  Workspace: exl3_moe_workspace_size. */
int32_t exl3_moe_with_gated_shared(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter,
                                   int32_t experts, const exl3_bank_t *bank, const uint32_t *inds, const void *scores,
                                   int32_t scores_dtype, int32_t topk, exl3_decode_t dec, int32_t verify_rows,
                                   const void *shared_down, const void *shared_gate, void *y, int32_t y_dtype,
                                   void *workspace, size_t workspace_bytes, hipStream_t stream);

/* `moeRagged` (src/exl3/root.zig:582-644) over a rate-grouped ragged bank (rate_groups.zig:22-140): each expert
 * decodes at its own (n_gate, n_up, n_down) read from the meta table.  `shared` and `shared_gate` as for exl3_moe and
 * exl3_moe_with_gated_shared (shared_gate non-null: y = T(T(routed) + T(sigmoid(gate) * shared)), gate [rows] in y's
 * dtype; it needs `shared`); the trunk's ragged call passes both (src/trunk.zig:4092).  verify_rows as exl3_moe.  At
 * prefill widths a bank whose rates are all lane-reader rates (`lane_rates_only`) takes the GEMM arm, each
 * workgroup at its expert's rate (`rate_groups.moePrefill`, rate_groups.zig:2039-2075). */
int32_t exl3_moe_ragged(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter,
                        const exl3_ragged_t *bank, const uint32_t *inds, const void *scores, int32_t scores_dtype,
                        int32_t topk, exl3_decode_t dec, int32_t verify_rows, int32_t clamp_limit,
                        const void *shared, const void *shared_gate, void *y, int32_t y_dtype, void *workspace,
                        size_t workspace_bytes, hipStream_t stream);

/* `moeGroups` (src/exl3/root.zig:646-703): a layer whose experts are split over `groups` uniform banks (banks[g] holds
 * group_experts[g] experts, router ids counted across the groups in order), each group's routed output computed in
 * f32 over every slot (a slot outside the group as local expert 0 with score 0, as the reference masks it), the
 * groups' outputs summed in f32 in group order and rounded to y's dtype once.  One group is `moe` itself.  banks and
 * group_experts are host arrays; every bank shares hidden and inter.  Refusals: EXL3_ERR_GROUP_MISSING without
 * groups, and exl3_moe's. */
size_t exl3_moe_groups_workspace_size(int32_t rows, int32_t topk, int32_t hidden, int32_t inter);
int32_t exl3_moe_groups(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter, int32_t groups,
                        const exl3_bank_t *banks, const int32_t *group_experts, const uint32_t *inds,
                        const void *scores, int32_t scores_dtype, int32_t topk, exl3_decode_t dec,
                        int32_t verify_rows, void *y, int32_t y_dtype, void *workspace, size_t workspace_bytes,
                        hipStream_t stream);

/* A routed layer and its shared expert in one call.  Replaces the caller's pair of calls: the shared expert as a
 * one-expert chain (inds 0, score 1; the pattern of src/dsv41/dsv41_model.zig:3000) and then `moeWithShared`
 * (src/exl3/root.zig:56-67) with that output.  The shared bank's rows run inside the routed launches (two launches
 * in all instead of four) and y = T(T(routed) + T(shared)), the rounding of the pair of calls (their k splits may
 * differ, so the f32 partial sums may round differently; both meet the same parity bar).  shared_bank is a
 * one-expert bank (trellis [1][hidden/16][inter/16][n] for gate/up, [1][inter/16][hidden/16][n] for down) with the
 * routed layer's inter; clamp_limit applies to both.  Up to 8 rows the shared rows join the per-slot launches (from
 * 2 rows one launch: the down workgroups wait, bounded, on a counter their group's gate/up workgroups raise);
 * wider batches the sorted (expert-window) launches, where the shared rows are windows of their own (three launches
 * in all instead of six); at prefill widths (the routed GEMM arm, from 4 slots per expert, not under verify_rows) the
 * shared expert is one more expert of the GEMM arm's launches, its rows extra slots, any y dtype, and y equals the
 * pair of calls bit for bit.  Returns EXL3_DECLINED (nothing launched) where the fused form does not serve: y dtype
 * f32 off the GEMM arm, routed projections at different rates, a shared rate other than the routed one (uniform
 * banks), rows whose routed, shared and combine fold words (3 x rows x hidden) exceed the fused finish's region, or
 * more fold arrivals than it holds; the caller then makes the two calls.  The _ragged form takes
 * `moeRagged`'s rate-grouped bank (src/exl3/root.zig:582-644); its shared bank keeps its own rate. */
size_t exl3_moe_with_shared_bank_workspace_size(int32_t rows, int32_t topk, int32_t hidden, int32_t inter);
int32_t exl3_moe_with_shared_bank(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter,
                                  int32_t experts, const exl3_bank_t *bank, const exl3_bank_t *shared_bank,
                                  const uint32_t *inds, const void *scores, int32_t scores_dtype, int32_t topk,
                                  exl3_decode_t dec, int32_t verify_rows, int32_t clamp_limit, void *y,
                                  int32_t y_dtype, void *workspace, size_t workspace_bytes, hipStream_t stream);
int32_t exl3_moe_ragged_with_shared_bank(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter,
                                         const exl3_ragged_t *bank, const exl3_bank_t *shared_bank,
                                         const uint32_t *inds, const void *scores, int32_t scores_dtype, int32_t topk,
                                         exl3_decode_t dec, int32_t verify_rows, int32_t clamp_limit, void *y,
                                         int32_t y_dtype, void *workspace, size_t workspace_bytes,
                                         hipStream_t stream);

/* `reconstructInner` (src/exl3/expert_exl3.zig:416-438) of expert `expert` of one per-tile-rate projection
 * (exl3_tiled_t's layout): the f16 inner matrix [in][out], each tile decoded at its own rate by the decoder the
 * routed GEMV multiplies with.  in a multiple of 16, out of 128. */
int32_t exl3_reconstruct_tiled(const uint16_t *trellis, const uint32_t *seg_off, const uint8_t *seg_k1,
                               int32_t expert, int32_t in_features, int32_t out_features, int32_t n_a, int32_t n_b,
                               exl3_decode_t dec, uint16_t *out, hipStream_t stream);

/* `moeRagged` (src/exl3/root.zig:582-644) over a per-tile-rate bank: the routed SwiGLU chain of exl3_moe (same
 * arguments, scores dtypes, clamp, `shared`, `shared_gate` and verify_rows), every tile at its own rate.  Up to 8 rows
 * the per-slot decode chain, wider batches the expert windows, prefill widths (not verify rows) the GEMM arm, whose
 * decode waves read each segment's offset and mask.  Workspace: exl3_moe_workspace_size.
 * The _with_shared_bank form runs a one-expert uniform shared bank (rate 16, 24, 32, 40, 48 or 64, decoded with the
 * routed codebook) inside the routed launches, as exl3_moe_with_shared_bank does, and declines where it does
 * (workspace: exl3_moe_with_shared_bank_workspace_size). */
int32_t exl3_moe_tiled(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter,
                       const exl3_tiled_t *bank, const uint32_t *inds, const void *scores, int32_t scores_dtype,
                       int32_t topk, exl3_decode_t dec, int32_t verify_rows, int32_t clamp_limit, const void *shared,
                       const void *shared_gate, void *y, int32_t y_dtype, void *workspace, size_t workspace_bytes,
                       hipStream_t stream);
int32_t exl3_moe_tiled_with_shared_bank(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter,
                                        const exl3_tiled_t *bank, const exl3_bank_t *shared_bank,
                                        const uint32_t *inds, const void *scores, int32_t scores_dtype, int32_t topk,
                                        exl3_decode_t dec, int32_t verify_rows, int32_t clamp_limit, void *y,
                                        int32_t y_dtype, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Router chain `moeRoutingChainOn` (src/moe_router.zig:22-62): top-k over f32 logits [rows][experts]
 * (ties to the lower expert index, listed in descending logit order), softmax over all experts, gathered and
 * renormalised over the k picked.  experts <= 1024, k <= 32. */
int32_t exl3_route_topk(const float *logits, int32_t rows, int32_t experts, int32_t k, uint32_t *inds,
                        float *scores, hipStream_t stream);

/* `layout.tileMajor` / `tileMajorInverse` (src/exl3/layout.zig:139-158): one projection of `experts` experts
 * between the pack order [IT][OT][n] and the pair-major order [OT/2][IT][2][n]. */
int32_t exl3_tile_major(const uint16_t *src, uint16_t *dst, int32_t experts, int32_t it, int32_t ot, int32_t n,
                        int32_t inverse, hipStream_t stream);

/* Trellis encoder search, `Encoder.encodeTile` (src/encoder/encode.zig:170-309) over `count` tiles: each row-major
 * 16x16 f32 tile of `tiles` [count][256] gets the packed codes [count][n] u16 of its least-squares tail-biting path
 * through the codebook (two passes: a free pass over the tile rolled by half pins the closing register, a pinned
 * pass writes the path), and, when `sse` is non-null, that path's f64 squared error [count].  Codes and errors are
 * the reference search's: f32 squared errors fused with the predecessor's f16 path cost, first minimum wins.
 * Codebooks MCG and MUL1 (and the 3INST extension), windows 12..16, every admitted rate whose fresh bits fit the
 * window; refusals: EXL3_ERR_CODEBOOK_UNSUPPORTED, EXL3_ERR_RATE_UNSUPPORTED, EXL3_ERR_WINDOW,
 * EXL3_ERR_WINDOW_TOO_NARROW.  The workspace holds the backpointers of the searches in flight; a smaller one than
 * exl3_encode_workspace_size() asks (but at least one workgroup's share) runs fewer searches at once. */
size_t exl3_encode_workspace_size(int32_t n, exl3_decode_t dec, int64_t count);
int32_t exl3_encode_tiles(const float *tiles, int64_t count, int32_t n, exl3_decode_t dec, uint16_t *packed,
                          double *sse, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* Whole-tensor quantizer, `quantizeTensor` (src/encoder/quantize.zig:600-626): a public weight w [in][out] f32 and
 * its input Hessian h [in][in] f32, with the sign vectors sign_in [in] / sign_out [out] (+-1), to the three tensors of
 * a pack: packed [in/16][out/16][n] u16, suh [in] and svh [out] as f16 bits, and the global scale g.  Regularizes
 * into the Hadamard basis (block-RMS input/output scales; out_scales 0 auto, 1 always, 2 never), rotates and
 * damps the Hessian and factors it as a 16-row block LDL, picks g by golden section over the codebook's bracket, and
 * searches the tiles in reverse LDLQ order with the error fed back through the factor -- the reference's arithmetic
 * throughout, so its codes.  The host pointers are read and written synchronously (the call returns when done); the
 * searches and the LDLQ run on `stream` in `workspace` (exl3_quantize_workspace_size bytes of device memory).
 * in and out are multiples of 128; refusals as exl3_encode_tiles, and EXL3_ERR_HESSIAN. */
size_t exl3_quantize_workspace_size(int32_t in, int32_t out, int32_t n, exl3_decode_t dec);
int32_t exl3_quantize_tensor(const float *w, const float *h, int32_t in, int32_t out, const float *sign_in,
                             const float *sign_out, int32_t n, exl3_decode_t dec, int32_t out_scales, uint16_t *packed,
                             uint16_t *suh, uint16_t *svh, float *g, void *workspace, size_t workspace_bytes,
                             hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif
