/*
 * CPU oracle for the EXL3/STQ trellis-quantized linear hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in plain C, the reference's CPU decoder and
 * reference arithmetic so that the HIP library can be checked against it.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only as the checker
 * (or, for the baseline, as the timed CPU port).  No product code path calls into it.
 *
 * Reference: beamivalice/sushi 1.7.2, src/exl3/expert_exl3.zig (cited per function in the .c).
 *
 * Parity status of each function (what pins it; see tests/test_oracle_*.py):
 *   ox_f32_to_f16 / ox_f16_to_f32 : exhaustive vs numpy's IEEE binary16 conversion.
 *   ox_bit_end                    : the reference's hand table (expert_exl3.zig:661-697) + closed form.
 *   ox_unpack_tile                : independent per-bit circular extraction (expert_exl3.zig:1051-1072).
 *   ox_tensor_core_perm           : bijection + reference fixtures (decoded tiles are position-exact).
 *   ox_decode_mcg / mul1          : reference KATs + golden fixtures' `inner` (bit-exact).
 *   ox_decode_hashmask            : reference KATs incl. rounded half sums (expert_exl3.zig:729-739).
 *   ox_decode_pair (PAIR1)        : reference KATs (expert_exl3.zig:770-795) + pair1 tile fixture.
 *   ox_table_row / ox_pair1_row   : sha256 digests of the tables equal the reference's pinned digests.
 *   ox_decode_3inst               : EXTENSION, not in the reference.  Pinned by closed form
 *                                   (LCG step then MCG's mask/xor/half-sum) and a linearity identity;
 *                                   the reference has no vectors for it ("parity unpinned" vs reference).
 *   ox_hadamard128                : Sylvester closed form (H*H = I, ±1/sqrt(128) entries) + fixtures' `public`.
 *   ox_reconstruct_inner/public   : golden fixtures, bit-exact.
 *   ox_prepare_input/inner_gemv/finish_output/ox_project : `project` vs dense matvec over `public`
 *                                   (relRms < 0.02, the reference's own bar) + FWHT equivalence.
 *   ox_moe_swiglu_host            : composition of ox_project + closed-form SwiGLU; checked against an
 *                                   independent numpy restatement over ox_decode_dense weights.
 *   ox_moe_swiglu_rows            : rows of ox_moe_swiglu_host over ragged banks; equals it row by row (and the
 *                                   threaded run equals the single-threaded one byte for byte).
 *   ox_*_tiled                    : EXTENSION (configs[4]'s per-tile K1/K2 map, no reference counterpart): the
 *                                   uniform functions applied tile by tile at each tile's own rate; equal to them
 *                                   when every tile has one rate, and to per-tile decodeTile reassembly otherwise.
 *   ox_gated_shared_term          : the rounding chain of REDUCE_GATED_SHARED_SOURCE; checked against numpy's
 *                                   float16 / an independent bf16 rounding of the same chain, every f16 and bf16 gate.
 *   ox_decode_dense               : equals the dense product diag(suh) H M H diag(svh) built by numpy.
 *   ox_route_topk                 : closed form (softmax, top-k, renormalise) vs numpy.
 *   ox_tile_major(_inverse)       : round trip + the reference's layout test (layout.zig:160-175).
 *   ox_viterbi_pass               : brute force over every tail-biting path on small windows (encode.zig:337-393).
 *   ox_exact_tail_biting          : the minimum of the brute force over every register.
 *   ox_encode_tile / ox_pack_states : the reference's search fixture (exl3_encode_tiles: packed codes and costs of
 *                                   the reference search, 13 codebook x rate x window configs, bit-exact); every
 *                                   packed tile decodes (ox_decode_tile) to the values the search scored; the
 *                                   half-roll warm-up pin reaches the exact tail-biting optimum (encode.zig:396-431).
 *   ox_quant_* / ox_quantize_tensor : the reference's tensor fixture (exl3_encode_tensor: regularized scales and
 *                                   inner matrix, and the packed codes, f16 scales and global scale of five whole
 *                                   tensors, bit-exact codes); the Cholesky factor multiplies back to its matrix and
 *                                   names the failing pivot; L carries H10 = L10 H00; the decoder's transform chain
 *                                   turns the regularized inner matrix back into the weight (quantize.zig:683-993).
 */
#ifndef SUSHI_EXL3_ORACLE_H
#define SUSHI_EXL3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    OX_CB_MUL1 = 0,
    OX_CB_MCG = 1,
    OX_CB_SPEC1 = 2,
    OX_CB_PAIR1 = 3,
    OX_CB_STD1 = 4,
    OX_CB_3INST = 5, /* extension: QTIP's 3INST, absent from the reference */
};

enum {
    OX_TABLE_NONE = -1,
    OX_TABLE_PAIR1_W16_V1 = 0,
    OX_TABLE_SPEC1_W15 = 1,
    OX_TABLE_SPEC1_W16 = 2,
    OX_TABLE_STD1 = 3,
};

typedef struct {
    int32_t codebook;    /* OX_CB_* */
    int32_t window_bits; /* 8..16 */
    int32_t table;       /* OX_TABLE_* or -1 */
} ox_decode;

typedef struct {
    uint32_t mult, rot, mask0, mask1, scale;
} ox_pair;

uint16_t ox_f32_to_f16(float f);
float ox_f16_to_f32(uint16_t h);

uint32_t ox_bit_end(uint32_t n, uint32_t t);
int ox_rate_admitted(uint32_t n);

uint16_t ox_decode_mcg(uint16_t cw);
uint16_t ox_decode_mul1(uint16_t cw);
uint16_t ox_decode_3inst(uint16_t cw);
uint16_t ox_decode_hashmask(uint16_t cw, uint32_t mult, uint32_t mask, uint32_t scale);
void ox_decode_pair(uint16_t cw, const ox_pair *p, uint16_t out[2]);

/* 1 when a row exists, 0 otherwise. */
int ox_pair1_row(uint32_t n, ox_pair *out);
int ox_table_row(int32_t table, uint32_t n, uint32_t row[4]);
int ox_table_count(void);
int ox_table_info(int32_t table, int32_t *codebook, int32_t *window_bits, uint32_t *n_lo, uint32_t *rows,
                  uint32_t *fields);

void ox_unpack_tile(const uint16_t *words, uint32_t n, uint16_t out[256]);
void ox_tensor_core_perm(uint32_t out[256]);
/* 0 ok; -1 no table row for this rate (the reference panics / refuses). */
int ox_decode_tile(const uint16_t *words, uint32_t n, ox_decode dec, uint16_t out[256]);
/* Decode a flat list of codewords (scalar codebooks) or of pair codewords (PAIR1: out has 2 per cw). */
int ox_decode_codewords(const uint16_t *cw, size_t count, uint32_t n, ox_decode dec, uint16_t *out);

void ox_hadamard128(float v[128]);
void ox_fwht128(float v[128]);

int ox_reconstruct_inner(const uint16_t *trellis, size_t in_features, size_t out_features, uint32_t n,
                         ox_decode dec, uint16_t *out);
int ox_reconstruct_public(const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh, size_t in_features,
                          size_t out_features, uint32_t n, ox_decode dec, uint16_t *out);

void ox_prepare_input(const float *x, const uint16_t *suh, size_t in_features, float *out);
int ox_inner_gemv(const uint16_t *trellis, const float *transformed, size_t in_features, size_t out_features,
                  uint32_t n, ox_decode dec, float *out);
void ox_finish_output(const float *inner, const uint16_t *svh, size_t out_features, float *out);
int ox_project(const float *x, const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh,
               size_t in_features, size_t out_features, uint32_t n, ox_decode dec, float *out);
/* rows x project; threads > 1 runs OpenMP over rows*output tiles (same arithmetic per element). */
int ox_project_rows(const float *x, size_t rows, const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh,
                    size_t in_features, size_t out_features, uint32_t n, ox_decode dec, int threads, float *out);

int ox_moe_swiglu_host(const float *x, const uint16_t *gate_t, const uint16_t *gate_suh, const uint16_t *gate_svh,
                       const uint16_t *up_t, const uint16_t *up_suh, const uint16_t *up_svh,
                       const uint16_t *down_t, const uint16_t *down_suh, const uint16_t *down_svh,
                       const uint32_t *slots, const float *weights, size_t topk, size_t hidden, size_t inter,
                       uint32_t n_gate, uint32_t n_up, uint32_t n_down, ox_decode dec, float clamp_limit,
                       float *y);

int ox_moe_swiglu_rows(const float *x, size_t rows, const uint16_t *gate_t, const uint16_t *gate_suh,
                       const uint16_t *gate_svh, const uint16_t *up_t, const uint16_t *up_suh, const uint16_t *up_svh,
                       const uint16_t *down_t, const uint16_t *down_suh, const uint16_t *down_svh,
                       const uint64_t *off_gate, const uint64_t *off_up, const uint64_t *off_down,
                       const uint32_t *n_gate, const uint32_t *n_up, const uint32_t *n_down, const uint32_t *slots,
                       const float *weights, size_t topk, size_t hidden, size_t inter, ox_decode dec,
                       float clamp_limit, int threads, float *y);

int ox_reconstruct_inner_tiled(const uint16_t *trellis, const uint32_t *seg_off, const uint8_t *seg_k1, size_t expert,
                               size_t in_features, size_t out_features, uint32_t n_a, uint32_t n_b, ox_decode dec,
                               uint16_t *out);
int ox_project_tiled(const float *x, const uint16_t *trellis, const uint32_t *seg_off, const uint8_t *seg_k1,
                     size_t expert, const uint16_t *suh, const uint16_t *svh, size_t in_features,
                     size_t out_features, uint32_t n_a, uint32_t n_b, ox_decode dec, float *out);
int ox_moe_swiglu_tiled_rows(const float *x, size_t rows, const uint16_t *const t[3], const uint32_t *const o[3],
                             const uint8_t *const k1[3], const uint16_t *const suh[3], const uint16_t *const svh[3],
                             uint32_t n_a, uint32_t n_b, const uint32_t *slots, const float *weights, size_t topk,
                             size_t hidden, size_t inter, ox_decode dec, float clamp_limit, int threads, float *y);
float ox_gated_shared_term(float gate, float shared, int dtype);
void ox_gated_shared_terms(const float *gate, const float *shared, size_t rows, size_t cols, int dtype, float *out);

int ox_decode_dense(const uint16_t *words, const uint16_t *suh, const uint16_t *svh, size_t in, size_t out,
                    uint32_t n, ox_decode dec, float *dst);

void ox_route_topk(const float *logits, size_t rows, size_t experts, size_t k, uint32_t *inds, float *scores);

void ox_tile_major(const uint16_t *src, uint16_t *dst, size_t it, size_t ot, size_t n);

/* Encoder search (src/encoder/encode.zig) */
double ox_viterbi_pass(const double *x, const uint8_t *ks, size_t steps, const double *table, uint32_t w,
                       int64_t pin, uint16_t *path);
double ox_exact_tail_biting(const double *x, const uint8_t *ks, size_t steps, const double *table, uint32_t w,
                            uint16_t *path);
void ox_pack_states(uint32_t n, const uint16_t states[256], uint16_t *out);
int ox_encode_tile(const float tile[256], uint32_t n, ox_decode dec, uint16_t *packed, float recon[256],
                   double *sse_out);

/* Quantizer (src/encoder/quantize.zig); mode 0 auto, 1 always, 2 never (OutScales). */
int ox_quant_regularize(const float *w, size_t in, size_t out, const float *sign_in, const float *sign_out, int mode,
                        const float *hdiag, float *inner, float *suh, float *svh);
int ox_quant_rotated_hessian(const float *h, const float *suh, size_t n, float *out);
size_t ox_cholesky_lower(double *a, size_t n);
int ox_quant_ldl_factor(const float *h, size_t n, float *l);
int ox_quant_global_scale(const float *inner, size_t rows, size_t cols, uint32_t n, ox_decode dec, float *g_out);
int ox_quant_ldlq(const float *inner, const float *l, size_t rows, size_t cols, uint32_t n, ox_decode dec,
                  uint16_t *packed, float *recon_out);
void ox_quant_signs(uint64_t seed, const char *name, size_t len, float *out);
int ox_quantize_tensor(const float *w, const float *h, size_t in, size_t out, const float *sign_in,
                       const float *sign_out, uint32_t n, ox_decode dec, int mode, uint16_t *packed, uint16_t *suh16,
                       uint16_t *svh16, float *g_out);
void ox_tile_major_inverse(const uint16_t *src, uint16_t *dst, size_t it, size_t ot, size_t n);

#ifdef __cplusplus
}
#endif
#endif
