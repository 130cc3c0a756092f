/*
 * CPU oracle for the EXL3/STQ trellis hot path -- TEST INFRASTRUCTURE ONLY (see exl3_oracle.h).
 *
 * A plain-C restatement of beamivalice/sushi's CPU decoder (src/exl3/expert_exl3.zig), its codebook tables
 * (src/exl3/codebook_tables.zig), the dense twin `decodeDense` (src/exl3/linear.zig:406-431), the MoE host
 * oracle `moeSwigluHost` (src/exl3/expert_exl3_kernels.zig:3059-3114), the router chain
 * (src/moe_router.zig:22-62) and the pair-major tile order (src/exl3/layout.zig:139-158).
 *
 * Arithmetic follows the reference's f32 order exactly (compile with -ffp-contract=off: the reference's
 * Zig never fuses a multiply into an add unless it says @mulAdd).
 */
#include "exl3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------------ */
/* binary16 <-> binary32, round to nearest even (the reference's @floatCast).                        */

float ox_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0x1Fu) {
        bits = sign | 0x7F800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {
        /* subnormal: man * 2^-24 is exact in binary32 */
        float v = (float)man * 5.9604644775390625e-08f;
        memcpy(&bits, &v, 4);
        bits |= sign;
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t ox_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) { /* inf / nan */
        if (ax == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
    if (ax >= 0x38800000u) {                                  /* normal binary16 range */
        uint32_t r = ax - 0x38000000u;                          /* rebias 127 -> 15 */
        uint32_t lsb = (r >> 13) & 1u;
        r += 0xFFFu + lsb;
        return (uint16_t)(sign | (r >> 13));
    }
    /* subnormal binary16 (or zero): q = value / 2^-24, rounded to nearest even */
    uint32_t e = ax >> 23;
    if (e < 102u) return (uint16_t)sign;
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126u - e; /* 14..24 */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q);
}

static inline float f16r(float v) { return ox_f16_to_f32(ox_f32_to_f16(v)); }

/* ------------------------------------------------------------------------------------------------ */
/* Rates: expert_exl3.zig:180-245                                                                   */

uint32_t ox_bit_end(uint32_t n, uint32_t t) { return ((t + 1u) * n) >> 4; }

int ox_rate_admitted(uint32_t n) { return (n % 2u == 0u) && n >= 16u && n <= 128u; } /* kFromPackedDim :241-245 */

/* ------------------------------------------------------------------------------------------------ */
/* Codebooks: expert_exl3.zig:10-11, :267-311                                                       */

static inline float half_pair_sum(uint32_t halves) {
    return ox_f16_to_f32((uint16_t)(halves & 0xFFFFu)) + ox_f16_to_f32((uint16_t)(halves >> 16));
}

uint16_t ox_decode_mcg(uint16_t cw) { /* decodeMcg, expert_exl3.zig:267-273 */
    uint32_t mixed = (uint32_t)cw * 0xCBAC1FEDu;
    uint32_t pair = 0x3B603B60u ^ (mixed & 0x8FFF8FFFu);
    return ox_f32_to_f16(half_pair_sum(pair));
}

uint16_t ox_decode_mul1(uint16_t cw) { /* decodeMul1, expert_exl3.zig:275-284 */
    uint32_t mixed = (uint32_t)cw * 0x83DCD12Du;
    uint32_t byte_sum = (mixed & 0xFFu) + ((mixed >> 8) & 0xFFu) + ((mixed >> 16) & 0xFFu) + (mixed >> 24);
    float h = ox_f16_to_f32((uint16_t)(0x6400u + byte_sum));
    float inverse = ox_f16_to_f32(0x1EEEu);
    float bias = ox_f16_to_f32(0xC931u);
    return ox_f32_to_f16(fmaf(h, inverse, bias));
}

/* EXTENSION (not in the reference): QTIP's 3INST codebook, as published with QTIP / exllamav3:
 * an LCG step x = 89226354 * x + 64248484 (mod 2^32), then MCG's mask/xor and the f16 half sum. */
uint16_t ox_decode_3inst(uint16_t cw) {
    uint32_t mixed = (uint32_t)cw * 89226354u + 64248484u;
    uint32_t pair = 0x3B603B60u ^ (mixed & 0x8FFF8FFFu);
    return ox_f32_to_f16(half_pair_sum(pair));
}

static uint16_t half_sum_scaled(uint32_t halves, uint32_t scale) { /* halfSumScaled, expert_exl3.zig:292-295 */
    uint16_t sum = ox_f32_to_f16(half_pair_sum(halves));
    return ox_f32_to_f16(ox_f16_to_f32(sum) * (float)scale);
}

uint16_t ox_decode_hashmask(uint16_t cw, uint32_t mult, uint32_t mask, uint32_t scale) { /* :288-290 */
    return half_sum_scaled(((uint32_t)cw * mult) & mask, scale);
}

static inline uint32_t rotl32(uint32_t v, uint32_t r) { return r == 0 ? v : (v << r) | (v >> (32u - r)); }

void ox_decode_pair(uint16_t cw, const ox_pair *p, uint16_t out[2]) { /* decodePair, expert_exl3.zig:298-301 */
    uint32_t product = (uint32_t)cw * p->mult;
    out[0] = half_sum_scaled(product & p->mask0, p->scale);
    out[1] = half_sum_scaled(rotl32(product, p->rot) & p->mask1, p->scale);
}

/* ------------------------------------------------------------------------------------------------ */
/* Tables: PAIR1 rows (expert_exl3.zig:24-46) and the STQ tables (codebook_tables.zig:101-200).      */

static const uint32_t PAIR1_ROWS[21][4] = {
    /* mult, rot, mask0, mask1 for n = 24, 26, ..., 64 */
    {0x58F41BF3u, 3, 0x8ED78C13u, 0x8EEE8C03u}, {0x58F41BF3u, 3, 0x8ED78C13u, 0x8EEE8C03u},
    {0x7AA2BE15u, 3, 0x8ED78C13u, 0x8ECE8C03u}, {0x7B229E11u, 3, 0x8ED78C13u, 0x8ECE8C03u},
    {0x3B22BE15u, 3, 0x8ED78C13u, 0x8ECE8C03u}, {0x46C63E17u, 19, 0x8F9A8E6Eu, 0x8E258FFEu},
    {0x46C63E17u, 19, 0x8F9A8E6Eu, 0x8E258FFEu}, {0x46C63E17u, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0x46C63E17u, 19, 0x8F9A8E6Eu, 0x8E258FFEu}, {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu}, {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu}, {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu}, {0xF75D60FFu, 19, 0x8E6E8F9Au, 0x8E258FFEu},
    {0x82439F67u, 19, 0x8E6E8F9Au, 0x8E258FAEu}, {0xE2C7FC0Du, 19, 0x8F408FB0u, 0x8F918F89u},
    {0xE2C7FC0Du, 19, 0x8F408FA0u, 0x8F118FC9u}, {0xE2C7FC0Du, 19, 0x8F408FA0u, 0x8F118FC9u},
    {0xE2C7FC0Du, 19, 0x8F408FA0u, 0x8F118FC9u},
};

int ox_pair1_row(uint32_t n, ox_pair *out) { /* pair1Pair, expert_exl3.zig:49-52 */
    if (n % 2u != 0u || n < 24u || n > 64u) return 0;
    const uint32_t *r = PAIR1_ROWS[(n - 24u) / 2u];
    out->mult = r[0];
    out->rot = r[1];
    out->mask0 = r[2];
    out->mask1 = r[3];
    out->scale = 4096u;
    return 1;
}

/* spec1-w15, n = 16..128 (codebook_tables.zig:110-170) */
static const uint32_t SPEC1_W15[57][2] = {
    {0x84d1cf89u, 0x8fe08947u}, {0x84c1cf49u, 0x8fe48a47u}, {0x84d1cfe9u, 0x8fe08a47u}, {0x84d1cfc9u, 0x8ff08b67u},
    {0x84c1cf49u, 0x8fe08b47u}, {0x84c1cf99u, 0x8fa08b66u}, {0x862c1d37u, 0x8ff28c50u}, {0x84641fb7u, 0x8fa08c40u},
    {0x846c1fa7u, 0x8fe08c80u}, {0x844c1fd7u, 0x8ffe8c98u}, {0x846c1fa7u, 0x8ffe8d10u}, {0x845c1f77u, 0x8ffa8e10u},
    {0x843c1fa7u, 0x8ffe8e40u}, {0x843c1fa7u, 0x8ffe8e40u}, {0x842c1fc7u, 0x8fff8f00u}, {0x843c1fb7u, 0x8ffe8f10u},
    {0x84181fb5u, 0x8fe08f80u}, {0x84081f75u, 0x8ffa8f72u}, {0x84081f75u, 0x8fd68fd0u}, {0x84241f27u, 0x8ffc8fc0u},
    {0x84081f73u, 0x8fe08f80u}, {0x84081f75u, 0x8fbe8ff0u}, {0x3fed4cefu, 0x8fe08fe0u}, {0x3fed4cefu, 0x8fc18ff2u},
    {0x3fed4cefu, 0x8ff08ff0u}, {0x3fed4cefu, 0x8fe28ff0u}, {0x3fed4cefu, 0x8fe08fe0u}, {0x80081b7bu, 0x8ff08fc8u},
    {0x80081b7bu, 0x8ff48fc0u}, {0x400036cbu, 0x8f448fffu}, {0x400036cbu, 0x8fe48fffu}, {0x400036cbu, 0x8f448ff9u},
    {0x8000387bu, 0x8fe08ff7u}, {0x8000387bu, 0x8fc08feeu}, {0x80003779u, 0x8fe88ffeu}, {0x80003779u, 0x8fc88ffcu},
    {0x80003779u, 0x8fca8ffcu}, {0x80003779u, 0x8fcc8ffeu}, {0x80003879u, 0x8ffc8fefu}, {0x50003851u, 0x8ff98fffu},
    {0xd0003751u, 0x8ff98fffu}, {0x50003851u, 0x8ff98ff6u}, {0xd0003931u, 0x8ff98fffu}, {0xd0003931u, 0x8ff98ffau},
    {0xd0003931u, 0x8ff48ffau}, {0x300031b1u, 0x8ffb8ffcu}, {0x300031b1u, 0x8ffa8ffeu}, {0x300031b1u, 0x8ffb8ffcu},
    {0xc00031f1u, 0x8ffe8ffau}, {0x400031f1u, 0x8ffe8ffeu}, {0x400031f1u, 0x8ffe8ffeu}, {0x40003931u, 0x8ffc8ffcu},
    {0x40003931u, 0x8ffc8ffcu}, {0x40003931u, 0x8ff88ffeu}, {0x40003931u, 0x8ff88ffcu}, {0x80003811u, 0x8ffc8ffcu},
    {0x80003811u, 0x8ffc8ffcu},
};

/* spec1-w16, n = 24..64 (codebook_tables.zig:173-197) */
static const uint32_t SPEC1_W16[21][2] = {
    {0x862d1c19u, 0x8fee8c30u}, {0x862d1d37u, 0x8fee8c30u}, {0x862d1d37u, 0x8ffe8c10u}, {0x842f1f37u, 0x8ffc8d10u},
    {0x840f1f67u, 0x8ffc8d10u}, {0x844f1f77u, 0x8ffe8d40u}, {0x840d1f37u, 0x8ffe8e10u}, {0x84091f33u, 0x8fe88e00u},
    {0x844d1f77u, 0x8fe08e00u}, {0x843c1fa7u, 0x8ffe8e40u}, {0x844c1f7fu, 0x8ffc8f02u}, {0x841c1fb9u, 0x8fe88f04u},
    {0x842c1fc7u, 0x8ffe8fd0u}, {0x83fc1fa3u, 0x8ffe8fd0u}, {0x83fc1fa3u, 0x8ffe8fc1u}, {0x83fc1fa3u, 0x8ffe8fd0u},
    {0x83fc1fa3u, 0x8fee8fc0u}, {0x84061f77u, 0x8fd08f80u}, {0x84081f6fu, 0x8ffe8fc0u}, {0x84081f25u, 0x8ffe8fe0u},
    {0x83f81f6fu, 0x8ff48fc0u},
};

/* std1: one pair at every rate n = 24..64 (codebook_tables.zig:200) */
static const uint32_t STD1_PAIR[2] = {0x840C1F37u, 0x8FFE8FD0u};

typedef struct {
    int32_t codebook, window_bits;
    uint32_t n_lo, rows, fields;
} table_info;

/* Order matches codebook_tables.zig `shipped` (:101-106). */
static const table_info TABLES[4] = {
    {OX_CB_PAIR1, 16, 24, 21, 4},
    {OX_CB_SPEC1, 15, 16, 57, 2},
    {OX_CB_SPEC1, 16, 24, 21, 2},
    {OX_CB_STD1, 15, 24, 21, 2},
};

int ox_table_count(void) { return 4; }

int ox_table_info(int32_t table, int32_t *codebook, int32_t *window_bits, uint32_t *n_lo, uint32_t *rows,
                  uint32_t *fields) {
    if (table < 0 || table >= 4) return 0;
    *codebook = TABLES[table].codebook;
    *window_bits = TABLES[table].window_bits;
    *n_lo = TABLES[table].n_lo;
    *rows = TABLES[table].rows;
    *fields = TABLES[table].fields;
    return 1;
}

int ox_table_row(int32_t table, uint32_t n, uint32_t row[4]) { /* Table.row, codebook_tables.zig:49-53 */
    if (table < 0 || table >= 4) return 0;
    const table_info *t = &TABLES[table];
    if (n % 2u != 0u || n < t->n_lo) return 0;
    uint32_t i = (n - t->n_lo) / 2u;
    if (i >= t->rows) return 0;
    row[2] = row[3] = 0;
    switch (table) {
    case OX_TABLE_PAIR1_W16_V1:
        memcpy(row, PAIR1_ROWS[i], 16);
        return 1;
    case OX_TABLE_SPEC1_W15:
        row[0] = SPEC1_W15[i][0];
        row[1] = SPEC1_W15[i][1];
        return 1;
    case OX_TABLE_SPEC1_W16:
        row[0] = SPEC1_W16[i][0];
        row[1] = SPEC1_W16[i][1];
        return 1;
    default:
        row[0] = STD1_PAIR[0];
        row[1] = STD1_PAIR[1];
        return 1;
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* Bitstream and tile layout: expert_exl3.zig:313-398                                               */

/* Stream bit b of a tile (MSB-first over u32 words, word i = hw[2i] | hw[2i+1] << 16). */
static inline uint32_t stream_word(const uint16_t *hw, uint32_t i) {
    return (uint32_t)hw[2u * i] | ((uint32_t)hw[2u * i + 1u] << 16);
}

void ox_unpack_tile(const uint16_t *words, uint32_t n, uint16_t out[256]) {
    /* Codeword t is the 16 stream bits ending (exclusively) at bitEnd(t); the stream is circular
     * (tail-biting), so the first windows reach back into the tile's last word (unpackTile :317-336). */
    const uint32_t nwords = n / 2u;
    const uint32_t total = 16u * n;
    for (uint32_t t = 0; t < 256u; t++) {
        uint32_t end = ox_bit_end(n, t);            /* exclusive */
        uint32_t last = (end + total - 1u) % total; /* last bit of the window */
        uint32_t wl = last / 32u;
        uint32_t wp = (wl + nwords - 1u) % nwords;
        uint64_t two = ((uint64_t)stream_word(words, wp) << 32) | stream_word(words, wl);
        uint32_t shift = 31u - (last % 32u); /* bits after `last` in its word */
        out[t] = (uint16_t)((two >> shift) & 0xFFFFu);
    }
}

void ox_tensor_core_perm(uint32_t out[256]) { /* tensorCorePerm, expert_exl3.zig:379-398 */
    for (uint32_t lane = 0; lane < 32u; lane++) {
        uint32_t r0 = (lane % 4u) * 2u;
        uint32_t c0 = lane / 4u;
        uint32_t rows[4] = {r0, r0 + 1u, r0 + 8u, r0 + 9u};
        for (uint32_t i = 0; i < 8u; i++) out[lane * 8u + i] = rows[i % 4u] * 16u + c0 + (i >= 4u ? 8u : 0u);
    }
}

static int hash_row_for(ox_decode dec, uint32_t n, uint32_t *mult, uint32_t *mask) { /* Decode.hashMask :168-173 */
    if (dec.codebook != OX_CB_SPEC1 && dec.codebook != OX_CB_STD1) return 0;
    if (dec.table < 0) return 0;
    uint32_t row[4];
    if (!ox_table_row(dec.table, n, row)) return 0;
    *mult = row[0];
    *mask = row[1];
    return 1;
}

static inline uint16_t window_mask(int32_t bits) { return bits >= 16 ? 0xFFFFu : (uint16_t)((1u << bits) - 1u); }

int ox_decode_tile(const uint16_t *words, uint32_t n, ox_decode dec, uint16_t out[256]) { /* decodeTile :338-357 */
    uint16_t cws[256];
    uint32_t perm[256];
    ox_unpack_tile(words, n, cws);
    ox_tensor_core_perm(perm);
    const uint16_t mask = window_mask(dec.window_bits);
    if (dec.codebook == OX_CB_PAIR1) {
        ox_pair p;
        if (!ox_pair1_row(n, &p)) return -1;
        for (uint32_t j = 0; j < 128u; j++) {
            uint16_t w[2];
            ox_decode_pair((uint16_t)(cws[2u * j + 1u] & mask), &p, w);
            out[perm[2u * j]] = w[0];
            out[perm[2u * j + 1u]] = w[1];
        }
        return 0;
    }
    uint32_t mult = 0, hmask = 0;
    int tabled = dec.codebook == OX_CB_SPEC1 || dec.codebook == OX_CB_STD1;
    if (tabled && !hash_row_for(dec, n, &mult, &hmask)) return -1;
    for (uint32_t i = 0; i < 256u; i++) {
        uint16_t cw = (uint16_t)(cws[i] & mask);
        uint16_t v;
        switch (dec.codebook) {
        case OX_CB_MCG: v = ox_decode_mcg(cw); break;
        case OX_CB_MUL1: v = ox_decode_mul1(cw); break;
        case OX_CB_3INST: v = ox_decode_3inst(cw); break;
        default: v = ox_decode_hashmask(cw, mult, hmask, 4096u); break;
        }
        out[perm[i]] = v;
    }
    return 0;
}

int ox_decode_codewords(const uint16_t *cw, size_t count, uint32_t n, ox_decode dec, uint16_t *out) {
    const uint16_t mask = window_mask(dec.window_bits);
    if (dec.codebook == OX_CB_PAIR1) {
        ox_pair p;
        if (!ox_pair1_row(n, &p)) return -1;
        for (size_t i = 0; i < count; i++) ox_decode_pair((uint16_t)(cw[i] & mask), &p, out + 2 * i);
        return 0;
    }
    uint32_t mult = 0, hmask = 0;
    int tabled = dec.codebook == OX_CB_SPEC1 || dec.codebook == OX_CB_STD1;
    if (tabled && !hash_row_for(dec, n, &mult, &hmask)) return -1;
    for (size_t i = 0; i < count; i++) {
        uint16_t c = (uint16_t)(cw[i] & mask);
        switch (dec.codebook) {
        case OX_CB_MCG: out[i] = ox_decode_mcg(c); break;
        case OX_CB_MUL1: out[i] = ox_decode_mul1(c); break;
        case OX_CB_3INST: out[i] = ox_decode_3inst(c); break;
        default: out[i] = ox_decode_hashmask(c, mult, hmask, 4096u); break;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------ */
/* Hadamard: expert_exl3.zig:7, :400-414                                                            */

#define HAD_SCALE 0.08838834764831845f

void ox_hadamard128(float v[128]) {
    /* Dense Sylvester product, entry(r, k) = (-1)^popcount(r & k) / sqrt(128), summed in k order. */
    float tmp[128];
    for (int r = 0; r < 128; r++) {
        float acc = 0.0f;
        for (int k = 0; k < 128; k++) {
            float e = (__builtin_popcount((unsigned)(r & k)) & 1) ? -HAD_SCALE : HAD_SCALE;
            acc += e * v[k];
        }
        tmp[r] = acc;
    }
    memcpy(v, tmp, sizeof(tmp));
}

/* O(n log n) butterfly of the same transform (summation order differs; used only by the timed
 * multi-core CPU variant and to cross-check the dense form within f32 rounding). */
void ox_fwht128(float v[128]) {
    for (int h = 1; h < 128; h <<= 1) {
        for (int i = 0; i < 128; i += 2 * h) {
            for (int j = i; j < i + h; j++) {
                float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
        }
    }
    for (int i = 0; i < 128; i++) v[i] *= HAD_SCALE;
}

/* ------------------------------------------------------------------------------------------------ */
/* Dense reconstruction: expert_exl3.zig:416-488                                                   */

int ox_reconstruct_inner(const uint16_t *trellis, size_t in_features, size_t out_features, uint32_t n,
                         ox_decode dec, uint16_t *out) {
    size_t it = in_features / 16, ot = out_features / 16;
    uint16_t tile[256];
    for (size_t tk = 0; tk < it; tk++) {
        for (size_t tn = 0; tn < ot; tn++) {
            if (ox_decode_tile(trellis + (tk * ot + tn) * n, n, dec, tile) != 0) return -1;
            for (size_t r = 0; r < 16; r++) memcpy(out + (tk * 16 + r) * out_features + tn * 16, tile + r * 16, 32);
        }
    }
    return 0;
}

int ox_reconstruct_public(const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh, size_t in_features,
                          size_t out_features, uint32_t n, ox_decode dec, uint16_t *out) {
    size_t total = in_features * out_features;
    uint16_t *inner = (uint16_t *)malloc(total * 2);
    float *w = (float *)malloc(total * 4);
    if (!inner || !w) {
        free(inner);
        free(w);
        return -2;
    }
    if (ox_reconstruct_inner(trellis, in_features, out_features, n, dec, inner) != 0) {
        free(inner);
        free(w);
        return -1;
    }
    for (size_t i = 0; i < total; i++) w[i] = ox_f16_to_f32(inner[i]);
    float vec[128];
    for (size_t rb = 0; rb < in_features; rb += 128) {
        for (size_t c = 0; c < out_features; c++) {
            for (size_t r = 0; r < 128; r++) vec[r] = w[(rb + r) * out_features + c];
            ox_hadamard128(vec);
            for (size_t r = 0; r < 128; r++) w[(rb + r) * out_features + c] = vec[r];
        }
    }
    for (size_t r = 0; r < in_features; r++) {
        float s = ox_f16_to_f32(suh[r]);
        for (size_t c = 0; c < out_features; c++) w[r * out_features + c] *= s;
    }
    for (size_t cb = 0; cb < out_features; cb += 128) {
        for (size_t r = 0; r < in_features; r++) {
            ox_hadamard128(w + r * out_features + cb);
        }
    }
    for (size_t c = 0; c < out_features; c++) {
        float s = ox_f16_to_f32(svh[c]);
        for (size_t r = 0; r < in_features; r++) w[r * out_features + c] *= s;
    }
    for (size_t i = 0; i < total; i++) out[i] = ox_f32_to_f16(w[i]);
    free(inner);
    free(w);
    return 0;
}

/* ------------------------------------------------------------------------------------------------ */
/* project: expert_exl3.zig:490-566                                                                */

void ox_prepare_input(const float *x, const uint16_t *suh, size_t in_features, float *out) {
    for (size_t i = 0; i < in_features; i++) out[i] = f16r(x[i]) * ox_f16_to_f32(suh[i]);
    for (size_t b = 0; b < in_features; b += 128) {
        ox_hadamard128(out + b);
        for (size_t i = 0; i < 128; i++) out[b + i] = f16r(out[b + i]);
    }
}

int ox_inner_gemv(const uint16_t *trellis, const float *transformed, size_t in_features, size_t out_features,
                  uint32_t n, ox_decode dec, float *out) {
    size_t it = in_features / 16, ot = out_features / 16;
    uint16_t tile[256];
    float wf[256];
    memset(out, 0, out_features * sizeof(float));
    for (size_t tk = 0; tk < it; tk++) {
        for (size_t tn = 0; tn < ot; tn++) {
            if (ox_decode_tile(trellis + (tk * ot + tn) * n, n, dec, tile) != 0) return -1;
            for (int i = 0; i < 256; i++) wf[i] = ox_f16_to_f32(tile[i]);
            const float *xb = transformed + tk * 16;
            float *yb = out + tn * 16;
            for (int r = 0; r < 16; r++) {
                float xv = xb[r];
                for (int c = 0; c < 16; c++) yb[c] += xv * wf[r * 16 + c];
            }
        }
    }
    for (size_t i = 0; i < out_features; i++) out[i] = f16r(out[i]);
    return 0;
}

void ox_finish_output(const float *inner, const uint16_t *svh, size_t out_features, float *out) {
    memcpy(out, inner, out_features * sizeof(float));
    for (size_t b = 0; b < out_features; b += 128) ox_hadamard128(out + b);
    for (size_t i = 0; i < out_features; i++) out[i] = f16r(out[i] * ox_f16_to_f32(svh[i]));
}

int ox_project(const float *x, const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh,
               size_t in_features, size_t out_features, uint32_t n, ox_decode dec, float *out) {
    float *transformed = (float *)malloc(in_features * sizeof(float));
    float *inner = (float *)malloc(out_features * sizeof(float));
    if (!transformed || !inner) {
        free(transformed);
        free(inner);
        return -2;
    }
    ox_prepare_input(x, suh, in_features, transformed);
    int rc = ox_inner_gemv(trellis, transformed, in_features, out_features, n, dec, inner);
    if (rc == 0) ox_finish_output(inner, svh, out_features, out);
    free(transformed);
    free(inner);
    return rc;
}

/* Multi-row project for the CPU baseline.  threads <= 1: the reference's single-threaded order,
 * row by row.  threads > 1: OpenMP over (row, output tile), each element's arithmetic identical
 * (a column's sum still runs tk by tk and r by r), so both variants give the same bytes. */
int ox_project_rows(const float *x, size_t rows, const uint16_t *trellis, const uint16_t *suh, const uint16_t *svh,
                    size_t in_features, size_t out_features, uint32_t n, ox_decode dec, int threads, float *out) {
    if (threads <= 1) {
        for (size_t r = 0; r < rows; r++) {
            int rc = ox_project(x + r * in_features, trellis, suh, svh, in_features, out_features, n, dec,
                                out + r * out_features);
            if (rc) return rc;
        }
        return 0;
    }
    size_t it = in_features / 16, ot = out_features / 16;
    float *prep = (float *)malloc(rows * in_features * sizeof(float));
    float *inner = (float *)malloc(rows * out_features * sizeof(float));
    if (!prep || !inner) {
        free(prep);
        free(inner);
        return -2;
    }
    int bad = 0;
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads) schedule(static)
#endif
    for (long r = 0; r < (long)rows; r++) ox_prepare_input(x + r * in_features, suh, in_features, prep + r * in_features);
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads) schedule(dynamic, 4) reduction(| : bad)
#endif
    for (long job = 0; job < (long)ot; job++) {
        uint16_t tile[256];
        float wf[256];
        float acc[64][16];
        for (size_t r0 = 0; r0 < rows; r0 += 64) {
            size_t nr = rows - r0 < 64 ? rows - r0 : 64;
            memset(acc, 0, sizeof(acc));
            for (size_t tk = 0; tk < it; tk++) {
                if (ox_decode_tile(trellis + (tk * ot + (size_t)job) * n, n, dec, tile) != 0) {
                    bad |= 1;
                    break;
                }
                for (int i = 0; i < 256; i++) wf[i] = ox_f16_to_f32(tile[i]);
                for (size_t rr = 0; rr < nr; rr++) {
                    const float *xb = prep + (r0 + rr) * in_features + tk * 16;
                    for (int r = 0; r < 16; r++) {
                        float xv = xb[r];
                        for (int c = 0; c < 16; c++) acc[rr][c] += xv * wf[r * 16 + c];
                    }
                }
            }
            for (size_t rr = 0; rr < nr; rr++)
                for (int c = 0; c < 16; c++) inner[(r0 + rr) * out_features + (size_t)job * 16 + c] = f16r(acc[rr][c]);
        }
    }
#ifdef _OPENMP
#pragma omp parallel for num_threads(threads) schedule(static)
#endif
    for (long r = 0; r < (long)rows; r++) ox_finish_output(inner + r * out_features, svh, out_features, out + r * out_features);
    free(prep);
    free(inner);
    return bad ? -1 : 0;
}

/* ------------------------------------------------------------------------------------------------ */
/* MoE host oracle: expert_exl3_kernels.zig:3059-3114 (+ the GPU mid's clamp, :2296-2305).          */

int ox_moe_swiglu_host(const float *x, const uint16_t *gate_t, const uint16_t *gate_suh, const uint16_t *gate_svh,
                       const uint16_t *up_t, const uint16_t *up_suh, const uint16_t *up_svh,
                       const uint16_t *down_t, const uint16_t *down_suh, const uint16_t *down_svh,
                       const uint32_t *slots, const float *weights, size_t topk, size_t hidden, size_t inter,
                       uint32_t n_gate, uint32_t n_up, uint32_t n_down, ox_decode dec, float clamp_limit,
                       float *y) {
    size_t tiles = (hidden / 16) * (inter / 16);
    float *gy = (float *)malloc(inter * 4), *uy = (float *)malloc(inter * 4), *h = (float *)malloc(inter * 4);
    float *dy = (float *)malloc(hidden * 4);
    int rc = 0;
    if (!gy || !uy || !h || !dy) rc = -2;
    memset(y, 0, hidden * sizeof(float));
    for (size_t k = 0; k < topk && rc == 0; k++) {
        size_t e = slots[k];
        rc = ox_project(x, gate_t + e * tiles * n_gate, gate_suh + e * hidden, gate_svh + e * inter, hidden, inter,
                        n_gate, dec, gy);
        if (rc) break;
        rc = ox_project(x, up_t + e * tiles * n_up, up_suh + e * hidden, up_svh + e * inter, hidden, inter, n_up,
                        dec, uy);
        if (rc) break;
        for (size_t i = 0; i < inter; i++) {
            float g = gy[i], u = uy[i];
            if (clamp_limit > 0.0f) {
                g = fminf(g, clamp_limit);
                u = fminf(fmaxf(u, -clamp_limit), clamp_limit);
            }
            h[i] = (g / (1.0f + expf(-g))) * u;
        }
        rc = ox_project(h, down_t + e * tiles * n_down, down_suh + e * inter, down_svh + e * hidden, inter, hidden,
                        n_down, dec, dy);
        if (rc) break;
        float w = weights[k];
        for (size_t i = 0; i < hidden; i++) y[i] += w * dy[i];
    }
    free(gy);
    free(uy);
    free(h);
    free(dy);
    return rc;
}

/* ------------------------------------------------------------------------------------------------ */
/* decodeDense: linear.zig:406-431                                                                   */

int ox_decode_dense(const uint16_t *words, const uint16_t *suh, const uint16_t *svh, size_t in, size_t out,
                    uint32_t n, ox_decode dec, float *dst) {
    uint16_t tile[256];
    size_t ot = out / 16;
    for (size_t tk = 0; tk < in / 16; tk++)
        for (size_t tn = 0; tn < ot; tn++) {
            if (ox_decode_tile(words + (tk * ot + tn) * n, n, dec, tile) != 0) return -1;
            for (size_t r = 0; r < 16; r++)
                for (size_t c = 0; c < 16; c++) dst[(tk * 16 + r) * out + tn * 16 + c] = ox_f16_to_f32(tile[r * 16 + c]);
        }
    float col[128];
    for (size_t b = 0; b < in; b += 128)
        for (size_t j = 0; j < out; j++) {
            for (size_t i = 0; i < 128; i++) col[i] = dst[(b + i) * out + j];
            ox_hadamard128(col);
            for (size_t i = 0; i < 128; i++) dst[(b + i) * out + j] = col[i];
        }
    for (size_t i = 0; i < in; i++) {
        float *row = dst + i * out;
        for (size_t o = 0; o < out; o += 128) ox_hadamard128(row + o);
        float su = ox_f16_to_f32(suh[i]);
        for (size_t j = 0; j < out; j++) row[j] *= su * ox_f16_to_f32(svh[j]);
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------ */
/* Router: moe_router.zig:22-62.  Top-k by logit (ties: lower expert index first, listed in          */
/* descending logit order), softmax over all experts, gathered and renormalised over the k picked.  */

void ox_route_topk(const float *logits, size_t rows, size_t experts, size_t k, uint32_t *inds, float *scores) {
    for (size_t r = 0; r < rows; r++) {
        const float *l = logits + r * experts;
        float mx = -INFINITY;
        for (size_t e = 0; e < experts; e++) mx = l[e] > mx ? l[e] : mx;
        double denom = 0.0;
        for (size_t e = 0; e < experts; e++) denom += exp((double)l[e] - (double)mx);
        uint32_t *ir = inds + r * k;
        for (size_t j = 0; j < k; j++) {
            size_t best = (size_t)-1;
            for (size_t e = 0; e < experts; e++) {
                int taken = 0;
                for (size_t q = 0; q < j; q++) taken |= ir[q] == e;
                if (taken) continue;
                if (best == (size_t)-1 || l[e] > l[best]) best = e;
            }
            ir[j] = (uint32_t)best;
        }
        double picked[64];
        double sum = 0.0;
        for (size_t j = 0; j < k; j++) {
            picked[j] = exp((double)l[ir[j]] - (double)mx) / denom;
            sum += picked[j];
        }
        for (size_t j = 0; j < k; j++) scores[r * k + j] = (float)(picked[j] / sum);
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* Pair-major tile order: layout.zig:139-158                                                        */

void ox_tile_major(const uint16_t *src, uint16_t *dst, size_t it, size_t ot, size_t n) {
    for (size_t pair = 0; pair < ot / 2; pair++)
        for (size_t tk = 0; tk < it; tk++)
            for (size_t o = 0; o < 2; o++)
                memcpy(dst + ((pair * it + tk) * 2 + o) * n, src + (tk * ot + pair * 2 + o) * n, n * 2);
}

void ox_tile_major_inverse(const uint16_t *src, uint16_t *dst, size_t it, size_t ot, size_t n) {
    for (size_t pair = 0; pair < ot / 2; pair++)
        for (size_t tk = 0; tk < it; tk++)
            for (size_t o = 0; o < 2; o++)
                memcpy(dst + (tk * ot + pair * 2 + o) * n, src + ((pair * it + tk) * 2 + o) * n, n * 2);
}

/* ------------------------------------------------------------------------------------------------ */
/* Encoder search: src/encoder/encode.zig                                                            */

/* viterbiPass (encode.zig:46-101): least-squares path of x through table[0..2^w), one codeword per step,
 * cw_t = ((cw_{t-1} << k_t) | f_t) & (2^w - 1).  pin >= 0 fixes the register entering step 0 (cw_0 >> k_0) and
 * requires the last codeword to carry it in its low w - k_0 bits.  f64 throughout; the first minimum wins. */
double ox_viterbi_pass(const double *x, const uint8_t *ks, size_t steps, const double *table, uint32_t w,
                       int64_t pin, uint16_t *path) {
    const size_t states = (size_t)1 << w;
    uint32_t kmin = 31;
    for (size_t i = 0; i < steps; i++) kmin = ks[i] < kmin ? ks[i] : kmin;
    const size_t stride = (size_t)1 << (w - kmin);
    double *prev = malloc(states * sizeof(double)), *next = malloc(states * sizeof(double));
    double *best = malloc(stride * sizeof(double));
    uint8_t *back = calloc(steps * stride, 1);
    const uint32_t k0 = ks[0];
    for (size_t cw = 0; cw < states; cw++) {
        double d = x[0] - table[cw];
        prev[cw] = (pin >= 0 && (int64_t)(cw >> k0) != pin) ? INFINITY : d * d;
    }
    for (size_t i = 1; i < steps; i++) {
        const uint32_t k = ks[i];
        const size_t s = (size_t)1 << (w - k), kk = (size_t)1 << k;
        uint8_t *row = back + i * stride;
        for (size_t low = 0; low < s; low++) { best[low] = prev[low]; row[low] = 0; }
        for (size_t j = 1; j < kk; j++)
            for (size_t low = 0; low < s; low++)
                if (prev[j * s + low] < best[low]) { best[low] = prev[j * s + low]; row[low] = (uint8_t)j; }
        for (size_t low = 0; low < s; low++)
            for (size_t f = 0; f < kk; f++) {
                double d = x[i] - table[low * kk + f];
                next[low * kk + f] = best[low] + d * d;
            }
        double *t = prev; prev = next; next = t;
    }
    double best_cost = INFINITY;
    size_t cur = 0;
    const size_t reg_mask = ((size_t)1 << (w - k0)) - 1;
    for (size_t cw = 0; cw < states; cw++) {
        if (pin >= 0 && (int64_t)(cw & reg_mask) != pin) continue;
        if (prev[cw] < best_cost) { best_cost = prev[cw]; cur = cw; }
    }
    path[steps - 1] = (uint16_t)cur;
    for (size_t i = steps - 1; i > 0; i--) {
        const uint32_t k = ks[i];
        size_t low = cur >> k;
        cur = ((size_t)back[i * stride + low] << (w - k)) | low;
        path[i - 1] = (uint16_t)cur;
    }
    free(prev); free(next); free(best); free(back);
    return best_cost;
}

/* exactTailBiting (encode.zig:104-118): every register in turn, the cheapest pinned pass. */
double ox_exact_tail_biting(const double *x, const uint8_t *ks, size_t steps, const double *table, uint32_t w,
                            uint16_t *path) {
    uint16_t *tmp = malloc(steps * sizeof(uint16_t));
    double best = INFINITY;
    for (int64_t reg = 0; reg < ((int64_t)1 << (w - ks[0])); reg++) {
        double c = ox_viterbi_pass(x, ks, steps, table, w, reg, tmp);
        if (c < best) { best = c; memcpy(path, tmp, steps * sizeof(uint16_t)); }
    }
    free(tmp);
    return best;
}

/* Encoder.packStates (encode.zig:296-309): the fresh k_t low bits of each state, MSB first, at the bits ending at
 * bitEnd(t), in the loader's stream order (32-bit big-endian words of two swapped halfwords). */
void ox_pack_states(uint32_t n, const uint16_t states[256], uint16_t *out) {
    memset(out, 0, n * sizeof(uint16_t));
    for (uint32_t t = 0; t < 256; t++) {
        const uint32_t end = ox_bit_end(n, t);
        const uint32_t k = end - (t == 0 ? 0 : ox_bit_end(n, t - 1));
        for (uint32_t b = 0; b < k; b++) {
            const uint16_t bit = (states[t] >> (k - 1 - b)) & 1u;
            const uint32_t p = end - k + b;
            const uint32_t half = (p / 32) * 2 + (p % 32 < 16 ? 1 : 0);
            out[half] |= (uint16_t)(bit << (15 - p % 16));
        }
    }
}

/* Encoder.encodeTile (encode.zig:170-294): the two-pass tail-biting search of one row-major 16x16 tile.  Pass 0 runs
 * free over the tile rolled by half and traces back to the register entering step 0; pass 1 is pinned to it and
 * writes the path.  Costs follow the reference's arithmetic: f32 squared error (fused with the predecessor's cost),
 * f16 path costs clamped at 65504, one-byte backpointers, first minimum wins.  Returns 0 and the path's f64 squared
 * error, or -1 codebook (not MCG/MUL1, or this build's 3INST extension), -2 rate, -3 window outside 12..16, -4 window
 * too narrow for the rate. */
int ox_encode_tile(const float tile[256], uint32_t n, ox_decode dec, uint16_t *packed, float recon[256],
                   double *sse_out) {
    if (dec.codebook != OX_CB_MCG && dec.codebook != OX_CB_MUL1 && dec.codebook != OX_CB_3INST) return -1;
    if (!ox_rate_admitted(n)) return -2;
    if (dec.window_bits < 12 || dec.window_bits > 16) return -3;
    const uint32_t w = (uint32_t)dec.window_bits;
    uint8_t ks[256];
    uint32_t kmin = 31, kmax = 0;
    for (uint32_t t = 0; t < 256; t++) {
        ks[t] = (uint8_t)(ox_bit_end(n, t) - (t == 0 ? 0 : ox_bit_end(n, t - 1)));
        kmin = ks[t] < kmin ? ks[t] : kmin;
        kmax = ks[t] > kmax ? ks[t] : kmax;
    }
    if (kmax >= w) return -4;
    uint32_t perm[256];
    ox_tensor_core_perm(perm);
    const size_t stride = (size_t)1 << (w - kmin);
    float *table = malloc(((size_t)1 << w) * sizeof(float));
    for (size_t cw = 0; cw < ((size_t)1 << w); cw++)
        table[cw] = ox_f16_to_f32(dec.codebook == OX_CB_MCG    ? ox_decode_mcg((uint16_t)cw)
                                  : dec.codebook == OX_CB_MUL1 ? ox_decode_mul1((uint16_t)cw)
                                                               : ox_decode_3inst((uint16_t)cw));
    uint16_t *costs[2] = {malloc(stride * sizeof(uint16_t)), malloc(stride * sizeof(uint16_t))};
    uint8_t *back = calloc(256 * stride, 1);
    float x[256];
    uint16_t path[256];
    for (int i = 0; i < 256; i++) x[i] = tile[perm[i]];
    const float h_inf = 65504.0f;
    size_t pin = 0;
    int pinned = 0;
    for (int pass = 0; pass < 2; pass++) {
        const size_t roll = pass == 0 ? 128 : 0;
        uint16_t *prev = costs[0], *curr = costs[1];
        for (size_t step = 0; step < 256; step++) {
            const size_t ri = (step + roll) & 255;
            const uint32_t k = ks[ri], k_next = ks[(ri + 1) & 255];
            const uint32_t kr = w - k_next;
            const size_t kk = (size_t)1 << k_next, edges = (size_t)1 << kr;
            const float target = x[ri];
            uint8_t *row = back + ri * stride;
            for (size_t e = 0; e < edges; e++) {
                float best = h_inf;
                uint8_t best_fresh = 0;
                for (size_t fresh = 0; fresh < kk; fresh++) {
                    const size_t cw = (fresh << kr) | e;
                    const size_t pred = cw >> k;
                    const float dh = table[cw] - target;
                    float err;
                    if (step == 0) {
                        if (pinned && pred != pin) err = h_inf;
                        else { float sq = dh * dh; err = sq < h_inf ? sq : h_inf; }
                    } else {
                        err = fmaf(dh, dh, ox_f16_to_f32(prev[pred]));
                    }
                    if (err < best) { best = err; best_fresh = (uint8_t)fresh; }
                }
                curr[e] = ox_f32_to_f16(best);
                row[e] = best_fresh;
            }
            uint16_t *t = prev; prev = curr; curr = t;
        }
        size_t edge = pin;
        if (pass == 0) {
            const size_t final_edges = (size_t)1 << (w - ks[0]);
            float best = h_inf;
            edge = 0;
            for (size_t e = 0; e < final_edges; e++) {
                const float v = ox_f16_to_f32(prev[e]);
                if (v < best) { best = v; edge = e; }
            }
        }
        for (size_t step_i = 256; step_i > 0;) {
            step_i--;
            const size_t ri = (step_i + roll) & 255;
            const uint32_t k = ks[ri], k_next = ks[(ri + 1) & 255];
            const uint32_t kr = w - k_next;
            const size_t state = ((size_t)back[ri * stride + edge] << kr) | edge;
            edge = state >> k;
            if (pass == 1) path[ri] = (uint16_t)state;
            else if (ri == 0) break;
        }
        pin = edge;
        pinned = 1;
    }
    ox_pack_states(n, path, packed);
    double sse = 0.0;
    for (int i = 0; i < 256; i++) {
        const double d = (double)x[i] - (double)table[path[i]];
        sse += d * d;
    }
    if (recon)
        for (int i = 0; i < 256; i++) recon[perm[i]] = table[path[i]];
    *sse_out = sse;
    free(table); free(costs[0]); free(costs[1]); free(back);
    return 0;
}
