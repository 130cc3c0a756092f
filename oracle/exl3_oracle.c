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

/* Rows of tokens through moeSwigluHost: row r takes slots / weights [r * topk, (r + 1) * topk).  threads > 1 runs
 * OpenMP over rows (each row's arithmetic is the single-row function's, so both give the same bytes).  The banks are
 * ragged: expert e of projection p starts at halfword off[p][e] of its trellis and decodes at rate n[p][e] (a
 * uniform bank is off[p][e] = e * tiles * n). */
int ox_moe_swiglu_rows(const float *x, size_t rows, const uint16_t *gate_t, const uint16_t *gate_suh,
                       const uint16_t *gate_svh, const uint16_t *up_t, const uint16_t *up_suh, const uint16_t *up_svh,
                       const uint16_t *down_t, const uint16_t *down_suh, const uint16_t *down_svh,
                       const uint64_t *off_gate, const uint64_t *off_up, const uint64_t *off_down,
                       const uint32_t *n_gate, const uint32_t *n_up, const uint32_t *n_down, const uint32_t *slots,
                       const float *weights, size_t topk, size_t hidden, size_t inter, ox_decode dec,
                       float clamp_limit, int threads, float *y) {
    int bad = 0;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 1 ? threads : 1) reduction(| : bad)
    for (long r = 0; r < (long)rows; r++) {
        float *yr = y + r * hidden;
        memset(yr, 0, hidden * sizeof(float));
        float *dy = (float *)malloc(hidden * sizeof(float));
        if (!dy) {
            bad |= 1;
            continue;
        }
        for (size_t k = 0; k < topk; k++) {
            const size_t e = slots[r * topk + k];
            const uint32_t one = 0;
            const float w1 = 1.0f;
            /* one expert through the single-row function, its bank pointers moved to expert e */
            int rc = ox_moe_swiglu_host(x + r * hidden, gate_t + off_gate[e], gate_suh + e * hidden,
                                        gate_svh + e * inter, up_t + off_up[e], up_suh + e * hidden, up_svh + e * inter,
                                        down_t + off_down[e], down_suh + e * inter, down_svh + e * hidden, &one, &w1, 1,
                                        hidden, inter, n_gate[e], n_up[e], n_down[e], dec, clamp_limit, dy);
            if (rc) {
                bad |= 1;
                break;
            }
            const float w = weights[r * topk + k];
            for (size_t i = 0; i < hidden; i++) yr[i] += w * dy[i];
        }
        free(dy);
    }
    return bad ? -1 : 0;
}

/* ------------------------------------------------------------------------------------------------ */
/* Per-tile rates: configs[4]'s seeded K1/K2 tile mix, a layout extension with no counterpart in the reference (whose  */
/* rate is per tensor or per expert group, layout.zig:56-62, rate_groups.zig:22-140).  Each tile decodes at its own   */
/* rate with decodeTile (expert_exl3.zig:338-357).  Layout of one bank of E experts, in_features x out_features:      */
/* segment (e, tk, s) = tiles (tk, 8s .. 8s + 7) of expert e lies contiguous from halfword 2 * seg_off[(e * it + tk)  */
/* * (ot / 8) + s] of the trellis, in column order, tile o at n_a halfwords when bit o of seg_k1[same index] is set,   */
/* else at n_b.                                                                                                      */

static const uint16_t *ox_tiled_tile(const uint16_t *trellis, const uint32_t *seg_off, const uint8_t *seg_k1,
                                     size_t seg, size_t o, uint32_t n_a, uint32_t n_b, uint32_t *n) {
    const uint8_t m = seg_k1[seg];
    size_t hw = 2 * (size_t)seg_off[seg];
    for (size_t q = 0; q < o; q++) hw += (m >> q) & 1 ? n_a : n_b;
    *n = (m >> o) & 1 ? n_a : n_b;
    return trellis + hw;
}

int ox_reconstruct_inner_tiled(const uint16_t *trellis, const uint32_t *seg_off, const uint8_t *seg_k1, size_t expert,
                               size_t in_features, size_t out_features, uint32_t n_a, uint32_t n_b, ox_decode dec,
                               uint16_t *out) {
    const size_t it = in_features / 16, ot = out_features / 16, segs = ot / 8;
    uint16_t tile[256];
    for (size_t tk = 0; tk < it; tk++)
        for (size_t tn = 0; tn < ot; tn++) {
            uint32_t n;
            const uint16_t *w = ox_tiled_tile(trellis, seg_off, seg_k1, (expert * it + tk) * segs + tn / 8, tn % 8,
                                              n_a, n_b, &n);
            if (ox_decode_tile(w, n, dec, tile) != 0) return -1;
            for (int r = 0; r < 16; r++)
                for (int c = 0; c < 16; c++)
                    out[(tk * 16 + r) * out_features + tn * 16 + c] = tile[r * 16 + c];
        }
    return 0;
}

/* `project` (expert_exl3.zig:546-566) over expert `expert` of a per-tile-rate bank. */
int ox_project_tiled(const float *x, const uint16_t *trellis, const uint32_t *seg_off, const uint8_t *seg_k1,
                     size_t expert, const uint16_t *suh, const uint16_t *svh, size_t in_features,
                     size_t out_features, uint32_t n_a, uint32_t n_b, ox_decode dec, float *out) {
    const size_t it = in_features / 16, ot = out_features / 16, segs = ot / 8;
    float *prep = (float *)malloc(in_features * sizeof(float));
    float *inner = (float *)malloc(out_features * sizeof(float));
    if (!prep || !inner) {
        free(prep);
        free(inner);
        return -2;
    }
    ox_prepare_input(x, suh, in_features, prep);
    memset(inner, 0, out_features * sizeof(float));
    uint16_t tile[256];
    float wf[256];
    int rc = 0;
    for (size_t tk = 0; tk < it && rc == 0; tk++)
        for (size_t tn = 0; tn < ot; tn++) {
            uint32_t n;
            const uint16_t *w = ox_tiled_tile(trellis, seg_off, seg_k1, (expert * it + tk) * segs + tn / 8, tn % 8,
                                              n_a, n_b, &n);
            if (ox_decode_tile(w, n, dec, tile) != 0) {
                rc = -1;
                break;
            }
            for (int i = 0; i < 256; i++) wf[i] = ox_f16_to_f32(tile[i]);
            const float *xb = prep + tk * 16;
            float *yb = inner + tn * 16;
            for (int r = 0; r < 16; r++)
                for (int c = 0; c < 16; c++) yb[c] += xb[r] * wf[r * 16 + c];
        }
    if (rc == 0) {
        for (size_t i = 0; i < out_features; i++) inner[i] = f16r(inner[i]);
        ox_finish_output(inner, svh, out_features, out);
    }
    free(prep);
    free(inner);
    return rc;
}

/* moeSwigluHost (expert_exl3_kernels.zig:3059-3114) over rows of tokens on per-tile-rate banks: t/o/k[p] are
 * projection p's trellis, seg_off and seg_k1 (gate, up, down); suh/svh as for a uniform bank.  OpenMP over rows. */
int ox_moe_swiglu_tiled_rows(const float *x, size_t rows, const uint16_t *const t[3], const uint32_t *const o[3],
                             const uint8_t *const k1[3], const uint16_t *const suh[3], const uint16_t *const svh[3],
                             uint32_t n_a, uint32_t n_b, const uint32_t *slots, const float *weights, size_t topk,
                             size_t hidden, size_t inter, ox_decode dec, float clamp_limit, int threads, float *y) {
    int bad = 0;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 1 ? threads : 1) reduction(| : bad)
    for (long r = 0; r < (long)rows; r++) {
        float *yr = y + r * hidden;
        memset(yr, 0, hidden * sizeof(float));
        float *gy = (float *)malloc(inter * 4), *uy = (float *)malloc(inter * 4), *h = (float *)malloc(inter * 4);
        float *dy = (float *)malloc(hidden * 4);
        if (!gy || !uy || !h || !dy) bad |= 1;
        for (size_t k = 0; k < topk && !bad; k++) {
            const size_t e = slots[r * topk + k];
            int rc = ox_project_tiled(x + r * hidden, t[0], o[0], k1[0], e, suh[0] + e * hidden, svh[0] + e * inter,
                                      hidden, inter, n_a, n_b, dec, gy);
            rc |= ox_project_tiled(x + r * hidden, t[1], o[1], k1[1], e, suh[1] + e * hidden, svh[1] + e * inter,
                                   hidden, inter, n_a, n_b, dec, uy);
            for (size_t i = 0; i < inter; i++) {
                float g = gy[i], u = uy[i];
                if (clamp_limit > 0.0f) {
                    g = fminf(g, clamp_limit);
                    u = fminf(fmaxf(u, -clamp_limit), clamp_limit);
                }
                h[i] = (g / (1.0f + expf(-g))) * u;
            }
            rc |= ox_project_tiled(h, t[2], o[2], k1[2], e, suh[2] + e * inter, svh[2] + e * hidden, inter, hidden,
                                   n_a, n_b, dec, dy);
            if (rc) {
                bad |= 1;
                break;
            }
            const float w = weights[r * topk + k];
            for (size_t i = 0; i < hidden; i++) yr[i] += w * dy[i];
        }
        free(gy);
        free(uy);
        free(h);
        free(dy);
    }
    return bad ? -1 : 0;
}

/* ------------------------------------------------------------------------------------------------ */
/* The gated shared expert's term: REDUCE_GATED_SHARED_SOURCE, expert_exl3_kernels.zig:2410-2431.  In T = dtype   */
/* (0 f16, 1 bf16, 2 f32): ex = T(exp|g|), rc = T(1 / T(1 + ex)), sig = g < 0 ? rc : T(1 - rc), term = T(sig * sh). */
/* exp is evaluated in double and rounded to float (the kernel's own choice for Metal's precise::exp).             */

static float ox_bf16r(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    if ((u & 0x7F800000u) == 0x7F800000u) { /* inf stays, NaN stays NaN */
        if (u & 0x007FFFFFu) u |= 0x00400000u;
    } else {
        u += 0x7FFFu + ((u >> 16) & 1u); /* round to nearest even */
    }
    u &= 0xFFFF0000u;
    memcpy(&v, &u, 4);
    return v;
}

static float ox_round_dt(int dtype, float v) { return dtype == 0 ? f16r(v) : dtype == 1 ? ox_bf16r(v) : v; }

float ox_gated_shared_term(float gate, float shared, int dtype) {
    const float ex = ox_round_dt(dtype, (float)exp(fabs((double)gate)));
    const float rc = ox_round_dt(dtype, 1.0f / ox_round_dt(dtype, 1.0f + ex));
    const float sig = gate < 0.0f ? rc : ox_round_dt(dtype, 1.0f - rc);
    return ox_round_dt(dtype, sig * shared);
}

/* out[r][c] = ox_gated_shared_term(gate[r], shared[r][c], dtype) over a [rows][cols] block. */
void ox_gated_shared_terms(const float *gate, const float *shared, size_t rows, size_t cols, int dtype, float *out) {
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) out[r * cols + c] = ox_gated_shared_term(gate[r], shared[r * cols + c], dtype);
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
/* A NaN logit selects as -inf (the fused router's "v > best" never takes it, moe_router.zig:137-141) */
/* and no expert is picked twice; the NaN still reaches the softmax, so the row's scores are NaN.   */

static double ox_route_key(float v) { return v != v ? -INFINITY : (double)v; }

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
                if (best == (size_t)-1 || ox_route_key(l[e]) > ox_route_key(l[best])) best = e;
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

/* ------------------------------------------------------------------------------------------------ */
/* Quantizer: src/encoder/quantize.zig (regularize, rotatedHessian, ldlFactor, globalScale, ldlq)     */

#define OXQ_HAD 128
static const float OXQ_SIGMA_REG = 0.025f;
static const float OXQ_CODEBOOK_SCALE = 1.24371088f;

/* fwht (quantize.zig:33-47) on a strided vector: butterflies, then x * (1/sqrt(128)) in T. */
static void oxq_fwht_f32(float *v, size_t step) {
    for (size_t h = 1; h < OXQ_HAD; h *= 2)
        for (size_t i = 0; i < OXQ_HAD; i += 2 * h)
            for (size_t j = i; j < i + h; j++) {
                const float a = v[j * step], b = v[(j + h) * step];
                v[j * step] = a + b;
                v[(j + h) * step] = a - b;
            }
    const float scale = 1.0f / sqrtf((float)OXQ_HAD);
    for (size_t k = 0; k < OXQ_HAD; k++) v[k * step] *= scale;
}

static void oxq_fwht_f64(double *v, size_t step) {
    for (size_t h = 1; h < OXQ_HAD; h *= 2)
        for (size_t i = 0; i < OXQ_HAD; i += 2 * h)
            for (size_t j = i; j < i + h; j++) {
                const double a = v[j * step], b = v[(j + h) * step];
                v[j * step] = a + b;
                v[(j + h) * step] = a - b;
            }
    const double scale = 1.0 / sqrt((double)OXQ_HAD);
    for (size_t k = 0; k < OXQ_HAD; k++) v[k * step] *= scale;
}

static int oxq_desc(const void *a, const void *b) {
    const float x = *(const float *)a, y = *(const float *)b;
    return (x < y) - (x > y);
}

/* chooseApplyOutScales (quantize.zig:88-116); mode 0 auto, 1 always, 2 never. */
static int oxq_apply_out_scales(int mode, const float *hdiag, size_t len) {
    const int forced = mode == 1 ? 1 : mode == 2 ? 0 : -1;
    if (!hdiag) return forced >= 0 ? forced : 1;
    double sum = 0;
    for (size_t i = 0; i < len; i++) sum += hdiag[i] > 0 ? hdiag[i] : 0.0f;
    const double mean = sum / (double)len;
    if (!isfinite(mean) || mean < 1e-20) return forced >= 0 ? forced : 0;
    if (forced >= 0) return forced;
    float *diag = malloc(len * sizeof(float));
    const float damp = (float)((double)OXQ_SIGMA_REG * mean);
    for (size_t i = 0; i < len; i++) diag[i] = sqrtf((hdiag[i] > 0 ? hdiag[i] : 0.0f) + damp);
    qsort(diag, len, sizeof(float), oxq_desc);
    const size_t cutoff = len / 50 > 1 ? len / 50 : 1;
    double top = 0, all = 0;
    for (size_t i = 0; i < len; i++) {
        if (i < cutoff) top += diag[i];
        all += diag[i];
    }
    free(diag);
    return top / all < 0.15;
}

/* regularize (quantize.zig:129-189): public weight [in][out] -> inner, suh, svh (f32), public =
 * diag(suh) H_L inner H_R diag(svh).  Returns 0, -1 geometry. */
int ox_quant_regularize(const float *w, size_t in, size_t out, const float *sign_in, const float *sign_out, int mode,
                        const float *hdiag, float *inner, float *suh, float *svh) {
    if (in == 0 || out == 0 || in % OXQ_HAD || out % OXQ_HAD) return -1;
    memcpy(inner, w, in * out * sizeof(float));
    memcpy(svh, sign_out, out * sizeof(float));
    float *os = calloc(out, sizeof(float));
    int apply = oxq_apply_out_scales(mode, hdiag, in);
    for (size_t c = 0; c < out; c++) {
        float total = 0;
        for (size_t r0 = 0; r0 < in; r0 += 32) {
            float block = 0;
            for (size_t r = r0; r < r0 + 32 && r < in; r++) block += inner[r * out + c] * inner[r * out + c];
            total += block;
        }
        os[c] = sqrtf(total / (float)in);
    }
    double mean_sum = 0;
    for (size_t c = 0; c < out; c++) mean_sum += os[c];
    const double out_mean = mean_sum / (double)out;
    if (out_mean <= 1e-30) {
        memset(os, 0, out * sizeof(float));
        if (mode != 0) apply = 1;
    } else {
        const float m = (float)out_mean;
        for (size_t c = 0; c < out; c++) os[c] /= m;
    }
    if (apply)
        for (size_t c = 0; c < out; c++) svh[c] = svh[c] * (fabsf(os[c]) < 1e-30f ? 0.1f : os[c]) + 1e-10f;
    for (size_t r = 0; r < in; r++)
        for (size_t c = 0; c < out; c++) inner[r * out + c] /= svh[c];
    for (size_t c = 0; c < out; c++)
        if (fabsf(os[c]) < 1e-30f) svh[c] = 0;
    for (size_t r = 0; r < in; r++)
        for (size_t b = 0; b < out; b += OXQ_HAD) oxq_fwht_f32(inner + r * out + b, 1);
    for (size_t r = 0; r < in; r++) {
        float total = 0;
        for (size_t c0 = 0; c0 < out; c0 += 32) {
            float block = 0;
            for (size_t c = c0; c < c0 + 32 && c < out; c++) block += inner[r * out + c] * inner[r * out + c];
            total += block;
        }
        float in_scale = sqrtf(total / (float)out);
        if (fabsf(in_scale) < 1e-30f) in_scale = 0.1f;
        suh[r] = sign_in[r] * in_scale / -OXQ_CODEBOOK_SCALE + 1e-10f;
    }
    for (size_t r = 0; r < in; r++)
        for (size_t c = 0; c < out; c++) inner[r * out + c] /= suh[r];
    for (size_t b = 0; b < in; b += OXQ_HAD)
        for (size_t c = 0; c < out; c++) oxq_fwht_f32(inner + b * out + c, out);
    free(os);
    return 0;
}

/* rotatedHessian (quantize.zig:192-207): H_L diag(suh) H diag(suh) H_L in f64, rounded to f32. */
int ox_quant_rotated_hessian(const float *h, const float *suh, size_t n, float *out) {
    if (n == 0 || n % OXQ_HAD) return -1;
    double *m = malloc(n * n * sizeof(double));
    for (size_t i = 0; i < n; i++)
        for (size_t j = 0; j < n; j++) m[i * n + j] = (double)h[i * n + j] * (double)suh[i] * (double)suh[j];
    for (size_t b = 0; b < n; b += OXQ_HAD)
        for (size_t c = 0; c < n; c++) oxq_fwht_f64(m + b * n + c, n);
    for (size_t r = 0; r < n; r++)
        for (size_t b = 0; b < n; b += OXQ_HAD) oxq_fwht_f64(m + r * n + b, 1);
    for (size_t i = 0; i < n * n; i++) out[i] = (float)m[i];
    free(m);
    return 0;
}

/* dotRows (quantize.zig:212-223): four f64 lanes over whole quads, reduced lane 0..3 in order, then the tail. */
static double oxq_dot(const double *a, const double *b, size_t len) {
    double acc[4] = {0, 0, 0, 0};
    size_t m = 0;
    for (; m + 4 <= len; m += 4)
        for (int l = 0; l < 4; l++) acc[l] += a[m + l] * b[m + l];
    double sum = ((acc[0] + acc[1]) + acc[2]) + acc[3];
    for (; m < len; m++) sum += a[m] * b[m];
    return sum;
}

/* choleskyLower (quantize.zig:225-247): blocked by 64, each block's contribution subtracted in block order. Returns
 * 0 or the 1-based index of the first pivot that is not positive. */
size_t ox_cholesky_lower(double *a, size_t n) {
    for (size_t k = 0; k < n; k += 64) {
        const size_t kb = n - k < 64 ? n - k : 64;
        for (size_t j = 0; j < kb; j++) {
            const size_t jj = k + j;
            const double d = a[jj * n + jj] - oxq_dot(a + jj * n + k, a + jj * n + k, j);
            if (!(d > 0)) return jj + 1;
            const double root = sqrt(d);
            a[jj * n + jj] = root;
            for (size_t i = j + 1; i < kb; i++) {
                const size_t ii = k + i;
                a[ii * n + jj] = (a[ii * n + jj] - oxq_dot(a + ii * n + k, a + jj * n + k, j)) / root;
            }
        }
        for (size_t i = k + kb; i < n; i++)
            for (size_t j = 0; j < kb; j++) {
                const size_t jj = k + j;
                a[i * n + jj] = (a[i * n + jj] - oxq_dot(a + i * n + k, a + jj * n + k, j)) / a[jj * n + jj];
            }
        for (size_t i = k + kb; i < n; i++)
            for (size_t j = k + kb; j <= i; j++) a[i * n + j] -= oxq_dot(a + i * n + k, a + j * n + k, kb);
    }
    return 0;
}

/* invertLowerBlock (quantize.zig:289-303) on a 16x16 block. */
static int oxq_invert_lower16(double *blk) {
    double inv[256] = {0};
    for (int c = 0; c < 16; c++) {
        const double d = blk[c * 16 + c];
        if (d == 0 || !isfinite(d)) return 0;
        inv[c * 16 + c] = 1.0 / d;
        for (int r = c + 1; r < 16; r++) {
            double sum = 0;
            for (int m = c; m < r; m++) sum += blk[r * 16 + m] * inv[m * 16 + c];
            inv[r * 16 + c] = -sum / blk[r * 16 + r];
        }
    }
    memcpy(blk, inv, sizeof(inv));
    return 1;
}

/* ldlFactor (quantize.zig:305-378): dampDiagonal, Cholesky in f64 (bumping the diagonal on a failed pivot, up to
 * 10 times), then each 16-column block of the f32 factor times its diagonal block's inverse, diagonal blocks
 * zeroed.  `h` [n][n] is taken as is (not modified).  Returns 0, -1 geometry, -2 not positive definite. */
int ox_quant_ldl_factor(const float *h_in, size_t n, float *l) {
    if (n == 0 || n % 16) return -1;
    float *h = malloc(n * n * sizeof(float));
    memcpy(h, h_in, n * n * sizeof(float));
    double diag_sum = 0;
    for (size_t i = 0; i < n; i++) {
        if (h[i * n + i] == 0) h[i * n + i] = 1;
        diag_sum += h[i * n + i];
    }
    const double diag_mean = diag_sum / (double)n;
    if (diag_mean > 0) {
        const float damp = (float)((double)OXQ_SIGMA_REG * diag_mean);
        for (size_t i = 0; i < n; i++) h[i * n + i] += damp;
    }
    double damped_sum = 0;
    for (size_t i = 0; i < n; i++) damped_sum += h[i * n + i];
    const double damped_mean = damped_sum / (double)n;
    double *c64 = malloc(n * n * sizeof(double));
    int rc = 0;
    for (int retries = 0;; retries++) {
        for (size_t i = 0; i < n * n; i++) c64[i] = h[i];
        if (ox_cholesky_lower(c64, n) == 0) break;
        if (retries + 1 > 10 || damped_mean <= 0) { rc = -2; break; }
        const float bump = (float)(2.0 * (double)OXQ_SIGMA_REG * damped_mean);
        for (size_t i = 0; i < n; i++) h[i * n + i] += bump;
    }
    if (rc == 0) {
        float *chol = malloc(n * n * sizeof(float));
        for (size_t i = 0; i < n; i++)
            for (size_t j = 0; j < n; j++) chol[i * n + j] = j <= i ? (float)c64[i * n + j] : 0.0f;
        memcpy(l, chol, n * n * sizeof(float));
        double blk[256];
        float inv[256];
        for (size_t c0 = 0; c0 < n && rc == 0; c0 += 16) {
            for (int i = 0; i < 16; i++)
                for (int j = 0; j < 16; j++) blk[i * 16 + j] = j <= i ? chol[(c0 + i) * n + c0 + j] : 0.0;
            if (!oxq_invert_lower16(blk)) { rc = -2; break; }
            for (int i = 0; i < 16; i++)
                for (int j = 0; j < 16; j++) inv[i * 16 + j] = j <= i ? (float)blk[i * 16 + j] : 0.0f;
            for (size_t r = c0 + 16; r < n; r++) {
                float row[16];
                for (int x = 0; x < 16; x++) {
                    float acc = 0;
                    for (int m = 0; m < 16; m++) acc += chol[r * n + c0 + m] * inv[m * 16 + x];
                    row[x] = acc;
                }
                memcpy(l + r * n + c0, row, sizeof(row));
            }
            for (int i = 0; i < 16; i++) memset(l + (c0 + i) * n + c0, 0, 16 * sizeof(float));
        }
        free(chol);
    }
    free(c64);
    free(h);
    return rc;
}

/* globalScale (quantize.zig:400-483): golden section over the codebook's bracket, scoring the mean squared error of
 * a wrapped diagonal of up to 128 sample tiles searched at inner * g and read back at 1/g. */
int ox_quant_global_scale(const float *inner, size_t rows, size_t cols, uint32_t n, ox_decode dec, float *g_out) {
    if (rows == 0 || cols == 0 || rows % OXQ_HAD || cols % OXQ_HAD) return -1;
    const size_t tk = rows / 16, tn = cols / 16;
    const size_t pair_count = (tk > tn ? tk : tn) * 3;
    const size_t stride = pair_count / 128 > 1 ? pair_count / 128 : 1;
    float *tiles = malloc(128 * 256 * sizeof(float));
    size_t count = 0;
    for (size_t p = 0; p < pair_count && count < 128; p += stride) {
        const size_t i = p / 3, wv = p % 3;
        const size_t r0 = (i % tk) * 16, c0 = ((i + wv) % tn) * 16;
        for (int r = 0; r < 16; r++) memcpy(tiles + count * 256 + r * 16, inner + (r0 + r) * cols + c0, 16 * sizeof(float));
        count++;
    }
    const double resphi64 = 2.0 - (1.0 + sqrt(5.0)) / 2.0;
    const float resphi = (float)resphi64;
    const float lo = dec.codebook == OX_CB_MUL1 ? 0.4f : 0.5f, hi = dec.codebook == OX_CB_MUL1 ? 1.2f : 1.5f;
    uint16_t packed[128];
    float scaled[256], recon[256];
    int rc = 0;
#define OXQ_SCORE(G, OUT)                                                                          \
    do {                                                                                           \
        double sse_ = 0;                                                                           \
        for (size_t t_ = 0; t_ < count; t_++) {                                                    \
            double dummy_;                                                                         \
            for (int v_ = 0; v_ < 256; v_++) scaled[v_] = tiles[t_ * 256 + v_] * (G);             \
            rc = ox_encode_tile(scaled, n, dec, packed, recon, &dummy_);                           \
            if (rc) break;                                                                         \
            for (int v_ = 0; v_ < 256; v_++) {                                                     \
                const float d_ = recon[v_] / (G) - tiles[t_ * 256 + v_];                           \
                sse_ += (double)(d_ * d_);                                                         \
            }                                                                                      \
        }                                                                                          \
        (OUT) = sse_ / (double)(count * 256);                                                      \
    } while (0)
    float a = lo, b = hi;
    float x1 = a + resphi * (b - a);
    float x2 = b - resphi * (b - a);
    double f1 = 0, f2 = 0;
    OXQ_SCORE(x1, f1);
    if (!rc) OXQ_SCORE(x2, f2);
    double width = (double)hi - (double)lo;
    size_t steps = 0;
    while (width > 0.03 && steps < 8) {
        width *= 1.0 - resphi64;
        steps++;
    }
    for (size_t s = 0; s < steps && !rc; s++) {
        const int left = f1 < f2;
        const float a_n = left ? a : x1, b_n = left ? x2 : b;
        const float probe = left ? a_n + resphi * (b_n - a_n) : b_n - resphi * (b_n - a_n);
        double fp;
        OXQ_SCORE(probe, fp);
        a = a_n;
        b = b_n;
        if (left) { x2 = x1; f2 = f1; x1 = probe; f1 = fp; }
        else { x1 = x2; f1 = f2; x2 = probe; f2 = fp; }
    }
#undef OXQ_SCORE
    free(tiles);
    if (rc) return rc;
    *g_out = (a + b) / 2.0f;
    return 0;
}

/* ldlq (quantize.zig:485-540): 16-row groups from the bottom, each searched after the error of the rows below it
 * is fed back through l; 128-row chunks carry the error of finished chunks to every row above in `prod`. */
int ox_quant_ldlq(const float *inner, const float *l, size_t rows, size_t cols, uint32_t n, ox_decode dec,
                  uint16_t *packed, float *recon_out) {
    const size_t out_tiles = cols / 16;
    float *rec = calloc(rows * cols, sizeof(float));
    float *prod = calloc(rows * cols, sizeof(float));
    float *comp = malloc(16 * cols * sizeof(float));
    float *err = malloc(cols * sizeof(float));
    int rc = 0;
    for (size_t j = rows; j > 0 && !rc;) {
        const size_t i = j > 128 ? j - 128 : 0;
        const size_t chunk = j - i;
        for (size_t bj = chunk; bj > 0 && !rc; bj -= 16) {
            const size_t bi = bj > 16 ? bj - 16 : 0;
            const size_t height = bj - bi;
            memcpy(comp, prod + (i + bi) * cols, height * cols * sizeof(float));
            for (size_t m = bj; m < chunk; m++) {
                for (size_t c = 0; c < cols; c++) err[c] = inner[(i + m) * cols + c] - rec[(i + m) * cols + c];
                for (size_t r = 0; r < height; r++) {
                    const float lv = l[(i + m) * rows + i + bi + r];
                    for (size_t c = 0; c < cols; c++) comp[r * cols + c] += lv * err[c];
                }
            }
            for (size_t r = 0; r < height; r++)
                for (size_t c = 0; c < cols; c++) comp[r * cols + c] = inner[(i + bi + r) * cols + c] + comp[r * cols + c];
            const size_t tk = (i + bi) / 16;
            for (size_t tn = 0; tn < out_tiles && !rc; tn++) {
                float tile[256], tile_rec[256];
                double sse;
                for (int r = 0; r < 16; r++) memcpy(tile + r * 16, comp + r * cols + tn * 16, 16 * sizeof(float));
                rc = ox_encode_tile(tile, n, dec, packed + (tk * out_tiles + tn) * n, tile_rec, &sse);
                for (int r = 0; r < 16; r++)
                    memcpy(rec + (i + bi + r) * cols + tn * 16, tile_rec + r * 16, 16 * sizeof(float));
            }
        }
        if (i > 0 && !rc)
            for (size_t m = 0; m < chunk; m++) {
                for (size_t c = 0; c < cols; c++) err[c] = inner[(i + m) * cols + c] - rec[(i + m) * cols + c];
                for (size_t r = 0; r < i; r++) {
                    const float lv = l[(i + m) * rows + r];
                    for (size_t c = 0; c < cols; c++) prod[r * cols + c] += lv * err[c];
                }
            }
        j = i;
    }
    if (recon_out && !rc) memcpy(recon_out, rec, rows * cols * sizeof(float));
    free(rec); free(prod); free(comp); free(err);
    return rc;
}

/* signs (quantize.zig:567-590): splitmix64 seeded by mixing `seed` with each byte of `name`; -1 where bit 0 is set. */
static uint64_t oxq_splitmix(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void ox_quant_signs(uint64_t seed, const char *name, size_t len, float *out) {
    uint64_t state = seed;
    for (const unsigned char *p = (const unsigned char *)name; *p; p++) state = oxq_splitmix(state ^ *p);
    state = oxq_splitmix(state);
    for (size_t i = 0; i < len; i++) {
        state = oxq_splitmix(state);
        out[i] = (state & 1) == 0 ? 1.0f : -1.0f;
    }
}

/* quantizeTensor (quantize.zig:600-626): public weight [in][out] and input Hessian [in][in] -> packed
 * [in/16][out/16][n], suh [in] and svh [out] as f16 bits, and the global scale g. */
int ox_quantize_tensor(const float *w, const float *h, size_t in, size_t out, const float *sign_in,
                       const float *sign_out, uint32_t n, ox_decode dec, int mode, uint16_t *packed, uint16_t *suh16,
                       uint16_t *svh16, float *g_out) {
    if (in == 0 || out == 0) return -10;
    if (in % OXQ_HAD || out % OXQ_HAD) return -11;
    float *hdiag = malloc(in * sizeof(float));
    for (size_t i = 0; i < in; i++) hdiag[i] = h[i * in + i];
    float *inner = malloc(in * out * sizeof(float)), *suh = malloc(in * sizeof(float)), *svh = malloc(out * sizeof(float));
    float *rot = malloc(in * in * sizeof(float)), *l = malloc(in * in * sizeof(float));
    int rc = ox_quant_regularize(w, in, out, sign_in, sign_out, mode, hdiag, inner, suh, svh);
    if (!rc) rc = ox_quant_rotated_hessian(h, suh, in, rot);
    if (!rc) rc = ox_quant_ldl_factor(rot, in, l);
    float g = 1.0f;
    if (!rc) rc = ox_quant_global_scale(inner, in, out, n, dec, &g);
    if (!rc) {
        for (size_t i = 0; i < in * out; i++) inner[i] *= g;
        rc = ox_quant_ldlq(inner, l, in, out, n, dec, packed, NULL);
    }
    if (!rc) {
        for (size_t i = 0; i < in; i++) suh16[i] = ox_f32_to_f16(suh[i] / g);
        for (size_t i = 0; i < out; i++) svh16[i] = ox_f32_to_f16(svh[i]);
        *g_out = g;
    }
    free(hdiag); free(inner); free(suh); free(svh); free(rot); free(l);
    return rc;
}
