// The C ABI (include/sushi_exl3_hip.h): validation, arm choice, workspace carving and launches.
//
// Every refusal happens before any launch (as the reference's `Exl3*` errors do, src/exl3/root.zig:104-133), and the
// library never allocates device memory: scratch comes from the caller's workspace.
#include <algorithm>
#include <atomic>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "sushi_exl3_hip.h"
#include "exl3_kernels.h"
#include "exl3_tables.h"

using namespace exl3;

namespace {

thread_local std::string g_err;

int32_t fail(int32_t code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int32_t fail(int32_t code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int32_t ok() {
    g_err.clear();
    return EXL3_OK;
}

int32_t launched(hipError_t e, const char *what) {
    if (e != hipSuccess) return fail(EXL3_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
    return ok();
}

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Every workspace starts with a fixed region that stays zero between calls.  Only the fused-finish GEMV touches it,
// either as arrival counters (its first MiB) or as the fold's 64-bit accumulators (the first 4 MiB) and their f64
// overflow words (the next 4 MiB), and every such launch leaves what it touched at zero again, so the region stays
// valid across calls of any arm (exl3_workspace_init zeroes it once after allocation).  Scratch of every arm begins
// after it.  Each counter owns a 128-byte line (COUNTER_STRIDE words): the splits of different output groups then
// never contend for one line in the L2's atomic unit.
constexpr size_t kFoldWords = FOLD_WORDS;
constexpr size_t kZeroBytes = 2 * kFoldWords * sizeof(unsigned long long);
constexpr size_t kCounterSlots = (size_t(1) << 20) / (sizeof(uint32_t) * COUNTER_STRIDE);
constexpr int kMaxDevices = 64;  // devices with per-device state (the no-alloc scratch, the CU count)

bool rate_admitted(int n) { return n >= 16 && n <= 128 && n % 2 == 0; }  // kFromPackedDim, expert_exl3.zig:241-245

// The rates the GEMV and the GEMM read with a lane reader.
bool lane_rate(int n) { return n == 16 || n == 24 || n == 32 || n == 40 || n == 48 || n == 64; }

// Arm overrides (exl3_set_override): one word per knob, INT32_MIN = unset.  Read with a relaxed load at each call,
// so an unset knob costs one load and nothing in the environment changes an arm.
std::atomic<int32_t> g_override[EXL3_KNOB_COUNT] = {};
struct OverrideInit {
    OverrideInit() {
        for (auto &o : g_override) o.store(INT32_MIN, std::memory_order_relaxed);
    }
} g_override_init;

int knob(exl3_knob k, int dflt) {
    const int32_t v = g_override[k].load(std::memory_order_relaxed);
    return v == INT32_MIN ? dflt : v;
}

// The decode family and constants for (dec, n); status on refusal.
int32_t resolve_decode(const exl3_decode_t &dec, int n, int *fam, DecodeK *k, bool per_rate_table = false) {
    if (dec.window_bits < 8 || dec.window_bits > 16)
        return fail(EXL3_ERR_WINDOW, "window %d is not a codeword width in 8..16", dec.window_bits);
    k->wmask = dec.window_bits >= 16 ? 0xFFFFu : ((1u << dec.window_bits) - 1u);
    k->mult = k->mask0 = k->mask1 = k->rot = 0;
    switch (dec.codebook) {
    case EXL3_CB_MCG: *fam = FAM_MCG; return ok();
    case EXL3_CB_MUL1: *fam = FAM_MUL1; return ok();
    case EXL3_CB_3INST: *fam = FAM_3INST; return ok();
    case EXL3_CB_SPEC1:
    case EXL3_CB_STD1: {
        // Decode.requireTable (expert_exl3.zig:162-164): a tabled codebook without its table has no pair.
        if (dec.table < 0 || dec.table > 3)
            return fail(EXL3_ERR_TABLE_UNKNOWN, "codebook %d needs a codebook table", dec.codebook);
        if (kTables[dec.table].codebook != dec.codebook)
            return fail(EXL3_ERR_TABLE_UNKNOWN, "table %d does not belong to codebook %d", dec.table, dec.codebook);
        *fam = FAM_HASH;
        if (per_rate_table) return ok();
        if (!table_row(dec.table, n, k->mult, k->mask0, k->mask1, k->rot))
            return fail(EXL3_ERR_RATE_MISSING, "table %d has no row for n=%d", dec.table, n);
        return ok();
    }
    case EXL3_CB_PAIR1: {
        if (dec.table >= 0 && dec.table != TABLE_PAIR1_W16_V1)
            return fail(EXL3_ERR_TABLE_UNKNOWN, "PAIR1 decodes only with table pair1-w16-v1");
        *fam = FAM_PAIR;
        if (per_rate_table) return ok();
        if (!table_row(TABLE_PAIR1_W16_V1, n, k->mult, k->mask0, k->mask1, k->rot))
            return fail(EXL3_ERR_RATE_MISSING, "PAIR1 has no pair row for n=%d (24..64 even)", n);
        return ok();
    }
    default: return fail(EXL3_ERR_TABLE_UNKNOWN, "unknown codebook %d", dec.codebook);
    }
}

bool dtype_ok(int dt) { return dt == EXL3_DT_F16 || dt == EXL3_DT_BF16 || dt == EXL3_DT_F32; }

float out_scale_of(int fam) { return (fam == FAM_HASH || fam == FAM_PAIR) ? 4096.0f : 1.0f; }

// Rows the decode GEMV serves (each weight decoded once, dotted against every row).  The reference's
// PROJECT_ROWS_MAX is 8 (project_rows.zig:456-459) with a 16-row mode beside it; here up to 16 rows stay on the
// GEMV, which beats a 128-row MFMA tile by far at such row counts.
constexpr int kRowsMax = 16;

struct GemvPlan {
    int splits;
    size_t counters_bytes, partial_bytes;
};

GemvPlan plan_gemv(int groups, int rows, int in, int out) {
    GemvPlan p;
    p.splits = knob(EXL3_KNOB_GEMV_SPLITS, 0);
    const int blocks = in / 128;
    // Up to four tile batches of TPW tiles per wave (eight from 8 rows): later batches' loads overlap the decode, and
    // fewer splits mean fewer fold arrivals.
    if (p.splits <= 0 || blocks % p.splits != 0 || in / p.splits > 2048)
        p.splits = gemv_default_splits(in, out, rows, groups, rows >= 8 ? 8 : 4);
    p.counters_bytes = kZeroBytes;
    p.partial_bytes = p.splits > 1 ? align_up((size_t)groups * p.splits * rows * out * sizeof(float)) : 0;
    return p;
}

// Prepared-input rows of the GEMM arm: whole 16-row tiles (the fragment-order layout pads the last tile).
size_t gemm_xp_bytes(int groups, int rows, int in) { return align_up((size_t)groups * ((rows + 15) / 16 * 16) * in * 2); }

// The dense GEMM body at a lane-reader rate (EXL3_KNOB_GEMM_ARM pins one): the ping-pong 512-row tile past 512 rows
// while its tiles still give most CUs a workgroup; from 257 to 512 rows, where they would not, the same tile with k
// in halves when that fills the chip; otherwise the decode-wave 256-row tile.  Measured at C3's 4096 x 14336:
// 512 rows 94.3 -> 91.4 us, 384 rows 91.1 -> 89.2 us on the split tile; 256 rows stay on the decode-wave tile
// (81.5 against 88.5 us).
// split_ok = false (a caller whose scratch cannot hold the halves' partials) turns arm 7 into the decode-wave tile.
int gemm_arm_for(int groups, int rows, int out, bool split_ok = true) {
    const int pinned = knob(EXL3_KNOB_GEMM_ARM, 0);
    const int arm = pinned ? pinned : gemm_default_arm(groups, rows, out);
    return arm == 7 && !split_ok ? 4 : arm;
}

// Arm 7 (k in halves) holds both halves' partials after the prepared input, and one counter per tile in the zeroed
// region; n = 40 never takes it (its reader does not fit the 512-row tile's registers).
bool gemm_uses_kpart(int groups, int rows, int out, int n, bool split_ok = true) {
    const bool lane_reader = n == 16 || n == 24 || n == 32 || n == 48 || n == 64;
    return lane_reader && gemm_arm_for(groups, rows, out, split_ok) == 7 &&
           (size_t)groups * ((rows + 511) / 512) * (out / 128) <= kCounterSlots;
}

// The k-halves tile's wait (100 MHz ticks): the first half of a tile to finish its main loop waits for the second and
// then each finishes half the rows; past the wait it hands the whole tile over (the second then finishes every row,
// as the tile did before the halves shared the finish).  Waiting pays only where every tile's second half is running
// beside it: 20 us when all the launch's workgroups fit on the device's CUs at one each, else no wait.
uint32_t gemm_split_wait(long workgroups) {
    const int pinned = knob(EXL3_KNOB_GEMM_SPLIT_WAIT, -1);
    if (pinned >= 0) return (uint32_t)pinned;
    static std::atomic<int> cus[kMaxDevices] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return workgroups <= n ? 2000u : 0u;
}

size_t gemm_bytes(int groups, int rows, int in, int out, int n, bool split_ok = true) {
    size_t b = kZeroBytes + gemm_xp_bytes(groups, rows, in);
    const bool lane_reader = n == 16 || n == 24 || n == 32 || n == 40 || n == 48 || n == 64;
    if (!lane_reader) b += align_up((size_t)groups * out * in * 2);  // the transposed f16 copy of other rates
    if (gemm_uses_kpart(groups, rows, out, n, split_ok)) b += align_up(gemm_kpart_bytes(groups, rows, out));
    return b;
}

// The decode GEMV's row groups for one bank: the rows run as ceil(rows / r) groups of r rows over the same weights
// (the last group holds the rest), each group decoding them -- more workgroups, each with an r-row input prologue and
// fold.  That pays where the weights are few beside those per-row costs: from 5 rows on a bank of at most 2048 x 2048
// (4 M weights), in two groups (r = ceil(rows / 2), at most 8).  Measured (MCG, us per call, whole against two
// groups): 2048 x 2048 n = 32, 5 / 8 / 9 / 12 / 16 rows 6.19 / 6.67 / 8.30 / 8.57 / 9.21 against 6.03 / 6.40 / 6.57
// (6.49 with r = 8) / 6.90 / 7.37, 3 and 4 rows 5.56 against 5.63 / 5.67; 4096 x 4096 n = 64 and 4096 x 14336
// n = 48 slower in groups at every row count from 3 to 16 (16 rows 13.84 against 14.31, 34.85 against 37.45).
// EXL3_KNOB_GEMV_ROWS_PER_GROUP pins r (a value of at least the rows keeps them whole).  Returns rows_total for
// GemvArgs (0: the rows stay one group).
int gemv_row_groups(int &groups, int &rows, int in, int out) {
    const int pinned = knob(EXL3_KNOB_GEMV_ROWS_PER_GROUP, 0);
    const bool small_bank = (long)in * out <= 2048L * 2048L;
    const int r = pinned > 0 ? pinned : (small_bank && rows >= 5) ? std::min(8, (rows + 1) / 2) : rows;
    if (groups != 1 || r >= rows) return 0;
    const int total = rows;
    groups = (rows + r - 1) / r;
    rows = r;
    return total;
}

size_t linear_ws(int groups, int rows, int in, int out, int n, bool split_ok = true) {
    if (rows <= 0) return 0;
    if (rows <= kRowsMax) {
        const GemvPlan p = plan_gemv(groups, rows, in, out);
        int g = groups, r = rows;  // the row groups' plan too (a row-major grouped output keeps the rows whole)
        gemv_row_groups(g, r, in, out);
        const GemvPlan q = plan_gemv(g, r, in, out);
        return std::max(p.counters_bytes + p.partial_bytes, q.counters_bytes + q.partial_bytes);
    }
    return gemm_bytes(groups, rows, in, out, n, split_ok);
}

// Every refusal of a linear call (all before any HIP call); fam / k receive the decode family and constants.
int32_t linear_checks(const void *x, int32_t x_dtype, int32_t groups, int32_t rows, int32_t in, int32_t out,
                      const uint16_t *trellis, int32_t n, const uint16_t *suh, const uint16_t *svh,
                      const exl3_decode_t &dec, const void *y, int32_t y_dtype, int *fam, DecodeK *k) {
    if (groups <= 0 || rows < 0 || in <= 0 || out <= 0 || in % 128 || out % 128)
        return fail(EXL3_ERR_BAD_SHAPE, "linear: groups=%d rows=%d in=%d out=%d (in and out must be multiples of 128)",
                    groups, rows, in, out);
    if (!rate_admitted(n)) return fail(EXL3_ERR_BAD_SHAPE, "linear: n=%d is not an admitted rate", n);
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype)) return fail(EXL3_ERR_BAD_DTYPE, "linear: unsupported dtype");
    int32_t rc = resolve_decode(dec, n, fam, k);
    if (rc) return rc;
    if (rows == 0) return ok();
    if (!x || !trellis || !suh || !svh || !y) return fail(EXL3_ERR_BAD_SHAPE, "linear: null operand");
    if (reinterpret_cast<uintptr_t>(x) % 4) return fail(EXL3_ERR_BAD_SHAPE, "linear: x must be 4-byte aligned");
    return ok();
}

// y_rows_major (decode-GEMV row counts only): group g's row r lands in output row r * groups + g, so y is
// [rows][groups * out] (linearGroupedRows's layout, src/exl3/linear.zig:97-117) instead of [groups][rows][out].
int32_t linear_impl(const void *x, int32_t x_dtype, int32_t groups, int32_t rows, int32_t in, int32_t out,
                    const uint16_t *trellis, int32_t n, const uint16_t *suh, const uint16_t *svh, exl3_decode_t dec,
                    void *y, int32_t y_dtype, void *ws, size_t ws_bytes, hipStream_t stream, bool split_ok = true,
                    bool y_rows_major = false) {
    int fam;
    DecodeK k;
    int32_t rc = linear_checks(x, x_dtype, groups, rows, in, out, trellis, n, suh, svh, dec, y, y_dtype, &fam, &k);
    if (rc || rows == 0) return rc;
    const size_t need = linear_ws(groups, rows, in, out, n, split_ok);
    if (ws_bytes < need || (need && (!ws || (reinterpret_cast<uintptr_t>(ws) % kAlign))))
        return fail(EXL3_ERR_WORKSPACE, "linear: workspace of %zu bytes (256-aligned) needed, got %zu", need, ws_bytes);
    char *w = static_cast<char *>(ws);
    if (rows <= kRowsMax) {
        const int banks = groups;
        const int rows_total = y_rows_major ? 0 : gemv_row_groups(groups, rows, in, out);
        GemvPlan p = plan_gemv(groups, rows, in, out);
        GemvArgs a{};
        a.x = x;
        a.x_dtype = x_dtype;
        a.rows = rows;
        a.in = in;
        a.out = out;
        a.x_div = 1;
        a.trellis[0] = trellis;
        a.suh[0] = suh;
        a.svh[0] = svh;
        a.n = n;
        a.bank_of = nullptr;
        a.bank_limit = banks;  // group g takes bank min(g, banks - 1): its own, or the one bank of row groups
        a.meta = nullptr;
        a.table = dec.table;
        a.k = k;
        a.out_scale = out_scale_of(fam);
        a.counters = reinterpret_cast<uint32_t *>(w);
        a.partial[0] = p.partial_bytes ? reinterpret_cast<float *>(w + p.counters_bytes) : nullptr;
        a.y = y;
        a.y_dtype = y_dtype;
        a.y_rows_major = y_rows_major ? 1 : 0;
        a.rows_total = rows_total;
        a.splits = p.splits;
        a.groups = groups;
        a.nproj = 1;
        a.fused_finish = (knob(EXL3_KNOB_GEMV_SEPARATE_FINISH, 0) == 0 &&
                          (size_t)groups * (out / 128) <= kCounterSlots) ? 1 : 0;
        a.partial_only = 0;
        // The fold (exact fixed-point accumulation, one atomic round trip per split) serves the fused finish of a
        // 16-bit output whenever its words fit the zeroed region and the splits fit its count field; the counters +
        // planes arm otherwise.  An f32 output never folds: the fold's 2^-24 fixed point would quantise it.
        a.fold = (a.fused_finish && p.splits > 1 && p.splits <= FOLD_MAX_SPLITS && y_dtype != EXL3_DT_F32 &&
                  (size_t)groups * rows * out <= kFoldWords && knob(EXL3_KNOB_GEMV_FOLD, 1) != 0)
                     ? reinterpret_cast<unsigned long long *>(w)
                     : nullptr;
        a.fold_arrivals = p.splits;
        return launched(run_gemv(fam, PRO_X, a, stream), "exl3_linear (gemv)");
    }
    if (y_rows_major) return fail(EXL3_ERR_BAD_SHAPE, "linear: the row-major grouped output serves up to %d rows", kRowsMax);
    GemmArgs g{};
    g.x = x;
    g.x_dtype = x_dtype;
    g.rows = rows;
    g.in = in;
    g.out = out;
    g.trellis = trellis;
    g.n = n;
    g.suh = suh;
    g.svh = svh;
    g.k = k;
    g.xp = reinterpret_cast<uint16_t *>(w + kZeroBytes);
    g.wt = reinterpret_cast<uint16_t *>(w + kZeroBytes + gemm_xp_bytes(groups, rows, in));
    g.y = y;
    g.y_dtype = y_dtype;
    g.groups = groups;
    g.arm = gemm_arm_for(groups, rows, out, split_ok);
    if (gemm_uses_kpart(groups, rows, out, n, split_ok)) {
        g.kpart = reinterpret_cast<float *>(w + kZeroBytes + gemm_xp_bytes(groups, rows, in));
        g.kctr = reinterpret_cast<uint32_t *>(w);
        g.kwait = gemm_split_wait(2L * groups * ((rows + 511) / 512) * (out / 128));
    }
    return launched(run_gemm(fam, g, stream), "exl3_linear (gemm)");
}

// Rows above which the routed layer takes the sorted arm (slots grouped into expert windows, each expert's tiles
// decoded once per window).  The reference's decode chain serves up to DECODE_ROWS_MAX = 16 rows and sends wider
// batches to moePrefill (src/exl3/root.zig:45-53); here the windows win from 9 rows on (measured at C4's shape:
// 12 rows 90.5 -> 88.2 us, 16 rows 115 -> 106 us; 4 and 6 rows stay faster per slot, 8 rows equal).
constexpr int kMoeDecodeRowsMax = 8;
// EXL3_KNOB_MOE_DECODE_ROWS_MAX moves that bound (tuning and tests; read by the workspace queries too).
int moe_decode_rows_max() { return knob(EXL3_KNOB_MOE_DECODE_ROWS_MAX, kMoeDecodeRowsMax); }

// Workgroups the per-slot MoE launches aim for: 1.5 per CU.
constexpr int kMoeSlotTargetWgs = 384;

struct MoePlan {
    bool windowed;
    int s1, s2;
    size_t gu_bytes, down_bytes, table_bytes;
    size_t total() const { return kZeroBytes + 2 * gu_bytes + down_bytes + table_bytes; }
};

// `extra`: token rows of a fused shared expert, whose planes follow the slots' (and whose groups of SH_ROWS rows join
// the grid).
MoePlan plan_moe(int nslots, int hidden, int inter, bool windowed, int extra = 0) {
    MoePlan p;
    p.windowed = windowed;
    // Window count lies between ceil(nslots / MOE_WINDOW_ROWS) and nslots; splits are planned for the fewest windows
    // (the most splits), so the planes fit whatever the routing turns out to be.
    const int groups = windowed ? (nslots + MOE_WINDOW_ROWS - 1) / MOE_WINDOW_ROWS + (extra + SH_ROWS - 1) / SH_ROWS
                                : nslots + extra;
    const int rows = windowed ? MOE_WINDOW_ROWS : 1;
    // Per-slot arm: at least 1.5 workgroups per CU and at most four batches of TPW tiles per wave (measured at C4's
    // shape, b = 1 and 8: the best of every split pair tried).  Sorted arm: up to eight batches (each window's
    // workgroup carries four rows per tile) and one workgroup per CU (measured at C4 b = 24 and 32).
    if (windowed) {
        // The window count is planned at its fewest, so the CU-round fill of the split tie-break would be judged on
        // the wrong grid: the plain target (one workgroup per CU) instead (C4 b = 32: splits 1/2 -> 1/1, -10%).
        p.s1 = gemv_default_splits(hidden, inter, rows, 2 * groups, 8, GEMV_TARGET_WGS);
        p.s2 = gemv_default_splits(inter, hidden, rows, groups, 8, GEMV_TARGET_WGS);
    } else {
        p.s1 = gemv_default_splits(hidden, inter, rows, 2 * groups, 4, kMoeSlotTargetWgs);
        p.s2 = gemv_default_splits(inter, hidden, rows, groups, 4, kMoeSlotTargetWgs);
    }
    // EXL3_KNOB_MOE_SPLITS1 / _SPLITS2 pin the gate/up and down split counts (whole 128-blocks; tuning and tests)
    const int f1 = knob(EXL3_KNOB_MOE_SPLITS1, 0), f2 = knob(EXL3_KNOB_MOE_SPLITS2, 0);
    if (f1 > 0 && (hidden / 128) % f1 == 0) p.s1 = f1;
    if (f2 > 0 && (inter / 128) % f2 == 0) p.s2 = f2;
    p.gu_bytes = align_up((size_t)(nslots + extra) * p.s1 * inter * sizeof(float));
    p.down_bytes = align_up((size_t)(nslots + extra) * p.s2 * hidden * sizeof(float));
    p.table_bytes = windowed ? align_up(sizeof(uint32_t)) + 2 * align_up((size_t)nslots * sizeof(uint32_t)) +
                                   align_up((size_t)nslots * MOE_WINDOW_ROWS * sizeof(uint32_t))
                             : 0;
    return p;
}

// The routed GEMM arm (prefill widths): slots sorted by expert into windows of up to MOE_GEMM_WINDOW_ROWS rows, each
// window's rows prepared into MFMA fragment order and run through the decode-once GEMM (each weight decoded once per
// window instead of once per 4-row GEMV window), then the mid, the down GEMM and the reduce.  Taken when the layer
// averages at least kMoeGemmMinSlotsPerExpert slots per expert (E = 256 top-8, per layer: C4's 4 slots per expert
// 350 us against 392 on the GEMV windows, 2 slots 310 against 238; C5's ragged bank 1583 against 2024 and 1403
// against 1270), on a bank whose decode waves have a reader: a uniform bank at one lane-reader rate, a ragged bank of
// lane-reader rates, or a per-tile-rate bank.
constexpr int kMoeGemmMinSlotsPerExpert = 4;

struct MoeGemmPlan {
    int max_windows, max_tiles;
    size_t tables, xp_gu, xp_down, planes_gu, planes_down;
    size_t total() const { return kZeroBytes + tables + 2 * xp_gu + xp_down + 2 * planes_gu + planes_down; }
};

// Windows and tiles for at most `experts` experts hit (the size queries use kMoeGemmMaxExperts).
MoeGemmPlan plan_moe_gemm(int nslots, int hidden, int inter, int experts) {
    MoeGemmPlan p;
    const int W = MOE_GEMM_WINDOW_ROWS;
    p.max_windows = std::min(nslots, experts + (nslots + W - 1) / W);
    p.max_tiles = (nslots + 15) / 16 + std::min(nslots, experts);
    p.tables = align_up(2 * sizeof(uint32_t)) + align_up((size_t)nslots * 4) + 4 * align_up((size_t)p.max_windows * 4) +
               align_up((size_t)p.max_tiles * 16) + align_up((size_t)kMoeGemmMaxChunks * experts * 4) +
               align_up((size_t)nslots * 4);
    p.xp_gu = align_up((size_t)p.max_tiles * 16 * hidden * 2);
    p.xp_down = align_up((size_t)p.max_tiles * 16 * inter * 2);
    p.planes_gu = align_up((size_t)nslots * inter * sizeof(float));
    p.planes_down = align_up((size_t)nslots * hidden * sizeof(float));
    return p;
}

bool moe_gemm_wanted(int nslots, int experts, bool gemm_bank) {
    const int k = knob(EXL3_KNOB_MOE_GEMM, -1);
    if (k == 0 || !gemm_bank || experts > kMoeGemmMaxExperts) return false;
    return k > 0 || (long)nslots >= (long)kMoeGemmMinSlotsPerExpert * experts;
}

bool moe_windowed(int rows, int nslots, int experts) {
    return rows > moe_decode_rows_max() && nslots <= kMoeWindowMaxSlots && experts <= kMoeWindowMaxExperts;
}

// EXL3_KNOB_MOE_WINDOWS = 0 keeps every row count on the per-slot chain (for comparing the arms).
bool moe_windows_enabled() { return knob(EXL3_KNOB_MOE_WINDOWS, 1) != 0; }

constexpr int kReduceMaxTopk = kMoeReduceMaxTopk;  // REDUCE_MAX_TOPK, expert_exl3_kernels.zig:2562

int32_t moe_common_checks(int32_t x_dtype, int32_t y_dtype, int32_t rows, int32_t hidden, int32_t inter,
                          int32_t topk, int32_t clamp_limit, int32_t scores_dtype) {
    if (clamp_limit < 0 || clamp_limit > 128)
        return fail(EXL3_ERR_INVALID_CLAMP, "moe: clamp limit %d outside 1..128 (0 = none)", clamp_limit);
    if (topk < 1 || topk > kReduceMaxTopk)
        return fail(EXL3_ERR_TOPK_EXCEEDS_REDUCE, "moe: top-k %d exceeds the reduce bank (1..%d)", topk, kReduceMaxTopk);
    if (rows < 0 || hidden <= 0 || inter <= 0 || hidden % 128 || inter % 128)
        return fail(EXL3_ERR_BAD_SHAPE, "moe: rows=%d hidden=%d inter=%d (multiples of 128)", rows, hidden, inter);
    if ((long)rows * topk > (1L << 24)) return fail(EXL3_ERR_BAD_SHAPE, "moe: too many slots");
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype)) return fail(EXL3_ERR_BAD_DTYPE, "moe: unsupported dtype");
    if (!dtype_ok(scores_dtype)) return fail(EXL3_ERR_BAD_DTYPE, "moe: scores dtype %d (f32, bf16 or f16)", scores_dtype);
    return ok();
}

// A one-expert shared bank run inside the routed launches (exl3_moe_with_shared_bank): its rows are appended to the
// per-slot groups.
struct SharedBank {
    const uint16_t *tr[3], *su[3], *sv[3];
    int n;
};

// On the GEMM arm the shared bank's rows join as one more expert (any y dtype).  Otherwise they need the per-slot
// arm, a 16-bit output dtype (the combine word holds both rounded sums), the routed and shared folds (routed, shared
// and combine words: three per output), and, for a uniform bank, the routed rate.  gemm_bank: the routed bank and the
// shared bank's rate can take the GEMM arm.
bool moe_shared_fusable(int rows, int topk, int hidden, int inter, int y_dtype, int experts, bool gemm_bank,
                        bool verify) {
    const int nslots = rows * topk;
    if (!verify && moe_gemm_wanted(nslots, experts, gemm_bank)) return experts < kMoeGemmMaxExperts;
    if (y_dtype == EXL3_DT_F32) return false;
    const bool windowed = rows > moe_decode_rows_max();
    if (windowed && !(moe_windows_enabled() && moe_windowed(rows, nslots, experts))) return false;
    const MoePlan p = plan_moe(nslots, hidden, inter, windowed, rows);
    return topk * p.s2 <= FOLD_MAX_SPLITS && (size_t)3 * rows * hidden <= kFoldWords;
}

// A per-tile-rate bank's segment tables, per projection (gate, up, down).
struct TiledTables {
    const uint32_t *off[3];
    const uint8_t *k1[3];
};

// One routed layer's launches.  n[3] are the projections' uniform rates (all 0 with a ragged `meta` or a per-tile-rate
// bank's tables `tt`); k is the decode of the gate's rate (per-rate constants of the other projections are resolved
// here).  shared / shared_gate: an already computed shared expert [rows][hidden] in y's dtype, added as it is or as
// sigmoid(gate) * shared.  verify: speculative-verify rows, which stay on the decode chain at every width (the
// reference's `rows <= DECODE_ROWS_MAX or verify_rows`, src/exl3/root.zig:169).
int32_t moe_launch(int fam, const DecodeK &k, const exl3_decode_t &dec, int table, const void *x, int32_t x_dtype,
                   int32_t rows, int32_t hidden, int32_t inter, int32_t experts, const uint16_t *const tr[3],
                   const uint16_t *const su[3], const uint16_t *const sv[3], const int n[3], const uint32_t *meta,
                   int meta_lane_only, const uint32_t *inds, const void *scores, int32_t scores_dtype, int32_t topk,
                   bool verify, int32_t clamp_limit, const void *shared, const void *shared_gate, void *y,
                   int32_t y_dtype, void *ws, size_t ws_bytes, hipStream_t stream, const SharedBank *sb = nullptr,
                   const TiledTables *tt = nullptr) {
    if (reinterpret_cast<uintptr_t>(x) % 4) return fail(EXL3_ERR_BAD_SHAPE, "moe: x must be 4-byte aligned");
    const int nslots = rows * topk;
    // The GEMM arm's banks: uniform at one lane-reader rate, ragged with lane-reader rates only (meta_lane_only), or
    // per-tile rates; a fused shared bank at a lane-reader rate (the routed rate with a uniform bank).
    const bool uniform_lane = !meta && !tt && n[0] == n[1] && n[1] == n[2] && lane_rate(n[0]);
    const bool gemm_bank = uniform_lane || (meta && meta_lane_only) || tt;
    const bool gemm_shared = !sb || (!shared && experts < kMoeGemmMaxExperts && lane_rate(sb->n) &&
                                     (!uniform_lane || sb->n == n[0]));
    if (!verify && gemm_bank && gemm_shared && moe_gemm_wanted(nslots, experts, true)) {
        // a shared bank's rows are slots nslots .. nslots + rows - 1 of one more expert (index `experts`)
        const int sh_rows = sb ? rows : 0;
        const MoeGemmPlan gp = plan_moe_gemm(nslots + sh_rows, hidden, inter, experts + (sb ? 1 : 0));
        if (ws_bytes < gp.total() || !ws || (reinterpret_cast<uintptr_t>(ws) % kAlign))
            return fail(EXL3_ERR_WORKSPACE, "moe: workspace of %zu bytes (256-aligned) needed, got %zu", gp.total(),
                        ws_bytes);
        char *w = static_cast<char *>(ws) + kZeroBytes;
        MoeGemmArgs g{};
        auto take = [&](size_t bytes) {
            char *p = w;
            w += bytes;
            return p;
        };
        uint32_t *counts = reinterpret_cast<uint32_t *>(take(align_up(2 * sizeof(uint32_t))));
        g.win.win_count = counts;
        g.win.tile_count = counts + 1;
        g.win.sorted = reinterpret_cast<uint32_t *>(take(align_up((size_t)(nslots + sh_rows) * 4)));
        g.win.win_expert = reinterpret_cast<uint32_t *>(take(align_up((size_t)gp.max_windows * 4)));
        g.win.win_rows = reinterpret_cast<uint32_t *>(take(align_up((size_t)gp.max_windows * 4)));
        g.win.win_start = reinterpret_cast<uint32_t *>(take(align_up((size_t)gp.max_windows * 4)));
        g.win.win_tile0 = reinterpret_cast<uint32_t *>(take(align_up((size_t)gp.max_windows * 4)));
        g.win.tile_info = reinterpret_cast<uint4 *>(take(align_up((size_t)gp.max_tiles * 16)));
        g.win.chunk_counts = reinterpret_cast<uint32_t *>(
            take(align_up((size_t)kMoeGemmMaxChunks * (experts + (sb ? 1 : 0)) * 4)));
        g.win.ranks = reinterpret_cast<uint32_t *>(take(align_up((size_t)(nslots + sh_rows) * 4)));
        uint16_t *xp_g = reinterpret_cast<uint16_t *>(take(gp.xp_gu));
        uint16_t *xp_u = reinterpret_cast<uint16_t *>(take(gp.xp_gu));
        uint16_t *xp_d = reinterpret_cast<uint16_t *>(take(gp.xp_down));
        float *pl_g = reinterpret_cast<float *>(take(gp.planes_gu));
        float *pl_u = reinterpret_cast<float *>(take(gp.planes_gu));
        float *pl_d = reinterpret_cast<float *>(take(gp.planes_down));
        hipError_t e = run_moe_gemm_windows(inds, nslots, experts, sh_rows, g.win, stream);
        if (e != hipSuccess) return launched(e, "exl3_moe (gemm windows)");
        g.x = x;
        g.x_dtype = x_dtype;
        g.topk = topk;
        g.experts = experts;
        g.nslots = nslots;
        g.sh = sb ? 1 : 0;
        g.n = uniform_lane ? n[0] : 0;
        g.sh_n = sb ? sb->n : 0;
        g.k = k;
        g.table = table;
        g.meta = meta;
        g.meta_col[0] = 0;
        g.meta_col[1] = 1;
        if (tt) {
            g.seg_off[0] = tt->off[0];
            g.seg_off[1] = tt->off[1];
            g.seg_k1[0] = tt->k1[0];
            g.seg_k1[1] = tt->k1[1];
        }
        g.clamp_limit = (float)clamp_limit;
        g.max_tiles = gp.max_tiles;
        g.max_windows = gp.max_windows;
        // gate and up: prepared inputs, then one GEMM launch for both (grid z = projection)
        g.in = hidden;
        g.out = inter;
        for (int i = 0; i < 2; i++) {
            g.trellis[i] = tr[i];
            g.suh[i] = su[i];
            g.sh_trellis[i] = sb ? sb->tr[i] : nullptr;
            g.sh_suh[i] = sb ? sb->su[i] : nullptr;
        }
        g.xp[0] = xp_g;
        g.xp[1] = xp_u;
        g.planes[0] = pl_g;
        g.planes[1] = pl_u;
        e = run_moe_gemm_prepare(g, 2, stream);
        if (e != hipSuccess) return launched(e, "exl3_moe (gemm prepare)");
        e = run_moe_gemm(fam, g, 2, stream);
        if (e != hipSuccess) return launched(e, "exl3_moe (gemm gate/up)");
        // the mid (down's prepared input), then the down GEMM
        MoeGemmArgs d = g;
        d.in = inter;
        d.out = hidden;
        d.mid_planes[0] = pl_g;
        d.mid_planes[1] = pl_u;
        d.mid_svh[0] = sv[0];
        d.mid_svh[1] = sv[1];
        d.down_suh = su[2];
        d.trellis[0] = tr[2];
        d.meta_col[0] = 2;
        if (tt) {
            d.seg_off[0] = tt->off[2];
            d.seg_k1[0] = tt->k1[2];
        }
        if (sb) {
            d.sh_mid_svh[0] = sb->sv[0];
            d.sh_mid_svh[1] = sb->sv[1];
            d.sh_down_suh = sb->su[2];
            d.sh_trellis[0] = sb->tr[2];
        }
        d.xp[0] = xp_d;
        d.planes[0] = pl_d;
        e = run_moe_gemm_mid(d, stream);
        if (e != hipSuccess) return launched(e, "exl3_moe (gemm mid)");
        e = run_moe_gemm(fam, d, 1, stream);
        if (e != hipSuccess) return launched(e, "exl3_moe (gemm down)");
        // the score-weighted reduce over each token's slots (+ a shared expert)
        ReduceArgs r{};
        r.part = pl_d;
        r.splits = 1;
        r.hidden = hidden;
        r.topk = topk;
        r.rows = rows;
        r.slots = inds;
        r.bank_limit = experts;
        r.scores = scores;
        r.score_dtype = scores_dtype;
        r.svh = sv[2];
        r.shared = shared;
        r.gate = shared ? shared_gate : nullptr;
        r.sh_part = sb ? pl_d + (size_t)nslots * hidden : nullptr;
        r.sh_svh = sb ? sb->sv[2] : nullptr;
        r.y = y;
        r.y_dtype = y_dtype;
        r.out_scale = 1.0f;
        return launched(run_moe_reduce(r, stream), "exl3_moe (gemm reduce)");
    }
    // With a fused shared bank its rows join either arm as groups of SH_ROWS rows placed first in the grid; planes
    // are kept per row (slots nslots .. nslots + rows - 1), so the plan counts rows more.
    const int sh_groups = sb ? (rows + SH_ROWS - 1) / SH_ROWS : 0;
    MoePlan p = plan_moe(nslots, hidden, inter, moe_windows_enabled() && moe_windowed(rows, nslots, experts),
                         sb ? rows : 0);
    const size_t need = p.total();
    if (ws_bytes < need || !ws || (reinterpret_cast<uintptr_t>(ws) % kAlign))
        return fail(EXL3_ERR_WORKSPACE, "moe: workspace of %zu bytes (256-aligned) needed, got %zu", need, ws_bytes);
    char *w = static_cast<char *>(ws) + kZeroBytes;
    float *gate_part = reinterpret_cast<float *>(w);
    float *up_part = reinterpret_cast<float *>(w + p.gu_bytes);
    float *down_part = reinterpret_cast<float *>(w + 2 * p.gu_bytes);
    const float scale = out_scale_of(fam);
    // 0) sorted arm: group the slots into expert windows
    uint32_t *win_count = nullptr, *win_expert = nullptr, *win_rows = nullptr, *win_slots = nullptr;
    int groups = nslots + sh_groups, grows = 1;
    if (p.windowed) {
        char *t = w + 2 * p.gu_bytes + p.down_bytes;
        win_count = reinterpret_cast<uint32_t *>(t);
        t += align_up(sizeof(uint32_t));
        win_expert = reinterpret_cast<uint32_t *>(t);
        t += align_up((size_t)nslots * sizeof(uint32_t));
        win_rows = reinterpret_cast<uint32_t *>(t);
        t += align_up((size_t)nslots * sizeof(uint32_t));
        win_slots = reinterpret_cast<uint32_t *>(t);
        hipError_t e = run_moe_windows(inds, nslots, experts, win_count, win_expert, win_rows, win_slots, stream);
        if (e != hipSuccess) return launched(e, "exl3_moe (windows)");
        groups = std::min(nslots, experts + (nslots + MOE_WINDOW_ROWS - 1) / MOE_WINDOW_ROWS) + sh_groups;
        grows = MOE_WINDOW_ROWS;
    }

    // 1) gate and up GEMVs of every slot (PAIR_GEMV_SOURCE): f32 planes [slot][split][inter]
    GemvArgs a{};
    a.x = x;
    a.x_dtype = x_dtype;
    a.rows = grows;
    a.in = hidden;
    a.out = inter;
    a.x_div = topk;
    a.win_count = win_count;
    a.win_expert = win_expert;
    a.win_rows = win_rows;
    a.win_slots = win_slots;
    for (int i = 0; i < 2; i++) {
        a.trellis[i] = tr[i];
        a.suh[i] = su[i];
        a.svh[i] = sv[i];
        a.meta_col[i] = i;
    }
    a.n = n[0];
    a.bank_of = inds;
    a.bank_limit = experts;
    a.meta = meta;
    a.meta_lane_only = meta_lane_only;
    if (tt) {
        for (int i = 0; i < 2; i++) {
            a.seg_off[i] = tt->off[i];
            a.seg_k1[i] = tt->k1[i];
        }
    }
    a.table = table;
    a.k = k;
    a.out_scale = scale;
    a.partial[0] = gate_part;
    a.partial[1] = up_part;
    a.splits = p.s1;
    a.groups = groups;
    a.nproj = 2;
    // Gate and up of a uniform bank at different rates (moeMixedDecode, src/exl3/root.zig:705-722): one launch each,
    // each at its own rate.
    const bool split_pair = !meta && !tt && n[0] != n[1];
    if (split_pair) a.nproj = 1;
    a.fused_finish = 0;
    a.partial_only = 1;
    if (sb) {
        a.sh_groups = sh_groups;
        a.sh_from = nslots;
        a.sh_rows = rows;
        a.sh_n = sb->n;
        for (int i = 0; i < 2; i++) {
            a.sh_trellis[i] = sb->tr[i];
            a.sh_suh[i] = sb->su[i];
            a.sh_svh[i] = sb->sv[i];
        }
    }
    GemvArgs u{};  // gate and up at different rates: up's own launch
    if (split_pair) {
        u = a;
        u.trellis[0] = tr[1];
        u.suh[0] = su[1];
        u.svh[0] = sv[1];
        u.partial[0] = up_part;
        u.n = n[1];
        int fam_u;
        if (resolve_decode(dec, n[1], &fam_u, &u.k)) return EXL3_ERR_RATE_MISSING;
    }

    // 2) SwiGLU mid + down GEMV of every slot (DOWN_FUSED_SOURCE): f32 planes [slot][split][hidden]
    GemvArgs d{};
    d.x = nullptr;
    d.x_dtype = x_dtype;
    d.rows = grows;
    d.in = inter;
    d.out = hidden;
    d.x_div = 1;
    d.win_count = win_count;
    d.win_expert = win_expert;
    d.win_rows = win_rows;
    d.win_slots = win_slots;
    d.mid_part[0] = gate_part;
    d.mid_part[1] = up_part;
    d.mid_splits = p.s1;
    d.mid_svh[0] = sv[0];
    d.mid_svh[1] = sv[1];
    d.clamp_limit = (float)clamp_limit;
    d.trellis[0] = tr[2];
    d.suh[0] = su[2];
    d.svh[0] = sv[2];
    d.meta_col[0] = 2;
    d.n = n[2];
    d.bank_of = inds;
    d.bank_limit = experts;
    d.meta = meta;
    d.meta_lane_only = meta_lane_only;
    if (tt) {
        d.seg_off[0] = tt->off[2];
        d.seg_k1[0] = tt->k1[2];
    }
    d.table = table;
    d.k = k;
    if (!meta && !tt && n[2] != n[0]) {
        int fam_d;
        if (resolve_decode(dec, n[2], &fam_d, &d.k)) return EXL3_ERR_RATE_MISSING;
    }
    d.out_scale = scale;
    d.partial[0] = down_part;
    d.splits = p.s2;
    d.groups = groups;
    d.nproj = 1;
    d.fused_finish = 0;
    d.partial_only = 1;
    // The down projection folds straight into a 16-bit y (score-weighted, exact fixed point, shared expert added by
    // the completing arrival) when every token's topk * splits arrivals fit the count field and its rows fit the
    // zeroed region; the planes + reduce launch otherwise (and for an f32 y, which the fixed point would quantise).
    const bool fold = sb || (topk * p.s2 <= FOLD_MAX_SPLITS && (size_t)rows * hidden <= kFoldWords &&
                             y_dtype != EXL3_DT_F32 && knob(EXL3_KNOB_MOE_FOLD, 1) != 0);
    if (fold) {
        d.partial_only = 0;
        d.fused_finish = 1;
        d.fold = static_cast<unsigned long long *>(ws);
        d.fold_arrivals = topk * p.s2;
        d.fold_topk = topk;
        d.fold_scores = scores;
        d.score_dtype = scores_dtype;
        d.fold_shared = shared;
        d.fold_gate = shared ? shared_gate : nullptr;
        d.y = y;
        d.y_dtype = y_dtype;
    }
    if (sb) {  // moe_shared_fusable checked that the three word sets fit the zeroed region
        d.sh_groups = sh_groups;
        d.sh_from = nslots;
        d.sh_rows = rows;
        d.sh_n = sb->n;
        d.sh_trellis[0] = sb->tr[2];
        d.sh_suh[0] = sb->su[2];
        d.sh_svh[0] = sb->sv[2];
        d.sh_mid_svh[0] = sb->sv[0];
        d.sh_mid_svh[1] = sb->sv[1];
        d.sh_fold = d.fold + (size_t)rows * hidden;
        d.fold_comb = d.fold + (size_t)2 * rows * hidden;
        d.fold_shared = nullptr;
        d.fold_gate = nullptr;
    }
    // The per-slot arm's gate/up and down as ONE launch (run_moe_chain): the down workgroups' tile loads go out while
    // gate/up runs and the second launch's start-up is gone, but each group's planes then cross XCDs through memory
    // (written through, a counter, L2-bypassing loads), which costs about what the kernel boundary did.  Taken where
    // it measured faster: 2 to 8 rows with a fused shared bank (C4's layer: 2 rows 26.9 -> 25.6 us, 4 rows 40.8 ->
    // 38.2, 8 rows 61.6 -> 59.1); one row (17.2 -> 19.4 us) and routed-only layers keep two launches.  It needs one
    // rate for the bank, the down folding into y and the counters clear of the fold words in use.
    // EXL3_KNOB_MOE_CHAIN pins it (1) or rules it out (0).
    const int groups_total = groups;
    const int chain_knob = knob(EXL3_KNOB_MOE_CHAIN, -1);
    const bool chain_wanted = chain_knob > 0 || (chain_knob < 0 && sb && rows >= 2);
    const bool chain = chain_wanted && !p.windowed && fold && !split_pair && !meta && !tt && n[0] == n[2] &&
                       lane_rate(n[0]) &&
                       (size_t)3 * rows * hidden <= kFoldWords - CHAIN_CTR_BYTES / sizeof(unsigned long long) &&
                       (size_t)2 * groups_total * COUNTER_STRIDE * sizeof(uint32_t) <= CHAIN_CTR_BYTES;
    hipError_t e;
    if (chain) {
        uint32_t *ctr = reinterpret_cast<uint32_t *>(static_cast<char *>(ws) + kZeroBytes - CHAIN_CTR_BYTES);
        a.chain_ctr = d.chain_ctr = ctr;
        a.chain_need = d.chain_need = (inter / 128) * p.s1 * 2;  // the group's gate/up workgroups
        a.chain_need2 = d.chain_need2 = (hidden / 128) * p.s2;   // its down workgroups
        e = run_moe_chain(fam, a, d, stream);
        if (e != hipSuccess) return launched(e, "exl3_moe (chain)");
        return ok();
    }
    e = run_gemv(fam, PRO_X, a, stream);
    if (e != hipSuccess) return launched(e, "exl3_moe (gate/up)");
    if (split_pair) {
        e = run_gemv(fam, PRO_X, u, stream);
        if (e != hipSuccess) return launched(e, "exl3_moe (up)");
    }
    e = run_gemv(fam, PRO_MID, d, stream);
    if (e != hipSuccess) return launched(e, "exl3_moe (down)");
    if (fold) return ok();

    // 3) score-weighted reduce (+ shared expert)
    ReduceArgs r{};
    r.part = down_part;
    r.splits = p.s2;
    r.hidden = hidden;
    r.topk = topk;
    r.rows = rows;
    r.slots = inds;
    r.bank_limit = experts;
    r.scores = scores;
    r.score_dtype = scores_dtype;
    r.svh = sv[2];
    r.shared = shared;
    r.gate = shared ? shared_gate : nullptr;
    r.y = y;
    r.y_dtype = y_dtype;
    r.out_scale = 1.0f;
    e = run_moe_reduce(r, stream);
    return launched(e, "exl3_moe (reduce)");
}

// ---- Static scratch for exl3_linear_noalloc ------------------------------------------------------------------
// The device memory of exl3_linear_noalloc: a file-scope device array that every GPU the library loads on holds
// until the process ends.  In host code `scratch` is only a stand-in for the symbol, never a device address: its
// address on a device comes from hipGetSymbolAddress, taken once per device (with that device current) at the
// entry point's first call there and kept per device; every launch and fill uses that address.  The first
// kZeroBytes carry the fused finish's counters, fold words and overflow words, which must start at zero: the same
// first call clears them with the fill kernel, and every call leaves them at zero again.
constexpr size_t kNoallocScratchBytes = EXL3_NOALLOC_SCRATCH_BYTES;
static_assert(kNoallocScratchBytes > kZeroBytes, "the static scratch holds the zeroed region and more");
std::mutex g_scratch_mu;
void *g_scratch_at[kMaxDevices] = {};

}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

namespace {

// This device's scratch address (set up on first use: symbol address, then the zeroed region cleared on `stream`).
int32_t noalloc_scratch(hipStream_t stream, void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return fail(EXL3_ERR_LAUNCH, "linear_noalloc: no current device (%s)", hipGetErrorString(e));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_at[dev]) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(stream, &cs);
        if (e != hipSuccess) return fail(EXL3_ERR_LAUNCH, "linear_noalloc: %s", hipGetErrorString(e));
        if (cs != hipStreamCaptureStatusNone)
            return fail(EXL3_ERR_WORKSPACE, "linear_noalloc: the first call on device %d sets up its static scratch "
                                            "and must run outside a stream capture", dev);
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(EXL3_ERR_LAUNCH, "linear_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
        e = run_fill_zero(p, kZeroBytes, stream);
        if (e != hipSuccess) return launched(e, "linear_noalloc (scratch set-up)");
        g_scratch_at[dev] = p;
    }
    *out = g_scratch_at[dev];
    return ok();
}

int32_t declined(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
int32_t declined(const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return EXL3_DECLINED;
}


// A bank whose three projections share one admitted rate, as a SharedBank (expert 0 of it serves).
int32_t shared_bank_checks(const exl3_bank_t *b, const char *what, SharedBank *out) {
    if (!b) return fail(EXL3_ERR_BAD_SHAPE, "%s: no bank", what);
    const exl3_proj_t *pr[3] = {&b->gate, &b->up, &b->down};
    for (int i = 0; i < 3; i++) {
        if (!rate_admitted(pr[i]->n) || !pr[i]->trellis || !pr[i]->suh || !pr[i]->svh)
            return fail(EXL3_ERR_BAD_SHAPE, "%s: projection %d has n=%d or a null operand", what, i, pr[i]->n);
        out->tr[i] = pr[i]->trellis;
        out->su[i] = pr[i]->suh;
        out->sv[i] = pr[i]->svh;
    }
    if (b->gate.n != b->up.n || b->gate.n != b->down.n)
        return fail(EXL3_ERR_BAD_SHAPE, "%s: gate/up/down rates differ", what);
    out->n = b->gate.n;
    return ok();
}

// A per-tile-rate bank: its rates, codebook and operands; the family, the constants at n_b (the kernels read both
// rates' rows from the table) and the segment tables.
int32_t tiled_checks(const exl3_tiled_t *b, const exl3_decode_t &dec, const char *what, int *fam, DecodeK *k,
                     TiledTables *tt) {
    if (!b || b->experts <= 0) return fail(EXL3_ERR_BAD_SHAPE, "%s: no bank", what);
    if (b->n_a != TILED_NA || b->n_b != TILED_NB)
        return fail(EXL3_ERR_BAD_SHAPE, "%s: tile rates %d / %d (the per-tile mix is n = %d / %d)", what, b->n_a,
                    b->n_b, TILED_NA, TILED_NB);
    for (int i = 0; i < 3; i++) {
        if (!b->trellis[i] || !b->seg_off[i] || !b->seg_k1[i] || !b->suh[i] || !b->svh[i])
            return fail(EXL3_ERR_BAD_SHAPE, "%s: projection %d has a null operand", what, i);
        if (reinterpret_cast<uintptr_t>(b->seg_k1[i]) % 4)
            return fail(EXL3_ERR_BAD_SHAPE, "%s: projection %d's seg_k1 must be 4-byte aligned", what, i);
        tt->off[i] = b->seg_off[i];
        tt->k1[i] = b->seg_k1[i];
    }
    DecodeK ka;
    int32_t rc = resolve_decode(dec, TILED_NA, fam, &ka);
    if (rc) return rc;
    rc = resolve_decode(dec, TILED_NB, fam, k);
    if (rc) return rc;
    if (*fam == FAM_PAIR || *fam == FAM_MUL1)
        return fail(EXL3_ERR_CODEBOOK_UNSUPPORTED, "%s: per-tile rates serve MCG, 3INST and the SPEC1 / STD1 hash rows",
                    what);
    return ok();
}

// A uniform bank's operands and rates, each rate's codebook row present; fam / k: the decode at the gate's rate.
int32_t moe_bank_checks(const exl3_bank_t *bank, int32_t experts, const exl3_decode_t &dec, int n[3], int *fam,
                        DecodeK *k) {
    if (!bank || experts <= 0) return fail(EXL3_ERR_BAD_SHAPE, "moe: no bank");
    const exl3_proj_t *pr[3] = {&bank->gate, &bank->up, &bank->down};
    for (int i = 0; i < 3; i++) {
        if (!rate_admitted(pr[i]->n) || !pr[i]->trellis || !pr[i]->suh || !pr[i]->svh)
            return fail(EXL3_ERR_BAD_SHAPE, "moe: projection %d has n=%d or a null operand", i, pr[i]->n);
        n[i] = pr[i]->n;
        int32_t rc = resolve_decode(dec, n[i], fam, k);  // every projection's rate must have its codebook row
        if (rc) return rc;
    }
    return resolve_decode(dec, n[0], fam, k);
}

// `moe` / `moeWithShared` / `moeWithGatedShared` over a uniform bank: every check, then the launches.
int32_t moe_uniform(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter, int32_t experts,
                    const exl3_bank_t *bank, const uint32_t *inds, const void *scores, int32_t scores_dtype,
                    int32_t topk, exl3_decode_t dec, bool verify, int32_t clamp_limit, const void *shared,
                    const void *shared_gate, void *y, int32_t y_dtype, void *workspace, size_t workspace_bytes,
                    hipStream_t stream) {
    int32_t rc = moe_common_checks(x_dtype, y_dtype, rows, hidden, inter, topk, clamp_limit, scores_dtype);
    if (rc) return rc;
    int n[3];
    int fam;
    DecodeK k;
    rc = moe_bank_checks(bank, experts, dec, n, &fam, &k);
    if (rc) return rc;
    if (rows == 0) return ok();
    if (!x || !inds || !scores || !y) return fail(EXL3_ERR_BAD_SHAPE, "moe: null operand");
    if (shared_gate && !shared) return fail(EXL3_ERR_BAD_SHAPE, "moe: a shared-expert gate without its shared expert");
    const uint16_t *tr[3] = {bank->gate.trellis, bank->up.trellis, bank->down.trellis};
    const uint16_t *su[3] = {bank->gate.suh, bank->up.suh, bank->down.suh};
    const uint16_t *sv[3] = {bank->gate.svh, bank->up.svh, bank->down.svh};
    return moe_launch(fam, k, dec, dec.table, x, x_dtype, rows, hidden, inter, experts, tr, su, sv, n, nullptr, 0,
                      inds, scores, scores_dtype, topk, verify, clamp_limit, shared, shared_gate, y, y_dtype,
                      workspace, workspace_bytes, stream);
}

}  // namespace

extern "C" {

int32_t exl3_abi_version(void) { return EXL3_ABI_VERSION; }

const char *exl3_last_error(void) { return g_err.c_str(); }

int32_t exl3_set_override(int32_t k, int32_t value, int32_t enable) {
    if (k < 0 || k >= EXL3_KNOB_COUNT) return fail(EXL3_ERR_BAD_SHAPE, "set_override: unknown knob %d", k);
    if (enable && value == INT32_MIN) return fail(EXL3_ERR_BAD_SHAPE, "set_override: value INT32_MIN is reserved");
    g_override[k].store(enable ? value : INT32_MIN, std::memory_order_relaxed);
    return ok();
}

int32_t exl3_decode_codewords(const uint16_t *codewords, int64_t count, int32_t n, exl3_decode_t dec, uint16_t *out,
                              hipStream_t stream) {
    if (count < 0) return fail(EXL3_ERR_BAD_SHAPE, "decode_codewords: negative count");
    if (!rate_admitted(n)) return fail(EXL3_ERR_BAD_SHAPE, "decode_codewords: n=%d is not an admitted rate", n);
    int fam;
    DecodeK k;
    int32_t rc = resolve_decode(dec, n, &fam, &k);
    if (rc) return rc;
    if (count == 0) return ok();
    if (!codewords || !out) return fail(EXL3_ERR_BAD_SHAPE, "decode_codewords: null operand");
    return launched(run_decode_codewords(fam, codewords, count, k, out, stream), "exl3_decode_codewords");
}

int32_t exl3_reconstruct_inner(const uint16_t *trellis, int32_t in_features, int32_t out_features, int32_t n,
                               exl3_decode_t dec, uint16_t *out, hipStream_t stream) {
    if (in_features <= 0 || out_features <= 0 || in_features % 16 || out_features % 16)
        return fail(EXL3_ERR_BAD_SHAPE, "reconstruct_inner: in=%d out=%d (multiples of 16)", in_features, out_features);
    if (!rate_admitted(n)) return fail(EXL3_ERR_BAD_SHAPE, "reconstruct_inner: n=%d is not an admitted rate", n);
    int fam;
    DecodeK k;
    int32_t rc = resolve_decode(dec, n, &fam, &k);
    if (rc) return rc;
    if (!trellis || !out) return fail(EXL3_ERR_BAD_SHAPE, "reconstruct_inner: null operand");
    return launched(run_reconstruct_inner(fam, trellis, in_features / 16, out_features / 16, n, k, out, stream),
                    "exl3_reconstruct_inner");
}

size_t exl3_linear_workspace_size(int32_t rows, int32_t in_features, int32_t out_features, int32_t n) {
    if (rows <= 0 || in_features <= 0 || out_features <= 0 || in_features % 128 || out_features % 128) return 0;
    return linear_ws(1, rows, in_features, out_features, n);
}

size_t exl3_linear_grouped_workspace_size(int32_t groups, int32_t rows, int32_t in_features, int32_t out_features,
                                          int32_t n) {
    if (groups <= 0 || rows <= 0 || in_features <= 0 || out_features <= 0 || in_features % 128 || out_features % 128)
        return 0;
    return linear_ws(groups, rows, in_features, out_features, n);
}

int32_t exl3_linear(const void *x, int32_t x_dtype, int32_t rows, int32_t in_features, int32_t out_features,
                    const uint16_t *trellis, int32_t n, const uint16_t *suh, const uint16_t *svh, exl3_decode_t dec,
                    void *y, int32_t y_dtype, void *workspace, size_t workspace_bytes, hipStream_t stream) {
    return linear_impl(x, x_dtype, 1, rows, in_features, out_features, trellis, n, suh, svh, dec, y, y_dtype,
                       workspace, workspace_bytes, stream);
}

int32_t exl3_linear_grouped(const void *x, int32_t x_dtype, int32_t groups, int32_t rows, int32_t in_features,
                            int32_t out_features, const uint16_t *trellis, int32_t n, const uint16_t *suh,
                            const uint16_t *svh, exl3_decode_t dec, void *y, int32_t y_dtype, void *workspace,
                            size_t workspace_bytes, hipStream_t stream) {
    return linear_impl(x, x_dtype, groups, rows, in_features, out_features, trellis, n, suh, svh, dec, y, y_dtype,
                       workspace, workspace_bytes, stream);
}

int32_t exl3_linear_noalloc(const void *x, int32_t x_dtype, int32_t rows, int32_t in_features, int32_t out_features,
                            const uint16_t *trellis, int32_t n, const uint16_t *suh, const uint16_t *svh,
                            exl3_decode_t dec, void *y, int32_t y_dtype, hipStream_t stream) {
    int fam;
    DecodeK k;
    int32_t rc = linear_checks(x, x_dtype, 1, rows, in_features, out_features, trellis, n, suh, svh, dec, y, y_dtype,
                               &fam, &k);
    if (rc || rows == 0) return rc;
    // The static scratch holds every arm's needs but the k-split GEMM's partials past its size: such a call takes
    // the decode-wave tile instead.
    const bool split_ok = linear_ws(1, rows, in_features, out_features, n) <= kNoallocScratchBytes;
    const size_t need = linear_ws(1, rows, in_features, out_features, n, split_ok);
    if (need > kNoallocScratchBytes)
        return fail(EXL3_ERR_WORKSPACE,
                    "linear_noalloc: rows=%d in=%d out=%d n=%d need %zu bytes of scratch, past the static scratch's %zu "
                    "(use exl3_linear with a workspace)", rows, in_features, out_features, n, need,
                    kNoallocScratchBytes);
    void *ws = nullptr;
    rc = noalloc_scratch(stream, &ws);
    if (rc) return rc;
    return linear_impl(x, x_dtype, 1, rows, in_features, out_features, trellis, n, suh, svh, dec, y, y_dtype, ws,
                       kNoallocScratchBytes, stream, split_ok);
}

size_t exl3_linear_pair_workspace_size(int32_t groups, int32_t rows, int32_t in_features, int32_t mid_features,
                                       int32_t out_features) {
    if (groups <= 0 || rows <= 0 || rows > kRowsMax || in_features <= 0 || mid_features <= 0 || out_features <= 0 ||
        in_features % 128 || mid_features % 128 || out_features % 128)
        return 0;
    // the two launches share the zeroed region and the split partials (one after the other on the stream); the
    // intermediate [rows][groups * mid] (at most 4 bytes an element) follows
    const size_t scratch = std::max(linear_ws(groups, rows, in_features, mid_features, 64),
                                    linear_ws(1, rows, groups * mid_features, out_features, 64));
    return align_up(scratch) + align_up((size_t)rows * groups * mid_features * 4);
}

int32_t exl3_linear_pair(const void *x, int32_t x_dtype, int32_t groups, int32_t rows, int32_t in_features,
                         int32_t mid_features, int32_t out_features, const uint16_t *a_trellis, int32_t a_n,
                         const uint16_t *a_suh, const uint16_t *a_svh, exl3_decode_t a_dec,
                         const uint16_t *b_trellis, int32_t b_n, const uint16_t *b_suh, const uint16_t *b_svh,
                         exl3_decode_t b_dec, void *y, int32_t y_dtype, void *workspace, size_t workspace_bytes,
                         hipStream_t stream) {
    int fam;
    DecodeK k;
    int32_t rc = linear_checks(x, x_dtype, groups, rows, in_features, mid_features, a_trellis, a_n, a_suh, a_svh,
                               a_dec, y, x_dtype, &fam, &k);
    if (rc) return rc;
    if (groups > 0 && mid_features > 0 && (long)groups * mid_features > (1L << 30))
        return fail(EXL3_ERR_BAD_SHAPE, "linear_pair: groups x mid too large");
    rc = linear_checks(x, x_dtype, 1, rows, groups * mid_features, out_features, b_trellis, b_n, b_suh, b_svh, b_dec, y,
                       y_dtype, &fam, &k);
    if (rc || rows == 0) return rc;
    if (rows > kRowsMax)
        return declined("linear_pair: declined (rows=%d past one decode launch of %d): run exl3_linear_grouped, "
                        "transpose, then exl3_linear", rows, kRowsMax);
    const size_t need = exl3_linear_pair_workspace_size(groups, rows, in_features, mid_features, out_features);
    if (workspace_bytes < need || !workspace || (reinterpret_cast<uintptr_t>(workspace) % kAlign))
        return fail(EXL3_ERR_WORKSPACE, "linear_pair: workspace of %zu bytes (256-aligned) needed, got %zu", need,
                    workspace_bytes);
    const size_t scratch = need - align_up((size_t)rows * groups * mid_features * 4);
    void *mid = static_cast<char *>(workspace) + scratch;
    rc = linear_impl(x, x_dtype, groups, rows, in_features, mid_features, a_trellis, a_n, a_suh, a_svh, a_dec, mid,
                     x_dtype, workspace, scratch, stream, true, /*y_rows_major=*/true);
    if (rc) return rc;
    return linear_impl(mid, x_dtype, 1, rows, groups * mid_features, out_features, b_trellis, b_n, b_suh, b_svh, b_dec,
                       y, y_dtype, workspace, scratch, stream);
}

int32_t exl3_workspace_init(void *workspace, size_t workspace_bytes, hipStream_t stream) {
    if (!workspace || workspace_bytes == 0) return ok();
    if (reinterpret_cast<uintptr_t>(workspace) % 4) return fail(EXL3_ERR_WORKSPACE, "workspace_init: misaligned");
    return launched(run_fill_zero(workspace, workspace_bytes, stream), "exl3_workspace_init");
}

size_t exl3_moe_workspace_size(int32_t rows, int32_t topk, int32_t hidden, int32_t inter) {
    if (rows <= 0 || topk <= 0 || hidden <= 0 || inter <= 0 || hidden % 128 || inter % 128) return 0;
    const int nslots = rows * topk;
    size_t need = plan_moe(nslots, hidden, inter, false).total();
    if (moe_windowed(rows, nslots, 1)) need = std::max(need, plan_moe(nslots, hidden, inter, true).total());
    // the GEMM arm, for any expert count it serves (a layer with fewer experts takes less)
    const int gk = knob(EXL3_KNOB_MOE_GEMM, -1);
    if (gk > 0 || (gk != 0 && nslots >= kMoeGemmMinSlotsPerExpert))
        need = std::max(need, plan_moe_gemm(nslots, hidden, inter, kMoeGemmMaxExperts).total());
    return need;
}

int32_t exl3_moe(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter, int32_t experts,
                 const exl3_bank_t *bank, const uint32_t *inds, const void *scores, int32_t scores_dtype, int32_t topk,
                 exl3_decode_t dec, int32_t verify_rows, int32_t clamp_limit, const void *shared, void *y,
                 int32_t y_dtype, void *workspace, size_t workspace_bytes, hipStream_t stream) {
    return moe_uniform(x, x_dtype, rows, hidden, inter, experts, bank, inds, scores, scores_dtype, topk, dec,
                       verify_rows != 0, clamp_limit, shared, nullptr, y, y_dtype, workspace, workspace_bytes, stream);
}

int32_t exl3_moe_with_gated_shared(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter,
                                   int32_t experts, const exl3_bank_t *bank, const uint32_t *inds, const void *scores,
                                   int32_t scores_dtype, int32_t topk, exl3_decode_t dec, int32_t verify_rows,
                                   const void *shared_down, const void *shared_gate, void *y, int32_t y_dtype,
                                   void *workspace, size_t workspace_bytes, hipStream_t stream) {
    if (!shared_down || !shared_gate)
        return fail(EXL3_ERR_BAD_SHAPE, "moe_with_gated_shared: the shared expert's output and its gate are required");
    return moe_uniform(x, x_dtype, rows, hidden, inter, experts, bank, inds, scores, scores_dtype, topk, dec,
                       verify_rows != 0, 0, shared_down, shared_gate, y, y_dtype, workspace, workspace_bytes, stream);
}

int32_t exl3_moe_ragged(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter,
                        const exl3_ragged_t *bank, const uint32_t *inds, const void *scores, int32_t scores_dtype,
                        int32_t topk, exl3_decode_t dec, int32_t verify_rows, int32_t clamp_limit,
                        const void *shared, const void *shared_gate, void *y, int32_t y_dtype, void *workspace,
                        size_t workspace_bytes, hipStream_t stream) {
    int32_t rc = moe_common_checks(x_dtype, y_dtype, rows, hidden, inter, topk, clamp_limit, scores_dtype);
    if (rc) return rc;
    if (!bank || bank->experts <= 0 || !bank->meta) return fail(EXL3_ERR_BAD_SHAPE, "moe_ragged: no bank");
    for (int i = 0; i < 3; i++)
        if (!bank->trellis[i] || !bank->suh[i] || !bank->svh[i])
            return fail(EXL3_ERR_BAD_SHAPE, "moe_ragged: projection %d has a null operand", i);
    int fam;
    DecodeK k;
    rc = resolve_decode(dec, 0, &fam, &k, /*per_rate_table=*/true);
    if (rc) return rc;
    if (rows == 0) return ok();
    if (!x || !inds || !scores || !y) return fail(EXL3_ERR_BAD_SHAPE, "moe_ragged: null operand");
    if (shared_gate && !shared)
        return fail(EXL3_ERR_BAD_SHAPE, "moe_ragged: a shared-expert gate without its shared expert");
    const int table = fam == FAM_PAIR ? (int)TABLE_PAIR1_W16_V1 : dec.table;
    const int n0[3] = {0, 0, 0};
    return moe_launch(fam, k, dec, table, x, x_dtype, rows, hidden, inter, bank->experts, bank->trellis, bank->suh,
                      bank->svh, n0, bank->meta, bank->lane_rates_only != 0, inds, scores, scores_dtype, topk,
                      verify_rows != 0, clamp_limit, shared, shared_gate, y, y_dtype, workspace, workspace_bytes,
                      stream);
}

size_t exl3_moe_groups_workspace_size(int32_t rows, int32_t topk, int32_t hidden, int32_t inter) {
    const size_t routed = exl3_moe_workspace_size(rows, topk, hidden, inter);
    if (routed == 0) return 0;
    const size_t nslots = (size_t)rows * topk, plane = align_up((size_t)rows * hidden * sizeof(float));
    return align_up(routed) + 2 * align_up(nslots * 4) + 2 * plane;
}

int32_t exl3_moe_groups(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter, int32_t groups,
                        const exl3_bank_t *banks, const int32_t *group_experts, const uint32_t *inds,
                        const void *scores, int32_t scores_dtype, int32_t topk, exl3_decode_t dec,
                        int32_t verify_rows, void *y, int32_t y_dtype, void *workspace, size_t workspace_bytes,
                        hipStream_t stream) {
    if (groups <= 0 || !banks || !group_experts)
        return fail(EXL3_ERR_GROUP_MISSING, "moe_groups: no group banks");
    int32_t rc = moe_common_checks(x_dtype, y_dtype, rows, hidden, inter, topk, 0, scores_dtype);
    if (rc) return rc;
    long total = 0;
    for (int g = 0; g < groups; g++) {  // every group's bank, before any launch
        int n[3], fam;
        DecodeK k;
        rc = moe_bank_checks(&banks[g], group_experts[g], dec, n, &fam, &k);
        if (rc) return rc;
        total += group_experts[g];
    }
    if (total > 0xFFFFFFFFL) return fail(EXL3_ERR_BAD_SHAPE, "moe_groups: too many experts");
    if (groups == 1)  // one bank: `moe` itself, rounded to y's dtype directly (root.zig:648)
        return moe_uniform(x, x_dtype, rows, hidden, inter, group_experts[0], &banks[0], inds, scores, scores_dtype,
                           topk, dec, verify_rows != 0, 0, nullptr, nullptr, y, y_dtype, workspace, workspace_bytes,
                           stream);
    if (rows == 0) return ok();
    if (!x || !inds || !scores || !y) return fail(EXL3_ERR_BAD_SHAPE, "moe_groups: null operand");
    const size_t need = exl3_moe_groups_workspace_size(rows, topk, hidden, inter);
    if (workspace_bytes < need || !workspace || (reinterpret_cast<uintptr_t>(workspace) % kAlign))
        return fail(EXL3_ERR_WORKSPACE, "moe_groups: workspace of %zu bytes (256-aligned) needed, got %zu", need,
                    workspace_bytes);
    const int nslots = rows * topk;
    const size_t routed = align_up(exl3_moe_workspace_size(rows, topk, hidden, inter));
    char *w = static_cast<char *>(workspace) + routed;
    uint32_t *local = reinterpret_cast<uint32_t *>(w);
    float *weight = reinterpret_cast<float *>(w + align_up((size_t)nslots * 4));
    float *acc = reinterpret_cast<float *>(w + 2 * align_up((size_t)nslots * 4));
    float *part = acc + align_up((size_t)rows * hidden * sizeof(float)) / sizeof(float);
    const size_t outs = (size_t)rows * hidden;
    uint32_t lo = 0;
    for (int g = 0; g < groups; g++) {
        // the group's partial in f32: slots outside it go to local expert 0 with score 0 (root.zig:662-678)
        hipError_t e = run_moe_group_routing(inds, scores, scores_dtype, nslots, lo, (uint32_t)group_experts[g],
                                             local, weight, stream);
        if (e != hipSuccess) return launched(e, "exl3_moe_groups (routing)");
        rc = moe_uniform(x, x_dtype, rows, hidden, inter, group_experts[g], &banks[g], local, weight, EXL3_DT_F32,
                         topk, dec, verify_rows != 0, 0, nullptr, nullptr, g == 0 ? acc : part, EXL3_DT_F32,
                         workspace, routed, stream);
        if (rc) return rc;
        if (g > 0) {
            e = run_add_f32(acc, part, outs, stream);  // the f32 sum in group order (root.zig:680-694)
            if (e != hipSuccess) return launched(e, "exl3_moe_groups (sum)");
        }
        lo += (uint32_t)group_experts[g];
    }
    return launched(run_cast_f32(acc, y, y_dtype, outs, stream), "exl3_moe_groups (cast)");  // one cast (:695-701)
}

size_t exl3_moe_with_shared_bank_workspace_size(int32_t rows, int32_t topk, int32_t hidden, int32_t inter) {
    const size_t routed = exl3_moe_workspace_size(rows, topk, hidden, inter);
    if (routed == 0) return 0;
    size_t need = std::max(routed, plan_moe(rows * topk, hidden, inter, false, rows).total());
    // the GEMM arm with the shared rows as one more expert's slots
    const int gk = knob(EXL3_KNOB_MOE_GEMM, -1);
    if (gk > 0 || (gk != 0 && rows * topk >= kMoeGemmMinSlotsPerExpert))
        need = std::max(need, plan_moe_gemm(rows * topk + rows, hidden, inter, kMoeGemmMaxExperts).total());
    if (moe_windowed(rows, rows * topk, 1)) need = std::max(need, plan_moe(rows * topk, hidden, inter, true, rows).total());
    return need;
}

int32_t exl3_moe_with_shared_bank(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter,
                                  int32_t experts, const exl3_bank_t *bank, const exl3_bank_t *shared_bank,
                                  const uint32_t *inds, const void *scores, int32_t scores_dtype, int32_t topk,
                                  exl3_decode_t dec, int32_t verify_rows, int32_t clamp_limit, void *y,
                                  int32_t y_dtype, void *workspace, size_t workspace_bytes, hipStream_t stream) {
    int32_t rc = moe_common_checks(x_dtype, y_dtype, rows, hidden, inter, topk, clamp_limit, scores_dtype);
    if (rc) return rc;
    if (!bank || experts <= 0) return fail(EXL3_ERR_BAD_SHAPE, "moe_with_shared_bank: no bank");
    SharedBank sb;
    bool whole = true;  // every projection admitted and present
    for (const exl3_proj_t *q : {&bank->gate, &bank->up, &bank->down})
        whole = whole && rate_admitted(q->n) && q->trellis && q->suh && q->svh;
    if (whole && (bank->gate.n != bank->up.n || bank->gate.n != bank->down.n))
        return declined("moe_with_shared_bank: declined (routed rates %d/%d/%d differ): run the shared expert as a "
                        "one-expert exl3_moe and pass it to exl3_moe as `shared`", bank->gate.n, bank->up.n,
                        bank->down.n);
    rc = shared_bank_checks(bank, "moe_with_shared_bank (routed)", &sb);
    if (rc) return rc;
    const int routed_n = sb.n;
    rc = shared_bank_checks(shared_bank, "moe_with_shared_bank (shared)", &sb);
    if (rc) return rc;
    int fam;
    DecodeK k;
    rc = resolve_decode(dec, routed_n, &fam, &k);
    if (rc) return rc;
    if (rows == 0) return ok();
    if (!x || !inds || !scores || !y) return fail(EXL3_ERR_BAD_SHAPE, "moe_with_shared_bank: null operand");
    if (sb.n != routed_n ||
        !moe_shared_fusable(rows, topk, hidden, inter, y_dtype, experts, lane_rate(routed_n), verify_rows))
        return declined("moe_with_shared_bank: declined (rows=%d, y dtype %d, rates %d/%d): run the shared expert as "
                        "a one-expert exl3_moe and pass it to exl3_moe as `shared`", rows, y_dtype, routed_n, sb.n);
    const uint16_t *tr[3] = {bank->gate.trellis, bank->up.trellis, bank->down.trellis};
    const uint16_t *su[3] = {bank->gate.suh, bank->up.suh, bank->down.suh};
    const uint16_t *sv[3] = {bank->gate.svh, bank->up.svh, bank->down.svh};
    const int n[3] = {routed_n, routed_n, routed_n};
    return moe_launch(fam, k, dec, dec.table, x, x_dtype, rows, hidden, inter, experts, tr, su, sv, n, nullptr, 0,
                      inds, scores, scores_dtype, topk, verify_rows != 0, clamp_limit, nullptr, nullptr, y, y_dtype,
                      workspace, workspace_bytes, stream, &sb);
}

int32_t exl3_moe_ragged_with_shared_bank(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter,
                                         const exl3_ragged_t *bank, const exl3_bank_t *shared_bank,
                                         const uint32_t *inds, const void *scores, int32_t scores_dtype, int32_t topk,
                                         exl3_decode_t dec, int32_t verify_rows, int32_t clamp_limit, void *y,
                                         int32_t y_dtype, void *workspace, size_t workspace_bytes,
                                         hipStream_t stream) {
    int32_t rc = moe_common_checks(x_dtype, y_dtype, rows, hidden, inter, topk, clamp_limit, scores_dtype);
    if (rc) return rc;
    if (!bank || bank->experts <= 0 || !bank->meta)
        return fail(EXL3_ERR_BAD_SHAPE, "moe_ragged_with_shared_bank: no bank");
    for (int i = 0; i < 3; i++)
        if (!bank->trellis[i] || !bank->suh[i] || !bank->svh[i])
            return fail(EXL3_ERR_BAD_SHAPE, "moe_ragged_with_shared_bank: projection %d has a null operand", i);
    SharedBank sb;
    rc = shared_bank_checks(shared_bank, "moe_ragged_with_shared_bank (shared)", &sb);
    if (rc) return rc;
    int fam;
    DecodeK k;
    rc = resolve_decode(dec, 0, &fam, &k, /*per_rate_table=*/true);
    if (rc) return rc;
    const int table = fam == FAM_PAIR ? (int)TABLE_PAIR1_W16_V1 : dec.table;
    // the shared bank decodes with the routed codebook at its own rate: its table must have that rate
    if ((fam == FAM_HASH || fam == FAM_PAIR)) {
        uint32_t m0, m1, m2, m3;
        if (!table_row(table, sb.n, m0, m1, m2, m3))
            return fail(EXL3_ERR_RATE_MISSING, "moe_ragged_with_shared_bank: table %d has no row for n=%d", table,
                        sb.n);
    }
    if (rows == 0) return ok();
    if (!x || !inds || !scores || !y) return fail(EXL3_ERR_BAD_SHAPE, "moe_ragged_with_shared_bank: null operand");
    const bool lane_only = bank->lane_rates_only != 0 && lane_rate(sb.n);
    if (!moe_shared_fusable(rows, topk, hidden, inter, y_dtype, bank->experts, lane_only, verify_rows))
        return declined("moe_ragged_with_shared_bank: declined (rows=%d, y dtype %d): run the shared expert as a "
                        "one-expert exl3_moe and pass it to exl3_moe_ragged as `shared`", rows, y_dtype);
    const int n0[3] = {0, 0, 0};
    return moe_launch(fam, k, dec, table, x, x_dtype, rows, hidden, inter, bank->experts, bank->trellis, bank->suh,
                      bank->svh, n0, bank->meta, lane_only, inds, scores, scores_dtype, topk, verify_rows != 0,
                      clamp_limit, nullptr, nullptr, y, y_dtype, workspace, workspace_bytes, stream, &sb);
}

int32_t exl3_reconstruct_tiled(const uint16_t *trellis, const uint32_t *seg_off, const uint8_t *seg_k1,
                               int32_t expert, int32_t in_features, int32_t out_features, int32_t n_a, int32_t n_b,
                               exl3_decode_t dec, uint16_t *out, hipStream_t stream) {
    if (in_features <= 0 || out_features <= 0 || in_features % 16 || out_features % 128 || expert < 0)
        return fail(EXL3_ERR_BAD_SHAPE, "reconstruct_tiled: in=%d out=%d expert=%d (in a multiple of 16, out of 128)",
                    in_features, out_features, expert);
    exl3_tiled_t b{};
    for (int i = 0; i < 3; i++) {
        b.trellis[i] = trellis;
        b.seg_off[i] = seg_off;
        b.seg_k1[i] = seg_k1;
        b.suh[i] = trellis;  // unused here: only the tables and rates are checked
        b.svh[i] = trellis;
    }
    b.experts = expert + 1;
    b.n_a = n_a;
    b.n_b = n_b;
    int fam;
    DecodeK ka, kb;
    TiledTables tt;
    int32_t rc = tiled_checks(&b, dec, "reconstruct_tiled", &fam, &kb, &tt);
    if (rc) return rc;
    rc = resolve_decode(dec, TILED_NA, &fam, &ka);
    if (rc) return rc;
    if (!out) return fail(EXL3_ERR_BAD_SHAPE, "reconstruct_tiled: null operand");
    return launched(run_reconstruct_tiled(fam, trellis, seg_off, seg_k1, expert, in_features / 16, out_features / 16,
                                          ka, kb, out, stream),
                    "exl3_reconstruct_tiled");
}

int32_t exl3_moe_tiled(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter,
                       const exl3_tiled_t *bank, const uint32_t *inds, const void *scores, int32_t scores_dtype,
                       int32_t topk, exl3_decode_t dec, int32_t verify_rows, int32_t clamp_limit, const void *shared,
                       const void *shared_gate, void *y, int32_t y_dtype, void *workspace, size_t workspace_bytes,
                       hipStream_t stream) {
    int32_t rc = moe_common_checks(x_dtype, y_dtype, rows, hidden, inter, topk, clamp_limit, scores_dtype);
    if (rc) return rc;
    int fam;
    DecodeK k;
    TiledTables tt;
    rc = tiled_checks(bank, dec, "moe_tiled", &fam, &k, &tt);
    if (rc) return rc;
    if (rows == 0) return ok();
    if (!x || !inds || !scores || !y) return fail(EXL3_ERR_BAD_SHAPE, "moe_tiled: null operand");
    if (shared_gate && !shared)
        return fail(EXL3_ERR_BAD_SHAPE, "moe_tiled: a shared-expert gate without its shared expert");
    const int n0[3] = {0, 0, 0};
    return moe_launch(fam, k, dec, dec.table, x, x_dtype, rows, hidden, inter, bank->experts, bank->trellis,
                      bank->suh, bank->svh, n0, nullptr, 0, inds, scores, scores_dtype, topk, verify_rows != 0,
                      clamp_limit, shared, shared_gate, y, y_dtype, workspace, workspace_bytes, stream, nullptr, &tt);
}

int32_t exl3_moe_tiled_with_shared_bank(const void *x, int32_t x_dtype, int32_t rows, int32_t hidden, int32_t inter,
                                        const exl3_tiled_t *bank, const exl3_bank_t *shared_bank,
                                        const uint32_t *inds, const void *scores, int32_t scores_dtype, int32_t topk,
                                        exl3_decode_t dec, int32_t verify_rows, int32_t clamp_limit, void *y,
                                        int32_t y_dtype, void *workspace, size_t workspace_bytes, hipStream_t stream) {
    int32_t rc = moe_common_checks(x_dtype, y_dtype, rows, hidden, inter, topk, clamp_limit, scores_dtype);
    if (rc) return rc;
    int fam;
    DecodeK k;
    TiledTables tt;
    rc = tiled_checks(bank, dec, "moe_tiled_with_shared_bank", &fam, &k, &tt);
    if (rc) return rc;
    SharedBank sb;
    rc = shared_bank_checks(shared_bank, "moe_tiled_with_shared_bank (shared)", &sb);
    if (rc) return rc;
    // the shared bank decodes with the routed codebook at its own rate: its table must have that rate
    if (fam == FAM_HASH) {
        uint32_t m0, m1, m2, m3;
        if (!table_row(dec.table, sb.n, m0, m1, m2, m3))
            return fail(EXL3_ERR_RATE_MISSING, "moe_tiled_with_shared_bank: table %d has no row for n=%d", dec.table,
                        sb.n);
    }
    if (rows == 0) return ok();
    if (!x || !inds || !scores || !y) return fail(EXL3_ERR_BAD_SHAPE, "moe_tiled_with_shared_bank: null operand");
    if (!lane_rate(sb.n) || !moe_shared_fusable(rows, topk, hidden, inter, y_dtype, bank->experts, true, verify_rows))
        return declined("moe_tiled_with_shared_bank: declined (rows=%d, y dtype %d, shared n=%d): run the shared expert "
                        "as a one-expert exl3_moe and pass it to exl3_moe_tiled as `shared`", rows, y_dtype, sb.n);
    const int n0[3] = {0, 0, 0};
    return moe_launch(fam, k, dec, dec.table, x, x_dtype, rows, hidden, inter, bank->experts, bank->trellis,
                      bank->suh, bank->svh, n0, nullptr, 0, inds, scores, scores_dtype, topk, verify_rows != 0,
                      clamp_limit, nullptr, nullptr, y, y_dtype, workspace, workspace_bytes, stream, &sb, &tt);
}

int32_t exl3_route_topk(const float *logits, int32_t rows, int32_t experts, int32_t k, uint32_t *inds, float *scores,
                        hipStream_t stream) {
    if (rows < 0 || experts <= 0 || experts > 1024 || k <= 0 || k > 32 || k > experts)
        return fail(EXL3_ERR_BAD_SHAPE, "route_topk: rows=%d experts=%d k=%d (experts <= 1024, k <= 32)", rows, experts,
                    k);
    if (rows == 0) return ok();
    if (!logits || !inds || !scores) return fail(EXL3_ERR_BAD_SHAPE, "route_topk: null operand");
    return launched(run_route_topk(logits, rows, experts, k, inds, scores, stream), "exl3_route_topk");
}

int32_t exl3_tile_major(const uint16_t *src, uint16_t *dst, int32_t experts, int32_t it, int32_t ot, int32_t n,
                        int32_t inverse, hipStream_t stream) {
    if (experts < 0 || it < 0 || ot < 0 || ot % 2 || n <= 0)
        return fail(EXL3_ERR_BAD_SHAPE, "tile_major: experts=%d it=%d ot=%d n=%d (ot even)", experts, it, ot, n);
    if (experts == 0 || it == 0 || ot == 0) return ok();
    if (!src || !dst || src == dst) return fail(EXL3_ERR_BAD_SHAPE, "tile_major: null or aliased operand");
    return launched(run_tile_major(src, dst, experts, it, ot, n, inverse, stream), "exl3_tile_major");
}

// ---- Trellis encoder search ------------------------------------------------------------------------------------

namespace {

struct EncodePlan {
    int w, stride, tiles_per_wg, grid_max;
    size_t per_wg;
};

// Encoder.init (src/encoder/encode.zig:120-160): the searchable codebooks (MCG, MUL1; 3INST as this build's
// extension), an admitted rate, a window of 12..16 bits wider than every step's fresh bits.
int32_t encode_plan(int32_t n, const exl3_decode_t &dec, int64_t count, EncodePlan *p) {
    if (dec.codebook != EXL3_CB_MCG && dec.codebook != EXL3_CB_MUL1 && dec.codebook != EXL3_CB_3INST)
        return fail(EXL3_ERR_CODEBOOK_UNSUPPORTED, "encode: codebook %d is not searchable (MCG, MUL1, 3INST)",
                    dec.codebook);
    if (!rate_admitted(n)) return fail(EXL3_ERR_RATE_UNSUPPORTED, "encode: n=%d is not an admitted rate", n);
    if (dec.window_bits < 12 || dec.window_bits > 16)
        return fail(EXL3_ERR_WINDOW, "encode: window %d is outside 12..16", dec.window_bits);
    if (count < 0) return fail(EXL3_ERR_BAD_SHAPE, "encode: negative tile count");
    int kmin = 31, kmax = 0;
    for (int t = 0; t < 256; t++) {
        const int k = (((t + 1) * n) >> 4) - ((t * n) >> 4);
        kmin = k < kmin ? k : kmin;
        kmax = k > kmax ? k : kmax;
    }
    if (kmax >= dec.window_bits)
        return fail(EXL3_ERR_WINDOW_TOO_NARROW, "encode: window %d carries no state at n=%d", dec.window_bits, n);
    p->w = dec.window_bits;
    p->stride = 1 << (p->w - kmin);
    // Tiles per workgroup: as many as keep the workgroup's LDS within about half a CU's 160 KB.
    p->tiles_per_wg = 1;
    for (int t = 16; t >= 2; t >>= 1)
        if (encode_lds_bytes(t, p->stride) <= 78 * 1024) { p->tiles_per_wg = t; break; }
    // A small batch (the quantizer's 16-row groups, the global scale's samples) spreads over the CUs first: fewer
    // tiles per workgroup until there is a workgroup per CU.
    while (p->tiles_per_wg > 1 && (count + p->tiles_per_wg - 1) / p->tiles_per_wg < 256) p->tiles_per_wg >>= 1;
    const size_t lds = encode_lds_bytes(p->tiles_per_wg, p->stride);
    int per_cu = (int)((160 * 1024) / lds);
    per_cu = per_cu < 1 ? 1 : per_cu > 4 ? 4 : per_cu;
    const int64_t batches = (count + p->tiles_per_wg - 1) / p->tiles_per_wg;
    const int64_t cap = 256LL * per_cu;
    p->grid_max = (int)(batches < cap ? batches : cap);
    p->per_wg = (size_t)p->tiles_per_wg * 256 * p->stride;
    return ok();
}

EncodeTuning tuning_of(const EncodePlan &p) { return EncodeTuning{p.stride, p.tiles_per_wg, p.grid_max, p.per_wg}; }

// quantizeTensor's admission (quantize.zig:118-127, :600-606) and the two search shapes it launches.
int32_t quantize_plan(int32_t in, int32_t out, int32_t n, const exl3_decode_t &dec, int32_t mode, EncodeTuning *tg,
                      EncodeTuning *tr) {
    if (in <= 0 || out <= 0) return fail(EXL3_ERR_BAD_SHAPE, "quantize: empty tensor %dx%d", in, out);
    if (in % 128 || out % 128)
        return fail(EXL3_ERR_BAD_SHAPE, "quantize: %dx%d is off the 128 grid (GeometryUnsupported)", in, out);
    if (mode < 0 || mode > 2) return fail(EXL3_ERR_BAD_SHAPE, "quantize: out_scales mode %d (0 auto, 1 always, 2 never)", mode);
    EncodePlan pg, pr;
    int32_t rc = encode_plan(n, dec, 128, &pg);
    if (rc) return rc;
    rc = encode_plan(n, dec, out / 16, &pr);
    if (rc) return rc;
    *tg = tuning_of(pg);
    *tr = tuning_of(pr);
    return ok();
}

}  // namespace

size_t exl3_encode_workspace_size(int32_t n, exl3_decode_t dec, int64_t count) {
    EncodePlan p;
    if (encode_plan(n, dec, count, &p) != EXL3_OK) return 0;
    return (size_t)p.grid_max * p.per_wg;
}

int32_t exl3_encode_tiles(const float *tiles, int64_t count, int32_t n, exl3_decode_t dec, uint16_t *packed,
                          double *sse, void *workspace, size_t workspace_bytes, hipStream_t stream) {
    EncodePlan p;
    int32_t rc = encode_plan(n, dec, count, &p);
    if (rc) return rc;
    if (count == 0) return ok();
    if (!tiles || !packed) return fail(EXL3_ERR_BAD_SHAPE, "encode: null operand");
    const size_t fit = workspace ? workspace_bytes / p.per_wg : 0;
    if (fit < 1)
        return fail(EXL3_ERR_WORKSPACE, "encode: workspace of %zu bytes holds no search (%zu per workgroup)",
                    workspace_bytes, p.per_wg);
    int fam;
    DecodeK k;
    rc = resolve_decode(dec, n, &fam, &k);
    if (rc) return rc;
    EncodeArgs a;
    a.tiles = tiles;
    a.count = count;
    a.n = n;
    a.w = p.w;
    a.k = k;
    a.packed = packed;
    a.sse = sse;
    a.recon = nullptr;
    a.back = static_cast<uint8_t *>(workspace);
    a.stride = p.stride;
    a.tiles_per_wg = p.tiles_per_wg;
    a.grid = (int)((size_t)p.grid_max < fit ? (size_t)p.grid_max : fit);
    return launched(run_encode(fam, a, stream), "exl3_encode_tiles");
}

size_t exl3_quantize_workspace_size(int32_t in, int32_t out, int32_t n, exl3_decode_t dec) {
    EncodeTuning tg, tr;
    if (quantize_plan(in, out, n, dec, 0, &tg, &tr) != EXL3_OK) return 0;
    return quantize_workspace_bytes(in, out, tg, tr);
}

int32_t exl3_quantize_tensor(const float *w, const float *h, int32_t in, int32_t out, const float *sign_in,
                             const float *sign_out, int32_t n, exl3_decode_t dec, int32_t out_scales, uint16_t *packed,
                             uint16_t *suh, uint16_t *svh, float *g, void *workspace, size_t workspace_bytes,
                             hipStream_t stream) {
    EncodeTuning tg, tr;
    int32_t rc = quantize_plan(in, out, n, dec, out_scales, &tg, &tr);
    if (rc) return rc;
    if (!w || !h || !sign_in || !sign_out || !packed || !suh || !svh || !g)
        return fail(EXL3_ERR_BAD_SHAPE, "quantize: null operand");
    if (!workspace || workspace_bytes < quantize_workspace_bytes(in, out, tg, tr))
        return fail(EXL3_ERR_WORKSPACE, "quantize: workspace of %zu bytes, %zu needed", workspace_bytes,
                    quantize_workspace_bytes(in, out, tg, tr));
    int fam;
    DecodeK k;
    rc = resolve_decode(dec, n, &fam, &k);
    if (rc) return rc;
    QuantArgs q{};
    q.w = w;
    q.h = h;
    q.sign_in = sign_in;
    q.sign_out = sign_out;
    q.in = in;
    q.out = out;
    q.n = n;
    q.w_bits = dec.window_bits;
    q.mode = out_scales;
    q.fam = fam;
    q.k = k;
    q.tune_g = tg;
    q.tune_rows = tr;
    q.packed = packed;
    q.suh = suh;
    q.svh = svh;
    q.g = g;
    q.workspace = workspace;
    q.workspace_bytes = workspace_bytes;
    q.stream = stream;
    std::string msg;
    switch (quantize_tensor(q, &msg)) {
    case QUANT_OK: return ok();
    case QUANT_HESSIAN: return fail(EXL3_ERR_HESSIAN, "quantize: %s (HessianNotPositiveDefinite)", msg.c_str());
    case QUANT_WORKSPACE: return fail(EXL3_ERR_WORKSPACE, "quantize: %s", msg.c_str());
    default: return fail(EXL3_ERR_LAUNCH, "quantize: %s", msg.c_str());
    }
}

}  // extern "C"
