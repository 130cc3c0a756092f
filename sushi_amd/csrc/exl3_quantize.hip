// Whole-tensor trellis quantizer: src/encoder/quantize.zig `quantizeTensor` (:600-626) on the host and the GPU.
//
// The host runs what is small or inherently ordered: the regularization into the Hadamard basis (:129-189), the
// rotated Hessian in f64 (:192-207), its damped, blocked Cholesky (:225-287, the trailing update spread over host
// threads, each element keeping the reference's four-lane dot order) and the 16-column block LDL factor
// (:305-378).  The GPU runs the searches: the global scale's golden section (:400-483) scores its sample tiles with
// the encoder kernel, and the reverse LDLQ (:485-540) keeps inner, reconstruction, factor and feedback resident in
// device memory, builds each 16-row group's compensated tiles, searches them, and carries each finished 128-row
// chunk's error to every row above -- every element summed in the reference's order, so the codes are its codes.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "exl3_kernels.h"

#pragma clang fp contract(off)

namespace exl3 {

namespace {

constexpr int HAD = 128;
constexpr float SIGMA_REG = 0.025f;
constexpr float CODEBOOK_SCALE = 1.24371088f;

// ---- device: reverse LDLQ -------------------------------------------------------------------------------------

// One 16-row group's compensated rows, written as row-major 16x16 tiles [cols/16][256]:
// comp = prod + sum over the chunk's rows m below the group of l[m][row] * (inner[m] - rec[m]), then inner + comp.
__global__ void ldlq_comp_kernel(const float *__restrict__ inner, const float *__restrict__ rec,
                                 const float *__restrict__ prod, const float *__restrict__ l, int rows, int cols,
                                 int i, int bi, int bj, int chunk, float *__restrict__ tiles) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int r = blockIdx.y;
    if (c >= cols) return;
    const int row = i + bi + r;
    float acc = prod[(size_t)row * cols + c];
    for (int m = bj; m < chunk; m++) {
        const size_t src = (size_t)(i + m) * cols + c;
        const float e = inner[src] - rec[src];
        acc += l[(size_t)(i + m) * rows + row] * e;
    }
    acc = inner[(size_t)row * cols + c] + acc;
    tiles[(size_t)(c >> 4) * 256 + r * 16 + (c & 15)] = acc;
}

// The searched group's reconstruction back into rec.
__global__ void ldlq_scatter_kernel(const float *__restrict__ recon, int cols, int row0, float *__restrict__ rec) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int r = blockIdx.y;
    if (c >= cols) return;
    rec[(size_t)(row0 + r) * cols + c] = recon[(size_t)(c >> 4) * 256 + r * 16 + (c & 15)];
}

// A finished chunk's error into every row above it: prod[r] += l[i + m][r] * (inner[i + m] - rec[i + m]), m in order.
__global__ void ldlq_prod_kernel(const float *__restrict__ inner, const float *__restrict__ rec,
                                 const float *__restrict__ l, int rows, int cols, int i, int chunk,
                                 float *__restrict__ prod) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int r = blockIdx.y;
    if (c >= cols) return;
    float acc = prod[(size_t)r * cols + c];
    for (int m = 0; m < chunk; m++) {
        const size_t src = (size_t)(i + m) * cols + c;
        const float e = inner[src] - rec[src];
        acc += l[(size_t)(i + m) * rows + r] * e;
    }
    prod[(size_t)r * cols + c] = acc;
}

// ---- host: regularize, rotated Hessian, factor -----------------------------------------------------------------

template <typename T>
void fwht(T *v, size_t step) {
    for (size_t h = 1; h < HAD; h *= 2)
        for (size_t i = 0; i < HAD; i += 2 * h)
            for (size_t j = i; j < i + h; j++) {
                const T a = v[j * step], b = v[(j + h) * step];
                v[j * step] = a + b;
                v[(j + h) * step] = a - b;
            }
    const T scale = T(1) / std::sqrt(T(HAD));
    for (size_t k = 0; k < HAD; k++) v[k * step] *= scale;
}

// f(i) for i in [lo, hi), interleaved over up to 16 host threads when there are at least min_count of them.
template <typename F>
void parallel_rows(size_t lo, size_t hi, F &&f, size_t min_count = 64);

// hadamardRows (quantize.zig:52-73): the FWHT down every column of each 128-row block, run as butterflies on whole
// rows so the inner loops are contiguous (each element sees the column transform's adds, subtracts and scale);
// column ranges go to host threads.
template <typename T>
void hadamard_down(T *m, size_t rows, size_t cols) {
    const size_t span = 256;
    parallel_rows(0, (cols + span - 1) / span, [&](size_t piece) {
        const size_t c0 = piece * span, c1 = std::min(cols, c0 + span);
        const T scale = T(1) / std::sqrt(T(HAD));
        for (size_t b = 0; b < rows; b += HAD) {
            T *blk = m + b * cols;
            for (size_t h = 1; h < HAD; h *= 2)
                for (size_t i = 0; i < HAD; i += 2 * h)
                    for (size_t j = i; j < i + h; j++) {
                        T *x = blk + j * cols, *y = blk + (j + h) * cols;
                        for (size_t c = c0; c < c1; c++) {
                            const T a = x[c], d = y[c];
                            x[c] = a + d;
                            y[c] = a - d;
                        }
                    }
            for (size_t r = 0; r < HAD; r++)
                for (size_t c = c0; c < c1; c++) blk[r * cols + c] *= scale;
        }
    }, 1);
}

// hadamardCols (quantize.zig:75-85): the FWHT along each row's 128-column blocks, rows over host threads.
template <typename T>
void hadamard_along(T *m, size_t rows, size_t cols) {
    parallel_rows(0, rows, [&](size_t r) {
        for (size_t b = 0; b < cols; b += HAD) fwht<T>(m + r * cols + b, 1);
    });
}

// chooseApplyOutScales (quantize.zig:88-116); mode 0 auto, 1 always, 2 never.
bool apply_out_scales(int mode, const std::vector<float> &hdiag) {
    const int forced = mode == 1 ? 1 : mode == 2 ? 0 : -1;
    double sum = 0;
    for (float v : hdiag) sum += std::max(v, 0.0f);
    const double mean = sum / (double)hdiag.size();
    if (!std::isfinite(mean) || mean < 1e-20) return forced >= 0 ? forced : false;
    if (forced >= 0) return forced;
    const float damp = (float)((double)SIGMA_REG * mean);
    std::vector<float> diag(hdiag.size());
    for (size_t i = 0; i < hdiag.size(); i++) diag[i] = std::sqrt(std::max(hdiag[i], 0.0f) + damp);
    std::sort(diag.begin(), diag.end(), [](float a, float b) { return a > b; });
    const size_t cutoff = std::max<size_t>(1, diag.size() / 50);
    double top = 0, all = 0;
    for (size_t i = 0; i < diag.size(); i++) {
        if (i < cutoff) top += diag[i];
        all += diag[i];
    }
    return top / all < 0.15;
}

// regularize (quantize.zig:129-189).
void regularize(const float *w, size_t in, size_t out, const float *sign_in, const float *sign_out, int mode,
                const std::vector<float> &hdiag, std::vector<float> &inner, std::vector<float> &suh,
                std::vector<float> &svh) {
    inner.assign(w, w + in * out);
    svh.assign(sign_out, sign_out + out);
    suh.assign(in, 0.0f);
    std::vector<float> os(out, 0.0f);
    bool apply = apply_out_scales(mode, hdiag);
    {
        std::vector<float> total(out, 0.0f), block(out);
        for (size_t r0 = 0; r0 < in; r0 += 32) {
            std::fill(block.begin(), block.end(), 0.0f);
            for (size_t r = r0; r < std::min(r0 + 32, in); r++)
                for (size_t c = 0; c < out; c++) block[c] += inner[r * out + c] * inner[r * out + c];
            for (size_t c = 0; c < out; c++) total[c] += block[c];
        }
        for (size_t c = 0; c < out; c++) os[c] = std::sqrt(total[c] / (float)in);
    }
    double mean_sum = 0;
    for (float v : os) mean_sum += v;
    const double out_mean = mean_sum / (double)out;
    if (out_mean <= 1e-30) {
        std::fill(os.begin(), os.end(), 0.0f);
        if (mode != 0) apply = true;
    } else {
        const float m = (float)out_mean;
        for (float &v : os) v /= m;
    }
    if (apply)
        for (size_t c = 0; c < out; c++) svh[c] = svh[c] * (std::fabs(os[c]) < 1e-30f ? 0.1f : os[c]) + 1e-10f;
    for (size_t r = 0; r < in; r++)
        for (size_t c = 0; c < out; c++) inner[r * out + c] /= svh[c];
    for (size_t c = 0; c < out; c++)
        if (std::fabs(os[c]) < 1e-30f) svh[c] = 0;
    hadamard_along<float>(inner.data(), in, out);
    for (size_t r = 0; r < in; r++) {
        float total = 0;
        for (size_t c0 = 0; c0 < out; c0 += 32) {
            float block = 0;
            for (size_t c = c0; c < std::min(c0 + 32, out); c++) block += inner[r * out + c] * inner[r * out + c];
            total += block;
        }
        float in_scale = std::sqrt(total / (float)out);
        if (std::fabs(in_scale) < 1e-30f) in_scale = 0.1f;
        suh[r] = sign_in[r] * in_scale / -CODEBOOK_SCALE + 1e-10f;
    }
    for (size_t r = 0; r < in; r++)
        for (size_t c = 0; c < out; c++) inner[r * out + c] /= suh[r];
    hadamard_down<float>(inner.data(), in, out);
}

// rotatedHessian (quantize.zig:192-207).
void rotated_hessian(const float *h, const std::vector<float> &suh, size_t n, std::vector<float> &out) {
    std::vector<double> m(n * n);
    for (size_t i = 0; i < n; i++)
        for (size_t j = 0; j < n; j++) m[i * n + j] = (double)h[i * n + j] * (double)suh[i] * (double)suh[j];
    hadamard_down<double>(m.data(), n, n);
    hadamard_along<double>(m.data(), n, n);
    out.resize(n * n);
    for (size_t i = 0; i < n * n; i++) out[i] = (float)m[i];
}

// dotRows (quantize.zig:212-223): four lanes over whole quads, the lanes reduced 0..3 in order, then the tail.
inline double dot_rows(const double *a, const double *b, size_t len) {
    double acc0 = 0, acc1 = 0, acc2 = 0, acc3 = 0;
    size_t m = 0;
    for (; m + 4 <= len; m += 4) {
        acc0 += a[m] * b[m];
        acc1 += a[m + 1] * b[m + 1];
        acc2 += a[m + 2] * b[m + 2];
        acc3 += a[m + 3] * b[m + 3];
    }
    double sum = ((acc0 + acc1) + acc2) + acc3;
    for (; m < len; m++) sum += a[m] * b[m];
    return sum;
}

template <typename F>
void parallel_rows(size_t lo, size_t hi, F &&f, size_t min_count) {
    const size_t count = hi > lo ? hi - lo : 0;
    unsigned threads = std::min<unsigned>(16, std::max(1u, std::thread::hardware_concurrency()));
    if (count < min_count || count < 2 || threads == 1) {
        for (size_t i = lo; i < hi; i++) f(i);
        return;
    }
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < threads; t++)
        pool.emplace_back([&, t] {
            for (size_t i = lo + t; i < hi; i += threads) f(i);
        });
    for (auto &th : pool) th.join();
}

// choleskyLower (quantize.zig:225-287): 0, or the 1-based index of the first pivot that is not positive.
size_t cholesky_lower(std::vector<double> &a, size_t n) {
    for (size_t k = 0; k < n; k += 64) {
        const size_t kb = std::min<size_t>(64, n - k);
        for (size_t j = 0; j < kb; j++) {
            const size_t jj = k + j;
            const double d = a[jj * n + jj] - dot_rows(&a[jj * n + k], &a[jj * n + k], j);
            if (!(d > 0)) return jj + 1;
            const double root = std::sqrt(d);
            a[jj * n + jj] = root;
            for (size_t i = j + 1; i < kb; i++) {
                const size_t ii = k + i;
                a[ii * n + jj] = (a[ii * n + jj] - dot_rows(&a[ii * n + k], &a[jj * n + k], j)) / root;
            }
        }
        parallel_rows(k + kb, n, [&](size_t i) {
            for (size_t j = 0; j < kb; j++) {
                const size_t jj = k + j;
                a[i * n + jj] = (a[i * n + jj] - dot_rows(&a[i * n + k], &a[jj * n + k], j)) / a[jj * n + jj];
            }
        });
        parallel_rows(k + kb, n, [&](size_t i) {
            for (size_t j = k + kb; j <= i; j++) a[i * n + j] -= dot_rows(&a[i * n + k], &a[j * n + k], kb);
        });
    }
    return 0;
}

bool invert_lower16(double *blk) {
    double inv[256] = {};
    for (int c = 0; c < 16; c++) {
        const double d = blk[c * 16 + c];
        if (d == 0 || !std::isfinite(d)) return false;
        inv[c * 16 + c] = 1.0 / d;
        for (int r = c + 1; r < 16; r++) {
            double sum = 0;
            for (int m = c; m < r; m++) sum += blk[r * 16 + m] * inv[m * 16 + c];
            inv[r * 16 + c] = -sum / blk[r * 16 + r];
        }
    }
    std::memcpy(blk, inv, sizeof(inv));
    return true;
}

// ldlFactor (quantize.zig:305-378): false when the Hessian is not positive definite after the retries.
bool ldl_factor(std::vector<float> h, size_t n, std::vector<float> &l) {
    double diag_sum = 0;
    for (size_t i = 0; i < n; i++) {
        if (h[i * n + i] == 0) h[i * n + i] = 1;
        diag_sum += h[i * n + i];
    }
    const double diag_mean = diag_sum / (double)n;
    if (diag_mean > 0) {
        const float damp = (float)((double)SIGMA_REG * diag_mean);
        for (size_t i = 0; i < n; i++) h[i * n + i] += damp;
    }
    double damped_sum = 0;
    for (size_t i = 0; i < n; i++) damped_sum += h[i * n + i];
    const double damped_mean = damped_sum / (double)n;
    std::vector<double> c64(n * n);
    for (int retries = 0;; retries++) {
        for (size_t i = 0; i < n * n; i++) c64[i] = h[i];
        if (cholesky_lower(c64, n) == 0) break;
        if (retries + 1 > 10 || damped_mean <= 0) return false;
        const float bump = (float)(2.0 * (double)SIGMA_REG * damped_mean);
        for (size_t i = 0; i < n; i++) h[i * n + i] += bump;
    }
    std::vector<float> chol(n * n);
    for (size_t i = 0; i < n; i++)
        for (size_t j = 0; j < n; j++) chol[i * n + j] = j <= i ? (float)c64[i * n + j] : 0.0f;
    l = chol;
    for (size_t c0 = 0; c0 < n; c0 += 16) {
        double blk[256];
        float inv[256];
        for (int i = 0; i < 16; i++)
            for (int j = 0; j < 16; j++) blk[i * 16 + j] = j <= i ? chol[(c0 + i) * n + c0 + j] : 0.0;
        if (!invert_lower16(blk)) return false;
        for (int i = 0; i < 16; i++)
            for (int j = 0; j < 16; j++) inv[i * 16 + j] = j <= i ? (float)blk[i * 16 + j] : 0.0f;
        parallel_rows(c0 + 16, n, [&](size_t r) {
            for (int x = 0; x < 16; x++) {
                float acc = 0;
                for (int m = 0; m < 16; m++) acc += chol[r * n + c0 + m] * inv[m * 16 + x];
                l[r * n + c0 + x] = acc;
            }
        });
        for (int i = 0; i < 16; i++) std::fill(l.begin() + (c0 + i) * n + c0, l.begin() + (c0 + i) * n + c0 + 16, 0.0f);
    }
    return true;
}

// f32 -> f16 bits, round to nearest even (the reference's f32ToF16Bits, expert_exl3.zig:263-265).
uint16_t f16_bits(float v) {
    const _Float16 h = (_Float16)v;
    uint16_t bits;
    std::memcpy(&bits, &h, 2);
    return bits;
}

struct Dev {
    float *inner, *rec, *prod, *l, *tiles, *recon;
    uint16_t *packed;
    uint8_t *back;
    size_t back_bytes;
};

hipError_t search(int fam, const DecodeK &k, int n, int w, const EncodeTuning &tune, const float *tiles,
                  int64_t count, uint16_t *packed, float *recon, const Dev &d, hipStream_t s) {
    EncodeArgs a{};
    a.tiles = tiles;
    a.count = count;
    a.n = n;
    a.w = w;
    a.k = k;
    a.packed = packed;
    a.sse = nullptr;
    a.recon = recon;
    a.back = d.back;
    a.stride = tune.stride;
    a.tiles_per_wg = tune.tiles_per_wg;
    const int64_t batches = (count + tune.tiles_per_wg - 1) / tune.tiles_per_wg;
    const int64_t fit = (int64_t)(d.back_bytes / tune.per_wg);
    a.grid = (int)std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(batches, fit), tune.grid_cap));
    return run_encode(fam, a, s);
}

#define HIP_TRY(expr)                                  \
    do {                                               \
        hipError_t e_ = (expr);                        \
        if (e_ != hipSuccess) return set(QUANT_LAUNCH, hipGetErrorString(e_)); \
    } while (0)

}  // namespace

size_t quantize_workspace_bytes(int in, int out, const EncodeTuning &tune_g, const EncodeTuning &tune_rows) {
    const size_t io = (size_t)in * out;
    const size_t tile_count = std::max<size_t>(out / 16, 128);
    const size_t back = std::max(tune_g.per_wg * (size_t)tune_g.grid_cap, tune_rows.per_wg * (size_t)tune_rows.grid_cap);
    auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
    return up(io * 4) * 3 + up((size_t)in * in * 4) + up(tile_count * 256 * 4) * 2 + up((size_t)in / 16 * (out / 16) * 256 * 2) +
           up(back);
}

int quantize_tensor(const QuantArgs &q, std::string *msg) {
    auto set = [&](int code, const std::string &m) {
        *msg = m;
        return code;
    };
    const size_t in = q.in, out = q.out;
    const size_t out_tiles = out / 16;
    // Carve the workspace.
    auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
    char *p = static_cast<char *>(q.workspace);
    Dev d{};
    d.inner = reinterpret_cast<float *>(p), p += up(in * out * 4);
    d.rec = reinterpret_cast<float *>(p), p += up(in * out * 4);
    d.prod = reinterpret_cast<float *>(p), p += up(in * out * 4);
    d.l = reinterpret_cast<float *>(p), p += up(in * in * 4);
    const size_t tile_count = std::max<size_t>(out_tiles, 128);
    d.tiles = reinterpret_cast<float *>(p), p += up(tile_count * 256 * 4);
    d.recon = reinterpret_cast<float *>(p), p += up(tile_count * 256 * 4);
    d.packed = reinterpret_cast<uint16_t *>(p), p += up(in / 16 * out_tiles * 256 * 2);
    d.back = reinterpret_cast<uint8_t *>(p);
    const size_t used = (size_t)(p - static_cast<char *>(q.workspace));
    if (used > q.workspace_bytes) return set(QUANT_WORKSPACE, "workspace too small");
    d.back_bytes = q.workspace_bytes - used;
    if (d.back_bytes < q.tune_g.per_wg || d.back_bytes < q.tune_rows.per_wg)
        return set(QUANT_WORKSPACE, "workspace leaves no room for a search");

    // Host: regularize, rotated Hessian, LDL factor.
    std::vector<float> hdiag(in);
    for (size_t i = 0; i < in; i++) hdiag[i] = q.h[i * in + i];
    std::vector<float> inner, suh, svh, rot, l;
    regularize(q.w, in, out, q.sign_in, q.sign_out, q.mode, hdiag, inner, suh, svh);
    rotated_hessian(q.h, suh, in, rot);
    if (!ldl_factor(rot, in, l)) return set(QUANT_HESSIAN, "the Hessian is not positive definite");

    // Global scale: golden section, each point a GPU search of the sample tiles.
    const size_t tk = in / 16, tn = out / 16;
    const size_t pair_count = std::max(tk, tn) * 3;
    const size_t stride = std::max<size_t>(1, pair_count / 128);
    std::vector<float> samples;
    for (size_t pp = 0; pp < pair_count && samples.size() < 128 * 256; pp += stride) {
        const size_t i = pp / 3, wv = pp % 3;
        const size_t r0 = (i % tk) * 16, c0 = ((i + wv) % tn) * 16;
        for (int r = 0; r < 16; r++)
            samples.insert(samples.end(), inner.begin() + (r0 + r) * out + c0, inner.begin() + (r0 + r) * out + c0 + 16);
    }
    const size_t count = samples.size() / 256;
    std::vector<float> scaled(samples.size()), recon(samples.size());
    int err_code = 0;
    auto score = [&](float g) -> double {
        for (size_t v = 0; v < samples.size(); v++) scaled[v] = samples[v] * g;
        hipError_t e = hipMemcpyAsync(d.tiles, scaled.data(), scaled.size() * 4, hipMemcpyHostToDevice, q.stream);
        if (e == hipSuccess) e = search(q.fam, q.k, q.n, q.w_bits, q.tune_g, d.tiles, (int64_t)count, d.packed, d.recon, d, q.stream);
        if (e == hipSuccess) e = hipMemcpyAsync(recon.data(), d.recon, recon.size() * 4, hipMemcpyDeviceToHost, q.stream);
        if (e == hipSuccess) e = hipStreamSynchronize(q.stream);
        if (e != hipSuccess) {
            err_code = QUANT_LAUNCH;
            *msg = hipGetErrorString(e);
            return 0.0;
        }
        double sse = 0;
        for (size_t v = 0; v < samples.size(); v++) {
            const float dd = recon[v] / g - samples[v];
            sse += (double)(dd * dd);
        }
        return sse / (double)(count * 256);
    };
    const double resphi64 = 2.0 - (1.0 + std::sqrt(5.0)) / 2.0;
    const float resphi = (float)resphi64;
    const float lo = q.fam == FAM_MUL1 ? 0.4f : 0.5f, hi = q.fam == FAM_MUL1 ? 1.2f : 1.5f;
    float a = lo, b = hi;
    float x1 = a + resphi * (b - a);
    float x2 = b - resphi * (b - a);
    double f1 = score(x1);
    double f2 = err_code ? 0.0 : score(x2);
    double width = (double)hi - (double)lo;
    size_t steps = 0;
    while (width > 0.03 && steps < 8) {
        width *= 1.0 - resphi64;
        steps++;
    }
    for (size_t s = 0; s < steps && !err_code; s++) {
        const bool left = f1 < f2;
        const float a_n = left ? a : x1, b_n = left ? x2 : b;
        const float probe = left ? a_n + resphi * (b_n - a_n) : b_n - resphi * (b_n - a_n);
        const double fp = score(probe);
        a = a_n;
        b = b_n;
        if (left) {
            x2 = x1, f2 = f1, x1 = probe, f1 = fp;
        } else {
            x1 = x2, f1 = f2, x2 = probe, f2 = fp;
        }
    }
    if (err_code) return err_code;
    const float g = (a + b) / 2.0f;
    for (float &v : inner) v *= g;

    // Reverse LDLQ on the device.
    HIP_TRY(hipMemcpyAsync(d.inner, inner.data(), in * out * 4, hipMemcpyHostToDevice, q.stream));
    HIP_TRY(hipMemcpyAsync(d.l, l.data(), in * in * 4, hipMemcpyHostToDevice, q.stream));
    HIP_TRY(run_fill_zero(d.rec, in * out * 4, q.stream));
    HIP_TRY(run_fill_zero(d.prod, in * out * 4, q.stream));
    const dim3 blk(256);
    const unsigned gx = (unsigned)((out + 255) / 256);
    for (size_t j = in; j > 0;) {
        const size_t i = j > 128 ? j - 128 : 0;
        const size_t chunk = j - i;
        for (size_t bj = chunk; bj > 0; bj -= 16) {
            const size_t bi = bj - 16;
            hipLaunchKernelGGL(ldlq_comp_kernel, dim3(gx, 16), blk, 0, q.stream, d.inner, d.rec, d.prod, d.l, (int)in,
                               (int)out, (int)i, (int)bi, (int)bj, (int)chunk, d.tiles);
            HIP_TRY(hipGetLastError());
            const size_t tkk = (i + bi) / 16;
            HIP_TRY(search(q.fam, q.k, q.n, q.w_bits, q.tune_rows, d.tiles, (int64_t)out_tiles,
                           d.packed + tkk * out_tiles * q.n, d.recon, d, q.stream));
            hipLaunchKernelGGL(ldlq_scatter_kernel, dim3(gx, 16), blk, 0, q.stream, d.recon, (int)out, (int)(i + bi),
                               d.rec);
            HIP_TRY(hipGetLastError());
        }
        if (i > 0) {
            hipLaunchKernelGGL(ldlq_prod_kernel, dim3(gx, (unsigned)i), blk, 0, q.stream, d.inner, d.rec, d.l, (int)in,
                               (int)out, (int)i, (int)chunk, d.prod);
            HIP_TRY(hipGetLastError());
        }
        j = i;
    }
    HIP_TRY(hipMemcpyAsync(q.packed, d.packed, in / 16 * out_tiles * q.n * 2, hipMemcpyDeviceToHost, q.stream));
    HIP_TRY(hipStreamSynchronize(q.stream));
    for (size_t i = 0; i < in; i++) q.suh[i] = f16_bits(suh[i] / g);
    for (size_t i = 0; i < out; i++) q.svh[i] = f16_bits(svh[i]);
    *q.g = g;
    return 0;
}

}  // namespace exl3
