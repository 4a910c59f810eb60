// B0 CPU baseline of the oracle (TEST INFRASTRUCTURE; see gat_oracle.cpp).
//
// The strong standard GAT layer of baseline/src/baseline_standard.cpp, timed
// by bench.py as the CPU baseline.  Compiled on its own with
// -fno-trapping-math so that the vector selects of exp/ELU vectorise; the
// rest of the oracle keeps default floating-point semantics (that flag changes
// the values libstdc++'s normal_distribution produces).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>
#include <omp.h>

namespace {
using Clock = std::chrono::steady_clock;
typedef float v16 __attribute__((vector_size(64)));
#ifdef __AVX512F__
constexpr int kMR = 6;  // 12 zmm accumulators
#else
constexpr int kMR = 3;  // 12 ymm accumulators (each v16 is two ymm)
#endif
double ms_since(Clock::time_point a) {
    return std::chrono::duration<double, std::milli>(Clock::now() - a).count();
}
inline float leak(float x) { return x >= 0 ? x : 0.2f * x; }  // baseline/include/gat.hpp:52
// FP32 -> BF16 round-to-nearest-even with NaN quieting: baseline/src/common.cpp:80-83.
inline uint16_t rne(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return uint16_t((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}
inline float expand(uint16_t b) {
    uint32_t u = uint32_t(b) << 16;
    float x;
    std::memcpy(&x, &u, 4);
    return x;
}

// Vectorisable exp for the CPU baseline (the reference uses icpx SVML
// _mm512_exp_ps, absent here).  Method: Cody & Waite (1980) argument
// reduction x = n*ln2 + r with ln2 split in a short-mantissa high part and a
// low part, then the degree-7 Taylor polynomial of e^r on |r| <= ln2/2
// (truncation error |r|^8/8! < 1.2e-8 relative), then scaling by 2^n through
// the exponent field.  Arguments below -87.33 return 0 (the softmax only
// evaluates x <= 0, where such values are below FP32's normal range).
inline float exp_cw(float x) {
    const bool under = x < -87.33f;  // e^x below 2^-126: returned as 0
    x = std::min(std::max(x, -87.33f), 88.7f);
    const float log2e = 1.44269504088896341f;
    const float ln2_hi = 0.693359375f;          // 0x3f318000: 9 significant bits
    const float ln2_lo = -2.12194440e-4f;       // ln2 - ln2_hi
    const float shifter = 12582912.0f;          // 1.5 * 2^23: adding it rounds to an integer
    const float n = (x * log2e + shifter) - shifter;
    float r = x - n * ln2_hi;
    r = r - n * ln2_lo;
    // Taylor coefficients 1/k!, k = 7..0, Horner form.
    float p = 1.0f / 5040.0f;
    p = p * r + 1.0f / 720.0f;
    p = p * r + 1.0f / 120.0f;
    p = p * r + 1.0f / 24.0f;
    p = p * r + 1.0f / 6.0f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    const int32_t e = int32_t(n) + 127;  // >= 1 after the clamp: always a normal power of two
    const uint32_t bits = uint32_t(e) << 23;
    float sc;
    std::memcpy(&sc, &bits, 4);
    return under ? 0.0f : p * sc;
}
// expm1 for x < 0 (ELU branch): series for small |x| avoids cancellation.
inline float expm1_neg(float x) {
    // Taylor series of e^x - 1 to x^8/8! for |x| <= 0.25 (|x|^9/9! < 1e-11),
    // exp(x) - 1 below; both evaluated and selected so the loop vectorises.
    float p = 1.0f / 40320.0f;
    p = p * x + 1.0f / 5040.0f;
    p = p * x + 1.0f / 720.0f;
    p = p * x + 1.0f / 120.0f;
    p = p * x + 1.0f / 24.0f;
    p = p * x + 1.0f / 6.0f;
    p = p * x + 0.5f;
    p = p * x + 1.0f;
    const float series = p * x;
    return x > -0.25f ? series : exp_cw(x) - 1.0f;
}
}  // namespace

extern "C" {

float or_exp_cw(float x) { return exp_cw(x); }
float or_expm1_neg(float x) { return expm1_neg(x); }

// ---------------------------------------------------------------- B0 (CPU baseline)
// Strong standard GAT layer: baseline/src/baseline_standard.cpp:98-108 stage
// order: convert (bf16 only) -> projection -> lr_from_z -> max_prescan ->
// standard_aggregate -> finish.  bf16 != 0 is the standard_bf16 semantics
// (RNE X and W, FP32 accumulate, FP32 Z and softmax state); bf16 == 0 is
// standard_fp32.  times[7] receives convert, projection, lr, max_prescan,
// aggregate, finish, total in milliseconds.  threads <= 0 keeps OpenMP's default.
// wq (bf16 weights as FP32 values) is prepared by the caller outside the timer,
// as prepare() does in baseline/src/common.cpp:97-119.
void or_standard_layer(uint64_t n, const uint64_t* row, const uint32_t* col, const float* x, int in,
                       int heads, int dim, const float* w, const float* al, const float* ar, int hidden,
                       int bf16, int threads, float* xq_scratch, float* z, float* left, float* right,
                       float* mx, float* den, float* out, double* times) {
    if (threads > 0) omp_set_num_threads(threads);
    const int K = heads, W = heads * dim;
    // Static weight preparation outside the stage timers (prepare(),
    // common.cpp:97-119): W in 32-column panels [panel][k][32], zero-padded.
    std::vector<float> wpanel_buf(size_t((W + 31) / 32) * in * 32, 0.0f);
    for (int k = 0; k < in; ++k)
        for (int c = 0; c < W; ++c) wpanel_buf[(size_t(c / 32) * in + k) * 32 + c % 32] = w[size_t(k) * W + c];
    const float* wpanel = wpanel_buf.data();
    const float* xin = x;
    auto t0 = Clock::now(), t = t0;
    // convert: common.cpp:85-93 (the bf16 value is kept widened to FP32).
    if (bf16) {
        const uint64_t cnt = n * uint64_t(in);
        #pragma omp parallel for schedule(static)
        for (uint64_t i = 0; i < cnt; ++i) xq_scratch[i] = expand(rne(x[i]));
        xin = xq_scratch;
    }
    times[0] = ms_since(t);
    t = Clock::now();
    // projection: FP32 GEMM on the prepacked 32-column panels of W, MR rows x
    // 32 columns of accumulators per step (vector registers).  bf16 products
    // are exact in FP32, so this equals BF16xBF16->FP32 up to the
    // accumulation order.
    {
        const int panels = (W + 31) / 32;
        const uint64_t row_blocks = (n + kMR - 1) / kMR;
        #pragma omp parallel for schedule(static)
        for (uint64_t rb = 0; rb < row_blocks; ++rb) {
            const uint64_t r0 = rb * kMR;
            const int rows = int(std::min<uint64_t>(kMR, n - r0));
            const float* arow[kMR];
            for (int r = 0; r < kMR; ++r) arow[r] = xin + (r0 + std::min(r, rows - 1)) * in;
            for (int pnl = 0; pnl < panels; ++pnl) {
                const float* bp = wpanel + size_t(pnl) * in * 32;
                v16 c[kMR][2];
                for (int r = 0; r < kMR; ++r) c[r][0] = c[r][1] = v16{};
                for (int k = 0; k < in; ++k) {
                    v16 b0, b1;
                    std::memcpy(&b0, bp + size_t(k) * 32, 64);
                    std::memcpy(&b1, bp + size_t(k) * 32 + 16, 64);
                    for (int r = 0; r < kMR; ++r) {
                        const float a = arow[r][k];
                        c[r][0] += a * b0;
                        c[r][1] += a * b1;
                    }
                }
                const int c0 = pnl * 32, cols = std::min(32, W - c0);
                for (int r = 0; r < rows; ++r) {
                    float tmp[32];
                    std::memcpy(tmp, &c[r][0], 64);
                    std::memcpy(tmp + 16, &c[r][1], 64);
                    std::memcpy(z + (r0 + r) * W + c0, tmp, size_t(cols) * 4);
                }
            }
        }
    }
    times[1] = ms_since(t);
    t = Clock::now();
    // lr_from_z: baseline_standard.cpp:7-20.
    #pragma omp parallel for schedule(static)
    for (uint64_t i = 0; i < n; ++i)
        for (int h = 0; h < K; ++h) {
            float l = 0, r = 0;
            #pragma omp simd reduction(+ : l, r)
            for (int d = 0; d < dim; ++d) {
                l += z[i * W + h * dim + d] * al[h * dim + d];
                r += z[i * W + h * dim + d] * ar[h * dim + d];
            }
            left[i * K + h] = l;
            right[i * K + h] = r;
        }
    times[2] = ms_since(t);
    t = Clock::now();
    // max_prescan: baseline_standard.cpp:44-51 (exact max; empty row -> 0).
    #pragma omp parallel for schedule(dynamic, 64)
    for (uint64_t i = 0; i < n; ++i) {
        float m[8];
        for (int h = 0; h < K; ++h) m[h] = -std::numeric_limits<float>::infinity();
        for (uint64_t e = row[i]; e < row[i + 1]; ++e)
            for (int h = 0; h < K; ++h) m[h] = std::max(m[h], right[size_t(col[e]) * K + h]);
        for (int h = 0; h < K; ++h) mx[i * K + h] = row[i] == row[i + 1] ? 0.0f : leak(m[h] + left[i * K + h]);
    }
    times[3] = ms_since(t);
    t = Clock::now();
    // standard_aggregate: baseline_standard.cpp:52-84 (one owner per row,
    // unnormalised sum and FP32 denominator).
    #pragma omp parallel
    {
        std::vector<float> acc(W);
        #pragma omp for schedule(dynamic, 64)
        for (uint64_t i = 0; i < n; ++i) {
            std::fill(acc.begin(), acc.end(), 0.0f);
            float dn[8] = {}, l[8] = {}, m[8] = {}, wgt[8];
            for (int h = 0; h < K; ++h) {
                l[h] = left[i * K + h];
                m[h] = mx[i * K + h];
            }
            for (uint64_t e = row[i]; e < row[i + 1]; ++e) {
                const size_t j = col[e];
                // Software prefetch of the Z row PF edges ahead (random 1 KB
                // gathers are latency-bound on one core otherwise).
                constexpr uint64_t PF = 6;
                if (e + PF < row[i + 1]) {
                    const char* zp = reinterpret_cast<const char*>(z + size_t(col[e + PF]) * W);
                    for (int off = 0; off < W * 4; off += 64) __builtin_prefetch(zp + off);
                }
                #pragma omp simd
                for (int h = 0; h < 8; ++h) {
                    const float r = right[j * K + (h < K ? h : 0)];
                    wgt[h] = h < K ? exp_cw(leak(l[h] + r) - m[h]) : 0.0f;
                    dn[h] += wgt[h];
                }
                const float* zj = z + j * W;
                for (int h = 0; h < K; ++h) {
                    const float f = wgt[h];
                    float* a = acc.data() + h * dim;
                    const float* zz = zj + h * dim;
                    #pragma omp simd
                    for (int d = 0; d < dim; ++d) a[d] += f * zz[d];
                }
            }
            for (int h = 0; h < K; ++h) den[i * K + h] = dn[h];
            std::copy(acc.begin(), acc.end(), out + i * W);
        }
    }
    times[4] = ms_since(t);
    t = Clock::now();
    // finish: baseline_standard.cpp:85-97 (normalise, then ELU on hidden layers).
    #pragma omp parallel for schedule(static)
    for (uint64_t i = 0; i < n; ++i)
        for (int h = 0; h < K; ++h) {
            const float dn = den[i * K + h];
            const float s = dn > 0 ? 1 / dn : 0;
            float* o = out + i * W + h * dim;
            #pragma omp simd
            for (int d = 0; d < dim; ++d) {
                const float v = o[d] * s;
                o[d] = hidden ? (v < 0 ? expm1_neg(std::min(v, 0.0f)) : v) : v;
            }
        }
    times[5] = ms_since(t);
    times[6] = ms_since(t0);
}

}  // extern "C"
