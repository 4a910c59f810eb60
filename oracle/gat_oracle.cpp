// CPU oracle for the three-layer multi-head GAT forward (TEST INFRASTRUCTURE).
//
// This library is the checker and the CPU baseline, never the product: only
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
// Every function restates the reference algorithm it cites (paths relative to
// the reference root).  It is compiled with g++ so that libstdc++'s mt19937 and
// normal/uniform distributions reproduce the reference's random weights.
//
// How each function is pinned (tests/test_oracle.py):
//   or_rne                 torch bfloat16 RNE on 2^20 random patterns, the ties of
//                          baseline/tests/boundaries.cpp:25-26, NaN quieting
//   or_random_param        errors of the reference's correctness log reproduced
//                          (baseline/runs/check-10808045/correctness.log); bitwise
//                          equality with the reference's files is parity unpinned:
//                          its icpx/libimf logf differs from glibc in the last ulp
//   or_boundary_*          same log; the feature bits (sinf) likewise parity unpinned
//   or_ref_layer (R0)      FP64 oracle < 1e-4 on 64 shapes, NumPy FP64 chain < 2e-4,
//                          smoke1024 checksum 221.971286 (+-1e-3), the logged errors
//   or_fp64_layer          NumPy FP64 restatement of baseline/tests/oracle.py (1e-9)
//   or_fixed_p_layer       fed R0's own p and den it reproduces R0's output (1e-6);
//                          a hand-computed three-node case
//   or_b1_layer            with weights p whose products p x round exactly in bf16 it
//                          equals or_fixed_p_layer on bf16 inputs bit for bit; a
//                          hand-computed case where the bf16 rounding of p x shows
//   or_standard_layer (B0) the logged standard_bf16 stage errors and chain error
//   or_degree_schedule,    numpy.lexsort on (degree, id); neighbor_steps definition;
//   or_permute_csr         row-by-row copy check
//   or_choose_R            hand-computed rho thresholds
//   or_errors              NumPy on hand-built vectors
// Bitwise parity with oneMKL's SGEMM order and SVML exp is parity unpinned
// (neither is available); both are tolerance-pinned as above.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <numeric>
#include <random>
#include <vector>
#include <omp.h>

namespace {
inline float leak(float x) { return x >= 0 ? x : 0.2f * x; }  // baseline/include/gat.hpp:52
inline float elu(float x) { return x >= 0 ? x : std::expm1(x); }  // baseline/include/gat.hpp:53

// FP32 -> BF16 round-to-nearest-even with NaN quieting: baseline/src/common.cpp:80-83.
inline uint16_t rne(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return uint16_t((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}
inline float expand(uint16_t b) {  // baseline/src/common.cpp:84
    uint32_t u = uint32_t(b) << 16;
    float x;
    std::memcpy(&x, &u, 4);
    return x;
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------- conversion
void or_rne(const float* x, uint16_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = rne(x[i]);
}

// ---------------------------------------------------------------- weights
// One layer of random_model: baseline/src/common.cpp:50-62.  The caller passes
// rng_seed = seed + 11*layer, exactly as common.cpp:55 seeds mt19937.
void or_random_param(int in, int heads, int dim, int rng_seed, float* w, float* al, float* ar) {
    std::mt19937 rng(rng_seed);
    std::normal_distribution<float> norm;
    const size_t width = size_t(heads) * dim;
    for (size_t i = 0; i < size_t(in) * width; ++i) w[i] = norm(rng) / std::sqrt(float(in));
    for (size_t i = 0; i < width; ++i) al[i] = norm(rng) / std::sqrt(float(dim));
    for (size_t i = 0; i < width; ++i) ar[i] = norm(rng) / std::sqrt(float(dim));
}
// Boundary-test parameters: baseline/tests/boundaries.cpp:8-9.
void or_boundary_param(int D, int K, int d, float* w, float* al, float* ar) {
    std::mt19937 rng(D + K + d);
    std::uniform_real_distribution<float> rnd(-.3f, .3f);
    for (size_t i = 0; i < size_t(D) * K * d; ++i) w[i] = rnd(rng);
    for (int i = 0; i < K * d; ++i) al[i] = rnd(rng);
    for (int i = 0; i < K * d; ++i) ar[i] = rnd(rng);
}
// Boundary-test features: baseline/tests/boundaries.cpp:13 (float sin).
void or_boundary_features(uint64_t count, float* x) {
    for (uint64_t i = 0; i < count; ++i) x[i] = std::sin(float(i) * .17f) * .5f;
}

// ---------------------------------------------------------------- R0 oracle
// R0 FP32 layer: baseline/src/ref_fp32.cpp:3-26.  The SGEMM is restated as a
// float dot product in ascending k (oneMKL's blocking order is not known; the
// difference is tolerance-level, pinned by the FP64 oracle below).  L/R follow
// lr_from_z(scalar=true) (baseline/src/baseline_standard.cpp:7-20).  score, p
// and alpha are [E][K]; any of them may be null.
void or_ref_layer(uint64_t n, const uint64_t* row, const uint32_t* col, const float* x, int in,
                  int heads, int dim, const float* w, const float* al, const float* ar, int hidden,
                  float* z, float* left, float* right, float* mx, float* den, float* score, float* p,
                  float* alpha, float* out) {
    const int K = heads, W = heads * dim;
    #pragma omp parallel for schedule(static)
    for (uint64_t i = 0; i < n; ++i) {
        float* zi = z + i * W;
        for (int c = 0; c < W; ++c) zi[c] = 0.0f;
        for (int k = 0; k < in; ++k) {
            const float a = x[i * in + k];
            const float* wk = w + size_t(k) * W;
            for (int c = 0; c < W; ++c) zi[c] += a * wk[c];
        }
        for (int h = 0; h < K; ++h) {
            float l = 0, r = 0;
            for (int d = 0; d < dim; ++d) {
                l += zi[h * dim + d] * al[h * dim + d];
                r += zi[h * dim + d] * ar[h * dim + d];
            }
            left[i * K + h] = l;
            right[i * K + h] = r;
        }
    }
    #pragma omp parallel
    {
        std::vector<float> sc, pv;
        #pragma omp for schedule(dynamic, 64)
        for (uint64_t i = 0; i < n; ++i) {
            const uint64_t b = row[i], e_end = row[i + 1], deg = e_end - b;
            sc.resize(deg * K);
            pv.resize(deg * K);
            float* oi = out + i * W;
            for (int c = 0; c < W; ++c) oi[c] = 0.0f;
            for (int h = 0; h < K; ++h) {
                float m = -std::numeric_limits<float>::infinity();
                for (uint64_t e = 0; e < deg; ++e) {
                    float s = leak(left[i * K + h] + right[size_t(col[b + e]) * K + h]);
                    sc[e * K + h] = s;
                    m = std::max(m, s);
                }
                mx[i * K + h] = deg == 0 ? 0.0f : m;
                float dn = 0;
                for (uint64_t e = 0; e < deg; ++e) {
                    float v = std::exp(sc[e * K + h] - m);
                    pv[e * K + h] = v;
                    dn += v;
                }
                den[i * K + h] = dn;
                for (uint64_t e = 0; e < deg; ++e) {
                    if (score) score[(b + e) * K + h] = sc[e * K + h];
                    if (p) p[(b + e) * K + h] = pv[e * K + h];
                    if (alpha) alpha[(b + e) * K + h] = pv[e * K + h] / dn;
                }
            }
            // ref_fp32.cpp:17-21 aggregates with alpha = p/den in edge order.
            for (uint64_t e = 0; e < deg; ++e) {
                const float* zj = z + size_t(col[b + e]) * W;
                for (int h = 0; h < K; ++h) {
                    const float a = pv[e * K + h] / den[i * K + h];
                    for (int d = 0; d < dim; ++d) oi[h * dim + d] += a * zj[h * dim + d];
                }
            }
            if (hidden)
                for (int c = 0; c < W; ++c) oi[c] = elu(oi[c]);
        }
    }
}

// ---------------------------------------------------------------- FP64 oracle
// Independent FP64 layer: baseline/tests/boundaries.cpp:15-21 (scalar
// projection/attention/softmax in double) plus the ELU of
// baseline/tests/oracle.py:53-54 when hidden.  Outputs are double.
void or_fp64_layer(uint64_t n, const uint64_t* row, const uint32_t* col, const float* x, int in,
                   int heads, int dim, const float* w, const float* al, const float* ar, int hidden,
                   double* z, double* left, double* right, double* mx, double* den, double* out) {
    const int K = heads, W = heads * dim;
    #pragma omp parallel for schedule(static)
    for (uint64_t i = 0; i < n; ++i) {
        for (int h = 0; h < K; ++h) {
            double l = 0, r = 0;
            for (int d = 0; d < dim; ++d) {
                double v = 0;
                for (int k = 0; k < in; ++k) v += double(x[i * in + k]) * w[size_t(k) * W + h * dim + d];
                z[i * W + h * dim + d] = v;
                l += v * al[h * dim + d];
                r += v * ar[h * dim + d];
            }
            left[i * K + h] = l;
            right[i * K + h] = r;
        }
    }
    #pragma omp parallel
    {
        std::vector<double> sc;
        #pragma omp for schedule(dynamic, 64)
        for (uint64_t i = 0; i < n; ++i) {
            const uint64_t b = row[i], deg = row[i + 1] - b;
            for (int h = 0; h < K; ++h) {
                sc.assign(deg, 0.0);
                double m = -INFINITY, dn = 0;
                for (uint64_t e = 0; e < deg; ++e) {
                    double v = left[i * K + h] + right[size_t(col[b + e]) * K + h];
                    v = v >= 0 ? v : .2 * v;
                    sc[e] = v;
                    m = std::max(m, v);
                }
                for (auto& v : sc) {
                    v = std::exp(v - m);
                    dn += v;
                }
                mx[i * K + h] = deg ? m : 0.0;
                den[i * K + h] = dn;
                for (int d = 0; d < dim; ++d) {
                    double s = 0;
                    for (uint64_t e = 0; e < deg; ++e) s += sc[e] * z[size_t(col[b + e]) * W + h * dim + d];
                    double o = dn > 0 ? s / dn : 0.0;
                    if (hidden && o < 0) o = std::expm1(o);
                    out[i * W + h * dim + d] = o;
                }
            }
        }
    }
}

// Fixed-p operator (baseline/bench/main.cpp:103-150): projection, then
// standard_aggregate with the fixture's p and den (baseline/src/
// baseline_standard.cpp:52-84) and finish without activation (:85-97).
// bf16 != 0 rounds X and W to bf16 first and keeps Z in FP32, as the
// reference's standard_bf16 projection does (cblas_gemm_bf16bf16f32); bf16 == 0
// is the FP32 master of main.cpp:136-137.  p [e][heads], den [n][heads].
void or_fixed_p_layer(uint64_t n, const uint64_t* row, const uint32_t* col, const float* x, int in,
                      int heads, int dim, const float* w, const float* p, const float* den, int bf16,
                      float* z, float* out) {
    const int K = heads, W = heads * dim;
    std::vector<float> wq(size_t(in) * W);
    for (size_t q = 0; q < wq.size(); ++q) wq[q] = bf16 ? expand(rne(w[q])) : w[q];
    #pragma omp parallel for schedule(static)
    for (uint64_t i = 0; i < n; ++i) {
        float* zi = z + i * W;
        for (int c = 0; c < W; ++c) zi[c] = 0.0f;
        for (int k = 0; k < in; ++k) {
            const float a = bf16 ? expand(rne(x[i * in + k])) : x[i * in + k];
            const float* wk = wq.data() + size_t(k) * W;
            for (int c = 0; c < W; ++c) zi[c] += a * wk[c];
        }
    }
    #pragma omp parallel for schedule(dynamic, 64)
    for (uint64_t i = 0; i < n; ++i) {
        float* oi = out + i * W;
        for (int c = 0; c < W; ++c) oi[c] = 0.0f;
        for (uint64_t e = row[i]; e < row[i + 1]; ++e) {
            const float* zj = z + uint64_t(col[e]) * W;
            for (int h = 0; h < K; ++h) {
                const float pe = p[e * K + h];
                for (int d = 0; d < dim; ++d) oi[h * dim + d] += pe * zj[h * dim + d];
            }
        }
        for (int h = 0; h < K; ++h) {
            const float d = den[i * K + h];
            const float scale = d > 0 ? 1 / d : 0;
            for (int c = 0; c < dim; ++c) oi[h * dim + c] *= scale;
        }
    }
}

// Neighbour-step TFS with bf16 weighted rows (B1, baseline/src/baseline_tfs.cpp:
// 16-110, and the explicit emulation of baseline/bench/main.cpp:139-143):
// out[i, h, :] = sum_e sum_k expand(rne(p[e, h] * xq[col[e], k])) * wq[k, h, :],
// then / den (0 if den == 0) and ELU when hidden.  xq and wq are bf16-rounded
// values held in FP32; p [e][heads] and den [n][heads] are given (computed
// from L/R and the exact max, or a fixture's).
void or_b1_layer(uint64_t n, const uint64_t* row, const uint32_t* col, const float* xq, int in, int heads,
                 int dim, const float* wq, const float* p, const float* den, int hidden, float* out) {
    const int K = heads, W = heads * dim;
    #pragma omp parallel for schedule(dynamic, 64)
    for (uint64_t i = 0; i < n; ++i) {
        float* oi = out + i * W;
        for (int c = 0; c < W; ++c) oi[c] = 0.0f;
        for (uint64_t e = row[i]; e < row[i + 1]; ++e) {
            const float* xj = xq + uint64_t(col[e]) * in;
            for (int h = 0; h < K; ++h) {
                const float pe = p[e * K + h];
                for (int k = 0; k < in; ++k) {
                    const float v = expand(rne(pe * xj[k]));
                    const float* wk = wq + size_t(k) * W + h * dim;
                    for (int d = 0; d < dim; ++d) oi[h * dim + d] += v * wk[d];
                }
            }
        }
        for (int h = 0; h < K; ++h) {
            const float d_ = den[i * K + h];
            const float scale = d_ > 0 ? 1 / d_ : 0;
            for (int c = 0; c < dim; ++c) {
                const float y = d_ > 0 ? oi[h * dim + c] * scale : 0.0f;
                oi[h * dim + c] = hidden ? elu(y) : y;
            }
        }
    }
}

// ---------------------------------------------------------------- schedule
// degree_schedule: baseline/src/common.cpp:120-125 (perm[sorted]=original row,
// ascending (degree, id); neighbor_steps = sum over 16-row tiles of the last
// row's degree).  Same order as degree_perm in
// implementation/src/gat_tfs_online.cpp:180-189.
void or_degree_schedule(uint64_t n, const uint64_t* row, uint32_t* perm, uint64_t* neighbor_steps) {
    std::iota(perm, perm + n, 0u);
    std::sort(perm, perm + n, [&](uint32_t a, uint32_t b) {
        auto da = row[a + 1] - row[a], db = row[b + 1] - row[b];
        return da != db ? da < db : a < b;
    });
    uint64_t steps = 0;
    for (uint64_t base = 0; base < n; base += 16) {
        uint32_t r = perm[std::min<uint64_t>(n, base + 16) - 1];
        steps += row[r + 1] - row[r];
    }
    *neighbor_steps = steps;
}
// CSR in degree-sorted order: prow[k] = sum of degrees of perm[0..k),
// pcol[prow[k]..prow[k+1]) = col[row[perm[k]]..row[perm[k]+1]).
void or_permute_csr(uint64_t n, const uint64_t* row, const uint32_t* col, const uint32_t* perm,
                    uint64_t* prow, uint32_t* pcol) {
    prow[0] = 0;
    for (uint64_t k = 0; k < n; ++k) {
        const uint64_t b = row[perm[k]], deg = row[perm[k] + 1] - b;
        std::copy(col + b, col + b + deg, pcol + prow[k]);
        prow[k + 1] = prow[k] + deg;
    }
}
// choose_R: implementation/src/gat_tfs_online.cpp:191-199.
int or_choose_R(uint64_t n, uint64_t e, const uint64_t* row) {
    uint64_t maxdeg = 0;
    for (uint64_t i = 0; i < n; ++i) maxdeg = std::max(maxdeg, row[i + 1] - row[i]);
    double avg = double(e) / n, rho = avg ? maxdeg / avg : 1.0;
    if (rho < 32) return 128;
    if (rho < 1024) return 64;
    if (rho < 20000) return 32;
    return 16;
}

// ---------------------------------------------------------------- metrics
// errors(): baseline/src/common.cpp:141-150.  out = {max_abs, mean_abs,
// relative_l2, rmse, p50, p90, p99}; returns 1 if every value is finite.
int or_errors(const float* ref, const float* got, uint64_t n, double* out) {
    std::vector<double> a;
    a.reserve(n);
    double sq = 0, dsum = 0, mx = 0, mean = 0;
    bool finite = true;
    for (uint64_t i = 0; i < n; ++i) {
        if (!std::isfinite(ref[i]) || !std::isfinite(got[i])) {
            finite = false;
            continue;
        }
        double d = double(got[i]) - ref[i], v = std::abs(d);
        mx = std::max(mx, v);
        mean += v;
        sq += d * d;
        dsum += double(ref[i]) * ref[i];
        a.push_back(v);
    }
    if (!finite || n == 0) {
        for (int k = 0; k < 7; ++k) out[k] = std::numeric_limits<double>::infinity();
        return 0;
    }
    out[0] = mx;
    out[1] = mean / n;
    out[2] = dsum > 0 ? std::sqrt(sq / dsum) : (sq == 0 ? 0 : std::numeric_limits<double>::infinity());
    out[3] = std::sqrt(sq / n);
    auto pct = [&](double q) {
        size_t k = std::min(a.size() - 1, size_t(std::ceil(q * a.size()) - 1));
        std::nth_element(a.begin(), a.begin() + k, a.end());
        return a[k];
    };
    out[4] = pct(.5);
    out[5] = pct(.9);
    out[6] = pct(.99);
    return 1;
}

int or_max_threads() { return omp_get_max_threads(); }
}
