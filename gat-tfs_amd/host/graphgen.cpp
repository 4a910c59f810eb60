// Seeded synthetic inputs for the GAT forward (declarations: include/gathost.h).
// All generators are counter-based (one hash per row / edge / element), so the
// output does not depend on the OpenMP thread count.
#include "gathost.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <numeric>
#include <random>
#include <vector>

#include <omp.h>

namespace {

inline uint64_t splitmix(uint64_t& s) {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
inline uint64_t mix(uint64_t a, uint64_t b) {
    uint64_t s = a * 0x9e3779b97f4a7c15ull ^ (b + 0x632be59bd9b4e019ull);
    splitmix(s);
    return splitmix(s);
}
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    uint64_t next() { return splitmix(s); }
    // Uniform in [0, m) (multiply-shift; bias below 2^-40 for the sizes used).
    uint64_t below(uint64_t m) { return uint64_t((unsigned __int128)next() * m >> 64); }
    double unit() { return double(next() >> 11) * 0x1.0p-53; }  // [0,1)
};

uint64_t prefix_rows(uint64_t n, const std::vector<uint32_t>& deg, uint64_t* row) {
    row[0] = 0;
    for (uint64_t i = 0; i < n; ++i) row[i + 1] = row[i] + deg[i];
    return row[n];
}

// k distinct values from [0, m), ascending.
void sample_distinct(Rng& rng, uint64_t m, uint64_t k, std::vector<uint32_t>& out) {
    out.clear();
    if (k == 0) return;
    if (k >= m) {
        out.resize(m);
        std::iota(out.begin(), out.end(), 0u);
        return;
    }
    if (k > m / 2) {  // draw the complement
        std::vector<uint32_t> excl;
        sample_distinct(rng, m, m - k, excl);
        out.reserve(k);
        size_t q = 0;
        for (uint64_t v = 0; v < m; ++v) {
            if (q < excl.size() && excl[q] == v) {
                ++q;
                continue;
            }
            out.push_back(uint32_t(v));
        }
        return;
    }
    while (out.size() < k) {
        const size_t need = k - out.size();
        for (size_t t = 0; t < need; ++t) out.push_back(uint32_t(rng.below(m)));
        std::sort(out.begin(), out.end());
        out.erase(std::unique(out.begin(), out.end()), out.end());
    }
}

}  // namespace

extern "C" {

uint64_t gathost_uniform_rows(uint64_t n, uint32_t mean_degree, uint64_t seed, uint64_t* row) {
    std::vector<uint32_t> deg(n);
    const uint64_t span = mean_degree > 1 ? 2ull * (mean_degree - 1) + 1 : 1;
    #pragma omp parallel for schedule(static)
    for (uint64_t i = 0; i < n; ++i) {
        Rng r(mix(seed, i));
        uint64_t extra = r.below(span);
        if (extra > n - 1) extra = n - 1;
        deg[i] = uint32_t(1 + extra);
    }
    return prefix_rows(n, deg, row);
}

uint64_t gathost_powerlaw_rows(uint64_t n, uint64_t edges, uint32_t max_degree, uint64_t seed,
                               uint64_t* row) {
    if (n == 0 || edges < n || max_degree == 0 || max_degree > n) return 0;
    const uint64_t extra_total = edges - n;
    const double target0 = double(max_degree - 1);
    std::vector<uint32_t> deg(n, 1);
    if (extra_total > 0) {
        if (target0 <= 0 || double(extra_total) > double(n) * target0) return 0;
        // sum_{r<n} (r+1)^-alpha == extra_total / target0, solved by bisection.
        const double want = double(extra_total) / target0;
        auto f = [&](double alpha) {
            double s = 0;
            #pragma omp parallel for reduction(+ : s) schedule(static)
            for (uint64_t r = 0; r < n; ++r) s += std::pow(double(r + 1), -alpha);
            return s;
        };
        double lo = 0.0, hi = 8.0;
        for (int it = 0; it < 48; ++it) {
            const double mid = 0.5 * (lo + hi);
            if (f(mid) > want) lo = mid;
            else hi = mid;
        }
        const double alpha = 0.5 * (lo + hi), total_w = f(alpha);
        // Seeded ranking of the nodes (Fisher-Yates).
        std::vector<uint32_t> node_of_rank(n);
        std::iota(node_of_rank.begin(), node_of_rank.end(), 0u);
        Rng rng(mix(seed, 0x7261'6e6bull));
        for (uint64_t r = n - 1; r > 0; --r) std::swap(node_of_rank[r], node_of_rank[rng.below(r + 1)]);
        std::vector<uint64_t> extra(n);
        std::vector<double> frac(n);
        uint64_t assigned = 0;
        for (uint64_t r = 0; r < n; ++r) {
            const double q = std::pow(double(r + 1), -alpha) / total_w * double(extra_total);
            uint64_t e = uint64_t(std::floor(q));
            if (e > n - 1) e = n - 1;
            extra[r] = e;
            frac[r] = q - std::floor(q);
            assigned += e;
        }
        std::vector<uint32_t> order(n);
        std::iota(order.begin(), order.end(), 0u);
        std::stable_sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) { return frac[a] > frac[b]; });
        for (uint64_t t = 0; assigned < extra_total && t < n; ++t) {
            if (extra[order[t]] < n - 1) {
                ++extra[order[t]];
                ++assigned;
            }
        }
        for (uint64_t r = 0; r < n; ++r) deg[node_of_rank[r]] = uint32_t(1 + extra[r]);
    }
    return prefix_rows(n, deg, row);
}

void gathost_fill_sources(uint64_t n, const uint64_t* row, uint64_t seed, uint32_t* col) {
    #pragma omp parallel
    {
        std::vector<uint32_t> s;
        #pragma omp for schedule(dynamic, 256)
        for (uint64_t i = 0; i < n; ++i) {
            const uint64_t deg = row[i + 1] - row[i];
            if (deg == 0) continue;
            Rng r(mix(seed ^ 0x736f'7572'6365ull, i));
            sample_distinct(r, n - 1, deg - 1, s);  // values in [0, n-1), shifted past i
            uint32_t* out = col + row[i];
            uint64_t q = 0;
            bool self_done = false;
            for (uint32_t v : s) {
                const uint32_t src = v >= i ? v + 1 : v;
                if (!self_done && src > i) {
                    out[q++] = uint32_t(i);
                    self_done = true;
                }
                out[q++] = src;
            }
            if (!self_done) out[q++] = uint32_t(i);
        }
    }
}

uint64_t gathost_rmat(int scale, uint64_t edges, double a, double b, double c, uint64_t seed,
                      uint64_t* row, uint32_t* col) {
    const uint64_t n = uint64_t(1) << scale;
    const uint64_t total = edges + n;
    // keys = (dst << 32) | src, bucketed by dst with a counting pass.
    std::vector<uint64_t> keys(total);
    #pragma omp parallel for schedule(static)
    for (uint64_t e = 0; e < edges; ++e) {
        Rng r(mix(seed, e));
        uint64_t dst = 0, src = 0;
        for (int lv = 0; lv < scale; ++lv) {
            const double u = r.unit();
            const uint64_t db = u >= a + b, sb = (u >= a && u < a + b) || u >= a + b + c;
            dst = (dst << 1) | db;
            src = (src << 1) | sb;
        }
        keys[e] = (dst << 32) | src;
    }
    #pragma omp parallel for schedule(static)
    for (uint64_t i = 0; i < n; ++i) keys[edges + i] = (i << 32) | i;
    std::vector<uint64_t> cnt(n + 1, 0);
    {
        std::vector<std::atomic<uint64_t>> ac(n);
        #pragma omp parallel for schedule(static)
        for (uint64_t i = 0; i < n; ++i) ac[i].store(0, std::memory_order_relaxed);
        #pragma omp parallel for schedule(static)
        for (uint64_t e = 0; e < total; ++e) ac[keys[e] >> 32].fetch_add(1, std::memory_order_relaxed);
        for (uint64_t i = 0; i < n; ++i) cnt[i + 1] = cnt[i] + ac[i].load();
        std::vector<uint32_t> bucket(total);
        std::vector<std::atomic<uint64_t>> pos(n);
        #pragma omp parallel for schedule(static)
        for (uint64_t i = 0; i < n; ++i) pos[i].store(cnt[i], std::memory_order_relaxed);
        #pragma omp parallel for schedule(static)
        for (uint64_t e = 0; e < total; ++e) {
            const uint64_t d = keys[e] >> 32;
            bucket[pos[d].fetch_add(1, std::memory_order_relaxed)] = uint32_t(keys[e]);
        }
        std::vector<uint32_t> udeg(n);
        #pragma omp parallel for schedule(dynamic, 1024)
        for (uint64_t i = 0; i < n; ++i) {
            auto* beg = bucket.data() + cnt[i];
            auto* end = bucket.data() + cnt[i + 1];
            std::sort(beg, end);
            udeg[i] = uint32_t(std::unique(beg, end) - beg);
        }
        row[0] = 0;
        for (uint64_t i = 0; i < n; ++i) row[i + 1] = row[i] + udeg[i];
        if (col) {
            #pragma omp parallel for schedule(dynamic, 1024)
            for (uint64_t i = 0; i < n; ++i)
                std::copy(bucket.data() + cnt[i], bucket.data() + cnt[i] + udeg[i], col + row[i]);
        }
    }
    return row[n];
}

void gathost_normal(uint64_t count, uint64_t seed, float* out) {
    const uint64_t pairs = (count + 1) / 2;
    #pragma omp parallel for schedule(static)
    for (uint64_t k = 0; k < pairs; ++k) {
        Rng r(mix(seed ^ 0x6e6f'726dull, k));
        const double u1 = 1.0 - r.unit(), u2 = r.unit();  // u1 in (0,1]
        const double rad = std::sqrt(-2.0 * std::log(u1)), th = 6.283185307179586 * u2;
        out[2 * k] = float(rad * std::cos(th));
        if (2 * k + 1 < count) out[2 * k + 1] = float(rad * std::sin(th));
    }
}

void gathost_glorot_param(int in, int heads, int dim, uint64_t seed, float* w, float* al, float* ar) {
    const uint64_t W = uint64_t(heads) * dim, wn = uint64_t(in) * W;
    const double bw = std::sqrt(6.0 / double(in + W)), ba = std::sqrt(6.0 / double(heads + dim));
    #pragma omp parallel for schedule(static)
    for (uint64_t i = 0; i < wn; ++i) {
        Rng r(mix(seed, i));
        w[i] = float((2.0 * r.unit() - 1.0) * bw);
    }
    for (uint64_t i = 0; i < W; ++i) {
        Rng r1(mix(seed ^ 0xa1ull, i)), r2(mix(seed ^ 0xa2ull, i));
        al[i] = float((2.0 * r1.unit() - 1.0) * ba);
        ar[i] = float((2.0 * r2.unit() - 1.0) * ba);
    }
}

void gathost_random_param(int in, int heads, int dim, int rng_seed, float* w, float* al, float* ar) {
    std::mt19937 rng(rng_seed);
    std::normal_distribution<float> norm;
    const size_t W = size_t(heads) * dim;
    for (size_t i = 0; i < size_t(in) * W; ++i) w[i] = norm(rng) / std::sqrt(float(in));
    for (size_t i = 0; i < W; ++i) al[i] = norm(rng) / std::sqrt(float(dim));
    for (size_t i = 0; i < W; ++i) ar[i] = norm(rng) / std::sqrt(float(dim));
}

}  // extern "C"
