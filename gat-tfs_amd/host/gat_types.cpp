// Formats and checks of the host harness.  Byte layouts follow the reference
// readers/writers so files interchange with it:
//   GATBIN1  magic[8] "GATBIN1\0", u64 n, u64 e, u32 din, u32 classes,
//            u64 row[n+1], u32 col[e], f32 x[n*din]      (baseline/src/common.cpp:31-44)
//   GATWGT1  magic[8], u32 layers=3, per layer u32 {in, heads, dim},
//            f32 w[in*heads*dim], f32 al[heads*dim], f32 ar[heads*dim]  (common.cpp:63-79)
//   GATFIX1  magic[8], u64 {n, e, in, heads, dim}, row, col, w, al, ar,
//            f32 input[n*in], f32 p[e*heads], f32 den[n*heads]         (common.cpp:171-194)
#include "gat_types.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <limits>
#include <random>
#include <stdexcept>

namespace gat {
namespace {

template <class T>
void read_into(std::ifstream& f, T* dst, size_t count) {
    if (count > size_t(std::numeric_limits<std::streamsize>::max()) / sizeof(T))
        throw std::runtime_error("section too large");
    f.read(reinterpret_cast<char*>(dst), std::streamsize(count * sizeof(T)));
    if (!f) throw std::runtime_error("truncated file");
}
template <class T>
void write_from(std::ofstream& f, const T* src, size_t count) {
    f.write(reinterpret_cast<const char*>(src), std::streamsize(count * sizeof(T)));
    if (!f) throw std::runtime_error("write failed");
}
void expect_magic(std::ifstream& f, const char* magic, const char* what) {
    char m[8];
    read_into(f, m, 8);
    if (std::memcmp(m, magic, 7) != 0) throw std::runtime_error(std::string("bad ") + what + " magic");
}
void put_magic(std::ofstream& f, const char* magic) {
    char m[8] = {};
    std::memcpy(m, magic, 7);
    write_from(f, m, 8);
}
uint32_t layer_in(int layer, int din) { return layer == 0 ? uint32_t(din) : 256u; }
uint32_t layer_heads(int layer) { return layer < 2 ? 8u : 1u; }
uint32_t layer_dim(int layer, int classes) { return layer < 2 ? 32u : uint32_t(classes); }

}  // namespace

size_t checked(uint64_t a, uint64_t b) {
    if (b && a > SIZE_MAX / b) throw std::runtime_error("size overflow");
    return size_t(a * b);
}

void require_finite(const std::vector<float>& a, const std::string& name) {
    for (size_t i = 0; i < a.size(); ++i)
        if (!std::isfinite(a[i])) throw std::runtime_error("nonfinite " + name + " index=" + std::to_string(i));
}

void Graph::validate() const {
    if (n == 0 || n > uint64_t(INT32_MAX) || din <= 0 || classes <= 0 || row.size() != n + 1 || col.size() != e ||
        x.size() != checked(n, uint64_t(din)))
        throw std::runtime_error("invalid graph sizes");
    if (row.front() != 0 || row.back() != e) throw std::runtime_error("bad CSR bounds");
    for (uint64_t i = 0; i < n; ++i)
        if (row[i] > row[i + 1]) throw std::runtime_error("nonmonotone CSR");
    for (uint32_t j : col)
        if (j >= n) throw std::runtime_error("source index out of bounds");
    require_finite(x, "graph input");
}

Graph load_graph(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open graph");
    expect_magic(f, "GATBIN1", "graph");
    Graph g;
    uint32_t d = 0, c = 0;
    read_into(f, &g.n, 1);
    read_into(f, &g.e, 1);
    read_into(f, &d, 1);
    read_into(f, &c, 1);
    if (g.n == 0 || g.n > uint64_t(INT32_MAX) || d == 0 || c == 0 || d > uint32_t(INT32_MAX) ||
        c > uint32_t(INT32_MAX))
        throw std::runtime_error("bad graph dimensions");
    g.din = int(d);
    g.classes = int(c);
    g.row.resize(g.n + 1);
    g.col.resize(checked(g.e, 1));
    g.x.resize(checked(g.n, d));
    read_into(f, g.row.data(), g.row.size());
    read_into(f, g.col.data(), g.col.size());
    read_into(f, g.x.data(), g.x.size());
    g.validate();
    return g;
}

void save_graph(const Graph& g, const std::string& path) {
    g.validate();
    std::ofstream f(path, std::ios::binary);
    put_magic(f, "GATBIN1");
    const uint32_t d = uint32_t(g.din), c = uint32_t(g.classes);
    write_from(f, &g.n, 1);
    write_from(f, &g.e, 1);
    write_from(f, &d, 1);
    write_from(f, &c, 1);
    write_from(f, g.row.data(), g.row.size());
    write_from(f, g.col.data(), g.col.size());
    write_from(f, g.x.data(), g.x.size());
}

void Param::validate() const {
    if (in <= 0 || heads <= 0 || heads > 8 || dim <= 0 || dim > 64 || w.size() != checked(uint64_t(in), width()) ||
        al.size() != size_t(width()) || ar.size() != size_t(width()))
        throw std::runtime_error("invalid parameter shape (heads <=8, head_dim <=64)");
    require_finite(w, "W");
    require_finite(al, "aL");
    require_finite(ar, "aR");
}

// random_model semantics (baseline/src/common.cpp:50-62): per layer an
// mt19937 seeded with seed + 11*layer and a standard normal_distribution<float>,
// W scaled by 1/sqrt(in), aL and aR by 1/sqrt(dim).
Model random_model(int din, int classes, int seed) {
    Model m;
    for (int layer = 0; layer < 3; ++layer) {
        Param p;
        p.in = int(layer_in(layer, din));
        p.heads = int(layer_heads(layer));
        p.dim = int(layer_dim(layer, classes));
        p.w.resize(checked(uint64_t(p.in), p.width()));
        p.al.resize(p.width());
        p.ar.resize(p.width());
        std::mt19937 rng(seed + 11 * layer);
        std::normal_distribution<float> normal;
        const float sw = std::sqrt(float(p.in)), sa = std::sqrt(float(p.dim));
        for (float& v : p.w) v = normal(rng) / sw;
        for (float& v : p.al) v = normal(rng) / sa;
        for (float& v : p.ar) v = normal(rng) / sa;
        p.validate();
        m.push_back(std::move(p));
    }
    return m;
}

void save_model(const Model& m, const std::string& path) {
    std::ofstream f(path, std::ios::binary);
    put_magic(f, "GATWGT1");
    const uint32_t count = uint32_t(m.size());
    write_from(f, &count, 1);
    for (const Param& p : m) {
        p.validate();
        const uint32_t shape[3] = {uint32_t(p.in), uint32_t(p.heads), uint32_t(p.dim)};
        write_from(f, shape, 3);
        write_from(f, p.w.data(), p.w.size());
        write_from(f, p.al.data(), p.al.size());
        write_from(f, p.ar.data(), p.ar.size());
    }
}

Model load_model(const std::string& path, int din, int classes) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open weights");
    expect_magic(f, "GATWGT1", "weights");
    uint32_t count = 0;
    read_into(f, &count, 1);
    if (count != 3) throw std::runtime_error("model must have 3 layers");
    Model m;
    for (int l = 0; l < 3; ++l) {
        uint32_t s[3];
        read_into(f, s, 3);
        if (s[0] != layer_in(l, din) || s[1] != layer_heads(l) || s[2] != layer_dim(l, classes))
            throw std::runtime_error("checkpoint model shape mismatch");
        Param p;
        p.in = int(s[0]);
        p.heads = int(s[1]);
        p.dim = int(s[2]);
        p.w.resize(checked(uint64_t(p.in), p.width()));
        p.al.resize(p.width());
        p.ar.resize(p.width());
        read_into(f, p.w.data(), p.w.size());
        read_into(f, p.al.data(), p.al.size());
        read_into(f, p.ar.data(), p.ar.size());
        p.validate();
        m.push_back(std::move(p));
    }
    return m;
}

void save_fixture(const Graph& g, const Param& p, const Fixture& q, const std::string& path) {
    if (q.input.size() != checked(g.n, uint64_t(p.in)) || q.p.size() != checked(g.e, uint64_t(p.heads)) ||
        q.den.size() != checked(g.n, uint64_t(p.heads)))
        throw std::runtime_error("bad fixture sizes");
    std::ofstream f(path, std::ios::binary);
    put_magic(f, "GATFIX1");
    const uint64_t sizes[5] = {g.n, g.e, uint64_t(p.in), uint64_t(p.heads), uint64_t(p.dim)};
    write_from(f, sizes, 5);
    write_from(f, g.row.data(), g.row.size());
    write_from(f, g.col.data(), g.col.size());
    write_from(f, p.w.data(), p.w.size());
    write_from(f, p.al.data(), p.al.size());
    write_from(f, p.ar.data(), p.ar.size());
    write_from(f, q.input.data(), q.input.size());
    write_from(f, q.p.data(), q.p.size());
    write_from(f, q.den.data(), q.den.size());
}

Fixture load_fixture(const Graph& g, const Param& p, const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open fixture");
    expect_magic(f, "GATFIX1", "fixture");
    uint64_t s[5];
    read_into(f, s, 5);
    if (s[0] != g.n || s[1] != g.e || s[2] != uint64_t(p.in) || s[3] != uint64_t(p.heads) || s[4] != uint64_t(p.dim))
        throw std::runtime_error("fixture shape mismatch");
    // The fixture carries its CSR and checkpoint so that an equal-shape but
    // different graph or model is rejected (common.cpp:175-186).
    std::vector<uint64_t> row(g.row.size());
    std::vector<uint32_t> col(g.col.size());
    read_into(f, row.data(), row.size());
    read_into(f, col.data(), col.size());
    if (row != g.row || col != g.col) throw std::runtime_error("fixture CSR mismatch");
    for (const std::vector<float>* master : {&p.w, &p.al, &p.ar}) {
        std::vector<float> v(master->size());
        read_into(f, v.data(), v.size());
        if (v != *master) throw std::runtime_error("fixture checkpoint mismatch");
    }
    Fixture q;
    q.input.resize(checked(g.n, uint64_t(p.in)));
    q.p.resize(checked(g.e, uint64_t(p.heads)));
    q.den.resize(checked(g.n, uint64_t(p.heads)));
    read_into(f, q.input.data(), q.input.size());
    read_into(f, q.p.data(), q.p.size());
    read_into(f, q.den.data(), q.den.size());
    require_finite(q.input, "fixture input");
    require_finite(q.p, "fixture p");
    require_finite(q.den, "fixture denominator");
    // p in [0,1], den = sum of p within 1e-5 relative, den > 0 on non-empty rows.
    for (uint64_t i = 0; i < g.n; ++i)
        for (int h = 0; h < p.heads; ++h) {
            float sum = 0;
            for (uint64_t e = g.row[i]; e < g.row[i + 1]; ++e) {
                const float v = q.p[e * p.heads + h];
                if (v < 0 || v > 1) throw std::runtime_error("fixture p outside [0,1]");
                sum += v;
            }
            const float d = q.den[i * p.heads + h];
            if (std::abs(sum - d) > 1e-5f * std::max(1.0f, sum) || (g.row[i] != g.row[i + 1] && d <= 0))
                throw std::runtime_error("fixture denominator mismatch");
        }
    return q;
}

// errors(): max-abs, mean-abs, relative L2, RMSE and the 50/90/99th
// percentiles of |difference|; any non-finite value marks the comparison
// non-finite with infinite metrics (baseline/src/common.cpp:141-150).
Error errors(const std::vector<float>& ref, const std::vector<float>& got) {
    if (ref.empty() || ref.size() != got.size()) throw std::runtime_error("comparison size mismatch");
    Error e;
    std::vector<double> diffs;
    diffs.reserve(ref.size());
    double sq = 0, norm = 0;
    for (size_t i = 0; i < ref.size(); ++i) {
        if (!std::isfinite(ref[i]) || !std::isfinite(got[i])) {
            e.finite = false;
            continue;
        }
        const double d = double(got[i]) - ref[i], a = std::abs(d);
        e.max_abs = std::max(e.max_abs, a);
        e.mean_abs += a;
        sq += d * d;
        norm += double(ref[i]) * ref[i];
        diffs.push_back(a);
    }
    const double inf = std::numeric_limits<double>::infinity();
    if (!e.finite) {
        e.max_abs = e.mean_abs = e.relative_l2 = e.rmse = e.p50 = e.p90 = e.p99 = inf;
        return e;
    }
    e.mean_abs /= double(ref.size());
    e.rmse = std::sqrt(sq / double(ref.size()));
    e.relative_l2 = norm > 0 ? std::sqrt(sq / norm) : (sq == 0 ? 0 : inf);
    auto pct = [&](double q) {
        const size_t k = std::min(diffs.size() - 1, size_t(std::ceil(q * double(diffs.size())) - 1));
        std::nth_element(diffs.begin(), diffs.begin() + long(k), diffs.end());
        return diffs[k];
    };
    e.p50 = pct(.5);
    e.p90 = pct(.9);
    e.p99 = pct(.99);
    return e;
}

void print_error(const std::string& path, int layer, const std::string& stage, const Error& e) {
    std::cout << std::setprecision(10) << "ERROR path=" << path << " layer=" << layer << " stage=" << stage
              << " finite=" << e.finite << " max_abs=" << e.max_abs << " mean_abs=" << e.mean_abs
              << " relative_l2=" << e.relative_l2 << " rmse=" << e.rmse << " p50=" << e.p50 << " p90=" << e.p90
              << " p99=" << e.p99 << "\n";
}

}  // namespace gat
