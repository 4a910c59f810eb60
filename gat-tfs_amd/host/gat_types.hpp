// Host containers and file formats of the GAT harness, with the field names
// and on-disk layouts of the reference (baseline/include/gat.hpp:32-131,
// baseline/src/common.cpp), so gat_gpu_path.hpp drives either.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace gat {

size_t checked(uint64_t a, uint64_t b);  // a*b or throw "size overflow"
void require_finite(const std::vector<float>& a, const std::string& name);

// Destination-row CSR with node features (GATBIN1).
struct Graph {
    uint64_t n = 0, e = 0;
    int din = 0, classes = 0;
    std::vector<uint64_t> row;
    std::vector<uint32_t> col;
    std::vector<float> x;
    void validate() const;
};
Graph load_graph(const std::string& path);
void save_graph(const Graph&, const std::string& path);

// One layer: W[in][heads*dim] row-major, head h = columns [h*dim, (h+1)*dim).
struct Param {
    int in = 0, heads = 0, dim = 0;
    std::vector<float> w, al, ar;
    int width() const { return heads * dim; }
    void validate() const;
};
using Model = std::vector<Param>;
Model random_model(int din, int classes, int seed);
Model load_model(const std::string& path, int din, int classes);
void save_model(const Model&, const std::string& path);

// Stage arrays of one layer.
struct Workspace {
    std::vector<float> z, left, right, max, den, out;
};
// Stage times in seconds.
struct Times {
    double convert = 0, projection = 0, lr = 0, max_prescan = 0, aggregate = 0, normalize = 0, activation = 0,
           total = 0;
};
// Fixed-p fixture (GATFIX1): the layer input plus p[e][K] and den[n][K].
struct Fixture {
    std::vector<float> input, p, den;
};
void save_fixture(const Graph&, const Param&, const Fixture&, const std::string& path);
Fixture load_fixture(const Graph&, const Param&, const std::string& path);

struct Error {
    double max_abs = 0, mean_abs = 0, relative_l2 = 0, rmse = 0, p50 = 0, p90 = 0, p99 = 0;
    bool finite = true;
};
Error errors(const std::vector<float>& ref, const std::vector<float>& actual);
void print_error(const std::string& path, int layer, const std::string& stage, const Error&);

}  // namespace gat
