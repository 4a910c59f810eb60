// gat_bench: the benchmark / correctness harness of the gfx950 GAT path.
//
// Mirrors the reference harness baseline/bench/main.cpp: `--key value`
// arguments against a whitelist with duplicates rejected (:9-16), a path
// registry dispatched by name (run_path, :21-25), modes benchmark /
// correctness / micro / export-fixture / fixed-p, and the same output lines (ENV,
// STATIC, CONFIG, ERROR, COLD, per-layer JSON, E2E, SUMMARY; :46-64, :169-182).
// Registered paths: gpu_fp32 and gpu_bf16 (include/gatgpu.h through
// gat_gpu_path.hpp).  Correctness compares against R0 stage dumps in the
// reference's --dump-prefix naming (<prefix>_layer<l>_<stage>.f32, :74-77);
// its own --dump-prefix writes the path's stages (<prefix>_<path>_layer<l>_
// <stage>.f32) and chained logits (<prefix>_model_<path>.f32, :96);
// `inspect` only loads and validates the inputs (no GPU).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <map>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "gat_gpu_path.hpp"
#include "gat_types.hpp"
#include "gathost.h"

using namespace gat;

namespace {

struct Args {
    std::map<std::string, std::string> v;
    Args(int argc, char** argv) {
        static const char* allowed[] = {"--graph", "--synthetic", "--din", "--classes", "--weights", "--seed",
                                        "--save-weights", "--save-graph", "--path", "--mode", "--layer",
                                        "--repeats", "--warmups", "--reference-prefix", "--dump-prefix",
                                        "--output", "--max-abs", "--rel-l2", "--fixture", "--dataflow",
                                        "--device", "--reference"};
        for (int i = 1; i < argc; ++i) {
            const std::string k = argv[i];
            if (k.rfind("--", 0) != 0 || i + 1 == argc) throw std::runtime_error("arguments must be --key value");
            if (std::find_if(std::begin(allowed), std::end(allowed), [&](const char* a) { return k == a; }) ==
                std::end(allowed))
                throw std::runtime_error("unknown option: " + k);
            if (!v.emplace(k, argv[++i]).second) throw std::runtime_error("duplicate argument: " + k);
        }
    }
    std::string get(const std::string& k, const std::string& def = "") const {
        auto it = v.find(k);
        return it == v.end() ? def : it->second;
    }
    int num(const std::string& k, int def) const { return std::stoi(get(k, std::to_string(def))); }
    bool has(const std::string& k) const { return v.count(k) != 0; }
};

std::vector<std::string> split(const std::string& s, char sep) {
    std::vector<std::string> out;
    std::stringstream ss(s);
    std::string item;
    while (std::getline(ss, item, sep)) out.push_back(item);
    return out;
}

// --synthetic uniform:N:MEAN:SEED | powerlaw:N:E:MAXDEG:SEED | rmat:SCALE:EDGES:SEED
Graph synthetic_graph(const std::string& spec, int din, int classes) {
    const auto f = split(spec, ':');
    Graph g;
    g.din = din;
    g.classes = classes;
    uint64_t seed = 0;
    if (f.size() == 4 && f[0] == "uniform") {
        g.n = std::stoull(f[1]);
        seed = std::stoull(f[3]);
        g.row.resize(g.n + 1);
        g.e = gathost_uniform_rows(g.n, uint32_t(std::stoul(f[2])), seed, g.row.data());
        g.col.resize(g.e);
        gathost_fill_sources(g.n, g.row.data(), seed, g.col.data());
    } else if (f.size() == 5 && f[0] == "powerlaw") {
        g.n = std::stoull(f[1]);
        seed = std::stoull(f[4]);
        g.row.resize(g.n + 1);
        g.e = gathost_powerlaw_rows(g.n, std::stoull(f[2]), uint32_t(std::stoul(f[3])), seed, g.row.data());
        if (g.e == 0) throw std::runtime_error("infeasible power-law request");
        g.col.resize(g.e);
        gathost_fill_sources(g.n, g.row.data(), seed, g.col.data());
    } else if (f.size() == 4 && f[0] == "rmat") {
        const int scale = std::stoi(f[1]);
        const uint64_t edges = std::stoull(f[2]);
        seed = std::stoull(f[3]);
        g.n = uint64_t(1) << scale;
        g.row.resize(g.n + 1);
        g.e = gathost_rmat(scale, edges, 0.57, 0.19, 0.19, seed, g.row.data(), nullptr);
        g.col.resize(g.e);
        gathost_rmat(scale, edges, 0.57, 0.19, 0.19, seed, g.row.data(), g.col.data());
    } else {
        throw std::runtime_error("bad --synthetic spec");
    }
    g.x.resize(checked(g.n, uint64_t(din)));
    gathost_normal(g.x.size(), seed + 1, g.x.data());
    g.validate();
    return g;
}

std::vector<float> read_dump(const std::string& path, size_t count) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open dump " + path);
    std::vector<float> v(count);
    f.read(reinterpret_cast<char*>(v.data()), std::streamsize(count * 4));
    if (!f) throw std::runtime_error("truncated dump " + path);
    return v;
}
void write_dump(const std::string& path, const std::vector<float>& v) {
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char*>(v.data()), std::streamsize(v.size() * 4));
    if (!f) throw std::runtime_error("cannot write dump " + path);
}

double pct(std::vector<double> x, double q) {
    std::sort(x.begin(), x.end());
    return x[std::min(x.size() - 1, size_t(std::ceil(q * double(x.size())) - 1))];
}

void print_times(const std::string& path, const std::string& mode, int layer, int rep, const Graph& g,
                 const Param& p, const Times& t) {
    std::cout << std::setprecision(10) << "{\"path\":\"" << path << "\",\"mode\":\"" << mode << "\",\"layer\":" << layer
              << ",\"rep\":" << rep << ",\"N\":" << g.n << ",\"E\":" << g.e << ",\"D\":" << p.in << ",\"K\":" << p.heads
              << ",\"d\":" << p.dim << ",\"precision\":\"" << (path == "gpu_fp32" ? "FP32" : "BF16_RNE_FP32_state")
              << "\",\"convert_ms\":" << t.convert * 1e3 << ",\"projection_ms\":" << t.projection * 1e3
              << ",\"lr_ms\":" << t.lr * 1e3 << ",\"max_prescan_ms\":" << t.max_prescan * 1e3
              << ",\"score_exp_aggregate_ms\":" << t.aggregate * 1e3 << ",\"normalize_ms\":" << t.normalize * 1e3
              << ",\"activation_ms\":" << t.activation * 1e3 << ",\"total_ms\":" << t.total * 1e3
              << ",\"gedge_per_s\":" << (t.total > 0 ? double(g.e) / t.total / 1e9 : 0) << "}\n";
}

// The path registry (run_path): every registered name maps to a callable
// with the per-layer signature.
struct PathRegistry {
    gatgpu_host::GpuPath* gpu = nullptr;
    int dataflow = GATGPU_AUTO;
    static bool known(const std::string& p) { return p == "gpu_fp32" || p == "gpu_bf16"; }
    void run(const std::string& path, const Graph& g, const Param& p, int layer, const std::vector<float>& input,
             Workspace& w, bool hidden, Times& t) const {
        if (path == "gpu_fp32") gpu->layer(g, p, layer, input, w, hidden, t, GATGPU_FP32, dataflow);
        else if (path == "gpu_bf16") gpu->layer(g, p, layer, input, w, hidden, t, GATGPU_BF16, dataflow);
        else throw std::runtime_error("bad path");
    }
};

int dataflow_of(const std::string& s) {
    if (s == "auto") return GATGPU_AUTO;
    if (s == "transform_first") return GATGPU_TRANSFORM_FIRST;
    if (s == "aggregate_first") return GATGPU_AGGREGATE_FIRST;
    if (s == "tfs_b1") return GATGPU_TFS_B1;
    throw std::runtime_error("bad --dataflow (auto | transform_first | aggregate_first | tfs_b1)");
}

int run(int argc, char** argv) {
    Args a(argc, argv);
    const std::string path = a.get("--path", "gpu_bf16"), mode = a.get("--mode", "benchmark");
    if (!PathRegistry::known(path)) throw std::runtime_error("bad path");
    if (mode != "benchmark" && mode != "correctness" && mode != "micro" && mode != "inspect" &&
        mode != "export-fixture" && mode != "fixed-p")
        throw std::runtime_error("bad mode");
    const int reps = a.num("--repeats", 5), warmups = a.num("--warmups", 2), layer = a.num("--layer", 0);
    if (reps < 1 || warmups < 0 || layer < 0 || layer > 3) throw std::runtime_error("invalid benchmark controls");
    const int dataflow = dataflow_of(a.get("--dataflow", "auto"));
    // ---- inputs (static: load, validate, model; untimed like main.cpp:44-56)
    const auto t_load = std::chrono::steady_clock::now();
    Graph g;
    if (a.has("--graph") == a.has("--synthetic")) throw std::runtime_error("give exactly one of --graph, --synthetic");
    if (a.has("--graph")) g = load_graph(a.get("--graph"));
    else g = synthetic_graph(a.get("--synthetic"), a.num("--din", 128), a.num("--classes", 40));
    Model model;
    if (a.has("--weights")) model = load_model(a.get("--weights"), g.din, g.classes);
    else {
        if (!a.has("--seed")) throw std::runtime_error("provide --weights checkpoint.bin or explicit --seed for synthetic fixture");
        model = random_model(g.din, g.classes, a.num("--seed", 11));
    }
    if (a.has("--save-weights")) save_model(model, a.get("--save-weights"));
    if (a.has("--save-graph")) save_graph(g, a.get("--save-graph"));
    const double load_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_load).count();
    std::cout << "ENV source_input=" << (a.has("--graph") ? a.get("--graph") : a.get("--synthetic"))
              << " checkpoint=" << (a.has("--weights") ? a.get("--weights") : "random_fixture_not_trained")
              << " device=" << a.num("--device", 0) << "\n";
    std::cout << "STATIC N=" << g.n << " E=" << g.e << " D=" << g.din << " C=" << g.classes
              << " load_ms=" << load_ms << " graph_policy=as_loaded_no_mutation\n";
    std::cout << "CONFIG mode=" << mode << " path=" << path << " layer=" << layer << " warmups=" << warmups
              << " repeats=" << reps << " dataflow=" << a.get("--dataflow", "auto") << "\n";
    if (mode == "inspect") return 0;
    if (mode == "export-fixture") {  // GATFIX1 from R0 dumps (main.cpp:126-128); no GPU needed
        const std::string pre = a.get("--reference-prefix");
        if (pre.empty()) throw std::runtime_error("--reference-prefix (R0 stage dumps) is required");
        const int l = layer ? layer : 2;
        const Param& p = model[l - 1];
        Fixture q;
        q.input = l == 1 ? g.x : read_dump(pre + "_layer" + std::to_string(l - 1) + "_output.f32", checked(g.n, uint64_t(p.in)));
        q.p = read_dump(pre + "_layer" + std::to_string(l) + "_p.f32", checked(g.e, uint64_t(p.heads)));
        q.den = read_dump(pre + "_layer" + std::to_string(l) + "_den.f32", checked(g.n, uint64_t(p.heads)));
        if (!a.has("--fixture")) throw std::runtime_error("--fixture output is required");
        save_fixture(g, p, q, a.get("--fixture"));
        std::cout << "FIXTURE saved layer=" << l << "\n";
        return 0;
    }

    gatgpu_host::GpuPath gpu(a.num("--device", 0));
    gpu.set_classes_hint(g.classes);
    PathRegistry reg{&gpu, dataflow};
    const int precision = path == "gpu_fp32" ? GATGPU_FP32 : GATGPU_BF16;

    if (mode == "correctness") {
        const std::string pre = a.get("--reference-prefix");
        if (pre.empty()) throw std::runtime_error("--reference-prefix (R0 stage dumps) is required");
        const bool have_abs = a.has("--max-abs"), have_rel = a.has("--rel-l2");
        if (have_abs != have_rel) throw std::runtime_error("set both --max-abs and --rel-l2");
        const double max_abs = have_abs ? std::stod(a.get("--max-abs")) : 0, rel = have_rel ? std::stod(a.get("--rel-l2")) : 0;
        bool pass = true, finite = true;
        auto check = [&](int l, const std::string& stage, const std::vector<float>& r, const std::vector<float>& v,
                         bool gate) {
            Error e = errors(r, v);
            print_error(path, l, stage, e);
            pass &= e.finite;
            finite &= e.finite;
            if (gate && have_abs) pass &= e.max_abs <= max_abs && e.relative_l2 <= rel;
        };
        // Per layer on the R0-chained input (main.cpp:71-90).
        std::vector<float> input = g.x;
        for (int l = 0; l < 3; ++l) {
            const Param& p = model[l];
            const std::string lp = pre + "_layer" + std::to_string(l + 1);
            const size_t nk = checked(g.n, uint64_t(p.heads)), nw = checked(g.n, uint64_t(p.width()));
            Workspace w;
            Times t;
            reg.run(path, g, p, l, input, w, l < 2, t);
            if (!w.z.empty()) check(l + 1, "Z", read_dump(lp + "_z.f32", nw), w.z, false);
            check(l + 1, "L", read_dump(lp + "_left.f32", nk), w.left, false);
            check(l + 1, "R", read_dump(lp + "_right.f32", nk), w.right, false);
            check(l + 1, "row_max", read_dump(lp + "_max.f32", nk), w.max, false);
            check(l + 1, "denominator", read_dump(lp + "_den.f32", nk), w.den, false);
            std::vector<float> ref_out = read_dump(lp + "_output.f32", nw);
            check(l + 1, "layer", ref_out, w.out, true);
            print_times(path, "correctness", l + 1, 0, g, p, t);
            if (a.has("--dump-prefix")) {
                // The reference dumps R0's stages here (main.cpp:74-77), which this
                // harness reads instead (--reference-prefix); it dumps the path's
                // own stages, named with the path: <prefix>_<path>_layer<l>_<stage>.f32.
                const std::string dp = a.get("--dump-prefix") + "_" + path + "_layer" + std::to_string(l + 1) + "_";
                for (auto item : {std::make_pair("output", &w.out), {"z", &w.z}, {"left", &w.left}, {"right", &w.right},
                                  {"max", &w.max}, {"den", &w.den}})
                    if (!item.second->empty()) write_dump(dp + item.first + ".f32", *item.second);
            }
            input = std::move(ref_out);
        }
        // The path's own three-layer chain against R0's (main.cpp:91-98).
        std::vector<float> logits;
        gpu.model(precision, &logits, dataflow);
        check(3, "model_path_specific_chain",
              read_dump(pre + "_layer3_output.f32", checked(g.n, uint64_t(model[2].width()))), logits, true);
        if (a.has("--output")) write_dump(a.get("--output"), logits);
        // The path's chained logits under the reference's name (main.cpp:96).
        if (a.has("--dump-prefix")) write_dump(a.get("--dump-prefix") + "_model_" + path + ".f32", logits);
        std::cout << "CORRECTNESS finite=" << finite << " accuracy_gate="
                  << (have_abs ? (pass ? "PASS" : "FAIL") : "UNCONFIGURED_NOT_ACCEPTED") << "\n";
        return pass ? 0 : 1;
    }

    if (mode == "fixed-p") {  // main.cpp:103-150: standard_op and, where it applies, tfs_op
        const int l = layer ? layer : 2;
        const Param& p = model[l - 1];
        if (!a.has("--fixture")) throw std::runtime_error("--fixture (GATFIX1) is required");
        const Fixture fixture = load_fixture(g, p, a.get("--fixture"));
        const bool tfs = precision == GATGPU_BF16 && p.dim == 32 && p.in <= 128 &&
                         (p.heads == 1 || p.heads == 2 || p.heads == 4 || p.heads == 8);
        Workspace sw, tw;
        Times t;
        gpu.fixed_p(g, p, l - 1, fixture, sw, t, precision);
        require_finite(sw.out, "fixed-p standard");
        if (tfs) {
            gpu.fixed_p(g, p, l - 1, fixture, tw, t, precision, GATGPU_TFS_B1);
            require_finite(tw.out, "fixed-p TFS");
            print_error("tfs_b1_fixed_p", l, "vs_standard_extra_pX_quantization_and_reduction", errors(sw.out, tw.out));
        }
        if (a.has("--reference")) {  // FP32 fixed-p master output (main.cpp:136-137), one f32 dump
            const std::vector<float> master = read_dump(a.get("--reference"), checked(g.n, uint64_t(p.width())));
            print_error(path + "_fixed_p", l, "vs_master_fixed_p", errors(master, sw.out));
            if (tfs) print_error("tfs_b1_fixed_p", l, "vs_master_fixed_p", errors(master, tw.out));
        }
        if (a.has("--output")) write_dump(a.get("--output"), sw.out);
        // Alternate the two operators each repetition (the reference's AB/BA policy).
        std::vector<double> st, tt, agg;
        for (int r = -warmups; r < reps; ++r) {
            Times s, u;
            const bool ab = (r & 1) == 0;
            if (ab) gpu.fixed_p(g, p, l - 1, fixture, sw, s, precision);
            if (tfs) gpu.fixed_p(g, p, l - 1, fixture, tw, u, precision, GATGPU_TFS_B1);
            if (!ab) gpu.fixed_p(g, p, l - 1, fixture, sw, s, precision);
            if (r >= 0) {
                st.push_back(s.total);
                agg.push_back(s.aggregate);
                print_times(path, "fixed-p", l, r, g, p, s);
                if (tfs) {
                    tt.push_back(u.total);
                    print_times("tfs_b1", "fixed-p", l, r, g, p, u);
                }
            }
        }
        std::cout << "FIXED_P path=" << path << " layer=" << l << " median_ms=" << pct(st, .5) * 1e3
                  << " median_aggregate_ms=" << pct(agg, .5) * 1e3
                  << " aggregate_gedge_per_s=" << double(g.e) / pct(agg, .5) / 1e9;
        if (tfs)
            std::cout << " median_tfs_ms=" << pct(tt, .5) * 1e3 << " speedup=" << pct(st, .5) / pct(tt, .5);
        std::cout << " conversion_included=true policy=AB_BA\n";
        return 0;
    }

    if (mode == "micro") {
        const int l = layer ? layer : 2;
        std::vector<float> input = g.x;
        for (int q = 0; q < l - 1; ++q) {  // input of layer l: the path's own chain
            Workspace w;
            Times t;
            reg.run(path, g, model[q], q, input, w, true, t);
            input = w.out;
        }
        std::vector<double> conv, proj, agg, tot;
        for (int r = -warmups; r < reps; ++r) {
            Workspace w;
            Times t;
            reg.run(path, g, model[l - 1], l - 1, input, w, l < 3, t);
            if (r >= 0) {
                conv.push_back(t.convert);
                proj.push_back(t.projection);
                agg.push_back(t.aggregate);
                tot.push_back(t.total);
            }
        }
        for (auto item : {std::make_pair("convert_rne", &conv), {"projection_lr", &proj},
                          {"prescan_softmax_aggregate_finish", &agg}, {"layer_total", &tot}})
            std::cout << "MICRO name=" << item.first << " layer=" << l << " median_ms=" << pct(*item.second, .5) * 1e3
                      << " p95_ms=" << pct(*item.second, .95) * 1e3 << "\n";
        return 0;
    }

    // ---- benchmark: device-resident model timing (main.cpp:153-183).  The
    // COLD line spans graph load to the first forward, uploads and weight
    // preparation included (main.cpp:169); each timed repeat prints the
    // per-layer stage times of that forward (main.cpp:177) and its E2E line.
    std::vector<double> totals;
    for (int l = 0; l < 3; ++l) gpu.set_layer(l, model[l]);
    gpu.set_graph(g);
    std::cout << "COLD startup_before_inference_ms="
              << std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_load).count()
              << " includes_graph_load=true\n";
    double cold = 0;
    for (int r = -warmups; r < reps; ++r) {
        const double s = gpu.model(precision, nullptr, dataflow);
        if (r == -warmups) cold = s;
        if (r >= 0) {
            totals.push_back(s);
            for (int l = 0; l < 3; ++l) {
                Times t;
                gpu.model_layer_times(l, t);
                print_times(path, "benchmark", l + 1, r, g, model[l], t);
            }
            std::cout << "E2E path=" << path << " rep=" << r << " layer=0 total_ms=" << s * 1e3
                      << " gedge_per_s=" << 3.0 * double(g.e) / s / 1e9 << " finite=1\n";
        }
    }
    if (a.has("--output")) {
        std::vector<float> logits;
        gpu.model(precision, &logits, dataflow);
        require_finite(logits, "benchmark output");
        write_dump(a.get("--output"), logits);
    }
    std::cout << "SUMMARY path=" << path << " median_ms=" << pct(totals, .5) * 1e3 << " p95_ms=" << pct(totals, .95) * 1e3
              << " cold_forward_ms=" << cold * 1e3 << " repeats=" << reps
              << " gedge_per_s=" << 3.0 * double(g.e) / pct(totals, .5) / 1e9 << "\n";
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        return run(argc, argv);
    } catch (const std::exception& e) {
        std::cerr << "FAIL " << e.what() << "\n";
        return 1;
    }
}
