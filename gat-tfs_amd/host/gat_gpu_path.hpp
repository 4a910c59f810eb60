// C++ adapter that registers the gfx950 path in a harness built around the
// reference's containers: gat::Graph (u64 row, u32 col, f32 x; din, classes),
// gat::Param (in, heads, dim, w, al, ar), gat::Workspace (z, left, right, max,
// den, out vectors) and gat::Times (convert, projection, lr, max_prescan,
// aggregate, normalize, activation, total in seconds) --
// baseline/include/gat.hpp:32-106.  It is templated on those types, so it
// compiles against the reference's own header or against any structs with the
// same field names (gat-tfs_amd/host/gat_types.hpp).
//
// gpu_layer() has the shape of the per-layer entry points the harness
// dispatches to in run_path (baseline/bench/main.cpp:21-25,
// baseline/include/gat.hpp:107-117): same inputs, same Workspace fields
// filled, same Times fields.  Every non-zero C-ABI return becomes a
// std::runtime_error, which the harness turns into "FAIL msg", exit 1
// (baseline/bench/main.cpp:184).
#pragma once
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "gatgpu.h"

namespace gatgpu_host {

inline void check(gatgpu_ctx* ctx, int rc, const char* what) {
    if (rc != GATGPU_OK)
        throw std::runtime_error(std::string(what) + ": " + gatgpu_last_error(ctx) + " (code " +
                                 std::to_string(rc) + ")");
}

// One device context plus the identity of what it currently holds, so a
// harness that calls the path layer by layer uploads the graph and each
// layer's weights once.
class GpuPath {
   public:
    explicit GpuPath(int device = 0) {
        gatgpu_ctx* c = nullptr;
        check(nullptr, gatgpu_create(device, &c), "gatgpu_create");
        ctx_ = c;
    }
    ~GpuPath() { gatgpu_destroy(ctx_); }
    GpuPath(const GpuPath&) = delete;
    GpuPath& operator=(const GpuPath&) = delete;
    gatgpu_ctx* ctx() const { return ctx_; }

    template <class Graph>
    void set_graph(const Graph& g) {
        if (graph_ == static_cast<const void*>(&g) && n_ == g.n && e_ == g.e) return;
        check(ctx_, gatgpu_set_graph(ctx_, g.n, g.e, g.row.data(), g.col.data()), "gatgpu_set_graph");
        check(ctx_, gatgpu_set_input(ctx_, g.n, int(g.din), g.x.data()), "gatgpu_set_input");
        graph_ = &g;
        fixture_ = nullptr;  // set_graph drops every fixture
        n_ = g.n;
        e_ = g.e;
    }

    template <class Param>
    void set_layer(int layer, const Param& p) {
        if (layer_[layer] == static_cast<const void*>(&p)) return;
        check(ctx_, gatgpu_set_layer(ctx_, layer, p.in, p.heads, p.dim, p.w.data(), p.al.data(), p.ar.data()),
              "gatgpu_set_layer");
        layer_[layer] = &p;
        if (fixture_layer_ == layer) fixture_ = nullptr;  // set_layer drops the layer's fixture
    }

    // The per-layer path: input -> w.out, times in seconds.  With `stages`
    // (the reference's correctness mode) also the stage vectors it compares
    // (z, left, right, max, den); without, w.out is the only copy back.
    template <class Graph, class Param, class Workspace, class Times>
    void layer(const Graph& g, const Param& p, int layer_index, const std::vector<float>& input, Workspace& w,
               bool hidden, Times& t, int precision, int dataflow = GATGPU_AUTO, bool stages = true) {
        set_graph(g);
        set_layer(layer_index, p);
        gatgpu_times gt{};
        check(ctx_,
              gatgpu_layer_forward(ctx_, layer_index, precision, dataflow, hidden ? 1 : 0, input.data(), &gt),
              "gatgpu_layer_forward");
        t.convert = gt.convert_ms * 1e-3;
        t.projection = gt.projection_ms * 1e-3;
        t.lr = gt.lr_ms * 1e-3;
        t.max_prescan = gt.max_prescan_ms * 1e-3;
        t.aggregate = gt.aggregate_ms * 1e-3;
        t.normalize = gt.normalize_ms * 1e-3;
        t.activation = gt.activation_ms * 1e-3;
        t.total = gt.total_ms * 1e-3;
        fetch(layer_index, GATGPU_STAGE_OUT, w.out);
        if (!stages) return;
        fetch(layer_index, GATGPU_STAGE_LEFT, w.left);
        fetch(layer_index, GATGPU_STAGE_RIGHT, w.right);
        fetch(layer_index, GATGPU_STAGE_MAX, w.max);
        fetch(layer_index, GATGPU_STAGE_DEN, w.den);
        fetch(layer_index, GATGPU_STAGE_Z, w.z);
    }

    // The fixed-p operator (baseline/bench/main.cpp:103-150): uploads the
    // fixture's p/den once per Fixture object, runs it on fixture.input --
    // "standard_op" with TRANSFORM_FIRST, "tfs_op" with GATGPU_TFS_B1 -- and
    // fills w.z (transform-first only), w.den, w.out and the Times fields.
    template <class Graph, class Param, class Fixture, class Workspace, class Times>
    void fixed_p(const Graph& g, const Param& p, int layer_index, const Fixture& f, Workspace& w, Times& t,
                 int precision, int dataflow = GATGPU_TRANSFORM_FIRST) {
        set_graph(g);
        set_layer(layer_index, p);
        if (fixture_ != static_cast<const void*>(&f) || fixture_layer_ != layer_index) {
            check(ctx_, gatgpu_set_fixed_p(ctx_, layer_index, f.p.data(), f.den.data()), "gatgpu_set_fixed_p");
            fixture_ = &f;
            fixture_layer_ = layer_index;
        }
        gatgpu_times gt{};
        check(ctx_,
              gatgpu_fixed_p_forward(ctx_, layer_index, precision, dataflow, f.input.data(), &gt),
              "gatgpu_fixed_p_forward");
        t.convert = gt.convert_ms * 1e-3;
        t.projection = gt.projection_ms * 1e-3;
        t.aggregate = gt.aggregate_ms * 1e-3;
        t.total = gt.total_ms * 1e-3;
        fetch(layer_index, GATGPU_STAGE_OUT, w.out);
        fetch(layer_index, GATGPU_STAGE_DEN, w.den);
        fetch(layer_index, GATGPU_STAGE_Z, w.z);
    }

    // Three layers chained on the device; returns the model time in seconds
    // (HIP events from layer 1's first kernel to layer 3's last; the logits
    // are copied back after the timer stops).
    template <class Graph, class Model>
    double model(const Graph& g, const Model& m, int precision, std::vector<float>* logits,
                 int dataflow = GATGPU_AUTO) {
        set_graph(g);
        for (int l = 0; l < 3; ++l) set_layer(l, m[l]);
        set_classes_hint(int(m[2].heads * m[2].dim));
        return model(precision, logits, dataflow);
    }
    double model(int precision, std::vector<float>* logits, int dataflow = GATGPU_AUTO) {
        double ms = 0;
        if (logits) logits->resize(size_t(n_) * classes_hint_);
        check(ctx_,
              gatgpu_model_forward(ctx_, precision, dataflow, logits ? logits->data() : nullptr, model_times_, &ms),
              "gatgpu_model_forward");
        return ms * 1e-3;
    }
    void set_classes_hint(int c) { classes_hint_ = c; }
    // Stage times (seconds) of layer l of the last model() call.
    template <class Times>
    void model_layer_times(int l, Times& t) const {
        const gatgpu_times& g = model_times_[l];
        t.convert = g.convert_ms * 1e-3;
        t.projection = g.projection_ms * 1e-3;
        t.lr = g.lr_ms * 1e-3;
        t.max_prescan = g.max_prescan_ms * 1e-3;
        t.aggregate = g.aggregate_ms * 1e-3;
        t.normalize = g.normalize_ms * 1e-3;
        t.activation = g.activation_ms * 1e-3;
        t.total = g.total_ms * 1e-3;
    }

   private:
    void fetch(int layer, int which, std::vector<float>& v) {
        uint64_t count = 0;
        check(ctx_, gatgpu_stage_size(ctx_, layer, which, &count), "gatgpu_stage_size");
        if (!count) {
            v.clear();
            return;
        }
        v.resize(count);
        check(ctx_, gatgpu_get_stage(ctx_, layer, which, v.data()), "gatgpu_get_stage");
    }
    gatgpu_ctx* ctx_ = nullptr;
    const void* graph_ = nullptr;
    const void* fixture_ = nullptr;
    int fixture_layer_ = -1;
    const void* layer_[3] = {nullptr, nullptr, nullptr};
    uint64_t n_ = 0, e_ = 0;
    int classes_hint_ = 0;
    gatgpu_times model_times_[3] = {};
};

}  // namespace gatgpu_host
