// The library context (gatgpu_ctx) and the helpers shared by the C-ABI
// translation units.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

#include "gatgpu.h"
#include "internal.hpp"

namespace gatgpu {

struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() { release(); }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
    // Grows to at least `b` bytes; contents are not preserved.
    hipError_t ensure(size_t b) {
        if (b <= bytes && p) return hipSuccess;
        release();
        if (b == 0) b = 1;
        hipError_t e = hipMalloc(&p, b);
        if (e == hipSuccess) bytes = b;
        else p = nullptr;
        return e;
    }
    template <class T>
    T* as() const {
        return static_cast<T*>(p);
    }
};

struct LayerState {
    bool set = false;
    int in = 0, heads = 0, dim = 0;
    DevBuf w32, wq32, al, ar, blr;
    DevBuf wpk32;  // FP32 MFMA fragments (projection_f32_supported shapes), else empty
    DevBuf z32, zbf, left, right, mx, den, out32, outbf, in32, inbf;
    // What the last forward of this layer produced.
    bool ran = false, z_valid = false, out32_valid = false, outbf_valid = false;
    bool out_original = false;  // out32 rows in original node order (else sorted order)
    int out_stride = 0;         // out32 row stride (floats): the width, or k1_out_stride when out_original
    bool xbf_valid = false;     // inbf holds the rounded layer input rows
    int xbf_stride = 0;         // their row stride (bf16 elements)
    int precision = -1;
    // bf16 MFMA projection weights (pack_projection_weights order)
    DevBuf wpk;
    int ksteps = 0, groups = 0, nmb = 0;
    // L/R-only block for the aggregate-first front end
    DevBuf wlr;
    int lr_ksteps = 0;
    int dataflow = 0;  // dataflow of the last forward
    // fixed-p fixture: p in degree-sorted edge order [e][heads], den [n][heads]
    DevBuf fixp, fixden;
    bool fixed_set = false;
    double prepare_ms = 0;  // wall time of the last set_layer
    int width() const { return heads * dim; }
};

// Split rows: rows of in-degree >= min are cut into chunks of `chunk` edges
// on separate waves.  Each aggregation family has its own plan; the values
// below were measured best on the 64.3M-edge power-law graph
// (100 -> 8x32 -> 8x32 -> 1x47, max in-degree 17 000): the sum form keeps
// many short chunks, the one-row-per-wave 8-head kernel fewer, longer ones,
// and the one-head kernel (8 rows per wave) splits only its heaviest rows.
// Small graphs (below kSmallGraphEdges edges) split more rows into shorter
// chunks, 512/256 for every kernel: their heaviest rows are a larger share of
// a short launch (169K-node, 2.5M-edge power-law graph: 0.88 ms against 1.23
// with the plans above).  Graphs with heavier rows scale a plan (chunk and
// min) by the smallest power of two that keeps the heaviest row within
// kMaxChunksPerRow chunks: each chunk reduces the maxima of all chunks of its
// row and the last one adds all partial sums, so many chunks per row cost
// more than they balance.  The 8-head kernel (one row per wave) scales min
// with the chunk; the sum form (32-row tiles) and the one-head kernel (8 rows
// per wave) hold a heavy row's neighbours at the same pace, and split from
// twice the chunk instead.  On the 100M-edge R-MAT graph (max in-degree
// 132 270) that gives 6144/2048 (8-head) and 4096/2048 (sum form, one head),
// the best of measured sweeps there (sum form: 7.4 ms against 8.4 at
// 8192/2048).
enum { kPlanAf = 0, kPlanVec = 1, kPlanOne = 2, kPlans = 3 };
constexpr uint32_t kPlanMin[kPlans] = {1024, 1536, 2048};
constexpr uint32_t kPlanChunk[kPlans] = {256, 512, 1024};
constexpr uint64_t kSmallGraphEdges = 16u << 20;
constexpr uint32_t kSmallPlanMin = 512, kSmallPlanChunk = 256;
constexpr uint64_t kMaxChunksPerRow = 96;
// Floats per split chunk in SplitTable::part: the widest partial row of the
// transform-first kernels (512 features, 8 denominators, 8 chunk maxima).
constexpr uint64_t kTfPartFloats = 512 + 16;
struct SplitPlan {
    uint32_t min = 0, chunk = 0;
    RowBins bins;        // split_begin: first split row (sorted position)
    SplitTable table;
    DevBuf k, first, mchunk, part, counter;
};

// Device buffers of one transform-first layer run: the context's per-layer
// buffers (sorted node order, sources relabelled) or any other set of
// buffers with the CSR sources and row permutation that index them.
struct TfBufs {
    const uint32_t* pcol = nullptr;  // CSR sources in the node order of the buffers below
    const uint32_t* perm = nullptr;  // sorted position -> row of L/R/max/den/out
    float *left = nullptr, *right = nullptr, *mx = nullptr, *den = nullptr;
    void* z = nullptr;               // bf16 [n][zs] or FP32 [n][zs]
    uint16_t* xbf = nullptr;         // bf16 input rows [n][16 ksteps] (FP32 input of a bf16 layer)
    float* out32 = nullptr;          // [n][W] + kF32Pad, or null
    uint16_t* outbf = nullptr;       // [n][W] (hidden bf16 layers), or null
    // Split-row scratch; null: the plan's own buffers.
    float* mchunk = nullptr;
    float* part = nullptr;
    uint32_t* counter = nullptr;
    bool fused_convert_ok = false;   // the FP32 input carries kF32Pad floats past its last row
    bool keep_xbf = false;           // write the rounded input rows to xbf even when the convert is fused
    const uint32_t* out_perm = nullptr;  // one-head kernel: output row of sorted position k
    int ostride = 0;                     // its out32 row stride (floats)
    // The next layer's projection in this layer's aggregation epilogue
    // (launch_aggregate_vec_next); the next layer then runs with projected.
    const NextProj* next = nullptr;
    bool projected = false;          // Z, L and R were written by the previous layer's epilogue
};

}  // namespace gatgpu

struct gatgpu_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    // graph and schedule
    bool graph = false;
    uint64_t n = 0, e = 0;
    gatgpu::DevBuf row, col, keys_a, keys_b, vals_a, vals_b, hist, scan_tmp, prow, pcol, small;
    uint32_t* sorted_deg = nullptr;
    uint32_t* perm = nullptr;     // sorted position -> original node
    // Node-indexed device state (features, Z, L, R, max, den, outputs) is kept
    // in sorted node order: node k is original node perm[k], rcol holds the
    // sorted CSR's sources as sorted positions, and the kernels get the
    // identity as their row permutation.  Inputs are gathered into this order
    // when they are uploaded and outputs are put back in original order.
    gatgpu::DevBuf invperm, ident, rcol, logits;
    std::vector<uint32_t> perm_h;
    uint64_t neighbor_steps = 0;
    uint32_t max_degree = 0;
    gatgpu::RowBins bins;
    // input
    bool input = false;
    int din = 0;
    gatgpu::DevBuf x32, xbf;
    gatgpu::DevBuf xorig;  // the features in original node order (x32 is their sorted-order copy)
    gatgpu::LayerState L[3];
    // options (in-degree thresholds)
    uint32_t block_min = 512;        // rows >= this take a block
    uint32_t split_min = 0;          // user option: rows >= this are split (0: per-kernel defaults)
    uint32_t split_chunk = 0;        // user option: edges per chunk (0: per-kernel defaults)
    bool keep_xbf = false;           // option GATGPU_OPT_KEEP_INPUT_BF16
    int fuse_next = 1;               // option GATGPU_OPT_FUSE_NEXT_PROJECTION (0 never, 1 large graphs, 2 always)
    gatgpu::SplitPlan plans[gatgpu::kPlans];
    hipEvent_t ev[16] = {};
    int cus = 256;  // compute units of the device
    gatgpu_static_times st{};  // wall times of the static steps
    void* scratch = nullptr;   // device address of this GPU's static scratch array (layer_static.hip)
};

namespace gatgpu {

int fail(gatgpu_ctx* c, int code, const std::string& msg);
int hip_fail(gatgpu_ctx* c, const char* what, hipError_t e);
#define HIPCHECK(ctx, expr)                                               \
    do {                                                                  \
        hipError_t _e = (expr);                                           \
        if (_e != hipSuccess) return ::gatgpu::hip_fail((ctx), #expr, _e); \
    } while (0)

// Row stride (elements) of Z for a layer of `heads` x `width / heads`.
int z_stride(int precision, int heads, int width, bool* r_in_z);
// What run_tf did: the FP32 input rows were rounded inside the projection
// (then b.xbf holds them only with b.keep_xbf); the one-head kernel wrote
// its rows through b.out_perm.
struct TfDone {
    bool fused_convert = false;
    bool out_perm_used = false;
};
// Projection + fused prescan/softmax/aggregation/normalise/ELU of layer l,
// transform-first, into the buffers of `b`.  Exactly one of src32 (FP32 rows
// [n][in]) and srcbf (bf16 rows [n][16 ksteps]) is set.  ev_base: first of 4
// events (start, after convert, after projection, after aggregate) or -1.
// fixed: the fixed-p operator (the layer's fixture p and den).
int run_tf(gatgpu_ctx* c, int l, int precision, bool hidden, const float* src32, const uint16_t* srcbf,
           int ev_base, bool fixed, const TfBufs& b, TfDone* done);

// Resolves the device address of the static scratch array of c->device
// (layer_static.hip) once per device; the device must be current.
int static_scratch_init(gatgpu_ctx* c);

}  // namespace gatgpu
