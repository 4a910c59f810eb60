// C ABI of the gfx950 GAT forward: context, device buffers, layer and model
// orchestration, HIP-event stage timing.  Declarations: include/gatgpu.h.
#include "gatgpu.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "context.hpp"

using namespace gatgpu;

namespace {
std::string g_create_error;  // message for failures before a context exists
}  // namespace

namespace gatgpu {

int fail(gatgpu_ctx* c, int code, const std::string& msg) {
    if (c) c->err = msg;
    else g_create_error = msg;
    return code;
}
int hip_fail(gatgpu_ctx* c, const char* what, hipError_t e) {
    return fail(c, e == hipErrorOutOfMemory ? GATGPU_ENOMEM : GATGPU_EDEVICE,
                std::string(what) + ": " + hipGetErrorString(e));
}

// Row stride (elements) of Z.  bf16: a multiple of 8 for 16-byte vector
// stores; a single-head layer with at most 60 features gets a 128-byte row
// (one cache line per gather) whose last 4 bytes hold R.  FP32: a multiple of 4.
int z_stride(int precision, int heads, int width, bool* r_in_z) {
    const bool rz = precision == GATGPU_BF16 && heads == 1 && width <= 60;
    if (r_in_z) *r_in_z = rz;
    if (rz) return 64;
    return precision == GATGPU_BF16 ? (width + 7) / 8 * 8 : (width + 3) / 4 * 4;
}

}  // namespace gatgpu

namespace {

using Clock = std::chrono::steady_clock;
double ms_wall(Clock::time_point a, Clock::time_point b) {
    return std::chrono::duration<double, std::milli>(b - a).count();
}

bool mul_overflows(uint64_t a, uint64_t b) { return b && a > UINT64_MAX / b; }

bool all_finite(const float* p, uint64_t count, uint64_t* bad) {
    for (uint64_t i = 0; i < count; ++i)
        if (!std::isfinite(p[i])) {
            *bad = i;
            return false;
        }
    return true;
}

int bind(gatgpu_ctx* c) {
    HIPCHECK(c, hipSetDevice(c->device));
    return GATGPU_OK;
}

// Sorted-position boundaries of the degree bins.
int compute_bins(gatgpu_ctx* c) {
    // Thresholds: block bin, each plan's split degree, then the short rows.
    uint32_t thr[2 + kPlans] = {c->block_min ? c->block_min - 1 : 0};
    thr[1 + kPlans] = kShortDeg;
    uint32_t maxdeg = 0;  // degrees are sorted ascending
    if (c->n) HIPCHECK(c, hipMemcpy(&maxdeg, c->sorted_deg + (c->n - 1), 4, hipMemcpyDeviceToHost));
    const bool small = c->e < kSmallGraphEdges;
    for (int q = 0; q < kPlans; ++q) {
        SplitPlan& P = c->plans[q];
        const uint32_t min0 = small ? kSmallPlanMin : kPlanMin[q], chunk0 = small ? kSmallPlanChunk : kPlanChunk[q];
        uint32_t f = 1;
        while (uint64_t(chunk0) * f * kMaxChunksPerRow < maxdeg && f < (1u << 12)) f *= 2;
        const uint32_t min_scaled = q == kPlanVec ? min0 * f : std::max(min0, 2 * chunk0 * f);
        P.min = c->split_min ? c->split_min : min_scaled;
        P.chunk = c->split_chunk ? c->split_chunk : chunk0 * f;
        thr[1 + q] = P.min - 1;
    }
    // block_min 0 means every row takes a block.
    HIPCHECK(c, c->small.ensure(128));
    // small[]: [0,4) max degree, [8,16) neighbor steps, [16,36) thresholds, [40,80) positions
    uint32_t* dthr = reinterpret_cast<uint32_t*>(c->small.as<char>() + 16);
    uint64_t* dpos = reinterpret_cast<uint64_t*>(c->small.as<char>() + 40);
    HIPCHECK(c, hipMemcpyAsync(dthr, thr, sizeof(thr), hipMemcpyHostToDevice, c->stream));
    HIPCHECK(c, launch_count_le(c->sorted_deg, c->n, dthr, 2 + kPlans, dpos, c->stream));
    uint64_t pos[2 + kPlans];
    HIPCHECK(c, hipMemcpyAsync(pos, dpos, sizeof(pos), hipMemcpyDeviceToHost, c->stream));
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    RowBins b;
    b.n = c->n;
    b.block_begin = c->block_min ? pos[0] : 0;
    b.short_end = pos[1 + kPlans];
    c->bins = b;
    std::vector<uint64_t> prow;
    for (int q = 0; q < kPlans; ++q) {
        SplitPlan& P = c->plans[q];
        P.bins = b;
        P.bins.split_begin = pos[1 + q] < b.block_begin ? b.block_begin : pos[1 + q];
        // Chunk table of the split rows, heaviest row first.
        const uint64_t split_begin = P.bins.split_begin;
        const uint64_t nsplit = b.n - split_begin;
        prow.resize(nsplit + 1);
        if (nsplit)
            HIPCHECK(c, hipMemcpy(prow.data(), c->prow.as<uint64_t>() + split_begin, (nsplit + 1) * 8,
                                  hipMemcpyDeviceToHost));
        std::vector<uint32_t> ck, cf;
        for (uint64_t r = nsplit; r-- > 0;) {
            const uint64_t deg = prow[r + 1] - prow[r];
            const uint64_t nch = (deg + P.chunk - 1) / P.chunk;
            const uint32_t first = uint32_t(ck.size());
            for (uint64_t t = 0; t < nch; ++t) {
                ck.push_back(uint32_t(split_begin + r));
                cf.push_back(first);
            }
        }
        SplitTable& t = P.table;
        t = SplitTable{};
        t.chunks = ck.size();
        t.chunk_edges = P.chunk;
        if (t.chunks) {
            HIPCHECK(c, P.k.ensure(ck.size() * 4));
            HIPCHECK(c, P.first.ensure(cf.size() * 4));
            HIPCHECK(c, P.mchunk.ensure(ck.size() * 8 * 4));
            HIPCHECK(c, P.part.ensure(ck.size() * (8 * 128 + 24) * 4));  // largest partial: aggregate-first U
            HIPCHECK(c, hipMemcpy(P.k.p, ck.data(), ck.size() * 4, hipMemcpyHostToDevice));
            HIPCHECK(c, hipMemcpy(P.first.p, cf.data(), cf.size() * 4, hipMemcpyHostToDevice));
            t.chunk_k = P.k.as<uint32_t>();
            t.chunk_first = P.first.as<uint32_t>();
            t.mchunk = P.mchunk.as<float>();
            t.part = P.part.as<float>();
        }
        // Arrivals of the split rows at their first chunks, then the two tile
        // counters of the aggregate-first sum form.
        HIPCHECK(c, P.counter.ensure((ck.size() + 2) * 4));
        HIPCHECK(c, hipMemset(P.counter.p, 0, (ck.size() + 2) * 4));
        t.counter = P.counter.as<uint32_t>();
    }
    return GATGPU_OK;
}

int build_schedule(gatgpu_ctx* c) {
    const uint64_t n = c->n;
    HIPCHECK(c, c->keys_a.ensure(n * 4));
    HIPCHECK(c, c->keys_b.ensure(n * 4));
    HIPCHECK(c, c->vals_a.ensure(n * 4));
    HIPCHECK(c, c->vals_b.ensure(n * 4));
    HIPCHECK(c, c->hist.ensure(radix_tile_hist_elems(n) * 4));
    HIPCHECK(c, c->scan_tmp.ensure(scan_tmp_bytes(n)));
    HIPCHECK(c, c->small.ensure(64));
    uint32_t* dmax = c->small.as<uint32_t>();
    HIPCHECK(c, hipMemsetAsync(dmax, 0, 4, c->stream));
    HIPCHECK(c, launch_degrees_and_ids(c->row.as<uint64_t>(), c->keys_a.as<uint32_t>(),
                                       c->vals_a.as<uint32_t>(), n, dmax, c->stream));
    uint32_t maxdeg = 0;
    HIPCHECK(c, hipMemcpyAsync(&maxdeg, dmax, 4, hipMemcpyDeviceToHost, c->stream));
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    c->max_degree = maxdeg;
    int bits = 0;
    while (bits < 32 && (maxdeg >> bits)) ++bits;
    const int passes = bits == 0 ? 1 : (bits + 7) / 8;
    HIPCHECK(c, radix_sort_by_degree(c->keys_a.as<uint32_t>(), c->vals_a.as<uint32_t>(),
                                     c->keys_b.as<uint32_t>(), c->vals_b.as<uint32_t>(),
                                     c->hist.as<uint32_t>(), n, passes, c->scan_tmp.p, c->stream,
                                     &c->sorted_deg, &c->perm));
    HIPCHECK(c, c->prow.ensure((n + 1) * 8));
    HIPCHECK(c, c->pcol.ensure((c->e + kPcolPad) * 4));
    HIPCHECK(c, hipMemsetAsync(c->pcol.as<uint32_t>() + c->e, 0, kPcolPad * 4, c->stream));
    HIPCHECK(c, exclusive_scan_u32_to_u64(c->sorted_deg, c->prow.as<uint64_t>(), n, c->scan_tmp.p,
                                          c->stream));
    HIPCHECK(c, hipMemcpyAsync(c->prow.as<uint64_t>() + n, &c->e, 8, hipMemcpyHostToDevice, c->stream));
    HIPCHECK(c, launch_permute_cols(c->row.as<uint64_t>(), c->col.as<uint32_t>(), c->perm,
                                    c->prow.as<uint64_t>(), c->pcol.as<uint32_t>(), n, c->e, c->stream));
    HIPCHECK(c, c->invperm.ensure(n * 4));
    HIPCHECK(c, c->ident.ensure(n * 4));
    HIPCHECK(c, c->rcol.ensure((c->e + kPcolPad) * 4));
    HIPCHECK(c, hipMemsetAsync(c->rcol.as<uint32_t>() + c->e, 0, kPcolPad * 4, c->stream));
    HIPCHECK(c, launch_relabel(c->perm, c->pcol.as<uint32_t>(), c->invperm.as<uint32_t>(), c->ident.as<uint32_t>(),
                               c->rcol.as<uint32_t>(), n, c->e, c->stream));
    c->perm_h.resize(n);
    HIPCHECK(c, hipMemcpyAsync(c->perm_h.data(), c->perm, n * 4, hipMemcpyDeviceToHost, c->stream));
    uint64_t* dsteps = reinterpret_cast<uint64_t*>(c->small.as<char>() + 8);
    HIPCHECK(c, hipMemsetAsync(dsteps, 0, 8, c->stream));
    HIPCHECK(c, launch_neighbor_steps(c->sorted_deg, n, dsteps, c->stream));
    HIPCHECK(c, hipMemcpyAsync(&c->neighbor_steps, dsteps, 8, hipMemcpyDeviceToHost, c->stream));
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    return compute_bins(c);
}

// AUTO selects aggregate-first where its sum form applies (bf16, 8 heads of
// 32 or 64, D_in <= 128: it gathers 256-byte input rows, plus R from its own
// array beyond 112 inputs, instead of 512- or 1024-byte Z rows) and the Z
// table would not fit the 256 MB Infinity Cache, so that transform-first
// gathers would come from HBM; transform-first everywhere else.  Measured:
// 64.3M-edge graph, 100 -> 8 x 32 (Z 1.25 GB): 5.9 ms against 6.8 ms for
// transform-first; R-MAT, 128 -> 8 x 64 (Z 4.3 GB): 8.4 ms against 17.9;
// 169K-node graph, 128 -> 8 x 32 (Z 87 MB): 0.30 ms against 0.29.
constexpr uint64_t kAfMinZBytes = uint64_t(256) << 20;
// fixed: the fixed-p operator, whose aggregate-first form is the neighbour-step kernel only.
int resolve_dataflow(const LayerState& L, int precision, int dataflow, uint64_t n, bool fixed = false) {
    const bool bf16 = precision == GATGPU_BF16;
    const bool sum_ok = bf16 && !fixed && aggregate_afsum_supported(L.in, L.heads, L.dim, n);
    const bool step_ok = bf16 && aggregate_af_supported(L.in, L.heads, L.dim);  // neighbour-step kernel
    if (dataflow == GATGPU_AUTO)
        return sum_ok && n * uint64_t(L.heads) * uint64_t(L.dim) * 2 > kAfMinZBytes ? GATGPU_AGGREGATE_FIRST
                                                                                  : GATGPU_TRANSFORM_FIRST;
    if (dataflow == GATGPU_AGGREGATE_FIRST && !sum_ok && !step_ok) return -1;
    if (dataflow == GATGPU_TFS_B1 && !step_ok) return -1;
    return dataflow;
}

float ms_between(hipEvent_t a, hipEvent_t b) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, a, b) != hipSuccess) return 0.0f;
    return ms;
}

// Rows of `width` floats at `stride` on the device to the dense host array
// [n][width]: one copy, or, for padded rows (the one-head kernel's logits),
// packed on the device first (identity gather into the logits buffer).
int download_rows_dense(gatgpu_ctx* c, float* host, const void* src, uint64_t stride, uint32_t width) {
    if (stride != width) {
        HIPCHECK(c, c->logits.ensure(c->n * uint64_t(width) * 4));
        HIPCHECK(c, launch_gather_rows(src, stride, c->logits.p, width, c->ident.as<uint32_t>(), c->n, c->n, width,
                                       c->stream));
        src = c->logits.p;
    }
    HIPCHECK(c, hipMemcpyAsync(host, src, c->n * uint64_t(width) * 4, hipMemcpyDeviceToHost, c->stream));
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    return GATGPU_OK;
}

// Aggregate-first bf16 layer: convert the input to bf16 rows of 128, the
// L/R-only MFMA front end (reordered contraction), then the aggregate-first
// kernels (tiles of 32 rows + split-row chunks).
int run_layer_af(gatgpu_ctx* c, int l, bool hidden, const float* src32, const uint16_t* srcbf, int ev_base,
                 int dataflow, bool fixed) {
    LayerState& Ls = c->L[l];
    if (fixed) hidden = false;
    const uint64_t n = c->n;
    const int K = Ls.heads, W = Ls.width(), D = Ls.in, xs = af_input_stride();
    HIPCHECK(c, Ls.left.ensure(n * K * 4));
    HIPCHECK(c, Ls.right.ensure(n * K * 4));
    HIPCHECK(c, Ls.mx.ensure(n * K * 4));
    HIPCHECK(c, Ls.den.ensure(n * K * 4));
    if (hidden) HIPCHECK(c, Ls.outbf.ensure(n * W * 2));
    else HIPCHECK(c, Ls.out32.ensure((n * W + kF32Pad) * 4));
    if (srcbf && D != xs) {  // chained bf16 input in another row layout
        HIPCHECK(c, Ls.in32.ensure((n * D + kF32Pad) * 4));
        HIPCHECK(c, launch_widen_bf16(srcbf, Ls.in32.as<float>(), n * D, c->stream));
        src32 = Ls.in32.as<float>();
        srcbf = nullptr;
    }
    if (src32) HIPCHECK(c, Ls.inbf.ensure(n * xs * 2));
    const bool rounds_input = src32 != nullptr;  // the rounded rows land in inbf
    // The fixed-p operator has no row max (the reference leaves it unset).
    if (fixed) HIPCHECK(c, hipMemsetAsync(Ls.mx.p, 0, n * K * 4, c->stream));
    // Sum form: the gather table is the bf16 input rows, with R in their tail
    // up to 112 inputs (beyond, the rows are full and R stays in its array).
    const bool sum_form = !fixed && dataflow == GATGPU_AGGREGATE_FIRST && aggregate_afsum_supported(D, K, Ls.dim, n);
    const bool r_tail = sum_form && D <= kXRFeat;
    ProjArgs pa{};
    pa.n = n;
    pa.ksteps = Ls.lr_ksteps;
    pa.wpk = Ls.wlr.as<uint4>();
    pa.groups = 1;
    pa.head_blocks = 0;
    pa.nmb = 2;
    // FP32 input, sum form: the L/R projection rounds the rows itself and
    // writes them into the gather table (the convert stage fused); with 7 k
    // steps it writes all 112 feature slots, zero past D (8 k steps: all 128).
    const bool fused_convert = sum_form && src32 && D % 4 == 0 &&
                               Ls.lr_ksteps * 16 == (r_tail ? kXRFeat : kXRStride) && projection_fp32_input(pa);
    if (ev_base >= 0) HIPCHECK(c, hipEventRecord(c->ev[ev_base], c->stream));
    if (src32 && !fused_convert) {
        HIPCHECK(c, launch_to_bf16_pad(src32, Ls.inbf.as<uint16_t>(), n, D, xs, c->stream));
        srcbf = Ls.inbf.as<uint16_t>();
    }
    if (ev_base >= 0) HIPCHECK(c, hipEventRecord(c->ev[ev_base + 1], c->stream));
    if (fused_convert) {
        pa.x32 = src32;
        pa.in = D;
        pa.xs = D;
        pa.xout = Ls.inbf.as<uint16_t>();
        pa.xouts = xs;
    } else {
        pa.x = srcbf;
        pa.xs = xs;
    }
    pa.width = 0;
    pa.heads = K;
    pa.left = Ls.left.as<float>();
    pa.right = Ls.right.as<float>();
    pa.tiles = (n + 31) / 32;
    if (r_tail) {  // R also goes into the tail of each input row
        pa.z = Ls.inbf.as<uint16_t>();
        pa.zs = kXRStride;
        pa.r_in_z = true;
        pa.r_off = kXRFeat;
    }
    HIPCHECK(c, launch_projection_mfma(pa, c->stream, c->cus));
    if (ev_base >= 0) HIPCHECK(c, hipEventRecord(c->ev[ev_base + 2], c->stream));
    if (sum_form) {
        AfsArgs a{};
        a.prow = c->prow.as<uint64_t>();
        a.pcol = c->rcol.as<uint32_t>();
        a.perm = c->ident.as<uint32_t>();
        a.L = Ls.left.as<float>();
        a.R = Ls.right.as<float>();
        // The rounded input rows: written by the fused convert, else the
        // converted (or chained bf16) rows the front end read.
        a.xr = reinterpret_cast<const uint32_t*>(fused_convert ? Ls.inbf.as<uint16_t>() : srcbf);
        a.wpk = Ls.wpk.as<uint4>();
        a.nmb = Ls.nmb;
        a.ksteps = Ls.ksteps;
        a.wq = Ls.wq32.as<float>();
        a.in = D;
        a.dim = Ls.dim;
        a.hidden = hidden;
        a.mx = Ls.mx.as<float>();
        a.den = Ls.den.as<float>();
        a.out32 = hidden ? nullptr : Ls.out32.as<float>();
        a.outbf = hidden ? Ls.outbf.as<uint16_t>() : nullptr;
        a.n = n;
        a.e = c->e;
        const SplitPlan& P = c->plans[kPlanAf];
        a.rows = P.bins.split_begin;
        a.short_rows = std::min(P.bins.short_end, a.rows);
        a.chunks = P.table.chunks;
        a.chunk_k = P.table.chunk_k;
        a.chunk_first = P.table.chunk_first;
        a.chunk_edges = P.table.chunk_edges;
        a.mchunk = P.table.mchunk;
        a.part = P.table.part;
        a.counter = P.table.counter;
        HIPCHECK(c, launch_aggregate_afsum(a, P.table, c->stream, c->cus));
    } else {
    AfArgs a{};
    a.prow = c->prow.as<uint64_t>();
    a.pcol = c->rcol.as<uint32_t>();
    a.perm = c->ident.as<uint32_t>();
    a.L = Ls.left.as<float>();
    a.R = Ls.right.as<float>();
    a.X = srcbf;
    a.wpk = Ls.wpk.as<uint4>();
    a.nmb = Ls.nmb;
    a.ksteps = Ls.ksteps;
    a.wq = Ls.wq32.as<float>();
    a.in = D;
    a.heads = K;
    a.hidden = hidden;
    a.mx = Ls.mx.as<float>();
    a.den = Ls.den.as<float>();
    a.out32 = hidden ? nullptr : Ls.out32.as<float>();
    a.outbf = hidden ? Ls.outbf.as<uint16_t>() : nullptr;
    a.n = n;
    a.e = c->e;
    const SplitPlan& P = c->plans[kPlanAf];
    a.rows = P.bins.split_begin;
    a.tiles = (a.rows + 31) / 32;
    a.chunks = P.table.chunks;
    a.chunk_k = P.table.chunk_k;
    a.chunk_first = P.table.chunk_first;
    a.chunk_edges = P.table.chunk_edges;
    a.mchunk = P.table.mchunk;
    a.part = P.table.part;
    a.counter = P.table.counter;
    a.b1 = dataflow == GATGPU_TFS_B1;
    a.fixp = fixed ? Ls.fixp.as<float>() : nullptr;
    a.fixden = fixed ? Ls.fixden.as<float>() : nullptr;
    HIPCHECK(c, launch_aggregate_af(a, c->stream, c->cus));
    }
    if (ev_base >= 0) HIPCHECK(c, hipEventRecord(c->ev[ev_base + 3], c->stream));
    Ls.out_original = false;
    Ls.out_stride = W;
    Ls.xbf_valid = rounds_input;
    Ls.xbf_stride = xs;
    Ls.ran = true;
    Ls.precision = GATGPU_BF16;
    Ls.dataflow = dataflow;
    Ls.z_valid = false;
    Ls.out32_valid = !hidden;
    Ls.outbf_valid = hidden;
    return GATGPU_OK;
}

// Host rows [n][width] FP32 in original node order to device rows in sorted
// node order (dst row k = host row perm[k]).  Staged through a device buffer;
// returns after the copy is enqueued and the staging buffer is released by a
// stream synchronisation.
hipError_t upload_rows_sorted(gatgpu_ctx* c, const float* host, int width, void* dst) {
    const uint64_t n = c->n;
    DevBuf tmp;
    hipError_t e = tmp.ensure(n * uint64_t(width) * 4);
    if (e != hipSuccess) return e;
    if ((e = hipMemcpyAsync(tmp.p, host, n * uint64_t(width) * 4, hipMemcpyHostToDevice, c->stream)) != hipSuccess)
        return e;
    if ((e = launch_gather_rows(tmp.p, uint64_t(width), dst, uint64_t(width), c->perm, n, n, uint32_t(width),
                                c->stream)) != hipSuccess)
        return e;
    return hipStreamSynchronize(c->stream);
}

// Device rows [n][stride] in sorted node order, `width` elements of `esize`
// bytes each, to host rows [n][width] in original order.
template <class T>
int download_rows_original(gatgpu_ctx* c, const void* src, uint64_t stride, int width, std::vector<T>& out) {
    const uint64_t n = c->n;
    std::vector<T> tmp(n * stride);
    HIPCHECK(c, hipMemcpy(tmp.data(), src, tmp.size() * sizeof(T), hipMemcpyDeviceToHost));
    out.resize(n * uint64_t(width));
    for (uint64_t k = 0; k < n; ++k)
        std::memcpy(&out[uint64_t(c->perm_h[k]) * width], &tmp[k * stride], size_t(width) * sizeof(T));
    return GATGPU_OK;
}

// x32 = the features in sorted node order (row k = original row perm[k]),
// with kF32Pad floats of zero padding.
int sort_features(gatgpu_ctx* c) {
    const uint64_t n = c->n;
    const int din = c->din;
    HIPCHECK(c, c->x32.ensure((n * din + kF32Pad) * 4));
    HIPCHECK(c, launch_gather_rows(c->xorig.p, uint64_t(din), c->x32.p, uint64_t(din), c->perm, n, n, uint32_t(din),
                                   c->stream));
    HIPCHECK(c, hipMemsetAsync(c->x32.as<float>() + n * din, 0, kF32Pad * 4, c->stream));
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    return GATGPU_OK;
}

// Runs layer l on the device.  ev_base: first of 4 events (start, after
// convert, after projection, after aggregate) or -1 for no timing.
// orig_out: write the FP32 output rows in original node order where the
// aggregation kernel can (the one-head kernel); Ls.out_original tells.
// Layer l's aggregation can carry layer l + 1's projection (model forward):
// both transform-first bf16, layer l of 8 heads x 32 whose projection takes
// the fast path (R then comes from its bf16 Z rows), layer l + 1 of one head
// of at most 60 columns over those 256 inputs (Z rows of 64 with R inside).
bool can_fuse_next(const gatgpu_ctx* c, int l, int precision, const int (&flows)[3]) {
    if (precision != GATGPU_BF16 || l < 0 || l > 1) return false;
    if (flows[l] != GATGPU_TRANSFORM_FIRST || flows[l + 1] != GATGPU_TRANSFORM_FIRST) return false;
    const LayerState& A = c->L[l];
    const LayerState& B = c->L[l + 1];
    const bool a_fast = A.groups == 1 && ((A.ksteps >= 1 && A.ksteps <= 8) || A.ksteps == 16);
    bool r_in_z = false;
    (void)z_stride(precision, B.heads, B.width(), &r_in_z);
    return A.heads == 8 && A.dim == 32 && a_fast && B.heads == 1 && r_in_z && B.in == 256 && B.ksteps == 16 &&
           B.groups == 1 && B.nmb > (B.width() + 31) / 32;
}

// fuse: kFuseNone; kFuseNext: this layer's aggregation also projects its
// output rows with layer l + 1's weights (launch_aggregate_vec_next);
// kProjected: layer l's Z, L and R were written that way by layer l - 1.
enum { kFuseNone = 0, kFuseNext = 1, kProjected = 2 };

int run_layer(gatgpu_ctx* c, int l, int precision, int dataflow, bool hidden, const float* host_input,
              int ev_base, bool fixed = false, bool orig_out = false, int fuse = kFuseNone) {
    LayerState& Ls = c->L[l];
    const uint64_t n = c->n;
    const int K = Ls.heads, W = Ls.width(), D = Ls.in;
    // ---- input (explicit host input is uploaded before the timed region)
    const float* src32 = nullptr;
    const uint16_t* srcbf = nullptr;
    if (fuse == kProjected) {
        // the input rows were consumed by the previous layer's epilogue
    } else if (host_input) {
        HIPCHECK(c, Ls.in32.ensure((n * D + kF32Pad) * 4));
        HIPCHECK(c, upload_rows_sorted(c, host_input, D, Ls.in32.p));
        HIPCHECK(c, hipMemsetAsync(Ls.in32.as<float>() + n * D, 0, kF32Pad * 4, c->stream));
        src32 = Ls.in32.as<float>();
    } else if (l == 0) {
        if (!c->input) return fail(c, GATGPU_ESTATE, "node features not set");
        if (c->din != D) return fail(c, GATGPU_EINVAL, "layer 0 input width differs from the features");
        src32 = c->x32.as<float>();
    } else {
        LayerState& P = c->L[l - 1];
        if (!P.ran || P.precision != precision)
            return fail(c, GATGPU_ESTATE, "previous layer has no output in this precision");
        if (P.width() != D) return fail(c, GATGPU_EINVAL, "layer input width differs from the previous output");
        if (precision == GATGPU_BF16 && P.outbf_valid) srcbf = P.outbf.as<uint16_t>();
        else if (P.out32_valid) src32 = P.out32.as<float>();
        else return fail(c, GATGPU_ESTATE, "previous layer output missing");
    }
    if (dataflow == GATGPU_AGGREGATE_FIRST || dataflow == GATGPU_TFS_B1)
        return run_layer_af(c, l, hidden, src32, srcbf, ev_base, dataflow, fixed);
    // ---- outputs
    HIPCHECK(c, Ls.left.ensure(n * K * 4));
    HIPCHECK(c, Ls.right.ensure(n * K * 4));
    HIPCHECK(c, Ls.mx.ensure(n * K * 4));
    HIPCHECK(c, Ls.den.ensure(n * K * 4));
    const bool bf16 = precision == GATGPU_BF16;
    const bool want_outbf = bf16 && hidden && !fixed;
    // FP32 rows written to original node order by the one-head kernel take
    // the kernel's padded stride: whole lines per scattered row.
    const int ostride = orig_out && !want_outbf && !fixed && K == 1 && W <= 64 ? k1_out_stride(bf16, W) : W;
    if (want_outbf) HIPCHECK(c, Ls.outbf.ensure(n * W * 2));
    else HIPCHECK(c, Ls.out32.ensure((n * uint64_t(ostride > W ? ostride : W) + kF32Pad) * 4));
    // bf16 path: X as [n][xs] bf16 (xs = ksteps*16, zero-padded), Z as [n][zs]
    // bf16 (zs = W rounded up to 8 for aligned vector stores).
    const int xs = Ls.ksteps * 16;
    const int zs = z_stride(precision, K, W, nullptr);
    if (bf16) {
        HIPCHECK(c, Ls.zbf.ensure(n * zs * 2));
        if (fuse != kProjected && srcbf && D != xs) {  // chained bf16 input without the padded layout
            HIPCHECK(c, Ls.in32.ensure((n * D + kF32Pad) * 4));
            HIPCHECK(c, launch_widen_bf16(srcbf, Ls.in32.as<float>(), n * D, c->stream));
            src32 = Ls.in32.as<float>();
            srcbf = nullptr;
        }
        if (src32) HIPCHECK(c, Ls.inbf.ensure(n * xs * 2));
    } else {
        HIPCHECK(c, Ls.z32.ensure(n * zs * 4));
    }
    TfBufs b;
    b.pcol = c->rcol.as<uint32_t>();
    b.perm = c->ident.as<uint32_t>();
    b.left = Ls.left.as<float>();
    b.right = Ls.right.as<float>();
    b.mx = Ls.mx.as<float>();
    b.den = Ls.den.as<float>();
    b.z = bf16 ? Ls.zbf.p : Ls.z32.p;
    b.xbf = Ls.inbf.as<uint16_t>();
    b.out32 = want_outbf ? nullptr : Ls.out32.as<float>();
    b.outbf = want_outbf ? Ls.outbf.as<uint16_t>() : nullptr;
    b.fused_convert_ok = true;  // the context's FP32 buffers carry kF32Pad floats of padding
    b.keep_xbf = c->keep_xbf;
    // Layer 3's one-head kernel writes its FP32 rows straight to original rows.
    if (orig_out && b.out32 && !fixed) {
        b.out_perm = c->perm;
        b.ostride = ostride;
    }
    NextProj nx;
    if (fuse == kFuseNext) {
        LayerState& N = c->L[l + 1];
        HIPCHECK(c, N.zbf.ensure(n * 64 * 2));
        HIPCHECK(c, N.left.ensure(n * 4));
        HIPCHECK(c, N.right.ensure(n * 4));
        nx.wpk = N.wpk.as<uint4>();
        nx.nmb = N.nmb;
        nx.head_blocks = (N.width() + 31) / 32;
        nx.z = N.zbf.as<uint16_t>();
        nx.left = N.left.as<float>();
        nx.right = N.right.as<float>();
        b.next = &nx;
    }
    b.projected = fuse == kProjected;
    TfDone done;
    if (int r = run_tf(c, l, precision, hidden, src32, srcbf, ev_base, fixed, b, &done)) return r;
    Ls.ran = true;
    Ls.precision = precision;
    Ls.dataflow = GATGPU_TRANSFORM_FIRST;
    Ls.z_valid = true;
    // With the next projection fused, only the split rows store their output.
    Ls.out32_valid = !want_outbf;
    Ls.outbf_valid = want_outbf && fuse != kFuseNext;
    Ls.out_original = done.out_perm_used;
    Ls.out_stride = done.out_perm_used ? ostride : W;
    Ls.xbf_valid = bf16 && src32 && (!done.fused_convert || c->keep_xbf);
    Ls.xbf_stride = xs;
    return GATGPU_OK;
}

}  // namespace

namespace gatgpu {

int run_tf(gatgpu_ctx* c, int l, int precision, bool hidden, const float* src32, const uint16_t* srcbf,
           int ev_base, bool fixed, const TfBufs& b, TfDone* done) {
    LayerState& Ls = c->L[l];
    const uint64_t n = c->n;
    const int K = Ls.heads, dim = Ls.dim, W = Ls.width(), D = Ls.in;
    const bool bf16 = precision == GATGPU_BF16;
    const int xs = Ls.ksteps * 16;
    bool r_in_z = false;
    const int zs = z_stride(precision, K, W, &r_in_z);
    // The fixed-p operator has no row max (the reference leaves it unset).
    if (fixed) HIPCHECK(c, hipMemsetAsync(b.mx, 0, n * K * 4, c->stream));
    if (ev_base >= 0) HIPCHECK(c, hipEventRecord(c->ev[ev_base], c->stream));
    // ---- projection arguments (bf16 path)
    ProjArgs pa{};
    pa.n = n;
    pa.xs = xs;
    pa.ksteps = Ls.ksteps;
    pa.wpk = Ls.wpk.as<uint4>();
    pa.groups = Ls.groups;
    pa.head_blocks = (W + 31) / 32;
    pa.nmb = Ls.nmb;
    pa.width = W;
    pa.heads = K;
    pa.z = static_cast<uint16_t*>(b.z);
    pa.zs = zs;
    pa.left = b.left;
    pa.right = b.right;
    pa.tiles = (n + 31) / 32;
    pa.r_in_z = r_in_z;
    pa.r_off = zs - 2;
    pa.ar = Ls.ar.as<float>();
    pa.al = Ls.al.as<float>();
    pa.r_from_z = bf16 && !fixed && r_from_z_supported(pa);
    // ---- convert (bf16 path, FP32 source only; a bf16 source was rounded in
    // the previous layer's epilogue, which equals convert() of that output).
    // Where the fast projection applies, the rounding happens in its loads.
    const bool fused = !b.projected && bf16 && src32 && b.fused_convert_ok && D % 4 == 0 &&
                       projection_fp32_input(pa);  // 16-byte aligned rows
    if (done) done->fused_convert = fused;
    if (b.projected) {
        // Z, L and R come from the previous layer's epilogue: no convert, no projection.
    } else if (bf16 && src32 && !fused) {
        HIPCHECK(c, launch_to_bf16_pad(src32, b.xbf, n, D, xs, c->stream));
        srcbf = b.xbf;
        src32 = nullptr;
    }
    if (ev_base >= 0) HIPCHECK(c, hipEventRecord(c->ev[ev_base + 1], c->stream));
    // ---- projection + L/R
    if (b.projected) {
        if (!bf16 || !r_in_z) return fail(c, GATGPU_EINVAL, "projected layer must be bf16 with R in its Z rows");
    } else if (bf16) {
        if (fused) {
            pa.x32 = src32;
            pa.xs = D;
            pa.in = D;
            if (b.keep_xbf) {  // the rounded rows also leave the kernel
                pa.xout = b.xbf;
                pa.xouts = xs;
            }
        } else {
            pa.x = srcbf;
        }
        HIPCHECK(c, launch_projection_mfma(pa, c->stream, c->cus));
    } else if (projection_f32_supported(D, K, dim)) {
        // FP32 MFMA: Z = X W and L/R = X B_LR (FP32 products and sums)
        ProjF32Args fa{};
        fa.x = src32;
        fa.n = n;
        fa.in = D;
        fa.xs = D;
        fa.wpk = Ls.wpk32.as<float>();
        fa.head_blocks = (W + 31) / 32;
        fa.width = W;
        fa.heads = K;
        fa.z = static_cast<float*>(b.z);
        fa.zs = zs;
        fa.left = b.left;
        fa.right = b.right;
        fa.tiles = (n + 31) / 32;
        HIPCHECK(c, launch_projection_f32(fa, c->stream));
    } else {
        HIPCHECK(c, launch_projection(src32, nullptr, Ls.w32.as<float>(), n, D, K, dim, Ls.al.as<float>(),
                                      Ls.ar.as<float>(), static_cast<float*>(b.z), nullptr, b.left, b.right,
                                      nullptr, zs, c->stream));
    }
    if (ev_base >= 0) HIPCHECK(c, hipEventRecord(c->ev[ev_base + 2], c->stream));
    // ---- fused prescan + softmax + aggregation + normalise + ELU
    AggArgs a{};
    a.prow = c->prow.as<uint64_t>();
    a.pcol = b.pcol;
    a.perm = b.perm;
    a.left = b.left;
    a.right = b.right;
    a.feat = b.z;
    a.feat_bf16 = bf16;
    a.fstride = zs;
    a.r_in_feat = r_in_z;
    a.heads = K;
    a.dim = dim;
    a.hidden = hidden;
    a.mx = b.mx;
    a.den = b.den;
    a.out32 = b.out32;
    a.outbf = b.outbf;
    a.n = c->n;
    a.e = c->e;
    a.r_from_z = pa.r_from_z;
    a.ar = Ls.ar.as<float>();
    const bool one_head = !fixed && !aggregate_vec_supported(a) && aggregate_k1_supported(a);
    if (one_head && a.out32) {
        a.out_perm = b.out_perm;
        a.ostride = b.ostride;
    }
    if (done) done->out_perm_used = a.out_perm != nullptr;
    // The one-head kernel takes its own split plan; the 8-head, generic and
    // fixed-p kernels the 8-head one.
    const SplitPlan& P = c->plans[one_head ? kPlanOne : kPlanVec];
    SplitTable t = P.table;
    if (b.mchunk) t.mchunk = b.mchunk;
    if (b.part) t.part = b.part;
    if (b.counter) t.counter = b.counter;
    if (b.next) {
        if (fixed || !aggregate_vec_next_supported(a, *b.next))
            return fail(c, GATGPU_EINVAL, "next-layer projection cannot be fused into this layer");
        HIPCHECK(c, launch_aggregate_vec_next(a, P.bins, t, *b.next, c->stream));
        // The split rows stored their output rows; the next layer's projection of them.
        const uint64_t s0 = P.bins.split_begin;
        if (s0 < n) {
            const LayerState& N = c->L[l + 1];
            ProjArgs np{};
            np.n = n - s0;
            np.xs = N.ksteps * 16;
            np.x = b.outbf + s0 * uint64_t(np.xs);
            np.ksteps = N.ksteps;
            np.wpk = N.wpk.as<uint4>();
            np.groups = N.groups;
            np.head_blocks = b.next->head_blocks;
            np.nmb = N.nmb;
            np.width = N.width();
            np.heads = N.heads;
            np.z = b.next->z + s0 * 64;
            np.zs = 64;
            np.left = b.next->left + s0;
            np.right = b.next->right + s0;
            np.tiles = (np.n + 31) / 32;
            np.r_in_z = true;
            np.r_off = 62;
            np.ar = N.ar.as<float>();
            HIPCHECK(c, launch_projection_mfma(np, c->stream, c->cus));
        }
    } else if (fixed) {
        HIPCHECK(c, launch_aggregate_fixed(a, Ls.fixp.as<float>(), Ls.fixden.as<float>(), P.bins, t, c->stream));
    } else {
        HIPCHECK(c, launch_aggregate_tf(a, P.bins, t, c->stream));
    }
    if (ev_base >= 0) HIPCHECK(c, hipEventRecord(c->ev[ev_base + 3], c->stream));
    return GATGPU_OK;
}

}  // namespace gatgpu

namespace {

void fill_times(gatgpu_ctx* c, int ev_base, gatgpu_times* t, int dataflow) {
    std::memset(t, 0, sizeof(*t));
    t->convert_ms = ms_between(c->ev[ev_base], c->ev[ev_base + 1]);
    // Transform-first: the MFMA projection with its fused L/R block.
    // Aggregate-first: the L/R front end only; the projection runs inside the
    // aggregation kernel and is counted in aggregate_ms.
    if (dataflow == GATGPU_AGGREGATE_FIRST || dataflow == GATGPU_TFS_B1)
        t->lr_ms = ms_between(c->ev[ev_base + 1], c->ev[ev_base + 2]);
    else t->projection_ms = ms_between(c->ev[ev_base + 1], c->ev[ev_base + 2]);
    t->aggregate_ms = ms_between(c->ev[ev_base + 2], c->ev[ev_base + 3]);
    t->total_ms = ms_between(c->ev[ev_base], c->ev[ev_base + 3]);
}

// Graph::validate (baseline/src/common.cpp:23-30) on the CSR arrays, plus
// the limits of this build: n < 2^31, e <= 2^40, in-degrees below 2^32 (the
// degree schedule sorts 32-bit degrees).  Rows are checked before sources.
int validate_csr(gatgpu_ctx* c, uint64_t n, uint64_t e, const uint64_t* row, const uint32_t* col) {
    if (!row || (e && !col)) return fail(c, GATGPU_EINVAL, "null CSR pointer");
    if (n == 0 || n > uint64_t(INT32_MAX)) return fail(c, GATGPU_EINVAL, "invalid graph sizes");
    if (e > (uint64_t(1) << 40)) return fail(c, GATGPU_EOVERFLOW, "edge count too large");
    if (row[0] != 0 || row[n] != e) return fail(c, GATGPU_EINVAL, "bad CSR bounds");
    for (uint64_t i = 0; i < n; ++i) {
        if (row[i] > row[i + 1]) return fail(c, GATGPU_EINVAL, "nonmonotone CSR");
        if (row[i + 1] - row[i] > UINT32_MAX)
            return fail(c, GATGPU_EOVERFLOW, "in-degree of row " + std::to_string(i) + " exceeds 2^32 - 1");
    }
    for (uint64_t k = 0; k < e; ++k)
        if (col[k] >= n) return fail(c, GATGPU_EINVAL, "source index out of bounds");
    return GATGPU_OK;
}

int check_ctx(gatgpu_ctx* c) {
    if (!c) return fail(nullptr, GATGPU_EINVAL, "null context");
    return bind(c);
}

}  // namespace

extern "C" {

int gatgpu_create(int device, gatgpu_ctx** out) {
    if (!out) return fail(nullptr, GATGPU_EINVAL, "null output pointer");
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
        return fail(nullptr, GATGPU_ENODEV, "no HIP device");
    if (device < 0 || device >= count) return fail(nullptr, GATGPU_ENODEV, "device ordinal out of range");
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess)
        return fail(nullptr, GATGPU_ENODEV, "cannot query device");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(nullptr, GATGPU_ENODEV, std::string("device is ") + prop.gcnArchName + ", need gfx950");
    auto* c = new (std::nothrow) gatgpu_ctx;
    if (!c) return fail(nullptr, GATGPU_ENOMEM, "host allocation failed");
    c->device = device;
    c->cus = prop.multiProcessorCount;
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return fail(nullptr, GATGPU_EDEVICE, "cannot create stream");
    }
    for (auto& e : c->ev)
        if (hipEventCreate(&e) != hipSuccess) {
            gatgpu_destroy(c);
            return fail(nullptr, GATGPU_EDEVICE, "cannot create events");
        }
    if (static_scratch_init(c) != GATGPU_OK) {
        const std::string msg = c->err;
        gatgpu_destroy(c);
        return fail(nullptr, GATGPU_EDEVICE, msg);
    }
    *out = c;
    return GATGPU_OK;
}

int gatgpu_destroy(gatgpu_ctx* c) {
    if (!c) return GATGPU_OK;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (auto& e : c->ev)
        if (e) (void)hipEventDestroy(e);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
    return GATGPU_OK;
}

const char* gatgpu_last_error(const gatgpu_ctx* c) { return c ? c->err.c_str() : g_create_error.c_str(); }

int gatgpu_validate_graph(uint64_t n, uint64_t e, const uint64_t* row, const uint32_t* col) {
    return validate_csr(nullptr, n, e, row, col);
}

int gatgpu_set_graph(gatgpu_ctx* c, uint64_t n, uint64_t e, const uint64_t* row, const uint32_t* col) {
    if (int r = check_ctx(c)) return r;
    auto t0 = Clock::now();
    if (int r = validate_csr(c, n, e, row, col)) return r;
    if (c->input && c->n != n) c->input = false;
    c->graph = false;
    for (auto& L : c->L) L.ran = L.fixed_set = false;
    c->n = n;
    c->e = e;
    auto t1 = Clock::now();
    HIPCHECK(c, c->row.ensure((n + 1) * 8));
    HIPCHECK(c, c->col.ensure(e * 4));
    HIPCHECK(c, hipMemcpyAsync(c->row.p, row, (n + 1) * 8, hipMemcpyHostToDevice, c->stream));
    if (e) HIPCHECK(c, hipMemcpyAsync(c->col.p, col, e * 4, hipMemcpyHostToDevice, c->stream));
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    auto t2 = Clock::now();
    if (int r = build_schedule(c)) return r;
    c->st.graph_check_ms = ms_wall(t0, t1);
    c->st.graph_h2d_ms = ms_wall(t1, t2);
    c->st.degree_sort_ms = ms_wall(t2, Clock::now());
    c->graph = true;
    if (c->input)  // the features follow the new node order
        if (int r = sort_features(c)) return r;
    return GATGPU_OK;
}

int gatgpu_set_layer(gatgpu_ctx* c, int layer, int in, int heads, int dim, const float* w,
                     const float* al, const float* ar) {
    if (int r = check_ctx(c)) return r;
    const auto t0 = Clock::now();
    if (layer < 0 || layer > 2) return fail(c, GATGPU_EINVAL, "layer must be 0, 1 or 2");
    if (in <= 0 || heads <= 0 || heads > 8 || dim <= 0 || dim > 64)
        return fail(c, GATGPU_EINVAL, "invalid parameter shape (heads <=8, head_dim <=64)");
    if (!w || !al || !ar) return fail(c, GATGPU_EINVAL, "null weight pointer");
    const uint64_t W = uint64_t(heads) * dim, wn = uint64_t(in) * W;
    uint64_t bad = 0;
    if (!all_finite(w, wn, &bad)) return fail(c, GATGPU_ENONFINITE, "nonfinite W index=" + std::to_string(bad));
    if (!all_finite(al, W, &bad)) return fail(c, GATGPU_ENONFINITE, "nonfinite aL index=" + std::to_string(bad));
    if (!all_finite(ar, W, &bad)) return fail(c, GATGPU_ENONFINITE, "nonfinite aR index=" + std::to_string(bad));
    LayerState& L = c->L[layer];
    L.set = false;
    L.ran = L.fixed_set = false;
    L.in = in;
    L.heads = heads;
    L.dim = dim;
    // Static preparation (prepare(), baseline/src/common.cpp:97-119): bf16
    // copy of W (kept as FP32 values) and B_LR = W a for the reordered front end.
    std::vector<float> wq(wn), blr(size_t(in) * 2 * heads);
    for (uint64_t i = 0; i < wn; ++i) wq[i] = bf16_widen(bf16_rne(w[i]));
    for (int k = 0; k < in; ++k)
        for (int h = 0; h < heads; ++h) {
            float l = 0, r = 0;
            for (int d = 0; d < dim; ++d) {
                const float wv = w[size_t(k) * W + h * dim + d];
                l += wv * al[h * dim + d];
                r += wv * ar[h * dim + d];
            }
            blr[size_t(k) * 2 * heads + h] = l;
            blr[size_t(k) * 2 * heads + heads + h] = r;
        }
    std::vector<uint16_t> packed;
    pack_projection_weights(wq.data(), al, ar, in, heads, dim, packed, L.ksteps, L.groups, L.nmb);
    HIPCHECK(c, L.wpk.ensure(packed.size() * 2));
    HIPCHECK(c, hipMemcpyAsync(L.wpk.p, packed.data(), packed.size() * 2, hipMemcpyHostToDevice, c->stream));
    std::vector<uint16_t> lrpacked;
    pack_lr_weights(wq.data(), al, ar, in, heads, dim, lrpacked, L.lr_ksteps);
    HIPCHECK(c, L.wlr.ensure(lrpacked.size() * 2));
    HIPCHECK(c, hipMemcpyAsync(L.wlr.p, lrpacked.data(), lrpacked.size() * 2, hipMemcpyHostToDevice, c->stream));
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    HIPCHECK(c, L.w32.ensure(wn * 4));
    HIPCHECK(c, L.wq32.ensure(wn * 4));
    HIPCHECK(c, L.al.ensure(W * 4));
    HIPCHECK(c, L.ar.ensure(W * 4));
    HIPCHECK(c, L.blr.ensure(blr.size() * 4));
    HIPCHECK(c, hipMemcpyAsync(L.w32.p, w, wn * 4, hipMemcpyHostToDevice, c->stream));
    HIPCHECK(c, hipMemcpyAsync(L.wq32.p, wq.data(), wn * 4, hipMemcpyHostToDevice, c->stream));
    HIPCHECK(c, hipMemcpyAsync(L.al.p, al, W * 4, hipMemcpyHostToDevice, c->stream));
    HIPCHECK(c, hipMemcpyAsync(L.ar.p, ar, W * 4, hipMemcpyHostToDevice, c->stream));
    HIPCHECK(c, hipMemcpyAsync(L.blr.p, blr.data(), blr.size() * 4, hipMemcpyHostToDevice, c->stream));
    std::vector<float> f32pk;
    if (projection_f32_supported(in, heads, dim)) {
        pack_projection_f32(w, blr.data(), in, heads, dim, f32pk);
        HIPCHECK(c, L.wpk32.ensure(f32pk.size() * 4));
        HIPCHECK(c, hipMemcpyAsync(L.wpk32.p, f32pk.data(), f32pk.size() * 4, hipMemcpyHostToDevice, c->stream));
    }
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    L.set = true;
    L.prepare_ms = ms_wall(t0, Clock::now());
    c->st.model_prepare_ms = 0;
    for (const auto& q : c->L)
        if (q.set) c->st.model_prepare_ms += q.prepare_ms;
    return GATGPU_OK;
}

int gatgpu_set_input(gatgpu_ctx* c, uint64_t n, int din, const float* x) {
    if (int r = check_ctx(c)) return r;
    if (!c->graph) return fail(c, GATGPU_ESTATE, "graph not set");
    if (n != c->n || din <= 0 || !x) return fail(c, GATGPU_EINVAL, "feature matrix does not match the graph");
    if (mul_overflows(n, uint64_t(din) * 4)) return fail(c, GATGPU_EOVERFLOW, "size overflow");
    const auto t0 = Clock::now();
    uint64_t bad = 0;
    if (!all_finite(x, n * din, &bad)) return fail(c, GATGPU_ENONFINITE, "nonfinite graph input index=" + std::to_string(bad));
    HIPCHECK(c, c->xorig.ensure(n * din * 4));
    HIPCHECK(c, hipMemcpyAsync(c->xorig.p, x, n * din * 4, hipMemcpyHostToDevice, c->stream));
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    const auto t1 = Clock::now();
    c->din = din;
    if (int r = sort_features(c)) return r;
    c->st.input_h2d_ms = ms_wall(t0, t1);
    c->st.input_permute_ms = ms_wall(t1, Clock::now());
    c->input = true;
    c->L[0].ran = false;
    return GATGPU_OK;
}

int gatgpu_degree_schedule(gatgpu_ctx* c, uint32_t* perm, uint64_t* steps) {
    if (int r = check_ctx(c)) return r;
    if (!c->graph) return fail(c, GATGPU_ESTATE, "graph not set");
    if (perm) HIPCHECK(c, hipMemcpy(perm, c->perm, c->n * 4, hipMemcpyDeviceToHost));
    if (steps) *steps = c->neighbor_steps;
    return GATGPU_OK;
}

int gatgpu_permuted_csr(gatgpu_ctx* c, uint64_t* prow, uint32_t* pcol) {
    if (int r = check_ctx(c)) return r;
    if (!c->graph) return fail(c, GATGPU_ESTATE, "graph not set");
    if (prow) HIPCHECK(c, hipMemcpy(prow, c->prow.p, (c->n + 1) * 8, hipMemcpyDeviceToHost));
    if (pcol && c->e) HIPCHECK(c, hipMemcpy(pcol, c->pcol.p, c->e * 4, hipMemcpyDeviceToHost));
    return GATGPU_OK;
}

int gatgpu_choose_R(gatgpu_ctx* c, int* r_out) {
    if (int r = check_ctx(c)) return r;
    if (!c->graph || !r_out) return fail(c, GATGPU_ESTATE, "graph not set");
    const double avg = double(c->e) / double(c->n);
    const double rho = avg ? c->max_degree / avg : 1.0;
    *r_out = rho < 32 ? 128 : rho < 1024 ? 64 : rho < 20000 ? 32 : 16;
    return GATGPU_OK;
}

int gatgpu_layer_forward(gatgpu_ctx* c, int layer, int precision, int dataflow, int hidden,
                         const float* input, gatgpu_times* times) {
    if (int r = check_ctx(c)) return r;
    if (layer < 0 || layer > 2) return fail(c, GATGPU_EINVAL, "layer must be 0, 1 or 2");
    if (precision != GATGPU_FP32 && precision != GATGPU_BF16) return fail(c, GATGPU_EINVAL, "bad precision");
    if (dataflow < GATGPU_AUTO || dataflow > GATGPU_TFS_B1) return fail(c, GATGPU_EINVAL, "bad dataflow");
    if (!c->graph) return fail(c, GATGPU_ESTATE, "graph not set");
    if (!c->L[layer].set) return fail(c, GATGPU_ESTATE, "layer weights not set");
    if (input) {
        uint64_t bad = 0;
        if (!all_finite(input, c->n * uint64_t(c->L[layer].in), &bad))
            return fail(c, GATGPU_ENONFINITE, "nonfinite layer input index=" + std::to_string(bad));
    }
    const int flow = resolve_dataflow(c->L[layer], precision, dataflow, c->n);
    if (flow < 0) return fail(c, GATGPU_EINVAL, "aggregate-first needs bf16 and in <= 128 with head_dim 32 (1/2/4/8 heads) or 8 heads of 64; TFS B1 head_dim 32");
    if (int r = run_layer(c, layer, precision, flow, hidden != 0, input, times ? 0 : -1)) return r;
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    HIPCHECK(c, hipGetLastError());
    if (times) fill_times(c, 0, times, c->L[layer].dataflow);
    return GATGPU_OK;
}

int gatgpu_set_fixed_p(gatgpu_ctx* c, int layer, const float* p, const float* den) {
    if (int r = check_ctx(c)) return r;
    if (layer < 0 || layer > 2) return fail(c, GATGPU_EINVAL, "layer must be 0, 1 or 2");
    if (!c->graph) return fail(c, GATGPU_ESTATE, "graph not set");
    LayerState& Ls = c->L[layer];
    if (!Ls.set) return fail(c, GATGPU_ESTATE, "layer weights not set");
    if ((c->e && !p) || !den) return fail(c, GATGPU_EINVAL, "null fixture pointer");
    Ls.fixed_set = false;
    const uint64_t n = c->n, e = c->e;
    const int K = Ls.heads;
    uint64_t bad = 0;
    if (!all_finite(p, e * K, &bad)) return fail(c, GATGPU_ENONFINITE, "nonfinite fixture p index=" + std::to_string(bad));
    if (!all_finite(den, n * K, &bad))
        return fail(c, GATGPU_ENONFINITE, "nonfinite fixture denominator index=" + std::to_string(bad));
    // load_fixture's checks (baseline/src/common.cpp:189-192): p in [0, 1], den
    // equal to the row's sum of p in edge order, positive on a non-empty row.
    std::vector<uint64_t> row(n + 1);
    HIPCHECK(c, hipMemcpy(row.data(), c->row.p, (n + 1) * 8, hipMemcpyDeviceToHost));
    for (uint64_t i = 0; i < n; ++i)
        for (int h = 0; h < K; ++h) {
            float sum = 0;
            for (uint64_t q = row[i]; q < row[i + 1]; ++q) {
                const float x = p[q * K + h];
                if (x < 0 || x > 1) return fail(c, GATGPU_EINVAL, "fixture p outside [0,1] at edge " + std::to_string(q));
                sum += x;
            }
            const float d = den[i * K + h];
            if (std::abs(sum - d) > 1e-5f * std::max(1.f, sum) || (row[i] != row[i + 1] && d <= 0))
                return fail(c, GATGPU_EINVAL, "fixture denominator mismatch at row " + std::to_string(i));
        }
    DevBuf tmp;
    HIPCHECK(c, tmp.ensure(e * K * 4));
    HIPCHECK(c, Ls.fixp.ensure(e * K * 4));
    HIPCHECK(c, Ls.fixden.ensure(n * K * 4));
    if (e) HIPCHECK(c, hipMemcpyAsync(tmp.p, p, e * K * 4, hipMemcpyHostToDevice, c->stream));
    HIPCHECK(c, upload_rows_sorted(c, den, K, Ls.fixden.p));
    HIPCHECK(c, launch_permute_edge_values(c->row.as<uint64_t>(), c->perm, c->prow.as<uint64_t>(), tmp.as<float>(),
                                           Ls.fixp.as<float>(), n, e, K, c->stream));
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    Ls.fixed_set = true;
    return GATGPU_OK;
}

int gatgpu_fixed_p_forward(gatgpu_ctx* c, int layer, int precision, int dataflow, const float* input,
                           gatgpu_times* times) {
    if (int r = check_ctx(c)) return r;
    if (layer < 0 || layer > 2) return fail(c, GATGPU_EINVAL, "layer must be 0, 1 or 2");
    if (precision != GATGPU_FP32 && precision != GATGPU_BF16) return fail(c, GATGPU_EINVAL, "bad precision");
    if (dataflow < GATGPU_AUTO || dataflow > GATGPU_TFS_B1) return fail(c, GATGPU_EINVAL, "bad dataflow");
    if (!c->graph) return fail(c, GATGPU_ESTATE, "graph not set");
    if (!c->L[layer].set) return fail(c, GATGPU_ESTATE, "layer weights not set");
    if (!c->L[layer].fixed_set) return fail(c, GATGPU_ESTATE, "fixture p/den not set for this layer");
    if (input) {
        uint64_t bad = 0;
        if (!all_finite(input, c->n * uint64_t(c->L[layer].in), &bad))
            return fail(c, GATGPU_ENONFINITE, "nonfinite layer input index=" + std::to_string(bad));
    }
    int flow = dataflow == GATGPU_AUTO ? GATGPU_TRANSFORM_FIRST : dataflow;
    if (flow != GATGPU_TRANSFORM_FIRST) {
        flow = resolve_dataflow(c->L[layer], precision, flow, c->n, true);
        if (flow < 0)
            return fail(c, GATGPU_EINVAL, "fixed-p aggregate-first needs bf16, head_dim 32, 1/2/4/8 heads and in <= 128");
    }
    if (int r = run_layer(c, layer, precision, flow, false, input, times ? 0 : -1, true)) return r;
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    HIPCHECK(c, hipGetLastError());
    if (times) fill_times(c, 0, times, flow);
    return GATGPU_OK;
}

int gatgpu_model_forward(gatgpu_ctx* c, int precision, int dataflow, float* logits, gatgpu_times* times,
                         double* total_ms) {
    if (int r = check_ctx(c)) return r;
    if (precision != GATGPU_FP32 && precision != GATGPU_BF16) return fail(c, GATGPU_EINVAL, "bad precision");
    if (dataflow < GATGPU_AUTO || dataflow > GATGPU_TFS_B1) return fail(c, GATGPU_EINVAL, "bad dataflow");
    if (!c->graph || !c->input) return fail(c, GATGPU_ESTATE, "graph or features not set");
    for (int l = 0; l < 3; ++l)
        if (!c->L[l].set) return fail(c, GATGPU_ESTATE, "layer weights not set");
    if (c->L[0].in != c->din || c->L[1].in != c->L[0].width() || c->L[2].in != c->L[1].width())
        return fail(c, GATGPU_EINVAL, "layer widths do not chain");
    // Per-stage events only when the caller asks for the per-layer times: each
    // event is a queue packet between kernels (13 of them cost 0.02-0.03 ms
    // per forward on the 2.5M-edge graph), so a total-only request records the
    // first and the last event alone.
    const bool stages = times != nullptr;
    const bool timed = stages || total_ms;
    int flows[3];
    for (int l = 0; l < 3; ++l) {
        // In the chained model, aggregate-first applies where the layer supports it.
        flows[l] = resolve_dataflow(c->L[l], precision, dataflow, c->n);
        if (flows[l] < 0) flows[l] = GATGPU_TRANSFORM_FIRST;
    }
    // Option 1 fuses on graphs of at least kSmallGraphEdges edges only.  On
    // smaller graphs each 32-row tile's waves aggregate their rows one after
    // another, and the tiles of the heaviest unsplit rows outlast the rest of
    // the launch: on the 2.5M-edge power-law graph the fused layer 2 took
    // 0.46 ms against 0.21 + 0.03 ms unfused.
    const bool fuse23 = (c->fuse_next == 2 || (c->fuse_next == 1 && c->e >= kSmallGraphEdges)) &&
                        can_fuse_next(c, 1, precision, flows);
    if (timed && !stages) HIPCHECK(c, hipEventRecord(c->ev[0], c->stream));
    for (int l = 0; l < 3; ++l) {
        const int fuse = !fuse23 ? kFuseNone : l == 1 ? kFuseNext : l == 2 ? kProjected : kFuseNone;
        if (int r = run_layer(c, l, precision, flows[l], l < 2, nullptr, stages ? 4 * l : -1, false, l == 2, fuse))
            return r;
    }
    // Logits in original node order, inside the timed forward: written so by
    // the last aggregation where it can, else gathered back (row i = sorted
    // row invperm[i]).
    const LayerState& L2 = c->L[2];
    const uint32_t C = uint32_t(L2.width());
    const void* logits_dev = L2.out32.p;
    if (!L2.out_original) {
        HIPCHECK(c, c->logits.ensure(c->n * C * 4));
        HIPCHECK(c, launch_gather_rows(L2.out32.p, C, c->logits.p, C, c->invperm.as<uint32_t>(), c->n, c->n, C,
                                       c->stream));
        logits_dev = c->logits.p;
    }
    if (timed) HIPCHECK(c, hipEventRecord(c->ev[12], c->stream));
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    HIPCHECK(c, hipGetLastError());
    if (times)
        for (int l = 0; l < 3; ++l) fill_times(c, 4 * l, &times[l], c->L[l].dataflow);
    if (total_ms) *total_ms = ms_between(c->ev[0], c->ev[12]);
    if (logits) {
        const auto t0 = Clock::now();
        if (int r = download_rows_dense(c, logits, logits_dev, L2.out_original ? uint64_t(L2.out_stride) : C, C))
            return r;
        c->st.logits_d2h_ms = ms_wall(t0, Clock::now());
    }
    return GATGPU_OK;
}

int gatgpu_get_static_times(gatgpu_ctx* c, gatgpu_static_times* out) {
    if (!c || !out) return fail(c, GATGPU_EINVAL, "null argument");
    *out = c->st;
    return GATGPU_OK;
}

int gatgpu_stage_size(gatgpu_ctx* c, int layer, int which, uint64_t* count) {
    if (int r = check_ctx(c)) return r;
    if (layer < 0 || layer > 2 || !count) return fail(c, GATGPU_EINVAL, "bad stage request");
    const LayerState& L = c->L[layer];
    *count = 0;
    if (!L.ran) return GATGPU_OK;
    switch (which) {
        case GATGPU_STAGE_Z:
            *count = L.z_valid ? c->n * L.width() : 0;
            break;
        case GATGPU_STAGE_LEFT:
        case GATGPU_STAGE_RIGHT:
        case GATGPU_STAGE_MAX:
        case GATGPU_STAGE_DEN:
            *count = c->n * L.heads;
            break;
        case GATGPU_STAGE_OUT:  // absent where the next projection was fused in
            *count = L.out32_valid || L.outbf_valid ? c->n * L.width() : 0;
            break;
        case GATGPU_STAGE_XBF:
            *count = L.xbf_valid ? c->n * L.in : 0;
            break;
        default:
            return fail(c, GATGPU_EINVAL, "bad stage selector");
    }
    return GATGPU_OK;
}

int gatgpu_get_stage(gatgpu_ctx* c, int layer, int which, float* host) {
    uint64_t count = 0;
    if (int r = gatgpu_stage_size(c, layer, which, &count)) return r;
    if (!count) return fail(c, GATGPU_ESTATE, "stage not available");
    if (!host) return fail(c, GATGPU_EINVAL, "null output");
    const LayerState& L = c->L[layer];
    const void* src = nullptr;
    bool bf = false;
    switch (which) {
        case GATGPU_STAGE_Z:
            bf = L.precision == GATGPU_BF16;
            src = bf ? L.zbf.p : L.z32.p;
            break;
        case GATGPU_STAGE_LEFT: src = L.left.p; break;
        case GATGPU_STAGE_RIGHT: src = L.right.p; break;
        case GATGPU_STAGE_MAX: src = L.mx.p; break;
        case GATGPU_STAGE_DEN: src = L.den.p; break;
        case GATGPU_STAGE_OUT:
            bf = !L.out32_valid;
            src = bf ? L.outbf.p : L.out32.p;
            break;
        case GATGPU_STAGE_XBF:
            bf = true;
            src = L.inbf.p;
            break;
    }
    // Device stages are in sorted node order; rows go back to original order.
    const int W = L.width();
    const int width = which == GATGPU_STAGE_XBF                             ? L.in
                      : (which == GATGPU_STAGE_Z || which == GATGPU_STAGE_OUT) ? W
                                                                               : L.heads;
    const uint64_t stride = which == GATGPU_STAGE_Z   ? uint64_t(z_stride(bf ? GATGPU_BF16 : GATGPU_FP32, L.heads, W, nullptr))
                            : which == GATGPU_STAGE_XBF ? uint64_t(L.xbf_stride)
                                                        : uint64_t(width);
    if (which == GATGPU_STAGE_OUT && !bf && L.out_original) {
        if (int r = download_rows_dense(c, host, src, uint64_t(L.out_stride), uint32_t(W))) return r;
    } else if (bf) {
        std::vector<uint16_t> rows;
        if (int r = download_rows_original(c, src, stride, width, rows)) return r;
        for (uint64_t i = 0; i < count; ++i) host[i] = bf16_widen(rows[i]);
    } else {
        std::vector<float> rows;
        if (int r = download_rows_original(c, src, stride, width, rows)) return r;
        std::memcpy(host, rows.data(), count * 4);
    }
    return GATGPU_OK;
}

int gatgpu_set_option(gatgpu_ctx* c, int key, int64_t value) {
    if (int r = check_ctx(c)) return r;
    if (value < 0 || value > int64_t(UINT32_MAX)) return fail(c, GATGPU_EINVAL, "option value out of range");
    switch (key) {
        case GATGPU_OPT_BLOCK_ROW_MIN_DEGREE: c->block_min = uint32_t(value); break;
        case GATGPU_OPT_SPLIT_ROW_MIN_DEGREE:  // 0: the per-kernel defaults
            c->split_min = uint32_t(value);
            break;
        case GATGPU_OPT_SPLIT_CHUNK_EDGES:  // 0: the per-kernel defaults
            if (value != 0 && value < 64) return fail(c, GATGPU_EINVAL, "split chunk must be >= 64 edges");
            c->split_chunk = uint32_t(value);
            break;
        case GATGPU_OPT_KEEP_INPUT_BF16:
            if (value > 1) return fail(c, GATGPU_EINVAL, "keep-input option is 0 or 1");
            c->keep_xbf = value != 0;
            return GATGPU_OK;
        case GATGPU_OPT_FUSE_NEXT_PROJECTION:
            if (value > 2) return fail(c, GATGPU_EINVAL, "fuse option is 0, 1 or 2");
            c->fuse_next = int(value);
            return GATGPU_OK;
        default: return fail(c, GATGPU_EINVAL, "unknown option");
    }
    if (c->graph) return compute_bins(c);
    return GATGPU_OK;
}

int gatgpu_synchronize(gatgpu_ctx* c) {
    if (int r = check_ctx(c)) return r;
    HIPCHECK(c, hipStreamSynchronize(c->stream));
    return GATGPU_OK;
}

void* gatgpu_stream(gatgpu_ctx* c) { return c ? static_cast<void*>(c->stream) : nullptr; }

}  // extern "C"
