// Allocation-free transform-first layer: gatgpu_layer_forward_static.
//
// Every intermediate of the layer (bf16 input rows, Z, L, R, max, den, the
// output before its final copy, split-row partial sums and arrival counters)
// lives in `scratch`, one static device array per GPU.  Its device address is
// resolved once per device by static_scratch_init (called from
// gatgpu_create with the device current); host code uses only that address,
// never the array's name.  The layer runs the same kernels as
// gatgpu_layer_forward, in original node order: the projection over the
// caller's rows as they are, the aggregation over the degree-sorted CSR with
// original source ids (pcol) and perm as its row permutation, so L, R, max,
// den and the output rows are indexed by original node.
#include <algorithm>
#include <mutex>

#include "context.hpp"

namespace {

constexpr uint64_t kScratchBytes = GATGPU_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

__global__ void k_fill_u32(uint32_t* p, uint64_t count, uint32_t v) {
    for (uint64_t i = blockIdx.x * uint64_t(blockDim.x) + threadIdx.x; i < count; i += uint64_t(gridDim.x) * blockDim.x)
        p[i] = v;
}

// Byte offsets of the intermediates inside the array (256-byte aligned).
struct StaticPlan {
    uint64_t xbf = 0, z = 0, left = 0, right = 0, mx = 0, den = 0, out = 0, mchunk = 0, part = 0, counter = 0;
    uint64_t chunks = 0, bytes = 0;
    bool outbf = false;
};

uint64_t take(uint64_t& at, uint64_t bytes) {
    const uint64_t off = at;
    at += (bytes + 255) / 256 * 256;
    return off;
}

StaticPlan plan_static(const gatgpu_ctx* c, int layer, int precision, bool hidden) {
    using namespace gatgpu;
    const LayerState& Ls = c->L[layer];
    const uint64_t n = c->n, K = uint64_t(Ls.heads), W = uint64_t(Ls.width());
    const bool bf16 = precision == GATGPU_BF16;
    const uint64_t zs = uint64_t(z_stride(precision, Ls.heads, Ls.width(), nullptr));
    StaticPlan p;
    uint64_t at = 0;
    if (bf16) p.xbf = take(at, n * uint64_t(Ls.ksteps) * 16 * 2);
    p.z = take(at, n * zs * (bf16 ? 2 : 4));
    p.left = take(at, n * K * 4);
    p.right = take(at, n * K * 4);
    p.mx = take(at, n * K * 4);
    p.den = take(at, n * K * 4);
    p.outbf = bf16 && hidden;
    p.out = take(at, p.outbf ? n * W * 2 : (n * W + kF32Pad) * 4);
    // Split rows of the 8-head and the one-head kernels' plans (whichever runs).
    p.chunks = std::max(c->plans[kPlanVec].table.chunks, c->plans[kPlanOne].table.chunks);
    p.mchunk = take(at, p.chunks * 8 * 4);
    p.part = take(at, p.chunks * kTfPartFloats * 4);
    p.counter = take(at, p.chunks * 4);
    p.bytes = at;
    return p;
}

int check_static_args(gatgpu_ctx* c, int layer, int precision) {
    using namespace gatgpu;
    if (!c) return fail(nullptr, GATGPU_EINVAL, "null context");
    if (layer < 0 || layer > 2) return fail(c, GATGPU_EINVAL, "layer must be 0, 1 or 2");
    if (precision != GATGPU_FP32 && precision != GATGPU_BF16) return fail(c, GATGPU_EINVAL, "bad precision");
    if (!c->graph) return fail(c, GATGPU_ESTATE, "graph not set");
    if (!c->L[layer].set) return fail(c, GATGPU_ESTATE, "layer weights not set");
    return GATGPU_OK;
}

}  // namespace

namespace gatgpu {

int static_scratch_init(gatgpu_ctx* c) {
    if (c->device < 0 || c->device >= kMaxDevices) return fail(c, GATGPU_ENODEV, "device ordinal beyond 63");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[c->device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(c, "hipGetSymbolAddress(scratch)", e);
        g_scratch_ptr[c->device] = p;
    }
    c->scratch = g_scratch_ptr[c->device];
    return GATGPU_OK;
}

}  // namespace gatgpu

extern "C" {

int gatgpu_static_scratch_need(gatgpu_ctx* c, int layer, int precision, int hidden, uint64_t* bytes) {
    if (int r = check_static_args(c, layer, precision)) return r;
    if (!bytes) return gatgpu::fail(c, GATGPU_EINVAL, "null output");
    *bytes = plan_static(c, layer, precision, hidden != 0).bytes;
    return GATGPU_OK;
}

int gatgpu_layer_forward_static(gatgpu_ctx* c, int layer, int precision, int hidden, const float* x, float* out) {
    using namespace gatgpu;
    if (int r = check_static_args(c, layer, precision)) return r;
    if (!x || !out) return fail(c, GATGPU_EINVAL, "null device pointer");
    if (!c->scratch) return fail(c, GATGPU_ESTATE, "static scratch array not resolved on this device");
    const StaticPlan p = plan_static(c, layer, precision, hidden != 0);
    if (p.bytes > kScratchBytes)
        return fail(c, GATGPU_EOVERFLOW,
                    "layer needs " + std::to_string(p.bytes) + " bytes of static scratch; the array holds " +
                        std::to_string(kScratchBytes));
    HIPCHECK(c, hipSetDevice(c->device));
    char* base = static_cast<char*>(c->scratch);
    const LayerState& Ls = c->L[layer];
    const uint64_t n = c->n, W = uint64_t(Ls.width());
    TfBufs b;
    b.pcol = c->pcol.as<uint32_t>();  // original source ids (with kPcolPad entries of padding)
    b.perm = c->perm;                 // sorted position -> original node
    b.left = reinterpret_cast<float*>(base + p.left);
    b.right = reinterpret_cast<float*>(base + p.right);
    b.mx = reinterpret_cast<float*>(base + p.mx);
    b.den = reinterpret_cast<float*>(base + p.den);
    b.z = base + p.z;
    b.xbf = precision == GATGPU_BF16 ? reinterpret_cast<uint16_t*>(base + p.xbf) : nullptr;
    b.out32 = p.outbf ? nullptr : reinterpret_cast<float*>(base + p.out);
    b.outbf = p.outbf ? reinterpret_cast<uint16_t*>(base + p.out) : nullptr;
    b.mchunk = reinterpret_cast<float*>(base + p.mchunk);
    b.part = reinterpret_cast<float*>(base + p.part);
    b.counter = reinterpret_cast<uint32_t*>(base + p.counter);
    b.fused_convert_ok = false;  // the caller's rows carry no padding: convert kernel first
    // The array keeps the previous call's contents: the arrival counters must start at zero.
    if (p.chunks) {
        const uint64_t blocks = std::min<uint64_t>((p.chunks + 255) / 256, 1024);
        k_fill_u32<<<dim3(uint32_t(blocks)), 256, 0, c->stream>>>(b.counter, p.chunks, 0u);
        HIPCHECK(c, hipGetLastError());
    }
    if (int r = run_tf(c, layer, precision, hidden != 0, x, nullptr, -1, false, b, nullptr)) return r;
    if (b.outbf) HIPCHECK(c, launch_widen_bf16(b.outbf, out, n * W, c->stream));
    else HIPCHECK(c, hipMemcpyAsync(out, b.out32, n * W * 4, hipMemcpyDeviceToDevice, c->stream));
    HIPCHECK(c, hipGetLastError());
    return GATGPU_OK;
}

}  // extern "C"
