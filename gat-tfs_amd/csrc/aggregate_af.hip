// Aggregate-first (TFS) GAT layer on bf16: gather the layer INPUT rows,
// project afterwards.
//
// Reference: tfs_online_fused (implementation/src/gat_tfs_online.cpp:200-283):
// per head U^h_i = sum_j p^h_ij X_j, then U^h_i W^h, / l^h_i, ELU.  The
// attention logits come from the reordered contraction L/R = X (W a)
// (prepare_attention, :48-73).  The reference uses an online max with
// rescaling; here the max is exact (the same M as the transform-first path),
// so U needs no rescale, and the projection of U is done once per row.
//
// Why: the gathered row is the input (D_in <= 128 bf16 = 256 bytes, two cache
// lines) instead of Z (8 heads x 32 bf16 = 512 bytes); layer 1 of a
// D_in=100/128 model moves half the bytes.
//
// Work split (tile kernel, 8 waves, one 32-row tile of degree-sorted rows at a
// time, persistent over tiles):
//   phase A  each wave runs 4 row groups of 16 lanes; a group owns one row and
//            lane c of the group owns input features 8c..8c+7 for all K heads
//            (64 FP32 accumulators).  Per batch of 16 edges the group scores
//            (edge, head) pairs -- one exp each -- and gathers the 16 source
//            rows with one 16-byte load per lane.  U is then split into bf16
//            hi + lo and written to LDS in MFMA B-operand order.
//   phase B  wave h multiplies U^h (32 rows x 128) by W^h on
//            v_mfma_f32_32x32x16_bf16 (hi and lo products accumulated in
//            FP32, ~16 mantissa bits of U), scales by 1/den, ELU, stores.
// Rows at or above the split threshold go to k_af_split: one wave per chunk,
// partial (U, den) to scratch, the last chunk to arrive adds the partials in
// chunk order and projects the row on the VALU from the bf16 W.
#include "internal.hpp"

namespace gatgpu {
namespace {

typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kTile = 32;        // rows per tile
constexpr int kXS = 128;         // input row stride (bf16), zero-padded
constexpr int kGL = 16;          // lanes per row group = 16-byte vectors per input row
constexpr int kGPW = kWave / kGL;  // row groups per wave
constexpr int kBE = 16;          // edges per scoring batch
constexpr int kUS = kXS / 8 + 1; // LDS row stride of U in 16-byte units (one pad unit: no bank conflicts)

__device__ inline void unpack8(const uint4& v, float (&f)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        f[2 * q] = __builtin_bit_cast(float, w[q] << 16);
        f[2 * q + 1] = __builtin_bit_cast(float, w[q] & 0xffff0000u);
    }
}

// Accumulates edges [beg, end) of one row into the group's U registers.
// Lane c (= lane % 16) of the group owns features 8c..8c+7 of every head.
// Max is exact: given (Mh of the scorer head) or, when the row fits one
// batch, found from the scored R values.
__device__ inline void group_rows(uint64_t beg, uint64_t end, bool find_max, const uint32_t* __restrict__ pcol,
                                  const float* __restrict__ R, const uint16_t* __restrict__ X, int K, float Lh,
                                  float& Mh, float* pb, uint32_t* jb, float (&acc)[8][8], float& dloc) {
    const int c = threadIdx.x % kGL;
    const int hs = c % 8;  // scorer head; pairs (t = c/8 + 2s, hs), s < 8
    for (uint64_t base = beg; base < end; base += kBE) {
        const uint64_t rem = end - base;
        const int cnt = rem < uint64_t(kBE) ? int(rem) : kBE;
        uint32_t jv[8];
        float rv[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int t = c / 8 + 2 * s;
            const bool ok = t < cnt && hs < K;
            jv[s] = t < cnt ? pcol[base + t] : 0u;
            rv[s] = ok ? R[uint64_t(jv[s]) * K + hs] : -INFINITY;
        }
        if (find_max) {  // the whole row is this batch
            float m = rv[0];
#pragma unroll
            for (int s = 1; s < 8; ++s) m = fmaxf(m, rv[s]);
            m = fmaxf(m, __shfl_xor(m, 8));
            Mh = cnt > 0 ? leaky(Lh + m) : 0.0f;
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int t = c / 8 + 2 * s;
            const float p = (t < cnt && hs < K) ? expf(leaky(Lh + rv[s]) - Mh) : 0.0f;
            dloc += p;
            pb[t * 8 + hs] = p;
            if (hs == 0) jb[t] = jv[s];
        }
        wave_sync();
        uint4 raw[kBE];
#pragma unroll
        for (int t = 0; t < kBE; ++t)
            raw[t] = t < cnt ? *reinterpret_cast<const uint4*>(X + uint64_t(jb[t]) * kXS + c * 8) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int t = 0; t < kBE; ++t) {
            const float4 p0 = *reinterpret_cast<const float4*>(pb + t * 8);
            const float4 p1 = *reinterpret_cast<const float4*>(pb + t * 8 + 4);
            const float p[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
            float f[8];
            unpack8(raw[t], f);
#pragma unroll
            for (int h = 0; h < 8; ++h)
#pragma unroll
                for (int x = 0; x < 8; ++x) acc[h][x] += p[h] * f[x];
        }
        wave_sync();
    }
}

// Exact max of R over [beg, end) for the scorer head, reduced within the group.
__device__ inline float group_max(uint64_t beg, uint64_t end, const uint32_t* __restrict__ pcol,
                                  const float* __restrict__ R, int K) {
    const int c = threadIdx.x % kGL, hs = c % 8;
    float m = -INFINITY;
    if (hs < K)
        for (uint64_t e = beg + c / 8; e < end; e += 2) m = fmaxf(m, R[uint64_t(pcol[e]) * K + hs]);
    return fmaxf(m, __shfl_xor(m, 8));
}

__global__ void __launch_bounds__(kThreads) k_af_tiles(AfArgs a) {
    __shared__ uint4 ut[2][8][kTile][kUS];          // U hi / lo, [head][row][k/8]
    __shared__ float pbuf[kWaves][kGPW][kBE * 8];    // scores [edge][head]
    __shared__ uint32_t jbuf[kWaves][kGPW][kBE];     // source ids
    __shared__ float dsh[kTile][8];                  // denominators
    const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int g = lane / kGL, c = lane % kGL, hs = c % 8;
    const int rs = w * kGPW + g;  // row slot of this group within the tile
    const int K = a.heads;
    for (uint64_t tile = blockIdx.x; tile < a.tiles; tile += gridDim.x) {
        // ---------------- phase A: aggregate 32 rows (one per group)
        const uint64_t idx = tile * kTile + rs;
        float acc[8][8];
#pragma unroll
        for (int h = 0; h < 8; ++h)
#pragma unroll
            for (int x = 0; x < 8; ++x) acc[h][x] = 0.0f;
        float dloc = 0.0f;
        bool have = idx < a.rows;
        uint32_t i = 0;
        uint64_t beg = 0, end = 0;
        if (have) {
            const uint64_t k = a.rows - 1 - idx;  // heaviest first
            i = a.perm[k];
            beg = a.prow[k];
            end = a.prow[k + 1];
            if (i >= a.n || beg > end || end > a.e) have = false;
        }
        // Every group runs the batch loop (an empty range for a missing or
        // shorter row): the wave-level LDS syncs inside stay uniform.
        const float Lh = have && hs < K ? a.L[uint64_t(i) * K + hs] : 0.0f;
        const uint64_t deg = have ? end - beg : 0;
        uint64_t wmax = deg;  // longest row of the wave
        for (int off = kGL; off < kWave; off <<= 1) {
            const uint64_t o = __shfl_xor(wmax, off);
            wmax = o > wmax ? o : wmax;
        }
        const bool single = wmax <= uint64_t(kBE);  // every row of the wave fits one batch
        float Mh = 0.0f;                             // empty row: max 0 (ref_fp32.cpp:11)
        if (!single && deg) Mh = leaky(Lh + group_max(beg, end, a.pcol, a.R, K));
        const uint64_t span = (wmax + kBE - 1) / kBE * kBE;
        for (uint64_t base = 0; base < span; base += kBE) {
            const uint64_t b0 = beg + base < end ? beg + base : end;
            const uint64_t b1 = beg + base + kBE < end ? beg + base + kBE : end;
            group_rows(b0, b1, single, a.pcol, a.R, a.X, K, Lh, Mh, pbuf[w][g], jbuf[w][g], acc, dloc);
        }
        dloc += __shfl_xor(dloc, 8);
        if (c < 8) dsh[rs][c] = (have && c < K) ? dloc : 0.0f;
        if (have && c < K) {
            a.mx[uint64_t(i) * K + c] = Mh;
            a.den[uint64_t(i) * K + c] = dloc;
        }
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float v0 = acc[h][2 * q], v1 = acc[h][2 * q + 1];
                const uint16_t h0 = bf16_rne(v0), h1 = bf16_rne(v1);
                hi[q] = uint32_t(h0) | (uint32_t(h1) << 16);
                lo[q] = uint32_t(bf16_rne(v0 - bf16_widen(h0))) | (uint32_t(bf16_rne(v1 - bf16_widen(h1))) << 16);
            }
            ut[0][h][rs][c] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            ut[1][h][rs][c] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        }
        __syncthreads();
        // ---------------- phase B: wave h projects head h of the 32 rows
        if (w < K) {
            const int h = w, half = lane / 32, col = lane % 32;
            f32x16 o;
#pragma unroll
            for (int r = 0; r < 16; ++r) o[r] = 0.0f;
            for (int ks = 0; ks < a.ksteps; ++ks) {
                const bf16x8 av = __builtin_bit_cast(bf16x8, a.wpk[(size_t(ks) * a.nmb + h) * kWave + lane]);
                const bf16x8 bh = __builtin_bit_cast(bf16x8, ut[0][h][col][2 * ks + half]);
                const bf16x8 bl = __builtin_bit_cast(bf16x8, ut[1][h][col][2 * ks + half]);
                o = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bh, o, 0, 0, 0);
                o = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bl, o, 0, 0, 0);
            }
            const uint64_t ridx = tile * kTile + col;
            if (ridx < a.rows) {
                const uint32_t ri = a.perm[a.rows - 1 - ridx];
                const float d = dsh[col][h];
                const float scale = d > 0.0f ? 1.0f / d : 0.0f;
                const int W = K * 32;
#pragma unroll
                for (int gq = 0; gq < 4; ++gq) {
                    const int f0 = h * 32 + 8 * gq + 4 * half;
                    float v[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float y = o[4 * gq + q] * scale;
                        v[q] = a.hidden ? elu(y) : y;
                    }
                    const uint64_t off = uint64_t(ri) * W + f0;
                    if (a.outbf)
                        *reinterpret_cast<uint2*>(a.outbf + off) =
                            make_uint2(uint32_t(bf16_rne(v[0])) | (uint32_t(bf16_rne(v[1])) << 16),
                                       uint32_t(bf16_rne(v[2])) | (uint32_t(bf16_rne(v[3])) << 16));
                    if (a.out32) *reinterpret_cast<float4*>(a.out32 + off) = make_float4(v[0], v[1], v[2], v[3]);
                }
            }
        }
        __syncthreads();
    }
}

// One wave per chunk of a split row; 4 groups take quarters of the chunk.
__global__ void __launch_bounds__(256) k_af_split(AfArgs a) {
    __shared__ float pbuf[4][kGPW][kBE * 8];
    __shared__ uint32_t jbuf[4][kGPW][kBE];
    __shared__ float tot[4][8 * kXS + 8];
    const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int g = lane / kGL, c = lane % kGL, hs = c % 8;
    const uint64_t ch = uint64_t(blockIdx.x) * 4 + w;
    if (ch >= a.chunks) return;
    const int K = a.heads, W = K * 32;
    const uint32_t k = a.chunk_k[ch], first = a.chunk_first[ch];
    const uint64_t rbeg = a.prow[k], rend = a.prow[k + 1];
    const uint32_t i = a.perm[k];
    if (i >= a.n || rbeg > rend || rend > a.e) return;
    const uint32_t nch = uint32_t((rend - rbeg + a.chunk_edges - 1) / a.chunk_edges);
    const uint64_t cbeg = rbeg + uint64_t(ch - first) * a.chunk_edges;
    const uint64_t cend = cbeg + a.chunk_edges < rend ? cbeg + a.chunk_edges : rend;
    float m = -INFINITY;
    if (hs < K)
        for (uint32_t q = lane / 8; q < nch; q += 8) m = fmaxf(m, a.mchunk[(first + q) * 8 + hs]);
    for (int off = 8; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
    const float Lh = hs < K ? a.L[uint64_t(i) * K + hs] : 0.0f;
    float Mh = leaky(Lh + m);
    // Quarter g of the chunk, padded to whole batches so the wave's syncs line up.
    const uint64_t len = cend - cbeg, q0 = cbeg + len * g / kGPW, q1 = cbeg + len * (g + 1) / kGPW;
    uint64_t span = q1 - q0;
    for (int off = kGL; off < kWave; off <<= 1) {
        const uint64_t o = __shfl_xor(span, off);
        span = o > span ? o : span;
    }
    float acc[8][8];
#pragma unroll
    for (int h = 0; h < 8; ++h)
#pragma unroll
        for (int x = 0; x < 8; ++x) acc[h][x] = 0.0f;
    float dloc = 0.0f;
    for (uint64_t base = 0; base < span; base += kBE) {
        const uint64_t b0 = q0 + base;
        group_rows(b0 < q1 ? b0 : q1, b0 + kBE < q1 ? b0 + kBE : q1, false, a.pcol, a.R, a.X, K, Lh, Mh,
                   pbuf[w][g], jbuf[w][g], acc, dloc);
    }
    // Sum the 4 groups (lanes c, c+16, c+32, c+48) and the scorer lanes of each head.
#pragma unroll
    for (int h = 0; h < 8; ++h)
#pragma unroll
        for (int x = 0; x < 8; ++x) {
            acc[h][x] += __shfl_xor(acc[h][x], 16);
            acc[h][x] += __shfl_xor(acc[h][x], 32);
        }
    for (int off = 8; off < kWave; off <<= 1) dloc += __shfl_xor(dloc, off);
    float* part = a.part + ch * (8 * kXS + 8);
    if (g == 0)
#pragma unroll
        for (int h = 0; h < 8; ++h)
#pragma unroll
            for (int x = 0; x < 8; x += 4)
                *reinterpret_cast<float4*>(part + h * kXS + c * 8 + x) =
                    make_float4(acc[h][x], acc[h][x + 1], acc[h][x + 2], acc[h][x + 3]);
    if (lane < 8) part[8 * kXS + lane] = dloc;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    uint32_t old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(a.counter + first, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __shfl(old, 0);
    if (old + 1 != nch) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // Last arrival: partials in chunk order into LDS, then out = U^h W^h / den.
    float* t = tot[w];
    for (int q = lane; q < 8 * kXS + 8; q += kWave) {
        float s = 0.0f;
        for (uint32_t cq = 0; cq < nch; ++cq) s += a.part[uint64_t(first + cq) * (8 * kXS + 8) + q];
        t[q] = s;
    }
    wave_sync();
    if (lane < K) {  // lanes < 8 score head `lane`
        a.mx[uint64_t(i) * K + lane] = Mh;
        a.den[uint64_t(i) * K + lane] = t[8 * kXS + lane];
    }
    if (lane == 0) a.counter[first] = 0;
    for (int f = lane; f < W; f += kWave) {
        const int h = f / 32;
        float s = 0.0f;
        for (int kk = 0; kk < a.in; ++kk) s += t[h * kXS + kk] * a.wq[size_t(kk) * W + f];
        const float d = t[8 * kXS + h];
        float y = s * (d > 0.0f ? 1.0f / d : 0.0f);
        if (a.hidden) y = elu(y);
        if (a.outbf) a.outbf[uint64_t(i) * W + f] = bf16_rne(y);
        if (a.out32) a.out32[uint64_t(i) * W + f] = y;
    }
}

}  // namespace

bool aggregate_af_supported(int in, int heads, int dim) { return in <= kXS && heads <= 8 && dim == 32; }

int af_input_stride() { return kXS; }

hipError_t launch_aggregate_af(const AfArgs& a, hipStream_t s, int cus) {
    if (a.heads > 8 || a.in > kXS) return hipErrorInvalidValue;
    if (a.chunks) {
        SplitTable t{};
        t.chunks = a.chunks;
        t.chunk_k = a.chunk_k;
        t.chunk_first = a.chunk_first;
        t.chunk_edges = a.chunk_edges;
        t.mchunk = const_cast<float*>(a.mchunk);
        hipError_t e = launch_split_prescan(a.prow, a.pcol, a.R, a.heads, t, a.e, s);
        if (e != hipSuccess) return e;
        k_af_split<<<dim3(uint32_t((a.chunks + 3) / 4)), 256, 0, s>>>(a);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (a.tiles) {
        uint64_t gx = a.tiles < uint64_t(cus) ? a.tiles : uint64_t(cus);
        k_af_tiles<<<dim3(uint32_t(gx)), kThreads, 0, s>>>(a);
    }
    return hipGetLastError();
}

}  // namespace gatgpu
