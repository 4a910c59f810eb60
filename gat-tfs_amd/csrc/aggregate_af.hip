// Aggregate-first GAT layer on bf16: gather the layer's INPUT rows and
// project each gathered row on the MFMA units, instead of gathering the
// projected Z rows.
//
// Reference: tfs_online_fused (implementation/src/gat_tfs_online.cpp:200-283)
// and the neighbour-step TFS of baseline/src/baseline_tfs.cpp:16-110: per
// destination tile, step s takes the s-th neighbour of every row and
// multiplies the gathered input rows by W_h with the output sums resident
// (tile registers there, VGPRs here).  The attention logits come from the
// reordered contraction L/R = X (W a) (prepare_attention, :48-73).
//
//   out[i, h] = ELU?( sum_j p_ijh (X_j W_h) / den_ih ),
//   p_ijh = exp(LeakyReLU(L_ih + R_jh) - M_ih),  M the row max
//   (kept as a running max with rescaling; the final M is exact).
//
// X_j W_h is formed in FP32 by the MFMA from the bf16 row and the bf16 W,
// i.e. the FP32 Z row of standard_bf16 (baseline_standard.cpp:3-6), and p is
// applied to it in FP32.  Summed over j this equals (sum_j p X_j) W up to
// rounding order, which is the aggregate-first identity.
//
// Why: the gathered row is the input (D_in <= 128 bf16, 256 bytes) instead of
// Z (8 heads x 32 bf16 = 512 bytes), so layer 1 of a D_in = 100/128 model
// moves about half the bytes; the per-edge projection costs 2 D W MACs per
// edge, which the MFMA units absorb (about 1.5 ms of MFMA time for 64M edges
// at 100 -> 256).
//
// Wave layout (v_mfma_f32_32x32x16_bf16, computed transposed as in
// projection_mfma.hip): A = 32 output features x 16 k of W^T from LDS,
// B = 16 k x 32 slots of X^T -- lane (half, slot) loads 8 consecutive input
// features of its slot's current neighbour with one 16-byte load -- and
// D = 32 features x 32 slots, so all 16 accumulators of a lane belong to one
// slot and one head: p is one scalar per (lane, head).  A wave owns 32 slots
// and up to 4 output blocks of 32 features (4 heads of 32); the other heads
// of the same slots go to the next wave of the workgroup, which gathers the
// same rows through the same L2.
//
// Slots: 32 consecutive degree-sorted rows (heaviest first), so the slots of
// a wave have about the same number of steps; or 32 chunks of split rows,
// whose partial sums a merge kernel adds in chunk order.  Whole rows keep an
// online softmax per (slot, head); chunks start from their row's exact max
// (per-chunk maxima of k_split_prescan), so their partials need no rescale.
#include "internal.hpp"

namespace gatgpu {
namespace {

typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kXS = 128;      // input row stride (bf16 elements), zero-padded
constexpr int kSlots = 32;    // destination slots per wave (MFMA N)
constexpr int kMB = 4;        // output blocks of 32 features per wave
constexpr int kPart = 8 * 128 + 8;  // floats per chunk in the split scratch
constexpr int kDenOff = 8 * 128;    // offset of the chunk's denominators

struct Items {
    uint64_t chunk_groups;  // ceil(chunks / 32)
    uint64_t tile_groups;   // ceil(rows / 32)
    int waves_per_item;     // ceil(blocks / kMB)
    int blocks;             // output blocks of 32 features (= heads at dim 32)
};

// Softmax modes: the online running max (aggregate-first), the exact row
// max precomputed by k_af_rowmax (B1), or fixture weights (fixed-p).
enum { kOnline = 0, kExact = 1, kFixed = 2 };

// Persistent workgroups: W^T fragments of every block in LDS once, then wave
// items (slot group, head group) heaviest first.  B1: the faithful
// neighbour-step TFS of baseline/src/baseline_tfs.cpp:16-110 -- the weighted
// row p X_j is rounded to bf16 (cvtneps_pbh there, v_cvt_pk_bf16_f32 here)
// and multiplied by W_h with the sums resident in the MFMA accumulators;
// otherwise the FP32 product X_j W_h is weighted by p afterwards.
template <int KS, int SM, bool B1>
__global__ void __launch_bounds__(kThreads, 2) k_af_ns(AfArgs a, Items it) {
    extern __shared__ uint4 wlds[];  // [block][ks][lane]
    const int nb_all = it.blocks;
    for (int q = threadIdx.x; q < nb_all * KS * kWave; q += kThreads) {
        const int lane = q % kWave, ks = (q / kWave) % KS, mb = q / (kWave * KS);
        wlds[q] = a.wpk[(size_t(ks) * a.nmb + mb) * kWave + lane];
    }
    __syncthreads();
    const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int l = threadIdx.x % kWave, half = l / 32, s = l % 32;
    const int K = a.heads;
    const uint64_t total = (it.chunk_groups + it.tile_groups) * uint64_t(it.waves_per_item);
    for (uint64_t gw = uint64_t(blockIdx.x) * kWaves + w; gw < total; gw += uint64_t(gridDim.x) * kWaves) {
        const uint64_t item = gw / it.waves_per_item;
        const int hg = int(gw % it.waves_per_item);
        const int mb0 = hg * kMB;
        const int nb = nb_all - mb0 < kMB ? nb_all - mb0 : kMB;
        // ---- this lane's slot
        const bool chunk_item = item < it.chunk_groups;
        bool valid = false;
        uint64_t beg = 0, end = 0, c = 0;
        uint32_t i = 0, first = 0, nch = 0;
        if (chunk_item) {
            c = item * kSlots + s;
            if (c < a.chunks) {
                const uint32_t k = a.chunk_k[c];
                first = a.chunk_first[c];
                const uint64_t rbeg = a.prow[k], rend = a.prow[k + 1];
                i = a.perm[k];
                nch = uint32_t((rend - rbeg + a.chunk_edges - 1) / a.chunk_edges);
                beg = rbeg + (c - first) * a.chunk_edges;
                end = beg + a.chunk_edges < rend ? beg + a.chunk_edges : rend;
                valid = i < a.n && rbeg <= rend && rend <= a.e && beg <= end;
            }
        } else {
            const uint64_t t = (item - it.chunk_groups) * kSlots + s;
            if (t < a.rows) {
                const uint64_t k = a.rows - 1 - t;
                i = a.perm[k];
                beg = a.prow[k];
                end = a.prow[k + 1];
                valid = i < a.n && beg <= end && end <= a.e;
            }
        }
        const uint64_t len = valid ? end - beg : 0;
        uint64_t steps = len;
        for (int off = 1; off < kWave; off <<= 1) {
            const uint64_t o = __shfl_xor(steps, off);
            steps = o > steps ? o : steps;
        }
        // ---- per head of this wave: L and the softmax state.  Online mode: a
        // chunk starts from the exact row max of its split row (per-chunk
        // maxima of k_split_prescan), so its m never moves and the partials
        // add up directly; a whole row keeps the running-maximum form of
        // tfs_online_fused (gat_tfs_online.cpp:86-117), rescaling its sums by
        // exp(m_old - m_new) when a step raises m.  The final m is max
        // leaky(L + R_j) = leaky(L + max R_j) bit for bit.  Exact mode reads
        // that max from a.mx (max_prescan, baseline_standard.cpp:44-51).
        float L[kMB], m[kMB], den[kMB];
#pragma unroll
        for (int q = 0; q < kMB; ++q) {
            L[q] = (SM != kFixed && valid && q < nb) ? a.L[uint64_t(i) * K + mb0 + q] : 0.0f;
            den[q] = 0.0f;
            m[q] = -INFINITY;
            if (SM == kExact && valid && q < nb) m[q] = a.mx[uint64_t(i) * K + mb0 + q];
        }
        if (SM == kOnline && chunk_item) {
#pragma unroll
            for (int q = 0; q < kMB; ++q) {
                float mc = -INFINITY;
                if (valid && q < nb)
                    for (uint32_t cq = 0; cq < nch; ++cq) mc = fmaxf(mc, a.mchunk[(first + cq) * 8 + mb0 + q]);
                if (valid) m[q] = leaky(L[q] + mc);
            }
        }
        // ---- neighbour steps: gather, project, weight, accumulate.
        f32x16 acc[kMB];
#pragma unroll
        for (int q = 0; q < kMB; ++q)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[q][r] = 0.0f;
        // Steps past a slot's last edge re-read that edge's row (weight 0), so
        // every load is unconditional and no absent row is ever multiplied.
        auto src = [&](uint64_t t) -> uint64_t { return a.pcol[len ? beg + (t < len ? t : len - 1) : 0]; };
        // rv: R of the source (softmax modes) or the fixture weight of the edge.
        auto fetch = [&](uint64_t j, uint64_t t, uint4 (&xf)[KS], float (&rv)[kMB]) {
            const uint16_t* xr = a.X + j * kXS + 8 * half;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) xf[ks] = *reinterpret_cast<const uint4*>(xr + 16 * ks);
            const uint64_t e = len ? beg + (t < len ? t : len - 1) : 0;
#pragma unroll
            for (int q = 0; q < kMB; ++q)
                rv[q] = SM == kFixed ? a.fixp[e * K + mb0 + (q < nb ? q : 0)] : a.R[j * K + mb0 + (q < nb ? q : 0)];
        };
        auto frag = [&](int q, int ks) {
            return __builtin_bit_cast(bf16x8, wlds[(size_t(mb0 + q) * KS + ks) * kWave + l]);
        };
        auto step = [&](uint64_t t, const uint4 (&x)[KS], const float (&rv)[kMB]) {
            const bool ok = t < len;
            float p[kMB], scale[kMB];
#pragma unroll
            for (int q = 0; q < kMB; ++q) {
                scale[q] = 1.0f;
                if constexpr (SM == kFixed) {
                    p[q] = ok ? rv[q] : 0.0f;
                } else if constexpr (SM == kExact) {
                    p[q] = ok ? exp_w(leaky(L[q] + rv[q]) - m[q]) : 0.0f;
                    den[q] += p[q];
                } else {
                    const float sc_ = leaky(L[q] + rv[q]);
                    const float mn = ok ? fmaxf(m[q], sc_) : m[q];
                    scale[q] = mn > m[q] ? exp_w(m[q] - mn) : 1.0f;  // exp(-inf) = 0 on the first edge
                    p[q] = ok ? exp_w(sc_ - mn) : 0.0f;
                    m[q] = mn;
                    den[q] = den[q] * scale[q] + p[q];
                }
            }
            if constexpr (B1) {
                // bf16(p X_j) W_h accumulated in the MFMA: k step outer, heads
                // inner (independent accumulation chains).
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const uint32_t wv[4] = {x[ks].x, x[ks].y, x[ks].z, x[ks].w};
                    float f[8];
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        f[2 * v] = __builtin_bit_cast(float, wv[v] << 16);
                        f[2 * v + 1] = __builtin_bit_cast(float, wv[v] & 0xffff0000u);
                    }
#pragma unroll
                    for (int q = 0; q < kMB; ++q) {
                        if (q >= nb) continue;
                        bf16x8 b;
#pragma unroll
                        for (int v = 0; v < 8; ++v) b[v] = (__bf16)(p[q] * f[v]);
                        acc[q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag(q, ks), b, acc[q], 0, 0, 0);
                    }
                }
                return;
            }
            // Two heads at a time: two independent MFMA chains, and the next
            // k-step's W fragments read from LDS while this one multiplies.
#pragma unroll
            for (int q0 = 0; q0 < kMB; q0 += 2) {
                if (q0 >= nb) continue;
                const bool two = q0 + 1 < nb;
                f32x16 T0, T1;
#pragma unroll
                for (int r = 0; r < 16; ++r) T0[r] = T1[r] = 0.0f;
                bf16x8 a0 = frag(q0, 0), a1 = frag(two ? q0 + 1 : q0, 0);
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    bf16x8 n0 = a0, n1 = a1;
                    if (ks + 1 < KS) {
                        n0 = frag(q0, ks + 1);
                        n1 = frag(two ? q0 + 1 : q0, ks + 1);
                    }
                    const bf16x8 b = __builtin_bit_cast(bf16x8, x[ks]);
                    T0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b, T0, 0, 0, 0);
                    if (two) T1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b, T1, 0, 0, 0);
                    a0 = n0;
                    a1 = n1;
                }
                // Rescale only when some slot of the wave raised its max.
                if (SM == kOnline && __any(scale[q0] != 1.0f))
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[q0][r] *= scale[q0];
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[q0][r] += p[q0] * T0[r];
                if (two) {
                    if (SM == kOnline && __any(scale[q0 + 1] != 1.0f))
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[q0 + 1][r] *= scale[q0 + 1];
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[q0 + 1][r] += p[q0 + 1] * T1[r];
                }
            }
        };
        // Ping-pong: the rows of step t + 1 are requested before step t's
        // MFMAs, and the source id of a step two steps before its rows, so a
        // step waits on one memory round trip that overlaps the previous step.
        uint4 xa[KS], xb[KS];
        float ra[kMB], rb[kMB];
        fetch(src(0), 0, xa, ra);
        uint64_t jb = src(1), ja = src(2);
        for (uint64_t t = 0; t < steps; t += 2) {
            fetch(jb, t + 1, xb, rb);
            jb = src(t + 3);
            step(t, xa, ra);
            if (t + 1 >= steps) break;
            fetch(ja, t + 2, xa, ra);
            ja = src(t + 4);
            step(t + 1, xb, rb);
        }
        float M[kMB];
#pragma unroll
        for (int q = 0; q < kMB; ++q) M[q] = len ? m[q] : 0.0f;  // empty row: max 0 (ref_fp32.cpp:11)
        if (!valid) continue;
        // ---- epilogue.  Lane (half, slot) holds features 32 mb + 16 half + 4 gq + {0..3}
        // (permuted packing of pack_projection_weights).
        const int W = it.blocks * 32;
        if (chunk_item) {
            float* part = a.part + c * kPart;
#pragma unroll
            for (int q = 0; q < kMB; ++q) {
                if (q >= nb) continue;
#pragma unroll
                for (int gq = 0; gq < 4; ++gq) {
                    const int f0 = (mb0 + q) * 32 + 16 * half + 4 * gq;
                    *reinterpret_cast<float4*>(part + f0) =
                        make_float4(acc[q][4 * gq], acc[q][4 * gq + 1], acc[q][4 * gq + 2], acc[q][4 * gq + 3]);
                }
                if (half == 0) part[kDenOff + mb0 + q] = den[q];
            }
            continue;
        }
#pragma unroll
        for (int q = 0; q < kMB; ++q) {
            if (q >= nb) continue;
            const int h = mb0 + q;
            if (SM == kFixed) den[q] = a.fixden[uint64_t(i) * K + h];  // the fixture's denominator
            const float scale = den[q] > 0.0f ? 1.0f / den[q] : 0.0f;
            if (half == 0) {
                if (SM == kOnline) a.mx[uint64_t(i) * K + h] = M[q];
                a.den[uint64_t(i) * K + h] = den[q];
            }
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                const int f0 = h * 32 + 16 * half + 4 * gq;
                float o[4];
#pragma unroll
                for (int x = 0; x < 4; ++x) {
                    const float y = den[q] > 0.0f ? acc[q][4 * gq + x] * scale : 0.0f;  // empty row: exact 0
                    o[x] = a.hidden ? elu_bf16(y) : y;
                }
                if (a.outbf)
                    *reinterpret_cast<uint2*>(a.outbf + uint64_t(i) * W + f0) =
                        make_uint2(bf16x2(o[0], o[1]), bf16x2(o[2], o[3]));
                if (a.out32)
                    *reinterpret_cast<float4*>(a.out32 + uint64_t(i) * W + f0) = make_float4(o[0], o[1], o[2], o[3]);
            }
        }
    }
}

// One wave per split row (found at its first chunk): adds the chunks' partial
// sums and denominators in chunk order, normalises, ELU, stores.
template <int SM>
__global__ void __launch_bounds__(kThreads) k_af_merge(AfArgs a, int blocks) {
    const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
    const uint64_t c = uint64_t(blockIdx.x) * kWaves + w;
    if (c >= a.chunks || a.chunk_first[c] != c) return;
    const uint32_t k = a.chunk_k[c];
    const uint64_t rbeg = a.prow[k], rend = a.prow[k + 1];
    const uint32_t i = a.perm[k];
    if (i >= a.n || rbeg > rend || rend > a.e) return;
    const uint32_t nch = uint32_t((rend - rbeg + a.chunk_edges - 1) / a.chunk_edges);
    if (c + nch > a.chunks) return;
    const int K = a.heads, W = blocks * 32;
    for (int f0 = 4 * l; f0 < W; f0 += 4 * kWave) {
        const int h = f0 / 32;
        float4 tot = make_float4(0.f, 0.f, 0.f, 0.f);
        float d = 0.0f, m = -INFINITY;
        for (uint32_t q = 0; q < nch; ++q) {
            const float* pq = a.part + (c + q) * kPart;
            const float4 v = *reinterpret_cast<const float4*>(pq + f0);
            tot.x += v.x;
            tot.y += v.y;
            tot.z += v.z;
            tot.w += v.w;
            d += pq[kDenOff + h];
            if (SM == kOnline) m = fmaxf(m, a.mchunk[(c + q) * 8 + h]);
        }
        if (SM == kFixed) d = a.fixden[uint64_t(i) * K + h];
        if (f0 % 32 == 0) {
            if (SM == kOnline) a.mx[uint64_t(i) * K + h] = leaky(a.L[uint64_t(i) * K + h] + m);
            a.den[uint64_t(i) * K + h] = d;
        }
        const float scale = d > 0.0f ? 1.0f / d : 0.0f;
        float o[4] = {tot.x * scale, tot.y * scale, tot.z * scale, tot.w * scale};
        if (!(d > 0.0f)) o[0] = o[1] = o[2] = o[3] = 0.0f;
        if (a.hidden)
#pragma unroll
            for (int x = 0; x < 4; ++x) o[x] = elu_bf16(o[x]);
        if (a.outbf)
            *reinterpret_cast<uint2*>(a.outbf + uint64_t(i) * W + f0) =
                make_uint2(bf16x2(o[0], o[1]), bf16x2(o[2], o[3]));
        if (a.out32)
            *reinterpret_cast<float4*>(a.out32 + uint64_t(i) * W + f0) = make_float4(o[0], o[1], o[2], o[3]);
    }
}

template <int KS, int SM, bool B1>
hipError_t launch_ns(const AfArgs& a, const Items& it, hipStream_t s, int cus) {
    const size_t lds = size_t(it.blocks) * KS * kWave * sizeof(uint4);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_af_ns<KS, SM, B1>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess) return e;
    }
    const uint64_t waves = (it.chunk_groups + it.tile_groups) * uint64_t(it.waves_per_item);
    uint64_t blocks = (waves + kWaves - 1) / kWaves;
    if (blocks > uint64_t(cus) * 2) blocks = uint64_t(cus) * 2;
    k_af_ns<KS, SM, B1><<<dim3(uint32_t(blocks)), kThreads, lds, s>>>(a, it);
    return hipGetLastError();
}

template <int SM, bool B1>
hipError_t launch_ns_ks(const AfArgs& a, const Items& it, hipStream_t s, int cus) {
    switch (a.ksteps) {
        case 1: return launch_ns<1, SM, B1>(a, it, s, cus);
        case 2: return launch_ns<2, SM, B1>(a, it, s, cus);
        case 3: return launch_ns<3, SM, B1>(a, it, s, cus);
        case 4: return launch_ns<4, SM, B1>(a, it, s, cus);
        case 5: return launch_ns<5, SM, B1>(a, it, s, cus);
        case 6: return launch_ns<6, SM, B1>(a, it, s, cus);
        case 7: return launch_ns<7, SM, B1>(a, it, s, cus);
        default: return launch_ns<8, SM, B1>(a, it, s, cus);
    }
}

// Exact row max for the B1 path (max_prescan, baseline_standard.cpp:44-51):
// M[i, h] = LeakyReLU(L[i, h] + max_j R[j, h]), 0 for an empty row.  One wave
// per degree-sorted row; lane l covers edges l / K + (64 / K) q of head l % K.
template <int K>
__global__ void __launch_bounds__(kThreads) k_af_rowmax(AfArgs a) {
    const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
    const uint64_t k = uint64_t(blockIdx.x) * kWaves + w;
    if (k >= a.n) return;
    const uint32_t i = a.perm[k];
    const uint64_t beg = a.prow[k], end = a.prow[k + 1];
    if (i >= a.n || beg > end || end > a.e) return;
    const int h = l % K;
    float m = -INFINITY;
    for (uint64_t e = beg + l / K; e < end; e += kWave / K) m = fmaxf(m, a.R[uint64_t(a.pcol[e]) * K + h]);
    for (int off = K; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (l < K) a.mx[uint64_t(i) * K + l] = end > beg ? leaky(a.L[uint64_t(i) * K + l] + m) : 0.0f;
}

hipError_t launch_rowmax(const AfArgs& a, hipStream_t s) {
    const dim3 grid(uint32_t((a.n + kWaves - 1) / kWaves));
    switch (a.heads) {
        case 1: k_af_rowmax<1><<<grid, kThreads, 0, s>>>(a); break;
        case 2: k_af_rowmax<2><<<grid, kThreads, 0, s>>>(a); break;
        case 4: k_af_rowmax<4><<<grid, kThreads, 0, s>>>(a); break;
        default: k_af_rowmax<8><<<grid, kThreads, 0, s>>>(a); break;
    }
    return hipGetLastError();
}

}  // namespace

bool aggregate_af_supported(int in, int heads, int dim) {
    return in <= kXS && (heads == 1 || heads == 2 || heads == 4 || heads == 8) && dim == 32;
}

int af_input_stride() { return kXS; }

hipError_t launch_aggregate_af(const AfArgs& a, hipStream_t s, int cus) {
    if (!aggregate_af_supported(a.in, a.heads, 32) || a.ksteps < 1 || a.ksteps > kXS / 16 || a.nmb < a.heads)
        return hipErrorInvalidValue;
    Items it{};
    it.blocks = a.heads;
    it.waves_per_item = (it.blocks + kMB - 1) / kMB;
    it.chunk_groups = (a.chunks + kSlots - 1) / kSlots;
    it.tile_groups = (a.rows + kSlots - 1) / kSlots;
    if (a.chunks && !a.fixp && !a.b1) {
        SplitTable t{};
        t.chunks = a.chunks;
        t.chunk_k = a.chunk_k;
        t.chunk_first = a.chunk_first;
        t.chunk_edges = a.chunk_edges;
        t.mchunk = const_cast<float*>(a.mchunk);
        hipError_t e = launch_split_prescan(a.prow, a.pcol, a.R, a.heads, t, a.e, s);
        if (e != hipSuccess) return e;
    }
    const int sm = a.fixp ? kFixed : a.b1 ? kExact : kOnline;
    if (sm == kExact) {
        hipError_t e = launch_rowmax(a, s);
        if (e != hipSuccess) return e;
    }
    if (it.chunk_groups + it.tile_groups) {
        hipError_t e = hipSuccess;
        if (sm == kOnline) e = launch_ns_ks<kOnline, false>(a, it, s, cus);
        else if (sm == kExact) e = launch_ns_ks<kExact, true>(a, it, s, cus);
        else if (a.b1) e = launch_ns_ks<kFixed, true>(a, it, s, cus);
        else e = launch_ns_ks<kFixed, false>(a, it, s, cus);
        if (e != hipSuccess) return e;
    }
    if (a.chunks) {
        const dim3 grid(uint32_t((a.chunks + kWaves - 1) / kWaves));
        if (sm == kOnline) k_af_merge<kOnline><<<grid, kThreads, 0, s>>>(a, it.blocks);
        else if (sm == kExact) k_af_merge<kExact><<<grid, kThreads, 0, s>>>(a, it.blocks);
        else k_af_merge<kFixed><<<grid, kThreads, 0, s>>>(a, it.blocks);
    }
    return hipGetLastError();
}

}  // namespace gatgpu
