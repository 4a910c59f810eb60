// Single-head aggregation for narrow rows (the output layer, 1 head x C <= 64
// classes).  Same mathematics as aggregate.hip (baseline_standard.cpp:44-97).
//
// A group of G lanes owns one destination row, so a wave works on 64/G rows
// at once.  Rows are taken in degree-sorted order, which gives the rows of a
// wave the same in-degree and therefore the same trip count.  Per batch of G
// edges, lane `sub` of the group scores edge `sub` (one exp per edge) and the
// group then walks the batch: source id and score are broadcast by a lane
// shuffle, and each lane gathers 16 bytes of the source's Z row (Z rows are
// padded to ZS = G*VEC... elements >= C, so the loads are aligned).  Rows at or
// above the split threshold are cut into chunks; a chunk takes a whole wave
// (each group a contiguous piece), and chunks merge exactly as in
// aggregate_vec.hip: exact row max from the per-chunk maxima, partial sums to
// scratch, the last arrival adds them in chunk order.
#include "internal.hpp"

namespace gatgpu {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;

template <class ZT, int G_>
struct K1 {
    static constexpr int G = G_;                      // lanes per row group (power of two)
    static constexpr int VEC = 16 / int(sizeof(ZT));  // features per lane
    static constexpr int GPW = kWave / G;             // row groups per wave
    static constexpr int MAXW = G * VEC;              // widest row handled
};

template <class ZT>
struct K1Args {
    const uint64_t* prow;
    const uint32_t* pcol;
    const uint32_t* perm;
    const float* L;
    const float* R;      // R of row j at R[j * rs] (a separate array, or inside the Z row)
    const ZT* Z;
    int W, zs, rs;
    bool hidden;
    float* mx;
    float* den;
    float* out32;
    uint16_t* outbf;
    uint64_t n, e, rows;
    uint64_t chunks;
    const uint32_t* chunk_k;
    const uint32_t* chunk_first;
    uint32_t chunk_edges;
    const float* mchunk;
    float* part;
    uint32_t* counter;
    const uint32_t* operm;  // output row of sorted position k: operm[k] (null: the node index)
    const float* ar;        // aR [W] when R is recomputed from the gathered rows
    int os;                 // out32 row stride: W, or G * VEC with operm (whole padded rows)
};

__device__ inline void unpack(const uint4& v, float (&f)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        f[2 * q] = __builtin_bit_cast(float, w[q] << 16);
        f[2 * q + 1] = __builtin_bit_cast(float, w[q] & 0xffff0000u);
    }
}
__device__ inline void unpack(const uint4& v, float (&f)[4]) {
    f[0] = __builtin_bit_cast(float, v.x);
    f[1] = __builtin_bit_cast(float, v.y);
    f[2] = __builtin_bit_cast(float, v.z);
    f[3] = __builtin_bit_cast(float, v.w);
}

// Max of R over [beg, end), reduced over the G lanes of the group.
template <class C>
__device__ inline float group_max(uint64_t beg, uint64_t end, const uint32_t* __restrict__ pcol,
                                  const float* __restrict__ R, int rs, int sub) {
    float m = -INFINITY;
    for (uint64_t e = beg + sub; e < end; e += C::G) m = fmaxf(m, R[uint64_t(pcol[e]) * rs]);
    for (int off = 1; off < C::G; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
    return m;
}

// Edges [beg, end) of one row into the group's accumulators.
template <class C, class ZT>
__device__ inline void group_accumulate(uint64_t beg, uint64_t end, const uint32_t* __restrict__ pcol,
                                        const float* __restrict__ R, int rs, const ZT* __restrict__ Z, int zs,
                                        int W, float Li, float Mi, int gbase, int sub, float (&acc)[C::VEC],
                                        float& dloc) {
    const bool reader = sub * C::VEC < W;
    for (uint64_t base = beg; base < end; base += C::G) {
        const uint64_t e = base + sub;
        const bool ev = e < end;
        const uint32_t j = ev ? pcol[e] : 0u;
        const float p = ev ? exp_w(leaky(Li + R[uint64_t(j) * rs]) - Mi) : 0.0f;
        dloc += p;
        const uint64_t rem = end - base;
        const int cnt = rem < uint64_t(C::G) ? int(rem) : C::G;
        uint4 raw[C::G];
        float pt[C::G];
#pragma unroll
        for (int t = 0; t < C::G; ++t) {
            const uint32_t jt = __shfl(j, gbase + t);
            pt[t] = __shfl(p, gbase + t);
            raw[t] = (t < cnt && reader) ? *reinterpret_cast<const uint4*>(Z + uint64_t(jt) * zs + sub * C::VEC)
                                         : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < C::G; ++t) {
            float f[C::VEC];
            unpack(raw[t], f);
#pragma unroll
            for (int x = 0; x < C::VEC; ++x) acc[x] += pt[t] * f[x];
        }
    }
}

// Edges [beg, end) of one row in a single pass, for Z rows that carry R in
// their last four bytes (lane G-1's 16-byte slice).  Each source row is
// fetched once: the batch's R values are broadcast from lane G-1 and every lane
// of the group scores the whole batch, so m, the accumulators and dsum stay
// identical across the group.  The softmax is kept online (the
// running-maximum form of tfs_online_fused, implementation/src/
// gat_tfs_online.cpp:86-117): when a batch raises the running maximum m, the
// accumulators and the denominator are rescaled by exp(m_old - m_new).  The
// final m equals leaky(L + max R) bit for bit, because leaky and the addition
// are monotone.
//
// RZ: rows of exactly G * 8 = 64 bf16 features with no room for R.  R of each
// gathered row is recomputed from it as the projection wrote it: lane sub
// takes the FMA chain of its 8 features with aR (p_sub), and the group adds
// ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)) by xor shuffles, so every
// lane gets the same bits as the R stage and each edge still fetches one line.
template <class C, bool RZ>
__device__ inline void group_online(uint64_t beg, uint64_t end, const uint32_t* __restrict__ pcol,
                                    const uint16_t* __restrict__ Z, int zs, int W, float Li, int gbase, int sub,
                                    const float (&arl)[C::VEC], float (&acc)[C::VEC], float& dsum, float& m) {
    static_assert(C::VEC == 8, "bf16 rows only");
    static_assert(!RZ || C::G == 8, "R from Z needs the 8-lane reduction order");
    // 32-bit edge counts (set_graph rejects rows of 2^32 edges or more).
    // Every lane loads its slice of every edge's line, with no bounds test:
    // edges past the end read row 0 (cached after its first use) and get
    // score -inf, weight 0; slices past W feed accumulators that are never
    // stored.  pcol carries kPcolPad entries past e for the id loads.
    const uint32_t total = uint32_t(end - beg);
    for (uint32_t done = 0; done < total; done += C::G) {
        const uint32_t left = total - done;
        const int cnt = left < uint32_t(C::G) ? int(left) : C::G;
        const uint32_t jr = pcol[beg + done + sub];
        const uint32_t j = sub < cnt ? jr : 0u;
        uint4 raw[C::G];
#pragma unroll
        for (int t = 0; t < C::G; ++t) {
            const uint32_t jt = __shfl(j, gbase + t);
            raw[t] = *reinterpret_cast<const uint4*>(Z + uint64_t(jt) * zs + sub * C::VEC);
        }
        float s[C::G];
        float mb = -INFINITY;
#pragma unroll
        for (int t = 0; t < C::G; ++t) {
            float r;
            if constexpr (RZ) {
                float f[C::VEC];
                unpack(raw[t], f);
                float pr = 0.0f;
#pragma unroll
                for (int x = 0; x < C::VEC; ++x) pr = __builtin_fmaf(f[x], arl[x], pr);
                pr += __shfl_xor(pr, 1);
                pr += __shfl_xor(pr, 2);
                r = pr + __shfl_xor(pr, 4);
            } else {
                r = __builtin_bit_cast(float, __shfl(raw[t].w, gbase + C::G - 1));
            }
            s[t] = t < cnt ? leaky(Li + r) : -INFINITY;
            mb = fmaxf(mb, s[t]);
        }
        if constexpr (RZ) {
            // Unpack the rows again below rather than keep 8 unpacked rows live.
#pragma unroll
            for (int t = 0; t < C::G; ++t) {
                uint32_t w0 = raw[t].x, w1 = raw[t].y, w2 = raw[t].z, w3 = raw[t].w;
                asm volatile("" : "+v"(w0), "+v"(w1), "+v"(w2), "+v"(w3));
                raw[t] = make_uint4(w0, w1, w2, w3);
            }
        }
        const float mn = fmaxf(m, mb);
        const float sc = exp_w(m - mn);  // 0 on the first batch (m = -inf)
        m = mn;
        dsum *= sc;
#pragma unroll
        for (int x = 0; x < C::VEC; ++x) acc[x] *= sc;
#pragma unroll
        for (int t = 0; t < C::G; ++t) {
            const float p = t < cnt ? exp_w(s[t] - mn) : 0.0f;
            dsum += p;
            float f[C::VEC];
            unpack(raw[t], f);
#pragma unroll
            for (int x = 0; x < C::VEC; ++x) acc[x] += p * f[x];
        }
    }
}

template <class C>
__device__ inline void store_row(uint32_t i, int W, int os, int sub, const float (&acc)[C::VEC], float d, bool hidden,
                                 float* out32, uint16_t* outbf) {
    const float scale = d > 0.0f ? 1.0f / d : 0.0f;
    if (out32 && os == C::G * C::VEC) {
        // Padded FP32 rows (the logits in original node order): each lane
        // stores its 16-byte pieces whole, zeros past W, so the scattered
        // rows are written as whole lines.
        static_assert(C::VEC % 4 == 0, "16-byte pieces");
#pragma unroll
        for (int x = 0; x < C::VEC; x += 4) {
            float y[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int f = sub * C::VEC + x + q;
                y[q] = f < W ? acc[x + q] * scale : 0.0f;
                if (hidden) y[q] = elu(y[q]);
            }
            *reinterpret_cast<float4*>(out32 + uint64_t(i) * os + sub * C::VEC + x) = make_float4(y[0], y[1], y[2], y[3]);
        }
        if (!outbf) return;
    }
#pragma unroll
    for (int x = 0; x < C::VEC; ++x) {
        const int f = sub * C::VEC + x;
        if (f >= W) continue;
        float y = acc[x] * scale;
        if (hidden) y = elu(y);
        if (out32 && os != C::G * C::VEC) out32[uint64_t(i) * W + f] = y;
        if (outbf) outbf[uint64_t(i) * W + f] = bf16_hw(y);
    }
}

// MODE 0: max pre-scan, then the accumulation pass (R from its own array);
// 1: one online pass, R in the last four bytes of each Z row; 2: one online
// pass, R recomputed from each Z row (one head of 64).
template <class C, class ZT, int MODE>
__global__ void __launch_bounds__(kThreads) k_agg_k1(K1Args<ZT> a) {
    const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int g = lane / C::G, sub = lane % C::G, gbase = g * C::G;
    const uint64_t wave = uint64_t(blockIdx.x) * kWavesPerBlock + w;
    float acc[C::VEC];
#pragma unroll
    for (int x = 0; x < C::VEC; ++x) acc[x] = 0.0f;
    float dloc = 0.0f;
    if (wave < a.chunks) {
        // ---------------- one chunk of a split row per wave
        const uint64_t c = wave;
        const uint32_t k = a.chunk_k[c], first = a.chunk_first[c];
        const uint64_t rbeg = a.prow[k], rend = a.prow[k + 1];
        const uint32_t i = a.perm[k];
        if (i >= a.n || rbeg > rend || rend > a.e) return;
        const uint32_t nch = uint32_t((rend - rbeg + a.chunk_edges - 1) / a.chunk_edges);
        const uint64_t cbeg = rbeg + uint64_t(c - first) * a.chunk_edges;
        const uint64_t cend = cbeg + a.chunk_edges < rend ? cbeg + a.chunk_edges : rend;
        float m = -INFINITY;
        for (uint32_t q = lane; q < nch; q += kWave) m = fmaxf(m, a.mchunk[(first + q) * 8]);
        for (int off = 1; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
        const float Li = a.L[i];
        const float Mi = leaky(Li + m);
        const uint64_t len = cend - cbeg;
        const uint64_t pb = cbeg + len * g / C::GPW, pe = cbeg + len * (g + 1) / C::GPW;
        group_accumulate<C, ZT>(pb, pe, a.pcol, a.R, a.rs, a.Z, a.zs, a.W, Li, Mi, gbase, sub, acc, dloc);
        for (int off = C::G; off < kWave; off <<= 1) {
#pragma unroll
            for (int x = 0; x < C::VEC; ++x) acc[x] += __shfl_xor(acc[x], off);
        }
        for (int off = 1; off < kWave; off <<= 1) dloc += __shfl_xor(dloc, off);
        float* part = a.part + c * (512 + 8);
        if (g == 0)
#pragma unroll
            for (int x = 0; x < C::VEC; ++x) part[sub * C::VEC + x] = acc[x];
        if (lane == 0) part[512] = dloc;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        uint32_t old = 0;
        if (lane == 0)
            old = __hip_atomic_fetch_add(a.counter + first, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __shfl(old, 0);
        if (old + 1 != nch) return;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        float tot[C::VEC];
#pragma unroll
        for (int x = 0; x < C::VEC; ++x) tot[x] = 0.0f;
        float dtot = 0.0f;
        for (uint32_t q = 0; q < nch; ++q) {
            const float* pq = a.part + uint64_t(first + q) * (512 + 8);
#pragma unroll
            for (int x = 0; x < C::VEC; ++x) tot[x] += pq[sub * C::VEC + x];
            dtot += pq[512];
        }
        if (lane == 0) {
            a.mx[i] = Mi;
            a.den[i] = dtot;
            a.counter[first] = 0;
        }
        if (g == 0) store_row<C>(a.operm ? a.operm[k] : i, a.W, a.os, sub, tot, dtot, a.hidden, a.out32, a.outbf);
        return;
    }
    // ---------------- 64/G whole rows per wave, heaviest first
    const uint64_t idx = (wave - a.chunks) * C::GPW + g;
    if (idx >= a.rows) return;  // whole groups exit; no wave-wide sync follows
    const uint64_t k = a.rows - 1 - idx;
    const uint32_t i = a.perm[k];
    const uint64_t beg = a.prow[k], end = a.prow[k + 1];
    if (i >= a.n || beg > end || end > a.e) return;
    const float Li = a.L[i];
    float Mi;
    if constexpr (MODE > 0) {
        float arl[C::VEC];
#pragma unroll
        for (int x = 0; x < C::VEC; ++x) arl[x] = MODE == 2 ? a.ar[sub * C::VEC + x] : 0.0f;
        float m = -INFINITY;
        group_online<C, MODE == 2>(beg, end, a.pcol, a.Z, a.zs, a.W, Li, gbase, sub, arl, acc, dloc, m);
        Mi = end > beg ? m : 0.0f;
    } else {
        const float m = group_max<C>(beg, end, a.pcol, a.R, a.rs, sub);
        Mi = end > beg ? leaky(Li + m) : 0.0f;
        group_accumulate<C, ZT>(beg, end, a.pcol, a.R, a.rs, a.Z, a.zs, a.W, Li, Mi, gbase, sub, acc, dloc);
        for (int off = 1; off < C::G; off <<= 1) dloc += __shfl_xor(dloc, off);
    }
    if (sub == 0) {
        a.mx[i] = Mi;
        a.den[i] = dloc;
    }
    store_row<C>(a.operm ? a.operm[k] : i, a.W, a.os, sub, acc, dloc, a.hidden, a.out32, a.outbf);
}

template <int G, class ZT>
hipError_t run(const AggArgs& g, const RowBins& bins, const SplitTable& t, hipStream_t s) {
    using C = K1<ZT, G>;
    // R read from the padding of the Z row when it was stored there (one
    // 128-byte line per edge), else from the separate array.
    const float* rptr = g.r_in_feat ? reinterpret_cast<const float*>(static_cast<const ZT*>(g.feat) + g.fstride - 2)
                                    : g.right;
    const int rs = g.r_in_feat ? int(g.fstride * sizeof(ZT) / 4) : 1;
    K1Args<ZT> a{g.prow, g.pcol, g.perm, g.left, rptr, static_cast<const ZT*>(g.feat), g.heads * g.dim,
                 g.fstride, rs, g.hidden, g.mx, g.den, g.out32, g.outbf, g.n, g.e, bins.split_begin, t.chunks,
                 t.chunk_k, t.chunk_first, t.chunk_edges, t.mchunk, t.part, t.counter, g.out_perm, g.ar,
                 g.out_perm && g.ostride ? g.ostride : g.heads * g.dim};
    if (a.os != a.W && (!a.operm || a.os != C::G * C::VEC)) return hipErrorInvalidValue;
    if (t.chunks) {
        hipError_t e = launch_split_prescan(g.prow, g.pcol, g.right, 1, t, g.e, s);
        if (e != hipSuccess) return e;
    }
    const uint64_t waves = t.chunks + (bins.split_begin + C::GPW - 1) / C::GPW;
    const dim3 grid(uint32_t((waves + kWavesPerBlock - 1) / kWavesPerBlock));
    if (!waves) return hipSuccess;
    if constexpr (sizeof(ZT) == 2 && G == 8) {
        if (g.r_in_feat) {
            // whole rows in one pass over their Z lines (R rides in the line)
            k_agg_k1<C, ZT, 1><<<grid, kThreads, 0, s>>>(a);
            return hipGetLastError();
        }
        if (g.r_from_z) {
            // whole rows in one pass, R recomputed from each line
            if (!g.ar || g.dim != 64 || g.fstride != 64) return hipErrorInvalidValue;
            k_agg_k1<C, ZT, 2><<<grid, kThreads, 0, s>>>(a);
            return hipGetLastError();
        }
    }
    k_agg_k1<C, ZT, 0><<<grid, kThreads, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace

int k1_out_stride(bool feat_bf16, int W) {
    if (feat_bf16) return K1<uint16_t, 8>::MAXW;
    return W <= 32 ? K1<float, 8>::MAXW : K1<float, 16>::MAXW;
}

bool aggregate_k1_supported(const AggArgs& g) {
    const int W = g.dim;
    if (g.heads != 1 || W > 64) return false;
    const int vec = g.feat_bf16 ? 8 : 4;
    return g.fstride % vec == 0 && g.fstride >= W;
}

hipError_t launch_aggregate_k1(const AggArgs& g, const RowBins& bins, const SplitTable& t, hipStream_t s) {
    const int W = g.dim;
    if (g.feat_bf16) return W <= 64 ? run<8, uint16_t>(g, bins, t, s) : hipErrorInvalidValue;
    if (W <= 32) return run<8, float>(g, bins, t, s);
    return run<16, float>(g, bins, t, s);
}

}  // namespace gatgpu
