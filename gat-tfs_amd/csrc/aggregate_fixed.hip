// Fixed-p transform-first aggregation: the operator of the reference
// harness's fixed-p mode (baseline/bench/main.cpp:103-150), i.e.
// standard_aggregate with fixed_p/fixed_den followed by finish(hidden = false)
// (baseline/src/baseline_standard.cpp:52-97):
//   out[i, h, :] = (sum_e p[e, h] Z[col[e], h, :]) * (den[i, h] > 0 ? 1 / den[i, h] : 0)
// The attention weights p and denominators den come from a fixture instead of
// the L/R front end, which isolates the gather-multiply-add from the softmax.
// The DEN stage is the fixture's den, as the reference stores it.
//
// p is read in degree-sorted edge order (permuted once when the fixture is
// uploaded), so a batch's weights are one contiguous run.  Layout and work
// items follow the softmax kernel of aggregate_vec.hip: one wave per row or
// split-row chunk, lane (slot, sub) reads vector sub of the edges with index
// slot (mod EPI), source ids arrive wave-uniform through scalar loads.  Chunks
// write partial sums; the last chunk to arrive adds them in chunk order.
#include "internal.hpp"

namespace gatgpu {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;

// VEC features per lane load: 16-byte vectors, or single elements (VEC 1)
// for rows whose vectors would straddle two heads.
template <class ZT, int VEC_, int EPI_, int VPL_>
struct FCfg {
    static constexpr int VEC = VEC_, EPI = EPI_, VPL = VPL_;
    static constexpr int LPR = kWave / EPI;        // lanes per source row
    static constexpr int COVER = LPR * VPL * VEC;  // features covered per row
    static constexpr int U = VPL > 1 ? 4 : EPI > 8 ? kWave / EPI : 8;  // loads per vector per batch
    static constexpr int BATCH = U * EPI;
    static constexpr int ACC = VPL * VEC;
    static_assert(VEC == 1 || VEC * int(sizeof(ZT)) == 16, "16-byte vectors or single elements");
    static_assert(BATCH <= int(kPcolPad), "a batch may read at most kPcolPad ids past the row");
};

template <class ZT>
struct FArgs {
    const uint64_t* prow;
    const uint32_t* pcol;
    const uint32_t* perm;
    const float* P;  // [e][K], degree-sorted edge order
    const float* D;  // [n][K], original row order
    const ZT* Z;
    int K, dim, W, zs;
    float* den;      // DEN stage [n][K]
    float* out32;    // [n][W]
    uint64_t n, e, rows;
    uint64_t chunks;
    const uint32_t* chunk_k;
    const uint32_t* chunk_first;
    uint32_t chunk_edges;
    float* part;
    uint32_t* counter;
};

// Raw lane load: a 16-byte vector, or one element widened to FP32.
template <int VEC>
struct RawOf {
    using type = uint4;
};
template <>
struct RawOf<1> {
    using type = float;
};

template <int VEC, class ZT>
__device__ inline typename RawOf<VEC>::type load_raw(const ZT* p, bool ok) {
    if constexpr (VEC == 1) {
        if (!ok) return 0.0f;
        if constexpr (sizeof(ZT) == 2) return bf16_widen(*reinterpret_cast<const uint16_t*>(p));
        else return *reinterpret_cast<const float*>(p);
    } else {
        return ok ? *reinterpret_cast<const uint4*>(p) : make_uint4(0, 0, 0, 0);
    }
}

template <int VEC, class ZT>
__device__ inline void unpack(const typename RawOf<VEC>::type& v, float (&f)[VEC]) {
    if constexpr (VEC == 1) {
        f[0] = v;
    } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        if constexpr (sizeof(ZT) == 2) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                f[2 * q] = __builtin_bit_cast(float, w[q] << 16);
                f[2 * q + 1] = __builtin_bit_cast(float, w[q] & 0xffff0000u);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) f[q] = __builtin_bit_cast(float, w[q]);
        }
    }
}

// Edges [beg, end) into acc.  h[v]: head of the lane's vector v (clamped to
// K - 1 for lanes past the row width, whose sums are never stored).
template <class C, class ZT>
__device__ inline void fixed_range(uint64_t beg, uint64_t end, const FArgs<ZT>& a, int slot, int sub,
                                   const int (&h)[C::VPL], float (&acc)[C::ACC]) {
    for (uint64_t base = beg; base < end; base += C::BATCH) {
        uint32_t js[C::BATCH];
#pragma unroll
        for (int t = 0; t < C::BATCH; ++t) js[t] = a.pcol[base + t];  // wave-uniform, padded past e
        typename RawOf<C::VEC>::type raw[C::U][C::VPL];
        float p[C::U][C::VPL];
#pragma unroll
        for (int u = 0; u < C::U; ++u) {
            uint32_t j = js[u * C::EPI];
#pragma unroll
            for (int q = 1; q < C::EPI; ++q) j = slot == q ? js[u * C::EPI + q] : j;
            const uint64_t e = base + uint64_t(u * C::EPI + slot);
            const bool ok = e < end;
            const ZT* row = a.Z + uint64_t(j) * a.zs;
#pragma unroll
            for (int v = 0; v < C::VPL; ++v) {
                const int f0 = (sub + C::LPR * v) * C::VEC;
                raw[u][v] = load_raw<C::VEC>(row + f0, ok && f0 < a.zs);
                p[u][v] = ok ? a.P[e * a.K + h[v]] : 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < C::U; ++u)
#pragma unroll
            for (int v = 0; v < C::VPL; ++v) {
                float f[C::VEC];
                unpack<C::VEC, ZT>(raw[u][v], f);
#pragma unroll
                for (int x = 0; x < C::VEC; ++x) acc[v * C::VEC + x] += p[u][v] * f[x];
            }
    }
    if constexpr (C::EPI > 1) {
        for (int off = C::LPR; off < kWave; off <<= 1)
#pragma unroll
            for (int x = 0; x < C::ACC; ++x) acc[x] += __shfl_xor(acc[x], off);
    }
}

template <class C, class ZT>
__device__ inline void store_fixed(uint32_t i, const FArgs<ZT>& a, int slot, int sub, const int (&h)[C::VPL],
                                   const float (&acc)[C::ACC]) {
    if (slot != 0) return;
#pragma unroll
    for (int v = 0; v < C::VPL; ++v) {
        const float d = a.D[uint64_t(i) * a.K + h[v]];
        const float scale = d > 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
        for (int x = 0; x < C::VEC; ++x) {
            const int f = (sub + C::LPR * v) * C::VEC + x;
            if (f >= a.W) continue;
            if (f % a.dim == 0) a.den[uint64_t(i) * a.K + h[v]] = d;
            a.out32[uint64_t(i) * a.W + f] = acc[v * C::VEC + x] * scale;
        }
    }
}

template <class C, class ZT>
__global__ void __launch_bounds__(kThreads) k_fixed(FArgs<ZT> a) {
    const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = threadIdx.x % kWave;
    const int slot = lane / C::LPR, sub = lane % C::LPR;
    const uint64_t item = uint64_t(blockIdx.x) * kWavesPerBlock + w;
    int h[C::VPL];
#pragma unroll
    for (int v = 0; v < C::VPL; ++v) {
        const int f0 = (sub + C::LPR * v) * C::VEC;
        h[v] = f0 < a.W ? f0 / a.dim : a.K - 1;
    }
    float acc[C::ACC];
#pragma unroll
    for (int x = 0; x < C::ACC; ++x) acc[x] = 0.0f;
    if (item < a.chunks) {
        // ---------------- chunk of a split row
        const uint64_t c = item;
        const uint32_t k = a.chunk_k[c], first = a.chunk_first[c];
        const uint64_t rbeg = a.prow[k], rend = a.prow[k + 1];
        const uint32_t i = a.perm[k];
        if (i >= a.n || rbeg > rend || rend > a.e) return;
        const uint32_t nch = uint32_t((rend - rbeg + a.chunk_edges - 1) / a.chunk_edges);
        const uint64_t beg = rbeg + uint64_t(c - first) * a.chunk_edges;
        const uint64_t end = beg + a.chunk_edges < rend ? beg + a.chunk_edges : rend;
        fixed_range<C, ZT>(beg, end, a, slot, sub, h, acc);
        float* part = a.part + c * (C::COVER + 8);
        if (slot == 0)
#pragma unroll
            for (int v = 0; v < C::VPL; ++v)
#pragma unroll
                for (int x = 0; x < C::VEC; ++x) part[(sub + C::LPR * v) * C::VEC + x] = acc[v * C::VEC + x];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        uint32_t old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(a.counter + first, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __shfl(old, 0);
        if (old + 1 != nch) return;  // not the last chunk of this row
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        float tot[C::ACC];
#pragma unroll
        for (int x = 0; x < C::ACC; ++x) tot[x] = 0.0f;
        for (uint32_t q = 0; q < nch; ++q) {
            const float* pq = a.part + uint64_t(first + q) * (C::COVER + 8);
#pragma unroll
            for (int v = 0; v < C::VPL; ++v)
#pragma unroll
                for (int x = 0; x < C::VEC; ++x) tot[v * C::VEC + x] += pq[(sub + C::LPR * v) * C::VEC + x];
        }
        if (lane == 0) a.counter[first] = 0;  // ready for the next launch
        store_fixed<C, ZT>(i, a, slot, sub, h, tot);
        return;
    }
    // ---------------- whole row, heaviest first
    const uint64_t widx = item - a.chunks;
    if (widx >= a.rows) return;
    const uint64_t k = a.rows - 1 - widx;
    const uint32_t i = a.perm[k];
    const uint64_t beg = a.prow[k], end = a.prow[k + 1];
    if (i >= a.n || beg > end || end > a.e) return;
    fixed_range<C, ZT>(beg, end, a, slot, sub, h, acc);
    store_fixed<C, ZT>(i, a, slot, sub, h, acc);
}

template <class C, class ZT>
hipError_t run(const FArgs<ZT>& a, hipStream_t s) {
    const uint64_t items = a.chunks + a.rows;
    if (!items) return hipSuccess;
    k_fixed<C, ZT><<<dim3(uint32_t((items + kWavesPerBlock - 1) / kWavesPerBlock)), kThreads, 0, s>>>(a);
    return hipGetLastError();
}

// 16-byte vectors when each lies inside one head and the padded row splits
// into a power-of-two number of vectors; single elements otherwise.
template <class ZT>
hipError_t dispatch(const FArgs<ZT>& a, hipStream_t s) {
    constexpr int VEC = 16 / int(sizeof(ZT));
    const bool vec_ok = (a.K == 1 || a.dim % VEC == 0) && a.zs % VEC == 0;
    const int vecs = a.zs / VEC;
    if (vec_ok) {
        switch (vecs) {
            case 4: return run<FCfg<ZT, VEC, 16, 1>, ZT>(a, s);
            case 8: return run<FCfg<ZT, VEC, 8, 1>, ZT>(a, s);
            case 16: return run<FCfg<ZT, VEC, 4, 1>, ZT>(a, s);
            case 32: return run<FCfg<ZT, VEC, 2, 1>, ZT>(a, s);
            case 64: return run<FCfg<ZT, VEC, 1, 1>, ZT>(a, s);
            case 128: return run<FCfg<ZT, VEC, 1, 2>, ZT>(a, s);
            default: break;
        }
    }
    const int nf = (a.W + kWave - 1) / kWave;
    if (nf <= 1) return run<FCfg<ZT, 1, 1, 1>, ZT>(a, s);
    if (nf <= 2) return run<FCfg<ZT, 1, 1, 2>, ZT>(a, s);
    if (nf <= 4) return run<FCfg<ZT, 1, 1, 4>, ZT>(a, s);
    if (nf <= 8) return run<FCfg<ZT, 1, 1, 8>, ZT>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_aggregate_fixed(const AggArgs& g, const float* p_sorted, const float* den_fixture,
                                  const RowBins& bins, const SplitTable& t, hipStream_t s) {
    const int W = g.heads * g.dim;
    if (g.heads < 1 || g.heads > 8 || W > 512 || g.fstride < W) return hipErrorInvalidValue;
    if (g.feat_bf16) {
        FArgs<uint16_t> a{g.prow, g.pcol, g.perm, p_sorted, den_fixture, static_cast<const uint16_t*>(g.feat),
                          g.heads, g.dim, W, g.fstride, g.den, g.out32, g.n, g.e, bins.split_begin, t.chunks,
                          t.chunk_k, t.chunk_first, t.chunk_edges, t.part, t.counter};
        return dispatch(a, s);
    }
    FArgs<float> a{g.prow, g.pcol, g.perm, p_sorted, den_fixture, static_cast<const float*>(g.feat),
                   g.heads, g.dim, W, g.fstride, g.den, g.out32, g.n, g.e, bins.split_begin, t.chunks,
                   t.chunk_k, t.chunk_first, t.chunk_edges, t.part, t.counter};
    return dispatch(a, s);
}

}  // namespace gatgpu
