// Vectorised transform-first aggregation for rows whose width is a multiple
// of one 16-byte vector per lane (8 bf16 or 4 FP32 features), e.g. 8 heads x
// 32 or 8 x 64.  Same mathematics as aggregate.hip (baseline_standard.cpp:44-97):
// exact row max first, then p = exp(LeakyReLU(L+R) - M), den = sum p,
// out = ELU?(sum p Z / den).
//
// Work items (one wave each, 4 waves per block):
//   * chunks of split rows (in-degree >= split_min): C edges each.  A first
//     kernel stores every chunk's per-head maximum; the aggregation kernel
//     reads the maxima of all chunks of its row, so every chunk uses the exact
//     row max, and the partial (sum p Z, sum p) of a chunk needs no rescaling.
//     Partials go to scratch; the last chunk to arrive (agent-scope acq_rel
//     counter) adds them in chunk order -- deterministic -- and finishes the row.
//   * whole rows below split_min, heaviest first.
//
// Lane roles inside a wave, per batch of EB edges:
//   scorer   pair q = lane + 64 s -> edge q / K, head q % K: one exp per (edge, head)
//   reader   slot = lane / LPR, sub = lane % LPR: loads 16 bytes of edge
//            (u*EPI + slot)'s row for u < NU, i.e. EPI edges per instruction.
// Scores and source ids pass from scorers to readers through LDS, laid out so
// that each reader fetches its NU values with 128-bit LDS reads.
#include "internal.hpp"

namespace gatgpu {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;

template <class ZT, int W_, int K_, int BE_>
struct Cfg {
    static constexpr int W = W_, K = K_, BE = BE_;    // BE: edges scored per block
    static constexpr int VEC = 16 / int(sizeof(ZT));  // features per 16-byte load
    static constexpr int DIM = W / K;
    static constexpr int LPR = W / VEC;               // lanes (16-byte vectors) per row
    static constexpr int EPI = LPR >= kWave ? 1 : kWave / LPR;  // edges per load instruction
    static constexpr int VPL = LPR <= kWave ? 1 : LPR / kWave;  // vectors per lane per edge
    static constexpr int NUB = BE / EPI;              // load instructions of a full block
    static constexpr int S = BE * K / kWave;          // (edge, head) scores per lane per block
    static constexpr int G = 8;                       // load instructions in flight per group
    static constexpr int ACC = VPL * VEC;
    static_assert(W % K == 0 && DIM % VEC == 0, "a vector must not straddle two heads");
    static_assert(LPR * EPI == kWave || LPR % kWave == 0, "lanes per row must divide or fill the wave");
    static_assert(BE % EPI == 0 && (BE * K) % kWave == 0 && NUB % G == 0, "block must fill whole groups");
    static_assert(kWave % K == 0, "heads must divide the wave");
};

struct SplitArgs {
    uint64_t chunks;
    const uint32_t* chunk_k;      // sorted position of the chunk's row
    const uint32_t* chunk_first;  // first chunk of that row
    uint32_t chunk_edges;
    float* mchunk;                // [chunks][8]
    float* part;                  // [chunks][W + 8]
    uint32_t* counter;            // [chunks], indexed by a row's first chunk
};

template <class ZT>
struct VArgs {
    const uint64_t* prow;
    const uint32_t* pcol;
    const uint32_t* perm;
    const float* L;
    const float* R;
    const ZT* Z;
    bool hidden;
    float* mx;
    float* den;
    float* out32;
    uint16_t* outbf;
    uint64_t n, e;
    uint64_t rows;  // non-split rows: sorted positions [0, rows)
    SplitArgs sp;
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

// Per-lane state of one row (or chunk) aggregation.
template <class C>
struct RowAcc {
    float acc[C::ACC];
    float dloc;
};

// Max of R[j, head] over edges [beg, end) for this lane's head, reduced over
// the lanes of the same head (lane l covers edges l/K, l/K + 64/K, ...).
template <class C>
__device__ inline float row_max(uint64_t beg, uint64_t end, const uint32_t* __restrict__ pcol,
                                const float* __restrict__ R) {
    const int lane = threadIdx.x % kWave, hs = lane % C::K;
    float m = -INFINITY;
    for (uint64_t e = beg + lane / C::K; e < end; e += kWave / C::K) m = fmaxf(m, R[uint64_t(pcol[e]) * C::K + hs]);
    for (int off = C::K; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
    return m;
}

// One block of cnt <= BE edges starting at base.  Every lane loads the source
// ids and R values of its S (edge, head) pairs once; with FIND_MAX (a row
// that fits one block) the exact row max comes from those registers, so R is
// read once per edge.  Scores and ids go to LDS in reader order, then the
// Z rows are gathered in groups of G 16-byte loads per lane, double-buffered
// so that one group's loads are in flight while the previous group's FMAs run.
template <class C, class ZT, bool FIND_MAX>
__device__ inline void block(uint64_t base, int cnt, const uint32_t* __restrict__ pcol,
                             const float* __restrict__ R, const ZT* __restrict__ Z, float Lh, float& Mh,
                             float* pb, uint32_t* jb, RowAcc<C>& st) {
    const int lane = threadIdx.x % kWave;
    const int hs = lane % C::K;
    const int slot = C::EPI > 1 ? lane / C::LPR : 0;
    const int sub = C::EPI > 1 ? lane % C::LPR : lane;
    uint32_t jv[C::S];
    float rv[C::S];
#pragma unroll
    for (int s = 0; s < C::S; ++s) {
        const int t = lane / C::K + (kWave / C::K) * s;
        jv[s] = t < cnt ? pcol[base + t] : 0u;
        rv[s] = t < cnt ? R[uint64_t(jv[s]) * C::K + hs] : -INFINITY;
    }
    if constexpr (FIND_MAX) {
        float m = rv[0];
#pragma unroll
        for (int s = 1; s < C::S; ++s) m = fmaxf(m, rv[s]);
        for (int off = C::K; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
        Mh = leaky(Lh + m);
    }
#pragma unroll
    for (int s = 0; s < C::S; ++s) {
        const int t = lane / C::K + (kWave / C::K) * s;
        const float p = t < cnt ? expf(leaky(Lh + rv[s]) - Mh) : 0.0f;
        st.dloc += p;
        const int u = t / C::EPI, sl = t % C::EPI;
        pb[(hs * C::EPI + sl) * C::NUB + u] = p;
        if (hs == 0) jb[sl * C::NUB + u] = jv[s];
    }
    wave_sync();
    int hr[C::VPL];
#pragma unroll
    for (int v = 0; v < C::VPL; ++v) hr[v] = ((sub + kWave * v) * C::VEC) / C::DIM;
    const int nu = (cnt + C::EPI - 1) / C::EPI;  // load instructions of this block
    uint4 buf[2][C::G][C::VPL];
    auto issue = [&](int b, int u0) {
#pragma unroll
        for (int q = 0; q < C::G; ++q) {
            const int u = u0 + q;
            const bool ok = u * C::EPI + slot < cnt;
            const uint32_t j = jb[slot * C::NUB + (u < C::NUB ? u : 0)];
            const ZT* row = Z + uint64_t(j) * C::W;
#pragma unroll
            for (int v = 0; v < C::VPL; ++v)
                buf[b][q][v] = ok ? *reinterpret_cast<const uint4*>(row + (sub + kWave * v) * C::VEC)
                                  : make_uint4(0, 0, 0, 0);
        }
    };
    auto consume = [&](int b, int u0) {
#pragma unroll
        for (int q = 0; q < C::G; ++q) {
            const int u = u0 + q < C::NUB ? u0 + q : 0;
#pragma unroll
            for (int v = 0; v < C::VPL; ++v) {
                const float p = pb[(hr[v] * C::EPI + slot) * C::NUB + u];
                float f[C::VEC];
                unpack(buf[b][q][v], f);
#pragma unroll
                for (int x = 0; x < C::VEC; ++x) st.acc[v * C::VEC + x] += p * f[x];
            }
        }
    };
    // Groups beyond nu load nothing (ok == false) and add zeros.
    issue(0, 0);
    for (int u0 = 0; u0 < nu; u0 += 2 * C::G) {
        if (u0 + C::G < nu) issue(1, u0 + C::G);
        consume(0, u0);
        if (u0 + C::G < nu) {
            if (u0 + 2 * C::G < nu) issue(0, u0 + 2 * C::G);
            consume(1, u0 + C::G);
        }
    }
    wave_sync();
}

// Edges [beg, end) of a row or chunk whose max is known (Mh) or, for a row
// that fits one block, found on the way.
template <class C, class ZT>
__device__ inline void accumulate(uint64_t beg, uint64_t end, bool find_max, const uint32_t* __restrict__ pcol,
                                  const float* __restrict__ R, const ZT* __restrict__ Z, float Lh, float& Mh,
                                  float* pb, uint32_t* jb, RowAcc<C>& st) {
    if (find_max) {
        block<C, ZT, true>(beg, int(end - beg), pcol, R, Z, Lh, Mh, pb, jb, st);
        return;
    }
    for (uint64_t base = beg; base < end; base += C::BE) {
        const uint64_t rem = end - base;
        block<C, ZT, false>(base, rem < uint64_t(C::BE) ? int(rem) : C::BE, pcol, R, Z, Lh, Mh, pb, jb, st);
    }
}

// Sum the denominators over scorer lanes of the same head (lanes < K end up
// with head lane's total) and the accumulators over the EPI edge slots.
template <class C>
__device__ inline void reduce_lanes(RowAcc<C>& st) {
    for (int off = C::K; off < kWave; off <<= 1) st.dloc += __shfl_xor(st.dloc, off);
    if constexpr (C::EPI > 1) {
#pragma unroll
        for (int x = 0; x < C::ACC; ++x)
            for (int off = C::LPR; off < kWave; off <<= 1) st.acc[x] += __shfl_xor(st.acc[x], off);
    }
}

// Normalise, ELU, store one output row (slot-0 lanes), den/M rows (lanes < K).
template <class C>
__device__ inline void finish_row(uint32_t i, const float (&acc)[C::ACC], const float* dsh, bool hidden,
                                  float* out32, uint16_t* outbf) {
    const int lane = threadIdx.x % kWave;
    if (C::EPI > 1 && lane >= C::LPR) return;  // slot-0 lanes hold the reduced sums
    const int sub = lane;
#pragma unroll
    for (int v = 0; v < C::VPL; ++v) {
        const int f0 = (sub + kWave * v) * C::VEC;
        const float d = dsh[f0 / C::DIM];
        const float scale = d > 0.0f ? 1.0f / d : 0.0f;
        float o[C::VEC];
#pragma unroll
        for (int x = 0; x < C::VEC; ++x) {
            float y = acc[v * C::VEC + x] * scale;
            o[x] = hidden ? elu(y) : y;
        }
        const uint64_t off = uint64_t(i) * C::W + f0;
        if (outbf) {
            uint32_t w[C::VEC / 2];
#pragma unroll
            for (int x = 0; x < C::VEC / 2; ++x)
                w[x] = uint32_t(bf16_rne(o[2 * x])) | (uint32_t(bf16_rne(o[2 * x + 1])) << 16);
            if constexpr (C::VEC == 8) *reinterpret_cast<uint4*>(outbf + off) = make_uint4(w[0], w[1], w[2], w[3]);
            else *reinterpret_cast<uint2*>(outbf + off) = make_uint2(w[0], w[1]);
        }
        if (out32) {
#pragma unroll
            for (int x = 0; x < C::VEC; x += 4)
                *reinterpret_cast<float4*>(out32 + off + x) = make_float4(o[x], o[x + 1], o[x + 2], o[x + 3]);
        }
    }
}

// Per-head max of R over a chunk's edges -> mchunk[c][h].
template <int K>
__global__ void __launch_bounds__(kThreads)
k_split_prescan(const uint64_t* __restrict__ prow, const uint32_t* __restrict__ pcol, const float* __restrict__ R,
                SplitArgs sp, uint64_t e_total) {
    const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const uint64_t c = uint64_t(blockIdx.x) * kWavesPerBlock + w;
    if (c >= sp.chunks) return;
    const uint32_t k = sp.chunk_k[c], first = sp.chunk_first[c];
    const uint64_t beg = prow[k] + uint64_t(c - first) * sp.chunk_edges;
    uint64_t end = beg + sp.chunk_edges;
    if (end > prow[k + 1]) end = prow[k + 1];
    if (end > e_total) end = e_total;
    const int h = lane % K;
    float m = -INFINITY;
    for (uint64_t e = beg + lane / K; e < end; e += kWave / K) m = fmaxf(m, R[uint64_t(pcol[e]) * K + h]);
    for (int off = K; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (lane < K) sp.mchunk[c * 8 + lane] = m;
}

template <class C, class ZT>
__global__ void __launch_bounds__(kThreads) k_agg_vec(VArgs<ZT> a) {
    __shared__ float pbuf[kWavesPerBlock][C::K * C::BE];
    __shared__ uint32_t jbuf[kWavesPerBlock][C::BE];
    __shared__ float dsh[kWavesPerBlock][8];
    const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const uint64_t item = uint64_t(blockIdx.x) * kWavesPerBlock + w;
    const int hs = lane % C::K;
    RowAcc<C> st;
#pragma unroll
    for (int x = 0; x < C::ACC; ++x) st.acc[x] = 0.0f;
    st.dloc = 0.0f;
    if (item < a.sp.chunks) {
        // ---------------- chunk of a split row
        const uint64_t c = item;
        const uint32_t k = a.sp.chunk_k[c], first = a.sp.chunk_first[c];
        const uint64_t rbeg = a.prow[k], rend = a.prow[k + 1];
        const uint32_t i = a.perm[k];
        if (i >= a.n || rbeg > rend || rend > a.e) return;
        const uint32_t nch = uint32_t((rend - rbeg + a.sp.chunk_edges - 1) / a.sp.chunk_edges);
        const uint64_t beg = rbeg + uint64_t(c - first) * a.sp.chunk_edges;
        const uint64_t end = beg + a.sp.chunk_edges < rend ? beg + a.sp.chunk_edges : rend;
        float m = -INFINITY;
        for (uint32_t q = lane / C::K; q < nch; q += kWave / C::K) m = fmaxf(m, a.sp.mchunk[(first + q) * 8 + hs]);
        for (int off = C::K; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
        const float Lh = a.L[uint64_t(i) * C::K + hs];
        float Mh = leaky(Lh + m);
        accumulate<C, ZT>(beg, end, false, a.pcol, a.R, a.Z, Lh, Mh, pbuf[w], jbuf[w], st);
        reduce_lanes<C>(st);
        float* part = a.sp.part + c * (C::W + 8);
        const int slot = C::EPI > 1 ? lane / C::LPR : 0;
        const int sub = C::EPI > 1 ? lane % C::LPR : lane;
        if (slot == 0)
#pragma unroll
            for (int v = 0; v < C::VPL; ++v)
#pragma unroll
                for (int x = 0; x < C::VEC; x += 4)
                    *reinterpret_cast<float4*>(part + (sub + kWave * v) * C::VEC + x) =
                        make_float4(st.acc[v * C::VEC + x], st.acc[v * C::VEC + x + 1], st.acc[v * C::VEC + x + 2],
                                    st.acc[v * C::VEC + x + 3]);
        if (lane < C::K) part[C::W + lane] = st.dloc;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        uint32_t old = 0;
        if (lane == 0)
            old = __hip_atomic_fetch_add(a.sp.counter + first, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __shfl(old, 0);
        if (old + 1 != nch) return;  // not the last chunk of this row
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        // Last arrival: add the partials of every chunk in chunk order.
        float tot[C::ACC];
#pragma unroll
        for (int x = 0; x < C::ACC; ++x) tot[x] = 0.0f;
        float dtot = 0.0f;
        for (uint32_t q = 0; q < nch; ++q) {
            const float* pq = a.sp.part + uint64_t(first + q) * (C::W + 8);
            if (slot == 0)
#pragma unroll
                for (int v = 0; v < C::VPL; ++v)
#pragma unroll
                    for (int x = 0; x < C::VEC; x += 4) {
                        const float4 t = *reinterpret_cast<const float4*>(pq + (sub + kWave * v) * C::VEC + x);
                        tot[v * C::VEC + x] += t.x;
                        tot[v * C::VEC + x + 1] += t.y;
                        tot[v * C::VEC + x + 2] += t.z;
                        tot[v * C::VEC + x + 3] += t.w;
                    }
            if (lane < C::K) dtot += pq[C::W + lane];
        }
        if (lane < C::K) {
            a.mx[uint64_t(i) * C::K + lane] = Mh;
            a.den[uint64_t(i) * C::K + lane] = dtot;
            dsh[w][lane] = dtot;
        }
        if (lane == 0) a.sp.counter[first] = 0;  // ready for the next launch
        wave_sync();
        finish_row<C>(i, tot, dsh[w], a.hidden, a.out32, a.outbf);
        return;
    }
    // ---------------- whole row, heaviest first
    const uint64_t widx = item - a.sp.chunks;
    if (widx >= a.rows) return;
    const uint64_t k = a.rows - 1 - widx;
    const uint32_t i = a.perm[k];
    const uint64_t beg = a.prow[k], end = a.prow[k + 1];
    if (i >= a.n || beg > end || end > a.e) return;
    const float Lh = a.L[uint64_t(i) * C::K + hs];
    const uint64_t deg = end - beg;
    // Empty row: max 0, denominator 0, output 0 (baseline/src/ref_fp32.cpp:11).
    float Mh = 0.0f;
    if (deg > uint64_t(C::BE)) Mh = leaky(Lh + row_max<C>(beg, end, a.pcol, a.R));
    if (deg) accumulate<C, ZT>(beg, end, deg <= uint64_t(C::BE), a.pcol, a.R, a.Z, Lh, Mh, pbuf[w], jbuf[w], st);
    reduce_lanes<C>(st);
    if (lane < C::K) {
        a.mx[uint64_t(i) * C::K + lane] = Mh;
        a.den[uint64_t(i) * C::K + lane] = st.dloc;
        dsh[w][lane] = st.dloc;
    }
    wave_sync();
    finish_row<C>(i, st.acc, dsh[w], a.hidden, a.out32, a.outbf);
}

template <class C, class ZT>
hipError_t run(const AggArgs& g, const RowBins& bins, const SplitTable& t, hipStream_t s) {
    VArgs<ZT> a{g.prow, g.pcol, g.perm, g.left, g.right, static_cast<const ZT*>(g.feat), g.hidden, g.mx, g.den,
                g.out32, g.outbf, g.n, g.e, bins.split_begin,
                SplitArgs{t.chunks, t.chunk_k, t.chunk_first, t.chunk_edges, t.mchunk, t.part, t.counter}};
    if (t.chunks) {
        hipError_t e = launch_split_prescan(g.prow, g.pcol, g.right, C::K, t, g.e, s);
        if (e != hipSuccess) return e;
    }
    const uint64_t items = t.chunks + bins.split_begin;
    if (items)
        k_agg_vec<C, ZT><<<dim3(uint32_t((items + kWavesPerBlock - 1) / kWavesPerBlock)), kThreads, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_split_prescan(const uint64_t* prow, const uint32_t* pcol, const float* right, int heads,
                                const SplitTable& t, uint64_t e, hipStream_t s) {
    if (!t.chunks) return hipSuccess;
    const SplitArgs sp{t.chunks, t.chunk_k, t.chunk_first, t.chunk_edges, t.mchunk, t.part, t.counter};
    const dim3 grid(uint32_t((t.chunks + kWavesPerBlock - 1) / kWavesPerBlock));
    switch (heads) {
        case 1: k_split_prescan<1><<<grid, kThreads, 0, s>>>(prow, pcol, right, sp, e); break;
        case 2: k_split_prescan<2><<<grid, kThreads, 0, s>>>(prow, pcol, right, sp, e); break;
        case 4: k_split_prescan<4><<<grid, kThreads, 0, s>>>(prow, pcol, right, sp, e); break;
        case 8: k_split_prescan<8><<<grid, kThreads, 0, s>>>(prow, pcol, right, sp, e); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool aggregate_vec_supported(const AggArgs& g) {
    const int W = g.heads * g.dim;
    return g.heads == 8 && (W == 256 || W == 512) && g.fstride == W;
}

hipError_t launch_aggregate_vec(const AggArgs& g, const RowBins& bins, const SplitTable& t, hipStream_t s) {
    const int W = g.heads * g.dim;
    if (g.heads != 8) return hipErrorInvalidValue;
    if (g.feat_bf16) {
        if (W == 256) return run<Cfg<uint16_t, 256, 8, 64>, uint16_t>(g, bins, t, s);
        if (W == 512) return run<Cfg<uint16_t, 512, 8, 64>, uint16_t>(g, bins, t, s);
    } else {
        if (W == 256) return run<Cfg<float, 256, 8, 64>, float>(g, bins, t, s);
        if (W == 512) return run<Cfg<float, 512, 8, 64>, float>(g, bins, t, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace gatgpu
