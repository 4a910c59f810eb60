// Fused exact-max softmax + CSR SpMM aggregation (transform-first GAT layer).
//
// For destination row i and head h (reference: max_prescan and
// standard_aggregate, baseline/src/baseline_standard.cpp:44-84, and finish,
// :85-97):
//   M[i,h]   = LeakyReLU(L[i,h] + max_{j in N(i)} R[j,h])      (0 for an empty row)
//   p_ij^h   = exp(LeakyReLU(L[i,h] + R[j,h]) - M[i,h])
//   den[i,h] = sum_j p_ij^h
//   out[i,h,:] = ELU?( (sum_j p_ij^h Z[j,h,:]) * (den>0 ? 1/den : 0) )
// Rows are visited in degree-sorted order through the permuted CSR (prow,
// pcol) and written back to their original index perm[k].  One owner per row
// (a wave or a block) writes each output row: no atomics outside split rows.
//
// Lane mapping inside a wave: with Kp = next power of two >= K heads, lane l
// scores edge (l / Kp) of the current batch for head (l % Kp), so a batch
// holds 64/Kp edges and one exp per (edge, head).  The scores go through LDS
// ([head][edge]) to the lanes that own the features: feature f = lane + 64q
// of the output row belongs to head f / dim.
#include "internal.hpp"

namespace gatgpu {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;

__device__ inline float load_feat(const float* p, uint64_t idx) { return p[idx]; }
__device__ inline float load_feat(const uint16_t* p, uint64_t idx) { return bf16_widen(p[idx]); }

struct Lanes {
    int kp_log2, kp, eb_count, eb, hh;
    bool hvalid;
};
__device__ inline Lanes lanes_for(int K) {
    Lanes l;
    l.kp_log2 = K <= 1 ? 0 : K <= 2 ? 1 : K <= 4 ? 2 : 3;
    l.kp = 1 << l.kp_log2;
    l.eb_count = kWave >> l.kp_log2;
    const int lane = threadIdx.x % kWave;
    l.eb = lane >> l.kp_log2;
    l.hh = lane & (l.kp - 1);
    l.hvalid = l.hh < K;
    return l;
}

// Max of R[j,hh] over edges [beg, end) handled by this lane's edge slot,
// reduced over the lanes of the same head.
__device__ inline float range_max(uint64_t beg, uint64_t end, const uint32_t* __restrict__ pcol,
                                  const float* __restrict__ R, int K, const Lanes& ln) {
    float m = -INFINITY;
    if (ln.hvalid)
        for (uint64_t e = beg + ln.eb; e < end; e += ln.eb_count)
            m = fmaxf(m, R[uint64_t(pcol[e]) * K + ln.hh]);
    for (int off = ln.kp; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
    return m;
}

// Accumulates edges [beg, end) of one row into acc (features lane+64q) and
// the lane's share of the denominator.
template <class ZT, int NF>
__device__ inline void range_accumulate(uint64_t beg, uint64_t end, const uint32_t* __restrict__ pcol,
                                        const float* __restrict__ R, const ZT* __restrict__ Z, int K,
                                        int W, int zs, float Lh, float Mh, const Lanes& ln, float* pbuf,
                                        uint32_t* jbuf, const int (&fhead)[NF], float (&acc)[NF],
                                        float& dloc) {
    const int lane = threadIdx.x % kWave;
    for (uint64_t base = beg; base < end; base += ln.eb_count) {
        const uint64_t e = base + ln.eb;
        const bool ev = e < end;
        const uint32_t j = ev ? pcol[e] : 0u;
        float p = 0.0f;
        if (ev && ln.hvalid) p = exp_w(leaky(Lh + R[uint64_t(j) * K + ln.hh]) - Mh);
        dloc += p;
        pbuf[ln.hh * ln.eb_count + ln.eb] = p;
        if (ln.hh == 0) jbuf[ln.eb] = j;
        wave_sync();
        const uint64_t rem = end - base;
        const int cnt = rem < uint64_t(ln.eb_count) ? int(rem) : ln.eb_count;
        for (int t = 0; t < cnt; ++t) {
            const ZT* zr = Z + uint64_t(jbuf[t]) * zs;
#pragma unroll
            for (int q = 0; q < NF; ++q) {
                const int f = lane + kWave * q;
                if (f < W) acc[q] += pbuf[fhead[q] * ln.eb_count + t] * load_feat(zr, f);
            }
        }
        wave_sync();
    }
}

template <int NF>
__device__ inline void store_row(float* out32, uint16_t* outbf, uint64_t i, int W, bool hidden,
                                 const float (&acc)[NF], const int (&fhead)[NF], const float* dsh) {
    const int lane = threadIdx.x % kWave;
#pragma unroll
    for (int q = 0; q < NF; ++q) {
        const int f = lane + kWave * q;
        if (f >= W) continue;
        const float d = dsh[fhead[q]];
        float v = acc[q] * (d > 0.0f ? 1.0f / d : 0.0f);
        if (hidden) v = elu(v);
        if (out32) out32[i * W + f] = v;
        if (outbf) outbf[i * W + f] = bf16_hw(v);
    }
}

template <class ZT>
struct KArgs {
    const uint64_t* prow;
    const uint32_t* pcol;
    const uint32_t* perm;
    const float* L;
    const float* R;
    const ZT* Z;
    int K, dim, zs;
    bool hidden;
    float* mx;
    float* den;
    float* out32;
    uint16_t* outbf;
    uint64_t n, e;
};

// One wave per row for sorted positions [k_begin, k_end), heaviest first.
template <class ZT, int NF>
__global__ void __launch_bounds__(kThreads) k_agg_wave(KArgs<ZT> a, uint64_t k_begin, uint64_t k_end) {
    __shared__ float pbuf[kWavesPerBlock][kWave];
    __shared__ uint32_t jbuf[kWavesPerBlock][kWave];
    __shared__ float dsh[kWavesPerBlock][8];
    const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const uint64_t widx = uint64_t(blockIdx.x) * kWavesPerBlock + w;
    if (widx >= k_end - k_begin) return;
    const uint64_t k = k_end - 1 - widx;
    const uint32_t i = a.perm[k];
    const uint64_t beg = a.prow[k], end = a.prow[k + 1];
    if (i >= a.n || beg > end || end > a.e) return;  // schedule invariants
    const int K = a.K, W = a.K * a.dim;
    const Lanes ln = lanes_for(K);
    const float Lh = ln.hvalid ? a.L[uint64_t(i) * K + ln.hh] : 0.0f;
    const float m = range_max(beg, end, a.pcol, a.R, K, ln);
    const float Mh = end > beg ? leaky(Lh + m) : 0.0f;
    if (lane < K) a.mx[uint64_t(i) * K + lane] = Mh;
    int fhead[NF];
    float acc[NF];
#pragma unroll
    for (int q = 0; q < NF; ++q) {
        const int f = lane + kWave * q;
        fhead[q] = f < W ? f / a.dim : 0;
        acc[q] = 0.0f;
    }
    float dloc = 0.0f;
    range_accumulate<ZT, NF>(beg, end, a.pcol, a.R, a.Z, K, W, a.zs, Lh, Mh, ln, pbuf[w], jbuf[w], fhead, acc,
                             dloc);
    for (int off = ln.kp; off < kWave; off <<= 1) dloc += __shfl_xor(dloc, off);
    if (lane < K) {
        a.den[uint64_t(i) * K + lane] = dloc;
        dsh[w][lane] = dloc;
    }
    wave_sync();
    store_row<NF>(a.out32, a.outbf, i, W, a.hidden, acc, fhead, dsh[w]);
}

// One block (4 waves) per row: each wave takes a contiguous quarter of the
// edges; partial maxima, sums and denominators meet in LDS.
template <class ZT, int NF>
__global__ void __launch_bounds__(kThreads) k_agg_block(KArgs<ZT> a, uint64_t k_begin, uint64_t k_end) {
    __shared__ float pbuf[kWavesPerBlock][kWave];
    __shared__ uint32_t jbuf[kWavesPerBlock][kWave];
    __shared__ float msh[kWavesPerBlock][8];
    __shared__ float dsh[kWavesPerBlock][8];
    __shared__ float accsh[kWavesPerBlock][NF * kWave];
    const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const uint64_t k = k_end - 1 - blockIdx.x;
    if (k < k_begin || k >= k_end) return;
    const uint32_t i = a.perm[k];
    const uint64_t beg = a.prow[k], end = a.prow[k + 1], deg = end - beg;
    if (i >= a.n || beg > end || end > a.e) return;  // schedule invariants (uniform per block)
    const uint64_t q0 = beg + deg * w / kWavesPerBlock, q1 = beg + deg * (w + 1) / kWavesPerBlock;
    const int K = a.K, W = a.K * a.dim;
    const Lanes ln = lanes_for(K);
    const float Lh = ln.hvalid ? a.L[uint64_t(i) * K + ln.hh] : 0.0f;
    const float mpart = range_max(q0, q1, a.pcol, a.R, K, ln);
    if (lane < K) msh[w][lane] = mpart;
    __syncthreads();
    float m = -INFINITY;
    if (ln.hvalid)
        for (int q = 0; q < kWavesPerBlock; ++q) m = fmaxf(m, msh[q][ln.hh]);
    const float Mh = deg ? leaky(Lh + m) : 0.0f;
    if (w == 0 && lane < K) a.mx[uint64_t(i) * K + lane] = Mh;
    int fhead[NF];
    float acc[NF];
#pragma unroll
    for (int q = 0; q < NF; ++q) {
        const int f = lane + kWave * q;
        fhead[q] = f < W ? f / a.dim : 0;
        acc[q] = 0.0f;
    }
    float dloc = 0.0f;
    range_accumulate<ZT, NF>(q0, q1, a.pcol, a.R, a.Z, K, W, a.zs, Lh, Mh, ln, pbuf[w], jbuf[w], fhead, acc,
                             dloc);
    for (int off = ln.kp; off < kWave; off <<= 1) dloc += __shfl_xor(dloc, off);
    if (lane < K) dsh[w][lane] = dloc;
#pragma unroll
    for (int q = 0; q < NF; ++q) accsh[w][q * kWave + lane] = acc[q];
    __syncthreads();
    if (w != 0) return;
    float dtot[8];
    for (int h = 0; h < 8; ++h) {
        float s = 0.0f;
        if (h < K)
            for (int q = 0; q < kWavesPerBlock; ++q) s += dsh[q][h];
        dtot[h] = s;
    }
    if (lane < K) a.den[uint64_t(i) * K + lane] = dtot[lane];
    float tot[NF];
#pragma unroll
    for (int q = 0; q < NF; ++q) {
        float s = 0.0f;
        for (int v = 0; v < kWavesPerBlock; ++v) s += accsh[v][q * kWave + lane];
        tot[q] = s;
    }
    store_row<NF>(a.out32, a.outbf, i, W, a.hidden, tot, fhead, dtot);
}

template <class ZT, int NF>
hipError_t dispatch(const AggArgs& g, const RowBins& bins, hipStream_t s) {
    KArgs<ZT> a{g.prow, g.pcol, g.perm, g.left, g.right, static_cast<const ZT*>(g.feat), g.heads, g.dim,
                g.fstride, g.hidden, g.mx, g.den, g.out32, g.outbf, g.n, g.e};
    // v1: every row below block_begin takes a wave; the rest a block each.
    const uint64_t wave_rows = bins.block_begin;
    if (wave_rows) {
        const uint64_t blocks = (wave_rows + kWavesPerBlock - 1) / kWavesPerBlock;
        k_agg_wave<ZT, NF><<<dim3(uint32_t(blocks)), kThreads, 0, s>>>(a, 0, wave_rows);
    }
    const uint64_t block_rows = bins.n - bins.block_begin;
    if (block_rows)
        k_agg_block<ZT, NF><<<dim3(uint32_t(block_rows)), kThreads, 0, s>>>(a, bins.block_begin, bins.n);
    return hipGetLastError();
}

template <class ZT>
hipError_t dispatch_nf(const AggArgs& g, const RowBins& bins, hipStream_t s) {
    const int W = g.heads * g.dim;
    if (W <= 64) return dispatch<ZT, 1>(g, bins, s);
    if (W <= 128) return dispatch<ZT, 2>(g, bins, s);
    if (W <= 256) return dispatch<ZT, 4>(g, bins, s);
    return dispatch<ZT, 8>(g, bins, s);
}

}  // namespace

hipError_t launch_aggregate_tf(const AggArgs& a, const RowBins& bins, const SplitTable& split,
                               hipStream_t s) {
    if (a.heads < 1 || a.heads > 8 || a.dim < 1 || a.heads * a.dim > 512) return hipErrorInvalidValue;
    if (aggregate_vec_supported(a)) return launch_aggregate_vec(a, bins, split, s);
    if (aggregate_k1_supported(a)) return launch_aggregate_k1(a, bins, split, s);
    // Generic path: a wave per row below block_begin, a block per row above
    // (split rows included).
    return a.feat_bf16 ? dispatch_nf<uint16_t>(a, bins, s) : dispatch_nf<float>(a, bins, s);
}

}  // namespace gatgpu
