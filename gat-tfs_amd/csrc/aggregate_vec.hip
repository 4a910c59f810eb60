// Vectorised transform-first aggregation for rows of 8 heads whose width is a
// multiple of one 16-byte vector per lane (8 bf16 or 4 FP32 features), i.e.
// 8 x 32 and 8 x 64.  Same mathematics as aggregate.hip
// (baseline_standard.cpp:44-97): p = exp(LeakyReLU(L+R) - M) with M the exact
// row max, den = sum p, out = ELU?(sum p Z / den).
//
// Work items, one wave each, in this order:
//   * chunks of split rows (in-degree >= split_min), C edges each.  A chunk
//     runs the online softmax over its edges as a whole row does and leaves
//     its partial (sum p Z, sum p) with its own max m_c in scratch; the last
//     chunk to arrive (agent-scope release/acquire around a relaxed counter)
//     scales each partial by e^(m_c - M), M the row max, adds them in chunk
//     order, which is deterministic, and finishes the row.
//   * whole rows below split_min, heaviest first.
//
// Lane layout.  A source row is LPR 16-byte vectors.  Lane (slot, sub), with
// slot = lane / LPR and sub = lane % LPR, reads vector sub of every edge whose
// index within the batch is slot (mod EPI); EPI = 64 / LPR edges share one
// load instruction, and a row wider than the wave gives a lane VPL vectors.
// Each vector lies inside one head, so a lane scores its own (edge, head)
// pairs: R[j][h] is one 4-byte load issued beside the lane's Z load (the
// lanes of one edge read one 32-byte R row), and exp is evaluated by each of
// the DIM/VEC lanes of a head.  That costs a few VALU operations per edge and
// removes the score exchange through LDS and its barriers.  Source ids are
// wave-uniform (one row per wave) and arrive with scalar loads, BATCH at a
// time; pcol carries kPcolPad entries past its end for that.
//
// Softmax state per lane and head: the running max m, the denominator and the
// accumulators, rescaled by exp(m_old - m_new) when a batch raises m (the
// running-maximum form of implementation/src/gat_tfs_online.cpp:86-117).  Each
// edge slot keeps its own state and the slots merge at the end of the row.
// Every source row is thus read once, and the final m is max leaky(L + R_j) =
// leaky(L + max R_j) bit for bit (leaky and the addition are monotone).  A
// chunk starts from the exact row max, so its m never moves.
#include "internal.hpp"

namespace gatgpu {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;

template <class ZT, int W_, int K_, int U_ = 0>
struct Cfg {
    static constexpr int W = W_, K = K_;
    static constexpr int VEC = 16 / int(sizeof(ZT));  // features per 16-byte load
    static constexpr int DIM = W / K;
    static constexpr int LPR = W / VEC;               // 16-byte vectors per row
    static constexpr int EPI = LPR >= kWave ? 1 : kWave / LPR;  // edges per load instruction
    static constexpr int VPL = LPR <= kWave ? 1 : LPR / kWave;  // vectors per lane per edge
    static constexpr int U = U_ ? U_ : VPL == 1 ? 8 : 4;  // load instructions per vector per batch
    static constexpr int BATCH = U * EPI;             // edges per batch
    static constexpr int ACC = VPL * VEC;
    static_assert(W % K == 0 && DIM % VEC == 0, "a vector must not straddle two heads");
    static_assert(LPR * EPI == kWave || LPR % kWave == 0, "lanes per row must divide or fill the wave");
    static_assert(2 * BATCH <= int(kPcolPad), "the id prefetch may read 2 BATCH - 1 entries past the row");
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
    const float* ar;  // aR [W] when R is recomputed from the gathered rows
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

// Softmax state of one lane: its VPL heads' running max, denominator, L,
// and the ACC accumulated features.
template <class C>
struct Lane {
    float acc[C::ACC];
    float den[C::VPL];
    float m[C::VPL];
    float L[C::VPL];
    int h[C::VPL];
    float ar[C::VEC];  // aR of the lane's features (R from the gathered row)
    uint32_t smask;    // all ones in the lanes of edge slot 1 (batch, O32)
};

// The weights and sums of a batch whose rows z and scores s are in (the form
// without R from Z; z is 0 and s unused for the edges outside the row, ok
// false): the batch max moves m (the sums rescaled by e^(m_old - m_new)),
// then each edge adds p = e^(s - m) to den and p z to the sums, in edge order.
// Products fuse into FMAs only within a statement, so the operations, and the
// bits, do not depend on the code around the sums (k_agg_vec, k_agg_vec_short).
template <class C>
__device__ inline void batch_sums(const uint4 (&z)[C::U][C::VPL], const float (&s)[C::U][C::VPL],
                                  const bool (&ok)[C::U], Lane<C>& st) {
#pragma clang fp contract(on)
#pragma unroll
    for (int v = 0; v < C::VPL; ++v) {
        float mb = -INFINITY;
#pragma unroll
        for (int u = 0; u < C::U; ++u) {
            const float mx = max_quiet(mb, s[u][v]);
            mb = ok[u] ? mx : mb;
        }
        const float mn = max_quiet(st.m[v], mb);
        const float sc = mn > st.m[v] ? exp_w(st.m[v] - mn) : 1.0f;  // exp(-inf) = 0 on a slot's first edge
        st.m[v] = mn;
        st.den[v] *= sc;
#pragma unroll
        for (int x = 0; x < C::VEC; ++x) st.acc[v * C::VEC + x] *= sc;
    }
#pragma unroll
    for (int u = 0; u < C::U; ++u) {
#pragma unroll
        for (int v = 0; v < C::VPL; ++v) {
            const float p = ok[u] ? exp_w(s[u][v] - st.m[v]) : 0.0f;
            st.den[v] += p;
            float f[C::VEC];
            unpack(z[u][v], f);
#pragma unroll
            for (int x = 0; x < C::VEC; ++x) st.acc[v * C::VEC + x] += p * f[x];
        }
    }
}

// One batch of edges [base, base + BATCH) clipped to end.  RZ (bf16 8 x 32
// or 8 x 64): R of the source is recomputed from the gathered row, R =
// Z_bf16 . aR, as an FMA chain over the lane's 8 features, (s0 + s1) + (s2 +
// s3) over the 4 lanes of a head of 32, and for a head of 64 the two quads'
// sums added -- the summation the projection used to store R -- so no R line
// is fetched.
// Source ids of edges [base, base + BATCH): wave-uniform scalar loads, which
// may run up to 2 BATCH - 1 entries past the last edge (pcol is padded).
template <class C>
__device__ inline void load_ids(const uint32_t* __restrict__ pcol, uint64_t base, uint32_t (&js)[C::BATCH]) {
    const auto* pc = read_only(pcol);
#pragma unroll
    for (int t = 0; t < C::BATCH; ++t) js[t] = pc[base + t];
}

// `left` (>= 1) edges of the row remain from the batch's first.  Edges past
// the end take the source of the batch's last edge: its row is loaded by this
// batch anyway, so the repeated load stays in the caches and no load needs a
// bounds test; their weight is 0 and they leave m alone.
// O32 (RZ, two edge slots, n W sizeof(ZT) <= 2^32, checked at launch): a
// lane's byte offset into Z is j0 RB + ((j1 - j0) RB & smask) + 16 sub for
// the slot-0 / slot-1 sources j0, j1 of a load (RB bytes per row; smask all
// ones in the slot-1 lanes), two VALU operations on scalar operands instead
// of a per-lane select and a 64-bit address.
// FREE (RZ): every edge slot has seen a valid edge before its first past-end
// edge (the row has at least EPI edges, or m starts at a chunk's finite row
// max), so m is finite there: a past-end edge is given the score -inf, which
// leaves m in place (scale e^0 = 1) and weighs 0 -- the values of the tested
// form, without its selects.
template <class C, class ZT, bool RZ, bool O32 = false, bool FREE = false>
__device__ inline void batch(uint32_t left, const uint32_t (&js)[C::BATCH], const float* __restrict__ R,
                             const ZT* __restrict__ Z, int slot, int sub, Lane<C>& st) {
    static_assert(!O32 || (RZ && C::EPI == 2 && C::VPL == 1), "32-bit offsets: the two-slot R-from-Z form");
    static_assert(!FREE || RZ, "unmasked weights: the R-from-Z form");
    uint32_t jc[C::BATCH];
    jc[0] = js[0];
#pragma unroll
    for (int t = 1; t < C::BATCH; ++t) jc[t] = uint32_t(t) < left ? js[t] : jc[t - 1];
    uint4 z[C::U][C::VPL];
    float s[C::U][C::VPL];
    bool ok[C::U];
#pragma unroll
    for (int u = 0; u < C::U; ++u) {
        ok[u] = slot < int(left) - u * C::EPI;
        if constexpr (O32) {
            constexpr uint32_t RB = C::W * sizeof(ZT);
            // scalar products, kept scalar (one v_and and one v_add3 per lane)
            uint32_t j0 = jc[2 * u] * RB;
            asm volatile("" : "+s"(j0));
            const uint32_t dj = (jc[2 * u + 1] - jc[2 * u]) * RB;
            const uint32_t off = j0 + (dj & st.smask) + uint32_t(sub * 16);
            z[u][0] = *reinterpret_cast<const uint4*>(reinterpret_cast<const unsigned char*>(Z) + off);
        } else {
            uint32_t j = jc[u * C::EPI];
#pragma unroll
            for (int q = 1; q < C::EPI; ++q) j = slot == q ? jc[u * C::EPI + q] : j;
            const ZT* row = Z + uint64_t(j) * C::W;
            // R gathered beside the row (one slot, whole rows per edge): edges
            // past the end issue no loads, which measured faster on graphs of
            // many short rows than re-reading the last row.
#pragma unroll
            for (int v = 0; v < C::VPL; ++v) {
                if constexpr (RZ) {
                    z[u][v] = *reinterpret_cast<const uint4*>(row + (sub + kWave * v) * C::VEC);
                } else {
                    z[u][v] = ok[u] ? *reinterpret_cast<const uint4*>(row + (sub + kWave * v) * C::VEC)
                                    : make_uint4(0, 0, 0, 0);
                    s[u][v] = leaky(st.L[v] + (ok[u] ? R[uint64_t(j) * C::K + st.h[v]] : 0.0f));
                }
            }
        }
    }
    if constexpr (RZ) {
        // Score, weigh and accumulate each edge as soon as its row is here
        // (the unpacked row is used twice, so it is not kept for a batch):
        // online per edge, the accumulators rescaled only when some lane of
        // the wave raised its max.
        static_assert(C::VEC == 8 && (C::DIM == 32 || C::DIM == 64) && C::VPL == 1, "R from Z: bf16 8 x 32 or 8 x 64 rows");
#pragma unroll
        for (int u = 0; u < C::U; ++u) {
            float f[C::VEC];
            unpack(z[u][0], f);
            float t = 0.0f;
#pragma unroll
            for (int x = 0; x < C::VEC; ++x) t = __builtin_fmaf(f[x], st.ar[x], t);
            t += quad_xor1(t);
            t += quad_xor2(t);
            if constexpr (C::DIM == 64) {
                // the other quad of the head's 8 lanes (DPP row_half_mirror:
                // lane i of each 8 takes lane 7 - i)
                t += __builtin_bit_cast(float,
                                        __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, t), 0x141, 0xF, 0xF, false));
            }
            const float sc_ = leaky(st.L[0] + t);
            float mn, scale, p;
            if constexpr (FREE) {
                const float sv = ok[u] ? sc_ : -INFINITY;
                mn = max_quiet(st.m[0], sv);
                scale = exp_w(st.m[0] - mn);  // exactly 1 when m stays; 0 on a slot's first edge
                p = exp_w(sv - mn);           // 0 past the end
            } else {
                const float mx = max_quiet(st.m[0], sc_);  // unconditional: no branch around the asm
                mn = ok[u] ? mx : st.m[0];
                scale = mn > st.m[0] ? exp_w(st.m[0] - mn) : 1.0f;  // exp(-inf) = 0 on a slot's first edge
                p = ok[u] ? exp_w(sc_ - mn) : 0.0f;
            }
            if (__any(scale != 1.0f)) {
                st.den[0] *= scale;
#pragma unroll
                for (int x = 0; x < C::VEC; ++x) st.acc[x] *= scale;
            }
            st.m[0] = mn;
            st.den[0] += p;
#pragma unroll
            for (int x = 0; x < C::VEC; ++x) st.acc[x] += p * f[x];
        }
        return;
    }
    batch_sums<C>(z, s, ok, st);
}

// The edge slots' states merged: afterwards every lane holds its heads'
// totals and m is the max over all the edges.
// (Lane pairs 16 and 32 apart exchange through v_permlane16/32_swap, in the
// VALU; max and + of the pair are commutative, so the order does not matter.)
template <int OFF>
__device__ inline float pair_max(float x) {
    if constexpr (OFF == 16) return xor16_max(x);
    else if constexpr (OFF == 32) return xor32_max(x);
    else return fmaxf(x, __shfl_xor(x, OFF));
}
template <int OFF>
__device__ inline float pair_add(float x) {
    if constexpr (OFF == 16) return xor16_add(x);
    else if constexpr (OFF == 32) return xor32_add(x);
    else return x + __shfl_xor(x, OFF);
}
template <class C, int OFF>
__device__ inline void merge_step(Lane<C>& st) {
    if constexpr (OFF < kWave) {
#pragma unroll
        for (int v = 0; v < C::VPL; ++v) {
            const float M = pair_max<OFF>(st.m[v]);
            const float f = st.m[v] == M ? 1.0f : exp_w(st.m[v] - M);
            st.m[v] = M;
            st.den[v] = pair_add<OFF>(st.den[v] * f);
#pragma unroll
            for (int x = 0; x < C::VEC; ++x) st.acc[v * C::VEC + x] = pair_add<OFF>(st.acc[v * C::VEC + x] * f);
        }
        merge_step<C, 2 * OFF>(st);
    }
}
template <class C>
__device__ inline void merge_slots(Lane<C>& st) {
    if constexpr (C::EPI > 1) merge_step<C, C::LPR>(st);
}

template <bool V>
struct Flag {
    static constexpr bool value = V;
};

// Edges [beg, end) of a row or chunk, then the edge slots merged.  EXACT: m
// holds a chunk's exact (finite) row max already.  O32: see batch.
template <class C, class ZT, bool RZ, bool O32 = false, bool EXACT = false, bool MERGE = true>
__device__ inline void aggregate(uint64_t beg, uint64_t end, const uint32_t* __restrict__ pcol,
                                 const float* __restrict__ R, const ZT* __restrict__ Z, int slot, int sub,
                                 Lane<C>& st) {
    uint32_t js[C::BATCH];
    load_ids<C>(pcol, beg, js);
    // 32-bit edge counts (set_graph rejects rows of 2^32 edges or more): the
    // loop's and the batch's tests stay on the scalar unit.
    const uint32_t total = uint32_t(end - beg);
    auto edges = [&](auto free) {
        for (uint32_t done = 0; done < total; done += C::BATCH) {
            // The next batch's ids are requested before this batch's rows arrive.
            uint32_t jn[C::BATCH];
            load_ids<C>(pcol, beg + done + C::BATCH, jn);
            batch<C, ZT, RZ, O32, decltype(free)::value>(total - done, js, R, Z, slot, sub, st);
#pragma unroll
            for (int t = 0; t < C::BATCH; ++t) js[t] = jn[t];
        }
    };
    // Unmasked weights once every slot starts with a valid edge (rows of at
    // least EPI edges) or from a finite max (chunks).
    if (RZ && (EXACT || total >= uint32_t(C::EPI))) edges(Flag<RZ>{});
    else edges(Flag<false>{});
    if constexpr (MERGE) merge_slots<C>(st);
}

// Normalise, ELU and store one output row from the slot-0 lanes; the first
// lane of each head also stores M and den.
template <class C>
__device__ inline void finish_row(uint32_t i, const float (&acc)[C::ACC], const float (&den)[C::VPL],
                                  const float (&M)[C::VPL], const int (&h)[C::VPL], int slot, int sub,
                                  bool hidden, float* mx, float* dn, float* out32,
                                  uint16_t* outbf) {
    if (slot != 0) return;
#pragma unroll
    for (int v = 0; v < C::VPL; ++v) {
        const int f0 = (sub + kWave * v) * C::VEC;
        if (f0 % C::DIM == 0) {
            mx[uint64_t(i) * C::K + h[v]] = M[v];
            dn[uint64_t(i) * C::K + h[v]] = den[v];
        }
        const float scale = den[v] > 0.0f ? 1.0f / den[v] : 0.0f;
        float o[C::VEC];
#pragma unroll
        for (int x = 0; x < C::VEC; ++x) o[x] = acc[v * C::VEC + x] * scale;
        if (hidden && out32) {
#pragma unroll
            for (int x = 0; x < C::VEC; ++x) o[x] = elu(o[x]);
        } else if (hidden) {  // stored as bf16 only
#pragma unroll
            for (int x = 0; x < C::VEC; ++x) o[x] = elu_bf16(o[x]);
        }
        const uint64_t off = uint64_t(i) * C::W + f0;
        if (outbf) {
            uint32_t w[C::VEC / 2];
#pragma unroll
            for (int x = 0; x < C::VEC / 2; ++x)
                w[x] = bf16x2(o[2 * x], o[2 * x + 1]);
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
    // kUnroll rounds of kWave / K edges in flight per lane (a 256-edge chunk
    // of 8 heads in one round trip for its ids and one for its R values):
    // the loads of a round do not wait for the previous round's.  Edges past
    // the end repeat the chunk's last edge, which leaves the max unchanged.
    constexpr int kStep = kWave / K, kUnroll = 32;
    float m = -INFINITY;
    for (uint64_t e0 = beg + lane / K; e0 < end; e0 += uint64_t(kUnroll) * kStep) {
        uint32_t j[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t e = e0 + uint64_t(u) * kStep;
            j[u] = pcol[e < end ? e : end - 1];
        }
        float r[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) r[u] = R[uint64_t(j[u]) * K + h];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) m = fmaxf(m, r[u]);
    }
    for (int off = K; off < kWave; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
    if (lane < K) sp.mchunk[c * 8 + lane] = m;
}

// Lane state at the start of a row or chunk: zero sums, the lane's head and aR.
template <class C, class ZT, bool RZ>
__device__ inline void init_lane(const VArgs<ZT>& a, int sub, Lane<C>& st) {
#pragma unroll
    for (int x = 0; x < C::ACC; ++x) st.acc[x] = 0.0f;
#pragma unroll
    for (int v = 0; v < C::VPL; ++v) {
        st.h[v] = ((sub + kWave * v) * C::VEC) / C::DIM;
        st.den[v] = 0.0f;
    }
#pragma unroll
    for (int x = 0; x < C::VEC; ++x) st.ar[x] = RZ ? a.ar[sub * C::VEC + x] : 0.0f;
    // A mask in a register, not a select on the slot: dj & smask is one AND.
    uint32_t sm = sub == int(threadIdx.x % kWave) ? 0u : ~0u;  // sub = lane in slot 0
    asm volatile("" : "+v"(sm));
    st.smask = sm;
}

// Floats per chunk partial: W sums, then 8 denominators and 8 maxima.
template <class C>
constexpr int part_floats() {
    return C::W + 16;
}

// Chunk c of a split row: its edges with the online softmax (as a whole row),
// the partial sums, denominators and the chunk's row max m_c to scratch; the
// last chunk of the row to arrive takes M = max_c m_c (the exact row max, as
// each m_c is exact over its chunk) and adds the partials in chunk order,
// each scaled by e^(m_c - M) -- the merge of tfs_online_fused's running
// maximum (implementation/src/gat_tfs_online.cpp:86-117) over chunks.
template <class C, class ZT, bool RZ, bool O32>
__device__ inline void run_chunk(const VArgs<ZT>& a, uint64_t c, int lane, int slot, int sub) {
    Lane<C> st;
    init_lane<C, ZT, RZ>(a, sub, st);
    const uint32_t k = a.sp.chunk_k[c], first = a.sp.chunk_first[c];
    const uint64_t rbeg = a.prow[k], rend = a.prow[k + 1];
    const uint32_t i = a.perm[k];
    if (i >= a.n || rbeg > rend || rend > a.e) return;
    const uint32_t nch = uint32_t((rend - rbeg + a.sp.chunk_edges - 1) / a.sp.chunk_edges);
    const uint64_t beg = rbeg + uint64_t(c - first) * a.sp.chunk_edges;
    const uint64_t end = beg + a.sp.chunk_edges < rend ? beg + a.sp.chunk_edges : rend;
#pragma unroll
    for (int v = 0; v < C::VPL; ++v) {
        st.L[v] = a.L[uint64_t(i) * C::K + st.h[v]];
        st.m[v] = -INFINITY;
    }
    aggregate<C, ZT, RZ, O32>(beg, end, a.pcol, a.R, a.Z, slot, sub, st);
    constexpr int PF = part_floats<C>();
    float* part = a.sp.part + c * PF;
    if (slot == 0) {
#pragma unroll
        for (int v = 0; v < C::VPL; ++v) {
            const int f0 = (sub + kWave * v) * C::VEC;
#pragma unroll
            for (int x = 0; x < C::VEC; x += 4)
                *reinterpret_cast<float4*>(part + f0 + x) =
                    make_float4(st.acc[v * C::VEC + x], st.acc[v * C::VEC + x + 1], st.acc[v * C::VEC + x + 2],
                                st.acc[v * C::VEC + x + 3]);
            if (f0 % C::DIM == 0) {
                part[C::W + st.h[v]] = st.den[v];
                part[C::W + 8 + st.h[v]] = st.m[v];
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    uint32_t old = 0;
    if (lane == 0)
        old = __hip_atomic_fetch_add(a.sp.counter + first, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __shfl(old, 0);
    if (old + 1 != nch) return;  // not the last chunk of this row
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // Last arrival: the row max over the chunks, then the partials of every
    // chunk in chunk order, scaled to it.
    float M[C::VPL];
#pragma unroll
    for (int v = 0; v < C::VPL; ++v) {
        M[v] = -INFINITY;
        for (uint32_t q = 0; q < nch; ++q) M[v] = fmaxf(M[v], a.sp.part[uint64_t(first + q) * PF + C::W + 8 + st.h[v]]);
    }
    float tot[C::ACC];
    float dtot[C::VPL];
#pragma unroll
    for (int x = 0; x < C::ACC; ++x) tot[x] = 0.0f;
#pragma unroll
    for (int v = 0; v < C::VPL; ++v) dtot[v] = 0.0f;
    for (uint32_t q = 0; q < nch; ++q) {
        const float* pq = a.sp.part + uint64_t(first + q) * PF;
#pragma unroll
        for (int v = 0; v < C::VPL; ++v) {
            const float mq = pq[C::W + 8 + st.h[v]];
            const float f = mq == M[v] ? 1.0f : exp_w(mq - M[v]);  // a chunk of only -inf scores: 0
            const int f0 = (sub + kWave * v) * C::VEC;
#pragma unroll
            for (int x = 0; x < C::VEC; x += 4) {
                const float4 t = *reinterpret_cast<const float4*>(pq + f0 + x);
                tot[v * C::VEC + x] += t.x * f;
                tot[v * C::VEC + x + 1] += t.y * f;
                tot[v * C::VEC + x + 2] += t.z * f;
                tot[v * C::VEC + x + 3] += t.w * f;
            }
            dtot[v] += pq[C::W + st.h[v]] * f;
        }
    }
    if (lane == 0) a.sp.counter[first] = 0;  // ready for the next launch
    finish_row<C>(i, tot, dtot, M, st.h, slot, sub, a.hidden, a.mx, a.den, a.out32, a.outbf);
}

// short_rows: the positions [0, short_rows) are k_agg_vec_short's.
template <class C, class ZT, bool RZ, bool O32>
__global__ void __launch_bounds__(kThreads) k_agg_vec(VArgs<ZT> a, uint64_t short_rows) {
    // The wave index is made wave-uniform so that row bounds and source ids
    // come in through scalar loads.
    const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = threadIdx.x % kWave;
    const int slot = C::EPI > 1 ? lane / C::LPR : 0;
    const int sub = C::EPI > 1 ? lane % C::LPR : lane;
    const uint64_t item = uint64_t(blockIdx.x) * kWavesPerBlock + w;
    if (item < a.sp.chunks) {
        run_chunk<C, ZT, RZ, O32>(a, item, lane, slot, sub);
        return;
    }
    // ---------------- whole row, heaviest first
    const uint64_t widx = item - a.sp.chunks;
    if (widx >= a.rows - short_rows) return;
    const uint64_t k = a.rows - 1 - widx;
    const uint32_t i = a.perm[k];
    const uint64_t beg = a.prow[k], end = a.prow[k + 1];
    if (i >= a.n || beg > end || end > a.e) return;
    Lane<C> st;
    init_lane<C, ZT, RZ>(a, sub, st);
#pragma unroll
    for (int v = 0; v < C::VPL; ++v) {
        st.L[v] = a.L[uint64_t(i) * C::K + st.h[v]];
        st.m[v] = -INFINITY;
    }
    aggregate<C, ZT, RZ, O32>(beg, end, a.pcol, a.R, a.Z, slot, sub, st);
    // Empty row: max 0, denominator 0, output 0 (baseline/src/ref_fp32.cpp:11).
    if (end == beg)
#pragma unroll
        for (int v = 0; v < C::VPL; ++v) st.m[v] = 0.0f;
    finish_row<C>(i, st.acc, st.den, st.m, st.h, slot, sub, a.hidden, a.mx, a.den, a.out32, a.outbf);
}

// Rows of at most kShortDeg edges, the sorted positions [0, a.short_rows), for
// bf16 rows with R in its own array: four consecutive positions per wave.  One
// round trip brings the four rows' bounds, one their ids and L, and one every
// edge's row and R, where a wave per row waits for those three round trips
// for each row (a 2^22-node R-MAT graph has 3.0M such rows, 4.6 % of its
// edges, which took 1.8 ms of its 8 x 64 layer that way).  Every load is
// issued, so that they leave together: edges past a row's end read its last
// edge again (an empty row its first id slot: padding or the next row's first
// id), and their rows and R are replaced by 0 before the sums, which so take
// the values and the operations of batch() on that row (U = 4 where the
// one-row-per-wave kernel has 8: the loads it skips add +0, which leaves its
// sums, never -0, unchanged).
template <class C>
__global__ void __launch_bounds__(kThreads) k_agg_vec_short(VArgs<uint16_t> a, uint64_t short_rows) {
    static_assert(C::VPL == 1 && C::BATCH >= int(kShortDeg), "one vector per lane and edge, one batch per row");
    constexpr int RW = 4;  // rows per wave
    constexpr uint32_t kNone = 0xffffffffu;
    const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = threadIdx.x % kWave;
    const int slot = C::EPI > 1 ? lane / C::LPR : 0;
    const int sub = C::EPI > 1 ? lane % C::LPR : lane;
    const uint64_t k0 = (uint64_t(blockIdx.x) * kWavesPerBlock + w) * RW;
    if (k0 >= short_rows) return;
    const auto* perm = read_only(a.perm);
    const auto* prow = read_only(a.prow);
    uint32_t ri[RW], cnt[RW];
    uint64_t rb[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const bool in = k0 + r < short_rows;
        const uint64_t k = in ? k0 + r : k0;
        const uint32_t i = perm[k];
        const uint64_t b = prow[k], e = prow[k + 1];
        // (the launch hands over rows of at most kShortDeg edges only)
        const bool good = in && i < a.n && b <= e && e <= a.e && e - b <= uint64_t(kShortDeg);
        ri[r] = good ? i : kNone;
        rb[r] = good ? b : 0;  // (a row not stored reads ids from pcol[0]: valid sources)
        cnt[r] = good ? uint32_t(e - b) : 0u;
    }
    Lane<C> st[RW];
    uint4 z[RW][C::U];
    float rv[RW][C::U];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        init_lane<C, uint16_t, false>(a, sub, st[r]);
        st[r].L[0] = a.L[uint64_t(ri[r] == kNone ? 0u : ri[r]) * C::K + st[r].h[0]];
        st[r].m[0] = -INFINITY;
        uint32_t js[C::BATCH], jc[C::BATCH];
        load_ids<C>(a.pcol, rb[r], js);
        jc[0] = js[0];
#pragma unroll
        for (int t = 1; t < C::BATCH; ++t) jc[t] = uint32_t(t) < cnt[r] ? js[t] : jc[t - 1];
#pragma unroll
        for (int u = 0; u < C::U; ++u) {
            uint32_t j = jc[u * C::EPI];
#pragma unroll
            for (int q = 1; q < C::EPI; ++q) j = slot == q ? jc[u * C::EPI + q] : j;
            z[r][u] = *reinterpret_cast<const uint4*>(a.Z + uint64_t(j) * C::W + sub * C::VEC);
            rv[r][u] = a.R[uint64_t(j) * C::K + st[r].h[0]];
        }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        bool ok[C::U];
        uint4 zz[C::U][1];
        float sc[C::U][1];
#pragma unroll
        for (int u = 0; u < C::U; ++u) {
            ok[u] = slot < int(cnt[r]) - u * C::EPI;
            zz[u][0] = ok[u] ? z[r][u] : make_uint4(0, 0, 0, 0);
            sc[u][0] = leaky(st[r].L[0] + (ok[u] ? rv[r][u] : 0.0f));
        }
        if (cnt[r] > 0) batch_sums<C>(zz, sc, ok, st[r]);
        merge_slots<C>(st[r]);
        if (cnt[r] == 0) st[r].m[0] = 0.0f;  // empty row: max 0, denominator 0, output 0
        if (ri[r] != kNone)
            finish_row<C>(ri[r], st[r].acc, st[r].den, st[r].m, st[r].h, slot, sub, a.hidden, a.mx, a.den, a.out32,
                          a.outbf);
    }
}

// Edge loads per lane and batch of the R-from-Z form.
constexpr int kURz = 4;

// ---------------- the next layer's projection fused into the tile epilogue
// (bf16 8 x 32 rows, R from Z; the next layer one head of at most 64 columns
// in rows of 64 bf16 with R as FP32 in the last four bytes).
//
// A block takes a tile of kNextTile consecutive non-split rows (sorted
// positions, heaviest tile first; the row buffers are in sorted order, so the
// position is the row index), wave w rows w, w + 4, ...  Each row is
// aggregated as in k_agg_vec and its output -- normalised, ELU, rounded to
// bf16, the bits the output store would write -- goes to an LDS tile row
// instead of HBM.  The tile is then multiplied by the next layer's W on
// v_mfma_f32_32x32x16_bf16 exactly as k_proj_fast does it (Z^T = W^T H^T,
// the same fragments, k steps in the same order into zeroed accumulators), so
// Z, L and R of the next layer carry the bits of the unfused projection.
// Wave 0 forms Z columns 0..31, wave 1 columns 32..63 (HB = 2), wave HB the
// L/R block, so each 128-byte Z row is written by two waves together, and L
// / R of the tile as whole lines.  The rows' max and den go to LDS too, and
// the wave left idle by the projection writes the tile's 32 x 8 of each as
// whole lines: written per row they were 32-byte pieces, and those partial
// lines, mixed into the gather's reads, cost 0.09 ms more per launch on the
// 64.3M-edge graph.  The row epilogue (normalise, ELU, bf16) is split
// between the two edge slots, 4 features each.  Split rows store their
// output rows as usual; the caller projects them afterwards.
constexpr int kNextTile = 32;
constexpr int kNextRowBytes = 512 + 16;  // padded: the 32 lanes of a B read hit distinct bank groups

// The two edge slots' states merged, the features split between them: on
// exit m and den are the row's in every lane, and lane (slot, sub) holds in
// tot the totals of features 4 slot .. 4 slot + 3 of vector sub.  One
// v_permlane32_swap per feature pair (x of the lower half with x + 4 of the
// upper) and one add, lower half's value first as in merge_step.
template <class C>
__device__ inline void merge_slots_split(Lane<C>& st, float (&tot)[4]) {
    static_assert(C::EPI == 2 && C::VPL == 1 && C::VEC == 8, "two edge slots of 8 features");
    const float M = pair_max<32>(st.m[0]);
    const float f = st.m[0] == M ? 1.0f : exp_w(st.m[0] - M);
    st.m[0] = M;
    st.den[0] = pair_add<32>(st.den[0] * f);
#pragma unroll
    for (int x = 0; x < 4; ++x) {
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(st.acc[x] * f), __float_as_uint(st.acc[x + 4] * f),
                                                        false, false);
        tot[x] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
}

template <class C>
__device__ inline void finish_row_tile(const Lane<C>& st, const float (&tot)[4], int slot, int sub,
                                       float* smd, unsigned char* trow) {
    static_assert(C::VEC == 8 && C::VPL == 1 && C::W == 256, "bf16 8 x 32 rows");
    if (slot == 0 && (sub * C::VEC) % C::DIM == 0) {
        smd[st.h[0]] = st.m[0];
        smd[kNextTile * C::K + st.h[0]] = st.den[0];
    }
    const float scale = st.den[0] > 0.0f ? 1.0f / st.den[0] : 0.0f;
    const uint32_t w0 = bf16x2(elu_bf16(tot[0] * scale), elu_bf16(tot[1] * scale));
    const uint32_t w1 = bf16x2(elu_bf16(tot[2] * scale), elu_bf16(tot[3] * scale));
    *reinterpret_cast<uint2*>(trow + 16 * sub + 8 * slot) = make_uint2(w0, w1);
}

template <class C, int HB, bool O32>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(8)))
k_agg_vec_next(VArgs<uint16_t> a, NextProj f, uint64_t chunk_blocks) {
    static_assert(HB == 1 || HB == 2, "one head of at most 64 columns");
    // Rows of H (bf16), then R of the next layer per row, the rows' max and
    // den (written out by the idle wave as whole lines), and which rows ran.
    constexpr int kMdOff = kNextTile * kNextRowBytes + kNextTile * 4;
    constexpr int kOkOff = kMdOff + 2 * kNextTile * C::K * 4;
    __shared__ __attribute__((aligned(16))) unsigned char tile[kOkOff + kNextTile];
    float* const smd = reinterpret_cast<float*>(tile + kMdOff);
    unsigned char* const tok = tile + kOkOff;
    const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = threadIdx.x % kWave;
    const int slot = lane / C::LPR, sub = lane % C::LPR;
    if (blockIdx.x < chunk_blocks) {
        const uint64_t item = uint64_t(blockIdx.x) * kWavesPerBlock + w;
        if (item < a.sp.chunks) run_chunk<C, uint16_t, true, O32>(a, item, lane, slot, sub);
        return;
    }
    const uint64_t p0 = (f.tiles - 1 - (uint64_t(blockIdx.x) - chunk_blocks)) * kNextTile;
    const int cnt = a.rows - p0 < uint64_t(kNextTile) ? int(a.rows - p0) : kNextTile;
#pragma unroll 1
    for (int r = w; r < kNextTile; r += kWavesPerBlock) {
        unsigned char* trow = tile + r * kNextRowBytes;
        bool stored = false;
        if (r < cnt) {
            const uint64_t k = p0 + r;
            const uint64_t beg = a.prow[k], end = a.prow[k + 1];
            if (beg <= end && end <= a.e) {
                Lane<C> st;
                init_lane<C, uint16_t, true>(a, sub, st);
                st.L[0] = a.L[k * C::K + st.h[0]];
                st.m[0] = -INFINITY;
                aggregate<C, uint16_t, true, O32, false, false>(beg, end, a.pcol, a.R, a.Z, slot, sub, st);
                float tot[4];
                merge_slots_split<C>(st, tot);
                if (end == beg) st.m[0] = 0.0f;  // empty row: max 0, den 0, output 0
                finish_row_tile<C>(st, tot, slot, sub, smd + r * C::K, trow);
                stored = true;
            }
        }
        if (lane == 0) tok[r] = stored;
        if (!stored) *reinterpret_cast<uint2*>(trow + 16 * sub + 8 * slot) = make_uint2(0, 0);
    }
    __syncthreads();
    // ---- the tile's Z^T = W^T H^T: lane (half, col) supplies H[col][16 ks + 8 half .. + 7].
    // Wave b < HB forms Z columns 32 b .. 32 b + 31, wave HB the L/R block
    // (head 0: L hi, R hi, L lo, R lo in registers 0, 4, 8, 12 of the lanes of
    // half 0), whose R goes to LDS for the row tails.
    typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
    typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
    const int half = lane / 32, col = lane % 32;
    const uint64_t k = p0 + col;
    const bool ok = col < cnt;
    float* const rsh = reinterpret_cast<float*>(tile + kNextTile * kNextRowBytes);
    uint32_t zp[8] = {};
    if (w == kWavesPerBlock - 1) {
        // The tile's max and den (sorted rows p0 .. p0 + 31, 8 heads): 1 KB
        // each, lane l rows l / 2, whole lines instead of 32-byte pieces.
        static_assert(HB + 1 < kWavesPerBlock && C::K == 8 && kNextTile * C::K == 4 * kWave, "layout");
        const int r = lane / 2;
        if (r < cnt && tok[r]) {
            const float4* s = reinterpret_cast<const float4*>(smd);
            reinterpret_cast<float4*>(a.mx + p0 * C::K)[lane] = s[lane];
            reinterpret_cast<float4*>(a.den + p0 * C::K)[lane] = s[kWave + lane];
        }
    }
    if (w <= HB) {
        const unsigned char* bsrc = tile + col * kNextRowBytes + 16 * half;
        const uint4* wsrc = f.wpk + size_t(w) * kWave + lane;
        f32x16 acc;
#pragma unroll
        for (int x = 0; x < 16; ++x) acc[x] = 0.0f;
        // Four k steps' fragments requested at a time (L2-resident W, LDS H):
        // the tile loop's registers, not more, are what the phase may use.
#pragma unroll
        for (int k4 = 0; k4 < 16; k4 += 4) {
            uint4 av[4], bv[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                av[q] = wsrc[size_t(k4 + q) * f.nmb * kWave];
                bv[q] = *reinterpret_cast<const uint4*>(bsrc + 32 * (k4 + q));
            }
#pragma unroll
            for (int q = 0; q < 4; ++q)
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av[q]),
                                                              __builtin_bit_cast(bf16x8, bv[q]), acc, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (w == HB) {
            const float lv = acc[0] + acc[8], rv = acc[4] + acc[12];
            if (half == 0) {
                rsh[col] = rv;
                if (ok) {
                    f.left[k] = lv;
                    f.right[k] = rv;
                }
            }
        } else {
#pragma unroll
            for (int x = 0; x < 8; ++x) zp[x] = bf16x2(acc[2 * x], acc[2 * x + 1]);
        }
    }
    __syncthreads();
    if (!ok || w > 1) return;
    // Row col: wave 0 stores bytes 0..63 (columns 0..31), wave 1 bytes 64..127
    // (columns 32..61 and R in the last four bytes).
    uint16_t* zr = f.z + k * 64 + 32 * w + 16 * half;
    uint4 v0 = make_uint4(zp[0], zp[1], zp[2], zp[3]), v1 = make_uint4(zp[4], zp[5], zp[6], zp[7]);
    if (w == 1) {
        if (HB == 1) v0 = v1 = make_uint4(0, 0, 0, 0);  // no columns past 31
        if (half == 1) v1.w = __builtin_bit_cast(uint32_t, rsh[col]);
    }
    *reinterpret_cast<uint4*>(zr) = v0;
    *reinterpret_cast<uint4*>(zr + 8) = v1;
}

// Byte offsets of every Z row fit 32 bits (the O32 form of batch).
template <class C, class ZT>
bool offsets32(uint64_t n) {
    return n <= (uint64_t(1) << 32) / (uint64_t(C::W) * sizeof(ZT));
}

// Split-row chunks and rows, one wave each, then (bf16 rows with R in its own
// array) the rows of at most kShortDeg edges four to a wave in a launch of
// their own.
template <class C, class ZT>
hipError_t run(const AggArgs& g, const RowBins& bins, const SplitTable& t, hipStream_t s) {
    VArgs<ZT> a{g.prow, g.pcol, g.perm, g.left, g.right, static_cast<const ZT*>(g.feat), g.hidden, g.mx, g.den,
                g.out32, g.outbf, g.n, g.e, bins.split_begin,
                SplitArgs{t.chunks, t.chunk_k, t.chunk_first, t.chunk_edges, t.mchunk, t.part, t.counter}, g.ar};
    // (With R from Z the rows of 8 x 64 layers still take the short launch,
    // which gathers R: the projection stored R = Z_bf16 . aR in the summation
    // order the main kernel recomputes it in, so both see the same scores.)
    uint64_t short_rows = 0;
    if constexpr (sizeof(ZT) == 2) {
        if (!g.r_from_z || C::W == 512) short_rows = std::min(bins.short_end, bins.split_begin);
    }
    const uint64_t items = t.chunks + bins.split_begin - short_rows;
    if constexpr (sizeof(ZT) == 2) {
        if (short_rows) {
            using CS = Cfg<uint16_t, C::W, C::K, 4>;
            const uint64_t waves = (short_rows + 3) / 4;
            k_agg_vec_short<CS>
                <<<dim3(uint32_t((waves + kWavesPerBlock - 1) / kWavesPerBlock)), kThreads, 0, s>>>(a, short_rows);
            if (hipError_t e = hipGetLastError(); e != hipSuccess || !items) return e;
        }
    }
    if (!items) return hipSuccess;
    const dim3 grid(uint32_t((items + kWavesPerBlock - 1) / kWavesPerBlock));
    if constexpr (sizeof(ZT) == 2 && C::W == 256) {
        if (g.r_from_z) {
            if (!g.ar) return hipErrorInvalidValue;
            using CR = Cfg<ZT, C::W, C::K, kURz>;
            if (offsets32<CR, ZT>(g.n)) k_agg_vec<CR, ZT, true, true><<<grid, kThreads, 0, s>>>(a, 0);
            else k_agg_vec<CR, ZT, true, false><<<grid, kThreads, 0, s>>>(a, 0);
            return hipGetLastError();
        }
    }
    if constexpr (sizeof(ZT) == 2 && C::W == 512) {
        if (g.r_from_z) {  // one edge slot: whole 1 KB rows, R from each
            if (!g.ar) return hipErrorInvalidValue;
            k_agg_vec<C, ZT, true, false><<<grid, kThreads, 0, s>>>(a, short_rows);
            return hipGetLastError();
        }
    }
    k_agg_vec<C, ZT, false, false><<<grid, kThreads, 0, s>>>(a, short_rows);
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

bool aggregate_vec_next_supported(const AggArgs& g, const NextProj& f) {
    return aggregate_vec_supported(g) && g.feat_bf16 && g.heads * g.dim == 256 && g.r_from_z && g.ar && g.hidden &&
           g.outbf && !g.out32 && (f.head_blocks == 1 || f.head_blocks == 2) && f.nmb > f.head_blocks && f.wpk &&
           f.z && f.left && f.right;
}

hipError_t launch_aggregate_vec_next(const AggArgs& g, const RowBins& bins, const SplitTable& t, NextProj f,
                                     hipStream_t s) {
    if (!aggregate_vec_next_supported(g, f)) return hipErrorInvalidValue;
    using C = Cfg<uint16_t, 256, 8, kURz>;
    VArgs<uint16_t> a{g.prow, g.pcol, g.perm, g.left, g.right, static_cast<const uint16_t*>(g.feat), g.hidden,
                      g.mx, g.den, g.out32, g.outbf, g.n, g.e, bins.split_begin,
                      SplitArgs{t.chunks, t.chunk_k, t.chunk_first, t.chunk_edges, t.mchunk, t.part, t.counter},
                      g.ar};
    f.tiles = (bins.split_begin + kNextTile - 1) / kNextTile;
    const uint64_t chunk_blocks = (t.chunks + kWavesPerBlock - 1) / kWavesPerBlock;
    const uint64_t blocks = chunk_blocks + f.tiles;
    if (!blocks) return hipSuccess;
    if (blocks > 0x7fffffffu) return hipErrorInvalidValue;
    const dim3 grid = dim3(uint32_t(blocks));
    const bool o32 = offsets32<C, uint16_t>(g.n);
    if (f.head_blocks == 2) {
        if (o32) k_agg_vec_next<C, 2, true><<<grid, kThreads, 0, s>>>(a, f, chunk_blocks);
        else k_agg_vec_next<C, 2, false><<<grid, kThreads, 0, s>>>(a, f, chunk_blocks);
    } else {
        if (o32) k_agg_vec_next<C, 1, true><<<grid, kThreads, 0, s>>>(a, f, chunk_blocks);
        else k_agg_vec_next<C, 1, false><<<grid, kThreads, 0, s>>>(a, f, chunk_blocks);
    }
    return hipGetLastError();
}

hipError_t launch_aggregate_vec(const AggArgs& g, const RowBins& bins, const SplitTable& t, hipStream_t s) {
    const int W = g.heads * g.dim;
    if (g.heads != 8) return hipErrorInvalidValue;
    if (g.feat_bf16) {
        if (W == 256) return run<Cfg<uint16_t, 256, 8>, uint16_t>(g, bins, t, s);
        if (W == 512) return run<Cfg<uint16_t, 512, 8>, uint16_t>(g, bins, t, s);
    } else {
        if (W == 256) return run<Cfg<float, 256, 8>, float>(g, bins, t, s);
        if (W == 512) return run<Cfg<float, 512, 8>, float>(g, bins, t, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace gatgpu
