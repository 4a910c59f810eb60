// Aggregate-first layer in its sum form, for D_in <= 112 inputs and 8 heads of
// 32: first U_ih = sum_j p_ijh X_j over the row's edges, then the projection
// U_ih W_h / den_ih.  This is the order of tfs_online_fused
// (implementation/src/gat_tfs_online.cpp:200-283), where a row tile's U panel
// is multiplied by W_h once its rows are summed.
//
//   out[i, h] = ELU?( (sum_j p_ijh X_j) W_h / den_ih ),
//   p_ijh = exp(LeakyReLU(L_ih + R_jh) - M_ih),  M the row max
//   (kept as a running max with rescaling; the final M is exact).
//
// Why: the gathered row is the bf16 input row with the source's R values in
// its tail, 256 bytes, where transform-first gathers the 512-byte Z row of
// 8 x 32 bf16 features.  A 100 -> 8 x 32 layer so moves about half the bytes.
//
// Gather table XR [n][128] bf16 (256-byte rows, 64 words of 4 bytes): X_j at
// [0, D_in), zeros up to 112, R_jh as FP32 in word 56 + h.
//
// The per-edge sums run on the matrix cores.  Per batch of 16 edges,
// v_mfma_f32_16x16x16_bf16 forms D[row][feature] += P[row][edge] X[edge][feature]
// with the edge as the contraction index (16x16x32 with 32-edge batches is the
// other instance of the same code: EPL edges per lane).  Lane l = 16 g + n
// (k group g takes edges 4g .. 4g + 3 of the batch) loads word 16 sb + n of
// each of its 4 edges' rows, sb = 0..3 (features 2(16 sb + n) and
// 2(16 sb + n) + 1): the low halves of those words are the B operand of an
// even-feature block, the high halves that of an odd-feature block.  Word
// 56 + h of a row is R_jh; a DPP rotation by 8 hands it from lane 8 + h of
// super-block 3 to lane h, which scores head h for its edges, keeps the
// running max m_h and the
// denominator, and splits p into hi + lo bf16 (p enters to about 2^-17): A
// row h holds the hi parts and row 8 + h the lo parts, so one MFMA per
// feature block takes both and D rows 8..15 sum the lo parts; the two sums
// of a head fold at the row end (fold_pair).  The weights are taken
// against a reference max m_h: the first batch's max, moved (with the sums
// rescaled by exp(m_old - m_new), the running-maximum form of
// gat_tfs_online.cpp:86-117) only when a batch's max exceeds it by more than
// kLazyMax, so p <= e^8 and most batches rescale nothing.  The exact row max
// M_h = leaky(L_h + max_j R_jh) is kept beside it (bit for bit, as leaky and
// the addition are monotone); the stored denominator is sum_j e^(s_j - M_h) =
// den e^(m_h - M_h), and U / den is the same quotient either way.  Lane (g, n),
// register r of block (sb, par) holds the hi sum (g = 0, 1) or the lo sum
// (g = 2, 3) of head 4 (g % 2) + r, feature 2(16 sb + n) + par.
//
// Blocks of 8 waves take tiles of consecutive degree-sorted rows (16 or 32,
// see k_afs_tiles).  A row's sums U_h go to LDS in the B-operand layout of
// v_mfma_f32_32x32x16_bf16, as a hi + lo pair of bf16 (U = hi + lo to about
// 2^-17 relative) for FP32 outputs and as one bf16 for bf16-stored hidden
// outputs, with den_h beside them.  After a barrier, wave h multiplies the
// tile's U_h by W_h (A fragments packed as for the projection, read from L2;
// two MFMA chains) and scales each output row by 1 / den_h: (U_h W_h) / den_h,
// the same quotient as (U_h / den_h) W_h, with one scaling per output row and
// head instead of one per summed feature.  Split rows: the first blocks of the
// same launch take one chunk per wave and sum its edges into scratch against
// maxima of its own (the lazy reference max and the exact max, as a tile row
// keeps them); the row's last chunk to arrive scales the chunks to a common
// reference, adds them in chunk order and projects the row on the VALU with
// the FP32 W.  The tile blocks take tiles from a counter, so those that start
// after the chunk blocks take fewer.
#include <type_traits>

#include "internal.hpp"

namespace gatgpu {
namespace {

typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;   // 8 = heads
constexpr int kTile = 2 * kWaves;          // rows per block tile (hi + lo S)
constexpr int kTileBf16 = 32;              // rows per block tile with one bf16 U
constexpr int kMaxKS = 8;                  // k steps of 16 features: D_in <= 128
constexpr int kRowWords = kXRStride / 2;   // 64 words of 4 bytes per XR row
constexpr int kEPL = 4;                    // edges per lane and batch (batches of 4 kEPL edges)
constexpr int kSB = 4;                     // super-blocks of 16 words per row
constexpr int kBlk = kTile * 32 + 32;      // bytes per (head, k step, hi|lo) block of U, padded
// Heads 4..7 sit this many bytes further on: with blocks 8 words apart modulo
// the banks, the 32 lanes that write U (k group g, lanes n) land on 32
// distinct banks: n % 8, + 8 for n / 8, + 16 for g.
constexpr int kHalfOff = 64;
constexpr int kSBytes = 8 * kMaxKS * 2 * kBlk + kHalfOff;
constexpr int kTRowBytes = 2 * 2 * kTile * 4;             // the tile's node ids (up to 2 x 32)
constexpr int kTDenBytes = 2 * 8 * (2 * kTile + 1) * 4;   // their denominators (2 x 8 heads x 33)
constexpr int kTQBytes = 4 * 4;                                // ring of the block's next tile indices
constexpr int kTMdBytes = 2 * 8 * 2 * kTile * 4;               // the tile rows' max and den stages (up to 32 rows)
constexpr int kLdsBytes = kSBytes + kTRowBytes + kTDenBytes + kTQBytes + kTMdBytes;  // S, ids, dens, tiles, stages
constexpr uint32_t kNoRow = 0xffffffffu;
constexpr int kPart = 8 * 128 + 24;        // floats per chunk partial: U_h rows of 128, den, m, mx
constexpr int kDenOff = 8 * 128;           // den_h against the chunk's reference max m_h
constexpr int kMOff = kDenOff + 8;         // the reference max m_h
constexpr int kMxOff = kDenOff + 16;       // the chunk's exact max of the scores
constexpr int kMergeFloats = 8 * kRowWords * 2;  // LDS floats of a wave that merges a split row

static_assert(32 <= int(kPcolPad), "an id request may read 31 entries past the row");
static_assert(kRowWords == 16 * kSB && kXRFeat == 112, "XR row: 4 super-blocks, R in words 56..63 (D <= 112)");

__device__ inline float lane_f(float x, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}

// Running sums of one row or chunk.  d[2 sb + par] are the D accumulators of
// the feature blocks; m, den and L live in the head lanes (n < 8, head n;
// den of the lane's own k group until combined).
// m is the reference max the weights p = e^(s - m) are taken against; mx is
// the running row max (exact).
struct Sums {
    f32x4 d[2 * kSB];
    float m, mx, den, L;
};

// A batch moves the reference max only when its own max exceeds it by more
// than this (so p <= e^8, far inside FP32 and bf16 range): most batches then
// need no rescaling of the sums.
constexpr float kLazyMax = 8.0f;

// Batches of 4 EPL edges: lane (g, n) takes edges EPL g .. EPL g + EPL - 1
// of a batch, the k group of v_mfma_f32_16x16x32_bf16 (EPL 8) or of
// v_mfma_f32_16x16x16_bf16 (EPL 4; smaller batches waste fewer slots on short
// rows).  The D layout is the same for both.
typedef short s16x4 __attribute__((ext_vector_type(4)));
template <int EPL>
struct Mfma;
template <>
struct Mfma<8> {
    static __device__ inline f32x4 run(const uint32_t (&a)[4], const uint32_t (&b)[4], f32x4 d) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, make_uint4(a[0], a[1], a[2], a[3])),
                                                       __builtin_bit_cast(bf16x8, make_uint4(b[0], b[1], b[2], b[3])),
                                                       d, 0, 0, 0);
    }
};
template <>
struct Mfma<4> {
    static __device__ inline f32x4 run(const uint32_t (&a)[2], const uint32_t (&b)[2], f32x4 d) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, make_uint2(a[0], a[1])),
                                                          __builtin_bit_cast(s16x4, make_uint2(b[0], b[1])), d, 0,
                                                          0, 0);
    }
};

// Edges [beg, end).  ids: lane id0 + t holds pcol[beg + t], t < 32 (requested
// by the caller ahead of time); each batch requests the next batch's ids the
// same way (pcol is padded past e).  EXACT: s.m holds the exact row max
// already (a chunk) and never moves.
// RSEP: the rows hold 128 input features and R comes from its own array
// ([n][8], loaded by the head lanes beside the row words).
// Source nodes of lane l's EPL edges of a batch with `left` (>= 1) edges to
// go, from ids (lane i0 + t holds the batch's edge t); edges past the end
// re-read the batch's last row (weight 0).  Byte indices of ds_bpermute: a
// lane constant, one min and one add per edge.
template <int EPL>
__device__ inline void batch_sources(uint32_t idv, int i0, uint32_t left, int l, uint32_t (&js)[EPL]) {
    constexpr int B = 4 * EPL;
    const int cnt = left < uint32_t(B) ? int(left) : B;
    const int g = l / 16;
#pragma unroll
    for (int t = 0; t < EPL; ++t)
        js[t] = uint32_t(__builtin_amdgcn_ds_bpermute(min(4 * (EPL * g + t), 4 * (cnt - 1)) + 4 * i0, int(idv)));
}

// The row words of lane l for the batch's sources jl (word 16 sb + n of each
// edge's row), and R of head n beside them when R has its own array.
// 32-bit byte offsets (n * 256 < 2^32 is checked at launch).
template <bool RSEP, int EPL>
__device__ inline void load_batch(const uint32_t* __restrict__ xr, const float* __restrict__ R,
                                  const uint32_t (&jl)[EPL], int l, uint32_t (&raw)[kSB][EPL], float (&rsep)[EPL]) {
    const int n = l % 16;
    const unsigned char* xb = reinterpret_cast<const unsigned char*>(xr);
    uint32_t off[EPL];
#pragma unroll
    for (int t = 0; t < EPL; ++t) off[t] = jl[t] * uint32_t(4 * kRowWords) + 4u * uint32_t(n);
    // Super-block 3 (the R words when R is in the row) first: scoring waits
    // only for those.
#pragma unroll
    for (int k = 0; k < kSB; ++k) {
        const int sb = (k + kSB - 1) % kSB;
#pragma unroll
        for (int t = 0; t < EPL; ++t) raw[sb][t] = *reinterpret_cast<const uint32_t*>(xb + off[t] + 64 * sb);
    }
#pragma unroll
    for (int t = 0; t < EPL; ++t) {
        if constexpr (RSEP) rsep[t] = n < 8 ? R[uint64_t(jl[t]) * 8 + n] : 0.0f;
        else rsep[t] = 0.0f;
    }
}

// A batch whose loads were issued ahead (the first batch of a row, requested
// before the previous row's epilogue).
template <int EPL>
struct Batch {
    uint32_t raw[kSB][EPL];
    float rsep[EPL];
};

// The first batch of edges [beg, end) (beg < end) requested into b.
template <bool RSEP, int EPL = kEPL>
__device__ inline void first_batch(const uint32_t* __restrict__ xr, const float* __restrict__ R, uint64_t beg,
                                   uint64_t end, int l, uint32_t ids, int id0, Batch<EPL>& b) {
    uint32_t jl[EPL];
    batch_sources<EPL>(ids, id0, uint32_t(end - beg), l, jl);
    load_batch<RSEP, EPL>(xr, R, jl, l, b.raw, b.rsep);
}

// The batches pass through b; PRE: b already holds the first batch
// (first_batch), whose loads are not issued again.
template <bool EXACT, bool RSEP, int EPL = kEPL, bool PRE = false>
__device__ inline void gather_sums(const uint32_t* __restrict__ pcol, const uint32_t* __restrict__ xr,
                                   const float* __restrict__ R, uint64_t beg, uint64_t end, int l, Sums& s,
                                   uint32_t ids, int id0, Batch<EPL>& b) {
    constexpr int B = 4 * EPL;  // edges per batch
    if (beg >= end) return;
    const int g = l / 16, n = l % 16;
    const bool head = n < 8;
    // Edge counts in 32 bits (set_graph rejects rows of 2^32 edges or more),
    // so that the loop's compares run on the scalar unit.
    const uint32_t total = uint32_t(end - beg);
    uint32_t jl[EPL] = {};
    if constexpr (!PRE) batch_sources<EPL>(ids, id0, total, l, jl);
    for (uint32_t done = 0; done < total; done += B) {
        const uint64_t base = beg + done;
        const uint32_t left = total - done;
        const uint32_t nids = pcol[(left > uint32_t(B) ? base + B : end) + uint32_t(l % 32)];
        const int cnt = left < uint32_t(B) ? int(left) : B;
        if (!PRE || done > 0) load_batch<RSEP, EPL>(xr, R, jl, l, b.raw, b.rsep);
        uint32_t (&raw)[kSB][EPL] = b.raw;
        float (&rsep)[EPL] = b.rsep;
        // ---- scores, batch max over the 4 k groups.  SPLIT (R in the row
        // tail, 4 edges per lane): head h's four edges of a k group are
        // scored by lanes h (edges 0, 1; R from lane h + 8 by a DPP rotation
        // within the row) and h + 8 (edges 2, 3; R_h is its own row word 56 +
        // h), whose weights lane h then takes over.  Otherwise the head lanes
        // score all four.  Both see the same scores in the same operations.
        constexpr bool SPLIT = !RSEP && !EXACT && EPL == 4;
        const int hf = n / 8;
        float sc[EPL];
        float mb = -INFINITY;
        if constexpr (SPLIT) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t from = uint32_t(__builtin_amdgcn_mov_dpp(int(raw[3][j]), 0x128, 0xF, 0xF, false));
                const float r = __builtin_bit_cast(float, hf ? raw[3][2 + j] : from);
                sc[j] = EPL * g + 2 * hf + j < cnt ? leaky(s.L + r) : -INFINITY;
                mb = fmaxf(mb, sc[j]);
            }
            mb = max_ror8(mb);
        } else {
#pragma unroll
            for (int t = 0; t < EPL; ++t) {
                const float r = RSEP ? rsep[t]
                                     : __builtin_bit_cast(float,
                                                          __builtin_amdgcn_mov_dpp(int(raw[3][t]), 0x128, 0xF, 0xF, false));
                sc[t] = (head && EPL * g + t < cnt) ? leaky(s.L + r) : -INFINITY;
                mb = fmaxf(mb, sc[t]);
            }
        }
        mb = xor32_max(xor16_max(mb));
        float scale = 1.0f;
        bool resc = false;
        if constexpr (!EXACT) {
            s.mx = max_quiet(s.mx, mb);
            // The first batch (m = -inf) sets m; a later one moves it (and
            // rescales the sums) only beyond m + kLazyMax.
            const bool up = mb > s.m + kLazyMax;
            resc = up && s.m != -INFINITY;
            const float mn = up ? mb : s.m;
            scale = up ? exp_w(s.m - mn) : 1.0f;  // exp(-inf) = 0 on the first batch (the sums are 0)
            s.m = mn;
        }
        // ---- A operand: row h = hi part of p_h, row 8 + h = lo part, for the
        // lane's edges (one MFMA per feature block takes both)
        uint32_t a[EPL / 2];
        float ps = 0.0f;
        if constexpr (SPLIT) {
            const float p0 = exp_w(sc[0] - s.m);  // -inf past the end: 0
            const float p1 = exp_w(sc[1] - s.m);
            const uint32_t hw = bf16x2(p0, p1);
            const uint32_t lw = bf16x2(p0 - __builtin_bit_cast(float, hw << 16), p1 - __builtin_bit_cast(float, hw & 0xffff0000u));
            const float pp = p0 + p1;
            // Lane h feeds row h: hi of edges 0, 1 (its own) and 2, 3 (lane
            // h + 8's); lane h + 8 feeds row 8 + h: lo of edges 0, 1 (lane h's)
            // and 2, 3 (its own).  One DPP exchange carries both halves.
            const uint32_t give = hf ? hw : lw;
            const uint32_t got = uint32_t(__builtin_amdgcn_mov_dpp(int(give), 0x128, 0xF, 0xF, false));
            a[0] = hf ? got : hw;
            a[1] = hf ? lw : got;
            const float po = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, pp), 0x128, 0xF,
                                                                                0xF, false));
            ps = pp + po;  // (p0 + p1) + (p2 + p3) in the head lanes
        } else {
#pragma unroll
            for (int q = 0; q < EPL / 2; ++q) {
                const float p0 = head ? exp_w(sc[2 * q] - s.m) : 0.0f;  // -inf past the end: 0
                const float p1 = head ? exp_w(sc[2 * q + 1] - s.m) : 0.0f;
                ps += p0 + p1;
                const uint32_t hw = bf16x2(p0, p1);
                const uint32_t lw = bf16x2(p0 - __builtin_bit_cast(float, hw << 16),
                                           p1 - __builtin_bit_cast(float, hw & 0xffff0000u));
                // rows 8..15: the lo parts of lane n - 8
                const uint32_t lo = uint32_t(__builtin_amdgcn_mov_dpp(int(lw), 0x128, 0xF, 0xF, false));
                a[q] = head ? hw : lo;
            }
        }
        s.den = s.den * scale + ps;
        if (!EXACT && __any(head && resc)) {
            // D register r of lane group g belongs to head 4 (g % 2) + r.
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float f = __shfl(scale, 4 * (g & 1) + r);
#pragma unroll
                for (int b = 0; b < 2 * kSB; ++b) s.d[b][r] *= f;
            }
        }
        // ---- B operands from the low / high halves of the words, and the MFMAs
#pragma unroll
        for (int sb = 0; sb < kSB; ++sb) {
            uint32_t ev[EPL / 2], od[EPL / 2];
#pragma unroll
            for (int q = 0; q < EPL / 2; ++q) {
                // low halves of w0, w1 (even features) and high halves (odd)
                const uint32_t w0 = raw[sb][2 * q], w1 = raw[sb][2 * q + 1];
                ev[q] = __builtin_amdgcn_perm(w1, w0, 0x05040100u);
                od[q] = __builtin_amdgcn_perm(w1, w0, 0x07060302u);
            }
            s.d[2 * sb] = Mfma<EPL>::run(a, ev, s.d[2 * sb]);
            s.d[2 * sb + 1] = Mfma<EPL>::run(a, od, s.d[2 * sb + 1]);
        }
        // The next batch's sources, formed while the MFMAs run so that its
        // loads leave at the top of the next iteration (past the last batch
        // they go unused).
        batch_sources<EPL>(nids, 0, left - B, l, jl);
    }
}

__device__ inline void zero_sums(Sums& s) {
#pragma unroll
    for (int b = 0; b < 2 * kSB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) s.d[b][r] = 0.0f;
    s.den = 0.0f;
}

// Denominator of head lane (n = h) over the 4 k groups.
__device__ inline float total_den(float den) {
    return xor32_add(xor16_add(den));
}

// U = hi sum + lo sum.  D register r of lane group g holds row 4 g + r: the
// hi parts' sums of head 4 (g % 2) + r in lanes g < 2, the lo parts' in lanes
// g >= 2, 32 lanes apart.  Registers r and r + 1 fold through one
// v_permlane32_swap (odd 32-lane row of the first operand with the even row
// of the second): afterwards lanes g < 2 hold U of head 4 g + r and lanes
// g >= 2 U of head 4 (g - 2) + r + 1.
__device__ inline float fold_pair(float x, float y) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}


// HL: U staged as hi + lo bf16 (FP32 outputs) for 16-row tiles.  Otherwise
// (bf16-stored hidden outputs) U is staged as one bf16 (its rounding is that
// of a bf16 projection input, 2^-9 relative): 32-row tiles (4 rows per wave,
// the MFMA's 32 columns all used), or 16-row tiles in two alternating buffers
// with one barrier per tile (a wave writes buffer t % 2 only after the
// barrier of tile t - 1, which every wave reaches after projecting tile t - 2
// from the same buffer).  Single-buffered tiles take a barrier before and
// after the projection.
// DIM: head width, 32 or 64 (wave h then multiplies U_h by the two 32-column
// blocks of W_h in turn).  KS = 8 (D_in > 112): R from its own array.
// The merge of split row c (its first chunk), by the wave of its last chunk
// to arrive: scales each chunk's sums and denominator by e^(m_c - M_ref),
// M_ref the largest of the chunks' reference maxima, and adds them in chunk
// order (the chunk merge of the running maximum, gat_tfs_online.cpp:86-117);
// then out_h = (U_h W_h) / den_h on the VALU with the FP32 (bf16-rounded) W;
// lane l computes columns 32 cb + 4 (l % 8) .. + 3 of head l / 8, for each
// 32-column block cb of the head.  sw: the wave's kMergeFloats of LDS.
__device__ void afs_merge_row(const AfsArgs& a, uint64_t c, int l, float* sw) {
    const uint32_t k = a.chunk_k[c];
    const uint64_t rbeg = a.prow[k], rend = a.prow[k + 1];
    const uint32_t i = a.perm[k];
    if (i >= a.n || rbeg > rend || rend > a.e) return;
    const uint32_t nch = uint32_t((rend - rbeg + a.chunk_edges - 1) / a.chunk_edges);
    if (c + nch > a.chunks) return;
    // The common reference M_ref and the exact max M (lanes 0..7, head l),
    // then the denominators scaled to M_ref in chunk order.
    float d = 0.0f, mref = -INFINITY;
    if (l < 8) {
        float mx = -INFINITY;
#pragma unroll 16
        for (uint32_t q = 0; q < nch; ++q) {
            mref = fmaxf(mref, a.part[(c + q) * kPart + kMOff + l]);
            mx = fmaxf(mx, a.part[(c + q) * kPart + kMxOff + l]);
        }
#pragma unroll 16
        for (uint32_t q = 0; q < nch; ++q) {
            const float* pq = a.part + (c + q) * kPart;
            d += pq[kDenOff + l] * exp_w(pq[kMOff + l] - mref);
        }
        a.mx[uint64_t(i) * 8 + l] = mx;
        a.den[uint64_t(i) * 8 + l] = d * exp_w(mref - mx);  // against the exact max
    }
    // U_h[f] into LDS (lane l adds features 2l, 2l + 1); the projected row is
    // scaled by 1 / den_h afterwards, as in the tile path.
    float dall[8], rall[8];  // read before any lane is masked off
#pragma unroll
    for (int h = 0; h < 8; ++h) {
        dall[h] = lane_f(d, h);
        rall[h] = lane_f(mref, h);
    }
    if (l < (a.in > kXRFeat ? kRowWords : kXRFeat / 2)) {
        // Chunk by chunk (the order of the sums); the loads of kMergeAhead
        // chunks are requested together, so the chain of partials runs at
        // L2 bandwidth rather than one round trip per chunk.
        constexpr uint32_t kMergeAhead = 2;
        float t[8][2];
#pragma unroll
        for (int h = 0; h < 8; ++h) t[h][0] = t[h][1] = 0.0f;
        auto add_chunks = [&](uint32_t q0, auto count) {
            constexpr uint32_t CNT = decltype(count)::value;
            float2 v[CNT][8];
            float mq[CNT][8];
#pragma unroll
            for (uint32_t u = 0; u < CNT; ++u)
#pragma unroll
                for (int h = 0; h < 8; ++h) {
                    const float* pq = a.part + (c + q0 + u) * kPart;
                    v[u][h] = *reinterpret_cast<const float2*>(pq + 2 * l + h * 128);
                    mq[u][h] = pq[kMOff + h];
                }
#pragma unroll
            for (uint32_t u = 0; u < CNT; ++u)
#pragma unroll
                for (int h = 0; h < 8; ++h) {
                    const float f = exp_w(mq[u][h] - rall[h]);
                    t[h][0] = __builtin_fmaf(v[u][h].x, f, t[h][0]);
                    t[h][1] = __builtin_fmaf(v[u][h].y, f, t[h][1]);
                }
        };
        uint32_t q = 0;
        for (; q + kMergeAhead <= nch; q += kMergeAhead) add_chunks(q, std::integral_constant<uint32_t, kMergeAhead>{});
        for (; q < nch; ++q) add_chunks(q, std::integral_constant<uint32_t, 1>{});
        // bf16-stored hidden outputs: U enters the projection as one bf16, as
        // in the tile path (the rounding of a bf16 projection input).
        const bool round_s = a.outbf != nullptr;
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            float s0 = t[h][0], s1 = t[h][1];
            if (round_s) {
                s0 = bf16_widen(bf16_hw(s0));
                s1 = bf16_widen(bf16_hw(s1));
            }
            sw[h * 128 + 2 * l] = s0;
            sw[h * 128 + 2 * l + 1] = s1;
        }
    }
    wave_sync();
    const int h = l / 8, width = 8 * a.dim;
    float inv = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q)
        if (q == h) inv = dall[q] > 0.0f ? 1.0f / dall[q] : 0.0f;
    for (int cb = 0; cb < a.dim / 32; ++cb) {
        const int c0 = a.dim * h + 32 * cb + 4 * (l % 8);
        float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const float* wcol = a.wq + c0;
        auto fma4 = [&](float sv, const float4& wv) {
            o[0] = __builtin_fmaf(sv, wv.x, o[0]);
            o[1] = __builtin_fmaf(sv, wv.y, o[1]);
            o[2] = __builtin_fmaf(sv, wv.z, o[2]);
            o[3] = __builtin_fmaf(sv, wv.w, o[3]);
        };
        // 16 rows of W requested at a time (L2-resident), then their FMAs in order.
        int f = 0;
        for (; f + 16 <= a.in; f += 16) {
            float4 wv[16];
#pragma unroll
            for (int x = 0; x < 16; ++x) wv[x] = *reinterpret_cast<const float4*>(wcol + uint64_t(f + x) * width);
#pragma unroll
            for (int x = 0; x < 16; ++x) fma4(sw[h * 128 + f + x], wv[x]);
        }
        for (; f < a.in; ++f) fma4(sw[h * 128 + f], *reinterpret_cast<const float4*>(wcol + uint64_t(f) * width));
#pragma unroll
        for (int x = 0; x < 4; ++x) o[x] *= inv;
        if (a.hidden)
#pragma unroll
            for (int x = 0; x < 4; ++x) o[x] = elu_bf16(o[x]);
        const uint64_t off = uint64_t(i) * width + c0;
        if (a.outbf)
            *reinterpret_cast<uint2*>(a.outbf + off) = make_uint2(bf16x2(o[0], o[1]), bf16x2(o[2], o[3]));
        if (a.out32) *reinterpret_cast<float4*>(a.out32 + off) = make_float4(o[0], o[1], o[2], o[3]);
    }
}

// Chunk c of a split row, one wave: sums against maxima of its own (the lazy
// reference max and the exact max) into part[c][h * 128 + f], the
// denominators and both maxima after them; the last chunk of the row to
// arrive (agent-scope release/acquire around a relaxed counter) merges the
// row.  sw: the wave's kMergeFloats of LDS.
__device__ void afs_chunk(const AfsArgs& a, uint64_t c, int l, float* sw) {
    const int g = l / 16, n = l % 16;
    const bool head = n < 8;
    if (c >= a.chunks) return;
    const uint32_t k = a.chunk_k[c], first = a.chunk_first[c];
    const uint64_t rbeg = a.prow[k], rend = a.prow[k + 1];
    const uint32_t i = a.perm[k];
    if (i >= a.n || rbeg > rend || rend > a.e) return;
    const uint64_t beg = rbeg + uint64_t(c - first) * a.chunk_edges;
    const uint64_t end = beg + a.chunk_edges < rend ? beg + a.chunk_edges : rend;
        const bool rsep = a.in > kXRFeat;
    Sums s;
    zero_sums(s);
    s.L = head || !rsep ? a.L[uint64_t(i) * 8 + n % 8] : 0.0f;  // (lanes h + 8 score half of head h's edges)
    s.m = s.mx = -INFINITY;
    Batch<kEPL> b;
    if (rsep) gather_sums<false, true>(a.pcol, a.xr, a.R, beg, end, l, s, a.pcol[beg + uint32_t(l % 32)], 0, b);
    else gather_sums<false, false>(a.pcol, a.xr, a.R, beg, end, l, s, a.pcol[beg + uint32_t(l % 32)], 0, b);
    const float den = total_den(s.den);
    float* part = a.part + c * kPart;
    {
        // lane (g, n): head 4 (g % 2) + q + (g >= 2) after fold_pair, q = 0, 2
        const int hb = 4 * (g & 1) + (g >> 1);
#pragma unroll
        for (int sb = 0; sb < kSB; ++sb) {
            const int P = 16 * sb + n;
            if (P >= (rsep ? kRowWords : kXRFeat / 2)) continue;
#pragma unroll
            for (int q = 0; q < 4; q += 2)
                *reinterpret_cast<float2*>(part + (hb + q) * 128 + 2 * P) =
                    make_float2(fold_pair(s.d[2 * sb][q], s.d[2 * sb][q + 1]),
                                fold_pair(s.d[2 * sb + 1][q], s.d[2 * sb + 1][q + 1]));
        }
    }
    if (head && g == 0) {
        part[kDenOff + n] = den;
        part[kMOff + n] = s.m;
        part[kMxOff + n] = s.mx;
    }
    const uint32_t nch = uint32_t((rend - rbeg + a.chunk_edges - 1) / a.chunk_edges);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    uint32_t old = 0;
    if (l == 0) old = __hip_atomic_fetch_add(a.counter + first, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __shfl(old, 0);
    if (old + 1 != nch) return;  // not the last chunk of this row
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (l == 0) a.counter[first] = 0;  // ready for the next launch
    afs_merge_row(a, first, l, sw);
}


template <int KS, bool HL, int TR, int DIM, bool SHORT>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) k_afs_tiles(AfsArgs a) {
    static_assert(TR == 16 || (TR == 32 && !HL), "16-row tiles, or 32-row tiles of one bf16");
    static_assert(!SHORT || !HL, "short rows: 32-row tiles of bf16-stored rows");
    static_assert(DIM == 32 || DIM == 64, "heads of 32 or 64");
    constexpr bool RSEP = KS == 8;
    constexpr int RPW = TR / kWaves;          // rows per wave and tile
    constexpr bool DB = !HL && TR == 16;      // two alternating U buffers
    constexpr int BLK = TR * 32 + 32;         // bytes per (head, k step[, hi|lo]) block of S
    static_assert(8 * kMaxKS * (HL ? 2 : DB ? 2 : 1) * BLK + kHalfOff <= kSBytes, "U fits");
    static_assert(2 * 8 * (TR + 1) * 4 <= kTDenBytes && 2 * TR * 4 <= kTRowBytes, "ids and denominators fit");
    extern __shared__ __attribute__((aligned(16))) unsigned char slds[];
    // Destination node of each tile row (kNoRow: none), for the projection stores.
    uint32_t* const trow_all = reinterpret_cast<uint32_t*>(slds + kSBytes);
    // den_h of tile row r at [h][r] (rows of TR + 1 floats: the 8 head lanes
    // that write a row's values, and the 32 lanes that read a head's, each
    // meet distinct banks).
    float* const tden_all = reinterpret_cast<float*>(slds + kSBytes + kTRowBytes);
    int buf = 0;
    const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int l = threadIdx.x % kWave;
    const int g = l / 16, n = l % 16;
    const bool head = n < 8;
    const uint32_t chunk_blocks = gridDim.x - a.tile_blocks;
    if (!SHORT && blockIdx.x < chunk_blocks) {
        // Split-row chunks, one per wave, in the first blocks: they start with
        // the launch, and the tile blocks that wait for their slots take fewer
        // tiles.
        static_assert(kWaves * kMergeFloats * 4 <= kSBytes, "merge scratch fits");
        afs_chunk(a, uint64_t(blockIdx.x) * kWaves + w, l, reinterpret_cast<float*>(slds) + w * kMergeFloats);
        return;
    }
    // Tiles in a dynamic order: the block's first three are tb, tb + G and
    // tb + 2G (G tile blocks); tile j + 3 is taken from the launch's counter
    // during tile j and published in the ring tq for tile j + 1, which
    // requests its bounds two tiles ahead.  The last tile block to finish
    // clears the counters for the next launch.
    const uint32_t tb = blockIdx.x - chunk_blocks, G = a.tile_blocks;
    uint32_t* const tq = reinterpret_cast<uint32_t*>(slds + kSBytes + kTRowBytes + kTDenBytes);
    // The tile rows' max (8 per row) and den stages, written out as whole
    // lines after the tile's barrier.
    float* const smd = reinterpret_cast<float*>(slds + kSBytes + kTRowBytes + kTDenBytes + kTQBytes);
    static_assert(2 * 8 * TR * 4 <= kTMdBytes, "stage rows fit");
    static_assert(!DB, "the stage rows are single-buffered: the next tile writes them after the closing barrier");
    uint32_t* const tctr = a.counter + a.chunks;  // [0] tiles taken past 3G, [1] tile blocks done
    const uint64_t span = a.rows - a.row_lo, tiles = (span + TR - 1) / TR;
    if (threadIdx.x == 0) tq[2] = tb + 2 * G;
    __syncthreads();
    // Bounds of the wave's rows of tile t (lane q < RPW: tile row w + 8 q),
    // requested one tile ahead (during the previous tile's projection).
    auto fetch_bounds = [&](uint64_t t, uint32_t& fi, uint64_t& fb, uint64_t& fe) {
        fi = kNoRow;
        fb = fe = 0;
        const uint64_t tpos = t * TR + w + kWaves * l;
        if (l < RPW && t < tiles && tpos < span) {
            const uint64_t k = a.rows - 1 - tpos;
            fi = a.perm[k];
            fb = a.prow[k];
            fe = a.prow[k + 1];
        }
    };
    // First source ids (lane 32 (q % 2) + t of ids[q / 2]) and L (lane
    // 8 q + h) of the wave's rows; a row with malformed bounds becomes kNoRow.
    constexpr int NID = (RPW + 1) / 2;
    auto fetch_ids = [&](uint32_t& fi, uint64_t fb, uint64_t fe, uint32_t (&ids)[NID], float& Lv) {
        if (fi != kNoRow && (fi >= a.n || fb > fe || fe > a.e)) fi = kNoRow;
#pragma unroll
        for (int c = 0; c < NID; ++c) {
            const int q = 2 * c + l / 32;
            const uint32_t qi = __shfl(fi, q);
            const uint64_t qb = (uint64_t(__shfl(uint32_t(fb >> 32), q)) << 32) | __shfl(uint32_t(fb), q);
            ids[c] = a.pcol[(q < RPW && qi != kNoRow ? qb : 0) + uint32_t(l % 32)];
        }
        Lv = 0.0f;
        const uint32_t qi = __shfl(fi, l / 8);
        if (l / 8 < RPW && qi != kNoRow) Lv = a.L[uint64_t(qi) * 8 + l % 8];
    };
    // Pipeline over the block's tiles: the bounds of tile t + 2 and the first
    // ids and L of tile t + 1 are requested at the start of tile t, so a tile
    // starts with its rows' first batches.
    uint32_t mi, nmi;
    uint64_t mb, me, nmb, nme;
    uint32_t idr[NID], nidr[NID];
    float Lall, nLall;
    fetch_bounds(tb, mi, mb, me);
    fetch_bounds(tb + uint64_t(G), nmi, nmb, nme);
    fetch_ids(mi, mb, me, idr, Lall);
    uint64_t tile = tb, tnext = tb + uint64_t(G);
    for (uint32_t j = 0; tile < tiles; ++j, buf ^= DB ? 1 : 0) {
        const uint64_t t2 = uint32_t(__builtin_amdgcn_readfirstlane(int(tq[(j + 2) & 3])));
        uint32_t taken = 0;
        if (threadIdx.x == 0)
            taken = 3 * G + __hip_atomic_fetch_add(tctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t* const trow = trow_all + buf * TR;
        float* const tden = tden_all + buf * 8 * (TR + 1);
        // ---- RPW rows per wave (tile rows w + 8 q): bounds in lane q, L in
        // lanes 8 q + h, first ids in idr.
        uint32_t n2mi;
        uint64_t n2mb, n2me;
        fetch_ids(nmi, nmb, nme, nidr, nLall);
        fetch_bounds(t2, n2mi, n2mb, n2me);
        // Row q of the wave: node, edge range and first ids.
        auto row_of = [&](int q, uint32_t& qi, uint64_t& qb, uint64_t& qe, uint32_t& qids) {
            qi = uint32_t(__builtin_amdgcn_readlane(int(mi), q));
            qb = (uint64_t(uint32_t(__builtin_amdgcn_readlane(int(mb >> 32), q))) << 32) |
                 uint32_t(__builtin_amdgcn_readlane(int(uint32_t(mb)), q));
            qe = (uint64_t(uint32_t(__builtin_amdgcn_readlane(int(me >> 32), q))) << 32) |
                 uint32_t(__builtin_amdgcn_readlane(int(uint32_t(me)), q));
            qids = q / 2 == 0 ? idr[0] : idr[(RPW + 1) / 2 - 1];
        };
        if constexpr (SHORT) {
            // ---- Short rows (this instance takes the sorted positions whose
            // rows have at most kShortDeg = 4 edges: on the 2^22-node R-MAT
            // graph 3.0M of the 4.2M rows).  The wave's four rows share one
            // 16-edge batch, k group g taking the edges of row g: one round trip
            // for four rows, where a row took one of its own.  Such a row has one
            // batch: its max is the batch's, nothing is rescaled, and its weights
            // p, max and denominator are those of a one-row batch bit for bit.
            // Row m = 4 v + x of the MFMA's A is row v's head 4 hf + x in pass hf:
            // that row's weights in k group v and zeros in the others.  U = (hi
            // parts' sum) + (lo parts' sum) from two MFMAs, the two sums a one-row
            // batch keeps in D rows h and 8 + h and fold_pair adds.
            static_assert(kShortDeg == kEPL && RPW == 4 && NID == 2, "one k group (4 edges) per row, four rows");
            uint32_t cnt = 0;  // edges of the lane's row g (0 for none)
#pragma unroll
            for (int q = 0; q < RPW; ++q) {
                uint32_t qi, qids;
                uint64_t qb, qe;
                row_of(q, qi, qb, qe, qids);
                if (l == 0) trow[w + kWaves * q] = qi;
                if (g == q) cnt = qi == kNoRow ? 0u : uint32_t(qe - qb);
            }
            // Sources: id t of row g (lane 32 (g % 2) + t of idr[g / 2]); past
            // the row's end its last edge again (weight 0), and an empty row
            // reads its first id slot (padding or the next row's).
            uint32_t jl[kEPL];
#pragma unroll
            for (int t = 0; t < kEPL; ++t) {
                const int src = 4 * (32 * (g & 1) + max(min(t, int(cnt) - 1), 0));
                const uint32_t v0 = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(idr[0])));
                const uint32_t v1 = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(idr[1])));
                jl[t] = (g >> 1) ? v1 : v0;
            }
            uint32_t raw[kSB][kEPL];
            float rsep[kEPL];
            load_batch<RSEP, kEPL>(a.xr, a.R, jl, l, raw, rsep);
            // Head lanes score their row's edges for head n: the row max, the
            // weights and their hi / lo parts, the denominator.
            const float Lq = __shfl(Lall, 8 * g + n % 8);
            float sc[kEPL];
            float mq = -INFINITY;
#pragma unroll
            for (int t = 0; t < kEPL; ++t) {
                const float r = RSEP ? rsep[t]
                                     : __builtin_bit_cast(
                                           float, __builtin_amdgcn_mov_dpp(int(raw[3][t]), 0x128, 0xF, 0xF, false));
                sc[t] = (head && t < int(cnt)) ? leaky(Lq + r) : -INFINITY;
                mq = fmaxf(mq, sc[t]);
            }
            const float mz = cnt > 0 ? mq : 0.0f;  // (an empty row: every weight 0)
            uint32_t hw[2], lw[2];
            float ps = 0.0f;
#pragma unroll
            for (int q2 = 0; q2 < 2; ++q2) {
                const float p0 = exp_w(sc[2 * q2] - mz);  // -inf past the end: 0
                const float p1 = exp_w(sc[2 * q2 + 1] - mz);
                ps += p0 + p1;
                hw[q2] = bf16x2(p0, p1);
                lw[q2] = bf16x2(p0 - __builtin_bit_cast(float, hw[q2] << 16),
                                p1 - __builtin_bit_cast(float, hw[q2] & 0xffff0000u));
            }
            const int r = w + kWaves * g;  // the lane's tile row
            if (head) {
                smd[r * 8 + n] = cnt > 0 ? mq : 0.0f;
                smd[(TR + r) * 8 + n] = cnt > 0 ? ps : 0.0f;
                tden[n * (TR + 1) + r] = ps;
            }
            // Pass hf: lane (g, n) supplies A row n at k = 4 g .. 4 g + 3, the
            // weights of head 4 hf + n % 4 from its k group's head lane where
            // row n / 4 is its own (g), zeros elsewhere.
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                const int srcl = 4 * (16 * g + 4 * hf + n % 4);
                const bool mine = n / 4 == g;
                uint32_t ah[2], al[2];
#pragma unroll
                for (int q2 = 0; q2 < 2; ++q2) {
                    const uint32_t th = uint32_t(__builtin_amdgcn_ds_bpermute(srcl, int(hw[q2])));
                    const uint32_t tl = uint32_t(__builtin_amdgcn_ds_bpermute(srcl, int(lw[q2])));
                    ah[q2] = mine ? th : 0u;
                    al[q2] = mine ? tl : 0u;
                }
#pragma unroll
                for (int sb = 0; sb < kSB; ++sb) {
                    uint32_t ev[2], od[2];
#pragma unroll
                    for (int q2 = 0; q2 < 2; ++q2) {
                        const uint32_t w0 = raw[sb][2 * q2], w1 = raw[sb][2 * q2 + 1];
                        ev[q2] = __builtin_amdgcn_perm(w1, w0, 0x05040100u);
                        od[q2] = __builtin_amdgcn_perm(w1, w0, 0x07060302u);
                    }
                    const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                    const f32x4 eh = Mfma<kEPL>::run(ah, ev, z), el = Mfma<kEPL>::run(al, ev, z);
                    const f32x4 oh = Mfma<kEPL>::run(ah, od, z), ol = Mfma<kEPL>::run(al, od, z);
                    // D register x of lane (g, n): A row 4 g + x, i.e. row g's head
                    // 4 hf + x, feature pair 16 sb + n; an empty row stages +0.
                    const int ks = 2 * sb + n / 8;
                    if (ks >= KS) continue;
#pragma unroll
                    for (int x = 0; x < 4; ++x) {
                        const int h = 4 * hf + x;
                        const float s0 = eh[x] + el[x], s1 = oh[x] + ol[x];
                        *reinterpret_cast<uint32_t*>(slds + 32 * r + 4 * (n % 8) + (h >= 4 ? kHalfOff : 0) +
                                                     ((buf * 8 + h) * kMaxKS + ks) * BLK) =
                            cnt > 0 ? bf16x2(s0, s1) : 0u;
                    }
                }
            }
            // (the projection's W fragment loads stay below: hoisted into the
            // batch they would hold their registers across its MFMAs)
            __builtin_amdgcn_sched_barrier(0);
        } else {
            // Each row's first batch is requested before the previous row's
            // epilogue (its loads then travel while that row's sums are staged).
            Batch<kEPL> pre;
            bool have_pre = false;  // wave-uniform
#pragma unroll 1
            for (int rr = 0; rr < RPW; ++rr) {
                const int r = w + kWaves * rr;
                uint32_t i, ids;
                uint64_t beg, end;
                row_of(rr, i, beg, end, ids);
                const float Lr = __shfl(Lall, 8 * rr + n % 8);
                if (l == 0) trow[r] = i;
                if (i == kNoRow) continue;
                Sums s;
                zero_sums(s);
                s.L = head || !RSEP ? Lr : 0.0f;  // (lanes h + 8 score half of head h's edges)
                s.m = s.mx = -INFINITY;
                if (!have_pre && beg < end) first_batch<RSEP>(a.xr, a.R, beg, end, l, ids, 32 * (rr % 2), pre);
                gather_sums<false, RSEP, kEPL, true>(a.pcol, a.xr, a.R, beg, end, l, s, ids, 32 * (rr % 2), pre);
                have_pre = false;
                if (rr + 1 < RPW) {
                    uint32_t ni, nids;
                    uint64_t nb, ne;
                    row_of(rr + 1, ni, nb, ne, nids);
                    if (ni != kNoRow && nb < ne) {
                        first_batch<RSEP>(a.xr, a.R, nb, ne, l, nids, 32 * ((rr + 1) % 2), pre);
                        have_pre = true;
                    }
                }
                const float den = total_den(s.den);  // against the reference max s.m
                if (head && g == 0) {
                    // empty row: max 0, denominator 0 (ref_fp32.cpp:11); else the
                    // denominator against the row max, sum e^(s - M) = den e^(m - M)
                    smd[r * 8 + n] = end > beg ? s.mx : 0.0f;
                    smd[(TR + r) * 8 + n] = end > beg ? den * exp_w(s.m - s.mx) : 0.0f;
                    tden[n * (TR + 1) + r] = den;  // against the reference max, as U
                }
                {
                    // After fold_pair, lane (g, n) holds U of head 4 (g % 2) + q + (g >= 2)
                    // for q = 0, 2.  Element (head h, feature pair P = 16 sb + n) of tile
                    // row r sits at block (h, P / 8[, hl]) + 32 r + 4 (P % 8): a per-lane
                    // base plus a compile-time offset for each (q, sb, hl); block index
                    // ((h * kMaxKS + ks) * 2 + hl) with hi + lo, (buf * 8 + h) * kMaxKS + ks
                    // without.  (With KS <= 7 the words of R, 56..63, fall in k step 7.)
                    const int gh = g & 1, up = g >> 1;
                    unsigned char* base =
                        slds + 32 * r + 4 * (n % 8) + kHalfOff * gh +
                        (HL ? 8 * kMaxKS * gh + 2 * kMaxKS * up + 2 * (n / 8)
                            : buf * 8 * kMaxKS + 4 * kMaxKS * gh + kMaxKS * up + n / 8) *
                            BLK;
#pragma unroll
                    for (int sb = 0; sb < kSB; ++sb) {
                        const int ks = 2 * sb + n / 8;
                        if (ks >= KS) continue;
#pragma unroll
                        for (int q = 0; q < 4; q += 2) {
                            const float s0 = fold_pair(s.d[2 * sb][q], s.d[2 * sb][q + 1]);
                            const float s1 = fold_pair(s.d[2 * sb + 1][q], s.d[2 * sb + 1][q + 1]);
                            const uint32_t hw = bf16x2(s0, s1);
                            if constexpr (HL) {
                                const uint32_t lw = bf16x2(s0 - __builtin_bit_cast(float, hw << 16),
                                                           s1 - __builtin_bit_cast(float, hw & 0xffff0000u));
                                unsigned char* e = base + (2 * kMaxKS * q + 4 * sb) * BLK;
                                *reinterpret_cast<uint32_t*>(e) = hw;
                                *reinterpret_cast<uint32_t*>(e + BLK) = lw;
                            } else {
                                *reinterpret_cast<uint32_t*>(base + (kMaxKS * q + 2 * sb) * BLK) = hw;
                            }
                        }
                    }
                }
            }
        }
        // W_h^T fragments of this wave's head (h = w; 1 KB per k step and
        // 32-column block, L2 resident), the first block's requested before
        // the barrier.  A wave-uniform base plus a 32-bit lane offset, made
        // opaque so that the addresses are formed here instead of being held
        // across the gather.  Head block NBH h + b sits in group (NBH h + b) / 8,
        // block (NBH h + b) % 8 of the packing.
        constexpr int NBH = DIM / 32;
        bf16x8 wf[KS];
        auto load_w = [&](int b) {
            uint32_t lo = uint32_t(l) * uint32_t(sizeof(uint4));
            asm volatile("" : "+v"(lo));
            const int hb = NBH * w + b;
            const unsigned char* wb = reinterpret_cast<const unsigned char*>(a.wpk) +
                                      (uint64_t(hb / 8) * a.ksteps * a.nmb + hb % 8) * kWave * sizeof(uint4);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
                wf[ks] = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const uint4*>(wb + uint64_t(ks) * a.nmb * kWave * sizeof(uint4) + lo));
        };
        load_w(0);
        if (threadIdx.x == 0) tq[(j + 3) & 3] = taken;
        __syncthreads();
        if (w == kWaves - 1) {
            // The tile's max and den stages: tile row r is sorted position
            // rows - 1 - (tile TR + r), so lane l takes row TR - 1 - l / 2 and
            // the lanes store consecutive 16-byte pieces (whole lines) where
            // each head lane used to store 4 bytes per row.
            const int r = TR - 1 - l / 2, q = 4 * (l % 2);
            if (r >= 0) {
                const uint32_t i = trow[r];
                if (i != kNoRow) {
                    *reinterpret_cast<float4*>(a.mx + uint64_t(i) * 8 + q) = *reinterpret_cast<const float4*>(smd + r * 8 + q);
                    *reinterpret_cast<float4*>(a.den + uint64_t(i) * 8 + q) =
                        *reinterpret_cast<const float4*>(smd + (TR + r) * 8 + q);
                }
            }
        }
        // 1 / den of the lane's output row (tile row l % 32) and head w; an
        // empty row has U = 0 and den = 0, and gives 0.
        float inv;
        {
            const float dv = tden[w * (TR + 1) + (l % 32) % TR];
            inv = dv > 0.0f ? 1.0f / dv : 0.0f;
        }
        // ---- wave h: the tile's U_h W_h / den_h.  B lane l reads tile row l % 16 (lanes
        // with l % 32 >= 16 repeat rows 0..15; their output columns are dropped).
        uint32_t P0[2][4];  // heads of 64: block 0's stored pieces, kept for the whole-line stores
#pragma unroll
        for (int b = 0; b < NBH; ++b) {
            if (b > 0) load_w(b);
            const int h = w;
            f32x16 dh, dl;
#pragma unroll
            for (int x = 0; x < 16; ++x) dh[x] = dl[x] = 0.0f;
            const int boff = (l % TR) * 32 + 16 * (l / 32) + (h >= 4 ? kHalfOff : 0);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                if constexpr (HL) {
                    const bf16x8 bh = __builtin_bit_cast(
                        bf16x8, *reinterpret_cast<const uint4*>(slds + ((h * kMaxKS + ks) * 2) * BLK + boff));
                    const bf16x8 bl = __builtin_bit_cast(
                        bf16x8, *reinterpret_cast<const uint4*>(slds + ((h * kMaxKS + ks) * 2 + 1) * BLK + boff));
                    dh = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[ks], bh, dh, 0, 0, 0);
                    dl = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[ks], bl, dl, 0, 0, 0);
                } else {
                    // even / odd k steps in two chains; heads of 64 one chain
                    // (the registers of the second hold block 0's stored pieces)
                    const bf16x8 bv = __builtin_bit_cast(
                        bf16x8, *reinterpret_cast<const uint4*>(slds + ((buf * 8 + h) * kMaxKS + ks) * BLK + boff));
                    if (NBH == 2 || ks % 2 == 0) dh = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[ks], bv, dh, 0, 0, 0);
                    else dl = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[ks], bv, dl, 0, 0, 0);
                }
            }
            // Lane (half, r) holds features DIM h + 32 b + 16 half + {0..15} of
            // tile row r (permuted packing).
            const int r = l % 32, half = l / 32;
            if constexpr (!HL) {
                // bf16 hidden rows (ELU).  Each store leaves the head block's 64
                // contiguous bytes of 16 rows, where one 16-byte piece per row
                // and lane half left before (3.171 -> 3.137 ms on the 64.3M-edge
                // layer): inside the lane quad (rows 4a .. 4a + 3), store j
                // takes rows 4a + 2j and 4a + 2j + 1, lane c writing piece
                // 2 half + c % 2 of row 4a + 2j + c / 2, read from quad lane
                // 2j + c / 2 by DPP.
                static_assert(TR == 32, "bf16 tiles hold 32 rows");
                uint32_t P[2][4];  // the lane's two 16-byte pieces (2 half, 2 half + 1)
#pragma unroll
                for (int q = 0; q < 2; ++q)
#pragma unroll
                    for (int x = 0; x < 4; ++x)
                        P[q][x] = NBH == 2 ? bf16x2(elu_bf16(dh[8 * q + 2 * x] * inv), elu_bf16(dh[8 * q + 2 * x + 1] * inv))
                                           : bf16x2(elu_bf16((dh[8 * q + 2 * x] + dl[8 * q + 2 * x]) * inv),
                                                    elu_bf16((dh[8 * q + 2 * x + 1] + dl[8 * q + 2 * x + 1]) * inv));
                const int c = l & 3;
                auto store_pair = [&](auto J) {
                    constexpr int j = decltype(J)::value;
                    constexpr int kSel = j ? 0xFA : 0x50;  // quad_perm [2j, 2j, 2j + 1, 2j + 1]
                    uint32_t T[4];
#pragma unroll
                    for (int x = 0; x < 4; ++x) {
                        const uint32_t a0 = uint32_t(__builtin_amdgcn_mov_dpp(int(P[0][x]), kSel, 0xF, 0xF, false));
                        const uint32_t a1 = uint32_t(__builtin_amdgcn_mov_dpp(int(P[1][x]), kSel, 0xF, 0xF, false));
                        T[x] = (c & 1) ? a1 : a0;
                    }
                    const uint32_t ij = trow[(r & ~3) + 2 * j + (c >> 1)];
                    if (ij != kNoRow)
                        *reinterpret_cast<uint4*>(a.outbf + uint64_t(ij) * (8 * DIM) + DIM * h + 32 * b + 16 * half +
                                                  8 * (c & 1)) = make_uint4(T[0], T[1], T[2], T[3]);
                };
                if constexpr (NBH == 1) {
                    store_pair(std::integral_constant<int, 0>{});
                    store_pair(std::integral_constant<int, 1>{});
                } else if (b == 0) {
#pragma unroll
                    for (int q = 0; q < 2; ++q)
#pragma unroll
                        for (int x = 0; x < 4; ++x) P0[q][x] = P[q][x];
                } else {
                    // Heads of 64: the head's 128 bytes of a row are one line,
                    // block b's piece q of half `half` at bytes 64 b + 32 half +
                    // 16 q.  Slot p of a lane is block p / 2, piece p % 2; a 4 x
                    // 4 transpose inside the lane quad (two DPP exchange stages,
                    // lane c taking slot p from quad lane c ^ 1, then c ^ 2)
                    // leaves lane c with slot c of rows 4a .. 4a + 3, so store j
                    // writes row 4a + j whole from the 8 lanes of quad a (both
                    // halves): 8 lines per instruction, where each block's
                    // stores wrote half lines of 16 rows.
                    uint32_t S[4][4], U[4][4], T[4][4];
#pragma unroll
                    for (int x = 0; x < 4; ++x) {
                        S[0][x] = P0[0][x];
                        S[1][x] = P0[1][x];
                        S[2][x] = P[0][x];
                        S[3][x] = P[1][x];
                    }
#pragma unroll
                    for (int p = 0; p < 4; ++p)
#pragma unroll
                        for (int v = 0; v < 4; ++v) {
                            const uint32_t o = uint32_t(__builtin_amdgcn_mov_dpp(int(S[p ^ 1][v]), 0xB1, 0xF, 0xF, false));
                            U[p][v] = (c & 1) == (p & 1) ? S[p][v] : o;  // quad_perm [1, 0, 3, 2]
                        }
#pragma unroll
                    for (int p = 0; p < 4; ++p)
#pragma unroll
                        for (int v = 0; v < 4; ++v) {
                            const uint32_t o = uint32_t(__builtin_amdgcn_mov_dpp(int(U[p ^ 2][v]), 0x4E, 0xF, 0xF, false));
                            T[p][v] = (c & 2) == (p & 2) ? U[p][v] : o;  // quad_perm [2, 3, 0, 1]
                        }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t ij = trow[(r & ~3) + j];
                        if (ij != kNoRow)
                            *reinterpret_cast<uint4*>(a.outbf + uint64_t(ij) * (8 * DIM) + DIM * h + 32 * (c / 2) +
                                                      16 * half + 8 * (c % 2)) =
                                make_uint4(T[j][0], T[j][1], T[j][2], T[j][3]);
                    }
                }
            } else {
                // FP32 outputs (the last layer, no ELU): 16 tile rows, 64 bytes
                // per lane.
                const uint32_t i = trow[r % TR];
                if (r < TR && i != kNoRow) {
                    const uint64_t off = uint64_t(i) * (8 * DIM) + DIM * h + 32 * b + 16 * half;
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        *reinterpret_cast<float4*>(a.out32 + off + 4 * q) =
                            make_float4((dh[4 * q] + dl[4 * q]) * inv, (dh[4 * q + 1] + dl[4 * q + 1]) * inv,
                                        (dh[4 * q + 2] + dl[4 * q + 2]) * inv, (dh[4 * q + 3] + dl[4 * q + 3]) * inv);
                }
            }
        }
        if constexpr (!DB) __syncthreads();
        mi = nmi;
        mb = nmb;
        me = nme;
        nmi = n2mi;
        nmb = n2mb;
        nme = n2me;
#pragma unroll
        for (int c = 0; c < NID; ++c) idr[c] = nidr[c];
        Lall = nLall;
        tile = tnext;
        tnext = t2;
    }
    if (threadIdx.x == 0) {
        const uint32_t done = __hip_atomic_fetch_add(tctr + 1, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (done + 1 == G) {
            __hip_atomic_store(tctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(tctr + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// One block per kWaves chunks of split rows, then a resident grid of tile
// blocks (two per CU) over the sorted positions [a.row_lo, a.rows).  a.counter
// holds chunks + 2 entries, zero between launches.  SHORT: tile blocks only.
template <int KS, bool HL, int TR, int DIM, bool SHORT>
hipError_t launch_tiles_hl(AfsArgs a, hipStream_t s, int cus) {
    if (a.row_lo > a.rows) return hipErrorInvalidValue;
    const uint64_t tiles = (a.rows - a.row_lo + TR - 1) / TR;
    uint64_t blocks = uint64_t(cus) * 2;
    if (blocks > tiles) blocks = tiles;
    const uint64_t chunk_blocks = SHORT ? 0 : (a.chunks + kWaves - 1) / kWaves;
    if (blocks + chunk_blocks == 0) return hipSuccess;
    if (tiles >= (uint64_t(1) << 31) || blocks + chunk_blocks > 0x7fffffffu) return hipErrorInvalidValue;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_afs_tiles<KS, HL, TR, DIM, SHORT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return e;
    a.tile_blocks = uint32_t(blocks);
    k_afs_tiles<KS, HL, TR, DIM, SHORT><<<dim3(uint32_t(chunk_blocks + blocks)), kThreads, kLdsBytes, s>>>(a);
    return hipGetLastError();
}

// FP32 outputs (the last layer, no ELU) keep U as hi + lo; bf16-stored hidden
// outputs stage one bf16, and their rows of at most kShortDeg edges (positions
// [0, a.short_rows)) go to the short-row instance in a launch of their own
// after the others (the two launches share the tile counters, which each
// leaves at zero).
template <int KS>
hipError_t launch_tiles(const AfsArgs& a, hipStream_t s, int cus) {
    if (a.hidden != (a.out32 == nullptr) || (a.out32 == nullptr) == (a.outbf == nullptr)) return hipErrorInvalidValue;
    if (a.short_rows > a.rows) return hipErrorInvalidValue;
    AfsArgs al = a;
    al.row_lo = 0;
    if (a.out32)
        return a.dim == 64 ? launch_tiles_hl<KS, true, 16, 64, false>(al, s, cus)
                           : launch_tiles_hl<KS, true, 16, 32, false>(al, s, cus);
    al.row_lo = a.short_rows;
    hipError_t e = a.dim == 64 ? launch_tiles_hl<KS, false, kTileBf16, 64, false>(al, s, cus)
                               : launch_tiles_hl<KS, false, kTileBf16, 32, false>(al, s, cus);
    if (e != hipSuccess || a.short_rows == 0) return e;
    AfsArgs as = a;
    as.rows = a.short_rows;
    as.row_lo = 0;
    return a.dim == 64 ? launch_tiles_hl<KS, false, kTileBf16, 64, true>(as, s, cus)
                       : launch_tiles_hl<KS, false, kTileBf16, 32, true>(as, s, cus);
}

}  // namespace

// Up to 128 inputs (up to 112 with R in the row tail, else R from its own
// array), 8 heads of 32 or 64.
bool aggregate_afsum_supported(int in, int heads, int dim, uint64_t n) {
    return in >= 1 && in <= kXRStride && heads == 8 && (dim == 32 || dim == 64) &&
           n <= (uint64_t(1) << 32) / (4 * kRowWords);
}

hipError_t launch_aggregate_afsum(const AfsArgs& a, const SplitTable& t, hipStream_t s, int cus) {
    if (!aggregate_afsum_supported(a.in, 8, a.dim, a.n) || a.nmb < 8 || a.ksteps != (a.in + 15) / 16 || !a.xr ||
        !a.wq || !a.R)
        return hipErrorInvalidValue;
    if (!a.counter) return hipErrorInvalidValue;
    hipError_t e = hipSuccess;
    switch (a.ksteps) {
        case 1: e = launch_tiles<1>(a, s, cus); break;
        case 2: e = launch_tiles<2>(a, s, cus); break;
        case 3: e = launch_tiles<3>(a, s, cus); break;
        case 4: e = launch_tiles<4>(a, s, cus); break;
        case 5: e = launch_tiles<5>(a, s, cus); break;
        case 6: e = launch_tiles<6>(a, s, cus); break;
        case 7: e = launch_tiles<7>(a, s, cus); break;
        default: e = launch_tiles<8>(a, s, cus); break;
    }
    return e;
}

}  // namespace gatgpu
