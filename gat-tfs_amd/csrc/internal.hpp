// Internal declarations shared by the HIP translation units of libgatgpu.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

namespace gatgpu {

constexpr int kWave = 64;  // CDNA4 wavefront

// ---------------------------------------------------------------- bf16 bits
// FP32 -> bf16 round-to-nearest-even, NaN quieted to (u>>16)|0x40; the
// conversion of baseline/src/common.cpp:80-83, written on raw bits so NaN
// payloads and ties match the reference exactly.
__host__ __device__ inline uint16_t bf16_rne(float x) {
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return uint16_t((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}
__host__ __device__ inline float bf16_widen(uint16_t b) {
    return __builtin_bit_cast(float, uint32_t(b) << 16);
}
// Device FP32 -> bf16 on the hardware converter (v_cvt_pk_bf16_f32, round to
// nearest even): the bits of bf16_rne for every non-NaN input.  Used where
// the values are finite by construction (sums and products of checked
// inputs); the input conversion kernels keep bf16_rne.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ inline uint32_t bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}
__device__ inline uint16_t bf16_hw(float x) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x)); }

// fmaxf for operands that are arithmetic results or lane copies of them,
// never a signalling NaN: the plain v_max_f32.  fmaxf puts a canonicalizing
// v_max x, x, x in front of every operand the compiler cannot trace to
// arithmetic (a DPP or permlane result); on quiet operands that is the
// identity, so the result is fmaxf's bit for bit.
__device__ inline float max_quiet(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// max_quiet(x, x of lane l ^ 8) within each row of 16 lanes: one v_max_f32
// with a DPP row rotation by 8 on its first operand.  The two wait states
// ahead of it are the DPP read-after-VALU-write hazard of the operand.
__device__ inline float max_ror8(float x) {
    float r;
    asm("s_nop 1\n\tv_max_f32_dpp %0, %1, %1 row_ror:8 row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(x));
    return r;
}

// max / sum of x over lanes l and l ^ 16 (l ^ 32): v_permlane16_swap
// (v_permlane32_swap) hands each lane the other half's value in the VALU,
// without the LDS round trip of a lane permute.  The swap returns the pair
// {x_l, x_(l^16)} in some order; max and + are commutative, so the result is
// that of fmaxf(x, __shfl_xor(x, 16)) (x + __shfl_xor(x, 16)) bit for bit.
// The max forms take quiet operands (see max_quiet).
__device__ inline float xor16_max(float x) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return max_quiet(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ inline float xor32_max(float x) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return max_quiet(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ inline float xor16_add(float x) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ inline float xor32_add(float x) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// LeakyReLU(x) = x >= 0 ? x : 0.2 x, as max(x, 0.2 x): for x >= 0 the rounded
// 0.2 x is at most x, for x < 0 it is above x, -0 and the infinities map to
// themselves and a NaN stays a NaN -- the same bits, one instruction fewer.
__device__ inline float leaky(float x) { return fmaxf(x, 0.2f * x); }
__device__ inline float elu(float x) { return x >= 0.0f ? x : expm1f(x); }


// Softmax weight e^x for x <= 0 as 2^(x log2 e) on the hardware base-2
// exponential (v_exp_f32): two instructions instead of the range-reduced
// expf.  exp_w(0) = 1 and exp_w(-inf) = 0 exactly; otherwise the relative
// error is about |x| 2^-24 (the rounded product) plus one ulp, below 2e-6
// wherever e^x is above 2^-30.
__device__ inline float exp_w(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// ELU for outputs that are stored as bf16: e^x - 1 from the hardware exp2
// (exp_w) where x < -1/8 (there |e^x - 1| > 0.11, so the exp2 error stays
// below 2e-6 of the result), and from the Taylor polynomial of e^x - 1 to
// x^4 / 24 above (remainder below x^5 / 120, under 2e-6 |x|).  The relative
// error is under 2e-6, against 2^-9 for the bf16 rounding that follows.
// Both pieces are evaluated and selected, with no branch per element (e^x of
// a positive x may overflow to inf there; it is not selected).
__device__ inline float elu_bf16(float x) {
    const float t = x * (1.0f + x * (0.5f + x * (1.0f / 6 + x * (1.0f / 24))));
    const float e = exp_w(x) - 1.0f;
    const float neg = x < -0.125f ? e : t;
    return x >= 0.0f ? x : neg;
}

// A buffer that no thread of the launch writes, seen through the constant
// address space: loads from it at wave-uniform addresses become scalar loads
// whatever stores the kernel makes elsewhere.
template <class T>
__device__ inline const __attribute__((address_space(4))) T* read_only(const T* p) {
    return (const __attribute__((address_space(4))) T*)(p);
}

// x from lane (lane ^ 1) and (lane ^ 2) within each group of four lanes (DPP
// quad permutations, no LDS round trip).
__device__ inline float quad_xor1(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
}
__device__ inline float quad_xor2(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false));
}

// Wave-local ordering of LDS traffic between lanes of one wavefront.
__device__ inline void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------- launches
// Every launcher returns hipSuccess or the launch error.

// schedule.hip
// deg[i] = row[i+1]-row[i], ids[i] = i, *maxdeg = max degree (atomicMax).
hipError_t launch_degrees_and_ids(const uint64_t* row, uint32_t* deg, uint32_t* ids, uint64_t n,
                                  uint32_t* maxdeg, hipStream_t s);
hipError_t radix_sort_by_degree(uint32_t* keys, uint32_t* vals, uint32_t* keys_alt,
                                uint32_t* vals_alt, uint32_t* tile_hist, uint64_t n, int passes,
                                void* scan_tmp, hipStream_t s, uint32_t** keys_out,
                                uint32_t** vals_out);
size_t radix_tile_hist_elems(uint64_t n);
size_t scan_tmp_bytes(uint64_t n);
hipError_t exclusive_scan_u32_to_u64(const uint32_t* in, uint64_t* out, uint64_t n, void* tmp,
                                     hipStream_t s);
hipError_t launch_permute_cols(const uint64_t* row, const uint32_t* col, const uint32_t* perm,
                               const uint64_t* prow, uint32_t* pcol, uint64_t n, uint64_t e,
                               hipStream_t s);
// Per-edge values ([e][K] floats) from original CSR order to degree-sorted order.
hipError_t launch_permute_edge_values(const uint64_t* row, const uint32_t* perm, const uint64_t* prow,
                                     const float* src, float* dst, uint64_t n, uint64_t e, int K, hipStream_t s);
hipError_t launch_neighbor_steps(const uint32_t* sorted_deg, uint64_t n, uint64_t* steps,
                                 hipStream_t s);
// Sorted node order: invperm (invperm[perm[k]] = k), ident (ident[k] = k) and
// rcol[q] = invperm[pcol[q]] (the sorted CSR's sources as sorted positions).
hipError_t launch_relabel(const uint32_t* perm, const uint32_t* pcol, uint32_t* invperm, uint32_t* ident,
                          uint32_t* rcol, uint64_t n, uint64_t e, hipStream_t s);
// dst row r = src row idx[r] (rows of `words` 4-byte words; strides in words;
// an index >= n_src gives a zero row).
hipError_t launch_gather_rows(const void* src, uint64_t src_stride_words, void* dst, uint64_t dst_stride_words,
                              const uint32_t* idx, uint64_t rows, uint64_t n_src, uint32_t words, hipStream_t s);
hipError_t launch_count_le(const uint32_t* sorted_deg, uint64_t n, const uint32_t* thresholds,
                           int count, uint64_t* positions, hipStream_t s);

// projection.hip
hipError_t launch_to_bf16(const float* x, uint16_t* y, uint64_t count, hipStream_t s);
hipError_t launch_widen_bf16(const uint16_t* x, float* y, uint64_t count, hipStream_t s);
// x [n][d] FP32 -> y [n][dp] bf16 with zero columns d..dp-1.
hipError_t launch_to_bf16_pad(const float* x, uint16_t* y, uint64_t n, int d, int dp, hipStream_t s);
// Z = X W with the L/R attention dots and the store of Z (FP32 or bf16).
// X is FP32 (x32 != null) or bf16 bits (xbf != null); W is FP32 values (for
// the bf16 path: bf16-rounded values).
hipError_t launch_projection(const float* x32, const uint16_t* xbf, const float* w, uint64_t n,
                             int in, int heads, int dim, const float* al, const float* ar,
                             float* z32, uint16_t* zbf, float* left, float* right, float* zscratch,
                             int zs, hipStream_t s);
// L/R only (aggregate-first front end): LR = X B_LR with B_LR = W a.
hipError_t launch_lr_reordered(const float* x32, const uint16_t* xbf, const float* blr,
                               uint64_t n, int in, int heads, float* left, float* right,
                               hipStream_t s);

// projection_mfma.hip: bf16 MFMA projection with the fused L/R block.
struct ProjArgs {
    const uint16_t* x;   // [n][xs] bf16 input, zero-padded to ksteps*16 columns
    const float* x32;    // or FP32 input [n][xs] (in valid columns, 16 floats of
                         // padding after the last row), rounded to bf16 in the kernel
    int in;              // valid input features (FP32 input)
    uint64_t n;
    int xs;              // row stride of x / x32 (elements)
    int ksteps;          // ceil(in / 16)
    const uint4* wpk;    // packed weights, pack_projection_weights() order
    int groups, head_blocks, nmb, width, heads;
    uint16_t* z;         // [n][zs] bf16 output
    int zs;              // row stride of z (elements, multiple of 8, >= width)
    float* left;         // [n][heads]
    float* right;        // [n][heads]
    uint64_t tiles;      // ceil(n / 32)
    bool r_in_z;         // also store R of head h as FP32 in z[row][r_off + 2h ..]
    int r_off;           // bf16 offset of R in the z row when r_in_z (one head: zs - 2)
    uint16_t* xout;      // FP32 input (or null): also store the rounded bf16 input
    int xouts;           // rows, features [0, 16 ksteps), at xout[row * xouts]
    bool r_from_z;       // bf16 8 x 32 or one head x 64: R = Z_bf16 . aR (the aggregation recomputes it)
    const float* ar;     // aR [256] when r_from_z
    const float* al;     // aL [heads * dim]: the W-stationary path forms L and R from FP32 Z
};
// R from the stored bf16 Z: the fast projection writes R = Z_bf16 . aR and
// the 8-head aggregation recomputes it from each gathered row instead of
// loading it (same FMA order, so both give the same bits).
bool r_from_z_supported(const ProjArgs& a);
int proj_blocks_per_group(int width);
// True when launch_projection_mfma takes the fast path for these arguments
// (one output group, 1..8 or 16 k steps, 0/1/2/8 head blocks); the FP32-input
// form requires it.
bool projection_fast_path(const ProjArgs& a);
// True when the fast path also takes FP32 input rows (rounding them itself).
bool projection_fp32_input(const ProjArgs& a);
void pack_projection_weights(const float* wq, const float* al, const float* ar, int in, int heads, int dim,
                             std::vector<uint16_t>& out, int& ksteps, int& groups, int& nmb);
hipError_t launch_projection_mfma(const ProjArgs& a, hipStream_t s, int cus);
void pack_lr_weights(const float* wq, const float* al, const float* ar, int in, int heads, int dim,
                     std::vector<uint16_t>& out, int& ksteps);

// FP32 projection on the MFMA units (projection_mfma.hip).
struct ProjF32Args {
    const float* x;      // [n][xs] FP32 input, xs == in
    uint64_t n;
    int in, xs;
    const float* wpk;    // pack_projection_f32() order
    int head_blocks, width, heads;
    float* z;            // [n][zs] FP32 output
    int zs;
    float* left;         // [n][heads]
    float* right;        // [n][heads]
    uint64_t tiles;      // ceil(n / 32)
};
bool projection_f32_supported(int in, int heads, int dim);
hipError_t launch_projection_f32(const ProjF32Args& a, hipStream_t s);
void pack_projection_f32(const float* w, const float* blr, int in, int heads, int dim, std::vector<float>& out);

// aggregate.hip
// Rows of at most this many edges share the sum form's 16-edge batches (four
// rows a batch).
constexpr uint32_t kShortDeg = 4;
struct RowBins {
    // Sorted positions [0, n) split by degree: [0, block_begin) one wave per
    // row, [block_begin, split_begin) one block per row, [split_begin, n)
    // several blocks per row.  [0, short_end): rows of at most kShortDeg edges.
    uint64_t block_begin = 0, split_begin = 0, n = 0, short_end = 0;
};
struct AggArgs {
    const uint64_t* prow;
    const uint32_t* pcol;
    const uint32_t* perm;
    const float* left;   // [n][K]
    const float* right;  // [n][K]
    const void* feat;    // Z [n][W] (TF) or X [n][D] (AF); FP32 or bf16
    bool feat_bf16;
    int fstride;         // row stride of feat in elements (>= W)
    bool r_in_feat;      // one head, bf16: R of row j is the FP32 at feat[j][fstride-2..fstride-1]
    int heads, dim;
    bool hidden;
    float* mx;       // [n][K]
    float* den;      // [n][K]
    float* out32;    // [n][W] or null
    uint16_t* outbf; // [n][W] or null
    uint64_t n, e;           // nodes and CSR entries (bounds of perm/prow values)
    bool r_from_z = false;   // bf16 8 x 32 or one head x 64: recompute R = Z_bf16 . aR from the gathered rows
    const float* ar = nullptr;
    // Output row of sorted position k (one-head kernel only): out_perm[k]
    // instead of the node index perm[k].  Null: the node index.
    const uint32_t* out_perm = nullptr;
    // Row stride of out32 (floats) where out_perm is set: k1_out_stride, so
    // that every scattered row is whole 128-byte lines.  0: W.
    int ostride = 0;
};
// The permuted column array carries kPcolPad zero entries past its e
// edges, so that kernels may load a whole batch of wave-uniform source ids
// at the end of the last row without a bounds test.
constexpr uint64_t kPcolPad = 64;
// FP32 feature buffers carry kF32Pad floats past their last row, so that the
// fused-convert projection may read a row's 16-feature tail unmasked.
constexpr uint64_t kF32Pad = 16;

// Split rows (sorted positions [split_begin, n)) cut into chunks of
// chunk_edges edges, heaviest rows first; built on the host from prow.
struct SplitTable {
    uint64_t chunks = 0;
    const uint32_t* chunk_k = nullptr;      // [chunks] sorted position of the row
    const uint32_t* chunk_first = nullptr;  // [chunks] first chunk of that row
    uint32_t chunk_edges = 256;
    float* mchunk = nullptr;                // [chunks][8] per-chunk max of R
    float* part = nullptr;                  // [chunks][W + 8] partial sums
    uint32_t* counter = nullptr;            // [chunks] arrival counters, zero between launches
};
hipError_t launch_aggregate_tf(const AggArgs& a, const RowBins& bins, const SplitTable& split,
                               hipStream_t s);
// Per-chunk maxima of R for split rows (heads 1, 2, 4 or 8).
hipError_t launch_split_prescan(const uint64_t* prow, const uint32_t* pcol, const float* right, int heads,
                                const SplitTable& t, uint64_t e, hipStream_t s);
// aggregate_fixed.hip: aggregation with fixture weights p (degree-sorted
// edge order, [e][K]) and fixture denominators ([n][K]); writes den and out32.
hipError_t launch_aggregate_fixed(const AggArgs& a, const float* p_sorted, const float* den_fixture,
                                  const RowBins& bins, const SplitTable& split, hipStream_t s);
// aggregate_k1.hip: one head, rows of at most 64 features.
bool aggregate_k1_supported(const AggArgs& a);
// Row stride (floats) of the one-head kernel's FP32 rows written to original
// node order: the kernel's widest row (G lanes x 16 bytes, 128 or 256 bytes),
// padded with zeros past the W classes.
int k1_out_stride(bool feat_bf16, int W);
hipError_t launch_aggregate_k1(const AggArgs& a, const RowBins& bins, const SplitTable& split,
                               hipStream_t s);
// aggregate_af.hip: aggregate-first bf16 layer (input rows <= 128, 32 features per head).
struct AfArgs {
    const uint64_t* prow;
    const uint32_t* pcol;
    const uint32_t* perm;
    const float* L;      // [n][heads] from the reordered contraction
    const float* R;      // [n][heads]
    const uint16_t* X;   // [n][128] bf16 layer input, zero-padded
    const uint4* wpk;    // projection weights in pack_projection_weights() order (one group)
    int nmb, ksteps;     // blocks per group and k steps of wpk
    const float* wq;     // [in][heads*32] bf16-rounded W as FP32 (split rows)
    int in, heads;
    bool hidden;
    float* mx;
    float* den;
    float* out32;
    uint16_t* outbf;
    uint64_t n, e;
    uint64_t rows;       // non-split rows: sorted positions [0, rows)
    uint64_t tiles;      // ceil(rows / 32)
    uint64_t chunks;
    const uint32_t* chunk_k;
    const uint32_t* chunk_first;
    uint32_t chunk_edges;
    const float* mchunk;
    float* part;         // [chunks][8*128 + 8]
    uint32_t* counter;
    bool b1;             // bf16(p X_j) W_h, exact max (faithful neighbour-step TFS)
    const float* fixp;   // fixed-p: fixture p in degree-sorted edge order [e][heads], else null
    const float* fixden; // fixed-p: fixture denominators [n][heads]
};
// aggregate_afsum.hip: aggregate-first in its sum form (U = sum p X, then U W),
// 8 heads x 32, D_in <= 112, over the XR gather table.
constexpr int kXRStride = 128;  // XR row: bf16 elements (256 bytes)
constexpr int kXRFeat = 112;    // feature slots; R_h as FP32 at bf16 offset kXRFeat + 2h
struct AfsArgs {
    const uint64_t* prow;
    const uint32_t* pcol;
    const uint32_t* perm;
    const float* L;      // [n][8]
    const float* R;      // [n][8] (per-chunk maxima of split rows; the scores when in > 112)
    const uint32_t* xr;  // XR as 4-byte words [n][64]: X, and R in words 56..63 when in <= 112
    const uint4* wpk;    // projection weights in pack_projection_weights() order (one group)
    int nmb, ksteps;     // blocks per group and k steps of wpk
    const float* wq;     // [in][8 dim] bf16-rounded W as FP32 (split rows)
    int in;
    int dim;             // head width: 32 or 64
    bool hidden;
    float* mx;
    float* den;
    float* out32;
    uint16_t* outbf;
    uint64_t n, e;
    uint64_t rows;       // non-split rows: sorted positions [0, rows)
    uint64_t short_rows; // of them [0, short_rows) have at most kShortDeg edges (bf16-stored outputs: shared batches)
    uint64_t row_lo;     // set by the launch: the positions [row_lo, rows) one kernel launch takes
    uint64_t chunks;
    const uint32_t* chunk_k;
    const uint32_t* chunk_first;
    uint32_t chunk_edges;
    float* mchunk;
    float* part;         // [chunks][8*128 + 24]
    uint32_t* counter;   // [chunks + 2]: row arrivals (at a row's first chunk), tiles taken, tile blocks done; zero between launches
    uint32_t tile_blocks;  // set by the launch: the blocks after the chunk blocks
};
// (n * 256 bytes must stay below 4 GiB: the gather uses 32-bit row offsets)
bool aggregate_afsum_supported(int in, int heads, int dim, uint64_t n);
hipError_t launch_aggregate_afsum(const AfsArgs& a, const SplitTable& t, hipStream_t s, int cus);
bool aggregate_af_supported(int in, int heads, int dim);
int af_input_stride();
hipError_t launch_aggregate_af(const AfArgs& a, hipStream_t s, int cus);
// aggregate_vec.hip: 16-byte vector path for 8 heads x (32 | 64).
bool aggregate_vec_supported(const AggArgs& a);
hipError_t launch_aggregate_vec(const AggArgs& a, const RowBins& bins, const SplitTable& split,
                                hipStream_t s);
// The 8 x 32 bf16 aggregation (R from Z, hidden, bf16 output rows) with the
// next layer's projection in its epilogue: a next layer of one head of at
// most 60 columns, whose Z rows are 64 bf16 with R as FP32 in the last four
// bytes.  Row buffers in sorted order (the row permutation is the identity).
// Non-split rows never store their output; split rows do (a.outbf), and the
// caller projects those rows afterwards with launch_projection_mfma.
struct NextProj {
    const uint4* wpk = nullptr;  // next layer's fragments, pack_projection_weights order (16 k steps, one group)
    int nmb = 0, head_blocks = 0;
    uint16_t* z = nullptr;       // [n][64]
    float* left = nullptr;       // [n]
    float* right = nullptr;      // [n]
    uint64_t tiles = 0;          // filled by the launcher
};
bool aggregate_vec_next_supported(const AggArgs& a, const NextProj& f);
hipError_t launch_aggregate_vec_next(const AggArgs& a, const RowBins& bins, const SplitTable& split, NextProj f,
                                     hipStream_t s);

}  // namespace gatgpu
