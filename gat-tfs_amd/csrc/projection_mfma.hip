// bf16 MFMA projection: Z = X W_all (bf16 in, FP32 accumulate, bf16 out)
// fused with the attention dots L = Z aL, R = Z aR.
//
// Reference: projection via cblas_gemm_bf16bf16f32 and lr_from_z
// (baseline/src/baseline_standard.cpp:3-20).  The dots are taken as one more
// MFMA output block against B_LR = W_bf16 a (the reordered contraction of
// lr_reordered, baseline_standard.cpp:29-43), with B_LR split into a bf16
// high part and a bf16 low part so the result carries ~16 mantissa bits of
// B_LR and FP32 accumulation -- the same value as the FP32 dot of the FP32 Z
// row with a up to rounding order.
//
// The product is computed transposed, Z^T = W^T X^T, on
// v_mfma_f32_32x32x16_bf16: A = 32 output features x 16 k of W^T (packed on
// the host in fragment order, read from LDS), B = 16 k x 32 graph rows of X^T
// (one 16-byte load per lane straight from the row-major X), D = 32 features
// x 32 rows, so each lane's accumulators hold 4 consecutive features of one
// graph row -- stored as 8-byte bf16 vectors without a transpose.
//
// Work split: one wave per 32-row tile, 8 waves per workgroup, persistent
// workgroups that copy their group's packed W into LDS once.  Output features
// are cut into groups of up to 8 blocks of 32; the last group also carries the
// L/R block.  Where W does not fit LDS (several groups, or one group of many
// k steps) the wide path keeps each tile's input in registers and streams W
// through LDS instead; for 8 heads x 64 the W-stationary path keeps W in
// registers and streams the tiles' input through LDS.
#include <utility>

#include "internal.hpp"

namespace gatgpu {
namespace {

typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kChunk = 16;  // X fragments held in registers at once (k = 256)

template <int NMB, bool LDS_A>
__global__ void __launch_bounds__(kThreads) k_proj_mfma(ProjArgs a) {
    extern __shared__ uint4 wlds[];
    const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
    const int g = blockIdx.y;
    const size_t gblocks = size_t(a.ksteps) * NMB * kWave;
    const uint4* wg = a.wpk + size_t(g) * gblocks;
    if constexpr (LDS_A) {
        for (size_t q = threadIdx.x; q < gblocks; q += kThreads) wlds[q] = wg[q];
        __syncthreads();
    }
    const uint4* wsrc = LDS_A ? wlds : wg;
    const int head_blocks = a.head_blocks - 8 * g < 8 ? a.head_blocks - 8 * g : 8;
    const bool has_lr = g == a.groups - 1;
    const int nblk = head_blocks + (has_lr ? 1 : 0);
    const int half = l / 32, col = l % 32;
    for (uint64_t tile = uint64_t(blockIdx.x) * kWaves + w; tile < a.tiles;
         tile += uint64_t(gridDim.x) * kWaves) {
        const uint64_t row = tile * 32 + col;
        const bool row_ok = row < a.n;
        f32x16 acc[NMB];
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mb][r] = 0.0f;
        const uint16_t* xrow = a.x + row * a.xs + 8 * half;
        for (int k0 = 0; k0 < a.ksteps; k0 += kChunk) {
            uint4 xf[kChunk];
#pragma unroll
            for (int q = 0; q < kChunk; ++q)
                xf[q] = (row_ok && k0 + q < a.ksteps) ? *reinterpret_cast<const uint4*>(xrow + (k0 + q) * 16)
                                                      : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int q = 0; q < kChunk; ++q) {
                if (k0 + q < a.ksteps) {
                    const bf16x8 b = __builtin_bit_cast(bf16x8, xf[q]);
                    const uint4* wk = wsrc + size_t(k0 + q) * NMB * kWave + l;
#pragma unroll
                    for (int mb = 0; mb < NMB; ++mb) {
                        if (mb < nblk) {
                            const bf16x8 av = __builtin_bit_cast(bf16x8, wk[mb * kWave]);
                            acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, b, acc[mb], 0, 0, 0);
                        }
                    }
                }
            }
        }
        if (!row_ok) continue;
        // Z: lane (half, col) holds features 32*gb + 16*half + 4*gq + {0..3} of row
        // (permuted packing).
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) {
            if (mb >= head_blocks) continue;
            const int gb = 8 * g + mb;
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                const int f0 = gb * 32 + 16 * half + 4 * gq;
                if (f0 >= a.width) continue;
                const uint32_t w0 = bf16x2(acc[mb][4 * gq], acc[mb][4 * gq + 1]);
                const uint32_t w1 = bf16x2(acc[mb][4 * gq + 2], acc[mb][4 * gq + 3]);
                *reinterpret_cast<uint2*>(a.z + row * a.zs + f0) = make_uint2(w0, w1);
            }
        }
        if (has_lr) {
            // LR block columns: [0,8) L hi, [8,16) R hi, [16,24) L lo, [24,32) R lo;
            // lane half h4 holds heads 4*h4 + {0..3} of each quarter in regs
            // {0..3}, {4..7}, {8..11}, {12..15}.
#pragma unroll
            for (int mb = 0; mb < NMB; ++mb) {
                if (mb != head_blocks) continue;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int h = 4 * half + q;
                    if (h < a.heads) {
                        const float rv = acc[mb][4 + q] + acc[mb][12 + q];
                        a.left[row * a.heads + h] = acc[mb][q] + acc[mb][8 + q];
                        a.right[row * a.heads + h] = rv;
                        if (a.r_in_z) *reinterpret_cast<float*>(a.z + row * a.zs + a.r_off + 2 * h) = rv;
                    }
                }
            }
        }
    }
}

// Fast path for one output group (head blocks HB <= 8 plus the L/R block)
// and KS <= 16 k steps, both compile-time: the W^T fragments of the group
// sit in LDS in [ks][block] order, each k step reads the HB + 1 fragments and
// issues HB + 1 independent MFMAs (no dependent chain between consecutive
// MFMAs, no branches between them), and the tile's X fragments are loaded
// unconditionally (rows past n re-read row n - 1 and are not stored).
// Head blocks use the permuted packing (pack_projection_weights): lane
// (half, col) ends with features 32 mb + 16 half + {0..15} of row col, so
// Z leaves as two 16-byte stores per block, or, in FULL layers, as whole
// 128-byte lines after a transpose inside each lane quad.  FULL: 0 any shape;
// 1 a layer of 8 heads x 32 with every store unconditional; 2 the same with
// R = Z_bf16 aR (what the aggregation recomputes from the gathered row).
// L/R-only launches (HB = 0: the aggregate-first front end, a streaming pass
// with KS KB of W) take a full grid, one tile per wave, and W is cheap to
// refetch; their LDS request holds them to two blocks (16 waves) per CU.
// With 7 k steps they write the gather-table rows as whole lines, after the
// same in-quad transpose (0.329 -> 0.309 ms on the 2.45M-row 100-input layer).
template <int KS, int HB, bool F32IN, int FULL>
__global__ void __launch_bounds__(kThreads) k_proj_fast(ProjArgs a) {
    static_assert(!FULL || HB == 8, "FULL layers are 8 heads x 32");
    constexpr bool ONE = HB == 0;  // one tile per wave, nothing requested ahead
    constexpr int NB = HB + 1;
    extern __shared__ uint4 wlds[];
    for (int q = threadIdx.x; q < KS * NB * kWave; q += kThreads) {
        const int lane = q % kWave, b = (q / kWave) % NB, ks = q / (kWave * NB);
        wlds[q] = a.wpk[(size_t(ks) * a.nmb + b) * kWave + lane];
    }
    // FULL layers keep aR (256 floats) after the fragments for R from the stored Z.
    float* arl = reinterpret_cast<float*>(wlds + KS * NB * kWave);
    if (FULL)
        for (int q = threadIdx.x; q < 256; q += kThreads) arl[q] = a.ar ? a.ar[q] : 0.0f;
    __syncthreads();
    const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
    const int half = l / 32, col = l % 32;
    // Raw input fragments of the tile: 16 bytes of bf16 per k step, or 32
    // bytes of FP32 (rounded to bf16 when used, so a load is never waited on
    // at issue).  Rolling two-part pipeline over the wave's tiles: each part
    // (k steps 0..KA-1, KA..KS-1) of tile t+1 is requested as soon as tile t
    // has multiplied that part, in the same registers.
    constexpr int KA = (KS + 1) / 2;
    constexpr int RW = F32IN ? 2 : 1;  // 16-byte loads per k step
    uint4 raw[KS][RW];
    auto load_ks = [&](uint64_t tile, int ks) {
        const uint64_t r = tile * 32 + col;
        const uint64_t rc = r < a.n ? r : a.n - 1;
        if constexpr (F32IN) {
            const float* p = a.x32 + rc * a.xs + 16 * ks + 8 * half;
            raw[ks][0] = *reinterpret_cast<const uint4*>(p);
            raw[ks][RW - 1] = *reinterpret_cast<const uint4*>(p + 4);
        } else {
            raw[ks][0] = *reinterpret_cast<const uint4*>(a.x + rc * a.xs + 16 * ks + 8 * half);
        }
    };
    // B operand of k step ks.  FP32 input (stride xs floats, `in` valid
    // features): rounded to bf16 here -- the convert stage, common.cpp:80-93,
    // fused; features >= in are zeroed.  The buffer carries 16 floats of
    // padding, so the last row's tail loads stay inside it.
    auto operand = [&](int ks) -> bf16x8 {
        if constexpr (F32IN) {
            const int f0 = 16 * ks + 8 * half;
            const float e[8] = {__builtin_bit_cast(float, raw[ks][0].x), __builtin_bit_cast(float, raw[ks][0].y),
                                __builtin_bit_cast(float, raw[ks][0].z), __builtin_bit_cast(float, raw[ks][0].w),
                                __builtin_bit_cast(float, raw[ks][RW - 1].x), __builtin_bit_cast(float, raw[ks][RW - 1].y),
                                __builtin_bit_cast(float, raw[ks][RW - 1].z), __builtin_bit_cast(float, raw[ks][RW - 1].w)};
            uint32_t w4[4];
#pragma unroll
            for (int x = 0; x < 4; ++x)
                w4[x] = bf16x2(f0 + 2 * x < a.in ? e[2 * x] : 0.0f, f0 + 2 * x + 1 < a.in ? e[2 * x + 1] : 0.0f);
            return __builtin_bit_cast(bf16x8, make_uint4(w4[0], w4[1], w4[2], w4[3]));
        } else {
            return __builtin_bit_cast(bf16x8, raw[ks][0]);
        }
    };
    const uint64_t stride = uint64_t(gridDim.x) * kWaves;
    uint64_t tile = uint64_t(blockIdx.x) * kWaves + w;
    const uint64_t last = a.tiles - 1;
    {
        const uint64_t t0 = tile < a.tiles ? tile : last;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) load_ks(t0, ks);
        // The first tile waits for all of its input here, so that the wait in
        // the loop only has the loop's own issue order to follow (a merge with
        // the prologue's order would make it wait for every store as well).
        // A single tile waits here too: waits per k step, between which the
        // converted input rows are stored, measured slower.
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    for (; tile < a.tiles; tile += stride) {
        const uint64_t row = tile * 32 + col;
        const uint64_t next = tile + stride < a.tiles ? tile + stride : last;
        f32x16 acc[NB];
#pragma unroll
        for (int mb = 0; mb < NB; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mb][r] = 0.0f;
        const uint64_t rs = row < a.n ? row : a.n - 1;  // lanes past n repeat row n - 1
        // XRL: the aggregate-first front end writing 7 k steps of rounded input
        // and R into 256-byte gather-table rows.  Lane (half, col) holds 16
        // bytes per k step, bytes 32 (ks % 4) + 16 half of line ks / 4; R of
        // its 4 heads is the fourth slot of line 1.  Each line leaves whole:
        // a 4 x 4 transpose of the slots inside the lane quad (two DPP
        // exchange stages) gives lane c slot c of the quad's 4 rows.
        constexpr bool XRL_OK = ONE && F32IN && KS == 7;
        const bool xrl = XRL_OK && a.xout && a.r_in_z && a.xout == a.z && a.xouts == kXRStride &&
                         a.zs == kXRStride && a.r_off == kXRFeat && a.heads == 8;
        uint4 xo[XRL_OK ? KS : 1];
        auto line_out = [&](const uint4 (&slot)[4], int line) {
            const int c = l & 3;
            uint32_t S[4][4], U[4][4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                S[p][0] = slot[p].x;
                S[p][1] = slot[p].y;
                S[p][2] = slot[p].z;
                S[p][3] = slot[p].w;
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
                    S[p][v] = (c & 2) == (p & 2) ? U[p][v] : o;  // quad_perm [2, 3, 0, 1]
                }
            // S[j]: slot c (bytes 32 c + 16 half of the line) of quad row j;
            // rows past n repeat row n - 1, as that row's lane did.
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint64_t rj = tile * 32 + uint64_t((col & ~3) + j);
                const uint64_t rsj = rj < a.n ? rj : a.n - 1;
                *reinterpret_cast<uint4*>(a.xout + rsj * kXRStride + 64 * line + 16 * c + 8 * half) =
                    make_uint4(S[j][0], S[j][1], S[j][2], S[j][3]);
            }
        };
        auto kstep = [&](int ks) {
            const bf16x8 b = operand(ks);
            if constexpr (F32IN) {
                if constexpr (XRL_OK) {
                    if (xrl) xo[ks] = __builtin_bit_cast(uint4, b);
                    else if (a.xout)
                        *reinterpret_cast<uint4*>(a.xout + rs * a.xouts + 16 * ks + 8 * half) =
                            __builtin_bit_cast(uint4, b);
                } else if (a.xout) {
                    *reinterpret_cast<uint4*>(a.xout + rs * a.xouts + 16 * ks + 8 * half) = __builtin_bit_cast(uint4, b);
                }
            }
            const uint4* wk = wlds + size_t(ks) * NB * kWave + l;
#pragma unroll
            for (int mb = 0; mb < NB; ++mb)
                acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wk[mb * kWave]), b,
                                                                  acc[mb], 0, 0, 0);
            // Keep each k step's fragment reads inside the step: hoisting all of
            // them ahead of the MFMAs would need KS * NB * 4 registers.
            __builtin_amdgcn_sched_barrier(0);
        };
        // Part A of this tile, then part A of the next tile requested into the
        // freed registers; part B of this tile, part B of the next tile, then
        // the stores.  Every load is unconditional, so each wait is exact.
#pragma unroll
        for (int ks = 0; ks < KA; ++ks) kstep(ks);
        if constexpr (XRL_OK) {
            if (xrl) {
                const uint4 l0[4] = {xo[0], xo[1], xo[2], xo[3]};
                line_out(l0, 0);
            }
        }
        if constexpr (!ONE) {
#pragma unroll
            for (int ks = 0; ks < KA; ++ks) load_ks(next, ks);
        }
#pragma unroll
        for (int ks = KA; ks < KS; ++ks) kstep(ks);
        // Part B of the next tile ahead of this tile's stores: the in-order
        // counter then lets the next tile's waits pass without these stores.
        if constexpr (!ONE) {
#pragma unroll
            for (int ks = KA; ks < KS; ++ks) load_ks(next, ks);
        }
        // A lane past n computed row n - 1 from the same input, so it stores
        // that row's own values to it (rs): no branch around the stores, which
        // keeps the wait counts of the next tile's loads exact.
        // FULL: all 8 heads and 32 HB features present (8 x 32): no per-store
        // bounds tests either.
        const bool full = FULL;
        float rz4[4] = {};  // R from the stored (bf16) Z of the lane's 4 heads (4 half + q)
        if constexpr (FULL != 0) {
            // Z rows leave as whole 128-byte lines.  Lane (half, col) holds 32
            // bytes of row col per head block: bytes 64 mb + 32 half + {0..31}.
            // Line k of the row is blocks 2k and 2k + 1, so the lane quad
            // (rows 4a .. 4a + 3, both halves) holds 4 rows x 8 pieces of 16
            // bytes of it, 4 pieces per lane (slot p: block 2k + p / 2, piece p
            // % 2).  A 4 x 4 transpose inside the quad (two DPP exchange stages,
            // lane c taking slot p from quad lane c ^ 1, then c ^ 2) leaves lane
            // c with slot c of the 4 rows, so store j writes row 4a + j whole
            // from the 8 lanes of quad a: 8 lines per instruction where the
            // direct stores wrote 16-byte pieces of 32 rows (0.565 -> 0.555 ms on
            // the 2.45M-row 256 -> 8 x 32 layer).
            const int c = l & 3;
#pragma unroll
            for (int k = 0; k < HB / 2; ++k) {
                uint32_t S[4][4];
#pragma unroll
                for (int m2 = 0; m2 < 2; ++m2) {
                    const int mb = 2 * k + m2;
                    uint32_t zp[8];  // the stored bf16 pairs
#pragma unroll
                    for (int x = 0; x < 8; ++x) zp[x] = bf16x2(acc[mb][2 * x], acc[mb][2 * x + 1]);
#pragma unroll
                    for (int x = 0; x < 8; ++x) S[2 * m2 + x / 4][x % 4] = zp[x];
                    if constexpr (FULL == 2) {
                        // R = Z_bf16 . aR with the summation the aggregation kernel
                        // uses: an FMA chain over each 8 features, then
                        // (s0 + s1) + (s2 + s3).
                        float s8[2];
#pragma unroll
                        for (int q8 = 0; q8 < 2; ++q8) {
                            float t = 0.0f;
#pragma unroll
                            for (int x = 0; x < 8; ++x) {
                                const uint32_t pr = zp[4 * q8 + x / 2];
                                const float zv = __builtin_bit_cast(float, (x & 1) ? (pr & 0xffff0000u) : (pr << 16));
                                t = __builtin_fmaf(zv, arl[32 * mb + 16 * half + 8 * q8 + x], t);
                            }
                            s8[q8] = t;
                        }
                        const float part = s8[0] + s8[1];
                        const float r = part + __shfl_xor(part, 32);
                        rz4[mb & 3] = (mb >> 2) == half ? r : rz4[mb & 3];
                    }
                }
                uint32_t U[4][4], T[4][4];
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
                // T[j]: slot c (line bytes 64 (c / 2) + 32 half + 16 (c % 2)) of
                // quad row j; rows past n repeat row n - 1, as that row's lane did.
                const int off = 64 * k + 32 * (c / 2) + 16 * half + 8 * (c % 2);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint64_t rj = tile * 32 + uint64_t((col & ~3) + j);
                    const uint64_t rsj = rj < a.n ? rj : a.n - 1;
                    *reinterpret_cast<uint4*>(a.z + rsj * a.zs + off) = make_uint4(T[j][0], T[j][1], T[j][2], T[j][3]);
                }
            }
        } else {
#pragma unroll
            for (int mb = 0; mb < HB; ++mb) {
#pragma unroll
                for (int q8 = 0; q8 < 2; ++q8) {
                    const int f0 = 32 * mb + 16 * half + 8 * q8;
                    if (f0 >= a.width) continue;
                    uint32_t w4[4];
#pragma unroll
                    for (int x = 0; x < 4; ++x) w4[x] = bf16x2(acc[mb][8 * q8 + 2 * x], acc[mb][8 * q8 + 2 * x + 1]);
                    *reinterpret_cast<uint4*>(a.z + rs * a.zs + f0) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
                }
            }
        }
        // L/R block: lane half h4 holds heads 4 h4 + {0..3} of each quarter
        // (L hi, R hi, L lo, R lo) in registers {0..3}, {4..7}, {8..11}, {12..15}.
        if (full || a.heads == 8) {
            // 8 heads: the lane's 4 consecutive L, R values leave as 16-byte
            // vectors (and R's 16 bytes in the Z row tail).
            const float4 lv = make_float4(acc[HB][0] + acc[HB][8], acc[HB][1] + acc[HB][9], acc[HB][2] + acc[HB][10],
                                          acc[HB][3] + acc[HB][11]);
            const float4 rv = make_float4(acc[HB][4] + acc[HB][12], acc[HB][5] + acc[HB][13], acc[HB][6] + acc[HB][14],
                                          acc[HB][7] + acc[HB][15]);
            *reinterpret_cast<float4*>(a.left + rs * 8 + 4 * half) = lv;
            if constexpr (FULL) {
                // Always one R store per lane (the lane's 4 heads), R from the
                // stored Z or from the L/R block: with no store under a branch
                // the waits for the next tile's loads stay exact.
                *reinterpret_cast<float4*>(a.right + rs * 8 + 4 * half) =
                    FULL == 2 ? make_float4(rz4[0], rz4[1], rz4[2], rz4[3]) : rv;
            } else {
                *reinterpret_cast<float4*>(a.right + rs * 8 + 4 * half) = rv;
                if constexpr (XRL_OK) {
                    if (xrl) {
                        const uint4 l1[4] = {xo[4], xo[5], xo[6],
                                             make_uint4(__float_as_uint(rv.x), __float_as_uint(rv.y),
                                                        __float_as_uint(rv.z), __float_as_uint(rv.w))};
                        line_out(l1, 1);
                    } else if (a.r_in_z) {
                        *reinterpret_cast<float4*>(a.z + rs * a.zs + a.r_off + 8 * half) = rv;
                    }
                } else if (a.r_in_z) {
                    *reinterpret_cast<float4*>(a.z + rs * a.zs + a.r_off + 8 * half) = rv;
                }
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int h = 4 * half + q;
                if (h < a.heads) {
                    const float rv = acc[HB][4 + q] + acc[HB][12 + q];
                    a.left[rs * a.heads + h] = acc[HB][q] + acc[HB][8 + q];
                    a.right[rs * a.heads + h] = rv;
                    if (a.r_in_z) *reinterpret_cast<float*>(a.z + rs * a.zs + a.r_off + 2 * h) = rv;
                }
            }
        }
    }
}

// Wide path: several output groups (more than 8 head blocks), or a group
// whose W fragments exceed LDS (e.g. 512 -> 8 x 64: 32 k steps x 17 blocks).
// Each wave keeps the whole input of its 32-row tile in registers (KS B
// fragments) and the block streams W^T one 32-feature output block at a time
// (KS fragments, KS KB) through two LDS slots its waves share: X is read from
// HBM once, each output block's fragments once per block from L2, and every
// output block (head blocks, then the L/R block) leaves straight from the
// accumulators.  The MFMA chain per block runs k steps in the order of the
// other paths, so Z and L/R carry the same bits.
//
// The slots are filled by direct global -> LDS loads (global_load_lds_dwordx4,
// one 1 KB k step per wave instruction, k steps split over the waves), issued
// for block ob + 1 while block ob multiplies: no registers hold fragments in
// transit.  The two slots are distinct LDS arrays and the block loop is
// unrolled by two, so the compiler can see that the loads into one slot do not
// alias the reads of the other and leaves them in flight.  Four waves per
// block, two blocks per CU (2 waves per SIMD at 32 k steps: the tile's input
// alone is 128 registers).  Measured on the 100.6M-edge R-MAT graph's
// 512 -> 8 x 64 projection: 2.73 ms with the fragments staged through
// registers, 2.63 ms with the direct loads; six-wave blocks at three waves
// per SIMD (168 registers, two-step read-ahead, spilled addresses) 3.04 ms.
//
// The step barrier orders LDS only (each wave first waits for its own loads
// into the next slot), so Z stores stay in flight across it; where every head
// block is full (DEL) a block's Z stores are also issued one step late,
// behind the next block's fragment loads, so the wait for those loads does
// not wait for them.  The one-head 512 -> 64 projection went 0.977 -> 0.94 ms;
// the 8 x 64 one is unchanged by both (and by fragments staged through
// registers after the MFMAs, whose fragment reads the compiler then waits for
// in order where it waits for every LDS-DMA load: 2.81 ms).
constexpr int kWideThreads = 256;  // the FP32 projection's block (k_proj_f32)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kWideWaves = kWideThreads / kWave;
constexpr int kWideBW = 4;  // waves per block of the bf16 wide path
typedef __attribute__((address_space(3))) void* lds_ptr;

template <int KS, bool F32IN, bool RZ, bool DEL>
__global__ void __launch_bounds__(kWideBW * kWave) __attribute__((amdgpu_waves_per_eu(2))) k_proj_wide(ProjArgs a) {
    __shared__ __attribute__((aligned(16))) u32x4 slot0[KS * kWave];
    __shared__ __attribute__((aligned(16))) u32x4 slot1[KS * kWave];
    // aR of the one head of 64 (RZ), read by the epilogue from LDS: a global
    // load there would sit behind the delayed Z stores in the in-order counter.
    __shared__ float arl[RZ ? 64 : 1];
    if constexpr (RZ)
        for (int q = threadIdx.x; q < 64; q += kWideBW * kWave) arl[q] = a.ar[q];
    const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave), l = threadIdx.x % kWave;
    const int half = l / 32, col = l % 32;
    const uint64_t row = (uint64_t(blockIdx.x) * kWideBW + w) * 32 + col;
    // Lanes past n recompute row n - 1 and store its own values to it.
    const uint64_t rs = row < a.n ? row : a.n - 1;
    bf16x8 xr[KS];
    if constexpr (F32IN) {
        // FP32 rows rounded to bf16 here (the convert stage, common.cpp:80-93,
        // fused); features >= in are zeroed, and the buffer's 16 floats of
        // padding keep the last row's tail loads inside it.
        const float* p = a.x32 + rs * a.xs + 8 * half;
        uint4 raw[KS][2];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            raw[ks][0] = *reinterpret_cast<const uint4*>(p + 16 * ks);
            raw[ks][1] = *reinterpret_cast<const uint4*>(p + 16 * ks + 4);
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int f0 = 16 * ks + 8 * half;
            const uint32_t e[8] = {raw[ks][0].x, raw[ks][0].y, raw[ks][0].z, raw[ks][0].w,
                                   raw[ks][1].x, raw[ks][1].y, raw[ks][1].z, raw[ks][1].w};
            uint32_t w4[4];
#pragma unroll
            for (int x = 0; x < 4; ++x)
                w4[x] = bf16x2(f0 + 2 * x < a.in ? __builtin_bit_cast(float, e[2 * x]) : 0.0f,
                               f0 + 2 * x + 1 < a.in ? __builtin_bit_cast(float, e[2 * x + 1]) : 0.0f);
            xr[ks] = __builtin_bit_cast(bf16x8, make_uint4(w4[0], w4[1], w4[2], w4[3]));
            if (a.xout)  // the rounded rows also leave the kernel (lanes past n rewrite row n - 1)
                *reinterpret_cast<uint4*>(a.xout + rs * a.xouts + f0) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
    } else {
        const uint16_t* p = a.x + rs * a.xs + 8 * half;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) xr[ks] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p + 16 * ks));
    }
    // Output block ob: head block ob (group ob / 8, block ob % 8), then the
    // L/R block, which sits after the head blocks of the last group.
    const int nob = a.head_blocks + 1;
    const int last_g = a.groups - 1;
    // Fragments of output block ob into dst: k step ks (64 lanes x 16 bytes)
    // is one wave instruction, k steps w, w + kWideBW, ... for wave w.
    // The address is a wave-uniform base plus the lane's 32-bit offset.
    const unsigned char* wbase = reinterpret_cast<const unsigned char*>(a.wpk);
    const uint32_t loff = uint32_t(l) * uint32_t(sizeof(u32x4));
    auto dma = [&](int ob, u32x4* dst) {
        const int g = ob < a.head_blocks ? ob / 8 : last_g;
        const int b = ob < a.head_blocks ? ob % 8 : a.head_blocks - 8 * last_g;
        const size_t boff = (size_t(g) * KS * a.nmb + b) * kWave * sizeof(u32x4);
        for (int ks = w; ks < KS; ks += kWideBW)
            __builtin_amdgcn_global_load_lds(wbase + (boff + size_t(ks) * a.nmb * kWave * sizeof(u32x4)) + loff,
                                             (lds_ptr)(dst + ks * kWave), 16, 0, 0);
    };
    // One head of 64 with r_from_z: R = Z_bf16 . aR in the order the one-head
    // aggregation recomputes it from a gathered row -- an FMA chain over each
    // 8 features (p0..p7), then ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)).
    // Lane half 0 holds p0, p1 (block 0) and p4, p5 (block 1); half 1 the others.
    float rlo = 0.0f, rhi = 0.0f;  // pair sums of head blocks 0 and 1
    // DEL (every head block full): block ob's Z pieces leave at the top of
    // step ob + 1, after block ob + 2's fragment loads are issued, so the wait
    // for those loads at the end of step ob + 1 (vmcnt(2)) leaves the two
    // stores in flight instead of waiting for them.
    uint32_t pend[2][4] = {};
    dma(0, slot0);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the tile's input and block 0's fragments
    __syncthreads();
    // Block ob from rd while block ob + 1's fragments land in wr.  Each wave
    // waits for its own loads into wr (and its previous stores) after the
    // MFMAs and before this block's stores, so the barrier then publishes wr.
    auto step = [&](int ob, const u32x4* rd, u32x4* wr) {
        if (ob + 1 < nob) dma(ob + 1, wr);
        if constexpr (DEL) {
            if (ob > 0) {
                // Each store writes block ob - 1's 64 bytes of 16 rows: in the
                // lane quad (rows 4 a .. 4 a + 3), store j takes rows 4 a + 2 j
                // and 4 a + 2 j + 1, lane c writing piece 2 half + c % 2 of row
                // 4 a + 2 j + c / 2, read from quad lane 2 j + c / 2 by DPP.
                const int c = l & 3;
                const uint64_t tbase = (uint64_t(blockIdx.x) * kWideBW + w) * 32;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    uint32_t T[4];
#pragma unroll
                    for (int x = 0; x < 4; ++x) {
                        const uint32_t a0 = uint32_t(j ? __builtin_amdgcn_mov_dpp(int(pend[0][x]), 0xFA, 0xF, 0xF, false)
                                                       : __builtin_amdgcn_mov_dpp(int(pend[0][x]), 0x50, 0xF, 0xF, false));
                        const uint32_t a1 = uint32_t(j ? __builtin_amdgcn_mov_dpp(int(pend[1][x]), 0xFA, 0xF, 0xF, false)
                                                       : __builtin_amdgcn_mov_dpp(int(pend[1][x]), 0x50, 0xF, 0xF, false));
                        T[x] = (c & 1) ? a1 : a0;
                    }
                    const uint64_t rj = tbase + uint64_t((col & ~3) + 2 * j + (c >> 1));
                    const uint64_t rsj = rj < a.n ? rj : a.n - 1;
                    *reinterpret_cast<uint4*>(a.z + rsj * a.zs + 32 * (ob - 1) + 16 * half + 8 * (c & 1)) =
                        make_uint4(T[0], T[1], T[2], T[3]);
                }
            }
        }
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
        const u32x4* wk = rd + l;
        // Fragments read four k steps ahead of their MFMA.
        constexpr int kAhead = KS < 4 ? KS : 4;
        u32x4 fr[kAhead];
#pragma unroll
        for (int ks = 0; ks < kAhead; ++ks) fr[ks] = wk[ks * kWave];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const u32x4 av = fr[ks % kAhead];
            if (ks + kAhead < KS) fr[ks % kAhead] = wk[(ks + kAhead) * kWave];
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av), xr[ks], acc, 0, 0, 0);
        }
        // Keep that order in the schedule: kAhead LDS reads, then one MFMA and
        // one read per k step.
        __builtin_amdgcn_sched_group_barrier(0x100, kAhead, 0);
#pragma unroll
        for (int ks = 0; ks + kAhead < KS; ++ks) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, kAhead, 0);
        if (DEL && ob > 0) __builtin_amdgcn_s_waitcnt(0x0F72);  // vmcnt(2): the loads into wr, not the 2 stores after them
        else __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads into wr
        __builtin_amdgcn_sched_barrier(0);
        if (ob < a.head_blocks) {
            // Permuted packing: lane (half, col) holds features 32 ob + 16 half + {0..15}.
            uint32_t w4[2][4];
#pragma unroll
            for (int q8 = 0; q8 < 2; ++q8)
#pragma unroll
                for (int x = 0; x < 4; ++x) w4[q8][x] = bf16x2(acc[8 * q8 + 2 * x], acc[8 * q8 + 2 * x + 1]);
            if (RZ) {
                // aR is read before this block's stores are issued: a load
                // behind them would wait for them (one in-order counter).
#pragma unroll
                for (int q8 = 0; q8 < 2; ++q8) {
                    const int f0 = 32 * ob + 16 * half + 8 * q8;
                    if (f0 < a.width) {
                        float t = 0.0f;
#pragma unroll
                        for (int x = 0; x < 4; ++x) {
                            t = __builtin_fmaf(__builtin_bit_cast(float, w4[q8][x] << 16), arl[f0 + 2 * x], t);
                            t = __builtin_fmaf(__builtin_bit_cast(float, w4[q8][x] & 0xffff0000u), arl[f0 + 2 * x + 1],
                                               t);
                        }
                        if (ob == 0) rlo = q8 == 0 ? t : rlo + t;
                        else rhi = q8 == 0 ? t : rhi + t;
                    }
                }
            }
            if constexpr (DEL) {
#pragma unroll
                for (int q8 = 0; q8 < 2; ++q8)
#pragma unroll
                    for (int x = 0; x < 4; ++x) pend[q8][x] = w4[q8][x];
            } else {
#pragma unroll
                for (int q8 = 0; q8 < 2; ++q8) {
                    const int f0 = 32 * ob + 16 * half + 8 * q8;
                    if (f0 < a.width)
                        *reinterpret_cast<uint4*>(a.z + rs * a.zs + f0) =
                            make_uint4(w4[q8][0], w4[q8][1], w4[q8][2], w4[q8][3]);
                }
            }
        } else {
            float rz = 0.0f;
            if (RZ) {
                const float lo = rlo + __shfl_xor(rlo, 32);
                const float hi = rhi + __shfl_xor(rhi, 32);
                rz = lo + hi;
            }
            // L/R block: lane half h4 holds heads 4 h4 + {0..3} of each quarter
            // (L hi, R hi, L lo, R lo) in registers {0..3}, {4..7}, {8..11}, {12..15}.
            if (a.heads == 8 && !a.r_in_z) {  // 16-byte vectors of the lane's 4 heads
                *reinterpret_cast<float4*>(a.left + rs * 8 + 4 * half) =
                    make_float4(acc[0] + acc[8], acc[1] + acc[9], acc[2] + acc[10], acc[3] + acc[11]);
                *reinterpret_cast<float4*>(a.right + rs * 8 + 4 * half) =
                    make_float4(acc[4] + acc[12], acc[5] + acc[13], acc[6] + acc[14], acc[7] + acc[15]);
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int h = 4 * half + q;
                    if (h < a.heads) {
                        const float rv = RZ ? rz : acc[4 + q] + acc[12 + q];
                        a.left[rs * a.heads + h] = acc[q] + acc[8 + q];
                        a.right[rs * a.heads + h] = rv;
                        if (a.r_in_z) *reinterpret_cast<float*>(a.z + rs * a.zs + a.r_off + 2 * h) = rv;
                    }
                }
            }
        }
        // The slots are LDS only, and each wave has waited for its own loads
        // into wr: an LDS-scoped barrier, which leaves the Z stores in flight.
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    for (int ob = 0; ob < nob; ob += 2) {
        step(ob, slot0, slot1);
        if (ob + 1 < nob) step(ob + 1, slot1, slot0);
    }
}

template <int KS, bool F32IN>
hipError_t launch_wide_io(const ProjArgs& a, hipStream_t s) {
    const uint64_t blocks = (a.tiles + kWideBW - 1) / kWideBW;
    if (blocks < 1 || blocks > 0x7fffffffu) return hipErrorInvalidValue;
    const bool del = a.width % 32 == 0;  // every head block full: its stores are unconditional
    if (a.r_from_z) {
        if (del) k_proj_wide<KS, F32IN, true, true><<<dim3(uint32_t(blocks)), kWideBW * kWave, 0, s>>>(a);
        else k_proj_wide<KS, F32IN, true, false><<<dim3(uint32_t(blocks)), kWideBW * kWave, 0, s>>>(a);
    } else {
        if (del) k_proj_wide<KS, F32IN, false, true><<<dim3(uint32_t(blocks)), kWideBW * kWave, 0, s>>>(a);
        else k_proj_wide<KS, F32IN, false, false><<<dim3(uint32_t(blocks)), kWideBW * kWave, 0, s>>>(a);
    }
    return hipGetLastError();
}

// s_waitcnt vmcnt(N), N < 64 (the counter's high bits sit at [15:14]).
template <int N>
__device__ __forceinline__ void wait_vm_const() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// f(integral_constant<int, I>) for I = 0 .. N - 1, in order.
template <class F, int... I>
__device__ __forceinline__ void for_each_const(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void unroll_const(F&& f) {
    for_each_const(f, std::make_integer_sequence<int, N>{});
}

// W-stationary wide path: 8 heads x 64 (16 head blocks), bf16 input, L and R
// in their own arrays (e.g. 512 -> 8 x 64).  Each wave keeps one head block's
// W^T fragments in registers for the whole launch (KS x 16 bytes per lane),
// and the tiles' input comes to it through LDS: blocks come in pairs, block
// p taking head blocks 0..7 and block pairs + p blocks 8..15 of the same
// tiles (the two share an XCD, so one of them finds each tile in L2), and
// every tile's input is requested kWsRing - 1 tiles ahead into an LDS ring
// (global_load_lds, the block's 8 waves sharing the k steps).  k_proj_wide
// instead streams W's fragments from L2 at every output block, and on a CU
// with HBM reads in flight those L2 hits wait as long as the reads.  Z is
// bit-equal to the other bf16 paths (each block's k steps in one chain, in
// order).  L and R are the FP32 Z row of the head against a_L and a_R, as
// lr_from_z forms them (baseline_standard.cpp:7-20), where the other paths
// multiply X by the hi/lo parts of W a: the two agree to FP32 rounding, not
// bit for bit.
constexpr int kWsWaves = 8;
constexpr int kWsRing = 4;  // tile inputs in LDS: the one multiplied and 3 requested ahead

template <int KS, bool RZ>
__global__ void __launch_bounds__(kWsWaves * kWave) __attribute__((amdgpu_waves_per_eu(2))) k_proj_ws(ProjArgs a,
                                                                                                   uint32_t pairs) {
    // The ring's slots are distinct arrays and the tile loop is unrolled by
    // kWsRing, so the compiler can tell the requests into one slot from the
    // reads of another and leaves them in flight.
    __shared__ __attribute__((aligned(16))) u32x4 ring0[KS * kWave];
    __shared__ __attribute__((aligned(16))) u32x4 ring1[KS * kWave];
    __shared__ __attribute__((aligned(16))) u32x4 ring2[KS * kWave];
    __shared__ __attribute__((aligned(16))) u32x4 ring3[KS * kWave];
    // L and R shares per tile row of the block's 4 heads (two head blocks
    // each), two tiles: [tile & 1][L, R][head][row][head block].
    __shared__ float plr[2][2][4][32][2];
    static_assert(kWsRing == 4 && KS % kWsWaves == 0, "four slots; the waves share the k steps evenly");
    const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave), l = threadIdx.x % kWave;
    const int half = l / 32, col = l % 32;
    const uint32_t g = blockIdx.x / pairs, p = blockIdx.x % pairs;
    const int ob = int(8 * g) + w;  // head block: head ob / 2, its features 32 (ob % 2) .. + 31
    // Row indices in 32 bits (the path takes fewer than 2^31 rows).
    const uint32_t nt = a.tiles > p ? uint32_t((a.tiles - 1 - p) / pairs + 1) : 0;
    const uint32_t n = uint32_t(a.n);
    if (nt == 0) return;  // (the launch gives every pair a tile)
    // W^T fragments of head block ob (group g, block w of the packing).
    bf16x8 wr[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
        wr[ks] = __builtin_bit_cast(bf16x8, a.wpk[((size_t(g) * KS + ks) * a.nmb + w) * kWave + l]);
    // a_L and a_R of the lane's 16 features (32 ob + 16 half + j).
    float alv[16], arv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        alv[j] = a.al[32 * ob + 16 * half + j];
        arv[j] = a.ar[32 * ob + 16 * half + j];
    }
    // Lanes past n recompute row n - 1 and store its own values to it.
    auto row_of = [&](uint32_t i) -> uint32_t {
        const uint32_t r = (p + i * pairs) * 32 + col;
        return r < n ? r : n - 1;
    };
    // Tile i's input into dst: this wave's k steps w, w + 8, ...  Past the
    // last tile the last one is requested again (into a slot no tile reads),
    // so every tile issues the same vector-memory instructions: kDma requests
    // and 3 stores (two Z pieces and one L or R value per row).
    constexpr int kDma = KS / kWsWaves;
    auto request = [&](uint32_t i, u32x4* dst) {
        const unsigned char* src =
            reinterpret_cast<const unsigned char*>(a.x + size_t(row_of(i < nt ? i : nt - 1)) * a.xs + 8 * half);
#pragma unroll
        for (int q = 0; q < kDma; ++q) {
            const int ks = w + kWsWaves * q;
            __builtin_amdgcn_global_load_lds(src + 32 * ks, (lds_ptr)(dst + ks * kWave), 16, 0, 0);
        }
    };
    // Wave w's value of the tile before: L (w < 4) or R of head 4 g + w % 4,
    // the shares of its two head blocks added.
    const int hw = w % 4;
    auto lr_value = [&](uint32_t i) -> float {
        const float2 v = *reinterpret_cast<const float2*>(&plr[i & 1][w < 4 ? 0 : 1][hw][l % 32][0]);
        return v.x + v.y;
    };
    float* const lr_out = (w < 4 ? a.left : a.right) + 4 * g + hw;
    request(0, ring0);
    request(1, ring1);
    request(2, ring2);
    wait_vm_const<2 * kDma>();  // tile 0's input (tiles 1 and 2 requested after it)
    __syncthreads();
    uint32_t prs = 0, prs2 = 0;  // the rows of the previous two tiles
    // RZ: the head block's share of R from the bf16 Z in the order the
    // 8-head aggregation recomputes it from a gathered row -- an FMA chain
    // over each 8 stored features (chunks c, c + 1 of the head), their sum,
    // the lane halves' sums added, then (in lr_value) the head's two blocks --
    // so both give R the same bits.  A tile's share is formed during the next
    // tile's MFMA chain, from its packed Z (zp), and published by that tile's
    // barrier; the R waves store R two tiles late.
    uint32_t zp[2][4] = {};
    auto r_share = [&]() -> float {
        float u[2];
#pragma unroll
        for (int q8 = 0; q8 < 2; ++q8) {
            float v = 0.0f;
#pragma unroll
            for (int x = 0; x < 8; ++x) {
                const uint32_t pr2 = zp[q8][x / 2];
                const float zv = __builtin_bit_cast(float, (x & 1) ? (pr2 & 0xffff0000u) : (pr2 << 16));
                v = __builtin_fmaf(zv, arv[8 * q8 + x], v);
            }
            u[q8] = v;
        }
        return u[0] + u[1];  // (the lane halves are added by the caller)
    };
    // Tile i from rd; tile i + 3 requested into rq.  At its end the wait for
    // tile i + 1's input: AFTER instructions were issued after that request.
    auto tile = [&](uint32_t i, const u32x4* rd, u32x4* rq, auto AFTER) {
        const uint32_t rs = row_of(i);
        request(i + 3, rq);  // into the slot tile i - 1 read
        if (l < 32) {
            // The tile before's L or R; tile 0 stores 0 to its own rows, which
            // tile 1 overwrites (same wave, same address).
            // (RZ: the R waves store tile i - 2's R; tile 1 also stores 0.)
            if (!RZ || w < 4) {
                if (i > 0) lr_out[size_t(prs) * 8] = lr_value(i - 1);
                else lr_out[size_t(rs) * 8] = 0.0f;
            } else {
                if (i > 1) lr_out[size_t(prs2) * 8] = lr_value(i - 2);
                else lr_out[size_t(rs) * 8] = 0.0f;
            }
        }
        float prv = 0.0f;  // RZ: the tile before's R share, formed among this tile's MFMAs
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
        // The tile's B fragments, read by ds_read_b128 written out here: the
        // compiler, which cannot tell the slots apart once several requests
        // are in flight, would wait for all of them before a compiled LDS
        // read.  The slot was filled and published before this tile (the
        // previous tile's vmcnt wait and barrier); each read is waited for
        // with lgkmcnt(kAhead - 1) -- LDS reads complete in order, so that
        // holds whatever else the counter carries.
        const uint32_t xaddr = uint32_t(reinterpret_cast<uintptr_t>(rd + l));
        constexpr int kAhead = 4;
        u32x4 fb[kAhead];
        auto rd_frag = [&](auto KSC) {
            constexpr int k = decltype(KSC)::value;
            u32x4 v;
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(xaddr), "i"(k * kWave * 16));
            fb[k % kAhead] = v;
        };
        unroll_const<kAhead>(rd_frag);
        auto step = [&](auto KSC) {
            constexpr int k = decltype(KSC)::value;
            u32x4 v = fb[k % kAhead];
            if constexpr (k + kAhead <= KS) {
                asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "i"(kAhead - 1));
            } else {
                asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "i"(KS - 1 - k));
            }
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wr[k], __builtin_bit_cast(bf16x8, v), acc, 0, 0, 0);
            if constexpr (k + kAhead < KS) rd_frag(std::integral_constant<int, k + kAhead>{});
            if constexpr (RZ && k == 1) prv = r_share();
        };
        unroll_const<KS>(step);
        // Z: lane (half, col) holds features 32 ob + 16 half + {0..15} of row
        // col, two 16-byte pieces.  Each store writes the head block's 64
        // bytes of 16 rows: inside the lane quad (rows 4 a .. 4 a + 3), store
        // j takes rows 4 a + 2 j and 4 a + 2 j + 1, lane c writing piece
        // 2 half + c % 2 of row 4 a + 2 j + c / 2, read from quad lane
        // 2 j + c / 2 by DPP.
        uint32_t P[2][4];
#pragma unroll
        for (int q8 = 0; q8 < 2; ++q8)
#pragma unroll
            for (int x = 0; x < 4; ++x) P[q8][x] = bf16x2(acc[8 * q8 + 2 * x], acc[8 * q8 + 2 * x + 1]);
        // The head block's share of L (and of R unless RZ) from FP32 Z: an
        // FMA chain over the lane's 16 features, the two lane halves added.
        float pl = 0.0f, pr = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) pl = __builtin_fmaf(acc[j], alv[j], pl);
        if constexpr (RZ) {
#pragma unroll
            for (int q8 = 0; q8 < 2; ++q8)
#pragma unroll
                for (int x = 0; x < 4; ++x) zp[q8][x] = P[q8][x];
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) pr = __builtin_fmaf(acc[j], arv[j], pr);
        }
        {
            const int c = l & 3;
            const uint32_t tbase = (p + i * pairs) * 32;
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
                const uint32_t rj = tbase + uint32_t((col & ~3) + 2 * j + (c >> 1));
                const uint32_t rsj = rj < n ? rj : n - 1;
                *reinterpret_cast<uint4*>(a.z + size_t(rsj) * a.zs + 32 * ob + 16 * half + 8 * (c & 1)) =
                    make_uint4(T[0], T[1], T[2], T[3]);
            };
            store_pair(std::integral_constant<int, 0>{});
            store_pair(std::integral_constant<int, 1>{});
        }
        pl += __shfl_xor(pl, 32);
        if constexpr (RZ) prv += __shfl_xor(prv, 32);
        if (l < 32) {
            plr[i & 1][0][w / 2][l][w % 2] = pl;
            if (RZ && i > 0) plr[(i - 1) & 1][1][w / 2][l][w % 2] = prv;
        }
        if constexpr (!RZ) {
            pr += __shfl_xor(pr, 32);
            if (l < 32) plr[i & 1][1][w / 2][l][w % 2] = pr;
        }
        wait_vm_const<decltype(AFTER)::value>();
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        prs2 = prs;
        prs = rs;
    };
    // After tile 1's request: tile 2's, then tile 0's request and stores.
    tile(0, ring0, ring3, std::integral_constant<int, 2 * kDma + 3>{});
    if (nt > 1) {
        // After tile 2's request: tiles 0 and 1's requests and stores.
        tile(1, ring1, ring0, std::integral_constant<int, 2 * kDma + 6>{});
        // After tile i + 1's request (made in tile i - 2): the stores of tiles
        // i - 2 .. i and the requests of tiles i - 1 and i.
        constexpr int kAfter = 2 * kDma + 9;
        for (uint32_t i = 2; i < nt; i += kWsRing) {
            tile(i, ring2, ring1, std::integral_constant<int, kAfter>{});
            if (i + 1 < nt) {
                tile(i + 1, ring3, ring2, std::integral_constant<int, kAfter>{});
                if (i + 2 < nt) {
                    tile(i + 2, ring0, ring3, std::integral_constant<int, kAfter>{});
                    if (i + 3 < nt) tile(i + 3, ring1, ring0, std::integral_constant<int, kAfter>{});
                }
            }
        }
    }
    if constexpr (RZ) {
        // R of tile nt - 2 (formed during tile nt - 1), then the last tile's.
        if (l < 32 && w >= 4 && nt > 1) lr_out[size_t(prs2) * 8] = lr_value(nt - 2);
        float pr = r_share();
        pr += __shfl_xor(pr, 32);
        if (l < 32) plr[(nt - 1) & 1][1][w / 2][l][w % 2] = pr;
        __syncthreads();
    }
    if (l < 32) lr_out[size_t(prs) * 8] = lr_value(nt - 1);
}

// The W-stationary path's shapes: bf16 input, 8 heads x 64 (two groups of 8
// full head blocks), L and R in their own arrays, 16 to 32 k steps; with or
// without R from the stored Z.
bool ws_ok(const ProjArgs& a) {
    return !a.x32 && !a.r_in_z && a.al && a.ar && a.heads == 8 && a.width == 512 && a.head_blocks == 16 &&
           a.groups == 2 && a.nmb == 9 && (a.ksteps == 16 || a.ksteps == 24 || a.ksteps == 32) && a.n < (1ull << 31);
}

template <int KS>
hipError_t launch_ws(const ProjArgs& a, hipStream_t s, int cus) {
    uint64_t pairs = uint64_t(cus) / 2;
    if (pairs > a.tiles) pairs = a.tiles;
    if (pairs < 1) return hipErrorInvalidValue;
    if (a.r_from_z) k_proj_ws<KS, true><<<dim3(uint32_t(2 * pairs)), kWsWaves * kWave, 0, s>>>(a, uint32_t(pairs));
    else k_proj_ws<KS, false><<<dim3(uint32_t(2 * pairs)), kWsWaves * kWave, 0, s>>>(a, uint32_t(pairs));
    return hipGetLastError();
}

// FP32 projection (the FP32 path's Z = X W and L/R = X B_LR) on
// v_mfma_f32_32x32x2_f32: FP32 products, FP32 accumulation.  Same work split
// as the wide path: a wave keeps the FP32 input of its 32-row tile in
// registers -- lane half h holds inputs [h KH, (h + 1) KH) of row col, so the
// MFMA's k index pair at step ks is (ks, KH + ks) and the loads are
// contiguous 16-byte vectors -- and the block streams W^T one 32-feature
// output block at a time (KH / 4 x 64 float4, 4 k steps per LDS read) through
// a two-slot LDS ring.  Head blocks use the permuted packing, so a lane ends
// with 16 consecutive features of its row; the last block is [B_L | B_R]
// (columns h and 8 + h), giving L and R of the reordered contraction
// (lr_reordered, baseline_standard.cpp:29-43) in FP32.
template <int KH>
__global__ void __launch_bounds__(kWideThreads) k_proj_f32(ProjF32Args a) {
    typedef float f32x4v __attribute__((ext_vector_type(4)));
    extern __shared__ f32x4v fring[];  // [2][KH / 4][kWave]
    constexpr int kFrags = KH / 4 * kWave;
    constexpr int kPer = (kFrags + kWideThreads - 1) / kWideThreads;
    const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
    const int half = l / 32, col = l % 32;
    const uint64_t row = (uint64_t(blockIdx.x) * kWideWaves + w) * 32 + col;
    const uint64_t rs = row < a.n ? row : a.n - 1;  // lanes past n repeat row n - 1
    float xr[KH];
    {
        const f32x4v* p = reinterpret_cast<const f32x4v*>(a.x + rs * a.xs + half * KH);
#pragma unroll
        for (int m = 0; m < KH / 4; ++m) {
            const f32x4v v = p[m];
            xr[4 * m] = v.x;
            xr[4 * m + 1] = v.y;
            xr[4 * m + 2] = v.z;
            xr[4 * m + 3] = v.w;
        }
    }
    const int nob = a.head_blocks + 1;
    f32x4v st[kPer];
    auto fetch = [&](int ob) {
        const f32x4v* src = reinterpret_cast<const f32x4v*>(a.wpk) + size_t(ob) * kFrags;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int q = threadIdx.x + i * kWideThreads;
            if (kFrags % kWideThreads == 0 || q < kFrags) st[i] = src[q];
        }
    };
    auto put = [&](int slot) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int q = threadIdx.x + i * kWideThreads;
            if (kFrags % kWideThreads == 0 || q < kFrags) fring[slot * kFrags + q] = st[i];
        }
    };
    fetch(0);
    put(0);
#pragma unroll
    for (int k = 0; k < KH; ++k) asm volatile("" ::"v"(xr[k]));  // input complete before the loop
    __syncthreads();
    for (int ob = 0; ob < nob; ++ob) {
        const int cur = ob & 1;
        const bool more = ob + 1 < nob;
        if (more) fetch(ob + 1);
        f32x16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
        const f32x4v* wk = fring + cur * kFrags + l;
#pragma unroll
        for (int k4 = 0; k4 < KH / 4; ++k4) {
            const f32x4v av = wk[k4 * kWave];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, xr[4 * k4], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, xr[4 * k4 + 1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, xr[4 * k4 + 2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, xr[4 * k4 + 3], acc, 0, 0, 0);
        }
        if (more) put(cur ^ 1);  // before the stores, as in the wide path
        __builtin_amdgcn_sched_barrier(0);
        if (ob < a.head_blocks) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int f0 = 32 * ob + 16 * half + 4 * q;
                if (f0 < a.width)
                    *reinterpret_cast<float4*>(a.z + rs * a.zs + f0) =
                        make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
            }
        } else {
            // Lane half h4 holds L of heads 4 h4 + {0..3} in registers 0..3 and
            // R of the same heads in registers 4..7.
            if (a.heads == 8) {
                *reinterpret_cast<float4*>(a.left + rs * 8 + 4 * half) = make_float4(acc[0], acc[1], acc[2], acc[3]);
                *reinterpret_cast<float4*>(a.right + rs * 8 + 4 * half) = make_float4(acc[4], acc[5], acc[6], acc[7]);
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int h = 4 * half + q;
                    if (h < a.heads) {
                        a.left[rs * a.heads + h] = acc[q];
                        a.right[rs * a.heads + h] = acc[4 + q];
                    }
                }
            }
        }
        __syncthreads();
    }
}

template <int KH>
hipError_t launch_f32_kh(const ProjF32Args& a, hipStream_t s) {
    const size_t lds = size_t(2) * (KH / 4) * kWave * 16;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_proj_f32<KH>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess) return e;
    }
    const uint64_t blocks = (a.tiles + kWideWaves - 1) / kWideWaves;
    if (blocks < 1 || blocks > 0x7fffffffu) return hipErrorInvalidValue;
    k_proj_f32<KH><<<dim3(uint32_t(blocks)), kWideThreads, lds, s>>>(a);
    return hipGetLastError();
}

constexpr size_t kOneTileLds = 56 * 1024;  // over a third of the CU's 160 KB

template <int KS, int HB, bool F32IN, int FULL>
hipError_t launch_fast_io(const ProjArgs& a, hipStream_t s, int cus) {
    const size_t lds = size_t(KS) * (HB + 1) * kWave * sizeof(uint4) + (FULL ? 256 * sizeof(float) : 0);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_proj_fast<KS, HB, F32IN, FULL>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess) return e;
    }
    // resident grid (1 or 2 blocks per CU), or one tile per wave for HB = 0
    // with the dynamic LDS raised to kOneTileLds (at most two blocks per CU:
    // a third block's streams measured slower, 0.40 against 0.33 ms on a
    // 2.45M x 100 input)
    const uint64_t wg_needed = (a.tiles + kWaves - 1) / kWaves;
    uint64_t gx = HB == 0 ? wg_needed : uint64_t(cus) * (lds <= 80 * 1024 ? 2 : 1);
    if (gx > wg_needed) gx = wg_needed;
    if (gx < 1) gx = 1;
    if (gx > 0x7fffffffu) return hipErrorInvalidValue;
    if (FULL == 2 && !a.ar) return hipErrorInvalidValue;
    const size_t req = HB == 0 && lds < kOneTileLds ? kOneTileLds : lds;
    k_proj_fast<KS, HB, F32IN, FULL><<<dim3(uint32_t(gx)), kThreads, req, s>>>(a);
    return hipGetLastError();
}

template <int KS, int HB>
hipError_t launch_fast(const ProjArgs& a, hipStream_t s, int cus) {
    if constexpr (HB == 8) {
        if (a.width == 256 && a.heads == 8 && !a.r_in_z) {
            if (a.r_from_z)
                return a.x32 ? launch_fast_io<KS, HB, true, 2>(a, s, cus) : launch_fast_io<KS, HB, false, 2>(a, s, cus);
            return a.x32 ? launch_fast_io<KS, HB, true, 1>(a, s, cus) : launch_fast_io<KS, HB, false, 1>(a, s, cus);
        }
    }
    return a.x32 ? launch_fast_io<KS, HB, true, 0>(a, s, cus) : launch_fast_io<KS, HB, false, 0>(a, s, cus);
}

template <int HB>
hipError_t launch_fast_ks(const ProjArgs& a, hipStream_t s, int cus) {
    switch (a.ksteps) {
        case 1: return launch_fast<1, HB>(a, s, cus);
        case 2: return launch_fast<2, HB>(a, s, cus);
        case 3: return launch_fast<3, HB>(a, s, cus);
        case 4: return launch_fast<4, HB>(a, s, cus);
        case 5: return launch_fast<5, HB>(a, s, cus);
        case 6: return launch_fast<6, HB>(a, s, cus);
        case 7: return launch_fast<7, HB>(a, s, cus);
        case 8: return launch_fast<8, HB>(a, s, cus);
        case 16: return launch_fast<16, HB>(a, s, cus);
        default: return hipErrorInvalidValue;
    }
}

bool fast_supported_impl(const ProjArgs& a) {
    const bool ks_ok = (a.ksteps >= 1 && a.ksteps <= 8) || a.ksteps == 16;
    const bool hb_ok = a.head_blocks == 0 || a.head_blocks == 1 || a.head_blocks == 2 || a.head_blocks == 8;
    return a.groups == 1 && ks_ok && hb_ok && a.n > 0;
}

template <int NMB>
hipError_t launch_nmb(const ProjArgs& a, hipStream_t s, int cus) {
    const size_t lds = size_t(a.ksteps) * NMB * kWave * sizeof(uint4);
    const uint64_t wg_needed = (a.tiles + kWaves - 1) / kWaves;
    if (lds <= 160 * 1024) {
        const int per_cu = lds <= 80 * 1024 ? 2 : 1;
        uint64_t gx = uint64_t(cus) * per_cu;
        if (gx > wg_needed) gx = wg_needed;
        if (gx < 1) gx = 1;
        if (lds > 64 * 1024) {
            hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_proj_mfma<NMB, true>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
            if (e != hipSuccess) return e;
        }
        k_proj_mfma<NMB, true><<<dim3(uint32_t(gx), uint32_t(a.groups)), kThreads, lds, s>>>(a);
    } else {
        uint64_t gx = wg_needed < 65535 * 16 ? wg_needed : 65535 * 16;
        if (gx < 1) gx = 1;
        k_proj_mfma<NMB, false><<<dim3(uint32_t(gx), uint32_t(a.groups)), kThreads, 0, s>>>(a);
    }
    return hipGetLastError();
}

}  // namespace

int proj_blocks_per_group(int width) {
    const int head_blocks = (width + 31) / 32;
    if (head_blocks >= 8) return 9;
    const int need = head_blocks + 1;
    return need <= 2 ? 2 : need <= 3 ? 3 : need <= 5 ? 5 : 9;
}

// Wide path: 8, 16, 24 or 32 k steps where the fast path does not apply and
// there are several output groups or one group's fragments exceed LDS.
bool wide_ks(const ProjArgs& a) {
    return a.n > 0 && (a.ksteps == 8 || a.ksteps == 16 || a.ksteps == 24 || a.ksteps == 32);
}

// One head of exactly 64 (no room for R in the 128-byte row): the wide path
// writes R = Z_bf16 . aR for the aggregation to recompute.
bool rz_one_head(const ProjArgs& a) { return wide_ks(a) && a.heads == 1 && a.width == 64 && !a.r_in_z; }

bool wide_supported_impl(const ProjArgs& a) {
    if (a.r_from_z) return rz_one_head(a) || ws_ok(a);
    const size_t group_lds = size_t(a.ksteps) * a.nmb * kWave * sizeof(uint4);
    return wide_ks(a) && !fast_supported_impl(a) && (a.groups > 1 || group_lds > 160 * 1024);
}

hipError_t launch_wide(const ProjArgs& a, hipStream_t s, int cus) {
    if (ws_ok(a) && cus >= 2) {
        switch (a.ksteps) {
            case 16: return launch_ws<16>(a, s, cus);
            case 24: return launch_ws<24>(a, s, cus);
            case 32: return launch_ws<32>(a, s, cus);
            default: break;
        }
    }
    if (a.r_from_z && !rz_one_head(a)) return hipErrorInvalidValue;  // (8 x 64: the W-stationary path only)
    switch (a.ksteps) {
        case 8: return a.x32 ? launch_wide_io<8, true>(a, s) : launch_wide_io<8, false>(a, s);
        case 16: return a.x32 ? hipErrorInvalidValue : launch_wide_io<16, false>(a, s);
        case 24: return a.x32 ? hipErrorInvalidValue : launch_wide_io<24, false>(a, s);
        case 32: return a.x32 ? hipErrorInvalidValue : launch_wide_io<32, false>(a, s);
        default: return hipErrorInvalidValue;
    }
}

bool projection_fast_path(const ProjArgs& a) { return fast_supported_impl(a); }

bool r_from_z_supported(const ProjArgs& a) {
    return (fast_supported_impl(a) && a.head_blocks == 8 && a.width == 256 && a.heads == 8 && !a.r_in_z) ||
           rz_one_head(a) || ws_ok(a);
}

// The FP32-input form holds 32 bytes per k step; at 16 k steps and 8 head
// blocks that no longer fits the registers.
// The wide path takes it at 8 k steps (the raw rows and their bf16 fragments
// both fit the registers).
bool projection_fp32_input(const ProjArgs& a) {
    if (a.r_from_z && a.heads == 1) return rz_one_head(a) && a.ksteps == 8;
    return (fast_supported_impl(a) && (a.ksteps <= 8 || a.head_blocks <= 2)) ||
           (wide_supported_impl(a) && a.ksteps == 8);
}

hipError_t launch_projection_mfma(const ProjArgs& a, hipStream_t s, int cus) {
    if (a.x32 && !projection_fp32_input(a)) return hipErrorInvalidValue;
    if (a.r_from_z && a.heads == 1) return rz_one_head(a) && a.ar ? launch_wide(a, s, cus) : hipErrorInvalidValue;
    if (fast_supported_impl(a)) {
        switch (a.head_blocks) {
            case 0: return launch_fast_ks<0>(a, s, cus);
            case 1: return launch_fast_ks<1>(a, s, cus);
            case 2: return launch_fast_ks<2>(a, s, cus);
            default: return launch_fast_ks<8>(a, s, cus);
        }
    }
    if (wide_supported_impl(a)) return launch_wide(a, s, cus);
    switch (a.nmb) {
        case 2: return launch_nmb<2>(a, s, cus);
        case 3: return launch_nmb<3>(a, s, cus);
        case 5: return launch_nmb<5>(a, s, cus);
        case 9: return launch_nmb<9>(a, s, cus);
        default: return hipErrorInvalidValue;
    }
}

// Packs W (bf16-rounded, [in][width]) and B_LR = W_bf16 a (hi/lo) into the
// A-fragment order [group][kstep][block][lane][8]: lane l of head block b at
// k step ks holds W^T[32 b + phi(l % 32)][16 ks + 8 (l / 32) + j], j = 0..7,
// with phi(c) = 16 ((c % 8) / 4) + 4 (c / 8) + c % 4; the L/R block is not
// permuted.
void pack_projection_weights(const float* wq, const float* al, const float* ar, int in, int heads, int dim,
                             std::vector<uint16_t>& out, int& ksteps, int& groups, int& nmb) {
    const int width = heads * dim;
    const int head_blocks = (width + 31) / 32;
    nmb = proj_blocks_per_group(width);
    groups = head_blocks >= 8 ? (head_blocks + 7) / 8 : 1;
    ksteps = (in + 15) / 16;
    // B_LR columns from the bf16 W in double, split into bf16 hi + lo.
    std::vector<float> lrcol(size_t(in) * 32, 0.0f);
    for (int k = 0; k < in; ++k)
        for (int h = 0; h < heads; ++h) {
            double l = 0, r = 0;
            for (int d = 0; d < dim; ++d) {
                const double wv = wq[size_t(k) * width + h * dim + d];
                l += wv * al[h * dim + d];
                r += wv * ar[h * dim + d];
            }
            const float lf = float(l), rf = float(r);
            const float lh = bf16_widen(bf16_rne(lf)), rh = bf16_widen(bf16_rne(rf));
            lrcol[size_t(k) * 32 + h] = lh;
            lrcol[size_t(k) * 32 + 8 + h] = rh;
            lrcol[size_t(k) * 32 + 16 + h] = bf16_widen(bf16_rne(lf - lh));
            lrcol[size_t(k) * 32 + 24 + h] = bf16_widen(bf16_rne(rf - rh));
        }
    out.assign(size_t(groups) * ksteps * nmb * kWave * 8, 0);
    for (int g = 0; g < groups; ++g) {
        const int hb = head_blocks - 8 * g < 8 ? head_blocks - 8 * g : 8;
        for (int ks = 0; ks < ksteps; ++ks)
            for (int b = 0; b < nmb; ++b) {
                const bool lr = g == groups - 1 && b == hb;
                if (b > hb || (b == hb && !lr)) continue;
                for (int l = 0; l < kWave; ++l)
                    for (int j = 0; j < 8; ++j) {
                        const int k = 16 * ks + 8 * (l / 32) + j, c = l % 32;
                        // Head blocks: A row c (= D row c) carries feature phi(c), so that the
                        // D rows a lane holds, 8 (r / 4) + 4 half + r % 4, are features
                        // 16 half + r -- 16 consecutive features per lane.
                        const int phi = 16 * ((c % 8) / 4) + 4 * (c / 8) + c % 4;
                        float v = 0.0f;
                        if (k < in) {
                            if (lr) v = lrcol[size_t(k) * 32 + c];
                            else if (32 * (8 * g + b) + phi < width)
                                v = wq[size_t(k) * width + 32 * (8 * g + b) + phi];
                        }
                        out[((((size_t(g) * ksteps + ks) * nmb + b) * kWave + l) * 8) + j] = bf16_rne(v);
                    }
            }
    }
}

// FP32 MFMA projection: 2 KH = in inputs with KH in {16, 32, 48, 64, 96, 128},
// any heads x dim up to 8 x 64.
bool projection_f32_supported(int in, int heads, int dim) {
    const int kh = in / 2;
    return in % 2 == 0 && (kh == 16 || kh == 32 || kh == 48 || kh == 64 || kh == 96 || kh == 128) && heads >= 1 &&
           heads <= 8 && dim >= 1 && heads * dim <= 512;
}

hipError_t launch_projection_f32(const ProjF32Args& a, hipStream_t s) {
    if (a.n == 0) return hipSuccess;
    if (!projection_f32_supported(a.in, a.heads, a.width / a.heads) || a.xs != a.in || a.zs % 4 != 0 ||
        a.zs < (a.width + 3) / 4 * 4 || a.head_blocks != (a.width + 31) / 32)
        return hipErrorInvalidValue;
    switch (a.in / 2) {
        case 16: return launch_f32_kh<16>(a, s);
        case 32: return launch_f32_kh<32>(a, s);
        case 48: return launch_f32_kh<48>(a, s);
        case 64: return launch_f32_kh<64>(a, s);
        case 96: return launch_f32_kh<96>(a, s);
        default: return launch_f32_kh<128>(a, s);
    }
}

// FP32 fragments [block][k4][lane][4] for k_proj_f32: head block b, lane
// (half, c), k step ks = 4 k4 + j holds W[half KH + ks][32 b + phi(c)] (phi
// as in pack_projection_weights); the last block holds B_L in rows 0..heads-1
// and B_R in rows 8..8+heads-1.  blr is [in][2 heads] (L columns, then R).
void pack_projection_f32(const float* w, const float* blr, int in, int heads, int dim, std::vector<float>& out) {
    const int width = heads * dim, hb = (width + 31) / 32, kh = in / 2;
    out.assign(size_t(hb + 1) * kh * kWave, 0.0f);
    for (int b = 0; b <= hb; ++b)
        for (int k4 = 0; k4 < kh / 4; ++k4)
            for (int l = 0; l < kWave; ++l)
                for (int j = 0; j < 4; ++j) {
                    const int c = l % 32, k = (l / 32) * kh + 4 * k4 + j;
                    float v = 0.0f;
                    if (b < hb) {
                        const int f = 32 * b + 16 * ((c % 8) / 4) + 4 * (c / 8) + c % 4;
                        if (f < width) v = w[size_t(k) * width + f];
                    } else if (c < heads) {
                        v = blr[size_t(k) * 2 * heads + c];
                    } else if (c >= 8 && c < 8 + heads) {
                        v = blr[size_t(k) * 2 * heads + heads + (c - 8)];
                    }
                    out[((size_t(b) * (kh / 4) + k4) * kWave + l) * 4 + j] = v;
                }
}

// Only the L/R block ([kstep][2][lane][8], block 1 zero): the reordered
// contraction LR = X (W_bf16 a) for the aggregate-first front end.
void pack_lr_weights(const float* wq, const float* al, const float* ar, int in, int heads, int dim,
                     std::vector<uint16_t>& out, int& ksteps) {
    const int width = heads * dim;
    ksteps = (in + 15) / 16;
    out.assign(size_t(ksteps) * 2 * kWave * 8, 0);
    for (int k = 0; k < in; ++k)
        for (int h = 0; h < heads; ++h) {
            double l = 0, r = 0;
            for (int d = 0; d < dim; ++d) {
                const double wv = wq[size_t(k) * width + h * dim + d];
                l += wv * al[h * dim + d];
                r += wv * ar[h * dim + d];
            }
            const float lf = float(l), rf = float(r);
            const float lh = bf16_widen(bf16_rne(lf)), rh = bf16_widen(bf16_rne(rf));
            const float cols[4] = {lh, rh, bf16_widen(bf16_rne(lf - lh)), bf16_widen(bf16_rne(rf - rh))};
            for (int qd = 0; qd < 4; ++qd) {
                const int c = 8 * qd + h;  // L hi, R hi, L lo, R lo at columns h, 8+h, 16+h, 24+h
                const int ks = k / 16, half = (k % 16) / 8, j = k % 8;
                out[((size_t(ks) * 2 + 0) * kWave + half * 32 + c) * 8 + j] = bf16_rne(cols[qd]);
            }
        }
}

}  // namespace gatgpu
