// Degree schedule on the GPU: the ascending (degree, id) permutation of
// destination rows and the CSR re-laid out in that order.
//
// Reference: degree_schedule (baseline/src/common.cpp:120-125) sorts row ids
// by (degree, id) with std::sort; degree_perm
// (implementation/src/gat_tfs_online.cpp:180-189) is the same order.  Here the
// order comes from an LSD radix sort of the degrees whose passes are stable,
// started from ids in ascending order, so equal degrees keep ascending ids and
// the result is identical to the reference's comparator sort.
#include "internal.hpp"

namespace gatgpu {
namespace {

constexpr int kThreads = 256;
constexpr int kItems = 8;
constexpr int kTile = kThreads * kItems;  // items per radix tile / scan tile

__global__ void __launch_bounds__(kThreads)
k_degrees(const uint64_t* __restrict__ row, uint32_t* __restrict__ deg, uint32_t* __restrict__ vals,
          uint64_t n, uint32_t* __restrict__ maxdeg) {
    uint32_t local = 0;
    for (uint64_t i = blockIdx.x * uint64_t(kThreads) + threadIdx.x; i < n;
         i += uint64_t(gridDim.x) * kThreads) {
        uint32_t d = uint32_t(row[i + 1] - row[i]);
        deg[i] = d;
        vals[i] = uint32_t(i);
        local = d > local ? d : local;
    }
    for (int off = 32; off > 0; off >>= 1) {
        uint32_t o = __shfl_xor(local, off);
        local = o > local ? o : local;
    }
    if ((threadIdx.x & (kWave - 1)) == 0) atomicMax(maxdeg, local);
}

// ---- radix pass 1: per-tile digit histogram, digit-major [digit][tile].
__global__ void __launch_bounds__(kThreads)
k_radix_hist(const uint32_t* __restrict__ keys, uint64_t n, int shift, uint32_t* __restrict__ hist,
             uint32_t tiles) {
    __shared__ uint32_t h[256];
    h[threadIdx.x] = 0;
    __syncthreads();
    const uint64_t base = uint64_t(blockIdx.x) * kTile;
    for (int j = 0; j < kItems; ++j) {
        uint64_t idx = base + uint64_t(j) * kThreads + threadIdx.x;
        if (idx < n) atomicAdd(&h[(keys[idx] >> shift) & 255u], 1u);
    }
    __syncthreads();
    hist[uint64_t(threadIdx.x) * tiles + blockIdx.x] = h[threadIdx.x];
}

// ---- radix pass 2: stable scatter.  Items of a tile are visited in strips
// (strip j holds positions base + j*256 + t, i.e. ascending order strip by
// strip); inside a strip the rank of an item among equal digits comes from a
// wave-level match mask (8 ballots) and per-wave counts in LDS, so the output
// order of equal digits equals the input order.
__global__ void __launch_bounds__(kThreads)
k_radix_scatter(const uint32_t* __restrict__ keys, const uint32_t* __restrict__ vals,
                uint32_t* __restrict__ keys_out, uint32_t* __restrict__ vals_out, uint64_t n, int shift,
                const uint32_t* __restrict__ offsets, uint32_t tiles) {
    __shared__ uint32_t running[256];
    __shared__ uint32_t wcnt[kThreads / kWave][256];
    const int t = threadIdx.x, w = t / kWave, lane = t % kWave;
    running[t] = offsets[uint64_t(t) * tiles + blockIdx.x];
    const uint64_t base = uint64_t(blockIdx.x) * kTile;
    const uint64_t lt_mask = (uint64_t(1) << lane) - 1;
    for (int j = 0; j < kItems; ++j) {
        for (int q = 0; q < kThreads / kWave; ++q) wcnt[q][t] = 0;
        const uint64_t idx = base + uint64_t(j) * kThreads + t;
        const bool valid = idx < n;
        uint32_t key = 0, val = 0;
        if (valid) {
            key = keys[idx];
            val = vals[idx];
        }
        const uint32_t digit = (key >> shift) & 255u;
        uint64_t match = __ballot(valid);
        for (int b = 0; b < 8; ++b) {
            const bool bit = (digit >> b) & 1u;
            const uint64_t bb = __ballot(bit);
            match &= bit ? bb : ~bb;
        }
        const uint32_t rank = __popcll(match & lt_mask);
        const uint32_t count = __popcll(match);
        __syncthreads();  // wcnt cleared, running visible
        if (valid && rank == 0) wcnt[w][digit] = count;
        __syncthreads();
        if (valid) {
            uint32_t pos = running[digit] + rank;
            for (int q = 0; q < w; ++q) pos += wcnt[q][digit];
            if (pos < n) {  // always true for a consistent histogram
                keys_out[pos] = key;
                vals_out[pos] = val;
            }
        }
        __syncthreads();  // every lane has read running[] for this strip
        uint32_t add = 0;
        for (int q = 0; q < kThreads / kWave; ++q) add += wcnt[q][t];
        running[t] += add;
        __syncthreads();  // before the next strip clears wcnt
    }
}

// ---- device-wide exclusive scan (tile sums -> scan of sums -> tile scan).
template <class In, class Out>
__global__ void __launch_bounds__(kThreads)
k_scan_tile_sums(const In* __restrict__ in, uint64_t n, Out* __restrict__ sums) {
    __shared__ Out red[kThreads / kWave];
    const uint64_t base = uint64_t(blockIdx.x) * kTile;
    Out s = 0;
    for (int j = 0; j < kItems; ++j) {
        uint64_t idx = base + uint64_t(j) * kThreads + threadIdx.x;
        if (idx < n) s += Out(in[idx]);
    }
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        Out total = 0;
        for (int q = 0; q < kThreads / kWave; ++q) total += red[q];
        sums[blockIdx.x] = total;
    }
}

// Block-wide exclusive scan of one value per thread; returns the block total.
template <class T>
__device__ T block_exclusive_scan(T v, T* lds_waves, T& total) {
    const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
    T inc = v;
    for (int off = 1; off < kWave; off <<= 1) {
        T o = __shfl_up(inc, off);
        if (lane >= off) inc += o;
    }
    if (lane == kWave - 1) lds_waves[w] = inc;
    __syncthreads();
    T before = 0;
    total = 0;
    for (int q = 0; q < kThreads / kWave; ++q) {
        if (q < w) before += lds_waves[q];
        total += lds_waves[q];
    }
    __syncthreads();
    return before + inc - v;
}

// Single-block exclusive scan of the tile sums, in place.
template <class Out>
__global__ void __launch_bounds__(kThreads) k_scan_sums(Out* __restrict__ sums, uint64_t count) {
    __shared__ Out lw[kThreads / kWave];
    Out carry = 0;
    for (uint64_t base = 0; base < count; base += kThreads) {
        uint64_t idx = base + threadIdx.x;
        Out v = idx < count ? sums[idx] : Out(0);
        Out total;
        Out ex = block_exclusive_scan(v, lw, total);
        if (idx < count) sums[idx] = carry + ex;
        carry += total;
    }
}

// Tile scan with the scanned tile offset.  Thread t owns items
// [t*kItems, t*kItems+kItems) of the tile (contiguous), so the per-thread
// serial scan followed by the block scan gives the ascending order.
template <class In, class Out>
__global__ void __launch_bounds__(kThreads)
// in and out may alias (in-place scan): each thread reads its items before writing them.
k_scan_apply(const In* in, uint64_t n, const Out* __restrict__ offs, Out* out) {
    __shared__ Out lw[kThreads / kWave];
    const uint64_t base = uint64_t(blockIdx.x) * kTile + uint64_t(threadIdx.x) * kItems;
    Out v[kItems];
    Out s = 0;
    for (int j = 0; j < kItems; ++j) {
        uint64_t idx = base + j;
        v[j] = idx < n ? Out(in[idx]) : Out(0);
        s += v[j];
    }
    Out total;
    Out run = block_exclusive_scan(s, lw, total) + offs[blockIdx.x];
    for (int j = 0; j < kItems; ++j) {
        uint64_t idx = base + j;
        if (idx < n) out[idx] = run;
        run += v[j];
    }
}

template <class In, class Out>
hipError_t exclusive_scan(const In* in, Out* out, uint64_t n, void* tmp, hipStream_t s) {
    const uint64_t tiles = (n + kTile - 1) / kTile;
    Out* sums = static_cast<Out*>(tmp);
    if (n == 0) return hipSuccess;
    k_scan_tile_sums<In, Out><<<dim3(uint32_t(tiles)), kThreads, 0, s>>>(in, n, sums);
    k_scan_sums<Out><<<1, kThreads, 0, s>>>(sums, tiles);
    k_scan_apply<In, Out><<<dim3(uint32_t(tiles)), kThreads, 0, s>>>(in, n, sums, out);
    return hipGetLastError();
}

// One wave copies one row's neighbour list into its sorted position.
__global__ void __launch_bounds__(kThreads)
k_permute_cols(const uint64_t* __restrict__ row, const uint32_t* __restrict__ col,
               const uint32_t* __restrict__ perm, const uint64_t* __restrict__ prow,
               uint32_t* __restrict__ pcol, uint64_t n, uint64_t e) {
    const uint64_t k = (uint64_t(blockIdx.x) * kThreads + threadIdx.x) / kWave;
    const int lane = threadIdx.x % kWave;
    if (k >= n) return;
    const uint32_t r = perm[k];
    if (r >= n) return;  // perm is a permutation of [0, n); guard against a corrupt one
    const uint64_t src = row[r], deg = row[r + 1] - src, dst = prow[k];
    if (dst > e || deg > e - dst) return;
    for (uint64_t q = lane; q < deg; q += kWave) pcol[dst + q] = col[src + q];
}

// The per-edge values of row perm[k] (K floats per edge, original CSR order)
// to their degree-sorted position: dst[(prow[k] + q) K + h] = src[(row[r] + q) K + h].
__global__ void __launch_bounds__(kThreads)
k_permute_edge_values(const uint64_t* __restrict__ row, const uint32_t* __restrict__ perm,
                      const uint64_t* __restrict__ prow, const float* __restrict__ src, float* __restrict__ dst,
                      uint64_t n, uint64_t e, int K) {
    const uint64_t k = (uint64_t(blockIdx.x) * kThreads + threadIdx.x) / kWave;
    const int lane = threadIdx.x % kWave;
    if (k >= n) return;
    const uint32_t r = perm[k];
    if (r >= n) return;
    const uint64_t s0 = row[r], deg = row[r + 1] - s0, d0 = prow[k];
    if (d0 > e || deg > e - d0 || s0 > e || deg > e - s0) return;
    const uint64_t cnt = deg * uint64_t(K);
    for (uint64_t q = lane; q < cnt; q += kWave) dst[d0 * K + q] = src[s0 * K + q];
}

// Sorted node order.  invperm[perm[k]] = k and ident[k] = k.
__global__ void __launch_bounds__(kThreads)
k_invert_perm(const uint32_t* __restrict__ perm, uint32_t* __restrict__ invperm, uint32_t* __restrict__ ident,
              uint64_t n) {
    for (uint64_t k = uint64_t(blockIdx.x) * kThreads + threadIdx.x; k < n; k += uint64_t(gridDim.x) * kThreads) {
        const uint32_t r = perm[k];
        if (r < n) invperm[r] = uint32_t(k);
        ident[k] = uint32_t(k);
    }
}

// rcol[q] = invperm[pcol[q]]: source ids of the sorted CSR as sorted positions.
__global__ void __launch_bounds__(kThreads)
k_relabel_cols(const uint32_t* __restrict__ pcol, const uint32_t* __restrict__ invperm, uint32_t* __restrict__ rcol,
               uint64_t e, uint64_t n) {
    for (uint64_t q = uint64_t(blockIdx.x) * kThreads + threadIdx.x; q < e; q += uint64_t(gridDim.x) * kThreads) {
        const uint32_t j = pcol[q];
        rcol[q] = j < n ? invperm[j] : 0u;
    }
}

// dst row r = src row idx[r], rows of `words` 4-byte words (row strides in
// words).  A block copies 64 rows at a time as one flat range of
// 64 * words words (32-bit index arithmetic within the range), so every
// thread has several independent loads in flight.
constexpr uint32_t kGatherRows = 64;
__global__ void __launch_bounds__(kThreads)
k_gather_rows(const uint32_t* __restrict__ src, uint64_t src_stride, uint32_t* __restrict__ dst, uint64_t dst_stride,
              const uint32_t* __restrict__ idx, uint64_t rows, uint64_t n_src, uint32_t words) {
    const uint64_t chunks = (rows + kGatherRows - 1) / kGatherRows;
    for (uint64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
        const uint64_t r0 = c * kGatherRows;
        const uint32_t nr = uint32_t(rows - r0 < kGatherRows ? rows - r0 : kGatherRows);
        const uint32_t total = nr * words;
        for (uint32_t t = threadIdx.x; t < total; t += kThreads) {
            const uint32_t rr = t / words, w = t - rr * words;
            const uint32_t q = idx[r0 + rr];
            dst[(r0 + rr) * dst_stride + w] = q < n_src ? src[uint64_t(q) * src_stride + w] : 0u;
        }
    }
}

// neighbor_steps = sum over 16-row tiles of the last (= largest) degree.
__global__ void __launch_bounds__(kThreads)
k_neighbor_steps(const uint32_t* __restrict__ sorted_deg, uint64_t n, uint64_t* __restrict__ steps) {
    const uint64_t tiles = (n + 15) / 16;
    uint64_t s = 0;
    for (uint64_t t = blockIdx.x * uint64_t(kThreads) + threadIdx.x; t < tiles;
         t += uint64_t(gridDim.x) * kThreads) {
        uint64_t last = (t * 16 + 16 < n ? t * 16 + 16 : n) - 1;
        s += sorted_deg[last];
    }
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (threadIdx.x % kWave == 0) atomicAdd(reinterpret_cast<unsigned long long*>(steps),
                                            static_cast<unsigned long long>(s));
}

// positions[q] = number of sorted rows with degree <= thresholds[q].
__global__ void k_count_le(const uint32_t* __restrict__ sorted_deg, uint64_t n,
                           const uint32_t* __restrict__ thr, int count, uint64_t* __restrict__ pos) {
    const int q = threadIdx.x;
    if (q >= count) return;
    uint64_t lo = 0, hi = n;  // first index with degree > thr
    const uint32_t t = thr[q];
    while (lo < hi) {
        uint64_t mid = (lo + hi) / 2;
        if (sorted_deg[mid] <= t) lo = mid + 1;
        else hi = mid;
    }
    pos[q] = lo;
}

uint32_t grid_for(uint64_t items, uint64_t per_block, uint32_t cap) {
    uint64_t g = (items + per_block - 1) / per_block;
    if (g < 1) g = 1;
    return uint32_t(g > cap ? cap : g);
}

}  // namespace

size_t radix_tile_hist_elems(uint64_t n) { return 256 * ((n + kTile - 1) / kTile); }
size_t scan_tmp_bytes(uint64_t n) { return 8 * ((n + kTile - 1) / kTile + 1); }

hipError_t launch_degrees_and_ids(const uint64_t* row, uint32_t* deg, uint32_t* ids, uint64_t n,
                                  uint32_t* maxdeg, hipStream_t s) {
    k_degrees<<<grid_for(n, kThreads, 4096), kThreads, 0, s>>>(row, deg, ids, n, maxdeg);
    return hipGetLastError();
}

hipError_t radix_sort_by_degree(uint32_t* keys, uint32_t* vals, uint32_t* keys_alt,
                                uint32_t* vals_alt, uint32_t* tile_hist, uint64_t n, int passes,
                                void* scan_tmp, hipStream_t s, uint32_t** keys_out,
                                uint32_t** vals_out) {
    const uint32_t tiles = uint32_t((n + kTile - 1) / kTile);
    const uint64_t hist_n = uint64_t(tiles) * 256;
    for (int p = 0; p < passes; ++p) {
        const int shift = 8 * p;
        k_radix_hist<<<tiles, kThreads, 0, s>>>(keys, n, shift, tile_hist, tiles);
        hipError_t err = exclusive_scan<uint32_t, uint32_t>(tile_hist, tile_hist, hist_n, scan_tmp, s);
        if (err != hipSuccess) return err;
        k_radix_scatter<<<tiles, kThreads, 0, s>>>(keys, vals, keys_alt, vals_alt, n, shift, tile_hist,
                                                   tiles);
        if ((err = hipGetLastError()) != hipSuccess) return err;
        uint32_t* t = keys;
        keys = keys_alt;
        keys_alt = t;
        t = vals;
        vals = vals_alt;
        vals_alt = t;
    }
    *keys_out = keys;
    *vals_out = vals;
    return hipGetLastError();
}

hipError_t exclusive_scan_u32_to_u64(const uint32_t* in, uint64_t* out, uint64_t n, void* tmp,
                                     hipStream_t s) {
    return exclusive_scan<uint32_t, uint64_t>(in, out, n, tmp, s);
}

hipError_t launch_permute_cols(const uint64_t* row, const uint32_t* col, const uint32_t* perm,
                               const uint64_t* prow, uint32_t* pcol, uint64_t n, uint64_t e,
                               hipStream_t s) {
    const uint64_t waves_per_block = kThreads / kWave;
    const uint64_t blocks = (n + waves_per_block - 1) / waves_per_block;
    k_permute_cols<<<dim3(uint32_t(blocks)), kThreads, 0, s>>>(row, col, perm, prow, pcol, n, e);
    return hipGetLastError();
}

hipError_t launch_permute_edge_values(const uint64_t* row, const uint32_t* perm, const uint64_t* prow,
                                     const float* src, float* dst, uint64_t n, uint64_t e, int K, hipStream_t s) {
    const uint64_t waves_per_block = kThreads / kWave;
    const uint64_t blocks = (n + waves_per_block - 1) / waves_per_block;
    k_permute_edge_values<<<dim3(uint32_t(blocks)), kThreads, 0, s>>>(row, perm, prow, src, dst, n, e, K);
    return hipGetLastError();
}

hipError_t launch_relabel(const uint32_t* perm, const uint32_t* pcol, uint32_t* invperm, uint32_t* ident,
                          uint32_t* rcol, uint64_t n, uint64_t e, hipStream_t s) {
    k_invert_perm<<<grid_for(n, kThreads, 4096), kThreads, 0, s>>>(perm, invperm, ident, n);
    if (e) k_relabel_cols<<<grid_for(e, kThreads, 8192), kThreads, 0, s>>>(pcol, invperm, rcol, e, n);
    return hipGetLastError();
}

hipError_t launch_gather_rows(const void* src, uint64_t src_stride_words, void* dst, uint64_t dst_stride_words,
                              const uint32_t* idx, uint64_t rows, uint64_t n_src, uint32_t words, hipStream_t s) {
    if (!rows || !words) return hipSuccess;
    if (words > (uint32_t(1) << 24)) return hipErrorInvalidValue;  // 64 * words must fit 32 bits
    k_gather_rows<<<grid_for((rows + kGatherRows - 1) / kGatherRows, 1, 16384), kThreads, 0, s>>>(
        static_cast<const uint32_t*>(src), src_stride_words, static_cast<uint32_t*>(dst), dst_stride_words, idx, rows,
        n_src, words);
    return hipGetLastError();
}

hipError_t launch_neighbor_steps(const uint32_t* sorted_deg, uint64_t n, uint64_t* steps,
                                 hipStream_t s) {
    k_neighbor_steps<<<grid_for((n + 15) / 16, kThreads, 1024), kThreads, 0, s>>>(sorted_deg, n, steps);
    return hipGetLastError();
}

hipError_t launch_count_le(const uint32_t* sorted_deg, uint64_t n, const uint32_t* thresholds,
                           int count, uint64_t* positions, hipStream_t s) {
    k_count_le<<<1, 64, 0, s>>>(sorted_deg, n, thresholds, count, positions);
    return hipGetLastError();
}

}  // namespace gatgpu
