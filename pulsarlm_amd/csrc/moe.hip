// Grouped GEMM over experts and the routed-experts MoE block, all on the device with no
// host synchronization.
//
// Counterpart of routed_experts (pulsarlm-core/src/engine/model/paged_forward.cpp:108-130):
//   stable argsort of the (token, k) assignments by expert, counts, int32 inclusive-end
//   offsets (at::cumsum), gathered rows, at::_grouped_mm(rows, gate_up^T, offsets),
//   act(g) * u, at::_grouped_mm(..., down^T, offsets), x top weight, index_add_ into [T, H].
// Here the experts are int4 (plm layout) and the GEMMs are the grouped MFMA kernel:
// * sort: a counting sort in three small kernels -- per-chunk histograms, a per-expert
//   scan over chunks, and a scatter in which each assignment's rank among the earlier
//   assignments of its expert in its chunk is counted directly -- stable and
//   deterministic, unlike the atomics of a GPU index_add_;
// * the gate_up GEMM gathers its A rows through the sorted token index instead of
//   materializing the gathered rows;
// * the scatter-back is a gather: each token sums its top_k weighted expert outputs in k
//   order in fp32 and rounds once, so the result does not depend on scheduling.
#include <algorithm>
#include <cstdlib>

#include "plm_common.hpp"

namespace plm {

int launch_grouped(const char* op, plm_format f, const void* x, bool bf16, const void* w, const void* scale,
                   plm_dtype scale_dtype, int64_t rows, int64_t n, int64_t k, int64_t block_n, int64_t group_size,
                   void* y, const int32_t* tiles, int64_t max_tiles, const int32_t* tile_count, const int32_t* row_index,
                   int shape,
                   hipStream_t s, bool swiglu);
int grouped_block_rows(int shape);
int grouped_shape_for(int64_t rows, int64_t n_experts);

namespace {

constexpr int kChunk = 256;  // assignments per sort chunk

// Per-chunk expert histogram: counts[chunk][e].
__global__ void __launch_bounds__(kChunk) moe_hist_kernel(const int32_t* __restrict__ experts, int64_t total,
                                                          int n_experts, int32_t* __restrict__ counts) {
    extern __shared__ int32_t hist[];
    for (int e = threadIdx.x; e < n_experts; e += kChunk) hist[e] = 0;
    __syncthreads();
    const int64_t a = static_cast<int64_t>(blockIdx.x) * kChunk + threadIdx.x;
    if (a < total) {
        const int e = experts[a];
        if (e >= 0 && e < n_experts) atomicAdd(&hist[e], 1);  // integer counts: order does not matter
    }
    __syncthreads();
    for (int e = threadIdx.x; e < n_experts; e += kChunk) counts[static_cast<int64_t>(blockIdx.x) * n_experts + e] = hist[e];
}

// Exclusive scan of v[0..n) into v (in place) by one workgroup of 1024 threads; returns the
// total in every thread. `buf` holds 1024 ints of LDS.
__device__ int32_t block_exclusive_scan(int32_t* v, int n, int32_t* buf) {
    int32_t carry = 0;
    for (int base = 0; base < n; base += 1024) {
        const int i = base + threadIdx.x;
        const int32_t x = i < n ? v[i] : 0;
        buf[threadIdx.x] = x;
        __syncthreads();
        for (int d = 1; d < 1024; d <<= 1) {  // Hillis-Steele inclusive scan
            const int32_t y = threadIdx.x >= static_cast<unsigned>(d) ? buf[threadIdx.x - d] : 0;
            __syncthreads();
            buf[threadIdx.x] += y;
            __syncthreads();
        }
        if (i < n) v[i] = carry + buf[threadIdx.x] - x;
        carry += buf[1023];
        __syncthreads();
    }
    return carry;
}

// Per expert (one workgroup each): exclusive scan of its chunk counts, in place, and the
// expert's total.
__global__ void __launch_bounds__(1024) moe_scan_chunks_kernel(int32_t* __restrict__ counts, int n_chunks,
                                                                int n_experts, int32_t* __restrict__ totals) {
    __shared__ int32_t buf[1024];
    __shared__ int32_t col[4096];
    const int e = blockIdx.x;
    int32_t carry = 0;
    for (int base = 0; base < n_chunks; base += 4096) {
        const int len = min(4096, n_chunks - base);
        for (int c = threadIdx.x; c < len; c += 1024) col[c] = counts[static_cast<int64_t>(base + c) * n_experts + e];
        __syncthreads();
        const int32_t tot = block_exclusive_scan(col, len, buf);
        for (int c = threadIdx.x; c < len; c += 1024)
            counts[static_cast<int64_t>(base + c) * n_experts + e] = carry + col[c];
        carry += tot;
        __syncthreads();
    }
    if (threadIdx.x == 0) totals[e] = carry;
}

// Start rows (exclusive scan over experts) and the inclusive-end offsets at::cumsum gives.
__global__ void __launch_bounds__(1024) moe_scan_experts_kernel(const int32_t* __restrict__ totals, int n_experts,
                                                                 int32_t* __restrict__ start,
                                                                 int32_t* __restrict__ offsets) {
    __shared__ int32_t buf[1024];
    __shared__ int32_t v[4096];
    for (int e = threadIdx.x; e < n_experts; e += 1024) v[e] = totals[e];
    __syncthreads();
    block_exclusive_scan(v, n_experts, buf);
    for (int e = threadIdx.x; e < n_experts; e += 1024) {
        start[e] = v[e];
        offsets[e] = v[e] + totals[e];
    }
}

// Scatter: sorted position of every assignment, the token it reads and its weight.
__global__ void __launch_bounds__(kChunk) moe_scatter_kernel(const int32_t* __restrict__ experts,
                                                             const float* __restrict__ weights, int64_t total, int top_k,
                                                             int n_experts, const int32_t* __restrict__ chunk_base,
                                                             const int32_t* __restrict__ start,
                                                             int32_t* __restrict__ sorted_token,
                                                             float* __restrict__ sorted_weight,
                                                             int32_t* __restrict__ position) {
    __shared__ int32_t chunk_experts[kChunk];
    const int64_t a = static_cast<int64_t>(blockIdx.x) * kChunk + threadIdx.x;
    const int e = a < total ? experts[a] : -1;
    chunk_experts[threadIdx.x] = e;
    __syncthreads();
    if (a >= total) return;
    if (e < 0 || e >= n_experts) {  // dropped: the combine skips it
        position[a] = -1;
        return;
    }
    int rank = 0;
    for (int j = 0; j < static_cast<int>(threadIdx.x); ++j) rank += chunk_experts[j] == e;
    const int32_t pos = start[e] + chunk_base[static_cast<int64_t>(blockIdx.x) * n_experts + e] + rank;
    sorted_token[pos] = static_cast<int32_t>(a / top_k);
    sorted_weight[pos] = weights[a];
    position[a] = pos;
}

// Expert e's rows [lo, hi) from caller-supplied inclusive-end offsets, clamped to
// [0, rows] and to hi >= lo, so offsets that are not a non-decreasing cumsum ending at
// `rows` cannot send tiles past the rows the caller sized x, y and the tile slots for.
__device__ __forceinline__ void expert_rows(const int32_t* __restrict__ offsets, int e, int32_t rows, int32_t& lo,
                                            int32_t& hi) {
    lo = e == 0 ? 0 : min(max(offsets[e - 1], 0), rows);
    hi = max(min(max(offsets[e], 0), rows), lo);
}

// Tile list for the grouped GEMM: expert e's rows [off[e-1], off[e]) in blocks of bm,
// written at the expert's tile prefix; slots past the last tile get rows = 0.
__global__ void __launch_bounds__(1024) moe_tiles_kernel(const int32_t* __restrict__ offsets, int n_experts,
                                                          int32_t rows, int bm, int64_t max_tiles,
                                                          int32_t* __restrict__ tiles, int32_t* __restrict__ count) {
    __shared__ int32_t buf[1024];
    __shared__ int32_t first_tile[4096];
    for (int e = threadIdx.x; e < n_experts; e += 1024) {
        int32_t lo, hi;
        expert_rows(offsets, e, rows, lo, hi);
        first_tile[e] = (hi - lo + bm - 1) / bm;
    }
    __syncthreads();
    const int32_t n_tiles = block_exclusive_scan(first_tile, n_experts, buf);
    if (threadIdx.x == 0) *count = static_cast<int32_t>(min<int64_t>(n_tiles, max_tiles));
    for (int e = threadIdx.x; e < n_experts; e += blockDim.x) {
        int32_t lo, hi;
        expert_rows(offsets, e, rows, lo, hi);
        int32_t t = first_tile[e];
        for (int32_t r = lo; r < hi && t < max_tiles; r += bm, ++t) {
            tiles[3 * t] = e;
            tiles[3 * t + 1] = r;
            tiles[3 * t + 2] = min(bm, hi - r);
        }
    }
    for (int64_t t = n_tiles + threadIdx.x; t < max_tiles; t += blockDim.x) {
        tiles[3 * t] = 0;
        tiles[3 * t + 1] = 0;
        tiles[3 * t + 2] = 0;
    }
}

// Sort, offsets and single-level tile list in one workgroup, for small batches: the same
// results as moe_hist/scan/scatter/tiles above (a stable sort by expert), in one launch
// instead of five. The assignments are split into 64-row chunks; the wavefront that owns a
// chunk ranks each assignment among the chunk's earlier ones with the same expert (one
// ballot per bit of the expert id) and writes the per-(expert, chunk) count into an
// expert-major LDS table. One exclusive scan of that table gives each (expert, chunk) its
// first sorted row, so an assignment's row is that base plus its rank.
constexpr int kSmallSortTable = 16384;  // experts x chunks held in LDS
constexpr int kSmallSortChunks = 128;   // chunks (8 per wavefront), so rows <= 8192

__global__ void __launch_bounds__(1024) moe_sort_small_kernel(
    const int32_t* __restrict__ experts, const float* __restrict__ weights, int rows, int top_k, int n_experts,
    int n_chunks, int bm, int64_t max_tiles, int32_t* __restrict__ sorted_token, float* __restrict__ sorted_weight,
    int32_t* __restrict__ position, int32_t* __restrict__ offsets, int32_t* __restrict__ tiles,
    int32_t* __restrict__ count) {
    __shared__ int32_t tab[kSmallSortTable];
    __shared__ int32_t buf[1024];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = n_experts * n_chunks;
    for (int i = tid; i < n; i += 1024) tab[i] = 0;
    __syncthreads();

    constexpr int kPerWave = kSmallSortChunks / 16;
    const uint64_t lanes_below = (uint64_t{1} << lane) - 1;
    int ex[kPerWave], rk[kPerWave];
    float wt[kPerWave];
#pragma unroll
    for (int j = 0; j < kPerWave; ++j) {  // all loads first: one latency, not one per chunk
        const int c = wave + 16 * j;
        const int a = c * 64 + lane;
        const bool in = c < n_chunks && a < rows;
        ex[j] = in ? experts[a] : -1;
        wt[j] = in ? weights[a] : 0.f;
    }
    // Lanes with the same expert: AND over the expert id's bits of that bit's ballot or its
    // complement (one ballot per bit instead of one pass per distinct expert).
    const int id_bits = 32 - __clz(max(n_experts - 1, 1));
#pragma unroll
    for (int j = 0; j < kPerWave; ++j) {
        const int c = wave + 16 * j;
        int e = ex[j];
        if (e >= n_experts) e = -1;  // out-of-range experts are skipped, as by the histogram
        uint64_t same = __ballot(e >= 0);
        if (same == 0) {  // wave-uniform: no assignment in this chunk
            ex[j] = -1;
            rk[j] = 0;
            continue;
        }
        for (int b = 0; b < id_bits; ++b) {  // wave-uniform
            const bool bit = (e >> b) & 1;
            const uint64_t plane = __ballot(bit);
            same &= bit ? plane : ~plane;
        }
        const int rank = __popcll(same & lanes_below);
        if (e >= 0 && rank == 0) tab[e * n_chunks + c] = __popcll(same);
        ex[j] = e;
        rk[j] = rank;
    }
    __syncthreads();

    // Exclusive scan of tab: P consecutive entries per thread, then across threads.
    const int per = (n + 1023) / 1024;
    int32_t local = 0;
    for (int q = 0; q < per; ++q) {
        const int i = tid * per + q;
        if (i < n) local += tab[i];
    }
    buf[tid] = local;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {
        const int32_t y = tid >= d ? buf[tid - d] : 0;
        __syncthreads();
        buf[tid] += y;
        __syncthreads();
    }
    const int32_t total = buf[1023];
    int32_t run = buf[tid] - local;
    for (int q = 0; q < per; ++q) {
        const int i = tid * per + q;
        if (i < n) {
            const int32_t v = tab[i];
            tab[i] = run;
            run += v;
        }
    }
    __syncthreads();

    // Inclusive-end offsets (the next expert's first row), and each expert's tile count.
    constexpr int kExpertsPerThread = 4096 / 1024;
    int32_t lo[kExpertsPerThread], hi[kExpertsPerThread];
#pragma unroll
    for (int q = 0; q < kExpertsPerThread; ++q) {
        const int e = tid + 1024 * q;
        lo[q] = hi[q] = 0;
        if (e < n_experts) {
            lo[q] = tab[e * n_chunks];
            hi[q] = e + 1 < n_experts ? tab[(e + 1) * n_chunks] : total;
            offsets[e] = hi[q];
        }
    }
#pragma unroll
    for (int j = 0; j < kPerWave; ++j) {
        const int c = wave + 16 * j;
        const int a = c * 64 + lane;
        if (ex[j] < 0) {  // dropped (out-of-range expert): the combine skips it
            if (c < n_chunks && a < rows) position[a] = -1;
            continue;
        }
        const int32_t pos = tab[ex[j] * n_chunks + c] + rk[j];
        sorted_token[pos] = a / top_k;
        sorted_weight[pos] = wt[j];
        position[a] = pos;
    }
    __syncthreads();  // tab is reused for the tile prefix below

#pragma unroll
    for (int q = 0; q < kExpertsPerThread; ++q) {
        const int e = tid + 1024 * q;
        if (e < n_experts) tab[e] = (hi[q] - lo[q] + bm - 1) / bm;
    }
    __syncthreads();
    const int32_t n_tiles = block_exclusive_scan(tab, n_experts, buf);
    if (tid == 0) *count = static_cast<int32_t>(min<int64_t>(n_tiles, max_tiles));
#pragma unroll
    for (int q = 0; q < kExpertsPerThread; ++q) {
        const int e = tid + 1024 * q;
        if (e >= n_experts) continue;
        int32_t t = tab[e];
        for (int32_t r = lo[q]; r < hi[q]; r += bm, ++t) {
            tiles[3 * t] = e;
            tiles[3 * t + 1] = r;
            tiles[3 * t + 2] = min(bm, hi[q] - r);
        }
    }
    for (int64_t t = n_tiles + tid; t < max_tiles; t += 1024) {
        tiles[3 * t] = 0;
        tiles[3 * t + 1] = 0;
        tiles[3 * t + 2] = 0;
    }
}

// Two-level tile lists for skewed groups: expert e's rows in full blocks of `bb` rows (a
// last block of at least `full` rows counts as full) go to `big`, the remaining rows
// (< full) to `small` in blocks of `sb`, so a heavily routed expert's weights are read once
// per big block instead of once per small one. Slots past the last tile get rows = 0.
__device__ __forceinline__ void tiles2_split(int32_t c, int bb, int full, int32_t& nbig, int32_t& rem) {
    nbig = c / bb;
    rem = c - nbig * bb;
    if (rem >= full) ++nbig, rem = 0;
}

__global__ void __launch_bounds__(1024) moe_tiles2_kernel(const int32_t* __restrict__ offsets, int n_experts,
                                                           int32_t rows, int bb, int sb, int full, int64_t max_big,
                                                           int64_t max_small, int32_t* __restrict__ big,
                                                           int32_t* __restrict__ small, int32_t* __restrict__ counts) {
    __shared__ int32_t buf[1024];
    __shared__ int32_t first_big[4096];
    __shared__ int32_t first_small[4096];
    for (int e = threadIdx.x; e < n_experts; e += 1024) {
        int32_t nbig, rem, lo, hi;
        expert_rows(offsets, e, rows, lo, hi);
        tiles2_split(hi - lo, bb, full, nbig, rem);
        first_big[e] = nbig;
        first_small[e] = (rem + sb - 1) / sb;
    }
    __syncthreads();
    const int32_t n_big = block_exclusive_scan(first_big, n_experts, buf);
    const int32_t n_small = block_exclusive_scan(first_small, n_experts, buf);
    if (threadIdx.x == 0) {
        counts[0] = static_cast<int32_t>(min<int64_t>(n_big, max_big));
        counts[1] = static_cast<int32_t>(min<int64_t>(n_small, max_small));
    }
    for (int e = threadIdx.x; e < n_experts; e += blockDim.x) {
        int32_t nbig, rem, lo, hi;
        expert_rows(offsets, e, rows, lo, hi);
        tiles2_split(hi - lo, bb, full, nbig, rem);
        int32_t r = lo, t = first_big[e];
        for (int b = 0; b < nbig && t < max_big; ++b, ++t, r += bb) {
            big[3 * t] = e;
            big[3 * t + 1] = r;
            big[3 * t + 2] = min(bb, hi - r);
        }
        r = lo + nbig * bb;  // where the big blocks end, also when their slots ran out
        t = first_small[e];
        for (; r < hi && t < max_small; r += sb, ++t) {
            small[3 * t] = e;
            small[3 * t + 1] = r;
            small[3 * t + 2] = min(sb, hi - r);
        }
    }
    for (int64_t t = n_big + threadIdx.x; t < max_big; t += blockDim.x) big[3 * t + 2] = 0;
    for (int64_t t = n_small + threadIdx.x; t < max_small; t += blockDim.x) small[3 * t + 2] = 0;
}

// act[r, i] = round(round(silu(g)) * u) with (g | u) = gu[r, :] (the reference's
// at::silu(gate) * up in the activation dtype). Eight values per thread (16-byte loads and
// stores; inter % 8 == 0 is checked by the caller).
template <bool BF16>
__global__ void __launch_bounds__(256) silu_mul_kernel(const uint16_t* __restrict__ gu, int64_t rows, int inter,
                                                       uint16_t* __restrict__ act) {
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
    if (i >= rows * inter) return;
    const int64_t r = i / inter, c = i % inter;
    const u32x4_t g = *reinterpret_cast<const u32x4_t*>(gu + r * 2 * inter + c);
    const u32x4_t u = *reinterpret_cast<const u32x4_t*>(gu + r * 2 * inter + inter + c);
    u32x4_t o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float v[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float gv = from_bits16<BF16>((g[q] >> (16 * h)) & 0xffffu);
            const float uv = from_bits16<BF16>((u[q] >> (16 * h)) & 0xffffu);
            v[h] = silu_times<BF16>(gv, uv);
        }
        o[q] = pack2<BF16>(v[0], v[1]);
    }
    *reinterpret_cast<u32x4_t*>(act + i) = o;
}

// out[t, h] = sum_j round(d[pos(t, j), h] * round(w[t, j])), summed in j order in fp32.
// One workgroup per token (its positions and weights are wave-uniform); eight consecutive
// h per thread (hidden % 8 == 0 is checked by the caller).
template <bool BF16>
__global__ void __launch_bounds__(256) moe_combine_kernel(const uint16_t* __restrict__ d,
                                                          const int32_t* __restrict__ position,
                                                          const float* __restrict__ weights, int top_k, int hidden,
                                                          uint16_t* __restrict__ out) {
    const int64_t t = blockIdx.x;
    const int h = (blockIdx.y * blockDim.x + threadIdx.x) * 8;
    if (h >= hidden) return;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < top_k; ++j) {
        const int32_t p = position[t * top_k + j];
        if (p < 0) continue;  // an assignment to an expert id outside [0, n_experts)
        const float w = round_to<BF16>(weights[t * top_k + j]);
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(d + static_cast<int64_t>(p) * hidden + h);
#pragma unroll
        for (int q = 0; q < 8; ++q)
            acc[q] += round_to<BF16>(from_bits16<BF16>((v[q / 2] >> (16 * (q % 2))) & 0xffffu) * w);
    }
    u32x4_t o;
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = pack2<BF16>(acc[2 * q], acc[2 * q + 1]);
    *reinterpret_cast<u32x4_t*>(out + t * hidden + h) = o;
}

struct moe_ws {
    int64_t counts, totals, start, sorted_token, sorted_weight, position, tiles, gu, act, d, total;
};

int64_t align256(int64_t v) { return round_up(v, 256); }

moe_ws moe_layout(int64_t tokens, int64_t top_k, int64_t n_experts, int64_t hidden, int64_t inter, int64_t max_tiles) {
    const int64_t rows = tokens * top_k;
    const int64_t chunks = ceil_div(rows, kChunk);
    moe_ws w{};
    int64_t off = kCounterBytes;  // the split-K counter region stays at the front
    auto take = [&](int64_t bytes) {
        const int64_t at = off;
        off += align256(std::max<int64_t>(bytes, 1));
        return at;
    };
    w.counts = take(chunks * n_experts * 4);
    w.totals = take(n_experts * 4);
    w.start = take(n_experts * 4);
    w.sorted_token = take(rows * 4);
    w.sorted_weight = take(rows * 4);
    w.position = take(rows * 4);
    w.tiles = take(max_tiles * 12 + 8);  // the tile lists, then their tile counts
    w.gu = take(rows * 2 * inter * 2);
    w.act = take(rows * inter * 2);
    w.d = take(rows * hidden * 2);
    w.total = off;
    return w;
}

// How a grouped GEMM over `rows` sorted rows is tiled. With many rows per expert (skewed
// routing at large batch), full 256-row blocks run on the 256 x 256 shape and the rest on
// 64-row tiles (two launches); otherwise one shape sized to the average rows per expert.
// (At T = 256 of the Zipf-routed benchmark block, 64-row blocks for the heavy experts and
// 16-row tiles for the rest measured slower than 16-row tiles throughout: the repeated
// weight reads of a heavy expert's concurrent tiles hit in L2.)
struct grouped_plan {
    bool two;
    int shape, shape_b;   // shapes of the first and second list
    int bb, sb, full;     // two lists: big and small block rows, rows that count as a full big block
    int64_t max_a, max_b;  // tile slots of the first and second list
    int64_t slots() const { return max_a + max_b; }
    // The tile lists' real tile counts (list a, list b) follow the lists: int32 index.
    int64_t count_at() const { return 3 * slots(); }
};

grouped_plan plan_grouped(int64_t rows, int64_t n_experts) {
    grouped_plan p{};
    p.two = rows >= 128 * n_experts;
    if (p.two) {
        // 256 x 256 blocks on 8 wavefronts of 256 x 32 (each strip dequantized once; 1-2 %
        // faster at T = 4096 than the 2 x 4 wavefront grid), then 64-row tiles.
        p.shape = 6, p.shape_b = 1;
        p.bb = 256, p.sb = 64, p.full = 192;
    }
    if (p.two) {
        p.max_a = rows / p.full + 1;
        // Each expert leaves fewer than `full` rows, in at most ceil(full / sb) small tiles, and
        // the small tiles hold all remaining rows plus at most one partial tile per expert.
        p.max_b = std::min<int64_t>(ceil_div(p.full, p.sb) * n_experts, ceil_div(rows, p.sb) + n_experts);
    } else {
        p.shape = grouped_shape_for(rows, n_experts);
        p.max_a = ceil_div(rows, grouped_block_rows(p.shape)) + n_experts;
    }
    return p;
}

bool small_sort_enabled() { return !knobs().moe_small_sort_off; }  // PLM_MOE_SMALL_SORT=0 (A/B)

int64_t moe_max_tiles(int64_t rows, int64_t n_experts) { return plan_grouped(rows, n_experts).slots(); }

int launch_sort(const char* op, const int32_t* experts, const float* weights, int64_t rows, int64_t top_k,
                int64_t n_experts, uint8_t* base, const moe_ws& l, int32_t* offsets, hipStream_t s) {
    const int64_t chunks = ceil_div(rows, kChunk);
    auto* counts = reinterpret_cast<int32_t*>(base + l.counts);
    auto* start = reinterpret_cast<int32_t*>(base + l.start);
    const size_t hist_lds = static_cast<size_t>(n_experts) * 4;
    moe_hist_kernel<<<static_cast<unsigned>(chunks), kChunk, hist_lds, s>>>(experts, rows, int(n_experts), counts);
    auto* totals = reinterpret_cast<int32_t*>(base + l.totals);
    moe_scan_chunks_kernel<<<static_cast<unsigned>(n_experts), 1024, 0, s>>>(counts, int(chunks), int(n_experts),
                                                                             totals);
    moe_scan_experts_kernel<<<1, 1024, 0, s>>>(totals, int(n_experts), start, offsets);
    moe_scatter_kernel<<<static_cast<unsigned>(chunks), kChunk, 0, s>>>(
        experts, weights, rows, int(top_k), int(n_experts), counts, start,
        reinterpret_cast<int32_t*>(base + l.sorted_token), reinterpret_cast<float*>(base + l.sorted_weight),
        reinterpret_cast<int32_t*>(base + l.position));
    PLM_HIP_LAUNCH_CHECK(op);
    return PLM_OK;
}

int launch_tiles(const char* op, const int32_t* offsets, int64_t n_experts, int64_t rows, const grouped_plan& p,
                 int32_t* tiles, hipStream_t s) {
    if (p.two)
        moe_tiles2_kernel<<<1, 1024, 0, s>>>(offsets, int(n_experts), int32_t(rows), p.bb, p.sb, p.full, p.max_a, p.max_b, tiles,
                                             tiles + 3 * p.max_a, tiles + p.count_at());
    else
        moe_tiles_kernel<<<1, 1024, 0, s>>>(offsets, int(n_experts), int32_t(rows), grouped_block_rows(p.shape),
                                            p.max_a, tiles, tiles + p.count_at());
    PLM_HIP_LAUNCH_CHECK(op);
    return PLM_OK;
}

int launch_plan(const char* op, const grouped_plan& p, const void* x, bool bf16, const void* w, const void* scale,
                plm_dtype scale_dtype, int64_t rows, int64_t n, int64_t k, int64_t block_n, int64_t group_size,
                void* y, const int32_t* tiles, const int32_t* row_index, hipStream_t s, bool swiglu = false) {
    if (int rc = launch_grouped(op, PLM_INT4, x, bf16, w, scale, scale_dtype, rows, n, k, block_n, group_size, y,
                                tiles, p.max_a, tiles + p.count_at(), row_index, p.shape, s, swiglu))
        return rc;
    if (!p.two) return PLM_OK;
    return launch_grouped(op, PLM_INT4, x, bf16, w, scale, scale_dtype, rows, n, k, block_n, group_size, y,
                          tiles + 3 * p.max_a, p.max_b, tiles + p.count_at() + 1, row_index, p.shape_b, s, swiglu);
}

bool fused_swiglu_off() { return knobs().moe_unfused; }  // PLM_MOE_UNFUSED (A/B: separate silu_mul)

}  // namespace
}  // namespace plm

using namespace plm;

extern "C" {

int plm_grouped_gemm(plm_format format, const void* x, plm_dtype x_dtype, const void* weight, const void* scale,
                     plm_dtype scale_dtype, const int32_t* offsets, int64_t n_experts, int64_t rows, int64_t n,
                     int64_t k, int64_t block_n, int64_t group_size, void* y, void* workspace,
                     size_t workspace_bytes, void* stream) {
    const char* op = "grouped_gemm";
    clear_error();
    PLM_CHECK_ARG(format == PLM_INT4 || format == PLM_FP8, op, "unknown weight format");
    PLM_CHECK_ARG(x_dtype == PLM_BF16 || x_dtype == PLM_FP16, op, "x must be fp16 or bf16");
    PLM_CHECK_ARG(scale_dtype == PLM_BF16 || scale_dtype == PLM_FP16 || scale_dtype == PLM_FP32, op,
                  "scale dtype must be bf16, fp16 or fp32");
    PLM_CHECK_ARG(n_experts > 0 && n_experts <= 4096, op, "n_experts must be in [1, 4096]");
    PLM_CHECK_ARG(rows >= 0 && n >= 0 && k >= 0 && block_n > 0, op, "bad sizes");
    PLM_CHECK_ARG(group_size > 0 && group_size % 16 == 0 && k % group_size == 0, op,
                  "group_size must be a positive multiple of 16 dividing K");
    if (rows == 0 || n == 0) return PLM_OK;
    PLM_CHECK_ARG(x && weight && scale && offsets && y, op, "null pointer");
    PLM_CHECK_ARG(aligned(x, 16) && aligned(weight, 16), op, "x and weight must be 16-byte aligned");
    PLM_CHECK_ARG(format == PLM_INT4, op, "grouped GEMMs take int4 experts");
    const grouped_plan p = plan_grouped(rows, n_experts);
    const int64_t need = kCounterBytes + p.slots() * 12 + 8;
    if (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < need) {
        set_error(op, "workspace of %lld bytes required, %zu given", static_cast<long long>(need), workspace_bytes);
        return PLM_ERR_WORKSPACE;
    }
    auto* tiles = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(workspace) + kCounterBytes);
    hipStream_t s = as_stream(stream);
    if (int rc = launch_tiles(op, offsets, n_experts, rows, p, tiles, s)) return rc;
    return launch_plan(op, p, x, x_dtype == PLM_BF16, weight, scale, scale_dtype, rows, n, k, block_n, group_size, y,
                       tiles, nullptr, s);
}

int64_t plm_grouped_gemm_workspace_bytes(int64_t rows, int64_t n_experts) {
    if (rows <= 0 || n_experts <= 0) return kCounterBytes;
    return kCounterBytes + plan_grouped(rows, n_experts).slots() * 12 + 8;
}

int64_t plm_moe_workspace_bytes(int64_t tokens, int64_t top_k, int64_t n_experts, int64_t hidden,
                                int64_t intermediate) {
    if (tokens <= 0 || top_k <= 0 || n_experts <= 0) return kCounterBytes;
    const int64_t rows = tokens * top_k;
    return moe_layout(tokens, top_k, n_experts, hidden, intermediate, moe_max_tiles(rows, n_experts)).total;
}

int plm_moe(const void* h, plm_dtype dtype, const int32_t* top_experts, const float* top_weights, int64_t tokens,
            int64_t top_k, int64_t n_experts, int64_t hidden, int64_t intermediate, const void* gate_up_weight,
            const void* gate_up_scale, const void* down_weight, const void* down_scale, plm_dtype scale_dtype,
            int64_t group_size, int32_t* offsets, void* out, void* workspace, size_t workspace_bytes, void* stream) {
    const char* op = "routed_experts";
    clear_error();
    PLM_CHECK_ARG(dtype == PLM_BF16 || dtype == PLM_FP16, op, "h must be fp16 or bf16");
    PLM_CHECK_ARG(scale_dtype == PLM_BF16 || scale_dtype == PLM_FP16 || scale_dtype == PLM_FP32, op,
                  "scale dtype must be bf16, fp16 or fp32");
    PLM_CHECK_ARG(tokens >= 0 && top_k > 0 && n_experts > 0 && n_experts <= 4096, op, "bad routing sizes");
    PLM_CHECK_ARG(hidden > 0 && intermediate > 0, op, "hidden and intermediate must be positive");
    PLM_CHECK_ARG(group_size > 0 && group_size % 16 == 0 && hidden % group_size == 0 && intermediate % group_size == 0,
                  op, "group_size must be a positive multiple of 16 dividing hidden and intermediate");
    PLM_CHECK_ARG(tokens * top_k <= (int64_t{1} << 30), op, "too many assignments");
    PLM_CHECK_ARG(hidden % 8 == 0 && intermediate % 8 == 0, op, "hidden and intermediate must be multiples of 8");
    PLM_CHECK_ARG(aligned(h, 16) && aligned(out, 16) && aligned(workspace, 16), op,
                  "h, out and workspace must be 16-byte aligned");
    if (tokens == 0) return PLM_OK;
    PLM_CHECK_ARG(h && top_experts && top_weights && gate_up_weight && gate_up_scale && down_weight && down_scale &&
                      offsets && out,
                  op, "null pointer");
    const int64_t rows = tokens * top_k;
    const grouped_plan p = plan_grouped(rows, n_experts);
    const moe_ws l = moe_layout(tokens, top_k, n_experts, hidden, intermediate, p.slots());
    if (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < l.total) {
        set_error(op, "workspace of %lld bytes required, %zu given", static_cast<long long>(l.total), workspace_bytes);
        return PLM_ERR_WORKSPACE;
    }
    auto* base = static_cast<uint8_t*>(workspace);
    hipStream_t s = as_stream(stream);
    const bool bf16 = dtype == PLM_BF16;
    auto* tiles = reinterpret_cast<int32_t*>(base + l.tiles);
    const int64_t chunks64 = ceil_div(rows, 64);
    if (!p.two && chunks64 <= kSmallSortChunks && n_experts * chunks64 <= kSmallSortTable && small_sort_enabled()) {
        moe_sort_small_kernel<<<1, 1024, 0, s>>>(
            top_experts, top_weights, int(rows), int(top_k), int(n_experts), int(chunks64),
            grouped_block_rows(p.shape), p.max_a, reinterpret_cast<int32_t*>(base + l.sorted_token),
            reinterpret_cast<float*>(base + l.sorted_weight), reinterpret_cast<int32_t*>(base + l.position), offsets,
            tiles, tiles + p.count_at());
        PLM_HIP_LAUNCH_CHECK(op);
    } else {
        if (int rc = launch_sort(op, top_experts, top_weights, rows, top_k, n_experts, base, l, offsets, s)) return rc;
        if (int rc = launch_tiles(op, offsets, n_experts, rows, p, tiles, s)) return rc;
    }
    if (intermediate % kTileN == 0 && !fused_swiglu_off()) {
        // gate_up with the activation in its epilogue: act [rows, I] = silu(g) * u directly.
        if (int rc = launch_plan(op, p, h, bf16, gate_up_weight, gate_up_scale, scale_dtype, rows, 2 * intermediate,
                                 hidden, 1, group_size, base + l.act, tiles,
                                 reinterpret_cast<const int32_t*>(base + l.sorted_token), s, true))
            return rc;
    } else {
        // gate_up: [rows, 2I] = h[sorted_token] @ gate_up_e^T, then the activation.
        if (int rc = launch_plan(op, p, h, bf16, gate_up_weight, gate_up_scale, scale_dtype, rows, 2 * intermediate,
                                 hidden, 1, group_size, base + l.gu, tiles,
                                 reinterpret_cast<const int32_t*>(base + l.sorted_token), s))
            return rc;
        const int64_t act_n = rows * intermediate;
        const unsigned act_blocks = static_cast<unsigned>(ceil_div(act_n / 8, 256));
        if (bf16)
            silu_mul_kernel<true><<<act_blocks, 256, 0, s>>>(
                reinterpret_cast<const uint16_t*>(base + l.gu), rows, int(intermediate),
                reinterpret_cast<uint16_t*>(base + l.act));
        else
            silu_mul_kernel<false><<<act_blocks, 256, 0, s>>>(
                reinterpret_cast<const uint16_t*>(base + l.gu), rows, int(intermediate),
                reinterpret_cast<uint16_t*>(base + l.act));
        PLM_HIP_LAUNCH_CHECK(op);
    }
    // down: [rows, H] = act @ down_e^T
    if (int rc = launch_plan(op, p, base + l.act, bf16, down_weight, down_scale, scale_dtype, rows, hidden,
                             intermediate, 1, group_size, base + l.d, tiles, nullptr, s))
        return rc;
    const dim3 cgrid(static_cast<unsigned>(tokens), static_cast<unsigned>(ceil_div(hidden / 8, 256)));
    if (bf16)
        moe_combine_kernel<true><<<cgrid, 256, 0, s>>>(
            reinterpret_cast<const uint16_t*>(base + l.d), reinterpret_cast<const int32_t*>(base + l.position),
            top_weights, int(top_k), int(hidden), static_cast<uint16_t*>(out));
    else
        moe_combine_kernel<false><<<cgrid, 256, 0, s>>>(
            reinterpret_cast<const uint16_t*>(base + l.d), reinterpret_cast<const int32_t*>(base + l.position),
            top_weights, int(top_k), int(hidden), static_cast<uint16_t*>(out));
    PLM_HIP_LAUNCH_CHECK(op);
    return PLM_OK;
}

}  // extern "C"
