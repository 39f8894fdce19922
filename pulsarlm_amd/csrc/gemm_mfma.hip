// MFMA dequant-GEMM for M > 16 (prefill): y[M, N] = x[M, K] @ dequant(W)^T.
//
// Counterpart of the reference's marlin_kernel at tile_m = 64 (pulsarlm-core/src/kernels/
// marlin.cu:251-389; dispatch :577-596) and its split-K combine
// (pulsarlm-core/inc/pulsarlm/kernels/dequant_gemm_common.cuh:99-133).
//
// gfx950 design:
// * Workgroup tile BM x 128 columns x 128-wide K steps; four wavefronts in a 2 x 2
//   grid, each owning (BM/2) x 64 outputs as 16 x 16 tiles of v_mfma_f32_16x16x32.
// * The x tile (bf16/fp16) and the packed weight tiles (1 KiB int4 / 2 KiB fp8 per
//   16-column strip, copied verbatim from the plm layout) are staged through LDS,
//   double buffered, with the next K step's global loads in flight during the
//   current step's MFMAs.
// * Each wavefront dequantizes its strips in registers to round(q * round(s)),
//   bit-identical to the reference's fragment values (marlin.cu:123-151,180-194),
//   with the shared dq_int4 / dq_fp8 sequences.
// * Split-K across workgroups when the output has too few tiles to fill the GPU,
//   reduced deterministically by the last workgroup to arrive.
#include <type_traits>

#include "plm_common.hpp"

namespace plm {

namespace {

constexpr int kWaves = 4;
constexpr int kBN = 128;                  // 8 strips
constexpr int kStrips = kBN / kTileN;     // 8
constexpr int kARowBytes = kTileK * 2 + 16;  // padded LDS row: 128 halves + 16 B

struct mfma_args {
    const uint16_t* x;
    const uint8_t* w;
    const void* scale;
    uint16_t* y;
    float* partial;
    uint32_t* counters;
    int scale_dtype, scale_cols;
    int m, n, k;
    int ktiles, strips, groups, group_size;
    int splits, tiles_per_split;
    int m_blocks;
};

template <plm_format F, bool BF16, int BM, bool UNIFORM>
__global__ void __launch_bounds__(kWaves * 64) mfma_kernel(mfma_args a) {
    constexpr int TB = fmt_traits<F>::tile_bytes;
    constexpr int MT = BM / 2 / 16;  // m tiles per wavefront
    constexpr int A_BYTES = BM * kARowBytes;
    constexpr int B_BYTES = kStrips * TB;
    constexpr int A_LOADS = BM * kTileK * 2 / 16 / (kWaves * 64);  // 16-byte loads per thread
    constexpr int B_LOADS = B_BYTES / 16 / (kWaves * 64);
    static_assert(A_LOADS * 16 * kWaves * 64 == BM * kTileK * 2, "A tile split");
    static_assert(B_LOADS * 16 * kWaves * 64 == B_BYTES, "B tile split");

    __shared__ __attribute__((aligned(16))) uint8_t lds[2][A_BYTES + B_BYTES];
    __shared__ uint32_t last_flag;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int col16 = lane & 15, kq = lane >> 4;
    const int mb = blockIdx.x % a.m_blocks;
    const int nb = blockIdx.x / a.m_blocks;
    const int split = blockIdx.y;
    const int m0 = mb * BM;
    const int strip0 = nb * kStrips;
    const int kt_begin = split * a.tiles_per_split;
    const int kt_end = min(kt_begin + a.tiles_per_split, a.ktiles);

    f32x4_t acc[MT][4];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    u32x4_t ra[A_LOADS], rb[B_LOADS];
    auto global_load = [&](int kt) {
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) {
            const int c = tid + i * kWaves * 64;  // 16-byte chunk id: row c/16, K chunk c%16
            const int row = m0 + c / 16;
            const int kk = kt * kTileK + (c % 16) * 8;
            if (row < a.m && kk < a.k)
                ra[i] = *reinterpret_cast<const u32x4_t*>(a.x + static_cast<int64_t>(row) * a.k + kk);
            else
                ra[i] = u32x4_t{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) {
            const int c = tid + i * kWaves * 64;  // chunk within the 8-strip tile group
            const int s = c / (TB / 16);
            const int within = c % (TB / 16);
            const int st = strip0 + s;
            if (st < a.strips)
                rb[i] = *reinterpret_cast<const u32x4_t*>(a.w + (static_cast<int64_t>(st) * a.ktiles + kt) * TB +
                                                          within * 16);
            else
                rb[i] = (F == PLM_INT4) ? u32x4_t{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u}
                                        : u32x4_t{0u, 0u, 0u, 0u};
        }
    };
    auto lds_store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) {
            const int c = tid + i * kWaves * 64;
            *reinterpret_cast<u32x4_t*>(&lds[buf][(c / 16) * kARowBytes + (c % 16) * 16]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) {
            const int c = tid + i * kWaves * 64;
            *reinterpret_cast<u32x4_t*>(&lds[buf][A_BYTES + c * 16]) = rb[i];
        }
    };

    if (kt_begin < kt_end) {
        global_load(kt_begin);
        lds_store(0);
    }
    __syncthreads();

    for (int kt = kt_begin; kt < kt_end; ++kt) {
        const int buf = (kt - kt_begin) & 1;
        if (kt + 1 < kt_end) global_load(kt + 1);

        // Scales of this wavefront's 4 strips (one per tile when the group spans it).
        auto scale_raw = [&](int j, int t) -> float {
            const int g = (kt * kTileK + 32 * t + 8 * kq) / a.group_size;
            const int st = min(strip0 + wn * 4 + j, a.strips - 1);
            const int64_t sidx =
                (static_cast<int64_t>(st) * a.groups + g) * a.scale_cols + (a.scale_cols == 1 ? 0 : col16);
            return load_scale(a.scale, sidx, a.scale_dtype);
        };
        float sr[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) sr[j] = UNIFORM ? scale_raw(j, 0) : 0.f;
        const uint8_t* la = &lds[buf][0];
        const uint8_t* lb = &lds[buf][A_BYTES];
        u32x4_t wv[4][TB / 1024];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int h = 0; h < TB / 1024; ++h)
                wv[j][h] = *reinterpret_cast<const u32x4_t*>(lb + (wn * 4 + j) * TB + h * 1024 + lane * 16);

#pragma unroll
        for (int t = 0; t < 4; ++t) {
            u32x4_t af[MT];
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const int row = wm * (BM / 2) + i * 16 + col16;
                af[i] = *reinterpret_cast<const u32x4_t*>(la + row * kARowBytes + (32 * t + 8 * kq) * 2);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float raw = UNIFORM ? sr[j] : scale_raw(j, t);
                u32x4_t b;
                if constexpr (F == PLM_INT4) {
                    b = dq_int4<BF16>(wv[j][0][t], make_int4_scale<BF16>(raw));
                } else {
                    b = dq_fp8<BF16>(wv[j][t >> 1][(t & 1) * 2], wv[j][t >> 1][(t & 1) * 2 + 1], round_to<BF16>(raw));
                }
#pragma unroll
                for (int i = 0; i < MT; ++i) acc[i][j] = mfma16x16x32<BF16>(af[i], b, acc[i][j]);
            }
        }
        __syncthreads();
        if (kt + 1 < kt_end) lds_store(buf ^ 1);
        __syncthreads();
    }

    // Epilogue: lane holds column col16 of strip (strip0 + wn*4 + j), rows 4*kq + r of m tile i.
    const int64_t mn = static_cast<int64_t>(a.m) * a.n;
    if (a.splits == 1) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int col = (strip0 + wn * 4 + j) * kTileN + col16;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = m0 + wm * (BM / 2) + i * 16 + 4 * kq + r;
                    if (row < a.m && col < a.n)
                        a.y[static_cast<int64_t>(row) * a.n + col] = static_cast<uint16_t>(to_bits16<BF16>(acc[i][j][r]));
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = (strip0 + wn * 4 + j) * kTileN + col16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm * (BM / 2) + i * 16 + 4 * kq + r;
                if (row < a.m && col < a.n)
                    store_partial(&a.partial[split * mn + static_cast<int64_t>(row) * a.n + col], acc[i][j][r]);
            }
        }
    if (!arrive_last(&a.counters[blockIdx.x], static_cast<uint32_t>(a.splits), &last_flag)) return;
    // Sum this tile's partials in split order; threads sweep the BM x 128 tile row-major.
    for (int e = tid; e < BM * kBN; e += kWaves * 64) {
        const int row = m0 + e / kBN;
        const int col = strip0 * kTileN + e % kBN;
        if (row < a.m && col < a.n) {
            const int64_t off = static_cast<int64_t>(row) * a.n + col;
            float s = 0.f;
            for (int sp = 0; sp < a.splits; ++sp) s += load_partial(&a.partial[sp * mn + off]);
            a.y[off] = static_cast<uint16_t>(to_bits16<BF16>(s));
        }
    }
}

struct mfma_config {
    int bm;
    int m_blocks, n_blocks;
    int splits, tiles_per_split;
};

mfma_config choose_mfma(int64_t m, int64_t n, int64_t k) {
    mfma_config c{};
    c.bm = 128;
    c.m_blocks = static_cast<int>(ceil_div(m, c.bm));
    c.n_blocks = static_cast<int>(ceil_div(n, kBN));
    const int64_t ktiles = ceil_div(k, kTileK);
    const int64_t tiles = static_cast<int64_t>(c.m_blocks) * c.n_blocks;
    const int64_t cus = cu_count();
    int64_t splits = 1;
    if (tiles < cus && tiles <= kMaxCounters) splits = std::min<int64_t>(ceil_div(cus, tiles), ktiles);
    c.tiles_per_split = static_cast<int>(ceil_div(ktiles, splits));
    c.splits = static_cast<int>(ceil_div(ktiles, c.tiles_per_split));
    return c;
}

}  // namespace

int64_t mfma_workspace_bytes(plm_format, int64_t m, int64_t n, int64_t k) {
    const mfma_config c = choose_mfma(m, n, k);
    if (c.splits <= 1) return 0;
    return kCounterBytes + static_cast<int64_t>(c.splits) * m * n * 4;
}

int launch_mfma(const char* op, plm_format f, const void* x, bool bf16, const void* w, const void* scale,
                plm_dtype scale_dtype, int64_t m, int64_t n, int64_t k, int64_t block_n, int64_t group_size, void* y,
                void* workspace, size_t workspace_bytes, hipStream_t s) {
    const mfma_config c = choose_mfma(m, n, k);
    const layout_dims d = make_dims(n, k, block_n, group_size);
    mfma_args a{};
    a.x = static_cast<const uint16_t*>(x);
    a.w = static_cast<const uint8_t*>(w);
    a.scale = scale;
    a.y = static_cast<uint16_t*>(y);
    a.scale_dtype = scale_dtype;
    a.scale_cols = d.scale_cols;
    a.m = static_cast<int>(m);
    a.n = static_cast<int>(n);
    a.k = static_cast<int>(k);
    a.ktiles = static_cast<int>(d.ktiles);
    a.strips = static_cast<int>(d.strips);
    a.groups = static_cast<int>(d.groups);
    a.group_size = static_cast<int>(group_size);
    a.splits = c.splits;
    a.tiles_per_split = c.tiles_per_split;
    a.m_blocks = c.m_blocks;
    if (c.splits > 1) {
        const int64_t need = mfma_workspace_bytes(f, m, n, k);
        if (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < need) {
            set_error(op, "workspace of %lld bytes required, %zu given", static_cast<long long>(need), workspace_bytes);
            return PLM_ERR_WORKSPACE;
        }
        a.counters = static_cast<uint32_t*>(workspace);
        a.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
    }
    dim3 grid(c.m_blocks * c.n_blocks, c.splits);
    const bool uniform = group_size % kTileK == 0;
    auto go = [&](auto fmt_tag, auto bf_tag, auto uni_tag) {
        mfma_kernel<decltype(fmt_tag)::value, decltype(bf_tag)::value, 128, decltype(uni_tag)::value>
            <<<grid, kWaves * 64, 0, s>>>(a);
    };
    using I4 = std::integral_constant<plm_format, PLM_INT4>;
    using F8 = std::integral_constant<plm_format, PLM_FP8>;
    using T = std::true_type;
    using Fa = std::false_type;
    if (f == PLM_INT4) {
        if (bf16) uniform ? go(I4{}, T{}, T{}) : go(I4{}, T{}, Fa{});
        else uniform ? go(I4{}, Fa{}, T{}) : go(I4{}, Fa{}, Fa{});
    } else {
        if (bf16) uniform ? go(F8{}, T{}, T{}) : go(F8{}, T{}, Fa{});
        else uniform ? go(F8{}, Fa{}, T{}) : go(F8{}, Fa{}, Fa{});
    }
    PLM_HIP_LAUNCH_CHECK(op);
    return PLM_OK;
}

}  // namespace plm
