// Non-repacked int4 GEMM: y[M, N] = x[M, K] @ W^T with W[n, k] = round(fp32(q[n, k] *
// scale[n, k / g])), q the signed nibbles of weight_packed int32 [N, K/8] (least significant
// first) and scale fp32 [N, K/g].
//
// Counterpart of gemm_int4_cuda / gemm_int4_split_cuda (pulsarlm-core/inc/pulsarlm/kernels/
// ops.hpp:272-297, pulsarlm-core/src/kernels/int4_gemm.cu:53-57,136-138,153-478), which the
// reference declares but never calls (its engine runs the repacked path). Kept simple, not
// tuned, with the reference's rounding (the product rounded to fp32, then to x's dtype):
//
// * The weights are read in place: one 32-bit word (8 consecutive K values of one row) is
//   exactly one lane's B fragment of v_mfma_f32_16x16x32. A lane (column n % 16, K block kq)
//   reads words 16 kt + 4 kq + t for t = 0..3 of a 128-wide K tile, and the x fragment of
//   MFMA step t holds the matching K values 128 kt + 32 kq + 8 t + 0..7: a permutation of K
//   applied to both operands, so the sum is unchanged.
// * A workgroup is 4 wavefronts over 64 rows x 64 columns, one 16-column strip per
//   wavefront (each weight dequantized once per workgroup), x fragments read from global.
// * Split-K (forced by gemm_int4_split_cuda, else when the tiles do not fill the GPU)
//   writes fp32 partials [splits][M][N]; a combine kernel sums them in split order and
//   rounds once, as the reference's combine_partials_kernel does.
#include <algorithm>

#include "plm_common.hpp"

namespace plm {

namespace {

constexpr int kPlainRows = 64;   // rows per workgroup: 4 MFMA row tiles per wavefront
constexpr int kPlainWaves = 4;   // one 16-column strip per wavefront
constexpr int kPlainMT = kPlainRows / 16;

// Eight values of one word, each round(fp32(q * s)), as four packed pairs (k, k + 1).
template <bool BF16> __device__ __forceinline__ u32x4_t dq_plain(uint32_t w, float s) {
    u32x4_t b;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        // Sign-extended nibbles 2j and 2j + 1 (an arithmetic shift of the nibble to the top).
        const float q0 = static_cast<float>(static_cast<int32_t>(w << (28 - 8 * j)) >> 28);
        const float q1 = static_cast<float>(static_cast<int32_t>(w << (24 - 8 * j)) >> 28);
        b[j] = pack2<BF16>(q0 * s, q1 * s);
    }
    return b;
}

template <bool BF16>
__global__ void __launch_bounds__(kPlainWaves * 64)
    plain_int4_kernel(const uint16_t* x, const int32_t* w, const float* scale, uint16_t* y, float* partial, int m,
                      int n, int k, int group_size, int tiles_per_split) {
    const int lane = threadIdx.x & 63;
    const int wave = uniform(threadIdx.x >> 6);
    const int col16 = lane & 15, kq = lane >> 4;
    const int row0 = blockIdx.x * kPlainRows;
    const int col = (blockIdx.y * kPlainWaves + wave) * kTileN + col16;
    const int split = blockIdx.z;
    const int ktiles = (k + kTileK - 1) / kTileK;
    const int kt_lo = split * tiles_per_split;
    const int kt_hi = min(kt_lo + tiles_per_split, ktiles);
    const int words = k / 8;
    const int groups = k / group_size;

    const int rows = min(kPlainRows, m - row0);
    const __amdgpu_buffer_rsrc_t xr =
        make_rsrc(x + static_cast<int64_t>(row0) * k, static_cast<uint32_t>(rows) * k * 2);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w, static_cast<uint32_t>(static_cast<int64_t>(n) * words * 4));
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(scale, static_cast<uint32_t>(static_cast<int64_t>(n) * groups * 4));
    const bool col_ok = col < n;
    const int w_row = col_ok ? col * words * 4 : kOOB;
    const int s_row = col_ok ? col * groups * 4 : kOOB;

    f32x4_t acc[kPlainMT];
#pragma unroll
    for (int i = 0; i < kPlainMT; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int kt = kt_lo; kt < kt_hi; ++kt) {
        uint32_t wv[4];
        float sv[4];
        u32x4_t xa[kPlainMT][4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int word = 16 * kt + 4 * kq + t;  // K values 8 word .. 8 word + 7
            const bool ok = word < words;
            wv[t] = buffer_load_u32(wr, ok ? w_row + word * 4 : kOOB, 0);
            sv[t] = __uint_as_float(buffer_load_u32(sr, ok ? s_row + (8 * word / group_size) * 4 : kOOB, 0));
            const int kx = 128 * kt + 32 * kq + 8 * t;  // the x values that pair with that word
#pragma unroll
            for (int i = 0; i < kPlainMT; ++i) {
                const int r = 16 * i + col16;
                xa[i][t] = buffer_load16(xr, (r < rows && kx < k) ? r * k * 2 + kx * 2 : kOOB, 0);
            }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const u32x4_t b = dq_plain<BF16>(wv[t], sv[t]);
#pragma unroll
            for (int i = 0; i < kPlainMT; ++i) acc[i] = mfma16x16x32<BF16>(xa[i][t], b, acc[i]);
        }
    }

    // Lane holds column col, rows 16 i + 4 kq + r.
    if (!col_ok) return;
#pragma unroll
    for (int i = 0; i < kPlainMT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int lr = 16 * i + 4 * kq + r;
            if (lr >= rows) continue;
            const int64_t o = static_cast<int64_t>(row0 + lr) * n + col;
            if (partial == nullptr) y[o] = static_cast<uint16_t>(to_bits16<BF16>(acc[i][r]));
            else partial[static_cast<int64_t>(split) * m * n + o] = acc[i][r];
        }
}

template <bool BF16>
__global__ void __launch_bounds__(256) plain_combine_kernel(const float* partial, uint16_t* y, int64_t mn, int splits) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < mn; i += static_cast<int64_t>(gridDim.x) * 256) {
        float v = 0.f;
        for (int s = 0; s < splits; ++s) v += partial[s * mn + i];
        y[i] = static_cast<uint16_t>(to_bits16<BF16>(v));
    }
}

struct plain_config {
    int m_blocks, n_blocks, splits, tiles_per_split;
};

plain_config choose_plain(int64_t m, int64_t n, int64_t k, int64_t num_splits) {
    plain_config c{};
    c.m_blocks = static_cast<int>(ceil_div(m, kPlainRows));
    c.n_blocks = static_cast<int>(ceil_div(n, kPlainWaves * kTileN));
    const int64_t ktiles = ceil_div(k, kTileK);
    const int64_t tiles = static_cast<int64_t>(c.m_blocks) * c.n_blocks;
    int64_t splits = num_splits;
    if (splits <= 0) splits = tiles >= cu_count() ? 1 : std::min<int64_t>(ceil_div(cu_count(), tiles), ktiles);
    // Splits past the K tiles stay (they contribute zero), as the reference allows.
    c.splits = static_cast<int>(splits);
    c.tiles_per_split = static_cast<int>(std::max<int64_t>(1, ceil_div(ktiles, splits)));
    return c;
}

}  // namespace

}  // namespace plm

using namespace plm;

extern "C" {

int64_t plm_gemm_int4_plain_workspace_bytes(int64_t m, int64_t n, int64_t k, int64_t num_splits) {
    if (m <= 0 || n <= 0 || k <= 0) return 0;
    const plain_config c = choose_plain(m, n, k, num_splits);
    return c.splits > 1 ? static_cast<int64_t>(c.splits) * m * n * 4 : 0;
}

int plm_gemm_int4_plain(const void* x, plm_dtype x_dtype, const int32_t* weight_packed, const float* weight_scale,
                        int64_t m, int64_t n, int64_t k, int64_t group_size, int64_t num_splits, void* y,
                        void* workspace, size_t workspace_bytes, void* stream) {
    const char* op = "gemm_int4";
    clear_error();
    PLM_CHECK_ARG(x_dtype == PLM_BF16 || x_dtype == PLM_FP16, op, "x must be fp16 or bf16");
    PLM_CHECK_ARG(m >= 0 && n >= 0 && k >= 0, op, "sizes must be non-negative");
    PLM_CHECK_ARG(group_size > 0 && group_size % 16 == 0 && k % group_size == 0, op,
                  "group_size must be a positive multiple of 16 dividing K");
    PLM_CHECK_ARG(num_splits >= 0, op, "num_splits must be >= 1 (0: automatic)");
    PLM_CHECK_ARG(n * (k / 2) < (int64_t{1} << 30) && m * k * 2 < (int64_t{1} << 30) && m <= (int64_t{1} << 24), op,
                  "weight and x must be below 1 GiB");
    if (m == 0 || n == 0) return PLM_OK;
    PLM_CHECK_ARG(x != nullptr && weight_packed != nullptr && weight_scale != nullptr && y != nullptr, op,
                  "null pointer");
    PLM_CHECK_ARG(aligned(x, 16) && aligned(weight_packed, 4) && aligned(weight_scale, 4) && aligned(y, 2), op,
                  "x must be 16-byte aligned, the weight and scales 4-byte aligned");
    const plain_config c = choose_plain(m, n, k, num_splits);
    float* partial = nullptr;
    if (c.splits > 1) {
        const int64_t need = static_cast<int64_t>(c.splits) * m * n * 4;
        if (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < need) {
            set_error(op, "workspace of %lld bytes required, %zu given", static_cast<long long>(need), workspace_bytes);
            return PLM_ERR_WORKSPACE;
        }
        PLM_CHECK_ARG(aligned(workspace, 4), op, "workspace must be 4-byte aligned");
        partial = static_cast<float*>(workspace);
    }
    const hipStream_t s = as_stream(stream);
    const dim3 grid(c.m_blocks, c.n_blocks, c.splits);
    const bool bf16 = x_dtype == PLM_BF16;
    const auto* xp = static_cast<const uint16_t*>(x);
    auto* yp = static_cast<uint16_t*>(y);
    const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k), g = static_cast<int>(group_size);
    if (bf16) plain_int4_kernel<true><<<grid, kPlainWaves * 64, 0, s>>>(xp, weight_packed, weight_scale, yp, partial, mi, ni, ki, g, c.tiles_per_split);
    else plain_int4_kernel<false><<<grid, kPlainWaves * 64, 0, s>>>(xp, weight_packed, weight_scale, yp, partial, mi, ni, ki, g, c.tiles_per_split);
    PLM_HIP_LAUNCH_CHECK(op);
    if (c.splits > 1) {
        const int64_t mn = m * n;
        const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(ceil_div(mn, 256), 4096));
        if (bf16) plain_combine_kernel<true><<<blocks, 256, 0, s>>>(partial, yp, mn, c.splits);
        else plain_combine_kernel<false><<<blocks, 256, 0, s>>>(partial, yp, mn, c.splits);
        PLM_HIP_LAUNCH_CHECK(op);
    }
    return PLM_OK;
}

}  // extern "C"
