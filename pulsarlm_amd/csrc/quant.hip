// Per-row (per-token) dynamic e4m3 quantization of activations for the W8A8 GEMM:
// scale = max(amax(row), 1e-12) / 448, codes = e4m3_rne(x / scale). No counterpart in
// the reference's GEMM path (its fp8 path is W8A16); the rule is the block quantizer of
// pulsarlm-core/tests/model/test_qwen3_5.cpp:301-311 applied per row.
#include "plm_common.hpp"

namespace plm {

namespace {

constexpr int kQThreads = 256;

// One workgroup per row. PERMUTED writes the lane order the fp8 MFMA kernels read:
// within each 128-wide K tile, byte 32 kq + 8 t + i holds k = 32 t + 8 kq + i; the row
// stride is ktiles * 128 and columns past K are zero. Otherwise the row is [K] bytes.
template <bool BF16, bool PERMUTED>
__global__ void __launch_bounds__(kQThreads) quantize_rows_kernel(const uint16_t* __restrict__ x, int k, int ktiles,
                                                                    uint8_t* __restrict__ out, float* __restrict__ sx) {
    const int row = blockIdx.x;
    const uint16_t* xr = x + static_cast<int64_t>(row) * k;
    float amax = 0.f;
    for (int i = threadIdx.x; i < k; i += kQThreads) amax = fmaxf(amax, fabsf(from_bits16<BF16>(xr[i])));
    // Reduce: within the wavefront, then across the four.
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    __shared__ float part[kQThreads / 64];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    const float scale = fmaxf(amax, 1e-12f) / 448.f;
    if (threadIdx.x == 0) sx[row] = scale;

    const int cols = PERMUTED ? ktiles * kTileK : k;
    uint8_t* orow = out + static_cast<int64_t>(row) * cols;
    // Four consecutive K per thread -> one dword (consecutive in both layouts).
    for (int k4 = threadIdx.x * 4; k4 < cols; k4 += kQThreads * 4) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (k4 + i < k) ? from_bits16<BF16>(xr[k4 + i]) / scale : 0.f;
        int packed = 0;
        packed = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], packed, false);
        packed = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], packed, true);
        int dst = k4;
        if constexpr (PERMUTED) {
            const int kt = k4 / kTileK, kin = k4 % kTileK;
            const int t = kin / 32, q = (kin % 32) / 8, i = kin % 8;
            dst = kt * kTileK + q * 32 + t * 8 + i;
        }
        *reinterpret_cast<int*>(orow + dst) = packed;
    }
}

}  // namespace

int launch_quantize_rows(const char* op, const void* x, bool bf16, int64_t m, int64_t k, uint8_t* out, float* sx,
                         bool permuted, hipStream_t s) {
    if (m == 0) return PLM_OK;
    const int ktiles = static_cast<int>(ceil_div(k, kTileK));
    dim3 grid(static_cast<unsigned>(m));
    auto xp = static_cast<const uint16_t*>(x);
    if (bf16) {
        if (permuted) quantize_rows_kernel<true, true><<<grid, kQThreads, 0, s>>>(xp, int(k), ktiles, out, sx);
        else quantize_rows_kernel<true, false><<<grid, kQThreads, 0, s>>>(xp, int(k), ktiles, out, sx);
    } else {
        if (permuted) quantize_rows_kernel<false, true><<<grid, kQThreads, 0, s>>>(xp, int(k), ktiles, out, sx);
        else quantize_rows_kernel<false, false><<<grid, kQThreads, 0, s>>>(xp, int(k), ktiles, out, sx);
    }
    PLM_HIP_LAUNCH_CHECK(op);
    return PLM_OK;
}

}  // namespace plm
