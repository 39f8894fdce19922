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

// The same quantization for rows of 8-value chunks (K % 8 == 0, x 16-byte aligned, out
// 8-byte aligned): each thread issues all its 16-byte chunk loads at once and keeps up to
// CAP chunks in registers, so the row is read once and a short row costs one load latency
// (the loop above reads it twice, two bytes at a time). Chunks past T * CAP are read again
// for the second pass. Same arithmetic, so the codes and scales are identical.
template <bool BF16> __device__ __forceinline__ float absmax8(const u32x4_t& v) {
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        a = fmaxf(a, fabsf(from_bits16<BF16>(v[j] & 0xffffu)));
        a = fmaxf(a, fabsf(from_bits16<BF16>(v[j] >> 16)));
    }
    return a;
}

template <bool BF16> __device__ __forceinline__ uint2 quant8(const u32x4_t& v, float scale) {
    int lo = 0, hi = 0;
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(from_bits16<BF16>(v[0] & 0xffffu) / scale,
                                         from_bits16<BF16>(v[0] >> 16) / scale, lo, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(from_bits16<BF16>(v[1] & 0xffffu) / scale,
                                         from_bits16<BF16>(v[1] >> 16) / scale, lo, true);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(from_bits16<BF16>(v[2] & 0xffffu) / scale,
                                         from_bits16<BF16>(v[2] >> 16) / scale, hi, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(from_bits16<BF16>(v[3] & 0xffffu) / scale,
                                         from_bits16<BF16>(v[3] >> 16) / scale, hi, true);
    return make_uint2(static_cast<uint32_t>(lo), static_cast<uint32_t>(hi));
}

// Byte offset of K value k8 (a multiple of 8) in an output row: 8 consecutive K stay
// consecutive in the lane-permuted layout too.
template <bool PERMUTED> __device__ __forceinline__ int chunk_dst(int k8) {
    if constexpr (!PERMUTED) return k8;
    const int kt = k8 / kTileK, kin = k8 % kTileK;
    return kt * kTileK + ((kin % 32) / 8) * 32 + (kin / 32) * 8;
}

template <bool BF16, bool PERMUTED, int T, int CAP>
__global__ void __launch_bounds__(T) quantize_rows_vec_kernel(const uint16_t* __restrict__ x, int k, int ktiles,
                                                             uint8_t* __restrict__ out, float* __restrict__ sx) {
    const int row = blockIdx.x;
    const int nch = k >> 3;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x + static_cast<int64_t>(row) * k, static_cast<uint32_t>(k) * 2);
    u32x4_t v[CAP];
#pragma unroll
    for (int c = 0; c < CAP; ++c) {
        const int ch = threadIdx.x + c * T;
        v[c] = buffer_load16(xr, ch < nch ? ch * 16 : kOOB);  // past the row: zeros, no access
    }
    float amax = 0.f;
    for (int ch = threadIdx.x + CAP * T; ch < nch; ch += T) amax = fmaxf(amax, absmax8<BF16>(buffer_load16(xr, ch * 16)));
#pragma unroll
    for (int c = 0; c < CAP; ++c)
        if (threadIdx.x + c * T < nch) amax = fmaxf(amax, absmax8<BF16>(v[c]));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    __shared__ float part[T / 64];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = part[0];
#pragma unroll
    for (int w = 1; w < T / 64; ++w) amax = fmaxf(amax, part[w]);
    const float scale = fmaxf(amax, 1e-12f) / 448.f;
    if (threadIdx.x == 0) sx[row] = scale;

    const int cols = PERMUTED ? ktiles * kTileK : k;
    uint8_t* orow = out + static_cast<int64_t>(row) * cols;
#pragma unroll
    for (int c = 0; c < CAP; ++c) {
        const int ch = threadIdx.x + c * T;
        if (ch < nch) *reinterpret_cast<uint2*>(orow + chunk_dst<PERMUTED>(ch * 8)) = quant8<BF16>(v[c], scale);
    }
    for (int ch = threadIdx.x + CAP * T; ch < nch; ch += T)
        *reinterpret_cast<uint2*>(orow + chunk_dst<PERMUTED>(ch * 8)) = quant8<BF16>(buffer_load16(xr, ch * 16), scale);
    // Columns past K (the permuted layout pads to whole tiles) hold zero codes.
    for (int ch = nch + threadIdx.x; ch < (cols >> 3); ch += T)
        *reinterpret_cast<uint2*>(orow + chunk_dst<PERMUTED>(ch * 8)) = make_uint2(0u, 0u);
}

template <bool BF16, bool PERMUTED>
void launch_vec(int64_t m, int k, int ktiles, const uint16_t* x, uint8_t* out, float* sx, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(m));
    // Few rows: 1024 threads a row for load parallelism; many rows: 256 (rows fill the GPU).
    if (m < 2 * cu_count()) quantize_rows_vec_kernel<BF16, PERMUTED, 1024, 4><<<grid, 1024, 0, s>>>(x, k, ktiles, out, sx);
    else quantize_rows_vec_kernel<BF16, PERMUTED, 256, 8><<<grid, 256, 0, s>>>(x, k, ktiles, out, sx);
}

}  // namespace

int launch_quantize_rows(const char* op, const void* x, bool bf16, int64_t m, int64_t k, uint8_t* out, float* sx,
                         bool permuted, hipStream_t s) {
    if (m == 0) return PLM_OK;
    const int ktiles = static_cast<int>(ceil_div(k, kTileK));
    dim3 grid(static_cast<unsigned>(m));
    auto xp = static_cast<const uint16_t*>(x);
    // (Offsets of chunks past the row must stay past the buffer: kOOB > 2 K.)
    if (k % 8 == 0 && k <= (int64_t{1} << 28) && aligned(x, 16) && aligned(out, 8)) {
        if (bf16) {
            if (permuted) launch_vec<true, true>(m, int(k), ktiles, xp, out, sx, s);
            else launch_vec<true, false>(m, int(k), ktiles, xp, out, sx, s);
        } else {
            if (permuted) launch_vec<false, true>(m, int(k), ktiles, xp, out, sx, s);
            else launch_vec<false, false>(m, int(k), ktiles, xp, out, sx, s);
        }
        PLM_HIP_LAUNCH_CHECK(op);
        return PLM_OK;
    }
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
