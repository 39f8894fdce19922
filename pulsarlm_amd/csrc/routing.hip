// MoE router and activation: route_top_k and silu_mul.
//
// Counterparts of route_top_k_cuda and silu_mul_cuda (pulsarlm-core/inc/pulsarlm/kernels/
// ops.hpp:37-43, pulsarlm-core/src/kernels/moe_routing.cu:56-131,137-200), the ops that feed
// routed_experts (pulsarlm-core/src/engine/model/qwen4_exp.cpp:542). Designed for gfx950:
//
// * route_top_k: one wavefront per token (four per workgroup, no workgroup barrier). The
//   wavefront takes the row maximum and the sum of exp(logit - max) with butterfly
//   reductions, keeps the token's probabilities in its own LDS area, and each lane tracks
//   the best (probability, expert) among its experts; each of the k rounds is one
//   wavefront argmax (higher probability, then lower expert) after which only the lane
//   that owned the winner rescans its experts. The k winners stay in registers (lane j
//   holds the j-th), their sum is taken in order j = 0 .. k-1 and each is divided by it.
//   The expert ids can be written as int64 (the reference's output) and/or int32 (what
//   plm_moe takes), so the router feeds the MoE block without a conversion or host sync.
// * silu_mul: y = round(round(silu(g)) * u) with silu(g) = g / (1 + exp(-g)) in fp32,
//   16 bytes per thread per operand where the row length allows.
#include <algorithm>

#include "plm_common.hpp"

namespace plm {

namespace {

constexpr int kRouteWaves = 4;
constexpr int64_t kRouteMaxExperts = 4096;
constexpr int64_t kRouteMaxTopK = 64;

template <int DT> __device__ __forceinline__ float value_at(const void* p, int64_t i) {
    if constexpr (DT == PLM_FP32) return static_cast<const float*>(p)[i];
    else if constexpr (DT == PLM_BF16) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    else return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(p)[i]));
}

// (v, e) ranks above (bv, be): higher probability, the lower expert among equals.
__device__ __forceinline__ bool ranks_above(float v, int e, float bv, int be) { return v > bv || (v == bv && e < be); }

template <int DT>
__global__ void __launch_bounds__(kRouteWaves * 64)
    route_top_k_kernel(const void* logits, int64_t row_stride, int64_t tokens, int experts, int k, float* weights,
                       int64_t* chosen64, int32_t* chosen32) {
    extern __shared__ float route_lds[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kRouteWaves + wave;
    if (t >= tokens) return;  // wave-uniform; nothing below synchronizes the workgroup
    float* p = route_lds + wave * experts;
    const int64_t base = t * row_stride;

    float mx = -INFINITY;
    for (int e = lane; e < experts; e += 64) mx = fmaxf(mx, value_at<DT>(logits, base + e));
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    float sum = 0.f;
    for (int e = lane; e < experts; e += 64) {
        const float s = expf(value_at<DT>(logits, base + e) - mx);
        p[e] = s;
        sum += s;
    }
    // A butterfly gives every lane the same total (each step adds the same two values).
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);

    float bv = -INFINITY;
    int be = experts;
    for (int e = lane; e < experts; e += 64) {
        const float q = p[e] / sum;
        p[e] = q;
        if (ranks_above(q, e, bv, be)) bv = q, be = e;
    }

    float my_top = 0.f;
    int my_expert = 0;
    for (int j = 0; j < k; ++j) {
        float v = bv;
        int e = be;
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(v, off);
            const int oe = __shfl_xor(e, off);
            if (ranks_above(ov, oe, v, e)) v = ov, e = oe;
        }
        if (lane == j) my_top = v, my_expert = e;
        if ((e & 63) == lane) {  // the owner drops the winner and finds its next best
            p[e] = -INFINITY;
            bv = -INFINITY;
            be = experts;
            for (int f = lane; f < experts; f += 64)
                if (ranks_above(p[f], f, bv, be)) bv = p[f], be = f;
        }
    }
    float total = 0.f;
    for (int j = 0; j < k; ++j) total += __shfl(my_top, j);
    if (lane < k) {
        weights[t * k + lane] = my_top / total;
        if (chosen64 != nullptr) chosen64[t * k + lane] = my_expert;
        if (chosen32 != nullptr) chosen32[t * k + lane] = my_expert;
    }
}

template <int DT> __device__ __forceinline__ float round_dt(float v) {
    if constexpr (DT == PLM_FP32) return v;
    else return round_to<DT == PLM_BF16>(v);
}

template <int DT> __device__ __forceinline__ float silu_mul1(float g, float u) {
    if constexpr (DT == PLM_FP32) return g / (1.f + expf(-g)) * u;
    else return round_dt<DT>(silu_times<DT == PLM_BF16>(g, u));
}

template <int DT> __device__ __forceinline__ void store_value(void* p, int64_t i, float v) {
    if constexpr (DT == PLM_FP32) static_cast<float*>(p)[i] = v;
    else static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(to_bits16<DT == PLM_BF16>(v));
}

// Row `row` of x is [g (n) | u (n)]; VEC values per thread (16 bytes) when n allows it.
template <int DT, int VEC>
__global__ void __launch_bounds__(256) silu_mul_op_kernel(const void* x, void* y, int64_t tokens, int64_t n) {
    constexpr int ES = DT == PLM_FP32 ? 4 : 2;
    const int64_t c0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * VEC;
    if (c0 >= n) return;
    for (int64_t row = blockIdx.y; row < tokens; row += gridDim.y) {
        const int64_t gi = row * 2 * n + c0, ui = gi + n, yi = row * n + c0;
        if constexpr (VEC == 1) {
            store_value<DT>(y, yi, silu_mul1<DT>(value_at<DT>(x, gi), value_at<DT>(x, ui)));
        } else {
            const u32x4_t gv = *reinterpret_cast<const u32x4_t*>(static_cast<const uint8_t*>(x) + gi * ES);
            const u32x4_t uv = *reinterpret_cast<const u32x4_t*>(static_cast<const uint8_t*>(x) + ui * ES);
            u32x4_t out;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                if constexpr (DT == PLM_FP32) {
                    out[w] = __float_as_uint(silu_mul1<DT>(__uint_as_float(gv[w]), __uint_as_float(uv[w])));
                } else {
                    constexpr bool BF = DT == PLM_BF16;
                    const float lo = silu_mul1<DT>(from_bits16<BF>(gv[w] & 0xffffu), from_bits16<BF>(uv[w] & 0xffffu));
                    const float hi = silu_mul1<DT>(from_bits16<BF>(gv[w] >> 16), from_bits16<BF>(uv[w] >> 16));
                    out[w] = to_bits16<BF>(lo) | (to_bits16<BF>(hi) << 16);
                }
            }
            *reinterpret_cast<u32x4_t*>(static_cast<uint8_t*>(y) + yi * ES) = out;
        }
    }
}

template <int DT>
void launch_silu_mul_t(const void* x, void* y, int64_t tokens, int64_t n, bool vec, hipStream_t s) {
    constexpr int VEC = DT == PLM_FP32 ? 4 : 8;
    const int64_t per = vec ? VEC : 1;
    dim3 grid(static_cast<unsigned>(ceil_div(n, 256 * per)), static_cast<unsigned>(std::min<int64_t>(tokens, 65535)));
    if (vec) silu_mul_op_kernel<DT, VEC><<<grid, 256, 0, s>>>(x, y, tokens, n);
    else silu_mul_op_kernel<DT, 1><<<grid, 256, 0, s>>>(x, y, tokens, n);
}

}  // namespace

}  // namespace plm

using namespace plm;

extern "C" {

int plm_route_top_k(const void* logits, plm_dtype dtype, int64_t tokens, int64_t experts, int64_t row_stride,
                    int64_t k, float* weights, int64_t* chosen, int32_t* chosen_i32, void* stream) {
    const char* op = "route_top_k";
    clear_error();
    PLM_CHECK_ARG(dtype == PLM_BF16 || dtype == PLM_FP16 || dtype == PLM_FP32, op, "logits must be fp32, fp16 or bf16");
    PLM_CHECK_ARG(experts >= 1 && experts <= kRouteMaxExperts && k >= 1 && k <= experts && k <= kRouteMaxTopK, op,
                  "experts must be at most %lld and k between 1 and the experts, at most %lld",
                  static_cast<long long>(kRouteMaxExperts), static_cast<long long>(kRouteMaxTopK));
    PLM_CHECK_ARG(tokens >= 0 && row_stride >= experts, op, "tokens must be non-negative and rows at least experts apart");
    PLM_CHECK_ARG(tokens <= (int64_t{1} << 31), op, "tokens must be below 2^31");
    if (tokens == 0) return PLM_OK;
    PLM_CHECK_ARG(logits != nullptr && weights != nullptr && (chosen != nullptr || chosen_i32 != nullptr), op,
                  "null pointer");
    const hipStream_t s = as_stream(stream);
    const dim3 grid(static_cast<unsigned>(ceil_div(tokens, kRouteWaves)));
    const size_t lds = static_cast<size_t>(kRouteWaves) * experts * sizeof(float);
    const int e = static_cast<int>(experts), kk = static_cast<int>(k);
    if (dtype == PLM_FP32)
        route_top_k_kernel<PLM_FP32><<<grid, kRouteWaves * 64, lds, s>>>(logits, row_stride, tokens, e, kk, weights, chosen, chosen_i32);
    else if (dtype == PLM_BF16)
        route_top_k_kernel<PLM_BF16><<<grid, kRouteWaves * 64, lds, s>>>(logits, row_stride, tokens, e, kk, weights, chosen, chosen_i32);
    else
        route_top_k_kernel<PLM_FP16><<<grid, kRouteWaves * 64, lds, s>>>(logits, row_stride, tokens, e, kk, weights, chosen, chosen_i32);
    PLM_HIP_LAUNCH_CHECK(op);
    return PLM_OK;
}

int plm_silu_mul(const void* x, plm_dtype dtype, int64_t tokens, int64_t n, void* y, void* stream) {
    const char* op = "silu_mul";
    clear_error();
    PLM_CHECK_ARG(dtype == PLM_BF16 || dtype == PLM_FP16 || dtype == PLM_FP32, op, "x must be fp32, fp16 or bf16");
    PLM_CHECK_ARG(tokens >= 0 && n >= 0, op, "sizes must be non-negative");
    if (tokens == 0 || n == 0) return PLM_OK;
    PLM_CHECK_ARG(x != nullptr && y != nullptr, op, "null pointer");
    const int es = dtype == PLM_FP32 ? 4 : 2;
    PLM_CHECK_ARG(aligned(x, es) && aligned(y, es), op, "x and y must be aligned to their element size");
    const bool vec = (n * es) % 16 == 0 && aligned(x, 16) && aligned(y, 16);
    const hipStream_t s = as_stream(stream);
    if (dtype == PLM_FP32) launch_silu_mul_t<PLM_FP32>(x, y, tokens, n, vec, s);
    else if (dtype == PLM_BF16) launch_silu_mul_t<PLM_BF16>(x, y, tokens, n, vec, s);
    else launch_silu_mul_t<PLM_FP16>(x, y, tokens, n, vec, s);
    PLM_HIP_LAUNCH_CHECK(op);
    return PLM_OK;
}

}  // extern "C"
