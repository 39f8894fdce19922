// Shared definitions for the gfx950 quantized-linear kernels: the tile layout
// constants, operand vector types, MFMA wrappers, dtype helpers and the C-ABI
// error plumbing.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "pulsarlm_amd.h"

namespace plm {

// ---------------------------------------------------------------------------
// Layout: 16 x 128 weight tiles, 64 lanes x 16 bytes per 1 KiB sub-tile.
// ---------------------------------------------------------------------------
constexpr int kTileN = 16;
constexpr int kTileK = 128;
constexpr int kSubTileBytes = 1024;

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

template <plm_format F> struct fmt_traits;
template <> struct fmt_traits<PLM_INT4> {
    static constexpr int tile_bytes = 1024;  // 16 x 128 x 4 bit
};
template <> struct fmt_traits<PLM_FP8> {
    static constexpr int tile_bytes = 2048;  // 16 x 128 x 8 bit
};

inline int64_t tile_bytes(plm_format f) { return f == PLM_INT4 ? 1024 : 2048; }

struct layout_dims {
    int64_t strips;     // ceil(N / 16)
    int64_t ktiles;     // ceil(K / 128)
    int64_t groups;     // ceil(ktiles * 128 / group_size): scale groups incl. padding
    int scale_cols;     // 16 (per column) or 1 (per strip)
};

inline layout_dims make_dims(int64_t n, int64_t k, int64_t block_n, int64_t group_size) {
    layout_dims d;
    d.strips = ceil_div(n, kTileN);
    d.ktiles = ceil_div(k, kTileK);
    d.groups = ceil_div(d.ktiles * kTileK, group_size);
    d.scale_cols = (block_n % kTileN == 0) ? 1 : kTileN;
    return d;
}

// Split-K workspaces start with a fixed region of arrival counters, so a
// workspace reused across calls of different shapes always finds its counters
// at the same place (and zero); partial sums follow it.
constexpr int64_t kCounterBytes = 64 * 1024;
constexpr int64_t kMaxCounters = kCounterBytes / 4;

inline int dtype_size(plm_dtype t) { return t == PLM_FP32 ? 4 : 2; }

// ---------------------------------------------------------------------------
// Vector types for MFMA operands.
// ---------------------------------------------------------------------------
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((ext_vector_type(8))) int i32x8_t;

// 16x16x32 MFMA with fp32 accumulation; the operand is 8 16-bit values per lane
// held as 4 packed dwords. A: lane l = row l%16, K block l/16. B: lane l = column
// l%16, same K block. D: lane l = column l%16, rows 4*(l/16) + i.
template <bool BF16>
__device__ __forceinline__ f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
    if constexpr (BF16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                      __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                     __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    }
}

typedef __attribute__((ext_vector_type(8))) uint32_t u32x8_t;
__device__ __forceinline__ u32x8_t u32x8_cat(u32x4_t lo, u32x4_t hi) {
    return u32x8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// 16x16x128 fp8 x fp8 (both OCP e4m3) MFMA, 32 bytes per lane per operand.
__device__ __forceinline__ f32x4_t mfma16x16x128_fp8(i32x8_t a, i32x8_t b, f32x4_t c) {
    // cbsz = blgp = 0 selects e4m3 for both operands; scale exponents 127 = x1.
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// ---------------------------------------------------------------------------
// 16-bit float helpers (bit level, RNE).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// Round to nearest even with gfx950's v_cvt_pk_bf16_f32 (a NaN stays a quiet NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f)));
}

__device__ __forceinline__ float round_bf16(float f) { return static_cast<float>(static_cast<__bf16>(f)); }

__device__ __forceinline__ float round_f16(float f) { return static_cast<float>(static_cast<_Float16>(f)); }

template <bool BF16> __device__ __forceinline__ float round_to(float f) {
    if constexpr (BF16) return round_bf16(f);
    else return round_f16(f);
}

template <bool BF16> __device__ __forceinline__ uint32_t to_bits16(float f) {
    if constexpr (BF16) return f32_to_bf16_bits(f);
    else return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f)));
}

template <bool BF16> __device__ __forceinline__ float from_bits16(uint32_t b) {
    if constexpr (BF16) return bf16_bits_to_f32(b);
    else return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
}

// Two fp32 -> one dword of two 16-bit values (lo = a), RNE.
template <bool BF16> __device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (BF16) {
        typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
        bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
        return __builtin_bit_cast(uint32_t, v);
    } else {
        typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;
        f16x2_t v = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
        return __builtin_bit_cast(uint32_t, v);
    }
}

// round(silu(g)) * u for g, u already in the activation dtype: the reference's
// at::silu(gate) * up (silu = g / (1 + exp(-g)) in fp32, rounded to the dtype before the
// product; the caller rounds the product). The fused MoE epilogue, the MoE's silu_mul
// kernel and plm_silu_mul all use this expression, so they give the same bits.
template <bool BF16> __device__ __forceinline__ float silu_times(float g, float u) {
    return round_to<BF16>(g / (1.f + expf(-g))) * u;
}

// Scale load in its stored dtype -> fp32.
__device__ __forceinline__ float load_scale(const void* base, int64_t index, int dtype) {
    if (dtype == PLM_FP32) return static_cast<const float*>(base)[index];
    const uint16_t b = static_cast<const uint16_t*>(base)[index];
    if (dtype == PLM_BF16) return bf16_bits_to_f32(b);
    return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

// e4m3 (fn) byte -> fp32, exact (subnormals included); the NaN codes are not handled.
__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
    const uint32_t sign = (c & 0x80u) << 24;
    const uint32_t e = (c >> 3) & 0xfu, m = c & 7u;
    // Normal: (1 + m/8) 2^(e-7) -> fp32 exponent e + 120. Subnormal: m 2^-9.
    const uint32_t normal = ((e + 120u) << 23) | (m << 20);
    const uint32_t sub = __float_as_uint(static_cast<float>(m) * 0.001953125f);
    return __uint_as_float(sign | (e == 0 ? sub : normal));
}

// ---------------------------------------------------------------------------
// Exact dequantization to the MFMA operand: round(q * round(s)), the value the
// reference's kernels feed their MMAs (pulsarlm-core/src/kernels/marlin.cu:78-84,
// 123-151,180-194).
//
// int4 runs on the matrix core. A lane's plm word holds 8 nibbles u = q + 8 of four
// columns and two K quads: lane l = 16 g + 4 c + i, nibble p holds column
// 4 c + r and K 8 g + 4 h + i of its 32-wide K slice, with r = 2 (p % 2) + p / 4 and
// h = (p % 4) / 2. v_bitop3 turns the nibbles into 16-bit floats a = base + u (exact),
// two per dword, and v_mfma_f32_4x4x4_16b (16 independent 4 x 4 x 4 products) with a
// diagonal B operand (block b: B[j][j] = s of column 4 (b % 4) + j) and C = -(base + 8) s
// gives D[i][j] = (base + u) s - (base + 8) s = q s exactly: every product fits fp32's
// 24 bits and the sum is exactly representable. Block b's D lands in lane 4 b + j,
// register i: column l % 16, K 8 g + 4 h + i -- the lane's B fragment of
// v_mfma_f32_16x16x32 (column l % 16, K 8 (l / 16) + 0..7) for h = 0, 1, with no
// shuffle. One v_cvt_pk per pair rounds once, to nearest even. Per word: 4 bitop3
// (+3 shifts for bf16, +1 for fp16), 2 small MFMAs and 4 converts, against 17 VALU ops
// for the same 8 weights per lane with v_fma_mix.
//   bf16: a = 128 + u (0x4300 | u); all four registers use nibbles at bits 0-3 of a
//         16-bit half, so three of the four dwords take a shift.
//   fp16: registers 0-1 take nibbles at bits 0-3 as 1024 + u (0x6400 | u), registers
//         2-3 nibbles at bits 4-7 as 64 + u (exponent 6: 0x5400 | u << 4), so one
//         shift (by 8) serves all four dwords; C = -(1032 or 72) s per register.
// The B diagonal and C are per lane (lane l's own column scale at register l % 4).
// Domain: (128 + u) s must stay finite, so bf16-rounded scales must be below 2^120 in
// magnitude (fp16 ones always are); plm_dequant has no such limit.
// ---------------------------------------------------------------------------
typedef __attribute__((ext_vector_type(4))) short s16x4_t;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4_t;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;

struct int4_scale {
    u32x2_t diag;  // B operand of the 4x4x4 MFMA: the lane's scale at register lane % 4
    float c;       // -(base + 8) * s for the lane's register lane % 4
};

template <bool BF16> __device__ __forceinline__ int4_scale make_int4_scale(float raw) {
    const int j = __lane_id() & 3;
    int4_scale k;
    uint32_t bits;
    float s;
    if constexpr (BF16) {
        s = round_bf16(raw);
        bits = f32_to_bf16_bits(s);
        k.c = -136.f * s;
    } else {
        s = round_f16(raw);
        bits = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(s)));
        k.c = (j < 2 ? -1032.f : -72.f) * s;
    }
    const uint32_t sh = (j & 1) ? bits << 16 : bits;
    k.diag[0] = j < 2 ? sh : 0u;
    k.diag[1] = j < 2 ? 0u : sh;
    return k;
}

__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) {
    return __builtin_amdgcn_bitop3_b32(a, mask, bits, 0xEA);  // (a & mask) | bits
}

template <bool BF16> __device__ __forceinline__ f32x4_t mfma4x4x4(u32x2_t a, u32x2_t b, f32x4_t c) {
    if constexpr (BF16) {
        return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4_t, a), __builtin_bit_cast(s16x4_t, b), c,
                                                      0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4_t, a), __builtin_bit_cast(f16x4_t, b), c, 0,
                                                  0, 0);
    }
}

template <bool BF16> __device__ __forceinline__ u32x4_t dq_int4(uint32_t w, const int4_scale& k) {
    u32x2_t a0, a1;
    if constexpr (BF16) {
        a0[0] = and_or(w, 0x000F000Fu, 0x43004300u);
        a0[1] = and_or(w >> 4, 0x000F000Fu, 0x43004300u);
        a1[0] = and_or(w >> 8, 0x000F000Fu, 0x43004300u);
        a1[1] = and_or(w >> 12, 0x000F000Fu, 0x43004300u);
    } else {
        const uint32_t w8 = w >> 8;
        a0[0] = and_or(w, 0x000F000Fu, 0x64006400u);
        a0[1] = and_or(w, 0x00F000F0u, 0x54005400u);
        a1[0] = and_or(w8, 0x000F000Fu, 0x64006400u);
        a1[1] = and_or(w8, 0x00F000F0u, 0x54005400u);
    }
    const f32x4_t c = {k.c, k.c, k.c, k.c};
    const f32x4_t d0 = mfma4x4x4<BF16>(a0, k.diag, c);
    const f32x4_t d1 = mfma4x4x4<BF16>(a1, k.diag, c);
    u32x4_t b;
    b[0] = pack2<BF16>(d0[0], d0[1]);
    b[1] = pack2<BF16>(d0[2], d0[3]);
    b[2] = pack2<BF16>(d1[0], d1[1]);
    b[3] = pack2<BF16>(d1[2], d1[3]);
    return b;
}

// Nibble position of (column c16 % 4, K quad h) in a plm int4 word (see above).
__host__ __device__ constexpr int int4_nibble_pos(int r, int h) { return 4 * (r & 1) + 2 * h + (r >> 1); }

// fp8: v_cvt_pk_f32_fp8 decodes two e4m3 bytes exactly; the product with the
// rounded scale is exact in fp32 (4 x 11 significant bits) and rounded once.
template <bool BF16> __device__ __forceinline__ u32x4_t dq_fp8(uint32_t lo, uint32_t hi, float s) {
    typedef __attribute__((ext_vector_type(2))) float f2;
    u32x4_t b;
    const f2 a0 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
    const f2 a1 = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
    const f2 a2 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
    const f2 a3 = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
    b[0] = pack2<BF16>(a0[0] * s, a0[1] * s);
    b[1] = pack2<BF16>(a1[0] * s, a1[1] * s);
    b[2] = pack2<BF16>(a2[0] * s, a2[1] * s);
    b[3] = pack2<BF16>(a3[0] * s, a3[1] * s);
    return b;
}

// Raw buffer loads: lanes whose offset is past num_records read 0 without a memory
// access, which is how rows >= M, columns >= K and idle tiles are skipped for free.
// Offsets at or past kOOB are outside every buffer the kernels build (checked on the host).
constexpr int kOOB = 0x40000000;

// launch_decode with the fused W8A8 quantizer requested, when its kernel does not apply to
// the shape (the caller then quantizes in a launch of its own). Not a plm_status value.
constexpr int kDecodeNotTaken = -1;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                             0x00020000);
}
__device__ __forceinline__ u32x4_t buffer_load16(__amdgpu_buffer_rsrc_t r, int offset) {
    return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0));
}
// voffset (per lane) + soffset (wave-uniform, an SGPR).
__device__ __forceinline__ u32x4_t buffer_load16(__amdgpu_buffer_rsrc_t r, int voffset, int soffset) {
    return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, 0));
}
#ifndef PLM_STREAM_POLICY
#define PLM_STREAM_POLICY 2
#endif
// Streaming (read-once) weights: the nontemporal policy (nt).
__device__ __forceinline__ u32x4_t buffer_load16_stream(__amdgpu_buffer_rsrc_t r, int voffset, int soffset) {
    return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, PLM_STREAM_POLICY));
}
__device__ __forceinline__ uint32_t buffer_load_u16(__amdgpu_buffer_rsrc_t r, int voffset, int soffset) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, voffset, soffset, 0);
}
__device__ __forceinline__ uint32_t buffer_load_u32(__amdgpu_buffer_rsrc_t r, int voffset, int soffset) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voffset, soffset, 0);
}
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
// 16 bytes per lane from a buffer straight into LDS (no VGPR staging): lane L writes
// lds + 16 * L, so `lds` (wave-uniform) is the base of the wavefront's 1 KiB. Counts in vmcnt;
// out-of-range lanes write zeros.
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t r, void* lds, int voffset, int soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voffset, soffset, 0,
                                             0);
}

// Scale bits as loaded (16-bit fp16/bf16 zero-extended, or fp32) -> fp32.
template <bool WIDE> __device__ __forceinline__ float scale_from_bits(uint32_t bits, bool bf16_storage) {
    if constexpr (WIDE) {
        return __uint_as_float(bits);
    } else {
        const float as_bf16 = __uint_as_float(bits << 16);
        const float as_f16 = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
        return bf16_storage ? as_bf16 : as_f16;
    }
}
template <bool WIDE> __device__ __forceinline__ uint32_t load_scale_bits(const void* base, int64_t index) {
    if constexpr (WIDE) return static_cast<const uint32_t*>(base)[index];
    else return static_cast<const uint16_t*>(base)[index];
}

// ---------------------------------------------------------------------------
// Split-K handshake. Partial sums are written and read with agent-scope relaxed
// atomics, which gfx950 issues as sc1 (coherent) stores/loads that bypass the
// per-XCD L2, so no agent-scope fence (an L2 writeback + invalidate of the whole
// cache) is needed: a workgroup waits for its own stores to complete, then one
// lane counts the arrival.
// ---------------------------------------------------------------------------
// Cache policy of buffer loads/stores that must be coherent across XCDs (sc1): the same
// policy agent-scope atomics get.
constexpr int kCoherent = 16;
__device__ __forceinline__ void store_partial(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_partial(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Call with every thread of the workgroup after its store_partial()s. Returns true
// in every thread of the last workgroup to arrive at `counter`, which is then reset.
__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t expected, uint32_t* lds_flag) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = atomicAdd(counter, 1u);
        const bool last = prev == expected - 1;
        if (last) atomicExch(counter, 0u);
        *lds_flag = last ? 1u : 0u;
    }
    __syncthreads();
    return *lds_flag != 0;
}

// ---------------------------------------------------------------------------
// Host-side error plumbing.
// ---------------------------------------------------------------------------
void set_error(const char* op, const char* fmt, ...);
void clear_error();

#define PLM_CHECK_ARG(cond, op, ...)                 \
    do {                                             \
        if (!(cond)) {                               \
            ::plm::set_error(op, __VA_ARGS__);       \
            return PLM_ERR_INVALID;                  \
        }                                            \
    } while (0)

#define PLM_HIP_LAUNCH_CHECK(op)                                                   \
    do {                                                                           \
        hipError_t e_ = hipGetLastError();                                         \
        if (e_ != hipSuccess) {                                                    \
            ::plm::set_error(op, "kernel launch failed: %s", hipGetErrorString(e_)); \
            return PLM_ERR_HIP;                                                    \
        }                                                                          \
    } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int cu_count();

// Measurement knobs: environment variables that force one kernel path against another for
// A/B timing on the same box (every setting stays within the GEMM tolerance). They are
// parsed once, at the first call that consults them, so no per-call path reads the
// environment; plm_internal_reload_tuning() re-parses them (tests only).
struct tuning {
    int64_t decode_max_m = -1;         // PLM_DECODE_MAX_M (0-32): plain decode/MFMA threshold
    bool w8a8_unfused = false;         // PLM_W8A8_UNFUSED: per-token quantizer in its own launch
    int decode_sp = 0, decode_tpw = 0, decode_nw = 0;  // PLM_DECODE="sp,tpw,nw"
    int rr_sg = -1, rr_nw = 0;         // PLM_DECODE_RR="sg,nw" (sg 0: round-robin kernel off)
    bool decode_no_xs = false;         // PLM_DECODE_NO_XS: x from global memory, not LDS
    char mfma_shape = 0;               // PLM_MFMA=<letter>: force one MFMA tile shape
    bool mfma_no_halves = false;       // PLM_MFMA_NO_HALVES
    bool mfma_no_tail = false;         // PLM_MFMA_NO_TAIL
    bool mfma_unsplit = false;         // PLM_MFMA_UNSPLIT: no K split and no tail launch
    int moe_rows = 0;                  // PLM_MOE_ROWS=16/32/64
    bool moe_small_sort_off = false;   // PLM_MOE_SMALL_SORT=0
    bool moe_unfused = false;          // PLM_MOE_UNFUSED
    bool moe_persist = false;          // PLM_MOE_PERSIST=1: persistent grouped launches
};
const tuning& knobs();

}  // namespace plm
