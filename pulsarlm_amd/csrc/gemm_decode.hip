// Bandwidth-first dequant-GEMM for decode (M <= 16, and 17-32 rows as two 16-row blocks):
// y[M, N] = x[M, K] @ dequant(W)^T.
//
// Counterpart of the reference's marlin_kernel at tile_m = 16 (pulsarlm-core/src/kernels/
// marlin.cu:251-389, dispatched for M <= 16 at :577-596) together with its split-K
// partial sum and combine (pulsarlm-core/inc/pulsarlm/kernels/dequant_gemm_common.cuh:
// 56-133). Designed for gfx950 rather than translated. Two kernels:
//
// decode_rr_kernel (scale groups a power-of-two multiple of 128, x fits in LDS, one load
// batch per wavefront): a workgroup owns whole strips over all of K, its wavefronts take
// K tiles round-robin, x and scales are staged per wavefront in LDS, weights stream with
// the nontemporal policy; see its own comment. Measured on MI355X it beats the kernel
// below at every Qwen3-8B shape except K = 12288, where a wavefront would hold 6 tiles.
//
// decode_kernel (every other case, including W8A8 and groups smaller than 128):
//
// * A wavefront owns SP 16-column strips over TPW consecutive 128-wide K tiles. Each
//   lane issues one 16-byte load per int4 tile (two per fp8 tile), so a wavefront's
//   load is one contiguous, fully coalesced 1 KiB, and all of a wavefront's loads are
//   in flight before the first MFMA.
// * Weights are dequantized in registers to exactly the reference's fragment values,
//   round(q * round(s)), with bitop3 + v_fma_mix_f32 + v_cvt_pk (about 2.1 VALU ops
//   per int4 weight; see dq_int4). When group_size is a multiple of 128 a lane's
//   16-byte load lies in one scale group, so its scale is loaded once, up front.
// * The x tile (16 rows, zero past M) is read straight from global memory; rows >= M
//   issue no load.
// * The NW wavefronts of a workgroup cover NW * TPW K tiles and reduce through LDS in a
//   fixed order; K splits across workgroups write fp32 partials and the last workgroup
//   to arrive at a column block sums them in split order, so results are deterministic.
#include <algorithm>

#include "plm_common.hpp"

namespace plm {

namespace {

struct decode_args {
    const uint16_t* x;
    const uint8_t* w;
    const void* scale;
    uint16_t* y;
    float* partial;      // [splits][M][N] fp32, used when splits > 1
    uint32_t* counters;  // [strip groups], zero on entry and exit
    int scale_dtype;
    int scale_cols;
    int m, n, k;
    int ktiles, strips, groups, group_size;
    int splits, tiles_per_split;
    // W8A8 only: e4m3 x in the lane-permuted layout [M][ktiles][128] and per-row scales.
    const uint8_t* xq;
    const float* x_scale;
    // x staged in LDS (M <= 4): bytes per row and per wavefront of the staging area.
    int xs_row, xs_wave;
    // W8A8 with the quantizer fused (QF): nonzero selects it; the row maxima and row scales
    // of the workgroup follow the wavefronts' staging areas in LDS.
    int quant_fused;
};

// x / s rounded to fp32 as the IEEE divide would for the quantizer's operands, from the
// reciprocal inv = 1 / s: q = x * inv, then one correction with the exact residual
// fma(-q, s, x), and x's sign (so -0 stays -0). An exhaustive check over every bf16 and
// fp16 x with |x| <= amax and every 16-bit amax (s = max(amax, 1e-12) / 448) finds the e4m3
// codes identical to those of x / s (the fp32 values differ only below 2^-60).
__device__ __forceinline__ float div_by_scale(float x, float s, float inv) {
    const float q = x * inv;
    return copysignf(__builtin_fmaf(__builtin_fmaf(-q, s, x), inv, q), x);
}

template <int CTRL, int ROW_MASK> __device__ __forceinline__ float dpp_f32(float x) {
    const int i = __builtin_bit_cast(int, x);
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(i, i, CTRL, ROW_MASK, 0xf, false));
}
__device__ __forceinline__ float wave_max_to_lane63(float v) {
    v = fmaxf(v, dpp_f32<0xB1, 0xf>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f32<0x4E, 0xf>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f32<0x141, 0xf>(v));  // row_half_mirror
    v = fmaxf(v, dpp_f32<0x140, 0xf>(v));  // row_mirror
    v = fmaxf(v, dpp_f32<0x142, 0xa>(v));  // row_bcast:15 into rows 1 and 3
    v = fmaxf(v, dpp_f32<0x143, 0xc>(v));  // row_bcast:31 into rows 2 and 3
    return v;
}

// One wavefront's batch of TPW K tiles for SP strips: weights, raw scale bits and x (RB
// blocks of 16 rows).
template <plm_format F, int SP, int TPW, bool A8, int RB> struct decode_batch {
    u32x4_t w[TPW][SP][fmt_traits<F>::tile_bytes / 1024];
    uint32_t s[TPW][SP];
    u32x4_t x[TPW][RB][A8 ? 2 : 4];  // bf16/fp16: 4 steps x 8 values; e4m3: 32 bytes
};

// Loads are raw buffer loads issued unconditionally, so no load sits behind a branch or
// feeds a select and a whole batch stays in flight (either would make the compiler wait
// on it at once). Everything that depends only on the wavefront (tile index, K offset,
// scale group) is computed in scalar registers and passed as the buffer's soffset; the
// per-lane voffset is fixed for the whole kernel. Out-of-range lanes or tiles (x rows
// >= M, tiles past the wavefront's range) get offsets past the buffer and read 0 without
// a memory access; tiles past the range are also skipped by a wave-uniform branch, and
// strips past N load a clamped strip whose outputs are never stored.
//
// A8 (W8A8): x arrives quantized to e4m3 with one fp32 scale per row; each 128-wide
// K tile is one v_mfma_scale_f32_16x16x128_f8f6f4 per strip on the raw weight bytes,
// the tile's partial is multiplied by its fp32 block scale, and the row scale is
// applied before the reduction.
//
// RB = 2 (16 < M <= 32, bf16/fp16 x read from global memory): each dequantized weight
// fragment feeds two MFMAs, one per 16-row block, so the weights are still read and
// dequantized once.
//
// QF (W8A8, M <= 4, one workgroup over all of K, every wavefront with a tile): the
// per-token quantizer runs inside the kernel, as in decode_rr_kernel. x is staged in
// bf16 / fp16 (XS); each wavefront takes the row maxima over its K range, the workgroup
// combines them through LDS, and each wavefront rewrites its staged x in place as e4m3 in
// the fp8 MFMA operand's lane order (128 bytes per row and tile), from which the A
// fragments are read. Same codes and row scales as plm_quantize_rows_e4m3.
template <plm_format F, bool BF16, int SP, int TPW, int NW, bool UNIFORM, bool WIDE, bool A8 = false, bool XS = false,
          int RB = 1, bool QF = false>
__global__ void __launch_bounds__(NW * 64) decode_kernel(decode_args a) {
    static_assert(RB == 1 || (!A8 && !XS), "two row blocks: bf16/fp16 x read from global memory only");
    static_assert(!QF || (A8 && XS && UNIFORM && RB == 1), "the fused quantizer stages bf16/fp16 x in LDS");
    constexpr int TB = fmt_traits<F>::tile_bytes;
    constexpr int ES = WIDE ? 4 : 2;  // scale element bytes
    const int lane = threadIdx.x & 63;
    const int wave = uniform(threadIdx.x >> 6);
    const int col16 = lane & 15;
    const int kq = lane >> 4;
    const int sg = blockIdx.x;
    const int split = blockIdx.y;
    // This workgroup's K tiles [kt_lo, kt_hi), dealt to its wavefronts in contiguous runs.
    const int kt_lo = split * a.tiles_per_split;
    const int kt_hi = min(kt_lo + a.tiles_per_split, a.ktiles);
    const int per_wave = (kt_hi - kt_lo + NW - 1) / NW;
    const int w_lo = kt_lo + wave * per_wave;
    const int w_hi = min(w_lo + per_wave, kt_hi);
    const bool bf16_scale = a.scale_dtype == PLM_BF16;

    // Buffers: one weight strip and its scales per j, and x.
    __amdgpu_buffer_rsrc_t wr[SP], sr[SP];
#pragma unroll
    for (int j = 0; j < SP; ++j) {
        const int stc = min(sg * SP + j, a.strips - 1);
        wr[j] = make_rsrc(a.w + static_cast<int64_t>(stc) * a.ktiles * TB, static_cast<uint32_t>(a.ktiles) * TB);
        sr[j] = make_rsrc(static_cast<const uint8_t*>(a.scale) + static_cast<int64_t>(stc) * a.groups * a.scale_cols * ES,
                          static_cast<uint32_t>(a.groups * a.scale_cols * ES));
    }
    const __amdgpu_buffer_rsrc_t xr =
        (A8 && !QF) ? make_rsrc(a.xq, static_cast<uint32_t>(a.m) * a.ktiles * kTileK)
           : make_rsrc(a.x, static_cast<uint32_t>(a.m) * a.k * 2);
    // bf16/fp16: row * K * 2 + 16 kq (+ 64 t + 256 kt); e4m3: row * ktiles * 128 + 32 kq (+ 128 kt).
    int x_lane[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int row = 16 * rb + col16;
        x_lane[rb] = (A8 && !QF) ? (row < a.m ? row * a.ktiles * kTileK : kOOB) + 32 * kq
                        : (row < a.m ? row * a.k * 2 : kOOB) + 16 * kq;
    }
    const int w_lane = lane * 16;
    const int s_lane = (a.scale_cols == 1 ? 0 : col16) * ES;

    auto load_batch = [&](decode_batch<F, SP, TPW, A8, RB>& b, int kt0) {
        // int4: the batch's scales first; they return first, so the scale constants can be
        // set up while the weight tiles are still arriving (fp8 measured no better).
        constexpr bool kScalesFirst = UNIFORM && F == PLM_INT4 && !A8;
        if constexpr (kScalesFirst) {
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) {
                const int kt = kt0 + tt;
                const int s_off = kt < w_hi ? (kt * kTileK / a.group_size) * a.scale_cols * ES : kOOB;
#pragma unroll
                for (int j = 0; j < SP; ++j) {
                    if constexpr (WIDE) b.s[tt][j] = buffer_load_u32(sr[j], s_lane, s_off);
                    else b.s[tt][j] = buffer_load_u16(sr[j], s_lane, s_off);
                }
            }
        }
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
            const int kt = kt0 + tt;
            const bool ok = kt < w_hi;  // wave-uniform
            const int w_off = ok ? kt * TB : kOOB;
            const int x_off = ok ? kt * kTileK * (A8 ? 1 : 2) : kOOB;
#pragma unroll
            for (int j = 0; j < SP; ++j) {
#pragma unroll
                for (int h = 0; h < TB / 1024; ++h) b.w[tt][j][h] = buffer_load16_stream(wr[j], w_lane + h * 1024, w_off);
                if constexpr (UNIFORM && !kScalesFirst) {
                    const int s_off = ok ? (kt * kTileK / a.group_size) * a.scale_cols * ES : kOOB;
                    if constexpr (WIDE) b.s[tt][j] = buffer_load_u32(sr[j], s_lane, s_off);
                    else b.s[tt][j] = buffer_load_u16(sr[j], s_lane, s_off);
                }
            }
            if constexpr (A8 && !QF) {
                b.x[tt][0][0] = buffer_load16(xr, x_lane[0], x_off);
                b.x[tt][0][1] = buffer_load16(xr, x_lane[0] + 16, x_off);
            } else if constexpr (!XS) {
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int t = 0; t < 4; ++t) b.x[tt][rb][t] = buffer_load16(xr, x_lane[rb] + 64 * t, x_off);
            }
        }
    };

    f32x4_t acc[RB][SP];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int j = 0; j < SP; ++j) acc[rb][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // XS: the wavefront copies its K range of x (rows < M, xs_row bytes each) into its own
    // LDS area with buffer loads to LDS, 1 KiB per instruction, instead of issuing four
    // mostly-empty 16-byte loads per K tile; the MFMA fragments are then read from LDS.
    extern __shared__ __attribute__((aligned(16))) uint8_t xs_lds[];
    uint8_t* xs_wave = xs_lds + wave * a.xs_wave;
    if constexpr (XS) {
        const int total = a.m * a.xs_row;
        for (int c = 0; c * 1024 < total; ++c) {  // wave-uniform
            const int o = c * 1024 + lane * 16;
            const int row = o / a.xs_row, col = o - row * a.xs_row;
            const int g = w_lo * kTileK * 2 + col;  // byte offset into the row
            const int off = (row < a.m && g < a.k * 2) ? row * a.k * 2 + g : kOOB;
            buffer_load_lds16(xr, xs_wave + c * 1024, off, 0);
        }
    }

    auto compute_batch = [&](const decode_batch<F, SP, TPW, A8, RB>& b, int kt0) {
        // int4 with uniform groups: the batch's scale constants and (staged) x fragments
        // are set up before its first dequant.
        [[maybe_unused]] int4_scale k4b[TPW][SP];
        [[maybe_unused]] u32x4_t xsb[TPW][4];
        if constexpr (F == PLM_INT4 && UNIFORM && !A8) {
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) {
#pragma unroll
                for (int j = 0; j < SP; ++j) k4b[tt][j] = make_int4_scale<BF16>(scale_from_bits<WIDE>(b.s[tt][j], bf16_scale));
                if constexpr (XS) {
                    const int kt = min(kt0 + tt, w_hi - 1);
                    const uint8_t* xr_lds = xs_wave + min(col16, a.m - 1) * a.xs_row + (kt - w_lo) * 256 + kq * 16;
#pragma unroll
                    for (int t = 0; t < 4; ++t) xsb[tt][t] = *reinterpret_cast<const u32x4_t*>(xr_lds + 64 * t);
                }
            }
        }
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
            const int kt = kt0 + tt;
            if (kt >= w_hi) break;  // wave-uniform
            if constexpr (A8) {  // x past K is already zero in the quantized copy
                u32x4_t x0, x1;
                if constexpr (QF) {  // e4m3 rows of xs_row / 2 bytes in the wavefront's area
                    const uint8_t* xp = xs_wave + min(col16, a.m - 1) * (a.xs_row >> 1) + (kt - w_lo) * kTileK + kq * 32;
                    x0 = *reinterpret_cast<const u32x4_t*>(xp);
                    x1 = *reinterpret_cast<const u32x4_t*>(xp + 16);
                } else {
                    x0 = b.x[tt][0][0];
                    x1 = b.x[tt][0][1];
                }
#pragma unroll
                for (int j = 0; j < SP; ++j) {
                    const float s = scale_from_bits<WIDE>(b.s[tt][j], bf16_scale);
                    const i32x8_t av = __builtin_bit_cast(i32x8_t, u32x8_cat(x0, x1));
                    const i32x8_t bv = __builtin_bit_cast(i32x8_t, u32x8_cat(b.w[tt][j][0], b.w[tt][j][TB / 1024 - 1]));
                    const f32x4_t part = mfma16x16x128_fp8(av, bv, f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[0][j][i] = __builtin_fmaf(s, part[i], acc[0][j][i]);
                }
                continue;
            }
            u32x4_t xs[RB][4];
            if constexpr (XS && F == PLM_INT4 && UNIFORM) {
#pragma unroll
                for (int t = 0; t < 4; ++t) xs[0][t] = xsb[tt][t];
            } else if constexpr (XS) {
                const uint8_t* xr_lds = xs_wave + min(col16, a.m - 1) * a.xs_row + (kt - w_lo) * 256 + kq * 16;
#pragma unroll
                for (int t = 0; t < 4; ++t) xs[0][t] = *reinterpret_cast<const u32x4_t*>(xr_lds + 64 * t);
            } else {
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int t = 0; t < 4; ++t) xs[rb][t] = b.x[tt][rb][t];
            }
            if ((kt + 1) * kTileK > a.k) {  // wave-uniform: partial last tile, zero x past K
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        if (kt * kTileK + 32 * t + 8 * kq >= a.k) xs[rb][t] = u32x4_t{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int j = 0; j < SP; ++j) {
                float s_tile = 0.f;
                int4_scale k4{};
                if constexpr (UNIFORM) {
                    const float raw = scale_from_bits<WIDE>(b.s[tt][j], bf16_scale);
                    s_tile = round_to<BF16>(raw);
                    if constexpr (F == PLM_INT4 && !A8) k4 = k4b[tt][j];
                }
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    float s = s_tile;
                    if constexpr (!UNIFORM) {
                        const int g = (kt * kTileK + 32 * t + 8 * kq) / a.group_size;
                        const uint32_t bits = WIDE ? buffer_load_u32(sr[j], s_lane + g * a.scale_cols * ES, 0)
                                                   : buffer_load_u16(sr[j], s_lane + g * a.scale_cols * ES, 0);
                        const float raw = scale_from_bits<WIDE>(bits, bf16_scale);
                        s = round_to<BF16>(raw);
                        if constexpr (F == PLM_INT4) k4 = make_int4_scale<BF16>(raw);
                    }
                    u32x4_t bop;
                    if constexpr (F == PLM_INT4) {
                        bop = dq_int4<BF16>(b.w[tt][j][0][t], k4);
                    } else {
                        const u32x4_t& v = b.w[tt][j][t >> 1];
                        bop = dq_fp8<BF16>(v[(t & 1) * 2], v[(t & 1) * 2 + 1], s);
                    }
#pragma unroll
                    for (int rb = 0; rb < RB; ++rb) acc[rb][j] = mfma16x16x32<BF16>(xs[rb][t], bop, acc[rb][j]);
                }
            }
        }
    };

    // One batch in flight per wavefront; latency is hidden by the other resident
    // wavefronts (a register double buffer gets rotated into copies that wait).
    // QF: the workgroup's row maxima [NW][4] and each wavefront's copy of the row scales
    // [NW][4] after the staging areas.
    [[maybe_unused]] float* amax_lds = reinterpret_cast<float*>(xs_lds + NW * a.xs_wave);
    [[maybe_unused]] float* scale_lds = amax_lds + NW * 4 + wave * 4;
    auto quantize_x = [&]() {
        if constexpr (QF) {
            const int chunks = a.xs_row >> 4;  // 16-byte chunks per staged row (16 per tile)
#pragma unroll 1
            for (int r = 0; r < a.m; ++r) {  // wave-uniform
                float mx = 0.f;
#pragma unroll 1
                for (int c = lane; c < chunks; c += 64) {
                    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xs_wave + r * a.xs_row + c * 16);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        mx = fmaxf(mx, fmaxf(fabsf(from_bits16<BF16>(v[j] & 0xffffu)),
                                             fabsf(from_bits16<BF16>(v[j] >> 16))));
                }
                mx = wave_max_to_lane63(mx);
                if (lane == 63) amax_lds[wave * 4 + r] = mx;
            }
            __syncthreads();
            // In place: chunk j (row j / chunks, K 8 (j % chunks) .. + 7) is read from byte
            // 16 j and its 8 codes go to byte 128 (j / 16) + 32 (j % 4) + 8 ((j / 4) % 4),
            // never past a byte this or an earlier pass has read.
#pragma unroll 1
            for (int r = 0; r < a.m; ++r) {  // wave-uniform
                float mx = 0.f;
#pragma unroll
                for (int w = 0; w < NW; ++w) mx = fmaxf(mx, amax_lds[w * 4 + r]);
                const float sc = fmaxf(mx, 1e-12f) / 448.f;
                const float inv = 1.f / sc;
                if (lane == 0) scale_lds[r] = sc;
#pragma unroll 1
                for (int c = lane; c < chunks; c += 64) {
                    const int j = r * chunks + c;
                    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xs_wave + j * 16);
                    auto div = [&](uint32_t bits) { return div_by_scale(from_bits16<BF16>(bits), sc, inv); };
                    int lo = 0, hi = 0;
                    lo = __builtin_amdgcn_cvt_pk_fp8_f32(div(v[0] & 0xffffu), div(v[0] >> 16), lo, false);
                    lo = __builtin_amdgcn_cvt_pk_fp8_f32(div(v[1] & 0xffffu), div(v[1] >> 16), lo, true);
                    hi = __builtin_amdgcn_cvt_pk_fp8_f32(div(v[2] & 0xffffu), div(v[2] >> 16), hi, false);
                    hi = __builtin_amdgcn_cvt_pk_fp8_f32(div(v[3] & 0xffffu), div(v[3] >> 16), hi, true);
                    *reinterpret_cast<uint2*>(xs_wave + 128 * (j >> 4) + 32 * (j & 3) + 8 * ((j >> 2) & 3)) =
                        make_uint2(static_cast<uint32_t>(lo), static_cast<uint32_t>(hi));
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
    };

    decode_batch<F, SP, TPW, A8, RB> b;
    for (int kt = w_lo; kt < w_hi; kt += TPW) {
        load_batch(b, kt);
        if constexpr (XS) {
            // The staging copy was issued before this batch's loads (weights and, for
            // uniform groups, scales): waiting until only those are outstanding means x has
            // landed. Later batches find it long done.
            constexpr int kBatchLoads = TPW * SP * (fmt_traits<F>::tile_bytes / 1024 + (UNIFORM ? 1 : 0));
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kBatchLoads) : "memory");
            if constexpr (QF) {
                if (kt == w_lo) quantize_x();  // every wavefront has a tile (checked on the host)
            }
        }
        compute_batch(b, kt);
    }
    if constexpr (A8) {  // row scales; rows past M are never stored
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float sx = QF ? scale_lds[min(4 * kq + i, a.m - 1)] : a.x_scale[min(4 * kq + i, a.m - 1)];
#pragma unroll
            for (int j = 0; j < SP; ++j) acc[0][j][i] *= sx;
        }
    }

    // Cross-wavefront reduction in a fixed order; slot rb * SP + j holds row block rb, strip j.
    __shared__ float red[NW][RB * SP][64][4];
    __shared__ uint32_t last_flag;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int j = 0; j < SP; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave][rb * SP + j][lane][i] = acc[rb][j][i];
    __syncthreads();

    constexpr int kElems = RB * SP * 64 * 4;
    constexpr int kPer = (kElems + NW * 64 - 1) / (NW * 64);
    float sum[kPer];
    int rows[kPer];
    int cols[kPer];
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        const int e = threadIdx.x + r * NW * 64;
        rows[r] = -1;
        if (e < kElems) {
            const int i = e & 3, ln = (e >> 2) & 63, slot = e >> 8, j = slot % SP, rb = slot / SP;
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) v += red[w][slot][ln][i];
            sum[r] = v;
            const int row = 16 * rb + 4 * (ln >> 4) + i;
            const int col = (sg * SP + j) * kTileN + (ln & 15);
            if (row < a.m && col < a.n) {
                rows[r] = row;
                cols[r] = col;
            }
        }
    }

    if (a.splits == 1) {
#pragma unroll
        for (int r = 0; r < kPer; ++r)
            if (rows[r] >= 0)
                a.y[static_cast<int64_t>(rows[r]) * a.n + cols[r]] = static_cast<uint16_t>(to_bits16<BF16>(sum[r]));
        return;
    }

    const int64_t mn = static_cast<int64_t>(a.m) * a.n;
#pragma unroll
    for (int r = 0; r < kPer; ++r)
        if (rows[r] >= 0) store_partial(&a.partial[split * mn + static_cast<int64_t>(rows[r]) * a.n + cols[r]], sum[r]);
    if (!arrive_last(&a.counters[sg], static_cast<uint32_t>(a.splits), &last_flag)) return;
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        if (rows[r] >= 0) {
            const int64_t off = static_cast<int64_t>(rows[r]) * a.n + cols[r];
            float v = 0.f;
            for (int sp = 0; sp < a.splits; ++sp) v += load_partial(&a.partial[sp * mn + off]);
            a.y[off] = static_cast<uint16_t>(to_bits16<BF16>(v));
        }
    }
}

// ---------------------------------------------------------------------------
// Round-robin decode kernel (M <= 4, scale groups a power-of-two multiple of 128).
//
// A workgroup owns SG strips over the whole of K, so no K split crosses workgroups and
// nothing waits on another workgroup. Its NW wavefronts take the K tiles round-robin
// (wavefront w takes tiles w, w + NW, ...): at each load step the workgroup's loads of a
// strip cover NW consecutive KiB. Each wavefront first copies into its own LDS area, with
// buffer loads to LDS, the x rows (< M) and the scales of its tiles (a few instructions
// instead of one scale load per tile); all address math is shifts and masks, so the
// weight loads issue right after. Weights are dequantized exactly (round(q * round(s)))
// into the MFMA operand; the wavefronts' partial sums are added through LDS in wavefront
// order and the workgroup stores y.
//
// SC: scale layout per (strip, group): 0 = 16 x 16-bit, 1 = 16 x fp32, 2 = 1 x fp32.
// ---------------------------------------------------------------------------
struct rr_args {
    const uint16_t* x;
    const uint8_t* w;
    const uint8_t* scale;
    uint16_t* y;
    int m, n, k;
    int ktiles, strips, groups;
    int tpg_shift;    // log2(group_size / 128)
    int nkt_shift;    // log2 of the per-wavefront tile slots (a power of two >= ceil(ktiles / NW))
    int x_bytes;      // per-wavefront x area: M rows x slots x 256 B, rounded to 1 KiB
    int wave_bytes;   // per-wavefront LDS area (x, then scales)
    int scale_dtype;
    // W8A8: e4m3 x in the quantizer's lane-permuted layout [M][ktiles][128] and row scales.
    const uint8_t* xq;
    const float* x_scale;
    // W8A8 with the quantizer fused (QF): offset of the wavefront's e4m3 x area in its LDS
    // area, and of the workgroup's per-wavefront row maxima after all wavefronts' areas.
    int qx_off, amax_off;
    int quant_fused;
};

template <int SC> struct rr_scale {
    static constexpr int eb = SC == 0 ? 32 : (SC == 1 ? 64 : 4);  // bytes per (strip, group)
    static constexpr int cs = eb < 16 ? eb : 16;                   // bytes per lane per copy
    static constexpr int parts_shift = SC == 0 ? 1 : (SC == 1 ? 2 : 0);
};

// Maximum of a non-negative float over the wavefront, in lane 63: DPP within each row of 16
// lanes (swap neighbours, swap pairs, half-row mirror, row mirror), then the row broadcasts
// carry row 0 into row 1 and rows 0-1 into rows 2-3. No LDS round trips.

//
// A8 (W8A8, fp8 weights): x is the per-token e4m3 copy, staged 128 bytes per (row, tile);
// each tile and strip is one v_mfma_scale_f32_16x16x128_f8f6f4 on the raw weight bytes, its
// partial scaled by the weight block scale, and the row scales applied at the end.
//
// QF (W8A8, M <= 4): the per-token quantizer runs inside this kernel. x is staged in bf16 /
// fp16 as for W8A16; each wavefront takes the row maxima over its K tiles, the workgroup
// (which covers all of K) combines them through LDS, and every wavefront rounds its own
// tiles to e4m3 into the lane-permuted order of the fp8 MFMA operand, with the same
// arithmetic as plm_quantize_rows_e4m3 (max(amax, 1e-12) / 448, fp32 divide, RNE), so the
// codes and scales are those of the two-launch path. Every workgroup repeats the row maxima
// over x (L2 traffic of M * K * 2 bytes per workgroup), which at M <= 4 costs less than
// the second launch. Its registers are capped at 64 (eight waves per SIMD): uncapped, the
// quantizer's temporaries took it to 73-75 and one 16-wavefront workgroup per CU, and the
// second round of workgroups then waits behind the first (measured: 14.3 us instead of
// 8.2 us at K = 5120, N = 7168). With 3-tile batches (40 tiles over 16 wavefronts) and
// the end-of-kernel row scales read from LDS, 64 holds without spills.
template <plm_format F, bool BF16, int SG, int NW, int CH, int SC, bool A8 = false, bool QF = false>
__global__ void __launch_bounds__(NW * 64, QF ? 8 : 1) decode_rr_kernel(rr_args a) {
    static_assert(!A8 || F == PLM_FP8, "W8A8 takes fp8 weights");
    static_assert(!QF || (A8 && SG == 1), "the fused quantizer is for W8A8, one strip per workgroup");
    constexpr int TB = fmt_traits<F>::tile_bytes;
    constexpr int NL = TB / 1024;  // 16-byte loads per lane per tile
    constexpr int EB = rr_scale<SC>::eb, CS = rr_scale<SC>::cs, PS = rr_scale<SC>::parts_shift;
    constexpr bool WIDE = SC != 0;
    const int lane = threadIdx.x & 63;
    const int wave = uniform(threadIdx.x >> 6);
    const int col16 = lane & 15;
    const int kq = lane >> 4;
    const int strip0 = blockIdx.x * SG;
    const int nkt_w = (a.ktiles - wave + NW - 1) / NW;  // this wavefront's tiles
    const int slots = 1 << a.nkt_shift;
    const bool bf16_scale = a.scale_dtype == PLM_BF16;

    extern __shared__ __attribute__((aligned(16))) uint8_t rr_lds[];
    uint8_t* xs = rr_lds + wave * a.wave_bytes;
    uint8_t* ss = xs + a.x_bytes;

    // x: 16-byte chunk j = (row, slot i, column o), LDS [row][slot][256 B] (A8: 128 B of e4m3).
    if constexpr (A8 && !QF) {
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.xq, static_cast<uint32_t>(a.m) * a.ktiles * kTileK);
        const int total = a.m << (a.nkt_shift + 3);
        for (int c = 0; c * 64 < total; ++c) {  // wave-uniform
            const int j = c * 64 + lane;
            const int o = j & 7, i = (j >> 3) & (slots - 1), row = j >> (a.nkt_shift + 3);
            const int off = (row < a.m && i < nkt_w) ? (row * a.ktiles + wave + NW * i) * kTileK + (o << 4) : kOOB;
            buffer_load_lds16(xr, xs + c * 1024, off, 0);
        }
    } else {
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, static_cast<uint32_t>(a.m) * a.k * 2);
        const int total = a.m << (a.nkt_shift + 4);
        for (int c = 0; c * 64 < total; ++c) {  // wave-uniform
            const int j = c * 64 + lane;
            const int o = j & 15, i = (j >> 4) & (slots - 1), row = j >> (a.nkt_shift + 4);
            const int kb = ((wave + NW * i) << 8) + (o << 4);  // byte offset in the row
            const int off = (row < a.m && i < nkt_w && kb < a.k * 2) ? row * a.k * 2 + kb : kOOB;
            buffer_load_lds16(xr, xs + c * 1024, off, 0);
        }
    }
    // Scales: entry (strip sj, slot i) of EB bytes, LDS [sj][slot][EB], CS bytes per lane.
    {
        const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.scale, static_cast<uint32_t>(a.strips) * a.groups * EB);
        const int total = (SG << a.nkt_shift) << PS;
        for (int c = 0; c * 64 < total; ++c) {  // wave-uniform
            const int j = c * 64 + lane;
            const int e = j >> PS, p = j & ((1 << PS) - 1);
            const int sj = e >> a.nkt_shift, i = e & (slots - 1);
            const int st = min(strip0 + sj, a.strips - 1);
            const int g = (wave + NW * i) >> a.tpg_shift;
            const int off = (sj < SG && i < nkt_w) ? (st * a.groups + g) * EB + p * CS : kOOB;
            auto* dst = (__attribute__((address_space(3))) void*)(ss + c * 64 * CS);
            if constexpr (CS == 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, dst, 16, off, 0, 0, 0);
            else __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, dst, 4, off, 0, 0, 0);
        }
    }
    asm volatile("" ::: "memory");  // the weight loads below are issued after the staging copies

    __amdgpu_buffer_rsrc_t wr[SG];
#pragma unroll
    for (int sj = 0; sj < SG; ++sj) {
        const int st = min(strip0 + sj, a.strips - 1);
        wr[sj] = make_rsrc(a.w + static_cast<int64_t>(st) * a.ktiles * TB, static_cast<uint32_t>(a.ktiles) * TB);
    }
    const int w_lane = lane * 16;

    f32x4_t acc[SG];
#pragma unroll
    for (int sj = 0; sj < SG; ++sj) acc[sj] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const int xrow = min(col16, a.m - 1);
    // QF: the workgroup's row maxima, [wavefront][4 rows] fp32 after every wavefront's area
    // (untouched until the kernel ends), and the e4m3 copy of this wavefront's x tiles.
    [[maybe_unused]] const float* amax_lds = reinterpret_cast<const float*>(rr_lds + a.amax_off);
    [[maybe_unused]] uint8_t* xq8 = xs + a.qx_off;
    // Each wavefront's copy of the row scales, [wavefront][4] after the maxima, for the end.
    [[maybe_unused]] float* scale_lds = reinterpret_cast<float*>(rr_lds + a.amax_off) + NW * 4 + wave * 4;
    auto row_scale = [&](int r) {
        float mx = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) mx = fmaxf(mx, amax_lds[w * 4 + r]);
        return fmaxf(mx, 1e-12f) / 448.f;
    };
    auto quantize_x = [&]() {
        if constexpr (QF) {
            const int chunks = nkt_w * 16;  // 16-byte chunks per row in this wavefront's tiles
#pragma unroll 1
            for (int r = 0; r < (a.m); ++r) {  // wave-uniform
                float mx = 0.f;
#pragma unroll 1
                for (int c = lane; c < chunks; c += 64) {
                    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(
                        xs + (((r << a.nkt_shift) + (c >> 4)) << 8) + ((c & 15) << 4));
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        mx = fmaxf(mx, fmaxf(fabsf(from_bits16<BF16>(v[j] & 0xffffu)),
                                             fabsf(from_bits16<BF16>(v[j] >> 16))));
                }
                mx = wave_max_to_lane63(mx);
                if (lane == 63) const_cast<float*>(amax_lds)[wave * 4 + r] = mx;
            }
            __syncthreads();
            // Chunk c of a (row, slot) holds K 8c .. 8c + 7 = 32 t + 8 kq + 0..7 with t = c / 4,
            // kq = c % 4; its codes go to byte 32 kq + 8 t of the slot's 128 bytes.
            const int per_row = nkt_w * 16;  // only this wavefront's tiles are read back
#pragma unroll 1
            for (int r = 0; r < (a.m); ++r) {  // wave-uniform
                const float sc = row_scale(r);
                const float inv = 1.f / sc;
                if (lane == 0) scale_lds[r] = sc;
#pragma unroll 1
                for (int j = lane; j < per_row; j += 64) {
                    const int c = j & 15, slot = (r << a.nkt_shift) + (j >> 4);
                    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xs + (slot << 8) + (c << 4));
                    auto div = [&](uint32_t bits) { return div_by_scale(from_bits16<BF16>(bits), sc, inv); };
                    int lo = 0, hi = 0;
                    lo = __builtin_amdgcn_cvt_pk_fp8_f32(div(v[0] & 0xffffu), div(v[0] >> 16), lo, false);
                    lo = __builtin_amdgcn_cvt_pk_fp8_f32(div(v[1] & 0xffffu), div(v[1] >> 16), lo, true);
                    hi = __builtin_amdgcn_cvt_pk_fp8_f32(div(v[2] & 0xffffu), div(v[2] >> 16), hi, false);
                    hi = __builtin_amdgcn_cvt_pk_fp8_f32(div(v[3] & 0xffffu), div(v[3] >> 16), hi, true);
                    *reinterpret_cast<uint2*>(xq8 + (slot << 7) + 32 * (c & 3) + 8 * (c >> 2)) =
                        make_uint2(static_cast<uint32_t>(lo), static_cast<uint32_t>(hi));
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
    };
    for (int i0 = 0; i0 < nkt_w; i0 += CH) {  // wave-uniform
        u32x4_t wv[CH][SG][NL];
#pragma unroll
        for (int ii = 0; ii < CH; ++ii) {
            const int i = i0 + ii;
            const int w_off = i < nkt_w ? (wave + NW * i) * TB : kOOB;
#pragma unroll
            for (int sj = 0; sj < SG; ++sj)
#pragma unroll
                for (int h = 0; h < NL; ++h) wv[ii][sj][h] = buffer_load16_stream(wr[sj], w_lane + h * 1024, w_off);
        }
        if (i0 == 0) {
            // The staging copies were issued before these loads: once only the weight loads
            // are outstanding, the wavefront's x and scales are in LDS.
            constexpr int kLoads = CH * SG * NL;
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLoads) : "memory");
            if constexpr (QF) quantize_x();  // every wavefront gets here (host: ktiles >= NW)
        }
        // int4: every tile's x fragments and (for up to four tiles x strips) scale constants
        // of this batch are read and set up before the first dequant, i.e. while the weight
        // loads are still in flight. Larger batches set the scales up per tile (registers).
        constexpr bool kScalesAhead = CH * SG <= 4;
        auto int4_scale_of = [&](int i, int sj) {
            const uint8_t* sp = ss + (((sj << a.nkt_shift) + i) * EB) + (SC == 2 ? 0 : col16 * (WIDE ? 4 : 2));
            const uint32_t bits = WIDE ? *reinterpret_cast<const uint32_t*>(sp)
                                       : static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(sp));
            return make_int4_scale<BF16>(scale_from_bits<WIDE>(bits, bf16_scale));
        };
        [[maybe_unused]] u32x4_t xfb[CH][4];
        [[maybe_unused]] int4_scale k4b[kScalesAhead ? CH : 1][kScalesAhead ? SG : 1];
        if constexpr (F == PLM_INT4 && !A8) {
#pragma unroll
            for (int ii = 0; ii < CH; ++ii) {
                const int i = min(i0 + ii, slots - 1);
                const uint8_t* xp = xs + (((xrow << a.nkt_shift) + i) << 8) + kq * 16;
#pragma unroll
                for (int t = 0; t < 4; ++t) xfb[ii][t] = *reinterpret_cast<const u32x4_t*>(xp + 64 * t);
                if constexpr (kScalesAhead) {
#pragma unroll
                    for (int sj = 0; sj < SG; ++sj) k4b[ii][sj] = int4_scale_of(i, sj);
                }
            }
        }
#pragma unroll
        for (int ii = 0; ii < CH; ++ii) {
            const int i = i0 + ii;
            if (i >= nkt_w) break;  // wave-uniform
            if constexpr (F == PLM_INT4 && !A8) {
#pragma unroll
                for (int sj = 0; sj < SG; ++sj) {
                    int4_scale k4;
                    if constexpr (kScalesAhead) k4 = k4b[ii][sj];
                    else k4 = int4_scale_of(i, sj);
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        acc[sj] = mfma16x16x32<BF16>(xfb[ii][t], dq_int4<BF16>(wv[ii][sj][0][t], k4), acc[sj]);
                }
                continue;
            }
            if constexpr (A8) {
                const uint8_t* xp = (QF ? xq8 : xs) + (((xrow << a.nkt_shift) + i) << 7) + kq * 32;
                const i32x8_t av = __builtin_bit_cast(
                    i32x8_t, u32x8_cat(*reinterpret_cast<const u32x4_t*>(xp), *reinterpret_cast<const u32x4_t*>(xp + 16)));
#pragma unroll
                for (int sj = 0; sj < SG; ++sj) {
                    const uint8_t* sp = ss + (((sj << a.nkt_shift) + i) * EB) + (SC == 2 ? 0 : col16 * (WIDE ? 4 : 2));
                    const uint32_t bits = WIDE ? *reinterpret_cast<const uint32_t*>(sp)
                                               : static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(sp));
                    const float sc = scale_from_bits<WIDE>(bits, bf16_scale);
                    const i32x8_t bv = __builtin_bit_cast(i32x8_t, u32x8_cat(wv[ii][sj][0], wv[ii][sj][NL - 1]));
                    const f32x4_t part = mfma16x16x128_fp8(av, bv, f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[sj][r] = __builtin_fmaf(sc, part[r], acc[sj][r]);
                }
                continue;
            }
            u32x4_t xf[4];
            const uint8_t* xp = xs + (((xrow << a.nkt_shift) + i) << 8) + kq * 16;
#pragma unroll
            for (int t = 0; t < 4; ++t) xf[t] = *reinterpret_cast<const u32x4_t*>(xp + 64 * t);
#pragma unroll
            for (int sj = 0; sj < SG; ++sj) {
                const uint8_t* sp = ss + (((sj << a.nkt_shift) + i) * EB) + (SC == 2 ? 0 : col16 * (WIDE ? 4 : 2));
                const uint32_t bits = WIDE ? *reinterpret_cast<const uint32_t*>(sp)
                                           : static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(sp));
                const float raw = scale_from_bits<WIDE>(bits, bf16_scale);
                if constexpr (F == PLM_INT4) {
                    const int4_scale k4 = make_int4_scale<BF16>(raw);
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        acc[sj] = mfma16x16x32<BF16>(xf[t], dq_int4<BF16>(wv[ii][sj][0][t], k4), acc[sj]);
                } else {
                    const float sc = round_to<BF16>(raw);
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const u32x4_t& v = wv[ii][sj][t >> 1];
                        acc[sj] = mfma16x16x32<BF16>(xf[t], dq_fp8<BF16>(v[(t & 1) * 2], v[(t & 1) * 2 + 1], sc), acc[sj]);
                    }
                }
            }
        }
    }

    if constexpr (A8) {  // row scales (rows 4 kq + r; rows past M are never stored)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float sx;
            // M <= 4: only rows 0..3 are stored.
            if constexpr (QF) sx = scale_lds[min(r, a.m - 1)];
            else sx = a.x_scale[min(4 * kq + r, a.m - 1)];
#pragma unroll
            for (int sj = 0; sj < SG; ++sj) acc[sj][r] *= sx;
        }
    }

    // Partial sums through LDS, over the staging areas once every wavefront is done with
    // them: red[sj][wave][lane < 16 RQ][4], rows 4 (lane / 16) + i of column lane % 16.
    const int rq = (a.m + 3) >> 2;
    float* red = reinterpret_cast<float*>(rr_lds);
    __syncthreads();
    if (lane < 16 * rq) {
#pragma unroll
        for (int sj = 0; sj < SG; ++sj)
            *reinterpret_cast<f32x4_t*>(red + (((sj * NW + wave) << 6) + lane) * 4) = acc[sj];
    }
    __syncthreads();
    for (int e = threadIdx.x; e < SG * 256; e += NW * 64) {
        const int c = e & 15, row = (e >> 4) & 15, sj = e >> 8;
        const int col = (strip0 + sj) * kTileN + c;
        if (row < a.m && col < a.n) {
            const int ln = c + 16 * (row >> 2), i = row & 3;
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) v += red[(((sj * NW + w) << 6) + ln) * 4 + i];
            a.y[static_cast<int64_t>(row) * a.n + col] = static_cast<uint16_t>(to_bits16<BF16>(v));
        }
    }
}

}  // namespace

struct decode_config {
    int sp;           // strips per wavefront
    int tpw;          // K tiles per load batch
    int nw;           // wavefronts per workgroup
    int splits;       // K splits across workgroups (1 = none)
    int tiles_per_split;
    int strip_groups;
};

decode_config choose_decode(plm_format f, int64_t m, int64_t n, int64_t k) {
    decode_config c{};
    const int64_t strips = ceil_div(n, kTileN), ktiles = ceil_div(k, kTileK);
    const int64_t cus = cu_count();
    // Measured on MI355X at the Qwen3-8B shapes (int4, g128): two strips per wavefront
    // (halving the x traffic per weight byte) pays when there are many strips or M > 4,
    // four when M > 4 and the strip groups still fill most of the GPU; otherwise one strip
    // and two K tiles per batch; 16 wavefronts split K.
    const int64_t groups4 = ceil_div(strips, 4);
    const int64_t wgs4 = groups4 * std::min<int64_t>(ceil_div(cus, groups4), std::max<int64_t>(1, ktiles / 16));
    // fp8 (2 KiB tiles) at M > 4, measured at the Qwen3-27B-like shapes: four-strip groups
    // when their workgroups, with the K split they get, fit one round of the CUs (o: 240) or K
    // is long enough that two-strip wavefronts would chain many load batches (down, 136 K
    // tiles); otherwise two strips on 8 wavefronts (qkv: 336 four-strip workgroups would take
    // two rounds; 15.4 -> 12.9 us at M=16, and o 12.6 -> 10.0 us the other way).
    const int64_t wgs4_split = groups4 * std::min<int64_t>(ceil_div(cus, groups4), ceil_div(ktiles, 16));
    if (strips >= 4 * cus) {
        c.sp = 2, c.tpw = 1, c.nw = 16;
    } else if (f == PLM_FP8 && m > 4 && ktiles >= 32) {
        if (wgs4_split <= cus || ktiles >= 96) c.sp = 4, c.tpw = 1, c.nw = 16;
        else c.sp = 2, c.tpw = 1, c.nw = 8;
    } else if (m > 4 && ktiles >= 32 && 4 * wgs4 >= 3 * cus) {
        c.sp = 4, c.tpw = 1, c.nw = 16;
    } else if (m > 4) {
        c.sp = 2, c.tpw = 1, c.nw = 8;
    } else {
        c.sp = 1, c.tpw = 2, c.nw = 16;
    }
    if (ktiles < 2 * c.nw) c.nw = ktiles >= 16 ? 8 : 4;
    if (knobs().decode_sp > 0) {  // PLM_DECODE="sp,tpw,nw" (tuning sweeps)
        c.sp = knobs().decode_sp;
        c.tpw = knobs().decode_tpw;
        c.nw = knobs().decode_nw;
    }
    if (c.sp == 4 && (c.tpw != 1 || c.nw != 16)) c.sp = 2;  // four strips: one instantiation only
    if (c.sp > 1) c.tpw = 1;                                 // two tiles per batch: one strip only
    c.strip_groups = static_cast<int>(ceil_div(strips, c.sp));
    // Split K across workgroups only when the column blocks alone cannot fill the GPU.
    int64_t splits = 1;
    if (c.strip_groups < cus && c.strip_groups <= kMaxCounters)
        splits = std::min<int64_t>(ceil_div(cus, c.strip_groups), ceil_div(ktiles, c.nw));
    c.tiles_per_split = static_cast<int>(ceil_div(ktiles, splits));
    c.splits = static_cast<int>(ceil_div(ktiles, c.tiles_per_split));
    return c;
}

int64_t decode_workspace_bytes(plm_format f, int64_t m, int64_t n, int64_t k) {
    const decode_config c = choose_decode(f, m, n, k);
    if (c.splits <= 1) return 0;
    return kCounterBytes + static_cast<int64_t>(c.splits) * m * n * 4;
}

namespace {
template <plm_format F, bool BF16, int SP, int TPW, int NW, int RB = 1>
void launch_decode_t(const decode_args& a, int strip_groups, bool uniform, hipStream_t s) {
    dim3 grid(strip_groups, a.splits);
    const bool wide = a.scale_dtype == PLM_FP32;
    if constexpr (RB == 2) {  // 16 < M <= 32: x from global memory, no W8A8
        if (uniform) {
            if (wide) decode_kernel<F, BF16, SP, TPW, NW, true, true, false, false, 2><<<grid, NW * 64, 0, s>>>(a);
            else decode_kernel<F, BF16, SP, TPW, NW, true, false, false, false, 2><<<grid, NW * 64, 0, s>>>(a);
        } else {
            if (wide) decode_kernel<F, BF16, SP, TPW, NW, false, true, false, false, 2><<<grid, NW * 64, 0, s>>>(a);
            else decode_kernel<F, BF16, SP, TPW, NW, false, false, false, false, 2><<<grid, NW * 64, 0, s>>>(a);
        }
        return;
    }
    if constexpr (F == PLM_FP8 && SP == 1 && TPW == 2 && NW == 16) {
        if (a.quant_fused) {  // W8A8 with the quantizer in the kernel (conditions: launch_decode)
            const size_t lds = static_cast<size_t>(NW) * a.xs_wave + NW * 32;
            if (wide) decode_kernel<F, BF16, SP, TPW, NW, true, true, true, true, 1, true><<<grid, NW * 64, lds, s>>>(a);
            else decode_kernel<F, BF16, SP, TPW, NW, true, false, true, true, 1, true><<<grid, NW * 64, lds, s>>>(a);
            return;
        }
    }
    if constexpr (F == PLM_FP8) {
        if (a.xq != nullptr) {  // W8A8 (group_size % 128 == 0 is checked by the caller)
            if (wide) decode_kernel<F, BF16, SP, TPW, NW, true, true, true><<<grid, NW * 64, 0, s>>>(a);
            else decode_kernel<F, BF16, SP, TPW, NW, true, false, true><<<grid, NW * 64, 0, s>>>(a);
            return;
        }
    }
    if (a.xs_wave > 0) {  // x staged in LDS
        const size_t lds = static_cast<size_t>(NW) * a.xs_wave;
        if (uniform) {
            if (wide) decode_kernel<F, BF16, SP, TPW, NW, true, true, false, true><<<grid, NW * 64, lds, s>>>(a);
            else decode_kernel<F, BF16, SP, TPW, NW, true, false, false, true><<<grid, NW * 64, lds, s>>>(a);
        } else {
            if (wide) decode_kernel<F, BF16, SP, TPW, NW, false, true, false, true><<<grid, NW * 64, lds, s>>>(a);
            else decode_kernel<F, BF16, SP, TPW, NW, false, false, false, true><<<grid, NW * 64, lds, s>>>(a);
        }
        return;
    }
    if (uniform) {
        if (wide) decode_kernel<F, BF16, SP, TPW, NW, true, true><<<grid, NW * 64, 0, s>>>(a);
        else decode_kernel<F, BF16, SP, TPW, NW, true, false><<<grid, NW * 64, 0, s>>>(a);
    } else {
        if (wide) decode_kernel<F, BF16, SP, TPW, NW, false, true><<<grid, NW * 64, 0, s>>>(a);
        else decode_kernel<F, BF16, SP, TPW, NW, false, false><<<grid, NW * 64, 0, s>>>(a);
    }
}

template <plm_format F, bool BF16, int SP, int TPW, int RB>
void launch_decode_nw(const decode_args& a, const decode_config& c, bool uniform, hipStream_t s) {
    switch (c.nw) {
        case 4: launch_decode_t<F, BF16, SP, TPW, 4, RB>(a, c.strip_groups, uniform, s); break;
        case 8: launch_decode_t<F, BF16, SP, TPW, 8, RB>(a, c.strip_groups, uniform, s); break;
        default: launch_decode_t<F, BF16, SP, TPW, 16, RB>(a, c.strip_groups, uniform, s); break;
    }
}

// Two tiles per batch only with one strip and one row block: the other combinations hold
// too many fragments for the 128 VGPRs of 1024-thread workgroups (they spilled) and were
// never the measured choice.
template <plm_format F, bool BF16, int SP, int RB>
void launch_decode_sp(const decode_args& a, const decode_config& c, bool uniform, hipStream_t s) {
    if constexpr (SP == 1 && RB == 1) {
        if (c.tpw == 2) {
            launch_decode_nw<F, BF16, SP, 2, RB>(a, c, uniform, s);
            return;
        }
    }
    launch_decode_nw<F, BF16, SP, 1, RB>(a, c, uniform, s);
}

template <plm_format F, bool BF16, int RB = 1>
void launch_decode_f(const decode_args& a, const decode_config& c, bool uniform, hipStream_t s) {
    if (c.sp == 1) launch_decode_sp<F, BF16, 1, RB>(a, c, uniform, s);
    else if (c.sp == 2) launch_decode_sp<F, BF16, 2, RB>(a, c, uniform, s);
    else launch_decode_t<F, BF16, 4, 1, 16, RB>(a, c.strip_groups, uniform, s);
}
}  // namespace

namespace {
template <plm_format F, bool BF16, int SG, int NW, int CH>
void launch_rr_t(const rr_args& a, int sc, int grid, size_t lds, hipStream_t s) {
    if constexpr (F == PLM_FP8) {
        if constexpr (SG == 1) {  // W8A8, quantizer in the kernel (3-tile batches; host: ktiles <= 3 NW)
            if (a.quant_fused) {
                if (sc == 0) decode_rr_kernel<F, BF16, SG, NW, 3, 0, true, true><<<grid, NW * 64, lds, s>>>(a);
                else if (sc == 1) decode_rr_kernel<F, BF16, SG, NW, 3, 1, true, true><<<grid, NW * 64, lds, s>>>(a);
                else decode_rr_kernel<F, BF16, SG, NW, 3, 2, true, true><<<grid, NW * 64, lds, s>>>(a);
                return;
            }
        }
        if (a.xq != nullptr) {  // W8A8
            if (sc == 0) decode_rr_kernel<F, BF16, SG, NW, CH, 0, true><<<grid, NW * 64, lds, s>>>(a);
            else if (sc == 1) decode_rr_kernel<F, BF16, SG, NW, CH, 1, true><<<grid, NW * 64, lds, s>>>(a);
            else decode_rr_kernel<F, BF16, SG, NW, CH, 2, true><<<grid, NW * 64, lds, s>>>(a);
            return;
        }
    }
    if (sc == 0) decode_rr_kernel<F, BF16, SG, NW, CH, 0><<<grid, NW * 64, lds, s>>>(a);
    else if (sc == 1) decode_rr_kernel<F, BF16, SG, NW, CH, 1><<<grid, NW * 64, lds, s>>>(a);
    else decode_rr_kernel<F, BF16, SG, NW, CH, 2><<<grid, NW * 64, lds, s>>>(a);
}
template <plm_format F, bool BF16, int NW, int CH>
void launch_rr_sg(const rr_args& a, int sc, int sg, size_t lds, hipStream_t s) {
    if constexpr (F == PLM_FP8) {  // fp8 tiles and 4-tile batches: at most two strips
        if (sg == 1) launch_rr_t<F, BF16, 1, NW, CH>(a, sc, a.strips, lds, s);
        else launch_rr_t<F, BF16, 2, NW, CH>(a, sc, static_cast<int>(ceil_div(a.strips, 2)), lds, s);
    } else {
        const int grid = static_cast<int>(ceil_div(a.strips, sg));
        switch (sg) {
            case 1: launch_rr_t<F, BF16, 1, NW, CH>(a, sc, grid, lds, s); break;
            case 2: launch_rr_t<F, BF16, 2, NW, CH>(a, sc, grid, lds, s); break;
            case 3: launch_rr_t<F, BF16, 3, NW, CH>(a, sc, grid, lds, s); break;
            case 4: launch_rr_t<F, BF16, 4, NW, CH>(a, sc, grid, lds, s); break;
            default: launch_rr_t<F, BF16, 6, NW, CH>(a, sc, grid, lds, s); break;
        }
    }
}
}  // namespace

struct rr_config {
    int sg = 0, nw = 0;  // sg == 0: not applicable
};

// Round-robin kernel choice (measured on MI355X at the Qwen3-8B shapes). M <= 4: one
// strip per workgroup, 16 wavefronts, or 8 when the strips alone give every CU four
// workgroups. M > 4 (x fills most of LDS, one workgroup per CU): strips grouped so that
// there is about one workgroup per CU.
// fp8 (2 KiB tiles) differs from int4 at the Qwen3-27B-like shapes (a sweep of every setting
// at M=1 and M=16): W8A16 at M <= 4 with fewer than 4 strips per CU takes two strips per
// workgroup when those fit one round of the CUs (o 8.3 -> 7.9 us, qkv 9.0 -> 8.6 us), and
// W8A8 above M=4 with many strips one strip on 8 wavefronts (gate_up at M=16 42.8 -> 39.0
// us). W8A8 at M <= 4 keeps one strip per workgroup for its fused quantizer (a two-strip
// fused variant measured slower: qkv 9.0 -> 9.7 us).
rr_config choose_rr(int64_t m, int64_t n, int64_t k, plm_format f, bool a8) {
    rr_config c;
    if (m > 16) return c;
    const int64_t strips = ceil_div(n, kTileN);
    const int64_t cus = cu_count();
    c.sg = 1;
    c.nw = 16;
    if (m <= 4) {
        if (strips >= 4 * cus) c.nw = 8;
        else if (f == PLM_FP8 && !a8 && ceil_div(strips, 2) <= cus) c.sg = 2;
    } else if (f == PLM_FP8 && a8 && strips >= 4 * cus) {
        c.nw = 8;
    } else {
        c.sg = 6;
        for (int sg : {1, 2, 3, 4}) {
            if (sg * cus >= strips) {
                c.sg = sg;
                break;
            }
        }
    }
    if (knobs().rr_sg == 0) return rr_config{};  // PLM_DECODE_RR="sg,nw" (tuning sweeps); "0" disables
    if (knobs().rr_sg > 0) {
        c.sg = knobs().rr_sg;
        c.nw = knobs().rr_nw;
    }
    (void)k;
    return c;
}

// x rows are staged in LDS for M up to this (above it the 16-byte loads of x are mostly full).
constexpr int64_t kStageMaxM = 4;
constexpr int64_t kStageMaxBytes = 96 * 1024;  // staging area per workgroup
bool no_x_staging() { return knobs().decode_no_xs; }  // A/B measurements

int launch_decode(const char* op, plm_format f, const void* x, bool bf16, const void* w, const void* scale,
                  plm_dtype scale_dtype, int64_t m, int64_t n, int64_t k, int64_t block_n, int64_t group_size,
                  void* y, void* workspace, size_t workspace_bytes, hipStream_t s, const uint8_t* xq,
                  const float* x_scale, bool quant_fused) {
    const decode_config c = choose_decode(f, m, n, k);
    const layout_dims d = make_dims(n, k, block_n, group_size);
    decode_args a{};
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
    a.xq = xq;
    a.x_scale = x_scale;
    if (m <= kStageMaxM && xq == nullptr && !no_x_staging()) {
        a.xs_row = static_cast<int>(ceil_div(c.tiles_per_split, c.nw)) * kTileK * 2;
        a.xs_wave = static_cast<int>(ceil_div(m * a.xs_row, 1024)) * 1024;
        if (static_cast<int64_t>(c.nw) * a.xs_wave > kStageMaxBytes) a.xs_row = a.xs_wave = 0;  // long K: direct loads
    }
    PLM_CHECK_ARG(c.splits > 0, op, "N = %lld is too large for the decode kernel", static_cast<long long>(n));
    // Buffer offsets stay below kOOB: x is at most 16 x K bf16, a weight strip K/128 tiles.
    PLM_CHECK_ARG(k <= (int64_t{1} << 24), op, "K must be at most 2^24");
    if (c.splits > 1) {
        const int64_t need = decode_workspace_bytes(f, m, n, k);
        if (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < need) {
            set_error(op, "workspace of %lld bytes required, %zu given", static_cast<long long>(need), workspace_bytes);
            return PLM_ERR_WORKSPACE;
        }
        a.counters = static_cast<uint32_t*>(workspace);
        a.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
    }
    const bool uniform = group_size % kTileK == 0;
    const int64_t tpg = group_size / kTileK;
    const int sc_mode = d.scale_cols == 16 ? (scale_dtype == PLM_FP32 ? 1 : 0) : (scale_dtype == PLM_FP32 ? 2 : -1);
    if (uniform && (tpg & (tpg - 1)) == 0 && sc_mode >= 0 && !no_x_staging()) {
        rr_config rc = choose_rr(m, n, k, f, xq != nullptr || quant_fused);
        // The fused quantizer takes at most three tiles per wavefront: 16 wavefronts where 8
        // would hold more (measured at N = 34816, K = 5120: 34.2 us, against 35.2 us for the
        // separate quantizer launch and 8 wavefronts).
        if (quant_fused && rc.sg == 1 && rc.nw == 8 && d.ktiles > 3 * 8) rc.nw = 16;
        if (rc.sg > 0) {
            rr_args r{};
            r.x = static_cast<const uint16_t*>(x);
            r.w = static_cast<const uint8_t*>(w);
            r.scale = static_cast<const uint8_t*>(scale);
            r.y = static_cast<uint16_t*>(y);
            r.m = static_cast<int>(m);
            r.n = static_cast<int>(n);
            r.k = static_cast<int>(k);
            r.ktiles = static_cast<int>(d.ktiles);
            r.strips = static_cast<int>(d.strips);
            r.groups = static_cast<int>(d.groups);
            r.scale_dtype = scale_dtype;
            r.xq = xq;
            r.x_scale = x_scale;
            r.quant_fused = quant_fused ? 1 : 0;
            while ((int64_t{1} << r.tpg_shift) < tpg) ++r.tpg_shift;
            const int64_t nkt = ceil_div(d.ktiles, rc.nw);
            while ((int64_t{1} << r.nkt_shift) < nkt) ++r.nkt_shift;
            const int64_t slots = int64_t{1} << r.nkt_shift;
            const int eb = sc_mode == 0 ? 32 : (sc_mode == 1 ? 64 : 4);
            r.x_bytes = static_cast<int>(round_up(m * slots * (xq != nullptr ? kTileK : 2 * kTileK), 1024));
            // Scale copies write whole instructions: 64 lanes x (16 or 4) bytes.
            const int64_t cs = eb < 16 ? eb : 16;
            const int64_t s_bytes = round_up(rc.sg * slots * eb, 64 * cs);
            // Fused quantizer: the wavefront's e4m3 x after its scales; after every wavefront's
            // area, the row maxima of all wavefronts, then their row scales (4 rows x fp32).
            r.qx_off = static_cast<int>(r.x_bytes + s_bytes);
            const int64_t q_bytes = quant_fused ? round_up(m * slots * kTileK, 1024) : 0;
            r.wave_bytes = static_cast<int>(r.x_bytes + s_bytes + q_bytes);
            r.amax_off = rc.nw * r.wave_bytes;
            const int64_t red = int64_t{rc.sg} * rc.nw * 64 * 16;
            const int64_t lds = std::max<int64_t>(int64_t{rc.nw} * r.wave_bytes + (quant_fused ? rc.nw * 32 : 0), red);
            // One batch of loads per wavefront (CH tiles) keeps every load in flight at once.
            const int64_t ch = f == PLM_FP8 ? 4 : (rc.nw == 16 ? 2 : 4);
            // The fused quantizer's barrier needs a tile for every wavefront; its register
            // budget holds one strip and at most three tiles per wavefront.
            const bool fused_ok = !quant_fused || (f == PLM_FP8 && m <= 4 && rc.sg == 1 && d.ktiles >= rc.nw &&
                                                   d.ktiles <= 3 * rc.nw);
            if (lds <= 160 * 1024 && slots <= ch && fused_ok) {
                const size_t l = static_cast<size_t>(lds);
                // CH: tiles per load batch (all of a wavefront's tiles at K = 4096).
                if (f == PLM_INT4) {
                    if (rc.nw == 16) {
                        if (bf16) launch_rr_sg<PLM_INT4, true, 16, 2>(r, sc_mode, rc.sg, l, s);
                        else launch_rr_sg<PLM_INT4, false, 16, 2>(r, sc_mode, rc.sg, l, s);
                    } else {
                        if (bf16) launch_rr_sg<PLM_INT4, true, 8, 4>(r, sc_mode, rc.sg, l, s);
                        else launch_rr_sg<PLM_INT4, false, 8, 4>(r, sc_mode, rc.sg, l, s);
                    }
                } else {
                    // fp8 (K = 5120 at the Qwen3-27B shapes: 40 tiles, up to 3 per wavefront).
                    if (rc.nw == 16) {
                        if (bf16) launch_rr_sg<PLM_FP8, true, 16, 4>(r, sc_mode, rc.sg, l, s);
                        else launch_rr_sg<PLM_FP8, false, 16, 4>(r, sc_mode, rc.sg, l, s);
                    } else {
                        if (bf16) launch_rr_sg<PLM_FP8, true, 8, 4>(r, sc_mode, rc.sg, l, s);
                        else launch_rr_sg<PLM_FP8, false, 8, 4>(r, sc_mode, rc.sg, l, s);
                    }
                }
                PLM_HIP_LAUNCH_CHECK(op);
                return PLM_OK;
            }
        }
    }
    if (quant_fused) {
        // The split-K kernel with the quantizer fused: one workgroup over all of K (the row
        // maxima stay inside it), x staged in LDS, every wavefront with a tile (all reach the
        // barrier), and the one instantiation (one strip, two-tile batches, 16 wavefronts).
        const int per_wave = static_cast<int>(ceil_div(c.tiles_per_split, c.nw));
        const bool ok = f == PLM_FP8 && m <= kStageMaxM && a.xs_wave > 0 && c.splits == 1 && uniform && c.sp == 1 &&
                        c.tpw == 2 && c.nw == 16 && (c.nw - 1) * per_wave < c.tiles_per_split &&
                        static_cast<int64_t>(c.nw) * a.xs_wave + c.nw * 32 <= 64 * 1024 * 2;
        if (!ok) return kDecodeNotTaken;
        a.quant_fused = 1;
        if (bf16) launch_decode_f<PLM_FP8, true>(a, c, uniform, s);
        else launch_decode_f<PLM_FP8, false>(a, c, uniform, s);
        PLM_HIP_LAUNCH_CHECK(op);
        return PLM_OK;
    }
    if (m > 16) {  // two 16-row blocks per MFMA pass (the caller sends W8A8 only up to 16 rows)
        PLM_CHECK_ARG(m <= 32 && xq == nullptr, op, "the decode kernels take at most 32 rows (16 for W8A8)");
        if (f == PLM_INT4) {
            if (bf16) launch_decode_f<PLM_INT4, true, 2>(a, c, uniform, s);
            else launch_decode_f<PLM_INT4, false, 2>(a, c, uniform, s);
        } else {
            if (bf16) launch_decode_f<PLM_FP8, true, 2>(a, c, uniform, s);
            else launch_decode_f<PLM_FP8, false, 2>(a, c, uniform, s);
        }
        PLM_HIP_LAUNCH_CHECK(op);
        return PLM_OK;
    }
    if (f == PLM_INT4) {
        if (bf16) launch_decode_f<PLM_INT4, true>(a, c, uniform, s);
        else launch_decode_f<PLM_INT4, false>(a, c, uniform, s);
    } else {
        if (bf16) launch_decode_f<PLM_FP8, true>(a, c, uniform, s);
        else launch_decode_f<PLM_FP8, false>(a, c, uniform, s);
    }
    PLM_HIP_LAUNCH_CHECK(op);
    return PLM_OK;
}

}  // namespace plm
