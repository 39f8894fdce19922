// Bandwidth-first dequant-GEMM for decode (M <= 16): y[M, N] = x[M, K] @ dequant(W)^T.
//
// Counterpart of the reference's marlin_kernel at tile_m = 16 (pulsarlm-core/src/kernels/
// marlin.cu:251-389, dispatched for M <= 16 at :577-596) together with its split-K
// partial sum and combine (pulsarlm-core/inc/pulsarlm/kernels/dequant_gemm_common.cuh:
// 56-133). Designed for gfx950 rather than translated:
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
};

// One wavefront's batch of TPW K tiles for SP strips: weights, raw scales and x.
template <plm_format F, int SP, int TPW> struct decode_batch {
    u32x4_t w[TPW][SP][fmt_traits<F>::tile_bytes / 1024];
    float s[TPW][SP];
    u32x4_t x[TPW][4];
};

template <plm_format F, bool BF16, int SP, int TPW, int NW, bool UNIFORM>
__global__ void __launch_bounds__(NW * 64) decode_kernel(decode_args a) {
    constexpr int TB = fmt_traits<F>::tile_bytes;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
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
    const bool row_ok = col16 < a.m;

    auto scale_index = [&](int st, int g) -> int64_t {
        return (static_cast<int64_t>(st < a.strips ? st : a.strips - 1) * a.groups + g) * a.scale_cols +
               (a.scale_cols == 1 ? 0 : col16);
    };

    auto load_batch = [&](decode_batch<F, SP, TPW>& b, int kt0) {
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
            const int kt = kt0 + tt;
            const bool kt_ok = kt < w_hi;
#pragma unroll
            for (int j = 0; j < SP; ++j) {
                const int st = sg * SP + j;
#pragma unroll
                for (int h = 0; h < TB / 1024; ++h) {
                    if (kt_ok && st < a.strips) {
                        const int64_t off =
                            ((static_cast<int64_t>(st) * a.ktiles + kt) * (TB / 1024) + h) * 1024 + lane * 16;
                        b.w[tt][j][h] = *reinterpret_cast<const u32x4_t*>(a.w + off);
                    } else {
                        b.w[tt][j][h] = (F == PLM_INT4)
                                            ? u32x4_t{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u}
                                            : u32x4_t{0u, 0u, 0u, 0u};
                    }
                }
                if constexpr (UNIFORM)
                    b.s[tt][j] = kt_ok ? load_scale(a.scale, scale_index(st, kt * kTileK / a.group_size),
                                                    a.scale_dtype)
                                       : 0.f;
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int k0 = kt * kTileK + 32 * t + 8 * kq;
                if (kt_ok && row_ok && k0 < a.k)
                    b.x[tt][t] = *reinterpret_cast<const u32x4_t*>(a.x + static_cast<int64_t>(col16) * a.k + k0);
                else
                    b.x[tt][t] = u32x4_t{0u, 0u, 0u, 0u};
            }
        }
    };

    f32x4_t acc[SP];
#pragma unroll
    for (int j = 0; j < SP; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    auto compute_batch = [&](const decode_batch<F, SP, TPW>& b, int kt0) {
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
            const int kt = kt0 + tt;
            if (kt >= w_hi) break;
#pragma unroll
            for (int j = 0; j < SP; ++j) {
                const int st = sg * SP + j;
                float s_tile = 0.f;
                int4_scale k4{};
                if constexpr (UNIFORM) {
                    s_tile = round_to<BF16>(b.s[tt][j]);
                    if constexpr (F == PLM_INT4) k4 = make_int4_scale<BF16>(b.s[tt][j]);
                }
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    float s = s_tile;
                    if constexpr (!UNIFORM) {
                        const int g = (kt * kTileK + 32 * t + 8 * kq) / a.group_size;
                        const float raw = load_scale(a.scale, scale_index(st, g), a.scale_dtype);
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
                    acc[j] = mfma16x16x32<BF16>(b.x[tt][t], bop, acc[j]);
                }
            }
        }
    };

    // Register double buffering: batch i+1's loads are in flight while batch i computes.
    decode_batch<F, SP, TPW> b0, b1;
    int kt = w_lo;
    if (kt < w_hi) load_batch(b0, kt);
    while (kt < w_hi) {
        if (kt + TPW < w_hi) load_batch(b1, kt + TPW);
        compute_batch(b0, kt);
        kt += TPW;
        if (kt >= w_hi) break;
        if (kt + TPW < w_hi) load_batch(b0, kt + TPW);
        compute_batch(b1, kt);
        kt += TPW;
    }

    // Cross-wavefront reduction in a fixed order.
    __shared__ float red[NW][SP][64][4];
    __shared__ uint32_t last_flag;
#pragma unroll
    for (int j = 0; j < SP; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][j][lane][i] = acc[j][i];
    __syncthreads();

    constexpr int kElems = SP * 64 * 4;
    constexpr int kPer = (kElems + NW * 64 - 1) / (NW * 64);
    float sum[kPer];
    int rows[kPer];
    int cols[kPer];
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        const int e = threadIdx.x + r * NW * 64;
        rows[r] = -1;
        if (e < kElems) {
            const int i = e & 3, ln = (e >> 2) & 63, j = e >> 8;
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) v += red[w][j][ln][i];
            sum[r] = v;
            const int row = 4 * (ln >> 4) + i;
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
    c.sp = (m > 4 && strips >= 2 * cus) ? 2 : 1;
    c.nw = ktiles >= 32 ? 16 : (ktiles >= 8 ? 8 : 4);
    c.tpw = 2;
    if (const char* env = getenv("PLM_DECODE")) {  // "sp,tpw,nw" for tuning sweeps
        int sp = 0, t = 0, nw = 0;
        if (sscanf(env, "%d,%d,%d", &sp, &t, &nw) == 3 && (sp == 1 || sp == 2) && (t == 1 || t == 2 || t == 4) &&
            (nw == 4 || nw == 8 || nw == 16)) {
            c.sp = sp;
            c.tpw = t;
            c.nw = nw;
        }
    }
    (void)f;
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
template <plm_format F, bool BF16, int SP, int TPW, int NW>
void launch_decode_t(const decode_args& a, int strip_groups, bool uniform, hipStream_t s) {
    dim3 grid(strip_groups, a.splits);
    if (uniform)
        decode_kernel<F, BF16, SP, TPW, NW, true><<<grid, NW * 64, 0, s>>>(a);
    else
        decode_kernel<F, BF16, SP, TPW, NW, false><<<grid, NW * 64, 0, s>>>(a);
}

template <plm_format F, bool BF16, int SP, int TPW>
void launch_decode_nw(const decode_args& a, const decode_config& c, bool uniform, hipStream_t s) {
    switch (c.nw) {
        case 4: launch_decode_t<F, BF16, SP, TPW, 4>(a, c.strip_groups, uniform, s); break;
        case 8: launch_decode_t<F, BF16, SP, TPW, 8>(a, c.strip_groups, uniform, s); break;
        default: launch_decode_t<F, BF16, SP, TPW, 16>(a, c.strip_groups, uniform, s); break;
    }
}

template <plm_format F, bool BF16, int SP>
void launch_decode_sp(const decode_args& a, const decode_config& c, bool uniform, hipStream_t s) {
    switch (c.tpw) {
        case 1: launch_decode_nw<F, BF16, SP, 1>(a, c, uniform, s); break;
        case 4: launch_decode_nw<F, BF16, SP, 4>(a, c, uniform, s); break;
        default: launch_decode_nw<F, BF16, SP, 2>(a, c, uniform, s); break;
    }
}

template <plm_format F, bool BF16>
void launch_decode_f(const decode_args& a, const decode_config& c, bool uniform, hipStream_t s) {
    if (c.sp == 1) launch_decode_sp<F, BF16, 1>(a, c, uniform, s);
    else launch_decode_sp<F, BF16, 2>(a, c, uniform, s);
}
}  // namespace

int launch_decode(const char* op, plm_format f, const void* x, bool bf16, const void* w, const void* scale,
                  plm_dtype scale_dtype, int64_t m, int64_t n, int64_t k, int64_t block_n, int64_t group_size,
                  void* y, void* workspace, size_t workspace_bytes, hipStream_t s) {
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
    PLM_CHECK_ARG(c.splits > 0, op, "N = %lld is too large for the decode kernel", static_cast<long long>(n));
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
