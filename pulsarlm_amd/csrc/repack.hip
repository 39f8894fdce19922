// Load-time conversions into the plm tile layout, the dense dequant, and the
// C-ABI plumbing shared by every entry point (errors, sizes, device queries).
//
// Counterparts in the reference: repack_weight_kernel / transpose_scale_kernel /
// repack<> (pulsarlm-core/src/kernels/marlin.cu:197-236,395-445) and its
// exports repack_int4_marlin_cuda / repack_fp8_marlin_cuda (marlin.cu:601-629).
#include <algorithm>
#include <cstdarg>
#include <cstdlib>
#include <mutex>
#include <vector>

#include "plm_common.hpp"

namespace plm {

namespace {
thread_local std::string g_error;
}

void set_error(const char* op, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_error = std::string(op) + ": " + buf;
}

void clear_error() { g_error.clear(); }

int cu_count() {
    static std::mutex mu;
    static std::vector<int> counts;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if (static_cast<int>(counts.size()) <= dev) counts.resize(dev + 1, 0);
    if (counts[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        counts[dev] = n;
    }
    return counts[dev];
}

namespace {
tuning parse_tuning() {
    tuning t;
    auto env = [](const char* name) { return getenv(name); };
    if (const char* e = env("PLM_DECODE_MAX_M")) t.decode_max_m = std::min<int64_t>(32, std::max<int64_t>(0, atoll(e)));
    t.w8a8_unfused = env("PLM_W8A8_UNFUSED") != nullptr;
    if (const char* e = env("PLM_DECODE")) {
        int sp = 0, tp = 0, nw = 0;
        if (sscanf(e, "%d,%d,%d", &sp, &tp, &nw) == 3 && (sp == 1 || sp == 2 || sp == 4) && (tp == 1 || tp == 2) &&
            (nw == 4 || nw == 8 || nw == 16))
            t.decode_sp = sp, t.decode_tpw = tp, t.decode_nw = nw;
    }
    if (const char* e = env("PLM_DECODE_RR")) {
        int sg = 0, nw = 0;
        const int got = sscanf(e, "%d,%d", &sg, &nw);
        if (got >= 1 && sg == 0) t.rr_sg = 0;
        else if (got == 2 && (sg == 1 || sg == 2 || sg == 3 || sg == 4 || sg == 6) && (nw == 8 || nw == 16))
            t.rr_sg = sg, t.rr_nw = nw;
    }
    t.decode_no_xs = env("PLM_DECODE_NO_XS") != nullptr;
    if (const char* e = env("PLM_MFMA")) t.mfma_shape = e[0];
    t.mfma_no_halves = env("PLM_MFMA_NO_HALVES") != nullptr;
    t.mfma_no_tail = env("PLM_MFMA_NO_TAIL") != nullptr;
    t.mfma_unsplit = env("PLM_MFMA_UNSPLIT") != nullptr;
    if (const char* e = env("PLM_MOE_ROWS")) t.moe_rows = atoi(e);
    if (const char* e = env("PLM_MOE_SMALL_SORT")) t.moe_small_sort_off = e[0] == '0';
    t.moe_unfused = env("PLM_MOE_UNFUSED") != nullptr;
    if (const char* e = env("PLM_MOE_PERSIST")) t.moe_persist = e[0] == '1';
    return t;
}
std::mutex g_tuning_mutex;
tuning g_tuning;
bool g_tuning_parsed = false;
}  // namespace

const tuning& knobs() {
    static const bool once = [] {
        std::lock_guard<std::mutex> lock(g_tuning_mutex);
        if (!g_tuning_parsed) g_tuning = parse_tuning(), g_tuning_parsed = true;
        return true;
    }();
    (void)once;
    return g_tuning;
}

namespace {

// One thread per 32-bit word of the int4 layout: word ((strip*KT + kt)*64 + lane)*4 + t,
// lane = 16 g + 4 c + i, holds in nibble int4_nibble_pos(r, h) the value q + 8 of column
// strip*16 + 4c + r at K = kt*128 + 32t + 8g + 4h + i (r, h in 0..3 x 0..1). The eight
// values come from one source int32 (K/8 index kt*16 + 4t + g, nibble 4h + i) of each of
// the four columns.
__global__ void repack_int4_kernel(const int32_t* __restrict__ src, uint32_t* __restrict__ dst, int64_t n,
                                   int64_t k, int64_t ktiles, int64_t total) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int t = static_cast<int>(idx & 3);
    const int lane = static_cast<int>((idx >> 2) & 63);
    const int64_t tile = idx >> 8;
    const int64_t kt = tile % ktiles;
    const int64_t strip = tile / ktiles;
    const int g = lane >> 4, c = (lane >> 2) & 3, i = lane & 3;
    const int64_t k8 = kt * kTileK + 32 * t + 8 * g;  // first K of the source word
    uint32_t word = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t col = strip * kTileN + 4 * c + r;
        const uint32_t sw = (col < n && k8 < k) ? static_cast<uint32_t>(src[col * (k / 8) + k8 / 8]) : 0u;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t nib = ((sw >> (4 * (4 * h + i))) & 0xfu) ^ 8u;  // padding: q = 0
            word |= nib << (4 * int4_nibble_pos(r, h));
        }
    }
    dst[idx] = word;
}

// One thread per dword of the fp8 layout: byte (((strip*KT + kt)*2 + h)*64 + lane)*16 + (t%2)*8 + i,
// t = 2h + (dword%4)/2, i = 4*(dword%2) + 0..3.
__global__ void repack_fp8_kernel(const uint8_t* __restrict__ src, uint32_t* __restrict__ dst, int64_t n, int64_t k,
                                  int64_t ktiles, int64_t total) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int d = static_cast<int>(idx & 3);
    const int lane = static_cast<int>((idx >> 2) & 63);
    const int h = static_cast<int>((idx >> 8) & 1);
    const int64_t tile = idx >> 9;
    const int64_t kt = tile % ktiles;
    const int64_t strip = tile / ktiles;
    const int t = 2 * h + (d >> 1);
    const int64_t col = strip * kTileN + (lane & 15);
    const int64_t k0 = kt * kTileK + 32 * t + 8 * (lane >> 4) + 4 * (d & 1);
    uint32_t word = 0;
    if (col < n && k0 < k) {
        const uint8_t* p = src + col * k + k0;
        word = static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8) | (static_cast<uint32_t>(p[2]) << 16) |
               (static_cast<uint32_t>(p[3]) << 24);
    }
    dst[idx] = word;
}

// int4 scales whose bf16 rounding reaches 2^120 in magnitude are outside the domain of the
// GEMM kernels' matrix-core dequant, which forms (128 + u) s in fp32 before subtracting
// 136 s: at |s| >= 2^120 that product overflows where the reference's round(q round(s))
// stays finite. The int4 repacks flag such scales (check: 1 = fp32 bits, 2 = bf16 bits).
__device__ __forceinline__ void flag_scale_domain(uint32_t bits, int check, uint32_t* flag) {
    if (check == 0) return;
    const float v = __uint_as_float(check == 1 ? bits : bits << 16);
    if (fabsf(round_bf16(v)) >= 0x1p120f) atomicOr(flag, 1u);
}

// Scales [ceil(N/bn), K/g] -> [strips][groups][cols], same element size; padding 0.
template <typename T>
__global__ void repack_scale_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t n, int64_t k,
                                    int64_t block_n, int64_t group_size, int64_t groups, int cols, int64_t total,
                                    int check, uint32_t* flag) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int c = static_cast<int>(idx % cols);
    const int64_t g = (idx / cols) % groups;
    const int64_t strip = idx / (cols * groups);
    const int64_t col = strip * kTileN + c;
    const int64_t src_groups = k / group_size;
    T v{};
    if (col < n && g < src_groups) v = src[(col / block_n) * src_groups + g];
    dst[idx] = v;
    flag_scale_domain(static_cast<uint32_t>(v), check, flag);
}

// Reference Marlin words -> plm int4 words (the mapping of repack_int4_kernel). Marlin
// word index ((cb*KTm + k/32)*8 + subtile)*32 + lane_m with lane_m = 4*(n%8) + pair holds,
// in nibble j + 4*odd, K offset 2*pair + odd + 8j (marlin.cu:86-117), already as q ^ 8.
__global__ void convert_marlin_int4_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst, int64_t n,
                                           int64_t k, int64_t ktiles, int64_t total) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int t = static_cast<int>(idx & 3);
    const int lane = static_cast<int>((idx >> 2) & 63);
    const int64_t tile = idx >> 8;
    const int64_t kt = tile % ktiles;
    const int64_t strip = tile / ktiles;
    const int g = lane >> 4, c = (lane >> 2) & 3, i = lane & 3;
    const int64_t ktm = ceil_div(k, 32);
    uint32_t word = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t col = strip * kTileN + 4 * c + r;
        const int64_t cb = col / 64, subtile = (col % 64) / 8;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t kk = kt * kTileK + 32 * t + 8 * g + 4 * h + i;
            uint32_t nib = 8u;  // padding: q = 0
            if (col < n && kk < k) {
                const int cm = static_cast<int>(kk % 32);
                const int pair = (cm % 8) / 2, odd = cm % 2, j = cm / 8;
                const int lane_m = static_cast<int>(col % 8) * 4 + pair;
                const uint32_t w = src[((cb * ktm + kk / 32) * 8 + subtile) * 32 + lane_m];
                nib = (w >> (4 * (j + 4 * odd))) & 0xfu;
            }
            word |= nib << (4 * int4_nibble_pos(r, h));
        }
    }
    dst[idx] = word;
}

// Reference fp8 Marlin words -> plm fp8 layout. Word w of lane_m holds K offsets
// 16w + 2*pair + {0, 1, 8, 9} in bytes 0..3 (marlin.cu:154-171).
__global__ void convert_marlin_fp8_kernel(const uint32_t* __restrict__ src, uint32_t* __restrict__ dst, int64_t n,
                                          int64_t k, int64_t ktiles, int64_t total) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int d = static_cast<int>(idx & 3);
    const int lane = static_cast<int>((idx >> 2) & 63);
    const int h = static_cast<int>((idx >> 8) & 1);
    const int64_t tile = idx >> 9;
    const int64_t kt = tile % ktiles;
    const int64_t strip = tile / ktiles;
    const int t = 2 * h + (d >> 1);
    const int64_t col = strip * kTileN + (lane & 15);
    const int64_t k0 = kt * kTileK + 32 * t + 8 * (lane >> 4) + 4 * (d & 1);
    uint32_t word = 0;
    if (col < n && k0 < k) {
        const int64_t ktm = ceil_div(k, 32);
        const int64_t cb = col / 64, subtile = (col % 64) / 8;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t kk = k0 + i;
            const int c = static_cast<int>(kk % 32);
            const int w = c / 16, cc = c % 16;
            const int pair = (cc % 8) / 2, sub = (cc % 2) + 2 * (cc / 8);
            const int lane_m = static_cast<int>(col % 8) * 4 + pair;
            const uint32_t src_word = src[(((cb * ktm + kk / 32) * 8 + subtile) * 2 + w) * 32 + lane_m];
            word |= ((src_word >> (8 * sub)) & 0xffu) << (8 * i);
        }
    }
    dst[idx] = word;
}

// scale_marlin fp32 [groups, rows] (marlin.cu:227-236) -> plm fp32 [strips][groups][cols].
__global__ void convert_marlin_scale_kernel(const float* __restrict__ src, float* __restrict__ dst, int64_t n,
                                            int64_t k, int64_t block_n, int64_t group_size, int64_t groups, int cols,
                                            int64_t total, int check, uint32_t* flag) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const int c = static_cast<int>(idx % cols);
    const int64_t g = (idx / cols) % groups;
    const int64_t strip = idx / (cols * groups);
    const int64_t col = strip * kTileN + c;
    const int64_t rows = ceil_div(n, block_n);
    float v = 0.f;
    if (col < n && g < k / group_size) v = src[g * rows + col / block_n];
    dst[idx] = v;
    flag_scale_domain(__float_as_uint(v), check, flag);
}

// Dense W[n, k] = round(q * round(scale)) in the output dtype, from the plm layout.
template <plm_format F, bool BF16>
__global__ void dequant_kernel(const uint8_t* __restrict__ w, const void* __restrict__ scale, int scale_dtype,
                               int64_t n, int64_t k, int64_t ktiles, int64_t group_size, int64_t groups, int cols,
                               uint16_t* __restrict__ out) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= n * k) return;
    const int64_t row = idx / k, col_k = idx % k;
    const int64_t strip = row / kTileN, kt = col_k / kTileK;
    const int kin = static_cast<int>(col_k % kTileK);
    const int t = kin / 32, kq = (kin % 32) / 8, i = kin % 8;
    const int lane = static_cast<int>(row % kTileN) + 16 * kq;
    float q;
    if constexpr (F == PLM_INT4) {
        const int c16 = static_cast<int>(row % kTileN);
        const int lane4 = 16 * kq + 4 * (c16 >> 2) + (i & 3);
        const uint32_t word = reinterpret_cast<const uint32_t*>(w)[((strip * ktiles + kt) * 64 + lane4) * 4 + t];
        const int pos = int4_nibble_pos(c16 & 3, i >> 2);
        q = static_cast<float>(static_cast<int>((word >> (4 * pos)) & 0xfu) - 8);
    } else {
        const int64_t off = ((strip * ktiles + kt) * 2 + t / 2) * 1024 + lane * 16 + (t % 2) * 8 + i;
        q = e4m3_to_f32(w[off]);
    }
    const int64_t sidx = (strip * groups + col_k / group_size) * cols + (cols == 1 ? 0 : row % kTileN);
    const float s = round_to<BF16>(load_scale(scale, sidx, scale_dtype));
    out[idx] = static_cast<uint16_t>(to_bits16<BF16>(q * s));
}

constexpr int kThreads = 256;

inline unsigned blocks_for(int64_t total) { return static_cast<unsigned>(ceil_div(total, kThreads)); }

int check_common(const char* op, plm_dtype scale_dtype, int64_t n, int64_t k, int64_t block_n, int64_t group_size) {
    PLM_CHECK_ARG(n >= 0 && k >= 0, op, "N and K must be non-negative");
    PLM_CHECK_ARG(block_n > 0, op, "block_n must be positive");
    PLM_CHECK_ARG(group_size > 0 && group_size % 16 == 0, op, "group_size must be a positive multiple of 16");
    PLM_CHECK_ARG(k % group_size == 0, op, "K must be a multiple of group_size");
    PLM_CHECK_ARG(scale_dtype == PLM_BF16 || scale_dtype == PLM_FP16 || scale_dtype == PLM_FP32, op,
                  "scale dtype must be bf16, fp16 or fp32");
    PLM_CHECK_ARG(n <= (int64_t{1} << 30) && k <= (int64_t{1} << 30), op, "N and K must be below 2^30");
    return PLM_OK;
}

// The scale-domain flag of the int4 repacks: one word per device in static device memory,
// addressed through hipGetSymbolAddress, cleared by a fill kernel before each checked repack
// and read back (with a stream synchronization: repacks run at load time) after it. Checked
// repacks hold g_check_mutex from the clear to the read, so that repacks from several host
// threads do not share one flag.
__device__ uint32_t scale_domain_flag;
std::mutex g_flag_mutex;
std::mutex g_check_mutex;
void* g_flag[64];

__global__ void clear_flag_kernel(uint32_t* p) { *p = 0u; }

int scale_flag_of_current_device(const char* op, uint32_t** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        set_error(op, "no usable current device");
        return PLM_ERR_HIP;
    }
    std::lock_guard<std::mutex> lock(g_flag_mutex);
    if (g_flag[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scale_domain_flag));
        if (e != hipSuccess || p == nullptr) {
            set_error(op, "hipGetSymbolAddress(scale_domain_flag) failed: %s", hipGetErrorString(e));
            return PLM_ERR_HIP;
        }
        g_flag[dev] = p;
    }
    *out = static_cast<uint32_t*>(g_flag[dev]);
    return PLM_OK;
}

// After a checked int4 scale repack was queued on `stream`: wait for it and reject the
// weights if a scale fell outside the kernels' domain.
int read_scale_flag(const char* op, uint32_t* flag, hipStream_t stream) {
    uint32_t host = 0;
    if (hipMemcpyAsync(&host, flag, sizeof(host), hipMemcpyDeviceToHost, stream) != hipSuccess ||
        hipStreamSynchronize(stream) != hipSuccess) {
        set_error(op, "reading the scale check failed: %s", hipGetErrorString(hipGetLastError()));
        return PLM_ERR_HIP;
    }
    PLM_CHECK_ARG(host == 0, op,
                  "int4 scales must be below 2^120 in magnitude after rounding to bf16 (the GEMM kernels form "
                  "(128 + q + 8) * scale in fp32)");
    return PLM_OK;
}

int launch_scale_repack(const char* op, const void* src, plm_dtype dt, int64_t n, int64_t k, int64_t block_n,
                        int64_t group_size, void* dst, hipStream_t stream, bool int4) {
    const layout_dims d = make_dims(n, k, block_n, group_size);
    const int64_t total = d.strips * d.groups * d.scale_cols;
    if (total == 0) return PLM_OK;
    // fp16 scales are below 65520 in magnitude: only fp32 and bf16 int4 scales are checked.
    const int check = !int4 ? 0 : dt == PLM_FP32 ? 1 : dt == PLM_BF16 ? 2 : 0;
    uint32_t* flag = nullptr;
    std::unique_lock<std::mutex> exclusive(g_check_mutex, std::defer_lock);
    if (check != 0) {
        exclusive.lock();
        if (int rc = scale_flag_of_current_device(op, &flag)) return rc;
        clear_flag_kernel<<<1, 1, 0, stream>>>(flag);
        PLM_HIP_LAUNCH_CHECK(op);
    }
    if (dt == PLM_FP32) {
        repack_scale_kernel<uint32_t><<<blocks_for(total), kThreads, 0, stream>>>(
            static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), n, k, block_n, group_size, d.groups,
            d.scale_cols, total, check, flag);
    } else {
        repack_scale_kernel<uint16_t><<<blocks_for(total), kThreads, 0, stream>>>(
            static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), n, k, block_n, group_size, d.groups,
            d.scale_cols, total, check, flag);
    }
    PLM_HIP_LAUNCH_CHECK(op);
    return check != 0 ? read_scale_flag(op, flag, stream) : PLM_OK;
}

}  // namespace
}  // namespace plm

using namespace plm;

extern "C" {
// Not part of the public ABI (include/pulsarlm_amd.h): re-reads the measurement knobs from the
// environment, so a test can select one path and then the other within one process. Not
// thread-safe against concurrent GEMM calls.
__attribute__((visibility("default"))) void plm_internal_reload_tuning() {
    std::lock_guard<std::mutex> lock(plm::g_tuning_mutex);
    plm::g_tuning = plm::parse_tuning();
    plm::g_tuning_parsed = true;
}
}  // extern "C"

extern "C" {

const char* plm_last_error(void) { return g_error.c_str(); }

const char* plm_version(void) { return "pulsarlm_amd 0.1 gfx950"; }

int64_t plm_weight_bytes(plm_format format, int64_t n, int64_t k) {
    if (n < 0 || k < 0 || (format != PLM_INT4 && format != PLM_FP8)) return -1;
    return ceil_div(n, kTileN) * ceil_div(k, kTileK) * tile_bytes(format);
}

int64_t plm_scale_bytes(int64_t n, int64_t k, int64_t block_n, int64_t group_size, plm_dtype scale_dtype) {
    if (n < 0 || k < 0 || block_n <= 0 || group_size <= 0 || group_size % 16 != 0) return -1;
    if (scale_dtype != PLM_BF16 && scale_dtype != PLM_FP16 && scale_dtype != PLM_FP32) return -1;
    const layout_dims d = make_dims(n, k, block_n, group_size);
    return d.strips * d.groups * d.scale_cols * dtype_size(scale_dtype);
}

int plm_repack_int4(const int32_t* weight_packed, const void* weight_scale, plm_dtype scale_dtype, int64_t n,
                    int64_t k, int64_t block_n, int64_t group_size, void* weight_out, void* scale_out,
                    void* stream) {
    const char* op = "repack_int4_marlin";
    clear_error();
    if (int rc = check_common(op, scale_dtype, n, k, block_n, group_size)) return rc;
    PLM_CHECK_ARG(k % 8 == 0, op, "K must be a multiple of 8");
    const int64_t total = ceil_div(n, kTileN) * ceil_div(k, kTileK) * 256;
    PLM_CHECK_ARG(total == 0 || (weight_packed && weight_out && weight_scale && scale_out), op, "null pointer");
    PLM_CHECK_ARG(aligned(weight_out, 16), op, "weight_out must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    if (total > 0) {
        repack_int4_kernel<<<blocks_for(total), kThreads, 0, s>>>(weight_packed, static_cast<uint32_t*>(weight_out),
                                                                  n, k, ceil_div(k, kTileK), total);
        PLM_HIP_LAUNCH_CHECK(op);
    }
    return launch_scale_repack(op, weight_scale, scale_dtype, n, k, block_n, group_size, scale_out, s, true);
}

int plm_repack_fp8(const uint8_t* weight, const void* weight_scale, plm_dtype scale_dtype, int64_t n, int64_t k,
                   int64_t block_n, int64_t group_size, void* weight_out, void* scale_out, void* stream) {
    const char* op = "repack_fp8_marlin";
    clear_error();
    if (int rc = check_common(op, scale_dtype, n, k, block_n, group_size)) return rc;
    const int64_t total = ceil_div(n, kTileN) * ceil_div(k, kTileK) * 512;
    PLM_CHECK_ARG(total == 0 || (weight && weight_out && weight_scale && scale_out), op, "null pointer");
    PLM_CHECK_ARG(aligned(weight_out, 16), op, "weight_out must be 16-byte aligned");
    hipStream_t s = as_stream(stream);
    if (total > 0) {
        repack_fp8_kernel<<<blocks_for(total), kThreads, 0, s>>>(weight, static_cast<uint32_t*>(weight_out), n, k,
                                                                 ceil_div(k, kTileK), total);
        PLM_HIP_LAUNCH_CHECK(op);
    }
    return launch_scale_repack(op, weight_scale, scale_dtype, n, k, block_n, group_size, scale_out, s, false);
}

int plm_convert_marlin(plm_format format, const int32_t* weight_marlin, const float* scale_marlin, int64_t n,
                       int64_t k, int64_t block_n, int64_t group_size, void* weight_out, void* scale_out,
                       void* stream) {
    const char* op = "convert_marlin";
    clear_error();
    if (int rc = check_common(op, PLM_FP32, n, k, block_n, group_size)) return rc;
    PLM_CHECK_ARG(format == PLM_INT4 || format == PLM_FP8, op, "unknown format");
    hipStream_t s = as_stream(stream);
    const int64_t ktiles = ceil_div(k, kTileK);
    const int64_t total = ceil_div(n, kTileN) * ktiles * (format == PLM_INT4 ? 256 : 512);
    PLM_CHECK_ARG(total == 0 || (weight_marlin && weight_out && scale_marlin && scale_out), op, "null pointer");
    if (total > 0) {
        if (format == PLM_INT4) {
            convert_marlin_int4_kernel<<<blocks_for(total), kThreads, 0, s>>>(
                reinterpret_cast<const uint32_t*>(weight_marlin), static_cast<uint32_t*>(weight_out), n, k, ktiles,
                total);
        } else {
            convert_marlin_fp8_kernel<<<blocks_for(total), kThreads, 0, s>>>(
                reinterpret_cast<const uint32_t*>(weight_marlin), static_cast<uint32_t*>(weight_out), n, k, ktiles,
                total);
        }
        PLM_HIP_LAUNCH_CHECK(op);
    }
    const layout_dims d = make_dims(n, k, block_n, group_size);
    const int64_t stotal = d.strips * d.groups * d.scale_cols;
    if (stotal > 0) {
        const int check = format == PLM_INT4 ? 1 : 0;
        uint32_t* flag = nullptr;
        std::unique_lock<std::mutex> exclusive(g_check_mutex, std::defer_lock);
        if (check != 0) {
            exclusive.lock();
            if (int rc = scale_flag_of_current_device(op, &flag)) return rc;
            clear_flag_kernel<<<1, 1, 0, s>>>(flag);
            PLM_HIP_LAUNCH_CHECK(op);
        }
        convert_marlin_scale_kernel<<<blocks_for(stotal), kThreads, 0, s>>>(
            scale_marlin, static_cast<float*>(scale_out), n, k, block_n, group_size, d.groups, d.scale_cols, stotal,
            check, flag);
        PLM_HIP_LAUNCH_CHECK(op);
        if (check != 0) return read_scale_flag(op, flag, s);
    }
    return PLM_OK;
}

int plm_dequant(plm_format format, const void* weight, const void* scale, plm_dtype scale_dtype, int64_t n, int64_t k,
                int64_t block_n, int64_t group_size, void* out, plm_dtype out_dtype, void* stream) {
    const char* op = "dequant";
    clear_error();
    if (int rc = check_common(op, scale_dtype, n, k, block_n, group_size)) return rc;
    PLM_CHECK_ARG(format == PLM_INT4 || format == PLM_FP8, op, "unknown format");
    PLM_CHECK_ARG(out_dtype == PLM_BF16 || out_dtype == PLM_FP16, op, "out dtype must be bf16 or fp16");
    const int64_t total = n * k;
    if (total == 0) return PLM_OK;
    PLM_CHECK_ARG(weight && scale && out, op, "null pointer");
    const layout_dims d = make_dims(n, k, block_n, group_size);
    hipStream_t s = as_stream(stream);
    auto w8 = static_cast<const uint8_t*>(weight);
    auto o = static_cast<uint16_t*>(out);
    const bool bf = out_dtype == PLM_BF16;
    if (format == PLM_INT4) {
        if (bf)
            dequant_kernel<PLM_INT4, true><<<blocks_for(total), kThreads, 0, s>>>(
                w8, scale, scale_dtype, n, k, d.ktiles, group_size, d.groups, d.scale_cols, o);
        else
            dequant_kernel<PLM_INT4, false><<<blocks_for(total), kThreads, 0, s>>>(
                w8, scale, scale_dtype, n, k, d.ktiles, group_size, d.groups, d.scale_cols, o);
    } else {
        if (bf)
            dequant_kernel<PLM_FP8, true><<<blocks_for(total), kThreads, 0, s>>>(
                w8, scale, scale_dtype, n, k, d.ktiles, group_size, d.groups, d.scale_cols, o);
        else
            dequant_kernel<PLM_FP8, false><<<blocks_for(total), kThreads, 0, s>>>(
                w8, scale, scale_dtype, n, k, d.ktiles, group_size, d.groups, d.scale_cols, o);
    }
    PLM_HIP_LAUNCH_CHECK(op);
    return PLM_OK;
}

}  // extern "C"
