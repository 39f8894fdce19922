// C-ABI GEMM entry points: argument checks (mirroring gemm<fmt>,
// pulsarlm-core/src/kernels/marlin.cu:538-576) and dispatch between the decode
// kernels (M <= 16, the reference's small_m switch at marlin.cu:577, and up to 32 rows
// where measured faster) and the MFMA kernel.
#include <algorithm>
#include <cstdlib>
#include <mutex>

#include "plm_common.hpp"

namespace plm {
int launch_decode(const char* op, plm_format f, const void* x, bool bf16, const void* w, const void* scale,
                  plm_dtype scale_dtype, int64_t m, int64_t n, int64_t k, int64_t block_n, int64_t group_size,
                  void* y, void* workspace, size_t workspace_bytes, hipStream_t s, const uint8_t* xq,
                  const float* x_scale, bool quant_fused = false);
int launch_mfma(const char* op, plm_format f, const void* x, bool bf16, const void* w, const void* scale,
                plm_dtype scale_dtype, int64_t m, int64_t n, int64_t k, int64_t block_n, int64_t group_size, void* y,
                void* workspace, size_t workspace_bytes, hipStream_t s, const uint8_t* xq, const float* x_scale);
int launch_quantize_rows(const char* op, const void* x, bool bf16, int64_t m, int64_t k, uint8_t* out, float* sx,
                         bool permuted, hipStream_t s);
int64_t decode_workspace_bytes(plm_format f, int64_t m, int64_t n, int64_t k);
int64_t mfma_workspace_bytes(plm_format f, int64_t m, int64_t n, int64_t k, bool a8);

// Decode kernels or MFMA kernel. The decode kernels take up to 32 rows (one or two 16-row
// MFMA blocks; W8A8 one). Measured on MI355X at the Qwen3-8B shapes (both paths at every M
// from 1 to 64): decode is 1.6-2.9x faster up to 16 rows, and 18-35 % faster from 17 to 32
// rows except for the widest layer (N = 24576, four or more 16-column strips per CU),
// where it stops winning above 24 rows. Environment PLM_DECODE_MAX_M (0-32) replaces the
// rule by a plain threshold, for measuring one path against the other at the same M.
int64_t decode_env_max_m() { return knobs().decode_max_m; }
bool use_decode(int64_t m, int64_t n) {
    if (decode_env_max_m() >= 0) return m <= decode_env_max_m();
    if (m <= 16) return true;
    return m <= 32 && (m <= 24 || ceil_div(n, kTileN) < 4 * cu_count());
}
bool use_decode_w8a8(int64_t m) { return m <= 16 && (decode_env_max_m() < 0 || m <= decode_env_max_m()); }

// Environment PLM_W8A8_UNFUSED: always quantize x in its own launch (A/B measurements and
// the bit-exactness test of the fused quantizer).
bool fused_quant_off() { return knobs().w8a8_unfused; }

const char* gemm_op_name(plm_format f) { return f == PLM_INT4 ? "gemm_int4_marlin" : "gemm_fp8_marlin"; }

int check_gemm(const char* op, plm_format f, const void* x, plm_dtype x_dtype, const void* w, const void* scale,
               plm_dtype scale_dtype, int64_t m, int64_t n, int64_t k, int64_t block_n, int64_t group_size,
               const void* y) {
    PLM_CHECK_ARG(f == PLM_INT4 || f == PLM_FP8, op, "unknown weight format");
    PLM_CHECK_ARG(x_dtype == PLM_BF16 || x_dtype == PLM_FP16, op, "x must be fp16 or bf16");
    PLM_CHECK_ARG(scale_dtype == PLM_BF16 || scale_dtype == PLM_FP16 || scale_dtype == PLM_FP32, op,
                  "scale dtype must be bf16, fp16 or fp32");
    PLM_CHECK_ARG(m >= 0 && n >= 0 && k >= 0, op, "sizes must be non-negative");
    PLM_CHECK_ARG(block_n > 0, op, "block_n must be positive");
    PLM_CHECK_ARG(group_size > 0 && group_size % 16 == 0, op, "group_size must be a positive multiple of 16");
    PLM_CHECK_ARG(k % group_size == 0, op, "K must be a multiple of group_size");
    PLM_CHECK_ARG(n <= (int64_t{1} << 30) && k <= (int64_t{1} << 30) && m <= (int64_t{1} << 30), op,
                  "sizes must be below 2^30");
    if (m == 0 || n == 0) return PLM_OK;
    PLM_CHECK_ARG(x != nullptr && w != nullptr && scale != nullptr && y != nullptr, op, "null pointer");
    PLM_CHECK_ARG(aligned(x, 16), op, "x must be 16-byte aligned");
    PLM_CHECK_ARG(aligned(w, 16), op, "weight must be 16-byte aligned");
    PLM_CHECK_ARG(aligned(scale, 4), op, "scale must be 4-byte aligned");
    PLM_CHECK_ARG(aligned(y, 2), op, "y must be 2-byte aligned");
    return PLM_OK;
}

}  // namespace plm

using namespace plm;

extern "C" {

int64_t plm_gemm_workspace_bytes(plm_format format, int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0) return 0;
    return use_decode(m, n) ? decode_workspace_bytes(format, m, n, k) : mfma_workspace_bytes(format, m, n, k, false);
}

int plm_gemm(plm_format format, const void* x, plm_dtype x_dtype, const void* weight, const void* scale,
             plm_dtype scale_dtype, int64_t m, int64_t n, int64_t k, int64_t block_n, int64_t group_size, void* y,
             void* workspace, size_t workspace_bytes, void* stream) {
    const char* op = gemm_op_name(format);
    clear_error();
    if (int rc = check_gemm(op, format, x, x_dtype, weight, scale, scale_dtype, m, n, k, block_n, group_size, y))
        return rc;
    if (m == 0 || n == 0) return PLM_OK;
    const bool bf16 = x_dtype == PLM_BF16;
    if (use_decode(m, n))
        return launch_decode(op, format, x, bf16, weight, scale, scale_dtype, m, n, k, block_n, group_size, y,
                             workspace, workspace_bytes, as_stream(stream), nullptr, nullptr);
    return launch_mfma(op, format, x, bf16, weight, scale, scale_dtype, m, n, k, block_n, group_size, y, workspace,
                       workspace_bytes, as_stream(stream), nullptr, nullptr);
}

}  // extern "C"

namespace plm {
namespace {
// W8A8 workspace: [split-K region of the GEMM, at least the counters][e4m3 x, M x ktiles x 128][row scales].
struct w8a8_ws {
    int64_t gemm, xq, sx, total;
};
w8a8_ws w8a8_layout(int64_t m, int64_t n, int64_t k) {
    w8a8_ws w{};
    // The split-K counters always keep the front of the workspace, even when this call
    // does not split, so scratch written here never lands on them.
    const int64_t gemm = use_decode_w8a8(m) ? decode_workspace_bytes(PLM_FP8, m, n, k)
                                            : mfma_workspace_bytes(PLM_FP8, m, n, k, true);
    w.gemm = round_up(std::max<int64_t>(gemm, kCounterBytes), 256);
    w.xq = round_up(m * ceil_div(k, kTileK) * kTileK, 256);
    w.sx = round_up(m * 4, 256);
    w.total = w.gemm + w.xq + w.sx;
    return w;
}
}  // namespace
}  // namespace plm

extern "C" {

int plm_quantize_rows_e4m3(const void* x, plm_dtype x_dtype, int64_t m, int64_t k, uint8_t* codes, float* x_scale,
                           void* stream) {
    const char* op = "quantize_rows_e4m3";
    clear_error();
    PLM_CHECK_ARG(x_dtype == PLM_BF16 || x_dtype == PLM_FP16, op, "x must be fp16 or bf16");
    PLM_CHECK_ARG(m >= 0 && k >= 0 && k % 4 == 0 && k <= (int64_t{1} << 30), op, "K must be a multiple of 4");
    if (m == 0 || k == 0) return PLM_OK;
    PLM_CHECK_ARG(x && codes && x_scale, op, "null pointer");
    PLM_CHECK_ARG(aligned(codes, 4), op, "codes must be 4-byte aligned");
    return launch_quantize_rows(op, x, x_dtype == PLM_BF16, m, k, codes, x_scale, false, as_stream(stream));
}

int64_t plm_gemm_w8a8_workspace_bytes(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0) return 0;
    return w8a8_layout(m, n, k).total;
}

int plm_gemm_w8a8(const void* x, plm_dtype x_dtype, const void* weight, const void* scale, plm_dtype scale_dtype,
                  int64_t m, int64_t n, int64_t k, int64_t block_n, int64_t group_size, void* y, void* workspace,
                  size_t workspace_bytes, void* stream) {
    const char* op = "gemm_fp8_w8a8";
    clear_error();
    if (int rc = check_gemm(op, PLM_FP8, x, x_dtype, weight, scale, scale_dtype, m, n, k, block_n, group_size, y))
        return rc;
    PLM_CHECK_ARG(group_size % kTileK == 0, op, "group_size must be a multiple of 128 for the fp8 MFMA");
    if (m == 0 || n == 0) return PLM_OK;
    const w8a8_ws l = w8a8_layout(m, n, k);
    if (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < l.total) {
        set_error(op, "workspace of %lld bytes required, %zu given", static_cast<long long>(l.total), workspace_bytes);
        return PLM_ERR_WORKSPACE;
    }
    auto* base = static_cast<uint8_t*>(workspace);
    auto* xq = base + l.gemm;
    auto* sx = reinterpret_cast<float*>(base + l.gemm + l.xq);
    const bool bf16 = x_dtype == PLM_BF16;
    hipStream_t s = as_stream(stream);
    if (use_decode_w8a8(m) && !fused_quant_off()) {  // M <= 4 with K in LDS: one launch
        const int rc = launch_decode(op, PLM_FP8, x, bf16, weight, scale, scale_dtype, m, n, k, block_n, group_size, y,
                                     base, static_cast<size_t>(l.gemm), s, nullptr, nullptr, true);
        if (rc != kDecodeNotTaken) return rc;
    }
    if (int rc = launch_quantize_rows(op, x, bf16, m, k, xq, sx, true, s)) return rc;
    if (use_decode_w8a8(m))
        return launch_decode(op, PLM_FP8, x, bf16, weight, scale, scale_dtype, m, n, k, block_n, group_size, y, base,
                             static_cast<size_t>(l.gemm), s, xq, sx);
    return launch_mfma(op, PLM_FP8, x, bf16, weight, scale, scale_dtype, m, n, k, block_n, group_size, y, base,
                       static_cast<size_t>(l.gemm), s, xq, sx);
}

}  // extern "C"


// ---------------------------------------------------------------------------
// plm_gemm_noalloc: plm_gemm with its split-K workspace in a fixed device array.
//
// `scratch` lives in the code object's static device memory, one copy per GPU the library
// runs on, held until the process ends. In host code its name is only a stand-in: the
// device address comes from hipGetSymbolAddress, taken once per device with that device
// current, and is what the kernels receive. The split-K kernels need the counter region
// (its first kCounterBytes) zero on entry and leave it zero on exit. The loader zero-fills
// the array (it has no initializer), and set-up also clears the counter region with a fill
// kernel on the caller's stream (no hipMemsetAsync, so a caller may capture the call). When
// that first call is being captured, the fill kernel becomes a node of the caller's graph
// and re-clears the counters on every replay, which is harmless; the symbol lookup runs in
// relaxed capture mode so it cannot invalidate the capture. Every call on a GPU shares that
// GPU's array: calls that overlap on one GPU race.
// ---------------------------------------------------------------------------
namespace plm {
namespace {
constexpr int64_t kScratchBytes = PLM_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes >= kCounterBytes && kScratchBytes % 256 == 0, "scratch size");
__device__ __attribute__((aligned(256))) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices];  // device address of `scratch` per device, once set up

__global__ void __launch_bounds__(256) zero_words_kernel(uint32_t* __restrict__ p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0u;
}

int scratch_of_current_device(const char* op, hipStream_t s, void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error(op, "no usable current device for the fixed scratch");
        return PLM_ERR_HIP;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch[dev] == nullptr) {
        void* p = nullptr;
        hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
        (void)hipThreadExchangeStreamCaptureMode(&mode);
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        (void)hipThreadExchangeStreamCaptureMode(&mode);
        if (e != hipSuccess || p == nullptr) {
            set_error(op, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
            return PLM_ERR_HIP;
        }
        constexpr int words = static_cast<int>(kCounterBytes / 4);
        zero_words_kernel<<<(words + 255) / 256, 256, 0, s>>>(static_cast<uint32_t*>(p), words);
        PLM_HIP_LAUNCH_CHECK(op);
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return PLM_OK;
}
}  // namespace
}  // namespace plm

extern "C" {

int plm_gemm_noalloc(plm_format format, const void* x, plm_dtype x_dtype, const void* weight, const void* scale,
                     plm_dtype scale_dtype, int64_t m, int64_t n, int64_t k, int64_t block_n, int64_t group_size,
                     void* y, void* stream) {
    const char* op = gemm_op_name(format);
    clear_error();
    if (int rc = check_gemm(op, format, x, x_dtype, weight, scale, scale_dtype, m, n, k, block_n, group_size, y))
        return rc;
    if (m == 0 || n == 0) return PLM_OK;
    const int64_t need = plm_gemm_workspace_bytes(format, m, n, k);
    PLM_CHECK_ARG(need <= kScratchBytes, op,
                  "this call needs %lld bytes of split-K scratch, above the fixed %lld of plm_gemm_noalloc "
                  "(use plm_gemm with a workspace)",
                  static_cast<long long>(need), static_cast<long long>(kScratchBytes));
    hipStream_t s = as_stream(stream);
    void* ws = nullptr;
    if (int rc = scratch_of_current_device(op, s, &ws)) return rc;
    const bool bf16 = x_dtype == PLM_BF16;
    if (use_decode(m, n))
        return launch_decode(op, format, x, bf16, weight, scale, scale_dtype, m, n, k, block_n, group_size, y, ws,
                             static_cast<size_t>(kScratchBytes), s, nullptr, nullptr);
    return launch_mfma(op, format, x, bf16, weight, scale, scale_dtype, m, n, k, block_n, group_size, y, ws,
                       static_cast<size_t>(kScratchBytes), s, nullptr, nullptr);
}

}  // extern "C"
