/*
 * pulsarlm_amd: MI355X (gfx950) quantized-linear hot path, C ABI.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t passed
 * as void* (NULL = the null stream), enqueues its work on that stream without
 * synchronizing, and returns a plm_status. On failure the message (prefixed
 * with the operation name, e.g. "gemm_int4_marlin: ...") is available from
 * plm_last_error() on the calling thread. Inputs are never modified.
 *
 * Weight layout ("plm tile layout", opaque to callers): the N x K weight is cut
 * into 16-row x 128-column tiles, strip-major (all K tiles of rows 0..15, then
 * rows 16..31, ...). An int4 tile is 1 KiB: 64 lanes x 16 bytes. Lane
 * 16 g + 4 c + i holds in its 32-bit word t = (k % 128) / 32 the offset-binary
 * nibbles (q + 8) of rows 4 c + r (r = 0..3) at K = 32 t + 8 g + 4 h + i (h = 0, 1),
 * (r, h) in nibble 4 (r % 2) + 2 h + r / 2: four rows by two K values, the operand
 * of the matrix-core dequant (see plm_common.hpp). An fp8 tile is 2 KiB, lane
 * (n % 16) + 16 * ((k % 32) / 8) holding the 8 consecutive K bytes k % 8 of its row:
 * two such 1 KiB halves (t / 2), each lane holding 8 bytes per t. Padding rows
 * and columns hold q = 0. Scales are stored in their source dtype as
 * [N/16 strips][ceil(K_pad / group_size) groups][16 or 1], one per column, or
 * one per strip when block_n is a multiple of 16.
 *
 * Workspace: GEMMs that split K across workgroups need per-tile arrival
 * counters (the first 64 KiB of the workspace) and fp32 partial sums (after them).
 * plm_gemm_workspace_bytes() gives the size; the
 * counter region must be zero before the first call that uses a workspace, and
 * every call leaves it zero again, so one zeroed workspace can be reused by
 * calls that are ordered on one stream. Calls that may overlap need separate
 * workspaces.
 */
#ifndef PULSARLM_AMD_H
#define PULSARLM_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum plm_status {
    PLM_OK = 0,
    PLM_ERR_INVALID = 1,   /* bad argument: shape, dtype, size or alignment */
    PLM_ERR_HIP = 2,       /* a HIP runtime call or kernel launch failed */
    PLM_ERR_WORKSPACE = 3  /* workspace missing or smaller than required */
} plm_status;

typedef enum plm_dtype {
    PLM_BF16 = 0,
    PLM_FP16 = 1,
    PLM_FP32 = 2
} plm_dtype;

typedef enum plm_format {
    PLM_INT4 = 0, /* signed int4, symmetric, group-wise scales */
    PLM_FP8 = 1   /* OCP e4m3 (fn); codes 0x7f/0xff (NaN) unsupported */
} plm_format;

/* Message for the last failing call on this thread ("" if none). */
const char* plm_last_error(void);

/* Library version string. */
const char* plm_version(void);

/* Bytes of the repacked weight for an N x K matrix in `format`
 * (counterpart of marlin_words, pulsarlm-core/src/kernels/marlin.cu:391-393). */
int64_t plm_weight_bytes(plm_format format, int64_t n, int64_t k);

/* Bytes of the repacked scales; -1 if the arguments are invalid. */
int64_t plm_scale_bytes(int64_t n, int64_t k, int64_t block_n, int64_t group_size, plm_dtype scale_dtype);

/*
 * Repack int4 weights for the GEMMs.
 * Replaces repack_int4_marlin_cuda (pulsarlm-core/inc/pulsarlm/kernels/ops.hpp:306-311,
 * pulsarlm-core/src/kernels/marlin.cu:601-620).
 *   weight_packed  int32 [N, K/8], 8 signed nibbles per int32 along K, least significant first
 *   weight_scale   [ceil(N/block_n), K/group_size] in scale_dtype, row-major
 *   weight_out     plm_weight_bytes(PLM_INT4, N, K) bytes, 16-byte aligned
 *   scale_out      plm_scale_bytes(...) bytes
 * group_size must be a positive multiple of 16 dividing K; block_n > 0.
 */
int plm_repack_int4(const int32_t* weight_packed, const void* weight_scale, plm_dtype scale_dtype,
                    int64_t n, int64_t k, int64_t block_n, int64_t group_size,
                    void* weight_out, void* scale_out, void* stream);

/* Repack e4m3 weights [N, K] (bytes). Replaces repack_fp8_marlin_cuda (ops.hpp:313-314,
 * marlin.cu:622-629). */
int plm_repack_fp8(const uint8_t* weight, const void* weight_scale, plm_dtype scale_dtype,
                   int64_t n, int64_t k, int64_t block_n, int64_t group_size,
                   void* weight_out, void* scale_out, void* stream);

/*
 * Convert weights already in the reference's Marlin layout (the (weight_marlin,
 * scale_marlin) pair that repack_*_marlin_cuda returns: int32 words and fp32
 * [K/group_size, ceil(N/block_n)] scales, marlin.cu:395-445) into the plm
 * layout, so a checkpoint repacked for the reference can be loaded as is.
 * The scales come out as PLM_FP32.
 */
int plm_convert_marlin(plm_format format, const int32_t* weight_marlin, const float* scale_marlin,
                       int64_t n, int64_t k, int64_t block_n, int64_t group_size,
                       void* weight_out, void* scale_out, void* stream);

/* Dense dequantized weight [N, K] in out_dtype (PLM_BF16 or PLM_FP16) from the
 * plm layout: W = round(q * round(scale)), round = RNE to out_dtype, exactly
 * what the reference's kernels feed their MMAs (marlin.cu:123-151,180-194). */
int plm_dequant(plm_format format, const void* weight, const void* scale, plm_dtype scale_dtype,
                int64_t n, int64_t k, int64_t block_n, int64_t group_size,
                void* out, plm_dtype out_dtype, void* stream);

/* Workspace bytes plm_gemm may use for an [M, K] x [N, K]^T call (0 if none). */
int64_t plm_gemm_workspace_bytes(plm_format format, int64_t m, int64_t n, int64_t k);

/*
 * y [M, N] = x [M, K] @ dequant(W)^T, x and y in x_dtype (PLM_BF16 or PLM_FP16),
 * fp32 accumulation. Replaces gemm_int4_marlin_cuda / gemm_fp8_marlin_cuda
 * (ops.hpp:316-332, marlin.cu:538-597,631-651).
 * M <= 16 (and up to 32 rows where measured faster) runs the bandwidth-first decode kernels;
 * larger M the MFMA kernel.
 * M == 0 or N == 0 returns PLM_OK without touching y.
 */
int plm_gemm(plm_format format, const void* x, plm_dtype x_dtype,
             const void* weight, const void* scale, plm_dtype scale_dtype,
             int64_t m, int64_t n, int64_t k, int64_t block_n, int64_t group_size,
             void* y, void* workspace, size_t workspace_bytes, void* stream);

/*
 * plm_gemm without a workspace argument and without any allocation: for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). No counterpart in the reference. The split-K partial sums and
 * arrival counters live in a fixed device array of PLM_NOALLOC_SCRATCH_BYTES inside the
 * library, one per GPU, held until the process ends; the first call on a device takes its
 * address and clears its counters (a kernel on `stream`). Calls needing more scratch than
 * that (plm_gemm_workspace_bytes) fail with PLM_ERR_INVALID. Every call on one GPU shares
 * that GPU's array, so calls that may overlap on one GPU (different streams or threads)
 * race: use plm_gemm with separate workspaces for those. Same arguments and results as
 * plm_gemm otherwise.
 */
#define PLM_NOALLOC_SCRATCH_BYTES (32 * 1024 * 1024)
int plm_gemm_noalloc(plm_format format, const void* x, plm_dtype x_dtype,
                     const void* weight, const void* scale, plm_dtype scale_dtype,
                     int64_t m, int64_t n, int64_t k, int64_t block_n, int64_t group_size,
                     void* y, void* stream);

/*
 * Per-row dynamic e4m3 quantization of x [M, K] (bf16/fp16, K % 4 == 0):
 * x_scale[m] = max(amax(x[m, :]), 1e-12) / 448, codes[m, k] = e4m3_rne(x[m, k] / x_scale[m]).
 * codes is [M, K] bytes, x_scale fp32 [M]. The rule is the block quantizer of
 * pulsarlm-core/tests/model/test_qwen3_5.cpp:301-311 applied per row; the
 * reference has no activation quantizer on its GEMM path.
 */
int plm_quantize_rows_e4m3(const void* x, plm_dtype x_dtype, int64_t m, int64_t k,
                           uint8_t* codes, float* x_scale, void* stream);

/* Workspace bytes plm_gemm_w8a8 needs (quantized x, row scales, split-K). */
int64_t plm_gemm_w8a8_workspace_bytes(int64_t m, int64_t n, int64_t k);

/*
 * W8A8: x is quantized per row (token) to e4m3 on the fly (as plm_quantize_rows_e4m3),
 * and multiplied with e4m3 weights on the fp8 MFMA:
 * y[m, n] = x_scale[m] * sum_g s[n, g] * sum_{k in g} e4m3(xq[m, k]) * e4m3(w[n, k]).
 * group_size must be a multiple of 128. No counterpart in the reference (its fp8
 * path is W8A16, gemm_fp8_marlin_cuda); x and y bf16 or fp16. At M <= 4 (M <= 2 for
 * long K) the quantization runs inside the GEMM kernel (one launch, the same codes,
 * scales and result); otherwise it is a launch of its own into the workspace.
 */
int plm_gemm_w8a8(const void* x, plm_dtype x_dtype,
                  const void* weight, const void* scale, plm_dtype scale_dtype,
                  int64_t m, int64_t n, int64_t k, int64_t block_n, int64_t group_size,
                  void* y, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Grouped GEMM over experts: rows [offsets[e-1], offsets[e]) of x (offsets
 * int32 [n_experts], inclusive ends, as at::cumsum produces in
 * pulsarlm-core/src/engine/model/paged_forward.cpp:120-121) are multiplied by
 * expert e's weight. weight holds n_experts repacked [N, K] matrices back to
 * back (plm_weight_bytes each), scale likewise (plm_scale_bytes each).
 * Replaces one at::_grouped_mm(rows, W^T, offsets) call of routed_experts
 * (paged_forward.cpp:124-125) for int4 experts (PLM_INT4 only).
 * The offsets are expected to be non-decreasing with offsets[n_experts-1] == rows.
 * Others are clamped on the device: each expert's rows are [clamp(offsets[e-1]),
 * max(clamp(offsets[e]), clamp(offsets[e-1]))) with clamp to [0, rows], so no tile
 * reads or writes outside rows [0, rows); rows no expert covers are not written.
 */
int plm_grouped_gemm(plm_format format, const void* x, plm_dtype x_dtype,
                     const void* weight, const void* scale, plm_dtype scale_dtype,
                     const int32_t* offsets, int64_t n_experts, int64_t rows,
                     int64_t n, int64_t k, int64_t block_n, int64_t group_size,
                     void* y, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes plm_grouped_gemm needs for `rows` rows over n_experts experts. */
int64_t plm_grouped_gemm_workspace_bytes(int64_t rows, int64_t n_experts);

/* Workspace bytes plm_moe needs. */
int64_t plm_moe_workspace_bytes(int64_t tokens, int64_t top_k, int64_t n_experts,
                                int64_t hidden, int64_t intermediate);

/*
 * routed_experts (paged_forward.cpp:108-130) for int4 experts and SiLU:
 *   out [T, H] = sum_j top_weights[t, j] * down_e(silu(g) * u), (g | u) = gate_up_e(h[t]),
 * e = top_experts[t, j] (int32 [T, top_k]), top_weights fp32 [T, top_k].
 * Assignments whose expert id lies outside [0, n_experts) (e.g. -1 padding) are
 * dropped: they add nothing to their token's sum and are not counted in offsets.
 * (The reference's index_add_ would raise on them.)
 * gate_up holds n_experts repacked [2I, H] weights, down n_experts [H, I].
 * Sorting by expert, offsets, gather, both grouped GEMMs, the activation and the
 * weighted scatter-back all run on the device with no host synchronization.
 * offsets (int32 [n_experts], written) receives the inclusive-end row offsets of
 * the stable sort, as at::cumsum(counts) in the reference. Stable and deterministic:
 * the same inputs give the same bits.
 */
int plm_moe(const void* h, plm_dtype dtype, const int32_t* top_experts, const float* top_weights,
            int64_t tokens, int64_t top_k, int64_t n_experts, int64_t hidden, int64_t intermediate,
            const void* gate_up_weight, const void* gate_up_scale,
            const void* down_weight, const void* down_scale, plm_dtype scale_dtype, int64_t group_size,
            int32_t* offsets, void* out, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Router: for each token t, the softmax in fp32 of its logits row (rows row_stride
 * elements apart, dtype PLM_FP32, PLM_FP16 or PLM_BF16), its k most probable experts in
 * descending order (the lower expert first among equal probabilities) and their
 * probabilities divided by their sum: weights fp32 [tokens, k]; the experts as int64
 * [tokens, k] into `chosen` and/or as int32 into `chosen_i32` (what plm_moe takes),
 * either may be NULL. experts <= 4096, 1 <= k <= min(experts, 64).
 * Replaces route_top_k_cuda (pulsarlm-core/inc/pulsarlm/kernels/ops.hpp:37-40,
 * pulsarlm-core/src/kernels/moe_routing.cu:56-110,137-166).
 */
int plm_route_top_k(const void* logits, plm_dtype dtype, int64_t tokens, int64_t experts, int64_t row_stride,
                    int64_t k, float* weights, int64_t* chosen, int32_t* chosen_i32, void* stream);

/*
 * y [tokens, n] = round(round(silu(g)) * u) for contiguous x [tokens, 2n] = [g | u],
 * silu(g) = g / (1 + exp(-g)) in fp32, round = to dtype (PLM_FP32, PLM_FP16, PLM_BF16).
 * Replaces silu_mul_cuda (ops.hpp:42-43, moe_routing.cu:112-131,168-192).
 */
int plm_silu_mul(const void* x, plm_dtype dtype, int64_t tokens, int64_t n, void* y, void* stream);

/*
 * Non-repacked int4 GEMM: y [M, N] = x [M, K] @ W^T in x_dtype (PLM_BF16 or PLM_FP16),
 * W[n, k] = round(fp32(q[n, k] * scale[n, k / group_size])) with q the signed nibbles of
 * weight_packed int32 [N, K/8] (least significant first) and weight_scale fp32 [N, K/g],
 * read in place (no repack). num_splits = 0 picks the K split; >= 1 forces it (the extra
 * splits past the K tiles contribute zero). The split partials go to the workspace
 * (plm_gemm_int4_plain_workspace_bytes; no zeroing needed) and are summed in split order.
 * Replaces gemm_int4_cuda / gemm_int4_split_cuda (ops.hpp:272-297, int4_gemm.cu:153-478).
 */
int64_t plm_gemm_int4_plain_workspace_bytes(int64_t m, int64_t n, int64_t k, int64_t num_splits);
int plm_gemm_int4_plain(const void* x, plm_dtype x_dtype, const int32_t* weight_packed, const float* weight_scale,
                        int64_t m, int64_t n, int64_t k, int64_t group_size, int64_t num_splits, void* y,
                        void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PULSARLM_AMD_H */
