// MFMA dequant-GEMM for M > 16 (prefill), its W8A8 form and its grouped (MoE) form:
// y[M, N] = x[M, K] @ dequant(W)^T.
//
// Counterpart of the reference's marlin_kernel at tile_m = 64 (pulsarlm-core/src/kernels/
// marlin.cu:251-389; dispatch :577-596) with its split-K combine
// (pulsarlm-core/inc/pulsarlm/kernels/dequant_gemm_common.cuh:99-133), and, in grouped
// mode, of one at::_grouped_mm of routed_experts (pulsarlm-core/src/engine/model/
// paged_forward.cpp:124-125).
//
// gfx950 design:
// * Workgroup tile (WM*MT*16) x (WN*NS*16) over 128-wide K steps; WM x WN wavefronts,
//   each owning MT x NS tiles of v_mfma_f32_16x16x32 (bf16/fp16) -- 128 x 64 per
//   wavefront in the large configuration (256 x 128 per workgroup, one wavefront per
//   SIMD with the full 512 registers), so each dequantized weight feeds 8 MFMAs and the
//   dequant VALU work is about half the MFMA time, interleaved with it. The int4 256 x 256
//   tile for plain calls uses 8 wavefronts of 256 x 32 each, so every strip is dequantized
//   by one wavefront only (a 2 x 4 wavefront grid would dequantize each strip twice).
// * The x tile and the packed weight tiles (1 KiB int4 / 2 KiB fp8 per 16-column strip,
//   copied verbatim from the plm layout) go from HBM straight into LDS with buffer loads to
//   LDS (no register staging), double-buffered: the next K step's loads land in one stage
//   while the current step's MFMAs read the other, with one barrier per K step. x rows are
//   XOR-swizzled in LDS so that fragment reads are free of bank conflicts; rows past M and
//   columns past K read as zeros through the buffer range instead of branches.
// * Weights are dequantized in registers to round(q * round(s)), bit-identical to the
//   reference's fragment values (shared dq_int4 / dq_fp8).
// * A8 (W8A8): x is e4m3 (quantized per row beforehand) and every 128-wide K tile is one
//   v_mfma_scale_f32_16x16x128_f8f6f4 per output tile on the raw weight bytes; the tile's
//   partial is scaled by the weight block scale and, at the end, by the row scale.
// * Grouped: each work tile is (expert, block of that expert's rows); rows may be gathered
//   through a row index (the tokens routed to the expert) and the expert's weights and
//   scales are found at a fixed stride.
// * Split-K across workgroups when the output has too few tiles to fill the GPU, reduced
//   deterministically by the last workgroup to arrive.
// * Grouped gate_up of the MoE block may fuse the activation: the workgroup's local strips
//   2p and 2p + 1 are the gate and up strips of one 16-column slice, so every wavefront
//   holds both halves of its outputs and the epilogue writes act = round(round(silu(g)) *
//   u) (the unfused silu_mul's expression) instead of the [rows, 2I] gate_up product.
#include <algorithm>
#include <type_traits>

#include "plm_common.hpp"

namespace plm {

struct mfma_args {
    const uint16_t* x;
    const uint8_t* w;
    const void* scale;
    uint16_t* y;
    float* partial;
    uint32_t* counters;
    int scale_dtype, scale_cols;
    int m, n, k;
    int ktiles, strips, groups, group_size;
    int splits, tiles_per_split;
    int m_blocks, n_blocks;
    int tile_base;  // plain calls: this launch's work tiles start at tile_base
    // A8
    const uint8_t* xq;      // e4m3 [M][ktiles][128], lane-permuted within each tile
    const float* x_scale;   // [M]
    // Grouped
    const int32_t* tiles;      // [max_tiles][3]: expert, first row, rows (rows == 0: idle)
    const int32_t* tile_count;  // the number of real tiles (a prefix of `tiles`)
    const int32_t* row_index;  // gather: A row r is x[row_index[r]] (null: x[r])
    int64_t w_expert_bytes;
    int64_t s_expert_bytes;
    // Grouped gate_up with the activation fused (0: off): the weight is [gate; up] with
    // swiglu_strips 16-column strips each; a workgroup takes gate strip p and up strip
    // swiglu_strips + p side by side and writes round(round(silu(g)) * u) into y [rows, 16 *
    // swiglu_strips] instead of the [rows, 2I] product.
    int swiglu_strips;
};

namespace {

template <bool A8> struct a_traits {
    static constexpr int row_bytes = A8 ? kTileK : kTileK * 2;  // one A row of one K tile
    static constexpr int slots = row_bytes / 16;                 // its 16-byte slots
};

// VO: the 16-byte epilogue (see its comment) is compiled in; the host selects it per launch.
template <plm_format F, bool BF16, bool UNIFORM, bool WIDE, bool A8, bool GROUPED, int WM, int WN, int MT, int NS,
          bool VO = false, bool PERSIST = false>
__global__ void __launch_bounds__(WM * WN * 64) mfma_kernel(mfma_args a) {
    constexpr int NW = WM * WN;  // wavefronts
    constexpr int NT = NW * 64;
    constexpr int TB = fmt_traits<F>::tile_bytes;
    constexpr int BM = WM * MT * 16;
    constexpr int BS = WN * NS;  // strips per workgroup
    constexpr int ARB = a_traits<A8>::row_bytes;
    constexpr int SLOTS = a_traits<A8>::slots;
    constexpr int RPC = 1024 / ARB;  // A rows per 1 KiB chunk
    constexpr int A_STAGE = BM * ARB;
    // fp8 W8A16 with one row of wavefronts: no two wavefronts share a weight strip, so each
    // loads its own strips' tiles for the next K step into registers and LDS holds only x
    // (the 2 KiB fp8 tiles of 16 strips would not fit beside two 64 KiB x stages). int4's
    // 1 KiB tiles fit; loading them the same way measured 8 % slower at M = 4096.
    constexpr bool BREG = F == PLM_FP8 && !A8 && !GROUPED && WM == 1;
    constexpr int B_STAGE = BREG ? 0 : BS * TB;
    constexpr int STAGE = A_STAGE + B_STAGE;
    constexpr int A_CHUNKS = A_STAGE / 1024, B_CHUNKS = B_STAGE / 1024;
    constexpr int A_PW = (A_CHUNKS + NW - 1) / NW;  // 1 KiB chunks each wavefront loads per K step
    constexpr int B_PW = (B_CHUNKS + NW - 1) / NW;
    static_assert(A_STAGE % 1024 == 0 && B_STAGE % 1024 == 0, "stages are whole 1 KiB chunks");
    constexpr int ST = UNIFORM ? 1 : 4;  // scale values per strip per K step
    constexpr int ES = WIDE ? 4 : 2;     // scale element bytes
    // Software-pipelined x fragments (see the K loop), for the one-row tall shapes.
    constexpr bool PIPE_A = UNIFORM && !A8 && WM == 1 && MT >= 8;
    // Fragments kept a slice ahead: all MT, or 12 for fp8, whose weight tiles already hold
    // two K steps of registers (16 would spill).
    // PERSIST keeps 8 fewer: the item loop needs the registers (the tall tile spills otherwise).
    constexpr int PD = F == PLM_FP8 ? MT - 4 : (PERSIST ? MT - 8 : MT);

    // Two stages of [A tile | weight tiles]. Stage s holds K step kt_begin + s (mod 2); the
    // loads of step kt + 1 go straight from HBM into the other stage while step kt computes.
    // The split-K arrival flag reuses the first word once the K loop is over (arrive_last
    // synchronizes the workgroup before writing it).
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * STAGE];
    uint32_t& last_flag = *reinterpret_cast<uint32_t*>(lds);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = uniform(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int col16 = lane & 15, kq = lane >> 4;
    const int split = blockIdx.y;
    const bool swiglu = GROUPED && a.swiglu_strips > 0;
    const int kt_begin = split * a.tiles_per_split;
    const int kt_end = min(kt_begin + a.tiles_per_split, a.ktiles);
    const int a_stride = A8 ? a.ktiles * kTileK : a.k * 2;
    const int strip_bytes = a.ktiles * TB;
    const bool bf16_scale = a.scale_dtype == PLM_BF16;
    const int s_row = a.groups * a.scale_cols * ES;  // scale bytes per strip
    const int s_lane = a.scale_cols == 1 ? 0 : col16 * ES;
    const int lrow = lane / SLOTS, lslot = lane % SLOTS;

    // Work items: plain calls take work tile blockIdx.x + tile_base (row block fastest);
    // grouped calls take (expert tile, column block) items. Workgroups are dealt to the 8
    // XCDs round-robin by id, so a grouped call gives out its real items in 8 contiguous runs,
    // one per XCD: the column blocks of a row tile (the same x rows) and the consecutive
    // tiles of an expert (the same weights) run on one XCD and share its L2; ids past the
    // real items exit. PERSIST (grouped only; an A/B option, measured slower than one item
    // per workgroup): the grid holds about one workgroup per slot the CUs keep resident, each
    // workgroup walks its XCD's run gridDim.x / 8 items apart and loads the next item's first
    // K step into the free LDS stage during the current item's epilogue.
    static_assert(!PERSIST || (GROUPED && !A8), "persistent launches are grouped ones");
    int items = 0, per_xcd = 0;
    if constexpr (GROUPED) {
        items = uniform(*a.tile_count) * a.n_blocks;
        per_xcd = (items + 7) >> 3;
    }
    auto item_at = [&](int pos) -> int {  // this workgroup's pos-th item, -1 past its last
        if constexpr (GROUPED) {
            const int idx = (blockIdx.x >> 3) + pos * (gridDim.x >> 3);
            if (idx >= per_xcd) return -1;
            const int it = (blockIdx.x & 7) * per_xcd + idx;
            return it < items ? it : -1;
        } else {
            return blockIdx.x + a.tile_base;
        }
    };

    // Everything that depends on the item: output tile, and the buffers and per-lane offsets
    // of its A rows, weight strips and scales.
    struct item_ctx {
        int nb, row0, rows;
        __amdgpu_buffer_rsrc_t a_rsrc, b_rsrc, s_rsrc;
        int a_gather[GROUPED ? A_PW : 1];  // grouped: the gathered rows' offsets
        int b_off[B_PW > 0 ? B_PW : 1];
        int s_strip[NS];  // byte offset of strip j's scales in s_rsrc
    };
    // SwiGLU (grouped): local strip s is gate strip (s even) or up strip (s odd) of slice
    // nb * BS / 2 + s / 2; otherwise strip strip0 + s.
    auto wstrip = [&](int nb, int s_local) -> int {
        if (swiglu) {
            const int slice = nb * (BS / 2) + (s_local >> 1);
            return slice < a.swiglu_strips ? slice + ((s_local & 1) ? a.swiglu_strips : 0) : -1;
        }
        return nb * BS + s_local < a.strips ? nb * BS + s_local : -1;
    };
    auto locate = [&](int item, item_ctx& c) -> bool {  // false: an idle grouped tile
        int expert = 0;
        if constexpr (GROUPED) {
            const int tile = item / a.n_blocks;
            c.nb = item % a.n_blocks;
            expert = a.tiles[3 * tile];
            c.row0 = a.tiles[3 * tile + 1];
            c.rows = a.tiles[3 * tile + 2];
            if (c.rows <= 0) return false;  // uniform across the workgroup
        } else {
            const int mb = item % a.m_blocks;
            c.nb = item / a.m_blocks;
            c.row0 = mb * BM;
            c.rows = min(BM, a.m - c.row0);
        }
        const int strip0 = c.nb * BS;
        // PERSIST: lane-derived offsets come from an opaque copy of the lane id, so that the
        // compiler recomputes them per item instead of hoisting them out of the item loop and
        // keeping them live across the K loop (the tall tile has no registers to spare).
        int llane = lane;
        if constexpr (PERSIST) asm volatile("" : "+v"(llane));
        const int lrow_l = llane / SLOTS;
        const uint8_t* wbase = a.w + (GROUPED ? expert * a.w_expert_bytes : 0);
        const uint8_t* sbase = static_cast<const uint8_t*>(a.scale) + (GROUPED ? expert * a.s_expert_bytes : 0);
        // A source: row-major rows of ARB bytes per K tile. Plain calls address rows from row0
        // and bound the buffer at `rows` rows; grouped calls gather rows through row_index
        // (the host checks every offset stays below kOOB) and keep the offsets in registers.
        if constexpr (GROUPED) {
            c.a_rsrc = make_rsrc(a.x, static_cast<uint32_t>(kOOB));
#pragma unroll
            for (int i = 0; i < A_PW; ++i) {
                const int r = (wave * A_PW + i) * RPC + lrow_l;
                int src = -1;
                if (r < c.rows) src = a.row_index != nullptr ? a.row_index[c.row0 + r] : c.row0 + r;
                c.a_gather[i] = src < 0 ? kOOB : src * a_stride;
            }
        } else {
            const uint8_t* base = A8 ? a.xq : reinterpret_cast<const uint8_t*>(a.x);
            c.a_rsrc = make_rsrc(base + static_cast<int64_t>(c.row0) * a_stride, static_cast<uint32_t>(c.rows * a_stride));
        }
        // Weights: this workgroup's strips are contiguous, ktiles * TB bytes each (with SwiGLU,
        // two runs of them, addressed from the expert's first strip).
        c.b_rsrc = swiglu ? make_rsrc(wbase, static_cast<uint32_t>(a.strips * strip_bytes))
                          : make_rsrc(wbase + static_cast<int64_t>(strip0) * strip_bytes,
                                      static_cast<uint32_t>(min(BS, a.strips - strip0) * strip_bytes));
#pragma unroll
        for (int i = 0; i < B_PW; ++i) {
            const int ch = wave * B_PW + i;
            const int sl = ch / (TB / 1024), in_strip = (ch % (TB / 1024)) * 1024 + llane * 16;
            if (swiglu) {
                const int ws = wstrip(c.nb, sl);
                c.b_off[i] = ws >= 0 ? ws * strip_bytes + in_strip : kOOB;
            } else {
                c.b_off[i] = sl * strip_bytes + in_strip;
            }
        }
        // Scales of this workgroup's strips ([strip][group][scale_cols], ES bytes each); strips
        // past N read as zero.
        c.s_rsrc = swiglu ? make_rsrc(sbase, static_cast<uint32_t>(a.strips * s_row))
                          : make_rsrc(sbase + static_cast<int64_t>(strip0) * s_row,
                                      static_cast<uint32_t>(min(BS, a.strips - strip0) * s_row));
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            if (swiglu) {
                const int ws = wstrip(c.nb, wn * NS + j);
                c.s_strip[j] = ws >= 0 ? ws * s_row : kOOB;
            } else {
                c.s_strip[j] = (wn * NS + j) * s_row;
            }
        }
        return true;
    };

    // Chunk c of the A tile is rows c*RPC .. c*RPC+RPC-1; lane L of its load writes slot L % SLOTS
    // of row c*RPC + L / SLOTS, which holds the row's 16-byte column (slot ^ row % SLOTS): the XOR
    // swizzle puts the 16 rows of one MFMA fragment read in 16 different bank groups.
    // Plain calls recompute the offsets per load (rows past `rows` fall outside the buffer).
    auto a_offset = [&](const item_ctx& c, int i, int kt) -> int {
        const int r = (wave * A_PW + i) * RPC + lrow;
        const int col = lslot ^ (r % SLOTS);
        const int row_off = GROUPED ? c.a_gather[GROUPED ? i : 0] : r * a_stride;
        if constexpr (!UNIFORM) {
            if (kt * kTileK + col * 8 >= a.k) return kOOB;  // K tail (bf16 x only)
        }
        return row_off + col * 16;
    };
    auto load_breg = [&](const item_ctx& c, u32x4_t (&dst)[NS][TB / 1024], int kt) {
#pragma unroll
        for (int j = 0; j < NS; ++j)
#pragma unroll
            for (int h = 0; h < TB / 1024; ++h)
                dst[j][h] = buffer_load16(c.b_rsrc, (wn * NS + j) * strip_bytes + h * 1024 + lane * 16, kt * TB);
    };
    auto issue = [&](const item_ctx& c, int kt, int stage) {
        uint8_t* sa = lds + stage * STAGE;
#pragma unroll
        for (int i = 0; i < A_PW; ++i)
            if (A_CHUNKS % NW == 0 || wave * A_PW + i < A_CHUNKS)  // wave-uniform
                buffer_load_lds16(c.a_rsrc, sa + (wave * A_PW + i) * 1024, a_offset(c, i, kt), kt * ARB);
#pragma unroll
        for (int i = 0; i < B_PW; ++i)
            if (B_CHUNKS % NW == 0 || wave * B_PW + i < B_CHUNKS)  // wave-uniform
                buffer_load_lds16(c.b_rsrc, sa + A_STAGE + (wave * B_PW + i) * 1024, c.b_off[i], kt * TB);
    };
    // Scales are loaded as raw bits one K step ahead and converted when used, so that no wait
    // on them stalls the tile loads in flight.
    auto scale_bits = [&](const item_ctx& c, int j, int kt, int t) -> uint32_t {
        int voff = s_lane + c.s_strip[j], soff = 0;
        if constexpr (UNIFORM) soff = uniform(kt * kTileK / a.group_size) * a.scale_cols * ES;
        else voff += (kt * kTileK + 32 * t + 8 * kq) / a.group_size * a.scale_cols * ES;
        if constexpr (WIDE) return buffer_load_u32(c.s_rsrc, voff, soff);
        else return buffer_load_u16(c.s_rsrc, voff, soff);
    };

    // Epilogue: lane holds column col16 of strip (strip0 + wn*NS + j), rows 4*kq + r of m tile i.
    auto epilogue = [&](const item_ctx& c, f32x4_t (&acc)[MT][NS], int last_stage) {
        const int strip0 = c.nb * BS;
        int ekq = kq, ecol = col16, elane = lane;
        if constexpr (PERSIST) asm volatile("" : "+v"(ekq), "+v"(ecol), "+v"(elane));
        if constexpr (GROUPED && NS % 2 == 0) {
            if (swiglu) {  // gate strip j, up strip j + 1 of slice nb * BS / 2 + (wn * NS + j) / 2
                const int inter = a.swiglu_strips * kTileN;
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int j = 0; j < NS; j += 2) {
                        const int col = (c.nb * (BS / 2) + (wn * NS + j) / 2) * kTileN + ecol;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int lr = wm * MT * 16 + i * 16 + 4 * ekq + r;
                            if (lr < c.rows && col < inter)
                                a.y[static_cast<int64_t>(c.row0 + lr) * inter + col] = static_cast<uint16_t>(
                                    to_bits16<BF16>(silu_times<BF16>(round_to<BF16>(acc[i][j][r]),
                                                                     round_to<BF16>(acc[i][j + 1][r]))));
                        }
                    }
                return;
            }
        }
        // With 16-byte aligned output rows, each m tile goes through the wavefront's own LDS area
        // (16 rows of 16 * NS columns; the row pitch is padded by 16 bytes so the four row groups
        // of one write land in different banks) and leaves as one 16-byte store per 8 columns of
        // a row, instead of a 2-byte store per element. Separate instantiations (VO) for the
        // launches that take it: compiled into the split-K kernels too, it changed their register
        // allocation and made down at M = 1024 10 % slower. PERSIST stages in the stage the last
        // K step read (the other one holds the next item's first loads).
        if (VO && a.splits == 1 && (a.n & 7) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0) {
            constexpr int EROW = 32 * NS + 16;
            static_assert(!VO || 1024 + NW * 16 * EROW <= (PERSIST ? STAGE : 2 * STAGE), "epilogue staging fits");
            __syncthreads();  // every wavefront is past the K loop's last reads of the stages
            // Past the split-K arrival flag.
            uint8_t* ew = lds + (PERSIST ? last_stage * STAGE : 0) + 1024 + wave * 16 * EROW;
            const int col0 = (strip0 + wn * NS) * kTileN;
#pragma unroll
            for (int i = 0; i < MT; ++i) {
#pragma unroll
                for (int j = 0; j < NS; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        *reinterpret_cast<uint16_t*>(ew + (4 * ekq + r) * EROW + (16 * j + ecol) * 2) =
                            static_cast<uint16_t>(to_bits16<BF16>(acc[i][j][r]));
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int c0 = 0; c0 < 32 * NS; c0 += 64) {  // 16 rows x 2 * NS chunks of 8 columns
                    const int ch16 = c0 + elane;
                    if (ch16 < 32 * NS) {
                        const int row = ch16 / (2 * NS), ch = ch16 % (2 * NS);
                        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ew + row * EROW + ch * 16);
                        const int lr = wm * MT * 16 + i * 16 + row;
                        const int col = col0 + ch * 8;
                        if (lr < c.rows && col < a.n)
                            *reinterpret_cast<u32x4_t*>(a.y + static_cast<int64_t>(c.row0 + lr) * a.n + col) = v;
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < NS; ++j) {
                const int col = (strip0 + wn * NS + j) * kTileN + ecol;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int lr = wm * MT * 16 + i * 16 + 4 * ekq + r;
                    if (lr < c.rows && col < a.n)
                        a.y[static_cast<int64_t>(c.row0 + lr) * a.n + col] =
                            static_cast<uint16_t>(to_bits16<BF16>(acc[i][j][r]));
                }
            }
    };

    int pos = 0;
    int item = item_at(0);
    if (item < 0) return;
    item_ctx cur;
    while (!locate(item, cur)) {
        if (!PERSIST) return;
        item = item_at(++pos);
        if (item < 0) return;
    }
    int stage0 = 0;      // the stage of this item's first K step
    bool loaded = false;  // its first K step is already in flight (PERSIST)
    for (;;) {
        f32x4_t acc[MT][NS];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < NS; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

        uint32_t sc[NS][ST];
        u32x4_t wreg[NS][TB / 1024], wnext[NS][TB / 1024];  // BREG: this and the next step's tiles
        if (kt_begin < kt_end) {
#pragma unroll
            for (int j = 0; j < NS; ++j)
#pragma unroll
                for (int t = 0; t < ST; ++t) sc[j][t] = scale_bits(cur, j, kt_begin, t);
            if (!loaded) issue(cur, kt_begin, stage0);
            if constexpr (BREG) load_breg(cur, wreg, kt_begin);
        }

        for (int kt = kt_begin; kt < kt_end; ++kt) {
            const int stage = stage0 ^ ((kt - kt_begin) & 1);
            // This step's tiles have landed (they are the only loads in flight) and every
            // wavefront is done with the other stage, which the next loads overwrite.
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            uint32_t scn[NS][ST];
            const bool more = kt + 1 < kt_end;
            if (more) {
#pragma unroll
                for (int j = 0; j < NS; ++j)
#pragma unroll
                    for (int t = 0; t < ST; ++t) scn[j][t] = scale_bits(cur, j, kt + 1, t);
                issue(cur, kt + 1, stage ^ 1);
                if constexpr (BREG) load_breg(cur, wnext, kt + 1);
            }

            const uint8_t* sa = lds + stage * STAGE;
            const uint8_t* sb = sa + A_STAGE;
            u32x4_t wv[NS][TB / 1024];
#pragma unroll
            for (int j = 0; j < NS; ++j)
#pragma unroll
                for (int h = 0; h < TB / 1024; ++h)
                    wv[j][h] = BREG ? wreg[j][h]
                                    : *reinterpret_cast<const u32x4_t*>(sb + (wn * NS + j) * TB + h * 1024 + lane * 16);

            if constexpr (A8) {
#pragma unroll
                for (int i = 0; i < MT; ++i) {
                    const uint8_t* ra = sa + (wm * MT * 16 + i * 16 + col16) * ARB;
                    const u32x4_t a0 = *reinterpret_cast<const u32x4_t*>(ra + (((2 * kq) ^ (col16 & 7)) * 16));
                    const u32x4_t a1 = *reinterpret_cast<const u32x4_t*>(ra + (((2 * kq + 1) ^ (col16 & 7)) * 16));
                    const i32x8_t av = __builtin_bit_cast(i32x8_t, u32x8_cat(a0, a1));
#pragma unroll
                    for (int j = 0; j < NS; ++j) {
                        const i32x8_t bv = __builtin_bit_cast(i32x8_t, u32x8_cat(wv[j][0], wv[j][TB / 1024 - 1]));
                        const f32x4_t part = mfma16x16x128_fp8(av, bv, f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                        for (int r = 0; r < 4; ++r) acc[i][j][r] = __builtin_fmaf(scale_from_bits<WIDE>(sc[j][0], bf16_scale), part[r], acc[i][j][r]);
                    }
                }
            } else if constexpr (PIPE_A) {
                // The MT x fragments of a K slice are held in registers and each is re-read for
                // the next slice right after its MFMAs, so a fragment read has a whole slice of
                // MFMAs (MT * NS) to land instead of the next two.
                auto frag = [&](int i, int t) {
                    const uint8_t* ra = sa + (wm * MT * 16 + i * 16 + col16) * ARB;
                    return *reinterpret_cast<const u32x4_t*>(ra + (((4 * t + kq) ^ col16) * 16));
                };
                u32x4_t af[PD];
#pragma unroll
                for (int i = 0; i < PD; ++i) af[i] = frag(i, 0);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    u32x4_t b[NS];
#pragma unroll
                    for (int j = 0; j < NS; ++j) {
                        const float raw = scale_from_bits<WIDE>(sc[j][UNIFORM ? 0 : t], bf16_scale);
                        if constexpr (F == PLM_INT4) {
                            b[j] = dq_int4<BF16>(wv[j][0][t], make_int4_scale<BF16>(raw));
                        } else {
                            b[j] = dq_fp8<BF16>(wv[j][t >> 1][(t & 1) * 2], wv[j][t >> 1][(t & 1) * 2 + 1],
                                                round_to<BF16>(raw));
                        }
                    }
#pragma unroll
                    for (int i = 0; i < PD; ++i) {
#pragma unroll
                        for (int j = 0; j < NS; ++j) acc[i][j] = mfma16x16x32<BF16>(af[i], b[j], acc[i][j]);
                        if (t < 3) af[i] = frag(i, t + 1);
                        __builtin_amdgcn_sched_barrier(0);  // keep the read here, a slice ahead
                    }
#pragma unroll
                    for (int i = PD; i < MT; ++i) {
                        const u32x4_t a1 = frag(i, t);
#pragma unroll
                        for (int j = 0; j < NS; ++j) acc[i][j] = mfma16x16x32<BF16>(a1, b[j], acc[i][j]);
                    }
                }
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    // Dequantize this 32-wide K slice of every strip once, then stream the x
                    // fragments past it: each weight fragment feeds MT MFMAs.
                    u32x4_t b[NS];
#pragma unroll
                    for (int j = 0; j < NS; ++j) {
                        const float raw = scale_from_bits<WIDE>(sc[j][UNIFORM ? 0 : t], bf16_scale);
                        if constexpr (F == PLM_INT4) {
                            b[j] = dq_int4<BF16>(wv[j][0][t], make_int4_scale<BF16>(raw));
                        } else {
                            b[j] = dq_fp8<BF16>(wv[j][t >> 1][(t & 1) * 2], wv[j][t >> 1][(t & 1) * 2 + 1],
                                                round_to<BF16>(raw));
                        }
                    }
#pragma unroll
                    for (int i = 0; i < MT; ++i) {
                        const uint8_t* ra = sa + (wm * MT * 16 + i * 16 + col16) * ARB;
                        const u32x4_t af = *reinterpret_cast<const u32x4_t*>(ra + (((4 * t + kq) ^ col16) * 16));
#pragma unroll
                        for (int j = 0; j < NS; ++j) acc[i][j] = mfma16x16x32<BF16>(af, b[j], acc[i][j]);
                    }
                }
            }
            if (more) {
#pragma unroll
                for (int j = 0; j < NS; ++j)
#pragma unroll
                    for (int t = 0; t < ST; ++t) sc[j][t] = scn[j][t];
                if constexpr (BREG) {
#pragma unroll
                    for (int j = 0; j < NS; ++j)
#pragma unroll
                        for (int h = 0; h < TB / 1024; ++h) wreg[j][h] = wnext[j][h];
                }
            }
        }
        // The stage the last K step read; the other one is free.
        const int last_stage = stage0 ^ ((kt_end - 1 - kt_begin) & 1);

        // PERSIST: the next item's first K step goes into the free stage now, so that its loads
        // are in flight during this item's epilogue (which stages through last_stage only).
        int next = -1;
        item_ctx nxt;
        if constexpr (PERSIST) {
            for (;;) {
                next = item_at(++pos);
                if (next < 0 || locate(next, nxt)) break;
            }
            if (next >= 0) issue(nxt, kt_begin, last_stage ^ 1);
        }

        if constexpr (A8) {
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = cur.row0 + wm * MT * 16 + i * 16 + 4 * kq + r;
                    const float sx = a.x_scale[min(row, a.m - 1)];
#pragma unroll
                    for (int j = 0; j < NS; ++j) acc[i][j][r] *= sx;
                }
        }

        // Split K (never PERSIST): every workgroup stores its accumulators in lane order (16
        // bytes per lane per MFMA tile, so each store instruction is one contiguous 1 KiB) into
        // its own slot of the work tile's partial area; the last workgroup to arrive reloads all
        // slots and sums them in split order, so the result does not depend on arrival order.
        // PLM_MEASURE_SKIP_REDUCTION (a measurement build only, never the shipped library): the
        // split workgroups write their own partial sums as the result, so timing the same
        // launches with and without it gives the cost of the split-K reduction (wrong results).
#ifndef PLM_MEASURE_SKIP_REDUCTION
#define PLM_MEASURE_SKIP_REDUCTION 0
#endif
        if (!PERSIST && a.splits > 1 && !PLM_MEASURE_SKIP_REDUCTION) {
            constexpr int TILE_BYTES = MT * NS * NT * 16;
            const __amdgpu_buffer_rsrc_t p_rsrc = make_rsrc(
                reinterpret_cast<uint8_t*>(a.partial) + static_cast<int64_t>(blockIdx.x) * a.splits * TILE_BYTES,
                static_cast<uint32_t>(a.splits * TILE_BYTES));
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < NS; ++j)
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, acc[i][j]), p_rsrc,
                                                           ((i * NS + j) * NT + tid) * 16, split * TILE_BYTES, kCoherent);
            if (!arrive_last(&a.counters[blockIdx.x], static_cast<uint32_t>(a.splits), &last_flag)) return;
            for (int sp = 0; sp < a.splits; ++sp) {
#pragma unroll
                for (int i = 0; i < MT; ++i)
#pragma unroll
                    for (int j = 0; j < NS; ++j) {
                        const f32x4_t v = __builtin_bit_cast(
                            f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(p_rsrc, ((i * NS + j) * NT + tid) * 16,
                                                                           sp * TILE_BYTES, kCoherent));
                        acc[i][j] = sp == 0 ? v : acc[i][j] + v;
                    }
            }
        }

        epilogue(cur, acc, last_stage);
        if (!PERSIST || next < 0) return;
        cur = nxt;
        stage0 = last_stage ^ 1;
        loaded = true;
    }
}

// Tile shapes: {WM, WN, MT, NS}.
struct shape {
    int wm, wn, mt, ns;
    constexpr int bm() const { return wm * mt * 16; }
    constexpr int bs() const { return wn * ns; }
};
// The 256-row shapes take int4 weights or W8A8 (fp8 weight tiles staged in LDS beside bf16 x
// would not fit); kTall also takes fp8 W8A16, whose weight tiles then go to registers.
constexpr shape kHuge{2, 4, 8, 4};   // 256 x 256, 8 wavefronts (two stages fill the 160 KiB LDS)
constexpr shape kWide{2, 4, 8, 3};   // 256 x 192, 8 wavefronts (N = 6144 gives whole rounds)
constexpr shape kTall{1, 8, 16, 2};  // 256 x 256, 8 wavefronts of 256 x 32: each strip dequantized once
constexpr shape kTallHalf{1, 8, 8, 2};  // 128 x 256, 8 wavefronts of 128 x 32 (tail launch of kTall)
constexpr shape kLarge{2, 2, 8, 4};  // 256 x 128, 4 wavefronts
constexpr shape kLarge8{2, 4, 8, 2};  // 256 x 128, 8 wavefronts of 128 x 32 (plain fp8 W8A16)
constexpr shape kSmall{2, 2, 4, 4};  // 128 x 128, 4 wavefronts
constexpr shape kSmall8{2, 4, 4, 2};  // 128 x 128, 8 wavefronts of 64 x 32 (int4): 2-12 % over kSmall
// Grouped calls also use short row blocks for experts with few rows.
constexpr shape kRows16{1, 4, 1, 2};  // 16 x 128
constexpr shape kRows64{1, 4, 4, 2};  // 64 x 128
constexpr shape kRows64w8{1, 8, 4, 1};  // 64 x 128, 8 wavefronts of one strip (plain int4 calls)
constexpr shape kRows32{1, 4, 2, 2};  // 32 x 128 (grouped)
constexpr shape kGroupedShapes[7] = {kRows16, kRows64, kSmall, kLarge, kHuge, kRows32, kTall};
constexpr shape shape_of(int id) {
    return id == 10 ? kTallHalf : id == 9 ? kLarge8 : id == 8 ? kRows64w8 : id == 7 ? kSmall8 : id == 6 ? kTall : id == 5 ? kWide : id == 4 ? kRows16 : id == 3 ? kRows64 : id == 2 ? kHuge : id == 1 ? kLarge : kSmall;
}
// Relative MFMA throughput per unit of tile area, measured on MI355X at the Qwen3-8B shapes.
constexpr double kShapeRate[10] = {0.75, 0.7, 1.0, 0.65, 0.3, 0.95, 1.03, 0.8, 0.7, 0.75};

}  // namespace

struct mfma_config {
    int shape;  // 0 small, 1 large, 2 huge, 3 rows64, 4 rows16, 5 wide, 6 tall
    int m_blocks, n_blocks;
    int splits, tiles_per_split;
    // Two launches when the tiles fill the CUs a whole number of times plus at most half a
    // round: the last tail_tiles work tiles run second, with K split tail_splits ways, so
    // the last round is shorter instead of half empty.
    int tail_tiles, tail_splits, tail_tiles_per_split;
    // The tall shape, when the tail is whole columns of work tiles: the tail runs
    // unsplit as 128-row halves of those tiles (shape 10), twice as many workgroups with no
    // partial sums to combine.
    bool tail_halves;
};

bool tail_halves_off() { return knobs().mfma_no_halves; }  // A/B measurements

bool no_tail() { return knobs().mfma_no_tail; }  // A/B measurements

// Tile shape and split count: the candidate with the least estimated time, counting whole
// rounds of workgroups over the CUs, a fixed cost of about three K tiles per workgroup
// (pipeline fill, epilogue) and half a K tile per split for the split-K reduction.
// The 256-row shapes with 12 or 16 strips need int4 weights, or fp8 weights with e4m3 x
// (W8A8): with bf16 x and 2 KiB fp8 tiles two stages would not fit the 160 KiB LDS.
mfma_config choose_mfma(plm_format f, int64_t m, int64_t n, int64_t k, bool a8) {
    const bool wide_ok = f == PLM_INT4 || a8;
    const bool tall_ok = wide_ok || f == PLM_FP8;  // fp8 W8A16 runs the tall shape with weights in registers
    const bool small8_ok = f == PLM_INT4 && !a8;
    // 256 x 128 on 8 wavefronts: 4-9 % faster than on 4 for fp8 W8A16 at the Qwen3-27B
    // shapes; for int4 the other shapes measured better.
    const bool large8_ok = f == PLM_FP8 && !a8;
    const int64_t cus = cu_count();
    const int64_t strips = ceil_div(n, kTileN), ktiles = ceil_div(k, kTileK);
    auto config = [&](int id) {
        const shape sh = shape_of(id);
        mfma_config c{};
        c.shape = id;
        c.m_blocks = static_cast<int>(ceil_div(m, sh.bm()));
        c.n_blocks = static_cast<int>(ceil_div(strips, sh.bs()));
        const int64_t tiles = static_cast<int64_t>(c.m_blocks) * c.n_blocks;
        int64_t splits = 1;
        if (tiles < cus && tiles <= kMaxCounters && !knobs().mfma_unsplit)
            splits = std::max<int64_t>(1, std::min<int64_t>(ceil_div(cus, tiles), ktiles / 4));
        c.tiles_per_split = static_cast<int>(ceil_div(ktiles, splits));
        c.splits = static_cast<int>(ceil_div(ktiles, c.tiles_per_split));
        const int64_t rem = tiles % cus;
        if (c.splits == 1 && tiles > cus && rem > 0 && 2 * rem <= cus && rem <= kMaxCounters && ktiles >= 8 &&
            !no_tail() && !knobs().mfma_unsplit) {
            const int64_t ts = std::min<int64_t>(cus / rem, ktiles / 4);
            c.tail_tiles_per_split = static_cast<int>(ceil_div(ktiles, ts));
            c.tail_splits = static_cast<int>(ceil_div(ktiles, c.tail_tiles_per_split));
            if (c.tail_splits >= 2) c.tail_tiles = static_cast<int>(rem);
            // (fp8 W8A16, whose tall shape keeps the weights in registers, measured slower.)
            if (id == 6 && (f == PLM_INT4 || a8) && rem % c.m_blocks == 0 && !tail_halves_off()) {
                c.tail_tiles = static_cast<int>(rem);
                c.tail_halves = true;
                c.tail_splits = 1;
                c.tail_tiles_per_split = static_cast<int>(ktiles);
            }
        }
        return c;
    };
    auto cost = [&](const mfma_config& c) {
        const shape sh = shape_of(c.shape);
        // fp8 W8A16 (2 KiB weight tiles dequantized to bf16): 128 x 128 measured 10-15 %
        // slower than 256 x 128 at the Qwen3-27B shapes, unlike int4; the tall shape (weights
        // in registers) measured 15 % faster than 256 x 128 for gate_up (1088 tiles) and slower
        // for the layers with 160-448 tiles, which a rate of 0.75 reproduces.
        double rate = kShapeRate[c.shape];
        if (f == PLM_FP8 && !a8 && c.shape == 0) rate = 0.5;
        if (f == PLM_FP8 && !a8 && c.shape == 6) rate = 0.75;
        if (f == PLM_FP8 && !a8 && c.shape == 9) rate = 0.72;
        const double area = static_cast<double>(sh.bm()) * sh.bs() / rate;
        const int64_t tiles = static_cast<int64_t>(c.m_blocks) * c.n_blocks;
        if (c.tail_halves) {  // half-area tiles, assumed 10 % less efficient
            const int64_t full_rounds = (tiles - c.tail_tiles) / cus;
            return (static_cast<double>(full_rounds) * (c.tiles_per_split + 3) + 0.55 * (ktiles + 3)) * area;
        }
        if (c.tail_tiles > 0) {
            const int64_t full_rounds = (tiles - c.tail_tiles) / cus;
            return (static_cast<double>(full_rounds) * (c.tiles_per_split + 3) + c.tail_tiles_per_split + 3 +
                    0.5 * c.tail_splits) * area;
        }
        const int64_t rounds = ceil_div(tiles * c.splits, cus);
        // The last workgroup of a split tile reads every split's partials: half a K tile each.
        const double reduce = c.splits > 1 ? 0.5 * c.splits : 0.0;
        return static_cast<double>(rounds) * (c.tiles_per_split + 3 + reduce) * area;
    };
    if (const char f = knobs().mfma_shape) {  // PLM_MFMA (tuning sweeps)
        const int id = f == 'G' ? 9 : f == 'Q' ? 8 : f == 'E' ? 7 : f == 'X' ? 6 : f == 'H' ? 2 : f == 'L' ? 1 : f == 'R' ? 3 : f == 'T' ? 4 : f == 'W' ? 5 : 0;
        return config(((id == 2 || id == 5) && !wide_ok) || (id == 6 && !tall_ok) || ((id == 7 || id == 8) && !small8_ok) ||
                              (id == 9 && !large8_ok) ? 1 : id);
    }
    mfma_config best = config(0);
    for (int id : {1, 2, 3, 5, 6, 7, 8, 9}) {
        if (((id == 2 || id == 5) && !wide_ok) || (id == 6 && !tall_ok) || ((id == 7 || id == 8) && !small8_ok) ||
            (id == 9 && !large8_ok))
            continue;
        const mfma_config c = config(id);
        if (cost(c) < cost(best)) best = c;
    }
    return best;
}

int64_t mfma_workspace_bytes(plm_format f, int64_t m, int64_t n, int64_t k, bool a8) {
    const mfma_config c = choose_mfma(f, m, n, k, a8);
    const shape sh = shape_of(c.shape);
    const int64_t tile_bytes = static_cast<int64_t>(sh.bm()) * sh.bs() * kTileN * 4;
    if (c.tail_halves) return 0;
    if (c.tail_tiles > 0) return kCounterBytes + static_cast<int64_t>(c.tail_tiles) * c.tail_splits * tile_bytes;
    if (c.splits <= 1) return 0;
    return kCounterBytes + static_cast<int64_t>(c.m_blocks) * c.n_blocks * c.splits * tile_bytes;
}

namespace {
template <plm_format F, bool BF16, bool UNIFORM, bool WIDE, bool A8, bool GROUPED>
void launch_shape(const mfma_args& a, int shape, dim3 grid, hipStream_t s) {
    // The 16-byte epilogue for the unsplit tall shapes.
    [[maybe_unused]] const bool vo = a.splits == 1 && (a.n & 7) == 0 && aligned(a.y, 16);
    if constexpr (!A8 && !GROUPED) {
        if (shape == 9) {
            mfma_kernel<F, BF16, UNIFORM, WIDE, A8, GROUPED, kLarge8.wm, kLarge8.wn, kLarge8.mt, kLarge8.ns>
                <<<grid, kLarge8.wm * kLarge8.wn * 64, 0, s>>>(a);
            return;
        }
    }
    if constexpr (F == PLM_FP8 && !A8 && !GROUPED) {  // weights in registers (BREG): tall only
        if (shape == 6) {
            mfma_kernel<F, BF16, UNIFORM, WIDE, A8, GROUPED, kTall.wm, kTall.wn, kTall.mt, kTall.ns>
                <<<grid, kTall.wm * kTall.wn * 64, 0, s>>>(a);
            return;
        }
    }
    if constexpr (((F == PLM_INT4 && !A8) || (F == PLM_FP8 && A8)) && !GROUPED) {
        if (shape == 2) {
            mfma_kernel<F, BF16, UNIFORM, WIDE, A8, GROUPED, kHuge.wm, kHuge.wn, kHuge.mt, kHuge.ns>
                <<<grid, kHuge.wm * kHuge.wn * 64, 0, s>>>(a);
            return;
        }
        if (shape == 5) {
            mfma_kernel<F, BF16, UNIFORM, WIDE, A8, GROUPED, kWide.wm, kWide.wn, kWide.mt, kWide.ns>
                <<<grid, kWide.wm * kWide.wn * 64, 0, s>>>(a);
            return;
        }
        if (shape == 7) {
            mfma_kernel<F, BF16, UNIFORM, WIDE, A8, GROUPED, kSmall8.wm, kSmall8.wn, kSmall8.mt, kSmall8.ns>
                <<<grid, kSmall8.wm * kSmall8.wn * 64, 0, s>>>(a);
            return;
        }
        if (shape == 10) {
            if (vo)
                mfma_kernel<F, BF16, UNIFORM, WIDE, A8, GROUPED, kTallHalf.wm, kTallHalf.wn, kTallHalf.mt, kTallHalf.ns,
                            true><<<grid, kTallHalf.wm * kTallHalf.wn * 64, 0, s>>>(a);
            else
                mfma_kernel<F, BF16, UNIFORM, WIDE, A8, GROUPED, kTallHalf.wm, kTallHalf.wn, kTallHalf.mt, kTallHalf.ns>
                    <<<grid, kTallHalf.wm * kTallHalf.wn * 64, 0, s>>>(a);
            return;
        }
        if (shape == 8) {
            mfma_kernel<F, BF16, UNIFORM, WIDE, A8, GROUPED, kRows64w8.wm, kRows64w8.wn, kRows64w8.mt, kRows64w8.ns>
                <<<grid, kRows64w8.wm * kRows64w8.wn * 64, 0, s>>>(a);
            return;
        }
        if (shape == 6) {
            if (vo)
                mfma_kernel<F, BF16, UNIFORM, WIDE, A8, GROUPED, kTall.wm, kTall.wn, kTall.mt, kTall.ns, true>
                    <<<grid, kTall.wm * kTall.wn * 64, 0, s>>>(a);
            else
                mfma_kernel<F, BF16, UNIFORM, WIDE, A8, GROUPED, kTall.wm, kTall.wn, kTall.mt, kTall.ns>
                    <<<grid, kTall.wm * kTall.wn * 64, 0, s>>>(a);
            return;
        }
    }
    if (shape == 4)
        mfma_kernel<F, BF16, UNIFORM, WIDE, A8, GROUPED, kRows16.wm, kRows16.wn, kRows16.mt, kRows16.ns>
            <<<grid, kRows16.wm * kRows16.wn * 64, 0, s>>>(a);
    else if (shape == 3)
        mfma_kernel<F, BF16, UNIFORM, WIDE, A8, GROUPED, kRows64.wm, kRows64.wn, kRows64.mt, kRows64.ns>
            <<<grid, kRows64.wm * kRows64.wn * 64, 0, s>>>(a);
    else if (shape >= 1)
        mfma_kernel<F, BF16, UNIFORM, WIDE, A8, GROUPED, kLarge.wm, kLarge.wn, kLarge.mt, kLarge.ns>
            <<<grid, kLarge.wm * kLarge.wn * 64, 0, s>>>(a);
    else
        mfma_kernel<F, BF16, UNIFORM, WIDE, A8, GROUPED, kSmall.wm, kSmall.wn, kSmall.mt, kSmall.ns>
            <<<grid, kSmall.wm * kSmall.wn * 64, 0, s>>>(a);
}

template <plm_format F, bool BF16, bool WIDE, bool GROUPED>
void launch_mode_w(const mfma_args& a, int large, bool uniform, bool a8, dim3 grid, hipStream_t s) {
    if constexpr (F == PLM_FP8 && !GROUPED) {
        if (a8) {
            launch_shape<F, BF16, true, WIDE, true, GROUPED>(a, large, grid, s);
            return;
        }
    }
    if (uniform) launch_shape<F, BF16, true, WIDE, false, GROUPED>(a, large, grid, s);
    else launch_shape<F, BF16, false, WIDE, false, GROUPED>(a, large, grid, s);
}

template <plm_format F, bool BF16, bool GROUPED>
void launch_mode(const mfma_args& a, int large, bool uniform, bool a8, dim3 grid, hipStream_t s) {
    if (a.scale_dtype == PLM_FP32) launch_mode_w<F, BF16, true, GROUPED>(a, large, uniform, a8, grid, s);
    else launch_mode_w<F, BF16, false, GROUPED>(a, large, uniform, a8, grid, s);
}

template <bool GROUPED>
void launch_all(plm_format f, bool bf16, const mfma_args& a, int large, bool uniform, bool a8, dim3 grid,
                hipStream_t s) {
    if (f == PLM_INT4) {
        if (bf16) launch_mode<PLM_INT4, true, GROUPED>(a, large, uniform, a8, grid, s);
        else launch_mode<PLM_INT4, false, GROUPED>(a, large, uniform, a8, grid, s);
    } else {
        if (bf16) launch_mode<PLM_FP8, true, GROUPED>(a, large, uniform, a8, grid, s);
        else launch_mode<PLM_FP8, false, GROUPED>(a, large, uniform, a8, grid, s);
    }
}

void fill_common(mfma_args& a, const void* x, const void* w, const void* scale, plm_dtype scale_dtype, int64_t m,
                 int64_t n, int64_t k, int64_t block_n, int64_t group_size, void* y) {
    const layout_dims d = make_dims(n, k, block_n, group_size);
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
}
}  // namespace

int launch_mfma(const char* op, plm_format f, const void* x, bool bf16, const void* w, const void* scale,
                plm_dtype scale_dtype, int64_t m, int64_t n, int64_t k, int64_t block_n, int64_t group_size, void* y,
                void* workspace, size_t workspace_bytes, hipStream_t s, const uint8_t* xq, const float* x_scale) {
    PLM_CHECK_ARG(k <= (int64_t{1} << 21), op, "K above 2^21 is not supported");
    const bool a8 = xq != nullptr;
    const mfma_config c = choose_mfma(f, m, n, k, a8);
    mfma_args a{};
    fill_common(a, x, w, scale, scale_dtype, m, n, k, block_n, group_size, y);
    a.splits = c.splits;
    a.tiles_per_split = c.tiles_per_split;
    a.m_blocks = c.m_blocks;
    a.n_blocks = c.n_blocks;
    a.xq = xq;
    a.x_scale = x_scale;
    if (c.splits > 1 || (c.tail_tiles > 0 && !c.tail_halves)) {
        const int64_t need = mfma_workspace_bytes(f, m, n, k, a8);
        if (workspace == nullptr || static_cast<int64_t>(workspace_bytes) < need) {
            set_error(op, "workspace of %lld bytes required, %zu given", static_cast<long long>(need), workspace_bytes);
            return PLM_ERR_WORKSPACE;
        }
        a.counters = static_cast<uint32_t*>(workspace);
        a.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
    }
    const bool uniform = group_size % kTileK == 0;
    const int tiles = c.m_blocks * c.n_blocks;
    if (c.tail_halves) {
        // Whole rounds of tall tiles, then the tail's columns of tiles as 128-row halves.
        const int nb_full = (tiles - c.tail_tiles) / c.m_blocks;
        launch_all<false>(f, bf16, a, c.shape, uniform, a8, dim3(tiles - c.tail_tiles, 1), s);
        PLM_HIP_LAUNCH_CHECK(op);
        const int mb2 = static_cast<int>(ceil_div(m, kTallHalf.bm()));
        a.m_blocks = mb2;
        a.tile_base = nb_full * mb2;
        launch_all<false>(f, bf16, a, 10, uniform, a8, dim3((c.n_blocks - nb_full) * mb2, 1), s);
        PLM_HIP_LAUNCH_CHECK(op);
        return PLM_OK;
    }
    if (c.tail_tiles > 0) {
        // Whole rounds of unsplit tiles, then the tail tiles with K split.
        launch_all<false>(f, bf16, a, c.shape, uniform, xq != nullptr, dim3(tiles - c.tail_tiles, 1), s);
        PLM_HIP_LAUNCH_CHECK(op);
        a.tile_base = tiles - c.tail_tiles;
        a.splits = c.tail_splits;
        a.tiles_per_split = c.tail_tiles_per_split;
        launch_all<false>(f, bf16, a, c.shape, uniform, xq != nullptr, dim3(c.tail_tiles, c.tail_splits), s);
        PLM_HIP_LAUNCH_CHECK(op);
        return PLM_OK;
    }
    launch_all<false>(f, bf16, a, c.shape, uniform, xq != nullptr, dim3(tiles, c.splits), s);
    PLM_HIP_LAUNCH_CHECK(op);
    return PLM_OK;
}

// Grouped: `tiles` holds max_tiles (expert, first row, rows) records built on the device;
// rows are in the grouped (sorted) order and `row_index` optionally gathers them from x.
// shape indexes kGroupedShapes (int4 experts only); 6 (256 x 256 tall) is for full blocks of rows.
namespace {
// PERSIST launches: about one workgroup per slot the kernel can hold resident (occupancy per CU
// times the CUs), a multiple of 8 so that every XCD gets the same number of workgroups, and
// never more than the items.
template <typename K>
unsigned persistent_grid(K kernel, int threads, unsigned items) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess || per_cu < 1)
        per_cu = 1;
    const unsigned slots = static_cast<unsigned>(per_cu * cu_count()) & ~7u;
    return std::max(8u, std::min(items, slots));
}

template <bool BF16, bool UNIFORM, bool WIDE, int I>
void launch_grouped_one(const mfma_args& a, dim3 grid, bool persist, hipStream_t s) {
    constexpr shape sh = kGroupedShapes[I];
    constexpr int threads = sh.wm * sh.wn * 64;
    if constexpr (I != 4) {  // the 256 x 256 two-row grid (unused by the MoE block) is never persistent
        if (persist) {
            auto* kernel = mfma_kernel<PLM_INT4, BF16, UNIFORM, WIDE, false, true, sh.wm, sh.wn, sh.mt, sh.ns, true, true>;
            grid.x = persistent_grid(kernel, threads, grid.x);
            kernel<<<grid, threads, 0, s>>>(a);
            return;
        }
    }
    mfma_kernel<PLM_INT4, BF16, UNIFORM, WIDE, false, true, sh.wm, sh.wn, sh.mt, sh.ns, true>
        <<<grid, threads, 0, s>>>(a);
}

template <bool BF16, bool UNIFORM, bool WIDE>
void launch_grouped_shape(const mfma_args& a, int shape, dim3 grid, bool persist, hipStream_t s) {
    switch (shape) {
        case 0: launch_grouped_one<BF16, UNIFORM, WIDE, 0>(a, grid, persist, s); break;
        case 1: launch_grouped_one<BF16, UNIFORM, WIDE, 1>(a, grid, persist, s); break;
        case 2: launch_grouped_one<BF16, UNIFORM, WIDE, 2>(a, grid, persist, s); break;
        case 3: launch_grouped_one<BF16, UNIFORM, WIDE, 3>(a, grid, persist, s); break;
        case 5: launch_grouped_one<BF16, UNIFORM, WIDE, 5>(a, grid, persist, s); break;
        case 6: launch_grouped_one<BF16, UNIFORM, WIDE, 6>(a, grid, persist, s); break;
        default: launch_grouped_one<BF16, UNIFORM, WIDE, 4>(a, grid, persist, s); break;
    }
}
}  // namespace

int grouped_block_rows(int shape) { return kGroupedShapes[std::min(std::max(shape, 0), 6)].bm(); }

// Row block for a grouped call, from the average rows per expert. At the Zipf-routed
// T = 256 block (16 rows per expert on average, the heaviest experts near 250) 32-row tiles
// measured 6 % faster than 16-row ones and 64-row ones 5 % slower: a weight tile is
// dequantized once per row block, and the dequant bounds these small GEMMs.
int grouped_rows_env() { return knobs().moe_rows; }  // PLM_MOE_ROWS=16/32/64 (tuning sweeps)
int grouped_shape_for(int64_t rows, int64_t n_experts) {
    const int64_t avg = ceil_div(rows, std::max<int64_t>(n_experts, 1));
    switch (grouped_rows_env()) {
        case 16: return 0;
        case 32: return 5;
        case 64: return 1;
        default: break;
    }
    if (avg <= 8) return 0;
    if (avg <= 24) return 5;
    if (avg <= 96) return 1;
    if (avg <= 192) return 2;
    return 3;
}

int launch_grouped(const char* op, plm_format f, const void* x, bool bf16, const void* w, const void* scale,
                   plm_dtype scale_dtype, int64_t rows, int64_t n, int64_t k, int64_t block_n, int64_t group_size,
                   void* y, const int32_t* tiles, int64_t max_tiles, const int32_t* tile_count,
                   const int32_t* row_index, int shape, hipStream_t s, bool swiglu) {
    PLM_CHECK_ARG(f == PLM_INT4, op, "grouped GEMMs take int4 experts");
    PLM_CHECK_ARG(k <= (int64_t{1} << 21) && rows * k * 2 < kOOB && n * k < (int64_t{1} << 40), op,
                  "problem too large");
    mfma_args a{};
    fill_common(a, x, w, scale, scale_dtype, rows, n, k, block_n, group_size, y);
    const struct shape sh = kGroupedShapes[std::min(std::max(shape, 0), 6)];
    a.splits = 1;
    a.tiles_per_split = a.ktiles;
    a.m_blocks = 1;
    a.n_blocks = static_cast<int>(ceil_div(a.strips, sh.bs()));
    if (swiglu) {  // [gate; up] with whole 16-column strips each: slices of bs / 2 strip pairs
        PLM_CHECK_ARG(n % (2 * kTileN) == 0 && sh.ns % 2 == 0, op, "fused activation needs 16 | intermediate");
        a.swiglu_strips = static_cast<int>(n / (2 * kTileN));
        a.n_blocks = static_cast<int>(ceil_div(a.swiglu_strips, sh.bs() / 2));
    }
    a.tiles = tiles;
    a.tile_count = tile_count;
    a.row_index = row_index;
    a.w_expert_bytes = ceil_div(n, kTileN) * ceil_div(k, kTileK) * tile_bytes(f);
    a.s_expert_bytes = static_cast<int64_t>(a.strips) * a.groups * a.scale_cols * dtype_size(scale_dtype);
    dim3 grid(static_cast<unsigned>(round_up(max_tiles * a.n_blocks, 8)), 1);  // whole XCD rounds
    const bool persist = knobs().moe_persist;  // A/B measurements: measured slower
    const bool uniform = group_size % kTileK == 0;
    const bool wide = scale_dtype == PLM_FP32;
    const int mode = (bf16 ? 4 : 0) + (uniform ? 2 : 0) + (wide ? 1 : 0);
    switch (mode) {
        case 0: launch_grouped_shape<false, false, false>(a, shape, grid, persist, s); break;
        case 1: launch_grouped_shape<false, false, true>(a, shape, grid, persist, s); break;
        case 2: launch_grouped_shape<false, true, false>(a, shape, grid, persist, s); break;
        case 3: launch_grouped_shape<false, true, true>(a, shape, grid, persist, s); break;
        case 4: launch_grouped_shape<true, false, false>(a, shape, grid, persist, s); break;
        case 5: launch_grouped_shape<true, false, true>(a, shape, grid, persist, s); break;
        case 6: launch_grouped_shape<true, true, false>(a, shape, grid, persist, s); break;
        default: launch_grouped_shape<true, true, true>(a, shape, grid, persist, s); break;
    }
    PLM_HIP_LAUNCH_CHECK(op);
    return PLM_OK;
}

}  // namespace plm

extern "C" {
// Not part of the public ABI (include/pulsarlm_amd.h): the MFMA kernel's plan for a plain GEMM,
// for bench.py's report of the split-K / tail decomposition. out[0..7]: tile rows, tile
// columns, work tiles, K splits, tail tiles, tail K splits, tail as 128-row halves (0/1), and
// whether this build skips the split-K reduction (a measurement build, results invalid).
__attribute__((visibility("default"))) void plm_internal_mfma_plan(int format, int64_t m, int64_t n, int64_t k, int a8,
                                                                  int32_t* out) {
    using namespace plm;
    const mfma_config c = choose_mfma(static_cast<plm_format>(format), m, n, k, a8 != 0);
    const shape sh = shape_of(c.shape);
    out[0] = sh.bm();
    out[1] = sh.bs() * kTileN;
    out[2] = c.m_blocks * c.n_blocks;
    out[3] = c.splits;
    out[4] = c.tail_tiles;
    out[5] = c.tail_halves ? 1 : c.tail_splits;
    out[6] = c.tail_halves ? 1 : 0;
    out[7] = PLM_MEASURE_SKIP_REDUCTION;
}
}  // extern "C"
