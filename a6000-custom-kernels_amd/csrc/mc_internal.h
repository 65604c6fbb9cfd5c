// mc_internal.h -- shared between the C++ host code and the gfx950 kernels.
//
// Geometry of the GEMV: each 64-lane wavefront owns one "step" of a routed
// pick (or of the shared expert): rows_per_step consecutive rows of one expert
// matrix.  A row is split into `nu` lane units of UNIT_ELEMS values; one lane
// computes one unit.  K-quant units are one 256-value super-block; legacy
// units are two 32-value blocks (so every unit starts on a 4-byte boundary).
#ifndef MC_INTERNAL_H
#define MC_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

namespace mc {

enum : int {
    T_F32 = 0, T_Q4_0 = 2, T_Q5_0 = 6, T_Q8_0 = 8, T_Q8_1 = 9,
    T_Q2_K = 10, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_Q8_K = 15
};

// Activation formats: q8_1 blocks, q8_K blocks, or fp32 rows that the GEMV
// quantizes to q8_1 itself (same codes and scales as the q8_1 quantizer).
enum : int { ACT_Q8_1 = 0, ACT_Q8_K = 1, ACT_F32 = 2 };

// Device stats buffer: [0] miss count, [1] resident-hit count,
// [2 .. 2+MISS_CAP) miss log of (cache_id << 12 | expert) entries
// (kernels/moe-cache.cu:34-40).
constexpr int MISS_CAP = 8190;
constexpr int HIT_WORD = 1;
constexpr int LOG_BASE = 2;
constexpr int STATS_WORDS = 2 + MISS_CAP;
constexpr int DEFAULT_MAX_PROMOTIONS = 48;

constexpr int WAVE = 64;

struct TypeGeom {
    int block_elems;
    int block_bytes;
    int unit_elems;   // values per lane unit
    int unit_bytes;   // bytes per lane unit
    int aligned;      // 1: unit offsets are multiples of 4 bytes; 0: only of 2
    int kquant;
};

inline constexpr TypeGeom type_geom(int t) {
    return t == T_Q4_0 ? TypeGeom{32, 18, 64, 36, 1, 0}
         : t == T_Q5_0 ? TypeGeom{32, 22, 64, 44, 1, 0}
         : t == T_Q8_0 ? TypeGeom{32, 34, 64, 68, 1, 0}
         : t == T_Q2_K ? TypeGeom{256, 84, 256, 84, 1, 1}
         : t == T_Q3_K ? TypeGeom{256, 110, 256, 110, 0, 1}
         : t == T_Q4_K ? TypeGeom{256, 144, 256, 144, 1, 1}
         : t == T_Q5_K ? TypeGeom{256, 176, 256, 176, 1, 1}
         : t == T_Q6_K ? TypeGeom{256, 210, 256, 210, 0, 1}
         : TypeGeom{0, 0, 0, 0, 0, 0};
}

inline constexpr bool type_supported(int t) { return type_geom(t).block_elems != 0; }

// Bytes of LDS one wave needs to stage one step of one matrix: the step's
// byte span (<= 64 units) plus up to 15 bytes of lead-in to the 16-byte
// aligned start and 4 bytes of over-read, in whole 1 KiB DMA rounds.
inline constexpr int span_lds_bytes(int t) {
    return ((WAVE * type_geom(t).unit_bytes + 20 + 1023) / 1024) * 1024;
}

// Kernel arguments (passed by value).
struct GemvArgs {
    // routed experts, resolved through tagged pointer tables (LSB=1: host memory)
    const uint64_t *tbl;          // [n_experts] up / plain projection
    const uint64_t *tbl_gate;     // [n_experts] gate projection, or null
    uint32_t *stamps;             // [n_experts] last-use clock of tbl's tensor, or null
    uint32_t *stamps_gate;        // [n_experts] of tbl_gate's tensor, or null
    uint32_t *stats;              // [STATS_WORDS], or null (no recording)
    const uint32_t *clock;        // device LRU clock (read, never a kernel-argument value)
    int32_t cache_id;             // registry id of tbl's tensor
    int32_t cache_id_gate;        // registry id of tbl_gate's tensor (-1: none)
    int32_t n_experts;
    int32_t has_gate;             // 1: fused gate present (through tbl_gate)
    uint64_t expert_bytes;        // bytes of one expert matrix
    // device-resident tensors: expert e at w_base + e * expert_bytes (no table
    // read on the way to the weights); null: resolve through tbl / tbl_gate
    const uint8_t *w_base;
    const uint8_t *w_gate_base;
    // activations
    const uint8_t *y;             // activation base (q8_1 or q8_K blocks)
    uint64_t y_bytes;             // addressable bytes from y (buffer range)
    int64_t stride_col_y;         // bytes between tokens
    int64_t stride_channel_y;     // bytes between channels
    uint32_t nchannels_y;
    const int32_t *ids;           // [n_tok][ids_stride]
    int64_t ids_stride;           // int32 elements
    // outputs
    float *dst;
    int64_t stride_col_dst;       // floats between tokens
    int64_t stride_channel_dst;   // floats between channels (picks)
    // fusion
    const float *x_bias;
    const float *gate_bias;
    const float *x_scale;
    const float *gate_scale;
    int64_t bias_stride;          // floats per expert
    int32_t glu_op;
    float glu_limit;
    // shared expert (dense)
    const uint8_t *sh_up;
    const uint8_t *sh_gate;
    float *sh_dst;
    int64_t sh_stride_col_dst;
    const uint8_t *sh_y;          // null: channel 0 of y
    uint64_t sh_y_bytes;
    int64_t sh_stride_col_y;      // bytes between tokens of sh_y
    int32_t sh_act_f32;           // FFN_DOWN_COMBINE: sh_y rows are fp32 (quantized by the shared wave)
    uint32_t sh_act_row_bytes;    // bytes of one sh_y row
    uint64_t sh_matrix_bytes;     // bytes of the shared matrix
    // shape
    int32_t ncols;                // K (ne00)
    int32_t nrows;                // rows per expert (ne01)
    int32_t n_used;               // picks per token (nchannels_dst)
    int32_t n_tok;                // tokens (ncols_dst)
    // tiling and LDS layout (filled by the launcher)
    int32_t rps;                  // rows per step of a routed matrix
    int32_t sh_rps;               // rows per step of the shared matrix
    int32_t tiles_per_pick;
    int32_t sh_tiles_per_tok;
    int32_t n_routed_tiles;
    int32_t n_tiles;
    int32_t rec;                  // 1: workgroup 0 is the pick recorder, tiles start at 1
    uint32_t act_row_bytes;       // bytes of one activation row
    uint32_t lds_span;            // LDS bytes per staged matrix span (up at 0, gate at lds_span)
    uint32_t lds_act;             // LDS offset of the staged activation row
    uint32_t lds_q8;              // LDS offset of the in-kernel q8_1 copy of an fp32 activation row
    uint32_t lds_total;           // dynamic LDS bytes per workgroup
    // fused decode kernels (mc_ffn.hip); FFN_NONE: the plain MUL_MAT_ID GEMV
    int32_t mode;
    int32_t nwaves;               // step waves per workgroup (FFN_GATE_UP_NORM: plus FFN_GU_PRO_WAVES)
    int32_t dot_act;              // fused kernels: the dots' activation format (ACT_Q8_1 or ACT_Q8_K)
    int32_t sh_per_wg;            // FFN_GATE_UP_NORM with hq: steps of a shared-expert workgroup (its
                                  //   first workgroups take only shared steps, about as many bytes as
                                  //   the routed workgroups' nwaves steps)
    int32_t mixed_wg;             // FFN_GATE_UP_NORM without hq: each of a token's wg_per_tok
                                  //   workgroups takes an even share of the routed steps, then of the
                                  //   shared steps (shares differ by at most one step)
    int32_t wg_per_tok;           // workgroups per token
    int32_t tiles_per_tok;        // steps per token: shared tiles first, then the routed picks'
    uint32_t lds_wave;            // LDS bytes of one wave's region (spans, activation staging)
    uint32_t lds_y;               // FFN_GATE_UP_NORM: q8_1 row
    uint32_t lds_sums;            // LDS offset of the activation row's 16-value sums (down + combine: in a wave's region)
    uint32_t lds_part;            // FFN_GATE_UP_NORM: counters + chunk sums; FFN_DOWN_COMBINE: row results [nwaves][rps]
    // FFN_GATE_UP_NORM: y = q8_1((x * rms_scale(x)) * nw), computed by every workgroup
    const float *nx;              // [n_tok][nx_stride] rows to normalize
    int64_t nx_stride;            // floats
    const float *nw;              // [ncols] norm weight, or null
    float eps;
    uint8_t *y_out;               // optional copy of the q8_1 rows (written by each token's first workgroup)
    int64_t y_out_stride;         // bytes
    uint8_t *hq;                  // optional q8_1 copy of the routed outputs: pick c of token t at
    int64_t hq_stride_col;        //   hq + t * hq_stride_col + c * hq_stride_pick (bytes); needs
    int64_t hq_stride_pick;       //   workgroups of exactly 32 rows of one matrix (one q8_1 block)
    uint8_t *hq_sh;               // ... of the shared expert's output: hq_sh + t * hq_sh_stride
    int64_t hq_sh_stride;
    // FFN_DOWN_COMBINE: x_out = residual + shared + sum_c router_w[c] * o_c (c ascending, fmaf)
    const float *router_w;        // [n_tok][n_used]
    const float *residual;        // [n_tok][x_stride], or null
    float *x_out;                 // [n_tok][x_stride]
    int64_t x_stride;             // floats
    // device status word (STATUS_* bits), set by a kernel that could not finish its work
    uint32_t *status;
    int32_t spin_limit;           // iterations of a bounded in-kernel wait before it gives up
};

// Bytes of the per-GPU device scratch of ggml_hip_moe_mul_mat_id_noalloc (mc_noalloc.hip):
// enough for the 512-token prefill of a 512-expert layer with 4096-value rows
// (q8_K rows 2.4 MB + grouped-GEMM workspace 54.6 MB).
constexpr uint64_t NOALLOC_SCRATCH_BYTES = 64ull << 20;

// Device status bits (ggml_hip_moe_check_status).
constexpr uint32_t STATUS_WAIT_TIMEOUT = 1u;   // a bounded wait of the fused gate/up kernel gave up
constexpr int32_t DEFAULT_SPIN_LIMIT = 1 << 22;

enum : int { FFN_NONE = 0, FFN_GATE_UP_NORM = 1, FFN_DOWN_COMBINE = 2 };
constexpr int FFN_GU_MAX_WAVES = 8;    // gate/up workgroups: up to 8 step waves sharing one normalized row
constexpr int FFN_GU_PRO_WAVES = 4;    // ... plus 4 waves that compute that row (no weight DMA of their own)
constexpr int FFN_DN_MAX_WAVES = 12;   // down + combine workgroups: one wave per pick + the shared expert
constexpr uint32_t FFN_LDS_MAX = 160 * 1024;

// LDS a GEMV workgroup may use, chosen so that 8 workgroups fit one CU's
// 160 KiB: a decode launch of ~2000 single-wave tiles is then resident at once.
constexpr uint32_t GEMV_LDS_BUDGET = 20 * 1024;
// Longest row of the plain GEMV: its activation row (and, for fp32 rows, the q8_1 copy) is
// staged in LDS beside two 64-unit spans, within FFN_LDS_MAX.
constexpr int GEMV_MAX_K = 65536;
constexpr int GEMV_MAX_K_F32 = 16384;

inline constexpr uint32_t round_up_1k(uint32_t b) { return (b + 1023u) & ~1023u; }

// LDS bytes staging `rows` rows of `row_bytes` (16-byte lead-in + 4-byte over-read, whole 1 KiB DMA rounds).
inline constexpr uint32_t span_bytes(uint32_t rows, uint32_t row_bytes) { return round_up_1k(rows * row_bytes + 20u); }

struct QuantArgs {
    const float *x;
    uint8_t *y;
    int64_t k;          // values per row
    int64_t nrows;
    int64_t x_stride;   // floats between rows
    int64_t y_stride;   // bytes between rows
};

struct CombineArgs {
    const float *o;          // [n_tok][n_used][o_stride] routed expert outputs
    int64_t o_stride;        // floats between picks
    const float *w;          // [n_tok][n_used] router weights
    const float *shared;     // [n_tok][shared_stride] shared-expert output, or null
    int64_t shared_stride;
    const float *residual;   // [n_tok][k], or null
    float *x_out;            // [n_tok][k], or null
    uint8_t *y;              // q8_1 rows of the combined vector
    int64_t y_stride;        // bytes between rows
    int64_t k;
    int32_t n_used;
    int32_t n_tok;
    int32_t rms_norm;        // quantize (x * rms scale) * norm_weight instead of x
    const float *norm_weight;  // [k] or null
    float eps;
};

// SSM_CONV (kernels/ssm-conv.cu): dst[s][t][r] = act(sum_j x[s][r][t + j] * w[r][j] (+ bias[r]))
struct SsmConvArgs {
    const float *x;          // conv_x: row (s, r) at x + s*x_nb2 + r*x_nb1 bytes, nc - 1 + n_t floats
    int64_t x_nb1, x_nb2;
    const void *w;           // taps: row r at w + r*w_nb1 bytes, nc values (F32 or F16)
    int64_t w_nb1;
    int32_t w_f16;
    const float *bias;       // [nr] or null (only with silu)
    int32_t silu;
    float *dst;              // element (s, t, r) at dst + s*dst_nb2 + t*dst_nb1 + 4r bytes
    int64_t dst_nb1, dst_nb2;
    int32_t nc;              // taps (d_conv)
    int32_t nr;              // channels (d_inner)
    int32_t n_t;             // tokens per sequence
    int32_t n_s;             // sequences
};

// Canonical order of the RMS sum of a row of k values (k % 256 == 0), shared by
// the combine kernel and the CPU oracle: chunk j holds values [256j, 256j+256);
// lane l of a 64-lane group accumulates v = x[256j + 4l + i] for i = 0..3 as
// a = fmaf(v, v, a) starting from 0; the 64 lane sums are tree-added (lane l +=
// lane l+off, off = 32, 16, ..., 1); chunk sums are added in ascending j starting
// from 0; s = 1 / sqrtf(sum/k + eps).
constexpr int RMS_CHUNK = 256;

// ---------------------------------------------------------------------------
// prefill-shaped MUL_MAT_ID (mc_mmq.hip)
// ---------------------------------------------------------------------------

constexpr int MMQ_COLS = 16;              // (token, slot) pairs per column block: the MFMA M dimension
constexpr int MMQ_WAVES = 4;              // waves per GEMM workgroup, 16 weight rows each
constexpr int MMQ_WAVES_PLAIN = 8;        // ... without a fused gate and one column block per pass
// Waves per grouped-GEMM workgroup.  A plain projection's workgroup that takes one
// column block per pass (down at prefill: K = 768, three super-blocks) takes 128 rows, so
// each expert's activation records are staged for half as many workgroups; with four
// column blocks per pass the 8-wave form needs more than 256 VGPRs (Q3_K, Q6_K).
constexpr int mmq_waves(bool gate, int maxb) { return !gate && maxb == 1 ? MMQ_WAVES_PLAIN : MMQ_WAVES; }
// Column blocks multiplied per pass over an expert's weights: 1 when the experts
// average at most MMQ_FEW_PAIRS pairs (most need one block, and the smaller LDS
// stages let more workgroups keep weight DMA in flight), else up to 4 (fewer
// passes over the weights when experts see many tokens).
constexpr int MMQ_MAX_BLOCKS = 4;
constexpr int MMQ_FEW_PAIRS = 12;
constexpr int MMQ_MAX_EXPERTS = 4096;
constexpr int MMQ_REC_BYTES = 4416;       // activation record of one (super-block, column block)

struct MmqArgs {
    const uint8_t *w;             // expert weights (device), expert e at w + e * expert_bytes
    const uint8_t *w_gate;        // gate weights of the same shape, or null (then no GLU)
    uint64_t expert_bytes;
    const uint8_t *y;             // q8_K activation rows
    int64_t stride_col_y;         // bytes between tokens
    int64_t stride_channel_y;     // bytes between channels
    int32_t nchannels_y;
    const int32_t *ids;           // [n_tok][ids_stride]
    int64_t ids_stride;
    float *dst;                   // dst[t * stride_col_dst + c * stride_channel_dst + row]
    int64_t stride_col_dst;
    int64_t stride_channel_dst;
    int32_t ncols;                // K (multiple of 256)
    int32_t nrows;                // rows per expert
    int32_t n_experts;
    int32_t n_used;
    int32_t n_tok;
    int32_t glu_op;
    float glu_limit;
    int32_t max_blocks;           // capacity of the column-block table
    uint8_t *ws;                  // workspace base and the byte offsets of its sections
    uint64_t ws_offsets, ws_blk_off, ws_list, ws_blk_tab, ws_packed, ws_total;
};

// Workspace sections for n_experts experts, n_pairs pairs and K values per row.
inline void mmq_layout(MmqArgs &a, int64_t n_pairs) {
    const auto up = [](uint64_t b) { return (b + 255u) & ~(uint64_t) 255u; };
    a.max_blocks = (int32_t) (a.n_experts + (n_pairs + MMQ_COLS - 1) / MMQ_COLS);
    uint64_t o = 0;
    a.ws_offsets = o; o = up(o + 4u * (uint64_t) (a.n_experts + 1));
    a.ws_blk_off = o; o = up(o + 4u * (uint64_t) (a.n_experts + 1));
    a.ws_list = o; o = up(o + 4u * (uint64_t) n_pairs);
    a.ws_blk_tab = o; o = up(o + 16u * (uint64_t) a.max_blocks);
    a.ws_packed = o; o = up(o + (uint64_t) MMQ_REC_BYTES * (uint64_t) a.max_blocks * (uint64_t) (a.ncols / 256));
    a.ws_total = o + 1024u;       // slack for the last DMA round
}

}  // namespace mc

#endif
