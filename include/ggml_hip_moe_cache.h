/*
 * ggml_hip_moe_cache.h -- C ABI of the MI355X (gfx950) pointer-table quantized
 * MoE expert GEMV and its hot-expert HBM cache.
 *
 * Drop-in boundary for ggml's HIP backend.  Every entry point below replaces
 * one function of the reference's kernels/moe-cache.cuh (cited per function).
 * The ABI is plain C: tensors are described by POD mirrors of the ggml fields
 * the path consumes, streams are passed as `void *` holding a hipStream_t, and
 * every function returns a status instead of aborting (the reference aborts
 * through CUDA_CHECK / GGML_ABORT: kernels/moe-cache.cu:475-480, 864).
 *
 * Status codes: 0 = success, < 0 = error (GGML_HIP_MOE_E_*, text in
 * ggml_hip_moe_last_error()).  Boolean predicates return 1 / 0.
 *
 * Ownership (kernels/moe-cache.cu:568-581): the library owns the pool, the
 * pointer tables, the stamp arrays and the global stats/clock it allocates;
 * the caller owns weights, host expert memory, activations, ids and outputs.
 * Host expert memory must outlive the library's use of it.
 *
 * Threading: registry and step work is serialized by one mutex
 * (kernels/moe-cache.cu:321, 526, 674); ggml_hip_moe_cache_wants() may be
 * called concurrently (kernels/moe-cache.cu:425-440).  All device work of one
 * call is ordered on the caller's stream.  Kernel arguments never change
 * between steps (the LRU clock is read from device memory), so a captured
 * hipGraph stays valid; ggml_hip_moe_cache_step() must run outside capture.
 */
#ifndef GGML_HIP_MOE_CACHE_H
#define GGML_HIP_MOE_CACHE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes of the functions below. */
enum {
    GGML_HIP_MOE_OK            = 0,
    GGML_HIP_MOE_E_INVALID     = -1,  /* bad argument, shape or stride */
    GGML_HIP_MOE_E_UNSUPPORTED = -2,  /* valid ggml, but a type / shape / fusion this path does not run */
    GGML_HIP_MOE_E_DEVICE      = -3,  /* a HIP runtime call failed */
    GGML_HIP_MOE_E_DISABLED    = -4,  /* the cache path was asked for while the cache is off */
    GGML_HIP_MOE_E_STATE       = -5,  /* wrong state (e.g. src0 not wanted, configure after registration) */
    GGML_HIP_MOE_E_TIMEOUT     = -6   /* a bounded in-kernel wait gave up (ggml_hip_moe_check_status) */
};

/* ggml_type values used by the path (ggml.h numbering) */
enum {
    GGML_HIP_MOE_TYPE_F32  = 0,
    GGML_HIP_MOE_TYPE_Q4_0 = 2,
    GGML_HIP_MOE_TYPE_Q5_0 = 6,
    GGML_HIP_MOE_TYPE_Q8_0 = 8,
    GGML_HIP_MOE_TYPE_Q8_1 = 9,
    GGML_HIP_MOE_TYPE_Q2_K = 10,
    GGML_HIP_MOE_TYPE_Q3_K = 11,
    GGML_HIP_MOE_TYPE_Q4_K = 12,
    GGML_HIP_MOE_TYPE_Q5_K = 13,
    GGML_HIP_MOE_TYPE_Q6_K = 14,
    GGML_HIP_MOE_TYPE_Q8_K = 15
};

/* ggml_glu_op values, plus the clamped SwiGLU the reference's epilogue names
 * (kernels/moe-cache.cu:264-280). */
enum {
    GGML_HIP_MOE_GLU_REGLU        = 0,
    GGML_HIP_MOE_GLU_GEGLU        = 1,
    GGML_HIP_MOE_GLU_SWIGLU       = 2,
    GGML_HIP_MOE_GLU_SWIGLU_OAI   = 3,
    GGML_HIP_MOE_GLU_GEGLU_ERF    = 4,
    GGML_HIP_MOE_GLU_GEGLU_QUICK  = 5,
    GGML_HIP_MOE_GLU_SWIGLU_CLAMP = 6
};

/* Activation formats accepted by the GEMV (src1 after quantization). */
enum {
    GGML_HIP_MOE_ACT_Q8_1 = 0, /* ggml-CUDA q8_1 blocks (36 B / 32 values): the reference's src1_q8_1 */
    GGML_HIP_MOE_ACT_Q8_K = 1, /* ggml-CPU q8_K blocks (292 B / 256 values), K-quant weights only */
    GGML_HIP_MOE_ACT_F32  = 2, /* fp32 rows, quantized to q8_1 inside the GEMV with the codes and
                                  scales ggml_hip_quantize_q8_1 produces (fuses that launch away) */
    GGML_HIP_MOE_ACT_SHARED_F32 = 0x100, /* ggml_hip_moe_ffn_down_combine flag: the shared
                                            expert's rows are fp32 (quantized in the launch) */
    GGML_HIP_MOE_ACT_DOT_Q8_K = 0x200    /* ggml_hip_moe_ffn_down_combine flag (with F32 rows):
                                            the rows are quantized to q8_K, as ggml-CPU's
                                            MUL_MAT_ID does for K-quant experts */
};

/* POD mirror of the ggml_tensor fields the path reads
 * (kernels/moe-cache.cu:87, 442-469, 525-541): type, ne, nb, data, name,
 * buffer (!= NULL) and view_src (!= NULL). */
typedef struct ggml_hip_moe_tensor {
    int32_t     type;
    int64_t     ne[4];
    uint64_t    nb[4];
    void       *data;
    const char *name;
    int32_t     has_buffer;
    int32_t     is_view;
} ggml_hip_moe_tensor;

/* Mirror of ggml_cuda_mm_fusion_args_device as the reference reads it
 * (kernels/moe-cache.cu:103-129), plus explicit fields for what the reference
 * leaves implicit. */
typedef struct ggml_hip_moe_fusion {
    const void  *gate;              /* device gate expert tensor (same type/shape as src0) when it has no table */
    const float *x_bias;            /* [n_experts][bias_stride] added to the up/plain output */
    const float *gate_bias;         /* [n_experts][bias_stride] added to the gate output */
    const float *x_scale;           /* [n_experts] multiplies the up/plain output (before bias) */
    const float *gate_scale;        /* [n_experts] multiplies the gate output (before bias) */
    int32_t      glu_op;            /* GGML_HIP_MOE_GLU_*; used when a gate is present (SWIGLU when fusion is NULL) */
    float        glu_limit;         /* SWIGLU_CLAMP limit */
    const void  *shared_up;         /* dense shared expert [ne01 x ne00], device memory */
    const void  *shared_gate;       /* dense shared gate, device memory, or NULL */
    float       *shared_dst;        /* shared expert output; token t at shared_dst + t*shared_stride_col_dst */
    int64_t      shared_stride_col_dst;
    /* -- extensions -- */
    int32_t      shared_type;       /* ggml_type of shared_up/shared_gate; < 0: same as src0 */
    const void  *shared_src1;       /* activation rows of the shared expert; NULL: channel 0 of src1 */
    int64_t      shared_stride_col_y; /* activation blocks between tokens of shared_src1 */
    int64_t      bias_stride;       /* floats per expert in x_bias/gate_bias; 0: stride_channel_dst */
} ggml_hip_moe_fusion;

/* ---------------------------------------------------------------------
 * Reference API (kernels/moe-cache.cuh:15-40)
 * --------------------------------------------------------------------- */

/* replaces ggml_cuda_moe_cache_enabled (kernels/moe-cache.cuh:15, moe-cache.cu:345-363):
 * GGML_HIP_MOE_CACHE (or GGML_CUDA_MOE_CACHE) set and not "0". */
int ggml_hip_moe_cache_enabled(void);

/* replaces ggml_cuda_moe_cache_wants (kernels/moe-cache.cuh:18, moe-cache.cu:442-469):
 * enabled, host-resident GPU-readable memory, supported type, ne[2] >= 2,
 * ne[3] == 1, not a view, contiguous. */
int ggml_hip_moe_cache_wants(const ggml_hip_moe_tensor *src0);

/* replaces ggml_cuda_moe_cache_mul_mat_vec_q (kernels/moe-cache.cuh:21-31, moe-cache.cu:821-868).
 * Registers src0 (and a host-resident gate) on first use, then runs the
 * pointer-table GEMV on `stream`.  Argument meaning follows the reference:
 * s01 is the weight row stride in blocks, stride_col_y / stride_channel_y are
 * in activation blocks (q8_1: 32 values), stride_col_dst / stride_channel_dst
 * in floats, ids_stride in int32 elements.  gate_host is the host-side fused
 * gate tensor (ggml_cuda_mm_fusion_args_host::gate) or NULL; fusion may be NULL. */
int ggml_hip_moe_cache_mul_mat_vec_q(
        const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *gate_host,
        const ggml_hip_moe_fusion *fusion,
        const void *src1_q8_1, const int32_t *ids_d, float *dst_d,
        int64_t ne00, int64_t ne01, int64_t ne02, int64_t ne03,
        int64_t ncols_dst, int64_t s01, int64_t s02, int64_t s03,
        int64_t nchannels_y, int64_t nchannels_dst,
        int64_t stride_col_y, int64_t stride_col_dst,
        int64_t stride_channel_y, int64_t stride_channel_dst,
        int64_t ids_stride, void *stream);

/* replaces ggml_cuda_moe_cache_step (kernels/moe-cache.cuh:34, moe-cache.cu:669-775):
 * miss-log readback, clock advance, 2nd-sighting admission, LRU eviction,
 * pool copies and batched table flush.  Call between graph launches. */
int ggml_hip_moe_cache_step(void *stream);

/* replaces ggml_cuda_moe_cache_active (kernels/moe-cache.cuh:37, moe-cache.cu:365-368) */
int ggml_hip_moe_cache_active(void);

/* replaces ggml_cuda_moe_cache_pin_host (kernels/moe-cache.cuh:40, moe-cache.cu:372-405):
 * 1 when t->data is (now) GPU-readable host memory.  Memory that is not yet
 * registered is registered only when GGML_HIP_MOE_CACHE_ALLOW_REGISTER=1;
 * memory from hipHostMalloc is recognized without registration. */
int ggml_hip_moe_cache_pin_host(const ggml_hip_moe_tensor *t);

/* ---------------------------------------------------------------------
 * Companion entry points of the same path
 * --------------------------------------------------------------------- */

/* The same GEMV for experts that already live in device memory (no table
 * registration, no stats): the upstream mul_mat_vec_q MoE call that the
 * reference's intercept falls through to (patches/apply_patches.py:48-62). */
int ggml_hip_mul_mat_vec_q_moe(
        const ggml_hip_moe_tensor *src0, const ggml_hip_moe_fusion *fusion,
        const void *src1_q8_1, const int32_t *ids_d, float *dst_d,
        int64_t ne00, int64_t ne01, int64_t ne02, int64_t ne03,
        int64_t ncols_dst, int64_t s01, int64_t s02, int64_t s03,
        int64_t nchannels_y, int64_t nchannels_dst,
        int64_t stride_col_y, int64_t stride_col_dst,
        int64_t stride_channel_y, int64_t stride_channel_dst,
        int64_t ids_stride, void *stream);

/* Both GEMV entry points with an explicit activation format
 * (GGML_HIP_MOE_ACT_*).  use_cache = 1 takes the cache path (src0 must satisfy
 * ggml_hip_moe_cache_wants), 0 the device-resident path.  With
 * GGML_HIP_MOE_ACT_Q8_K the activation strides count q8_K blocks (256 values), with
 * GGML_HIP_MOE_ACT_F32 they count floats (src1 and shared_src1 are fp32 rows). */
int ggml_hip_moe_mul_mat_vec_ex(
        int use_cache, int act_format,
        const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *gate_host,
        const ggml_hip_moe_fusion *fusion,
        const void *src1, const int32_t *ids_d, float *dst_d,
        int64_t ne00, int64_t ne01, int64_t ne02,
        int64_t ncols_dst, int64_t nchannels_y, int64_t nchannels_dst,
        int64_t stride_col_y, int64_t stride_col_dst,
        int64_t stride_channel_y, int64_t stride_channel_dst,
        int64_t ids_stride, void *stream);

/* q8_1 activation quantizer with ggml-CUDA quantize_q8_1 semantics (the
 * producer of src1_q8_1, patches/apply_patches.py:52): nrows rows of k fp32
 * values (x row stride x_stride floats) -> nrows rows of k/32 q8_1 blocks
 * (y row stride y_stride blocks).  k % 32 == 0. */
int ggml_hip_quantize_q8_1(const float *x, void *y, int64_t k, int64_t nrows,
                           int64_t x_stride, int64_t y_stride, void *stream);

/* ggml-CPU activation quantizers on the GPU: q8_K (quantize_row_q8_K_ref,
 * patches/trace-hook/ggml-cpu.c:308-340 vec_dot_type) into q8_K blocks, and
 * q8_0 (quantize_row_q8_0_ref, :249-274) written in q8_1 layout (s = 0). */
int ggml_hip_quantize_q8_K(const float *x, void *y, int64_t k, int64_t nrows,
                           int64_t x_stride, int64_t y_stride, void *stream);
int ggml_hip_quantize_q8_0_as_q8_1(const float *x, void *y, int64_t k, int64_t nrows,
                                   int64_t x_stride, int64_t y_stride, void *stream);

/* The MoE output combine that follows MUL_MAT_ID in a ggml graph (MUL by the
 * router weights, ADD of the shared expert and of the residual), fused with the
 * RMSNorm (RMS_NORM, then MUL by the norm weight) in front of the next MoE block
 * and the q8_1 quantization of its result for the next GEMV:
 *   x[t] = residual[t] + shared[t] + sum_{j < n_used} w[t][j] * o[t][j]   (j ascending, fused multiply-add)
 *   v[t] = rms_norm ? (x[t] * (1/sqrt(mean(x[t]^2) + eps))) * norm_weight : x[t]   (norm_weight optional)
 *   y[t] = q8_1(v[t])
 * The mean of squares is summed in a fixed order (256-value chunks, see mc_internal.h), so results are
 * deterministic.  o: [n_tok][n_used][o_stride] floats (n_used <= 16); w: [n_tok][n_used]; shared:
 * [n_tok][shared_stride] or NULL; residual: [n_tok][k] or NULL; x_out: [n_tok][k] or NULL; y_q8_1: n_tok
 * rows, y_stride blocks apart; norm_weight: [k] or NULL; k % 256 == 0, k <= 8192; fp32 pointers
 * 16-byte aligned, o_stride and shared_stride multiples of 4.  No reference counterpart (ggml runs
 * these as separate ops). */
int ggml_hip_moe_combine_q8_1(const float *o, int64_t o_stride, const float *w, int32_t n_used,
                              const float *shared, int64_t shared_stride, const float *residual,
                              float *x_out, void *y_q8_1, int64_t y_stride, int64_t k, int64_t n_tok,
                              int32_t rms_norm, const float *norm_weight, float eps, void *stream);

/* ---------------------------------------------------------------------
 * Fused decode FFN block: two launches per MoE block instead of four.
 * No reference counterpart: ggml runs RMS_NORM, MUL, quantize_q8_1,
 * MUL_MAT_ID, the router-weight MUL and the ADDs as separate ops; these
 * produce bit-identical results to ggml_hip_moe_combine_q8_1 followed by the
 * MUL_MAT_ID GEMVs above (same steps, same arithmetic order).  K-quant
 * experts (Q2_K..Q6_K) and K-quant (or no) shared experts.
 * --------------------------------------------------------------------- */

/* Gate/up MUL_MAT_ID (ggml_hip_moe_mul_mat_vec_ex arguments: src0 = up, gate via
 * gate_host / fusion->gate, GLU, bias, scale, shared expert) whose activation is
 * computed in the same launch from the fp32 residual rows x:
 *   y[t] = q8_1((x[t] * (1/sqrt(mean(x[t]^2) + eps))) * norm_weight)   (norm_weight may be NULL)
 * with the mean of squares in the canonical order of ggml_hip_moe_combine_q8_1.
 * Every pick and the shared expert (fusion->shared_src1 must be NULL) read y[t].
 * x: [ncols_dst][stride_col_x] floats, 16-byte aligned rows; ne00 % 256 == 0, ne00 <= 8192.
 * y_out (optional): receives y, rows y_out_stride q8_1 blocks apart.
 * dst_q8_1 / shared_dst_q8_1 (optional): the q8_1 quantization of the outputs (the down
 * projection's input, as ggml_hip_quantize_q8_1 of dst would give), pick c of token t at
 * dst_q8_1 + (t*q8_stride_col + c*q8_stride_channel) q8_1 blocks, the shared expert's at
 * shared_dst_q8_1 + t*shared_q8_stride_col blocks; needs ne01 % 32 == 0 and at most 16 units
 * per row (ne00 <= 4096).  With dst_q8_1 but no shared_dst_q8_1 the shared expert's rows are
 * only written in fp32 (fusion->shared_dst); the launch then splits the shared matrix into
 * workgroups of about a routed workgroup's bytes, and the down projection quantizes that
 * row itself (GGML_HIP_MOE_ACT_SHARED_F32). */
int ggml_hip_moe_ffn_gate_up_norm(
        int use_cache, const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *gate_host,
        const ggml_hip_moe_fusion *fusion, const float *x, const float *norm_weight, float eps,
        const int32_t *ids_d, float *dst_d, int64_t ne00, int64_t ne01, int64_t ne02,
        int64_t ncols_dst, int64_t nchannels_dst, int64_t stride_col_x, int64_t stride_col_dst,
        int64_t stride_channel_dst, int64_t ids_stride, void *y_out, int64_t y_out_stride,
        void *dst_q8_1, int64_t q8_stride_col, int64_t q8_stride_channel,
        void *shared_dst_q8_1, int64_t shared_q8_stride_col, void *stream);

/* ggml_hip_moe_ffn_gate_up_norm with the normalized row in act_format:
 * GGML_HIP_MOE_ACT_Q8_1 (as above), or GGML_HIP_MOE_ACT_Q8_K: y[t] is quantized to q8_K
 * blocks (ggml-CPU's quantize_row_q8_K_ref on the same fp32 values) and every dot runs on
 * them, as ggml-CPU's MUL_MAT_ID does for K-quant experts; y_out then receives q8_K rows
 * (y_out_stride in 292-byte blocks) and dst_q8_1 / shared_dst_q8_1 must be NULL (the down
 * launch quantizes the fp32 outputs itself: GGML_HIP_MOE_ACT_F32 | GGML_HIP_MOE_ACT_DOT_Q8_K). */
int ggml_hip_moe_ffn_gate_up_norm_ex(
        int use_cache, int act_format, const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *gate_host,
        const ggml_hip_moe_fusion *fusion, const float *x, const float *norm_weight, float eps,
        const int32_t *ids_d, float *dst_d, int64_t ne00, int64_t ne01, int64_t ne02,
        int64_t ncols_dst, int64_t nchannels_dst, int64_t stride_col_x, int64_t stride_col_dst,
        int64_t stride_channel_dst, int64_t ids_stride, void *y_out, int64_t y_out_stride,
        void *dst_q8_1, int64_t q8_stride_col, int64_t q8_stride_channel,
        void *shared_dst_q8_1, int64_t shared_q8_stride_col, void *stream);

/* Down MUL_MAT_ID over the n_used = nchannels_dst picks of each token (pick c reads
 * activation row src1 + t*stride_col_y + c*stride_channel_y, q8_1 blocks or floats
 * per act_format), plus fusion->shared_up on fusion->shared_src1, combined in the
 * same launch:
 *   x_out[t] = residual[t] + shared[t] + sum_{c < n_used} router_w[t][c] * o_c[t]   (c ascending, fused multiply-add)
 * residual may be NULL or equal to x_out; router_w: [ncols_dst][n_used]; x rows
 * stride_col_x floats apart; n_used (+1 with a shared expert) <= 12.  x_bias / x_scale
 * fusion apply to the routed picks; an out-of-range expert id contributes 0.
 * act_format | GGML_HIP_MOE_ACT_SHARED_F32: fusion->shared_src1 holds fp32 rows
 * (fusion->shared_stride_col_y floats apart, 16-byte aligned) beside q8_1 routed rows; the
 * shared wave quantizes its row with the q8_1 quantizer's arithmetic (same results as
 * passing that row's ggml_hip_quantize_q8_1). */
int ggml_hip_moe_ffn_down_combine(
        int use_cache, int act_format, const ggml_hip_moe_tensor *src0, const ggml_hip_moe_fusion *fusion,
        const void *src1, const int32_t *ids_d, const float *router_w, const float *residual, float *x_out,
        int64_t ne00, int64_t ne01, int64_t ne02, int64_t ncols_dst, int64_t nchannels_dst,
        int64_t stride_col_y, int64_t stride_channel_y, int64_t stride_col_x, int64_t ids_stride, void *stream);


/* ---------------------------------------------------------------------
 * Prefill-shaped MUL_MAT_ID (many tokens).  The reference routes only batch-1
 * decode to its pointer-table GEMV and leaves many-token MUL_MAT_ID to
 * upstream ggml's MMQ path (results/final.patch:45-48); this is its gfx950
 * counterpart: the (token, slot) pairs are grouped by expert and multiplied
 * with int8 MFMA.
 * --------------------------------------------------------------------- */

/* Bytes of device workspace ggml_hip_moe_mul_mat_q needs for ne00 columns, ne02
 * experts and n_pairs = tokens * slots (no initialisation required). */
int64_t ggml_hip_moe_mul_mat_q_workspace_bytes(int64_t ne00, int64_t ne02, int64_t n_pairs);

/* MUL_MAT_ID over device-resident K-quant experts (Q2_K..Q6_K) with q8_K
 * activations (ggml_hip_quantize_q8_K; the ggml-CPU vec_dot_type of these types):
 *   dst[t*stride_col_dst + c*stride_channel_dst + r] = W[ids[c + t*ids_stride]][r] . y(t, c)
 * with y(t, c) the q8_K row (c % nchannels_y)*stride_channel_y + t*stride_col_y (strides in
 * q8_K blocks of 256 values).  fusion may carry gate (same shape, device) with glu_op/glu_limit:
 * dst = GLU(gate . y, W . y); other fusion fields are not supported here.  Expert ids outside
 * [0, ne02) are skipped.  src1 and workspace 256-byte aligned, weights 16-byte aligned
 * (Q2_K: 4-byte, Q3_K/Q6_K: 2-byte, a gate at the up matrix's address mod 4). */
int ggml_hip_moe_mul_mat_q(const ggml_hip_moe_tensor *src0, const ggml_hip_moe_fusion *fusion,
                           const void *src1_q8_K, const int32_t *ids_d, float *dst_d,
                           int64_t ne00, int64_t ne01, int64_t ne02,
                           int64_t ncols_dst, int64_t nchannels_y, int64_t nchannels_dst,
                           int64_t stride_col_y, int64_t stride_col_dst,
                           int64_t stride_channel_y, int64_t stride_channel_dst,
                           int64_t ids_stride, void *workspace, int64_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------
 * Configuration, introspection and teardown (the reference reads env vars
 * once and never frees; kernels/moe-cache.cu:315-363)
 * --------------------------------------------------------------------- */

typedef struct ggml_hip_moe_config {
    int32_t     enabled;        /* 1 / 0 */
    int32_t     slots;          /* pool slots per expert tensor; < 0: every expert */
    double      budget_gb;      /* total pool budget in GiB; <= 0: free HBM minus margin */
    double      margin_gb;      /* HBM kept free at registration (reference: 2 GiB) */
    const char *seed_path;      /* seed file; NULL or "": none */
    int32_t     max_promotions; /* per step (reference: 48) */
    int32_t     verbose;        /* registration / step lines on stderr */
    int32_t     async_promotions; /* 1: ggml_hip_moe_cache_step issues the promotion copies on a
                                   * second stream of its own (env GGML_HIP_MOE_CACHE_ASYNC=1): the
                                   * next token no longer waits for them, results are unchanged,
                                   * and which of its reads hit the pool depends on timing.
                                   * 0 (default): the reference's order on the caller's stream. */
} ggml_hip_moe_config;

/* Replaces the env-derived settings; must be called before the first registration. */
int ggml_hip_moe_cache_configure(const ggml_hip_moe_config *cfg);
/* Current settings (after env parsing). */
int ggml_hip_moe_cache_get_config(ggml_hip_moe_config *out);

typedef struct ggml_hip_moe_entry_info {
    int32_t  id;             /* cache id (registration order) */
    int32_t  type;
    int32_t  n_experts;
    int32_t  n_slots;
    uint64_t expert_bytes;
    int32_t  n_resident;     /* occupied slots */
    uint32_t stamps_clock;
} ggml_hip_moe_entry_info;

/* Number of registered tensors. */
int ggml_hip_moe_cache_num_entries(void);
/* Info of entry `id`. */
int ggml_hip_moe_cache_entry_info(int32_t id, ggml_hip_moe_entry_info *out);
/* slot_of[n_experts] (-1 = cold) and expert_of[n_slots] (-1 = free) of entry `id`. */
int ggml_hip_moe_cache_entry_slots(int32_t id, int32_t *slot_of, int32_t n_experts, int32_t *expert_of, int32_t n_slots);
/* Host mirror of the pointer table of entry `id`, decoded: for expert e,
 * out[e] = slot (>= 0, LSB=0 entry into the pool) or -1 (LSB=1 entry to host memory). */
int ggml_hip_moe_cache_entry_table(int32_t id, int32_t *out, int32_t n_experts);
/* Raw device table / stamp array addresses of entry `id` (for device-side checks). */
int ggml_hip_moe_cache_entry_device(int32_t id, void **d_tbl, void **d_stamps, void **pool);
/* Device addresses of the global stats words and the LRU clock. */
int ggml_hip_moe_cache_device_globals(void **d_stats, void **d_clock);
/* Copies the first n_words device stats words ([0] misses, [1] hits, [2..] miss
 * log) to out, ordered after all work on `stream`, and waits for the copy. */
int ggml_hip_moe_cache_stats_snapshot(uint32_t *out, int32_t n_words, void *stream);
/* Copies entry `id`'s device stamp array (n >= n_experts) to out, as above. */
int ggml_hip_moe_cache_stamps_snapshot(int32_t id, uint32_t *out, int32_t n, void *stream);

typedef struct ggml_hip_moe_totals {
    uint64_t steps, hits, misses, promotions, evictions;
    uint32_t clock;
    uint32_t last_step_misses, last_step_hits;
    uint32_t admission_size;
} ggml_hip_moe_totals;
int ggml_hip_moe_cache_totals(ggml_hip_moe_totals *out);

/* Frees every pool/table/stat allocation and forgets all registrations
 * (the reference has no teardown). */
int ggml_hip_moe_cache_reset(void);

/* ---------------------------------------------------------------------
 * MUL_MAT_ID at the ggml op level: the caller side of the reference's
 * intercept (patches/apply_patches.py:42-62 / results/final.patch:66-82, where
 * ggml-cuda has already derived the strides and quantized src1), as one call
 * that takes the op's tensors.
 *
 *   src0  expert weights [K, R, E] (any supported type; host-resident tensors
 *         take the pointer-table cache path when ggml_hip_moe_cache_wants(src0))
 *   src1  fp32 activations [K, channels, tokens] (channels 1: every slot reads
 *         the token's row; n_used: one row per slot), rows contiguous
 *   ids   int32 [n_used, tokens], any row stride (a top-k view)
 *   dst   fp32 [R, n_used, tokens], any row strides
 *
 * Strides are derived from ne/nb as ggml-cuda does (ids_stride = ids->nb[1]/4,
 * stride_channel_dst = dst->nb[1]/4, stride_col_dst = dst->nb[2]/4); src1 is
 * quantized into `workspace` (q8_1 rows for the GEMV, q8_K rows for the grouped
 * GEMM) and the op runs on `stream`:
 *   - the pointer-table cache GEMV when the cache wants src0;
 *   - the expert-grouped int8-MFMA GEMM (ggml_hip_moe_mul_mat_q) for K-quant
 *     experts with more than 8 tokens (ggml-cuda's MMVQ batch limit) when the
 *     fusion is at most gate + GLU and the weights are aligned for it;
 *   - the device-resident GEMV otherwise.
 * gate_host / fusion as in ggml_hip_moe_cache_mul_mat_vec_q.  The workspace (256-
 * byte aligned) must hold ggml_hip_moe_mul_mat_id_workspace_bytes(...) bytes
 * (-1: the tensors are not a supported MUL_MAT_ID).
 * --------------------------------------------------------------------- */
int64_t ggml_hip_moe_mul_mat_id_workspace_bytes(const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *src1,
                                                const ggml_hip_moe_tensor *ids, const ggml_hip_moe_fusion *fusion);
int ggml_hip_moe_mul_mat_id(const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *src1,
                            const ggml_hip_moe_tensor *ids, const ggml_hip_moe_tensor *dst,
                            const ggml_hip_moe_tensor *gate_host, const ggml_hip_moe_fusion *fusion,
                            void *workspace, int64_t workspace_bytes, void *stream);

/* ggml_hip_moe_mul_mat_id for callers that cannot allocate (code under graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): no
 * counterpart in the reference.  Same arguments and results as
 * ggml_hip_moe_mul_mat_id without gate_host and workspace: the workspace is a
 * library-held device array of 64 MiB per GPU (kept until the process ends), and
 * no call allocates.  Device-resident experts only (host-resident experts take
 * the cache path, whose registration allocates: GGML_HIP_MOE_E_UNSUPPORTED); a
 * call whose ggml_hip_moe_mul_mat_id_workspace_bytes exceeds 64 MiB returns
 * GGML_HIP_MOE_E_UNSUPPORTED.  Every call on one GPU uses the same array: calls
 * that overlap on one GPU (concurrent streams, or another thread) race; calls
 * ordered on one stream do not. */
int ggml_hip_moe_mul_mat_id_noalloc(const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *src1,
                                    const ggml_hip_moe_tensor *ids, const ggml_hip_moe_tensor *dst,
                                    const ggml_hip_moe_fusion *fusion, void *stream);

/* ---------------------------------------------------------------------
 * Graph-level fusion detection: the decision ggml-cuda's graph evaluator makes
 * before the reference's intercept (patches/apply_patches.py:42-62,
 * results/final.patch:66-82), producing the fusion arguments the intercept
 * consumes (kernels/moe-cache.cu:109-129).  The caller mirrors the nodes of a
 * MoE FFN block (ggml's op, sources and result tensor) into an array.
 * --------------------------------------------------------------------- */

enum {
    GGML_HIP_MOE_OP_MUL_MAT    = 1,   /* dst = src0 (weights) x src1 */
    GGML_HIP_MOE_OP_MUL_MAT_ID = 2,   /* src0 experts, src1 activations, src2 ids */
    GGML_HIP_MOE_OP_ADD_ID     = 3,   /* dst = src0 + src1[:, src2 (ids)] (per-expert bias rows) */
    GGML_HIP_MOE_OP_MUL        = 4,   /* dst = src0 * src1 */
    GGML_HIP_MOE_OP_ADD        = 5,   /* dst = src0 + src1 */
    GGML_HIP_MOE_OP_GLU        = 6,   /* dst = glu_op(src0, src1); swapped: the roles of src0 and src1 exchanged */
    GGML_HIP_MOE_OP_OTHER      = 7
};

/* One graph node: its op, its result tensor, and for each source either the index of
 * the producing node in the same array (src[k] >= 0) or a leaf tensor (src[k] < 0:
 * leaf[k], e.g. weights, biases, the ids, an input computed elsewhere).  A MUL by a
 * per-expert scale has a leaf src1 of ne [1, n_experts] and src2 = the ids (ggml's
 * get_rows of the scale by the ids, folded into the node). */
typedef struct ggml_hip_moe_node {
    int32_t             op;
    ggml_hip_moe_tensor t;
    int32_t             src[3];
    ggml_hip_moe_tensor leaf[3];
    int32_t             glu_op;       /* GLU: GGML_HIP_MOE_GLU_* */
    float               glu_limit;    /* GLU: SWIGLU_CLAMP limit */
    int32_t             glu_swapped;  /* GLU: 1 when src0 is the up (value) operand and src1 the gate */
} ggml_hip_moe_node;

/* For the MUL_MAT_ID node i_up, the largest fusable pattern around it:
 *   up path    MUL_MAT_ID(w_up, x, ids) [-> MUL(x_scale, ids)] [-> ADD_ID(x_bias, ids)]
 *   gate path  MUL_MAT_ID(w_gate, x, ids) [-> MUL(gate_scale, ids)] [-> ADD_ID(gate_bias, ids)]
 *   GLU(gate path, up path)
 *   shared     MUL_MAT(sh_up, x), MUL_MAT(sh_gate, x), GLU(sh_gate, sh_up) on the same x
 * Every absorbed intermediate must have the next node as its only consumer, the gate
 * MUL_MAT_ID must match the up one (type, shape, activations, ids), and the GLU ops must
 * agree.  Fills *fusion (glu_op, biases, scales, shared_* with shared_dst = the shared
 * GLU's tensor; gate = the gate's data when the cache does not want w_up) and
 * *gate_host (the gate weights, for the cache path; *has_gate_host = 0 when none),
 * sets covered[k] = 1 for every node the fused call computes (covered has n_nodes
 * entries) and *out_node to the node whose tensor receives the result.  Returns the
 * number of covered nodes (1: nothing fused, a plain MUL_MAT_ID), or < 0 when node
 * i_up is not a MUL_MAT_ID or the array is malformed. */
int ggml_hip_moe_fusion_detect(const ggml_hip_moe_node *nodes, int32_t n_nodes, int32_t i_up,
                               ggml_hip_moe_fusion *fusion, ggml_hip_moe_tensor *gate_host,
                               int32_t *has_gate_host, int32_t *covered, int32_t *out_node);

/* ---------------------------------------------------------------------
 * SSM_CONV with F32 or F16 conv weights (kernels/ssm-conv.cu:117-217: the
 * reference's ssm_conv_f32_cuda / ggml_cuda_op_ssm_conv, templated on the
 * weight type so that F16 conv1d weights work; the fused ADD(bias) + SiLU).
 *   dst[s][t][r] = act(sum_{j<nc} src0[s][r][t + j] * src1[r][j] (+ bias[r]))
 * src0 = conv_x (F32, rows of nc - 1 + n_t floats: byte strides src0_nb1 per
 * channel, src0_nb2 per sequence, src0_nb0 = 4); src1 = conv1d weight, type 0
 * (F32) or 1 (F16), src1_nb1 bytes per channel; dst F32 with dst_nb0 = 4,
 * dst_nb1 per token, dst_nb2 per sequence.  fuse_silu applies SiLU; bias (nr
 * floats) requires it (the reference asserts the same).  nc in {3, 4, 5, 9, 15}
 * as in the reference; nr need not be a multiple of 128 (the reference asserts
 * it).  Taps are summed in ascending order with fused multiply-adds from 0,
 * then the bias is added.
 * --------------------------------------------------------------------- */
int ggml_hip_ssm_conv_f32(const float *src0, int64_t src0_nb0, int64_t src0_nb1, int64_t src0_nb2,
                          const void *src1, int32_t src1_type, int64_t src1_nb1,
                          const float *bias, int32_t fuse_silu,
                          float *dst, int64_t dst_nb0, int64_t dst_nb1, int64_t dst_nb2,
                          int64_t nc, int64_t nr, int64_t n_t, int64_t n_s, void *stream);

/* ---------------------------------------------------------------------
 * Routing trace (patches/trace-hook/ggml-cpu.c:1-9, :1597-1617): one binary
 * record per MUL_MAT_ID, appended to a file, input of the seed builder
 * (a6000-custom-kernels_amd/seed.py, the restatement of tools/make_seed.py):
 *   u32 namelen, u32 n_used, u32 n_tok, u32 n_exp (little endian),
 *   char name[namelen] (the tensor name cut to 120 bytes, no terminator),
 *   i32 ids[n_used * n_tok] (token-major, ggml's ids layout).
 * ---------------------------------------------------------------------
 *
 * Appends one record to `path` (NULL: the file named by GGML_HIP_MOE_TRACE,
 * alias GGML_MOE_TRACE; no such variable: nothing is written and 0 is returned).
 * ids is host memory.  The file is opened in append mode on first use and kept
 * open, as the reference's hook does; records from concurrent callers are
 * serialised.  Returns 0 or a negative status (open/write failure, bad sizes). */
int ggml_hip_moe_trace_append(const char *path, const char *name, const int32_t *ids,
                              int64_t n_used, int64_t n_tok, int64_t n_exp);

/* Flushes and closes every trace file opened by ggml_hip_moe_trace_append. */
int ggml_hip_moe_trace_close(void);

/* Device-side errors of the launches on `stream` since the last call: waits for the
 * stream, then returns 0, or GGML_HIP_MOE_E_TIMEOUT when a fused gate/up launch
 * (ggml_hip_moe_ffn_gate_up_norm) had a bounded wait give up -- its workgroups then
 * skip their rows, so those launches' outputs are not valid -- and clears the
 * condition.  The word is per GPU (the current device).  No reference counterpart:
 * the reference's kernel has no in-kernel waits. */
int ggml_hip_moe_check_status(void *stream);

/* Debug: polls a bounded in-kernel wait makes before it gives up (n < 0: the default,
 * 2^22).  0 makes every such wait give up at once, which tests the timeout path with
 * every kernel still exiting normally.  Applies to launches issued after the call. */
int ggml_hip_moe_debug_set_spin_limit(int64_t n);

/* Text of the last error on this thread. */
const char *ggml_hip_moe_last_error(void);

/* Library version string. */
const char *ggml_hip_moe_version(void);

#ifdef __cplusplus
}
#endif
#endif /* GGML_HIP_MOE_CACHE_H */
