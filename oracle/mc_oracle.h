/*
 * mc_oracle.h -- CPU oracle for the pointer-table quantized MoE expert GEMV.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: it is linked or
 * loaded by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
 * leg, and by nothing else.  The product (the HIP library under
 * a6000-custom-kernels_amd/) never calls it.
 *
 * What it restates:
 *   - ggml block layouts Q4_0/Q5_0/Q8_0/Q2_K/Q3_K/Q4_K/Q5_K/Q6_K and their
 *     dequantizers (upstream ggml @11fe0215, not vendored by the reference;
 *     named by the reference at kernels/moe-cache.cu:44-70, 407-421);
 *   - the activation quantizers: q8_1 with ggml-CUDA semantics (the format of
 *     `src1_q8_1` handed to the GEMV, patches/apply_patches.py:52), q8_0 and
 *     q8_K with ggml-CPU reference semantics (vec_dot_type table,
 *     patches/trace-hook/ggml-cpu.c:249-340);
 *   - the per-type dot products against those activations;
 *   - ggml's CPU MUL_MAT_ID (patches/trace-hook/ggml-cpu.c:1492-1767) followed
 *     by the unfused post-ops the GPU fuses: per-expert scale, per-expert bias
 *     and the GLU against the gate projection, plus the shared expert
 *     (kernels/moe-cache.cu:103-107, 240-284).
 *
 * Pinning (how each part is checked without running the reference, which
 * cannot be built here): tests/test_oracle_formats.py and
 * tests/test_oracle_mmid.py -- hand-built known-answer blocks, closed-form
 * special cases, integer-sum identities, fp64 dequantized dot products and
 * brute force on tiny inputs.  The two GLU ops the reference calls without
 * defining (SWIGLU_OAI, SWIGLU_CLAMP) are checked against the gpt-oss and
 * DeepSeek-V4 model definitions of the transformers package
 * (tests/test_oracle_glu_models.py).  Parity unpinned: only what no function
 * here restates -- the rounding of upstream ggml-CUDA's own vec_dot_*_q8_1
 * kernels, which the GEMV does not follow bit for bit (it follows the CPU
 * integer-offset formulation restated here).
 */
#ifndef MC_ORACLE_H
#define MC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml_type numeric values (ggml.h) */
enum {
    OR_F32 = 0, OR_F16 = 1, OR_Q4_0 = 2, OR_Q5_0 = 6, OR_Q8_0 = 8, OR_Q8_1 = 9,
    OR_Q2_K = 10, OR_Q3_K = 11, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14, OR_Q8_K = 15
};

/* activation quantization semantics for the dot products */
enum {
    OR_ACT_CPU  = 0, /* ggml CPU vec_dot_type: q8_0 (34 B / 32) for Q4_0/Q5_0/Q8_0, q8_K (292 B / 256) for K-quants */
    OR_ACT_Q8_1 = 1, /* ggml-CUDA q8_1 (36 B / 32): half d, half s = sum(x), int8 qs[32] */
    OR_ACT_Q8_0_AS_Q8_1 = 2 /* q8_1 layout whose d/qs follow q8_0 CPU rounding (x * (1/d)); s is unused */
};

/* GLU ops (ggml_glu_op numbering, plus SWIGLU_CLAMP used by the reference's fused epilogue) */
enum {
    OR_GLU_REGLU = 0, OR_GLU_GEGLU = 1, OR_GLU_SWIGLU = 2, OR_GLU_SWIGLU_OAI = 3,
    OR_GLU_GEGLU_ERF = 4, OR_GLU_GEGLU_QUICK = 5, OR_GLU_SWIGLU_CLAMP = 6
};

uint16_t or_fp32_to_fp16(float f);
float    or_fp16_to_fp32(uint16_t h);

int     or_type_supported(int type);
int     or_block_elems(int type);
size_t  or_block_bytes(int type);
size_t  or_row_bytes(int type, int64_t k);

void or_dequantize_row(int type, const void *x, float *y, int64_t k);

/* Synthetic weight quantizer: produces valid blocks of `type` approximating x.
 * (The blocks are a shared input of the GPU path and of this oracle, so this
 * quantizer does not need to reproduce ggml's own quantizer.) */
void or_quantize_row_weights(int type, const float *x, void *y, int64_t k);

/* Activation quantizers */
void or_quantize_q8_1(const float *x, void *y, int64_t k);     /* CUDA quantize_q8_1 semantics */
void or_quantize_q8_0(const float *x, void *y, int64_t k);     /* quantize_row_q8_0_ref */
void or_quantize_q8_0_as_q8_1(const float *x, void *y, int64_t k);
void or_quantize_q8_K(const float *x, void *y, int64_t k);     /* quantize_row_q8_K_ref */

/* Activation row layout for (weight type, semantics) */
int    or_act_type(int wtype, int act_kind);          /* OR_Q8_0 / OR_Q8_K / OR_Q8_1 */
size_t or_act_row_bytes(int wtype, int act_kind, int64_t k);
void   or_quantize_act_row(int wtype, int act_kind, const float *x, void *y, int64_t k);

/* Dot of one weight row (k elements of `wtype`) with one activation row. */
float or_vec_dot(int wtype, int act_kind, int64_t k, const void *w, const void *a);
/* ggml-CPU vec_dot with q8_0 / q8_K activations: AVX2 for Q2_K and Q4_K (bit-identical
 * to or_vec_dot's scalar path) unless or_set_simd(0), scalar otherwise. */
float or_vec_dot_cpu(int wtype, int64_t k, const void *w, const void *a);
void or_set_simd(int on);

/* Exact integer partial sums of one block (for bit-exact checks):
 * out[j] for the block's sub-blocks, as documented in mc_oracle.c. */
int or_block_isums(int wtype, const void *wblock, const int8_t *q8, int32_t *out);

float or_glu(int op, float gate, float up, float limit);

/* ------------------------------------------------------------------------
 * MUL_MAT_ID (+ fused post-ops) over pre-quantized activation rows.
 * dst[t*dst_stride_col + c*dst_stride_channel + r] for token t, slot c, row r.
 * Activation row for (t, c): act + (c % nchannels_y)*act_stride_channel + t*act_stride_col (bytes).
 * ------------------------------------------------------------------------ */
typedef struct or_mmid_args {
    int      type;          /* routed weight type */
    int64_t  ne00, ne01;    /* K (columns), rows per expert */
    int32_t  n_as;          /* number of experts */
    size_t   nb01, nb02;    /* row bytes, expert bytes */
    const void *src0;       /* up (or plain) expert weights */
    const void *gate;       /* gate expert weights (same type/shape) or NULL */
    const float *x_bias, *gate_bias; int64_t bias_stride;   /* [n_as][bias_stride] floats */
    const float *x_scale, *gate_scale;                      /* [n_as] */
    int32_t  glu_op; float glu_limit;
    /* shared expert (dense, one matrix); sh_dst[t*sh_stride_col_dst + r] */
    int32_t  sh_type; const void *sh_up; const void *sh_gate; float *sh_dst; int64_t sh_stride_col_dst;
    const void *sh_act; size_t sh_act_stride_col;            /* NULL: channel-0 activation of each token */
    /* routing */
    const int32_t *ids; int32_t n_ids; int32_t n_tok; int64_t ids_stride;
    /* activations */
    int32_t  act_kind; const void *act; int64_t nchannels_y; size_t act_stride_col, act_stride_channel;
    /* output */
    float   *dst; int64_t dst_stride_col, dst_stride_channel;
    int32_t  nthreads;
} or_mmid_args;

int or_mul_mat_id(const or_mmid_args *a);

/* Plain per-expert MUL_MAT_ID restated from ggml_compute_forward_mul_mat_id:
 * quantize fp32 src1 to the CPU vec_dot_type, group (slot, token) pairs by
 * expert, per expert chunk rows over threads, vec_dot per row.  Output layout
 * as above.  Returns 0 on success. */
int or_cpu_mul_mat_id_f32(int type, int64_t ne00, int64_t ne01, int32_t n_as,
                          const void *src0, size_t nb01, size_t nb02,
                          const float *src1, int64_t ne11, int64_t src1_stride_row, int64_t src1_stride_tok,
                          const int32_t *ids, int32_t n_ids, int32_t n_tok, int64_t ids_stride,
                          float *dst, int64_t dst_stride_col, int64_t dst_stride_channel,
                          int32_t nthreads);

/* MoE output combine + RMSNorm + q8_1 quantization (the GPU's fused combine kernel):
 * x[t][i] = residual + shared + sum_j w[t][j]*o[t][j][i], accumulated left to right with fmaf (x_out required);
 * rms_norm: s = 1/sqrtf(or_rms_sum(x[t])/k + eps), v = (x*s)*norm_weight[i] (weight optional); else v = x;
 * y[t] = q8_1(v). */
void or_combine_q8_1(const float *o, int64_t o_stride, const float *w, int32_t n_used, const float *shared,
                     int64_t shared_stride, const float *residual, float *x_out, void *y, int64_t k, int64_t n_tok,
                     int32_t rms_norm, const float *norm_weight, float eps);
/* Sum of squares of k values (k % 256 == 0) in the GPU kernels' fixed order (mc_oracle.c). */
float or_rms_sum(const float *x, int64_t k);

/* SSM_CONV (kernels/ssm-conv.cu:5-57, ssm_conv_f32): for each sequence s, channel r and
 * token t, sumf = 0; sumf = fmaf(x[s][r][t + j], w[r][j], sumf) for j = 0..nc-1 (the CUDA
 * build contracts `sumf += x*w` into fused multiply-adds); with silu: sumf += bias[r] (when
 * given), then sumf / (1 + expf(-sumf)).  x rows hold nc - 1 + n_t floats (x_row floats
 * apart, x_seq floats per sequence); w is F32 (w_f16 = 0) or F16 bits, w_row elements per
 * channel; dst[s][t][r] at s*dst_seq + t*dst_tok + r floats. */
void or_ssm_conv_f32(const float *x, int64_t x_row, int64_t x_seq, const void *w, int w_f16, int64_t w_row,
                     const float *bias, int silu, float *dst, int64_t dst_tok, int64_t dst_seq,
                     int64_t nc, int64_t nr, int64_t n_t, int64_t n_s);

/* Deterministic generator used by the synthetic workloads (splitmix64 + Box-Muller). */
uint64_t or_splitmix64(uint64_t *state);
void or_fill_normal(uint64_t seed, float mean, float std, float *out, int64_t n);
void or_topk_uniform(uint64_t seed, int32_t n_experts, int32_t k, int32_t n_tok, int32_t *ids);

int or_omp_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
