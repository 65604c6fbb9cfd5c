// mc_kernels.hip -- gfx950 kernels of the pointer-table quantized MoE GEMV.
//
// Replaces the CUDA kernel moe_cache_gemv (kernels/moe-cache.cu:76-291) and
// the upstream quantize_q8_1 it consumes (patches/apply_patches.py:52).
//
// GEMV design (one 64-lane wavefront per workgroup, one "step" per workgroup):
//   * The pick (token, slot) is resolved through the tagged pointer table:
//     LSB=0 -> HBM pool slot, LSB=1 -> pinned host memory read zero-copy.
//   * The step's contiguous byte span (rows_per_step whole rows of the expert
//     matrix) is streamed into LDS with 16-byte buffer->LDS DMA loads
//     (buffer_load_dwordx4 ... lds): fully coalesced, no VGPR staging, and the
//     buffer descriptor bounds every read to the expert matrix.
//   * Each lane owns one unit (a K-quant super-block or two legacy blocks) and
//     keeps the matching int8 activation slice in registers, so the only LDS
//     traffic is the weight redistribution.
//   * Integer dots use v_dot4_i32_i8; scales are applied per 32-value group
//     (q8_1 activations) or per super-block (q8_K activations).
//   * Row partials are summed in a fixed order (deterministic), then the fused
//     epilogue applies scale -> bias -> GLU (kernels/moe-cache.cu:240-284).
//   * Workgroup 0 also runs the pick recorder: stamps, hit counter and the miss
//     log written at canonical positions (pick order, up before gate), one
//     legal ordering of the reference's atomicAdd-ordered log
//     (kernels/moe-cache.cu:159-204).
#include <hip/hip_runtime.h>

#include "mc_core.h"
#include "mc_internal.h"
#include "mc_step.h"

namespace mc {

// ---------------------------------------------------------------------------
// one step of one matrix pair (up [+ gate]) for one pick (mc_step.h)
// ---------------------------------------------------------------------------

// A row of more than 64 units (legacy types above K = 4096, K-quants above 16384):
// the step is that one row, streamed through the spans in chunks of 64 units; lane l
// dots unit 64j + l of chunk j and keeps its own sum, the 64 lane sums are added at
// the end (a fixed order).  On entry the activation row (q8_1 or q8_K blocks) is in
// LDS at arow with, for q8_1, its 16-value sums at rs16; the expert is resolved.
template <int T, int AQ>
__device__ __forceinline__ void wide_row_dots(const GemvArgs &a, StepCtx &s, uint8_t *lds, const uint8_t *arow,
                                              const int16_t *rs16, float &su, float &sg) {
    constexpr TypeGeom G = type_geom(T);
    constexpr int UE = G.unit_elems;
    constexpr int AUB = AQ == ACT_Q8_1 ? UE / 32 * 36 : 292;
    const int lane = threadIdx.x % WAVE;
    const int nu = a.ncols / UE;
    const u32 mbytes = (u32) (s.shared ? a.sh_matrix_bytes : a.expert_bytes);
    const u32 row_start = (u32) s.row0 * (u32) nu * (u32) G.unit_bytes;
    float pu = 0.0f, pg = 0.0f;
    for (int c0 = 0; c0 < nu; c0 += WAVE) {
        const int nuc = min(WAVE, nu - c0);
        const u32 start = row_start + (u32) c0 * (u32) G.unit_bytes;
        const u32 nbytes = (u32) nuc * (u32) G.unit_bytes;
        // the previous chunk's LDS reads have all returned (their values were used): the spans are free
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (s.wgate) dma_span<T>(s.wgate, mbytes, start, nbytes, lds + a.lds_span);
        const int n_up = dma_span<T>(s.wup, mbytes, start, nbytes, lds);
        const bool active = lane < nuc;
        const int col = c0 + lane;
        Act<UE> A;
        const int16_t *us16 = AQ == ACT_Q8_1 ? rs16 + (u32) col * (UE / 16) : nullptr;
        if (active) load_act_lds<UE, AQ, AQ == ACT_Q8_1>(A, arow + (u32) col * AUB, us16);
        if (s.wgate) {
            wait_loads_at_most(n_up);
            if (active) pg += span_unit_dot<T, AQ>(lds + a.lds_span, span_lead(s.wgate, start), lane, A);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (active) pu += span_unit_dot<T, AQ>(lds, span_lead(s.wup, start), lane, A);
    }
    su = row_group_sum(pu, WAVE);
    sg = s.wgate ? row_group_sum(pg, WAVE) : 0.0f;
}

template <int T, int ACT>
__device__ __forceinline__ void run_step(const GemvArgs &a, uint8_t *lds, bool shared, int tile) {
    constexpr int AQ = ACT == ACT_F32 ? ACT_Q8_1 : ACT;          // block format the dots read
    StepCtx s = step_locate(a, shared, tile);
    const bool wide = a.ncols / type_geom(T).unit_elems > WAVE;
    // the activation row depends only on (token, slot): its DMA goes out first
    const uint8_t *ybase;
    u32 yrow, ybytes;
    if (!shared) {
        ybase = a.y;
        ybytes = (u32) a.y_bytes;
        yrow = (u32) ((int64_t) (s.c % (int) a.nchannels_y) * a.stride_channel_y + (int64_t) s.t * a.stride_col_y);
    } else if (a.sh_y) {
        ybase = a.sh_y;
        ybytes = (u32) a.sh_y_bytes;
        yrow = (u32) ((int64_t) s.t * a.sh_stride_col_y);
    } else {
        ybase = a.y;
        ybytes = (u32) a.y_bytes;
        yrow = (u32) ((int64_t) s.t * a.stride_col_y);
    }
    const u32 alead = dma_bytes(ybase, ybytes, yrow, a.act_row_bytes, lds + a.lds_act);
    if (wide) step_resolve(a, s);                          // the chunks are streamed by wide_row_dots
    else step_issue<T>(a, s, lds);
    if (!s.valid) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }
    // the activation row went out first: it is in LDS while the weight spans still land
    wait_loads_at_most(s.n_gate + s.n_up);
    const uint8_t *arow = lds + a.lds_act + alead;
    if constexpr (ACT == ACT_F32) {
        // fp32 activations: the wave quantizes its staged row to q8_1 blocks in LDS
        quantize_row_lds((const float *) arow, lds + a.lds_q8, a.ncols);
        arow = lds + a.lds_q8;
    }
    float su, sg;
    if (wide) {
        int16_t *rs16 = (int16_t *) (lds + a.lds_sums);
        if constexpr (AQ == ACT_Q8_1) row_sums16_lds(arow, a.ncols, rs16);
        wide_row_dots<T, AQ>(a, s, lds, arow, rs16, su, sg);
    } else if constexpr (AQ == ACT_Q8_1) {
        // the row's 16-value code sums, once per wave (min / offset terms of the dots)
        int16_t *rs16 = (int16_t *) (lds + a.lds_sums);
        row_sums16_lds(arow, a.ncols, rs16);
        wait_loads_at_most(s.wgate ? s.n_up : 0);       // gate span landed (its dot runs while up lands)
        step_dots<T, AQ, true>(a, s, lds, arow, su, sg, rs16);
    } else {
        wait_loads_at_most(s.wgate ? s.n_up : 0);
        step_dots<T, AQ>(a, s, lds, arow, su, sg);
    }
    step_store<T>(a, s, su, sg);
}

// One wave per workgroup.  Workgroup 0 is the pick recorder when anything is
// recorded; then the shared-expert steps (the heaviest, dispatched first), then
// the routed steps.  Dynamic LDS: [up span | gate span | activation row | 16-value sums].
template <int TW, int TS, int ACT>
__global__ __launch_bounds__(WAVE) void mc_gemv_kernel(const GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    if (a.rec && blockIdx.x == 0) {
        record_picks(a);
        return;
    }
    const int tile = (int) blockIdx.x - a.rec;
    const int n_sh = a.sh_tiles_per_tok * a.n_tok;
    if (tile >= n_sh) {
        run_step<TW, ACT>(a, lds, false, tile - n_sh);
    } else if constexpr (TS != 0) {
        run_step<TS, ACT>(a, lds, true, tile);
    }
}

// ---------------------------------------------------------------------------
// activation quantizers
// ---------------------------------------------------------------------------

// ggml-CUDA quantize_q8_1: 32 lanes per block; amax / sum via xor butterflies
// (offsets 16, 8, 4, 2, 1); d = amax / 127 (IEEE division);
// q = amax == 0 ? 0 : roundf(x / d); ds = (half(d), half(sum)).
__global__ __launch_bounds__(256) void mc_quantize_q8_1_kernel(const QuantArgs a) {
    const int64_t nblk = a.k / 32;
    const int64_t gid = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gid / 32;                // global block index over rows
    const int l = (int) (gid & 31);
    const bool valid = blk < nblk * a.nrows;
    const int64_t row = valid ? blk / nblk : 0, b = valid ? blk % nblk : 0;
    const float x = valid ? a.x[row * a.x_stride + b * 32 + l] : 0.0f;
    float amax = fabsf(x), sum = x;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) {
        amax = fmaxf(amax, xor_lanes_rt(amax, off));
        sum += xor_lanes_rt(sum, off);
    }
    if (!valid) return;
    const float d = amax / 127.0f;
    const int8_t q = amax == 0.0f ? (int8_t) 0 : (int8_t) roundf(x / d);
    uint8_t *yb = a.y + row * a.y_stride + b * 36;
    yb[4 + l] = (uint8_t) q;
    if (l == 0) {
        const u32 ds = (u32) f2h_bits(d) | ((u32) f2h_bits(sum) << 16);
        *(u32 *) yb = ds;
    }
}

// quantize_row_q8_0_ref in q8_1 layout: d = amax / 127, id = d ? 1/d : 0, q = roundf(x * id), s = 0.
__global__ __launch_bounds__(256) void mc_quantize_q8_0_as_q8_1_kernel(const QuantArgs a) {
    const int64_t nblk = a.k / 32;
    const int64_t gid = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gid / 32;
    const int l = (int) (gid & 31);
    const bool valid = blk < nblk * a.nrows;
    const int64_t row = valid ? blk / nblk : 0, b = valid ? blk % nblk : 0;
    const float x = valid ? a.x[row * a.x_stride + b * 32 + l] : 0.0f;
    float amax = fabsf(x);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, xor_lanes_rt(amax, off));
    if (!valid) return;
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    float xs;
    {
#pragma clang fp contract(off)
        xs = x * id;
    }
    uint8_t *yb = a.y + row * a.y_stride + b * 36;
    yb[4 + l] = (uint8_t) (int8_t) roundf(xs);
    if (l == 0) *(u32 *) yb = (u32) f2h_bits(d);
}

// quantize_row_q8_K_ref: per 256 values, max = signed value of the first largest |x|,
// iscale = -127/max, q = min(127, round_half_even(iscale * x)), d = 1/iscale,
// bsums = sums of 16.  One 64-lane wave per block, 4 values per lane.
__global__ __launch_bounds__(64) void mc_quantize_q8_K_kernel(const QuantArgs a) {
    const int64_t nblk = a.k / 256;
    const int64_t blk = blockIdx.x;
    if (blk >= nblk * a.nrows) return;
    const int64_t row = blk / nblk, b = blk % nblk;
    const int lane = threadIdx.x;
    const float *xb = a.x + row * a.x_stride + b * 256;
    float xv[4];
    float amax = -1.0f;
    int aidx = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        xv[i] = xb[4 * lane + i];
        const float ax = fabsf(xv[i]);
        if (ax > amax) { amax = ax; aidx = 4 * lane + i; }
    }
    // reduce (amax, first index): larger amax wins, ties keep the lower index
#pragma unroll
    for (int off = WAVE / 2; off > 0; off >>= 1) {
        const float oa = __shfl_xor(amax, off, WAVE);
        const int oi = __shfl_xor(aidx, off, WAVE);
        if (oa > amax || (oa == amax && oi < aidx)) { amax = oa; aidx = oi; }
    }
    uint8_t *yb = a.y + row * a.y_stride + b * 292;
    if (amax == 0.0f) {
        *(u32 *) (yb + 4 + 4 * lane) = 0u;
        if (lane < 8) *(u32 *) (yb + 260 + 4 * lane) = 0u;
        if (lane == 0) *(float *) yb = 0.0f;
        return;
    }
    // the signed value at aidx, from the lane that holds it (no second read of the row)
    const int own = aidx & 3;
    const float mine = own == 0 ? xv[0] : own == 1 ? xv[1] : own == 2 ? xv[2] : xv[3];
    const float mx = __shfl(mine, aidx >> 2, WAVE);
    const float iscale = -127.0f / mx;
    int qs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float p;
        {
#pragma clang fp contract(off)
            p = iscale * xv[i];
        }
        int v = (int) rintf(p);
        qs[i] = v < 127 ? v : 127;
    }
    // the lane's four codes in one 4-byte store (blocks are 292 bytes: 4-byte aligned)
    *(u32 *) (yb + 4 + 4 * lane) = (u32) (uint8_t) qs[0] | ((u32) (uint8_t) qs[1] << 8) |
                                   ((u32) (uint8_t) qs[2] << 16) | ((u32) (uint8_t) qs[3] << 24);
    // bsums: 16 values = 4 lanes
    int s = qs[0] + qs[1] + qs[2] + qs[3];
    s += __shfl_xor(s, 1, WAVE);
    s += __shfl_xor(s, 2, WAVE);
    if ((lane & 3) == 0) *(int16_t *) (yb + 260 + 2 * (lane >> 2)) = (int16_t) s;
    if (lane == 0) *(float *) yb = 1.0f / iscale;
}

// MoE combine + RMSNorm + q8_1 quantization of the result, one 1024-thread
// workgroup (16 waves) per token row; wave w handles the 256-value chunks w and
// w + 16 of the row in registers (combine_chunk / quantize_chunk, mc_core.h):
//   x = residual + shared + sum_j w[j] * o[j]   (j ascending, fmaf) -> x_out
//   s = 1 / sqrtf(sum of the canonical chunk sums (ascending) / k + eps)
//   y = q8_1((x * s) * norm_weight)   (rms_norm; y = q8_1(x) otherwise)
// This is the weighted sum ggml performs after MUL_MAT_ID (MUL by the router
// weights, then ADDs), the RMS_NORM + MUL in front of the next MoE block and the
// quantize_q8_1 of the next GEMV's input, in one launch.  The norm weights are
// loaded before the workgroup barrier, so the second phase does not wait on memory.
constexpr int COMBINE_MAX_K = 8192;
constexpr int COMBINE_THREADS = 1024;
constexpr int COMBINE_WAVES = COMBINE_THREADS / WAVE;
constexpr int COMBINE_CHUNKS_PER_WAVE = COMBINE_MAX_K / RMS_CHUNK / COMBINE_WAVES;

__global__ __launch_bounds__(COMBINE_THREADS) void mc_combine_q8_1_kernel(const CombineArgs a) {
    __shared__ float chunk_sum[COMBINE_MAX_K / RMS_CHUNK];
    const int64_t t = blockIdx.x;
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int nchunk = (int) (a.k / RMS_CHUNK);
    const bool norm = a.rms_norm != 0;
    float xv[COMBINE_CHUNKS_PER_WAVE][4];
    v4f nwv[COMBINE_CHUNKS_PER_WAVE];
#pragma unroll
    for (int ci = 0; ci < COMBINE_CHUNKS_PER_WAVE; ++ci) {
        const int j = wave + COMBINE_WAVES * ci;
        nwv[ci] = v4f{1.0f, 1.0f, 1.0f, 1.0f};
        if (j < nchunk) {
            if (norm && a.norm_weight) nwv[ci] = *(const v4f *) (a.norm_weight + j * RMS_CHUNK + 4 * lane);
            const float cs = combine_chunk(a.o + t * a.n_used * a.o_stride, a.o_stride, a.w + t * a.n_used, a.n_used,
                                           a.shared ? a.shared + t * a.shared_stride : nullptr,
                                           a.residual ? a.residual + t * a.k : nullptr,
                                           a.x_out ? a.x_out + t * a.k : nullptr, j, xv[ci]);
            if (lane == 0) chunk_sum[j] = cs;
        }
    }
    float s = 1.0f;
    if (norm) {
        __syncthreads();
        float ss = 0.0f;                     // every wave adds the chunk sums in the same order
        for (int j = 0; j < nchunk; ++j) ss += chunk_sum[j];
        s = 1.0f / sqrtf(ss / (float) a.k + a.eps);
    }
#pragma unroll
    for (int ci = 0; ci < COMBINE_CHUNKS_PER_WAVE; ++ci) {
        const int j = wave + COMBINE_WAVES * ci;
        if (j < nchunk) quantize_chunk(xv[ci], norm, s, nwv[ci], a.y + t * a.y_stride, j);
    }
}

// ---------------------------------------------------------------------------
// host-side launchers
// ---------------------------------------------------------------------------

template <int TW, int TS, int ACT>
static hipError_t launch_t(const GemvArgs &a, hipStream_t s) {
    // rows of more than 16K values stage activation rows beyond the default 64 KiB of LDS
    if (a.lds_total > 64u * 1024u) {
        static_cast<void>(hipFuncSetAttribute((const void *) mc_gemv_kernel<TW, TS, ACT>,
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int) FFN_LDS_MAX));
    }
    hipLaunchKernelGGL((mc_gemv_kernel<TW, TS, ACT>), dim3((unsigned) (a.n_tiles + a.rec)), dim3(WAVE),
                       a.lds_total, s, a);
    return hipGetLastError();
}

template <int TW, int ACT>
static hipError_t launch_ts(const GemvArgs &a, int ts, hipStream_t s) {
    switch (ts) {
        case 0: return launch_t<TW, 0, ACT>(a, s);
        case T_Q4_0: return launch_t<TW, T_Q4_0, ACT>(a, s);
        case T_Q5_0: return launch_t<TW, T_Q5_0, ACT>(a, s);
        case T_Q8_0: return launch_t<TW, T_Q8_0, ACT>(a, s);
        case T_Q2_K: return launch_t<TW, T_Q2_K, ACT>(a, s);
        case T_Q3_K: return launch_t<TW, T_Q3_K, ACT>(a, s);
        case T_Q4_K: return launch_t<TW, T_Q4_K, ACT>(a, s);
        case T_Q5_K: return launch_t<TW, T_Q5_K, ACT>(a, s);
        case T_Q6_K: return launch_t<TW, T_Q6_K, ACT>(a, s);
        default: return hipErrorInvalidValue;
    }
}

template <int TW>
static hipError_t launch_act(const GemvArgs &a, int ts, int act, hipStream_t s) {
    if (act == ACT_Q8_1) return launch_ts<TW, ACT_Q8_1>(a, ts, s);
    if (act == ACT_F32) return launch_ts<TW, ACT_F32>(a, ts, s);
    if constexpr (type_geom(TW).kquant) {
        if (act == ACT_Q8_K) {
            // q8_K activations exist for K-quant shared experts only
            switch (ts) {
                case 0: return launch_t<TW, 0, ACT_Q8_K>(a, s);
                case T_Q2_K: return launch_t<TW, T_Q2_K, ACT_Q8_K>(a, s);
                case T_Q3_K: return launch_t<TW, T_Q3_K, ACT_Q8_K>(a, s);
                case T_Q4_K: return launch_t<TW, T_Q4_K, ACT_Q8_K>(a, s);
                case T_Q5_K: return launch_t<TW, T_Q5_K, ACT_Q8_K>(a, s);
                case T_Q6_K: return launch_t<TW, T_Q6_K, ACT_Q8_K>(a, s);
                default: return hipErrorInvalidValue;
            }
        }
    }
    return hipErrorInvalidValue;
}

// Rows per step for a matrix with nu units of row_bytes per row: the most rows
// (<= 64 / nu) whose staged spans (nspan of them) fit GEMV_LDS_BUDGET beside the
// activation row.
static int fit_rows_per_step(int nu, uint32_t row_bytes, int nspan, uint32_t act_span) {
    int r = WAVE / nu;
    while (r > 1 && nspan * span_bytes((uint32_t) r, row_bytes) + act_span > GEMV_LDS_BUDGET) --r;
    return r;
}

int launch_ffn(GemvArgs a, int tw, int ts, int act, void *stream);   // mc_ffn.hip

// Fills the tiling and LDS fields of `a` and launches.  Returns a hipError_t value.
int launch_gemv(GemvArgs a, int tw, int ts, int act, void *stream) {
    if (a.mode != FFN_NONE) return launch_ffn(a, tw, ts, act, stream);
    const TypeGeom g = type_geom(tw);
    const int nu = a.ncols / g.unit_elems;
    const uint32_t rb = (uint32_t) nu * (uint32_t) g.unit_bytes;
    a.act_row_bytes = act == ACT_Q8_1 ? (uint32_t) (a.ncols / 32 * 36)
                    : act == ACT_Q8_K ? (uint32_t) (a.ncols / 256 * 292) : (uint32_t) a.ncols * 4u;
    // fp32 rows also need room for their q8_1 copy
    const uint32_t q8_bytes = act == ACT_F32 ? ((uint32_t) (a.ncols / 32 * 36) + 15u) & ~15u : 0u;
    // q8_1 rows (given or made from fp32) also get their 16-value sums
    const uint32_t sums_bytes = act == ACT_Q8_K ? 0u : ((uint32_t) (a.ncols / 8) + 15u) & ~15u;
    const uint32_t act_span = round_up_1k(a.act_row_bytes + 20u) + q8_bytes + sums_bytes;
    if (ts == 0 || !a.sh_up) ts = 0;
    const int nspan = (a.has_gate || (ts != 0 && a.sh_gate)) ? 2 : 1;
    // a row of more than 64 units is one step, staged 64 units at a time (wide_row_dots)
    a.rps = nu > WAVE ? 1 : fit_rows_per_step(nu, rb, nspan, act_span);
    a.tiles_per_pick = (a.nrows + a.rps - 1) / a.rps;
    a.n_routed_tiles = a.tiles_per_pick * a.n_used * a.n_tok;
    uint32_t span = nu > WAVE ? span_bytes(1u, (uint32_t) WAVE * (uint32_t) g.unit_bytes) : span_bytes((uint32_t) a.rps, rb);
    a.sh_rps = 0;
    a.sh_tiles_per_tok = 0;
    if (ts != 0) {
        const TypeGeom gs = type_geom(ts);
        const int nus = a.ncols / gs.unit_elems;
        const uint32_t rbs = (uint32_t) nus * (uint32_t) gs.unit_bytes;
        a.sh_rps = nus > WAVE ? 1 : fit_rows_per_step(nus, rbs, nspan, act_span);
        a.sh_tiles_per_tok = (a.nrows + a.sh_rps - 1) / a.sh_rps;
        const uint32_t sspan = nus > WAVE ? span_bytes(1u, (uint32_t) WAVE * (uint32_t) gs.unit_bytes)
                                          : span_bytes((uint32_t) a.sh_rps, rbs);
        span = sspan > span ? sspan : span;
    }
    a.lds_span = span;
    a.lds_act = (uint32_t) nspan * span;
    a.lds_q8 = a.lds_act + act_span - q8_bytes - sums_bytes;
    a.lds_sums = a.lds_act + act_span - sums_bytes;
    a.lds_total = a.lds_act + act_span;
    if (a.lds_total > FFN_LDS_MAX) return (int) hipErrorInvalidValue;
    a.rec = (a.stats || a.stamps || a.stamps_gate) ? 1 : 0;
    a.n_tiles = a.n_routed_tiles + a.sh_tiles_per_tok * a.n_tok;
    if (a.n_tiles <= 0) return (int) hipSuccess;
    hipStream_t s = (hipStream_t) stream;
    switch (tw) {
        case T_Q4_0: return (int) launch_act<T_Q4_0>(a, ts, act, s);
        case T_Q5_0: return (int) launch_act<T_Q5_0>(a, ts, act, s);
        case T_Q8_0: return (int) launch_act<T_Q8_0>(a, ts, act, s);
        case T_Q2_K: return (int) launch_act<T_Q2_K>(a, ts, act, s);
        case T_Q3_K: return (int) launch_act<T_Q3_K>(a, ts, act, s);
        case T_Q4_K: return (int) launch_act<T_Q4_K>(a, ts, act, s);
        case T_Q5_K: return (int) launch_act<T_Q5_K>(a, ts, act, s);
        case T_Q6_K: return (int) launch_act<T_Q6_K>(a, ts, act, s);
        default: return (int) hipErrorInvalidValue;
    }
}

int launch_combine(const CombineArgs &c, void *stream) {
    if (c.n_tok <= 0 || c.k <= 0) return (int) hipSuccess;
    if (c.k > COMBINE_MAX_K || c.k % RMS_CHUNK || c.n_used > COMBINE_MAX_USED) return (int) hipErrorInvalidValue;
    hipLaunchKernelGGL(mc_combine_q8_1_kernel, dim3((unsigned) c.n_tok), dim3(COMBINE_THREADS), 0,
                       (hipStream_t) stream, c);
    return (int) hipGetLastError();
}

int launch_quantize(int kind, const QuantArgs &q, void *stream) {
    hipStream_t s = (hipStream_t) stream;
    if (q.nrows <= 0 || q.k <= 0) return (int) hipSuccess;
    if (kind == 0 || kind == 2) {
        const int64_t threads = q.nrows * q.k;
        const unsigned grid = (unsigned) ((threads + 255) / 256);
        if (kind == 0) hipLaunchKernelGGL(mc_quantize_q8_1_kernel, dim3(grid), dim3(256), 0, s, q);
        else hipLaunchKernelGGL(mc_quantize_q8_0_as_q8_1_kernel, dim3(grid), dim3(256), 0, s, q);
    } else {
        const unsigned grid = (unsigned) (q.nrows * (q.k / 256));
        hipLaunchKernelGGL(mc_quantize_q8_K_kernel, dim3(grid), dim3(64), 0, s, q);
    }
    return (int) hipGetLastError();
}

}  // namespace mc
