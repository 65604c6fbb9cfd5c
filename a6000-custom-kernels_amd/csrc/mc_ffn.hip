// mc_ffn.hip -- fused decode kernels for one MoE FFN block (a few tokens).
//
// ggml evaluates a MoE block as RMS_NORM -> MUL(norm weight) -> quantize_q8_1 ->
// MUL_MAT_ID(gate, up) + GLU -> quantize -> MUL_MAT_ID(down) -> MUL(router
// weights) -> sum over slots -> ADD(shared expert) -> ADD(residual).  The
// pointer-table GEMV the reference adds (kernels/moe-cache.cu:76-291) is the
// MUL_MAT_ID part.  For batch-1 decode every launch boundary costs microseconds
// of dispatch and drain against a few microseconds of HBM time, so these two
// kernels cover the whole block in two launches, with the GEMV steps of
// mc_step.h unchanged:
//
//   mc_ffn_gate_up_kernel      (FFN_GATE_UP_NORM)
//     workgroups of up to 8 step waves, one GEMV step (gate+up rows of one pick,
//     or of the shared expert) per wave, and 4 prologue waves.  While the steps'
//     weight spans stream into LDS, the prologue waves compute
//     y = q8_1((x * s) * nw), s = 1/sqrt(mean(x^2) + eps) in the canonical RMS
//     order (mc_internal.h), from the fp32 residual row x, and every step wave's
//     dots read that row.  Bit-identical to the combine kernel's y followed by the
//     q8_1 GEMV.
//
//   mc_ffn_down_combine_kernel (FFN_DOWN_COMBINE)
//     one workgroup per (token, block of rows): one wave per pick computes the
//     rows of its down projection (wave 0: the shared expert, whose span is the
//     largest), the results meet in LDS, and wave 0 writes
//     x_out = residual + shared + sum_c w_c * o_c (fmaf, c ascending) -- the
//     combine kernel's arithmetic, without o in HBM.  The activation rows are fp32
//     (quantized to q8_1 by each wave) or the q8_1 rows the gate/up kernel wrote.
//
// A plain __syncthreads() would wait for every LDS-writing DMA of the wave
// (its release fence drains them); lds_barrier() waits for LDS operations only,
// and the gate/up kernel hands the normalized row to its step waves through LDS
// counters instead of a barrier.
#include <hip/hip_runtime.h>

#include <mutex>

#include "mc_core.h"
#include "mc_internal.h"
#include "mc_step.h"

namespace mc {

__device__ __forceinline__ int lane_of() { return (int) (threadIdx.x % WAVE); }

// ---------------------------------------------------------------------------
// device status word
// ---------------------------------------------------------------------------

// STATUS_* bits set by a kernel that could not finish its work (a bounded wait
// that gave up).  One word per GPU for the life of the process.  Host code never
// passes this name to a kernel: it uses the address hipGetSymbolAddress returns
// with that GPU current (status_address), which differs from GPU to GPU.
static __device__ __align__(256) u32 status_word[64];

constexpr int MAX_DEVICES = 64;

// Device address of the current GPU's status word (looked up once per GPU).
int status_address(u32 **out) {
    static std::mutex m;
    static u32 *addr[MAX_DEVICES] = {};
    int d = 0;
    hipError_t err = hipGetDevice(&d);
    if (err != hipSuccess) return (int) err;
    if (d < 0 || d >= MAX_DEVICES) return (int) hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(m);
    if (!addr[d]) {
        void *p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(status_word));
        if (err != hipSuccess) return (int) err;
        addr[d] = (u32 *) p;
    }
    *out = addr[d];
    return (int) hipSuccess;
}

// ---------------------------------------------------------------------------
// gate/up with the RMSNorm + q8_1 prologue
// ---------------------------------------------------------------------------

// Waits (bounded: a.spin_limit polls) until the LDS counter reaches n.  On timeout it
// sets STATUS_WAIT_TIMEOUT in the status word (the host reads it with
// ggml_hip_moe_check_status) and returns false; the caller then skips the work that
// needed the count and still exits.  The LDS reads a wave issues afterwards are
// ordered after this read by the LDS unit.
__device__ __forceinline__ bool wait_lds_count(const GemvArgs &a, const u32 *cnt, u32 n) {
    for (int it = 0; it < a.spin_limit; ++it) {
        if (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= n) return true;
        __builtin_amdgcn_s_sleep(1);
    }
    if (threadIdx.x % WAVE == 0)
        __hip_atomic_fetch_or(a.status, STATUS_WAIT_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return false;
}

// A prologue wave p of token t handles chunks j = p + NP * ci, ci < PC: loads them
// (x and the norm weights, into registers; an index past the row is clamped to the
// last chunk, whose results it then rewrites with identical bytes, so loads,
// arithmetic and stores are branch-free and the chunks' divisions interleave),
// counts itself in sync[2] once the loads are issued (the step waves hold their
// weight DMA until then, so these loads are not queued behind the weight stream),
// publishes the chunks' canonical sums and counts them in sync[0], waits for the
// other prologue waves' sums, and writes q8_1((x * scale) * nw) of its chunks to the
// LDS row (and to y_out when asked), counted in sync[1].
template <int PC, int AQ>
__device__ __forceinline__ void gu_prologue(const GemvArgs &a, int t, int p, float *red, uint8_t *ys, int16_t *s16,
                                            u32 *sync, bool write_y_out) {
    constexpr int NP = FFN_GU_PRO_WAVES;
    const int lane = threadIdx.x % WAVE;
    const int K = a.ncols, nchunk = K / RMS_CHUNK;
    const float *xr = a.nx + (int64_t) t * a.nx_stride;
    v4f xv[PC], nwv[PC];
#pragma unroll
    for (int ci = 0; ci < PC; ++ci) {
        const int j = min(p + NP * ci, nchunk - 1);
        xv[ci] = *(const v4f *) (xr + RMS_CHUNK * j + 4 * lane);
        nwv[ci] = a.nw ? *(const v4f *) (a.nw + RMS_CHUNK * j + 4 * lane) : v4f{1.0f, 1.0f, 1.0f, 1.0f};
    }
    if (lane == 0) __hip_atomic_fetch_add(sync + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    float cs[PC];
    rms_chunk_sums<PC>(xv, cs);
    if (lane == 0) {
#pragma unroll
        for (int ci = 0; ci < PC; ++ci) red[min(p + NP * ci, nchunk - 1)] = cs[ci];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");      // the sums are in LDS before the count
    if (lane == 0) __hip_atomic_fetch_add(sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    wait_lds_count(a, sync, (u32) NP);            // on timeout the row is wrong and the status word says so
    // ascending, as every other producer of y: all NP * PC slots are read at once (128-bit
    // LDS reads, no read waits on an add) and the slots past the row add +0.0, which leaves
    // the non-negative sum's bits unchanged
    float rv[NP * PC];
#pragma unroll
    for (int j = 0; j < NP * PC; j += 4) {
        const v4f r4 = *(const v4f *) (red + j);
        rv[j] = r4.x;
        rv[j + 1] = r4.y;
        rv[j + 2] = r4.z;
        rv[j + 3] = r4.w;
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NP * PC; ++j) ss += j < nchunk ? rv[j] : 0.0f;
    const float scale = 1.0f / sqrtf(ss / (float) K + a.eps);
    int jc[PC];
#pragma unroll
    for (int ci = 0; ci < PC; ++ci) jc[ci] = min(p + NP * ci, nchunk - 1);
    if constexpr (AQ == ACT_Q8_K) {
        // one q8_K block per chunk (256 values), written to the LDS row and to y_out when asked
        float v[PC][4];
        uint8_t *yb[PC], *yo[PC];
#pragma unroll
        for (int ci = 0; ci < PC; ++ci) {
            v[ci][0] = (xv[ci].x * scale) * nwv[ci].x;
            v[ci][1] = (xv[ci].y * scale) * nwv[ci].y;
            v[ci][2] = (xv[ci].z * scale) * nwv[ci].z;
            v[ci][3] = (xv[ci].w * scale) * nwv[ci].w;
            yb[ci] = ys + Q8K_LDS_STRIDE * jc[ci];
            yo[ci] = a.y_out + (int64_t) t * a.y_out_stride + 292 * jc[ci];     // used only with write_y_out
        }
        q8K_chunks<PC>(v, yb, yo, write_y_out);
    } else {
        // one chunk per trip of a rolled loop: the unrolled form interleaves the PC chunks'
        // dependency chains but is PC times the code, which every dispatch fetches into a cold
        // instruction cache (this launch alternates with the down launch); measured 0.1 us faster
#pragma unroll 1
        for (int ci = 0; ci < PC; ++ci) {
            v4f x1[1] = {xv[0]}, n1[1] = {nwv[0]};
            int j1[1] = {jc[0]};
#pragma unroll
            for (int k = 1; k < PC; ++k) {
                if (ci == k) {
                    x1[0] = xv[k];
                    n1[0] = nwv[k];
                    j1[0] = jc[k];
                }
            }
            quantize_chunks<1, Q8_1_LDS_STRIDE>(x1, n1, scale, ys, j1, s16);
        }
        if (write_y_out) {
#pragma unroll
            for (int ci = 0; ci < PC; ++ci) {
                const float x4[4] = {xv[ci].x, xv[ci].y, xv[ci].z, xv[ci].w};
                quantize_chunk<true>(x4, true, scale, nwv[ci], a.y_out + (int64_t) t * a.y_out_stride,
                                     min(p + NP * ci, nchunk - 1));
            }
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");      // the row is in LDS before the count
    if (lane == 0) __hip_atomic_fetch_add(sync + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// q8_1 copy of the GLU outputs: the workgroup's steps cover exactly one 32-row block
// of one matrix (the host arranges the tiling).  Each step wave puts its rows into the
// LDS block (zeros for a skipped step) and counts itself; the wave that completes the
// count quantizes the block with the q8_1 quantizer's arithmetic (32 lanes: amax and
// sum by xor butterflies, d = amax / 127, roundf(x / d)) and writes its 36 bytes.
__device__ __forceinline__ void gu_block_q8_1(const GemvArgs &a, int t, int local0, int sw, int rps, bool ran, int rl,
                                              float v, float *h32, u32 *cnt) {
    const int lane = threadIdx.x % WAVE;
    if (ran) {
        if (rl >= 0) h32[sw * rps + rl] = v;
    } else if (lane < rps) {
        h32[sw * rps + lane] = 0.0f;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");      // the rows are in LDS before the count
    u32 old = 0u;
    if (lane == 0) old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    old = (u32) __builtin_amdgcn_readfirstlane((int) old);
    if (old != (u32) a.nwaves - 1) return;
    uint8_t *blk;
    if (local0 < a.sh_tiles_per_tok) {
        blk = a.hq_sh + (int64_t) t * a.hq_sh_stride + (local0 * a.sh_rps / 32) * 36;
    } else {
        const int tile = local0 - a.sh_tiles_per_tok;
        const int c = tile / a.tiles_per_pick;
        blk = a.hq + (int64_t) t * a.hq_stride_col + (int64_t) c * a.hq_stride_pick +
              ((tile % a.tiles_per_pick) * a.rps / 32) * 36;
    }
    const float x = lane < 32 ? h32[lane] : 0.0f;
    float d, sum;
    const int8_t q = q8_1_lane(x, d, sum);
    if (lane < 32) blk[4 + lane] = (uint8_t) q;
    if (lane == 0) *(u32 *) blk = (u32) f2h_bits(d) | ((u32) f2h_bits(sum) << 16);
}

// Workgroup: FFN_GU_PRO_WAVES prologue waves, then nwaves step waves (one GEMV step
// each).  The step waves issue their weight spans first and only wait for the
// normalized row once their gate span has landed; no workgroup barrier follows the
// start, so no wave waits for another wave's weight stream.
// Dynamic LDS: [nwaves x (up span | gate span)] [q8_1 row] [5 counters (32 bytes) | 32 chunk sums | 32-row block |
// 16-value sums of the row (int16)]
template <int TW, int TS, int AQ>
__global__ __launch_bounds__((FFN_GU_MAX_WAVES + FFN_GU_PRO_WAVES) *WAVE) void mc_ffn_gate_up_kernel(const GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int NP = FFN_GU_PRO_WAVES;
    // the wave index is uniform across the wave: keep it (and the step) in scalar registers
    const int wave = __builtin_amdgcn_readfirstlane((int) (threadIdx.x / WAVE));
    if (a.rec && blockIdx.x == 0) {
        if (wave == 0) record_picks(a);
        return;
    }
    const int b = (int) blockIdx.x - a.rec;
    const int t = b / a.wg_per_tok;
    uint8_t *ys = lds + a.lds_y;
    u32 *sync = (u32 *) (lds + a.lds_part);
    float *red = (float *) (lds + a.lds_part + 32);
    int16_t *s16 = (int16_t *) (lds + a.lds_part + 32 + 4 * 32 + 4 * 32);   // 16-value sums of y
    if (threadIdx.x == 0) {
        sync[0] = 0u;
        sync[1] = 0u;
        sync[2] = 0u;
        sync[3] = 0u;
        sync[4] = 0u;
    }
    lds_barrier();                                            // counters set; nothing is in flight yet
    if (wave < NP) {
        const bool y_out = a.y_out && (b % a.wg_per_tok) == 0;
        if (a.ncols <= 4 * NP * RMS_CHUNK) gu_prologue<4, AQ>(a, t, wave, red, ys, s16, sync, y_out);
        else gu_prologue<8192 / RMS_CHUNK / NP, AQ>(a, t, wave, red, ys, s16, sync, y_out);
        return;
    }
    const int sw = wave - NP;
    const int bt = b % a.wg_per_tok;
    int local0 = 0, local;                                      // local: this wave's step
    bool sh, run;
    if (a.mixed_wg) {
        // waves 0 .. nr-1 take this workgroup's share of the routed steps, the next ns waves its
        // share of the shared steps; shares differ by at most one step between workgroups
        const int G = a.wg_per_tok, NS = a.sh_tiles_per_tok, NR = a.tiles_per_tok - NS;
        const int nr = NR / G + (bt < NR % G ? 1 : 0), ns = NS / G + (bt < NS % G ? 1 : 0);
        sh = sw >= nr;
        local = sh ? bt * (NS / G) + min(bt, NS % G) + (sw - nr) : NS + bt * (NR / G) + min(bt, NR % G) + sw;
        run = sw < nr + ns && (TS != 0 || !sh);
    } else {
        // the first nsh_wg workgroups of a token take sh_per_wg shared steps each, the others
        // nwaves routed steps each (whole 32-row blocks of one matrix when hq is written)
        const int nsh_wg = a.sh_per_wg > 0 ? (a.sh_tiles_per_tok + a.sh_per_wg - 1) / a.sh_per_wg : 0;
        sh = bt < nsh_wg;
        local0 = sh ? bt * a.sh_per_wg : a.sh_tiles_per_tok + (bt - nsh_wg) * a.nwaves;
        local = local0 + sw;
        run = (sh ? sw < a.sh_per_wg && local < a.sh_tiles_per_tok : local < a.tiles_per_tok) && (TS != 0 || !sh);
    }
    // the first n_early step waves (one per SIMD) issue their spans before the others, so their
    // bytes land early in the stream and their dots overlap the rest of it (0.1-0.2 us off a
    // launch of mixed workgroups; no change in workgroups of 32-row blocks)
    const int n_early = a.nwaves / 2;
    const bool early = sw < n_early, late = n_early > 0 && !early;
    uint8_t *span = lds + (u32) sw * a.lds_wave;
    StepCtx s;
    if (run) {
        s = sh ? step_locate(a, true, t * a.sh_tiles_per_tok + local)
               : step_locate(a, false, t * a.n_used * a.tiles_per_pick + (local - a.sh_tiles_per_tok));
        step_resolve(a, s);
        run = s.valid;
    }
    if (run) {
        wait_lds_count(a, sync + 2, (u32) NP);                // the prologue's loads go out first
        if (late) wait_lds_count(a, sync + 4, (u32) n_early);   // then the early waves' spans
        if (sh) {
            if constexpr (TS != 0) step_dma<TS, true>(a, s, span);
        } else {
            step_dma<TW, true>(a, s, span);
        }
        if (early && lane_of() == 0) __hip_atomic_fetch_add(sync + 4, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        wait_loads_at_most(s.wgate ? s.n_up : 0);             // gate span landed (up may still land)
        run = wait_lds_count(a, sync + 1, (u32) NP);          // the normalized row is complete
    } else if (early && lane_of() == 0) {
        __hip_atomic_fetch_add(sync + 4, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    float v = 0.0f;
    int rl = -1;
    if (run) {
        float su, sg;
        if (sh) {
            if constexpr (TS != 0) {
                step_dots<TS, AQ, true, AQ == ACT_Q8_K ? Q8K_LDS_STRIDE : Q8_1_LDS_STRIDE>(a, s, span, ys, su, sg, s16);
                rl = step_store<TS>(a, s, su, sg, v);
            }
        } else {
            step_dots<TW, AQ, true, AQ == ACT_Q8_K ? Q8K_LDS_STRIDE : Q8_1_LDS_STRIDE>(a, s, span, ys, su, sg, s16);
            rl = step_store<TW>(a, s, su, sg, v);
        }
    }
    if (a.hq && (!sh || a.hq_sh)) gu_block_q8_1(a, t, local0, sw, sh ? a.sh_rps : a.rps, run, rl, v, red + 32, sync + 3);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");      // a step skipped after a timeout: its DMA has landed
}

// ---------------------------------------------------------------------------
// down projection + combine
// ---------------------------------------------------------------------------
// Dynamic LDS: [nwaves x (span | activation staging | q8_1 row | 16-value sums)] [row results nwaves x rps]
// ACT: the routed rows' format (q8_1 or fp32); AQ: the dots' format (q8_1, or q8_K of fp32 rows)
template <int TW, int TS, int ACT, int AQ>
__global__ __launch_bounds__(FFN_DN_MAX_WAVES *WAVE) void mc_ffn_down_combine_kernel(const GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    static_assert(AQ == ACT_Q8_1 || ACT == ACT_F32, "q8_K dots quantize fp32 rows");
    const int wave = __builtin_amdgcn_readfirstlane((int) (threadIdx.x / WAVE)), lane = threadIdx.x % WAVE;
    if (a.rec && blockIdx.x == 0) {
        if (wave == 0) record_picks(a);
        return;
    }
    const int b = (int) blockIdx.x - a.rec;
    const int t = b / a.wg_per_tok;
    const int rt = b % a.wg_per_tok;                    // row tile
    // wave 0 is the shared expert's (its larger span goes out first), then pick c = wave - off
    const int off = a.nwaves > a.n_used ? 1 : 0;
    const bool sh = off && wave == 0;
    uint8_t *span = lds + (u32) wave * a.lds_wave;
    float *part = (float *) (lds + a.lds_part);         // [nwaves][rps]
    const int rps = a.rps;

    StepCtx s = sh ? step_locate(a, true, t * a.sh_tiles_per_tok + rt)
                   : step_locate(a, false, (t * a.n_used + wave - off) * a.tiles_per_pick + rt);
    // activation row of the wave's pick (or of the shared expert), first
    const uint8_t *ybase;
    u32 yrow, ybytes;
    if (!sh) {
        ybase = a.y;
        ybytes = (u32) a.y_bytes;
        yrow = (u32) ((int64_t) (s.c % (int) a.nchannels_y) * a.stride_channel_y + (int64_t) s.t * a.stride_col_y);
    } else {
        ybase = a.sh_y;
        ybytes = (u32) a.sh_y_bytes;
        yrow = (u32) ((int64_t) s.t * a.sh_stride_col_y);
    }
    // the shared expert's row may be fp32 (sh_act_f32) beside q8_1 routed rows
    const bool qf32 = ACT == ACT_F32 || (sh && a.sh_act_f32);
    const u32 alead = dma_bytes(ybase, ybytes, yrow, sh ? a.sh_act_row_bytes : a.act_row_bytes, span + a.lds_act);
    if (sh) {
        if constexpr (TS != 0) step_issue<TS>(a, s, span);
    } else {
        step_issue<TW>(a, s, span);
    }
    float v = 0.0f;                                     // an out-of-range expert id contributes 0
    int nu = 1;
    if (s.valid) {
        // the activation row went out first: it is in LDS while the weights still land
        wait_loads_at_most(s.n_up);
        const uint8_t *arow = span + a.lds_act + alead;
        if (qf32) {
            if constexpr (AQ == ACT_Q8_K) quantize_row_lds_q8K((const float *) arow, span + a.lds_q8, a.ncols);
            else quantize_row_lds((const float *) arow, span + a.lds_q8, a.ncols);
            arow = span + a.lds_q8;
        }
        // the row's 16-value code sums, once per wave (the K-quant dots' min terms; q8_K
        // blocks carry them)
        int16_t *rs16 = (int16_t *) (span + a.lds_sums);
        if constexpr (AQ == ACT_Q8_1) row_sums16_lds(arow, a.ncols, rs16);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        float su = 0.0f, sg = 0.0f;
        if (sh) {
            if constexpr (TS != 0) {
                step_dots<TS, AQ, true, AQ == ACT_Q8_K ? Q8K_LDS_STRIDE : 0>(a, s, span, arow, su, sg, rs16);
                nu = a.ncols / type_geom(TS).unit_elems;
            }
            v = su;
        } else {
            step_dots<TW, AQ, true, AQ == ACT_Q8_K ? Q8K_LDS_STRIDE : 0>(a, s, span, arow, su, sg, rs16);
            nu = a.ncols / type_geom(TW).unit_elems;
            const int rl = lane / nu;
            v = routed_value(a, s, s.row0 + (rl < s.nrows_here ? rl : 0), su, sg);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");     // an invalid step's activation DMA too
    {
        const int rl = lane / nu;
        if (s.valid) {
            if (lane % nu == 0 && rl < s.nrows_here) part[wave * rps + rl] = v;
        } else if (lane < s.nrows_here) {
            part[wave * rps + lane] = 0.0f;
        }
    }
    lds_barrier();
    // x = residual + shared + sum_c w_c * o_c, one lane per row
    if (wave == 0 && lane < s.nrows_here) {
        const int row = s.row0 + lane;
        float x = a.residual ? a.residual[(int64_t) t * a.x_stride + row] : 0.0f;
        if (off) x += part[lane];
        const float *w = a.router_w + (int64_t) t * a.n_used;
        for (int c = 0; c < a.n_used; ++c) x = fmaf(w[c], part[(c + off) * rps + lane], x);
        a.x_out[(int64_t) t * a.x_stride + row] = x;
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

template <class K>
static hipError_t launch_big_lds(K kernel, unsigned grid, unsigned block, uint32_t lds, const GemvArgs &a, hipStream_t s) {
    static_cast<void>(hipFuncSetAttribute((const void *) kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int) FFN_LDS_MAX));
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(block), lds, s, a);
    return hipGetLastError();
}

template <int TW, int TS, int AQ>
static hipError_t launch_gu_t(const GemvArgs &a, hipStream_t s) {
    return launch_big_lds(mc_ffn_gate_up_kernel<TW, TS, AQ>, (unsigned) (a.rec + a.n_tok * a.wg_per_tok),
                          (unsigned) ((a.nwaves + FFN_GU_PRO_WAVES) * WAVE), a.lds_total, a, s);
}

template <int TW, int TS, int ACT, int AQ>
static hipError_t launch_dn_t(const GemvArgs &a, hipStream_t s) {
    return launch_big_lds(mc_ffn_down_combine_kernel<TW, TS, ACT, AQ>, (unsigned) (a.rec + a.n_tok * a.wg_per_tok),
                          (unsigned) (a.nwaves * WAVE), a.lds_total, a, s);
}

template <int TW, int TS>
static hipError_t launch_mode(const GemvArgs &a, int act, hipStream_t s) {
    const bool q8k = a.dot_act == ACT_Q8_K;
    if (a.mode == FFN_GATE_UP_NORM)
        return q8k ? launch_gu_t<TW, TS, ACT_Q8_K>(a, s) : launch_gu_t<TW, TS, ACT_Q8_1>(a, s);
    if (q8k) return act == ACT_F32 ? launch_dn_t<TW, TS, ACT_F32, ACT_Q8_K>(a, s) : hipErrorInvalidValue;
    if (act == ACT_F32) return launch_dn_t<TW, TS, ACT_F32, ACT_Q8_1>(a, s);
    return launch_dn_t<TW, TS, ACT_Q8_1, ACT_Q8_1>(a, s);
}

template <int TW>
static hipError_t launch_ts(const GemvArgs &a, int ts, int act, hipStream_t s) {
    switch (ts) {
        case 0: return launch_mode<TW, 0>(a, act, s);
        case T_Q2_K: return launch_mode<TW, T_Q2_K>(a, act, s);
        case T_Q3_K: return launch_mode<TW, T_Q3_K>(a, act, s);
        case T_Q4_K: return launch_mode<TW, T_Q4_K>(a, act, s);
        case T_Q5_K: return launch_mode<TW, T_Q5_K>(a, act, s);
        case T_Q6_K: return launch_mode<TW, T_Q6_K>(a, act, s);
        default: return hipErrorInvalidValue;
    }
}

static uint32_t round16(uint32_t b) { return (b + 15u) & ~15u; }

// Tiling and LDS layout of the fused kernels; returns hipErrorInvalidValue when
// the shape does not fit (the host validated types and alignment).
static hipError_t ffn_layout(GemvArgs &a, int tw, int ts, int act, int n_cu) {
    const TypeGeom g = type_geom(tw);
    const int nu = a.ncols / g.unit_elems;
    const uint32_t rb = (uint32_t) nu * (uint32_t) g.unit_bytes;
    const int nus = ts ? a.ncols / type_geom(ts).unit_elems : 1;
    const uint32_t rbs = ts ? (uint32_t) nus * (uint32_t) type_geom(ts).unit_bytes : 0u;
    const int nspan = a.has_gate || (ts && a.sh_gate) ? 2 : 1;
    a.rec = (a.stats || a.stamps || a.stamps_gate) ? 1 : 0;
    if (a.mode == FFN_GATE_UP_NORM) {
        if (a.ncols % RMS_CHUNK || a.ncols > 8192) return hipErrorInvalidValue;
        // the normalized row: q8_1 blocks, or q8_K blocks (one per 256 values) for q8_K dots
        const uint32_t yrow = (uint32_t) (a.ncols / 256) * (a.dot_act == ACT_Q8_K ? Q8K_LDS_STRIDE : Q8_1_LDS_STRIDE);
        const uint32_t common = round16(yrow) + 32u + 4u * 32u + 4u * 32u + 2u * (uint32_t) (a.ncols / 16);
        int rps, sh_rps;
        if (a.hq) {
            // workgroups of exactly one q8_1 block of rows: steps of a power-of-two row count
            int r = 1;
            while (2 * r <= WAVE / nu && 2 * r <= 32) r *= 2;
            if (ts) {
                int rs = 1;
                while (2 * rs <= WAVE / nus && 2 * rs <= 32) rs *= 2;
                if (rs < r) r = rs;
            }
            if (32 / r > FFN_GU_MAX_WAVES || a.nrows % 32) return hipErrorInvalidValue;
            rps = sh_rps = r;
            a.nwaves = 32 / r;
        } else {
            // shared steps of at most a routed step's bytes (the shared matrix rows are often
            // wider, a larger type): every wave's span is then about the same size
            rps = WAVE / nu;
            sh_rps = 0;
            if (ts) {
                sh_rps = (int) ((uint32_t) rps * rb / rbs);
                sh_rps = sh_rps < 1 ? 1 : (sh_rps > WAVE / nus ? WAVE / nus : sh_rps);
            }
        }
        for (;;) {
            a.tiles_per_pick = (a.nrows + rps - 1) / rps;
            a.sh_tiles_per_tok = ts ? (a.nrows + sh_rps - 1) / sh_rps : 0;
            a.tiles_per_tok = a.sh_tiles_per_tok + a.n_used * a.tiles_per_pick;
            if (!a.hq) {
                // mixed workgroups: a token's steps spread over every CU (one workgroup per CU, each
                // with an even share of the routed steps, then of the shared steps), more
                // workgroups when a share would exceed FFN_GU_MAX_WAVES steps
                const int NR = a.n_used * a.tiles_per_pick, NS = a.sh_tiles_per_tok;
                int G = n_cu / a.n_tok;
                G = G < 1 ? 1 : G;
                while ((NR + G - 1) / G + (NS + G - 1) / G > FFN_GU_MAX_WAVES) ++G;
                a.wg_per_tok = G;
                a.nwaves = (NR + G - 1) / G + (NS + G - 1) / G;
            }
            // spans sized to the 16-byte chunk the DMA writes last (+ lead-in and over-read)
            const uint32_t sr = round16((uint32_t) rps * rb + 20u);
            const uint32_t ss = ts ? round16((uint32_t) sh_rps * rbs + 20u) : 0u;
            a.lds_span = sr > ss ? sr : ss;
            a.lds_wave = (uint32_t) nspan * a.lds_span;
            if ((uint32_t) a.nwaves * a.lds_wave + common <= FFN_LDS_MAX) break;
            if (a.hq) return hipErrorInvalidValue;
            if (ts && ss >= sr && sh_rps > 1) --sh_rps;
            else if (rps > 1) --rps;
            else return hipErrorInvalidValue;
        }
        a.rps = rps;
        a.sh_rps = sh_rps;
        a.mixed_wg = a.hq ? 0 : 1;
        a.sh_per_wg = 0;
        if (a.hq) {
            // shared-expert workgroups of about the bytes of a routed one: the shared matrix rows
            // are often wider (a larger type), and the launch ends with its slowest workgroup.
            // Its q8_1 blocks (hq_sh) need whole 32-row workgroups.
            if (ts) {
                const double rstep = (double) rps * rb, sstep = (double) sh_rps * rbs;
                int n = a.hq_sh ? a.nwaves : (int) (a.nwaves * rstep / sstep);   // at most a routed one's bytes
                a.sh_per_wg = n < 1 ? 1 : (n > a.nwaves ? a.nwaves : n);
            }
            const int nsh_wg = a.sh_per_wg ? (a.sh_tiles_per_tok + a.sh_per_wg - 1) / a.sh_per_wg : 0;
            a.wg_per_tok = nsh_wg + (a.tiles_per_tok - a.sh_tiles_per_tok + a.nwaves - 1) / a.nwaves;
        }
        a.lds_y = (uint32_t) a.nwaves * a.lds_wave;
        a.lds_part = a.lds_y + round16(yrow);
        a.lds_total = a.lds_part + 32u + 4u * 32u + 4u * 32u + 2u * (uint32_t) (a.ncols / 16);
        a.n_tiles = a.tiles_per_tok * a.n_tok;
        return hipSuccess;
    }
    // FFN_DOWN_COMBINE: one wave per pick (+ the shared expert), common rows per step
    a.nwaves = a.n_used + (ts ? 1 : 0);
    if (a.nwaves > FFN_DN_MAX_WAVES || nspan != 1) return hipErrorInvalidValue;
    int rps = WAVE / nu;
    if (ts && WAVE / nus < rps) rps = WAVE / nus;
    // enough workgroups for every CU: at most nrows * n_tok / 256 rows each
    const int fill = (a.nrows * a.n_tok + 255) / 256;
    if (fill < rps) rps = fill < 1 ? 1 : fill;
    const uint32_t q8_row = a.dot_act == ACT_Q8_K ? (uint32_t) (a.ncols / 256 * Q8K_LDS_STRIDE) : (uint32_t) (a.ncols / 32 * 36);
    const uint32_t q8_bytes = act == ACT_F32 || (ts && a.sh_act_f32) ? round16(q8_row) : 0u;
    const uint32_t arow_max = ts && a.sh_act_row_bytes > a.act_row_bytes ? a.sh_act_row_bytes : a.act_row_bytes;
    for (;;) {
        const uint32_t sr = span_bytes((uint32_t) rps, rb);
        const uint32_t ss = ts ? span_bytes((uint32_t) rps, rbs) : 0u;
        a.lds_span = sr > ss ? sr : ss;
        a.lds_act = a.lds_span;
        a.lds_q8 = a.lds_act + round_up_1k(arow_max + 20u);
        a.lds_sums = a.lds_q8 + q8_bytes;
        a.lds_wave = a.lds_sums + round16(2u * (uint32_t) (a.ncols / 16));
        a.lds_part = (uint32_t) a.nwaves * a.lds_wave;
        a.lds_total = a.lds_part + 4u * (uint32_t) (a.nwaves * rps);
        if (a.lds_total <= FFN_LDS_MAX) break;
        if (rps > 1) --rps;
        else return hipErrorInvalidValue;
    }
    a.rps = rps;
    a.sh_rps = rps;
    a.tiles_per_pick = (a.nrows + rps - 1) / rps;
    a.sh_tiles_per_tok = ts ? a.tiles_per_pick : 0;
    a.wg_per_tok = a.tiles_per_pick;
    a.tiles_per_tok = a.wg_per_tok;
    a.n_tiles = a.wg_per_tok * a.n_tok;
    return hipSuccess;
}

// Compute units of the current GPU (looked up once per GPU; 256 when the query fails).
static int cu_count() {
    static std::mutex m;
    static int cache[MAX_DEVICES] = {};
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= MAX_DEVICES) return 256;
    std::lock_guard<std::mutex> lock(m);
    if (!cache[d]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess || n <= 0) n = 256;
        cache[d] = n;
    }
    return cache[d];
}

// Fused decode launch (a.mode != FFN_NONE): tiling, LDS layout, dispatch on the
// routed type (K-quants) and the shared-expert type (none or a K-quant).
int launch_ffn(GemvArgs a, int tw, int ts, int act, void *stream) {
    if (ts == 0 || !a.sh_up) ts = 0;
    if (a.mode == FFN_GATE_UP_NORM) act = ACT_Q8_1;
    a.act_row_bytes = act == ACT_Q8_1 ? (uint32_t) (a.ncols / 32 * 36) : (uint32_t) a.ncols * 4u;
    a.sh_act_row_bytes = act == ACT_Q8_1 && !a.sh_act_f32 ? (uint32_t) (a.ncols / 32 * 36) : (uint32_t) a.ncols * 4u;
    hipError_t err = ffn_layout(a, tw, ts, act, cu_count());
    if (err != hipSuccess) return (int) err;
    if (a.n_tiles <= 0) return (int) hipSuccess;
    hipStream_t s = (hipStream_t) stream;
    switch (tw) {
        case T_Q2_K: return (int) launch_ts<T_Q2_K>(a, ts, act, s);
        case T_Q3_K: return (int) launch_ts<T_Q3_K>(a, ts, act, s);
        case T_Q4_K: return (int) launch_ts<T_Q4_K>(a, ts, act, s);
        case T_Q5_K: return (int) launch_ts<T_Q5_K>(a, ts, act, s);
        case T_Q6_K: return (int) launch_ts<T_Q6_K>(a, ts, act, s);
        default: return (int) hipErrorInvalidValue;
    }
}

}  // namespace mc
