// mc_step.h -- the per-wave "step" of the decode GEMV, shared by the plain
// MUL_MAT_ID kernel (mc_kernels.hip) and the fused decode kernels (mc_ffn.hip).
//
// A step is rows [row0, row0 + rows_per_step) of one expert matrix pair
// (up [+ gate]) for one pick (token t, slot c), or of the shared expert:
//   step_locate  -> which pick / rows (no memory access)
//   step_issue   -> routing id and weight addresses (scalar loads), then the
//                   gate span and the up span streamed into LDS (buffer->LDS DMA)
//   step_dots    -> the lane-unit dots against an activation row already in LDS
//                   (gate dot while the up span lands), row sums in fixed order
//   step_store   -> scale -> bias -> GLU epilogue and the dst / shared_dst store
//                   (kernels/moe-cache.cu:240-284)
// record_picks is the pick recorder (stamps, hit counter, canonical miss log).
#ifndef MC_STEP_H
#define MC_STEP_H

#include <hip/hip_runtime.h>

#include "mc_core.h"
#include "mc_internal.h"

namespace mc {

// ---------------------------------------------------------------------------
// pick recorder: stamps, hit count, canonical miss log (kernels/moe-cache.cu:159-204)
// ---------------------------------------------------------------------------

// One wave.  Miss-log entries are written at canonical positions (pick order,
// token-major, up before gate): one legal ordering of the reference's
// atomicAdd-ordered log; the multiset and the counters are the reference's.
// The gate is recorded only when it has a cache entry of its own
// (cache_id_gate >= 0): a device-resident gate reached through a resident
// table for addressing leaves no stamp, hit or miss, as the reference's null
// tbl_gate does (kernels/moe-cache.cu:178-201, :804).
static __device__ void record_picks(const GemvArgs &a) {
    const int lane = threadIdx.x % WAVE;
    const int n_picks = a.n_tok * a.n_used;
    const u32 clk = a.clock ? *a.clock : 0u;
    const bool rec_gate = a.tbl_gate && a.cache_id_gate >= 0;
    for (int p0 = 0; p0 < n_picks; p0 += WAVE) {
        const int p = p0 + lane;
        int e = -1;
        u32 miss_up = 0, miss_gate = 0, hits = 0;
        if (p < n_picks) {
            const int t = p / a.n_used, c = p % a.n_used;
            e = a.ids[c + (int64_t) t * a.ids_stride];
            if (e >= 0 && e < a.n_experts) {
                const uint64_t pu = a.tbl[e];
                if (a.stamps) a.stamps[e] = clk;
                miss_up = (u32) (pu & 1u);
                hits += 1u - miss_up;
                if (rec_gate) {
                    const uint64_t pg = a.tbl_gate[e];
                    if (a.stamps_gate) a.stamps_gate[e] = clk;
                    miss_gate = (u32) (pg & 1u);
                    hits += 1u - miss_gate;
                }
            }
        }
        if (!a.stats) continue;
        // exclusive prefix sum of miss counts across the wave (pick order)
        const u32 nm = miss_up + miss_gate;
        u32 incl = nm;
#pragma unroll
        for (int off = 1; off < WAVE; off <<= 1) {
            const u32 v = (u32) __shfl_up((int) incl, off, WAVE);
            if (lane >= off) incl += v;
        }
        const u32 total = (u32) __shfl((int) incl, WAVE - 1, WAVE);
        u32 hsum = hits;
#pragma unroll
        for (int off = WAVE / 2; off > 0; off >>= 1) hsum += (u32) __shfl_xor((int) hsum, off, WAVE);
        u32 start = 0;
        if (lane == 0) {
            start = atomicAdd(a.stats, total);
            if (hsum) atomicAdd(a.stats + HIT_WORD, hsum);
        }
        start = (u32) __shfl((int) start, 0, WAVE);
        const u32 pos = start + incl - nm;
        if (miss_up && pos < (u32) MISS_CAP) a.stats[LOG_BASE + pos] = ((u32) a.cache_id << 12) | (u32) e;
        if (miss_gate && pos + miss_up < (u32) MISS_CAP)
            a.stats[LOG_BASE + pos + miss_up] = ((u32) a.cache_id_gate << 12) | (u32) e;
    }
}

// Weight addresses of expert e: affine for device-resident tensors, else the
// tagged table entries (LSB cleared), both entries read before either is
// waited on so the two scalar loads overlap.
__device__ __forceinline__ void resolve_expert(const GemvArgs &a, int e, const uint8_t *&wup, const uint8_t *&wgate) {
    if (a.w_base) {
        wup = a.w_base + (uint64_t) e * a.expert_bytes;
        wgate = a.has_gate ? a.w_gate_base + (uint64_t) e * a.expert_bytes : nullptr;
        return;
    }
    const uint64_t *tg = a.has_gate ? a.tbl_gate : a.tbl;
    uint64_t pu, pg;
    // the compiler would wait for the first scalar load before issuing the second
    asm volatile("s_load_dwordx2 %0, %2, 0x0\n\t"
                 "s_load_dwordx2 %1, %3, 0x0\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&s"(pu), "=&s"(pg)
                 : "s"(a.tbl + e), "s"(tg + e)
                 : "memory");
    wup = (const uint8_t *) (uintptr_t) (pu & ~(uint64_t) 1);
    wgate = a.has_gate ? (const uint8_t *) (uintptr_t) (pg & ~(uint64_t) 1) : nullptr;
}

struct StepCtx {
    int t, c;                     // token, slot (c = 0 for the shared expert)
    int e;                        // expert id (routed)
    int row0, rps, nrows_here;
    bool shared, valid;
    const uint8_t *wup, *wgate;   // weight matrices (gate null: none)
    u32 start;                    // byte offset of row0 in the matrices
    int n_gate, n_up;             // DMA instructions of the gate span and of the up span (issued last)
};

// Which pick and rows `tile` covers: routed tiles are pick-major
// (pick = t * n_used + c, then row tiles), shared tiles token-major.
__device__ __forceinline__ StepCtx step_locate(const GemvArgs &a, bool shared, int tile) {
    StepCtx s;
    s.shared = shared;
    s.e = 0;
    s.valid = true;
    s.wup = nullptr;
    s.wgate = nullptr;
    s.start = 0;
    s.n_gate = 0;
    s.n_up = 0;
    if (!shared) {
        s.rps = a.rps;
        const int pick = tile / a.tiles_per_pick;
        s.row0 = (tile % a.tiles_per_pick) * s.rps;
        s.t = pick / a.n_used;
        s.c = pick % a.n_used;
    } else {
        s.rps = a.sh_rps;
        s.t = tile / a.sh_tiles_per_tok;
        s.row0 = (tile % a.sh_tiles_per_tok) * s.rps;
        s.c = 0;
    }
    s.nrows_here = min(s.rps, a.nrows - s.row0);
    return s;
}

// Routing id and weight addresses.  An out-of-range expert id leaves valid = false.
__device__ __forceinline__ void step_resolve(const GemvArgs &a, StepCtx &s) {
    if (!s.shared) {
        s.e = sload(a.ids + s.c + (int64_t) s.t * a.ids_stride);
        if (s.e < 0 || s.e >= a.n_experts) {
            s.valid = false;
            return;
        }
        resolve_expert(a, s.e, s.wup, s.wgate);
    } else {
        s.wup = a.sh_up;
        s.wgate = a.sh_gate;
    }
}

// The DMA of the gate span (to span + lds_span) and the up span (to span) of a valid step
// (MASK_TAIL: dma_span's 16-byte destination sizing).
template <int T, bool MASK_TAIL = false>
__device__ __forceinline__ void step_dma(const GemvArgs &a, StepCtx &s, uint8_t *span) {
    constexpr TypeGeom G = type_geom(T);
    const int nu = a.ncols / G.unit_elems;
    const u32 RB = (u32) nu * G.unit_bytes;
    const u32 mbytes = (u32) (s.shared ? a.sh_matrix_bytes : a.expert_bytes);
    s.start = (u32) s.row0 * RB;
    const u32 nbytes = (u32) s.nrows_here * RB;
    if (s.wgate) s.n_gate = dma_span<T, MASK_TAIL>(s.wgate, mbytes, s.start, nbytes, span + a.lds_span);
    s.n_up = dma_span<T, MASK_TAIL>(s.wup, mbytes, s.start, nbytes, span);
}

// step_resolve, then step_dma (nothing is issued for an out-of-range expert id).
template <int T>
__device__ __forceinline__ void step_issue(const GemvArgs &a, StepCtx &s, uint8_t *span) {
    step_resolve(a, s);
    if (s.valid) step_dma<T>(a, s, span);
}

// The wave's dots for a valid step.  On entry the activation row (q8_1 or q8_K
// blocks) is in LDS at arow and, when there is a gate, the gate span has landed
// (the caller waited for at most n_up outstanding loads); the up span is waited
// for here.  Returns the row sums (valid in lane row_local * nu of each row).
template <int T, int AQ, bool S16 = false, int ASTRIDE = 0>
__device__ __forceinline__ void step_dots(const GemvArgs &a, const StepCtx &s, const uint8_t *span,
                                          const uint8_t *arow, float &su, float &sg, const int16_t *s16 = nullptr) {
    constexpr TypeGeom G = type_geom(T);
    constexpr int UE = G.unit_elems;
    // activation bytes per unit in the row (ASTRIDE: a padded LDS layout)
    constexpr int AUB = ASTRIDE ? ASTRIDE : AQ == ACT_Q8_1 ? UE / 32 * 36 : 292;
    const int lane = threadIdx.x % WAVE;
    const int nu = a.ncols / UE;
    const int row_local = lane / nu, col = lane % nu;
    const bool active = row_local < s.nrows_here;
    const int unit = row_local * nu + col;
    const uint8_t *aslice = arow + (u32) col * AUB;
    Act<UE> A;
    float pu = 0.0f, pg = 0.0f;
    // precomputed 16-value activation sums of the unit, when the caller has them (K-quant units)
    // (q8_K units carry their own bsums)
    const int16_t *us16 = S16 && AQ != ACT_Q8_K ? s16 + (u32) col * (UE / 16) : nullptr;
    if (s.wgate) {
        if (active) {
            load_act_lds<UE, AQ, S16>(A, aslice, us16);
            pg = span_unit_dot<T, AQ>(span + a.lds_span, span_lead(s.wgate, s.start), unit, A);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (active) pu = span_unit_dot<T, AQ>(span, span_lead(s.wup, s.start), unit, A);
    } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (active) {
            load_act_lds<UE, AQ, S16>(A, aslice, us16);
            pu = span_unit_dot<T, AQ>(span, span_lead(s.wup, s.start), unit, A);
        }
    }
    // row sums across the nu lanes of each row (cross-lane adds, no LDS)
    su = row_group_sum(pu, nu);
    sg = s.wgate ? row_group_sum(pg, nu) : 0.0f;
}

// Epilogue value of row `row` of a routed pick: scale -> bias -> GLU.
__device__ __forceinline__ float routed_value(const GemvArgs &a, const StepCtx &s, int row, float su, float sg) {
    float up = su;
    if (a.x_scale) up *= a.x_scale[s.e];
    if (a.x_bias) up += a.x_bias[(int64_t) s.e * a.bias_stride + row];
    if (!s.wgate) return up;
    float g = sg;
    if (a.gate_scale) g *= a.gate_scale[s.e];
    if (a.gate_bias) g += a.gate_bias[(int64_t) s.e * a.bias_stride + row];
    return glu_apply(a.glu_op, g, up, a.glu_limit);
}

// The output value of the row this lane reports (the first lane of each row group);
// returns the row's index within the step, or -1 for the other lanes.
template <int T>
__device__ __forceinline__ int step_value(const GemvArgs &a, const StepCtx &s, float su, float sg, float &v) {
    const int lane = threadIdx.x % WAVE;
    const int nu = a.ncols / type_geom(T).unit_elems;
    const int row_local = lane / nu, col = lane % nu;
    if (row_local >= s.nrows_here || col != 0) return -1;
    const int row = s.row0 + row_local;
    v = s.shared ? (s.wgate ? glu_apply(a.glu_op, sg, su, a.glu_limit) : su) : routed_value(a, s, row, su, sg);
    return row_local;
}

// Stores the step's rows to dst (routed) or sh_dst (shared); returns step_value's row.
template <int T>
__device__ __forceinline__ int step_store(const GemvArgs &a, const StepCtx &s, float su, float sg, float &v) {
    const int rl = step_value<T>(a, s, su, sg, v);
    if (rl < 0) return rl;
    const int row = s.row0 + rl;
    if (!s.shared) a.dst[(int64_t) s.c * a.stride_channel_dst + (int64_t) s.t * a.stride_col_dst + row] = v;
    else a.sh_dst[(int64_t) s.t * a.sh_stride_col_dst + row] = v;
    return rl;
}

template <int T>
__device__ __forceinline__ void step_store(const GemvArgs &a, const StepCtx &s, float su, float sg) {
    float v;
    step_store<T>(a, s, su, sg, v);
}

}  // namespace mc

#endif
