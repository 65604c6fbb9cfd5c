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

#include "mc_internal.h"

namespace mc {

typedef uint32_t u32;
typedef int32_t i32;

// ---------------------------------------------------------------------------
// small device helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ float h2f(u32 bits16) {
    return (float) __builtin_bit_cast(_Float16, (uint16_t) (bits16 & 0xFFFFu));
}

__device__ __forceinline__ uint16_t f2h_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16) f);   // v_cvt_f16_f32, round to nearest even
}

__device__ __forceinline__ int sdot4(u32 a, u32 b, int c) {
    return __builtin_amdgcn_sdot4((int) a, (int) b, c, false);
}

__device__ __forceinline__ u32 byte_of(u32 w, int i) { return (w >> (8 * i)) & 0xFFu; }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, u32 nbytes) {
    // gfx9 raw buffer: stride 0, num_records in bytes, dword3 = 0x00020000
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short) 0, (int) nbytes, 0x00020000);
}

__device__ __forceinline__ u32 bload(__amdgpu_buffer_rsrc_t r, u32 off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// ---------------------------------------------------------------------------
// activation slice of one lane: UE int8 values, one scale per 32, sums per 16
// ---------------------------------------------------------------------------

template <int UE>
struct Act {
    u32 q[UE / 4];
    float d[UE / 32];
    int s16[UE / 16];
};

template <int UE, int ACT>
__device__ __forceinline__ void load_act(Act<UE> &A, __amdgpu_buffer_rsrc_t r, u32 row_off, int col) {
    if constexpr (ACT == ACT_Q8_1) {
#pragma unroll
        for (int b = 0; b < UE / 32; ++b) {
            const u32 off = row_off + (u32) (col * (UE / 32) + b) * 36u;
            A.d[b] = h2f(bload(r, off));
#pragma unroll
            for (int k = 0; k < 8; ++k) A.q[8 * b + k] = bload(r, off + 4u + 4u * k);
        }
    } else {
        static_assert(UE == 256, "q8_K activations pair with 256-value units");
        const u32 off = row_off + (u32) col * 292u;
        const float d = __builtin_bit_cast(float, bload(r, off));
#pragma unroll
        for (int b = 0; b < 8; ++b) A.d[b] = d;
#pragma unroll
        for (int k = 0; k < 64; ++k) A.q[k] = bload(r, off + 4u + 4u * k);
    }
#pragma unroll
    for (int s = 0; s < UE / 16; ++s) {
        int t = sdot4(A.q[4 * s + 0], 0x01010101u, 0);
        t = sdot4(A.q[4 * s + 1], 0x01010101u, t);
        t = sdot4(A.q[4 * s + 2], 0x01010101u, t);
        A.s16[s] = sdot4(A.q[4 * s + 3], 0x01010101u, t);
    }
}

// ---------------------------------------------------------------------------
// LDS word readers for one unit
// ---------------------------------------------------------------------------

struct WordsAligned {            // unit starts on a 4-byte boundary
    const u32 *p;
    __device__ __forceinline__ u32 operator[](int i) const { return p[i]; }
};

struct WordsShifted {            // unit starts on a 2-byte boundary: realign with v_alignbyte
    const u32 *p;
    u32 sh;                      // byte shift 0..3
    __device__ __forceinline__ u32 operator[](int i) const { return __builtin_amdgcn_alignbyte(p[i + 1], p[i], sh); }
};

// ---------------------------------------------------------------------------
// per-type unit dot products
// ---------------------------------------------------------------------------

// Q2_K: scales[16] | qs[64] | d | dmin.  Element i = 128h + 32j + l uses
// (qs[32h + l] >> 2j) & 3 and sub-block scale byte i >> 4 (lo 4: scale, hi 4: min).
template <int ACT, class W>
__device__ __forceinline__ float dot_q2_K(const W &w, const Act<256> &A) {
    const u32 dm = w[20];
    const float d = h2f(dm), dmin = h2f(dm >> 16);
    u32 sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[i] = w[i];
    float accI = 0.0f, accM = 0.0f;
    int isum = 0, msum = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        u32 q[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) q[k] = w[4 + 8 * h + k];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int g = 4 * h + j;
            // j < 3: keep the 2-bit field in place (value * 4^j); j == 3: shift down
            const int jj = j < 3 ? j : 0;
            int d0 = 0, d1 = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const u32 v0 = j < 3 ? (q[k] & (0x03030303u << (2 * j))) : ((q[k] >> 6) & 0x03030303u);
                const u32 v1 = j < 3 ? (q[k + 4] & (0x03030303u << (2 * j))) : ((q[k + 4] >> 6) & 0x03030303u);
                d0 = sdot4(v0, A.q[8 * g + k], d0);
                d1 = sdot4(v1, A.q[8 * g + 4 + k], d1);
            }
            const u32 b0 = byte_of(sc[(2 * g) >> 2], (2 * g) & 3);
            const u32 b1 = byte_of(sc[(2 * g + 1) >> 2], (2 * g + 1) & 3);
            const int is = (int) (b0 & 0xF) * d0 + (int) (b1 & 0xF) * d1;
            const int ms = (int) (b0 >> 4) * A.s16[2 * g] + (int) (b1 >> 4) * A.s16[2 * g + 1];
            if constexpr (ACT == ACT_Q8_K) {
                isum += is >> (2 * jj);
                msum += ms;
            } else {
                const float fi = (float) is * (jj == 0 ? 1.0f : (jj == 1 ? 0.25f : 0.0625f));
                accI = fmaf(A.d[g], fi, accI);
                accM = fmaf(A.d[g], (float) ms, accM);
            }
        }
    }
    if constexpr (ACT == ACT_Q8_K) {
#pragma clang fp contract(off)
        const float dall = A.d[0] * d, dmn = A.d[0] * dmin;
        return dall * (float) isum - dmn * (float) msum;
    } else {
        return d * accI - dmin * accM;
    }
}

// Q3_K: hmask[32] | qs[64] | scales[12] | d.  Element i = 128h + 32j + l:
// low2 = (qs[32h + l] >> 2j) & 3, hbit = hmask[l] bit (4h + j), code = low2 + 4*hbit - 4;
// 6-bit scale of sub-block s: low 4 from byte s (s < 8) or byte s-8 >> 4, high 2 from
// byte 8 + (s & 3) bits 2*(s >> 2); value - 32.
template <int ACT, class W>
__device__ __forceinline__ float dot_q3_K(const W &w, const Act<256> &A) {
    const float d = h2f(w[27]);
    const u32 A0 = w[24], A1 = w[25], A2 = w[26];
    u32 S[4];
    S[0] = (A0 & 0x0F0F0F0Fu) | ((A2 & 0x03030303u) << 4);
    S[1] = (A1 & 0x0F0F0F0Fu) | (((A2 >> 2) & 0x03030303u) << 4);
    S[2] = ((A0 >> 4) & 0x0F0F0F0Fu) | (((A2 >> 4) & 0x03030303u) << 4);
    S[3] = ((A1 >> 4) & 0x0F0F0F0Fu) | (((A2 >> 6) & 0x03030303u) << 4);
    u32 hm[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) hm[k] = w[k];
    float acc = 0.0f;
    int isum = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        u32 q[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) q[k] = w[8 + 8 * h + k];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int g = 4 * h + j;
            int d0 = 0, d1 = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const u32 u0 = ((q[k] >> (2 * j)) & 0x03030303u) | (((hm[k] >> (4 * h + j)) & 0x01010101u) << 2);
                const u32 u1 = ((q[k + 4] >> (2 * j)) & 0x03030303u) | (((hm[k + 4] >> (4 * h + j)) & 0x01010101u) << 2);
                d0 = sdot4(u0, A.q[8 * g + k], d0);
                d1 = sdot4(u1, A.q[8 * g + 4 + k], d1);
            }
            d0 -= 4 * A.s16[2 * g];
            d1 -= 4 * A.s16[2 * g + 1];
            const int s0 = 2 * g, s1 = 2 * g + 1;
            const int sc0 = (int) byte_of(S[s0 >> 2], s0 & 3) - 32;
            const int sc1 = (int) byte_of(S[s1 >> 2], s1 & 3) - 32;
            const int is = sc0 * d0 + sc1 * d1;
            if constexpr (ACT == ACT_Q8_K) isum += is;
            else acc = fmaf(A.d[g], (float) is, acc);
        }
    }
    if constexpr (ACT == ACT_Q8_K) {
#pragma clang fp contract(off)
        const float dall = A.d[0] * d;
        return dall * (float) isum;
    } else {
        return d * acc;
    }
}

// 6-bit scales/mins of Q4_K / Q5_K from the 12 scale bytes (three words S0..S2):
// sub-block j < 4: sc = b[j] & 63, m = b[j+4] & 63;
// j >= 4: sc = (b[j+4] & 15) | (b[j-4] >> 6) << 4, m = (b[j+4] >> 4) | (b[j] >> 6) << 4.
__device__ __forceinline__ void kq_scales(u32 S0, u32 S1, u32 S2, u32 &SC0, u32 &SC1, u32 &M0, u32 &M1) {
    SC0 = S0 & 0x3F3F3F3Fu;
    M0 = S1 & 0x3F3F3F3Fu;
    SC1 = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
    M1 = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
}

// Q4_K: d | dmin | scales[12] | qs[128].  Chunk c = i / 64: low nibbles of
// qs[32c..32c+31] are sub-block 2c, high nibbles sub-block 2c+1.
// Q5_K: d | dmin | scales[12] | qh[32] | qs[128]; high bit of element l of
// sub-block g is qh[l] bit g.
template <int ACT, bool Q5, class W>
__device__ __forceinline__ float dot_q45_K(const W &w, const Act<256> &A) {
    const u32 dm = w[0];
    const float d = h2f(dm), dmin = h2f(dm >> 16);
    u32 SC0, SC1, M0, M1;
    kq_scales(w[1], w[2], w[3], SC0, SC1, M0, M1);
    constexpr int QS = Q5 ? 12 : 4;
    float accI = 0.0f, accM = 0.0f;
    int isum = 0, msum = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        u32 q[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) q[k] = w[QS + 8 * c + k];
#pragma unroll
        for (int hi = 0; hi < 2; ++hi) {
            const int g = 2 * c + hi;
            int dot = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                u32 v = hi ? ((q[k] >> 4) & 0x0F0F0F0Fu) : (q[k] & 0x0F0F0F0Fu);
                if constexpr (Q5) v |= ((w[4 + k] >> g) & 0x01010101u) << 4;
                dot = sdot4(v, A.q[8 * g + k], dot);
            }
            const int sc = (int) byte_of(g < 4 ? SC0 : SC1, g & 3);
            const int m = (int) byte_of(g < 4 ? M0 : M1, g & 3);
            const int is = sc * dot;
            const int ms = m * (A.s16[2 * g] + A.s16[2 * g + 1]);
            if constexpr (ACT == ACT_Q8_K) {
                isum += is;
                msum += ms;
            } else {
                accI = fmaf(A.d[g], (float) is, accI);
                accM = fmaf(A.d[g], (float) ms, accM);
            }
        }
    }
    if constexpr (ACT == ACT_Q8_K) {
#pragma clang fp contract(off)
        const float dall = A.d[0] * d, dmn = A.d[0] * dmin;
        return dall * (float) isum - dmn * (float) msum;
    } else {
        return d * accI - dmin * accM;
    }
}

// Q6_K: ql[128] | qh[64] | scales[16] (int8) | d.  Element i = 128n + 32q + l:
// low 4 = ql[64n + 32(q & 1) + l] (q >= 2: high nibble), high 2 = (qh[32n + l] >> 2q) & 3,
// code - 32; scale byte i >> 4.
template <int ACT, class W>
__device__ __forceinline__ float dot_q6_K(const W &w, const Act<256> &A) {
    const float d = h2f(w[52]);
    u32 sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[i] = w[48 + i];
    float acc = 0.0f;
    int isum = 0;
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        u32 qh[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) qh[k] = w[32 + 8 * n + k];
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const int g = 4 * n + qq;
            int d0 = 0, d1 = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const u32 ql = w[16 * n + 8 * (qq & 1) + k];
                const u32 v = ((qq >> 1) ? ((ql >> 4) & 0x0F0F0F0Fu) : (ql & 0x0F0F0F0Fu)) |
                              (((qh[k] >> (2 * qq)) & 0x03030303u) << 4);
                if (k < 4) d0 = sdot4(v, A.q[8 * g + k], d0);
                else       d1 = sdot4(v, A.q[8 * g + k], d1);
            }
            d0 -= 32 * A.s16[2 * g];
            d1 -= 32 * A.s16[2 * g + 1];
            const int s0 = 2 * g, s1 = 2 * g + 1;
            const int sc0 = (int) (int8_t) byte_of(sc[s0 >> 2], s0 & 3);
            const int sc1 = (int) (int8_t) byte_of(sc[s1 >> 2], s1 & 3);
            const int is = sc0 * d0 + sc1 * d1;
            if constexpr (ACT == ACT_Q8_K) isum += is;
            else acc = fmaf(A.d[g], (float) is, acc);
        }
    }
    if constexpr (ACT == ACT_Q8_K) {
#pragma clang fp contract(off)
        const float dall = A.d[0] * d;
        return dall * (float) isum;
    } else {
        return d * acc;
    }
}

// spread the low 4 bits of x to bit 0 of the 4 bytes
__device__ __forceinline__ u32 spread4(u32 x) { return ((x & 0xFu) * 0x00204081u) & 0x01010101u; }

// Legacy units: two 32-value blocks.  Q4_0 = d | qs[16] (low nibble: j, high: j+16),
// offset 8.  Q5_0 = d | qh[4] | qs[16] (5th bit of value j is qh bit j), offset 16.
// Q8_0 = d | int8 qs[32].
template <int T, class W>
__device__ __forceinline__ float dot_legacy(const W &w, const Act<64> &A) {
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        int sumi = 0;
        float dw;
        if constexpr (T == T_Q4_0) {
            // block 0 at byte 0 (qs at 2: realign), block 1 at byte 18 (qs at 20)
            dw = b == 0 ? h2f(w[0]) : h2f(w[4] >> 16);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const u32 q = b == 0 ? __builtin_amdgcn_alignbyte(w[k + 1], w[k], 2) : w[5 + k];
                sumi = sdot4(q & 0x0F0F0F0Fu, A.q[8 * b + k], sumi);
                sumi = sdot4((q >> 4) & 0x0F0F0F0Fu, A.q[8 * b + 4 + k], sumi);
            }
            sumi -= 8 * (A.s16[2 * b] + A.s16[2 * b + 1]);
        } else if constexpr (T == T_Q5_0) {
            // block 0 at byte 0 (qh at 2, qs at 6), block 1 at byte 22 (qh at 24, qs at 28)
            dw = b == 0 ? h2f(w[0]) : h2f(w[5] >> 16);
            const u32 qh = b == 0 ? __builtin_amdgcn_alignbyte(w[1], w[0], 2) : w[6];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const u32 q = b == 0 ? __builtin_amdgcn_alignbyte(w[k + 2], w[k + 1], 2) : w[7 + k];
                const u32 lo = (q & 0x0F0F0F0Fu) | (spread4(qh >> (4 * k)) << 4);
                const u32 hi = ((q >> 4) & 0x0F0F0F0Fu) | (spread4(qh >> (16 + 4 * k)) << 4);
                sumi = sdot4(lo, A.q[8 * b + k], sumi);
                sumi = sdot4(hi, A.q[8 * b + 4 + k], sumi);
            }
            sumi -= 16 * (A.s16[2 * b] + A.s16[2 * b + 1]);
        } else {
            // block 0 at byte 0 (qs at 2), block 1 at byte 34 (qs at 36)
            dw = b == 0 ? h2f(w[0]) : h2f(w[8] >> 16);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const u32 q = b == 0 ? __builtin_amdgcn_alignbyte(w[k + 1], w[k], 2) : w[9 + k];
                sumi = sdot4(q, A.q[8 * b + k], sumi);
            }
        }
        acc += (float) sumi * dw * A.d[b];
    }
    return acc;
}

template <int T, int ACT, class W>
__device__ __forceinline__ float unit_dot(const W &w, const Act<type_geom(T).unit_elems> &A) {
    if constexpr (T == T_Q2_K) return dot_q2_K<ACT>(w, A);
    else if constexpr (T == T_Q3_K) return dot_q3_K<ACT>(w, A);
    else if constexpr (T == T_Q4_K) return dot_q45_K<ACT, false>(w, A);
    else if constexpr (T == T_Q5_K) return dot_q45_K<ACT, true>(w, A);
    else if constexpr (T == T_Q6_K) return dot_q6_K<ACT>(w, A);
    else return dot_legacy<T>(w, A);
}

// ---------------------------------------------------------------------------
// GLU (kernels/moe-cache.cu:264-280; ggml unary definitions)
// ---------------------------------------------------------------------------

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float glu_apply(int op, float g, float up, float limit) {
    switch (op) {
        case 0: return up * (g > 0.0f ? g : 0.0f);                                                   // REGLU
        case 1: return up * (0.5f * g * (1.0f + tanhf(0.79788456080286535587989211986876f * g * (1.0f + 0.044715f * g * g)))); // GEGLU
        case 2: return up * silu_f(g);                                                               // SWIGLU
        case 3: {                                                                                    // SWIGLU_OAI
            const float x = fminf(g, 7.0f);
            const float u = fmaxf(fminf(up, 7.0f), -7.0f);
            return x / (1.0f + expf(-x * 1.702f)) * (1.0f + u);
        }
        case 4: return up * (0.5f * g * (1.0f + erff(g * 0.70710678118654752440f)));               // GEGLU_ERF
        case 5: return up * (g / (1.0f + expf(-1.702f * g)));                                       // GEGLU_QUICK
        case 6: {                                                                                    // SWIGLU_CLAMP
            const float x = fminf(g, limit);
            const float u = fmaxf(fminf(up, limit), -limit);
            return silu_f(x) * u;
        }
        default: return up * g;
    }
}

// ---------------------------------------------------------------------------
// pick recorder (workgroup 0): stamps, hit count, canonical miss log
// ---------------------------------------------------------------------------

__device__ void record_picks(const GemvArgs &a) {
    const int lane = threadIdx.x;
    const int n_picks = a.n_tok * a.n_used;
    const u32 clk = a.clock ? *a.clock : 0u;
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
                if (a.tbl_gate) {
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

// ---------------------------------------------------------------------------
// one step of one matrix pair (up [+ gate]) for one pick
// ---------------------------------------------------------------------------

typedef __attribute__((address_space(3))) void lds_void_t;

template <int T>
__device__ __forceinline__ void dma_span(const uint8_t *base, u32 base_bytes, u32 start, u32 nbytes, uint8_t *lds) {
    // stream [start, start + nbytes) of the matrix at `base` into lds: lds[x] = byte (start & ~15) + x
    const uintptr_t abase = (uintptr_t) base & ~(uintptr_t) 15;
    const u32 skew = (u32) ((uintptr_t) base - abase);
    const __amdgpu_buffer_rsrc_t r = make_rsrc((const void *) abase, base_bytes + skew);
    const u32 a0 = (start + skew) & ~15u;
    const u32 lead = (start + skew) - a0;
    const int rounds = (int) ((lead + nbytes + 1023u) >> 10);
    constexpr int MAXR = span_lds_bytes(T) / 1024;
    const u32 lane_off = a0 + 16u * threadIdx.x;
#pragma unroll
    for (int i = 0; i < MAXR; ++i) {
        if (i < rounds) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *) (lds + 1024 * i), 16, lane_off + 1024u * i, 0, 0, 0);
        }
    }
}

template <int T, int ACT>
__device__ __forceinline__ void run_step(const GemvArgs &a, uint8_t *lds, float *red, bool shared, int tile) {
    constexpr TypeGeom G = type_geom(T);
    constexpr int UE = G.unit_elems, UB = G.unit_bytes;
    constexpr int SPAN = span_lds_bytes(T);
    const int lane = threadIdx.x;
    const int K = a.ncols;
    const int nu = K / UE;                   // units per row (<= 64, checked on the host)
    const int rps = WAVE / nu;               // rows per step
    const u32 RB = (u32) nu * UB;            // row bytes

    int t, c = 0, e = 0, row0;
    const uint8_t *wup, *wgate = nullptr;
    u32 mbytes;
    const uint8_t *ybase;
    u32 yrow, ybytes;
    if (!shared) {
        const int pick = tile / a.tiles_per_pick;
        row0 = (tile % a.tiles_per_pick) * rps;
        t = pick / a.n_used;
        c = pick % a.n_used;
        e = a.ids[c + (int64_t) t * a.ids_stride];
        if (e < 0 || e >= a.n_experts) return;
        wup = (const uint8_t *) (uintptr_t) (a.tbl[e] & ~(uint64_t) 1);
        if (a.has_gate) wgate = (const uint8_t *) (uintptr_t) (a.tbl_gate[e] & ~(uint64_t) 1);
        mbytes = (u32) a.expert_bytes;
        ybase = a.y;
        ybytes = (u32) a.y_bytes;
        yrow = (u32) ((int64_t) (c % (int) a.nchannels_y) * a.stride_channel_y + (int64_t) t * a.stride_col_y);
    } else {
        const int st = tile - a.n_routed_tiles;
        t = st / a.sh_tiles_per_tok;
        row0 = (st % a.sh_tiles_per_tok) * rps;
        wup = a.sh_up;
        wgate = a.sh_gate;
        mbytes = (u32) a.sh_matrix_bytes;
        if (a.sh_y) {
            ybase = a.sh_y;
            ybytes = (u32) a.sh_y_bytes;
            yrow = (u32) ((int64_t) t * a.sh_stride_col_y);
        } else {
            ybase = a.y;
            ybytes = (u32) a.y_bytes;
            yrow = (u32) ((int64_t) t * a.stride_col_y);
        }
    }
    const int nrows_here = min(rps, a.nrows - row0);
    const u32 start = (u32) row0 * RB, nbytes = (u32) nrows_here * RB;

    // issue the weight DMA first (it does not depend on the activations)
    dma_span<T>(wup, mbytes, start, nbytes, lds);
    if (wgate) dma_span<T>(wgate, mbytes, start, nbytes, lds + SPAN);

    // this lane's activation slice (column `col` of the row)
    const int row_local = lane / nu, col = lane % nu;
    const bool active = row_local < nrows_here;
    Act<UE> A;
    {
        const __amdgpu_buffer_rsrc_t ry = make_rsrc(ybase, ybytes);
        load_act<UE, ACT>(A, ry, yrow, col);
    }

    // the DMA writes LDS asynchronously; wait for it before reading
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    const uintptr_t abase_up = (uintptr_t) wup & ~(uintptr_t) 15;
    const u32 lead = (u32) ((start + ((uintptr_t) wup - abase_up)) & 15u);
    float pu = 0.0f, pg = 0.0f;
    if (active) {
        const u32 uoff = lead + (u32) (row_local * nu + col) * UB;
        if constexpr (G.aligned) {
            pu = unit_dot<T, ACT>(WordsAligned{(const u32 *) (lds + uoff)}, A);
        } else {
            pu = unit_dot<T, ACT>(WordsShifted{(const u32 *) (lds + (uoff & ~3u)), uoff & 3u}, A);
        }
        if (wgate) {
            const uintptr_t abase_g = (uintptr_t) wgate & ~(uintptr_t) 15;
            const u32 leadg = (u32) ((start + ((uintptr_t) wgate - abase_g)) & 15u);
            const u32 goff = leadg + (u32) (row_local * nu + col) * UB;
            if constexpr (G.aligned) {
                pg = unit_dot<T, ACT>(WordsAligned{(const u32 *) (lds + SPAN + goff)}, A);
            } else {
                pg = unit_dot<T, ACT>(WordsShifted{(const u32 *) (lds + SPAN + (goff & ~3u)), goff & 3u}, A);
            }
        }
    }

    // row sums in a fixed order: lane (r*nu) adds the nu partials of row r left to right
    red[lane] = pu;
    red[WAVE + lane] = pg;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (active && col == 0) {
        float su = 0.0f, sg = 0.0f;
        for (int i = 0; i < nu; ++i) {
            su += red[lane + i];
            sg += red[WAVE + lane + i];
        }
        const int row = row0 + row_local;
        float out;
        if (!shared) {
            float up = su;
            if (a.x_scale) up *= a.x_scale[e];
            if (a.x_bias) up += a.x_bias[(int64_t) e * a.bias_stride + row];
            out = up;
            if (wgate) {
                float g = sg;
                if (a.gate_scale) g *= a.gate_scale[e];
                if (a.gate_bias) g += a.gate_bias[(int64_t) e * a.bias_stride + row];
                out = glu_apply(a.glu_op, g, up, a.glu_limit);
            }
            a.dst[(int64_t) c * a.stride_channel_dst + (int64_t) t * a.stride_col_dst + row] = out;
        } else {
            out = wgate ? glu_apply(a.glu_op, sg, su, a.glu_limit) : su;
            a.sh_dst[(int64_t) t * a.sh_stride_col_dst + row] = out;
        }
    }
}

template <int TW, int TS, int ACT>
__global__ __launch_bounds__(WAVE) void mc_gemv_kernel(const GemvArgs a) {
    constexpr int SPAN = span_lds_bytes(TW) > span_lds_bytes(TS) ? span_lds_bytes(TW) : span_lds_bytes(TS);
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * SPAN + 16];
    __shared__ float red[2 * WAVE + 64];
    if (blockIdx.x == 0) record_picks(a);
    const int tile = blockIdx.x;
    if (tile < a.n_routed_tiles) {
        run_step<TW, ACT>(a, lds, red, false, tile);
    } else if constexpr (TS != 0) {
        run_step<TS, ACT>(a, lds, red, true, tile);
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
        amax = fmaxf(amax, __shfl_xor(amax, off, 32));
        sum += __shfl_xor(sum, off, 32);
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
    for (int off = 16; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 32));
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
        for (int i = 0; i < 4; ++i) yb[4 + 4 * lane + i] = 0;
        if (lane < 8) *(u32 *) (yb + 260 + 4 * lane) = 0u;
        if (lane == 0) *(float *) yb = 0.0f;
        return;
    }
    const float mx = xb[aidx];
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
        yb[4 + 4 * lane + i] = (uint8_t) (int8_t) qs[i];
    }
    // bsums: 16 values = 4 lanes
    int s = qs[0] + qs[1] + qs[2] + qs[3];
    s += __shfl_xor(s, 1, WAVE);
    s += __shfl_xor(s, 2, WAVE);
    if ((lane & 3) == 0) *(int16_t *) (yb + 260 + 2 * (lane >> 2)) = (int16_t) s;
    if (lane == 0) *(float *) yb = 1.0f / iscale;
}

// MoE combine + next-layer quantization, one 1024-thread workgroup per token row:
//   x = residual + shared + sum_j w[j] * o[j]      (j ascending, fmaf), written to x_out;
//   optional weightless RMSNorm of x (the ffn_norm in front of the next MoE block):
//     thread t accumulates x[t + 1024 i]^2 with fmaf over i, the 1024 partials are
//     tree-summed (offsets 512 .. 1), scale = 1 / sqrtf(sum / k + eps);
//   then q8_1 quantization of x * scale exactly like mc_quantize_q8_1_kernel.
// This is the weighted sum ggml performs after MUL_MAT_ID (MUL by the router
// weights, then ADDs) fused with the quantize_q8_1 of the next GEMV's input.
// Every thread issues all of its loads before the first use (the row is small
// and latency, not bandwidth, bounds this kernel).
constexpr int COMBINE_MAX_K = 8192;
constexpr int COMBINE_THREADS = 1024;
constexpr int COMBINE_MAX_USED = 16;

__global__ __launch_bounds__(COMBINE_THREADS) void mc_combine_q8_1_kernel(const CombineArgs a) {
    __shared__ float xs[COMBINE_MAX_K];
    __shared__ float part[COMBINE_THREADS];
    const int64_t t = blockIdx.x;
    const int tid = threadIdx.x;
    constexpr int PER = COMBINE_MAX_K / COMBINE_THREADS;
    float wj[COMBINE_MAX_USED];
#pragma unroll
    for (int j = 0; j < COMBINE_MAX_USED; ++j) wj[j] = j < a.n_used ? a.w[t * a.n_used + j] : 0.0f;
    float ss = 0.0f;
#pragma unroll
    for (int r = 0; r < PER; ++r) {
        const int64_t i = tid + (int64_t) r * COMBINE_THREADS;
        if (i >= a.k) break;
        float ov[COMBINE_MAX_USED];
#pragma unroll
        for (int j = 0; j < COMBINE_MAX_USED; ++j) ov[j] = j < a.n_used ? a.o[(t * a.n_used + j) * a.o_stride + i] : 0.0f;
        float x = a.residual ? a.residual[t * a.k + i] : 0.0f;
        if (a.shared) x += a.shared[t * a.shared_stride + i];
#pragma unroll
        for (int j = 0; j < COMBINE_MAX_USED; ++j)
            if (j < a.n_used) x = fmaf(wj[j], ov[j], x);
        if (a.x_out) a.x_out[t * a.k + i] = x;
        xs[i] = x;
        ss = fmaf(x, x, ss);
    }
    float scale = 1.0f;
    if (a.rms_norm) {
        part[tid] = ss;
        __syncthreads();
        for (int off = COMBINE_THREADS / 2; off > 0; off >>= 1) {
            if (tid < off) part[tid] += part[tid + off];
            __syncthreads();
        }
        scale = 1.0f / sqrtf(part[0] / (float) a.k + a.eps);
    } else {
        __syncthreads();
    }
    const int grp = tid >> 5, l = tid & 31;
    for (int64_t b = grp; b < a.k / 32; b += COMBINE_THREADS / 32) {
        float x;
        {
#pragma clang fp contract(off)
            x = xs[b * 32 + l] * scale;
        }
        float amax = fabsf(x), sum = x;
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) {
            amax = fmaxf(amax, __shfl_xor(amax, off, 32));
            sum += __shfl_xor(sum, off, 32);
        }
        const float d = amax / 127.0f;
        const int8_t q = amax == 0.0f ? (int8_t) 0 : (int8_t) roundf(x / d);
        uint8_t *yb = a.y + t * a.y_stride + b * 36;
        yb[4 + l] = (uint8_t) q;
        if (l == 0) *(u32 *) yb = (u32) f2h_bits(d) | ((u32) f2h_bits(sum) << 16);
    }
}

// ---------------------------------------------------------------------------
// host-side launchers
// ---------------------------------------------------------------------------

template <int TW, int TS, int ACT>
static hipError_t launch_t(const GemvArgs &a, hipStream_t s) {
    hipLaunchKernelGGL((mc_gemv_kernel<TW, TS, ACT>), dim3((unsigned) a.n_tiles), dim3(WAVE), 0, s, a);
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

// Fills the tiling fields of `a` and launches.  Returns a hipError_t value.
int launch_gemv(GemvArgs a, int tw, int ts, int act, void *stream) {
    const TypeGeom g = type_geom(tw);
    const int nu = a.ncols / g.unit_elems;
    const int rps = WAVE / nu;
    a.tiles_per_pick = (a.nrows + rps - 1) / rps;
    a.n_routed_tiles = a.tiles_per_pick * a.n_used * a.n_tok;
    a.sh_tiles_per_tok = 0;
    if (ts != 0 && a.sh_up) {
        const int nus = a.ncols / type_geom(ts).unit_elems;
        const int rpss = WAVE / nus;
        a.sh_tiles_per_tok = (a.nrows + rpss - 1) / rpss;
    } else {
        ts = 0;
    }
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
    if (c.k > COMBINE_MAX_K || c.n_used > COMBINE_MAX_USED) return (int) hipErrorInvalidValue;
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
