// mc_core.h -- device-side building blocks shared by the per-op GEMV kernels and
// the persistent decode kernel: fp16/int8 helpers, buffer descriptors, the
// per-lane activation slice, LDS word readers, the per-type unit dot products,
// the GLU epilogue and the buffer->LDS span DMA.  Device code only (gfx950).
#ifndef MC_CORE_H
#define MC_CORE_H

#include <hip/hip_runtime.h>

#include "mc_internal.h"

// Cache-policy bits of the decode GEMV's weight DMA (buffer->LDS loads).  Each span
// is contiguous and read once per launch, so it goes out non-temporal (nt, bit 1):
// the stream then does not push the activation rows, ids and tables, which every
// workgroup reads, out of L2.
#ifndef MC_WEIGHT_CPOL
#define MC_WEIGHT_CPOL 2
#endif

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

// a . b over four int8 lanes with no accumulator (the VOP3 form takes the constant 0,
// where the accumulating form would need a zeroed register first)
__device__ __forceinline__ int sdot4_z(u32 a, u32 b) {
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// a . b over two int16 lanes, no accumulator
__device__ __forceinline__ int sdot2_z(u32 a, u32 b) {
    int r;
    asm("v_dot2_i32_i16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

typedef short v2i16 __attribute__((ext_vector_type(2)));
// c + a . b over two int16 lanes
__device__ __forceinline__ int sdot2(u32 a, u32 b, int c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(v2i16, a), __builtin_bit_cast(v2i16, b), c, false);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, u32 nbytes) {
    // gfx9 raw buffer: stride 0, num_records in bytes, dword3 = 0x00020000
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short) 0, (int) nbytes, 0x00020000);
}

// One 16-byte-per-lane buffer->LDS DMA load (1 KiB per wave) to dst, with cache policy
// CPOL (0, or 2: nt), issued from inline assembly.  For the intrinsic form the compiler
// places an s_waitcnt vmcnt(0) before the wave's next LDS access of any kind (it cannot
// tell which LDS bytes the DMA writes): the first poll of an LDS counter or read of the
// activation row after a span's DMA then waited for the whole span, so the gate dot never
// ran while the up span landed.  The compiler does not see this form's LDS write, so every
// reader of the DMA'd bytes waits for them itself (wait_loads_at_most, s_waitcnt vmcnt).
// M0 (the LDS destination) is saved and restored around the load; one wait state separates
// the M0 write from the load that reads it.  dst is a generic pointer into LDS, whose low 32
// bits are the LDS address (an address-space cast would add a null check per load).
template <int CPOL>
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint8_t *dst, u32 voff) {
    static_assert(CPOL == 0 || CPOL == 2, "cache policy: 0 or nt");
    const u32 la = (u32) __builtin_amdgcn_readfirstlane((int) (u32) (uintptr_t) dst);
    u32 saved;
    if constexpr (CPOL == 2)
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %2, %3, 0 offen nt lds\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved)
                     : "s"(la), "v"(voff), "s"(r)
                     : "memory");
    else
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %2, %3, 0 offen lds\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved)
                     : "s"(la), "v"(voff), "s"(r)
                     : "memory");
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
    u32 s2[UE / 32];             // s16[2i] | s16[2i+1] << 16 (int16 lanes)
};

// Sums of each 16 int8 activation values (the min/offset terms of the dots).
template <int UE>
__device__ __forceinline__ void act_sums(Act<UE> &A) {
#pragma unroll
    for (int s = 0; s < UE / 16; ++s) {
        int t = sdot4(A.q[4 * s + 0], 0x01010101u, 0);
        t = sdot4(A.q[4 * s + 1], 0x01010101u, t);
        t = sdot4(A.q[4 * s + 2], 0x01010101u, t);
        A.s16[s] = sdot4(A.q[4 * s + 3], 0x01010101u, t);
    }
#pragma unroll
    for (int i = 0; i < UE / 32; ++i) A.s2[i] = ((u32) A.s16[2 * i] & 0xFFFFu) | ((u32) A.s16[2 * i + 1] << 16);
}

typedef u32 v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// The lane's activation slice from an LDS copy of its row: UE/32 q8_1 blocks of
// 36 bytes, or one 292-byte q8_K block, at p (4-byte aligned).  When p is 16-byte
// aligned (q8_1 slices of 256 values are 288 bytes: 18 chunks) the slice is read
// with 128-bit LDS reads, else with 32-bit reads.
template <int UE, int ACT, bool S16 = false>
__device__ __forceinline__ void load_act_lds(Act<UE> &A, const uint8_t *p, const int16_t *s16 = nullptr) {
    constexpr int NW = ACT == ACT_Q8_1 ? UE / 32 * 9 : 73;
    u32 w[NW];
    if (NW % 4 == 1 && ((uintptr_t) p & 15u) == 0) {
        // a 16-byte aligned q8_K block (the padded LDS rows): 18 128-bit reads and one 32-bit read
        const v4u *q = (const v4u *) __builtin_assume_aligned(p, 16);
#pragma unroll
        for (int i = 0; i < NW / 4; ++i) {
            const v4u v = q[i];
            w[4 * i] = v.x;
            w[4 * i + 1] = v.y;
            w[4 * i + 2] = v.z;
            w[4 * i + 3] = v.w;
        }
        w[NW - 1] = ((const u32 *) p)[NW - 1];
    } else if (NW % 4 == 0 && ((uintptr_t) p & 15u) == 0) {
        const v4u *q = (const v4u *) __builtin_assume_aligned(p, 16);
#pragma unroll
        for (int i = 0; i < NW / 4; ++i) {
            const v4u v = q[i];
            w[4 * i] = v.x;
            w[4 * i + 1] = v.y;
            w[4 * i + 2] = v.z;
            w[4 * i + 3] = v.w;
        }
    } else {
        const u32 *q = (const u32 *) p;
#pragma unroll
        for (int i = 0; i < NW; ++i) w[i] = q[i];
    }
    if constexpr (ACT == ACT_Q8_1) {
#pragma unroll
        for (int b = 0; b < UE / 32; ++b) {
            A.d[b] = h2f(w[9 * b]);
#pragma unroll
            for (int k = 0; k < 8; ++k) A.q[8 * b + k] = w[9 * b + 1 + k];
        }
    } else {
        static_assert(UE == 256, "q8_K activations pair with 256-value units");
        const float d = __builtin_bit_cast(float, w[0]);
#pragma unroll
        for (int b = 0; b < 8; ++b) A.d[b] = d;
#pragma unroll
        for (int k = 0; k < 64; ++k) A.q[k] = w[1 + k];
    }
    if constexpr (S16) {
        // the 16-value sums precomputed next to the row (exact integer sums of the same codes):
        // a separate int16 array for q8_1 rows, the block's own bsums for q8_K
#pragma unroll
        for (int i = 0; i < UE / 32; ++i) {
            const u32 pair = ACT == ACT_Q8_K ? w[65 + i] : ((const u32 *) s16)[i];
            A.s2[i] = pair;
            A.s16[2 * i] = (int) (int16_t) (pair & 0xFFFFu);
            A.s16[2 * i + 1] = (int) (int16_t) (pair >> 16);
        }
    } else {
        act_sums(A);
    }
}

// ---------------------------------------------------------------------------
// LDS word readers for one unit
// ---------------------------------------------------------------------------

struct WordsAligned {            // unit starts on a 4-byte boundary
    const u32 *p;
    __device__ __forceinline__ u32 operator[](int i) const { return p[i]; }
};

template <int NW>
struct WordsRegs {               // unit already in registers
    u32 w[NW];
    __device__ __forceinline__ u32 operator[](int i) const { return w[i]; }
};

// A 16-byte aligned unit of NW words read from LDS with 128-bit reads: units whose
// size is an odd number of 16-byte chunks (Q4_K 9, Q5_K 11) then hit distinct bank
// groups in every 8-lane phase, where 32-bit reads at that stride conflict 8 ways.
template <int NW>
__device__ __forceinline__ WordsRegs<NW> lds_unit_b128(const uint8_t *p) {
    WordsRegs<NW> r;
    const v4u *q = (const v4u *) __builtin_assume_aligned(p, 16);
#pragma unroll
    for (int i = 0; i < NW / 4; ++i) {
        const v4u v = q[i];
        r.w[4 * i] = v.x;
        r.w[4 * i + 1] = v.y;
        r.w[4 * i + 2] = v.z;
        r.w[4 * i + 3] = v.w;
    }
    return r;
}

struct WordsShifted {            // unit starts on a 2-byte boundary: realign with v_alignbyte
    const u32 *p;
    u32 sh;                      // byte shift 0..3
    __device__ __forceinline__ u32 operator[](int i) const { return __builtin_amdgcn_alignbyte(p[i + 1], p[i], sh); }
};

// ---------------------------------------------------------------------------
// per-type unit dot products
// ---------------------------------------------------------------------------

// Integer scale products use 24-bit multiplies (full rate): every integer
// partial sum below is bounded by 16 * 63 * 127 < 2^23 in magnitude and every
// sub-block scale by 128, so the products are exact.

// Q2_K: scales[16] | qs[64] | d | dmin.  Element i = 128h + 32j + l uses
// (qs[32h + l] >> 2j) & 3 and sub-block scale byte i >> 4 (lo 4: scale, hi 4: min).
// The 2-bit fields of j < 3 stay in place (value * 4^j): the factor 4^-j is folded
// into the activation scale (exact, a power of two).  The min term of each 32-value
// group is one v_dot2 of the two 4-bit mins (int16 lanes) with the packed 16-value sums.
template <int ACT, class W>
__device__ __forceinline__ float dot_q2_K(const W &w, const Act<256> &A) {
    const u32 dm = w[20];
    const float d = h2f(dm), dmin = h2f(dm >> 16);
    u32 sc[4], mh[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sc[i] = w[i];
        mh[i] = (sc[i] >> 4) & 0x0F0F0F0Fu;
    }
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
                d0 = k == 0 ? sdot4_z(v0, A.q[8 * g + k]) : sdot4(v0, A.q[8 * g + k], d0);
                d1 = k == 0 ? sdot4_z(v1, A.q[8 * g + 4 + k]) : sdot4(v1, A.q[8 * g + 4 + k], d1);
            }
            const int kb = 2 * (g & 1);                   // scale bytes 2g, 2g+1 of word g / 2
            const u32 wsc = sc[g >> 1];
            const int is = __mul24((int) ((wsc >> (8 * kb)) & 0xFu), d0) + __mul24((int) ((wsc >> (8 * kb + 8)) & 0xFu), d1);
            const u32 mp = __builtin_amdgcn_perm(0u, mh[g >> 1], kb == 0 ? 0x0C010C00u : 0x0C030C02u);
            const int ms = sdot2_z(mp, A.s2[g]);
            if constexpr (ACT == ACT_Q8_K) {
                isum += is >> (2 * jj);
                msum += ms;
            } else {
                const float dj = jj == 0 ? A.d[g] : A.d[g] * (jj == 1 ? 0.25f : 0.0625f);
                accI = fmaf(dj, (float) is, accI);
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
            const int is = __mul24(sc0, d0) + __mul24(sc1, d1);
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
            const int is = __mul24(sc, dot);
            const int ms = __mul24(m, A.s16[2 * g] + A.s16[2 * g + 1]);
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
            const int is = __mul24(sc0, d0) + __mul24(sc1, d1);
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

// x * sigmoid(x) with the hardware exp2 and reciprocal: a few ulp from the IEEE
// x / (1 + expf(-x)), far inside the GEMV tolerance, and ~40 fewer instructions in the
// epilogue every wave ends with.  Large |x| saturate exactly: exp(-x) -> inf gives -0,
// exp(-x) -> 0 gives x.
__device__ __forceinline__ float silu_f(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

__device__ __forceinline__ float glu_apply(int op, float g, float up, float limit) {
#pragma clang fp contract(off)          // every caller rounds each step alike (GEGLU's 1 + c * g * g)
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



typedef __attribute__((address_space(3))) void lds_void_t;

// Streams [start, start + nbytes) of the matrix at `base` into lds (lds[x] = byte
// (start & ~15) + x of the 16-byte aligned view); returns the number of DMA
// instructions issued (one per KiB).  The destination holds whole 1 KiB rounds
// (lanes of the last round past the span write zeros: the descriptor ends with the
// span), or with MASK_TAIL only round_up_16(lead + nbytes) bytes: the last round is
// then issued separately with the lanes past the span switched off (it costs the
// plain GEMV a few percent, so only the kernels short of LDS use it).
template <int T, bool MASK_TAIL = false>
__device__ __forceinline__ int dma_span(const uint8_t *base, u32 base_bytes, u32 start, u32 nbytes, uint8_t *lds) {
    const uintptr_t abase = (uintptr_t) base & ~(uintptr_t) 15;
    const u32 skew = (u32) ((uintptr_t) base - abase);
    // the descriptor ends with the span (rounded up to its 16-byte chunk): the lanes of the
    // last round that lie past it read zeros instead of fetching the next step's rows
    const u32 end = min(base_bytes + skew, (start + skew + nbytes + 15u) & ~15u);
    const __amdgpu_buffer_rsrc_t r = make_rsrc((const void *) abase, end);
    const u32 a0 = (start + skew) & ~15u;
    const u32 lead = (start + skew) - a0;
    const int rounds = (int) ((lead + nbytes + 1023u) >> 10);
    constexpr int MAXR = span_lds_bytes(T) / 1024;
    const u32 lane_off = a0 + 16u * (threadIdx.x % WAVE);
    if constexpr (!MASK_TAIL) {
#pragma unroll
        for (int i = 0; i < MAXR; ++i) {
            if (i < rounds) {
                lds_dma16<MC_WEIGHT_CPOL>(r, lds + 1024 * i, lane_off + 1024u * i);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < MAXR; ++i) {
            if (i < rounds - 1)
                lds_dma16<MC_WEIGHT_CPOL>(r, lds + 1024 * i, lane_off + 1024u * i);
        }
        const u32 last = (u32) (rounds - 1);
        if (16u * (threadIdx.x % WAVE) < lead + nbytes - 1024u * last)
            lds_dma16<MC_WEIGHT_CPOL>(r, lds + 1024 * last, lane_off + 1024u * last);
    }
    return rounds;
}

// Waits until at most n of this wave's vector memory loads are outstanding
// (loads complete in issue order, so every earlier load has landed).  vmcnt
// holds 6 bits: n >= 63 waits for at most 63.
__device__ __forceinline__ void wait_loads_at_most(int n) {
    switch (n) {
#define MC_WAITCASE(k) case k: asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); break;
        MC_WAITCASE(0) MC_WAITCASE(1) MC_WAITCASE(2) MC_WAITCASE(3) MC_WAITCASE(4) MC_WAITCASE(5) MC_WAITCASE(6) MC_WAITCASE(7)
        MC_WAITCASE(8) MC_WAITCASE(9) MC_WAITCASE(10) MC_WAITCASE(11) MC_WAITCASE(12) MC_WAITCASE(13) MC_WAITCASE(14) MC_WAITCASE(15)
        MC_WAITCASE(16) MC_WAITCASE(17) MC_WAITCASE(18) MC_WAITCASE(19) MC_WAITCASE(20) MC_WAITCASE(21) MC_WAITCASE(22) MC_WAITCASE(23)
        MC_WAITCASE(24) MC_WAITCASE(25) MC_WAITCASE(26) MC_WAITCASE(27) MC_WAITCASE(28) MC_WAITCASE(29) MC_WAITCASE(30) MC_WAITCASE(31)
        MC_WAITCASE(32) MC_WAITCASE(33) MC_WAITCASE(34) MC_WAITCASE(35) MC_WAITCASE(36) MC_WAITCASE(37) MC_WAITCASE(38) MC_WAITCASE(39)
        MC_WAITCASE(40) MC_WAITCASE(41) MC_WAITCASE(42) MC_WAITCASE(43) MC_WAITCASE(44) MC_WAITCASE(45) MC_WAITCASE(46) MC_WAITCASE(47)
        MC_WAITCASE(48) MC_WAITCASE(49) MC_WAITCASE(50) MC_WAITCASE(51) MC_WAITCASE(52) MC_WAITCASE(53) MC_WAITCASE(54) MC_WAITCASE(55)
        MC_WAITCASE(56) MC_WAITCASE(57) MC_WAITCASE(58) MC_WAITCASE(59) MC_WAITCASE(60) MC_WAITCASE(61) MC_WAITCASE(62)
#undef MC_WAITCASE
        default: asm volatile("s_waitcnt vmcnt(63)" ::: "memory"); break;
    }
}

// Cross-lane moves that stay off the LDS crossbar (which the weight DMA keeps busy):
// DPP inside a 16-lane row, gfx950 permlane swaps across rows.
template <int CTRL, int BANKS = 0xF>
__device__ __forceinline__ float dpp_f(float old, float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                                 CTRL, 0xF, BANKS, false));
}
constexpr int DPP_QUAD_XOR1 = 0xB1, DPP_QUAD_XOR2 = 0x4E, DPP_ROW_SHL4 = 0x104, DPP_ROW_SHL8 = 0x108,
              DPP_ROW_SHR4 = 0x114, DPP_ROW_SHR8 = 0x118, DPP_WAVE_SHL1 = 0x130, DPP_ROW_HALF_MIRROR = 0x141;

// lanes 0..31 receive lanes 32..63 (v_permlane32_swap: the source operand's low half takes
// the destination operand's high half)
__device__ __forceinline__ float from_lane_plus32(float v) {
    const u32 b = __builtin_bit_cast(u32, v);
    return __builtin_bit_cast(float, (u32) __builtin_amdgcn_permlane32_swap(b, b, false, false)[1]);
}
// lanes 16g .. 16g+15 of even rows g receive the next row (v_permlane16_swap)
__device__ __forceinline__ float from_lane_plus16(float v) {
    const u32 b = __builtin_bit_cast(u32, v);
    return __builtin_bit_cast(float, (u32) __builtin_amdgcn_permlane16_swap(b, b, false, false)[1]);
}
// lane l receives lane l ^ 4 (within 8-lane groups): row_shl:4 into banks 0 and 2, row_shr:4 into 1 and 3
__device__ __forceinline__ float from_lane_xor4(float v) {
    return dpp_f<DPP_ROW_SHR4, 0xA>(dpp_f<DPP_ROW_SHL4, 0x5>(v, v), v);
}
// lane l receives lane l ^ M
template <int M>
__device__ __forceinline__ float xor_lanes(float v) {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "lane xor mask");
    if constexpr (M == 1) return dpp_f<DPP_QUAD_XOR1>(0.0f, v);
    if constexpr (M == 2) return dpp_f<DPP_QUAD_XOR2>(0.0f, v);
    if constexpr (M == 4) return from_lane_xor4(v);
    if constexpr (M == 8) return dpp_f<DPP_ROW_SHR8, 0xC>(dpp_f<DPP_ROW_SHL8, 0x3>(v, v), v);
    const u32 b = __builtin_bit_cast(u32, v);
    const int lane = threadIdx.x % WAVE;
    if constexpr (M == 16) {
        // even rows take the swap's source half (the next row), odd rows its destination half
        const auto p = __builtin_amdgcn_permlane16_swap(b, b, false, false);
        return __builtin_bit_cast(float, (u32) ((lane & 16) ? p[0] : p[1]));
    }
    const auto p = __builtin_amdgcn_permlane32_swap(b, b, false, false);
    return __builtin_bit_cast(float, (u32) ((lane & 32) ? p[0] : p[1]));
}
// xor_lanes with a mask that full unrolling makes a constant
__device__ __forceinline__ float xor_lanes_rt(float v, int m) {
    switch (m) {
        case 1: return xor_lanes<1>(v);
        case 2: return xor_lanes<2>(v);
        case 4: return xor_lanes<4>(v);
        case 8: return xor_lanes<8>(v);
        case 16: return xor_lanes<16>(v);
        default: return xor_lanes<32>(v);
    }
}
// lane l receives lane l + 1 across the whole wave (DPP wave_shl:1; lane 63 keeps its value)
__device__ __forceinline__ float wave_shl1(float v) { return dpp_f<DPP_WAVE_SHL1>(v, v); }

// Workgroup barrier for data exchanged through LDS (ordinary LDS writes, or DMA
// writes each wave has already waited for with its own vmcnt): unlike
// __syncthreads(), whose release fence drains every outstanding load, it leaves
// the buffer->LDS DMAs still in flight (the next stage of a pipeline) alone.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Uniform loads through the scalar data cache (read-only data: routing ids and
// pointer tables, which no kernel writes while it runs).
template <class V>
__device__ __forceinline__ V sload(const V *p) {
    return *(const __attribute__((address_space(4))) V *) p;
}

// Sum over the nu consecutive lanes of each row group (lane r*nu .. r*nu+nu-1):
// xor butterfly when nu is a power of two (total in every lane of the group),
// else lane r*nu adds lanes r*nu+1 .. r*nu+nu-1 in order (total in lane r*nu).
// Every exchange is a DPP move or a permlane swap (see xor_lanes / wave_shl1), so
// the sums stay off the LDS crossbar.
__device__ __forceinline__ float row_group_sum(float v, int nu) {
    if ((nu & (nu - 1)) == 0) {
        if (nu >= 64) v += xor_lanes<32>(v);
        if (nu >= 32) v += xor_lanes<16>(v);
        if (nu >= 16) v += xor_lanes<8>(v);
        if (nu >= 8) v += xor_lanes<4>(v);
        if (nu >= 4) v += xor_lanes<2>(v);
        if (nu >= 2) v += xor_lanes<1>(v);
        return v;
    }
    float s = v, o = v;
    for (int i = 1; i < nu; ++i) {
        o = wave_shl1(o);                 // lane l: v of lane l + i
        s += o;
    }
    return s;
}

// Streams bytes [off, off + nbytes) of `base` (a buffer of base_bytes bytes) into
// LDS with 16-byte buffer->LDS DMA loads from the 16-byte aligned address at or
// below base + off.  Returns the lead: byte `off` lands at lds[lead] (lead < 16).
// The LDS destination must hold round_up_1k(lead + nbytes) bytes.
__device__ __forceinline__ u32 dma_bytes(const uint8_t *base, u32 base_bytes, u32 off, u32 nbytes, uint8_t *lds) {
    const uintptr_t abase = (uintptr_t) base & ~(uintptr_t) 15;
    const u32 skew = (u32) ((uintptr_t) base - abase);
    const u32 end = min(base_bytes + skew, (off + skew + nbytes + 15u) & ~15u);   // no fetch past the range
    const __amdgpu_buffer_rsrc_t r = make_rsrc((const void *) abase, end);
    const u32 a0 = (off + skew) & ~15u;
    const u32 lead = (off + skew) - a0;
    const int rounds = (int) ((lead + nbytes + 1023u) >> 10);
    const u32 lane_off = a0 + 16u * (threadIdx.x % WAVE);
    for (int i = 0; i < rounds; ++i)
        lds_dma16<0>(r, lds + 1024 * i, lane_off + 1024u * i);
    return lead;
}

// Byte offset, inside the LDS copy made by dma_span, of byte `start` of the matrix at `base`.
__device__ __forceinline__ u32 span_lead(const uint8_t *base, u32 start) {
    const uintptr_t abase = (uintptr_t) base & ~(uintptr_t) 15;
    return (u32) ((start + ((uintptr_t) base - abase)) & 15u);
}

// Dot of the lane's unit `unit` of a DMA'd span (lead from span_lead) with its activation slice.
template <int T, int ACT>
__device__ __forceinline__ float span_unit_dot(const uint8_t *lds_span, u32 lead, int unit,
                                               const Act<type_geom(T).unit_elems> &A) {
    constexpr TypeGeom G = type_geom(T);
    const u32 uoff = lead + (u32) unit * G.unit_bytes;
    if constexpr (G.aligned && G.unit_bytes % 16 == 0) {
        if ((uoff & 15u) == 0) return unit_dot<T, ACT>(lds_unit_b128<G.unit_bytes / 4>(lds_span + uoff), A);
    }
    if constexpr (G.aligned) {
        return unit_dot<T, ACT>(WordsAligned{(const u32 *) (lds_span + uoff)}, A);
    } else {
        return unit_dot<T, ACT>(WordsShifted{(const u32 *) (lds_span + (uoff & ~3u)), uoff & 3u}, A);
    }
}

// Makes a wave's LDS writes visible to the wave's later LDS reads (single-wave workgroups).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Row sums of a step in a fixed order: lane r*nu adds the nu lane partials of row r left to right.
// red: 64 floats of LDS.  The sum is valid in lanes with (lane % nu) == 0.
__device__ __forceinline__ float step_row_sum(float *red, float v, int nu) {
    const int lane = threadIdx.x % WAVE;
    red[lane] = v;
    wave_lds_sync();
    float s = 0.0f;
    if (lane % nu == 0 && lane + nu <= WAVE)
        for (int i = 0; i < nu; ++i) s += red[lane + i];
    wave_lds_sync();
    return s;
}

// q8 codes roundf(v / d) of values |v| <= amax, d = amax / 127 (IEEE), with one hardware
// reciprocal per block (v_rcp_f32, relative error at most 2^-23) instead of a division per
// value.  For a normal, finite d the product y = v * rcp(d) is within 2^-15 of fl(v / d):
// |v / d| <= 127 (1 + 2^-24), the reciprocal's error and the product's rounding add at most
// 1.5 * 2^-23 * 127 < 2^-15.4, and fl(v / d) itself is within 2^-17 of v / d.  So wherever y
// lies at least 2^-14 away from a half-integer, rint(y) == roundf(fl(v / d)).  The remaining
// values, and every value of a block whose d is zero, subnormal or not finite, are flagged
// (slow) for the division.  (d <= FLT_MAX / 127 keeps rcp(d) a normal number.)
__device__ __forceinline__ bool q8_scale_ok(float d) { return d >= 0x1p-126f && d <= 0x1.fffffep+127f; }

// The reciprocal the shortcut multiplies by (1 when the block takes the division).
__device__ __forceinline__ float q8_inv(float d, bool d_ok) { return __builtin_amdgcn_rcpf(d_ok ? d : 1.0f); }

__device__ __forceinline__ int q8_code_fast(float v, float inv, bool d_ok, bool &slow) {
    const float y = v * (d_ok ? inv : 0.0f);
    const float r = __builtin_rintf(y);
    slow = !d_ok || fabsf(y - r) >= 0.5f - 0x1p-14f;
    return (int) r;
}

// The division of the flagged values (d = 0 divides by 1; the caller writes 0 for it).
__device__ __forceinline__ int q8_code_exact(float v, float d) { return (int) roundf(v / (d != 0.0f ? d : 1.0f)); }

// q8_1 quantization of one 32-value block spread over a 32-lane half-wave (the
// arithmetic of ggml-CUDA quantize_q8_1): amax over the half-wave, d = amax/127
// (IEEE division), q = amax == 0 ? 0 : roundf(x/d).  Also returns the xor-butterfly sum.
__device__ __forceinline__ int8_t q8_1_lane(float x, float &d, float &sum) {
    float amax = fabsf(x);
    sum = x;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) {
        amax = fmaxf(amax, xor_lanes_rt(amax, off));
        sum += xor_lanes_rt(sum, off);
    }
    d = amax / 127.0f;
    const bool dok = q8_scale_ok(d);
    bool slow;
    int q = q8_code_fast(x, q8_inv(d, dok), dok, slow);
    if (__builtin_amdgcn_ballot_w64(slow) != 0) {            // rare: see q8_code_fast
        if (slow) q = q8_code_exact(x, d);
    }
    return amax == 0.0f ? (int8_t) 0 : (int8_t) q;
}

// q8_1 blocks of the k fp32 values at x (LDS, 4-byte aligned, k % 32 == 0) into
// q (LDS, 36-byte blocks, 4-byte aligned) with the arithmetic of the q8_1
// quantizer: amax over each 32 values, d = amax / 127 (IEEE division),
// code = amax == 0 ? 0 : roundf(x / d).  Two lanes own one block (16 values
// each, one partner exchange), so there is no chain of cross-lane reductions.
// The block's s half is left unset: the dot products read only d and the codes.
__device__ __forceinline__ void quantize_row_lds(const float *x, uint8_t *q, int k) {
    const int lane = threadIdx.x % WAVE;
    const int nblk = k / 32;
    for (int b0 = 0; b0 < nblk; b0 += WAVE / 2) {
        const int b = b0 + lane / 2, half = lane & 1;
        const bool on = b < nblk;
        float v[16];
        const float *src = x + (on ? b : 0) * 32 + 16 * half;
        if (((uintptr_t) x & 15u) == 0) {
            const v4f *s4 = (const v4f *) __builtin_assume_aligned(src, 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const v4f w = s4[i];
                v[4 * i] = w.x;
                v[4 * i + 1] = w.y;
                v[4 * i + 2] = w.z;
                v[4 * i + 3] = w.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = src[i];
        }
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
        amax = fmaxf(amax, xor_lanes<1>(amax));              // the partner lane of the block
        const float d = amax / 127.0f;
        const bool dok = q8_scale_ok(d);
        const float inv = q8_inv(d, dok);
        int qv[16];
        u32 slow = 0u;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            bool sl;
            qv[i] = q8_code_fast(v[i], inv, dok, sl);
            slow |= (sl ? 1u : 0u) << i;
        }
        if (__builtin_amdgcn_ballot_w64(slow != 0u) != 0) {  // rare: see q8_code_fast
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (slow & (1u << i)) qv[i] = q8_code_exact(v[i], d);
        }
        u32 packed[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            u32 wd = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int code = amax == 0.0f ? 0 : qv[4 * i + j];
                wd |= ((u32) code & 0xFFu) << (8 * j);
            }
            packed[i] = wd;
        }
        if (on) {
            u32 *dst = (u32 *) (q + b * 36 + 4 + 16 * half);
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = packed[i];
            if (half == 0) *(u32 *) (q + b * 36) = (u32) f2h_bits(d);   // same access type as the readers
        }
    }
    wave_lds_sync();
}

// Sum of squares of one 256-value chunk in the canonical RMS order (mc_internal.h):
// lane l holds values 4l .. 4l+3 of the chunk in xv; returned in every lane.  The
// shuffle-down tree (offsets 32 .. 1, lane l < off adds lane l + off) runs on permlane
// swaps and DPP: lane 0's operands at every level are exactly the tree's (the other
// lanes' values are not used).
__device__ __forceinline__ float rms_chunk_sum(const float xv[4]) {
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) a = fmaf(xv[k], xv[k], a);
    a += from_lane_plus32(a);
    a += from_lane_plus16(a);
    a += dpp_f<DPP_ROW_SHL8>(0.0f, a);
    a += dpp_f<DPP_ROW_SHL4>(0.0f, a);
    a += dpp_f<DPP_QUAD_XOR2>(0.0f, a);
    a += dpp_f<DPP_QUAD_XOR1>(0.0f, a);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 0));
}

constexpr int COMBINE_MAX_USED = 16;

// One 64-lane wave: the 256 combined values of chunk j of a row, lane l holding
// values 256j + 4l .. 256j + 4l + 3 (16-byte loads; rows 16-byte aligned):
//   x = residual + shared + sum_c w[c] * o[c]   (c ascending, fmaf)
// into xv (registers) and x_out (when given); returns the chunk's RMS sum in the
// canonical order (mc_internal.h) in every lane.
__device__ __forceinline__ float combine_chunk(const float *o, int64_t o_stride, const float *w, int n_used,
                                               const float *shared, const float *residual, float *x_out, int j,
                                               float xv[4]) {
    const int lane = threadIdx.x % WAVE;
    const int64_t i0 = (int64_t) j * RMS_CHUNK + 4 * lane;
    float wc[COMBINE_MAX_USED];
#pragma unroll
    for (int c = 0; c < COMBINE_MAX_USED; ++c) wc[c] = c < n_used ? w[c] : 0.0f;
    v4f ov[COMBINE_MAX_USED];
#pragma unroll
    for (int c = 0; c < COMBINE_MAX_USED; ++c)
        if (c < n_used) ov[c] = *(const v4f *) (o + c * o_stride + i0);
    v4f x = residual ? *(const v4f *) (residual + i0) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if (shared) {
        const v4f sh = *(const v4f *) (shared + i0);
        x.x += sh.x;
        x.y += sh.y;
        x.z += sh.z;
        x.w += sh.w;
    }
#pragma unroll
    for (int c = 0; c < COMBINE_MAX_USED; ++c) {
        if (c < n_used) {
            x.x = fmaf(wc[c], ov[c].x, x.x);
            x.y = fmaf(wc[c], ov[c].y, x.y);
            x.z = fmaf(wc[c], ov[c].z, x.z);
            x.w = fmaf(wc[c], ov[c].w, x.w);
        }
    }
    if (x_out) *(v4f *) (x_out + i0) = x;
    xv[0] = x.x;
    xv[1] = x.y;
    xv[2] = x.z;
    xv[3] = x.w;
    return rms_chunk_sum(xv);
}

// Maximum over the 8-lane group of each lane (lanes 8g .. 8g+7), all by DPP: the two quad
// exchanges, then the mirror inside the half-row (which pairs each quad with the other
// quad of its group).  fmaxf is exact, so the result equals any other reduction order.
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, dpp_f<DPP_QUAD_XOR1>(0.0f, v));
    v = fmaxf(v, dpp_f<DPP_QUAD_XOR2>(0.0f, v));
    v = fmaxf(v, dpp_f<DPP_ROW_HALF_MIRROR>(0.0f, v));
    return v;
}

// One 64-lane wave: q8_1 of the 256 values v of chunk j into y (row base), lane l
// holding values 4l .. 4l+3 of the chunk in xv, with v = (x * s) * nw[i] under norm
// (nw optional) and v = x otherwise.  Eight lanes form one 32-value block.  The
// arithmetic is the q8_1 quantizer's (q8_1_lane): amax, d = amax / 127,
// code = amax == 0 ? 0 : roundf(v / d), and the block sum in the quantizer's
// xor-butterfly order (offsets 16, 8, 4 across lanes, then 2, 1 inside the lane).
// WITH_SUM = false leaves the sum field 0: the K-quant dots read only d and the codes.
// No contraction: the block sum adds the rounded values v, as the quantizer does; an FMA of
// (x * s) * nw into the first add (the compiler's choice differs between callers) changed a
// sum's fp16 rounding in 2 of 192 blocks of a 6144-value row.
template <bool WITH_SUM = true>
__device__ __forceinline__ void quantize_chunk(const float xv[4], bool norm, float s, const v4f nwv, uint8_t *y,
                                               int j) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x % WAVE;
    float v[4] = {xv[0], xv[1], xv[2], xv[3]};
    if (norm) {
        const float nw[4] = {nwv.x, nwv.y, nwv.z, nwv.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = (v[k] * s) * nw[k];
    }
    const float amax = max8(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    float sum = 0.0f;
    if constexpr (WITH_SUM) {
        float t[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
        for (int off = 4; off > 0; off >>= 1) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float o = off == 4 ? from_lane_xor4(t[k])
                                         : off == 2 ? dpp_f<DPP_QUAD_XOR2>(0.0f, t[k]) : dpp_f<DPP_QUAD_XOR1>(0.0f, t[k]);
                t[k] += o;
            }
        }
        const float t2[4] = {t[0] + t[2], t[1] + t[3], t[2] + t[0], t[3] + t[1]};
        sum = t2[0] + t2[1];
    }
    const float d = amax / 127.0f;
    const bool dok = q8_scale_ok(d);
    const float inv = q8_inv(d, dok);
    int q[4];
    u32 slow = 0u;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        bool sl;
        q[k] = q8_code_fast(v[k], inv, dok, sl);
        slow |= (sl ? 1u : 0u) << k;
    }
    if (__builtin_amdgcn_ballot_w64(slow != 0u) != 0) {      // rare: see q8_code_fast
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if (slow & (1u << k)) q[k] = q8_code_exact(v[k], d);
    }
    u32 packed = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int code = amax == 0.0f ? 0 : q[k];
        packed |= ((u32) code & 0xFFu) << (8 * k);
    }
    const int i = j * RMS_CHUNK + 4 * lane;               // first value of this lane in the row
    uint8_t *yb = y + (i / 32) * 36;
    *(u32 *) (yb + 4 + (i % 32)) = packed;
    // the eight lanes of a block store the same scale word (no branch around the store)
    *(u32 *) yb = (u32) f2h_bits(d) | (WITH_SUM ? ((u32) f2h_bits(sum) << 16) : 0u);
}

// One 64-lane wave: the q8_K blocks (292 bytes at yb[i]: d, qs[256], bsums[16]) of N groups
// of 256 values v[i], lane l holding values 4l .. 4l+3 of each, with the arithmetic of
// ggml's quantize_row_q8_K_ref: max = the signed value of the first largest |v| (strictly
// larger wins, so the lowest index among ties), iscale = -127 / max,
// q = min(127, rint(iscale * v)) (round half to even, as its nearest_int), d = 1 / iscale,
// bsums = sums of each 16 codes; an all-zero block gets d = 0 and zero codes and sums.
// The N blocks go stage by stage so their dependency chains (cross-lane maxima, divisions)
// interleave; cross-lane steps stay on DPP / permlane (no LDS traffic).  With `second`,
// yb2[i] receives a copy of each block.
template <int N>
__device__ __forceinline__ void q8K_chunks(const float (&v)[N][4], uint8_t *const (&yb)[N], uint8_t *const (&yb2)[N],
                                           bool second) {
    const int lane = threadIdx.x % WAVE;
    float am[N], amax[N], cand[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        am[i] = -1.0f;
        cand[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float ax = fabsf(v[i][j]);
            if (ax > am[i]) {
                am[i] = ax;
                cand[i] = v[i][j];
            }
        }
        amax[i] = am[i];
    }
#pragma unroll
    for (int i = 0; i < N; ++i) amax[i] = fmaxf(amax[i], xor_lanes<32>(amax[i]));
#pragma unroll
    for (int i = 0; i < N; ++i) amax[i] = fmaxf(amax[i], xor_lanes<16>(amax[i]));
#pragma unroll
    for (int i = 0; i < N; ++i) amax[i] = fmaxf(amax[i], xor_lanes<8>(amax[i]));
#pragma unroll
    for (int i = 0; i < N; ++i) amax[i] = fmaxf(amax[i], xor_lanes<4>(amax[i]));
#pragma unroll
    for (int i = 0; i < N; ++i) amax[i] = fmaxf(amax[i], xor_lanes<2>(amax[i]));
#pragma unroll
    for (int i = 0; i < N; ++i) amax[i] = fmaxf(amax[i], xor_lanes<1>(amax[i]));
    float d[N], iscale[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        // the lowest lane holding the maximum, and its first such value
        const uint64_t hit = __builtin_amdgcn_ballot_w64(am[i] == amax[i]);
        const int l0 = hit ? __builtin_ctzll(hit) : 0;
        const float mx = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cand[i]), l0));
        // (all-NaN lanes leave amax at -1: a zero block)
        iscale[i] = amax[i] > 0.0f ? -127.0f / mx : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < N; ++i) d[i] = amax[i] > 0.0f ? 1.0f / iscale[i] : 0.0f;
    u32 packed[N];
    int sum[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        packed[i] = 0u;
        sum[i] = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float p;
            {
#pragma clang fp contract(off)
                p = iscale[i] * v[i][j];
            }
            int c = (int) __builtin_rintf(p);
            c = amax[i] > 0.0f ? (c < 127 ? c : 127) : 0;
            packed[i] |= ((u32) c & 0xFFu) << (8 * j);
            sum[i] += c;                                 // 16 codes = 4 lanes
        }
    }
#pragma unroll
    for (int i = 0; i < N; ++i) sum[i] += __builtin_amdgcn_update_dpp(0, sum[i], DPP_QUAD_XOR1, 0xF, 0xF, false);
#pragma unroll
    for (int i = 0; i < N; ++i) sum[i] += __builtin_amdgcn_update_dpp(0, sum[i], DPP_QUAD_XOR2, 0xF, 0xF, false);
#pragma unroll
    for (int i = 0; i < N; ++i) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            if (c == 1 && !second) continue;
            uint8_t *y = c == 0 ? yb[i] : yb2[i];
            *(u32 *) (y + 4 + 4 * lane) = packed[i];
            if ((lane & 3) == 0) *(int16_t *) (y + 260 + 2 * (lane >> 2)) = (int16_t) sum[i];
            if (lane == 0) *(float *) y = d[i];
        }
    }
}

// Stride of q8_K blocks in the fused kernels' LDS rows: 292 bytes padded to a 16-byte
// multiple, so every block is read with 128-bit LDS reads.
constexpr int Q8K_LDS_STRIDE = 304;

// Stride of the 256-value units (eight q8_1 blocks, 288 bytes) of the fused gate/up kernel's LDS
// activation row: 16 bytes of padding per unit.  With the packed 288-byte stride the 16 units of a
// 4096-value row lie 72 dwords apart, so their 16-byte reads by one instruction share 8 bank groups
// of the 64 banks (a 2-way conflict); 76 dwords apart they use 16 distinct groups.
constexpr int Q8_1_LDS_STRIDE = 304;

// G blocks b0 .. b0 + G - 1 of quantize_row_lds_q8K, interleaved.
template <int G>
__device__ __forceinline__ void q8K_row_blocks(const float *x, uint8_t *q, int b0, bool al) {
    const int lane = threadIdx.x % WAVE;
    float v[G][4];
    uint8_t *yb[G];
#pragma unroll
    for (int i = 0; i < G; ++i) {
        const float *src = x + 256 * (b0 + i) + 4 * lane;
        if (al) {
            const v4f x4 = *(const v4f *) __builtin_assume_aligned(src, 16);
            v[i][0] = x4.x;
            v[i][1] = x4.y;
            v[i][2] = x4.z;
            v[i][3] = x4.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[i][j] = src[j];
        }
        yb[i] = q + Q8K_LDS_STRIDE * (b0 + i);
    }
    q8K_chunks<G>(v, yb, yb, false);
}

// The wave's fp32 row of k values (k a multiple of 256) as q8_K blocks, Q8K_LDS_STRIDE
// apart: four blocks per pass, then the remaining one to three together (a 768-value row
// is one pass of three), so no block is quantized twice.
__device__ __forceinline__ void quantize_row_lds_q8K(const float *x, uint8_t *q, int k) {
    const bool al = ((uintptr_t) x & 15u) == 0;
    const int nblk = k / 256;
    int b0 = 0;
    for (; b0 + 4 <= nblk; b0 += 4) q8K_row_blocks<4>(x, q, b0, al);
    switch (nblk - b0) {
        case 3: q8K_row_blocks<3>(x, q, b0, al); break;
        case 2: q8K_row_blocks<2>(x, q, b0, al); break;
        case 1: q8K_row_blocks<1>(x, q, b0, al); break;
        default: break;
    }
    wave_lds_sync();
}

// 16-value sums of the codes of a q8_1 row of k values in LDS (36-byte blocks from p,
// 4-byte aligned) into s16[0 .. k/16): sum i covers codes 16i .. 16i+15, one sum per
// lane and pass.  These are the integers act_sums forms for each unit of the row, so
// a wave computes them once instead of every lane of a unit column repeating them.
__device__ __forceinline__ void row_sums16_lds(const uint8_t *p, int k, int16_t *s16) {
    const int lane = threadIdx.x % WAVE;
    for (int i = lane; i < k / 16; i += WAVE) {
        const u32 *q = (const u32 *) (p + (i >> 1) * 36 + 4 + 16 * (i & 1));
        int t = sdot4(q[0], 0x01010101u, 0);
        t = sdot4(q[1], 0x01010101u, t);
        t = sdot4(q[2], 0x01010101u, t);
        t = sdot4(q[3], 0x01010101u, t);
        s16[i] = (int16_t) t;
    }
    asm volatile("" ::: "memory");    // the wave's LDS writes stay ahead of its reads
}

// The same arithmetic for N chunks of one wave, written stage by stage so that the N
// dependency chains (cross-lane steps, divisions) interleave instead of running one
// after another.  rms_chunk_sums = rms_chunk_sum per chunk; quantize_chunks =
// quantize_chunk<false> per chunk under norm (chunk index j[i]), plus the 16-value code
// sums of each chunk into s16[16 j[i] ..].
template <int N>
__device__ __forceinline__ void rms_chunk_sums(const v4f xv[N], float out[N]) {
    float a[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        a[i] = fmaf(xv[i].x, xv[i].x, 0.0f);
        a[i] = fmaf(xv[i].y, xv[i].y, a[i]);
        a[i] = fmaf(xv[i].z, xv[i].z, a[i]);
        a[i] = fmaf(xv[i].w, xv[i].w, a[i]);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) a[i] += from_lane_plus32(a[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) a[i] += from_lane_plus16(a[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) a[i] += dpp_f<DPP_ROW_SHL8>(0.0f, a[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) a[i] += dpp_f<DPP_ROW_SHL4>(0.0f, a[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) a[i] += dpp_f<DPP_QUAD_XOR2>(0.0f, a[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) a[i] += dpp_f<DPP_QUAD_XOR1>(0.0f, a[i]);
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a[i]), 0));
}

// USTRIDE: bytes from one 256-value chunk's eight q8_1 blocks to the next chunk's in y (288:
// packed, as ggml stores the row; Q8_1_LDS_STRIDE: padded, so that 16 chunks' 16-byte LDS reads
// fall in 16 distinct bank groups).
template <int N, int USTRIDE = 288>
__device__ __forceinline__ void quantize_chunks(const v4f xv[N], const v4f nwv[N], float s, uint8_t *y, const int j[N],
                                                int16_t *s16) {
    const int lane = threadIdx.x % WAVE;
    float v[N][4], amax[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        v[i][0] = (xv[i].x * s) * nwv[i].x;
        v[i][1] = (xv[i].y * s) * nwv[i].y;
        v[i][2] = (xv[i].z * s) * nwv[i].z;
        v[i][3] = (xv[i].w * s) * nwv[i].w;
        amax[i] = fmaxf(fmaxf(fabsf(v[i][0]), fabsf(v[i][1])), fmaxf(fabsf(v[i][2]), fabsf(v[i][3])));
    }
#pragma unroll
    for (int i = 0; i < N; ++i) amax[i] = fmaxf(amax[i], dpp_f<DPP_QUAD_XOR1>(0.0f, amax[i]));
#pragma unroll
    for (int i = 0; i < N; ++i) amax[i] = fmaxf(amax[i], dpp_f<DPP_QUAD_XOR2>(0.0f, amax[i]));
#pragma unroll
    for (int i = 0; i < N; ++i) amax[i] = fmaxf(amax[i], dpp_f<DPP_ROW_HALF_MIRROR>(0.0f, amax[i]));
    float d[N], inv[N];
    bool dok[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        d[i] = amax[i] / 127.0f;
        dok[i] = q8_scale_ok(d[i]);
        inv[i] = q8_inv(d[i], dok[i]);
    }
    int q[N][4];
    u32 slow = 0u;
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            bool sl;
            q[i][k] = q8_code_fast(v[i][k], inv[i], dok[i], sl);
            slow |= (sl ? 1u : 0u) << (4 * i + k);
        }
    // rare (values next to a rounding boundary, degenerate blocks): one wave-uniform branch
    if (__builtin_amdgcn_ballot_w64(slow != 0u) != 0) {
#pragma unroll
        for (int i = 0; i < N; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (slow & (1u << (4 * i + k))) q[i][k] = q8_code_exact(v[i][k], d[i]);
    }
    u32 packed[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        packed[i] = 0u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int code = amax[i] == 0.0f ? 0 : q[i][k];
            packed[i] |= ((u32) code & 0xFFu) << (8 * k);
        }
    }
    int cs[N];
#pragma unroll
    for (int i = 0; i < N; ++i) cs[i] = sdot4(packed[i], 0x01010101u, 0);
#pragma unroll
    for (int i = 0; i < N; ++i) cs[i] += __builtin_amdgcn_update_dpp(0, cs[i], DPP_QUAD_XOR1, 0xF, 0xF, false);
#pragma unroll
    for (int i = 0; i < N; ++i) cs[i] += __builtin_amdgcn_update_dpp(0, cs[i], DPP_QUAD_XOR2, 0xF, 0xF, false);
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int e = 4 * lane;                          // value index within chunk j[i]
        uint8_t *yb = y + j[i] * USTRIDE + (e / 32) * 36;
        *(u32 *) (yb + 4 + (e % 32)) = packed[i];
        *(u32 *) yb = (u32) f2h_bits(d[i]);
        s16[16 * j[i] + lane / 4] = (int16_t) cs[i];
    }
}

}  // namespace mc

#endif
