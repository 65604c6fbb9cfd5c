// mc_mmq.hip -- prefill-shaped MUL_MAT_ID on gfx950: the (token, slot) pairs are
// grouped by expert and each expert's weights are multiplied against all of its
// pairs at once with int8 MFMA (v_mfma_i32_16x16x32_i8).
//
// Replaces the many-token MUL_MAT_ID path the reference leaves to upstream
// ggml (MMQ; results/final.patch:45-48 only routes batch-1 decode to the
// pointer-table GEMV).  Activations are q8_K rows (one scale per 256 values,
// exact 16-value sums), the ggml-CPU vec_dot_type of the K-quants
// (patches/trace-hook/ggml-cpu.c:308-340): the sub-block products of a
// super-block then accumulate exactly in int32, with one float update per
// super-block.  Q4_K/Q5_K scale each 32-value MFMA result by its 6-bit
// sub-block scale; Q2_K (16-value groups) folds its 4-bit scales into the
// weight codes and takes the min term from a second MFMA; Q3_K and Q6_K
// (16-value groups, signed scales) split each sub-block into one MFMA per group.
//
// Three launches:
//   1. mc_mmq_group_kernel  (one workgroup): pair counts per expert, offsets,
//      the pair list grouped by expert and a table of 16-pair column blocks.
//   2. mc_mmq_pack_kernel: per (super-block, column block) one record holding the
//      MFMA A fragments of the 16 pairs' activation codes, their q8_K scales and
//      32-value sums (zeros for empty columns).
//   3. mc_mmq_gemm_kernel<T, GATE>: one workgroup per (64 weight rows, or 128 without a
//      fused gate and with one column block per pass; expert);
//      per super-block it DMAs the rows' weight blocks and the records of up
//      to MAXB column blocks into LDS (double-buffered), each wave
//      multiplies 16 weight rows against them, and the epilogue applies the GLU
//      (when a gate matrix is fused) and scatters to dst[token][slot][row].
// The position of a pair inside its expert's group depends on atomic order, but
// every pair's result is computed by the same integer MFMA sums and the same
// float operations wherever it lands, so the output does not depend on it.
#include <hip/hip_runtime.h>

#include "mc_core.h"
#include "mc_internal.h"

namespace mc {

typedef int v4i __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// 1. grouping
// ---------------------------------------------------------------------------

constexpr int MMQ_GROUP_THREADS = 1024;

// Exclusive prefix sum over a 1024-thread workgroup (each thread one value).
__device__ __forceinline__ int block_exclusive_scan(int v, int *lds_waves, int &total) {
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
    int incl = v;
#pragma unroll
    for (int off = 1; off < WAVE; off <<= 1) {
        const int o = __shfl_up(incl, off, WAVE);
        if (lane >= off) incl += o;
    }
    if (lane == WAVE - 1) lds_waves[wave] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0;
        for (int i = 0; i < MMQ_GROUP_THREADS / WAVE; ++i) {
            const int t = lds_waves[i];
            lds_waves[i] = run;
            run += t;
        }
        lds_waves[MMQ_GROUP_THREADS / WAVE] = run;
    }
    __syncthreads();
    total = lds_waves[MMQ_GROUP_THREADS / WAVE];
    const int r = lds_waves[wave] + incl - v;
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(MMQ_GROUP_THREADS) void mc_mmq_group_kernel(const MmqArgs a) {
    __shared__ int cnt[MMQ_MAX_EXPERTS];
    __shared__ int fill[MMQ_MAX_EXPERTS];
    __shared__ int scan_tmp[MMQ_GROUP_THREADS / WAVE + 1];
    int *offsets = (int *) (a.ws + a.ws_offsets);      // [E + 1]
    int *blk_off = (int *) (a.ws + a.ws_blk_off);      // [E + 1]
    int *list = (int *) (a.ws + a.ws_list);            // [n_pairs]
    int *blk_tab = (int *) (a.ws + a.ws_blk_tab);      // [max_blocks][4]: expert, first position, pairs
    const int E = a.n_experts, n_pairs = a.n_tok * a.n_used;
    for (int e = threadIdx.x; e < E; e += MMQ_GROUP_THREADS) {
        cnt[e] = 0;
        fill[e] = 0;
    }
    __syncthreads();
    for (int p = threadIdx.x; p < n_pairs; p += MMQ_GROUP_THREADS) {
        const int t = p / a.n_used, c = p % a.n_used;
        const int e = a.ids[c + (int64_t) t * a.ids_stride];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // offsets and column-block offsets: experts in ascending order, 4 per thread
    constexpr int PER = MMQ_MAX_EXPERTS / MMQ_GROUP_THREADS;
    int c4[PER], b4[PER], csum = 0, bsum = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = threadIdx.x * PER + i;
        c4[i] = e < E ? cnt[e] : 0;
        b4[i] = (c4[i] + MMQ_COLS - 1) / MMQ_COLS;
        csum += c4[i];
        bsum += b4[i];
    }
    int ctot, btot;
    int crun = block_exclusive_scan(csum, scan_tmp, ctot);
    int brun = block_exclusive_scan(bsum, scan_tmp, btot);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = threadIdx.x * PER + i;
        if (e < E) {
            offsets[e] = crun;
            blk_off[e] = brun;
            for (int b = 0; b < b4[i]; ++b) {
                int *row = blk_tab + 4 * (brun + b);
                row[0] = e;
                row[1] = crun + MMQ_COLS * b;
                row[2] = min(MMQ_COLS, c4[i] - MMQ_COLS * b);
                row[3] = 0;
            }
            fill[e] = crun;
        }
        crun += c4[i];
        brun += b4[i];
    }
    if (threadIdx.x == 0) {
        offsets[E] = ctot;
        blk_off[E] = btot;
    }
    __syncthreads();
    for (int p = threadIdx.x; p < n_pairs; p += MMQ_GROUP_THREADS) {
        const int t = p / a.n_used, c = p % a.n_used;
        const int e = a.ids[c + (int64_t) t * a.ids_stride];
        if (e >= 0 && e < E) list[atomicAdd(&fill[e], 1)] = p;
    }
}

// ---------------------------------------------------------------------------
// 2. activation records
// ---------------------------------------------------------------------------

// Record of one (super-block s, column block b), at ws_packed + (s * max_blocks + b) * MMQ_REC_BYTES:
//   [0, 4096)     A fragments: sub-block sb, lane l -> 8 codes of pair l % 16, values 32 sb + 8 (l / 16) .. +7
//   [4096, 4160)  d8[16]: the pairs' q8_K scales
//   [4160, 4416)  S[16][8] int16: the pairs' 32-value code sums per sub-block
constexpr int MMQ_REC_FRAG = 0, MMQ_REC_D8 = 4096, MMQ_REC_SUM = 4160;

// One wave per record: lane l = col + 16 kq fills the A fragments of pair col, values
// 8 kq .. 8 kq + 7 of every sub-block (for a fixed sub-block the 64 lanes write 512
// contiguous bytes); the lanes with kq = 0 write the pair's scale and sums.
__global__ __launch_bounds__(256) void mc_mmq_pack_kernel(const MmqArgs a) {
    const int n_sb = a.ncols / 256;
    const int64_t gid = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;   // (super-block, block, lane)
    const int lane = (int) (gid % WAVE);
    const int64_t sb_b = gid / WAVE;
    const int b = (int) (sb_b % a.max_blocks);
    const int s = (int) (sb_b / a.max_blocks);
    const int *blk_off = (const int *) (a.ws + a.ws_blk_off);
    if (s >= n_sb || b >= blk_off[a.n_experts]) return;
    const int col = lane % MMQ_COLS, kq = lane / MMQ_COLS;
    const int *row = (const int *) (a.ws + a.ws_blk_tab) + 4 * b;
    uint8_t *rec = a.ws + a.ws_packed + ((int64_t) s * a.max_blocks + b) * MMQ_REC_BYTES;
    uint64_t *frag = (uint64_t *) (rec + MMQ_REC_FRAG);
    float *d8 = (float *) (rec + MMQ_REC_D8);
    int16_t *sums = (int16_t *) (rec + MMQ_REC_SUM) + 8 * col;
    if (col >= row[2]) {                      // empty column: zero codes, scale and sums
#pragma unroll
        for (int sb = 0; sb < 8; ++sb) frag[sb * 64 + lane] = 0;
        if (kq == 0) {
            d8[col] = 0.0f;
            *(v4u *) sums = v4u{0u, 0u, 0u, 0u};
        }
        return;
    }
    const int p = ((const int *) (a.ws + a.ws_list))[row[1] + col];
    const int t = p / a.n_used, c = p % a.n_used;
    const uint8_t *blk = a.y + (int64_t) (c % a.nchannels_y) * a.stride_channel_y + (int64_t) t * a.stride_col_y +
                         (int64_t) s * 292;
    const uint64_t *qs = (const uint64_t *) (blk + 4);     // q8_K: d (4 B) | qs[256] | bsums[16] int16
#pragma unroll
    for (int sb = 0; sb < 8; ++sb) frag[sb * 64 + lane] = qs[4 * sb + kq];
    if (kq == 0) {
        d8[col] = *(const float *) blk;
        const int16_t *bs = (const int16_t *) (blk + 260);
#pragma unroll
        for (int sb = 0; sb < 8; ++sb) sums[sb] = (int16_t) (bs[2 * sb] + bs[2 * sb + 1]);
    }
}

// ---------------------------------------------------------------------------
// 3. grouped GEMM
// ---------------------------------------------------------------------------

// LDS tile geometry of one row's super-block and the DMA pieces that fill it:
//   Q4_K/Q5_K (144/176 B): 16-byte pieces, rows back to back;
//   Q2_K (84 B): dword pieces, rows back to back;
//   Q3_K / Q6_K (110 / 210 B, a row's super-blocks only 2-byte aligned in memory):
//   the dword-aligned 112 / 212-byte window around each super-block, rows back to back; the
//   super-block starts sh = (its address & 3) bytes into its window (0 or 2), and
//   the decode reads its words with byte alignment (v_alignbyte).  The window's
//   extra two bytes belong to a neighbouring super-block (or read as zeros past
//   the buffer) and are never used.  (Buffer->LDS DMA of 1- or 2-byte pieces writes
//   one dword per lane, so it cannot pack 2-byte aligned rows.)
template <int T, int NW = MMQ_WAVES>
struct MmqTile {
    static constexpr int ROWS = 16 * NW;                                // weight rows per workgroup
    static constexpr int SBB = type_geom(T).block_bytes;
    static constexpr bool WIN = SBB % 4 != 0;
    static constexpr int DB = SBB % 16 == 0 ? 16 : 4;                  // bytes per lane and DMA
    static constexpr int RP = WIN ? SBB + 2 : SBB;                      // LDS row pitch
    static constexpr int CH = RP / DB;                                  // pieces per row
    static constexpr int N_INS = ROWS * RP / (WAVE * DB);               // wave DMA instructions per tile
    static constexpr uint32_t WT = ROWS * RP;                           // LDS tile bytes
    static_assert(!WIN || SBB % 4 == 2, "windows cover super-blocks that are 2-byte aligned");
    static_assert(ROWS * RP % (WAVE * DB) == 0, "whole DMA instructions per tile");
};

// Per-lane byte offsets of the wave's weight-tile DMA instructions (instruction
// wave + NW k), without the super-block term s * SBB: they depend only on the
// workgroup's rows, so they are computed once, not per stage.  Piece q of the tile is
// part q % CH of row q / CH.  A windowed type's window starts at the dword below its
// super-block; as the part offset DB (q % CH) is a multiple of 4, that rounding can be
// applied to the sum (row start + part + s * SBB).
template <int T, int NW>
struct MmqLanes {
    static constexpr int K = (MmqTile<T, NW>::N_INS + NW - 1) / NW;
    uint32_t off[K];            // b0 + (row0 + q / CH) * row_bytes + DB * (q % CH)
};

template <int T, int NW>
__device__ __forceinline__ void mmq_lanes(const MmqArgs &a, const uint8_t *wbase, int row0, int wave, MmqLanes<T, NW> &L) {
    using G = MmqTile<T, NW>;
    static_assert(G::DB % 4 == 0, "part offsets are dword multiples");
    const int lane = threadIdx.x % WAVE;
    const uint32_t row_bytes = (uint32_t) (a.ncols / 256) * G::SBB;
    const uint32_t b0 = (uint32_t) ((uintptr_t) wbase & 3u);     // 0 except for a 2-byte aligned Q6_K expert
#pragma unroll
    for (int k = 0; k < MmqLanes<T, NW>::K; ++k) {
        const int q = (wave + NW * k) * WAVE + lane;
        L.off[k] = b0 + (uint32_t) (row0 + q / G::CH) * row_bytes + (uint32_t) G::DB * (uint32_t) (q % G::CH);
    }
}

// Issues the DMA of super-block s: 16 NW weight rows (one super-block, or its
// window, each; rows row_bytes apart in memory, back to back in LDS) and nb
// activation records.  wave is the wave's index, uniform across the wave.
template <int T, int NW>
__device__ __forceinline__ void mmq_issue(const MmqArgs &a, const uint8_t *wbase, const MmqLanes<T, NW> &L, int wave, int s,
                                          int blk0, int nb, uint8_t *wl, uint8_t *rl) {
    using G = MmqTile<T, NW>;
    const int lane = threadIdx.x % WAVE;
    const uint32_t b0 = (uint32_t) ((uintptr_t) wbase & 3u);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(wbase - b0, (uint32_t) a.expert_bytes + b0);
    const uint32_t so = (uint32_t) s * G::SBB;
#pragma unroll
    for (int k = 0; k < MmqLanes<T, NW>::K; ++k) {
        const int i = wave + NW * k;
        if (i >= G::N_INS) break;
        const uint32_t off = G::WIN ? (L.off[k] + so) & ~3u : L.off[k] + so;
        lds_void_t *dst = (lds_void_t *) (wl + WAVE * G::DB * i);
        if constexpr (G::DB == 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, dst, 16, off, 0, 0, 0);
        else __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, dst, 4, off, 0, 0, 0);
    }
    if (nb <= 0) return;
    const uint8_t *recs = a.ws + a.ws_packed + ((int64_t) s * a.max_blocks + blk0) * MMQ_REC_BYTES;
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(recs, (uint32_t) nb * MMQ_REC_BYTES);
    const int rounds = (nb * MMQ_REC_BYTES + 1023) / 1024;
    for (int i = wave; i < rounds; i += NW)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_void_t *) (rl + 1024 * i), 16, 1024u * i + 16u * lane, 0, 0, 0);
}

template <int NW>
__device__ __forceinline__ int mmq_issue_count(int nb, int wave, int n_ins) {
    int n = 0;
    for (int i = wave; i < n_ins; i += NW) ++n;
    for (int i = wave; i < (nb * MMQ_REC_BYTES + 1023) / 1024; i += NW) ++n;
    return n;
}

// d8 * d * isum - d8 * dmin * msum, the q8_K super-block result (products unfused).
__device__ __forceinline__ float mmq_superblock_value(float d8, float d, float dmin, int isum, int msum) {
#pragma clang fp contract(off)
    const float dall = d8 * d, dmn = d8 * dmin;
    return dall * (float) isum - dmn * (float) msum;
}

// Decoded scale words of one K-quant row super-block (Q4_K/Q5_K): d, dmin and the
// packed 6-bit sub-block scales and mins (kq_scales).
struct RowScales {
    float d, dmin;
    u32 SC0, SC1, M0, M1;
};

__device__ __forceinline__ RowScales row_scales(const u32 *w) {
    RowScales r;
    r.d = h2f(w[0]);
    r.dmin = h2f(w[0] >> 16);
    kq_scales(w[1], w[2], w[3], r.SC0, r.SC1, r.M0, r.M1);
    return r;
}

// B fragments of sub-blocks 2c and 2c+1 for this lane (weight row lane % 16, values
// 8 (lane / 16) .. +7 of each sub-block) from the row's super-block at w.
template <int T>
__device__ __forceinline__ void row_frags(const u32 *w, int c, int kq, long &lo, long &hi) {
    constexpr bool Q5 = T == T_Q5_K;
    constexpr int QS = Q5 ? 12 : 4;                         // dword offset of qs[128]
    const u32 q0 = w[QS + 8 * c + 2 * kq], q1 = w[QS + 8 * c + 2 * kq + 1];
    u32 lo0 = q0 & 0x0F0F0F0Fu, lo1 = q1 & 0x0F0F0F0Fu;
    u32 hi0 = (q0 >> 4) & 0x0F0F0F0Fu, hi1 = (q1 >> 4) & 0x0F0F0F0Fu;
    if constexpr (Q5) {                                      // high bit of element l of sub-block g: qh[l] bit g
        const u32 h0 = w[4 + 2 * kq], h1 = w[4 + 2 * kq + 1];
        lo0 |= ((h0 >> (2 * c)) & 0x01010101u) << 4;
        lo1 |= ((h1 >> (2 * c)) & 0x01010101u) << 4;
        hi0 |= ((h0 >> (2 * c + 1)) & 0x01010101u) << 4;
        hi1 |= ((h1 >> (2 * c + 1)) & 0x01010101u) << 4;
    }
    lo = (long) (((uint64_t) lo1 << 32) | lo0);
    hi = (long) (((uint64_t) hi1 << 32) | hi0);
}

// Sub-block products of one matrix against one column block, accumulated into isum.
__device__ __forceinline__ void mmq_mfma_pair(long a_lo, long a_hi, long b_lo, long b_hi, u32 SC, int c,
                                              int (&isum)[4]) {
    const v4i rl = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_lo, b_lo, v4i{0, 0, 0, 0}, 0, 0, 0);
    const v4i rh = __builtin_amdgcn_mfma_i32_16x16x32_i8(a_hi, b_hi, v4i{0, 0, 0, 0}, 0, 0, 0);
    const int sl = (int) byte_of(SC, (2 * c) & 3), sh = (int) byte_of(SC, (2 * c + 1) & 3);
#pragma unroll
    for (int i = 0; i < 4; ++i) isum[i] += __mul24(sl, rl[i]) + __mul24(sh, rh[i]);
}

// The eight sub-block mins (bytes of M0, M1) as int16 pairs (m_2k, m_2k+1), the
// layout of a record's 32-value code sums.
__device__ __forceinline__ void mins_pairs(u32 M0, u32 M1, u32 (&mp)[4]) {
    mp[0] = __builtin_amdgcn_perm(0u, M0, 0x0C010C00u);
    mp[1] = __builtin_amdgcn_perm(0u, M0, 0x0C030C02u);
    mp[2] = __builtin_amdgcn_perm(0u, M1, 0x0C010C00u);
    mp[3] = __builtin_amdgcn_perm(0u, M1, 0x0C030C02u);
}

// Sum of the eight sub-block mins times a pair's 32-value code sums (eight int16 in
// s4, sub-blocks 2k and 2k+1 in word k): four v_dot2 (exact integers).
__device__ __forceinline__ int mins_dot(const u32 (&mp)[4], const v4u s4) {
    int r = sdot2_z(mp[0], s4.x);
    r = sdot2(mp[1], s4.y, r);
    r = sdot2(mp[2], s4.z, r);
    return sdot2(mp[3], s4.w, r);
}

// One super-block of one 16-row weight tile (the wave's rows, the lane's row =
// lane % 16) of the up matrix (and the gate) against nb column blocks: acc[b][i]
// for pair 4 (lane / 16) + i of block b.
template <int T, bool GATE, int MAXB>
__device__ __forceinline__ void mmq_superblock(const uint8_t *wrow_up, const uint8_t *wrow_gate, const uint8_t *recs,
                                               int nb, float (&acc)[MAXB][4], float (&accg)[MAXB][4]) {
    const int lane = threadIdx.x % WAVE;
    const int kq = lane / 16;
    const u32 *wu = (const u32 *) wrow_up;
    const u32 *wg = (const u32 *) wrow_gate;
    const RowScales su = row_scales(wu);
    RowScales sg{};
    if constexpr (GATE) sg = row_scales(wg);
    u32 mpu[4], mpg[4] = {0u, 0u, 0u, 0u};
    mins_pairs(su.M0, su.M1, mpu);
    if constexpr (GATE) mins_pairs(sg.M0, sg.M1, mpg);
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
        if (b >= nb) break;
        const uint8_t *rec = recs + b * MMQ_REC_BYTES;
        const long *af = (const long *) (rec + MMQ_REC_FRAG);
        int iu[4] = {0, 0, 0, 0}, ig[4] = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const long a_lo = af[(2 * c) * 64 + lane], a_hi = af[(2 * c + 1) * 64 + lane];
            long b_lo, b_hi;
            row_frags<T>(wu, c, kq, b_lo, b_hi);
            mmq_mfma_pair(a_lo, a_hi, b_lo, b_hi, c < 2 ? su.SC0 : su.SC1, c, iu);
            if constexpr (GATE) {
                row_frags<T>(wg, c, kq, b_lo, b_hi);
                mmq_mfma_pair(a_lo, a_hi, b_lo, b_hi, c < 2 ? sg.SC0 : sg.SC1, c, ig);
            }
        }
        const v4f d8 = *(const v4f *) (rec + MMQ_REC_D8 + 16 * kq);
        const float d8a[4] = {d8.x, d8.y, d8.z, d8.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const v4u s4 = *(const v4u *) (rec + MMQ_REC_SUM + 16 * (4 * kq + i));
            acc[b][i] += mmq_superblock_value(d8a[i], su.d, su.dmin, iu[i], mins_dot(mpu, s4));
            if constexpr (GATE) accg[b][i] += mmq_superblock_value(d8a[i], sg.d, sg.dmin, ig[i], mins_dot(mpg, s4));
        }
    }
}

// B fragments of one Q2_K row super-block (84 bytes at w: scales[16], qs[64], d, dmin)
// for this lane (weight row lane % 16, values 8 kq .. 8 kq + 7 of each 32-value
// sub-block, kq = lane / 16).  Element 128 h + 32 j + l is bits 2j of qs[32 h + l]
// in 16-value group 8 h + 2 j + l / 16; a lane's eight values share one group.
//   bq[sb]: the codes times the group's 4-bit scale (at most 3 * 15 = 45, so one
//           32-bit multiply scales four bytes without carries);
//   bm[sb]: the group's 4-bit min in all eight bytes (its MFMA against the
//           activation codes is the min term's sum over the group).
__device__ __forceinline__ void q2K_frags(const u32 *w, int kq, long (&bq)[8], long (&bm)[8]) {
    const int hk = kq >> 1;                                 // which half of the 32 values
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const u32 c0 = w[4 + 8 * h + 2 * kq], c1 = w[4 + 8 * h + 2 * kq + 1];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // scales[8 h + 2 j + hk] = byte 2 (j & 1) + hk of word 2 h + j / 2
            const u32 sbyte = (w[2 * h + (j >> 1)] >> (8 * (2 * (j & 1) + hk))) & 0xFFu;
            const u32 sc = sbyte & 0xFu, m = sbyte >> 4;
            const u32 lo = ((c0 >> (2 * j)) & 0x03030303u) * sc;
            const u32 hi = ((c1 >> (2 * j)) & 0x03030303u) * sc;
            const u32 mm = m * 0x01010101u;
            bq[4 * h + j] = (long) (((uint64_t) hi << 32) | lo);
            bm[4 * h + j] = (long) (((uint64_t) mm << 32) | mm);
        }
    }
}

// Q2_K: one super-block of the wave's 16-row tile against nb column blocks.  The
// scaled-code and min MFMAs accumulate the super-block's isum and msum directly
// (exact int32), then one float update per pair as for the other K-quants.
template <bool GATE, int MAXB>
__device__ __forceinline__ void mmq_superblock_q2K(const uint8_t *wrow_up, const uint8_t *wrow_gate,
                                                   const uint8_t *recs, int nb, float (&acc)[MAXB][4],
                                                   float (&accg)[MAXB][4]) {
    const int lane = threadIdx.x % WAVE;
    const int kq = lane / 16;
    const u32 *wu = (const u32 *) wrow_up;
    const u32 *wg = (const u32 *) wrow_gate;
    long qu[8], mu[8], qg[8], mg[8];
    q2K_frags(wu, kq, qu, mu);
    const float du = h2f(wu[20]), dmu = h2f(wu[20] >> 16);
    float dg = 0.0f, dmg = 0.0f;
    if constexpr (GATE) {
        q2K_frags(wg, kq, qg, mg);
        dg = h2f(wg[20]);
        dmg = h2f(wg[20] >> 16);
    }
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
        if (b >= nb) break;
        const uint8_t *rec = recs + b * MMQ_REC_BYTES;
        const long *af = (const long *) (rec + MMQ_REC_FRAG);
        v4i iu = {0, 0, 0, 0}, su = {0, 0, 0, 0}, ig = {0, 0, 0, 0}, sg = {0, 0, 0, 0};
#pragma unroll
        for (int sb = 0; sb < 8; ++sb) {
            const long a = af[sb * 64 + lane];
            iu = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, qu[sb], iu, 0, 0, 0);
            su = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, mu[sb], su, 0, 0, 0);
            if constexpr (GATE) {
                ig = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, qg[sb], ig, 0, 0, 0);
                sg = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, mg[sb], sg, 0, 0, 0);
            }
        }
        const v4f d8 = *(const v4f *) (rec + MMQ_REC_D8 + 16 * kq);
        const float d8a[4] = {d8.x, d8.y, d8.z, d8.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[b][i] += mmq_superblock_value(d8a[i], du, dmu, iu[i], su[i]);
            if constexpr (GATE) accg[b][i] += mmq_superblock_value(d8a[i], dg, dmg, ig[i], sg[i]);
        }
    }
}

// Q6_K row super-block (ql[128], qh[64], scales[16] int8, d) sh bytes into its LDS
// window w.  Element 128 n + 32 j + l (n = 0, 1; j = 0..3; l = 0..31) is
//   ((ql[64 n + 32 (j & 1) + l] >> 4 (j >> 1)) & 15 | ((qh[32 n + l] >> 2 j) & 3) << 4) - 32
// in 16-value group 8 n + 2 j + l / 16.  B fragment of sub-block 4 n + j for this lane
// (values 8 kq .. 8 kq + 7): the eight codes as int8.  code - 32 is the code with
// bit 5 flipped read as a 6-bit two's complement number, so it is sign-extended
// from bit 5 (bits 6 and 7 set where bit 5 is), bytewise without carries.
__device__ __forceinline__ u32 win_word(const u32 *w, u32 sh, int k) {
    // word k of a super-block that starts sh bytes into the dword-aligned window w
    return __builtin_amdgcn_alignbyte(w[k + 1], w[k], sh);
}

__device__ __forceinline__ long q6K_codes(const u32 *w, u32 sh, int n, int j, int kq) {
    const int qlw = 16 * n + 8 * (j & 1) + 2 * kq;          // ql word of values 8 kq ..
    const int qhw = 32 + 8 * n + 2 * kq;                    // qh word (qh starts at byte 128)
    u32 r[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const u32 lo = (win_word(w, sh, qlw + h) >> (4 * (j >> 1))) & 0x0F0F0F0Fu;
        const u32 hi = ((win_word(w, sh, qhw + h) >> (2 * j)) & 0x03030303u) << 4;
        const u32 t = (lo | hi) ^ 0x20202020u;
        const u32 sgn = t & 0x20202020u;
        r[h] = t | (sgn << 1) | (sgn << 2);
    }
    return (long) (((uint64_t) r[1] << 32) | r[0]);
}

// Q6_K: one super-block of the wave's 16-row tile against nb column blocks.  A lane's
// eight values share one 16-value group (even for kq < 2, odd otherwise), so each
// 32-value sub-block takes two MFMAs, one with only the even group's lanes and one
// with only the odd group's, each scaled by its group's int8 scale; no min term.
// Q3_K row super-block (hmask[32], qs[64], scales[12], d) sh bytes into its LDS window
// w.  Element 128 h + 32 j + l (h = 0, 1; j = 0..3; l = 0..31) is
//   ((qs[32 h + l] >> 2 j) & 3) - ((hmask[l] >> (4 h + j)) & 1 ? 0 : 4)
// in 16-value group 8 h + 2 j + l / 16.  B fragment of sub-block 4 h + j for this lane:
// the eight codes as int8: (low | high << 2) ^ 4 is the code's 3-bit two's complement,
// sign-extended from bit 2 (bits 3..7 set where bit 2 is, bytewise without carries).
__device__ __forceinline__ long q3K_codes(const u32 *w, u32 sh, int h, int j, int kq) {
    u32 r[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const u32 lo = (win_word(w, sh, 8 + 8 * h + 2 * kq + i) >> (2 * j)) & 0x03030303u;   // qs at byte 32
        const u32 hb = (win_word(w, sh, 2 * kq + i) >> (4 * h + j)) & 0x01010101u;          // hmask at byte 0
        const u32 t = (lo | (hb << 2)) ^ 0x04040404u;
        r[i] = t | ((t & 0x04040404u) * 62u);
    }
    return (long) (((uint64_t) r[1] << 32) | r[0]);
}

// The 6-bit scale of 16-value group g (ggml's Q3_K packing: low nibbles in bytes
// 0..7, two high bits per scale in bytes 8..11), offset by -32.
__device__ __forceinline__ int q3K_scale(const u32 *w, u32 sh, int g) {
    const u32 a03 = win_word(w, sh, 24), a47 = win_word(w, sh, 25), a8b = win_word(w, sh, 26);   // scales at byte 96
    const u32 lw = (g & 7) < 4 ? a03 : a47;
    const u32 lo = (lw >> (8 * (g & 3) + 4 * (g >> 3))) & 0xFu;
    const u32 hi = (a8b >> (8 * (g & 3) + 2 * (g >> 2))) & 3u;
    return (int) (lo | (hi << 4)) - 32;
}

// The B fragment (codes) and the even / odd group scales of sub-block sb for a
// 16-value-group type whose super-blocks arrive in windows (Q3_K, Q6_K).
template <int T>
__device__ __forceinline__ void g16_subblock(const u32 *w, u32 sh, int sb, int kq, long &codes, int &se, int &so) {
    const int n = sb >> 2, j = sb & 3;
    if constexpr (T == T_Q6_K) {
        // scales[8 n + 2 j] and [8 n + 2 j + 1]: bytes 2 (j & 1) and 2 (j & 1) + 1 of word 48 + 2 n + j / 2
        codes = q6K_codes(w, sh, n, j, kq);
        const u32 sw = win_word(w, sh, 48 + 2 * n + (j >> 1)) >> (16 * (j & 1));
        se = (int) (int8_t) (sw & 0xFFu);
        so = (int) (int8_t) ((sw >> 8) & 0xFFu);
    } else {
        codes = q3K_codes(w, sh, n, j, kq);
        se = q3K_scale(w, sh, 8 * n + 2 * j);
        so = q3K_scale(w, sh, 8 * n + 2 * j + 1);
    }
}

// Byte offset of d in a super-block of a 16-value-group type.
template <int T>
constexpr int g16_d_offset() { return T == T_Q6_K ? 208 : 108; }

// A window that starts on its super-block (sh = 0) ends two bytes past it; at the very
// end of a matrix those bytes lie outside the buffer, and the DMA returns the whole
// last dword (d and the two bytes) as zeros.  For that super-block (tail) d is read
// from memory instead: gup / ggt point at the super-block's bytes in the up / gate
// matrix.
//
// Q3_K / Q6_K: one super-block of the wave's 16-row tile against nb column blocks.  A
// lane's eight values share one 16-value group (even for kq < 2, odd otherwise), so
// each 32-value sub-block takes two MFMAs, one with only the even group's lanes and
// one with only the odd group's, each scaled by its group's scale; no min term.
template <int T, bool GATE, int MAXB>
__device__ __forceinline__ void mmq_superblock_g16(const uint8_t *wrow_up, const uint8_t *wrow_gate, u32 sh,
                                                   bool tail, const uint8_t *gup, const uint8_t *ggt,
                                                   const uint8_t *recs, int nb, float (&acc)[MAXB][4],
                                                   float (&accg)[MAXB][4]) {
    constexpr int DO = g16_d_offset<T>();
    const int lane = threadIdx.x % WAVE;
    const int kq = lane / 16;
    const bool even = kq < 2;
    const u32 *wu = (const u32 *) wrow_up;
    const u32 *wg = (const u32 *) wrow_gate;
    long cu[8], cg[8];
    int seu[8], sou[8], seg[8], sog[8];
#pragma unroll
    for (int sb = 0; sb < 8; ++sb) {
        g16_subblock<T>(wu, sh, sb, kq, cu[sb], seu[sb], sou[sb]);
        if constexpr (GATE) g16_subblock<T>(wg, sh, sb, kq, cg[sb], seg[sb], sog[sb]);
    }
    const float du = h2f(tail ? (u32) * (const uint16_t *) (gup + DO) : win_word(wu, sh, DO / 4));
    const float dg = GATE ? h2f(tail ? (u32) * (const uint16_t *) (ggt + DO) : win_word(wg, sh, DO / 4)) : 0.0f;
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
        if (b >= nb) break;
        const uint8_t *rec = recs + b * MMQ_REC_BYTES;
        const long *af = (const long *) (rec + MMQ_REC_FRAG);
        int iu[4] = {0, 0, 0, 0}, ig[4] = {0, 0, 0, 0};
#pragma unroll
        for (int sb = 0; sb < 8; ++sb) {
            const long a = af[sb * 64 + lane];
            const v4i ue = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, even ? cu[sb] : 0l, v4i{0, 0, 0, 0}, 0, 0, 0);
            const v4i uo = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, even ? 0l : cu[sb], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) iu[i] += __mul24(seu[sb], ue[i]) + __mul24(sou[sb], uo[i]);
            if constexpr (GATE) {
                const v4i ge = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, even ? cg[sb] : 0l, v4i{0, 0, 0, 0}, 0, 0, 0);
                const v4i go = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, even ? 0l : cg[sb], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) ig[i] += __mul24(seg[sb], ge[i]) + __mul24(sog[sb], go[i]);
            }
        }
        const v4f d8 = *(const v4f *) (rec + MMQ_REC_D8 + 16 * kq);
        const float d8a[4] = {d8.x, d8.y, d8.z, d8.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[b][i] += mmq_superblock_value(d8a[i], du, 0.0f, iu[i], 0);
            if constexpr (GATE) accg[b][i] += mmq_superblock_value(d8a[i], dg, 0.0f, ig[i], 0);
        }
    }
}

template <int T, bool GATE, int MAXB>
__global__ __launch_bounds__(mmq_waves(GATE, MAXB) * WAVE) void mc_mmq_gemm_kernel(const MmqArgs a) {
    constexpr int NW = mmq_waves(GATE, MAXB);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    using G = MmqTile<T, NW>;
    constexpr int N_INS = G::N_INS;
    constexpr uint32_t WT = G::WT;                          // weight tile bytes per matrix and super-block
    // the wave index is uniform across the wave: keep it (and the loops over it) scalar
    const int lane = threadIdx.x % WAVE, wave = __builtin_amdgcn_readfirstlane((int) (threadIdx.x / WAVE));
    const int e = blockIdx.y;
    const int *blk_off = (const int *) (a.ws + a.ws_blk_off);
    const int blk_first = blk_off[e], nblk = blk_off[e + 1] - blk_first;
    if (nblk <= 0) return;
    const int row0 = blockIdx.x * G::ROWS;
    const int n_sb = a.ncols / 256;
    const uint8_t *wup = a.w + (int64_t) e * a.expert_bytes;
    const uint8_t *wgt = GATE ? a.w_gate + (int64_t) e * a.expert_bytes : nullptr;
    // LDS: two stages of [up tile | gate tile | records]
    const uint32_t stage = (GATE ? 2u : 1u) * WT + MAXB * MMQ_REC_BYTES + 1024u;
    const int *blk_tab = (const int *) (a.ws + a.ws_blk_tab);
    const int *list = (const int *) (a.ws + a.ws_list);
    MmqLanes<T, NW> lanes;                                  // the gate's DMA has the same offsets
    mmq_lanes<T, NW>(a, wup, row0, wave, lanes);

    for (int g0 = 0; g0 < nblk; g0 += MAXB) {
        const int nb = min(MAXB, nblk - g0);
        float acc[MAXB][4], accg[MAXB][4];
#pragma unroll
        for (int b = 0; b < MAXB; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[b][i] = accg[b][i] = 0.0f;
        const int per_stage = mmq_issue_count<NW>(nb, wave, N_INS) + (GATE ? mmq_issue_count<NW>(0, wave, N_INS) : 0);
        auto issue = [&](int s) {
            uint8_t *st = lds + (uint32_t) (s & 1) * stage;
            mmq_issue<T, NW>(a, wup, lanes, wave, s, blk_first + g0, nb, st, st + (GATE ? 2 : 1) * WT);
            if (GATE) mmq_issue<T, NW>(a, wgt, lanes, wave, s, blk_first + g0, 0, st + WT, nullptr);
        };
        issue(0);
        for (int s = 0; s < n_sb; ++s) {
            if (s + 1 < n_sb) {
                issue(s + 1);
                wait_loads_at_most(per_stage);                // stage s has landed for this wave
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            lds_barrier();                                    // ... and for every wave (stage s + 1 stays in flight)
            const uint8_t *st = lds + (uint32_t) (s & 1) * stage;
            const uint8_t *recs = st + (GATE ? 2 : 1) * WT;
            const uint32_t roff = (uint32_t) (16 * wave + lane % 16) * G::RP;
            if constexpr (T == T_Q2_K) mmq_superblock_q2K<GATE, MAXB>(st + roff, st + WT + roff, recs, nb, acc, accg);
            else if constexpr (G::WIN) {
                // where this row's super-block starts in its window: the same address
                // arithmetic as mmq_issue (both matrices of an expert share it when the
                // gate's base has the up's alignment, which the entry point checks)
                const int wrow = row0 + 16 * wave + lane % 16;
                const uint32_t b0 = (uint32_t) ((uintptr_t) wup & 3u);
                const uint32_t rel = (uint32_t) wrow * (uint32_t) (n_sb * G::SBB) + (uint32_t) s * G::SBB;
                const uint32_t sh = (b0 + rel) & 3u;
                // rows past nrows (the last tile's padding) are never stored and never read from memory
                const bool tail = wrow < a.nrows && sh == 0 && rel + G::RP > (uint32_t) a.expert_bytes;
                mmq_superblock_g16<T, GATE, MAXB>(st + roff, st + WT + roff, sh, tail, wup + rel,
                                                  GATE ? wgt + rel : nullptr, recs, nb, acc, accg);
            }
            else mmq_superblock<T, GATE, MAXB>(st + roff, st + WT + roff, recs, nb, acc, accg);
            lds_barrier();                                    // stage s is free for s + 2
        }
        // scatter: pair 4 (lane / 16) + i of each block, weight row lane % 16 of the wave's tile
        const int row = row0 + 16 * wave + lane % 16;
        if (row < a.nrows) {
#pragma unroll
            for (int b = 0; b < MAXB; ++b) {
                if (b >= nb) break;
                const int *tab = blk_tab + 4 * (blk_first + g0 + b);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int slot = 4 * (lane / 16) + i;
                    if (slot >= tab[2]) continue;
                    const int p = list[tab[1] + slot];
                    const int t = p / a.n_used, c = p % a.n_used;
                    const float out = GATE ? glu_apply(a.glu_op, accg[b][i], acc[b][i], a.glu_limit) : acc[b][i];
                    a.dst[(int64_t) t * a.stride_col_dst + (int64_t) c * a.stride_channel_dst + row] = out;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------

template <int T, int MAXB>
static hipError_t launch_mmq_tb(const MmqArgs &a, hipStream_t s) {
    using GG = MmqTile<T, mmq_waves(true, MAXB)>;
    using GP = MmqTile<T, mmq_waves(false, MAXB)>;
    const bool gate = a.w_gate != nullptr;
    const uint32_t stage = gate ? 2u * GG::WT + MAXB * MMQ_REC_BYTES + 1024u : GP::WT + MAXB * MMQ_REC_BYTES + 1024u;
    const int rows = gate ? GG::ROWS : GP::ROWS;
    const dim3 grid((unsigned) ((a.nrows + rows - 1) / rows), (unsigned) a.n_experts);
    // more than the default 64 KiB of dynamic LDS: raise the kernel's limit once
    static const hipError_t attr_gate = hipFuncSetAttribute((const void *) mc_mmq_gemm_kernel<T, true, MAXB>,
        hipFuncAttributeMaxDynamicSharedMemorySize, (int) (2 * (2 * GG::WT + MAXB * MMQ_REC_BYTES + 1024u)));
    static const hipError_t attr_plain = hipFuncSetAttribute((const void *) mc_mmq_gemm_kernel<T, false, MAXB>,
        hipFuncAttributeMaxDynamicSharedMemorySize, (int) (2 * (GP::WT + MAXB * MMQ_REC_BYTES + 1024u)));
    if (attr_gate != hipSuccess) return attr_gate;
    if (attr_plain != hipSuccess) return attr_plain;
    if (gate) hipLaunchKernelGGL((mc_mmq_gemm_kernel<T, true, MAXB>), grid, dim3(mmq_waves(true, MAXB) * WAVE), 2 * stage, s, a);
    else hipLaunchKernelGGL((mc_mmq_gemm_kernel<T, false, MAXB>), grid, dim3(mmq_waves(false, MAXB) * WAVE), 2 * stage, s, a);
    return hipGetLastError();
}

template <int T>
static hipError_t launch_mmq_t(const MmqArgs &a, hipStream_t s) {
    const int64_t pairs = (int64_t) a.n_tok * a.n_used;
    if (pairs <= (int64_t) MMQ_FEW_PAIRS * a.n_experts) return launch_mmq_tb<T, 1>(a, s);
    return launch_mmq_tb<T, MMQ_MAX_BLOCKS>(a, s);
}

// Grouping, activation records and the grouped GEMM; a.ws holds the workspace.
int launch_mmq(const MmqArgs &a, int type, void *stream) {
    hipStream_t s = (hipStream_t) stream;
    if (a.n_tok <= 0 || a.n_used <= 0) return (int) hipSuccess;
    if (a.n_experts > MMQ_MAX_EXPERTS || a.ncols % 256) return (int) hipErrorInvalidValue;
    hipLaunchKernelGGL(mc_mmq_group_kernel, dim3(1), dim3(MMQ_GROUP_THREADS), 0, s, a);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return (int) err;
    const int64_t threads = (int64_t) a.max_blocks * WAVE * (a.ncols / 256);
    hipLaunchKernelGGL(mc_mmq_pack_kernel, dim3((unsigned) ((threads + 255) / 256)), dim3(256), 0, s, a);
    if ((err = hipGetLastError()) != hipSuccess) return (int) err;
    switch (type) {
        case T_Q2_K: return (int) launch_mmq_t<T_Q2_K>(a, s);
        case T_Q3_K: return (int) launch_mmq_t<T_Q3_K>(a, s);
        case T_Q4_K: return (int) launch_mmq_t<T_Q4_K>(a, s);
        case T_Q6_K: return (int) launch_mmq_t<T_Q6_K>(a, s);
        case T_Q5_K: return (int) launch_mmq_t<T_Q5_K>(a, s);
        default: return (int) hipErrorInvalidValue;
    }
}

}  // namespace mc
