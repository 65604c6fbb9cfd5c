// mc_ssm_conv.hip -- the SSM depthwise causal convolution (ggml SSM_CONV) with F32
// or F16 conv weights and the optional fused bias + SiLU, on gfx950.
//
// Replaces kernels/ssm-conv.cu:5-217 (the reference's F16-weight fix of ggml's
// ssm_conv_f32 / ssm_conv_long_token_f32):
//   dst[s][t][r] = act( sum_{j < nc} x[s][r][t + j] * w[r][j]  (+ bias[r]) )
// x is conv_x: per sequence s and channel r a row of nc - 1 + n_t floats (time
// contiguous); w[r] holds the channel's nc taps (F32 or F16); dst is token-major
// with the channels contiguous.  act is SiLU when fused; bias comes only with it
// (kernels/ssm-conv.cu:160-161).  The sum is the reference's: taps in ascending
// j, each product added with one fused multiply-add starting from 0, then the
// bias.
//
// One workgroup (4 waves) per (64 channels, 64 tokens, sequence): the x tile
// (64 rows of 64 + nc - 1 floats) is read into LDS with the lanes along time
// (coalesced, all of a thread's loads in flight at once); each wave then takes
// 16 tokens with one channel per lane, keeps its 16 + nc - 1 window values in
// registers and writes 64 contiguous channels per token (coalesced).
// HBM-bound: x is read once and dst written once.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "mc_core.h"
#include "mc_internal.h"

namespace mc {

constexpr int SSM_CH = 64;                  // channels per workgroup (one per lane)
constexpr int SSM_TT = 64;                  // tokens per workgroup
constexpr int SSM_WAVES = 4;
constexpr int SSM_TW = SSM_TT / SSM_WAVES;  // tokens per wave

// LDS row pitch in floats: the tile's columns, made odd so the 64 lanes of a
// column read (one channel row each) fall in distinct banks.
constexpr int ssm_pitch(int nc) { return (SSM_TT + nc - 1) | 1; }

template <int NC, bool F16W, bool SILU>
__global__ __launch_bounds__(SSM_WAVES * WAVE) void mc_ssm_conv_kernel(const SsmConvArgs a) {
    constexpr int P = ssm_pitch(NC);
    constexpr int COLS = SSM_TT + NC - 1;
    constexpr int N_EL = SSM_CH * P;                              // the tile, row pitch P
    constexpr int PER = (N_EL + SSM_WAVES * WAVE - 1) / (SSM_WAVES * WAVE);
    __shared__ float tile[N_EL];
    const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
    const int t0 = blockIdx.y * SSM_TT, r0 = blockIdx.x * SSM_CH, s = blockIdx.z;
    const int n_ch = min(SSM_CH, (int) (a.nr - r0));
    const int n_cols = min(COLS, (int) (a.n_t - t0) + NC - 1);   // x columns this tile reads
    const uint8_t *xs = (const uint8_t *) a.x + (int64_t) s * a.x_nb2;
    // every load of the thread is issued before the first LDS write (one memory
    // latency per tile); tile element i is (row i / P, column i % P)
    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = (int) threadIdx.x + SSM_WAVES * WAVE * k;
        const int row = i / P, col = i % P;
        v[k] = 0.0f;
        if (i < N_EL && row < n_ch && col < n_cols)
            // non-temporal: the input is read once per tile, while the taps and bias,
            // which every tile reads, stay in L2
            v[k] = __builtin_nontemporal_load(((const float *) (xs + (int64_t) (r0 + row) * a.x_nb1)) + t0 + col);
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = (int) threadIdx.x + SSM_WAVES * WAVE * k;
        if (i < N_EL) tile[i] = v[k];
    }
    // the lane's channel taps and bias
    const int r = r0 + lane;
    float w[NC];
    float b = 0.0f;
    if (lane < n_ch) {
        const uint8_t *wr = (const uint8_t *) a.w + (int64_t) r * a.w_nb1;
#pragma unroll
        for (int j = 0; j < NC; ++j)
            w[j] = F16W ? __half2float(((const __half *) wr)[j]) : ((const float *) wr)[j];
        if (a.bias) b = a.bias[r];
    } else {
#pragma unroll
        for (int j = 0; j < NC; ++j) w[j] = 0.0f;
    }
    __syncthreads();
    if (lane >= n_ch) return;
    // the wave's window: x columns tb .. tb + SSM_TW + NC - 2 of this channel
    const int tb = wave * SSM_TW;
    float xv[SSM_TW + NC - 1];
#pragma unroll
    for (int i = 0; i < SSM_TW + NC - 1; ++i) xv[i] = tile[lane * P + tb + i];
    float *ds = (float *) ((uint8_t *) a.dst + (int64_t) s * a.dst_nb2);
#pragma unroll
    for (int i = 0; i < SSM_TW; ++i) {
        const int t = t0 + tb + i;
        if (t >= a.n_t) break;
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < NC; ++j) acc = fmaf(xv[i + j], w[j], acc);
        if (SILU) {
            acc += b;
            acc = acc / (1.0f + expf(-acc));
        }
        ((float *) ((uint8_t *) ds + (int64_t) t * a.dst_nb1))[r] = acc;
    }
}

template <int NC>
static hipError_t launch_ssm_nc(const SsmConvArgs &a, hipStream_t st) {
    // channel tiles vary fastest: consecutive workgroups go to different XCDs, and
    // the token tiles of one channel block (which share the 128-byte lines at their
    // seams) land nr / 64 workgroups apart, on the same XCD when that is a multiple of 8
    const dim3 grid((unsigned) ((a.nr + SSM_CH - 1) / SSM_CH), (unsigned) ((a.n_t + SSM_TT - 1) / SSM_TT),
                    (unsigned) a.n_s);
    const dim3 block(SSM_WAVES * WAVE);
    if (a.w_f16) {
        if (a.silu) hipLaunchKernelGGL((mc_ssm_conv_kernel<NC, true, true>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((mc_ssm_conv_kernel<NC, true, false>), grid, block, 0, st, a);
    } else {
        if (a.silu) hipLaunchKernelGGL((mc_ssm_conv_kernel<NC, false, true>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((mc_ssm_conv_kernel<NC, false, false>), grid, block, 0, st, a);
    }
    return hipGetLastError();
}

// The reference's kernel sizes (kernels/ssm-conv.cu:138-145); others are refused.
int launch_ssm_conv(const SsmConvArgs &a, void *stream) {
    hipStream_t st = (hipStream_t) stream;
    if (a.n_t <= 0 || a.n_s <= 0 || a.nr <= 0) return (int) hipSuccess;
    switch (a.nc) {
        case 3: return (int) launch_ssm_nc<3>(a, st);
        case 4: return (int) launch_ssm_nc<4>(a, st);
        case 5: return (int) launch_ssm_nc<5>(a, st);
        case 9: return (int) launch_ssm_nc<9>(a, st);
        case 15: return (int) launch_ssm_nc<15>(a, st);
        default: return (int) hipErrorInvalidValue;
    }
}

}  // namespace mc
