// Read-floor probe for bench.py --read-floor (measurement only, not part of the library).
//
// floor_read_steps: one wave per GEMV step of the fused gate/up launch, the same step list
// and workgroup shape (waves_per_wg steps per workgroup), each wave streaming its step's gate
// and up spans into LDS with the kernel's buffer->LDS DMA and non-temporal policy, then
// waiting for them; no dots, no prologue, no stores but one dword per workgroup.  It prices
// the bytes of one gate/up launch with nothing else in the way.
// floor_empty: a launch of the same grid that does nothing (the dispatch/drain cost).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __attribute__((address_space(3))) void lds_void_t;

struct FloorStep {
    const uint8_t *gate;    // span starts (16-byte aligned by the host)
    const uint8_t *up;
    uint32_t bytes;         // bytes of each span (<= region / 2 - 16)
    uint32_t pad;
};

__global__ __launch_bounds__(512) void floor_read_steps(const FloorStep *steps, int n_steps, int waves_per_wg,
                                                        uint32_t region, uint32_t *out) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int wave = __builtin_amdgcn_readfirstlane((int) (threadIdx.x / 64)), lane = threadIdx.x % 64;
    const int st = (int) blockIdx.x * waves_per_wg + wave;
    uint32_t v = 0;
    if (st < n_steps) {
        const FloorStep s = steps[st];
        const int rounds = (int) ((s.bytes + 1023u) >> 10);
        uint8_t *dst = lds + (uint32_t) wave * region;
        const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc((void *) s.gate, (short) 0, (int) s.bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t ru = __builtin_amdgcn_make_buffer_rsrc((void *) s.up, (short) 0, (int) s.bytes, 0x00020000);
        for (int i = 0; i < rounds; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rg, (lds_void_t *) (dst + 1024 * i), 16, 16u * lane + 1024u * i, 0, 0, 2);
        for (int i = 0; i < rounds; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ru, (lds_void_t *) (dst + region / 2 + 1024 * i), 16,
                                                     16u * lane + 1024u * i, 0, 0, 2);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        v = ((const uint32_t *) dst)[lane];
    }
    if (lane == 0 && wave == 0) out[blockIdx.x] = v;
}

__global__ void floor_empty() {}

// Returns a hipError_t value; -1 for a step list or region the kernel cannot hold.
extern "C" int floor_launch(const void *steps, int n_steps, int waves_per_wg, unsigned region, unsigned max_bytes,
                            uint32_t *out, void *stream) {
    if (n_steps <= 0 || waves_per_wg < 1 || waves_per_wg > 8 || region % 16 || max_bytes + 1024 > region / 2)
        return -1;
    const unsigned lds = (unsigned) waves_per_wg * region;
    if (lds > 160u * 1024u) return -1;
    static bool attr = false;
    if (!attr) {
        static_cast<void>(hipFuncSetAttribute((const void *) floor_read_steps,
                                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        attr = true;
    }
    const unsigned grid = (unsigned) ((n_steps + waves_per_wg - 1) / waves_per_wg);
    hipLaunchKernelGGL(floor_read_steps, dim3(grid), dim3(64 * waves_per_wg), lds, (hipStream_t) stream,
                       (const FloorStep *) steps, n_steps, waves_per_wg, region, out);
    return (int) hipGetLastError();
}

extern "C" int floor_launch_empty(unsigned grid, unsigned block, void *stream) {
    hipLaunchKernelGGL(floor_empty, dim3(grid), dim3(block), 0, (hipStream_t) stream);
    return (int) hipGetLastError();
}
