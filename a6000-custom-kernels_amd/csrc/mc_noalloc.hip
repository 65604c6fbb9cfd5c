// mc_noalloc.hip -- the device scratch of ggml_hip_moe_mul_mat_id_noalloc.
//
// That entry point runs the op-level MUL_MAT_ID (activation quantization, then the
// decode GEMV or the expert-grouped int8-MFMA GEMM) for callers that cannot
// allocate (code under graph capture, tight serving loops), with this array as its
// workspace: the quantized activation rows and the grouped GEMM's pair lists and
// activation records.  Each GPU holds its own copy for the life of the process.
// Host code never passes the array's name to a kernel (in host code that name is a
// host-side stand-in, not a device address): it uses the address that
// hipGetSymbolAddress returns with that GPU current (scratch_address).
#include <hip/hip_runtime.h>

#include <mutex>

#include "mc_internal.h"

namespace mc {

static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_SCRATCH_DEVICES = 64;
}

// Device address of the current GPU's scratch (looked up once per GPU, with that GPU current).
int scratch_address(void **out, size_t *bytes) {
    static std::mutex m;
    static void *addr[MAX_SCRATCH_DEVICES] = {};
    int d = 0;
    hipError_t err = hipGetDevice(&d);
    if (err != hipSuccess) return (int) err;
    if (d < 0 || d >= MAX_SCRATCH_DEVICES) return (int) hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(m);
    if (!addr[d]) {
        void *p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return (int) err;
        addr[d] = p;
    }
    *out = addr[d];
    *bytes = (size_t) NOALLOC_SCRATCH_BYTES;
    return (int) hipSuccess;
}

}  // namespace mc
