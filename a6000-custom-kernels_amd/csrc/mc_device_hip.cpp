// mc_device_hip.cpp -- HIP runtime implementation of the device layer.
#include <hip/hip_runtime.h>

#include "mc_device.h"

namespace mc {

int launch_gemv(GemvArgs a, int tw, int ts, int act, void *stream);   // mc_kernels.hip
int launch_quantize(int kind, const QuantArgs &q, void *stream);      // mc_kernels.hip
int launch_combine(const CombineArgs &c, void *stream);               // mc_kernels.hip
int launch_mmq(const MmqArgs &m, int type, void *stream);            // mc_mmq.hip
int launch_ssm_conv(const SsmConvArgs &a, void *stream);              // mc_ssm_conv.hip
int status_address(uint32_t **p);                                     // mc_ffn.hip
int scratch_address(void **p, size_t *bytes);                         // mc_noalloc.hip

namespace {

struct HipDevice final : Device {
    const char *name() const override { return "hip"; }
    int malloc_dev(void **p, size_t n) override { return (int) hipMalloc(p, n); }
    int free_dev(void *p) override { return (int) hipFree(p); }
    int malloc_host(void **p, size_t n) override { return (int) hipHostMalloc(p, n, hipHostMallocDefault); }
    int free_host(void *p) override { return (int) hipHostFree(p); }
    int copy_h2d(void *dst, const void *src, size_t n, void *s) override {
        return (int) hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, (hipStream_t) s);
    }
    int copy_d2h(void *dst, const void *src, size_t n, void *s) override {
        return (int) hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, (hipStream_t) s);
    }
    int memset_dev(void *dst, int v, size_t n, void *s) override {
        return (int) hipMemsetAsync(dst, v, n, (hipStream_t) s);
    }
    int sync(void *s) override { return (int) hipStreamSynchronize((hipStream_t) s); }
    int stream_create(void **s) override {
        return (int) hipStreamCreateWithFlags((hipStream_t *) s, hipStreamNonBlocking);   // default priority
    }
    int stream_destroy(void *s) override { return (int) hipStreamDestroy((hipStream_t) s); }
    int event_create(void **e) override { return (int) hipEventCreateWithFlags((hipEvent_t *) e, hipEventDisableTiming); }
    int event_destroy(void *e) override { return (int) hipEventDestroy((hipEvent_t) e); }
    int event_record(void *e, void *s) override { return (int) hipEventRecord((hipEvent_t) e, (hipStream_t) s); }
    int stream_wait_event(void *s, void *e) override { return (int) hipStreamWaitEvent((hipStream_t) s, (hipEvent_t) e, 0); }
    int event_sync(void *e) override { return (int) hipEventSynchronize((hipEvent_t) e); }
    int mem_info(size_t *f, size_t *t) override { return (int) hipMemGetInfo(f, t); }
    int ptr_kind(const void *p) override {
        hipPointerAttribute_t attr;
        const hipError_t err = hipPointerGetAttributes(&attr, p);
        if (err != hipSuccess) {
            (void) hipGetLastError();   // an unregistered pointer is not an error state
            return PTR_UNREGISTERED;
        }
        // only host memory qualifies for the cache (kernels/moe-cache.cu:437 accepts cudaMemoryTypeHost alone)
        if (attr.type == hipMemoryTypeHost) return PTR_HOST;
        if (attr.type == hipMemoryTypeManaged) return PTR_MANAGED;
        if (attr.type == hipMemoryTypeDevice) return PTR_DEVICE;
        return PTR_UNREGISTERED;
    }
    int host_device_ptr(const void *host, void **dev) override {
        return (int) hipHostGetDevicePointer(dev, const_cast<void *>(host), 0);
    }
    int register_host(void *base, size_t n) override {
        const hipError_t err = hipHostRegister(base, n, hipHostRegisterPortable | hipHostRegisterMapped);
        if (err != hipSuccess) (void) hipGetLastError();
        return (int) err;
    }
    int launch_gemv(const GemvArgs &a, int tw, int ts, int act, void *s) override {
        return mc::launch_gemv(a, tw, ts, act, s);
    }
    int launch_quantize(int kind, const QuantArgs &q, void *s) override { return mc::launch_quantize(kind, q, s); }
    int launch_combine(const CombineArgs &c, void *s) override { return mc::launch_combine(c, s); }
    int launch_mmq(const MmqArgs &m, int type, void *s) override { return mc::launch_mmq(m, type, s); }
    int launch_ssm_conv(const SsmConvArgs &a, void *s) override { return mc::launch_ssm_conv(a, s); }
    int status_address(uint32_t **p) override { return mc::status_address(p); }
    int scratch_address(void **p, size_t *bytes) override { return mc::scratch_address(p, bytes); }
    const char *error_string(int code) override { return hipGetErrorString((hipError_t) code); }
};

}  // namespace

Device *default_device() {
    static HipDevice dev;
    return &dev;
}

}  // namespace mc
