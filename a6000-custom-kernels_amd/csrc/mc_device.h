// mc_device.h -- the thin device layer the host registry talks to.
//
// The product library implements it with the HIP runtime and the gfx950
// kernels (mc_device_hip.cpp).  The registry / step code (mc_host.cpp) only
// ever calls through this interface, so the same code can be linked against a
// host-memory simulation for CPU tests of the cache logic (no compute).
#ifndef MC_DEVICE_H
#define MC_DEVICE_H

#include <stddef.h>
#include <stdint.h>

#include "mc_internal.h"

namespace mc {

enum PtrKind : int { PTR_ERROR = -1, PTR_UNREGISTERED = 0, PTR_HOST = 1, PTR_DEVICE = 2, PTR_MANAGED = 3 };

struct Device {
    virtual ~Device() = default;
    virtual const char *name() const = 0;
    virtual int malloc_dev(void **p, size_t n) = 0;
    virtual int free_dev(void *p) = 0;
    virtual int malloc_host(void **p, size_t n) = 0;                       // pinned, device-readable
    virtual int free_host(void *p) = 0;
    virtual int copy_h2d(void *dst, const void *src, size_t n, void *stream) = 0;   // async on stream
    virtual int copy_d2h(void *dst, const void *src, size_t n, void *stream) = 0;   // async on stream
    virtual int memset_dev(void *dst, int v, size_t n, void *stream) = 0;           // async on stream
    virtual int sync(void *stream) = 0;
    // a second stream (default priority) and events ordering it against the caller's stream
    virtual int stream_create(void **stream) = 0;
    virtual int stream_destroy(void *stream) = 0;
    virtual int event_create(void **event) = 0;
    virtual int event_destroy(void *event) = 0;
    virtual int event_record(void *event, void *stream) = 0;
    virtual int stream_wait_event(void *stream, void *event) = 0;
    virtual int event_sync(void *event) = 0;
    virtual int mem_info(size_t *free_b, size_t *total_b) = 0;
    virtual int ptr_kind(const void *p) = 0;                               // PtrKind
    virtual int host_device_ptr(const void *host, void **dev) = 0;         // device-visible address of host memory
    virtual int register_host(void *base, size_t n) = 0;
    virtual int launch_gemv(const GemvArgs &a, int tw, int ts, int act, void *stream) = 0;
    virtual int launch_quantize(int kind, const QuantArgs &q, void *stream) = 0;
    virtual int launch_combine(const CombineArgs &c, void *stream) = 0;
    virtual int launch_mmq(const MmqArgs &m, int type, void *stream) = 0;
    virtual int launch_ssm_conv(const SsmConvArgs &a, void *stream) = 0;
    virtual int status_address(uint32_t **p) = 0;                          // device status word of the current device
    virtual int scratch_address(void **p, size_t *bytes) = 0;              // no-alloc scratch of the current device
    virtual const char *error_string(int code) = 0;
};

// The device this library was linked with.
Device *default_device();

}  // namespace mc

#endif
