// sim_device.cpp -- TEST ONLY.  A host-memory stand-in for the device layer
// (a6000-custom-kernels_amd/csrc/mc_device.h) so that the registry, seeding,
// budget and LRU step code of mc_host.cpp runs unchanged on a CPU-only machine.
//
// "Device" and "pinned host" allocations are plain malloc'ed blocks tracked by
// kind; copies are immediate memcpy.  launch_gemv performs only the pick
// recorder's bookkeeping (stamps, hit counter, canonical miss log) exactly as
// the GPU recorder does; it computes no GEMV output.  Quantize launches fail.
#include <stdlib.h>
#include <string.h>

#include <map>
#include <mutex>

#include "mc_device.h"

namespace mc {
namespace {

struct Region {
    size_t n;
    int kind;
};

struct SimDevice final : Device {
    std::mutex m;
    std::map<uintptr_t, Region> regions;   // base -> (size, kind)
    size_t free_b = 64ull << 30, total_b = 64ull << 30;
    long long n_gemv = 0, n_h2d = 0, n_d2h = 0, n_sync = 0, bytes_h2d = 0, n_alloc = 0;
    int fail_alloc_after = -1;            // < 0: never
    int fail_h2d_after = -1;              // < 0: never

    const char *name() const override { return "sim"; }
    int alloc(void **p, size_t n, int kind) {
        std::lock_guard<std::mutex> l(m);
        if (fail_alloc_after == 0) return 2;   // hipErrorOutOfMemory
        if (fail_alloc_after > 0) --fail_alloc_after;
        n_alloc++;
        void *q = malloc(n ? n : 1);
        if (!q) return 2;
        memset(q, 0xCD, n);
        regions[(uintptr_t) q] = Region{n, kind};
        *p = q;
        return 0;
    }
    int release(void *p) {
        std::lock_guard<std::mutex> l(m);
        auto it = regions.find((uintptr_t) p);
        if (it == regions.end()) return 1;
        regions.erase(it);
        free(p);
        return 0;
    }
    int malloc_dev(void **p, size_t n) override { return alloc(p, n, PTR_DEVICE); }
    int free_dev(void *p) override { return release(p); }
    int malloc_host(void **p, size_t n) override { return alloc(p, n, PTR_HOST); }
    int free_host(void *p) override { return release(p); }
    int copy_h2d(void *d, const void *s, size_t n, void *) override {
        if (fail_h2d_after == 0) return 1;     // hipErrorInvalidValue
        if (fail_h2d_after > 0) --fail_h2d_after;
        memcpy(d, s, n);
        n_h2d++;
        bytes_h2d += (long long) n;
        return 0;
    }
    int copy_d2h(void *d, const void *s, size_t n, void *) override {
        memcpy(d, s, n);
        n_d2h++;
        return 0;
    }
    int memset_dev(void *d, int v, size_t n, void *) override {
        memset(d, v, n);
        return 0;
    }
    int sync(void *) override {
        n_sync++;
        return 0;
    }
    // every simulated copy completes when issued: streams and events only keep count
    long long live_streams = 0, live_events = 0, n_event_sync = 0;
    int stream_create(void **s) override {
        std::lock_guard<std::mutex> l(m);
        *s = new char(0);
        live_streams++;
        return 0;
    }
    int stream_destroy(void *s) override {
        std::lock_guard<std::mutex> l(m);
        delete (char *) s;
        live_streams--;
        return 0;
    }
    int event_create(void **e) override {
        std::lock_guard<std::mutex> l(m);
        *e = new char(0);
        live_events++;
        return 0;
    }
    int event_destroy(void *e) override {
        std::lock_guard<std::mutex> l(m);
        delete (char *) e;
        live_events--;
        return 0;
    }
    int event_record(void *, void *) override { return 0; }
    int stream_wait_event(void *, void *) override { return 0; }
    int event_sync(void *) override {
        n_event_sync++;
        return 0;
    }
    int mem_info(size_t *f, size_t *t) override {
        *f = free_b;
        *t = total_b;
        return 0;
    }
    int ptr_kind(const void *p) override {
        std::lock_guard<std::mutex> l(m);
        const uintptr_t a = (uintptr_t) p;
        auto it = regions.upper_bound(a);
        if (it == regions.begin()) return PTR_UNREGISTERED;
        --it;
        if (a >= it->first && a < it->first + it->second.n) return it->second.kind;
        return PTR_UNREGISTERED;
    }
    int host_device_ptr(const void *h, void **d) override {
        *d = const_cast<void *>(h);
        return 0;
    }
    int register_host(void *base, size_t n) override {
        std::lock_guard<std::mutex> l(m);
        regions[(uintptr_t) base] = Region{n, PTR_HOST | 0x100};
        return 0;
    }
    // recorder semantics of mc_kernels.hip:record_picks, sequentially
    int launch_gemv(const GemvArgs &a, int, int, int, void *) override {
        n_gemv++;
        const uint32_t clk = a.clock ? *a.clock : 0u;
        for (int p = 0; p < a.n_tok * a.n_used; ++p) {
            const int t = p / a.n_used, c = p % a.n_used;
            const int e = a.ids[c + (int64_t) t * a.ids_stride];
            if (e < 0 || e >= a.n_experts) continue;
            const uint64_t pu = a.tbl[e];
            if (a.stamps) a.stamps[e] = clk;
            const uint32_t mu = (uint32_t) (pu & 1u);
            uint32_t mg = 0, hits = 1u - mu;
            if (a.tbl_gate && a.cache_id_gate >= 0) {     // a gate without a cache entry is not recorded
                const uint64_t pg = a.tbl_gate[e];
                if (a.stamps_gate) a.stamps_gate[e] = clk;
                mg = (uint32_t) (pg & 1u);
                hits += 1u - mg;
            }
            if (!a.stats) continue;
            const uint32_t pos = a.stats[0];
            a.stats[0] += mu + mg;
            a.stats[HIT_WORD] += hits;
            if (mu && pos < (uint32_t) MISS_CAP) a.stats[LOG_BASE + pos] = ((uint32_t) a.cache_id << 12) | (uint32_t) e;
            if (mg && pos + mu < (uint32_t) MISS_CAP)
                a.stats[LOG_BASE + pos + mu] = ((uint32_t) a.cache_id_gate << 12) | (uint32_t) e;
        }
        return 0;
    }
    int launch_quantize(int, const QuantArgs &, void *) override { return 98; }
    int launch_combine(const CombineArgs &, void *) override { return 98; }
    int launch_mmq(const MmqArgs &, int, void *) override { return 98; }
    int launch_ssm_conv(const SsmConvArgs &, void *) override { return 98; }
    // stand-in for the no-alloc scratch: a fixed host block (kernels never run here)
    size_t scratch_bytes = 1u << 20;
    alignas(256) static inline unsigned char scratch_block[1u << 20];
    int scratch_address(void **p, size_t *bytes) override {
        *p = scratch_block;
        *bytes = scratch_bytes;
        return 0;
    }
    uint32_t status = 0;                  // no kernel runs here: stays 0 unless a test sets it
    int status_address(uint32_t **p) override {
        *p = &status;
        return 0;
    }
    const char *error_string(int code) override {
        return code == 2 ? "out of memory (sim)" : code == 98 ? "not simulated" : "sim error";
    }
};

SimDevice g_sim;

}  // namespace

Device *default_device() { return &g_sim; }

}  // namespace mc

// test hooks
extern "C" {

void mc_sim_set_mem_info(uint64_t free_b, uint64_t total_b) {
    mc::g_sim.free_b = free_b;
    mc::g_sim.total_b = total_b;
}

void *mc_sim_host_alloc(uint64_t n) {
    void *p = nullptr;
    return mc::g_sim.malloc_host(&p, n) ? nullptr : p;
}

void *mc_sim_plain_alloc(uint64_t n) { return malloc(n); }

void *mc_sim_dev_alloc(uint64_t n) {
    void *p = nullptr;
    return mc::g_sim.malloc_dev(&p, n) ? nullptr : p;
}

int mc_sim_free(void *p) { return mc::g_sim.release(p); }

void mc_sim_fail_alloc_after(int n) { mc::g_sim.fail_alloc_after = n; }

void mc_sim_fail_h2d_after(int n) { mc::g_sim.fail_h2d_after = n; }

void mc_sim_set_status(uint32_t v) { mc::g_sim.status = v; }

// number of device / pinned allocations made so far (the no-alloc entry must not add any)
long long mc_sim_alloc_count(void) { return mc::g_sim.n_alloc; }

// live allocations of the simulated device (device, pinned host and registered regions)
long long mc_sim_live_regions(void) {
    std::lock_guard<std::mutex> l(mc::g_sim.m);
    return (long long) mc::g_sim.regions.size();
}

// live streams and events of the simulated device
void mc_sim_live_streams_events(long long *out2) {
    out2[0] = mc::g_sim.live_streams;
    out2[1] = mc::g_sim.live_events;
}

void mc_sim_counters(long long *out5) {
    out5[0] = mc::g_sim.n_gemv;
    out5[1] = mc::g_sim.n_h2d;
    out5[2] = mc::g_sim.n_d2h;
    out5[3] = mc::g_sim.n_sync;
    out5[4] = mc::g_sim.bytes_h2d;
}

}  // extern "C"
