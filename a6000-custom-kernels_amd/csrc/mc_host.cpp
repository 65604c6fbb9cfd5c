// mc_host.cpp -- host side of the pointer-table MoE GEMV: configuration,
// per-tensor registration (pointer table, HBM pool, stamps), seed loading,
// the between-graph LRU promotion step and the C ABI.
//
// Restates the host half of kernels/moe-cache.cu (:293-868) for one MI355X:
//   * pools are sized for 288 GB of HBM3E: by default every expert of a tensor
//     gets a slot and the budget is whatever hipMemGetInfo reports free minus a
//     margin (reference: 320 slots, 30 GiB, 2 GiB margin; :317-318, :549-556);
//   * host expert memory is addressed on the device through
//     hipHostGetDevicePointer, not the raw host address;
//   * errors return a status (reference: CUDA_CHECK / GGML_ABORT aborts).
#include <errno.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/ggml_hip_moe_cache.h"
#include "mc_device.h"
#include "mc_internal.h"

namespace mc {
namespace {

thread_local std::string t_last_error;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    t_last_error = buf;
    return code;
}

constexpr int E_INVALID = -1;
constexpr int E_UNSUPPORTED = -2;
constexpr int E_DEVICE = -3;
constexpr int E_DISABLED = -4;
constexpr int E_STATE = -5;
constexpr int E_TIMEOUT = -6;

int32_t g_spin_limit = DEFAULT_SPIN_LIMIT;             // bounded in-kernel waits (debug setter below)

// ---------------------------------------------------------------------------
// configuration (kernels/moe-cache.cu:330-363)
// ---------------------------------------------------------------------------

struct Config {
    bool enabled = false;
    int slots = -1;                       // < 0: every expert of the tensor
    double budget_gb = 0.0;               // <= 0: adaptive (free HBM - margin)
    double margin_gb = 2.0;
    std::string seed_path;
    int max_promotions = DEFAULT_MAX_PROMOTIONS;
    bool verbose = false;
    bool debug = false;
    bool allow_register = false;
    bool async_promotions = false;        // promotion copies on a second stream (see step_locked)
};

Config g_cfg;
bool g_cfg_ready = false;

const char *env2(const char *hip_name, const char *cuda_name) {
    const char *v = getenv(hip_name);
    if (!v && cuda_name) v = getenv(cuda_name);
    return v;
}

void read_env_locked() {
    if (g_cfg_ready) return;
    Config c;
    const char *en = env2("GGML_HIP_MOE_CACHE", "GGML_CUDA_MOE_CACHE");
    c.enabled = en && en[0] && en[0] != '0';
    if (const char *s = env2("GGML_HIP_MOE_CACHE_SLOTS", "GGML_CUDA_MOE_CACHE_SLOTS")) c.slots = std::max(0, atoi(s));
    if (const char *s = env2("GGML_HIP_MOE_CACHE_BUDGET_GB", "GGML_CUDA_MOE_CACHE_BUDGET_GB")) {
        const double gb = atof(s);
        if (gb > 0) c.budget_gb = gb;
    }
    if (const char *s = getenv("GGML_HIP_MOE_CACHE_MARGIN_GB")) c.margin_gb = std::max(0.0, atof(s));
    if (const char *s = env2("GGML_HIP_MOE_CACHE_SEED", "GGML_CUDA_MOE_CACHE_SEED")) c.seed_path = s;
    if (const char *s = getenv("GGML_HIP_MOE_CACHE_MAX_PROMOTIONS")) c.max_promotions = std::max(0, atoi(s));
    c.debug = env2("GGML_HIP_MOE_CACHE_DEBUG", "GGML_CUDA_MOE_CACHE_DEBUG") != nullptr;
    c.verbose = c.debug || getenv("GGML_HIP_MOE_CACHE_VERBOSE") != nullptr;
    const char *ar = getenv("GGML_HIP_MOE_CACHE_ALLOW_REGISTER");
    c.allow_register = ar && ar[0] == '1';
    const char *as = getenv("GGML_HIP_MOE_CACHE_ASYNC");
    c.async_promotions = as && as[0] == '1';
    g_cfg = c;
    g_cfg_ready = true;
    if (g_cfg.enabled && g_cfg.verbose) {
        fprintf(stderr, "moe-cache: enabled, slots=%d budget=%s margin=%.1f GB\n", g_cfg.slots,
                g_cfg.budget_gb > 0 ? "fixed" : "adaptive", g_cfg.margin_gb);
    }
}

// ---------------------------------------------------------------------------
// registry state (kernels/moe-cache.cu:297-328)
// ---------------------------------------------------------------------------

struct Entry {
    int32_t id = -1;
    int type = 0;
    const char *data = nullptr;          // host base of the expert tensor (copy source)
    uintptr_t dev_base = 0;              // device-visible address of `data`
    size_t expert_bytes = 0;
    int n_experts = 0;
    int n_slots = 0;
    char *pool = nullptr;                // device, n_slots * expert_bytes
    uint64_t *d_tbl = nullptr;           // device, tagged pointers
    std::vector<uint64_t> h_tbl;         // host mirror
    uint32_t *d_stamps = nullptr;        // device, last-use clock per expert (a slice of the stamps arena,
                                         // or its own allocation when the arena is full)
    bool stamps_in_arena = false;
    size_t stamps_off = 0;               // word offset of the slice in the arena
    std::vector<int32_t> slot_of;        // expert -> slot (-1: cold)
    std::vector<int32_t> expert_of;      // slot -> expert (-1: free)
    std::vector<uint32_t> h_stamps;      // host mirror of d_stamps for eviction
    uint32_t stamps_clock = 0;           // clock at the last mirror refresh
    bool tbl_dirty = false;
    uint64_t *h_tbl_stage[2] = {nullptr, nullptr};   // pinned table snapshots (asynchronous promotions)
    std::string name;
};

// Table of a device-resident expert tensor (no pool, no stats).
struct Resident {
    uint64_t *d_tbl = nullptr;
    std::vector<uint64_t> h_tbl;
    int n_experts = 0;
    int cap = 0;                         // entries d_tbl can hold
    size_t expert_bytes = 0;
};

std::mutex g_mutex;                                  // registry + step
std::unordered_map<const char *, Entry *> g_by_data;
std::vector<Entry *> g_all;
std::unordered_map<const void *, Resident *> g_resident;
uint32_t *g_d_stats = nullptr;                       // device [STATS_WORDS]
uint32_t *g_h_stats = nullptr;                       // pinned host mirror (+1 word: clock staging)
uint32_t *g_d_clock = nullptr;
uint32_t g_h_clock = 0;
// every tensor's eviction stamps in one device array (and its pinned mirror), so a step reads
// the stamps it needs with one copy
constexpr size_t STAMPS_ARENA_WORDS = size_t(1) << 20;
uint32_t *g_d_stamps_arena = nullptr;
uint32_t *g_h_stamps_arena = nullptr;
size_t g_stamps_used = 0;                            // words handed out
size_t g_used = 0;                                   // pool bytes allocated
std::unordered_map<uint32_t, int> g_admission;       // (id << 12 | expert) -> sightings
std::unordered_map<std::string, std::vector<int>> g_seed;
bool g_seed_loaded = false;
ggml_hip_moe_totals g_totals = {};

// asynchronous promotions: the copy stream, the event ordering it after the compute stream's
// demotions, and the event of its last table flush (waited for before the next step)
void *g_copy_stream = nullptr;
void *g_order_event = nullptr;
void *g_copy_event = nullptr;
bool g_copy_pending = false;

std::unordered_map<const void *, int> g_ptr_kind;    // cached residency test
std::mutex g_ptr_mutex;

Device *dev() { return default_device(); }

int dev_err(int code, const char *what) {
    return fail(E_DEVICE, "moe-cache: %s failed on %s: %s (%d)", what, dev()->name(), dev()->error_string(code), code);
}

int ptr_kind_cached(const void *p) {
    std::lock_guard<std::mutex> lock(g_ptr_mutex);
    auto it = g_ptr_kind.find(p);
    if (it != g_ptr_kind.end()) return it->second;
    const int k = dev()->ptr_kind(p);
    g_ptr_kind[p] = k;
    return k;
}

bool is_contiguous(const ggml_hip_moe_tensor *t) {
    const TypeGeom g = type_geom(t->type);
    if (g.block_elems == 0 || t->ne[0] % g.block_elems) return false;
    const uint64_t rb = (uint64_t) (t->ne[0] / g.block_elems) * g.block_bytes;
    return t->nb[0] == (uint64_t) g.block_bytes && t->nb[1] == rb && t->nb[2] == rb * (uint64_t) t->ne[1] &&
           t->nb[3] == t->nb[2] * (uint64_t) t->ne[2];
}

int init_globals_locked(void *stream) {
    if (g_d_stats) return 0;
    int rc;
    if ((rc = dev()->malloc_dev((void **) &g_d_stats, sizeof(uint32_t) * STATS_WORDS))) return dev_err(rc, "stats alloc");
    if ((rc = dev()->malloc_host((void **) &g_h_stats, sizeof(uint32_t) * (STATS_WORDS + 2)))) return dev_err(rc, "pinned stats alloc");
    if ((rc = dev()->malloc_dev((void **) &g_d_clock, sizeof(uint32_t)))) return dev_err(rc, "clock alloc");
    if ((rc = dev()->malloc_dev((void **) &g_d_stamps_arena, sizeof(uint32_t) * STAMPS_ARENA_WORDS))) return dev_err(rc, "stamps arena alloc");
    if ((rc = dev()->malloc_host((void **) &g_h_stamps_arena, sizeof(uint32_t) * STAMPS_ARENA_WORDS)))
        return dev_err(rc, "pinned stamps arena alloc");
    g_stamps_used = 0;
    memset(g_h_stats, 0, sizeof(uint32_t) * (STATS_WORDS + 2));
    if ((rc = dev()->memset_dev(g_d_stats, 0, sizeof(uint32_t) * STATS_WORDS, stream))) return dev_err(rc, "stats clear");
    if ((rc = dev()->memset_dev(g_d_clock, 0, sizeof(uint32_t), stream))) return dev_err(rc, "clock clear");
    g_h_clock = 0;
    return 0;
}

// seed file: lines "tensorname id1,id2,..." (kernels/moe-cache.cu:483-523)
void load_seed_locked() {
    if (g_seed_loaded) return;
    g_seed_loaded = true;
    const std::string &path = g_cfg.seed_path;
    if (path.empty()) return;
    FILE *f = fopen(path.c_str(), "r");
    if (!f) {
        if (g_cfg.verbose) fprintf(stderr, "moe-cache: seed file %s not found, starting cold\n", path.c_str());
        return;
    }
    static char line[1 << 16];
    while (fgets(line, sizeof(line), f)) {
        char *sp = strchr(line, ' ');
        if (!sp) continue;
        *sp = 0;
        std::vector<int> ids;
        char *p = sp + 1;
        while (*p) {
            char *end = nullptr;
            const long v = strtol(p, &end, 10);
            if (end == p) break;
            ids.push_back((int) v);
            p = (*end == ',') ? end + 1 : end;
        }
        g_seed[line] = std::move(ids);
    }
    fclose(f);
    if (g_cfg.verbose) fprintf(stderr, "moe-cache: loaded seed for %zu tensors from %s\n", g_seed.size(), path.c_str());
}

uint64_t host_entry(const Entry *e, int expert) {
    return (uint64_t) (e->dev_base + (uintptr_t) expert * e->expert_bytes) | 1ull;
}
uint64_t pool_entry(const Entry *e, int slot) { return (uint64_t) (uintptr_t) (e->pool + (size_t) slot * e->expert_bytes); }

// registration (kernels/moe-cache.cu:525-622)
int get_or_create_locked(const ggml_hip_moe_tensor *src0, void *stream, Entry **out) {
    int rc = init_globals_locked(stream);
    if (rc) return rc;
    auto it = g_by_data.find((const char *) src0->data);
    if (it != g_by_data.end()) {
        *out = it->second;
        return 0;
    }
    void *dbase = nullptr;
    if ((rc = dev()->host_device_ptr(src0->data, &dbase))) return dev_err(rc, "hipHostGetDevicePointer");

    Entry *e = new Entry();
    e->id = (int32_t) g_all.size();
    e->type = src0->type;
    e->data = (const char *) src0->data;
    e->dev_base = (uintptr_t) dbase;
    e->expert_bytes = (size_t) src0->nb[2];
    e->n_experts = (int) src0->ne[2];
    e->name = src0->name ? src0->name : "";

    const size_t eb = e->expert_bytes;
    long long slots = g_cfg.slots < 0 ? (long long) e->n_experts : (long long) g_cfg.slots;
    if (g_cfg.budget_gb > 0) {
        const size_t budget = (size_t) (g_cfg.budget_gb * 1024.0 * 1024.0 * 1024.0);
        const size_t free_budget = budget > g_used ? budget - g_used : 0;
        if ((size_t) slots * eb > free_budget) slots = (long long) (free_budget / eb);
    }
    size_t free_b = 0, total_b = 0;
    if ((rc = dev()->mem_info(&free_b, &total_b))) {
        delete e;
        return dev_err(rc, "hipMemGetInfo");
    }
    const size_t margin = (size_t) (g_cfg.margin_gb * 1024.0 * 1024.0 * 1024.0);
    const size_t usable = free_b > margin ? free_b - margin : 0;
    if ((size_t) slots * eb > usable) slots = (long long) (usable / eb);
    if (slots > e->n_experts) slots = e->n_experts;
    e->n_slots = (int) slots;

    // Any failure below frees what this registration allocated and registers nothing, so
    // a later call never finds an entry whose device table was not written.
    auto abandon = [&](int code, const char *what) {
        if (e->pool) dev()->free_dev(e->pool);
        if (e->d_stamps && !e->stamps_in_arena) dev()->free_dev(e->d_stamps);
        if (e->d_tbl) dev()->free_dev(e->d_tbl);
        delete e;
        return dev_err(code, what);
    };
    e->h_tbl.resize(e->n_experts);
    for (int i = 0; i < e->n_experts; ++i) e->h_tbl[i] = host_entry(e, i);
    if ((rc = dev()->malloc_dev((void **) &e->d_tbl, sizeof(uint64_t) * e->n_experts))) return abandon(rc, "table alloc");
    const size_t sw = ((size_t) e->n_experts + 63) & ~(size_t) 63;      // 256-byte slices
    if (g_d_stamps_arena && g_stamps_used + sw <= STAMPS_ARENA_WORDS) {
        e->d_stamps = g_d_stamps_arena + g_stamps_used;
        e->stamps_in_arena = true;
        e->stamps_off = g_stamps_used;
        g_stamps_used += sw;                       // (an abandoned registration leaves its slice unused)
    } else if ((rc = dev()->malloc_dev((void **) &e->d_stamps, sizeof(uint32_t) * e->n_experts))) {
        return abandon(rc, "stamps alloc");
    }
    if ((rc = dev()->memset_dev(e->d_stamps, 0, sizeof(uint32_t) * e->n_experts, stream))) return abandon(rc, "stamps clear");
    e->h_stamps.assign(e->n_experts, 0);
    e->slot_of.assign(e->n_experts, -1);
    e->expert_of.assign(e->n_slots, -1);
    if (e->n_slots > 0 && (rc = dev()->malloc_dev((void **) &e->pool, (size_t) e->n_slots * eb))) return abandon(rc, "pool alloc");

    // seed slots 0..k-1 in seed order, skipping out-of-range and repeated ids
    load_seed_locked();
    auto sit = g_seed.find(e->name);
    int seeded = 0;
    if (sit != g_seed.end() && e->n_slots > 0) {
        for (const int expert : sit->second) {
            if (seeded >= e->n_slots) break;
            if (expert < 0 || expert >= e->n_experts || e->slot_of[expert] >= 0) continue;
            const int slot = seeded;
            if ((rc = dev()->copy_h2d(e->pool + (size_t) slot * eb, e->data + (size_t) expert * eb, eb, stream)))
                return abandon(rc, "seed copy");
            e->h_tbl[expert] = pool_entry(e, slot);
            e->slot_of[expert] = slot;
            e->expert_of[slot] = expert;
            seeded += 1;
        }
    }
    // one upload covers the host entries and every seeded slot, ordered after the copies
    if ((rc = dev()->copy_h2d(e->d_tbl, e->h_tbl.data(), sizeof(uint64_t) * e->n_experts, stream)))
        return abandon(rc, "table upload");
    if (e->n_slots > 0) g_used += (size_t) e->n_slots * eb;
    g_by_data[e->data] = e;
    g_all.push_back(e);
    if (g_cfg.verbose) {
        fprintf(stderr, "moe-cache: registered %s type=%d experts=%d slot_bytes=%zu slots=%d seeded=%d (pool %.1f MB, total %.2f GB, free HBM %.2f GB)\n",
                e->name.empty() ? "<tensor>" : e->name.c_str(), e->type, e->n_experts, eb, e->n_slots, seeded,
                (double) e->n_slots * eb / (1024.0 * 1024.0), (double) g_used / (1024.0 * 1024.0 * 1024.0),
                (double) free_b / (1024.0 * 1024.0 * 1024.0));
    }
    *out = e;
    return 0;
}

// LRU slot acquisition (kernels/moe-cache.cu:628-667)
int acquire_slot_locked(Entry *e, void *stream, int *slot_out) {
    *slot_out = -1;
    if (e->n_slots == 0) return 0;
    for (int s = 0; s < e->n_slots; ++s) {
        if (e->expert_of[s] < 0) {
            *slot_out = s;
            return 0;
        }
    }
    if (e->stamps_clock != g_h_clock) {
        int rc;
        if ((rc = dev()->copy_d2h(e->h_stamps.data(), e->d_stamps, sizeof(uint32_t) * e->n_experts, stream))) return dev_err(rc, "stamps readback");
        if ((rc = dev()->sync(stream))) return dev_err(rc, "stream sync");
        e->stamps_clock = g_h_clock;
    }
    int victim_slot = -1;
    uint32_t best = UINT32_MAX;
    for (int s = 0; s < e->n_slots; ++s) {
        const int expert = e->expert_of[s];
        const uint32_t stamp = expert >= 0 ? e->h_stamps[expert] : 0;
        if (stamp < best) {
            best = stamp;
            victim_slot = s;
        }
    }
    if (victim_slot < 0) return 0;
    const int victim = e->expert_of[victim_slot];
    if (victim >= 0) {
        e->slot_of[victim] = -1;
        e->h_tbl[victim] = host_entry(e, victim);
        e->tbl_dirty = true;
        g_totals.evictions += 1;
    }
    e->expert_of[victim_slot] = -1;
    *slot_out = victim_slot;
    return 0;
}

// between-graph promotion step (kernels/moe-cache.cu:669-775)
// Waits for the previous step's asynchronous promotions (copy stream) to finish.
int wait_copies_locked() {
    if (!g_copy_pending) return 0;
    int rc;
    if ((rc = dev()->event_sync(g_copy_event))) return dev_err(rc, "promotion copies");
    g_copy_pending = false;
    return 0;
}

// Uploads entry e's host table through its pinned snapshot `which` on `stream` (the
// snapshot keeps the bytes of this upload while the host table changes).
int upload_table_staged_locked(Entry *e, int which, void *stream) {
    int rc;
    if (!e->h_tbl_stage[which]) {
        void *p = nullptr;
        if ((rc = dev()->malloc_host(&p, sizeof(uint64_t) * e->n_experts))) return dev_err(rc, "table staging");
        e->h_tbl_stage[which] = (uint64_t *) p;
    }
    memcpy(e->h_tbl_stage[which], e->h_tbl.data(), sizeof(uint64_t) * e->n_experts);
    if ((rc = dev()->copy_h2d(e->d_tbl, e->h_tbl_stage[which], sizeof(uint64_t) * e->n_experts, stream)))
        return dev_err(rc, "table flush");
    return 0;
}

// The step between tokens (kernels/moe-cache.cu:742-775): stats readback, clock, admission on
// the second sighting, LRU promotion, one table upload per touched tensor.
//
// The eviction stamps of every tensor the miss log could make evict are read back in one
// batch with one wait, so the loop below never waits on the stream (its lazy readback in
// acquire_slot_locked finds them fresh); the decisions are those of reading them lazily.
//
// With async_promotions the promotion copies leave the caller's stream: the demotions
// (victims back to their host entries) are uploaded on it first, so the next token's
// kernels never read a slot that is being overwritten; the copies and then the promoted
// entries' table upload go on a second stream ordered after that upload.  A kernel running
// meanwhile reads each table entry either before or after its 8-byte update, and both point
// at the expert's bytes, so results are unchanged; which reads hit the pool (the hit / miss
// counts and stamps) then depends on timing.
int step_locked(void *stream) {
    int rc;
    if ((rc = wait_copies_locked())) return rc;
    if ((rc = dev()->copy_d2h(g_h_stats, g_d_stats, sizeof(uint32_t) * STATS_WORDS, stream))) return dev_err(rc, "stats readback");
    if ((rc = dev()->sync(stream))) return dev_err(rc, "stream sync");
    uint32_t n = g_h_stats[0];
    if (n > (uint32_t) MISS_CAP) n = MISS_CAP;
    const uint32_t step_hits = g_h_stats[HIT_WORD];

    g_h_clock += 1;
    g_h_stats[STATS_WORDS] = g_h_clock;          // pinned staging word for the clock upload
    if ((rc = dev()->copy_h2d(g_d_clock, &g_h_stats[STATS_WORDS], sizeof(uint32_t), stream))) return dev_err(rc, "clock upload");
    if ((rc = dev()->memset_dev(g_d_stats, 0, 2 * sizeof(uint32_t), stream))) return dev_err(rc, "stats reset");

    g_totals.steps += 1;
    g_totals.misses += n;
    g_totals.hits += step_hits;
    g_totals.clock = g_h_clock;
    g_totals.last_step_misses = n;
    g_totals.last_step_hits = step_hits;
    if (g_cfg.verbose && g_totals.steps % 64 == 0) {
        size_t resident = 0;
        for (const Entry *e : g_all)
            for (int s = 0; s < e->n_slots; ++s) resident += e->expert_of[s] >= 0 ? 1 : 0;
        fprintf(stderr, "moe-cache: step %llu: hits=%u misses=%u (totals: hits %llu, misses %llu, promos %llu), resident %zu\n",
                (unsigned long long) g_totals.steps, step_hits, n, (unsigned long long) g_totals.hits,
                (unsigned long long) g_totals.misses, (unsigned long long) g_totals.promotions, resident);
    }
    if (n == 0) return 0;

    // stamps of the tensors that may evict: more possible promotions (second sightings, counted on
    // a copy of the admission counts) than free slots; the arena's used prefix comes back in one copy
    {
        std::unordered_map<uint32_t, int> counts;
        std::unordered_map<Entry *, uint32_t> possible;
        for (uint32_t i = 0; i < n; ++i) {
            const uint32_t packed = g_h_stats[LOG_BASE + i];
            const int32_t cid = (int32_t) (packed >> 12);
            auto it = counts.find(packed);
            if (it == counts.end()) {
                auto ga = g_admission.find(packed);
                it = counts.emplace(packed, ga == g_admission.end() ? 0 : ga->second).first;
            }
            if (++it->second < 2) continue;
            it->second = 0;
            if (cid >= 0 && cid < (int32_t) g_all.size()) possible[g_all[cid]] += 1;
        }
        std::vector<Entry *> need;
        bool arena = false;
        for (auto &kv : possible) {
            Entry *e = kv.first;
            if (e->n_slots == 0 || e->stamps_clock == g_h_clock) continue;
            uint32_t free_slots = 0;
            for (int sl = 0; sl < e->n_slots; ++sl) free_slots += e->expert_of[sl] < 0 ? 1 : 0;
            if (free_slots >= kv.second) continue;
            need.push_back(e);
            if (e->stamps_in_arena) {
                arena = true;
            } else if ((rc = dev()->copy_d2h(e->h_stamps.data(), e->d_stamps, sizeof(uint32_t) * e->n_experts, stream))) {
                return dev_err(rc, "stamps readback");
            }
        }
        if (arena && (rc = dev()->copy_d2h(g_h_stamps_arena, g_d_stamps_arena, sizeof(uint32_t) * g_stamps_used, stream)))
            return dev_err(rc, "stamps readback");
        if (!need.empty() && (rc = dev()->sync(stream))) return dev_err(rc, "stream sync");
        for (Entry *e : need) {
            if (e->stamps_in_arena)
                memcpy(e->h_stamps.data(), g_h_stamps_arena + e->stamps_off, sizeof(uint32_t) * e->n_experts);
            e->stamps_clock = g_h_clock;
        }
    }

    // admission: promote on the 2nd sighting; the count resets even when promotion fails
    struct Promo { Entry *e; int slot, expert; };
    std::vector<Promo> deferred;                     // asynchronous promotions
    const bool async = g_cfg.async_promotions;
    int promoted = 0;
    for (uint32_t i = 0; i < n && promoted < g_cfg.max_promotions; ++i) {
        const uint32_t packed = g_h_stats[LOG_BASE + i];
        const int32_t cid = (int32_t) (packed >> 12);
        const int32_t expert = (int32_t) (packed & 0xFFF);
        int &count = g_admission[packed];
        count += 1;
        if (count < 2) continue;
        count = 0;
        if (cid < 0 || cid >= (int32_t) g_all.size()) continue;
        Entry *e = g_all[cid];
        if (expert < 0 || expert >= e->n_experts || e->slot_of[expert] >= 0) continue;
        int slot;
        if ((rc = acquire_slot_locked(e, stream, &slot))) return rc;
        if (slot < 0) continue;
        if (async) {
            deferred.push_back(Promo{e, slot, expert});
        } else {
            if ((rc = dev()->copy_h2d(e->pool + (size_t) slot * e->expert_bytes, e->data + (size_t) expert * e->expert_bytes,
                                      e->expert_bytes, stream)))
                return dev_err(rc, "promotion copy");
            e->h_tbl[expert] = pool_entry(e, slot);
            e->tbl_dirty = true;
        }
        e->slot_of[expert] = slot;
        e->expert_of[slot] = expert;
        promoted += 1;
        g_totals.promotions += 1;
    }
    if (!async) {
        // one table upload per touched tensor, after the pool copies
        for (Entry *e : g_all) {
            if (!e->tbl_dirty) continue;
            if ((rc = dev()->copy_h2d(e->d_tbl, e->h_tbl.data(), sizeof(uint64_t) * e->n_experts, stream))) return dev_err(rc, "table flush");
            e->tbl_dirty = false;
        }
    } else {
        // demotions on the caller's stream, ahead of the next token's kernels
        for (Entry *e : g_all) {
            if (!e->tbl_dirty) continue;
            if ((rc = upload_table_staged_locked(e, 0, stream))) return rc;
            e->tbl_dirty = false;
        }
        if (!deferred.empty()) {
            if (!g_copy_stream && (rc = dev()->stream_create(&g_copy_stream))) return dev_err(rc, "copy stream");
            if (!g_order_event && (rc = dev()->event_create(&g_order_event))) return dev_err(rc, "event");
            if (!g_copy_event && (rc = dev()->event_create(&g_copy_event))) return dev_err(rc, "event");
            if ((rc = dev()->event_record(g_order_event, stream))) return dev_err(rc, "event record");
            if ((rc = dev()->stream_wait_event(g_copy_stream, g_order_event))) return dev_err(rc, "stream wait");
            // a slot taken twice this step (its first promotion evicted again) keeps its last expert
            for (const Promo &p : deferred) {
                if (p.e->expert_of[p.slot] != p.expert) continue;
                if ((rc = dev()->copy_h2d(p.e->pool + (size_t) p.slot * p.e->expert_bytes,
                                          p.e->data + (size_t) p.expert * p.e->expert_bytes, p.e->expert_bytes,
                                          g_copy_stream)))
                    return dev_err(rc, "promotion copy");
                p.e->h_tbl[p.expert] = pool_entry(p.e, p.slot);
                p.e->tbl_dirty = true;
            }
            for (Entry *e : g_all) {
                if (!e->tbl_dirty) continue;
                if ((rc = upload_table_staged_locked(e, 1, g_copy_stream))) return rc;
                e->tbl_dirty = false;
            }
            if ((rc = dev()->event_record(g_copy_event, g_copy_stream))) return dev_err(rc, "event record");
            g_copy_pending = true;
        }
    }
    if (g_admission.size() > 8192) {
        for (auto it = g_admission.begin(); it != g_admission.end();) {
            if (it->second == 0) it = g_admission.erase(it);
            else ++it;
        }
    }
    g_totals.admission_size = (uint32_t) g_admission.size();
    return 0;
}

int resident_table_locked(const void *data, int n_experts, size_t eb, void *stream, Resident **out) {
    // The table of a device-resident tensor is a pure function of (base, n_experts,
    // expert_bytes).  Allocators reuse addresses, so a cached table whose shape no
    // longer matches is rewritten in place (stream-ordered after earlier launches).
    int rc;
    Resident *r;
    auto it = g_resident.find(data);
    if (it != g_resident.end()) {
        r = it->second;
        if (r->n_experts == n_experts && r->expert_bytes == eb) {
            *out = r;
            return 0;
        }
        // earlier launches and the previous upload (from h_tbl) must be done first
        if ((rc = dev()->sync(stream))) return dev_err(rc, "stream sync");
        if (r->cap < n_experts) {
            if ((rc = dev()->free_dev(r->d_tbl))) return dev_err(rc, "resident table free");
            r->d_tbl = nullptr;
        }
    } else {
        r = new Resident();
        g_resident[data] = r;
    }
    if (!r->d_tbl) {
        if ((rc = dev()->malloc_dev((void **) &r->d_tbl, sizeof(uint64_t) * (size_t) n_experts))) {
            g_resident.erase(data);
            delete r;
            return dev_err(rc, "resident table alloc");
        }
        r->cap = n_experts;
    }
    r->n_experts = n_experts;
    r->expert_bytes = eb;
    r->h_tbl.resize(n_experts);
    for (int i = 0; i < n_experts; ++i) r->h_tbl[i] = (uint64_t) ((uintptr_t) data + (uintptr_t) i * eb);
    if ((rc = dev()->copy_h2d(r->d_tbl, r->h_tbl.data(), sizeof(uint64_t) * n_experts, stream))) return dev_err(rc, "resident table upload");
    *out = r;
    return 0;
}

bool wants_impl(const ggml_hip_moe_tensor *src0) {
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        read_env_locked();
        if (!g_cfg.enabled) return false;
    }
    if (!src0 || !src0->has_buffer || !src0->data) return false;
    if (ptr_kind_cached(src0->data) != PTR_HOST) {
        if (g_cfg.debug && src0->ne[2] > 1)
            fprintf(stderr, "moe-cache: wants? %s type=%d ne2=%lld ptr=%p: not GPU-readable host memory\n",
                    src0->name ? src0->name : "<tensor>", src0->type, (long long) src0->ne[2], src0->data);
        return false;
    }
    if (!type_supported(src0->type)) return false;
    if (src0->ne[2] < 2 || src0->ne[3] != 1 || src0->is_view) return false;
    return is_contiguous(src0);
}

// Inputs of the fused decode kernels (GemvArgs fields of the same names).
struct FfnExtra {
    int mode = FFN_NONE;
    const float *nx = nullptr;
    int64_t nx_stride = 0;
    const float *nw = nullptr;
    float eps = 0.0f;
    uint8_t *y_out = nullptr;
    int64_t y_out_stride = 0;
    uint8_t *hq = nullptr;
    int64_t hq_stride_col = 0, hq_stride_pick = 0;
    uint8_t *hq_sh = nullptr;
    int64_t hq_sh_stride = 0;
    const float *router_w = nullptr;
    const float *residual = nullptr;
    float *x_out = nullptr;
    int64_t x_stride = 0;
    bool sh_act_f32 = false;         // FFN_DOWN_COMBINE: the shared expert's rows are fp32
    int dot_act = ACT_Q8_1;          // the dots' activation format (ACT_Q8_1 or ACT_Q8_K)
};

// Shared validation + launch of the GEMV (and of the fused decode kernels when fx is given).
int gemv_common(int use_cache, int act, const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *gate_host,
                const ggml_hip_moe_fusion *fusion, const void *src1, const int32_t *ids_d, float *dst_d,
                int64_t ne00, int64_t ne01, int64_t ne02, int64_t ncols_dst, int64_t nchannels_y, int64_t nchannels_dst,
                int64_t stride_col_y, int64_t stride_col_dst, int64_t stride_channel_y, int64_t stride_channel_dst,
                int64_t ids_stride, void *stream, const FfnExtra *fx = nullptr, bool no_tables = false) {
    const int mode = fx ? fx->mode : FFN_NONE;
    if (!src0 || !src1 || !ids_d || !dst_d) return fail(E_INVALID, "moe-gemv: null argument");
    const int tw = src0->type;
    if (!type_supported(tw)) return fail(E_UNSUPPORTED, "moe-gemv: unsupported expert type %d", tw);
    const TypeGeom g = type_geom(tw);
    if (ne00 <= 0 || ne01 <= 0 || ne02 <= 0 || ncols_dst <= 0 || nchannels_dst <= 0 || nchannels_y <= 0)
        return fail(E_INVALID, "moe-gemv: empty shape");
    if (ne00 % g.unit_elems) return fail(E_UNSUPPORTED, "moe-gemv: ne00=%lld is not a multiple of %d", (long long) ne00, g.unit_elems);
    // the plain GEMV streams rows of more than 64 units in chunks; the fused decode kernels
    // hold one row per step (at most 64 units)
    if (mode != FFN_NONE && ne00 / g.unit_elems > WAVE)
        return fail(E_UNSUPPORTED, "moe-ffn: ne00=%lld exceeds %d units per row", (long long) ne00, WAVE);
    if (ne00 > GEMV_MAX_K || (act == ACT_F32 && ne00 > GEMV_MAX_K_F32))
        return fail(E_UNSUPPORTED, "moe-gemv: ne00=%lld exceeds the staged activation row (%d values, %d for fp32 rows)",
                    (long long) ne00, GEMV_MAX_K, GEMV_MAX_K_F32);
    if (src0->ne[0] != ne00 || src0->ne[1] != ne01 || src0->ne[2] != ne02 || !is_contiguous(src0))
        return fail(E_INVALID, "moe-gemv: src0 shape/strides do not match the call");
    if (act != ACT_Q8_1 && act != ACT_Q8_K && act != ACT_F32)
        return fail(E_INVALID, "moe-gemv: unknown activation format %d", act);
    if (act == ACT_Q8_K && !g.kquant) return fail(E_UNSUPPORTED, "moe-gemv: q8_K activations need K-quant weights");
    const size_t eb = (size_t) src0->nb[2];
    if (eb > 0xFFFFFFF0ull) return fail(E_UNSUPPORTED, "moe-gemv: expert matrix larger than 4 GiB");
    if (ids_stride < nchannels_dst) return fail(E_INVALID, "moe-gemv: ids_stride < nchannels_dst");
    if (ne02 > 4096) return fail(E_UNSUPPORTED, "moe-gemv: more than 4096 experts cannot be packed in the miss log");

    int ts = 0;
    const void *sh_up = fusion ? fusion->shared_up : nullptr;
    if (sh_up) {
        ts = fusion->shared_type < 0 ? tw : fusion->shared_type;
        if (!type_supported(ts)) return fail(E_UNSUPPORTED, "moe-gemv: unsupported shared-expert type %d", ts);
        if (ne00 % type_geom(ts).unit_elems || (mode != FFN_NONE && ne00 / type_geom(ts).unit_elems > WAVE))
            return fail(E_UNSUPPORTED, "moe-gemv: shared-expert row length not supported");
        if (act == ACT_Q8_K && !type_geom(ts).kquant) return fail(E_UNSUPPORTED, "moe-gemv: q8_K activations need a K-quant shared expert");
        if (!fusion->shared_dst && mode != FFN_DOWN_COMBINE) return fail(E_INVALID, "moe-gemv: shared_up without shared_dst");
    }
    if (mode != FFN_NONE) {
        // the fused decode kernels are built for K-quant experts (and K-quant shared experts)
        if (!g.kquant || (ts && !type_geom(ts).kquant))
            return fail(E_UNSUPPORTED, "moe-ffn: fused decode kernels take K-quant experts (type %d, shared %d)", tw, ts);
    }
    const bool aligned_ok = g.aligned ? ((((uintptr_t) src0->data) | eb) & 3u) == 0 : ((((uintptr_t) src0->data) | eb) & 1u) == 0;
    if (!aligned_ok) return fail(E_UNSUPPORTED, "moe-gemv: expert base/size alignment not supported");

    GemvArgs a = {};
    // strides count activation blocks (q8_1: 32 values, q8_K: 256) or floats (fp32 rows)
    const int ablk_bytes = act == ACT_Q8_1 ? 36 : act == ACT_Q8_K ? 292 : 4;
    const int ablk_elems = act == ACT_Q8_1 ? 32 : act == ACT_Q8_K ? 256 : 1;
    if (act == ACT_F32 && (((uintptr_t) src1) & 3u)) return fail(E_INVALID, "moe-gemv: misaligned fp32 activations");
    if (ne00 % ablk_elems) return fail(E_INVALID, "moe-gemv: ne00 not a multiple of the activation block");
    const int64_t act_row = ne00 / ablk_elems * ablk_bytes;
    a.y = (const uint8_t *) src1;
    a.stride_col_y = stride_col_y * ablk_bytes;
    a.stride_channel_y = stride_channel_y * ablk_bytes;
    a.nchannels_y = (uint32_t) nchannels_y;
    const int64_t y_extent = (nchannels_y - 1) * a.stride_channel_y + (ncols_dst - 1) * a.stride_col_y + act_row;
    if (y_extent <= 0 || y_extent > 0xFFFFFFF0ll) return fail(E_INVALID, "moe-gemv: activation extent out of range");
    a.y_bytes = (uint64_t) y_extent;
    a.ids = ids_d;
    a.ids_stride = ids_stride;
    a.dst = dst_d;
    a.stride_col_dst = stride_col_dst;
    a.stride_channel_dst = stride_channel_dst;
    a.ncols = (int32_t) ne00;
    a.nrows = (int32_t) ne01;
    a.n_used = (int32_t) nchannels_dst;
    a.n_tok = (int32_t) ncols_dst;
    a.n_experts = (int32_t) ne02;
    a.expert_bytes = eb;
    a.cache_id = -1;
    a.cache_id_gate = -1;
    a.glu_op = 2;                  // SWIGLU unless the fusion says otherwise (kernels/moe-cache.cu:116)
    a.bias_stride = stride_channel_dst;
    a.spin_limit = __atomic_load_n(&g_spin_limit, __ATOMIC_RELAXED);
    if (fusion) {
        a.x_bias = fusion->x_bias;
        a.gate_bias = fusion->gate_bias;
        a.x_scale = fusion->x_scale;
        a.gate_scale = fusion->gate_scale;
        a.bias_stride = fusion->bias_stride > 0 ? fusion->bias_stride : stride_channel_dst;
        a.glu_op = fusion->glu_op;
        a.glu_limit = fusion->glu_limit;
        if (sh_up) {
            a.sh_up = (const uint8_t *) sh_up;
            a.sh_gate = (const uint8_t *) fusion->shared_gate;
            a.sh_dst = fusion->shared_dst;
            a.sh_stride_col_dst = fusion->shared_stride_col_dst;
            a.sh_matrix_bytes = (uint64_t) (ne00 / type_geom(ts).block_elems) * type_geom(ts).block_bytes * (uint64_t) ne01;
            if (fusion->shared_src1) {
                // fp32 shared rows beside q8_1 routed rows: strides in floats
                const bool shf = fx && fx->sh_act_f32;
                const int64_t sh_blk = shf ? 4 : ablk_bytes, sh_row = shf ? ne00 * 4 : act_row;
                if (shf && (((uintptr_t) fusion->shared_src1) & 15u))
                    return fail(E_INVALID, "moe-ffn: fp32 shared rows must be 16-byte aligned");
                a.sh_act_f32 = shf ? 1 : 0;
                a.sh_y = (const uint8_t *) fusion->shared_src1;
                a.sh_stride_col_y = fusion->shared_stride_col_y * sh_blk;
                a.sh_y_bytes = (uint64_t) ((ncols_dst - 1) * a.sh_stride_col_y + sh_row);
            }
        }
    }

    const bool gate_wants = use_cache && gate_host ? wants_impl(gate_host) : false;
    std::lock_guard<std::mutex> lock(g_mutex);
    read_env_locked();
    int rc;
    if (use_cache) {
        if (!g_cfg.enabled) return fail(E_DISABLED, "moe-cache: not enabled (GGML_HIP_MOE_CACHE)");
        Entry *e = nullptr, *ge = nullptr;
        if ((rc = get_or_create_locked(src0, stream, &e))) return rc;
        a.tbl = e->d_tbl;
        a.stamps = e->d_stamps;
        a.cache_id = e->id;
        a.stats = g_d_stats;
        a.clock = g_d_clock;
        if (gate_host && fusion && fusion->gate) {
            return fail(E_INVALID, "moe-gemv: gate given both as host tensor and as device pointer");
        }
        if (gate_host) {
            if (gate_host->type != tw || gate_host->ne[0] != ne00 || gate_host->ne[1] != ne01 || gate_host->ne[2] != ne02 ||
                gate_host->nb[2] != src0->nb[2])
                return fail(E_INVALID, "moe-gemv: gate tensor does not match src0");
            if (gate_wants) {
                if ((rc = get_or_create_locked(gate_host, stream, &ge))) return rc;
                a.tbl_gate = ge->d_tbl;
                a.stamps_gate = ge->d_stamps;
                a.cache_id_gate = ge->id;
            } else {
                Resident *r;
                if ((rc = resident_table_locked(gate_host->data, (int) ne02, eb, stream, &r))) return rc;
                a.tbl_gate = r->d_tbl;
            }
            a.has_gate = 1;
        }
    } else if (!no_tables) {
        Resident *r;
        if ((rc = resident_table_locked(src0->data, (int) ne02, eb, stream, &r))) return rc;
        a.tbl = r->d_tbl;
    }
    if (fusion && fusion->gate) {
        // device-resident experts are addressed affinely (w_base below); the table only serves
        // the cache path, whose up tensor goes through a table too
        if (!no_tables) {
            Resident *r;
            if ((rc = resident_table_locked(fusion->gate, (int) ne02, eb, stream, &r))) return rc;
            a.tbl_gate = r->d_tbl;
        }
        a.has_gate = 1;
    }
    if (!use_cache) {
        // every expert is device memory at a fixed stride: the kernel computes the
        // address instead of reading the (identical) resident table entry
        a.w_base = (const uint8_t *) src0->data;
        a.w_gate_base = a.has_gate ? (const uint8_t *) fusion->gate : nullptr;
    }
    if (fx) {
        a.mode = fx->mode;
        a.nx = fx->nx;
        a.nx_stride = fx->nx_stride;
        a.nw = fx->nw;
        a.eps = fx->eps;
        a.y_out = fx->y_out;
        a.y_out_stride = fx->y_out_stride;
        a.hq = fx->hq;
        a.hq_stride_col = fx->hq_stride_col;
        a.hq_stride_pick = fx->hq_stride_pick;
        a.hq_sh = fx->hq_sh;
        a.hq_sh_stride = fx->hq_sh_stride;
        a.dot_act = fx->dot_act;
        a.router_w = fx->router_w;
        a.residual = fx->residual;
        a.x_out = fx->x_out;
        a.x_stride = fx->x_stride;
    }
    if ((rc = dev()->status_address(&a.status))) return dev_err(rc, "status word lookup");
    if ((rc = dev()->launch_gemv(a, tw, ts, act, stream))) return dev_err(rc, mode == FFN_NONE ? "GEMV launch" : "fused FFN launch");
    return 0;
}

int quantize_common(int kind, const float *x, void *y, int64_t k, int64_t nrows, int64_t x_stride, int64_t y_stride, void *stream) {
    const int be = kind == 1 ? 256 : 32;
    const int bb = kind == 1 ? 292 : 36;
    if (!x || !y) return fail(E_INVALID, "quantize: null argument");
    if (k <= 0 || nrows < 0 || k % be) return fail(E_INVALID, "quantize: k=%lld must be a positive multiple of %d", (long long) k, be);
    if (x_stride < k || y_stride < k / be) return fail(E_INVALID, "quantize: row stride smaller than the row");
    if (((uintptr_t) y & 3u) || ((uintptr_t) x & 3u)) return fail(E_INVALID, "quantize: misaligned buffers");
    QuantArgs q;
    q.x = x;
    q.y = (uint8_t *) y;
    q.k = k;
    q.nrows = nrows;
    q.x_stride = x_stride;
    q.y_stride = y_stride * bb;
    const int rc = dev()->launch_quantize(kind, q, stream);
    if (rc) return dev_err(rc, "quantize launch");
    return 0;
}

// ---------------------------------------------------------------------------
// MUL_MAT_ID at the op level: strides from the tensors, path choice, workspace
// ---------------------------------------------------------------------------

constexpr int GGML_TYPE_F32_ = 0, GGML_TYPE_I32_ = 26;
constexpr int64_t MMID_GEMV_MAX_TOKENS = 8;   // ggml-cuda's MMVQ batch limit; more tokens take the grouped GEMM

struct MmidPlan {
    bool cache = false, mmq = false;
    int64_t K = 0, R = 0, E = 0, n_used = 0, n_tok = 0, ne11 = 0;
    int kind = 0;                 // activation quantizer: 0 q8_1, 1 q8_K
    int64_t blk = 32, blk_bytes = 36;
    uint64_t y_bytes = 0, y_span = 0, ws_mmq = 0;
};

bool mmq_fusion_ok(const ggml_hip_moe_fusion *f) {
    return !f || !(f->x_bias || f->gate_bias || f->x_scale || f->gate_scale || f->shared_up);
}

int mmid_plan(const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *src1, const ggml_hip_moe_tensor *ids,
              const ggml_hip_moe_tensor *dst, const ggml_hip_moe_tensor *gate_host, const ggml_hip_moe_fusion *f,
              MmidPlan &p) {
    if (!src0 || !src1 || !ids) return fail(E_INVALID, "mul_mat_id: null tensor");
    if (!type_supported(src0->type)) return fail(E_UNSUPPORTED, "mul_mat_id: expert type %d is not supported", src0->type);
    p.K = src0->ne[0];
    p.R = src0->ne[1];
    p.E = src0->ne[2];
    p.n_used = ids->ne[0];
    p.n_tok = ids->ne[1];
    p.ne11 = src1->ne[1];
    if (src0->ne[3] != 1 || src1->ne[3] != 1 || ids->ne[2] != 1 || ids->ne[3] != 1)
        return fail(E_UNSUPPORTED, "mul_mat_id: 4-d batches are not supported");
    if (src1->type != GGML_TYPE_F32_ || src1->nb[0] != 4 || src1->ne[0] != p.K || src1->ne[2] != p.n_tok ||
        p.ne11 < 1 || (src1->nb[1] | src1->nb[2]) & 3 || src1->nb[1] < p.K * 4)
        return fail(E_INVALID, "mul_mat_id: src1 must be fp32 [K, channels, tokens] with contiguous rows");
    if (ids->type != GGML_TYPE_I32_ || ids->nb[0] != 4 || ids->nb[1] % 4 || ids->nb[1] < 4 * p.n_used || p.n_used < 1)
        return fail(E_INVALID, "mul_mat_id: ids must be int32 [n_used, tokens] with contiguous rows");
    if (dst && (dst->type != GGML_TYPE_F32_ || dst->nb[0] != 4 || dst->ne[0] != p.R || dst->ne[1] != p.n_used ||
                dst->ne[2] != p.n_tok || (dst->nb[1] | dst->nb[2]) & 3))
        return fail(E_INVALID, "mul_mat_id: dst must be fp32 [rows, n_used, tokens]");
    p.cache = wants_impl(src0);
    const TypeGeom g = type_geom(src0->type);
    const uint64_t eb = (uint64_t) src0->nb[2];
    const uintptr_t walign = src0->type == T_Q3_K || src0->type == T_Q6_K ? 1u : src0->type == T_Q2_K ? 3u : 15u;
    p.mmq = !p.cache && !gate_host && g.kquant && p.n_tok > MMID_GEMV_MAX_TOKENS && mmq_fusion_ok(f) &&
            p.E <= MMQ_MAX_EXPERTS && p.K % 256 == 0 &&
            !(((uintptr_t) src0->data | eb | (uintptr_t) (f ? f->gate : nullptr)) & walign) &&
            !((src0->type == T_Q3_K || src0->type == T_Q6_K) && f && f->gate &&
              (((uintptr_t) f->gate ^ (uintptr_t) src0->data) & 3u));
    p.kind = p.mmq ? 1 : 0;
    p.blk = p.mmq ? 256 : 32;
    p.blk_bytes = p.mmq ? 292 : 36;
    if (p.K % p.blk) return fail(E_UNSUPPORTED, "mul_mat_id: K=%lld is not a multiple of %lld", (long long) p.K, (long long) p.blk);
    p.y_span = (uint64_t) (p.n_tok * p.ne11) * (uint64_t) (p.K / p.blk * p.blk_bytes);
    p.y_bytes = (p.y_span + 255) & ~(uint64_t) 255;
    if (p.mmq) {
        MmqArgs a = {};
        a.ncols = (int32_t) p.K;
        a.n_experts = (int32_t) p.E;
        mmq_layout(a, p.n_tok * p.n_used);
        p.ws_mmq = a.ws_total;
    }
    return 0;
}


// The op-level MUL_MAT_ID once planned: src1 quantized into the workspace, then the
// grouped GEMM or the GEMV (no_tables: device-resident experts addressed affinely,
// no resident pointer table is built, so nothing is allocated).
int mmid_run(const MmidPlan &p, const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *src1,
             const ggml_hip_moe_tensor *ids, const ggml_hip_moe_tensor *dst, const ggml_hip_moe_tensor *gate_host,
             const ggml_hip_moe_fusion *fusion, uint8_t *y, void *stream, bool no_tables) {
    int rc;
    // activations: every (token, channel) row quantized back to back (q8_1 for the GEMV, q8_K for the grouped GEMM)
    const int64_t nb_row = p.K / p.blk;                        // activation blocks per row
    const float *x = (const float *) src1->data;
    const int64_t xs1 = src1->nb[1] / 4, xs2 = src1->nb[2] / 4;
    if (xs2 == xs1 * p.ne11) {
        if ((rc = quantize_common(p.kind, x, y, p.K, p.ne11 * p.n_tok, xs1, nb_row, stream))) return rc;
    } else {
        for (int64_t t = 0; t < p.n_tok; ++t)
            if ((rc = quantize_common(p.kind, x + t * xs2, y + t * p.ne11 * nb_row * p.blk_bytes, p.K, p.ne11, xs1, nb_row,
                                      stream)))
                return rc;
    }
    const int64_t ids_stride = ids->nb[1] / 4;
    const int64_t sc_dst = dst->nb[2] / 4, sch_dst = dst->nb[1] / 4;
    if (p.mmq) {
        return ggml_hip_moe_mul_mat_q(src0, fusion, y, (const int32_t *) ids->data, (float *) dst->data,
                                      p.K, p.R, p.E, p.n_tok, p.ne11, p.n_used, p.ne11 * nb_row, sc_dst, nb_row, sch_dst,
                                      ids_stride, y + p.y_bytes, (int64_t) p.ws_mmq, stream);
    }
    return gemv_common(p.cache ? 1 : 0, ACT_Q8_1, src0, gate_host, fusion, y, (const int32_t *) ids->data,
                       (float *) dst->data, p.K, p.R, p.E, p.n_tok, p.ne11, p.n_used, p.ne11 * nb_row, sc_dst, nb_row,
                       sch_dst, ids_stride, stream, nullptr, no_tables);
}


// ---------------------------------------------------------------------------
// graph-level fusion detection (the decision ggml-cuda makes before the
// intercept, patches/apply_patches.py:42-62; consumed at kernels/moe-cache.cu:109-129)
// ---------------------------------------------------------------------------

constexpr int OP_MUL_MAT = 1, OP_MUL_MAT_ID = 2, OP_ADD_ID = 3, OP_MUL = 4, OP_GLU = 6;

struct Graph {
    const ggml_hip_moe_node *n;
    int count;
    std::vector<int> uses;              // consumers of each node
    std::vector<int> sole;              // the only consumer, or -1

    Graph(const ggml_hip_moe_node *nodes, int cnt) : n(nodes), count(cnt), uses(cnt, 0), sole(cnt, -1) {
        for (int k = 0; k < cnt; ++k)
            for (int s = 0; s < 3; ++s) {
                const int j = nodes[k].src[s];
                if (j >= 0 && j < cnt && j != k) {
                    uses[j] += 1;
                    sole[j] = uses[j] == 1 ? k : -1;
                }
            }
    }
    // the same source: one node, or leaves over the same memory and shape
    bool same_src(int a, int sa, int b, int sb) const {
        const int ia = n[a].src[sa], ib = n[b].src[sb];
        if (ia >= 0 || ib >= 0) return ia == ib;
        const ggml_hip_moe_tensor &x = n[a].leaf[sa], &y = n[b].leaf[sb];
        return x.data == y.data && x.type == y.type && !memcmp(x.ne, y.ne, sizeof(x.ne)) && !memcmp(x.nb, y.nb, sizeof(x.nb));
    }
    // data pointer of a node's source (node result or leaf)
    const ggml_hip_moe_tensor &src_tensor(int k, int s) const {
        const int j = n[k].src[s];
        return j >= 0 ? n[j].t : n[k].leaf[s];
    }
};

// Follows an expert path from MUL_MAT_ID node `mm`: an optional MUL by a per-expert scale leaf
// with the same ids, then an optional ADD_ID by a per-expert bias leaf with the same ids -- the
// order in which the kernels apply them (kernels/moe-cache.cu:246-252, :257-262).  Returns the
// path's last node; bias / scale receive the leaves' data.
int follow_expert_path(const Graph &g, int mm, const float **bias, int64_t *bias_stride, const float **scale,
                       std::vector<int> &path) {
    int cur = mm;
    path.push_back(cur);
    const ggml_hip_moe_node &m = g.n[mm];
    const int64_t rows = m.t.ne[0];
    const int64_t n_exp = g.src_tensor(mm, 0).ne[2];
    int nxt = g.sole[cur];
    if (nxt >= 0 && g.n[nxt].op == OP_MUL && g.n[nxt].src[0] == cur && g.n[nxt].src[1] < 0 &&
        g.same_src(nxt, 2, mm, 2)) {
        const ggml_hip_moe_tensor &sc = g.n[nxt].leaf[1];
        if (sc.type == 0 && sc.ne[0] == 1 && sc.ne[1] == n_exp && sc.nb[1] == 4) {
            *scale = (const float *) sc.data;
            cur = nxt;
            path.push_back(cur);
            nxt = g.sole[cur];
        }
    }
    if (nxt >= 0 && g.n[nxt].op == OP_ADD_ID && g.n[nxt].src[0] == cur && g.n[nxt].src[1] < 0 &&
        g.same_src(nxt, 2, mm, 2)) {
        const ggml_hip_moe_tensor &b = g.n[nxt].leaf[1];
        if (b.type == 0 && b.ne[0] == rows && b.ne[1] == n_exp && b.nb[0] == 4 && b.nb[1] % 4 == 0) {
            *bias = (const float *) b.data;
            *bias_stride = (int64_t) (b.nb[1] / 4);
            cur = nxt;
            path.push_back(cur);
        }
    }
    return cur;
}

// routing trace files opened by ggml_hip_moe_trace_append: path -> append stream
std::mutex g_trace_mutex;
std::unordered_map<std::string, FILE *> g_trace_files;

}  // namespace
}  // namespace mc

using namespace mc;

extern "C" {

int ggml_hip_moe_cache_enabled(void) {
    std::lock_guard<std::mutex> lock(g_mutex);
    read_env_locked();
    return g_cfg.enabled ? 1 : 0;
}

int ggml_hip_moe_cache_wants(const ggml_hip_moe_tensor *src0) { return wants_impl(src0) ? 1 : 0; }

int ggml_hip_moe_cache_mul_mat_vec_q(const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *gate_host,
                                     const ggml_hip_moe_fusion *fusion, const void *src1_q8_1, const int32_t *ids_d,
                                     float *dst_d, int64_t ne00, int64_t ne01, int64_t ne02, int64_t ne03,
                                     int64_t ncols_dst, int64_t s01, int64_t s02, int64_t s03, int64_t nchannels_y,
                                     int64_t nchannels_dst, int64_t stride_col_y, int64_t stride_col_dst,
                                     int64_t stride_channel_y, int64_t stride_channel_dst, int64_t ids_stride, void *stream) {
    (void) s02; (void) s03;
    if (!src0) return fail(E_INVALID, "moe-gemv: null src0");
    if (ne03 != 1) return fail(E_UNSUPPORTED, "moe-gemv: ne03 != 1");
    const TypeGeom g = type_geom(src0->type);
    if (g.block_elems && s01 != ne00 / g.block_elems) return fail(E_UNSUPPORTED, "moe-gemv: non-contiguous rows (s01)");
    if (!wants_impl(src0)) return fail(E_STATE, "moe-cache: src0 does not qualify for the cache path (wants() == 0)");
    return gemv_common(1, ACT_Q8_1, src0, gate_host, fusion, src1_q8_1, ids_d, dst_d, ne00, ne01, ne02, ncols_dst, nchannels_y,
                       nchannels_dst, stride_col_y, stride_col_dst, stride_channel_y, stride_channel_dst, ids_stride, stream);
}

int ggml_hip_mul_mat_vec_q_moe(const ggml_hip_moe_tensor *src0, const ggml_hip_moe_fusion *fusion, const void *src1_q8_1,
                               const int32_t *ids_d, float *dst_d, int64_t ne00, int64_t ne01, int64_t ne02, int64_t ne03,
                               int64_t ncols_dst, int64_t s01, int64_t s02, int64_t s03, int64_t nchannels_y,
                               int64_t nchannels_dst, int64_t stride_col_y, int64_t stride_col_dst, int64_t stride_channel_y,
                               int64_t stride_channel_dst, int64_t ids_stride, void *stream) {
    (void) s02; (void) s03;
    if (!src0) return fail(E_INVALID, "moe-gemv: null src0");
    if (ne03 != 1) return fail(E_UNSUPPORTED, "moe-gemv: ne03 != 1");
    const TypeGeom g = type_geom(src0->type);
    if (g.block_elems && s01 != ne00 / g.block_elems) return fail(E_UNSUPPORTED, "moe-gemv: non-contiguous rows (s01)");
    return gemv_common(0, ACT_Q8_1, src0, nullptr, fusion, src1_q8_1, ids_d, dst_d, ne00, ne01, ne02, ncols_dst, nchannels_y,
                       nchannels_dst, stride_col_y, stride_col_dst, stride_channel_y, stride_channel_dst, ids_stride, stream);
}

int ggml_hip_moe_mul_mat_vec_ex(int use_cache, int act_format, const ggml_hip_moe_tensor *src0,
                                const ggml_hip_moe_tensor *gate_host, const ggml_hip_moe_fusion *fusion, const void *src1,
                                const int32_t *ids_d, float *dst_d, int64_t ne00, int64_t ne01, int64_t ne02,
                                int64_t ncols_dst, int64_t nchannels_y, int64_t nchannels_dst, int64_t stride_col_y,
                                int64_t stride_col_dst, int64_t stride_channel_y, int64_t stride_channel_dst,
                                int64_t ids_stride, void *stream) {
    if (use_cache && !wants_impl(src0)) return fail(E_STATE, "moe-cache: src0 does not qualify for the cache path (wants() == 0)");
    if (!use_cache && gate_host) return fail(E_INVALID, "moe-gemv: gate_host is for the cache path; pass fusion->gate");
    return gemv_common(use_cache ? 1 : 0, act_format, src0, gate_host, fusion, src1, ids_d, dst_d, ne00, ne01, ne02, ncols_dst,
                       nchannels_y, nchannels_dst, stride_col_y, stride_col_dst, stride_channel_y, stride_channel_dst,
                       ids_stride, stream);
}

int ggml_hip_moe_ffn_gate_up_norm(int use_cache, const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *gate_host,
                                  const ggml_hip_moe_fusion *fusion, const float *x, const float *norm_weight, float eps,
                                  const int32_t *ids_d, float *dst_d, int64_t ne00, int64_t ne01, int64_t ne02,
                                  int64_t ncols_dst, int64_t nchannels_dst, int64_t stride_col_x, int64_t stride_col_dst,
                                  int64_t stride_channel_dst, int64_t ids_stride, void *y_out, int64_t y_out_stride,
                                  void *dst_q8_1, int64_t q8_stride_col, int64_t q8_stride_channel,
                                  void *shared_dst_q8_1, int64_t shared_q8_stride_col, void *stream) {
    return ggml_hip_moe_ffn_gate_up_norm_ex(use_cache, ACT_Q8_1, src0, gate_host, fusion, x, norm_weight, eps, ids_d, dst_d,
                                            ne00, ne01, ne02, ncols_dst, nchannels_dst, stride_col_x, stride_col_dst,
                                            stride_channel_dst, ids_stride, y_out, y_out_stride, dst_q8_1, q8_stride_col,
                                            q8_stride_channel, shared_dst_q8_1, shared_q8_stride_col, stream);
}

int ggml_hip_moe_ffn_gate_up_norm_ex(int use_cache, int act_format, const ggml_hip_moe_tensor *src0,
                                     const ggml_hip_moe_tensor *gate_host, const ggml_hip_moe_fusion *fusion, const float *x,
                                     const float *norm_weight, float eps, const int32_t *ids_d, float *dst_d, int64_t ne00,
                                     int64_t ne01, int64_t ne02, int64_t ncols_dst, int64_t nchannels_dst,
                                     int64_t stride_col_x, int64_t stride_col_dst, int64_t stride_channel_dst,
                                     int64_t ids_stride, void *y_out, int64_t y_out_stride, void *dst_q8_1,
                                     int64_t q8_stride_col, int64_t q8_stride_channel, void *shared_dst_q8_1,
                                     int64_t shared_q8_stride_col, void *stream) {
    if (!x) return fail(E_INVALID, "moe-ffn: null x");
    if (act_format != ACT_Q8_1 && act_format != ACT_Q8_K)
        return fail(E_UNSUPPORTED, "moe-ffn: the normalized row is q8_1 or q8_K (act_format %d)", act_format);
    const bool q8k = act_format == ACT_Q8_K;
    if (q8k && (dst_q8_1 || shared_dst_q8_1))
        return fail(E_UNSUPPORTED, "moe-ffn: q8_K dots write fp32 outputs only (the down launch quantizes them)");
    if (dst_q8_1) {
        if (ne01 % 32) return fail(E_UNSUPPORTED, "moe-ffn: q8_1 outputs need ne01 %% 32 == 0");
        if (ne00 / 256 > 16) return fail(E_UNSUPPORTED, "moe-ffn: q8_1 outputs need at most 16 units per row");
        if ((((uintptr_t) dst_q8_1) | ((uintptr_t) shared_dst_q8_1)) & 3u)
            return fail(E_INVALID, "moe-ffn: q8_1 outputs must be 4-byte aligned");
    }
    if (use_cache && !wants_impl(src0)) return fail(E_STATE, "moe-cache: src0 does not qualify for the cache path (wants() == 0)");
    if (!use_cache && gate_host) return fail(E_INVALID, "moe-gemv: gate_host is for the cache path; pass fusion->gate");
    if (ne00 <= 0 || ne00 % 256 || ne00 > 8192) return fail(E_UNSUPPORTED, "moe-ffn: ne00=%lld must be a multiple of 256 up to 8192", (long long) ne00);
    if ((((uintptr_t) x) & 15u) || (stride_col_x & 3) || (ncols_dst > 1 && stride_col_x < ne00))
        return fail(E_INVALID, "moe-ffn: x rows must be 16-byte aligned and not overlap");
    if (norm_weight && (((uintptr_t) norm_weight) & 15u)) return fail(E_INVALID, "moe-ffn: norm_weight must be 16-byte aligned");
    if (y_out && ((((uintptr_t) y_out) & 3u) || (ncols_dst > 1 && y_out_stride < ne00 / (q8k ? 256 : 32))))
        return fail(E_INVALID, "moe-ffn: y_out rows must be 4-byte aligned and not overlap");
    if (fusion && fusion->shared_src1) return fail(E_INVALID, "moe-ffn: the shared expert reads the normalized row (shared_src1 must be NULL)");
    FfnExtra fx;
    fx.mode = FFN_GATE_UP_NORM;
    fx.nx = x;
    fx.nx_stride = stride_col_x;
    fx.nw = norm_weight;
    fx.eps = eps;
    fx.y_out = (uint8_t *) y_out;
    fx.y_out_stride = y_out_stride * (q8k ? 292 : 36);
    fx.dot_act = q8k ? ACT_Q8_K : ACT_Q8_1;
    fx.hq = (uint8_t *) dst_q8_1;
    fx.hq_stride_col = q8_stride_col * 36;
    fx.hq_stride_pick = q8_stride_channel * 36;
    fx.hq_sh = (uint8_t *) shared_dst_q8_1;
    fx.hq_sh_stride = shared_q8_stride_col * 36;
    // the dots read the q8_1 row built in LDS; src1 stands in for the activation argument
    return gemv_common(use_cache ? 1 : 0, ACT_Q8_1, src0, gate_host, fusion, x, ids_d, dst_d, ne00, ne01, ne02, ncols_dst,
                       1, nchannels_dst, 0, stride_col_dst, 0, stride_channel_dst, ids_stride, stream, &fx);
}

int ggml_hip_moe_ffn_down_combine(int use_cache, int act_format, const ggml_hip_moe_tensor *src0,
                                  const ggml_hip_moe_fusion *fusion, const void *src1, const int32_t *ids_d,
                                  const float *router_w, const float *residual, float *x_out, int64_t ne00, int64_t ne01,
                                  int64_t ne02, int64_t ncols_dst, int64_t nchannels_dst, int64_t stride_col_y,
                                  int64_t stride_channel_y, int64_t stride_col_x, int64_t ids_stride, void *stream) {
    if (!router_w || !x_out) return fail(E_INVALID, "moe-ffn: null router weights or x_out");
    if (use_cache && !wants_impl(src0)) return fail(E_STATE, "moe-cache: src0 does not qualify for the cache path (wants() == 0)");
    const bool sh_f32 = (act_format & GGML_HIP_MOE_ACT_SHARED_F32) != 0;
    const bool dot_q8k = (act_format & GGML_HIP_MOE_ACT_DOT_Q8_K) != 0;
    act_format &= ~(GGML_HIP_MOE_ACT_SHARED_F32 | GGML_HIP_MOE_ACT_DOT_Q8_K);
    if (act_format != ACT_Q8_1 && act_format != ACT_F32) return fail(E_UNSUPPORTED, "moe-ffn: down activations are q8_1 or fp32 rows");
    if (dot_q8k && act_format != ACT_F32) return fail(E_UNSUPPORTED, "moe-ffn: q8_K dots quantize fp32 rows (act_format F32)");
    if (fusion && (fusion->gate || fusion->shared_gate || fusion->gate_bias || fusion->gate_scale))
        return fail(E_INVALID, "moe-ffn: the down projection takes no gate");
    if (fusion && fusion->shared_up && !fusion->shared_src1) return fail(E_INVALID, "moe-ffn: shared expert without its activation row (shared_src1)");
    if (stride_col_x < ne01 && ncols_dst > 1) return fail(E_INVALID, "moe-ffn: x rows overlap");
    if ((((uintptr_t) x_out) | ((uintptr_t) residual) | ((uintptr_t) router_w)) & 3u) return fail(E_INVALID, "moe-ffn: misaligned fp32 buffers");
    FfnExtra fx;
    fx.mode = FFN_DOWN_COMBINE;
    fx.sh_act_f32 = sh_f32 || act_format == ACT_F32;
    fx.dot_act = dot_q8k ? ACT_Q8_K : ACT_Q8_1;
    fx.router_w = router_w;
    fx.residual = residual;
    fx.x_out = x_out;
    fx.x_stride = stride_col_x;
    // dst strides only set the default per-expert bias stride (ne01); the kernel writes x_out
    return gemv_common(use_cache ? 1 : 0, act_format, src0, nullptr, fusion, src1, ids_d, x_out, ne00, ne01, ne02, ncols_dst,
                       nchannels_dst, nchannels_dst, stride_col_y, ne01 * nchannels_dst, stride_channel_y, ne01, ids_stride,
                       stream, &fx);
}

int ggml_hip_moe_cache_step(void *stream) {
    std::lock_guard<std::mutex> lock(g_mutex);
    read_env_locked();
    if (!g_cfg.enabled || g_all.empty()) return 0;
    return step_locked(stream);
}

int ggml_hip_moe_cache_active(void) {
    std::lock_guard<std::mutex> lock(g_mutex);
    return g_all.empty() ? 0 : 1;
}

int ggml_hip_moe_cache_pin_host(const ggml_hip_moe_tensor *t) {
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        read_env_locked();
        if (!g_cfg.enabled) return 0;
    }
    if (!t || !t->has_buffer || !t->data) return 0;
    const int kind = dev()->ptr_kind(t->data);
    if (kind == PTR_HOST) return 1;
    if (kind == PTR_DEVICE || kind == PTR_MANAGED || kind == PTR_ERROR) return 0;
    if (!g_cfg.allow_register) {
        fail(E_STATE, "moe-cache: %s is not GPU-readable; allocate it with hipHostMalloc or set GGML_HIP_MOE_CACHE_ALLOW_REGISTER=1",
             t->name ? t->name : "<tensor>");
        return 0;
    }
    const uintptr_t page = 4096;
    const uintptr_t base = (uintptr_t) t->data & ~(page - 1);
    const uint64_t nbytes = t->nb[3] ? t->nb[3] : t->nb[2] * (uint64_t) t->ne[2];
    const uintptr_t end = ((uintptr_t) t->data + nbytes + page - 1) & ~(page - 1);
    const int rc = dev()->register_host((void *) base, end - base);
    {
        std::lock_guard<std::mutex> lock(g_ptr_mutex);
        g_ptr_kind.erase(t->data);
    }
    if (rc) {
        fail(E_DEVICE, "moe-cache: failed to pin %s: %s", t->name ? t->name : "<tensor>", dev()->error_string(rc));
        return 0;
    }
    return 1;
}

int ggml_hip_quantize_q8_1(const float *x, void *y, int64_t k, int64_t nrows, int64_t x_stride, int64_t y_stride, void *stream) {
    return quantize_common(0, x, y, k, nrows, x_stride, y_stride, stream);
}

int ggml_hip_quantize_q8_K(const float *x, void *y, int64_t k, int64_t nrows, int64_t x_stride, int64_t y_stride, void *stream) {
    return quantize_common(1, x, y, k, nrows, x_stride, y_stride, stream);
}

int ggml_hip_quantize_q8_0_as_q8_1(const float *x, void *y, int64_t k, int64_t nrows, int64_t x_stride, int64_t y_stride,
                                   void *stream) {
    return quantize_common(2, x, y, k, nrows, x_stride, y_stride, stream);
}

int ggml_hip_moe_combine_q8_1(const float *o, int64_t o_stride, const float *w, int32_t n_used, const float *shared,
                              int64_t shared_stride, const float *residual, float *x_out, void *y_q8_1, int64_t y_stride,
                              int64_t k, int64_t n_tok, int32_t rms_norm, const float *norm_weight, float eps,
                              void *stream) {
    if (!y_q8_1 || (n_used > 0 && (!o || !w))) return fail(E_INVALID, "combine: null argument");
    if (k <= 0 || k % 256 || k > 8192 || n_used < 0 || n_used > 16 || n_tok < 0 || (n_used > 0 && o_stride < k) ||
        (shared && shared_stride < k) || y_stride < k / 32)
        return fail(E_INVALID, "combine: bad shape");
    if ((uintptr_t) y_q8_1 & 3u) return fail(E_INVALID, "combine: misaligned output");
    // the kernel moves 4 floats per lane: rows and strides on 16-byte boundaries
    if ((((uintptr_t) o | (uintptr_t) shared | (uintptr_t) residual | (uintptr_t) x_out | (uintptr_t) norm_weight) & 15u) ||
        (o_stride & 3) || (shared_stride & 3))
        return fail(E_INVALID, "combine: fp32 rows and strides must be 16-byte aligned");
    CombineArgs c;
    c.o = o;
    c.o_stride = o_stride;
    c.w = w;
    c.shared = shared;
    c.shared_stride = shared_stride;
    c.residual = residual;
    c.x_out = x_out;
    c.y = (uint8_t *) y_q8_1;
    c.y_stride = y_stride * 36;
    c.k = k;
    c.n_used = n_used;
    c.n_tok = (int32_t) n_tok;
    c.rms_norm = rms_norm != 0;
    c.norm_weight = norm_weight;
    c.eps = eps;
    const int rc = dev()->launch_combine(c, stream);
    if (rc) return dev_err(rc, "combine launch");
    return 0;
}

int64_t ggml_hip_moe_mul_mat_q_workspace_bytes(int64_t ne00, int64_t ne02, int64_t n_pairs) {
    if (ne00 <= 0 || ne00 % 256 || ne02 <= 0 || n_pairs < 0) return 0;
    MmqArgs a = {};
    a.ncols = (int32_t) ne00;
    a.n_experts = (int32_t) ne02;
    mmq_layout(a, n_pairs);
    return (int64_t) a.ws_total;
}

int ggml_hip_moe_mul_mat_q(const ggml_hip_moe_tensor *src0, const ggml_hip_moe_fusion *fusion, const void *src1_q8_K,
                           const int32_t *ids_d, float *dst_d, int64_t ne00, int64_t ne01, int64_t ne02,
                           int64_t ncols_dst, int64_t nchannels_y, int64_t nchannels_dst, int64_t stride_col_y,
                           int64_t stride_col_dst, int64_t stride_channel_y, int64_t stride_channel_dst,
                           int64_t ids_stride, void *workspace, int64_t workspace_bytes, void *stream) {
    if (!src0 || !src0->data || !src1_q8_K || !ids_d || !dst_d || !workspace)
        return fail(E_INVALID, "mul_mat_q: null argument");
    const int tw = src0->type;
    if (tw != T_Q2_K && tw != T_Q3_K && tw != T_Q4_K && tw != T_Q5_K && tw != T_Q6_K)
        return fail(E_UNSUPPORTED, "mul_mat_q: expert type %d is not supported", tw);
    if (ne00 <= 0 || ne00 % 256 || ne01 <= 0 || ne02 <= 0 || ncols_dst <= 0 || nchannels_dst <= 0 || nchannels_y <= 0)
        return fail(E_INVALID, "mul_mat_q: bad shape");
    if (ne02 > MMQ_MAX_EXPERTS) return fail(E_UNSUPPORTED, "mul_mat_q: more than %d experts", MMQ_MAX_EXPERTS);
    if (src0->ne[0] != ne00 || src0->ne[1] != ne01 || src0->ne[2] != ne02 || !is_contiguous(src0))
        return fail(E_INVALID, "mul_mat_q: src0 shape/strides do not match the call");
    if (ids_stride < nchannels_dst) return fail(E_INVALID, "mul_mat_q: ids_stride < nchannels_dst");
    if (ncols_dst * nchannels_dst > INT32_MAX) return fail(E_INVALID, "mul_mat_q: too many pairs");
    if (fusion && (fusion->x_bias || fusion->gate_bias || fusion->x_scale || fusion->gate_scale || fusion->shared_up))
        return fail(E_UNSUPPORTED, "mul_mat_q: only the gate/GLU fusion is supported");
    const uint64_t eb = (uint64_t) src0->nb[2];
    if (eb > 0xFFFFFFF0ull) return fail(E_UNSUPPORTED, "mul_mat_q: expert matrix larger than 4 GiB");
    // the weight tiles are fetched in 16-byte pieces (Q4_K/Q5_K), dwords (Q2_K) or dword windows
    // around 2-byte aligned super-blocks (Q3_K/Q6_K: the gate must share the up matrix's alignment)
    const bool windows = tw == T_Q3_K || tw == T_Q6_K;
    const uintptr_t walign = windows ? 1u : tw == T_Q2_K ? 3u : 15u;
    if (((uintptr_t) src0->data | eb | (uintptr_t) (fusion ? fusion->gate : nullptr)) & walign)
        return fail(E_UNSUPPORTED, "mul_mat_q: expert weights must be %d-byte aligned", (int) walign + 1);
    if (windows && fusion && fusion->gate && (((uintptr_t) fusion->gate ^ (uintptr_t) src0->data) & 3u))
        return fail(E_UNSUPPORTED, "mul_mat_q: Q3_K/Q6_K gate and up matrices must share their address mod 4");
    if (((uintptr_t) src1_q8_K | (uintptr_t) workspace) & 255u)
        return fail(E_INVALID, "mul_mat_q: activations and workspace must be 256-byte aligned");
    MmqArgs a = {};
    a.w = (const uint8_t *) src0->data;
    a.w_gate = fusion ? (const uint8_t *) fusion->gate : nullptr;
    a.expert_bytes = eb;
    a.y = (const uint8_t *) src1_q8_K;
    a.stride_col_y = stride_col_y * 292;
    a.stride_channel_y = stride_channel_y * 292;
    a.nchannels_y = (int32_t) nchannels_y;
    a.ids = ids_d;
    a.ids_stride = ids_stride;
    a.dst = dst_d;
    a.stride_col_dst = stride_col_dst;
    a.stride_channel_dst = stride_channel_dst;
    a.ncols = (int32_t) ne00;
    a.nrows = (int32_t) ne01;
    a.n_experts = (int32_t) ne02;
    a.n_used = (int32_t) nchannels_dst;
    a.n_tok = (int32_t) ncols_dst;
    a.glu_op = fusion ? fusion->glu_op : 2;
    a.glu_limit = fusion ? fusion->glu_limit : 0.0f;
    a.ws = (uint8_t *) workspace;
    mmq_layout(a, ncols_dst * nchannels_dst);
    if ((uint64_t) workspace_bytes < a.ws_total)
        return fail(E_INVALID, "mul_mat_q: workspace of %lld bytes, %llu needed", (long long) workspace_bytes,
                    (unsigned long long) a.ws_total);
    const int rc = dev()->launch_mmq(a, tw, stream);
    if (rc) return dev_err(rc, "mul_mat_q launch");
    return 0;
}

int64_t ggml_hip_moe_mul_mat_id_workspace_bytes(const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *src1,
                                                const ggml_hip_moe_tensor *ids, const ggml_hip_moe_fusion *fusion) {
    MmidPlan p;
    if (mmid_plan(src0, src1, ids, nullptr, nullptr, fusion, p)) return -1;
    return (int64_t) (p.y_bytes + p.ws_mmq);
}

int ggml_hip_moe_mul_mat_id(const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *src1,
                            const ggml_hip_moe_tensor *ids, const ggml_hip_moe_tensor *dst,
                            const ggml_hip_moe_tensor *gate_host, const ggml_hip_moe_fusion *fusion, void *workspace,
                            int64_t workspace_bytes, void *stream) {
    if (!dst) return fail(E_INVALID, "mul_mat_id: null dst");
    MmidPlan p;
    int rc;
    if ((rc = mmid_plan(src0, src1, ids, dst, gate_host, fusion, p))) return rc;
    if (p.n_tok == 0) return 0;
    if (!workspace || ((uintptr_t) workspace & 255u)) return fail(E_INVALID, "mul_mat_id: workspace must be 256-byte aligned");
    if ((uint64_t) workspace_bytes < p.y_bytes + p.ws_mmq)
        return fail(E_INVALID, "mul_mat_id: workspace of %lld bytes, %llu needed", (long long) workspace_bytes,
                    (unsigned long long) (p.y_bytes + p.ws_mmq));
    return mmid_run(p, src0, src1, ids, dst, gate_host, fusion, (uint8_t *) workspace, stream, false);
}

int ggml_hip_moe_mul_mat_id_noalloc(const ggml_hip_moe_tensor *src0, const ggml_hip_moe_tensor *src1,
                                    const ggml_hip_moe_tensor *ids, const ggml_hip_moe_tensor *dst,
                                    const ggml_hip_moe_fusion *fusion, void *stream) {
    if (!dst) return fail(E_INVALID, "mul_mat_id_noalloc: null dst");
    MmidPlan p;
    int rc;
    if ((rc = mmid_plan(src0, src1, ids, dst, nullptr, fusion, p))) return rc;
    if (p.cache)
        return fail(E_UNSUPPORTED, "mul_mat_id_noalloc: host-resident experts take the cache path, whose registration "
                    "allocates the HBM pool; this entry takes device-resident experts only");
    void *ws = nullptr;
    size_t cap = 0;
    if ((rc = dev()->scratch_address(&ws, &cap))) return dev_err(rc, "scratch lookup");
    const uint64_t need = p.y_bytes + p.ws_mmq;
    if (need > (uint64_t) cap)
        return fail(E_UNSUPPORTED, "mul_mat_id_noalloc: this call needs %llu bytes of workspace, the library's "
                    "scratch holds %llu (use ggml_hip_moe_mul_mat_id with a workspace of that size)",
                    (unsigned long long) need, (unsigned long long) cap);
    if (p.n_tok == 0) return 0;
    return mmid_run(p, src0, src1, ids, dst, nullptr, fusion, (uint8_t *) ws, stream, true);
}

int ggml_hip_ssm_conv_f32(const float *src0, int64_t src0_nb0, int64_t src0_nb1, int64_t src0_nb2, const void *src1,
                          int32_t src1_type, int64_t src1_nb1, const float *bias, int32_t fuse_silu, float *dst,
                          int64_t dst_nb0, int64_t dst_nb1, int64_t dst_nb2, int64_t nc, int64_t nr, int64_t n_t,
                          int64_t n_s, void *stream) {
    if (!src0 || !src1 || !dst) return fail(E_INVALID, "ssm_conv: null argument");
    if (src1_type != 0 && src1_type != 1) return fail(E_UNSUPPORTED, "ssm_conv: weight type %d (F32 or F16 only)", src1_type);
    if (nc != 3 && nc != 4 && nc != 5 && nc != 9 && nc != 15)
        return fail(E_UNSUPPORTED, "ssm_conv: only kernel sizes 3, 4, 5, 9, 15 are supported (got %lld)", (long long) nc);
    if (bias && !fuse_silu) return fail(E_INVALID, "ssm_conv: a fused bias comes with the fused SiLU");
    if (nr <= 0 || n_t < 0 || n_s < 0 || nr > INT32_MAX || n_t > INT32_MAX || n_s > 65535)
        return fail(E_INVALID, "ssm_conv: bad shape (nr %lld, n_t %lld, n_s %lld)", (long long) nr, (long long) n_t,
                    (long long) n_s);
    if (src0_nb0 != 4 || dst_nb0 != 4) return fail(E_INVALID, "ssm_conv: conv_x and dst rows must be contiguous floats");
    const size_t esz = src1_type ? 2 : 4;
    if (src0_nb1 < (nc - 1 + n_t) * 4 || (src0_nb1 | src0_nb2) & 3 || (n_s > 1 && src0_nb2 < src0_nb1 * nr))
        return fail(E_INVALID, "ssm_conv: conv_x strides (nb1 %lld, nb2 %lld)", (long long) src0_nb1, (long long) src0_nb2);
    if (src1_nb1 < nc * (int64_t) esz || src1_nb1 % (int64_t) esz)
        return fail(E_INVALID, "ssm_conv: weight row stride %lld", (long long) src1_nb1);
    if (dst_nb1 < nr * 4 || (dst_nb1 | dst_nb2) & 3 || (n_s > 1 && dst_nb2 < dst_nb1 * n_t))
        return fail(E_INVALID, "ssm_conv: dst strides (nb1 %lld, nb2 %lld)", (long long) dst_nb1, (long long) dst_nb2);
    if ((uintptr_t) src0 & 3 || (uintptr_t) dst & 3 || (uintptr_t) src1 & (esz - 1) || (uintptr_t) bias & 3)
        return fail(E_INVALID, "ssm_conv: misaligned pointer");
    SsmConvArgs a = {};
    a.x = src0;
    a.x_nb1 = src0_nb1;
    a.x_nb2 = src0_nb2;
    a.w = src1;
    a.w_nb1 = src1_nb1;
    a.w_f16 = src1_type;
    a.bias = bias;
    a.silu = fuse_silu ? 1 : 0;
    a.dst = dst;
    a.dst_nb1 = dst_nb1;
    a.dst_nb2 = dst_nb2;
    a.nc = (int32_t) nc;
    a.nr = (int32_t) nr;
    a.n_t = (int32_t) n_t;
    a.n_s = (int32_t) n_s;
    const int rc = dev()->launch_ssm_conv(a, stream);
    if (rc) return dev_err(rc, "ssm_conv launch");
    return 0;
}

int ggml_hip_moe_cache_configure(const ggml_hip_moe_config *cfg) {
    if (!cfg) return fail(E_INVALID, "configure: null config");
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_all.empty()) return fail(E_STATE, "configure: tensors are already registered (call reset first)");
    Config c;
    c.enabled = cfg->enabled != 0;
    c.slots = cfg->slots;
    c.budget_gb = cfg->budget_gb;
    c.margin_gb = cfg->margin_gb >= 0 ? cfg->margin_gb : 2.0;
    c.seed_path = cfg->seed_path ? cfg->seed_path : "";
    c.max_promotions = cfg->max_promotions >= 0 ? cfg->max_promotions : DEFAULT_MAX_PROMOTIONS;
    c.verbose = cfg->verbose != 0;
    c.debug = false;
    c.allow_register = g_cfg.allow_register;
    c.async_promotions = cfg->async_promotions != 0;
    g_cfg = c;
    g_cfg_ready = true;
    g_seed.clear();
    g_seed_loaded = false;
    return 0;
}

int ggml_hip_moe_cache_get_config(ggml_hip_moe_config *out) {
    if (!out) return fail(E_INVALID, "get_config: null");
    std::lock_guard<std::mutex> lock(g_mutex);
    read_env_locked();
    out->enabled = g_cfg.enabled;
    out->slots = g_cfg.slots;
    out->budget_gb = g_cfg.budget_gb;
    out->margin_gb = g_cfg.margin_gb;
    out->seed_path = g_cfg.seed_path.c_str();
    out->max_promotions = g_cfg.max_promotions;
    out->verbose = g_cfg.verbose;
    out->async_promotions = g_cfg.async_promotions ? 1 : 0;
    return 0;
}

int ggml_hip_moe_cache_num_entries(void) {
    std::lock_guard<std::mutex> lock(g_mutex);
    return (int) g_all.size();
}

int ggml_hip_moe_cache_entry_info(int32_t id, ggml_hip_moe_entry_info *out) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!out || id < 0 || id >= (int32_t) g_all.size()) return fail(E_INVALID, "entry_info: bad id %d", id);
    const Entry *e = g_all[id];
    out->id = e->id;
    out->type = e->type;
    out->n_experts = e->n_experts;
    out->n_slots = e->n_slots;
    out->expert_bytes = e->expert_bytes;
    int res = 0;
    for (int s = 0; s < e->n_slots; ++s) res += e->expert_of[s] >= 0;
    out->n_resident = res;
    out->stamps_clock = e->stamps_clock;
    return 0;
}

int ggml_hip_moe_cache_entry_slots(int32_t id, int32_t *slot_of, int32_t n_experts, int32_t *expert_of, int32_t n_slots) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (id < 0 || id >= (int32_t) g_all.size()) return fail(E_INVALID, "entry_slots: bad id %d", id);
    const Entry *e = g_all[id];
    if (slot_of) {
        if (n_experts < e->n_experts) return fail(E_INVALID, "entry_slots: slot_of too small");
        memcpy(slot_of, e->slot_of.data(), sizeof(int32_t) * e->n_experts);
    }
    if (expert_of) {
        if (n_slots < e->n_slots) return fail(E_INVALID, "entry_slots: expert_of too small");
        if (e->n_slots) memcpy(expert_of, e->expert_of.data(), sizeof(int32_t) * e->n_slots);
    }
    return 0;
}

int ggml_hip_moe_cache_entry_table(int32_t id, int32_t *out, int32_t n_experts) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (id < 0 || id >= (int32_t) g_all.size()) return fail(E_INVALID, "entry_table: bad id %d", id);
    const Entry *e = g_all[id];
    if (!out || n_experts < e->n_experts) return fail(E_INVALID, "entry_table: buffer too small");
    for (int i = 0; i < e->n_experts; ++i) {
        const uint64_t v = e->h_tbl[i];
        if (v & 1ull) {
            if (v != host_entry(e, i)) return fail(E_STATE, "entry_table: corrupt host entry %d", i);
            out[i] = -1;
        } else {
            const uint64_t off = v - (uint64_t) (uintptr_t) e->pool;
            if (!e->pool || off % e->expert_bytes || off / e->expert_bytes >= (uint64_t) e->n_slots)
                return fail(E_STATE, "entry_table: corrupt pool entry %d", i);
            out[i] = (int32_t) (off / e->expert_bytes);
        }
    }
    return 0;
}

int ggml_hip_moe_cache_entry_device(int32_t id, void **d_tbl, void **d_stamps, void **pool) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (id < 0 || id >= (int32_t) g_all.size()) return fail(E_INVALID, "entry_device: bad id %d", id);
    const Entry *e = g_all[id];
    if (d_tbl) *d_tbl = e->d_tbl;
    if (d_stamps) *d_stamps = e->d_stamps;
    if (pool) *pool = e->pool;
    return 0;
}

int ggml_hip_moe_cache_device_globals(void **d_stats, void **d_clock) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (d_stats) *d_stats = g_d_stats;
    if (d_clock) *d_clock = g_d_clock;
    return 0;
}

int ggml_hip_moe_cache_stats_snapshot(uint32_t *out, int32_t n_words, void *stream) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!out || n_words < 0 || n_words > STATS_WORDS) return fail(E_INVALID, "stats_snapshot: bad buffer");
    if (!g_d_stats) return fail(E_STATE, "stats_snapshot: nothing registered");
    int rc;
    if ((rc = dev()->copy_d2h(out, g_d_stats, sizeof(uint32_t) * n_words, stream))) return dev_err(rc, "stats snapshot");
    if ((rc = dev()->sync(stream))) return dev_err(rc, "stream sync");
    return 0;
}

int ggml_hip_moe_cache_stamps_snapshot(int32_t id, uint32_t *out, int32_t n, void *stream) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (id < 0 || id >= (int32_t) g_all.size()) return fail(E_INVALID, "stamps_snapshot: bad id %d", id);
    const Entry *e = g_all[id];
    if (!out || n < e->n_experts) return fail(E_INVALID, "stamps_snapshot: buffer too small");
    int rc;
    if ((rc = dev()->copy_d2h(out, e->d_stamps, sizeof(uint32_t) * e->n_experts, stream))) return dev_err(rc, "stamps snapshot");
    if ((rc = dev()->sync(stream))) return dev_err(rc, "stream sync");
    return 0;
}

int ggml_hip_moe_cache_totals(ggml_hip_moe_totals *out) {
    if (!out) return fail(E_INVALID, "totals: null");
    std::lock_guard<std::mutex> lock(g_mutex);
    *out = g_totals;
    out->clock = g_h_clock;
    out->admission_size = (uint32_t) g_admission.size();
    return 0;
}

int ggml_hip_moe_cache_reset(void) {
    std::lock_guard<std::mutex> lock(g_mutex);
    int first_rc = 0;
    auto note = [&](int rc) { if (rc && !first_rc) first_rc = rc; };
    // pending promotion copies write into the pools freed below
    if (g_copy_pending) note(dev()->event_sync(g_copy_event));
    g_copy_pending = false;
    if (g_copy_event) note(dev()->event_destroy(g_copy_event));
    if (g_order_event) note(dev()->event_destroy(g_order_event));
    if (g_copy_stream) note(dev()->stream_destroy(g_copy_stream));
    g_copy_event = g_order_event = g_copy_stream = nullptr;
    for (Entry *e : g_all) {
        for (uint64_t *&st : e->h_tbl_stage)
            if (st) note(dev()->free_host(st));
        if (e->pool) note(dev()->free_dev(e->pool));
        if (e->d_tbl) note(dev()->free_dev(e->d_tbl));
        if (e->d_stamps && !e->stamps_in_arena) note(dev()->free_dev(e->d_stamps));
        delete e;
    }
    g_all.clear();
    g_by_data.clear();
    for (auto &kv : g_resident) {
        if (kv.second->d_tbl) note(dev()->free_dev(kv.second->d_tbl));
        delete kv.second;
    }
    g_resident.clear();
    if (g_d_stats) note(dev()->free_dev(g_d_stats));
    if (g_d_clock) note(dev()->free_dev(g_d_clock));
    if (g_h_stats) note(dev()->free_host(g_h_stats));
    if (g_d_stamps_arena) note(dev()->free_dev(g_d_stamps_arena));
    if (g_h_stamps_arena) note(dev()->free_host(g_h_stamps_arena));
    g_d_stats = g_d_clock = g_h_stats = g_d_stamps_arena = g_h_stamps_arena = nullptr;
    g_stamps_used = 0;
    g_h_clock = 0;
    g_used = 0;
    g_admission.clear();
    g_seed.clear();
    g_seed_loaded = false;
    g_totals = {};
    {
        std::lock_guard<std::mutex> l2(g_ptr_mutex);
        g_ptr_kind.clear();
    }
    if (first_rc) return dev_err(first_rc, "reset free");
    return 0;
}

// ---------------------------------------------------------------------------
// routing trace (patches/trace-hook/ggml-cpu.c:1597-1617)
// ---------------------------------------------------------------------------

int ggml_hip_moe_trace_append(const char *path, const char *name, const int32_t *ids, int64_t n_used, int64_t n_tok,
                              int64_t n_exp) {
    if (!path) path = env2("GGML_HIP_MOE_TRACE", "GGML_MOE_TRACE");
    if (!path || !*path) return 0;
    if (n_used < 0 || n_tok < 0 || n_exp < 0 || n_used > 0xFFFFFFFFll || n_tok > 0xFFFFFFFFll ||
        n_exp > 0xFFFFFFFFll || (n_used * n_tok > 0 && !ids))
        return fail(E_INVALID, "trace_append: bad record (n_used %lld, n_tok %lld, n_exp %lld)", (long long) n_used,
                    (long long) n_tok, (long long) n_exp);
    // the hook copies the name into a zeroed 128-byte buffer with strncpy(.., 120)
    char nbuf[128] = {0};
    strncpy(nbuf, name ? name : "?", 120);
    const uint32_t hdr[4] = {(uint32_t) strlen(nbuf), (uint32_t) n_used, (uint32_t) n_tok, (uint32_t) n_exp};
    std::lock_guard<std::mutex> lock(g_trace_mutex);
    FILE *&f = g_trace_files[path];
    if (!f && !(f = fopen(path, "ab"))) {
        g_trace_files.erase(path);
        return fail(E_INVALID, "trace_append: cannot open %s: %s", path, strerror(errno));
    }
    const size_t n_ids = (size_t) (n_used * n_tok);
    if (fwrite(hdr, sizeof(uint32_t), 4, f) != 4 || fwrite(nbuf, 1, hdr[0], f) != hdr[0] ||
        (n_ids && fwrite(ids, sizeof(int32_t), n_ids, f) != n_ids))
        return fail(E_INVALID, "trace_append: write to %s failed", path);
    return 0;
}

int ggml_hip_moe_trace_close(void) {
    std::lock_guard<std::mutex> lock(g_trace_mutex);
    int rc = 0;
    for (auto &kv : g_trace_files)
        if (kv.second && fclose(kv.second) != 0 && !rc) rc = fail(E_INVALID, "trace_close: %s", kv.first.c_str());
    g_trace_files.clear();
    return rc;
}

int ggml_hip_moe_fusion_detect(const ggml_hip_moe_node *nodes, int32_t n_nodes, int32_t i_up, ggml_hip_moe_fusion *fusion,
                               ggml_hip_moe_tensor *gate_host, int32_t *has_gate_host, int32_t *covered, int32_t *out_node) {
    if (!nodes || n_nodes <= 0 || !fusion || !gate_host || !has_gate_host || !covered || !out_node)
        return fail(E_INVALID, "fusion_detect: null argument");
    if (i_up < 0 || i_up >= n_nodes || nodes[i_up].op != OP_MUL_MAT_ID)
        return fail(E_INVALID, "fusion_detect: node %d is not a MUL_MAT_ID", i_up);
    for (int k = 0; k < n_nodes; ++k)
        for (int s = 0; s < 3; ++s)
            if (nodes[k].src[s] >= n_nodes) return fail(E_INVALID, "fusion_detect: node %d source %d out of range", k, s);
    const Graph g(nodes, n_nodes);
    memset(fusion, 0, sizeof(*fusion));
    memset(gate_host, 0, sizeof(*gate_host));
    for (int k = 0; k < n_nodes; ++k) covered[k] = 0;
    fusion->glu_op = GGML_HIP_MOE_GLU_SWIGLU;
    fusion->shared_type = -1;
    *has_gate_host = 0;
    *out_node = i_up;
    covered[i_up] = 1;

    // up path, then the GLU that consumes it
    std::vector<int> up_path;
    const float *x_bias = nullptr, *x_scale = nullptr;
    int64_t x_bias_stride = 0;
    const int up_end = follow_expert_path(g, i_up, &x_bias, &x_bias_stride, &x_scale, up_path);
    const int glu = g.sole[up_end];
    int gate_mm = -1, gate_end = -1;
    std::vector<int> gate_path;
    const float *g_bias = nullptr, *g_scale = nullptr;
    int64_t g_bias_stride = 0;
    if (glu >= 0 && nodes[glu].op == OP_GLU) {
        const bool sw = nodes[glu].glu_swapped != 0;
        const int up_slot = sw ? 0 : 1, gate_slot = sw ? 1 : 0;
        if (nodes[glu].src[up_slot] == up_end) {
            // the gate operand must be the end of a matching gate MUL_MAT_ID path
            const int ge = nodes[glu].src[gate_slot];
            int cand = ge;
            // walk back through at most an ADD_ID and a MUL to the gate MUL_MAT_ID
            for (int hop = 0; hop < 2 && cand >= 0 && nodes[cand].op != OP_MUL_MAT_ID; ++hop) cand = nodes[cand].src[0];
            if (cand >= 0 && cand != i_up && nodes[cand].op == OP_MUL_MAT_ID && g.same_src(cand, 1, i_up, 1) &&
                g.same_src(cand, 2, i_up, 2)) {
                const ggml_hip_moe_tensor &wu = g.src_tensor(i_up, 0), &wg = g.src_tensor(cand, 0);
                const bool same_shape = wu.type == wg.type && !memcmp(wu.ne, wg.ne, sizeof(wu.ne)) && wu.nb[2] == wg.nb[2] &&
                                        wu.nb[1] == wg.nb[1];
                if (same_shape && g.uses[cand] == 1) {
                    gate_end = follow_expert_path(g, cand, &g_bias, &g_bias_stride, &g_scale, gate_path);
                    if (gate_end == ge) gate_mm = cand;
                }
            }
        }
        // every absorbed intermediate feeds only the next node of its path
        bool ok = gate_mm >= 0;
        for (size_t k = 0; ok && k + 1 < up_path.size(); ++k) ok = g.sole[up_path[k]] == up_path[k + 1];
        for (size_t k = 0; ok && k + 1 < gate_path.size(); ++k) ok = g.sole[gate_path[k]] == gate_path[k + 1];
        ok = ok && g.sole[up_end] == glu && g.sole[gate_end] == glu;
        if (x_bias && g_bias && x_bias_stride != g_bias_stride) ok = false;
        const int op = ok ? nodes[glu].glu_op : -1;
        if (op < GGML_HIP_MOE_GLU_REGLU || op > GGML_HIP_MOE_GLU_SWIGLU_CLAMP) ok = false;
        // the gate goes to the kernel as a host tensor for the cache path (registered with its own
        // table when host-resident), else as device memory that the kernel reads directly
        const bool cache_up = ok && wants_impl(&g.src_tensor(i_up, 0));
        if (ok && !cache_up && ptr_kind_cached(g.src_tensor(gate_mm, 0).data) != PTR_DEVICE) ok = false;
        if (ok) {
            fusion->glu_op = op;
            fusion->glu_limit = nodes[glu].glu_limit;
            fusion->x_bias = x_bias;
            fusion->x_scale = x_scale;
            fusion->gate_bias = g_bias;
            fusion->gate_scale = g_scale;
            fusion->bias_stride = x_bias ? x_bias_stride : g_bias_stride;
            if (cache_up) {
                *gate_host = g.src_tensor(gate_mm, 0);
                *has_gate_host = 1;
            } else {
                fusion->gate = g.src_tensor(gate_mm, 0).data;
            }
            for (int k : up_path) covered[k] = 1;
            for (int k : gate_path) covered[k] = 1;
            covered[glu] = 1;
            *out_node = glu;
        }
    }
    if (*out_node == i_up) {
        // no gate: the up path's bias and scale alone still fuse into the plain GEMV
        bool ok = true;
        for (size_t k = 0; ok && k + 1 < up_path.size(); ++k) ok = g.sole[up_path[k]] == up_path[k + 1];
        if (ok && up_path.size() > 1) {
            fusion->x_bias = x_bias;
            fusion->x_scale = x_scale;
            fusion->bias_stride = x_bias_stride;
            for (int k : up_path) covered[k] = 1;
            *out_node = up_end;
        }
    }

    // shared expert on the same activations: MUL_MAT(sh_up, x), MUL_MAT(sh_gate, x), GLU(sh_gate, sh_up)
    const bool routed_glu = *out_node != i_up && nodes[*out_node].op == OP_GLU;
    {
        const ggml_hip_moe_tensor &x = g.src_tensor(i_up, 1);
        const int64_t rows = nodes[i_up].t.ne[0], K = g.src_tensor(i_up, 0).ne[0];
        for (int k = 0; k < n_nodes; ++k) {
            if (nodes[k].op != OP_GLU || covered[k]) continue;
            const bool sw = nodes[k].glu_swapped != 0;
            const int su = nodes[k].src[sw ? 0 : 1], sg = nodes[k].src[sw ? 1 : 0];
            if (su < 0 || sg < 0 || nodes[su].op != OP_MUL_MAT || nodes[sg].op != OP_MUL_MAT) continue;
            if (g.uses[su] != 1 || g.uses[sg] != 1) continue;
            const ggml_hip_moe_tensor &xu = g.src_tensor(su, 1), &xg = g.src_tensor(sg, 1);
            if (xu.data != x.data || xg.data != x.data) continue;     // the routed experts' input rows
            const ggml_hip_moe_tensor &wu = g.src_tensor(su, 0), &wg = g.src_tensor(sg, 0);
            if (wu.type != wg.type || !type_supported(wu.type) || wu.ne[0] != K || wu.ne[1] != rows ||
                memcmp(wu.ne, wg.ne, sizeof(wu.ne)) || wu.ne[2] != 1)
                continue;
            if (routed_glu && nodes[k].glu_op != fusion->glu_op) continue;          // one GLU op per launch
            if (ptr_kind_cached(wu.data) != PTR_DEVICE || ptr_kind_cached(wg.data) != PTR_DEVICE) continue;
            const ggml_hip_moe_tensor &out = nodes[k].t;
            if (out.type != 0 || out.nb[0] != 4 || out.nb[1] % 4) continue;
            fusion->shared_up = wu.data;
            fusion->shared_gate = wg.data;
            fusion->shared_type = wu.type;
            fusion->shared_dst = (float *) out.data;
            fusion->shared_stride_col_dst = (int64_t) (out.nb[1] / 4);
            if (!routed_glu) {
                fusion->glu_op = nodes[k].glu_op;
                fusion->glu_limit = nodes[k].glu_limit;
            }
            covered[su] = covered[sg] = covered[k] = 1;
            break;
        }
    }
    int n = 0;
    for (int k = 0; k < n_nodes; ++k) n += covered[k];
    return n;
}

int ggml_hip_moe_check_status(void *stream) {
    uint32_t *status = nullptr;
    int rc;
    if ((rc = dev()->status_address(&status))) return dev_err(rc, "status word lookup");
    uint32_t *h = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        if ((rc = init_globals_locked(stream))) return rc;
        h = &g_h_stats[STATS_WORDS + 1];                  // pinned staging word
        if ((rc = dev()->copy_d2h(h, status, sizeof(uint32_t), stream))) return dev_err(rc, "status readback");
        if ((rc = dev()->sync(stream))) return dev_err(rc, "stream sync");
        const uint32_t v = *h;
        if (v == 0) return 0;
        if ((rc = dev()->memset_dev(status, 0, sizeof(uint32_t), stream))) return dev_err(rc, "status clear");
        if ((rc = dev()->sync(stream))) return dev_err(rc, "stream sync");
        return fail(E_TIMEOUT, "moe-ffn: a bounded in-kernel wait gave up (status 0x%x): the outputs of the fused "
                    "gate/up launches since the last check are not valid", v);
    }
}

int ggml_hip_moe_debug_set_spin_limit(int64_t n) {
    const int32_t v = n < 0 ? DEFAULT_SPIN_LIMIT : (int32_t) std::min<int64_t>(n, INT32_MAX);
    __atomic_store_n(&g_spin_limit, v, __ATOMIC_RELAXED);
    return 0;
}

const char *ggml_hip_moe_last_error(void) { return t_last_error.c_str(); }

const char *ggml_hip_moe_version(void) { return "ggml-hip-moe-cache 0.1 (gfx950)"; }

}  // extern "C"
