// mh_runtime.hip — libmidge_hip runtime: init/shutdown, errors, the
// registered-region table (host mmap range -> HBM copy at identical offsets),
// device allocations, scratch and pointer resolution.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <map>
#include <string>
#include <vector>

#include "mh_internal.h"

namespace mh {
namespace {

thread_local char g_err[1024];

struct Region {
    const uint8_t *host;
    uint64_t bytes;
    uint8_t *dev;
};

// Live objects holding device memory outside the tables below (decode
// plans): mh_shutdown releases their memory through the callback.
struct Owner {
    void *key;
    void (*release)(void *);
};

struct State {
    bool inited = false;
    int device = -1;
    int cus = 0;
    hipStream_t own = nullptr;
    hipStream_t cur = nullptr;
    // registered regions, keyed by host base and by device base (lookups
    // are O(log n): a lazily registered model holds tens of thousands)
    std::map<uintptr_t, Region> regions;
    std::map<uintptr_t, uint64_t> region_dev;   // device base -> bytes
    std::map<uintptr_t, uint64_t> allocs;   // device base -> bytes (mh_alloc)
    std::vector<Owner> owners;
    uint64_t allocated = 0;
    uint64_t cap = 0;                       // 0 = no cap
    void *scratch[S_COUNT] = {};
    uint64_t scratch_bytes[S_COUNT] = {};
    unsigned *flag_host[F_COUNT] = {};      // async_flag: host-mapped pinned words
    unsigned *flag_dev[F_COUNT] = {};
};

State g;
uint64_t g_epoch = 0;   // successful mh_init calls

// Path switches (sw, mh_set_switch), read from the environment by mh_init.
const char *const kSwitchNames[SW_COUNT] = {"NO_MFMA", "NO_FUSED", "ATTN_SPLIT", "COOP", "Q8_NO_ROWS", "BATCH_GEMV", "SPLIT_ROUTE"};
bool g_sw[SW_COUNT] = {};
void read_switches() {
    char name[64];
    for (int i = 0; i < SW_COUNT; i++) {
        snprintf(name, sizeof(name), "MIDGE_HIP_%s", kSwitchNames[i]);
        const char *v = getenv(name);
        g_sw[i] = v && v[0] && v[0] != '0';
    }
}

// Host-mapped error flags of asynchronous work (checked by mh_sync).
std::vector<std::pair<unsigned *, const char *>> g_async;

// Kernel timing records (mh_profile_*).
struct ProfRec {
    const char *name;
    hipEvent_t start, stop;
};
bool g_prof = false;
std::vector<ProfRec> g_prof_pending;
std::map<std::string, std::pair<double, uint64_t>> g_prof_done;   // name -> (total ms, launches)

uint64_t env_cap() {
    const char *s = getenv("MIDGE_HIP_MAX_BYTES");
    if (!s || !*s) return 0;
    return strtoull(s, nullptr, 10);
}

int dev_malloc(void **p, uint64_t bytes, const char *what) {
    g.cap = env_cap();
    if (g.cap && g.allocated + bytes > g.cap)
        return fail(MH_E_NOMEM, "%s: %llu bytes would exceed MIDGE_HIP_MAX_BYTES=%llu",
                    what, (unsigned long long)bytes, (unsigned long long)g.cap);
    hipError_t e = hipMalloc(p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(MH_E_NOMEM, "%s: hipMalloc(%llu) failed: %s", what,
                    (unsigned long long)bytes, hipGetErrorString(e));
    }
    g.allocated += bytes;
    return MH_OK;
}

}  // namespace

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_err[0] = 0; }

int dev_alloc(void **p, uint64_t bytes, const char *what) { return dev_malloc(p, bytes, what); }

void dev_release(void *p, uint64_t bytes) {
    if (!p) return;
    (void)hipFree(p);
    g.allocated = g.allocated >= bytes ? g.allocated - bytes : 0;
}

void register_owner(void *key, void (*release)(void *)) { g.owners.push_back(Owner{key, release}); }

void unregister_owner(void *key) {
    for (size_t i = 0; i < g.owners.size(); i++)
        if (g.owners[i].key == key) {
            g.owners.erase(g.owners.begin() + (long)i);
            return;
        }
}

void watch_async_error(unsigned *flag, const char *msg) { g_async.push_back({flag, msg}); }

int sync_checked(hipStream_t s) {
    MH_HIP(hipStreamSynchronize(s));
    for (auto &a : g_async)
        if (*(volatile unsigned *)a.first) {
            *(volatile unsigned *)a.first = 0;
            return fail(MH_E_HIP, "%s", a.second);
        }
    return MH_OK;
}

void unwatch_async_error(unsigned *flag) {
    for (size_t i = 0; i < g_async.size(); i++)
        if (g_async[i].first == flag) {
            g_async.erase(g_async.begin() + (long)i);
            return;
        }
}

bool profiling() { return g_prof; }

void prof_begin(const char *name, hipStream_t s) {
    ProfRec r{name, nullptr, nullptr};
    if (hipEventCreate(&r.start) != hipSuccess || hipEventCreate(&r.stop) != hipSuccess) {
        (void)hipGetLastError();
        return;
    }
    (void)hipEventRecord(r.start, s);
    g_prof_pending.push_back(r);
}

void prof_end(hipStream_t s) {
    if (!g_prof_pending.empty() && g_prof_pending.back().stop) (void)hipEventRecord(g_prof_pending.back().stop, s);
}

void prof_add(const char *name, double ms) {
    auto &acc = g_prof_done[name];
    acc.first += ms;
    acc.second += 1;
}

static int prof_collect() {
    for (ProfRec &r : g_prof_pending) {
        MH_HIP(hipEventSynchronize(r.stop));
        float ms = 0.f;
        MH_HIP(hipEventElapsedTime(&ms, r.start, r.stop));
        auto &acc = g_prof_done[r.name];
        acc.first += ms;
        acc.second += 1;
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    g_prof_pending.clear();
    return MH_OK;
}

int hip_check(hipError_t e, const char *what) {
    if (e == hipSuccess) return MH_OK;
    (void)hipGetLastError();
    return fail(MH_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool initialised() { return g.inited; }

int require_init() {
    if (!g.inited) return fail(MH_E_NOINIT, "mh_init() has not succeeded");
    return MH_OK;
}

hipStream_t stream() { return g.cur; }
int device_cus() { return g.cus; }
int current_device() { return g.device; }

int wt_bytes(int dt, int64_t rows, int64_t cols, uint64_t *db, uint64_t *sb) {
    if (rows < 0 || cols < 0) return fail(MH_E_ARG, "negative shape %lld x %lld", (long long)rows, (long long)cols);
    switch (dt) {
    case MH_DT_F32: *db = (uint64_t)rows * cols * 4; *sb = 0; return MH_OK;
    case MH_DT_Q8R: *db = (uint64_t)rows * cols; *sb = (uint64_t)rows * 4; return MH_OK;
    case MH_DT_Q4G32:
    case MH_DT_MXFP4:
        if (cols % 32) return fail(MH_E_ARG, "4-bit g32 tensor needs cols %% 32 == 0 (cols=%lld)", (long long)cols);
        *db = (uint64_t)rows * cols / 2;
        *sb = (uint64_t)rows * (cols / 32) * 2;
        return MH_OK;
    }
    return fail(MH_E_DTYPE, "unknown dtype %d", dt);
}

static uint64_t span_of(uint64_t bytes) { return bytes; }
static uint64_t span_of(const Region &r) { return r.bytes; }

// The entry of a base -> bytes map whose range holds address a, or end().
template <class M>
static typename M::const_iterator containing(const M &m, uintptr_t a) {
    auto it = m.upper_bound(a);
    if (it == m.begin()) return m.end();
    --it;
    return a < it->first + span_of(it->second) ? it : m.end();
}

// Device allocation containing [p, p+bytes), via our own tables first and
// the HIP runtime otherwise.
static int check_device_range(const void *p, uint64_t bytes, const char *what) {
    uintptr_t a = (uintptr_t)p;
    auto it = containing(g.allocs, a);
    if (it != g.allocs.end()) {
        if (a + bytes > it->first + it->second)
            return fail(MH_E_RANGE, "%s: %llu bytes at %p overrun its allocation", what, (unsigned long long)bytes, p);
        return MH_OK;
    }
    auto rd = containing(g.region_dev, a);
    if (rd != g.region_dev.end()) {
        if (a + bytes > rd->first + rd->second)
            return fail(MH_E_RANGE, "%s: %llu bytes at %p overrun the region", what, (unsigned long long)bytes, p);
        return MH_OK;
    }
    hipPointerAttribute_t attr;
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(MH_E_UNREGISTERED, "%s: %p is neither in a registered region nor device memory", what, p);
    }
    if (attr.type != hipMemoryTypeDevice)
        return fail(MH_E_UNREGISTERED, "%s: %p is not device memory", what, p);
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) != hipSuccess) {
        (void)hipGetLastError();
        return fail(MH_E_UNREGISTERED, "%s: cannot size the allocation of %p", what, p);
    }
    if (a + bytes > (uintptr_t)base + size)
        return fail(MH_E_RANGE, "%s: %llu bytes at %p overrun its allocation", what,
                    (unsigned long long)bytes, p);
    return MH_OK;
}

int resolve_weight(const void *p, uint64_t bytes, const void **dev, const char *what) {
    if (!p) return fail(MH_E_ARG, "%s: NULL pointer", what);
    uintptr_t a = (uintptr_t)p;
    auto it = containing(g.regions, a);
    if (it != g.regions.end()) {
        const Region &r = it->second;
        if (a + bytes > it->first + r.bytes)
            return fail(MH_E_RANGE, "%s: %llu bytes at %p run past the registered region", what,
                        (unsigned long long)bytes, p);
        *dev = r.dev + (a - it->first);
        return MH_OK;
    }
    MH_TRY(check_device_range(p, bytes, what));
    *dev = p;
    return MH_OK;
}

int resolve_dev(const void *p, uint64_t bytes, const char *what) {
    if (!p) return fail(MH_E_ARG, "%s: NULL pointer", what);
    if (containing(g.regions, (uintptr_t)p) != g.regions.end())
        return fail(MH_E_ARG, "%s: %p is a registered host pointer; _dev calls need device memory", what, p);
    return check_device_range(p, bytes, what);
}

int resolve_wt(const mh_wt *t, DevWT *out, const char *what) {
    if (!t) return fail(MH_E_ARG, "%s: NULL tensor", what);
    uint64_t db, sb;
    MH_TRY(wt_bytes(t->dt, t->rows, t->cols, &db, &sb));
    if (t->rows < 1 || t->cols < 1) return fail(MH_E_ARG, "%s: empty tensor %lld x %lld", what,
                                                (long long)t->rows, (long long)t->cols);
    out->dt = t->dt;
    out->rows = t->rows;
    out->cols = t->cols;
    const void *d = nullptr, *s = nullptr;
    MH_TRY(resolve_weight(t->data, db, &d, what));
    if (sb) MH_TRY(resolve_weight(t->scales, sb, &s, what));
    out->data = (const uint8_t *)d;
    out->scales = s;
    return MH_OK;
}

uint64_t init_epoch() { return g_epoch; }

bool sw(Switch s) { return g_sw[s]; }

int async_flag(AsyncFlag id, const char *msg, unsigned **dev) {
    if (!g.flag_host[id]) {
        unsigned *h = nullptr, *d = nullptr;
        MH_HIP(hipHostMalloc((void **)&h, sizeof(unsigned), hipHostMallocMapped));
        *h = 0;
        const hipError_t e = hipHostGetDevicePointer((void **)&d, h, 0);
        if (e != hipSuccess) {
            (void)hipHostFree(h);
            return hip_check(e, "hipHostGetDevicePointer (error flag)");
        }
        g.flag_host[id] = h;
        g.flag_dev[id] = d;
        watch_async_error(h, msg);
    }
    *dev = g.flag_dev[id];
    return MH_OK;
}

int scratch(Scratch slot, uint64_t bytes, void **p, bool *fresh) {
    if (fresh) *fresh = false;
    if (bytes <= g.scratch_bytes[slot] && g.scratch[slot]) {
        *p = g.scratch[slot];
        return MH_OK;
    }
    if (fresh) *fresh = true;
    if (g.scratch[slot]) {
        MH_HIP(hipStreamSynchronize(g.cur));
        MH_HIP(hipFree(g.scratch[slot]));
        g.allocated -= g.scratch_bytes[slot];
        g.scratch[slot] = nullptr;
        g.scratch_bytes[slot] = 0;
    }
    uint64_t want = bytes < 4096 ? 4096 : bytes + bytes / 4;
    MH_TRY(dev_malloc(&g.scratch[slot], want, "scratch"));
    g.scratch_bytes[slot] = want;
    *p = g.scratch[slot];
    return MH_OK;
}

}  // namespace mh

using namespace mh;

extern "C" {

const char *mh_last_error(void) { return g_err; }

int mh_init(int device) {
    clear_error();
    if (g.inited) {
        if (device != g.device) return fail(MH_E_ARG, "already initialised on device %d", g.device);
        return MH_OK;
    }
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
        (void)hipGetLastError();
        return fail(MH_E_HIP, "no HIP device available (%s)", hipGetErrorString(e));
    }
    if (device < 0 || device >= n) return fail(MH_E_ARG, "device %d out of range (%d devices)", device, n);
    MH_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    MH_HIP(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(MH_E_UNSUPPORTED, "device %d is %s; libmidge_hip is built for gfx950 only", device,
                    prop.gcnArchName);
    MH_HIP(hipStreamCreateWithFlags(&g.own, hipStreamNonBlocking));
    g.cur = g.own;
    g.device = device;
    g.cus = prop.multiProcessorCount;
    g.cap = env_cap();
    g.inited = true;
    ++g_epoch;
    read_switches();
    const int rc = sample_static_setup(device);
    if (rc) {
        (void)hipStreamDestroy(g.own);
        g = State();
        return rc;
    }
    return MH_OK;
}

int mh_shutdown(void) {
    clear_error();
    if (!g.inited) return MH_OK;
    (void)hipStreamSynchronize(g.cur);
    // live plans first (their release callbacks unregister them)
    while (!g.owners.empty()) {
        const Owner o = g.owners.back();
        g.owners.pop_back();
        o.release(o.key);
    }
    g_async.clear();
    for (int i = 0; i < F_COUNT; i++)
        if (g.flag_host[i]) (void)hipHostFree(g.flag_host[i]);
    for (auto &r : g.regions) (void)hipFree(r.second.dev);
    g.regions.clear();
    g.region_dev.clear();
    for (auto &a : g.allocs) (void)hipFree((void *)a.first);
    g.allocs.clear();
    for (int i = 0; i < S_COUNT; i++) {
        if (g.scratch[i]) (void)hipFree(g.scratch[i]);
        g.scratch[i] = nullptr;
        g.scratch_bytes[i] = 0;
    }
    (void)hipStreamDestroy(g.own);
    g = State();
    return MH_OK;
}

int mh_profile_enable(int on) {
    clear_error();
    MH_TRY(require_init());
    if (!on) MH_TRY(prof_collect());
    g_prof = on != 0;
    return MH_OK;
}

int mh_profile_reset(void) {
    clear_error();
    MH_TRY(require_init());
    MH_TRY(prof_collect());
    g_prof_done.clear();
    return MH_OK;
}

int mh_profile_query(const char *name, double *total_ms, uint64_t *launches) {
    clear_error();
    if (!name || !total_ms || !launches) return fail(MH_E_ARG, "mh_profile_query: NULL argument");
    MH_TRY(require_init());
    MH_TRY(prof_collect());
    auto it = g_prof_done.find(name);
    *total_ms = it == g_prof_done.end() ? 0.0 : it->second.first;
    *launches = it == g_prof_done.end() ? 0 : it->second.second;
    return MH_OK;
}

int mh_set_switch(const char *name, int on) {
    clear_error();
    if (!name) return fail(MH_E_ARG, "mh_set_switch: NULL name");
    for (int i = 0; i < SW_COUNT; i++)
        if (strcmp(name, kSwitchNames[i]) == 0) {
            g_sw[i] = on != 0;
            return MH_OK;
        }
    return fail(MH_E_ARG, "mh_set_switch: unknown switch '%s'", name);
}

int mh_set_stream(void *s) {
    clear_error();
    MH_TRY(require_init());
    g.cur = s ? (hipStream_t)s : g.own;
    return MH_OK;
}

void *mh_get_stream(void) { return (void *)g.cur; }

int mh_sync(void) {
    clear_error();
    MH_TRY(require_init());
    return sync_checked(g.cur);
}

int mh_register_region(const void *host_base, uint64_t bytes, void **dev_base) {
    clear_error();
    MH_TRY(require_init());
    if (!host_base || !bytes || !dev_base) return fail(MH_E_ARG, "register_region: NULL base/out or zero size");
    uintptr_t a = (uintptr_t)host_base;
    if (bytes > UINTPTR_MAX - a) return fail(MH_E_ARG, "register_region: [%p, +%llu) wraps the address space", host_base,
                                             (unsigned long long)bytes);
    {
        // the nearest region at or below a, and the first one above it
        auto hi = g.regions.upper_bound(a);
        bool overlap = hi != g.regions.end() && hi->first < a + bytes;
        if (hi != g.regions.begin()) {
            auto lo = std::prev(hi);
            overlap = overlap || a < lo->first + lo->second.bytes;
        }
        if (overlap)
            return fail(MH_E_ARG, "register_region: [%p, +%llu) overlaps a registered region", host_base,
                        (unsigned long long)bytes);
    }
    void *d = nullptr;
    MH_TRY(dev_malloc(&d, bytes, "register_region"));
    hipError_t e = hipMemcpy(d, host_base, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
        g.allocated -= bytes;
        return hip_check(e, "register_region upload");
    }
    g.regions[a] = Region{(const uint8_t *)host_base, bytes, (uint8_t *)d};
    g.region_dev[(uintptr_t)d] = bytes;
    *dev_base = d;
    return MH_OK;
}

int mh_unregister_region(const void *host_base) {
    clear_error();
    MH_TRY(require_init());
    auto it = g.regions.find((uintptr_t)host_base);
    if (it == g.regions.end()) return fail(MH_E_ARG, "unregister_region: %p is not a registered base", host_base);
    MH_HIP(hipStreamSynchronize(g.cur));
    MH_HIP(hipFree(it->second.dev));
    g.allocated -= it->second.bytes;
    g.region_dev.erase((uintptr_t)it->second.dev);
    g.regions.erase(it);
    return MH_OK;
}

int mh_alloc(uint64_t bytes, void **dev) {
    clear_error();
    MH_TRY(require_init());
    if (!dev) return fail(MH_E_ARG, "mh_alloc: NULL out pointer");
    void *p = nullptr;
    MH_TRY(dev_malloc(&p, bytes, "mh_alloc"));
    g.allocs[(uintptr_t)p] = bytes ? bytes : 1;
    *dev = p;
    return MH_OK;
}

int mh_free(void *dev) {
    clear_error();
    MH_TRY(require_init());
    auto it = g.allocs.find((uintptr_t)dev);
    if (it == g.allocs.end()) return fail(MH_E_ARG, "mh_free: %p was not returned by mh_alloc", dev);
    MH_HIP(hipStreamSynchronize(g.cur));
    MH_HIP(hipFree(dev));
    g.allocated -= it->second;
    g.allocs.erase(it);
    return MH_OK;
}

int mh_h2d(void *dst, const void *src, uint64_t bytes) {
    clear_error();
    MH_TRY(require_init());
    if (!src) return fail(MH_E_ARG, "mh_h2d: NULL source");
    if (!bytes) return MH_OK;
    MH_TRY(resolve_dev(dst, bytes, "mh_h2d destination"));
    MH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g.cur));
    MH_HIP(hipStreamSynchronize(g.cur));
    return MH_OK;
}

int mh_d2h(void *dst, const void *src, uint64_t bytes) {
    clear_error();
    MH_TRY(require_init());
    if (!dst) return fail(MH_E_ARG, "mh_d2h: NULL destination");
    if (!bytes) return MH_OK;
    MH_TRY(resolve_dev(src, bytes, "mh_d2h source"));
    MH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g.cur));
    MH_HIP(hipStreamSynchronize(g.cur));
    return MH_OK;
}

}  // extern "C"
