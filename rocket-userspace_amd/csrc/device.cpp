// device.cpp — the HIP device shim behind rocket_npu.h: handle table, buffer objects,
// bounded waits, operand staging and the dispatch counters.
//
// Replaces the DRM-accel shim of reference src/rocket_npu.c (open :470-525, BO
// alloc/free :538-590, PREP with deadline :612-725, FINI :727-739, submit :745-892,
// counters :121-128).
#include "internal.h"

#include <errno.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <thread>

namespace rk {

namespace {

constexpr int kMaxHandles = 256;
std::mutex g_table_mu;
std::shared_ptr<Handle> g_table[kMaxHandles];

// Dispatch counters: relaxed atomics (calls on different handles run on different threads).
std::atomic<uint64_t> g_submits{0}, g_tasks{0};
std::atomic<long> g_busy_poll_us{-1};    // -1: not yet read from ROCKET_BUSY_POLL

long wait_ms()
{
    static std::atomic<long> ms{-1};
    long v = ms.load(std::memory_order_relaxed);
    if (v < 0) {
        const char *e = getenv("ROCKET_WAIT_MS");
        v = e ? atol(e) : 8000;
        if (v < 1) v = 8000;
        ms.store(v, std::memory_order_relaxed);
    }
    return v;
}

long busy_poll_us()
{
    long v = g_busy_poll_us.load(std::memory_order_relaxed);
    if (v < 0) {
        const char *e = getenv("ROCKET_BUSY_POLL");
        v = e ? atol(e) : 200;
        if (v < 0) v = 0;
        g_busy_poll_us.store(v, std::memory_order_relaxed);
    }
    return v;
}

// ROCKET_MM_PROFILE (read once, as the reference's knob, rocket_matmul.c:71-125): every
// staged call adds its phase times to process totals, printed as one INFO line at exit.
bool mm_profile()
{
    static const bool on = getenv("ROCKET_MM_PROFILE") != nullptr;
    return on;
}

struct PhaseTotals { double stage = 0, submit = 0, wait = 0, read = 0; long calls = 0; };
std::mutex g_prof_mu;
PhaseTotals g_prof;
bool g_prof_armed = false;

void prof_dump()
{
    std::lock_guard<std::mutex> g(g_prof_mu);
    ROCKET_LOGI("ROCKET profile total(ms): stage=%.3f submit=%.3f wait=%.3f read=%.3f over %ld calls\n", g_prof.stage,
                g_prof.submit, g_prof.wait, g_prof.read, g_prof.calls);
}

void prof_add(double stage, double submit, double wait, double read)
{
    std::lock_guard<std::mutex> g(g_prof_mu);
    if (!g_prof_armed) {
        atexit(prof_dump);
        g_prof_armed = true;
    }
    g_prof.stage += stage;
    g_prof.submit += submit;
    g_prof.wait += wait;
    g_prof.read += read;
    g_prof.calls++;
}

// Adds the scope's host time (ms) to `acc` when profiling is on.
struct PhaseTimer {
    double *acc;
    std::chrono::steady_clock::time_point t0;
    explicit PhaseTimer(double &a) : acc(mm_profile() ? &a : nullptr)
    {
        if (acc) t0 = std::chrono::steady_clock::now();
    }
    ~PhaseTimer()
    {
        if (acc) *acc += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    }
};

// ROCKET_DEV named a device node in the reference; here it selects a HIP device index.
// A plain number is the index; a path ending in digits ("/dev/accel/accel1") uses them.
int env_device()
{
    const char *e = getenv("ROCKET_DEV");
    if (!e || !*e) return 0;
    const char *p = e + strlen(e);
    while (p > e && p[-1] >= '0' && p[-1] <= '9') p--;
    return *p ? atoi(p) : 0;
}

// Waits on `s` until done or `deadline_ns` (monotonic, 0 = poll once).
int wait_stream(hipStream_t s, int64_t budget_ns, const char *who, bool quiet_busy)
{
    const auto t0 = std::chrono::steady_clock::now();
    const long spin_us = busy_poll_us();
    for (;;) {
        const hipError_t e = hipStreamQuery(s);
        if (e == hipSuccess) return ROCKET_OK;
        if (e != hipErrorNotReady) {
            (void)hipGetLastError();
            ROCKET_LOGE("%s: device error while waiting: %s\n", who, hipGetErrorString(e));
            return ROCKET_E_DEVICE;
        }
        const int64_t el = std::chrono::duration_cast<std::chrono::nanoseconds>(
                               std::chrono::steady_clock::now() - t0).count();
        if (el >= budget_ns) {
            if (!quiet_busy)
                ROCKET_LOGE("%s: WAIT TIMEOUT after %lld ms (ROCKET_WAIT_MS)\n", who,
                            (long long)(el / 1000000));
            return quiet_busy ? -EBUSY : ROCKET_E_DEVICE;
        }
        if (el > spin_us * 1000) std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
}

}  // namespace

std::shared_ptr<Handle> handle_get(int fd)
{
    if (fd < 0 || fd >= kMaxHandles) return nullptr;
    std::lock_guard<std::mutex> g(g_table_mu);
    return g_table[fd];
}

bool handle_bind(Handle *h)
{
    return hipSetDevice(h->device) == hipSuccess;
}

int handle_wait(Handle *h, const char *who)
{
    const int rc = wait_stream(h->stream, (int64_t)wait_ms() * 1000000, who, false);
    if (rc) h->dirty = true;
    return rc;
}

void count_launch(uint64_t workgroups)
{
    g_submits.fetch_add(1, std::memory_order_relaxed);
    g_tasks.fetch_add(workgroups, std::memory_order_relaxed);
}

bool is_device_ptr(const void *p, int device)
{
    if (!p) return false;
    hipPointerAttribute_t a;
    if (hipPointerGetAttributes(&a, p) != hipSuccess) {
        (void)hipGetLastError();     // plain host memory: not an error for us
        return false;
    }
    if (a.type == hipMemoryTypeManaged || a.isManaged) return true;
    return a.type == hipMemoryTypeDevice && a.device == device;
}

void *dev_alloc(size_t bytes, const char *who)
{
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 256) != hipSuccess) {
        (void)hipGetLastError();
        ROCKET_LOGE("%s: device allocation of %zu bytes failed\n", who, bytes);
        return nullptr;
    }
    return p;
}

void dev_free(void *p)
{
    if (p) (void)hipFree(p);
}

Locked::Locked(int fd) : ref_(handle_get(fd))
{
    if (!ref_) return;
    ref_->mu.lock();
    // a rocket_close that ran between the lookup and the lock has released the buffers
    if (ref_->closed || !handle_bind(ref_.get())) {
        ref_->mu.unlock();
        ref_.reset();
        return;
    }
    h = ref_.get();
}

Locked::~Locked()
{
    if (h) h->mu.unlock();
}

// ---- Call: operand staging for one entry-point invocation ----

bool Call::direct_(const void *p) const
{
    if (!p || ((uintptr_t)p & 15u) != 0) return false;
    return h_->trust_device || is_device_ptr(p, h_->device);
}

void Call::want(const void *p, size_t bytes)
{
    if (!direct_(p)) need_ += round_(bytes);
}

int Call::begin()
{
    PhaseTimer pt(t_stage_);
    if (h_->dirty) {                     // an earlier wait gave up: drain before reuse
        if (hipStreamSynchronize(h_->stream) != hipSuccess) { (void)hipGetLastError(); return err_ = ROCKET_E_DEVICE; }
        h_->dirty = false;
    }
    if (need_ > h_->arena_cap) {
        if (hipStreamSynchronize(h_->stream) != hipSuccess) { (void)hipGetLastError(); return err_ = ROCKET_E_DEVICE; }
        dev_free(h_->arena);
        h_->arena = nullptr;
        h_->arena_cap = 0;
        const size_t cap = need_ + need_ / 4;
        h_->arena = dev_alloc(cap, who_);
        if (!h_->arena) return err_ = ROCKET_E_NOMEM;
        h_->arena_cap = cap;
    }
    return ROCKET_OK;
}

void *Call::scratch(size_t bytes)
{
    const size_t r = round_(bytes);
    if (err_ || used_ + r > h_->arena_cap) { if (!err_) err_ = ROCKET_E_NOMEM; return nullptr; }
    void *d = static_cast<char *>(h_->arena) + used_;
    used_ += r;
    return d;
}

void *Call::in(const void *p, size_t bytes)
{
    if (direct_(p)) return const_cast<void *>(p);
    PhaseTimer pt(t_stage_);
    host_io_ = true;
    void *d = scratch(bytes);
    if (!d) return nullptr;
    if (hipMemcpyAsync(d, p, bytes, hipMemcpyDefault, h_->stream) != hipSuccess) {
        (void)hipGetLastError();
        ROCKET_LOGE("%s: host-to-device copy failed\n", who_);
        err_ = ROCKET_E_DEVICE;
        return nullptr;
    }
    return d;
}

void *Call::out(void *p, size_t bytes)
{
    if (direct_(p)) return p;
    host_io_ = true;
    void *d = scratch(bytes);
    if (!d) return nullptr;
    back_.push_back({p, d, bytes});
    return d;
}

int Call::launch(const Launch &L0)
{
    if (err_) return err_;
    PhaseTimer pt(t_submit_);
    Launch L = L0;
    L.stream = h_->stream;
    uint64_t blocks = 0;
    const hipError_t e = gemm_launch(L, &blocks);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        ROCKET_LOGE("%s: kernel launch rejected: %s\n", who_, hipGetErrorString(e));
        return err_ = (e == hipErrorInvalidValue) ? ROCKET_E_SHAPE : ROCKET_E_DEVICE;
    }
    count_launch(blocks);
    return ROCKET_OK;
}

int Call::finish()
{
    const int rc = finish_();
    if (mm_profile()) prof_add(t_stage_, t_submit_, t_wait_, t_read_);
    return rc;
}

int Call::finish_()
{
    if (err_) {
        PhaseTimer pt(t_wait_);
        (void)handle_wait(h_, who_);   // leave nothing half-queued behind an error
        return err_;
    }
    if (!host_io_ && back_.empty() && h_->async) return ROCKET_OK;
    size_t total = 0;
    for (const Back &b : back_) total += round_(b.bytes);
    {
        PhaseTimer pt(t_read_);
        if (total > h_->pin_cap) {
            if (hipStreamSynchronize(h_->stream) != hipSuccess) { (void)hipGetLastError(); return ROCKET_E_DEVICE; }
            if (h_->pin) (void)hipHostFree(h_->pin);
            h_->pin = nullptr;
            h_->pin_cap = 0;
            if (hipHostMalloc(&h_->pin, total, hipHostMallocDefault) != hipSuccess) {
                (void)hipGetLastError();
                ROCKET_LOGE("%s: pinned staging of %zu bytes failed\n", who_, total);
                h_->pin = nullptr;
                return ROCKET_E_NOMEM;
            }
            h_->pin_cap = total;
        }
        size_t off = 0;
        for (const Back &b : back_) {
            if (hipMemcpyAsync(static_cast<char *>(h_->pin) + off, b.src, b.bytes, hipMemcpyDeviceToHost,
                               h_->stream) != hipSuccess) {
                (void)hipGetLastError();
                ROCKET_LOGE("%s: device-to-host copy failed\n", who_);
                (void)handle_wait(h_, who_);
                return ROCKET_E_DEVICE;
            }
            off += round_(b.bytes);
        }
    }
    {
        PhaseTimer pt(t_wait_);
        const int rc = handle_wait(h_, who_);
        if (rc) return rc;
    }
    PhaseTimer pt(t_read_);
    size_t off = 0;
    for (const Back &b : back_) {
        memcpy(b.dst, static_cast<char *>(h_->pin) + off, b.bytes);
        off += round_(b.bytes);
    }
    return ROCKET_OK;
}

}  // namespace rk

using namespace rk;

// =====================================================================================
// rocket_npu.h
// =====================================================================================
extern "C" {

int rocket_open(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        ROCKET_LOGD("rocket_open: no HIP device\n");
        return -ENODEV;
    }
    const int dev = env_device();
    if (dev < 0 || dev >= n) {
        ROCKET_LOGE("rocket_open: ROCKET_DEV selects device %d of %d\n", dev, n);
        return -ENODEV;
    }
    if (hipSetDevice(dev) != hipSuccess) { (void)hipGetLastError(); return -ENODEV; }
    std::shared_ptr<Handle> h(new (std::nothrow) Handle);
    if (!h) return -ENOMEM;
    h->device = dev;
    if (hipStreamCreateWithFlags(&h->own, hipStreamNonBlocking) != hipSuccess) {
        (void)hipGetLastError();
        return -ENODEV;
    }
    h->stream = h->own;
    {
        std::lock_guard<std::mutex> g(g_table_mu);
        for (int i = 0; i < kMaxHandles; i++)
            if (!g_table[i]) { g_table[i] = std::move(h); return i; }
    }
    (void)hipStreamDestroy(h->own);
    return -EMFILE;
}

void rocket_close(int fd)
{
    if (fd < 0 || fd >= kMaxHandles) return;
    std::shared_ptr<Handle> h;
    {
        std::lock_guard<std::mutex> g(g_table_mu);
        h = std::move(g_table[fd]);
        g_table[fd].reset();
    }
    if (!h) return;
    {   // waits for a call in flight on this handle; later lookups find the slot empty and
        // a caller that looked up before the close sees `closed` under the lock
        std::lock_guard<std::mutex> g(h->mu);
        h->closed = true;
        if (hipSetDevice(h->device) == hipSuccess) {
            (void)hipStreamSynchronize(h->stream);
            dev_free(h->arena);
            h->arena = nullptr;
            h->arena_cap = 0;
            if (h->pin) (void)hipHostFree(h->pin);
            h->pin = nullptr;
            h->pin_cap = 0;
            (void)hipStreamDestroy(h->own);
            h->own = h->stream = nullptr;
        }
        (void)hipGetLastError();
    }
    // the Handle itself is freed with its last reference (this one, or a caller's)
}

// ---- affinity (no host fan-out on this device) ----
static thread_local int t_affinity_base = 0;
void rocket_affinity_set_base(int base) { t_affinity_base = base < 0 ? 0 : base; }
int  rocket_affinity_get_base(void) { return t_affinity_base; }
void rocket_pin_worker(int worker_idx) { (void)worker_idx; }
int  rocket_num_big_cores(void) { return 0; }

// ---- buffer objects: pinned host pages mapped into the GPU's address space ----
static std::atomic<uint32_t> g_bo_handle{1};

int rocket_bo_alloc(int fd, size_t size, rocket_bo *bo)
{
    if (!bo || size == 0) return -EINVAL;
    memset(bo, 0, sizeof(*bo));
    Locked L(fd);
    if (!L.ok()) return -EBADF;
    const size_t sz = (size + 4095) & ~(size_t)4095;
    void *p = nullptr;
    if (hipHostMalloc(&p, sz, hipHostMallocMapped) != hipSuccess) {
        (void)hipGetLastError();
        ROCKET_LOGE("rocket_bo_alloc: %zu bytes failed\n", sz);
        return -ENOMEM;
    }
    void *d = nullptr;
    if (hipHostGetDevicePointer(&d, p, 0) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipHostFree(p);
        return -ENOMEM;
    }
    memset(p, 0, sz);
    bo->handle = g_bo_handle.fetch_add(1);
    bo->dma_address = (uint64_t)(uintptr_t)d;
    bo->mmap_offset = 0;
    bo->size = sz;
    bo->ptr = p;
    return 0;
}

void rocket_bo_free(int fd, rocket_bo *bo)
{
    (void)fd;
    if (!bo || !bo->ptr) return;
    (void)hipHostFree(bo->ptr);
    (void)hipGetLastError();
    memset(bo, 0, sizeof(*bo));
}

int rocket_bo_prep(int fd, rocket_bo *bo, int dir, uint64_t timeout_ns)
{
    (void)dir;
    if (!bo || !bo->ptr) return -EINVAL;
    Locked L(fd);
    if (!L.ok()) return -EBADF;
    // the reference saturates huge relative timeouts instead of overflowing (:682-710)
    const int64_t budget = timeout_ns > (uint64_t)INT64_MAX ? INT64_MAX : (int64_t)timeout_ns;
    return wait_stream(L.h->stream, budget, "rocket_bo_prep", true);
}

int rocket_bo_fini(int fd, rocket_bo *bo)
{
    (void)fd;
    return (bo && bo->ptr) ? 0 : -EINVAL;
}

static int ranges_ok(const rocket_bo *bo, const rocket_bo_range *r, unsigned n)
{
    if (!bo || !bo->ptr) return 0;
    if (n && !r) return 0;
    uint64_t end = 0;
    for (unsigned i = 0; i < n; i++) {
        if (r[i].size == 0 || r[i].offset < end) return 0;          // ascending, disjoint
        if (r[i].offset > bo->size || r[i].size > bo->size - r[i].offset) return 0;
        end = r[i].offset + r[i].size;
    }
    return 1;
}

int rocket_bo_prep_ranges(int fd, rocket_bo *bo, const rocket_bo_range *r, unsigned n,
                          uint64_t timeout_ns)
{
    if (!ranges_ok(bo, r, n)) return -EINVAL;
    return rocket_bo_prep(fd, bo, 0, timeout_ns);
}

int rocket_bo_fini_ranges(int fd, rocket_bo *bo, const rocket_bo_range *r, unsigned n)
{
    if (!ranges_ok(bo, r, n)) return -EINVAL;
    return rocket_bo_fini(fd, bo);
}

int  rocket_bo_ranges_supported(void) { return 1; }
int  rocket_batched_submit_supported(void) { return 0; }
int  rocket_ppu_done_supported(void) { return 0; }
int  rocket_batch_completion_tracked(void) { return 0; }
void rocket_busy_poll_set_us(long us) { g_busy_poll_us.store(us <= 0 ? 0 : us); }

// ---- register-program submission: no register-command processor on a GPU ----
static int submit_unsupported(int fd, const char *who)
{
    if (!handle_get(fd)) return -EBADF;
    ROCKET_LOGD("%s: no register programs on MI355X; use the rocket_matmul_* entries\n", who);
    return ROCKET_E_UNSUPPORTED;
}

int rocket_submit_matmul(int fd, const rocket_bo *regcmd_bo, uint32_t regcmd_count,
                         const uint32_t *in_handles, uint32_t n_in,
                         const uint32_t *out_handles, uint32_t n_out, uint32_t timeout_ms)
{
    (void)regcmd_bo; (void)regcmd_count; (void)in_handles; (void)n_in; (void)out_handles;
    (void)n_out; (void)timeout_ms;
    return submit_unsupported(fd, "rocket_submit_matmul");
}

int rocket_submit_matmul_flags(int fd, const rocket_bo *regcmd_bo, uint32_t regcmd_count,
                               const uint32_t *in_handles, uint32_t n_in,
                               const uint32_t *out_handles, uint32_t n_out, uint32_t job_flags)
{
    (void)regcmd_bo; (void)regcmd_count; (void)in_handles; (void)n_in; (void)out_handles;
    (void)n_out; (void)job_flags;
    return submit_unsupported(fd, "rocket_submit_matmul_flags");
}

int rocket_submit_tasks(int fd, const rocket_task_desc *tasks, uint32_t n_tasks,
                        const uint32_t *in_handles, uint32_t n_in,
                        const uint32_t *out_handles, uint32_t n_out)
{
    (void)tasks; (void)n_tasks; (void)in_handles; (void)n_in; (void)out_handles; (void)n_out;
    return submit_unsupported(fd, "rocket_submit_tasks");
}

int rocket_submit_tasks_flags(int fd, const rocket_task_desc *tasks, uint32_t n_tasks,
                              const uint32_t *in_handles, uint32_t n_in,
                              const uint32_t *out_handles, uint32_t n_out, uint32_t job_flags)
{
    (void)tasks; (void)n_tasks; (void)in_handles; (void)n_in; (void)out_handles; (void)n_out;
    (void)job_flags;
    return submit_unsupported(fd, "rocket_submit_tasks_flags");
}

size_t rocket_submit_scratch_size(uint32_t max_tasks)
{
    return (size_t)max_tasks * 2 * sizeof(uint64_t);
}

int rocket_submit_tasks_pre(int fd, void *scratch, const rocket_task_desc *tasks, uint32_t n_tasks,
                            const uint32_t *in_handles, uint32_t n_in,
                            const uint32_t *out_handles, uint32_t n_out, uint32_t job_flags)
{
    (void)scratch; (void)tasks; (void)n_tasks; (void)in_handles; (void)n_in; (void)out_handles;
    (void)n_out; (void)job_flags;
    return submit_unsupported(fd, "rocket_submit_tasks_pre");
}

int rocket_submit_jobs(int fd, const rocket_job_desc *jobs, uint32_t n_jobs)
{
    (void)jobs; (void)n_jobs;
    return submit_unsupported(fd, "rocket_submit_jobs");
}

uint64_t rocket_submit_ioctl_count(void) { return g_submits.load(std::memory_order_relaxed); }
uint64_t rocket_submit_task_count(void) { return g_tasks.load(std::memory_order_relaxed); }
void     rocket_submit_counters_reset(void)
{
    g_submits.store(0, std::memory_order_relaxed);
    g_tasks.store(0, std::memory_order_relaxed);
}

}  // extern "C"
