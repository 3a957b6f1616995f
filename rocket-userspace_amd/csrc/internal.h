// internal.h — handle table, operand staging and waits shared by the entry points.
#pragma once

#include <hip/hip_runtime.h>

#include <memory>
#include <mutex>
#include <stddef.h>
#include <stdint.h>
#include <vector>

#include "gemm.h"
#include "rocket_log.h"
#include "rocket_npu.h"

namespace rk {

// One open "fd": a HIP device, the stream its work runs on, and reusable device / pinned
// host buffers for staging host operands. Calls on one handle are serialised by `mu`;
// different handles run independently.
struct Handle {
    int device = 0;
    hipStream_t own = nullptr;     // created by rocket_open
    hipStream_t stream = nullptr;  // own, or one bound with rocket_hip_set_stream
    bool async = false;            // device-only calls return without waiting
    bool trust_device = false;     // every operand is device memory: skip classification
    bool dirty = false;            // a wait timed out: drain before reusing buffers
    bool closed = false;           // rocket_close ran: buffers released, no further work
    void *arena = nullptr;  size_t arena_cap = 0;   // device staging
    void *pin = nullptr;    size_t pin_cap = 0;     // pinned host staging for results
    std::mutex mu;
};

// Handle lookup: empty for a closed / invalid fd. The table holds one reference and every
// lookup another, so a handle outlives a concurrent rocket_close until its last user drops
// the reference; such a user sees `closed` once it holds the handle's lock.
std::shared_ptr<Handle> handle_get(int fd);

// Sets the handle's device current on the calling thread.
bool handle_bind(Handle *h);

// Waits for the handle's queued work, bounded by ROCKET_WAIT_MS (default 8000 ms).
// Returns ROCKET_OK, or ROCKET_E_DEVICE on a runtime error or time-out (logged with `who`).
int handle_wait(Handle *h, const char *who);

// Process-wide dispatch counters (rocket_submit_ioctl_count / _task_count).
void count_launch(uint64_t workgroups);

// True when p is device memory of `device` (or managed memory), usable in place.
bool is_device_ptr(const void *p, int device);

// Stages one call's operands. in()/out() return the device address the kernel uses:
// the caller's own pointer when it is 16-byte-aligned device memory, otherwise a slice
// of the handle's arena (inputs copied in, results copied back by finish()).
class Call {
public:
    Call(Handle *h, const char *who) : h_(h), who_(who) {}
    // Reserve arena space before in()/out(): sum of every host operand's bytes.
    void want(const void *p, size_t bytes);
    void want_scratch(size_t bytes) { need_ += round_(bytes); }
    int  begin();                          // grows the arena if needed
    void *in(const void *p, size_t bytes);  // device view of an input
    void *out(void *p, size_t bytes);       // device view of an output
    void *scratch(size_t bytes);            // arena scratch (not copied)
    int  launch(const Launch &L);           // enqueue one GEMM launch
    int  finish();                          // copy results back and wait (unless async)
    hipStream_t stream() const { return h_->stream; }
    const char *who() const { return who_; }
    bool host_io() const { return host_io_; }

private:
    static size_t round_(size_t b) { return (b + 255) & ~(size_t)255; }
    bool direct_(const void *p) const;
    int finish_();
    // ROCKET_MM_PROFILE: host milliseconds of this call's phases (staging copies and arena
    // growth, kernel enqueue, the bounded wait, result copy-out), added to the process totals
    // when the call finishes
    double t_stage_ = 0, t_submit_ = 0, t_wait_ = 0, t_read_ = 0;
    Handle *h_;
    const char *who_;
    size_t need_ = 0, used_ = 0;
    bool host_io_ = false;
    int err_ = 0;
    struct Back { void *dst; const void *src; size_t bytes; };
    std::vector<Back> back_;
};

// Allocation helpers that log on failure.
void *dev_alloc(size_t bytes, const char *who);
void  dev_free(void *p);

// RAII lock + bind for an fd. ok() false: bad or closed fd (ROCKET_E_DEVICE).
struct Locked {
    explicit Locked(int fd);
    ~Locked();
    Locked(const Locked &) = delete;
    Locked &operator=(const Locked &) = delete;
    bool ok() const { return h != nullptr; }
    Handle *h = nullptr;

private:
    std::shared_ptr<Handle> ref_;
};

}  // namespace rk
