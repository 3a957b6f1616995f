/*
 * rocket_npu.h — device shim of the MI355X (gfx950) librocketnpu.
 *
 * Same prototypes, enum values and struct layouts as the reference shim
 * (reference include/rocket_npu.h:41-304), so a caller that was built against the
 * RK3588 library relinks against this one unchanged. The DRM-accel calls underneath
 * are replaced by HIP:
 *
 *   reference (DRM ioctl)                 this library (HIP)
 *   rocket_open      DRM_IOCTL_VERSION     slot in a handle table {device, stream, arena}
 *   rocket_bo_alloc  CREATE_BO + mmap      hipHostMalloc(mapped): ptr = host view,
 *                                          dma_address = device view of the same pages
 *   rocket_bo_prep   PREP_BO (fence wait)  hipStreamSynchronize on the handle's stream,
 *                                          bounded by the caller's timeout
 *   rocket_bo_fini   FINI_BO (flush)       no-op (mapped pinned memory is coherent)
 *   rocket_submit_*  SUBMIT (regcmd)       ROCKET_E_UNSUPPORTED: there is no register
 *                                          program on this device; the matmul entries in
 *                                          rocket_matmul.h launch HIP kernels directly
 *
 * Error convention (reference rocket_npu.h:25-36): 0 on success, a negative
 * rocket_status on failure; rocket_open returns a negative errno.
 */
#ifndef ROCKET_NPU_H
#define ROCKET_NPU_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status vocabulary (values fixed by reference rocket_npu.h:41-48). */
enum rocket_status {
    ROCKET_OK            =  0,
    ROCKET_E_SHAPE       = -1,   /* unsupported shape or bad argument */
    ROCKET_E_TILING      = -2,   /* valid shape, wrong tiling here: re-pack / fall back */
    ROCKET_E_NOMEM       = -3,   /* allocation failed */
    ROCKET_E_DEVICE      = -4,   /* HIP runtime / device failure */
    ROCKET_E_UNSUPPORTED = -5,   /* not available on this device or path */
};

/* Buffer object (layout of reference rocket_npu.h:51-57). On MI355X `ptr` is the
 * CPU view and `dma_address` the GPU virtual address of the same pinned pages;
 * `handle` indexes the library's BO table; `mmap_offset` is 0. */
typedef struct {
    uint32_t handle;
    uint64_t dma_address;
    uint64_t mmap_offset;
    size_t   size;
    void    *ptr;
} rocket_bo;

/* ---- device open / close (reference rocket_npu.h:63-64) ----
 * rocket_open selects HIP device ROCKET_DEV (an index, default 0), creates a
 * stream for the handle and returns the handle index (>= 0), or -ENODEV / -ENOMEM. */
int  rocket_open(void);
void rocket_close(int fd);

/* ---- CPU-affinity hints (reference rocket_npu.h:84-98) ----
 * Kept for ABI compatibility. The fan-out they tuned is a single GPU grid here, so
 * they only record the base; rocket_pin_worker is a no-op and rocket_num_big_cores
 * returns 0 ("no distinct big cluster"). */
void rocket_affinity_set_base(int base);
int  rocket_affinity_get_base(void);
void rocket_pin_worker(int worker_idx);
int  rocket_num_big_cores(void);

/* ---- buffers, cache brackets, fences (reference rocket_npu.h:108-156) ---- */
int  rocket_bo_alloc(int fd, size_t size, rocket_bo *bo);
void rocket_bo_free(int fd, rocket_bo *bo);
/* Waits for the handle's queued GPU work (dir 0) before the CPU reads; timeout_ns is
 * relative; 0 polls and returns -EBUSY when work is still queued. */
int  rocket_bo_prep(int fd, rocket_bo *bo, int dir, uint64_t timeout_ns);
int  rocket_bo_fini(int fd, rocket_bo *bo);

typedef struct { uint64_t offset, size; } rocket_bo_range;
/* Ranges are validated exactly as the reference kernel does (ascending,
 * non-overlapping, inside the BO; -EINVAL otherwise); n == 0 means the whole BO. */
int  rocket_bo_prep_ranges(int fd, rocket_bo *bo, const rocket_bo_range *r,
                           unsigned n, uint64_t timeout_ns);
int  rocket_bo_fini_ranges(int fd, rocket_bo *bo, const rocket_bo_range *r,
                           unsigned n);
int  rocket_bo_ranges_supported(void);           /* 1: ranged brackets are honoured */

/* Kernel-feature probes of the NPU uAPI: none applies to a GPU, all return 0. */
int  rocket_batched_submit_supported(void);
int  rocket_ppu_done_supported(void);
int  rocket_batch_completion_tracked(void);
void rocket_busy_poll_set_us(long us);

/* ---- register-program submission (reference rocket_npu.h:173-290) ----
 * There is no register-command processor on MI355X. Every submit entry validates its
 * arguments and returns ROCKET_E_UNSUPPORTED without touching the device. */
int  rocket_submit_matmul(int fd,
                          const rocket_bo *regcmd_bo, uint32_t regcmd_count,
                          const uint32_t *in_handles,  uint32_t n_in,
                          const uint32_t *out_handles, uint32_t n_out,
                          uint32_t timeout_ms);
int  rocket_submit_matmul_flags(int fd,
                                const rocket_bo *regcmd_bo, uint32_t regcmd_count,
                                const uint32_t *in_handles,  uint32_t n_in,
                                const uint32_t *out_handles, uint32_t n_out,
                                uint32_t job_flags);

#define ROCKET_JOB_BATCHED      (1u << 0)
#define ROCKET_JOB_NO_DPU_DONE  (1u << 1)
#define ROCKET_JOB_PPU_DONE     (1u << 2)

typedef struct { uint32_t regcmd; uint32_t regcmd_count; } rocket_task_desc;

int  rocket_submit_tasks(int fd,
                         const rocket_task_desc *tasks, uint32_t n_tasks,
                         const uint32_t *in_handles,  uint32_t n_in,
                         const uint32_t *out_handles, uint32_t n_out);
int  rocket_submit_tasks_flags(int fd,
                               const rocket_task_desc *tasks, uint32_t n_tasks,
                               const uint32_t *in_handles,  uint32_t n_in,
                               const uint32_t *out_handles, uint32_t n_out,
                               uint32_t job_flags);
size_t rocket_submit_scratch_size(uint32_t max_tasks);
int    rocket_submit_tasks_pre(int fd, void *scratch,
                               const rocket_task_desc *tasks, uint32_t n_tasks,
                               const uint32_t *in_handles,  uint32_t n_in,
                               const uint32_t *out_handles, uint32_t n_out,
                               uint32_t job_flags);

typedef struct {
    const rocket_task_desc *tasks;  uint32_t n_tasks;
    const uint32_t *in_handles;     uint32_t n_in;
    const uint32_t *out_handles;    uint32_t n_out;
} rocket_job_desc;

int  rocket_submit_jobs(int fd, const rocket_job_desc *jobs, uint32_t n_jobs);

/* Process-wide dispatch counters (reference rocket_npu.h:295-304). On MI355X one
 * "submit" is one kernel launch and one "task" is one workgroup of it. Plain,
 * non-atomic counters, as in the reference. */
uint64_t rocket_submit_ioctl_count(void);
uint64_t rocket_submit_task_count(void);
void     rocket_submit_counters_reset(void);

#ifdef __cplusplus
}
#endif
#endif /* ROCKET_NPU_H */
