// noalloc.cpp — rocket_matmul_int4_prepacked_gw_f32in_noalloc: the W4A8 resident product on
// fp32 activations without any device allocation (rocket_quant.h).
//
// The entry it mirrors quantises A into the handle's arena, which the library grows with
// hipMalloc on demand. Here the int8 codes and row scales go to `scratch`, a file-scope
// device array of kScratchBytes that each GPU holds for the life of the process. Host code
// never uses the array's name as an address: its device address is resolved once per device
// with hipGetSymbolAddress (that device current) and kept in g_scratch[].
//
// Every call on one GPU shares that GPU's array. Calls queued on one stream run in order and
// are safe; calls that overlap on one GPU (two handles, or streams, running at once) race on
// the array. Nothing in it needs clearing: the pre-pass writes every code and scale the GEMM
// reads.
//
// Under HIP graph capture of the handle's stream the entry only records its two launches: it
// neither waits for them (stream queries and synchronisation are illegal while a stream
// captures) nor drains a handle left dirty by an earlier wait that gave up (that case is
// refused, since draining would invalidate the capture). A replayed graph writes Cf when it
// runs. Nothing it records is a memset or a copy.
#include "ops.h"
#include "resident.h"
#include "rocket_hip.h"
#include "rocket_quant.h"

#include <mutex>

// codes (M * K bytes, rounded up to 256) + row scales (M * 4)
constexpr size_t kScratchBytes = 16u << 20;

static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_scratch_mu;
void *g_scratch[kMaxDevices];   // device address of `scratch` on each device (null: not resolved)

// The array's address on the calling thread's current device (`device`); null on failure.
void *scratch_on(int device)
{
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            ROCKET_LOGE("rocket_matmul_int4_prepacked_gw_f32in_noalloc: scratch address on device %d: %s\n", device,
                        hipGetErrorString(e));
            return nullptr;
        }
        g_scratch[device] = p;
    }
    return g_scratch[device];
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

}  // namespace

using namespace rk;

extern "C" {

int rocket_matmul_int4_prepacked_gw_f32in_noalloc(rocket_i4_ctx *ctx, int M, int K, int N, const float *A,
                                                   const float *b_scale, float *Cf, rocket_i4_weights *w)
{   // the checks of rocket_matmul_int4_prepacked_gw_f32in, then the scratch and operand rules
    static const char *who = "rocket_matmul_int4_prepacked_gw_f32in_noalloc";
    if (!ctx || !w || w->group <= 0 || !A || !b_scale || !Cf) return ROCKET_E_SHAPE;
    if (M % 4 != 0 || M <= 0) {
        ROCKET_LOGE("%s: M=%d must be a positive multiple of 4 — pad rows caller-side\n", who, M);
        return ROCKET_E_SHAPE;
    }
    if (K != w->K || N != w->N) {
        ROCKET_LOGE("%s: shape K=%d N=%d != packed %d/%d\n", who, K, N, w->K, w->N);
        return ROCKET_E_SHAPE;
    }
    // the pre-pass reads A and the GEMM writes Cf in 16-byte vectors, straight from the caller's
    // pointers (the entry it mirrors stages misaligned operands through its arena instead)
    if (((uintptr_t)A & 15u) || ((uintptr_t)Cf & 15u)) {
        ROCKET_LOGE("%s: A (%p) and Cf (%p) must be 16-byte aligned (nothing is staged without allocation)\n", who,
                    (const void *)A, (void *)Cf);
        return ROCKET_E_SHAPE;
    }
    const size_t codes = align256((size_t)M * K), need = codes + (size_t)M * sizeof(float);
    if (need > kScratchBytes) {
        ROCKET_LOGE("%s: M*K = %zu needs %zu scratch bytes, above the fixed %zu (split the rows)\n", who,
                    (size_t)M * K, need, kScratchBytes);
        return ROCKET_E_SHAPE;
    }
    Locked L(rocket_i4_ctx_fd(ctx));
    if (!L.ok()) return ROCKET_E_DEVICE;
    // nothing is staged: every operand must already be device memory of this GPU
    if (!L.h->trust_device && (!is_device_ptr(A, L.h->device) || !is_device_ptr(b_scale, L.h->device) ||
                               !is_device_ptr(Cf, L.h->device))) {
        ROCKET_LOGE("%s: A, b_scale and Cf must be device memory (no host staging without allocation)\n", who);
        return ROCKET_E_SHAPE;
    }
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(L.h->stream, &cap) != hipSuccess) {
        (void)hipGetLastError();
        return ROCKET_E_DEVICE;
    }
    const bool capturing = cap == hipStreamCaptureStatusActive;
    if (L.h->dirty) {   // an earlier wait gave up: drain before reuse
        if (capturing) {
            ROCKET_LOGE("%s: an earlier wait on this handle gave up; draining it would invalidate the capture\n", who);
            return ROCKET_E_DEVICE;
        }
        if (hipStreamSynchronize(L.h->stream) != hipSuccess) { (void)hipGetLastError(); return ROCKET_E_DEVICE; }
        L.h->dirty = false;
    }
    char *base = static_cast<char *>(scratch_on(L.h->device));
    if (!base) return ROCKET_E_DEVICE;
    int8_t *Aq = reinterpret_cast<int8_t *>(base);
    float *rs = reinterpret_cast<float *>(base + codes);

    QuantRows q;
    q.n = 1;
    q.K = K;
    q.M[0] = M;
    q.A[0] = A;
    q.Aq[0] = Aq;
    q.row_scale[0] = rs;
    uint64_t blocks = 0;
    if (quant_rows(q, L.h->stream, &blocks) != hipSuccess) {
        (void)hipGetLastError();
        ROCKET_LOGE("%s: quantisation launch rejected\n", who);
        return ROCKET_E_SHAPE;
    }
    count_launch(blocks);

    Launch g;
    g.fmt_a = Fmt::I8;
    g.fmt_b = Fmt::I4P;
    g.epi = Epi::GW;
    g.N = N;
    g.K = K;
    g.kbeg = 0;
    g.kend = K;
    g.group = w->group;
    g.kt = gw_period(w->group);
    g.rowscale = 1;
    g.nprob = 1;
    g.prob[0] = Problem{M, Aq, w->dev, Cf, rs, b_scale, nullptr};
    g.stream = L.h->stream;
    const hipError_t e = gemm_launch(g, &blocks);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        ROCKET_LOGE("%s: kernel launch rejected: %s\n", who, hipGetErrorString(e));
        if (!capturing) (void)handle_wait(L.h, who);
        return e == hipErrorInvalidValue ? ROCKET_E_SHAPE : ROCKET_E_DEVICE;
    }
    count_launch(blocks);
    if (L.h->async || capturing) return ROCKET_OK;
    return handle_wait(L.h, who);
}

}  // extern "C"
