// shim_check.cpp — drives every device-free path of librocketnpu's host code under the host
// AddressSanitizer and UndefinedBehaviorSanitizer (built by tests/native/sanitize.mk, run by
// tests/test_sanitizers.py on a machine without a GPU): planners, argument rejections, the
// log channel, hardware profiles, the serialised-weight reader on intact and corrupted
// blobs, the fp64 host references of the FFN and attention blocks (checked bit for bit against
// the oracle, built into the same binary), and handle-table calls from several threads.
// Exit status 0 when every check passes; a sanitizer report aborts the run.
#include <errno.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <string>
#include <thread>
#include <vector>

#include "rocket_attn.h"
#include "rocket_ffn.h"
#include "rocket_hip.h"
#include "rocket_hw_profile.h"
#include "rocket_log.h"
#include "rocket_matmul.h"
#include "rocket_npu.h"
#include "rocket_quant.h"
#include "rocket_weights_io.h"

extern "C" {
#include "oracle.h"
}

static int g_fail = 0;
#define CHECK(c)                                                                     \
    do {                                                                             \
        if (!(c)) {                                                                  \
            fprintf(stderr, "shim_check: %s:%d: CHECK(%s) failed\n", __FILE__, __LINE__, #c); \
            g_fail++;                                                                \
        }                                                                            \
    } while (0)

static std::atomic<int> g_logged{0};
static void log_cb(rocket_log_level lvl, const char *msg, void *ud)
{
    (void)lvl;
    (void)ud;
    if (msg && msg[0]) g_logged++;
}

static std::vector<uint16_t> f16v(size_t n, uint64_t seed, float lo, float hi)
{
    std::vector<float> f(n);
    rko_gen_f32_uniform(f.data(), n, seed, lo, hi);
    std::vector<uint16_t> h(n);
    rko_f32_to_f16_n(f.data(), h.data(), n);
    return h;
}
static const _Float16 *H(const std::vector<uint16_t> &v) { return reinterpret_cast<const _Float16 *>(v.data()); }
static _Float16 *H(std::vector<uint16_t> &v) { return reinterpret_cast<_Float16 *>(v.data()); }

static void planners()
{
    int mt = 0, kt = 0, nt = 0;
    CHECK(rocket_matmul_plan(64, 256, 128, &mt, &kt, &nt) > 0 && mt > 0 && kt == 256 && nt > 0);
    CHECK(rocket_matmul_plan(6, 256, 128, &mt, &kt, &nt) == ROCKET_E_SHAPE);       // M % 4
    CHECK(rocket_matmul_plan(64, 48, 128, &mt, &kt, &nt) == ROCKET_E_SHAPE);       // K % 32
    CHECK(rocket_matmul_plan(64, 256, 120, nullptr, nullptr, nullptr) == ROCKET_E_SHAPE);
    CHECK(rocket_matmul_plan((1 << 24) + 4, 32, 16, nullptr, nullptr, nullptr) == ROCKET_E_SHAPE);
    CHECK(rocket_matmul_plan(0, 32, 16, nullptr, nullptr, nullptr) == ROCKET_E_SHAPE);
    CHECK(rocket_matmul_plan(-4, 32, 16, nullptr, nullptr, nullptr) == ROCKET_E_SHAPE);
    CHECK(rocket_matmul_plan_int8(512, 4096, 4096, &mt, &kt, &nt) > 0);
    CHECK(rocket_matmul_plan_int8(512, 4096, 4080, &mt, &kt, &nt) == ROCKET_E_SHAPE);
    CHECK(rocket_matmul_plan_int8_gw(512, 3840, 15360, 128, &mt, &kt, &nt) > 0 && kt == 128);
    CHECK(rocket_matmul_plan_int8_gw(512, 3840, 15360, 48, &mt, &kt, &nt) == ROCKET_E_SHAPE);
    CHECK(rocket_matmul_plan_int8_gw(512, 3840, 15360, 0, &mt, &kt, &nt) == ROCKET_E_SHAPE);
    CHECK(rocket_matmul_plan_int8_gw(512, 3840, 15360, 1 << 30, &mt, &kt, &nt) == ROCKET_E_SHAPE);
    CHECK(rocket_matmul_plan_int4(512, 3840, 15360, &mt, &kt, &nt) > 0);
    CHECK(rocket_matmul_plan_int4(512, 3840, 15328, &mt, &kt, &nt) == ROCKET_E_SHAPE);   // N % 64
    CHECK(rocket_matmul_plan_int16(512, 4096, 4096, &mt, &kt, &nt) > 0);
    CHECK(rocket_matmul_plan_bf16(2048, 15360, 3840, &mt, &kt, &nt) > 0);
    CHECK(rocket_matmul_plan_tf32(2048, 15360, 3840, &mt, &kt, &nt) > 0);
    CHECK(rocket_matmul_plan_tf32(2048, 15368, 3840, &mt, &kt, &nt) == ROCKET_E_SHAPE);
    CHECK(rocket_matmul_plan_int8_rk3576(64, 64, 64, &mt, &kt, &nt) == ROCKET_E_UNSUPPORTED);
}

// Calls on a handle that is not open, and malformed arguments: refused before any device use.
static void rejections()
{
    const int bad = 77;
    std::vector<int8_t> a(64 * 256), b(128 * 256);
    std::vector<int32_t> c(64 * 128);
    std::vector<float> fs(64 * 128), as(64 * 8), bs(128 * 8);
    CHECK(rocket_matmul_int8(bad, 64, 256, 128, a.data(), b.data(), c.data()) == ROCKET_E_DEVICE);
    CHECK(rocket_matmul_int8(bad, 6, 256, 128, a.data(), b.data(), c.data()) == ROCKET_E_SHAPE);
    CHECK(rocket_matmul_int8(bad, 64, 256, 128, nullptr, b.data(), c.data()) == ROCKET_E_SHAPE);
    CHECK(rocket_matmul_int8_groupwise(bad, 64, 256, 128, a.data(), b.data(), as.data(), bs.data(), fs.data(), 32) ==
          ROCKET_E_DEVICE);
    CHECK(rocket_matmul_int8_groupwise(bad, 64, 256, 128, a.data(), b.data(), as.data(), bs.data(), fs.data(), 48) ==
          ROCKET_E_SHAPE);
    CHECK(rocket_matmul_int4_groupwise(bad, 64, 256, 128, a.data(), b.data(), as.data(), bs.data(), fs.data(), 672) ==
          ROCKET_E_SHAPE);   // 49 * group >= 32767
    CHECK(rocket_matmul_int8_groupwise_dump(bad, 64, 256, 128, a.data(), b.data(), as.data(), bs.data(), fs.data(),
                                            32, 60, 8, c.data()) == ROCKET_E_SHAPE);   // window past M
    CHECK(rocket_matmul_bf16(bad, 64, 256, 128, fs.data(), fs.data(), fs.data()) == ROCKET_E_DEVICE);
    CHECK(rocket_matmul_tf32(bad, 64, 40, 128, fs.data(), fs.data(), fs.data()) == ROCKET_E_SHAPE);
    const _Float16 *hn = nullptr;
    CHECK(rocket_matmul_fp16_batch(bad, 64, 256, 128, 0, &hn, &hn, nullptr) == ROCKET_E_SHAPE);
    CHECK(rocket_quantize_rows_int8(bad, 4, 12, fs.data(), a.data(), fs.data()) == ROCKET_E_SHAPE);   // K % 8
    CHECK(rocket_quantize_rows_int8(bad, 4, 16, fs.data(), a.data(), fs.data()) == ROCKET_E_DEVICE);
    CHECK(rocket_matmul_int8_prepacked_gw_grouped(nullptr, 2, nullptr, 256, 128, nullptr, nullptr, nullptr, nullptr,
                                                  nullptr) == ROCKET_E_SHAPE);
    CHECK(rocket_matmul_int4_prepacked_gw_f32in_noalloc(nullptr, 4, 256, 128, fs.data(), bs.data(), fs.data(),
                                                        nullptr) == ROCKET_E_SHAPE);
    CHECK(rocket_submit_matmul(bad, nullptr, 0, nullptr, 0, nullptr, 0, 0) == -EBADF);
    rocket_bo bo;
    memset(&bo, 0, sizeof bo);
    CHECK(rocket_bo_alloc(bad, 4096, &bo) == -EBADF);
    CHECK(rocket_bo_alloc(bad, 0, &bo) == -EINVAL);
    CHECK(rocket_bo_prep(bad, &bo, 0, 0) == -EINVAL);
    rocket_close(-1);
    rocket_close(bad);
    rocket_close(1 << 20);
    CHECK(rocket_hip_stream(bad) == nullptr);
    CHECK(rocket_hip_set_mode(bad, 0) == ROCKET_E_DEVICE);
    CHECK(rocket_mm_batch_create(bad) == nullptr);
}

static void logs_and_profiles()
{
    rocket_log_set_callback(log_cb, nullptr);
    rocket_log_set_level(ROCKET_LOG_DEBUG);
    CHECK(rocket_log_get_level() == ROCKET_LOG_DEBUG);
    const int before = g_logged.load();
    rocket_log(ROCKET_LOG_INFO, "shim_check %d %s\n", 1, "info");
    std::string longmsg(5000, 'x');   // longer than the channel's line buffer
    rocket_log(ROCKET_LOG_ERROR, "%s\n", longmsg.c_str());
    CHECK(g_logged.load() == before + 2);
    rocket_log_set_level(ROCKET_LOG_ERROR);
    rocket_log(ROCKET_LOG_INFO, "dropped\n");
    CHECK(g_logged.load() == before + 2);
    const rocket_hw_profile *p = rocket_hw_current();
    CHECK(p && p->name && strcmp(p->name, "mi355x") == 0);
    CHECK(rocket_hw_by_name("rk3588") == &rocket_hw_rk3588);
    CHECK(rocket_hw_by_name("no-such-chip") == nullptr);
    CHECK(rocket_hw_by_name(nullptr) == nullptr);
    CHECK(rocket_hw_dtype_supported(p, precision_int8));
}

static std::vector<uint8_t> slurp(const char *path)
{
    std::vector<uint8_t> v;
    FILE *f = fopen(path, "rb");
    if (!f) return v;
    uint8_t buf[4096];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) v.insert(v.end(), buf, buf + n);
    fclose(f);
    return v;
}

static void weights_reader(const char *dir)
{
    CHECK(rocket_weights_xxh64(nullptr, 0) == 0xEF46DB3751D8E999ull);
    for (const char *name : {"weights_int4_g32.rktw", "weights_int8_pc.rktw"}) {
        char path[4096];
        snprintf(path, sizeof path, "%s/%s", dir, name);
        std::vector<uint8_t> blob = slurp(path);
        CHECK(blob.size() > 64);
        if (blob.size() <= 64) continue;
        rocket_weights_info info;
        CHECK(rocket_weights_info_read(blob.data(), blob.size(), &info) == 0);
        // every truncation and every single-bit flip is refused, and nothing reads past the end
        for (size_t len = 0; len < blob.size(); len += (len < 80 ? 1 : 97)) {
            std::vector<uint8_t> t(blob.begin(), blob.begin() + len);
            CHECK(rocket_weights_info_read(t.empty() ? nullptr : t.data(), t.size(), &info) != 0);
        }
        for (size_t pos = 0; pos < blob.size(); pos += (pos < 64 ? 1 : 131)) {
            std::vector<uint8_t> t = blob;
            t[pos] ^= 0x20;
            CHECK(rocket_weights_info_read(t.data(), t.size(), &info) != 0);
        }
    }
}

static void host_references()
{
    // gated FFN, GEGLU and MLP (fd < 0), against the oracle bit for bit
    const int M = 4, Hd = 64, I = 96;
    auto x = f16v((size_t)M * Hd, 71, -1, 1), wg = f16v((size_t)I * Hd, 72, -0.3f, 0.3f),
         wu = f16v((size_t)I * Hd, 73, -0.3f, 0.3f), wd = f16v((size_t)Hd * I, 74, -0.15f, 0.15f),
         b1 = f16v(I, 75, -1, 1);
    for (int kind : {ROCKET_ACTIVATION_SILU, ROCKET_ACTIVATION_GELU}) {
        std::vector<uint16_t> got((size_t)M * Hd), want((size_t)M * Hd);
        rocket_ffn_ref_fp16(M, Hd, I, H(x), H(wg), H(wu), H(wd), kind, H(got));
        rko_ffn_f16(M, Hd, I, x.data(), wg.data(), wu.data(), wd.data(), kind, want.data());
        CHECK(got == want);
        CHECK(rocket_ffn_fp16(-1, M, Hd, I, H(x), H(wg), H(wu), H(wd), kind, H(got)) == 0 && got == want);
        std::vector<uint16_t> p(I), pw(I);
        rocket_geglu_ref_fp16(H(wg), H(wu), kind, H(p), I);
        rko_geglu_f16(wg.data(), wu.data(), kind, pw.data(), I);
        CHECK(p == pw);
        for (bool bias : {false, true}) {
            std::vector<uint16_t> o((size_t)M * Hd), ow((size_t)M * Hd);
            CHECK(rocket_mlp_fp16_fused(-1, M, Hd, I, Hd, H(x), H(wg), bias ? H(b1) : nullptr, H(wd), kind, H(o)) == 0);
            rko_mlp_f16(M, Hd, I, Hd, x.data(), wg.data(), bias ? b1.data() : nullptr, wd.data(), kind, ow.data());
            CHECK(o == ow);
        }
    }
    // flash attention (grouped heads, mask, soft-cap) and self-attention
    const int nh = 4, nkvh = 2, T = 21, nkv = 37, dk = 64, dv = 32;
    auto Q = f16v((size_t)nh * T * dk, 81, -1, 1), K = f16v((size_t)nkvh * nkv * dk, 82, -1, 1),
         V = f16v((size_t)nkvh * dv * nkv, 83, -1, 1), mask = f16v((size_t)T * nkv, 84, -3, 0);
    for (float cap : {0.0f, 20.0f}) {
        std::vector<uint16_t> o((size_t)nh * T * dv), ow((size_t)nh * T * dv);
        CHECK(rocket_flash_attn_fp16(-1, T, nkv, dk, dv, nh, nkvh, 0.125f, cap, H(Q), H(K), H(V), H(mask), H(o)) == 0);
        rko_flash_attn_f16(T, nkv, dk, dv, nh, nkvh, 0.125f, cap, Q.data(), K.data(), V.data(), mask.data(), ow.data());
        CHECK(o == ow);
    }
    const int Ts = 19, d = 64, heads = 2;
    auto xs = f16v((size_t)Ts * d, 91, -1, 1);
    std::vector<std::vector<uint16_t>> W, B;
    for (int i = 0; i < 4; i++) {
        W.push_back(f16v((size_t)d * d, 92 + i, -0.1f, 0.1f));
        B.push_back(f16v(d, 96 + i, -0.1f, 0.1f));
    }
    std::vector<uint16_t> o((size_t)Ts * d), ow((size_t)Ts * d);
    CHECK(rocket_mha_self_fp16(-1, Ts, d, heads, H(xs), H(W[0]), H(B[0]), H(W[1]), nullptr, H(W[2]), H(B[2]), H(W[3]),
                               H(B[3]), H(o)) == 0);
    rko_mha_self_f16(Ts, d, heads, xs.data(), W[0].data(), B[0].data(), W[1].data(), nullptr, W[2].data(), B[2].data(),
                     W[3].data(), B[3].data(), ow.data());
    CHECK(o == ow);
}

// Handle-table entry points from several threads at once (no GPU here: rocket_open fails and
// every call on a missing handle is refused); the sanitizers watch the table and log locks.
static void threads()
{
    std::vector<std::thread> ts;
    std::atomic<int> bad{0};
    for (int t = 0; t < 4; t++)
        ts.emplace_back([&bad, t] {
            std::vector<int8_t> a(64 * 256), b(128 * 256);
            std::vector<int32_t> c(64 * 128);
            for (int i = 0; i < 200; i++) {
                const int fd = rocket_open();
                if (fd >= 0) rocket_close(fd);
                if (rocket_matmul_int8(200 + t, 64, 256, 128, a.data(), b.data(), c.data()) != ROCKET_E_DEVICE) bad++;
                rocket_close(200 + t);
                rocket_submit_counters_reset();
                (void)rocket_submit_ioctl_count();
            }
        });
    for (auto &t : ts) t.join();
    CHECK(bad.load() == 0);
}

int main(int argc, char **argv)
{
    const char *golden = argc > 1 ? argv[1] : "tests/golden";
    planners();
    rejections();
    logs_and_profiles();
    weights_reader(golden);
    host_references();
    threads();
    rocket_log_set_callback(nullptr, nullptr);
    if (g_fail) {
        fprintf(stderr, "shim_check: %d check(s) failed\n", g_fail);
        return 1;
    }
    printf("shim_check: all checks passed\n");
    return 0;
}
