// A C++ host harness that drives the C-ABI the way the reference's engine drives its KV8 path, with no Python on the
// path: the engine's cell reservation with its reclaim retry (fn/runtime/runtime.cpp:1483-1537 engine::ensure_cells /
// reclaim over kv_pages and kv_reclaim_victim), the prompt chunk's append (prompt.cpp:2653-2700 -> qsp_kv), and the
// decode step of every full-attention layer (layer.cpp:660-695 -> attn::attend with the depth on the device, one
// captured graph replayed while the context advances; attend.h:108). It checks what the engine relies on and exits
// non-zero on any mismatch:
//   * reservation: a slot that does not fit makes the engine reclaim the least recently released idle slot and retry;
//     the active slots keep their pages;
//   * decode: every replay of the one captured graph (device contexts advancing by T, new cells written by the
//     launch) gives outputs bitwise equal to the same launch run eagerly on a second pool holding the same cells, and
//     within 1e-3 plus one fp16 ulp of fnkv_attn_decode at the same host contexts (a different split of the cells:
//     fp32 sums in another order, so an output may round to the neighbouring fp16 value);
//   * a context past the bound: nothing written, the refused-depth bit set, the other sequences unchanged.
// Usage: engine_step [steps] (default 8). Prints one line a phase and "engine_step ok".
#include "fnkv.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

constexpr int32_t kD = FNKV_HEAD_DIM;
constexpr int32_t kHq = 16, kHkv = 2, kLayers = 2, kT = 3;

#define HIP_CHECK(x)                                                                                               \
    do {                                                                                                           \
        const hipError_t e_ = (x);                                                                                 \
        if (e_ != hipSuccess) {                                                                                    \
            std::fprintf(stderr, "%s:%d: %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_));                 \
            std::exit(2);                                                                                          \
        }                                                                                                          \
    } while (0)

#define FN_CHECK(x)                                                                                                \
    do {                                                                                                           \
        const int rc_ = (x);                                                                                       \
        if (rc_ != FNKV_OK) {                                                                                      \
            std::fprintf(stderr, "%s:%d: %s: status %d: %s\n", __FILE__, __LINE__, #x, rc_, fnkv_last_error());     \
            std::exit(3);                                                                                          \
        }                                                                                                          \
    } while (0)

[[noreturn]] void fail(const std::string & what) {
    std::fprintf(stderr, "engine_step: FAILED: %s\n", what.c_str());
    std::exit(1);
}

// seeded fp16 values ~ U(-2, 2) (a few channels x8, as BASELINE's K/V outliers)
std::vector<_Float16> rows16(uint64_t seed, size_t n) {
    std::vector<_Float16> v(n);
    uint64_t x = seed * 0x9E3779B97F4A7C15ull + 1;
    for (size_t i = 0; i < n; ++i) {
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        float f = static_cast<float>((x >> 40) & 0xFFFF) / 16384.0f - 2.0f;
        if (i % kD == 3 || i % kD == 77) {
            f *= 8.0f;
        }
        v[i] = static_cast<_Float16>(f);
    }
    return v;
}

template <typename T> T * to_device(const std::vector<T> & h) {
    T * d = nullptr;
    HIP_CHECK(hipMalloc(&d, h.size() * sizeof(T)));
    HIP_CHECK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
}

// The engine's slot bookkeeping (runtime.cpp's s_[i].busy / released) and its ensure_cells: reserve, and when the
// pool is full reclaim the least recently released idle slot (kv_reclaim_victim) and retry.
struct engine_slots {
    fnkv_pool * pool;
    std::vector<int32_t> active;
    std::vector<uint64_t> released;
    uint64_t clock = 0;
    int32_t reclaims = 0;

    bool ensure_cells(int32_t slot, int64_t cells) {
        for (;;) {
            int32_t full = 0;
            const int rc = fnkv_pool_ensure(pool, slot, cells, &full);
            if (rc == FNKV_OK) {
                return true;
            }
            if (!full) {
                fail(std::string("ensure: ") + fnkv_last_error());
            }
            std::vector<fnkv_slot_view> v(active.size());
            for (size_t i = 0; i < v.size(); ++i) {
                v[i].active = active[i];
                v[i].pages = fnkv_pool_mapped_pages(pool, static_cast<int32_t>(i));
                v[i].released = released[i];
            }
            const int32_t victim = fnkv_reclaim_victim(v.data(), static_cast<int32_t>(v.size()), slot);
            if (victim < 0) {
                return false;
            }
            FN_CHECK(fnkv_pool_trim(pool, victim, 0));
            ++reclaims;
        }
    }
    void release(int32_t slot) {
        active[size_t(slot)] = 0;
        released[size_t(slot)] = ++clock;
    }
};

} // namespace

int main(int argc, char ** argv) {
    const int32_t steps = argc > 1 ? std::atoi(argv[1]) : 8;
    if (steps < 1 || steps > 64) {
        fail("steps must be 1 .. 64");
    }
    int n_dev = 0;
    HIP_CHECK(hipGetDeviceCount(&n_dev));
    if (n_dev < 1) {
        fail("no GPU");
    }
    HIP_CHECK(hipSetDevice(0));

    // ---- reservation with reclaim: 6 slots, a pool too small for all of them at once ----
    const std::vector<int64_t> ctx0 = {3000, 9000 + 17, 20000 + 5}; // the decoding sequences' contexts at step 0
    std::vector<int64_t> cap(ctx0.size());
    int32_t need = 0;
    for (size_t i = 0; i < ctx0.size(); ++i) {
        cap[i] = ctx0[i] + int64_t(kT) * steps;
        need += fnkv_pages_for(cap[i], FNKV_PAGE_TOKENS, INT32_MAX);
    }
    const int32_t n_slots = 6, n_pages = need + 24;
    fnkv_pool * pool = nullptr;
    FN_CHECK(fnkv_pool_create(n_slots, n_pages, FNKV_PAGE_TOKENS, kLayers, kHkv, 0, 0, &pool));
    engine_slots es{pool, std::vector<int32_t>(n_slots, 0), std::vector<uint64_t>(n_slots, 0)};
    // three finished sequences hold most of the pool (released in order 3, 5, 4), then the three live ones reserve
    for (int32_t s : {3, 5, 4}) {
        es.active[size_t(s)] = 1;
        if (!es.ensure_cells(s, int64_t(n_pages / 3) * FNKV_PAGE_TOKENS)) {
            fail("filler reservation");
        }
        es.release(s);
    }
    for (int32_t s = 0; s < 3; ++s) {
        es.active[size_t(s)] = 1;
        if (!es.ensure_cells(s, cap[size_t(s)])) {
            fail("live reservation " + std::to_string(s));
        }
    }
    if (es.reclaims < 1 || fnkv_pool_mapped_pages(pool, 3) != 0) {
        fail("the pool should have reclaimed slot 3 (released first) before the others");
    }
    std::printf("reservation: %d reclaim(s), slot 3 reclaimed first, %d of %d pages free\n", es.reclaims,
                fnkv_pool_free_pages(pool), n_pages);

    // a second pool holding the same cells: the eager reference launches run there
    fnkv_pool * twin = nullptr;
    FN_CHECK(fnkv_pool_create(4, need + 8, FNKV_PAGE_TOKENS, kLayers, kHkv, 0, 0, &twin));
    for (int32_t s = 0; s < 3; ++s) {
        FN_CHECK(fnkv_pool_ensure(twin, s, cap[size_t(s)], nullptr));
    }

    // ---- the prompt: every sequence's cells before the first decode step, each layer (qsp_kv's role) ----
    hipStream_t st;
    HIP_CHECK(hipStreamCreate(&st));
    std::vector<void *> frees;
    for (int32_t s = 0; s < 3; ++s) {
        const int32_t rows = static_cast<int32_t>(ctx0[size_t(s)] - kT);
        for (int32_t layer = 0; layer < kLayers; ++layer) {
            _Float16 * k = to_device(rows16(1000 + 10 * s + layer, size_t(rows) * kHkv * kD));
            _Float16 * v = to_device(rows16(2000 + 10 * s + layer, size_t(rows) * kHkv * kD));
            FN_CHECK(fnkv_q8_append(pool, s, layer, 0, rows, k, v, FNKV_F16, st));
            FN_CHECK(fnkv_q8_append(twin, s, layer, 0, rows, k, v, FNKV_F16, st));
            frees.push_back(k);
            frees.push_back(v);
        }
    }
    HIP_CHECK(hipStreamSynchronize(st));
    std::printf("prompt: %d sequences x %d layers appended\n", 3, kLayers);

    // ---- decode: one graph over every layer, the contexts on the device ----
    const int32_t n_seq = 3;
    const int32_t slots[3] = {0, 1, 2};
    const size_t q_elems = size_t(n_seq) * kT * kHq * kD, kv_elems = size_t(n_seq) * kT * kHkv * kD;
    const int64_t ws_bytes = fnkv_decode_workspace_bytes(pool, n_seq, cap.data(), kT, kHq);
    if (ws_bytes <= 0) {
        fail("workspace size");
    }
    // the host-context launches plan their own splits: their workspace is the largest over the steps
    int64_t ws_host = ws_bytes;
    for (int32_t step = 0; step < steps; ++step) {
        std::vector<int64_t> c(ctx0);
        for (auto & x : c) {
            x += int64_t(kT) * step;
        }
        const int64_t b = fnkv_decode_workspace_bytes(twin, n_seq, c.data(), kT, kHq);
        ws_host = b > ws_host ? b : ws_host;
    }
    void * ws = nullptr;
    void * ws_twin = nullptr;
    int64_t * ctx_dev = nullptr;
    uint32_t * err = nullptr;
    _Float16 *q = nullptr, *kn = nullptr, *vn = nullptr, *out = nullptr, *out_ref = nullptr;
    HIP_CHECK(hipMalloc(&ws, ws_bytes));
    HIP_CHECK(hipMalloc(&ws_twin, ws_host));
    // the workspaces start zeroed once (their fold counters; every launch leaves them at zero)
    HIP_CHECK(hipMemset(ws, 0, ws_bytes));
    HIP_CHECK(hipMemset(ws_twin, 0, ws_host));
    HIP_CHECK(hipMalloc(&ctx_dev, sizeof(int64_t) * n_seq));
    HIP_CHECK(hipMalloc(&err, sizeof(uint32_t)));
    HIP_CHECK(hipMalloc(&q, sizeof(_Float16) * q_elems * kLayers));
    HIP_CHECK(hipMalloc(&kn, sizeof(_Float16) * kv_elems * kLayers));
    HIP_CHECK(hipMalloc(&vn, sizeof(_Float16) * kv_elems * kLayers));
    HIP_CHECK(hipMalloc(&out, sizeof(_Float16) * q_elems * kLayers));
    HIP_CHECK(hipMalloc(&out_ref, sizeof(_Float16) * q_elems * kLayers));
    const float scale = 1.0f / 16.0f;
    auto decode_all_layers = [&](fnkv_pool * p, _Float16 * o, void * w) {
        for (int32_t layer = 0; layer < kLayers; ++layer) {
            FN_CHECK(fnkv_attn_decode_dev(p, n_seq, slots, ctx_dev, cap.data(), kT, layer, kHq, scale,
                                          q + layer * q_elems, kn + layer * kv_elems, vn + layer * kv_elems,
                                          FNKV_F16, o + layer * q_elems, w, ws_bytes, err, st));
        }
    };
    // the step's inputs (q and the new rows) and the device contexts are written before each replay
    auto set_step = [&](int32_t step, const int64_t * ctx) {
        for (int32_t layer = 0; layer < kLayers; ++layer) {
            const std::vector<_Float16> hq = rows16(50000 + 100 * step + layer, q_elems);
            const std::vector<_Float16> hk = rows16(60000 + 100 * step + layer, kv_elems);
            const std::vector<_Float16> hv = rows16(70000 + 100 * step + layer, kv_elems);
            HIP_CHECK(hipMemcpyAsync(q + layer * q_elems, hq.data(), hq.size() * 2, hipMemcpyHostToDevice, st));
            HIP_CHECK(hipMemcpyAsync(kn + layer * kv_elems, hk.data(), hk.size() * 2, hipMemcpyHostToDevice, st));
            HIP_CHECK(hipMemcpyAsync(vn + layer * kv_elems, hv.data(), hv.size() * 2, hipMemcpyHostToDevice, st));
        }
        HIP_CHECK(hipMemcpyAsync(ctx_dev, ctx, sizeof(int64_t) * n_seq, hipMemcpyHostToDevice, st));
        HIP_CHECK(hipMemsetAsync(err, 0, sizeof(uint32_t), st));
        HIP_CHECK(hipStreamSynchronize(st)); // the host buffers above go out of scope
    };

    std::vector<int64_t> ctx(ctx0);
    set_step(0, ctx.data());
    decode_all_layers(pool, out, ws); // once eagerly (the library's one-time set-up), then captured
    HIP_CHECK(hipStreamSynchronize(st));
    hipGraph_t graph;
    hipGraphExec_t exec;
    HIP_CHECK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    decode_all_layers(pool, out, ws);
    HIP_CHECK(hipStreamEndCapture(st, &graph));
    HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));

    std::vector<uint16_t> got(q_elems * kLayers), want(q_elems * kLayers), host(q_elems * kLayers);
    float worst = 0.0f;
    hipEvent_t e0, e1;
    HIP_CHECK(hipEventCreate(&e0));
    HIP_CHECK(hipEventCreate(&e1));
    float graph_ms = 0.0f;
    for (int32_t step = 0; step < steps; ++step) {
        set_step(step, ctx.data());
        HIP_CHECK(hipEventRecord(e0, st));
        HIP_CHECK(hipGraphLaunch(exec, st));
        HIP_CHECK(hipEventRecord(e1, st));
        HIP_CHECK(hipStreamSynchronize(st));
        float ms = 0.0f;
        HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
        graph_ms += ms;
        uint32_t herr = 0;
        HIP_CHECK(hipMemcpy(&herr, err, sizeof(herr), hipMemcpyDeviceToHost));
        if (herr != 0) {
            fail("step " + std::to_string(step) + ": error word " + std::to_string(herr));
        }
        HIP_CHECK(hipMemcpy(got.data(), out, got.size() * 2, hipMemcpyDeviceToHost));
        // the same launches eagerly on the twin pool (their new cells written by the launch too): bitwise
        decode_all_layers(twin, out_ref, ws_twin);
        HIP_CHECK(hipStreamSynchronize(st));
        HIP_CHECK(hipMemcpy(want.data(), out_ref, want.size() * 2, hipMemcpyDeviceToHost));
        if (std::memcmp(got.data(), want.data(), got.size() * 2) != 0) {
            fail("step " + std::to_string(step) + ": graph replay differs from the eager launch");
        }
        // the host-context launch (its own split plan; it rewrites the same new cells): within 1e-3
        for (int32_t layer = 0; layer < kLayers; ++layer) {
            FN_CHECK(fnkv_attn_decode(twin, n_seq, slots, ctx.data(), kT, layer, kHq, scale, q + layer * q_elems,
                                      kn + layer * kv_elems, vn + layer * kv_elems, FNKV_F16,
                                      out_ref + layer * q_elems, ws_twin, ws_host, st));
        }
        HIP_CHECK(hipStreamSynchronize(st));
        HIP_CHECK(hipMemcpy(host.data(), out_ref, host.size() * 2, hipMemcpyDeviceToHost));
        bool close = true;
        for (size_t i = 0; i < host.size(); ++i) {
            _Float16 a, b;
            std::memcpy(&a, &got[i], 2);
            std::memcpy(&b, &host[i], 2);
            const float fa = static_cast<float>(a), fb = static_cast<float>(b);
            const float d = std::fabs(fa - fb);
            const float ulp = std::ldexp(1.0f, std::ilogb(std::fmax(std::fabs(fb), 6.1e-5f)) - 10); // fp16 spacing
            close = close && d <= 1e-3f + ulp;
            worst = d - ulp > worst ? d - ulp : worst;
        }
        if (!close) {
            fail("step " + std::to_string(step) + ": device-context and host-context launches differ by " +
                 std::to_string(worst) + " beyond one fp16 ulp");
        }
        for (auto & c : ctx) {
            c += kT;
        }
    }
    std::printf("decode: %d steps of one graph (%d layers, T = %d, contexts %lld/%lld/%lld at step 0), each bitwise "
                "the eager launch, within %.2e (beyond one fp16 ulp) of the host-context launch; %.1f us a step\n",
                steps, kLayers, kT, static_cast<long long>(ctx0[0]), static_cast<long long>(ctx0[1]),
                static_cast<long long>(ctx0[2]), worst, 1000.0f * graph_ms / steps);

    // ---- a context past its bound: nothing written for that sequence, the refused-depth bit set ----
    std::vector<int64_t> bad(ctx0);
    bad[1] = cap[1] + 1;
    set_step(steps, bad.data());
    const std::vector<uint16_t> sentinel(q_elems * kLayers, 0x7E00); // fp16 NaN bits
    HIP_CHECK(hipMemcpy(out, sentinel.data(), sentinel.size() * 2, hipMemcpyHostToDevice));
    HIP_CHECK(hipGraphLaunch(exec, st));
    HIP_CHECK(hipStreamSynchronize(st));
    uint32_t herr = 0;
    HIP_CHECK(hipMemcpy(&herr, err, sizeof(herr), hipMemcpyDeviceToHost));
    HIP_CHECK(hipMemcpy(got.data(), out, got.size() * 2, hipMemcpyDeviceToHost));
    if ((herr & FNKV_DEV_ERR_DEPTH) == 0) {
        fail("a context past its bound did not set the refused-depth bit");
    }
    const size_t per_seq = size_t(kT) * kHq * kD;
    for (int32_t layer = 0; layer < kLayers; ++layer) {
        for (int32_t s = 0; s < n_seq; ++s) {
            const uint16_t * o = got.data() + layer * q_elems + s * per_seq;
            bool untouched = true, written = true;
            for (size_t i = 0; i < per_seq; ++i) {
                untouched = untouched && o[i] == 0x7E00;
                written = written && o[i] != 0x7E00;
            }
            if (s == 1 ? !untouched : !written) {
                fail("refused launch: sequence " + std::to_string(s) + " layer " + std::to_string(layer));
            }
        }
    }
    std::printf("refusal: error word %u, the refused sequence's rows untouched, the others written\n", herr);

    // ---- the engine finishes: the live sequences' pages back to the pool ----
    for (int32_t s = 0; s < 3; ++s) {
        es.release(s);
        FN_CHECK(fnkv_pool_trim(pool, s, 0));
    }
    if (fnkv_pool_free_pages(pool) != n_pages - fnkv_pool_mapped_pages(pool, 4) - fnkv_pool_mapped_pages(pool, 5)) {
        fail("free pages after the trims");
    }
    HIP_CHECK(hipGraphExecDestroy(exec));
    HIP_CHECK(hipGraphDestroy(graph));
    for (void * p : frees) {
        HIP_CHECK(hipFree(p));
    }
    for (void * p : {static_cast<void *>(ws), ws_twin, static_cast<void *>(ctx_dev), static_cast<void *>(err),
                     static_cast<void *>(q), static_cast<void *>(kn), static_cast<void *>(vn),
                     static_cast<void *>(out), static_cast<void *>(out_ref)}) {
        HIP_CHECK(hipFree(p));
    }
    HIP_CHECK(hipEventDestroy(e0));
    HIP_CHECK(hipEventDestroy(e1));
    HIP_CHECK(hipStreamDestroy(st));
    fnkv_pool_destroy(twin);
    fnkv_pool_destroy(pool);
    std::printf("engine_step ok\n");
    return 0;
}
