// The reference's production decode attention as one call over the 8-bit pool: fn::qsa::attn::attend
// (fn/kernels/qsa/attend.h:57-141). For B <= 5 rows of one sequence it prepares each row's query heads and its new
// cell's k (F32 RMS norm and IMROPE, attend.cu:151-198, the rule of imrope.cuh:14-20), writes the new cells' K and V
// into the pool in the pool's 8-bit format, attends each row over its selection body (the sparse launch,
// sparse.hip), and finishes each (row, head) with the sigmoid gate into F32 and FNFL's int8 activation format
// (attend.cu:619-655, act_warp.cuh:12-37), all in stream order:
//   1. qsa_prepare_kernel: a wave a (row, query head) or (row, KV head): q as fp16 (the attention's operand; the exact
//      1/16 is applied as the score scale), k as F32 for the new-cell quantizer;
//   2. the sparse decode launch, its new cells from that F32 k and the caller's F32 v;
//   3. the merge with the gated epilogue.
// Differences from the reference's kernel: the query operand is fp16 (the reference keeps q in F32; the attention is
// held to the same 2e-3 bound as every other launch here), depth is a host value, and the cache is the paged pool.
#include "../../include/fnkv.h"
#include "common.h"
#include "decode_common.h"
#include "rope.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <string>

namespace fnkv {
namespace {

constexpr int32_t kQStride = 512; // qfull: [q | gate] a head (attend.h:54)

struct qsa_prep_args {
    const float * qfull;
    const float * kv_k;
    const float * q_norm;
    const float * k_norm;
    const int32_t * pos;
    float theta_scale;
    int32_t T, hq, h_kv;
    uint16_t * q16;  // [T][hq][256]
    float * k_rope;  // [T][h_kv][256]
    float * q_f32;   // optional [T][hq][256]
    float * k_f32;   // optional [T][h_kv][256]
};

__global__ __launch_bounds__(64) void qsa_prepare_kernel(qsa_prep_args a) {
    const int32_t t = static_cast<int32_t>(blockIdx.x), r = static_cast<int32_t>(blockIdx.y);
    const int32_t lane = static_cast<int32_t>(threadIdx.x);
    float y[4];
    if (r < a.hq) {
        norm_rope(y, a.qfull + (t * a.hq + r) * kQStride, a.q_norm, a.pos, a.T, t, a.theta_scale, lane);
        const int32_t o = (t * a.hq + r) * 256;
        if (a.q_f32 != nullptr) {
            reinterpret_cast<float4 *>(a.q_f32 + o)[lane] = make_float4(y[0], y[1], y[2], y[3]);
        }
        reinterpret_cast<uint2 *>(a.q16 + o)[lane] = pack4_f16(y, 1.0f);
        return;
    }
    const int32_t kvh = r - a.hq;
    norm_rope(y, a.kv_k + (t * a.h_kv + kvh) * 256, a.k_norm, a.pos, a.T, t, a.theta_scale, lane);
    const int32_t o = (t * a.h_kv + kvh) * 256;
    reinterpret_cast<float4 *>(a.k_rope + o)[lane] = make_float4(y[0], y[1], y[2], y[3]);
    if (a.k_f32 != nullptr) {
        reinterpret_cast<float4 *>(a.k_f32 + o)[lane] = make_float4(y[0], y[1], y[2], y[3]);
    }
}

int64_t up16(int64_t x) { return (x + 15) & ~int64_t(15); }

// rows a launch takes: G * rows <= FNKV_MAX_ROWS (the reference's card, 12 heads on one KV head, serves 5 rows as 4 + 1)
int32_t rows_per_launch(int32_t G) { return G >= FNKV_MAX_ROWS ? 1 : FNKV_MAX_ROWS / G; }

// words of row t's body (qsa.h:77-81): 2 + K + tail for the row at position q = depth + t
int64_t body_words(int64_t q) {
    const int64_t n_vis = (q + 1) / 4;
    return 2 + (n_vis < 512 ? n_vis : 512) + (q + 1 - 4 * n_vis);
}

// the sparse workspace the largest of the row launches needs
int64_t sparse_ws_max(const fnkv_pool * pool, int64_t depth, int32_t T, int32_t hq, int32_t G) {
    const int32_t per = rows_per_launch(G);
    int64_t need = 0;
    for (int32_t c0 = 0; c0 < T; c0 += per) {
        const int64_t b = fnkv_sparse_workspace_bytes(pool, depth + c0, T - c0 < per ? T - c0 : per, hq);
        if (b < 0) {
            return -1;
        }
        need = b > need ? b : need;
    }
    return need;
}

bool aligned16(const void * p) { return p != nullptr && (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

} // namespace
} // namespace fnkv

using fnkv::set_error;

extern "C" {

int64_t fnkv_qsa_workspace_bytes(const fnkv_pool * pool, int64_t depth, int32_t T, int32_t hq) {
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    if (p == nullptr || T <= 0 || T > FNKV_DATC_MAX_ROWS || hq <= 0 || hq % p->h_kv() != 0) {
        return -1;
    }
    const int64_t sp = fnkv::sparse_ws_max(pool, depth, T, hq, hq / p->h_kv());
    if (sp < 0) {
        return -1;
    }
    return fnkv::up16(sp) + fnkv::up16(int64_t(T) * hq * 256 * 2) + int64_t(T) * p->h_kv() * 256 * 4;
}

int fnkv_qsa_attend(const fnkv_pool * pool, int32_t slot, int64_t depth, int32_t T, int32_t layer, int32_t hq,
                    const float * qfull, const float * kv_k, const float * kv_v, const float * q_norm,
                    const float * k_norm, const int32_t * pos, float theta_scale, const void * body,
                    const void * offsets, float * out, int8_t * codes, float * scales, float * q_f32, float * k_f32,
                    void * ws, int64_t ws_bytes, void * stream) {
    using fnkv::aligned16;
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    const int64_t need = fnkv_qsa_workspace_bytes(pool, depth, T, hq);
    if (p == nullptr || need < 0 || !aligned16(qfull) || !aligned16(kv_k) || !aligned16(kv_v) || !aligned16(q_norm) ||
        !aligned16(k_norm) || pos == nullptr || (reinterpret_cast<uintptr_t>(pos) & 3) != 0 || !aligned16(out) ||
        codes == nullptr || (reinterpret_cast<uintptr_t>(codes) & 3) != 0 || scales == nullptr ||
        (reinterpret_cast<uintptr_t>(scales) & 7) != 0 || (q_f32 != nullptr && !aligned16(q_f32)) ||
        (k_f32 != nullptr && !aligned16(k_f32)) || !aligned16(ws) || !std::isfinite(theta_scale)) {
        set_error("fnkv_qsa_attend: argument outside the contract");
        return FNKV_ERR_ARG;
    }
    if (ws_bytes < need) {
        set_error("fnkv_qsa_attend: workspace too small (fnkv_qsa_workspace_bytes)");
        return FNKV_ERR_ARG;
    }
    const int32_t G = hq / p->h_kv();
    const int64_t sp = fnkv::up16(fnkv::sparse_ws_max(pool, depth, T, hq, G));
    uint8_t * w = static_cast<uint8_t *>(ws);
    uint16_t * q16 = reinterpret_cast<uint16_t *>(w + sp);
    float * k_rope = reinterpret_cast<float *>(w + sp + fnkv::up16(int64_t(T) * hq * 256 * 2));
    hipStream_t st = static_cast<hipStream_t>(stream);
    // every check of the sparse launches is made here too, before the prepare is enqueued: a refusal enqueues nothing
    fnkv::sparse_gate gate = {qfull + 256, 512, out, codes, scales};
    fnkv::qsa_prep_args pa = {qfull, kv_k, q_norm, k_norm, pos, theta_scale, T, hq, p->h_kv(), q16, k_rope, q_f32,
                              k_f32};
    if (T <= 0 || T > fnkv::kSelMaxRows || depth < 0 || layer < 0 || layer >= p->layers() || slot < 0 ||
        slot >= p->pages().n_slots() || depth + T > p->mapped_cells(slot) || depth + T > fnkv::kSelMaxCells ||
        G > FNKV_MAX_ROWS || body == nullptr ||
        offsets == nullptr || (reinterpret_cast<uintptr_t>(body) & 3) != 0 ||
        (reinterpret_cast<uintptr_t>(offsets) & 3) != 0) {
        set_error("fnkv_qsa_attend: rows, heads, layer or cells outside the contract");
        return FNKV_ERR_ARG;
    }
    hipLaunchKernelGGL(fnkv::qsa_prepare_kernel, dim3(static_cast<uint32_t>(T), static_cast<uint32_t>(hq + p->h_kv())),
                       dim3(64), 0, st, pa);
    // rows in launches of at most FNKV_MAX_ROWS query rows a KV head, in order: a later launch's rows see the earlier
    // rows' new cells (stream order), each row's body starts where the previous rows' words end
    const int32_t per = fnkv::rows_per_launch(G);
    const uint32_t * bw = static_cast<const uint32_t *>(body);
    for (int32_t c0 = 0; c0 < T; c0 += per) {
        const int32_t tc = T - c0 < per ? T - c0 : per;
        const int64_t hk = int64_t(p->h_kv()) * 256;
        fnkv::sparse_gate gc = {gate.gate + int64_t(c0) * hq * 512, 512, out + int64_t(c0) * hq * 256,
                                codes + int64_t(c0) * hq * 256, scales + int64_t(c0) * hq * 16};
        const int rc = fnkv::sparse_launch(p, slot, depth + c0, tc, layer, hq, 1.0f / 16.0f,
                                           q16 + int64_t(c0) * hq * 256, bw, offsets, k_rope + c0 * hk,
                                           kv_v + c0 * hk, FNKV_F32, nullptr, &gc, ws, sp, st, "fnkv_qsa_attend");
        if (rc != FNKV_OK) {
            return rc;
        }
        for (int32_t t = c0; t < c0 + tc; ++t) {
            bw += fnkv::body_words(depth + t);
        }
    }
    return FNKV_OK;
}

} // extern "C"
