// The reference's production decode attention as one call over the 8-bit pool: fn::qsa::attn::attend
// (fn/kernels/qsa/attend.h:57-141). For B <= 5 rows of one sequence it prepares each row's query heads and its new
// cell's k (F32 RMS norm and IMROPE, attend.cu:151-198, the rule of imrope.cuh:14-20), writes the new cells' K and V
// into the pool in the pool's 8-bit format, attends each row over its selection body (the sparse launch,
// sparse.hip), and finishes each (row, head) with the sigmoid gate into F32 and FNFL's int8 activation format
// (attend.cu:619-655, act_warp.cuh:12-37), all in stream order:
//   1. qsa_prepare_kernel: a wave a (row, query head) or (row, KV head): q as fp16 hi + lo (the attention's operands,
//      about 22 significant bits of the F32 q; the exact 1/16 is applied as the score scale); the new cell's K (the
//      normed, roped k) and V quantized into the pool;
//   2. the sparse decode launch (each row its own splits);
//   3. the merge with the gated epilogue.
// At most 16 query heads a KV head skip step 1: the sparse launch forms each row's query heads in LDS while the row's
// selection builds, and every workgroup that reads a new cell's tile writes that cell first (a row's own cell also
// by its owner when no workgroup reads it; fused_prep, decode.hip). Workgroups that write the same cell store the same
// bytes, and the arithmetic is the prepare kernel's, so the outputs are bitwise those of the three launches.
// Differences from the reference's kernel: the query enters the matrix cores as two fp16 parts (the reference keeps q
// in F32; hi + lo carries it to about 2^-22 relative, and the output meets the reference checker's 1e-5 normalized
// bound, qa2_test.cpp:58), depth is a host value, and the cache is the paged pool.
#include "../../include/fnkv.h"
#include "common.h"
#include "decode_common.h"
#include "rope.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <string>

namespace fnkv {
namespace {

constexpr int32_t kQStride = 512; // qfull: [q | gate] a head (attend.h:54)

struct qsa_prep_args {
    pool_view pv;
    const int32_t * table; // the slot's page table
    int32_t layer;
    int64_t depth;
    const int32_t * depth_dev; // set: the depth is this device word, and depth + T <= max_cells or nothing is written
    int64_t max_cells;
    const float * qfull;
    const float * kv_k;
    const float * kv_v;
    const float * q_norm;
    const float * k_norm;
    const int32_t * pos;
    float theta_scale;
    int32_t T, hq, h_kv;
    uint16_t * q16;  // [T][hq][256]
    uint16_t * q16_lo; // [T][hq][256]: fp16(q - q16), the operand's low parts
    float * q_f32;   // optional [T][hq][256]
    float * k_f32;   // optional [T][h_kv][256]
};

__global__ __launch_bounds__(64) void qsa_prepare_kernel(qsa_prep_args a) {
    if (a.depth_dev != nullptr) {
        a.depth = *a.depth_dev;
        if (a.depth < 0 || a.depth + a.T > a.max_cells) {
            return; // the attention's launch reports the refusal
        }
    }
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
        float lo[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            lo[e] = y[e] - static_cast<float>(static_cast<_Float16>(y[e]));
        }
        reinterpret_cast<uint2 *>(a.q16_lo + o)[lane] = pack4_f16(lo, 1.0f);
        return;
    }
    // the row's new cell: K (normed, roped) and V in the pool's format at depth + t
    const int32_t kvh = r - a.hq;
    norm_rope(y, a.kv_k + (t * a.h_kv + kvh) * 256, a.k_norm, a.pos, a.T, t, a.theta_scale, lane);
    const int32_t o = (t * a.h_kv + kvh) * 256;
    if (a.k_f32 != nullptr) {
        reinterpret_cast<float4 *>(a.k_f32 + o)[lane] = make_float4(y[0], y[1], y[2], y[3]);
    }
    const int64_t pos = a.depth + t;
    uint8_t * tile = tile_of(a.pv, a.table, a.layer, kvh, pos);
    quantize_store_fmt(y, lane, tile, static_cast<int32_t>(pos & 31), 0, a.pv.format);
    float v[4];
    load4<true>(a.kv_v + o, lane, v);
    quantize_store_fmt(v, lane, tile, static_cast<int32_t>(pos & 31), 1, a.pv.format);
}

int64_t up16(int64_t x) { return (x + 15) & ~int64_t(15); }

bool aligned16(const void * p) { return p != nullptr && (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

} // namespace

// attn::attend over the pool (the three launches, or two for one row of at most 16 query heads a KV head); dd set:
// the depth is read on the device, `depth` is ignored and the plan is dd->max_cells'
int qsa_launch(const fnkv_pool * pool, int32_t slot, int64_t depth, int32_t T, int32_t layer, int32_t hq,
               const float * qfull, const float * kv_k, const float * kv_v, const float * q_norm, const float * k_norm,
               const int32_t * pos, float theta_scale, const void * body, const void * offsets, float * out,
               int8_t * codes, float * scales, float * q_f32, float * k_f32, void * ws, int64_t ws_bytes,
               hipStream_t st, const dev_depth * dd, const char * who, bool check_only = false) {
    const std::string name(who);
    const kv_pool * p = pool_of(pool);
    if (dd != nullptr) {
        if (dd->depth == nullptr || dd->err == nullptr || (reinterpret_cast<uintptr_t>(dd->depth) & 3) != 0 ||
            (reinterpret_cast<uintptr_t>(dd->err) & 3) != 0 || T <= 0 || dd->max_cells < T) {
            set_error(name + ": the device depth and error words (4-byte aligned) and max_cells >= rows required");
            return FNKV_ERR_ARG;
        }
        depth = dd->max_cells - T;
    }
    const int64_t need = fnkv_qsa_workspace_bytes(pool, depth, T, hq);
    if (p == nullptr || need < 0 || !aligned16(qfull) || !aligned16(kv_k) || !aligned16(kv_v) || !aligned16(q_norm) ||
        !aligned16(k_norm) || pos == nullptr || (reinterpret_cast<uintptr_t>(pos) & 3) != 0 || !aligned16(out) ||
        codes == nullptr || (reinterpret_cast<uintptr_t>(codes) & 3) != 0 || scales == nullptr ||
        (reinterpret_cast<uintptr_t>(scales) & 7) != 0 || (q_f32 != nullptr && !aligned16(q_f32)) ||
        (k_f32 != nullptr && !aligned16(k_f32)) || !aligned16(ws) || !std::isfinite(theta_scale)) {
        set_error(name + ": argument outside the contract");
        return FNKV_ERR_ARG;
    }
    if (ws_bytes < need) {
        set_error(name + ": workspace too small");
        return FNKV_ERR_ARG;
    }
    const int32_t G = hq / p->h_kv();
    const int64_t sp = up16(fnkv_sparse_workspace_bytes(pool, depth, T, hq));
    uint8_t * w = static_cast<uint8_t *>(ws);
    uint16_t * q16 = reinterpret_cast<uint16_t *>(w + sp);
    uint16_t * q16_lo = q16 + int64_t(T) * hq * 256;
    // every check of the sparse launch is made here too, before the prepare is enqueued: a refusal enqueues nothing
    sparse_gate gate = {qfull + 256, 512, out, codes, scales};
    if (T <= 0 || T > kSelMaxRows || depth < 0 || layer < 0 || layer >= p->layers() || slot < 0 ||
        slot >= p->pages().n_slots() || depth + T > p->mapped_cells(slot) || depth + T > kSelMaxCells ||
        G > FNKV_MAX_ROWS || body == nullptr || offsets == nullptr || (reinterpret_cast<uintptr_t>(body) & 3) != 0 ||
        (reinterpret_cast<uintptr_t>(offsets) & 3) != 0) {
        set_error(name + ": rows, heads, layer or cells outside the contract");
        return FNKV_ERR_ARG;
    }
    if (check_only) {
        return FNKV_OK;
    }
    // at most 16 query heads a KV head: the sparse launch prepares its rows itself (one launch fewer);
    // FNKV_QSA_TWO_KERNELS=1 keeps the separate prepare launch, for comparison
    static const int32_t two = env_int_once("FNKV_QSA_TWO_KERNELS", 0);
    if (G <= 16 && two == 0) {
        fused_prep fp;
        fp.qfull = qfull;
        fp.kv_k = kv_k;
        fp.kv_v = kv_v;
        fp.q_norm = q_norm;
        fp.k_norm = k_norm;
        fp.pos = pos;
        fp.theta_scale = theta_scale;
        fp.q_f32 = q_f32;
        fp.k_f32 = k_f32;
        fp.rows = T;
        return sparse_launch(pool, slot, depth, T, layer, hq, 1.0f / 16.0f, q16, body, offsets, kv_k, kv_v, FNKV_F32,
                             nullptr, &gate, ws, sp, st, who, &fp, dd, q16_lo);
    }
    const pool_view pv = p->view();
    qsa_prep_args pa = {pv, pv.table + int64_t(slot) * pv.table_stride, layer, depth,
                        dd != nullptr ? dd->depth : nullptr, dd != nullptr ? dd->max_cells : 0, qfull, kv_k, kv_v,
                        q_norm, k_norm, pos, theta_scale, T, hq, p->h_kv(), q16, q16_lo, q_f32, k_f32};
    hipLaunchKernelGGL(qsa_prepare_kernel, dim3(static_cast<uint32_t>(T), static_cast<uint32_t>(hq + p->h_kv())),
                       dim3(64), 0, st, pa);
    return sparse_launch(pool, slot, depth, T, layer, hq, 1.0f / 16.0f, q16, body, offsets, nullptr, nullptr, FNKV_F32,
                         nullptr, &gate, ws, sp, st, who, nullptr, dd, q16_lo);
}

} // namespace fnkv

using fnkv::set_error;

extern "C" {

int64_t fnkv_qsa_workspace_bytes(const fnkv_pool * pool, int64_t depth, int32_t T, int32_t hq) {
    const int64_t sp = fnkv_sparse_workspace_bytes(pool, depth, T, hq);
    if (sp < 0) {
        return -1;
    }
    return fnkv::up16(sp) + 2 * int64_t(T) * hq * 256 * 2; // q's fp16 hi and lo parts
}

int fnkv_qsa_attend(const fnkv_pool * pool, int32_t slot, int64_t depth, int32_t T, int32_t layer, int32_t hq,
                    const float * qfull, const float * kv_k, const float * kv_v, const float * q_norm,
                    const float * k_norm, const int32_t * pos, float theta_scale, const void * body,
                    const void * offsets, float * out, int8_t * codes, float * scales, float * q_f32, float * k_f32,
                    void * ws, int64_t ws_bytes, void * stream) {
    return fnkv::qsa_launch(pool, slot, depth, T, layer, hq, qfull, kv_k, kv_v, q_norm, k_norm, pos, theta_scale, body,
                            offsets, out, codes, scales, q_f32, k_f32, ws, ws_bytes, static_cast<hipStream_t>(stream),
                            nullptr, "fnkv_qsa_attend");
}

int64_t fnkv_attend_workspace_bytes(const fnkv_pool * pool, int32_t max_cells, int32_t rows, int32_t hq) {
    if (rows <= 0 || max_cells < rows) {
        return -1;
    }
    return fnkv_qsa_workspace_bytes(pool, int64_t(max_cells) - rows, rows, hq);
}

namespace {
// one lane's checks and launches
int attend_one(int32_t rows, const fnkv_attend_args * a, hipStream_t st, const char * who, bool check_only) {
    if (a == nullptr) {
        fnkv::set_error(std::string(who) + ": null args");
        return FNKV_ERR_ARG;
    }
    const fnkv::dev_depth dd = {a->depth, a->max_cells, a->err};
    return fnkv::qsa_launch(a->pool, a->slot, 0, rows, a->layer, a->hq, a->qfull, a->kv_k, a->kv_v, a->q_norm,
                            a->k_norm, a->pos, a->theta_scale, a->body, a->offsets, a->out, a->codes, a->scales,
                            a->q_f32, a->k_f32, a->ws, a->ws_bytes, st, &dd, who, check_only);
}
} // namespace

int fnkv_attend(int32_t rows, const fnkv_attend_args * a, void * stream) {
    return attend_one(rows, a, static_cast<hipStream_t>(stream), "fnkv_attend", false);
}

int fnkv_attend_lanes(int32_t lanes, int32_t rows, const fnkv_attend_args * a, void * stream) {
    if (lanes < 2 || lanes > FNKV_MAX_LANES || a == nullptr) {
        fnkv::set_error("fnkv_attend_lanes: lanes outside 2 .. " + std::to_string(FNKV_MAX_LANES));
        return FNKV_ERR_ARG;
    }
    // every lane is checked before any is enqueued (the host checks of a lane enqueue nothing): all or nothing
    for (int32_t u = 0; u < lanes; ++u) {
        if (attend_one(rows, &a[u], nullptr, "fnkv_attend_lanes", true) != FNKV_OK) {
            fnkv::set_error("fnkv_attend_lanes: lane " + std::to_string(u) + ": " + fnkv::last_error());
            return FNKV_ERR_ARG;
        }
        for (int32_t v = 0; v < u; ++v) { // lanes are distinct sequences: no two write the same cells
            if (a[v].pool == a[u].pool && a[v].slot == a[u].slot) {
                fnkv::set_error("fnkv_attend_lanes: lanes " + std::to_string(v) + " and " + std::to_string(u) +
                                " name the same slot");
                return FNKV_ERR_ARG;
            }
        }
    }
    for (int32_t u = 0; u < lanes; ++u) {
        const int rc = attend_one(rows, &a[u], static_cast<hipStream_t>(stream), "fnkv_attend_lanes", false);
        if (rc != FNKV_OK) {
            return rc;
        }
    }
    return FNKV_OK;
}

} // extern "C"
