// The prompt path's own contract over the pool: fn::qsa::qsp_kv and qsp_attend (fn/kernels/qsa/qsa_prompt.h:90-124,
// qsa_prompt_attn.cu:90-122, 229-471).
//   qsp_kv:     row t's k = IMROPE(RMS norm(kv_k) k_norm) at the row's rope position and v = kv_v, quantized by the
//               pool's rule (Q8_0 or KV8) at cell pos0 + t. A wave a (row, KV head); the arithmetic is fnkv_qsa_attend's
//               prepare (rope.h), so the codes are bitwise the pool quantizer's of the same F32 k.
//   qsp_attend: row t's query heads q = IMROPE(RMS norm(qfull[h][0..255]) q_norm) (fp16, the score scale 1/16 applied
//               in F32), attention over the row's selection body (its blocks' 4 cells each, then its tail; the bodies
//               in the reference's slab layout: slab k = rows 128 k .., its bodies at body + k * 128 * 517 words, row
//               i's at byte offset offsets[129 k + i]), out = o sigmoid(gate) in F32 (optional) and fp16, bit 0 of *err
//               for a value fp16 cannot hold. The attention is the sparse decode kernels' (each row its own selection,
//               the pool's codes exact, fp32 accumulation; one launch a chunk of up to kQspChunk rows, the rows side by
//               side), then the gated merge.
// The rope position of row t: planes[4 t + plane] when planes are given (the reference's supplied rows, [rows][4]),
// else pos0 + rope_off + t on every plane.
#include "../../include/fnkv.h"
#include "common.h"
#include "decode_common.h"
#include "q8_0.h"
#include "rope.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <string>

namespace fnkv {
namespace {

constexpr int32_t kQspChunk = 512; // prompt rows a launch (bounds the split partials of the workspace)

struct qsp_args {
    pool_view pv;
    const int32_t * table;
    int32_t layer, pos0, rows, hq, h_kv, rope_off;
    const int32_t * planes;
    float theta_scale;
    const float * src;  // qfull [rows][hq][512] (q) or kv_k [rows][h_kv][256] (kv)
    const float * norm; // q_norm or k_norm
    const float * kv_v; // kv: [rows][h_kv][256]
    uint16_t * q16;     // q: [rows][hq][256]
};

__device__ __forceinline__ int32_t qsp_pos(const qsp_args & a, int32_t t, int32_t lane) {
    return a.planes != nullptr ? a.planes[4 * t + rope_plane(lane)] : a.pos0 + a.rope_off + t;
}

// a wave a (row, query head): the prepared query as fp16 (the attention's operand)
__global__ __launch_bounds__(64) void qsp_q_kernel(qsp_args a) {
    const int32_t t = static_cast<int32_t>(blockIdx.x), h = static_cast<int32_t>(blockIdx.y);
    const int32_t lane = static_cast<int32_t>(threadIdx.x);
    const float4 x = reinterpret_cast<const float4 *>(a.src + (int64_t(t) * a.hq + h) * 512)[lane];
    const float4 g = reinterpret_cast<const float4 *>(a.norm)[lane];
    float s, c, y[4];
    rope_angle(s, c, qsp_pos(a, t, lane), a.theta_scale, lane);
    norm_rope_apply(y, x, g, s, c, lane);
    reinterpret_cast<uint2 *>(a.q16 + (int64_t(t) * a.hq + h) * 256)[lane] = pack4_f16(y, 1.0f);
}

// a wave a (row, KV head): k normed and roped, then k and v quantized into the pool at cell pos0 + t
__global__ __launch_bounds__(64) void qsp_kv_kernel(qsp_args a) {
    const int32_t t = static_cast<int32_t>(blockIdx.x), kvh = static_cast<int32_t>(blockIdx.y);
    const int32_t lane = static_cast<int32_t>(threadIdx.x);
    const int64_t o = (int64_t(t) * a.h_kv + kvh) * 256;
    const float4 x = reinterpret_cast<const float4 *>(a.src + o)[lane];
    const float4 g = reinterpret_cast<const float4 *>(a.norm)[lane];
    float s, c, y[4];
    rope_angle(s, c, qsp_pos(a, t, lane), a.theta_scale, lane);
    norm_rope_apply(y, x, g, s, c, lane);
    const int64_t pos = int64_t(a.pos0) + t;
    uint8_t * tile = tile_of(a.pv, a.table, a.layer, kvh, pos);
    quantize_store_fmt(y, lane, tile, static_cast<int32_t>(pos & 31), 0, a.pv.format);
    float v[4];
    load4<true>(a.kv_v + o, lane, v);
    quantize_store_fmt(v, lane, tile, static_cast<int32_t>(pos & 31), 1, a.pv.format);
}

bool al16(const void * p) { return p != nullptr && (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
bool al4(const void * p) { return p != nullptr && (reinterpret_cast<uintptr_t>(p) & 3) == 0; }

// the rope positions the launch reads must lie in the rows' planes or be the text positions; the cells must be mapped
bool qsp_common(const kv_pool * p, int32_t slot, int32_t layer, int32_t pos0, int32_t rows, const std::string & who) {
    if (p == nullptr || slot < 0 || slot >= p->pages().n_slots() || layer < 0 || layer >= p->layers() || rows < 1 ||
        rows > FNKV_QSP_MAX_ROWS || pos0 < 0 || int64_t(pos0) + rows > p->mapped_cells(slot) ||
        int64_t(pos0) + rows > kSelMaxCells) {
        set_error(who + ": slot, layer, rows (1 .. 4,096) or cells outside the contract (the rows' cells mapped)");
        return false;
    }
    return true;
}

} // namespace
} // namespace fnkv

using fnkv::set_error;

extern "C" {

int fnkv_qsp_kv(const fnkv_qsp_kv_args * a, void * stream) {
    const fnkv::kv_pool * p = a != nullptr ? fnkv::pool_of(a->pool) : nullptr;
    if (a == nullptr || !fnkv::qsp_common(p, a->slot, a->layer, a->pos0, a->rows, "fnkv_qsp_kv")) {
        if (a == nullptr) {
            set_error("fnkv_qsp_kv: null args");
        }
        return FNKV_ERR_ARG;
    }
    if (!fnkv::al16(a->kv_k) || !fnkv::al16(a->kv_v) || !fnkv::al16(a->k_norm) ||
        (a->planes != nullptr && !fnkv::al4(a->planes)) || !std::isfinite(a->theta_scale)) {
        set_error("fnkv_qsp_kv: kv_k, kv_v, k_norm must be 16-byte aligned device arrays, planes 4-byte aligned");
        return FNKV_ERR_ARG;
    }
    const fnkv::pool_view pv = p->view();
    fnkv::qsp_args q = {pv, pv.table + int64_t(a->slot) * pv.table_stride, a->layer, a->pos0, a->rows, 0, p->h_kv(),
                        a->rope_off, a->planes, a->theta_scale, a->kv_k, a->k_norm, a->kv_v, nullptr};
    hipLaunchKernelGGL(fnkv::qsp_kv_kernel, dim3(static_cast<uint32_t>(a->rows), static_cast<uint32_t>(p->h_kv())),
                       dim3(64), 0, static_cast<hipStream_t>(stream), q);
    if (hipGetLastError() != hipSuccess) {
        set_error("fnkv_qsp_kv: launch failed");
        return FNKV_ERR_HIP;
    }
    return FNKV_OK;
}

int64_t fnkv_qsp_workspace_bytes(const fnkv_pool * pool, int32_t pos0, int32_t rows, int32_t hq) {
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    if (p == nullptr || rows < 1 || rows > FNKV_QSP_MAX_ROWS || pos0 < 0 || hq <= 0 || hq % p->h_kv() != 0 ||
        hq / p->h_kv() > FNKV_MAX_ROWS) {
        return -1;
    }
    const int32_t n = std::min(rows, fnkv::kQspChunk);
    // the fp16 queries of every row, then the deepest chunk's partials (every chunk's plan is at most that)
    const int64_t q_bytes = (int64_t(rows) * hq * 256 * 2 + 255) & ~int64_t(255);
    return q_bytes + fnkv::prompt_ws_bytes(*p, int64_t(pos0) + rows, n, hq / p->h_kv());
}

int fnkv_qsp_attend(const fnkv_qsp_attend_args * a, void * stream) {
    const fnkv::kv_pool * p = a != nullptr ? fnkv::pool_of(a->pool) : nullptr;
    if (a == nullptr || !fnkv::qsp_common(p, a->slot, a->layer, a->pos0, a->rows, "fnkv_qsp_attend")) {
        if (a == nullptr) {
            set_error("fnkv_qsp_attend: null args");
        }
        return FNKV_ERR_ARG;
    }
    const int64_t need = fnkv_qsp_workspace_bytes(a->pool, a->pos0, a->rows, a->hq);
    if (need < 0 || !fnkv::al16(a->qfull) || !fnkv::al16(a->q_norm) || !fnkv::al4(a->body) ||
        !fnkv::al4(a->offsets) || !fnkv::al16(a->out16) || (a->out != nullptr && !fnkv::al16(a->out)) ||
        (a->err != nullptr && !fnkv::al4(a->err)) || (a->planes != nullptr && !fnkv::al4(a->planes)) ||
        !fnkv::al16(a->ws) || !std::isfinite(a->theta_scale)) {
        set_error("fnkv_qsp_attend: heads, alignment (qfull, q_norm, out16, out, ws: 16 B) or null arrays outside "
                  "the contract");
        return FNKV_ERR_ARG;
    }
    if (a->ws_bytes < need) {
        set_error("fnkv_qsp_attend: workspace too small (fnkv_qsp_workspace_bytes)");
        return FNKV_ERR_ARG;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    const fnkv::pool_view pv = p->view();
    uint8_t * w = static_cast<uint8_t *>(a->ws);
    uint16_t * q16 = reinterpret_cast<uint16_t *>(w);
    const int64_t q_bytes = (int64_t(a->rows) * a->hq * 256 * 2 + 255) & ~int64_t(255);
    fnkv::qsp_args q = {pv, nullptr, a->layer, a->pos0, a->rows, a->hq, p->h_kv(), a->rope_off, a->planes,
                        a->theta_scale, a->qfull, a->q_norm, nullptr, q16};
    hipLaunchKernelGGL(fnkv::qsp_q_kernel, dim3(static_cast<uint32_t>(a->rows), static_cast<uint32_t>(a->hq)),
                       dim3(64), 0, st, q);
    for (int32_t r0 = 0; r0 < a->rows; r0 += fnkv::kQspChunk) {
        const int32_t n = std::min(fnkv::kQspChunk, a->rows - r0);
        const int64_t rows_off = int64_t(r0) * a->hq * 256;
        const int rc = fnkv::prompt_launch(
            *p, a->slot, a->layer, a->pos0, r0, n, a->hq, q16 + rows_off, static_cast<const uint32_t *>(a->body),
            a->offsets, a->qfull + int64_t(r0) * a->hq * 512 + 256, a->out != nullptr ? a->out + rows_off : nullptr,
            a->out16 + rows_off, a->err, w + q_bytes, st);
        if (rc != FNKV_OK) {
            set_error("fnkv_qsp_attend: launch failed");
            return rc;
        }
    }
    if (hipGetLastError() != hipSuccess) {
        set_error("fnkv_qsp_attend: launch failed");
        return FNKV_ERR_HIP;
    }
    return FNKV_OK;
}

} // extern "C"
