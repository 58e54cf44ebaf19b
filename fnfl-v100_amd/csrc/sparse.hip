// Sparse (QSA) attention at decode rows: each of T <= 5 query rows of one sequence attends only to its selection —
// the reference's selected-block body (fn/kernels/qsa/qsa.h:77-81: per row K ascending 4-cell block IDs, then its
// tail cells), at most 512 blocks and 3 tail cells a row — instead of its whole causal context. This is the reference's
// production decode path (attn::attend over the body, fn/kernels/qsa/attend.h:97-141, cell expansion
// attend.cu:405-421), here over the Q8_0 / KV8 pool.
//
// How (MI355X):
//   * The decode kernels (decode_kernel<1, true>, decode_rows_kernel<NT, true>) walk the selection's tiles instead of
//     a range of consecutive cells. Each workgroup rebuilds the selection in LDS from the bodies (sparse_build: row
//     t's 8 bits a 32-cell tile, one a 4-cell block; the tiles any row selected in ascending order, by a block-wide
//     scan) and takes entries s * S .. s * S + S - 1 of that list; a lane's four scores of a tile half are one 4-cell
//     block, so the row's mask enters the softmax as one bit a half, the causal limit (own position) as in the dense
//     launch. The rows' own cells are written by the workgroup that reads their tile (split 0 when no row selects
//     it). A split past the list's end returns at once; split 0 of head 0 stores the list's length.
//   * merge_kernel folds the splits that ran (it reads the list's length).
// Tiles are read whole (17,408 B) even when one block of them is selected: the pool's layout is tile-granular, and
// selections that cluster (sinks, local windows, topical runs) share tiles across blocks and rows.
#include "../../include/fnkv.h"
#include "common.h"
#include "layout.h"
#include "mfma.h"
#include "q8_0.h"
#include "decode_common.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <string>

namespace fnkv {

#ifdef FNKV_TIMING
uint64_t * timing_buffer();
#endif

// The launch shape of a sparse step: each of the T rows runs as its own n_splits splits (a row's list: at most its
// 513 tiles), the entries a split takes, the partials of every row.
struct sparse_plan {
    int32_t n_max = 0, per_split = 0, n_splits = 0;
    int64_t po_off = 0, pml_off = 0, bytes = 0;
};
sparse_plan plan_sparse(const kv_pool & p, int64_t depth, int32_t T, int32_t G) {
    sparse_plan pl;
    const int32_t n_tiles = static_cast<int32_t>((depth + T + kTileTokens - 1) / kTileTokens);
    pl.n_max = std::min(n_tiles, kSelTopBlocks + 1); // a row's blocks' tiles and its tail's
    int32_t want = std::max(1, device_cus(p.device()) / (p.h_kv() * T));
    static const int32_t want_knob = env_int_once("FNKV_SPARSE_WANT", 0); // splits a row and head, for measurement
    if (want_knob > 0) {
        want = want_knob;
    }
    pl.per_split = std::min(64, std::max(1, (pl.n_max + want - 1) / want));
    pl.n_splits = (pl.n_max + pl.per_split - 1) / pl.per_split;
    auto up16 = [](int64_t x) { return (x + 15) & ~int64_t(15); };
    pl.po_off = up16(int64_t(T) * 4); // each row's list length first
    pl.pml_off = up16(pl.po_off + int64_t(T) * pl.n_splits * p.h_kv() * G * kHeadDim * 4);
    pl.bytes = up16(pl.pml_off + int64_t(T) * pl.n_splits * p.h_kv() * G * 2 * 4);
    return pl;
}

// The sparse launch (validation, the decode kernels' sparse instantiation, the merge); `gate` set: the merge writes
// the gated F32 output and its activation format instead of the fp16 out. Returns a status; nothing is enqueued
// unless it is FNKV_OK.
int sparse_launch(const fnkv_pool * pool, int32_t slot, int64_t depth, int32_t T, int32_t layer, int32_t hq, float scale,
                  const void * q, const void * body, const void * offsets, const void * k_new, const void * v_new,
                  int32_t new_dtype, void * out, const sparse_gate * gate, void * ws, int64_t ws_bytes,
                  hipStream_t st, const char * who, const fused_prep * fp, const dev_depth * dd,
                  const uint16_t * q_lo) {
    const kv_pool * p = pool_of(pool);
    const std::string name(who);
    if (dd != nullptr) { // the plan is the bound's: the deepest rows' tiles
        if (dd->depth == nullptr || dd->err == nullptr || (reinterpret_cast<uintptr_t>(dd->depth) & 3) != 0 ||
            (reinterpret_cast<uintptr_t>(dd->err) & 3) != 0 || dd->max_cells < T) {
            set_error(name + ": the device depth and error words (4-byte aligned) and max_cells >= rows required");
            return FNKV_ERR_ARG;
        }
        depth = dd->max_cells - T;
    }
    if (p == nullptr || slot < 0 || slot >= p->pages().n_slots() || T <= 0 || T > kSelMaxRows || depth < 0 ||
        layer < 0 || layer >= p->layers() || hq <= 0 || hq % p->h_kv() != 0 || q == nullptr || body == nullptr ||
        offsets == nullptr || (out == nullptr && gate == nullptr) || ws == nullptr || !(scale > 0.0f) ||
        !std::isfinite(scale) || ((k_new == nullptr) != (v_new == nullptr)) ||
        (new_dtype != FNKV_F16 && new_dtype != FNKV_F32)) {
        set_error(name + ": argument outside the contract");
        return FNKV_ERR_ARG;
    }
    const int32_t G = hq / p->h_kv();
    const int64_t ctx = depth + T;
    if (G > FNKV_MAX_ROWS || ctx > kSelMaxCells || ctx > p->mapped_cells(slot)) {
        set_error(name + ": G = " + std::to_string(G) + " (at most " + std::to_string(FNKV_MAX_ROWS) +
                  ") or cells " + std::to_string(ctx) + " outside the slot's mapped cells (at most " +
                  std::to_string(kSelMaxCells) + ")");
        return FNKV_ERR_ARG;
    }
    if ((reinterpret_cast<uintptr_t>(q) & 15) != 0 || (reinterpret_cast<uintptr_t>(q_lo) & 15) != 0 || (reinterpret_cast<uintptr_t>(out) & 15) != 0 ||
        (reinterpret_cast<uintptr_t>(ws) & 15) != 0 || (reinterpret_cast<uintptr_t>(body) & 3) != 0 ||
        (reinterpret_cast<uintptr_t>(offsets) & 3) != 0) {
        set_error(name + ": q, out and ws must be 16-byte aligned, body and offsets 4-byte aligned");
        return FNKV_ERR_ARG;
    }
    const sparse_plan pl = plan_sparse(*p, depth, T, G);
    if (ws_bytes < pl.bytes) {
        set_error(name + ": workspace too small");
        return FNKV_ERR_ARG;
    }
    uint8_t * w = static_cast<uint8_t *>(ws);

    // several rows: their new cells first (a row may read an earlier row's new cell; the rows run side by side); one
    // row: the launch writes it, by the split that reads its tile
    if (fp != nullptr && (G > 16 || fp->rows != T)) {
        set_error(name + ": a launch that prepares its rows takes at most 16 query heads a KV head");
        return FNKV_ERR_ARG;
    }
    if (k_new != nullptr && T > 1 && fp == nullptr) {
        if (append_enqueue(*p, slot, layer, depth, dd != nullptr ? dd->depth : nullptr, ctx, T, k_new, v_new,
                           new_dtype, st) != FNKV_OK) {
            set_error(name + ": launch failed");
            return FNKV_ERR_HIP;
        }
    }
    dec_args a;
    a.pv = p->view();
    a.q = static_cast<const uint16_t *>(q);
    a.k_new = T == 1 ? k_new : nullptr;
    a.v_new = T == 1 ? v_new : nullptr;
    a.new_f32 = new_dtype == FNKV_F32 ? 1 : 0;
    a.po = reinterpret_cast<float *>(w + pl.po_off);
    a.pml = reinterpret_cast<float *>(w + pl.pml_off);
    a.c2 = scale * 1.4426950408889634f;
    a.layer = layer;
    a.T = T;
    a.G = G;
    a.hq = hq;
    a.R = G * T; // each row's view takes G of them
    a.n_seq = 1;
    a.split_tokens = 0;
    a.strided = 0;
    for (int32_t i = 0; i < FNKV_MAX_SEQS; ++i) {
        a.slot[i] = slot;
        a.ctx[i] = ctx;
    }
    a.split0[0] = 0;
    for (int32_t i = 1; i <= FNKV_MAX_SEQS; ++i) {
        a.split0[i] = pl.n_splits;
    }
    a.sel_body = static_cast<const uint32_t *>(body);
    a.sel_n = reinterpret_cast<int32_t *>(w);
    a.sel_split = pl.per_split;
    if (fp != nullptr) {
        a.fp = *fp;
    }
    a.q_lo = q_lo;
    if (dd != nullptr) {
        a.depth_dev = dd->depth;
        a.err = dd->err;
    }
#ifdef FNKV_TIMING
    a.ts = timing_buffer();
#endif
    launch_decode_sparse(*p, (G + 15) / 16,
                         dim3(static_cast<uint32_t>(pl.n_splits), static_cast<uint32_t>(p->h_kv()),
                              static_cast<uint32_t>(T)),
                         a, st);
    merge_args m;
    m.po = a.po;
    m.pml = a.pml;
    m.out = static_cast<uint16_t *>(out);
    // the rows fold as sequences of one step token each ([row][split] partials, row r's out at row r)
    m.T = 1;
    m.G = G;
    m.hq = hq;
    m.R = G;
    m.h_kv = p->h_kv();
    m.n_seq = T;
    for (int32_t i = 0; i <= FNKV_MAX_SEQS; ++i) {
        m.split0[i] = (i < T ? i : T) * pl.n_splits;
    }
    m.sel_n = a.sel_n;
    m.sel_split = pl.per_split;
    if (dd != nullptr) {
        m.depth_dev = dd->depth;
        m.cap[0] = ctx;
        m.T_dev = T;
    }
    if (gate != nullptr) {
        m.gate = gate->gate;
        m.gate_stride = gate->stride;
        m.out_f32 = gate->out_f32;
        m.codes = gate->codes;
        m.act_scales = gate->scales;
    }
    launch_merge(m, st);
    if (hipGetLastError() != hipSuccess) {
        set_error(name + ": launch failed");
        return FNKV_ERR_HIP;
    }
    return FNKV_OK;
}

// Prompt rows (qsp_attend): rows row0 .. row0 + n - 1 of a prompt half at positions pos0 + row, each over its own
// selection body (the slab layout), q16 the rows' prepared fp16 queries [n][hq][256], then the gated merge into the
// F32 (optional) and fp16 outputs. The caller has checked the arguments; ws holds prompt_ws_bytes(pool, cells, n, hq).
int64_t prompt_ws_bytes(const kv_pool & p, int64_t cells, int32_t n, int32_t G) {
    return plan_sparse(p, cells - n, n, G).bytes;
}

int prompt_launch(const kv_pool & p, int32_t slot, int32_t layer, int32_t pos0, int32_t row0, int32_t n, int32_t hq,
                  const uint16_t * q16, const uint32_t * body, const int32_t * offsets, const float * gate,
                  float * out_f32, uint16_t * out16, uint32_t * err, void * ws, hipStream_t st) {
    const int32_t G = hq / p.h_kv();
    const int64_t last = int64_t(pos0) + row0 + n; // cells the chunk's last row sees
    const sparse_plan pl = plan_sparse(p, last - n, n, G);
    uint8_t * w = static_cast<uint8_t *>(ws);
    dec_args a;
    a.pv = p.view();
    a.q = q16;
    a.k_new = nullptr;
    a.v_new = nullptr;
    a.new_f32 = 0;
    a.po = reinterpret_cast<float *>(w + pl.po_off);
    a.pml = reinterpret_cast<float *>(w + pl.pml_off);
    a.c2 = (1.0f / 16.0f) * 1.4426950408889634f;
    a.layer = layer;
    a.T = n;
    a.G = G;
    a.hq = hq;
    a.R = G * n;
    a.n_seq = 1;
    a.split_tokens = 0;
    a.strided = 0;
    for (int32_t i = 0; i < FNKV_MAX_SEQS; ++i) {
        a.slot[i] = slot;
        a.ctx[i] = last;
    }
    a.split0[0] = 0;
    for (int32_t i = 1; i <= FNKV_MAX_SEQS; ++i) {
        a.split0[i] = pl.n_splits;
    }
    a.sel_body = body;
    a.sel_n = reinterpret_cast<int32_t *>(w);
    a.sel_split = pl.per_split;
    a.sel_offsets = offsets;
    a.sel_row0 = row0;
#ifdef FNKV_TIMING
    a.ts = timing_buffer();
#endif
    launch_decode_sparse(p, (G + 15) / 16,
                         dim3(static_cast<uint32_t>(pl.n_splits), static_cast<uint32_t>(p.h_kv()),
                              static_cast<uint32_t>(n)),
                         a, st);
    merge_args m;
    m.po = a.po;
    m.pml = a.pml;
    m.out = nullptr;
    m.T = 1;
    m.G = G;
    m.hq = hq;
    m.R = G;
    m.h_kv = p.h_kv();
    m.n_seq = n;
    m.uniform_splits = pl.n_splits;
    m.sel_n = a.sel_n;
    m.sel_split = pl.per_split;
    m.gate = gate;
    m.gate_stride = 512;
    m.out_f32 = out_f32;
    m.out16 = out16;
    m.err = err;
    launch_merge(m, st);
    return hipGetLastError() == hipSuccess ? FNKV_OK : FNKV_ERR_HIP;
}

} // namespace fnkv

using fnkv::set_error;

extern "C" {

int64_t fnkv_sparse_workspace_bytes(const fnkv_pool * pool, int64_t depth, int32_t T, int32_t hq) {
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    if (p == nullptr || T <= 0 || T > fnkv::kSelMaxRows || depth < 0 || hq <= 0 || hq % p->h_kv() != 0) {
        return -1;
    }
    return fnkv::plan_sparse(*p, depth, T, hq / p->h_kv()).bytes;
}

int fnkv_attn_sparse(const fnkv_pool * pool, int32_t slot, int64_t depth, int32_t T, int32_t layer, int32_t hq,
                     float scale, const void * q, const void * body, const void * offsets, const void * k_new,
                     const void * v_new, int32_t new_dtype, void * out, void * ws, int64_t ws_bytes, void * stream) {
    return fnkv::sparse_launch(pool, slot, depth, T, layer, hq, scale, q, body, offsets, k_new, v_new,
                               new_dtype, out, nullptr, ws, ws_bytes, static_cast<hipStream_t>(stream),
                               "fnkv_attn_sparse");
}

int fnkv_attn_sparse_dev(const fnkv_pool * pool, int32_t slot, const int32_t * depth, int64_t max_cells, int32_t T,
                         int32_t layer, int32_t hq, float scale, const void * q, const void * body,
                         const void * offsets, const void * k_new, const void * v_new, int32_t new_dtype, void * out,
                         void * ws, int64_t ws_bytes, uint32_t * err, void * stream) {
    const fnkv::dev_depth dd = {depth, max_cells, err};
    return fnkv::sparse_launch(pool, slot, 0, T, layer, hq, scale, q, body, offsets, k_new, v_new, new_dtype, out,
                               nullptr, ws, ws_bytes, static_cast<hipStream_t>(stream), "fnkv_attn_sparse_dev",
                               nullptr, &dd);
}

} // extern "C"
