// Sparse (QSA) attention at decode rows: each of T <= 5 query rows of one sequence attends only to its selection —
// the reference's selected-block body (fn/kernels/qsa/qsa.h:77-81: per row K ascending 4-cell block IDs, then its
// tail cells), at most 512 blocks and 3 tail cells a row — instead of its whole causal context. This is the reference's
// production decode path (attn::attend over the body, fn/kernels/qsa/attend.h:97-141, cell expansion
// attend.cu:405-421), here over the Q8_0 / KV8 pool.
//
// How (MI355X):
//   * sparse_plan_kernel (one workgroup of 1,024 threads): writes the step's new cells (the rows' own positions, which
//     a row's selection need not include), then turns the rows' bodies into per-tile masks in LDS — row t's 8 bits a
//     32-cell tile, one a 4-cell block — and compacts the tiles any row selected into an ascending list with their
//     masks (a scan over the tiles; the order, and so every result, is independent of scheduling).
//   * The decode kernels (decode_kernel<1, true>, decode_rows_kernel<NT, true>) walk that list instead of a range of
//     consecutive cells: split s takes entries s * S .. s * S + S - 1; a lane's four scores of a tile half are one
//     4-cell block, so the row's mask enters the softmax as one bit a half, the causal limit (own position) as in the
//     dense launch. A split past the list's end returns at once.
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
#include <string>

namespace fnkv {

constexpr int32_t kSelMaxCells = 262144 + 32;                              // history a launch (the reference's max_cells)
constexpr int32_t kSelMaxTiles = (kSelMaxCells + kTileTokens - 1) / kTileTokens; // 8,193
constexpr int32_t kSelTopBlocks = 512;                                     // blocks a row (qsa.h top_blocks)
constexpr int32_t kSelMaxRows = 5;                                         // rows a launch (qsa.h max_rows)
constexpr int32_t kPlanThreads = 1024;

struct sparse_plan_args {
    pool_view pv;
    int32_t slot, layer, T;
    int64_t depth;
    const uint32_t * body;   // the rows' bodies (qsa.h layout), U32 words
    const void * k_new;      // optional [T][h_kv][256] (fp16 / fp32): the rows' own cells, written here
    const void * v_new;
    int32_t new_f32;
    int32_t * sel_n;     // out: the list's length
    int32_t * sel_tiles; // out: ascending logical tiles
    uint2 * sel_masks;   // out: their masks
};

__global__ __launch_bounds__(kPlanThreads) void sparse_plan_kernel(sparse_plan_args a) {
    __shared__ uint32_t mlo[kSelMaxTiles]; // rows 0 .. 3: row t's 8 block bits at bit 8 t
    __shared__ uint32_t mhi[kSelMaxTiles]; // row 4
    __shared__ int32_t wsum[kPlanThreads / 64];
    const int32_t tid = static_cast<int32_t>(threadIdx.x);
    const int32_t lane = tid & 63, wave = tid >> 6;
    const int64_t ctx = a.depth + a.T;
    const int32_t n_tiles = static_cast<int32_t>((ctx + kTileTokens - 1) / kTileTokens);
    const pool_view & pv = a.pv;
    const int32_t * table = pv.table + int64_t(a.slot) * pv.table_stride;

    // the rows' own cells (a wave a (row, head, K or V)); the attention launch reads them after this kernel ends
    if (a.k_new != nullptr) {
        for (int32_t job = wave; job < a.T * pv.h_kv * 2; job += kPlanThreads / 64) {
            const int32_t kv = job & 1, h = (job >> 1) % pv.h_kv, t = (job >> 1) / pv.h_kv;
            const int64_t src = (int64_t(t) * pv.h_kv + h) * kHeadDim;
            float x[4];
            if (a.new_f32) {
                load4<true>(static_cast<const float *>(kv ? a.v_new : a.k_new) + src, lane, x);
            } else {
                load4<false>(static_cast<const uint16_t *>(kv ? a.v_new : a.k_new) + src, lane, x);
            }
            const int64_t pos = a.depth + t;
            quantize_store_fmt(x, lane, tile_of(pv, table, a.layer, h, pos), static_cast<int32_t>(pos & 31), kv,
                               pv.format);
        }
    }

    for (int32_t i = tid; i < n_tiles; i += kPlanThreads) {
        mlo[i] = 0u;
        mhi[i] = 0u;
    }
    __syncthreads();
    // each row's blocks into the masks. A row at position q sees block b whole when 4 b + 3 <= q; its tail (cells
    // 4 n_vis .. q, n_vis = (q + 1) / 4) is block n_vis up to its own position, which the attention's causal limit
    // cuts. Entries outside the row's whole blocks are ignored, so no body can make the launch read past its cells.
    // The body's layout follows from depth and T alone (qsa.h:77-81, body_offset): row t's words start after the
    // earlier rows' 2 + K + tail, so the rows are found from the positions, and no word past the body is read.
    int32_t off = 0;
    for (int32_t t = 0; t < a.T; ++t) {
        const uint32_t * body = a.body + off;
        const int64_t q = a.depth + t;
        const int32_t n_vis = static_cast<int32_t>((q + 1) / 4);
        const int32_t k_full = std::min(n_vis, kSelTopBlocks);
        off += 2 + k_full + static_cast<int32_t>((q + 1) % 4);
        const int32_t K = std::min(std::max(static_cast<int32_t>(body[0]), 0), k_full);
        uint32_t * m = t < 4 ? mlo : mhi;
        const int32_t shift = 8 * (t & 3);
        for (int32_t i = tid; i < K; i += kPlanThreads) {
            const int32_t b = static_cast<int32_t>(body[2 + i]);
            if (b >= 0 && b < n_vis) {
                atomicOr(&m[b >> 3], 1u << (shift + (b & 7)));
            }
        }
        if (tid == 0 && (q + 1) % 4 != 0) {
            atomicOr(&m[n_vis >> 3], 1u << (shift + (n_vis & 7)));
        }
    }
    __syncthreads();

    // compact: thread i scans tiles i * per .. (i + 1) * per - 1 in order; a block-wide exclusive scan of the counts
    // gives each thread its first slot in the ascending list
    const int32_t per = (n_tiles + kPlanThreads - 1) / kPlanThreads;
    const int32_t t0 = tid * per, t1 = std::min(n_tiles, t0 + per);
    int32_t cnt = 0;
    for (int32_t i = t0; i < t1; ++i) {
        cnt += (mlo[i] | mhi[i]) != 0u ? 1 : 0;
    }
    int32_t incl = cnt; // inclusive scan within the wave
#pragma unroll
    for (int32_t o = 1; o < 64; o <<= 1) {
        const int32_t y = __shfl_up(incl, o);
        incl += lane >= o ? y : 0;
    }
    if (lane == 63) {
        wsum[wave] = incl;
    }
    __syncthreads();
    int32_t base = 0;
    for (int32_t w = 0; w < wave; ++w) {
        base += wsum[w];
    }
    int32_t pos = base + incl - cnt;
    for (int32_t i = t0; i < t1; ++i) {
        const uint32_t lo = mlo[i], hi = mhi[i];
        if ((lo | hi) != 0u) {
            a.sel_tiles[pos] = i;
            a.sel_masks[pos] = uint2{lo, hi};
            ++pos;
        }
    }
    if (tid == kPlanThreads - 1) {
        *a.sel_n = base + incl;
    }
}

// The launch shape of a sparse step: the list's largest length, the entries a split takes, the splits.
struct sparse_plan {
    int32_t n_max = 0, per_split = 0, n_splits = 0;
    int64_t list_off = 0, mask_off = 0, po_off = 0, pml_off = 0, bytes = 0;
};
sparse_plan plan_sparse(const kv_pool & p, int64_t depth, int32_t T, int32_t R) {
    sparse_plan pl;
    const int32_t n_tiles = static_cast<int32_t>((depth + T + kTileTokens - 1) / kTileTokens);
    pl.n_max = std::min(n_tiles, T * (kSelTopBlocks + 1)); // each row: its blocks' tiles and its tail's
    const int32_t want = std::max(1, device_cus(p.device()) / p.h_kv());
    pl.per_split = std::min(64, std::max(1, (pl.n_max + want - 1) / want));
    pl.n_splits = (pl.n_max + pl.per_split - 1) / pl.per_split;
    auto up16 = [](int64_t x) { return (x + 15) & ~int64_t(15); };
    pl.list_off = 16;
    pl.mask_off = up16(pl.list_off + int64_t(pl.n_max) * 4);
    pl.po_off = up16(pl.mask_off + int64_t(pl.n_max) * 8);
    pl.pml_off = up16(pl.po_off + int64_t(pl.n_splits) * p.h_kv() * R * kHeadDim * 4);
    pl.bytes = up16(pl.pml_off + int64_t(pl.n_splits) * p.h_kv() * R * 2 * 4);
    return pl;
}

} // namespace fnkv

using fnkv::set_error;

extern "C" {

int64_t fnkv_sparse_workspace_bytes(const fnkv_pool * pool, int64_t depth, int32_t T, int32_t hq) {
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    if (p == nullptr || T <= 0 || T > fnkv::kSelMaxRows || depth < 0 || hq <= 0 || hq % p->h_kv() != 0) {
        return -1;
    }
    return fnkv::plan_sparse(*p, depth, T, (hq / p->h_kv()) * T).bytes;
}

int fnkv_attn_sparse(const fnkv_pool * pool, int32_t slot, int64_t depth, int32_t T, int32_t layer, int32_t hq,
                     float scale, const void * q, const void * body, const void * offsets, const void * k_new,
                     const void * v_new, int32_t new_dtype, void * out, void * ws, int64_t ws_bytes, void * stream) {
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    if (p == nullptr || slot < 0 || slot >= p->pages().n_slots() || T <= 0 || T > fnkv::kSelMaxRows || depth < 0 ||
        layer < 0 || layer >= p->layers() || hq <= 0 || hq % p->h_kv() != 0 || q == nullptr || body == nullptr ||
        offsets == nullptr || out == nullptr || ws == nullptr || !(scale > 0.0f) || !std::isfinite(scale) ||
        ((k_new == nullptr) != (v_new == nullptr)) || (new_dtype != FNKV_F16 && new_dtype != FNKV_F32)) {
        set_error("fnkv_attn_sparse: argument outside the contract");
        return FNKV_ERR_ARG;
    }
    const int32_t G = hq / p->h_kv();
    const int32_t R = G * T;
    const int64_t ctx = depth + T;
    if (R > FNKV_MAX_ROWS || ctx > fnkv::kSelMaxCells || ctx > p->mapped_cells(slot)) {
        set_error("fnkv_attn_sparse: G * T = " + std::to_string(R) + " (at most " + std::to_string(FNKV_MAX_ROWS) +
                  ") or cells " + std::to_string(ctx) + " outside the slot's mapped cells (at most " +
                  std::to_string(fnkv::kSelMaxCells) + ")");
        return FNKV_ERR_ARG;
    }
    if ((reinterpret_cast<uintptr_t>(q) & 15) != 0 || (reinterpret_cast<uintptr_t>(out) & 15) != 0 ||
        (reinterpret_cast<uintptr_t>(ws) & 15) != 0 || (reinterpret_cast<uintptr_t>(body) & 3) != 0 ||
        (reinterpret_cast<uintptr_t>(offsets) & 3) != 0) {
        set_error("fnkv_attn_sparse: q, out and ws must be 16-byte aligned, body and offsets 4-byte aligned");
        return FNKV_ERR_ARG;
    }
    const fnkv::sparse_plan pl = fnkv::plan_sparse(*p, depth, T, R);
    if (ws_bytes < pl.bytes) {
        set_error("fnkv_attn_sparse: workspace too small (fnkv_sparse_workspace_bytes)");
        return FNKV_ERR_ARG;
    }
    uint8_t * w = static_cast<uint8_t *>(ws);
    hipStream_t st = static_cast<hipStream_t>(stream);

    fnkv::sparse_plan_args pa;
    pa.pv = p->view();
    pa.slot = slot;
    pa.layer = layer;
    pa.T = T;
    pa.depth = depth;
    pa.body = static_cast<const uint32_t *>(body);
    pa.k_new = k_new;
    pa.v_new = v_new;
    pa.new_f32 = new_dtype == FNKV_F32 ? 1 : 0;
    pa.sel_n = reinterpret_cast<int32_t *>(w);
    pa.sel_tiles = reinterpret_cast<int32_t *>(w + pl.list_off);
    pa.sel_masks = reinterpret_cast<uint2 *>(w + pl.mask_off);
    hipLaunchKernelGGL(fnkv::sparse_plan_kernel, dim3(1), dim3(fnkv::kPlanThreads), 0, st, pa);

    fnkv::dec_args a;
    a.pv = p->view();
    a.q = static_cast<const uint16_t *>(q);
    a.k_new = nullptr; // written by the plan kernel
    a.v_new = nullptr;
    a.new_f32 = 0;
    a.po = reinterpret_cast<float *>(w + pl.po_off);
    a.pml = reinterpret_cast<float *>(w + pl.pml_off);
    a.c2 = scale * 1.4426950408889634f;
    a.layer = layer;
    a.T = T;
    a.G = G;
    a.hq = hq;
    a.R = R;
    a.n_seq = 1;
    a.split_tokens = 0;
    for (int32_t i = 0; i < FNKV_MAX_SEQS; ++i) {
        a.slot[i] = slot;
        a.ctx[i] = ctx;
    }
    a.split0[0] = 0;
    for (int32_t i = 1; i <= FNKV_MAX_SEQS; ++i) {
        a.split0[i] = pl.n_splits;
    }
    a.sel_tiles = pa.sel_tiles;
    a.sel_masks = pa.sel_masks;
    a.sel_n = pa.sel_n;
    a.sel_split = pl.per_split;
#ifdef FNKV_TIMING
    a.ts = nullptr;
#endif
    fnkv::launch_decode_sparse(*p, (R + 15) / 16, dim3(static_cast<uint32_t>(pl.n_splits),
                                                        static_cast<uint32_t>(p->h_kv())), a, st);
    fnkv::merge_args m;
    m.po = a.po;
    m.pml = a.pml;
    m.out = static_cast<uint16_t *>(out);
    m.T = T;
    m.G = G;
    m.hq = hq;
    m.R = R;
    m.h_kv = p->h_kv();
    m.n_seq = 1;
    for (int32_t i = 0; i <= FNKV_MAX_SEQS; ++i) {
        m.split0[i] = a.split0[i];
    }
    m.sel_n = pa.sel_n;
    m.sel_split = pl.per_split;
    fnkv::launch_merge(m, st);
    if (hipGetLastError() != hipSuccess) {
        set_error("fnkv_attn_sparse: launch failed");
        return FNKV_ERR_HIP;
    }
    return FNKV_OK;
}

} // extern "C"
