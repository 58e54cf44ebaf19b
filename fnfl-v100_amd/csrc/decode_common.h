// Shared by the decode kernels (decode.hip): launch arguments, the fused append of the step's new
// cells, the Q operands, the score and softmax steps of one 32-token tile.
#pragma once

#include "../../include/fnkv.h"
#include "common.h"
#include "layout.h"
#include "mfma.h"
#include "q8_0.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

namespace fnkv {

constexpr float kNegInf = -__builtin_inff();
constexpr int32_t kCodeBytes = 16384;  // a tile's K and V codes
constexpr int32_t kScaleBytes = 1024;  // a tile's K and V scales
constexpr int32_t kGroupLds = kCodeBytes + 2 * kScaleBytes;

// A one-row sparse launch that prepares its own row (fnkv_qsa_attend at T = 1): the attend's inputs. Each workgroup
// forms its KV head's query rows (F32 RMS norm and IMROPE, fp16) while its selection builds, and the workgroup that
// reads the new cell's tile writes the cell's K (normed, roped) and V in the pool's format.
struct fused_prep {
    const float * qfull = nullptr; // [rows][hq][512]: each head's q, then its gate; null: the launch reads q
    const float * kv_k = nullptr;  // [rows][h_kv][256]
    const float * kv_v = nullptr;  // [rows][h_kv][256]
    const float * q_norm = nullptr;
    const float * k_norm = nullptr;
    const int32_t * pos = nullptr; // [4][rows]
    float theta_scale = 0.0f;
    float * q_f32 = nullptr; // optional [rows][hq][256]
    float * k_f32 = nullptr; // optional [rows][h_kv][256]
    int32_t rows = 1;        // the call's rows: row z (grid.z) is qfull's, pos's column and q_f32's row z; its new
                             // cell depth + z is kv_k / kv_v / k_f32's row z
};

struct dec_args {
    pool_view pv;
    const uint16_t * q; // fp16 [n_seq][T][hq][256]
    const void * k_new; // optional [n_seq][T][h_kv][256] fp16 / fp32: the step's new cells, appended by the launch
    const void * v_new;
    int32_t new_f32;
    float * po;         // [total_splits][h_kv][R][256] partial accumulators
    float * pml;        // [total_splits][h_kv][R][2] partial (m, l), base-2 domain
    float c2;           // scale * log2(e)
    int32_t layer, T, G, hq, R, n_seq, split_tokens;
    // dense: 1 when a sequence's n splits stride over its tiles (split j takes tiles j, j + n, ...; at most 64 a
    // split), 0 when split j takes the cells j split_tokens .. + split_tokens - 1
    int32_t strided;
    int32_t slot[FNKV_MAX_SEQS];
    // each sequence's context; with ctx_dev (dense) or depth_dev (sparse) set, the host's bound on it instead (the
    // launch's grid and workspace follow from the bound, the work from the device word, so one captured launch
    // serves every step up to the bound)
    int64_t ctx[FNKV_MAX_SEQS];
    int32_t split0[FNKV_MAX_SEQS + 1]; // first split of each sequence; split0[n_seq] = total
    const int64_t * ctx_dev = nullptr;   // dense: device contexts [n_seq], read by the launch; null: ctx[] are the contexts
    const int32_t * depth_dev = nullptr; // sparse: device depth (cells before the rows); ctx[0] bounds depth + T
    uint32_t * err = nullptr;            // with a device word: FNKV_DEV_ERR_DEPTH for a refused context (nothing written)
    // a sparse launch (one sequence, rows at positions ctx - T ..): the rows' selection bodies (qsa.h layout) and
    // where split 0 of head 0 stores the length of the selection's tile list for the merge (the list's entries are
    // spread over the launched splits: sparse_split_size; sel_split is the host's bound on a split's entries)
    const uint32_t * sel_body;
    int32_t * sel_n;
    int32_t sel_split;
    // prompt rows (qsp_attend): the bodies sit in slabs of kSlabRows rows (kSlabWords words a slab), row r's at word
    // offsets[(r / kSlabRows) * (kSlabRows + 1) + r % kSlabRows] / 4 of its slab; the launch's rows are rows
    // sel_row0 .. of that layout. Null: the rows' bodies are packed in order (qsa.h:77-81)
    const int32_t * sel_offsets = nullptr;
    int32_t sel_row0 = 0;
    fused_prep fp;
    // a sparse launch whose query is F32: q's fp16 low parts (fp16(q - hi), [T][hq][256], hi in q); the scores then
    // take q as hi + lo (about 22 significant bits). With fp.qfull set the launch forms both itself and only the
    // pointer's presence is read.
    const uint16_t * q_lo = nullptr;
    // the split-K fold inside the launch (stream kernel, grid resident at once): fold state words (kFoldWords a
    // (sequence, KV head); zeroed before a workspace's first launch, each launch leaves them ready for the next), the
    // fp16 output, and the bound of every wait
    // (real-time ticks, 100 MHz). Null: the splits' partials go to the merge kernel.
    uint32_t * fold = nullptr;
    uint16_t * out = nullptr;
    int64_t fold_spin = 0;
#ifdef FNKV_TIMING
    uint64_t * ts; // per workgroup: 16 real-time stamps (instrumented builds only)
#endif
};
// fold state of a (sequence, KV head): the arrival counter, a spare word, and a state word per row; a launch adds
// kFoldEpoch to the counter in all (more than any pair's splits)
constexpr int32_t kFoldWords = 2 + FNKV_MAX_ROWS;
constexpr uint32_t kFoldEpoch = 1024;

#ifdef FNKV_TIMING
#define FNKV_STAMP(k)                                                                                                \
    do {                                                                                                             \
        if (a.ts != nullptr && threadIdx.x == 0) {                                                                   \
            a.ts[(blockIdx.y * gridDim.x + blockIdx.x) * 16 + (k)] = __builtin_amdgcn_s_memrealtime();                   \
            a.ts[(blockIdx.y * gridDim.x + blockIdx.x) * 16 + 7] =                                                       \
                (uint64_t(__builtin_amdgcn_s_getreg((15 << 11) | 20)) << 32) |                                           \
                uint64_t(__builtin_amdgcn_s_getreg((31 << 11) | 4));                                                     \
        }                                                                                                            \
        __builtin_amdgcn_s_waitcnt(0);                                                                               \
    } while (0)
#define FNKV_STAMP_WAVE()                                                                                            \
    do {                                                                                                             \
        if (a.ts != nullptr && (threadIdx.x & 63) == 0 && a.sel_body == nullptr) {                                   \
            a.ts[(blockIdx.y * gridDim.x + blockIdx.x) * 16 + 8 + (threadIdx.x >> 6)] =                              \
                __builtin_amdgcn_s_memrealtime();                                                                    \
        }                                                                                                            \
        __builtin_amdgcn_s_waitcnt(0);                                                                               \
    } while (0)
#endif
#if defined(FNKV_TIMING) && defined(FNKV_TIMING_PHASES)
// phase clocks of wave 0 (20-bit shader cycle counter, no memory counters touched), summed over the loop: a build of
// their own, since the clock reads constrain the loop's schedule (and its registers) more than the stamps do
#define FNKV_PHASE_DECL() uint32_t ph_last = 0, ph_sum[8] = {0, 0, 0, 0, 0, 0, 0, 0}
#define FNKV_PHASE(p)                                                                                                \
    do {                                                                                                             \
        const uint32_t now = static_cast<uint32_t>(__builtin_amdgcn_s_memtime());                                  \
        if ((p) > 0) {                                                                                               \
            ph_sum[(p)-1] += now - ph_last;                                                                          \
        }                                                                                                            \
        ph_last = now;                                                                                               \
    } while (0)
#define FNKV_PHASE_STORE()                                                                                           \
    do {                                                                                                             \
        if (a.ts != nullptr && threadIdx.x == 0) {                                                                   \
            for (int p_ = 0; p_ < 8; ++p_) {                                                                         \
                a.ts[4096 * 16 + (blockIdx.y * gridDim.x + blockIdx.x) * 8 + p_] = ph_sum[p_];                        \
            }                                                                                                        \
        }                                                                                                            \
    } while (0)
#else
#define FNKV_PHASE_DECL()                                                                                            \
    do {                                                                                                             \
    } while (0)
#define FNKV_PHASE(p)                                                                                                \
    do {                                                                                                             \
    } while (0)
#define FNKV_PHASE_STORE()                                                                                           \
    do {                                                                                                             \
    } while (0)
#endif
#ifndef FNKV_TIMING
#define FNKV_STAMP_WAVE()                                                                                            \
    do {                                                                                                             \
    } while (0)
#define FNKV_STAMP(k)                                                                                                \
    do {                                                                                                             \
    } while (0)
#endif

// A sparse launch's selection as the workgroup sees it. Every workgroup rebuilds its row's list in LDS from the row's
// body (a few KB): the tiles the row selected, in ascending order, each with its 8 block bits (a 4-cell block a bit;
// the list entry's second word), are the list whose entries the splits take in turn. Rebuilding costs each workgroup
// one read of the body, which replaces the launch (and the memory round trip) that a separate planning kernel would
// add.
constexpr int32_t kSelMaxCells = 262144 + 32; // the reference's max_cells
constexpr int32_t kSelTopBlocks = 512;        // blocks a row (qsa.h)
constexpr int32_t kSelMaxRows = 5;
constexpr int32_t kSelMaxThreads = 512;
constexpr int32_t kSlabRows = 128;                          // prompt rows a slab (qsa_prompt.h prompt_slab)
constexpr int64_t kSlabWords = int64_t(kSlabRows) * (2 + kSelTopBlocks + 3); // a slab's bodies (max_row_words each)

// list entries a split takes when n_sel entries go to n_splits splits (at most 64: the host launches enough splits)
__host__ __device__ inline int32_t sparse_split_size(int32_t n_sel, int32_t n_splits) {
    const int32_t s = (n_sel + n_splits - 1) / n_splits;
    return s < 1 ? 1 : s;
}
constexpr int32_t kSelLds = (kSelTopBlocks + 1 + kSelMaxThreads / 64 + 1 + 64) * 4; // the build's scratch
constexpr int32_t kSelSlice = 64 * 8; // a split's entries (logical tile | row 4's bits << 16, rows 0-3's bits)

// hook: the caller's work while the body's loads are in flight (ALU only; run by every thread)
// The row view's selection (one row at q = ctx - 1): its K = min(n_vis, 512) block IDs (qsa.h:63-66: ascending) that
// lie in 0 .. n_vis - 1 (others are ignored), then its tail block n_vis when (q + 1) % 4 != 0; the list is the tiles of
// those blocks in order, each entry (tile | 0, the tile's 8 block bits) with the run of list blocks that share its tile
// (at most 8, distinct blocks being ascending). Two block-wide scans over at most 513 entries, no per-tile bitmap.
// Each thread keeps the blocks it loaded through the build (compaction keeps their order, so its kept blocks sit at
// consecutive list positions) and loads their physical pages as soon as the IDs arrive: the page-table round trip
// runs under the scans instead of after them, and the split's pages come out in page_l (lane i: entry i's page).
template <int32_t THREADS, typename HOOK>
__device__ void sparse_build(const dec_args & a, const int32_t * table, uint8_t * smem, uint2 * slice,
                             int32_t split, int32_t & n_tiles, int32_t & tile_l, int32_t & page_l,
                             int32_t & rank_of_new, const HOOK & hook) {
    static_assert(THREADS <= kSelMaxThreads && THREADS % 64 == 0, "scratch size");
    constexpr int32_t PER = (kSelTopBlocks + THREADS - 1) / THREADS; // consecutive IDs a thread
    constexpr int32_t WAVES = THREADS / 64;
    int32_t * blk = reinterpret_cast<int32_t *>(smem);   // [kSelTopBlocks + 1] the kept blocks, in order
    int32_t * wsum = blk + kSelTopBlocks + 1;             // [WAVES] wave totals of a scan
    int32_t * own = wsum + WAVES;                         // [1] the entry holding the row's own cell's tile
    int32_t * spage = own + 1;                            // [64] the split's entries' physical pages
    const int32_t tid = static_cast<int32_t>(threadIdx.x), lane = tid & 63, wave = tid >> 6;
    const int64_t q = a.ctx[0] - 1;
    const int32_t n_vis = static_cast<int32_t>((q + 1) / 4);
    const int32_t K = n_vis < kSelTopBlocks ? n_vis : kSelTopBlocks;
    const bool tail = (q + 1) % 4 != 0;
    const bool tail_mine = tail && tid == THREADS - 1; // the last thread: the tail comes after every kept block
    // a block-wide exclusive scan of one count a thread (thread order), and its total; the barriers leave global
    // loads in flight
    auto scan = [&](int32_t x, int32_t & excl, int32_t & total) {
        int32_t incl = x;
#pragma unroll
        for (int32_t o = 1; o < 64; o <<= 1) {
            const int32_t y = __shfl_up(incl, o);
            incl += lane >= o ? y : 0;
        }
        if (lane == 63) {
            wsum[wave] = incl;
        }
        barrier_keep_loads();
        int32_t wb = 0, tot = 0;
#pragma unroll
        for (int32_t w = 0; w < WAVES; ++w) {
            const int32_t v = wsum[w];
            wb += w < wave ? v : 0;
            tot += v;
        }
        excl = wb + incl - x;
        total = tot;
        barrier_keep_loads(); // wsum is free again
    };
    // the row's block IDs (one memory round trip), then the caller's work, then the kept blocks' pages
    int32_t b[PER];
#pragma unroll
    for (int32_t k = 0; k < PER; ++k) {
        const int32_t i = tid * PER + k;
        b[k] = i < K ? static_cast<int32_t>(a.sel_body[2 + i]) : -1;
    }
    int32_t tail_pg = tail_mine ? table[n_vis >> 6] : 0;
    if (tid == 0) {
        *own = -1;
    }
    hook();
    bool keep[PER];
    int32_t pg[PER];
    int32_t cnt = 0;
#pragma unroll
    for (int32_t k = 0; k < PER; ++k) {
        keep[k] = b[k] >= 0 && b[k] < n_vis;
        pg[k] = keep[k] ? table[b[k] >> 6] : 0; // block -> tile (8 blocks) -> page (8 tiles)
        cnt += keep[k] ? 1 : 0;
    }
    // the kept blocks, compacted in order, then the tail block (past every whole one)
    int32_t first = 0, n_kept = 0;
    scan(cnt, first, n_kept);
    int32_t pos[PER];
#pragma unroll
    for (int32_t k = 0, p = first; k < PER; ++k) {
        pos[k] = p;
        if (keep[k]) {
            blk[p++] = b[k];
        }
    }
    if (tail_mine) {
        blk[n_kept] = n_vis;
    }
    const int32_t n_all = n_kept + (tail ? 1 : 0);
    barrier_keep_loads();
    // a tile's first block in the list heads its entry; the entry's bits are its run's blocks
    auto head_bits = [&](int32_t i, int32_t v) -> uint32_t {
        if (i != 0 && (blk[i - 1] >> 3) == (v >> 3)) {
            return 0u;
        }
        uint32_t m = 0u;
        for (int32_t jj = i; jj < n_all && (blk[jj] >> 3) == (v >> 3); ++jj) {
            m |= 1u << (blk[jj] & 7);
        }
        return m;
    };
    int32_t heads = 0;
    uint32_t bits[PER];
#pragma unroll
    for (int32_t k = 0; k < PER; ++k) {
        bits[k] = keep[k] ? head_bits(pos[k], b[k]) : 0u;
        heads += bits[k] != 0u ? 1 : 0;
    }
    const uint32_t tail_bits = tail_mine ? head_bits(n_kept, n_vis) : 0u;
    heads += tail_bits != 0u ? 1 : 0;
    int32_t idx = 0, n_sel = 0;
    scan(heads, idx, n_sel);
    // the entries spread over all the launched splits (S each, the last ones short), so every workgroup gets work
    const int32_t S = sparse_split_size(n_sel, static_cast<int32_t>(gridDim.x));
    const int32_t e0 = split * S;
    const int32_t own_tile = static_cast<int32_t>(q >> 5);
    auto put = [&](int32_t tile, uint32_t m, int32_t page) {
        if (idx >= e0 && idx < e0 + S) {
            slice[idx - e0] = uint2{static_cast<uint32_t>(tile), m};
            spage[idx - e0] = page;
        }
        if (tile == own_tile) {
            *own = idx;
        }
        ++idx;
    };
#pragma unroll
    for (int32_t k = 0; k < PER; ++k) {
        if (bits[k] != 0u) {
            put(b[k] >> 3, bits[k], pg[k]);
        }
    }
    if (tail_bits != 0u) {
        put(n_vis >> 3, tail_bits, tail_pg);
    }
    barrier_keep_loads();
    const int32_t left = n_sel - e0;
    n_tiles = left < 0 ? 0 : left < S ? left : S;
    if (lane < n_tiles) {
        tile_l = static_cast<int32_t>(slice[lane].x & 0xffffu);
        page_l = spage[lane];
    }
    if (split == 0 && blockIdx.y == 0 && tid == 0) {
        *a.sel_n = n_sel;
    }
    // the row's own cell: written by the split that reads its tile (split 0 when no entry holds it)
    const int32_t o = *own;
    rank_of_new = (o >= 0 ? o / S : 0) == split ? 1 : 0;
    __syncthreads(); // the LDS is the ring's from here
}

// The tiles a workgroup walks. Dense: its split's consecutive cells begin .. end, lane i holding the physical page
// of the split's logical page i. Sparse: entries e0 .. e0 + n_tiles - 1 of the selection's tile list, kept in LDS
// (slice: past the ring) and, with LANES, also in lanes (lane i: entry i); lane i holds entry i's physical page.
// Tile ti of the walk is then a lane read (without LANES, plus one LDS read) either way.
__device__ __forceinline__ int32_t seq_of(const dec_args & a, int32_t split);

// A sparse launch runs each of its T rows as its own set of splits (blockIdx.z = row): this is the launch as row z
// sees it, one step token at position depth + z with its G query rows, its selection body (the words after the
// earlier rows', qsa.h:77-81), its list length slot and its region of the partials ([row][split][head][G] rows). With
// several rows the new cells are in the pool before the launch (a row may read an earlier row's new cell), or, when
// the launch prepares its rows (fused_prep), every workgroup that reads a new cell's tile writes the cell first; one
// row writes its own from k_new, by the split that reads its tile.
__device__ __forceinline__ dec_args sparse_row_view(const dec_args & in) {
    dec_args a = in;
    const int32_t z = static_cast<int32_t>(blockIdx.z);
    const int64_t depth = in.depth_dev != nullptr ? int64_t(*in.depth_dev) : in.ctx[0] - in.T;
    int64_t words = 0;
    if (in.sel_offsets != nullptr) { // a prompt row: its slab, then its offset in the slab
        const int32_t r = in.sel_row0 + z, slab = r / kSlabRows;
        words = int64_t(slab) * kSlabWords + in.sel_offsets[slab * (kSlabRows + 1) + r % kSlabRows] / 4;
    } else {
        for (int32_t t = 0; t < z; ++t) {
            const int64_t q = depth + t;
            const int64_t n_vis = (q + 1) / 4;
            words += 2 + (n_vis < 512 ? n_vis : 512) + (q + 1) % 4;
        }
    }
    const int64_t rows_all = int64_t(gridDim.x) * gridDim.y * in.G; // a row's partial rows
    a.T = 1;
    a.R = in.G;
    // a device depth outside 0 .. the bound (ctx[0] - T): marked by a negative context (sparse_refused)
    a.ctx[0] = in.depth_dev != nullptr && (depth < 0 || depth + in.T > in.ctx[0]) ? -1 : depth + z + 1;
    a.depth_dev = nullptr;
    a.q = in.q + int64_t(z) * in.hq * 256;
    if (in.q_lo != nullptr) {
        a.q_lo = in.q_lo + int64_t(z) * in.hq * 256;
    }
    a.sel_body = in.sel_body + words;
    a.sel_n = in.sel_n + z;
    a.po = in.po + int64_t(z) * rows_all * 256;
    a.pml = in.pml + int64_t(z) * rows_all * 2;
    if (in.T != 1) {
        a.k_new = nullptr;
        a.v_new = nullptr;
    }
    return a;
}

// A lane's page-table entry, loaded by every lane (a lane past the walk reads entry 0; guard_unmapped replaces its
// value), so the load is not under a branch: there the compiler would first wait for every load issued before it
// (the launch's Q rows)
__device__ __forceinline__ int32_t page_of(const int32_t * table, bool active, int32_t idx) {
    return table[active ? idx : 0];
}

template <bool SP, bool LANES = true> struct split_src {
    int32_t n_tiles = 0;
    int32_t page_lane = 0;
    int32_t new_mine = 0; // sparse: the new cells (bit t: cell ctx - T + t) this workgroup writes
    int64_t begin = 0;   // sparse: unused; dense: walk tile i is the sequence's tile g0 + stride i
    int32_t g0 = 0, stride = 1;
    const uint2 * slice = nullptr;
    uint32_t ent_x = 0, ent_y = 0; // sparse with LANES: lane i holds entry i (register reads instead of LDS reads)

    // ctx: the sequence's context (dense, strided: the page lookups are sized by the bound a.ctx[s], so they need
    // not wait for a context read from the device)
    template <int32_t THREADS>
    __device__ __forceinline__ void init(const dec_args & a, const int32_t * table, int32_t split, int64_t b,
                                         int64_t e, int32_t lane, uint8_t * smem, uint8_t * slice_lds,
                                         int64_t ctx = 0) {
        init<THREADS>(a, table, split, b, e, lane, smem, slice_lds, ctx, [] {});
    }
    // hook (sparse): work overlapped with the selection's loads (sparse_build)
    template <int32_t THREADS, typename HOOK>
    __device__ __forceinline__ void init(const dec_args & a, const int32_t * table, int32_t split, int64_t b,
                                         int64_t e, int32_t lane, uint8_t * smem, uint8_t * slice_lds,
                                         int64_t ctx, const HOOK & hook) {
        if constexpr (SP) {
            uint2 * sl = reinterpret_cast<uint2 *>(slice_lds);
            int32_t tile_l = 0, page_l = 0;
            sparse_build<THREADS>(a, table, smem, sl, split, n_tiles, tile_l, page_l, new_mine, hook);
            slice = sl;
            if (lane < n_tiles) {
                page_lane = page_l;
                if constexpr (LANES) {
                    ent_x = sl[lane].x;
                    ent_y = sl[lane].y;
                }
            }
        } else {
            // at most 64 walk tiles (splits of at most 2,048 cells), lane i holding walk tile i's page: contiguous,
            // the split's own cells; strided, split j of the sequence's n takes its tiles j, j + n, ...
            if (a.strided) {
                const int32_t s = seq_of(a, split);
                const int32_t j = split - a.split0[s], n = a.split0[s + 1] - a.split0[s];
                const int32_t tiles_cap = static_cast<int32_t>((a.ctx[s] + kTileTokens - 1) / kTileTokens);
                const int32_t cap_n = tiles_cap > j ? (tiles_cap - j + n - 1) / n : 0;
                page_lane = page_of(table, lane < cap_n, (j + n * lane) >> 3);
                const int32_t tiles = static_cast<int32_t>((ctx + kTileTokens - 1) / kTileTokens);
                g0 = j;
                stride = n;
                n_tiles = tiles > j ? (tiles - j + n - 1) / n : 0;
                return;
            } else {
                g0 = static_cast<int32_t>(b / kTileTokens);
                stride = 1;
                n_tiles = static_cast<int32_t>((e - b + kTileTokens - 1) / kTileTokens);
            }
            page_lane = page_of(table, lane < n_tiles, (g0 + stride * lane) >> 3);
        }
    }
    // A strided walk sized by the host's bound: its tile count for the sequence's actual context (read from the
    // device after the page lookups were issued)
    __device__ __forceinline__ void recount(int64_t ctx) {
        const int32_t tiles = static_cast<int32_t>((ctx + kTileTokens - 1) / kTileTokens);
        n_tiles = tiles > g0 ? (tiles - g0 + stride - 1) / stride : 0;
    }
    // A walk tile whose page is not mapped (page-table entry -1: the slot was trimmed under a captured launch, outside
    // the contract): its lanes read page 0 instead, so nothing faults, and the workgroup is told (uniform) so that it
    // writes no output for its sequence (its partials carry a NaN max: the merge writes nothing for such a row).
    // Lanes past the walk take page 0 too. Every dense walk calls this once its tile count is final.
    __device__ __forceinline__ bool guard_unmapped(int32_t lane) {
        const bool neg = lane < n_tiles && page_lane < 0;
        if (neg || lane >= n_tiles) {
            page_lane = 0;
        }
        return __any(neg);
    }
    __device__ __forceinline__ uint2 entry(int32_t ti) const {
        if constexpr (LANES) {
            return uint2{static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int32_t>(ent_x), ti)),
                         static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int32_t>(ent_y), ti))};
        } else {
            const uint2 v = slice[ti];
            return uint2{static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int32_t>(v.x))),
                         static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int32_t>(v.y)))};
        }
    }
    // byte offset of walk tile ti within the (layer, head) plane of the pool
    __device__ __forceinline__ int64_t tile_off(const pool_view & pv, int32_t ti) const {
        if constexpr (SP) {
            const int32_t phys = __builtin_amdgcn_readlane(page_lane, ti);
            const int32_t t8 = static_cast<int32_t>(entry(ti).x & 7u);
            return int64_t(phys) * pv.page_stride + int64_t(t8) * kTileBytes;
        } else {
            const int32_t phys = __builtin_amdgcn_readlane(page_lane, ti);
            return int64_t(phys) * pv.page_stride + int64_t((g0 + stride * ti) & 7) * kTileBytes;
        }
    }
    // the first cell of walk tile ti
    __device__ __forceinline__ int64_t tok0(int32_t ti) const {
        if constexpr (SP) {
            return int64_t(entry(ti).x & 0xffffu) * kTileTokens;
        } else {
            return int64_t(g0 + stride * ti) * kTileTokens;
        }
    }
    // the visibility bits of tile_softmax for this lane (query row of step token t_row, lane group qg)
    __device__ __forceinline__ uint32_t vis(int32_t ti, int32_t t_row, int32_t qg) const {
        if constexpr (SP) {
            const uint2 en = entry(ti);
            const uint32_t byte = t_row < 4 ? (en.y >> (8 * t_row)) : (en.x >> 16);
            return ((byte >> qg) & 1u) | (((byte >> (4 + qg)) & 1u) << 1);
        } else {
            return 3u;
        }
    }
};

// A dense sequence's context: the host's, or the device word's (ctx_dev). A sparse launch's row view holds its own.
template <bool SP> __device__ __forceinline__ int64_t seq_ctx(const dec_args & a, int32_t s) {
    if constexpr (!SP) {
        if (a.ctx_dev != nullptr) {
            // a vector load: a scalar one would hold up every later kernel-argument read until it returned
            return *(const volatile __attribute__((address_space(1))) int64_t *)(a.ctx_dev + s);
        }
    }
    return a.ctx[s];
}

// A device context outside T .. the host's bound: the sequence's workgroups write nothing (its first workgroup sets
// the error bit). Uniform across the workgroup.
template <bool SP>
__device__ __forceinline__ bool refused(const dec_args & a, int32_t s, int64_t ctx, int32_t sp, int32_t kvh) {
    if constexpr (!SP) {
        if (a.ctx_dev != nullptr && (ctx < a.T || ctx > a.ctx[s])) {
            if (sp == 0 && kvh == 0 && threadIdx.x == 0 && a.err != nullptr) {
                atomicOr(a.err, FNKV_DEV_ERR_DEPTH);
            }
            return true;
        }
    }
    return false;
}

// A dense walk over an unmapped page (split_src::guard_unmapped): with a device word, FNKV_DEV_ERR_DEPTH is set
__device__ __forceinline__ void report_unmapped(const dec_args & a, bool unmapped) {
    if (unmapped && threadIdx.x == 0 && a.err != nullptr) {
        atomicOr(a.err, FNKV_DEV_ERR_DEPTH);
    }
}

// A sparse row view refused by its device depth (sparse_row_view): nothing is written; the first workgroup of row 0
// sets the error bit.
__device__ __forceinline__ bool sparse_refused(const dec_args & a) {
    if (a.ctx[0] >= 0) {
        return false;
    }
    if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0 && a.err != nullptr) {
        atomicOr(a.err, FNKV_DEV_ERR_DEPTH);
    }
    return true;
}

// the step token of this lane's query row (rt * 16 + j); padding rows take the last
__device__ __forceinline__ int32_t t_of_row(const dec_args & a, int32_t rt, int32_t j) {
    const int32_t row = rt * 16 + j;
    return row < a.R ? row / a.G : a.T - 1;
}

// the split merge's arguments (merge_kernel): partials of n_seq sequences, split0 as in dec_args; for a sparse
// launch sel_n / sel_split bound the splits that ran
struct merge_args {
    const float * po;
    const float * pml;
    uint16_t * out; // fp16 [n_seq][T][hq][256]
    int32_t T, G, hq, R, h_kv, n_seq;
    int32_t split0[FNKV_MAX_SEQS + 1];
    const int32_t * sel_n; // sparse: each sequence's (row's) selection list length
    int32_t sel_split;
    // the launch's device word (dec_args): a refused sequence's (or sparse launch's) outputs are left as they were;
    // dense strided splits past a shorter context hold nothing
    const int64_t * ctx_dev = nullptr;
    const int32_t * depth_dev = nullptr;
    int64_t cap[FNKV_MAX_SEQS] = {0};
    int32_t T_dev = 0; // the launch's step tokens (rows of a sparse launch)
    // every sequence (row) holds uniform_splits splits: sequence s's first is s * uniform_splits (0: split0[])
    int32_t uniform_splits = 0;
    // the gated form's prompt output (qsp_attend): out16 fp16 [rows][hq][256] of the gated value (out_f32 optional),
    // bit 0 of *err set for a value that fp16 cannot hold (|x| > 65,504, or NaN); null: the activation format
    // the gated form (fn/kernels/qsa/attend.cu:619-655's finish): with out_f32 set, row (t, h)'s value d is written as
    // o / (1 + exp(-gate[(t hq + h) gate_stride + d])) in F32 [T][hq][256] with its int8 activation format (codes
    // [T][hq 256], act_scales [T][hq 8][2]) instead of the fp16 out
    const float * gate = nullptr;
    int32_t gate_stride = 0;
    float * out_f32 = nullptr;
    int8_t * codes = nullptr;
    float * act_scales = nullptr;
    uint16_t * out16 = nullptr;
    uint32_t * err = nullptr;
};

class kv_pool;
// host: the merge launch, and the sparse instantiation of the decode kernels (decode.hip)
void launch_merge(const merge_args & m, hipStream_t st);
// host: the dense launch's one-stream-a-wave kernel for NT = 1 .. 3 row tiles (stream.hip)
void launch_stream(int32_t device, int32_t NT, dim3 grid, const dec_args & a, hipStream_t st);
// the split size (cells) of a dense launch run by the stream kernel with NT row tiles
int32_t choose_split_stream(int32_t n_seq, const int64_t * ctx, int32_t h_kv, int32_t cus, int32_t NT);
void launch_decode_sparse(const kv_pool & p, int32_t NT, dim3 grid, const dec_args & a, hipStream_t st);
// host: a sparse launch over the pool (sparse.hip), optionally with the gated merge (merge_args' gated form)
struct sparse_gate {
    const float * gate;
    int32_t stride;
    float * out_f32;
    int8_t * codes;
    float * scales;
};
// a launch's depth read from device memory (the reference's depth word, attend.h:108): depth + T <= max_cells or
// the launch writes nothing and ORs FNKV_DEV_ERR_DEPTH into *err
struct dev_depth {
    const int32_t * depth;
    int64_t max_cells;
    uint32_t * err;
};
// dd set: `depth` is not read; the plan (grid, workspace) follows from dd->max_cells. q_lo set: q's fp16 low parts
// beside q (dec_args::q_lo), 16-byte aligned
int sparse_launch(const fnkv_pool * pool, int32_t slot, int64_t depth, int32_t T, int32_t layer, int32_t hq, float scale,
                  const void * q, const void * body, const void * offsets, const void * k_new, const void * v_new,
                  int32_t new_dtype, void * out, const sparse_gate * gate, void * ws, int64_t ws_bytes,
                  hipStream_t st, const char * who, const fused_prep * fp = nullptr, const dev_depth * dd = nullptr,
                  const uint16_t * q_lo = nullptr);
// host: prompt rows over their selection bodies (sparse.hip): the workspace of a chunk of n rows whose last row sees
// `cells` cells, and the chunk's launches (the sparse kernels, then the gated merge into out16 / out_f32 / err)
int64_t prompt_ws_bytes(const kv_pool & p, int64_t cells, int32_t n, int32_t G);
int prompt_launch(const kv_pool & p, int32_t slot, int32_t layer, int32_t pos0, int32_t row0, int32_t n, int32_t hq,
                  const uint16_t * q16, const uint32_t * body, const int32_t * offsets, const float * gate,
                  float * out_f32, uint16_t * out16, uint32_t * err, void * ws, hipStream_t st);
// LDS of the one-row sparse launch's formed query rows (after the tile buffers and the selection slice)
constexpr int32_t kFusedQLds = 16 * kHeadDim * 2;

__device__ __forceinline__ int32_t seq_of(const dec_args & a, int32_t split) {
    int32_t s = 0;
    while (s + 1 < a.n_seq && a.split0[s + 1] <= split) {
        ++s;
    }
    return s;
}

// The step's new cells ctx - T .. ctx - 1 that fall in this split [begin, end): quantized and written here (each
// position lies in exactly one split, so one workgroup writes it and only that workgroup reads it in this launch).
// The barrier's workgroup-scope release / acquire makes the stores visible to the workgroup's own later loads; an
// agent-scope fence would write back and invalidate the whole L2 under every other workgroup's stream.
// A sparse launch's workgroup writes the new cells set in `mine` (bit t: cell ctx - T + t) for its head.
template <int WAVES>
__device__ __forceinline__ void append_owned_cells(const dec_args & a, const int32_t * table, int32_t kvh,
                                                   int64_t ctx, int32_t mine, int32_t wave, int32_t lane) {
    if (a.k_new == nullptr || mine == 0) {
        return;
    }
    const pool_view & pv = a.pv;
    const int64_t first_new = ctx - a.T;
    for (int32_t job = wave; job < 2 * a.T; job += WAVES) {
        const int32_t t = job >> 1, kv = job & 1;
        if (((mine >> t) & 1) == 0) {
            continue;
        }
        const int64_t pos = first_new + t;
        const int64_t src = (int64_t(t) * pv.h_kv + kvh) * kHeadDim;
        float x[4];
        if (a.new_f32) {
            load4<true>(static_cast<const float *>(kv ? a.v_new : a.k_new) + src, lane, x);
        } else {
            load4<false>(static_cast<const uint16_t *>(kv ? a.v_new : a.k_new) + src, lane, x);
        }
        quantize_store_fmt(x, lane, tile_of(pv, table, a.layer, kvh, pos), static_cast<int32_t>(pos & 31), kv,
                           pv.format);
    }
    __syncthreads();
}

template <int WAVES>
__device__ __forceinline__ void append_new_cells(const dec_args & a, const int32_t * table, int32_t s, int32_t kvh,
                                                 int64_t ctx, int64_t begin, int64_t end, int32_t sj, int32_t sn,
                                                 int32_t wave, int32_t lane) {
    if (a.k_new == nullptr) {
        return;
    }
    const pool_view & pv = a.pv;
    const int64_t first_new = ctx - a.T;
    // a new cell is written by the workgroup whose walk holds its tile: the split of its cell range, or (strided,
    // sn splits) split tile % sn
    for (int32_t job = wave; job < 2 * a.T; job += WAVES) {
        const int64_t pos = first_new + (job >> 1);
        const bool mine = sn != 0 ? static_cast<int32_t>((pos >> 5) % sn) == sj : (pos >= begin && pos < end);
        if (!mine) {
            continue;
        }
        const int32_t kv = job & 1;
        if (table[pos >> 8] < 0) {
            continue; // an unmapped page (outside the contract): nothing is written
        }
        const int64_t src = ((int64_t(s) * a.T + (pos - first_new)) * pv.h_kv + kvh) * kHeadDim;
        float x[4];
        if (a.new_f32) {
            load4<true>(static_cast<const float *>(kv ? a.v_new : a.k_new) + src, lane, x);
        } else {
            load4<false>(static_cast<const uint16_t *>(kv ? a.v_new : a.k_new) + src, lane, x);
        }
        quantize_store_fmt(x, lane, tile_of(pv, table, a.layer, kvh, pos), static_cast<int32_t>(pos & 31), kv,
                           pv.format);
    }
    __syncthreads();
}

// Query row tile rt (row 16 rt + j of the G T rows of KV head kvh; padding rows read as zero and take the last
// token's causal limit): the Q operands (B of S^T = K Q^T: lane (row j, group qg) holds q[row][32 b + 8 qg .. + 7])
// and the bias operand. K codes enter the MFMA as 1152 + code, so S^T carries 1152 * sum_b s_k[t][b] * sigma_b[row]
// with sigma_b the block's sum of q; one MFMA a half computes that sum from the K scales (A: s_k twice) and sigma_b as
// hi + lo fp16 (B: lane (row j, qg) holds sigma_hi for qg 0, sigma_lo for qg 1, else 0), and one FMA a score takes it
// back out. lim: the row's last visible cell.
// load_q_operands only issues the loads; q_sums reads them, so a kernel can issue its first tile copies in between.
__device__ __forceinline__ void load_q_operands(const dec_args & a, int32_t s, int64_t ctx, int32_t kvh, int32_t rt,
                                                int32_t j, int32_t qg, half8 (&qop)[kBlocks], int64_t & lim) {
    const int32_t row = rt * 16 + j;
    const bool real_row = row < a.R;
    const int32_t t_row = real_row ? row / a.G : a.T - 1;
    lim = ctx - a.T + t_row;
    const uint16_t * qrow =
        a.q + ((int64_t(s) * a.T + t_row) * a.hq + int64_t(kvh) * a.G + (real_row ? row % a.G : 0)) * kHeadDim;
#pragma unroll
    for (int b = 0; b < kBlocks; ++b) {
        u32x4 v = {0, 0, 0, 0};
        if (real_row) {
            v = *reinterpret_cast<const u32x4 *>(qrow + b * kQK + 8 * qg);
        }
        qop[b] = __builtin_bit_cast(half8, v);
    }
}

// The scores' optional second Q operand: none (q is the fp16 operand alone), or q's fp16 low parts, block b's from
// qlo(b), chained into the same MFMA results as the hi parts (the K codes then enter exactly, without the bias).
struct no_qlo {
    __device__ half8 operator()(int) const { return half8{}; }
};
template <typename QLOP> constexpr bool has_qlo = !std::is_same<QLOP, no_qlo>::value;

// sig: the row's per-block sums of q (the bias correction's operand), as fp16 hi (qg = 0) and lo (qg = 1) parts
__device__ __forceinline__ half8 q_sums(const half8 (&qop)[kBlocks], int32_t qg) {
    float sigma[kBlocks];
#pragma unroll
    for (int b = 0; b < kBlocks; ++b) {
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            sum += static_cast<float>(qop[b][i]);
        }
        sigma[b] = rows_sum(sum);
    }
    half8 sig;
#pragma unroll
    for (int b = 0; b < kBlocks; ++b) {
        const _Float16 hi = static_cast<_Float16>(sigma[b]);
        const _Float16 lo = static_cast<_Float16>(sigma[b] - static_cast<float>(hi));
        sig[b] = qg == 0 ? hi : qg == 1 ? lo : static_cast<_Float16>(0.0f);
    }
    return sig;
}

// S^T = K Q^T for one 16-token half h of a tile from its K codes (kb) and scales (sc_tile + kKScales ...) in LDS:
// the returned r-th value is the score of token 16 h + 4 qg + r against this lane's row j, unscaled (q . k).
// The Q operand of block b comes from qop(b): registers, or LDS where registers are short.
// PAIR (KV8 pools): the two blocks of a 64-value group share one scale, so their MFMAs chain into one result and
// the scale applies once a group.
template <typename QOP, bool PAIR = false, typename QLOP = no_qlo>
__device__ __forceinline__ floatx4 tile_scores_half(const uint8_t * kb, const uint8_t * sc_tile, const QOP & qop,
                                                    half8 sig, int32_t j, int32_t qg, int32_t lane, int32_t h,
                                                    const QLOP & qlo = QLOP()) {
    const half8 zero8 = {};
    // this lane's score rows are tokens 16 h + 4 qg + r; their K scales, all 8 blocks
    half8 ks[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        ks[r] = *reinterpret_cast<const half8 *>(sc_tile + kKScales + (16 * h + 4 * qg + r) * 16);
    }
    // the bias term: A = this lane's token row of K scales (twice), B = sigma hi / lo. With q's low parts the codes
    // enter exactly instead: the bias's partial sums (1152 sum q) would cost the fp32 accumulation ~8 bits
    floatx4 corr = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (!has_qlo<QLOP>) {
        const half8 srow = qg < 2 ? *reinterpret_cast<const half8 *>(sc_tile + kKScales + (16 * h + j) * 16) : zero8;
        corr = mfma16(srow, sig, floatx4{0.0f, 0.0f, 0.0f, 0.0f});
    }
    floatx4 acc_s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) { // blocks 4 hb .. 4 hb + 3 (fewer live results)
        floatx4 t[4];
#pragma unroll
        for (int ld = 2 * hb; ld < 2 * hb + 2; ++ld) {
            const u32x4 kw = *reinterpret_cast<const u32x4 *>(kb + h * 4096 + ld * 1024 + lane * 16);
#pragma unroll
            for (int bb = 0; bb < 2; ++bb) {
                const int b = 2 * ld + bb;
                const half8 ka = widen8<has_qlo<QLOP>>(kw[2 * bb], kw[2 * bb + 1]);
                if constexpr (PAIR) { // group ld = blocks 2 ld, 2 ld + 1 (one 1 KiB chunk)
                    t[ld - 2 * hb] = mfma16(ka, qop(b), bb == 0 ? floatx4{0.0f, 0.0f, 0.0f, 0.0f} : t[ld - 2 * hb]);
                    if constexpr (has_qlo<QLOP>) {
                        t[ld - 2 * hb] = mfma16(ka, qlo(b), t[ld - 2 * hb]);
                    }
                } else {
                    t[b - 4 * hb] = mfma16(ka, qop(b), floatx4{0.0f, 0.0f, 0.0f, 0.0f});
                    if constexpr (has_qlo<QLOP>) {
                        t[b - 4 * hb] = mfma16(ka, qlo(b), t[b - 4 * hb]);
                    }
                }
            }
        }
        if constexpr (PAIR) {
#pragma unroll
            for (int ld = 2 * hb; ld < 2 * hb + 2; ++ld) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    acc_s[r] = __builtin_fmaf(static_cast<float>(ks[r][2 * ld]), t[ld - 2 * hb][r], acc_s[r]);
                }
            }
        } else {
#pragma unroll
            for (int b = 4 * hb; b < 4 * hb + 4; ++b) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    acc_s[r] = __builtin_fmaf(static_cast<float>(ks[r][b]), t[b - 4 * hb][r], acc_s[r]);
                }
            }
        }
    }
    if constexpr (has_qlo<QLOP>) {
        return acc_s;
    }
    floatx4 sc;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        sc[r] = __builtin_fmaf(-1152.0f, corr[r], acc_s[r]);
    }
    return sc;
}

// both halves: sc[h][r] is the score of token 16 h + 4 qg + r against this lane's row j
template <bool PAIR = false, typename QOP, typename QLOP = no_qlo>
__device__ __forceinline__ void tile_scores(const uint8_t * kb, const uint8_t * sc_tile, const QOP & qop, half8 sig,
                                            int32_t j, int32_t qg, int32_t lane, floatx4 (&sc)[2],
                                            const QLOP & qlo = QLOP()) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        sc[h] = tile_scores_half<QOP, PAIR, QLOP>(kb, sc_tile, qop, sig, j, qg, lane, h, qlo);
#ifndef FNKV_NO_HALF_SB
        __builtin_amdgcn_sched_barrier(0); // one half's operands live at a time
#endif
    }
}

// Online softmax (base 2) of a tile's scores for this lane's row, tokens past lim_rel (tile-relative) masked. The
// row's reference m_run moves only when the tile's max exceeds it by more than kLazyLog2 (then alpha = 2^(m_old - m),
// the factor the row's accumulators take before this tile's terms; else alpha = 1), so the rescale of the
// accumulators is rare; the weights pf[4 h + r] = 2^(c2 sc - m_run) stay <= 2^kLazyLog2 = 64, which keeps a weight
// times a V scale (at most 65504 / 127) inside fp16. alpha is the same in the row's four lanes.
constexpr float kLazyLog2 = 6.0f;
// vis: bit h set when this lane's 4 cells of half h (one 4-cell block) are in its row's selection (dense: 3).
// EXACT_MAX (the launches that take q as hi + lo): m_run follows every new max and the weights are 2^(c2 sc - m_run
// + kLazyLog2), the row's largest exactly 64 (the same bound). The weights, l and the accumulators then carry a
// common 2^6, which cancels in every fold (l and O scale together); the gain: a weight times a V scale keeps 6 more
// bits above fp16's subnormal range in its lo part (a weight near 1 times a scale near 2^-6 has lo near 2^-18).
template <bool EXACT_MAX = false>
__device__ __forceinline__ void tile_softmax(const floatx4 (&sc)[2], int32_t lim_rel, float c2, int32_t qg,
                                             float & m_run, float & l_run, float (&pf)[8], float & alpha,
                                             uint32_t vis = 3) {
    // the max runs on the raw scores (c2 > 0 keeps the order); each weight is one FMA and one exp2
    float raw[8];
    float mx = kNegInf;
    if (__all(lim_rel >= 31 && vis == 3)) { // the whole tile is visible to every row of the wave
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                raw[4 * h + r] = sc[h][r];
                mx = fmaxf(mx, raw[4 * h + r]);
            }
        }
    } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float x = (16 * h + 4 * qg + r <= lim_rel && ((vis >> h) & 1u)) ? sc[h][r] : kNegInf;
                raw[4 * h + r] = x;
                mx = fmaxf(mx, x);
            }
        }
    }
    mx = rows_max(mx) * c2;
    const bool move = mx > m_run + (EXACT_MAX ? 0.0f : kLazyLog2); // m_run = -inf: any visible score moves it
    const float m_new = move ? mx : m_run;
    const float m_use = m_new == kNegInf ? 0.0f : m_new;
    alpha = move ? __builtin_amdgcn_exp2f(m_run - m_use) : 1.0f;
    const float m_pf = EXACT_MAX ? m_use - kLazyLog2 : m_use;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        pf[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(raw[i], c2, -m_pf));
    }
    l_run = __builtin_fmaf(l_run, alpha, sum8(pf));
    m_run = m_new;
}

} // namespace fnkv
