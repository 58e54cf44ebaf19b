// The draft block's dense F16 attention (DA-TC, fn/kernels/draft/draft.h:47-83): the prepare of a round's rows (F32
// RMS norm and IMROPE of the query heads and of k, the F16 K / V cache writes, q / 16 in F16) and the attention of one
// row over every cell before it (or over a selection body, SP2), gated by sigmoid(gate) and written in F32 and in the
// int8 activation format. The caches are flat F16 [max_cells][256] arrays of one KV head, 1,024 B a cell for K and V.
//
// How (MI355X):
//   * prepare: a workgroup a row, a wave a query head (12) and one for k / v; a lane holds 4 of the 256 values.
//   * attend: a fixed grid of kGrid workgroups of 4 waves (the depth is a device word, so the grid cannot depend on
//     it); the first A = min(kGrid, ceil(tiles / 4)) stride over the 32-cell tiles, wave w of workgroup b taking
//     tiles w + 4 (b + A i), so the workgroups read one window of the caches together (measured: a contiguous range
//     a workgroup streams ~18% slower). A wave's step, all on the matrix cores (v_mfma_f32_16x16x32_f16):
//       S^T = K Q^T: K rows straight from HBM into registers (buffer loads; cells past the row read as zeros), the 12
//         heads (padded to 16) of q16 held in registers for the whole launch; lane l ends with head l % 16's scores
//         of cells 4 (l / 16) .. + 3 of each 16-cell half, so the online softmax needs no transposition: its max
//         and sum cross the four 16-lane rows by two lane swaps.
//       O^T += V^T P^T: the lane's own 8 rounded probabilities are the B operand as they stand (the MFMA's k slots
//         mapped onto those 8 cells); the V tile comes into the wave's LDS buffer by direct global-to-LDS copies (two
//         cells a copy, copies padded apart) and each lane's A operand (8 cells of one dimension) is two transposing
//         reads (ds_read_b64_tr_b16). The accumulators hold O^T, so the per-head rescale is the lane's own.
//     The next tile's K (registers) and V (the other LDS buffer) are in flight while one is computed. The 4 waves
//     fold into one partial per workgroup in LDS.
//   * fold: a workgroup per (head, 32-value run): the partials folded in workgroup order with exp(m_c - M), the gate,
//     the F32 output and the run's activation format.
// Numerics (draft.h:69-77): exact F16 products, F32 accumulation, P rounded to F16 (nearest even), l the sum of the
// rounded P; every reduction order is fixed, so reruns are bitwise.
#include "../../include/fnkv.h"
#include "common.h"
#include "mfma.h"
#include "rope.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <mutex>
#include <string>

namespace fnkv {
namespace {

constexpr int32_t kHeads = FNKV_DATC_HEADS;
constexpr int32_t kD = 256;
constexpr int32_t kQS = FNKV_DATC_QSTRIDE;
constexpr int32_t kGrid = 256;          // attention workgroups
constexpr int32_t kWaves = 4;
constexpr int32_t kTile = 32;           // cells a wave's step
constexpr int32_t kPartFloats = kHeads * kD + 2 * kHeads; // a workgroup's O [12][256], then m [12] and l [12]
constexpr int32_t kVPair = 2 * 512 + 64;                  // LDS bytes of two cells' V rows, padded
constexpr int32_t kVBuf = (kTile / 2) * kVPair;           // a tile's V rows: 17,408 B (two a wave)
constexpr int32_t kOStride = kD + 4;                      // floats a head's row of a wave's O in LDS (wave fold)
constexpr int32_t kFoldLds = kWaves * kHeads * kOStride * 4; // the waves' O, over the V buffers at the end
constexpr int32_t kMlLds = kFoldLds > 2 * kWaves * kVBuf ? kFoldLds : 2 * kWaves * kVBuf; // waves' m, l: past both
constexpr int32_t kQLds = kMlLds + 2 * kWaves * 16 * 4;      // the fused step's q16 [12][256]
constexpr int32_t kAttendLds = kQLds + kHeads * kD * 2;
constexpr int32_t kSelRatio = 4, kSelBlocks = 512;
constexpr uint32_t kOob = 0x80000000u;                    // a buffer offset past every cache: reads as zero
constexpr int32_t kEmptyTile = 1 << 30;                   // a tile base past every row: an empty step

static_assert(kGrid == 256, "the fold: a thread's partial weight, 8 groups of kGrid / 8 partials");

#ifdef FNKV_TIMING
__device__ uint64_t * g_datc_ts;
} // namespace
uint64_t * timing_buffer();
namespace {
// instrumented builds: real-time stamps of workgroup `slot`'s phases (16 a workgroup; attend slots 0..255, fold
// 256..351, prepare 352..)
#define DATC_STAMP(slot, k)                                                                                          \
    do {                                                                                                             \
        if (ts != nullptr && threadIdx.x == 0) {                                                                     \
            ts[(slot) * 16 + (k)] = __builtin_amdgcn_s_memrealtime();                                                \
        }                                                                                                            \
    } while (0)
#else
#define DATC_STAMP(slot, k) ((void)0)
#endif

// ---- prepare ----

// the prepare's refusal: a row's cell outside the caches, or rows past the round's
__device__ __forceinline__ bool prepare_refused(const fnkv_datc_prepare_args & a, int32_t rows) {
    const int32_t nb = *a.n_before, stride = *a.stride;
    return nb < 0 || static_cast<int64_t>(nb) + a.row0 + rows > a.max_cells || a.row0 + rows > stride;
}

__global__ __launch_bounds__(64 * (kHeads + 1)) void datc_prepare_kernel(fnkv_datc_prepare_args a, int32_t rows) {
    const int32_t wave = static_cast<int32_t>(threadIdx.x) / 64, lane = static_cast<int32_t>(threadIdx.x) % 64;
    const int32_t t = static_cast<int32_t>(blockIdx.x);
#ifdef FNKV_TIMING
    uint64_t * ts = g_datc_ts;
#endif
    DATC_STAMP(352 + t, 0);
    const int32_t nb = *a.n_before, stride = *a.stride;
    if (nb < 0 || static_cast<int64_t>(nb) + a.row0 + rows > a.max_cells || a.row0 + rows > stride) {
        if (threadIdx.x == 0) {
            atomicOr(a.err, FNKV_DEV_ERR_DRAFT_DEPTH);
        }
        return;
    }
    const int32_t col = a.row0 + t;
    float y[4];
    if (wave < kHeads) {
        if (a.qfull == nullptr) {
            return;
        }
        norm_rope(y, a.qfull + (t * kHeads + wave) * kQS, a.q_norm, a.pos, stride, col, a.theta_scale, lane);
        if (a.q_f32 != nullptr) {
            reinterpret_cast<float4 *>(a.q_f32 + (t * kHeads + wave) * kD)[lane] = make_float4(y[0], y[1], y[2], y[3]);
        }
        reinterpret_cast<uint2 *>(a.q16 + (t * kHeads + wave) * kD)[lane] = pack4_f16(y, 1.0f / 16.0f);
        DATC_STAMP(352 + t, 1);
        return;
    }
    norm_rope(y, a.kv_k + t * kD, a.k_norm, a.pos, stride, col, a.theta_scale, lane);
    if (a.k_f32 != nullptr) {
        reinterpret_cast<float4 *>(a.k_f32 + t * kD)[lane] = make_float4(y[0], y[1], y[2], y[3]);
    }
    const int64_t at = (static_cast<int64_t>(nb) + col) * kD;
    reinterpret_cast<uint2 *>(a.k_cache + at)[lane] = pack4_f16(y, 1.0f);
    const float4 v4 = reinterpret_cast<const float4 *>(a.kv_v + t * kD)[lane];
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    reinterpret_cast<uint2 *>(a.v_cache + at)[lane] = pack4_f16(v, 1.0f);
}

// ---- attend ----

// The row's logical cells: n of them; cell i is i (dense) or, SP2, the i-th of the selection (its K blocks' cells,
// then 4 n_vis .. N + row0). valid false: the launch must write nothing (a depth outside the caches, a body not made
// at this depth).
struct datc_shape {
    int32_t n = 0, K = 0, n_vis = 0, n_tiles = 0, active = 0;
    bool valid = false;
};

template <bool SP> __device__ __forceinline__ datc_shape datc_shape_of(const fnkv_datc_attend_args & a) {
    datc_shape s;
    const int32_t nb = *a.n_before;
    const int64_t n64 = static_cast<int64_t>(nb) + a.row0 + 1;
    s.n_vis = nb / kSelRatio;
    s.K = SP ? static_cast<int32_t>(a.body[0]) : 0;
    s.valid = nb >= 0 && n64 <= a.max_cells && (!SP || s.K == min(s.n_vis, kSelBlocks));
    if (!s.valid) {
        return s;
    }
    s.n = SP ? kSelRatio * s.K + static_cast<int32_t>(n64) - kSelRatio * s.n_vis : static_cast<int32_t>(n64);
    s.n_tiles = (s.n + kTile - 1) / kTile;
    s.active = min(kGrid, (s.n_tiles + kWaves - 1) / kWaves);
    return s;
}

// logical cell i (< n) to its cache cell
template <bool SP>
__device__ __forceinline__ int32_t cell_of(const fnkv_datc_attend_args & a, const datc_shape & s, int32_t i) {
    if constexpr (!SP) {
        return i;
    } else {
        return i < kSelRatio * s.K ? kSelRatio * static_cast<int32_t>(a.body[2 + i / kSelRatio]) + (i & 3)
                                   : kSelRatio * s.n_vis + (i - kSelRatio * s.K);
    }
}

// K of a tile in registers, as the S^T operand
struct k_tile {
    u32x4 r[2][8]; // [16-cell half][32-dim slice]: lane l's 8 dims 32 j + 8 (l / 16) .. of cell 16 half + l % 16
};

// LDS byte offset of cell c's V row in a tile buffer: two cells a copy (contiguous), copies kVPair apart
__device__ __forceinline__ int32_t v_cell_off(int32_t c) {
    return (c >> 1) * kVPair + (c & 1) * 512;
}

// issue one tile's 32 loads: K into registers, V into the wave's LDS buffer; cells past the row read as zeros
template <bool SP>
__device__ __forceinline__ void issue_tile(const fnkv_datc_attend_args & a, const datc_shape & s, rsrc_t rk, rsrc_t rv,
                                           int32_t base, k_tile & kt, uint8_t * vbuf, int32_t lane) {
    // SP2: lane l < 32 resolves logical cell base + l (a body word) and the others take it by lane exchange; dense:
    // logical cell i is cell i
    int32_t mine = 0;
    if constexpr (SP) {
        const int32_t li = base + (lane & 31);
        mine = li < s.n ? cell_of<SP>(a, s, li) : -1;
    }
    auto cell = [&](int32_t i) {
        if constexpr (SP) {
            return __shfl(mine, i, 64);
        } else {
            return base + i < s.n ? base + i : -1;
        }
    };
    const int32_t g = lane / 16;
#pragma unroll
    for (int32_t h = 0; h < 2; ++h) {
        const int32_t c = cell(16 * h + lane % 16);
        const uint32_t off = c >= 0 ? static_cast<uint32_t>(c) * 512u + 16u * static_cast<uint32_t>(g) : kOob;
#pragma unroll
        for (int32_t j = 0; j < 8; ++j) {
            kt.r[h][j] = buf_load16(rk, static_cast<int32_t>(off), 64 * j);
        }
    }
#pragma unroll
    for (int32_t c2 = 0; c2 < kTile / 2; ++c2) {
        const int32_t c = cell(2 * c2 + lane / 32);
        const uint32_t off = c >= 0 ? static_cast<uint32_t>(c) * 512u + 16u * static_cast<uint32_t>(lane % 32) : kOob;
        buf_lds16(rv, vbuf + c2 * kVPair, static_cast<int32_t>(off), 0);
    }
}

// 4 fp16 values by the transposing LDS read (ds_read_b64_tr_b16): within each 16-lane group, lane j supplies the
// address of 4 consecutive values M[j][0..3]; lane i receives M[4 k + i / 4][i % 4] for k = 0..3
__device__ __forceinline__ u32x2 lds_read_tr4(const uint8_t * p) {
    typedef short short4v __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) short4v * lds_s4;
    const short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(p));
    return __builtin_bit_cast(u32x2, r);
}

// one tile's step: the next tile's loads issued (K into kn, V into vnext), then, once this tile's have landed (K in kt,
// V in vbuf), the scores, the online softmax (m, l of head lane % 16), O^T rescaled and accumulated. The two LDS
// buffers are distinct restrict pointers here, which tells the compiler that the reads of vbuf do not depend on the
// copies into vnext: it then waits for this tile's copies only, not for the next tile's.
// STEP: kIssueNext (issue the next tile, then wait for this one), kNextIssued (the next tile is already in flight:
// wait for this one), kLast (no next tile: wait for everything)
constexpr int kIssueNext = 0, kNextIssued = 1, kLast = 2;
template <bool SP, int STEP>
__device__ __forceinline__ void tile_step(const fnkv_datc_attend_args & a, const datc_shape & s, rsrc_t rk, rsrc_t rv,
                                          const k_tile & kt, k_tile & kn, const uint8_t * __restrict__ vbuf,
                                          uint8_t * __restrict__ vnext, int32_t base, int32_t next_base,
                                          const half8 (&qb)[8], float & m_run, float & l_run, floatx4 (&o)[16],
                                          int32_t lane) {
    // the next tile's loads go out before anything of this step (the scheduler may not sink them below the scores)
    if constexpr (STEP == kIssueNext) {
        issue_tile<SP>(a, s, rk, rv, next_base, kn, vnext, lane);
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<32>();
    } else if constexpr (STEP == kNextIssued) {
        wait_vmcnt<32>();
    } else {
        wait_vmcnt<0>();
    }
    __builtin_amdgcn_sched_barrier(0);
#ifdef FNKV_TIMING
    {
        uint64_t * ts = g_datc_ts;
        if (ts != nullptr && threadIdx.x == 0 && ts[blockIdx.x * 16 + 1] == 0) {
            ts[blockIdx.x * 16 + 1] = __builtin_amdgcn_s_memrealtime();
        }
    }
#endif
    const int32_t n = s.n;
    const int32_t g = lane / 16;
    floatx4 st[2];
#pragma unroll
    for (int32_t h = 0; h < 2; ++h) {
        floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int32_t j = 0; j < 8; ++j) {
            acc = mfma16(__builtin_bit_cast(half8, kt.r[h][j]), qb[j], acc);
        }
        st[h] = acc;
    }
    // lane l: head l % 16, cells 16 h + 4 g + i
    float sv[8];
    float mx = -INFINITY;
#pragma unroll
    for (int32_t h = 0; h < 2; ++h) {
#pragma unroll
        for (int32_t i = 0; i < 4; ++i) {
            const float v = base + 16 * h + 4 * g + i < n ? st[h][i] : -INFINITY;
            sv[4 * h + i] = v;
            mx = fmaxf(mx, v);
        }
    }
    mx = rows_max(mx);
    const float m_new = fmaxf(m_run, mx);
    u32x4 pw;
    float sum = 0.0f;
#pragma unroll
    for (int32_t i = 0; i < 4; ++i) {
        const _Float16 p0 = static_cast<_Float16>(expf(sv[2 * i] - m_new));
        const _Float16 p1 = static_cast<_Float16>(expf(sv[2 * i + 1] - m_new));
        sum += static_cast<float>(p0);
        sum += static_cast<float>(p1);
        pw[i] = __builtin_bit_cast(uint32_t, half2v{p0, p1});
    }
    sum = rows_sum(sum);
    const float alpha = expf(m_run - m_new); // 0 for the wave's first tile (m_run = -inf)
    m_run = m_new;
    l_run = __builtin_fmaf(l_run, alpha, sum);
    const half8 pb = __builtin_bit_cast(half8, pw);
    // the A operand of dims 16 db + i (i = l % 16): k slots 8 g .. + 3 are cells 4 g .. + 3, slots 8 g + 4 .. + 7
    // cells 16 + 4 g .. + 3 (pb's order); lane j = l % 16 of the group addresses cell (j / 4) of each four, dims
    // 4 (j % 4) .. + 3 of the 16
    const int32_t j = lane % 16;
    const uint8_t * r0 = vbuf + v_cell_off(4 * g + j / 4) + 8 * (j % 4);
    const uint8_t * r1 = vbuf + v_cell_off(16 + 4 * g + j / 4) + 8 * (j % 4);
#pragma unroll
    for (int32_t db = 0; db < 16; ++db) {
        const u32x2 lo = lds_read_tr4(r0 + 32 * db);
        const u32x2 hi = lds_read_tr4(r1 + 32 * db);
        const u32x4 va = {lo[0], lo[1], hi[0], hi[1]};
        o[db] = mfma16(__builtin_bit_cast(half8, va), pb, o[db] * alpha);
    }
}

// FUSED: the wave's three heads' inputs and the lane's position are loaded before the first tile's loads (the loads
// return in order: issued after them, they would wait for the whole tile), then the tile is issued (unconditionally: a
// wave without tiles issues the empty tile, zeros and no memory traffic, so the waits for the q inputs count past the
// tile's loads instead of draining them at a branch join), then the heads are formed into LDS while it is in flight.
// The V buffer and the q rows are distinct LDS regions (restrict), so the q writes need not wait for the V copies.
template <bool SP, bool TWO>
__device__ __forceinline__ void fused_first_tile(const fnkv_datc_attend_args & a, const fnkv_datc_prepare_args & pa,
                                                 const datc_shape & s, rsrc_t rk, rsrc_t rv, int32_t base,
                                                 int32_t base1, k_tile & kt, k_tile & kt1, uint8_t * __restrict__ vbuf,
                                                 uint8_t * __restrict__ vbuf1, uint16_t * __restrict__ ql,
                                                 half8 (&qb)[8], int32_t b, int32_t wave, int32_t lane) {
    constexpr int32_t kPer = kHeads / kWaves;
    float4 xq[kPer];
#pragma unroll
    for (int32_t i = 0; i < kPer; ++i) {
        xq[i] = reinterpret_cast<const float4 *>(pa.qfull + (kPer * wave + i) * kQS)[lane];
    }
    const float4 gq = reinterpret_cast<const float4 *>(pa.q_norm)[lane];
    const int32_t pq = rope_pos(pa.pos, *pa.stride, pa.row0, lane);
    __builtin_amdgcn_sched_barrier(0);
    issue_tile<SP>(a, s, rk, rv, base, kt, vbuf, lane);
    if constexpr (TWO) {
        issue_tile<SP>(a, s, rk, rv, base1, kt1, vbuf1, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    float sn, cs;
    rope_angle(sn, cs, pq, pa.theta_scale, lane);
#pragma unroll
    for (int32_t i = 0; i < kPer; ++i) {
        const int32_t h = kPer * wave + i;
        float y[4];
        norm_rope_apply(y, xq[i], gq, sn, cs, lane);
        const uint2 q4 = pack4_f16(y, 1.0f / 16.0f);
        reinterpret_cast<uint2 *>(ql + h * kD)[lane] = q4;
        if (b == 0) {
            reinterpret_cast<uint2 *>(pa.q16 + h * kD)[lane] = q4;
            if (pa.q_f32 != nullptr) {
                reinterpret_cast<float4 *>(pa.q_f32 + h * kD)[lane] = make_float4(y[0], y[1], y[2], y[3]);
            }
        }
    }
    // the workgroup's q rows complete in LDS; the barrier waits for the LDS writes only (a __syncthreads would also
    // drain the tile's copies into LDS)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    const int32_t h = lane % 16, g = lane / 16;
#pragma unroll
    for (int32_t j = 0; j < 8; ++j) {
        u32x4 v = {0u, 0u, 0u, 0u};
        if (h < kHeads) {
            v = *reinterpret_cast<const u32x4 *>(ql + h * kD + 32 * j + 8 * g);
        }
        qb[j] = __builtin_bit_cast(half8, v);
    }
}

// FUSED (the draft step, fnkv_datc_step): the prepare of the one row folded in. Every workgroup forms the row's q
// itself (wave w heads 3 w .. 3 w + 2, under its first tile's loads) into LDS; workgroup 0 also writes q16 (and q_f32);
// the wave whose walk holds the row's cell writes its K and V (and k_f32) before issuing any load. The attention and
// its partials are then those of the prepare and attend launches in turn, bit for bit.
template <bool SP, bool FUSED>
__global__ __launch_bounds__(64 * kWaves, 1) void datc_attend_kernel(fnkv_datc_attend_args a,
                                                                     fnkv_datc_prepare_args pa) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int32_t wave = static_cast<int32_t>(threadIdx.x) / 64, lane = static_cast<int32_t>(threadIdx.x) % 64;
    const datc_shape s = datc_shape_of<SP>(a);
    if (!s.valid || (FUSED && prepare_refused(pa, 1))) {
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            atomicOr(a.err, FNKV_DEV_ERR_DRAFT_DEPTH);
        }
        return;
    }
    const int32_t b = static_cast<int32_t>(blockIdx.x);
    if (b >= s.active) {
        return;
    }
#ifdef FNKV_TIMING
    uint64_t * ts = g_datc_ts;
#endif
    DATC_STAMP(b, 0);
    // the grid strides over the tiles: wave w of workgroup b takes tiles w + 4 (b + A i), so at any moment the
    // workgroups read one window of the caches together
    const int32_t first = wave + kWaves * b, per = kWaves * s.active;
    const int32_t cnt = s.n_tiles > first ? (s.n_tiles - first + per - 1) / per : 0;
    const uint32_t cache_bytes = static_cast<uint32_t>(a.max_cells) * 512u;
    const rsrc_t rk = make_rsrc(a.k_cache, static_cast<int32_t>(cache_bytes));
    const rsrc_t rv = make_rsrc(a.v_cache, static_cast<int32_t>(cache_bytes));
    uint8_t * vb0 = smem + wave * 2 * kVBuf;
    uint8_t * vb1 = vb0 + kVBuf;
    auto tile_base = [&](int32_t k) { return k < cnt ? (first + per * k) * kTile : kEmptyTile; };
    if constexpr (FUSED) {
        // the row's cell: written by the wave whose walk holds its tile (its last), before any of that wave's loads
        const int32_t cell_l = s.n - 1; // the row's own cell is the last logical cell (dense and SP2)
        if (cnt > 0 && (cell_l / kTile - first) % per == 0 && cell_l / kTile >= first) {
            const int32_t nb = *pa.n_before;
            float y[4];
            norm_rope(y, pa.kv_k, pa.k_norm, pa.pos, *pa.stride, pa.row0, pa.theta_scale, lane);
            if (pa.k_f32 != nullptr) {
                reinterpret_cast<float4 *>(pa.k_f32)[lane] = make_float4(y[0], y[1], y[2], y[3]);
            }
            const int64_t at = (static_cast<int64_t>(nb) + pa.row0) * kD;
            reinterpret_cast<uint2 *>(pa.k_cache + at)[lane] = pack4_f16(y, 1.0f);
            const float4 v4 = reinterpret_cast<const float4 *>(pa.kv_v)[lane];
            const float v[4] = {v4.x, v4.y, v4.z, v4.w};
            reinterpret_cast<uint2 *>(pa.v_cache + at)[lane] = pack4_f16(v, 1.0f);
            // the stores complete (into L2: the vector L1 writes through, and no wave of this CU has read the tile in
            // this launch) before this wave, the only one that reads the tile, issues its loads
            __threadfence_block();
        }
    }
    // q16 as the B operand: lane l holds head l % 16's dims 32 j + 8 (l / 16) .. + 7 (heads 12..15 zero); loaded
    // before the first tile (FUSED: formed after the first tile's loads are issued)
    half8 qb[8];
    k_tile ka, kb;
    // one tile in flight while the other is computed; in the loop every step issues its 32 loads (the wave's last
    // pair may take an empty tile: cells beyond the row, zeros, no memory traffic) and the loop runs whole pairs, so a
    // step waits for exactly the loads issued before the last 32; an odd last tile is a step of its own that issues
    // nothing
    float m_run = -INFINITY, l_run = 0.0f;
    floatx4 o[16];
#pragma unroll
    for (int32_t db = 0; db < 16; ++db) {
        o[db] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    if constexpr (FUSED) {
        // a wave with two tiles or more also issues its second before forming q, then tile 0's step issues nothing
        // and the walk goes on from tile 1 with the buffers' roles swapped; a wave with one tile (or none: the empty
        // tile) issues only that (an empty second tile's copies measured slower at shallow depths). Each path runs
        // to its end on its own, so the compiler's wait counts never merge two paths' outstanding loads.
        if (cnt > 1) {
            fused_first_tile<SP, true>(a, pa, s, rk, rv, tile_base(0), tile_base(1), ka, kb, vb0, vb1,
                                       reinterpret_cast<uint16_t *>(smem + kQLds), qb, b, wave, lane);
            tile_step<SP, kNextIssued>(a, s, rk, rv, ka, kb, vb0, vb1, tile_base(0), 0, qb, m_run, l_run, o, lane);
            int32_t k = 1;
            for (; k + 1 < cnt; k += 2) {
                tile_step<SP, kIssueNext>(a, s, rk, rv, kb, ka, vb1, vb0, tile_base(k), tile_base(k + 1), qb, m_run,
                                          l_run, o, lane);
                tile_step<SP, kIssueNext>(a, s, rk, rv, ka, kb, vb0, vb1, tile_base(k + 1), tile_base(k + 2), qb,
                                          m_run, l_run, o, lane);
            }
            if (k < cnt) {
                tile_step<SP, kLast>(a, s, rk, rv, kb, ka, vb1, vb0, tile_base(k), 0, qb, m_run, l_run, o, lane);
            }
        } else {
            fused_first_tile<SP, false>(a, pa, s, rk, rv, tile_base(0), 0, ka, kb, vb0, vb1,
                                        reinterpret_cast<uint16_t *>(smem + kQLds), qb, b, wave, lane);
            if (cnt == 1) {
                tile_step<SP, kLast>(a, s, rk, rv, ka, kb, vb0, vb1, tile_base(0), 0, qb, m_run, l_run, o, lane);
            }
        }
    } else {
        const int32_t h = lane % 16, g = lane / 16;
#pragma unroll
        for (int32_t j = 0; j < 8; ++j) {
            u32x4 v = {0u, 0u, 0u, 0u};
            if (h < kHeads) {
                v = *reinterpret_cast<const u32x4 *>(a.q16 + h * kD + 32 * j + 8 * g);
            }
            qb[j] = __builtin_bit_cast(half8, v);
        }
    }
    if (!FUSED && cnt > 0) {
        issue_tile<SP>(a, s, rk, rv, tile_base(0), ka, vb0, lane);
        int32_t k = 0;
        for (; k + 1 < cnt; k += 2) {
            tile_step<SP, kIssueNext>(a, s, rk, rv, ka, kb, vb0, vb1, tile_base(k), tile_base(k + 1), qb, m_run, l_run, o,
                                lane);
            tile_step<SP, kIssueNext>(a, s, rk, rv, kb, ka, vb1, vb0, tile_base(k + 1), tile_base(k + 2), qb, m_run, l_run,
                                o, lane);
        }
        if (k < cnt) {
            tile_step<SP, kLast>(a, s, rk, rv, ka, kb, vb0, vb1, tile_base(k), 0, qb, m_run, l_run, o, lane);
        }
    }
    wait_vmcnt<0>(); // the last (empty) copies land before the fold below reuses the buffers
    DATC_STAMP(b, 2);
    // fold the waves: M, the waves' weights, then O summed in wave order
    float * ml = reinterpret_cast<float *>(smem + kMlLds); // a wave still in its last step owns its V buffer
    if (lane < 16) {
        ml[wave * 16 + lane] = m_run;
        ml[kWaves * 16 + wave * 16 + lane] = l_run;
    }
    __syncthreads(); // also: every wave is done with its V buffers
    const int32_t h = lane % 16, g = lane / 16;
    float M = -INFINITY;
#pragma unroll
    for (int32_t w = 0; w < kWaves; ++w) {
        M = fmaxf(M, ml[w * 16 + h]);
    }
    const float scale = expf(m_run - M); // 0 for a wave without tiles
    float * ow = reinterpret_cast<float *>(smem) + wave * kHeads * kOStride;
    if (h < kHeads) {
#pragma unroll
        for (int32_t db = 0; db < 16; ++db) {
            *reinterpret_cast<floatx4 *>(ow + h * kOStride + 16 * db + 4 * g) = o[db] * scale;
        }
    }
    __syncthreads();
    float * part = reinterpret_cast<float *>(a.part) + static_cast<int64_t>(b) * kPartFloats;
    const int32_t d = static_cast<int32_t>(threadIdx.x);
    const float * of = reinterpret_cast<const float *>(smem);
#pragma unroll
    for (int32_t hh = 0; hh < kHeads; ++hh) {
        float acc = of[hh * kOStride + d];
#pragma unroll
        for (int32_t w = 1; w < kWaves; ++w) {
            acc += of[w * kHeads * kOStride + hh * kOStride + d];
        }
        part[hh * kD + d] = acc;
    }
    if (threadIdx.x < kHeads) {
        float Mh = -INFINITY;
#pragma unroll
        for (int32_t w = 0; w < kWaves; ++w) {
            Mh = fmaxf(Mh, ml[w * 16 + d]);
        }
        float L = 0.0f;
#pragma unroll
        for (int32_t w = 0; w < kWaves; ++w) {
            L = __builtin_fmaf(ml[kWaves * 16 + w * 16 + d], expf(ml[w * 16 + d] - Mh), L);
        }
        part[kHeads * kD + d] = Mh;
        part[kHeads * kD + kHeads + d] = L;
    }
    DATC_STAMP(b, 3);
}

// the fold of (head h, values 32 r .. 32 r + 31): the active partials in workgroup order, the gate, the F32 output and
// its activation-format run (act_run). Thread t takes partials t / 32 + 8 i of value t % 32 and issues all its loads
// before the reductions that weigh them.
template <bool SP, bool FUSED>
__global__ __launch_bounds__(256) void datc_fold_kernel(fnkv_datc_attend_args a, fnkv_datc_prepare_args pa) {
    constexpr int32_t kPer = kGrid / 8;
    __shared__ float w_of[kGrid];
    __shared__ float wred[2][4];
    __shared__ float accs[8][32];
    const int32_t h = static_cast<int32_t>(blockIdx.x) / 8, r = static_cast<int32_t>(blockIdx.x) % 8;
    const int32_t t = static_cast<int32_t>(threadIdx.x), wave = t / 64;
#ifdef FNKV_TIMING
    uint64_t * ts = g_datc_ts;
#endif
    DATC_STAMP(256 + blockIdx.x, 0);
    const int32_t grp = t / 32, dl = t % 32;
    const int32_t dd = h * kD + 32 * r + dl;
    const float * part = reinterpret_cast<const float *>(a.part);
    // every partial's values are loaded before the depth word is known; those past the active workgroups (stale,
    // possibly not finite) are dropped by selection, never weighted
    float ov[kPer];
#pragma unroll
    for (int32_t i = 0; i < kPer; ++i) {
        ov[i] = part[static_cast<int64_t>(grp + 8 * i) * kPartFloats + dd];
    }
    const float m_raw = part[static_cast<int64_t>(t) * kPartFloats + kHeads * kD + h];
    const float l_raw = part[static_cast<int64_t>(t) * kPartFloats + kHeads * kD + kHeads + h];
    const float gate = t < 32 ? a.qfull[h * kQS + kD + 32 * r + dl] : 0.0f;
    const datc_shape s = datc_shape_of<SP>(a);
    if (!s.valid || (FUSED && prepare_refused(pa, 1))) {
        return;
    }
    const float m_t = t < s.active ? m_raw : -INFINITY;
    const float l_t = t < s.active ? l_raw : 0.0f;
    float mx = m_t;
#pragma unroll
    for (int32_t o = 32; o > 0; o >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    }
    if ((t & 63) == 0) {
        wred[0][wave] = mx;
    }
    __syncthreads();
    const float M = fmaxf(fmaxf(wred[0][0], wred[0][1]), fmaxf(wred[0][2], wred[0][3]));
    const float wt = t < s.active ? expf(m_t - M) : 0.0f;
    w_of[t] = wt;
    float lw = l_t * wt;
#pragma unroll
    for (int32_t o = 32; o > 0; o >>= 1) {
        lw += __shfl_xor(lw, o, 64);
    }
    if ((t & 63) == 0) {
        wred[1][wave] = lw;
    }
    __syncthreads();
    const float L = (wred[1][0] + wred[1][1]) + (wred[1][2] + wred[1][3]);
    float acc = 0.0f;
#pragma unroll
    for (int32_t i = 0; i < kPer; ++i) {
        acc = grp + 8 * i < s.active ? __builtin_fmaf(ov[i], w_of[grp + 8 * i], acc) : acc;
    }
    accs[grp][dl] = acc;
    __syncthreads();
    if (t >= 32) {
        return;
    }
    const float A = ((accs[0][dl] + accs[1][dl]) + (accs[2][dl] + accs[3][dl])) +
                    ((accs[4][dl] + accs[5][dl]) + (accs[6][dl] + accs[7][dl]));
    const float y = A / L * (1.0f / (1.0f + expf(-gate)));
    a.out[dd] = y;
    const float yv[1] = {y};
    int8_t qv[1];
    float ds[2];
    act_run<1, 32>(yv, qv, ds);
    a.codes[dd] = qv[0];
    if (dl == 0) {
        a.scales[2 * (h * 8 + r)] = ds[0];
        a.scales[2 * (h * 8 + r) + 1] = ds[1];
    }
    DATC_STAMP(256 + blockIdx.x, 1);
}

bool aligned(const void * p, uintptr_t n) {
    return p != nullptr && reinterpret_cast<uintptr_t>(p) % n == 0;
}

} // namespace
} // namespace fnkv

using fnkv::set_error;

extern "C" {

float fnkv_rope_theta_scale(void) {
    return powf(10000000.0f, -2.0f / static_cast<float>(fnkv::kNRot));
}

int64_t fnkv_datc_part_bytes(void) {
    return static_cast<int64_t>(sizeof(float)) * fnkv::kGrid * fnkv::kPartFloats;
}

int fnkv_datc_prepare(int32_t rows, const fnkv_datc_prepare_args * a, void * stream) {
    using fnkv::aligned;
    if (a == nullptr || rows < 1 || rows > FNKV_DATC_MAX_ROWS || a->row0 < 0 || a->row0 + rows > FNKV_DATC_MAX_ROWS ||
        a->max_cells < 1 || !aligned(a->kv_k, 16) || !aligned(a->kv_v, 16) || !aligned(a->k_norm, 16) ||
        a->n_before == nullptr || a->pos == nullptr || a->stride == nullptr || !aligned(a->k_cache, 16) ||
        !aligned(a->v_cache, 16) || a->err == nullptr || (a->k_f32 != nullptr && !aligned(a->k_f32, 16)) ||
        !std::isfinite(a->theta_scale) ||
        (a->qfull != nullptr && (!aligned(a->qfull, 16) || !aligned(a->q_norm, 16) || !aligned(a->q16, 16) ||
                                 (a->q_f32 != nullptr && !aligned(a->q_f32, 16))))) {
        set_error("fnkv_datc_prepare: argument outside the contract");
        return FNKV_ERR_ARG;
    }
#ifdef FNKV_TIMING
    {
        uint64_t * tb = fnkv::timing_buffer();
        (void)hipMemcpyToSymbolAsync(HIP_SYMBOL(fnkv::g_datc_ts), &tb, sizeof(tb), 0, hipMemcpyHostToDevice,
                                     static_cast<hipStream_t>(stream));
    }
#endif
    hipLaunchKernelGGL(fnkv::datc_prepare_kernel, dim3(static_cast<uint32_t>(rows)), dim3(64 * (fnkv::kHeads + 1)), 0,
                       static_cast<hipStream_t>(stream), *a, rows);
    if (hipGetLastError() != hipSuccess) {
        set_error("fnkv_datc_prepare: launch failed");
        return FNKV_ERR_HIP;
    }
    return FNKV_OK;
}

} // extern "C"

namespace fnkv {
namespace {

bool attend_args_ok(const fnkv_datc_attend_args * a) {
    // the caches are addressed by 32-bit buffer offsets: at most 4,194,303 cells (2 GiB a cache)
    return a != nullptr && a->row0 >= 0 &&
           a->row0 < (a->body != nullptr ? FNKV_DATC_MAX_SPARSE_ROW : FNKV_DATC_MAX_ROWS) && a->max_cells >= 1 &&
           a->max_cells < (1 << 22) && aligned(a->qfull, 16) && aligned(a->k_cache, 16) && aligned(a->v_cache, 16) &&
           a->n_before != nullptr && aligned(a->part, 16) && aligned(a->out, 16) && a->codes != nullptr &&
           aligned(a->scales, 8) && a->err != nullptr && (a->body == nullptr || aligned(a->body, 4));
}

template <bool FUSED>
int launch_attend(const fnkv_datc_attend_args & a, const fnkv_datc_prepare_args & pa, hipStream_t st) {
    static std::once_flag attr_once[64]; // once per device; a racing first caller waits for it
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev >= 0 && dev < 64) {
        std::call_once(attr_once[dev], []() {
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(datc_attend_kernel<false, FUSED>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kAttendLds);
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(datc_attend_kernel<true, FUSED>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kAttendLds);
            (void)hipGetLastError();
        });
    }
    if (a.body != nullptr) {
        hipLaunchKernelGGL((datc_attend_kernel<true, FUSED>), dim3(kGrid), dim3(64 * kWaves), kAttendLds, st, a, pa);
        hipLaunchKernelGGL((datc_fold_kernel<true, FUSED>), dim3(kHeads * 8), dim3(256), 0, st, a, pa);
    } else {
        hipLaunchKernelGGL((datc_attend_kernel<false, FUSED>), dim3(kGrid), dim3(64 * kWaves), kAttendLds, st, a, pa);
        hipLaunchKernelGGL((datc_fold_kernel<false, FUSED>), dim3(kHeads * 8), dim3(256), 0, st, a, pa);
    }
    return hipGetLastError() == hipSuccess ? FNKV_OK : FNKV_ERR_HIP;
}

} // namespace
} // namespace fnkv

extern "C" {

int fnkv_datc_attend(const fnkv_datc_attend_args * a, void * stream) {
    if (!fnkv::attend_args_ok(a) || !fnkv::aligned(a->q16, 16)) {
        set_error("fnkv_datc_attend: argument outside the contract");
        return FNKV_ERR_ARG;
    }
    const fnkv_datc_prepare_args none = {};
    if (fnkv::launch_attend<false>(*a, none, static_cast<hipStream_t>(stream)) != FNKV_OK) {
        set_error("fnkv_datc_attend: launch failed");
        return FNKV_ERR_HIP;
    }
    return FNKV_OK;
}

int fnkv_datc_step(const fnkv_datc_prepare_args * p, const fnkv_datc_attend_args * a, void * stream) {
    using fnkv::aligned;
    if (p == nullptr || !fnkv::attend_args_ok(a) || p->qfull == nullptr || p->row0 != a->row0 ||
        p->k_cache != a->k_cache || p->v_cache != a->v_cache || p->n_before != a->n_before ||
        p->max_cells != a->max_cells || !aligned(p->qfull, 16) || !aligned(p->kv_k, 16) || !aligned(p->kv_v, 16) ||
        !aligned(p->q_norm, 16) || !aligned(p->k_norm, 16) || p->pos == nullptr || p->stride == nullptr ||
        !aligned(p->q16, 16) || (p->q_f32 != nullptr && !aligned(p->q_f32, 16)) ||
        (p->k_f32 != nullptr && !aligned(p->k_f32, 16)) || !std::isfinite(p->theta_scale)) {
        set_error("fnkv_datc_step: argument outside the contract");
        return FNKV_ERR_ARG;
    }
    if (fnkv::launch_attend<true>(*a, *p, static_cast<hipStream_t>(stream)) != FNKV_OK) {
        set_error("fnkv_datc_step: launch failed");
        return FNKV_ERR_HIP;
    }
    return FNKV_OK;
}

} // extern "C"
