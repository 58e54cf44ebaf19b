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

namespace fnkv {

constexpr float kNegInf = -__builtin_inff();
constexpr int32_t kCodeBytes = 16384;  // a tile's K and V codes
constexpr int32_t kScaleBytes = 1024;  // a tile's K and V scales
constexpr int32_t kGroupLds = kCodeBytes + 2 * kScaleBytes;

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
    int32_t slot[FNKV_MAX_SEQS];
    int64_t ctx[FNKV_MAX_SEQS];
    int32_t split0[FNKV_MAX_SEQS + 1]; // first split of each sequence; split0[n_seq] = total
    // a sparse launch (one sequence): the ascending union of the logical tiles the rows' selections touch, each
    // row's 4-cell blocks in it (row t's 8 bits at bit 8 t of .x for t < 4, of .y for t = 4), their count (device),
    // and the entries a split takes (split s: entries s * sel_split ..)
    const int32_t * sel_tiles;
    const uint2 * sel_masks;
    const int32_t * sel_n;
    int32_t sel_split;
#ifdef FNKV_TIMING
    uint64_t * ts; // per workgroup: 16 real-time stamps (instrumented builds only)
#endif
};

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
        if (a.ts != nullptr && (threadIdx.x & 63) == 0) {                                                            \
            a.ts[(blockIdx.y * gridDim.x + blockIdx.x) * 16 + 8 + (threadIdx.x >> 6)] =                              \
                __builtin_amdgcn_s_memrealtime();                                                                    \
        }                                                                                                            \
        __builtin_amdgcn_s_waitcnt(0);                                                                               \
    } while (0)
// phase clocks of wave 0 (20-bit shader cycle counter, no memory counters touched), summed over the loop
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
#define FNKV_STAMP_WAVE()                                                                                            \
    do {                                                                                                             \
    } while (0)
#define FNKV_STAMP(k)                                                                                                \
    do {                                                                                                             \
    } while (0)
#endif

// The tiles a workgroup walks. Dense: its split's consecutive cells begin .. end, lane i holding the physical page
// of the split's logical page i. Sparse: entries e0 .. e0 + n_tiles - 1 of the selection's tile list, lane i holding
// entry i's logical tile, physical page and row masks. Tile ti of the walk is then a lane read either way.
template <bool SP> struct split_src {
    int32_t n_tiles = 0;
    int32_t page_lane = 0;
    int32_t tile_lane = 0;
    uint32_t mlo_lane = 0, mhi_lane = 0;
    int64_t begin = 0;

    __device__ __forceinline__ void init(const dec_args & a, const int32_t * table, int32_t split, int64_t b,
                                         int64_t e, int32_t lane) {
        if constexpr (SP) {
            const int32_t e0 = split * a.sel_split;
            const int32_t left = *a.sel_n - e0;
            n_tiles = left < 0 ? 0 : left < a.sel_split ? left : a.sel_split;
            if (lane < n_tiles) {
                tile_lane = a.sel_tiles[e0 + lane];
                const uint2 m = a.sel_masks[e0 + lane];
                mlo_lane = m.x;
                mhi_lane = m.y;
                page_lane = table[tile_lane >> 3];
            }
        } else {
            begin = b;
            n_tiles = static_cast<int32_t>((e - b + kTileTokens - 1) / kTileTokens);
            const int32_t n_pages = static_cast<int32_t>((e - b + kPageTokens - 1) / kPageTokens);
            page_lane = lane < n_pages ? table[(b >> 8) + lane] : 0;
        }
    }
    // byte offset of walk tile ti within the (layer, head) plane of the pool
    __device__ __forceinline__ int64_t tile_off(const pool_view & pv, int32_t ti) const {
        if constexpr (SP) {
            const int32_t phys = __builtin_amdgcn_readlane(page_lane, ti);
            const int32_t t8 = __builtin_amdgcn_readlane(tile_lane, ti) & 7;
            return int64_t(phys) * pv.page_stride + int64_t(t8) * kTileBytes;
        } else {
            const int32_t phys = __builtin_amdgcn_readlane(page_lane, ti >> 3);
            return int64_t(phys) * pv.page_stride + int64_t(ti & 7) * kTileBytes;
        }
    }
    // the first cell of walk tile ti
    __device__ __forceinline__ int64_t tok0(int32_t ti) const {
        if constexpr (SP) {
            return int64_t(__builtin_amdgcn_readlane(tile_lane, ti)) * kTileTokens;
        } else {
            return begin + int64_t(ti) * kTileTokens;
        }
    }
    // the visibility bits of tile_softmax for this lane (query row of step token t_row, lane group qg)
    __device__ __forceinline__ uint32_t vis(int32_t ti, int32_t t_row, int32_t qg) const {
        if constexpr (SP) {
            const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int32_t>(mlo_lane), ti));
            const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int32_t>(mhi_lane), ti));
            const uint32_t byte = t_row < 4 ? (lo >> (8 * t_row)) : hi;
            return ((byte >> qg) & 1u) | (((byte >> (4 + qg)) & 1u) << 1);
        } else {
            return 3u;
        }
    }
};

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
    const int32_t * sel_n;
    int32_t sel_split;
};

class kv_pool;
// host: the merge launch, and the sparse instantiation of the decode kernels (decode.hip)
void launch_merge(const merge_args & m, hipStream_t st);
void launch_decode_sparse(const kv_pool & p, int32_t NT, dim3 grid, const dec_args & a, hipStream_t st);

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
template <int WAVES>
__device__ __forceinline__ void append_new_cells(const dec_args & a, const int32_t * table, int32_t s, int32_t kvh,
                                                 int64_t ctx, int64_t begin, int64_t end, int32_t wave,
                                                 int32_t lane) {
    if (a.k_new == nullptr) {
        return;
    }
    const pool_view & pv = a.pv;
    const int64_t first_new = ctx - a.T;
    const int64_t p0 = begin > first_new ? begin : first_new;
    const int32_t nrow = static_cast<int32_t>(end - p0);
    if (nrow <= 0) {
        return;
    }
    for (int32_t job = wave; job < 2 * nrow; job += WAVES) {
        const int64_t pos = p0 + (job >> 1);
        const int32_t kv = job & 1;
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
__device__ __forceinline__ void load_q_operands(const dec_args & a, int32_t s, int32_t kvh, int32_t rt, int32_t j,
                                                int32_t qg, half8 (&qop)[kBlocks], int64_t & lim) {
    const int32_t row = rt * 16 + j;
    const bool real_row = row < a.R;
    const int32_t t_row = real_row ? row / a.G : a.T - 1;
    lim = a.ctx[s] - a.T + t_row;
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
template <typename QOP>
__device__ __forceinline__ floatx4 tile_scores_half(const uint8_t * kb, const uint8_t * sc_tile, const QOP & qop,
                                                    half8 sig, int32_t j, int32_t qg, int32_t lane, int32_t h) {
    const half8 zero8 = {};
    // this lane's score rows are tokens 16 h + 4 qg + r; their K scales, all 8 blocks
    half8 ks[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        ks[r] = *reinterpret_cast<const half8 *>(sc_tile + kKScales + (16 * h + 4 * qg + r) * 16);
    }
    // the bias term: A = this lane's token row of K scales (twice), B = sigma hi / lo
    const half8 srow = qg < 2 ? *reinterpret_cast<const half8 *>(sc_tile + kKScales + (16 * h + j) * 16) : zero8;
    const floatx4 corr = mfma16(srow, sig, floatx4{0.0f, 0.0f, 0.0f, 0.0f});
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
                const half8 ka = widen8_biased(kw[2 * bb], kw[2 * bb + 1]);
                t[b - 4 * hb] = mfma16(ka, qop(b), floatx4{0.0f, 0.0f, 0.0f, 0.0f});
            }
        }
#pragma unroll
        for (int b = 4 * hb; b < 4 * hb + 4; ++b) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                acc_s[r] = __builtin_fmaf(static_cast<float>(ks[r][b]), t[b - 4 * hb][r], acc_s[r]);
            }
        }
    }
    floatx4 sc;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        sc[r] = __builtin_fmaf(-1152.0f, corr[r], acc_s[r]);
    }
    return sc;
}

// both halves: sc[h][r] is the score of token 16 h + 4 qg + r against this lane's row j
template <typename QOP>
__device__ __forceinline__ void tile_scores(const uint8_t * kb, const uint8_t * sc_tile, const QOP & qop, half8 sig,
                                            int32_t j, int32_t qg, int32_t lane, floatx4 (&sc)[2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        sc[h] = tile_scores_half(kb, sc_tile, qop, sig, j, qg, lane, h);
        __builtin_amdgcn_sched_barrier(0); // one half's operands live at a time
    }
}

// Online softmax (base 2) of a tile's scores for this lane's row, tokens past lim_rel (tile-relative) masked. The
// row's reference m_run moves only when the tile's max exceeds it by more than kLazyLog2 (then alpha = 2^(m_old - m),
// the factor the row's accumulators take before this tile's terms; else alpha = 1), so the rescale of the
// accumulators is rare; the weights pf[4 h + r] = 2^(c2 sc - m_run) stay <= 2^kLazyLog2 = 64, which keeps a weight
// times a V scale (at most 65504 / 127) inside fp16. alpha is the same in the row's four lanes.
constexpr float kLazyLog2 = 6.0f;
// vis: bit h set when this lane's 4 cells of half h (one 4-cell block) are in its row's selection (dense: 3).
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
    const bool move = mx > m_run + kLazyLog2; // m_run = -inf: any visible score moves it
    const float m_new = move ? mx : m_run;
    const float m_use = m_new == kNegInf ? 0.0f : m_new;
    alpha = move ? __builtin_amdgcn_exp2f(m_run - m_use) : 1.0f;
    float lsum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        pf[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(raw[i], c2, -m_use));
        lsum += pf[i];
    }
    l_run = __builtin_fmaf(l_run, alpha, lsum);
    m_run = m_new;
}

} // namespace fnkv
