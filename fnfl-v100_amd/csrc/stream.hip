// Dense decode / speculative-verify attention over the page pool, one tile stream a wave (the launches with host or
// device contexts: fnkv_attn_decode, fnkv_attn_decode_dev, fnkv_attn_decode_noalloc; fnkv_attend's dense calls).
//
// What it computes is decode.hip's: for query row (t, head h) of a sequence holding ctx cells,
//   o = sum_c softmax_c(q . k_c * scale) v_c over cells c <= ctx - T + t,
// with the decoded Q8_0 (or KV8) cells, fp32 scores, softmax statistics and accumulators, and the split-K partials
// (m, l, acc) folded by the merge as the reference's finish does (fn/kernels/qsa/attend.cu:621-655).
//
// How (MI355X): a workgroup of 8 waves (two a SIMD) owns one (sequence, KV head, split of the cells); wave w walks
// the split's tiles w, w + 8, ... on its own, and computes every query row of the KV head (NT row tiles of 16:
// G T <= 16 NT) itself, so the loop has no workgroup barrier and no exchange of P, and a SIMD's two waves co-issue
// one's VALU work with the other's MFMAs:
//   * a tile goes straight from HBM into the wave's LDS slot (its layout is the tile's): the K half (K codes and K
//     scales) as soon as the scores have read the previous tile's, the V half (V codes and V scales) as soon as PV
//     has, so each half's latency hides under the other half's work (the first tile's V half only once its K half is
//     in: the launch's first requests are the waves' K halves alone);
//   * the K codes are widened once a tile (one byte permute makes two codes the fp16 values 1152 + code) and feed the
//     S^T = K Q^T MFMA of every row tile (the Q operands sit once in LDS for the workgroup); each block's K scale is
//     one FMA a score; one MFMA a half takes the 1152 bias back out against the rows' q sums;
//   * online softmax in base 2 on the S^T registers, which are already the B operand of O^T = V^T P^T; P times the
//     block's V scale enters the matrix core as fp16 hi + lo (~2^-20 relative); the accumulators O^T (NT x 64
//     registers) stay in VGPRs (NT <= 2 within a wave's 256);
//   * one MFMA pair a tile against the V scales (and a row of ones) gives each row's V bias sums and its l;
//   * a KV8 pool (group-64 scales, stored at both blocks of a group) takes the KV8 instantiation: a group's two score
//     MFMAs chain before its one scale FMA, and its P x V-scale products serve both of its blocks;
//   * after the loop each wave writes its unscaled (m, l, acc) into its own tile slot, and the workgroup folds the
//     eight waves' rows from there (each scaled by 2^(m - M) as it is read) and writes the split's partial.
#include "../../include/fnkv.h"
#include "common.h"
#include "decode_common.h"
#include "layout.h"
#include "mfma.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <mutex>

namespace fnkv {

template <int NT> struct stream_shape {
    static_assert(NT >= 1 && NT <= 3, "G T <= 48 rows");
    static constexpr int WAVES = 8;
    // NT = 3: the rows split over two waves of a SIMD that walk the same tiles (waves 0-3 row tiles 0 and 1, waves
    // 4-7 row tile 2: a wave's accumulators for at most two row tiles fit its registers); each loads the tile itself,
    // the second load served by L2 (cacheable loads). NT <= 2: each wave its own tile stream, every row tile,
    // streaming loads.
    static constexpr int GROUPS = NT == 3 ? 2 : 1;
    static constexpr int STREAMS = WAVES / GROUPS;
    static constexpr int AUX = NT == 3 ? 0 : kStreamAux;
    static constexpr int SLOT = kTileBytes;          // a tile, in its HBM layout
    static constexpr int RING = WAVES * SLOT;        // 139,264 B
    static constexpr int QOPS = NT * kBlocks * 1024; // the Q operands: [row tile][block][lane] 16 B
    static constexpr int OSTRIDE = kHeadDim + 4;     // floats a row of the fold buffer
    static constexpr int LDS = RING + QOPS; // the 8-wave fold reuses the tile slots
    static_assert(LDS <= 160 * 1024, "LDS");
    // a half tile is 9 loads: 8 chunks of codes and half of the scales chunk; the wave waits for one half with the
    // other half's 9 issued after it
    static constexpr int HALF_LOADS = 9;
};

// S^T = K Q^T of one tile for NT row tiles from the K codes (kb) and the scales chunk (sc) in LDS: sc_out[rt][h][r]
// is the score (q . k, unscaled) of token 16 h + 4 qg + r against row 16 rt + j. Each 1 KiB chunk of K codes is
// widened once and feeds the MFMAs of every row tile. KV8: a chunk's two blocks are one 64-value group with one
// scale, so their two MFMAs chain and the group takes one FMA a score.
template <int NT, bool KV8>
__device__ __forceinline__ void stream_scores(const uint8_t * kb, const uint8_t * sc, const uint8_t * qs,
                                              const half8 (&sig)[NT], int32_t j, int32_t qg, int32_t lane,
                                              floatx4 (&s_out)[NT][2]) {
    const half8 zero8 = {};
    // a chunk's operands: its 16 K codes a lane and the row tiles' Q operands of its two blocks; each chunk's are read
    // from LDS one chunk ahead, while the previous chunk's MFMAs run
    auto kw_at = [&](int c) { return *reinterpret_cast<const u32x4 *>(kb + (c >> 2) * 4096 + (c & 3) * 1024 + lane * 16); };
    auto qo_at = [&](int rt, int b) { return *reinterpret_cast<const half8 *>(qs + (rt * kBlocks + b) * 1024 + lane * 16); };
    u32x4 kw_next = kw_at(0);
    half8 qo_next[NT][2];
#pragma unroll
    for (int rt = 0; rt < NT; ++rt) {
        qo_next[rt][0] = qo_at(rt, 0);
        qo_next[rt][1] = qo_at(rt, 1);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        half8 ks[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            ks[r] = *reinterpret_cast<const half8 *>(sc + (16 * h + 4 * qg + r) * 16);
        }
        // the bias term: A = the token row's K scales (lanes qg < 2), B = the row's per-block q sums (hi, lo)
        const half8 srow = qg < 2 ? *reinterpret_cast<const half8 *>(sc + (16 * h + j) * 16) : zero8;
        // the scores start from the bias term (-1152 times it) and take each block's term with one FMA a score
        floatx4 acc_s[NT];
#pragma unroll
        for (int rt = 0; rt < NT; ++rt) {
            acc_s[rt] = mfma16(srow, sig[rt], floatx4{0.0f, 0.0f, 0.0f, 0.0f}) * -1152.0f;
        }
#pragma unroll
        for (int ld = 0; ld < 4; ++ld) { // one 1 KiB chunk: blocks 2 ld, 2 ld + 1
            const int c = 4 * h + ld;
            const u32x4 kw = kw_next;
            half8 qo[NT][2];
#pragma unroll
            for (int rt = 0; rt < NT; ++rt) {
                qo[rt][0] = qo_next[rt][0];
                qo[rt][1] = qo_next[rt][1];
            }
            if (c + 1 < 8) {
                kw_next = kw_at(c + 1);
#pragma unroll
                for (int rt = 0; rt < NT; ++rt) {
                    qo_next[rt][0] = qo_at(rt, 2 * ((c + 1) & 3));
                    qo_next[rt][1] = qo_at(rt, 2 * ((c + 1) & 3) + 1);
                }
            }
            floatx4 t[NT][2];
#pragma unroll
            for (int bb = 0; bb < 2; ++bb) {
                const half8 ka = widen8<false>(kw[2 * bb], kw[2 * bb + 1]);
#pragma unroll
                for (int rt = 0; rt < NT; ++rt) {
                    if constexpr (KV8) { // the group's second block adds to its first
                        t[rt][0] = mfma16(ka, qo[rt][bb], bb == 0 ? floatx4{0.0f, 0.0f, 0.0f, 0.0f} : t[rt][0]);
                    } else {
                        t[rt][bb] = mfma16(ka, qo[rt][bb], floatx4{0.0f, 0.0f, 0.0f, 0.0f});
                    }
                }
            }
#pragma unroll
            for (int bb = 0; bb < (KV8 ? 1 : 2); ++bb) {
#pragma unroll
                for (int rt = 0; rt < NT; ++rt) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        acc_s[rt][r] =
                            __builtin_fmaf(static_cast<float>(ks[r][2 * ld + bb]), t[rt][bb][r], acc_s[rt][r]);
                    }
                }
            }
            // pin the chunk's FMAs here (the optimizer would otherwise sink them past the later chunks' MFMAs and
            // keep every chunk's results live at once)
#pragma unroll
            for (int rt = 0; rt < NT; ++rt) {
                __asm__ volatile("" : "+v"(acc_s[rt]));
            }
            __builtin_amdgcn_sched_barrier(0); // one chunk's operands live at a time
        }
#pragma unroll
        for (int rt = 0; rt < NT; ++rt) {
            s_out[rt][h] = acc_s[rt];
        }
    }
}

// Online softmax (base 2) of one row tile's tile scores, tokens past lim_rel masked: the row's reference max moves
// only when the tile's max exceeds it by more than kLazyLog2 (then alpha = 2^(m_old - m_new), else 1), so a weight
// stays <= 64 and a weight times a V scale stays inside fp16. l is not kept here: the PV step's MFMA against a row
// of ones sums the weights.
__device__ __forceinline__ void stream_softmax(const floatx4 (&sc)[2], int32_t lim_rel, float c2, int32_t qg,
                                               float & m_run, float (&pf)[8], float & alpha) {
    float raw[8];
    float mx = kNegInf;
    if (__all(lim_rel >= 31)) {
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
                const float x = 16 * h + 4 * qg + r <= lim_rel ? sc[h][r] : kNegInf;
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
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        pf[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(raw[i], c2, -m_use));
    }
    m_run = m_new;
}

// ---- the split-K fold inside the launch ----
//
// With a.fold set (the launch's grid fits the device at once), the splits of a (sequence, KV head) fold among
// themselves, as the reference's finish does after its grid barrier (fn/kernels/qsa/attend.cu:621-655): each split
// writes its partial (m, l, acc) with device-scope stores, waits for them, and adds one to the pair's arrival counter;
// row r is then folded by the pair's split r mod n (its owner), which polls the counter until all n splits have
// arrived (M = max m_j, L = sum l_j 2^(m_j - M), o = sum acc_j 2^(m_j - M) / L, in a fixed order) and writes the
// fp16 output. Every wait is bounded by a.fold_spin (real-time ticks): an owner that times out marks its rows given
// up, and the last split to arrive (which never waits for arrivals) folds them. The counter is never reset: the last
// split rounds it up to the next multiple of kFoldEpoch, so a launch's arrivals start at a multiple of it (the
// workspace's fold region starts zeroed, as the reference's counter: attend.h:89-93) and the quotient numbers the
// launch; a row's state word holds that number (above two bits: 1 taken by its owner, 2 given up).
// Fold-state words of a (sequence, KV head): [0] arrivals, [1] unused, [2 + r] row r's state.

__device__ __forceinline__ void store_agent(float * p, floatx4 v) {
    uint64_t * q = reinterpret_cast<uint64_t *>(p);
    __hip_atomic_store(q, __builtin_bit_cast(uint64_t, float2{v[0], v[1]}), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, __builtin_bit_cast(uint64_t, float2{v[2], v[3]}), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent2(float * p, float x, float y) {
    __hip_atomic_store(reinterpret_cast<uint64_t *>(p), __builtin_bit_cast(uint64_t, float2{x, y}), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 load_agent2(const float * p) {
    return __builtin_bit_cast(float2, __hip_atomic_load(reinterpret_cast<const uint64_t *>(p), __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ uint32_t load_agent(const uint32_t * p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 4 output values of row r (values c0 .. c0 + 3) as fp16, scaled by inv
__device__ __forceinline__ void store_out4(const dec_args & a, int32_t s, int32_t kvh, int32_t r, int32_t c0, floatx4 v,
                                           float inv) {
    const int32_t t = r / a.G, h = kvh * a.G + r % a.G;
    uint16_t * dst = a.out + ((int64_t(s) * a.T + t) * a.hq + h) * kHeadDim + c0;
    uint2 pk;
    pk.x = uint32_t(__half_as_ushort(__float2half_rn(v[0] * inv))) |
           (uint32_t(__half_as_ushort(__float2half_rn(v[1] * inv))) << 16);
    pk.y = uint32_t(__half_as_ushort(__float2half_rn(v[2] * inv))) |
           (uint32_t(__half_as_ushort(__float2half_rn(v[3] * inv))) << 16);
    *reinterpret_cast<uint2 *>(dst) = pk;
}

__device__ __forceinline__ floatx4 load_agent4(const float * p) {
    const float2 x = load_agent2(p), y = load_agent2(p + 2);
    return floatx4{x.x, x.y, y.x, y.y};
}

// Fold the rows in `mask` (bit k: row sp + k n) of the pair (s, kvh) from the n splits' partials and write them; all
// 512 threads take part. A row is 4 shares (split i to share i mod 4), a share 64 threads of 4 values each folding
// its splits in order with a running max; then the 4 shares fold in order in LDS. Two rows a pass. The order of every
// operation is fixed by the row alone, so any split that folds a row writes the same bits.
template <int THREADS>
__device__ void fold_rows(const dec_args & a, int32_t s, int32_t kvh, int32_t sp, int32_t n, uint32_t mask,
                          uint8_t * smem) {
    static_assert(THREADS == 512, "8 slots of 64 threads");
    constexpr int32_t kShares = 4, kBatch = 16;
    const int32_t tid = static_cast<int32_t>(threadIdx.x);
    const int32_t slot = tid >> 6, c = tid & 63;
    const int32_t rr = slot >> 2, g = slot & 3; // the pass's row (0, 1) and this slot's share
    const int32_t s0 = a.split0[s], h_kv = a.pv.h_kv;
    floatx4 * part = reinterpret_cast<floatx4 *>(smem); // [slot][64][2]: (m, l, -, -), acc
    while (mask != 0) {
        int32_t rows[2] = {-1, -1};
        for (int32_t m = 0; m < 2 && mask != 0; ++m) {
            const int32_t k = __builtin_ctz(mask);
            mask &= mask - 1;
            rows[m] = sp + k * n;
        }
        const int32_t r = rows[rr];
        if (r >= 0) {
            float M = kNegInf, L = 0.0f;
            bool bad_share = false;
            floatx4 A = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int32_t i0 = g; i0 < n; i0 += kBatch * kShares) {
                float2 mlv[kBatch];
                floatx4 v[kBatch];
#pragma unroll
                for (int q = 0; q < kBatch; ++q) {
                    const int32_t i = i0 + q * kShares;
                    mlv[q] = float2{kNegInf, 0.0f};
                    v[q] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
                    if (i < n) {
                        const int64_t prow = (int64_t(s0 + i) * h_kv + kvh) * a.R + r;
                        mlv[q] = load_agent2(a.pml + prow * 2);
                        v[q] = load_agent4(a.po + prow * kHeadDim + 4 * c);
                    }
                }
#pragma unroll
                for (int q = 0; q < kBatch; ++q) {
                    bad_share = bad_share || mlv[q].x != mlv[q].x;
                    const float mn = fmaxf(M, mlv[q].x);
                    const float mu = mn == kNegInf ? 0.0f : mn;
                    const float fo = __builtin_amdgcn_exp2f(M - mu), fn = __builtin_amdgcn_exp2f(mlv[q].x - mu);
                    L = __builtin_fmaf(L, fo, mlv[q].y * fn);
                    A = A * fo + v[q] * fn;
                    M = mn;
                }
            }
            part[(slot * 64 + c) * 2 + 0] = floatx4{M, L, bad_share ? 1.0f : 0.0f, 0.0f};
            part[(slot * 64 + c) * 2 + 1] = A;
        }
        __syncthreads();
        if (g == 0 && r >= 0) { // the row's 4 shares in order
            float M = kNegInf, L = 0.0f;
            bool bad = false;
            floatx4 A = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int32_t gg = 0; gg < kShares; ++gg) {
                const floatx4 ml = part[((rr * 4 + gg) * 64 + c) * 2 + 0];
                bad = bad || ml[2] != 0.0f;
                const floatx4 p = part[((rr * 4 + gg) * 64 + c) * 2 + 1];
                const float mn = fmaxf(M, ml[0]);
                const float mu = mn == kNegInf ? 0.0f : mn;
                const float fo = __builtin_amdgcn_exp2f(M - mu), fn = __builtin_amdgcn_exp2f(ml[0] - mu);
                L = __builtin_fmaf(L, fo, ml[1] * fn);
                A = A * fo + p * fn;
                M = mn;
            }
            const int32_t t = r / a.G, h = kvh * a.G + r % a.G;
            const float inv = bad ? 0.0f : 1.0f / L;
            uint2 pk;
            pk.x = uint32_t(__half_as_ushort(__float2half_rn(A[0] * inv))) |
                   (uint32_t(__half_as_ushort(__float2half_rn(A[1] * inv))) << 16);
            pk.y = uint32_t(__half_as_ushort(__float2half_rn(A[2] * inv))) |
                   (uint32_t(__half_as_ushort(__float2half_rn(A[3] * inv))) << 16);
            if (!bad) { // a split that saw an unmapped page marks its partial: nothing is written for the row
                *reinterpret_cast<uint2 *>(a.out + ((int64_t(s) * a.T + t) * a.hq + h) * kHeadDim + 4 * c) = pk;
            }
        }
        __syncthreads(); // part is rewritten by the next pass
    }
}

// The split's part of the pair's fold (the protocol above); called by every thread after the partial's stores
template <int THREADS>
__device__ void fold_splits(const dec_args & a, int32_t s, int32_t kvh, int32_t sp, int32_t n, uint8_t * smem) {
    const int32_t tid = static_cast<int32_t>(threadIdx.x);
    uint32_t * st = a.fold + (int64_t(s) * a.pv.h_kv + kvh) * kFoldWords;
    uint32_t * shared_word = reinterpret_cast<uint32_t *>(smem + 16384); // past fold_rows' LDS
    const int32_t R = a.R;
    // this split's rows: sp, sp + n, ... (bit k: row sp + k n)
    uint32_t own = 0;
    for (int32_t r = sp, k = 0; r < R; r += n, ++k) {
        own |= 1u << k;
    }
    wait_vmcnt<0>(); // this thread's partial stores are complete (device scope)
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(st, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old % kFoldEpoch == static_cast<uint32_t>(n - 1)) { // the last: round the count up to the next epoch
            __hip_atomic_fetch_add(st, kFoldEpoch - static_cast<uint32_t>(n), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        shared_word[0] = old;
    }
    __syncthreads();
    const uint32_t old = shared_word[0];
    const uint32_t base = old - old % kFoldEpoch;
    const uint32_t tag = (base / kFoldEpoch + 1) << 2; // this launch's row-state tag (the epoch), low bits the state
    const bool last = old % kFoldEpoch == static_cast<uint32_t>(n - 1);
    if (!last) {
        if (own == 0) {
            return;
        }
        // poll (bounded) until every split has arrived; then take the rows, or give them up to the last split
        if (tid == 0) {
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            bool all = false;
            for (;;) {
                if (load_agent(st) - base >= static_cast<uint32_t>(n)) {
                    all = true;
                    break;
                }
                if (__builtin_amdgcn_s_memrealtime() - t0 > static_cast<uint64_t>(a.fold_spin)) {
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            for (uint32_t m = own; m != 0; m &= m - 1) {
                __hip_atomic_store(st + 2 + sp + __builtin_ctz(m) * n, tag | (all ? 1u : 2u), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
            shared_word[1] = all ? own : 0u;
        }
        __syncthreads();
        const uint32_t mine = shared_word[1];
        if (mine != 0) {
            fold_rows<THREADS>(a, s, kvh, sp, n, mine, smem);
        }
        return;
    }
    // the last split: its own rows at once; then, polling every other row's state in parallel (lane r of wave 0),
    // the rows their owners gave up (or, past every owner's bound, never decided) as well
    fold_rows<THREADS>(a, s, kvh, sp, n, own, smem);
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    const uint64_t patience = 2 * static_cast<uint64_t>(a.fold_spin) + 10000; // past every owner's own bound
    if (tid < 64) {
        const int32_t r = tid;
        const bool mine = r < R && r >= sp && (r - sp) % n == 0;
        bool take = false;
        bool pending = r < R && !mine;
        while (__any(pending)) {
            if (pending) {
                const uint32_t w = load_agent(st + 2 + r);
                if ((w & ~3u) == tag) {
                    pending = false;
                    take = (w & 3u) == 2u;
                }
            }
            if (__builtin_amdgcn_s_memrealtime() - t0 > patience) {
                take = take || pending;
                pending = false;
            }
            if (__any(pending)) {
                __builtin_amdgcn_s_sleep(1);
            }
        }
        const uint64_t b = __ballot(take);
        if (tid == 0) {
            shared_word[1] = static_cast<uint32_t>(b);
        }
    }
    __syncthreads();
    for (uint32_t m = shared_word[1]; m != 0; m &= m - 1) {
        const int32_t r = __builtin_ctz(m);
        fold_rows<THREADS>(a, s, kvh, r % n, n, 1u << (r / n), smem);
    }
}

template <int NT, bool KV8>
__global__ __launch_bounds__(512, 1) void stream_kernel(dec_args a) {
    using SH = stream_shape<NT>;
    constexpr int WAVES = SH::WAVES, STREAMS = SH::STREAMS;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    FNKV_STAMP(5);
    const int32_t lane = static_cast<int32_t>(threadIdx.x) & 63;
    const int32_t wave = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(threadIdx.x) >> 6);
    const int32_t j = lane & 15, qg = lane >> 4;
    const int32_t split = static_cast<int32_t>(blockIdx.x);
    const int32_t kvh = static_cast<int32_t>(blockIdx.y);
    const int32_t s = seq_of(a, split);
    const int32_t sp = split - a.split0[s];
    // the context (host contexts), or the host's bound on it (device contexts: the walk is strided and its page
    // lookups are sized by the bound, so the device word is read after they are issued)
    int64_t ctx = a.ctx[s];
    const int64_t begin = int64_t(sp) * a.split_tokens;
    const pool_view & pv = a.pv;
    const int32_t * table = pv.table + int64_t(a.slot[s]) * pv.table_stride;

    // The Q operands of every row tile go into LDS once (the workgroup's waves share them: wave w loads operands w,
    // w + 8, ...); their loads are issued first, beside the page-table read
    uint8_t * const qs = smem + SH::RING;
    constexpr int PER = NT * kBlocks / WAVES;
    // (a padding row takes the last real row's q, loaded unconditionally: a load under a branch would make the
    // compiler wait for it before the page-table read; padding rows are computed like the others and never folded or
    // written)
    u32x4 qv[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int32_t c = wave + e * WAVES, rt = c / kBlocks, b = c % kBlocks;
        const int32_t row = rt * 16 + j < a.R ? rt * 16 + j : a.R - 1;
        const int32_t t_row = row / a.G;
        qv[e] = *reinterpret_cast<const u32x4 *>(
            a.q + ((int64_t(s) * a.T + t_row) * a.hq + int64_t(kvh) * a.G + row % a.G) * kHeadDim + b * kQK + 8 * qg);
    }
    split_src<false> src;
    src.template init<64 * WAVES>(a, table, split, begin, ctx < begin + a.split_tokens ? ctx : begin + a.split_tokens,
                                  lane, smem, nullptr, ctx);
    if (a.ctx_dev != nullptr) {
        ctx = seq_ctx<false>(a, s);
        src.recount(ctx);
    }
    const int64_t end = ctx < begin + a.split_tokens ? ctx : begin + a.split_tokens;
    FNKV_STAMP(6);
    if (refused<false>(a, s, ctx, sp, kvh)) {
        return;
    }
    const bool unmapped = src.guard_unmapped(lane);
    report_unmapped(a, unmapped);
    // uniform in the workgroup; readfirstlane keeps the walk's arithmetic and the loop control scalar
    const int32_t n_tiles = __builtin_amdgcn_readfirstlane(src.n_tiles);
    FNKV_STAMP(0);
    // the step's new cells are written by the workgroup whose walk holds their tile (append_new_cells); only such a
    // workgroup waits for its stores before its loads
    if (a.k_new != nullptr && !unmapped) {
        bool owns = false;
        for (int32_t t = 0; t < a.T; ++t) {
            const int64_t pos = ctx - a.T + t;
            owns |= a.strided ? static_cast<int32_t>((pos >> 5) % src.stride) == src.g0 : (pos >= begin && pos < end);
        }
        if (owns) {
            append_new_cells<WAVES>(a, table, s, kvh, ctx, begin, end, src.g0, a.strided ? src.stride : 0, wave,
                                    lane);
        }
    }

    // this wave's tile stream (walk tiles st, st + STREAMS, ...) and row group (its row tiles)
    const int32_t st = wave % STREAMS, grp = wave / STREAMS;
    const int32_t n_w = __builtin_amdgcn_readfirstlane(n_tiles > st ? (n_tiles - st + STREAMS - 1) / STREAMS : 0);
    const uint8_t * layer_base = pv.base + int64_t(a.layer) * pv.layer_stride + int64_t(kvh) * kPageBlock;
    uint8_t * const slot = smem + wave * SH::SLOT;
    const int32_t lane16 = lane * 16;
    // iteration i's tile; past the wave's last tile a placeholder (the first tile, every lane reading its first
    // 16 bytes of each chunk), so every iteration issues the same loads and the waits are fixed counts
    auto tile_at = [&](int32_t i) -> const uint8_t * {
        const int32_t ti = i < n_w ? st + i * STREAMS : 0;
        return layer_base + src.tile_off(pv, n_tiles > 0 ? ti : 0);
    };
    // half V = 0: the K codes (chunks 0-7) and the K scales (the scales chunk's lanes 0-31); V = 1: the V codes
    // (chunks 8-15) and the V scales (its lanes 32-63)
    auto issue_half = [&](int32_t i, int32_t V) {
        const rsrc_t r = make_rsrc(tile_at(i), kTileBytes);
        const int32_t voff = i < n_w ? lane16 : 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            buf_lds16<SH::AUX>(r, slot + (8 * V + c) * 1024, voff, (8 * V + c) * 1024);
        }
        if ((lane >> 5) == V) {
            buf_lds16<SH::AUX>(r, slot + kKScales, voff, kKScales);
        }
        keep_issued();
    };

    // the first tile's K half alone: the launch's first requests are every wave's K codes, so the scores start
    // before the V halves are in (V(0) is issued once K(0) has landed)
    if (n_w > 0) {
        issue_half(0, 0);
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        *reinterpret_cast<u32x4 *>(qs + (wave + e * WAVES) * 1024 + lane * 16) = qv[e];
    }
    barrier_keep_loads(); // the Q operands are in LDS (the tile loads stay in flight)
    FNKV_STAMP(1);
    const int32_t n_split = a.split0[s + 1] - a.split0[s];
    const bool direct = a.fold != nullptr && n_split == 1;
    const half8 zero8 = {};
    const _Float16 one = static_cast<_Float16>(1.0f);
    const half8 ones8 = {one, one, one, one, one, one, one, one};

    // The walk and the fold for a wave holding row tiles RTB .. RTB + NTW - 1 (every wave passes the same barriers)
    auto run = [&](auto ntw_c, auto rtb_c) {
        constexpr int32_t NTW = decltype(ntw_c)::value, RTB = decltype(rtb_c)::value;
        const uint8_t * const qw = qs + RTB * kBlocks * 1024; // this wave's row tiles' Q operands
        // each lane's bias operands (the rows' per-block q sums) and each row's last visible cell
        half8 sig[NTW];
        int64_t lim[NTW];
#pragma unroll
        for (int rt = 0; rt < NTW; ++rt) {
            half8 qop[kBlocks];
#pragma unroll
            for (int b = 0; b < kBlocks; ++b) {
                qop[b] = *reinterpret_cast<const half8 *>(qw + (rt * kBlocks + b) * 1024 + lane * 16);
            }
            sig[rt] = q_sums(qop, qg);
            lim[rt] = ctx - a.T + t_of_row(a, RTB + rt, j);
        }
        floatx4 acc[NTW][kBlocks][2];
        floatx4 lv[NTW]; // lane (row j, qg): rows 4 qg + e of sum_t P s_v[t][b] (b < 8) and sum_t P (row 8)
        float m_run[NTW];
#pragma unroll
        for (int rt = 0; rt < NTW; ++rt) {
            lv[rt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            m_run[rt] = kNegInf;
#pragma unroll
            for (int b = 0; b < kBlocks; ++b) {
                acc[rt][b][0] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
                acc[rt][b][1] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }

        // Iteration i: wait for K(i), scores, issue K(i + 1), softmax, wait for V(i), PV, issue V(i + 1). V(0) is
        // issued once K(0) has landed, so it loads under tile 0's scores.
        if (n_w > 0) {
            wait_vmcnt<0>();
            issue_half(0, 1);
        }
        FNKV_PHASE_DECL();
        for (int32_t i = 0; i < n_w; ++i) {
            FNKV_PHASE(0 + (i > 0 ? 7 : 0));
            wait_vmcnt<SH::HALF_LOADS>(); // K(i) has landed (V(i) may be pending)
            FNKV_PHASE(1);
            // the scores and the softmax are the longer dependent chain: their wave issues first on a shared SIMD,
            // so the two waves of a SIMD alternate phases rather than one running ahead
            __builtin_amdgcn_s_setprio(1);
            const uint8_t * kb = slot;
            const uint8_t * sc = kb + kKScales;
            floatx4 scv[NTW][2];
            stream_scores<NTW, KV8>(kb, sc, qw, sig, j, qg, lane, scv);
            issue_half(i + 1, 0); // the scores' reads of K(i) are done (their values are in registers)
            FNKV_PHASE(2);
            const int64_t tok0 = src.tok0(st + i * STREAMS);
            half8 ph[NTW], pl[NTW];
#pragma unroll
            for (int rt = 0; rt < NTW; ++rt) {
                const int64_t lr = lim[rt] - tok0;
                const int32_t lim_rel = lr > 64 ? 64 : static_cast<int32_t>(lr < -1 ? -1 : lr);
                float pf[8];
                float alpha;
                stream_softmax(scv[rt], lim_rel, a.c2, qg, m_run[rt], pf, alpha);
                if (__any(alpha != 1.0f)) {
#pragma unroll
                    for (int b = 0; b < kBlocks; ++b) {
                        acc[rt][b][0] *= alpha;
                        acc[rt][b][1] *= alpha;
                    }
                    lv[rt] *= alpha;
                }
                split_hilo(pf, ph[rt], pl[rt]);
            }
            FNKV_PHASE(3);
            __builtin_amdgcn_s_setprio(0);
            wait_vmcnt<SH::HALF_LOADS>(); // V(i) has landed (K(i + 1) may be pending)
            FNKV_PHASE(4);
            // A of the bias MFMAs: lane (block j < 8, qg) holds s_v[token(qg, slot)][j], lanes j = 8 ones (l)
            const half8 sva =
                j < 8 ? *reinterpret_cast<const half8 *>(sc + 512 + qg * 128 + j * 16) : j == 8 ? ones8 : zero8;
#pragma unroll
            for (int rt = 0; rt < NTW; ++rt) {
                lv[rt] = mfma16(sva, ph[rt], lv[rt]);
                lv[rt] = mfma16(sva, pl[rt], lv[rt]);
            }
            // each block's V codes and scales are read from LDS one block ahead
            u32x4 vw_next = *reinterpret_cast<const u32x4 *>(kb + kVCodes + lane * 16);
            half8 vs_next = *reinterpret_cast<const half8 *>(sc + 512 + qg * 128);
            // KV8: a group's two blocks share their scales, so its P x V-scale products serve both
            half8 phs[NTW], pls[NTW];
#pragma unroll
            for (int b = 0; b < kBlocks; ++b) {
                const u32x4 vw = vw_next;
                const half8 vs = vs_next;
                if (b + 1 < kBlocks) {
                    vw_next = *reinterpret_cast<const u32x4 *>(kb + kVCodes + (b + 1) * 1024 + lane * 16);
                    if (!KV8 || (b & 1) == 1) {
                        vs_next = *reinterpret_cast<const half8 *>(sc + 512 + qg * 128 + (b + 1) * 16);
                    }
                }
                const half8 va0 = widen8<false>(vw[0], vw[1]);
                const half8 va1 = widen8<false>(vw[2], vw[3]);
#pragma unroll
                for (int rt = 0; rt < NTW; ++rt) {
                    if (!KV8 || (b & 1) == 0) {
                        scale_hilo_pk(ph[rt], pl[rt], vs, phs[rt], pls[rt]);
                    }
                    const half8 hi = phs[rt], lo = pls[rt];
                    acc[rt][b][0] = mfma16(va0, hi, acc[rt][b][0]);
                    acc[rt][b][1] = mfma16(va1, hi, acc[rt][b][1]);
                    acc[rt][b][0] = mfma16(va0, lo, acc[rt][b][0]);
                    acc[rt][b][1] = mfma16(va1, lo, acc[rt][b][1]);
                }
                __builtin_amdgcn_sched_barrier(0); // one block's operands live at a time
            }
            issue_half(i + 1, 1);
            FNKV_PHASE(5);
        }
        FNKV_PHASE_STORE();
        wait_vmcnt<0>();
        FNKV_STAMP_WAVE();

        // the V bias: acc[rt][b] carries 1152 lv[rt][b]; lv[rt][b] of this lane's row sits in lane (j, b / 4),
        // element b % 4; the row's l in lane (j, 2), element 0
        float l_row[NTW];
#pragma unroll
        for (int rt = 0; rt < NTW; ++rt) {
#pragma unroll
            for (int b = 0; b < kBlocks; ++b) {
                const float lb = __shfl(lv[rt][b & 3], j + 16 * (b >> 2));
                acc[rt][b][0] -= 1152.0f * lb;
                acc[rt][b][1] -= 1152.0f * lb;
            }
            l_row[rt] = __shfl(lv[rt][0], j + 32);
        }

        // ---- fold the STREAMS waves holding each row tile (fixed order), then the workgroup's row: the output itself
        // when the split is its sequence's only one, else the split's partial. A wave writes a row tile's unscaled
        // accumulators and its rows' (m, l) into its own tile slot as soon as its walk has ended (no other wave
        // reads that slot), so the first waves' writes run beside the last waves' walks; the reads scale each
        // holder's values by 2^(m - M). Pass k folds each group's k-th row tile. ----
        constexpr int32_t OS = SH::OSTRIDE;
        constexpr int32_t ML = 16 * OS;                 // floats: (m, l) of the slot's 16 rows, after its values
        static_assert((ML + 16 * 2) * 4 <= SH::SLOT, "a row tile's fold buffer fits a tile slot");
        constexpr int32_t PASSES = SH::GROUPS == 1 ? NT : 2;
        float * const mine = reinterpret_cast<float *>(slot);
#pragma unroll
        for (int32_t k = 0; k < PASSES; ++k) {
            if (k < NTW) {
                if ((RTB + k) * 16 + j < a.R) { // padding rows are not folded
#pragma unroll
                    for (int b = 0; b < kBlocks; ++b) {
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh) {
                            *reinterpret_cast<floatx4 *>(mine + j * OS + 16 * (2 * b + hh) + 4 * qg) = acc[k][b][hh];
                        }
                    }
                }
                if (qg == 0) {
                    *reinterpret_cast<float2 *>(mine + ML + 2 * j) = float2{m_run[k], l_row[k]};
                }
            }
            __syncthreads();
            if (k == 0) {
                FNKV_STAMP(2);
            }
            // thread -> (row, values c0 .. c0 + 3 and 128 + c0 .. + 3) of each of the pass's row tiles: 16 rows x 32
            // groups (a row's 32 threads read consecutive 16-byte pieces of each holder's slot, conflict-free)
#pragma unroll
            for (int32_t g = 0; g < SH::GROUPS; ++g) {
                const int32_t ntw_g = SH::GROUPS == 1 ? NT : (g == 0 ? 2 : 1);
                const int32_t rtb_g = g == 0 ? 0 : 2;
                if (k >= ntw_g) {
                    continue;
                }
                const int32_t rt = rtb_g + k;
                const int32_t t = static_cast<int32_t>(threadIdx.x);
                const int32_t rrow = t >> 5, c0 = (t & 31) * 4;
                const int32_t r = rt * 16 + rrow;
                if (r >= a.R) {
                    continue;
                }
                const float * const hold = reinterpret_cast<const float *>(smem + g * STREAMS * SH::SLOT);
                float2 mlw[STREAMS];
                float Mr = kNegInf;
#pragma unroll
                for (int w = 0; w < STREAMS; ++w) {
                    mlw[w] = *reinterpret_cast<const float2 *>(hold + w * (SH::SLOT / 4) + ML + 2 * rrow);
                    Mr = fmaxf(Mr, mlw[w].x);
                }
                const float Mr_use = Mr == kNegInf ? 0.0f : Mr;
                float L = 0.0f;
                floatx4 sum[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
                for (int w = 0; w < STREAMS; ++w) {
                    const float f = __builtin_amdgcn_exp2f(mlw[w].x - Mr_use);
                    L = __builtin_fmaf(mlw[w].y, f, L);
#pragma unroll
                    for (int c = 0; c < 2; ++c) {
                        const floatx4 v =
                            *reinterpret_cast<const floatx4 *>(hold + w * (SH::SLOT / 4) + rrow * OS + c0 + 128 * c);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            sum[c][e] = __builtin_fmaf(v[e], f, sum[c][e]);
                        }
                    }
                }
                if (unmapped) {
                    Mr = __builtin_nanf(""); // the merge (or the fold) writes nothing for this row
                }
                if (direct && !unmapped) {
                    store_out4(a, s, kvh, r, c0, sum[0], 1.0f / L);
                    store_out4(a, s, kvh, r, 128 + c0, sum[1], 1.0f / L);
                } else if (!direct) {
                    const int64_t prow = (int64_t(split) * pv.h_kv + kvh) * a.R + r;
                    float * dst = a.po + prow * kHeadDim + c0;
                    if (a.fold != nullptr) { // read by other workgroups in this launch: device-scope stores
                        store_agent(dst, sum[0]);
                        store_agent(dst + 128, sum[1]);
                        if ((t & 31) == 0) {
                            store_agent2(a.pml + prow * 2, Mr, L);
                        }
                    } else {
                        *reinterpret_cast<floatx4 *>(dst) = sum[0];
                        *reinterpret_cast<floatx4 *>(dst + 128) = sum[1];
                        if ((t & 31) == 0) {
                            a.pml[prow * 2 + 0] = Mr;
                            a.pml[prow * 2 + 1] = L;
                        }
                    }
                }
            }
            if (k + 1 < PASSES) {
                __syncthreads(); // the slots are rewritten by the next pass
            }
        }
    };
    if constexpr (SH::GROUPS == 1) {
        run(std::integral_constant<int32_t, NT>(), std::integral_constant<int32_t, 0>());
    } else {
        if (grp == 0) {
            run(std::integral_constant<int32_t, 2>(), std::integral_constant<int32_t, 0>());
        } else {
            run(std::integral_constant<int32_t, 1>(), std::integral_constant<int32_t, 2>());
        }
    }
    FNKV_STAMP(3);
    if (a.fold != nullptr && !direct) {
        fold_splits<64 * WAVES>(a, s, kvh, sp, n_split, smem);
    }
    FNKV_STAMP(4);
}

// The split size (cells) for these contexts: the fewest rounds of one workgroup a CU times a workgroup's time, which
// is its waves' longest walk (the split's tiles over its tile streams, rounded up) plus a fixed cost (the ramp, the fold of the
// waves and the partial's write, counted as three tiles); larger splits (fewer partials) win ties.
int32_t choose_split_stream(int32_t n_seq, const int64_t * ctx, int32_t h_kv, int32_t cus, int32_t NT) {
    const int32_t streams = NT == 3 ? stream_shape<3>::STREAMS : stream_shape<1>::STREAMS;
    int32_t best = kPageTokens;
    int64_t best_cost = INT64_MAX;
    for (int32_t sz = kPageTokens; sz <= 8 * kPageTokens; sz += kTileTokens) {
        int64_t wgs = 0;
        for (int32_t i = 0; i < n_seq; ++i) {
            wgs += (ctx[i] + sz - 1) / sz;
        }
        wgs *= h_kv;
        const int64_t rounds = (wgs + cus - 1) / cus;
        const int64_t wave_tiles = (sz / kTileTokens + streams - 1) / streams;
        const int64_t cost = rounds * (wave_tiles + 3);
        if (cost <= best_cost) {
            best_cost = cost;
            best = sz;
        }
    }
    return best;
}

template <int NT> void set_stream_attr() {
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(stream_kernel<NT, false>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, stream_shape<NT>::LDS);
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(stream_kernel<NT, true>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, stream_shape<NT>::LDS);
}

// the dense launch's kernel for NT row tiles (1 .. 3) and the pool's format, its LDS attribute set once per device
void launch_stream(int32_t device, int32_t NT, dim3 grid, const dec_args & a, hipStream_t st) {
    static std::once_flag attr_once[64];
    if (device >= 0 && device < 64) {
        std::call_once(attr_once[device], [device]() {
            int32_t cur = 0;
            (void)hipGetDevice(&cur);
            (void)hipSetDevice(device);
            set_stream_attr<1>();
            set_stream_attr<2>();
            set_stream_attr<3>();
            (void)hipGetLastError();
            (void)hipSetDevice(cur);
        });
    }
    const dim3 block(64 * stream_shape<1>::WAVES);
    const bool kv8 = a.pv.format == kFormatKV8;
    if (NT == 1) {
        if (kv8) {
            hipLaunchKernelGGL((stream_kernel<1, true>), grid, block, stream_shape<1>::LDS, st, a);
        } else {
            hipLaunchKernelGGL((stream_kernel<1, false>), grid, block, stream_shape<1>::LDS, st, a);
        }
    } else if (NT == 2) {
        if (kv8) {
            hipLaunchKernelGGL((stream_kernel<2, true>), grid, block, stream_shape<2>::LDS, st, a);
        } else {
            hipLaunchKernelGGL((stream_kernel<2, false>), grid, block, stream_shape<2>::LDS, st, a);
        }
    } else {
        if (kv8) {
            hipLaunchKernelGGL((stream_kernel<3, true>), grid, block, stream_shape<3>::LDS, st, a);
        } else {
            hipLaunchKernelGGL((stream_kernel<3, false>), grid, block, stream_shape<3>::LDS, st, a);
        }
    }
}

} // namespace fnkv
