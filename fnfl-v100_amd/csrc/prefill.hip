// Chunked-prefill attention on the matrix cores: `rows` query tokens of one sequence (the chunk just appended, at
// positions ctx - rows .. ctx - 1) attend causally to the sequence's cells 0 .. ctx - 1 of one layer in the pool.
//
// What it computes (the reference's prompt attention, fn/kernels/qsa/qsa_prompt.h:50-58 and qsa_prompt_attn.cu:
// 229-436, made dense and causal, on the pool's codes): S = Q K^T * scale, online softmax, O = P V, fp16 out. The
// reference rounds its K/V operand to fp16 once (q4_h4, qsa_prompt_attn.cu:195-207) and P to fp16, within a loose
// 2e-2 bound; here every product carries ~19 bits or more, so the result meets 2e-3 against fp64 even when a few
// cells dominate: the K and V codes go to the matrix cores exactly (an int8 code is an exact fp16 integer), each K
// block's scale multiplies that block's fp32 scores, and P times each V block's scales enters as hi + lo fp16.
//
// How (MI355X): matrix-core bound (4 d flops a visible (query, key) pair and head), so K/V tiles are converted once
// a workgroup and shared by all its query rows.
//   * A workgroup (8 waves, two a SIMD, so one wave's matrix-core work overlaps the other's VALU work) owns 256 query
//     rows (256 / G query tokens x the G heads of one KV head); each wave owns two 16-row tiles, so each operand
//     read from LDS feeds two MFMAs. Its waves walk the key tiles (32 tokens) of the workgroup's key split in order;
//     the splits (blockIdx.z) fill the device when the row blocks alone do not, and a merge kernel folds them.
//   * Each tile's codes go from HBM straight into the registers of the wave that converts them (wave w: K chunk w
//     and V chunk w, a tile ahead), its scales chunk into a small LDS ring; every wave writes its two chunks as fp16
//     operand planes (K codes, V codes; double-buffered: tile k + 1's while tile k is computed), and four waves
//     write the K scales in the scores' lane order beside them; then every wave runs S^T = K Q^T (one
//     v_mfma_f32_16x16x32_f16 a block, half and row tile, then one FMA a score for the block's scale) and
//     O^T += V^T P^T (two a 16-value tile and row tile: the codes against (P x V scale) hi and lo). Against
//     dequantized hi + lo K and V planes this halves the operand bytes each wave reads from LDS and cuts the MFMAs a
//     wave and tile from 159 to 96.
//   * The softmax (base 2, the running max moved lazily) runs on the S^T registers as in the decode kernel; P feeds
//     the PV MFMA in place.
#include "../../include/fnkv.h"
#include "common.h"
#include "layout.h"
#include "mfma.h"

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>

namespace fnkv {

#ifdef FNKV_TIMING
uint64_t * timing_buffer();
#define PF_T(i)                                                                                                    \
    do {                                                                                                           \
        const uint64_t now_ = __builtin_amdgcn_s_memtime();                                                        \
        if ((i) > 0) {                                                                                             \
            pf_ph[(i)-1] += now_ - pf_last;                                                                        \
        }                                                                                                          \
        pf_last = now_;                                                                                            \
    } while (0)
#else
#define PF_T(i)                                                                                                    \
    do {                                                                                                           \
    } while (0)
#endif

constexpr int32_t kPfWaves = 8;                      // two a SIMD
constexpr int32_t kPfNT = 2;                         // 16-row tiles a wave (each plane read serves both)
constexpr int32_t kPfRows = kPfWaves * kPfNT * 16;   // 256 rows a workgroup
constexpr int32_t kPfPlane = 16 * 1024;             // one fp16 operand plane of a tile
constexpr int32_t kPfKsc = 512;                      // the K scales in the scores' lane order: [half][block][qg][4]
constexpr int32_t kPfKscOff = 2 * kPfPlane;
constexpr int32_t kPfSet = kPfKscOff + kPfKsc;       // a tile's planes: K codes, V codes, K scales
constexpr int32_t kPfScaleRing = 4;                  // tiles' scale chunks (K then V scales, 1 KiB), a ring
constexpr int32_t kPfPages = 2048;                   // the split's page table entries held in LDS (a split <= 512 K cells)
constexpr int32_t kPfLds = 2 * kPfSet + kPfScaleRing * 1024 + kPfPages * 4; // planes double-buffered, ring, pages
constexpr float kPfNegInf = -__builtin_inff();
constexpr float kPfLazyLog2 = 6.0f; // the running max moves only past this margin

struct pf_args {
    pool_view pv;
    const uint16_t * q; // fp16 [rows][hq][256]
    uint16_t * out;     // fp16 [rows][hq][256]
    float * po;         // split partials (n_split > 1): acc [split][h_kv][row blocks * kPfRows][256]
    float * pml;        // ... and (m, l) [split][h_kv][row blocks * kPfRows][2]
    float c2;           // scale * log2(e)
    int64_t ctx;        // cells of the sequence (the chunk included)
    int32_t rows, G, hq, layer, slot;
    int32_t n_split, split_tiles; // key tiles split over blockIdx.z: split z takes tiles z * split_tiles ..
#ifdef FNKV_TIMING
    uint64_t * ts; // per wave: phase cycle sums (instrumented builds only)
#endif
};

// this wave's code chunks of a tile (K chunk w, then V chunk w: 16 B a lane each) into registers
__device__ __forceinline__ void pf_load_codes(const uint8_t * tile, int32_t wave, int32_t lane, u32x4 (&c)[2]) {
    __asm__ __volatile__("" ::: "memory"); // younger than every load issued before (the waits count on it)
    c[0] = stream_load16(tile + kKCodes + wave * 1024 + lane * 16);
    c[1] = stream_load16(tile + kVCodes + wave * 1024 + lane * 16);
    keep_issued();
}

__global__ __launch_bounds__(64 * kPfWaves, 1) void prefill_kernel(pf_args a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int32_t lane = static_cast<int32_t>(threadIdx.x) & 63;
    const int32_t wave = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(threadIdx.x) >> 6);
    const int32_t j = lane & 15, qg = lane >> 4;
    const int32_t kvh = static_cast<int32_t>(blockIdx.y);
    const int32_t tok_per_wg = kPfRows / a.G;
    const int32_t t_first = static_cast<int32_t>(blockIdx.x) * tok_per_wg;
    const int64_t pos_first = a.ctx - a.rows; // position of query token 0
    const int32_t t_last = min(a.rows, t_first + tok_per_wg) - 1;
    const int64_t key_end = pos_first + t_last + 1; // keys the block's last query sees
    const int32_t n_tiles_all = static_cast<int32_t>((key_end + kTileTokens - 1) / kTileTokens);
    // this workgroup's key tiles: its split's share of those the block's queries see
    const int32_t ts0 = static_cast<int32_t>(blockIdx.z) * a.split_tiles;
    const int32_t n_tiles = max(0, min(n_tiles_all, ts0 + a.split_tiles) - ts0);

    const pool_view & pv = a.pv;
    const int32_t * table = pv.table + int64_t(a.slot) * pv.table_stride;
    const uint8_t * layer_base = pv.base + int64_t(a.layer) * pv.layer_stride + int64_t(kvh) * kPageBlock;
    uint8_t * const plane_base = smem;
    uint8_t * const ring_base = smem + 2 * kPfSet;
    // the split's page table entries, copied into LDS once: a tile's address is then an LDS read, not a memory round
    // trip on the path to its copy
    int32_t * const pages = reinterpret_cast<int32_t *>(ring_base + kPfScaleRing * 1024);
    const int32_t page0 = (ts0 * kTileTokens) >> 8;
    const int32_t n_pages = n_tiles > 0 ? (((ts0 + n_tiles - 1) * kTileTokens) >> 8) - page0 + 1 : 0;
    for (int32_t i = static_cast<int32_t>(threadIdx.x); i < n_pages; i += 64 * kPfWaves) {
        pages[i] = table[page0 + i];
    }
    __syncthreads();
    auto tile_ptr = [&](int32_t li) -> const uint8_t * { // the split's li-th tile (past the last: the last again)
        li = li < n_tiles ? li : n_tiles - 1;
        const int64_t tok = int64_t(ts0 + li) * kTileTokens;
        const int32_t phys = __builtin_amdgcn_readfirstlane(pages[(tok >> 8) - page0]);
        return layer_base + int64_t(phys) * pv.page_stride + int64_t((tok & 255) >> 5) * kTileBytes;
    };
    auto ring = [&](int32_t li) { return ring_base + (li & (kPfScaleRing - 1)) * 1024; };
    auto issue_ring_at = [&](int32_t li, const uint8_t * tp) { // wave 0: tile li (at tp)'s scales chunk into its slot
        if (wave == 0) {
            lds_load16(tp + kKScales + lane * 16, ring(li));
        }
    };
    auto issue_ring = [&](int32_t li) { issue_ring_at(li, tile_ptr(li)); };
    u32x4 codes[2];
#ifdef FNKV_TIMING
    uint64_t pf_ph[8] = {0, 0, 0, 0, 0, 0, 0, 0}, pf_last = 0;
#endif
    // the first tile's copies before the Q loads (their latencies overlap)
    if (n_tiles > 0) {
        issue_ring(0);
        pf_load_codes(tile_ptr(0), wave, lane, codes);
    }

    // Q operands (B of S^T = K Q^T) of this wave's two row tiles, and each row's causal limit
    half8 qop[kPfNT][kBlocks];
    int32_t lim[kPfNT]; // each row's last visible cell, relative to the split's first
#pragma unroll
    for (int nt = 0; nt < kPfNT; ++nt) {
        const int32_t r = (wave * kPfNT + nt) * 16 + j;
        const int32_t t = t_first + r / a.G;
        const bool real = t < a.rows;
        lim[nt] = static_cast<int32_t>((real ? pos_first + t : pos_first + t_last) - int64_t(ts0) * kTileTokens);
        const uint16_t * qrow = a.q + (int64_t(real ? t : t_last) * a.hq + int64_t(kvh) * a.G + r % a.G) * kHeadDim;
#pragma unroll
        for (int b = 0; b < kBlocks; ++b) {
            u32x4 v = {0, 0, 0, 0};
            if (real) {
                v = *reinterpret_cast<const u32x4 *>(qrow + b * kQK + 8 * qg);
            }
            qop[nt][b] = __builtin_bit_cast(half8, v);
        }
    }
    floatx4 acc[kPfNT][16];
    float m_run[kPfNT], l_run[kPfNT];
#pragma unroll
    for (int nt = 0; nt < kPfNT; ++nt) {
        m_run[nt] = kPfNegInf;
        l_run[nt] = 0.0f;
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            acc[nt][m] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }

    // this wave's chunks of tile ti (in `codes`) -> the operand planes of set ti & 1: K and V codes as exact fp16
    // integers, and (waves 0-3) the K scales in the scores' lane order. K chunk w covers tokens 16 (w / 4) .. + 15 and
    // blocks 2 (w % 4), 2 (w % 4) + 1; V chunk w the MFMA tiles 2 w, 2 w + 1 of block w (the V scales stay in the
    // ring, already in the PV operand's slot order)
    auto dequant = [&](int32_t ti) {
        const uint8_t * rg = ring(ti); // K scales [32 tokens][8 blocks], then V scales [4 lane groups][8 blocks][8]
        uint8_t * pl = plane_base + (ti & 1) * kPfSet;
        {
            const int32_t h = wave >> 2, ld = wave & 3;
#pragma unroll
            for (int bb = 0; bb < 2; ++bb) {
                const int32_t b = 2 * ld + bb;
                const int32_t off = ((h * kBlocks + b) * 64 + lane) * 16;
                *reinterpret_cast<half8 *>(pl + off) = widen8(codes[0][2 * bb], codes[0][2 * bb + 1]);
            }
        }
        if (wave < 4) { // entry ((h, b, qg), r) = the scale of token 16 h + 4 qg + r, block b
            const int32_t e = static_cast<int32_t>(threadIdx.x);
            const int32_t r = e & 3, g = (e >> 2) & 3, b = (e >> 4) & 7, h = e >> 7;
            *reinterpret_cast<uint16_t *>(pl + kPfKscOff + e * 2) =
                *reinterpret_cast<const uint16_t *>(rg + (16 * h + 4 * g + r) * 16 + b * 2);
        }
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
            const int32_t off = ((2 * wave + mm) * 64 + lane) * 16;
            *reinterpret_cast<half8 *>(pl + kPfPlane + off) = widen8(codes[1][2 * mm], codes[1][2 * mm + 1]);
        }
    };

    // tile ti on planes set ti & 1: scores, then `between` (the next tile's conversion, its VALU work beside the last
    // score MFMAs and the softmax's dependent chains), online softmax, PV
    auto compute = [&](int32_t ti, auto && between) {
        const uint8_t * pl = plane_base + (ti & 1) * kPfSet;
        floatx4 sc[kPfNT][2];
#pragma unroll
        for (int nt = 0; nt < kPfNT; ++nt) {
            sc[nt][0] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            sc[nt][1] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        // S^T block by block: the block's MFMA on the exact codes, then its K scale (the lane's four tokens) by one
        // FMA a score; the next block's operands are read from LDS while this block's MFMAs run
        auto kc_at = [&](int hb) { return *reinterpret_cast<const half8 *>(pl + (hb * 64 + lane) * 16); };
        auto ks_at = [&](int hb) { return *reinterpret_cast<const half4v *>(pl + kPfKscOff + (hb * 4 + qg) * 8); };
        half8 kc_next = kc_at(0);
        half4v ks_next = ks_at(0);
#pragma unroll
        for (int hb = 0; hb < 2 * kBlocks; ++hb) {
            const int h = hb / kBlocks, b = hb % kBlocks;
            const half8 kc = kc_next;
            const half4v ks = ks_next;
            if (hb + 1 < 2 * kBlocks) {
                kc_next = kc_at(hb + 1);
                ks_next = ks_at(hb + 1);
            }
            floatx4 t[kPfNT];
#pragma unroll
            for (int nt = 0; nt < kPfNT; ++nt) {
                t[nt] = mfma16(kc, qop[nt][b], floatx4{0.0f, 0.0f, 0.0f, 0.0f});
            }
#pragma unroll
            for (int nt = 0; nt < kPfNT; ++nt) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    sc[nt][h][r] = __builtin_fmaf(static_cast<float>(ks[r]), t[nt][r], sc[nt][h][r]);
                }
                __asm__ volatile("" : "+v"(sc[nt][h]));
            }
            if (hb & 1) {
                __builtin_amdgcn_sched_barrier(0); // two blocks' products live at a time
            }
        }
#ifdef FNKV_TIMING
        {
            const uint64_t now_ = __builtin_amdgcn_s_memtime();
            pf_ph[4] += now_ - pf_last;
            pf_last = now_;
        }
#endif
        between();
        half8 ph[kPfNT], plo[kPfNT];
#pragma unroll
        for (int nt = 0; nt < kPfNT; ++nt) {
            // this lane's tokens 16 h + r of the tile (r = 4 qg + 0..3) are visible to its row while <= rel
            const int32_t rel = lim[nt] - ti * kTileTokens - 4 * qg;
            float v[8];
            float mx = kPfNegInf;
            if (__all(rel >= 16 + 3)) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        v[4 * h + r] = sc[nt][h][r];
                        mx = fmaxf(mx, sc[nt][h][r]);
                    }
                }
            } else {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float x = 16 * h + r <= rel ? sc[nt][h][r] : kPfNegInf;
                        v[4 * h + r] = x;
                        mx = fmaxf(mx, x);
                    }
                }
            }
            mx = rows_max(mx) * a.c2;
            const bool move = mx > m_run[nt] + kPfLazyLog2; // m_run = -inf: any visible score moves it
            const float m_new = move ? mx : m_run[nt];
            const float m_use = m_new == kPfNegInf ? 0.0f : m_new;
            const float alpha = move ? __builtin_amdgcn_exp2f(m_run[nt] - m_use) : 1.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                v[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(v[i], a.c2, -m_use));
            }
            split_hilo(v, ph[nt], plo[nt]);
            l_run[nt] = __builtin_fmaf(l_run[nt], alpha, sum8(v));
            m_run[nt] = m_new;
            if (__any(alpha != 1.0f)) {
#pragma unroll
                for (int m = 0; m < 16; ++m) {
                    acc[nt][m] *= alpha;
                }
            }
        }
#ifdef FNKV_TIMING
        {
            const uint64_t now_ = __builtin_amdgcn_s_memtime();
            pf_ph[5] += now_ - pf_last;
            pf_last = now_;
        }
#endif
        // O^T += V^T P^T block by block: P times the block's V scales (this lane's 8 tokens) as hi + lo fp16 (to
        // ~2^-19), against the exact codes
        const uint8_t * rgv = ring(ti) + 512 + qg * 128;
#pragma unroll
        for (int b = 0; b < kBlocks; ++b) {
            const half8 v0 = *reinterpret_cast<const half8 *>(pl + kPfPlane + ((2 * b) * 64 + lane) * 16);
            const half8 v1 = *reinterpret_cast<const half8 *>(pl + kPfPlane + ((2 * b + 1) * 64 + lane) * 16);
            const half8 vsb = *reinterpret_cast<const half8 *>(rgv + b * 16);
#pragma unroll
            for (int nt = 0; nt < kPfNT; ++nt) {
                half8 hi, lo;
                scale_hilo_pk(ph[nt], plo[nt], vsb, hi, lo);
                acc[nt][2 * b] = mfma16(v0, hi, acc[nt][2 * b]);
                acc[nt][2 * b + 1] = mfma16(v1, hi, acc[nt][2 * b + 1]);
                acc[nt][2 * b] = mfma16(v0, lo, acc[nt][2 * b]);
                acc[nt][2 * b + 1] = mfma16(v1, lo, acc[nt][2 * b + 1]);
            }
            if (b & 1) {
                __builtin_amdgcn_sched_barrier(0); // two blocks' operands live at a time
            }
        }
    };

    // Iteration ti: [tile ti + 1's scales have landed (wave 0 waited); barrier: planes ti complete, planes
    // (ti + 1) & 1 free] [tile ti's scores] [this wave's codes of tile ti + 1 (loaded during iteration ti - 1) ->
    // planes (ti + 1) & 1] [tile ti + 2's scales and codes issued] [tile ti's softmax and PV]. Every iteration issues
    // the same loads (past the last tile: the last again), so the vmcnt counts are exact: a wave's two code loads,
    // after them nothing; wave 0 issues the scales copy first.
    if (n_tiles > 0) {
        wait_vmcnt<0>();
        __syncthreads(); // tile 0's codes and scales have landed
        dequant(0);
        issue_ring(1);
        pf_load_codes(tile_ptr(1), wave, lane, codes);
    }
    for (int32_t ti = 0; ti < n_tiles; ++ti) {
        PF_T(0);
        if (wave == 0) {
            wait_vmcnt<2>(); // tile ti + 1's scales (its two code loads may be in flight)
        }
        barrier_keep_loads();
        PF_T(1);
        PF_T(2);
        // tile ti + 2's address now: its page-table read (LDS) then waits for nothing else
        const uint8_t * const tp2 = tile_ptr(ti + 2);
        compute(ti, [&] {
            wait_vmcnt<0>(); // this wave's codes of tile ti + 1
            dequant(ti + 1);
            issue_ring_at(ti + 2, tp2);
            pf_load_codes(tp2, wave, lane, codes);
        });
        PF_T(4);
    }
    wait_vmcnt<0>();
#ifdef FNKV_TIMING
    if (lane == 0 && a.ts != nullptr) {
        const int64_t wg = (int64_t(blockIdx.z) * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
        for (int i = 0; i < 8; ++i) {
            a.ts[(wg * kPfWaves + wave) * 8 + i] = pf_ph[i];
        }
    }
#endif

    // ---- one split: normalise and write; several: the unnormalised partial (acc, m, l) for the merge ----
    if (a.n_split > 1) {
        const int64_t prow0 = (int64_t(blockIdx.z) * gridDim.y + kvh) * (int64_t(gridDim.x) * kPfRows) +
                              int64_t(blockIdx.x) * kPfRows;
#pragma unroll
        for (int nt = 0; nt < kPfNT; ++nt) {
            const float l = rows_sum(l_run[nt]);
            const int64_t prow = prow0 + (wave * kPfNT + nt) * 16 + j;
            float * po = a.po + prow * kHeadDim + 4 * qg;
#pragma unroll
            for (int m = 0; m < 16; ++m) {
                *reinterpret_cast<floatx4 *>(po + 16 * m) = acc[nt][m];
            }
            if (qg == 0) {
                *reinterpret_cast<float2 *>(a.pml + prow * 2) = float2{m_run[nt], l};
            }
        }
        return;
    }
#pragma unroll
    for (int nt = 0; nt < kPfNT; ++nt) {
        float l = l_run[nt];
        l = rows_sum(l);
        const int32_t r = (wave * kPfNT + nt) * 16 + j;
        const int32_t t = t_first + r / a.G;
        if (t < a.rows) {
            const float inv = 1.0f / l;
            uint16_t * o = a.out + (int64_t(t) * a.hq + int64_t(kvh) * a.G + r % a.G) * kHeadDim + 4 * qg;
#pragma unroll
            for (int m = 0; m < 16; ++m) {
                uint2 pk;
                pk.x = uint32_t(__half_as_ushort(__float2half_rn(acc[nt][m][0] * inv))) |
                       (uint32_t(__half_as_ushort(__float2half_rn(acc[nt][m][1] * inv))) << 16);
                pk.y = uint32_t(__half_as_ushort(__float2half_rn(acc[nt][m][2] * inv))) |
                       (uint32_t(__half_as_ushort(__float2half_rn(acc[nt][m][3] * inv))) << 16);
                *reinterpret_cast<uint2 *>(o + 16 * m) = pk;
            }
        }
    }
}

// Folds the splits' partials of each (query token, head): M = max m_z, L = sum l_z 2^(m_z - M), O = sum acc_z
// 2^(m_z - M) / L, in split order. A thread takes 4 values of one row; 64 threads a row.
__global__ __launch_bounds__(256) void prefill_merge_kernel(pf_args a, int32_t rows_pad) {
    const int32_t tid = static_cast<int32_t>(threadIdx.x);
    const int64_t item = int64_t(blockIdx.x) * 4 + (tid >> 6); // (kvh, row) over h_kv x rows_pad
    const int32_t c4 = (tid & 63) * 4;
    const int32_t h_kv = a.pv.h_kv;
    if (item >= int64_t(h_kv) * rows_pad) {
        return;
    }
    const int32_t kvh = static_cast<int32_t>(item / rows_pad);
    const int32_t R = static_cast<int32_t>(item % rows_pad);
    const int32_t tok_per_wg = kPfRows / a.G;
    const int32_t blk = R / kPfRows, r = R % kPfRows;
    const int32_t t = blk * tok_per_wg + r / a.G;
    if (t >= a.rows) {
        return;
    }
    float M = kPfNegInf;
    for (int32_t z = 0; z < a.n_split; ++z) {
        M = fmaxf(M, a.pml[((int64_t(z) * h_kv + kvh) * rows_pad + R) * 2]);
    }
    const float M_use = M == kPfNegInf ? 0.0f : M;
    float L = 0.0f;
    floatx4 A = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int32_t z = 0; z < a.n_split; ++z) {
        const int64_t prow = (int64_t(z) * h_kv + kvh) * rows_pad + R;
        const float2 ml = *reinterpret_cast<const float2 *>(a.pml + prow * 2);
        const float f = __builtin_amdgcn_exp2f(ml.x - M_use);
        L = __builtin_fmaf(ml.y, f, L);
        A += *reinterpret_cast<const floatx4 *>(a.po + prow * kHeadDim + c4) * f;
    }
    const float inv = 1.0f / L;
    uint16_t * o = a.out + (int64_t(t) * a.hq + int64_t(kvh) * a.G + r % a.G) * kHeadDim + c4;
    uint2 pk;
    pk.x = uint32_t(__half_as_ushort(__float2half_rn(A[0] * inv))) |
           (uint32_t(__half_as_ushort(__float2half_rn(A[1] * inv))) << 16);
    pk.y = uint32_t(__half_as_ushort(__float2half_rn(A[2] * inv))) |
           (uint32_t(__half_as_ushort(__float2half_rn(A[3] * inv))) << 16);
    *reinterpret_cast<uint2 *>(o) = pk;
}

// The launch shape: row blocks of kPfRows rows, and the key split that fills the device (a split keeps at least 16
// tiles); the workspace the splits' partials need (0 for one split).
struct pf_plan {
    int32_t row_blocks = 0, n_split = 1, split_tiles = 0, rows_pad = 0;
    int64_t ws_bytes = 0;
};
pf_plan plan_prefill(const kv_pool & p, int64_t ctx, int32_t rows, int32_t G) {
    pf_plan pl;
    const int32_t tok_per_wg = kPfRows / G;
    pl.row_blocks = (rows + tok_per_wg - 1) / tok_per_wg;
    pl.rows_pad = pl.row_blocks * kPfRows;
    const int32_t max_tiles = static_cast<int32_t>((ctx + kTileTokens - 1) / kTileTokens);
    const int32_t base = pl.row_blocks * p.h_kv();
    const int32_t cus = device_cus(p.device());
    int32_t ns = (cus + base - 1) / base;
    ns = std::min(ns, std::max(1, max_tiles / 16));
    // a split's pages fit the kernel's LDS copy of the table
    ns = std::max(ns, (max_tiles + kPfPages * kTilesPerPage - kTilesPerPage - 1) / (kPfPages * kTilesPerPage - kTilesPerPage));
    ns = std::min(ns, 64);
    pl.n_split = std::max(1, ns);
    pl.split_tiles = (max_tiles + pl.n_split - 1) / pl.n_split;
    if (pl.n_split > 1) {
        pl.ws_bytes = int64_t(pl.n_split) * p.h_kv() * pl.rows_pad * (kHeadDim + 2) * 4;
    }
    return pl;
}

} // namespace fnkv

using fnkv::set_error;

extern "C" {

int64_t fnkv_prefill_workspace_bytes(const fnkv_pool * pool, int64_t ctx, int32_t rows, int32_t hq) {
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    if (p == nullptr || rows <= 0 || ctx < rows || hq <= 0 || hq % p->h_kv() != 0 ||
        fnkv::kPfRows % (hq / p->h_kv()) != 0) {
        return -1;
    }
    return fnkv::plan_prefill(*p, ctx, rows, hq / p->h_kv()).ws_bytes;
}

int fnkv_attn_prefill(const fnkv_pool * pool, int32_t slot, int32_t layer, int64_t ctx, int32_t rows, int32_t hq,
                      float scale, const void * q, void * out, void * ws, int64_t ws_bytes, void * stream) {
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    if (p == nullptr || slot < 0 || slot >= p->pages().n_slots() || layer < 0 || layer >= p->layers() || rows <= 0 ||
        ctx < rows || ctx > p->mapped_cells(slot) || hq <= 0 || hq % p->h_kv() != 0 || q == nullptr ||
        out == nullptr || !(scale > 0.0f) || !std::isfinite(scale)) {
        set_error("fnkv_attn_prefill: argument outside the contract");
        return FNKV_ERR_ARG;
    }
    const int32_t G = hq / p->h_kv();
    if (fnkv::kPfRows % G != 0) {
        set_error("fnkv_attn_prefill: the GQA group must divide 256");
        return FNKV_ERR_ARG;
    }
    if ((reinterpret_cast<uintptr_t>(q) & 15) != 0 || (reinterpret_cast<uintptr_t>(out) & 7) != 0) {
        set_error("fnkv_attn_prefill: q must be 16-byte and out 8-byte aligned");
        return FNKV_ERR_ARG;
    }
    fnkv::pf_args a;
    a.pv = p->view();
    a.q = static_cast<const uint16_t *>(q);
    a.out = static_cast<uint16_t *>(out);
    a.c2 = scale * 1.4426950408889634f;
    a.ctx = ctx;
    a.rows = rows;
    a.G = G;
    a.hq = hq;
    a.layer = layer;
    a.slot = slot;
    fnkv::pf_plan pl = fnkv::plan_prefill(*p, ctx, rows, G);
    if (pl.n_split > 1 && (ws == nullptr || ws_bytes < pl.ws_bytes || (reinterpret_cast<uintptr_t>(ws) & 15) != 0)) {
        // no (or too small a) workspace: one split, written directly
        pl.n_split = 1;
        pl.split_tiles = static_cast<int32_t>((ctx + fnkv::kTileTokens - 1) / fnkv::kTileTokens);
    }
    a.n_split = pl.n_split;
    a.split_tiles = pl.split_tiles;
#ifdef FNKV_TIMING
    a.ts = fnkv::timing_buffer();
#endif
    a.po = static_cast<float *>(ws);
    a.pml = a.po == nullptr ? nullptr : a.po + int64_t(pl.n_split) * p->h_kv() * pl.rows_pad * fnkv::kHeadDim;
    static std::once_flag attr_once[64]; // once per device; a racing first caller waits for it
    const int32_t dev = p->device();
    if (dev >= 0 && dev < 64) {
        std::call_once(attr_once[dev], [dev]() {
            int32_t cur = 0;
            (void)hipGetDevice(&cur);
            (void)hipSetDevice(dev);
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(fnkv::prefill_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, fnkv::kPfLds);
            (void)hipGetLastError();
            (void)hipSetDevice(cur);
        });
    }
    const dim3 grid(static_cast<uint32_t>(pl.row_blocks), static_cast<uint32_t>(p->h_kv()),
                    static_cast<uint32_t>(pl.n_split));
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(fnkv::prefill_kernel, grid, dim3(64 * fnkv::kPfWaves), fnkv::kPfLds, st, a);
    if (pl.n_split > 1) {
        const int64_t items = int64_t(p->h_kv()) * pl.rows_pad;
        hipLaunchKernelGGL(fnkv::prefill_merge_kernel, dim3(static_cast<uint32_t>((items + 3) / 4)), dim3(256), 0, st,
                           a, pl.rows_pad);
    }
    if (hipGetLastError() != hipSuccess) {
        set_error("fnkv_attn_prefill: launch failed");
        return FNKV_ERR_HIP;
    }
    return FNKV_OK;
}

} // extern "C"
