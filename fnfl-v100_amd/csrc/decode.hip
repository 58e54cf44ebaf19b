// Decode and speculative-verify attention over the Q8_0 page pool (T = 1 .. 6 query tokens a sequence), split-K
// over pages with a log-sum-exp merge: the dense launches' host side (fnkv_attn_decode, _dev, _noalloc; their kernel
// is stream.hip's), the kernels of the sparse launches over selection bodies (sparse.hip, qsa.hip, qsp.hip run them),
// and the split merge of both.
//
// What it computes (the reference's decode attention, fn/kernels/qsa/attend.h:8-34; dense: causal over the whole
// context, on BASELINE's Q8_0 format): for query row (t, head h) of a sequence holding ctx cells,
//   o = sum_c softmax_c(q . k_c * scale) v_c over cells c <= ctx - T + t (sparse: over the row's selected cells),
// with k_c, v_c the decoded Q8_0 values (code * fp32(d)); scores, softmax statistics and accumulators in fp32; fp16
// out. The split-K partials (m, l, acc) fold in a fixed order as the reference's finish does (attend.cu:621-655):
// M = max m_j, L = sum l_j e^(m_j - M), A = sum acc_j e^(m_j - M), o = A / L.
//
// How the sparse kernels run (MI355X): a workgroup owns one (row, KV head, split of the row's selected tiles).
//   * A tile (32 tokens, 17,408 B: K and V codes, K and V scales) arrives as fully coalesced 1 KiB chunks: the K
//     codes and the scales straight into LDS (global_load_lds / buffer loads to LDS), the V codes into registers.
//   * The tile layout (layout.h) puts each lane's 16 B exactly where v_mfma_f32_16x16x32_f16 wants its operand: one
//     byte permute makes two codes the fp16 values 1152 + code (exact), and one MFMA a tile half takes the 1152 bias
//     back out (against the K scales and the rows' q sums for S, against the V scales and P for O).
//   * S^T = K Q^T one Q8_0 block (32 values) per MFMA; the block's scale folds in with one FMA per score. The G query
//     heads sharing the KV head are the MFMA's 16-wide column side (rows padded to 16 n).
//   * Online softmax in the base-2 domain on the S^T registers (a column's 4 lanes reduce with two lane swaps); P
//     lands as the B operand of O^T = V^T P^T without moving: each PV MFMA covers 16 values of one block, whose V
//     scale multiplies P once per block; the product goes to the matrix core as hi + lo fp16 (two MFMAs), which
//     keeps it to ~2^-22 relative where a single fp16 operand would err by 2^-11.
//   * Row tiles: decode_kernel<1> (up to 16 heads) runs eight independent tile streams, one a wave;
//     decode_rows_kernel<2> / <3> (up to 32 / 48) group two / three waves on one stream, each computing S and the
//     softmax of its row tile and PV of a share of the value blocks for all, P exchanged in LDS.
//   * The waves' partials merge in LDS; the workgroup writes (m, l, acc[256]) a row; merge_kernel folds the splits.
// The kernels are templates over SP (sparse); only their sparse instantiations are built (the dense launches moved
// to stream.hip), so their SP = false branches are not compiled.
#include "../../include/fnkv.h"
#include "common.h"
#include "layout.h"
#include "mfma.h"
#include "q8_0.h"
#include "decode_common.h"
#include "rope.h"

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

namespace fnkv {

// The new cells when the sparse launch prepares its rows (fused_prep): row z's view (ctx = depth + z + 1) writes
// cell depth + c, for c in `cells` (bit c): K = the F32 RMS norm and IMROPE of kv_k's row c (and k_f32's row c when
// `own`: the cell is row z's own and this workgroup its owner), V = kv_v's row c, each in the pool's format. Several
// workgroups may write one cell (every one that reads its tile, so its own loads follow its own stores); they store
// the same bytes.
// sn, cs: the row's own position's rope angle (cell z's); own_x, own_g: cell z's k row and the k norm (the wave of
// job 2 z), or its v row (the wave of job 2 z + 1), loaded early
template <int WAVES>
__device__ __forceinline__ void append_cells_fused(const dec_args & a, const int32_t * table, int32_t kvh,
                                                   int64_t ctx, uint32_t cells, bool own, float sn, float cs,
                                                   float4 own_x, float4 own_g, int32_t wave, int32_t lane) {
    const int32_t z = static_cast<int32_t>(blockIdx.z);
    const int64_t depth = ctx - 1 - z;
    const pool_view & pv = a.pv;
    for (int32_t job = wave; job < 2 * (z + 1); job += WAVES) {
        const int32_t c = job >> 1, kv = job & 1;
        if (((cells >> c) & 1u) == 0) {
            continue;
        }
        const int64_t pos = depth + c;
        const int64_t src = (int64_t(c) * pv.h_kv + kvh) * kHeadDim;
        float x[4];
        if (kv == 0) {
            if (c == z) {
                norm_rope_apply(x, own_x, own_g, sn, cs, lane);
            } else {
                norm_rope(x, a.fp.kv_k + src, a.fp.k_norm, a.fp.pos, a.fp.rows, c, a.fp.theta_scale, lane);
            }
            if (own && c == z && a.fp.k_f32 != nullptr) {
                reinterpret_cast<float4 *>(a.fp.k_f32 + src)[lane] = make_float4(x[0], x[1], x[2], x[3]);
            }
        } else if (c == z) {
            x[0] = own_x.x;
            x[1] = own_x.y;
            x[2] = own_x.z;
            x[3] = own_x.w;
        } else {
            load4<true>(a.fp.kv_v + src, lane, x);
        }
        quantize_store_fmt(x, lane, tile_of(pv, table, a.layer, kvh, pos), static_cast<int32_t>(pos & 31), kv,
                           pv.format);
    }
    __syncthreads();
}

// A tile group is NT waves sharing one tile stream, wave r of the group computing row tile r (query rows 16 r ..
// 16 r + 15); a workgroup holds GR groups (8 waves for NT = 1 and 2, 6 for NT = 3: two waves a SIMD).
template <int NT> struct dec_shape {
    static constexpr int GR = NT == 1 ? 8 : NT == 2 ? 4 : 2;
    static constexpr int WAVES = NT * GR;
};


// A tile is 17 chunks of 1 KiB: 8 of K codes, 8 of V codes, 1 of scales. The K codes and the scale chunk stream into
// the group's LDS slot (wave r of a group of NT issuing chunks r, r + NT, ... of those 9); every wave loads the V
// codes straight into its registers, where they already sit in the PV operand's layout.

template <int NT, int C>
__device__ __forceinline__ void issue_chunk(const uint8_t * tile, uint8_t * kbuf, uint8_t * sslot, int32_t lane) {
    if (C < 8) {
        // four chunks share one base: the immediate offset moves both the global and the LDS address
        lds_load16<(C & 3) * 1024>(tile + kKCodes + (C >> 2) * 4096 + lane * 16, kbuf + (C >> 2) * 4096);
    } else {
        lds_load16<0>(tile + kKScales + lane * 16, sslot);
    }
}

template <int NT>
__device__ __forceinline__ void issue_k(const uint8_t * tile, uint8_t * kbuf, uint8_t * sslot, int32_t r,
                                        int32_t lane) {
    if (NT == 1) {
        issue_chunk<NT, 0>(tile, kbuf, sslot, lane);
        issue_chunk<NT, 1>(tile, kbuf, sslot, lane);
        issue_chunk<NT, 2>(tile, kbuf, sslot, lane);
        issue_chunk<NT, 3>(tile, kbuf, sslot, lane);
        issue_chunk<NT, 4>(tile, kbuf, sslot, lane);
        issue_chunk<NT, 5>(tile, kbuf, sslot, lane);
        issue_chunk<NT, 6>(tile, kbuf, sslot, lane);
        issue_chunk<NT, 7>(tile, kbuf, sslot, lane);
        issue_chunk<NT, 8>(tile, kbuf, sslot, lane);
    } else {
#pragma unroll
        for (int32_t i = 0; i < (9 + NT - 1) / NT; ++i) {
            const int32_t c = r + i * NT;
            if (c < 8) {
                lds_load16<0>(tile + kKCodes + c * 1024 + lane * 16, kbuf + c * 1024);
            } else if (c == 8) {
                lds_load16<0>(tile + kKScales + lane * 16, sslot);
            }
        }
    }
}

// wait until only this wave's share of a tile's K copy (issued after what we wait for) may be outstanding
template <int NT> __device__ __forceinline__ void wait_part_k(int32_t r) {
    if (NT == 1) {
        wait_vmcnt<9>();
    } else if (NT == 2) {
        if (r == 0) {
            wait_vmcnt<5>();
        } else {
            wait_vmcnt<4>();
        }
    } else {
        if (r == 2) {
            wait_vmcnt<2>();
        } else {
            wait_vmcnt<3>();
        }
    }
}

template <int NT> __device__ __forceinline__ void group_sync() {
    if (NT > 1) {
        barrier_keep_loads();
    }
}

// KV8 (the pool's format is FNFL's group-64 rule): a scale serves two 32-value blocks, so the score MFMAs of a group
// chain and P x (V scale) is formed once a group.
// QLO (sparse launches with a.q_lo): the scores take q as fp16 hi + lo, the low parts in LDS after the selection
// slice ([block][lane] 16 B, the region the one-row launch forms its query rows in).
template <int NT, bool SP, bool KV8 = false, bool QLO = false>
__global__ __launch_bounds__(64 * dec_shape<NT>::WAVES, 1) void decode_kernel(dec_args a_in) {
    static_assert(!QLO || (SP && NT == 1 && dec_shape<NT>::WAVES == kBlocks), "QLO: one row tile, a wave a block");
    constexpr int GR = dec_shape<NT>::GR;
    constexpr int WAVES = dec_shape<NT>::WAVES;
    const int32_t lane = static_cast<int32_t>(threadIdx.x) & 63;
    // the wave index is uniform in a wave; readfirstlane tells the compiler so (scalar registers, no waterfall loops)
    const int32_t wave = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(threadIdx.x) >> 6);
    const int32_t kvh = static_cast<int32_t>(blockIdx.y);
    // A launch that prepares its row: the row's inputs are loaded first, before the row view's dependent reads of the
    // depth word and the selection offsets, so their latencies overlap. Wave w takes the KV head's query heads w and
    // w + 8 (a head past G loads head G - 1 and is not used); the row's own cell's inputs are loaded by every wave
    // (the K row or, for the wave of its V job, the V row) and used by the two waves whose jobs they are.
    // (unset without a prepare: an arbitrary value, never read, so no zeroing waits on the loads of the other path)
    float4 xq[2], gq, own_x, own_g;
    int32_t pq;
    {
        const float u = __builtin_nondeterministic_value(0.0f);
        xq[0] = xq[1] = gq = own_x = own_g = make_float4(u, u, u, u);
        pq = __builtin_nondeterministic_value(0);
    }
    if constexpr (SP) {
        if (a_in.fp.qfull != nullptr) {
            const int32_t zc = static_cast<int32_t>(blockIdx.z);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int32_t h = wave + 8 * i < a_in.G ? wave + 8 * i : a_in.G - 1;
                xq[i] = reinterpret_cast<const float4 *>(
                    a_in.fp.qfull + (int64_t(zc) * a_in.hq + kvh * a_in.G + h) * 512)[lane];
            }
            gq = reinterpret_cast<const float4 *>(a_in.fp.q_norm)[lane];
            pq = rope_pos(a_in.fp.pos, a_in.fp.rows, zc, lane);
            const int64_t crow = (int64_t(zc) * a_in.pv.h_kv + kvh) * kHeadDim;
            own_x = reinterpret_cast<const float4 *>((wave == (2 * zc + 1) % WAVES ? a_in.fp.kv_v : a_in.fp.kv_k) +
                                                     crow)[lane];
            own_g = reinterpret_cast<const float4 *>(a_in.fp.k_norm)[lane];
        }
    }
    const dec_args a = SP ? sparse_row_view(a_in) : a_in;
    if constexpr (SP) {
        if (sparse_refused(a)) {
            return;
        }
        FNKV_STAMP(8); // the wave stamps (8..) are not taken in sparse launches
    }
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int32_t grp = wave / NT, rt = wave % NT; // tile group and row tile
    const int32_t j = lane & 15, qg = lane >> 4;
    const int32_t split = static_cast<int32_t>(blockIdx.x);
    const int32_t s = SP ? 0 : seq_of(a, split); // a sparse launch is one sequence (constant: no scratch copy of a)
    const int32_t sp = split - a.split0[s];
    const int64_t ctx = seq_ctx<SP>(a, s);
    const int64_t begin = int64_t(sp) * a.split_tokens;
    const int64_t end = ctx < begin + a.split_tokens ? ctx : begin + a.split_tokens;
    const pool_view & pv = a.pv;
    const int32_t * table = pv.table + int64_t(a.slot[s]) * pv.table_stride;
    // the split's tiles (at most 64), lane i holding tile i's page: a tile's page is then a lane read, not a memory
    // load on the path to its copy. Loaded first: the page table, the Q rows and the first tile are then one memory
    // latency each but overlapped, not three in a row.
    half8 qop[kBlocks];
    int64_t lim;
    if constexpr (SP) { // the Q rows' latency hidden behind the selection's build
        if (a.fp.qfull == nullptr) {
            load_q_operands(a, s, ctx, kvh, rt, j, qg, qop, lim);
        }
    }
    // QLO: thread c loads the low part of operand (block c / 64, lane c % 64); stored to LDS after the build
    u32x4 qlo_ld = {0, 0, 0, 0};
    if constexpr (QLO) {
        if (a.fp.qfull == nullptr) {
            const int32_t L = static_cast<int32_t>(threadIdx.x) & 63, b = static_cast<int32_t>(threadIdx.x) >> 6;
            const int32_t row = L & 15;
            if (row < a.R) {
                const int32_t t_row = row / a.G;
                qlo_ld = *reinterpret_cast<const u32x4 *>(
                    a.q_lo + ((int64_t(s) * a.T + t_row) * a.hq + int64_t(kvh) * a.G + row % a.G) * kHeadDim +
                    b * kQK + 8 * (L >> 4));
            }
        }
    }
    split_src<SP> src;
    // a launch that prepares its row: the row's rope angle while the selection's loads are in flight
    float sn = 0.0f, cs = 0.0f;
    src.template init<64 * WAVES>(a, table, split, begin, end, lane, smem, smem + GR * kGroupLds, ctx, [&] {
        if (SP && a.fp.qfull != nullptr) {
            int32_t p = pq;
            __asm__ volatile("" : "+v"(p)); // the position's load is waited for here, not where it was issued
            rope_angle(sn, cs, p, a.fp.theta_scale, lane);
        }
    });
    if (refused<SP>(a, s, ctx, sp, kvh)) {
        return;
    }
    bool unmapped = false;
    if constexpr (!SP) {
        unmapped = src.guard_unmapped(lane);
        report_unmapped(a, unmapped);
    }
    const int32_t n_tiles = src.n_tiles;
    if (SP && n_tiles == 0) {
        return; // past the selection's tiles (the merge reads only the splits that hold some)
    }
    FNKV_STAMP(0);

    if constexpr (SP) {
        if (a.fp.qfull != nullptr) {
            // the KV head's query rows as fp16 in LDS (after the tile buffers and the selection slice), then each
            // lane's operands from there; split 0 also writes the F32 rows
            uint16_t * ql = reinterpret_cast<uint16_t *>(smem + GR * kGroupLds + kSelSlice);
            uint2 lo_pk[2] = {make_uint2(0, 0), make_uint2(0, 0)}; // QLO: fp16(y - hi), heads >= G zero
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int32_t h = wave + 8 * i;
                if (h < a.G) {
                    float y[4];
                    norm_rope_apply(y, xq[i], gq, sn, cs, lane);
                    reinterpret_cast<uint2 *>(ql + h * kHeadDim)[lane] = pack4_f16(y, 1.0f);
                    if constexpr (QLO) {
                        float lo[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            lo[e] = y[e] - static_cast<float>(static_cast<_Float16>(y[e]));
                        }
                        lo_pk[i] = pack4_f16(lo, 1.0f);
                    }
                    if (split == 0 && a.fp.q_f32 != nullptr) {
                        reinterpret_cast<float4 *>(
                            a.fp.q_f32 + (int64_t(blockIdx.z) * a.hq + kvh * a.G + h) * kHeadDim)[lane] =
                            make_float4(y[0], y[1], y[2], y[3]);
                    }
                }
            }
            barrier_keep_loads(); // the rows are in LDS (the F32 rows' stores need not have landed)
#pragma unroll
            for (int b = 0; b < kBlocks; ++b) {
                u32x4 v = {0, 0, 0, 0};
                if (j < a.G) {
                    v = *reinterpret_cast<const u32x4 *>(ql + j * kHeadDim + b * kQK + 8 * qg);
                }
                qop[b] = __builtin_bit_cast(half8, v);
            }
            if constexpr (QLO) {
                // the low parts fp16(y - hi) into the same region, as operands: value 4 lane + i of head h is
                // element 4 (lane & 1) + i of operand (block lane / 8, lane (h, (lane & 7) / 2)); heads >= G zero
                barrier_keep_loads(); // every operand read above
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int32_t h = wave + 8 * i;
                    *reinterpret_cast<uint2 *>(smem + GR * kGroupLds + kSelSlice +
                                               ((lane >> 3) * 64 + ((lane & 7) >> 1) * 16 + h) * 16 + (lane & 1) * 8) =
                        lo_pk[i];
                }
            }
            lim = ctx - 1;
            // the row's own cell when this split owns it, and every earlier row's cell whose tile this split reads
            uint32_t cells = static_cast<uint32_t>(src.new_mine & 1) << blockIdx.z;
            for (int32_t c = 0; c < static_cast<int32_t>(blockIdx.z); ++c) {
                const uint32_t tile_c = static_cast<uint32_t>((ctx - 1 - static_cast<int32_t>(blockIdx.z) + c) >> 5);
                const bool hit = lane < n_tiles && (src.ent_x & 0xffffu) == tile_c;
                cells |= __any(hit) ? (1u << c) : 0u;
            }
            append_cells_fused<WAVES>(a, table, kvh, ctx, cells, (src.new_mine & 1) != 0, sn, cs, own_x, own_g,
                                      wave, lane); // ends with a barrier
        } else {
            if constexpr (QLO) {
                *reinterpret_cast<u32x4 *>(smem + GR * kGroupLds + kSelSlice + threadIdx.x * 16) = qlo_ld;
            }
            append_owned_cells<WAVES>(a, table, kvh, ctx, src.new_mine, wave, lane);
            if constexpr (QLO) {
                __syncthreads();
            }
        }
    } else {
        append_new_cells<WAVES>(a, table, s, kvh, ctx, begin, end, src.g0, a.strided ? src.stride : 0, wave, lane);
    }
    FNKV_STAMP(1);
    if constexpr (!SP) {
        load_q_operands(a, s, ctx, kvh, rt, j, qg, qop, lim);
    }

    floatx4 acc[16];
    floatx4 lv = {0.0f, 0.0f, 0.0f, 0.0f}; // sum_t P[t][row] s_v[t][b]: lane (row j, qg) holds b = 4 qg + r
    float m_run = kNegInf, l_run = 0.0f;
#pragma unroll
    for (int m = 0; m < 16; ++m) {
        acc[m] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    // LDS addresses are formed as smem + offset (never through an array of pointers, which would turn the reads
    // into generic flat loads that wait on every outstanding global load)
    uint8_t * const gbase = smem + grp * kGroupLds;
    auto kbuf = [&](int32_t slot) -> uint8_t * { return gbase + slot * 8192; };
    auto sslot = [&](int32_t slot) -> uint8_t * { return gbase + kCodeBytes + slot * kScaleBytes; };
    const uint8_t * layer_base = pv.base + int64_t(a.layer) * pv.layer_stride + int64_t(kvh) * kPageBlock;
    auto tile_ptr = [&](int32_t ti) -> const uint8_t * { return layer_base + src.tile_off(pv, ti); };
    const int32_t t_row = t_of_row(a, rt, j);
    u32x4 vreg[8];
    auto vload = [&](const uint8_t * tile) {
        // after every earlier instruction that touches memory: the V loads stay younger than the K copy issued
        // before them, which the vmcnt waits below count on
        __asm__ __volatile__("" ::: "memory");
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            // one row tile: read once, streamed past the caches; several: the group's other waves read the same
            // bytes right after, so they stay cacheable (cfg2v: 310 against 336 MB of HBM reads a launch)
            if constexpr (NT == 1) {
                vreg[i] = stream_load16(tile + kVCodes + i * 1024 + lane * 16);
            } else {
                vreg[i] = *reinterpret_cast<const u32x4 *>(tile + kVCodes + i * 1024 + lane * 16);
            }
        }
    };
    const half8 zero8 = {};

    // One tile of the group's stream per iteration. Tile k's K codes and scales were copied into LDS slot k % 2
    // during iteration k - 1, its V codes loaded into this wave's registers at the end of iteration k - 1; tile
    // k + 1's K half starts into the other slot as soon as tile k's has landed, its V codes once PV(k) has read
    // tile k's.
    // Every iteration issues the same loads on every path (a group past its last tile re-reads its last tile, an L2
    // hit), so the vmcnt counts below, and the compiler's own, are exact rather than a path-merge's zero.
    const int32_t n_iter = (((n_tiles + GR - 1) / GR) + 1) & ~1;
    const int32_t last_tile = n_tiles - 1;
    FNKV_STAMP(2);
    {
        const uint8_t * t0p = tile_ptr(grp < last_tile ? grp : last_tile);
        issue_k<NT>(t0p, kbuf(0), sslot(0), rt, lane);
        vload(t0p);
    }
    const uint8_t * const qlo_base = smem + GR * kGroupLds + kSelSlice;
    auto qlo_lds = [&](int b) { return *reinterpret_cast<const half8 *>(qlo_base + (b * 64 + lane) * 16); };
    half8 sig = {}; // QLO: the codes enter exactly, no bias operand
    if constexpr (!QLO) {
        sig = q_sums(qop, qg);
    }
    FNKV_PHASE_DECL();
    for (int32_t it = 0; it < n_iter; ++it) {
        FNKV_PHASE(0 + (it > 0 ? 7 : 0));
        const int32_t ti = grp + it * GR;
        const bool have = ti < n_tiles;
        const int32_t tn = ti + GR < last_tile ? ti + GR : last_tile;
        const uint8_t * next_ptr = tile_ptr(tn);
        wait_vmcnt<8>(); // tile k's K half has landed (only its 8 V loads may be younger)
        FNKV_PHASE(1);
        group_sync<NT>(); // ... for every wave of the group; tile k - 1's slot is no longer read
        FNKV_PHASE(2);
        issue_k<NT>(next_ptr, kbuf((it + 1) & 1), sslot((it + 1) & 1), rt, lane);
        if (have) {
        const uint8_t * kb = kbuf(it & 1);
        const uint8_t * sc_tile = sslot(it & 1) - kKScales; // scale offsets are tile-relative
        const int64_t tok0 = src.tok0(ti);

        floatx4 sc[2];
        if constexpr (QLO) {
            tile_scores<KV8>(kb, sc_tile, [&](int b) { return qop[b]; }, sig, j, qg, lane, sc, qlo_lds);
        } else {
            tile_scores<KV8>(kb, sc_tile, [&](int b) { return qop[b]; }, sig, j, qg, lane, sc);
        }

        FNKV_PHASE(3);
        // ---- online softmax (base 2); P stays in the registers that feed the PV MFMA ----
        const int64_t lim_rel64 = lim - tok0;
        const int32_t lim_rel = lim_rel64 > 64 ? 64 : static_cast<int32_t>(lim_rel64 < -1 ? -1 : lim_rel64);
        float pf[8];
        {
            float alpha;
            tile_softmax<QLO>(sc, lim_rel, a.c2, qg, m_run, l_run, pf, alpha, src.vis(ti, t_row, qg));
            if (__any(alpha != 1.0f)) {
#pragma unroll
                for (int m = 0; m < 16; ++m) {
                    acc[m] *= alpha;
                }
                lv *= alpha;
            }
        }

        FNKV_PHASE(4);
        wait_part_k<NT>(rt); // tile k's V codes (tile k + 1's K copy is younger)
        FNKV_PHASE(5);
        // ---- O^T += V^T P^T: MFMA tile m covers values 16 m .. 16 m + 15 of block m / 2 ----
        // P times the block's V scale goes to the matrix core as hi + lo fp16 (fp16 alone would leave a 2^-11
        // relative error per term, too coarse when a few large cells dominate). The V codes enter as 1152 + code;
        // lv accumulates sum_t P s_v per block (one MFMA pair a tile) so the bias comes out once, at the end.
        const half8 pfh = to_half8_rtz(pf);
        half8 pfl;
        {
            float r8[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                r8[i] = pf[i] - static_cast<float>(pfh[i]);
            }
            pfl = to_half8_rtz(r8);
        }
        if constexpr (!QLO) { // QLO: the codes enter exactly (the bias would amplify lo's rounding 1152 / |code|-fold)
            // A: lane (block b = j, qg) holds s_v[token(qg, s)][b] for its 8 slots s (zero for b >= 8)
            const half8 sva = j < 8 ? *reinterpret_cast<const half8 *>(sc_tile + kVScales + qg * 128 + j * 16) : zero8;
            lv = mfma16(sva, pfh, lv);
            lv = mfma16(sva, pfl, lv);
        }
        half8 ph, pl;
#pragma unroll
        for (int ld = 0; ld < 8; ++ld) {
            if (!KV8 || (ld & 1) == 0) { // KV8: block ld + 1 shares block ld's scale
                const half8 vs = *reinterpret_cast<const half8 *>(sc_tile + kVScales + qg * 128 + ld * 16);
                scale_hilo<QLO>(pf, pfh, vs, ph, pl);
            }
            const half8 va0 = widen8<QLO>(vreg[ld][0], vreg[ld][1]);
            const half8 va1 = widen8<QLO>(vreg[ld][2], vreg[ld][3]);
            acc[2 * ld] = mfma16(va0, ph, acc[2 * ld]);
            acc[2 * ld + 1] = mfma16(va1, ph, acc[2 * ld + 1]);
            acc[2 * ld] = mfma16(va0, pl, acc[2 * ld]);
            acc[2 * ld + 1] = mfma16(va1, pl, acc[2 * ld + 1]);
        }
        }
        FNKV_PHASE(6);
        vload(next_ptr);
    }
    FNKV_PHASE_STORE();
    wait_vmcnt<0>();
    FNKV_STAMP(3);
    FNKV_STAMP_WAVE();

    // the V bias: acc[m] carries 1152 * lv[b = m / 2]; lv[b] of this lane's row sits in lane (j, b / 4), element b % 4
    if constexpr (!QLO) {
        float lb[kBlocks];
#pragma unroll
        for (int b = 0; b < kBlocks; ++b) {
            lb[b] = __shfl(lv[b & 3], j + 16 * (b >> 2));
        }
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            acc[m] -= 1152.0f * lb[m >> 1];
        }
    }

    // ---- merge the groups per row tile in LDS, write the workgroup's partial ----
    l_run = rows_sum(l_run);
    constexpr int32_t kOStride = kHeadDim + 4;
    __syncthreads(); // the tile buffers are no longer read
    FNKV_STAMP(5);
    float * ml = reinterpret_cast<float *>(smem);                        // [waves][16 rows][2]
    float * ob = reinterpret_cast<float *>(smem + WAVES * 16 * 2 * 4);   // [waves][16 rows][kOStride]
    if (qg == 0) {
        ml[(wave * 16 + j) * 2 + 0] = m_run;
        ml[(wave * 16 + j) * 2 + 1] = l_run;
    }
    __syncthreads();
    {
        float M = kNegInf;
#pragma unroll
        for (int g = 0; g < GR; ++g) {
            M = fmaxf(M, ml[((g * NT + rt) * 16 + j) * 2]);
        }
        const float f = __builtin_amdgcn_exp2f(m_run - (M == kNegInf ? 0.0f : M));
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            *reinterpret_cast<floatx4 *>(ob + (wave * 16 + j) * kOStride + 16 * m + 4 * qg) = acc[m] * f;
        }
    }
    __syncthreads();
    FNKV_STAMP(6);
    // thread -> (row tile, row, 16 values): NT * 16 rows x 256 values over the workgroup's threads
    for (int32_t item = static_cast<int32_t>(threadIdx.x); item < NT * 16 * 16; item += 64 * WAVES) {
        const int32_t rtile = item / 256, rrow = (item / 16) % 16, c0 = (item % 16) * 16;
        const int32_t r = rtile * 16 + rrow;
        if (r >= a.R) {
            continue;
        }
        const int64_t prow = (int64_t(split) * pv.h_kv + kvh) * a.R + r;
        float * dst = a.po + prow * kHeadDim + c0;
#pragma unroll
        for (int c = 0; c < 16; c += 4) {
            floatx4 sum = *reinterpret_cast<const floatx4 *>(ob + ((0 * NT + rtile) * 16 + rrow) * kOStride + c0 + c);
#pragma unroll
            for (int g = 1; g < GR; ++g) {
                sum += *reinterpret_cast<const floatx4 *>(ob + ((g * NT + rtile) * 16 + rrow) * kOStride + c0 + c);
            }
            *reinterpret_cast<floatx4 *>(dst + c) = sum;
        }
        if ((item & 15) == 0) {
            float Mr = kNegInf;
#pragma unroll
            for (int g = 0; g < GR; ++g) {
                Mr = fmaxf(Mr, ml[((g * NT + rtile) * 16 + rrow) * 2]);
            }
            const float Mr_use = Mr == kNegInf ? 0.0f : Mr;
            float L = 0.0f;
#pragma unroll
            for (int g = 0; g < GR; ++g) {
                const int32_t w = g * NT + rtile;
                L += ml[(w * 16 + rrow) * 2 + 1] * __builtin_amdgcn_exp2f(ml[(w * 16 + rrow) * 2] - Mr_use);
            }
            a.pml[prow * 2 + 0] = unmapped ? __builtin_nanf("") : Mr; // NaN: the merge writes nothing
            a.pml[prow * 2 + 1] = L;
        }
    }
    FNKV_STAMP(4);
}

// ---- G T > 16 rows: a group of NT waves shares each tile; rows split for QK, value blocks split for PV ----
//
// Wave w of a group computes S^T and the online softmax of query row tile w (rows 16 w .. 16 w + 15) from the
// group's K copy in LDS, and hands its P (as fp16 hi + lo, the PV operand) and the per-row rescale factor to the
// group's other waves through LDS. Then every wave accumulates O^T for ALL the group's row tiles over its own share
// of the value blocks (NT = 2: 4 blocks each; NT = 3: 3, 3, 2), from V codes it loaded into its registers: each V byte
// is loaded once, widened once, and a wave's accumulators stay at 64 - 72 registers. K streams through a ring of SK
// LDS slots (SK - 1 tiles ahead), V through two register buffers (two tiles ahead); the loop is unrolled by two so
// the buffers are fixed registers. The Q operands stay in registers at NT = 2 and sit once in LDS at NT = 3. The
// groups of the second half run half an iteration behind the first (see the loop), so the two waves sharing a SIMD
// are in different phases.
// (two groups a workgroup at NT = 2, two workgroups a CU, measured slower when this kernel served dense launches)
#ifndef FNKV_QK_PRIO
#define FNKV_QK_PRIO 1
#endif
constexpr int16_t kQkPrio = FNKV_QK_PRIO; // wave priority (s_setprio) of the scores + softmax phase
template <int NT, bool SP = false, bool QLO = false> struct rows_shape {
    static constexpr int GR = NT == 2 ? 4 : 2;                      // tile groups a workgroup
    static constexpr int WAVES = NT * GR;
    static constexpr int SK = NT == 2 ? 3 : QLO ? 4 : 6;            // K ring slots a group (QLO: room for q's lo)
    static constexpr int NBM = (kBlocks + NT - 1) / NT;             // value blocks a wave (the last may own fewer)
    static constexpr int CK = (9 + NT - 1) / NT;                    // 1 KiB K chunks a wave issues a tile
    static constexpr int KSLOT = kCodeBytes / 2 + kScaleBytes;      // K codes, then the tile's K and V scales
    static constexpr int PX = 2 * NT * 64 * 32;                     // P: [parity][row tile][lane] ph, pl
    static constexpr int AX = 2 * NT * 16 * 4;                      // rescale factors: [parity][row tile][row]
    static constexpr int GROUP_LDS = SK * KSLOT + PX + AX;
    static constexpr int Q_LDS = NT == 2 ? 0 : NT * kBlocks * 64 * 16; // Q operands (NT = 3), shared by the groups
    static constexpr int QLO_LDS = QLO ? NT * kBlocks * 64 * 16 : 0;    // q's low parts (QLO), after them
    // loads a wave has issued after tile k's K chunks when it waits for them (top of iteration k), and after tile
    // k's V codes when it waits for those (before PV of iteration k)
    static constexpr int WAIT_K = NBM + (SK - 2) * (CK + NBM);
    static constexpr int WAIT_V = 2 * CK + NBM;
};

template <int NT, bool SP, bool KV8 = false, bool QLO = false>
__global__ __launch_bounds__((64 * rows_shape<NT, SP, QLO>::WAVES), 1) void decode_rows_kernel(dec_args a_in) {
    static_assert(!QLO || SP, "QLO: sparse launches");
    const dec_args a = SP ? sparse_row_view(a_in) : a_in;
    if constexpr (SP) {
        if (sparse_refused(a)) {
            return;
        }
    }
    using SH = rows_shape<NT, SP, QLO>;
    constexpr int GR = SH::GR, WAVES = SH::WAVES, SK = SH::SK, NBM = SH::NBM, CK = SH::CK;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int32_t lane = static_cast<int32_t>(threadIdx.x) & 63;
    // the wave index is uniform in a wave; readfirstlane tells the compiler so (scalar registers, no waterfall loops)
    const int32_t wave = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(threadIdx.x) >> 6);
    const int32_t grp = wave / NT, w = wave % NT; // tile group; this wave's row tile and block share
    const int32_t j = lane & 15, qg = lane >> 4;
    const int32_t split = static_cast<int32_t>(blockIdx.x);
    const int32_t kvh = static_cast<int32_t>(blockIdx.y);
    const int32_t s = SP ? 0 : seq_of(a, split); // a sparse launch is one sequence (constant: no scratch copy of a)
    const int32_t sp = split - a.split0[s];
    const int64_t ctx = seq_ctx<SP>(a, s);
    const int64_t begin = int64_t(sp) * a.split_tokens;
    const int64_t end = ctx < begin + a.split_tokens ? ctx : begin + a.split_tokens;
    const pool_view & pv = a.pv;
    const int32_t * table = pv.table + int64_t(a.slot[s]) * pv.table_stride;
    // the split's tiles, lane i holding tile i's page, loaded first (with the Q rows below, and the first tiles
    // issued before the Q sums wait: overlapped latencies, not three in a row)
    if constexpr (SP) {
        FNKV_STAMP(6);
    }
    half8 sig; // set once the first tiles are issued
    int64_t lim;
    // the Q operands: in registers at NT = 2; at NT = 3 registers are short and they sit once in LDS (after the
    // groups' buffers), the same for every group
    constexpr bool kQReg = NT == 2;
    half8 qreg[kBlocks];
    if constexpr (SP) { // the Q rows' latency hidden behind the selection's build
        load_q_operands(a, s, ctx, kvh, w, j, qg, qreg, lim);
    }
    // QLO: the workgroup loads q's low parts as operands ([row tile][block][lane] 16 B), chunk c = thread + i WAVES 64
    constexpr int QLO_PER = QLO ? NT * kBlocks * 64 / (64 * WAVES) : 1;
    static_assert(!QLO || QLO_PER * 64 * WAVES == NT * kBlocks * 64, "QLO: whole chunks a thread");
    u32x4 qlo_ld[QLO_PER];
    if constexpr (QLO) {
#pragma unroll
        for (int i = 0; i < QLO_PER; ++i) {
            const int32_t c = static_cast<int32_t>(threadIdx.x) + i * 64 * WAVES;
            const int32_t L = c & 63, b = (c >> 6) % kBlocks, row = (c >> 9) * 16 + (L & 15);
            qlo_ld[i] = u32x4{0, 0, 0, 0};
            if (row < a.R) {
                qlo_ld[i] = *reinterpret_cast<const u32x4 *>(
                    a.q_lo + ((int64_t(s) * a.T + row / a.G) * a.hq + int64_t(kvh) * a.G + row % a.G) * kHeadDim +
                    b * kQK + 8 * (L >> 4));
            }
        }
    }
    split_src<SP, NT == 2> src; // NT = 3 is short of registers: its entries stay in LDS
    src.template init<64 * WAVES>(a, table, split, begin, end, lane, smem,
                                  smem + GR * SH::GROUP_LDS + SH::Q_LDS + SH::QLO_LDS, ctx);
    if (refused<SP>(a, s, ctx, sp, kvh)) {
        return;
    }
    bool unmapped = false;
    if constexpr (!SP) {
        unmapped = src.guard_unmapped(lane);
        report_unmapped(a, unmapped);
    }
    const int32_t n_tiles = src.n_tiles;
    if (SP && n_tiles == 0) {
        return; // past the selection's tiles (the merge reads only the splits that hold some)
    }
    FNKV_STAMP(0);
    if constexpr (SP) {
        append_owned_cells<WAVES>(a, table, kvh, ctx, src.new_mine, wave, lane);
    } else {
        append_new_cells<WAVES>(a, table, s, kvh, ctx, begin, end, src.g0, a.strided ? src.stride : 0, wave, lane);
    }
    FNKV_STAMP(1);

    uint8_t * const qlds = smem + GR * SH::GROUP_LDS; // [row tile][block][lane] 16 B
    uint8_t * const qlo_base = qlds + SH::Q_LDS;        // QLO: the same layout
    if constexpr (QLO) { // read after the loop's first barrier
#pragma unroll
        for (int i = 0; i < QLO_PER; ++i) {
            *reinterpret_cast<u32x4 *>(qlo_base + (threadIdx.x + i * 64 * WAVES) * 16) = qlo_ld[i];
        }
    }
    auto qlo_lds = [&](int b) {
        return *reinterpret_cast<const half8 *>(qlo_base + (w * kBlocks + b) * 1024 + lane * 16);
    };
    if constexpr (!SP) {
        load_q_operands(a, s, ctx, kvh, w, j, qg, qreg, lim);
    }
    auto qop_lds = [&](int b) {
        if constexpr (kQReg) {
            return qreg[b];
        } else {
            return *reinterpret_cast<const half8 *>(qlds + (w * kBlocks + b) * 1024 + lane * 16);
        }
    };

    const int32_t b0 = NT == 2 ? 4 * w : 3 * w; // this wave's value blocks b0 .. b0 + nb - 1
    const int32_t nb = NT == 2 ? 4 : (w < 2 ? 3 : 2);
    floatx4 acc[NT][NBM][2];
    floatx4 lv[NT];
#pragma unroll
    for (int rt = 0; rt < NT; ++rt) {
        lv[rt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < NBM; ++i) {
            acc[rt][i][0] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            acc[rt][i][1] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    float m_run = kNegInf, l_run = 0.0f; // row tile w

    // LDS of the group, addressed as smem + offset (never through arrays of pointers)
    const uint32_t gofs = static_cast<uint32_t>(grp * SH::GROUP_LDS);
    auto kslot = [&](int32_t slot) -> uint8_t * { return smem + gofs + slot * SH::KSLOT; };
    auto pslot = [&](int32_t par, int32_t rt) -> uint8_t * {
        return smem + gofs + SK * SH::KSLOT + (par * NT + rt) * 2048;
    };
    auto aslot = [&](int32_t par, int32_t rt) -> float * {
        return reinterpret_cast<float *>(smem + gofs + SK * SH::KSLOT + SH::PX + (par * NT + rt) * 64);
    };

    const uint8_t * layer_base = pv.base + int64_t(a.layer) * pv.layer_stride + int64_t(kvh) * kPageBlock;
    const int32_t last_tile = n_tiles - 1;
    auto tile_ptr = [&](int32_t k) -> const uint8_t * { // the group's tile of iteration k (the last tile past the end)
        int32_t ti = grp + k * GR;
        ti = ti < last_tile ? ti : last_tile;
        return layer_base + src.tile_off(pv, ti);
    };
    const int32_t t_row = t_of_row(a, w, j);
    const int32_t lane16 = lane * 16;
    // chunk c of a tile (c < 8: K codes, c = 8: the scales) into its place in a ring slot
    auto issue_chunk = [&](const uint8_t * tile, uint8_t * dst, int32_t c) {
        const rsrc_t r = make_rsrc(tile, kTileBytes);
        if (c < 8) {
            buf_lds16(r, dst + c * 1024, lane16, kKCodes + c * 1024);
        } else {
            buf_lds16(r, dst + kCodeBytes / 2, lane16, kKScales);
        }
    };
    // this wave's chunks c = w, w + NT, ... of a tile; past the ninth chunk it copies its first chunk again (the same
    // bytes to the same place), which keeps every wave's count at CK
    auto issue_k = [&](const uint8_t * tile, int32_t slot) {
        uint8_t * dst = kslot(slot);
#pragma unroll
        for (int32_t i = 0; i < CK; ++i) {
            const int32_t c = w + i * NT;
            issue_chunk(tile, dst, c <= 8 ? c : w);
        }
    };
    // the prologue's placeholders for V loads before tile 0: NBM more copies of this wave's first chunk of a tile
    // whose K copy it has just issued
    auto issue_placeholder = [&](const uint8_t * tile, int32_t slot) {
#pragma unroll
        for (int32_t i = 0; i < NBM; ++i) {
            issue_chunk(tile, kslot(slot), w);
        }
    };
    u32x4 vbuf0[NBM], vbuf1[NBM];
    auto load_v = [&](const uint8_t * tile, u32x4 (&vb)[NBM]) {
        __asm__ __volatile__("" ::: "memory"); // younger than every load issued before (the waits count on it)
        const rsrc_t r = make_rsrc(tile, kTileBytes);
#pragma unroll
        for (int32_t i = 0; i < NBM; ++i) {
            const int32_t b = b0 + i < kBlocks ? b0 + i : kBlocks - 1;
            vb[i] = buf_load16(r, lane16, kVCodes + b * 1024);
        }
        keep_issued(); // older than every load issued after
    };

    // The groups of the workgroup's second half run half an iteration behind the first half (their PV of tile
    // k - 1 falls between the barriers where the first half computes tile k's scores, and their scores of tile k
    // where the first half accumulates PV of tile k). Each SIMD holds one wave of each half, so the matrix-core
    // heavy PV of one overlaps the VALU-heavy scores and softmax of the other instead of both doing the same phase.
    // Every wave passes the same barriers: two an iteration, n_iter + 1 iterations.
    const int32_t n_iter = (((n_tiles + GR - 1) / GR) + 1) & ~1;
    const bool late = grp >= GR / 2;
    const half8 zero8 = {};
    FNKV_PHASE_DECL();

    // scores and softmax of tile k (row tile w) -> P and the rescale factor into the exchange buffers of parity PAR
    auto qk_phase = [&](auto par_c, int32_t k) {
        constexpr int32_t par = decltype(par_c)::value;
        if (grp + k * GR >= n_tiles) {
            return;
        }
        // the scores and softmax are the loop's longest dependent chain: their wave issues first on a shared SIMD
        __builtin_amdgcn_s_setprio(kQkPrio);
        const uint8_t * kb = kslot(k % SK);
        const uint8_t * sc_tile = kb + kCodeBytes / 2 - kKScales; // scale offsets are tile-relative
        const int64_t tok0 = src.tok0(grp + k * GR);
        floatx4 sc[2];
        if constexpr (QLO) {
            tile_scores<KV8>(kb, sc_tile, qop_lds, sig, j, qg, lane, sc, qlo_lds);
        } else {
            tile_scores<KV8>(kb, sc_tile, qop_lds, sig, j, qg, lane, sc);
        }
        const int64_t lim_rel64 = lim - tok0;
        const int32_t lim_rel = lim_rel64 > 64 ? 64 : static_cast<int32_t>(lim_rel64 < -1 ? -1 : lim_rel64);
        float pf[8];
        float alpha;
        tile_softmax<QLO>(sc, lim_rel, a.c2, qg, m_run, l_run, pf, alpha, src.vis(grp + k * GR, t_row, qg));
        half8 ph, pl;
        split_hilo(pf, ph, pl);
        u32x4 * px = reinterpret_cast<u32x4 *>(pslot(par, w) + lane * 32);
        px[0] = __builtin_bit_cast(u32x4, ph);
        px[1] = __builtin_bit_cast(u32x4, pl);
        if (qg == 0) {
            aslot(par, w)[j] = alpha;
        }
        __builtin_amdgcn_s_setprio(0);
    };
    // O^T += V^T P^T of tile k over this wave's value blocks, for every row tile, from the exchange buffers of
    // parity PAR and the V codes in vb
    auto pv_phase = [&](auto par_c, int32_t k, u32x4 (&vb)[NBM]) {
        constexpr int32_t par = decltype(par_c)::value;
        if (k < 0 || grp + k * GR >= n_tiles) {
            return;
        }
        wait_vmcnt<SH::WAIT_V>(); // tile k's V codes (the K copies and V codes issued after them may be pending)
        const uint8_t * sc_tile = kslot(k % SK) + kCodeBytes / 2 - kKScales;
        const half8 sva = j < 8 ? *reinterpret_cast<const half8 *>(sc_tile + kVScales + qg * 128 + j * 16) : zero8;
        half8 ph[NT], pl[NT];
#pragma unroll
        for (int32_t rt = 0; rt < NT; ++rt) {
            const u32x4 * px = reinterpret_cast<const u32x4 *>(pslot(par, rt) + lane * 32);
            ph[rt] = __builtin_bit_cast(half8, px[0]);
            pl[rt] = __builtin_bit_cast(half8, px[1]);
            const float alpha = aslot(par, rt)[j];
            if (__any(alpha != 1.0f)) {
#pragma unroll
                for (int32_t i = 0; i < NBM; ++i) {
                    acc[rt][i][0] *= alpha;
                    acc[rt][i][1] *= alpha;
                }
                lv[rt] *= alpha;
            }
            if constexpr (!QLO) { // QLO: the codes enter exactly
                lv[rt] = mfma16(sva, ph[rt], lv[rt]);
                lv[rt] = mfma16(sva, pl[rt], lv[rt]);
            }
        }
        half8 hi[NT], lo[NT];
#pragma unroll
        for (int32_t i = 0; i < NBM; ++i) {
            if (i < nb) {
                const half8 va0 = widen8<QLO>(vb[i][0], vb[i][1]);
                const half8 va1 = widen8<QLO>(vb[i][2], vb[i][3]);
                // KV8: an odd block shares the scale of the block before it (when this wave holds both)
                if (!KV8 || ((b0 + i) & 1) == 0 || i == 0) {
                    const half8 vs = *reinterpret_cast<const half8 *>(sc_tile + kVScales + qg * 128 + (b0 + i) * 16);
#pragma unroll
                    for (int32_t rt = 0; rt < NT; ++rt) {
                        scale_hilo_pk(ph[rt], pl[rt], vs, hi[rt], lo[rt]);
                    }
                }
                // the hi terms of every row tile, then the lo terms: dependent MFMAs 2 NT apart
#pragma unroll
                for (int32_t rt = 0; rt < NT; ++rt) {
                    acc[rt][i][0] = mfma16(va0, hi[rt], acc[rt][i][0]);
                    acc[rt][i][1] = mfma16(va1, hi[rt], acc[rt][i][1]);
                }
#pragma unroll
                for (int32_t rt = 0; rt < NT; ++rt) {
                    acc[rt][i][0] = mfma16(va0, lo[rt], acc[rt][i][0]);
                    acc[rt][i][1] = mfma16(va1, lo[rt], acc[rt][i][1]);
                }
            }
        }
    };

    // First half. Issue order, identical in the prologue and every iteration: K(k + SK - 1), then V(k + 2)
    // (k = -(SK - 1) .. -1 in the prologue, placeholders where k + 2 < 0). Iteration k: [wait K(k), barrier A,
    // issue K(k + SK - 1) into the slot of tile k - 1, scores of k] [barrier B, PV of k, issue V(k + 2)].
    auto early_iteration = [&](auto par_c, int32_t k, u32x4 (&vb)[NBM]) {
        FNKV_PHASE(0 + (k > 0 ? 7 : 0));
        wait_vmcnt<SH::WAIT_K>(); // this wave's chunks of tile k's K copy have landed
        FNKV_PHASE(1);
        barrier_keep_loads();     // ... every wave's; slot (k - 1) % SK and P buffers of k - 2 are free
        FNKV_PHASE(2);
        issue_k(tile_ptr(k + SK - 1), (k + SK - 1) % SK);
        qk_phase(par_c, k);
        FNKV_PHASE(3);
        barrier_keep_loads(); // every row tile's P and factors are in LDS
        FNKV_PHASE(4);
        pv_phase(par_c, k, vb);
        FNKV_PHASE(6);
        load_v(tile_ptr(k + 2), vb);
    };
    // Second half. Issue order: V(k + 1), then K(k + SK - 1) (prologue k = -(SK - 1) .. -1, placeholders where
    // k + 1 < 0). Iteration k: [barrier A, PV of k - 1, issue V(k + 1)] [wait K(k), barrier B, issue K(k + SK - 1)
    // into the slot of tile k - 1, scores of k].
    auto late_iteration = [&](auto par_c, int32_t k, u32x4 (&vb_prev)[NBM]) {
        constexpr int32_t par = decltype(par_c)::value;
        barrier_keep_loads(); // P of tile k - 1 is in LDS
        pv_phase(std::integral_constant<int32_t, 1 - par>(), k - 1, vb_prev);
        load_v(tile_ptr(k + 1), vb_prev);
        wait_vmcnt<SH::WAIT_K>(); // this wave's chunks of tile k's K copy have landed
        barrier_keep_loads();     // ... every wave's; PV of k - 1 no longer reads slot (k - 1) % SK
        issue_k(tile_ptr(k + SK - 1), (k + SK - 1) % SK);
        qk_phase(par_c, k);
    };

    // after the prologue's copies are issued: the bias operand from the Q rows, and at NT = 3 the Q operands into
    // LDS (group 0's waves; read after the loop's first barrier)
    auto q_finish = [&]() {
        if constexpr (!QLO) { // QLO: the codes enter exactly, no bias operand
            sig = q_sums(qreg, qg);
        }
        if constexpr (!kQReg) {
            if (grp == 0) {
#pragma unroll
                for (int b = 0; b < kBlocks; ++b) {
                    *reinterpret_cast<half8 *>(qlds + (w * kBlocks + b) * 1024 + lane * 16) = qreg[b];
                }
            }
        }
    };

    if (!late) {
#pragma unroll
        for (int32_t k = -(SK - 1); k < 0; ++k) {
            issue_k(tile_ptr(k + SK - 1), k + SK - 1);
            if (k + 2 == 0) {
                load_v(tile_ptr(0), vbuf0);
            } else if (k + 2 == 1) {
                load_v(tile_ptr(1), vbuf1);
            } else {
                issue_placeholder(tile_ptr(k + SK - 1), k + SK - 1);
            }
        }
        q_finish();
        FNKV_STAMP(2);
        for (int32_t k = 0; k < n_iter; k += 2) {
            early_iteration(std::integral_constant<int32_t, 0>(), k, vbuf0);
            early_iteration(std::integral_constant<int32_t, 1>(), k + 1, vbuf1);
        }
        early_iteration(std::integral_constant<int32_t, 0>(), n_iter, vbuf0); // past the end: barriers only
    } else {
#pragma unroll
        for (int32_t k = -(SK - 1); k < 0; ++k) {
            if (k + 1 == 0) {
                load_v(tile_ptr(0), vbuf0);
            } else {
                issue_placeholder(tile_ptr(k + SK - 1), k + SK - 1); // the copy issued just below
            }
            issue_k(tile_ptr(k + SK - 1), k + SK - 1);
        }
        q_finish();
        for (int32_t k = 0; k < n_iter; k += 2) {
            late_iteration(std::integral_constant<int32_t, 0>(), k, vbuf1);
            late_iteration(std::integral_constant<int32_t, 1>(), k + 1, vbuf0);
        }
        late_iteration(std::integral_constant<int32_t, 0>(), n_iter, vbuf1); // PV of the last tile
    }
    wait_vmcnt<0>();
    FNKV_PHASE_STORE();
    FNKV_STAMP(3);
    FNKV_STAMP_WAVE();

    // the V bias: acc[rt][i] carries 1152 * lv[rt][b0 + i]; lv[rt][b] of this lane's row sits in lane (j, b / 4),
    // element b % 4 (QLO: no bias, the codes entered exactly)
#pragma unroll
    for (int32_t rt = 0; rt < (QLO ? 0 : NT); ++rt) {
        float lb[kBlocks];
#pragma unroll
        for (int b = 0; b < kBlocks; ++b) {
            lb[b] = __shfl(lv[rt][b & 3], j + 16 * (b >> 2));
        }
#pragma unroll
        for (int32_t i = 0; i < NBM; ++i) {
            float l = lb[0];
#pragma unroll
            for (int b = 1; b < kBlocks; ++b) {
                l = b0 + i == b ? lb[b] : l;
            }
            acc[rt][i][0] -= 1152.0f * l;
            acc[rt][i][1] -= 1152.0f * l;
        }
    }

    // ---- merge the groups in LDS, write the workgroup's partial ----
    l_run = rows_sum(l_run);
    constexpr int32_t kRows = NT * 16;
    constexpr int32_t kOStride = kHeadDim + 4;
    __syncthreads(); // the ring and exchange buffers are no longer read
    float * ml = reinterpret_cast<float *>(smem);                     // [group][row][2]
    float * ob = reinterpret_cast<float *>(smem + GR * kRows * 2 * 4); // [group][row][kOStride]
    if (qg == 0) {
        ml[(grp * kRows + w * 16 + j) * 2 + 0] = m_run;
        ml[(grp * kRows + w * 16 + j) * 2 + 1] = l_run;
    }
    __syncthreads();
#pragma unroll
    for (int32_t rt = 0; rt < NT; ++rt) {
        float M = kNegInf;
#pragma unroll
        for (int g = 0; g < GR; ++g) {
            M = fmaxf(M, ml[(g * kRows + rt * 16 + j) * 2]);
        }
        const float f = __builtin_amdgcn_exp2f(ml[(grp * kRows + rt * 16 + j) * 2] - (M == kNegInf ? 0.0f : M));
        float * orow = ob + (grp * kRows + rt * 16 + j) * kOStride;
#pragma unroll
        for (int32_t i = 0; i < NBM; ++i) {
            if (i < nb) {
                *reinterpret_cast<floatx4 *>(orow + (b0 + i) * 32 + 4 * qg) = acc[rt][i][0] * f;
                *reinterpret_cast<floatx4 *>(orow + (b0 + i) * 32 + 16 + 4 * qg) = acc[rt][i][1] * f;
            }
        }
    }
    __syncthreads();
    // thread -> (row, 16 values): kRows x 256 values over the workgroup's threads
    for (int32_t item = static_cast<int32_t>(threadIdx.x); item < kRows * 16; item += 64 * WAVES) {
        const int32_t r = item / 16, c0 = (item % 16) * 16;
        if (r >= a.R) {
            continue;
        }
        const int64_t prow = (int64_t(split) * pv.h_kv + kvh) * a.R + r;
        float * dst = a.po + prow * kHeadDim + c0;
#pragma unroll
        for (int c = 0; c < 16; c += 4) {
            floatx4 sum = *reinterpret_cast<const floatx4 *>(ob + r * kOStride + c0 + c);
#pragma unroll
            for (int g = 1; g < GR; ++g) {
                sum += *reinterpret_cast<const floatx4 *>(ob + (g * kRows + r) * kOStride + c0 + c);
            }
            *reinterpret_cast<floatx4 *>(dst + c) = sum;
        }
        if ((item & 15) == 0) {
            float Mr = kNegInf;
#pragma unroll
            for (int g = 0; g < GR; ++g) {
                Mr = fmaxf(Mr, ml[(g * kRows + r) * 2]);
            }
            const float Mr_use = Mr == kNegInf ? 0.0f : Mr;
            float L = 0.0f;
#pragma unroll
            for (int g = 0; g < GR; ++g) {
                L += ml[(g * kRows + r) * 2 + 1] * __builtin_amdgcn_exp2f(ml[(g * kRows + r) * 2] - Mr_use);
            }
            a.pml[prow * 2 + 0] = unmapped ? __builtin_nanf("") : Mr; // NaN: the merge writes nothing
            a.pml[prow * 2 + 1] = L;
        }
    }
    FNKV_STAMP(4);
}

// Fold the splits of each (sequence, KV head, row): one workgroup a (row, 32 values); 256 threads = 8 float4
// columns x 32 split groups. Group g folds splits g, g + 32, ... in order with a running max (all its loads
// independent, so they are in flight together: one memory round trip), then the 32 groups fold in order in LDS
// (deterministic: the same order for every launch).
// The splits of sequence s that hold partials: its first s0 and count n; false when the launch refused the sequence
// (its outputs are left as they were)
__device__ __forceinline__ bool merge_splits(const merge_args & a, int32_t s, int32_t & s0, int32_t & n) {
    s0 = a.uniform_splits > 0 ? s * a.uniform_splits : a.split0[s];
    n = a.uniform_splits > 0 ? a.uniform_splits : a.split0[s + 1] - s0;
    if (a.ctx_dev != nullptr) { // a device context: strided splits past its tiles held nothing
        const int64_t c = a.ctx_dev[s];
        if (c < a.T_dev || c > a.cap[s]) {
            return false;
        }
        const int64_t tiles = (c + kTileTokens - 1) / kTileTokens;
        n = tiles < n ? static_cast<int32_t>(tiles) : n;
    }
    if (a.depth_dev != nullptr) {
        const int64_t d = *a.depth_dev;
        if (d < 0 || d + a.T_dev > a.cap[0]) {
            return false;
        }
    }
    if (a.sel_n != nullptr) { // a sparse launch: only the splits that hold selected tiles ran
        const int32_t S = sparse_split_size(a.sel_n[s], n);
        const int32_t used = (a.sel_n[s] + S - 1) / S;
        n = used < n ? used : n;
    }
    return true;
}

__global__ __launch_bounds__(256) void merge_kernel(merge_args a) {
    __shared__ float sM[4];
    __shared__ float sL[4];
    __shared__ floatx4 sA[4][8];
    const int32_t tid = static_cast<int32_t>(threadIdx.x);
    const int32_t c4 = tid & 7, g = tid >> 3;
    const int32_t chunk = static_cast<int32_t>(blockIdx.x) & 7;
    int32_t rest = static_cast<int32_t>(blockIdx.x) >> 3;
    const int32_t r = rest % a.R;
    rest /= a.R;
    const int32_t kvh = rest % a.h_kv;
    const int32_t s = rest / a.h_kv;
    int32_t s0 = 0, n = 0;
    if (!merge_splits(a, s, s0, n)) {
        return;
    }
    float m = kNegInf, l = 0.0f;
    int32_t bad = 0; // a split that saw an unmapped page marked its partial with a NaN max: nothing is written
    floatx4 A = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
    for (int32_t i = g; i < n; i += 32) {
        const int64_t prow = (int64_t(s0 + i) * a.h_kv + kvh) * a.R + r;
        const float2 ml = *reinterpret_cast<const float2 *>(a.pml + prow * 2);
        bad |= ml.x != ml.x ? 1 : 0;
        const floatx4 o = *reinterpret_cast<const floatx4 *>(a.po + prow * kHeadDim + chunk * 32 + c4 * 4);
        const float m_new = fmaxf(m, ml.x);
        const float m_use = m_new == kNegInf ? 0.0f : m_new;
        const float f_old = __builtin_amdgcn_exp2f(m - m_use);
        const float f_new = __builtin_amdgcn_exp2f(ml.x - m_use);
        A = A * f_old + o * f_new;
        l = __builtin_fmaf(l, f_old, ml.y * f_new);
        m = m_new;
    }
    // the 32 groups fold pairwise: the wave's 8 by lane exchange (lanes l, l ^ 8, l ^ 16, l ^ 32 share c4), then the
    // 4 waves' results in LDS, in wave order
    auto fold = [](float & m0, float & l0, floatx4 & A0, float m1, float l1, floatx4 A1) {
        const float mn = fmaxf(m0, m1);
        const float mu = mn == kNegInf ? 0.0f : mn;
        const float f0 = __builtin_amdgcn_exp2f(m0 - mu), f1 = __builtin_amdgcn_exp2f(m1 - mu);
        A0 = A0 * f0 + A1 * f1;
        l0 = __builtin_fmaf(l0, f0, l1 * f1);
        m0 = mn;
    };
#pragma unroll
    for (int32_t o = 8; o < 64; o <<= 1) {
        floatx4 A1;
#pragma unroll
        for (int32_t e = 0; e < 4; ++e) {
            A1[e] = __shfl_xor(A[e], o, 64);
        }
        fold(m, l, A, __shfl_xor(m, o, 64), __shfl_xor(l, o, 64), A1);
    }
    const int32_t wave = tid >> 6;
    if ((tid & 63) < 8) {
        sA[wave][c4] = A;
        if (c4 == 0) {
            sM[wave] = m;
            sL[wave] = l;
        }
    }
    if (__syncthreads_or(bad)) {
        return;
    }
    if (tid < 8) {
        float Ms = sM[0], Ls = sL[0];
        floatx4 As = sA[0][tid];
#pragma unroll
        for (int32_t w = 1; w < 4; ++w) {
            fold(Ms, Ls, As, sM[w], sL[w], sA[w][tid]);
        }
        const int32_t t = r / a.G, h = kvh * a.G + r % a.G;
        const int64_t row = (int64_t(s) * a.T + t) * a.hq + h;
        if (a.gate != nullptr) {
            // the gate, the F32 output and its activation run (the run's 32 values are lanes 0..7's), or the prompt
            // path's fp16 output
            const float * gr = a.gate + row * a.gate_stride + chunk * 32 + tid * 4;
            float y[4];
#pragma unroll
            for (int32_t e = 0; e < 4; ++e) {
                y[e] = As[e] / Ls * (1.0f / (1.0f + expf(-gr[e])));
            }
            if (a.out_f32 != nullptr) {
                *reinterpret_cast<float4 *>(a.out_f32 + row * kHeadDim + chunk * 32 + tid * 4) =
                    make_float4(y[0], y[1], y[2], y[3]);
            }
            if (a.out16 != nullptr) {
                bool bad = false;
                uint16_t hb[4];
#pragma unroll
                for (int32_t e = 0; e < 4; ++e) {
                    bad = bad || !(fabsf(y[e]) <= 65504.0f);
                    hb[e] = __half_as_ushort(__float2half_rn(y[e]));
                }
                *reinterpret_cast<uint2 *>(a.out16 + row * kHeadDim + chunk * 32 + tid * 4) =
                    make_uint2(uint32_t(hb[0]) | (uint32_t(hb[1]) << 16), uint32_t(hb[2]) | (uint32_t(hb[3]) << 16));
                if (bad && a.err != nullptr) {
                    atomicOr(a.err, 1u);
                }
                return;
            }
            int8_t q[4];
            float ds[2];
            act_run<4, 8>(y, q, ds);
            *reinterpret_cast<uint32_t *>(a.codes + row * kHeadDim + chunk * 32 + tid * 4) =
                uint32_t(uint8_t(q[0])) | (uint32_t(uint8_t(q[1])) << 8) | (uint32_t(uint8_t(q[2])) << 16) |
                (uint32_t(uint8_t(q[3])) << 24);
            if (tid == 0) {
                a.act_scales[(row * 8 + chunk) * 2] = ds[0];
                a.act_scales[(row * 8 + chunk) * 2 + 1] = ds[1];
            }
            return;
        }
        uint16_t * o = a.out + row * kHeadDim + chunk * 32 + tid * 4;
        const float inv = 1.0f / Ls;
        uint2 pk;
        pk.x = uint32_t(__half_as_ushort(__float2half_rn(As[0] * inv))) |
               (uint32_t(__half_as_ushort(__float2half_rn(As[1] * inv))) << 16);
        pk.y = uint32_t(__half_as_ushort(__float2half_rn(As[2] * inv))) |
               (uint32_t(__half_as_ushort(__float2half_rn(As[3] * inv))) << 16);
        *reinterpret_cast<uint2 *>(o) = pk;
    }
}

// LDS of a decode launch: the groups' tile buffers, or the merge's (m, l) and partial rows, whichever is larger
template <int NT, bool SP, bool QLO = false> int32_t rows_lds() {
    using SH = rows_shape<NT, SP, QLO>;
    const int32_t ring = SH::GR * SH::GROUP_LDS + SH::Q_LDS + SH::QLO_LDS;
    const int32_t merge = SH::GR * NT * 16 * 2 * 4 + SH::GR * NT * 16 * (kHeadDim + 4) * 4;
    return SP ? std::max(std::max(ring + kSelSlice, merge), kSelLds) : std::max(ring, merge);
}
// the sparse kernels' dynamic LDS for nt row tiles (qlo: q's low parts after the selection slice)
int32_t decode_lds(int32_t nt, bool qlo = false) {
    if (nt == 1) {
        constexpr int32_t waves = dec_shape<1>::WAVES;
        const int32_t tiles = dec_shape<1>::GR * kGroupLds;
        const int32_t merge = waves * 16 * 2 * 4 + waves * 16 * (kHeadDim + 4) * 4;
        return std::max(std::max(tiles + kSelSlice + kFusedQLds, merge), kSelLds);
    }
    if (nt == 2) {
        return qlo ? rows_lds<2, true, true>() : rows_lds<2, true>();
    }
    return qlo ? rows_lds<3, true, true>() : rows_lds<3, true>();
}

// The split-K fold inside the dense launch (stream.hip) is off by default: measured against the merge kernel on one
// box it is slower (cfg1 43.8-44.2 against 42.0-43.0 us a launch, cfg2 58.9 against 55.0-55.6 us). FNKV_DECODE_FOLD=1
// (read once) or fnkv_test_decode_fold turns it on. The bound of its waits (real-time ticks of 10 ns) is 200 us, far
// past any launch's spread of arrivals; tests lower it to drive the given-up-row path from the host.
std::atomic<int32_t> g_fold_mode{-1}; // -1: the environment's choice
std::atomic<int64_t> g_fold_spin{20000};
bool fold_enabled() {
    const int32_t m = g_fold_mode.load(std::memory_order_relaxed);
    if (m >= 0) {
        return m != 0;
    }
    static const int32_t knob = env_int_once("FNKV_DECODE_FOLD", 0);
    return knob != 0;
}
int64_t fold_spin_ticks() { return g_fold_spin.load(std::memory_order_relaxed); }

int32_t env_int_once(const char * name, int32_t dflt) {
    const char * e = std::getenv(name);
    return e != nullptr ? std::atoi(e) : dflt;
}

int32_t device_cus(int32_t device) {
    // threads racing on the first query each store the same count
    static std::atomic<int32_t> cache[64];
    if (device < 0 || device >= 64) {
        return 256;
    }
    int32_t n = cache[device].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n <= 0) {
            (void)hipGetLastError();
            n = 256;
        }
        cache[device].store(n, std::memory_order_relaxed);
    }
    return n;
}

struct dec_plan {
    int32_t split_tokens = 0, total = 0, strided = 0;
    int32_t split0[FNKV_MAX_SEQS + 1] = {0};
    // the workspace: the fold state (first, at a fixed place: its words persist from launch to launch, zero), then
    // the partials
    int64_t fold_bytes = 0, po_bytes = 0, pml_bytes = 0;
    bool fold = false; // the stream kernel folds the splits itself (no merge launch)
};

dec_plan plan_decode(const kv_pool & p, int32_t n_seq, const int64_t * ctx, int32_t R) {
    dec_plan pl;
    const int32_t cus = device_cus(p.device());
    pl.split_tokens =
        choose_split_stream(n_seq, ctx, p.h_kv(), cus, (R + 15) / 16);
    // tuning knob for measurement: FNKV_SPLIT_TOKENS (a multiple of 32 from 256 to 2,048), read once per process
    static const int32_t split_knob = env_int_once("FNKV_SPLIT_TOKENS", 0);
    if (split_knob >= kPageTokens && split_knob <= 8 * kPageTokens && split_knob % kTileTokens == 0) {
        pl.split_tokens = split_knob;
    }
    pl.split0[0] = 0;
    for (int32_t i = 0; i < n_seq; ++i) {
        pl.split0[i + 1] = pl.split0[i] + static_cast<int32_t>((ctx[i] + pl.split_tokens - 1) / pl.split_tokens);
    }
    // one row tile (R <= 16): the splits of a sequence stride over its tiles, so at any moment the workgroups read
    // one window of the sequence together, and host and device contexts split alike (device contexts always stride:
    // decode_launch); more rows: contiguous splits
    pl.strided = R <= 16 ? 1 : 0;
    pl.total = pl.split0[n_seq];
    pl.fold_bytes = (int64_t(FNKV_MAX_SEQS) * p.h_kv() * kFoldWords * 4 + 255) & ~int64_t(255);
    pl.po_bytes = int64_t(pl.total) * p.h_kv() * R * kHeadDim * 4;
    pl.pml_bytes = int64_t(pl.total) * p.h_kv() * R * 2 * 4;
    // the fold waits for the other splits of its pair, so every workgroup of the launch must be resident at once:
    // one a CU (the stream kernel's LDS)
    pl.fold = fold_enabled() && int64_t(pl.total) * p.h_kv() <= cus;
    return pl;
}

// The plain fp16 output's fold: one workgroup a whole row (256 values), GRP waves = 64 float4 columns x GRP split
// groups (one a wave: group g folds splits g, g + GRP, ... with a running max, its loads in flight together), then
// the waves in order in LDS. An eighth of merge_kernel's workgroups: at these sizes a launch's cost is mostly the
// dispatch of its workgroups.
template <int GRP> __global__ __launch_bounds__(64 * GRP) void merge_row_kernel(merge_args a) {
    __shared__ float sM[GRP];
    __shared__ float sL[GRP];
    __shared__ floatx4 sA[GRP][64];
    const int32_t tid = static_cast<int32_t>(threadIdx.x);
    const int32_t c4 = tid & 63, g = tid >> 6;
    int32_t rest = static_cast<int32_t>(blockIdx.x);
    const int32_t r = rest % a.R;
    rest /= a.R;
    const int32_t kvh = rest % a.h_kv;
    const int32_t s = rest / a.h_kv;
    int32_t s0 = 0, n = 0;
    if (!merge_splits(a, s, s0, n)) {
        return;
    }
    float m = kNegInf, l = 0.0f;
    int32_t bad = 0; // a split that saw an unmapped page marked its partial with a NaN max: nothing is written
    floatx4 A = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
    for (int32_t i = g; i < n; i += GRP) {
        const int64_t prow = (int64_t(s0 + i) * a.h_kv + kvh) * a.R + r;
        const float2 ml = *reinterpret_cast<const float2 *>(a.pml + prow * 2);
        bad |= ml.x != ml.x ? 1 : 0;
        const floatx4 o = *reinterpret_cast<const floatx4 *>(a.po + prow * kHeadDim + c4 * 4);
        const float m_new = fmaxf(m, ml.x);
        const float m_use = m_new == kNegInf ? 0.0f : m_new;
        const float f_old = __builtin_amdgcn_exp2f(m - m_use);
        const float f_new = __builtin_amdgcn_exp2f(ml.x - m_use);
        A = A * f_old + o * f_new;
        l = __builtin_fmaf(l, f_old, ml.y * f_new);
        m = m_new;
    }
    sA[g][c4] = A;
    if (c4 == 0) {
        sM[g] = m;
        sL[g] = l;
    }
    if (__syncthreads_or(bad)) {
        return;
    }
    if (g != 0) {
        return;
    }
    float Ms = sM[0], Ls = sL[0];
    floatx4 As = sA[0][c4];
#pragma unroll
    for (int32_t w = 1; w < GRP; ++w) {
        const float mn = fmaxf(Ms, sM[w]);
        const float mu = mn == kNegInf ? 0.0f : mn;
        const float f0 = __builtin_amdgcn_exp2f(Ms - mu), f1 = __builtin_amdgcn_exp2f(sM[w] - mu);
        As = As * f0 + sA[w][c4] * f1;
        Ls = __builtin_fmaf(Ls, f0, sL[w] * f1);
        Ms = mn;
    }
    const int32_t t = r / a.G, h = kvh * a.G + r % a.G;
    const int64_t row = (int64_t(s) * a.T + t) * a.hq + h;
    const float inv = 1.0f / Ls;
    uint2 pk;
    pk.x = uint32_t(__half_as_ushort(__float2half_rn(As[0] * inv))) |
           (uint32_t(__half_as_ushort(__float2half_rn(As[1] * inv))) << 16);
    pk.y = uint32_t(__half_as_ushort(__float2half_rn(As[2] * inv))) |
           (uint32_t(__half_as_ushort(__float2half_rn(As[3] * inv))) << 16);
    *reinterpret_cast<uint2 *>(a.out + row * kHeadDim + c4 * 4) = pk;
}

void launch_merge(const merge_args & m, hipStream_t st) {
    // the plain fp16 output with at most 96 splits a sequence (cfg1's 67; cfg2's 128 fold faster over more threads):
    // a workgroup a row; otherwise a workgroup a (row, 32 values)
    int32_t most = m.uniform_splits;
    for (int32_t i = 0; m.uniform_splits == 0 && i < m.n_seq; ++i) {
        most = std::max(most, m.split0[i + 1] - m.split0[i]);
    }
    if (m.gate == nullptr && most <= 96) {
        hipLaunchKernelGGL(merge_row_kernel<8>, dim3(static_cast<uint32_t>(m.n_seq * m.h_kv * m.R)), dim3(512), 0, st,
                           m);
        return;
    }
    hipLaunchKernelGGL(merge_kernel, dim3(static_cast<uint32_t>(m.n_seq * m.h_kv * m.R * 8)), dim3(256), 0, st, m);
}

// the sparse kernels' instantiations for the pool's format (KV8) and the q form (QLO)
template <bool KV8, bool QLO = false> void set_decode_attrs() {
    constexpr bool SP = true;
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(decode_kernel<1, SP, KV8, QLO>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, decode_lds(1, QLO));
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(decode_rows_kernel<2, SP, KV8, QLO>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, decode_lds(2, QLO));
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(decode_rows_kernel<3, SP, KV8, QLO>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, decode_lds(3, QLO));
}

template <bool KV8, bool QLO = false> void launch_decode_fmt(int32_t NT, dim3 grid, const dec_args & a, hipStream_t st) {
    constexpr bool SP = true;
    if (NT == 1) {
        hipLaunchKernelGGL((decode_kernel<1, SP, KV8, QLO>), grid, dim3(64 * dec_shape<1>::WAVES),
                           decode_lds(1, QLO), st, a);
    } else if (NT == 2) {
        hipLaunchKernelGGL((decode_rows_kernel<2, SP, KV8, QLO>), grid, dim3(64 * rows_shape<2, SP, QLO>::WAVES),
                           decode_lds(2, QLO), st, a);
    } else {
        hipLaunchKernelGGL((decode_rows_kernel<3, SP, KV8, QLO>), grid, dim3(64 * rows_shape<3, SP, QLO>::WAVES),
                           decode_lds(3, QLO), st, a);
    }
}

// the sparse decode kernel for NT row tiles and the pool's format, its LDS attribute set once per device
void launch_decode_sparse(const kv_pool & p, int32_t NT, dim3 grid, const dec_args & a, hipStream_t st) {
    // once per device, before any launch of it returns: a thread arriving while another sets the attributes waits
    static std::once_flag attr_once[64];
    const int32_t dev = p.device();
    if (dev >= 0 && dev < 64) {
        std::call_once(attr_once[dev], [dev]() {
            int32_t cur = 0;
            (void)hipGetDevice(&cur);
            (void)hipSetDevice(dev);
            set_decode_attrs<false>();
            set_decode_attrs<true>();
            set_decode_attrs<false, true>();
            set_decode_attrs<true, true>();
            (void)hipGetLastError();
            (void)hipSetDevice(cur);
        });
    }
    if (a.q_lo != nullptr) {
        if (a.pv.format == kFormatKV8) {
            launch_decode_fmt<true, true>(NT, grid, a, st);
        } else {
            launch_decode_fmt<false, true>(NT, grid, a, st);
        }
        return;
    }
    if (a.pv.format == kFormatKV8) {
        launch_decode_fmt<true>(NT, grid, a, st);
    } else {
        launch_decode_fmt<false>(NT, grid, a, st);
    }
}

} // namespace fnkv

using fnkv::set_error;

#ifdef FNKV_TIMING
static uint64_t * g_timing = nullptr;
extern "C" void fnkv_debug_timing(void * buf) { g_timing = static_cast<uint64_t *>(buf); }
namespace fnkv {
uint64_t * timing_buffer() { return g_timing; }
}
#endif

namespace fnkv {

// The dense decode launch: ctx holds each sequence's context (ctx_dev null) or the host's bound on the device word
// ctx_dev[i] (then the splits stride over the sequence's tiles, so every depth up to the bound spreads over the same
// grid, and a context outside T .. bound sets FNKV_DEV_ERR_DEPTH in *err and writes nothing for that sequence).
int decode_launch(const fnkv_pool * pool, int32_t n_seq, const int32_t * slots, const int64_t * ctx,
                  const int64_t * ctx_dev, uint32_t * err, int32_t T, int32_t layer, int32_t hq, float scale,
                  const void * q, const void * k_new, const void * v_new, int32_t new_dtype, void * out, void * ws,
                  int64_t ws_bytes, hipStream_t st, const char * who) {
    const std::string name(who);
    const kv_pool * p = pool_of(pool);
    if (p == nullptr || n_seq <= 0 || n_seq > FNKV_MAX_SEQS || slots == nullptr || ctx == nullptr || T <= 0 ||
        layer < 0 || layer >= p->layers() || hq <= 0 || hq % p->h_kv() != 0 || q == nullptr || out == nullptr ||
        ws == nullptr || !(scale > 0.0f) || !std::isfinite(scale) || ((k_new == nullptr) != (v_new == nullptr)) ||
        (new_dtype != FNKV_F16 && new_dtype != FNKV_F32)) {
        set_error(name + ": argument outside the contract");
        return FNKV_ERR_ARG;
    }
    const int32_t G = hq / p->h_kv();
    const int32_t R = G * T;
    if (R > FNKV_MAX_ROWS) {
        set_error(name + ": G * T = " + std::to_string(R) + " exceeds " + std::to_string(FNKV_MAX_ROWS));
        return FNKV_ERR_ARG;
    }
    if ((reinterpret_cast<uintptr_t>(q) & 15) != 0 || (reinterpret_cast<uintptr_t>(out) & 15) != 0 ||
        (reinterpret_cast<uintptr_t>(ws) & 15) != 0) {
        set_error(name + ": q, out and ws must be 16-byte aligned");
        return FNKV_ERR_ARG;
    }
    for (int32_t i = 0; i < n_seq; ++i) {
        if (slots[i] < 0 || slots[i] >= p->pages().n_slots() || ctx[i] < T || ctx[i] > p->mapped_cells(slots[i])) {
            set_error(name + ": sequence " + std::to_string(i) + " (slot " + std::to_string(slots[i]) + ", " +
                      (ctx_dev != nullptr ? "bound " : "ctx ") + std::to_string(ctx[i]) +
                      ") outside the slot's mapped cells");
            return FNKV_ERR_ARG;
        }
        // with the new cells written by the launch, two sequences in one slot would write the same cells
        for (int32_t k = 0; k < i && k_new != nullptr; ++k) {
            if (slots[k] == slots[i]) {
                set_error(name + ": slot " + std::to_string(slots[i]) + " appears twice in a launch that appends");
                return FNKV_ERR_ARG;
            }
        }
    }
    const dec_plan pl = plan_decode(*p, n_seq, ctx, R);
    if (ws_bytes < pl.fold_bytes + pl.po_bytes + pl.pml_bytes) {
        set_error(name + ": workspace too small");
        return FNKV_ERR_ARG;
    }
    dec_args a;
    a.pv = p->view();
    a.q = static_cast<const uint16_t *>(q);
    a.k_new = k_new;
    a.v_new = v_new;
    a.new_f32 = new_dtype == FNKV_F32 ? 1 : 0;
    a.po = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) + pl.fold_bytes);
    a.pml = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) + pl.fold_bytes + pl.po_bytes);
    if (pl.fold) {
        a.fold = static_cast<uint32_t *>(ws);
        a.out = static_cast<uint16_t *>(out);
        a.fold_spin = fold_spin_ticks();
    }
    a.c2 = scale * 1.4426950408889634f;
    a.layer = layer;
    a.T = T;
    a.G = G;
    a.hq = hq;
    a.R = R;
    a.n_seq = n_seq;
    a.split_tokens = pl.split_tokens;
    a.strided = ctx_dev != nullptr ? 1 : pl.strided;
    a.sel_body = nullptr;
    a.sel_n = nullptr;
    a.sel_split = 0;
    a.ctx_dev = ctx_dev;
    a.err = err;
    for (int32_t i = 0; i < FNKV_MAX_SEQS; ++i) {
        a.slot[i] = i < n_seq ? slots[i] : 0;
        a.ctx[i] = i < n_seq ? ctx[i] : 0;
    }
    for (int32_t i = 0; i <= FNKV_MAX_SEQS; ++i) {
        a.split0[i] = i <= n_seq ? pl.split0[i] : pl.total;
    }
#ifdef FNKV_TIMING
    a.ts = g_timing;
#endif
    const dim3 grid(static_cast<uint32_t>(pl.total), static_cast<uint32_t>(p->h_kv()));
    launch_stream(p->device(), (R + 15) / 16, grid, a, st);
    if (pl.fold) {
        if (hipGetLastError() != hipSuccess) {
            set_error(name + ": launch failed");
            return FNKV_ERR_HIP;
        }
        return FNKV_OK;
    }
    merge_args m;
    m.po = a.po;
    m.pml = a.pml;
    m.out = static_cast<uint16_t *>(out);
    m.T = T;
    m.G = G;
    m.hq = hq;
    m.R = R;
    m.h_kv = p->h_kv();
    m.n_seq = n_seq;
    m.sel_n = nullptr;
    m.sel_split = 0;
    m.ctx_dev = ctx_dev;
    m.T_dev = T;
    for (int32_t i = 0; i <= FNKV_MAX_SEQS; ++i) {
        m.split0[i] = a.split0[i];
    }
    for (int32_t i = 0; i < FNKV_MAX_SEQS; ++i) {
        m.cap[i] = a.ctx[i];
    }
    launch_merge(m, st);
    if (hipGetLastError() != hipSuccess) {
        set_error(name + ": launch failed");
        return FNKV_ERR_HIP;
    }
    return FNKV_OK;
}

// The no-allocation variant's workspace: the split partials of fnkv_attn_decode_noalloc live in this file-scope
// device array (each device that runs the library holds its own copy until the process ends). Host code never passes
// the array's name to a kernel (on the host it is only a stand-in for the symbol): it asks each device once, when the
// first pool on that device is created, for the array's device address and uses that.
//
// One device's array serves one (pool, stream) pair at a time: the first fnkv_attn_decode_noalloc call on a device
// binds it to that call's pool and stream, and calls from another pool or on another stream are refused (they could
// run while the bound pair's last call is still in flight) until the bound pool is destroyed, which drains the device
// and releases the binding.
constexpr int64_t kNoAllocScratchBytes = int64_t(16) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int32_t kScratchDevices = 64;
struct scratch_binding {
    void * ptr = nullptr;               // the array's device address on this device
    const kv_pool * owner = nullptr;    // the pool bound to it, or null
    hipStream_t stream = nullptr;       // the stream its calls run on (valid while owner is set)
};
std::mutex g_scratch_mu;
scratch_binding g_scratch[kScratchDevices];
} // namespace

bool scratch_init(int32_t device, std::string & err) {
    if (device < 0 || device >= kScratchDevices) {
        err = "fnkv_pool_create: device index outside 0 .. 63";
        return false;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[device].ptr != nullptr) {
        return true;
    }
    int32_t cur = 0;
    if (hipGetDevice(&cur) != hipSuccess || hipSetDevice(device) != hipSuccess) {
        err = "fnkv_pool_create: cannot make the pool's device current";
        return false;
    }
    void * ptr = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    (void)hipSetDevice(cur);
    if (rc != hipSuccess || ptr == nullptr) {
        err = std::string("fnkv_pool_create: hipGetSymbolAddress of the decode scratch failed: ") +
              hipGetErrorString(rc);
        return false;
    }
    g_scratch[device].ptr = ptr;
    return true;
}

void scratch_release(const kv_pool * pool) {
    const int32_t device = pool->device();
    if (device < 0 || device >= kScratchDevices) {
        return;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[device].owner != pool) {
        return;
    }
    int32_t cur = 0;
    if (hipGetDevice(&cur) == hipSuccess && hipSetDevice(device) == hipSuccess) {
        (void)hipDeviceSynchronize();
        (void)hipSetDevice(cur);
    }
    g_scratch[device].owner = nullptr;
    g_scratch[device].stream = nullptr;
}

// the device address of the scratch for a call of `pool` on `stream`, binding the pair on the device's first call;
// null (with the error set) when another pool or stream holds it
static void * scratch_claim(const kv_pool * pool, hipStream_t stream) {
    const int32_t device = pool->device();
    if (device < 0 || device >= kScratchDevices) {
        set_error("fnkv_attn_decode_noalloc: device index outside 0 .. 63");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    scratch_binding & b = g_scratch[device];
    if (b.ptr == nullptr) {
        set_error("fnkv_attn_decode_noalloc: the decode scratch of the pool's device was never looked up");
        return nullptr;
    }
    if (b.owner == nullptr) {
        b.owner = pool;
        b.stream = stream;
    } else if (b.owner != pool) {
        set_error("fnkv_attn_decode_noalloc: the device's scratch is bound to another pool (calls could overlap); "
                  "destroy that pool first or use fnkv_attn_decode_dev");
        return nullptr;
    } else if (b.stream != stream) {
        set_error("fnkv_attn_decode_noalloc: the device's scratch is bound to another stream of this pool (calls "
                  "could overlap); keep one stream or use fnkv_attn_decode_dev");
        return nullptr;
    }
    return b.ptr;
}

} // namespace fnkv

extern "C" {

int64_t fnkv_decode_workspace_bytes(const fnkv_pool * pool, int32_t n_seq, const int64_t * ctx, int32_t T, int32_t hq) {
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    if (p == nullptr || n_seq <= 0 || n_seq > FNKV_MAX_SEQS || ctx == nullptr || T <= 0 || hq <= 0 ||
        hq % p->h_kv() != 0) {
        return -1;
    }
    const int32_t R = (hq / p->h_kv()) * T;
    const fnkv::dec_plan pl = fnkv::plan_decode(*p, n_seq, ctx, R);
    return pl.fold_bytes + pl.po_bytes + pl.pml_bytes + 256;
}

void fnkv_test_decode_fold(int32_t mode, int64_t spin_ticks) {
    fnkv::g_fold_mode.store(mode < 0 ? -1 : (mode != 0 ? 1 : 0), std::memory_order_relaxed);
    fnkv::g_fold_spin.store(spin_ticks < 0 ? 20000 : spin_ticks, std::memory_order_relaxed);
}

int fnkv_attn_decode(const fnkv_pool * pool, int32_t n_seq, const int32_t * slots, const int64_t * ctx, int32_t T,
                     int32_t layer, int32_t hq, float scale, const void * q, const void * k_new, const void * v_new,
                     int32_t new_dtype, void * out, void * ws, int64_t ws_bytes, void * stream) {
    return fnkv::decode_launch(pool, n_seq, slots, ctx, nullptr, nullptr, T, layer, hq, scale, q, k_new, v_new,
                               new_dtype, out, ws, ws_bytes, static_cast<hipStream_t>(stream), "fnkv_attn_decode");
}

int fnkv_attn_decode_dev(const fnkv_pool * pool, int32_t n_seq, const int32_t * slots, const int64_t * ctx,
                         const int64_t * max_ctx, int32_t T, int32_t layer, int32_t hq, float scale, const void * q,
                         const void * k_new, const void * v_new, int32_t new_dtype, void * out, void * ws,
                         int64_t ws_bytes, uint32_t * err, void * stream) {
    if (ctx == nullptr || err == nullptr || (reinterpret_cast<uintptr_t>(ctx) & 7) != 0 ||
        (reinterpret_cast<uintptr_t>(err) & 3) != 0) {
        fnkv::set_error("fnkv_attn_decode_dev: ctx (8-byte aligned) and err (4-byte aligned) device words required");
        return FNKV_ERR_ARG;
    }
    return fnkv::decode_launch(pool, n_seq, slots, max_ctx, ctx, err, T, layer, hq, scale, q, k_new, v_new,
                               new_dtype, out, ws, ws_bytes, static_cast<hipStream_t>(stream),
                               "fnkv_attn_decode_dev");
}

int fnkv_attn_decode_noalloc(const fnkv_pool * pool, int32_t n_seq, const int32_t * slots, const int64_t * ctx,
                             const int64_t * max_ctx, int32_t T, int32_t layer, int32_t hq, float scale,
                             const void * q, const void * k_new, const void * v_new, int32_t new_dtype, void * out,
                             uint32_t * err, void * stream) {
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    if (p == nullptr || hq <= 0 || max_ctx == nullptr) {
        fnkv::set_error("fnkv_attn_decode_noalloc: argument outside the contract");
        return FNKV_ERR_ARG;
    }
    const int64_t need = fnkv_decode_workspace_bytes(pool, n_seq, max_ctx, T, hq);
    if (need < 0) {
        fnkv::set_error("fnkv_attn_decode_noalloc: argument outside the contract");
        return FNKV_ERR_ARG;
    }
    if (need > fnkv::kNoAllocScratchBytes) {
        fnkv::set_error("fnkv_attn_decode_noalloc: the launch needs " + std::to_string(need) +
                        " bytes of split partials, more than the library's fixed " +
                        std::to_string(fnkv::kNoAllocScratchBytes) + "-byte scratch (use fnkv_attn_decode_dev)");
        return FNKV_ERR_ARG;
    }
    if (ctx == nullptr || err == nullptr || (reinterpret_cast<uintptr_t>(ctx) & 7) != 0 ||
        (reinterpret_cast<uintptr_t>(err) & 3) != 0) {
        fnkv::set_error("fnkv_attn_decode_noalloc: ctx (8-byte aligned) and err (4-byte aligned) device words required");
        return FNKV_ERR_ARG;
    }
    void * ws = fnkv::scratch_claim(p, static_cast<hipStream_t>(stream));
    if (ws == nullptr) {
        return FNKV_ERR_ARG;
    }
    return fnkv::decode_launch(pool, n_seq, slots, max_ctx, ctx, err, T, layer, hq, scale, q, k_new, v_new, new_dtype,
                               out, ws, fnkv::kNoAllocScratchBytes, static_cast<hipStream_t>(stream),
                               "fnkv_attn_decode_noalloc");
}

} // extern "C"
