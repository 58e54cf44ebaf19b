// Decode and speculative-verify attention over the Q8_0 page pool (T = 1 .. 6 query tokens a sequence), split-K
// over pages with a log-sum-exp merge.
//
// What it computes (the reference's decode attention, fn/kernels/qsa/attend.h:8-34, made dense and causal over the
// whole context, on BASELINE's Q8_0 format): for query row (t, head h) of a sequence holding ctx cells,
//   o = sum_c softmax_c(q . k_c * scale) v_c over cells c <= ctx - T + t, with k_c, v_c the decoded Q8_0 values
// (code * fp32(d)); scores, softmax statistics and accumulators in fp32; fp16 out. The split-K partials (m, l, acc)
// fold in a fixed order as the reference's finish does (attend.cu:621-655): M = max m_j, L = sum l_j e^(m_j - M),
// A = sum acc_j e^(m_j - M), o = A / L.
//
// How (MI355X): HBM-bound, so every byte is read once and the math rides the matrix cores.
//   * A workgroup (4 waves) owns one (sequence, KV head, split of the cells); its waves take the split's 32-token
//     tiles round-robin. Each tile (17,408 B: K and V codes, K and V scales) streams HBM -> LDS by 17 direct
//     global_load_lds_dwordx4 (1 KiB each, fully coalesced), double-buffered per wave.
//   * The tile layout (layout.h) puts each lane's 16 B exactly where v_mfma_f32_16x16x32_f16 wants its operand, so a
//     ds_read_b128 at lane * 16 feeds the matrix core: codes widen to fp16 exactly (byte permute + packed subtract).
//   * S^T = K Q^T one Q8_0 block (32 values) per MFMA; the block's fp32 scale folds in with one FMA per score.
//     The G query heads x T tokens sharing the KV head are the MFMA's 16-wide column side (rows padded to 16 n).
//   * Online softmax in the base-2 domain on the S^T registers (a column's 4 lanes reduce with two shuffles); P
//     lands as the B operand of O^T = V^T P^T without moving: each PV MFMA covers 16 values d of one block b, whose V
//     scale multiplies P in fp32 once per block; the product goes to the matrix core as hi + lo fp16 (two MFMAs),
//     which keeps it to ~2^-22 relative where a single fp16 operand would err by 2^-11.
//   * The 4 waves' partials merge in LDS; the workgroup writes (m, l, acc[256]) a row; merge_kernel folds the splits.
#include "../../include/fnkv.h"
#include "common.h"
#include "layout.h"
#include "mfma.h"
#include "q8_0.h"

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <vector>

namespace fnkv {

constexpr int32_t kWaves = 4;
constexpr float kNegInf = -__builtin_inff();

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
};

__device__ __forceinline__ int32_t seq_of(const dec_args & a, int32_t split) {
    int32_t s = 0;
    while (s + 1 < a.n_seq && a.split0[s + 1] <= split) {
        ++s;
    }
    return s;
}

// issue the 17 LDS loads of one tile into buf (a wave's 17,408 B)
__device__ __forceinline__ void tile_to_lds(const uint8_t * tile, uint8_t * buf, int32_t lane) {
#pragma unroll
    for (int32_t i = 0; i < 16; ++i) {
        lds_load16(tile + i * 1024 + lane * 16, buf + i * 1024);
    }
    lds_load16(tile + 16384 + lane * 16, buf + 16384);
}

template <int NT>
__global__ __launch_bounds__(256, 1) void decode_kernel(dec_args a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int32_t lane = static_cast<int32_t>(threadIdx.x) & 63;
    const int32_t wave = static_cast<int32_t>(threadIdx.x) >> 6;
    const int32_t j = lane & 15, qg = lane >> 4;
    const int32_t split = static_cast<int32_t>(blockIdx.x);
    const int32_t kvh = static_cast<int32_t>(blockIdx.y);
    const int32_t s = seq_of(a, split);
    const int32_t sp = split - a.split0[s];
    const int64_t ctx = a.ctx[s];
    const int64_t begin = int64_t(sp) * a.split_tokens;
    const int64_t end = ctx < begin + a.split_tokens ? ctx : begin + a.split_tokens;
    const int32_t n_tiles = static_cast<int32_t>((end - begin + kTileTokens - 1) / kTileTokens);

    const pool_view & pv = a.pv;
    const int32_t * table = pv.table + int64_t(a.slot[s]) * pv.table_stride;

    // the step's new cells ctx - T .. ctx - 1 that fall in this split: quantized and written here (each position lies
    // in exactly one split, so one workgroup writes it), then made visible to this workgroup's own reads
    if (a.k_new != nullptr) {
        const int64_t first_new = ctx - a.T;
        const int64_t p0 = begin > first_new ? begin : first_new;
        const int32_t nrow = static_cast<int32_t>(end - p0);
        if (nrow > 0) {
            for (int32_t job = wave; job < 2 * nrow; job += kWaves) {
                const int64_t pos = p0 + (job >> 1);
                const int32_t kv = job & 1;
                const int64_t src = ((int64_t(s) * a.T + (pos - first_new)) * pv.h_kv + kvh) * kHeadDim;
                float x[4];
                if (a.new_f32) {
                    load4<true>(static_cast<const float *>(kv ? a.v_new : a.k_new) + src, lane, x);
                } else {
                    load4<false>(static_cast<const uint16_t *>(kv ? a.v_new : a.k_new) + src, lane, x);
                }
                quantize_store(x, lane, tile_of(pv, table, a.layer, kvh, pos), static_cast<int32_t>(pos & 31), kv);
            }
            __threadfence();
            __syncthreads();
        }
    }

    // this lane's query rows (one per row tile: row nt * 16 + j) and causal limits; the Q operands go to LDS once
    // (B operand layout: [nt][block][lane] 16 B) and are read back per use, keeping them out of the registers
    uint8_t * qlds = smem + kWaves * 2 * kTileBytes;
    int64_t lim[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int32_t r = nt * 16 + j;
        const bool real = r < a.R;
        const int32_t t = real ? r / a.G : a.T - 1;
        lim[nt] = ctx - a.T + t;
        const uint16_t * qrow =
            a.q + ((int64_t(s) * a.T + t) * a.hq + int64_t(kvh) * a.G + (real ? r % a.G : 0)) * kHeadDim;
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) {
            const int b = 2 * wave + bb;
            u32x4 v = {0, 0, 0, 0};
            if (real) {
                v = *reinterpret_cast<const u32x4 *>(qrow + b * kQK + 8 * qg);
            }
            *reinterpret_cast<u32x4 *>(qlds + ((nt * kBlocks + b) * 64 + lane) * 16) = v;
        }
    }
    __syncthreads();

    floatx4 acc[NT][16];
    float m_run[NT], l_run[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        m_run[nt] = kNegInf;
        l_run[nt] = 0.0f;
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            acc[nt][m] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }

    uint8_t * wbuf = smem + wave * 2 * kTileBytes;
    const uint8_t * layer_base = pv.base + int64_t(a.layer) * pv.layer_stride + int64_t(kvh) * kPageBlock;
    auto tile_ptr = [&](int32_t ti) -> const uint8_t * {
        const int64_t tok = begin + int64_t(ti) * kTileTokens;
        const int32_t phys = table[tok >> 8];
        return layer_base + int64_t(phys) * pv.page_stride + int64_t((tok & 255) >> 5) * kTileBytes;
    };

    int32_t ti = wave;
    if (ti < n_tiles) {
        tile_to_lds(tile_ptr(ti), wbuf, lane);
    }
    int32_t stage = 0;
    for (; ti < n_tiles; ti += kWaves) {
        uint8_t * buf = wbuf + stage * kTileBytes;
        if (ti + kWaves < n_tiles) {
            tile_to_lds(tile_ptr(ti + kWaves), wbuf + (stage ^ 1) * kTileBytes, lane);
            wait_vmcnt<17>();
        } else {
            wait_vmcnt<0>();
        }
        const int64_t tok0 = begin + int64_t(ti) * kTileTokens;

        // ---- S^T = K Q^T for the tile's two 16-token halves ----
        floatx4 sc[NT][2];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            sc[nt][0] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            sc[nt][1] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int ld = 0; ld < 4; ++ld) {
            const u32x4 k0 = *reinterpret_cast<const u32x4 *>(buf + kKCodes + ld * 1024 + lane * 16);
            const u32x4 k1 = *reinterpret_cast<const u32x4 *>(buf + kKCodes + 4096 + ld * 1024 + lane * 16);
            // the K scales of blocks 2 ld, 2 ld + 1 for this lane's score rows (tokens 16 h + 4 qg + r)
            half2v ks[2][4];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    ks[h][r] = *reinterpret_cast<const half2v *>(buf + kKScales + (16 * h + 4 * qg + r) * 16 + ld * 4);
                }
            }
#pragma unroll
            for (int bb = 0; bb < 2; ++bb) {
                const int b = 2 * ld + bb;
                const half8 ka0 = widen8(k0[2 * bb], k0[2 * bb + 1]);
                const half8 ka1 = widen8(k1[2 * bb], k1[2 * bb + 1]);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const half8 qb = *reinterpret_cast<const half8 *>(qlds + ((nt * kBlocks + b) * 64 + lane) * 16);
                    const floatx4 z = {0.0f, 0.0f, 0.0f, 0.0f};
                    const floatx4 t0 = mfma16(ka0, qb, z);
                    const floatx4 t1 = mfma16(ka1, qb, z);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        sc[nt][0][r] = __builtin_fmaf(static_cast<float>(ks[0][r][bb]), t0[r], sc[nt][0][r]);
                        sc[nt][1][r] = __builtin_fmaf(static_cast<float>(ks[1][r][bb]), t1[r], sc[nt][1][r]);
                    }
                }
            }
        }

        // ---- online softmax (base 2), P as the PV B operand ----
        float pf[NT][8];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            float (&v)[8] = pf[nt];
            float mx = kNegInf;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t pos = tok0 + 16 * h + 4 * qg + r;
                    const float x = pos <= lim[nt] ? sc[nt][h][r] * a.c2 : kNegInf;
                    v[4 * h + r] = x;
                    mx = fmaxf(mx, x);
                }
            }
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float m_new = fmaxf(m_run[nt], mx);
            const float m_use = m_new == kNegInf ? 0.0f : m_new;
            const float alpha = __builtin_amdgcn_exp2f(m_run[nt] - m_use);
            float lsum = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                v[i] = __builtin_amdgcn_exp2f(v[i] - m_use);
                lsum += v[i];
            }
            l_run[nt] = __builtin_fmaf(l_run[nt], alpha, lsum);
            m_run[nt] = m_new;
            if (__any(alpha != 1.0f)) {
#pragma unroll
                for (int m = 0; m < 16; ++m) {
                    acc[nt][m] *= alpha;
                }
            }
        }

        // ---- O^T += V^T P^T: MFMA tile m covers values 16 m .. 16 m + 15 of block m / 2 ----
#pragma unroll
        for (int ld = 0; ld < 8; ++ld) {
            const u32x4 vv = *reinterpret_cast<const u32x4 *>(buf + kVCodes + ld * 1024 + lane * 16);
            const half8 vs = *reinterpret_cast<const half8 *>(buf + kVScales + qg * 128 + ld * 16);
            // P times the block's V scale in fp32, carried to the MFMA as hi + lo fp16 (fp16 alone would leave a
            // 2^-11 relative error per term, too coarse when a few large cells dominate)
            half8 ph[NT], pl[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                float x[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    x[i] = pf[nt][i] * static_cast<float>(vs[i]);
                }
                split_hilo(x, ph[nt], pl[nt]);
            }
#pragma unroll
            for (int mm = 0; mm < 2; ++mm) {
                const half8 va = widen8(vv[2 * mm], vv[2 * mm + 1]);
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    acc[nt][2 * ld + mm] = mfma16(va, ph[nt], acc[nt][2 * ld + mm]);
                    acc[nt][2 * ld + mm] = mfma16(va, pl[nt], acc[nt][2 * ld + mm]);
                }
            }
        }
        stage ^= 1;
    }

    // ---- merge the 4 waves in LDS, write the workgroup's partial ----
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        l_run[nt] += __shfl_xor(l_run[nt], 16);
        l_run[nt] += __shfl_xor(l_run[nt], 32);
    }
    constexpr int32_t kOStride = kHeadDim + 4;
    float * ml = reinterpret_cast<float *>(smem);                   // [4 waves][16 rows][2]
    float * ob = reinterpret_cast<float *>(smem + 4 * 16 * 2 * 4);  // [4 waves][16 rows][kOStride]
    const int32_t gsplit = split;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        __syncthreads(); // staging (or the previous row tile) no longer read
        if (qg == 0) {
            ml[(wave * 16 + j) * 2 + 0] = m_run[nt];
            ml[(wave * 16 + j) * 2 + 1] = l_run[nt];
        }
        __syncthreads();
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            M = fmaxf(M, ml[(w * 16 + j) * 2]);
        }
        const float M_use = M == kNegInf ? 0.0f : M;
        const float f = __builtin_amdgcn_exp2f(m_run[nt] - M_use);
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            *reinterpret_cast<floatx4 *>(ob + (wave * 16 + j) * kOStride + 16 * m + 4 * qg) = acc[nt][m] * f;
        }
        __syncthreads();
        // thread -> (row, 16 values)
        const int32_t tid = static_cast<int32_t>(threadIdx.x);
        const int32_t row = tid >> 4, c0 = (tid & 15) * 16;
        const int32_t r = nt * 16 + row;
        if (r < a.R) {
            const int64_t prow = (int64_t(gsplit) * pv.h_kv + kvh) * a.R + r;
            float * dst = a.po + prow * kHeadDim + c0;
#pragma unroll
            for (int c = 0; c < 16; c += 4) {
                floatx4 sum = *reinterpret_cast<const floatx4 *>(ob + (0 * 16 + row) * kOStride + c0 + c);
#pragma unroll
                for (int w = 1; w < kWaves; ++w) {
                    sum += *reinterpret_cast<const floatx4 *>(ob + (w * 16 + row) * kOStride + c0 + c);
                }
                *reinterpret_cast<floatx4 *>(dst + c) = sum;
            }
            if ((tid & 15) == 0) {
                float Mr = kNegInf;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    Mr = fmaxf(Mr, ml[(w * 16 + row) * 2]);
                }
                const float Mr_use = Mr == kNegInf ? 0.0f : Mr;
                float L = 0.0f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    L += ml[(w * 16 + row) * 2 + 1] * __builtin_amdgcn_exp2f(ml[(w * 16 + row) * 2] - Mr_use);
                }
                a.pml[prow * 2 + 0] = Mr;
                a.pml[prow * 2 + 1] = L;
            }
        }
    }
}

// Fold the splits of each (sequence, KV head, row): one workgroup a (row, 32 values); 256 threads = 8 float4
// columns x 32 split groups, each group summing its splits in order, the groups folded in order (deterministic).
struct merge_args {
    const float * po;
    const float * pml;
    uint16_t * out; // fp16 [n_seq][T][hq][256]
    int32_t T, G, hq, R, h_kv, n_seq;
    int32_t split0[FNKV_MAX_SEQS + 1];
};

__global__ __launch_bounds__(256) void merge_kernel(merge_args a) {
    __shared__ float sM[32];
    __shared__ floatx4 sA[32][8];
    __shared__ float sL[32];
    const int32_t tid = static_cast<int32_t>(threadIdx.x);
    const int32_t c4 = tid & 7, g = tid >> 3;
    const int32_t chunk = static_cast<int32_t>(blockIdx.x) & 7;
    int32_t rest = static_cast<int32_t>(blockIdx.x) >> 3;
    const int32_t r = rest % a.R;
    rest /= a.R;
    const int32_t kvh = rest % a.h_kv;
    const int32_t s = rest / a.h_kv;
    const int32_t s0 = a.split0[s], n = a.split0[s + 1] - s0;
    float M = kNegInf;
    for (int32_t i = g; i < n; i += 32) {
        M = fmaxf(M, a.pml[((int64_t(s0 + i) * a.h_kv + kvh) * a.R + r) * 2]);
    }
    if (c4 == 0) {
        sM[g] = M;
    }
    __syncthreads();
    M = kNegInf;
    for (int32_t i = 0; i < 32; ++i) {
        M = fmaxf(M, sM[i]);
    }
    const float M_use = M == kNegInf ? 0.0f : M;
    floatx4 A = {0.0f, 0.0f, 0.0f, 0.0f};
    float L = 0.0f;
    for (int32_t i = g; i < n; i += 32) {
        const int64_t prow = (int64_t(s0 + i) * a.h_kv + kvh) * a.R + r;
        const float w = __builtin_amdgcn_exp2f(a.pml[prow * 2] - M_use);
        L = __builtin_fmaf(a.pml[prow * 2 + 1], w, L);
        const floatx4 o = *reinterpret_cast<const floatx4 *>(a.po + prow * kHeadDim + chunk * 32 + c4 * 4);
        A += o * w;
    }
    sA[g][c4] = A;
    if (c4 == 0) {
        sL[g] = L;
    }
    __syncthreads();
    if (tid < 8) {
        floatx4 As = sA[0][tid];
        float Ls = sL[0];
        for (int32_t i = 1; i < 32; ++i) {
            As += sA[i][tid];
            Ls += sL[i];
        }
        const int32_t t = r / a.G, h = kvh * a.G + r % a.G;
        uint16_t * o = a.out + ((int64_t(s) * a.T + t) * a.hq + h) * kHeadDim + chunk * 32 + tid * 4;
        const float inv = 1.0f / Ls;
        uint2 pk;
        pk.x = uint32_t(__half_as_ushort(__float2half_rn(As[0] * inv))) |
               (uint32_t(__half_as_ushort(__float2half_rn(As[1] * inv))) << 16);
        pk.y = uint32_t(__half_as_ushort(__float2half_rn(As[2] * inv))) |
               (uint32_t(__half_as_ushort(__float2half_rn(As[3] * inv))) << 16);
        *reinterpret_cast<uint2 *>(o) = pk;
    }
}

int32_t device_cus(int32_t device) {
    static int32_t cache[64] = {0};
    if (device < 0 || device >= 64) {
        return 256;
    }
    if (cache[device] == 0) {
        int32_t n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n <= 0) {
            hipGetLastError();
            n = 256;
        }
        cache[device] = n;
    }
    return cache[device];
}

// the split size (tokens, a multiple of the page) for these contexts: the fewest rounds of one workgroup a CU times
// the split, preferring larger splits (fewer partials) on ties
int32_t choose_split(int32_t n_seq, const int64_t * ctx, int32_t h_kv, int32_t cus) {
    int32_t best = kPageTokens;
    double best_cost = 1e300;
    for (int32_t st = kPageTokens; st <= 16384; st *= 2) {
        int64_t wgs = 0;
        for (int32_t i = 0; i < n_seq; ++i) {
            wgs += (ctx[i] + st - 1) / st;
        }
        wgs *= h_kv;
        const int64_t rounds = (wgs + cus - 1) / cus;
        // a workgroup's fixed cost (ramp, partial write and merge) counted as 96 tokens of streaming
        const double cost = double(rounds) * (double(st) + 96.0);
        if (cost <= best_cost) {
            best_cost = cost;
            best = st;
        }
    }
    return best;
}

struct dec_plan {
    int32_t split_tokens = 0, total = 0;
    int32_t split0[FNKV_MAX_SEQS + 1] = {0};
    int64_t po_bytes = 0, pml_bytes = 0;
};

dec_plan plan_decode(const kv_pool & p, int32_t n_seq, const int64_t * ctx, int32_t R) {
    dec_plan pl;
    pl.split_tokens = choose_split(n_seq, ctx, p.h_kv(), device_cus(p.device()));
    pl.split0[0] = 0;
    for (int32_t i = 0; i < n_seq; ++i) {
        pl.split0[i + 1] = pl.split0[i] + static_cast<int32_t>((ctx[i] + pl.split_tokens - 1) / pl.split_tokens);
    }
    pl.total = pl.split0[n_seq];
    pl.po_bytes = int64_t(pl.total) * p.h_kv() * R * kHeadDim * 4;
    pl.pml_bytes = int64_t(pl.total) * p.h_kv() * R * 2 * 4;
    return pl;
}

} // namespace fnkv

using fnkv::set_error;

extern "C" {

int64_t fnkv_decode_workspace_bytes(const fnkv_pool * pool, int32_t n_seq, const int64_t * ctx, int32_t T, int32_t hq) {
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    if (p == nullptr || n_seq <= 0 || n_seq > FNKV_MAX_SEQS || ctx == nullptr || T <= 0 || hq <= 0 ||
        hq % p->h_kv() != 0) {
        return -1;
    }
    const int32_t R = (hq / p->h_kv()) * T;
    const fnkv::dec_plan pl = fnkv::plan_decode(*p, n_seq, ctx, R);
    return pl.po_bytes + pl.pml_bytes + 256;
}

int fnkv_attn_decode(const fnkv_pool * pool, int32_t n_seq, const int32_t * slots, const int64_t * ctx, int32_t T,
                     int32_t layer, int32_t hq, float scale, const void * q, const void * k_new, const void * v_new,
                     int32_t new_dtype, void * out, void * ws, int64_t ws_bytes, void * stream) {
    const fnkv::kv_pool * p = fnkv::pool_of(pool);
    if (p == nullptr || n_seq <= 0 || n_seq > FNKV_MAX_SEQS || slots == nullptr || ctx == nullptr || T <= 0 ||
        layer < 0 || layer >= p->layers() || hq <= 0 || hq % p->h_kv() != 0 || q == nullptr || out == nullptr ||
        ws == nullptr || !(scale > 0.0f) || !std::isfinite(scale) || ((k_new == nullptr) != (v_new == nullptr)) ||
        (new_dtype != FNKV_F16 && new_dtype != FNKV_F32)) {
        set_error("fnkv_attn_decode: argument outside the contract");
        return FNKV_ERR_ARG;
    }
    const int32_t G = hq / p->h_kv();
    const int32_t R = G * T;
    if (R > FNKV_MAX_ROWS) {
        set_error("fnkv_attn_decode: G * T = " + std::to_string(R) + " exceeds " + std::to_string(FNKV_MAX_ROWS));
        return FNKV_ERR_ARG;
    }
    if ((reinterpret_cast<uintptr_t>(q) & 15) != 0 || (reinterpret_cast<uintptr_t>(out) & 15) != 0 ||
        (reinterpret_cast<uintptr_t>(ws) & 15) != 0) {
        set_error("fnkv_attn_decode: q, out and ws must be 16-byte aligned");
        return FNKV_ERR_ARG;
    }
    for (int32_t i = 0; i < n_seq; ++i) {
        if (slots[i] < 0 || slots[i] >= p->pages().n_slots() || ctx[i] < T || ctx[i] > p->mapped_cells(slots[i])) {
            set_error("fnkv_attn_decode: sequence " + std::to_string(i) + " (slot " + std::to_string(slots[i]) +
                      ", ctx " + std::to_string(ctx[i]) + ") outside the slot's mapped cells");
            return FNKV_ERR_ARG;
        }
    }
    const fnkv::dec_plan pl = fnkv::plan_decode(*p, n_seq, ctx, R);
    if (ws_bytes < pl.po_bytes + pl.pml_bytes) {
        set_error("fnkv_attn_decode: workspace too small");
        return FNKV_ERR_ARG;
    }
    fnkv::dec_args a;
    a.pv = p->view();
    a.q = static_cast<const uint16_t *>(q);
    a.k_new = k_new;
    a.v_new = v_new;
    a.new_f32 = new_dtype == FNKV_F32 ? 1 : 0;
    a.po = static_cast<float *>(ws);
    a.pml = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) + pl.po_bytes);
    a.c2 = scale * 1.4426950408889634f;
    a.layer = layer;
    a.T = T;
    a.G = G;
    a.hq = hq;
    a.R = R;
    a.n_seq = n_seq;
    a.split_tokens = pl.split_tokens;
    for (int32_t i = 0; i < FNKV_MAX_SEQS; ++i) {
        a.slot[i] = i < n_seq ? slots[i] : 0;
        a.ctx[i] = i < n_seq ? ctx[i] : 0;
    }
    for (int32_t i = 0; i <= FNKV_MAX_SEQS; ++i) {
        a.split0[i] = i <= n_seq ? pl.split0[i] : pl.total;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<uint32_t>(pl.total), static_cast<uint32_t>(p->h_kv()));
    const int32_t NT = (R + 15) / 16;
    const size_t lds = size_t(fnkv::kWaves) * 2 * fnkv::kTileBytes + size_t(NT) * fnkv::kBlocks * 64 * 16;
    static bool attr_set[64] = {false};
    const int32_t dev = p->device();
    if (dev >= 0 && dev < 64 && !attr_set[dev]) {
        int32_t cur = 0;
        hipGetDevice(&cur);
        hipSetDevice(dev);
        hipFuncSetAttribute(reinterpret_cast<const void *>(fnkv::decode_kernel<1>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
        hipFuncSetAttribute(reinterpret_cast<const void *>(fnkv::decode_kernel<2>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
        hipFuncSetAttribute(reinterpret_cast<const void *>(fnkv::decode_kernel<3>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
        hipGetLastError();
        hipSetDevice(cur);
        attr_set[dev] = true;
    }
    if (NT == 1) {
        hipLaunchKernelGGL(fnkv::decode_kernel<1>, grid, dim3(256), lds, st, a);
    } else if (NT == 2) {
        hipLaunchKernelGGL(fnkv::decode_kernel<2>, grid, dim3(256), lds, st, a);
    } else {
        hipLaunchKernelGGL(fnkv::decode_kernel<3>, grid, dim3(256), lds, st, a);
    }
    fnkv::merge_args m;
    m.po = a.po;
    m.pml = a.pml;
    m.out = static_cast<uint16_t *>(out);
    m.T = T;
    m.G = G;
    m.hq = hq;
    m.R = R;
    m.h_kv = p->h_kv();
    m.n_seq = n_seq;
    for (int32_t i = 0; i <= FNKV_MAX_SEQS; ++i) {
        m.split0[i] = a.split0[i];
    }
    hipLaunchKernelGGL(fnkv::merge_kernel, dim3(static_cast<uint32_t>(n_seq * p->h_kv() * R * 8)), dim3(256), 0, st,
                       m);
    if (hipGetLastError() != hipSuccess) {
        set_error("fnkv_attn_decode: launch failed");
        return FNKV_ERR_HIP;
    }
    return FNKV_OK;
}

} // extern "C"
