/*
 * fnkv — MI355X (gfx950) 8-bit paged KV cache: the page pool, the Q8_0 append and the attention that reads it.
 *
 * The C-ABI drop-in for the reference's KV8 path. Plain pointers and sizes only; streams are hipStream_t passed as
 * void *. Every call that enqueues work returns FNKV_OK or an error code with NOTHING enqueued when an argument is
 * outside the contract (the reference's rule, fn/kernels/qsa/attend.h:139-141); fnkv_last_error() then holds the
 * message (the reference's std::string & err, fn/model/kv_pool.h:80-86). Host calls are not thread-safe with respect
 * to one pool (the reference's engine thread owns its pool, kv_pool.h:12-15).
 *
 * Geometry: pages of FNKV_PAGE_TOKENS tokens; head_dim 256; Q8_0 blocks of 32 values with an fp16 scale.
 * Query heads hq = G * h_kv (GQA group G); one launch serves G * T <= 48 query rows per KV head.
 */
#ifndef FNKV_H
#define FNKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FNKV_PAGE_TOKENS 256
#define FNKV_HEAD_DIM 256
#define FNKV_QK 32          /* values a Q8_0 block (ggml QK8_0, ggml-common.h:258) */
#define FNKV_MAX_SEQS 16    /* sequences a decode launch */
#define FNKV_MAX_ROWS 48    /* G * T a KV head */

enum fnkv_status {
    FNKV_OK = 0,
    FNKV_ERR_ARG = 1,      /* an argument outside the contract; nothing enqueued */
    FNKV_ERR_CAPACITY = 2, /* the pool's free pages do not suffice; nothing taken */
    FNKV_ERR_HIP = 3,      /* a HIP call failed */
};

enum fnkv_dtype { FNKV_F16 = 0, FNKV_F32 = 1 };

/* the pool's code format: ggml's Q8_0 (a fp16 scale a 32-value block, ggml-quants.c:274-297), or FNFL's KV8 (a fp16
 * scale a 64-value group, divide and round to even, fn/quant/kv_q8_ref.h:5-13, fn/kernels/qsa/kv_q8.cuh:1-12) */
enum fnkv_format { FNKV_FMT_Q8_0 = 0, FNKV_FMT_KV8 = 1 };

typedef struct fnkv_pool fnkv_pool;

/* the message of the calling thread's last failed call ("" when none) */
const char * fnkv_last_error(void);

/* ---- the page book, host only (fn/model/kv_pool.h:31-62) ---- */

/* kv_pages::pages_for (kv_pool.h:39, kv_pool.cpp:103-108): ceil(cells / page_cells), at most n_pages, 0 for none */
int32_t fnkv_pages_for(int64_t cells, int32_t page_cells, int32_t n_pages);

/* kv_slot_view (kv_pool.h:56-60) */
typedef struct {
    int32_t active;    /* a request or a read on the slot: never reclaimed */
    int32_t pages;     /* pages it holds */
    uint64_t released; /* release order (0: never used) */
} fnkv_slot_view;

/* kv_reclaim_victim (kv_pool.h:61, kv_pool.cpp:146-158): the least recently released idle slot holding pages, never
 * for_slot; -1 when none */
int32_t fnkv_reclaim_victim(const fnkv_slot_view * views, int32_t n, int32_t for_slot);

/* ---- the pool (fn/model/kv_pool.h:63-138) ---- */

/* kv_pool::init (kv_pool.h:73-75): n_pages physical pages of page_tokens tokens shared by n_slots slots, each slot's
 * logical range slot_tokens (0: the whole pool); every page holds `layers` layers x h_kv heads of Q8_0 K and V.
 * Device memory on `device`: n_pages * layers * h_kv * fnkv_page_block_bytes(). page_tokens must be 256. */
int fnkv_pool_create(int32_t n_slots, int32_t n_pages, int32_t page_tokens, int32_t layers, int32_t h_kv,
                     int64_t slot_tokens, int32_t device, fnkv_pool ** out);
/* kv_pool::init for a pool of either code format (format: enum fnkv_format). The reference's KV8 class is its
 * --fnfl-kv-format q8 pool (fn/kernels/qsa/kv_q8.cuh:8-11, state.h:88-91); fnkv_pool_create is this with FNKV_FMT_Q8_0. */
int fnkv_pool_create_fmt(int32_t n_slots, int32_t n_pages, int32_t page_tokens, int32_t layers, int32_t h_kv,
                         int64_t slot_tokens, int32_t format, int32_t device, fnkv_pool ** out);
/* the pool's code format (enum fnkv_format); -1 for null */
int32_t fnkv_pool_format(const fnkv_pool * pool);
/* kv_pool::~kv_pool (kv_pool.cpp:162-205); null is a no-op */
void fnkv_pool_destroy(fnkv_pool * pool);

/* kv_pool::ensure (kv_pool.h:80-83, kv_pool.cpp:448-501): the slot's logical prefix of at least `cells` cells (capped
 * at the slot range) backed by pages, the new pages zeroed, the device page table updated; synchronous. One
 * transaction: on failure the slot's pages are unchanged; *capacity (optional) is 1 when the free pages did not
 * suffice (FNKV_ERR_CAPACITY). */
int fnkv_pool_ensure(fnkv_pool * pool, int32_t slot, int64_t cells, int32_t * capacity);
/* kv_pool::trim (kv_pool.h:84-86, kv_pool.cpp:503-516): the slot's pages past pages_for(keep_cells) back to the free
 * list (keep 0: all). The caller has drained every consumer of them. */
int fnkv_pool_trim(fnkv_pool * pool, int32_t slot, int64_t keep_cells);
/* kv_pool::mapped_cells (kv_pool.h:90) */
int64_t fnkv_pool_mapped_cells(const fnkv_pool * pool, int32_t slot);
/* kv_pages::free_pages / n_pages / mapped / physical (kv_pool.h:33-38) */
int32_t fnkv_pool_free_pages(const fnkv_pool * pool);
int32_t fnkv_pool_n_pages(const fnkv_pool * pool);
int32_t fnkv_pool_mapped_pages(const fnkv_pool * pool, int32_t slot);
int32_t fnkv_pool_physical(const fnkv_pool * pool, int32_t slot, int32_t logical);
/* the slot's page table (physical page of each mapped logical page) into out[cap]; returns the count */
int32_t fnkv_page_table(const fnkv_pool * pool, int32_t slot, int32_t * out, int32_t cap);
/* kv_pool::ledger (kv_pool.h:96-97, kv_pool.cpp:544-570): the startup lines, '\n'-separated, into buf[cap] */
int32_t fnkv_pool_ledger(const fnkv_pool * pool, char * buf, int32_t cap);
/* kv_pool::test_fail_map (kv_pool.h:98-103): TEST ONLY — the next ensure fails after readying `after` of its new pages
 * (a mid-transaction failure); -1: off */
void fnkv_pool_test_fail(fnkv_pool * pool, int32_t after);
/* bytes of one (page, layer, head) block: 256 tokens of K and V codes and scales */
int64_t fnkv_page_block_bytes(void);
/* the pool's device allocation and its size */
void * fnkv_pool_device_base(const fnkv_pool * pool);
int64_t fnkv_pool_device_bytes(const fnkv_pool * pool);

/* ---- the append (fn/kernels/qsa/qsa_prompt.h:90-104 qsp_kv, attend.cu:218-260 prepare) ---- */

/* Quantizes rows new K and V rows (k, v: [rows][h_kv][256] of dtype, device) by the pool's rule — Q8_0: ggml's
 * quantize_row_q8_0_ref (ggml-quants.c:274-297); KV8: kv_q8_quantize_group (fn/quant/kv_q8_ref.cpp:72-87, device
 * kv8::quantize8, fn/kernels/qsa/kv_q8.cuh:29-52) — and writes them at the slot's positions pos0 .. pos0 + rows - 1
 * of `layer` through the page table (cell pos: logical page pos / 256, offset pos % 256). The positions must be
 * mapped (fnkv_pool_ensure). */
int fnkv_q8_append(fnkv_pool * pool, int32_t slot, int32_t layer, int64_t pos0, int32_t rows, const void * k,
                   const void * v, int32_t dtype, void * stream);

/* Reads the slot's cells tok0 .. tok0 + n_tok - 1 of (layer, head, kv: 0 K, 1 V) back as ggml block_q8_0 (34 B a
 * block, 8 blocks a cell) into out (device, n_tok * 272 bytes): the interchange form of the stored codes. */
int fnkv_export_q8_0(const fnkv_pool * pool, int32_t slot, int32_t layer, int32_t head, int32_t kv, int64_t tok0,
                     int32_t n_tok, void * out, void * stream);

/* Reads the slot's cells tok0 .. tok0 + n_tok - 1 of (layer, head, kv) of a KV8 pool back in the reference's KV8
 * form: codes int8 [n_tok][256] and the group scales fp16 bits [n_tok][4] (device), the arrays the reference keeps
 * cell-major (kv_q8.cuh:8-11). */
int fnkv_export_kv8(const fnkv_pool * pool, int32_t slot, int32_t layer, int32_t head, int32_t kv, int64_t tok0,
                    int32_t n_tok, void * codes, void * scales, void * stream);

/* ---- decode / speculative verify attention (fn/kernels/qsa/attend.h:97-151 attend, attend_lanes) ---- */

/* The workspace a decode launch over these sequences needs (bytes; device memory the caller allocates and zeroes
 * once before its first use: its first bytes hold the counters of the launch's split-K fold, which every launch
 * leaves ready for the next, as the reference's attend workspace, attend.h:89-93). ctx[n_seq] as for
 * fnkv_attn_decode. */
int64_t fnkv_decode_workspace_bytes(const fnkv_pool * pool, int32_t n_seq, const int64_t * ctx, int32_t T, int32_t hq);

/* Dense causal attention of T query tokens of each of n_seq sequences over their pooled Q8_0 K/V of `layer`.
 * slots[n_seq], ctx[n_seq] host arrays: sequence i lives in slot slots[i] and holds ctx[i] cells, its T new ones
 * included; query t of it sits at position ctx[i] - T + t and sees cells 0 .. ctx[i] - T + t.
 * k_new, v_new (optional, both or neither; dtype new_dtype, [n_seq][T][h_kv][256]): the step's new cells, quantized
 * (the fnkv_q8_append rule) and written at positions ctx[i] - T .. ctx[i] - 1 by this launch before it reads them, as
 * the reference's attend writes its rows' cells (attend.h:100-108); null: those cells were appended already.
 * q: fp16 [n_seq][T][hq][256], out: fp16 [n_seq][T][hq][256] (device). Scores q.k * scale (the reference: 1/16),
 * softmax and accumulation in fp32, split-K over pages merged by log-sum-exp. hq = G * h_kv with G * T <= 48.
 * Replaces fn::qsa::attn::attend / attend_lanes (fn/kernels/qsa/attend.h:141, :151) for dense Q8_0 KV. */
int fnkv_attn_decode(const fnkv_pool * pool, int32_t n_seq, const int32_t * slots, const int64_t * ctx, int32_t T,
                     int32_t layer, int32_t hq, float scale, const void * q, const void * k_new, const void * v_new,
                     int32_t new_dtype, void * out, void * ws, int64_t ws_bytes, void * stream);

/* The device error word's refused-depth bit (fn/kernels/qsa/attend.h:91-92, :108-110: "sets the error word (2)"): a
 * launch that reads its context or depth from device memory and finds it outside its contract writes nothing for the
 * sequence concerned and ORs this bit into the caller-cleared word. (The reference's bit 1, an acquire timeout, has no
 * counterpart: no launch here waits on another workgroup.) */
#define FNKV_DEV_ERR_DEPTH 2u

/* fnkv_attn_decode with each sequence's context read from device memory by the launch, the reference's device depth
 * (attend.h:108, "read by the launch (TG1)"): ctx[n_seq] (device, int64) is read when the launch runs, so one
 * captured graph serves every decode step; max_ctx[n_seq] (host) bounds it and fixes the grid and the workspace
 * (fnkv_decode_workspace_bytes(pool, n_seq, max_ctx, T, hq)), each at most the slot's mapped cells when called. A
 * sequence whose ctx[i] is below T or above max_ctx[i] is refused on the device: nothing of it is written (neither
 * its new cells nor its out rows) and FNKV_DEV_ERR_DEPTH is ORed into *err (device, caller-cleared); the other
 * sequences run. Splits of a sequence take its 32-token tiles in turn (split j of n: tiles j, j + n, ...), so a context
 * below its bound still spreads over every split. Otherwise as fnkv_attn_decode (whose G * T <= 16 launches split the
 * same way: for equal contexts and bounds their outputs are bitwise equal). The slots must stay mapped up to max_ctx
 * while a captured launch may run (no fnkv_pool_trim below it); a launch that nevertheless finds an unmapped page reads
 * nothing from it, writes nothing for that sequence and ORs FNKV_DEV_ERR_DEPTH into *err. Replaces the depth contract
 * of fn::qsa::attn::attend (attend.h:97-141). */
int fnkv_attn_decode_dev(const fnkv_pool * pool, int32_t n_seq, const int32_t * slots, const int64_t * ctx,
                         const int64_t * max_ctx, int32_t T, int32_t layer, int32_t hq, float scale, const void * q,
                         const void * k_new, const void * v_new, int32_t new_dtype, void * out, void * ws,
                         int64_t ws_bytes, uint32_t * err, void * stream);

/* No counterpart in the reference: fnkv_attn_decode_dev for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Arguments and results as
 * fnkv_attn_decode_dev's, bitwise, without ws / ws_bytes: the split partials live in a fixed 16 MiB device array of the
 * library (one a GPU, held until the process ends), and the call allocates nothing. A launch whose partials
 * (fnkv_decode_workspace_bytes(pool, n_seq, max_ctx, T, hq)) exceed 16 MiB is refused (FNKV_ERR_ARG, nothing
 * enqueued); cfg-sized launches (4 sequences of 8K-64K at T = 3, or one of 262,144 at T = 5) need 6-11 MiB. Every
 * call on one GPU shares that array (it starts zeroed and every call leaves its fold counters ready for the next), so
 * the array is bound to one pool and one stream at a time: the first call on a GPU binds its pool and stream, and a
 * call from another pool, or on another stream, is refused (FNKV_ERR_ARG, nothing enqueued) until the bound pool is
 * destroyed (fnkv_pool_destroy drains the GPU and releases the binding). The array's address is looked up when the
 * first pool on a GPU is created, so the call itself makes no lookup and may be captured into a HIP graph. Calls on the
 * bound stream from several host threads are not refused and must be serialized by the caller. */
int fnkv_attn_decode_noalloc(const fnkv_pool * pool, int32_t n_seq, const int32_t * slots, const int64_t * ctx,
                             const int64_t * max_ctx, int32_t T, int32_t layer, int32_t hq, float scale,
                             const void * q, const void * k_new, const void * v_new, int32_t new_dtype, void * out,
                             uint32_t * err, void * stream);

/* Test hook, no counterpart in the reference: the dense decode launches' split-K fold inside the launch (mode 1; 0:
 * the partials go to a second, merge launch, the default; negative: the FNKV_DECODE_FOLD environment variable's
 * choice) and the bound of its waits (real-time ticks of 10 ns; negative: the default, 20,000). A tiny bound makes the
 * splits that fold rows give them up to the last split to arrive, which folds them instead (the same outputs,
 * bitwise), so tests drive that path from the host. Affects launches planned after the call, in every thread. */
void fnkv_test_decode_fold(int32_t mode, int64_t spin_ticks);

/* ---- sparse (QSA) attention at decode rows (fn/kernels/qsa/attend.h:97-141 attend over a selection body) ---- */

/* The workspace a sparse launch at this depth needs (bytes; no zeroing needed); -1 outside the contract. */
int64_t fnkv_sparse_workspace_bytes(const fnkv_pool * pool, int64_t depth, int32_t T, int32_t hq);

/* Attention of T (1..5) query rows of the sequence in `slot`, row t at position depth + t, each over its own
 * selection: body (device, U32 words) in the reference's selected-block layout (fn/kernels/qsa/qsa.h:77-81): row t
 * has K = min((q + 1) / 4, 512) ascending 4-cell block IDs and its tail cells 4 ((q + 1) / 4) .. q, the rows packed in
 * order (2 + K + tail words each). offsets (device, I32 [T + 1]) is the reference's byte-offset array; the launch
 * derives the same offsets from depth and T (they depend on nothing else) and reads no word past the body. Block IDs
 * outside the row's whole blocks are ignored. k_new / v_new (optional, [T][h_kv][256] of new_dtype): the rows' own
 * cells, written at depth .. depth + T - 1 before any row reads (a row's selection need not include them). q, out:
 * fp16 [T][hq][256]; scores q.k * scale, softmax and accumulation in fp32, over the pool's codes exactly as the dense
 * launch. depth + T <= 262,176 and mapped; hq / h_kv <= FNKV_MAX_ROWS (each row runs as its own splits, side by side,
 * after the new cells are written). */
int fnkv_attn_sparse(const fnkv_pool * pool, int32_t slot, int64_t depth, int32_t T, int32_t layer, int32_t hq,
                     float scale, const void * q, const void * body, const void * offsets, const void * k_new,
                     const void * v_new, int32_t new_dtype, void * out, void * ws, int64_t ws_bytes, void * stream);

/* fnkv_attn_sparse with the depth read from device memory (attend.h:108): depth (device, int32) is read by the launch;
 * max_cells (host) bounds depth + T, fixes the plan (workspace: fnkv_sparse_workspace_bytes(pool, max_cells - T, T,
 * hq)) and must not exceed the slot's mapped cells. A depth with depth + T beyond max_cells (or below 0) writes
 * nothing — no new cells, no out rows — and ORs FNKV_DEV_ERR_DEPTH into *err (device, caller-cleared). The body's
 * layout follows the depth read. */
int fnkv_attn_sparse_dev(const fnkv_pool * pool, int32_t slot, const int32_t * depth, int64_t max_cells, int32_t T,
                         int32_t layer, int32_t hq, float scale, const void * q, const void * body,
                         const void * offsets, const void * k_new, const void * v_new, int32_t new_dtype, void * out,
                         void * ws, int64_t ws_bytes, uint32_t * err, void * stream);

/* ---- the reference's decode attention with its prepare and gate (fn/kernels/qsa/attend.h:57-141 attn::attend) ---- */

/* The workspace of fnkv_qsa_attend at this depth (bytes; no zeroing needed); -1 outside the contract. */
int64_t fnkv_qsa_workspace_bytes(const fnkv_pool * pool, int64_t depth, int32_t T, int32_t hq);

/* attn::attend (attend.h:97-141, args :57-91) over the pool, for T (1..5) rows of the sequence in `slot`, row t at
 * position depth + t: each row's query heads and its new cell's k get the F32 RMS norm (eps 1e-6) and IMROPE
 * (attend.cu:151-198; positions pos, device I32 [4][T], plane p of row t at pos[p T + t]; theta_scale
 * fnkv_rope_theta_scale()), the new cells' K (normed, roped) and V are written into the pool at depth .. depth + T - 1
 * in its format, each row attends over its selection body (as fnkv_attn_sparse, but q enters as fp16 hi + lo, about
 * 22 bits of the F32 q, the codes exactly and P with 6 more bits; scores q . k / 16; within the reference checker's
 * 1e-5 normalized bound, qa2_test.cpp:58), and each (row, head) is finished with its gate: out = o / (1 + exp(-gate)) in F32 with its int8 activation format.
 * qfull: F32 [T][hq][512] (each head's q, then its gate); kv_k, kv_v: F32 [T][h_kv][256]; q_norm, k_norm: F32 [256];
 * out: F32 [T][hq][256]; codes: int8 [T][hq 256]; scales: F32 [T][hq 8][2]; q_f32, k_f32 (optional): the F32 q
 * [T][hq][256] and k [T][h_kv][256] after the norm and rope. Three launches in stream order: the prepare (which
 * writes the new cells), the attention (each row its own splits), the gated merge; at most 16 query heads a KV head:
 * two (the attention forms each row's query heads and writes the new cells itself, bitwise the same outputs).
 * hq / h_kv <= FNKV_MAX_ROWS. */
int fnkv_qsa_attend(const fnkv_pool * pool, int32_t slot, int64_t depth, int32_t T, int32_t layer, int32_t hq,
                    const float * qfull, const float * kv_k, const float * kv_v, const float * q_norm,
                    const float * k_norm, const int32_t * pos, float theta_scale, const void * body,
                    const void * offsets, float * out, int8_t * codes, float * scales, float * q_f32, float * k_f32,
                    void * ws, int64_t ws_bytes, void * stream);

/* fn::qsa::attn::args (attend.h:57-91) over the pool: the cache pair (k_cache, v_cache, k_scale, v_scale) is the pool's
 * slot and layer; the workspace is the caller's (no zeroing needed: nothing here carries state between launches) and
 * the error word is its own field (the reference's ws.error). */
typedef struct {
    const fnkv_pool * pool;
    int32_t slot;
    int32_t layer;
    int32_t hq;              /* query heads (the reference's card: 12 on one KV head) */
    const float * qfull;     /* F32 [rows][hq][512]: each head's q, then its gate */
    const float * kv_k;      /* F32 [rows][h_kv][256], before the norm */
    const float * kv_v;      /* F32 [rows][h_kv][256] */
    const float * q_norm;    /* [256] */
    const float * k_norm;    /* [256] */
    const uint32_t * body;   /* the selection body of the rows (qsa.h:77-81 layout) */
    const int32_t * offsets; /* [rows + 1] its byte offsets */
    const int32_t * pos;     /* [4][rows] the rope planes of each row */
    const int32_t * depth;   /* device: cells before the rows, read by the launch (TG1) */
    int32_t max_cells;       /* host: depth + rows beyond it writes nothing and sets FNKV_DEV_ERR_DEPTH */
    float theta_scale;       /* fnkv_rope_theta_scale() */
    float * out;             /* F32 [rows][hq][256], gated */
    int8_t * codes;          /* [rows][hq 256] the activation format */
    float * scales;          /* [rows][hq 8][2] */
    float * q_f32;           /* optional [rows][hq][256]: q after the norm and rope */
    float * k_f32;           /* optional [rows][h_kv][256]: the new cells' F32 k before quantizing */
    void * ws;               /* fnkv_attend_workspace_bytes of device memory */
    int64_t ws_bytes;
    uint32_t * err;          /* device error word, caller-cleared */
} fnkv_attend_args;

#define FNKV_MAX_LANES 4 /* lanes of a joint verify round (attend.h:143-151: 2 .. 4) */

/* attn::workspace_bytes (attend.h:85) for launches of `rows` rows up to max_cells; -1 outside the contract */
int64_t fnkv_attend_workspace_bytes(const fnkv_pool * pool, int32_t max_cells, int32_t rows, int32_t hq);

/* attn::attend (attend.h:97-141): fnkv_qsa_attend's computation with the depth read on the device, so one captured
 * graph serves every step; max_cells at most the slot's mapped cells and 262,176. A refused depth writes nothing
 * (no new cells, no outputs) and sets FNKV_DEV_ERR_DEPTH. FNKV_ERR_ARG with nothing enqueued for an argument outside
 * the contract. */
int fnkv_attend(int32_t rows, const fnkv_attend_args * a, void * stream);

/* attn::attend_lanes (attend.h:143-151): the joint verify round of `lanes` (2 .. FNKV_MAX_LANES) sequences, lane u
 * on its own arguments a[u] (distinct slots), every lane's rows the same count. Each lane's launches are fnkv_attend's
 * on its arguments, enqueued lane after lane, so each lane's outputs and written cells are bitwise its lone call's;
 * a lane at a refused depth sets its own error word and writes nothing, the others run. Every lane is checked before
 * anything is enqueued: FNKV_ERR_ARG with nothing enqueued when any lane is outside the contract. */
int fnkv_attend_lanes(int32_t lanes, int32_t rows, const fnkv_attend_args * a, void * stream);

/* ---- the prompt path's own contract: qsp_kv and qsp_attend (fn/kernels/qsa/qsa_prompt.h:90-124) ---- */

#define FNKV_QSP_MAX_ROWS 4096 /* rows a call (qsa_prompt.h prompt_max_rows) */

/* fn::qsa::qsp_kv_args (qsa_prompt.h:90-102) over the pool: the caches are the pool's slot and layer (its format:
 * Q8_0 or KV8) */
typedef struct {
    const fnkv_pool * pool;
    int32_t slot;
    int32_t layer;
    const float * kv_k;     /* F32 [rows][h_kv][256], before the norm */
    const float * kv_v;     /* F32 [rows][h_kv][256] */
    const float * k_norm;   /* [256] */
    int32_t rows, pos0;     /* rows 1 .. FNKV_QSP_MAX_ROWS at cells pos0 .. pos0 + rows - 1 (mapped) */
    int32_t rope_off;       /* row t's rotary position pos0 + rope_off + t (every plane) when planes is null */
    const int32_t * planes; /* optional device [rows][4]: row t's rope planes (t, h, w, e) */
    float theta_scale;      /* fnkv_rope_theta_scale() */
} fnkv_qsp_kv_args;

/* qsp_kv (qsa_prompt.h:104, qsa_prompt_attn.cu:90-122, 440-454): row t's k = IMROPE(RMS norm(kv_k) k_norm) at its
 * rope position and v = kv_v, written at cell pos0 + t in the pool's format (the codes bitwise the pool quantizer's of
 * that F32 k). FNKV_ERR_ARG with nothing enqueued outside the contract. */
int fnkv_qsp_kv(const fnkv_qsp_kv_args * a, void * stream);

/* fn::qsa::qsp_attend_args (qsa_prompt.h:106-122) over the pool */
typedef struct {
    const fnkv_pool * pool;
    int32_t slot;
    int32_t layer;
    int32_t hq;              /* query heads (the reference's card: 12 on one KV head) */
    const float * qfull;     /* F32 [rows][hq][512]: each head's q, then its gate */
    const float * q_norm;    /* [256] */
    const uint32_t * body;   /* the rows' selection bodies, slab layout: slab k (rows 128 k ..) at body + k 128 517 */
    const int32_t * offsets; /* [slabs][129]: row i of slab k's body at byte offsets[129 k + i] of its slab */
    int32_t rows, pos0;      /* row t at position pos0 + t (its cells, and every cell it selects, written) */
    float * out;             /* optional F32 [rows][hq][256] */
    uint16_t * out16;        /* fp16 [rows][hq][256] */
    uint32_t * err;          /* optional device word: bit 0 for an output fp16 cannot hold (|x| > 65,504, NaN) */
    int32_t rope_off;        /* as fnkv_qsp_kv_args */
    const int32_t * planes;
    float theta_scale;
    void * ws;               /* fnkv_qsp_workspace_bytes of device memory (no zeroing needed) */
    int64_t ws_bytes;
} fnkv_qsp_attend_args;

/* the workspace of fnkv_qsp_attend for these rows at pos0 (bytes); -1 outside the contract */
int64_t fnkv_qsp_workspace_bytes(const fnkv_pool * pool, int32_t pos0, int32_t rows, int32_t hq);

/* qsp_attend (qsa_prompt.h:124, qsa_prompt_attn.cu:229-471): each row's query heads q = IMROPE(RMS norm(q) q_norm)
 * attend over the row's selection body (its blocks' 4 cells each, then its tail) with scores q . k / 16, softmax and
 * accumulation in F32 over the pool's codes, and out = o / (1 + exp(-gate)) goes to out (F32, optional) and out16
 * (fp16, nearest even), bit 0 of *err for a value fp16 cannot hold. The reference rounds q / 16 and its K / V to fp16
 * and holds the result to 2e-2 (its prompt test's bound); here q enters as fp16 and every other product keeps ~22
 * bits, held to 2e-3. FNKV_ERR_ARG with nothing enqueued outside the contract. */
int fnkv_qsp_attend(const fnkv_qsp_attend_args * a, void * stream);

/* ---- chunked-prefill attention (fn/kernels/qsa/qsa_prompt.h:106-124 qsp_attend) ---- */

/* the workspace a prefill launch of this shape uses (bytes; 0: none; -1: a shape outside the contract) */
int64_t fnkv_prefill_workspace_bytes(const fnkv_pool * pool, int64_t ctx, int32_t rows, int32_t hq);

/* Causal attention of `rows` query tokens (positions ctx - rows .. ctx - 1 of the slot, already appended) over the
 * slot's cells 0 .. ctx - 1 of `layer`, on the matrix cores with fp32 accumulation: K and V (code x scale) as exact
 * hi + lo fp16 operands, P as hi + lo fp16 (the reference's prompt attention rounds its operands to fp16 once,
 * qsa_prompt.h:55-58; this keeps ~22 bits a product). q: fp16 [rows][hq][256], out: fp16 [rows][hq][256].
 * ws: fnkv_prefill_workspace_bytes bytes of device memory (no zeroing needed) for the key-split partials when the
 * query rows alone do not fill the device; null (or smaller): one split, no workspace. The GQA group hq / h_kv must
 * divide 256 (a workgroup's query rows). */
int fnkv_attn_prefill(const fnkv_pool * pool, int32_t slot, int32_t layer, int64_t ctx, int32_t rows, int32_t hq,
                      float scale, const void * q, void * out, void * ws, int64_t ws_bytes, void * stream);

/* ---- the draft block's dense F16 attention, DA-TC (fn/kernels/draft/draft.h:47-83, 159-218) ----
 *
 * One KV head, its FNKV_DATC_HEADS query heads, flat F16 caches k_cache / v_cache [max_cells][256] owned by the
 * caller (not the pool). prepare: per row the F32 RMS norm (eps 1e-6) and IMROPE of each query head and of k, the F16
 * (nearest even) K and V written at cell n_before + row0 + t, q / 16 rounded to F16; attend: the one row row0 over
 * cells 0 .. n_before + row0 (or over a selection body, SP2), S = q16 . K with exact F16 products and F32
 * accumulation, the online softmax in F32 with P rounded to F16 and l the sum of the rounded P, P V, the fold of the
 * partials, then out = o * sigmoid(gate) in F32 and its int8 activation format (32-value runs: codes and {d, s}, the
 * rule of fn/quant/act_ref.h:10-13). n_before, pos and stride are device words read by the launches (graph
 * capturable). A cell at or past max_cells (or, SP2, a body whose K is not this depth's) sets FNKV_DEV_ERR_DRAFT_DEPTH
 * in *err and writes nothing. Arguments outside the contract: FNKV_ERR_ARG, nothing enqueued. */
#define FNKV_DATC_HEADS 12         /* query heads a KV head (draft.h:166 n_head) */
#define FNKV_DATC_QSTRIDE 512      /* qfull: [q | gate] a head (draft.h:168 q_stride) */
#define FNKV_DATC_MAX_ROWS 5       /* rows a prepare (draft.h:159 max_rows) */
#define FNKV_DATC_MAX_SPARSE_ROW 4 /* SP2: row0 below this (draft.h:178 max_sparse_steps) */
#define FNKV_DEV_ERR_DRAFT_DEPTH (1u << 24) /* the reference's err_draft_depth bit (fn/xchg/xchg.h:230) */

/* fn::draft::prepare_args (draft.h:192-213) without the exchange-slot releases (release_hc, release_hmix: the card
 * exchange is not part of this library) */
typedef struct {
    const float * qfull;     /* F32 [rows][12][512], or null: K and V only (the catch-up) */
    const float * kv_k;      /* F32 [rows][256], before the norm */
    const float * kv_v;      /* F32 [rows][256] */
    const float * q_norm;    /* [256] */
    const float * k_norm;    /* [256] */
    const int32_t * n_before; /* device: cells before the round's rows */
    const int32_t * pos;     /* device: rope planes [4][*stride] (t, h, w, e) */
    const int32_t * stride;  /* device: the round's rows */
    int32_t row0;            /* this launch's first row in the round */
    float theta_scale;       /* fnkv_rope_theta_scale() */
    uint16_t * k_cache;      /* F16 [max_cells][256] */
    uint16_t * v_cache;
    int32_t max_cells;
    uint16_t * q16;          /* F16 [rows][12][256]: q / 16; unused without qfull */
    float * q_f32;           /* optional [rows][12][256]: the F32 q before the scale */
    float * k_f32;           /* optional [rows][256]: the F32 k before rounding */
    uint32_t * err;          /* device error word (FNKV_DEV_ERR_DRAFT_DEPTH) */
} fnkv_datc_prepare_args;

/* fn::draft::attend_args (draft.h:215-235) */
typedef struct {
    const uint16_t * q16;    /* the row's prepared q16 [12][256] */
    const float * qfull;     /* the row's F32 [12][512]: its gates (floats 256..511 of each head) */
    const uint16_t * k_cache; /* F16 [max_cells][256] */
    const uint16_t * v_cache;
    const int32_t * n_before; /* device */
    int32_t row0;            /* the row's index in the round; its cell is n_before + row0 */
    int32_t max_cells;
    void * part;             /* fnkv_datc_part_bytes() of device scratch (no zeroing needed) */
    float * out;             /* F32 [3072], gated */
    int8_t * codes;          /* [3072] the activation format */
    float * scales;          /* [96][2] */
    uint32_t * err;
    /* SP2, optional: a select body made at depth N - 1 (N = *n_before): U32 K = min(N / 4, 512), the tail count, then
     * K ascending block IDs; the row attends the K blocks' cells, then cells 4 (N / 4) .. N + row0 in order (row0 <
     * FNKV_DATC_MAX_SPARSE_ROW). Null: every cell 0 .. N + row0. */
    const uint32_t * body;
} fnkv_datc_attend_args;

/* rope_theta_scale (fn/kernels/qsa/attend.cu:830-832): powf(1e7, -2 / 64) */
float fnkv_rope_theta_scale(void);

/* part_bytes (draft.h:237): the attend's scratch */
int64_t fnkv_datc_part_bytes(void);

/* datc_prepare (draft.h:243, datc.cu:560-578): one launch for rows 1..5 (row0 + rows <= 5) */
int fnkv_datc_prepare(int32_t rows, const fnkv_datc_prepare_args * a, void * stream);

/* datc_attend (draft.h:244, datc.cu:582-604): two launches (the split attention, then the fold with the gate) */
int fnkv_datc_attend(const fnkv_datc_attend_args * a, void * stream);

/* The draft step row as one call: datc_prepare(1, p) then datc_attend(a) in stream order (draft.h:47-78, the
 * contract and its publication by the kernel boundary), in two launches instead of three: the attention forms the
 * row's q itself and its one reading wave writes the row's K / V before reading them. Outputs (q16, q_f32, k_f32, the
 * caches' new cell, out, codes, scales) bitwise those of the two calls. p and a name the same caches, depth word,
 * max_cells and row0; a->q16 is not read. A refusal of either (the row's cell at or past max_cells, row0 past *stride,
 * a body not made at this depth) sets FNKV_DEV_ERR_DRAFT_DEPTH and writes nothing. */
int fnkv_datc_step(const fnkv_datc_prepare_args * p, const fnkv_datc_attend_args * a, void * stream);

#ifdef __cplusplus
}
#endif

#endif /* FNKV_H */
