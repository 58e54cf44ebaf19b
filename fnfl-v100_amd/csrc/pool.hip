// The page book, the reclaim choice and the pool (host), plus the pool's C-ABI.
//   kv_pages            follows fn/model/kv_pool.cpp:85-144 (same rules: pages_for rounding capped at the pool;
//                       take is all-or-nothing, lowest free page first; give pops last-first); the free pages are
//                       a bitset here, so take is a count-trailing-zeros scan and give sets bits.
//   kv_reclaim_victim   follows kv_pool.cpp:146-158 (strict < on the release order: ties go to the lower slot).
//   kv_pool             kv_pool.h:63-138 re-designed: one HBM allocation of physical pages plus an int32 page table a
//                       slot (the kernels gather through it) instead of VMM-mapped virtual ranges; ensure/trim keep
//                       the reference's transaction rules (kv_pool.cpp:448-516): all or nothing, new pages zeroed
//                       synchronously before the call returns, trim after the caller drained the consumers.
#include "../../include/fnkv.h"
#include "common.h"
#include "kv_pool.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>

namespace fnkv {

// ---- errors ----

static thread_local std::string g_err;

void set_error(const std::string & e) { g_err = e; }
const char * last_error() { return g_err.c_str(); }

// ---- kv_pages ----

void kv_pages::init(int32_t n_slots, int32_t n_pages) {
    n_pages_ = std::max(0, n_pages);
    n_free_ = n_pages_;
    rows_.assign(size_t(std::max(0, n_slots)), {});
    free_bits_.assign(size_t((n_pages_ + 63) / 64), ~uint64_t(0));
    if (n_pages_ % 64 != 0) {
        free_bits_.back() = (uint64_t(1) << (n_pages_ % 64)) - 1; // pages past the last are never free
    }
}

int32_t kv_pages::mapped(int32_t slot) const {
    return (slot < 0 || slot >= n_slots()) ? 0 : static_cast<int32_t>(rows_[size_t(slot)].size());
}

int32_t kv_pages::physical(int32_t slot, int32_t logical) const {
    if (logical < 0 || logical >= mapped(slot)) {
        return -1;
    }
    return rows_[size_t(slot)][size_t(logical)];
}

int32_t kv_pages::pages_for(int64_t cells, int32_t page_cells, int32_t n_pages) {
    if (cells <= 0 || page_cells <= 0) {
        return 0;
    }
    const int64_t n = cells / page_cells + (cells % page_cells != 0 ? 1 : 0);
    return static_cast<int32_t>(std::min<int64_t>(n, n_pages));
}

bool kv_pages::take(int32_t slot, int32_t want, std::vector<int32_t> & taken) {
    taken.clear();
    if (slot < 0 || slot >= n_slots() || want > n_pages_) {
        return false;
    }
    const int32_t need = want - mapped(slot);
    if (need <= 0) {
        return true;
    }
    if (need > n_free_) {
        return false;
    }
    // the lowest `need` set bits, word by word, in ascending order
    taken.reserve(size_t(need));
    for (size_t w = 0; w < free_bits_.size() && int32_t(taken.size()) < need; ++w) {
        uint64_t & word = free_bits_[w];
        while (word != 0 && int32_t(taken.size()) < need) {
            const int32_t bit = __builtin_ctzll(word);
            word &= word - 1;
            taken.push_back(int32_t(w) * 64 + bit);
        }
    }
    n_free_ -= need;
    std::vector<int32_t> & row = rows_[size_t(slot)];
    row.insert(row.end(), taken.begin(), taken.end());
    return true;
}

void kv_pages::give(int32_t slot, int32_t keep, std::vector<int32_t> & out) {
    out.clear();
    if (slot < 0 || slot >= n_slots()) {
        return;
    }
    std::vector<int32_t> & row = rows_[size_t(slot)];
    const size_t k = size_t(std::max(0, keep));
    while (row.size() > k) {
        const int32_t p = row.back();
        row.pop_back();
        out.push_back(p);
        free_bits_[size_t(p) / 64] |= uint64_t(1) << (p % 64);
        ++n_free_;
    }
}

int32_t kv_reclaim_victim(const std::vector<kv_slot_view> & s, int32_t for_slot) {
    int32_t best = -1;
    for (size_t i = 0; i < s.size(); ++i) {
        const int32_t si = static_cast<int32_t>(i);
        if (si == for_slot || s[i].active || s[i].pages <= 0) {
            continue;
        }
        if (best < 0 || s[i].released < s[size_t(best)].released) {
            best = si;
        }
    }
    return best;
}

// ---- kv_pool ----

__global__ void zero_pages_kernel(uint8_t * base, const int32_t * pages, int32_t n, int64_t layer_stride,
                                  int64_t page_stride, int32_t chunks_a_page) {
    // one workgroup a (layer, page, 16 KiB chunk); 256 lanes x 4 x 16 B
    const int64_t w = blockIdx.x;
    const int32_t chunk = static_cast<int32_t>(w % chunks_a_page);
    const int64_t lp = w / chunks_a_page;
    const int32_t pi = static_cast<int32_t>(lp % n);
    const int64_t layer = lp / n;
    uint8_t * p = base + layer * layer_stride + int64_t(pages[pi]) * page_stride + int64_t(chunk) * 16384;
    const int64_t lim = page_stride - int64_t(chunk) * 16384;
    const uint4 z = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int32_t r = 0; r < 4; ++r) {
        const int64_t off = int64_t(r * 256 + static_cast<int32_t>(threadIdx.x)) * 16;
        if (off < lim) {
            *reinterpret_cast<uint4 *>(p + off) = z;
        }
    }
}

kv_pool::~kv_pool() { release_all(); }

void kv_pool::release_all() {
    if (base_ != nullptr || table_dev_ != nullptr || stage_dev_ != nullptr || stage_host_ != nullptr ||
        stream_ != nullptr) {
        int32_t cur = 0;
        hipGetDevice(&cur);
        hipSetDevice(device_);
        if (stream_ != nullptr) {
            hipStreamSynchronize(stream_);
            hipStreamDestroy(stream_);
        }
        if (base_ != nullptr) {
            hipFree(base_);
        }
        if (table_dev_ != nullptr) {
            hipFree(table_dev_);
        }
        if (stage_dev_ != nullptr) {
            hipFree(stage_dev_);
        }
        if (stage_host_ != nullptr) {
            hipHostFree(stage_host_);
        }
        hipSetDevice(cur);
    }
    base_ = nullptr;
    table_dev_ = nullptr;
    stage_dev_ = nullptr;
    stage_host_ = nullptr;
    stream_ = nullptr;
}

bool kv_pool::init(int32_t n_slots, int32_t n_pages, int32_t page_cells, int32_t layers, int32_t h_kv,
                   int64_t slot_cells, int32_t device, std::string & err, int32_t format) {
    release_all();
    if (n_slots <= 0 || n_pages <= 0 || layers <= 0 || h_kv <= 0) {
        err = "KV pool: slots, pages, layers and heads must be positive";
        return false;
    }
    if (format != kFormatQ8_0 && format != kFormatKV8) {
        err = "KV pool: unknown code format " + std::to_string(format);
        return false;
    }
    if (page_cells != kPageTokens) {
        err = "KV pool: pages are " + std::to_string(kPageTokens) + " tokens (asked " + std::to_string(page_cells) +
              ")";
        return false;
    }
    const int64_t cap = int64_t(n_pages) * page_cells;
    if (slot_cells <= 0) {
        slot_cells = cap;
    }
    if (slot_cells > cap) {
        err = "KV pool: a slot's range exceeds the pool";
        return false;
    }
    n_slots_ = n_slots;
    format_ = format;
    page_cells_ = page_cells;
    layers_ = layers;
    h_kv_ = h_kv;
    device_ = device;
    slot_cells_ = slot_cells;
    table_stride_ = kv_pages::pages_for(slot_cells, page_cells, n_pages);
    bytes_ = int64_t(layers) * n_pages * h_kv * kPageBlock;
    int32_t cur = 0;
    hipGetDevice(&cur);
    if (hipSetDevice(device) != hipSuccess) {
        err = "KV pool: no device " + std::to_string(device);
        return false;
    }
    bool ok = hipMalloc(&base_, size_t(bytes_)) == hipSuccess;
    ok = ok && hipMalloc(&table_dev_, sizeof(int32_t) * size_t(n_slots) * size_t(table_stride_)) == hipSuccess;
    // the staging of ensure/trim, allocated once: the new pages' list (n_pages entries at most) and a page-table row,
    // pinned on the host and on the device, and the pool's own stream (default priority) that orders their copies
    // and the zeroing kernel
    const size_t stage = sizeof(int32_t) * (size_t(n_pages) + size_t(table_stride_));
    ok = ok && hipMalloc(&stage_dev_, stage) == hipSuccess;
    ok = ok && hipHostMalloc(reinterpret_cast<void **>(&stage_host_), stage, hipHostMallocDefault) == hipSuccess;
    ok = ok && hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking) == hipSuccess;
    if (ok) {
        std::vector<int32_t> none(size_t(n_slots) * size_t(table_stride_), -1);
        ok = hipMemcpy(table_dev_, none.data(), none.size() * sizeof(int32_t), hipMemcpyHostToDevice) == hipSuccess;
    }
    hipSetDevice(cur);
    if (!ok) {
        hipGetLastError();
        release_all();
        err = "KV pool: allocating " + std::to_string(bytes_) + " bytes of HBM failed";
        return false;
    }
    pages_.init(n_slots, n_pages);
    return true;
}

// The new pages' bytes zeroed on the pool's stream: their list copied through the pinned staging (no allocation,
// no host wait here; finish() waits)
bool kv_pool::zero_pages(const std::vector<int32_t> & phys, std::string & err) {
    if (phys.empty()) {
        return true;
    }
    std::copy(phys.begin(), phys.end(), stage_host_);
    bool ok = hipMemcpyAsync(stage_dev_, stage_host_, phys.size() * sizeof(int32_t), hipMemcpyHostToDevice,
                             stream_) == hipSuccess;
    if (ok) {
        const int64_t page_stride = int64_t(h_kv_) * kPageBlock;
        const int32_t chunks = static_cast<int32_t>((page_stride + 16383) / 16384);
        const int64_t grid = int64_t(layers_) * int64_t(phys.size()) * chunks;
        hipLaunchKernelGGL(zero_pages_kernel, dim3(static_cast<uint32_t>(grid)), dim3(256), 0, stream_, base_,
                           stage_dev_, static_cast<int32_t>(phys.size()), int64_t(pages_.n_pages()) * page_stride,
                           page_stride, chunks);
        ok = hipGetLastError() == hipSuccess;
    }
    if (!ok) {
        err = "KV pool: zeroing new pages failed";
    }
    return ok;
}

// The slot's page-table row (its mapped pages, then -1) written on the pool's stream after the zeroing it follows
bool kv_pool::upload_table(int32_t slot, std::string & err) {
    int32_t * row = stage_host_ + pages_.n_pages();
    const std::vector<int32_t> & t = pages_.table(slot);
    std::fill(row, row + table_stride_, -1);
    std::copy(t.begin(), t.end(), row);
    if (hipMemcpyAsync(table_dev_ + int64_t(slot) * table_stride_, row, size_t(table_stride_) * sizeof(int32_t),
                       hipMemcpyHostToDevice, stream_) != hipSuccess) {
        err = "KV pool: page table upload failed";
        return false;
    }
    return true;
}

// ensure/trim are synchronous, as the reference's are: the pool's stream drained before they return, so work the
// caller enqueues afterwards on any stream sees the zeroed pages and the new table row
bool kv_pool::finish(std::string & err) {
    if (hipStreamSynchronize(stream_) != hipSuccess) {
        hipGetLastError();
        err = "KV pool: page setup failed on the device";
        return false;
    }
    return true;
}

bool kv_pool::ensure(int32_t slot, int64_t cells, std::string & err, bool * capacity) {
    if (capacity != nullptr) {
        *capacity = false;
    }
    if (base_ == nullptr || slot < 0 || slot >= n_slots_) {
        err = "KV pool: no slot " + std::to_string(slot);
        return false;
    }
    const int32_t first = pages_.mapped(slot);
    const int32_t want = kv_pages::pages_for(std::min<int64_t>(cells, slot_cells_), page_cells_, pages_.n_pages());
    if (want <= first) {
        return true;
    }
    std::vector<int32_t> taken;
    if (!pages_.take(slot, want, taken)) {
        if (capacity != nullptr) {
            *capacity = true;
        }
        err = "KV pool: slot " + std::to_string(slot) + " needs " + std::to_string(want - first) + " more pages of " +
              std::to_string(page_cells_) + " cells for " + std::to_string(cells) + " cells; " +
              std::to_string(pages_.free_pages()) + " of " + std::to_string(pages_.n_pages()) + " are free";
        return false;
    }
    int32_t cur = 0;
    hipGetDevice(&cur);
    hipSetDevice(device_);
    bool ok = true;
    if (fail_after_ >= 0) {
        // TEST ONLY: the transaction fails after readying fail_after_ of its new pages
        std::vector<int32_t> part(taken.begin(), taken.begin() + std::min<size_t>(size_t(fail_after_), taken.size()));
        zero_pages(part, err);
        finish(err);
        fail_after_ = -1;
        err = "KV pool: page setup (TEST: an injected failure)";
        ok = false;
    } else {
        ok = zero_pages(taken, err) && upload_table(slot, err);
        ok = finish(err) && ok;
    }
    if (!ok) {
        std::string e2;
        finish(e2); // the staging is free again
        std::vector<int32_t> back;
        pages_.give(slot, first, back);
        upload_table(slot, e2) && finish(e2);
    }
    hipSetDevice(cur);
    return ok;
}

bool kv_pool::trim(int32_t slot, int64_t keep_cells, std::string & err) {
    if (base_ == nullptr || slot < 0 || slot >= n_slots_) {
        err = "KV pool: no slot " + std::to_string(slot);
        return false;
    }
    const int32_t keep = kv_pages::pages_for(keep_cells, page_cells_, pages_.n_pages());
    std::vector<int32_t> out;
    pages_.give(slot, keep, out);
    int32_t cur = 0;
    hipGetDevice(&cur);
    hipSetDevice(device_);
    const bool ok = upload_table(slot, err) && finish(err);
    hipSetDevice(cur);
    return ok;
}

std::vector<std::string> kv_pool::ledger() const {
    std::vector<std::string> out;
    char b[512];
    snprintf(b, sizeof b,
             "KV pool: %d pages of %d cells (%lld cells shared by %d slots; a slot's logical range %lld cells); "
             "%d layers x %d KV heads of %s K and V, %lld bytes a page, %.3f GiB of HBM on device %d",
             pages_.n_pages(), page_cells_, static_cast<long long>(capacity_cells()), n_slots_,
             static_cast<long long>(slot_cells_), layers_, h_kv_, format_ == kFormatKV8 ? "KV8 (group 64)" : "Q8_0",
             static_cast<long long>(int64_t(layers_) * h_kv_ * kPageBlock), double(bytes_) / 1073741824.0, device_);
    out.emplace_back(b);
    snprintf(b, sizeof b, "KV pool: page table %d slots x %d entries (int32); %d of %d pages free", n_slots_,
             table_stride_, pages_.free_pages(), pages_.n_pages());
    out.emplace_back(b);
    return out;
}

pool_view kv_pool::view() const {
    pool_view v;
    v.base = base_;
    v.table = table_dev_;
    v.page_stride = int64_t(h_kv_) * kPageBlock;
    v.layer_stride = int64_t(pages_.n_pages()) * v.page_stride;
    v.table_stride = table_stride_;
    v.h_kv = h_kv_;
    v.format = format_;
    return v;
}

} // namespace fnkv

struct fnkv_pool {
    fnkv::kv_pool p;
};

using fnkv::set_error;

extern "C" {

const char * fnkv_last_error(void) { return fnkv::last_error(); }

int32_t fnkv_pages_for(int64_t cells, int32_t page_cells, int32_t n_pages) {
    return fnkv::kv_pages::pages_for(cells, page_cells, n_pages);
}

int32_t fnkv_reclaim_victim(const fnkv_slot_view * views, int32_t n, int32_t for_slot) {
    std::vector<fnkv::kv_slot_view> v(size_t(std::max(0, n)));
    for (int32_t i = 0; i < n; ++i) {
        v[size_t(i)].active = views[i].active != 0;
        v[size_t(i)].pages = views[i].pages;
        v[size_t(i)].released = views[i].released;
    }
    return fnkv::kv_reclaim_victim(v, for_slot);
}

int fnkv_pool_create(int32_t n_slots, int32_t n_pages, int32_t page_tokens, int32_t layers, int32_t h_kv,
                     int64_t slot_tokens, int32_t device, fnkv_pool ** out) {
    return fnkv_pool_create_fmt(n_slots, n_pages, page_tokens, layers, h_kv, slot_tokens, FNKV_FMT_Q8_0, device, out);
}

int fnkv_pool_create_fmt(int32_t n_slots, int32_t n_pages, int32_t page_tokens, int32_t layers, int32_t h_kv,
                         int64_t slot_tokens, int32_t format, int32_t device, fnkv_pool ** out) {
    if (out == nullptr) {
        set_error("fnkv_pool_create: null out");
        return FNKV_ERR_ARG;
    }
    *out = nullptr;
    fnkv_pool * p = new fnkv_pool;
    std::string err;
    if (!p->p.init(n_slots, n_pages, page_tokens, layers, h_kv, slot_tokens, device, err, format)) {
        delete p;
        set_error(err);
        return err.find("HBM") != std::string::npos ? FNKV_ERR_HIP : FNKV_ERR_ARG;
    }
    if (!fnkv::scratch_init(device, err)) {
        delete p;
        set_error(err);
        return FNKV_ERR_HIP;
    }
    *out = p;
    return FNKV_OK;
}

void fnkv_pool_destroy(fnkv_pool * pool) {
    if (pool != nullptr) {
        fnkv::scratch_release(&pool->p);
    }
    delete pool;
}

int32_t fnkv_pool_format(const fnkv_pool * pool) { return pool == nullptr ? -1 : pool->p.format(); }

int fnkv_pool_ensure(fnkv_pool * pool, int32_t slot, int64_t cells, int32_t * capacity) {
    if (capacity != nullptr) {
        *capacity = 0;
    }
    if (pool == nullptr) {
        set_error("fnkv_pool_ensure: null pool");
        return FNKV_ERR_ARG;
    }
    std::string err;
    bool cap = false;
    if (pool->p.ensure(slot, cells, err, &cap)) {
        return FNKV_OK;
    }
    set_error(err);
    if (capacity != nullptr) {
        *capacity = cap ? 1 : 0;
    }
    if (cap) {
        return FNKV_ERR_CAPACITY;
    }
    return (slot < 0 || slot >= pool->p.pages().n_slots()) ? FNKV_ERR_ARG : FNKV_ERR_HIP;
}

int fnkv_pool_trim(fnkv_pool * pool, int32_t slot, int64_t keep_cells) {
    if (pool == nullptr) {
        set_error("fnkv_pool_trim: null pool");
        return FNKV_ERR_ARG;
    }
    std::string err;
    if (pool->p.trim(slot, keep_cells, err)) {
        return FNKV_OK;
    }
    set_error(err);
    return (slot < 0 || slot >= pool->p.pages().n_slots()) ? FNKV_ERR_ARG : FNKV_ERR_HIP;
}

int64_t fnkv_pool_mapped_cells(const fnkv_pool * pool, int32_t slot) {
    return pool == nullptr ? 0 : pool->p.mapped_cells(slot);
}
int32_t fnkv_pool_free_pages(const fnkv_pool * pool) { return pool == nullptr ? 0 : pool->p.pages().free_pages(); }
int32_t fnkv_pool_n_pages(const fnkv_pool * pool) { return pool == nullptr ? 0 : pool->p.pages().n_pages(); }
int32_t fnkv_pool_mapped_pages(const fnkv_pool * pool, int32_t slot) {
    return pool == nullptr ? 0 : pool->p.pages().mapped(slot);
}
int32_t fnkv_pool_physical(const fnkv_pool * pool, int32_t slot, int32_t logical) {
    return pool == nullptr ? -1 : pool->p.pages().physical(slot, logical);
}

int32_t fnkv_page_table(const fnkv_pool * pool, int32_t slot, int32_t * out, int32_t cap) {
    if (pool == nullptr || slot < 0 || slot >= pool->p.pages().n_slots()) {
        return 0;
    }
    const std::vector<int32_t> & t = pool->p.pages().table(slot);
    const int32_t n = static_cast<int32_t>(t.size());
    for (int32_t i = 0; i < n && i < cap && out != nullptr; ++i) {
        out[i] = t[size_t(i)];
    }
    return n;
}

int32_t fnkv_pool_ledger(const fnkv_pool * pool, char * buf, int32_t cap) {
    if (pool == nullptr || buf == nullptr || cap <= 0) {
        return 0;
    }
    std::string all;
    for (const std::string & l : pool->p.ledger()) {
        all += l;
        all += '\n';
    }
    const int32_t n = static_cast<int32_t>(std::min<size_t>(all.size(), size_t(cap - 1)));
    std::memcpy(buf, all.data(), size_t(n));
    buf[n] = '\0';
    return n;
}

void fnkv_pool_test_fail(fnkv_pool * pool, int32_t after) {
    if (pool != nullptr) {
        pool->p.test_fail(after);
    }
}

int64_t fnkv_page_block_bytes(void) { return fnkv::kPageBlock; }
void * fnkv_pool_device_base(const fnkv_pool * pool) { return pool == nullptr ? nullptr : pool->p.device_base(); }
int64_t fnkv_pool_device_bytes(const fnkv_pool * pool) { return pool == nullptr ? 0 : pool->p.device_bytes(); }

} // extern "C"

namespace fnkv {
const kv_pool * pool_of(const fnkv_pool * p) { return p == nullptr ? nullptr : &p->p; }
} // namespace fnkv
