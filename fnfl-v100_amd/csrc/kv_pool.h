// The host side of the pool: the page book (fn/model/kv_pool.h:31-51 kv_pages), the reclaim choice
// (kv_pool.h:56-61) and the pool itself (kv_pool.h:63-138), re-designed for one MI355X: instead of mapping physical
// pages into per-slot virtual ranges (the reference's CUDA VMM, kv_pool.cpp:393-446), the pool is one HBM allocation
// of physical pages and every slot has a row of an int32 page table that the kernels gather through.
#pragma once

#include "layout.h"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

namespace fnkv {

// The page book: physical pages 0 .. n_pages - 1, each slot's logical pages in order (its page-table row), and the
// free pages as a bitset (bit p of word p / 64 set when page p is free), so taking the lowest free pages is a scan of
// set bits and returning pages is setting them: O(n_pages / 64) a call. The rule the reference's KATs pin is the
// order: take hands out the lowest free pages in ascending order, give returns a slot's pages last first.
class kv_pages {
  public:
    void init(int32_t n_slots, int32_t n_pages);
    int32_t n_slots() const { return static_cast<int32_t>(rows_.size()); }
    int32_t n_pages() const { return n_pages_; }
    int32_t free_pages() const { return n_free_; }
    int32_t mapped(int32_t slot) const;
    int32_t physical(int32_t slot, int32_t logical) const; // -1 when not mapped
    static int32_t pages_for(int64_t cells, int32_t page_cells, int32_t n_pages);
    // the slot's next want - mapped(slot) pages, lowest free first; false with nothing taken when they do not fit
    bool take(int32_t slot, int32_t want, std::vector<int32_t> & taken);
    // the slot's logical pages keep .. mapped - 1 back to the free set, last first (out in that order)
    void give(int32_t slot, int32_t keep, std::vector<int32_t> & out);
    const std::vector<int32_t> & table(int32_t slot) const { return rows_[size_t(slot)]; }

  private:
    int32_t n_pages_ = 0, n_free_ = 0;
    std::vector<std::vector<int32_t>> rows_; // each slot's physical page a logical page
    std::vector<uint64_t> free_bits_;
};

struct kv_slot_view {
    bool active = false;
    int32_t pages = 0;
    uint64_t released = 0;
};
int32_t kv_reclaim_victim(const std::vector<kv_slot_view> & s, int32_t for_slot);

class kv_pool {
  public:
    kv_pool() = default;
    ~kv_pool();
    kv_pool(const kv_pool &) = delete;
    kv_pool & operator=(const kv_pool &) = delete;

    bool init(int32_t n_slots, int32_t n_pages, int32_t page_cells, int32_t layers, int32_t h_kv, int64_t slot_cells,
              int32_t device, std::string & err, int32_t format = kFormatQ8_0);
    bool ensure(int32_t slot, int64_t cells, std::string & err, bool * capacity = nullptr);
    bool trim(int32_t slot, int64_t keep_cells, std::string & err);
    int64_t mapped_cells(int32_t slot) const { return int64_t(pages_.mapped(slot)) * page_cells_; }
    int64_t capacity_cells() const { return int64_t(pages_.n_pages()) * page_cells_; }
    int64_t slot_cells() const { return slot_cells_; }
    const kv_pages & pages() const { return pages_; }
    int32_t page_cells() const { return page_cells_; }
    int32_t layers() const { return layers_; }
    int32_t h_kv() const { return h_kv_; }
    int32_t device() const { return device_; }
    int32_t format() const { return format_; }
    int64_t device_bytes() const { return bytes_; }
    uint8_t * device_base() const { return base_; }
    std::vector<std::string> ledger() const;
    void test_fail(int32_t after) { fail_after_ = after; }
    pool_view view() const;

  private:
    bool zero_pages(const std::vector<int32_t> & phys, std::string & err);
    bool upload_table(int32_t slot, std::string & err);
    bool finish(std::string & err);
    void release_all();

    int32_t n_slots_ = 0, page_cells_ = 0, layers_ = 0, h_kv_ = 0, device_ = 0, table_stride_ = 0;
    int32_t format_ = kFormatQ8_0;
    int64_t slot_cells_ = 0, bytes_ = 0;
    uint8_t * base_ = nullptr;
    int32_t * table_dev_ = nullptr;
    int32_t * stage_dev_ = nullptr;  // ensure's staging: n_pages page ids, then one table row
    int32_t * stage_host_ = nullptr; // pinned, the same layout
    hipStream_t stream_ = nullptr;   // the pool's own stream (default priority)
    kv_pages pages_;
    int32_t fail_after_ = -1;
};

// The no-allocation decode's device scratch (decode.hip). scratch_init looks its address up on `device` (once per
// device, at pool creation, so that no lookup ever runs under stream capture); scratch_release gives up `pool`'s claim
// on its device's scratch (after the device has drained), when the pool is destroyed.
bool scratch_init(int32_t device, std::string & err);
void scratch_release(const kv_pool * pool);

} // namespace fnkv
