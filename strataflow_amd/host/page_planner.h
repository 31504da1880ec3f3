// page_planner.h - host bookkeeping of the paged KV cache (pure C++, no HIP).
//
// KvStore answers the same questions as the reference's sf::KvStore
// (src/kv/kv_store.h:30-95): fill position, n_ctx bound, the resident window W
// and which absolute position a write at `pos` pushes out of it.  PagePlanner
// lifts that to pages: every sequence owns a page table (logical page ->
// device page id, cold page id or none), device pages come from one pool
// shared by all sequences in a seeded order, and a page whose last position
// leaves the window is either moved to the host cold pool (lossless, the
// reference semantics: engine.cpp:2620-2661 copies the evicted column to the
// RAM cold store before the write) or dropped (opt-in sliding window, whose
// attention never reads it again).  The planner only decides; the caller
// executes the returned actions (copies, waits, table edits) in order.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

namespace sfa {

class KvStore {
public:
    // window == 0 or window >= n_ctx means full residency (no paging).
    KvStore(uint32_t n_ctx, uint64_t bytes_per_token, uint32_t window = 0);

    bool advance(uint32_t n_tokens);  // false (and no change) past n_ctx
    void reset() { used_ = 0; }
    bool can_fit(uint32_t n_tokens) const { return uint64_t(used_) + n_tokens <= n_ctx_; }
    uint32_t used() const { return used_; }
    uint32_t capacity() const { return n_ctx_; }
    uint64_t bytes() const { return uint64_t(used_) * bytes_per_token_; }

    uint32_t window() const { return window_; }
    bool paging() const { return window_ < n_ctx_; }
    uint32_t ring_col(uint32_t pos) const { return pos % window_; }
    // positions of 0..pos held in the window / pushed out of it
    uint32_t resident_count(uint32_t pos) const { return pos + 1 < window_ ? pos + 1 : window_; }
    uint32_t cold_count(uint32_t pos) const { return pos + 1 - resident_count(pos); }
    // true when writing `pos` pushes absolute position *evicted out of the window
    bool evicts(uint32_t pos, uint32_t *evicted) const;

private:
    uint32_t n_ctx_;
    uint64_t bytes_per_token_;
    uint32_t window_;
    uint32_t used_ = 0;
};

// With deferred eviction (PagePlanner's async_evict) a page that leaves the
// window is copied to its cold page while its table slot still names the device
// page (the data is the same, and attention may read either); kRetire later
// points the slot at the cold page and frees the device page, once the copy is
// known complete (retire_completed) or, when an allocation needs the page,
// at once with `wait` set: the caller then orders its later work after that
// copy.  Without it, kEvict edits the slot and frees the page immediately.
struct PageAction {
    enum Kind : int { kAlloc = 0, kEvict = 1, kDrop = 2, kRetire = 3 };
    Kind kind;
    int32_t seq;
    int32_t lpage;    // logical page of the sequence
    int32_t dev;      // device page (allocated, or released by kEvict / kDrop / kRetire)
    int32_t cold;     // cold page written by kEvict / named by kRetire, else -1
    uint64_t evict;   // kEvict / kRetire: the eviction's serial number
    bool wait;        // kRetire: the copy may still be in flight
    bool edit;        // the action changes the table slot (seq, lpage)
};

struct PlannerStats {
    int64_t allocated = 0;   // device pages handed out
    int64_t evicted = 0;     // pages moved to the cold pool
    int64_t dropped = 0;     // pages released without a copy (sliding window)
    int64_t dev_in_use = 0;  // device pages held (evictions in flight included)
    int64_t cold_in_use = 0;
    int64_t in_flight = 0;   // evictions whose device page is not yet retired
};

class PagePlanner {
public:
    // keep_cold: lossless (evicted pages go to the cold pool) vs sliding window
    // (evicted pages are dropped).  A sequence holds at most
    // ceil(window / page_size) + 1 device pages.
    PagePlanner(int n_seq, int page_size, uint32_t n_ctx, uint32_t window, int n_pages,
                int n_cold_pages, bool keep_cold, uint64_t seed, bool async_evict = false);

    // Plans writing positions [used, used + n_tok) of sequence `seq`, in order,
    // and advances its KvStore.  n_tok <= page_size.  Returns 0 or an sf_status
    // code (1 invalid argument, 4 out of memory).  On error the planner may be
    // partly advanced: callers restore a copy taken before (see plan_step).
    int plan(int seq, int n_tok, std::vector<PageAction> *actions);

    // plan() for every sequence of a step (n_tok[n_seq]), all or nothing: on
    // any error, an exception included, the planner is left as it was and
    // `actions` as it came in.  Never throws.
    int plan_step(const int32_t *n_tok, std::vector<PageAction> *actions) noexcept;

    // Retires the `n` oldest evictions in flight (their copies are known
    // complete): kRetire actions without wait.
    void retire_completed(int n, std::vector<PageAction> *actions);

    // Releases every page of a sequence and rewinds it to position 0.  A page
    // whose eviction is still in flight stays held until it is retired.
    void reset(int seq, std::vector<PageAction> *actions);

    // Serial numbers of the evictions in flight, oldest first.
    std::vector<uint64_t> in_flight() const;

    int n_seq() const { return (int)stores_.size(); }
    int page_size() const { return page_size_; }
    int max_pages() const { return max_pages_; }
    const KvStore &store(int seq) const { return stores_[seq]; }
    // [n_seq][max_pages]: id >= 0 device page, <= -2 cold page (-2 - id), -1 none
    const std::vector<int32_t> &table() const { return table_; }
    const PlannerStats &stats() const { return stats_; }
    // first position the sequence attends under the sliding window (0 when lossless)
    uint32_t attend_lo(int seq) const;

private:
    struct Pending {
        int32_t seq, lpage, dev, cold;
        uint64_t evict;
        bool orphan;  // the sequence was reset: no table edit at retirement
    };

    int32_t take_device_page(std::vector<PageAction> *actions);
    int32_t take_cold_page();
    uint64_t next_random();
    void retire_front(bool wait, std::vector<PageAction> *actions);

    int page_size_;
    int max_pages_;
    bool keep_cold_;
    bool async_;
    uint64_t next_evict_ = 0;
    std::vector<Pending> pending_;  // evictions in flight, oldest first
    std::vector<KvStore> stores_;
    std::vector<int32_t> table_;
    std::vector<int32_t> free_dev_;
    std::vector<int32_t> free_cold_;
    uint64_t rng_;
    PlannerStats stats_;
};

}  // namespace sfa
