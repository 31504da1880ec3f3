// page_planner.cpp - see page_planner.h.
#include "page_planner.h"

namespace sfa {

KvStore::KvStore(uint32_t n_ctx, uint64_t bytes_per_token, uint32_t window)
    : n_ctx_(n_ctx), bytes_per_token_(bytes_per_token),
      window_(window == 0 || window > n_ctx ? n_ctx : window) {}

bool KvStore::advance(uint32_t n_tokens) {
    if (!can_fit(n_tokens)) return false;
    used_ += n_tokens;
    return true;
}

bool KvStore::evicts(uint32_t pos, uint32_t *evicted) const {
    if (pos < window_) return false;
    if (evicted) *evicted = pos - window_;
    return true;
}

PagePlanner::PagePlanner(int n_seq, int page_size, uint32_t n_ctx, uint32_t window, int n_pages,
                         int n_cold_pages, bool keep_cold, uint64_t seed, bool async_evict)
    : page_size_(page_size),
      max_pages_((int)((n_ctx + (uint32_t)page_size - 1) / (uint32_t)page_size)),
      keep_cold_(keep_cold),
      async_(async_evict && keep_cold),
      rng_(seed) {
    stores_.reserve(n_seq);
    for (int b = 0; b < n_seq; ++b) stores_.emplace_back(n_ctx, 0, window);
    table_.assign((std::size_t)n_seq * max_pages_, -1);
    // free lists are stacks; handing out pages from a seeded random slot
    // scatters logical pages over the pool
    free_dev_.reserve(n_pages);
    for (int i = n_pages - 1; i >= 0; --i) free_dev_.push_back(i);
    free_cold_.reserve(n_cold_pages);
    for (int i = n_cold_pages - 1; i >= 0; --i) free_cold_.push_back(i);
}

uint64_t PagePlanner::next_random() {
    // splitmix64
    uint64_t z = (rng_ += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void PagePlanner::retire_front(bool wait, std::vector<PageAction> *actions) {
    const Pending pd = pending_.front();
    actions->push_back({PageAction::kRetire, pd.seq, pd.lpage, pd.dev, pd.cold, pd.evict, wait, !pd.orphan});
    pending_.erase(pending_.begin());
    if (!pd.orphan) table_[(std::size_t)pd.seq * max_pages_ + pd.lpage] = -2 - pd.cold;
    free_dev_.push_back(pd.dev);
    --stats_.dev_in_use;
    --stats_.in_flight;
}

void PagePlanner::retire_completed(int n, std::vector<PageAction> *actions) {
    for (int i = 0; i < n && !pending_.empty(); ++i) retire_front(false, actions);
}

std::vector<uint64_t> PagePlanner::in_flight() const {
    std::vector<uint64_t> out;
    out.reserve(pending_.size());
    for (const Pending &pd : pending_) out.push_back(pd.evict);
    return out;
}

int32_t PagePlanner::take_device_page(std::vector<PageAction> *actions) {
    // no free page: the oldest eviction in flight gives its page up now (the
    // caller waits for that copy before the page is written)
    if (free_dev_.empty() && !pending_.empty()) retire_front(true, actions);
    if (free_dev_.empty()) return -1;
    const size_t i = (std::size_t)(next_random() % free_dev_.size());
    const int32_t id = free_dev_[i];
    free_dev_[i] = free_dev_.back();
    free_dev_.pop_back();
    return id;
}

int32_t PagePlanner::take_cold_page() {
    if (free_cold_.empty()) return -1;
    const int32_t id = free_cold_.back();
    free_cold_.pop_back();
    return id;
}

uint32_t PagePlanner::attend_lo(int seq) const {
    const KvStore &st = stores_[seq];
    if (keep_cold_ || !st.paging() || st.used() == 0) return 0;
    const uint32_t pos = st.used() - 1;
    return pos + 1 > st.window() ? pos + 1 - st.window() : 0;
}

int PagePlanner::plan(int seq, int n_tok, std::vector<PageAction> *actions) {
    if (seq < 0 || seq >= (int)stores_.size() || n_tok < 0 || n_tok > page_size_) return 1;
    KvStore &st = stores_[seq];
    if (!st.can_fit((uint32_t)n_tok)) return 1;
    const uint32_t P = (uint32_t)page_size_;
    int32_t *row = &table_[(std::size_t)seq * max_pages_];

    // replay the step on counters first, so a step that would run out of
    // pages changes nothing (a page evicted at one position is reusable by an
    // allocation at a later position of the same step)
    {
        // pages of evictions in flight count as free: an allocation retires them
        int64_t dev_free = (int64_t)(free_dev_.size() + pending_.size());
        int64_t cold_free = (int64_t)free_cold_.size();
        for (uint32_t pos = st.used(); pos < st.used() + (uint32_t)n_tok; ++pos) {
            uint32_t e;
            if (st.evicts(pos, &e) && e % P == P - 1 && row[e / P] >= 0) {
                ++dev_free;
                if (keep_cold_ && --cold_free < 0) return 4;
            }
            if (pos % P == 0 && row[pos / P] == -1 && --dev_free < 0) return 4;
        }
    }

    for (uint32_t pos = st.used(); pos < st.used() + (uint32_t)n_tok; ++pos) {
        uint32_t e;
        // the write of `pos` pushes position e out of the window; when e
        // closes its page, the whole page has left the window
        if (st.evicts(pos, &e) && e % P == P - 1 && row[e / P] >= 0) {
            const int32_t lp = (int32_t)(e / P);
            const int32_t dev = row[lp];
            if (keep_cold_) {
                const int32_t c = take_cold_page();
                const uint64_t id = next_evict_++;
                actions->push_back({PageAction::kEvict, seq, lp, dev, c, id, false, !async_});
                ++stats_.evicted;
                ++stats_.cold_in_use;
                if (async_) {
                    // the slot keeps the device page until the copy is retired
                    pending_.push_back({seq, lp, dev, c, id, false});
                    ++stats_.in_flight;
                } else {
                    row[lp] = -2 - c;
                    free_dev_.push_back(dev);
                    --stats_.dev_in_use;
                }
            } else {
                actions->push_back({PageAction::kDrop, seq, lp, dev, -1, 0, false, true});
                row[lp] = -1;
                ++stats_.dropped;
                free_dev_.push_back(dev);
                --stats_.dev_in_use;
            }
        }
        if (pos % P == 0 && row[pos / P] == -1) {
            const int32_t dev = take_device_page(actions);
            actions->push_back({PageAction::kAlloc, seq, (int32_t)(pos / P), dev, -1, 0, false, true});
            row[pos / P] = dev;
            ++stats_.allocated;
            ++stats_.dev_in_use;
        }
    }
    st.advance((uint32_t)n_tok);
    return 0;
}

int PagePlanner::plan_step(const int32_t *n_tok, std::vector<PageAction> *actions) noexcept {
    try {
        const size_t n0 = actions->size();
        PagePlanner saved = *this;
        for (int b = 0; b < n_seq(); ++b) {
            int rc;
            try {
                rc = plan(b, n_tok[b], actions);
            } catch (...) {
                rc = 4;
            }
            if (rc != 0) {
                *this = std::move(saved);
                actions->resize(n0);
                return rc;
            }
        }
        return 0;
    } catch (...) {  // the snapshot itself could not be taken: nothing changed
        return 4;
    }
}

void PagePlanner::reset(int seq, std::vector<PageAction> *actions) {
    if (seq < 0 || seq >= (int)stores_.size()) return;
    int32_t *row = &table_[(std::size_t)seq * max_pages_];
    for (int lp = 0; lp < max_pages_; ++lp) {
        const int32_t id = row[lp];
        Pending *pd = nullptr;
        if (id >= 0)
            for (Pending &q : pending_)
                if (!q.orphan && q.seq == seq && q.lpage == lp) pd = &q;
        if (pd != nullptr) {
            // the copy is in flight: its cold page is released now (a later
            // copy into it is ordered after this one), the device page at
            // retirement, without a table edit
            pd->orphan = true;
            free_cold_.push_back(pd->cold);
            --stats_.cold_in_use;
        } else if (id >= 0) {
            free_dev_.push_back(id);
            --stats_.dev_in_use;
            actions->push_back({PageAction::kDrop, seq, lp, id, -1, 0, false, true});
        } else if (id <= -2) {
            free_cold_.push_back(-2 - id);
            --stats_.cold_in_use;
        }
        row[lp] = -1;
    }
    stores_[seq].reset();
}

}  // namespace sfa
