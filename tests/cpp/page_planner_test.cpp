// CPU unit test of the host page bookkeeping (strataflow_amd/host/page_planner.*).
// Built and run by tests/test_page_planner.py with g++; prints "ok <n>" on success.
//
// Pins KvStore to the reference's window arithmetic (src/kv/kv_store.h:30-95:
// W = min(window, n_ctx) with 0 meaning n_ctx, resident = min(pos+1, W),
// evicted position = pos - W once pos >= W) and the planner's page invariants:
// every position a sequence has written is reachable through its table
// (device page while its page overlaps the last W positions, cold page after,
// or released under the sliding window), pages are never shared, the pool is
// never exceeded, placement is a function of the seed, and a step that runs out
// of pages changes nothing.
#include <cstdio>
#include <cstdlib>
#include <new>
#include <set>
#include <vector>

#include "page_planner.h"

// Allocation failure injection for the all-or-nothing checks: when
// g_fail_countdown reaches zero, the next operator new throws.
static long g_fail_countdown = -1;

void *operator new(std::size_t n) {
    if (g_fail_countdown >= 0 && g_fail_countdown-- == 0) throw std::bad_alloc();
    if (void *p = std::malloc(n ? n : 1)) return p;
    throw std::bad_alloc();
}
void operator delete(void *p) noexcept { std::free(p); }
void operator delete(void *p, std::size_t) noexcept { std::free(p); }

static int g_checks = 0;
#define CHECK(c)                                                              \
    do {                                                                      \
        ++g_checks;                                                           \
        if (!(c)) {                                                           \
            std::fprintf(stderr, "%s:%d: CHECK(%s) failed\n", __FILE__, __LINE__, #c); \
            std::exit(1);                                                     \
        }                                                                     \
    } while (0)

using sfa::KvStore;
using sfa::PageAction;
using sfa::PagePlanner;

static void test_kv_store() {
    KvStore full(64, 10);  // window 0 -> n_ctx
    CHECK(full.window() == 64 && !full.paging());
    CHECK(full.resident_count(63) == 64 && full.cold_count(63) == 0);
    uint32_t e = 12345;
    CHECK(!full.evicts(63, &e) && e == 12345);
    CHECK(full.advance(60) && full.used() == 60 && full.bytes() == 600);
    CHECK(full.can_fit(4) && !full.can_fit(5));
    CHECK(!full.advance(5) && full.used() == 60);  // refused, unchanged
    full.reset();
    CHECK(full.used() == 0);

    KvStore big(64, 1, 1000);  // window above n_ctx -> n_ctx
    CHECK(big.window() == 64 && !big.paging());

    KvStore w(64, 1, 4);
    CHECK(w.window() == 4 && w.paging());
    CHECK(w.ring_col(0) == 0 && w.ring_col(5) == 1 && w.ring_col(63) == 3);
    CHECK(w.resident_count(0) == 1 && w.resident_count(3) == 4 && w.resident_count(40) == 4);
    CHECK(w.cold_count(3) == 0 && w.cold_count(4) == 1 && w.cold_count(40) == 37);
    CHECK(!w.evicts(3, &e));
    CHECK(w.evicts(4, &e) && e == 0);
    CHECK(w.evicts(40, &e) && e == 36);
}

// Checks one sequence's table against its fill position.
static void check_table(const PagePlanner &pl, int seq, uint32_t window, bool keep_cold) {
    const int P = pl.page_size();
    const uint32_t used = pl.store(seq).used();
    const int32_t *row = &pl.table()[(size_t)seq * pl.max_pages()];
    const uint32_t n_pages_used = (used + P - 1) / P;
    for (int lp = 0; lp < pl.max_pages(); ++lp) {
        const int32_t id = row[lp];
        if ((uint32_t)lp >= n_pages_used) {
            CHECK(id == -1);
            continue;
        }
        // the page is resident iff its last position is still inside the window
        const uint32_t last = (uint32_t)(lp + 1) * P - 1;
        const bool in_window = used == 0 || last + window >= used;  // last >= used - window
        if (in_window) {
            CHECK(id >= 0);
        } else if (keep_cold) {
            CHECK(id <= -2);
        } else {
            CHECK(id == -1);
        }
    }
}

static void test_planner_lossless(bool keep_cold) {
    const int n_seq = 3, P = 32;
    const uint32_t n_ctx = 1024, W = 100;  // window not a page multiple
    const int win_pages = (W + P - 1) / P + 1;
    const int n_pages = n_seq * win_pages;
    PagePlanner pl(n_seq, P, n_ctx, W, n_pages, keep_cold ? n_seq * 32 : 0, keep_cold, 7);
    std::vector<PageAction> acts;
    int64_t evicted = 0, dropped = 0, allocated = 0;
    // ragged steps: sequence b takes (b + 1) * 7 % 33 tokens per step
    for (int step = 0; step < 120; ++step) {
        for (int b = 0; b < n_seq; ++b) {
            const int n = ((b + 1) * 7 + step) % 33;
            if (!pl.store(b).can_fit(n)) continue;
            acts.clear();
            CHECK(pl.plan(b, n, &acts) == 0);
            for (const PageAction &a : acts) {
                if (a.kind == PageAction::kAlloc) ++allocated;
                if (a.kind == PageAction::kEvict) {
                    ++evicted;
                    CHECK(a.cold >= 0);
                }
                if (a.kind == PageAction::kDrop) ++dropped;
                CHECK(a.seq == b && a.dev >= 0 && a.dev < n_pages);
            }
            check_table(pl, b, W, keep_cold);
        }
        // no device page is shared and the pool is never exceeded
        std::set<int32_t> dev, cold;
        for (int32_t id : pl.table()) {
            if (id >= 0) CHECK(dev.insert(id).second);
            if (id <= -2) CHECK(cold.insert(id).second);
        }
        CHECK((int)dev.size() <= n_pages);
        CHECK((int64_t)dev.size() == pl.stats().dev_in_use);
        CHECK((int64_t)cold.size() == pl.stats().cold_in_use);
    }
    CHECK(allocated == pl.stats().allocated && evicted == pl.stats().evicted &&
          dropped == pl.stats().dropped);
    CHECK(keep_cold ? (evicted > 0 && dropped == 0) : (dropped > 0 && evicted == 0));
    // each sequence holds at most ceil(W / P) + 1 device pages
    for (int b = 0; b < n_seq; ++b) {
        int held = 0;
        for (int lp = 0; lp < pl.max_pages(); ++lp) held += pl.table()[(size_t)b * pl.max_pages() + lp] >= 0;
        CHECK(held <= win_pages);
    }
    // attend_lo: 0 when lossless, used - W under the window
    for (int b = 0; b < n_seq; ++b) {
        const uint32_t used = pl.store(b).used();
        CHECK(pl.attend_lo(b) == (keep_cold || used <= W ? 0u : used - W));
    }
}

static void test_no_paging_when_window_covers_ctx() {
    PagePlanner pl(2, 32, 256, 0, 16, 0, true, 1);
    std::vector<PageAction> acts;
    for (int i = 0; i < 8; ++i)
        for (int b = 0; b < 2; ++b) CHECK(pl.plan(b, 32, &acts) == 0);
    CHECK(pl.stats().evicted == 0 && pl.stats().dropped == 0 && pl.stats().allocated == 16);
    CHECK(pl.plan(0, 1, &acts) == 1);  // past n_ctx
}

static void test_seeded_placement() {
    auto run = [](uint64_t seed) {
        PagePlanner pl(2, 32, 512, 64, 8, 32, true, seed);
        std::vector<PageAction> acts;
        for (int i = 0; i < 12; ++i)
            for (int b = 0; b < 2; ++b) pl.plan(b, 32, &acts);
        return pl.table();
    };
    CHECK(run(5) == run(5));
    CHECK(run(5) != run(6));
}

static void test_out_of_pages_is_atomic() {
    // 3 device pages for 2 sequences with a 64-position window (3 pages each)
    PagePlanner pl(2, 32, 512, 64, 3, 64, true, 3);
    std::vector<PageAction> acts;
    CHECK(pl.plan(0, 32, &acts) == 0);
    CHECK(pl.plan(0, 32, &acts) == 0);
    CHECK(pl.plan(1, 32, &acts) == 0);  // pool now full
    const std::vector<int32_t> before = pl.table();
    const uint32_t used0 = pl.store(0).used();
    acts.clear();
    CHECK(pl.plan(0, 1, &acts) == 4);  // needs a fourth page
    CHECK(acts.empty() && pl.table() == before && pl.store(0).used() == used0);
    // releasing sequence 1 frees its page for sequence 0
    acts.clear();
    pl.reset(1, &acts);
    CHECK(acts.size() == 1 && acts[0].kind == PageAction::kDrop);
    CHECK(pl.store(1).used() == 0);
    CHECK(pl.plan(0, 1, &acts) == 0);
    // a step may reuse a page evicted earlier in the same step: sequence 0 at
    // position 95 evicts page 0 (its last position 31 leaves the 64 window)
    // and allocates page 3 at position 96 from it
    PagePlanner q(1, 32, 512, 64, 3, 8, true, 3);
    acts.clear();
    CHECK(q.plan(0, 32, &acts) == 0 && q.plan(0, 32, &acts) == 0 && q.plan(0, 31, &acts) == 0);
    acts.clear();
    CHECK(q.plan(0, 2, &acts) == 0);
    CHECK(acts.size() == 2 && acts[0].kind == PageAction::kEvict && acts[1].kind == PageAction::kAlloc);
    CHECK(acts[0].dev == acts[1].dev);
}

// Deferred eviction: the evicted page's slot keeps its device page until the
// eviction is retired; then it names the cold page and the device page is free.
// Completed copies retire in eviction order; an allocation that finds no free
// page retires the oldest in-flight eviction at once (wait set).
static void test_deferred_eviction() {
    const int n_seq = 3, P = 32;
    const uint32_t n_ctx = 2048, W = 100;
    const int win_pages = (W + P - 1) / P + 1;
    for (int slack : {0, 2}) {
        const int n_pages = n_seq * win_pages + slack;
        PagePlanner pl(n_seq, P, n_ctx, W, n_pages, n_seq * 64, true, 11, true);
        PagePlanner sync(n_seq, P, n_ctx, W, n_pages, n_seq * 64, true, 11, false);
        std::vector<PageAction> acts;
        std::set<uint64_t> issued;
        int waits = 0, retired = 0;
        for (int step = 0; step < 200; ++step) {
            int32_t n_tok[n_seq];
            for (int b = 0; b < n_seq; ++b) {
                n_tok[b] = (step < 6 ? 30 : 1) + (b == 1 && step % 5 == 0);
                if (!pl.store(b).can_fit(n_tok[b])) n_tok[b] = 0;
            }
            // copies known complete: every eighth step, all those in flight
            // or half of them
            acts.clear();
            const std::vector<uint64_t> fl = pl.in_flight();
            const int done = step % 8 == 7 ? (int)fl.size() : step % 8 == 3 ? (int)fl.size() / 2 : 0;
            pl.retire_completed(done, &acts);
            CHECK((int)acts.size() == std::min<int>(done, (int)fl.size()));
            for (size_t i = 0; i < acts.size(); ++i) {
                CHECK(acts[i].kind == PageAction::kRetire && !acts[i].wait && acts[i].evict == fl[i]);
                ++retired;
            }
            acts.clear();
            CHECK(pl.plan_step(n_tok, &acts) == 0);
            std::vector<PageAction> sacts;
            CHECK(sync.plan_step(n_tok, &sacts) == 0);
            for (const PageAction &a : acts) {
                if (a.kind == PageAction::kEvict) {
                    CHECK(!a.edit && issued.insert(a.evict).second);
                } else if (a.kind == PageAction::kRetire) {
                    CHECK(a.wait && issued.count(a.evict) == 1);  // issued before, maybe this step
                    ++waits;
                    ++retired;
                }
            }
            // same logical bookkeeping as immediate eviction, and every page
            // out of the window is cold or still in flight on its device page
            const std::vector<uint64_t> now = pl.in_flight();
            CHECK(pl.stats().in_flight == (int64_t)now.size());
            CHECK(pl.stats().evicted == sync.stats().evicted);
            CHECK(pl.stats().cold_in_use == sync.stats().cold_in_use);
            std::set<int32_t> dev;
            for (int b = 0; b < n_seq; ++b) {
                CHECK(pl.store(b).used() == sync.store(b).used());
                for (int lp = 0; lp < pl.max_pages(); ++lp) {
                    const size_t i = (size_t)b * pl.max_pages() + lp;
                    const int32_t a = pl.table()[i], y = sync.table()[i];
                    if (y >= 0) {
                        CHECK(a >= 0);  // resident in both (placement may differ)
                    } else if (y == -1) {
                        CHECK(a == -1);
                    } else {
                        CHECK(a <= -2 || a >= 0);  // cold, or device page in flight
                    }
                    if (a >= 0) CHECK(dev.insert(a).second);
                }
            }
            CHECK((int)dev.size() <= n_pages);
            CHECK((int64_t)dev.size() <= pl.stats().dev_in_use);
        }
        CHECK(retired + (int)pl.in_flight().size() == (int)issued.size() && !issued.empty());
        // an exact pool must retire in-flight pages to allocate
        if (slack == 0) CHECK(waits > 0);
        // retiring everything gives the immediate-eviction tables
        acts.clear();
        pl.retire_completed((int)pl.in_flight().size(), &acts);
        for (int b = 0; b < n_seq; ++b)
            for (int lp = 0; lp < pl.max_pages(); ++lp) {
                const size_t i = (size_t)b * pl.max_pages() + lp;
                CHECK((pl.table()[i] <= -2) == (sync.table()[i] <= -2));
                CHECK((pl.table()[i] == -1) == (sync.table()[i] == -1));
            }
        CHECK(pl.stats().in_flight == 0 && pl.stats().dev_in_use == sync.stats().dev_in_use);
    }
}

// A reset while a sequence's eviction is in flight: the slot is cleared at
// once, the cold page released, and the later retirement edits nothing.
static void test_reset_with_eviction_in_flight() {
    PagePlanner pl(2, 32, 512, 64, 8, 32, true, 5, true);
    std::vector<PageAction> acts;
    const int32_t fill[2] = {32, 32};
    for (int i = 0; i < 3; ++i) CHECK(pl.plan_step(fill, &acts) == 0);
    const int32_t one[2] = {1, 1};
    acts.clear();
    CHECK(pl.plan_step(one, &acts) == 0);  // position 96: page 0 of each leaves the window
    CHECK(pl.in_flight().size() == 2 && pl.stats().cold_in_use == 2);
    acts.clear();
    pl.reset(1, &acts);
    CHECK(pl.stats().cold_in_use == 1 && pl.stats().in_flight == 2);
    for (int lp = 0; lp < pl.max_pages(); ++lp) CHECK(pl.table()[(size_t)pl.max_pages() + lp] == -1);
    acts.clear();
    pl.retire_completed(2, &acts);
    CHECK(acts.size() == 2 && acts[0].edit && !acts[1].edit);
    CHECK(pl.table()[0] <= -2 && pl.stats().in_flight == 0);
}

// plan_step is all or nothing, whatever allocation fails inside it.
static void test_plan_step_all_or_nothing() {
    for (bool async : {false, true}) {
        for (long k = 0;; ++k) {
            PagePlanner pl(3, 32, 1024, 64, 3 * 4, 3 * 32, true, 9, async);
            std::vector<PageAction> acts;
            const int32_t warm[3] = {32, 20, 32};
            for (int i = 0; i < 4; ++i) CHECK(pl.plan_step(warm, &acts) == 0);
            const std::vector<int32_t> table = pl.table();
            const std::vector<uint64_t> fl = pl.in_flight();
            const uint32_t used[3] = {pl.store(0).used(), pl.store(1).used(), pl.store(2).used()};
            const int64_t ev = pl.stats().evicted, al = pl.stats().allocated;
            acts.assign(3, PageAction{});
            const int32_t step[3] = {32, 32, 31};
            g_fail_countdown = k;
            const int rc = pl.plan_step(step, &acts);
            const bool failed = g_fail_countdown < 0;
            g_fail_countdown = -1;
            if (rc == 0) {
                CHECK(!failed && pl.store(0).used() == used[0] + 32);
                break;
            }
            CHECK(rc == 4 && failed);
            CHECK(acts.size() == 3 && pl.table() == table && pl.in_flight() == fl);
            CHECK(pl.store(0).used() == used[0] && pl.store(1).used() == used[1] &&
                  pl.store(2).used() == used[2]);
            CHECK(pl.stats().evicted == ev && pl.stats().allocated == al);
            CHECK(k < 10000);
        }
    }
}

int main() {
    test_kv_store();
    test_planner_lossless(true);
    test_planner_lossless(false);
    test_no_paging_when_window_covers_ctx();
    test_seeded_placement();
    test_out_of_pages_is_atomic();
    test_deferred_eviction();
    test_reset_with_eviction_in_flight();
    test_plan_step_all_or_nothing();
    std::printf("ok %d\n", g_checks);
    return 0;
}
