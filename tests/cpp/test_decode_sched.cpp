// Host walk of the split-K decode schedule (powerinfer_x64_amd/csrc/decode_sched.hpp,
// the functions the gfx950 decode and merge kernels call) over every workgroup of a
// launch, for well-formed and malformed tables: context lengths past the page-table
// row, negative or huge lengths, page ids outside the pool.  It checks, without a GPU,
// that every index the kernels form stays in bounds:
//   - page-table reads inside the sequence's row of max_pages entries;
//   - pool blocks inside n_pages x n_kv_heads;
//   - partial slots inside batch x n_kv_heads + grid, each written by one run;
// and that the work is covered exactly once: every item by one workgroup, every page
// of every (sequence, KV head) by one wave, and every run the merge reads was written.
// Exit status 0 = all cases pass; the failing case is printed otherwise.
#include "decode_sched.hpp"

#include <climits>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <random>
#include <vector>

using namespace pi::sched;

namespace {

int g_fail = 0;

#define CHECK(c, ...)                                          \
    do {                                                       \
        if (!(c)) {                                            \
            if (g_fail++ < 20) {                               \
                std::printf("FAIL %s:%d %s: ", __FILE__, __LINE__, #c); \
                std::printf(__VA_ARGS__);                      \
                std::printf("\n");                             \
            }                                                  \
            return false;                                      \
        }                                                      \
    } while (0)

struct Case {
    const char* name;
    int n_kv, max_pages, n_pages, item_pages, grid;
    std::vector<int32_t> ctx;  // [batch]
    std::vector<int32_t> pt;   // [batch][max_pages]
};

// Mirrors decode_kernel / decode_merge_kernel (decode.hip) step for step,
// with the kernels' own schedule functions.  merge_runs must give exactly the
// number of runs that write a partial (none is left out of the merge).
bool walk(const Case& c) {
    const int batch = (int)c.ctx.size(), n_kv = c.n_kv, mp = c.max_pages, ip = c.item_pages;
    std::vector<int> s_cum(batch + 1, 0);
    for (int b = 0; b < batch; ++b) s_cum[b + 1] = s_cum[b] + items_of(seq_tokens(c.ctx[b], mp), ip);
    const int per_kv = s_cum[batch];
    const int n_items = n_kv * per_kv;
    const int chunk = (n_items + c.grid - 1) / c.grid;
    const long long n_slots = (long long)batch * n_kv + c.grid;
    std::vector<int> item_seen(n_items, 0);
    std::vector<int> page_seen((size_t)batch * n_kv * mp, 0);
    std::map<long long, std::pair<int, int>> slot_owner;  // slot -> (b, kvh)
    std::vector<char> whole((size_t)batch * n_kv, 0);
    // runs that wrote a partial, per segment: the merge must fold every one of them
    std::vector<int> n_partial((size_t)batch * n_kv, 0);
    // run table (workgroup of run 1, number of runs) written by the segment's first run
    std::vector<std::pair<int, int>> table((size_t)batch * n_kv, {-1, -1});
    for (int w = 0; w < c.grid && n_items > 0; ++w) {
        int cur = w * chunk;
        const int end = imin(n_items, cur + chunk);
        if (cur >= end) continue;
        int b = find_seq(s_cum.data(), batch, n_kv, cur);
        while (cur < end) {
            const Run r = run_at(s_cum.data(), c.ctx.data(), mp, n_kv, ip, b, cur, end);
            b = r.b;
            CHECK(r.b >= 0 && r.b < batch, "%s: b=%d", c.name, r.b);
            CHECK(r.kvh >= 0 && r.kvh < n_kv, "%s: kvh=%d", c.name, r.kvh);
            CHECK(r.run_end > cur && r.run_end <= end, "%s: run [%d, %d) in [.., %d)", c.name, cur, r.run_end, end);
            CHECK(r.len >= 0 && r.len <= kPage * mp, "%s: len=%d", c.name, r.len);
            CHECK(r.pg0 >= 0 && r.pg0 <= r.pg1 && r.pg1 <= mp, "%s: pages [%d, %d) of %d", c.name, r.pg0, r.pg1, mp);
            for (int i = cur; i < r.run_end; ++i) item_seen[i]++;
            if (cur == r.seg0) {
                auto& t = table[(size_t)r.b * n_kv + r.kvh];
                CHECK(t.second == -1, "%s: run table of (b %d, kvh %d) written twice", c.name, r.b, r.kvh);
                int wg1;
                const int n_runs = merge_runs(s_cum.data(), n_kv, chunk, r.b, r.kvh, &wg1);
                t = {wg1, n_runs};
            }
            for (int sub = r.pg0; sub < r.pg1; sub += kSubPages) {
                for (int wave = 0; wave < kWaves; ++wave) {
                    int first, n_my;
                    sub_pages(sub, r.pg1, wave, &first, &n_my);
                    CHECK(n_my <= 64, "%s: %d pages for one wave", c.name, n_my);
                    for (int j = 0; j < n_my; ++j) {
                        const int idx = first + kWaves * j;
                        CHECK(idx >= r.pg0 && idx < r.pg1, "%s: page index %d outside [%d, %d)", c.name, idx, r.pg0, r.pg1);
                        CHECK(idx < mp, "%s: page-table read %d of a %d-entry row", c.name, idx, mp);
                        page_seen[((size_t)r.b * n_kv + r.kvh) * mp + idx]++;
                        const int32_t pid = c.pt[(size_t)r.b * mp + idx];
                        const bool ok = page_ok(pid, c.n_pages);
                        const long long blk = (long long)(ok ? pid : 0) * n_kv + r.kvh;
                        CHECK(blk >= 0 && blk < (long long)c.n_pages * n_kv, "%s: pool block %lld", c.name, blk);
                        const int valid = ok ? imin(r.len - idx * kPage, kPage) : 0;
                        CHECK(valid >= 0 && valid <= kPage && (!ok || valid > 0), "%s: valid=%d", c.name, valid);
                    }
                }
            }
            const long long slot = run_slot(cur == r.seg0, r.b, r.kvh, n_kv, batch, w);
            CHECK(slot >= 0 && slot < n_slots, "%s: slot %lld of %lld", c.name, slot, n_slots);
            if (r.whole) {
                whole[(size_t)r.b * n_kv + r.kvh] = 1;
            } else {
                CHECK(!slot_owner.count(slot), "%s: slot %lld written twice", c.name, slot);
                slot_owner[slot] = {r.b, r.kvh};
                n_partial[(size_t)r.b * n_kv + r.kvh]++;
            }
            cur = r.run_end;
        }
    }
    for (int i = 0; i < n_items; ++i) CHECK(item_seen[i] == 1, "%s: item %d covered %d times", c.name, i, item_seen[i]);
    for (int b = 0; b < batch; ++b) {
        const int pages_b = (seq_tokens(c.ctx[b], mp) + kPage - 1) / kPage;
        for (int kvh = 0; kvh < n_kv; ++kvh)
            for (int i = 0; i < mp; ++i) {
                const int seen = page_seen[((size_t)b * n_kv + kvh) * mp + i];
                CHECK(seen == (i < pages_b ? 1 : 0), "%s: (b %d, kvh %d) page %d read %d times", c.name, b, kvh, i, seen);
            }
    }
    // merge kernel: every segment split over several workgroups reads only slots its runs wrote
    for (int b = 0; b < batch && n_items > 0; ++b) {
        if (s_cum[b + 1] == s_cum[b]) continue;
        for (int kvh = 0; kvh < n_kv; ++kvh) {
            const auto t = table[(size_t)b * n_kv + kvh];
            CHECK(t.second != -1, "%s: run table of (b %d, kvh %d) never written", c.name, b, kvh);
            const int wg1 = t.first, n_runs = t.second;
            CHECK(n_runs >= 1 && n_runs <= c.grid + 1 && n_runs <= 1024, "%s: %d runs", c.name, n_runs);
            if (n_runs == 1) {
                CHECK(whole[(size_t)b * n_kv + kvh], "%s: (b %d, kvh %d) one run but not whole", c.name, b, kvh);
                continue;
            }
            CHECK(n_partial[(size_t)b * n_kv + kvh] == n_runs, "%s: (b %d, kvh %d) %d partial runs, table says %d",
                  c.name, b, kvh, n_partial[(size_t)b * n_kv + kvh], n_runs);
            for (int r = 0; r < n_runs; ++r) {
                const long long slot = run_slot(r == 0, b, kvh, n_kv, batch, wg1 + r - 1);
                auto it = slot_owner.find(slot);
                CHECK(it != slot_owner.end() && it->second.first == b && it->second.second == kvh,
                      "%s: merge of (b %d, kvh %d) reads slot %lld run %d not written by it", c.name, b, kvh, slot, r);
            }
        }
    }
    return true;
}

Case make(const char* name, std::mt19937& rng, int batch, int n_kv, int max_pages, int ip, int grid,
          int ctx_lo, int ctx_hi, double bad_ctx, double bad_page) {
    Case c;
    c.name = name;
    c.n_kv = n_kv;
    c.max_pages = max_pages;
    c.item_pages = ip;
    c.grid = grid;
    c.n_pages = batch * max_pages + 3;
    std::uniform_int_distribution<int> len(ctx_lo, ctx_hi);
    std::uniform_real_distribution<double> u(0, 1);
    std::uniform_int_distribution<int> pg(0, c.n_pages - 1);
    const int32_t wild[] = {-1, -7, INT_MIN, c.n_pages, c.n_pages + 1, INT_MAX};
    const int32_t wild_len[] = {-1, INT_MIN, 16 * max_pages + 1, 16 * max_pages + 16, INT_MAX};
    for (int b = 0; b < batch; ++b) {
        int32_t L = len(rng);
        if (u(rng) < bad_ctx) L = wild_len[rng() % 5];
        c.ctx.push_back(L);
        for (int i = 0; i < max_pages; ++i) {
            int32_t p = pg(rng);
            if (u(rng) < bad_page) p = wild[rng() % 6];
            c.pt.push_back(p);
        }
    }
    return c;
}

}  // namespace

int main() {
    std::mt19937 rng(0x5EED);
    int n = 0;
    const int ips[] = {1, 2, 4, 8, 16};
    const int grids[] = {1, 2, 3, 7, 64, 255, 256, 511, 1023};
    for (int ip : ips)
        for (int grid : grids) {
            // well-formed ragged batches (C2-like shapes, scaled down)
            n += walk(make("ragged", rng, 32, 8, 64, ip, grid, 0, 64 * 16, 0.0, 0.0));
            n += walk(make("one_seq", rng, 1, 32, 40, ip, grid, 513, 513, 0.0, 0.0));
            // malformed lengths: past the row, negative, INT_MAX, INT_MIN
            n += walk(make("bad_ctx", rng, 24, 2, 50, ip, grid, 0, 50 * 16, 0.5, 0.0));
            // malformed page ids: negative, >= n_pages, INT_MAX
            n += walk(make("bad_pages", rng, 16, 4, 33, ip, grid, 1, 33 * 16, 0.0, 0.3));
            n += walk(make("all_bad", rng, 8, 2, 20, ip, grid, 0, 20 * 16, 1.0, 1.0));
            n += walk(make("empty", rng, 5, 3, 4, ip, grid, 0, 0, 0.0, 0.0));
        }
    // a long row (sub-runs of 256 pages) and a big batch
    n += walk(make("long", rng, 2, 2, 4096, 16, 1023, 40000, 65536, 0.0, 0.01));
    n += walk(make("long_bad", rng, 3, 2, 4096, 16, 300, 60000, 65536, 1.0, 0.05));
    n += walk(make("batch4096", rng, 4096, 1, 3, 1, 1023, 0, 48, 0.05, 0.05));
    std::printf("%d cases, %d failures\n", n, g_fail);
    return g_fail == 0 ? 0 : 1;
}
