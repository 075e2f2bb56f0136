// decode_sched.hpp -- the work schedule of the split-K decode kernel: which
// (sequence, KV head) segment, pages and partial slot each workgroup run
// touches.  Plain integer arithmetic shared by the gfx950 kernels
// (decode.hip) and a host-side walk that checks every index they form stays
// in bounds for any table contents (tests/cpp/test_decode_sched.cpp).
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define PI_HD __host__ __device__ __forceinline__
#else
#define PI_HD inline
#endif

namespace pi {
namespace sched {

constexpr int kPage = 16;   // tokens per page
constexpr int kWaves = 4;   // wavefronts per decode workgroup
constexpr int kSubPages = 64 * kWaves;  // pages of one sub-run (a wave's page ids fit one VGPR)

PI_HD int imin(int a, int b) { return a < b ? a : b; }
PI_HD int imax(int a, int b) { return a > b ? a : b; }

// Tokens of a sequence the launch reads: its context length clamped to
// [0, 16 * max_pages], so a malformed length never reads past the
// sequence's page-table row.
PI_HD int seq_tokens(int32_t ctx_len, int max_pages) {
    return imin(imax(ctx_len, 0), kPage * max_pages);
}

// Work items of a sequence of `len` tokens: ceil(pages / item_pages).
PI_HD int items_of(int len, int item_pages) {
    const int pages = (len + kPage - 1) / kPage;
    return (pages + item_pages - 1) / item_pages;
}

// A page id names a page of the pool only inside [0, n_pages); any other
// value is read as page 0 with every token masked.
PI_HD bool page_ok(int32_t pid, int n_pages) { return pid >= 0 && pid < n_pages; }

// Largest b with n_kv * s_cum[b] <= item (s_cum non-decreasing, s_cum[0] = 0).
PI_HD int find_seq(const int* s_cum, int batch, int n_kv, int item) {
    int lo = 0, hi = batch - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (n_kv * s_cum[mid] <= item) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// One run: consecutive items [cur, run_end) of the segment (b, kvh), which
// holds items [seg0, seg0 + nb) and pages [pg0, pg1) of the sequence's row.
struct Run {
    int b, kvh, seg0, run_end, len, pg0, pg1;
    bool whole;  // the run covers its whole segment
};

// The run starting at item `cur` of a workgroup whose range ends at `end`;
// `b` is the sequence of the previous run (or find_seq's answer).  s_cum
// holds the prefix sums of items_of(seq_tokens(.)) over the batch.
PI_HD Run run_at(const int* s_cum, const int32_t* ctx_len, int max_pages, int n_kv,
                 int item_pages, int b, int cur, int end) {
    Run r;
    int nb = s_cum[b + 1] - s_cum[b];
    while (nb == 0 || cur >= n_kv * s_cum[b + 1]) {  // skip empty / finished sequences
        ++b;
        nb = s_cum[b + 1] - s_cum[b];
    }
    r.b = b;
    r.kvh = (cur - n_kv * s_cum[b]) / nb;
    r.seg0 = n_kv * s_cum[b] + r.kvh * nb;
    r.run_end = imin(end, r.seg0 + nb);
    r.len = seq_tokens(ctx_len[b], max_pages);
    const int n_pages_b = (r.len + kPage - 1) / kPage;
    r.pg0 = (cur - r.seg0) * item_pages;
    r.pg1 = imin(n_pages_b, (r.run_end - r.seg0) * item_pages);
    r.whole = cur == r.seg0 && r.run_end == r.seg0 + nb;
    return r;
}

// Pages of wave `wave` in the sub-run starting at page `sub` of a run ending
// at page `pg1`: first + kWaves * j for j < n_my.
PI_HD void sub_pages(int sub, int pg1, int wave, int* first, int* n_my) {
    const int sub_end = imin(sub + kSubPages, pg1);
    *first = sub + wave;
    *n_my = *first < sub_end ? (sub_end - *first + kWaves - 1) / kWaves : 0;
}

// Partial slot of a run.  A run either starts its segment (slot = segment
// index b * n_kv + kvh) or starts its workgroup's item range (slot =
// batch * n_kv + workgroup), so batch * n_kv + grid slots cover any launch
// whatever the context lengths.
PI_HD long long run_slot(bool seg_start, int b, int kvh, int n_kv, int batch, int wg) {
    return seg_start ? (long long)b * n_kv + kvh : (long long)batch * n_kv + wg;
}

// The merge of segment (b, kvh) of nb > 0 items: its runs start at seg0 and
// at every workgroup boundary inside it.  Returns the number of runs (1: the
// decode kernel wrote the output itself) and the workgroup of run 1.
PI_HD int merge_runs(const int* s_cum, int n_kv, int chunk, int b, int kvh, int* wg1) {
    const int nb = s_cum[b + 1] - s_cum[b];
    const int seg0 = n_kv * s_cum[b] + kvh * nb;
    const int seg1 = seg0 + nb;
    const int first_cut = (seg0 / chunk + 1) * chunk;  // first workgroup boundary after seg0
    *wg1 = first_cut / chunk;
    if (first_cut >= seg1) return 1;
    return 1 + (seg1 - 1 - first_cut) / chunk + 1;
}

}  // namespace sched
}  // namespace pi
