// paged_step.h -- the per-step KV append of a decode batch, shared by the page
// pool (paged.hip) and the decode step (decode.hip), and the prefill's view of
// the paged attention (attention.hip).
#pragma once

#include <vector>

#include "be42_common.h"

namespace be42 {

constexpr int kArgTok = 64;   // tokens (or layer slots) of one append launch

// Bookkeeping of one token for each of n distinct layer slots: position,
// physical page, whether the page is new (page table entry to publish), and
// the pages that became full (centroid + hash to compute).
struct AppendStepArgs {
    int n, max_logical;
    int pos[kArgTok], phys[kArgTok], slot[kArgTok], publish[kArgTok];
    int n_seal;
    int seal_phys[kArgTok], seal_slot[kArgTok], seal_logical[kArgTok], seal_nidx[kArgTok];
    int seal_of[kArgTok];   // per token: its entry in the seal list, or -1
};

// What plan_append_step changed in the pool's host bookkeeping, so that a
// step that fails before its launches are queued can give it back (the
// device never saw those pages).  One log may span several plans.
struct PlanUndo {
    int free_top = -2;       // free-stack top before the first plan (-2: nothing logged)
    std::vector<int> slot, len, nidx;   // per slot first touched: logical pages, pages indexed
    std::vector<int> sealed;            // pages the plans marked registered
};

// host: allocate pages and fill the bookkeeping (paged.c:195-272 per slot);
// undo (may be NULL) logs the changes
int plan_append_step(be42_kv_pool *pool, const int *slots, const int *pos, int n, AppendStepArgs *out,
                     PlanUndo *undo = nullptr);
// restore the host bookkeeping logged in undo (pages back on the free stack
// in their order, page-table entries unmapped, counters and flags reset)
void undo_append_plans(be42_kv_pool *pool, const PlanUndo &undo);
// device: RoPE of the n tokens' q [n][n_heads*hd] and k [n][n_kv*hd] at
// position *pos_p (table rows [pos][hd/2]; not rotated at or past rope_len),
// then the store of their K/V rows and the seal of the pages they fill, in
// one launch; the bookkeeping is read from a_dev (device memory), so no host
// value of the step enters the launch
int launch_rope_append_step_dev(const be42_kv_pool &P, const AppendStepArgs *a_dev, int n, float *q, float *k,
                                const float *v, const float *cos_t, const float *sin_t, const int *pos_p,
                                int rope_len, int n_heads, hipStream_t st);

// A run of n consecutive positions of one layer slot, appended with one
// store launch and one seal launch from page lists in device memory.
struct AppendRun {
    int layer, layer_base, pos0, n, first_blk, n_pages, n_new, new_first, n_seal, n_log, n_idx, list_len;
};
// ints of page lists a run of n positions needs
inline int append_run_list_cap(int n) { return 4 * (n / 16 + 2); }
// host: allocate the run's pages and write its lists to L (host memory of
// append_run_list_cap(n) ints)
int plan_append_run(be42_kv_pool *pool, int layer, int pos0, int n, int *L, AppendRun *out);
// device: the run's store and seal, its lists (as planned) at d_lists
int launch_append_run(const be42_kv_pool &P, const AppendRun &r, const int *d_lists, const float *k, const float *v,
                      hipStream_t s);

// device: the router (k_route, lsh.hip) of n_queries queries; lim (device,
// optional) as in lsh_attention_prefix; cand / ncand / qhash optional
int launch_route(const be42_kv_pool &P, const float *q, const int *slots, const int *lim, int n_queries, int H,
                 int k_sel, int cap, int *sel, int *nsel, int sel_stride, int *cand, int *ncand, uint16_t *qhash,
                 hipStream_t s);

// device: paged attention of n_queries queries of the slots slots[b] (device
// array), query b seeing only the first lim[b] positions of its slot (its
// pages, LSH index and last page as they were when position lim[b] - 1 was
// the newest), each computed exactly as a one-query decode launch computes it
// (attention.hip); needs k_sel <= 64, groups of <= 4 heads, head_dim 64/128.
// sel / nsel: device workspace of n_queries selections (sel_stride >=
// prefix_sel_stride(k_sel) ints each) and counts.
inline int prefix_sel_stride(int k_sel) { return k_sel > 64 ? k_sel : 64; }
int lsh_attention_prefix(const be42_kv_pool &P, const float *q, const int *slots, const int *lim, int n_queries,
                         int n_heads, int k_sel, int cand_cap, float scale, float *out, int *sel, int *nsel,
                         int sel_stride, hipStream_t s);

// be42_lsh_attention that, when the launch splits each (query, KV head) pair
// over several workgroups, also writes the output rows as GEMV digit planes
// (xdig_prepare's layout, k = n_heads * head_dim; none when xdig is null) and
// sets *done; a split launch's bounded waits report to the device word *err
int lsh_attention_digits(const be42_kv_pool &P, const float *q, const int *slots, int n_queries, int n_heads,
                         int k_sel, int cand_cap, float scale, float *out, int *sel, int *n_sel, int sel_stride,
                         void *xdig, bool fp8, bool *done, int *err, hipStream_t s);

}  // namespace be42
