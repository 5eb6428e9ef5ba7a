// paged_step.h -- the per-step KV append of a decode batch, shared by the page
// pool (paged.hip) and the decode step (decode.hip).
#pragma once

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

// host: allocate pages and fill the bookkeeping (paged.c:195-272 per slot)
int plan_append_step(be42_kv_pool *pool, const int *slots, const int *pos, int n, AppendStepArgs *out);
// device: RoPE of the n tokens' q [n][n_heads*hd] and k [n][n_kv*hd] at
// position *pos_p (table rows [pos][hd/2]; not rotated at or past rope_len),
// then the store of their K/V rows and the seal of the pages they fill, in
// one launch; the bookkeeping is read from a_dev (device memory), so no host
// value of the step enters the launch
int launch_rope_append_step_dev(const be42_kv_pool &P, const AppendStepArgs *a_dev, int n, float *q, float *k,
                                const float *v, const float *cos_t, const float *sin_t, const int *pos_p,
                                int rope_len, int n_heads, hipStream_t st);

}  // namespace be42
