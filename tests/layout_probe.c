/* Prints sizeof/offsetof of the drop-in ABI structs; compiled against
 * include/be42_engine.h, or with -DUSE_REF against the reference headers,
 * by tests/test_dropin_abi.py. */
#include <stdio.h>
#include <stddef.h>
#ifdef USE_REF
#include "tensor/tensor.h"
#include "compute/ops_lsh.h"
#include "memory/paged.h"
#include "compute/ops_quant.h"
#include "memory/kv_cache.h"
#include "compute/ops_attention.h"
#include "compute/ops.h"
#include "compute/ops_rope.h"
#else
#include "be42_engine.h"
#endif
#define O(T, f) printf(#T "." #f " %zu\n", offsetof(T, f))
#define S(T) printf(#T " %zu\n", sizeof(T))
int main(void) {
  S(t_lsh_ctx); O(t_lsh_ctx, hp_transposed); O(t_lsh_ctx, dim); O(t_lsh_ctx, initialized);
  S(t_block_acc); O(t_block_acc, count); O(t_block_acc, start_pos);
  S(t_lsh_index); O(t_lsh_index, block_starts); O(t_lsh_index, block_lens); O(t_lsh_index, n_blocks);
  O(t_lsh_index, bucket_heads); O(t_lsh_index, chain_next); O(t_lsh_index, active); O(t_lsh_index, block_size);
  S(t_kv_block); O(t_kv_block, v_quant); O(t_kv_block, k_scales); O(t_kv_block, v_scales); O(t_kv_block, centroid);
  O(t_kv_block, n_tokens); O(t_kv_block, start_pos); O(t_kv_block, layer_idx); O(t_kv_block, lsh_registered); O(t_kv_block, lsh_hash);
  S(t_block_manager); O(t_block_manager, page_table); O(t_block_manager, free_stack); O(t_block_manager, free_top);
  O(t_block_manager, capacity); O(t_block_manager, n_layers); O(t_block_manager, n_kv_heads); O(t_block_manager, head_dim);
  O(t_block_manager, max_logical); O(t_block_manager, logical_len);
  S(t_paged_kv_cache); O(t_paged_kv_cache, layer_idx); O(t_paged_kv_cache, n_blocks); O(t_paged_kv_cache, n_tokens);
  S(t_block_score); O(t_block_score, phys_idx); O(t_block_score, score);
  S(t_arena); O(t_arena, size); O(t_arena, offset);
  O(t_kv_cache, v); O(t_kv_cache, max_seq_len); O(t_kv_cache, num_heads); O(t_kv_cache, head_dim); O(t_kv_cache, current_seq_len);
  S(t_kv_init_params); S(t_evict_params); O(t_evict_params, w); O(t_evict_params, keep_k); O(t_evict_params, scratch);
  S(t_attention_params); O(t_attention_params, kv_cache); O(t_attention_params, output); O(t_attention_params, n_heads);
  O(t_attention_params, scale); O(t_attention_params, topk_idx); O(t_attention_params, attend_k);
  S(t_rope_ctx); O(t_rope_ctx, pos); O(t_rope_ctx, theta_base); O(t_rope_ctx, mscale); O(t_rope_ctx, orig_ctx);
  O(t_rope_ctx, thetas_cache);
  S(t_rope_cache); O(t_rope_cache, sin_table); O(t_rope_cache, head_dim); O(t_rope_cache, max_seq_len);
  O(t_tensor, shape); O(t_tensor, stride); O(t_tensor, ndim); O(t_tensor, size); O(t_tensor, dtype);
  printf("DTYPE_F32 %d DTYPE_BF16 %d\n", (int)DTYPE_F32, (int)DTYPE_BF16);
  return 0;
}
