/*
 * pbattn.h -- C ABI of the paged-attention decode kernel (MI355X, gfx950).
 *
 * One decode step of grouped-query attention over a paged KV cache: every sequence
 * brings one query token per query head and attends over its whole context, whose keys
 * and values sit in cache slots found through the sequence's block table
 * (slot = block_table[b][t / block_size] * block_size + t % block_size).
 *
 * Reference interface replaced (aryavolkan/pagedbatch):
 *   pagedbatch/model.py:201-224   Attention.forward: K/V written to their slots, each
 *                                 sequence's context gathered through its slot table,
 *                                 KV heads repeated n_rep times (query head h reads KV
 *                                 head h / n_rep), scaled_dot_product_attention
 *   pagedbatch/block_manager.py:88-91   slot = block * block_size + offset
 * The reference gathers the context, repeats the KV heads and calls SDPA per batch
 * group; this kernel reads each K/V row once per (sequence, KV head) and serves the
 * n_rep query heads that share it, in fp32.
 */
#ifndef PBATTN_H
#define PBATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * out[b][h][:] = softmax_t(scale * q[b][h] . K[t]) @ V over t < context_lens[b], with
 * K, V the rows of KV head h / (n_heads / n_kv_heads) at the sequence's slots.
 *   q             device float[rows][n_heads][head_dim]
 *   k_cache       device bf16 (raw uint16) [n_slots][n_kv_heads][head_dim]
 *   v_cache       same layout as k_cache
 *   block_table   device int32[rows][max_blocks]
 *   context_lens  device int32[rows], each in [1, max_context]
 *   max_context   host bound on every context_lens[b]
 *   out           device float[rows][n_heads][head_dim]
 * head_dim must be 64 or 128, n_heads a multiple of n_kv_heads with at most 8 query heads
 * per KV head, max_context <= 2^20, n_slots < 2^31; q,
 * k_cache and v_cache 16-byte aligned. A slot outside [0, n_slots) (a corrupt block table)
 * makes that sequence's output NaN instead of reading out of bounds. Returns 0 or a
 * negative PBS_ERR_* code (pbs_last_error() says why); asynchronous on `stream`.
 */
int pba_decode_attention(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, int64_t n_slots,
                         const int32_t* block_table, int64_t max_blocks, const int32_t* context_lens,
                         int64_t rows, int n_heads, int n_kv_heads, int head_dim, int block_size, int max_context,
                         float scale, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PBATTN_H */
