/*
 * pblmhead.h -- C ABI of the fused lm_head + greedy kernel (MI355X, gfx950).
 *
 * The step before the sampler: logits = hidden @ weight^T for the last token of every
 * sequence, in bf16 with fp32 accumulation on the matrix cores, with each row's greedy
 * token (the index of its first maximum, or of its first NaN) taken in the same kernel's
 * epilogue. A step whose rows are all greedy then needs neither the logits write nor the
 * sampler's read of them; a mixed step writes the logits once and samples only its
 * stochastic rows from them (pbs_sample with a row_map).
 *
 * Reference interface replaced (aryavolkan/pagedbatch):
 *   pagedbatch/model.py:283        logits = self.lm_head(hidden[batch.last_token_index])
 *                                  (nn.Linear(hidden, vocab, bias=False), weight [vocab,
 *                                  hidden], tied to the embedding, model dtype bf16)
 *   pagedbatch/sampling.py:12-13   greedy rows: int(torch.argmax(logits_row))
 *   pagedbatch/engine.py:133-139   the per-row loop that reaches sample_token
 */
#ifndef PBLMHEAD_H
#define PBLMHEAD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Device workspace bytes pbs_lm_head_argmax needs: 8 per (row, 64-column tile). The
 * call overwrites it; its contents between calls do not matter. */
size_t pbs_lm_head_workspace_bytes(int64_t rows, int64_t vocab);

/*
 *   hidden        device bf16 (raw uint16) [rows][hidden_dim], rows hidden_stride apart
 *   weight        device bf16 (raw uint16) [vocab][hidden_dim], contiguous
 *   out_logits    device bf16 (raw uint16) [rows][vocab], or NULL to skip the write
 *                 (every row greedy): each value is the fp32 dot product rounded to
 *                 bf16 (nearest, ties to even), as the reference's bf16 Linear returns
 *   out_token     device int32[rows]: torch.argmax of the row's bf16 logits (lowest
 *                 index among equal maxima, -0 equal to +0; the first NaN if any)
 *   workspace     device memory of at least pbs_lm_head_workspace_bytes(rows, vocab)
 * hidden_dim must be a positive multiple of 64, hidden_stride >= hidden_dim,
 * vocab * hidden_dim * 2 and rows * hidden_stride * 2 below 2^31 bytes. The hidden and
 * weight pointers must be 16-byte aligned (hidden_stride a multiple of 8). Returns 0 or
 * a negative PBS_ERR_* code (pbs_last_error() says why); asynchronous on `stream`.
 */
int pbs_lm_head_argmax(const uint16_t* hidden, int64_t hidden_stride, const uint16_t* weight, int64_t rows,
                       int64_t hidden_dim, int64_t vocab, uint16_t* out_logits, int32_t* out_token,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * pbs_lm_head_argmax without a workspace argument and without any allocation, for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). It has no counterpart in the reference. The kernels use the library's
 * own per-GPU scratch array (4 MiB, kept until the process ends), so rows * ceil(vocab /
 * 64) must not exceed 524288 (PBS_ERR_WORKSPACE otherwise; e.g. 256 rows of a 131072
 * vocab). The scratch belongs to the device current at the call; its address is looked up
 * on the first call on each device. Calls that overlap on one GPU (several streams or
 * threads at once) share that array and race: serialize them.
 */
int pbs_lm_head_argmax_noalloc(const uint16_t* hidden, int64_t hidden_stride, const uint16_t* weight, int64_t rows,
                               int64_t hidden_dim, int64_t vocab, uint16_t* out_logits, int32_t* out_token,
                               void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PBLMHEAD_H */
