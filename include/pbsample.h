/*
 * pbsample.h -- C ABI of the MI355X (gfx950) token sampler.
 *
 * One call samples one token per output row from a [rows, vocab] logits
 * matrix that already lives in device memory: greedy argmax, temperature,
 * top-k and top-p (nucleus) filtering, then an inverse-CDF draw from one
 * caller-supplied uniform per row.
 *
 * Reference interface replaced (aryavolkan/pagedbatch):
 *   pagedbatch/sampling.py:10-27   sample_token(logits[vocab], params, generator) -> int
 *   pagedbatch/engine.py:133-139   the per-row loop that calls it once per sampled row
 *   pagedbatch/config.py:134-158   SamplingParams (temperature, top_p, top_k)
 * The reference does all of this with torch ops on one row at a time; this
 * library does all rows of one engine step in one kernel launch.
 *
 * Semantics per output row b (logits row r = row_map ? row_map[b] : b):
 *   temperature[b] == 0  -> greedy: index of the first maximum; if the row
 *                           holds a NaN, the index of the first NaN
 *                           (torch.argmax, sampling.py:12-13).
 *   otherwise            -> x = fp32(logit) / temperature (IEEE division,
 *                           sampling.py:14); top-k keeps x >= k-th largest x
 *                           when 0 < top_k < vocab (sampling.py:15-17);
 *                           top-p keeps the shortest prefix of the order
 *                           (x descending, index ascending) whose exclusive
 *                           softmax mass is <= top_p when top_p < 1
 *                           (sampling.py:18-25); the token is the first
 *                           element of the kept set, in that same order,
 *                           whose cumulative softmax mass exceeds
 *                           uniform[b] * (kept mass). This is the
 *                           inverse-CDF form of sampling.py:26-27.
 *
 * All pointers except the host-side ones noted are device pointers. Calls are
 * asynchronous on `stream`; the library allocates nothing per call and keeps
 * no state between calls, so calls from several threads on several streams
 * are independent.
 */
#ifndef PBSAMPLE_H
#define PBSAMPLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PBS_ABI_VERSION 1

/* logits element types */
enum {
  PBS_DTYPE_F32 = 0,
  PBS_DTYPE_F16 = 1,
  PBS_DTYPE_BF16 = 2
};

/* return codes of the entry points */
enum {
  PBS_OK = 0,
  PBS_ERR_INVALID_ARGUMENT = -1,
  PBS_ERR_UNSUPPORTED_DTYPE = -2,
  PBS_ERR_HIP = -3,
  PBS_ERR_WORKSPACE = -4
};

/* per-row status written to out_status[b] */
enum {
  PBS_ROW_OK = 0,
  PBS_ROW_NAN = 1,           /* stochastic row holds a NaN: the reference's
                                multinomial raises RuntimeError (sampling.py:27) */
  PBS_ROW_NONFINITE = 2,     /* stochastic row whose largest scaled logit is
                                +inf, or every scaled logit is -inf: softmax is
                                NaN and the reference raises (sampling.py:26-27) */
  PBS_ROW_BAD_PARAM = 3      /* temperature < 0 or NaN, top_p outside (0, 1],
                                top_k < 0, uniform outside [0, 1), or row_map
                                entry outside [0, n_logit_rows) */
};

/* Per-row diagnostics filled by pbs_sample_debug (test and benchmark use). */
typedef struct pbs_row_info {
  int32_t token;
  int32_t status;
  float x_max;       /* largest scaled logit */
  float x_kth;       /* k-th largest scaled logit (top-k active), else -inf */
  float x_cut;       /* scaled logit of the last kept token in sorted order */
  int32_t n_cut_tie; /* tokens whose scaled logit equals x_cut (within the top-k set) */
  int32_t n_cut_keep;/* of those, how many are kept (the lowest indices) */
  int32_t n_kept;    /* size of the kept set */
  double z_k;        /* sum of exp(x - x_max) over the top-k set */
  double z_p;        /* sum of exp(x - x_max) over the kept set */
  double target;     /* uniform * z_p: the point the inverse CDF is evaluated at */
} pbs_row_info;

/* Returns PBS_ABI_VERSION. */
int pbs_abi_version(void);

/* Message of the last failed call on the calling thread ("" if none). */
const char* pbs_last_error(void);

/* Device workspace bytes pbs_sample needs for this shape (0 today: every
 * kernel keeps its per-row state in LDS). Callers pass at least this much. */
size_t pbs_workspace_bytes(int64_t rows, int64_t vocab, int dtype);

/*
 * Sample one token per output row.
 *   logits        device, dtype elements, row r starts at logits + r*row_stride
 *   n_logit_rows  number of rows in logits (row_map entries are checked against it)
 *   rows          number of output rows
 *   row_stride    elements between consecutive logits rows (>= vocab)
 *   row_map       device int32[rows] or NULL (identity); lets one logits row be
 *                 sampled many times and lets the engine skip rows whose chunk
 *                 does not sample (scheduler.py:39-42)
 *   temperature   device float[rows]   (0 = greedy)
 *   top_k         device int32[rows]   (0 or >= vocab = off)
 *   top_p         device float[rows]   (1 = off)
 *   uniform       device float[rows]   in [0, 1); ignored for greedy rows
 *   out_token     device int32[rows]
 *   out_status    device int32[rows]   PBS_ROW_* codes
 */
int pbs_sample(const void* logits, int dtype, int64_t n_logit_rows, int64_t rows, int64_t vocab,
               int64_t row_stride, const int32_t* row_map, const float* temperature,
               const int32_t* top_k, const float* top_p, const float* uniform, int32_t* out_token,
               int32_t* out_status, void* workspace, size_t workspace_bytes, void* stream);

/*
 * pbs_sample plus diagnostics for parity tests: out_probs (device
 * float[rows*vocab], the final softmax over the kept set, 0 elsewhere; may be
 * NULL), out_kept (device uint8[rows*vocab], 1 for kept tokens; may be NULL)
 * and out_info (device pbs_row_info[rows]; may be NULL unless out_probs or
 * out_kept is requested). Greedy rows report probability 1 on their token.
 * Tokens and statuses are identical to pbs_sample's for the same inputs.
 */
int pbs_sample_debug(const void* logits, int dtype, int64_t n_logit_rows, int64_t rows, int64_t vocab,
                     int64_t row_stride, const int32_t* row_map, const float* temperature,
                     const int32_t* top_k, const float* top_p, const float* uniform,
                     int32_t* out_token, int32_t* out_status, float* out_probs, uint8_t* out_kept,
                     pbs_row_info* out_info, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Greedy-only steps: the token of every output row is the index of the first maximum of
 * its logits row, or of the first NaN if the row holds one (torch.argmax,
 * pagedbatch/sampling.py:12-13, reached through the per-row loop at
 * pagedbatch/engine.py:133-139 when every sampled row has temperature 0). Tokens are
 * identical to pbs_sample's with temperature 0 on every row; only a row_map entry outside
 * [0, n_logit_rows) gives a status other than PBS_ROW_OK (PBS_ROW_BAD_PARAM, token 0).
 * The kernel keeps no histogram, so it needs none of pbs_sample's per-row parameters and
 * streams the logits at a higher rate.
 */
int pbs_argmax(const void* logits, int dtype, int64_t n_logit_rows, int64_t rows, int64_t vocab,
               int64_t row_stride, const int32_t* row_map, int32_t* out_token, int32_t* out_status,
               void* stream);

/* finish reasons written by pbs_finish_reasons */
enum {
  PBS_FINISH_NONE = 0,
  PBS_FINISH_STOP = 1,       /* "stop" */
  PBS_FINISH_LENGTH = 2      /* "length" */
};

/*
 * The finish reason of each sampled sequence after its new token, computed on the device
 * so that the engine reads tokens and reasons back in one copy instead of inspecting
 * each token on the host. Replaces pagedbatch/engine.py:173-182 (Engine._finish_reason),
 * called per sampled row at engine.py:149 after the token is appended:
 *   STOP    if !ignore_eos[b] and (tokens[b] == eos_token_id or tokens[b] is one of row
 *           b's stop ids)
 *   LENGTH  otherwise, if num_output[b] >= max_tokens[b] or num_tokens[b] >= max_model_len
 *   NONE    otherwise
 *   tokens        device int32[rows] (pbs_sample's out_token)
 *   eos_token_id  the model's EOS id (ModelConfig.eos_token_id), -1 for none
 *   ignore_eos    device uint8[rows]   (SamplingParams.ignore_eos)
 *   stop_offsets  device int32[rows + 1]: row b's stop ids are
 *                 stop_ids[stop_offsets[b] .. stop_offsets[b + 1])
 *   stop_ids      device int32[stop_offsets[rows]] (SamplingParams.stop_token_ids); may
 *                 be NULL when no row has any
 *   num_output    device int32[rows]   output tokens of the sequence, this one included
 *   max_tokens    device int32[rows]   (SamplingParams.max_tokens)
 *   num_tokens    device int32[rows]   prompt + output tokens, this one included
 *   max_model_len EngineConfig.max_model_len
 *   out_reason    device int32[rows]   PBS_FINISH_* codes
 */
int pbs_finish_reasons(const int32_t* tokens, int64_t rows, int32_t eos_token_id, const uint8_t* ignore_eos,
                       const int32_t* stop_offsets, const int32_t* stop_ids, const int32_t* num_output,
                       const int32_t* max_tokens, const int32_t* num_tokens, int32_t max_model_len,
                       int32_t* out_reason, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PBSAMPLE_H */
