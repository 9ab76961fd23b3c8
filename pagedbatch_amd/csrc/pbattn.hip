// Paged-attention decode kernel for gfx950 (CDNA4), part of libpbsample.so.
//
// One decode step of grouped-query attention over a paged KV cache
// (pagedbatch/model.py:201-224): one workgroup per (sequence, KV head) reads each K and
// V row of that head once and serves the n_rep query heads that share it.
//
//   1. The query rows of the group go to LDS; every thread takes context positions
//      t = tid, tid + 256, ...: its slot through the block table
//      (pagedbatch/block_manager.py:88-91), the K row (64 bf16, eight 16-byte loads) and
//      the n_rep scaled dot products, in fp32, into an LDS score table.
//   2. Per query head: the maximum and the sum of exp(score - max) (block reductions).
//   3. V rows in tiles of 256 positions staged through LDS (eight independent 16-byte
//      loads per thread), then threads (position group, dim) accumulate
//      sum_t p[t] * V[t][dim] for every query head.
// Memory: (K + V) * context * 128 B per (sequence, KV head), read once; HBM-bound for
// long contexts, launch- and latency-bound for short ones.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pbattn.h"
#include "pbsample.h"

namespace pbs {
int report_error(int code, const char* msg);
}

namespace pba {

constexpr int NT = 256;
constexpr int D = 64;
constexpr int MAX_REP = 8;
constexpr int MAX_CONTEXT = 2048;

struct Args {
  const float* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t n_slots;
  const int32_t* block_table;
  int64_t max_blocks;
  const int32_t* context_lens;
  int n_heads, n_kv_heads, rep, block_size, max_context;
  float scale;
  float* out;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// N values at once, max or sum over the workgroup: shuffles inside each wave, then the
// waves' results through LDS (red: [NT / 64][N]); every thread gets the totals
template <bool MAX, int N>
__device__ __forceinline__ void block_reduce_n(float (&v)[N], float* red) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    for (int off = 32; off > 0; off >>= 1) {
      const float o = __shfl_xor(v[i], off, 64);
      v[i] = MAX ? fmaxf(v[i], o) : v[i] + o;
    }
  }
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int i = 0; i < N; ++i) red[w * N + i] = v[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; ++i) {
    float r = red[i];
    for (int ww = 1; ww < NT / 64; ++ww) r = MAX ? fmaxf(r, red[ww * N + i]) : r + red[ww * N + i];
    v[i] = r;
  }
}

__global__ __launch_bounds__(NT) void k_decode(Args a) {
  extern __shared__ float lds[];
  uint4* vt = (uint4*)lds;                           // [NT][D / 8]: a tile of V rows
  float* qs = (float*)(vt + NT * (D / 8));           // [rep][D]
  float* red = qs + MAX_REP * D;                     // [NT / 64][MAX_REP + 1]
  float* part = red + (NT / 64) * (MAX_REP + 1);     // [NT / D][MAX_REP][D] partial sums
  int* slot_s = (int*)(part + (NT / D) * MAX_REP * D);  // [max_context]
  float* sc = (float*)(slot_s + a.max_context);      // [rep][max_context]

  const int b = blockIdx.x / a.n_kv_heads;
  const int kvh = blockIdx.x % a.n_kv_heads;
  const int rep = a.rep;
  const int L = a.context_lens[b];
  const int tid = threadIdx.x;
  float* out = a.out + ((size_t)b * a.n_heads + (size_t)kvh * rep) * D;
  if (L < 1 || L > a.max_context) {  // out of the declared range: no reads, NaN out
    for (int i = tid; i < rep * D; i += NT) out[i] = __int_as_float(0x7fc00000);
    return;
  }
  for (int i = tid; i < rep * D; i += NT) qs[i] = a.q[((size_t)b * a.n_heads + (size_t)kvh * rep) * D + i];
  __syncthreads();

  // 1. scores
  int bad = 0;
  float mx[MAX_REP];
#pragma unroll
  for (int h = 0; h < MAX_REP; ++h) mx[h] = -INFINITY;
  for (int t = tid; t < L; t += NT) {
    const int64_t blk = a.block_table[(size_t)b * a.max_blocks + t / a.block_size];
    const int64_t slot = blk * a.block_size + t % a.block_size;
    const bool ok = blk >= 0 && slot >= 0 && slot < a.n_slots;
    bad |= ok ? 0 : 1;
    slot_s[t] = ok ? (int)slot : -1;
    float acc[MAX_REP];
#pragma unroll
    for (int h = 0; h < MAX_REP; ++h) acc[h] = 0.0f;
    if (ok) {
      const uint4* kr = (const uint4*)(a.k + ((size_t)slot * a.n_kv_heads + kvh) * D);
#pragma unroll
      for (int c = 0; c < D / 8; ++c) {
        const uint4 w = kr[c];
        const float kv[8] = {bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y),
                             bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w)};
#pragma unroll
        for (int h = 0; h < MAX_REP; ++h) {
          if (h < rep) {
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h] = fmaf(qs[h * D + c * 8 + e], kv[e], acc[h]);
          }
        }
      }
    }
#pragma unroll
    for (int h = 0; h < MAX_REP; ++h) {
      if (h < rep) {
        const float sv = acc[h] * a.scale;
        sc[h * a.max_context + t] = sv;
        mx[h] = fmaxf(mx[h], sv);
      }
    }
  }
  // 2. one block reduction for every head's maximum and the corrupt-slot flag, one for
  //    every head's sum of exponentials (the weights replace the scores in place)
  float mv[MAX_REP + 1];
#pragma unroll
  for (int h = 0; h < MAX_REP; ++h) mv[h] = mx[h];
  mv[MAX_REP] = bad ? 1.0f : 0.0f;
  block_reduce_n<true>(mv, red);
  if (mv[MAX_REP] > 0.0f) {  // a corrupt slot anywhere in the context: NaN out
    for (int i = tid; i < rep * D; i += NT) out[i] = __int_as_float(0x7fc00000);
    return;
  }
  float sum[MAX_REP + 1];
#pragma unroll
  for (int h = 0; h <= MAX_REP; ++h) sum[h] = 0.0f;
  for (int t = tid; t < L; t += NT) {
#pragma unroll
    for (int h = 0; h < MAX_REP; ++h) {
      if (h < rep) {
        const float e = __expf(sc[h * a.max_context + t] - mv[h]);
        sc[h * a.max_context + t] = e;
        sum[h] += e;
      }
    }
  }
  block_reduce_n<false>(sum, red);

  // 3. weighted sum of the V rows, in tiles of NT positions staged through LDS (every
  //    thread issues its eight 16-byte loads of a tile at once); thread (q4, d) then takes
  //    dim d and the tile's positions q4, q4 + 4, ... for every query head (one V element
  //    read serves them all); the four position groups' partial sums meet in LDS
  const int d = tid & (D - 1), q4 = tid >> 6;
  float acc[MAX_REP];
#pragma unroll
  for (int h = 0; h < MAX_REP; ++h) acc[h] = 0.0f;
  for (int t0 = 0; t0 < L; t0 += NT) {
    const int n = min(NT, L - t0);
    __syncthreads();  // the previous tile is consumed
#pragma unroll
    for (int i0 = 0; i0 < NT * (D / 8); i0 += NT) {
      const int i = i0 + tid, r = i >> 3;
      if (r < n) vt[i] = ((const uint4*)(a.v + ((size_t)slot_s[t0 + r] * a.n_kv_heads + kvh) * D))[i & 7];
    }
    __syncthreads();
    for (int r = q4; r < n; r += NT / D) {
      const float vv = __uint_as_float((uint32_t)((const uint16_t*)(vt + r * (D / 8)))[d] << 16);
#pragma unroll
      for (int h = 0; h < MAX_REP; ++h)
        if (h < rep) acc[h] = fmaf(sc[h * a.max_context + t0 + r], vv, acc[h]);
    }
  }
#pragma unroll
  for (int h = 0; h < MAX_REP; ++h)
    if (h < rep) part[(q4 * MAX_REP + h) * D + d] = acc[h];
  __syncthreads();
  for (int p = tid; p < rep * D; p += NT) {
    const int h = p / D, dd = p % D;
    float tot = 0.0f;
#pragma unroll
    for (int g = 0; g < NT / D; ++g) tot += part[(g * MAX_REP + h) * D + dd];
    float s = 1.0f;
#pragma unroll
    for (int hh = 0; hh < MAX_REP; ++hh) s = (hh == h) ? sum[hh] : s;
    out[p] = tot / s;
  }
}

}  // namespace pba

extern "C" int pba_decode_attention(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, int64_t n_slots,
                                    const int32_t* block_table, int64_t max_blocks, const int32_t* context_lens,
                                    int64_t rows, int n_heads, int n_kv_heads, int head_dim, int block_size,
                                    int max_context, float scale, float* out, void* stream) {
  using namespace pba;
  if (rows < 0) return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "rows is negative");
  if (rows == 0) return PBS_OK;
  if (!q || !k_cache || !v_cache || !block_table || !context_lens || !out)
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "null device pointer");
  if (head_dim != D) return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "head_dim must be 64");
  if (n_kv_heads < 1 || n_heads < n_kv_heads || n_heads % n_kv_heads != 0 || n_heads / n_kv_heads > MAX_REP)
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT,
                             "n_heads must be a multiple of n_kv_heads, at most 8 query heads per KV head");
  if (block_size < 1 || max_blocks < 1 || n_slots < 1)
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "block_size, max_blocks and n_slots must be positive");
  if (max_context < 1 || max_context > MAX_CONTEXT || (int64_t)max_context > max_blocks * block_size)
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT,
                             "max_context must be in [1, 2048] and covered by max_blocks * block_size");
  if (rows * n_kv_heads > 0x7fffffff) return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "too many rows");
  if (n_slots > 0x7fffffff)  // slot numbers are kept as 32-bit ints in LDS
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "n_slots must be below 2^31");
  Args a;
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.n_slots = n_slots;
  a.block_table = block_table;
  a.max_blocks = max_blocks;
  a.context_lens = context_lens;
  a.n_heads = n_heads;
  a.n_kv_heads = n_kv_heads;
  a.rep = n_heads / n_kv_heads;
  a.block_size = block_size;
  a.max_context = max_context;
  a.scale = scale;
  a.out = out;
  const size_t lds = sizeof(uint4) * NT * (D / 8) +
                     sizeof(float) * (MAX_REP * D + (NT / 64) * (MAX_REP + 1) + (NT / D) * MAX_REP * D) +
                     sizeof(int) * max_context + sizeof(float) * (size_t)a.rep * max_context;
  if (lds > 64 * 1024) {
    const hipError_t ea = hipFuncSetAttribute((const void*)k_decode, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (ea != hipSuccess) return pbs::report_error(PBS_ERR_HIP, hipGetErrorString(ea));
  }
  hipLaunchKernelGGL(k_decode, dim3((unsigned)(rows * n_kv_heads)), dim3(NT), lds, (hipStream_t)stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return pbs::report_error(PBS_ERR_HIP, hipGetErrorString(e));
  return PBS_OK;
}
