// Paged-attention decode kernel for gfx950 (CDNA4), part of libpbsample.so.
//
// One decode step of grouped-query attention over a paged KV cache
// (pagedbatch/model.py:201-224): one workgroup of four waves per (sequence, KV head) reads
// each K and V row of that head once and serves the n_rep query heads that share it.
//
// Each wave takes chunks of 64 context positions (wave w: chunks w, w + 4, ...). Lane l
// holds 8 of the 64 dims (8 (l % 8) ..) of 8 positions (8 j + l / 8, j < 8): its slots
// through the block table (pagedbatch/block_manager.py:88-91), then the K and V pieces of
// those rows, all issued together (16-byte loads, eight lanes per 128-byte row). The eight
// lanes of a position finish its dot products with three DPP steps, which leaves the scores
// in the lanes that hold the matching V pieces, so the weighted sum needs no exchange.
// Each wave keeps an online softmax (running maximum, sum and weighted V sum per query
// head); the four waves meet once in LDS at the end. fp32 throughout.
// Memory: (K + V) * context * 128 B per (sequence, KV head), read once; at decode batch
// sizes the kernel is latency-bound: two dependent loads (block table, then K and V) and
// one barrier.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pbattn.h"
#include "pbsample.h"

namespace pbs {
int report_error(int code, const char* msg);
}

namespace pba {

constexpr int NT = 256;
constexpr int NW = NT / 64;  // waves per workgroup
constexpr int MAX_REP = 8;
constexpr int MAX_CONTEXT = 1 << 20;  // positions stay below 2^22 (the block-index split)
constexpr int QUAD_XOR1 = 0xb1, QUAD_XOR2 = 0x4e, ROW_HALF_MIRROR = 0x141;

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

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, true));
}

// sum over the 8 lanes of a group (lanes 8 g .. 8 g + 7): quad swaps, then the half-row
// mirror pairs quad 0 of the group with quad 1; every lane ends with the total
__device__ __forceinline__ float group8_sum(float v) {
  v += dpp_f<QUAD_XOR1>(v);
  v += dpp_f<QUAD_XOR2>(v);
  return v + dpp_f<ROW_HALF_MIRROR>(v);
}

// across the 8 groups of a wave (lanes l, l ^ 8, ..., l ^ 56), without LDS: a DPP rotate by
// 8 inside each 16-lane row pairs l with l ^ 8. v_permlane16_swap (v_permlane32_swap) of a
// value with itself returns two registers that hold, in every lane, its own value and the
// value of lane l ^ 16 (l ^ 32) in the same order for both lanes of a pair, so combining
// the two gives both lanes the same result.
constexpr int ROW_ROR8 = 0x128;
__device__ __forceinline__ float groups_max(float v) {
  v = fmaxf(v, dpp_f<ROW_ROR8>(v));
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(c[0]), __uint_as_float(c[1]));
}
__device__ __forceinline__ float groups_sum(float v) {
  v += dpp_f<ROW_ROR8>(v);
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}

// DH: the head size (64 or 128); each lane holds DPL = DH / 8 dims of NJ positions, so a
// chunk is 8 NJ positions and a lane's K and V pieces stay at 128 bytes each (64 for more
// than four query heads of 128, whose query and accumulator registers leave less room)
template <int REP, int DH>
__global__ __launch_bounds__(NT) void k_decode(Args a) {
  constexpr int DPL = DH / 8;                          // dims per lane
  constexpr int NJ = DH == 64 ? 8 : (REP > 4 ? 2 : 4);  // positions per lane and chunk
  constexpr int CH = 8 * NJ;       // positions per chunk
  constexpr int NQ = DPL / 8;      // 16-byte pieces per lane and row
  __shared__ float m_s[NW][REP], s_s[NW][REP];
  __shared__ float acc_s[NW][REP][DH];
  __shared__ int bad_s[NW];

  const int b = blockIdx.x / a.n_kv_heads;
  const int kvh = blockIdx.x % a.n_kv_heads;
  const int L = a.context_lens[b];
  const int tid = threadIdx.x, l = tid & 63, w = tid >> 6;
  const int g = l >> 3, e0 = DPL * (l & 7);
  float* out = a.out + ((size_t)b * a.n_heads + (size_t)kvh * REP) * DH;
  if (L < 1 || L > a.max_context) {  // out of the declared range: no reads, NaN out
    for (int i = tid; i < REP * DH; i += NT) out[i] = __int_as_float(0x7fc00000);
    return;
  }
  // the lane's DPL dims of every query head of the group
  float qv[REP][DPL];
  {
    const float4* qp = (const float4*)(a.q + ((size_t)b * a.n_heads + (size_t)kvh * REP) * DH + e0);
#pragma unroll
    for (int h = 0; h < REP; ++h)
#pragma unroll
      for (int i = 0; i < DPL / 4; ++i) {
        const float4 x = qp[h * (DH / 4) + i];
        qv[h][4 * i] = x.x, qv[h][4 * i + 1] = x.y, qv[h][4 * i + 2] = x.z, qv[h][4 * i + 3] = x.w;
      }
  }
  // position p -> (block index, offset): (p + 0.5) * fl(1 / block_size) is within
  // (p + 0.5) * 2^-23 of the exact quotient, below its 0.5 / block_size distance from an
  // integer for every p < 2^22, so the truncation is exact
  const float inv_bs = 1.0f / (float)a.block_size;
  const int32_t* bt = a.block_table + (size_t)b * a.max_blocks;

  float m_run[REP], s_run[REP], acc[REP][DPL];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    m_run[h] = -__builtin_inff();
    s_run[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[h][e] = 0.0f;
  }
  int bad = 0;
  for (int t0 = CH * w; t0 < L; t0 += CH * NW) {
    // slots of the lane's positions t0 + 8 j + g (positions past the context read slot 0,
    // a bad block-table entry reads slot 0 and marks the sequence)
    int64_t row[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int pos = t0 + 8 * j + g;
      const int bi = (int)(((float)pos + 0.5f) * inv_bs);
      const int32_t blk = pos < L ? bt[bi] : 0;
      const int64_t slot = (int64_t)blk * a.block_size + (pos - bi * a.block_size);
      const bool ok = blk >= 0 && slot < a.n_slots;
      bad |= (pos < L && !ok) ? 1 : 0;
      row[j] = ((ok && pos < L) ? slot : 0) * a.n_kv_heads + kvh;
    }
    uint4 kq[NJ][NQ], vq[NJ][NQ];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < NQ; ++i) kq[j][i] = *(const uint4*)(a.k + row[j] * DH + e0 + 8 * i);
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < NQ; ++i) vq[j][i] = *(const uint4*)(a.v + row[j] * DH + e0 + 8 * i);

    // scores of the lane's NJ positions for every head (-inf past the context)
    float sc[REP][NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float kv[DPL];
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        kv[8 * i] = bf16_lo(kq[j][i].x), kv[8 * i + 1] = bf16_hi(kq[j][i].x);
        kv[8 * i + 2] = bf16_lo(kq[j][i].y), kv[8 * i + 3] = bf16_hi(kq[j][i].y);
        kv[8 * i + 4] = bf16_lo(kq[j][i].z), kv[8 * i + 5] = bf16_hi(kq[j][i].z);
        kv[8 * i + 6] = bf16_lo(kq[j][i].w), kv[8 * i + 7] = bf16_hi(kq[j][i].w);
      }
#pragma unroll
      for (int h = 0; h < REP; ++h) {
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < DPL; ++e) d = fmaf(qv[h][e], kv[e], d);
        d = group8_sum(d) * a.scale;
        sc[h][j] = (t0 + 8 * j + g < L) ? d : -__builtin_inff();
      }
    }
    // online softmax update of every head
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      float mc = sc[h][0];
#pragma unroll
      for (int j = 1; j < NJ; ++j) mc = fmaxf(mc, sc[h][j]);
      mc = groups_max(mc);
      const float mn = fmaxf(m_run[h], mc);  // finite: the chunk holds a position < L
      const float alpha = __expf(m_run[h] - mn);
      m_run[h] = mn;
      float ps = 0.0f;
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[h][e] *= alpha;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const float pj = __expf(sc[h][j] - mn);
        ps += pj;
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
          const uint4 vw = vq[j][i];
          acc[h][8 * i] = fmaf(pj, bf16_lo(vw.x), acc[h][8 * i]);
          acc[h][8 * i + 1] = fmaf(pj, bf16_hi(vw.x), acc[h][8 * i + 1]);
          acc[h][8 * i + 2] = fmaf(pj, bf16_lo(vw.y), acc[h][8 * i + 2]);
          acc[h][8 * i + 3] = fmaf(pj, bf16_hi(vw.y), acc[h][8 * i + 3]);
          acc[h][8 * i + 4] = fmaf(pj, bf16_lo(vw.z), acc[h][8 * i + 4]);
          acc[h][8 * i + 5] = fmaf(pj, bf16_hi(vw.z), acc[h][8 * i + 5]);
          acc[h][8 * i + 6] = fmaf(pj, bf16_lo(vw.w), acc[h][8 * i + 6]);
          acc[h][8 * i + 7] = fmaf(pj, bf16_hi(vw.w), acc[h][8 * i + 7]);
        }
      }
      s_run[h] = s_run[h] * alpha + ps;
    }
  }
  // the wave's totals: the 8 groups hold disjoint positions (the lanes of a group hold the
  // same ones); waves without a position keep m = -inf, s = 0, acc = 0
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    s_run[h] = groups_sum(s_run[h]);
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[h][e] = groups_sum(acc[h][e]);
  }
  const bool wave_bad = __any(bad);
  if (l < 8) {
#pragma unroll
    for (int h = 0; h < REP; ++h) {
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc_s[w][h][e0 + e] = acc[h][e];
      if (l == 0) {
        m_s[w][h] = m_run[h];
        s_s[w][h] = s_run[h];
      }
    }
    if (l == 0) bad_s[w] = wave_bad ? 1 : 0;
  }
  __syncthreads();
  bool any_bad = false;
#pragma unroll
  for (int ww = 0; ww < NW; ++ww) any_bad |= bad_s[ww] != 0;
  for (int i = tid; i < REP * DH; i += NT) {
    const int h = i / DH, d = i % DH;
    if (any_bad) {  // a corrupt slot anywhere in the context: NaN out
      out[i] = __int_as_float(0x7fc00000);
      continue;
    }
    float mx = m_s[0][h];
#pragma unroll
    for (int ww = 1; ww < NW; ++ww) mx = fmaxf(mx, m_s[ww][h]);
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float f = __expf(m_s[ww][h] - mx);  // 0 for a wave without positions
      num = fmaf(f, acc_s[ww][h][d], num);
      den = fmaf(f, s_s[ww][h], den);
    }
    out[i] = num / den;
  }
}

template <int DH>
void launch_decode(const Args& a, dim3 grid, hipStream_t st) {
  switch (a.rep) {
    case 1: hipLaunchKernelGGL((k_decode<1, DH>), grid, dim3(NT), 0, st, a); break;
    case 2: hipLaunchKernelGGL((k_decode<2, DH>), grid, dim3(NT), 0, st, a); break;
    case 3: hipLaunchKernelGGL((k_decode<3, DH>), grid, dim3(NT), 0, st, a); break;
    case 4: hipLaunchKernelGGL((k_decode<4, DH>), grid, dim3(NT), 0, st, a); break;
    case 5: hipLaunchKernelGGL((k_decode<5, DH>), grid, dim3(NT), 0, st, a); break;
    case 6: hipLaunchKernelGGL((k_decode<6, DH>), grid, dim3(NT), 0, st, a); break;
    case 7: hipLaunchKernelGGL((k_decode<7, DH>), grid, dim3(NT), 0, st, a); break;
    default: hipLaunchKernelGGL((k_decode<8, DH>), grid, dim3(NT), 0, st, a); break;
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
  if (head_dim != 64 && head_dim != 128)
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "head_dim must be 64 or 128");
  if (n_kv_heads < 1 || n_heads < n_kv_heads || n_heads % n_kv_heads != 0 || n_heads / n_kv_heads > MAX_REP)
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT,
                             "n_heads must be a multiple of n_kv_heads, at most 8 query heads per KV head");
  if (block_size < 1 || max_blocks < 1 || n_slots < 1)
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "block_size, max_blocks and n_slots must be positive");
  if (max_context < 1 || max_context > MAX_CONTEXT || (int64_t)max_context > max_blocks * block_size)
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT,
                             "max_context must be in [1, 1048576] and covered by max_blocks * block_size");
  if (rows * n_kv_heads > 0x7fffffff) return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "too many rows");
  if (n_slots > 0x7fffffff)
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "n_slots must be below 2^31");
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15u)
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "q, k_cache and v_cache must be 16-byte aligned");
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
  const dim3 grid((unsigned)(rows * n_kv_heads));
  if (head_dim == 64) launch_decode<64>(a, grid, (hipStream_t)stream);
  else launch_decode<128>(a, grid, (hipStream_t)stream);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return pbs::report_error(PBS_ERR_HIP, hipGetErrorString(e));
  return PBS_OK;
}
