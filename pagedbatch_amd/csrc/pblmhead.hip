// Fused lm_head + greedy kernel for gfx950 (CDNA4), part of libpbsample.so.
//
// logits[b][v] = sum_k hidden[b][k] * weight[v][k] (pagedbatch/model.py:283, bf16
// nn.Linear without bias) on the matrix cores (v_mfma_f32_32x32x16_bf16, fp32
// accumulation), and in the same launch each row's torch.argmax over the bf16 logits
// (pagedbatch/sampling.py:12-13).
//
// One wave per workgroup owns 64 vocab columns (two 32-column MFMA tiles) and walks the
// rows in blocks of 64 (two 32-row tiles). Both operands are K-contiguous, so each lane
// reads its MFMA fragments straight from memory: per 64-element chunk of the hidden
// dimension, 64 contiguous bytes of one weight row (or hidden row) per lane, lanes 0-31
// taking the chunk's first half and lanes 32-63 its second. The four 16-byte pieces feed
// four MFMA steps; A and B assign the chunk's elements to the same K slots, so the sum is
// over every element exactly once whatever order the hardware uses inside a step. Four
// chunks of weight fragments are in flight while one multiplies; the loop is unrolled by
// four, so each buffer is refilled in place once its multiplies are issued (a copy of a
// register whose load is outstanding would wait for that load), and it holds no branch,
// so the compiler's waits before each multiply cover only the loads that multiply needs. The weight (vocab x
// hidden x 2 bytes, 56.6 MB for a 49152 x 576 head) is read from HBM once per row block:
// at decode batch sizes the kernel is HBM-bound on it, not MFMA-bound.
//
// Epilogue: the 64 x 64 fp32 tile is rounded to bf16 (nearest, ties to even) into LDS;
// from there the wave writes the logits rows (when asked) and each lane scans one row of
// the tile for its largest value as a key (ordered bf16 value, then the complement of the
// column, so the maximum key is the first maximum; NaN above everything), one 64-bit key
// per (row, tile) into the workspace. A second, tiny kernel reduces each row's keys to
// its token.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "pblmhead.h"
#include "pbsample.h"

namespace pbs {
int report_error(int code, const char* msg);
int report_errorf(int code, const char* fmt, ...);
}  // namespace pbs

namespace pbl {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int TM = 64;        // rows per block: two 32-row MFMA tiles
constexpr int TN = 64;        // vocab columns per workgroup: two 32-column MFMA tiles
constexpr int KC = 64;        // hidden elements per chunk: four MFMA steps of 16
constexpr int LROW = TN + 2;  // bf16 per tile row in LDS (the padding spreads the banks)
constexpr int WD = 4;         // weight chunks in flight per wave

struct Args {
  const uint16_t* hidden;
  const uint16_t* weight;
  uint16_t* out_logits;
  unsigned long long* part;  // [rows][tiles]: each (row, tile)'s largest (value, first column) key
  int64_t hstride;              // elements between hidden rows
  int rows, hdim, vocab;
};

// bf16 of an fp32 value: round to nearest, ties to even; NaN stays a (quiet) NaN
__device__ __forceinline__ uint32_t bf16_rne(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x0040u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// order of a bf16 value as an unsigned key: -0 folded onto +0, NaN above everything
__device__ __forceinline__ uint32_t ord_bf16(uint32_t r) {
  r = (r == 0x8000u) ? 0u : r;
  if ((r & 0x7fffu) > 0x7f80u) return 0xffffu;
  return r ^ ((r & 0x8000u) ? 0xffffu : 0x8000u);
}

// 32-bit key of a bf16 value in column c (< 64) of a tile: ordered value, then 63 - c
__device__ __forceinline__ uint32_t tile_key(uint32_t raw, int c) { return (ord_bf16(raw) << 16) | (uint32_t)(63 - c); }

// the lane's 64 bytes of one operand row: four 16-byte buffer loads, the whole offset in
// the VGPR operand, so rows past the buffer's end read zeros
__device__ __forceinline__ void load_frag(__amdgpu_buffer_rsrc_t rs, uint32_t off, u4 (&d)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
    d[i] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16u * (uint32_t)i, 0, 0));
}

// Operand fragments and accumulators of one wave's 64 x 64 block.
struct Frags {
  u4 w[WD][2][4];   // weight fragments of WD chunks (two column tiles each)
  u4 h[2][2][4];    // hidden fragments (two row tiles), one chunk ahead, two buffers
  f32x16 acc[2][2];
};

// Chunk kc0 + I of a group (kc0 a multiple of WD): its weight fragments sit in buffer
// I % WD and its hidden fragments in buffer I % 2. LH: load the next chunk's hidden
// fragments first; LW: refill the weight buffer with chunk kc0 + I + WD after the
// multiplies are issued. Everything is fixed at compile time, so the waits the compiler
// places before each multiply cover exactly the loads it needs.
template <int I, bool LH, bool LW>
__device__ __forceinline__ void kstep(Frags& f, __amdgpu_buffer_rsrc_t wrs, __amdgpu_buffer_rsrc_t hrs,
                                      const uint32_t (&woff)[2], const uint32_t (&hoff)[2], int kc) {
  constexpr int B = I % WD, P = I & 1;
  if constexpr (LH) {
#pragma unroll
    for (int t = 0; t < 2; ++t) load_frag(hrs, hoff[t] + (uint32_t)((kc + 1) * KC * 2), f.h[P ^ 1][t]);
  }
  __builtin_amdgcn_sched_barrier(0);  // the loads stay ahead of the multiplies
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        f.acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, f.h[P][i][s]),
                                                              __builtin_bit_cast(bf16x8, f.w[B][j][s]), f.acc[i][j],
                                                              0, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (LW) {
#pragma unroll
    for (int t = 0; t < 2; ++t) load_frag(wrs, woff[t] + (uint32_t)((kc + WD) * KC * 2), f.w[B][t]);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// the last R chunks (1 <= R < 2 WD), starting at kc0
template <int R, int I = 0>
__device__ __forceinline__ void ktail(Frags& f, __amdgpu_buffer_rsrc_t wrs, __amdgpu_buffer_rsrc_t hrs,
                                      const uint32_t (&woff)[2], const uint32_t (&hoff)[2], int kc0) {
  if constexpr (I < R) {
    kstep<I, (I + 1 < R), (I + WD < R)>(f, wrs, hrs, woff, hoff, kc0 + I);
    ktail<R, I + 1>(f, wrs, hrs, woff, hoff, kc0);
  }
}

// The 64 x 64 block of one wave: bf16 to the wave's LDS tile, the logits rows from there
// (when asked), and each tile row's largest key into part[row][tile_id].
__device__ __forceinline__ void epilogue(const Args& a, uint16_t* tile, const f32x16 (&acc)[2][2], int m0, int n0,
                                         int tile_id, int ntiles, int l, int half, int r32) {
    // the tile in bf16 to LDS: accumulator register v of lane l holds row
    // 8 (v / 4) + 4 (l / 32) + v % 4 and column l % 32 of its 32 x 32 tile
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int row = 32 * i + 8 * (v >> 2) + 4 * half + (v & 3);
          tile[row * LROW + 32 * j + r32] = (uint16_t)bf16_rne(acc[i][j][v]);
        }
    __threadfence_block();  // the wave's tile writes are done before any lane reads them
    __builtin_amdgcn_wave_barrier();

    if (a.out_logits) {
      // eight lanes per row, 16 bytes each; rows and columns past the ends are skipped
#pragma unroll 1
      for (int r0 = 0; r0 < TM; r0 += 8) {
        const int row = r0 + (l >> 3);
        const int c = 8 * (l & 7);
        const int gr = m0 + row, gc = n0 + c;
        if (gr < a.rows && gc < a.vocab) {
          uint16_t* dst = a.out_logits + (int64_t)gr * a.vocab + gc;
          const uint16_t* src = tile + row * LROW + c;
          if (gc + 8 <= a.vocab && ((uintptr_t)dst & 15u) == 0u) {
            const uint32_t* s32 = (const uint32_t*)src;  // c is even and rows are 132 bytes apart
            u4 q;
#pragma unroll
            for (int e = 0; e < 4; ++e) q[e] = s32[e];
            *(u4*)dst = q;
          } else {
            for (int e = 0; e < 8 && gc + e < a.vocab; ++e) dst[e] = src[e];
          }
        }
      }
    }

    // lane l: the largest key of tile row l (two columns per 32-bit LDS read, all reads
    // in flight); columns past the vocab count as nothing
    const uint32_t* trow = (const uint32_t*)(tile + l * LROW);
    const int ncol = min(TN, a.vocab - n0);
    uint32_t best = 0u;
    if (ncol == TN) {
#pragma unroll
      for (int c2 = 0; c2 < TN / 2; ++c2) {
        const uint32_t q = trow[c2];
        best = max(best, max(tile_key(q & 0xffffu, 2 * c2), tile_key(q >> 16, 2 * c2 + 1)));
      }
    } else {
      for (int c = 0; c < ncol; ++c) best = max(best, tile_key(tile[l * LROW + c], c));
    }
    if (m0 + l < a.rows) {
      const uint32_t col = (uint32_t)n0 + 63u - (best & 0xffffu);
      a.part[(int64_t)(m0 + l) * ntiles + tile_id] =
          ((unsigned long long)(best >> 16) << 32) | (unsigned long long)(0xffffffffu - col);
    }
  __threadfence_block();  // the tile is rewritten by the next row block
  __builtin_amdgcn_wave_barrier();
}

__global__ __launch_bounds__(64) void k_lmhead(Args a) {
  __shared__ uint16_t tile[TM * LROW];
    const int l = threadIdx.x;
  const int n0 = blockIdx.x * TN;
  const int half = l >> 5;  // which 32-element half of a chunk the lane reads
  const int r32 = l & 31;   // the lane's row within a 32-row (or 32-column) MFMA tile
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.weight, (short)0, (int)((int64_t)a.vocab * a.hdim * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t hrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.hidden, (short)0, (int)((int64_t)a.rows * a.hstride * 2), 0x00020000);
  const int nk = a.hdim / KC;
  // byte offsets of the lane's weight rows (two column tiles) at chunk 0
  uint32_t woff[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) woff[t] = (uint32_t)((((int64_t)(n0 + 32 * t + r32)) * a.hdim + 32 * half) * 2);

  for (int m0 = 0; m0 < a.rows; m0 += TM) {
    uint32_t hoff[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) hoff[t] = (uint32_t)((((int64_t)(m0 + 32 * t + r32)) * a.hstride + 32 * half) * 2);
    Frags f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) f.acc[i][j] = (f32x16){};
#pragma unroll
    for (int d = 0; d < WD; ++d)
      if (d < nk) {
#pragma unroll
        for (int t = 0; t < 2; ++t) load_frag(wrs, woff[t] + (uint32_t)(d * KC * 2), f.w[d][t]);
      }
#pragma unroll
    for (int t = 0; t < 2; ++t) load_frag(hrs, hoff[t], f.h[0][t]);
    // whole groups of WD chunks while another group follows them (every load valid), then
    // the last 1 .. 2 WD - 1 chunks
    int kc0 = 0;
    for (; kc0 + 2 * WD <= nk; kc0 += WD) {
      kstep<0, true, true>(f, wrs, hrs, woff, hoff, kc0);
      kstep<1, true, true>(f, wrs, hrs, woff, hoff, kc0 + 1);
      kstep<2, true, true>(f, wrs, hrs, woff, hoff, kc0 + 2);
      kstep<3, true, true>(f, wrs, hrs, woff, hoff, kc0 + 3);
    }
    switch (nk - kc0) {
      case 1: ktail<1>(f, wrs, hrs, woff, hoff, kc0); break;
      case 2: ktail<2>(f, wrs, hrs, woff, hoff, kc0); break;
      case 3: ktail<3>(f, wrs, hrs, woff, hoff, kc0); break;
      case 4: ktail<4>(f, wrs, hrs, woff, hoff, kc0); break;
      case 5: ktail<5>(f, wrs, hrs, woff, hoff, kc0); break;
      case 6: ktail<6>(f, wrs, hrs, woff, hoff, kc0); break;
      default: ktail<7>(f, wrs, hrs, woff, hoff, kc0); break;
    }

    epilogue(a, tile, f.acc, m0, n0, (int)blockIdx.x, (int)gridDim.x, l, half, r32);
    __syncthreads();  // the tile is rewritten by the next row block
  }
}

// ---------------------------------------------------------------------------------------
// hidden_dim <= 1024: three waves per workgroup (192 columns) share the 64-row hidden block
// in LDS, so the hidden fragments come from LDS (their own counter) and the memory
// counter tracks weight loads only: each wait before a multiply covers exactly the weight
// chunk it needs, with the later chunks still in flight.
// ---------------------------------------------------------------------------------------
constexpr int LW_WAVES = 3;
constexpr int LDS_HMAX = 1024;  // largest hidden_dim of this kernel

// weight-only fragments and accumulators of one wave
struct FragsW {
  u4 w[WD][2][4];
  f32x16 acc[2][2];
};

// hidden fragments of chunk kc for row tiles 0 and 1 from the LDS block (row stride hs)
__device__ __forceinline__ void lds_frags(const uint16_t* hb, int hs, int r32, int half, int kc, u4 (&h)[2][4]) {
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int s = 0; s < 4; ++s)
      h[t][s] = *(const u4*)(hb + (32 * t + r32) * hs + kc * KC + 32 * half + 8 * s);
}

template <int I, bool LW>
__device__ __forceinline__ void kstep_lds(FragsW& f, __amdgpu_buffer_rsrc_t wrs, const uint32_t (&woff)[2],
                                          const uint16_t* hb, int hs, int r32, int half, int kc) {
  constexpr int B = I % WD;
  u4 h[2][4];
  lds_frags(hb, hs, r32, half, kc, h);
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        f.acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, h[i][s]),
                                                              __builtin_bit_cast(bf16x8, f.w[B][j][s]), f.acc[i][j],
                                                              0, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (LW) {
#pragma unroll
    for (int t = 0; t < 2; ++t) load_frag(wrs, woff[t] + (uint32_t)((kc + WD) * KC * 2), f.w[B][t]);
  }
  __builtin_amdgcn_sched_barrier(0);
}

template <int R, int I = 0>
__device__ __forceinline__ void ktail_lds(FragsW& f, __amdgpu_buffer_rsrc_t wrs, const uint32_t (&woff)[2],
                                          const uint16_t* hb, int hs, int r32, int half, int kc0) {
  if constexpr (I < R) {
    kstep_lds<I, (I + WD < R)>(f, wrs, woff, hb, hs, r32, half, kc0 + I);
    ktail_lds<R, I + 1>(f, wrs, woff, hb, hs, r32, half, kc0);
  }
}

__global__ __launch_bounds__(64 * LW_WAVES) void k_lmhead_lds(Args a) {
  extern __shared__ uint16_t smem[];
  const int hs = a.hdim + 8;  // LDS row stride of the hidden block (the pad spreads the banks)
  uint16_t* hb = smem;        // [TM][hs]
  const int tid = threadIdx.x, l = tid & 63, wv = tid >> 6;
  uint16_t* tile = smem + TM * hs + wv * TM * LROW;
  const int tile_id = blockIdx.x * LW_WAVES + wv;
  const int ntiles = (a.vocab + TN - 1) / TN;
  const int n0 = tile_id * TN;
  const bool active = tile_id < ntiles;  // waves past the last tile only help load the hidden block
  const int half = l >> 5, r32 = l & 31;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.weight, (short)0, (int)((int64_t)a.vocab * a.hdim * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t hrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.hidden, (short)0, (int)((int64_t)a.rows * a.hstride * 2), 0x00020000);
  const int nk = a.hdim / KC;
  uint32_t woff[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) woff[t] = (uint32_t)((((int64_t)(n0 + 32 * t + r32)) * a.hdim + 32 * half) * 2);

  for (int m0 = 0; m0 < a.rows; m0 += TM) {
    FragsW f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) f.acc[i][j] = (f32x16){};
    // The hidden block (64 rows, zeros past the last, x hidden_dim; 16 bytes per piece):
    // up to 24 pieces per thread in flight at once, and the first weight chunks go out
    // right behind them, so the two latencies overlap.
    const int per_row = a.hdim / 8;
    const int npiece = TM * per_row;
    constexpr int SB = 24;
    for (int q0 = tid; q0 < npiece; q0 += SB * 64 * LW_WAVES) {
      u4 v[SB];
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int q = q0 + u * 64 * LW_WAVES;
        const int r = q / per_row, c = q - r * per_row;
        v[u] = q < npiece ? __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(
                                                   hrs, (uint32_t)((((int64_t)(m0 + r)) * a.hstride + 8 * c) * 2),
                                                   0, 0))
                          : (u4){0u, 0u, 0u, 0u};
      }
      // (every thread takes this first batch: npiece >= 64 * 8 > 64 * LW_WAVES)
      if (q0 == tid && active) {
#pragma unroll
        for (int d = 0; d < WD; ++d)
          if (d < nk) {
#pragma unroll
            for (int t = 0; t < 2; ++t) load_frag(wrs, woff[t] + (uint32_t)(d * KC * 2), f.w[d][t]);
          }
      }
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int q = q0 + u * 64 * LW_WAVES;
        const int r = q / per_row, c = q - r * per_row;
        if (q < npiece) *(u4*)(hb + r * hs + 8 * c) = v[u];
      }
    }
    __syncthreads();
    if (active) {
      int kc0 = 0;
      for (; kc0 + 2 * WD <= nk; kc0 += WD) {
        kstep_lds<0, true>(f, wrs, woff, hb, hs, r32, half, kc0);
        kstep_lds<1, true>(f, wrs, woff, hb, hs, r32, half, kc0 + 1);
        kstep_lds<2, true>(f, wrs, woff, hb, hs, r32, half, kc0 + 2);
        kstep_lds<3, true>(f, wrs, woff, hb, hs, r32, half, kc0 + 3);
      }
      switch (nk - kc0) {
        case 1: ktail_lds<1>(f, wrs, woff, hb, hs, r32, half, kc0); break;
        case 2: ktail_lds<2>(f, wrs, woff, hb, hs, r32, half, kc0); break;
        case 3: ktail_lds<3>(f, wrs, woff, hb, hs, r32, half, kc0); break;
        case 4: ktail_lds<4>(f, wrs, woff, hb, hs, r32, half, kc0); break;
        case 5: ktail_lds<5>(f, wrs, woff, hb, hs, r32, half, kc0); break;
        case 6: ktail_lds<6>(f, wrs, woff, hb, hs, r32, half, kc0); break;
        default: ktail_lds<7>(f, wrs, woff, hb, hs, r32, half, kc0); break;
      }
      epilogue(a, tile, f.acc, m0, n0, tile_id, ntiles, l, half, r32);
    }
    __syncthreads();  // the hidden block and the tiles are rewritten by the next row block
  }
}

// One workgroup of 256 threads per row: the largest of the row's tile keys (up to four
// independent loads in flight per thread, so the row costs about one memory latency); its
// low word is the complement of the first maximum's column. A second launch, because the
// tiles of a row are spread over every XCD: making their keys visible to one workgroup
// inside the first launch would take a device-scope release per workgroup, which writes
// back that XCD's L2.
__global__ __launch_bounds__(256) void k_lmhead_finish(const unsigned long long* part, int ntiles,
                                                      int32_t* out_token) {
  __shared__ unsigned long long red[4];
  const int b = blockIdx.x, t = threadIdx.x;
  const unsigned long long* row = part + (int64_t)b * ntiles;
  unsigned long long best = 0u;
  for (int i0 = t; i0 < ntiles; i0 += 4 * 256) {
    unsigned long long k[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) k[u] = (i0 + 256 * u < ntiles) ? row[i0 + 256 * u] : 0ull;
#pragma unroll
    for (int u = 0; u < 4; ++u) best = k[u] > best ? k[u] : best;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(best, off, 64);
    best = o > best ? o : best;
  }
  if ((t & 63) == 0) red[t >> 6] = best;
  __syncthreads();
  if (t == 0) {
#pragma unroll
    for (int w = 1; w < 4; ++w) best = red[w] > best ? red[w] : best;
    out_token[b] = (int32_t)(0xffffffffu - (uint32_t)best);
  }
}

}  // namespace pbl

// The workspace of pbs_lm_head_argmax_noalloc: one array per GPU, in the library's own
// device memory, kept until the process ends. Host code never passes `scratch` itself (its
// host-side name is not a device address): the device address comes from
// hipGetSymbolAddress, once per device, with that device current.
constexpr size_t SCRATCH_KEYS = (size_t)1 << 19;  // 4 MiB: rows x 64-column tiles of 8 bytes
static __device__ __align__(256) unsigned long long scratch[SCRATCH_KEYS];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[MAX_DEVICES];  // scratch's device address on each GPU (null until its first call)

int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return pbs::report_errorf(PBS_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= MAX_DEVICES) return pbs::report_errorf(PBS_ERR_HIP, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return pbs::report_errorf(PBS_ERR_HIP, "hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return PBS_OK;
}
}  // namespace

extern "C" {

size_t pbs_lm_head_workspace_bytes(int64_t rows, int64_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  return (size_t)rows * (size_t)((vocab + pbl::TN - 1) / pbl::TN) * sizeof(uint64_t);
}

int pbs_lm_head_argmax(const uint16_t* hidden, int64_t hidden_stride, const uint16_t* weight, int64_t rows,
                       int64_t hidden_dim, int64_t vocab, uint16_t* out_logits, int32_t* out_token,
                       void* workspace, size_t workspace_bytes, void* stream) {
  if (rows < 0) return pbs::report_errorf(PBS_ERR_INVALID_ARGUMENT, "rows is negative (%lld)", (long long)rows);
  if (rows == 0) return PBS_OK;
  if (!hidden || !weight || !out_token || !workspace)
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "null device pointer among the required arguments");
  if (hidden_dim <= 0 || hidden_dim % pbl::KC != 0)
    return pbs::report_errorf(PBS_ERR_INVALID_ARGUMENT, "hidden_dim %lld is not a positive multiple of %d",
                              (long long)hidden_dim, pbl::KC);
  if (vocab <= 0) return pbs::report_errorf(PBS_ERR_INVALID_ARGUMENT, "vocab %lld <= 0", (long long)vocab);
  if (hidden_stride < hidden_dim || hidden_stride % 8 != 0)
    return pbs::report_errorf(PBS_ERR_INVALID_ARGUMENT, "hidden_stride %lld: below hidden_dim or not a multiple of 8",
                              (long long)hidden_stride);
  if (vocab * hidden_dim * 2 >= ((int64_t)1 << 31) || rows * hidden_stride * 2 >= ((int64_t)1 << 31))
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "weight or hidden larger than 2^31 bytes");
  if (((uintptr_t)hidden & 15u) != 0u || ((uintptr_t)weight & 15u) != 0u)
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "hidden and weight must be 16-byte aligned");
  if (((uintptr_t)workspace & 7u) != 0u)
    return pbs::report_error(PBS_ERR_INVALID_ARGUMENT, "workspace must be 8-byte aligned");
  if (workspace_bytes < pbs_lm_head_workspace_bytes(rows, vocab))
    return pbs::report_errorf(PBS_ERR_WORKSPACE, "workspace of %zu bytes, %zu needed", workspace_bytes,
                              pbs_lm_head_workspace_bytes(rows, vocab));
  pbl::Args a;
  a.hidden = hidden;
  a.weight = weight;
  a.out_logits = out_logits;
  a.part = (unsigned long long*)workspace;
  a.hstride = hidden_stride;
  a.rows = (int)rows;
  a.hdim = (int)hidden_dim;
  a.vocab = (int)vocab;
  const unsigned ntiles = (unsigned)((vocab + pbl::TN - 1) / pbl::TN);
  if (hidden_dim <= pbl::LDS_HMAX) {
    const size_t lds = ((size_t)pbl::TM * (size_t)(hidden_dim + 8) + (size_t)pbl::LW_WAVES * pbl::TM * pbl::LROW) * 2;
    static bool attr_set = false;  // every device takes the same attribute value
    if (!attr_set) {
      const hipError_t ea =
          hipFuncSetAttribute((const void*)pbl::k_lmhead_lds, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)((pbl::TM * (pbl::LDS_HMAX + 8) + pbl::LW_WAVES * pbl::TM * pbl::LROW) * 2));
      if (ea != hipSuccess)
        return pbs::report_errorf(PBS_ERR_HIP, "hipFuncSetAttribute failed: %s", hipGetErrorString(ea));
      attr_set = true;
    }
    hipLaunchKernelGGL(pbl::k_lmhead_lds, dim3((ntiles + pbl::LW_WAVES - 1) / pbl::LW_WAVES),
                       dim3(64 * pbl::LW_WAVES), lds, (hipStream_t)stream, a);
  } else {
    hipLaunchKernelGGL(pbl::k_lmhead, dim3(ntiles), dim3(64), 0, (hipStream_t)stream, a);
  }
  hipLaunchKernelGGL(pbl::k_lmhead_finish, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream,
                     (const unsigned long long*)a.part, (int)ntiles, out_token);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return pbs::report_errorf(PBS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  return PBS_OK;
}

int pbs_lm_head_argmax_noalloc(const uint16_t* hidden, int64_t hidden_stride, const uint16_t* weight, int64_t rows,
                               int64_t hidden_dim, int64_t vocab, uint16_t* out_logits, int32_t* out_token,
                               void* stream) {
  if (rows < 0) return pbs::report_errorf(PBS_ERR_INVALID_ARGUMENT, "rows is negative (%lld)", (long long)rows);
  if (rows == 0) return PBS_OK;
  if (vocab > 0 && pbs_lm_head_workspace_bytes(rows, vocab) > sizeof(scratch))
    return pbs::report_errorf(PBS_ERR_WORKSPACE,
                              "rows x vocab tiles need %zu bytes of scratch, the library holds %zu per GPU "
                              "(rows * ceil(vocab / 64) <= %zu)",
                              pbs_lm_head_workspace_bytes(rows, vocab), sizeof(scratch), SCRATCH_KEYS);
  // every other argument is checked by pbs_lm_head_argmax, before anything is launched
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != PBS_OK) return rc;
  return pbs_lm_head_argmax(hidden, hidden_stride, weight, rows, hidden_dim, vocab, out_logits, out_token, ws,
                            sizeof(scratch), stream);
}

}  // extern "C"
