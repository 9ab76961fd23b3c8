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
// Epilogue: the 64 x 64 fp32 tile goes to LDS; from there the wave writes the logits rows
// in bf16 (when asked; nearest, ties to even) and each lane takes one row of the tile: its
// largest fp32 value (NaN-propagating), rounded to bf16 once, fixes the lowest fp32 value
// that rounds to the same logit, and the first column at or above that bound is the row's
// first maximum among the bf16 logits. One 64-bit key per (row, tile) goes to the
// workspace (ordered bf16 value, then the complement of the column, so the largest key is
// the first maximum; NaN above everything). A second, tiny kernel reduces each row's keys
// to its token.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <utility>

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
constexpr int TST = TN + 8;   // fp32 per tile row in LDS (rows 4 apart sit 32 banks apart)
constexpr int WD = 4;         // weight chunks in flight per wave

struct Args {
  const uint16_t* hidden;
  const uint16_t* weight;
  uint16_t* out_logits;
  unsigned long long* part;  // [rows][tiles]: each (row, tile)'s largest (value, first column) key
  int64_t hstride;              // elements between hidden rows
  int rows, hdim, vocab;
  int kslice;                   // k_lmhead_lds: hidden elements per LDS-resident slice (divides hdim)
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

// The smallest fp32 value whose bf16 rounding (nearest, ties to even) is the bf16 value b;
// for b = +-0 the smallest one rounding to -0, since -0 and +0 compare equal as logits. b
// is not NaN. A value x no larger than the row's maximum, whose rounding is b, rounds to b
// exactly when x >= this bound (the rounding is monotonic).
__device__ __forceinline__ float bf16_class_low(uint32_t b) {
  if (b == 0u) b = 0x8000u;
  const uint32_t odd = b & 1u;  // a tie goes to the even neighbour
  if (b & 0x8000u) return b == 0xff80u ? -__builtin_inff() : __uint_as_float((b << 16) + 0x8000u - odd);
  return __uint_as_float((b << 16) - 0x8000u + odd);
}

// two fp32 values to packed bf16 (v_cvt_pk_bf16_f32: nearest, ties to even; the first in
// the low half)
__device__ __forceinline__ uint32_t pack_bf16(float x, float y) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x, y}, bf16x2));
}

// The 64 x 64 block of one wave: the fp32 tile to the wave's LDS tile, the bf16 logits rows
// from there (when asked), and each tile row's first maximum as a key into
// part[row][tile_id]: the row's largest fp32 value, rounded to bf16 once, gives the bound
// every value equal to the maximum as a bf16 logit reaches, and the first column at or
// above it is the first maximum; a NaN anywhere in the row makes the first NaN the answer.
__device__ __forceinline__ void epilogue(const Args& a, float* tile, const f32x16 (&acc)[2][2], int m0, int n0,
                                         int tile_id, int ntiles, int l, int half, int r32) {
  // accumulator register v of lane l holds row 8 (v / 4) + 4 (l / 32) + v % 4 and column
  // l % 32 of its 32 x 32 tile
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = 32 * i + 8 * (v >> 2) + 4 * half + (v & 3);
        tile[row * TST + 32 * j + r32] = acc[i][j][v];
      }
  __threadfence_block();  // the wave's tile writes are done before any lane reads them
  __builtin_amdgcn_wave_barrier();

  if (a.out_logits) {
    // eight lanes per row, eight columns (16 bytes of bf16) each; rows and columns past
    // the ends are skipped
#pragma unroll 1
    for (int r0 = 0; r0 < TM; r0 += 8) {
      const int row = r0 + (l >> 3);
      const int c = 8 * (l & 7);
      const int gr = m0 + row, gc = n0 + c;
      if (gr < a.rows && gc < a.vocab) {
        const float4 x0 = *(const float4*)(tile + row * TST + c);
        const float4 x1 = *(const float4*)(tile + row * TST + c + 4);
        const u4 q = {pack_bf16(x0.x, x0.y), pack_bf16(x0.z, x0.w), pack_bf16(x1.x, x1.y), pack_bf16(x1.z, x1.w)};
        uint16_t* dst = a.out_logits + (int64_t)gr * a.vocab + gc;
        if (gc + 8 <= a.vocab && ((uintptr_t)dst & 15u) == 0u) {
          *(u4*)dst = q;
        } else {
          for (int e = 0; e < 8 && gc + e < a.vocab; ++e) dst[e] = (uint16_t)(q[e >> 1] >> (16 * (e & 1)));
        }
      }
    }
  }

  // lane l: row l of the tile. Columns past the vocab (zero weights, so 0, or NaN beside
  // an infinite hidden value) are overwritten with -inf first; column 0 always exists, so
  // the first column at or above any bound is a real one. The logits reads above come
  // first: the wave's LDS operations complete in order.
  const int ncol = min(TN, a.vocab - n0);
  if (ncol < TN) {
#pragma unroll 1
    for (int c = ncol; c < TN; ++c) tile[l * TST + c] = -__builtin_inff();
  }
  float x[TN];
#pragma unroll
  for (int c4 = 0; c4 < TN / 4; ++c4) {
    const float4 q = *(const float4*)(tile + l * TST + 4 * c4);
    x[4 * c4] = q.x, x[4 * c4 + 1] = q.y, x[4 * c4 + 2] = q.z, x[4 * c4 + 3] = q.w;
  }
  float m = x[0];  // the largest value; NaN if the row holds one
#pragma unroll
  for (int c = 1; c + 1 < TN; c += 2)
    m = __builtin_elementwise_maximum(__builtin_elementwise_maximum(m, x[c]), x[c + 1]);
  m = __builtin_elementwise_maximum(m, x[TN - 1]);
  uint32_t ord;
  int first = 0;
  if (m != m) {  // the first NaN
    ord = 0xffffu;
#pragma unroll
    for (int c = TN - 1; c >= 0; --c) first = (x[c] != x[c]) ? c : first;
  } else {
    const uint32_t b = bf16_rne(m);
    ord = ord_bf16(b);
    const float lo = bf16_class_low(b);
#pragma unroll
    for (int c = TN - 1; c >= 0; --c) first = (x[c] >= lo) ? c : first;
  }
  if (m0 + l < a.rows) {
    const uint32_t col = (uint32_t)(n0 + first);
    a.part[(int64_t)(m0 + l) * ntiles + tile_id] =
        ((unsigned long long)ord << 32) | (unsigned long long)(0xffffffffu - col);
  }
  __threadfence_block();  // the tile is rewritten by the next row block
  __builtin_amdgcn_wave_barrier();
}

__global__ __launch_bounds__(64) void k_lmhead(Args a) {
  __shared__ float tile[TM * TST];
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
// Three waves per workgroup (192 columns) share the 64-row hidden block in LDS: the whole
// hidden dimension up to 1024, or larger ones in equal slices of at most 1024 staged one
// after the other (the accumulators carry over). The hidden fragments come from LDS
// (their own counter), so the memory counter tracks weight loads only: each wait before
// a multiply covers exactly the weight chunk it needs, with the later chunks in flight.
// ---------------------------------------------------------------------------------------
constexpr int LW_WAVES = 3;
constexpr int LDS_HMAX = 1024;  // largest hidden_dim of this kernel
// LDS bytes: the hidden block (64 rows of hidden_dim + 8 bf16), and the waves' fp32 tiles
// that replace it after the multiplies
constexpr size_t lds_hidden_bytes(int hdim) { return (size_t)TM * (size_t)(hdim + 8) * 2; }
constexpr size_t LDS_TILES = (size_t)LW_WAVES * TM * TST * 4;

// weight-only fragments and accumulators of one wave, D weight chunks in flight
template <int D>
struct FragsW {
  u4 w[D][2][4];
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

template <int D, int I, bool LW>
__device__ __forceinline__ void kstep_lds(FragsW<D>& f, __amdgpu_buffer_rsrc_t wrs, const uint32_t (&woff)[2],
                                          const uint16_t* hb, int hs, int r32, int half, int kc) {
  constexpr int B = I % D;
  u4 h[2][4];
  lds_frags(hb, hs, r32, half, kc, h);
  __builtin_amdgcn_sched_barrier(0);  // all eight LDS reads go out before the first multiply
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
    for (int t = 0; t < 2; ++t) load_frag(wrs, woff[t] + (uint32_t)((kc + D) * KC * 2), f.w[B][t]);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// chunks kc0 .. kc0 + D - 1 of a group (another group follows: every refill is valid)
template <int D, int I = 0>
__device__ __forceinline__ void kgroup_lds(FragsW<D>& f, __amdgpu_buffer_rsrc_t wrs, const uint32_t (&woff)[2],
                                           const uint16_t* hb, int hs, int r32, int half, int kc0) {
  if constexpr (I < D) {
    kstep_lds<D, I, true>(f, wrs, woff, hb, hs, r32, half, kc0 + I);
    kgroup_lds<D, I + 1>(f, wrs, woff, hb, hs, r32, half, kc0);
  }
}

// the last R chunks (D <= R < 2 D, or R = the whole row when it has fewer than 2 D)
template <int D, int R, int I = 0>
__device__ __forceinline__ void ktail_lds(FragsW<D>& f, __amdgpu_buffer_rsrc_t wrs, const uint32_t (&woff)[2],
                                          const uint16_t* hb, int hs, int r32, int half, int kc0) {
  if constexpr (I < R) {
    kstep_lds<D, I, (I + D < R)>(f, wrs, woff, hb, hs, r32, half, kc0 + I);
    ktail_lds<D, R, I + 1>(f, wrs, woff, hb, hs, r32, half, kc0);
  }
}

// D weight chunks in flight per wave: the launch takes the largest of 1, 2, 4 that is at
// most the row's chunk count nk, so every chunk of the prologue is one the wave
// multiplies (four measured fastest at hidden_dim 576: three, five, six and eight were
// 2-20 % slower); R = D + nk % D is the length of the last group. One tail per kernel: tails
// of several lengths in one kernel make the register allocation of every path worse.
template <int D, int R>
__global__ __launch_bounds__(64 * LW_WAVES) void k_lmhead_lds(Args a) {
  // the hidden block while the waves multiply, then (after a barrier) the waves' fp32
  // tiles over it
  extern __shared__ __align__(16) uint16_t smem[];
  const int ks = a.kslice;    // hidden elements per slice: hidden_dim in one or more slices
  const int hs = ks + 8;      // LDS row stride of the hidden block (the pad spreads the banks)
  uint16_t* hb = smem;        // [TM][hs]
  const int tid = threadIdx.x, l = tid & 63, wv = tid >> 6;
  float* tile = (float*)smem + wv * TM * TST;
  const int tile_id = blockIdx.x * LW_WAVES + wv;
  const int ntiles = (a.vocab + TN - 1) / TN;
  const int n0 = tile_id * TN;
  const bool active = tile_id < ntiles;  // waves past the last tile only help load the hidden block
  const int half = l >> 5, r32 = l & 31;
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.weight, (short)0, (int)((int64_t)a.vocab * a.hdim * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t hrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.hidden, (short)0, (int)((int64_t)a.rows * a.hstride * 2), 0x00020000);
  const int nk = ks / KC;  // chunks per slice
  const int nsl = a.hdim / ks;
  uint32_t woff0[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) woff0[t] = (uint32_t)((((int64_t)(n0 + 32 * t + r32)) * a.hdim + 32 * half) * 2);

  for (int m0 = 0; m0 < a.rows; m0 += TM) {
    FragsW<D> f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) f.acc[i][j] = (f32x16){};
    // the slices of the hidden dimension, each staged like a whole block; the
    // accumulators carry over, and the barrier after each slice's multiplies frees the
    // LDS block for the next slice (or, after the last, for the tiles)
#pragma unroll 1
    for (int sl = 0; sl < nsl; ++sl) {
      const int k0 = sl * ks;  // the slice's first hidden element
      uint32_t woff[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) woff[t] = woff0[t] + (uint32_t)(k0 * 2);
      // The hidden block (64 rows, zeros past the last, x hidden_dim; 16 bytes per piece) in
      // batches of up to 24 pieces per thread in flight. The first weight chunks go out right
      // behind the last batch, unconditionally (chunks past the row's end or past the
      // buffer's end read harmless data or zeros, never used), so the wait before that
      // batch's LDS writes leaves them in flight and the two latencies overlap.
      const int per_row = ks / 8;
      const int npiece = TM * per_row;
      constexpr int SB = 24, SSTEP = 64 * LW_WAVES;
      // piece q -> (row q / per_row, column piece): ((q + 0.5) * fl(1 / per_row)) is within
      // 2e-3 of (q + 0.5) / per_row for q < 2^14, and that quotient is at least
      // 0.5 / per_row >= 1 / 256 from an integer, so the truncation is exact
      const float inv_pr = 1.0f / (float)per_row;
      const int nbatch = (npiece - tid + SB * SSTEP - 1) / (SB * SSTEP);  // >= 1: npiece >= 512 > tid
      auto batch_loads = [&](int q0, u4 (&v)[SB]) {
#pragma unroll
        for (int u = 0; u < SB; ++u) {
          const int q = min(q0 + u * SSTEP, npiece - 1);
          const int r = (int)(((float)q + 0.5f) * inv_pr), c = q - r * per_row;
          v[u] = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(
                                            hrs, (uint32_t)((((int64_t)(m0 + r)) * a.hstride + k0 + 8 * c) * 2), 0, 0));
        }
      };
      // (a clamped piece is the last one, loaded and stored again with the same value)
      auto batch_stores = [&](int q0, const u4 (&v)[SB]) {
#pragma unroll
        for (int u = 0; u < SB; ++u) {
          const int q = min(q0 + u * SSTEP, npiece - 1);
          const int r = (int)(((float)q + 0.5f) * inv_pr), c = q - r * per_row;
          *(u4*)(hb + r * hs + 8 * c) = v[u];
        }
      };
      for (int b = 0; b + 1 < nbatch; ++b) {
        u4 v[SB];
        batch_loads(tid + b * SB * SSTEP, v);
        batch_stores(tid + b * SB * SSTEP, v);
      }
      {
        const int q0 = tid + (nbatch - 1) * SB * SSTEP;
        u4 v[SB];
        batch_loads(q0, v);
#pragma unroll
        for (int d = 0; d < D; ++d)
#pragma unroll
          for (int t = 0; t < 2; ++t) load_frag(wrs, woff[t] + (uint32_t)(d * KC * 2), f.w[d][t]);
        batch_stores(q0, v);
      }
      __syncthreads();
      if (active) {
        // whole groups of D chunks while another group follows them, then the last R
        int kc0 = 0;
        for (; kc0 + 2 * D <= nk; kc0 += D) kgroup_lds<D>(f, wrs, woff, hb, hs, r32, half, kc0);
        ktail_lds<D, R>(f, wrs, woff, hb, hs, r32, half, kc0);
      }
      __syncthreads();  // every wave's hidden reads are done: the next slice or the tiles overwrite the block
    }
    if (active) epilogue(a, tile, f.acc, m0, n0, tile_id, ntiles, l, half, r32);
    __syncthreads();  // the tiles are read before the next row block's hidden block
  }
}

// the k_lmhead_lds instantiation for a row of nk chunks (1 <= nk <= LDS_HMAX / KC)
template <int D, int... Rs>
const void* lds_kernel_for(int r, std::integer_sequence<int, Rs...>) {
  const void* k = nullptr;
  ((k = (r == D + Rs) ? (const void*)k_lmhead_lds<D, D + Rs> : k), ...);
  return k;
}
inline const void* lds_kernel(int nk) {
  if (nk >= 4) return lds_kernel_for<4>(4 + nk % 4, std::make_integer_sequence<int, 4>{});
  if (nk >= 2) return lds_kernel_for<2>(2 + nk % 2, std::make_integer_sequence<int, 2>{});
  return (const void*)k_lmhead_lds<1, 1>;
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

// k_lmhead_lds may take more than 64 KiB of dynamic LDS: raise the limit of the kernel for
// nk chunks once per device, on its first launch there (the first attribute call on a
// kernel loads its code, so the others are left alone)
constexpr int LDS_KERNELS = pbl::LDS_HMAX / pbl::KC;
std::atomic<bool> g_lds_attr[MAX_DEVICES][LDS_KERNELS + 1];

int lds_attribute(int nk) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return pbs::report_errorf(PBS_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= MAX_DEVICES) return pbs::report_errorf(PBS_ERR_HIP, "device index %d out of range", dev);
  if (g_lds_attr[dev][nk].load(std::memory_order_acquire)) return PBS_OK;
  e = hipFuncSetAttribute(pbl::lds_kernel(nk), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)std::max(pbl::lds_hidden_bytes(pbl::LDS_HMAX), pbl::LDS_TILES));
  if (e != hipSuccess) return pbs::report_errorf(PBS_ERR_HIP, "hipFuncSetAttribute failed: %s", hipGetErrorString(e));
  g_lds_attr[dev][nk].store(true, std::memory_order_release);
  return PBS_OK;
}

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
  // the LDS-resident hidden block: hidden_dim whole, or in the fewest equal slices of at
  // most LDS_HMAX elements (each a multiple of 64); otherwise the L2-fragment kernel
  int kslice = 0;
  if (hidden_dim <= pbl::LDS_HMAX) {
    kslice = (int)hidden_dim;
  } else {
    for (int n = 2; n <= 16 && !kslice; ++n)
      if (hidden_dim % (pbl::KC * n) == 0 && hidden_dim / n <= pbl::LDS_HMAX) kslice = (int)(hidden_dim / n);
  }
  a.kslice = kslice;
  if (kslice) {
    const size_t lds = std::max(pbl::lds_hidden_bytes(kslice), pbl::LDS_TILES);
    if (lds > 64 * 1024) {
      const int rc = lds_attribute(kslice / pbl::KC);
      if (rc != PBS_OK) return rc;
    }
    const dim3 grid((ntiles + pbl::LW_WAVES - 1) / pbl::LW_WAVES), block(64 * pbl::LW_WAVES);
    void* args[] = {&a};
    const hipError_t el = hipLaunchKernel(pbl::lds_kernel(kslice / pbl::KC), grid, block, args, lds,
                                          (hipStream_t)stream);
    if (el != hipSuccess) return pbs::report_errorf(PBS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(el));
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
