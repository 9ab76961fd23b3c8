// pbsample.hip -- gfx950 (MI355X) token sampler: greedy / temperature / top-k / top-p / draw.
//
// Replaces the per-row torch op chain of pagedbatch/sampling.py:10-27 (called once per
// row from pagedbatch/engine.py:133-139) with one launch per engine step: one 1024-thread
// workgroup per output row, the row held in VGPRs after a single coalesced 16-byte-load
// pass over HBM (or re-streamed from memory when it does not fit), per-row selection
// state in LDS.
//
// Selection works on order-preserving integer keys ("ords") of the values:
//   16-bit logits (bf16 / fp16): every distinct value has its own ord, so a 64K-bin
//     count histogram in LDS (packed u16 counters) is an exact summary of the row. The
//     softmax weight exp(x - max) depends only on the value, so the mass of a value is
//     count * weight, computed once per distinct value in fp64. Top-k threshold, top-p
//     cutoff and the inverse-CDF draw are prefix searches over that histogram in
//     descending value order; only "which of the tied tokens" looks at indices again.
//   fp32 logits: x = fp32(v)/T per element (exact division), searches by bisection on
//     32-bit ords of x with exact fp64 mass sums.
//
// The order everywhere is (scaled value descending, index ascending): the order
// pagedbatch's top-p sort establishes (sampling.py:19), with ties broken by index.

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "pbsample.h"

namespace pbs {

constexpr int NT = 1024;           // threads per workgroup: one workgroup per row
constexpr int NWAVE = NT / 64;     // wave64
constexpr int HIST_WORDS = 32768;  // 64K packed u16 counters = 128 KB of LDS
constexpr int NGROUP = 256;        // histogram groups of 256 ords (high byte of a 16-bit ord)

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// Workgroup barrier that orders LDS traffic only. Unlike __syncthreads() it does not make
// the wave wait for its outstanding global loads, so row chunks keep streaming in while
// the workgroup synchronises on LDS state.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---------------------------------------------------------------------------------------
// wave64 primitives on DPP (no LDS round trips). Lanes whose DPP source is outside the
// row, or whose row is masked off, receive `old` (the operation's identity).
// ---------------------------------------------------------------------------------------
constexpr int ROW_SHR1 = 0x111, ROW_SHR2 = 0x112, ROW_SHR4 = 0x114, ROW_SHR8 = 0x118;
constexpr int ROW_BCAST15 = 0x142, ROW_BCAST31 = 0x143;

template <int CTRL, int RM = 0xf>
__device__ __forceinline__ uint32_t dpp(uint32_t v, uint32_t old) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, RM, 0xf, false);
}

__device__ __forceinline__ uint32_t bcast_u32(uint32_t v, int lane) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}
__device__ __forceinline__ float bcast_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ double bcast_f64(double v, int lane) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = bcast_u32((uint32_t)b, lane), hi = bcast_u32((uint32_t)(b >> 32), lane);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// inclusive prefix sums in lane order
__device__ __forceinline__ uint32_t wscan_u32(uint32_t v) {
  v += dpp<ROW_SHR1>(v, 0u);
  v += dpp<ROW_SHR2>(v, 0u);
  v += dpp<ROW_SHR4>(v, 0u);
  v += dpp<ROW_SHR8>(v, 0u);
  v += dpp<ROW_BCAST15, 0xa>(v, 0u);
  v += dpp<ROW_BCAST31, 0xc>(v, 0u);
  return v;
}
template <int CTRL, int RM = 0xf>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = dpp<CTRL, RM>((uint32_t)b, 0u), hi = dpp<CTRL, RM>((uint32_t)(b >> 32), 0u);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double wscan_f64(double v) {
  v += dpp_f64<ROW_SHR1>(v);
  v += dpp_f64<ROW_SHR2>(v);
  v += dpp_f64<ROW_SHR4>(v);
  v += dpp_f64<ROW_SHR8>(v);
  v += dpp_f64<ROW_BCAST15, 0xa>(v);
  v += dpp_f64<ROW_BCAST31, 0xc>(v);
  return v;
}
__device__ __forceinline__ uint32_t wsum_u32(uint32_t v) { return bcast_u32(wscan_u32(v), 63); }
__device__ __forceinline__ double wsum_f64(double v) { return bcast_f64(wscan_f64(v), 63); }

__device__ __forceinline__ float wmax_f32(float v) {
  const uint32_t ninf = 0xff800000u;
#define PBS_MAXSTEP(C, R) v = fmaxf(v, __uint_as_float(dpp<C, R>(__float_as_uint(v), ninf)))
  PBS_MAXSTEP(ROW_SHR1, 0xf);
  PBS_MAXSTEP(ROW_SHR2, 0xf);
  PBS_MAXSTEP(ROW_SHR4, 0xf);
  PBS_MAXSTEP(ROW_SHR8, 0xf);
  PBS_MAXSTEP(ROW_BCAST15, 0xa);
  PBS_MAXSTEP(ROW_BCAST31, 0xc);
#undef PBS_MAXSTEP
  return bcast_f32(v, 63);
}
__device__ __forceinline__ int wmin_i32(int v) {
  const uint32_t big = 0x7fffffffu;
#define PBS_MINSTEP(C, R) v = min(v, (int)dpp<C, R>((uint32_t)v, big))
  PBS_MINSTEP(ROW_SHR1, 0xf);
  PBS_MINSTEP(ROW_SHR2, 0xf);
  PBS_MINSTEP(ROW_SHR4, 0xf);
  PBS_MINSTEP(ROW_SHR8, 0xf);
  PBS_MINSTEP(ROW_BCAST15, 0xa);
  PBS_MINSTEP(ROW_BCAST31, 0xc);
#undef PBS_MINSTEP
  return (int)bcast_u32((uint32_t)v, 63);
}

__device__ __forceinline__ uint32_t wmax_u32(uint32_t v) {
#define PBS_UMAXSTEP(C, R) v = max(v, dpp<C, R>(v, 0u))
  PBS_UMAXSTEP(ROW_SHR1, 0xf);
  PBS_UMAXSTEP(ROW_SHR2, 0xf);
  PBS_UMAXSTEP(ROW_SHR4, 0xf);
  PBS_UMAXSTEP(ROW_SHR8, 0xf);
  PBS_UMAXSTEP(ROW_BCAST15, 0xa);
  PBS_UMAXSTEP(ROW_BCAST31, 0xc);
#undef PBS_UMAXSTEP
  return bcast_u32(v, 63);
}
__device__ __forceinline__ uint32_t wmin_u32(uint32_t v) {
#define PBS_UMINSTEP(C, R) v = min(v, dpp<C, R>(v, 0xffffffffu))
  PBS_UMINSTEP(ROW_SHR1, 0xf);
  PBS_UMINSTEP(ROW_SHR2, 0xf);
  PBS_UMINSTEP(ROW_SHR4, 0xf);
  PBS_UMINSTEP(ROW_SHR8, 0xf);
  PBS_UMINSTEP(ROW_BCAST15, 0xa);
  PBS_UMINSTEP(ROW_BCAST31, 0xc);
#undef PBS_UMINSTEP
  return bcast_u32(v, 63);
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }
__device__ __forceinline__ int first_lane(uint64_t m) { return __ffsll((unsigned long long)m) - 1; }

// exp(d) for d <= 0 in fp64: Cody-Waite reduction by ln 2 (fdlibm's split constants),
// degree-13 Taylor polynomial on |r| <= ln(2)/2 (truncation < 1e-17), exact scaling.
__device__ __forceinline__ double exp_neg(double d) {
  if (!(d > -745.2)) return 0.0;
  const double n = rint(d * 1.4426950408889634074);
  double r = fma(-n, 6.93147180369123816490e-01, d);
  r = fma(-n, 1.90821492927058770002e-10, r);
  double q = 1.0 / 6227020800.0;  // 1/13!
  q = fma(q, r, 1.0 / 479001600.0);
  q = fma(q, r, 1.0 / 39916800.0);
  q = fma(q, r, 1.0 / 3628800.0);
  q = fma(q, r, 1.0 / 362880.0);
  q = fma(q, r, 1.0 / 40320.0);
  q = fma(q, r, 1.0 / 5040.0);
  q = fma(q, r, 1.0 / 720.0);
  q = fma(q, r, 1.0 / 120.0);
  q = fma(q, r, 1.0 / 24.0);
  q = fma(q, r, 1.0 / 6.0);
  q = fma(q, r, 0.5);
  q = fma(q, r, 1.0);
  q = fma(q, r, 1.0);
  return ldexp(q, (int)n);
}

// ---------------------------------------------------------------------------------------
// element types and keys
// ---------------------------------------------------------------------------------------
template <int DT>
struct DTraits;
template <>
struct DTraits<PBS_DTYPE_F32> {
  static constexpr int EPV = 4;  // elements per 16-byte vector
  static constexpr bool B16 = false;
};
template <>
struct DTraits<PBS_DTYPE_F16> {
  static constexpr int EPV = 8;
  static constexpr bool B16 = true;
};
template <>
struct DTraits<PBS_DTYPE_BF16> {
  static constexpr int EPV = 8;
  static constexpr bool B16 = true;
};

template <int DT>
__device__ __forceinline__ uint32_t elem_raw(const u4& q, int e) {
  if constexpr (DTraits<DT>::B16) {
    const uint32_t w = q[e >> 1];
    return (e & 1) ? (w >> 16) : (w & 0xffffu);
  } else {
    return q[e];
  }
}

template <int DT>
__device__ __forceinline__ float raw_to_float(uint32_t raw) {
  if constexpr (DT == PBS_DTYPE_BF16) {
    return __uint_as_float(raw << 16);
  } else if constexpr (DT == PBS_DTYPE_F16) {
    return __half2float(__ushort_as_half((unsigned short)raw));
  } else {
    return __uint_as_float(raw);
  }
}

// Order-preserving keys. -0 is folded onto +0 first so that the two zeros, which compare
// equal, form one tie group. NaNs land above +inf (positive) or below -inf (negative);
// stochastic rows holding NaN are rejected before any key is used.
__device__ __forceinline__ uint32_t ord16(uint32_t raw) {
  raw = (raw == 0x8000u) ? 0u : raw;
  return raw ^ ((raw & 0x8000u) ? 0xffffu : 0x8000u);
}
__device__ __forceinline__ uint32_t raw_of_ord16(uint32_t o) {
  return (o & 0x8000u) ? (o ^ 0x8000u) : (o ^ 0xffffu);
}
__device__ __forceinline__ uint32_t ord32(float x) {
  uint32_t b = __float_as_uint(x);
  b = (b == 0x80000000u) ? 0u : b;
  return b ^ ((b & 0x80000000u) ? 0xffffffffu : 0x80000000u);
}
__device__ __forceinline__ float float_of_ord32(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o ^ 0x80000000u) : (o ^ 0xffffffffu));
}
template <int DT>
__device__ __forceinline__ uint32_t ord16_neg_inf() {
  return DT == PBS_DTYPE_BF16 ? ord16(0xff80u) : ord16(0xfc00u);
}
template <int DT>
__device__ __forceinline__ uint32_t ord16_pos_inf() {
  return DT == PBS_DTYPE_BF16 ? ord16(0x7f80u) : ord16(0x7c00u);
}

typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// ords of the two 16-bit values packed in w, without folding -0 onto +0 (-0 gets ord
// 0x7fff, which the histogram merges into +0's 0x8000 after the stream)
__device__ __forceinline__ uint32_t ord16_pair(uint32_t w) {
  const s16x2 sg = __builtin_bit_cast(s16x2, w) >> (s16x2){15, 15};
  return w ^ (__builtin_bit_cast(uint32_t, sg) | 0x80008000u);
}
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}
__device__ __forceinline__ uint32_t pk_min_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}

// x = RN(a / T), the IEEE single-precision quotient of sampling.py:14.
// With r = RN(1/T): q0 = RN(a*r) is within an ulp of a/T, the FMA residual a - q0*T is
// exact, and q1 = RN(q0 + res*r) is the correctly rounded quotient (Markstein's
// theorem); the second correction makes the "within an ulp" premise certain. Every
// intermediate must stay normal: zero, inf and NaN divide exactly by multiplication,
// subnormal inputs and quotients near the under/overflow thresholds take the full
// division sequence.
struct Divider {
  float T, r;
  int elo, ehi;  // biased exponents of a for which the FMA sequence is safe
  __device__ __forceinline__ void init(float T_) {
    T = T_;
    r = 1.0f / T_;
    const int et = (int)((__float_as_uint(T_) >> 23) & 0xff);
    // |a| in [2^(e-127), 2^(e-126)) and |T| in [2^(et-127), 2^(et-126)) put the quotient's
    // biased exponent in [e-et+126, e-et+128]. Keep it in [26, 253] (correction terms stay
    // normal, no overflow) and keep the residual a - q*T, about 2^-24 |a|, normal (e >= 26).
    // T and 1/T must be normal themselves, otherwise every element takes the full division.
    if (et >= 1 && et <= 250) {
      elo = max(26, et - 100);
      ehi = min(254, et + 125);
    } else {
      elo = 1;
      ehi = 0;
    }
  }
  __device__ __forceinline__ float operator()(float a) const {
    const int e = (int)((__float_as_uint(a) >> 23) & 0xff);
    if (e >= elo && e <= ehi) {
      float q = a * r;
      float res = fmaf(-q, T, a);
      q = fmaf(res, r, q);
      res = fmaf(-q, T, a);
      return fmaf(res, r, q);
    }
    if ((__float_as_uint(a) & 0x7fffffffu) == 0u) return a * r;  // +-0
    if (e == 255) return a * r;                                   // +-inf, NaN
    return a / T;
  }
};

// ---------------------------------------------------------------------------------------
// kernel arguments and per-row shared state
// ---------------------------------------------------------------------------------------
struct KArgs {
  const void* logits;
  int64_t n_logit_rows;
  int64_t row_stride;  // elements
  int vocab;
  int nvec;            // 16-byte vectors per row (vector sources), ceil(vocab/EPV) otherwise
  const int32_t* row_map;
  const float* temperature;
  const int32_t* top_k;
  const float* top_p;
  const float* uniform;
  int32_t* out_token;
  int32_t* out_status;
  float* out_probs;
  uint8_t* out_kept;
  pbs_row_info* out_info;
};

struct RowState {
  int status;
  float m;             // largest scaled logit
  float x_kth;
  float x_cut;
  uint32_t kord_lo;    // top-k set = ords >= kord_lo
  uint32_t cut_lo;     // ords in [cut_lo, cut_hi]: the cutoff tie group (n_cut_keep kept)
  uint32_t cut_hi;     // ords above cut_hi are kept whole
  int n_cut_tie;
  int n_cut_keep;
  int n_kept;
  uint32_t sel_lo, sel_hi;  // tie group the draw landed in
  int sel_rank;             // index rank inside it
  int sel_n;                // its size
  double zk, zp, target;
};

struct __align__(16) Smem {
  uint32_t hist[HIST_WORDS];     // 16-bit rows: packed u16 counts per ord; reused by index selection
  uint32_t gcount[NGROUP];       // count of each group of 256 ords
  uint32_t gabove_cnt[NGROUP];   // count strictly above the group (descending order)
  double gmass[NGROUP];          // fp64 mass of each group
  double gabove_mass[NGROUP];    // mass strictly above the group
  double red_d[NWAVE];
  float red_f[NWAVE];
  int red_i[2 * NWAVE];
  int sel_jstar, sel_rank, sel_index;
  RowState st;
};

// ---------------------------------------------------------------------------------------
// block reductions (1024 threads, 16 waves)
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float block_max_f(float v, Smem& s) {
  v = wmax_f32(v);
  if (lane_id() == 0) s.red_f[wave_id()] = v;
  __syncthreads();
  float r = s.red_f[0];
#pragma unroll
  for (int w = 1; w < NWAVE; ++w) r = fmaxf(r, s.red_f[w]);
  __syncthreads();
  return r;
}

// row maximum (NaN-free values) and whether any thread saw a NaN: returns NaN then
__device__ __forceinline__ float block_max_nan(float v, int nan, Smem& s) {
  v = wmax_f32(v);
  nan = (int)(wsum_u32((uint32_t)(nan != 0)) != 0u);
  if (lane_id() == 0) {
    s.red_f[wave_id()] = v;
    s.red_i[wave_id()] = nan;
  }
  __syncthreads();
  float r = s.red_f[0];
  int any = s.red_i[0];
#pragma unroll
  for (int w = 1; w < NWAVE; ++w) {
    r = fmaxf(r, s.red_f[w]);
    any |= s.red_i[w];
  }
  __syncthreads();
  return any ? __int_as_float(0x7fc00000) : r;
}

__device__ __forceinline__ int block_min_i(int v, Smem& s) {
  v = wmin_i32(v);
  if (lane_id() == 0) s.red_i[wave_id()] = v;
  __syncthreads();
  int r = s.red_i[0];
#pragma unroll
  for (int w = 1; w < NWAVE; ++w) r = min(r, s.red_i[w]);
  __syncthreads();
  return r;
}

// argmax with the lowest-index tie rule over (val, idx) pairs; NaN never enters
__device__ __forceinline__ void block_argmax(float& bv, int& bi, Smem& s) {
  const float wm = wmax_f32(bv);
  const int wi = wmin_i32(bv == wm ? bi : INT32_MAX);
  if (lane_id() == 0) {
    s.red_f[wave_id()] = wm;
    s.red_i[wave_id()] = wi;
  }
  __syncthreads();
  bv = s.red_f[0];
  bi = s.red_i[0];
#pragma unroll
  for (int w = 1; w < NWAVE; ++w) {
    const float ov = s.red_f[w];
    const int oi = s.red_i[w];
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __syncthreads();
}

// exclusive prefix over threads in thread order; returns the workgroup total in `total`
__device__ __forceinline__ int block_excl_scan_i(int v, Smem& s, int& total) {
  const uint32_t incl = wscan_u32((uint32_t)v);
  if (lane_id() == 63) s.red_i[NWAVE + wave_id()] = (int)incl;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    const int x = s.red_i[NWAVE + w];
    before += (w < wave_id()) ? x : 0;
    tot += x;
  }
  __syncthreads();
  total = tot;
  return before + (int)incl - v;
}

// ---------------------------------------------------------------------------------------
// row sources: where chunk j of the row comes from
//   RegRow<NCH>: NCH 16-byte vectors per thread loaded once into VGPRs (one HBM pass)
//   MemRow:      chunks re-read from memory on every pass (rows too large for the VGPRs)
//   ScalarRow:   like MemRow with element loads, for rows that are not 16-byte aligned or
//                whose vocab is not a multiple of the vector width
// Element (j, t, e) is logits index (j*NT + t)*EPV + e.
// ---------------------------------------------------------------------------------------
template <int DT, int NCH>
struct RegRow {
  static constexpr int EPV = DTraits<DT>::EPV;
  static constexpr bool kStore = true;
  static constexpr bool kVector = true;
  u4 r[NCH];
  const u4* row;
  int nvec;
  int vocab;
  __device__ __forceinline__ void init(const void* base, int nvec_, int vocab_) {
    row = (const u4*)base;
    nvec = nvec_;
    vocab = vocab_;
  }
  // Unconditional loads of a clamped address keep the code straight-line, so the
  // compiler waits for each chunk only when it is first used.
  __device__ __forceinline__ void load() {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int v = j * NT + (int)threadIdx.x;
      r[j] = __builtin_nontemporal_load(row + (v < nvec ? v : nvec - 1));
    }
  }
  // f(j, q, base_index, valid): q is the 16-byte vector, base_index its first element
  template <class F>
  __device__ __forceinline__ void for_each(F&& f) const {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int v = j * NT + (int)threadIdx.x;
      f(j, r[j], v * EPV, v < nvec);
    }
  }
  __device__ __forceinline__ int nchunks() const { return NCH; }
  __device__ __forceinline__ void store(int j, const u4& q) { r[j] = q; }
};

template <int DT>
struct MemRow {
  static constexpr int EPV = DTraits<DT>::EPV;
  static constexpr bool kStore = false;
  static constexpr bool kVector = true;
  const u4* row;
  int nvec;
  int vocab;
  __device__ __forceinline__ void init(const void* base, int nvec_, int vocab_) {
    row = (const u4*)base;
    nvec = nvec_;
    vocab = vocab_;
  }
  __device__ __forceinline__ void load() {}
  template <class F>
  __device__ __forceinline__ void for_each(F&& f) const {
    const int nch = (nvec + NT - 1) / NT;
    for (int j = 0; j < nch; ++j) {
      const int v = j * NT + (int)threadIdx.x;
      const u4 q = row[v < nvec ? v : nvec - 1];
      f(j, q, v * EPV, v < nvec);
    }
  }
  __device__ __forceinline__ int nchunks() const { return (nvec + NT - 1) / NT; }
  __device__ __forceinline__ void store(int, const u4&) {}
};

template <int DT>
struct ScalarRow {
  static constexpr int EPV = DTraits<DT>::EPV;
  static constexpr bool kStore = false;
  static constexpr bool kVector = false;
  const uint8_t* row;
  int nvec;  // ceil(vocab / EPV)
  int vocab;
  __device__ __forceinline__ void init(const void* base, int nvec_, int vocab_) {
    row = (const uint8_t*)base;
    nvec = nvec_;
    vocab = vocab_;
  }
  __device__ __forceinline__ void load() {}
  template <class F>
  __device__ __forceinline__ void for_each(F&& f) const {
    const int nch = (nvec + NT - 1) / NT;
    for (int j = 0; j < nch; ++j) {
      const int v = j * NT + (int)threadIdx.x;
      u4 q = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        const int i = v * EPV + e;
        if (i < vocab) {
          if constexpr (DTraits<DT>::B16) {
            const uint32_t h = ((const uint16_t*)row)[i];
            q[e >> 1] |= (e & 1) ? (h << 16) : h;
          } else {
            q[e] = ((const uint32_t*)row)[i];
          }
        }
      }
      f(j, q, v * EPV, v < nvec);
    }
  }
  __device__ __forceinline__ int nchunks() const { return (nvec + NT - 1) / NT; }
  __device__ __forceinline__ void store(int, const u4&) {}
};

template <class Src>
__device__ __forceinline__ bool elem_valid(const Src& src, bool vvalid, int idx) {
  if constexpr (Src::kVector) {
    return vvalid;
  } else {
    return idx < src.vocab;
  }
}

// ---------------------------------------------------------------------------------------
// index selection: the rank-th (0-based, ascending index) element whose raw bits satisfy
// `match`. Every thread calls it and gets the index, or -1 if there are fewer matches.
// Chunk j of the row covers indices [j*NT*EPV, (j+1)*NT*EPV); the chunk holding the answer
// is found from per-chunk counts (in s.hist) and the thread from a scan inside it.
// ---------------------------------------------------------------------------------------
template <int DT, class Src, class M>
__device__ __forceinline__ int select_index(const Src& src, Smem& s, M&& match, int rank) {
  constexpr int EPV = DTraits<DT>::EPV;
  const int nch = src.nchunks();
  for (int j = threadIdx.x; j < nch; j += NT) s.hist[j] = 0u;
  __syncthreads();
  src.for_each([&](int j, const u4& q, int base, bool vvalid) {
    int c = 0;
#pragma unroll
    for (int e = 0; e < EPV; ++e) c += (elem_valid(src, vvalid, base + e) && match(elem_raw<DT>(q, e))) ? 1 : 0;
    if (c) atomicAdd(&s.hist[j], (uint32_t)c);
  });
  __syncthreads();
  if (wave_id() == 0) {
    int run = 0, jstar = -1, rr = 0;
    for (int j0 = 0; j0 < nch; j0 += 64) {
      const int j = j0 + lane_id();
      const int c = (j < nch) ? (int)s.hist[j] : 0;
      const int incl = (int)wscan_u32((uint32_t)c);
      const uint64_t hit = ballot(run + incl > rank);
      if (hit) {
        const int L = first_lane(hit);
        jstar = j0 + L;
        rr = rank - (run + (int)bcast_u32((uint32_t)(incl - c), L));
        break;
      }
      run += (int)bcast_u32((uint32_t)incl, 63);
    }
    if (lane_id() == 0) {
      s.sel_jstar = jstar;
      s.sel_rank = rr;
      s.sel_index = -1;
    }
  }
  __syncthreads();
  const int jstar = s.sel_jstar;
  const int rr = s.sel_rank;
  if (jstar < 0) return -1;
  int c = 0;
  int my_idx[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) my_idx[e] = -1;
  src.for_each([&](int j, const u4& q, int base, bool vvalid) {
    if (j == jstar) {
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        const bool hm = elem_valid(src, vvalid, base + e) && match(elem_raw<DT>(q, e));
        my_idx[e] = hm ? base + e : -1;
        c += hm ? 1 : 0;
      }
    }
  });
  int total;
  const int ex = block_excl_scan_i(c, s, total);
  if (rr >= ex && rr < ex + c) {
    int k = rr - ex;
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      if (my_idx[e] >= 0) {
        if (k == 0) s.sel_index = my_idx[e];
        --k;
      }
    }
  }
  __syncthreads();
  const int r = s.sel_index;
  __syncthreads();
  return r;
}

// Index selection for register-resident rows. The per-(chunk, wave) match counts come
// from ballots of the per-element compares (scalar popcounts, skipped for chunks where the
// wave has no match), so the pass costs one compare per element; only the wave holding
// the answer then looks at lanes.
template <int DT, int NCH, class M>
__device__ __forceinline__ int select_index_reg(const RegRow<DT, NCH>& src, Smem& s, M&& match, int rank) {
  constexpr int EPV = DTraits<DT>::EPV;
  static_assert(NCH * NWAVE <= 256, "chunk table must fit 4 entries per lane");
  const int l = lane_id(), w = wave_id();
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const bool vv = j * NT + (int)threadIdx.x < src.nvec;
    uint64_t mk[EPV];
    uint64_t any = 0;
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      mk[e] = ballot(vv && match(elem_raw<DT>(src.r[j], e)));
      any |= mk[e];
    }
    uint32_t c = 0;
    if (any) {
#pragma unroll
      for (int e = 0; e < EPV; ++e) c += (uint32_t)__popcll(mk[e]);
    }
    if (l == 0) s.hist[j * NWAVE + w] = c;
  }
  __syncthreads();
  if (w == 0) {
    // positions p = j*NWAVE + wave, in index order; lane l holds p = 4l .. 4l+3
    uint32_t c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = (4 * l + i < NCH * NWAVE) ? s.hist[4 * l + i] : 0u;
    const uint32_t tot = c[0] + c[1] + c[2] + c[3];
    const uint32_t incl = wscan_u32(tot);
    const uint64_t hit = ballot(incl > (uint32_t)rank);
    int pos = -1, rr = 0;
    if (hit) {
      const int L = first_lane(hit);
      uint32_t run = incl - tot;
      int fi = 3, fr = 0;
      bool found = false;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (!found && run + c[i] > (uint32_t)rank) {
          fi = i;
          fr = rank - (int)run;
          found = true;
        }
        run += c[i];
      }
      pos = (int)bcast_u32((uint32_t)(4 * l + fi), L);
      rr = (int)bcast_u32((uint32_t)fr, L);
    }
    if (l == 0) {
      s.sel_jstar = pos;
      s.sel_rank = rr;
      s.sel_index = -1;
    }
  }
  __syncthreads();
  const int pos = s.sel_jstar;
  if (pos < 0) {
    __syncthreads();
    return -1;
  }
  const int jstar = pos / NWAVE, wstar = pos % NWAVE, rr = s.sel_rank;
  if (w == wstar) {
    uint32_t bits = 0;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if (j == jstar) {
        const bool vv = j * NT + (int)threadIdx.x < src.nvec;
#pragma unroll
        for (int e = 0; e < EPV; ++e) bits |= (vv && match(elem_raw<DT>(src.r[j], e))) ? (1u << e) : 0u;
      }
    }
    const uint32_t cnt = (uint32_t)__popc(bits);
    const uint32_t incl = wscan_u32(cnt);
    const uint32_t excl = incl - cnt;
    if ((uint32_t)rr >= excl && (uint32_t)rr < incl) {
      uint32_t b = bits;
      for (uint32_t k = (uint32_t)rr - excl; k > 0; --k) b &= b - 1u;
      s.sel_index = (jstar * NT + (int)threadIdx.x) * EPV + (__ffs(b) - 1);
    }
  }
  __syncthreads();
  const int r = s.sel_index;
  __syncthreads();
  return r;
}

// the only element whose raw bits satisfy `match` (the caller knows there is exactly one)
template <int DT, class Src, class M>
__device__ __forceinline__ int locate_unique(const Src& src, Smem& s, M&& match) {
  constexpr int EPV = DTraits<DT>::EPV;
  if (threadIdx.x == 0) s.sel_index = -1;
  __syncthreads();
  src.for_each([&](int, const u4& q, int base, bool vvalid) {
#pragma unroll
    for (int e = 0; e < EPV; ++e)
      if (elem_valid(src, vvalid, base + e) && match(elem_raw<DT>(q, e))) s.sel_index = base + e;
  });
  __syncthreads();
  const int r = s.sel_index;
  __syncthreads();
  return r;
}

__device__ __forceinline__ void write_info(const KArgs& a, int b, int tok, int status, const RowState& st) {
  a.out_token[b] = tok;
  a.out_status[b] = status;
  if (a.out_info) {
    pbs_row_info inf;
    inf.token = tok;
    inf.status = status;
    inf.x_max = st.m;
    inf.x_kth = st.x_kth;
    inf.x_cut = st.x_cut;
    inf.n_cut_tie = st.n_cut_tie;
    inf.n_cut_keep = st.n_cut_keep;
    inf.n_kept = st.n_kept;
    inf.z_k = st.zk;
    inf.z_p = st.zp;
    inf.target = st.target;
    a.out_info[b] = inf;
  }
}

__device__ __forceinline__ void write_error(const KArgs& a, int b, int status, float m) {
  RowState st = {};
  st.m = m;
  st.x_kth = -INFINITY;
  write_info(a, b, 0, status, st);
}

// ---------------------------------------------------------------------------------------
// 16-bit rows: searches over the LDS histogram
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t hist_count(const Smem& s, uint32_t o) {
  const uint32_t w = s.hist[o >> 1];
  return (o & 1u) ? (w >> 16) : (w & 0xffffu);
}

template <int DT>
__device__ __forceinline__ float scaled16(uint32_t o, float T) {
  return raw_to_float<DT>(raw_of_ord16(o)) / T;
}
// softmax weight of one distinct 16-bit value relative to the row maximum m, in fp64 from
// the exact fp32 scaled value (pagedbatch takes softmax of the fp32 scaled row, sampling.py:26)
template <int DT>
__device__ __forceinline__ double weight16(uint32_t o, float T, float m) {
  return exp_neg((double)scaled16<DT>(o, T) - (double)m);
}

// One group's 256 bins as seen by a wave, restricted to ords >= lo: lane l holds the bins
// at descending positions 4l..4l+3 (ords g*256+255-4l-i), their counts and masses.
template <int DT>
struct GroupScan {
  uint32_t g;
  uint32_t n[4];
  double w[4];  // mass of each bin (count * weight)
  __device__ __forceinline__ void load(const Smem& s, uint32_t g_, uint32_t lo, float T, float m, bool want_mass) {
    g = g_;
    const int l = lane_id();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t o = g * 256u + 255u - (uint32_t)(4 * l + i);
      n[i] = (o >= lo) ? hist_count(s, o) : 0u;
      w[i] = (want_mass && n[i]) ? (double)n[i] * weight16<DT>(o, T, m) : 0.0;
    }
  }
  __device__ __forceinline__ uint32_t ord(int l, int i) const { return g * 256u + 255u - (uint32_t)(4 * l + i); }
  // count / mass of the group's bins with ord >= t
  __device__ __forceinline__ uint32_t count_ge(uint32_t t) const {
    const int l = lane_id();
    uint32_t c = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) c += (ord(l, i) >= t) ? n[i] : 0u;
    return wsum_u32(c);
  }
  __device__ __forceinline__ double mass_ge(uint32_t t) const {
    const int l = lane_id();
    double c = 0.0;
#pragma unroll
    for (int i = 0; i < 4; ++i) c += (ord(l, i) >= t) ? w[i] : 0.0;
    return wsum_f64(c);
  }
  // first ord (descending) whose inclusive count from the top of the group reaches need
  __device__ __forceinline__ uint32_t find_count(uint32_t need) const {
    const int l = lane_id();
    const uint32_t tot = n[0] + n[1] + n[2] + n[3];
    const uint32_t incl = wscan_u32(tot);
    const uint64_t hit = ballot(incl >= need);
    const int L = hit ? first_lane(hit) : 63;
    uint32_t run = incl - tot;
    int found = -1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (found < 0 && run + n[i] >= need) found = i;
      run += n[i];
    }
    return bcast_u32(ord(l, found < 0 ? 3 : found), L);
  }
  // first ord (descending) whose inclusive mass, starting from `base` above the group,
  // exceeds target; the lowest non-empty ord if rounding keeps it at or below the target.
  // `above` gets the cumulative mass strictly above the returned ord.
  __device__ __forceinline__ uint32_t find_mass(double base, double target, double& above) const {
    const int l = lane_id();
    const double tot = w[0] + w[1] + w[2] + w[3];
    const double incl = wscan_f64(tot);
    double excl = __shfl_up(incl, 1);
    if (l == 0) excl = 0.0;
    uint64_t hit = ballot(base + incl > target);
    bool last = false;
    if (!hit) {
      hit = ballot(n[0] + n[1] + n[2] + n[3] > 0u);
      last = true;
    }
    const int L = last ? 63 - __clzll((unsigned long long)hit) : first_lane(hit);
    double run = base + excl;
    int found = -1;
    double ab = 0.0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool take = last ? (n[i] > 0u) : (found < 0 && run + w[i] > target);
      if (take) {
        found = i;
        ab = run;
      }
      run += w[i];
    }
    above = bcast_f64(ab, L);
    return bcast_u32(ord(l, found < 0 ? 3 : found), L);
  }
};

// Ords whose scaled value equals that of ord o. Distinct 16-bit values only meet after the
// division by T at the under/overflow ends; the map is monotone, so binary search.
template <int DT>
__device__ __forceinline__ void tie_range16(uint32_t o, float T, uint32_t& lo, uint32_t& hi) {
  const float x = scaled16<DT>(o, T);
  uint32_t a = ord16_neg_inf<DT>(), b = o;
  if (o == 0u || scaled16<DT>(o - 1u, T) < x) {
    a = o;
  } else {
    while (a < b) {
      const uint32_t mid = a + (b - a) / 2;
      if (scaled16<DT>(mid, T) >= x) b = mid; else a = mid + 1;
    }
  }
  lo = a;
  a = o;
  b = ord16_pos_inf<DT>();
  if (o >= b || scaled16<DT>(o + 1u, T) > x) {
    b = o;
  } else {
    while (a < b) {
      const uint32_t mid = a + (b - a + 1) / 2;
      if (scaled16<DT>(mid, T) <= x) a = mid; else b = mid - 1;
    }
  }
  hi = a;
}

// the group holding the need-th element (descending), over ords >= lo whose partial lowest
// group has count cnt_lo; -1 if fewer elements
__device__ __forceinline__ int find_group_count(const Smem& s, uint32_t lo, uint32_t cnt_lo, uint32_t need) {
  const int l = lane_id();
  const uint32_t glo = lo >> 8;
  int found = -1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t g = (uint32_t)(4 * l + i);
    const uint32_t ab = s.gabove_cnt[g];
    const uint32_t c = g > glo ? s.gcount[g] : (g == glo ? cnt_lo : 0u);
    if (c && ab < need && need <= ab + c) found = (int)g;
  }
  const uint64_t hit = ballot(found >= 0);
  return hit ? (int)bcast_u32((uint32_t)found, first_lane(hit)) : -1;
}

// the group whose cumulative mass interval [above, above + mass) holds target, over ords
// >= lo whose partial lowest group has mass mass_lo. Groups tile the cumulative exactly
// because each group's upper end is the next lower group's stored "above".
__device__ __forceinline__ int find_group_mass(const Smem& s, uint32_t lo, double mass_lo, double total, double target) {
  const int l = lane_id();
  const uint32_t glo = lo >> 8;
  int found = -1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t g = (uint32_t)(4 * l + i);
    if (g < glo) continue;
    const double ab = s.gabove_mass[g];
    const double end = (g == glo) ? ab + mass_lo : (g == 0 ? total : s.gabove_mass[g - 1]);
    const bool nonempty = (g == glo) ? mass_lo > 0.0 : s.gmass[g] > 0.0;
    if (nonempty && ab <= target && target < end) found = (int)g;
  }
  const uint64_t hit = ballot(found >= 0);
  return hit ? (int)bcast_u32((uint32_t)found, first_lane(hit)) : -1;
}

// count / mass of ords >= t (t inside the histogram range)
template <int DT>
__device__ __forceinline__ uint32_t count_ge(const Smem& s, uint32_t t, float T, float m) {
  GroupScan<DT> gs;
  gs.load(s, t >> 8, t, T, m, false);
  return s.gabove_cnt[t >> 8] + gs.count_ge(t);
}
template <int DT>
__device__ __forceinline__ double mass_ge(const Smem& s, uint32_t t, float T, float m) {
  GroupScan<DT> gs;
  gs.load(s, t >> 8, t, T, m, true);
  return s.gabove_mass[t >> 8] + gs.mass_ge(t);
}

// ---------------------------------------------------------------------------------------
// 16-bit stochastic row
// ---------------------------------------------------------------------------------------

// Index of the rank-th lowest-index element whose ord lies in [lo, hi]. A single ord (the
// usual case) is matched on its raw bits: both zero encodings for the +0 ord.
template <int DT, class Src>
__device__ __forceinline__ int select_tied16(const Src& src, Smem& s, uint32_t lo, uint32_t hi, int rank) {
  if (lo == hi) {
    const uint32_t r0 = raw_of_ord16(lo);
    const uint32_t r1 = (r0 == 0u) ? 0x8000u : r0;
    auto eq = [=](uint32_t raw) { return raw == r0 || raw == r1; };
    if constexpr (Src::kStore) {
      return select_index_reg(src, s, eq, rank);
    } else {
      return select_index<DT>(src, s, eq, rank);
    }
  }
  auto in = [=](uint32_t raw) {
    const uint32_t o = ord16(raw);
    return o >= lo && o <= hi;
  };
  if constexpr (Src::kStore) {
    return select_index_reg(src, s, in, rank);
  } else {
    return select_index<DT>(src, s, in, rank);
  }
}

// Top-k threshold, top-p cutoff and draw position from the histogram summaries. Runs on
// wave 0 only and leaves the result in s.st.
template <int DT>
__device__ __forceinline__ void resolve16(Smem& s, int V, float T, int kk, float p, float u, float m) {
  RowState st = {};
  st.status = PBS_ROW_OK;
  st.m = m;
  st.x_kth = -INFINITY;
  const uint32_t total_cnt = s.gabove_cnt[0] + s.gcount[0];
  const double total_mass = s.gabove_mass[0] + s.gmass[0];
  // a u16 counter wraps only if one value occurs more than 65535 times
  if (total_cnt != (uint32_t)V) {
    st.status = -1;
    if (lane_id() == 0) s.st = st;
    return;
  }

  // top-k (sampling.py:15-17): K = ords >= kord_lo
  uint32_t kord_lo = 0u;
  if (kk > 0 && kk < V) {
    const int g = find_group_count(s, 0u, s.gcount[0], (uint32_t)kk);
    GroupScan<DT> gs;
    gs.load(s, (uint32_t)g, 0u, T, m, false);
    const uint32_t o = gs.find_count((uint32_t)kk - s.gabove_cnt[g]);
    uint32_t lo, hi;
    tie_range16<DT>(o, T, lo, hi);
    kord_lo = lo;
    st.x_kth = scaled16<DT>(o, T);
  }
  st.kord_lo = kord_lo;
  const uint32_t glo = kord_lo >> 8;
  GroupScan<DT> gk;
  gk.load(s, glo, kord_lo, T, m, true);
  const uint32_t cnt_lo = gk.count_ge(kord_lo);
  const double mass_lo = gk.mass_ge(kord_lo);
  const uint32_t nk = s.gabove_cnt[glo] + cnt_lo;
  const double zk = (kord_lo == 0u) ? total_mass : s.gabove_mass[glo] + mass_lo;
  st.zk = zk;

  // top-p (sampling.py:18-25): the shortest prefix (value desc, index asc) whose
  // exclusive mass is <= p*Z; inside the cutoff tie group the lowest indices survive
  bool have_cut = false;
  double above_cut = 0.0;
  if (p < 1.0f) {
    const double tau = (double)p * zk;
    const int g = find_group_mass(s, kord_lo, mass_lo, total_mass, tau);
    if (g >= 0) {
      GroupScan<DT> gs;
      gs.load(s, (uint32_t)g, kord_lo, T, m, true);
      double ab;
      const uint32_t o = gs.find_mass(s.gabove_mass[g], tau, ab);
      uint32_t lo, hi;
      tie_range16<DT>(o, T, lo, hi);
      lo = max(lo, kord_lo);
      double B;
      uint32_t n_above, n_ge;
      if (lo == o && hi == o) {
        B = ab;
        n_ge = s.gabove_cnt[g] + gs.count_ge(o);
        n_above = n_ge - hist_count(s, o);
      } else {
        B = mass_ge<DT>(s, hi + 1u, T, m);
        n_above = count_ge<DT>(s, hi + 1u, T, m);
        n_ge = count_ge<DT>(s, lo, T, m);
      }
      st.cut_lo = lo;
      st.cut_hi = hi;
      st.n_cut_tie = (int)(n_ge - n_above);
      const double w = weight16<DT>(o, T, m);
      double kf = (w > 0.0) ? floor((tau - B) / w) + 1.0 : (double)st.n_cut_tie;
      kf = fmax(1.0, fmin(kf, (double)st.n_cut_tie));
      st.n_cut_keep = (int)kf;
      st.zp = B + (double)st.n_cut_keep * w;
      st.n_kept = (int)n_above + st.n_cut_keep;
      st.x_cut = scaled16<DT>(o, T);
      above_cut = B;
      have_cut = true;
    }
  }
  if (!have_cut) {
    // no top-p, or p*Z reaches the whole top-k set: all of K is kept, and K's lowest value
    // is the cutoff tie group
    const int g = find_group_count(s, kord_lo, cnt_lo, nk);
    GroupScan<DT> gs;
    gs.load(s, (uint32_t)g, kord_lo, T, m, false);
    const uint32_t o = gs.find_count(nk - s.gabove_cnt[g]);
    uint32_t lo, hi;
    tie_range16<DT>(o, T, lo, hi);
    lo = max(lo, kord_lo);
    st.cut_lo = lo;
    st.cut_hi = hi;
    st.n_cut_tie = (lo == o && hi == o) ? (int)hist_count(s, o) : (int)(nk - count_ge<DT>(s, hi + 1u, T, m));
    st.n_cut_keep = st.n_cut_tie;
    st.zp = zk;
    st.n_kept = (int)nk;
    st.x_cut = scaled16<DT>(o, T);
    above_cut = (lo == o && hi == o) ? zk - (double)st.n_cut_tie * weight16<DT>(o, T, m) : mass_ge<DT>(s, hi + 1u, T, m);
  }

  // draw (sampling.py:26-27, inverse-CDF form): the first kept element whose cumulative
  // mass exceeds u * Z_P
  const double t = (double)u * st.zp;
  st.target = t;
  bool in_cut = true;
  if (t < above_cut) {
    const uint32_t plo = st.cut_hi + 1u;
    GroupScan<DT> gp;
    gp.load(s, plo >> 8, plo, T, m, true);
    const double mass_plo = gp.mass_ge(plo);
    const int g = find_group_mass(s, plo, mass_plo, total_mass, t);
    if (g >= 0) {
      GroupScan<DT> gs;
      gs.load(s, (uint32_t)g, plo, T, m, true);
      double ab;
      const uint32_t o = gs.find_mass(s.gabove_mass[g], t, ab);
      uint32_t lo, hi;
      tie_range16<DT>(o, T, lo, hi);
      lo = max(lo, plo);
      double B;
      int n;
      if (lo == o && hi == o) {
        B = ab;
        n = (int)hist_count(s, o);
      } else {
        B = mass_ge<DT>(s, hi + 1u, T, m);
        n = (int)(count_ge<DT>(s, lo, T, m) - count_ge<DT>(s, hi + 1u, T, m));
      }
      const double w = weight16<DT>(o, T, m);
      const double rf = (w > 0.0) ? floor((t - B) / w) : 0.0;
      st.sel_lo = lo;
      st.sel_hi = hi;
      st.sel_n = n;
      st.sel_rank = (int)fmax(0.0, fmin(rf, (double)(n - 1)));
      in_cut = false;
    }
  }
  if (in_cut) {
    const double w = weight16<DT>(st.cut_hi, T, m);
    const double rf = (w > 0.0) ? floor((t - above_cut) / w) : 0.0;
    st.sel_lo = st.cut_lo;
    st.sel_hi = st.cut_hi;
    st.sel_n = st.n_cut_keep;
    st.sel_rank = (int)fmax(0.0, fmin(rf, (double)(st.n_cut_keep - 1)));
  }
  if (lane_id() == 0) s.st = st;
}

template <int DT, class Src>
__device__ __forceinline__ void sample_row16(const KArgs& a, Smem& s, Src& src, int b, float T, int kk, float p, float u) {
  constexpr int EPV = DTraits<DT>::EPV;
  const int V = a.vocab;

  // stream: histogram of ords, row max, NaN flag. The histogram is cleared while the
  // row's loads are in flight; the barrier orders LDS only.
  {
    u4* h4 = (u4*)s.hist;
    for (int i = threadIdx.x; i < HIST_WORDS / 4; i += NT) h4[i] = (u4){0u, 0u, 0u, 0u};
  }
  lds_barrier();
  // packed u16 extremes of the ords: the maximum gives the row max, and NaNs (ords above
  // +inf or below -inf) show up in either extreme
  uint32_t pmax = 0u, pmin = 0xffffffffu;
  src.for_each([&](int, const u4& q, int base, bool vvalid) {
    if constexpr (Src::kVector) {
      if (vvalid) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t op = ord16_pair(q[d]);
          pmax = pk_max_u16(pmax, op);
          pmin = pk_min_u16(pmin, op);
          __hip_atomic_fetch_add(&s.hist[(op >> 1) & 0x7fffu], 1u + (op & 1u) * 0xffffu, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_WORKGROUP);
          __hip_atomic_fetch_add(&s.hist[op >> 17], 1u + ((op >> 16) & 1u) * 0xffffu, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_WORKGROUP);
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        if (elem_valid(src, vvalid, base + e)) {
          const uint32_t o = ord16_pair(elem_raw<DT>(q, e)) & 0xffffu;
          pmax = max(pmax, o);
          pmin = min(pmin, 0xffff0000u | o);
          __hip_atomic_fetch_add(&s.hist[o >> 1], 1u + (o & 1u) * 0xffffu, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_WORKGROUP);
        }
      }
    }
  });
  uint32_t omax = max(pmax & 0xffffu, pmax >> 16), omin = min(pmin & 0xffffu, pmin >> 16);
  omax = wmax_u32(omax);
  omin = wmin_u32(omin);
  if (lane_id() == 0) {
    s.red_i[wave_id()] = (int)omax;
    s.red_i[NWAVE + wave_id()] = (int)omin;
  }
  __syncthreads();
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    omax = max(omax, (uint32_t)s.red_i[w]);
    omin = min(omin, (uint32_t)s.red_i[NWAVE + w]);
  }
  const bool nan = omax > ord16_pos_inf<DT>() || omin < ord16_neg_inf<DT>();
  const float m = raw_to_float<DT>(raw_of_ord16(omax)) / T;
  if (nan || !(m > -INFINITY && m < INFINITY)) {
    if (threadIdx.x == 0) write_error(a, b, nan ? PBS_ROW_NAN : PBS_ROW_NONFINITE, nan ? NAN : m);
    return;
  }
  // -0 was counted under ord 0x7fff (high half of word 0x3fff); merge it into +0 (0x8000,
  // low half of word 0x4000), so the two zeros form one tie group
  if (threadIdx.x == 0) {
    const uint32_t nz = s.hist[0x3fff] >> 16;
    if (nz) {
      s.hist[0x3fff] -= nz << 16;
      s.hist[0x4000] += nz;
    }
  }
  __syncthreads();

  // group summaries, all waves: wave w owns groups w, w+16, ...; empty groups are skipped
  for (int g = wave_id(); g < NGROUP; g += NWAVE) {
    const int l = lane_id();
    const uint32_t w0 = s.hist[g * 128 + 2 * l], w1 = s.hist[g * 128 + 2 * l + 1];
    uint32_t cnt = 0;
    double ms = 0.0;
    if (ballot((w0 | w1) != 0u)) {
      const uint32_t n[4] = {w0 & 0xffffu, w0 >> 16, w1 & 0xffffu, w1 >> 16};
      double part = 0.0;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n[i]) part += (double)n[i] * weight16<DT>((uint32_t)(g * 256 + 4 * l + i), T, m);
      cnt = wsum_u32(n[0] + n[1] + n[2] + n[3]);
      ms = wsum_f64(part);
    }
    if (l == 0) {
      s.gcount[g] = cnt;
      s.gmass[g] = ms;
    }
  }
  __syncthreads();
  if (wave_id() == 0) {
    // top-down exclusive prefixes: lane l holds groups 255-4l .. 252-4l
    const int l = lane_id();
    uint32_t c[4];
    double w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c[i] = s.gcount[255 - 4 * l - i];
      w[i] = s.gmass[255 - 4 * l - i];
    }
    const uint32_t ct = c[0] + c[1] + c[2] + c[3];
    const double wt = ((w[0] + w[1]) + w[2]) + w[3];
    const uint32_t ci = wscan_u32(ct);
    const double wi = wscan_f64(wt);
    double we = __shfl_up(wi, 1);
    if (l == 0) we = 0.0;
    uint32_t rc = ci - ct;
    double rw = we;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s.gabove_cnt[255 - 4 * l - i] = rc;
      s.gabove_mass[255 - 4 * l - i] = rw;
      rc += c[i];
      rw += w[i];
    }
  }
  __syncthreads();
  if (wave_id() == 0) resolve16<DT>(s, V, T, kk, p, u, m);
  __syncthreads();
  const RowState st = s.st;
  __syncthreads();
  if (st.status != PBS_ROW_OK) {
    if (threadIdx.x == 0) write_error(a, b, PBS_ROW_NONFINITE, m);
    return;
  }

  // which of the tied tokens: the sel_rank-th lowest index with ord in [sel_lo, sel_hi]
  const int tok = select_tied16<DT>(src, s, st.sel_lo, st.sel_hi, st.sel_rank);
  if (threadIdx.x == 0) write_info(a, b, tok < 0 ? 0 : tok, PBS_ROW_OK, st);
}

// ---------------------------------------------------------------------------------------
// fp32 stochastic row: exact bisection on 32-bit ords of the scaled values.
// Every probe is one pass over the row with fp64 accumulation in a fixed order, so the
// result is deterministic. Register-resident rows keep x = v/T in place after the first
// pass; rows streamed from memory redo the (exact) division on every pass.
// ---------------------------------------------------------------------------------------

// exp(x - m) for fp32 x <= m: the difference and the scaling by log2(e) in fp64, the
// fractional power of two on the hardware exp2 (|f| <= 1/2), the integer part exact.
__device__ __forceinline__ float weight32(float x, float m) {
  if (!(x > -INFINITY)) return 0.0f;
  double t = ((double)x - (double)m) * 1.4426950408889634074;
  t = fmax(t, -400.0);
  const double n = rint(t);
  const float f = (float)(t - n);
  return ldexpf(__builtin_amdgcn_exp2f(f), (int)n);
}

template <class Src>
__device__ __forceinline__ float x_of(const Divider& dv, uint32_t raw) {
  if constexpr (Src::kStore) {
    return __uint_as_float(raw);
  } else {
    return dv(__uint_as_float(raw));
  }
}

// count and mass (relative to m) of elements with ord32(x) >= t
template <class Src>
__device__ __forceinline__ void f32_ge(const Src& src, Smem& s, const Divider& dv, uint32_t t, float m, bool want_mass,
                       uint32_t& cnt, double& mass) {
  uint32_t c = 0;
  double ms = 0.0;
  src.for_each([&](int, const u4& q, int base, bool vvalid) {
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (elem_valid(src, vvalid, base + e)) {
        const float x = x_of<Src>(dv, q[e]);
        if (ord32(x) >= t) {
          ++c;
          if (want_mass) part += weight32(x, m);
        }
      }
    }
    ms += (double)part;
  });
  c = wsum_u32(c);
  ms = wsum_f64(ms);
  if (lane_id() == 0) {
    s.red_i[wave_id()] = (int)c;
    s.red_d[wave_id()] = ms;
  }
  __syncthreads();
  uint32_t ct = 0;
  double mt = 0.0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    ct += (uint32_t)s.red_i[w];
    mt += s.red_d[w];
  }
  __syncthreads();
  cnt = ct;
  mass = mt;
}

// largest o in [lo, hi] with count(ord >= o) >= need; count(ord >= lo) >= need is given
template <class Src>
__device__ __forceinline__ uint32_t f32_bisect_count(const Src& src, Smem& s, const Divider& dv, uint32_t lo, uint32_t hi,
                                     uint32_t need) {
  while (lo < hi) {
    const uint32_t mid = lo + (uint32_t)(((uint64_t)hi - lo + 1) / 2);
    uint32_t c;
    double ms;
    f32_ge(src, s, dv, mid, 0.0f, false, c, ms);
    if (c >= need) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// largest o in [lo, hi] with mass(ord >= o) > target; mass(ord >= lo) > target is given
template <class Src>
__device__ __forceinline__ uint32_t f32_bisect_mass(const Src& src, Smem& s, const Divider& dv, uint32_t lo, uint32_t hi,
                                    double target, float m) {
  while (lo < hi) {
    const uint32_t mid = lo + (uint32_t)(((uint64_t)hi - lo + 1) / 2);
    uint32_t c;
    double ms;
    f32_ge(src, s, dv, mid, m, true, c, ms);
    if (ms > target) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// The first pass reads `src0` (registers when resident); the bisection passes re-stream
// the row from memory (`src`), so no register copy of the row stays live across them.
template <class Src0, class Src>
__device__ __forceinline__ void sample_row32(const KArgs& a, Smem& s, const Src0& src0, const Src& src, int b,
                                             float T, int kk, float p, float u) {
  const int V = a.vocab;
  Divider dv;
  dv.init(T);
  // stream: max of x = v/T, NaN flag
  float xmax = -INFINITY;
  int nan = 0;
  src0.for_each([&](int, const u4& q, int base, bool vvalid) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x = dv(__uint_as_float(q[e]));
      if (elem_valid(src0, vvalid, base + e)) {
        xmax = fmaxf(xmax, x);
        nan |= (x != x) ? 1 : 0;
      }
    }
  });
  const float m = block_max_nan(xmax, nan, s);
  if (m != m || !(m > -INFINITY && m < INFINITY)) {
    if (threadIdx.x == 0) write_error(a, b, m != m ? PBS_ROW_NAN : PBS_ROW_NONFINITE, m);
    return;
  }
  const uint32_t ord_lo = ord32(-INFINITY);
  const uint32_t ord_m = ord32(m);
  RowState st = {};
  st.m = m;
  st.x_kth = -INFINITY;
  uint32_t c;
  double ms;

  // top-k: kord = k-th largest ord
  uint32_t kord = ord_lo;
  if (kk > 0 && kk < V) {
    kord = f32_bisect_count(src, s, dv, ord_lo, ord_m, (uint32_t)kk);
    st.x_kth = float_of_ord32(kord);
  }
  st.kord_lo = kord;
  f32_ge(src, s, dv, kord, m, true, c, ms);
  const double zk = ms;
  const uint32_t nk = c;
  st.zk = zk;

  // top-p cutoff: the ord where the descending cumulative mass first exceeds p*Z
  uint32_t cut;
  double above_cut;
  if (p < 1.0f && zk * (double)p < zk) {
    const double tau = (double)p * zk;
    cut = f32_bisect_mass(src, s, dv, kord, ord_m, tau, m);
    uint32_t n_above, n_ge;
    f32_ge(src, s, dv, cut + 1u, m, true, n_above, above_cut);
    f32_ge(src, s, dv, cut, m, false, n_ge, ms);
    st.n_cut_tie = (int)(n_ge - n_above);
    const double w = (double)weight32(float_of_ord32(cut), m);
    double kf = (w > 0.0) ? floor((tau - above_cut) / w) + 1.0 : (double)st.n_cut_tie;
    kf = fmax(1.0, fmin(kf, (double)st.n_cut_tie));
    st.n_cut_keep = (int)kf;
    st.zp = above_cut + (double)st.n_cut_keep * w;
    st.n_kept = (int)n_above + st.n_cut_keep;
  } else {
    // keep all of K: the cutoff group is K's lowest value
    cut = f32_bisect_count(src, s, dv, kord, ord_m, nk);
    uint32_t n_above;
    f32_ge(src, s, dv, cut + 1u, m, true, n_above, above_cut);
    st.n_cut_tie = (int)(nk - n_above);
    st.n_cut_keep = st.n_cut_tie;
    st.zp = zk;
    st.n_kept = (int)nk;
  }
  st.cut_lo = cut;
  st.cut_hi = cut;
  st.x_cut = float_of_ord32(cut);

  // draw
  const double t = (double)u * st.zp;
  st.target = t;
  uint32_t sel = cut;
  int rank;
  if (t < above_cut) {
    sel = f32_bisect_mass(src, s, dv, cut + 1u, ord_m, t, m);
    double B;
    uint32_t n_above, n_ge;
    f32_ge(src, s, dv, sel + 1u, m, true, n_above, B);
    f32_ge(src, s, dv, sel, m, false, n_ge, ms);
    const double w = (double)weight32(float_of_ord32(sel), m);
    const double rf = (w > 0.0) ? floor((t - B) / w) : 0.0;
    rank = (int)fmax(0.0, fmin(rf, (double)((int)(n_ge - n_above) - 1)));
  } else {
    const double w = (double)weight32(float_of_ord32(cut), m);
    const double rf = (w > 0.0) ? floor((t - above_cut) / w) : 0.0;
    rank = (int)fmax(0.0, fmin(rf, (double)(st.n_cut_keep - 1)));
  }
  const int tok = select_index<PBS_DTYPE_F32>(src, s, [&](uint32_t raw) {
    return ord32(x_of<Src>(dv, raw)) == sel;
  }, rank);

  if (threadIdx.x == 0) write_info(a, b, tok < 0 ? 0 : tok, PBS_ROW_OK, st);
}

// ---------------------------------------------------------------------------------------
// one row
// ---------------------------------------------------------------------------------------
template <int DT, class Src>
__device__ __forceinline__ void sample_row(const KArgs& a, Smem& s, Src& src, int b) {
  constexpr int EPV = DTraits<DT>::EPV;
  constexpr bool B16 = DTraits<DT>::B16;
  const int64_t lrow = a.row_map ? (int64_t)a.row_map[b] : (int64_t)b;
  const float T = a.temperature[b];
  const int kk = a.top_k[b];
  const float p = a.top_p[b];
  const bool greedy = (T == 0.0f);
  const float u = greedy ? 0.0f : a.uniform[b];
  const bool bad = !(lrow >= 0 && lrow < a.n_logit_rows) || !(T >= 0.0f) || !(T <= 3.4028235e38f) ||
                   !(p > 0.0f && p <= 1.0f) || kk < 0 || (!greedy && !(u >= 0.0f && u < 1.0f));
  if (bad) {
    if (threadIdx.x == 0) write_error(a, b, PBS_ROW_BAD_PARAM, NAN);
    return;
  }
  const size_t elt = B16 ? 2 : 4;
  src.init((const uint8_t*)a.logits + (size_t)lrow * (size_t)a.row_stride * elt, a.nvec, a.vocab);
  src.load();

  if (greedy) {
    // torch.argmax (sampling.py:13): first NaN if any, else the first maximum
    float bv = -INFINITY;
    int bi = INT32_MAX;
    int nan_i = INT32_MAX;
    src.for_each([&](int, const u4& q, int base, bool vvalid) {
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        const float v = raw_to_float<DT>(elem_raw<DT>(q, e));
        const int idx = base + e;
        if (elem_valid(src, vvalid, idx)) {
          // elements arrive in increasing index order per thread: strict > keeps the first
          if (v > bv || (bi == INT32_MAX && v == v)) {
            bv = v;
            bi = idx;
          }
          nan_i = (v != v) ? min(nan_i, idx) : nan_i;
        }
      }
    });
    nan_i = block_min_i(nan_i, s);
    block_argmax(bv, bi, s);
    if (threadIdx.x == 0) {
      RowState st = {};
      st.m = bv;
      st.x_kth = -INFINITY;
      st.x_cut = bv;
      const int tok = (nan_i != INT32_MAX) ? nan_i : (bi == INT32_MAX ? 0 : bi);
      write_info(a, b, tok, PBS_ROW_OK, st);
    }
    return;
  }
  if constexpr (B16) {
    sample_row16<DT>(a, s, src, b, T, kk, p, u);
  } else if constexpr (Src::kVector) {
    MemRow<DT> mem;
    mem.init((const uint8_t*)a.logits + (size_t)lrow * (size_t)a.row_stride * elt, a.nvec, a.vocab);
    sample_row32(a, s, src, mem, b, T, kk, p, u);
  } else {
    sample_row32(a, s, src, src, b, T, kk, p, u);
  }
}

// ---------------------------------------------------------------------------------------
// diagnostics (pbs_sample_debug): final probabilities and kept mask of each row, rebuilt
// from the row's pbs_row_info. The kept set is {x >= x_kth} intersected with
// {x > x_cut} plus the n_cut_keep lowest-index elements with x == x_cut. Greedy rows get
// probability 1 on their token. Runs after k_sample on the same stream.
// ---------------------------------------------------------------------------------------
template <int DT, class Src>
__device__ __forceinline__ void debug_row(const KArgs& a, Smem& s, Src& src, int b) {
  constexpr int EPV = DTraits<DT>::EPV;
  constexpr bool B16 = DTraits<DT>::B16;
  const int V = a.vocab;
  const pbs_row_info inf = a.out_info[b];
  const int64_t obase = (int64_t)b * V;
  const float T = a.temperature[b];
  const int64_t lrow = a.row_map ? (int64_t)a.row_map[b] : (int64_t)b;
  if (inf.status != PBS_ROW_OK || T == 0.0f) {
    for (int i = threadIdx.x; i < V; i += NT) {
      const bool hit = inf.status == PBS_ROW_OK && i == inf.token;
      if (a.out_probs) a.out_probs[obase + i] = hit ? 1.0f : 0.0f;
      if (a.out_kept) a.out_kept[obase + i] = hit ? 1 : 0;
    }
    return;
  }
  src.init((const uint8_t*)a.logits + (size_t)lrow * (size_t)a.row_stride * (B16 ? 2 : 4), a.nvec, V);
  Divider dv;
  dv.init(T);
  const float xk = inf.x_kth, xc = inf.x_cut, m = inf.x_max;
  const double zp = inf.z_p;
  const int cut_index = inf.n_cut_keep > 0 ? select_index<DT>(src, s, [&](uint32_t raw) {
    const float x = dv(raw_to_float<DT>(raw));
    return x == xc && x >= xk;
  }, inf.n_cut_keep - 1) : -1;
  src.for_each([&](int, const u4& q, int base, bool vvalid) {
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      const int idx = base + e;
      if (elem_valid(src, vvalid, idx)) {
        const float x = dv(raw_to_float<DT>(elem_raw<DT>(q, e)));
        const bool kept = x >= xk && (x > xc || (x == xc && idx <= cut_index));
        if (a.out_probs) a.out_probs[obase + idx] = kept ? (float)(exp_neg((double)x - (double)m) / zp) : 0.0f;
        if (a.out_kept) a.out_kept[obase + idx] = kept ? 1 : 0;
      }
    }
  });
}

template <int DT, bool VEC>
__global__ __launch_bounds__(NT) void k_debug(KArgs a) {
  __shared__ Smem s;
  if constexpr (VEC) {
    MemRow<DT> src;
    debug_row<DT>(a, s, src, blockIdx.x);
  } else {
    ScalarRow<DT> src;
    debug_row<DT>(a, s, src, blockIdx.x);
  }
}

// NCH > 0: rows held in NCH VGPR vectors per thread; 0: re-streamed 16-byte vectors;
// -1: element loads (unaligned rows or vocab not a multiple of the vector width)
template <int DT, int NCH>
__global__ __launch_bounds__(NT) void k_sample(KArgs a) {
  __shared__ Smem s;
  const int b = blockIdx.x;
  if constexpr (NCH > 0) {
    RegRow<DT, NCH> src;
    sample_row<DT>(a, s, src, b);
  } else if constexpr (NCH == 0) {
    MemRow<DT> src;
    sample_row<DT>(a, s, src, b);
  } else {
    ScalarRow<DT> src;
    sample_row<DT>(a, s, src, b);
  }
}

}  // namespace pbs

// =========================================================================================
// C ABI
// =========================================================================================
namespace {

thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

template <int DT>
int launch_dt(const pbs::KArgs& a, int64_t rows, bool vec, hipStream_t stream) {
  using namespace pbs;
  const dim3 grid((unsigned)rows), block(NT);
  if (!vec) {
    hipLaunchKernelGGL((k_sample<DT, -1>), grid, block, 0, stream, a);
  } else {
    const int nch = (a.nvec + NT - 1) / NT;
    if (nch <= 1) hipLaunchKernelGGL((k_sample<DT, 1>), grid, block, 0, stream, a);
    else if (nch <= 2) hipLaunchKernelGGL((k_sample<DT, 2>), grid, block, 0, stream, a);
    else if (nch <= 4) hipLaunchKernelGGL((k_sample<DT, 4>), grid, block, 0, stream, a);
    else if (nch <= 8) hipLaunchKernelGGL((k_sample<DT, 8>), grid, block, 0, stream, a);
    else if (nch <= 12) hipLaunchKernelGGL((k_sample<DT, 12>), grid, block, 0, stream, a);
    else if (nch <= 16) hipLaunchKernelGGL((k_sample<DT, 16>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((k_sample<DT, 0>), grid, block, 0, stream, a);
  }
  if (a.out_probs || a.out_kept) {
    if (vec) hipLaunchKernelGGL((k_debug<DT, true>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((k_debug<DT, false>), grid, block, 0, stream, a);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PBS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  return PBS_OK;
}

int sample_impl(const void* logits, int dtype, int64_t n_logit_rows, int64_t rows, int64_t vocab,
                int64_t row_stride, const int32_t* row_map, const float* temperature, const int32_t* top_k,
                const float* top_p, const float* uniform, int32_t* out_token, int32_t* out_status,
                float* out_probs, uint8_t* out_kept, pbs_row_info* out_info, void* stream) {
  g_last_error[0] = '\0';
  if (dtype != PBS_DTYPE_F32 && dtype != PBS_DTYPE_F16 && dtype != PBS_DTYPE_BF16)
    return fail(PBS_ERR_UNSUPPORTED_DTYPE, "unsupported dtype code %d", dtype);
  if (rows < 0 || n_logit_rows < 0) return fail(PBS_ERR_INVALID_ARGUMENT, "negative row count");
  if (rows == 0) return PBS_OK;
  if (vocab < 1 || vocab > (int64_t(1) << 27))
    return fail(PBS_ERR_INVALID_ARGUMENT, "vocab %lld outside [1, 2^27]", (long long)vocab);
  if (rows > INT32_MAX) return fail(PBS_ERR_INVALID_ARGUMENT, "too many rows");
  if (row_stride < vocab)
    return fail(PBS_ERR_INVALID_ARGUMENT, "row_stride %lld < vocab %lld", (long long)row_stride, (long long)vocab);
  if (!logits || !temperature || !top_k || !top_p || !uniform || !out_token || !out_status)
    return fail(PBS_ERR_INVALID_ARGUMENT, "null pointer argument");
  if ((out_probs || out_kept) && !out_info)
    return fail(PBS_ERR_INVALID_ARGUMENT, "out_probs / out_kept need out_info");
  if (!row_map && n_logit_rows < rows)
    return fail(PBS_ERR_INVALID_ARGUMENT, "rows %lld > n_logit_rows %lld without row_map", (long long)rows,
                (long long)n_logit_rows);
  const int elt = dtype == PBS_DTYPE_F32 ? 4 : 2;
  const int epv = 16 / elt;
  const bool vec = ((uintptr_t)logits % 16 == 0) && ((row_stride * elt) % 16 == 0) && (vocab % epv == 0);
  pbs::KArgs a;
  a.logits = logits;
  a.n_logit_rows = n_logit_rows;
  a.row_stride = row_stride;
  a.vocab = (int)vocab;
  a.nvec = (int)((vocab + epv - 1) / epv);
  a.row_map = row_map;
  a.temperature = temperature;
  a.top_k = top_k;
  a.top_p = top_p;
  a.uniform = uniform;
  a.out_token = out_token;
  a.out_status = out_status;
  a.out_probs = out_probs;
  a.out_kept = out_kept;
  a.out_info = out_info;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case PBS_DTYPE_F32: return launch_dt<PBS_DTYPE_F32>(a, rows, vec, st);
    case PBS_DTYPE_F16: return launch_dt<PBS_DTYPE_F16>(a, rows, vec, st);
    default: return launch_dt<PBS_DTYPE_BF16>(a, rows, vec, st);
  }
}

}  // namespace

extern "C" {

int pbs_abi_version(void) { return PBS_ABI_VERSION; }

const char* pbs_last_error(void) { return g_last_error; }

size_t pbs_workspace_bytes(int64_t rows, int64_t vocab, int dtype) {
  (void)rows;
  (void)vocab;
  (void)dtype;
  return 0;
}

int pbs_sample(const void* logits, int dtype, int64_t n_logit_rows, int64_t rows, int64_t vocab,
               int64_t row_stride, const int32_t* row_map, const float* temperature, const int32_t* top_k,
               const float* top_p, const float* uniform, int32_t* out_token, int32_t* out_status,
               void* workspace, size_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  return sample_impl(logits, dtype, n_logit_rows, rows, vocab, row_stride, row_map, temperature, top_k, top_p,
                     uniform, out_token, out_status, nullptr, nullptr, nullptr, stream);
}

int pbs_sample_debug(const void* logits, int dtype, int64_t n_logit_rows, int64_t rows, int64_t vocab,
                     int64_t row_stride, const int32_t* row_map, const float* temperature,
                     const int32_t* top_k, const float* top_p, const float* uniform, int32_t* out_token,
                     int32_t* out_status, float* out_probs, uint8_t* out_kept, pbs_row_info* out_info,
                     void* workspace, size_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  return sample_impl(logits, dtype, n_logit_rows, rows, vocab, row_stride, row_map, temperature, top_k, top_p,
                     uniform, out_token, out_status, out_probs, out_kept, out_info, stream);
}

}  // extern "C"
