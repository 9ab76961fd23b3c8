// pbsample.hip -- gfx950 (MI355X) token sampler: greedy / temperature / top-k / top-p / draw.
//
// Replaces the per-row torch op chain of pagedbatch/sampling.py:10-27 (called once per
// row from pagedbatch/engine.py:133-139) with one launch per engine step: one 512-thread
// workgroup (8 waves) per output row, the row held in VGPRs after a single coalesced
// 16-byte-load pass over HBM (or re-streamed from memory when it does not fit), per-row
// selection state in LDS. Steps whose rows are all greedy take pbs_argmax's kernel
// (k_argmax) instead: no histogram, so several small workgroups share a CU.
//
// Selection works on order-preserving integer keys ("ords") of the values:
//   16-bit logits (bf16 / fp16): every distinct value has its own ord, so a 64K-bin
//     count histogram in LDS (packed u16 counters) is an exact summary of the row. The
//     softmax weight exp(x - max) depends only on the value, so the mass of a value is
//     count * weight, computed once per distinct value in fp64. Top-k threshold, top-p
//     cutoff and the inverse-CDF draw are prefix searches over that histogram in
//     descending value order; only "which of the tied tokens" looks at indices again.
//   fp32 logits: a histogram of the top 16 bits of each x = fp32(v)/T (exact division)
//     bounds every cumulative mass; one more pass gathers the elements of the few bins
//     the searches land in and sums the exact mass above them; the searches finish in
//     that list. Rows the list cannot hold fall back to bisection on 32-bit ords with
//     exact fp64 mass sums.
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

// Translation units. The library is built from several compilations of this file so that
// they run in parallel: PBS_TU_DTYPE=n compiles the kernels of one logits type and
// launch_dt<n>; PBS_TU_ABI compiles the C ABI and the finish kernel. Without either macro
// the file is the whole library in one unit.
#if defined(PBS_TU_DTYPE)
#define PBS_WANT_KERNELS 1
#define PBS_WANT_ABI 0
#elif defined(PBS_TU_ABI)
#define PBS_WANT_KERNELS 0
#define PBS_WANT_ABI 1
#else
#define PBS_WANT_KERNELS 1
#define PBS_WANT_ABI 1
#endif

namespace pbs {

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

// one launch of the sampler for logits type DT (defined with the kernels)
template <int DT>
int launch_dt(const KArgs& a, int64_t rows, bool vec, hipStream_t stream);
// one launch of the all-greedy kernel (argmax of every row) for logits type DT
template <int DT>
int launch_argmax(const KArgs& a, int64_t rows, bool vec, hipStream_t stream);

// error reporting shared by the translation units (pbs_last_error reads it)
int report_error(int code, const char* msg);
int report_errorf(int code, const char* fmt, ...);

}  // namespace pbs

#if PBS_WANT_KERNELS
namespace pbs {

constexpr int NT = 512;            // threads per workgroup: one workgroup per row
constexpr int NWAVE = NT / 64;     // wave64
constexpr int HIST_WORDS = 32768;  // 64K packed u16 counters = 128 KB of LDS
constexpr int NGROUP = 256;        // histogram groups of 256 ords (high byte of a 16-bit ord)
constexpr int PIPE = 4;            // 16-byte loads per thread in flight while a row streams in
constexpr int NBUCKET = 256;       // fp32 rows: buckets per level of a list search

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

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
constexpr int ROW_ROR8 = 0x128, ROW_HALF_MIRROR = 0x141, QUAD_XOR1 = 0xb1, QUAD_XOR2 = 0x4e;

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
// a value the program knows to be the same in every lane (an LDS word all lanes read, for
// example), made visibly wave-uniform: branches on it become scalar branches
__device__ __forceinline__ uint32_t uni_u32(uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); }
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
// all rows written, lanes without a source lane read 0 (bound_ctrl): no zeroed old value
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_z(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, true);
}
template <int CTRL, int RM = 0xf>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  uint32_t lo, hi;
  if constexpr (RM == 0xf) {
    lo = dpp_z<CTRL>((uint32_t)b);
    hi = dpp_z<CTRL>((uint32_t)(b >> 32));
  } else {
    lo = dpp<CTRL, RM>((uint32_t)b, 0u);
    hi = dpp<CTRL, RM>((uint32_t)(b >> 32), 0u);
  }
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
__device__ __forceinline__ float wscan_f32(float v) {
  v += __uint_as_float(dpp<ROW_SHR1>(__float_as_uint(v), 0u));
  v += __uint_as_float(dpp<ROW_SHR2>(__float_as_uint(v), 0u));
  v += __uint_as_float(dpp<ROW_SHR4>(__float_as_uint(v), 0u));
  v += __uint_as_float(dpp<ROW_SHR8>(__float_as_uint(v), 0u));
  v += __uint_as_float(dpp<ROW_BCAST15, 0xa>(__float_as_uint(v), 0u));
  v += __uint_as_float(dpp<ROW_BCAST31, 0xc>(__float_as_uint(v), 0u));
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

// exp(x - m) for fp32 x <= m, in fp32 on the hardware exp2: exp2(RN(RN(x - m) * log2 e)).
// The roundings of the difference and the product perturb the exponent by at most
// 2^-23 |x - m|, so the error relative to the largest weight (1, at x = m) stays below
// max(e^-d * d) * 2^-23 ~ 5e-8 plus the exp2 error of about one ulp: far inside the
// tolerances on probabilities (1e-5) and on CDF boundaries (1e-6 of the total mass).
// Deterministic; returned in fp64 for the sums.
__device__ __forceinline__ double weight_f(float x, float m) {
  if (!(x > -INFINITY)) return 0.0;
  return (double)__builtin_amdgcn_exp2f((x - m) * 1.44269504088896341f);
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

// the largest element of one 16-byte vector (NaN ignored); nan |= the vector holds a NaN
template <int DT>
__device__ __forceinline__ float vec_max(const u4& q, bool& nan) {
  constexpr int EPV = DTraits<DT>::EPV;
  float e[EPV];
#pragma unroll
  for (int i = 0; i < EPV; ++i) e[i] = raw_to_float<DT>(elem_raw<DT>(q, i));
  bool n = false;
#pragma unroll
  for (int i = 0; i < EPV; i += 2) n |= __builtin_isunordered(e[i], e[i + 1]);
  nan |= n;
#pragma unroll
  for (int w = 1; w < EPV; w *= 2) {
#pragma unroll
    for (int i = 0; i + w < EPV; i += 2 * w) e[i] = fmaxf(e[i], e[i + w]);
  }
  return e[0];
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
// acc + low half + high half of w (one v_dot2_u32_u16)
__device__ __forceinline__ uint32_t add_u16_pair(uint32_t w, uint32_t acc) {
  return __builtin_amdgcn_udot2(__builtin_bit_cast(u16x2, w), (u16x2){1, 1}, acc, false);
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
  int qlo, qhi;  // biased exponents of a whose quotient is certainly normal and finite
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
      qlo = max(1, et - 124);
      qhi = min(254, et + 124);
    } else {
      elo = 1;
      ehi = 0;
      qlo = 1;
      qhi = 0;
    }
  }
  // the FMA sequence alone: exact for a with biased exponent in [elo, ehi]
  __device__ __forceinline__ float fma_seq(float a) const {
    float q = a * r;
    float res = fmaf(-q, T, a);
    q = fmaf(res, r, q);
    res = fmaf(-q, T, a);
    return fmaf(res, r, q);
  }
  __device__ __forceinline__ bool safe_exp(int e) const { return e >= elo && e <= ehi; }
  // a with biased exponent e in [qlo, qhi] has a normal, finite quotient a / T (its
  // exponent lies in [e - et + 126, e - et + 128], one step inside the limits)
  __device__ __forceinline__ bool quotient_normal(int e) const { return e >= qlo && e <= qhi; }
  // operator() behind one wave-uniform branch: the FMA sequence when every active lane
  // may take it (latency-bound code, where per-lane branches cost more than the division)
  __device__ __forceinline__ float uniform(float a) const {
    if (__all(safe_exp((int)((__float_as_uint(a) >> 23) & 0xff)))) return fma_seq(a);
    return (*this)(a);
  }
  __device__ __forceinline__ float operator()(float a) const {
    const int e = (int)((__float_as_uint(a) >> 23) & 0xff);
    if (e >= elo && e <= ehi) return fma_seq(a);
    if ((__float_as_uint(a) & 0x7fffffffu) == 0u) return a * r;  // +-0
    if (e == 255) return a * r;                                   // +-inf, NaN
    return a / T;
  }
};

// T == 1: the quotient is the value itself
struct UnitDivider {
  __device__ __forceinline__ float operator()(float a) const { return a; }
};

// The four quotients of one 16-byte vector of fp32 values. Divider: the FMA sequence for
// all four, then the general division behind one wave-uniform branch, taken only when some
// lane holds an element the FMA sequence does not cover (no per-element branches).
__device__ __forceinline__ void div4(const UnitDivider&, const u4& q, float x[4]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) x[e] = __uint_as_float(q[e]);
}
__device__ __forceinline__ void div4(const Divider& dv, const u4& q, float x[4]) {
  bool ok = true;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[e] = dv.fma_seq(__uint_as_float(q[e]));
    ok = ok && dv.safe_exp((int)((q[e] >> 23) & 0xffu));
  }
  if (__builtin_expect(__any(!ok), 0)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = dv(__uint_as_float(q[e]));
  }
}

// ---------------------------------------------------------------------------------------
// kernel arguments and per-row shared state
// ---------------------------------------------------------------------------------------

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

// A tie group located by a search (16-bit rows): its ord range, count, mass above it and
// per-element weight.
struct TieGroup {
  uint32_t lo, hi;
  uint32_t n;        // elements with ord in [lo, hi]
  uint32_t n_above;  // elements above hi
  double above;      // mass above hi
  double w;          // weight of one element
};

struct __align__(16) Smem {
  uint32_t hist[HIST_WORDS];     // 16-bit rows: packed u16 count per raw pattern; reused by index selection
  uint32_t gcount[NGROUP];       // count of each group of 256 ords
  uint32_t gabove_cnt[NGROUP];   // count strictly above the group (descending order)
  double gmass[NGROUP];          // fp64 mass of each group
  double gabove_mass[NGROUP];    // mass strictly above the group
  union {
    double subabove[NGROUP * 8];  // 16-bit rows: mass of the subgroups (32 ords) above each one, in its group
    struct {                      // fp32 rows
      double gmass_hi[NGROUP];    // upper bounds of the group masses (gmass holds the lower bounds)
      double gabove_hi[NGROUP];   // upper bound of the mass above each group
      uint64_t bmass[NBUCKET];    // list searches: fixed-point mass per bucket
      uint32_t bcnt[NBUCKET];     //   and entries per bucket
    } f32;
  };
  uint32_t seg_n[NWAVE];         // fp32 rows: entries each wave gathered into its list segment
  uint64_t pick;                 // fp32 rows: the entry a list search found
  uint32_t cand[NWAVE], cand_cnt[NWAVE], last[NWAVE], last_cnt[NWAVE];  // list searches, per wave
  double cand_excl[NWAVE], last_excl[NWAVE];
  double red_d[NWAVE];
  double red_d2[NWAVE];
  float red_f[NWAVE];
  int red_i[2 * NWAVE];

  int sel_jstar, sel_rank, sel_index;
  TieGroup spec[2];              // 16-bit rows: cutoff and guessed draw, searched side by side
  int spec_ok[2];
  uint32_t res_lo, res_hi;       // 16-bit rows: the drawn tie group (ords) and the rank in it
  int res_rank, res_ok;
  RowState st;
};

// ---------------------------------------------------------------------------------------
// block reductions (NT = 512 threads, NWAVE = 8 waves)
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
  static constexpr int D = NCH < PIPE ? NCH : PIPE;  // loads in flight per thread
  u4 r[NCH];
  const u4* row;
  int nvec;
  int vocab;
  __device__ __forceinline__ void init(const void* base, int nvec_, int vocab_) {
    row = (const u4*)base;
    nvec = nvec_;
    vocab = vocab_;
  }
  // Raw buffer loads whose whole offset is in the VGPR operand, so the buffer's range check
  // returns zeros past the row end (the check covers that operand; nothing is read past the
  // row), the code stays straight-line and the compiler waits for each chunk only when it
  // is first used. Non-temporal: the row is read from memory exactly once.
  __device__ __forceinline__ void load_chunk(int j) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)row, (short)0, nvec * 16, 0x00020000);
    r[j] = __builtin_bit_cast(
        u4, __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)(j * NT + (int)threadIdx.x) * 16u, 0, 2));
  }
  // issues the first D chunks; stream() issues the rest as it consumes the row
  __device__ __forceinline__ void load() {
#pragma unroll
    for (int j = 0; j < D; ++j) load_chunk(j);
  }
  // The first pass: f(j, q, base_index, valid) on chunk j while chunk j + D loads, so the
  // work on the row overlaps its arrival. Every chunk stays in registers for later passes.
  template <class F>
  __device__ __forceinline__ void stream(F&& f) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if (j + D < NCH) load_chunk(j + D);
      const int v = j * NT + (int)threadIdx.x;
      f(j, r[j], v * EPV, v < nvec);
      __builtin_amdgcn_sched_barrier(0);  // keeps the loads interleaved with the work
    }
  }
  // later passes over the resident row
  template <class F>
  __device__ __forceinline__ void for_each(F&& f) const {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int v = j * NT + (int)threadIdx.x;
      f(j, r[j], v * EPV, v < nvec);
    }
  }
  __device__ __forceinline__ int nchunks() const { return NCH; }
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
  // Every pass streams the row again: raw buffer loads four chunks per step, the next four
  // issued before the current four are used, so eight loads per thread are in flight
  // instead of one. The whole offset is in the VGPR operand, so the buffer's range check
  // returns zeros for the chunks past the row end that the last step reads ahead, and
  // nothing past the row is read.
  template <class F>
  __device__ __forceinline__ void for_each(F&& f) const {
    const int nch = (nvec + NT - 1) / NT;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)row, (short)0, nvec * 16, 0x00020000);
    auto ld = [&](int j) {
      return __builtin_bit_cast(
          u4, __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)(j * NT + (int)threadIdx.x) * 16u, 0, 0));
    };
    u4 a0 = ld(0), a1 = ld(1), a2 = ld(2), a3 = ld(3);
    for (int j = 0; j < nch; j += 4) {
      const u4 b0 = ld(j + 4), b1 = ld(j + 5), b2 = ld(j + 6), b3 = ld(j + 7);
      const int v = j * NT + (int)threadIdx.x;
      f(j, a0, v * EPV, v < nvec);
      if (j + 1 < nch) f(j + 1, a1, (v + NT) * EPV, v + NT < nvec);
      if (j + 2 < nch) f(j + 2, a2, (v + 2 * NT) * EPV, v + 2 * NT < nvec);
      if (j + 3 < nch) f(j + 3, a3, (v + 3 * NT) * EPV, v + 3 * NT < nvec);
      a0 = b0;
      a1 = b1;
      a2 = b2;
      a3 = b3;
    }
  }
  template <class F>
  __device__ __forceinline__ void stream(F&& f) const {
    for_each(f);
  }
  __device__ __forceinline__ int nchunks() const { return (nvec + NT - 1) / NT; }
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
  template <class F>
  __device__ __forceinline__ void stream(F&& f) const {
    for_each(f);
  }
  __device__ __forceinline__ int nchunks() const { return (nvec + NT - 1) / NT; }
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

// Index selection for register-resident 16-bit rows: the rank-th lowest-index element
// whose key lies in [lo, lo + span]. The key is the raw 16-bit pattern (ORD = false: a
// range of values of one sign is a contiguous range of raws) or the unfolded ord (ORD =
// true: ranges that take in both -0 and +0). Per-(chunk, wave) match counts locate the
// answer: every lane counts its matches in each chunk with packed 16-bit ops, and one
// transposed reduction across the wave leaves each chunk's total in a known lane (no
// branch or scalar dependency per chunk); only the wave holding the answer then looks at
// its lanes.
__device__ __forceinline__ uint32_t pk_sub_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) - __builtin_bit_cast(u16x2, b));
}
template <bool ORD>
__device__ __forceinline__ uint32_t key16x2(uint32_t w) {
  if constexpr (ORD) return ord16_pair(w);
  else return w;
}
// match bits of the 8 elements of one 16-byte vector (bit e for element e)
template <bool ORD>
__device__ __forceinline__ uint32_t match_bits16(const u4& q, uint32_t lo2, uint32_t span) {
  uint32_t bits = 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t dl = pk_sub_u16(key16x2<ORD>(q[d]), lo2);
    bits |= ((dl & 0xffffu) <= span ? 1u : 0u) << (2 * d);
    bits |= ((dl >> 16) <= span ? 1u : 0u) << (2 * d + 1);
  }
  return bits;
}

// Elements of one 16-byte vector whose key is NOT in [lo, lo + span]: a half of
// key - lo (mod 2^16) that is <= span becomes 0 (xor when span == 0, saturating
// subtraction otherwise), min(., 1) marks the others, packed adds and one dot product with
// (1, 1) count them. `one2` is (1, 1) held opaque by the caller.
template <bool ORD, bool EXACT>
__device__ __forceinline__ uint32_t lane_misses16(const u4& q, uint32_t lo2, uint32_t span2, uint32_t one2) {
  uint32_t m[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    uint32_t x;
    if constexpr (EXACT) {
      x = key16x2<ORD>(q[d]) ^ lo2;
    } else {
      x = __builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat(
                                           __builtin_bit_cast(u16x2, pk_sub_u16(key16x2<ORD>(q[d]), lo2)),
                                           __builtin_bit_cast(u16x2, span2)));
    }
    m[d] = pk_min_u16(x, one2);
  }
  const uint32_t s = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, m[0]) + __builtin_bit_cast(u16x2, m[1]) +
                                                      (__builtin_bit_cast(u16x2, m[2]) + __builtin_bit_cast(u16x2, m[3])));
  return add_u16_pair(s, 0u);
}

// Wave totals of 32 per-lane counters held as 16 packed u16 pairs (pair r = counters 2r,
// 2r + 1; every total fits 16 bits). Each stage halves the pairs a lane carries and sums
// it with a partner lane: lane bit 5 (permlane32 swap), bit 4 (permlane16 swap), bit 3
// (row rotate by 8), bit 2 (half-row mirror) pick the pair kept, then the quad sums. Lane l
// ends with the totals of pair (l >> 2) & 15.
__device__ __forceinline__ uint32_t wave_totals16(const uint32_t (&P)[16]) {
  const int l = lane_id();
  uint32_t s1[8], s2[4], s3[2];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(P[i], P[i + 8], false, false);
    s1[i] = r[0] + r[1];  // lanes 0-31: pair i, lanes 32-63: pair i + 8
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto r = __builtin_amdgcn_permlane16_swap(s1[i], s1[i + 4], false, false);
    s2[i] = r[0] + r[1];  // odd 16-lane rows: pair + 4
  }
  const bool b3 = (l & 8) != 0, b2 = (l & 4) != 0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t keep = b3 ? s2[i + 2] : s2[i], send = b3 ? s2[i] : s2[i + 2];
    s3[i] = keep + dpp<ROW_ROR8>(send, 0u);
  }
  const uint32_t keep = b2 ? s3[1] : s3[0], send = b2 ? s3[0] : s3[1];
  uint32_t t = keep + dpp<ROW_HALF_MIRROR>(send, 0u);
  t += dpp<QUAD_XOR1>(t, 0u);
  t += dpp<QUAD_XOR2>(t, 0u);
  return t;
}

// r[j] for a run-time, wave-uniform j < N: a switch on j (scalar compares and branches,
// only the taken case moves a vector). The empty asm statement in each case keeps the
// cases apart: merged into selects, or into one indexed load from the row array, they
// would cost N times the moves or move the row to scratch.
template <int N>
__device__ __forceinline__ u4 pick_chunk(const u4 (&r)[N], int j) {
  u4 q = {0u, 0u, 0u, 0u};
  switch (j) {
#define PBS_PICK(i)                                                  \
  case i:                                                            \
    if constexpr (i < N) {                                           \
      uint32_t a = r[i].x, b = r[i].y, c = r[i].z, d = r[i].w;       \
      asm volatile("" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));         \
      q = (u4){a, b, c, d};                                          \
    }                                                                \
    break;
    PBS_PICK(0) PBS_PICK(1) PBS_PICK(2) PBS_PICK(3) PBS_PICK(4) PBS_PICK(5) PBS_PICK(6) PBS_PICK(7)
    PBS_PICK(8) PBS_PICK(9) PBS_PICK(10) PBS_PICK(11) PBS_PICK(12) PBS_PICK(13) PBS_PICK(14) PBS_PICK(15)
    PBS_PICK(16) PBS_PICK(17) PBS_PICK(18) PBS_PICK(19) PBS_PICK(20) PBS_PICK(21) PBS_PICK(22) PBS_PICK(23)
    PBS_PICK(24) PBS_PICK(25) PBS_PICK(26) PBS_PICK(27) PBS_PICK(28) PBS_PICK(29) PBS_PICK(30) PBS_PICK(31)
#undef PBS_PICK
    default:
      break;
  }
  return q;
}

// With `out` (token and status arrays, row b) the lane that finds the element writes the
// row's result itself and SEL_WRITTEN is returned: no barrier hands the index to wave 0.
constexpr int SEL_WRITTEN = -2;
template <bool ORD, int DT, int NCH>
__device__ __forceinline__ int select_index_reg16(const RegRow<DT, NCH>& src, Smem& s, uint32_t lo, uint32_t span,
                                                  int rank, const KArgs* out = nullptr, int b = 0) {
  static_assert(NCH * NWAVE <= 256 && NCH <= 32, "chunk table must fit 4 entries per lane");
  const int l = lane_id(), w = wave_id();
  const uint32_t lo2 = lo | (lo << 16);
  {
    const uint32_t span2 = span | (span << 16);
    // (1, 1) through an empty asm: with a visible constant the compiler rewrites the packed
    // min(x, 1) as two compares and two selects
    uint32_t one2 = 0x00010001u;
    asm("" : "+v"(one2));
    // per-lane misses of every vector, chunks 2r and 2r + 1 packed in P[r]; vectors past
    // the row end hold zeros (the loads' range check) and are corrected for below
    uint32_t P[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) P[r] = 0u;
    if (span == 0u) {
#pragma unroll
      for (int j = 0; j < NCH; ++j) P[j >> 1] |= lane_misses16<ORD, true>(src.r[j], lo2, span2, one2) << (16 * (j & 1));
    } else {
#pragma unroll
      for (int j = 0; j < NCH; ++j) P[j >> 1] |= lane_misses16<ORD, false>(src.r[j], lo2, span2, one2) << (16 * (j & 1));
    }
    const uint32_t t = wave_totals16(P);
    if ((l & 3) == 0) {
      // matches = 8 per valid lane of the (chunk, wave) minus the valid lanes' misses; a
      // lane past the row end counted 8 misses unless the key of 0 lies in the range
      const uint32_t zero_in = (((key16x2<ORD>(0u) & 0xffffu) - lo) & 0xffffu) <= span ? 1u : 0u;
      const int r = l >> 2;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int j = 2 * r + h;
        if (j < NCH) {
          const int first = j * NT + w * 64;
          const uint32_t nlanes = (uint32_t)min(64, max(0, src.nvec - first));
          const uint32_t miss_all = (t >> (16 * h)) & 0xffffu;
          s.hist[j * NWAVE + w] = 8u * nlanes - miss_all + 8u * (64u - nlanes) * (1u - zero_in);
        }
      }
    }
  }
  __syncthreads();
  // every wave scans the totals (positions p = j*NWAVE + wave are in index order; lane l
  // holds p = 4l .. 4l+3), so no second barrier hands the answer around
  int pos = -1, rr = 0;
  {
    uint32_t c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t hv = s.hist[4 * l + i];  // in range for every lane; masked after the load
      c[i] = (4 * l + i < NCH * NWAVE) ? hv : 0u;
    }
    const uint32_t tot = c[0] + c[1] + c[2] + c[3];
    const uint32_t incl = wscan_u32(tot);
    const uint64_t hit = ballot(incl > (uint32_t)rank);
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
  }
  if (pos < 0) {
    if (threadIdx.x == 0) {
      if (out) {
        out->out_token[b] = 0;
        out->out_status[b] = PBS_ROW_OK;
      } else {
        s.sel_index = -1;
      }
    }
  } else {
    const int jstar = pos / NWAVE, wstar = pos % NWAVE;
    if (w == wstar) {
      const u4 q = pick_chunk<NCH>(src.r, jstar);
      const uint32_t bits = (jstar * NT + (int)threadIdx.x < src.nvec) ? match_bits16<ORD>(q, lo2, span) : 0u;
      const uint32_t cnt = (uint32_t)__popc(bits);
      const uint32_t incl = wscan_u32(cnt);
      const uint32_t excl = incl - cnt;
      if ((uint32_t)rr >= excl && (uint32_t)rr < incl) {
        uint32_t mb = bits;
        for (uint32_t k = (uint32_t)rr - excl; k > 0; --k) mb &= mb - 1u;
        const int idx = (jstar * NT + (int)threadIdx.x) * 8 + (__ffs(mb) - 1);
        if (out) {
          out->out_token[b] = idx;
          out->out_status[b] = PBS_ROW_OK;
        } else {
          s.sel_index = idx;
        }
      }
    }
  }
  if (out) return SEL_WRITTEN;
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
// 16-bit rows: the histogram
//
// hist counts every raw 16-bit pattern r of the row in half (r & 1) of word r >> 1 (u16
// counters). Ords map to raws one to one (raw_of_ord16), and the 256 ords of a group g
// are one aligned block of 256 raws: block g - 128 for g >= 128 (non-negative values, raw
// ascending with the ord) and block 255 - g below (negative values, raw descending).
// ---------------------------------------------------------------------------------------
// unfolded ord of one raw: -0 gets 0x7fff, +0 0x8000 (adjacent, and tied after scaling)
__device__ __forceinline__ uint32_t ord16u(uint32_t raw) { return raw ^ ((raw & 0x8000u) ? 0xffffu : 0x8000u); }

__device__ __forceinline__ uint32_t hist_count_raw(const Smem& s, uint32_t raw) {
  const uint32_t w = s.hist[raw >> 1];
  return (raw & 1u) ? (w >> 16) : (w & 0xffffu);
}
__device__ __forceinline__ uint32_t hist_count(const Smem& s, uint32_t o) { return hist_count_raw(s, raw_of_ord16(o)); }

// counts of ords o0 .. o0+3 (o0 % 4 == 0), in ord order: one 8-byte LDS read
__device__ __forceinline__ void counts4(const Smem& s, uint32_t o0, uint32_t n[4]) {
  if (o0 & 0x8000u) {
    const uint32_t* h = &s.hist[(o0 & 0x7fffu) >> 1];
    const uint32_t w0 = h[0], w1 = h[1];
    n[0] = w0 & 0xffffu;
    n[1] = w0 >> 16;
    n[2] = w1 & 0xffffu;
    n[3] = w1 >> 16;
  } else {
    // raws 0xfffc - o0 .. 0xffff - o0 hold ords o0 + 3 .. o0
    const uint32_t* h = &s.hist[(0xfffcu - o0) >> 1];
    const uint32_t w0 = h[0], w1 = h[1];
    n[3] = w0 & 0xffffu;
    n[2] = w0 >> 16;
    n[1] = w1 & 0xffffu;
    n[0] = w1 >> 16;
  }
}

// Adds the two 16-bit values packed in w. The byte address of raw r's counter word is
// (r >> 1) * 4, and the increment 1 << 16 * (r & 1); the packed 16-bit shift puts each
// value's low bit at bit 4 of its own half, where the 32-bit shift reads its amount.
__device__ __forceinline__ void hist_add_pair(Smem& s, uint32_t w) {
  const uint32_t t = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, w) << (u16x2){4, 4});
  uint8_t* h = (uint8_t*)s.hist;
  __hip_atomic_fetch_add((uint32_t*)(h + ((w << 1) & 0x1fffcu)), 1u << (t & 31u), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_WORKGROUP);
  __hip_atomic_fetch_add((uint32_t*)(h + ((w >> 15) & 0x1fffcu)), 1u << ((t >> 16) & 31u), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void hist_add_one(Smem& s, uint32_t raw) {
  __hip_atomic_fetch_add(&s.hist[raw >> 1], 1u << ((raw & 1u) << 4), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <int DT>
__device__ __forceinline__ float scaled16(uint32_t o, const Divider& dv) {
  return dv.uniform(raw_to_float<DT>(raw_of_ord16(o)));
}
// softmax weight of one distinct value relative to the row maximum m, in fp64 from the
// exact fp32 scaled value (pagedbatch takes softmax of the fp32 scaled row, sampling.py:26)
template <int DT>
__device__ __forceinline__ double weight16(uint32_t o, const Divider& dv, float m) {
  return weight_f(scaled16<DT>(o, dv), m);
}
// whether every value of group g divides by the FMA sequence: the group's smallest and
// largest magnitudes (raw low byte 0x00 and 0xff) bound its exponents
template <int DT>
__device__ __forceinline__ bool group_fma16(uint32_t g, const Divider& dv) {
  const uint32_t rb = raw_of_ord16(g << 8) & 0xff00u;
  const int e0 = (int)((__float_as_uint(raw_to_float<DT>(rb)) >> 23) & 0xff);
  const int e1 = (int)((__float_as_uint(raw_to_float<DT>(rb | 0xffu)) >> 23) & 0xff);
  return dv.safe_exp(e0) && dv.safe_exp(e1);
}
template <int DT>
__device__ __forceinline__ float weight16f(uint32_t o, const Divider& dv, float m) {
  const float x = scaled16<DT>(o, dv);
  return (x > -INFINITY) ? __builtin_amdgcn_exp2f((x - m) * 1.44269504088896341f) : 0.0f;
}

// Ords whose scaled value equals that of ord o. Neighbouring 16-bit values differ by at
// least 2^-11 relative, far more than fp32 rounding, so they only meet after the division
// by T where the quotient is subnormal, zero or infinite (-0 meets +0 there too); the map
// is monotone, so binary search.
template <int DT>
__device__ __forceinline__ void tie_range16(uint32_t o, const Divider& dv, uint32_t& lo, uint32_t& hi) {
  // most values: a normal quotient, known from the exponents alone (no division)
  if (dv.quotient_normal((int)((__float_as_uint(raw_to_float<DT>(raw_of_ord16(o))) >> 23) & 0xff))) {
    lo = hi = o;
    return;
  }
  const float x = scaled16<DT>(o, dv);
  const float ax = fabsf(x);
  if (ax >= 1.17549435e-38f && ax <= 3.40282347e38f) {
    lo = hi = o;
    return;
  }
  uint32_t a = ord16_neg_inf<DT>(), b = o;
  if (o <= a || scaled16<DT>(o - 1u, dv) < x) {
    a = o;
  } else {
    while (a < b) {
      const uint32_t mid = a + (b - a) / 2;
      if (scaled16<DT>(mid, dv) >= x) b = mid; else a = mid + 1;
    }
  }
  lo = a;
  a = o;
  b = ord16_pos_inf<DT>();
  if (o >= b || scaled16<DT>(o + 1u, dv) > x) {
    b = o;
  } else {
    while (a < b) {
      const uint32_t mid = a + (b - a + 1) / 2;
      if (scaled16<DT>(mid, dv) <= x) a = mid; else b = mid - 1;
    }
  }
  hi = a;
}

// ---------------------------------------------------------------------------------------
// searches. Wave-local: a wave runs them on LDS state no one writes meanwhile, so they
// need no barrier. Three levels, in descending ord order: groups of 256 ords (count and
// mass prefix tables), subgroups of 32 ords (the mass above each, from the mass pass) and
// single ords (weights computed on the spot, one per lane, an fp32 scan).
// ---------------------------------------------------------------------------------------
struct BinHit {
  uint32_t o;          // the ord found
  uint32_t cnt;        // elements at o
  uint32_t cnt_above;  // elements above o
  double mass_above;   // their mass
  double w;            // weight of one element at o
};

// the lowest non-empty group (latest in descending order) whose elements start at or
// before the need-th one: the group holding it
__device__ __forceinline__ int find_group_count(const Smem& s, uint32_t need) {
  const int l = lane_id();
  int found = -1;
#pragma unroll
  for (int i = 3; i >= 0; --i) {
    const uint32_t g = 4u * (uint32_t)l + (uint32_t)i;
    // both loads unconditional (bitwise and): a short-circuit test would wait for each
    // load in turn
    const uint32_t gc = s.gcount[g], ga = s.gabove_cnt[g];
    if ((gc != 0u) & (ga < need)) found = (int)g;
  }
  // lanes hold ascending groups: the first lane with a hit has the lowest
  const uint64_t hit = ballot(found >= 0);
  return hit ? (int)bcast_u32((uint32_t)found, first_lane(hit)) : -1;
}

// the lowest group >= lo >> 8 with mass, whose mass starts at or before target: the group
// holding it (a target that rounding puts past the group's end falls to its lowest element)
__device__ __forceinline__ int find_group_mass(const Smem& s, uint32_t lo, double target) {
  const int l = lane_id();
  const uint32_t glo = lo >> 8;
  int found = -1;
#pragma unroll
  for (int i = 3; i >= 0; --i) {
    const uint32_t g = 4u * (uint32_t)l + (uint32_t)i;
    const double gm = s.gmass[g], ga = s.gabove_mass[g];  // unconditional, as above
    if ((g >= glo) & (gm > 0.0) & (ga <= target)) found = (int)g;
  }
  const uint64_t hit = ballot(found >= 0);
  return hit ? (int)bcast_u32((uint32_t)found, first_lane(hit)) : -1;
}

// elements of group g with ord > o (4 ords per lane)
__device__ __forceinline__ uint32_t count_above_in_group(const Smem& s, uint32_t g, uint32_t o) {
  const int l = lane_id();
  uint32_t n4[4];
  counts4(s, g * 256u + 4u * (uint32_t)l, n4);
  uint32_t c = 0u;
#pragma unroll
  for (int i = 0; i < 4; ++i) c += (g * 256u + 4u * (uint32_t)l + (uint32_t)i > o) ? n4[i] : 0u;
  return wsum_u32(c);
}

// the need-th element (descending) of group g: its ord, count and the count above it
__device__ __forceinline__ void bins_count(const Smem& s, uint32_t g, uint32_t need, uint32_t& o, uint32_t& cnt,
                                           uint32_t& above) {
  const int l = lane_id();
  uint32_t n4[4];
  counts4(s, g * 256u + 252u - 4u * (uint32_t)l, n4);  // lane l: ords 255-4l .. 252-4l
  const uint32_t ct = n4[0] + n4[1] + n4[2] + n4[3];
  const uint32_t ci = wscan_u32(ct);
  const uint64_t hit = ballot(ci >= need);
  const int L = hit ? first_lane(hit) : 63;
  uint32_t run = ci - ct;
  int fi = 0;
  uint32_t fc = 0u, fa = 0u;
  bool done = false;
#pragma unroll
  for (int i = 3; i >= 0; --i) {
    if (!done && run + n4[i] >= need) {
      fi = i;
      fc = n4[i];
      fa = run;
      done = true;
    }
    run += n4[i];
  }
  o = g * 256u + 252u - 4u * (uint32_t)L + bcast_u32((uint32_t)fi, L);
  cnt = bcast_u32(fc, L);
  above = bcast_u32(fa, L);
}

// Ords 4l .. 4l+3 of group g for lane l (lanes ascending; from lane 63 down they run
// from the top): their counts (ords below lo count 0), fp32 weights exp(x - m) and the
// lane's mass, sum of count * weight with explicit FMAs in ascending ord order, so that
// every caller gets the same bits. One branch per group takes the FMA division for all
// four ords when the group's exponents allow it (an empty ord then adds 0 * w = +0).
template <int DT>
__device__ __forceinline__ float lane_ords16(const Smem& s, uint32_t g, uint32_t lo, const Divider& dv, float m,
                                             uint32_t (&n4)[4], float (&w4)[4]) {
  const uint32_t ob = g * 256u + 4u * (uint32_t)lane_id();
  counts4(s, ob, n4);
  if (group_fma16<DT>(g, dv)) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float x = dv.fma_seq(raw_to_float<DT>(raw_of_ord16(ob + (uint32_t)k)));
      w4[k] = __builtin_amdgcn_exp2f((x - m) * 1.44269504088896341f);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) w4[k] = n4[k] ? weight16f<DT>(ob + (uint32_t)k, dv, m) : 0.0f;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (ob + (uint32_t)k < lo) n4[k] = 0u;
  float lsum = (float)n4[0] * w4[0];
#pragma unroll
  for (int k = 1; k < 4; ++k) lsum = __builtin_fmaf((float)n4[k], w4[k], lsum);
  return lsum;
}

// mass of the elements of subgroup k of g with ord > o, and the weight of ord o
// (lanes 0..31: one ord each)
template <int DT>
__device__ __forceinline__ void mass_above_in_sub(const Smem& s, uint32_t g, uint32_t k, uint32_t o,
                                                  const Divider& dv, float m, double& mass, double& w) {
  const int l = lane_id();
  const uint32_t ol = g * 256u + 32u * k + 31u - (uint32_t)(l & 31);
  const uint32_t hc = hist_count(s, ol);  // every lane's ol is in range: load first, then mask
  const uint32_t c = (l < 32 && ol > o) ? hc : 0u;
  const float part = c ? (float)c * weight16f<DT>(ol, dv, m) : 0.0f;
  mass = (double)bcast_f32(wscan_f32(part), 63);
  w = (double)weight16f<DT>(o, dv, m);
}

// mass of the elements with ord > o from the prefix tables: the groups above o's group,
// the subgroups above its subgroup, and the ords above it in its subgroup (fp32 inside
// the subgroup), the same tables the searches' cumulative masses come from
template <int DT>
__device__ __forceinline__ double mass_above16(const Smem& s, uint32_t o, const Divider& dv, float m) {
  const uint32_t g = o >> 8, k = (o & 255u) >> 5;
  double ma, w;
  mass_above_in_sub<DT>(s, g, k, o, dv, m, ma, w);
  return s.gabove_mass[g] + s.subabove[g * 8u + k] + ma;
}

// the need-th element (descending) over all ords
template <int DT>
__device__ __forceinline__ bool find_by_count(const Smem& s, uint32_t need, const Divider& dv, float m, BinHit& h) {
  const int g = find_group_count(s, need);
  if (g < 0) return false;
  uint32_t ca;
  bins_count(s, (uint32_t)g, need - s.gabove_cnt[g], h.o, h.cnt, ca);
  const uint32_t k = (h.o & 255u) >> 5;
  double ma;
  mass_above_in_sub<DT>(s, (uint32_t)g, k, h.o, dv, m, ma, h.w);
  h.cnt_above = s.gabove_cnt[g] + ca;
  h.mass_above = s.gabove_mass[g] + s.subabove[(uint32_t)g * 8u + k] + ma;
  return true;
}

// The ord level of a search: subgroup k of group g, whose share of the target is
// r - start (r: the target less the mass above the group, start: the mass above the
// subgroup in the group).
template <int DT>
__device__ __forceinline__ bool find_in_sub(const Smem& s, uint32_t lo, uint32_t g, int k, double r, double start,
                                            const Divider& dv, float m, BinHit& h) {
  const int l = lane_id();
  // elements above the subgroup in the group (independent of the bin search below)
  uint32_t n4[4];
  counts4(s, g * 256u + 4u * (uint32_t)l, n4);
  uint32_t ca = 0u;
#pragma unroll
  for (int i = 0; i < 4; ++i) ca += (4 * l + i >= 32 * k + 32) ? n4[i] : 0u;
  // ords: lanes 0..31, descending; fp32 masses and scan inside one subgroup (its share of
  // the total is summed in fp64 above)
  const uint32_t ol = g * 256u + 32u * (uint32_t)k + 31u - (uint32_t)(l & 31);
  const uint32_t hc = hist_count(s, ol);  // every lane's ol is in range: load first, then mask
  const uint32_t c = (l < 32 && ol >= lo) ? hc : 0u;
  const float wt = c ? weight16f<DT>(ol, dv, m) : 0.0f;
  const float ms = (float)c * wt;
  const float mi = wscan_f32(ms);
  const uint32_t ci = wscan_u32(c);
  const float rs = (float)(r - start);
  uint64_t hit = ballot(l < 32 && mi > rs);
  if (!hit) {
    const uint64_t ne = ballot(ms > 0.0f);
    if (!ne) return false;
    hit = 1ull << (63 - __clzll((unsigned long long)ne));
  }
  const int L = first_lane(hit);
  h.o = g * 256u + 32u * (uint32_t)k + 31u - (uint32_t)L;
  h.cnt = bcast_u32(c, L);
  h.w = (double)bcast_f32(wt, L);
  h.mass_above = s.gabove_mass[g] + start + (double)bcast_f32(mi - ms, L);
  h.cnt_above = s.gabove_cnt[g] + wsum_u32(ca) + bcast_u32(ci - c, L);
  return true;
}

// the first ord >= lo (descending) whose cumulative mass from the top exceeds target; if
// rounding keeps the cumulative at or below it, the lowest ord >= lo with mass there
template <int DT>
__device__ __forceinline__ bool find_by_mass(const Smem& s, uint32_t lo, double target, const Divider& dv, float m,
                                             BinHit& h) {
  const int gi = find_group_mass(s, lo, target);
  if (gi < 0) return false;
  const uint32_t g = (uint32_t)gi;
  const double r = target - s.gabove_mass[g];
  const int l = lane_id();
  // subgroup (lanes 0..7, one each): the lowest one in range, with mass, whose interval
  // [above_k, above_{k-1}) starts at or before r; the intervals tile the group exactly
  const uint32_t klo = (g == (lo >> 8)) ? (lo & 255u) >> 5 : 0u;
  const uint32_t kl = (uint32_t)(l & 7);
  const double st_k = s.subabove[g * 8u + kl];
  const double sa_prev = s.subabove[g * 8u + (kl ? kl - 1u : 0u)], gm_g = s.gmass[g];
  const double en_k = kl ? sa_prev : gm_g;
  const uint64_t ks = ballot(l < 8 && kl >= klo && en_k > st_k && st_k <= r);
  if (!ks) return false;
  const int k = first_lane(ks);
  const double start = bcast_f64(st_k, k);
  return find_in_sub<DT>(s, lo, g, k, r, start, dv, m, h);
}

// The same search when the answer is expected in subgroup k of group g (the tie group
// after a known one): false, with nothing found, unless the target lies in that
// subgroup's interval, which is then the one find_by_mass would pick.
template <int DT>
__device__ __forceinline__ bool find_by_mass_near(const Smem& s, uint32_t lo, double target, uint32_t g, uint32_t k,
                                                  const Divider& dv, float m, BinHit& h) {
  const double r = target - s.gabove_mass[g];
  const double st = s.subabove[g * 8u + k];
  const double sa_prev = s.subabove[g * 8u + (k ? k - 1u : 0u)], gm_g = s.gmass[g];
  const double en = k ? sa_prev : gm_g;
  if (!(r >= st && r < en)) return false;
  return find_in_sub<DT>(s, lo, g, (int)k, r, st, dv, m, h);
}

// count and mass of the elements with ord >= t (whole wave; the rare tie-range path)
template <int DT>
__device__ __forceinline__ void count_mass_ge(const Smem& s, uint32_t t, const Divider& dv, float m, uint32_t& cnt,
                                              double& mass) {
  if (t > 0xffffu) {
    cnt = 0u;
    mass = 0.0;
    return;
  }
  const uint32_t g = t >> 8;
  const int l = lane_id();
  uint32_t n4[4];
  counts4(s, g * 256u + 4u * (uint32_t)l, n4);
  uint32_t c = 0u;
  double w = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t o = g * 256u + 4u * (uint32_t)l + (uint32_t)i;
    if (o >= t && n4[i]) {
      c += n4[i];
      w += (double)n4[i] * weight16<DT>(o, dv, m);
    }
  }
  cnt = wsum_u32(c) + s.gabove_cnt[g];
  mass = wsum_f64(w) + s.gabove_mass[g];
}

template <int DT>
__device__ __forceinline__ TieGroup tie_group(const Smem& s, const BinHit& h, uint32_t range_lo, const Divider& dv,
                                              float m) {
  TieGroup t;
  tie_range16<DT>(h.o, dv, t.lo, t.hi);
  t.lo = max(t.lo, range_lo);
  t.w = h.w;
  if (t.lo == h.o && t.hi == h.o) {
    t.n = h.cnt;
    t.n_above = h.cnt_above;
    t.above = h.mass_above;
  } else {
    uint32_t c_ge;
    double m_ge;
    count_mass_ge<DT>(s, t.hi + 1u, dv, m, t.n_above, t.above);
    count_mass_ge<DT>(s, t.lo, dv, m, c_ge, m_ge);
    t.n = c_ge - t.n_above;
  }
  return t;
}

// The k-th largest element by counts alone (before any mass is known): its ord, the ord
// range of its tie group, the group's count and the count above it. Wave-local: the
// counts above each group come from a wave scan of the group counts.
struct KthCount {
  uint32_t o, lo, hi, n, n_above;
  bool ok;
};

// elements with ord >= t (whole wave, from the group counts)
__device__ __forceinline__ uint32_t count_ge_local(const Smem& s, uint32_t t) {
  if (t > 0xffffu) return 0u;
  const uint32_t g = t >> 8;
  const int l = lane_id();
  uint32_t c = 0u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t gc = s.gcount[4 * l + i];
    c += (4u * (uint32_t)l + (uint32_t)i > g) ? gc : 0u;
  }
  return wsum_u32(c) + count_above_in_group(s, g, t - 1u);
}

template <int DT>
__device__ __forceinline__ KthCount kth_by_count(const Smem& s, uint32_t need, const Divider& dv) {
  const int l = lane_id();
  KthCount r = {};
  // lane l holds groups 255-4l .. 252-4l (descending); the scan gives the count above each
  uint32_t c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = s.gcount[255 - 4 * l - i];
  const uint32_t ct = (c[0] + c[1]) + (c[2] + c[3]);
  uint32_t run = wscan_u32(ct) - ct;
  int fi = -1;
  uint32_t fa = 0u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (fi < 0 && c[i] && run + c[i] >= need) {
      fi = i;
      fa = run;
    }
    run += c[i];
  }
  const uint64_t hit = ballot(fi >= 0);
  if (!hit) return r;
  const int L = first_lane(hit);
  const uint32_t g = 255u - 4u * (uint32_t)L - bcast_u32((uint32_t)fi, L);
  const uint32_t above_g = bcast_u32(fa, L);
  uint32_t cnt, ca;
  bins_count(s, g, need - above_g, r.o, cnt, ca);
  tie_range16<DT>(r.o, dv, r.lo, r.hi);
  if (r.lo == r.o && r.hi == r.o) {
    r.n = cnt;
    r.n_above = above_g + ca;
  } else {
    r.n_above = count_ge_local(s, r.hi + 1u);
    r.n = count_ge_local(s, r.lo) - r.n_above;
  }
  r.ok = true;
  return r;
}

// Top-k threshold, top-p cutoff and draw position from the histogram summaries. With
// top-p the cutoff and a guessed draw run side by side in waves 0 and 1 (one barrier).
// s.res_ok = 0 if a u16 counter wrapped (one value more than 65535 times) or a search
// found nothing: the caller then takes the general path.
template <int DT>
__device__ __forceinline__ void resolve16(Smem& s, int V, const Divider& dv, int kk, const KthCount& kc, float p,
                                          float u, float m, bool want_info, RowState& st) {
  // Wave 0 searches (and wave 1 beside it, for the guessed draw): the other waves wait at
  // the barriers instead of competing for their SIMDs' issue slots with copies of the same
  // work (waves w and w + 4 share a SIMD). Wave 0 leaves the selection in s.res_*, which
  // the caller reads after its next barrier; st is filled in wave 0 only.
  const int wv = wave_id();
  const bool side = p < 1.0f;
  const bool topk = kk > 0 && kk < V;
  BinHit h;
  uint32_t k_lo = 0u;
  uint32_t nk = (uint32_t)V;
  double zk = 0.0;
  TieGroup kt = {};
  if (wv < (side ? 2 : 1)) {
    zk = s.gabove_mass[0] + s.gmass[0];
    // top-k (sampling.py:15-17): K = ords >= the tie group of the k-th largest element,
    // found by counts before the masses (kth_by_count); Z_K = the mass above its tie
    // group plus the group's count times its weight
    if (topk) {
      kt.lo = kc.lo;
      kt.hi = kc.hi;
      kt.n = kc.n;
      kt.n_above = kc.n_above;
      kt.above = mass_above16<DT>(s, kc.hi, dv, m);
      kt.w = weight16<DT>(kc.o, dv, m);
      k_lo = kt.lo;
      zk = kt.above + (double)kt.n * kt.w;
      nk = kt.n_above + kt.n;
    }
    // top-p (sampling.py:18-25): keep the shortest prefix whose exclusive mass is <= p * Z_K.
    // Z_P lies in (tau, tau + one weight], so the draw's target u Z_P is close to u tau:
    // wave 0 searches the cutoff while wave 1 searches the draw for u tau; the guess is
    // kept below if u Z_P falls in the tie group it found.
    if (side) {
      const double tau = (double)p * zk;
      const bool ok = find_by_mass<DT>(s, k_lo, wv == 1 ? (double)u * tau : tau, dv, m, h);
      const TieGroup tg = ok ? tie_group<DT>(s, h, k_lo, dv, m) : TieGroup{};
      if (lane_id() == 0) {
        s.spec[wv] = tg;
        s.spec_ok[wv] = ok ? 1 : 0;
      }
    }
  }
  if (side) __syncthreads();
  if (wv != 0) return;

  // a u16 counter wrapped if the group counts do not add up to V (the general path then
  // takes the row)
  bool ok = s.gabove_cnt[0] + s.gcount[0] == (uint32_t)V;
  st = RowState{};
  st.status = PBS_ROW_OK;
  st.m = m;
  st.x_kth = topk ? scaled16<DT>(kc.o, dv) : -INFINITY;
  st.zk = zk;
  TieGroup ct = kt;
  int n_keep;
  double zp;
  const double tau = (double)p * zk;
  const bool cut = side && s.spec_ok[0] != 0;
  const bool have_guess = side && s.spec_ok[1] != 0;
  if (cut) ct = s.spec[0];
  if (cut) {
    const double kf = (ct.w > 0.0) ? floor((tau - ct.above) / ct.w) + 1.0 : (double)ct.n;
    n_keep = (int)fmax(1.0, fmin(kf, (double)ct.n));
    zp = ct.above + (double)n_keep * ct.w;
    st.n_kept = (int)ct.n_above + n_keep;
  } else {
    // all of K is kept; the cutoff group is K's lowest value (for the diagnostics only: the
    // draw below searches all of K)
    if (!topk && want_info) {
      if (find_by_count<DT>(s, nk, dv, m, h))
        ct = tie_group<DT>(s, h, 0u, dv, m);
      else
        ok = false;
    }
    n_keep = (int)ct.n;
    zp = zk;
    st.n_kept = (int)nk;
  }
  st.x_cut = scaled16<DT>(ct.hi, dv);
  st.n_cut_tie = (int)ct.n;
  st.n_cut_keep = n_keep;
  st.zp = zp;
  st.cut_lo = ct.lo;
  st.cut_hi = ct.hi;
  st.kord_lo = k_lo;

  // draw (sampling.py:26-27, inverse-CDF form): the first kept element whose cumulative
  // mass exceeds u * Z_P. With a top-p cutoff it lies in the cutoff tie group unless t is
  // below the mass above that group; without one, anywhere in K.
  const double t = (double)u * zp;
  st.target = t;
  TieGroup dt = ct;
  int n_avail = n_keep;
  if (ok && (!cut || t < ct.above)) {
    const TieGroup guess = s.spec[1];
    if (cut && have_guess && guess.lo > ct.hi && t >= guess.above && t < guess.above + (double)guess.n * guess.w) {
      dt = guess;
    } else {
      // below the guess (u Z_P past its tie group): first the guess's own subgroup, which
      // skips the group and subgroup levels when the target lies there
      const uint32_t dlo = cut ? ct.hi + 1u : k_lo;
      bool found = cut && have_guess && guess.lo > ct.hi && t >= guess.above &&
                   find_by_mass_near<DT>(s, dlo, t, guess.lo >> 8, (guess.lo & 255u) >> 5, dv, m, h);
      if (!found) found = find_by_mass<DT>(s, dlo, t, dv, m, h);
      if (found)
        dt = tie_group<DT>(s, h, dlo, dv, m);
      else
        ok = false;
    }
    n_avail = (int)dt.n;
  }
  st.sel_lo = dt.lo;
  st.sel_hi = dt.hi;
  st.sel_n = n_avail;
  st.sel_rank = (int)fmax(0.0, fmin((dt.w > 0.0) ? floor((t - dt.above) / dt.w) : 0.0, (double)(n_avail - 1)));
  if (lane_id() == 0) {
    s.res_lo = st.sel_lo;
    s.res_hi = st.sel_hi;
    s.res_rank = st.sel_rank;
    s.res_ok = ok ? 1 : 0;
  }
}

// Index of the rank-th lowest-index element whose ord lies in [lo, hi].
template <int DT, class Src>
__device__ __forceinline__ int select_tied16(const Src& src, Smem& s, uint32_t lo, uint32_t hi, int rank,
                                             const KArgs* out = nullptr, int b = 0) {
  // the caller's barrier after the searches (which read the histogram) comes first: the
  // selection reuses it
  if constexpr (Src::kStore) {
    // values of one sign: a contiguous range of raws (non-negative ords lo.. map to raws
    // lo - 0x8000.., negative ones to raws 0xffff - hi ..)
    if (lo >= 0x8000u || hi < 0x8000u)
      return select_index_reg16<false>(src, s, lo >= 0x8000u ? lo - 0x8000u : 0xffffu - hi, hi - lo, rank, out, b);
    // a range taking in both -0 and +0 (rare): the same selection on unfolded ords
    return select_index_reg16<true>(src, s, lo, hi - lo, rank, out, b);
  } else {
    return select_index<DT>(src, s, [=](uint32_t raw) { return ord16u(raw) - lo <= hi - lo; }, rank);
  }
}

// clears the histogram and the NaN counter (every thread takes a share)
__device__ __forceinline__ void hist_clear(Smem& s) {
  u4* h4 = (u4*)s.hist;
#pragma unroll
  for (int i = 0; i < HIST_WORDS / 4 / NT; ++i) h4[i * NT + threadIdx.x] = (u4){0u, 0u, 0u, 0u};
}

// group counts: thread t sums raws [128t, 128t + 128) (half a group, sixteen 16-byte LDS
// reads, rotated by lane so that a wave's reads spread over the banks)
template <int DT>
__device__ __forceinline__ void hist_group_counts(Smem& s) {
  const int l = lane_id();
  const u4* h4 = (const u4*)s.hist + threadIdx.x * 16;
  uint32_t c0 = 0u, c1 = 0u, c2 = 0u, c3 = 0u;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const u4 qv = h4[(i + l) & 15];
    c0 = add_u16_pair(qv.x, c0);
    c1 = add_u16_pair(qv.y, c1);
    c2 = add_u16_pair(qv.z, c2);
    c3 = add_u16_pair(qv.w, c3);
  }
  uint32_t c = (c0 + c1) + (c2 + c3);
  c += dpp<0xb1>(c, 0u);  // quad_perm [1,0,3,2]: the other half of the block
  if ((l & 1) == 0) {
    const uint32_t blk = threadIdx.x >> 1;
    s.gcount[blk < 128u ? blk + 128u : 255u - blk] = c;
  }
}

// The tail of a 16-bit row once the histogram is complete and the row maximum m is known:
// group counts, the k-th element by counts (top-k rows), group masses from the k-th
// element's group up, prefix tables, the searches (waves 0 and 1) and the selection.
// Returns false when the general path must take the row (a u16 counter wrapped).
template <int DT, class Src>
__device__ __forceinline__ bool tail16(const KArgs& a, Smem& s, Src& src, int b, const Divider& dv, float m, int kk,
                                       float p, float u) {
  const int V = a.vocab;
  const int l = lane_id(), wv = wave_id();

  hist_group_counts<DT>(s);
  __syncthreads();

  // top-k (sampling.py:15-17): the k-th element by counts; only its tie group and the
  // groups above it (K) need masses
  const bool topk = kk > 0 && kk < V;
  KthCount kc = {};
  uint32_t glo = 0u;
  if (topk) {
    kc = kth_by_count<DT>(s, (uint32_t)kk, dv);
    if (!kc.ok) return false;
    glo = kc.lo >> 8;
  }

  // group masses: the non-empty groups from glo up, ranked and dealt round-robin to the
  // waves; lane l weighs ords 4l .. 4l+3 of the group (the other groups get mass 0)
  {
    uint32_t ne = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) ne |= (s.gcount[4 * l + i] != 0u && 4u * (uint32_t)l + (uint32_t)i >= glo ? 1u : 0u) << i;
    if (wv == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (!((ne >> i) & 1u)) s.gmass[4 * l + i] = 0.0;
    }
    const uint32_t cnt = (uint32_t)__popc(ne);
    const uint32_t incl = wscan_u32(cnt);
    const uint32_t excl = incl - cnt;
    const uint32_t total = bcast_u32(incl, 63);
#pragma unroll 1
    for (uint32_t r = (uint32_t)wv; r < total; r += NWAVE) {
      const bool mine = r >= excl && r < incl;
      const int L = first_lane(ballot(mine));
      // the owning lane's (r - excl)-th set bit of ne (rank <= 3, no loop)
      const uint32_t k = mine ? r - excl : 0u;
      const uint32_t b1 = ne & (ne - 1u), b2 = b1 & (b1 - 1u), b3 = b2 & (b2 - 1u);
      const uint32_t bits = k == 0u ? ne : k == 1u ? b1 : k == 2u ? b2 : b3;
      const uint32_t g = bcast_u32(4u * (uint32_t)l + (uint32_t)(__ffs(bits) - 1), L);
      // the lanes' masses (fp32) summed by an fp64 wave scan: the group mass is the total
      // and the mass above subgroup k (ords 32k .. 32k+31, lanes 8k .. 8k+7) is the total
      // less the scan at lane 8k+7
      uint32_t n4[4];
      float w4[4];
      const float pf = lane_ords16<DT>(s, g, 0u, dv, m, n4, w4);
      const double incl = wscan_f64((double)pf);
      const double gm = bcast_f64(incl, 63);
      if ((l & 7) == 7) s.subabove[g * 8u + (uint32_t)(l >> 3)] = gm - incl;
      if (l == 0) s.gmass[g] = gm;
    }
  }
  __syncthreads();
  if (wv == 0) {
    // top-down exclusive prefixes: lane l holds groups 255-4l .. 252-4l
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
    uint32_t rc = ci - ct;
    double rw = wi - wt;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s.gabove_cnt[255 - 4 * l - i] = rc;
      s.gabove_mass[255 - 4 * l - i] = rw;
      rc += c[i];
      rw += w[i];
    }
  }
  __syncthreads();
  RowState st;
  resolve16<DT>(s, V, dv, kk, kc, p, u, m, a.out_info != nullptr, st);
  __syncthreads();
  if (!s.res_ok) return false;  // a counter wrapped

  // which of the tied tokens: the sel_rank-th lowest index with ord in [sel_lo, sel_hi]
  // without diagnostics the selecting lane writes the token itself
  const int tok = select_tied16<DT>(src, s, s.res_lo, s.res_hi, s.res_rank, a.out_info ? nullptr : &a, b);
  if (tok != SEL_WRITTEN && threadIdx.x == 0) write_info(a, b, tok < 0 ? 0 : tok, PBS_ROW_OK, st);
  return true;
}

// ---------------------------------------------------------------------------------------
// 16-bit stochastic row
//
// The stream builds the histogram and every thread's largest and smallest ord (packed u16
// max / min), so the row maximum and the NaN test are known at the stream's barrier, with
// no pass over the histogram for them.
// ---------------------------------------------------------------------------------------
template <int DT, class Src>
__device__ __forceinline__ bool sample_row16(const KArgs& a, Smem& s, Src& src, int b, float T, int kk, float p,
                                             float u) {
  constexpr int EPV = DTraits<DT>::EPV;
  const int V = a.vocab;
  const int l = lane_id(), wv = wave_id();
  Divider dv;
  dv.init(T);  // (its division overlaps the first loads)

  // stream: the histogram and the thread's ord range (packed u16 max / min of the unfolded
  // ords). The histogram is cleared while the first loads are in flight; the barrier
  // orders LDS only.
  hist_clear(s);
  lds_barrier();
  uint32_t omx = 0u, omn = 0xffffffffu;
  src.stream([&](int, const u4& q, int base, bool vvalid) {
    if constexpr (Src::kVector) {
      if (vvalid) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          hist_add_pair(s, q[d]);
          const uint32_t o2 = ord16_pair(q[d]);
          omx = pk_max_u16(omx, o2);
          omn = pk_min_u16(omn, o2);
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < EPV; ++e)
        if (elem_valid(src, vvalid, base + e)) {
          const uint32_t raw = elem_raw<DT>(q, e);
          hist_add_one(s, raw);
          const uint32_t o = ord16u(raw);
          omx = pk_max_u16(omx, o | (o << 16));
          omn = pk_min_u16(omn, o | (o << 16));
        }
    }
  });
  {
    const uint32_t mx = wmax_u32(max(omx & 0xffffu, omx >> 16));
    const uint32_t mn = wmin_u32(min(omn & 0xffffu, omn >> 16));
    if (l == 0) {
      s.red_i[wv] = (int)mx;
      s.red_i[NWAVE + wv] = (int)mn;
    }
  }
  __syncthreads();
  uint32_t omax = 0u, omin = 0xffffu;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    omax = max(omax, (uint32_t)s.red_i[w]);
    omin = min(omin, (uint32_t)s.red_i[NWAVE + w]);
  }
  omax = uni_u32(omax);
  omin = uni_u32(omin);
  // NaN (multinomial raises on it, sampling.py:27): ords above +inf or below -inf
  if (omax > ord16u(DT == PBS_DTYPE_BF16 ? 0x7f80u : 0x7c00u) ||
      omin < ord16u(DT == PBS_DTYPE_BF16 ? 0xff80u : 0xfc00u)) {
    if (threadIdx.x == 0) write_error(a, b, PBS_ROW_NAN, NAN);
    return true;
  }
  const float m = scaled16<DT>(omax, dv);
  if (!(m > -INFINITY && m < INFINITY)) {
    if (threadIdx.x == 0) write_error(a, b, PBS_ROW_NONFINITE, m);
    return true;
  }

  return tail16<DT>(a, s, src, b, dv, m, kk, p, u);
}

// ---------------------------------------------------------------------------------------
// General stochastic row (fp32 logits, and 16-bit rows whose histogram counters would
// wrap): exact bisection on 32-bit ords of x = fp32(v)/T. Every probe is one pass over
// the row with fp64 accumulation in a fixed order, so the result is deterministic. The
// first pass streams `src0` (registers when the row fits); the bisection passes re-read
// the row (`src`), redoing the exact division per element.
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

template <int DT, class Div>
__device__ __forceinline__ float x_at(const Div& dv, const u4& q, int e) {
  return dv(raw_to_float<DT>(elem_raw<DT>(q, e)));
}

// count and mass (relative to m) of elements with ord32(x) >= t
template <int DT, class Src>
__device__ __forceinline__ void bis_ge(const Src& src, Smem& s, const Divider& dv, uint32_t t, float m,
                                       bool want_mass, uint32_t& cnt, double& mass) {
  constexpr int EPV = DTraits<DT>::EPV;
  uint32_t c = 0;
  double ms = 0.0;
  src.for_each([&](int, const u4& q, int base, bool vvalid) {
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      if (elem_valid(src, vvalid, base + e)) {
        const float x = x_at<DT>(dv, q, e);
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
template <int DT, class Src>
__device__ __forceinline__ uint32_t bis_count(const Src& src, Smem& s, const Divider& dv, uint32_t lo, uint32_t hi,
                                              uint32_t need) {
  while (lo < hi) {
    const uint32_t mid = lo + (uint32_t)(((uint64_t)hi - lo + 1) / 2);
    uint32_t c;
    double ms;
    bis_ge<DT>(src, s, dv, mid, 0.0f, false, c, ms);
    if (c >= need) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// largest o in [lo, hi] with mass(ord >= o) > target; mass(ord >= lo) > target is given
template <int DT, class Src>
__device__ __forceinline__ uint32_t bis_mass(const Src& src, Smem& s, const Divider& dv, uint32_t lo, uint32_t hi,
                                             double target, float m) {
  while (lo < hi) {
    const uint32_t mid = lo + (uint32_t)(((uint64_t)hi - lo + 1) / 2);
    uint32_t c;
    double ms;
    bis_ge<DT>(src, s, dv, mid, m, true, c, ms);
    if (ms > target) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// First pass over the row: max of x and the NaN flag (returns NaN then).
template <int DT, class Src>
__device__ __forceinline__ float bis_max(Src& src, Smem& s, const Divider& dv, bool streaming) {
  constexpr int EPV = DTraits<DT>::EPV;
  float xmax = -INFINITY;
  int nan = 0;
  auto f = [&](int, const u4& q, int base, bool vvalid) {
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      const float x = x_at<DT>(dv, q, e);
      if (elem_valid(src, vvalid, base + e)) {
        xmax = fmaxf(xmax, x);
        nan |= (x != x) ? 1 : 0;
      }
    }
  };
  if (streaming) src.stream(f);
  else src.for_each(f);
  return block_max_nan(xmax, nan, s);
}

template <int DT, class Src>
__device__ __forceinline__ void sample_row_bisect(const KArgs& a, Smem& s, const Src& src, int b, float m,
                                                  const Divider& dv, int kk, float p, float u) {
  const int V = a.vocab;
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
    kord = bis_count<DT>(src, s, dv, ord_lo, ord_m, (uint32_t)kk);
    st.x_kth = float_of_ord32(kord);
  }
  st.kord_lo = kord;
  bis_ge<DT>(src, s, dv, kord, m, true, c, ms);
  const double zk = ms;
  const uint32_t nk = c;
  st.zk = zk;

  // top-p cutoff: the ord where the descending cumulative mass first exceeds p*Z
  uint32_t cut;
  double above_cut;
  if (p < 1.0f && zk * (double)p < zk) {
    const double tau = (double)p * zk;
    cut = bis_mass<DT>(src, s, dv, kord, ord_m, tau, m);
    uint32_t n_above, n_ge;
    bis_ge<DT>(src, s, dv, cut + 1u, m, true, n_above, above_cut);
    bis_ge<DT>(src, s, dv, cut, m, false, n_ge, ms);
    st.n_cut_tie = (int)(n_ge - n_above);
    const double w = (double)weight32(float_of_ord32(cut), m);
    double kf = (w > 0.0) ? floor((tau - above_cut) / w) + 1.0 : (double)st.n_cut_tie;
    kf = fmax(1.0, fmin(kf, (double)st.n_cut_tie));
    st.n_cut_keep = (int)kf;
    st.zp = above_cut + (double)st.n_cut_keep * w;
    st.n_kept = (int)n_above + st.n_cut_keep;
  } else {
    // keep all of K: the cutoff group is K's lowest value
    cut = bis_count<DT>(src, s, dv, kord, ord_m, nk);
    uint32_t n_above;
    bis_ge<DT>(src, s, dv, cut + 1u, m, true, n_above, above_cut);
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
    sel = bis_mass<DT>(src, s, dv, cut + 1u, ord_m, t, m);
    double B;
    uint32_t n_above, n_ge;
    bis_ge<DT>(src, s, dv, sel + 1u, m, true, n_above, B);
    bis_ge<DT>(src, s, dv, sel, m, false, n_ge, ms);
    const double w = (double)weight32(float_of_ord32(sel), m);
    const double rf = (w > 0.0) ? floor((t - B) / w) : 0.0;
    rank = (int)fmax(0.0, fmin(rf, (double)((int)(n_ge - n_above) - 1)));
  } else {
    const double w = (double)weight32(float_of_ord32(cut), m);
    const double rf = (w > 0.0) ? floor((t - above_cut) / w) : 0.0;
    rank = (int)fmax(0.0, fmin(rf, (double)(st.n_cut_keep - 1)));
  }
  const int tok = select_index<DT>(src, s, [&](uint32_t raw) { return ord32(dv(raw_to_float<DT>(raw))) == sel; },
                                   rank);

  if (threadIdx.x == 0) write_info(a, b, tok < 0 ? 0 : tok, PBS_ROW_OK, st);
}

// ---------------------------------------------------------------------------------------
// fp32 stochastic rows.
//
// Bins are the top 16 bits of key = ord32(x): 65536 consecutive fp32 values each. The
// stream histograms them (u16 counters, indexed like the 16-bit rows' raws) and sums the
// row's softmax mass with a running maximum per thread. From the counts and each bin's
// value range come a lower and an upper bound on every bin's mass, and so on every
// cumulative from the top: a search by count lands on one bin; a search by mass lands
// between the bin where the upper bounds cross the target (the cumulative can cross no
// earlier) and the bin where the lower bounds do (no later). One more pass gathers those
// windows' elements into LDS as entries E = (~key << 32 | index), whose ascending order is
// the sampling order (value descending, index ascending), and sums the exact mass above
// each window. Searches in the gathered list narrow an interval of E over 256 buckets per
// level; weights enter the bucket sums as fixed-point integers, so every sum is exact and
// independent of the gather's order. Top-k rows whose k-th element lies within the top few
// thousand gather everything from its bin up instead and resolve from that list alone.
// Rows whose windows hold more elements than LDS takes, or whose counters wrap, take the
// bisection path.
// ---------------------------------------------------------------------------------------
constexpr uint32_t LIST_CAP = HIST_WORDS / 2;  // entries of the list, which reuses the histogram
constexpr uint32_t SEG = LIST_CAP / NWAVE;     // list segment of each wave
constexpr uint32_t SMALLK_CAP = 4096;          // top-k rows resolved from one list up to this size
constexpr float LOG2E_F = 1.44269504088896341f;
constexpr double FIXQ = 0x1p-38;               // fixed-point weight unit

// exp(x - m) as the fp32 searches compute it: fp32 difference and product, hardware exp2
__device__ __forceinline__ float wexp(float x, float m) {
  return (x > -INFINITY) ? __builtin_amdgcn_exp2f((x - m) * LOG2E_F) : 0.0f;
}
// the same weight for x that is not NaN, without the test (x = -inf gives exp2(-inf) = 0)
__device__ __forceinline__ float wexp_num(float x, float m) { return __builtin_amdgcn_exp2f((x - m) * LOG2E_F); }
// ord32(x) for x that is not NaN: x + 0 turns -0 into +0 and leaves every other value alone
__device__ __forceinline__ uint32_t ord32_num(float x) {
  const uint32_t b = __float_as_uint(x + 0.0f);
  return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}
// floor(w * 2^38) for 0 <= w < 2: at most 2^39, so 2^14 of them sum exactly in a double
__device__ __forceinline__ uint64_t fixq(float w) {
  return (uint64_t)((double)w * 0x1p38);
}
// histogram index of x: the top 16 bits of its pattern, -0 folded onto +0 (the raw whose
// unfolded ord is ord32(x) >> 16)
__device__ __forceinline__ uint32_t bin_raw32(float x) {
  const uint32_t b = __float_as_uint(x);
  return (b == 0x80000000u) ? 0u : (b >> 16);
}
// (HIP's min/max on mixed 64-bit integer types resolve to the double overloads: these do not)
__device__ __forceinline__ uint64_t min_u64(uint64_t a, uint64_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint32_t key_of(uint64_t e) { return ~(uint32_t)(e >> 32); }
__device__ __forceinline__ int index_of(uint64_t e) { return (int)(uint32_t)e; }
__device__ __forceinline__ float value_of(uint64_t e) { return float_of_ord32(key_of(e)); }
// the interval of E holding key k, and the one holding bins [lo, hi]
__device__ __forceinline__ uint64_t e_first(uint32_t key) { return (uint64_t)(~key) << 32; }
__device__ __forceinline__ uint64_t e_last(uint32_t key) { return ((uint64_t)(~key) << 32) | 0xffffffffull; }
__device__ __forceinline__ uint64_t e_bins_first(uint32_t hi) { return e_first((hi << 16) | 0xffffu); }
__device__ __forceinline__ uint64_t e_bins_last(uint32_t lo) { return e_last(lo << 16); }

// Bounds on wexp(x, m) over the x of bin o that a row with maximum m can hold. wexp is
// monotone up to its last-ulp rounding; the factors cover that and the fp32 partial sums
// of the exact passes. The lowest key of the -inf bin is a NaN pattern: weight 0.
__device__ __forceinline__ void bin_bounds(uint32_t o, float m, float& wlo, float& whi) {
  const float xlo = float_of_ord32(o << 16);
  const float xhi = fminf(float_of_ord32((o << 16) | 0xffffu), m);
  wlo = wexp(xlo, m) * 0.999998f;
  whi = wexp(xhi, m) * 1.000002f;
}

// elements in bins >= t (whole wave)
__device__ __forceinline__ uint32_t count_bins_ge(const Smem& s, uint32_t t) {
  if (t > 0xffffu) return 0u;
  const uint32_t g = t >> 8;
  return count_above_in_group(s, g, t - 1u) + s.gabove_cnt[g];
}

// lower (HI = false) or upper bound of the mass in bins > o (whole wave)
template <bool HI>
__device__ __forceinline__ double bound_above(const Smem& s, uint32_t o, float m) {
  const uint32_t g = o >> 8;
  const int l = lane_id();
  uint32_t n4[4];
  counts4(s, g * 256u + 4u * (uint32_t)l, n4);
  double w = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t b = g * 256u + 4u * (uint32_t)l + (uint32_t)i;
    if (b > o && n4[i]) {
      float wl, wh;
      bin_bounds(b, m, wl, wh);
      w += (double)n4[i] * (double)(HI ? wh : wl);
    }
  }
  return wsum_f64(w) + (HI ? s.f32.gabove_hi[g] : s.gabove_mass[g]);
}

// The bin >= lo (descending from the top) where the cumulative bound mass, upper bounds
// (HI) or lower bounds, first exceeds target; the lowest non-empty bin >= lo if it never
// does. Whole wave, no barrier.
template <bool HI>
__device__ __forceinline__ uint32_t find_bin_bound(const Smem& s, uint32_t lo, double target, float m) {
  const double* above = HI ? s.f32.gabove_hi : s.gabove_mass;
  const int l = lane_id();
  const uint32_t glo = lo >> 8;
  // the lowest non-empty group >= glo whose mass starts at or before target
  int found = -1, lowest = -1;
#pragma unroll
  for (int i = 3; i >= 0; --i) {
    const uint32_t g = 4u * (uint32_t)l + (uint32_t)i;
    if (g >= glo && s.gcount[g]) {
      lowest = (int)g;
      if (above[g] <= target) found = (int)g;
    }
  }
  const uint64_t hit = ballot(found >= 0);
  int gi;
  if (hit) {
    gi = (int)bcast_u32((uint32_t)found, first_lane(hit));
  } else {
    const uint64_t any = ballot(lowest >= 0);
    gi = any ? (int)bcast_u32((uint32_t)lowest, first_lane(any)) : (int)glo;
  }
  const uint32_t g = (uint32_t)gi;
  // lane l: bins 255-4l .. 252-4l of the group, descending
  uint32_t n4[4];
  counts4(s, g * 256u + 252u - 4u * (uint32_t)l, n4);
  double w[4];
  uint32_t ne = 0u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t o = g * 256u + 255u - 4u * (uint32_t)l - (uint32_t)i;
    const uint32_t c = (o >= lo) ? n4[3 - i] : 0u;
    float wl, wh;
    bin_bounds(o, m, wl, wh);
    w[i] = (double)c * (double)(HI ? wh : wl);
    ne |= (c != 0u ? 1u : 0u) << i;
  }
  const double wt = ((w[0] + w[1]) + w[2]) + w[3];
  const double wi = wscan_f64(wt);
  const double base = above[g];
  const uint64_t h = ballot(base + wi > target);
  int L, fi = 0;
  if (h) {
    L = first_lane(h);
    double run = base + (wi - wt);
    bool done = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (!done && run + w[i] > target) {
        fi = i;
        done = true;
      }
      run += w[i];
    }
  } else {
    const uint64_t nz = ballot(ne != 0u);
    L = nz ? 63 - __clzll((unsigned long long)nz) : 0;
    fi = ne ? 31 - __clz(ne) : 0;
  }
  return g * 256u + 255u - 4u * (uint32_t)L - bcast_u32((uint32_t)fi, L);
}

// One pass over the row: every element whose bin lies in one of the NW windows [lo_i,
// hi_i] (they may overlap) goes into L, unsorted; above_i gets the exact mass of the
// elements in bins above window i. Each wave fills its own segment of SEG entries, no
// atomics, in one of two ways:
//   cols: every lane appends to its own column of the segment (entry slot * 64 + lane,
//     COL_CAP slots, a full lane writing on into a spare last slot), with no cross-lane
//     work per element; one pass at the end compacts the columns into the segment's
//     first entries, slot by slot. Returns false if a column overflowed.
//   otherwise: a ballot and lane ranks per element whose vector holds an entry.
// Returns false if a segment overflowed. The list's order is irrelevant to its readers.
constexpr uint32_t COL_CAP = SEG / 64 - 1;  // entries per lane column (the last slot is spare)
template <int DT, int NW, class Src, class Div>
__device__ __forceinline__ bool gather_bins(const Src& src, Smem& s, uint64_t* L, const Div& dv, float m,
                                                uint32_t lo0, uint32_t hi0, uint32_t lo1, uint32_t hi1,
                                                uint32_t lo2, uint32_t hi2, double& above0, double& above1,
                                                double& above2, bool cols) {
  const uint32_t lo[3] = {lo0, lo1, lo2}, hi[3] = {hi0, hi1, hi2};
  uint64_t* const seg = L + wave_id() * SEG;
  const uint32_t ln = (uint32_t)lane_id();
  uint32_t wn = 0u;  // entries the wave appended (uniform)
  uint32_t lc = 0u;  // cols: entries this lane appended (may pass COL_CAP: overflow)
  __syncthreads();   // the histogram the list overwrites is no longer read
  double acc[NW];
#pragma unroll
  for (int r = 0; r < NW; ++r) acc[r] = 0.0;
  src.for_each([&](int, const u4& q, int base, bool vvalid) {
    float part[NW];
#pragma unroll
    for (int r = 0; r < NW; ++r) part[r] = 0.0f;
    if constexpr (Src::kVector) {
      // Straight-line work per element (no NaN reaches this pass); the appends sit behind
      // one ballot per vector, which is empty for nearly every vector.
      float xs[4];
      div4(dv, q, xs);
      uint32_t key[4];
      bool in[4];
      bool any = false;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        key[e] = ord32_num(xs[e]);
        const uint32_t o = key[e] >> 16;
        const float w = vvalid ? wexp_num(xs[e], m) : 0.0f;
        bool hit = false;
#pragma unroll
        for (int r = 0; r < NW; ++r) {
          part[r] += (o > hi[r]) ? w : 0.0f;
          hit = hit || (o - lo[r] <= hi[r] - lo[r]);
        }
        in[e] = vvalid && hit;
        any = any || in[e];
      }
      if (cols) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (in[e]) {
            seg[min(lc, COL_CAP) * 64u + ln] = ((uint64_t)(~key[e]) << 32) | (uint32_t)(base + e);
            ++lc;
          }
        }
      } else if (ballot(any)) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint64_t bal = ballot(in[e]);
          const uint32_t slot = wn + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                               __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
          if (in[e] && slot < SEG) seg[slot] = ((uint64_t)(~key[e]) << 32) | (uint32_t)(base + e);
          wn += (uint32_t)__popcll(bal);
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = x_at<DT>(dv, q, e);
        const uint32_t key = ord32(x);
        const uint32_t o = key >> 16;
        const bool ok = elem_valid(src, vvalid, base + e);
        const float w = ok ? wexp(x, m) : 0.0f;
        bool in = false;
#pragma unroll
        for (int r = 0; r < NW; ++r) {
          part[r] += (o > hi[r]) ? w : 0.0f;
          in = in || (o - lo[r] <= hi[r] - lo[r]);
        }
        const uint64_t bal = ballot(ok && in);
        if (bal) {
          const uint32_t slot = wn + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                               __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
          if (ok && in && slot < SEG) seg[slot] = ((uint64_t)(~key) << 32) | (uint32_t)(base + e);
          wn += (uint32_t)__popcll(bal);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < NW; ++r) acc[r] += (double)part[r];
  });
  double tot[3] = {0.0, 0.0, 0.0};
#pragma unroll
  for (int r = 0; r < NW; ++r) {
    const double a = wsum_f64(acc[r]);
    if (lane_id() == 0) s.red_d[wave_id()] = a;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) tot[r] += s.red_d[w];
    __syncthreads();
  }
  above0 = tot[0];
  above1 = tot[1];
  above2 = tot[2];
  if (cols) {
    if (ballot(lc > COL_CAP)) {
      wn = SEG + 1u;  // a column overflowed: the caller gathers again with ballots
    } else {
      // slot by slot, the entries of the lanes that have one move to the next free entries
      // of the segment: every destination lies at or before its source (at most 64 entries
      // per earlier slot went before it), in a slot already read
      const uint32_t nslot = wmax_u32(lc);
      for (uint32_t k = 0u; k < nslot; ++k) {
        const bool has = k < lc;
        const uint64_t bal = ballot(has);
        if (has) {
          const uint64_t e = seg[k * 64u + ln];
          seg[wn + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u))] = e;
        }
        wn += (uint32_t)__popcll(bal);
      }
    }
  }
  if (lane_id() == 0) s.seg_n[wave_id()] = wn;
  __syncthreads();
  bool ok = true;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) ok = ok && s.seg_n[w] <= SEG;
  return ok;
}

// gather_bins with lane columns when the windows are dense (one element in 256 or more, so
// that most of the wave's 256-element vectors hold an entry and the ballot path's skip of
// empty vectors saves little) and hold few enough elements that no column should fill (at
// most 12 per lane on average, against COL_CAP); else with ballots. A column that overflows anyway
// (entries crowded into few lanes) costs one more pass with ballots. The histogram must
// still be intact (the counts decide).
constexpr uint32_t COLS_MAX = 12u * NT;
template <int DT, int NW, class Src, class Div>
__device__ __forceinline__ bool gather_windows(const Src& src, Smem& s, uint64_t* L, const Div& dv, float m,
                                               uint32_t lo0, uint32_t hi0, uint32_t lo1, uint32_t hi1,
                                               uint32_t lo2, uint32_t hi2, double& above0, double& above1,
                                               double& above2) {
  const uint32_t lo[3] = {lo0, lo1, lo2}, hi[3] = {hi0, hi1, hi2};
  uint32_t n_in = 0u;  // elements in the windows, counted once per window they lie in
#pragma unroll
  for (int r = 0; r < NW; ++r) n_in += count_bins_ge(s, lo[r]) - count_bins_ge(s, hi[r] + 1u);
  const bool cols = Src::kVector && n_in <= COLS_MAX && (uint64_t)n_in * 256u >= (uint64_t)src.vocab;
  if (gather_bins<DT, NW>(src, s, L, dv, m, lo0, hi0, lo1, hi1, lo2, hi2, above0, above1, above2, cols))
    return true;
  return cols && gather_bins<DT, NW>(src, s, L, dv, m, lo0, hi0, lo1, hi1, lo2, hi2, above0, above1, above2, false);
}

// count and fixed-point mass (FIXQ units, exact) of the list's entries in [ea, eb]; each
// wave reads its own segment
template <bool MASS>
__device__ __forceinline__ void list_sum(Smem& s, const uint64_t* L, uint64_t ea, uint64_t eb, float m,
                                         uint32_t& cnt, double& mass) {
  uint32_t c = 0u;
  uint64_t q = 0u;
  const uint64_t* const seg = L + wave_id() * SEG;
  const int sn = (int)s.seg_n[wave_id()];
  for (int i = lane_id(); i < sn; i += 64) {
    const uint64_t e = seg[i];
    if (e >= ea && e <= eb) {
      ++c;
      if (MASS) q += fixq(wexp(value_of(e), m));
    }
  }
  c = wsum_u32(c);
  const double qd = MASS ? wsum_f64((double)q) : 0.0;
  if (lane_id() == 0) {
    s.red_i[wave_id()] = (int)c;
    s.red_d[wave_id()] = qd;
  }
  __syncthreads();
  cnt = 0u;
  mass = 0.0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    cnt += (uint32_t)s.red_i[w];
    mass += s.red_d[w];
  }
  __syncthreads();
}

struct Pick {
  uint64_t e;   // the entry (~0: the interval held none)
  double excl;  // cumulative before it
  double w;     // its weight (fixed-point, as the cumulative counts it)
};

// The first entry of the list in [ea, eb], in ascending order, whose inclusive cumulative
// from `base` exceeds target: weights are the entries' fixed-point masses (MASS) or 1 (a
// count). If none does, the last entry with weight. Each level spreads the interval over
// NBUCKET buckets, sums them exactly and keeps the bucket where the cumulative crosses,
// until one entry is left.
template <bool MASS>
__device__ __forceinline__ Pick list_pick(Smem& s, const uint64_t* L, uint64_t ea, uint64_t eb, float m,
                                          double base, double target) {
  const int t = threadIdx.x, l = lane_id(), wv = wave_id();
  const uint64_t* const seg = L + wv * SEG;
  const int sn = (int)s.seg_n[wv];
  const double unit = MASS ? FIXQ : 1.0;
  uint64_t lo = ea, hi = eb;
  double B = base;
  uint32_t cnt = 0u;
#pragma unroll 1
  for (int level = 0; level < 8; ++level) {
    const uint64_t span = hi - lo;
    const int sh = (span >> 8) ? 64 - __clzll((unsigned long long)(span >> 8)) : 0;
    if (t < NBUCKET) {
      s.f32.bmass[t] = 0u;
      s.f32.bcnt[t] = 0u;
    }
    __syncthreads();
    for (int i = l; i < sn; i += 64) {
      const uint64_t e = seg[i];
      if (e >= lo && e <= hi) {
        const uint32_t bk = (uint32_t)((e - lo) >> sh);
        atomicAdd(&s.f32.bcnt[bk], 1u);
        if (MASS) atomicAdd((unsigned long long*)&s.f32.bmass[bk], (unsigned long long)fixq(wexp(value_of(e), m)));
      }
    }
    __syncthreads();
    // buckets in ascending order: thread t < NBUCKET holds bucket t (waves 0-3)
    uint32_t c = 0u;
    double v = 0.0;
    if (t < NBUCKET) {
      c = s.f32.bcnt[t];
      v = MASS ? (double)s.f32.bmass[t] : (double)c;
    }
    const double vi = wscan_f64(v);  // integers below 2^53: exact
    if (l == 63) s.red_d2[wv] = vi;
    __syncthreads();
    double before = 0.0;
#pragma unroll
    for (int k = 0; k < NBUCKET / 64; ++k) before += (k < wv) ? s.red_d2[k] : 0.0;
    const double excl = before + vi - v;
    const bool cross = t < NBUCKET && v > 0.0 && B + (excl + v) * unit > target;
    const uint64_t hc = ballot(cross);
    const uint64_t hl = ballot(t < NBUCKET && v > 0.0);
    if (l == 0) {
      s.cand[wv] = hc ? (uint32_t)(64 * wv + first_lane(hc)) : 0xffffffffu;
      s.last[wv] = hl ? (uint32_t)(64 * wv + 63 - __clzll((unsigned long long)hl)) : 0xffffffffu;
    }
    if (hc && l == first_lane(hc)) {
      s.cand_excl[wv] = excl;
      s.cand_cnt[wv] = c;
    }
    if (hl && l == 63 - __clzll((unsigned long long)hl)) {
      s.last_excl[wv] = excl;
      s.last_cnt[wv] = c;
    }
    __syncthreads();
    uint32_t bk = 0xffffffffu, lb = 0xffffffffu;
    double bex = 0.0, lex = 0.0;
    uint32_t bc = 0u, lc = 0u;
#pragma unroll
    for (int k = 0; k < NBUCKET / 64; ++k) {
      const uint32_t ck = s.cand[k];
      if (ck != 0xffffffffu && bk == 0xffffffffu) {
        bk = ck;
        bex = s.cand_excl[k];
        bc = s.cand_cnt[k];
      }
      const uint32_t lk = s.last[k];
      if (lk != 0xffffffffu) {
        lb = lk;
        lex = s.last_excl[k];
        lc = s.last_cnt[k];
      }
    }
    if (bk == 0xffffffffu) {
      bk = lb;
      bex = lex;
      bc = lc;
    }
    if (bk == 0xffffffffu) {
      // no entry with weight in the interval
      Pick p;
      p.e = ~0ull;
      p.excl = B;
      p.w = 0.0;
      return p;
    }
    B += bex * unit;
    cnt = bc;
    lo += (uint64_t)bk << sh;
    hi = min_u64(hi, lo + (((uint64_t)1 << sh) - 1u));
    if (cnt == 1u || sh == 0) break;
  }
  // the interval now holds one entry (or one value of E)
  if (t == 0) s.pick = ~0ull;
  __syncthreads();
  for (int i = l; i < sn; i += 64) {
    const uint64_t e = seg[i];
    if (e >= lo && e <= hi) s.pick = e;
  }
  __syncthreads();
  Pick p;
  p.e = s.pick;
  p.excl = B;
  p.w = MASS ? (double)fixq(wexp(value_of(p.e), m)) * FIXQ : 1.0;
  __syncthreads();
  return p;
}

// Returns false, with m set, when the row must take the bisection path (a counter wrapped
// or a window holds too many elements). `src0` streams the row once (it may keep it in
// registers); the later passes read `src`.
template <int DT, class Src0, class Src, class Div>
__device__ __forceinline__ bool sample_row32(const KArgs& a, Smem& s, Src0& src0, const Src& src, int b,
                                             const Div& dv, int kk, float p, float u, float& m_out) {
  const int V = a.vocab;
  const int l = lane_id(), wv = wave_id();
  uint64_t* const big = (uint64_t*)s.hist;  // the list, once the histogram is no longer read
  // the kept-set counts (ties kept at the cutoff, kept elements) only feed the row
  // diagnostics: without them the list passes that count them are skipped
  const bool diag = a.out_info != nullptr;

  // stream: histogram, row maximum, NaN, and sum_i exp(x_i - xmax) with the thread's
  // running maximum xmax (rescaled once per 16-byte vector)
  hist_clear(s);
  lds_barrier();
  float xmax = -INFINITY;
  double zs = 0.0;
  int nan = 0;
  src0.stream([&](int, const u4& q, int base, bool vvalid) {
    float xs[4];
    if constexpr (Src0::kVector) {
      // whole vectors are valid or not: one branch per vector, the bins of two values
      // (top 16 bits, -0 folded by x + 0) packed into one word for hist_add_pair
      div4(dv, q, xs);
      if (vvalid) {
        uint32_t bb[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) bb[e] = __float_as_uint(xs[e] + 0.0f);
        hist_add_pair(s, (bb[1] & 0xffff0000u) | (bb[0] >> 16));
        hist_add_pair(s, (bb[3] & 0xffff0000u) | (bb[2] >> 16));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) xs[e] = -INFINITY;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok = elem_valid(src0, vvalid, base + e);
        const float x = x_at<DT>(dv, q, e);
        if (ok) hist_add_one(s, bin_raw32(x));
        xs[e] = ok ? x : -INFINITY;
      }
    }
    nan |= (__builtin_isunordered(xs[0], xs[1]) || __builtin_isunordered(xs[2], xs[3])) ? 1 : 0;
    const float cm = fmaxf(fmaxf(xs[0], xs[1]), fmaxf(xs[2], xs[3]));
    const float mn = fmaxf(xmax, cm);
    const float mr = (mn > -INFINITY) ? mn : 0.0f;
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) part += __builtin_amdgcn_exp2f((xs[e] - mr) * LOG2E_F);
    zs = fma(zs, (double)__builtin_amdgcn_exp2f((xmax - mr) * LOG2E_F), (double)part);
    xmax = mn;
  });
  const float m = block_max_nan(xmax, nan, s);  // its barriers also complete the histogram
  m_out = m;
  if (m != m || !(m > -INFINITY && m < INFINITY)) {
    if (threadIdx.x == 0) write_error(a, b, m != m ? PBS_ROW_NAN : PBS_ROW_NONFINITE, m);
    return true;
  }
  {
    const double zt = (xmax > -INFINITY) ? zs * (double)__builtin_amdgcn_exp2f((xmax - m) * LOG2E_F) : 0.0;
    const double zw = wsum_f64(zt);
    if (l == 0) s.red_d2[wv] = zw;
  }
  hist_group_counts<DT>(s);
  __syncthreads();
  double z_all = 0.0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) z_all += s.red_d2[w];
  {
    uint32_t c = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) c += s.gcount[4 * l + i];
    if (wsum_u32(c) != (uint32_t)V) return false;  // a u16 counter wrapped
  }

  // lower (gmass) and upper (gmass_hi) bounds of the group masses: the non-empty groups
  // dealt round-robin to the waves, lane l bounding bins 4l .. 4l+3 of the group
  {
    uint32_t ne = 0u;
#pragma unroll
    for (int i = 0; i < 4; ++i) ne |= (s.gcount[4 * l + i] != 0u ? 1u : 0u) << i;
    if (wv == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (!((ne >> i) & 1u)) {
          s.gmass[4 * l + i] = 0.0;
          s.f32.gmass_hi[4 * l + i] = 0.0;
        }
      }
    }
    const uint32_t cnt = (uint32_t)__popc(ne);
    const uint32_t incl = wscan_u32(cnt);
    const uint32_t excl = incl - cnt;
    const uint32_t total = bcast_u32(incl, 63);
#pragma unroll 1
    for (uint32_t r = (uint32_t)wv; r < total; r += NWAVE) {
      const bool mine = r >= excl && r < incl;
      const int L = first_lane(ballot(mine));
      uint32_t bits = ne;
      for (uint32_t k = mine ? r - excl : 0u; k > 0u; --k) bits &= bits - 1u;
      const uint32_t g = bcast_u32(4u * (uint32_t)l + (uint32_t)(__ffs(bits) - 1), L);
      uint32_t n4[4];
      counts4(s, g * 256u + 4u * (uint32_t)l, n4);
      double plo = 0.0, phi = 0.0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float wl, wh;
        bin_bounds(g * 256u + 4u * (uint32_t)l + (uint32_t)k, m, wl, wh);
        plo += (double)n4[k] * (double)wl;
        phi += (double)n4[k] * (double)wh;
      }
      plo = wsum_f64(plo);
      phi = wsum_f64(phi);
      if (l == 0) {
        s.gmass[g] = plo;
        s.f32.gmass_hi[g] = phi;
      }
    }
  }
  __syncthreads();
  if (wv == 0) {
    // top-down exclusive prefixes: lane l holds groups 255-4l .. 252-4l
    uint32_t c[4];
    double w0[4], w1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c[i] = s.gcount[255 - 4 * l - i];
      w0[i] = s.gmass[255 - 4 * l - i];
      w1[i] = s.f32.gmass_hi[255 - 4 * l - i];
    }
    const uint32_t ct = c[0] + c[1] + c[2] + c[3];
    const double t0 = ((w0[0] + w0[1]) + w0[2]) + w0[3];
    const double t1 = ((w1[0] + w1[1]) + w1[2]) + w1[3];
    uint32_t rc = wscan_u32(ct) - ct;
    double r0 = wscan_f64(t0) - t0, r1 = wscan_f64(t1) - t1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s.gabove_cnt[255 - 4 * l - i] = rc;
      s.gabove_mass[255 - 4 * l - i] = r0;
      s.f32.gabove_hi[255 - 4 * l - i] = r1;
      rc += c[i];
      r0 += w0[i];
      r1 += w1[i];
    }
  }
  __syncthreads();

  RowState st = {};
  st.m = m;
  st.x_kth = -INFINITY;
  const bool cut = p < 1.0f;

  // top-k (sampling.py:15-17): K = the elements with key >= kmin; the k-th lies in bin klo
  const bool topk = kk > 0 && kk < V;
  uint32_t klo = 0u, kc = 0u, kabove = 0u;
  if (topk) {
    const int g = find_group_count(s, (uint32_t)kk);
    uint32_t ca;
    bins_count(s, (uint32_t)g, (uint32_t)kk - s.gabove_cnt[g], klo, kc, ca);
    kabove = s.gabove_cnt[g] + ca;  // elements in bins above klo
  }

  if (topk && kabove + kc <= SMALLK_CAP) {
    // Everything from the k-th element's bin up fits in one list: the whole row resolves
    // from it (two passes over the row in all).
    double a0, a1, a2;
    if (!gather_windows<DT, 1>(src, s, big, dv, m, klo, 0xffffu, 0u, 0u, 0u, 0u, a0, a1, a2)) return false;
    const Pick pk = list_pick<false>(s, big, 0ull, ~0ull, m, 0.0, (double)(kk - 1));
    if (pk.e == ~0ull) return false;
    const uint32_t kmin = key_of(pk.e);
    const uint64_t eK = e_last(kmin);
    st.x_kth = float_of_ord32(kmin);
    st.kord_lo = kmin;
    uint32_t nK, kties = 0u;
    double zq, dummy;
    list_sum<true>(s, big, 0ull, eK, m, nK, zq);
    if (diag) list_sum<false>(s, big, e_first(kmin), eK, m, kties, dummy);
    st.zk = zq * FIXQ;
    uint64_t eD = eK;  // the draw's last candidate
    if (cut) {
      const Pick pc = list_pick<true>(s, big, 0ull, eK, m, 0.0, (double)p * st.zk);
      if (pc.e == ~0ull) return false;
      const uint32_t ckey = key_of(pc.e);
      if (diag) {
        uint32_t nkept, ntie, nkeep;
        list_sum<false>(s, big, 0ull, pc.e, m, nkept, dummy);
        list_sum<false>(s, big, e_first(ckey), e_last(ckey), m, ntie, dummy);
        list_sum<false>(s, big, e_first(ckey), pc.e, m, nkeep, dummy);
        st.n_cut_tie = (int)ntie;
        st.n_cut_keep = (int)nkeep;
        st.n_kept = (int)nkept;
      }
      st.x_cut = float_of_ord32(ckey);
      st.zp = pc.excl + pc.w;
      eD = pc.e;
    } else {
      st.x_cut = st.x_kth;
      st.n_cut_tie = st.n_cut_keep = (int)kties;
      st.n_kept = (int)nK;
      st.zp = st.zk;
    }
    // the draw (sampling.py:26-27, inverse-CDF form)
    st.target = (double)u * st.zp;
    const Pick pd = list_pick<true>(s, big, 0ull, eD, m, 0.0, st.target);
    if (pd.e == ~0ull) return false;
    if (threadIdx.x == 0) write_info(a, b, index_of(pd.e), PBS_ROW_OK, st);
    return true;
  }

  // Windows. Z_K lies in [zlo, zhi]: exact (up to rounding) without top-k, bounded by the
  // bins above klo and the k-th's share of bin klo with it. The cutoff (top-p,
  // sampling.py:18-25) is the first element of K whose inclusive mass exceeds tau = p Z_K:
  // in bins [c_lo, c_hi]. Z_P, its inclusive mass, lies in (tau, tau + its weight], which
  // bounds the draw's target u Z_P (u Z_K without a cutoff): the draw lies in bins
  // [d_lo, d_hi]. Every window lies at or above klo.
  // Each pair of searches (the bounds on Z_K, the cutoff's window, the draw's window) runs
  // in waves 0 and 1 side by side, the two results handed over in LDS (s.red_d, s.red_i):
  // the same calls on the same state as in one wave, so the same results.
  double zlo = z_all, zhi = z_all;
  if (topk) {
    float wl, wh;
    bin_bounds(klo, m, wl, wh);
    if (wv == 0) {
      const double b0 = bound_above<false>(s, klo, m);
      if (l == 0) s.red_d[0] = b0;
    } else if (wv == 1) {
      const double b1 = bound_above<true>(s, klo, m);
      if (l == 0) s.red_d[1] = b1;
    }
    __syncthreads();
    zlo = s.red_d[0] + (double)(kk - (int)kabove) * (double)wl;
    zhi = s.red_d[1] + (double)kc * (double)wh;
  }
  uint32_t c_lo = 0u, c_hi = 0u;
  double t_lo, t_hi;
  if (cut) {
    const double tau_lo = (double)p * zlo * (1.0 - 1e-6), tau_hi = (double)p * zhi * (1.0 + 1e-6);
    if (wv == 0) {
      const uint32_t ob = find_bin_bound<true>(s, klo, tau_lo, m);
      if (l == 0) s.red_i[0] = (int)ob;
    } else if (wv == 1) {
      const uint32_t oa = find_bin_bound<false>(s, klo, tau_hi, m);
      if (l == 0) s.red_i[1] = (int)oa;
    }
    __syncthreads();
    const uint32_t ob = (uint32_t)s.red_i[0], oa = (uint32_t)s.red_i[1];
    c_lo = min(oa, ob);
    c_hi = max(oa, ob);
    float wl, wh;
    bin_bounds(c_hi, m, wl, wh);
    t_lo = (double)u * tau_lo * (1.0 - 1e-6);
    t_hi = (double)u * (tau_hi + (double)wh) * (1.0 + 1e-6);
  } else {
    t_lo = (double)u * zlo * (1.0 - 1e-6);
    t_hi = (double)u * zhi * (1.0 + 1e-6);
  }
  if (wv == 0) {
    const uint32_t r = find_bin_bound<true>(s, klo, t_lo, m);
    if (l == 0) s.red_i[2] = (int)r;
  } else if (wv == 1) {
    const uint32_t r = find_bin_bound<false>(s, klo, t_hi, m);
    if (l == 0) s.red_i[3] = (int)r;
  }
  __syncthreads();
  const uint32_t d_hi = (uint32_t)s.red_i[2], d_lo = (uint32_t)s.red_i[3];
  const uint32_t dlo = min(d_lo, d_hi), dhi = max(d_lo, d_hi);
  // every element above the cutoff window is in K (the window lies at or above klo)
  const uint32_t n_above_c = cut ? count_bins_ge(s, c_hi + 1u) : 0u;
  const uint32_t n_neg_inf = hist_count(s, ord32(-INFINITY) >> 16);
  // windows: the draw's, then the cutoff's and the k-th element's bin when they apply
  double above_d, above_c = 0.0, above_k = 0.0, a2;
  bool fits;
  if (cut && topk) fits = gather_windows<DT, 3>(src, s, big, dv, m, dlo, dhi, c_lo, c_hi, klo, klo, above_d, above_c, above_k);
  else if (cut) fits = gather_windows<DT, 2>(src, s, big, dv, m, dlo, dhi, c_lo, c_hi, 0u, 0u, above_d, above_c, a2);
  else if (topk) fits = gather_windows<DT, 2>(src, s, big, dv, m, dlo, dhi, klo, klo, 0u, 0u, above_d, above_k, a2);
  else fits = gather_windows<DT, 1>(src, s, big, dv, m, dlo, dhi, 0u, 0u, 0u, 0u, above_d, a2, a2);
  if (!fits) return false;
  double dummy;

  uint64_t eK = ~0ull;  // last entry of K
  double zk = z_all;
  uint32_t nk = (uint32_t)V;
  if (topk) {
    const Pick pk = list_pick<false>(s, big, e_bins_first(klo), e_bins_last(klo), m, 0.0,
                                     (double)(kk - 1 - (int)kabove));
    if (pk.e == ~0ull) return false;
    const uint32_t kmin = key_of(pk.e);
    eK = e_last(kmin);
    st.x_kth = float_of_ord32(kmin);
    st.kord_lo = kmin;
    uint32_t cnt, kties = 0u;
    double zq;
    // Z_K: the mass above bin klo, plus its entries down to the last of K
    list_sum<true>(s, big, e_bins_first(klo), eK, m, cnt, zq);
    zk = above_k + zq * FIXQ;
    nk = kabove + cnt;
    if (diag) list_sum<false>(s, big, e_first(kmin), eK, m, kties, dummy);
    st.x_cut = st.x_kth;
    st.n_cut_tie = st.n_cut_keep = (int)kties;
  } else {
    // every element is kept: the lowest "cutoff" value is -inf, with all its ties
    st.x_cut = -INFINITY;
    st.n_cut_tie = st.n_cut_keep = (int)n_neg_inf;
  }
  st.zk = zk;
  st.zp = zk;
  st.n_kept = (int)nk;

  uint64_t ec = ~0ull;  // the cutoff's entry
  if (cut) {
    const uint64_t ea = e_bins_first(c_hi);
    const Pick pc = list_pick<true>(s, big, ea, min_u64(e_bins_last(c_lo), eK), m, above_c, (double)p * zk);
    if (pc.e == ~0ull) return false;
    ec = pc.e;
    const uint32_t ckey = key_of(ec);
    if (diag) {
      uint32_t cnt, ntie, nkeep;
      list_sum<false>(s, big, ea, ec, m, cnt, dummy);
      list_sum<false>(s, big, e_first(ckey), e_last(ckey), m, ntie, dummy);
      list_sum<false>(s, big, e_first(ckey), ec, m, nkeep, dummy);
      st.n_cut_tie = (int)ntie;
      st.n_cut_keep = (int)nkeep;
      st.n_kept = (int)(n_above_c + cnt);
    }
    st.x_cut = float_of_ord32(ckey);
    st.zp = pc.excl + pc.w;
  }
  // the draw (sampling.py:26-27, inverse-CDF form): in the cutoff window, up to the
  // cutoff, when the target lies at or past the mass above that window; else in the draw
  // window
  const double t = (double)u * st.zp;
  st.target = t;
  const bool in_c = cut && t >= above_c;
  const uint64_t first = e_bins_first(in_c ? c_hi : dhi);
  const uint64_t last = min_u64(min_u64(e_bins_last(in_c ? c_lo : dlo), eK), ec);
  const Pick pd = list_pick<true>(s, big, first, last, m, in_c ? above_c : above_d, t);
  if (pd.e == ~0ull) return false;
  if (threadIdx.x == 0) write_info(a, b, index_of(pd.e), PBS_ROW_OK, st);
  return true;
}

// ---------------------------------------------------------------------------------------
// one row
// ---------------------------------------------------------------------------------------
template <int DT, class Src>
__device__ __forceinline__ void sample_row(const KArgs& a, Smem& s, Src& src, int b) {
  constexpr int EPV = DTraits<DT>::EPV;
  constexpr bool B16 = DTraits<DT>::B16;
  const size_t elt = B16 ? 2 : 4;
  // Without a row map the logits row is b (the host checked rows <= n_logit_rows): its
  // first loads go out before the row's parameters arrive, not after.
  const bool mapped = a.row_map != nullptr;
  if (!mapped) {
    src.init((const uint8_t*)a.logits + (size_t)b * (size_t)a.row_stride * elt, a.nvec, a.vocab);
    src.load();
  }
  const int64_t lrow = mapped ? (int64_t)a.row_map[b] : (int64_t)b;
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
  if (mapped) {
    src.init((const uint8_t*)a.logits + (size_t)lrow * (size_t)a.row_stride * elt, a.nvec, a.vocab);
    src.load();
  }

  if (greedy) {
    // torch.argmax (sampling.py:13): first NaN if any, else the first maximum
    float bv = -INFINITY;
    int bi = INT32_MAX;
    int nan_i = INT32_MAX;
    if constexpr (Src::kVector) {
      // per vector: its maximum, one compare with the running best and a copy of the best
      // vector, whose first element equal to the maximum is resolved at the end; a NaN is
      // only flagged, and a row holding one is scanned again for its first NaN
      bool nan = false;
      int bvec = -1;
      u4 bq = {0u, 0u, 0u, 0u};
      src.stream([&](int, const u4& q, int base, bool vvalid) {
        if (vvalid) {
          // vectors reach a thread in increasing index order: strict > keeps the first
          const float m = vec_max<DT>(q, nan);
          const bool up = m > bv;
          bv = up ? m : bv;
          bvec = up ? base : bvec;
          bq = up ? q : bq;
        }
      });
      if (bvec >= 0) {
        int e = EPV - 1;
#pragma unroll
        for (int i = EPV - 2; i >= 0; --i) e = (raw_to_float<DT>(elem_raw<DT>(bq, i)) == bv) ? i : e;
        bi = bvec + e;
      }
      if (__syncthreads_or(nan)) {
        // re-read from memory (the row's registers are dead by now): each thread's first NaN
        const uint8_t* rp = (const uint8_t*)a.logits + (size_t)lrow * (size_t)a.row_stride * elt;
        for (int i = (int)threadIdx.x; i < a.vocab; i += NT) {
          const float v = B16 ? raw_to_float<DT>(((const uint16_t*)rp)[i]) : raw_to_float<DT>(((const uint32_t*)rp)[i]);
          if (v != v) {
            nan_i = i;
            break;
          }
        }
      }
    } else {
      src.stream([&](int, const u4& q, int base, bool vvalid) {
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
    }
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
  Divider dv;
  dv.init(T);
  if constexpr (Src::kVector) {
    // Passes after the first re-read the row (from cache when it was just read), so no
    // register copy of it stays live across them. 16-bit rows get here only when a
    // histogram counter wrapped (one value more than 65535 times); their first pass
    // re-reads the row as well.
    MemRow<DT> mem;
    mem.init((const uint8_t*)a.logits + (size_t)lrow * (size_t)a.row_stride * elt, a.nvec, a.vocab);
    float m;
    if constexpr (B16) {
      if (sample_row16<DT>(a, s, src, b, T, kk, p, u)) return;
      m = bis_max<DT>(mem, s, dv, false);
    } else {
      if (T == 1.0f) {
        if (sample_row32<DT>(a, s, src, mem, b, UnitDivider{}, kk, p, u, m)) return;
      } else {
        if (sample_row32<DT>(a, s, src, mem, b, dv, kk, p, u, m)) return;
      }
    }
    sample_row_bisect<DT>(a, s, mem, b, m, dv, kk, p, u);
  } else {
    float m;
    if constexpr (B16) {
      if (sample_row16<DT>(a, s, src, b, T, kk, p, u)) return;
      m = bis_max<DT>(src, s, dv, false);
    } else {
      if (T == 1.0f) {
        if (sample_row32<DT>(a, s, src, src, b, UnitDivider{}, kk, p, u, m)) return;
      } else {
        if (sample_row32<DT>(a, s, src, src, b, dv, kk, p, u, m)) return;
      }
    }
    sample_row_bisect<DT>(a, s, src, b, m, dv, kk, p, u);
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

template <int DT>
int launch_dt(const KArgs& a, int64_t rows, bool vec, hipStream_t stream) {
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
    else if (nch <= 24) hipLaunchKernelGGL((k_sample<DT, 24>), grid, block, 0, stream, a);
    else if (nch <= 32) hipLaunchKernelGGL((k_sample<DT, 32>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((k_sample<DT, 0>), grid, block, 0, stream, a);
  }
  if (a.out_probs || a.out_kept) {
    if (vec) hipLaunchKernelGGL((k_debug<DT, true>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((k_debug<DT, false>), grid, block, 0, stream, a);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return report_errorf(PBS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  return PBS_OK;
}

// ---------------------------------------------------------------------------------------
// All-greedy steps: torch.argmax of every row (sampling.py:12-13), first NaN if any, else
// the first maximum. Pure streaming: no histogram, so the workgroups are small (256
// threads, a few dozen bytes of LDS) and several share a CU. Each thread keeps eight
// 16-byte loads in flight (two groups of four, the next group issued before the current
// one is read) and does per-vector work only: the vector's maximum, one compare with the
// running best, and a copy of the best vector, whose first element equal to the maximum is
// resolved once at the end. A NaN is only flagged on the way (one unordered compare per
// pair); a row that holds one is scanned again for its first NaN.
// ---------------------------------------------------------------------------------------
constexpr int NT_AM = 256;
constexpr int G_AM = 4;


template <int DT, bool VEC>
__global__ __launch_bounds__(NT_AM) void k_argmax(KArgs a) {
  constexpr int EPV = DTraits<DT>::EPV;
  constexpr size_t ELT = DTraits<DT>::B16 ? 2 : 4;
  __shared__ float red_v[NT_AM / 64];
  __shared__ int red_i[NT_AM / 64];
  __shared__ int red_nan[NT_AM / 64];
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  const int64_t lrow = a.row_map ? (int64_t)a.row_map[b] : (int64_t)b;
  if (!(lrow >= 0 && lrow < a.n_logit_rows)) {
    if (t == 0) {
      a.out_token[b] = 0;
      a.out_status[b] = PBS_ROW_BAD_PARAM;
    }
    return;
  }
  const uint8_t* row = (const uint8_t*)a.logits + (size_t)lrow * (size_t)a.row_stride * ELT;
  auto elem = [&](int i) {
    return DTraits<DT>::B16 ? raw_to_float<DT>(((const uint16_t*)row)[i]) : raw_to_float<DT>(((const uint32_t*)row)[i]);
  };
  // the thread's candidate: its largest value (NaN aside) and the lowest index holding it;
  // INT32_MAX when every value it saw was -inf or NaN
  float bv = -INFINITY;
  int bi = INT32_MAX;
  bool nan = false;
  if constexpr (VEC) {
    const int nvec = a.nvec;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)row, (short)0, nvec * 16, 0x00020000);
    // the whole offset goes in the VGPR operand, which the buffer's range check covers
    auto ld = [&](int j) {
      return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)(j * NT_AM + t) * 16u, 0, 2));
    };
    const int nch = (nvec + NT_AM - 1) / NT_AM;
    int bvec = -1;
    u4 bq = {0u, 0u, 0u, 0u};
    u4 cur[G_AM], nxt[G_AM];
#pragma unroll
    for (int k = 0; k < G_AM; ++k) cur[k] = ld(k);
    for (int j0 = 0; j0 < nch; j0 += G_AM) {
#pragma unroll
      for (int k = 0; k < G_AM; ++k) nxt[k] = ld(j0 + G_AM + k);  // past the row: zeros, never read
#pragma unroll
      for (int k = 0; k < G_AM; ++k) {
        const int v = (j0 + k) * NT_AM + t;
        if (v < nvec) {
          // vectors reach a thread in increasing index order: strict > keeps the first
          const float m = vec_max<DT>(cur[k], nan);
          const bool up = m > bv;
          bv = up ? m : bv;
          bvec = up ? v : bvec;
          bq = up ? cur[k] : bq;
        }
      }
#pragma unroll
      for (int k = 0; k < G_AM; ++k) cur[k] = nxt[k];
    }
    if (bvec >= 0) {
      int e = EPV - 1;
#pragma unroll
      for (int i = EPV - 2; i >= 0; --i) e = (raw_to_float<DT>(elem_raw<DT>(bq, i)) == bv) ? i : e;
      bi = bvec * EPV + e;
    }
  } else {
    for (int i = t; i < a.vocab; i += NT_AM) {
      const float v = elem(i);
      nan |= (v != v);
      const bool up = v > bv;
      bv = up ? v : bv;
      bi = up ? i : bi;
    }
  }
  // block reduction: the largest value, lowest index on ties; the NaN flags ride the same
  // barrier
  const int w = t >> 6;
  {
    const float wm = wmax_f32(bv);
    const int wi = wmin_i32(bv == wm ? bi : INT32_MAX);
    const bool wnan = __any(nan);
    if ((t & 63) == 0) {
      red_v[w] = wm;
      red_i[w] = wi;
      red_nan[w] = wnan ? 1 : 0;
    }
  }
  __syncthreads();
  bool any_nan = false;
#pragma unroll
  for (int k = 0; k < NT_AM / 64; ++k) any_nan |= red_nan[k] != 0;
  if (any_nan) {
    // a row holding a NaN: its first NaN, found by a second pass, and the reduction again
    int ni = INT32_MAX;
    for (int i = t; i < a.vocab; i += NT_AM) {
      if (elem(i) != elem(i)) {
        ni = i;
        break;
      }
    }
    bv = ni != INT32_MAX ? INFINITY : -INFINITY;
    bi = ni;
    const float wm = wmax_f32(bv);
    const int wi = wmin_i32(bv == wm ? bi : INT32_MAX);
    __syncthreads();  // every thread has read the flags before the table is rewritten
    if ((t & 63) == 0) {
      red_v[w] = wm;
      red_i[w] = wi;
    }
    __syncthreads();
  }
  if (t == 0) {
    float v = red_v[0];
    int i = red_i[0];
#pragma unroll
    for (int k = 1; k < NT_AM / 64; ++k) {
      if (red_v[k] > v || (red_v[k] == v && red_i[k] < i)) {
        v = red_v[k];
        i = red_i[k];
      }
    }
    // every value -inf (no candidate anywhere): index 0, as torch.argmax gives
    a.out_token[b] = i == INT32_MAX ? 0 : i;
    a.out_status[b] = PBS_ROW_OK;
  }
}

template <int DT>
int launch_argmax(const KArgs& a, int64_t rows, bool vec, hipStream_t stream) {
  const dim3 grid((unsigned)rows), block(NT_AM);
  if (vec) hipLaunchKernelGGL((k_argmax<DT, true>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((k_argmax<DT, false>), grid, block, 0, stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return report_errorf(PBS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  return PBS_OK;
}

}  // namespace pbs

#if defined(PBS_TU_DTYPE)
template int pbs::launch_dt<PBS_TU_DTYPE>(const pbs::KArgs&, int64_t, bool, hipStream_t);
template int pbs::launch_argmax<PBS_TU_DTYPE>(const pbs::KArgs&, int64_t, bool, hipStream_t);
#endif
#endif  // PBS_WANT_KERNELS

#if PBS_WANT_ABI
namespace pbs {

// ---------------------------------------------------------------------------------------
// Finish reasons after a step's tokens (pagedbatch/engine.py:173-182): one thread per
// sequence, reading the token the sampler wrote and the sequence's stop rule.
// ---------------------------------------------------------------------------------------
struct FinishArgs {
  const int32_t* tokens;
  int64_t rows;
  int32_t eos;  // -1: the model has none
  const uint8_t* ignore_eos;
  const int32_t* stop_offsets;
  const int32_t* stop_ids;
  const int32_t* num_output;
  const int32_t* max_tokens;
  const int32_t* num_tokens;
  int32_t max_model_len;
  int32_t* out_reason;
};

__global__ __launch_bounds__(256) void k_finish(FinishArgs f) {
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (b >= f.rows) return;
  const int32_t tok = f.tokens[b];
  int32_t reason = PBS_FINISH_NONE;
  if (!f.ignore_eos[b]) {
    bool stop = f.eos >= 0 && tok == f.eos;
    for (int32_t i = f.stop_offsets[b]; i < f.stop_offsets[b + 1] && !stop; ++i) stop = f.stop_ids[i] == tok;
    if (stop) reason = PBS_FINISH_STOP;
  }
  if (reason == PBS_FINISH_NONE && (f.num_output[b] >= f.max_tokens[b] || f.num_tokens[b] >= f.max_model_len))
    reason = PBS_FINISH_LENGTH;
  f.out_reason[b] = reason;
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
    case PBS_DTYPE_F32: return pbs::launch_dt<PBS_DTYPE_F32>(a, rows, vec, st);
    case PBS_DTYPE_F16: return pbs::launch_dt<PBS_DTYPE_F16>(a, rows, vec, st);
    default: return pbs::launch_dt<PBS_DTYPE_BF16>(a, rows, vec, st);
  }
}

}  // namespace

namespace pbs {
int report_error(int code, const char* msg) { return fail(code, "%s", msg); }
int report_errorf(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}
}  // namespace pbs

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

int pbs_argmax(const void* logits, int dtype, int64_t n_logit_rows, int64_t rows, int64_t vocab,
               int64_t row_stride, const int32_t* row_map, int32_t* out_token, int32_t* out_status,
               void* stream) {
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
  if (!logits || !out_token || !out_status) return fail(PBS_ERR_INVALID_ARGUMENT, "null pointer argument");
  if (!row_map && n_logit_rows < rows)
    return fail(PBS_ERR_INVALID_ARGUMENT, "rows %lld > n_logit_rows %lld without row_map", (long long)rows,
                (long long)n_logit_rows);
  const int elt = dtype == PBS_DTYPE_F32 ? 4 : 2;
  const int epv = 16 / elt;
  const bool vec = ((uintptr_t)logits % 16 == 0) && ((row_stride * elt) % 16 == 0) && (vocab % epv == 0);
  pbs::KArgs a = {};
  a.logits = logits;
  a.n_logit_rows = n_logit_rows;
  a.row_stride = row_stride;
  a.vocab = (int)vocab;
  a.nvec = (int)((vocab + epv - 1) / epv);
  a.row_map = row_map;
  a.out_token = out_token;
  a.out_status = out_status;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case PBS_DTYPE_F32: return pbs::launch_argmax<PBS_DTYPE_F32>(a, rows, vec, st);
    case PBS_DTYPE_F16: return pbs::launch_argmax<PBS_DTYPE_F16>(a, rows, vec, st);
    default: return pbs::launch_argmax<PBS_DTYPE_BF16>(a, rows, vec, st);
  }
}

int pbs_finish_reasons(const int32_t* tokens, int64_t rows, int32_t eos_token_id, const uint8_t* ignore_eos,
                       const int32_t* stop_offsets, const int32_t* stop_ids, const int32_t* num_output,
                       const int32_t* max_tokens, const int32_t* num_tokens, int32_t max_model_len,
                       int32_t* out_reason, void* stream) {
  if (rows < 0) return fail(PBS_ERR_INVALID_ARGUMENT, "rows is negative (%lld)", (long long)rows);
  if (rows > ((int64_t)1 << 31)) return fail(PBS_ERR_INVALID_ARGUMENT, "rows (%lld) above 2^31", (long long)rows);
  if (rows == 0) return PBS_OK;
  if (!tokens || !ignore_eos || !stop_offsets || !num_output || !max_tokens || !num_tokens || !out_reason)
    return fail(PBS_ERR_INVALID_ARGUMENT, "null device pointer among the required arguments");
  if (eos_token_id < -1) return fail(PBS_ERR_INVALID_ARGUMENT, "eos_token_id below -1 (%d)", eos_token_id);
  pbs::FinishArgs f;
  f.tokens = tokens;
  f.rows = rows;
  f.eos = eos_token_id;
  f.ignore_eos = ignore_eos;
  f.stop_offsets = stop_offsets;
  f.stop_ids = stop_ids;
  f.num_output = num_output;
  f.max_tokens = max_tokens;
  f.num_tokens = num_tokens;
  f.max_model_len = max_model_len;
  f.out_reason = out_reason;
  hipLaunchKernelGGL(pbs::k_finish, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, (hipStream_t)stream, f);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PBS_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  return PBS_OK;
}

}  // extern "C"

#endif  // PBS_WANT_ABI
