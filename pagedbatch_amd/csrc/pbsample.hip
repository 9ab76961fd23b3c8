// pbsample.hip -- gfx950 (MI355X) token sampler: greedy / temperature / top-k / top-p / draw.
//
// Replaces the per-row torch op chain of pagedbatch/sampling.py:10-27 (called once per
// row from pagedbatch/engine.py:133-139) with one launch per engine step: one 1024-thread
// workgroup per output row, the row held in VGPRs after a single coalesced 16-byte-load
// pass over HBM (or re-streamed from memory when it does not fit), per-row selection
// state in LDS.
//
// Selection is done on order-preserving integer keys ("ords") of the values:
//   16-bit logits (bf16 / fp16): every distinct value has its own ord, so a 64K-bin
//     count histogram in LDS (packed u16 counters) is an exact summary of the row. The
//     softmax weight exp(x - max) depends only on the value, so masses per value are
//     count * weight, computed once per distinct value in fp64. Top-k threshold, top-p
//     cutoff and the inverse-CDF draw are all prefix-sum searches over that histogram,
//     in descending value order; only the final "which of the tied tokens" step looks
//     at element indices again.
//   fp32 logits: x = fp32(v)/T is computed per element (exact division) and the same
//     searches run on 32-bit ords of x (see the fp32 section below).
//
// The sorted order everywhere is (scaled value descending, index ascending): the order
// pagedbatch's top-p sort establishes (sampling.py:19), with ties broken by index.

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>
#include <string.h>

#include "pbsample.h"

namespace pbs {

constexpr int NT = 1024;            // threads per workgroup: one workgroup per row
constexpr int NWAVE = NT / 64;      // wave64
constexpr int HIST_WORDS = 32768;   // 64K packed u16 counters = 128 KB of LDS
constexpr int NGROUP = 256;         // histogram groups of 256 bins (high byte of a 16-bit ord)
constexpr int CAND_CAP = HIST_WORDS / 2;  // fp32 candidates (8 B each) that fit in the histogram area

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

template <class T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <class T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
  return v;
}

// inclusive prefix sum over the 64 lanes in lane order
template <class T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  const int l = lane_id();
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    T n = __shfl_up(v, o);
    if (l >= o) v += n;
  }
  return v;
}

// ---------------------------------------------------------------------------------------
// element types
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
// ord of -inf: ords below it are negative NaNs
template <int DT>
__device__ __forceinline__ uint32_t ord16_neg_inf() {
  return DT == PBS_DTYPE_BF16 ? ord16(0xff80u) : ord16(0xfc00u);
}

// x = RN(a / T), the IEEE single-precision quotient of sampling.py:14.
// With r = RN(1/T): q0 = RN(a*r) is within an ulp of a/T, the FMA residual a - q0*T is
// exact, and q1 = RN(q0 + res*r) is the correctly rounded quotient (Markstein's
// theorem); the second correction makes the "within an ulp" premise certain. The
// argument must keep every intermediate normal: zero, inf and NaN divide exactly by
// multiplication, subnormal inputs and results near the under/overflow threshold take
// the full division sequence.
struct Divider {
  float T, r;
  int elo, ehi;  // biased exponents of a for which the FMA sequence is safe
  __device__ void init(float T_) {
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
  int nvec;            // 16-byte vectors per row (vector sources)
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
  int token;
  float m;             // largest scaled logit
  float x_kth;
  float x_cut;
  uint32_t kord_lo;    // top-k set = ords >= kord_lo
  uint32_t cut_lo;     // ords in [cut_lo, cut_hi] are the cutoff tie group (n_cut_keep kept)
  uint32_t cut_hi;     // ords above cut_hi are kept whole
  int n_cut_tie;
  int n_cut_keep;
  int n_kept;
  uint32_t sel_lo, sel_hi;
  int sel_jstar;
  int sel_rank;
  int sel_index;
  double zk, zp, target;
};

struct __align__(16) Smem {
  uint32_t hist[HIST_WORDS];  // 16-bit rows: packed u16 counts per ord; reused by index selection
  uint32_t gcount[NGROUP];
  double gmass[NGROUP];
  double red_d[NWAVE];
  float red_f[NWAVE];
  int red_i[2 * NWAVE];
  int red_i2[NWAVE];
  RowState st;
};

// ---------------------------------------------------------------------------------------
// block reductions (1024 threads, 16 waves)
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ float block_max_f(float v, Smem& s) {
  v = wave_max(v);
  if (lane_id() == 0) s.red_f[wave_id()] = v;
  __syncthreads();
  float r = s.red_f[0];
#pragma unroll
  for (int w = 1; w < NWAVE; ++w) r = fmaxf(r, s.red_f[w]);
  __syncthreads();
  return r;
}

__device__ __forceinline__ int block_or_i(int v, Smem& s) {
  v = wave_max(v);
  if (lane_id() == 0) s.red_i[wave_id()] = v;
  __syncthreads();
  int r = 0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) r |= s.red_i[w];
  __syncthreads();
  return r;
}

__device__ __forceinline__ int block_min_i(int v, Smem& s) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
  if (lane_id() == 0) s.red_i[wave_id()] = v;
  __syncthreads();
  int r = s.red_i[0];
#pragma unroll
  for (int w = 1; w < NWAVE; ++w) r = min(r, s.red_i[w]);
  __syncthreads();
  return r;
}

// argmax with the lowest-index tie rule; (val, idx) pairs, NaN never enters
__device__ __forceinline__ void block_argmax(float& bv, int& bi, Smem& s) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane_id() == 0) {
    s.red_f[wave_id()] = bv;
    s.red_i[wave_id()] = bi;
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
  const int incl = wave_incl_scan(v);
  if (lane_id() == 63) s.red_i2[wave_id()] = incl;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    const int x = s.red_i2[w];
    before += (w < wave_id()) ? x : 0;
    tot += x;
  }
  __syncthreads();
  total = tot;
  return before + incl - v;
}

// ---------------------------------------------------------------------------------------
// row sources: where chunk j of the row comes from
//   RegRow<NCH>: all NCH 16-byte vectors per thread loaded once into VGPRs (one HBM pass)
//   MemRow:      chunks re-read from memory on every pass (rows too large for the VGPRs)
//   ScalarRow:   like MemRow but element loads, for rows that are not 16-byte aligned or
//                whose vocab is not a multiple of the vector width
// Element (j, t, e) is logits index (j*NT + t)*EPV + e.
// ---------------------------------------------------------------------------------------
template <int DT, int NCH>
struct RegRow {
  static constexpr int EPV = DTraits<DT>::EPV;
  u4 r[NCH];
  const u4* row;
  int nvec;
  int vocab;
  __device__ void init(const void* base, int nvec_, int vocab_) {
    row = (const u4*)base;
    nvec = nvec_;
    vocab = vocab_;
  }
  __device__ __forceinline__ void load() {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int v = j * NT + (int)threadIdx.x;
      r[j] = __builtin_nontemporal_load(row + (v < nvec ? v : nvec - 1));
    }
  }
  // f(j, q, base_index, valid) with q the 16-byte vector and base_index its first element
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
  static constexpr bool kStore = true;
  static constexpr bool kVector = true;
};

template <int DT>
struct MemRow {
  static constexpr int EPV = DTraits<DT>::EPV;
  const u4* row;
  int nvec;
  int vocab;
  __device__ void init(const void* base, int nvec_, int vocab_) {
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
  static constexpr bool kStore = false;
  static constexpr bool kVector = true;
};

template <int DT>
struct ScalarRow {
  static constexpr int EPV = DTraits<DT>::EPV;
  const uint8_t* row;
  int nvec;  // ceil(vocab / EPV)
  int vocab;
  __device__ void init(const void* base, int nvec_, int vocab_) {
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
  static constexpr bool kStore = false;
  static constexpr bool kVector = false;
};

// element validity inside a vector: vector sources cover whole vectors only
template <class Src>
__device__ __forceinline__ bool elem_valid(const Src& src, bool vvalid, int idx) {
  if constexpr (Src::kVector) {
    return vvalid;
  } else {
    return idx < src.vocab;
  }
}

// ---------------------------------------------------------------------------------------
// 16-bit rows: searches over the LDS histogram
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t hist_count(const Smem& s, uint32_t o) {
  const uint32_t w = s.hist[o >> 1];
  return (o & 1u) ? (w >> 16) : (w & 0xffffu);
}

// softmax weight of one distinct 16-bit value relative to the row maximum m, in fp64 from
// the exact fp32 scaled value (pagedbatch takes softmax of the fp32 scaled row, sampling.py:26)
template <int DT>
__device__ __forceinline__ float scaled16(uint32_t o, float T) {
  return raw_to_float<DT>(raw_of_ord16(o)) / T;
}
template <int DT>
__device__ __forceinline__ double weight16(uint32_t o, float T, float m) {
  return exp((double)scaled16<DT>(o, T) - (double)m);
}

// The histogram restricted to ords >= lo. Group glo = lo >> 8 is partial; its restricted
// count and mass are carried here, the other groups come from the per-group summaries.
struct View16 {
  uint32_t lo, glo, cnt_glo;
  double mass_glo;
};

// Whole-wave helpers below: every lane calls them and every lane gets the result.
// Lane l owns positions 4l..4l+3 of a 256-long descending sequence (groups or bins).

template <int DT>
__device__ View16 make_view(const Smem& s, uint32_t lo, float T, float m) {
  View16 v;
  v.lo = lo;
  v.glo = lo >> 8;
  const int l = lane_id();
  uint32_t c = 0;
  double ms = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t o = v.glo * 256u + (uint32_t)(4 * l + i);
    if (o >= lo) {
      const uint32_t n = hist_count(s, o);
      c += n;
      if (n) ms += (double)n * weight16<DT>(o, T, m);
    }
  }
  v.cnt_glo = wave_sum(c);
  v.mass_glo = wave_sum(ms);
  return v;
}

__device__ __forceinline__ uint32_t view_gcount(const Smem& s, const View16& v, uint32_t g) {
  return g < v.glo ? 0u : (g == v.glo ? v.cnt_glo : s.gcount[g]);
}
__device__ __forceinline__ double view_gmass(const Smem& s, const View16& v, uint32_t g) {
  return g < v.glo ? 0.0 : (g == v.glo ? v.mass_glo : s.gmass[g]);
}

__device__ uint32_t view_total_count(const Smem& s, const View16& v) {
  uint32_t c = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) c += view_gcount(s, v, (uint32_t)(4 * lane_id() + i));
  return wave_sum(c);
}
__device__ double view_total_mass(const Smem& s, const View16& v) {
  double c = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i) c += view_gmass(s, v, (uint32_t)(4 * lane_id() + i));
  return wave_sum(c);
}

// count / mass of ords >= t inside the view
__device__ uint32_t view_count_ge(const Smem& s, const View16& v, uint32_t t) {
  t = max(t, v.lo);
  if (t > 0xffffu) return 0u;
  const uint32_t g0 = t >> 8;
  const int l = lane_id();
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t g = (uint32_t)(4 * l + i);
    if (g > g0) acc += view_gcount(s, v, g);
    const uint32_t o = g0 * 256u + g;  // bins of the partial group, 4 per lane
    if (o >= t) acc += hist_count(s, o);
  }
  return wave_sum(acc);
}
template <int DT>
__device__ double view_mass_ge(const Smem& s, const View16& v, uint32_t t, float T, float m) {
  t = max(t, v.lo);
  if (t > 0xffffu) return 0.0;
  const uint32_t g0 = t >> 8;
  const int l = lane_id();
  double acc = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t g = (uint32_t)(4 * l + i);
    if (g > g0) acc += view_gmass(s, v, g);
    const uint32_t o = g0 * 256u + g;
    if (o >= t) {
      const uint32_t n = hist_count(s, o);
      if (n) acc += (double)n * weight16<DT>(o, T, m);
    }
  }
  return wave_sum(acc);
}

// Descending search over groups: first group whose inclusive prefix count reaches `need`.
// Returns the group and the count strictly above it, or -1 if the view holds fewer.
__device__ int find_group_count(const Smem& s, const View16& v, uint32_t need, uint32_t& above) {
  const int l = lane_id();
  uint32_t c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = view_gcount(s, v, 255u - (uint32_t)(4 * l + i));
  const uint32_t tot = c[0] + c[1] + c[2] + c[3];
  const uint32_t incl = wave_incl_scan(tot);
  const uint64_t hit = __ballot(incl >= need);
  if (hit == 0) return -1;
  const int L = __ffsll((unsigned long long)hit) - 1;
  uint32_t run = __shfl(incl - tot, L);
  int found = -1;
  uint32_t ab = 0;
  if (l == L) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (found < 0 && run + c[i] >= need) {
        found = 255 - (4 * l + i);
        ab = run;
      }
      run += c[i];
    }
  }
  above = __shfl(ab, L);
  return __shfl(found, L);
}

// Descending search over the bins of group g (ords >= v.lo): first ord whose inclusive
// prefix count (starting from 0 at the top of the group) reaches `need`.
__device__ int find_bin_count(const Smem& s, const View16& v, uint32_t g, uint32_t need, uint32_t& above) {
  const int l = lane_id();
  uint32_t c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t o = g * 256u + 255u - (uint32_t)(4 * l + i);
    c[i] = (o >= v.lo) ? hist_count(s, o) : 0u;
  }
  const uint32_t tot = c[0] + c[1] + c[2] + c[3];
  const uint32_t incl = wave_incl_scan(tot);
  const uint64_t hit = __ballot(incl >= need);
  if (hit == 0) return -1;
  const int L = __ffsll((unsigned long long)hit) - 1;
  uint32_t run = __shfl(incl - tot, L);
  int found = -1;
  uint32_t ab = 0;
  if (l == L) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (found < 0 && run + c[i] >= need) {
        found = (int)(g * 256u + 255u - (uint32_t)(4 * l + i));
        ab = run;
      }
      run += c[i];
    }
  }
  above = __shfl(ab, L);
  return __shfl(found, L);
}

// Descending search over groups: first group whose inclusive prefix mass exceeds target.
__device__ int find_group_mass(const Smem& s, const View16& v, double target, double& above) {
  const int l = lane_id();
  double c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = view_gmass(s, v, 255u - (uint32_t)(4 * l + i));
  const double tot = c[0] + c[1] + c[2] + c[3];
  const double incl = wave_incl_scan(tot);
  double excl = __shfl_up(incl, 1);
  if (l == 0) excl = 0.0;
  const uint64_t hit = __ballot(incl > target);
  if (hit == 0) return -1;
  const int L = __ffsll((unsigned long long)hit) - 1;
  double run = __shfl(excl, L);
  int found = -1;
  double ab = 0.0;
  if (l == L) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (found < 0 && run + c[i] > target) {
        found = 255 - (4 * l + i);
        ab = run;
      }
      run += c[i];
    }
  }
  above = __shfl(ab, L);
  return __shfl(found, L);
}

// Descending search over the bins of group g (ords >= v.lo), the mass above the group
// being `base`: first ord whose inclusive cumulative exceeds target. If rounding keeps the
// cumulative at or below the target through the whole group, the group's lowest non-empty
// ord is returned. `above` gets the cumulative strictly above the returned ord.
template <int DT>
__device__ int find_bin_mass(const Smem& s, const View16& v, uint32_t g, double base, double target,
                             float T, float m, double& above) {
  const int l = lane_id();
  double c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t o = g * 256u + 255u - (uint32_t)(4 * l + i);
    const uint32_t n = (o >= v.lo) ? hist_count(s, o) : 0u;
    c[i] = n ? (double)n * weight16<DT>(o, T, m) : 0.0;
  }
  const double tot = c[0] + c[1] + c[2] + c[3];
  const double incl = wave_incl_scan(tot);
  double excl = __shfl_up(incl, 1);
  if (l == 0) excl = 0.0;
  uint64_t hit = __ballot(base + incl > target);
  bool last_resort = false;
  int L;
  if (hit == 0) {
    hit = __ballot(tot > 0.0);
    if (hit == 0) return -1;
    L = 63 - __clzll((unsigned long long)hit);
    last_resort = true;
  } else {
    L = __ffsll((unsigned long long)hit) - 1;
  }
  double run = base + __shfl(excl, L);
  int found = -1;
  double ab = 0.0;
  if (l == L) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool take = last_resort ? (c[i] > 0.0) : (found < 0 && run + c[i] > target);
      if (take) {
        found = (int)(g * 256u + 255u - (uint32_t)(4 * l + i));
        ab = run;
      }
      run += c[i];
    }
  }
  above = __shfl(ab, L);
  return __shfl(found, L);
}

// lowest non-empty ord of a view holding n >= 1 elements
__device__ int lowest_ord(const Smem& s, const View16& v, uint32_t n) {
  uint32_t ab = 0, ab2 = 0;
  const int g = find_group_count(s, v, n, ab);
  return find_bin_count(s, v, (uint32_t)g, n - ab, ab2);
}

// Ords whose scaled value equals that of ord o. Distinct 16-bit values only meet after the
// division by T at the under/overflow ends; the map is monotone, so binary search.
template <int DT>
__device__ void tie_range16(uint32_t o, float T, uint32_t ord_min, uint32_t ord_max, uint32_t& lo,
                            uint32_t& hi) {
  const float x = scaled16<DT>(o, T);
  uint32_t a = ord_min, b = o;
  while (a < b) {
    const uint32_t mid = a + (b - a) / 2;
    if (scaled16<DT>(mid, T) >= x) b = mid; else a = mid + 1;
  }
  lo = a;
  a = o;
  b = ord_max;
  while (a < b) {
    const uint32_t mid = a + (b - a + 1) / 2;
    if (scaled16<DT>(mid, T) <= x) a = mid; else b = mid - 1;
  }
  hi = a;
}

// ---------------------------------------------------------------------------------------
// index selection: the rank-th (0-based, ascending index) element whose raw bits satisfy
// `match`. Every thread calls it and gets the index, or -1 if there are fewer matches.
// Chunk j of the row covers indices [j*NT*EPV, (j+1)*NT*EPV), so the chunk holding the
// answer is found from per-chunk counts and the thread from a scan inside that chunk.
// Uses s.hist as the per-chunk counters.
// ---------------------------------------------------------------------------------------
template <int DT, class Src, class M>
__device__ int select_index(const Src& src, Smem& s, M&& match, int rank) {
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
      const int incl = wave_incl_scan(c);
      const uint64_t hit = __ballot(run + incl > rank);
      if (hit) {
        const int L = __ffsll((unsigned long long)hit) - 1;
        jstar = j0 + L;
        rr = rank - (run + __shfl(incl - c, L));
        break;
      }
      run += __shfl(incl, 63);
    }
    if (lane_id() == 0) {
      s.st.sel_jstar = jstar;
      s.st.sel_rank = rr;
      s.st.sel_index = -1;
    }
  }
  __syncthreads();
  const int jstar = s.st.sel_jstar;
  if (jstar < 0) return -1;
  const int rr = s.st.sel_rank;
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
        if (k == 0) s.st.sel_index = my_idx[e];
        --k;
      }
    }
  }
  __syncthreads();
  const int r = s.st.sel_index;
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
// 16-bit stochastic row
// ---------------------------------------------------------------------------------------
template <int DT, class Src>
__device__ void sample_row16(const KArgs& a, Smem& s, Src& src, int b, float T, int kk, float p, float u) {
  constexpr int EPV = DTraits<DT>::EPV;
  const int V = a.vocab;

  // stream: histogram of ords, row max, NaN flag. The histogram is cleared while the
  // row's loads are in flight; only LDS is ordered by the barrier.
  {
    u4* h4 = (u4*)s.hist;
    for (int i = threadIdx.x; i < HIST_WORDS / 4; i += NT) h4[i] = (u4){0u, 0u, 0u, 0u};
  }
  lds_barrier();
  float vmax = -INFINITY;
  int nan = 0;
  src.for_each([&](int, const u4& q, int base, bool vvalid) {
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
      const uint32_t raw = elem_raw<DT>(q, e);
      if (elem_valid(src, vvalid, base + e)) {
        const float v = raw_to_float<DT>(raw);
        vmax = fmaxf(vmax, v);
        nan |= (v != v) ? 1 : 0;
        const uint32_t o = ord16(raw);
        __hip_atomic_fetch_add(&s.hist[o >> 1], 1u << ((o & 1u) << 4), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
  });
  nan = block_or_i(nan, s);
  vmax = block_max_f(vmax, s);
  const float m = vmax / T;
  if (nan || !(m > -INFINITY && m < INFINITY)) {
    if (threadIdx.x == 0) write_error(a, b, nan ? PBS_ROW_NAN : PBS_ROW_NONFINITE, m);
    return;
  }

  // group summaries: count and fp64 mass of each group of 256 ords
  for (int g = wave_id(); g < NGROUP; g += NWAVE) {
    const int l = lane_id();
    uint32_t n[4];
    uint32_t cnt = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      n[i] = hist_count(s, (uint32_t)(g * 256 + 4 * l + i));
      cnt += n[i];
    }
    cnt = wave_sum(cnt);
    double ms = 0.0;
    if (cnt) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n[i]) ms += (double)n[i] * weight16<DT>((uint32_t)(g * 256 + 4 * l + i), T, m);
      ms = wave_sum(ms);
    }
    if (l == 0) {
      s.gcount[g] = cnt;
      s.gmass[g] = ms;
    }
  }
  __syncthreads();

  // targets, resolved by wave 0
  if (wave_id() == 0) {
    const uint32_t ord_min = ord16_neg_inf<DT>();
    const uint32_t ord_max = ord16(DT == PBS_DTYPE_BF16 ? 0x7f80u : 0x7c00u);
    RowState st = {};
    st.status = PBS_ROW_OK;
    st.m = m;
    st.x_kth = -INFINITY;
    const View16 vall = make_view<DT>(s, 0u, T, m);
    // the u16 counters wrap only if one value occurs more than 65535 times
    if (view_total_count(s, vall) != (uint32_t)V) st.status = -1;

    // top-k (sampling.py:15-17): K = ords >= kord_lo
    uint32_t kord_lo = 0u;
    if (st.status == PBS_ROW_OK && kk > 0 && kk < V) {
      uint32_t ab = 0, ab2 = 0;
      const int g = find_group_count(s, vall, (uint32_t)kk, ab);
      const int o = find_bin_count(s, vall, (uint32_t)g, (uint32_t)kk - ab, ab2);
      uint32_t lo, hi;
      tie_range16<DT>((uint32_t)o, T, ord_min, ord_max, lo, hi);
      kord_lo = lo;
      st.x_kth = scaled16<DT>((uint32_t)o, T);
    }
    st.kord_lo = kord_lo;
    const View16 vk = make_view<DT>(s, kord_lo, T, m);
    const double zk = view_total_mass(s, vk);
    const uint32_t nk = view_total_count(s, vk);
    st.zk = zk;

    // top-p (sampling.py:18-25): the shortest prefix (value desc, index asc) whose
    // exclusive mass is <= p*Z; inside the cutoff tie group the lowest indices survive
    int o_cut = -1;
    if (p < 1.0f) {
      const double tau = (double)p * zk;
      double ab = 0.0, ab2 = 0.0;
      const int g = find_group_mass(s, vk, tau, ab);
      if (g >= 0) o_cut = find_bin_mass<DT>(s, vk, (uint32_t)g, ab, tau, T, m, ab2);
      if (o_cut >= 0) {
        uint32_t lo, hi;
        tie_range16<DT>((uint32_t)o_cut, T, ord_min, ord_max, lo, hi);
        st.cut_lo = max(lo, kord_lo);
        st.cut_hi = hi;
        const double B = view_mass_ge<DT>(s, vk, hi + 1u, T, m);
        const uint32_t n_above = view_count_ge(s, vk, hi + 1u);
        st.n_cut_tie = (int)(view_count_ge(s, vk, st.cut_lo) - n_above);
        const double w = weight16<DT>((uint32_t)o_cut, T, m);
        double kf = (w > 0.0) ? floor((tau - B) / w) + 1.0 : (double)st.n_cut_tie;
        kf = fmax(1.0, fmin(kf, (double)st.n_cut_tie));
        st.n_cut_keep = (int)kf;
        st.zp = B + (double)st.n_cut_keep * w;
        st.n_kept = (int)n_above + st.n_cut_keep;
        st.x_cut = scaled16<DT>((uint32_t)o_cut, T);
      }
    }
    if (o_cut < 0) {
      // no top-p, or p*Z reaches the whole top-k set: everything in K is kept
      const int ol = lowest_ord(s, vk, nk);
      uint32_t lo, hi;
      tie_range16<DT>((uint32_t)ol, T, ord_min, ord_max, lo, hi);
      st.cut_lo = max(lo, kord_lo);
      st.cut_hi = hi;
      st.n_cut_tie = (int)(nk - view_count_ge(s, vk, hi + 1u));
      st.n_cut_keep = st.n_cut_tie;
      st.zp = zk;
      st.n_kept = (int)nk;
      st.x_cut = scaled16<DT>((uint32_t)ol, T);
    }

    // draw (sampling.py:26-27, inverse-CDF form): first kept element whose cumulative
    // mass exceeds u * Z_P
    const double t = (double)u * st.zp;
    st.target = t;
    const double above_cut = view_mass_ge<DT>(s, vk, st.cut_hi + 1u, T, m);
    bool in_cut = true;
    if (t < above_cut) {
      const View16 vp = make_view<DT>(s, st.cut_hi + 1u, T, m);
      double ab = 0.0, ab2 = 0.0;
      const int g = find_group_mass(s, vp, t, ab);
      const int o = (g >= 0) ? find_bin_mass<DT>(s, vp, (uint32_t)g, ab, t, T, m, ab2) : -1;
      if (o >= 0) {
        uint32_t lo, hi;
        tie_range16<DT>((uint32_t)o, T, ord_min, ord_max, lo, hi);
        st.sel_lo = max(lo, st.cut_hi + 1u);
        st.sel_hi = hi;
        const double B = view_mass_ge<DT>(s, vp, hi + 1u, T, m);
        const int n = (int)(view_count_ge(s, vp, st.sel_lo) - view_count_ge(s, vp, hi + 1u));
        const double w = weight16<DT>((uint32_t)o, T, m);
        double rf = (w > 0.0) ? floor((t - B) / w) : 0.0;
        st.sel_rank = (int)fmax(0.0, fmin(rf, (double)(n - 1)));
        in_cut = false;
      }
    }
    if (in_cut) {
      st.sel_lo = st.cut_lo;
      st.sel_hi = st.cut_hi;
      const double w = weight16<DT>(st.cut_hi, T, m);
      double rf = (w > 0.0) ? floor((t - above_cut) / w) : 0.0;
      st.sel_rank = (int)fmax(0.0, fmin(rf, (double)(st.n_cut_keep - 1)));
    }
    if (lane_id() == 0) s.st = st;
  }
  __syncthreads();
  const RowState st = s.st;
  __syncthreads();
  if (st.status != PBS_ROW_OK) {
    if (threadIdx.x == 0) write_error(a, b, PBS_ROW_NONFINITE, m);
    return;
  }

  // which of the tied tokens: the sel_rank-th lowest index with ord in [sel_lo, sel_hi]
  const uint32_t sel_lo = st.sel_lo, sel_hi = st.sel_hi;
  const int tok = select_index<DT>(src, s, [&](uint32_t raw) {
    const uint32_t o = ord16(raw);
    return o >= sel_lo && o <= sel_hi;
  }, st.sel_rank);

  if (a.out_probs || a.out_kept) {
    const uint32_t cut_lo = st.cut_lo, cut_hi = st.cut_hi;
    int cut_index = -1;
    if (st.n_cut_keep > 0)
      cut_index = select_index<DT>(src, s, [&](uint32_t raw) {
        const uint32_t o = ord16(raw);
        return o >= cut_lo && o <= cut_hi;
      }, st.n_cut_keep - 1);
    const int64_t obase = (int64_t)b * V;
    src.for_each([&](int, const u4& q, int base, bool vvalid) {
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        const int idx = base + e;
        if (elem_valid(src, vvalid, idx)) {
          const uint32_t o = ord16(elem_raw<DT>(q, e));
          const bool kept = o >= st.kord_lo && (o > cut_hi || (o >= cut_lo && idx <= cut_index));
          if (a.out_probs) a.out_probs[obase + idx] = kept ? (float)(weight16<DT>(o, T, m) / st.zp) : 0.0f;
          if (a.out_kept) a.out_kept[obase + idx] = kept ? 1 : 0;
        }
      }
    });
  }
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
__device__ void f32_ge(const Src& src, Smem& s, const Divider& dv, uint32_t t, float m, bool want_mass,
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
  c = wave_sum(c);
  ms = wave_sum(ms);
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
__device__ uint32_t f32_bisect_count(const Src& src, Smem& s, const Divider& dv, uint32_t lo, uint32_t hi,
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
__device__ uint32_t f32_bisect_mass(const Src& src, Smem& s, const Divider& dv, uint32_t lo, uint32_t hi,
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

template <class Src>
__device__ void sample_row32(const KArgs& a, Smem& s, Src& src, int b, float T, int kk, float p, float u) {
  const int V = a.vocab;
  Divider dv;
  dv.init(T);
  // stream: x = v/T (kept in place when the row is register resident), max, NaN flag
  float xmax = -INFINITY;
  int nan = 0;
  src.for_each([&](int j, const u4& q, int base, bool vvalid) {
    u4 xq;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x = dv(__uint_as_float(q[e]));
      xq[e] = __float_as_uint(x);
      if (elem_valid(src, vvalid, base + e)) {
        xmax = fmaxf(xmax, x);
        nan |= (x != x) ? 1 : 0;
      }
    }
    if constexpr (Src::kStore) src.store(j, xq);
  });
  nan = block_or_i(nan, s);
  const float m = block_max_f(xmax, s);
  if (nan || !(m > -INFINITY && m < INFINITY)) {
    if (threadIdx.x == 0) write_error(a, b, nan ? PBS_ROW_NAN : PBS_ROW_NONFINITE, m);
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
  if (p < 1.0f && zk * (double)p < zk) {
    const double tau = (double)p * zk;
    cut = f32_bisect_mass(src, s, dv, kord, ord_m, tau, m);
    double B;
    uint32_t n_above, n_ge;
    f32_ge(src, s, dv, cut + 1u, m, true, n_above, B);
    f32_ge(src, s, dv, cut, m, false, n_ge, ms);
    st.n_cut_tie = (int)(n_ge - n_above);
    const double w = (double)weight32(float_of_ord32(cut), m);
    double kf = (w > 0.0) ? floor((tau - B) / w) + 1.0 : (double)st.n_cut_tie;
    kf = fmax(1.0, fmin(kf, (double)st.n_cut_tie));
    st.n_cut_keep = (int)kf;
    st.zp = B + (double)st.n_cut_keep * w;
    st.n_kept = (int)n_above + st.n_cut_keep;
  } else {
    // keep all of K: the cutoff group is K's lowest value
    cut = f32_bisect_count(src, s, dv, kord, ord_m, nk);
    uint32_t n_above;
    f32_ge(src, s, dv, cut + 1u, m, false, n_above, ms);
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
  double above_cut;
  f32_ge(src, s, dv, cut + 1u, m, true, c, above_cut);
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

  if (a.out_probs || a.out_kept) {
    int cut_index = -1;
    if (st.n_cut_keep > 0)
      cut_index = select_index<PBS_DTYPE_F32>(src, s, [&](uint32_t raw) {
        return ord32(x_of<Src>(dv, raw)) == cut;
      }, st.n_cut_keep - 1);
    const int64_t obase = (int64_t)b * V;
    src.for_each([&](int, const u4& q, int base, bool vvalid) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int idx = base + e;
        if (elem_valid(src, vvalid, idx)) {
          const float x = x_of<Src>(dv, q[e]);
          const uint32_t o = ord32(x);
          const bool kept = o >= kord && (o > cut || (o == cut && idx <= cut_index));
          if (a.out_probs) a.out_probs[obase + idx] = kept ? (float)((double)weight32(x, m) / st.zp) : 0.0f;
          if (a.out_kept) a.out_kept[obase + idx] = kept ? 1 : 0;
        }
      }
    });
  }
  if (threadIdx.x == 0) write_info(a, b, tok < 0 ? 0 : tok, PBS_ROW_OK, st);
}

// ---------------------------------------------------------------------------------------
// one row
// ---------------------------------------------------------------------------------------
template <int DT, class Src>
__device__ void sample_row(const KArgs& a, Smem& s, Src& src, int b) {
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
  } else {
    sample_row32(a, s, src, b, T, kk, p, u);
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
  if (row_stride < vocab) return fail(PBS_ERR_INVALID_ARGUMENT, "row_stride %lld < vocab %lld",
                                      (long long)row_stride, (long long)vocab);
  if (!logits || !temperature || !top_k || !top_p || !uniform || !out_token || !out_status)
    return fail(PBS_ERR_INVALID_ARGUMENT, "null pointer argument");
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
