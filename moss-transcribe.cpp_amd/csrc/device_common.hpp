// device_common.hpp - device helpers shared by the per-op kernels and the
// persistent step kernel (q8_0 activation conversion, activation-panel layout,
// the MFMA tile accumulator, KV loads, argmax keys).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace mtg {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

namespace dev {

// ---------------------------------------------------------------------------
// Canonical arithmetic. The oracle (oracle/oracle.cpp) restates every one of
// these orders, so device results equal the oracle's bit for bit:
//  * exp: Cody-Waite reduction x = n ln2 + r, degree-7 Taylor polynomial in
//    Horner form with fmaf, ldexp; 0 below -87, inf above 88.7.
//  * q8_0 dot: K split in 4 slices of block pairs; per slice even and odd
//    blocks accumulate acc = fmaf(isum, dw*dx, acc) in block order; slices add
//    ((s0 + s1) + s2) + s3 per parity; result = even + odd.
//  * row sums of squares (RMSNorm): 64 partials (lane l holds elements
//    16l..16l+15 of a 1024 row, or l and l+64 of a 128 head), each a sequential
//    double sum of float squares, reduced by the xor butterfly 32,16,8,4,2,1.
//  * attention: keys in chunks of 64; score = fmaf chain over head_dim; per chunk
//    max, p = exp(w - max), l = butterfly sum of p over the 64 keys, O = fmaf
//    chain over the keys; chunks merged in order with f = exp(m_c - M),
//    L = fmaf(l_c, f, L), O = fmaf(O_c, f, O), out = O / L.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float dev_expf(float x) {
  // straight-line code: the out-of-range cases are selected at the end, so that
  // independent exponentials can interleave
  const float n = rintf(__fmul_rn(x, 1.44269504f));
  float r = fmaf(n, -0.693145752f, x);
  r = fmaf(n, -1.42860677e-06f, r);
  float p = 1.98412698e-4f;             // 1/5040
  p = fmaf(p, r, 1.38888889e-3f);       // 1/720
  p = fmaf(p, r, 8.33333333e-3f);       // 1/120
  p = fmaf(p, r, 4.16666667e-2f);       // 1/24
  p = fmaf(p, r, 1.66666667e-1f);       // 1/6
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const float e = ldexpf(p, (int)fminf(fmaxf(n, -200.0f), 200.0f));
  return x < -87.0f ? 0.0f : (x > 88.7f ? INFINITY : e);  // every result a normal float
}

// Correctly rounded square root of a non-negative float. The hardware estimate
// is within one ulp; the neighbour whose rounding interval holds x is chosen by
// comparing x with the squared midpoints, all exact in double (a float has 24
// significant bits, a midpoint 25, its square at most 50).
__device__ __forceinline__ float dev_sqrtf(float x) {
  const float s = __builtin_sqrtf(x);
  const float up = __uint_as_float(__float_as_uint(s) + 1u);
  const float dn = __uint_as_float(__float_as_uint(s) - 1u);
  const double xd = (double)x;
  const double mu = ((double)s + (double)up) * 0.5, md = ((double)s + (double)dn) * 0.5;
  const float r = xd > mu * mu ? up : (xd < md * md ? dn : s);
  return (!(x > 0.0f) || x == INFINITY) ? s : r;  // selects, no branches
}

// 1 / sqrt(mean + eps) of an RMSNorm row, correctly rounded at every step.
__device__ __forceinline__ float dev_rms_scale(float mean, float eps) {
  return __fdiv_rn(1.0f, dev_sqrtf(__fadd_rn(mean, eps)));
}

// silu(g) * u with the canonical exp and a correctly rounded division.
// erf by its Maclaurin series in double, a fixed number of terms per range of
// |z| (the oracle evaluates the same operations); +-1 from |z| >= 4. The
// divisions by n + 1 and 2 n + 1 are multiplications by their double
// reciprocals, rounded once at compile time (the oracle's table holds the same
// values).
template <int N>
struct ErfRecip {
  double inv_next[N], inv_odd[N];
  constexpr ErfRecip() : inv_next(), inv_odd() {
    for (int n = 0; n < N; ++n) {
      inv_next[n] = 1.0 / (double)(n + 1);
      inv_odd[n] = 1.0 / (double)(2 * n + 1);
    }
  }
};
__constant__ constexpr ErfRecip<76> kErfRecip{};
__device__ __forceinline__ double dev_erf_series(double z) {
  const ErfRecip<76>& tab = kErfRecip;
  const double a = fabs(z);
  if (a >= 4.0) return z < 0.0 ? -1.0 : 1.0;
  const int terms = a < 1.0 ? 28 : (a < 2.0 ? 44 : (a < 3.0 ? 60 : 76));
  const double a2 = __dmul_rn(a, a);
  double term = a, sum = 0.0;
#pragma unroll 4
  for (int n = 0; n < terms; ++n) {
    sum = __dadd_rn(sum, __dmul_rn(term, tab.inv_odd[n]));
    term = -__dmul_rn(__dmul_rn(term, a2), tab.inv_next[n]);
  }
  const double r = __dmul_rn(sum, 1.1283791670955126);  // 2 / sqrt(pi)
  return z < 0.0 ? -r : r;
}
// ggml_gelu_erf: 0.5 x (1 + erf(x / sqrt 2)), evaluated left to right
__device__ __forceinline__ float dev_gelu_erf(float x) {
  const float z = __fmul_rn(x, 0.70710678118654752440f);
  const float e = (float)dev_erf_series((double)z);
  return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, e));
}
// dev_gelu_erf of N values at once: the N erf series run in lock step, each
// element stopping at its own term count, so every element sees exactly the
// operations of dev_gelu_erf; the N independent chains hide the latency of the
// dependent double multiplies.
template <int N>
__device__ __forceinline__ void dev_gelu_erf_n(float (&x)[N]) {
  const ErfRecip<76>& tab = kErfRecip;
  double a2[N], term[N], sum[N];
  int terms[N], tmax = 0;
#pragma unroll
  for (int e = 0; e < N; ++e) {
    const double a = fabs((double)__fmul_rn(x[e], 0.70710678118654752440f));
    terms[e] = a >= 4.0 ? 0 : (a < 1.0 ? 28 : (a < 2.0 ? 44 : (a < 3.0 ? 60 : 76)));
    tmax = max(tmax, terms[e]);
    a2[e] = __dmul_rn(a, a);
    term[e] = a;
    sum[e] = 0.0;
  }
  for (int n = 0; n < tmax; ++n) {
    const double io = tab.inv_odd[n], in = tab.inv_next[n];
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const double s1 = __dadd_rn(sum[e], __dmul_rn(term[e], io));
      const double t1 = -__dmul_rn(__dmul_rn(term[e], a2[e]), in);
      const bool live = n < terms[e];
      sum[e] = live ? s1 : sum[e];
      term[e] = live ? t1 : term[e];
    }
  }
#pragma unroll
  for (int e = 0; e < N; ++e) {
    const float z = __fmul_rn(x[e], 0.70710678118654752440f);
    const double r = terms[e] == 0 ? 1.0 : __dmul_rn(sum[e], 1.1283791670955126);
    const float er = (float)(z < 0.0f ? -r : r);
    x[e] = __fmul_rn(__fmul_rn(0.5f, x[e]), __fadd_rn(1.0f, er));
  }
}
// ggml_silu: x / (1 + exp(-x))
__device__ __forceinline__ float dev_silu(float x) { return __fdiv_rn(x, __fadd_rn(1.0f, dev_expf(-x))); }

__device__ __forceinline__ float dev_swiglu(float g, float u) {
  return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, dev_expf(-g))), u);
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}

// ------------------------------------------------------ lane exchanges ---
// lane_xor<O>(v): the value of lane (lane ^ O) of a 64-lane wave, with VALU
// lane moves instead of LDS permutes: DPP quad_perm (O = 1, 2), two bank-masked
// row rotations (O = 4: lanes 0-3 / 8-11 of a row take lane + 4, the others
// lane - 4), row_ror:8 (O = 8), and the gfx950 row / half-wave swaps (O = 16, 32:
// each half keeps the value that crossed over).
template <int O>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
  const int x = (int)v;
  if constexpr (O == 1) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);
  } else if constexpr (O == 2) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);
  } else if constexpr (O == 4) {
    const int t = __builtin_amdgcn_update_dpp(x, x, 0x12C, 0xF, 0x5, false);
    return (uint32_t)__builtin_amdgcn_update_dpp(t, x, 0x124, 0xF, 0xA, false);
  } else if constexpr (O == 8) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false);
  } else if constexpr (O == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (threadIdx.x & 16) ? r[0] : r[1];
  } else {
    static_assert(O == 32, "lane_xor: 1, 2, 4, 8, 16 or 32");
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (threadIdx.x & 32) ? r[0] : r[1];
  }
}
template <int O>
__device__ __forceinline__ float lane_xor_f(float v) {
  return __uint_as_float(lane_xor<O>(__float_as_uint(v)));
}
template <int O>
__device__ __forceinline__ uint64_t lane_xor_u64(uint64_t v) {
  return ((uint64_t)lane_xor<O>((uint32_t)(v >> 32)) << 32) | lane_xor<O>((uint32_t)v);
}
template <int O>
__device__ __forceinline__ double lane_xor_d(double v) {
  return __longlong_as_double((long long)lane_xor_u64<O>((uint64_t)__double_as_longlong(v)));
}

// ------------------------------------------------------ wave reductions ---
// A reduction step needs op(x_lane, x_partner), not the exchange itself; for a
// commutative op (IEEE add, max) either operand order gives the same bits, so the
// steps use cheaper lane moves than lane_xor and every lane still ends with the
// value of the xor butterfly:
//   * O = 32, 16: the half-wave / row swap of two copies leaves one member of
//     each (lane, lane ^ O) pair in each register: op(a, b).
//   * O = 8, 4, 2, 1 inside a 16-lane row: row_ror:O. ror 8 is xor 8; once the
//     steps 8, 4, .. above O are done the values are symmetric under xor with
//     those bits, and lane + O (mod 16) differs from lane ^ O only in them.
// The DPP moves read with bound_ctrl, so the compiler may fold them into the op.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __uint_as_float(dpp_u<CTRL>(__float_as_uint(x)));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double x) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  return __longlong_as_double(
      (long long)(((uint64_t)dpp_u<CTRL>((uint32_t)(b >> 32)) << 32) | dpp_u<CTRL>((uint32_t)b)));
}
constexpr int kDppRor8 = 0x128, kDppRor4 = 0x124, kDppRor2 = 0x122, kDppRor1 = 0x121;
constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

// The members of every (lane, lane ^ O) pair, O = 16 or 32, one in a and one in b.
template <int O>
__device__ __forceinline__ void pair_split(uint32_t x, uint32_t& a, uint32_t& b) {
  if constexpr (O == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    a = r[0];
    b = r[1];
  } else {
    static_assert(O == 32, "pair_split: 16 or 32");
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    a = r[0];
    b = r[1];
  }
}
template <int O>
__device__ __forceinline__ float pair_add_f(float v) {
  uint32_t a, b;
  pair_split<O>(__float_as_uint(v), a, b);
  return __fadd_rn(__uint_as_float(a), __uint_as_float(b));
}
template <int O>
__device__ __forceinline__ float pair_max_f(float v) {
  uint32_t a, b;
  pair_split<O>(__float_as_uint(v), a, b);
  return fmaxf(__uint_as_float(a), __uint_as_float(b));
}
template <int O>
__device__ __forceinline__ double pair_add_d(double v) {
  const uint64_t bits = (uint64_t)__double_as_longlong(v);
  uint32_t alo, blo, ahi, bhi;
  pair_split<O>((uint32_t)bits, alo, blo);
  pair_split<O>((uint32_t)(bits >> 32), ahi, bhi);
  return __longlong_as_double((long long)(((uint64_t)ahi << 32) | alo)) +
         __longlong_as_double((long long)(((uint64_t)bhi << 32) | blo));
}
// max over non-negative floats (their bit patterns order as unsigned integers)
template <int O>
__device__ __forceinline__ uint32_t pair_max_u(uint32_t v) {
  uint32_t a, b;
  pair_split<O>(v, a, b);
  return max(a, b);
}

// xor butterfly 32, 16, 8, 4, 2, 1 (the canonical order of every wave sum)
__device__ __forceinline__ double wave_sum_d(double v) {
  v = pair_add_d<32>(v);
  v = pair_add_d<16>(v);
  v += dpp_d<kDppRor8>(v);
  v += dpp_d<kDppRor4>(v);
  v += dpp_d<kDppRor2>(v);
  v += dpp_d<kDppRor1>(v);
  return v;
}
// amax of non-negative values over 8 consecutive lanes (aligned groups)
__device__ __forceinline__ float group8_max_nonneg(float v) {
  uint32_t u = __float_as_uint(v);
  u = max(u, dpp_u<kDppQuadXor1>(u));
  u = max(u, dpp_u<kDppQuadXor2>(u));
  u = max(u, dpp_u<kDppHalfMirror>(u));
  return __uint_as_float(u);
}
// amax of non-negative values over 32 consecutive lanes (aligned halves)
__device__ __forceinline__ float group32_max_nonneg(float v) {
  uint32_t u = __float_as_uint(group8_max_nonneg(v));
  u = max(u, dpp_u<kDppMirror>(u));
  return __uint_as_float(pair_max_u<16>(u));
}
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o) {
  switch (o) {
    case 1: return lane_xor_u64<1>(v);
    case 2: return lane_xor_u64<2>(v);
    case 4: return lane_xor_u64<4>(v);
    case 8: return lane_xor_u64<8>(v);
    case 16: return lane_xor_u64<16>(v);
    default: return lane_xor_u64<32>(v);
  }
}

// q8_0 activation conversion of one 32-element block held by 8 consecutive lanes
// (4 elements each): d = amax/127 rounded to f16, codes = rint(x * 127/amax).
// Returns the f32 value of the stored f16 scale.
__device__ __forceinline__ float quant_block8(const float v[4], int8_t q[4]) {
  const float amax =
      group8_max_nonneg(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  const float d = __fdiv_rn(amax, 127.0f);
  const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
  for (int e = 0; e < 4; ++e) q[e] = (int8_t)rintf(__fmul_rn(v[e], id));
  return __half2float(__float2half_rn(d));
}

// Panel position of element k of verify row t (see mtg_internal.hpp).
__device__ __forceinline__ void panel_store4(Panel p, int bps, int t, int k, const int8_t q[4]) {
  const int b = k >> 5, bp = b >> 1, par = b & 1, half = (k >> 4) & 1, byte = k & 15;
  const int cg = t >> 3, j = par * 8 + (t & 7), g = 2 * par + half, lane = j + 16 * g;
  uint32_t packed = (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) |
                    ((uint32_t)(uint8_t)q[2] << 16) | ((uint32_t)(uint8_t)q[3] << 24);
  *(uint32_t*)(p.codes + ((size_t)(cg * bps + bp)) * 1024 + lane * 16 + byte) = packed;
}
__device__ __forceinline__ void panel_store_scale(Panel p, int bps, int t, int block, float d) {
  const int bp = block >> 1, par = block & 1, cg = t >> 3, j = par * 8 + (t & 7);
  p.scales[(size_t)(cg * bps + bp) * 16 + j] = d;
}

// ----------------------------------------------------------- GEMM core ------
// One wave accumulates a 16-row tile over block pairs [bp0, bp1) for every
// column group: acc[cg][r] holds rows 4*(lane/16)+r of column lane%16, split by
// block parity (columns 0-7 even blocks, 8-15 odd blocks of rows t = col%8).
template <int G>
__device__ __forceinline__ void tile_accumulate(const uint8_t* __restrict__ tile, int bp0, int bp1,
                                                const uint8_t* __restrict__ pcodes,
                                                const float* __restrict__ pscales, int bps,
                                                float acc[G][4]) {
  const int lane = threadIdx.x & 63;
  const int par = (lane & 15) >> 3;
  const int srow = par * 16 + 4 * (lane >> 4);
  const v4i zero = {0, 0, 0, 0};
#pragma unroll 4
  for (int bp = bp0; bp < bp1; ++bp) {  // 4 pairs in flight per wave
    const uint8_t* unit = tile + (size_t)bp * kUnitBytes;
    const v4i a = *(const v4i*)(unit + lane * 16);
    const uint2 sw = *(const uint2*)(unit + 1024 + srow * 2);
    float dw[4];
    dw[0] = half_bits_to_float((uint16_t)(sw.x & 0xffff));
    dw[1] = half_bits_to_float((uint16_t)(sw.x >> 16));
    dw[2] = half_bits_to_float((uint16_t)(sw.y & 0xffff));
    dw[3] = half_bits_to_float((uint16_t)(sw.y >> 16));
#pragma unroll
    for (int cg = 0; cg < G; ++cg) {
      const v4i b = *(const v4i*)(pcodes + ((size_t)(cg * bps + bp)) * 1024 + lane * 16);
      const float dx = pscales[(size_t)(cg * bps + bp) * 16 + (lane & 15)];
      const v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, zero, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[cg][r] = fmaf((float)c[r], dw[r] * dx, acc[cg][r]);
    }
  }
}

// One wave computes a whole tile in the canonical order: four slice
// accumulators, summed ((s0 + s1) + s2) + s3, then even + odd parity.
template <int G>
__device__ __forceinline__ void tile_accumulate_canonical(const uint8_t* __restrict__ tile, int bps,
                                                          const uint8_t* __restrict__ pcodes,
                                                          const float* __restrict__ pscales,
                                                          float acc[G][4]) {
  float part[4][G][4];
#pragma unroll
  for (int sl = 0; sl < 4; ++sl) {
#pragma unroll
    for (int cg = 0; cg < G; ++cg)
#pragma unroll
      for (int r = 0; r < 4; ++r) part[sl][cg][r] = 0.0f;
    tile_accumulate<G>(tile, (bps * sl) / 4, (bps * (sl + 1)) / 4, pcodes, pscales, bps, part[sl]);
  }
#pragma unroll
  for (int cg = 0; cg < G; ++cg)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = __fadd_rn(__fadd_rn(__fadd_rn(part[0][cg][r], part[1][cg][r]), part[2][cg][r]), part[3][cg][r]);
      acc[cg][r] = __fadd_rn(v, dpp_f<kDppRor8>(v));
    }
}

__device__ __forceinline__ float kv_load(const void* base, int f16, size_t idx) {
  return f16 ? __half2float(((const __half*)base)[idx]) : ((const float*)base)[idx];
}
__device__ __forceinline__ v4f kv_load4(const void* base, int f16, size_t idx) {
  if (f16) {
    const uint2 raw = *(const uint2*)((const __half*)base + idx);
    v4f r;
    r[0] = half_bits_to_float((uint16_t)(raw.x & 0xffff));
    r[1] = half_bits_to_float((uint16_t)(raw.x >> 16));
    r[2] = half_bits_to_float((uint16_t)(raw.y & 0xffff));
    r[3] = half_bits_to_float((uint16_t)(raw.y >> 16));
    return r;
  }
  return *(const v4f*)((const float*)base + idx);
}

__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {
  if (v == 0.0f) v = 0.0f;  // -0 and +0 compare equal in the reference
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
}


// Device-coherent accesses for data exchanged between workgroups inside one
// launch (they bypass the non-coherent caches; no cache maintenance needed).
__device__ __forceinline__ uint32_t ld_coh_u32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coh(const float* p) {
  return __uint_as_float(__hip_atomic_load((const uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ void st_coh(float* p, float v) {
  __hip_atomic_store((uint32_t*)p, __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_coh_u64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh_u64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <bool COH>
__device__ __forceinline__ void st_f(float* p, float v) {
  if (COH) st_coh(p, v);
  else *p = v;
}

__device__ __forceinline__ float wave_max_f(float v) {
  v = pair_max_f<32>(v);
  v = pair_max_f<16>(v);
  v = fmaxf(v, dpp_f<kDppRor8>(v));
  v = fmaxf(v, dpp_f<kDppRor4>(v));
  v = fmaxf(v, dpp_f<kDppRor2>(v));
  v = fmaxf(v, dpp_f<kDppRor1>(v));
  return v;
}
__device__ __forceinline__ float wave_sum_f(float v) {
  v = pair_add_f<32>(v);
  v = pair_add_f<16>(v);
  v = __fadd_rn(v, dpp_f<kDppRor8>(v));
  v = __fadd_rn(v, dpp_f<kDppRor4>(v));
  v = __fadd_rn(v, dpp_f<kDppRor2>(v));
  v = __fadd_rn(v, dpp_f<kDppRor1>(v));
  return v;
}
// N values reduced side by side, step by step, each in the order of wave_sum_d /
// wave_sum_f.
template <int N>
__device__ __forceinline__ void wave_sum_d_n(double* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = pair_add_d<32>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = pair_add_d<16>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_d<kDppRor8>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_d<kDppRor4>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_d<kDppRor2>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] += dpp_d<kDppRor1>(v[i]);
}
// a + b of the members of every (lane, lane ^ O) pair of two double registers
// at once (O = 32: half-wave swap, O = 16: swap of 16-lane rows): lanes whose
// bit O is clear end with a's pair sum, the others with b's.
template <int O>
__device__ __forceinline__ double swap_add_d(double a, double b) {
  const uint64_t ab = (uint64_t)__double_as_longlong(a), bb = (uint64_t)__double_as_longlong(b);
  uint32_t lo[2], hi[2];
  if constexpr (O == 32) {
    const auto l = __builtin_amdgcn_permlane32_swap((uint32_t)ab, (uint32_t)bb, false, false);
    const auto h = __builtin_amdgcn_permlane32_swap((uint32_t)(ab >> 32), (uint32_t)(bb >> 32), false, false);
    lo[0] = l[0], lo[1] = l[1], hi[0] = h[0], hi[1] = h[1];
  } else {
    static_assert(O == 16, "swap_add_d: 16 or 32");
    const auto l = __builtin_amdgcn_permlane16_swap((uint32_t)ab, (uint32_t)bb, false, false);
    const auto h = __builtin_amdgcn_permlane16_swap((uint32_t)(ab >> 32), (uint32_t)(bb >> 32), false, false);
    lo[0] = l[0], lo[1] = l[1], hi[0] = h[0], hi[1] = h[1];
  }
  return __longlong_as_double((long long)(((uint64_t)hi[0] << 32) | lo[0])) +
         __longlong_as_double((long long)(((uint64_t)hi[1] << 32) | lo[1]));
}

// The RMSNorm scales dev_rms_scale(S_j / K) of N rows (N even), S_j the wave sum
// of the lanes' double partials v[j] in wave_sum_d's pairing. The rows travel
// packed across the lanes: one half-wave swap reduces rows 2k and 2k + 1 together
// (row 2k then in lanes 0-31, row 2k + 1 in 32-63), one row swap two such
// registers (four rows, one per 16-lane row: 4q, 4q + 2, 4q + 1, 4q + 3), the DPP
// steps the rest. Lane q of each 16-lane row evaluates register q's scale there
// (the same operations in any lane); every lane reads the N scales back. Every
// lane of the wave must be active.
template <int N, int K>
__device__ __forceinline__ void rms_scales(const double (&v)[N], float eps, float (&scale)[N]) {
  static_assert(N % 2 == 0 && N <= 32, "an even number of rows, at most 32");
  constexpr int P = N / 2, Q = (P + 1) / 2;
  double a[P], r[Q];
#pragma unroll
  for (int k = 0; k < P; ++k) a[k] = swap_add_d<32>(v[2 * k], v[2 * k + 1]);
#pragma unroll
  for (int q = 0; q < Q; ++q) r[q] = 2 * q + 1 < P ? swap_add_d<16>(a[2 * q], a[2 * q + 1]) : pair_add_d<16>(a[2 * q]);
#pragma unroll
  for (int q = 0; q < Q; ++q) r[q] += dpp_d<kDppRor8>(r[q]);
#pragma unroll
  for (int q = 0; q < Q; ++q) r[q] += dpp_d<kDppRor4>(r[q]);
#pragma unroll
  for (int q = 0; q < Q; ++q) r[q] += dpp_d<kDppRor2>(r[q]);
#pragma unroll
  for (int q = 0; q < Q; ++q) r[q] += dpp_d<kDppRor1>(r[q]);
  const int lane = threadIdx.x & 63;
  double mine = r[0];
#pragma unroll
  for (int q = 1; q < Q; ++q) mine = (lane & 15) == q ? r[q] : mine;
  const int sc = __builtin_bit_cast(int, dev_rms_scale((float)(mine / (double)K), eps));
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const int w = j % 4, src = j / 4 + (w == 0 ? 0 : w == 1 ? 32 : w == 2 ? 16 : 48);
    // held in a vector register: N scalar registers live through the row loop
    // would add to the scalar spills of the larger kernels
    float x = __builtin_bit_cast(float, __builtin_amdgcn_readlane(sc, src));
    asm volatile("" : "+v"(x));
    scale[j] = x;
  }
}

template <int N>
__device__ __forceinline__ void wave_sum_f_n(float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = pair_add_f<32>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = pair_add_f<16>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = __fadd_rn(v[i], dpp_f<kDppRor8>(v[i]));
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = __fadd_rn(v[i], dpp_f<kDppRor4>(v[i]));
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = __fadd_rn(v[i], dpp_f<kDppRor2>(v[i]));
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = __fadd_rn(v[i], dpp_f<kDppRor1>(v[i]));
}
// Position of key k of a 64-key chunk in a permuted probability row (key
// 4 s + kk at kk * 16 + s).
__device__ __forceinline__ int sp_key_pos(int key) { return (key & 3) * 16 + (key >> 2); }
// The value of lane ^ 4 within groups of 8 lanes: a row rotation right by n
// gives lane l the value of lane l - n (mod 16), so lanes with bit 2 clear take
// the rotation by 12 (lane l + 4) and the others the rotation by 4 (lane l - 4).
__device__ __forceinline__ uint32_t lane_xor4(uint32_t v) {
  const uint32_t from_up = dpp_u<0x12C>(v), from_dn = dpp_u<0x124>(v);
  return (threadIdx.x & 4) ? from_dn : from_up;
}
// Order-preserving integer key of a float that is not NaN (signed compare), and
// back; max is exact in any order.
__device__ __forceinline__ int ord_key(float x) {
  const int b = __float_as_int(x);
  return b ^ ((b >> 31) & 0x7FFFFFFF);
}
__device__ __forceinline__ float ord_val(int k) { return __int_as_float(k ^ ((k >> 31) & 0x7FFFFFFF)); }
template <int N>
__device__ __forceinline__ void wave_max_i_n(int* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    uint32_t a, b;
    pair_split<32>((uint32_t)v[i], a, b);
    v[i] = max((int)a, (int)b);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    uint32_t a, b;
    pair_split<16>((uint32_t)v[i], a, b);
    v[i] = max((int)a, (int)b);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = max(v[i], (int)dpp_u<kDppRor8>((uint32_t)v[i]));
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = max(v[i], (int)dpp_u<kDppRor4>((uint32_t)v[i]));
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = max(v[i], (int)dpp_u<kDppRor2>((uint32_t)v[i]));
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = max(v[i], (int)dpp_u<kDppRor1>((uint32_t)v[i]));
}

// max of a 64-bit key over the wave (exact in any order); both halves take the
// same lane moves, so each pair of halves stays one lane's key
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  uint32_t alo, blo, ahi, bhi;
  pair_split<32>((uint32_t)v, alo, blo);
  pair_split<32>((uint32_t)(v >> 32), ahi, bhi);
  v = max(((uint64_t)ahi << 32) | alo, ((uint64_t)bhi << 32) | blo);
  pair_split<16>((uint32_t)v, alo, blo);
  pair_split<16>((uint32_t)(v >> 32), ahi, bhi);
  v = max(((uint64_t)ahi << 32) | alo, ((uint64_t)bhi << 32) | blo);
  uint64_t o = ((uint64_t)dpp_u<kDppRor8>((uint32_t)(v >> 32)) << 32) | dpp_u<kDppRor8>((uint32_t)v);
  v = max(v, o);
  o = ((uint64_t)dpp_u<kDppRor4>((uint32_t)(v >> 32)) << 32) | dpp_u<kDppRor4>((uint32_t)v);
  v = max(v, o);
  o = ((uint64_t)dpp_u<kDppRor2>((uint32_t)(v >> 32)) << 32) | dpp_u<kDppRor2>((uint32_t)v);
  v = max(v, o);
  o = ((uint64_t)dpp_u<kDppRor1>((uint32_t)(v >> 32)) << 32) | dpp_u<kDppRor1>((uint32_t)v);
  return max(v, o);
}

// exact integer wave sum (any order is exact)
__device__ __forceinline__ int wave_sum_i(int v) {
  uint32_t a, b;
  pair_split<32>((uint32_t)v, a, b);
  v = (int)a + (int)b;
  pair_split<16>((uint32_t)v, a, b);
  v = (int)a + (int)b;
  v += (int)dpp_u<kDppRor8>((uint32_t)v);
  v += (int)dpp_u<kDppRor4>((uint32_t)v);
  v += (int)dpp_u<kDppRor2>((uint32_t)v);
  v += (int)dpp_u<kDppRor1>((uint32_t)v);
  return v;
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  uint32_t a, b;
  pair_split<32>(v, a, b);
  v = min(a, b);
  pair_split<16>(v, a, b);
  v = min(a, b);
  v = min(v, dpp_u<kDppRor8>(v));
  v = min(v, dpp_u<kDppRor4>(v));
  v = min(v, dpp_u<kDppRor2>(v));
  v = min(v, dpp_u<kDppRor1>(v));
  return v;
}
__device__ __forceinline__ float f16_round(float v) { return __half2float(__float2half_rn(v)); }

// ------------------------------------------------------------- attention ----
constexpr int kChunk = kChunkKeys;  // keys per attention chunk (canonical)

// Where the keys and values of one kv head come from: the cache, except keys at
// or after new_from, which are rows (key - new_from) of knew/vnew (LDS).
struct AttnSrc {
  const void* kc;
  const void* vc;
  int f16;
  size_t head_base;  // element offset of the kv head in the cache
  const float* knew;
  const float* vnew;
  int new_from;      // >= kvlen when every key is in the cache
};

// Scores, chunk softmax and P.V of keys [key0, key0+64) for ncol query columns
// held in q (LDS, [col][128], already f16-rounded for an f16 cache). col ->
// query row col_t(col) = col % T. Writes (m, l) and O of each column. 256
// threads. LDS: vbuf [64][128], sp [kMaxCols][64].
__device__ __forceinline__ v4f attn_row4(const AttnSrc& a, bool is_v, int key, int d) {
  if (key >= a.new_from) return *(const v4f*)((is_v ? a.vnew : a.knew) + (key - a.new_from) * kHeadDim + d);
  return kv_load4(is_v ? a.vc : a.kc, a.f16, a.head_base + (size_t)key * kHeadDim + d);
}

template <bool COH>
__device__ void attn_chunk(const AttnSrc& a, const float* q, int ncol, int T, int past, int kvlen,
                           int key0, float scale, float* vbuf, float* sp, float* out_ml,
                           float* out_o) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // 1. V chunk -> LDS (zeros past kvlen); unrolled so that the loads are in flight together
#pragma unroll
  for (int idx = tid; idx < kChunk * kHeadDim / 4; idx += 256) {
    const int j = idx >> 5, d = (idx & 31) * 4, key = key0 + j;
    const v4f v = key < kvlen ? attn_row4(a, true, key, d) : (v4f){0.f, 0.f, 0.f, 0.f};
    *(v4f*)(vbuf + j * kHeadDim + d) = v;
  }
  // 2. scores: thread = (key, 8 columns)
  {
    const int key = key0 + lane, c0 = wave * 8;
    const bool kvalid = key < kvlen;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    if (c0 < ncol && kvalid) {
#pragma unroll 8
      for (int d = 0; d < kHeadDim; d += 4) {
        const v4f kf = attn_row4(a, false, key, d);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const v4f qf = *(const v4f*)(q + (c0 + i) * kHeadDim + d);
          acc[i] = fmaf(qf[0], kf[0], acc[i]);
          acc[i] = fmaf(qf[1], kf[1], acc[i]);
          acc[i] = fmaf(qf[2], kf[2], acc[i]);
          acc[i] = fmaf(qf[3], kf[3], acc[i]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int col = c0 + i;
      if (col < ncol) {
        const int t = col % T;
        sp[col * kChunk + lane] = (kvalid && key <= past + t) ? __fmul_rn(acc[i], scale) : -INFINITY;
      }
    }
  }
  __syncthreads();
  // 3. chunk softmax per column (one wave per column, lane = key)
  for (int col = wave; col < ncol; col += 4) {
    const float w = sp[col * kChunk + lane];
    const float m = wave_max_f(w);
    float p = (m == -INFINITY || w == -INFINITY) ? 0.0f : dev_expf(__fsub_rn(w, m));
    if (a.f16) p = f16_round(p);
    const float l = wave_sum_f(p);
    sp[col * kChunk + lane] = p;
    if (lane == 0) {
      st_f<COH>(out_ml + col * 2, m);
      st_f<COH>(out_ml + col * 2 + 1, l);
    }
  }
  __syncthreads();
  // 4. O[col][d] = sum over the 64 keys in order of p * v
  {
    const int d = tid & 127, c0 = (tid >> 7) * 16;
    float o[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = 0.0f;
    if (c0 < ncol) {
      for (int j = 0; j < kChunk; ++j) {
        const float v = vbuf[j * kHeadDim + d];
#pragma unroll
        for (int i = 0; i < 16; ++i) o[i] = fmaf(sp[(c0 + i < ncol ? c0 + i : 0) * kChunk + j], v, o[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (c0 + i < ncol) st_f<COH>(out_o + (c0 + i) * kHeadDim + d, o[i]);
  }
  __syncthreads();
}

// Merge the chunk partials of one query column (canonical order); returns
// element d of the attention output. part_ml/part_o point at chunk 0 of the
// column, consecutive chunks `stride_ml` / `stride_o` floats apart. Lane c of a
// wave loads (m, l) of chunk c0 + c, so a round of loads covers 64 chunks; the
// O values come 16 chunks per round; f = exp(m_c - M) is computed once per
// chunk and read by every thread (readlane) for the two chunk-ordered chains.
template <bool COH>
__device__ __forceinline__ float attn_merge(const float* part_ml, const float* part_o, int nch,
                                            size_t stride_ml, size_t stride_o, int d) {
  auto ld = [](const float* p) { return COH ? ld_coh(p) : *p; };
  const int lane = threadIdx.x & 63;
  float M = -INFINITY;
  for (int c0 = 0; c0 < nch; c0 += 64) {
    const float m = c0 + lane < nch ? ld(part_ml + (size_t)(c0 + lane) * stride_ml) : -INFINITY;
    M = fmaxf(M, wave_max_f(m));
  }
  float L = 0.0f, O = 0.0f;
  for (int c0 = 0; c0 < nch; c0 += 64) {
    const int c = c0 + lane;
    const float m = c < nch ? ld(part_ml + (size_t)c * stride_ml) : -INFINITY;
    const float l = c < nch ? ld(part_ml + (size_t)c * stride_ml + 1) : 0.0f;
    const float f = m == -INFINITY ? 0.0f : dev_expf(__fsub_rn(m, M));
    const int nb = min(64, nch - c0);
    for (int i0 = 0; i0 < nb; i0 += 16) {
      float o[16];
#pragma unroll
      for (int i = 0; i < 16; ++i)
        o[i] = i0 + i < nb ? ld(part_o + (size_t)(c0 + i0 + i) * stride_o + d) : 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (i0 + i >= nb) break;
        const float mc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m), i0 + i));
        if (mc == -INFINITY) continue;
        const float fc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f), i0 + i));
        const float lc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l), i0 + i));
        L = fmaf(lc, fc, L);
        O = fmaf(o[i], fc, O);
      }
    }
  }
  return __fdiv_rn(O, L);
}

// ------------------------------------- f16 / q4_K weight activations ---
// 1 / sqrt(mean(x^2) + eps) of a hidden row (K == 1024), the canonical double sum:
// lane l sums elements 16l..16l+15, then the butterfly. Called by wave 0.
__device__ __forceinline__ float row_rms_scale(const float* xr, int K, float eps) {
  const int lane = threadIdx.x & 63;
  double s = 0.0;
  for (int e = 0; e < 16; ++e) {
    const float v = xr[lane * 16 + e];
    s += (double)__fmul_rn(v, v);
  }
  s = wave_sum_d(s);
  return dev_rms_scale((float)(s / (double)K), eps);
}

// ggml quantize_row_q8_K_ref of one 256-block held one element per thread of a
// 256-thread workgroup: the element of largest magnitude (the first one on ties)
// gives max with its sign, iscale = -127/max, codes = min(127, nearest(iscale*x)),
// d = 1/iscale, bsums over 16-element groups.
// Threads 0..255 hold the block; in a larger workgroup the others pass the
// barrier only.
__device__ __forceinline__ void q8k_block256(float y, const ActQ8K& a, int t, int K, int b) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const bool active = tid < 256;
  __shared__ float s_y[256];
  __shared__ uint64_t s_key[4];
  if (active) s_y[tid] = y;
  // first maximum of |y|: larger magnitude, then lower index
  const uint64_t key = ((uint64_t)__float_as_uint(fabsf(y)) << 32) | (uint32_t)(255 - tid);
  const uint64_t wk = wave_max_u64(key);
  if (active && lane == 0) s_key[wave] = wk;
  __syncthreads();
  if (!active) return;
  uint64_t best = s_key[0];
  for (int w = 1; w < 4; ++w) best = s_key[w] > best ? s_key[w] : best;
  const float maxv = s_y[255 - (int)(best & 0xffffffffu)];
  int q = 0;
  float d = 0.0f;
  if ((best >> 32) != 0) {  // amax > 0
    const float iscale = __fdiv_rn(-127.0f, maxv);
    q = min(127, (int)rintf(__fmul_rn(iscale, y)));
    d = __fdiv_rn(1.0f, iscale);
  }
  a.qs[(size_t)t * K + b * 256 + tid] = (int8_t)q;
  // bsums: the 16 lanes of a DPP row hold one group
  int s = q;
  s += (int)dpp_u<kDppRor8>((uint32_t)s);
  s += (int)dpp_u<kDppRor4>((uint32_t)s);
  s += (int)dpp_u<kDppRor2>((uint32_t)s);
  s += (int)dpp_u<kDppRor1>((uint32_t)s);
  if ((tid & 15) == 0) a.bsums[(size_t)t * (K / 16) + b * 16 + (tid >> 4)] = s;
  if (tid == 0) a.d[(size_t)t * (K / 256) + b] = d;
}

// get_scale_min_k4 of the 8 sub-blocks from the 12 packed bytes held in three
// words (byte i in word i / 4)
__device__ __forceinline__ void q4k_scales_w(uint32_t w0, uint32_t w1, uint32_t w2, int sc[8], int mn[8]) {
  const uint32_t wd[3] = {w0, w1, w2};
  auto by = [&](int i) { return (int)((wd[i >> 2] >> (8 * (i & 3))) & 0xffu); };
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    sc[j] = by(j) & 63;
    mn[j] = by(j + 4) & 63;
  }
#pragma unroll
  for (int j = 4; j < 8; ++j) {
    sc[j] = (by(j + 4) & 0xF) | ((by(j - 4) >> 6) << 4);
    mn[j] = (by(j + 4) >> 4) | ((by(j) >> 6) << 4);
  }
}

}  // namespace dev
}  // namespace mtg
