// oracle.cpp - CPU restatement of the reference speculative verify path.
//
// TEST INFRASTRUCTURE ONLY: the oracle libmtg's parity tests compare against, and
// the timed CPU baseline of bench.py. Nothing in the product links or loads this file.
//
// The reference executes these ops through ggml's CPU backend, which is not
// vendored in the reference tree (third_party/ggml is an empty submodule), so the
// arithmetic below restates ggml's published CPU semantics as the reference uses
// them. Where ggml's exact float summation order is not knowable here, the
// oracle uses a plain sequential order; the per-block integer dots of q8_0 and
// q4_K are exact by construction.
#include "oracle.h"

#include <omp.h>
#ifdef __AVX2__
#include <immintrin.h>
#endif

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <new>
#include <set>
#include <vector>

namespace {

// ---------------------------------------------------------------- f16 -------
// IEEE binary16 conversions, round-to-nearest-even, after the magic-number
// method published by F. Giesen ("half <-> float conversions", 2012).
uint16_t f2h(float value) {
  uint32_t u;
  std::memcpy(&u, &value, 4);
  const uint32_t sign = u & 0x80000000u;
  u ^= sign;
  uint16_t out;
  if (u >= (uint32_t)(127 + 16) << 23) {
    out = (u > 0x7f800000u) ? 0x7e00 : 0x7c00;  // NaN -> quiet NaN, overflow -> inf
  } else if (u < (uint32_t)113 << 23) {
    // Result is subnormal or zero: let an FP add align the mantissa (RNE).
    const uint32_t magic_u = (uint32_t)((127 - 15) + (23 - 10) + 1) << 23;
    float magic, f;
    std::memcpy(&magic, &magic_u, 4);
    std::memcpy(&f, &u, 4);
    f += magic;
    uint32_t r;
    std::memcpy(&r, &f, 4);
    out = (uint16_t)(r - magic_u);
  } else {
    const uint32_t mant_odd = (u >> 13) & 1u;
    u += ((uint32_t)(15 - 127) << 23) + 0xfffu;
    u += mant_odd;
    out = (uint16_t)(u >> 13);
  }
  return (uint16_t)(out | (sign >> 16));
}

float h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      exp = 127 - 15 + 1;
      while (!(man & 0x400u)) {
        man <<= 1;
        --exp;
      }
      man &= 0x3ffu;
      bits = sign | (exp << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// ------------------------------------------------------ canonical order ----
// The float operation order the oracle fixes for every reduction whose order
// ggml's SIMD code leaves machine-specific; the device kernels use the same
// order, so both sides agree bit for bit (moss-transcribe.cpp_amd/csrc/
// device_common.hpp states the same contract).

// exp: Cody-Waite reduction x = n*ln2 + r (ln2 split in two floats),
// degree-7 Taylor polynomial of e^r in Horner form with fmaf, ldexp.
float exp_c(float x) {
  if (x < -87.0f) return 0.0f;
  if (x > 88.7f) return INFINITY;
  const float n = std::nearbyint(x * 1.44269504f);
  float r = std::fma(n, -0.693145752f, x);
  r = std::fma(n, -1.42860677e-06f, r);
  float p = 1.98412698e-4f;
  p = std::fma(p, r, 1.38888889e-3f);
  p = std::fma(p, r, 8.33333333e-3f);
  p = std::fma(p, r, 4.16666667e-2f);
  p = std::fma(p, r, 1.66666667e-1f);
  p = std::fma(p, r, 0.5f);
  p = std::fma(p, r, 1.0f);
  p = std::fma(p, r, 1.0f);
  return std::ldexp(p, (int)n);
}

// xor butterfly (32, 16, 8, 4, 2, 1) over 64 partials, as a wave reduces them.
template <class F>
F butterfly64(F v[64]) {
  for (int o = 32; o > 0; o >>= 1) {
    F w[64];
    for (int l = 0; l < 64; ++l) w[l] = v[l] + v[l ^ o];
    for (int l = 0; l < 64; ++l) v[l] = w[l];
  }
  return v[0];
}

// ------------------------------------------------------------ blocks -------
#pragma pack(push, 1)
struct BlockQ8 {  // ggml block_q8_0: 34 bytes (src/cpu_q8.cpp:17 relies on it)
  uint16_t d;
  int8_t qs[32];
};
struct BlockQ8K {  // ggml block_q8_K: activation side of the q4_K dot
  float d;
  int8_t qs[256];
  int16_t bsums[16];
};
struct BlockQ4K {  // ggml block_q4_K: 144 bytes per 256 weights
  uint16_t d;
  uint16_t dmin;
  uint8_t scales[12];
  uint8_t qs[128];
};
#pragma pack(pop)
static_assert(sizeof(BlockQ8) == 34, "q8_0 block");
static_assert(sizeof(BlockQ4K) == 144, "q4_K block");

// ggml x86 CPU activation quantizer (quantize_row_q8_0, AVX path):
// amax over the block, d = amax/127 stored as f16, codes = round-half-even of
// x * (127/amax). Used by ggml_mul_mat for vec_dot_type == Q8_0
// (asserted by the reference at src/cpu_q8.cpp:23-24).
void quantize_q8_0_act(const float* x, int64_t k, BlockQ8* y) {
  for (int64_t b = 0; b < k / 32; ++b) {
    const float* v = x + b * 32;
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(v[j]));
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    y[b].d = f2h(d);
    for (int j = 0; j < 32; ++j) y[b].qs[j] = (int8_t)std::nearbyint(v[j] * id);
  }
}

// ggml quantize_row_q8_K_ref: signed max, iscale = -127/max, nearest int,
// clamp to 127, d = 1/iscale, bsums over 16-element groups.
int nearest_int(float f) {
  float val = f + 12582912.0f;
  int i;
  std::memcpy(&i, &val, 4);
  return (i & 0x007fffff) - 0x00400000;
}
void quantize_q8_k_act(const float* x, int64_t k, BlockQ8K* y) {
  for (int64_t b = 0; b < k / 256; ++b) {
    const float* v = x + b * 256;
    float max = 0.0f, amax = 0.0f;
    for (int j = 0; j < 256; ++j) {
      const float ax = std::fabs(v[j]);
      if (ax > amax) {
        amax = ax;
        max = v[j];
      }
    }
    if (amax == 0.0f) {
      y[b].d = 0.0f;
      std::memset(y[b].qs, 0, 256);
      std::memset(y[b].bsums, 0, sizeof(y[b].bsums));
      continue;
    }
    const float iscale = -127.0f / max;
    for (int j = 0; j < 256; ++j) y[b].qs[j] = (int8_t)std::min(127, nearest_int(iscale * v[j]));
    for (int g = 0; g < 16; ++g) {
      int s = 0;
      for (int i = 0; i < 16; ++i) s += y[b].qs[g * 16 + i];
      y[b].bsums[g] = (int16_t)s;
    }
    y[b].d = 1.0f / iscale;
  }
}

// q4_K 6-bit scale/min unpacking (GGUF q4_K format, get_scale_min_k4).
void q4k_scale_min(int j, const uint8_t* q, int* sc, int* mn) {
  if (j < 4) {
    *sc = q[j] & 63;
    *mn = q[j + 4] & 63;
  } else {
    *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    *mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

int32_t q8_block_dot(const BlockQ8& a, const BlockQ8& b) {
  int32_t s = 0;
  for (int j = 0; j < 32; ++j) s += (int32_t)a.qs[j] * (int32_t)b.qs[j];
  return s;
}

// Exact int32 dots of nb consecutive 32-element int8 blocks (any order of the
// integer adds gives the same sum). With AVX2: |w| (as unsigned) times x with
// w's sign by vpmaddubsw (a pair sum is at most 2 * 128 * 127, no saturation:
// activation codes lie in [-127, 127]), vpmaddwd to int32, then eight blocks'
// horizontal sums at once.
void block_dots(const int8_t* w, const int8_t* x, int nb, int32_t* out) {
  int b = 0;
#ifdef __AVX2__
  const __m256i ones = _mm256_set1_epi16(1);
  for (; b + 8 <= nb; b += 8) {
    __m256i s[8];
    for (int i = 0; i < 8; ++i) {
      const __m256i wv = _mm256_loadu_si256((const __m256i*)(w + (size_t)(b + i) * 32));
      const __m256i xv = _mm256_loadu_si256((const __m256i*)(x + (size_t)(b + i) * 32));
      const __m256i p = _mm256_maddubs_epi16(_mm256_sign_epi8(wv, wv), _mm256_sign_epi8(xv, wv));
      s[i] = _mm256_madd_epi16(p, ones);
    }
    const __m256i h01 = _mm256_hadd_epi32(s[0], s[1]), h23 = _mm256_hadd_epi32(s[2], s[3]);
    const __m256i h45 = _mm256_hadd_epi32(s[4], s[5]), h67 = _mm256_hadd_epi32(s[6], s[7]);
    const __m256i h0123 = _mm256_hadd_epi32(h01, h23), h4567 = _mm256_hadd_epi32(h45, h67);
    // lanes: [0123 low halves | 0123 high halves], the same for 4567
    const __m256i lo = _mm256_permute2x128_si256(h0123, h4567, 0x20);
    const __m256i hi = _mm256_permute2x128_si256(h0123, h4567, 0x31);
    _mm256_storeu_si256((__m256i*)(out + b), _mm256_add_epi32(lo, hi));
  }
#endif
  for (; b < nb; ++b) {
    int32_t s = 0;
    for (int j = 0; j < 32; ++j) s += (int32_t)w[(size_t)b * 32 + j] * (int32_t)x[(size_t)b * 32 + j];
    out[b] = s;
  }
}

// mul_mat(q8_0 W, f32 x) as ggml runs it: x quantized to q8_0, then
// y = sum over blocks of (d_w * d_x) * isum with an exact int32 isum per
// 32-block. Canonical float order: K in 4 slices of block pairs, even and odd
// blocks in separate fma chains per slice, slices added in order, even + odd.
void mul_mat_q8(const BlockQ8* w, int k, int n, const float* x, int T, float* y) {
  const int nb = k / 32, bps = nb / 2;
  std::vector<BlockQ8> xq((size_t)T * nb);
  for (int t = 0; t < T; ++t) quantize_q8_0_act(x + (size_t)t * k, k, xq.data() + (size_t)t * nb);
  // activation codes and scales unpacked once; per row the weight codes and
  // scales once, the exact int32 block sums of every row t, then the chains
  std::vector<int8_t> xc((size_t)T * k);
  std::vector<float> xd((size_t)T * nb);
  for (size_t i = 0; i < xq.size(); ++i) {
    std::memcpy(&xc[i * 32], xq[i].qs, 32);
    xd[i] = h2f(xq[i].d);
  }
#pragma omp parallel
  {
    std::vector<int8_t> wc(k);
    std::vector<float> wd(nb);
    std::vector<int32_t> isum((size_t)T * nb);
#pragma omp for schedule(static)
    for (int r = 0; r < n; ++r) {
      const BlockQ8* wr = w + (size_t)r * nb;
      for (int b = 0; b < nb; ++b) {
        std::memcpy(&wc[(size_t)b * 32], wr[b].qs, 32);
        wd[b] = h2f(wr[b].d);
      }
      for (int t = 0; t < T; ++t) block_dots(wc.data(), &xc[(size_t)t * k], nb, &isum[(size_t)t * nb]);
      for (int t = 0; t < T; ++t) {
        const float* xdt = &xd[(size_t)t * nb];
        const int32_t* is = &isum[(size_t)t * nb];
        float e[4], o[4];
        for (int sl = 0; sl < 4; ++sl) {
          e[sl] = o[sl] = 0.0f;
          for (int bp = (bps * sl) / 4; bp < (bps * (sl + 1)) / 4; ++bp) {
            const int b0 = 2 * bp, b1 = 2 * bp + 1;
            e[sl] = std::fma((float)is[b0], wd[b0] * xdt[b0], e[sl]);
            o[sl] = std::fma((float)is[b1], wd[b1] * xdt[b1], o[sl]);
          }
        }
        const float ev = ((e[0] + e[1]) + e[2]) + e[3];
        const float ov = ((o[0] + o[1]) + o[2]) + o[3];
        y[(size_t)t * n + r] = ev + ov;
      }
    }
  }
}

// mul_mat(f16 W, f32 x): x converted to f16 (vec_dot_type F16), f32 accumulation
// (ggml vec_dot_f16). Canonical order: K in 64 consecutive segments, each an fma
// chain from 0 (a product of two f16 values is exact in f32), the 64 partials
// reduced by the xor butterfly. ggml's own SIMD order is not pinned.
void mul_mat_f16(const uint16_t* w, int k, int n, const float* x, int T, float* y) {
  std::vector<float> xh((size_t)T * k);
  for (size_t i = 0; i < xh.size(); ++i) xh[i] = h2f(f2h(x[i]));
  const int seg = k / 64;
#pragma omp parallel
  {
    std::vector<float> wf(k);  // the row decoded once
#pragma omp for schedule(static)
    for (int r = 0; r < n; ++r) {
      const uint16_t* wr = w + (size_t)r * k;
      for (int i = 0; i < k; ++i) wf[i] = h2f(wr[i]);
      for (int t = 0; t < T; ++t) {
        const float* xr = xh.data() + (size_t)t * k;
        float part[64];
        for (int l = 0; l < 64; ++l) {
          float acc = 0.0f;
          for (int e = 0; e < seg; ++e) acc = std::fma(wf[l * seg + e], xr[l * seg + e], acc);
          part[l] = acc;
        }
        y[(size_t)t * n + r] = butterfly64(part);
      }
    }
  }
}

// mul_mat(f32 W, f32 x): vec_dot_type F32, x as it is (ggml vec_dot_f32).
// Canonical order: the f16 one's segments and butterfly, each segment an fma
// chain from 0 (every step rounds once: fma(w, x, acc)).
void mul_mat_f32(const float* w, int k, int n, const float* x, int T, float* y) {
  const int seg = k / 64;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < n; ++r) {
    const float* wr = w + (size_t)r * k;
    for (int t = 0; t < T; ++t) {
      const float* xr = x + (size_t)t * k;
      float part[64];
      for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int e = 0; e < seg; ++e) acc = std::fma(wr[l * seg + e], xr[l * seg + e], acc);
        part[l] = acc;
      }
      y[(size_t)t * n + r] = butterfly64(part);
    }
  }
}

// mul_mat(q4_K W, f32 x): x quantized to q8_K; per 256-superblock exact int32
// sums sum_j sc_j * dot_j and sum_j mn_j * bsum_j, combined as
// (d_w*d_x)*dot - (dmin_w*d_x)*min.
void mul_mat_q4k(const BlockQ4K* w, int k, int n, const float* x, int T, float* y) {
  const int nb = k / 256;
  std::vector<BlockQ8K> xq((size_t)T * nb);
  for (int t = 0; t < T; ++t) quantize_q8_k_act(x + (size_t)t * k, k, xq.data() + (size_t)t * nb);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < n; ++r) {
    const BlockQ4K* wr = w + (size_t)r * nb;
    for (int t = 0; t < T; ++t) {
      const BlockQ8K* xr = xq.data() + (size_t)t * nb;
      float acc = 0.0f;
      for (int b = 0; b < nb; ++b) {
        int32_t dot = 0, mins = 0;
        for (int s = 0; s < 8; ++s) {
          int sc, mn;
          q4k_scale_min(s, wr[b].scales, &sc, &mn);
          const uint8_t* q = wr[b].qs + (s / 2) * 32;
          int32_t sub = 0;
          for (int l = 0; l < 32; ++l) {
            const int v = (s & 1) ? (q[l] >> 4) : (q[l] & 0xF);
            sub += v * xr[b].qs[s * 32 + l];
          }
          dot += sc * sub;
          mins += mn * (xr[b].bsums[2 * s] + xr[b].bsums[2 * s + 1]);
        }
        const float d = h2f(wr[b].d) * xr[b].d;
        const float dmin = h2f(wr[b].dmin) * xr[b].d;
        acc += d * (float)dot;
        acc -= dmin * (float)mins;
      }
      y[(size_t)t * n + r] = acc;
    }
  }
}

void mul_mat(int wtype, const void* w, int k, int n, const float* x, int T, float* y) {
  if (wtype == MTG_TYPE_Q8_0) mul_mat_q8((const BlockQ8*)w, k, n, x, T, y);
  else if (wtype == MTG_TYPE_F16) mul_mat_f16((const uint16_t*)w, k, n, x, T, y);
  else if (wtype == MTG_TYPE_F32) mul_mat_f32((const float*)w, k, n, x, T, y);
  else mul_mat_q4k((const BlockQ4K*)w, k, n, x, T, y);
}

// ggml_rms_norm (x*x in float, summed in double, mean cast to float,
// 1/sqrtf), then ggml_mul by the gain as a separate op (src/qwen3.cpp:27-30).
// Canonical double-sum order: 64 partials (16 consecutive elements each for a
// 1024 row; elements l and l+64 for a 128 head) reduced by the butterfly.
double sum_squares(const float* x, int n) {
  double part[64];
  if (n == 1024) {
    for (int l = 0; l < 64; ++l) {
      double s = 0.0;
      for (int e = 0; e < 16; ++e) s += (double)(x[16 * l + e] * x[16 * l + e]);
      part[l] = s;
    }
    return butterfly64(part);
  }
  if (n == 128) {
    for (int l = 0; l < 64; ++l) part[l] = (double)(x[l] * x[l]) + (double)(x[l + 64] * x[l + 64]);
    return butterfly64(part);
  }
  double s = 0.0;
  for (int i = 0; i < n; ++i) s += (double)(x[i] * x[i]);
  return s;
}

void rms_norm(const float* x, const float* w, int n, float eps, float* y) {
  const float mean = (float)(sum_squares(x, n) / n);
  const float scale = 1.0f / std::sqrt(mean + eps);
  for (int i = 0; i < n; ++i) {
    const float v = x[i] * scale;
    y[i] = v * w[i];
  }
}

// ------------------------------------------------- ggml generic order ------
// The second order of the oracle (orc_set_order(m, ORC_ORDER_GGML_GENERIC)):
// the float order of ggml's generic (scalar) CPU kernels, the portable C path of
// the same ops (the reference's Xeon runs ggml's x86 SIMD kernels, whose order is
// machine-specific and not reproducible here). Integer block dots stay exact;
// what changes is every float reduction: sequential block sums, double
// accumulation where ggml's scalar code accumulates in double, soft_max_ext over
// the common length with the causal mask, and the context at each query's valid
// length (src/qwen3.cpp:157-189, src/cpu_context.cpp:13-32). It measures how far
// the canonical order is from an independent, published one.

// ggml_vec_dot_q8_0_q8_0 (generic): sumf += (float)isum * (d_w * d_x), block by block.
void mul_mat_q8_generic(const BlockQ8* w, int k, int n, const float* x, int T, float* y) {
  const int nb = k / 32;
  std::vector<BlockQ8> xq((size_t)T * nb);
  for (int t = 0; t < T; ++t) quantize_q8_0_act(x + (size_t)t * k, k, xq.data() + (size_t)t * nb);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < n; ++r) {
    const BlockQ8* wr = w + (size_t)r * nb;
    for (int t = 0; t < T; ++t) {
      const BlockQ8* xr = xq.data() + (size_t)t * nb;
      float sumf = 0.0f;
      for (int b = 0; b < nb; ++b) {
        const float isum = (float)q8_block_dot(wr[b], xr[b]);
        sumf = sumf + isum * (h2f(wr[b].d) * h2f(xr[b].d));
      }
      y[(size_t)t * n + r] = sumf;
    }
  }
}

// ggml_vec_dot_f16 (generic): x rounded to f16, sum of (double)(w * x) in order.
void mul_mat_f16_generic(const uint16_t* w, int k, int n, const float* x, int T, float* y) {
  std::vector<float> xh((size_t)T * k);
  for (size_t i = 0; i < xh.size(); ++i) xh[i] = h2f(f2h(x[i]));
#pragma omp parallel for schedule(static)
  for (int r = 0; r < n; ++r) {
    const uint16_t* wr = w + (size_t)r * k;
    for (int t = 0; t < T; ++t) {
      const float* xr = xh.data() + (size_t)t * k;
      double sumf = 0.0;
      for (int i = 0; i < k; ++i) sumf += (double)(h2f(wr[i]) * xr[i]);
      y[(size_t)t * n + r] = (float)sumf;
    }
  }
}

// ggml_vec_dot_q4_K_q8_K (generic): per superblock eight int32 lane sums
// aux[l] = sum over sub-blocks j and 8-element groups g of sc_j * q4 * q8 at
// element 32 j + 8 g + l; sums[l] += d * aux[l] (float, d = d_w * d_x);
// sumf -= dmin * sum_j bsum_j * mn_(j/2); at the end sumf += sums[0..7].
void mul_mat_q4k_generic(const BlockQ4K* w, int k, int n, const float* x, int T, float* y) {
  const int nb = k / 256;
  std::vector<BlockQ8K> xq((size_t)T * nb);
  for (int t = 0; t < T; ++t) quantize_q8_k_act(x + (size_t)t * k, k, xq.data() + (size_t)t * nb);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < n; ++r) {
    const BlockQ4K* wr = w + (size_t)r * nb;
    for (int t = 0; t < T; ++t) {
      const BlockQ8K* xr = xq.data() + (size_t)t * nb;
      float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      float sumf = 0.0f;
      for (int b = 0; b < nb; ++b) {
        int32_t aux[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int32_t sumi = 0;
        for (int s = 0; s < 8; ++s) {
          int sc, mn;
          q4k_scale_min(s, wr[b].scales, &sc, &mn);
          sumi += (xr[b].bsums[2 * s] + xr[b].bsums[2 * s + 1]) * mn;
          const uint8_t* q = wr[b].qs + (s / 2) * 32;
          for (int g = 0; g < 4; ++g)
            for (int l = 0; l < 8; ++l) {
              const int e = 8 * g + l;
              const int v = (s & 1) ? (q[e] >> 4) : (q[e] & 0xF);
              aux[l] += sc * (v * xr[b].qs[s * 32 + e]);
            }
        }
        const float d = h2f(wr[b].d) * xr[b].d;
        for (int l = 0; l < 8; ++l) sums[l] = sums[l] + d * (float)aux[l];
        const float dmin = h2f(wr[b].dmin) * xr[b].d;
        sumf = sumf - dmin * (float)sumi;
      }
      for (int l = 0; l < 8; ++l) sumf = sumf + sums[l];
      y[(size_t)t * n + r] = sumf;
    }
  }
}

// ggml_vec_dot_f32 (generic): sum of (double)(w * x) in order.
void mul_mat_f32_generic(const float* w, int k, int n, const float* x, int T, float* y) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < n; ++r) {
    const float* wr = w + (size_t)r * k;
    for (int t = 0; t < T; ++t) {
      const float* xr = x + (size_t)t * k;
      double sumf = 0.0;
      for (int i = 0; i < k; ++i) sumf += (double)(wr[i] * xr[i]);
      y[(size_t)t * n + r] = (float)sumf;
    }
  }
}

void mul_mat_generic(int wtype, const void* w, int k, int n, const float* x, int T, float* y) {
  if (wtype == MTG_TYPE_Q8_0) mul_mat_q8_generic((const BlockQ8*)w, k, n, x, T, y);
  else if (wtype == MTG_TYPE_F16) mul_mat_f16_generic((const uint16_t*)w, k, n, x, T, y);
  else if (wtype == MTG_TYPE_F32) mul_mat_f32_generic((const float*)w, k, n, x, T, y);
  else mul_mat_q4k_generic((const BlockQ4K*)w, k, n, x, T, y);
}

// ggml_compute_forward_rms_norm_f32 (generic): sum of (double)(x*x) in order,
// mean = (float)(sum / n), scale = 1.0f / sqrtf(mean + eps), y = x * scale; then
// ggml_mul by the gain (src/qwen3.cpp:27-30).
void rms_norm_generic(const float* x, const float* w, int n, float eps, float* y) {
  double sum = 0.0;
  for (int i = 0; i < n; ++i) sum += (double)(x[i] * x[i]);
  const float mean = (float)(sum / n);
  const float scale = 1.0f / std::sqrt(mean + eps);
  for (int i = 0; i < n; ++i) {
    const float v = x[i] * scale;
    y[i] = v * w[i];
  }
}

// NEOX RoPE as ggml_rope_ext builds it (src/qwen3.cpp:108-118, mode NEOX):
// theta_scale = powf(base, -2/n_dims); theta_0 = pos, theta_{i+1} = theta_i *
// theta_scale in float; pairs (i, i + n_dims/2); ext_factor 0, attn_factor 1.
void rope_table(int pos, int n_dims, float base, float* cs) {
  const float theta_scale = std::pow(base, -2.0f / (float)n_dims);
  float theta = (float)pos;
  for (int i = 0; i < n_dims / 2; ++i) {
    cs[2 * i] = std::cos(theta);
    cs[2 * i + 1] = std::sin(theta);
    theta *= theta_scale;
  }
}
void rope_apply(float* x, int n_dims, const float* cs) {
  const int half = n_dims / 2;
  for (int i = 0; i < half; ++i) {
    const float x0 = x[i], x1 = x[i + half];
    const float c = cs[2 * i], s = cs[2 * i + 1];
    x[i] = x0 * c - x1 * s;
    x[i + half] = x0 * s + x1 * c;
  }
}

// ggml_soft_max_ext(scores, mask, scale) row: scale, add mask, max, expf and a
// double sum, multiply by (float)(1/sum) (op order of src/cpu_softmax.cpp:27-36
// with the mask add of soft_max_ext).
void softmax_row(const float* s, int n, float scale, const float* mask, float* out) {
  std::vector<float> w(n);
  for (int i = 0; i < n; ++i) {
    w[i] = s[i] * scale;
    if (mask) w[i] += mask[i];
  }
  float max = -INFINITY;
  for (int i = 0; i < n; ++i) max = std::max(max, w[i]);
  double sum = 0.0;
  for (int i = 0; i < n; ++i) {
    const float e = std::exp(w[i] - max);
    sum += (double)e;
    out[i] = e;
  }
  const float inv = (float)(1.0 / sum);
  for (int i = 0; i < n; ++i) out[i] *= inv;
}

float swiglu(float g, float u) { return (g / (1.0f + exp_c(-g))) * u; }
// ggml_silu_f32 (x / (1 + expf(-x))) times up, with the C library's expf.
float swiglu_generic(float g, float u) { return (g / (1.0f + std::exp(-g))) * u; }

}  // namespace

// ------------------------------------------------------------- model -------
struct orc_model {
  mtg_hparams hp{};
  int wtype = MTG_TYPE_Q8_0;
  int kv_type = MTG_TYPE_F32;
  int max_seq = 0, past = 0;
  int order = ORC_ORDER_CANONICAL;  // float order of every reduction (orc_set_order)
  std::vector<std::vector<uint8_t>> wq, wk, wv, wo, wg, wu, wd;
  std::vector<std::vector<float>> attn_norm, q_norm, k_norm, ffn_norm;
  std::vector<uint8_t> embd;
  std::vector<float> out_norm;
  // KV cache [layer][kv_head][pos][head_dim], f32 or f16 bits.
  std::vector<float> k32, v32;
  std::vector<uint16_t> k16, v16;
  size_t layer_stride = 0;  // elements per layer
};

namespace {
size_t row_bytes(int type, int64_t k) {
  if (type == MTG_TYPE_Q8_0) return (size_t)(k / 32) * 34;
  if (type == MTG_TYPE_F16) return (size_t)k * 2;
  if (type == MTG_TYPE_Q4_K) return (size_t)(k / 256) * 144;
  return (size_t)k * 4;
}
std::vector<uint8_t> copy_matrix(const void* p, int type, int64_t k, int64_t n) {
  const size_t bytes = row_bytes(type, k) * (size_t)n;
  std::vector<uint8_t> v(bytes);
  std::memcpy(v.data(), p, bytes);
  return v;
}

void embed_row(const orc_model& m, int32_t id, float* out) {
  const int H = m.hp.hidden;
  const uint8_t* row = m.embd.data() + row_bytes(m.wtype, H) * (size_t)id;
  if (m.wtype == MTG_TYPE_Q8_0) {
    const BlockQ8* b = (const BlockQ8*)row;
    for (int i = 0; i < H; ++i) out[i] = h2f(b[i / 32].d) * (float)b[i / 32].qs[i % 32];
  } else if (m.wtype == MTG_TYPE_F16) {
    const uint16_t* h = (const uint16_t*)row;
    for (int i = 0; i < H; ++i) out[i] = h2f(h[i]);
  } else if (m.wtype == MTG_TYPE_F32) {
    std::memcpy(out, row, (size_t)H * 4);
  } else {
    const BlockQ4K* b = (const BlockQ4K*)row;
    for (int sb = 0; sb < H / 256; ++sb) {
      const float d = h2f(b[sb].d), dmin = h2f(b[sb].dmin);
      for (int s = 0; s < 8; ++s) {
        int sc, mn;
        q4k_scale_min(s, b[sb].scales, &sc, &mn);
        const float d1 = d * (float)sc, m1 = dmin * (float)mn;
        const uint8_t* q = b[sb].qs + (s / 2) * 32;
        for (int l = 0; l < 32; ++l) {
          const int v = (s & 1) ? (q[l] >> 4) : (q[l] & 0xF);
          out[sb * 256 + s * 32 + l] = d1 * (float)v - m1;
        }
      }
    }
  }
}

inline float kv_get(const orc_model& m, bool is_k, size_t idx) {
  if (m.kv_type == MTG_TYPE_F32) return is_k ? m.k32[idx] : m.v32[idx];
  return h2f(is_k ? m.k16[idx] : m.v16[idx]);
}
inline void kv_set(orc_model& m, bool is_k, size_t idx, float v) {
  if (m.kv_type == MTG_TYPE_F32) (is_k ? m.k32 : m.v32)[idx] = v;
  else (is_k ? m.k16 : m.v16)[idx] = f2h(v);  // ggml_cpy f32 -> f16
}

void norm_op(const orc_model& m, const float* x, const float* w, int n, float* y) {
  if (m.order == ORC_ORDER_GGML_GENERIC) rms_norm_generic(x, w, n, m.hp.rms_eps, y);
  else rms_norm(x, w, n, m.hp.rms_eps, y);
}
void gemm_op(const orc_model& m, const void* w, int k, int n, const float* x, int T, float* y) {
  if (m.order == ORC_ORDER_GGML_GENERIC) mul_mat_generic(m.wtype, w, k, n, x, T, y);
  else mul_mat(m.wtype, w, k, n, x, T, y);
}

// The eager attention in ggml's generic order (src/qwen3.cpp:157-189): scores
// = mul_mat(K, q) with ggml_vec_dot_f32 (double accumulation; an f16 cache takes
// q rounded to f16 and ggml_vec_dot_f16), soft_max_ext(scores, mask, 1/sqrt(D))
// over the common length past + T with the causal mask (0 / -inf), then
// cpu_causal_context: out[f] = dot(V[0..past+t][f], P[t][0..past+t]) at the
// valid length (src/cpu_context.cpp:13-32), again a double-accumulated dot.
void attention_generic(const orc_model& m, int l, const float* q, int T, float* o) {
  const mtg_hparams& hp = m.hp;
  const int D = hp.head_dim, NH = hp.n_heads, NKV = hp.n_kv_heads, QN = NH * D;
  const int past = m.past, kv = past + T, groups = NH / NKV;
  const size_t base = (size_t)l * m.layer_stride;
  const bool f16kv = m.kv_type == MTG_TYPE_F16;
  const float scale = 1.0f / std::sqrt((float)D);
#pragma omp parallel for collapse(2) schedule(static)
  for (int h = 0; h < NH; ++h)
    for (int t = 0; t < T; ++t) {
      const int g = h / groups;
      std::vector<float> qv(D), sc(kv), mask(kv), p(kv);
      const float* qh = q + (size_t)t * QN + (size_t)h * D;
      for (int d = 0; d < D; ++d) qv[d] = f16kv ? h2f(f2h(qh[d])) : qh[d];
      for (int j = 0; j < kv; ++j) {
        const size_t kb = base + ((size_t)g * m.max_seq + j) * D;
        double acc = 0.0;
        for (int d = 0; d < D; ++d) acc += (double)(kv_get(m, true, kb + d) * qv[d]);
        sc[j] = (float)acc;
        mask[j] = j <= past + t ? 0.0f : -INFINITY;
      }
      softmax_row(sc.data(), kv, scale, mask.data(), p.data());
      if (f16kv)
        for (int j = 0; j < kv; ++j) p[j] = h2f(f2h(p[j]));
      float* oh = o + (size_t)t * QN + (size_t)h * D;
      const int valid = past + t + 1;
      for (int d = 0; d < D; ++d) {
        double acc = 0.0;
        for (int j = 0; j < valid; ++j)
          acc += (double)(kv_get(m, false, base + ((size_t)g * m.max_seq + j) * D + d) * p[j]);
        oh[d] = (float)acc;
      }
    }
}

// Eager GQA attention of T query rows at positions past .. past + T - 1 over a
// cache of NKV heads x max_seq positions x D (f32, or f16 bits when f16kv)
// holding keys [0, past + T): scores K.Q in f32, soft_max_ext(scale 1/sqrt(D),
// causal mask), context over each query's valid length (src/qwen3.cpp:157-189,
// src/cpu_context.cpp:13-32). q, o: [T][NH * D]. Canonical order: keys in chunks
// of 64; score = fma chain over D; per chunk max, p = exp(w - max) (f16-rounded
// for an f16 cache, whose q is f16-rounded too), l = butterfly sum of p, O = fma
// chain over the chunk's keys; the chunks merged in order: M = max of the chunk
// maxima, f = exp(m_c - M), L = fma(l_c, f, L), O = fma(O_c, f, O), out = O / L.
void attention_canonical(const void* kc, const void* vc, bool f16kv, int max_seq, int past, int T, int NH, int NKV,
                         int D, const float* q, float* o) {
  const int QN = NH * D, groups = NH / NKV, kv = past + T;
  const float scale = 1.0f / std::sqrt((float)D);
  const int nch = (kv + 63) / 64;
  const float* k32 = (const float*)kc;
  const float* v32 = (const float*)vc;
  const uint16_t* k16 = (const uint16_t*)kc;
  const uint16_t* v16 = (const uint16_t*)vc;
  // per (kv head, chunk): the chunk's K transposed ([d][key]) and V ([key][d])
  // decoded once, zeros past kv, then every query of the kv head: the chains
  // run over d (scores) and over the keys (P.V) in order, 64 scores or D
  // outputs side by side; then per (head, row) the chunks merged in order
  std::vector<float> qv((size_t)T * QN);
  for (size_t i = 0; i < qv.size(); ++i) qv[i] = f16kv ? h2f(f2h(q[i])) : q[i];
  std::vector<float> cm((size_t)NH * T * nch), cl((size_t)NH * T * nch), co((size_t)NH * T * nch * D);
#pragma omp parallel
  {
    std::vector<float> kt((size_t)D * 64), vt((size_t)64 * D);
#pragma omp for collapse(2) schedule(dynamic)
    for (int g = 0; g < NKV; ++g)
      for (int c = 0; c < nch; ++c) {
        float* __restrict__ ktp = kt.data();
        float* __restrict__ vcp = vt.data();
        for (int j = 0; j < 64; ++j) {
          const int key = 64 * c + j;
          const size_t kb = ((size_t)g * max_seq + key) * D;
          if (key >= kv) {
            for (int d = 0; d < D; ++d) ktp[(size_t)d * 64 + j] = vcp[(size_t)j * D + d] = 0.0f;
          } else if (!f16kv) {
            for (int d = 0; d < D; ++d) {
              ktp[(size_t)d * 64 + j] = k32[kb + d];
              vcp[(size_t)j * D + d] = v32[kb + d];
            }
          } else {
            for (int d = 0; d < D; ++d) {
              ktp[(size_t)d * 64 + j] = h2f(k16[kb + d]);
              vcp[(size_t)j * D + d] = h2f(v16[kb + d]);
            }
          }
        }
        for (int h = g * groups; h < (g + 1) * groups; ++h)
          for (int t = 0; t < T; ++t) {
            const float* qh = &qv[(size_t)t * QN + (size_t)h * D];
            float s[64], w[64], p[64];
            for (int j = 0; j < 64; ++j) s[j] = 0.0f;
            for (int d = 0; d < D; ++d) {
              const float qd = qh[d];
              const float* __restrict__ kd = ktp + (size_t)d * 64;
              for (int j = 0; j < 64; ++j) s[j] = std::fma(qd, kd[j], s[j]);
            }
            float mx = -INFINITY;
            for (int j = 0; j < 64; ++j) {
              const int key = 64 * c + j;
              w[j] = (key < kv && key <= past + t) ? s[j] * scale : -INFINITY;
              mx = std::max(mx, w[j]);
            }
            for (int j = 0; j < 64; ++j) {
              p[j] = (mx == -INFINITY || w[j] == -INFINITY) ? 0.0f : exp_c(w[j] - mx);
              if (f16kv) p[j] = h2f(f2h(p[j]));
            }
            float pl[64];
            std::memcpy(pl, p, sizeof(pl));
            const size_t it = ((size_t)h * T + t) * nch + c;
            cm[it] = mx;
            cl[it] = butterfly64(pl);
            float* __restrict__ oc = &co[it * D];
            for (int d = 0; d < D; ++d) oc[d] = 0.0f;
            for (int j = 0; j < 64; ++j) {
              const float pj = p[j];
              const float* __restrict__ vj = vcp + (size_t)j * D;
              for (int d = 0; d < D; ++d) oc[d] = std::fma(pj, vj[d], oc[d]);
            }
          }
      }
  }
#pragma omp parallel for collapse(2) schedule(static)
  for (int h = 0; h < NH; ++h)
    for (int t = 0; t < T; ++t) {
      const size_t i0 = ((size_t)h * T + t) * nch;
      float M = -INFINITY;
      for (int c = 0; c < nch; ++c) M = std::max(M, cm[i0 + c]);
      float* oh = o + (size_t)t * QN + (size_t)h * D;
      for (int d = 0; d < D; ++d) {
        float L = 0.0f, acc = 0.0f;
        for (int c = 0; c < nch; ++c) {
          if (cm[i0 + c] == -INFINITY) continue;
          const float f = exp_c(cm[i0 + c] - M);
          L = std::fma(cl[i0 + c], f, L);
          acc = std::fma(co[(i0 + c) * D + d], f, acc);
        }
        oh[d] = acc / L;
      }
    }
}

// One qwen3_layer_forward over T rows at positions past..past+T-1
// (src/qwen3.cpp:62-218 with the device-cache path, transposed-V semantics and
// the causal-context op of src/cpu_context.cpp:13-32).
void layer_forward(orc_model& m, int l, float* x, int T) {
  const mtg_hparams& hp = m.hp;
  const int H = hp.hidden, D = hp.head_dim, NH = hp.n_heads, NKV = hp.n_kv_heads;
  const int QN = NH * D, KN = NKV * D, F = hp.intermediate;
  const int past = m.past;
  std::vector<float> xn((size_t)T * H), q((size_t)T * QN), k((size_t)T * KN), v((size_t)T * KN);
  for (int t = 0; t < T; ++t) norm_op(m, x + (size_t)t * H, m.attn_norm[l].data(), H, xn.data() + (size_t)t * H);
  gemm_op(m, m.wq[l].data(), H, QN, xn.data(), T, q.data());
  gemm_op(m, m.wk[l].data(), H, KN, xn.data(), T, k.data());
  gemm_op(m, m.wv[l].data(), H, KN, xn.data(), T, v.data());
  // per-head q/k RMSNorm over head_dim, then NEOX RoPE at pos = past + t
  std::vector<float> cs(D);
  std::vector<float> tmp(D);
  for (int t = 0; t < T; ++t) {
    rope_table(past + t, D, hp.rope_base, cs.data());
    for (int h = 0; h < NH; ++h) {
      float* qh = q.data() + (size_t)t * QN + (size_t)h * D;
      norm_op(m, qh, m.q_norm[l].data(), D, tmp.data());
      rope_apply(tmp.data(), D, cs.data());
      std::memcpy(qh, tmp.data(), D * sizeof(float));
    }
    for (int h = 0; h < NKV; ++h) {
      float* kh = k.data() + (size_t)t * KN + (size_t)h * D;
      norm_op(m, kh, m.k_norm[l].data(), D, tmp.data());
      rope_apply(tmp.data(), D, cs.data());
      std::memcpy(kh, tmp.data(), D * sizeof(float));
    }
  }
  // KV store at past (src/qwen3.cpp:123-139)
  const size_t base = (size_t)l * m.layer_stride;
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < NKV; ++h)
      for (int d = 0; d < D; ++d) {
        const size_t idx = base + ((size_t)h * m.max_seq + (size_t)(past + t)) * D + d;
        kv_set(m, true, idx, k[(size_t)t * KN + (size_t)h * D + d]);
        kv_set(m, false, idx, v[(size_t)t * KN + (size_t)h * D + d]);
      }
  // eager GQA attention (src/qwen3.cpp:157-189)
  std::vector<float> o((size_t)T * QN);
  if (m.order == ORC_ORDER_GGML_GENERIC) {
    attention_generic(m, l, q.data(), T, o.data());
  } else {
    const bool f16kv = m.kv_type == MTG_TYPE_F16;
    const void* kc = f16kv ? (const void*)(m.k16.data() + base) : (const void*)(m.k32.data() + base);
    const void* vc = f16kv ? (const void*)(m.v16.data() + base) : (const void*)(m.v32.data() + base);
    attention_canonical(kc, vc, f16kv, m.max_seq, past, T, NH, NKV, D, q.data(), o.data());
  }
  // o-proj + residual, FFN pre-norm, SwiGLU, down + residual
  std::vector<float> ao((size_t)T * H);
  gemm_op(m, m.wo[l].data(), QN, H, o.data(), T, ao.data());
  for (size_t i = 0; i < (size_t)T * H; ++i) x[i] = x[i] + ao[i];
  for (int t = 0; t < T; ++t) norm_op(m, x + (size_t)t * H, m.ffn_norm[l].data(), H, xn.data() + (size_t)t * H);
  std::vector<float> g((size_t)T * F), u((size_t)T * F), act((size_t)T * F);
  gemm_op(m, m.wg[l].data(), H, F, xn.data(), T, g.data());
  gemm_op(m, m.wu[l].data(), H, F, xn.data(), T, u.data());
  const bool generic = m.order == ORC_ORDER_GGML_GENERIC;
  for (size_t i = 0; i < act.size(); ++i) act[i] = generic ? swiglu_generic(g[i], u[i]) : swiglu(g[i], u[i]);
  gemm_op(m, m.wd[l].data(), F, H, act.data(), T, ao.data());
  for (size_t i = 0; i < (size_t)T * H; ++i) x[i] = x[i] + ao[i];
}

}  // namespace

extern "C" {

uint16_t orc_f32_to_f16(float f) { return f2h(f); }
float orc_exp(float x) { return exp_c(x); }
float orc_f16_to_f32(uint16_t h) { return h2f(h); }
void orc_quantize_q8_0_act(const float* x, int64_t k, void* blocks) {
  quantize_q8_0_act(x, k, (BlockQ8*)blocks);
}
void orc_quantize_q8_k_act(const float* x, int64_t k, void* blocks) {
  quantize_q8_k_act(x, k, (BlockQ8K*)blocks);
}
int32_t orc_q8_0_block_dot(const void* a, const void* b) {
  return q8_block_dot(*(const BlockQ8*)a, *(const BlockQ8*)b);
}
void orc_q8_0_block_dots(const int8_t* w, const int8_t* x, int32_t nb, int32_t* out) {
  block_dots(w, x, nb, out);
}
void orc_mul_mat(int32_t wtype, const void* w, int32_t k, int32_t n, const float* x, int32_t T,
                 float* y) {
  mul_mat(wtype, w, k, n, x, T, y);
}
void orc_mul_mat_generic(int32_t wtype, const void* w, int32_t k, int32_t n, const float* x, int32_t T,
                         float* y) {
  mul_mat_generic(wtype, w, k, n, x, T, y);
}
void orc_rms_norm(const float* x, const float* w, int32_t n, float eps, float* y) {
  rms_norm(x, w, n, eps, y);
}
void orc_rope_neox(float* x, int32_t n_dims, int32_t pos, float base) {
  std::vector<float> cs(n_dims);
  rope_table(pos, n_dims, base, cs.data());
  rope_apply(x, n_dims, cs.data());
}
void orc_softmax(const float* s, int32_t n, float scale, const float* mask, float* out) {
  softmax_row(s, n, scale, mask, out);
}
// cpu_causal_context (src/cpu_context.cpp:13-32): out[h][q][f] =
// sum_{k < past+q+1} v[h/groups][k][f] * p[h][q][k], exactly the valid length.
void orc_causal_context(const float* v, const float* p, int32_t head_dim, int32_t kv_heads,
                        int32_t heads, int32_t queries, int32_t kv_len, float* out) {
  const int groups = heads / kv_heads, past = kv_len - queries;
  for (int h = 0; h < heads; ++h)
    for (int q = 0; q < queries; ++q)
      for (int f = 0; f < head_dim; ++f) {
        float acc = 0.0f;
        for (int k = 0; k < past + q + 1; ++k)
          acc += v[((size_t)(h / groups) * kv_len + k) * head_dim + f] *
                 p[((size_t)h * queries + q) * kv_len + k];
        out[((size_t)h * queries + q) * head_dim + f] = acc;
      }
}

void orc_attention(const void* k, const void* v, int32_t f16kv, int32_t max_seq, int32_t past, int32_t T,
                   int32_t heads, int32_t kv_heads, int32_t head_dim, const float* q, float* out) {
  attention_canonical(k, v, f16kv != 0, max_seq, past, T, heads, kv_heads, head_dim, q, out);
}

void orc_set_threads(int n) {
  if (n > 0) omp_set_num_threads(n);
}

int orc_create(const mtg_model_desc* desc, int32_t max_seq, int32_t kv_type, orc_model** out) {
  if (!desc || !out || max_seq <= 0) return MTG_ERR_INVALID;
  if (kv_type != MTG_TYPE_F32 && kv_type != MTG_TYPE_F16) return MTG_ERR_UNSUPPORTED;
  const mtg_hparams& hp = desc->hp;
  if (hp.hidden <= 0 || hp.n_layers <= 0 || hp.n_heads <= 0 || hp.n_kv_heads <= 0 ||
      hp.head_dim <= 0 || hp.n_heads % hp.n_kv_heads)
    return MTG_ERR_INVALID;
  auto m = std::unique_ptr<orc_model>(new (std::nothrow) orc_model());
  if (!m) return MTG_ERR_NOMEM;
  m->hp = hp;
  m->wtype = desc->weight_type;
  m->kv_type = kv_type;
  m->max_seq = max_seq;
  const int H = hp.hidden, D = hp.head_dim, QN = hp.n_heads * D, KN = hp.n_kv_heads * D,
            F = hp.intermediate;
  for (int l = 0; l < hp.n_layers; ++l) {
    const mtg_layer_tensors& L = desc->layers[l];
    m->wq.push_back(copy_matrix(L.attn_q, m->wtype, H, QN));
    m->wk.push_back(copy_matrix(L.attn_k, m->wtype, H, KN));
    m->wv.push_back(copy_matrix(L.attn_v, m->wtype, H, KN));
    m->wo.push_back(copy_matrix(L.attn_o, m->wtype, QN, H));
    m->wg.push_back(copy_matrix(L.ffn_gate, m->wtype, H, F));
    m->wu.push_back(copy_matrix(L.ffn_up, m->wtype, H, F));
    m->wd.push_back(copy_matrix(L.ffn_down, m->wtype, F, H));
    m->attn_norm.emplace_back(L.attn_norm, L.attn_norm + H);
    m->q_norm.emplace_back(L.attn_q_norm, L.attn_q_norm + D);
    m->k_norm.emplace_back(L.attn_k_norm, L.attn_k_norm + D);
    m->ffn_norm.emplace_back(L.ffn_norm, L.ffn_norm + H);
  }
  m->embd = copy_matrix(desc->token_embd, m->wtype, H, hp.vocab);
  m->out_norm.assign(desc->output_norm, desc->output_norm + H);
  m->layer_stride = (size_t)hp.n_kv_heads * max_seq * D;
  const size_t total = m->layer_stride * hp.n_layers;
  if (kv_type == MTG_TYPE_F32) {
    m->k32.assign(total, 0.0f);
    m->v32.assign(total, 0.0f);
  } else {
    m->k16.assign(total, 0);
    m->v16.assign(total, 0);
  }
  *out = m.release();
  return MTG_OK;
}

void orc_destroy(orc_model* m) { delete m; }
int32_t orc_past_len(const orc_model* m) { return m ? m->past : 0; }

// CpuSpeculativeDecoder::rewind (src/cpu_speculative.cpp:22-24).
int orc_rewind(orc_model* m, int32_t position) {
  if (!m || position < 0 || position > m->past) return MTG_ERR_STATE;
  m->past = position;
  return MTG_OK;
}

// embed_rows_f32 host path: dequantize the selected token_embd rows
// (src/generate.cpp:33-66).
int orc_embed(orc_model* m, const int32_t* ids, int32_t n, float* out) {
  if (!m || !ids || n <= 0 || !out) return MTG_ERR_INVALID;
  for (int i = 0; i < n; ++i) {
    if (ids[i] < 0 || ids[i] >= m->hp.vocab) return MTG_ERR_INVALID;
    embed_row(*m, ids[i], out + (size_t)i * m->hp.hidden);
  }
  return MTG_OK;
}

// Qwen3Decoder::run (src/qwen3_decoder.cpp:91-160): 28 layers over T rows at
// past, final RMSNorm * output_norm on every row, past += T.
int orc_run(orc_model* m, const float* embeds, int32_t T, float* hidden_out) {
  if (!m || !embeds || T <= 0) return MTG_ERR_INVALID;
  if (m->past + T > m->max_seq) return MTG_ERR_CAPACITY;
  const int H = m->hp.hidden;
  std::vector<float> x(embeds, embeds + (size_t)T * H);
  for (int l = 0; l < m->hp.n_layers; ++l) layer_forward(*m, l, x.data(), T);
  m->past += T;
  if (hidden_out)
    for (int t = 0; t < T; ++t)
      norm_op(*m, x.data() + (size_t)t * H, m->out_norm.data(), H, hidden_out + (size_t)t * H);
  return MTG_OK;
}

int orc_prefill(orc_model* m, const float* embeds, int32_t S, float* hidden_out) {
  if (!m) return MTG_ERR_INVALID;
  m->past = 0;
  return orc_run(m, embeds, S, hidden_out);
}

// logits_from_hidden (src/qwen3_decoder.cpp:174-205), row by row.
int orc_logits(orc_model* m, const float* hidden, int32_t T, float* logits_out) {
  if (!m || !hidden || T <= 0 || !logits_out) return MTG_ERR_INVALID;
  gemm_op(*m, m->embd.data(), m->hp.hidden, m->hp.vocab, hidden, T, logits_out);
  return MTG_OK;
}

int orc_set_order(orc_model* m, int32_t order) {
  if (!m || (order != ORC_ORDER_CANONICAL && order != ORC_ORDER_GGML_GENERIC)) return MTG_ERR_INVALID;
  m->order = order;
  return MTG_OK;
}

// cpu_ngram_draft (src/cpu_speculative.cpp:27-38): for n = min(16,|h|-1)..2
// the latest earlier occurrence of the last-n suffix; up to `maximum` tokens
// that follow it.
int32_t orc_ngram_draft(const int32_t* h, int32_t size, int32_t maximum, int32_t* out) {
  if (maximum <= 0 || size < 3) return 0;
  for (int n = std::min<int>(16, size - 1); n >= 2; --n)
    for (int start = size - n - 1; start >= 0; --start) {
      if (std::equal(h + size - n, h + size, h + start)) {
        const int begin = start + n;
        const int count = std::min<int>(maximum, size - begin);
        for (int i = 0; i < count; ++i) out[i] = h[begin + i];
        return count;
      }
    }
  return 0;
}

// cpu_greedy_choice (src/cpu_speculative.cpp:39-50): first maximum (strict >)
// after dividing positive / multiplying negative logits of the distinct ids of
// the last 100 history entries by the penalty.
int32_t orc_greedy_choice(const float* raw, int32_t n, const int32_t* history, int32_t nh,
                          float penalty) {
  if (!raw || n <= 0) return -1;
  std::vector<float> adj(raw, raw + n);
  if (penalty > 1.0f) {
    std::set<int32_t> recent;
    for (int i = std::max(0, nh - 100); i < nh; ++i) recent.insert(history[i]);
    for (int32_t id : recent)
      if (id >= 0 && id < n) adj[id] = adj[id] > 0 ? adj[id] / penalty : adj[id] * penalty;
  }
  int best = 0;
  for (int i = 1; i < n; ++i)
    if (adj[i] > adj[best]) best = i;
  return best;
}

// One verify step: append all T rows, logits of every row, greedy choice of
// row i over history ++ tokens[0..i], leading matches.
int orc_verify(orc_model* m, const int32_t* tokens, int32_t T, const int32_t* history,
               int32_t n_history, float penalty, int32_t* choice_out, int32_t* n_match_out,
               float* hidden_out, float* logits_out) {
  if (!m || !tokens || T <= 0 || T > MTG_MAX_BATCH || !choice_out || !n_match_out)
    return MTG_ERR_INVALID;
  const int H = m->hp.hidden, V = m->hp.vocab;
  std::vector<float> emb((size_t)T * H), hid((size_t)T * H), logits((size_t)T * V);
  int rc = orc_embed(m, tokens, T, emb.data());
  if (rc) return rc;
  rc = orc_run(m, emb.data(), T, hid.data());
  if (rc) return rc;
  orc_logits(m, hid.data(), T, logits.data());
  std::vector<int32_t> hist(history, history + (history ? n_history : 0));
  int match = 0;
  bool run = true;
  for (int i = 0; i < T; ++i) {
    hist.push_back(tokens[i]);
    choice_out[i] = orc_greedy_choice(logits.data() + (size_t)i * V, V, hist.data(),
                                      (int)hist.size(), penalty);
    if (run && i + 1 < T && tokens[i + 1] == choice_out[i]) ++match;
    else run = false;
  }
  *n_match_out = match;
  if (hidden_out) std::memcpy(hidden_out, hid.data(), hid.size() * sizeof(float));
  if (logits_out) std::memcpy(logits_out, logits.data(), logits.size() * sizeof(float));
  return MTG_OK;
}

int orc_kv_write(orc_model* m, const void* k, const void* v, int32_t n_pos) {
  if (!m || !k || !v || n_pos < 0 || n_pos > m->max_seq) return MTG_ERR_INVALID;
  const int L = m->hp.n_layers, NKV = m->hp.n_kv_heads, D = m->hp.head_dim;
  const size_t es = m->kv_type == MTG_TYPE_F32 ? 4 : 2;
  for (int l = 0; l < L; ++l)
    for (int h = 0; h < NKV; ++h) {
      const size_t src = (((size_t)l * NKV + h) * n_pos) * D;
      const size_t dst = (size_t)l * m->layer_stride + (size_t)h * m->max_seq * D;
      if (es == 4) {
        std::memcpy(&m->k32[dst], (const float*)k + src, (size_t)n_pos * D * 4);
        std::memcpy(&m->v32[dst], (const float*)v + src, (size_t)n_pos * D * 4);
      } else {
        std::memcpy(&m->k16[dst], (const uint16_t*)k + src, (size_t)n_pos * D * 2);
        std::memcpy(&m->v16[dst], (const uint16_t*)v + src, (size_t)n_pos * D * 2);
      }
    }
  m->past = n_pos;
  return MTG_OK;
}

int orc_kv_read(const orc_model* m, void* k, void* v, int32_t n_pos) {
  if (!m || !k || !v || n_pos < 0 || n_pos > m->max_seq) return MTG_ERR_INVALID;
  const int L = m->hp.n_layers, NKV = m->hp.n_kv_heads, D = m->hp.head_dim;
  for (int l = 0; l < L; ++l)
    for (int h = 0; h < NKV; ++h) {
      const size_t dst = (((size_t)l * NKV + h) * n_pos) * D;
      const size_t src = (size_t)l * m->layer_stride + (size_t)h * m->max_seq * D;
      if (m->kv_type == MTG_TYPE_F32) {
        std::memcpy((float*)k + dst, &m->k32[src], (size_t)n_pos * D * 4);
        std::memcpy((float*)v + dst, &m->v32[src], (size_t)n_pos * D * 4);
      } else {
        std::memcpy((uint16_t*)k + dst, &m->k16[src], (size_t)n_pos * D * 2);
        std::memcpy((uint16_t*)v + dst, &m->v16[src], (size_t)n_pos * D * 2);
      }
    }
  return MTG_OK;
}

// The controller loop of cpu_speculative_generate (src/cpu_speculative.cpp:
// 89-137), continuing from an existing target state: emit the seed (eos /
// token_limit stops), budget = min(max_draft, max_new-|ids|, remaining-1), draft,
// append seed+drafts, accept while the draft equals the greedy choice of the
// previous row, the terminating token is emitted but not kept, logical rewind.
int orc_controller(orc_target* tg, int32_t first_seed, const int32_t* prior_ids, int32_t n_prior,
                   int32_t max_new, int32_t max_steps, int32_t eos, float penalty,
                   int32_t max_draft, mtg_draft_fn draft, void* user, int32_t* ids_out,
                   int32_t* n_ids_out, mtg_gen_stats* stats) {
  if (!tg || !tg->verify || !ids_out || !n_ids_out || max_new <= 0) return MTG_ERR_INVALID;
  penalty = std::max(1.0f, std::min(1.5f, penalty));
  std::vector<int32_t> ids(prior_ids, prior_ids + (prior_ids ? n_prior : 0));
  const size_t first_new = ids.size();
  mtg_gen_stats st{};
  int stop = 0;
  auto emit = [&](int32_t id) {
    ids.push_back(id);
    if (id == eos) stop = 1;
    else if ((int)(ids.size() - first_new) >= max_new) stop = 2;
  };
  int32_t raw_choice = first_seed;
  int steps = 0;
  int rc = MTG_OK;
  std::vector<int32_t> proposal(MTG_MAX_BATCH), choice(MTG_MAX_BATCH);
  while (!stop) {
    if (max_steps > 0 && steps >= max_steps) break;
    const int32_t seed = raw_choice;
    emit(seed);
    if (stop) break;
    const int before = tg->past;
    const int remaining = tg->max_seq - tg->past;
    if (remaining < 1) {  // append of the seed fails: break (src/cpu_speculative.cpp:113-114)
      stop = 3;
      break;
    }
    const int budget = std::max(0, std::min({max_draft, max_new - (int)(ids.size() - first_new),
                                              remaining - 1, MTG_MAX_BATCH - 1}));
    int np = draft ? draft(user, ids.data(), (int)ids.size(), budget, proposal.data())
                   : orc_ngram_draft(ids.data(), (int)ids.size(), budget, proposal.data());
    np = std::max(0, std::min(np, budget));
    for (int i = 0; i < np; ++i)
      if (proposal[i] < 0 || proposal[i] >= tg->vocab) { rc = MTG_ERR_INVALID; break; }
    if (rc) break;
    std::vector<int32_t> inputs{seed};
    inputs.insert(inputs.end(), proposal.begin(), proposal.begin() + np);
    int32_t n_match = 0;
    // history for row i = ids before the seed ++ inputs[0..i]
    rc = tg->verify(tg, inputs.data(), (int)inputs.size(), ids.data(), (int)ids.size() - 1,
                    penalty, choice.data(), &n_match);
    if (rc) break;
    tg->past += (int)inputs.size();
    ++steps;
    ++st.target_calls;
    st.drafted_calls += np > 0;
    st.proposed += np;
    st.target_input_tokens += (int)inputs.size();
    int keep = 1;
    raw_choice = choice[0];
    for (int i = 0; i < np; ++i) {
      if (proposal[i] != choice[i]) break;
      ++st.accepted;
      emit(proposal[i]);
      if (stop) break;
      ++keep;
      raw_choice = choice[i + 1];
    }
    const int position = before + keep;
    if (tg->past != position) {
      tg->past = position;
      ++st.rewinds;
    }
  }
  st.stop_reason = stop;
  st.next_seed = raw_choice;
  const int n_new = (int)(ids.size() - first_new);
  std::memcpy(ids_out, ids.data() + first_new, (size_t)n_new * sizeof(int32_t));
  *n_ids_out = n_new;
  if (stats) *stats = st;
  return rc;
}

namespace {
int model_verify(orc_target* tg, const int32_t* tokens, int32_t T, const int32_t* history,
                 int32_t n_history, float penalty, int32_t* choice_out, int32_t* n_match_out) {
  orc_model* m = (orc_model*)tg->self;
  m->past = tg->past;
  return orc_verify(m, tokens, T, history, n_history, penalty, choice_out, n_match_out, nullptr,
                    nullptr);
}
}  // namespace

int orc_generate_from(orc_model* m, int32_t first_seed, const int32_t* prior_ids,
                      int32_t n_prior, int32_t max_new, int32_t max_steps, int32_t eos,
                      float penalty, int32_t max_draft, mtg_draft_fn draft, void* user,
                      int32_t* ids_out, int32_t* n_ids_out, mtg_gen_stats* stats) {
  if (!m) return MTG_ERR_INVALID;
  orc_target tg{m, model_verify, m->past, m->max_seq, m->hp.vocab};
  const int rc = orc_controller(&tg, first_seed, prior_ids, n_prior, max_new, max_steps, eos,
                                penalty, max_draft, draft, user, ids_out, n_ids_out, stats);
  m->past = tg.past;
  return rc;
}

}  // extern "C"

// ===================================================== Whisper encoder ======
// WhisperEncoder::encode (src/whisper_encoder.cpp:103-209) and
// AudioAdaptor::apply (src/audio_adaptor.cpp:38-97) with the same canonical
// orders as the decoder step: q8_0 linears as mul_mat_q8, the attention's
// 64-key chunks merged in order, double sums over 64 partials + butterfly.
namespace {

// erf by its Maclaurin series in double, a fixed number of terms per range of
// |z| (the device evaluates the same operations); erf(z) = +-1 from |z| >= 4,
// where 1 - erf(4) = 1.5e-8 no longer moves a float. The divisions by n + 1 and
// 2 n + 1 are multiplications by their double reciprocals (a shared table).
constexpr int kErfTerms = 76;
struct ErfTable {
  double inv_next[kErfTerms], inv_odd[kErfTerms];
  constexpr ErfTable() : inv_next(), inv_odd() {
    for (int n = 0; n < kErfTerms; ++n) {
      inv_next[n] = 1.0 / (double)(n + 1);
      inv_odd[n] = 1.0 / (double)(2 * n + 1);
    }
  }
};
constexpr ErfTable kErf{};
double erf_series(double z) {
  const double a = std::fabs(z);
  if (a >= 4.0) return z < 0.0 ? -1.0 : 1.0;
  const int terms = a < 1.0 ? 28 : (a < 2.0 ? 44 : (a < 3.0 ? 60 : 76));
  const double a2 = a * a;
  double term = a, sum = 0.0;
  for (int n = 0; n < terms; ++n) {
    sum = sum + term * kErf.inv_odd[n];
    term = -(term * a2) * kErf.inv_next[n];
  }
  const double r = sum * 1.1283791670955126;  // 2 / sqrt(pi)
  return z < 0.0 ? -r : r;
}

// ggml_gelu_erf (0.5 x (1 + erf(x / sqrt 2)), src/whisper_encoder.cpp:119-123)
float gelu_erf(float x) {
  const float z = x * 0.70710678118654752440f;
  const float e = (float)erf_series((double)z);
  return (0.5f * x) * (1.0f + e);
}

// 64 partials of n / 64 consecutive elements (sequential double sums), butterfly
double sum64(const double* v, int n) {
  double part[64];
  const int per = n / 64;
  for (int l = 0; l < 64; ++l) {
    double s = 0.0;
    for (int e = 0; e < per; ++e) s += v[l * per + e];
    part[l] = s;
  }
  return butterfly64(part);
}

// layer_norm (src/ggml_extend.hpp:57-63): ggml_norm (mean and variance summed in
// double, scale = 1 / sqrtf(variance + eps)), then * w, then + b. n: a multiple of 64.
void layer_norm(const float* x, const float* w, const float* b, int n, float eps, float* y) {
  std::vector<double> t((size_t)n);
  for (int i = 0; i < n; ++i) t[i] = (double)x[i];
  const float mean = (float)(sum64(t.data(), n) / (double)n);
  for (int i = 0; i < n; ++i) {
    const float v = x[i] - mean;
    y[i] = v;
    t[i] = (double)(v * v);
  }
  const float variance = (float)(sum64(t.data(), n) / (double)n);
  const float scale = 1.0f / std::sqrt(variance + eps);
  for (int i = 0; i < n; ++i) y[i] = (y[i] * scale) * w[i] + b[i];
}

// conv1d_ph_f32 (src/whisper_encoder.cpp:32-44): f32 im2col (pad 1, kernel 3)
// and mul_mat; canonical order: one fma chain per output over (ic, k), k fastest.
void conv1d(const float* w, int ic, int oc, const float* x, int L, int stride, float* y) {
  const int OL = (L - 1) / stride + 1;
#pragma omp parallel for schedule(static)
  for (int t = 0; t < OL; ++t)
    for (int o = 0; o < oc; ++o) {
      const float* wr = w + (size_t)o * ic * 3;
      float acc = 0.0f;
      for (int c = 0; c < ic; ++c)
        for (int k = 0; k < 3; ++k) {
          const int xi = t * stride + k - 1;
          const float xv = (xi >= 0 && xi < L) ? x[(size_t)c * L + xi] : 0.0f;
          acc = std::fma(wr[c * 3 + k], xv, acc);
        }
      y[(size_t)t * oc + o] = acc;
    }
}

// the encoder's bidirectional attention (src/whisper_encoder.cpp:164-180):
// scores K.Q, soft_max_ext with scale 1/sqrt(head_dim) and no mask, context
// V.P. Canonical order as the decoder step: 64-key chunks, score = fma chain
// over head_dim, chunk max, p = exp(w - max), l = butterfly, O = fma chain over
// the chunk's keys, chunks merged in order with f = exp(m_c - M).
void enc_attention(const float* q, const float* k, const float* v, int T, int NH, int D, float* out) {
  const int W = NH * D, nch = (T + 63) / 64;
  const float scale = 1.0f / std::sqrt((float)D);
#pragma omp parallel for collapse(2) schedule(static)
  for (int h = 0; h < NH; ++h)
    for (int t = 0; t < T; ++t) {
      std::vector<float> cm(nch), cl(nch), co((size_t)nch * D);
      const float* qh = q + (size_t)t * W + (size_t)h * D;
      for (int c = 0; c < nch; ++c) {
        float wv[64], p[64];
        float mx = -INFINITY;
        for (int j = 0; j < 64; ++j) {
          const int key = 64 * c + j;
          if (key < T) {
            const float* kr = k + (size_t)key * W + (size_t)h * D;
            float s = 0.0f;
            for (int d = 0; d < D; ++d) s = std::fma(qh[d], kr[d], s);
            wv[j] = s * scale;
          } else {
            wv[j] = -INFINITY;
          }
          mx = std::max(mx, wv[j]);
        }
        for (int j = 0; j < 64; ++j) p[j] = wv[j] == -INFINITY ? 0.0f : exp_c(wv[j] - mx);
        float pl[64];
        std::memcpy(pl, p, sizeof(pl));
        cm[c] = mx;
        cl[c] = butterfly64(pl);
        for (int d = 0; d < D; ++d) {
          float acc = 0.0f;
          for (int j = 0; j < 64; ++j) {
            const int key = 64 * c + j;
            const float vv = key < T ? v[(size_t)key * W + (size_t)h * D + d] : 0.0f;
            acc = std::fma(p[j], vv, acc);
          }
          co[(size_t)c * D + d] = acc;
        }
      }
      float M = -INFINITY;
      for (int c = 0; c < nch; ++c) M = std::max(M, cm[c]);
      float* oh = out + (size_t)t * W + (size_t)h * D;
      for (int d = 0; d < D; ++d) {
        float L = 0.0f, acc = 0.0f;
        for (int c = 0; c < nch; ++c) {
          const float f = exp_c(cm[c] - M);
          L = std::fma(cl[c], f, L);
          acc = std::fma(co[(size_t)c * D + d], f, acc);
        }
        oh[d] = acc / L;
      }
    }
}

// linear (src/ggml_extend.hpp:50-55): mul_mat (q8_0, f16 or q4_K weights, the
// decoder's canonical orders) then + bias
void linear_wt(int wtype, const std::vector<uint8_t>& w, const float* bias, int k, int n, const float* x, int T,
               float* y) {
  mul_mat(wtype, w.data(), k, n, x, T, y);
  if (bias)
    for (int t = 0; t < T; ++t)
      for (int i = 0; i < n; ++i) y[(size_t)t * n + i] = y[(size_t)t * n + i] + bias[i];
}

struct EncLayer {
  std::vector<float> attn_ln_w, attn_ln_b, q_b, v_b, o_b, ffn_ln_w, ffn_ln_b, fc1_b, fc2_b;
  std::vector<uint8_t> q_w, k_w, v_w, o_w, fc1_w, fc2_w;
};

std::vector<float> copy_f(const float* p, size_t n) { return std::vector<float>(p, p + n); }
// the bytes of an n x k matrix of wtype (ggml block layouts)
std::vector<uint8_t> copy_w(int wtype, const void* p, size_t n, size_t k) {
  const size_t row = wtype == MTG_TYPE_F16   ? k * 2
                     : wtype == MTG_TYPE_F32  ? k * 4
                     : wtype == MTG_TYPE_Q4_K ? k / 256 * 144
                                              : k / 32 * 34;
  const uint8_t* b = (const uint8_t*)p;
  return std::vector<uint8_t>(b, b + n * row);
}

}  // namespace

struct orc_encoder {
  mtg_encoder_hparams hp;
  int wtype = MTG_TYPE_Q8_0;
  std::vector<float> conv1_w, conv1_b, conv2_w, conv2_b, pos, ln_post_w, ln_post_b;
  std::vector<EncLayer> layers;
  std::vector<uint8_t> ad_fc1_w, ad_fc2_w;
  std::vector<float> ad_fc1_b, ad_fc2_b, ad_ln_w, ad_ln_b;
  std::vector<float> last;  // the last encode's rows
  int last_rows = 0;
};

extern "C" {

float orc_gelu_erf(float x) { return gelu_erf(x); }
void orc_layer_norm(const float* x, const float* w, const float* b, int32_t n, float eps, float* y) {
  layer_norm(x, w, b, n, eps, y);
}
void orc_conv1d(const float* w, int32_t ic, int32_t oc, const float* x, int32_t L, int32_t stride, float* y) {
  conv1d(w, ic, oc, x, L, stride, y);
}
void orc_enc_attention(const float* q, const float* k, const float* v, int32_t T, int32_t n_heads,
                       int32_t head_dim, float* out) {
  enc_attention(q, k, v, T, n_heads, head_dim, out);
}

int orc_encoder_create(const mtg_encoder_desc* d, orc_encoder** out) {
  if (!d || !out) return MTG_ERR_INVALID;
  const int wt = d->weight_type;
  if (wt != MTG_TYPE_Q8_0 && wt != MTG_TYPE_F16 && wt != MTG_TYPE_F32 && wt != MTG_TYPE_Q4_K) return MTG_ERR_INVALID;
  const mtg_encoder_hparams& hp = d->hp;
  const size_t D = hp.d_model, F = hp.ffn, M = hp.n_mels, R = (size_t)(hp.n_frames - 1) / 2 + 1;
  auto e = std::make_unique<orc_encoder>();
  e->hp = hp;
  e->wtype = wt;
  e->conv1_w = copy_f(d->conv1_w, D * M * 3);
  e->conv1_b = copy_f(d->conv1_b, D);
  e->conv2_w = copy_f(d->conv2_w, D * D * 3);
  e->conv2_b = copy_f(d->conv2_b, D);
  e->pos = copy_f(d->pos_embd, R * D);
  e->ln_post_w = copy_f(d->ln_post_w, D);
  e->ln_post_b = copy_f(d->ln_post_b, D);
  for (int l = 0; l < hp.n_layers; ++l) {
    const mtg_encoder_layer& s = d->layers[l];
    EncLayer L;
    L.attn_ln_w = copy_f(s.attn_ln_w, D);
    L.attn_ln_b = copy_f(s.attn_ln_b, D);
    L.q_w = copy_w(wt, s.q_w, D, D);
    L.k_w = copy_w(wt, s.k_w, D, D);
    L.v_w = copy_w(wt, s.v_w, D, D);
    L.o_w = copy_w(wt, s.o_w, D, D);
    L.q_b = copy_f(s.q_b, D);
    L.v_b = copy_f(s.v_b, D);
    L.o_b = copy_f(s.o_b, D);
    L.ffn_ln_w = copy_f(s.ffn_ln_w, D);
    L.ffn_ln_b = copy_f(s.ffn_ln_b, D);
    L.fc1_w = copy_w(wt, s.fc1_w, F, D);
    L.fc1_b = copy_f(s.fc1_b, F);
    L.fc2_w = copy_w(wt, s.fc2_w, D, F);
    L.fc2_b = copy_f(s.fc2_b, D);
    e->layers.push_back(std::move(L));
  }
  const size_t H = hp.hidden, IN = D * hp.merge;
  e->ad_fc1_w = copy_w(wt, d->ad_fc1_w, H, IN);
  e->ad_fc1_b = copy_f(d->ad_fc1_b, H);
  e->ad_fc2_w = copy_w(wt, d->ad_fc2_w, H, H);
  e->ad_fc2_b = copy_f(d->ad_fc2_b, H);
  e->ad_ln_w = copy_f(d->ad_ln_w, H);
  e->ad_ln_b = copy_f(d->ad_ln_b, H);
  *out = e.release();
  return MTG_OK;
}

void orc_encoder_destroy(orc_encoder* e) { delete e; }

int orc_encoder_encode(orc_encoder* e, const float* mel, float* out, int32_t* rows_out) {
  if (!e || !mel) return MTG_ERR_INVALID;
  const mtg_encoder_hparams& hp = e->hp;
  const int D = hp.d_model, F = hp.ffn, NF = hp.n_frames, NH = hp.n_heads, hd = D / NH;
  const int R = (NF - 1) / 2 + 1;
  // conv stem: conv1 + bias, gelu; conv2 (stride 2) + bias, gelu; + pos_embd
  std::vector<float> c1((size_t)NF * D), c1t((size_t)D * NF), x((size_t)R * D);
  conv1d(e->conv1_w.data(), hp.n_mels, D, mel, NF, 1, c1.data());
  for (int t = 0; t < NF; ++t)
    for (int o = 0; o < D; ++o) c1t[(size_t)o * NF + t] = gelu_erf(c1[(size_t)t * D + o] + e->conv1_b[o]);
  conv1d(e->conv2_w.data(), D, D, c1t.data(), NF, 2, x.data());
  for (int t = 0; t < R; ++t)
    for (int o = 0; o < D; ++o) {
      const size_t i = (size_t)t * D + o;
      x[i] = gelu_erf(x[i] + e->conv2_b[o]) + e->pos[i];
    }
  std::vector<float> xn((size_t)R * D), q((size_t)R * D), k((size_t)R * D), v((size_t)R * D), a((size_t)R * D),
      f((size_t)R * F);
  for (const EncLayer& L : e->layers) {
    for (int t = 0; t < R; ++t)
      layer_norm(x.data() + (size_t)t * D, L.attn_ln_w.data(), L.attn_ln_b.data(), D, 1e-5f, xn.data() + (size_t)t * D);
    linear_wt(e->wtype, L.q_w, L.q_b.data(), D, D, xn.data(), R, q.data());
    linear_wt(e->wtype, L.k_w, nullptr, D, D, xn.data(), R, k.data());
    linear_wt(e->wtype, L.v_w, L.v_b.data(), D, D, xn.data(), R, v.data());
    enc_attention(q.data(), k.data(), v.data(), R, NH, hd, a.data());
    linear_wt(e->wtype, L.o_w, L.o_b.data(), D, D, a.data(), R, q.data());
    for (size_t i = 0; i < x.size(); ++i) x[i] = x[i] + q[i];
    for (int t = 0; t < R; ++t)
      layer_norm(x.data() + (size_t)t * D, L.ffn_ln_w.data(), L.ffn_ln_b.data(), D, 1e-5f, xn.data() + (size_t)t * D);
    linear_wt(e->wtype, L.fc1_w, L.fc1_b.data(), D, F, xn.data(), R, f.data());
    for (float& y : f) y = gelu_erf(y);
    linear_wt(e->wtype, L.fc2_w, L.fc2_b.data(), F, D, f.data(), R, q.data());
    for (size_t i = 0; i < x.size(); ++i) x[i] = x[i] + q[i];
  }
  e->last.assign((size_t)R * D, 0.0f);
  for (int t = 0; t < R; ++t)
    layer_norm(x.data() + (size_t)t * D, e->ln_post_w.data(), e->ln_post_b.data(), D, 1e-5f,
               e->last.data() + (size_t)t * D);
  e->last_rows = R;
  if (out) std::memcpy(out, e->last.data(), e->last.size() * sizeof(float));
  if (rows_out) *rows_out = R;
  return MTG_OK;
}

int orc_encoder_adapt(orc_encoder* e, const float* rows, int32_t T, float* out, int32_t* n_out) {
  if (!e || !out || T < 0) return MTG_ERR_INVALID;
  const mtg_encoder_hparams& hp = e->hp;
  if (!rows) {
    if (T > e->last_rows) return MTG_ERR_INVALID;
    rows = e->last.data();
  }
  const int D = hp.d_model, H = hp.hidden, IN = D * hp.merge, N = T / hp.merge;
  if (n_out) *n_out = N;
  if (N <= 0) return MTG_OK;
  // [D * merge, N]: merge consecutive rows per adaptor row (a plain view)
  std::vector<float> h1((size_t)N * H), h2((size_t)N * H);
  linear_wt(e->wtype, e->ad_fc1_w, e->ad_fc1_b.data(), IN, H, rows, N, h1.data());
  for (float& y : h1) y = y / (1.0f + exp_c(-y));  // ggml_silu
  linear_wt(e->wtype, e->ad_fc2_w, e->ad_fc2_b.data(), H, H, h1.data(), N, h2.data());
  for (int t = 0; t < N; ++t)
    layer_norm(h2.data() + (size_t)t * H, e->ad_ln_w.data(), e->ad_ln_b.data(), H, hp.adaptor_eps,
               out + (size_t)t * H);
  return MTG_OK;
}

}  // extern "C"
