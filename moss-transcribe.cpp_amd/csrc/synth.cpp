// synth.cpp - seeded synthetic Qwen3 weights (the workload generator) and host-side
// block-format helpers. Stands in for the GGUF loader (src/model_loader.cpp:21-114),
// which has no checkpoint to read here.
#include <cmath>
#include <cstring>
#include <memory>
#include <new>
#include <thread>
#include <vector>

#include "../../include/mtg_verify.h"

namespace {

uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// Box-Muller on two counter-derived uniforms in (0, 1), evaluated in double.
float normal_at(uint64_t seed, uint64_t index) {
  const uint64_t h1 = splitmix64(seed * 0xD1B54A32D192ED03ull + index);
  const uint64_t h2 = splitmix64(h1 ^ 0xA0761D6478BD642Full);
  const double u1 = ((double)(h1 >> 11) + 0.5) * (1.0 / 9007199254740992.0);
  const double u2 = ((double)(h2 >> 11) + 0.5) * (1.0 / 9007199254740992.0);
  return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
}

template <class F>
void parallel_rows(int64_t n, F fn) {
  unsigned nt = std::thread::hardware_concurrency();
  if (nt == 0) nt = 1;
  if (nt > 32) nt = 32;
  if (n < 64) nt = 1;
  std::vector<std::thread> th;
  for (unsigned i = 0; i < nt; ++i)
    th.emplace_back([=]() {
      for (int64_t r = (n * i) / nt; r < (n * (i + 1)) / nt; ++r) fn(r);
    });
  for (auto& t : th) t.join();
}

#pragma pack(push, 1)
struct BlockQ8 {
  uint16_t d;
  int8_t qs[32];
};
struct BlockQ4K {
  uint16_t d, dmin;
  uint8_t scales[12];
  uint8_t qs[128];
};
#pragma pack(pop)

}  // namespace

extern "C" {

// IEEE binary16 round-to-nearest-even (magic-number method, F. Giesen 2012).
uint16_t mtg_f32_to_f16(float value) {
  uint32_t u;
  std::memcpy(&u, &value, 4);
  const uint32_t sign = u & 0x80000000u;
  u ^= sign;
  uint16_t out;
  if (u >= (uint32_t)(127 + 16) << 23) {
    out = (u > 0x7f800000u) ? 0x7e00 : 0x7c00;
  } else if (u < (uint32_t)113 << 23) {
    const uint32_t magic_u = (uint32_t)((127 - 15) + (23 - 10) + 1) << 23;
    float magic, f;
    std::memcpy(&magic, &magic_u, 4);
    std::memcpy(&f, &u, 4);
    f += magic;
    uint32_t r;
    std::memcpy(&r, &f, 4);
    out = (uint16_t)(r - magic_u);
  } else {
    const uint32_t odd = (u >> 13) & 1u;
    u += ((uint32_t)(15 - 127) << 23) + 0xfffu;
    u += odd;
    out = (uint16_t)(u >> 13);
  }
  return (uint16_t)(out | (sign >> 16));
}

float mtg_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      exp = 113;
      while (!(man & 0x400u)) {
        man <<= 1;
        --exp;
      }
      bits = sign | (exp << 23) | ((man & 0x3ffu) << 13);
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

void mtg_normal_fill(uint64_t seed, uint64_t first, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = normal_at(seed, first + i);
}

size_t mtg_row_bytes(int32_t type, int64_t k) {
  switch (type) {
    case MTG_TYPE_Q8_0: return (size_t)(k / 32) * 34;
    case MTG_TYPE_F16: return (size_t)k * 2;
    case MTG_TYPE_Q4_K: return (size_t)(k / 256) * 144;
    default: return (size_t)k * 4;
  }
}

// ggml quantize_row_q8_0_ref / the GGUF converter's Q8_0 rule:
// d = amax/127, codes = roundf(x * (1/d)) (half away from zero), d as f16.
void mtg_quantize_q8_0_weight(const float* x, int64_t k, void* blocks) {
  BlockQ8* y = (BlockQ8*)blocks;
  for (int64_t b = 0; b < k / 32; ++b) {
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = std::fmax(amax, std::fabs(x[b * 32 + j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    y[b].d = mtg_f32_to_f16(d);
    for (int j = 0; j < 32; ++j) y[b].qs[j] = (int8_t)std::roundf(x[b * 32 + j] * id);
  }
}

// q4_K weights for the long-context workload: per 32-element sub-block an affine
// range [min, max] (min clamped to <= 0) with 6-bit scale/min codes against the
// super-block's f16 d and dmin; 4-bit codes. The dequantized value is
// d*sc*q - dmin*m as the GGUF q4_K format defines it.
void mtg_quantize_q4_k(const float* x, int64_t k, void* blocks) {
  BlockQ4K* y = (BlockQ4K*)blocks;
  for (int64_t b = 0; b < k / 256; ++b) {
    const float* v = x + b * 256;
    float scale[8], minv[8];
    float max_scale = 0.0f, max_min = 0.0f;
    for (int s = 0; s < 8; ++s) {
      float lo = 0.0f, hi = -INFINITY;
      for (int l = 0; l < 32; ++l) {
        lo = std::fmin(lo, v[s * 32 + l]);
        hi = std::fmax(hi, v[s * 32 + l]);
      }
      scale[s] = (hi - lo) / 15.0f;
      minv[s] = -lo;
      max_scale = std::fmax(max_scale, scale[s]);
      max_min = std::fmax(max_min, minv[s]);
    }
    const float d = max_scale / 63.0f, dmin = max_min / 63.0f;
    y[b].d = mtg_f32_to_f16(d);
    y[b].dmin = mtg_f32_to_f16(dmin);
    const float dq = mtg_f16_to_f32(y[b].d), dmq = mtg_f16_to_f32(y[b].dmin);
    int sc[8], mn[8];
    for (int s = 0; s < 8; ++s) {
      sc[s] = dq > 0 ? (int)std::fmin(63.0f, std::roundf(scale[s] / dq)) : 0;
      mn[s] = dmq > 0 ? (int)std::fmin(63.0f, std::roundf(minv[s] / dmq)) : 0;
    }
    std::memset(y[b].scales, 0, 12);
    for (int s = 0; s < 4; ++s) {
      y[b].scales[s] = (uint8_t)(sc[s] | ((sc[s + 4] >> 4) << 6));
      y[b].scales[s + 4] = (uint8_t)(mn[s] | ((mn[s + 4] >> 4) << 6));
      y[b].scales[s + 8] = (uint8_t)((sc[s + 4] & 0xF) | ((mn[s + 4] & 0xF) << 4));
    }
    for (int s = 0; s < 8; ++s) {
      const float step = dq * (float)sc[s], off = dmq * (float)mn[s];
      for (int l = 0; l < 32; ++l) {
        int q = step > 0 ? (int)std::roundf((v[s * 32 + l] + off) / step) : 0;
        q = q < 0 ? 0 : q > 15 ? 15 : q;
        uint8_t& byte = y[b].qs[(s / 2) * 32 + l];
        if (s & 1) byte = (uint8_t)((byte & 0x0F) | (q << 4));
        else byte = (uint8_t)((byte & 0xF0) | q);
      }
    }
  }
}

void mtg_dequantize(int32_t type, const void* blocks, int64_t k, float* out) {
  if (type == MTG_TYPE_Q8_0) {
    const BlockQ8* b = (const BlockQ8*)blocks;
    for (int64_t i = 0; i < k; ++i) out[i] = mtg_f16_to_f32(b[i / 32].d) * (float)b[i / 32].qs[i % 32];
  } else if (type == MTG_TYPE_F16) {
    const uint16_t* h = (const uint16_t*)blocks;
    for (int64_t i = 0; i < k; ++i) out[i] = mtg_f16_to_f32(h[i]);
  } else if (type == MTG_TYPE_Q4_K) {
    const BlockQ4K* b = (const BlockQ4K*)blocks;
    for (int64_t sb = 0; sb < k / 256; ++sb) {
      const float d = mtg_f16_to_f32(b[sb].d), dmin = mtg_f16_to_f32(b[sb].dmin);
      const uint8_t* q = b[sb].scales;
      for (int s = 0; s < 8; ++s) {
        int sc, mn;
        if (s < 4) {
          sc = q[s] & 63;
          mn = q[s + 4] & 63;
        } else {
          sc = (q[s + 4] & 0xF) | ((q[s - 4] >> 6) << 4);
          mn = (q[s + 4] >> 4) | ((q[s] >> 6) << 4);
        }
        for (int l = 0; l < 32; ++l) {
          const uint8_t byte = b[sb].qs[(s / 2) * 32 + l];
          const int v = (s & 1) ? (byte >> 4) : (byte & 0xF);
          out[sb * 256 + s * 32 + l] = d * (float)sc * (float)v - dmin * (float)mn;
        }
      }
    }
  } else {
    std::memcpy(out, blocks, (size_t)k * 4);
  }
}

}  // extern "C"

// --------------------------------------------------------- synthetic model --
struct mtg_synth_model {
  mtg_model_desc desc{};
  std::vector<mtg_layer_tensors> layers;
  std::vector<std::vector<uint8_t>> store;
};

namespace {

const void* make_matrix(mtg_synth_model& m, int type, int64_t k, int64_t n, uint64_t seed, float std) {
  const size_t rb = mtg_row_bytes(type, k);
  m.store.emplace_back(rb * (size_t)n);
  uint8_t* base = m.store.back().data();
  parallel_rows(n, [&](int64_t r) {
    std::vector<float> row((size_t)k);
    for (int64_t i = 0; i < k; ++i) row[i] = std * normal_at(seed, (uint64_t)(r * k + i));
    uint8_t* dst = base + rb * (size_t)r;
    if (type == MTG_TYPE_Q8_0) mtg_quantize_q8_0_weight(row.data(), k, dst);
    else if (type == MTG_TYPE_Q4_K) mtg_quantize_q4_k(row.data(), k, dst);
    else if (type == MTG_TYPE_F32) std::memcpy(dst, row.data(), (size_t)k * 4);
    else {
      uint16_t* h = (uint16_t*)dst;
      for (int64_t i = 0; i < k; ++i) h[i] = mtg_f32_to_f16(row[i]);
    }
  });
  return base;
}

const float* make_gain(mtg_synth_model& m, int64_t n, uint64_t seed, float jitter) {
  m.store.emplace_back((size_t)n * 4);
  float* g = (float*)m.store.back().data();
  for (int64_t i = 0; i < n; ++i) g[i] = 1.0f + jitter * normal_at(seed, (uint64_t)i);
  return g;
}

}  // namespace

extern "C" {

int mtg_synth_create(const mtg_hparams* hp, int32_t weight_type, uint64_t seed, float std,
                     float gain_jitter, mtg_synth_model** out) {
  if (!hp || !out) return MTG_ERR_INVALID;
  if (weight_type != MTG_TYPE_Q8_0 && weight_type != MTG_TYPE_F16 && weight_type != MTG_TYPE_F32 &&
      weight_type != MTG_TYPE_Q4_K)
    return MTG_ERR_UNSUPPORTED;
  const int64_t H = hp->hidden, D = hp->head_dim, QN = (int64_t)hp->n_heads * D,
                KN = (int64_t)hp->n_kv_heads * D, F = hp->intermediate;
  const int64_t blk = weight_type == MTG_TYPE_Q4_K ? 256 : 32;
  if (H % blk || QN % blk || F % blk || hp->n_layers <= 0 || hp->vocab <= 0) return MTG_ERR_INVALID;
  try {
    auto m = std::make_unique<mtg_synth_model>();
    m->store.reserve((size_t)hp->n_layers * 11 + 4);
    m->layers.resize(hp->n_layers);
    auto tseed = [&](int layer, int which) {
      return splitmix64(seed * 0x9E3779B97F4A7C15ull + (uint64_t)layer * 64 + (uint64_t)which);
    };
    for (int l = 0; l < hp->n_layers; ++l) {
      mtg_layer_tensors& t = m->layers[l];
      t.attn_q = make_matrix(*m, weight_type, H, QN, tseed(l, 0), std);
      t.attn_k = make_matrix(*m, weight_type, H, KN, tseed(l, 1), std);
      t.attn_v = make_matrix(*m, weight_type, H, KN, tseed(l, 2), std);
      t.attn_o = make_matrix(*m, weight_type, QN, H, tseed(l, 3), std);
      t.ffn_gate = make_matrix(*m, weight_type, H, F, tseed(l, 4), std);
      t.ffn_up = make_matrix(*m, weight_type, H, F, tseed(l, 5), std);
      t.ffn_down = make_matrix(*m, weight_type, F, H, tseed(l, 6), std);
      t.attn_norm = make_gain(*m, H, tseed(l, 7), gain_jitter);
      t.attn_q_norm = make_gain(*m, D, tseed(l, 8), gain_jitter);
      t.attn_k_norm = make_gain(*m, D, tseed(l, 9), gain_jitter);
      t.ffn_norm = make_gain(*m, H, tseed(l, 10), gain_jitter);
    }
    m->desc.hp = *hp;
    m->desc.weight_type = weight_type;
    m->desc.token_embd = make_matrix(*m, weight_type, H, hp->vocab, tseed(1 << 20, 0), std);
    m->desc.output_norm = make_gain(*m, H, tseed(1 << 20, 1), gain_jitter);
    m->desc.layers = m->layers.data();
    *out = m.release();
    return MTG_OK;
  } catch (const std::bad_alloc&) {
    return MTG_ERR_NOMEM;
  }
}

void mtg_synth_free(mtg_synth_model* m) { delete m; }
const mtg_model_desc* mtg_synth_desc(const mtg_synth_model* m) { return m ? &m->desc : nullptr; }

}  // extern "C"
