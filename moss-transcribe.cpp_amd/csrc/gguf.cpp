// gguf.cpp - GGUF model file -> mtg_model_desc (the decoder part of
// ModelLoader::load / read_config, src/model_loader.cpp:21-169).
//
// The file is memory-mapped; the header, metadata and tensor table are parsed
// with bounds checks on every read (GGUF v2/v3: magic, version, tensor count,
// metadata count, typed key/value pairs, tensor infos {name, dims, type,
// offset}, data section aligned to general.alignment). The decoder's tensors are
// found by the names the reference's loader reads (src/qwen3.cpp:33-56,
// src/qwen3_decoder.cpp:53-57) and checked for shape and type; the
// hyper-parameters come from the mtd.text.* keys with the reference's defaults
// (src/model_loader.cpp:116-129). Norm gains stored as f16 are widened to f32, as
// promote_small_f16_to_f32 does (src/model_loader.cpp:176-246). Matrix bytes are
// handed to mtg_create straight from the mapping.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <deque>
#include <map>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "kernels.hpp"

namespace {

enum : uint32_t {
  GG_U8 = 0, GG_I8 = 1, GG_U16 = 2, GG_I16 = 3, GG_U32 = 4, GG_I32 = 5, GG_F32 = 6, GG_BOOL = 7,
  GG_STR = 8, GG_ARR = 9, GG_U64 = 10, GG_I64 = 11, GG_F64 = 12
};

struct Value {
  uint32_t type = 0;
  uint64_t u = 0;  // integer and bool values
  int64_t i = 0;
  double f = 0.0;
  std::string s;
  uint32_t arr_type = 0;
  uint64_t arr_n = 0;
};

struct TensorInfo {
  uint32_t type = 0;
  int n_dims = 0;
  uint64_t ne[4] = {1, 1, 1, 1};
  uint64_t offset = 0;  // from the start of the data section
  const uint8_t* data = nullptr;
  size_t bytes = 0;
};

// ggml block sizes / bytes of the types a tensor table may hold (for the data
// bounds check); 0 = unknown type.
void type_geometry(uint32_t t, int* blck, size_t* bytes) {
  switch (t) {
    case 0: *blck = 1; *bytes = 4; return;      // F32
    case 1: *blck = 1; *bytes = 2; return;      // F16
    case 2: *blck = 32; *bytes = 18; return;    // Q4_0
    case 3: *blck = 32; *bytes = 20; return;    // Q4_1
    case 6: *blck = 32; *bytes = 22; return;    // Q5_0
    case 7: *blck = 32; *bytes = 24; return;    // Q5_1
    case 8: *blck = 32; *bytes = 34; return;    // Q8_0
    case 10: *blck = 256; *bytes = 84; return;  // Q2_K
    case 11: *blck = 256; *bytes = 110; return; // Q3_K
    case 12: *blck = 256; *bytes = 144; return; // Q4_K
    case 13: *blck = 256; *bytes = 176; return; // Q5_K
    case 14: *blck = 256; *bytes = 210; return; // Q6_K
    case 30: *blck = 1; *bytes = 2; return;     // BF16
    default: *blck = 0; *bytes = 0; return;
  }
}

struct Reader {
  const uint8_t* p;
  size_t n, off = 0;
  bool ok = true;
  bool need(size_t k) {
    if (!ok || k > n - off) ok = false;
    return ok;
  }
  template <class T>
  T get() {
    T v{};
    if (need(sizeof(T))) {
      std::memcpy(&v, p + off, sizeof(T));
      off += sizeof(T);
    }
    return v;
  }
  std::string str() {
    const uint64_t len = get<uint64_t>();
    if (!ok || len > (uint64_t)(n - off)) {
      ok = false;
      return {};
    }
    std::string s((const char*)p + off, (size_t)len);
    off += (size_t)len;
    return s;
  }
  void skip(size_t k) {
    if (need(k)) off += k;
  }
};

size_t scalar_size(uint32_t t) {
  switch (t) {
    case GG_U8: case GG_I8: case GG_BOOL: return 1;
    case GG_U16: case GG_I16: return 2;
    case GG_U32: case GG_I32: case GG_F32: return 4;
    case GG_U64: case GG_I64: case GG_F64: return 8;
    default: return 0;
  }
}

void read_scalar(Reader& r, uint32_t t, Value& v) {
  switch (t) {
    case GG_U8: v.u = r.get<uint8_t>(); v.i = (int64_t)v.u; v.f = (double)v.u; break;
    case GG_I8: v.i = r.get<int8_t>(); v.u = (uint64_t)v.i; v.f = (double)v.i; break;
    case GG_U16: v.u = r.get<uint16_t>(); v.i = (int64_t)v.u; v.f = (double)v.u; break;
    case GG_I16: v.i = r.get<int16_t>(); v.u = (uint64_t)v.i; v.f = (double)v.i; break;
    case GG_U32: v.u = r.get<uint32_t>(); v.i = (int64_t)v.u; v.f = (double)v.u; break;
    case GG_I32: v.i = r.get<int32_t>(); v.u = (uint64_t)v.i; v.f = (double)v.i; break;
    case GG_F32: v.f = r.get<float>(); break;
    case GG_BOOL: v.u = r.get<uint8_t>() != 0; v.i = (int64_t)v.u; break;
    case GG_U64: v.u = r.get<uint64_t>(); v.i = (int64_t)v.u; v.f = (double)v.u; break;
    case GG_I64: v.i = r.get<int64_t>(); v.u = (uint64_t)v.i; v.f = (double)v.i; break;
    case GG_F64: v.f = r.get<double>(); break;
    default: r.ok = false;
  }
}

}  // namespace

struct mtg_gguf {
  std::string error;
  int code = MTG_OK;
  void* map = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  std::map<std::string, Value> kv;
  std::map<std::string, TensorInfo> tensors;
  std::vector<std::string> order;  // tensor names in file order
  // the decoder view, built by mtg_gguf_model
  mtg_model_desc desc{};
  std::vector<mtg_layer_tensors> layers;
  std::vector<std::vector<float>> widened;  // f16 norm gains as f32
  // the encoder view, built by mtg_gguf_encoder
  mtg_encoder_desc enc{};
  std::vector<mtg_encoder_layer> enc_layers;
  std::deque<std::vector<float>> enc_widened;  // f16 vectors as f32 (stable addresses)
  ~mtg_gguf() {
    if (map) munmap(map, size);
  }
  int fail(int c, const std::string& msg) {
    error = msg;
    code = c;
    return c;
  }
  uint64_t get_u(const char* key, uint64_t dflt) const {
    auto it = kv.find(key);
    if (it == kv.end() || it->second.type == GG_STR || it->second.type == GG_ARR || it->second.type == GG_F32 ||
        it->second.type == GG_F64)
      return dflt;
    return it->second.u;
  }
  double get_f(const char* key, double dflt) const {
    auto it = kv.find(key);
    if (it == kv.end()) return dflt;
    if (it->second.type == GG_F32 || it->second.type == GG_F64) return it->second.f;
    if (scalar_size(it->second.type)) return (double)it->second.i;
    return dflt;
  }
};

namespace {
thread_local std::string g_gguf_error;

int parse(mtg_gguf& g) {
  Reader r{(const uint8_t*)g.map, g.size};
  const uint32_t magic = r.get<uint32_t>();
  if (!r.ok || magic != 0x46554747u) return g.fail(MTG_ERR_INVALID, "not a GGUF file (bad magic)");
  g.version = r.get<uint32_t>();
  if (g.version != 2 && g.version != 3) return g.fail(MTG_ERR_UNSUPPORTED, "GGUF version " + std::to_string(g.version));
  const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
  if (!r.ok || n_tensors > (1u << 24) || n_kv > (1u << 24)) return g.fail(MTG_ERR_INVALID, "GGUF header truncated");
  for (uint64_t i = 0; i < n_kv && r.ok; ++i) {
    std::string key = r.str();
    Value v;
    v.type = r.get<uint32_t>();
    if (v.type == GG_STR) {
      v.s = r.str();
    } else if (v.type == GG_ARR) {
      v.arr_type = r.get<uint32_t>();
      v.arr_n = r.get<uint64_t>();
      if (v.arr_type == GG_STR) {
        for (uint64_t j = 0; j < v.arr_n && r.ok; ++j) (void)r.str();
      } else {
        const size_t es = scalar_size(v.arr_type);
        if (!es || v.arr_n > (uint64_t)(r.n - r.off) / es) r.ok = false;
        else r.skip((size_t)v.arr_n * es);
      }
    } else {
      read_scalar(r, v.type, v);
    }
    if (r.ok) g.kv[key] = v;
  }
  if (!r.ok) return g.fail(MTG_ERR_INVALID, "GGUF metadata truncated or malformed");
  for (uint64_t i = 0; i < n_tensors && r.ok; ++i) {
    std::string name = r.str();
    TensorInfo t;
    t.n_dims = (int)r.get<uint32_t>();
    if (t.n_dims < 1 || t.n_dims > 4) r.ok = false;
    for (int d = 0; d < t.n_dims && r.ok; ++d) t.ne[d] = r.get<uint64_t>();
    t.type = r.get<uint32_t>();
    t.offset = r.get<uint64_t>();
    if (r.ok) {
      if (g.tensors.count(name)) return g.fail(MTG_ERR_INVALID, "duplicate tensor " + name);
      g.order.push_back(name);
      g.tensors[name] = t;
    }
  }
  if (!r.ok) return g.fail(MTG_ERR_INVALID, "GGUF tensor table truncated or malformed");
  const uint64_t align = g.get_u("general.alignment", 32);
  if (align == 0 || (align & (align - 1))) return g.fail(MTG_ERR_INVALID, "bad general.alignment");
  const size_t data_off = (size_t)((r.off + align - 1) / align * align);
  for (auto& kvp : g.tensors) {
    TensorInfo& t = kvp.second;
    int blck = 0;
    size_t bb = 0;
    type_geometry(t.type, &blck, &bb);
    if (!blck) continue;  // unknown type: the model check rejects it if it is used
    uint64_t nel = 1;
    for (int d = 0; d < 4; ++d) {
      if (t.ne[d] && nel > ~0ull / t.ne[d]) return g.fail(MTG_ERR_INVALID, "tensor too large: " + kvp.first);
      nel *= t.ne[d];
    }
    if (t.ne[0] % (uint64_t)blck) return g.fail(MTG_ERR_INVALID, "row not a whole number of blocks: " + kvp.first);
    t.bytes = (size_t)(nel / (uint64_t)blck * bb);
    if (t.offset % align || data_off > g.size || t.offset > g.size - data_off || t.bytes > g.size - data_off - t.offset)
      return g.fail(MTG_ERR_INVALID, "tensor data outside the file: " + kvp.first);
    t.data = (const uint8_t*)g.map + data_off + t.offset;
  }
  return MTG_OK;
}

const char* type_name(uint32_t t) {
  switch (t) {
    case 0: return "f32";
    case 1: return "f16";
    case 8: return "q8_0";
    case 12: return "q4_K";
    default: return "other";
  }
}

}  // namespace

extern "C" {

int mtg_gguf_open(const char* path, mtg_gguf** out) {
  if (!out) return MTG_ERR_INVALID;
  *out = nullptr;
  g_gguf_error.clear();
  if (!path) return MTG_ERR_INVALID;
  auto g = std::unique_ptr<mtg_gguf>(new (std::nothrow) mtg_gguf());
  if (!g) return MTG_ERR_NOMEM;
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) {
    g_gguf_error = std::string("cannot open ") + path;
    mtg::set_call_error(g_gguf_error);
    return MTG_ERR_INVALID;
  }
  struct stat st {};
  if (fstat(fd, &st) != 0 || st.st_size < 24) {
    ::close(fd);
    g_gguf_error = std::string("not a GGUF file (too short): ") + path;
    return MTG_ERR_INVALID;
  }
  g->size = (size_t)st.st_size;
  g->map = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (g->map == MAP_FAILED) {
    g->map = nullptr;
    g_gguf_error = std::string("mmap failed: ") + path;
    return MTG_ERR_NOMEM;
  }
  try {
    const int rc = parse(*g);
    if (rc) {
      g_gguf_error = g->error;
      mtg::set_call_error(g->error);
      return rc;
    }
  } catch (...) {
    g_gguf_error = "GGUF parse: out of memory";
    return MTG_ERR_NOMEM;
  }
  *out = g.release();
  return MTG_OK;
}

void mtg_gguf_close(mtg_gguf* g) { delete g; }

const char* mtg_gguf_error(const mtg_gguf* g) { return g ? g->error.c_str() : g_gguf_error.c_str(); }

int64_t mtg_gguf_n_tensors(const mtg_gguf* g) { return g ? (int64_t)g->order.size() : 0; }

int mtg_gguf_tensor(const mtg_gguf* g, const char* name, int32_t* type, int64_t* ne, const void** data,
                    size_t* bytes) {
  if (!g || !name) return MTG_ERR_INVALID;
  auto it = g->tensors.find(name);
  if (it == g->tensors.end()) return MTG_ERR_INVALID;
  const TensorInfo& t = it->second;
  if (type) *type = (int32_t)t.type;
  if (ne)
    for (int d = 0; d < 4; ++d) ne[d] = (int64_t)t.ne[d];
  if (data) *data = t.data;
  if (bytes) *bytes = t.bytes;
  return MTG_OK;
}

// Hyper-parameters and tensors of the Qwen3 decoder (read_config's mtd.text.*
// keys with the same defaults; qwen3_load_layer's and Qwen3Decoder::load's
// names). The returned description points into the mapping (and, for f16 norm
// gains, into buffers the handle owns): valid until mtg_gguf_close.
const mtg_model_desc* mtg_gguf_model(mtg_gguf* g) {
  if (!g) return nullptr;
  try {
    mtg_hparams hp{};
    hp.vocab = (int32_t)g->get_u("mtd.text.vocab_size", 151936);
    hp.hidden = (int32_t)g->get_u("mtd.text.hidden", 1024);
    hp.intermediate = (int32_t)g->get_u("mtd.text.ffn", 3072);
    hp.n_layers = (int32_t)g->get_u("mtd.text.n_layers", 28);
    hp.n_heads = (int32_t)g->get_u("mtd.text.n_heads", 16);
    hp.n_kv_heads = (int32_t)g->get_u("mtd.text.n_kv_heads", 8);
    hp.head_dim = (int32_t)g->get_u("mtd.text.head_dim", 128);
    hp.rms_eps = (float)g->get_f("mtd.text.rms_eps", 1e-6);
    hp.rope_base = (float)g->get_f("mtd.text.rope_theta", 1e6);
    if (hp.vocab <= 0 || hp.hidden <= 0 || hp.intermediate <= 0 || hp.n_layers <= 0 || hp.n_heads <= 0 ||
        hp.n_kv_heads <= 0 || hp.head_dim <= 0) {
      g->fail(MTG_ERR_INVALID, "bad mtd.text.* hyper-parameters");
      return nullptr;
    }
    const int64_t H = hp.hidden, QN = (int64_t)hp.n_heads * hp.head_dim, KN = (int64_t)hp.n_kv_heads * hp.head_dim,
                  F = hp.intermediate, D = hp.head_dim;
    auto find = [&](const std::string& name, const TensorInfo** t) -> bool {
      auto it = g->tensors.find(name);
      if (it == g->tensors.end()) {
        g->fail(MTG_ERR_INVALID, "missing tensor " + name);
        return false;
      }
      *t = &it->second;
      return true;
    };
    const TensorInfo* embd = nullptr;
    if (!find("token_embd.weight", &embd)) return nullptr;
    const uint32_t wtype = embd->type;
    if (wtype != MTG_TYPE_Q8_0 && wtype != MTG_TYPE_F16 && wtype != MTG_TYPE_F32 && wtype != MTG_TYPE_Q4_K) {
      g->fail(MTG_ERR_UNSUPPORTED, std::string("weight type ") + type_name(wtype) + " (" + std::to_string(wtype) +
                                       ") is not supported: q8_0, f16, f32 or q4_K");
      return nullptr;
    }
    auto matrix = [&](const std::string& name, int64_t k, int64_t n, const void** out) -> bool {
      const TensorInfo* t = nullptr;
      if (!find(name, &t)) return false;
      if (t->type != wtype) {
        g->fail(MTG_ERR_UNSUPPORTED, name + " is " + type_name(t->type) + ", token_embd.weight " + type_name(wtype) +
                                         ": mixed weight types are not supported");
        return false;
      }
      if (t->n_dims != 2 || (int64_t)t->ne[0] != k || (int64_t)t->ne[1] != n) {
        g->fail(MTG_ERR_INVALID, name + ": shape [" + std::to_string(t->ne[0]) + ", " + std::to_string(t->ne[1]) +
                                     "], expected [" + std::to_string(k) + ", " + std::to_string(n) + "]");
        return false;
      }
      *out = t->data;
      return true;
    };
    auto gain = [&](const std::string& name, int64_t n, const float** out) -> bool {
      const TensorInfo* t = nullptr;
      if (!find(name, &t)) return false;
      if (t->ne[0] != (uint64_t)n || t->ne[1] * t->ne[2] * t->ne[3] != 1) {
        g->fail(MTG_ERR_INVALID, name + ": expected " + std::to_string(n) + " elements");
        return false;
      }
      if (t->type == 0) {
        *out = (const float*)t->data;  // aligned by the data section's alignment
      } else if (t->type == 1) {
        g->widened.emplace_back((size_t)n);
        const uint16_t* h = (const uint16_t*)t->data;
        for (int64_t i = 0; i < n; ++i) g->widened.back()[(size_t)i] = mtg_f16_to_f32(h[i]);
        *out = g->widened.back().data();
      } else {
        g->fail(MTG_ERR_UNSUPPORTED, name + ": norm gains must be f32 or f16");
        return false;
      }
      return true;
    };
    g->widened.clear();
    g->widened.reserve((size_t)hp.n_layers * 4 + 1);
    g->layers.assign((size_t)hp.n_layers, mtg_layer_tensors{});
    if (!matrix("token_embd.weight", H, hp.vocab, &g->desc.token_embd)) return nullptr;
    for (int i = 0; i < hp.n_layers; ++i) {
      mtg_layer_tensors& L = g->layers[(size_t)i];
      const std::string b = "qwen3.blk." + std::to_string(i) + ".";
      if (!gain(b + "attn_norm.weight", H, &L.attn_norm) || !matrix(b + "attn_q.weight", H, QN, &L.attn_q) ||
          !matrix(b + "attn_k.weight", H, KN, &L.attn_k) || !matrix(b + "attn_v.weight", H, KN, &L.attn_v) ||
          !matrix(b + "attn_o.weight", QN, H, &L.attn_o) || !gain(b + "attn_q_norm.weight", D, &L.attn_q_norm) ||
          !gain(b + "attn_k_norm.weight", D, &L.attn_k_norm) || !gain(b + "ffn_norm.weight", H, &L.ffn_norm) ||
          !matrix(b + "ffn_gate.weight", H, F, &L.ffn_gate) || !matrix(b + "ffn_up.weight", H, F, &L.ffn_up) ||
          !matrix(b + "ffn_down.weight", F, H, &L.ffn_down))
        return nullptr;
    }
    if (!gain("qwen3.output_norm.weight", H, &g->desc.output_norm)) return nullptr;
    g->desc.hp = hp;
    g->desc.weight_type = (int32_t)wtype;
    g->desc.layers = g->layers.data();
    return &g->desc;
  } catch (...) {
    g->fail(MTG_ERR_NOMEM, "out of memory");
    return nullptr;
  }
}

// The Whisper encoder + adaptor tensors (reference WhisperEncoder /
// AudioAdaptor constructors, src/whisper_encoder.cpp:64-95,
// src/audio_adaptor.cpp:22-34) and the mtd.audio.* / adaptor keys with
// read_config's defaults (src/model_loader.cpp:130-144).
const mtg_encoder_desc* mtg_gguf_encoder(mtg_gguf* g) {
  if (!g) return nullptr;
  try {
    mtg_encoder_hparams hp{};
    hp.n_mels = (int32_t)g->get_u("mtd.audio.mel_bins", 80);
    hp.d_model = (int32_t)g->get_u("mtd.audio.d_model", 1024);
    hp.n_layers = (int32_t)g->get_u("mtd.audio.n_layers", 24);
    hp.n_heads = (int32_t)g->get_u("mtd.audio.n_heads", 16);
    hp.ffn = (int32_t)g->get_u("mtd.audio.ffn", 4096);
    const int64_t src_pos = (int64_t)g->get_u("mtd.audio.max_src_pos", 1500);
    hp.n_frames = (int32_t)(2 * src_pos);
    hp.merge = (int32_t)g->get_u("mtd.audio_merge_size", 4);
    hp.hidden = (int32_t)g->get_u("mtd.text.hidden", 1024);
    hp.adaptor_eps = (float)g->get_f("mtd.adaptor_norm_eps", 1e-6);
    if (hp.n_mels <= 0 || hp.d_model <= 0 || hp.n_layers < 0 || hp.n_heads <= 0 || hp.ffn <= 0 || src_pos <= 0 ||
        hp.merge <= 0 || hp.hidden <= 0) {
      g->fail(MTG_ERR_INVALID, "bad mtd.audio.* hyper-parameters");
      return nullptr;
    }
    const int64_t D = hp.d_model, F = hp.ffn, M = hp.n_mels, H = hp.hidden, IN = D * hp.merge;
    const TensorInfo* q0 = nullptr;
    auto find = [&](const std::string& name, const TensorInfo** t) -> bool {
      auto it = g->tensors.find(name);
      if (it == g->tensors.end()) {
        g->fail(MTG_ERR_INVALID, "missing tensor " + name);
        return false;
      }
      *t = &it->second;
      return true;
    };
    // the matrices' type: the converter writes f32, f16 or q8_0 (--dtype), and
    // `cli quantize q4_k` turns the encoder and adaptor matrices into q4_K
    // (src/cli.cpp:106-130); all of them share it
    if (!find(hp.n_layers > 0 ? "enc.blk.0.attn_q.w" : "adaptor.fc1.w", &q0)) return nullptr;
    const uint32_t wtype = q0->type;
    if (wtype != MTG_TYPE_Q8_0 && wtype != MTG_TYPE_F16 && wtype != MTG_TYPE_F32 && wtype != MTG_TYPE_Q4_K) {
      g->fail(MTG_ERR_UNSUPPORTED, std::string("encoder weight type ") + type_name(wtype) +
                                       " is not supported: q8_0, f16, f32 or q4_K");
      return nullptr;
    }
    auto matrix = [&](const std::string& name, int64_t k, int64_t n, const void** out) -> bool {
      const TensorInfo* t = nullptr;
      if (!find(name, &t)) return false;
      if (t->type != wtype) {
        g->fail(MTG_ERR_UNSUPPORTED, name + " is " + type_name(t->type) + ": the encoder matrices must all be " +
                                         type_name(wtype));
        return false;
      }
      if (t->n_dims != 2 || (int64_t)t->ne[0] != k || (int64_t)t->ne[1] != n) {
        g->fail(MTG_ERR_INVALID, name + ": shape [" + std::to_string(t->ne[0]) + ", " + std::to_string(t->ne[1]) +
                                     "], expected [" + std::to_string(k) + ", " + std::to_string(n) + "]");
        return false;
      }
      *out = t->data;
      return true;
    };
    // f32 (or f16, widened) tensor of n elements in any shape
    auto vec = [&](const std::string& name, int64_t n, const float** out) -> bool {
      const TensorInfo* t = nullptr;
      if (!find(name, &t)) return false;
      if ((int64_t)(t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]) != n) {
        g->fail(MTG_ERR_INVALID, name + ": expected " + std::to_string(n) + " elements");
        return false;
      }
      if (t->type == 0) {
        *out = (const float*)t->data;
      } else if (t->type == 1) {
        g->enc_widened.emplace_back((size_t)n);
        const uint16_t* h = (const uint16_t*)t->data;
        for (int64_t i = 0; i < n; ++i) g->enc_widened.back()[(size_t)i] = mtg_f16_to_f32(h[i]);
        *out = g->enc_widened.back().data();
      } else {
        g->fail(MTG_ERR_UNSUPPORTED, name + ": must be f32 or f16");
        return false;
      }
      return true;
    };
    g->enc_widened.clear();
    mtg_encoder_desc& e = g->enc;
    e = mtg_encoder_desc{};
    if (!vec("enc.conv1.w", D * M * 3, &e.conv1_w) || !vec("enc.conv1.b", D, &e.conv1_b) ||
        !vec("enc.conv2.w", D * D * 3, &e.conv2_w) || !vec("enc.conv2.b", D, &e.conv2_b) ||
        !vec("enc.pos_embd", src_pos * D, &e.pos_embd) || !vec("enc.ln_post.w", D, &e.ln_post_w) ||
        !vec("enc.ln_post.b", D, &e.ln_post_b))
      return nullptr;
    g->enc_layers.assign((size_t)hp.n_layers, mtg_encoder_layer{});
    for (int i = 0; i < hp.n_layers; ++i) {
      mtg_encoder_layer& L = g->enc_layers[(size_t)i];
      const std::string b = "enc.blk." + std::to_string(i) + ".";
      if (!vec(b + "attn_ln.w", D, &L.attn_ln_w) || !vec(b + "attn_ln.b", D, &L.attn_ln_b) ||
          !matrix(b + "attn_q.w", D, D, &L.q_w) || !vec(b + "attn_q.b", D, &L.q_b) ||
          !matrix(b + "attn_k.w", D, D, &L.k_w) || !matrix(b + "attn_v.w", D, D, &L.v_w) ||
          !vec(b + "attn_v.b", D, &L.v_b) || !matrix(b + "attn_out.w", D, D, &L.o_w) ||
          !vec(b + "attn_out.b", D, &L.o_b) || !vec(b + "ffn_ln.w", D, &L.ffn_ln_w) ||
          !vec(b + "ffn_ln.b", D, &L.ffn_ln_b) || !matrix(b + "ffn_1.w", D, F, &L.fc1_w) ||
          !vec(b + "ffn_1.b", F, &L.fc1_b) || !matrix(b + "ffn_2.w", F, D, &L.fc2_w) ||
          !vec(b + "ffn_2.b", D, &L.fc2_b))
        return nullptr;
    }
    if (!matrix("adaptor.fc1.w", IN, H, &e.ad_fc1_w) || !vec("adaptor.fc1.b", H, &e.ad_fc1_b) ||
        !matrix("adaptor.fc2.w", H, H, &e.ad_fc2_w) || !vec("adaptor.fc2.b", H, &e.ad_fc2_b) ||
        !vec("adaptor.ln.w", H, &e.ad_ln_w) || !vec("adaptor.ln.b", H, &e.ad_ln_b))
      return nullptr;
    e.hp = hp;
    e.weight_type = (int32_t)wtype;
    e.layers = g->enc_layers.data();
    return &e;
  } catch (...) {
    g->fail(MTG_ERR_NOMEM, "out of memory");
    return nullptr;
  }
}

int mtg_encoder_create_from_gguf(const char* path, mtg_encoder** out) {
  if (!out) return MTG_ERR_INVALID;
  *out = nullptr;
  mtg_gguf* g = nullptr;
  int rc = mtg_gguf_open(path, &g);
  if (rc) return rc;
  const mtg_encoder_desc* d = mtg_gguf_encoder(g);
  if (!d) {
    g_gguf_error = g->error;
    rc = g->code ? g->code : MTG_ERR_INVALID;
    mtg_gguf_close(g);
    return rc;
  }
  rc = mtg_encoder_create(d, out);
  mtg_gguf_close(g);  // the encoder holds its own copies
  return rc;
}

int mtg_create_from_gguf(const char* path, int32_t max_seq, int32_t kv_type, mtg_ctx** out) {
  if (!out) return MTG_ERR_INVALID;
  *out = nullptr;
  mtg_gguf* g = nullptr;
  int rc = mtg_gguf_open(path, &g);
  if (rc) return rc;
  const mtg_model_desc* d = mtg_gguf_model(g);
  if (!d) {
    g_gguf_error = g->error;
    mtg::set_call_error(g->error);
    rc = g->code ? g->code : MTG_ERR_INVALID;
    mtg_gguf_close(g);
    return rc;
  }
  rc = mtg_create(d, max_seq, kv_type, out);
  mtg_gguf_close(g);  // mtg_create uploaded the tensors
  return rc;
}

}  // extern "C"
