// runtime.cpp - device decoder state and the verify step (host side).
//
// Replaces Qwen3Decoder (src/qwen3_decoder.cpp:20-205) and the graph execution of
// src/backend.cpp:216-240 for the verify path: weights are uploaded once and
// re-tiled into MFMA panels, the KV cache stays resident in HBM, and one verify
// step is a fixed kernel sequence replayed from a captured HIP graph (one graph per
// column-group count and penalty mode); only the step descriptor goes in and
// T + 2 ints come back per step.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "runtime.hpp"

namespace mtg {

namespace {

size_t q8_tiles_bytes(int n, int k) { return (size_t)(n / 16) * (k / kPairK) * kUnitBytes; }

}  // namespace

Ctx::~Ctx() {
  for (auto& g : graphs)
    if (g.exec) hipGraphExecDestroy(g.exec);
  for (void* p : allocations) hipFree(p);
  if (gen_ids_dev) hipFree(gen_ids_dev);
  if (gen_aux_dev) hipFree(gen_aux_dev);
  if (gen_state_dev) hipFree(gen_state_dev);
  if (gen_state_host) hipHostFree(gen_state_host);
  for (auto& slot : gen_events)
    for (auto& e : slot)
      if (e) hipEventDestroy(e);
  for (auto& e : gen_chunk_ev)
    if (e) hipEventDestroy(e);
  if (ev_start) hipEventDestroy(ev_start);
  if (ev_stop) hipEventDestroy(ev_stop);
  if (desc_host) hipHostFree(desc_host);
  if (result_host) hipHostFree(result_host);
  if (stream) hipStreamDestroy(stream);
}

int Ctx::fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  error = buf;
  return code;
}

int Ctx::check(hipError_t e, const char* what) {
  if (e == hipSuccess) return MTG_OK;
  return fail(MTG_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

void* Ctx::dalloc(size_t bytes, bool zero) {
  void* p = nullptr;
  if (hipMalloc(&p, bytes ? bytes : 16) != hipSuccess) return nullptr;
  allocations.push_back(p);
  if (zero && hipMemset(p, 0, bytes ? bytes : 16) != hipSuccess) return nullptr;
  return p;
}

int Ctx::upload_q8(const void* blocks, int n, int k, uint8_t* dst, uint8_t* staging) {
  const size_t raw = (size_t)n * (k / 32) * 34;
  int rc = check(hipMemcpyAsync(staging, blocks, raw, hipMemcpyHostToDevice, stream), "upload weights");
  if (rc) return rc;
  launch_q8_retile(stream, staging, n, k, dst);
  rc = check(hipGetLastError(), "retile launch");
  if (rc) return rc;
  return check(hipStreamSynchronize(stream), "retile");
}

size_t Ctx::weight_bytes(int n, int k) const {
  if (wtype == MTG_TYPE_Q8_0) return q8_tiles_bytes(n, k);
  if (wtype == MTG_TYPE_F16) return (size_t)n * k * 2;
  if (wtype == MTG_TYPE_F32) return (size_t)n * k * 4;
  return (size_t)n * (k / 256) * 144;  // q4_K
}

int Ctx::upload_weights(const void* src, int n, int k, uint8_t* dst, uint8_t* staging) {
  if (wtype == MTG_TYPE_Q8_0) return upload_q8(src, n, k, dst, staging);
  return check(hipMemcpy(dst, src, weight_bytes(n, k), hipMemcpyHostToDevice), "upload weights");
}

int Ctx::init(const mtg_model_desc* d, int max_seq_in, int kv_type_in) {
  hp = d->hp;
  max_seq = max_seq_in;
  kv_type = kv_type_in;
  const int H = hp.hidden, D = hp.head_dim, NH = hp.n_heads, NKV = hp.n_kv_heads;
  const int QN = NH * D, KN = NKV * D, F = hp.intermediate, L = hp.n_layers, V = hp.vocab;
  wtype = d->weight_type;
  if (wtype != MTG_TYPE_Q8_0 && wtype != MTG_TYPE_F16 && wtype != MTG_TYPE_F32 && wtype != MTG_TYPE_Q4_K)
    return fail(MTG_ERR_UNSUPPORTED, "weight type %d is not supported", wtype);
  if (wtype != MTG_TYPE_Q8_0 && (!wt_shape_supported(wtype, H) || !wt_shape_supported(wtype, QN) ||
                                 !wt_shape_supported(wtype, F)))
    return fail(MTG_ERR_UNSUPPORTED, "shape not supported for weight type %d (f16, f32: K of 1024, 2048 or "
                "3072; q4_K: K a multiple of 256)", wtype);
  if ((wtype == MTG_TYPE_F16 || wtype == MTG_TYPE_F32) && H != 1024)
    return fail(MTG_ERR_UNSUPPORTED, "f16 and f32 weights need hidden 1024 (their lm_head kernels)");
  if ((wtype == MTG_TYPE_F16 || wtype == MTG_TYPE_F32) && weight_bytes(V, H) >= ((size_t)1 << 31))
    return fail(MTG_ERR_UNSUPPORTED, "f16 / f32 weights: the lm_head's copy of token_embd must stay under 2 GiB");
  if (kv_type != MTG_TYPE_F32 && kv_type != MTG_TYPE_F16)
    return fail(MTG_ERR_UNSUPPORTED, "kv type %d", kv_type);
  if (D != kHeadDim || NH != 2 * NKV || H % kPairK || QN % kPairK || F % kPairK || V % 16 ||
      H % 16 || F % 16 || L <= 0 || max_seq <= 0)
    return fail(MTG_ERR_UNSUPPORTED,
                "shape not supported: head_dim 128, n_heads = 2*n_kv_heads, hidden/intermediate "
                "multiples of 64, vocab multiple of 16");
  int rc = check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "stream");
  if (rc) return rc;
  if (const char* cc = std::getenv("ROCPROF_COUNTER_COLLECTION"))
    counter_collection = cc[0] != '\0' && std::strcmp(cc, "0") != 0 && std::strcmp(cc, "false") != 0 &&
                         std::strcmp(cc, "False") != 0;
  if (hipHostMalloc((void**)&desc_host, sizeof(StepDesc), hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc((void**)&result_host, sizeof(StepResult), hipHostMallocDefault) != hipSuccess)
    return fail(MTG_ERR_NOMEM, "pinned host buffers");
  std::memset(desc_host, 0, sizeof(StepDesc));
  std::memset(result_host, 0, sizeof(StepResult));
  if (hipHostGetDevicePointer((void**)&result_map, result_host, 0) != hipSuccess)
    return fail(MTG_ERR_DEVICE, "mapped result buffer");

  // weights
  uint8_t* staging = nullptr;  // q8_0 rows before the re-tiling
  if (wtype == MTG_TYPE_Q8_0) {
    size_t staging_bytes = (size_t)V * (H / 32) * 34;
    staging_bytes = std::max(staging_bytes, (size_t)F * (H / 32) * 34);
    staging_bytes = std::max(staging_bytes, (size_t)H * (F / 32) * 34);
    staging = (uint8_t*)dalloc(staging_bytes, false);
    if (!staging) return fail(MTG_ERR_NOMEM, "staging buffer");
  }
  layers.resize(L);
  const int NQKV = QN + 2 * KN;
  for (int l = 0; l < L; ++l) {
    const mtg_layer_tensors& s = d->layers[l];
    Layer& y = layers[l];
    y.wqkv = (uint8_t*)dalloc(weight_bytes(NQKV, H), false);
    y.wo = (uint8_t*)dalloc(weight_bytes(H, QN), false);
    y.wg = (uint8_t*)dalloc(weight_bytes(F, H), false);
    y.wu = (uint8_t*)dalloc(weight_bytes(F, H), false);
    y.wd = (uint8_t*)dalloc(weight_bytes(H, F), false);
    y.attn_norm = (float*)dalloc(H * 4, false);
    y.ffn_norm = (float*)dalloc(H * 4, false);
    y.q_norm = (float*)dalloc(D * 4, false);
    y.k_norm = (float*)dalloc(D * 4, false);
    if (!y.wqkv || !y.wo || !y.wg || !y.wu || !y.wd || !y.attn_norm || !y.ffn_norm || !y.q_norm ||
        !y.k_norm)
      return fail(MTG_ERR_NOMEM, "layer %d weights", l);
    if ((rc = upload_weights(s.attn_q, QN, H, y.wqkv, staging))) return rc;
    if ((rc = upload_weights(s.attn_k, KN, H, y.wqkv + weight_bytes(QN, H), staging))) return rc;
    if ((rc = upload_weights(s.attn_v, KN, H, y.wqkv + weight_bytes(QN + KN, H), staging))) return rc;
    if ((rc = upload_weights(s.attn_o, H, QN, y.wo, staging))) return rc;
    if ((rc = upload_weights(s.ffn_gate, F, H, y.wg, staging))) return rc;
    if ((rc = upload_weights(s.ffn_up, F, H, y.wu, staging))) return rc;
    if ((rc = upload_weights(s.ffn_down, H, F, y.wd, staging))) return rc;
    if ((rc = check(hipMemcpy(y.attn_norm, s.attn_norm, H * 4, hipMemcpyHostToDevice), "norms")) ||
        (rc = check(hipMemcpy(y.ffn_norm, s.ffn_norm, H * 4, hipMemcpyHostToDevice), "norms")) ||
        (rc = check(hipMemcpy(y.q_norm, s.attn_q_norm, D * 4, hipMemcpyHostToDevice), "norms")) ||
        (rc = check(hipMemcpy(y.k_norm, s.attn_k_norm, D * 4, hipMemcpyHostToDevice), "norms")))
      return rc;
  }
  embd = (uint8_t*)dalloc(weight_bytes(V, H), false);
  out_norm = (float*)dalloc(H * 4, false);
  if (!embd || !out_norm) return fail(MTG_ERR_NOMEM, "token_embd");
  if ((rc = upload_weights(d->token_embd, V, H, embd, staging))) return rc;
  if (wtype == MTG_TYPE_F16 || wtype == MTG_TYPE_F32) {  // the lm_head reads a copy in its MFMA operand order
    lm_copy = (uint8_t*)dalloc(weight_bytes(V, H), false);
    if (!lm_copy) return fail(MTG_ERR_NOMEM, "lm_head copy of token_embd");
    launch_lm16_retile(stream, wtype, embd, V, lm_copy);
    if ((rc = check(hipGetLastError(), "lm_head copy launch")) || (rc = check(hipStreamSynchronize(stream), "lm_head copy")))
      return rc;
  }
  if ((rc = check(hipMemcpy(out_norm, d->output_norm, H * 4, hipMemcpyHostToDevice), "norms")))
    return rc;
  if (staging) {
    hipFree(staging);
    allocations.erase(std::find(allocations.begin(), allocations.end(), (void*)staging));
  }

  // RoPE table: the float recurrence of ggml's rope cache, built once on the host.
  std::vector<float> table((size_t)max_seq * D);
  const float theta_scale = std::pow(hp.rope_base, -2.0f / (float)D);
  for (int p = 0; p < max_seq; ++p) {
    float theta = (float)p;
    for (int i = 0; i < D / 2; ++i) {
      table[(size_t)p * D + 2 * i] = std::cos(theta);
      table[(size_t)p * D + 2 * i + 1] = std::sin(theta);
      theta *= theta_scale;
    }
  }
  rope = (float*)dalloc(table.size() * 4, false);
  if (!rope) return fail(MTG_ERR_NOMEM, "rope table");
  if ((rc = check(hipMemcpy(rope, table.data(), table.size() * 4, hipMemcpyHostToDevice), "rope")))
    return rc;

  // KV cache
  const size_t es = kv_type == MTG_TYPE_F32 ? 4 : 2;
  kv_layer_bytes = (size_t)NKV * max_seq * D * es;
  kcache = (uint8_t*)dalloc(kv_layer_bytes * L, true);
  vcache = (uint8_t*)dalloc(kv_layer_bytes * L, true);
  if (!kcache || !vcache) return fail(MTG_ERR_NOMEM, "KV cache of %d positions", max_seq);

  // activations and step buffers
  const int R = kMaxRows;
  x = (float*)dalloc((size_t)R * H * 4, true);
  qkv = (float*)dalloc((size_t)R * NQKV * 4, true);
  qbuf = (float*)dalloc((size_t)R * QN * 4, true);
  obuf = (float*)dalloc((size_t)R * QN * 4, true);
  act = (float*)dalloc((size_t)R * F * 4, true);
  hid = (float*)dalloc((size_t)R * H * 4, true);
  embeds_dev = (float*)dalloc((size_t)R * H * 4, true);
  logits = (float*)dalloc((size_t)R * V * 4, true);
  bitmap = (uint32_t*)dalloc((size_t)R * ((V + 31) / 32) * 4, true);
  part_keys = (uint64_t*)dalloc((size_t)kLmWorkgroups * R * 8, true);
  auto panel = [&](int K) {
    Panel p;
    p.codes = (uint8_t*)dalloc((size_t)kMaxGroups * (K / kPairK) * 1024, true);
    p.scales = (float*)dalloc((size_t)kMaxGroups * (K / kPairK) * 16 * 4, true);
    return p;
  };
  panel_h = panel(H);
  panel_o = panel(QN);
  panel_f = panel(F);
  if (wtype != MTG_TYPE_Q8_0) {
    const int KM = std::max(H, std::max(QN, F));
    wact.f16h = (uint16_t*)dalloc((size_t)R * KM * 2, true);
    wact.q8k.qs = (int8_t*)dalloc((size_t)R * KM, true);
    wact.q8k.d = (float*)dalloc((size_t)R * (KM / 256 + 1) * 4, true);
    wact.q8k.bsums = (int32_t*)dalloc((size_t)R * (KM / 16) * 4, true);
    if (wtype == MTG_TYPE_F32) wact.f32 = (float*)dalloc((size_t)R * KM * 4, true);
    if (!wact.f16h || !wact.q8k.qs || !wact.q8k.d || !wact.q8k.bsums || (wtype == MTG_TYPE_F32 && !wact.f32))
      return fail(MTG_ERR_NOMEM, "activation buffers");
  }
  const size_t chunks = (size_t)NKV * ((max_seq + kChunkKeys - 1) / kChunkKeys);
  work.part_ml = (float*)dalloc(chunks * kMaxCols * 2 * 4, true);
  work.part_o = (float*)dalloc(chunks * kMaxCols * D * 4, true);
  desc_dev = (StepDesc*)dalloc(sizeof(StepDesc), true);
  result_dev = (StepResult*)dalloc(sizeof(StepResult), true);
  if (!x || !qkv || !qbuf || !obuf || !act || !hid || !embeds_dev || !logits || !bitmap ||
      !part_keys || !panel_h.codes || !panel_h.scales || !panel_o.codes || !panel_o.scales ||
      !panel_f.codes || !panel_f.scales || !work.part_ml || !work.part_o || !desc_dev || !result_dev)
    return fail(MTG_ERR_NOMEM, "step buffers");
  if ((rc = check(prepare_kernels(), "kernel attributes"))) return rc;
  if ((rc = check(prepare_kernels_wt(), "kernel attributes"))) return rc;
  if ((rc = check(prepare_kernels_pf(), "kernel attributes"))) return rc;
  if ((rc = init_step_kernel())) return rc;
  return check(hipDeviceSynchronize(), "init");
}

// Parameters of the persistent step kernel: one workgroup per CU, the layer
// table and the per-workgroup partial buffers live in device memory.
int Ctx::init_step_kernel() {
  int dev = 0, cus = 0;
  int rc = check(hipGetDevice(&dev), "device");
  if (rc) return rc;
  if ((rc = check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "CU count")))
    return rc;
  const int H = hp.hidden, F = hp.intermediate, V = hp.vocab;
  // the persistent kernel streams q8_0 panel tiles, or f16 / f32 rows (8-row steps)
  if ((wtype != MTG_TYPE_Q8_0 && wtype != MTG_TYPE_F16 && wtype != MTG_TYPE_F32) ||
      !step_kernel_supported(H, hp.n_heads, hp.n_kv_heads, hp.head_dim, F, hp.n_layers, cus) ||
      prepare_step_kernels() != hipSuccess) {
    (void)hipGetLastError();
    exec = kExecGraph;  // other shapes and smaller devices: the per-op kernels
    return MTG_OK;
  }
  nwg = step_kernel_workgroups();
  std::vector<LayerDev> table(hp.n_layers);
  for (int l = 0; l < hp.n_layers; ++l) {
    const Layer& y = layers[l];
    LayerDev& d = table[l];
    d.wqkv = y.wqkv;
    d.wo = y.wo;
    d.wg = y.wg;
    d.wu = y.wu;
    d.wd = y.wd;
    d.attn_norm = y.attn_norm;
    d.ffn_norm = y.ffn_norm;
    d.q_norm = y.q_norm;
    d.k_norm = y.k_norm;
    d.kc = kcache + kv_layer_bytes * l;
    d.vc = vcache + kv_layer_bytes * l;
  }
  StepParams P{};
  for (int l = 0; l < hp.n_layers; ++l) P.layer[l] = table[l];
  P.H = H;
  P.NH = hp.n_heads;
  P.NKV = hp.n_kv_heads;
  P.F = F;
  P.V = V;
  P.L = hp.n_layers;
  P.max_seq = max_seq;
  P.kv_f16 = kv_type == MTG_TYPE_F16;
  P.eps = hp.rms_eps;
  P.embd = embd;
  P.lm_copy = lm_copy;
  P.out_norm = out_norm;
  P.rope = rope;
  P.embeds = embeds_dev;
  P.x = x;
  P.qkv = qkv;
  P.o = obuf;
  P.act = act;
  P.hid = hid;
  P.logits = logits;
  P.max_chunks = (max_seq + kChunkKeys - 1) / kChunkKeys;
  P.part_ml = work.part_ml;  // same layout as the per-op kernels
  P.part_o = work.part_o;
  P.bitmap = bitmap;
  P.part_keys = (uint64_t*)dalloc((size_t)nwg * kMaxRows * 8, true);
  P.oq = (int8_t*)dalloc((size_t)kMaxRows * hp.n_heads * hp.head_dim, true);
  P.oqs = (float*)dalloc((size_t)kMaxRows * hp.n_heads * hp.head_dim / 32 * 4, true);
  P.aq = (int8_t*)dalloc((size_t)kMaxRows * F, true);
  P.aqs = (float*)dalloc((size_t)kMaxRows * F / 32 * 4, true);
  if (wtype == MTG_TYPE_F16) {
    P.oh = (uint16_t*)dalloc((size_t)kMaxRows * hp.n_heads * hp.head_dim * 2, true);
    P.ah = (uint16_t*)dalloc((size_t)kMaxRows * F * 2, true);
    if (!P.oh || !P.ah) return fail(MTG_ERR_NOMEM, "step kernel buffers");
  }
  if (wtype == MTG_TYPE_F32) {
    P.o32 = (float*)dalloc((size_t)kMaxRows * hp.n_heads * hp.head_dim * 4, true);
    P.a32 = (float*)dalloc((size_t)kMaxRows * F * 4, true);
    if (!P.o32 || !P.a32) return fail(MTG_ERR_NOMEM, "step kernel buffers");
  }
  P.result = result_map;  // choices and n_match go straight to pinned host memory
  P.flags = (uint32_t*)dalloc((size_t)nwg * kFlagStride * 4, true);
  P.qkvt = (uint32_t*)dalloc(qkvt_bytes(), true);
  P.err = &result_dev->err;
  P.wait_polls = kWaitPolls;
  P.wait_ticks = kWaitTicks;
  P.timing = nullptr;
  params_dev = (StepParams*)dalloc(sizeof(StepParams), false);
  if (!P.part_ml || !P.part_o || !P.part_keys || !P.flags || !P.qkvt || !P.oq || !P.oqs || !P.aq || !P.aqs ||
      !params_dev)
    return fail(MTG_ERR_NOMEM, "step kernel buffers");
  if ((rc = check(hipMemcpy(params_dev, &P, sizeof(P), hipMemcpyHostToDevice), "step params")))
    return rc;
  params_host = P;
  step_ok = true;
  return MTG_OK;
}

KvLayer Ctx::kv_layer(int l) const {
  KvLayer k;
  k.k = kcache + kv_layer_bytes * l;
  k.v = vcache + kv_layer_bytes * l;
  k.f16 = kv_type == MTG_TYPE_F16;
  k.max_seq = max_seq;
  return k;
}

// The kernel sequence of one step (src/qwen3_decoder.cpp:91-160 + 174-205).
void Ctx::enqueue(int G, int mode) {
  const int H = hp.hidden, NH = hp.n_heads, NKV = hp.n_kv_heads, D = hp.head_dim;
  const int QN = NH * D, KN = NKV * D, F = hp.intermediate, V = hp.vocab;
  const float eps = hp.rms_eps;
  hipStream_t s = stream;
  if (wtype != MTG_TYPE_Q8_0) {
    enqueue_wt(mode);
    return;
  }
  if (mode != kModeLogits) {
    launch_embed(s, desc_dev, embd, H, embeds_dev, x);
    for (int l = 0; l < hp.n_layers; ++l) {
      const Layer& y = layers[l];
      const KvLayer kv = kv_layer(l);
      launch_norm_quant(s, desc_dev, x, H, y.attn_norm, eps, panel_h, nullptr);
      launch_gemm_store(s, G, desc_dev, y.wqkv, QN + 2 * KN, H, panel_h, qkv);
      launch_qk_rope_append(s, desc_dev, qkv, NH, NKV, y.q_norm, y.k_norm, eps, rope, qbuf, kv);
      launch_attention(s, desc_dev, qbuf, NH, NKV, kv, work, panel_o, obuf);
      launch_gemm_residual(s, G, desc_dev, y.wo, H, QN, panel_o, x);
      launch_norm_quant(s, desc_dev, x, H, y.ffn_norm, eps, panel_h, nullptr);
      launch_gemm_swiglu(s, G, desc_dev, y.wg, y.wu, F, H, panel_h, act);
      launch_norm_quant(s, desc_dev, act, F, nullptr, eps, panel_f, nullptr);
      launch_gemm_residual(s, G, desc_dev, y.wd, H, F, panel_f, x);
    }
    launch_norm_quant(s, desc_dev, x, H, out_norm, eps, panel_h, hid);
  } else {
    // logits of given final-normed rows: quantize them as they are
    launch_norm_quant(s, desc_dev, embeds_dev, H, nullptr, eps, panel_h, nullptr);
  }
  if (mode == kModeAppend) return;
  if (mode == kModeVerifyPenalty) launch_penalty_bitmap(s, desc_dev, V, bitmap);
  launch_lm_head(s, G, desc_dev, embd, V, H, panel_h, bitmap, logits, part_keys);
  launch_accept(s, desc_dev, part_keys, result_dev);
}

// The same step for f16 / q4_K weights: the activation of every GEMM is converted
// to the weight type's vec_dot_type first (kernels_wt.hip).
void Ctx::enqueue_wt(int mode) {
  const int H = hp.hidden, NH = hp.n_heads, NKV = hp.n_kv_heads, D = hp.head_dim;
  const int QN = NH * D, KN = NKV * D, F = hp.intermediate, V = hp.vocab;
  const float eps = hp.rms_eps;
  hipStream_t s = stream;
  if (mode != kModeLogits) {
    launch_embed_wt(s, wtype, desc_dev, embd, H, embeds_dev, x);
    for (int l = 0; l < hp.n_layers; ++l) {
      const Layer& y = layers[l];
      const KvLayer kv = kv_layer(l);
      if (wtype == MTG_TYPE_F16 && H == 1024) {  // the norm inside the f16 GEMM
        launch_gemm_f16_norm(s, 0, desc_dev, y.wqkv, nullptr, QN + 2 * KN, x, y.attn_norm, eps, qkv);
      } else {
        launch_act_wt(s, wtype, desc_dev, x, H, y.attn_norm, eps, wact, nullptr);
        launch_gemm_wt(s, wtype, 0, desc_dev, y.wqkv, nullptr, QN + 2 * KN, H, wact, qkv);
      }
      launch_qk_rope_append(s, desc_dev, qkv, NH, NKV, y.q_norm, y.k_norm, eps, rope, qbuf, kv);
      launch_attn_chunks(s, desc_dev, qbuf, NH, NKV, kv, work);
      launch_attn_combine_wt(s, wtype, desc_dev, work, NH, attn_max_chunks(kv), wact);
      launch_gemm_wt(s, wtype, 1, desc_dev, y.wo, nullptr, H, QN, wact, x);
      if (wtype == MTG_TYPE_F16 && H == 1024) {
        launch_gemm_f16_norm(s, 2, desc_dev, y.wg, y.wu, F, x, y.ffn_norm, eps, act);
      } else {
        launch_act_wt(s, wtype, desc_dev, x, H, y.ffn_norm, eps, wact, nullptr);
        launch_gemm_wt(s, wtype, 2, desc_dev, y.wg, y.wu, F, H, wact, act);
      }
      if (wtype == MTG_TYPE_F16 || wtype == MTG_TYPE_F32) {
        // the f16 gate/up GEMM leaves the SwiGLU rows as f16 in act's memory, the
        // f32 one as the f32 rows the down projection takes as they are
        WtAct down_in = wact;
        down_in.f16h = (uint16_t*)act;
        down_in.f32 = act;
        launch_gemm_wt(s, wtype, 1, desc_dev, y.wd, nullptr, H, F, down_in, x);
      } else {
        launch_act_wt(s, wtype, desc_dev, act, F, nullptr, eps, wact, nullptr);
        launch_gemm_wt(s, wtype, 1, desc_dev, y.wd, nullptr, H, F, wact, x);
      }
    }
    launch_act_wt(s, wtype, desc_dev, x, H, out_norm, eps, wact, hid);
  } else {
    launch_act_wt(s, wtype, desc_dev, embeds_dev, H, nullptr, eps, wact, nullptr);
  }
  if (mode == kModeAppend) return;
  if (mode == kModeVerifyPenalty) launch_penalty_bitmap(s, desc_dev, V, bitmap);
  launch_lm_head_wt(s, wtype, desc_dev, lm_copy ? lm_copy : embd, V, H, wact, bitmap, logits, part_keys);
  launch_accept(s, desc_dev, part_keys, result_dev);
}

int Ctx::run(int mode, int T, bool want_hidden, bool want_logits, float* hidden_out,
             float* logits_out) {
  const int G = (T + 7) / 8;
  int rc = MTG_OK;
  const bool step_mode = mode == kModeVerify || mode == kModeVerifyPenalty || mode == kModeAppend;
  // the f16- and f32-weight variants of the step kernel run steps of up to 8 rows;
  // longer ones, and steps beyond the KV length limit, take the per-op kernels
  const int max_keys = step_max_keys > 0 ? step_max_keys
                       : wtype == MTG_TYPE_F16 ? kStepF16MaxKeys
                       : wtype == MTG_TYPE_F32 ? kStepF32MaxKeys
                                               : std::numeric_limits<int>::max();
  const bool on_step = exec == kExecStep && step_ok && step_mode && (wtype == MTG_TYPE_Q8_0 || G == 1) &&
                       (int64_t)past + T <= max_keys;
  const bool timed = timing && mode != kModeLogits;
  if (timed && (rc = check(hipEventRecord(ev_start, stream), "timing event"))) return rc;
  bool aborting = false;
  if (on_step) {
    // the step kernel takes the descriptor as a kernel argument
    if (epoch > 0xF0000000u) {  // progress words restart before they could wrap
      if ((rc = check(hipMemsetAsync(params_host.flags, 0, (size_t)nwg * kFlagStride * 4, stream), "flags"))) return rc;
      // the tags of the exchanged q|k|v values come from the same counter
      if ((rc = check(hipMemsetAsync(params_host.qkvt, 0, qkvt_bytes(), stream), "tags"))) return rc;
      epoch = 0;
    }
    const int smode = mode == kModeAppend ? kStepAppend : kStepVerify;
    result_host->n_match = -1;  // the kernel's acceptance overwrites it
    result_host->err = 0;
    if (abort_next) {
      abort_next = false;
      aborting = true;
      if ((rc = check(hipMemsetAsync(&result_dev->err, 1, sizeof(int32_t), stream), "abort")))
        return rc;
    }
    if ((rc = check(launch_step(stream, G, kv_type == MTG_TYPE_F16, step_wf(), params_dev, desc_host, epoch, smode,
                                    params_host.timing != nullptr), "step kernel launch")))
      return rc;
    epoch += step_progress_per_step(hp.n_layers);
  } else {
    if ((rc = enqueue_per_op(G, mode))) return rc;
  }
  if (timed && (rc = check(hipEventRecord(ev_stop, stream), "timing event"))) return rc;
  // the step kernel's verify writes its choices into the mapped host buffer; the
  // other paths (per-op kernels, appends) bring the result over with a copy
  const bool mapped = on_step && (mode == kModeVerify || mode == kModeVerifyPenalty);
  if (!mapped && (rc = check(hipMemcpyAsync(result_host, result_dev, sizeof(StepResult),
                                             hipMemcpyDeviceToHost, stream), "result")))
    return rc;
  if ((rc = check(hipStreamSynchronize(stream), "step"))) return rc;
  if (mapped && result_host->n_match < 0) {
    // the kernel left before its acceptance: a bounded wait ran out
    (void)hipMemcpy(&result_host->err, &result_dev->err, sizeof(int32_t), hipMemcpyDeviceToHost);
    if (!result_host->err) return fail(MTG_ERR_DEVICE, "step kernel: no result");
  }
  if (on_step && !result_host->err) ++step_runs;
  if (result_host->err) {
    // a bounded wait ran out and every workgroup left the kernel; only positions
    // from `past` on were written, so the step can run again
    (void)hipMemset(&result_dev->err, 0, sizeof(int32_t));
    result_host->err = 0;
    if (aborting || !on_step)
      return fail(MTG_ERR_DEVICE, "step kernel: a bounded wait ran out (step abandoned)");
    // the same step on the per-op kernels (its workgroups need no co-residency)
    ++step_fallbacks;
    // a timed step counts the abandoned launch and its rerun: the event pair is
    // read now and then brackets the per-op kernels
    float ms_abandoned = 0.0f;
    if (timed && ((rc = check(hipEventElapsedTime(&ms_abandoned, ev_start, ev_stop), "timing")) ||
                  (rc = check(hipEventRecord(ev_start, stream), "timing event"))))
      return rc;
    if ((rc = enqueue_per_op(G, mode))) return rc;
    if (timed && (rc = check(hipEventRecord(ev_stop, stream), "timing event"))) return rc;
    if ((rc = check(hipMemcpyAsync(result_host, result_dev, sizeof(StepResult), hipMemcpyDeviceToHost,
                                   stream), "result")))
      return rc;
    if ((rc = check(hipStreamSynchronize(stream), "fallback step"))) return rc;
    if (timed) {
      float ms_rerun = 0.0f;
      if ((rc = check(hipEventElapsedTime(&ms_rerun, ev_start, ev_stop), "timing"))) return rc;
      timing_ms += (double)ms_abandoned + ms_rerun;
      ++timing_launches;
      timing_past += desc_host->past;
      timing_rows += T;
    }
  } else if (timed) {
    float ms = 0.0f;
    if ((rc = check(hipEventElapsedTime(&ms, ev_start, ev_stop), "timing"))) return rc;
    timing_ms += ms;
    ++timing_launches;
    timing_past += desc_host->past;
    timing_rows += T;
  }
  if (want_hidden && hidden_out &&
      (rc = check(hipMemcpy(hidden_out, hid, (size_t)T * hp.hidden * 4, hipMemcpyDeviceToHost), "hidden")))
    return rc;
  if (want_logits && logits_out &&
      (rc = check(hipMemcpy(logits_out, logits, (size_t)T * hp.vocab * 4, hipMemcpyDeviceToHost), "logits")))
    return rc;
  return MTG_OK;
}

// The per-op kernels of one step: the descriptor goes to device memory, then
// the captured graph (or the eager sequence) runs on the stream.
int Ctx::enqueue_per_op(int G, int mode) {
  int rc = check(hipMemcpyAsync(desc_dev, desc_host, sizeof(StepDesc), hipMemcpyHostToDevice, stream),
                 "step descriptor");
  if (rc) return rc;
  // Under counter collection the graph path is not taken: replaying the per-op
  // graph of a prefill append under `rocprofv3 --pmc` once ended in a SIGSEGV inside
  // hipGraphLaunch (below it, the profiler's dispatch interception). Eager launches
  // run the same kernels in the same order, so the counters describe the same work.
  if (exec == kExecEager || counter_collection) {
    enqueue(G, mode);
    return check(hipGetLastError(), "kernel launch");
  }
  GraphSlot& slot = graphs[(G - 1) * kModes + mode];
  if (!slot.exec) {
    hipGraph_t g = nullptr;
    if ((rc = check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "capture"))) return rc;
    enqueue(G, mode);
    if ((rc = check(hipStreamEndCapture(stream, &g), "end capture"))) return rc;
    rc = check(hipGraphInstantiate(&slot.exec, g, nullptr, nullptr, 0), "instantiate");
    hipGraphDestroy(g);
    if (rc) return rc;
  }
  return check(hipGraphLaunch(slot.exec, stream), "graph launch");
}

void Ctx::fill_desc(int T, bool use_embeds, float penalty, const int32_t* tokens,
                    const int32_t* history, int n_history, bool write_logits) {
  StepDesc& d = *desc_host;
  d.T = T;
  d.past = past;
  d.groups = (T + 7) / 8;
  d.use_embeds = use_embeds ? 1 : 0;
  d.penalty = penalty;
  d.write_logits = write_logits ? 1 : 0;
  for (int i = 0; i < kMaxRows; ++i) d.tokens[i] = (tokens && i < T) ? tokens[i] : 0;
  d.n_pen = 0;
  d.pen_base = 0;
  if (penalty > 1.0f) {
    // window of row i = last 100 of history ++ tokens[0..i]
    const int nh = history ? n_history : 0;
    const int start = std::max(0, nh + 1 - kPenaltyWindow);
    int n = 0;
    for (int i = start; i < nh; ++i) d.pen_ids[n++] = history[i];
    for (int i = 0; i < T; ++i) d.pen_ids[n++] = tokens[i];
    d.n_pen = n;
    d.pen_base = nh - start;
  }
}

int Ctx::verify(const int32_t* tokens, int T, const int32_t* history, int n_history,
                float penalty, int32_t* choice_out, int32_t* n_match_out, float* hidden_out,
                float* logits_out) {
  if (!tokens || T <= 0 || T > kMaxRows || !choice_out || !n_match_out)
    return fail(MTG_ERR_INVALID, "verify: bad arguments (T=%d)", T);
  if (past + T > max_seq) return fail(MTG_ERR_CAPACITY, "sequence exceeds max_seq");
  for (int i = 0; i < T; ++i)
    if (tokens[i] < 0 || tokens[i] >= hp.vocab) return fail(MTG_ERR_INVALID, "token id %d", tokens[i]);
  fill_desc(T, false, penalty, tokens, history, n_history, logits_out != nullptr);
  const int mode = penalty > 1.0f ? kModeVerifyPenalty : kModeVerify;
  int rc = run(mode, T, true, true, hidden_out, logits_out);
  if (rc) return rc;
  past += T;
  for (int i = 0; i < T; ++i) choice_out[i] = result_host->choice[i];
  *n_match_out = result_host->n_match;
  return MTG_OK;
}

int Ctx::append(const float* embeds, int T, float* hidden_out) {
  if (!embeds || T <= 0 || T > kMaxRows) return fail(MTG_ERR_INVALID, "append: bad arguments");
  if (past + T > max_seq) return fail(MTG_ERR_CAPACITY, "sequence exceeds max_seq");
  int rc = check(hipMemcpyAsync(embeds_dev, embeds, (size_t)T * hp.hidden * 4, hipMemcpyHostToDevice,
                                stream), "embeddings");
  if (rc) return rc;
  fill_desc(T, true, 1.0f, nullptr, nullptr, 0, false);
  if ((rc = run(kModeAppend, T, true, false, hidden_out, nullptr))) return rc;
  past += T;
  return MTG_OK;
}

// Qwen3Decoder::prefill (src/qwen3_decoder.cpp:162-166): the fused prompt rows
// run from position 0; hidden_out (nullable) gets every row's final-normed
// hidden state.
int Ctx::prefill(const float* embeds, int S, float* hidden_out) {
  if (!embeds || S <= 0) return fail(MTG_ERR_INVALID, "prefill: bad arguments");
  if (S > max_seq) return fail(MTG_ERR_CAPACITY, "prefill exceeds max_seq");
  past = 0;
  const bool blocks = prefill_fast_enabled && S <= pf_max_context() && hp.hidden == 1024 &&
                      hp.head_dim == kHeadDim;
  if (blocks) return wtype == MTG_TYPE_Q8_0 ? prefill_blocks(embeds, S, hidden_out)
                                            : prefill_blocks_wt(embeds, S, hidden_out);
  const int H = hp.hidden;
  for (int s0 = 0; s0 < S; s0 += kMaxRows) {
    const int n = std::min(kMaxRows, S - s0);
    const int rc = append(embeds + (size_t)s0 * H, n, hidden_out ? hidden_out + (size_t)s0 * H : nullptr);
    if (rc) return rc;
  }
  return MTG_OK;
}

// The prompt in blocks of kPfRows rows: per layer RMSNorm + q8_0 conversion, the
// fused q|k|v GEMM, q/k norm + RoPE + KV append, causal attention over the cache,
// o-proj + residual, RMSNorm, gate/up + SwiGLU, q8_0, down + residual; each
// weight matrix is streamed once per block. Same arithmetic as the verify path.
int Ctx::prefill_blocks(const float* embeds, int S, float* hidden_out) {
  const int H = hp.hidden, NH = hp.n_heads, NKV = hp.n_kv_heads, D = hp.head_dim;
  const int QN = NH * D, KN = NKV * D, NQKV = QN + 2 * KN, F = hp.intermediate;
  const float eps = hp.rms_eps;
  const int R = kPfRows;
  if (!pf.x) {
    pf.x = (float*)dalloc((size_t)R * H * 4, false);
    pf.qkv = (float*)dalloc((size_t)R * NQKV * 4, false);
    pf.q = (float*)dalloc((size_t)R * QN * 4, false);
    pf.act = (float*)dalloc((size_t)R * F * 4, false);
    pf.hid = (float*)dalloc((size_t)R * H * 4, false);
    const int KM = std::max(H, std::max(QN, F));
    pf.codes = (int8_t*)dalloc((size_t)R * KM, false);
    pf.scales = (float*)dalloc((size_t)R * (KM / 32) * 4, false);
    if (!pf.x || !pf.qkv || !pf.q || !pf.act || !pf.hid || !pf.codes || !pf.scales)
      return fail(MTG_ERR_NOMEM, "prefill buffers");
  }
  hipStream_t s = stream;
  int rc = MTG_OK;
  if (!ev_start && (rc = check(hipEventCreate(&ev_start), "event"))) return rc;
  if (!ev_stop && (rc = check(hipEventCreate(&ev_stop), "event"))) return rc;
  if ((rc = check(hipEventRecord(ev_start, s), "event"))) return rc;
  for (int c0 = 0; c0 < S; c0 += R) {
    const int n = std::min(R, S - c0);
    if ((rc = check(hipMemcpyAsync(pf.x, embeds + (size_t)c0 * H, (size_t)n * H * 4, hipMemcpyHostToDevice, s),
                    "prompt rows")))
      return rc;
    for (int l = 0; l < hp.n_layers; ++l) {
      const Layer& y = layers[l];
      const KvLayer kv = kv_layer(l);
      launch_pf_norm_quant(s, pf.x, n, y.attn_norm, eps, pf.codes, pf.scales, nullptr);
      launch_pf_gemm(s, PF_EPI_STORE, y.wqkv, nullptr, NQKV, H, pf.codes, pf.scales, n, pf.qkv);
      launch_pf_qk_rope(s, pf.qkv, n, c0, NH, NKV, y.q_norm, y.k_norm, eps, rope, pf.q, kv);
      launch_pf_attn(s, pf.q, NH, NKV, kv, c0, n, pf.codes, pf.scales);
      launch_pf_gemm(s, PF_EPI_RESID, y.wo, nullptr, H, QN, pf.codes, pf.scales, n, pf.x);
      launch_pf_norm_quant(s, pf.x, n, y.ffn_norm, eps, pf.codes, pf.scales, nullptr);
      launch_pf_gemm(s, PF_EPI_SWIGLU, y.wg, y.wu, F, H, pf.codes, pf.scales, n, pf.act);
      launch_pf_quant(s, pf.act, n, F, pf.codes, pf.scales);
      launch_pf_gemm(s, PF_EPI_RESID, y.wd, nullptr, H, F, pf.codes, pf.scales, n, pf.x);
    }
    launch_pf_norm_quant(s, pf.x, n, out_norm, eps, pf.codes, pf.scales, pf.hid);
    if ((rc = check(hipGetLastError(), "prefill launch"))) return rc;
    if (hidden_out &&
        (rc = check(hipMemcpyAsync(hidden_out + (size_t)c0 * H, pf.hid, (size_t)n * H * 4, hipMemcpyDeviceToHost, s),
                    "hidden rows")))
      return rc;
  }
  if ((rc = check(hipEventRecord(ev_stop, s), "event"))) return rc;
  if ((rc = check(hipStreamSynchronize(s), "prefill"))) return rc;
  float ms = 0.0f;
  if ((rc = check(hipEventElapsedTime(&ms, ev_start, ev_stop), "event"))) return rc;
  last_prefill_ms = ms;
  past = S;
  return MTG_OK;
}

// The block prefill for f16 and q4_K weights (prefill_wt.hip): the same layer
// sequence as prefill_blocks, with each GEMM's activation in the weight type's
// vec_dot_type (f16 rows or q8_K blocks) and the attention output as f32 rows.
int Ctx::prefill_blocks_wt(const float* embeds, int S, float* hidden_out) {
  const int H = hp.hidden, NH = hp.n_heads, NKV = hp.n_kv_heads, D = hp.head_dim;
  const int QN = NH * D, KN = NKV * D, NQKV = QN + 2 * KN, F = hp.intermediate;
  const float eps = hp.rms_eps;
  const int R = kPfRows;
  const int KM = std::max(H, std::max(QN, F));
  if (!pf.x) {
    pf.x = (float*)dalloc((size_t)R * H * 4, false);
    pf.qkv = (float*)dalloc((size_t)R * NQKV * 4, false);
    pf.q = (float*)dalloc((size_t)R * QN * 4, false);
    pf.act = (float*)dalloc((size_t)R * F * 4, false);
    pf.hid = (float*)dalloc((size_t)R * H * 4, false);
    pf.codes = (int8_t*)dalloc((size_t)R * KM, false);
    pf.scales = (float*)dalloc((size_t)R * (KM / 32) * 4, false);
    if (!pf.x || !pf.qkv || !pf.q || !pf.act || !pf.hid || !pf.codes || !pf.scales)
      return fail(MTG_ERR_NOMEM, "prefill buffers");
  }
  if (!pf.o) {
    pf.o = (float*)dalloc((size_t)R * QN * 4, false);
    bool ok = true;
    if (wtype == MTG_TYPE_F16) {
      ok = (pf.wact.f16h = (uint16_t*)dalloc((size_t)R * KM * 2, false)) != nullptr;
    } else if (wtype == MTG_TYPE_F32) {
      ok = (pf.wact.f32 = (float*)dalloc((size_t)R * KM * 4, false)) != nullptr;
    } else {
      pf.wact.q8k.qs = (int8_t*)dalloc((size_t)R * KM, false);
      pf.wact.q8k.d = (float*)dalloc((size_t)R * (KM / 256) * 4, false);
      pf.wact.q8k.bsums = (int32_t*)dalloc((size_t)R * (KM / 16) * 4, false);
      ok = pf.wact.q8k.qs && pf.wact.q8k.d && pf.wact.q8k.bsums;
    }
    if (!pf.o || !ok) return fail(MTG_ERR_NOMEM, "prefill buffers");
  }
  hipStream_t s = stream;
  int rc = MTG_OK;
  if (!ev_start && (rc = check(hipEventCreate(&ev_start), "event"))) return rc;
  if (!ev_stop && (rc = check(hipEventCreate(&ev_stop), "event"))) return rc;
  if ((rc = check(hipEventRecord(ev_start, s), "event"))) return rc;
  const WtAct& A = pf.wact;
  for (int c0 = 0; c0 < S; c0 += R) {
    const int n = std::min(R, S - c0);
    if ((rc = check(hipMemcpyAsync(pf.x, embeds + (size_t)c0 * H, (size_t)n * H * 4, hipMemcpyHostToDevice, s),
                    "prompt rows")))
      return rc;
    for (int l = 0; l < hp.n_layers; ++l) {
      const Layer& y = layers[l];
      const KvLayer kv = kv_layer(l);
      launch_pf_act_wt(s, wtype, pf.x, n, H, y.attn_norm, eps, A);
      launch_pf_gemm_wt(s, wtype, PF_EPI_STORE, y.wqkv, nullptr, NQKV, H, A, n, pf.qkv);
      launch_pf_qk_rope(s, pf.qkv, n, c0, NH, NKV, y.q_norm, y.k_norm, eps, rope, pf.q, kv);
      launch_pf_attn(s, pf.q, NH, NKV, kv, c0, n, nullptr, nullptr, pf.o);
      launch_pf_act_wt(s, wtype, pf.o, n, QN, nullptr, eps, A);
      launch_pf_gemm_wt(s, wtype, PF_EPI_RESID, y.wo, nullptr, H, QN, A, n, pf.x);
      launch_pf_act_wt(s, wtype, pf.x, n, H, y.ffn_norm, eps, A);
      launch_pf_gemm_wt(s, wtype, PF_EPI_SWIGLU, y.wg, y.wu, F, H, A, n, pf.act);
      launch_pf_act_wt(s, wtype, pf.act, n, F, nullptr, eps, A);
      launch_pf_gemm_wt(s, wtype, PF_EPI_RESID, y.wd, nullptr, H, F, A, n, pf.x);
    }
    launch_pf_norm_quant(s, pf.x, n, out_norm, eps, pf.codes, pf.scales, pf.hid);
    if ((rc = check(hipGetLastError(), "prefill launch"))) return rc;
    if (hidden_out &&
        (rc = check(hipMemcpyAsync(hidden_out + (size_t)c0 * H, pf.hid, (size_t)n * H * 4, hipMemcpyDeviceToHost, s),
                    "hidden rows")))
      return rc;
  }
  if ((rc = check(hipEventRecord(ev_stop, s), "event"))) return rc;
  if ((rc = check(hipStreamSynchronize(s), "prefill"))) return rc;
  float ms = 0.0f;
  if ((rc = check(hipEventElapsedTime(&ms, ev_start, ev_stop), "event"))) return rc;
  last_prefill_ms = ms;
  past = S;
  return MTG_OK;
}

int Ctx::logits_of(const float* hidden, int T, float* logits_out) {
  if (!hidden || T <= 0 || !logits_out) return fail(MTG_ERR_INVALID, "logits: bad arguments");
  for (int t0 = 0; t0 < T; t0 += kMaxRows) {
    const int n = std::min(kMaxRows, T - t0);
    int rc = check(hipMemcpyAsync(embeds_dev, hidden + (size_t)t0 * hp.hidden,
                                  (size_t)n * hp.hidden * 4, hipMemcpyHostToDevice, stream),
                   "hidden rows");
    if (rc) return rc;
    fill_desc(n, true, 1.0f, nullptr, nullptr, 0, true);
    if ((rc = run(kModeLogits, n, false, true, nullptr, logits_out + (size_t)t0 * hp.vocab)))
      return rc;
  }
  return MTG_OK;
}

int Ctx::embed(const int32_t* ids, int n, float* out) {
  if (!ids || n <= 0 || !out) return fail(MTG_ERR_INVALID, "embed: bad arguments");
  for (int i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= hp.vocab) return fail(MTG_ERR_INVALID, "token id %d", ids[i]);
  for (int i0 = 0; i0 < n; i0 += kMaxRows) {
    const int c = std::min(kMaxRows, n - i0);
    fill_desc(c, false, 1.0f, ids + i0, nullptr, 0, false);
    int rc = check(hipMemcpyAsync(desc_dev, desc_host, sizeof(StepDesc), hipMemcpyHostToDevice,
                                  stream), "descriptor");
    if (rc) return rc;
    if (wtype == MTG_TYPE_Q8_0) launch_embed(stream, desc_dev, embd, hp.hidden, embeds_dev, x);
    else launch_embed_wt(stream, wtype, desc_dev, embd, hp.hidden, embeds_dev, x);
    if ((rc = check(hipMemcpyAsync(out + (size_t)i0 * hp.hidden, x, (size_t)c * hp.hidden * 4,
                                   hipMemcpyDeviceToHost, stream), "embed rows")))
      return rc;
    if ((rc = check(hipStreamSynchronize(stream), "embed"))) return rc;
  }
  return MTG_OK;
}

int Ctx::kv_io(void* k, void* v, int n_pos, bool write) {
  if (!k || !v || n_pos < 0 || n_pos > max_seq) return fail(MTG_ERR_INVALID, "kv: bad arguments");
  const size_t es = kv_type == MTG_TYPE_F32 ? 4 : 2;
  const size_t row = (size_t)hp.head_dim * es, chunk = row * n_pos;
  for (int l = 0; l < hp.n_layers; ++l)
    for (int h = 0; h < hp.n_kv_heads; ++h) {
      const size_t dev_off = kv_layer_bytes * l + (size_t)h * max_seq * row;
      const size_t host_off = ((size_t)l * hp.n_kv_heads + h) * chunk;
      for (int which = 0; which < 2; ++which) {
        uint8_t* dev = (which ? vcache : kcache) + dev_off;
        uint8_t* host = (uint8_t*)(which ? v : k) + host_off;
        const hipError_t e = write ? hipMemcpy(dev, host, chunk, hipMemcpyHostToDevice)
                                   : hipMemcpy(host, dev, chunk, hipMemcpyDeviceToHost);
        if (int rc = check(e, "kv copy")) return rc;
      }
    }
  if (write) past = n_pos;
  return MTG_OK;
}

}  // namespace mtg

namespace mtg {

// The controller on the device: one k_gen_ctrl pass, then step launches in
// chunks of kChunkSteps (each runs the controller pass on its own outcome), the
// state looked at once per chunk. A step that leaves before its acceptance ends
// the run with g.err set and that step undone.
int Ctx::generate_device(GenState& g, int32_t* ids, int cap, const int32_t* prompt_ids,
                         const int32_t* stream_ids) {
  constexpr int kChunkSteps = 8;
  int rc = MTG_OK;
  if (!step_ok || exec != kExecStep || g.max_draft + 1 > kMaxRows)
    return fail(MTG_ERR_UNSUPPORTED, "device generation needs the step kernel and max_draft <= %d", kMaxRows - 1);
  if ((wtype == MTG_TYPE_F16 || wtype == MTG_TYPE_F32) && g.max_draft + 1 > 8)
    return fail(MTG_ERR_UNSUPPORTED, "device generation with f16 or f32 weights needs max_draft <= 7 (8-row steps)");
  // the 16-row step variant when a step can hold more than 8 rows
  const int G = g.max_draft + 1 > 8 ? 2 : 1;
  // the stream drafter's prompt ids and stream period, in one device buffer
  const size_t aux = (size_t)g.n_prompt + (size_t)g.period;
  if (aux > (size_t)gen_aux_cap) {
    if (gen_aux_dev) (void)hipFree(gen_aux_dev);
    gen_aux_dev = nullptr;
    gen_aux_cap = 0;
    if ((rc = check(hipMalloc((void**)&gen_aux_dev, aux * 4), "drafter ids"))) return rc;
    gen_aux_cap = (int)aux;
  }
  if (g.n_prompt > 0 &&
      (rc = check(hipMemcpyAsync(gen_aux_dev, prompt_ids, (size_t)g.n_prompt * 4, hipMemcpyHostToDevice, stream),
                  "drafter prompt")))
    return rc;
  if (g.period > 0 && (rc = check(hipMemcpyAsync(gen_aux_dev + g.n_prompt, stream_ids, (size_t)g.period * 4,
                                                 hipMemcpyHostToDevice, stream),
                                  "drafter stream")))
    return rc;
  const int32_t* prompt_dev = g.n_prompt > 0 ? gen_aux_dev : nullptr;
  const int32_t* stream_dev = g.period > 0 ? gen_aux_dev + g.n_prompt : nullptr;
  if (cap > gen_cap) {
    if (gen_ids_dev) (void)hipFree(gen_ids_dev);
    gen_ids_dev = nullptr;
    gen_cap = 0;
    if ((rc = check(hipMalloc((void**)&gen_ids_dev, (size_t)cap * 4), "generation ids"))) return rc;
    gen_cap = cap;
  }
  if (!gen_state_dev && (rc = check(hipMalloc((void**)&gen_state_dev, sizeof(GenState)), "generation state")))
    return rc;
  if (!gen_state_host &&
      (rc = check(hipHostMalloc((void**)&gen_state_host, 2 * sizeof(GenState), hipHostMallocDefault),
                  "generation state")))
    return rc;
  *gen_state_host = g;
  if ((rc = check(hipMemcpyAsync(gen_state_dev, gen_state_host, sizeof(GenState), hipMemcpyHostToDevice, stream),
                  "generation state")))
    return rc;
  if (g.n_ids > 0 && (rc = check(hipMemcpyAsync(gen_ids_dev, ids, (size_t)g.n_ids * 4, hipMemcpyHostToDevice, stream),
                                 "generation ids")))
    return rc;
  const uint32_t pps = step_progress_per_step(hp.n_layers);
  const int kv_f16 = kv_type == MTG_TYPE_F16;
  StepDesc unused{};
  result_host->err = 0;
  // launch timing: an event pair around every step launch of a chunk; once the
  // chunk's state is back, the launches that ran a step (the first ones) count
  if (!gen_chunk_ev[0]) {
    for (auto& e : gen_chunk_ev)
      if ((rc = check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "event"))) return rc;
  }
  if (timing && !gen_events[0][0]) {
    for (auto& slot : gen_events)
      for (auto& e : slot)
        if ((rc = check(hipEventCreate(&e), "event"))) return rc;
  }
  int64_t rows0 = g.issued_rows, past0 = g.issued_past;
  const int64_t steps_begin = g.steps;
  int64_t steps0 = g.steps, err0 = g.err;
  const GenCtl ctl{gen_state_dev, gen_ids_dev, desc_dev, prompt_dev, stream_dev};
  // the first controller pass issues the first step; every step launch then runs
  // the pass on its own outcome (commit, stop rules, the next step's draft)
  launch_gen_ctrl(stream, ctl, result_map, &result_dev->err);
  if ((rc = check(hipGetLastError(), "controller launch"))) return rc;
  int64_t launched = 0;
  int chunk_steps[2] = {0, 0};
  // one chunk of step launches (with a step limit, no more than steps are left)
  // and the copy of the state behind it, into slot `slot`
  auto issue = [&](int slot) -> int {
    if (epoch > 0xF0000000u - (uint32_t)kChunkSteps * pps) {  // progress words restart before they could wrap
      if ((rc = check(hipMemsetAsync(params_host.flags, 0, (size_t)nwg * kFlagStride * 4, stream), "flags"))) return rc;
      if ((rc = check(hipMemsetAsync(params_host.qkvt, 0, qkvt_bytes(), stream), "tags"))) return rc;
      epoch = 0;
    }
    int steps = kChunkSteps;
    if (g.max_steps > 0) steps = (int)std::min<int64_t>(kChunkSteps, std::max<int64_t>(0, g.max_steps - launched));
    for (int i = 0; i < steps; ++i) {
      if (timing && (rc = check(hipEventRecord(gen_events[slot][2 * i], stream), "timing event"))) return rc;
      if ((rc = check(launch_step(stream, G, kv_f16, step_wf(), params_dev, &unused, epoch, kStepVerify,
                                  false, desc_dev, &ctl),
                      "step kernel launch")))
        return rc;
      if (timing && (rc = check(hipEventRecord(gen_events[slot][2 * i + 1], stream), "timing event"))) return rc;
      epoch += pps;
    }
    launched += steps;
    chunk_steps[slot] = steps;
    if ((rc = check(hipMemcpyAsync(gen_state_host + slot, gen_state_dev, sizeof(GenState), hipMemcpyDeviceToHost,
                                   stream),
                    "generation state")))
      return rc;
    return check(hipEventRecord(gen_chunk_ev[slot], stream), "chunk event");
  };
  auto limit_reached = [&]() { return g.max_steps > 0 && launched >= g.max_steps; };
  // Two chunks in flight: the next chunk is enqueued before the host waits for
  // the current one's state, so the device does not idle at a chunk boundary.
  // Launches after the loop has stopped return at once.
  if ((rc = issue(0))) return rc;
  int cur = 0;
  for (;;) {
    const bool next = !limit_reached();
    if (next && (rc = issue(cur ^ 1))) return rc;
    if ((rc = check(hipEventSynchronize(gen_chunk_ev[cur]), "generation"))) return rc;
    const GenState& st = gen_state_host[cur];
    // the launches of the chunk that ran a step come first: each committed one
    // step, or left with the error that ended the loop
    const int64_t ran = std::min<int64_t>(chunk_steps[cur], (st.steps - steps0) + (st.err - err0));
    if (timing) {
      for (int i = 0; i < (int)ran; ++i) {
        float ms = 0.0f;
        if ((rc = check(hipEventElapsedTime(&ms, gen_events[cur][2 * i], gen_events[cur][2 * i + 1]), "timing")))
          return rc;
        timing_ms += ms;
      }
      timing_launches += ran;
      timing_rows += st.issued_rows - rows0;
      timing_past += st.issued_past - past0;
    }
    steps0 = st.steps;
    err0 = st.err;
    rows0 = st.issued_rows;
    past0 = st.issued_past;
    if (st.done || !next) break;  // without a next chunk the last step's pass has stopped the loop
    cur ^= 1;
  }
  // the chunk still in flight runs launches that return at once; the state is final
  if ((rc = check(hipStreamSynchronize(stream), "generation"))) return rc;
  if ((rc = check(hipMemcpy(gen_state_host, gen_state_dev, sizeof(GenState), hipMemcpyDeviceToHost),
                  "generation state")))
    return rc;
  g = *gen_state_host;
  if ((rc = check(hipMemcpy(ids, gen_ids_dev, (size_t)g.n_ids * 4, hipMemcpyDeviceToHost), "generation ids")))
    return rc;
  if (g.err) {
    // the abandoned step wrote only positions from its `before` on
    (void)hipMemset(&result_dev->err, 0, sizeof(int32_t));
    ++step_fallbacks;
  }
  step_runs += g.steps - steps_begin;
  past = g.past;
  return MTG_OK;
}

}  // namespace mtg
