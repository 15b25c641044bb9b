// runtime.hpp - the device decoder context behind the C ABI.
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "mtg_internal.hpp"
#include "step_kernel.hpp"

namespace mtg {

enum { kModeVerify = 0, kModeVerifyPenalty = 1, kModeAppend = 2, kModeLogits = 3, kModes = 4 };
// How a step is executed: one persistent kernel, or the per-op kernels replayed
// from a captured graph, or the per-op kernels launched one by one.
enum { kExecStep = 0, kExecGraph = 1, kExecEager = 2 };

struct Layer {
  uint8_t *wqkv = nullptr, *wo = nullptr, *wg = nullptr, *wu = nullptr, *wd = nullptr;
  float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
};

struct GraphSlot {
  hipGraphExec_t exec = nullptr;
};

struct Ctx {
  mtg_hparams hp{};
  int max_seq = 0, kv_type = MTG_TYPE_F32, past = 0;
  int wtype = MTG_TYPE_Q8_0;  // q8_0: MFMA panel tiles; f16 / q4_K: GGUF rows (kernels_wt.hip)
  int exec = kExecStep;
  // rocprofv3 collects hardware counters in this process (ROCPROF_COUNTER_COLLECTION):
  // the per-op kernels then launch one by one instead of from a graph
  bool counter_collection = false;
  // persistent step kernel
  int nwg = 0;
  bool step_ok = false;  // the persistent step kernel is usable for this model / device
  uint32_t epoch = 0;
  bool abort_next = false;  // raise the error word before the next step-kernel launch
  int64_t step_fallbacks = 0;  // steps rerun on the per-op kernels after a wait ran out
  int64_t step_runs = 0;       // steps that ran to their end on the persistent kernel
  int step_max_keys = 0;       // KV length limit of the persistent kernel (0: the weight type's default)
  // the step kernel's weight variant: 0 q8_0 tiles, 1 f16 rows, 2 f32 rows
  int step_wf() const { return wtype == MTG_TYPE_F16 ? 1 : wtype == MTG_TYPE_F32 ? 2 : 0; }
  StepParams* params_dev = nullptr;
  StepParams params_host{};
  uint64_t* timing_dev = nullptr;  // step-kernel phase clock marks (profiling)
  // launch timing: HIP events around every step's device work on `stream`
  bool timing = false;
  hipEvent_t ev_start = nullptr, ev_stop = nullptr;
  double timing_ms = 0.0;
  int64_t timing_launches = 0, timing_past = 0, timing_rows = 0;
  std::string error;
  hipStream_t stream = nullptr;
  std::vector<void*> allocations;
  std::vector<Layer> layers;
  uint8_t* embd = nullptr;
  uint8_t* lm_copy = nullptr;  // f16 / f32 weights: the lm_head's re-tiled copy of embd
  float* out_norm = nullptr;
  float* rope = nullptr;
  uint8_t *kcache = nullptr, *vcache = nullptr;
  size_t kv_layer_bytes = 0;
  float *x = nullptr, *qkv = nullptr, *qbuf = nullptr, *obuf = nullptr, *act = nullptr,
        *hid = nullptr, *embeds_dev = nullptr, *logits = nullptr;
  uint32_t* bitmap = nullptr;
  uint64_t* part_keys = nullptr;
  Panel panel_h{}, panel_o{}, panel_f{};
  WtAct wact{};  // f16 / q4_K weights: the activation of the next GEMM
  AttnWork work{};
  StepDesc* desc_dev = nullptr;
  StepResult* result_dev = nullptr;
  StepDesc* desc_host = nullptr;      // pinned
  StepResult* result_host = nullptr;  // pinned
  StepResult* result_map = nullptr;   // result_host as the device sees it (the step kernel writes it)
  GraphSlot graphs[2 * kModes];
  // prompt prefill over blocks of up to kPfRows rows (prefill.hip), allocated at
  // the first prefill
  static constexpr int kPfRows = 2048;
  struct PfBuffers {
    float *x = nullptr, *qkv = nullptr, *q = nullptr, *act = nullptr, *hid = nullptr;
    int8_t* codes = nullptr;
    float* scales = nullptr;
    // f16 / q4_K weights: the attention output rows and the GEMM activation
    float* o = nullptr;
    WtAct wact{};
  } pf;
  bool prefill_fast_enabled = true;
  double last_prefill_ms = 0.0;  // device time of the last prefill (HIP events)

  ~Ctx();
  int fail(int code, const char* fmt, ...);
  int check(hipError_t e, const char* what);
  void* dalloc(size_t bytes, bool zero);
  int upload_q8(const void* blocks, int n, int k, uint8_t* dst, uint8_t* staging);
  // bytes of an n x k weight matrix on the device, and its upload
  size_t weight_bytes(int n, int k) const;
  // the step kernel's tagged q|k|v exchange: [rows][q|k|v] (value, tag) pairs
  size_t qkvt_bytes() const {
    return (size_t)kMaxRows * (hp.n_heads + 2 * hp.n_kv_heads) * hp.head_dim * 8;
  }
  int upload_weights(const void* src, int n, int k, uint8_t* dst, uint8_t* staging);
  int init(const mtg_model_desc* d, int max_seq, int kv_type);
  KvLayer kv_layer(int l) const;
  void enqueue(int G, int mode);
  void enqueue_wt(int mode);
  void fill_desc(int T, bool use_embeds, float penalty, const int32_t* tokens,
                 const int32_t* history, int n_history, bool write_logits);
  int run(int mode, int T, bool want_hidden, bool want_logits, float* hidden_out,
          float* logits_out);
  int enqueue_per_op(int G, int mode);
  int verify(const int32_t* tokens, int T, const int32_t* history, int n_history, float penalty,
             int32_t* choice_out, int32_t* n_match_out, float* hidden_out, float* logits_out);
  int append(const float* embeds, int T, float* hidden_out);
  // reset + S prompt rows; the block path when the weights are q8_0 and the
  // context fits the prefill attention, else verify-size appends
  int prefill(const float* embeds, int S, float* hidden_out);
  int prefill_blocks(const float* embeds, int S, float* hidden_out);
  int prefill_blocks_wt(const float* embeds, int S, float* hidden_out);
  int logits_of(const float* hidden, int T, float* logits_out);
  int embed(const int32_t* ids, int n, float* out);
  int kv_io(void* k, void* v, int n_pos, bool write);
  int init_step_kernel();
  // the speculative controller on the device (generate.hip): runs from state g
  // (first_new / limits / n_ids / past / raw_choice set) over ids[0, n_ids), with
  // room for cap ids; returns with g and ids as the device left them
  GenState* gen_state_dev = nullptr;  // device copies, grown on demand
  int32_t* gen_ids_dev = nullptr;
  int gen_cap = 0;
  int32_t* gen_aux_dev = nullptr;  // the stream drafter's prompt ids, then its stream period
  int gen_aux_cap = 0;
  // the device loop keeps two chunks of step launches in flight: per chunk slot an
  // event pair per launch (launch timing), the event after its state copy, and
  // the pinned copy of the state
  hipEvent_t gen_events[2][16] = {};
  hipEvent_t gen_chunk_ev[2] = {};
  GenState* gen_state_host = nullptr;  // pinned, [2]
  int generate_device(GenState& g, int32_t* ids, int cap, const int32_t* prompt_ids, const int32_t* stream_ids);
};

}  // namespace mtg

struct mtg_ctx {
  mtg::Ctx impl;
};
