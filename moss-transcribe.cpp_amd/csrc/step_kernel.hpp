// step_kernel.hpp - the persistent verify-step kernel (step_kernel.hip).
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#include "mtg_internal.hpp"

namespace mtg {

enum { kStepVerify = 0, kStepAppend = 1 };

// One decoder layer's device tensors.
struct LayerDev {
  const uint8_t *wqkv, *wo, *wg, *wu, *wd;  // MFMA panel tiles
  const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
  uint8_t *kc, *vc;                          // KV cache of the layer
};

// Constant for a context; lives in device memory.
struct StepParams {
  int H, NH, NKV, F, V, L, max_seq, kv_f16, bps_max, max_chunks;
  float eps;
  const LayerDev* layers;
  const uint8_t* embd;
  const float* out_norm;
  const float* rope;
  const float* embeds;  // host rows uploaded for append
  float *x, *qkv, *o, *act, *hid, *logits;
  float *part_ml, *part_o;  // [kv head][chunk][col][2] and [kv head][chunk][col][head_dim]
  uint32_t* bitmap;
  uint64_t* part_keys;      // [nwg][16]
  StepResult* result;
  uint32_t* flags;          // [nwg] barrier arrival words
  uint32_t* release;        // barrier release word (written by workgroup 0)
  int32_t* err;             // raised by a wait that ran out (inside *result)
  uint64_t* timing;         // nullable: workgroup 0 records the clock after every barrier
};

int step_barriers(int n_layers, int mode);
size_t step_lds_bytes(int G, int bps_max);
hipError_t prepare_step_kernels(int bps_max);
hipError_t launch_step(hipStream_t s, int G, int nwg, const StepParams* P, const StepDesc* desc,
                       uint32_t epoch, int mode, int bps_max);

}  // namespace mtg
