// noalloc.hip - mtg_q8_mul_mat_dev_noalloc: the q8_0 GEMM entry point without
// any allocation, for callers that cannot allocate device memory (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// mtg_q8_mul_mat_dev allocates, per call, a step descriptor and the activation
// panel (B operand codes + scales) of the GEMM. This variant keeps both in one
// file-scope device array, `scratch`, that every call on a GPU shares:
//   [0, 768)            StepDesc (only T and groups are read)
//   [768, 768 + 128K)   panel codes, kMaxGroups x (K/64) x 1024 bytes
//   then                panel scales, kMaxGroups x (K/64) x 16 floats
// sized for K <= kNoAllocMaxK. Its device address is taken once per device with
// hipGetSymbolAddress; the host uses only that address. A prep kernel writes the
// descriptor and zeroes the panel codes (the block-diagonal operand needs zeros
// off its diagonal), so each call is three kernel launches on the caller's stream
// and nothing else: no hipMalloc, hipFree, memcpy or memset.
#include <hip/hip_runtime.h>

#include <mutex>

#include "kernels.hpp"

namespace mtg {
namespace {

constexpr int kNoAllocMaxK = 4096;
constexpr size_t kDescBytes = 768;  // a multiple of 256 that holds the descriptor
constexpr size_t kCodesBytes = (size_t)kMaxGroups * (kNoAllocMaxK / kPairK) * kPanelPairBytes;
constexpr size_t kScalesBytes = (size_t)kMaxGroups * (kNoAllocMaxK / kPairK) * 16 * sizeof(float);
constexpr size_t kScratchBytes = kDescBytes + kCodesBytes + kScalesBytes;
static_assert(sizeof(StepDesc) <= kDescBytes, "descriptor slot");

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::once_flag g_once[kMaxDevices];
uint8_t* g_ptr[kMaxDevices];
hipError_t g_status[kMaxDevices];

// Descriptor fields the GEMM path reads, then zeros over the panel codes of K.
__global__ void __launch_bounds__(256) k_noalloc_prep(uint8_t* base, int T, int K) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    StepDesc* d = (StepDesc*)base;
    d->T = T;
    d->past = 0;
    d->groups = (T + 7) / 8;
    d->use_embeds = 0;
    d->penalty = 1.0f;
    d->n_pen = 0;
    d->pen_base = 0;
    d->write_logits = 0;
  }
  uint4* codes = (uint4*)(base + kDescBytes);
  const size_t n16 = (size_t)kMaxGroups * (K / kPairK) * kPanelPairBytes / 16;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    codes[i] = make_uint4(0u, 0u, 0u, 0u);
}

// The device address of `scratch` on the current device (taken once per device).
hipError_t scratch_ptr(uint8_t** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::call_once(g_once[dev], [dev] {
    void* p = nullptr;
    g_status[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_ptr[dev] = g_status[dev] == hipSuccess ? (uint8_t*)p : nullptr;
  });
  *out = g_ptr[dev];
  return g_status[dev];
}

}  // namespace
}  // namespace mtg

extern "C" int mtg_q8_mul_mat_dev_noalloc(const mtg_q8_packed* w, const float* x_dev, int32_t T,
                                          float* y_dev, void* stream) {
  using namespace mtg;
  if (!w || !x_dev || !y_dev || T <= 0 || T > MTG_MAX_BATCH) {
    set_call_error("q8_mul_mat_dev_noalloc: bad arguments");
    return MTG_ERR_INVALID;
  }
  int k = 0, n = 0;
  const uint8_t* tiles = q8_packed_view(w, &k, &n);
  if (k > kNoAllocMaxK) {
    set_call_error("q8_mul_mat_dev_noalloc: K = " + std::to_string(k) + " exceeds the static scratch "
                   "(K <= " + std::to_string(kNoAllocMaxK) + "); use mtg_q8_mul_mat_dev");
    return MTG_ERR_CAPACITY;
  }
  uint8_t* base = nullptr;
  hipError_t e = scratch_ptr(&base);
  if (e != hipSuccess || !base) {
    set_call_error(std::string("q8_mul_mat_dev_noalloc: scratch address: ") + hipGetErrorString(e));
    return MTG_ERR_DEVICE;
  }
  hipStream_t s = (hipStream_t)stream;
  const StepDesc* desc = (const StepDesc*)base;
  Panel panel;
  panel.codes = base + kDescBytes;
  panel.scales = (float*)(base + kDescBytes + kCodesBytes);
  hipLaunchKernelGGL(k_noalloc_prep, dim3(16), dim3(256), 0, s, base, (int)T, k);
  launch_norm_quant(s, desc, x_dev, k, nullptr, 0.0f, panel, nullptr);
  launch_gemm_store(s, (T + 7) / 8, desc, tiles, n, k, panel, y_dev);
  e = hipGetLastError();
  if (e != hipSuccess) {
    set_call_error(std::string("q8_mul_mat_dev_noalloc: launch: ") + hipGetErrorString(e));
    return MTG_ERR_DEVICE;
  }
  return MTG_OK;
}
