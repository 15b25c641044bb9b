// Whole generation on the device: the speculative controller of
// cpu_speculative_generate (reference src/cpu_speculative.cpp:68-147) as passes of
// gen_ctrl_pass (gen_ctrl.hpp). k_gen_ctrl runs the first pass of a device loop
// (it issues the first step); after that the step kernel's device-descriptor
// variant runs a pass itself once its acceptance is done (its workgroup 0: the
// commit, the stop rules and the next step's draft and descriptor), so a device
// loop is one launch per step. Once a pass stops the loop the remaining launches
// return at once. The host enqueues the step launches in chunks and looks at the
// state once per chunk: no per-step host round trip.
#include <hip/hip_runtime.h>

#include "gen_ctrl.hpp"
#include "kernels.hpp"

namespace mtg {
namespace {

__global__ void __launch_bounds__(kGenThreads)
k_gen_ctrl(GenCtl c, const StepResult* __restrict__ res, const int32_t* __restrict__ step_err) {
  __shared__ int32_t s_ids[kGenLdsIds];
  __shared__ int s_red[kGenThreads / 64];
  __shared__ int s_small[4];
  const GenStepOutcome prev{res->n_match < 0 || *step_err != 0, res->choice, res->n_match};
  gen_ctrl_pass(c, prev, true, s_ids, s_red, s_small);
}

}  // namespace

void launch_gen_ctrl(hipStream_t s, const GenCtl& c, const StepResult* res_map, const int32_t* step_err) {
  k_gen_ctrl<<<1, kGenThreads, 0, s>>>(c, res_map, step_err);
}

}  // namespace mtg
