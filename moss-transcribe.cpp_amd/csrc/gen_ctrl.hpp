// gen_ctrl.hpp - one pass of the speculative controller of cpu_speculative_generate
// (reference src/cpu_speculative.cpp:68-147) on the device, run by one workgroup of
// kGenThreads threads: by k_gen_ctrl (generate.hip) before the first step of a
// device loop, and by the device-descriptor variant of the step kernel at its end,
// on the step it has just verified. A pass
//   1. takes the previous step's result (greedy choices, leading matches) and
//      commits it: accepted drafts, the raw choice that seeds the next step, the
//      rewind of the KV position (:115-135);
//   2. applies the stop rules (:90-98, :109-114): eos, the token limit, a full
//      KV cache, a step limit;
//   3. drafts the next step with cpu_ngram_draft (:27-38) over the committed ids
//      (with the stream drafter: over prompt ++ committed ids, the proposal
//      completed from a periodic token stream, as mtg_stream_draft does) and
//      writes the next step descriptor (seed + drafts, position, repetition
//      penalty window) to device memory.
#pragma once

#include <hip/hip_runtime.h>

#include "mtg_internal.hpp"

namespace mtg {

constexpr int kGenThreads = 256;
constexpr int kGenLdsIds = 8192;  // committed ids staged in LDS for the draft search

// The controller's device memory, a kernel argument of k_gen_ctrl and of the
// step kernel's device-descriptor variant (g == nullptr: no controller pass).
struct GenCtl {
  GenState* g;
  int32_t* ids;
  StepDesc* desc;
  const int32_t* prompt;  // the stream drafter's prompt ids (n_prompt)
  const int32_t* stream;  // one period of its stream (period)
};

// The outcome of the step the pass takes: `take` is false when no step is
// pending; `failed` when it left before its acceptance (a bounded wait ran out).
struct GenStepOutcome {
  bool failed;
  const int32_t* choice;  // the rows' greedy choices
  int n_match;
};

namespace gen {

__device__ __forceinline__ int block_max(int v, int* red) {
  for (int o = 32; o >= 1; o >>= 1) v = max(v, __shfl_xor(v, o));
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  int r = red[0];
  for (int i = 1; i < kGenThreads / 64; ++i) r = max(r, red[i]);
  __syncthreads();
  return r;
}

// one id appended to the committed sequence, with the stop rules of
// cpu_speculative_generate's emit (:90-98): eos stops (1), so does the
// max_new-th new id (2)
__device__ __forceinline__ void emit(GenState* g, int32_t* ids, int32_t id) {
  ids[g->n_ids++] = id;
  if (id == g->eos) g->stop = 1;
  else if (g->n_ids - g->first_new >= g->max_new) g->stop = 2;
}

}  // namespace gen

// One controller pass. s_ids: kGenLdsIds ints of LDS; s_red: kGenThreads / 64
// ints; s_small: 4 ints. When the pass stops the loop it writes T = 0 into the
// descriptor only if desc_on_stop (a step kernel still running may read it
// otherwise; the next launches also return on g->done).
__device__ __forceinline__ void gen_ctrl_pass(const GenCtl& c, const GenStepOutcome& prev, bool desc_on_stop,
                                              int32_t* s_ids, int* s_red, int* s_small) {
  GenState* __restrict__ g = c.g;
  int32_t* __restrict__ ids = c.ids;
  StepDesc* __restrict__ desc = c.desc;
  const int tid = threadIdx.x;
  int& s_go = s_small[0];
  int& s_n = s_small[1];
  int& s_budget = s_small[2];
  int& s_before = s_small[3];
  if (tid == 0) {
    bool go = !g->done;
    if (go && g->pending) {
      // 1. the previous step's result
      g->pending = 0;
      if (prev.failed) {
        // the step left before its acceptance: undo its seed and stop here; the
        // host finishes from this state
        g->err = 1;
        g->done = 1;
        g->n_ids -= 1;
        g->past = g->before;
        go = false;
      } else {
        const int before = g->before, np = g->np, n_match = prev.n_match;
        ++g->steps;
        ++g->target_calls;
        g->drafted_calls += np > 0;
        g->proposed += np;
        g->target_input_tokens += np + 1;
        int keep = 1;
        int32_t raw = prev.choice[0];
        for (int i = 0; i < np && i < n_match; ++i) {
          ++g->accepted;
          gen::emit(g, ids, g->proposal[i]);
          if (g->stop) break;  // the terminating token is emitted, not kept (:128)
          ++keep;
          raw = prev.choice[i + 1];
        }
        if (keep != np + 1) ++g->rewinds;  // :131-135
        g->past = before + keep;
        g->raw_choice = raw;
        if (g->stop) {
          g->done = 1;
          go = false;
        }
      }
    }
    if (go) {
      // 2. the next step's seed and the stop rules before it
      if (g->max_steps > 0 && g->steps >= g->max_steps) {
        g->done = 1;
        go = false;
      } else {
        const int32_t seed = g->raw_choice;
        gen::emit(g, ids, seed);
        if (g->stop) {
          g->done = 1;
          go = false;
        } else if (g->max_seq - g->past < 1) {
          // no room for the seed's row (:113-114)
          g->stop = 3;
          g->done = 1;
          go = false;
        } else {
          const int before = g->past;
          s_budget = max(0, min(min(g->max_draft, g->max_new - (g->n_ids - g->first_new)), g->max_seq - before - 1));
          s_before = before;
        }
      }
    }
    s_go = go;
    s_n = g->n_ids;
  }
  __syncthreads();
  if (!s_go) {
    if (tid == 0 && desc_on_stop) desc->T = 0;
    return;
  }
  // 3. cpu_ngram_draft over the history h = prompt ++ ids[0, n): the longest
  // suffix n-gram (16 .. 2) that occurred before, at its latest start; the ids that
  // followed it are the draft, completed up to the budget from the stream
  // (position of h's next id + k, modulo the period) when there is one
  const int n = s_n, budget = s_budget, n_prompt = g->n_prompt, period = g->period;
  const int nh_all = n_prompt + n;
  const bool staged = nh_all <= kGenLdsIds;
  if (staged)
    for (int i = tid; i < nh_all; i += kGenThreads) s_ids[i] = i < n_prompt ? c.prompt[i] : ids[i - n_prompt];
  __syncthreads();
  auto hist_at = [&](int i) { return staged ? s_ids[i] : (i < n_prompt ? c.prompt[i] : ids[i - n_prompt]); };
  auto id_at = [&](int i) { return hist_at(n_prompt + i); };  // committed id i
  // One pass over the ends e (2 <= e < |h|) of the candidate n-grams instead of
  // one pass per length: c(e), the length (at most 16) of the common suffix of
  // h[0, e) and h, is >= len exactly when the len-gram ending at e matches h's
  // suffix. The longest matching length is then the largest c(e) >= 2, and its
  // latest start belongs to the largest e with that c(e): the draft begins at e.
  int begin = -1;
  if (budget > 0 && nh_all >= 3) {
    const int lmax = min(16, nh_all - 1);
    int key = -1;  // c(e) << 26 | e, the largest over this thread's ends
    for (int e = nh_all - 1 - tid; e >= 2; e -= kGenThreads) {
      int cl = 0;
      while (cl < lmax && cl < e && hist_at(e - 1 - cl) == hist_at(nh_all - 1 - cl)) ++cl;
      if (cl >= 2) key = max(key, (cl << 26) | e);
      if (cl == lmax) break;  // this thread's later ends are smaller
    }
    key = gen::block_max(key, s_red);
    if (key >= 0) begin = key & ((1 << 26) - 1);
  }
  const int n_gram = begin >= 0 ? min(budget, nh_all - begin) : 0;
  const int np = period > 0 ? budget : n_gram;
  // the step descriptor: rows {seed, drafts} at `before`; the penalty window of
  // row i is the last 100 ids before the seed ++ rows 0..i (fill_desc's layout)
  const int T = np + 1, nh = n - 1;
  const bool pen = g->penalty > 1.0f;
  const int pstart = max(0, nh + 1 - kPenaltyWindow);
  const int nwin = nh - pstart;
  if (tid < kMaxRows) {
    int32_t tok = 0;
    if (tid == 0) tok = id_at(n - 1);  // the seed, emitted last
    else if (tid - 1 < n_gram) tok = hist_at(begin + tid - 1);
    else if (tid < T) tok = c.stream[(nh_all + tid - 1) % period];
    desc->tokens[tid] = tok;
    if (tid >= 1 && tid < T) g->proposal[tid - 1] = tok;
    if (pen && tid < T) desc->pen_ids[nwin + tid] = tok;
  }
  if (pen)
    for (int i = tid; i < nwin; i += kGenThreads) desc->pen_ids[i] = id_at(pstart + i);
  if (tid == 0) {
    desc->T = T;
    desc->past = s_before;
    desc->groups = (T + 7) / 8;
    desc->use_embeds = 0;
    desc->penalty = g->penalty;
    desc->n_pen = pen ? nwin + T : 0;
    desc->pen_base = pen ? nwin : 0;
    desc->write_logits = 0;
    g->np = np;
    g->before = s_before;
    g->pending = 1;
    ++g->issued;
    g->issued_rows += T;
    g->issued_past += s_before;
  }
}

}  // namespace mtg
