// mtg_internal.hpp - data layouts shared by the gfx950 kernels and the host runtime.
//
// HBM layouts (all chosen for the kernels, not for the GGUF file):
//
// * q8_0 matrix "N rows of K" -> MFMA panel tiles. Rows are grouped in tiles of 16,
//   K in block pairs of 64 (two 32-element q8_0 blocks). One (tile, pair) unit is
//   1088 bytes: 1024 code bytes laid out as the A operand of
//   v_mfma_i32_16x16x64_i8 (lane l: row l%16, block 2*pair + (l/16)/2, bytes
//   16*((l/16)%2)..+16), then 64 bytes of f16 scales [parity][row]. A tile is the
//   K/64 units of its rows, contiguous, so one wave streams a tile with 16-byte
//   loads and no bytes are added to the 34-byte q8_0 blocks.
// * activation panel: the B operand of the same MFMA for up to 8 verify rows
//   (one column group; two groups cover 16 rows). For block pair bp and lane l
//   (j = l%16, g = l/16): column j is row t = j%8 of block 2*bp + j/8; lanes with
//   g/2 != j/8 hold zeros (block-diagonal, so each MFMA returns two exact
//   per-block int32 dots). Per (group, pair): 1024 code bytes + 16 f32 scales.
// * KV cache: [layer][kv_head][position][head_dim], f32 or f16.
#pragma once

#include <stdint.h>

#include "../../include/mtg_verify.h"

namespace mtg {

constexpr int kTileRows = 16;
constexpr int kPairK = 64;
constexpr int kUnitBytes = 1088;       // 1024 codes + 32 f16 scales
constexpr int kPanelPairBytes = 1024;  // activation codes per (group, pair)
constexpr int kMaxRows = MTG_MAX_BATCH;
constexpr int kMaxGroups = 2;          // column groups of 8 rows
constexpr int kChunkKeys = 64;         // keys per attention chunk
constexpr int kMaxCols = 2 * MTG_MAX_BATCH;  // attention query columns (2 q heads x rows)
constexpr int kHeadDim = 128;
constexpr int kPenaltyWindow = 100;
constexpr int kLmWorkgroups = 1024;    // lm_head grid (grid-stride over tiles)

// Per-step inputs, written by the host before every verify step and read by every
// kernel of the step (so a captured graph can be replayed for any T and past).
struct StepDesc {
  int32_t T;          // verify rows (1..16)
  int32_t past;       // KV positions before the step
  int32_t groups;     // column groups: (T + 7) / 8
  int32_t use_embeds; // 1: x comes from host embeddings, 0: from tokens
  float penalty;      // > 1 enables the repetition penalty
  int32_t n_pen;      // entries in pen_ids
  int32_t pen_base;   // pen window of row i is [max(0, pen_base + i - 99), pen_base + i + 1)
  int32_t write_logits;
  int32_t tokens[kMaxRows];
  int32_t pen_ids[kPenaltyWindow + kMaxRows];
};

// Results of one verify step (T + 2 ints travel back to the host).
struct StepResult {
  int32_t choice[kMaxRows];
  int32_t n_match;
  int32_t err;  // nonzero: a grid-barrier wait of the step kernel ran out
};

// The device-side speculative controller's state (generate.hip): set up by
// the host, advanced by k_gen_ctrl between verify steps.
struct GenState {
  // set by the host
  int32_t first_new;  // committed ids before the run (prior ids)
  int32_t max_new, max_steps, eos, max_draft, max_seq;
  float penalty;
  // the stream drafter (mtg_stream_draft): text ids before generation, prepended to
  // the committed ids for the n-gram search, and a periodic stream that completes
  // the proposal (n_prompt = period = 0: the plain n-gram drafter)
  int32_t n_prompt, period;
  // the controller's state
  int32_t n_ids;       // committed ids
  int32_t past;        // KV position
  int32_t raw_choice;  // seed of the next step
  int32_t steps;
  int32_t done;        // the loop ended: stop gives the reason (0: the step limit)
  int32_t stop;        // 1 eos, 2 token limit, 3 KV cache full
  int32_t err;         // a step left before its acceptance (its seed is undone)
  int32_t pending;     // a step was issued and its result is not yet taken
  int32_t before, np;  // position and draft count of that step
  int32_t proposal[kMaxRows];
  int64_t target_calls, drafted_calls, proposed, accepted, target_input_tokens, rewinds;
  // steps issued so far, their rows and the sum of their start positions (the
  // host's launch timing counts the launches that ran a step)
  int64_t issued, issued_rows, issued_past;
};

}  // namespace mtg
