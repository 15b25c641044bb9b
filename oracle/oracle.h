/* oracle.h - CPU restatement of moss-transcribe.cpp's speculative verify path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle libmtg's parity tests
 * compare against, and the timed CPU baseline of bench.py. Only tests/,
 * __graft_entry__.smoke() and the bench's cpu_baseline leg load it; the product
 * never does.
 *
 * It restates, in plain C++ loops, the arithmetic the reference runs through ggml's
 * CPU backend (ggml itself is an un-vendored submodule and cannot be built):
 *   decoder step        src/qwen3_decoder.cpp:91-160, src/qwen3.cpp:62-218
 *   lm_head             src/qwen3_decoder.cpp:174-205
 *   causal context      src/cpu_context.cpp:13-32
 *   softmax op order    src/cpu_softmax.cpp:27-36
 *   controller/policy   src/cpu_speculative.cpp:19-50, 68-147
 *   embedding rows      src/generate.cpp:33-111
 * Every function below names the reference lines it follows in oracle.cpp.
 */
#ifndef MTG_ORACLE_H
#define MTG_ORACLE_H

#include <stdint.h>
#include "../include/mtg_verify.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orc_model orc_model;

int orc_create(const mtg_model_desc* desc, int32_t max_seq, int32_t kv_type, orc_model** out);

/* Float order of every reduction of the step. CANONICAL (the default): the order
 * the device kernels share with the oracle bit for bit (64-key attention chunks
 * merged in order, 4-slice q8_0 sums, butterfly sums). GGML_GENERIC: the order of
 * ggml's generic scalar CPU kernels (sequential block sums, double-accumulated
 * dots, soft_max_ext over the whole row then the context at the valid length),
 * an independent published order to measure the canonical one against. */
enum { ORC_ORDER_CANONICAL = 0, ORC_ORDER_GGML_GENERIC = 1 };
int orc_set_order(orc_model* m, int32_t order);
void orc_destroy(orc_model* m);
int32_t orc_past_len(const orc_model* m);
int orc_rewind(orc_model* m, int32_t position);
void orc_set_threads(int n);

int orc_embed(orc_model* m, const int32_t* ids, int32_t n, float* out);
int orc_run(orc_model* m, const float* embeds, int32_t T, float* hidden_out);
int orc_prefill(orc_model* m, const float* embeds, int32_t S, float* hidden_out);
int orc_logits(orc_model* m, const float* hidden, int32_t T, float* logits_out);
int orc_verify(orc_model* m, const int32_t* tokens, int32_t T, const int32_t* history,
               int32_t n_history, float penalty, int32_t* choice_out, int32_t* n_match_out,
               float* hidden_out, float* logits_out);
int orc_kv_write(orc_model* m, const void* k, const void* v, int32_t n_pos);
int orc_kv_read(const orc_model* m, void* k, void* v, int32_t n_pos);

int32_t orc_ngram_draft(const int32_t* history, int32_t n, int32_t maximum, int32_t* out);
int32_t orc_greedy_choice(const float* raw, int32_t n, const int32_t* history, int32_t n_history,
                          float penalty);

/* The controller loop alone, over any target (a scripted one in the policy
 * tests, an orc_model through orc_generate_from). */
struct orc_target;
/* Runs T rows at target->past; the controller then advances target->past. */
typedef int (*orc_verify_fn)(struct orc_target* target, const int32_t* tokens, int32_t T,
                             const int32_t* history, int32_t n_history, float penalty,
                             int32_t* choice_out, int32_t* n_match_out);
typedef struct orc_target {
  void* self;
  orc_verify_fn verify;
  int32_t past;     /* kept in sync by the controller: += T on verify, then rewind */
  int32_t max_seq;
  int32_t vocab;
} orc_target;
int orc_controller(orc_target* target, int32_t first_seed, const int32_t* prior_ids,
                   int32_t n_prior, int32_t max_new, int32_t max_steps, int32_t eos, float penalty,
                   int32_t max_draft, mtg_draft_fn draft, void* user, int32_t* ids_out,
                   int32_t* n_ids_out, mtg_gen_stats* stats);

int orc_generate_from(orc_model* m, int32_t first_seed, const int32_t* prior_ids, int32_t n_prior,
                      int32_t max_new, int32_t max_steps, int32_t eos, float penalty,
                      int32_t max_draft, mtg_draft_fn draft, void* user, int32_t* ids_out,
                      int32_t* n_ids_out, mtg_gen_stats* stats);

/* primitives, exposed for unit tests */
uint16_t orc_f32_to_f16(float f);
float orc_exp(float x); /* the exp of attention and SiLU */
float orc_f16_to_f32(uint16_t h);
void orc_quantize_q8_0_act(const float* x, int64_t k, void* blocks);
void orc_quantize_q8_k_act(const float* x, int64_t k, void* blocks);
int32_t orc_q8_0_block_dot(const void* a, const void* b);
/* the canonical q8_0 GEMM's exact int32 dots of nb consecutive 32-code blocks (x in [-127, 127]) */
void orc_q8_0_block_dots(const int8_t* w, const int8_t* x, int32_t nb, int32_t* out);
void orc_mul_mat(int32_t wtype, const void* w, int32_t k, int32_t n, const float* x, int32_t T,
                 float* y);
/* the same product in ggml's generic scalar order (ORC_ORDER_GGML_GENERIC) */
void orc_mul_mat_generic(int32_t wtype, const void* w, int32_t k, int32_t n, const float* x, int32_t T,
                         float* y);
void orc_rms_norm(const float* x, const float* w, int32_t n, float eps, float* y);
void orc_rope_neox(float* x, int32_t n_dims, int32_t pos, float base);
void orc_softmax(const float* s, int32_t n, float scale, const float* mask, float* out);
void orc_causal_context(const float* v, const float* p, int32_t head_dim, int32_t kv_heads,
                        int32_t heads, int32_t queries, int32_t kv_len, float* out);
/* The decoder step's attention in the canonical order (chunks of 64 keys merged
 * in order): T query rows q [T][heads * head_dim] at positions
 * past .. past + T - 1 over k, v [kv_heads][max_seq][head_dim] holding keys
 * [0, past + T) (f32, or f16 bits when f16kv; q then rounded to f16). */
void orc_attention(const void* k, const void* v, int32_t f16kv, int32_t max_seq, int32_t past, int32_t T,
                   int32_t heads, int32_t kv_heads, int32_t head_dim, const float* q, float* out);

/* ---- Whisper encoder + audio adaptor (src/whisper_encoder.cpp:103-209,
 * src/audio_adaptor.cpp:38-97) ---- */
typedef struct orc_encoder orc_encoder;
int orc_encoder_create(const mtg_encoder_desc* desc, orc_encoder** out);
void orc_encoder_destroy(orc_encoder* e);
int orc_encoder_encode(orc_encoder* e, const float* mel, float* out, int32_t* rows_out);
int orc_encoder_adapt(orc_encoder* e, const float* rows, int32_t T, float* out, int32_t* n_out);
/* its parts */
float orc_gelu_erf(float x);
void orc_layer_norm(const float* x, const float* w, const float* b, int32_t n, float eps, float* y);
/* y [OL][oc] = conv1d of x [ic][L] with w [oc][ic][3], pad 1, stride s (no bias) */
void orc_conv1d(const float* w, int32_t ic, int32_t oc, const float* x, int32_t L, int32_t stride, float* y);
/* unmasked multi-head attention, q / k / v / out [T][n_heads * head_dim] */
void orc_enc_attention(const float* q, const float* k, const float* v, int32_t T, int32_t n_heads,
                       int32_t head_dim, float* out);

#ifdef __cplusplus
}
#endif
#endif
