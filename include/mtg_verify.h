/* mtg_verify.h - C ABI of the MI355X speculative draft->verify decode path.
 *
 * The library (libmtg.so) runs the Qwen3 target pass of moss-transcribe.cpp's
 * speculative decoder on one gfx950 GPU: T verify rows (seed + drafts) go through
 * all decoder layers as one batch over a persistent device KV cache, followed by
 * the tied lm_head, a greedy first-max choice per row (optional repetition
 * penalty) and longest-prefix acceptance on the device.
 *
 * Reference interfaces each entry point replaces (paths relative to the
 * moss-transcribe.cpp source tree):
 *   mtg_create/mtg_destroy    Qwen3Decoder::load, ~Qwen3Decoder     src/qwen3_decoder.cpp:16-85
 *   mtg_prefill               Qwen3Decoder::prefill                 src/qwen3_decoder.cpp:162-166
 *   mtg_append                CpuSpeculativeDecoder::append -> run  src/cpu_speculative.cpp:19-21,
 *                                                                    src/qwen3_decoder.cpp:91-160
 *   mtg_logits                Qwen3Decoder::logits_from_hidden      src/qwen3_decoder.cpp:174-205
 *   mtg_embed                 embed_rows_f32                        src/generate.cpp:68-111
 *   mtg_verify                append + lazy logits + cpu_greedy_choice + accept loop
 *                                                                    src/cpu_speculative.cpp:109-130
 *   mtg_rewind/mtg_past_len   CpuSpeculativeDecoder::rewind, Qwen3Decoder::past_len
 *                                                                    src/cpu_speculative.cpp:22-24,
 *                                                                    src/qwen3_decoder.hpp:55
 *   mtg_remaining             CpuSpeculativeDecoder::remaining       src/cpu_speculative.cpp:25
 *   mtg_generate              cpu_speculative_generate               src/cpu_speculative.cpp:68-147
 *   mtg_speculative_run       the loop of cpu_speculative_generate   src/cpu_speculative.cpp:89-137
 *   mtg_ngram_draft           cpu_ngram_draft                        src/cpu_speculative.cpp:27-38
 *   mtg_greedy_choice         cpu_greedy_choice                      src/cpu_speculative.cpp:39-50
 *   mtg_q8_pack/mtg_q8_mul_mat  cpu_pack_q8 / cpu_decode_mul_mat     src/cpu_q8.hpp:13-27,
 *                                                                    src/cpu_q8.cpp:30-129
 *   mtg_causal_context        cpu_causal_context                     src/cpu_context.hpp:7-10,
 *                                                                    src/cpu_context.cpp:13-56
 *   mtg_last_error            moss_transcribe_capi_last_error        include/moss_transcribe_capi.h:50-53
 *
 * Conventions: every function returns an int status (MTG_OK == 0, negative on
 * error) and never lets a C++ exception cross; the error text is owned by the
 * context (mtg_last_error). Calls on one context are serialized by the caller
 * (as the reference serializes graph execution). Host pointers are plain host
 * memory; the *_dev entry points take device pointers.
 */
#ifndef MTG_VERIFY_H
#define MTG_VERIFY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MTG_ABI_VERSION 1
#define MTG_MAX_BATCH 16 /* verify rows per step (seed + up to 15 drafts) */

/* Tensor element types, numbered as ggml numbers them (ggml.h GGML_TYPE_*). */
enum {
  MTG_TYPE_F32 = 0,
  MTG_TYPE_F16 = 1,
  MTG_TYPE_Q8_0 = 8,
  MTG_TYPE_Q4_K = 12
};

enum {
  MTG_OK = 0,
  MTG_ERR_INVALID = -1,     /* bad argument (reference: returns false / throws) */
  MTG_ERR_UNSUPPORTED = -2, /* shape or type not handled (reference: nullptr fallback) */
  MTG_ERR_DEVICE = -3,      /* HIP runtime error */
  MTG_ERR_CAPACITY = -4,    /* past + T > max_seq (reference: run() returns false) */
  MTG_ERR_NOMEM = -5,
  MTG_ERR_STATE = -6        /* invalid rewind / call order */
};

/* Decoder dimensions (reference: Qwen3Hparams, src/qwen3.hpp:7). */
typedef struct mtg_hparams {
  int32_t hidden;       /* 1024 */
  int32_t n_heads;      /* 16 */
  int32_t n_kv_heads;   /* 8 */
  int32_t head_dim;     /* 128 */
  int32_t intermediate; /* 3072 */
  int32_t n_layers;     /* 28 */
  int32_t vocab;        /* 151936 */
  float rope_base;      /* 1e6 */
  float rms_eps;        /* 1e-6 */
} mtg_hparams;

/* One decoder layer, tensor names of the reference GGUF (src/qwen3.cpp:44-54).
 * Matrices are row-major "N rows of K" in ggml block layout of weight_type:
 * ggml ne = [K, N]. Norm gains are f32. */
typedef struct mtg_layer_tensors {
  const float* attn_norm;   /* [hidden] */
  const void* attn_q;       /* N = n_heads*head_dim, K = hidden */
  const void* attn_k;       /* N = n_kv_heads*head_dim, K = hidden */
  const void* attn_v;       /* N = n_kv_heads*head_dim, K = hidden */
  const void* attn_o;       /* N = hidden, K = n_heads*head_dim */
  const float* attn_q_norm; /* [head_dim] */
  const float* attn_k_norm; /* [head_dim] */
  const float* ffn_norm;    /* [hidden] */
  const void* ffn_gate;     /* N = intermediate, K = hidden */
  const void* ffn_up;       /* N = intermediate, K = hidden */
  const void* ffn_down;     /* N = hidden, K = intermediate */
} mtg_layer_tensors;

typedef struct mtg_model_desc {
  mtg_hparams hp;
  int32_t weight_type;              /* MTG_TYPE_Q8_0, MTG_TYPE_F16, MTG_TYPE_F32 or MTG_TYPE_Q4_K */
  const void* token_embd;           /* N = vocab, K = hidden; also the tied lm_head */
  const float* output_norm;         /* [hidden] */
  const mtg_layer_tensors* layers;  /* n_layers entries */
} mtg_model_desc;

typedef struct mtg_ctx mtg_ctx;

int mtg_abi_version(void);

/* Upload weights (re-tiled for the gfx950 kernels) and allocate a KV cache of
 * max_seq positions of kv_type (MTG_TYPE_F32 or MTG_TYPE_F16). The host tensors
 * may be freed after the call. A context owns one HIP stream on the current
 * device; its calls are not synchronized with each other, so one host thread
 * uses it at a time (distinct contexts may run side by side). */
int mtg_create(const mtg_model_desc* desc, int32_t max_seq, int32_t kv_type, mtg_ctx** out);
void mtg_destroy(mtg_ctx* ctx);
const char* mtg_last_error(const mtg_ctx* ctx);

int32_t mtg_past_len(const mtg_ctx* ctx);
int32_t mtg_remaining(const mtg_ctx* ctx);
/* Logical rewind; fails with MTG_ERR_STATE unless 0 <= position <= past_len. */
int mtg_rewind(mtg_ctx* ctx, int32_t position);

/* Dequantized embedding rows of ids (token-major, n x hidden floats). */
int mtg_embed(mtg_ctx* ctx, const int32_t* ids, int32_t n, float* out);

/* reset + run S rows; hidden_out (nullable) receives the final-normed hidden of
 * every row (S x hidden). The rows go through the decoder in blocks of up to
 * 2,048 (each weight matrix streamed once per block, causal attention over the
 * cache), for every weight type; with mtg_prefill_mode(ctx, 0) in verify
 * batches of up to MTG_MAX_BATCH. Both give the same bits. */
int mtg_prefill(mtg_ctx* ctx, const float* embeds, int32_t S, float* hidden_out);
/* blocks != 0 (the default): the block prefill where it applies; 0: verify-size
 * batches (no counterpart in the reference; for comparing the two paths). */
int mtg_prefill_mode(mtg_ctx* ctx, int32_t blocks);
/* Device time of the last block prefill in ms (HIP events on the context's
 * stream, uploads of the rows included). */
double mtg_last_prefill_ms(const mtg_ctx* ctx);

/* Append T (1..MTG_MAX_BATCH) embedding rows at past_len; past_len += T.
 * hidden_out (nullable) receives T x hidden final-normed rows. */
int mtg_append(mtg_ctx* ctx, const float* embeds, int32_t T, float* hidden_out);

/* Tied lm_head for T rows of final-normed hidden: logits_out T x vocab. */
int mtg_logits(mtg_ctx* ctx, const float* hidden, int32_t T, float* logits_out);

/* One verify step. tokens = {seed, draft_1 .. draft_{T-1}}. Appends all T rows
 * at past_len (past_len += T), computes the greedy choice after every row with
 * the repetition penalty applied over the last 100 ids of
 * history ++ tokens[0..i] (penalty <= 1 disables it), and the number of leading
 * drafts equal to the choice of the row before them:
 *   n_match = max m such that tokens[i+1] == choice[i] for all i < m.
 * Only T+1 ints come back from the device; hidden_out / logits_out (nullable)
 * additionally return T x hidden / T x vocab floats for parity checks.
 * Stop rules and the rewind to past + keep are the caller's (mtg_generate). */
int mtg_verify(mtg_ctx* ctx, const int32_t* tokens, int32_t T,
               const int32_t* history, int32_t n_history, float penalty,
               int32_t* choice_out, int32_t* n_match_out,
               float* hidden_out, float* logits_out);

/* KV cache exchange, layout [layer][kv_head][position][head_dim] in kv_type.
 * mtg_kv_write sets past_len = n_pos. */
int mtg_kv_write(mtg_ctx* ctx, const void* k, const void* v, int32_t n_pos);
int mtg_kv_read(mtg_ctx* ctx, void* k, void* v, int32_t n_pos);

/* ---- speculative generation controller (host C++) ---- */

/* Draft hook: write up to `budget` proposals for the committed ids into out and
 * return the count (reference: CpuSpeculativeHooks::draft, src/cpu_speculative.hpp:11). */
typedef int32_t (*mtg_draft_fn)(void* user, const int32_t* ids, int32_t n_ids, int32_t budget,
                                int32_t* out);
/* Commit hook, called after every step with the committed ids and whether a stop
 * rule fired (reference: CpuSpeculativeHooks::committed, src/cpu_speculative.hpp:14). */
typedef void (*mtg_commit_fn)(void* user, const int32_t* ids, int32_t n_ids, int32_t past_len,
                              int32_t stopped);

typedef struct mtg_gen_stats {
  int64_t target_calls, drafted_calls, proposed, accepted, target_input_tokens, rewinds;
  double prefill_seconds, verify_seconds, draft_seconds;
  int32_t stop_reason; /* 0 none/error, 1 eos, 2 token_limit, 3 KV cache full */
  int32_t next_seed;   /* greedy choice of the last kept row (the next step's seed) */
} mtg_gen_stats;

/* A decoder the controller drives (reference: the Qwen3Decoder that
 * cpu_speculative_generate appends to and rewinds, src/cpu_speculative.cpp:17-26).
 * verify runs T rows {seed, drafts} at *past (the controller then sets *past to
 * past + T) and returns the greedy choice after every row and the number of
 * leading drafts equal to the choice of the row before them, as mtg_verify does;
 * the controller rewinds by writing *past. A nonzero return aborts the loop. */
typedef int32_t (*mtg_target_verify_fn)(void* self, const int32_t* tokens, int32_t T,
                                        const int32_t* history, int32_t n_history, float penalty,
                                        int32_t* choice_out, int32_t* n_match_out);
typedef struct mtg_target {
  void* self;
  mtg_target_verify_fn verify;
  int32_t* past;   /* the target's past_len */
  int32_t max_seq;
  int32_t vocab;
} mtg_target;

/* The loop of cpu_speculative_generate over any target, continuing from its
 * current state: emit the seed (eos / token-limit stops), budget =
 * min(max_draft, max_new - emitted, max_seq - past - 1), draft (draft == NULL:
 * mtg_ngram_draft), verify seed + drafts, emit the drafts that equal the greedy
 * choice of the row before them (a stopping token is emitted but not kept),
 * logical rewind to past + kept. first_seed: the greedy choice of the last row
 * already in the target. prior_ids (nullable): ids committed before, visible to
 * the drafter and the penalty window. max_steps <= 0: until a stop rule fires.
 * Returns the verify callback's status or MTG_ERR_INVALID (bad draft id). */
int mtg_speculative_run(const mtg_target* target, int32_t first_seed, const int32_t* prior_ids,
                        int32_t n_prior, int32_t max_new, int32_t max_steps, int32_t eos,
                        float penalty, int32_t max_draft, mtg_draft_fn draft,
                        mtg_commit_fn commit, void* user, int32_t* ids_out, int32_t* n_ids_out,
                        mtg_gen_stats* stats);

/* cpu_speculative_generate on the device decoder: prefill `seq` fused rows, take
 * the first greedy seed, then loop {draft <= max_draft, verify, accept, rewind}
 * until eos or max_new tokens. draft == NULL uses mtg_ngram_draft. ids_out must
 * hold max_new ids. */
int mtg_generate(mtg_ctx* ctx, const float* fused, int32_t seq, int32_t max_new, int32_t eos,
                 float penalty, int32_t max_draft, mtg_draft_fn draft, mtg_commit_fn commit,
                 void* user, int32_t* ids_out, int32_t* n_ids_out, mtg_gen_stats* stats);

/* mtg_speculative_run on the device decoder, from its current KV state. */
int mtg_generate_from(mtg_ctx* ctx, int32_t first_seed, const int32_t* prior_ids,
                      int32_t n_prior, int32_t max_new, int32_t max_steps, int32_t eos,
                      float penalty, int32_t max_draft, mtg_draft_fn draft, mtg_commit_fn commit,
                      void* user, int32_t* ids_out, int32_t* n_ids_out, mtg_gen_stats* stats);

/* mtg_generate_from with the whole loop on the device (reference
 * cpu_speculative_generate, src/cpu_speculative.cpp:68-147, with
 * cpu_ngram_draft, :27-38): a controller kernel between the verify steps commits
 * each step's accepted ids, applies the stop rules, drafts the next step and
 * writes its descriptor, so the host neither drafts nor waits per step (it looks
 * at the state every 8 steps). Same ids, counters, stop reason and KV position
 * as mtg_generate_from with draft == NULL. No draft or commit hooks; stats carry
 * no draft time (verify_seconds is the whole run). MTG_ERR_UNSUPPORTED unless
 * the step kernel runs this model (q8_0, f16 or f32 weights, MTG_EXEC_STEP_KERNEL);
 * max_draft is clamped to MTG_MAX_BATCH - 1 as in mtg_generate_from (above 7 the
 * 16-row step kernel runs every step; with f16 or f32 weights, whose step kernel
 * runs 8 rows, a max_draft above 7 returns MTG_ERR_UNSUPPORTED). Every step runs on the
 * step kernel, also past mtg_set_step_max_keys. A step abandoned on a bounded wait
 * is finished by the host controller from the same state. */
int mtg_generate_device(mtg_ctx* ctx, int32_t first_seed, const int32_t* prior_ids, int32_t n_prior,
                        int32_t max_new, int32_t max_steps, int32_t eos, float penalty, int32_t max_draft,
                        int32_t* ids_out, int32_t* n_ids_out, mtg_gen_stats* stats);

/* Draft hook for long-context workloads (pass mtg_stream_draft as `draft` and a
 * mtg_stream_drafter as `user`): the reference n-gram proposal over
 * prompt ++ ids, completed up to the budget from a periodic token stream
 * aligned to the absolute position of the next token. */
typedef struct mtg_stream_drafter {
  const int32_t* prompt; /* text ids that precede generation */
  int32_t n_prompt;
  const int32_t* stream; /* one period of the token stream */
  int32_t period;        /* 0: n-gram proposal only */
} mtg_stream_drafter;
int32_t mtg_stream_draft(void* user, const int32_t* ids, int32_t n_ids, int32_t budget,
                         int32_t* out);

/* mtg_generate_device with the stream drafter run by the device controller: the
 * draft hook the reference loop calls every step (CpuSpeculativeHooks::draft,
 * src/cpu_speculative.cpp:105) as mtg_generate_from calls it with
 * draft = mtg_stream_draft and user = drafter: the n-gram proposal over
 * prompt ++ committed ids, completed from the periodic stream. The drafter's
 * arrays are copied to the device at the call. drafter == NULL: mtg_generate_device.
 * Same ids, counters, stop reason and KV position as that host loop. */
int mtg_generate_device_stream(mtg_ctx* ctx, int32_t first_seed, const int32_t* prior_ids, int32_t n_prior,
                               int32_t max_new, int32_t max_steps, int32_t eos, float penalty, int32_t max_draft,
                               const mtg_stream_drafter* drafter, int32_t* ids_out, int32_t* n_ids_out,
                               mtg_gen_stats* stats);

/* How a step runs on the device. MTG_EXEC_STEP_KERNEL (the default for the
 * Qwen3-0.6B shape with q8_0, f16 or f32 weights on a device with at least 256
 * CUs): one persistent dataflow kernel per step (f16 and f32 weights: steps of up
 * to 8 rows; longer ones take the per-op graph). MTG_EXEC_GRAPH (the default otherwise): the
 * per-op kernels, replayed from a captured HIP graph. MTG_EXEC_EAGER: the per-op
 * kernels launched one by one (profiling). All modes produce the same results. */
enum { MTG_EXEC_STEP_KERNEL = 0, MTG_EXEC_GRAPH = 1, MTG_EXEC_EAGER = 2 };
int mtg_set_exec_mode(mtg_ctx* ctx, int32_t mode);
int32_t mtg_exec_mode(const mtg_ctx* ctx);

/* Path selection by context length (no counterpart in the reference, which has
 * one CPU path): in MTG_EXEC_STEP_KERNEL mode a verify / append step whose KV
 * length (past_len + rows) exceeds max_keys runs on the per-op graph instead of
 * the persistent kernel. max_keys <= 0 restores the default: no limit for q8_0
 * weights; 5,120 for f16 weights, whose per-op attention (three workgroups per
 * CU) overtakes the persistent kernel's at longer contexts on MI355X, and 8,192
 * (the longest measured length) for f32 weights. The device loop (mtg_generate_device) always runs the persistent
 * kernel. mtg_step_kernel_runs counts the steps that ran to their end on the
 * persistent kernel. */
int mtg_set_step_max_keys(mtg_ctx* ctx, int32_t max_keys);
int64_t mtg_step_kernel_runs(const mtg_ctx* ctx);

/* Diagnostics: copy an internal activation buffer of the last step (16 rows):
 * the residual stream, the fused q|k|v projection, the attention output, the
 * SwiGLU activation or the final-normed hidden rows. */
enum { MTG_DEBUG_X = 0, MTG_DEBUG_QKV = 1, MTG_DEBUG_O = 2, MTG_DEBUG_ACT = 3, MTG_DEBUG_HIDDEN = 4 };
int mtg_debug_copy(mtg_ctx* ctx, int32_t which, void* out, size_t bytes);

/* Failure-path check (no counterpart in the reference): the next step on the
 * persistent kernel starts with its error word raised, so every bounded wait of
 * that launch gives up at its first poll and every workgroup leaves, as after a
 * wait that ran out. The step returns MTG_ERR_DEVICE without advancing past_len;
 * the following steps run normally. */
int mtg_debug_abort_next_step(mtg_ctx* ctx);

/* Bounded waits (no counterpart in the reference): every wait of the persistent
 * step kernel gives up after a poll limit or 50 ms of device clock, raising the
 * error word so that every workgroup leaves; the step then runs again on the
 * per-op kernels (which need no co-resident workgroups) and
 * mtg_step_fallbacks counts it. mtg_debug_wait_limit sets the poll limit (<= 0:
 * the default, 2^23) so that a test can force that path from the host. */
int mtg_debug_wait_limit(mtg_ctx* ctx, int32_t polls);
int64_t mtg_step_fallbacks(const mtg_ctx* ctx);

/* Profiling of the persistent step kernel: when enabled, the kernel records a
 * 100 MHz device clock into MTG_PROFILE_SLOTS slots. Workgroup 0, slots 0..1023:
 * 0 at the start; for layer l at 3 + 12 l + {0, 1}: QKV inputs ready / QKV
 * published, {2, 3}: attention, {4, 5}: o-proj, {6, 7}: down (when workgroup 0
 * has those roles); at 3 + 12 L the lm_head start, + 1 its end, + 2 / + 3 the
 * acceptance (verify steps), + 4 its keys loaded, + 5 its choices reduced. Every workgroup w, layer 1, slots 1024 + 32 w + k:
 * k = 0..11 ready / published of QKV, attention, merge, o-proj, gate-up, down;
 * 12 / 13 first poll and poll count of the o-proj or gate-up wait, 14 / 15 of the
 * attention wait; 16..23 the attention item's stages. mtg_step_profile_read
 * copies the slots of the last step (returns the count). */
#define MTG_PROFILE_SLOTS 9216
int mtg_step_profile(mtg_ctx* ctx, int32_t enable);
int32_t mtg_step_profile_read(mtg_ctx* ctx, uint64_t* marks, int32_t n);

/* Launch timing: when enabled, every verify / append step's device work is
 * bracketed by two HIP events on the context's stream; the read-out gives the
 * summed event time, the number of timed steps and the sums of their past_len
 * and row counts (so a caller can divide the algorithmic bytes per step by the
 * measured time). A step whose persistent kernel gave up on a bounded wait counts
 * once, with the time of the abandoned launch plus that of its rerun on the
 * per-op kernels (mtg_step_fallbacks counts such steps). Enabling resets the sums. */
int mtg_launch_timing(mtg_ctx* ctx, int32_t enable);
int mtg_launch_timing_read(const mtg_ctx* ctx, double* total_ms, int64_t* launches,
                           int64_t* past_sum, int64_t* rows_sum);

/* Host policy functions (reference: cpu_ngram_draft, cpu_greedy_choice). */
int32_t mtg_ngram_draft(const int32_t* history, int32_t n, int32_t maximum, int32_t* out);
int32_t mtg_greedy_choice(const float* raw, int32_t n, const int32_t* history, int32_t n_history,
                          float penalty);

/* ---- kernel-level entry points on device pointers ---- */

typedef struct mtg_q8_packed mtg_q8_packed;
/* Upload and re-tile one q8_0 matrix (N rows of K, K % 64 == 0, N % 16 == 0).
 * Returns MTG_ERR_UNSUPPORTED for other shapes (the caller keeps its own path). */
int mtg_q8_pack(const void* blocks, int32_t k, int32_t n, mtg_q8_packed** out);
void mtg_q8_free(mtg_q8_packed* p);
/* Download the tiles and restore the n rows of q8_0 blocks they were packed from
 * (reference: PackedQ8::round_trip_exact, src/cpu_q8.hpp:17). */
int mtg_q8_unpack(const mtg_q8_packed* p, void* blocks);
/* y_dev[t][n] = q8_0 dot of the packed rows with x_dev[t][:] (T x K floats,
 * quantized to q8_0 per 32-block on the device), T in 1..MTG_MAX_BATCH. */
int mtg_q8_mul_mat_dev(const mtg_q8_packed* w, const float* x_dev, int32_t T, float* y_dev);

/* mtg_q8_mul_mat_dev without any allocation (no counterpart in the reference;
 * for callers that cannot allocate device memory: code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The descriptor and the
 * activation panel live in one static device array per GPU (about 137 KiB, held
 * until the process ends) instead of per-call hipMalloc; K is limited to 4096
 * (MTG_ERR_CAPACITY above, with the reason in mtg_last_error(NULL)). The call
 * enqueues three kernels on `stream` (NULL: the default stream) and returns
 * without waiting; the caller synchronizes. Every call on one GPU shares the
 * array, so calls that overlap on one GPU (other streams, other threads) race:
 * serialize them. */
int mtg_q8_mul_mat_dev_noalloc(const mtg_q8_packed* w, const float* x_dev, int32_t T, float* y_dev,
                               void* stream);

/* out_dev[h][q][f] = sum_{k <= past+q} v[h/groups][k][f] * p[h][q][k]
 * v_dev: [kv_heads][kv_len][head_dim] f32, p_dev: [heads][queries][kv_len] f32,
 * past = kv_len - queries; each query reads exactly its valid length. */
int mtg_causal_context_dev(const float* v_dev, const float* p_dev, int32_t head_dim,
                           int32_t kv_heads, int32_t heads, int32_t queries, int32_t kv_len,
                           float* out_dev);

/* ---- GGUF model files (reference: ModelLoader::load / read_config,
 * src/model_loader.cpp:21-169; tensor names src/qwen3.cpp:33-56,
 * src/qwen3_decoder.cpp:53-57) ---- */

typedef struct mtg_gguf mtg_gguf;
/* Map and parse a GGUF (v2 / v3) file: header, metadata, tensor table, every
 * tensor's data range checked against the file. On failure the reason is in
 * mtg_gguf_error(NULL) (and mtg_last_error(NULL)). */
int mtg_gguf_open(const char* path, mtg_gguf** out);
void mtg_gguf_close(mtg_gguf* g);
const char* mtg_gguf_error(const mtg_gguf* g);
int64_t mtg_gguf_n_tensors(const mtg_gguf* g);
/* One tensor by name: ggml type, ne[4], data in the mapping, bytes. */
int mtg_gguf_tensor(const mtg_gguf* g, const char* name, int32_t* type, int64_t* ne, const void** data,
                    size_t* bytes);
/* The Qwen3 decoder of the file: hyper-parameters from the mtd.text.* keys
 * (the reference's defaults where absent), every tensor found by name and
 * checked for shape and for one weight type (q8_0, f16, f32 or q4_K); f16 norm
 * gains are widened to f32. NULL on failure (mtg_gguf_error). The description
 * stays valid until mtg_gguf_close. */
const mtg_model_desc* mtg_gguf_model(mtg_gguf* g);
/* mtg_gguf_open + mtg_gguf_model + mtg_create; the file is unmapped before
 * returning. */
int mtg_create_from_gguf(const char* path, int32_t max_seq, int32_t kv_type, mtg_ctx** out);

/* ---- Whisper encoder + audio adaptor (reference: WhisperEncoder,
 * src/whisper_encoder.cpp:64-209, and AudioAdaptor, src/audio_adaptor.cpp:22-97)
 * ---- */

typedef struct mtg_encoder_hparams {
  int32_t n_mels;    /* mtd.audio.mel_bins (80) */
  int32_t n_frames;  /* mel frames of one chunk (3000); the encoder emits (n_frames - 1) / 2 + 1 rows */
  int32_t d_model;   /* mtd.audio.d_model (1024) */
  int32_t n_layers;  /* mtd.audio.n_layers (24) */
  int32_t n_heads;   /* mtd.audio.n_heads (16, head_dim 64) */
  int32_t ffn;       /* mtd.audio.ffn (4096) */
  int32_t merge;     /* mtd.audio_merge_size (4): frames per adaptor row */
  int32_t hidden;    /* the adaptor's output width, text hidden (1024) */
  float adaptor_eps; /* mtd.adaptor_norm_eps (1e-6); the encoder's LayerNorms use 1e-5 */
} mtg_encoder_hparams;

/* One encoder layer, names of the reference GGUF (src/whisper_encoder.cpp:76-94):
 * the projection and FFN matrices in the weight type, [out][in] rows of GGUF
 * blocks; norms and biases f32. */
typedef struct mtg_encoder_layer {
  const float *attn_ln_w, *attn_ln_b;   /* enc.blk.N.attn_ln.{w,b} [d] */
  const void *q_w, *k_w, *v_w, *o_w;    /* enc.blk.N.attn_{q,k,v,out}.w [d][d] */
  const float *q_b, *v_b, *o_b;         /* their biases [d] (attn_k has none) */
  const float *ffn_ln_w, *ffn_ln_b;     /* enc.blk.N.ffn_ln.{w,b} */
  const void* fc1_w;                    /* enc.blk.N.ffn_1.w [ffn][d] */
  const float* fc1_b;
  const void* fc2_w;                    /* enc.blk.N.ffn_2.w [d][ffn] */
  const float* fc2_b;
} mtg_encoder_layer;

typedef struct mtg_encoder_desc {
  mtg_encoder_hparams hp;
  int32_t weight_type;                  /* of every matrix: MTG_TYPE_Q8_0, _F16, _F32 or _Q4_K */
  const float *conv1_w, *conv1_b;       /* enc.conv1.{w,b}: [d][n_mels][3], [d] */
  const float *conv2_w, *conv2_b;       /* enc.conv2.{w,b}: [d][d][3], [d] (stride 2) */
  const float* pos_embd;                /* enc.pos_embd [rows][d] */
  const float *ln_post_w, *ln_post_b;   /* enc.ln_post.{w,b} */
  const mtg_encoder_layer* layers;
  const void* ad_fc1_w;                 /* adaptor.fc1.w [hidden][d * merge] */
  const float* ad_fc1_b;
  const void* ad_fc2_w;                 /* adaptor.fc2.w [hidden][hidden] */
  const float* ad_fc2_b;
  const float *ad_ln_w, *ad_ln_b;       /* adaptor.ln.{w,b} */
} mtg_encoder_desc;

typedef struct mtg_encoder mtg_encoder;
/* Upload an encoder + adaptor. Weights q8_0 (the converter's q8_0 dtype), f16
 * (its f16 dtype) or q4_K (`cli quantize q4_k`, src/cli.cpp:106-130) in the GGUF
 * block layout; head_dim 64, d_model and hidden 1,024, ffn a multiple of 64
 * (f16: the K of every matrix 1,024, 2,048, 3,072 or 4,096; q4_K: multiples of
 * 256), else MTG_ERR_UNSUPPORTED. */
int mtg_encoder_create(const mtg_encoder_desc* desc, mtg_encoder** out);
void mtg_encoder_destroy(mtg_encoder* e);
const char* mtg_encoder_error(const mtg_encoder* e);
/* WhisperEncoder::encode: mel [n_mels][n_frames] (frames fastest) through the
 * conv stem, the layers and ln_post. The rows stay on the device for
 * mtg_encoder_adapt; out (nullable) receives them, [rows][d]. */
int mtg_encoder_encode(mtg_encoder* e, const float* mel, float* out, int32_t* rows_out);
/* AudioAdaptor::apply on T encoder rows: rows (nullable: the last encode's rows
 * on the device), trimmed to a multiple of merge, merge consecutive rows per
 * adaptor row, fc1 + SiLU, fc2, LayerNorm -> out [N][hidden], N = T / merge. */
int mtg_encoder_adapt(mtg_encoder* e, const float* rows, int32_t T, float* out, int32_t* n_out);
/* device time of the last encode / adapt call, ms (HIP events) */
double mtg_encoder_last_ms(const mtg_encoder* e);
/* The encoder + adaptor tensors of a mapped GGUF file (enc.*, adaptor.*) and the
 * mtd.audio.* keys with read_config's defaults (src/model_loader.cpp:130-144);
 * n_frames = 2 * mtd.audio.max_src_pos. f16 vectors are widened to f32. NULL on
 * failure (mtg_gguf_error). Valid until mtg_gguf_close. */
const mtg_encoder_desc* mtg_gguf_encoder(mtg_gguf* g);
/* mtg_gguf_open + mtg_gguf_encoder + mtg_encoder_create; errors in
 * mtg_gguf_error(NULL). */
int mtg_encoder_create_from_gguf(const char* path, mtg_encoder** out);

/* ---- synthetic model (workload generator for the benchmark and tests) ---- */

typedef struct mtg_synth_model mtg_synth_model;
/* Seeded N(0, std) weights quantized to weight_type, norm gains
 * 1 + gain_jitter * N(0,1). */
int mtg_synth_create(const mtg_hparams* hp, int32_t weight_type, uint64_t seed, float std,
                     float gain_jitter, mtg_synth_model** out);
void mtg_synth_free(mtg_synth_model* m);
const mtg_model_desc* mtg_synth_desc(const mtg_synth_model* m);

/* Standard normal stream shared by the workload generators:
 * out[i] = N(0,1) sample number (first + i) of the stream named by seed. */
void mtg_normal_fill(uint64_t seed, uint64_t first, float* out, size_t n);

/* Weight quantizers of the synthetic model. q8_0: ggml's reference rule as the
 * GGUF converter applies it (d = amax/127 stored f16, codes = roundf(x * 1/d));
 * block = {f16 d, int8 qs[32]}. */
void mtg_quantize_q8_0_weight(const float* x, int64_t k, void* blocks);
void mtg_quantize_q4_k(const float* x, int64_t k, void* blocks);
void mtg_dequantize(int32_t type, const void* blocks, int64_t k, float* out);
size_t mtg_row_bytes(int32_t type, int64_t k);
uint16_t mtg_f32_to_f16(float f);
float mtg_f16_to_f32(uint16_t h);

#ifdef __cplusplus
}
#endif

#endif /* MTG_VERIFY_H */
