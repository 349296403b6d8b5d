/*
 * daiza_hip.h — C ABI of the MI355X (gfx950) batch-1 Q1_0 decode library.
 *
 * Every entry point returns int: DZ_OK (0) or a negative status.  The negative
 * values map onto the reference's error enum BonsaiError (Daiza-engine/src/lib.rs:42-78):
 *   DZ_ERR_TENSOR      -> BonsaiError::Tensor       (shape / layout violations)
 *   DZ_ERR_MODEL       -> BonsaiError::Model        (bad config, missing tensor)
 *   DZ_ERR_UNSUPPORTED -> BonsaiError::Unsupported  (shapes this build does not implement)
 *   DZ_ERR_DEVICE      -> device/runtime failure (HIP error, no gfx950 device)
 * dz_last_error() returns a thread-local message for the last failure.
 *
 * Ownership: the library owns device memory and handles.  Host pointers passed in
 * are borrowed for the duration of the call; host outputs are written before the
 * call returns (the reference reads ctx.logits_buf right after forward_single_token).
 * A context owns one HIP stream and is not thread safe, the same contract as the
 * reference's `&mut ForwardContext`.  No C++ exception crosses this boundary.
 */
#ifndef DAIZA_HIP_H
#define DAIZA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DZ_OK 0
#define DZ_ERR_TENSOR (-1)
#define DZ_ERR_MODEL (-2)
#define DZ_ERR_UNSUPPORTED (-3)
#define DZ_ERR_DEVICE (-4)

/*
 * Model hyper-parameters.  Field meaning follows Config (Daiza-engine/src/model/config.rs:12-76);
 * Bonsai-27B values in comments.  Layer i is full attention when (i+1) % full_attn_interval == 0
 * (config.rs:161-167).
 */
typedef struct dz_config {
  int32_t n_layers;            /* 64      block_count */
  int32_t hidden;              /* 5120    embedding_length */
  int32_t ffn;                 /* 17408   feed_forward_length */
  int32_t vocab;               /* 248320 */
  int32_t n_head;              /* 24      attention.head_count */
  int32_t n_head_kv;           /* 4       attention.head_count_kv */
  int32_t head_dim;            /* 256     attention.key_length (this build: 256) */
  int32_t rope_dim;            /* 64      rope.dimension_count */
  float rope_base;             /* 1e7     rope.freq_base */
  float rms_eps;               /* 1e-6    attention.layer_norm_rms_epsilon */
  int32_t full_attn_interval;  /* 4 */
  int32_t ssm_conv_kernel;     /* 4       (this build: 4) */
  int32_t ssm_state;           /* 128     ssm.state_size = head_k_dim = head_v_dim (this build: 128) */
  int32_t ssm_k_heads;         /* 16      ssm.group_count */
  int32_t ssm_v_heads;         /* 48      ssm.time_step_rank */
  int32_t embd_f16;            /* 1: f16 token embedding; 0: Q1_0 (reference GGUF) */
  int32_t max_ctx;             /* KV-cache capacity in tokens */
} dz_config;

/* Fills cfg with the Bonsai-27B shape (Config::default, config.rs:47-76) and max_ctx. */
void dz_config_bonsai27b(dz_config* cfg, int32_t max_ctx);

const char* dz_last_error(void);

/* Selects the HIP device for subsequent calls on this thread; fails unless it is gfx950. */
int dz_device_init(int device);

/* ===================== matrix level: Q1_0Matrix (weights.rs:83-1208) ===================== */

typedef struct dz_mat dz_mat;

/*
 * Uploads one Q1_0 matrix given in the reference's AoS block layout
 * (Q1_0Matrix::bytes, weights.rs:83-102; 18 bytes per 128 weights, row r at r*(cols/128)*18).
 * cols must be a multiple of 128.  The device copy is repacked into the GEMV's layout;
 * the bytes themselves are unchanged (dz_q1_0_dequant_rows recovers them bit-exactly).
 * Replaces Q1_0Matrix::from_gguf (weights.rs:90-102).
 */
int dz_q1_0_upload(const uint8_t* aos, size_t rows, size_t cols, dz_mat** out);
int dz_q1_0_free(dz_mat* m);
int dz_q1_0_shape(const dz_mat* m, size_t* rows, size_t* cols);

/* y = W x (accumulate = 0) or y += W x (accumulate = 1); host x[cols], y[rows].
 * Replaces matvec_into_slice (weights.rs:123-325) and matvec_add_into_slice (weights.rs:334-465). */
int dz_q1_0_matvec(dz_mat* m, const float* x, float* y, int accumulate);

/* Several matrices sharing x and cols, one device pass (n <= 8).
 * Replaces matvec_multi_into_slice (weights.rs:831-972). */
int dz_q1_0_matvec_multi(dz_mat* const* mats, int n, const float* x, float* const* ys);

/* n columns at once: y[i] = W x[i] (accumulate = 0) or y[i] += W x[i] for i < n; host x[n][cols],
 * y[n][rows].  Runs on the matrix cores with the activations split into three f16 parts (33
 * significant bits: f32 width) and exact ±scale weights, so it agrees with an f32 dot product to
 * within f32 accumulation order.  Replaces matvec_batch_into_slice / matvec_add_batch_into_slice
 * (weights.rs:475-682, 976-980). */
int dz_q1_0_matvec_batch(dz_mat* m, const float* x, int n, float* y, int accumulate);

/* Same as dz_q1_0_matvec on device pointers, enqueued on `stream` (a hipStream_t, NULL = default),
 * without a host synchronisation.  The token loop uses the fused kernels instead.
 * Calls on different streams run one after another on the device, in the order they were made
 * (the one-launch product shares one buffer of split-K partials and needs its whole grid resident);
 * the first call that comes on a second stream waits on the host for the device to drain, later
 * stream changes wait on the device.  A launch whose bounded wait for
 * those partials gives up leaves NaN in the rows it could not form and is reported as
 * DZ_ERR_DEVICE by dz_q1_0_matvec_dev_status (or by the next synchronous dz_q1_0_matvec*). */
int dz_q1_0_matvec_dev(dz_mat* m, const float* x_dev, float* y_dev, int accumulate, void* stream);

/* Synchronises `stream` (NULL = the library's) and every dz_q1_0_matvec_dev launch made before,
 * and returns DZ_ERR_DEVICE if any of them gave up on a wait since the last check, else DZ_OK.
 * No counterpart in the reference, whose matvec is synchronous: the status of the asynchronous
 * form above. */
int dz_q1_0_matvec_dev_status(void* stream);

/* dz_q1_0_matvec_dev that allocates nothing, for callers that cannot call hipMalloc (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation); no counterpart in the
 * reference.  The split-K partial sums go to a fixed per-device workspace of
 * dz_q1_0_noalloc_max_partials() floats (16 MiB, held until the process ends): a matrix needs
 * ceil(cols/512) * (rows rounded up to 64) of them, and a larger one is refused with
 * DZ_ERR_UNSUPPORTED.  dz_device_init must have run.  Every call on a device shares its workspace,
 * so calls that overlap on one device (several streams or threads) race. */
int dz_q1_0_matvec_dev_noalloc(dz_mat* m, const float* x_dev, float* y_dev, int accumulate, void* stream);
size_t dz_q1_0_noalloc_max_partials(void);

/* Split-K form on device pointers: writes part_dev[t][r] for K tiles t = 0..ceil(cols/512)-1 and
 * rows r < dz_q1_0_partials_ld(m) (row count padded to 64), so that y[r] = sum_t part[t][r] in
 * tile order.  For callers that fuse the tile sum into their next kernel, as the token loop does
 * for every projection; y = W x of matvec_into_slice (weights.rs:123-325) without the final sum. */
int dz_q1_0_gemv_partials(dz_mat* m, const float* x_dev, float* part_dev, void* stream);
size_t dz_q1_0_partials_ld(const dz_mat* m);
int dz_q1_0_ntiles(const dz_mat* m);

/* Dequantised rows [r0, r0+n) as f32, w = (bit*2 - 1) * f16_to_f32(scale) with the reference's
 * f16_to_f32 (quant.rs:39-74) bit for bit, including its handling of subnormal scales.
 * Replaces dequantize_q1_0_row_into (quant.rs:161-194) / row_into_slice (weights.rs:106). */
int dz_q1_0_dequant_rows(dz_mat* m, size_t r0, size_t n, float* out);

/* ===================== model level: forward_single_token / forward_batch ===================== */

typedef struct dz_model dz_model;
typedef struct dz_ctx dz_ctx;

/* One named host tensor, GGUF naming (LoadedWeights::load_all, weights.rs:1308-1379):
 *   "token_embd.weight" (Q1_0, or F16 when cfg.embd_f16), "output_norm.weight" (F32),
 *   "output.weight" (Q1_0), "blk.N.<name>" per layer.
 * type: 0 = F32, 1 = F16, 41 = Q1_0 (GGUF TensorType, gguf/tensor_info.rs:41,66).
 * ssm_conv1d.weight is given as in GGUF, [qkv_dim][conv_kernel] (the reference transposes at load). */
typedef struct dz_tensor {
  const char* name;
  int32_t type;
  const void* data;
  size_t n_bytes;
} dz_tensor;

int dz_model_create(const dz_config* cfg, const dz_tensor* tensors, int n_tensors, dz_model** out);

/* ---- GGUF files (Daiza-engine/src/gguf) ----
 * dz_gguf_open: GgufFile::open (gguf/parser.rs:40-119): maps the file read-only and parses the v3
 * header, the metadata table (metadata.rs) and the tensor table (tensor_info.rs:41-201; dims in GGUF
 * order, dims[0] = columns; Q1_0 is type 41); the data section starts at the next multiple of
 * general.alignment (default 32).  The tensors stay slices of the mapping until dz_gguf_close.
 * dz_gguf_tensor_info: *offset is the absolute file offset of the data, *n_bytes 0 for a type this
 * path does not use (only F32, F16, BF16 and Q1_0 are sized).  dz_gguf_tensor_data: the data in
 * the mapping, or NULL. */
typedef struct dz_gguf dz_gguf;
int dz_gguf_open(const char* path, dz_gguf** out);
int dz_gguf_close(dz_gguf* g);
int dz_gguf_n_tensors(const dz_gguf* g);
int dz_gguf_tensor_info(const dz_gguf* g, int i, const char** name, int32_t* type, int32_t* n_dims, uint64_t* dims,
                        uint64_t* offset, uint64_t* n_bytes);
const void* dz_gguf_tensor_data(const dz_gguf* g, int i);
/* Config::from_metadata (model/config.rs:76-160): the Bonsai-27B defaults overridden by every
 * qwen35.* key present (architecture must be "qwen35"); embd_f16 from token_embd.weight's type;
 * *eos_token_id (may be NULL) from tokenizer.ggml.eos_token_id (default 248046). */
int dz_gguf_config(const dz_gguf* g, int32_t max_ctx, dz_config* cfg, int32_t* eos_token_id);
/* Config::context_length (model/config.rs:52, 92-93): qwen35.context_length when stored as a 64-bit
 * integer (Metadata::get_u64), else 262144.  Sizes nothing here; the DZSS cfg_hash includes it. */
int dz_gguf_context_length(const dz_gguf* g, uint64_t* out);
/* LoadedWeights::load_all (model/weights.rs:1308-1379): the file's tensors by name through
 * dz_model_create (the file stays open only for the call). */
int dz_model_create_gguf(const dz_gguf* g, const dz_config* cfg, dz_model** out);

/* Synthetic model with the generator of daiza_synth.h (BASELINE.json config 4 when cfg is Bonsai-27B). */
int dz_model_create_synth(const dz_config* cfg, uint64_t seed, dz_model** out);
int dz_model_free(dz_model* m);
int dz_model_weight_bytes(const dz_model* m, uint64_t* q1_bytes);

/* Context = ModelState + ForwardContext (forward.rs:32-131): KV caches, SSM states, position.
 * If a forward fails with DZ_ERR_DEVICE because a device-side wait gave up, the launch may have
 * updated part of the state; the context then refuses every forward with DZ_ERR_DEVICE until
 * dz_ctx_reset.  (The reference's forward cannot fail part-way; this has no counterpart there.) */
int dz_ctx_create(dz_model* m, dz_ctx** out);
int dz_ctx_free(dz_ctx* c);
int dz_ctx_reset(dz_ctx* c);          /* ModelState::reset (forward.rs:66-76) */
int dz_ctx_pos(const dz_ctx* c);      /* ModelState::pos */

/*
 * One token: embed -> 64 blocks -> output norm -> lm_head -> pos += 1.
 * logits_or_null receives vocab f32 values (ctx.logits_buf); argmax_or_null receives the greedy
 * token (lowest index among equal maxima, simd_exp.rs:551-598).
 * Replaces forward_single_token (forward.rs:204-375).
 */
int dz_forward_token(dz_ctx* c, uint32_t token, float* logits_or_null, uint32_t* argmax_or_null);

/*
 * n tokens at positions start_pos.. (start_pos must equal the context position).
 * Last-position logits to last_logits_or_null; per-position logits [n][vocab] to
 * per_pos_logits_or_null.  Replaces forward_batch (forward.rs:394-1407).
 */
int dz_forward_batch(dz_ctx* c, const uint32_t* ids, int n, int start_pos,
                     float* last_logits_or_null, float* per_pos_logits_or_null);

/*
 * Greedy decode of n tokens entirely on the device: the first forward consumes `first_token`,
 * each next input is the argmax of the previous logits.  out_tokens[i] = argmax after forward i.
 * Mirrors the greedy loop of Engine::generate_inner (engine.rs:850-871) without the EOS stop.
 */
int dz_decode_greedy(dz_ctx* c, uint32_t first_token, int n, uint32_t* out_tokens);

/*
 * The greedy loop of Engine::generate_inner (engine.rs:850-871) with its EOS stop: like
 * dz_decode_greedy, but a pick equal to eos_id (>= 0; Config::eos_token_id, config.rs:69, is 248046)
 * ends the loop before that token is forwarded.  *n_forwarded receives the number of forwards run
 * (0 when first_token is eos_id); out_tokens[i] (i < *n_forwarded) is the pick after forward i, so the
 * loop stopped on EOS exactly when out_tokens[*n_forwarded - 1] == eos_id.  The position advances by
 * *n_forwarded and the context's logits are those of the last forward.
 */
int dz_decode_greedy_eos(dz_ctx* c, uint32_t first_token, int n, int32_t eos_id, uint32_t* out_tokens,
                         int* n_forwarded);

/* Last computed logits (vocab f32) of the context. */
int dz_ctx_logits(dz_ctx* c, float* logits);
/* Vocabulary size of the context's model (the length of a logits row). */
int dz_ctx_vocab(const dz_ctx* c, int* vocab);

/* ---- speculative verify ----
 * The reference verifies drafts one forward_single_token at a time and forwards only accepted
 * ones (engine.rs:1255-1470); here the k drafts run in one n-token forward and the accepted
 * prefix is kept afterwards.
 *
 * dz_verify_forward: forward of draft[0..k) at positions pos .. pos+k-1 (forward_batch with
 * per_pos_logits, forward.rs:1319-1337).  per_pos_logits_or_null[i] (k rows of vocab) = logits after
 * draft[i].  The DeltaNet states and conv rings are left unchanged and per-token rollback records
 * are kept; the position does not move.
 * dz_verify_commit: keeps the first n_accept drafts (0..k) exactly as if only they had been
 * forwarded (DeltaNet updates replayed in the scan's order, conv rings, KV length via the position
 * as KvCache::truncate does, kv_cache.rs:119-130; the context's logits = after draft n_accept-1).
 * Any other forward, reset, set_pos or truncate discards a pending verify. */
int dz_verify_forward(dz_ctx* c, const uint32_t* draft, int k, float* per_pos_logits_or_null);
int dz_verify_commit(dz_ctx* c, int n_accept);

/* SamplingParams (sampling.rs:22-32) without the repetition penalties, which the verify path does
 * not apply by default (engine.rs:1332). */
typedef struct dz_sampling {
  float temperature;  /* <= 0: greedy */
  int32_t top_k;
  float top_p;
} dz_sampling;

/* LcgRng::next_f32 (sampling.rs:14-18); *state is the generator state (seeded e.g. 0xC0FFEE). */
float dz_lcg_next(uint64_t* state);
/*
 * Sampled decode of n tokens: the first forward consumes first_token, each next input is
 * sample_top_k_top_p_into (sampling.rs:144-247) of the previous logits with *sp and the generator
 * *rng_state (advanced by one draw per token, as LcgRng::next_f32); out_tokens[i] = the sample
 * after forward i.  Mirrors the decode loop of Engine::generate_inner (engine.rs:850-862) without
 * its EOS stop and with penalties off.  On the token kernel the top-k, the softmax over it, the
 * top-p cut and the draw run on the device with no host round trip per token: for top_k <= 32
 * inside the one token-kernel launch of the call, for top_k <= 64 in kernels between per-token
 * launches (also with DAIZA_PTK_SAMPLE=0); a larger top_k, or the graph path, samples on the host
 * from each forward's logits.  Candidates are ranked by logit, the lowest index first among equal
 * values.  temperature <= 0 is dz_decode_greedy (no draw).
 */
int dz_decode_sample(dz_ctx* c, uint32_t first_token, int n, const dz_sampling* sp, uint64_t* rng_state,
                     uint32_t* out_tokens);
/* sample_top_k_top_p_into (sampling.rs:144-247) over logits[n]. */
int dz_sample(const float* logits, int n, const dz_sampling* params, uint64_t* rng_state, uint32_t* out);
/* leviathan_check (engine.rs:1791-1819): greedy = argmax(target) == token; else accept iff
 * u < p[token]/q[token] of the untempered softmaxes (softmax_pair_single_avx2, simd_exp.rs:656-767). */
int dz_leviathan_check(const float* target, const float* draft, int n, uint32_t token, const dz_sampling* params,
                       uint64_t* rng_state, int* accepted);
/* sample_bonus (engine.rs:1833-1866): sample from norm(max(0, p - q)) (residual_max_zero_sum_avx2,
 * simd_exp.rs:605-642), or from the target when the residual has no mass. */
int dz_sample_bonus(const float* target, const float* draft, int n, const dz_sampling* params, uint64_t* rng_state,
                    uint32_t* out);
/*
 * One speculative step: verify draft[0..k) against the context (its logits predict draft[0]) with
 * Leviathan acceptance in order, then keep the accepted prefix.  On the first rejection the bonus
 * is sample_bonus of that position's target and draft logits (greedy: the target's argmax); with
 * every draft accepted it is sampled from the logits after the last draft.  An accepted eos_id
 * (>= 0) ends the step unforwarded with *bonus = 0xFFFFFFFF, as the reference stops there.  The
 * bonus is not forwarded (the caller's next forward takes it, as the reference's Phase 3 does).
 * draft_logits: [k][vocab] (may be NULL when greedy).  Random draws follow the reference's order:
 * one per verified draft, one for the bonus.
 */
int dz_spec_verify(dz_ctx* c, const uint32_t* draft, int k, const float* draft_logits, const dz_sampling* params,
                   int32_t eos_id, uint64_t* rng_state, int* n_accepted, uint32_t* bonus);

/* ---- state access (ModelState fields; layouts are the reference's) ---- */
/* SSM layer state S[v_heads][128 (v index i)][128 (k index j)] (cache/ssm_state.rs:10-39) and
 * the conv ring hist[conv_kernel][qkv_dim] with its head index (oldest row). */
int dz_ctx_set_ssm_state(dz_ctx* c, int layer, const float* state, const float* conv_hist, int conv_head);
int dz_ctx_get_ssm_state(dz_ctx* c, int layer, float* state, float* conv_hist, int* conv_head);
/* KV cache of an attention layer, per-kvh [len][head_dim] (cache/kv_cache.rs:17-130). */
int dz_ctx_set_kv(dz_ctx* c, int layer, const float* k, const float* v, int len);
int dz_ctx_get_kv(dz_ctx* c, int layer, float* k, float* v, int len);
int dz_ctx_kv_len(dz_ctx* c, int layer);
int dz_kv_truncate(dz_ctx* c, int len);                    /* KvCache::truncate (kv_cache.rs:119-130) */
int dz_ctx_set_pos(dz_ctx* c, int pos);

/*
 * One mixer step of one layer on host h[hidden]: h += mixer(rmsnorm(h)), where mixer is the
 * Gated DeltaNet (ssm_forward_into, ssm.rs:425-616) or gated attention
 * (attention_forward_into, attention.rs:56-208); uses and advances that layer's state at the
 * context position (BASELINE configs 2 and 3).
 */
int dz_ctx_mixer_step(dz_ctx* c, int layer, float* h);

/* dz_ctx_mixer_step on device vectors h_dev[hidden] -> h_out_dev[hidden] (may be the same buffer),
 * enqueued on the context's stream without a host synchronisation (for timing one layer-step with
 * the weights, state and input resident in HBM).  Advances the position like dz_ctx_mixer_step. */
int dz_ctx_mixer_step_dev(dz_ctx* c, int layer, const float* h_dev, float* h_out_dev);

/* ---- session snapshots: DZSS v1 (Daiza-runtime/src/session_persist.rs:47-312) ----
 * dz_ctx_save writes the context's state as Session::save_to_disk does: a 128-byte header ("DZSS",
 * version 1, cfg_hash, pos, history length, block count, think flag, system-prompt flag), the history
 * tokens, then per layer the KV cache (kind 0: per_token, len, K and V as [seq][kv head][dim]) or the
 * DeltaNet state (kind 1: S[v head][i][j], the conv ring [conv_kernel][qkv_dim], conv_head), then the
 * system prompt if one is given.  History, think flag and system prompt belong to the reference's
 * Session, not to the context: the caller passes them (system_prompt NULL = none).
 * dz_ctx_load checks magic, version, cfg_hash and block count, reads the whole file, and only then
 * replaces the context's state (reset, position, every layer), so a refused file leaves the context
 * as it was; a successful load also clears a failed launch's refusal.  history / system_prompt may be
 * NULL; with a buffer too small (history_cap tokens, prompt_cap bytes including the terminating 0)
 * it fails with DZ_ERR_TENSOR before touching the context.
 * context_length is Config::context_length (262144 for Bonsai-27B, qwen35.context_length), one of
 * the fields of the reference's cfg_hash; dz_session_cfg_hash is that hash (Rust's DefaultHasher,
 * SipHash-1-3 with zero keys, over block_count, hidden, head_count, head_count_kv, head_dim,
 * full_attention_interval, ssm_state_size, ssm_time_step_rank, ssm_conv_kernel, context_length). */
uint64_t dz_session_cfg_hash(const dz_config* cfg, uint64_t context_length);
int dz_ctx_save(dz_ctx* c, const char* path, uint64_t context_length, const uint32_t* history, uint64_t n_history,
                int32_t think_enabled, const char* system_prompt);
int dz_ctx_load(dz_ctx* c, const char* path, uint64_t context_length, uint32_t* history, uint64_t history_cap,
                uint64_t* n_history, int32_t* think_enabled, char* system_prompt, uint64_t prompt_cap,
                uint64_t* prompt_len);

/*
 * ModelState::clone (Daiza-engine/src/model/forward.rs:31-77, derive(Clone); the reference clones it
 * for Session::save_to_disk_async, Daiza-runtime/src/session_persist.rs:153-186) between contexts:
 * dst takes src's position, DeltaNet states, conv rings, cached K/V rows [0, pos), token log and the
 * last forward's logits; src is unchanged.  This is the checkpoint/restore of a context: copy into a
 * spare context of the same model to checkpoint, copy back to restore.  The models must have the same
 * shape (DZ_ERR_MODEL otherwise); src's position must fit dst's max_ctx (DZ_ERR_TENSOR).  A pending
 * dz_verify_forward on dst is dropped; src's refusal after a failed launch is copied with its state.
 */
int dz_ctx_copy_state(dz_ctx* dst, const dz_ctx* src);

/* The context's HIP stream (hipStream_t), for callers that time or order work around it. */
void* dz_ctx_stream(dz_ctx* c);

/*
 * 1 if this context's forwards (dz_forward_token / dz_forward_batch / dz_decode_greedy) run in the
 * persistent token kernel (one launch per call, the default for the shapes it covers),
 * 0 if they replay the per-kernel token graph.  Setting DAIZA_PTK=0 in the environment before
 * dz_ctx_create selects the graph.  Diagnostic only; it has no counterpart in the reference.
 */
int dz_ctx_token_kernel(const dz_ctx* c);

#ifdef __cplusplus
}
#endif
#endif /* DAIZA_HIP_H */
