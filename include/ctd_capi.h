/*
 * ctd_capi.h -- C entry points of the C++ training layer (libctd.so).
 *
 * A thin handle-based wrapper over ctd::nn::Model + ctd::optim::AdamW that
 * runs the ctd_train step (tools/ctd_train/main.cpp:348-398 of the reference:
 * forward_train_masked -> backward -> clip_grad_norm_ -> AdamW::step ->
 * zero_grad) for harnesses that are not C++ (the Python bench and parity
 * tests).  Every function returns 0 or a negative status; after a failure
 * ctd_last_error() holds the exception text of the C++ layer.
 */
#ifndef CTD_CAPI_H
#define CTD_CAPI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CTD_EXCEPTION (-10)

typedef struct ctd_model_config {
  int32_t vocab_size, hidden_size, intermediate_size, num_layers;
  int32_t num_heads, num_kv_heads, head_dim, qk_norm;
  float rms_norm_eps, rope_theta;
  float rope_factor, rope_low_freq_factor, rope_high_freq_factor;
  int32_t rope_original_max_pos;
} ctd_model_config;

typedef struct ctd_step_times {
  float forward_ms, backward_ms, clip_ms, optimizer_ms, total_ms;
  float loss, grad_norm, mask_sum;
  /* Offloaded AdamW: device time of the most recent finished step's
   * transfers and updates (first copy in to last copy out), which run behind
   * the next step's forward; 0 before one has finished or without offload. */
  float optimizer_stream_ms;
} ctd_step_times;

typedef struct ctd_memory {
  uint64_t allocated, peak_allocated, reserved, peak_reserved, pinned_host;
  uint64_t device_used, device_total; /* hipMemGetInfo now: total - free, total */
  /* Highest hipMemGetInfo total - free since ctd_reset_peak_memory, sampled
   * whenever the allocator obtains a segment and at each train step's phase
   * boundaries; the allocator's segments obtained and cache flushes (segments
   * given back to serve a request); its cap (0: none). */
  uint64_t peak_device_used, device_mallocs, cache_flushes, limit;
} ctd_memory;

/* Statistics of an allocation history replayed on the host (ctd_alloc_replay). */
typedef struct ctd_alloc_replay_stats {
  uint64_t peak_allocated, peak_reserved, reserved_end, segments_obtained, cache_flushes;
} ctd_alloc_replay_stats;

typedef struct ctd_gemm_profile {
  int64_t launches;
  double flops;     /* algorithmic 2*M*N*K summed over launches */
  double total_ms;  /* summed HIP-event durations of those launches */
} ctd_gemm_profile;

typedef void* ctd_trainer_t;

const char* ctd_last_error(void);

/* Presets by name: "smollm2-135m", "smollm2-360m", "qwen3-0.6b", "qwen3-1.7b",
 * "llama3.2-1b" (include/ctd/nn/model.h:39-124 of the reference). */
int ctd_preset_config(const char* name, ctd_model_config* out);

/* Builds a model with seeded synthetic weights on the device: every matrix
 * (and the embedding) ~ N(0, init_std); norm weights = norm_value, or
 * ~ N(0, init_std) when norm_value is NaN.  The parameter list follows
 * Model::collect_parameters. */
int ctd_trainer_create(const ctd_model_config* cfg, uint64_t seed, float init_std,
                       float norm_value, ctd_trainer_t* out);
int ctd_trainer_destroy(ctd_trainer_t t);

int ctd_trainer_num_params(ctd_trainer_t t, int64_t* n);
/* name (NUL-terminated, truncated to cap), numel, decay group (1) or not (0). */
int ctd_trainer_param_info(ctd_trainer_t t, int64_t i, char* name, size_t cap, int64_t* numel,
                           int32_t* decay);
int ctd_trainer_set_param(ctd_trainer_t t, int64_t i, const float* host, int64_t numel);
int ctd_trainer_get_param(ctd_trainer_t t, int64_t i, float* host, int64_t numel);
/* Copies the accumulated gradient; returns -1 if the parameter has none. */
int ctd_trainer_get_grad(ctd_trainer_t t, int64_t i, float* host, int64_t numel);

int ctd_trainer_set_checkpointing(ctd_trainer_t t, int32_t on);
/* Batch: ids/targets int64 [B,T], mask fp32 [B,T] (NULL = all ones), host memory. */
int ctd_trainer_set_batch(ctd_trainer_t t, const int64_t* ids, const int64_t* targets,
                          const float* mask, int64_t B, int64_t T);
/* Synthetic batch generated on the host: ids uniform in [0,V) from `seed`,
 * targets = ids shifted by one, and (masked != 0) a zero prefix of
 * 20-60% of each row (assistant-turn masking). */
int ctd_trainer_synthetic_batch(ctd_trainer_t t, int64_t B, int64_t T, uint64_t seed,
                                int32_t masked);

/* loss = Model::forward_train_masked(...); backward too when `backward`. */
int ctd_trainer_forward_backward(ctd_trainer_t t, int32_t backward, float* loss);
/* Final hidden states before the LM head for the current batch, [B*T*d] floats. */
int ctd_trainer_hidden(ctd_trainer_t t, float* host, int64_t numel);

/* One decoder block in isolation (TransformerBlock::forward_train): x and dy
 * are host [B,T,d]; y = block(x) (wrapped in autograd::checkpoint when
 * `checkpoint`), then y.backward(dy); y_out and dx_out (host, may be NULL)
 * receive y and dL/dx, and the block's parameter grads accumulate. */
int ctd_trainer_block_step(ctd_trainer_t t, int64_t layer, const float* x, const float* dy,
                           int64_t B, int64_t T, int32_t checkpoint, float* y_out, float* dx_out);

int ctd_trainer_make_optimizer(ctd_trainer_t t, float lr, float weight_decay, float beta1,
                               float beta2, float eps, int32_t offload, int64_t chunk_elems);
int ctd_trainer_clip(ctd_trainer_t t, float max_norm, float* total_norm);
int ctd_trainer_opt_step(ctd_trainer_t t);
int ctd_trainer_zero_grad(ctd_trainer_t t);
int ctd_trainer_get_opt_state(ctd_trainer_t t, int64_t i, float* m, float* v, int64_t numel);
int ctd_trainer_step_count(ctd_trainer_t t, int64_t* steps);
/* Offloaded AdamW: waits for the last step() to finish, then reports its
 * device time from its first copy in to its last copy out, the optimizer
 * state it moved per direction (m and v, all of it copied out inside that
 * time), and how much of that state a prefetch during the backward pass had
 * already copied in before step() (zeros without offload).  Any output may
 * be NULL. */
int ctd_trainer_offload_stats(ctd_trainer_t t, double* stream_ms, double* bytes_per_direction,
                              double* prefetched_bytes);
/* Upper bound, in optimizer-state chunks, of what train_step's backward
 * prefetches for the offloaded step (default 32; 0 turns the prefetch off).
 * The staged m/v of the first parameter are device memory held from late in
 * the backward until their copy out. */
/* Per-direction figures of the most recent finished offloaded step
 * (optim::OffloadStats): device ms of the copies in (first to last) and of the
 * copies out with the updates between them, the bytes each moved (m and v
 * together), the prefetched bytes per direction and the bytes per direction
 * left on the host because no parameter in them had a gradient. */
typedef struct ctd_offload_detail {
  double stream_ms, h2d_ms, d2h_ms, h2d_bytes, d2h_bytes, prefetch_bytes, skipped_bytes;
} ctd_offload_detail;
int ctd_trainer_offload_detail(ctd_trainer_t t, ctd_offload_detail* out);

int ctd_trainer_set_prefetch_chunks(ctd_trainer_t t, int64_t chunks);
/* Layer whose re-run in train_step's backward starts that prefetch: a layer
 * index, -1 for none, or -2 (the default) for ctd::train's estimate from the
 * model and batch (include/ctd/train.h, optimizer_prefetch_layer). */
int ctd_trainer_set_prefetch_layer(ctd_trainer_t t, int32_t layer);

/* One full training step (forward, backward, clip to max_norm when > 0,
 * optimizer step, zero_grad) with HIP-event phase times. */
int ctd_trainer_train_step(ctd_trainer_t t, float max_norm, ctd_step_times* times);

int ctd_trainer_synchronize(ctd_trainer_t t);
int ctd_memory_stats(ctd_memory* out);
int ctd_reset_peak_memory(void);
/* Caps the bytes the device allocator holds (0: no cap); see
 * ctd::set_device_memory_limit. */
int ctd_set_device_memory_limit(uint64_t bytes);
/* Gives cached free segments back to the driver (synchronises). */
int ctd_empty_device_cache(void);
/* Allocation history (ctd::start_allocation_history): start, label, stop and
 * write to path. */
int ctd_alloc_history_start(void);
int ctd_alloc_history_mark(const char* label);
int ctd_alloc_history_stop(const char* path);
/* Replays a recorded history on the allocator's placement policy with a
 * host-only backend (no GPU needed); limit as for the device allocator. */
int ctd_alloc_replay(const char* path, uint64_t limit, ctd_alloc_replay_stats* out);

/* Kernel timing: while enabled, every ember_gemm_f32 and fused-attention call
 * launched by the ops layer is bracketed by HIP events on the compute stream;
 * collect resolves them into out[6]: [0..3] GEMMs indexed by 2*transa + transb
 * (one entry per kernel instantiation: NN, NT, TN, TT), [4] attention forward,
 * [5] attention backward (flops: the algorithmic count, no recompute). */
int ctd_gemm_profile_enable(int32_t on);
int ctd_gemm_profile_collect(ctd_gemm_profile* out);

/* Weights (HF names) to `path` and optimizer state to `path`.opt.safetensors
 * (tools/ctd_train/main.cpp:208-234 layout); load restores both. */
int ctd_trainer_save(ctd_trainer_t t, const char* path);
int ctd_trainer_load(ctd_trainer_t t, const char* path);

/* Forward + backward of (loss * scale) into the gradients, which accumulate
 * (ctd_train's micro-batch step, main.cpp:354-365); loss receives the
 * unscaled loss. */
int ctd_trainer_accumulate(ctd_trainer_t t, float scale, float* loss);
/* Learning rate of every group for the next opt_step (AdamW::set_lr). */
int ctd_trainer_set_lr(ctd_trainer_t t, float lr);

/* ---- the ctd_train driver (include/ctd/train.h) */
/* Runs ctd_train with the JSON config at config_path (its directory is the run
 * directory: loss.jsonl, checkpoints). */
int ctd_train_run(const char* config_path);
/* Learning rate of a step: linear warmup, then cosine to lr * min_lr_ratio. */
int ctd_train_lr_at_step(int32_t step, int32_t warmup_steps, int32_t total_steps, float lr,
                         float min_lr_ratio, float* out);
/* Loads a split (int32 tokens, int8 mask; seq_len per document) and assembles
 * the batch of the B documents `docs` into host buffers of B*(seq_len-1)
 * entries; num_docs receives the split size.  B = 0 only loads. */
int ctd_train_host_batch(const char* tok_path, const char* mask_path, int32_t seq_len,
                         const int64_t* docs, int64_t B, int64_t* ids, int64_t* targets,
                         float* mask, float* sum_mask, int64_t* num_docs);
/* One loss.jsonl line (val != 0: a validation record) into buf. */
int ctd_train_event_json(int32_t step, float loss, float lr, float grad_norm,
                         double tokens_per_sec, double wall_s, int32_t val, char* buf,
                         size_t cap);

/* ---- inference (include/ctd/nn/kv_cache.h, Model::forward with a cache,
 * include/ctd/sampling.h) */
typedef void* ctd_kvcache_t;
/* A zero-filled KV cache for the trainer's model: batch x max_seq rows. */
int ctd_kvcache_create(ctd_trainer_t t, int64_t batch, int64_t max_seq, ctd_kvcache_t* out);
int ctd_kvcache_destroy(ctd_kvcache_t c);
int ctd_kvcache_len(ctd_kvcache_t c, int64_t* current_len);
/* Model::forward(ids [B,T] host int64, cache (NULL: none), position_start)
 * -> logits [B,T,V] into host memory; last_only: forward_last_logits, [B,1,V]. */
int ctd_trainer_forward_cached(ctd_trainer_t t, ctd_kvcache_t cache, const int64_t* ids,
                               int64_t B, int64_t T, int32_t position_start, int32_t last_only,
                               float* logits, int64_t numel);
/* ctd::sample over host logits [B,V] (copied to the device first when
 * on_device), `draws` times in a row from one mt19937_64(seed):
 * out[d*B + b] is draw d of row b. */
int ctd_sample(const float* logits, int64_t B, int64_t V, float temperature, int32_t top_k,
               float top_p, uint64_t seed, int32_t draws, int32_t on_device, int64_t* out);

/* The generation loop of ctd_generate (ctd::generate::generate_loop) on the
 * trainer's model, batch 1: prefill of prompt[P], then max_new tokens, each
 * sampled from the last logits and fed back through the KV cache (max_seq
 * rows).  tokens[max_new] receives them; prefill_ms / decode_ms are host wall
 * times (prompt in to first token known; the token loop). */
int ctd_trainer_generate(ctd_trainer_t t, const int64_t* prompt, int64_t P, int32_t max_new,
                         float temperature, int32_t top_k, float top_p, uint64_t seed,
                         int64_t max_seq, int64_t* tokens, double* prefill_ms,
                         double* decode_ms);

/* Rows per chunk of the fused LM head + loss (ops::set_linear_cross_entropy_chunk_rows;
 * 0 = automatic). */
int ctd_set_head_chunk_rows(int64_t rows);
/* Whether the fused LM head + loss skips rows whose mask value is 0
 * (ops::set_linear_cross_entropy_active_rows; default 1). */
int ctd_set_head_active_rows(int32_t on);

/* Device bytes the attention backward may keep dS in
 * (ops::set_attention_backward_ds_bytes; -1 = default, 0 = recompute). */
int ctd_set_attn_ds_bytes(int64_t bytes);
/* Whether a recorded attention forward keeps its scores for its backward
 * (ops::set_attention_keep_scores; default 0). */
int ctd_set_attn_keep_scores(int32_t on);

#ifdef __cplusplus
}
#endif
#endif /* CTD_CAPI_H */
