/*
 * paged_infer_amd.h -- C ABI of the MI355X-native int8 projection + paged-attention path.
 *
 * Drop-in boundary for Paged-Infer's three seams (reference = Rohanr14/Paged-Infer):
 *   1. kernel tier  : src/math.rs (quantize_rows_i8, matvec/matmat int8), src/attention.rs
 *                     (PagedAttention::run), src/memory/layout.rs (KvLayout::copy_block)
 *   2. memory tier  : src/memory/{allocator,block_table,prefix_cache,kv_cache_manager}.rs
 *   3. model tier   : src/model.rs (LlamaWeights::decode_batch_into / prefill_batched)
 * and the GPU plugin seam of src/model.rs:296-353 + src/gpu.rs (GpuForwardContext /
 * GpuLinear), which in the reference refuses int8 weights.
 *
 * Conventions (all entry points):
 *   - Plain pointers and sizes only; no torch or HIP types. Streams are passed as `void*`
 *     (a hipStream_t; NULL = the context's own stream).
 *   - Every function returns pia_status; the reference panics on a shape mismatch, this ABI
 *     returns PIA_ERR_INVALID and leaves a message in pia_last_error().
 *   - "_dev" functions take device pointers and are asynchronous on the given stream;
 *     functions without the suffix take host pointers and are synchronous (the reference's
 *     semantics: GpuLinear::apply blocks on readback, src/gpu.rs:234-276).
 *   - The context owns device weights and the device KV cache; callers own every other buffer.
 *   - Single-threaded callers, like the reference's Engine (src/engine.rs:485).
 */
#ifndef PAGED_INFER_AMD_H
#define PAGED_INFER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t pia_status;
enum {
  PIA_OK = 0,
  PIA_ERR_INVALID = 1,   /* shape / argument error (the reference asserts) */
  PIA_ERR_HIP = 2,       /* a HIP runtime call failed */
  PIA_ERR_OOM = 3,       /* device allocation failed */
  PIA_ERR_NO_DEVICE = 4, /* no usable gfx950 device */
};

/* Message for the last non-OK status returned on this thread. */
const char* pia_last_error(void);
/* Library version string. */
const char* pia_version(void);

/* ------------------------------------------------------------------------------------ */
/* Context: one device + one stream (replaces GpuContext, src/gpu.rs:40-148).            */
/* ------------------------------------------------------------------------------------ */
typedef struct pia_context pia_context;

pia_status pia_context_create(int device, pia_context** out);
pia_status pia_context_destroy(pia_context* ctx);
pia_status pia_context_synchronize(pia_context* ctx);
/* The context's stream as a hipStream_t. */
void* pia_context_stream(pia_context* ctx);

/* Device memory helpers for callers that have no HIP runtime of their own. */
pia_status pia_malloc(pia_context* ctx, size_t bytes, void** dptr);
pia_status pia_free(pia_context* ctx, void* dptr);
pia_status pia_memcpy_h2d(pia_context* ctx, void* dst, const void* src, size_t bytes);
pia_status pia_memcpy_d2h(pia_context* ctx, void* dst, const void* src, size_t bytes);

/* ------------------------------------------------------------------------------------ */
/* Kernel tier.                                                                           */
/* ------------------------------------------------------------------------------------ */

/* quantize_rows_i8 (src/math.rs:456-469), on the host. Per row: scale = max|w|/127 (1.0 for
 * an all-zero row), q = clamp(round_half_away(w/scale), -127, 127). Bit-exact. */
pia_status pia_quantize_rows_i8(const float* w, int64_t rows, int64_t cols, int8_t* q, float* scales);

/* The same quantizer on the device, bit-exact with the host one (IEEE divide, roundf). */
pia_status pia_quantize_rows_i8_dev(pia_context* ctx, const float* w, int64_t rows, int64_t cols, int8_t* q,
                                    float* scales, void* stream);

/* matvec_i8_weight_parallel (src/math.rs:473-512): out[r] = dot(W[r,:], x) * scales[r].
 * W is row-major [rows][cols] int8. */
pia_status pia_matvec_i8(pia_context* ctx, float* out, const float* x, const int8_t* w, const float* scales,
                         int64_t rows, int64_t cols);
pia_status pia_matvec_i8_dev(pia_context* ctx, float* out, const float* x, const int8_t* w, const float* scales,
                             int64_t rows, int64_t cols, void* stream);

/* matmat_i8_weight_parallel (src/math.rs:223-275): out_rb[r][b] = dot(W[r], x_br[b]) * s[r].
 * Output is [row][batch], as in the reference (the caller transposes). From 5 batch rows, when
 * cols is a multiple of 64 and the pointers are 16-byte aligned, the matmat and apply forms run on
 * the int8 matrix cores (activations as three 8-bit digits of a 23-bit fixed-point image per row,
 * exact integer accumulation; |error| <= 2^-23 * 2^e * sum|w| * scale per output, max|x_b| < 2^e)
 * with the digits in the context's workspace: calls on one context must not overlap. */
pia_status pia_matmat_i8(pia_context* ctx, float* out_rb, const float* x_br, const int8_t* w, const float* scales,
                         int64_t batch, int64_t rows, int64_t cols);
pia_status pia_matmat_i8_dev(pia_context* ctx, float* out_rb, const float* x_br, const int8_t* w,
                             const float* scales, int64_t batch, int64_t rows, int64_t cols, void* stream);

/* Projection::apply_batched for Int8 (src/model.rs:247-259): out_br[b][r], i.e. matmat
 * followed by transpose_rb_to_br, fused. */
pia_status pia_qlinear_apply_dev(pia_context* ctx, float* out_br, const float* x_br, const int8_t* w,
                                 const float* scales, int64_t batch, int64_t rows, int64_t cols, void* stream);
/* Host-pointer form of the above (same reference function), synchronous. */
pia_status pia_qlinear_apply(pia_context* ctx, float* out_br, const float* x_br, const int8_t* w,
                             const float* scales, int64_t batch, int64_t rows, int64_t cols);
/* No counterpart in the reference: pia_qlinear_apply_dev for callers that cannot allocate
 * device memory (graph capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * kernels and results; the matrix-core path's scratch (activation digits, split-K partials) is a
 * fixed per-device array set up when a context is created, so it allocates nothing. Limits:
 * batch <= 64, cols <= 16384 (PIA_ERR_INVALID beyond). Calls on one GPU share that scratch:
 * overlapping calls on one device race (order them on one stream). */
pia_status pia_qlinear_apply_noalloc_dev(pia_context* ctx, float* out_br, const float* x_br, const int8_t* w,
                                         const float* scales, int64_t batch, int64_t rows, int64_t cols,
                                         void* stream);

/* KV cache layout (src/memory/layout.rs:17-78): f32
 * [num_layers][num_blocks][block_size][num_kv_heads][k|v][head_dim]. */
typedef struct pia_kv_layout {
  int64_t num_layers, num_blocks, block_size, num_kv_heads, head_dim;
} pia_kv_layout;

/* One attention entry (AttnEntry, src/attention.rs:59-85): attends to start..=pos. Its
 * logical->physical block map is tables[table_off .. table_off + table_len); logical blocks
 * at or past table_len are unmapped and masked to -inf. */
typedef struct pia_attn_entry {
  int32_t pos, start, table_off, table_len;
} pia_attn_entry;

/* PagedAttention::run (src/attention.rs:141-264) for one layer: q/out [n][num_heads][head_dim],
 * kv read-only and already holding this step's K/V. `entries` and `tables` are device
 * arrays. Requires num_heads % num_kv_heads == 0 (the reference asserts the same). */
pia_status pia_paged_attention_dev(pia_context* ctx, float* out, const float* q, const float* kv,
                                   const pia_kv_layout* layout, int64_t num_heads, const pia_attn_entry* entries,
                                   const int32_t* tables, int64_t n, int64_t layer, void* stream);

/* The per-step KV write of run_layers_batch (src/model.rs:1093-1107; single-sequence form
 * :868-878): k/v [n][num_kv_heads][head_dim] (post-RoPE K, V) stored at each entry's pos, found
 * through its block table as get_physical_location does; unmapped positions are skipped. Only
 * pos, table_off and table_len of each entry are read. Block ids are checked against the cache
 * on the host (the entries and the used table range are read back). */
pia_status pia_kv_write_dev(pia_context* ctx, float* kv, const pia_kv_layout* layout, const float* k, const float* v,
                           const pia_attn_entry* entries, const int32_t* tables, int64_t n, int64_t layer,
                           void* stream);

/* KvLayout::copy_block (src/memory/layout.rs:82-96): copy one physical block, all layers. */
pia_status pia_kv_copy_block_dev(pia_context* ctx, float* kv, const pia_kv_layout* layout, int64_t src,
                                 int64_t dst, void* stream);

/* sampling::argmax (src/sampling.rs:140-147) per row of logits [n][vocab]; f32 total order,
 * the last maximal index wins ties. */
pia_status pia_argmax_dev(pia_context* ctx, int32_t* out, const float* logits, int64_t n, int64_t vocab,
                          void* stream);

/* ------------------------------------------------------------------------------------ */
/* Memory tier: refcounted block pool, prefix cache, copy-on-write (host logic).          */
/* ------------------------------------------------------------------------------------ */
typedef struct pia_kvm pia_kvm;     /* KvCacheManager (src/memory/kv_cache_manager.rs:38-403) */
typedef struct pia_table pia_table; /* BlockTable (src/memory/block_table.rs:27-93) */

typedef struct pia_admission { /* Admission (kv_cache_manager.rs:27-36) */
  int64_t cached_tokens, reused_blocks, allocated_blocks;
} pia_admission;

typedef struct pia_kvm_stats { /* PrefixCacheStats (prefix_cache.rs:52-74) + cow_copies */
  uint64_t hits, misses, inserts, evictions, tokens_saved, cow_copies;
  int64_t available_blocks, total_blocks, active_sequences, cached_entries;
} pia_kvm_stats;

/* block_hash (src/memory/prefix_cache.rs:28-40): chained FNV-1a; ROOT_HASH is 0. */
uint64_t pia_block_hash(uint64_t parent, const uint32_t* tokens, int64_t n);

pia_status pia_kvm_create(int64_t total_blocks, int64_t block_size, int32_t enable_prefix_cache, pia_kvm** out);
pia_status pia_kvm_destroy(pia_kvm* m);
/* admit (kv_cache_manager.rs:116-195). *admitted = 0 and *out_table = NULL when the prompt
 * cannot be housed even after evicting cold cache entries. */
pia_status pia_kvm_admit(pia_kvm* m, int64_t seq_id, const uint32_t* tokens, int64_t n, uint64_t tick,
                         int32_t* admitted, pia_table** out_table, pia_admission* info);
/* publish_prompt_blocks (:204-218); returns the number of newly published blocks. */
pia_status pia_kvm_publish(pia_kvm* m, const pia_table* t, int64_t* published);
/* append_block (:223-252). */
pia_status pia_kvm_append_block(pia_kvm* m, int64_t seq_id, pia_table* t, uint64_t tick, int32_t* ok);
/* fork (:262-281): the child maps every parent block. */
pia_status pia_kvm_fork(pia_kvm* m, const pia_table* parent, int64_t child_seq, uint64_t tick, pia_table** out);
/* ensure_writable (:289-327): copy-on-write of the block holding token_pos. When a copy is
 * made, the block data moves on the device (kv, laid out as `layout`) on ctx's stream. */
pia_status pia_kvm_ensure_writable(pia_kvm* m, int64_t seq_id, pia_table* t, int64_t token_pos,
                                   pia_context* ctx, float* kv, const pia_kv_layout* layout, int32_t* copied);
pia_status pia_kvm_touch(pia_kvm* m, int64_t seq_id, uint64_t tick);
/* release_sequence (:339-345). */
pia_status pia_kvm_release(pia_kvm* m, int64_t seq_id);
/* clear (:100-112). */
pia_status pia_kvm_clear(pia_kvm* m);
pia_status pia_kvm_stats_get(const pia_kvm* m, pia_kvm_stats* out);
pia_status pia_kvm_ref_count(const pia_kvm* m, int64_t block, int64_t* out);

pia_status pia_table_create(pia_table** out);
pia_status pia_table_destroy(pia_table* t);
int64_t pia_table_len(const pia_table* t);
/* Physical block ids in logical order (int32, table_len entries). */
pia_status pia_table_blocks(const pia_table* t, int32_t* out);
pia_status pia_table_append(pia_table* t, int64_t block);
/* Per-slot provenance: hash (0 when none), has_hash and cached flags. */
pia_status pia_table_slot(const pia_table* t, int64_t i, uint64_t* hash, int32_t* has_hash, int32_t* cached);

/* ------------------------------------------------------------------------------------ */
/* Model tier: device-resident Llama weights + device KV cache.                           */
/* ------------------------------------------------------------------------------------ */
typedef struct pia_model pia_model;

typedef struct pia_model_config { /* LlamaConfig (src/model.rs:15-35) */
  int64_t hidden, layers, heads, kv_heads, inter, vocab;
  float rms_eps, rope_theta;
  int64_t attention_window; /* < 0: None (full causal attention) */
} pia_model_config;

/* Projection slots, in the reference's names (src/model.rs:357-375). */
enum {
  PIA_WQ = 0, PIA_WK = 1, PIA_WV = 2, PIA_WO = 3,
  PIA_W1 = 4, /* gate_proj */
  PIA_W2 = 5, /* down_proj */
  PIA_W3 = 6, /* up_proj */
  PIA_LM_HEAD = 7,
};
enum { PIA_NORM_ATTN = 0, PIA_NORM_FFN = 1, PIA_NORM_FINAL = 2 };

pia_status pia_model_create(pia_context* ctx, const pia_model_config* cfg, pia_model** out);
pia_status pia_model_destroy(pia_model* m);
/* token_embeddings: bf16 [vocab][hidden] (raw little-endian bits), as the reference keeps them. */
pia_status pia_model_set_embedding(pia_model* m, const uint16_t* bf16);
/* Norm weight (f32 [hidden]); layer is ignored for PIA_NORM_FINAL. */
pia_status pia_model_set_norm(pia_model* m, int64_t layer, int32_t which, const float* w);
/* Projection::Int8 from already-quantized host data (QuantizedLinear, src/model.rs:165-199). */
pia_status pia_model_set_proj_i8(pia_model* m, int64_t layer, int32_t which, const int8_t* q, const float* scales);
/* Projection::F32 from host f32 weights (PackedLinear, src/model.rs:140-163). */
pia_status pia_model_set_proj_f32(pia_model* m, int64_t layer, int32_t which, const float* w);
/* The config the model was created with. */
pia_status pia_model_get_config(const pia_model* m, pia_model_config* out);

/* LlamaConfig::from_hf_config (src/model.rs:57-95): the architecture from a HuggingFace
 * config.json. Fields absent from the file (or not of the reference's JSON type: unsigned
 * integers for sizes, numbers for rms_norm_eps / rope_theta) keep LlamaConfig::default()
 * (TinyLlama-1.1B, src/model.rs:37-53); num_key_value_heads defaults to num_attention_heads;
 * attention_window is -1 (None). A missing or malformed file is PIA_ERR_INVALID. */
pia_status pia_hf_config_read(const char* path, pia_model_config* out);

/* ModelLoader::load_weights (src/model.rs:388-447): every tensor of a bf16 HuggingFace Llama
 * safetensors checkpoint into a model created with the checkpoint's config. quantization:
 * 0 = Projection::F32 (bf16 widened), 1 = Projection::Int8 (quantize_rows_i8 on the device,
 * bit-exact with pia_quantize_rows_i8 of the widened rows) for the seven projections of every
 * layer. lm_head_int8: 0 keeps the LM head f32 as the reference's loader does; 1 quantizes it
 * too. Without lm_head.weight the embedding matrix is used (tied weights). A missing tensor,
 * a dtype other than BF16 or a shape the config does not imply is PIA_ERR_INVALID naming the
 * tensor, reported before anything is uploaded. */
pia_status pia_model_load_safetensors(pia_model* m, const char* path, int32_t quantization, int32_t lm_head_int8);
/* Bytes of device projection weights (LlamaWeights::weight_bytes, src/model.rs:590-608). */
int64_t pia_model_weight_bytes(const pia_model* m);

/* Allocate (or re-allocate, zeroed) the device KV cache: num_blocks blocks of block_size. */
pia_status pia_model_kv_alloc(pia_model* m, int64_t num_blocks, int64_t block_size);
/* Device pointer of the KV cache and its layout. */
pia_status pia_model_kv(pia_model* m, float** kv, pia_kv_layout* layout);

/* decode_batch_into (src/model.rs:1184-1207): one token per entry at positions[b], block
 * table tables[table_off[b] .. +table_len[b]). Writes this step's K/V, runs every layer and
 * the LM head. logits (host, [batch][vocab]) and argmax (host, [batch]) may each be NULL. */
pia_status pia_model_decode(pia_model* m, const uint32_t* tokens, const int64_t* positions,
                            const int64_t* table_off, const int64_t* table_len, const int32_t* tables,
                            int64_t batch, float* logits, int32_t* argmax);

/* prefill_batched (src/model.rs:1222-1255): the n prompt tokens of one sequence at
 * start_pos.. through every layer in one pass (causal), LM head on the last position only.
 * logits (host, [vocab]) and argmax (host, [1]) may be NULL. */
pia_status pia_model_prefill(pia_model* m, const uint32_t* tokens, int64_t n, int64_t start_pos,
                             const int32_t* table, int64_t table_len, float* logits, int32_t* argmax);

/* Decode path. 0 (default): one launch per kernel. 1: a batch-1 decode runs as one persistent
 * launch (every layer and the LM head, one workgroup per CU, stages separated by grid
 * barriers) when every projection is int8 and the shape fits, else one launch per kernel.
 * pia_model_decode_path_used reports the path of the last pia_model_decode (0 per-kernel,
 * 1 persistent, -1 none yet). No counterpart in the reference (it has no GPU int8 path). */
pia_status pia_model_set_decode_path(pia_model* m, int32_t path);
int32_t pia_model_decode_path_used(const pia_model* m);
/* Diagnostics (no counterpart in the reference): what the last pia_model_decode copied from the
 * host. Block tables stay on the device between decode steps (per-entry slots); a step sends
 * its tokens and entries, plus only the table slots whose block ids changed since the previous
 * step (append_block, copy-on-write remap) as (slot, id) pairs, or the whole table image when the
 * batch's layout changed or most slots differ. *bytes = host-to-device bytes of the step,
 * *table_patches = slots patched, *table_full = 1 when the image was re-sent. */
pia_status pia_model_last_upload(const pia_model* m, int64_t* bytes, int64_t* table_patches, int32_t* table_full);
/* Diagnostics (no counterpart in the reference): the shared-prefix attention of the last
 * pia_model_decode. When the entries' tables begin with the same physical blocks (prefix-cache
 * hits and forks, src/memory/kv_cache_manager.rs:116-327), the K/V of those blocks are read once
 * per group and kv head instead of once per entry; *virtual_entries = rows of that pass
 * (0: not used), *shared_splits = its token splits. */
pia_status pia_model_last_shared(const pia_model* m, int64_t* virtual_entries, int64_t* shared_splits);

/* ------------------------------------------------------------------------------------ */
/* Sampling (src/sampling.rs).                                                            */
/* ------------------------------------------------------------------------------------ */
typedef struct pia_sampling { /* Sampler's settings (src/sampling.rs:43-52) */
  float temperature; /* <= 0: greedy argmax, no draw */
  float top_p;       /* >= 1: no nucleus cut */
  int32_t top_k;     /* 0: disabled */
  int32_t reserved;  /* must be 0 */
} pia_sampling;

/* Rng::new (src/sampling.rs:20-25): the xorshift64* state for a seed. */
uint64_t pia_rng_new(uint64_t seed);

/* Sampler::sample (src/sampling.rs:74-138) for n rows of logits (device, pitch ld floats):
 * out[i] (device) = the token drawn for row i with params[i] (device), advancing the
 * xorshift64* state rng_state[i] (device) by one draw when temperature > 0. Ranking is
 * f32::total_cmp descending with equal logits in ascending index order (the reference's
 * unstable sort leaves their order unspecified).
 * mode 0 (PIA_SAMPLE_REFERENCE): the reference's arithmetic order -- a device sort, then the
 *   f32 running sums in ranking order -- so the token is the reference's; uses a workspace of
 *   about 28 bytes per logit held by the context, grown on demand (a grow synchronizes the
 *   device).
 * mode 1 (PIA_SAMPLE_EXACT_SUMS): no sort; radix searches with exact fixed-point sums. The
 *   token differs from the reference's only where the draw lies within the reference's f32
 *   summation rounding (up to vocab * 2^-24 relative) of a cumulative boundary. */
enum { PIA_SAMPLE_REFERENCE = 0, PIA_SAMPLE_EXACT_SUMS = 1 };
pia_status pia_sample_dev(pia_context* ctx, int32_t* out, const float* logits, int64_t ld, int64_t n, int64_t vocab,
                          const pia_sampling* params, uint64_t* rng_state, int32_t mode, void* stream);

/* Sample from the logits the last pia_model_decode (rows 0..n-1, n <= its batch) or
 * pia_model_prefill (n = 1) left on the device, as pia_sample_dev does, with host arrays:
 * params[n], rng_state[n] (advanced in place) and out[n]. The engine's per-sequence
 * Sampler::sample on the batch logits (src/engine.rs:741-756), without copying logits to the
 * host. */
pia_status pia_model_sample(pia_model* m, const pia_sampling* params, uint64_t* rng_state, int64_t n, int32_t mode,
                            int32_t* out);

/* ------------------------------------------------------------------------------------ */
/* Speculative verification (src/speculative.rs, src/engine.rs:595-761).                  */
/* ------------------------------------------------------------------------------------ */
/* PromptLookupDrafter::draft (src/speculative.rs:71-101): up to k tokens that followed the
 * most recent earlier occurrence of the longest suffix of context[0..n) whose length is in
 * [min_ngram, max_ngram] (the engine uses 2, 8). Writes *n_out <= k tokens to out. */
pia_status pia_prompt_lookup_draft(const uint32_t* context, int64_t n, int64_t k, int64_t min_ngram,
                                   int64_t max_ngram, uint32_t* out, int64_t* n_out);
/* verify_greedy (src/speculative.rs:204-223): the leading drafts equal to the model's argmax
 * are accepted; *corrected = model_argmax[*n_accepted]. n_argmax must be n_drafts + 1. */
pia_status pia_verify_greedy(const uint32_t* drafts, int64_t n_drafts, const uint32_t* model_argmax,
                             int64_t n_argmax, int64_t* n_accepted, uint32_t* corrected);

typedef struct pia_spec_group { /* SpecGroup (src/engine.rs:175-182) */
  int64_t pos;        /* position of the held token; token j sits at pos + j */
  int64_t n_tokens;   /* 1 (the held token) + number of drafts */
  int64_t tokens_off; /* tokens[tokens_off .. + n_tokens): held token, then the drafts */
  int64_t table_off;  /* the sequence's block table: tables[table_off .. + table_len) */
  int64_t table_len;
} pia_spec_group;

/* Engine::run_groups + commit's verification (src/engine.rs:702-783): every group's positions
 * flattened into batched decode passes of at most `capacity` entries (0 = one pass), each
 * position's greedy argmax written to predictions (flattened group order, sum of n_tokens),
 * then verify_greedy per group into n_accepted[g] / corrected[g] (either may be NULL).
 * *passes (may be NULL) = model passes run. Block tables must already cover every position
 * and be writable there (ensure_writable), as the engine's plan_step guarantees. */
pia_status pia_model_verify_groups(pia_model* m, const pia_spec_group* groups, int64_t n_groups,
                                   const uint32_t* tokens, const int32_t* tables, int64_t capacity,
                                   uint32_t* predictions, int64_t* n_accepted, uint32_t* corrected, int64_t* passes);

/* Per-kernel timing of the last pia_model_decode / pia_model_prefill call (HIP events around
 * every launch on the context stream), accumulated per class: 0 = q/k/v projection, 1 = o,
 * 2 = gate/up, 3 = down, 4 = LM head, 5 = attention, 6 = everything else, 7 = the persistent
 * batch-1 decode step (all of a step in one launch). `bytes` are the
 * algorithmic bytes of those launches, `calls` their number. Enable with
 * pia_model_profile(m, 1); profiled calls run without graph replay. No counterpart in the
 * reference (its benches time whole steps). */
pia_status pia_model_profile(pia_model* m, int32_t enable);
pia_status pia_model_profile_get(pia_model* m, double* ms_per_class, int64_t* bytes_per_class,
                                 int64_t* calls_per_class, int32_t n_class);
/* Mean device time of one launch of a projection class (0..4 above) at `batch`, from a graph
 * of that class's launches over every layer (the model's weights, buffers and kernels of a
 * decode step), and the algorithmic bytes of one launch. Overwrites the activation buffers.
 * No counterpart in the reference. */
pia_status pia_model_bench_class(pia_model* m, int32_t cls, int64_t batch, int32_t reps, double* us,
                                 int64_t* bytes);

/* ------------------------------------------------------------------------------------ */
/* Diagnostics (no counterpart in the reference).                                         */
/* ------------------------------------------------------------------------------------ */
/* Device time of one int8 projection launch of shape rows x cols at `batch` (the kernel the
 * model uses for that shape): `reps` launches captured in one graph, cycling through enough
 * distinct weight copies (>= 1 GiB) that every launch streams from HBM, HIP events around a
 * replay; *us = mean microseconds per launch. Also reports the launch's
 * algorithmic bytes (int8 weights + scales + activations in + results out). */
/* flags: 1 = fused RMSNorm prologue, 2 = SwiGLU epilogue, 4 = residual-add epilogue,
 * 8 = matrix-core path (digit split; the digit conversion is timed with it), 16 (with 8) = the
 * digits are written once before the timed launches, which then time the projection alone. */
pia_status pia_bench_projection(pia_context* ctx, int64_t rows, int64_t cols, int64_t batch, int32_t reps,
                                int32_t flags, double* us, int64_t* bytes);

/* ------------------------------------------------------------------------------------ */
/* Synthetic inputs (no counterpart in the reference: seeded data for tests and benches). */
/* ------------------------------------------------------------------------------------ */
/* n samples of N(0, std^2) as f32 from (seed, stream): SplitMix64 + Box-Muller in f64. */
pia_status pia_synth_normal(uint64_t seed, uint64_t stream, float std, float* out, int64_t n);
/* f32 -> bf16 bits, round to nearest even. */
pia_status pia_f32_to_bf16(const float* in, uint16_t* out, int64_t n);

#ifdef __cplusplus
}
#endif
#endif /* PAGED_INFER_AMD_H */
