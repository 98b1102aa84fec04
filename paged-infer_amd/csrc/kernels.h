// Launchers for the gfx950 kernels. All take device pointers and enqueue on `st`.
// Shapes are validated by the caller (model / C ABI); launchers assert the invariants
// the kernels' indexing relies on.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "paged_infer_amd.h"

namespace pia {

// Slots per batch row of the fused argmax: spreading the atomics over 256 addresses keeps
// thousands of workgroups from serializing on one.
constexpr int kArgmaxSlots = 256;

// Batch from which int8 projections run on the matrix cores instead of the streaming GEMV.
constexpr int64_t kMfmaMinBatch = 5;

// Digit matrix of the matrix-core projection (see gemm_mfma.hip): batch entries in groups of
// 16, entry b's digit plane j is digit row (3 (b / 16) + j) * 16 + b % 16; storage is k-step
// major (the 64 bytes of every digit row for one 64-column k-step are contiguous).
__host__ __device__ inline int digit_row(int b, int j) { return ((b >> 4) * 3 + j) * 16 + (b & 15); }
__host__ __device__ inline int64_t digit_off(int64_t n, int64_t k, int64_t nrows) {
  return ((k >> 6) * nrows + n) * 64 + (k & 63);
}
// Groups of 16 batch entries: 48 digit rows and 16 power-of-two factors each.
int64_t digit_groups(int64_t batch);

// Epilogue of a projection: store, accumulate into the destination (residual add, as
// src/model.rs:1127-1129 and :1165-1167 do with proj_out / ff_down), or SwiGLU over
// interleaved gate/up row pairs (src/math.rs:293-302).
enum class Epi : int { Store = 0, Add = 1, Swiglu = 2 };

// y[b][r] = dot(W[r, :cols], xn[b]) * (scales ? scales[r] : 1), xn = x or RMSNorm(x) * norm_w
// when norm_w is set; written to out[b*osb + r*osr] (Store), added to it (Add), or for
// Swiglu out[b*osb + (r/2)*osr] = silu(y[b][r]) * y[b][r+1] for even r.
// W is int8 (wkind 1, scales required) or f32 (wkind 0), row stride ldw elements.
struct GemvArgs {
  int wkind;
  const void* W;
  int64_t ldw;
  const float* scales;
  const float* x;
  int64_t ldx;
  const float* norm_w;
  float eps;
  float* out;
  int64_t osb, osr;
  int64_t rows, cols, batch;
  Epi epi;
  // Optional fused greedy argmax (Store only): the max over rows of
  // (f32 total-order key of out[b][r]) << 32 | r lands in one of the kArgmaxSlots slots
  // amax[b * kArgmaxSlots + i]; the caller zeroes them first and takes the max of the slots.
  unsigned long long* amax = nullptr;
};
void launch_gemv(const GemvArgs& args, hipStream_t st);

// Batched int8 projection on the int8 matrix cores (see gemm_mfma.hip). launch_xdigits writes
// the activations (optionally RMSNorm(x) * norm_w) as three signed 8-bit digits of a 23-bit
// fixed-point image per row into the workspace `xq` (xdigits_bytes); launch_gemm_i8_mfma then
// computes the projection with exact int32 accumulation and the epilogues of launch_gemv.
// Weight rows must be zero-padded to a multiple of 64 bytes (ldw >= that).
int64_t xdigits_bytes(int64_t batch, int64_t cols);
void launch_xdigits(const float* x, int64_t ldx, const float* norm_w, float eps, int64_t batch, int64_t cols,
                    void* xq, hipStream_t st);
// Split-K workspace of the decode GEMM: exact 64-bit partial sums of up to `pairs` (row tile,
// K slice) pairs of 128 rows x 64 entries, then one counter per row tile (zero when allocated,
// left zero by every launch). Launches that would need more pairs split less.
constexpr int64_t kDecSplitPairs = 512;
struct DecSplitWork {
  unsigned long long* ws;
  unsigned* cnt;
  int64_t pairs;
};
int64_t dec_split_bytes(int64_t pairs = kDecSplitPairs);
DecSplitWork dec_split_work(void* base, int64_t pairs = kDecSplitPairs);
void launch_gemm_i8_mfma(const int8_t* W, int64_t ldw, const float* scales, const void* xq, float* out, int64_t osb,
                         int64_t osr, int64_t rows, int64_t cols, int64_t batch, Epi epi, unsigned long long* amax,
                         const DecSplitWork* split, hipStream_t st);

// out[r] = RMSNorm(x[r]) * w  (src/math.rs:4-22), rows of n, row strides ldx / ldo.
void launch_rmsnorm(const float* x, int64_t ldx, const float* w, float* out, int64_t ldo, int64_t rows, int64_t n,
                    float eps, hipStream_t st);

// x[b] = bf16 embedding row (tokens[b] % vocab) widened to f32 (src/model.rs:1015-1020).
// Also zeroes amax[0 .. batch * kArgmaxSlots) (this step's fused-argmax slots) when given.
void launch_embed(const int32_t* tokens, const uint16_t* embed, float* x, int64_t ldx, int64_t batch, int64_t hidden,
                  int64_t vocab, unsigned long long* amax, hipStream_t st);

// NeoX RoPE on q (num_heads) and k (num_kv_heads) in place inside qkv rows (stride ldq; q at
// column 0, k at heads*hd, v at (heads+kv_heads)*hd), then K/V scatter into the paged cache
// for every entry whose position is mapped (src/model.rs:1068-1107).
void launch_rope_kv_write(float* qkv, int64_t ldq, const pia_attn_entry* entries, const int32_t* tables,
                          const float* rope_cos, const float* rope_sin, float* kv, const pia_kv_layout& layout,
                          int64_t heads, int64_t batch, int64_t layer, hipStream_t st);

// K/V scatter alone (src/model.rs:1093-1107): k/v rows [n][num_kv_heads * head_dim] to each
// entry's slot at its pos; entries whose pos is unmapped write nothing.
void launch_kv_write(const float* k, const float* v, const pia_attn_entry* entries, const int32_t* tables, float* kv,
                     const pia_kv_layout& layout, int64_t n, int64_t layer, hipStream_t st);

// PagedAttention::run for one layer (see attention.hip). `plan` picks the token split;
// `work` (attention_work_bytes) is needed when plan.splits > 1 (a combine kernel follows).
// When `fused`, q rows are the raw qkv rows (RoPE applied in the kernel) and each entry's own
// K/V is rotated and written by the kernel; only valid when no entry reads a cache slot
// written by another entry of the same launch.
struct AttnPlan {
  int64_t split;   // tokens per workgroup (a multiple of chunk)
  int64_t splits;  // workgroups per (entry, kv head), <= 128
  int64_t chunk;   // tokens per inner step: 256, 128 or 64
};
AttnPlan plan_attention(int64_t n, int64_t num_kv_heads, int64_t head_dim, int64_t max_window, int num_cus);
int64_t attention_work_bytes(int64_t n, int64_t heads, int64_t head_dim, int64_t splits);
struct AttnLaunch {
  const float* q;
  int64_t ldq;
  float* out;
  int64_t ldo;
  float* kv;
  const pia_kv_layout* layout;
  int64_t heads;
  const pia_attn_entry* entries;
  const int32_t* tables;
  int64_t n, layer;
  AttnPlan plan;
  void* work;
  bool fused;
  const float* rope_cos;
  const float* rope_sin;
  // Entries are consecutive positions of one sequence sharing one block table (a prefill):
  // from kPrefillTileMin entries (head_dim 64 or 128, not fused) a query-tiled kernel runs
  // instead, which reads each K/V row once per tile of positions.
  bool prefill = false;
  // Shared-prefix decode (fused launches only): n_shared virtual entries over the shared
  // leading blocks of groups of entries (see attention.hip) write their partials into split
  // slots [0, shared_splits) of `work`; the main launch covers each entry's remaining tokens
  // (its entry's start) in the slots after them, and the combine merges all of them.
  const pia_attn_entry* shared_entries = nullptr;
  const int32_t* shared_vmap = nullptr;  // [n_shared][2]: real entry, split slot
  int64_t n_shared = 0, shared_splits = 0;
};
// Query rows (positions x heads of one kv head) per tile of the shared-prefix / prefill kernel.
int64_t attention_tile_rows();
constexpr int64_t kPrefillTileMin = 64;
void launch_attention(const AttnLaunch& a, hipStream_t st);

// Spin for about `us` microseconds (one thread; bounded by the device clock). Used only to let
// the host enqueue ahead of the device while per-kernel events are being recorded.
void launch_spin(double us, hipStream_t st);

// h[b][i] = silu(gu[b][i]) * gu[b][inter + i]  (src/math.rs:293-302).
void launch_swiglu(const float* gu, int64_t ldgu, float* h, int64_t ldh, int64_t batch, int64_t inter,
                   hipStream_t st);

void launch_argmax(const float* logits, int64_t ld, int32_t* out, int64_t n, int64_t vocab, hipStream_t st);

void launch_quantize_rows(const float* w, int64_t rows, int64_t cols, int8_t* q, float* scales, hipStream_t st);
// Sampler::sample on the device (sampling.hip). mode 0: the reference's arithmetic order (a
// device sort, then in-order f32 sums; needs sample_workspace_bytes(n, vocab) of workspace);
// mode 1: radix search with exact fixed-point sums (no workspace).
size_t sample_workspace_bytes(int64_t n, int64_t vocab);
// Rows whose temperature is <= 0 or whose top_k is in 1..sample_topk_max(): the reference's
// order without a sort of the vocabulary (the kept tokens are selected, then sorted in LDS).
int64_t sample_topk_max();
void launch_sample_topk(const float* logits, int64_t ld, int64_t n, int64_t vocab, const pia_sampling* params,
                        uint64_t* rng, int32_t* out, hipStream_t st);
void launch_sample(const float* logits, int64_t ld, int64_t n, int64_t vocab, const pia_sampling* params,
                   uint64_t* rng, int32_t* out, int mode, void* workspace, size_t workspace_bytes, hipStream_t st);

// Checkpoint loading: bf16 rows [rows][cols] quantized (bit-exact with launch_quantize_rows of
// the widened rows) or widened, source row r written to destination row r * row_step.
void launch_quantize_rows_bf16(const uint16_t* w, int64_t rows, int64_t cols, int8_t* q, int64_t ldq, float* scales,
                               int64_t row_step, hipStream_t st);
void launch_widen_rows_bf16(const uint16_t* w, int64_t rows, int64_t cols, float* out, int64_t ldo, int64_t row_step,
                            hipStream_t st);

// Persistent batch-1 decode step (decode_step.hip): every layer and the LM head in one
// launch of one workgroup per CU, stages separated by grid barriers. All layer projections
// must be int8; the LM head may be int8 or f32.
struct StepLayer {
  const int8_t* qkv;  // [qkv_rows][ld_h]: q, k, v rows
  const float* qkv_s;
  const int8_t* o;  // [hidden][ld_h]
  const float* o_s;
  const int8_t* gu;  // [2*inter][ld_h]: gate/up rows interleaved
  const float* gu_s;
  const int8_t* down;  // [hidden][ld_i]
  const float* down_s;
  const float* attn_norm;
  const float* ffn_norm;
};
struct StepParams {
  int layers, hidden, heads, hkv, inter, vocab, qkv_rows;
  int64_t ld_h, ld_i, ld_lm;  // weight row strides in elements
  float eps, scale;
  const StepLayer* L;  // device array [layers]
  const void* lm;      // int8 or f32 [vocab][ld_lm]
  const float* lm_s;
  const float* final_norm;
  const uint16_t* embed;
  float* kv;
  int num_blocks, block_size;
  const float* rope_cos;
  const float* rope_sin;
  const int32_t* token;          // [1]
  const pia_attn_entry* entry;   // [1]
  const int32_t* tables;
  float* x;        // [hidden] residual stream
  float* qkv_buf;  // [qkv_rows]
  float* attn;     // [hidden]
  float* h;        // [inter]
  float* part;     // [heads][max_splits][hd + 2]
  float* logits;   // [vocab]
  unsigned long long* amax;  // [kArgmaxSlots]
  unsigned* flags;           // [num_cus * 32]
  unsigned* attn_cnt;        // [hkv * 32] finished splits per kv head (zero between steps)
  unsigned* step_ctr;        // [1]
  int* err;                  // [1]
  int max_splits;            // token splits per kv head
  unsigned long long* trace;  // optional [16 * layers + 2] stage timestamps (workgroup 0), or null
};
struct StepShape {
  int64_t hidden, heads, hkv, hd, inter, vocab, qkv_rows;
  int64_t max_splits, max_tokens;  // token splits per kv head; tokens per split
  bool lm_i8;
};
constexpr size_t kMaxStepSmem = 96 * 1024;
// nullptr when the step kernel handles this shape on a device with num_cus CUs, else why not.
const char* decode_step_unsupported(const StepShape& s, int num_cus);
size_t decode_step_smem(const StepShape& s);
// Token splits per kv head for a grid of num_cus workgroups.
int decode_step_splits(int num_cus, int64_t hkv);
void launch_decode_step(const StepParams& p, const StepShape& s, int num_cus, hipStream_t st);

void launch_copy_block(float* kv, const pia_kv_layout& layout, int64_t src, int64_t dst, hipStream_t st);

// tab[patch[2i]] = patch[2i + 1] for i < n (the changed slots of device-resident block tables).
void launch_table_patch(int32_t* tab, const int32_t* patch, int64_t n, hipStream_t st);

}  // namespace pia
