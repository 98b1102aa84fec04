// Launchers for the gfx950 kernels. All take device pointers and enqueue on `st`.
// Shapes are validated by the caller (model / C ABI); launchers assert the invariants
// the kernels' indexing relies on.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "paged_infer_amd.h"

namespace pia {

// Epilogue of a projection: store, or accumulate into the destination (residual add, as
// src/model.rs:1127-1129 and :1165-1167 do with proj_out / ff_down).
enum class Epi : int { Store = 0, Add = 1 };

// out[b*osb + r*osr] (=|+=) dot(W[r, :cols], x[b*ldx + :cols]) * (scales ? scales[r] : 1).
// W is int8 (wkind 1, scales required) or f32 (wkind 0), row stride ldw elements.
void launch_gemv(int wkind, const void* W, int64_t ldw, const float* scales, const float* x, int64_t ldx, float* out,
                 int64_t osb, int64_t osr, int64_t rows, int64_t cols, int64_t batch, Epi epi, hipStream_t st);

// Batched int8 projection on MFMA for batch >= 16 (decode batches and prefill).
// Activations are split into three signed 8-bit digits per row (exact for the 23-bit
// fixed-point image of x); weights stay int8; accumulation is exact int32.
// `xq` workspace: see xdigits_bytes(). out[b*osb + r*osr] (=|+=) as launch_gemv.
int64_t xdigits_bytes(int64_t batch, int64_t cols);
void launch_xdigits(const float* x, int64_t ldx, int64_t batch, int64_t cols, void* xq, hipStream_t st);
void launch_gemm_i8_mfma(const int8_t* W, int64_t ldw, const float* scales, const void* xq, float* out, int64_t osb,
                         int64_t osr, int64_t rows, int64_t cols, int64_t batch, Epi epi, hipStream_t st);

// out[r] = RMSNorm(x[r]) * w  (src/math.rs:4-22), rows of n, row strides ldx / ldo.
void launch_rmsnorm(const float* x, int64_t ldx, const float* w, float* out, int64_t ldo, int64_t rows, int64_t n,
                    float eps, hipStream_t st);

// x[b] = bf16 embedding row (tokens[b] % vocab) widened to f32 (src/model.rs:1015-1020).
void launch_embed(const int32_t* tokens, const uint16_t* embed, float* x, int64_t ldx, int64_t batch, int64_t hidden,
                  int64_t vocab, hipStream_t st);

// NeoX RoPE on q (num_heads) and k (num_kv_heads) in place inside qkv rows (stride ldq; q at
// column 0, k at heads*hd, v at (heads+kv_heads)*hd), then K/V scatter into the paged cache
// for every entry whose position is mapped (src/model.rs:1068-1107).
void launch_rope_kv_write(float* qkv, int64_t ldq, const pia_attn_entry* entries, const int32_t* tables,
                          const float* rope_cos, const float* rope_sin, float* kv, const pia_kv_layout& layout,
                          int64_t heads, int64_t batch, int64_t layer, hipStream_t st);

// PagedAttention::run for one layer. q rows have stride ldq, out rows stride ldo.
// `work` must hold attention_work_bytes(...) bytes when more than one split is used.
int64_t attention_splits(int64_t max_window);
int64_t attention_work_bytes(int64_t n, int64_t heads, int64_t head_dim, int64_t splits);
void launch_attention(const float* q, int64_t ldq, float* out, int64_t ldo, const float* kv,
                      const pia_kv_layout& layout, int64_t heads, const pia_attn_entry* entries,
                      const int32_t* tables, int64_t n, int64_t layer, int64_t splits, void* work, hipStream_t st);

// h[b][i] = silu(gu[b][i]) * gu[b][inter + i]  (src/math.rs:293-302).
void launch_swiglu(const float* gu, int64_t ldgu, float* h, int64_t ldh, int64_t batch, int64_t inter,
                   hipStream_t st);

void launch_argmax(const float* logits, int64_t ld, int32_t* out, int64_t n, int64_t vocab, hipStream_t st);

void launch_quantize_rows(const float* w, int64_t rows, int64_t cols, int8_t* q, float* scales, hipStream_t st);

void launch_copy_block(float* kv, const pia_kv_layout& layout, int64_t src, int64_t dst, hipStream_t st);

}  // namespace pia
