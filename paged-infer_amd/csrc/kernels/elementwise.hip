// Small per-row kernels of a decode step: embedding gather, RMSNorm, NeoX RoPE fused with the
// paged K/V scatter, SwiGLU, greedy argmax, the on-device quantizer and the copy-on-write
// block copy. The library is built with -ffp-contract=off, so each expression below rounds
// exactly as the reference's f32 code does (no fused multiply-add unless written).
#include "common.h"
#include "kernels.h"

namespace pia {
namespace {

constexpr int kThreads = 256;

__device__ inline float block_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.0f;
  if (threadIdx.x == 0) {
    for (int w = 0; w < kThreads / 64; ++w) t += red[w];
    red[kThreads / 64] = t;
  }
  __syncthreads();
  const float r = red[kThreads / 64];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kThreads) void k_embed(const int32_t* __restrict__ tokens, const uint16_t* __restrict__ emb,
                                                    float* __restrict__ x, int64_t ldx, int64_t hidden, int64_t vocab,
                                                    unsigned long long* __restrict__ amax) {
  const int b = blockIdx.x;
  if (amax && threadIdx.x < kArgmaxSlots) amax[b * kArgmaxSlots + threadIdx.x] = 0ull;
  const int64_t tok = static_cast<int64_t>(static_cast<uint32_t>(tokens[b])) % vocab;
  const uint16_t* src = emb + tok * hidden;
  float* dst = x + static_cast<int64_t>(b) * ldx;
  for (int64_t i = threadIdx.x; i < hidden; i += kThreads) dst[i] = __uint_as_float(static_cast<uint32_t>(src[i]) << 16);
}

// src/math.rs:4-22 with a parallel sum of squares.
__global__ __launch_bounds__(kThreads) void k_rmsnorm(const float* __restrict__ x, int64_t ldx,
                                                      const float* __restrict__ w, float* __restrict__ out,
                                                      int64_t ldo, int n, float eps) {
  __shared__ float red[kThreads / 64 + 1];
  const float* xr = x + static_cast<int64_t>(blockIdx.x) * ldx;
  float* orow = out + static_cast<int64_t>(blockIdx.x) * ldo;
  constexpr int kPer = 16;  // rows up to 4096 stay in registers; longer rows take a second pass
  float v[kPer];
  float ss = 0.0f;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int i = threadIdx.x + u * kThreads;
    v[u] = i < n ? xr[i] : 0.0f;
    ss += v[u] * v[u];
  }
  for (int i = threadIdx.x + kPer * kThreads; i < n; i += kThreads) ss += xr[i] * xr[i];
  ss = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int i = threadIdx.x + u * kThreads;
    if (i < n) orow[i] = (v[u] * inv) * w[i];
  }
  for (int i = threadIdx.x + kPer * kThreads; i < n; i += kThreads) orow[i] = (xr[i] * inv) * w[i];
}

// src/model.rs:1068-1107: rotate every q head and (once) every kv head, then write K and V
// for the entry's position into the paged cache if its logical block is mapped.
__global__ __launch_bounds__(kThreads) void k_rope_kv(float* __restrict__ qkv, int64_t ldq,
                                                      const pia_attn_entry* __restrict__ entries,
                                                      const int32_t* __restrict__ tables,
                                                      const float* __restrict__ rc, const float* __restrict__ rs,
                                                      float* __restrict__ kv, int64_t layer_slots, int block_size,
                                                      int heads, int hkv, int hd) {
  const int b = blockIdx.x;
  const pia_attn_entry en = entries[b];
  const int half = hd / 2;
  const float* c = rc + static_cast<int64_t>(en.pos) * half;
  const float* s = rs + static_cast<int64_t>(en.pos) * half;
  float* row = qkv + static_cast<int64_t>(b) * ldq;
  for (int idx = threadIdx.x; idx < heads * half; idx += kThreads) {
    const int h = idx / half, j = idx % half;
    float* xh = row + h * hd;
    const float a = xh[j], bb = xh[j + half];
    xh[j] = a * c[j] - bb * s[j];
    xh[j + half] = bb * c[j] + a * s[j];
  }
  float* k = row + heads * hd;
  const float* v = k + hkv * hd;
  const int lb = en.pos / block_size;
  const bool mapped = lb < en.table_len;
  int64_t base = 0;
  if (mapped) {
    const int64_t slot = static_cast<int64_t>(tables[en.table_off + lb]) * block_size + en.pos % block_size;
    base = (layer_slots + slot) * hkv * 2 * hd;
  }
  for (int idx = threadIdx.x; idx < hkv * half; idx += kThreads) {
    const int h = idx / half, j = idx % half;
    float* xh = k + h * hd;
    const float a = xh[j], bb = xh[j + half];
    const float r0 = a * c[j] - bb * s[j];
    const float r1 = bb * c[j] + a * s[j];
    xh[j] = r0;
    xh[j + half] = r1;
    if (mapped) {
      kv[base + static_cast<int64_t>(h) * 2 * hd + j] = r0;
      kv[base + static_cast<int64_t>(h) * 2 * hd + j + half] = r1;
    }
  }
  if (mapped)
    for (int idx = threadIdx.x; idx < hkv * hd; idx += kThreads) {
      const int h = idx / hd, d = idx % hd;
      kv[base + (static_cast<int64_t>(h) * 2 + 1) * hd + d] = v[idx];
    }
}

// K/V scatter of one entry per workgroup: k/v rows [n][hkv * hd] to the entry's cache slot
// (src/model.rs:1093-1107); an unmapped position writes nothing.
__global__ __launch_bounds__(kThreads) void k_kv_write(const float* __restrict__ k, const float* __restrict__ v,
                                                       const pia_attn_entry* __restrict__ entries,
                                                       const int32_t* __restrict__ tables, float* __restrict__ kv,
                                                       int64_t layer_slots, int block_size, int hkv, int hd) {
  const int b = blockIdx.x;
  const pia_attn_entry en = entries[b];
  const int lb = en.pos / block_size;
  if (lb >= en.table_len) return;
  const int64_t slot = static_cast<int64_t>(tables[en.table_off + lb]) * block_size + en.pos % block_size;
  float* dst = kv + (layer_slots + slot) * hkv * 2 * hd;
  const float* kr = k + static_cast<int64_t>(b) * hkv * hd;
  const float* vr = v + static_cast<int64_t>(b) * hkv * hd;
  for (int idx = threadIdx.x; idx < hkv * hd; idx += kThreads) {
    const int h = idx / hd, d = idx % hd;
    dst[static_cast<int64_t>(h) * 2 * hd + d] = kr[idx];
    dst[(static_cast<int64_t>(h) * 2 + 1) * hd + d] = vr[idx];
  }
}

__global__ __launch_bounds__(kThreads) void k_swiglu(const float* __restrict__ gu, int64_t ldgu, float* __restrict__ h,
                                                     int64_t ldh, int inter) {
  const int b = blockIdx.y;
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i >= inter) return;
  const float g = gu[static_cast<int64_t>(b) * ldgu + i];
  const float u = gu[static_cast<int64_t>(b) * ldgu + inter + i];
  const float silu = g / (1.0f + expf(-g));
  h[static_cast<int64_t>(b) * ldh + i] = silu * u;
}

// f32 total order key (f32::total_cmp): larger key = later in the order.
__device__ inline int32_t total_key(float f) {
  const int32_t b = __float_as_int(f);
  return b ^ static_cast<int32_t>(static_cast<uint32_t>(b >> 31) >> 1);
}

// src/sampling.rs:140-147: max_by(total_cmp) keeps the last of equal maxima.
__global__ __launch_bounds__(kThreads) void k_argmax(const float* __restrict__ logits, int64_t ld,
                                                     int32_t* __restrict__ out, int vocab) {
  __shared__ int32_t rk[kThreads / 64];
  __shared__ int32_t ri[kThreads / 64];
  const float* row = logits + static_cast<int64_t>(blockIdx.x) * ld;
  int32_t bk = INT32_MIN, bi = -1;
  for (int i = threadIdx.x; i < vocab; i += kThreads) {
    const int32_t k = total_key(row[i]);
    if (bi < 0 || k > bk || (k == bk && i > bi)) bk = k, bi = i;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const int32_t ok = __shfl_xor(bk, off, 64), oi = __shfl_xor(bi, off, 64);
    if (oi >= 0 && (bi < 0 || ok > bk || (ok == bk && oi > bi))) bk = ok, bi = oi;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) rk[wave] = bk, ri[wave] = bi;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 0; w < kThreads / 64; ++w)
      if (ri[w] >= 0 && (bi < 0 || rk[w] > bk || (rk[w] == bk && ri[w] > bi))) bk = rk[w], bi = ri[w];
    out[blockIdx.x] = bi < 0 ? 0 : bi;
  }
}

// Source element of a weight row: f32 as is, or bf16 bits widened exactly (bits << 16, the
// conversion of half::bf16::to_f32 that src/model.rs:455-460 applies at load).
__device__ inline float widen(float v) { return v; }
__device__ inline float widen(uint16_t v) { return __uint_as_float(static_cast<uint32_t>(v) << 16); }

// src/math.rs:456-469 on the device. IEEE division and roundf (half away from zero) make it
// bit-identical to the host quantizer; the row max is order independent. Source row r lands
// at destination row r * row_step (pitch ldq, scale at scales[r * row_step]).
template <typename Src>
__global__ __launch_bounds__(kThreads) void k_quantize(const Src* __restrict__ w, int64_t cols,
                                                       int8_t* __restrict__ q, int64_t ldq,
                                                       float* __restrict__ scales, int64_t row_step) {
  __shared__ float red[kThreads / 64 + 1];
  const Src* row = w + static_cast<int64_t>(blockIdx.x) * cols;
  const int64_t dst_row = static_cast<int64_t>(blockIdx.x) * row_step;
  float m = 0.0f;
  for (int64_t i = threadIdx.x; i < cols; i += kThreads) m = fmaxf(m, fabsf(widen(row[i])));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[wave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.0f;
    for (int i = 0; i < kThreads / 64; ++i) t = fmaxf(t, red[i]);
    red[kThreads / 64] = t;
  }
  __syncthreads();
  const float max_abs = red[kThreads / 64];
  const float scale = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
  if (threadIdx.x == 0) scales[dst_row] = scale;
  int8_t* qrow = q + dst_row * ldq;
  for (int64_t i = threadIdx.x; i < cols; i += kThreads) {
    float v = roundf(widen(row[i]) / scale);
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    qrow[i] = static_cast<int8_t>(v);
  }
}

// PackedLinear::from_tensor (src/model.rs:140-163): bf16 rows widened to f32, row r at
// destination row r * row_step (pitch ldo).
__global__ __launch_bounds__(kThreads) void k_widen_rows(const uint16_t* __restrict__ w, int64_t cols,
                                                         float* __restrict__ out, int64_t ldo, int64_t row_step) {
  const uint16_t* row = w + static_cast<int64_t>(blockIdx.x) * cols;
  float* orow = out + static_cast<int64_t>(blockIdx.x) * row_step * ldo;
  for (int64_t i = threadIdx.x; i < cols; i += kThreads) orow[i] = widen(row[i]);
}

// KvLayout::copy_block: blockIdx.y = layer.
__global__ __launch_bounds__(kThreads) void k_copy_block(float* __restrict__ kv, int64_t num_blocks, int64_t stride,
                                                         int64_t src, int64_t dst) {
  const int64_t layer = blockIdx.y;
  const float4* s = reinterpret_cast<const float4*>(kv + (layer * num_blocks + src) * stride);
  float4* d = reinterpret_cast<float4*>(kv + (layer * num_blocks + dst) * stride);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < stride / 4;
       i += static_cast<int64_t>(gridDim.x) * kThreads)
    d[i] = s[i];
}

}  // namespace

void launch_embed(const int32_t* tokens, const uint16_t* embed, float* x, int64_t ldx, int64_t batch, int64_t hidden,
                  int64_t vocab, unsigned long long* amax, hipStream_t st) {
  if (batch == 0) return;
  hipLaunchKernelGGL(k_embed, dim3(static_cast<unsigned>(batch)), dim3(kThreads), 0, st, tokens, embed, x, ldx, hidden,
                     vocab, amax);
  PIA_HIP(hipGetLastError());
}

void launch_rmsnorm(const float* x, int64_t ldx, const float* w, float* out, int64_t ldo, int64_t rows, int64_t n,
                    float eps, hipStream_t st) {
  if (rows == 0) return;
  hipLaunchKernelGGL(k_rmsnorm, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, st, x, ldx, w, out, ldo,
                     static_cast<int>(n), eps);
  PIA_HIP(hipGetLastError());
}

void launch_rope_kv_write(float* qkv, int64_t ldq, const pia_attn_entry* entries, const int32_t* tables,
                          const float* rope_cos, const float* rope_sin, float* kv, const pia_kv_layout& L,
                          int64_t heads, int64_t batch, int64_t layer, hipStream_t st) {
  if (batch == 0) return;
  PIA_REQUIRE(L.head_dim % 2 == 0, "rope: head_dim must be even");
  hipLaunchKernelGGL(k_rope_kv, dim3(static_cast<unsigned>(batch)), dim3(kThreads), 0, st, qkv, ldq, entries, tables,
                     rope_cos, rope_sin, kv, layer * L.num_blocks * L.block_size, static_cast<int>(L.block_size),
                     static_cast<int>(heads), static_cast<int>(L.num_kv_heads), static_cast<int>(L.head_dim));
  PIA_HIP(hipGetLastError());
}

void launch_kv_write(const float* k, const float* v, const pia_attn_entry* entries, const int32_t* tables, float* kv,
                     const pia_kv_layout& L, int64_t n, int64_t layer, hipStream_t st) {
  if (n == 0) return;
  PIA_REQUIRE(layer >= 0 && layer < L.num_layers, "kv_write: layer out of range");
  PIA_REQUIRE(n < (int64_t(1) << 31), "kv_write: too many entries");
  hipLaunchKernelGGL(k_kv_write, dim3(static_cast<unsigned>(n)), dim3(kThreads), 0, st, k, v, entries, tables, kv,
                     layer * L.num_blocks * L.block_size, static_cast<int>(L.block_size),
                     static_cast<int>(L.num_kv_heads), static_cast<int>(L.head_dim));
  PIA_HIP(hipGetLastError());
}

void launch_swiglu(const float* gu, int64_t ldgu, float* h, int64_t ldh, int64_t batch, int64_t inter,
                   hipStream_t st) {
  if (batch == 0) return;
  dim3 grid(static_cast<unsigned>((inter + kThreads - 1) / kThreads), static_cast<unsigned>(batch));
  hipLaunchKernelGGL(k_swiglu, grid, dim3(kThreads), 0, st, gu, ldgu, h, ldh, static_cast<int>(inter));
  PIA_HIP(hipGetLastError());
}

void launch_argmax(const float* logits, int64_t ld, int32_t* out, int64_t n, int64_t vocab, hipStream_t st) {
  if (n == 0) return;
  hipLaunchKernelGGL(k_argmax, dim3(static_cast<unsigned>(n)), dim3(kThreads), 0, st, logits, ld, out,
                     static_cast<int>(vocab));
  PIA_HIP(hipGetLastError());
}

void launch_quantize_rows(const float* w, int64_t rows, int64_t cols, int8_t* q, float* scales, hipStream_t st) {
  if (rows == 0) return;
  PIA_REQUIRE(rows < (int64_t(1) << 31), "quantize: too many rows");
  hipLaunchKernelGGL(k_quantize<float>, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, st, w, cols, q, cols,
                     scales, int64_t(1));
  PIA_HIP(hipGetLastError());
}

void launch_quantize_rows_bf16(const uint16_t* w, int64_t rows, int64_t cols, int8_t* q, int64_t ldq, float* scales,
                               int64_t row_step, hipStream_t st) {
  if (rows == 0) return;
  PIA_REQUIRE(rows < (int64_t(1) << 31), "quantize: too many rows");
  PIA_REQUIRE(ldq >= cols && row_step >= 1, "quantize: bad destination pitch");
  hipLaunchKernelGGL(k_quantize<uint16_t>, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, st, w, cols, q, ldq,
                     scales, row_step);
  PIA_HIP(hipGetLastError());
}

void launch_widen_rows_bf16(const uint16_t* w, int64_t rows, int64_t cols, float* out, int64_t ldo, int64_t row_step,
                            hipStream_t st) {
  if (rows == 0) return;
  PIA_REQUIRE(rows < (int64_t(1) << 31), "widen: too many rows");
  PIA_REQUIRE(ldo >= cols && row_step >= 1, "widen: bad destination pitch");
  hipLaunchKernelGGL(k_widen_rows, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, st, w, cols, out, ldo,
                     row_step);
  PIA_HIP(hipGetLastError());
}

namespace {
__global__ __launch_bounds__(kThreads) void k_table_patch(int32_t* __restrict__ tab, const int32_t* __restrict__ patch,
                                                          int n) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i < n) tab[patch[2 * i]] = patch[2 * i + 1];
}
}  // namespace

void launch_table_patch(int32_t* tab, const int32_t* patch, int64_t n, hipStream_t st) {
  PIA_REQUIRE(n >= 0 && n < (int64_t(1) << 30), "table patch: bad count");
  if (n == 0) return;
  hipLaunchKernelGGL(k_table_patch, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, st,
                     tab, patch, static_cast<int>(n));
  PIA_HIP(hipGetLastError());
}

void launch_copy_block(float* kv, const pia_kv_layout& L, int64_t src, int64_t dst, hipStream_t st) {
  PIA_REQUIRE(src != dst, "copy_block called with src == dst");
  PIA_REQUIRE(src >= 0 && dst >= 0 && src < L.num_blocks && dst < L.num_blocks, "copy_block: block out of range");
  const int64_t stride = L.block_size * L.num_kv_heads * 2 * L.head_dim;
  PIA_REQUIRE(stride % 4 == 0, "copy_block: block stride must be a multiple of 4 floats");
  const int64_t chunks = (stride / 4 + kThreads - 1) / kThreads;
  dim3 grid(static_cast<unsigned>(std::min<int64_t>(chunks, 64)), static_cast<unsigned>(L.num_layers));
  hipLaunchKernelGGL(k_copy_block, grid, dim3(kThreads), 0, st, kv, L.num_blocks, stride, src, dst);
  PIA_HIP(hipGetLastError());
}

}  // namespace pia

namespace pia {
namespace {
__global__ void k_spin(uint64_t ticks) {
  const uint64_t t0 = wall_clock64();
  while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(32);
}
}  // namespace

void launch_spin(double us, hipStream_t st) {
  PIA_REQUIRE(us >= 0 && us <= 20000, "spin: at most 20 ms");
  static int rate_khz = 0;
  if (!rate_khz) {
    int dev = 0;
    PIA_HIP(hipGetDevice(&dev));
    PIA_HIP(hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, dev));
    if (rate_khz <= 0) rate_khz = 100000;
  }
  const uint64_t ticks = static_cast<uint64_t>(us * rate_khz / 1000.0);
  hipLaunchKernelGGL(k_spin, dim3(1), dim3(1), 0, st, ticks);
  PIA_HIP(hipGetLastError());
}
}  // namespace pia
