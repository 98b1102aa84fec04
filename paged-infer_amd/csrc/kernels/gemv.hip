// Weight-streaming projection for small decode batches: one wavefront owns R output rows;
// each lane streams VEC contiguous weight elements per step (16 int8 = one 128-bit load),
// widens them in registers and accumulates in f32 against the activation vectors of the
// batch, so every weight byte is fetched from HBM once per launch. The per-row scale is
// applied after the wavefront reduction, as the reference does (src/math.rs:486-492:
// dot_i8(row, x) * scale).
//
// Fusions (each removes a launch and a round trip of the activations through HBM):
//   - prologue RMSNorm (src/math.rs:4-22): when `norm_w` is given the workgroup computes
//     1/rms of every batch row itself and normalizes x on the fly;
//   - epilogue residual add (src/model.rs:1127-1129, 1165-1167): out += proj;
//   - epilogue SwiGLU (src/math.rs:293-302): gate and up rows are interleaved in HBM
//     (row 2i = gate i, row 2i+1 = up i) and the wave that owns both writes silu(g) * u.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace pia {
namespace {

// Raw weight registers for VEC elements, loaded with one vector instruction, widened later.
template <typename TW, int VEC>
struct Raw;
template <>
struct Raw<int8_t, 16> {
  int4 v;
  __device__ void load(const int8_t* p) { v = *reinterpret_cast<const int4*>(p); }
  __device__ void zero() { v = make_int4(0, 0, 0, 0); }
  __device__ void widen(float (&w)[16]) const {
    const int d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) w[4 * k + j] = static_cast<float>((d[k] << (24 - 8 * j)) >> 24);
  }
};
template <>
struct Raw<int8_t, 4> {
  int v;
  __device__ void load(const int8_t* p) { v = *reinterpret_cast<const int*>(p); }
  __device__ void zero() { v = 0; }
  __device__ void widen(float (&w)[4]) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = static_cast<float>((v << (24 - 8 * j)) >> 24);
  }
};
template <>
struct Raw<int8_t, 1> {
  int8_t v;
  __device__ void load(const int8_t* p) { v = *p; }
  __device__ void zero() { v = 0; }
  __device__ void widen(float (&w)[1]) const { w[0] = static_cast<float>(v); }
};
template <>
struct Raw<float, 4> {
  float4 v;
  __device__ void load(const float* p) { v = *reinterpret_cast<const float4*>(p); }
  __device__ void zero() { v = make_float4(0.f, 0.f, 0.f, 0.f); }
  __device__ void widen(float (&w)[4]) const { w[0] = v.x, w[1] = v.y, w[2] = v.z, w[3] = v.w; }
};
template <>
struct Raw<float, 1> {
  float v;
  __device__ void load(const float* p) { v = *p; }
  __device__ void zero() { v = 0.f; }
  __device__ void widen(float (&w)[1]) const { w[0] = v; }
};

template <int VEC>
__device__ inline void load_x(const float* p, float (&x)[VEC]) {
  if constexpr (VEC % 4 == 0) {
#pragma unroll
    for (int k = 0; k < VEC / 4; ++k) {
      const float4 v = reinterpret_cast<const float4*>(p)[k];
      x[4 * k] = v.x, x[4 * k + 1] = v.y, x[4 * k + 2] = v.z, x[4 * k + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < VEC; ++k) x[k] = p[k];
  }
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

constexpr int kWaves = 4;  // wavefronts per workgroup
constexpr int64_t kMaxStagedCols = 16384;  // batch-1 vectors up to this length are staged in LDS
constexpr int kMaxNormBatch = 64;
constexpr int64_t kMaxGemvnBatch = 4;  // batches up to this size take the LDS-staged kernel
static_assert(kMaxGemvnBatch <= 4, "launch_gemvn instantiates groups of up to 4 rows");

enum { kEpiStore = 0, kEpiAdd = 1, kEpiSwiglu = 2 };

// f32 -> u32 preserving f32::total_cmp order (src/sampling.rs:140-147 compares with total_cmp).
__device__ inline uint32_t order_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ inline unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const unsigned long long o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

// UNR chunks of 64*VEC columns per load batch: every weight load of a batch is issued before
// the first use, so a wavefront pays one HBM round trip per batch, not one per chunk.
template <typename TW, int VEC, int R, int NB, int UNR, int EPI, bool NORM, bool AMAX>
__global__ __launch_bounds__(64 * kWaves) void k_gemv(const TW* __restrict__ W, int64_t ldw,
                                                      const float* __restrict__ S, const float* __restrict__ X,
                                                      int64_t ldx, const float* __restrict__ NW, float eps,
                                                      float* __restrict__ O, int64_t osb, int64_t osr, int rows,
                                                      int cols, int batch, unsigned long long* __restrict__ amax) {
  __shared__ float inv_s[NORM ? kMaxNormBatch : 1];
  __shared__ float red[kWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * kWaves + wave) * R;
  const TW* wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) wrow[r] = W + static_cast<int64_t>(min(row0 + r, rows - 1)) * ldw;
  const int main_cols = cols - cols % VEC;
  const int rem = cols - main_cols;
  constexpr int kStep = 64 * VEC * UNR;

  Raw<TW, VEC> raw[UNR][R];
  auto load_batch = [&](int base) {
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int c = base + (u * 64 + lane) * VEC;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (c < main_cols) raw[u][r].load(wrow[r] + c);
        else raw[u][r].zero();
      }
    }
  };
  load_batch(0);  // in flight while the RMSNorm prologue runs

  if constexpr (NORM) {
    // 1/rms of each batch row (src/math.rs:12-18), computed by the whole workgroup; the row is
    // read with 16-byte loads, all in flight together (cols % 4 == 0 on this path).
    for (int b = 0; b < batch; ++b) {
      const float* xr = X + static_cast<int64_t>(b) * ldx;
      float ss = 0.0f;
      if (cols % 4 == 0 && (reinterpret_cast<uintptr_t>(xr) & 15) == 0) {
        const float4* x4 = reinterpret_cast<const float4*>(xr);
        const int n4 = cols / 4;
        for (int i0 = threadIdx.x; i0 < n4; i0 += 4 * 64 * kWaves) {
          float4 v[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int i = i0 + u * 64 * kWaves;
            v[u] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) ss += v[u].x * v[u].x + v[u].y * v[u].y + v[u].z * v[u].z + v[u].w * v[u].w;
        }
      } else {
        for (int i = threadIdx.x; i < cols; i += 64 * kWaves) ss += xr[i] * xr[i];
      }
      ss = wave_sum(ss);
      if (lane == 0) red[wave] = ss;
      __syncthreads();
      if (threadIdx.x == 0) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) t += red[w];
        inv_s[b] = 1.0f / sqrtf(t / static_cast<float>(cols) + eps);
      }
      __syncthreads();
    }
  }
  if (row0 >= rows) return;

  for (int b0 = 0; b0 < batch; b0 += NB) {
    float acc[R][NB];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[r][b] = 0.0f;

    for (int base = 0; base < main_cols; base += kStep) {
      if (base != 0 || b0 != 0) load_batch(base);
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const int c = base + (u * 64 + lane) * VEC;
        if (c < main_cols) {
          float nw[VEC];
          if constexpr (NORM) load_x<VEC>(NW + c, nw);
          float w[R][VEC];
#pragma unroll
          for (int r = 0; r < R; ++r) raw[u][r].widen(w[r]);
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            if (b0 + b < batch) {
              float xv[VEC];
              load_x<VEC>(X + static_cast<int64_t>(b0 + b) * ldx + c, xv);
              if constexpr (NORM) {
                const float inv = inv_s[b0 + b];
#pragma unroll
                for (int j = 0; j < VEC; ++j) xv[j] = (xv[j] * inv) * nw[j];
              }
#pragma unroll
              for (int r = 0; r < R; ++r)
#pragma unroll
                for (int j = 0; j < VEC; ++j) acc[r][b] = __builtin_fmaf(w[r][j], xv[j], acc[r][b]);
            }
          }
        }
      }
    }
    if (lane < rem) {
      const int c = main_cols + lane;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b0 + b < batch) {
          float xv = X[static_cast<int64_t>(b0 + b) * ldx + c];
          if constexpr (NORM) xv = (xv * inv_s[b0 + b]) * NW[c];
#pragma unroll
          for (int r = 0; r < R; ++r) acc[r][b] = __builtin_fmaf(static_cast<float>(wrow[r][c]), xv, acc[r][b]);
        }
      }
    }

    float mine = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float s = wave_sum(acc[r][b]);
        if (lane == r * NB + b) mine = s;
      }
    const int r_l = lane / NB, b_l = lane % NB;
    const int row = row0 + r_l, bb = b0 + b_l;
    if constexpr (EPI == kEpiSwiglu) {
      // Lanes (r, b) and (r + 1, b) hold the gate and up results of output row (row0 + r) / 2.
      const float up = __shfl_down(mine, NB, 64);
      if (lane < R * NB && (r_l & 1) == 0 && row + 1 < rows && bb < batch) {
        const float g = S ? mine * S[row] : mine;
        const float u = S ? up * S[row + 1] : up;
        const float silu = g / (1.0f + expf(-g));
        O[static_cast<int64_t>(bb) * osb + static_cast<int64_t>(row >> 1) * osr] = silu * u;
      }
    } else {
      const bool valid = lane < R * NB && row < rows && bb < batch;
      float v = 0.0f;
      if (valid) {
        v = S ? mine * S[row] : mine;
        float* o = O + static_cast<int64_t>(bb) * osb + static_cast<int64_t>(row) * osr;
        if (EPI == kEpiAdd) *o = *o + v;
        else *o = v;
      }
      if constexpr (AMAX) {
        // Greedy argmax fused into the LM head: max of (order key, row) per batch row; ties in
        // the key keep the larger row, i.e. the last maximal index.
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          unsigned long long cand = 0;
          if (valid && b_l == b)
            cand = (static_cast<unsigned long long>(order_key(v)) << 32) | static_cast<uint32_t>(row);
          cand = wave_max_u64(cand);
          if (lane == 0 && b0 + b < batch)
            atomicMax(&amax[(b0 + b) * kArgmaxSlots + ((blockIdx.x * kWaves + wave) & (kArgmaxSlots - 1))], cand);
        }
      }
    }
  }
}

// Batch-1 int8 projection with the activation vector staged once per workgroup in LDS.
// The vector's loads (and the norm weights') are issued before the weight loads, so the
// RMSNorm reduction runs while the weights are in flight; the main loop then reads the
// normalized vector from LDS instead of L2. LDS layout: column c at c + 4 * (c / 64), which
// makes each lane's 16 consecutive floats start on a distinct group of banks.
constexpr int kXPre = 8;  // float4 of the vector per thread loaded before the weights
__device__ inline int xs_index(int c) { return c + ((c >> 6) << 2); }

template <int R, int UNR, int EPI, bool NORM, bool AMAX>
__global__ __launch_bounds__(64 * kWaves) void k_gemv1(const int8_t* __restrict__ W, int64_t ldw,
                                                       const float* __restrict__ S, const float* __restrict__ X,
                                                       const float* __restrict__ NW, float eps, float* __restrict__ O,
                                                       int64_t osr, int rows, int cols,
                                                       unsigned long long* __restrict__ amax) {
  extern __shared__ __align__(16) float xs[];
  __shared__ float red[kWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * kWaves + wave) * R;
  constexpr int kStep = 64 * 16 * UNR;
  const int n4 = cols >> 2;                              // cols % 4 == 0 on this path
  const int kpad = (cols + 1023) / 1024 * 1024;          // zero padded to whole 1024-column chunks
  const float4* X4 = reinterpret_cast<const float4*>(X);
  const float4* NW4 = reinterpret_cast<const float4*>(NW);

  // 1. The vector (and norm weights): the first kXPre float4 per thread.
  float4 xv[kXPre], wv[kXPre];
#pragma unroll
  for (int u = 0; u < kXPre; ++u) {
    const int i = threadIdx.x + u * 64 * kWaves;
    xv[u] = i < n4 ? X4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (NORM) wv[u] = i < n4 ? NW4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  // 2. The first batch of weights.
  const int8_t* wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) wrow[r] = W + static_cast<int64_t>(min(row0 + r, rows - 1)) * ldw;
  Raw<int8_t, 16> raw[UNR][R];
  auto load_batch = [&](int base) {
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int c = base + (u * 64 + lane) * 16;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (c < cols) raw[u][r].load(wrow[r] + c);
        else raw[u][r].zero();
      }
    }
  };
  load_batch(0);
  // 3. Vector into LDS (the rest of a long vector now), sum of squares, zero padding.
  float ss = 0.0f;
  auto put4 = [&](int i, float4 v) {
    float* d = xs + xs_index(4 * i);
    d[0] = v.x, d[1] = v.y, d[2] = v.z, d[3] = v.w;
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  };
#pragma unroll
  for (int u = 0; u < kXPre; ++u) {
    const int i = threadIdx.x + u * 64 * kWaves;
    if (i < n4) put4(i, xv[u]);
  }
  for (int i = threadIdx.x + kXPre * 64 * kWaves; i < n4; i += 64 * kWaves) put4(i, X4[i]);
  for (int c = cols + threadIdx.x; c < kpad; c += 64 * kWaves) xs[xs_index(c)] = 0.0f;
  if constexpr (NORM) {
    // RMSNorm (src/math.rs:4-22): x * (1/rms) * w, in that order.
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) t += red[w];
    const float inv = 1.0f / sqrtf(t / static_cast<float>(cols) + eps);
    auto norm4 = [&](int i, float4 v, float4 w) {
      float* d = xs + xs_index(4 * i);
      d[0] = (v.x * inv) * w.x, d[1] = (v.y * inv) * w.y, d[2] = (v.z * inv) * w.z, d[3] = (v.w * inv) * w.w;
    };
#pragma unroll
    for (int u = 0; u < kXPre; ++u) {
      const int i = threadIdx.x + u * 64 * kWaves;
      if (i < n4) norm4(i, xv[u], wv[u]);
    }
    for (int i = threadIdx.x + kXPre * 64 * kWaves; i < n4; i += 64 * kWaves) {
      const float* d = xs + xs_index(4 * i);
      norm4(i, make_float4(d[0], d[1], d[2], d[3]), NW4[i]);
    }
  }
  __syncthreads();
  // Waves past the last row skip the work but stay for the workgroup's argmax reduction.
  const bool active = row0 < rows;

  // 4. Stream the rows against the staged vector.
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  for (int base = 0; active && base < cols; base += kStep) {
    if (base != 0) load_batch(base);
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int c = base + (u * 64 + lane) * 16;
      if (c < cols) {
        float x16[16];
        const float4* xp = reinterpret_cast<const float4*>(xs + xs_index(c));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 v = xp[q];
          x16[4 * q] = v.x, x16[4 * q + 1] = v.y, x16[4 * q + 2] = v.z, x16[4 * q + 3] = v.w;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float w[16];
          raw[u][r].widen(w);
#pragma unroll
          for (int j = 0; j < 16; ++j) acc[r] = __builtin_fmaf(w[j], x16[j], acc[r]);
        }
      }
    }
  }
  float mine = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float s = wave_sum(acc[r]);
    if (lane == r) mine = s;
  }
  const int row = row0 + lane;
  if constexpr (EPI == kEpiSwiglu) {
    // Lanes r and r + 1 hold the gate and up results of output row (row0 + r) / 2.
    const float up = __shfl_down(mine, 1, 64);
    if (active && lane < R && (lane & 1) == 0 && row + 1 < rows) {
      const float g = mine * S[row];
      const float u = up * S[row + 1];
      const float silu = g / (1.0f + expf(-g));
      O[static_cast<int64_t>(row >> 1) * osr] = silu * u;
    }
  } else {
    const bool valid = active && lane < R && row < rows;
    float v = 0.0f;
    if (valid) {
      v = mine * S[row];
      float* o = O + static_cast<int64_t>(row) * osr;
      if (EPI == kEpiAdd) *o = *o + v;
      else *o = v;
    }
    if constexpr (AMAX) {
      // Greedy argmax: max of (order key, row) over the workgroup's rows, then one atomic per
      // workgroup into one of the slots.
      __shared__ unsigned long long wbest[kWaves];
      unsigned long long cand = valid ? (static_cast<unsigned long long>(order_key(v)) << 32) | static_cast<uint32_t>(row) : 0ull;
      cand = wave_max_u64(cand);
      if (lane == 0) wbest[wave] = cand;
      __syncthreads();
      if (threadIdx.x == 0) {
        unsigned long long m = wbest[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) m = wbest[w] > m ? wbest[w] : m;
        if (m) atomicMax(&amax[blockIdx.x & (kArgmaxSlots - 1)], m);
      }
    }
  }
}

template <int R, int UNR, int EPI>
void go1(const GemvArgs& g, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((g.rows + kWaves * R - 1) / (kWaves * R)));
  const int kpad = static_cast<int>((g.cols + 1023) / 1024 * 1024);
  const size_t smem = static_cast<size_t>(kpad + kpad / 16) * 4;
  const auto* w = static_cast<const int8_t*>(g.W);
#define PIA_GEMV1(NORM, AMAX)                                                                                \
  do {                                                                                                       \
    static bool raised = false;                                                                              \
    if (!raised && smem > 65536) {                                                                           \
      PIA_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemv1<R, UNR, EPI, NORM, AMAX>),           \
                                  hipFuncAttributeMaxDynamicSharedMemorySize,                                \
                                  static_cast<int>((kMaxStagedCols + kMaxStagedCols / 16) * 4)));            \
      raised = true;                                                                                         \
    }                                                                                                        \
    hipLaunchKernelGGL((k_gemv1<R, UNR, EPI, NORM, AMAX>), grid, dim3(64 * kWaves), smem, st, w, g.ldw,      \
                       g.scales, g.x, g.norm_w, g.eps, g.out, g.osr, static_cast<int>(g.rows),               \
                       static_cast<int>(g.cols), g.amax);                                                    \
  } while (0)
  if constexpr (EPI == kEpiStore) {
    if (g.amax) {
      if (g.norm_w) PIA_GEMV1(true, true);
      else PIA_GEMV1(false, true);
      return;
    }
  }
  if (g.norm_w) PIA_GEMV1(true, false);
  else PIA_GEMV1(false, false);
#undef PIA_GEMV1
}

template <int R, int UNR>
void go1_epi(const GemvArgs& g, hipStream_t st) {
  if (g.epi == Epi::Add) go1<R, UNR, kEpiAdd>(g, st);
  else if (g.epi == Epi::Swiglu) go1<R, UNR, kEpiSwiglu>(g, st);
  else go1<R, UNR, kEpiStore>(g, st);
}

template <int R>
void go1_unr(const GemvArgs& g, hipStream_t st) {
  const int64_t chunks = (g.cols / 16 + 63) / 64;
  if (chunks <= 1) go1_epi<R, 1>(g, st);
  else if (chunks <= 2) go1_epi<R, 2>(g, st);
  else if (chunks <= 4) go1_epi<R, 4>(g, st);
  else if (chunks <= 6) go1_epi<R, 6>(g, st);
  else go1_epi<R, 8>(g, st);
}

// Small-batch (2..NB rows) int8 projection: the batch-1 kernel's scheme with every batch row
// staged in LDS (normalized there when RMSNorm is fused), so each weight byte is fetched once
// and applied to all NB rows from registers. Row b of the batch lives at xs + b * stride.
constexpr int64_t kMaxGemvnSmem = 156 * 1024;  // LDS a workgroup of this kernel may take

__host__ __device__ inline int64_t gemvn_stride(int64_t cols) {
  const int64_t kpad = (cols + 1023) / 1024 * 1024;
  return kpad + kpad / 16;
}

template <int R, int NB, int UNR, int EPI, bool NORM, bool AMAX>
__global__ __launch_bounds__(64 * kWaves) void k_gemvn(const int8_t* __restrict__ W, int64_t ldw,
                                                       const float* __restrict__ S, const float* __restrict__ X,
                                                       int64_t ldx, const float* __restrict__ NW, float eps,
                                                       float* __restrict__ O, int64_t osb, int64_t osr, int rows,
                                                       int cols, int batch, unsigned long long* __restrict__ amax) {
  extern __shared__ __align__(16) float xs[];
  __shared__ float red[NB][kWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * kWaves + wave) * R;
  constexpr int kStep = 64 * 16 * UNR;
  const int n4 = cols >> 2;
  const int kpad = (cols + 1023) / 1024 * 1024;
  const int stride = static_cast<int>(gemvn_stride(cols));

  // 1. The first batch of weights, in flight while the activations are staged.
  const int8_t* wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) wrow[r] = W + static_cast<int64_t>(min(row0 + r, rows - 1)) * ldw;
  Raw<int8_t, 16> raw[UNR][R];
  auto load_batch = [&](int base) {
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int c = base + (u * 64 + lane) * 16;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (c < cols) raw[u][r].load(wrow[r] + c);
        else raw[u][r].zero();
      }
    }
  };
  load_batch(0);

  // 2. Activation rows into LDS (zeros for rows past `batch` and for the column padding), with
  // each row's sum of squares.
  float ss[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    ss[b] = 0.0f;
    float* xb = xs + b * stride;
    const float4* X4 = reinterpret_cast<const float4*>(X + static_cast<int64_t>(b) * ldx);
    for (int i = threadIdx.x; i < n4; i += 64 * kWaves) {
      const float4 v = b < batch ? X4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      float* d = xb + xs_index(4 * i);
      d[0] = v.x, d[1] = v.y, d[2] = v.z, d[3] = v.w;
      ss[b] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    for (int c = cols + threadIdx.x; c < kpad; c += 64 * kWaves) xb[xs_index(c)] = 0.0f;
  }
  if constexpr (NORM) {
    // RMSNorm (src/math.rs:4-22) of every row: x * (1/rms) * w, in that order.
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float t = wave_sum(ss[b]);
      if (lane == 0) red[b][wave] = t;
    }
    __syncthreads();
    const float4* NW4 = reinterpret_cast<const float4*>(NW);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float t = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) t += red[b][w];
      const float inv = 1.0f / sqrtf(t / static_cast<float>(cols) + eps);
      float* xb = xs + b * stride;
      for (int i = threadIdx.x; i < n4; i += 64 * kWaves) {
        float* d = xb + xs_index(4 * i);
        const float4 w = NW4[i];
        d[0] = (d[0] * inv) * w.x, d[1] = (d[1] * inv) * w.y, d[2] = (d[2] * inv) * w.z, d[3] = (d[3] * inv) * w.w;
      }
    }
  }
  __syncthreads();
  const bool active = row0 < rows;

  // 3. Stream the rows against the staged batch.
  float acc[R][NB];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[r][b] = 0.0f;
  for (int base = 0; active && base < cols; base += kStep) {
    if (base != 0) load_batch(base);
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int c = base + (u * 64 + lane) * 16;
      if (c < cols) {
        float w[R][16];
#pragma unroll
        for (int r = 0; r < R; ++r) raw[u][r].widen(w[r]);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const float4* xp = reinterpret_cast<const float4*>(xs + b * stride + xs_index(c));
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float4 v = xp[q];
#pragma unroll
            for (int r = 0; r < R; ++r) {
              acc[r][b] = __builtin_fmaf(w[r][4 * q], v.x, acc[r][b]);
              acc[r][b] = __builtin_fmaf(w[r][4 * q + 1], v.y, acc[r][b]);
              acc[r][b] = __builtin_fmaf(w[r][4 * q + 2], v.z, acc[r][b]);
              acc[r][b] = __builtin_fmaf(w[r][4 * q + 3], v.w, acc[r][b]);
            }
          }
        }
      }
    }
  }

  // 4. Lane r * NB + b holds row0 + r for batch row b.
  float mine = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float t = wave_sum(acc[r][b]);
      if (lane == r * NB + b) mine = t;
    }
  const int r_l = lane / NB, b_l = lane % NB;
  const int row = row0 + r_l;
  if constexpr (EPI == kEpiSwiglu) {
    const float up = __shfl_down(mine, NB, 64);
    if (active && lane < R * NB && (r_l & 1) == 0 && row + 1 < rows && b_l < batch) {
      const float g = mine * S[row];
      const float u = up * S[row + 1];
      const float silu = g / (1.0f + expf(-g));
      O[static_cast<int64_t>(b_l) * osb + static_cast<int64_t>(row >> 1) * osr] = silu * u;
    }
  } else {
    const bool valid = active && lane < R * NB && row < rows && b_l < batch;
    float v = 0.0f;
    if (valid) {
      v = mine * S[row];
      float* o = O + static_cast<int64_t>(b_l) * osb + static_cast<int64_t>(row) * osr;
      if (EPI == kEpiAdd) *o = *o + v;
      else *o = v;
    }
    if constexpr (AMAX) {
      // Per batch row: max of (order key, row) over the workgroup, one atomic per row.
      __shared__ unsigned long long wbest[NB][kWaves];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        unsigned long long cand = 0;
        if (valid && b_l == b)
          cand = (static_cast<unsigned long long>(order_key(v)) << 32) | static_cast<uint32_t>(row);
        cand = wave_max_u64(cand);
        if (lane == 0) wbest[b][wave] = cand;
      }
      __syncthreads();
      if (threadIdx.x < NB && static_cast<int>(threadIdx.x) < batch) {
        unsigned long long m = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) m = wbest[threadIdx.x][w] > m ? wbest[threadIdx.x][w] : m;
        if (m) atomicMax(&amax[threadIdx.x * kArgmaxSlots + (blockIdx.x & (kArgmaxSlots - 1))], m);
      }
    }
  }
}

template <int R, int NB, int UNR, int EPI>
void gon(const GemvArgs& g, int64_t b0, int64_t nb, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((g.rows + kWaves * R - 1) / (kWaves * R)));
  const size_t smem = static_cast<size_t>(NB * gemvn_stride(g.cols)) * 4;
  const auto* w = static_cast<const int8_t*>(g.W);
  const float* x = g.x + b0 * g.ldx;
  float* o = g.out + b0 * g.osb;
  unsigned long long* am = g.amax ? g.amax + b0 * kArgmaxSlots : nullptr;
#define PIA_GEMVN(NORM, AMAX)                                                                                \
  do {                                                                                                       \
    static bool raised = false;                                                                              \
    if (!raised) {                                                                                           \
      PIA_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemvn<R, NB, UNR, EPI, NORM, AMAX>),       \
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kMaxGemvnSmem))); \
      raised = true;                                                                                         \
    }                                                                                                        \
    hipLaunchKernelGGL((k_gemvn<R, NB, UNR, EPI, NORM, AMAX>), grid, dim3(64 * kWaves), smem, st, w, g.ldw,  \
                       g.scales, x, g.ldx, g.norm_w, g.eps, o, g.osb, g.osr, static_cast<int>(g.rows),        \
                       static_cast<int>(g.cols), static_cast<int>(nb), am);                                  \
  } while (0)
  if constexpr (EPI == kEpiStore) {
    if (g.amax) {
      if (g.norm_w) PIA_GEMVN(true, true);
      else PIA_GEMVN(false, true);
      return;
    }
  }
  if (g.norm_w) PIA_GEMVN(true, false);
  else PIA_GEMVN(false, false);
#undef PIA_GEMVN
}

template <int R, int NB, int UNR>
void gon_epi(const GemvArgs& g, int64_t b0, int64_t nb, hipStream_t st) {
  if (g.epi == Epi::Add) gon<R, NB, UNR, kEpiAdd>(g, b0, nb, st);
  else if (g.epi == Epi::Swiglu) gon<R, NB, UNR, kEpiSwiglu>(g, b0, nb, st);
  else gon<R, NB, UNR, kEpiStore>(g, b0, nb, st);
}

template <int NB>
void gon_nb(const GemvArgs& g, int64_t b0, int64_t nb, hipStream_t st) {
  // 4 rows per wavefront for tall matrices, 2 otherwise; batches of up to 4 column chunks
  // per lane in flight (the NB accumulators per row take the registers UNR 8 would).
  const int64_t chunks = (g.cols / 16 + 63) / 64;
  if (g.rows >= 4 * kWaves * 512) {
    if (chunks <= 2) gon_epi<4, NB, 2>(g, b0, nb, st);
    else gon_epi<4, NB, 4>(g, b0, nb, st);
  } else {
    if (chunks <= 2) gon_epi<2, NB, 2>(g, b0, nb, st);
    else gon_epi<2, NB, 4>(g, b0, nb, st);
  }
}

// The batch (at most kMaxGemvnBatch rows) in groups of at most 4 rows whose staged activations
// fit in LDS.
void launch_gemvn(const GemvArgs& g, hipStream_t st) {
  const int64_t row_bytes = gemvn_stride(g.cols) * 4;
  int64_t nb_max = 4;
  while (nb_max > 1 && nb_max * row_bytes > kMaxGemvnSmem) nb_max /= 2;
  for (int64_t b0 = 0; b0 < g.batch; b0 += nb_max) {
    const int64_t nb = std::min<int64_t>(nb_max, g.batch - b0);
    if (nb <= 2) gon_nb<2>(g, b0, nb, st);
    else gon_nb<4>(g, b0, nb, st);
  }
}

struct Launch {
  const void* W;
  int64_t ldw;
  const float* S;
  const float* X;
  int64_t ldx;
  const float* NW;
  float eps;
  float* O;
  int64_t osb, osr;
  int rows, cols, batch;
  unsigned long long* amax;
  hipStream_t st;
};

template <typename TW, int VEC, int R, int NB, int UNR, int EPI>
void go(const Launch& a) {
  dim3 grid((a.rows + kWaves * R - 1) / (kWaves * R));
  const TW* w = static_cast<const TW*>(a.W);
#define PIA_GEMV_LAUNCH(NORM, AMAX)                                                                       \
  hipLaunchKernelGGL((k_gemv<TW, VEC, R, NB, UNR, EPI, NORM, AMAX>), grid, dim3(64 * kWaves), 0, a.st, w, \
                     a.ldw, a.S, a.X, a.ldx, a.NW, a.eps, a.O, a.osb, a.osr, a.rows, a.cols, a.batch, a.amax)
  if constexpr (EPI == kEpiStore) {
    if (a.amax) {
      if (a.NW) PIA_GEMV_LAUNCH(true, true);
      else PIA_GEMV_LAUNCH(false, true);
      return;
    }
  }
  if (a.NW) PIA_GEMV_LAUNCH(true, false);
  else PIA_GEMV_LAUNCH(false, false);
#undef PIA_GEMV_LAUNCH
}

template <typename TW, int VEC, int R, int NB, int UNR>
void by_epi(const Launch& a, Epi epi) {
  if (epi == Epi::Add) go<TW, VEC, R, NB, UNR, kEpiAdd>(a);
  else if (epi == Epi::Swiglu) go<TW, VEC, R, NB, UNR, kEpiSwiglu>(a);
  else go<TW, VEC, R, NB, UNR, kEpiStore>(a);
}

template <typename TW, int VEC, int R, int NB>
void by_unr(const Launch& a, Epi epi) {
  // Chunks of 64*VEC columns a lane covers; batches of up to 8 chunks in flight per lane.
  const int chunks = (a.cols / VEC + 63) / 64;
  if (chunks <= 1) by_epi<TW, VEC, R, NB, 1>(a, epi);
  else if (chunks <= 2) by_epi<TW, VEC, R, NB, 2>(a, epi);
  else if (chunks <= 4) by_epi<TW, VEC, R, NB, 4>(a, epi);
  else if (chunks <= 6) by_epi<TW, VEC, R, NB, 6>(a, epi);
  else by_epi<TW, VEC, R, NB, 8>(a, epi);
}

template <typename TW, int VEC, int R>
void by_nb(const Launch& a, Epi epi) {
  if (a.batch == 1) by_unr<TW, VEC, R, 1>(a, epi);
  else if (a.batch == 2) by_unr<TW, VEC, R, 2>(a, epi);
  else by_unr<TW, VEC, R, 4>(a, epi);
}

template <typename TW, int VEC>
void by_r(const Launch& a, Epi epi) {
  // 4 rows per wavefront for tall matrices; 2 when that would leave CUs idle (2 is the
  // smallest tile that keeps a SwiGLU gate/up pair in one wavefront).
  if (a.rows >= 4 * kWaves * 512) by_nb<TW, VEC, 4>(a, epi);
  else by_nb<TW, VEC, 2>(a, epi);
}

inline bool aligned(const void* p, int64_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace

void launch_gemv(const GemvArgs& g, hipStream_t st) {
  PIA_REQUIRE(g.rows > 0 && g.cols > 0 && g.batch > 0, "gemv: empty shape");
  PIA_REQUIRE(g.rows < (int64_t(1) << 31) && g.cols < (int64_t(1) << 31) && g.batch < (int64_t(1) << 31),
              "gemv: shape exceeds int32 indexing");
  PIA_REQUIRE(g.ldw >= g.cols && g.ldx >= g.cols, "gemv: leading dimension smaller than cols");
  PIA_REQUIRE(!g.norm_w || g.batch <= kMaxNormBatch, "gemv: fused RMSNorm supports at most 64 rows");
  PIA_REQUIRE(g.epi != Epi::Swiglu || g.rows % 2 == 0, "gemv: SwiGLU epilogue needs interleaved row pairs");
  PIA_REQUIRE(!g.amax || g.epi == Epi::Store, "gemv: fused argmax needs the Store epilogue");
  Launch a{g.W, g.ldw, g.scales, g.x, g.ldx, g.norm_w, g.eps, g.out, g.osb, g.osr,
           static_cast<int>(g.rows), static_cast<int>(g.cols), static_cast<int>(g.batch), g.amax, st};
  const bool xv16 = g.ldx % 16 == 0 && aligned(g.x, 64) && (!g.norm_w || aligned(g.norm_w, 64));
  const bool xv4 = g.ldx % 4 == 0 && aligned(g.x, 16) && (!g.norm_w || aligned(g.norm_w, 16));
  if (g.wkind == 1 && g.batch == 1 && g.cols % 16 == 0 && g.ldw % 16 == 0 && aligned(g.W, 16) && aligned(g.x, 16) &&
      (!g.norm_w || aligned(g.norm_w, 16)) && g.cols <= kMaxStagedCols) {
    PIA_REQUIRE(g.scales != nullptr, "gemv: int8 weights need scales");
    if (g.rows >= 4 * kWaves * 512) go1_unr<4>(g, st);
    else go1_unr<2>(g, st);
    PIA_HIP(hipGetLastError());
    return;
  }
  if (g.wkind == 1 && g.batch > 1 && g.batch <= kMaxGemvnBatch && g.cols % 16 == 0 && g.ldw % 16 == 0 &&
      aligned(g.W, 16) && g.ldx % 4 == 0 && aligned(g.x, 16) && (!g.norm_w || aligned(g.norm_w, 16)) &&
      2 * gemvn_stride(g.cols) * 4 <= kMaxGemvnSmem) {
    PIA_REQUIRE(g.scales != nullptr, "gemv: int8 weights need scales");
    launch_gemvn(g, st);
    PIA_HIP(hipGetLastError());
    return;
  }
  if (g.wkind == 1) {
    PIA_REQUIRE(g.scales != nullptr, "gemv: int8 weights need scales");
    if (g.ldw % 16 == 0 && aligned(g.W, 16) && xv16) by_r<int8_t, 16>(a, g.epi);
    else if (g.ldw % 4 == 0 && aligned(g.W, 4) && xv4) by_r<int8_t, 4>(a, g.epi);
    else by_r<int8_t, 1>(a, g.epi);
  } else {
    if (g.ldw % 4 == 0 && aligned(g.W, 16) && xv4) by_r<float, 4>(a, g.epi);
    else by_r<float, 1>(a, g.epi);
  }
  PIA_HIP(hipGetLastError());
}

}  // namespace pia
