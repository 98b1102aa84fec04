// Batched int8 projection on the matrix cores (decode batches >= 8 and prefill).
//
// The reference multiplies int8 weights by f32 activations in f32 (src/math.rs:223-275). On
// gfx950 the int8 matrix core (v_mfma_i32_16x16x64_i8) is 2x the bf16 rate and consumes the
// stored weights as they are, with no widening. To feed it f32 activations without losing
// f32-level accuracy, each activation row x_b is written in 23-bit fixed point relative to its
// own power-of-two range, v = rint(x * 2^(22 - e_b)) with max|x_b| < 2^e_b, and v is split
// into three signed base-256 digits, v = d0 + 256 d1 + 65536 d2. Each digit is an int8
// column of the B operand, so one MFMA pass computes sum_k W[r][k] * d_j[b][k] for all three
// digits exactly in int32. The epilogue recombines y = (C0 + 256 C1 + 65536 C2) * 2^(e_b-22)
// * scale[r]. The only rounding is the fixed-point image of x (|error| <= 2^-23 max|x_b| per
// element) and the final conversion -- tighter than an f32 accumulation of the same dot.
#include <cmath>

#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace pia {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
// Whole 64-entry chunks from which the LDS-tiled kernel takes over (prefill sizes).
constexpr int64_t kTileMinChunks = 4;
// Workgroups a split-K decode launch aims for (batch 32: 256 beat 512, and 512 beat 1024).
constexpr int64_t kDecTargetGroups = 256;
constexpr int kDecMinSplitTiles = 3;        // digit column tiles (16 columns) needed to split
constexpr int64_t kDecMinSteps = 8;        // 64-byte k-steps per slice, at least
constexpr int64_t kDecMaxSplit = 8;

__device__ inline float block_reduce_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) t += red[w];
  return t;
}
__device__ inline float block_reduce_max(float v, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) t = fmaxf(t, red[w]);
  return t;
}

// One workgroup per activation row b (rows >= batch write zero digits). Optional RMSNorm.
__global__ __launch_bounds__(kThreads) void k_xdigits(const float* __restrict__ x, int64_t ldx,
                                                      const float* __restrict__ nw, float eps, int cols, int batch,
                                                      int kpad, int8_t* __restrict__ dig, float* __restrict__ pow2) {
  __shared__ float red[kThreads / 64];
  const int b = blockIdx.x;
  int8_t* d0 = dig + static_cast<int64_t>(3 * b) * kpad;
  int8_t* d1 = d0 + kpad;
  int8_t* d2 = d1 + kpad;
  if (b >= batch) {
    for (int k = threadIdx.x; k < kpad; k += kThreads) d0[k] = d1[k] = d2[k] = 0;
    if (threadIdx.x == 0) pow2[b] = 0.0f;
    return;
  }
  const float* xr = x + static_cast<int64_t>(b) * ldx;
  // The row is held in registers: kPer values per thread, loaded together (cols <= kThreads *
  // kPer; longer rows take the strided path).
  constexpr int kPer = 64;
  float xv[kPer];
  const bool in_regs = cols <= kThreads * kPer;
  float inv = 1.0f;
  if (in_regs) {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int k = threadIdx.x + u * kThreads;
      xv[u] = k < cols ? xr[k] : 0.0f;
    }
    if (nw) {
      float ss = 0.0f;
#pragma unroll
      for (int u = 0; u < kPer; ++u) ss += xv[u] * xv[u];
      ss = block_reduce_sum(ss, red);
      inv = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int k = threadIdx.x + u * kThreads;
        xv[u] = k < cols ? (xv[u] * inv) * nw[k] : 0.0f;
      }
    }
  } else if (nw) {
    float ss = 0.0f;
    for (int k = threadIdx.x; k < cols; k += kThreads) ss += xr[k] * xr[k];
    ss = block_reduce_sum(ss, red);
    inv = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
  }
  float m = 0.0f;
  if (in_regs) {
#pragma unroll
    for (int u = 0; u < kPer; ++u) m = fmaxf(m, fabsf(xv[u]));
  } else {
    for (int k = threadIdx.x; k < cols; k += kThreads) m = fmaxf(m, fabsf(nw ? (xr[k] * inv) * nw[k] : xr[k]));
  }
  m = block_reduce_max(m, red);
  int e = 0;
  if (m > 0.0f) (void)frexpf(m, &e);  // m = f * 2^e, f in [0.5, 1): max|x| < 2^e
  const int sh = 22 - e;
  auto put = [&](int k, float v_in) {
    const int v = static_cast<int>(rintf(ldexpf(v_in, sh)));  // |v| <= 2^22
    const int a0 = ((v + 128) & 255) - 128;
    const int v1 = (v - a0) >> 8;
    const int a1 = ((v1 + 128) & 255) - 128;
    const int a2 = (v1 - a1) >> 8;  // |a2| <= 64
    d0[k] = static_cast<int8_t>(a0);
    d1[k] = static_cast<int8_t>(a1);
    d2[k] = static_cast<int8_t>(a2);
  };
  if (in_regs) {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int k = threadIdx.x + u * kThreads;
      if (k < kpad) put(k, xv[u]);  // zero beyond cols: kpad <= cols + 63 <= kThreads * kPer + 63
    }
    for (int k = kThreads * kPer + threadIdx.x; k < kpad; k += kThreads) put(k, 0.0f);
  } else {
    for (int k = threadIdx.x; k < kpad; k += kThreads) put(k, k < cols ? (nw ? (xr[k] * inv) * nw[k] : xr[k]) : 0.0f);
  }
  if (threadIdx.x == 0) pow2[b] = ldexpf(1.0f, -sh);
}

// The same digits with one wavefront per activation row (four rows per workgroup): shuffle
// reductions only, 16-byte loads, four digits per 32-bit store. For rows of up to
// 64 * 4 * kV4 <= 8192 floats with cols % 4 == 0 and 16-byte aligned rows; the row is held
// in registers between the reductions and the digit split. Longer rows keep one workgroup
// per row (k_xdigits), which spreads them over more lanes.
template <int kV4, int W>
__global__ __launch_bounds__(256) void k_xdigits_wave(const float* __restrict__ x, int64_t ldx,
                                                      const float* __restrict__ nw, float eps, int cols, int batch,
                                                      int groups, int kpad, int8_t* __restrict__ dig,
                                                      float* __restrict__ pow2) {
  // W wavefronts per row (4 / W rows per workgroup); the row's lanes are sub * 64 + lane.
  __shared__ float red[2][4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = wave % W, first = wave - sub;  // this row's first wave
  const int rl = sub * 64 + lane;                // lane within the row
  const int b = blockIdx.x * (4 / W) + wave / W;
  const bool live = b < groups;
  const bool real = b < batch;
  int* d0 = reinterpret_cast<int*>(dig + static_cast<int64_t>(3 * (live ? b : 0)) * kpad);
  int* d1 = d0 + kpad / 4;
  int* d2 = d1 + kpad / 4;
  const int n4 = cols >> 2, kp4 = kpad >> 2;
  const float4* x4 = reinterpret_cast<const float4*>(x + static_cast<int64_t>(real ? b : 0) * ldx);
  float4 v[kV4];
#pragma unroll
  for (int u = 0; u < kV4; ++u) {
    const int i = rl + 64 * W * u;
    v[u] = (real && i < n4) ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  // Row sum over the W waves: wave shuffle, then the partials through LDS.
  auto row_reduce = [&](float t, int slot, bool is_max) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float o = __shfl_xor(t, off, 64);
      t = is_max ? fmaxf(t, o) : t + o;
    }
    if (W == 1) return t;
    if (lane == 0) red[slot][wave] = t;
    __syncthreads();
    float r = red[slot][first];
#pragma unroll
    for (int w = 1; w < W; ++w) r = is_max ? fmaxf(r, red[slot][first + w]) : r + red[slot][first + w];
    return r;
  };
  if (nw) {
    const float4* w4 = reinterpret_cast<const float4*>(nw);
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < kV4; ++u) ss += v[u].x * v[u].x + v[u].y * v[u].y + v[u].z * v[u].z + v[u].w * v[u].w;
    ss = row_reduce(ss, 0, false);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
#pragma unroll
    for (int u = 0; u < kV4; ++u) {
      const int i = rl + 64 * W * u;
      if (real && i < n4) {
        const float4 w = w4[i];
        v[u] = make_float4((v[u].x * inv) * w.x, (v[u].y * inv) * w.y, (v[u].z * inv) * w.z, (v[u].w * inv) * w.w);
      }
    }
  }
  float m = 0.0f;
#pragma unroll
  for (int u = 0; u < kV4; ++u) m = fmaxf(m, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
  m = row_reduce(m, 1, true);
  if (!live) return;
  int e = 0;
  if (m > 0.0f) (void)frexpf(m, &e);  // m = f * 2^e, f in [0.5, 1): max|x| < 2^e
  const int sh = 22 - e;
  auto split = [&](float f, int& a0, int& a1, int& a2) {
    const int q = static_cast<int>(rintf(ldexpf(f, sh)));  // |q| <= 2^22
    a0 = ((q + 128) & 255) - 128;
    const int q1 = (q - a0) >> 8;
    a1 = ((q1 + 128) & 255) - 128;
    a2 = (q1 - a1) >> 8;  // |a2| <= 64
  };
  auto pack = [](int a, int b_, int c, int d) {
    return (a & 255) | ((b_ & 255) << 8) | ((c & 255) << 16) | (d << 24);
  };
  // Rows past the batch (zero digits) have v == 0 and m == 0: every digit is 0.
#pragma unroll
  for (int u = 0; u < kV4; ++u) {
    const int i = rl + 64 * W * u;
    if (i < n4) {
      int a[4], bb[4], c[4];
      split(v[u].x, a[0], bb[0], c[0]);
      split(v[u].y, a[1], bb[1], c[1]);
      split(v[u].z, a[2], bb[2], c[2]);
      split(v[u].w, a[3], bb[3], c[3]);
      d0[i] = pack(a[0], a[1], a[2], a[3]);
      d1[i] = pack(bb[0], bb[1], bb[2], bb[3]);
      d2[i] = pack(c[0], c[1], c[2], c[3]);
    }
  }
  for (int i = n4 + rl; i < kp4; i += 64 * W) d0[i] = d1[i] = d2[i] = 0;  // the k-step padding
  if (rl == 0) pow2[b] = real ? ldexpf(1.0f, -sh) : 0.0f;
}

enum { kEpiStore = 0, kEpiAdd = 1, kEpiSwiglu = 2 };

__device__ inline uint32_t order_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Decode GEMM: one workgroup per 16 weight rows x NT*16 digit columns (all of the batch's
// digits for NT <= 12); the 4 wavefronts split K (interleaved 64-wide steps) and their int32
// partial sums are added in LDS. Every weight byte is read once per launch.
//
// Split K (gridDim.z > 1, for launches with fewer row tiles than CUs): workgroup z covers the
// z-th slice of the k-steps and stores its exact partial sums c0 + 256 c1 + 65536 c2 in its
// own 64-bit slots of the workspace `ws`; the last slice of a row tile to arrive adds the
// slices in slice order (exact integers: the result does not depend on arrival order), runs
// the epilogue and resets the tile's counter for the next launch.
template <int NT, int EPI, bool AMAX>
__global__ __launch_bounds__(kThreads) void k_gemm_dec(const int8_t* __restrict__ W, int64_t ldw,
                                                       const float* __restrict__ S, const int8_t* __restrict__ D,
                                                       int kpad, const float* __restrict__ pow2,
                                                       float* __restrict__ O, int64_t osb, int64_t osr, int rows,
                                                       int batch, unsigned long long* __restrict__ amax,
                                                       unsigned long long* __restrict__ ws,
                                                       unsigned* __restrict__ cnt) {
  __shared__ int csum[4][16][NT * 16];
  __shared__ long long tot[16][64];
  __shared__ int last;
  __shared__ unsigned long long best[AMAX ? 64 : 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = blockIdx.x * 16;
  if (AMAX && threadIdx.x < 64) best[threadIdx.x] = 0ull;
  // grid.y: chunk of `batch` entries (64 per chunk when there are several).
  D += static_cast<int64_t>(blockIdx.y) * 3 * batch * kpad;
  O += static_cast<int64_t>(blockIdx.y) * batch * osb;
  pow2 += static_cast<int64_t>(blockIdx.y) * batch;
  if (AMAX) amax += static_cast<int64_t>(blockIdx.y) * batch * kArgmaxSlots;
  const int r_l = lane & 15, kg = lane >> 4;  // operand row / column within the tile, k group
  const int8_t* wp = W + static_cast<int64_t>(min(row0 + r_l, rows - 1)) * ldw + kg * 16;
  const int8_t* dp = D + static_cast<int64_t>(r_l) * kpad + kg * 16;
  v4i acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = v4i{0, 0, 0, 0};
  const int nsplit = gridDim.z;
  const int per = (kpad / 64 + nsplit - 1) / nsplit;
  const int ks0 = blockIdx.z * per, ksteps = min(kpad / 64, ks0 + per);
  constexpr int kU = 4;  // k-steps per wave whose loads are in flight together
  for (int s0 = ks0 + wave; s0 < ksteps; s0 += 4 * kU) {
    v4i a[kU];
    v4i bm[kU][NT];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int s = s0 + 4 * u;
      if (s < ksteps) {
        a[u] = *reinterpret_cast<const v4i*>(wp + s * 64);
#pragma unroll
        for (int t = 0; t < NT; ++t)
          bm[u][t] = *reinterpret_cast<const v4i*>(dp + static_cast<int64_t>(t * 16) * kpad + s * 64);
      } else {
        a[u] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < NT; ++t) bm[u][t] = v4i{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u], bm[u][t], acc[t], 0, 0, 0);
  }
  // 16x16 int32 result tile t: lane holds rows 4*(lane/16) + v, column lane % 16.
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) csum[wave][4 * kg + v][t * 16 + r_l] = acc[t][v];
  __syncthreads();

  // This workgroup's sum for (tile row r, batch entry b); the three digit columns of b are
  // 3b, 3b+1, 3b+2.
  auto partial = [&](int r, int b) {
    int64_t c[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int col = 3 * b + j;
      c[j] = static_cast<int64_t>(csum[0][r][col]) + csum[1][r][col] + csum[2][r][col] + csum[3][r][col];
    }
    return c[0] + 256 * c[1] + 65536 * c[2];
  };
  if (nsplit > 1) {
    // Slot of slice z: ws[tile][z][16][64]; agent-scope stores, visible on every XCD once done.
    const int64_t tile = static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x;
    unsigned long long* wt = ws + tile * kDecMaxSplit * 16 * 64;
    for (int idx = threadIdx.x; idx < 16 * batch; idx += kThreads) {
      const int r = idx / batch, b = idx % batch;
      __hip_atomic_store(wt + (static_cast<int64_t>(blockIdx.z) * 16 + r) * 64 + b,
                         static_cast<unsigned long long>(partial(r, b)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // Waiting for the stores to complete (no cache writeback fence) orders them before the
    // counter increment.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
      unsigned* c = cnt + tile;
      const unsigned old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = old == static_cast<unsigned>(nsplit - 1);
      if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    for (int idx = threadIdx.x; idx < 16 * batch; idx += kThreads) {
      const int r = idx / batch, b = idx % batch;
      long long t = 0;
      for (int z = 0; z < nsplit; ++z)
        t += static_cast<long long>(__hip_atomic_load(wt + (static_cast<int64_t>(z) * 16 + r) * 64 + b,
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      tot[r][b] = t;
    }
    __syncthreads();
  }
  auto total = [&](int r, int b) -> int64_t { return nsplit > 1 ? tot[r][b] : partial(r, b); };

  // Epilogue: thread -> (row, batch entry).
  for (int idx = threadIdx.x; idx < 16 * batch; idx += kThreads) {
    const int r = idx / batch, b = idx % batch;
    const int row = row0 + r;
    const int64_t sum = total(r, b);
    const float y = static_cast<float>(sum) * pow2[b];
    if constexpr (EPI == kEpiSwiglu) {
      if ((r & 1) == 0 && row + 1 < rows) {
        const float yu = static_cast<float>(total(r + 1, b)) * pow2[b];
        const float g = y * S[row];
        const float u = yu * S[row + 1];
        const float silu = g / (1.0f + expf(-g));
        O[static_cast<int64_t>(b) * osb + static_cast<int64_t>(row >> 1) * osr] = silu * u;
      }
    } else if (row < rows) {
      const float v = y * S[row];
      float* o = O + static_cast<int64_t>(b) * osb + static_cast<int64_t>(row) * osr;
      if (EPI == kEpiAdd) *o = *o + v;
      else *o = v;
      if constexpr (AMAX) {
        const unsigned long long cand = (static_cast<unsigned long long>(order_key(v)) << 32) | static_cast<uint32_t>(row);
        atomicMax(&best[b], cand);  // LDS: the 16 rows of this tile first
      }
    }
  }
  if constexpr (AMAX) {
    __syncthreads();
    // Then one atomic per batch entry and workgroup, spread over the slots.
    if (threadIdx.x < batch)
      atomicMax(&amax[threadIdx.x * kArgmaxSlots + (blockIdx.x & (kArgmaxSlots - 1))], best[threadIdx.x]);
  }
}

// Tall-matrix decode GEMM: one workgroup per 64 weight rows (wave w owns rows 16w..16w+15 over
// the full K) x NT*16 digit columns. The digit operand is staged once per workgroup in LDS, in
// double-buffered KC-byte K chunks (row pitch padded by 16 bytes against bank conflicts). The
// next chunk's weights and digits are loaded into registers before the current chunk's MFMAs
// and written to LDS after them, so one memory round trip overlaps one chunk of compute.
template <int NT>
struct Rows64 {
  static constexpr int kN = NT * 16;
  static constexpr int kKC = NT <= 6 ? 512 : 256;          // bytes of K per stage
  static constexpr int kPitch = kKC + 16;                  // LDS row pitch
  static constexpr int kDig = kN * (kKC / 16) / kThreads;  // 16-byte digit loads per thread
  static_assert(kN * (kKC / 16) % kThreads == 0, "digit tile must split evenly");
};

template <int NT, int EPI, bool AMAX>
__global__ __launch_bounds__(kThreads) void k_gemm_rows64(const int8_t* __restrict__ W, int64_t ldw,
                                                          const float* __restrict__ S, const int8_t* __restrict__ D,
                                                          int kpad, const float* __restrict__ pow2,
                                                          float* __restrict__ O, int64_t osb, int64_t osr, int rows,
                                                          int batch, unsigned long long* __restrict__ amax) {
  using T = Rows64<NT>;
  constexpr int kN = T::kN, kKC = T::kKC, kPitch = T::kPitch, kDig = T::kDig, kU = kKC / 64;
  extern __shared__ __align__(16) int8_t lds[];  // [2][kN][kPitch] digits; reused as int32 C [64][kN]
  __shared__ unsigned long long best[AMAX ? 64 : 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = blockIdx.x * 64;
  D += static_cast<int64_t>(blockIdx.y) * 3 * batch * kpad;
  O += static_cast<int64_t>(blockIdx.y) * batch * osb;
  pow2 += static_cast<int64_t>(blockIdx.y) * batch;
  if (AMAX) amax += static_cast<int64_t>(blockIdx.y) * batch * kArgmaxSlots;
  if (AMAX && threadIdx.x < 64) best[threadIdx.x] = 0ull;
  const int r_l = lane & 15, kg = lane >> 4;
  const int8_t* wp = W + static_cast<int64_t>(min(row0 + wave * 16 + r_l, rows - 1)) * ldw + kg * 16;
  const int nchunks = (kpad + kKC - 1) / kKC;

  auto load_d = [&](int c, v4i (&d)[kDig]) {
#pragma unroll
    for (int i = 0; i < kDig; ++i) {
      const int idx = threadIdx.x + i * kThreads;
      const int n = idx / (kKC / 16), j = (idx % (kKC / 16)) * 16;
      const int k = c * kKC + j;
      d[i] = k < kpad ? *reinterpret_cast<const v4i*>(D + static_cast<int64_t>(n) * kpad + k) : v4i{0, 0, 0, 0};
    }
  };
  auto store_d = [&](int c, const v4i (&d)[kDig]) {
    int8_t* dst = lds + (c & 1) * kN * kPitch;
#pragma unroll
    for (int i = 0; i < kDig; ++i) {
      const int idx = threadIdx.x + i * kThreads;
      const int n = idx / (kKC / 16), j = (idx % (kKC / 16)) * 16;
      *reinterpret_cast<v4i*>(dst + n * kPitch + j) = d[i];
    }
  };
  auto load_w = [&](int c, v4i (&a)[kU]) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int k = c * kKC + u * 64;
      a[u] = k < kpad ? *reinterpret_cast<const v4i*>(wp + k) : v4i{0, 0, 0, 0};
    }
  };

  v4i acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = v4i{0, 0, 0, 0};
  v4i a_cur[kU], a_next[kU], d_next[kDig];
  load_w(0, a_cur);
  load_d(0, d_next);
  store_d(0, d_next);
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    const bool more = c + 1 < nchunks;
    if (more) {
      load_w(c + 1, a_next);
      load_d(c + 1, d_next);
    }
    const int8_t* buf = lds + (c & 1) * kN * kPitch;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const v4i b = *reinterpret_cast<const v4i*>(buf + (t * 16 + r_l) * kPitch + u * 64 + kg * 16);
        acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_cur[u], b, acc[t], 0, 0, 0);
      }
    }
    // Buffer (c + 1) & 1 was last read in iteration c - 1, before that iteration's barrier.
    if (more) store_d(c + 1, d_next);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kU; ++u) a_cur[u] = a_next[u];
  }

  // C tile in LDS: [64 rows][kN] int32 (the digit buffers are no longer needed).
  int* csum = reinterpret_cast<int*>(lds);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) csum[(wave * 16 + 4 * kg + v) * kN + t * 16 + r_l] = acc[t][v];
  __syncthreads();

  for (int idx = threadIdx.x; idx < 64 * batch; idx += kThreads) {
    const int r = idx / batch, b = idx % batch;
    const int row = row0 + r;
    const int* cr = csum + r * kN + 3 * b;
    const int64_t sum = static_cast<int64_t>(cr[0]) + 256 * static_cast<int64_t>(cr[1]) + 65536 * static_cast<int64_t>(cr[2]);
    const float y = static_cast<float>(sum) * pow2[b];
    if constexpr (EPI == kEpiSwiglu) {
      if ((r & 1) == 0 && row + 1 < rows) {
        const int* cu = cr + kN;
        const int64_t su = static_cast<int64_t>(cu[0]) + 256 * static_cast<int64_t>(cu[1]) + 65536 * static_cast<int64_t>(cu[2]);
        const float yu = static_cast<float>(su) * pow2[b];
        const float g = y * S[row];
        const float u = yu * S[row + 1];
        const float silu = g / (1.0f + expf(-g));
        O[static_cast<int64_t>(b) * osb + static_cast<int64_t>(row >> 1) * osr] = silu * u;
      }
    } else if (row < rows) {
      const float v = y * S[row];
      float* o = O + static_cast<int64_t>(b) * osb + static_cast<int64_t>(row) * osr;
      if (EPI == kEpiAdd) *o = *o + v;
      else *o = v;
      if constexpr (AMAX) {
        const unsigned long long cand = (static_cast<unsigned long long>(order_key(v)) << 32) | static_cast<uint32_t>(row);
        atomicMax(&best[b], cand);
      }
    }
  }
  if constexpr (AMAX) {
    __syncthreads();
    if (threadIdx.x < batch)
      atomicMax(&amax[threadIdx.x * kArgmaxSlots + (blockIdx.x & (kArgmaxSlots - 1))], best[threadIdx.x]);
  }
}

template <int NT>
size_t rows64_smem() {
  const size_t dig = 2 * static_cast<size_t>(Rows64<NT>::kN) * Rows64<NT>::kPitch;
  const size_t cs = 64 * static_cast<size_t>(Rows64<NT>::kN) * 4;
  return dig > cs ? dig : cs;
}

template <int NT, int EPI, bool AMAX>
void go_rows64(const int8_t* W, int64_t ldw, const float* S, const int8_t* D, int kpad, const float* pow2, float* O,
               int64_t osb, int64_t osr, int rows, int batch, int chunks, unsigned long long* amax, hipStream_t st) {
  const size_t smem = rows64_smem<NT>();
  static bool raised = false;
  if (!raised && smem > 65536) {
    PIA_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemm_rows64<NT, EPI, AMAX>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem)));
    raised = true;
  }
  hipLaunchKernelGGL((k_gemm_rows64<NT, EPI, AMAX>), dim3((rows + 63) / 64, chunks), dim3(kThreads), smem, st, W, ldw,
                     S, D, kpad, pow2, O, osb, osr, rows, batch, amax);
}

template <int NT>
void go_dec(const int8_t* W, int64_t ldw, const float* S, const int8_t* D, int kpad, const float* pow2, float* O,
            int64_t osb, int64_t osr, int rows, int batch, int chunks, Epi epi, unsigned long long* amax,
            const DecSplitWork* split, hipStream_t st) {
  // Tall matrices: 64-row tiles with the digits shared through LDS (enough tiles to fill the
  // CUs); short ones: 16-row tiles whose 4 wavefronts split K.
  if (static_cast<int64_t>((rows + 63) / 64) * chunks >= 96) {
    if (epi == Epi::Add) go_rows64<NT, kEpiAdd, false>(W, ldw, S, D, kpad, pow2, O, osb, osr, rows, batch, chunks, amax, st);
    else if (epi == Epi::Swiglu)
      go_rows64<NT, kEpiSwiglu, false>(W, ldw, S, D, kpad, pow2, O, osb, osr, rows, batch, chunks, amax, st);
    else if (amax) go_rows64<NT, kEpiStore, true>(W, ldw, S, D, kpad, pow2, O, osb, osr, rows, batch, chunks, amax, st);
    else go_rows64<NT, kEpiStore, false>(W, ldw, S, D, kpad, pow2, O, osb, osr, rows, batch, chunks, amax, st);
    return;
  }
  // Split K so that a launch has about kDecTargetGroups workgroups, each slice at least
  // kDecMinSteps k-steps long.
  const int64_t tiles = static_cast<int64_t>((rows + 15) / 16) * chunks;
  int nsplit = 1;
  // Below three digit tiles (batch < 11) a workgroup's MFMA work per k-step is too small for
  // the slice handshake to pay off.
  if (split && split->ws && NT >= kDecMinSplitTiles && tiles <= split->max_tiles) {
    const int64_t want = (kDecTargetGroups + tiles - 1) / tiles;
    const int64_t cap = (kpad / 64) / kDecMinSteps;
    nsplit = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>({want, cap, kDecMaxSplit})));
  }
  unsigned long long* ws = nsplit > 1 ? split->ws : nullptr;
  unsigned* cnt = nsplit > 1 ? split->cnt : nullptr;
  dim3 grid((rows + 15) / 16, chunks, nsplit);
  if (epi == Epi::Add)
    hipLaunchKernelGGL((k_gemm_dec<NT, kEpiAdd, false>), grid, dim3(kThreads), 0, st, W, ldw, S, D, kpad, pow2, O, osb,
                       osr, rows, batch, amax, ws, cnt);
  else if (epi == Epi::Swiglu)
    hipLaunchKernelGGL((k_gemm_dec<NT, kEpiSwiglu, false>), grid, dim3(kThreads), 0, st, W, ldw, S, D, kpad, pow2, O,
                       osb, osr, rows, batch, amax, ws, cnt);
  else if (amax)
    hipLaunchKernelGGL((k_gemm_dec<NT, kEpiStore, true>), grid, dim3(kThreads), 0, st, W, ldw, S, D, kpad, pow2, O,
                       osb, osr, rows, batch, amax, ws, cnt);
  else
    hipLaunchKernelGGL((k_gemm_dec<NT, kEpiStore, false>), grid, dim3(kThreads), 0, st, W, ldw, S, D, kpad, pow2, O,
                       osb, osr, rows, batch, amax, ws, cnt);
}

typedef int v16i __attribute__((ext_vector_type(16)));

// Prefill GEMM (many batch entries): one workgroup per 128 weight rows x 192 digit columns
// (64 batch entries). Both operand tiles go through LDS in 64-byte K stages, double buffered:
// the next stage's global loads are in registers while the current stage's MFMAs run. Four
// waves, each 64 rows x 96 columns = 2 x 3 tiles of v_mfma_i32_32x32x32_i8.
namespace tile {
constexpr int kBM = 128, kBN = 192, kBK = 64;
constexpr int kPitch = kBK + 16;  // LDS row pitch in bytes (staggers rows across banks)
constexpr int kStage = (kBM + kBN) * kPitch;
constexpr int kWLoads = kBM * kBK / 16 / kThreads;  // 16-byte loads per thread per stage: 2
constexpr int kDLoads = kBN * kBK / 16 / kThreads;  // 3
constexpr size_t kSmem = 2 * kStage > 64 * kBN * 4 ? 2 * kStage : 64 * kBN * 4;
}  // namespace tile

template <int EPI>
__global__ __launch_bounds__(kThreads) void k_gemm_tile(const int8_t* __restrict__ W, int64_t ldw,
                                                        const float* __restrict__ S, const int8_t* __restrict__ D,
                                                        int kpad, const float* __restrict__ pow2,
                                                        float* __restrict__ O, int64_t osb, int64_t osr, int rows) {
  using namespace tile;
  extern __shared__ __align__(16) int8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * kBM;
  const int col0 = blockIdx.y * kBN;  // digit rows of D; batch entries 64 * blockIdx.y ..
  const int wr = wave & 1, wc = wave >> 1;
  const int r_l = lane & 31, kh = lane >> 5;

  // Global -> register staging of one K stage: thread t covers 16-byte segment (t % 4) of
  // rows t / 4, t / 4 + 64, ... of each tile.
  const int seg = tid & 3, trow = tid >> 2;
  const int8_t* wsrc[kWLoads];
  const int8_t* dsrc[kDLoads];
#pragma unroll
  for (int u = 0; u < kWLoads; ++u)
    wsrc[u] = W + static_cast<int64_t>(min(row0 + trow + 64 * u, rows - 1)) * ldw + seg * 16;
#pragma unroll
  for (int u = 0; u < kDLoads; ++u) dsrc[u] = D + static_cast<int64_t>(col0 + trow + 64 * u) * kpad + seg * 16;
  v4i wreg[kWLoads], dreg[kDLoads];
  auto gload = [&](int kt) {
    const int64_t off = static_cast<int64_t>(kt) * kBK;
#pragma unroll
    for (int u = 0; u < kWLoads; ++u) wreg[u] = *reinterpret_cast<const v4i*>(wsrc[u] + off);
#pragma unroll
    for (int u = 0; u < kDLoads; ++u) dreg[u] = *reinterpret_cast<const v4i*>(dsrc[u] + off);
  };
  auto sstore = [&](int buf) {
    int8_t* ws = lds + buf * kStage;
    int8_t* ds = ws + kBM * kPitch;
#pragma unroll
    for (int u = 0; u < kWLoads; ++u) *reinterpret_cast<v4i*>(ws + (trow + 64 * u) * kPitch + seg * 16) = wreg[u];
#pragma unroll
    for (int u = 0; u < kDLoads; ++u) *reinterpret_cast<v4i*>(ds + (trow + 64 * u) * kPitch + seg * 16) = dreg[u];
  };

  v16i acc[2][3];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

  const int nk = kpad / kBK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) gload(kt + 1);
    const int8_t* ws = lds + (kt & 1) * kStage;
    const int8_t* ds = ws + kBM * kPitch;
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      v4i a[2], b[3];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const v4i*>(ws + (wr * 64 + i * 32 + r_l) * kPitch + kk + kh * 16);
#pragma unroll
      for (int j = 0; j < 3; ++j)
        b[j] = *reinterpret_cast<const v4i*>(ds + (wc * 96 + j * 32 + r_l) * kPitch + kk + kh * 16);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    // Buffer (kt + 1) & 1 was last read in iteration kt - 1, before that iteration's barrier.
    if (more) sstore((kt + 1) & 1);
    __syncthreads();
  }

  // Epilogue, 64 weight rows at a time: the C tile half goes to LDS ([64][kBN] int32), then
  // thread -> (row, batch entry) recombines the entry's three digit columns. 32x32 result
  // layout: lane holds column lane % 32 and, in register v, row 8 * (v / 4) + 4 * (lane / 32)
  // + v % 4.
  int* ct = reinterpret_cast<int*>(lds);
  for (int half = 0; half < 2; ++half) {
    if (wr == half) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int r = i * 32 + 8 * (v >> 2) + 4 * kh + (v & 3);
            ct[r * kBN + wc * 96 + j * 32 + r_l] = acc[i][j][v];
          }
    }
    __syncthreads();
    const int b0 = col0 / 3;  // first batch entry of the tile
    for (int idx = tid; idx < 64 * (kBN / 3); idx += kThreads) {
      const int r = idx / (kBN / 3), b = idx % (kBN / 3);
      const int row = row0 + half * 64 + r;
      const int* cr = ct + r * kBN + 3 * b;
      const int64_t sum = static_cast<int64_t>(cr[0]) + 256 * static_cast<int64_t>(cr[1]) + 65536 * static_cast<int64_t>(cr[2]);
      const float y = static_cast<float>(sum) * pow2[b0 + b];
      if constexpr (EPI == kEpiSwiglu) {
        if ((r & 1) == 0 && row + 1 < rows) {
          const int* cu = cr + kBN;
          const int64_t su = static_cast<int64_t>(cu[0]) + 256 * static_cast<int64_t>(cu[1]) + 65536 * static_cast<int64_t>(cu[2]);
          const float yu = static_cast<float>(su) * pow2[b0 + b];
          const float g = y * S[row];
          const float u = yu * S[row + 1];
          const float silu = g / (1.0f + expf(-g));
          O[static_cast<int64_t>(b0 + b) * osb + static_cast<int64_t>(row >> 1) * osr] = silu * u;
        }
      } else if (row < rows) {
        const float v = y * S[row];
        float* o = O + static_cast<int64_t>(b0 + b) * osb + static_cast<int64_t>(row) * osr;
        if (EPI == kEpiAdd) *o = *o + v;
        else *o = v;
      }
    }
    __syncthreads();
  }
}

template <int EPI>
void go_tile(const int8_t* W, int64_t ldw, const float* S, const int8_t* D, int kpad, const float* pow2, float* O,
             int64_t osb, int64_t osr, int rows, int tiles_n, hipStream_t st) {
  static bool raised = false;
  if (!raised && tile::kSmem > 65536) {
    PIA_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemm_tile<EPI>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(tile::kSmem)));
    raised = true;
  }
  hipLaunchKernelGGL((k_gemm_tile<EPI>), dim3((rows + tile::kBM - 1) / tile::kBM, tiles_n), dim3(kThreads), tile::kSmem,
                     st, W, ldw, S, D, kpad, pow2, O, osb, osr, rows);
}

}  // namespace

int64_t digit_cols(int64_t batch) { return (3 * batch + 15) / 16 * 16; }

// Digit rows written by k_xdigits: whole triples covering digit_cols(batch) columns.
int64_t digit_rows(int64_t batch) { return (digit_cols(batch) + 2) / 3 * 3; }

int64_t xdigits_bytes(int64_t batch, int64_t cols) {
  const int64_t kpad = (cols + 63) / 64 * 64;
  return (digit_rows(batch) * kpad + 255) / 256 * 256 + digit_rows(batch) / 3 * 4;
}

void launch_xdigits(const float* x, int64_t ldx, const float* norm_w, float eps, int64_t batch, int64_t cols,
                    void* xq, hipStream_t st) {
  PIA_REQUIRE(batch > 0 && cols > 0 && cols < (int64_t(1) << 30), "xdigits: bad shape");
  const int64_t kpad = (cols + 63) / 64 * 64;
  const int64_t n = digit_rows(batch);
  int8_t* dig = static_cast<int8_t*>(xq);
  float* pow2 = reinterpret_cast<float*>(dig + (n * kpad + 255) / 256 * 256);
  const int64_t groups = n / 3;  // digit-column triples (batch rows, padded with zeros)
  const bool vec = cols % 4 == 0 && ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                   (!norm_w || (reinterpret_cast<uintptr_t>(norm_w) & 15) == 0);
  const int64_t v4 = (cols / 4 + 63) / 64;  // float4 per lane
  if (vec && v4 <= 64) {
    // One wavefront per row up to 2048 floats, two up to 4096, four beyond (at most 16
    // float4 per lane in registers).
#define PIA_XDW(V, W)                                                                                            \
  hipLaunchKernelGGL((k_xdigits_wave<V, W>), dim3(static_cast<unsigned>((groups + 4 / W - 1) / (4 / W))), dim3(256), \
                     0, st, x, ldx, norm_w, eps, static_cast<int>(cols), static_cast<int>(batch),                 \
                     static_cast<int>(groups), static_cast<int>(kpad), dig, pow2)
    if (v4 <= 8) PIA_XDW(8, 1);
    else if (v4 <= 16) PIA_XDW(8, 2);
    else if (v4 <= 32) PIA_XDW(8, 4);
    else PIA_XDW(16, 4);
#undef PIA_XDW
  } else {
    hipLaunchKernelGGL(k_xdigits, dim3(static_cast<unsigned>(groups)), dim3(kThreads), 0, st, x, ldx, norm_w, eps,
                       static_cast<int>(cols), static_cast<int>(batch), static_cast<int>(kpad), dig, pow2);
  }
  PIA_HIP(hipGetLastError());
}

int64_t dec_split_bytes(int64_t max_tiles) { return max_tiles * kDecMaxSplit * 16 * 64 * 8 + max_tiles * 4; }

void launch_gemm_i8_mfma(const int8_t* W, int64_t ldw, const float* scales, const void* xq, float* out, int64_t osb,
                         int64_t osr, int64_t rows, int64_t cols, int64_t batch, Epi epi, unsigned long long* amax,
                         const DecSplitWork* split, hipStream_t st) {
  const int64_t kpad = (cols + 63) / 64 * 64;
  PIA_REQUIRE(ldw >= kpad && ldw % 16 == 0, "gemm: weight rows must be padded to a multiple of 64 bytes");
  PIA_REQUIRE(scales != nullptr, "gemm: int8 weights need scales");
  PIA_REQUIRE(rows > 0 && rows < (int64_t(1) << 31), "gemm: bad row count");
  PIA_REQUIRE(epi != Epi::Swiglu || rows % 2 == 0, "gemm: SwiGLU needs interleaved row pairs");
  PIA_REQUIRE(!amax || epi == Epi::Store, "gemm: fused argmax needs the Store epilogue");
  const int8_t* dig = static_cast<const int8_t*>(xq);
  const int64_t n = digit_rows(batch);
  const float* pow2 = reinterpret_cast<const float*>(dig + (n * kpad + 255) / 256 * 256);
  const int r = static_cast<int>(rows), k = static_cast<int>(kpad);
  // Column tiles of 64 batch entries (12 x 16 digit columns) along grid.y, then the ragged
  // remainder as its own launch.
  const int64_t full = batch / 64;
  auto launch = [&](int64_t b0, int64_t chunks, int nb) {
    const int nt = static_cast<int>(digit_cols(nb) / 16);
    const int8_t* D = dig + 3 * b0 * kpad;
    float* O = out + b0 * osb;
    unsigned long long* am = amax ? amax + b0 * kArgmaxSlots : nullptr;
    const float* p2 = pow2 + b0;
    switch (nt) {
#define PIA_NT(N)                                                                                     \
  case N:                                                                                             \
    go_dec<N>(W, ldw, scales, D, k, p2, O, osb, osr, r, nb, static_cast<int>(chunks), epi, am, split, st); \
    break;
      PIA_NT(1) PIA_NT(2) PIA_NT(3) PIA_NT(4) PIA_NT(5) PIA_NT(6) PIA_NT(7) PIA_NT(8) PIA_NT(9) PIA_NT(10)
      PIA_NT(11) PIA_NT(12)
#undef PIA_NT
      default: fail(PIA_ERR_INVALID, "gemm: bad column tile");
    }
  };
  if (full >= kTileMinChunks && !amax) {
    // Many batch entries (prefill): the LDS-tiled kernel over the whole 64-entry chunks.
    if (epi == Epi::Add) go_tile<kEpiAdd>(W, ldw, scales, dig, k, pow2, out, osb, osr, r, static_cast<int>(full), st);
    else if (epi == Epi::Swiglu) go_tile<kEpiSwiglu>(W, ldw, scales, dig, k, pow2, out, osb, osr, r, static_cast<int>(full), st);
    else go_tile<kEpiStore>(W, ldw, scales, dig, k, pow2, out, osb, osr, r, static_cast<int>(full), st);
  } else if (full) {
    launch(0, full, 64);
  }
  if (batch % 64) launch(full * 64, 1, static_cast<int>(batch % 64));
  PIA_HIP(hipGetLastError());
}

}  // namespace pia
