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
// * scale[r]. The only rounding is the fixed-point image of x (|error| <= 2^(e_b - 23) per
// element, max|x_b| < 2^e_b) and the final conversions. On rows without outliers that is
// tighter than an f32 accumulation of the same dot; an entry whose row holds a channel 1000x
// the others sees its small elements on a grid ~2^-12 of their size (tests bound both cases).
//
// Digit layout (every kernel here): batch entries in groups of 16; entry b's digit plane j is
// digit row (3 (b / 16) + j) * 16 + b % 16 of the [48 * groups][kpad] digit matrix.
#include <cmath>
#include <cstdlib>

#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace pia {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
// Whole 64-entry chunks from which the LDS-tiled kernel takes over (prefill sizes).
constexpr int64_t kTileMinChunks = 4;
// Workgroups a split-K decode launch aims for.
constexpr int64_t kDecTargetGroups = 256;
constexpr int64_t kDecMinSteps = 8;  // 64-byte k-steps per slice, at least
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
                                                      int kpad, int nrows, int8_t* __restrict__ dig,
                                                      float* __restrict__ pow2) {
  __shared__ float red[kThreads / 64];
  const int b = blockIdx.x;
  const int n0 = digit_row(b, 0), n1 = digit_row(b, 1), n2 = digit_row(b, 2);
  auto D = [&](int n, int k) -> int8_t& { return dig[digit_off(n, k, nrows)]; };
  if (b >= batch) {
    for (int k = threadIdx.x; k < kpad; k += kThreads) D(n0, k) = D(n1, k) = D(n2, k) = 0;
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
    D(n0, k) = static_cast<int8_t>(a0);
    D(n1, k) = static_cast<int8_t>(a1);
    D(n2, k) = static_cast<int8_t>(a2);
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

// The same digits with W wavefronts per activation row (4 / W rows per workgroup; the launch
// uses W = 4): shuffle reductions (and the W partials through LDS), 16-byte loads, four digits
// per 32-bit store. For rows of up to 64 * W * kV4 floats with cols % 4 == 0 and 16-byte
// aligned rows; the row is held in registers between the reductions and the digit split.
// Longer rows use k_xdigits.
template <int kV4, int W>
__global__ __launch_bounds__(256) void k_xdigits_wave(const float* __restrict__ x, int64_t ldx,
                                                      const float* __restrict__ nw, float eps, int cols, int batch,
                                                      int groups, int kpad, int nrows, int8_t* __restrict__ dig,
                                                      float* __restrict__ pow2) {
  // W wavefronts per row (4 / W rows per workgroup); the row's lanes are sub * 64 + lane.
  __shared__ float red[2][4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = wave % W, first = wave - sub;  // this row's first wave
  const int rl = sub * 64 + lane;                // lane within the row
  const int b = blockIdx.x * (4 / W) + wave / W;
  const bool live = b < groups;
  const bool real = b < batch;
  // Four digits per 32-bit store: float4 index i covers columns 4i .. 4i + 3 of one k-step.
  const int bb0 = live ? b : 0;
  const int n0 = digit_row(bb0, 0), n1 = digit_row(bb0, 1), n2 = digit_row(bb0, 2);
  int* dw = reinterpret_cast<int*>(dig);
  auto at = [&](int n, int i) -> int& { return dw[digit_off(n, 4 * i, nrows) >> 2]; };
  const int n4 = cols >> 2, kp4 = kpad >> 2;
  const float4* x4 = reinterpret_cast<const float4*>(x + static_cast<int64_t>(real ? b : 0) * ldx);
  float4 v[kV4], nv[kV4];
  const float4* w4 = reinterpret_cast<const float4*>(nw);
#pragma unroll
  for (int u = 0; u < kV4; ++u) {
    const int i = rl + 64 * W * u;
    v[u] = (real && i < n4) ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    // The norm weights are loaded with the row (not after the reduction): one memory round trip.
    if (nw) nv[u] = (real && i < n4) ? w4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
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
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < kV4; ++u) ss += v[u].x * v[u].x + v[u].y * v[u].y + v[u].z * v[u].z + v[u].w * v[u].w;
    ss = row_reduce(ss, 0, false);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
#pragma unroll
    for (int u = 0; u < kV4; ++u) {
      const int i = rl + 64 * W * u;
      if (real && i < n4) {
        const float4 w = nv[u];
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
      at(n0, i) = pack(a[0], a[1], a[2], a[3]);
      at(n1, i) = pack(bb[0], bb[1], bb[2], bb[3]);
      at(n2, i) = pack(c[0], c[1], c[2], c[3]);
    }
  }
  for (int i = n4 + rl; i < kp4; i += 64 * W) at(n0, i) = at(n1, i) = at(n2, i) = 0;  // the k-step padding
  if (rl == 0) pow2[b] = real ? ldexpf(1.0f, -sh) : 0.0f;
}

enum { kEpiStore = 0, kEpiAdd = 1, kEpiSwiglu = 2 };

__device__ inline uint32_t order_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Decode GEMM (batches of up to 64 entries per launch chunk): one workgroup per 64*RT weight rows
// (wave w owns rows 16*RT*w .. +16*RT, RT 16-row operand tiles) x all 16*NT digit columns of the
// chunk's entries, over one K slice (grid.z) of the 64-byte k-steps.
//
// The weight stream is the HBM-bound part; the digits are small, shared by every workgroup and
// L2-resident. Each k-step's weights (per wave) and digits (per workgroup, 16 bytes per thread)
// are issued PD k-steps ahead into a register ring, so the in-order completion counter never
// has to drain the weight stream to reach a digit load; a k-step's digits go to LDS one k-step
// before use (double buffer, one barrier per k-step) and every wave reads them from there.
//
// Digit layout: entry b's digit j is digit row (3 (b / 16) + j) * 16 + b % 16, so in the
// 16x16 result tiles 3g, 3g+1, 3g+2 lane l holds the three digit sums of entry 16g + l % 16
// for rows 4 (l / 16) + v: the epilogue recombines c0 + 256 c1 + 65536 c2 in registers.
//
// Split K (gridDim.z > 1, short matrices): slice z stores its exact 64-bit sums in its own
// workspace slots (agent-scope stores, completed before the counter increment); the last slice
// of a row tile to arrive adds the slices in slice order (exact: the result does not depend on
// the arrival order), runs the epilogue and resets the tile's counter for the next launch.
namespace dec {
// LDS: digit row n of a k-step at n * 64, its 16-byte chunk c at position c ^ ((n >> 1) & 3).
// The swizzle spreads the 16 rows one operand read touches over every bank group (measured:
// TinyLlama down projection at batch 32 24.3 -> 16.5 us with it, against padded rows).
constexpr int kPitch = 64;
__device__ inline int chunk_pos(int n, int c) { return (c ^ ((n >> 1) & 3)) * 16; }
}  // namespace dec

template <int NG, int RT, int PD, int EPI, bool AMAX>
__global__ __launch_bounds__(kThreads, 2) void k_gemm_dec(const int8_t* __restrict__ W, int64_t ldw,
                                                          const float* __restrict__ S, const int8_t* __restrict__ D,
                                                          int kpad, int nrows, const float* __restrict__ pow2,
                                                       float* __restrict__ O, int64_t osb, int64_t osr, int rows,
                                                       int batch, unsigned long long* __restrict__ amax,
                                                       unsigned long long* __restrict__ ws,
                                                       unsigned* __restrict__ cnt) {
  constexpr int NT = 3 * NG, N = 16 * NT;
  constexpr int DV = (N * 4 + kThreads - 1) / kThreads;  // 16-byte digit loads per thread per k-step
  constexpr int kRows = 64 * RT;                          // weight rows per workgroup
  __shared__ __align__(16) int8_t dl[2][N * dec::kPitch];
  __shared__ int last;
  __shared__ unsigned long long best[AMAX ? 64 : 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r_l = lane & 15, kq = lane >> 4;
  const int wrow0 = blockIdx.x * kRows + wave * 16 * RT;  // this wave's first row
  if (AMAX && tid < 64) best[tid] = 0ull;
  // grid.y: chunk of 64 entries (192 digit rows, 64 pow2 values, 64 output columns).
  D += static_cast<int64_t>(blockIdx.y) * 192 * 64;
  const int64_t dstep = static_cast<int64_t>(nrows) * 64;  // bytes per k-step of the digit matrix
  O += static_cast<int64_t>(blockIdx.y) * 64 * osb;
  pow2 += static_cast<int64_t>(blockIdx.y) * 64;
  if (AMAX) amax += static_cast<int64_t>(blockIdx.y) * 64 * kArgmaxSlots;

  const int8_t* wp[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
    wp[rt] = W + static_cast<int64_t>(min(wrow0 + rt * 16 + r_l, rows - 1)) * ldw + kq * 16;
  // Every load and LDS store below is unconditional (no lane-divergent branches, no skipped
  // refills), so the compiler's wait counts see the same number of loads in flight on every
  // path and keep the ring in flight. Threads past the digit tile repeat the last segment
  // (same data to the same LDS bytes); refills past the slice re-read its last k-step.
  const int8_t* dp[DV];
  int doff[DV];
#pragma unroll
  for (int i = 0; i < DV; ++i) {
    const int idx = min(tid + i * kThreads, N * 4 - 1);
    const int n = idx >> 2, seg = idx & 3;
    dp[i] = D + n * 64 + seg * 16;
    doff[i] = n * dec::kPitch + dec::chunk_pos(n, seg);
  }

  const int nsplit = gridDim.z;
  const int ksteps = kpad / 64;
  const int per = (ksteps + nsplit - 1) / nsplit;
  const int c0 = blockIdx.z * per, c1 = min(ksteps, c0 + per);
  // Workgroups start their slice at staggered k-steps (the integer sums do not depend on the
  // order), so concurrent loads spread over the memory channels. Logical step c of the slice
  // reads physical k-step c0 + (c - c0 + rot) mod len; refills past the slice repeat its last.
  const int len = max(c1 - c0, 1);
  const int rot = static_cast<int>((blockIdx.x * 5u) % static_cast<unsigned>(len));
  auto phys = [&](int c) {
    int j = min(c - c0, len - 1) + rot;
    return c0 + (j >= len ? j - len : j);
  };

  v4i wr[PD][RT], dr[PD][DV];
  auto load_w = [&](int c, v4i (&w)[RT]) {
    const int64_t off = static_cast<int64_t>(phys(c)) * 64;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) w[rt] = *reinterpret_cast<const v4i*>(wp[rt] + off);
  };
  auto load_d = [&](int c, v4i (&d)[DV]) {
    const int64_t off = static_cast<int64_t>(phys(c)) * dstep;
#pragma unroll
    for (int i = 0; i < DV; ++i) d[i] = *reinterpret_cast<const v4i*>(dp[i] + off);
  };
  auto store_d = [&](int stage, const v4i (&d)[DV]) {
#pragma unroll
    for (int i = 0; i < DV; ++i) *reinterpret_cast<v4i*>(&dl[stage][doff[i]]) = d[i];
  };

  v4i acc[RT][NT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[rt][t] = v4i{0, 0, 0, 0};

#pragma unroll
  for (int i = 0; i < PD; ++i) load_w(c0 + i, wr[i]);
#pragma unroll
  for (int i = 0; i < PD; ++i) load_d(c0 + i, dr[i]);
  store_d(0, dr[0]);
  __syncthreads();
  // One k-step: MFMAs on ring slot i (chunk c) and the LDS stage the previous step filled; then
  // the next k-step's digits (loaded PD - 1 steps ago) into the other stage, which every wave
  // finished reading before the previous barrier.
  auto step = [&](int c, int i, const v4i (&w)[RT], const v4i (&dnext)[DV]) {
    const int stage = (c - c0) & 1;
    const int8_t* buf = dl[stage] + r_l * dec::kPitch + dec::chunk_pos(r_l, kq);  // rows t * 16 + r_l
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const v4i b = *reinterpret_cast<const v4i*>(buf + t * 16 * dec::kPitch);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) acc[rt][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w[rt], b, acc[rt][t], 0, 0, 0);
    }
    store_d(stage ^ 1, dnext);
  };
  // Whole groups of PD k-steps with no exit inside a group (an early exit would let the
  // compiler sink the refills to their first use, serializing the stream), then the tail
  // from the ring without refills.
  int c = c0;
  for (; c + PD <= c1; c += PD) {
#pragma unroll
    for (int i = 0; i < PD; ++i) {
      step(c + i, i, wr[i], dr[(i + 1) % PD]);
      load_w(c + i + PD, wr[i]);
      load_d(c + i + PD, dr[i]);
      __syncthreads();
    }
  }
#pragma unroll
  for (int i = 0; i < PD; ++i) {
    if (c + i < c1) {
      step(c + i, i, wr[i], dr[(i + 1) % PD]);
      __syncthreads();
    }
  }

  // Exact integer sum of entry b = 16 g + r_l for row 4 kq + v of tile rt.
  auto digits_sum = [&](int rt, int g, int v) -> long long {
    return static_cast<long long>(acc[rt][3 * g][v]) + 256ll * acc[rt][3 * g + 1][v] +
           65536ll * acc[rt][3 * g + 2][v];
  };
  long long tot[RT][NG][4];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) tot[rt][g][v] = digits_sum(rt, g, v);

  if (nsplit > 1) {
    // Slots of pair (tile, z): [kRows rows][64 entries] 64-bit sums.
    const int64_t tile = static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x;
    unsigned long long* base = ws + tile * nsplit * kRows * 64;
    const int lrow = wave * 16 * RT + kq * 4;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          __hip_atomic_store(base + (static_cast<int64_t>(blockIdx.z) * kRows + lrow + rt * 16 + v) * 64 + g * 16 + r_l,
                             static_cast<unsigned long long>(tot[rt][g][v]), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    // Waiting for the stores to complete (no cache writeback) orders them before the counter
    // increment; the last slice's agent-scope loads are issued only after it has seen the count.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      unsigned* cp = cnt + tile;
      const unsigned old = __hip_atomic_fetch_add(cp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = old == static_cast<unsigned>(nsplit - 1);
      if (last) __hip_atomic_store(cp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    // Slice by slice (in slice order), every value of a slice loaded before any is added: one
    // round trip per slice, not per value.
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int v = 0; v < 4; ++v) tot[rt][g][v] = 0;
    for (int z = 0; z < nsplit; ++z) {
      unsigned long long part[RT][NG][4];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            part[rt][g][v] = __hip_atomic_load(
                base + (static_cast<int64_t>(z) * kRows + lrow + rt * 16 + v) * 64 + g * 16 + r_l, __ATOMIC_RELAXED,
                __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
          for (int v = 0; v < 4; ++v) tot[rt][g][v] += static_cast<long long>(part[rt][g][v]);
    }
  }

  // Epilogue: lane -> rows 4 kq + v of each tile, entries 16 g + r_l.
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const int b = g * 16 + r_l;
    const bool live = b < batch;
    const float p2 = live ? pow2[b] : 0.0f;
    unsigned long long mine = 0ull;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int rbase = wrow0 + rt * 16 + kq * 4;
      if constexpr (EPI == kEpiSwiglu) {
#pragma unroll
        for (int v = 0; v < 4; v += 2) {
          const int row = rbase + v;  // even: gate row, row + 1 the matching up row
          if (live && row + 1 < rows) {
            const float y = static_cast<float>(tot[rt][g][v]) * p2;
            const float yu = static_cast<float>(tot[rt][g][v + 1]) * p2;
            const float gt = y * S[row];
            const float u = yu * S[row + 1];
            const float silu = gt / (1.0f + expf(-gt));
            O[static_cast<int64_t>(b) * osb + static_cast<int64_t>(row >> 1) * osr] = silu * u;
          }
        }
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = rbase + v;
          if (live && row < rows) {
            const float val = static_cast<float>(tot[rt][g][v]) * p2 * S[row];
            float* o = O + static_cast<int64_t>(b) * osb + static_cast<int64_t>(row) * osr;
            if (EPI == kEpiAdd) *o = *o + val;
            else *o = val;
            if constexpr (AMAX) {
              const unsigned long long cand =
                  (static_cast<unsigned long long>(order_key(val)) << 32) | static_cast<uint32_t>(row);
              mine = cand > mine ? cand : mine;
            }
          }
        }
      }
    }
    if constexpr (AMAX) {
      // Lanes r_l, r_l + 16, r_l + 32, r_l + 48 hold the same entry: reduce them, then the waves
      // of the workgroup in LDS.
#pragma unroll
      for (int off = 16; off < 64; off <<= 1) {
        const unsigned long long o = __shfl_xor(mine, off, 64);
        mine = o > mine ? o : mine;
      }
      if (kq == 0 && live) atomicMax(&best[b], mine);
    }
  }
  if constexpr (AMAX) {
    __syncthreads();
    if (tid < batch && tid < 64)
      atomicMax(&amax[tid * kArgmaxSlots + (blockIdx.x & (kArgmaxSlots - 1))], best[tid]);
  }
}

// Choice of a decode launch: RT operand tiles per wave, K slices.
struct DecPlan {
  int rt, nsplit;
};

DecPlan plan_dec(int64_t rows, int64_t kpad, int nb, int64_t chunks, int64_t max_pairs) {
  const bool split_ok = max_pairs > 1;
  const int ng = (nb + 15) / 16;
  // Two row tiles per wave halve the digit operand's traffic per weight byte (L2 -> LDS ->
  // registers), which is what limits these launches from 32 entries on; they pay where the
  // matrix still fills the CUs with 128-row tiles (measured: Llama-3-8B gate/up yes; q/k/v, o,
  // down and every TinyLlama projection no).
  int rt = ng >= 2 && rows >= 24576 ? 2 : 1;
  if (const char* e = std::getenv("PIA_DEC_RT")) rt = std::atoi(e) == 1 ? 1 : 2;
  const int64_t tiles = (rows + 64 * rt - 1) / (64 * rt) * chunks;
  int nsplit = 1;
  if (split_ok) {
    int64_t target = kDecTargetGroups;
    if (const char* e = std::getenv("PIA_DEC_TARGET")) target = std::max<int64_t>(1, std::atoll(e));
    // Split only launches that leave most CUs idle: the slices' partial sums cost a round trip
    // through the coherence point (two workgroups fit on a CU).
    const int64_t want = 2 * tiles <= target ? (target + tiles - 1) / tiles : 1;
    const int64_t cap = (kpad / 64) / kDecMinSteps;
    nsplit = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>({want, cap, kDecMaxSplit})));
    if (tiles * nsplit > max_pairs) nsplit = static_cast<int>(std::max<int64_t>(1, max_pairs / tiles));
  }
  return {rt, nsplit};
}

template <int NG, int RT, int PD>
void go_dec_rt(const int8_t* W, int64_t ldw, const float* S, const int8_t* D, int kpad, int nrows, const float* pow2, float* O,
               int64_t osb, int64_t osr, int rows, int batch, int chunks, Epi epi, unsigned long long* amax,
               int nsplit, const DecSplitWork* split, hipStream_t st) {
  unsigned long long* ws = nsplit > 1 ? split->ws : nullptr;
  unsigned* cnt = nsplit > 1 ? split->cnt : nullptr;
  const dim3 grid((rows + 64 * RT - 1) / (64 * RT), chunks, nsplit);
#define PIA_DEC(E, A)                                                                                          \
  hipLaunchKernelGGL((k_gemm_dec<NG, RT, PD, E, A>), grid, dim3(kThreads), 0, st, W, ldw, S, D, kpad, nrows, pow2, O, osb, \
                     osr, rows, batch, amax, ws, cnt)
  if (epi == Epi::Add) PIA_DEC(kEpiAdd, false);
  else if (epi == Epi::Swiglu) PIA_DEC(kEpiSwiglu, false);
  else if (amax) PIA_DEC(kEpiStore, true);
  else PIA_DEC(kEpiStore, false);
#undef PIA_DEC
}

template <int NG>
void go_dec(const int8_t* W, int64_t ldw, const float* S, const int8_t* D, int kpad, int nrows, const float* pow2, float* O,
            int64_t osb, int64_t osr, int rows, int batch, int chunks, Epi epi, unsigned long long* amax,
            const DecSplitWork* split, hipStream_t st) {
  const DecPlan pl = plan_dec(rows, kpad, batch, chunks, split && split->ws ? split->pairs : 0);
  // Ring depth: k-steps in flight per wave (register budget: acc RT*3*NG*4, ring PD*(RT + DV)*4).
  // Ring depth 4: two workgroups per CU (registers <= 256 per lane, no accumulator copies)
  // beat a deeper ring at one workgroup per CU on every measured shape.
  constexpr int PD = 4;
  if (pl.rt == 2) go_dec_rt<NG, 2, PD>(W, ldw, S, D, kpad, nrows, pow2, O, osb, osr, rows, batch, chunks, epi, amax, pl.nsplit, split, st);
  else go_dec_rt<NG, 1, PD>(W, ldw, S, D, kpad, nrows, pow2, O, osb, osr, rows, batch, chunks, epi, amax, pl.nsplit, split, st);
}

typedef int v16i __attribute__((ext_vector_type(16)));

// Prefill GEMM (many batch entries): workgroup tiles of weight rows x digit columns whose
// operand stages go straight from memory to LDS, each wave multiplying its block of the tile
// with v_mfma_i32_32x32x32_i8 (shapes and measurements below).
namespace tile {
// Tile: kBM = 32 TI WRW weight rows x kBN = 96 WCW digit rows (32 WCW batch entries), WRW x WCW
// waves, each owning a 32 TI x 96 block of the result (TI x 3 MFMA 32x32 tiles); K stages of
// kBK bytes in two LDS buffers, filled by direct global -> LDS loads one stage ahead. Where
// the time goes (TinyLlama projections at 2048 tokens, 128 x 192 tile): the stage loop alone
// (no operand loads, no epilogue) issues int8 MFMA at about 55% of the rate a pure MFMA loop
// reaches; the operand loads add about half of that time again, the epilogue a sixth. Deeper
// load pipelines (3 and 4 stages) measured no faster. The 256 x 384 tile (8 waves, 128 x 96
// each) reads half the operand bytes per multiply-add; it is used when its grid still gives
// every CU two workgroups (the gate/up projection of a long prefill).
constexpr int kBK = 64;
constexpr int kPitch = kBK;  // LDS row pitch in bytes
// 16-byte chunk c of tile row n sits at position c ^ ((n >> 2) & 3). A 32x32x32 operand read
// takes chunk kk / 16 + lane / 32 of rows lane % 32; the LDS serves 16 lanes of a 16-byte read
// per cycle, and this swizzle puts the 16 rows of each such group on distinct banks (measured
// with SQ_LDS_BANK_CONFLICT: 0 conflict cycles, against 4 per read with (n >> 1) & 3).
__device__ inline int chunk_pos(int n, int c) { return (c ^ ((n >> 2) & 3)) * 16; }
template <int TI, int WRW, int WCW>
struct Shape {
  static constexpr int kBM = 32 * TI * WRW, kBN = 96 * WCW, kWaves = WRW * WCW, kThreads = 64 * kWaves;
  static constexpr int kStage = (kBM + kBN) * kPitch;
  static constexpr size_t kSmem = 2 * kStage;
};
using Big = Shape<4, 2, 4>;  // 256 x 384, 8 waves (the other shape: Shape<2, 2, 2>, 128 x 192, 4 waves)
}  // namespace tile

// Global -> LDS load of 16 bytes per lane with no register staging: lane l's bytes land at
// LDS byte lds_base + 16 l (global_load_lds_dwordx4; M0 holds the wave-uniform LDS base and is
// restored after). The compiler does not see the LDS write: callers order it with explicit
// vmcnt waits and barriers (both also compiler memory barriers).
__device__ __forceinline__ void load_lds16(const void* g, unsigned lds_base) {
  unsigned saved;
  // One wait state between the M0 write and the load that reads it.
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(g), "s"(lds_base)
               : "memory");
}
__device__ __forceinline__ void wait_vmcnt0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

template <int EPI, int TI, int WRW, int WCW>
__global__ __launch_bounds__(64 * WRW * WCW, 2) void k_gemm_tile(const int8_t* __restrict__ W, int64_t ldw,
                                                                 const float* __restrict__ S,
                                                                 const int8_t* __restrict__ D, int kpad, int nrows,
                                                                 const float* __restrict__ pow2, float* __restrict__ O,
                                                                 int64_t osb, int64_t osr, int rows) {
  using namespace tile;
  using Sh = Shape<TI, WRW, WCW>;
  constexpr int kBM = Sh::kBM, kBN = Sh::kBN, kWaves = Sh::kWaves, kStage = Sh::kStage;
  constexpr int kLoads = (kBM + kBN) / 16;  // direct loads per stage (16 rows each)
  constexpr int kPerWave = (kLoads + kWaves - 1) / kWaves;
  extern __shared__ __align__(16) int8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * kBM;
  const int col0 = blockIdx.y * kBN;  // digit rows of D; batch entries kBN / 3 * blockIdx.y ..
  const int wr = wave % WRW, wc = wave / WRW;
  const int r_l = lane & 31, kh = lane >> 5;

  // Direct load L = wave + kWaves q fills rows 16 L .. + 16 of the stage (weights first, then
  // digits); lane l writes LDS slot l % 4 of row 16 L + l / 4, which holds (swizzled) global
  // chunk (l % 4) ^ ((row >> 2) & 3) of that row.
  const int8_t* src[kPerWave];
  bool digit[kPerWave];
#pragma unroll
  for (int q = 0; q < kPerWave; ++q) {
    const int n = 16 * min(wave + kWaves * q, kLoads - 1) + lane / 4;
    digit[q] = n >= kBM;
    src[q] = digit[q] ? D + static_cast<int64_t>(col0 + n - kBM) * 64 + chunk_pos(n, lane & 3)
                      : W + static_cast<int64_t>(min(row0 + n, rows - 1)) * ldw + chunk_pos(n, lane & 3);
  }
  const unsigned lds0 = static_cast<unsigned>(reinterpret_cast<uintptr_t>(lds));
  const int nk = kpad / kBK;
  auto issue = [&](int kt, int b) {
    const int64_t off = static_cast<int64_t>(kt) * kBK;
    const int64_t doff = static_cast<int64_t>(kt) * nrows * 64;  // k-step-major digits
#pragma unroll
    for (int q = 0; q < kPerWave; ++q)
      if (wave + kWaves * q < kLoads)
        load_lds16(src[q] + (digit[q] ? doff : off),
                   __builtin_amdgcn_readfirstlane(lds0 + b * kStage + 16 * (wave + kWaves * q) * kPitch));
  };

  v16i acc[TI][3];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

  // Stage kt + 1 is in flight while stage kt is multiplied (more stages in flight measured no
  // faster).
  issue(0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    const int b = kt & 1;
    wait_vmcnt0();    // this wave's part of stage kt has landed
    __syncthreads();  // ... every wave's; and buffer 1 - b (stage kt - 1) is free
    if (kt + 1 < nk) issue(kt + 1, 1 - b);
    const int8_t* ws = lds + b * kStage;
    const int8_t* ds = ws + kBM * kPitch;
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      v4i a[TI], bb[3];
#pragma unroll
      for (int i = 0; i < TI; ++i)
        a[i] = *reinterpret_cast<const v4i*>(ws + ((wr * TI + i) * 32 + r_l) * kPitch + chunk_pos(r_l, kk / 16 + kh));
#pragma unroll
      for (int j = 0; j < 3; ++j)
        bb[j] = *reinterpret_cast<const v4i*>(ds + (wc * 96 + j * 32 + r_l) * kPitch + chunk_pos(r_l, kk / 16 + kh));
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], bb[j], acc[i][j], 0, 0, 0);
    }
  }

  // Epilogue in registers. The three digit columns of a batch entry are 16 apart inside a
  // 48-column group (digit_row), so in the 32x32 result layout (lane holds column lane % 32
  // and, in register v, row 8 (v / 4) + 4 (lane / 32) + v % 4) one exchange between lanes l and
  // l ^ 16 gives every lane the three digits of one entry: lanes c < 16 of the wave's columns
  // take entry c (columns c, c + 16 of tile 0 and c of tile 1), lanes c >= 16 entry c
  // (columns c of tile 1, c - 16 and c of tile 2). Each lane then owns 4 consecutive rows per
  // register quad and writes them as one vector where the output layout allows.
  const int e = wc * 32 + r_l;                  // entry of this lane within the tile
  const int eg = col0 / 3 + e;                  // global batch entry
  const bool lo = r_l < 16;
  const float p2 = pow2[eg];
  float* orow = O + static_cast<int64_t>(eg) * osb;
  const bool vec = osr == 1 && (osb & 3) == 0;  // 16-byte aligned rows of 4 (8-byte pairs for SwiGLU)
#pragma unroll
  for (int i = 0; i < TI; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float y[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int v = 4 * q + t;
        const int x0 = acc[i][0][v], x1 = acc[i][1][v], x2 = acc[i][2][v];
        const int sw = __shfl_xor(lo ? x2 : x0, 16, 64);
        const int d0 = lo ? x0 : x1, d2 = lo ? x1 : x2;
        const int64_t sum = static_cast<int64_t>(d0) + 256 * static_cast<int64_t>(sw) + 65536 * static_cast<int64_t>(d2);
        y[t] = static_cast<float>(sum) * p2;
      }
      const int base = row0 + (wr * TI + i) * 32 + 8 * q + 4 * kh;  // rows base .. base + 3
      if constexpr (EPI == kEpiSwiglu) {
        float o2[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int row = base + 2 * h;
          const float g = y[2 * h] * S[min(row, rows - 1)];
          const float u = y[2 * h + 1] * S[min(row + 1, rows - 1)];
          o2[h] = g / (1.0f + expf(-g)) * u;
        }
        if (vec && base + 3 < rows) {
          *reinterpret_cast<float2*>(orow + (base >> 1)) = make_float2(o2[0], o2[1]);
        } else {
#pragma unroll
          for (int h = 0; h < 2; ++h)
            if (base + 2 * h + 1 < rows) orow[static_cast<int64_t>((base >> 1) + h) * osr] = o2[h];
        }
      } else {
        float o4[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) o4[t] = y[t] * S[min(base + t, rows - 1)];
        if (vec && base + 3 < rows) {
          float4* dst = reinterpret_cast<float4*>(orow + base);
          if constexpr (EPI == kEpiAdd) {
            const float4 old = *dst;
            *dst = make_float4(old.x + o4[0], old.y + o4[1], old.z + o4[2], old.w + o4[3]);
          } else {
            *dst = make_float4(o4[0], o4[1], o4[2], o4[3]);
          }
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (base + t < rows) {
              float* o = orow + static_cast<int64_t>(base + t) * osr;
              if (EPI == kEpiAdd) *o = *o + o4[t];
              else *o = o4[t];
            }
        }
      }
    }
  }
}

template <int EPI, int TI, int WRW, int WCW>
void go_tile_shape(const int8_t* W, int64_t ldw, const float* S, const int8_t* D, int kpad, int nrows,
                   const float* pow2, float* O, int64_t osb, int64_t osr, int rows, int tiles_n, hipStream_t st) {
  using Sh = tile::Shape<TI, WRW, WCW>;
  static bool raised = false;
  if (!raised && Sh::kSmem > 65536) {
    PIA_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemm_tile<EPI, TI, WRW, WCW>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(Sh::kSmem)));
    raised = true;
  }
  hipLaunchKernelGGL((k_gemm_tile<EPI, TI, WRW, WCW>), dim3((rows + Sh::kBM - 1) / Sh::kBM, tiles_n),
                     dim3(Sh::kThreads), Sh::kSmem, st, W, ldw, S, D, kpad, nrows, pow2, O, osb, osr, rows);
}

// `chunks` whole 64-entry chunks of digits from D (pow2 and O at the same first entry): the
// 256 x 384 tile over pairs of chunks when its grid gives every CU at least two workgroups,
// the 128 x 192 tile otherwise and for an odd last chunk.
template <int EPI>
void go_tile(const int8_t* W, int64_t ldw, const float* S, const int8_t* D, int kpad, int nrows, const float* pow2,
             float* O, int64_t osb, int64_t osr, int rows, int chunks, hipStream_t st) {
  int dev = 0, cus = 0;
  PIA_HIP(hipGetDevice(&dev));
  PIA_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const int64_t big_grid = static_cast<int64_t>((rows + tile::Big::kBM - 1) / tile::Big::kBM) * (chunks / 2);
  const bool big = big_grid >= 2 * cus;
  int done = 0;
  if (big) {
    go_tile_shape<EPI, 4, 2, 4>(W, ldw, S, D, kpad, nrows, pow2, O, osb, osr, rows, chunks / 2, st);
    done = chunks / 2 * 2;
  }
  if (done < chunks) {
    const int64_t b0 = 64 * static_cast<int64_t>(done);
    go_tile_shape<EPI, 2, 2, 2>(W, ldw, S, D + 3 * b0 * 64, kpad, nrows, pow2 + b0, O + b0 * osb, osb, osr, rows,
                                chunks - done, st);
  }
}

}  // namespace

int64_t digit_groups(int64_t batch) { return (batch + 15) / 16; }

int64_t xdigits_bytes(int64_t batch, int64_t cols) {
  const int64_t kpad = (cols + 63) / 64 * 64, g = digit_groups(batch);
  return (48 * g * kpad + 255) / 256 * 256 + 16 * g * 4;
}

void launch_xdigits(const float* x, int64_t ldx, const float* norm_w, float eps, int64_t batch, int64_t cols,
                    void* xq, hipStream_t st) {
  PIA_REQUIRE(batch > 0 && cols > 0 && cols < (int64_t(1) << 30), "xdigits: bad shape");
  const int64_t kpad = (cols + 63) / 64 * 64;
  const int64_t n = 48 * digit_groups(batch);
  int8_t* dig = static_cast<int8_t*>(xq);
  float* pow2 = reinterpret_cast<float*>(dig + (n * kpad + 255) / 256 * 256);
  const int64_t groups = n / 3;  // entries written (batch rows, padded with zero rows to whole groups)
  const bool vec = cols % 4 == 0 && ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                   (!norm_w || (reinterpret_cast<uintptr_t>(norm_w) & 15) == 0);
  const int64_t v4 = (cols / 4 + 63) / 64;  // float4 per lane
  if (vec && v4 <= 64) {
    // Four wavefronts (one workgroup) per row: the launch is latency-bound, and spreading a row
    // over 256 lanes shortens each lane's load / reduce / store chain (batch 32: 13.8 k vs
    // 13.2 k tok/s with one wavefront per 2048-float row; Llama-3-8B batch 64: 8.30 k vs 8.13 k
    // with two per 4096); at most 16 float4 per lane in registers.
#define PIA_XDW(V, W)                                                                                            \
  hipLaunchKernelGGL((k_xdigits_wave<V, W>), dim3(static_cast<unsigned>((groups + 4 / W - 1) / (4 / W))), dim3(256), \
                     0, st, x, ldx, norm_w, eps, static_cast<int>(cols), static_cast<int>(batch),                 \
                     static_cast<int>(groups), static_cast<int>(kpad), static_cast<int>(n), dig, pow2)
    if (v4 <= 8) PIA_XDW(2, 4);
    else if (v4 <= 16) PIA_XDW(4, 4);
    else if (v4 <= 32) PIA_XDW(8, 4);
    else PIA_XDW(16, 4);
#undef PIA_XDW
  } else {
    hipLaunchKernelGGL(k_xdigits, dim3(static_cast<unsigned>(groups)), dim3(kThreads), 0, st, x, ldx, norm_w, eps,
                       static_cast<int>(cols), static_cast<int>(batch), static_cast<int>(kpad), static_cast<int>(n), dig,
                       pow2);
  }
  PIA_HIP(hipGetLastError());
}

int64_t dec_split_bytes(int64_t pairs) { return pairs * 128 * 64 * 8 + pairs * 4; }

DecSplitWork dec_split_work(void* base, int64_t pairs) {
  return DecSplitWork{static_cast<unsigned long long*>(base),
                      reinterpret_cast<unsigned*>(static_cast<char*>(base) + pairs * 128 * 64 * 8), pairs};
}

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
  const int64_t n = 48 * digit_groups(batch);
  const float* pow2 = reinterpret_cast<const float*>(dig + (n * kpad + 255) / 256 * 256);
  const int r = static_cast<int>(rows), k = static_cast<int>(kpad), nr = static_cast<int>(n);
  // Chunks of 64 batch entries (4 groups, 192 digit rows) along grid.y, then the ragged
  // remainder as its own launch.
  const int64_t full = batch / 64;
  auto launch = [&](int64_t b0, int64_t chunks, int nb) {
    const int8_t* D = dig + 3 * b0 * 64;  // b0 is a multiple of 64: whole groups (rows 3 b0 ..)
    float* O = out + b0 * osb;
    unsigned long long* am = amax ? amax + b0 * kArgmaxSlots : nullptr;
    const float* p2 = pow2 + b0;
    const int c = static_cast<int>(chunks);
    switch (digit_groups(nb)) {
      case 1: go_dec<1>(W, ldw, scales, D, k, nr, p2, O, osb, osr, r, nb, c, epi, am, split, st); break;
      case 2: go_dec<2>(W, ldw, scales, D, k, nr, p2, O, osb, osr, r, nb, c, epi, am, split, st); break;
      case 3: go_dec<3>(W, ldw, scales, D, k, nr, p2, O, osb, osr, r, nb, c, epi, am, split, st); break;
      default: go_dec<4>(W, ldw, scales, D, k, nr, p2, O, osb, osr, r, nb, c, epi, am, split, st); break;
    }
  };
  if (full >= kTileMinChunks && !amax) {
    // Many batch entries (prefill): the LDS-tiled kernel over the whole 64-entry chunks.
    if (epi == Epi::Add) go_tile<kEpiAdd>(W, ldw, scales, dig, k, nr, pow2, out, osb, osr, r, static_cast<int>(full), st);
    else if (epi == Epi::Swiglu) go_tile<kEpiSwiglu>(W, ldw, scales, dig, k, nr, pow2, out, osb, osr, r, static_cast<int>(full), st);
    else go_tile<kEpiStore>(W, ldw, scales, dig, k, nr, pow2, out, osb, osr, r, static_cast<int>(full), st);
  } else if (full) {
    launch(0, full, 64);
  }
  if (batch % 64) launch(full * 64, 1, static_cast<int>(batch % 64));
  PIA_HIP(hipGetLastError());
}

}  // namespace pia
