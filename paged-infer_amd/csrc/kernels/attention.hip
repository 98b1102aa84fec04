// Paged-attention decode over the refcounted block pool (src/attention.rs:141-264).
//
// One workgroup per (token split, kv head, entry): the G = num_heads / num_kv_heads query
// heads that share a kv head are handled together, so every K and V vector is read from HBM
// once per entry and used for all G heads (the reference's grouped lanes,
// src/attention.rs:12-21). The block table is resolved once per token into LDS and
// unmapped logical blocks score -inf (src/attention.rs:233-240). Long windows are split
// along the token axis; each split keeps its running max and sum and a second kernel
// combines them (log-sum-exp), which is exact algebra of the reference's full-window
// softmax with a different rounding order.
#include <cfloat>

#include "common.h"
#include "kernels.h"

namespace pia {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxHd = 128;

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int G>
__global__ __launch_bounds__(kThreads) void k_attn(const float* __restrict__ q, int64_t ldq, float* __restrict__ out,
                                                   int64_t ldo, const float* __restrict__ kv, int64_t layer_slots,
                                                   int block_size, int hkv, int hd, float scale,
                                                   const pia_attn_entry* __restrict__ entries,
                                                   const int32_t* __restrict__ tables, int split, int nsplit,
                                                   float* __restrict__ part_o, float* __restrict__ part_ml) {
  extern __shared__ float smem[];
  float* qs = smem;                                              // [G][hd]
  float* sc = qs + G * hd;                                       // [G][kThreads]
  float* stat = sc + G * kThreads;                               // [G][2]
  int* slot_of = reinterpret_cast<int*>(stat + 2 * G);           // [kThreads]
  float* red = reinterpret_cast<float*>(slot_of + kThreads);     // [ngrp][G][hd]

  const int s = blockIdx.x, kvh = blockIdx.y, e = blockIdx.z;
  const int tid = threadIdx.x;
  const pia_attn_entry en = entries[e];
  const int heads = hkv * G;
  const int t0 = en.start + s * split;
  const int t1 = min(en.pos + 1, t0 + split);
  const int count = max(0, t1 - t0);

  for (int i = tid; i < G * hd; i += kThreads) qs[i] = q[static_cast<int64_t>(e) * ldq + kvh * G * hd + i];
  {
    int slot = -1;
    const int t = t0 + tid;
    if (tid < count) {
      const int lb = t / block_size;
      if (lb < en.table_len) slot = tables[en.table_off + lb] * block_size + (t % block_size);
    }
    slot_of[tid] = slot;
  }
  __syncthreads();

  // Scores: thread tid <-> token t0 + tid.
  {
    const int slot = slot_of[tid];
    float acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = 0.0f;
    if (slot >= 0) {
      const float* kp = kv + ((static_cast<int64_t>(layer_slots) + slot) * hkv + kvh) * 2 * hd;
      for (int d = 0; d < hd; d += 4) {
        const float4 k4 = *reinterpret_cast<const float4*>(kp + d);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float* qg = qs + g * hd + d;
          acc[g] = __builtin_fmaf(qg[0], k4.x, acc[g]);
          acc[g] = __builtin_fmaf(qg[1], k4.y, acc[g]);
          acc[g] = __builtin_fmaf(qg[2], k4.z, acc[g]);
          acc[g] = __builtin_fmaf(qg[3], k4.w, acc[g]);
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) sc[g * kThreads + tid] = acc[g] * scale;
    } else {
#pragma unroll
      for (int g = 0; g < G; ++g) sc[g * kThreads + tid] = -INFINITY;
    }
  }
  __syncthreads();

  // Per-head max and sum of exp over this split (one wavefront per head, round robin).
  {
    const int wave = tid >> 6, lane = tid & 63;
    for (int g = wave; g < G; g += kThreads / 64) {
      float* row = sc + g * kThreads;
      float m = -INFINITY;
      for (int i = lane; i < kThreads; i += 64) m = fmaxf(m, row[i]);
      m = wave_max(m);
      float l = 0.0f;
      for (int i = lane; i < kThreads; i += 64) {
        const float p = (m == -INFINITY) ? 0.0f : expf(row[i] - m);
        row[i] = p;
        l += p;
      }
      l = wave_sum(l);
      if (lane == 0) {
        stat[2 * g] = m;
        stat[2 * g + 1] = l;
      }
    }
  }
  __syncthreads();

  // V accumulation: hd/4 threads per token group, each owning 4 consecutive dims.
  const int tpg = hd / 4;
  const int ngrp = kThreads / tpg;
  const int grp = tid / tpg, d4 = (tid % tpg) * 4;
  if (grp < ngrp) {
    float o[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) o[g][0] = o[g][1] = o[g][2] = o[g][3] = 0.0f;
    for (int i = grp; i < count; i += ngrp) {
      const int slot = slot_of[i];
      if (slot < 0) continue;
      const float4 v4 =
          *reinterpret_cast<const float4*>(kv + ((static_cast<int64_t>(layer_slots) + slot) * hkv + kvh) * 2 * hd + hd + d4);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float p = sc[g * kThreads + i];
        o[g][0] = __builtin_fmaf(p, v4.x, o[g][0]);
        o[g][1] = __builtin_fmaf(p, v4.y, o[g][1]);
        o[g][2] = __builtin_fmaf(p, v4.z, o[g][2]);
        o[g][3] = __builtin_fmaf(p, v4.w, o[g][3]);
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[(grp * G + g) * hd + d4 + j] = o[g][j];
  }
  __syncthreads();

  for (int idx = tid; idx < G * hd; idx += kThreads) {
    float acc = 0.0f;
    for (int gr = 0; gr < ngrp; ++gr) acc += red[gr * G * hd + idx];
    const int g = idx / hd, d = idx % hd;
    const int h = kvh * G + g;
    if (nsplit == 1) {
      const float l = stat[2 * g + 1];
      out[static_cast<int64_t>(e) * ldo + h * hd + d] = l > 0.0f ? acc / l : 0.0f;
    } else {
      const int64_t ps = (static_cast<int64_t>(e) * heads + h) * nsplit + s;
      part_o[ps * hd + d] = acc;
      if (d == 0) {
        part_ml[2 * ps] = stat[2 * g];
        part_ml[2 * ps + 1] = stat[2 * g + 1];
      }
    }
  }
}

// Log-sum-exp combine of the token splits of one (entry, head).
__global__ __launch_bounds__(kMaxHd) void k_attn_combine(const float* __restrict__ part_o,
                                                         const float* __restrict__ part_ml, float* __restrict__ out,
                                                         int64_t ldo, int heads, int hd, int nsplit) {
  const int eh = blockIdx.x;
  const int e = eh / heads, h = eh % heads;
  const int d = threadIdx.x;
  const float* ml = part_ml + static_cast<int64_t>(eh) * nsplit * 2;
  float m = -INFINITY;
  for (int s = 0; s < nsplit; ++s) m = fmaxf(m, ml[2 * s]);
  if (d >= hd) return;
  float val = 0.0f;
  if (m != -INFINITY) {
    float l = 0.0f, acc = 0.0f;
    for (int s = 0; s < nsplit; ++s) {
      const float ms = ml[2 * s];
      if (ms == -INFINITY) continue;
      const float w = expf(ms - m);
      l = __builtin_fmaf(ml[2 * s + 1], w, l);
      acc = __builtin_fmaf(part_o[(static_cast<int64_t>(eh) * nsplit + s) * hd + d], w, acc);
    }
    val = l > 0.0f ? acc / l : 0.0f;
  }
  out[static_cast<int64_t>(e) * ldo + h * hd + d] = val;
}

size_t attn_smem_bytes(int g, int hd) {
  const int ngrp = kThreads / (hd / 4);
  return sizeof(float) * (g * hd + g * kThreads + 2 * g) + sizeof(int) * kThreads + sizeof(float) * ngrp * g * hd;
}

}  // namespace

int64_t attention_splits(int64_t max_window) { return max_window <= kThreads ? 1 : (max_window + kThreads - 1) / kThreads; }

int64_t attention_work_bytes(int64_t n, int64_t heads, int64_t head_dim, int64_t splits) {
  if (splits <= 1) return 0;
  return n * heads * splits * (head_dim + 2) * static_cast<int64_t>(sizeof(float));
}

void launch_attention(const float* q, int64_t ldq, float* out, int64_t ldo, const float* kv,
                      const pia_kv_layout& L, int64_t heads, const pia_attn_entry* entries, const int32_t* tables,
                      int64_t n, int64_t layer, int64_t splits, void* work, hipStream_t st) {
  PIA_REQUIRE(L.num_kv_heads > 0 && heads % L.num_kv_heads == 0,
              "attention: num_heads must be a multiple of num_kv_heads");
  PIA_REQUIRE(L.head_dim % 4 == 0 && L.head_dim <= kMaxHd, "attention: head_dim must be a multiple of 4 and <= 128");
  PIA_REQUIRE(layer >= 0 && layer < L.num_layers, "attention: layer out of range");
  PIA_REQUIRE(L.num_blocks * L.block_size < (int64_t(1) << 31), "attention: too many cache slots for int32 indexing");
  PIA_REQUIRE(splits >= 1 && splits < 65536, "attention: bad split count");
  PIA_REQUIRE(splits == 1 || work != nullptr, "attention: split-K needs a workspace");
  if (n == 0) return;
  const int g = static_cast<int>(heads / L.num_kv_heads);
  const int hd = static_cast<int>(L.head_dim);
  const float scale = 1.0f / sqrtf(static_cast<float>(hd));
  const int64_t layer_slots = layer * L.num_blocks * L.block_size;
  float* part_o = static_cast<float*>(work);
  float* part_ml = part_o ? part_o + n * heads * splits * hd : nullptr;
  dim3 grid(static_cast<unsigned>(splits), static_cast<unsigned>(L.num_kv_heads), static_cast<unsigned>(n));
  const size_t smem = attn_smem_bytes(g, hd);
  const int bs = static_cast<int>(L.block_size), hkv = static_cast<int>(L.num_kv_heads);
  const int ns = static_cast<int>(splits);
#define PIA_ATTN_CASE(GV)                                                                                  \
  case GV:                                                                                                 \
    hipLaunchKernelGGL(k_attn<GV>, grid, dim3(kThreads), smem, st, q, ldq, out, ldo, kv, layer_slots, bs, hkv, \
                       hd, scale, entries, tables, kThreads, ns, part_o, part_ml);                         \
    break;
  if (smem > 65536) {
    static bool raised[17] = {};
    if (!raised[g]) {
      const void* fn = g == 16 ? reinterpret_cast<const void*>(k_attn<16>) : reinterpret_cast<const void*>(k_attn<8>);
      PIA_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem)));
      raised[g] = true;
    }
  }
  switch (g) {
    PIA_ATTN_CASE(1)
    PIA_ATTN_CASE(2)
    PIA_ATTN_CASE(4)
    PIA_ATTN_CASE(8)
    PIA_ATTN_CASE(16)
    default:
      fail(PIA_ERR_INVALID, "attention: kv_group must be 1, 2, 4, 8 or 16");
  }
#undef PIA_ATTN_CASE
  PIA_HIP(hipGetLastError());
  if (splits > 1) {
    hipLaunchKernelGGL(k_attn_combine, dim3(static_cast<unsigned>(n * heads)), dim3(kMaxHd), 0, st, part_o, part_ml,
                       out, ldo, static_cast<int>(heads), hd, ns);
    PIA_HIP(hipGetLastError());
  }
}

}  // namespace pia
