// Paged-attention decode over the refcounted block pool (src/attention.rs:141-264).
//
// One workgroup per (token split, kv head, entry): the G = num_heads / num_kv_heads query
// heads that share a kv head are handled together, so every K and V vector is read from HBM
// once per entry and used for all G heads (the reference's grouped lanes,
// src/attention.rs:12-21). The block table is resolved once per token into LDS and
// unmapped logical blocks score -inf (src/attention.rs:233-240). The window is split along
// the token axis so that short batches still fill the chip; each split keeps its max and
// sum, and the last split of an (entry, kv head) to finish combines them (log-sum-exp). That
// is exact algebra of the reference's full-window softmax with a different rounding order.
//
// FUSED variant (decode batches whose entries never read a slot another entry writes): the
// workgroup also applies NeoX RoPE to its q heads and, in the split holding the entry's own
// position, rotates k, writes k and v into the cache and uses them straight from LDS
// (src/model.rs:1068-1107 then :1111-1118), so a decode layer's attention is one launch.
#include <cfloat>
#include <cstdlib>

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

struct AttnParams {
  const float* q;  // query rows (raw qkv rows when fused)
  int64_t ldq;
  float* out;
  int64_t ldo;
  float* kv;
  int64_t layer_slots;  // layer * num_blocks * block_size
  int block_size, hkv, hd, heads;
  float scale;
  const pia_attn_entry* entries;
  const int32_t* tables;
  int split, nsplit, chunk;
  // Partial outputs of split s go to split slot split_base + s of nstride slots per (entry,
  // head); the slots below split_base belong to the shared-prefix launch.
  int split_base, nstride;
  float* part_o;
  float* part_ml;
  const float* rope_cos;
  const float* rope_sin;
};

// HD: compile-time head_dim (0 = runtime p.hd, for unusual shapes); every loop over the head
// dimension and over the tokens of a chunk issues its loads before their first use.
//
// A workgroup owns the tokens [t0, t1) of one (entry, kv head): the whole window when
// p.nsplit == 1, else one split. It walks them in chunks of 256 / TPT tokens with a running
// (online) softmax: per chunk the new maximum rescales the running sum and the V accumulators.
template <int G, int HD, int TPT, bool FUSED>
__global__ __launch_bounds__(kThreads) void k_attn(AttnParams p) {
  extern __shared__ __align__(16) float smem[];
  const int hd = HD ? HD : p.hd;
  constexpr int kChunk = kThreads / TPT;                    // tokens per chunk
  float* qs = smem;                                         // [G][hd]
  float* sc = qs + G * hd;                                  // [G][kChunk]
  float* stat = sc + G * kChunk;                            // [G][4]: m, l, alpha, -
  float* knew = stat + 4 * G;                               // [hd]  (fused: this entry's k)
  float* vnew = knew + hd;                                  // [hd]
  int* slot_of = reinterpret_cast<int*>(vnew + hd);         // [kChunk]
  float* red = reinterpret_cast<float*>(slot_of + kChunk);  // [ngrp][G][hd]

  const int s = blockIdx.x, kvh = blockIdx.y, e = blockIdx.z;
  const int tid = threadIdx.x;
  const pia_attn_entry en = p.entries[e];
  const int t0 = en.start + s * p.split;
  const int t1 = min(en.pos + 1, t0 + p.split);
  const int half = hd / 2;
  const float* qrow = p.q + static_cast<int64_t>(e) * p.ldq;
  const bool own = FUSED && en.pos >= t0 && en.pos < t1;  // this workgroup holds the entry's token
  const int64_t kv_head_stride = 2 * static_cast<int64_t>(hd);
  auto kv_at = [&](int slot) { return p.kv + ((p.layer_slots + slot) * p.hkv + kvh) * kv_head_stride; };

  if (FUSED) {
    const float* c = p.rope_cos + static_cast<int64_t>(en.pos) * half;
    const float* sn = p.rope_sin + static_cast<int64_t>(en.pos) * half;
    for (int i = tid; i < G * half; i += kThreads) {
      const int g = i / half, j = i % half;
      const float* qh = qrow + (kvh * G + g) * hd;
      const float a = qh[j], b = qh[j + half];
      qs[g * hd + j] = a * c[j] - b * sn[j];
      qs[g * hd + j + half] = b * c[j] + a * sn[j];
    }
    if (own) {
      int own_slot = -1;
      const int lb = en.pos / p.block_size;
      if (lb < en.table_len) own_slot = p.tables[en.table_off + lb] * p.block_size + en.pos % p.block_size;
      const float* kr = qrow + (p.heads + kvh) * hd;
      const float* vr = qrow + (p.heads + p.hkv + kvh) * hd;
      float* dst = own_slot >= 0 ? kv_at(own_slot) : nullptr;
      for (int j = tid; j < half; j += kThreads) {
        const float a = kr[j], b = kr[j + half];
        const float r0 = a * c[j] - b * sn[j];
        const float r1 = b * c[j] + a * sn[j];
        knew[j] = r0;
        knew[j + half] = r1;
        if (dst) dst[j] = r0, dst[j + half] = r1;
      }
      for (int d = tid; d < hd; d += kThreads) {
        vnew[d] = vr[d];
        if (dst) dst[hd + d] = vr[d];
      }
    }
  } else {
    for (int i = tid; i < G * hd; i += kThreads) qs[i] = qrow[kvh * G * hd + i];
  }
  if (tid < G) {
    stat[4 * tid] = -INFINITY;
    stat[4 * tid + 1] = 0.0f;
  }

  const int tpg = hd / 4;
  const int ngrp = kThreads / tpg;
  const int grp = tid / tpg, d4 = (tid % tpg) * 4;
  float o[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g) o[g][0] = o[g][1] = o[g][2] = o[g][3] = 0.0f;

  for (int c0 = t0; c0 < t1; c0 += kChunk) {
    const int count = min(kChunk, t1 - c0);
    if (tid < kChunk) {
      int slot = -1;
      if (tid < count) {
        const int t = c0 + tid;
        const int lb = t / p.block_size;
        if (lb < en.table_len) slot = p.tables[en.table_off + lb] * p.block_size + (t % p.block_size);
      }
      slot_of[tid] = slot;
    }
    __syncthreads();

    // Scores: TPT threads per token, each covering hd / TPT dims, reduced by lane shuffles.
    {
      const int tok = tid / TPT, part = tid % TPT;
      const int seg = hd / TPT;
      const int slot = tok < count ? slot_of[tok] : -1;
      float acc[G];
#pragma unroll
      for (int g = 0; g < G; ++g) acc[g] = 0.0f;
      if (slot >= 0) {
        const float* kp = (FUSED && own && c0 + tok == en.pos) ? knew : kv_at(slot);
        kp += part * seg;
        const float* qp = qs + part * seg;
        if constexpr (HD != 0) {
          constexpr int kSeg = HD / TPT;
          float4 k4[kSeg / 4];
#pragma unroll
          for (int i = 0; i < kSeg / 4; ++i) k4[i] = reinterpret_cast<const float4*>(kp)[i];
#pragma unroll
          for (int i = 0; i < kSeg / 4; ++i)
#pragma unroll
            for (int g = 0; g < G; ++g) {
              const float4 q4 = reinterpret_cast<const float4*>(qp + g * HD)[i];
              acc[g] = __builtin_fmaf(q4.x, k4[i].x, acc[g]);
              acc[g] = __builtin_fmaf(q4.y, k4[i].y, acc[g]);
              acc[g] = __builtin_fmaf(q4.z, k4[i].z, acc[g]);
              acc[g] = __builtin_fmaf(q4.w, k4[i].w, acc[g]);
            }
        } else {
          for (int d = 0; d < seg; d += 4) {
            const float4 k4 = *reinterpret_cast<const float4*>(kp + d);
#pragma unroll
            for (int g = 0; g < G; ++g) {
              const float* qg = qp + g * hd + d;
              acc[g] = __builtin_fmaf(qg[0], k4.x, acc[g]);
              acc[g] = __builtin_fmaf(qg[1], k4.y, acc[g]);
              acc[g] = __builtin_fmaf(qg[2], k4.z, acc[g]);
              acc[g] = __builtin_fmaf(qg[3], k4.w, acc[g]);
            }
          }
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int off = TPT / 2; off >= 1; off >>= 1) acc[g] += __shfl_xor(acc[g], off, 64);
      if (part == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) sc[g * kChunk + tok] = slot >= 0 ? acc[g] * p.scale : -INFINITY;
      }
    }
    __syncthreads();

    // Running max / sum per head (one wavefront per head, round robin); sc becomes p.
    {
      const int wave = tid >> 6, lane = tid & 63;
      for (int g = wave; g < G; g += kThreads / 64) {
        float* row = sc + g * kChunk;
        float m = -INFINITY;
        for (int i = lane; i < kChunk; i += 64) m = fmaxf(m, row[i]);
        m = wave_max(m);
        const float m_old = stat[4 * g];
        const float m_new = fmaxf(m_old, m);
        float l = 0.0f;
        for (int i = lane; i < kChunk; i += 64) {
          const float pr = (m_new == -INFINITY) ? 0.0f : expf(row[i] - m_new);
          row[i] = pr;
          l += pr;
        }
        l = wave_sum(l);
        if (lane == 0) {
          const float alpha = (m_old == -INFINITY) ? 0.0f : expf(m_old - m_new);
          stat[4 * g] = m_new;
          stat[4 * g + 1] = __builtin_fmaf(stat[4 * g + 1], alpha, l);
          stat[4 * g + 2] = alpha;
        }
      }
    }
    __syncthreads();

    // V accumulation: hd/4 threads per token group, 4 consecutive dims each. With a
    // compile-time head_dim every token of the chunk a thread owns is loaded before the first
    // FMA (kChunk / ngrp loads in flight); otherwise 4 at a time.
    if (grp < ngrp) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float alpha = stat[4 * g + 2];
        o[g][0] *= alpha, o[g][1] *= alpha, o[g][2] *= alpha, o[g][3] *= alpha;
      }
      constexpr int kVTfull = HD ? kChunk / (kThreads / (HD ? HD / 4 : 1)) : 4;
      constexpr int kVT = kVTfull < 16 ? kVTfull : 16;  // tokens per thread per pass
      for (int i0 = grp; i0 < count; i0 += kVT * ngrp) {
        float4 v4[kVT];
        int idx[kVT];
#pragma unroll
        for (int u = 0; u < kVT; ++u) {
          const int i = i0 + u * ngrp;
          const int slot = i < count ? slot_of[i] : -1;
          idx[u] = slot >= 0 ? i : -1;
          if (slot >= 0) {
            const float* vp = (FUSED && own && c0 + i == en.pos) ? vnew : kv_at(slot) + hd;
            v4[u] = *reinterpret_cast<const float4*>(vp + d4);
          } else {
            v4[u] = make_float4(0.f, 0.f, 0.f, 0.f);
          }
        }
#pragma unroll
        for (int u = 0; u < kVT; ++u) {
          if (idx[u] < 0) continue;
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const float pr = sc[g * kChunk + idx[u]];
            o[g][0] = __builtin_fmaf(pr, v4[u].x, o[g][0]);
            o[g][1] = __builtin_fmaf(pr, v4[u].y, o[g][1]);
            o[g][2] = __builtin_fmaf(pr, v4[u].z, o[g][2]);
            o[g][3] = __builtin_fmaf(pr, v4[u].w, o[g][3]);
          }
        }
      }
    }
    __syncthreads();  // slot_of / sc are rewritten by the next chunk
  }

  if (grp < ngrp) {
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
    if (p.nstride == 1) {
      const float l = stat[4 * g + 1];
      p.out[static_cast<int64_t>(e) * p.ldo + h * hd + d] = l > 0.0f ? acc / l : 0.0f;
    } else {
      const int64_t ps = (static_cast<int64_t>(e) * p.heads + h) * p.nstride + p.split_base + s;
      p.part_o[ps * hd + d] = acc;
      if (d == 0) {
        p.part_ml[2 * ps] = stat[4 * g];
        p.part_ml[2 * ps + 1] = stat[4 * g + 1];
      }
    }
  }
}

// Log-sum-exp combine of the splits of one (entry, head): all loads issued up front.
__global__ __launch_bounds__(kMaxHd) void k_attn_combine(const float* __restrict__ part_o,
                                                         const float* __restrict__ part_ml, float* __restrict__ out,
                                                         int64_t ldo, int heads, int hd, int nsplit) {
  __shared__ float w[kThreads / 2];
  __shared__ float lsum;
  const int eh = blockIdx.x;
  const int e = eh / heads, h = eh % heads;
  const int t = threadIdx.x;
  const float* ml = part_ml + static_cast<int64_t>(eh) * nsplit * 2;
  // The first kPre splits' outputs do not depend on the maxima: their loads go out with them.
  constexpr int kPre = 16;
  const float* po = part_o + static_cast<int64_t>(eh) * nsplit * hd + t;
  float pv[kPre];
#pragma unroll
  for (int u = 0; u < kPre; ++u) pv[u] = (t < hd && u < nsplit) ? po[static_cast<int64_t>(u) * hd] : 0.0f;
  // nsplit <= 128 = blockDim: thread k owns split k.
  const float mk = t < nsplit ? ml[2 * t] : -INFINITY;
  const float lk = t < nsplit ? ml[2 * t + 1] : 0.0f;
  float m = mk;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  __shared__ float mw[2];
  if ((t & 63) == 0) mw[t >> 6] = m;
  __syncthreads();
  m = fmaxf(mw[0], mw[1]);
  const float wk = (m == -INFINITY || mk == -INFINITY) ? 0.0f : expf(mk - m);
  if (t < nsplit) w[t] = wk;
  float l = lk * wk;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) l += __shfl_xor(l, off, 64);
  __shared__ float lw[2];
  if ((t & 63) == 0) lw[t >> 6] = l;
  __syncthreads();
  if (t == 0) lsum = lw[0] + lw[1];
  __syncthreads();
  if (t >= hd) return;
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < kPre; ++u)
    if (u < nsplit) acc = __builtin_fmaf(pv[u], w[u], acc);
  int k = kPre;
  for (; k + 8 <= nsplit; k += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = po[static_cast<int64_t>(k + u) * hd];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = __builtin_fmaf(v[u], w[k + u], acc);
  }
  for (; k < nsplit; ++k) acc = __builtin_fmaf(po[static_cast<int64_t>(k) * hd], w[k], acc);
  out[static_cast<int64_t>(e) * ldo + h * hd + t] = lsum > 0.0f ? acc / lsum : 0.0f;
}

// ---------------------------------------------------------------------------------------
// Prefill attention: the entries of one launch are consecutive positions of one sequence
// sharing one block table (prefill_batched, src/model.rs:1222-1255), and their K/V are
// already in the cache. The same kernel runs the shared-prefix decode pass (SHARED).
//
// A workgroup owns kRowsTile = 64 query rows of one kv head, 16 per wave: row r is query
// r / G, head kvh * G + r % G (QT = 64 / G consecutive positions times the G heads of the
// group). It walks the tokens its positions attend to in chunks of kRc, staged in LDS, so each
// K and V row is read once per 64 rows instead of once per G; the next chunk's block ids are
// resolved and its K/V loads are in flight during the current chunk. Per wave and chunk the
// scores are formed transposed, S^T = K Q^T, on the f32 matrix cores (v_mfma_f32_16x16x4f32;
// each lane's dims are one contiguous quarter of the head, so its K reads are 16-byte and the
// dot is the same sum in another order). In that layout the lane holding a score is the lane
// that feeds it to P.V as the A operand, so softmax and P.V run from registers with no round
// trip of P through LDS. The output dims are permuted per lane (column c holds dims
// c * HD / 16 ..) so V is read in 16-byte pieces too; the per-row rescale factors reach the
// output layout by shuffles.
constexpr int kRowsTile = 64;
constexpr int kPfPad = 4;  // floats of padding per LDS row of K and V (bank spread)
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct PfParams {
  const float* q;  // rows [n][ldq]: head h at column h * hd (post-RoPE)
  int64_t ldq;
  float* out;
  int64_t ldo;
  const float* kv;
  int64_t layer_slots;
  int block_size, hkv, heads, n;
  float scale;
  const pia_attn_entry* entries;
  const int32_t* tables;
  // Shared-prefix decode (SHARED): entries are virtual, one per (member, shared split) of a
  // group of decode entries whose tables share their leading blocks; vmap[2 v] is the real
  // entry whose (raw, un-rotated) q row the virtual entry v reads, vmap[2 v + 1] its split
  // slot. RoPE at the real entry's position is applied while Q is staged, and the raw
  // (max, sum, output) partials go to part_ml / part_o as k_attn's splits do.
  const int* vmap;
  const pia_attn_entry* real;
  const float* rope_cos;
  const float* rope_sin;
  float* part_o;
  float* part_ml;
  int nstride;
};

template <int HD>
constexpr int rows_chunk() {
  return HD <= 64 ? 64 : 32;
}

template <int G, int HD, bool SHARED>
__device__ __forceinline__ void attn_tile(const PfParams& p, int tile) {
  constexpr int R = kRowsTile;        // query rows per workgroup
  constexpr int QT = R / G;           // query positions per workgroup
  constexpr int kRc = rows_chunk<HD>();
  constexpr int TT = kRc / 16;        // token tiles per chunk
  constexpr int DQ = HD / 4;          // dims per lane quarter in S^T
  constexpr int DT = HD / 16;         // output dim tiles (dims per lane column)
  constexpr int KS = HD + kPfPad;     // LDS row stride of K and V (floats)
  constexpr int KV4 = kRc * HD / 4 / kThreads;  // float4 of K (and of V) per thread per chunk
  static_assert(HD % 64 == 0 && QT >= 1 && KV4 >= 1 && kThreads == 256, "row-tiled attention shape");
  extern __shared__ __align__(16) float smem[];
  float* Ks = smem;                    // [kRc][KS]
  float* Vs = Ks + kRc * KS;           // [kRc][KS]
  float* qstage = smem;                // [R][HD] query rows, before the first chunk only
  static_assert(2 * kRc * KS >= R * HD, "the query rows are staged where K/V go");
  // Per chunk c, in buffer c % 3 (resolved two chunks ahead): block ids, whether every token
  // is mapped, and the float offset of each token's K row.
  int* slots = reinterpret_cast<int*>(Vs + kRc * KS);  // [3][kRc]
  int* qpos = slots + 3 * kRc;         // [QT]
  int* qstart = qpos + QT;             // [QT]
  int* mapped = qstart + QT;           // [4]
  int64_t* rowoff = reinterpret_cast<int64_t*>(mapped + 4);  // [3][kRc]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int j16 = lane & 15, q4 = lane >> 4;
  const int kvh = blockIdx.y;
  const int e0 = tile * QT;
  const pia_attn_entry first = p.entries[e0];
  const int table_off = first.table_off, table_len = first.table_len;
  for (int i = tid; i < QT; i += kThreads) {
    const int e = e0 + i;
    if (e < p.n) {
      const pia_attn_entry en = p.entries[e];
      qpos[i] = en.pos;
      qstart[i] = en.start;
    } else {
      qpos[i] = -1;
      qstart[i] = 0x7fffffff;
    }
  }
  if constexpr (SHARED) {
    constexpr int half = HD / 2;
    for (int i = tid; i < R * half; i += kThreads) {
      const int r = i / half, jj = i % half;
      const int e = e0 + r / G;
      float a = 0.0f, b = 0.0f;
      if (e < p.n) {
        const int er = p.vmap[2 * e];
        const int pos = p.real[er].pos;
        const float* qh = p.q + static_cast<int64_t>(er) * p.ldq + (kvh * G + r % G) * HD;
        const float c = p.rope_cos[static_cast<int64_t>(pos) * half + jj];
        const float sn = p.rope_sin[static_cast<int64_t>(pos) * half + jj];
        const float x0 = qh[jj], x1 = qh[jj + half];
        a = x0 * c - x1 * sn;
        b = x1 * c + x0 * sn;
      }
      qstage[r * HD + jj] = a;
      qstage[r * HD + jj + half] = b;
    }
  } else {
    for (int i = tid; i < R * (HD / 4); i += kThreads) {
      const int r = i / (HD / 4), d = (i % (HD / 4)) * 4;
      const int e = e0 + r / G;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (e < p.n)
        v = *reinterpret_cast<const float4*>(p.q + static_cast<int64_t>(e) * p.ldq + (kvh * G + r % G) * HD + d);
      *reinterpret_cast<float4*>(qstage + r * HD + d) = v;
    }
  }
  __syncthreads();
  int lo = 0x7fffffff, hi = -1;
  for (int i = 0; i < QT; ++i)
    if (qpos[i] >= 0) lo = min(lo, qstart[i]), hi = max(hi, qpos[i]);
  if (hi < 0) return;  // uniform over the workgroup
  const int nchunks = hi >= lo ? (hi - lo) / kRc + 1 : 0;

  // This lane's row (S^T layout) and its query quarter of dims, in registers.
  const int row = wave * 16 + j16;
  const int rpos = qpos[row / G], rstart = qstart[row / G];
  float qv[DQ];
#pragma unroll
  for (int m = 0; m < DQ; m += 4) {
    const float4 v = *reinterpret_cast<const float4*>(qstage + row * HD + q4 * DQ + m);
    qv[m] = v.x, qv[m + 1] = v.y, qv[m + 2] = v.z, qv[m + 3] = v.w;
  }

  const int64_t head_stride = 2 * static_cast<int64_t>(HD);
  auto resolve = [&](int c) {
    if (tid < kRc) {
      const int b = c % 3;
      const int t = lo + c * kRc + tid;
      int slot = -1;
      if (t <= hi) {
        const int lb = t / p.block_size;
        if (lb < table_len) slot = p.tables[table_off + lb] * p.block_size + t % p.block_size;
      }
      slots[b * kRc + tid] = slot;
      // Unmapped tokens read slot 0 of the layer (always inside the cache); zeroed in LDS.
      rowoff[b * kRc + tid] = ((p.layer_slots + max(slot, 0)) * p.hkv + kvh) * head_stride;
      const unsigned long long unmapped = __ballot(slot < 0);
      if (tid == 0) mapped[b] = unmapped == 0;
    }
  };
  // The loads stay raw in registers while in flight; unmapped tokens (which read slot 0 of the
  // layer, always inside the cache) are zeroed when the chunk is written to LDS.
  float4 kreg[KV4], vreg[KV4];
  bool kept[KV4];
  auto load = [&](int c) {
    const int* sl = slots + (c % 3) * kRc;
    const int64_t* ro = rowoff + (c % 3) * kRc;
#pragma unroll
    for (int u = 0; u < KV4; ++u) {
      const int i = tid + u * kThreads;
      const int t = i / (HD / 4), d = (i % (HD / 4)) * 4;
      const float* src = p.kv + ro[t] + d;
      kreg[u] = *reinterpret_cast<const float4*>(src);
      vreg[u] = *reinterpret_cast<const float4*>(src + HD);
      kept[u] = sl[t] >= 0;
    }
  };
  auto zero_unless = [](bool keep, const float4& x) {
    return make_float4(keep ? x.x : 0.f, keep ? x.y : 0.f, keep ? x.z : 0.f, keep ? x.w : 0.f);
  };

  const float scale2 = p.scale * 1.44269504088896341f;  // softmax scale times log2(e)
  float m = -INFINITY, lsum = 0.0f;  // this lane's row: running max (base 2), partial sum over its tokens
  f32x4 acc[DT];                     // O rows 4 * q4 + v, dims j16 * DT + dt
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (nchunks > 0) {
    resolve(0);
    if (nchunks > 1) resolve(1);
    __syncthreads();
    load(0);
  }
  for (int c = 0; c < nchunks; ++c) {
    const int* cur = slots + (c % 3) * kRc;
    const bool cur_mapped = mapped[c % 3];
    const int c0 = lo + c * kRc;
#pragma unroll
    for (int u = 0; u < KV4; ++u) {
      const int i = tid + u * kThreads;
      const int t = i / (HD / 4), d = (i % (HD / 4)) * 4;
      if (cur_mapped) {
        *reinterpret_cast<float4*>(Ks + t * KS + d) = kreg[u];
        *reinterpret_cast<float4*>(Vs + t * KS + d) = vreg[u];
      } else {
        *reinterpret_cast<float4*>(Ks + t * KS + d) = zero_unless(kept[u], kreg[u]);
        *reinterpret_cast<float4*>(Vs + t * KS + d) = zero_unless(kept[u], vreg[u]);
      }
    }
    __syncthreads();
    // Buffer (c + 2) % 3 was last read in chunk c - 1; chunk c + 1's ids were resolved before
    // the last barrier, so its K/V loads go out now and are in flight for the whole chunk.
    if (c + 2 < nchunks) resolve(c + 2);
    if (c + 1 < nchunks) load(c + 1);
    // S^T tiles: token tt * 16 + 4 q4 + v, row j16 of this wave.
    // The TT tiles' dependency chains are interleaved so consecutive MFMAs are independent.
    f32x4 st[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) st[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const float* kr = Ks + j16 * KS + q4 * DQ;
#pragma unroll
    for (int m4 = 0; m4 < DQ; m4 += 4) {
      float4 k4[TT];
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) k4[tt] = *reinterpret_cast<const float4*>(kr + tt * 16 * KS + m4);
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) st[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[tt].x, qv[m4], st[tt], 0, 0, 0);
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) st[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[tt].y, qv[m4 + 1], st[tt], 0, 0, 0);
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) st[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[tt].z, qv[m4 + 2], st[tt], 0, 0, 0);
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) st[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[tt].w, qv[m4 + 3], st[tt], 0, 0, 0);
    }
    // Scale (base-2 logits: exp(x) = 2^(x log2 e)), mask, running max over the row (the 4
    // lanes j16 + 16 q share a row). A chunk inside every window of the wave's rows, with all
    // of its tokens mapped, needs no mask (the common case: all but the diagonal chunks).
    const bool full = cur_mapped && __all(c0 >= rstart && c0 + kRc - 1 <= rpos);
    float mx = -INFINITY;
    if (full) {
#pragma unroll
      for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          st[tt][v] *= scale2;
          mx = fmaxf(mx, st[tt][v]);
        }
    } else {
#pragma unroll
      for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int tk = tt * 16 + 4 * q4 + v;
          const int t = c0 + tk;
          const bool ok = cur[tk] >= 0 && t >= rstart && t <= rpos;
          st[tt][v] = ok ? st[tt][v] * scale2 : -INFINITY;
          mx = fmaxf(mx, st[tt][v]);
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m, mx);
    const float alpha = (m == -INFINITY) ? 1.0f : __builtin_amdgcn_exp2f(m - m_new);
    // A row with no visible token yet keeps m = -inf; its probabilities are 0.
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    float ps = 0.0f;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float pr = __builtin_amdgcn_exp2f(st[tt][v] - m_use);
        st[tt][v] = pr;
        ps += pr;
      }
    lsum = __builtin_fmaf(lsum, alpha, ps);
    m = m_new;
    // Output rows 4 q4 + v take the factor of the lane that owns that row in the S^T layout.
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float av = __shfl(alpha, 4 * q4 + v, 64);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt][v] *= av;
    }
    // P.V: k-step (tt, v) takes token tt * 16 + 4 q4 + v on lane quarter q4.
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float* vr = Vs + (tt * 16 + 4 * q4 + v) * KS + j16 * DT;
        float vv[DT];
#pragma unroll
        for (int d4 = 0; d4 < DT; d4 += 4) {
          const float4 x = *reinterpret_cast<const float4*>(vr + d4);
          vv[d4] = x.x, vv[d4 + 1] = x.y, vv[d4 + 2] = x.z, vv[d4 + 3] = x.w;
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(st[tt][v], vv[dt], acc[dt], 0, 0, 0);
      }
    __syncthreads();  // Ks / Vs are rewritten by the next chunk
  }
  // Row sums over the 4 lanes of each row, then moved to the output layout with the maxima.
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int orow = wave * 16 + 4 * q4 + v;
    const float lv = __shfl(lsum, 4 * q4 + v, 64);
    const float mv = __shfl(m, 4 * q4 + v, 64);
    const int e = e0 + orow / G;
    if (e >= p.n || qpos[orow / G] < 0) continue;
    const int h = kvh * G + orow % G;
    if constexpr (SHARED) {
      const int64_t ps_ = (static_cast<int64_t>(p.vmap[2 * e]) * p.heads + h) * p.nstride + p.vmap[2 * e + 1];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) p.part_o[ps_ * HD + j16 * DT + dt] = acc[dt][v];
      if (j16 == 0) {
        p.part_ml[2 * ps_] = mv * 0.69314718055994531f;  // natural-log units, as k_attn writes
        p.part_ml[2 * ps_ + 1] = lv;
      }
    } else {
      float* dst = p.out + static_cast<int64_t>(e) * p.ldo + h * HD + j16 * DT;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) dst[dt] = lv > 0.0f ? acc[dt][v] / lv : 0.0f;
    }
  }
}

// One tile per workgroup, longest windows first (shared-prefix pass: uniform work), or, for a
// causal prefill, the pair (t, ntiles - 1 - t): every workgroup then does about the same work
// and the launch has no tail of short tiles behind the long ones (TinyLlama 2048-token prefill:
// attention 5.19 -> 4.22 ms per sequence).
template <int G, int HD, bool SHARED>
__global__ __launch_bounds__(kThreads, 2) void k_attn_prefill(PfParams p, int ntiles, int paired) {
  const int x = static_cast<int>(blockIdx.x);
  const int b = ntiles - 1 - x;
  attn_tile<G, HD, SHARED>(p, b);
  if (paired && x < b) {
    __syncthreads();  // the LDS of the first tile is rewritten by the second
    attn_tile<G, HD, SHARED>(p, x);
  }
}

template <int HD>
size_t rows_smem_bytes() {
  constexpr int kRc = rows_chunk<HD>();
  constexpr int QT = kRowsTile;  // upper bound (G = 1)
  return sizeof(float) * (2 * kRc * (HD + kPfPad)) + sizeof(int) * (3 * kRc + 2 * QT + 4) + sizeof(int64_t) * 3 * kRc;
}

// Compute units of the current device (queried once per device).
int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  PIA_HIP(hipGetDevice(&dev));
  PIA_REQUIRE(dev >= 0 && dev < 64, "attention: device index out of range");
  if (cus[dev] == 0) {
    int n = 0;
    PIA_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
    cus[dev] = n > 0 ? n : 1;
  }
  return cus[dev];
}

template <int G, int HD, bool SHARED>
void go_prefill(const PfParams& p, hipStream_t st) {
  constexpr int QT = kRowsTile / G;
  const size_t smem = rows_smem_bytes<HD>();
  static bool done = false;
  if (!done) {
    PIA_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(k_attn_prefill<G, HD, SHARED>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem)));
    done = true;
  }
  const int ntiles = (p.n + QT - 1) / QT;
  // Pairing balances the causal triangle but halves the grid: it is used only where the paired
  // grid still gives every CU its two workgroups (TinyLlama 2048-token prefill: 5.19 -> 4.22 ms
  // of attention per sequence; a 256-token prefill resumed after a long prefix, 16 tiles per
  // kv head, runs about twice as long per launch when paired).
  // PIA_PREFILL_PAIR=1 / 0 forces pairing on / off (read at every launch; used by the tests).
  const char* force = std::getenv("PIA_PREFILL_PAIR");
  const bool fill = static_cast<int64_t>((ntiles + 1) / 2) * p.hkv >= 2 * static_cast<int64_t>(device_cus());
  const int paired = !SHARED && (force ? std::atoi(force) != 0 : fill);
  dim3 grid(static_cast<unsigned>(paired ? (ntiles + 1) / 2 : ntiles), static_cast<unsigned>(p.hkv));
  hipLaunchKernelGGL((k_attn_prefill<G, HD, SHARED>), grid, dim3(kThreads), smem, st, p, ntiles, paired);
}

template <int HD, bool SHARED = false>
void prefill_by_g(const PfParams& p, int g, hipStream_t st) {
  switch (g) {
    case 1: go_prefill<1, HD, SHARED>(p, st); break;
    case 2: go_prefill<2, HD, SHARED>(p, st); break;
    case 4: go_prefill<4, HD, SHARED>(p, st); break;
    case 8: go_prefill<8, HD, SHARED>(p, st); break;
    case 16: go_prefill<16, HD, SHARED>(p, st); break;
    default: fail(PIA_ERR_INVALID, "attention: kv_group must be 1, 2, 4, 8 or 16");
  }
}

size_t attn_smem_bytes(int g, int hd, int chunk) {
  const int ngrp = kThreads / (hd / 4);
  return sizeof(float) * (g * hd + g * chunk + 4 * g + 2 * hd) + sizeof(int) * chunk + sizeof(float) * ngrp * g * hd;
}

template <int G, int HD, int TPT, bool F>
void set_smem(size_t smem) {
  static bool done = false;
  if (!done && smem > 65536) {
    PIA_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(k_attn<G, HD, TPT, F>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(smem)));
    done = true;
  }
}

template <int G, int HD, int TPT>
void go(const AttnParams& p, dim3 grid, size_t smem, bool fused, hipStream_t st) {
  if (fused) {
    set_smem<G, HD, TPT, true>(smem);
    hipLaunchKernelGGL((k_attn<G, HD, TPT, true>), grid, dim3(kThreads), smem, st, p);
  } else {
    set_smem<G, HD, TPT, false>(smem);
    hipLaunchKernelGGL((k_attn<G, HD, TPT, false>), grid, dim3(kThreads), smem, st, p);
  }
}

template <int G, int HD>
void by_tpt(const AttnParams& p, dim3 grid, size_t smem, bool fused, hipStream_t st) {
  const int tpt = kThreads / p.chunk;
  if (tpt == 1) go<G, HD, 1>(p, grid, smem, fused, st);
  else if (tpt == 2) go<G, HD, 2>(p, grid, smem, fused, st);
  else go<G, HD, 4>(p, grid, smem, fused, st);
}

template <int G>
void by_hd(const AttnParams& p, dim3 grid, size_t smem, bool fused, hipStream_t st) {
  if (p.hd == 64) by_tpt<G, 64>(p, grid, smem, fused, st);
  else if (p.hd == 128) by_tpt<G, 128>(p, grid, smem, fused, st);
  else if (p.hd == 32) by_tpt<G, 32>(p, grid, smem, fused, st);
  else by_tpt<G, 0>(p, grid, smem, fused, st);
}

}  // namespace

AttnPlan plan_attention(int64_t n, int64_t num_kv_heads, int64_t head_dim, int64_t max_window, int num_cus) {
  // Enough workgroups for ~2 per CU: (entry, kv head) pairs times token splits. Small batches
  // also shrink the chunk (64 or 128 tokens spread each token over 4 or 2 threads, which needs
  // head_dim % (4 * TPT) == 0) so that short windows still split. Splits are combined by a
  // second kernel; at most kThreads / 2 of them.
  const int64_t w = std::max<int64_t>(1, max_window);
  const int64_t pairs = std::max<int64_t>(1, n * num_kv_heads);
  // Workgroups-per-CU target of the split: 2, or 4 from 512 (entry, kv head) pairs on (long
  // windows at large batches: Llama-3-8B batch 64 attention 3.41 -> 3.26 ms per step; at 128
  // pairs 4 is slower). PIA_ATTN_WGS_PER_CU overrides it.
  static const int64_t per_cu_env = [] {
    const char* e = std::getenv("PIA_ATTN_WGS_PER_CU");
    const long v = e ? std::strtol(e, nullptr, 10) : 0;
    return v > 0 ? static_cast<int64_t>(v) : int64_t(0);
  }();
  const int64_t per_cu = per_cu_env ? per_cu_env : (pairs >= 512 ? 4 : 2);
  int64_t want = (per_cu * static_cast<int64_t>(num_cus) + pairs - 1) / pairs;
  // PIA_ATTN_MAX_SPLITS caps the split count (the reference's PAGED_INFER_ATTN_LANES_PER_THREAD
  // plays the same role for its lane schedule, src/attention.rs:46-55).
  static const int64_t cap = [] {
    const char* e = std::getenv("PIA_ATTN_MAX_SPLITS");
    const long v = e ? std::strtol(e, nullptr, 10) : 0;
    return v > 0 ? static_cast<int64_t>(v) : int64_t(0);
  }();
  if (cap) want = std::min(want, cap);
  AttnPlan plan{w, 1, kThreads};
  for (int chunk : {256, 128, 64}) {
    const int tpt = kThreads / chunk;
    if (head_dim % (4 * tpt) != 0) break;
    plan.chunk = chunk;
    plan.splits = std::min<int64_t>(std::min<int64_t>((w + chunk - 1) / chunk, want), kThreads / 2);
    if (plan.splits >= want) break;
  }
  plan.splits = std::max<int64_t>(1, plan.splits);
  int64_t split = (w + plan.splits - 1) / plan.splits;
  split = (split + plan.chunk - 1) / plan.chunk * plan.chunk;
  plan.split = split;
  plan.splits = (w + split - 1) / split;
  return plan;
}

int64_t attention_tile_rows() { return kRowsTile; }

int64_t attention_work_bytes(int64_t n, int64_t heads, int64_t head_dim, int64_t splits) {
  if (splits <= 1) return 0;
  return n * heads * splits * (head_dim + 2) * static_cast<int64_t>(sizeof(float));
}

void launch_attention(const AttnLaunch& a, hipStream_t st) {
  const pia_kv_layout& L = *a.layout;
  PIA_REQUIRE(L.num_kv_heads > 0 && a.heads % L.num_kv_heads == 0,
              "attention: num_heads must be a multiple of num_kv_heads");
  PIA_REQUIRE(L.head_dim % 4 == 0 && L.head_dim <= kMaxHd, "attention: head_dim must be a multiple of 4 and <= 128");
  PIA_REQUIRE(a.layer >= 0 && a.layer < L.num_layers, "attention: layer out of range");
  PIA_REQUIRE(L.num_blocks * L.block_size < (int64_t(1) << 31), "attention: too many cache slots for int32 indexing");
  PIA_REQUIRE(a.plan.splits >= 1 && a.plan.splits <= kThreads / 2, "attention: at most 128 token splits");
  PIA_REQUIRE(a.plan.chunk == 64 || a.plan.chunk == 128 || a.plan.chunk == 256, "attention: bad chunk size");
  PIA_REQUIRE(a.plan.split >= 1 && a.plan.split % a.plan.chunk == 0, "attention: split must be whole chunks");
  PIA_REQUIRE(L.head_dim % (4 * (kThreads / a.plan.chunk)) == 0, "attention: chunk size does not fit head_dim");
  PIA_REQUIRE(a.plan.splits == 1 || a.work, "attention: split windows need a workspace");
  PIA_REQUIRE(!a.fused || (a.rope_cos && a.rope_sin), "attention: fused RoPE needs the rotary tables");
  if (a.n == 0) return;
  const int g = static_cast<int>(a.heads / L.num_kv_heads);
  const int hd = static_cast<int>(L.head_dim);
  // PIA_PREFILL_TILE_MIN overrides the entry count from which prefills use the tiled kernel.
  static const int64_t tile_min = [] {
    const char* e = std::getenv("PIA_PREFILL_TILE_MIN");
    const long v = e ? std::strtol(e, nullptr, 10) : 0;
    return v > 0 ? static_cast<int64_t>(v) : kPrefillTileMin;
  }();
  if (a.prefill && !a.fused && a.n >= tile_min && (hd == 64 || hd == 128)) {
    PIA_REQUIRE(a.n < (int64_t(1) << 31), "attention: too many entries");
    PfParams pf{a.q,       a.ldq,  a.out, a.ldo, a.kv, a.layer * L.num_blocks * L.block_size, static_cast<int>(L.block_size),
                static_cast<int>(L.num_kv_heads), static_cast<int>(a.heads), static_cast<int>(a.n),
                1.0f / sqrtf(static_cast<float>(hd)), a.entries, a.tables};
    pf.nstride = 1;
    if (hd == 64) prefill_by_g<64>(pf, g, st);
    else prefill_by_g<128>(pf, g, st);
    PIA_HIP(hipGetLastError());
    return;
  }
  AttnParams p;
  p.q = a.q;
  p.ldq = a.ldq;
  p.out = a.out;
  p.ldo = a.ldo;
  p.kv = a.kv;
  p.layer_slots = a.layer * L.num_blocks * L.block_size;
  p.block_size = static_cast<int>(L.block_size);
  p.hkv = static_cast<int>(L.num_kv_heads);
  p.hd = hd;
  p.heads = static_cast<int>(a.heads);
  p.scale = 1.0f / sqrtf(static_cast<float>(hd));
  p.entries = a.entries;
  p.tables = a.tables;
  p.split = static_cast<int>(a.plan.split);
  p.chunk = static_cast<int>(a.plan.chunk);
  p.nsplit = static_cast<int>(a.plan.splits);
  p.split_base = static_cast<int>(a.n_shared ? a.shared_splits : 0);
  p.nstride = p.split_base + p.nsplit;
  p.part_o = static_cast<float*>(a.work);
  p.part_ml = p.part_o ? p.part_o + a.n * a.heads * p.nstride * hd : nullptr;
  if (a.n_shared) {
    PIA_REQUIRE(a.fused && !a.prefill && (hd == 64 || hd == 128) && a.shared_entries && a.shared_vmap && a.work &&
                    a.shared_splits >= 1 && p.nstride <= kThreads / 2,
                "attention: shared-prefix decode needs a fused launch, head_dim 64 or 128 and a workspace");
    PfParams sp{a.q, a.ldq, nullptr, 0, a.kv, p.layer_slots, p.block_size, p.hkv, p.heads,
                static_cast<int>(a.n_shared), p.scale, a.shared_entries, a.tables, a.shared_vmap, a.entries,
                a.rope_cos, a.rope_sin, p.part_o, p.part_ml, p.nstride};
    if (hd == 64) prefill_by_g<64, true>(sp, g, st);
    else prefill_by_g<128, true>(sp, g, st);
    PIA_HIP(hipGetLastError());
  }
  p.rope_cos = a.rope_cos;
  p.rope_sin = a.rope_sin;
  dim3 grid(static_cast<unsigned>(a.plan.splits), static_cast<unsigned>(L.num_kv_heads), static_cast<unsigned>(a.n));
  const size_t smem = attn_smem_bytes(g, hd, static_cast<int>(a.plan.chunk));
  switch (g) {
    case 1: by_hd<1>(p, grid, smem, a.fused, st); break;
    case 2: by_hd<2>(p, grid, smem, a.fused, st); break;
    case 4: by_hd<4>(p, grid, smem, a.fused, st); break;
    case 8: by_hd<8>(p, grid, smem, a.fused, st); break;
    case 16: by_hd<16>(p, grid, smem, a.fused, st); break;
    default: fail(PIA_ERR_INVALID, "attention: kv_group must be 1, 2, 4, 8 or 16");
  }
  PIA_HIP(hipGetLastError());
  if (p.nstride > 1) {
    hipLaunchKernelGGL(k_attn_combine, dim3(static_cast<unsigned>(a.n * a.heads)), dim3(kMaxHd), 0, st, p.part_o,
                       p.part_ml, a.out, a.ldo, static_cast<int>(a.heads), hd, p.nstride);
    PIA_HIP(hipGetLastError());
  }
}

}  // namespace pia
