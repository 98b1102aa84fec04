// Persistent batch-1 decode step: one launch runs every layer and the LM head
// (decode_batch_into at batch 1, src/model.rs:1184-1207 -> run_layers_batch :968-1177).
//
// Why: at batch 1 a TinyLlama layer streams 47 MB of int8 weights in ~6 MB pieces, and a
// separate launch per piece pays launch and first-byte latency that is larger than the
// transfer itself. Here one workgroup per CU stays resident for the whole step and the
// pieces are separated by grid barriers instead of kernel boundaries. Each wave streams
// its rows of every projection through a ring of kRing weight slices; the next projection's
// first slices are issued before the barrier that precedes it, so they arrive while the
// workgroup waits.
//
// Stages of one layer (each ends in a grid barrier):
//   A  qkv = Wqkv . RMSNorm(x) * attn_norm            (rows split over all waves)
//   B  attention: NeoX RoPE on q and this token's k, K/V write into the paged cache, online
//      softmax over a token split of one kv head (all q heads of its group); the last split
//      of a kv head to finish combines the splits (log-sum-exp) into attn
//   D  x += Wo . attn                                  (residual kept in the owning lanes)
//   E  h = SwiGLU(Wgu . RMSNorm(x) * ffn_norm)         (gate/up rows interleaved in HBM)
//   F  x += Wdown . h
// then logits = Wlm . RMSNorm(x) * final_norm with the greedy argmax fused.
//
// Cross-workgroup data (qkv, partials, attn, x, h) moves through agent-scope relaxed atomic
// loads and stores, which gfx950 performs at the device coherence point (the per-XCD L2s
// are not coherent with each other); every wave waits for its stores before its
// workgroup raises its barrier flag. A barrier wait that exceeds its spin budget sets an
// error flag that every workgroup checks, so the grid always drains.
#include <cfloat>

#include "common.h"
#include "kernels.h"

namespace pia {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kRound = 4;        // weight slices per half of the double buffer
constexpr int kFlagStride = 32;  // u32 words between barrier flags (one 128-byte line each)
constexpr int kSpinLimit = 1 << 20;
constexpr int kMinSplitTokens = 16;

template <typename T>
__device__ inline T ald(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ inline void ast(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ inline unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const unsigned long long o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}
// f32 -> u32 preserving f32::total_cmp order (src/sampling.rs:140-147).
__device__ inline uint32_t order_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// ---------------------------------------------------------------------------------------
// Grid barrier: workgroup g publishes flags[g * kFlagStride] = epoch; every workgroup waits
// until all flags have reached the epoch (wrap-safe compare). Returns false when the kernel
// must stop (a barrier timed out somewhere).
// ---------------------------------------------------------------------------------------
struct Sync {
  unsigned* flags;
  int* err;
  unsigned epoch;
};

// The wave that polls the flags. It streams no weights: a poll load cannot complete before
// every older load of its wave has returned, so it must have none in flight.
constexpr int kPollWave = kWaves - 1;

// Arrival: every wave of the workgroup has waited for its own stores (s_waitcnt vmcnt(0));
// then the workgroup's flag goes up. The flag store is issued before the next stage's weight
// loads, so it does not queue behind them.
__device__ void grid_arrive(Sync& s) {
  ++s.epoch;
  __syncthreads();
  if (threadIdx.x == 0) ast(&s.flags[blockIdx.x * kFlagStride], s.epoch);
}

// Wait until every workgroup's flag has reached the epoch (wrap-safe compare). Returns false
// when the kernel must stop (a wait ran out of its spin budget somewhere).
__device__ bool grid_wait(Sync& s, int* abort_lds) {
  if ((threadIdx.x >> 6) == kPollWave) {
    // Lane i watches flags i, i + 64, ...: all of them are loaded together each round and
    // the wave leaves when every flag has reached the epoch.
    const int lane = threadIdx.x & 63;
    const int nwg = static_cast<int>(gridDim.x);
    for (int spins = 0;; ++spins) {
      unsigned v[kThreads / 64];
#pragma unroll
      for (int k = 0; k < kThreads / 64; ++k) {
        const int w = lane + 64 * k;
        v[k] = w < nwg ? ald(&s.flags[w * kFlagStride]) : s.epoch;
      }
      bool done = true;
#pragma unroll
      for (int k = 0; k < kThreads / 64; ++k) done = done && static_cast<int>(v[k] - s.epoch) >= 0;
      if (__all(done)) break;
      if (spins > kSpinLimit) {
        if (lane == 0) ast(s.err, 1);
        *abort_lds = 1;
        break;
      }
      if ((spins & 63) == 63 && ald(s.err)) {
        *abort_lds = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
  return *abort_lds == 0;
}

// ---------------------------------------------------------------------------------------
// Weight stream. A unit is a pair of rows (row pairs keep a SwiGLU gate/up pair in one
// wave); a slice is one unit x one chunk of columns (64 lanes x 16 int8).
// ---------------------------------------------------------------------------------------
struct Seg {
  const char* base;  // matrix bytes
  int64_t ld_bytes;  // row stride in bytes
  int rows, K, nch;  // rows; valid columns; chunks per row
  int u0, u1;        // this wave's units
};

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// Pointers read from the layer table are generic to the compiler, which would make their
// loads flat loads; flat loads also count against the LDS wait counter, so every LDS read of
// the activations would wait for the weights in flight. These casts keep them global loads.
template <typename T>
__device__ inline const __attribute__((address_space(1))) T* gptr(const T* p) {
  return (const __attribute__((address_space(1))) T*)p;
}

// Double-buffered weight stream: while the slices of one round (buffer A or B) are multiplied,
// the next round's loads are in flight in the other buffer. The loads are ordinary
// (compiler-tracked) loads and every round issues exactly 2 * kRound of them, so the wait
// before a round's first use is a fixed count of younger loads.
struct Stream {
  static constexpr int kPer = 16;  // int8 per lane per chunk
  static constexpr int kChunk = 64 * kPer;
  v4i A[kRound][2], B[kRound][2];
  // Load cursor: the segment being loaded and its next unit / chunk. Past the segment's last
  // slice the stream issues dummy loads (of a row the wave already read), so every round is
  // the same number of loads.
  Seg cur;
  int lu, lc;

  __device__ static void widen(const v4i& v, float (&w)[16]) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) w[4 * k + j] = static_cast<float>((v[k] << (24 - 8 * j)) >> 24);
  }
  __device__ __forceinline__ void load_round(v4i (&buf)[kRound][2], int lane) {
#pragma unroll
    for (int j = 0; j < kRound; ++j) {
      const bool real = lu < cur.u1;
      const int col0 = (real ? lc : 0) * kChunk + lane * kPer;
      const int col = col0 < cur.K ? col0 : 0;  // lanes past the row read its start (times zero)
      // Dummy slices re-read the wave's own first row (or, with no rows, a row near its
      // share): spread over the matrix, they hit in L2 instead of piling onto one line.
      const int r0 = real ? 2 * lu : min(2 * cur.u0, cur.rows - 1);
      const int64_t o0 = static_cast<int64_t>(r0) * cur.ld_bytes + col;
      const int64_t o1 = real && r0 + 1 < cur.rows ? o0 + cur.ld_bytes : o0;
      buf[j][0] = *gptr(reinterpret_cast<const v4i*>(cur.base + o0));
      buf[j][1] = *gptr(reinterpret_cast<const v4i*>(cur.base + o1));
      if (real && ++lc == cur.nch) lc = 0, ++lu;
    }
  }
  // Start streaming segment s: its first round goes in flight (into A).
  __device__ __forceinline__ void prime(const Seg& s, int lane) {
    cur = s;
    lu = s.u0;
    lc = 0;
    load_round(A, lane);
  }
  // Slices i0 .. i0 + kRound - 1 (those below n) of the current unit walk.
  __device__ __forceinline__ void compute_round(const v4i (&buf)[kRound][2], int i0, int n, int nch, const float* xs,
                                                int lane, int& cu, int& cc, float& a0, float& a1, float& res0,
                                                float& res1) {
#pragma unroll
    for (int j = 0; j < kRound; ++j) {
      if (i0 + j < n) {
        float w0[kPer], w1[kPer], xv[kPer];
        const float* xp = xs + cc * kChunk + lane * kPer;
#pragma unroll
        for (int q = 0; q < kPer / 4; ++q) {
          const float4 v = reinterpret_cast<const float4*>(xp)[q];
          xv[4 * q] = v.x, xv[4 * q + 1] = v.y, xv[4 * q + 2] = v.z, xv[4 * q + 3] = v.w;
        }
        widen(buf[j][0], w0);
        widen(buf[j][1], w1);
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
          a0 = __builtin_fmaf(w0[q], xv[q], a0);
          a1 = __builtin_fmaf(w1[q], xv[q], a1);
        }
        if (++cc == nch) {
          const float t0 = wave_sum(a0), t1 = wave_sum(a1);
          if (lane == cu) res0 = t0, res1 = t1;
          a0 = a1 = 0.0f;
          cc = 0;
          ++cu;
        }
      }
    }
  }
  // Multiply this wave's units of segment `s` (primed: its first round is in A) by the
  // activations xs (LDS, zero padded to nch * kChunk). Unit k's two raw dot products end up
  // in lane k's res0 / res1.
  __device__ __forceinline__ void run(const Seg& s, const float* xs, int lane, float& res0, float& res1) {
    const int n = (s.u1 - s.u0) * s.nch;
    int cu = 0, cc = 0;
    float a0 = 0.0f, a1 = 0.0f;
    for (int i = 0; i < n; i += 2 * kRound) {
      load_round(B, lane);
      compute_round(A, i, n, s.nch, xs, lane, cu, cc, a0, a1, res0, res1);
      load_round(A, lane);
      compute_round(B, i + kRound, n, s.nch, xs, lane, cu, cc, a0, a1, res0, res1);
    }
  }
};

// ---------------------------------------------------------------------------------------
// The step.
// ---------------------------------------------------------------------------------------
// Units of `rows` owned by global wave w out of nw: an even split of the row pairs.
// w == nw (the polling wave) owns nothing.
__device__ inline void wave_units(int rows, int w, int nw, int& u0, int& u1) {
  const int units = (rows + 1) / 2;
  u0 = static_cast<int>(static_cast<int64_t>(units) * w / nw);
  u1 = w < nw ? static_cast<int>(static_cast<int64_t>(units) * (w + 1) / nw) : u0;
}

__device__ inline int ws_u0(int rows, int w, int nw) {
  int u0, u1;
  wave_units(rows, w, nw, u0, u1);
  return u0;
}
__device__ inline int ws_units(int rows, int w, int nw) {
  int u0, u1;
  wave_units(rows, w, nw, u0, u1);
  return u1 - u0;
}

__device__ inline Seg make_seg(const void* W, int64_t ld, int rows, int K, int w, int nw) {
  Seg s;
  s.base = static_cast<const char*>(W);
  s.ld_bytes = ld;
  s.rows = rows;
  s.K = K;
  s.nch = (K + Stream::kChunk - 1) / Stream::kChunk;
  wave_units(rows, w, nw, s.u0, s.u1);
  return s;
}

__device__ inline float block_sum(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) t += red[w];
  return t;
}
__device__ inline float block_max(float v, float* red) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) t = fmaxf(t, red[w]);
  return t;
}

// Load n floats of a vector into LDS (coherent loads when other workgroups wrote it), zero
// padded to npad; with norm_w, RMSNorm(v) * norm_w (src/math.rs:4-22) instead.
__device__ void load_vec(const float* src, int n, int npad, const float* norm_w, float eps, float* xs, float* red) {
  // All loads of the vector are issued before the first use (n <= kVecPer * kThreads).
  constexpr int kVecPer = 32;
  float v[kVecPer];
#pragma unroll
  for (int u = 0; u < kVecPer; ++u) {
    const int i = threadIdx.x + u * kThreads;
    v[u] = i < n ? ald(src + i) : 0.0f;
  }
  float ss = 0.0f;
#pragma unroll
  for (int u = 0; u < kVecPer; ++u) {
    const int i = threadIdx.x + u * kThreads;
    if (i < npad) xs[i] = v[u];
    ss += v[u] * v[u];
  }
  if (norm_w) {
    const float t = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(t / static_cast<float>(n) + eps);
    const auto* nw = gptr(norm_w);
    for (int i = threadIdx.x; i < n; i += kThreads) xs[i] = (xs[i] * inv) * nw[i];
  }
  __syncthreads();
}

// The embedding row of the token (bf16 widened, src/model.rs:1015-1020), normalized.
__device__ void load_embed(const StepParams& p, int tok, int npad, const float* norm_w, float* xs, float* red) {
  const uint16_t* row = p.embed + static_cast<int64_t>(tok) * p.hidden;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < p.hidden; i += kThreads) {
    const float v = __uint_as_float(static_cast<uint32_t>(row[i]) << 16);
    xs[i] = v;
    ss += v * v;
  }
  for (int i = p.hidden + threadIdx.x; i < npad; i += kThreads) xs[i] = 0.0f;
  const float t = block_sum(ss, red);
  const float inv = 1.0f / sqrtf(t / static_cast<float>(p.hidden) + p.eps);
  const auto* nw = gptr(norm_w);
  for (int i = threadIdx.x; i < p.hidden; i += kThreads) xs[i] = (xs[i] * inv) * nw[i];
  __syncthreads();
}

// Token split of the attention window start..=pos: S splits of T tokens per kv head.
__device__ inline void attn_split(const pia_attn_entry en, int max_splits, int& S, int& T) {
  const int W = en.pos + 1 - en.start;
  S = min(max_splits, max(1, (W + kMinSplitTokens - 1) / kMinSplitTokens));
  T = (W + S - 1) / S;
}

// Log-sum-exp combine of the S splits of the G q heads of kv head kvh (the reference's single
// softmax over the whole window, src/math.rs:405-426, regrouped):
// attn[h] = sum_s w_s o_s / sum_s w_s l_s with w_s = exp(m_s - max_s m_s).
template <int HD>
__device__ void combine_group(const StepParams& p, int kvh, int S, float* lds) {
  const int G = p.heads / p.hkv;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  float* ml = lds;          // [G][S][2]
  float* w = ml + 2 * G * S;  // [G][S]
  float* lsum = w + G * S;  // [G]
  const float* part = p.part + static_cast<int64_t>(kvh * G) * S * (HD + 2);
  for (int i = tid; i < G * S; i += kThreads) {
    const float* q = part + static_cast<int64_t>(i) * (HD + 2) + HD;  // i = g * S + s
    ml[2 * i] = ald(q);
    ml[2 * i + 1] = ald(q + 1);
  }
  __syncthreads();
  for (int g = wave; g < G; g += kWaves) {
    float m = -INFINITY;
    for (int k = lane; k < S; k += 64) m = fmaxf(m, ml[2 * (g * S + k)]);
    m = wave_max(m);
    float l = 0.0f;
    for (int k = lane; k < S; k += 64) {
      const float mk = ml[2 * (g * S + k)];
      const float wk = (m == -INFINITY || mk == -INFINITY) ? 0.0f : expf(mk - m);
      w[g * S + k] = wk;
      l += ml[2 * (g * S + k) + 1] * wk;
    }
    l = wave_sum(l);
    if (lane == 0) lsum[g] = l;
  }
  __syncthreads();
  for (int idx = tid; idx < G * HD; idx += kThreads) {
    const int g = idx / HD, d = idx % HD;
    const float* po = part + static_cast<int64_t>(g) * S * (HD + 2) + d;
    float acc = 0.0f;
    int k = 0;
    for (; k + 8 <= S; k += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = ald(po + (k + u) * (HD + 2));
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = __builtin_fmaf(v[u], w[g * S + k + u], acc);
    }
    for (; k < S; ++k) acc = __builtin_fmaf(ald(po + k * (HD + 2)), w[g * S + k], acc);
    const float l = lsum[g];
    ast(p.attn + (kvh * G + g) * HD + d, l > 0.0f ? acc / l : 0.0f);
  }
  __syncthreads();
}

// One attention work item (src/attention.rs:141-264 for one kv head and a token range):
// tokens [t0, t1) of kv head kvh for all G q heads of its group. Writes per q head the
// split's max m, exp-sum l and unnormalized sum_t p_t V_t; the last split of the kv head to
// finish then combines the group into attn.
// LDS: qs[G][HD], kn[HD], vn[HD], slot[T], sc[G][T], st[G][2].
template <int HD>
__device__ void attn_item(const StepParams& p, int layer, int kvh, int s, int S, int T, const pia_attn_entry en,
                          float* lds) {
  const int G = p.heads / p.hkv;
  constexpr int half = HD / 2;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  float* qs = lds;
  float* kn = qs + G * HD;
  float* vn = kn + HD;
  int* slot = reinterpret_cast<int*>(vn + HD);
  float* sc = reinterpret_cast<float*>(slot + T);
  float* st = sc + G * T;
  const int t0 = en.start + s * T;
  const int t1 = min(en.pos + 1, t0 + T);
  const int cnt = max(0, t1 - t0);
  const bool own = en.pos >= t0 && en.pos < t1;
  const float* c = p.rope_cos + static_cast<int64_t>(en.pos) * half;
  const float* sn = p.rope_sin + static_cast<int64_t>(en.pos) * half;
  const int64_t layer_slots = static_cast<int64_t>(layer) * p.num_blocks * p.block_size;
  auto kv_at = [&](int sl) { return p.kv + ((layer_slots + sl) * p.hkv + kvh) * (2 * HD); };

  // q heads of the group, NeoX-rotated (src/math.rs:343-367, src/model.rs:1068-1080).
  for (int i = tid; i < G * half; i += kThreads) {
    const int g = i / half, j = i % half;
    float* qh = p.qkv_buf + (kvh * G + g) * HD;
    const float a = ald(qh + j), b = ald(qh + j + half);
    qs[g * HD + j] = a * c[j] - b * sn[j];
    qs[g * HD + j + half] = b * c[j] + a * sn[j];
  }
  for (int i = tid; i < cnt; i += kThreads) {
    const int t = t0 + i;
    const int lb = t / p.block_size;
    slot[i] = lb < en.table_len ? p.tables[en.table_off + lb] * p.block_size + t % p.block_size : -1;
  }
  if (own) {
    // This token's k (rotated once per kv head, src/model.rs:1081-1091) and v, written into
    // the cache when its block is mapped (src/model.rs:868-878).
    const int lb = en.pos / p.block_size;
    const int own_slot = lb < en.table_len ? p.tables[en.table_off + lb] * p.block_size + en.pos % p.block_size : -1;
    float* kr = p.qkv_buf + (p.heads + kvh) * HD;
    float* vr = p.qkv_buf + (p.heads + p.hkv + kvh) * HD;
    float* dst = own_slot >= 0 ? kv_at(own_slot) : nullptr;
    for (int j = tid; j < half; j += kThreads) {
      const float a = ald(kr + j), b = ald(kr + j + half);
      const float r0 = a * c[j] - b * sn[j];
      const float r1 = b * c[j] + a * sn[j];
      kn[j] = r0;
      kn[j + half] = r1;
      if (dst) dst[j] = r0, dst[j + half] = r1;
    }
    for (int d = tid; d < HD; d += kThreads) {
      const float v = ald(vr + d);
      vn[d] = v;
      if (dst) dst[HD + d] = v;
    }
  }
  __syncthreads();

  // Scores s_t = dot(q_g, K_t) * (1/sqrt(hd)); unmapped tokens -inf (src/attention.rs:233-240).
  for (int idx = tid; idx < G * cnt; idx += kThreads) {
    const int g = idx / cnt, i = idx % cnt;
    const int sl = slot[i];
    float v = -INFINITY;
    if (sl >= 0) {
      // This token's k is in LDS; the others are read from the cache (separate paths keep
      // the cache reads global loads rather than generic ones).
      const bool mine = own && t0 + i == en.pos;
      const auto* kg = gptr(reinterpret_cast<const v4f*>(kv_at(sl)));
      const v4f* kl = reinterpret_cast<const v4f*>(kn);
      const v4f* qg = reinterpret_cast<const v4f*>(qs + g * HD);
      float acc = 0.0f;
      // K in blocks of 32 floats: each block's loads are in flight together.
      constexpr int kB = HD < 32 ? HD / 4 : 8;
#pragma unroll
      for (int q0 = 0; q0 < HD / 4; q0 += kB) {
        v4f k4[kB];
#pragma unroll
        for (int q = 0; q < kB; ++q) {
          const v4f kv_g = kg[q0 + q];  // a valid address in either case
          k4[q] = mine ? kl[q0 + q] : kv_g;
        }
#pragma unroll
        for (int q = 0; q < kB; ++q) {
          const v4f q4 = qg[q0 + q];
          acc = __builtin_fmaf(q4.x, k4[q].x, acc);
          acc = __builtin_fmaf(q4.y, k4[q].y, acc);
          acc = __builtin_fmaf(q4.z, k4[q].z, acc);
          acc = __builtin_fmaf(q4.w, k4[q].w, acc);
        }
      }
      v = acc * p.scale;
    }
    sc[g * T + i] = v;
  }
  __syncthreads();
  // Max and exp-sum per q head (one wave per head); sc becomes p.
  for (int g = wave; g < G; g += kWaves) {
    float m = -INFINITY;
    for (int i = lane; i < cnt; i += 64) m = fmaxf(m, sc[g * T + i]);
    m = wave_max(m);
    float l = 0.0f;
    for (int i = lane; i < cnt; i += 64) {
      const float pr = m == -INFINITY ? 0.0f : expf(sc[g * T + i] - m);
      sc[g * T + i] = pr;
      l += pr;
    }
    l = wave_sum(l);
    if (lane == 0) st[2 * g] = m, st[2 * g + 1] = l;
  }
  __syncthreads();
  // o[g][d] = sum_t p[g][t] V_t[d]: thread (g, d), the V loads of 8 tokens in flight.
  for (int idx = tid; idx < G * HD; idx += kThreads) {
    const int g = idx / HD, d = idx % HD;
    float acc = 0.0f;
    for (int i0 = 0; i0 < cnt; i0 += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = i0 + u;
        const int sl = i < cnt ? slot[i] : -1;
        v[u] = sl >= 0 ? ((own && t0 + i == en.pos) ? vn[d] : *gptr(kv_at(sl) + HD + d)) : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = i0 + u;
        if (i < cnt && slot[i] >= 0) acc = __builtin_fmaf(sc[g * T + i], v[u], acc);
      }
    }
    const int h = kvh * G + g;
    float* out = p.part + (static_cast<int64_t>(h) * S + s) * (HD + 2);
    ast(out + d, acc);
    if (d == 0) {
      ast(out + HD, st[2 * g]);
      ast(out + HD + 1, st[2 * g + 1]);
    }
  }
  // The last split of this kv head to finish combines all of them: its counter increment
  // comes after every other split's (completed) partial stores.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  int* last = reinterpret_cast<int*>(lds);
  if (tid == 0) {
    unsigned* cnt = p.attn_cnt + kvh * kFlagStride;
    const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *last = old == static_cast<unsigned>(S - 1);
    if (*last) ast(cnt, 0u);  // ready for the next layer (whose splits start after a grid barrier)
  }
  __syncthreads();
  const bool do_combine = *last != 0;
  __syncthreads();
  if (do_combine) combine_group<HD>(p, kvh, S, lds);
}

// Optional stage timestamps (workgroup 0, device wall clock), for tuning.
#define PIA_STEP_MARK(i)                                                   \
  do {                                                                     \
    if (p.trace && blockIdx.x == 0 && threadIdx.x == 0) p.trace[i] = wall_clock64(); \
  } while (0)
// Latest arrival over all workgroups (at a stage's end, before its barrier).
#define PIA_STEP_ARRIVE(i)                                                                     \
  do {                                                                                         \
    if (p.trace && threadIdx.x == 0)                                                          \
      __hip_atomic_fetch_max(p.trace + 16 * p.layers + 2 + (i), wall_clock64(), __ATOMIC_RELAXED, \
                             __HIP_MEMORY_SCOPE_AGENT);                                        \
  } while (0)

template <int HD>
__global__ __launch_bounds__(kThreads) void k_decode_step(StepParams p) {
  extern __shared__ __align__(16) float lds[];
  __shared__ float red[kWaves];
  __shared__ int abort_flag;
  const int lane = threadIdx.x & 63;
  // Projection rows go to the kWaves - 1 streaming waves of each workgroup; the polling wave
  // gets none (gw == nw: an empty share), so it never has weight loads in flight when it
  // polls, and no stage waits on its late start.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = gridDim.x * (kWaves - 1);
  const int gw = wave == kPollWave ? nw : blockIdx.x * (kWaves - 1) + wave;
  if (threadIdx.x == 0) abort_flag = 0;
  Sync sy{p.flags, p.err, ald(p.step_ctr) * 1024u};
  const pia_attn_entry en = p.entry[0];
  const int tok = static_cast<int>(static_cast<int64_t>(static_cast<uint32_t>(p.token[0])) % p.vocab);
  if (blockIdx.x == 0 && threadIdx.x < kArgmaxSlots) ast(p.amax + threadIdx.x, 0ull);

  // Residual stream rows owned by this wave (the o and down projections' rows): lane k holds
  // rows 2(u0+k) and 2(u0+k)+1, starting from the embedding.
  int xu0, xu1;
  wave_units(p.hidden, gw, nw, xu0, xu1);
  float xr0 = 0.0f, xr1 = 0.0f;
  {
    const int k = xu0 + lane;
    const uint16_t* row = p.embed + static_cast<int64_t>(tok) * p.hidden;
    if (k < xu1) {
      xr0 = __uint_as_float(static_cast<uint32_t>(row[2 * k]) << 16);
      if (2 * k + 1 < p.hidden) xr1 = __uint_as_float(static_cast<uint32_t>(row[2 * k + 1]) << 16);
    }
  }
  const int pad_h = (p.hidden + 1023) / 1024 * 1024;
  const int pad_i = (p.inter + 1023) / 1024 * 1024;
  int S, T;
  attn_split(en, p.max_splits, S, T);

  Stream ws;
  ws.prime(make_seg(p.L[0].qkv, p.ld_h, p.qkv_rows, p.hidden, gw, nw), lane);
  // End of a stage: own stores complete, the workgroup's flag up, the next segment's first
  // round in flight (streaming waves only), then the wait for every other workgroup.
  const bool poller = wave == kPollWave;
  auto stage_end = [&](const Seg* next, int mark) -> bool {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    PIA_STEP_ARRIVE(mark);
    grid_arrive(sy);
    if (next && !poller) ws.prime(*next, lane);
    return grid_wait(sy, &abort_flag);
  };

  for (int l = 0; l < p.layers; ++l) {
    const StepLayer L = p.L[l];
    // Segment descriptors are built where they are used (few scalar registers live at once).
    auto seg_o = [&] { return make_seg(L.o, p.ld_h, p.hidden, p.hidden, gw, nw); };
    auto seg_gu = [&] { return make_seg(L.gu, p.ld_h, 2 * p.inter, p.hidden, gw, nw); };
    auto seg_dn = [&] { return make_seg(L.down, p.ld_i, p.hidden, p.inter, gw, nw); };
    auto seg_next = [&] {
      return l + 1 < p.layers ? make_seg(p.L[l + 1].qkv, p.ld_h, p.qkv_rows, p.hidden, gw, nw)
                              : make_seg(p.lm, p.ld_lm, p.vocab, p.hidden, gw, nw);
    };
    float r0 = 0.0f, r1 = 0.0f;

    // A: qkv = Wqkv . RMSNorm(x) * attn_norm (src/model.rs:1047-1066).
    if (l == 0) load_embed(p, tok, pad_h, L.attn_norm, lds, red);
    else load_vec(p.x, p.hidden, pad_h, L.attn_norm, p.eps, lds, red);
    PIA_STEP_MARK(16 * l + 0);
    {
      const Seg sq = make_seg(L.qkv, p.ld_h, p.qkv_rows, p.hidden, gw, nw);
      ws.run(sq, lds, lane, r0, r1);
    }
    if (lane < ws_units(p.qkv_rows, gw, nw)) {
      const int row = 2 * (ws_u0(p.qkv_rows, gw, nw) + lane);
      ast(p.qkv_buf + row, r0 * gptr(L.qkv_s)[row]);
      if (row + 1 < p.qkv_rows) ast(p.qkv_buf + row + 1, r1 * gptr(L.qkv_s)[row + 1]);
    }
    PIA_STEP_MARK(16 * l + 1);
    {
      const Seg sn = seg_o();
      if (!stage_end(&sn, 16 * l + 1)) return;
    }
    PIA_STEP_MARK(16 * l + 2);

    // B: attention over (kv head, token split) items; the last split of each kv head
    // combines its group into attn.
    for (int it = blockIdx.x; it < p.hkv * S; it += gridDim.x) attn_item<HD>(p, l, it / S, it % S, S, T, en, lds);
    PIA_STEP_MARK(16 * l + 3);
    if (!stage_end(nullptr, 16 * l + 3)) return;
    PIA_STEP_MARK(16 * l + 4);
    PIA_STEP_MARK(16 * l + 5);
    PIA_STEP_MARK(16 * l + 6);

    // D: x += Wo . attn (src/model.rs:1120-1129).
    load_vec(p.attn, p.hidden, pad_h, nullptr, 0.0f, lds, red);
    PIA_STEP_MARK(16 * l + 7);
    ws.run(seg_o(), lds, lane, r0, r1);
    if (lane < xu1 - xu0) {
      const int row = 2 * (xu0 + lane);
      xr0 = xr0 + r0 * gptr(L.o_s)[row];
      ast(p.x + row, xr0);
      if (row + 1 < p.hidden) {
        xr1 = xr1 + r1 * gptr(L.o_s)[row + 1];
        ast(p.x + row + 1, xr1);
      }
    }
    PIA_STEP_MARK(16 * l + 8);
    {
      const Seg sn = seg_gu();
      if (!stage_end(&sn, 16 * l + 8)) return;
    }
    PIA_STEP_MARK(16 * l + 9);

    // E: h = SwiGLU(Wgu . RMSNorm(x) * ffn_norm) (src/model.rs:1131-1160, src/math.rs:293-302).
    load_vec(p.x, p.hidden, pad_h, L.ffn_norm, p.eps, lds, red);
    PIA_STEP_MARK(16 * l + 10);
    ws.run(seg_gu(), lds, lane, r0, r1);
    if (lane < ws_units(2 * p.inter, gw, nw)) {
      const int row = 2 * (ws_u0(2 * p.inter, gw, nw) + lane);
      const float g = r0 * gptr(L.gu_s)[row];
      const float u = r1 * gptr(L.gu_s)[row + 1];
      const float silu = g / (1.0f + expf(-g));
      ast(p.h + (row >> 1), silu * u);
    }
    PIA_STEP_MARK(16 * l + 11);
    {
      const Seg sn = seg_dn();
      if (!stage_end(&sn, 16 * l + 11)) return;
    }
    PIA_STEP_MARK(16 * l + 12);

    // F: x += Wdown . h (src/model.rs:1162-1167).
    load_vec(p.h, p.inter, pad_i, nullptr, 0.0f, lds, red);
    PIA_STEP_MARK(16 * l + 13);
    ws.run(seg_dn(), lds, lane, r0, r1);
    if (lane < xu1 - xu0) {
      const int row = 2 * (xu0 + lane);
      xr0 = xr0 + r0 * gptr(L.down_s)[row];
      ast(p.x + row, xr0);
      if (row + 1 < p.hidden) {
        xr1 = xr1 + r1 * gptr(L.down_s)[row + 1];
        ast(p.x + row + 1, xr1);
      }
    }
    PIA_STEP_MARK(16 * l + 14);
    {
      const Seg sn = seg_next();
      if (!stage_end(&sn, 16 * l + 14)) return;
    }
  }

  // LM head on RMSNorm(x) * final_norm with the greedy argmax fused (src/model.rs:1199-1206,
  // src/sampling.rs:140-147: the last maximal index wins, so ties keep the larger row).
  PIA_STEP_MARK(16 * p.layers);
  load_vec(p.x, p.hidden, pad_h, p.final_norm, p.eps, lds, red);
  float r0 = 0.0f, r1 = 0.0f;
  const Seg s_lm = make_seg(p.lm, p.ld_lm, p.vocab, p.hidden, gw, nw);
  ws.run(s_lm, lds, lane, r0, r1);
  unsigned long long cand = 0;
  if (lane < s_lm.u1 - s_lm.u0) {
    const int row = 2 * (s_lm.u0 + lane);
    const float y0 = r0 * gptr(p.lm_s)[row];
    p.logits[row] = y0;
    cand = (static_cast<unsigned long long>(order_key(y0)) << 32) | static_cast<uint32_t>(row);
    if (row + 1 < p.vocab) {
      const float y1 = r1 * gptr(p.lm_s)[row + 1];
      p.logits[row + 1] = y1;
      const unsigned long long c1 = (static_cast<unsigned long long>(order_key(y1)) << 32) | static_cast<uint32_t>(row + 1);
      cand = c1 > cand ? c1 : cand;
    }
  }
  cand = wave_max_u64(cand);
  if (lane == 0 && cand)
    __hip_atomic_fetch_max(p.amax + (gw & (kArgmaxSlots - 1)), cand, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  PIA_STEP_MARK(16 * p.layers + 1);
  // Every workgroup read the step counter before the first barrier; the next step's epochs
  // start above all of this step's.
  if (blockIdx.x == 0 && threadIdx.x == 0) ast(p.step_ctr, ald(p.step_ctr) + 1u);
}

template <int HD>
void go(const StepParams& p, int nwg, size_t smem, hipStream_t st) {
  static bool raised = false;
  if (!raised) {
    PIA_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(k_decode_step<HD>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kMaxStepSmem)));
    raised = true;
  }
  hipLaunchKernelGGL((k_decode_step<HD>), dim3(nwg), dim3(kThreads), smem, st, p);
}

template <int HD>
int occupancy() {
  static int occ = -1;
  if (occ < 0) {
    PIA_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(k_decode_step<HD>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kMaxStepSmem)));
    int v = 0;
    PIA_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, k_decode_step<HD>, kThreads, kMaxStepSmem));
    occ = v;
  }
  return occ;
}

}  // namespace

size_t decode_step_smem(const StepShape& s) {
  const int64_t pad = std::max((s.hidden + 1023) / 1024 * 1024, (s.inter + 1023) / 1024 * 1024);
  const int64_t g = s.heads / s.hkv;
  const int64_t attn = g * s.hd + 2 * s.hd + s.max_tokens + g * s.max_tokens + 2 * g;
  return static_cast<size_t>(std::max<int64_t>({pad, attn, s.max_splits})) * 4;
}

const char* decode_step_unsupported(const StepShape& s, int num_cus) {
  if (!s.lm_i8) return "the LM head must be int8";
  if (num_cus < 1 || num_cus > kThreads) return "one workgroup per CU: at most 512 CUs (one barrier flag per thread)";
  if (s.hd != 32 && s.hd != 64 && s.hd != 128) return "head_dim must be 32, 64 or 128";
  if (s.hkv <= 0 || s.heads % s.hkv != 0) return "num_heads must be a multiple of num_kv_heads";
  if (s.heads / s.hkv > 64) return "kv group too large";
  if (s.hidden % 2 != 0) return "hidden size must be even";
  if (s.hidden > 32 * kThreads || s.inter > 32 * kThreads) return "hidden or FFN size above 16384";
  const int64_t nw = static_cast<int64_t>(num_cus) * (kWaves - 1);
  for (int64_t rows : {s.qkv_rows, s.hidden, 2 * s.inter, s.vocab})
    if ((rows + 1) / 2 > 64 * nw) return "a projection has more than 64 row pairs per wave";
  if (s.max_splits < 1 || s.max_splits > kThreads) return "bad token split count";
  if (decode_step_smem(s) > kMaxStepSmem) return "activations do not fit in LDS";
  const int occ = s.hd == 32 ? occupancy<32>() : s.hd == 64 ? occupancy<64>() : occupancy<128>();
  if (occ < 1) return "the step kernel does not fit on a CU";
  return nullptr;
}

int decode_step_splits(int num_cus, int64_t hkv) {
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(kThreads, num_cus / hkv)));
}

void launch_decode_step(const StepParams& p, const StepShape& s, int num_cus, hipStream_t st) {
  const char* why = decode_step_unsupported(s, num_cus);
  PIA_REQUIRE(why == nullptr, why ? why : "");
  const size_t smem = decode_step_smem(s);
  if (s.hd == 32) go<32>(p, num_cus, smem, st);
  else if (s.hd == 64) go<64>(p, num_cus, smem, st);
  else go<128>(p, num_cus, smem, st);
  PIA_HIP(hipGetLastError());
}

}  // namespace pia
