// Temperature / top-k / nucleus sampling on the device (Sampler::sample, src/sampling.rs:74-138)
// with the reference's xorshift64* generator (src/sampling.rs:15-41), one workgroup per entry.
//
// The reference ranks the whole vocabulary with a sort and walks prefix sums in that order.
// Here every prefix condition (the k-th token, the first token whose cumulative mass reaches
// top_p, the first token whose cumulative mass exceeds the uniform draw) is found by a radix
// search over 32-bit total-order keys: four 8-bit passes, each a histogram of the candidates
// sharing the key prefix found so far, then one pass over the tokens tied on the final key
// (ranked by ascending index, the order a stable sort would give equal logits). No sort, no
// scratch memory beyond LDS.
//
// Probabilities are handled as unnormalized weights exp((l - max) / T) in 2^-40 fixed point,
// so every histogram and cumulative sum is exact integer arithmetic: the result does not
// depend on thread timing, and dividing by the total and the nucleus renormalization reduce
// to comparisons against scaled thresholds. The reference accumulates the same weights in f32
// in sorted order; the two choose the same token unless the draw falls within that f32
// rounding (~1e-6 relative) of a cumulative boundary.
//
// That fast path is opt-in. The default path reproduces the reference's arithmetic order so
// that the token is the reference's: a stable device radix sort ranks every row (f32::total_cmp
// descending, equal logits by ascending index), the exponentials and divisions run in
// parallel, and the three running sums the reference accumulates in f32 (the total, the
// nucleus cumulative and its renormalization, the cumulative walked against the draw) are
// accumulated in order by one lane, reading the probabilities in 4096-float chunks staged
// through LDS by the whole workgroup.
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <cstdint>

#include "common.h"
#include "kernels.h"

namespace pia {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr double kFix = 1099511627776.0;  // 2^40

// f32::total_cmp order as an unsigned key: larger key = later in the order.
__device__ inline uint32_t order_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ inline float key_value(uint32_t k) { return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k); }

// A position in the ranking: larger key first, equal keys by ascending index.
struct Rank {
  uint32_t key;
  int32_t idx;  // -1: no bound (every token qualifies)
};
__device__ inline bool at_or_before(uint32_t k, int i, const Rank& r) {
  return r.idx < 0 || k > r.key || (k == r.key && i <= r.idx);
}

struct Shared {
  unsigned long long hist[256];
  unsigned long long wsum[kWaves];
  unsigned long long scan[kThreads];
  uint32_t umax[kWaves];
  int32_t found_digit;
  unsigned long long found_above;
  int32_t found_idx;
  unsigned long long found_cum;
};

__device__ inline unsigned long long wave_sum_u64(unsigned long long v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ unsigned long long block_sum_u64(unsigned long long v, Shared& sh) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  v = wave_sum_u64(v);
  if (lane == 0) sh.wsum[wave] = v;
  __syncthreads();
  unsigned long long t = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) t += sh.wsum[w];
  __syncthreads();
  return t;
}

// Parameters of one entry's weights: the kept set so far and the fixed-point weight.
struct Ctx {
  const float* row;
  int vocab;
  float max_logit, inv_temp;
  Rank keep_k;  // top-k bound
  Rank keep_p;  // nucleus bound
};

// f(i, logit) for every token of the row in thread-strided order, eight loads in flight per
// thread (a runtime-bounded loop would otherwise wait for one load per iteration).
template <typename F>
__device__ inline void for_each_strided(const float* __restrict__ row, int vocab, F&& f) {
  for (int i0 = threadIdx.x; i0 < vocab; i0 += 8 * kThreads) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * kThreads;
      v[u] = i < vocab ? row[i] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * kThreads;
      if (i < vocab) f(i, v[u]);
    }
  }
}

// f(i, logit) for tokens i0..i1-1 in order, eight loads in flight.
template <typename F>
__device__ inline void for_each_range(const float* __restrict__ row, int i0, int i1, F&& f) {
  for (int b = i0; b < i1; b += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = b + u < i1 ? row[b + u] : 0.0f;
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (b + u < i1) f(b + u, v[u]);
  }
}

// Weight of token i (key k) for a search: 1 per token (count) or its fixed-point probability
// weight, 0 outside the kept set.
template <bool MASS>
__device__ inline unsigned long long weight(const Ctx& c, int i, uint32_t k, float logit) {
  if (!at_or_before(k, i, c.keep_k) || !at_or_before(k, i, c.keep_p)) return 0;
  if (!MASS) return 1;
  const float e = expf((logit - c.max_logit) * c.inv_temp);
  return static_cast<unsigned long long>(static_cast<double>(e) * kFix);
}

// First token in ranking order at which the cumulative weight reaches `thr` (>= 1). Returns
// {key, idx} with the cumulative weight through it in *cum; idx = -1 when the total weight
// stays below thr.
template <bool MASS>
__device__ Rank find_crossing(const Ctx& c, unsigned long long thr, Shared& sh, unsigned long long* cum) {
  const int tid = threadIdx.x;
  uint32_t prefix = 0, mask = 0;
  unsigned long long above = 0;  // weight of candidates ranked before the current key range
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int d = tid; d < 256; d += kThreads) sh.hist[d] = 0;
    __syncthreads();
    // Consecutive tokens of one thread often share a digit (the early passes put nearly all
    // tokens in a few bins): merge runs in registers before touching LDS.
    int run_d = -1;
    unsigned long long run_w = 0;
    for_each_strided(c.row, c.vocab, [&](int i, float logit) {
      const uint32_t k = order_key(logit);
      if ((k & mask) != prefix) return;
      const unsigned long long w = weight<MASS>(c, i, k, logit);
      if (!w) return;
      const int d = (k >> shift) & 255;
      if (d != run_d) {
        if (run_w) atomicAdd(&sh.hist[run_d], run_w);
        run_d = d, run_w = 0;
      }
      run_w += w;
    });
    if (run_w) atomicAdd(&sh.hist[run_d], run_w);
    __syncthreads();
    // Wave 0: lane l owns digits 255-4l .. 252-4l (descending); an inclusive scan over lanes
    // gives each lane the weight ranked before its digits.
    if (tid < 64) {
      unsigned long long loc[4], s = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) loc[j] = sh.hist[255 - 4 * tid - j], s += loc[j];
      unsigned long long incl = s;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const unsigned long long o = __shfl_up(incl, off, 64);
        if (tid >= off) incl += o;
      }
      const unsigned long long before = above + incl - s;
      const bool hit = before + s >= thr && before < thr;
      const unsigned long long ballot = __ballot(hit);
      if (tid == 0) sh.found_digit = -1;
      if (hit && (ballot & ((1ull << tid) - 1)) == 0) {
        unsigned long long b = before;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (b + loc[j] >= thr) {
            sh.found_digit = 255 - 4 * tid - j;
            sh.found_above = b;
            break;
          }
          b += loc[j];
        }
      }
    }
    __syncthreads();
    const int d = sh.found_digit;
    if (d < 0) {
      __syncthreads();
      *cum = 0;
      return Rank{0, -1};
    }
    above = sh.found_above;
    prefix |= static_cast<uint32_t>(d) << shift;
    mask |= 255u << shift;
    __syncthreads();
  }
  // Tokens tied on the final key, in ascending index: contiguous chunks per thread, an
  // exclusive scan of the chunk weights, then the chunk holding the crossing walks its tokens.
  const int chunk = (c.vocab + kThreads - 1) / kThreads;
  const int i0 = tid * chunk, i1 = min(c.vocab, i0 + chunk);
  unsigned long long local = 0;
  for_each_range(c.row, i0, i1, [&](int i, float logit) {
    const uint32_t k = order_key(logit);
    if (k == prefix) local += weight<MASS>(c, i, k, logit);
  });
  if (tid == 0) sh.found_idx = -1, sh.found_cum = 0;
  sh.scan[tid] = local;
  __syncthreads();
  // Hillis-Steele inclusive scan over the kThreads chunk weights.
  for (int off = 1; off < kThreads; off <<= 1) {
    const unsigned long long o = tid >= off ? sh.scan[tid - off] : 0;
    __syncthreads();
    sh.scan[tid] += o;
    __syncthreads();
  }
  const unsigned long long excl = above + sh.scan[tid] - local;
  if (local && excl < thr && excl + local >= thr) {
    unsigned long long b = excl;
    for (int i = i0; i < i1; ++i) {
      const float logit = c.row[i];
      const uint32_t k = order_key(logit);
      if (k != prefix) continue;
      b += weight<MASS>(c, i, k, logit);
      if (b >= thr) {
        sh.found_idx = i;
        sh.found_cum = b;
        break;
      }
    }
  }
  __syncthreads();
  const Rank r{prefix, sh.found_idx};
  *cum = sh.found_cum;
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kThreads) void k_sample(const float* __restrict__ logits, int64_t ld, int vocab,
                                                     const pia_sampling* __restrict__ params,
                                                     uint64_t* __restrict__ rng, int32_t* __restrict__ out) {
  __shared__ Shared sh;
  const int e = blockIdx.x, tid = threadIdx.x;
  const pia_sampling sp = params[e];
  Ctx c;
  c.row = logits + static_cast<int64_t>(e) * ld;
  c.vocab = vocab;
  c.keep_k = Rank{0, -1};
  c.keep_p = Rank{0, -1};

  // Top token: the largest key (its value is max_logit; ties share the value). With
  // temperature <= 0 the answer is argmax, the last of equal maxima (src/sampling.rs:140-147).
  uint32_t kmax = 0;
  int imax = -1;
  for_each_strided(c.row, vocab, [&](int i, float logit) {
    const uint32_t k = order_key(logit);
    if (imax < 0 || k > kmax || (k == kmax && i > imax)) kmax = k, imax = i;
  });
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t ok = __shfl_xor(kmax, off, 64);
    const int oi = __shfl_xor(imax, off, 64);
    if (oi >= 0 && (imax < 0 || ok > kmax || (ok == kmax && oi > imax))) kmax = ok, imax = oi;
  }
  __shared__ int32_t wimax[kWaves];
  if ((tid & 63) == 0) sh.umax[tid >> 6] = kmax, wimax[tid >> 6] = imax;
  __syncthreads();
  kmax = 0, imax = -1;
  for (int w = 0; w < kWaves; ++w)
    if (wimax[w] >= 0 && (imax < 0 || sh.umax[w] > kmax || (sh.umax[w] == kmax && wimax[w] > imax)))
      kmax = sh.umax[w], imax = wimax[w];
  if (!(sp.temperature > 0.0f)) {
    if (tid == 0) out[e] = imax;
    return;
  }
  c.max_logit = key_value(kmax);
  c.inv_temp = 1.0f / sp.temperature;

  unsigned long long cum = 0;
  if (sp.top_k > 0 && sp.top_k < vocab) c.keep_k = find_crossing<false>(c, static_cast<unsigned long long>(sp.top_k), sh, &cum);

  // Total weight of the kept tokens.
  unsigned long long local = 0;
  for_each_strided(c.row, vocab, [&](int i, float logit) { local += weight<true>(c, i, order_key(logit), logit); });
  unsigned long long total = block_sum_u64(local, sh);

  // Nucleus: the first token whose cumulative share reaches top_p is the last one kept.
  if (sp.top_p < 1.0f) {
    double t = ceil(static_cast<double>(sp.top_p) * static_cast<double>(total));
    unsigned long long thr = t < 1.0 ? 1ull : static_cast<unsigned long long>(t);
    if (thr <= total) {
      c.keep_p = find_crossing<true>(c, thr, sh, &cum);
      total = cum;
    }
  }

  // One uniform draw (Rng::next_f32), then the first token whose cumulative weight exceeds
  // draw * total.
  __shared__ float draw;
  if (tid == 0) {
    uint64_t x = rng[e];
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    rng[e] = x;
    draw = static_cast<float>((x * 0x2545F4914F6CDD1Dull) >> 40) / 16777216.0f;
  }
  __syncthreads();
  const unsigned long long thr =
      static_cast<unsigned long long>(floor(static_cast<double>(draw) * static_cast<double>(total))) + 1;
  const Rank pick = find_crossing<true>(c, thr, sh, &cum);
  if (tid == 0) out[e] = pick.idx >= 0 ? pick.idx : imax;
}

// ---------------------------------------------------------------------------------------
// Reference-order path.
// ---------------------------------------------------------------------------------------
constexpr int kSerialChunk = 4096;

// Sort key of token i of row r: rows in order, then f32::total_cmp descending.
__global__ __launch_bounds__(256) void k_sort_keys(const float* __restrict__ logits, int64_t ld, int vocab,
                                                   unsigned long long* __restrict__ keys, uint32_t* __restrict__ vals) {
  const int r = blockIdx.y;
  const float* row = logits + static_cast<int64_t>(r) * ld;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < vocab; i += gridDim.x * 256) {
    const int64_t o = static_cast<int64_t>(r) * vocab + i;
    keys[o] = (static_cast<unsigned long long>(r) << 32) | static_cast<unsigned long long>(~order_key(row[i]));
    vals[o] = static_cast<uint32_t>(i);
  }
}

struct SerialShared {
  float buf[kSerialChunk + 64];  // + zero padding to whole groups + one group of over-read
  float value;
  int pos;
  int stop;
};

// One lane walks v[0..n) in order, 32 values per group, the next group's LDS reads issued
// before this group's additions; the whole workgroup stages each chunk through LDS (zero
// padded to a whole group: adding +0.0 leaves a non-negative running sum unchanged).
// MODE 0: the running sum of all n values (returned in sh.value).
// MODE 1: the first j with sum(v[0..j]) >= thr; MODE 2: the first j with thr < sum(v[0..j]).
// The running sum never decreases (the values are >= 0), so the additions run branch-free and
// only the group in which the sum first crosses is walked again, from the same starting value
// (the same sequence of f32 additions). Returns that j, or n.
template <int MODE>
__device__ int serial_walk(const float* __restrict__ v, int n, float thr, SerialShared& sh) {
  const int tid = threadIdx.x;
  float acc = 0.0f;  // thread 0's running sum
  int found = n;
  for (int c0 = 0; c0 < n; c0 += kSerialChunk) {
    const int len = min(kSerialChunk, n - c0);
    const int padded = (len + 31) / 32 * 32;
    for (int j = tid; j < padded; j += blockDim.x) sh.buf[j] = j < len ? v[c0 + j] : 0.0f;
    __syncthreads();
    if (tid == 0) {
      int stop = -1;
      const float4* b4 = reinterpret_cast<const float4*>(sh.buf);
      float4 cur[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) cur[q] = b4[q];
      for (int g = 0; g * 32 < padded; ++g) {
        float4 nxt[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) nxt[q] = b4[(g + 1) * 8 + q];
        const float start = acc;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          acc += cur[q].x;
          acc += cur[q].y;
          acc += cur[q].z;
          acc += cur[q].w;
        }
        if (MODE != 0 && (MODE == 1 ? acc >= thr : thr < acc)) {
          float c = start;
          for (int j = 0; j < 32; ++j) {
            c += sh.buf[g * 32 + j];
            if (MODE == 1 ? c >= thr : thr < c) {
              stop = c0 + g * 32 + j;
              break;
            }
          }
          break;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) cur[q] = nxt[q];
      }
      sh.stop = stop;
      sh.value = acc;
    }
    __syncthreads();
    const int stop = sh.stop;
    if (tid == 0) acc = sh.value;
    __syncthreads();
    if (stop >= 0) {
      found = stop;
      break;
    }
  }
  return found;
}

__global__ __launch_bounds__(256) void k_sample_ordered(const float* __restrict__ logits, int64_t ld, int vocab,
                                                        const pia_sampling* __restrict__ params,
                                                        uint64_t* __restrict__ rng, const uint32_t* __restrict__ sorted,
                                                        float* __restrict__ probs, int32_t* __restrict__ out) {
  __shared__ SerialShared sh;
  __shared__ uint32_t wk[4];
  __shared__ int32_t wi[4];
  const int r = blockIdx.x, tid = threadIdx.x;
  const pia_sampling sp = params[r];
  const float* row = logits + static_cast<int64_t>(r) * ld;
  if (!(sp.temperature > 0.0f)) {
    // argmax: the last of equal maxima (src/sampling.rs:140-147).
    uint32_t bk = 0;
    int bi = -1;
    for (int i = tid; i < vocab; i += 256) {
      const uint32_t k = order_key(row[i]);
      if (bi < 0 || k > bk || (k == bk && i > bi)) bk = k, bi = i;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const uint32_t ok = __shfl_xor(bk, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      if (oi >= 0 && (bi < 0 || ok > bk || (ok == bk && oi > bi))) bk = ok, bi = oi;
    }
    if ((tid & 63) == 0) wk[tid >> 6] = bk, wi[tid >> 6] = bi;
    __syncthreads();
    if (tid == 0) {
      for (int w = 0; w < 4; ++w)
        if (wi[w] >= 0 && (bi < 0 || wk[w] > bk || (wk[w] == bk && wi[w] > bi))) bk = wk[w], bi = wi[w];
      out[r] = bi;
    }
    return;
  }
  const uint32_t* order = sorted + static_cast<int64_t>(r) * vocab;
  float* p = probs + static_cast<int64_t>(r) * vocab;
  const int keep = sp.top_k > 0 ? min(sp.top_k, vocab) : vocab;
  const float inv_temp = 1.0f / sp.temperature;
  const float max_logit = row[order[0]];
  // exp of the f32 argument, correctly rounded to f32 (through f64), as libm's expf is.
  for (int j = tid; j < keep; j += 256)
    p[j] = static_cast<float>(exp(static_cast<double>((row[order[j]] - max_logit) * inv_temp)));
  __syncthreads();
  serial_walk<0>(p, keep, 0.0f, sh);  // total: the in-order f32 sum
  const float total = sh.value;
  __syncthreads();
  for (int j = tid; j < keep; j += 256) p[j] = p[j] / total;
  __syncthreads();
  int cut = keep;
  if (sp.top_p < 1.0f) {
    // Nucleus: the first cumulative >= top_p is the last token kept; then the renormalization.
    const int hit = serial_walk<1>(p, keep, sp.top_p, sh);
    cut = hit < keep ? hit + 1 : keep;
    __syncthreads();
    serial_walk<0>(p, cut, 0.0f, sh);
    const float rn = sh.value;
    __syncthreads();
    for (int j = tid; j < cut; j += 256) p[j] = p[j] / rn;
    __syncthreads();
  }
  __shared__ float draw;
  if (tid == 0) {
    uint64_t x = rng[r];
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    rng[r] = x;
    draw = static_cast<float>((x * 0x2545F4914F6CDD1Dull) >> 40) / 16777216.0f;
  }
  __syncthreads();
  const int pick = serial_walk<2>(p, cut, draw, sh);
  if (tid == 0) out[r] = static_cast<int32_t>(order[pick < cut ? pick : cut - 1]);
}

// ---------------------------------------------------------------------------------------
// Small top-k, reference order, no sort of the vocabulary.
// ---------------------------------------------------------------------------------------
constexpr int kTopkMax = 1024;
constexpr int kTopkLdsVocab = 32768;  // rows up to this many logits are staged in LDS

// Rows with temperature <= 0 (argmax) or 0 < top_k <= kTopkMax: the radix search finds the
// k-th token of the ranking, the kept tokens are gathered into LDS and bitonic-sorted there by
// (logit total order descending, index ascending), and one lane runs the reference's in-order
// arithmetic over at most kTopkMax values (the same operations as k_sample_ordered).
__global__ __launch_bounds__(kThreads) void k_sample_topk(const float* __restrict__ logits, int64_t ld, int vocab,
                                                          const pia_sampling* __restrict__ params,
                                                          uint64_t* __restrict__ rng, int32_t* __restrict__ out) {
  extern __shared__ __align__(16) float lrow[];  // the row's logits, when they fit (vocab <= kTopkLdsVocab)
  __shared__ Shared sh;
  __shared__ unsigned long long sk[kTopkMax];  // (~key << 32 | index): ascending = ranking order
  __shared__ float pr[kTopkMax];
  __shared__ int count;
  __shared__ float bval;
  __shared__ int bpos;
  const int e = blockIdx.x, tid = threadIdx.x;
  const pia_sampling sp = params[e];
  Ctx c;
  c.row = logits + static_cast<int64_t>(e) * ld;
  c.vocab = vocab;
  c.keep_k = Rank{0, -1};
  c.keep_p = Rank{0, -1};
  if (!(sp.temperature > 0.0f)) {
    uint32_t kmax = 0;
    int imax = -1;
    for_each_strided(c.row, vocab, [&](int i, float logit) {
      const uint32_t k = order_key(logit);
      if (imax < 0 || k > kmax || (k == kmax && i > imax)) kmax = k, imax = i;
    });
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const uint32_t ok = __shfl_xor(kmax, off, 64);
      const int oi = __shfl_xor(imax, off, 64);
      if (oi >= 0 && (imax < 0 || ok > kmax || (ok == kmax && oi > imax))) kmax = ok, imax = oi;
    }
    __shared__ uint32_t wk[kWaves];
    __shared__ int32_t wi[kWaves];
    if ((tid & 63) == 0) wk[tid >> 6] = kmax, wi[tid >> 6] = imax;
    __syncthreads();
    if (tid == 0) {
      for (int w = 0; w < kWaves; ++w)
        if (wi[w] >= 0 && (imax < 0 || wk[w] > kmax || (wk[w] == kmax && wi[w] > imax))) kmax = wk[w], imax = wi[w];
      out[e] = imax;
    }
    return;
  }
  const int keep = min(sp.top_k, vocab);
  // Every later pass reads the row from LDS when it fits.
  if (vocab <= kTopkLdsVocab) {
    for_each_strided(c.row, vocab, [&](int i, float logit) { lrow[i] = logit; });
    __syncthreads();
    c.row = lrow;
  }
  // The keep-th token of the ranking, then every token at or before it.
  unsigned long long cum = 0;
  const Rank bound = keep < vocab ? find_crossing<false>(c, static_cast<unsigned long long>(keep), sh, &cum) : Rank{0, -1};
  if (tid == 0) count = 0;
  int n2 = 1;
  while (n2 < keep) n2 <<= 1;
  for (int j = tid; j < n2; j += kThreads) sk[j] = ~0ull;
  __syncthreads();
  for_each_strided(c.row, vocab, [&](int i, float logit) {
    const uint32_t k = order_key(logit);
    if (at_or_before(k, i, bound)) {
      const int slot = atomicAdd(&count, 1);
      if (slot < kTopkMax) sk[slot] = (static_cast<unsigned long long>(~k) << 32) | static_cast<uint32_t>(i);
    }
  });
  __syncthreads();
  // Bitonic sort of n2 entries, ascending.
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int j = tid; j < n2; j += kThreads) {
        const int o = j ^ stride;
        if (o > j) {
          const bool up = (j & size) == 0;
          const unsigned long long a = sk[j], b = sk[o];
          if ((a > b) == up) sk[j] = b, sk[o] = a;
        }
      }
      __syncthreads();
    }
  }
  // The reference's arithmetic over the kept tokens in ranking order (src/sampling.rs:95-136).
  const float inv_temp = 1.0f / sp.temperature;
  const float max_logit = c.row[static_cast<uint32_t>(sk[0])];
  for (int j = tid; j < keep; j += kThreads)
    pr[j] = static_cast<float>(exp(static_cast<double>((c.row[static_cast<uint32_t>(sk[j])] - max_logit) * inv_temp)));
  __syncthreads();
  if (tid == 0) {
    float total = 0.0f;
    for (int j = 0; j < keep; ++j) total += pr[j];
    bval = total;
  }
  __syncthreads();
  const float total = bval;
  for (int j = tid; j < keep; j += kThreads) pr[j] = pr[j] / total;
  __syncthreads();
  int cut = keep;
  if (sp.top_p < 1.0f) {
    if (tid == 0) {
      float cumulative = 0.0f;
      int cc = keep;
      for (int j = 0; j < keep; ++j) {
        cumulative += pr[j];
        if (cumulative >= sp.top_p) {
          cc = j + 1;
          break;
        }
      }
      float renorm = 0.0f;
      for (int j = 0; j < cc; ++j) renorm += pr[j];
      bpos = cc;
      bval = renorm;
    }
    __syncthreads();
    cut = bpos;
    const float rn = bval;
    for (int j = tid; j < cut; j += kThreads) pr[j] = pr[j] / rn;
    __syncthreads();
  }
  if (tid == 0) {
    uint64_t x = rng[e];
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    rng[e] = x;
    const float target = static_cast<float>((x * 0x2545F4914F6CDD1Dull) >> 40) / 16777216.0f;
    float cumulative = 0.0f;
    int pick = cut - 1;
    for (int j = 0; j < cut; ++j) {
      cumulative += pr[j];
      if (target < cumulative) {
        pick = j;
        break;
      }
    }
    out[e] = static_cast<int32_t>(static_cast<uint32_t>(sk[pick]));
  }
}

}  // namespace

size_t sample_workspace_bytes(int64_t n, int64_t vocab) {
  const size_t N = static_cast<size_t>(n) * static_cast<size_t>(vocab);
  size_t temp = 0;
  PIA_HIP(hipcub::DeviceRadixSort::SortPairs(nullptr, temp, static_cast<const unsigned long long*>(nullptr),
                                             static_cast<unsigned long long*>(nullptr),
                                             static_cast<const uint32_t*>(nullptr), static_cast<uint32_t*>(nullptr),
                                             static_cast<int>(N), 0, 64));
  auto up = [](size_t b) { return (b + 255) / 256 * 256; };
  return 2 * up(N * 8) + 2 * up(N * 4) + up(N * 4) + up(temp);
}

void launch_sample_topk(const float* logits, int64_t ld, int64_t n, int64_t vocab, const pia_sampling* params,
                        uint64_t* rng, int32_t* out, hipStream_t st) {
  if (n == 0) return;
  PIA_REQUIRE(vocab > 0 && vocab < (int64_t(1) << 31) && ld >= vocab, "sample: bad vocabulary / pitch");
  const size_t smem = vocab <= kTopkLdsVocab ? static_cast<size_t>(vocab) * 4 : 0;
  static bool raised = false;
  if (!raised) {
    PIA_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(k_sample_topk), hipFuncAttributeMaxDynamicSharedMemorySize,
                                kTopkLdsVocab * 4));
    raised = true;
  }
  hipLaunchKernelGGL(k_sample_topk, dim3(static_cast<unsigned>(n)), dim3(kThreads), smem, st, logits, ld,
                     static_cast<int>(vocab), params, rng, out);
  PIA_HIP(hipGetLastError());
}

int64_t sample_topk_max() { return kTopkMax; }

void launch_sample(const float* logits, int64_t ld, int64_t n, int64_t vocab, const pia_sampling* params,
                   uint64_t* rng, int32_t* out, int mode, void* workspace, size_t workspace_bytes, hipStream_t st) {
  if (n == 0) return;
  PIA_REQUIRE(vocab > 0 && vocab < (int64_t(1) << 31), "sample: vocabulary size out of range");
  PIA_REQUIRE(ld >= vocab, "sample: row pitch below the vocabulary size");
  PIA_REQUIRE(n < (int64_t(1) << 31), "sample: too many rows");
  PIA_REQUIRE(mode == 0 || mode == 1, "sample: mode must be 0 (reference order) or 1 (exact sums)");
  if (mode == 1) {
    hipLaunchKernelGGL(k_sample, dim3(static_cast<unsigned>(n)), dim3(kThreads), 0, st, logits, ld,
                       static_cast<int>(vocab), params, rng, out);
    PIA_HIP(hipGetLastError());
    return;
  }
  const size_t N = static_cast<size_t>(n) * static_cast<size_t>(vocab);
  PIA_REQUIRE(N < (size_t(1) << 31), "sample: rows x vocabulary too large for one sort");
  PIA_REQUIRE(workspace && workspace_bytes >= sample_workspace_bytes(n, vocab), "sample: workspace too small");
  auto up = [](size_t b) { return (b + 255) / 256 * 256; };
  char* w = static_cast<char*>(workspace);
  auto* kin = reinterpret_cast<unsigned long long*>(w);
  auto* kout = reinterpret_cast<unsigned long long*>(w + up(N * 8));
  auto* vin = reinterpret_cast<uint32_t*>(w + 2 * up(N * 8));
  auto* vout = reinterpret_cast<uint32_t*>(w + 2 * up(N * 8) + up(N * 4));
  auto* probs = reinterpret_cast<float*>(w + 2 * up(N * 8) + 2 * up(N * 4));
  void* temp = w + 2 * up(N * 8) + 3 * up(N * 4);
  size_t temp_bytes = workspace_bytes - (2 * up(N * 8) + 3 * up(N * 4));
  const unsigned gx = static_cast<unsigned>(std::min<int64_t>((vocab + 255) / 256, 64));
  hipLaunchKernelGGL(k_sort_keys, dim3(gx, static_cast<unsigned>(n)), dim3(256), 0, st, logits, ld,
                     static_cast<int>(vocab), kin, vin);
  PIA_HIP(hipGetLastError());
  int row_bits = 0;
  while ((int64_t(1) << row_bits) < n) ++row_bits;
  PIA_HIP(hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, kin, kout, vin, vout, static_cast<int>(N), 0,
                                             32 + row_bits, st));
  hipLaunchKernelGGL(k_sample_ordered, dim3(static_cast<unsigned>(n)), dim3(256), 0, st, logits, ld,
                     static_cast<int>(vocab), params, rng, vout, probs, out);
  PIA_HIP(hipGetLastError());
}

}  // namespace pia
