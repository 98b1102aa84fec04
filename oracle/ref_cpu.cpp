// CPU restatement of Paged-Infer's QUANT=int8 projection path and paged-attention decode.
//
// TEST INFRASTRUCTURE ONLY. This file is the parity oracle and the timed CPU baseline
// ("port"). Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
// load it, and only as the checker -- never as the product path.
//
// It restates, operation for operation, the reference's x86_64 AVX2+FMA CPU path so that
// its f32 results carry the same rounding as the reference on the same inputs:
//   quantize_rows_i8                 src/math.rs:456-469
//   dot / dot_i8 / dot_*_multi        src/simd.rs:114-153, 228-262, 279-329 (x86 module)
//   axpy                              src/simd.rs:331-349
//   matvec_i8 / matmat_i8 (+ f32)     src/math.rs:93-129, 164-275, 473-512
//   rms_norm, silu/swiglu             src/math.rs:4-22, 293-302
//   rope_table / rope_rotate (NeoX)   src/math.rs:331-367
//   softmax_in_place                  src/math.rs:405-426
//   PagedAttention::run               src/attention.rs:141-264 (+ for_each_block :279-295)
//   run_layers_batch                  src/model.rs:968-1177
//   decode_batch_into                 src/model.rs:1184-1207
//   prefill_batched                   src/model.rs:1222-1255
//   argmax                            src/sampling.rs:140-147
//   Rng (xorshift64*), Sampler::sample src/sampling.rs:15-138
// Rayon's row/lane parallelism is replaced by a fixed worker pool; it changes no arithmetic
// (every output element is produced by exactly one task, as in the reference).
//
// Build: oracle/Makefile (g++ -O2 -ffp-contract=off; the AVX2 kernels are enabled per
// function, and a portable lane-by-lane emulation with fmaf gives identical bits on hosts
// without AVX2).

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace {

// ---------------------------------------------------------------------------------------
// Worker pool: parallel_for(n, grain, fn(begin, end)).
// ---------------------------------------------------------------------------------------
class Pool {
 public:
  explicit Pool(int n) { resize(n); }
  ~Pool() { stop(); }

  int size() const { return nthreads_; }

  void resize(int n) {
    stop();
    nthreads_ = std::max(1, n);
    quit_ = false;
    for (int i = 1; i < nthreads_; ++i) workers_.emplace_back([this] { worker(); });
  }

  void parallel_for(int64_t n, int64_t grain, const std::function<void(int64_t, int64_t)>& fn) {
    if (n <= 0) return;
    if (nthreads_ == 1 || n <= grain) {
      fn(0, n);
      return;
    }
    {
      std::lock_guard<std::mutex> lk(mu_);
      job_ = &fn;
      n_ = n;
      grain_ = grain;
      next_.store(0);
      active_ = nthreads_ - 1;
      ++gen_;
    }
    cv_.notify_all();
    run_chunks();
    std::unique_lock<std::mutex> lk(mu_);
    done_cv_.wait(lk, [this] { return active_ == 0; });
    job_ = nullptr;
  }

 private:
  void run_chunks() {
    for (;;) {
      int64_t b = next_.fetch_add(grain_);
      if (b >= n_) break;
      (*job_)(b, std::min(n_, b + grain_));
    }
  }
  void worker() {
    uint64_t seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return quit_ || gen_ != seen; });
        if (quit_) return;
        seen = gen_;
      }
      run_chunks();
      {
        std::lock_guard<std::mutex> lk(mu_);
        if (--active_ == 0) done_cv_.notify_one();
      }
    }
  }
  void stop() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      quit_ = true;
    }
    cv_.notify_all();
    for (auto& t : workers_) t.join();
    workers_.clear();
  }

  int nthreads_ = 1;
  std::vector<std::thread> workers_;
  std::mutex mu_;
  std::condition_variable cv_, done_cv_;
  const std::function<void(int64_t, int64_t)>* job_ = nullptr;
  int64_t n_ = 0, grain_ = 1;
  std::atomic<int64_t> next_{0};
  int active_ = 0;
  uint64_t gen_ = 0;
  bool quit_ = false;
};

Pool& pool() {
  static Pool p(std::max(1u, std::thread::hardware_concurrency()));
  return p;
}

bool g_force_portable = false;

bool have_avx2() {
  static const bool ok = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
  return ok && !g_force_portable;
}

// ---------------------------------------------------------------------------------------
// Inner products. Accumulator structure of src/simd.rs x86::dot / x86::dot_i8: four 8-lane
// accumulators over 32-element chunks, an 8-element tail into accumulator 0, the reduction
// (a0+a1)+(a2+a3), the hsum ((s0+s2)+(s1+s3)) with s_k = v_k + v_{k+4}, then a scalar tail
// with a separately rounded multiply and add.
// ---------------------------------------------------------------------------------------
__attribute__((target("avx2,fma"))) inline float hsum256(__m256 v) {
  __m128 lo = _mm256_castps256_ps128(v);
  __m128 hi = _mm256_extractf128_ps(v, 1);
  __m128 s = _mm_add_ps(lo, hi);
  s = _mm_add_ps(s, _mm_movehl_ps(s, s));
  s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 0x55));
  return _mm_cvtss_f32(s);
}

__attribute__((target("avx2,fma"))) inline __m256 widen_i8(const int8_t* p) {
  return _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64(reinterpret_cast<const __m128i*>(p))));
}

__attribute__((target("avx2,fma"))) inline __m256 load_w8(const int8_t* p) { return widen_i8(p); }
__attribute__((target("avx2,fma"))) inline __m256 load_w8(const float* p) { return _mm256_loadu_ps(p); }

// One weight row against BT activation vectors (stride apart). BT == 1 is dot / dot_i8.
template <int BT, typename W>
__attribute__((target("avx2,fma"))) void dot_multi_avx2(const W* w, const float* x, int64_t stride,
                                                       int64_t n, float* out) {
  __m256 acc[BT][4];
  for (int b = 0; b < BT; ++b)
    for (int j = 0; j < 4; ++j) acc[b][j] = _mm256_setzero_ps();
  int64_t i = 0;
  for (; i + 32 <= n; i += 32) {
    for (int j = 0; j < 4; ++j) {
      __m256 wv = load_w8(w + i + 8 * j);
      for (int b = 0; b < BT; ++b)
        acc[b][j] = _mm256_fmadd_ps(wv, _mm256_loadu_ps(x + b * stride + i + 8 * j), acc[b][j]);
    }
  }
  for (; i + 8 <= n; i += 8) {
    __m256 wv = load_w8(w + i);
    for (int b = 0; b < BT; ++b)
      acc[b][0] = _mm256_fmadd_ps(wv, _mm256_loadu_ps(x + b * stride + i), acc[b][0]);
  }
  for (int b = 0; b < BT; ++b) {
    __m256 s = _mm256_add_ps(_mm256_add_ps(acc[b][0], acc[b][1]), _mm256_add_ps(acc[b][2], acc[b][3]));
    float total = hsum256(s);
    for (int64_t k = i; k < n; ++k) {
      float prod = static_cast<float>(w[k]) * x[b * stride + k];
      total = total + prod;
    }
    out[b] = total;
  }
}

// Lane-by-lane emulation of dot_multi_avx2 with identical rounding (fmaf per lane).
template <typename W>
float dot_portable(const W* w, const float* x, int64_t n) {
  float acc[4][8] = {};
  int64_t i = 0;
  for (; i + 32 <= n; i += 32)
    for (int j = 0; j < 4; ++j)
      for (int l = 0; l < 8; ++l)
        acc[j][l] = std::fmaf(static_cast<float>(w[i + 8 * j + l]), x[i + 8 * j + l], acc[j][l]);
  for (; i + 8 <= n; i += 8)
    for (int l = 0; l < 8; ++l) acc[0][l] = std::fmaf(static_cast<float>(w[i + l]), x[i + l], acc[0][l]);
  float v[8];
  for (int l = 0; l < 8; ++l) v[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
  float s[4];
  for (int k = 0; k < 4; ++k) s[k] = v[k] + v[k + 4];
  float total = (s[0] + s[2]) + (s[1] + s[3]);
  for (; i < n; ++i) {
    float prod = static_cast<float>(w[i]) * x[i];
    total = total + prod;
  }
  return total;
}

template <typename W>
inline float dot_any(const W* w, const float* x, int64_t n) {
  if (have_avx2()) {
    float r;
    dot_multi_avx2<1, W>(w, x, n, n, &r);
    return r;
  }
  return dot_portable<W>(w, x, n);
}

// out += weight * v  (src/simd.rs:331-349): fused over 8-lane chunks, unfused scalar tail.
void axpy(float* out, float weight, const float* v, int64_t n) {
  int64_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int l = 0; l < 8; ++l) out[i + l] = std::fmaf(weight, v[i + l], out[i + l]);
  for (; i < n; ++i) {
    float prod = weight * v[i];
    out[i] = out[i] + prod;
  }
}

// ---------------------------------------------------------------------------------------
// Projections.
// ---------------------------------------------------------------------------------------
struct Proj {
  int32_t kind;  // 0 = f32 weights, 1 = int8 weights + per-row f32 scales
  int32_t pad;
  int64_t rows, cols;
  const int8_t* q;
  const float* scales;
  const float* f;
};

// out[r] = dot(W[r], x) (* scale[r])   -- matvec_*_weight_parallel
void matvec(const Proj& p, float* out, const float* x) {
  pool().parallel_for(p.rows, 16, [&](int64_t r0, int64_t r1) {
    for (int64_t r = r0; r < r1; ++r) {
      if (p.kind == 1) out[r] = dot_any<int8_t>(p.q + r * p.cols, x, p.cols) * p.scales[r];
      else out[r] = dot_any<float>(p.f + r * p.cols, x, p.cols);
    }
  });
}

// out_rb[r][b] -- matmat_*_weight_parallel with tiles of 4/2/1. dot_multi<BT> is bit-identical
// to BT separate dots, so the tile decomposition is a speed choice only.
template <typename W>
void matmat_row(const W* wr, const float* x_br, int64_t batch, int64_t cols, float* o) {
  if (!have_avx2()) {
    for (int64_t b = 0; b < batch; ++b) o[b] = dot_portable<W>(wr, x_br + b * cols, cols);
    return;
  }
  int64_t b = 0;
  for (; b + 4 <= batch; b += 4) dot_multi_avx2<4, W>(wr, x_br + b * cols, cols, cols, o + b);
  for (; b + 2 <= batch; b += 2) dot_multi_avx2<2, W>(wr, x_br + b * cols, cols, cols, o + b);
  for (; b < batch; ++b) dot_multi_avx2<1, W>(wr, x_br + b * cols, cols, cols, o + b);
}

void matmat(const Proj& p, float* out_rb, const float* x_br, int64_t batch) {
  pool().parallel_for(p.rows, 8, [&](int64_t r0, int64_t r1) {
    for (int64_t r = r0; r < r1; ++r) {
      float* o = out_rb + r * batch;
      if (p.kind == 1) {
        matmat_row<int8_t>(p.q + r * p.cols, x_br, batch, p.cols, o);
        for (int64_t b = 0; b < batch; ++b) o[b] = o[b] * p.scales[r];
      } else {
        matmat_row<float>(p.f + r * p.cols, x_br, batch, p.cols, o);
      }
    }
  });
}

// Projection::apply_batched: matmat into [row][batch], then transpose to [batch][row].
void apply_batched(const Proj& p, float* out_br, const float* x_br, int64_t batch, std::vector<float>& stage) {
  stage.resize(p.rows * batch);
  matmat(p, stage.data(), x_br, batch);
  for (int64_t r = 0; r < p.rows; ++r)
    for (int64_t b = 0; b < batch; ++b) out_br[b * p.rows + r] = stage[r * batch + b];
}

// ---------------------------------------------------------------------------------------
// Elementwise math.
// ---------------------------------------------------------------------------------------
void rms_norm(float* x, const float* w, int64_t n, float eps) {
  float ss = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    float sq = x[i] * x[i];
    ss = ss + sq;
  }
  ss = ss / static_cast<float>(n);
  float inv = 1.0f / std::sqrt(ss + eps);
  for (int64_t i = 0; i < n; ++i) {
    float t = x[i] * inv;
    x[i] = t * w[i];
  }
}

inline float silu(float x) { return x / (1.0f + std::exp(-x)); }

void rope_table(int64_t pos, int64_t hd, float theta, float* cos_out, float* sin_out) {
  int64_t half = hd / 2;
  for (int64_t j = 0; j < half; ++j) {
    float freq = 1.0f / std::pow(theta, static_cast<float>(2 * j) / static_cast<float>(hd));
    float a = static_cast<float>(pos) * freq;
    cos_out[j] = std::cos(a);
    sin_out[j] = std::sin(a);
  }
}

void rope_rotate_neox(float* x, const float* c, const float* s, int64_t hd) {
  int64_t half = hd / 2;
  for (int64_t j = 0; j < half; ++j) {
    float a = x[j], b = x[j + half];
    float ac = a * c[j], bs = b * s[j], bc = b * c[j], as = a * s[j];
    x[j] = ac - bs;
    x[j + half] = bc + as;
  }
}

void softmax_in_place(float* x, int64_t n) {
  if (n == 0) return;
  float mx = -INFINITY;
  for (int64_t i = 0; i < n; ++i) mx = std::fmax(mx, x[i]);
  if (!std::isfinite(mx)) {
    for (int64_t i = 0; i < n; ++i) x[i] = 0.0f;
    return;
  }
  float sum = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    x[i] = std::exp(x[i] - mx);
    sum = sum + x[i];
  }
  float inv = 1.0f / std::fmax(sum, 1e-12f);
  for (int64_t i = 0; i < n; ++i) x[i] = x[i] * inv;
}

inline float bf16_to_f32(uint16_t h) {
  uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

}  // namespace

// =========================================================================================
// C ABI of the oracle.
// =========================================================================================
extern "C" {

struct orc_config {
  int64_t hidden, layers, heads, kv_heads, inter, vocab;
  float eps, theta;
  int64_t window;  // < 0: full causal attention (attention_window = None)
};

struct orc_layer {
  const float* attn_norm;
  Proj wq, wk, wv, wo;
  const float* ffn_norm;
  Proj w1, w2, w3;  // gate, down, up (reference naming)
};

// One attention entry: attends to start..=pos; its logical->physical blocks are
// tables[table_off .. table_off+table_len]; logical blocks at or past table_len are unmapped.
struct orc_entry {
  int64_t pos, start, table_off, table_len;
};

struct orc_model {
  orc_config c;
  const uint16_t* embed;
  const float* final_norm;
  Proj lm_head;
  std::vector<orc_layer> layers;
};

void orc_set_threads(int n) { pool().resize(n); }
int orc_threads(void) { return pool().size(); }
void orc_force_portable(int on) { g_force_portable = on != 0; }
int orc_have_avx2(void) { return have_avx2() ? 1 : 0; }

// math.rs:456-469. Rust's f32::round is half-away-from-zero == C roundf; `as i8` saturates,
// and the clamp makes every value representable.
void orc_quantize_rows_i8(const float* w, int64_t rows, int64_t cols, int8_t* q, float* scales) {
  pool().parallel_for(rows, 4, [&](int64_t r0, int64_t r1) {
    for (int64_t r = r0; r < r1; ++r) {
      const float* row = w + r * cols;
      float max_abs = 0.0f;
      for (int64_t c = 0; c < cols; ++c) max_abs = std::fmax(max_abs, std::fabs(row[c]));
      float scale = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
      scales[r] = scale;
      for (int64_t c = 0; c < cols; ++c) {
        float v = std::roundf(row[c] / scale);
        v = std::fmin(std::fmax(v, -127.0f), 127.0f);
        q[r * cols + c] = static_cast<int8_t>(v);
      }
    }
  });
}

float orc_dot_i8(const int8_t* w, const float* x, int64_t n) { return dot_any<int8_t>(w, x, n); }
float orc_dot(const float* a, const float* b, int64_t n) { return dot_any<float>(a, b, n); }

void orc_matvec_i8(float* out, const float* x, const int8_t* w, const float* s, int64_t rows, int64_t cols) {
  Proj p{1, 0, rows, cols, w, s, nullptr};
  matvec(p, out, x);
}
void orc_matmat_i8(float* out_rb, const float* x_br, const int8_t* w, const float* s, int64_t batch,
                   int64_t rows, int64_t cols) {
  Proj p{1, 0, rows, cols, w, s, nullptr};
  matmat(p, out_rb, x_br, batch);
}
void orc_matvec_f32(float* out, const float* x, const float* w, int64_t rows, int64_t cols) {
  Proj p{0, 0, rows, cols, nullptr, nullptr, w};
  matvec(p, out, x);
}

void orc_rope_table(int64_t pos, int64_t hd, float theta, float* c, float* s) { rope_table(pos, hd, theta, c, s); }
void orc_softmax(float* x, int64_t n) { softmax_in_place(x, n); }
void orc_rms_norm(float* x, const float* w, int64_t n, float eps) { rms_norm(x, w, n, eps); }

int64_t orc_argmax(const float* logits, int64_t n) {
  // max_by(total_cmp): on equal keys the later element wins.
  auto key = [](float f) {
    int32_t b;
    std::memcpy(&b, &f, 4);
    return b ^ static_cast<int32_t>(static_cast<uint32_t>(b >> 31) >> 1);
  };
  if (n <= 0) return 0;
  int64_t best = 0;
  int32_t bk = key(logits[0]);
  for (int64_t i = 1; i < n; ++i) {
    int32_t k = key(logits[i]);
    if (k >= bk) {
      bk = k;
      best = i;
    }
  }
  return best;
}

// PagedAttention::run (attention.rs:141-264) for one layer. q/out: [n][heads][hd].
// kv: [layers][num_blocks][block_size][kv_heads][2][hd].
void orc_paged_attention(float* out, const float* q, const float* kv, int64_t num_layers, int64_t num_blocks,
                         int64_t block_size, int64_t kv_heads, int64_t hd, int64_t heads, const orc_entry* entries,
                         const int32_t* tables, int64_t n, int64_t layer) {
  (void)num_layers;
  const int64_t kv_group = heads / kv_heads;
  const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
  const int64_t token_stride = kv_heads * 2 * hd;
  auto index = [&](int64_t pb, int64_t off, int64_t h, int64_t isv) {
    return ((((layer * num_blocks + pb) * block_size + off) * kv_heads + h) * 2 + isv) * hd;
  };
  pool().parallel_for(n * heads, 1, [&](int64_t l0, int64_t l1) {
    std::vector<float> scores;
    for (int64_t lane = l0; lane < l1; ++lane) {
      const orc_entry& e = entries[lane / heads];
      const int64_t h = lane % heads, kvh = h / kv_group;
      const float* qh = q + lane * hd;
      float* oh = out + lane * hd;
      const int64_t used = e.pos + 1 > e.start ? e.pos + 1 - e.start : 0;
      for (int64_t d = 0; d < hd; ++d) oh[d] = 0.0f;
      if (used == 0) continue;
      scores.assign(used, 0.0f);
      // for_each_block (attention.rs:279-295): one table lookup per block run.
      for (int pass = 0; pass < 2; ++pass) {
        int64_t t = e.start;
        while (t <= e.pos) {
          int64_t off = t % block_size;
          int64_t take = std::min(block_size - off, e.pos + 1 - t);
          int64_t lb = t / block_size;
          bool mapped = lb < e.table_len;
          int64_t si0 = t - e.start;
          if (pass == 0) {
            if (mapped) {
              int64_t pb = tables[e.table_off + lb];
              int64_t base = index(pb, off, kvh, 0);
              for (int64_t i = 0; i < take; ++i)
                scores[si0 + i] = dot_any<float>(qh, kv + base + i * token_stride, hd) * scale;
            } else {
              for (int64_t i = 0; i < take; ++i) scores[si0 + i] = -INFINITY;
            }
          } else if (mapped) {
            int64_t pb = tables[e.table_off + lb];
            int64_t base = index(pb, off, kvh, 1);
            for (int64_t i = 0; i < take; ++i) {
              float wgt = scores[si0 + i];
              if (wgt == 0.0f) continue;
              axpy(oh, wgt, kv + base + i * token_stride, hd);
            }
          }
          t += take;
        }
        if (pass == 0) softmax_in_place(scores.data(), used);
      }
    }
  });
}

orc_model* orc_model_create(const orc_config* c, const uint16_t* embed, const float* final_norm, const Proj* lm_head) {
  auto* m = new orc_model;
  m->c = *c;
  m->embed = embed;
  m->final_norm = final_norm;
  m->lm_head = *lm_head;
  m->layers.resize(c->layers);
  return m;
}
void orc_model_set_layer(orc_model* m, int64_t i, const orc_layer* l) { m->layers[i] = *l; }
void orc_model_destroy(orc_model* m) { delete m; }

}  // extern "C"

namespace {

// run_layers_batch (model.rs:968-1177): leaves each entry's final normalized hidden in x.
void run_layers_batch(const orc_model* m, const uint32_t* tokens, const int64_t* positions, const orc_entry* entries,
                      const int32_t* tables, int64_t batch, float* kv, int64_t num_blocks, int64_t block_size,
                      std::vector<float>& x) {
  const orc_config& c = m->c;
  const int64_t hidden = c.hidden, hd = c.hidden / c.heads, kv_dim = c.kv_heads * hd, inter = c.inter;
  const int64_t half = hd / 2;
  std::vector<float> xb(batch * hidden), q(batch * hidden), k(batch * kv_dim), v(batch * kv_dim),
      attn(batch * hidden), proj(batch * hidden), gate(batch * inter), up(batch * inter), down(batch * hidden),
      stage, rc(batch * half), rs(batch * half);
  x.assign(batch * hidden, 0.0f);
  for (int64_t b = 0; b < batch; ++b) rope_table(positions[b], hd, c.theta, &rc[b * half], &rs[b * half]);
  for (int64_t b = 0; b < batch; ++b) {
    int64_t tok = static_cast<int64_t>(tokens[b]) % c.vocab;
    for (int64_t i = 0; i < hidden; ++i) x[b * hidden + i] = bf16_to_f32(m->embed[tok * hidden + i]);
  }
  auto kv_index = [&](int64_t layer, int64_t pb, int64_t off, int64_t h, int64_t isv) {
    return ((((layer * num_blocks + pb) * block_size + off) * c.kv_heads + h) * 2 + isv) * hd;
  };
  for (int64_t li = 0; li < c.layers; ++li) {
    const orc_layer& L = m->layers[li];
    for (int64_t b = 0; b < batch; ++b) {
      std::memcpy(&xb[b * hidden], &x[b * hidden], hidden * 4);
      rms_norm(&xb[b * hidden], L.attn_norm, hidden, c.eps);
    }
    apply_batched(L.wq, q.data(), xb.data(), batch, stage);
    apply_batched(L.wk, k.data(), xb.data(), batch, stage);
    apply_batched(L.wv, v.data(), xb.data(), batch, stage);
    for (int64_t b = 0; b < batch; ++b) {
      for (int64_t h = 0; h < c.heads; ++h) rope_rotate_neox(&q[b * hidden + h * hd], &rc[b * half], &rs[b * half], hd);
      for (int64_t h = 0; h < c.kv_heads; ++h) rope_rotate_neox(&k[b * kv_dim + h * hd], &rc[b * half], &rs[b * half], hd);
    }
    for (int64_t b = 0; b < batch; ++b) {
      const orc_entry& e = entries[b];
      int64_t lb = positions[b] / block_size, off = positions[b] % block_size;
      if (lb >= e.table_len) continue;  // unmapped position: the write is skipped
      int64_t pb = tables[e.table_off + lb];
      for (int64_t h = 0; h < c.kv_heads; ++h) {
        std::memcpy(kv + kv_index(li, pb, off, h, 0), &k[b * kv_dim + h * hd], hd * 4);
        std::memcpy(kv + kv_index(li, pb, off, h, 1), &v[b * kv_dim + h * hd], hd * 4);
      }
    }
    orc_paged_attention(attn.data(), q.data(), kv, c.layers, num_blocks, block_size, c.kv_heads, hd, c.heads, entries,
                        tables, batch, li);
    apply_batched(L.wo, proj.data(), attn.data(), batch, stage);
    for (int64_t i = 0; i < batch * hidden; ++i) x[i] = x[i] + proj[i];
    for (int64_t b = 0; b < batch; ++b) {
      std::memcpy(&xb[b * hidden], &x[b * hidden], hidden * 4);
      rms_norm(&xb[b * hidden], L.ffn_norm, hidden, c.eps);
    }
    apply_batched(L.w1, gate.data(), xb.data(), batch, stage);
    apply_batched(L.w3, up.data(), xb.data(), batch, stage);
    for (int64_t i = 0; i < batch * inter; ++i) gate[i] = silu(gate[i]) * up[i];
    apply_batched(L.w2, down.data(), gate.data(), batch, stage);
    for (int64_t i = 0; i < batch * hidden; ++i) x[i] = x[i] + down[i];
  }
  for (int64_t b = 0; b < batch; ++b) rms_norm(&x[b * hidden], m->final_norm, hidden, c.eps);
}

// AttnEntry::new (attention.rs:71-78): start = (pos+1).saturating_sub(window).
int64_t window_start(int64_t pos, int64_t window) {
  if (window < 0) return 0;
  return pos + 1 > window ? pos + 1 - window : 0;
}

}  // namespace

extern "C" {

// decode_batch_into (model.rs:1184-1207). entries[b].pos must equal positions[b]; start is
// recomputed from the model's window. logits: [batch][vocab].
void orc_decode_batch(const orc_model* m, const uint32_t* tokens, const int64_t* positions, const int64_t* table_off,
                      const int64_t* table_len, const int32_t* tables, int64_t batch, float* kv, int64_t num_blocks,
                      int64_t block_size, float* logits) {
  std::vector<orc_entry> entries(batch);
  for (int64_t b = 0; b < batch; ++b)
    entries[b] = {positions[b], window_start(positions[b], m->c.window), table_off[b], table_len[b]};
  std::vector<float> x, stage;
  run_layers_batch(m, tokens, positions, entries.data(), tables, batch, kv, num_blocks, block_size, x);
  apply_batched(m->lm_head, logits, x.data(), batch, stage);
}

// prefill_batched (model.rs:1222-1255): chunks of chunk_size positions of one sequence, then
// the LM head (matvec) on the final position only. logits: [vocab].
void orc_prefill(const orc_model* m, const uint32_t* tokens, int64_t n, int64_t start_pos, const int32_t* table,
                 int64_t table_len, float* kv, int64_t num_blocks, int64_t block_size, int64_t chunk_size, float* logits) {
  chunk_size = std::max<int64_t>(1, chunk_size);
  std::vector<float> x;
  int64_t last = 0;
  for (int64_t c0 = 0; c0 < n; c0 += chunk_size) {
    int64_t len = std::min(chunk_size, n - c0);
    std::vector<int64_t> pos(len);
    std::vector<orc_entry> entries(len);
    for (int64_t i = 0; i < len; ++i) {
      pos[i] = start_pos + c0 + i;
      entries[i] = {pos[i], window_start(pos[i], m->c.window), 0, table_len};
    }
    run_layers_batch(m, tokens + c0, pos.data(), entries.data(), table, len, kv, num_blocks, block_size, x);
    last = len - 1;
  }
  matvec(m->lm_head, logits, &x[last * m->c.hidden]);
}

// ---------------------------------------------------------------------------------------
// Sampling (src/sampling.rs).
// ---------------------------------------------------------------------------------------
// Rng::new (sampling.rs:20-25): the seed folded with a constant so that 0 is not a fixed point.
uint64_t orc_rng_new(uint64_t seed) { return seed ^ 0x9E3779B97F4A7C15ull; }

// Rng::next_u64 (sampling.rs:27-34): xorshift64* -- three xor-shifts of the state, output the
// state times a 64-bit odd constant (wrapping).
uint64_t orc_rng_next_u64(uint64_t* state) {
  uint64_t x = *state;
  x ^= x >> 12;
  x ^= x << 25;
  x ^= x >> 27;
  *state = x;
  return x * 0x2545F4914F6CDD1Dull;
}

// Rng::next_f32 (sampling.rs:36-40): the top 24 bits over 2^24, in [0, 1).
float orc_rng_next_f32(uint64_t* state) {
  return static_cast<float>(orc_rng_next_u64(state) >> 40) / static_cast<float>(1u << 24);
}

// Sampler::sample (sampling.rs:74-138). Rank by f32::total_cmp descending (the reference's
// unstable sort leaves equal logits in an unspecified order; here they keep ascending index),
// keep top_k, exponentiate relative to the top logit, normalize by the sequential f32 sum,
// cut the nucleus at the first cumulative >= top_p and renormalize, then walk the cumulative
// to the first value above one uniform draw. temperature <= 0: argmax, no draw.
int64_t orc_sample(const float* logits, int64_t n, float temperature, float top_p, int64_t top_k,
                   uint64_t* state) {
  if (n <= 0) return -1;
  if (temperature <= 0.0f) return orc_argmax(logits, n);
  auto key = [](float f) {
    int32_t b;
    std::memcpy(&b, &f, 4);
    return b ^ static_cast<int32_t>(static_cast<uint32_t>(b >> 31) >> 1);
  };
  std::vector<uint32_t> order(static_cast<size_t>(n));
  for (int64_t i = 0; i < n; ++i) order[i] = static_cast<uint32_t>(i);
  std::stable_sort(order.begin(), order.end(),
                   [&](uint32_t a, uint32_t b) { return key(logits[a]) > key(logits[b]); });
  const size_t keep = top_k == 0 ? order.size() : std::min<size_t>(static_cast<size_t>(top_k), order.size());
  order.resize(keep);
  const float inv_temp = 1.0f / temperature;
  const float max_logit = logits[order[0]];
  std::vector<float> probs(keep);
  for (size_t i = 0; i < keep; ++i) probs[i] = expf((logits[order[i]] - max_logit) * inv_temp);
  float total = 0.0f;
  for (float p : probs) total += p;
  for (float& p : probs) p /= total;
  if (top_p < 1.0f) {
    float cumulative = 0.0f;
    size_t cut = probs.size();
    for (size_t i = 0; i < probs.size(); ++i) {
      cumulative += probs[i];
      if (cumulative >= top_p) {
        cut = i + 1;
        break;
      }
    }
    probs.resize(cut);
    order.resize(cut);
    float renorm = 0.0f;
    for (float p : probs) renorm += p;
    for (float& p : probs) p /= renorm;
  }
  const float target = orc_rng_next_f32(state);
  float cumulative = 0.0f;
  for (size_t i = 0; i < probs.size(); ++i) {
    cumulative += probs[i];
    if (target < cumulative) return order[i];
  }
  return order.back();
}

}  // extern "C"
