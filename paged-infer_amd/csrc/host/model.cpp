// Device-resident Llama weights + paged KV cache, and the batched forward pass
// (LlamaWeights::run_layers_batch / decode_batch_into / prefill_batched, src/model.rs:968-1255).
//
// Weight layout in HBM: q/k/v rows concatenated into one [hidden + 2*kv_dim][ld] matrix and
// gate/up rows into one [2*inter][ld] matrix, so a decode layer streams its weights in four
// launches; rows are padded to 16 bytes (int8) so every lane issues aligned 128-bit loads.
// Activations are [batch][ld] f32 with ld a multiple of 16 floats.
#include <algorithm>
#include <array>
#include <cmath>
#include <map>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../common.h"
#include "../kernels.h"
#include "context.h"

namespace pia {
namespace {

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Rows up to which RMSNorm is fused into the projection that consumes it.
constexpr int64_t kFusedNormRows = 64;

struct Proj {
  int kind = -1;  // -1 unset, 0 f32, 1 int8
  int64_t rows = 0, cols = 0, ld = 0;
  DeviceBuffer w, s;
  uint32_t filled = 0;  // bitmask of filled sub-matrices
};

struct Layer {
  DeviceBuffer attn_norm, ffn_norm;
  Proj qkv, o, gu, down;
};

// Per-launch timing, by kernel class.
struct Prof {
  bool on = false;
  struct Rec {
    int cls;
    int64_t bytes;
    hipEvent_t a, b;
  };
  std::vector<hipEvent_t> pool;
  std::vector<Rec> recs;
  size_t used = 0;
  static constexpr int kClasses = 8;
  double ms[kClasses] = {};
  int64_t bytes[kClasses] = {};
  int64_t calls[kClasses] = {};

  hipEvent_t ev() {
    if (used == pool.size()) {
      hipEvent_t e;
      PIA_HIP(hipEventCreate(&e));
      pool.push_back(e);
    }
    return pool[used++];
  }
  void reset() {
    recs.clear();
    used = 0;
  }
  ~Prof() {
    for (auto e : pool) (void)hipEventDestroy(e);
  }
};

}  // namespace
}  // namespace pia

using namespace pia;

struct pia_model {
  pia_context* ctx = nullptr;
  pia_model_config cfg{};
  int64_t hd = 0, kvd = 0, qkv_rows = 0;
  int64_t ld_h = 0, ld_qkv = 0, ld_i = 0, ld_v = 0;
  DeviceBuffer embed, final_norm;
  bool embed_set = false, final_norm_set = false;
  std::vector<Layer> layers;
  Proj lm_head;

  DeviceBuffer kv;
  pia_kv_layout layout{};

  DeviceBuffer rope_cos, rope_sin;
  int64_t rope_len = 0;

  int64_t cap = 0;  // rows of activation scratch
  DeviceBuffer x, xb, qkv, attn, h, logits, amax, attn_work, step, xq;
  DeviceBuffer dec_split;  // split-K partial sums and counters of the decode GEMM
  bool dec_split_on = true;
  int64_t mfma_min = kMfmaMinBatch;
  bool replay_graphs = true;  // diagnostic PIA_NO_GRAPH=1: decode steps launch eagerly
  bool shared_prefix = true;  // diagnostic PIA_SHARED_PREFIX=0: no shared-prefix attention
  int64_t logit_rows = 0;  // rows of `logits` the last decode / prefill wrote
  DeviceBuffer samp;       // sampling parameters, generator states and drawn tokens
  // Decode block tables, device-resident between steps: entry b's table in slots
  // [b * tab_cap, b * tab_cap + table_len). tab_mirror holds what the device holds (-1: unknown),
  // so a step uploads only the slots that changed (append_block / copy-on-write remap).
  DeviceBuffer tab_dev;
  std::vector<int32_t> tab_mirror;
  int64_t tab_cap = 0, tab_rows = 0;
  // The last decode's host-to-device bytes: step inputs, table patches, whether the whole
  // table image was re-sent.
  int64_t up_bytes = 0, up_patches = 0;
  bool up_full = false;
  int64_t last_shared = 0, last_shared_splits = 0;  // virtual entries / splits of the last decode's shared prefix
  PinnedBuffer pin, pin_out;
  Prof prof;

  // Persistent batch-1 decode step (decode_step.hip).
  int decode_path = 0;        // 0: per-kernel launches, 1: persistent step at batch 1 when the shape allows
  int last_path = -1;         // path of the last decode: 0 per-kernel launches, 1 persistent step
  int step_state = -1;        // -1 not checked since the last weight change, 0 unsupported, 1 ready
  bool step_disabled = false;  // a grid barrier timed out: per-kernel launches from then on
  StepShape step_shape{};
  DeviceBuffer step_layers, step_part, step_ctrl, step_trace;  // ctrl: flags[num_cus * 32], step counter, error flag

  // Replayable decode / prefill steps. Every kernel argument is a device pointer into the
  // buffers above, so a graph stays valid until one of them is reallocated.
  std::map<std::array<int64_t, 8>, hipGraphExec_t> graphs;

  ~pia_model() { drop_graphs(); }

  hipStream_t st() const { return ctx->stream; }

  void drop_graphs() {
    for (auto& kv_ : graphs) (void)hipGraphExecDestroy(kv_.second);
    graphs.clear();
  }
  void grow(DeviceBuffer& b, size_t need) {
    if (need <= b.bytes) return;
    PIA_HIP(hipStreamSynchronize(st()));
    drop_graphs();
    b.ensure(need);
  }

  void begin(int cls, int64_t bytes, hipEvent_t* b) {
    if (!prof.on) return;
    hipEvent_t a = prof.ev();
    *b = prof.ev();
    PIA_HIP(hipEventRecord(a, st()));
    prof.recs.push_back({cls, bytes, a, *b});
  }
  void end(hipEvent_t b) {
    if (prof.on) PIA_HIP(hipEventRecord(b, st()));
  }
  template <typename F>
  void timed(int cls, int64_t bytes, F&& f) {
    hipEvent_t b = nullptr;
    begin(cls, bytes, &b);
    f();
    end(b);
  }

  void ensure_cap(int64_t rows) {
    if (rows <= cap) return;
    const int64_t c = std::max<int64_t>(rows, 8);
    grow(x, c * ld_h * 4);
    grow(xb, c * ld_h * 4);
    grow(qkv, c * ld_qkv * 4);
    grow(attn, c * ld_h * 4);
    grow(h, c * ld_i * 4);
    grow(amax, c * kArgmaxSlots * 8);
    grow(xq, xdigits_bytes(c, std::max(cfg.hidden, cfg.inter)));
    if (!dec_split.ptr) {
      dec_split.ensure(dec_split_bytes());
      PIA_HIP(hipMemset(dec_split.ptr, 0, dec_split_bytes()));  // launches leave it zero
    }
    cap = c;
  }

  void ensure_rope(int64_t max_pos) {
    if (max_pos < rope_len) return;
    int64_t n = std::max<int64_t>(1024, rope_len);
    while (n <= max_pos) n *= 2;
    const int64_t half = hd / 2;
    std::vector<float> c(n * half), s(n * half);
    // rope_table (src/math.rs:331-341), with the same libm calls as the reference's f32 methods.
    for (int64_t j = 0; j < half; ++j) {
      const float freq = 1.0f / powf(cfg.rope_theta, static_cast<float>(2 * j) / static_cast<float>(hd));
      for (int64_t p = 0; p < n; ++p) {
        const float a = static_cast<float>(p) * freq;
        c[p * half + j] = cosf(a);
        s[p * half + j] = sinf(a);
      }
    }
    PIA_HIP(hipStreamSynchronize(st()));
    drop_graphs();
    rope_cos.release();
    rope_sin.release();
    rope_cos.ensure(c.size() * 4);
    rope_sin.ensure(s.size() * 4);
    PIA_HIP(hipMemcpy(rope_cos.ptr, c.data(), c.size() * 4, hipMemcpyHostToDevice));
    PIA_HIP(hipMemcpy(rope_sin.ptr, s.data(), s.size() * 4, hipMemcpyHostToDevice));
    rope_len = n;
  }

  // Algorithmic bytes of one projection launch: int8 weights + scales (or f32 weights),
  // activations in, results out.
  static int64_t proj_bytes(const Proj& p, int64_t batch, Epi epi) {
    const int64_t wb = p.kind == 1 ? p.rows * p.cols + 4 * p.rows : 4 * p.rows * p.cols;
    const int64_t outr = epi == Epi::Swiglu ? p.rows / 2 : p.rows;
    return wb + 4 * batch * p.cols + 4 * batch * outr;
  }

  // Algorithmic bytes of one persistent decode step: every projection's weights and scales
  // read once, the K/V of the mapped window, and the activations of each stage.
  int64_t step_bytes(int64_t mapped_tokens) const {
    int64_t b = proj_bytes(lm_head, 1, Epi::Store);
    for (const auto& L : layers)
      b += proj_bytes(L.qkv, 1, Epi::Store) + proj_bytes(L.o, 1, Epi::Add) + proj_bytes(L.gu, 1, Epi::Swiglu) +
           proj_bytes(L.down, 1, Epi::Add);
    return b + cfg.layers * (mapped_tokens * cfg.kv_heads * 2 * hd * 4 + 2 * cfg.hidden * 4);
  }

  // Profiling classes (pia_model_profile_get): projections by role, attention, the rest.
  int proj_class(const Proj& p) const {
    if (&p == &lm_head) return 4;
    for (const auto& L : layers) {
      if (&p == &L.qkv) return 0;
      if (&p == &L.o) return 1;
      if (&p == &L.gu) return 2;
      if (&p == &L.down) return 3;
    }
    return 6;
  }

  void gemv(const Proj& p, const float* x_in, int64_t ldx, const float* norm_w, float* out, int64_t ldo,
            int64_t batch, Epi epi, unsigned long long* amax_out = nullptr) {
    const int cls = proj_class(p);
    if (p.kind == 1 && batch >= mfma_min) {
      timed(6, 0, [&] { launch_xdigits(x_in, ldx, norm_w, cfg.rms_eps, batch, p.cols, xq.ptr, st()); });
      hipEvent_t b = nullptr;
      begin(cls, proj_bytes(p, batch, epi), &b);
      const DecSplitWork split = dec_split_work(dec_split.ptr);
      launch_gemm_i8_mfma(static_cast<const int8_t*>(p.w.ptr), p.ld, p.s.as<float>(), xq.ptr, out, ldo, 1, p.rows,
                          p.cols, batch, epi, amax_out, dec_split_on ? &split : nullptr, st());
      end(b);
      return;
    }
    hipEvent_t b = nullptr;
    begin(cls, proj_bytes(p, batch, epi), &b);
    GemvArgs g{p.kind, p.w.ptr, p.ld, p.kind == 1 ? p.s.as<float>() : nullptr, x_in, ldx, norm_w, cfg.rms_eps,
               out, ldo, 1, p.rows, p.cols, batch, epi, amax_out};
    launch_gemv(g, st());
    end(b);
  }

  // A projection whose input is RMSNorm(x) * w: fused into the projection for small batches,
  // a separate normalization pass into xb for large ones.
  void normed_gemv(const Proj& p, const float* X, const float* norm_w, int64_t n, float* out, int64_t ldo, Epi epi,
                   unsigned long long* amax_out = nullptr) {
    if (n <= kFusedNormRows || (p.kind == 1 && n >= mfma_min)) {
      gemv(p, X, ld_h, norm_w, out, ldo, n, epi, amax_out);
    } else {
      timed(6, 0, [&] { launch_rmsnorm(X, ld_h, norm_w, xb.as<float>(), ld_h, n, cfg.hidden, cfg.rms_eps, st()); });
      gemv(p, xb.as<float>(), ld_h, nullptr, out, ldo, n, epi, amax_out);
    }
  }

  void check_complete() const {
    PIA_REQUIRE(embed_set && final_norm_set, "model: embedding and final norm must be set");
    PIA_REQUIRE(lm_head.kind >= 0 && lm_head.filled == 1, "model: lm_head not set");
    for (const auto& L : layers) {
      PIA_REQUIRE(L.qkv.filled == 7 && L.o.filled == 1 && L.gu.filled == 3 && L.down.filled == 1,
                  "model: every projection of every layer must be set");
      PIA_REQUIRE(L.attn_norm.ptr && L.ffn_norm.ptr, "model: every layer norm must be set");
    }
    PIA_REQUIRE(kv.ptr != nullptr, "model: KV cache not allocated (pia_model_kv_alloc)");
  }

  struct StepDev {
    const int32_t* tokens;
    const pia_attn_entry* entries;
    const int32_t* tables;
    // Shared-prefix decode: virtual entries and their (entry, split slot) map, n_shared of them.
    const pia_attn_entry* shared_entries = nullptr;
    const int32_t* shared_vmap = nullptr;
    int64_t n_shared = 0, shared_splits = 0;
  };

  // run_layers_batch (src/model.rs:968-1177) for `n` rows whose step inputs are already on the
  // device; leaves the residual stream (before the final norm) in x.
  // `prefill`: the entries are consecutive positions of one sequence sharing one table.
  void run_layers(int64_t n, const StepDev& in, const AttnPlan& plan, bool fused, int64_t mapped_tokens,
                  bool prefill = false) {
    const auto& c = cfg;
    const int64_t attn_bytes = mapped_tokens * c.kv_heads * 2 * hd * 4 + 2 * n * c.hidden * 4;
    float* X = x.as<float>();
    float* QKV = qkv.as<float>();
    float* ATT = attn.as<float>();
    float* H = h.as<float>();
    timed(6, 0, [&] {
      launch_embed(in.tokens, embed.as<uint16_t>(), X, ld_h, n, c.hidden, c.vocab, amax.as<unsigned long long>(), st());
    });
    for (int64_t l = 0; l < c.layers; ++l) {
      Layer& L = layers[l];
      normed_gemv(L.qkv, X, L.attn_norm.as<float>(), n, QKV, ld_qkv, Epi::Store);
      timed(5, attn_bytes, [&] {
        if (!fused)
          launch_rope_kv_write(QKV, ld_qkv, in.entries, in.tables, rope_cos.as<float>(), rope_sin.as<float>(),
                               kv.as<float>(), layout, c.heads, n, l, st());
        AttnLaunch a{QKV, ld_qkv, ATT, ld_h, kv.as<float>(), &layout, c.heads, in.entries, in.tables, n, l, plan,
                     attn_work.ptr, fused, rope_cos.as<float>(), rope_sin.as<float>(), prefill,
                     in.shared_entries, in.shared_vmap, in.n_shared, in.shared_splits};
        launch_attention(a, st());
      });
      gemv(L.o, ATT, ld_h, nullptr, X, ld_h, n, Epi::Add);
      normed_gemv(L.gu, X, L.ffn_norm.as<float>(), n, H, ld_i, Epi::Swiglu);
      gemv(L.down, H, ld_i, nullptr, X, ld_h, n, Epi::Add);
    }
  }

  // Whether the persistent step kernel runs this model's batch-1 decode (checked once per
  // weight change; builds the device array of layer pointers it reads).
  bool step_ready() {
    if (decode_path != 1 || step_disabled || cfg.attention_window == 0) return false;
    if (step_state >= 0) return step_state == 1;
    step_state = 0;
    if (lm_head.kind != 1) return false;
    for (const auto& L : layers)
      if (L.qkv.kind != 1 || L.o.kind != 1 || L.gu.kind != 1 || L.down.kind != 1) return false;
    const int ncu = ctx->num_cus;
    StepShape s{};
    s.hidden = cfg.hidden, s.heads = cfg.heads, s.hkv = cfg.kv_heads, s.hd = hd, s.inter = cfg.inter;
    s.vocab = cfg.vocab, s.qkv_rows = qkv_rows, s.lm_i8 = true;
    s.max_splits = decode_step_splits(ncu, cfg.kv_heads);
    const int64_t g = cfg.heads / cfg.kv_heads;
    s.max_tokens = std::min<int64_t>(2048, (static_cast<int64_t>(kMaxStepSmem) / 4 - g * hd - 2 * hd - 2 * g) / (1 + g));
    if (s.max_tokens < 16 || decode_step_unsupported(s, ncu)) return false;
    std::vector<StepLayer> v(cfg.layers);
    for (int64_t l = 0; l < cfg.layers; ++l) {
      const Layer& L = layers[l];
      v[l] = StepLayer{static_cast<const int8_t*>(L.qkv.w.ptr), L.qkv.s.as<float>(),
                       static_cast<const int8_t*>(L.o.w.ptr),   L.o.s.as<float>(),
                       static_cast<const int8_t*>(L.gu.w.ptr),  L.gu.s.as<float>(),
                       static_cast<const int8_t*>(L.down.w.ptr), L.down.s.as<float>(),
                       L.attn_norm.as<float>(),                  L.ffn_norm.as<float>()};
    }
    grow(step_layers, v.size() * sizeof(StepLayer));
    PIA_HIP(hipMemcpy(step_layers.ptr, v.data(), v.size() * sizeof(StepLayer), hipMemcpyHostToDevice));
    grow(step_part, static_cast<size_t>(cfg.heads) * s.max_splits * (hd + 2) * 4);
    const size_t ctrl = (static_cast<size_t>(ncu) * 32 + 64 + cfg.kv_heads * 32) * 4;
    if (step_ctrl.bytes < ctrl) {
      grow(step_ctrl, ctrl);
      PIA_HIP(hipMemset(step_ctrl.ptr, 0, ctrl));
    }
    if (std::getenv("PIA_STEP_TRACE")) grow(step_trace, (32 * cfg.layers + 4) * 8);
    step_shape = s;
    step_state = 1;
    return true;
  }
  // PIA_STEP_TRACE=1: mean device-clock microseconds of each stage of the last step, to stderr.
  void print_step_trace() {
    const int64_t n = 16 * cfg.layers + 2;
    std::vector<unsigned long long> t(2 * n);
    PIA_HIP(hipMemcpy(t.data(), step_trace.ptr, 2 * n * 8, hipMemcpyDeviceToHost));
    PIA_HIP(hipMemset(step_trace.ptr, 0, 2 * n * 8));
    int khz = 100000;
    (void)hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, ctx->device);
    const double us = 1e3 / khz;
    // Per stage (A qkv, B attention, D o, E gate/up, F down): WG 0's start, the latest
    // arrival of any workgroup at the stage's barrier, WG 0's exit from it.
    const int start[5] = {0, 2, 6, 9, 12}, arrive[5] = {1, 3, 8, 11, 14}, exitm[5] = {2, 4, 9, 12, -1};
    static const char* names[5] = {"A.qkv", "B.attn", "D.o", "E.gu", "F.down"};
    double work[5] = {}, bar[5] = {};
    for (int64_t l = 1; l < cfg.layers; ++l)
      for (int k = 0; k < 5; ++k) {
        const unsigned long long s0 = t[16 * l + start[k]], a = t[n + 16 * l + arrive[k]];
        const unsigned long long e = exitm[k] >= 0 ? t[16 * l + exitm[k]] : (l + 1 < cfg.layers ? t[16 * (l + 1)] : t[16 * cfg.layers]);
        work[k] += static_cast<double>(static_cast<long long>(a - s0)) * us;
        bar[k] += static_cast<double>(static_cast<long long>(e - a)) * us;
      }
    std::fprintf(stderr, "[step trace] per layer (us): slowest-WG work / barrier exit after last arrival:");
    for (int k = 0; k < 5; ++k)
      std::fprintf(stderr, " %s=%.2f/%.2f", names[k], work[k] / (cfg.layers - 1), bar[k] / (cfg.layers - 1));
    std::fprintf(stderr, " | LM=%.2f total=%.1f\n", static_cast<double>(t[n - 1] - t[n - 2]) * us,
                 static_cast<double>(t[n - 1] - t[0]) * us);
  }
  unsigned* step_flags() const { return step_ctrl.as<unsigned>(); }
  unsigned* step_counter() const { return step_ctrl.as<unsigned>() + ctx->num_cus * 32; }
  int* step_err() const { return reinterpret_cast<int*>(step_ctrl.as<unsigned>() + ctx->num_cus * 32 + 32); }

  // decode_batch_into at batch 1 as one launch (see decode_step.hip).
  void launch_step(const StepDev& in) {
    StepParams p{};
    p.layers = static_cast<int>(cfg.layers), p.hidden = static_cast<int>(cfg.hidden);
    p.heads = static_cast<int>(cfg.heads), p.hkv = static_cast<int>(cfg.kv_heads);
    p.inter = static_cast<int>(cfg.inter), p.vocab = static_cast<int>(cfg.vocab);
    p.qkv_rows = static_cast<int>(qkv_rows);
    p.ld_h = layers[0].qkv.ld, p.ld_i = layers[0].down.ld, p.ld_lm = lm_head.ld;
    p.eps = cfg.rms_eps, p.scale = 1.0f / sqrtf(static_cast<float>(hd));
    p.L = step_layers.as<StepLayer>();
    p.lm = lm_head.w.ptr, p.lm_s = lm_head.s.as<float>();
    p.final_norm = final_norm.as<float>(), p.embed = embed.as<uint16_t>();
    p.kv = kv.as<float>(), p.num_blocks = static_cast<int>(layout.num_blocks);
    p.block_size = static_cast<int>(layout.block_size);
    p.rope_cos = rope_cos.as<float>(), p.rope_sin = rope_sin.as<float>();
    p.token = in.tokens, p.entry = in.entries, p.tables = in.tables;
    p.x = x.as<float>(), p.qkv_buf = qkv.as<float>(), p.attn = attn.as<float>(), p.h = h.as<float>();
    p.part = step_part.as<float>(), p.logits = logits.as<float>(), p.amax = amax.as<unsigned long long>();
    p.flags = step_flags(), p.step_ctr = step_counter(), p.err = step_err();
    p.attn_cnt = step_counter() + 64;
    p.max_splits = static_cast<int>(step_shape.max_splits);
    p.trace = step_trace.as<unsigned long long>();
    launch_decode_step(p, step_shape, ctx->num_cus, st());
  }

  // Copy the fused-argmax slots back, take the max of each row's slots (the low 32 bits are
  // the winning row) and wait for the step.
  void read_argmax(int32_t* out, int64_t batch, bool step = false) {
    const size_t bytes = batch * kArgmaxSlots * 8;
    PIA_REQUIRE(bytes <= amax.bytes, "argmax read-back larger than the argmax slots");
    pin_out.ensure(bytes + 64);
    PIA_HIP(hipMemcpyAsync(pin_out.ptr, amax.ptr, bytes, hipMemcpyDeviceToHost, st()));
    int* err_h = reinterpret_cast<int*>(static_cast<char*>(pin_out.ptr) + bytes);
    if (step) PIA_HIP(hipMemcpyAsync(err_h, step_err(), 4, hipMemcpyDeviceToHost, st()));
    PIA_HIP(hipStreamSynchronize(st()));
    if (step && *err_h) {
      // A grid barrier ran out of its spin budget (the grid was not co-resident): the step's
      // results are void. Later steps use per-kernel launches.
      PIA_HIP(hipMemset(step_err(), 0, 4));
      step_disabled = true;
      drop_graphs();
      fail(PIA_ERR_HIP, "persistent decode step: grid barrier timed out; per-kernel launches from now on");
    }
    const auto* v = static_cast<const unsigned long long*>(pin_out.ptr);
    if (out)
      for (int64_t b = 0; b < batch; ++b) {
        unsigned long long best = 0;
        for (int i = 0; i < kArgmaxSlots; ++i) best = std::max(best, v[b * kArgmaxSlots + i]);
        out[b] = static_cast<int32_t>(best & 0xffffffffull);
      }
  }

  void finish_prof() {
    for (int i = 0; i < Prof::kClasses; ++i) prof.ms[i] = 0, prof.bytes[i] = 0, prof.calls[i] = 0;
    if (!prof.on) return;
    PIA_HIP(hipStreamSynchronize(st()));
    for (auto& r : prof.recs) {
      float t = 0;
      PIA_HIP(hipEventElapsedTime(&t, r.a, r.b));
      prof.ms[r.cls] += t;
      prof.bytes[r.cls] += r.bytes;
      prof.calls[r.cls] += 1;
    }
    prof.reset();
  }

  // Run `body` eagerly (one-shot calls such as prefill; profiling, where a short device spin
  // first lets the host enqueue ahead so each kernel's events bracket only that kernel), or
  // through a cached graph for `key` (decode steps, replayed every step).
  template <typename F>
  void run_step(const std::array<int64_t, 8>& key, bool replay, F&& body) {
    if (!replay_graphs) replay = false;
    if (!replay && !prof.on) {
      body();
      return;
    }
    if (prof.on) {
      prof.reset();
      launch_spin(3000.0, st());
      body();
      return;
    }
    auto it = graphs.find(key);
    if (it == graphs.end()) {
      hipGraph_t g = nullptr;
      PIA_HIP(hipStreamBeginCapture(st(), hipStreamCaptureModeRelaxed));
      try {
        body();
      } catch (...) {
        (void)hipStreamEndCapture(st(), &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      PIA_HIP(hipStreamEndCapture(st(), &g));
      hipGraphExec_t exec = nullptr;
      const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      PIA_HIP(e);
      it = graphs.emplace(key, exec).first;
    }
    PIA_HIP(hipGraphLaunch(it->second, st()));
  }
};

namespace {

void alloc_proj(Proj& p, int kind, int64_t rows, int64_t cols) {
  p.kind = kind;
  p.rows = rows;
  p.cols = cols;
  p.ld = round_up(cols, kind == 1 ? 64 : 4);  // int8 rows: whole 64-byte MFMA k-steps
  const int64_t esz = kind == 1 ? 1 : 4;
  p.w.ensure(rows * p.ld * esz);
  PIA_HIP(hipMemset(p.w.ptr, 0, rows * p.ld * esz));
  if (kind == 1) p.s.ensure(rows * 4);
  p.filled = 0;
}

// Copy `rows` host rows of `cols` into p at device rows r0, r0 + step, ..., with row padding.
void upload_rows(Proj& p, int64_t r0, int64_t rows, int64_t step, const void* src, const float* scales) {
  const int64_t esz = p.kind == 1 ? 1 : 4;
  PIA_HIP(hipMemcpy2D(static_cast<char*>(p.w.ptr) + r0 * p.ld * esz, step * p.ld * esz, src, p.cols * esz,
                      p.cols * esz, rows, hipMemcpyHostToDevice));
  if (p.kind == 1)
    PIA_HIP(hipMemcpy2D(p.s.as<float>() + r0, step * 4, scales, 4, 4, rows, hipMemcpyHostToDevice));
}

struct Target {
  Proj* p;
  int64_t r0, rows, cols;
  uint32_t bit;
  int64_t row_step = 1;  // device rows between consecutive source rows
};

Target target_of(pia_model* m, int64_t layer, int32_t which) {
  const auto& c = m->cfg;
  if (which == PIA_LM_HEAD) return {&m->lm_head, 0, c.vocab, c.hidden, 1};
  PIA_REQUIRE(layer >= 0 && layer < c.layers, "layer index out of range");
  Layer& L = m->layers[layer];
  switch (which) {
    case PIA_WQ: return {&L.qkv, 0, c.hidden, c.hidden, 1};
    case PIA_WK: return {&L.qkv, c.hidden, m->kvd, c.hidden, 2};
    case PIA_WV: return {&L.qkv, c.hidden + m->kvd, m->kvd, c.hidden, 4};
    case PIA_WO: return {&L.o, 0, c.hidden, c.hidden, 1};
    // gate / up rows interleaved: row 2i = gate i, row 2i + 1 = up i (SwiGLU epilogue).
    case PIA_W1: return {&L.gu, 0, c.inter, c.hidden, 1, 2};
    case PIA_W3: return {&L.gu, 1, c.inter, c.hidden, 2, 2};
    case PIA_W2: return {&L.down, 0, c.hidden, c.inter, 1};
    default: fail(PIA_ERR_INVALID, "unknown projection slot");
  }
}

int64_t total_rows(pia_model* m, const Proj* p) {
  const auto& c = m->cfg;
  if (p == &m->lm_head) return c.vocab;
  for (auto& L : m->layers) {
    if (p == &L.qkv) return m->qkv_rows;
    if (p == &L.o) return c.hidden;
    if (p == &L.gu) return 2 * c.inter;
    if (p == &L.down) return c.hidden;
  }
  return 0;
}

// The slot's projection group, (re)allocated for `kind`, with every replayable step dropped.
Target prepare_slot(pia_model* m, int64_t layer, int32_t which, int kind) {
  Target t = target_of(m, layer, which);
  PIA_HIP(hipSetDevice(m->ctx->device));
  PIA_HIP(hipStreamSynchronize(m->st()));
  if (t.p->kind != kind) {
    PIA_REQUIRE(t.p->filled == 0 || t.p->kind < 0,
                "fused projection group mixes int8 and f32 slots; set every slot of the group with one kind");
    alloc_proj(*t.p, kind, total_rows(m, t.p), t.cols);
    PIA_HIP(hipDeviceSynchronize());  // the zero fill of the row padding precedes later stream work
  }
  m->drop_graphs();  // a re-allocated projection moves; the step kernel's pointer table too
  m->step_state = -1;
  return t;
}

void set_proj(pia_model* m, int64_t layer, int32_t which, int kind, const void* data, const float* scales) {
  PIA_REQUIRE(m && data, "null argument");
  PIA_REQUIRE(kind == 0 || scales, "int8 projection needs scales");
  Target t = prepare_slot(m, layer, which, kind);
  upload_rows(*t.p, t.r0, t.rows, t.row_step, data, scales);
  t.p->filled |= t.bit;
}

}  // namespace

namespace pia {
void model_set_proj_bf16_dev(pia_model* m, int64_t layer, int32_t which, int kind, const uint16_t* src, int64_t rows,
                             int64_t cols) {
  PIA_REQUIRE(m && src, "null argument");
  PIA_REQUIRE(kind == 0 || kind == 1, "projection kind must be 0 (f32) or 1 (int8)");
  const Target want = target_of(m, layer, which);
  PIA_REQUIRE(rows == want.rows && cols == want.cols, "projection shape does not match the model config");
  Target t = prepare_slot(m, layer, which, kind);
  Proj& p = *t.p;
  if (kind == 1)
    launch_quantize_rows_bf16(src, t.rows, t.cols, p.w.as<int8_t>() + t.r0 * p.ld, p.ld, p.s.as<float>() + t.r0,
                              t.row_step, m->st());
  else
    launch_widen_rows_bf16(src, t.rows, t.cols, p.w.as<float>() + t.r0 * p.ld, p.ld, t.row_step, m->st());
  PIA_HIP(hipStreamSynchronize(m->st()));
  p.filled |= t.bit;
}
}  // namespace pia

extern "C" {

pia_status pia_model_create(pia_context* ctx, const pia_model_config* cfg, pia_model** out) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx && cfg && out, "null argument");
  const auto& c = *cfg;
  PIA_REQUIRE(c.hidden > 0 && c.layers > 0 && c.heads > 0 && c.kv_heads > 0 && c.inter > 0 && c.vocab > 0,
              "model dimensions must be positive");
  PIA_REQUIRE(c.hidden % c.heads == 0, "hidden_size must be a multiple of num_attention_heads");
  PIA_REQUIRE(c.heads % c.kv_heads == 0, "num_attention_heads must be a multiple of num_key_value_heads");
  auto* m = new pia_model;
  m->ctx = ctx;
  m->cfg = c;
  m->hd = c.hidden / c.heads;
  m->kvd = c.kv_heads * m->hd;
  m->qkv_rows = c.hidden + 2 * m->kvd;
  m->ld_h = round_up(c.hidden, 16);
  m->ld_qkv = round_up(m->qkv_rows, 16);
  m->ld_i = round_up(c.inter, 16);
  m->ld_v = round_up(c.vocab, 16);
  m->layers.resize(c.layers);
  // Diagnostic override of the batch from which decode projections use the matrix cores.
  if (const char* e = std::getenv("PIA_MFMA_MIN_BATCH")) m->mfma_min = std::max<int64_t>(2, std::atoll(e));
  // Diagnostic: PIA_DEC_SPLIT=0 turns the decode GEMM's split K off.
  if (const char* e = std::getenv("PIA_DEC_SPLIT")) m->dec_split_on = std::atoi(e) != 0;
  if (const char* e = std::getenv("PIA_NO_GRAPH")) m->replay_graphs = std::atoi(e) == 0;
  if (const char* e = std::getenv("PIA_SHARED_PREFIX")) m->shared_prefix = std::atoi(e) != 0;
  *out = m;
  PIA_API_END
}

// Must run before the context's destruction (the model enqueues work on the context stream).
pia_status pia_model_destroy(pia_model* m) {
  if (m) {
    (void)hipSetDevice(m->ctx->device);
    (void)hipStreamSynchronize(m->ctx->stream);
    delete m;
  }
  return PIA_OK;
}

pia_status pia_model_set_embedding(pia_model* m, const uint16_t* bf16) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && bf16, "null argument");
  const size_t bytes = static_cast<size_t>(m->cfg.vocab) * m->cfg.hidden * 2;
  PIA_HIP(hipStreamSynchronize(m->st()));
  m->drop_graphs();
  m->embed.ensure(bytes);
  PIA_HIP(hipMemcpy(m->embed.ptr, bf16, bytes, hipMemcpyHostToDevice));
  m->embed_set = true;
  PIA_API_END
}

pia_status pia_model_set_norm(pia_model* m, int64_t layer, int32_t which, const float* w) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && w, "null argument");
  DeviceBuffer* dst = nullptr;
  if (which == PIA_NORM_FINAL) {
    dst = &m->final_norm;
    m->final_norm_set = true;
  } else {
    PIA_REQUIRE(layer >= 0 && layer < m->cfg.layers, "layer index out of range");
    PIA_REQUIRE(which == PIA_NORM_ATTN || which == PIA_NORM_FFN, "unknown norm slot");
    dst = which == PIA_NORM_ATTN ? &m->layers[layer].attn_norm : &m->layers[layer].ffn_norm;
  }
  PIA_HIP(hipStreamSynchronize(m->st()));
  m->drop_graphs();
  m->step_state = -1;
  dst->ensure(m->cfg.hidden * 4);
  PIA_HIP(hipMemcpy(dst->ptr, w, m->cfg.hidden * 4, hipMemcpyHostToDevice));
  PIA_API_END
}

pia_status pia_model_set_proj_i8(pia_model* m, int64_t layer, int32_t which, const int8_t* q, const float* scales) {
  PIA_API_BEGIN
  set_proj(m, layer, which, 1, q, scales);
  PIA_API_END
}

pia_status pia_model_set_proj_f32(pia_model* m, int64_t layer, int32_t which, const float* w) {
  PIA_API_BEGIN
  set_proj(m, layer, which, 0, w, nullptr);
  PIA_API_END
}

pia_status pia_model_get_config(const pia_model* m, pia_model_config* out) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && out, "null argument");
  *out = m->cfg;
  PIA_API_END
}

int64_t pia_model_weight_bytes(const pia_model* m) {
  if (!m) return 0;
  auto pb = [](const Proj& p) -> int64_t {
    if (p.kind == 1) return p.rows * p.cols + 4 * p.rows;
    if (p.kind == 0) return 4 * p.rows * p.cols;
    return 0;
  };
  int64_t t = pb(m->lm_head);
  for (const auto& L : m->layers) t += pb(L.qkv) + pb(L.o) + pb(L.gu) + pb(L.down);
  return t;
}

pia_status pia_model_kv_alloc(pia_model* m, int64_t num_blocks, int64_t block_size) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && num_blocks > 0 && block_size > 0, "bad KV shape");
  PIA_HIP(hipSetDevice(m->ctx->device));
  m->layout = pia_kv_layout{m->cfg.layers, num_blocks, block_size, m->cfg.kv_heads, m->hd};
  const size_t bytes = static_cast<size_t>(m->cfg.layers) * num_blocks * block_size * m->cfg.kv_heads * 2 * m->hd * 4;
  PIA_HIP(hipStreamSynchronize(m->st()));
  m->drop_graphs();  // captured steps hold the old cache address
  m->kv.release();
  m->kv.ensure(bytes);
  PIA_HIP(hipMemset(m->kv.ptr, 0, bytes));
  PIA_API_END
}

pia_status pia_model_kv(pia_model* m, float** kv, pia_kv_layout* layout) {
  PIA_API_BEGIN
  PIA_REQUIRE(m, "null model");
  if (kv) *kv = m->kv.as<float>();
  if (layout) *layout = m->layout;
  PIA_API_END
}

pia_status pia_model_set_decode_path(pia_model* m, int32_t path) {
  PIA_API_BEGIN
  PIA_REQUIRE(m, "null model");
  PIA_REQUIRE(path == 0 || path == 1, "decode path must be 0 (per-kernel launches) or 1 (persistent step)");
  if (path != m->decode_path) {
    PIA_HIP(hipStreamSynchronize(m->st()));
    m->drop_graphs();
    m->decode_path = path;
    m->step_state = -1;
  }
  PIA_API_END
}

int32_t pia_model_decode_path_used(const pia_model* m) { return m ? m->last_path : -1; }

pia_status pia_model_last_shared(const pia_model* m, int64_t* virtual_entries, int64_t* shared_splits) {
  PIA_API_BEGIN
  PIA_REQUIRE(m, "null model");
  if (virtual_entries) *virtual_entries = m->last_shared;
  if (shared_splits) *shared_splits = m->last_shared_splits;
  PIA_API_END
}

pia_status pia_model_last_upload(const pia_model* m, int64_t* bytes, int64_t* table_patches, int32_t* table_full) {
  PIA_API_BEGIN
  PIA_REQUIRE(m, "null model");
  if (bytes) *bytes = m->up_bytes;
  if (table_patches) *table_patches = m->up_patches;
  if (table_full) *table_full = m->up_full ? 1 : 0;
  PIA_API_END
}

pia_status pia_model_profile(pia_model* m, int32_t enable) {
  PIA_API_BEGIN
  PIA_REQUIRE(m, "null model");
  m->prof.on = enable != 0;
  PIA_API_END
}

pia_status pia_model_profile_get(pia_model* m, double* ms, int64_t* bytes, int64_t* calls, int32_t n) {
  PIA_API_BEGIN
  PIA_REQUIRE(m, "null model");
  for (int i = 0; i < n && i < Prof::kClasses; ++i) {
    if (ms) ms[i] = m->prof.ms[i];
    if (bytes) bytes[i] = m->prof.bytes[i];
    if (calls) calls[i] = m->prof.calls[i];
  }
  PIA_API_END
}

// Device time per launch of one projection class (0 = q/k/v, 1 = o, 2 = gate/up, 3 = down,
// 4 = LM head) at `batch`: the class's launches for every layer (the model's own weights and
// buffers, the exact kernels and arguments of a decode step) captured `reps` times in one graph,
// HIP events around a replay. Inter-kernel gaps inside a graph are ~0.25 us on MI355X.
pia_status pia_model_bench_class(pia_model* m, int32_t cls, int64_t batch, int32_t reps, double* us,
                                 int64_t* bytes) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && us && bytes, "null argument");
  PIA_REQUIRE(cls >= 0 && cls <= 4 && batch > 0 && batch <= kFusedNormRows && reps > 0 && reps <= 100,
              "bad profiling request");
  m->check_complete();
  PIA_HIP(hipSetDevice(m->ctx->device));
  m->ensure_cap(batch);
  m->grow(m->logits, batch * m->ld_v * 4);
  const bool prof_was = m->prof.on;
  m->prof.on = false;
  hipStream_t st = m->st();
  float* X = m->x.as<float>();
  float* H = m->h.as<float>();
  auto launch = [&](int64_t l) {
    Layer& L = m->layers[l];
    switch (cls) {
      case 0: m->normed_gemv(L.qkv, X, L.attn_norm.as<float>(), batch, m->qkv.as<float>(), m->ld_qkv, Epi::Store); break;
      case 1: m->gemv(L.o, m->attn.as<float>(), m->ld_h, nullptr, X, m->ld_h, batch, Epi::Add); break;
      case 2: m->normed_gemv(L.gu, X, L.ffn_norm.as<float>(), batch, H, m->ld_i, Epi::Swiglu); break;
      case 3: m->gemv(L.down, H, m->ld_i, nullptr, X, m->ld_h, batch, Epi::Add); break;
      default:
        m->normed_gemv(m->lm_head, X, m->final_norm.as<float>(), batch, m->logits.as<float>(), m->ld_v, Epi::Store,
                       m->amax.as<unsigned long long>());
    }
  };
  const int64_t per = cls == 4 ? 1 : m->cfg.layers;
  const Proj& probe = cls == 4 ? m->lm_head : cls == 0 ? m->layers[0].qkv : cls == 1 ? m->layers[0].o
                      : cls == 2 ? m->layers[0].gu : m->layers[0].down;
  PIA_HIP(hipMemsetAsync(X, 0, batch * m->ld_h * 4, st));  // finite inputs for the timed launches
  PIA_HIP(hipMemsetAsync(H, 0, batch * m->ld_i * 4, st));
  PIA_HIP(hipMemsetAsync(m->attn.ptr, 0, batch * m->ld_h * 4, st));
  for (int64_t l = 0; l < per; ++l) launch(l);  // warm: also fills the digit workspace
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  PIA_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
  try {
    for (int r = 0; r < reps; ++r)
      for (int64_t l = 0; l < per; ++l) launch(l);
  } catch (...) {
    (void)hipStreamEndCapture(st, &graph);
    if (graph) (void)hipGraphDestroy(graph);
    m->prof.on = prof_was;
    throw;
  }
  PIA_HIP(hipStreamEndCapture(st, &graph));
  PIA_HIP(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
  hipEvent_t e0, e1;
  PIA_HIP(hipEventCreate(&e0));
  PIA_HIP(hipEventCreate(&e1));
  PIA_HIP(hipGraphLaunch(exec, st));
  PIA_HIP(hipEventRecord(e0, st));
  PIA_HIP(hipGraphLaunch(exec, st));
  PIA_HIP(hipEventRecord(e1, st));
  PIA_HIP(hipStreamSynchronize(st));
  float ms = 0;
  PIA_HIP(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  (void)hipGraphExecDestroy(exec);
  (void)hipGraphDestroy(graph);
  m->prof.on = prof_was;
  *us = 1e3 * ms / static_cast<double>(reps * per);
  *bytes = pia_model::proj_bytes(probe, batch, cls == 2 ? Epi::Swiglu : Epi::Store);
  PIA_API_END
}

}  // extern "C"

namespace {

int64_t window_start(int64_t pos, int64_t window) {
  if (window < 0) return 0;
  return pos + 1 > window ? pos + 1 - window : 0;
}

// Stage tokens, entries and tables in one pinned buffer and one host->device copy. The
// device step buffer keeps its address across calls (captured graphs read it).
pia_model::StepDev upload_step(pia_model* m, const std::vector<int32_t>& tok, const std::vector<pia_attn_entry>& ent,
                               const int32_t* tables, int64_t ntab) {
  const size_t n = tok.size();
  const size_t off_e = round_up(n * 4, 256), off_t = off_e + round_up(n * sizeof(pia_attn_entry), 256);
  const size_t total = off_t + round_up(std::max<int64_t>(ntab, 1) * 4, 256);
  PIA_HIP(hipStreamSynchronize(m->st()));  // the pinned staging buffer may still be in flight
  m->pin.ensure(total);
  m->grow(m->step, std::max<size_t>(total, 1 << 16));
  char* p = static_cast<char*>(m->pin.ptr);
  std::memcpy(p, tok.data(), n * 4);
  std::memcpy(p + off_e, ent.data(), n * sizeof(pia_attn_entry));
  if (ntab) std::memcpy(p + off_t, tables, ntab * 4);
  PIA_HIP(hipMemcpyAsync(m->step.ptr, p, total, hipMemcpyHostToDevice, m->st()));
  char* d = static_cast<char*>(m->step.ptr);
  return {reinterpret_cast<const int32_t*>(d), reinterpret_cast<const pia_attn_entry*>(d + off_e),
          reinterpret_cast<const int32_t*>(d + off_t)};
}

// Decode step inputs: tokens and entries (every step) plus the block tables, which stay on the
// device in per-entry slots of tab_cap ids; only the slots whose ids differ from the device copy
// travel, as (slot, id) pairs applied by a scatter kernel, unless the layout changed or most
// slots differ (then the whole image). Host entries index the caller's flat `tables`; the
// device entries index the resident slots.
struct SharePlan {
  std::vector<int32_t> start;         // per entry: first token the per-entry launch covers
  std::vector<pia_attn_entry> vent;   // virtual entries (table_off = index of the group's first entry)
  std::vector<int32_t> vmap;          // [vent][2]: entry, split slot
  int64_t splits = 0;
};

pia_model::StepDev upload_decode_step(pia_model* m, const std::vector<int32_t>& tok,
                                      const std::vector<pia_attn_entry>& ent, const int32_t* tables,
                                      const SharePlan* sh = nullptr) {
  const int64_t n = static_cast<int64_t>(tok.size());
  int64_t maxlen = 1;
  for (const auto& e : ent) maxlen = std::max<int64_t>(maxlen, e.table_len);
  const int64_t cap = round_up(maxlen, 64);
  bool full = false;
  if (cap > m->tab_cap || n > m->tab_rows) {
    const int64_t ncap = std::max(cap, m->tab_cap), nrows = std::max<int64_t>(round_up(n, 8), m->tab_rows);
    PIA_HIP(hipStreamSynchronize(m->st()));
    m->drop_graphs();  // captured steps hold the old table address
    m->tab_dev.release();
    m->tab_dev.ensure(nrows * ncap * 4);
    m->tab_cap = ncap, m->tab_rows = nrows;
    m->tab_mirror.assign(nrows * ncap, -1);
    full = true;
  }
  const int64_t tc = m->tab_cap;
  std::vector<int32_t> patch;
  if (!full) {
    for (int64_t b = 0; b < n; ++b)
      for (int32_t i = 0; i < ent[b].table_len; ++i) {
        const int64_t slot = b * tc + i;
        const int32_t id = tables[ent[b].table_off + i];
        if (m->tab_mirror[slot] != id) {
          patch.push_back(static_cast<int32_t>(slot));
          patch.push_back(id);
        }
      }
    full = static_cast<int64_t>(patch.size() / 2) * 8 > n * tc;  // most slots changed: send the image
  }
  std::vector<pia_attn_entry> dent(ent);
  for (int64_t b = 0; b < n; ++b) {
    dent[b].table_off = static_cast<int32_t>(b * tc);
    if (sh) dent[b].start = sh->start[b];
  }
  const int64_t nv = sh ? static_cast<int64_t>(sh->vent.size()) : 0;
  std::vector<pia_attn_entry> vdev(nv);
  for (int64_t v = 0; v < nv; ++v) {
    vdev[v] = sh->vent[v];
    vdev[v].table_off = static_cast<int32_t>(sh->vent[v].table_off * tc);
  }
  const size_t off_v = round_up(n * 4, 256);  // virtual entries and map right after the tokens
  const size_t off_m = off_v + round_up(nv * sizeof(pia_attn_entry), 256);
  const size_t off_e = off_m + round_up(nv * 8, 256), off_t = off_e + round_up(n * sizeof(pia_attn_entry), 256);
  const size_t tab_bytes = full ? static_cast<size_t>(n * tc * 4) : patch.size() * 4;
  const size_t total = off_t + round_up(std::max<size_t>(tab_bytes, 4), 256);
  PIA_HIP(hipStreamSynchronize(m->st()));  // the pinned staging buffer may still be in flight
  m->pin.ensure(total);
  m->grow(m->step, std::max<size_t>(total, 1 << 16));
  char* p = static_cast<char*>(m->pin.ptr);
  std::memcpy(p, tok.data(), n * 4);
  if (nv) {
    std::memcpy(p + off_v, vdev.data(), nv * sizeof(pia_attn_entry));
    std::memcpy(p + off_m, sh->vmap.data(), nv * 8);
  }
  std::memcpy(p + off_e, dent.data(), n * sizeof(pia_attn_entry));
  char* d = static_cast<char*>(m->step.ptr);
  if (full) {
    auto* img = reinterpret_cast<int32_t*>(p + off_t);
    for (int64_t b = 0; b < n; ++b)
      for (int64_t i = 0; i < tc; ++i) {
        const int32_t id = i < ent[b].table_len ? tables[ent[b].table_off + i] : 0;
        img[b * tc + i] = id;
        m->tab_mirror[b * tc + i] = id;
      }
    PIA_HIP(hipMemcpyAsync(d, p, off_t, hipMemcpyHostToDevice, m->st()));
    PIA_REQUIRE(tab_bytes <= m->tab_dev.bytes && off_t + tab_bytes <= m->pin.bytes, "block-table image exceeds its buffers");
    PIA_HIP(hipMemcpyAsync(m->tab_dev.ptr, img, tab_bytes, hipMemcpyHostToDevice, m->st()));
  } else {
    PIA_REQUIRE(off_t + tab_bytes <= m->pin.bytes && off_t + tab_bytes <= m->step.bytes, "table patch exceeds the staging buffers");
    if (!patch.empty()) std::memcpy(p + off_t, patch.data(), tab_bytes);
    PIA_HIP(hipMemcpyAsync(d, p, off_t + tab_bytes, hipMemcpyHostToDevice, m->st()));
    launch_table_patch(m->tab_dev.as<int32_t>(), reinterpret_cast<const int32_t*>(d + off_t),
                       static_cast<int64_t>(patch.size() / 2), m->st());
    for (size_t i = 0; i < patch.size(); i += 2) m->tab_mirror[patch[i]] = patch[i + 1];
  }
  m->up_bytes = static_cast<int64_t>(n * 4 + n * sizeof(pia_attn_entry) + tab_bytes + nv * (sizeof(pia_attn_entry) + 8));
  m->up_patches = static_cast<int64_t>(patch.size() / 2);
  m->up_full = full;
  m->last_shared = nv;
  m->last_shared_splits = nv ? sh->splits : 0;
  pia_model::StepDev out{reinterpret_cast<const int32_t*>(d), reinterpret_cast<const pia_attn_entry*>(d + off_e),
                         m->tab_dev.as<int32_t>()};
  if (nv) {
    out.shared_entries = reinterpret_cast<const pia_attn_entry*>(d + off_v);
    out.shared_vmap = reinterpret_cast<const int32_t*>(d + off_m);
    out.n_shared = nv;
    out.shared_splits = sh->splits;
  }
  return out;
}

// Shared-prefix decode plan (src/memory/prefix_cache.rs maps one physical block into many
// sequences' tables): entries whose tables begin with the same physical blocks form a group;
// the blocks every member holds at the same logical index, up to the block before each
// member's current position, are its shared prefix. Their K/V are read once per group by the
// query-tiled kernel (all members' query heads of one kv head per tile) instead of once per
// entry; each entry's own launch covers the rest of its window. Used when every entry is in a
// group with at least kMinSharedTokens shared tokens (no sliding window).
bool plan_shared_prefix(const pia_model* m, const std::vector<pia_attn_entry>& ent, const int32_t* tables,
                        SharePlan& sh) {
  constexpr int64_t kMinSharedTokens = 128;
  const int64_t n = static_cast<int64_t>(ent.size()), bs = m->layout.block_size;
  if (n < 2 || m->cfg.attention_window >= 0 || (m->hd != 64 && m->hd != 128)) return false;
  std::map<int32_t, std::vector<int64_t>> groups;
  for (int64_t b = 0; b < n; ++b) {
    if (ent[b].start != 0 || ent[b].table_len < 1) return false;
    groups[tables[ent[b].table_off]].push_back(b);
  }
  const int64_t g = m->cfg.heads / m->cfg.kv_heads;
  const int64_t qt = attention_tile_rows() / g;  // entries per tile
  if (qt < 1) return false;
  const int64_t chunk = m->hd <= 64 ? 64 : 32;
  std::vector<std::pair<std::vector<int64_t>, int64_t>> gl;  // members, shared tokens
  int64_t tiles = 0;
  sh.start.assign(n, 0);
  for (auto& kv_ : groups) {
    const auto& mem = kv_.second;
    if (mem.size() < 2) return false;
    const pia_attn_entry& f = ent[mem[0]];
    int64_t blocks = f.table_len;
    for (int64_t b : mem) {
      const pia_attn_entry& e = ent[b];
      blocks = std::min<int64_t>(blocks, std::min<int64_t>(e.table_len, e.pos / bs));
      int64_t i = 0;
      while (i < blocks && tables[e.table_off + i] == tables[f.table_off + i]) ++i;
      blocks = i;
    }
    const int64_t len = blocks * bs;
    if (len < kMinSharedTokens) return false;
    for (int64_t b : mem) sh.start[b] = static_cast<int32_t>(len);
    tiles += (static_cast<int64_t>(mem.size()) + qt - 1) / qt;
    gl.emplace_back(mem, len);
  }
  // Shared splits: about two workgroups per CU over (tiles x kv heads x splits).
  int64_t max_len = 0;
  for (auto& x : gl) max_len = std::max(max_len, x.second);
  const int64_t want = (2 * m->ctx->num_cus + tiles * m->cfg.kv_heads - 1) / (tiles * m->cfg.kv_heads);
  sh.splits = std::max<int64_t>(1, std::min<int64_t>({want, 16, (max_len + chunk - 1) / chunk}));
  for (auto& x : gl) {
    const auto& mem = x.first;
    const int64_t len = x.second;
    const int64_t per = round_up((len + sh.splits - 1) / sh.splits, chunk);
    for (int64_t s = 0; s < sh.splits; ++s) {
      const int64_t a = std::min(len, s * per), b = std::min(len, (s + 1) * per);
      for (size_t t0 = 0; t0 < mem.size(); t0 += qt)
        for (int64_t i = 0; i < qt; ++i) {
          const size_t k = t0 + i;
          const int64_t who = k < mem.size() ? mem[k] : mem[0];
          // [a, b): an empty range still writes its (neutral) partials; padding rows (pos -1)
          // write nothing.
          const int32_t pos = k < mem.size() ? static_cast<int32_t>(b - 1) : -1;
          sh.vent.push_back(pia_attn_entry{pos, static_cast<int32_t>(a), static_cast<int32_t>(mem[0]),
                                           ent[mem[0]].table_len});
          sh.vmap.push_back(static_cast<int32_t>(who));
          sh.vmap.push_back(static_cast<int32_t>(s));
        }
    }
  }
  return true;
}

int64_t mapped_in_window(const pia_attn_entry& e, int64_t bs) {
  // Tokens of start..=pos that fall inside mapped logical blocks (the K/V actually read).
  const int64_t end = std::min<int64_t>(e.pos + 1, static_cast<int64_t>(e.table_len) * bs);
  return std::max<int64_t>(0, end - e.start);
}

// The fused attention writes each entry's K/V inside the attention launch, so it is only
// used when no entry can read a slot another entry of the batch writes: the block each entry
// writes must appear in no other entry's table (always true for decode batches after
// copy-on-write; never for prefill chunks, whose entries share one table).
bool fusable(const std::vector<pia_attn_entry>& ent, const int32_t* tables, int64_t bs, int64_t window) {
  if (window == 0) return false;  // the K/V write must still happen with an empty window
  std::map<int32_t, int> owner;   // written block -> entry
  for (size_t b = 0; b < ent.size(); ++b) {
    const int64_t lb = ent[b].pos / bs;
    if (lb < ent[b].table_len) {
      const int32_t blk = tables[ent[b].table_off + lb];
      if (!owner.emplace(blk, static_cast<int>(b)).second) return false;
    }
  }
  if (owner.empty()) return true;
  for (size_t b = 0; b < ent.size(); ++b)
    for (int32_t i = 0; i < ent[b].table_len; ++i) {
      auto it = owner.find(tables[ent[b].table_off + i]);
      if (it != owner.end() && it->second != static_cast<int>(b)) return false;
    }
  return true;
}

}  // namespace

extern "C" {

pia_status pia_model_decode(pia_model* m, const uint32_t* tokens, const int64_t* positions, const int64_t* table_off,
                            const int64_t* table_len, const int32_t* tables, int64_t batch, float* logits,
                            int32_t* argmax) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && tokens && positions && table_off && table_len, "null argument");
  PIA_REQUIRE(batch > 0, "decode needs at least one sequence");
  m->check_complete();
  PIA_HIP(hipSetDevice(m->ctx->device));
  const auto& c = m->cfg;
  int64_t ntab = 0, max_pos = 0, max_window = 1, mapped = 0;
  std::vector<int32_t> tok(batch);
  std::vector<pia_attn_entry> ent(batch);
  for (int64_t b = 0; b < batch; ++b) {
    PIA_REQUIRE(positions[b] >= 0 && positions[b] < (int64_t(1) << 30), "position out of range");
    PIA_REQUIRE(table_off[b] >= 0 && table_len[b] >= 0 && table_off[b] + table_len[b] < (int64_t(1) << 31),
                "bad table offset/length");
    ntab = std::max(ntab, table_off[b] + table_len[b]);
    max_pos = std::max(max_pos, positions[b]);
    tok[b] = static_cast<int32_t>(tokens[b]);
    const int64_t st = window_start(positions[b], c.attention_window);
    ent[b] = pia_attn_entry{static_cast<int32_t>(positions[b]), static_cast<int32_t>(st),
                            static_cast<int32_t>(table_off[b]), static_cast<int32_t>(table_len[b])};
    max_window = std::max(max_window, positions[b] + 1 - st);
    mapped += mapped_in_window(ent[b], m->layout.block_size);
  }
  PIA_REQUIRE(ntab == 0 || tables, "null block tables");
  for (int64_t i = 0; i < ntab; ++i)
    PIA_REQUIRE(tables[i] >= 0 && tables[i] < m->layout.num_blocks, "block table entry out of range");
  const bool fused = fusable(ent, tables, m->layout.block_size, c.attention_window);
  SharePlan sh;
  bool shared = fused && m->shared_prefix && plan_shared_prefix(m, ent, tables, sh);
  int64_t own_window = max_window;  // tokens the per-entry launch covers
  if (shared) {
    own_window = 1;
    for (int64_t b = 0; b < batch; ++b) own_window = std::max<int64_t>(own_window, ent[b].pos + 1 - sh.start[b]);
  }
  AttnPlan plan = plan_attention(batch, c.kv_heads, m->hd, own_window, m->ctx->num_cus);
  if (shared && plan.splits + sh.splits > 128) {
    shared = false;
    sh = SharePlan{};
    plan = plan_attention(batch, c.kv_heads, m->hd, max_window, m->ctx->num_cus);
  }
  m->ensure_cap(batch);
  m->ensure_rope(max_pos);
  m->grow(m->logits, batch * m->ld_v * 4);
  const int64_t wb = attention_work_bytes(batch, c.heads, m->hd, plan.splits + (shared ? sh.splits : 0));
  if (wb) m->grow(m->attn_work, wb);
  const bool step = batch == 1 && m->step_ready() &&
                    max_window <= m->step_shape.max_splits * m->step_shape.max_tokens;
  const pia_model::StepDev in = upload_decode_step(m, tok, ent, tables, shared ? &sh : nullptr);
  if (step) {
    m->run_step({2, 1, 0, 0, 0, 0, 0, 0}, true, [&] {
      m->timed(7, m->step_bytes(mapped), [&] { m->launch_step(in); });
    });
  } else {
    m->run_step({0, batch, plan.split, plan.splits, plan.chunk, fused ? 1 : 0, in.n_shared, in.shared_splits}, true,
                [&] {
      m->run_layers(batch, in, plan, fused, mapped);
      m->normed_gemv(m->lm_head, m->x.as<float>(), m->final_norm.as<float>(), batch, m->logits.as<float>(), m->ld_v,
                     Epi::Store, m->amax.as<unsigned long long>());
    });
  }
  if (logits) {
    PIA_REQUIRE(static_cast<size_t>(batch * m->ld_v * 4) <= m->logits.bytes, "logits read-back exceeds the logits buffer");
    PIA_HIP(hipMemcpy2DAsync(logits, c.vocab * 4, m->logits.ptr, m->ld_v * 4, c.vocab * 4, batch,
                             hipMemcpyDeviceToHost, m->st()));
  }
  m->last_path = step ? 1 : 0;
  m->logit_rows = batch;
  m->read_argmax(argmax, batch, step);
  if (step && m->step_trace.ptr) m->print_step_trace();
  m->finish_prof();
  PIA_API_END
}

pia_status pia_model_prefill(pia_model* m, const uint32_t* tokens, int64_t n, int64_t start_pos, const int32_t* table,
                             int64_t table_len, float* logits, int32_t* argmax) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && tokens, "null argument");
  PIA_REQUIRE(n > 0, "prefill needs at least one token");
  PIA_REQUIRE(start_pos >= 0 && start_pos + n < (int64_t(1) << 30), "position out of range");
  PIA_REQUIRE(table_len >= 0 && table_len < (int64_t(1) << 31) && (table_len == 0 || table), "bad block table");
  m->check_complete();
  PIA_HIP(hipSetDevice(m->ctx->device));
  const auto& c = m->cfg;
  for (int64_t i = 0; i < table_len; ++i)
    PIA_REQUIRE(table[i] >= 0 && table[i] < m->layout.num_blocks, "block table entry out of range");
  std::vector<int32_t> tok(n);
  std::vector<pia_attn_entry> ent(n);
  int64_t max_window = 1, mapped = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t pos = start_pos + i;
    const int64_t st = window_start(pos, c.attention_window);
    tok[i] = static_cast<int32_t>(tokens[i]);
    ent[i] = pia_attn_entry{static_cast<int32_t>(pos), static_cast<int32_t>(st), 0, static_cast<int32_t>(table_len)};
    max_window = std::max(max_window, pos + 1 - st);
    mapped += mapped_in_window(ent[i], m->layout.block_size);
  }
  const AttnPlan plan = plan_attention(n, c.kv_heads, m->hd, max_window, m->ctx->num_cus);
  const bool fused = n == 1 && fusable(ent, table, m->layout.block_size, c.attention_window);
  m->ensure_cap(n);
  m->ensure_rope(start_pos + n);
  m->grow(m->logits, m->ld_v * 4);
  const int64_t wb = attention_work_bytes(n, c.heads, m->hd, plan.splits);
  if (wb) m->grow(m->attn_work, wb);
  const pia_model::StepDev in = upload_step(m, tok, ent, table, table_len);
  m->run_step({1, n, plan.split, plan.splits, plan.chunk, fused ? 1 : 0, 0, 0}, false, [&] {
    m->run_layers(n, in, plan, fused, mapped, true);
    // Only the last position pays for the LM head (src/model.rs:1249-1254).
    m->normed_gemv(m->lm_head, m->x.as<float>() + (n - 1) * m->ld_h, m->final_norm.as<float>(), 1,
                   m->logits.as<float>(), m->ld_v, Epi::Store, m->amax.as<unsigned long long>());
  });
  if (logits) PIA_HIP(hipMemcpyAsync(logits, m->logits.ptr, c.vocab * 4, hipMemcpyDeviceToHost, m->st()));
  m->logit_rows = 1;
  m->read_argmax(argmax, 1);
  m->finish_prof();
  PIA_API_END
}

pia_status pia_model_sample(pia_model* m, const pia_sampling* params, uint64_t* rng_state, int64_t n, int32_t mode,
                            int32_t* out) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && params && rng_state && out, "null argument");
  PIA_REQUIRE(n > 0 && n <= m->logit_rows, "sample: no logits for that many rows (decode or prefill first)");
  for (int64_t i = 0; i < n; ++i) {
    PIA_REQUIRE(params[i].top_k >= 0 && params[i].reserved == 0, "sample: bad sampling parameters");
    PIA_REQUIRE(params[i].temperature == params[i].temperature && params[i].top_p == params[i].top_p,
                "sample: NaN temperature or top_p");
  }
  PIA_HIP(hipSetDevice(m->ctx->device));
  // One upload of [params][states] and one download of [states][tokens] through pinned staging
  // (the previous decode's uploads from it finished before that call returned).
  const size_t pb = static_cast<size_t>(n) * sizeof(pia_sampling), rb = static_cast<size_t>(n) * 8;
  const size_t ob = static_cast<size_t>(n) * 4;
  m->grow(m->samp, pb + rb + ob);
  m->pin.ensure(pb + rb);
  m->pin_out.ensure(rb + ob);
  std::memcpy(m->pin.ptr, params, pb);
  std::memcpy(static_cast<char*>(m->pin.ptr) + pb, rng_state, rb);
  char* d = static_cast<char*>(m->samp.ptr);
  PIA_HIP(hipMemcpyAsync(d, m->pin.ptr, pb + rb, hipMemcpyHostToDevice, m->st()));
  // Every row greedy or with a small top-k: no sort of the vocabulary is needed, and the result
  // is the reference's in either mode.
  bool small_k = true;
  for (int64_t i = 0; i < n; ++i)
    small_k = small_k && (!(params[i].temperature > 0.0f) || (params[i].top_k > 0 && params[i].top_k <= sample_topk_max()));
  if (small_k)
    launch_sample_topk(m->logits.as<float>(), m->ld_v, n, m->cfg.vocab, reinterpret_cast<const pia_sampling*>(d),
                       reinterpret_cast<uint64_t*>(d + pb), reinterpret_cast<int32_t*>(d + pb + rb), m->st());
  else
    sample_with_context(m->ctx, reinterpret_cast<int32_t*>(d + pb + rb), m->logits.as<float>(), m->ld_v, n,
                        m->cfg.vocab, reinterpret_cast<const pia_sampling*>(d), reinterpret_cast<uint64_t*>(d + pb),
                        mode, m->st());
  PIA_HIP(hipMemcpyAsync(m->pin_out.ptr, d + pb, rb + ob, hipMemcpyDeviceToHost, m->st()));
  PIA_HIP(hipStreamSynchronize(m->st()));
  std::memcpy(rng_state, m->pin_out.ptr, rb);
  std::memcpy(out, static_cast<char*>(m->pin_out.ptr) + rb, ob);
  PIA_API_END
}

}  // extern "C"

