// Context, device-memory helpers and the kernel-tier C ABI (src/math.rs, src/attention.rs,
// src/memory/layout.rs seams), plus the synthetic-input helpers.
#include <cmath>
#include <algorithm>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../common.h"
#include "../kernels.h"
#include "context.h"

namespace pia {

namespace {
thread_local std::string g_last_error;
}

void set_last_error(const std::string& msg) { g_last_error = msg; }

hipStream_t stream_of(pia_context* ctx, void* stream) {
  return stream ? static_cast<hipStream_t>(stream) : ctx->stream;
}

DeviceBuffer::~DeviceBuffer() { release(); }

void DeviceBuffer::release() {
  if (ptr) (void)hipFree(ptr);
  ptr = nullptr;
  bytes = 0;
}

void DeviceBuffer::ensure(size_t need) {
  if (need <= bytes) return;
  release();
  PIA_HIP(hipMalloc(&ptr, need));
  bytes = need;
}

PinnedBuffer::~PinnedBuffer() {
  if (ptr) (void)hipHostFree(ptr);
}

void PinnedBuffer::ensure(size_t need) {
  if (need <= bytes) return;
  if (ptr) (void)hipHostFree(ptr);
  ptr = nullptr;
  bytes = 0;
  PIA_HIP(hipHostMalloc(&ptr, need, hipHostMallocDefault));
  bytes = need;
}

void check_layout(const pia_kv_layout* L) {
  PIA_REQUIRE(L != nullptr, "null kv layout");
  PIA_REQUIRE(L->num_layers > 0 && L->num_blocks > 0 && L->block_size > 0 && L->num_kv_heads > 0 && L->head_dim > 0,
              "kv layout dimensions must be positive");
}

namespace {
// Reads a launch's device entries and the block-table range they use back to the host and
// checks them: non-negative fields, and every physical block the kernels will read (logical
// blocks of start..=pos, or of pos alone when `pos_only`) inside the cache. Out-of-range ids
// become an error here instead of an out-of-bounds access on the device.
std::vector<pia_attn_entry> read_checked_entries(const pia_attn_entry* entries, const int32_t* tables, int64_t n,
                                                 const pia_kv_layout& L, bool pos_only, hipStream_t st) {
  std::vector<pia_attn_entry> host(n);
  PIA_HIP(hipMemcpyAsync(host.data(), entries, n * sizeof(pia_attn_entry), hipMemcpyDeviceToHost, st));
  PIA_HIP(hipStreamSynchronize(st));
  int64_t need = 0;
  for (const auto& e : host) {
    PIA_REQUIRE(e.pos >= 0 && e.start >= 0 && e.table_len >= 0 && e.table_off >= 0, "negative entry field");
    const int64_t last = std::min<int64_t>(e.table_len, e.pos / L.block_size + 1);
    if (last > 0) need = std::max<int64_t>(need, e.table_off + last);
  }
  if (need == 0) return host;
  PIA_REQUIRE(tables != nullptr, "null block table");
  std::vector<int32_t> tab(need);
  PIA_HIP(hipMemcpyAsync(tab.data(), tables, need * sizeof(int32_t), hipMemcpyDeviceToHost, st));
  PIA_HIP(hipStreamSynchronize(st));
  for (const auto& e : host) {
    const int64_t last = std::min<int64_t>(e.table_len, e.pos / L.block_size + 1);
    for (int64_t lb = (pos_only ? e.pos : e.start) / L.block_size; lb < last; ++lb) {
      const int32_t id = tab[e.table_off + lb];
      PIA_REQUIRE(id >= 0 && id < L.num_blocks, "block table names a block outside the cache");
    }
  }
  return host;
}
}  // namespace

// quantize_rows_i8 (src/math.rs:456-469) on the host, rows split over threads (each row is
// independent, so the split changes no result).
void quantize_rows_host(const float* w, int64_t rows, int64_t cols, int8_t* q, float* scales) {
  auto body = [&](int64_t r0, int64_t r1) {
    for (int64_t r = r0; r < r1; ++r) {
      const float* row = w + r * cols;
      float max_abs = 0.0f;
      for (int64_t c = 0; c < cols; ++c) max_abs = std::fmax(max_abs, std::fabs(row[c]));
      const float scale = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
      scales[r] = scale;
      int8_t* qr = q + r * cols;
      for (int64_t c = 0; c < cols; ++c) {
        float v = std::roundf(row[c] / scale);
        v = std::fmin(std::fmax(v, -127.0f), 127.0f);
        qr[c] = static_cast<int8_t>(v);
      }
    }
  };
  const int64_t work = rows * cols;
  const unsigned nt = work < (int64_t(1) << 20) ? 1u : std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (nt == 1) {
    body(0, rows);
    return;
  }
  std::vector<std::thread> ts;
  const int64_t per = (rows + nt - 1) / nt;
  for (unsigned t = 0; t < nt; ++t) {
    const int64_t r0 = t * per, r1 = std::min(rows, r0 + per);
    if (r0 < r1) ts.emplace_back(body, r0, r1);
  }
  for (auto& t : ts) t.join();
}

}  // namespace pia

using namespace pia;

namespace pia {
void sample_with_context(pia_context* ctx, int32_t* out, const float* logits, int64_t ld, int64_t n, int64_t vocab,
                         const pia_sampling* params, uint64_t* rng_state, int32_t mode, hipStream_t st) {
  PIA_REQUIRE(n >= 0, "negative row count");
  if (n == 0) return;
  PIA_REQUIRE(out && logits && params && rng_state, "null argument");
  PIA_REQUIRE(mode == PIA_SAMPLE_REFERENCE || mode == PIA_SAMPLE_EXACT_SUMS, "unknown sampling mode");
  size_t ws = 0;
  if (mode == PIA_SAMPLE_REFERENCE) {
    PIA_REQUIRE(vocab > 0 && n * vocab < (int64_t(1) << 31), "sample: rows x vocabulary too large for one sort");
    ws = sample_workspace_bytes(n, vocab);
    if (ctx->sample_ws.bytes < ws) {
      PIA_HIP(hipDeviceSynchronize());  // the old workspace may still be in use by queued work
      ctx->sample_ws.ensure(ws);
    }
  }
  launch_sample(logits, ld, n, vocab, params, rng_state, out, mode, ctx->sample_ws.ptr, ctx->sample_ws.bytes, st);
}
bool projection_on_matrix_cores(const GemvArgs& g) {
  const bool a16 = (reinterpret_cast<uintptr_t>(g.W) & 15) == 0 && (reinterpret_cast<uintptr_t>(g.x) & 15) == 0;
  return g.wkind == 1 && g.batch >= kMfmaMinBatch && g.cols % 64 == 0 && g.ldw % 64 == 0 && g.ldx % 4 == 0 && a16 &&
         g.norm_w == nullptr && g.amax == nullptr && g.scales != nullptr;
}

void launch_projection(pia_context* ctx, const GemvArgs& g, hipStream_t st) {
  if (!projection_on_matrix_cores(g)) {
    launch_gemv(g, st);
    return;
  }
  PIA_REQUIRE(g.rows > 0 && g.rows < (int64_t(1) << 31) && g.batch < (int64_t(1) << 31) && g.cols < (int64_t(1) << 30),
              "projection: shape exceeds int32 indexing");
  const size_t dig = xdigits_bytes(g.batch, g.cols), split = dec_split_bytes();
  if (ctx->proj_digits.bytes < dig || ctx->proj_split.bytes < split) {
    PIA_HIP(hipDeviceSynchronize());  // the old workspace may still be in use by queued work
    ctx->proj_digits.ensure(dig);
    if (ctx->proj_split.bytes < split) {
      ctx->proj_split.ensure(split);
      PIA_HIP(hipMemset(ctx->proj_split.ptr, 0, split));  // every launch leaves the counters zero
    }
  }
  const DecSplitWork sw = dec_split_work(ctx->proj_split.ptr);
  launch_xdigits(g.x, g.ldx, nullptr, 0.0f, g.batch, g.cols, ctx->proj_digits.ptr, st);
  launch_gemm_i8_mfma(static_cast<const int8_t*>(g.W), g.ldw, g.scales, ctx->proj_digits.ptr, g.out, g.osb, g.osr,
                      g.rows, g.cols, g.batch, g.epi, nullptr, &sw, st);
}

}  // namespace pia

extern "C" {

const char* pia_last_error(void) { return g_last_error.c_str(); }
const char* pia_version(void) { return "paged-infer-amd 0.1 (gfx950)"; }

pia_status pia_context_create(int device, pia_context** out) {
  PIA_API_BEGIN
  PIA_REQUIRE(out != nullptr, "null output pointer");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) fail(PIA_ERR_NO_DEVICE, "no HIP device available");
  PIA_REQUIRE(device >= 0 && device < n, "device index out of range");
  PIA_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  PIA_HIP(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    fail(PIA_ERR_NO_DEVICE, std::string("this library is built for gfx950; device is ") + prop.gcnArchName);
  auto* ctx = new pia_context;
  ctx->device = device;
  ctx->num_cus = prop.multiProcessorCount;
  PIA_HIP(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
  try {
    noalloc_setup(device, ctx->stream);
  } catch (...) {
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    throw;
  }
  *out = ctx;
  PIA_API_END
}

pia_status pia_context_destroy(pia_context* ctx) {
  PIA_API_BEGIN
  if (!ctx) return PIA_OK;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  PIA_API_END
}

pia_status pia_context_synchronize(pia_context* ctx) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx, "null context");
  PIA_HIP(hipStreamSynchronize(ctx->stream));
  PIA_API_END
}

void* pia_context_stream(pia_context* ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

pia_status pia_malloc(pia_context* ctx, size_t bytes, void** dptr) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx && dptr, "null argument");
  PIA_HIP(hipSetDevice(ctx->device));
  PIA_HIP(hipMalloc(dptr, bytes ? bytes : 1));
  PIA_API_END
}

pia_status pia_free(pia_context* ctx, void* dptr) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx, "null context");
  if (dptr) PIA_HIP(hipFree(dptr));
  PIA_API_END
}

pia_status pia_memcpy_h2d(pia_context* ctx, void* dst, const void* src, size_t bytes) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx, "null context");
  PIA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  PIA_HIP(hipStreamSynchronize(ctx->stream));
  PIA_API_END
}

pia_status pia_memcpy_d2h(pia_context* ctx, void* dst, const void* src, size_t bytes) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx, "null context");
  PIA_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  PIA_HIP(hipStreamSynchronize(ctx->stream));
  PIA_API_END
}

pia_status pia_quantize_rows_i8(const float* w, int64_t rows, int64_t cols, int8_t* q, float* scales) {
  PIA_API_BEGIN
  PIA_REQUIRE(rows >= 0 && cols >= 0, "negative shape");
  PIA_REQUIRE(rows == 0 || cols == 0 || (w && q && scales), "null argument");
  quantize_rows_host(w, rows, cols, q, scales);
  PIA_API_END
}

pia_status pia_quantize_rows_i8_dev(pia_context* ctx, const float* w, int64_t rows, int64_t cols, int8_t* q,
                                    float* scales, void* stream) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx, "null context");
  PIA_REQUIRE(rows >= 0 && cols >= 0, "negative shape");
  launch_quantize_rows(w, rows, cols, q, scales, stream_of(ctx, stream));
  PIA_API_END
}

uint64_t pia_rng_new(uint64_t seed) { return seed ^ 0x9E3779B97F4A7C15ull; }

pia_status pia_sample_dev(pia_context* ctx, int32_t* out, const float* logits, int64_t ld, int64_t n, int64_t vocab,
                          const pia_sampling* params, uint64_t* rng_state, int32_t mode, void* stream) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx, "null context");
  PIA_HIP(hipSetDevice(ctx->device));
  sample_with_context(ctx, out, logits, ld, n, vocab, params, rng_state, mode, stream_of(ctx, stream));
  PIA_API_END
}

pia_status pia_matvec_i8_dev(pia_context* ctx, float* out, const float* x, const int8_t* w, const float* scales,
                             int64_t rows, int64_t cols, void* stream) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx && out && x && w && scales, "null argument");
  launch_projection(ctx, GemvArgs{1, w, cols, scales, x, cols, nullptr, 0.f, out, 0, 1, rows, cols, 1, Epi::Store},
                    stream_of(ctx, stream));
  PIA_API_END
}

pia_status pia_matmat_i8_dev(pia_context* ctx, float* out_rb, const float* x_br, const int8_t* w,
                             const float* scales, int64_t batch, int64_t rows, int64_t cols, void* stream) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx && out_rb && x_br && w && scales, "null argument");
  launch_projection(ctx, GemvArgs{1, w, cols, scales, x_br, cols, nullptr, 0.f, out_rb, 1, batch, rows, cols, batch,
                                  Epi::Store},
                    stream_of(ctx, stream));
  PIA_API_END
}

pia_status pia_qlinear_apply_dev(pia_context* ctx, float* out_br, const float* x_br, const int8_t* w,
                                 const float* scales, int64_t batch, int64_t rows, int64_t cols, void* stream) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx && out_br && x_br && w && scales, "null argument");
  launch_projection(ctx, GemvArgs{1, w, cols, scales, x_br, cols, nullptr, 0.f, out_br, rows, 1, rows, cols, batch,
                                  Epi::Store},
                    stream_of(ctx, stream));
  PIA_API_END
}

pia_status pia_matvec_i8(pia_context* ctx, float* out, const float* x, const int8_t* w, const float* scales,
                         int64_t rows, int64_t cols) {
  return pia_matmat_i8(ctx, out, x, w, scales, 1, rows, cols);
}

namespace {
// Host-pointer projection: stage w, scales and x on the device, run the int8 GEMV with the
// given output strides (batch stride osb, row stride osr), copy the result back, synchronize.
pia_status host_projection(pia_context* ctx, float* out, const float* x_br, const int8_t* w, const float* scales,
                           int64_t batch, int64_t rows, int64_t cols, int64_t osb, int64_t osr) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx && out && x_br && w && scales, "null argument");
  PIA_REQUIRE(rows > 0 && cols > 0 && batch > 0, "empty shape");
  PIA_HIP(hipSetDevice(ctx->device));
  DeviceBuffer dw, ds, dx, dout;
  dw.ensure(rows * cols);
  ds.ensure(rows * sizeof(float));
  dx.ensure(batch * cols * sizeof(float));
  dout.ensure(batch * rows * sizeof(float));
  hipStream_t st = ctx->stream;
  PIA_HIP(hipMemcpyAsync(dw.ptr, w, rows * cols, hipMemcpyHostToDevice, st));
  PIA_HIP(hipMemcpyAsync(ds.ptr, scales, rows * sizeof(float), hipMemcpyHostToDevice, st));
  PIA_HIP(hipMemcpyAsync(dx.ptr, x_br, batch * cols * sizeof(float), hipMemcpyHostToDevice, st));
  launch_projection(ctx,
                    GemvArgs{1, dw.ptr, cols, static_cast<const float*>(ds.ptr), static_cast<const float*>(dx.ptr),
                             cols, nullptr, 0.f, static_cast<float*>(dout.ptr), osb, osr, rows, cols, batch, Epi::Store},
                    st);
  PIA_HIP(hipMemcpyAsync(out, dout.ptr, batch * rows * sizeof(float), hipMemcpyDeviceToHost, st));
  PIA_HIP(hipStreamSynchronize(st));
  PIA_API_END
}
}  // namespace

pia_status pia_matmat_i8(pia_context* ctx, float* out_rb, const float* x_br, const int8_t* w, const float* scales,
                         int64_t batch, int64_t rows, int64_t cols) {
  return host_projection(ctx, out_rb, x_br, w, scales, batch, rows, cols, 1, batch);
}

pia_status pia_qlinear_apply(pia_context* ctx, float* out_br, const float* x_br, const int8_t* w,
                             const float* scales, int64_t batch, int64_t rows, int64_t cols) {
  return host_projection(ctx, out_br, x_br, w, scales, batch, rows, cols, rows, 1);
}

pia_status pia_paged_attention_dev(pia_context* ctx, float* out, const float* q, const float* kv,
                                   const pia_kv_layout* layout, int64_t num_heads, const pia_attn_entry* entries,
                                   const int32_t* tables, int64_t n, int64_t layer, void* stream) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx, "null context");
  check_layout(layout);
  PIA_REQUIRE(n >= 0, "negative entry count");
  if (n == 0) return PIA_OK;
  PIA_REQUIRE(out && q && kv && entries, "null argument");
  // Entries live on the device; the split count must cover the widest window. Read them (and
  // the block ids they use) back once, to size the split and validate the ids.
  hipStream_t st = stream_of(ctx, stream);
  const std::vector<pia_attn_entry> host = read_checked_entries(entries, tables, n, *layout, false, st);
  int64_t widest = 1;
  for (const auto& e : host) widest = std::max<int64_t>(widest, e.pos + 1 - e.start);
  const int64_t hd = layout->head_dim;
  const AttnPlan plan = plan_attention(n, layout->num_kv_heads, hd, widest, ctx->num_cus);
  DeviceBuffer work;
  const int64_t wb = attention_work_bytes(n, num_heads, hd, plan.splits);
  if (wb) work.ensure(wb);
  AttnLaunch a{q, num_heads * hd, out, num_heads * hd, const_cast<float*>(kv), layout, num_heads, entries, tables,
               n, layer, plan, work.ptr, false, nullptr, nullptr};
  launch_attention(a, st);
  PIA_HIP(hipStreamSynchronize(st));
  PIA_API_END
}

pia_status pia_kv_write_dev(pia_context* ctx, float* kv, const pia_kv_layout* layout, const float* k, const float* v,
                           const pia_attn_entry* entries, const int32_t* tables, int64_t n, int64_t layer,
                           void* stream) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx, "null context");
  check_layout(layout);
  PIA_REQUIRE(n >= 0, "negative entry count");
  PIA_REQUIRE(layer >= 0 && layer < layout->num_layers, "kv_write: layer out of range");
  if (n == 0) return PIA_OK;
  PIA_REQUIRE(kv && k && v && entries, "null argument");
  hipStream_t st = stream_of(ctx, stream);
  (void)read_checked_entries(entries, tables, n, *layout, true, st);
  launch_kv_write(k, v, entries, tables, kv, *layout, n, layer, st);
  PIA_API_END
}

pia_status pia_kv_copy_block_dev(pia_context* ctx, float* kv, const pia_kv_layout* layout, int64_t src, int64_t dst,
                                 void* stream) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx && kv, "null argument");
  check_layout(layout);
  launch_copy_block(kv, *layout, src, dst, stream_of(ctx, stream));
  PIA_API_END
}

pia_status pia_argmax_dev(pia_context* ctx, int32_t* out, const float* logits, int64_t n, int64_t vocab, void* stream) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx && out && logits, "null argument");
  PIA_REQUIRE(vocab > 0, "empty vocabulary");
  launch_argmax(logits, vocab, out, n, vocab, stream_of(ctx, stream));
  PIA_API_END
}

pia_status pia_bench_projection(pia_context* ctx, int64_t rows, int64_t cols, int64_t batch, int32_t reps,
                                int32_t flags, double* us, int64_t* bytes) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx && us && bytes, "null argument");
  PIA_REQUIRE(rows > 0 && cols > 0 && batch > 0 && reps > 0 && reps <= 1000, "bad benchmark shape");
  PIA_HIP(hipSetDevice(ctx->device));
  PIA_REQUIRE(!(flags & 2) || rows % 2 == 0, "SwiGLU needs an even row count");
  const int64_t ldw = (cols + 63) / 64 * 64, ldx = (cols + 15) / 16 * 16;
  // Enough distinct weight copies (>= 1 GiB in total) that consecutive launches stream from
  // HBM instead of hitting the 256 MB Infinity Cache.
  const int64_t wbytes = rows * ldw;
  const int ncopy = static_cast<int>(std::min<int64_t>(64, std::max<int64_t>(2, ((int64_t(1) << 30) + wbytes - 1) / wbytes)));
  DeviceBuffer w, s, x, y, nw, xq;
  w.ensure(wbytes * ncopy);
  s.ensure(rows * 4);
  x.ensure(batch * ldx * 4);
  y.ensure(batch * rows * 4);
  nw.ensure(ldx * 4);
  xq.ensure(xdigits_bytes(batch, cols));
  DeviceBuffer split_buf;
  split_buf.ensure(dec_split_bytes());
  PIA_HIP(hipMemset(split_buf.ptr, 0, dec_split_bytes()));
  const DecSplitWork split = dec_split_work(split_buf.ptr);
  {
    std::vector<int8_t> hw(wbytes);
    for (size_t i = 0; i < hw.size(); ++i) hw[i] = static_cast<int8_t>((i * 2654435761u >> 13) % 255 - 127);
    for (int c = 0; c < ncopy; ++c)
      PIA_HIP(hipMemcpy(static_cast<int8_t*>(w.ptr) + c * wbytes, hw.data(), hw.size(), hipMemcpyHostToDevice));
    std::vector<float> hs(rows, 0.01f), hx(batch * ldx);
    for (size_t i = 0; i < hx.size(); ++i) hx[i] = static_cast<float>((i * 40503u) % 2001) / 1000.0f - 1.0f;
    PIA_HIP(hipMemcpy(s.ptr, hs.data(), hs.size() * 4, hipMemcpyHostToDevice));
    PIA_HIP(hipMemcpy(x.ptr, hx.data(), hx.size() * 4, hipMemcpyHostToDevice));
    std::vector<float> hn(ldx, 1.0f);
    PIA_HIP(hipMemcpy(nw.ptr, hn.data(), hn.size() * 4, hipMemcpyHostToDevice));
  }
  const Epi epi = (flags & 2) ? Epi::Swiglu : (flags & 4) ? Epi::Add : Epi::Store;
  const float* norm = (flags & 1) ? nw.as<float>() : nullptr;
  hipStream_t st = ctx->stream;
  auto one = [&](int i) {
    const int8_t* wi = static_cast<int8_t*>(w.ptr) + (i % ncopy) * wbytes;
    if (flags & 8) {
      // flags & 16: the digits are written once before the timed launches (projection alone).
      if (!(flags & 16) || i == 0) launch_xdigits(x.as<float>(), ldx, norm, 1e-5f, batch, cols, xq.ptr, st);
      launch_gemm_i8_mfma(wi, ldw, s.as<float>(), xq.ptr, y.as<float>(), rows, 1, rows, cols, batch, epi, nullptr,
                          &split, st);
    } else {
      launch_gemv(GemvArgs{1, wi, ldw, s.as<float>(), x.as<float>(), ldx, norm, 1e-5f, y.as<float>(), rows, 1, rows,
                           cols, batch, epi},
                  st);
    }
  };
  one(0);
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  PIA_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
  for (int i = 0; i < reps; ++i) one(i + 1);
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
  *us = 1e3 * ms / reps;
  *bytes = rows * cols + 4 * rows + 4 * batch * cols + 4 * batch * rows;
  PIA_API_END
}

// SplitMix64 stream -> Box-Muller in f64 -> f32. Deterministic for (seed, stream, index).
pia_status pia_synth_normal(uint64_t seed, uint64_t stream, float std_dev, float* out, int64_t n) {
  PIA_API_BEGIN
  PIA_REQUIRE(n >= 0 && (n == 0 || out), "bad output");
  auto body = [=](int64_t i0, int64_t i1) {
    auto mix = [](uint64_t z) {
      z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
      z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
      return z ^ (z >> 31);
    };
    const uint64_t key = mix(seed ^ mix(stream + 0x9E3779B97F4A7C15ull));
    for (int64_t i = i0 & ~int64_t(1); i < i1; i += 2) {
      const uint64_t pair = static_cast<uint64_t>(i) >> 1;
      const uint64_t a = mix(key + 2 * pair * 0x9E3779B97F4A7C15ull);
      const uint64_t b = mix(key + (2 * pair + 1) * 0x9E3779B97F4A7C15ull);
      const double u1 = (static_cast<double>(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);
      const double u2 = static_cast<double>(b >> 11) * (1.0 / 9007199254740992.0);
      const double r = std::sqrt(-2.0 * std::log(u1));
      const double t = 6.283185307179586 * u2;
      if (i >= i0 && i < i1) out[i] = static_cast<float>(r * std::cos(t) * std_dev);
      if (i + 1 >= i0 && i + 1 < i1) out[i + 1] = static_cast<float>(r * std::sin(t) * std_dev);
    }
  };
  const unsigned nt = n < (int64_t(1) << 20) ? 1u : std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (nt == 1) {
    body(0, n);
  } else {
    std::vector<std::thread> ts;
    const int64_t per = ((n + nt - 1) / nt + 1) & ~int64_t(1);
    for (unsigned t = 0; t < nt; ++t) {
      const int64_t i0 = t * per, i1 = std::min(n, i0 + per);
      if (i0 < i1) ts.emplace_back(body, i0, i1);
    }
    for (auto& t : ts) t.join();
  }
  PIA_API_END
}

pia_status pia_f32_to_bf16(const float* in, uint16_t* out, int64_t n) {
  PIA_API_BEGIN
  PIA_REQUIRE(n >= 0 && (n == 0 || (in && out)), "bad argument");
  for (int64_t i = 0; i < n; ++i) {
    uint32_t u;
    std::memcpy(&u, &in[i], 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
      out[i] = static_cast<uint16_t>((u >> 16) | 0x40);  // quiet NaN
    } else {
      const uint32_t rounding = 0x7fffu + ((u >> 16) & 1u);
      out[i] = static_cast<uint16_t>((u + rounding) >> 16);
    }
  }
  PIA_API_END
}

}  // extern "C"
