// Allocation-free form of the kernel tier's int8 projection (Projection::apply_batched for
// Int8, src/model.rs:247-259), for callers that cannot allocate device memory: code recorded
// into a graph, tight serving loops, harnesses that forbid hipMalloc.
//
// The matrix-core path needs scratch memory beyond the inputs and outputs: the activation
// digits (three 8-bit digits of a 23-bit fixed-point image per row) and the split-K partial
// sums with their per-tile counters. Here they live in one file-scope device array, `scratch`,
// of fixed size; each GPU the library runs on holds its own copy until the process ends. Its
// device address is taken once per device, with that device current, when a context is created
// on it (hipGetSymbolAddress), and only that address is handed to kernels: in host code the
// array's name is a host-side stand-in, not a device address.
//
// Every call on one GPU shares that GPU's scratch: calls that overlap (different streams, or
// different contexts on one device, without ordering) race. The split-K counters start at
// zero and every launch leaves them at zero; the digits are rewritten by every call.
#include <mutex>

#include "common.h"
#include "kernels.h"
#include "host/context.h"

namespace pia {
namespace {

constexpr int64_t kNaMaxBatch = 64;     // batch rows per call
constexpr int64_t kNaMaxCols = 16384;   // input columns
constexpr int64_t kNaSplitPairs = 64;   // split-K (row tile, K slice) pairs
constexpr size_t kNaDigitBytes = (48 * 4 * kNaMaxCols + 255) / 256 * 256 + 4 * 64 * 4;  // 64 rows: 4 groups
constexpr size_t kNaSplitOff = (kNaDigitBytes + 255) / 256 * 256;
constexpr size_t kNaBytes = kNaSplitOff + kNaSplitPairs * 128 * 64 * 8 + kNaSplitPairs * 4;

__device__ __align__(256) unsigned char scratch[kNaBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};

__global__ void k_zero_u32(unsigned* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}

}  // namespace

int64_t noalloc_scratch_bytes() { return static_cast<int64_t>(kNaBytes); }

void noalloc_setup(int device, hipStream_t st) {
  std::lock_guard<std::mutex> lk(g_mu);
  PIA_REQUIRE(device >= 0 && device < kMaxDevices, "device index out of range");
  if (g_scratch[device]) return;
  PIA_HIP(hipSetDevice(device));
  void* p = nullptr;
  PIA_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  PIA_REQUIRE(p != nullptr, "no device address for the projection scratch");
  const DecSplitWork sw = dec_split_work(static_cast<char*>(p) + kNaSplitOff, kNaSplitPairs);
  hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(256), 0, st, sw.cnt, static_cast<int>(kNaSplitPairs));
  PIA_HIP(hipGetLastError());
  PIA_HIP(hipStreamSynchronize(st));
  g_scratch[device] = p;
}

namespace {
void* scratch_of(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  PIA_REQUIRE(device >= 0 && device < kMaxDevices && g_scratch[device],
              "projection scratch not set up on this device (create the context first)");
  return g_scratch[device];
}
}  // namespace
}  // namespace pia

using namespace pia;

extern "C" pia_status pia_qlinear_apply_noalloc_dev(pia_context* ctx, float* out_br, const float* x_br,
                                                    const int8_t* w, const float* scales, int64_t batch, int64_t rows,
                                                    int64_t cols, void* stream) {
  PIA_API_BEGIN
  PIA_REQUIRE(ctx && out_br && x_br && w && scales, "null argument");
  PIA_REQUIRE(batch > 0 && rows > 0 && cols > 0, "empty shape");
  PIA_REQUIRE(batch <= kNaMaxBatch && cols <= kNaMaxCols,
              "qlinear_apply_noalloc: at most 64 batch rows and 16384 columns (fixed scratch)");
  PIA_REQUIRE(rows < (int64_t(1) << 31), "qlinear_apply_noalloc: too many rows");
  hipStream_t st = stream_of(ctx, stream);
  const GemvArgs g{1, w, cols, scales, x_br, cols, nullptr, 0.f, out_br, rows, 1, rows, cols, batch, Epi::Store};
  if (!projection_on_matrix_cores(g)) {
    launch_gemv(g, st);  // the streaming GEMV uses no scratch
    return PIA_OK;
  }
  char* base = static_cast<char*>(scratch_of(ctx->device));
  PIA_REQUIRE(xdigits_bytes(batch, cols) <= static_cast<int64_t>(kNaDigitBytes), "qlinear_apply_noalloc: digit scratch");
  const DecSplitWork sw = dec_split_work(base + kNaSplitOff, kNaSplitPairs);
  launch_xdigits(x_br, cols, nullptr, 0.0f, batch, cols, base, st);
  launch_gemm_i8_mfma(w, cols, scales, base, out_br, rows, 1, rows, cols, batch, Epi::Store, nullptr, &sw, st);
  PIA_API_END
}
