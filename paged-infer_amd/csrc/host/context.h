// Host-side state shared by the C ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "paged_infer_amd.h"
#include "../kernels.h"

namespace pia {

// Grow-only device allocation.
struct DeviceBuffer {
  void* ptr = nullptr;
  size_t bytes = 0;
  DeviceBuffer() = default;
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  DeviceBuffer(DeviceBuffer&& o) noexcept : ptr(o.ptr), bytes(o.bytes) { o.ptr = nullptr, o.bytes = 0; }
  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
      release();
      ptr = o.ptr, bytes = o.bytes;
      o.ptr = nullptr, o.bytes = 0;
    }
    return *this;
  }
  ~DeviceBuffer();
  void ensure(size_t need);
  void release();
  template <typename T>
  T* as() const {
    return static_cast<T*>(ptr);
  }
};

// Grow-only pinned host allocation (hipHostMalloc).
struct PinnedBuffer {
  void* ptr = nullptr;
  size_t bytes = 0;
  PinnedBuffer() = default;
  PinnedBuffer(const PinnedBuffer&) = delete;
  PinnedBuffer& operator=(const PinnedBuffer&) = delete;
  ~PinnedBuffer();
  void ensure(size_t need);
};

}  // namespace pia

struct pia_context {
  int device = 0;
  int num_cus = 0;
  hipStream_t stream = nullptr;
  pia::DeviceBuffer sample_ws;  // sort keys / indices / probabilities of pia_sample_dev
  // Kernel-tier projections on the matrix cores: activation digits, split-K partials + counters.
  pia::DeviceBuffer proj_digits, proj_split;
};

namespace pia {
hipStream_t stream_of(pia_context* ctx, void* stream);
void check_layout(const pia_kv_layout* L);
void quantize_rows_host(const float* w, int64_t rows, int64_t cols, int8_t* q, float* scales);
// Fill projection slot `which` of `layer` from device bf16 rows [rows][cols]: kind 1 quantizes
// them on the device (bit-exact with the host quantizer), kind 0 widens them to f32.
// pia_sample_dev with the context's workspace, on stream st.
void sample_with_context(pia_context* ctx, int32_t* out, const float* logits, int64_t ld, int64_t n, int64_t vocab,
                         const pia_sampling* params, uint64_t* rng_state, int32_t mode, hipStream_t st);
// The kernel tier's int8 projection (matvec / matmat / apply_batched): batches of at least
// kMfmaMinBatch rows whose rows are whole 64-byte k-steps run the matrix-core path (digits in
// the context's workspace, so calls on one context must be ordered), the rest the GEMV.
void launch_projection(pia_context* ctx, const GemvArgs& g, hipStream_t st);
// Whether launch_projection takes the matrix-core path for g.
bool projection_on_matrix_cores(const GemvArgs& g);
// The allocation-free projection's per-device scratch (projection_noalloc.hip): set up once
// per device when a context is created on it.
void noalloc_setup(int device, hipStream_t st);
int64_t noalloc_scratch_bytes();
void model_set_proj_bf16_dev(pia_model* m, int64_t layer, int32_t which, int kind, const uint16_t* src, int64_t rows,
                             int64_t cols);
}  // namespace pia
