// Weight-streaming projection for decode batches (batch 1..15): one wavefront owns R output
// rows; each lane streams VEC contiguous weight elements per step (16 int8 = one 128-bit
// load), widens them in registers and accumulates in f32 against the activation vectors of
// up to NB batch entries, so every weight byte is fetched from HBM once per launch. The
// per-row scale is applied after the wavefront reduction, as the reference does
// (src/math.rs:486-492: dot_i8(row, x) * scale).
#include "common.h"
#include "kernels.h"

namespace pia {
namespace {

template <typename TW, int VEC>
__device__ inline void load_w(const TW* p, float (&w)[VEC]);

template <>
__device__ inline void load_w<int8_t, 16>(const int8_t* p, float (&w)[16]) {
  const int4 v = *reinterpret_cast<const int4*>(p);
  const int d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) w[4 * k + j] = static_cast<float>((d[k] << (24 - 8 * j)) >> 24);
}
template <>
__device__ inline void load_w<int8_t, 8>(const int8_t* p, float (&w)[8]) {
  const int2 v = *reinterpret_cast<const int2*>(p);
  const int d[2] = {v.x, v.y};
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) w[4 * k + j] = static_cast<float>((d[k] << (24 - 8 * j)) >> 24);
}
template <>
__device__ inline void load_w<int8_t, 4>(const int8_t* p, float (&w)[4]) {
  const int d = *reinterpret_cast<const int*>(p);
#pragma unroll
  for (int j = 0; j < 4; ++j) w[j] = static_cast<float>((d << (24 - 8 * j)) >> 24);
}
template <>
__device__ inline void load_w<int8_t, 1>(const int8_t* p, float (&w)[1]) {
  w[0] = static_cast<float>(*p);
}
template <>
__device__ inline void load_w<float, 4>(const float* p, float (&w)[4]) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  w[0] = v.x, w[1] = v.y, w[2] = v.z, w[3] = v.w;
}
template <>
__device__ inline void load_w<float, 1>(const float* p, float (&w)[1]) {
  w[0] = *p;
}

template <int VEC>
__device__ inline void load_x(const float* p, float (&x)[VEC]) {
  if constexpr (VEC % 4 == 0) {
#pragma unroll
    for (int k = 0; k < VEC / 4; ++k) {
      const float4 v = reinterpret_cast<const float4*>(p)[k];
      x[4 * k] = v.x, x[4 * k + 1] = v.y, x[4 * k + 2] = v.z, x[4 * k + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int k = 0; k < VEC; ++k) x[k] = p[k];
  }
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

constexpr int kWaves = 4;  // wavefronts per workgroup

template <typename TW, int VEC, int R, int NB, int EPI>
__global__ __launch_bounds__(64 * kWaves) void k_gemv(const TW* __restrict__ W, int64_t ldw,
                                                      const float* __restrict__ S, const float* __restrict__ X,
                                                      int64_t ldx, float* __restrict__ O, int64_t osb, int64_t osr,
                                                      int rows, int cols, int batch) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * R;
  if (row0 >= rows) return;

  const TW* wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) wrow[r] = W + static_cast<int64_t>(min(row0 + r, rows - 1)) * ldw;
  const int main_cols = cols - cols % VEC;
  const int rem = cols - main_cols;

  // Batch groups run back to back over the same R weight rows: the first group streams them
  // from HBM, later groups hit in cache.
  for (int b0 = 0; b0 < batch; b0 += NB) {
    float acc[R][NB];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[r][b] = 0.0f;

    for (int c = lane * VEC; c < main_cols; c += 64 * VEC) {
      float w[R][VEC];
#pragma unroll
      for (int r = 0; r < R; ++r) load_w<TW, VEC>(wrow[r] + c, w[r]);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b0 + b < batch) {
          float xv[VEC];
          load_x<VEC>(X + static_cast<int64_t>(b0 + b) * ldx + c, xv);
#pragma unroll
          for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < VEC; ++j) acc[r][b] = __builtin_fmaf(w[r][j], xv[j], acc[r][b]);
        }
      }
    }
    if (lane < rem) {
      const int c = main_cols + lane;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float w = static_cast<float>(wrow[r][c]);
#pragma unroll
        for (int b = 0; b < NB; ++b)
          if (b0 + b < batch) acc[r][b] = __builtin_fmaf(w, X[static_cast<int64_t>(b0 + b) * ldx + c], acc[r][b]);
      }
    }

    float mine = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float s = wave_sum(acc[r][b]);
        if (lane == r * NB + b) mine = s;
      }
    if (lane < R * NB) {
      const int r = lane / NB, b = lane % NB;
      const int row = row0 + r, bb = b0 + b;
      if (row < rows && bb < batch) {
        const float v = S ? mine * S[row] : mine;
        float* o = O + static_cast<int64_t>(bb) * osb + static_cast<int64_t>(row) * osr;
        if (EPI == 1) *o = *o + v;
        else *o = v;
      }
    }
  }
}

template <typename TW, int VEC, int R, int NB>
void dispatch_epi(const TW* W, int64_t ldw, const float* S, const float* X, int64_t ldx, float* O, int64_t osb,
                  int64_t osr, int rows, int cols, int batch, Epi epi, hipStream_t st) {
  dim3 grid((rows + kWaves * R - 1) / (kWaves * R));
  if (epi == Epi::Add)
    hipLaunchKernelGGL((k_gemv<TW, VEC, R, NB, 1>), grid, dim3(64 * kWaves), 0, st, W, ldw, S, X, ldx, O, osb, osr,
                       rows, cols, batch);
  else
    hipLaunchKernelGGL((k_gemv<TW, VEC, R, NB, 0>), grid, dim3(64 * kWaves), 0, st, W, ldw, S, X, ldx, O, osb, osr,
                       rows, cols, batch);
}

template <typename TW, int VEC, int R>
void dispatch_nb(const TW* W, int64_t ldw, const float* S, const float* X, int64_t ldx, float* O, int64_t osb,
                 int64_t osr, int rows, int cols, int batch, Epi epi, hipStream_t st) {
  if (batch == 1) dispatch_epi<TW, VEC, R, 1>(W, ldw, S, X, ldx, O, osb, osr, rows, cols, batch, epi, st);
  else if (batch == 2) dispatch_epi<TW, VEC, R, 2>(W, ldw, S, X, ldx, O, osb, osr, rows, cols, batch, epi, st);
  else if (batch <= 4) dispatch_epi<TW, VEC, R, 4>(W, ldw, S, X, ldx, O, osb, osr, rows, cols, batch, epi, st);
  else dispatch_epi<TW, VEC, R, 8>(W, ldw, S, X, ldx, O, osb, osr, rows, cols, batch, epi, st);
}

template <typename TW, int VEC>
void dispatch_r(const TW* W, int64_t ldw, const float* S, const float* X, int64_t ldx, float* O, int64_t osb,
                int64_t osr, int rows, int cols, int batch, Epi epi, hipStream_t st) {
  // Prefer 4 rows per wavefront (more bytes in flight per lane); fall back to fewer rows
  // when that would leave most of the 256 CUs idle.
  if (rows >= 4 * kWaves * 512) dispatch_nb<TW, VEC, 4>(W, ldw, S, X, ldx, O, osb, osr, rows, cols, batch, epi, st);
  else if (rows >= 2 * kWaves * 256) dispatch_nb<TW, VEC, 2>(W, ldw, S, X, ldx, O, osb, osr, rows, cols, batch, epi, st);
  else dispatch_nb<TW, VEC, 1>(W, ldw, S, X, ldx, O, osb, osr, rows, cols, batch, epi, st);
}

inline bool aligned(const void* p, int64_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace

void launch_gemv(int wkind, const void* W, int64_t ldw, const float* scales, const float* x, int64_t ldx, float* out,
                 int64_t osb, int64_t osr, int64_t rows, int64_t cols, int64_t batch, Epi epi, hipStream_t st) {
  PIA_REQUIRE(rows > 0 && cols > 0 && batch > 0, "gemv: empty shape");
  PIA_REQUIRE(rows < (int64_t(1) << 31) && cols < (int64_t(1) << 31) && batch < (int64_t(1) << 31),
              "gemv: shape exceeds int32 indexing");
  PIA_REQUIRE(ldw >= cols && ldx >= cols, "gemv: leading dimension smaller than cols");
  const int r = static_cast<int>(rows), c = static_cast<int>(cols), b = static_cast<int>(batch);
  if (wkind == 1) {
    PIA_REQUIRE(scales != nullptr, "gemv: int8 weights need scales");
    const auto* w = static_cast<const int8_t*>(W);
    if (ldw % 16 == 0 && ldx % 16 == 0 && aligned(w, 16) && aligned(x, 64))
      dispatch_r<int8_t, 16>(w, ldw, scales, x, ldx, out, osb, osr, r, c, b, epi, st);
    else if (ldw % 4 == 0 && ldx % 4 == 0 && aligned(w, 4) && aligned(x, 16))
      dispatch_r<int8_t, 4>(w, ldw, scales, x, ldx, out, osb, osr, r, c, b, epi, st);
    else
      dispatch_r<int8_t, 1>(w, ldw, scales, x, ldx, out, osb, osr, r, c, b, epi, st);
  } else {
    const auto* w = static_cast<const float*>(W);
    if (ldw % 4 == 0 && ldx % 4 == 0 && aligned(w, 16) && aligned(x, 16))
      dispatch_r<float, 4>(w, ldw, scales, x, ldx, out, osb, osr, r, c, b, epi, st);
    else
      dispatch_r<float, 1>(w, ldw, scales, x, ldx, out, osb, osr, r, c, b, epi, st);
  }
  PIA_HIP(hipGetLastError());
}

}  // namespace pia
