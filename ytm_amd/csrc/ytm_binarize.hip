// ytm_binarize.hip -- gfx950 kernels of the host-preprocessing binarizers that produce the
// Tsetlin Machine's boolean inputs (src/tm_utils/binarizer.py): thermometer and one-hot
// binning of every input value against a threshold list, and the collapse of binned rows
// back to bin indices.
//
// Element i of the input becomes `width` uint32 outputs [i * width, (i + 1) * width): one
// thread per output value, so the writes (the dominant HBM traffic, width * 4 bytes per
// input value) are coalesced and each input value is read from the cache width times.
// Comparisons use the type numpy promotes the operands to: double, or int64 when both the
// data and the thresholds are integers.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ytm_internal.h"

namespace ytm {

namespace {

constexpr int kBinBlock = 256;

template <typename T, typename C>
__device__ __forceinline__ C as_cmp(T v) {
  return (C)v;
}

// Thermometer (binarizer.py:63-73 and the ThermometerBinarizer of :5-22): output j of
// element i is X[i] >= t[j], j < nthr.
// One-hot (binarizer.py:75-86): output j of element i is t[j] <= X[i] < t[j + 1], j < nthr-1;
// with edge bins the outputs are [X[i] < t[0], those nthr - 1, X[i] >= t[nthr - 1]].
template <typename T, typename C, bool ONEHOT>
__global__ __launch_bounds__(kBinBlock) void binarize_kernel(const T* __restrict__ X, int64_t n,
                                                             const C* __restrict__ t, int nthr, int edge,
                                                             uint32_t* __restrict__ out) {
  const int width = ONEHOT ? nthr - 1 + (edge ? 2 : 0) : nthr;
  const int64_t total = n * width;
  for (int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; o < total;
       o += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = o / width;
    const int j = (int)(o - i * width);
    const C v = as_cmp<T, C>(X[i]);
    bool r;
    if (!ONEHOT) {
      r = v >= t[j];
    } else if (edge && j == 0) {
      r = v < t[0];
    } else if (edge && j == width - 1) {
      r = v >= t[nthr - 1];
    } else {
      const int b = edge ? j - 1 : j;
      r = v >= t[b] && v < t[b + 1];
    }
    out[o] = r ? 1u : 0u;
  }
}

// Collapse of binned rows (binarizer.py:88-105): thermometer -> index of the last non-zero
// value + 1 (0 for none); one-hot -> index of the first maximum (np.argmax); minus 1 with
// edge bins.  One thread per row.
template <bool ONEHOT>
__global__ __launch_bounds__(kBinBlock) void collapse_kernel(const uint32_t* __restrict__ B, int64_t rows,
                                                             int64_t width, int edge, int64_t* __restrict__ out) {
  for (int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; r < rows; r += (int64_t)gridDim.x * blockDim.x) {
    const uint32_t* row = B + r * width;
    int64_t v = 0;
    if (!ONEHOT) {
      for (int64_t j = width - 1; j >= 0; --j)
        if (row[j] != 0u) {
          v = j + 1;
          break;
        }
    } else {
      uint32_t best = width > 0 ? row[0] : 0u;
      for (int64_t j = 1; j < width; ++j)
        if (row[j] > best) {
          best = row[j];
          v = j;
        }
    }
    out[r] = edge ? v - 1 : v;
  }
}

int grid_of(int64_t items) {
  int64_t g = (items + kBinBlock - 1) / kBinBlock;
  return (int)(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

template <typename C, bool ONEHOT>
hipError_t launch_typed(const void* X, int dtype, int64_t n, const C* t, int nthr, int edge, uint32_t* out,
                        hipStream_t s) {
  const int width = ONEHOT ? nthr - 1 + (edge ? 2 : 0) : nthr;
  const int grid = grid_of(n * width);
#define YTM_BIN_CASE(code, T)                                                                         \
  case code:                                                                                          \
    binarize_kernel<T, C, ONEHOT><<<grid, kBinBlock, 0, s>>>((const T*)X, n, t, nthr, edge, out);    \
    break;
  switch (dtype) {
    YTM_BIN_CASE(YTM_DTYPE_U8, uint8_t)
    YTM_BIN_CASE(YTM_DTYPE_I8, int8_t)
    YTM_BIN_CASE(YTM_DTYPE_U16, uint16_t)
    YTM_BIN_CASE(YTM_DTYPE_I16, int16_t)
    YTM_BIN_CASE(YTM_DTYPE_U32, uint32_t)
    YTM_BIN_CASE(YTM_DTYPE_I32, int32_t)
    YTM_BIN_CASE(YTM_DTYPE_I64, int64_t)
    YTM_BIN_CASE(YTM_DTYPE_F32, float)
    YTM_BIN_CASE(YTM_DTYPE_F64, double)
    default:
      return hipErrorInvalidValue;
  }
#undef YTM_BIN_CASE
  return hipGetLastError();
}

}  // namespace

hipError_t launch_binarize(const void* X, int dtype, int64_t n, const void* t, bool int_thresholds, int nthr,
                           bool onehot, int edge, uint32_t* out, hipStream_t s) {
  if (int_thresholds)
    return onehot ? launch_typed<int64_t, true>(X, dtype, n, (const int64_t*)t, nthr, edge, out, s)
                  : launch_typed<int64_t, false>(X, dtype, n, (const int64_t*)t, nthr, edge, out, s);
  return onehot ? launch_typed<double, true>(X, dtype, n, (const double*)t, nthr, edge, out, s)
                : launch_typed<double, false>(X, dtype, n, (const double*)t, nthr, edge, out, s);
}

hipError_t launch_collapse_bins(const uint32_t* B, int64_t rows, int64_t width, bool onehot, int edge, int64_t* out,
                                hipStream_t s) {
  if (onehot)
    collapse_kernel<true><<<grid_of(rows), kBinBlock, 0, s>>>(B, rows, width, edge, out);
  else
    collapse_kernel<false><<<grid_of(rows), kBinBlock, 0, s>>>(B, rows, width, edge, out);
  return hipGetLastError();
}

}  // namespace ytm
