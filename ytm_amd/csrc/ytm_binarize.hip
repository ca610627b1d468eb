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
//
// The encode fused with the binning (encode_binned_kernel) takes the raw values instead of
// the binned uint32 array and bins each value where encode reads it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ytm_encode.h"
#include "ytm_internal.h"

namespace ytm {

namespace {

constexpr int kBinBlock = 256;

template <typename T, typename C>
__device__ __forceinline__ C as_cmp(T v) {
  return (C)v;
}

// Level j of value v (width levels, nthr thresholds t).
// Thermometer (binarizer.py:63-73 and the ThermometerBinarizer of :5-22): v >= t[j], j < nthr.
// One-hot (binarizer.py:75-86): t[j] <= v < t[j + 1], j < nthr - 1; with edge bins the levels
// are [v < t[0], those nthr - 1, v >= t[nthr - 1]].
template <typename C, bool ONEHOT>
__device__ __forceinline__ bool bin_level(C v, const C* __restrict__ t, int nthr, int edge, int width, int j) {
  if (!ONEHOT) return v >= t[j];
  if (edge && j == 0) return v < t[0];
  if (edge && j == width - 1) return v >= t[nthr - 1];
  const int b = edge ? j - 1 : j;
  return v >= t[b] && v < t[b + 1];
}

// Output o of the binning: level o % width of element o / width.
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
    out[o] = bin_level<C, ONEHOT>(as_cmp<T, C>(X[i]), t, nthr, edge, width, j) ? 1u : 0u;
  }
}

// Pixel values of the fused encode: binned value f of a sample is level f % width of its raw
// value f / width, the layout of the binarizers' outputs (the levels of a value last, so that
// binarize_rgb's channel-major c * ch + j is level j of channel c).
template <typename T, typename C, bool ONEHOT>
struct BinnedPixels {
  const T* X;
  int64_t Fr;  // raw values per sample
  const C* t;
  int nthr, edge, width;
  __device__ __forceinline__ bool operator()(int64_t e, int64_t f) const {
    const int64_t i = f / width;
    const int j = (int)(f - i * width);
    return bin_level<C, ONEHOT>(as_cmp<T, C>(X[e * Fr + i]), t, nthr, edge, width, j);
  }
  // the same for f < 2^31, in 32-bit arithmetic (encode_staged)
  __device__ __forceinline__ bool bit32(int64_t e, int f) const {
    const int i = (int)((unsigned)f / (unsigned)width);
    const int j = f - i * width;
    return bin_level<C, ONEHOT>(as_cmp<T, C>(X[e * Fr + i]), t, nthr, edge, width, j);
  }
};

// encode of the binned raw values of N samples (encode_words, ytm_encode.h): the same words
// as binning them (binarize_kernel) and encoding the result.
template <typename T, typename C, bool ONEHOT>
__global__ __launch_bounds__(256) void encode_binned_kernel(const T* __restrict__ X, int64_t N, int64_t Fr,
                                                            const C* __restrict__ t, int nthr, int edge,
                                                            uint32_t* __restrict__ out, Geom g) {
  const int width = ONEHOT ? nthr - 1 + (edge ? 2 : 0) : nthr;
  encode_words(BinnedPixels<T, C, ONEHOT>{X, Fr, t, nthr, edge, width}, N, out, g);
}

// Several patches: a block per sample, its binned pixel bits staged in LDS (encode_staged).
template <typename T, typename C, bool ONEHOT>
__global__ __launch_bounds__(256) void encode_binned_staged_kernel(const T* __restrict__ X, int64_t N, int64_t Fr,
                                                                   const C* __restrict__ t, int nthr, int edge,
                                                                   uint32_t* __restrict__ out, Geom g) {
  const int width = ONEHOT ? nthr - 1 + (edge ? 2 : 0) : nthr;
  encode_staged(BinnedPixels<T, C, ONEHOT>{X, Fr, t, nthr, edge, width}, N, out, g);
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

template <typename C, bool ONEHOT>
hipError_t launch_encode_typed(const void* X, int dtype, int64_t N, int64_t Fr, const C* t, int nthr, int edge,
                               uint32_t* out, const Geom& g, hipStream_t s) {
  const bool staged = encode_staged_fits(g);
  const int grid = staged ? (int)(N < 65536 ? (N > 0 ? N : 1) : 65536) : grid_of(N * g.P * g.W);
  const size_t lds = staged ? (size_t)encode_staged_lds_bytes(g) : 0;
#define YTM_ENC_CASE(code, T)                                                                                    \
  case code:                                                                                                     \
    if (staged)                                                                                                  \
      encode_binned_staged_kernel<T, C, ONEHOT><<<grid, 256, lds, s>>>((const T*)X, N, Fr, t, nthr, edge, out, g); \
    else                                                                                                         \
      encode_binned_kernel<T, C, ONEHOT><<<grid, 256, 0, s>>>((const T*)X, N, Fr, t, nthr, edge, out, g);         \
    break;
  switch (dtype) {
    YTM_ENC_CASE(YTM_DTYPE_U8, uint8_t)
    YTM_ENC_CASE(YTM_DTYPE_I8, int8_t)
    YTM_ENC_CASE(YTM_DTYPE_U16, uint16_t)
    YTM_ENC_CASE(YTM_DTYPE_I16, int16_t)
    YTM_ENC_CASE(YTM_DTYPE_U32, uint32_t)
    YTM_ENC_CASE(YTM_DTYPE_I32, int32_t)
    YTM_ENC_CASE(YTM_DTYPE_I64, int64_t)
    YTM_ENC_CASE(YTM_DTYPE_F32, float)
    YTM_ENC_CASE(YTM_DTYPE_F64, double)
    default:
      return hipErrorInvalidValue;
  }
#undef YTM_ENC_CASE
  return hipGetLastError();
}

}  // namespace

hipError_t launch_encode_binned(const void* X, int dtype, int64_t N, int64_t Fr, const void* t, bool int_thresholds,
                                int nthr, bool onehot, int edge, uint32_t* out, const Geom& g, hipStream_t s) {
  if (int_thresholds)
    return onehot ? launch_encode_typed<int64_t, true>(X, dtype, N, Fr, (const int64_t*)t, nthr, edge, out, g, s)
                  : launch_encode_typed<int64_t, false>(X, dtype, N, Fr, (const int64_t*)t, nthr, edge, out, g, s);
  return onehot ? launch_encode_typed<double, true>(X, dtype, N, Fr, (const double*)t, nthr, edge, out, g, s)
                : launch_encode_typed<double, false>(X, dtype, N, Fr, (const double*)t, nthr, edge, out, g, s);
}

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
