// ytm_encode.h -- the encoding of samples into literal words (encode_batch,
// src/cutm/cuda/kernel.cu:76-152) as a closed form per output word, shared by the plain
// encode (uint32 pixel values, any value > 0 set; ytm_kernels.hip) and the encode fused with
// the binarizers (raw values binned on the fly; ytm_binarize.hip).
#ifndef YTM_ENCODE_H
#define YTM_ENCODE_H

#include "ytm_device.h"

namespace ytm {

// Pixel values of the plain encode: value f of sample e, set when above 0.
struct PlainPixels {
  const uint32_t* X;
  int64_t F;  // values per sample
  __device__ __forceinline__ bool operator()(int64_t e, int64_t f) const { return X[e * F + f] > 0u; }
};

// Positive literal li of patch (py, px) of sample e, the pixels read through pix(e, f) with
// f the flat index dim0 * dim2 * y + dim2 * x + z of the reference's input rows.
template <typename Pix>
__device__ __forceinline__ uint32_t positive_literal(const Pix& pix, int64_t e, const Geom& g, int64_t li, int64_t py,
                                                     int64_t px) {
  const int64_t ty = g.dim1 - g.pd1, tx = g.dim0 - g.pd0;
  int64_t idx = li;
  bool therm = false;
  if (g.encode_loc) {
    if (li < ty) return li < py ? 1u : 0u;
    if (li < ty + tx) return (li - ty) < px ? 1u : 0u;
    idx = li - ty - tx;
  } else {
    // The thermometer loops of kernel.cu:101-121 run even without ENCODE_LOC and write
    // over the first pixel literals; reproduced as-is.
    therm = (li < py) || (li >= ty && li < ty + px);
  }
  const int64_t row = (int64_t)g.pd0 * g.dim2;
  const int64_t ry = idx / row, rem = idx % row;
  const int64_t rx = rem / g.dim2, z = rem % g.dim2;
  return (therm || pix(e, (py + ry) * ((int64_t)g.dim0 * g.dim2) + (px + rx) * g.dim2 + z)) ? 1u : 0u;
}

// Encoded words of N samples, one thread per output word (e, p, w); every bit is what
// encode_batch leaves in it: negated literal l + L/2 = NOT positive literal l (the prefilled
// negated half is cleared exactly where a positive bit is set); positives are the y/x
// thermometers and the patch pixels; bits >= L stay 0 (the reference memsets the output
// first).
template <typename Pix>
__device__ __forceinline__ void encode_words(const Pix& pix, int64_t N, uint32_t* __restrict__ out, const Geom& g) {
  const int64_t total = N * g.P * g.W;
  const int64_t xw = g.dim0 - g.pd0 + 1;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t w = idx % g.W;
    const int64_t ep = idx / g.W;
    const int64_t p = ep % g.P, e = ep / g.P;
    const int64_t py = p / xw, px = p % xw;
    uint32_t word = 0u;
    for (int b = 0; b < 32; ++b) {
      const int64_t l = w * 32 + b;
      if (l >= g.L) break;
      uint32_t bit;
      if (g.append_negated && l >= g.Lh)
        bit = positive_literal(pix, e, g, l - g.Lh, py, px) ^ 1u;
      else
        bit = positive_literal(pix, e, g, l, py, px);
      word |= bit << b;
    }
    out[idx] = word;
  }
}

}  // namespace ytm

#endif  // YTM_ENCODE_H
