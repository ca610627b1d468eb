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
  __device__ __forceinline__ bool bit32(int64_t e, int f) const { return X[e * F + f] > 0u; }
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

// Several patches (or one wide patch): the same words as encode_words, a block per sample
// at a time.  The sample's F pixel bits pix(e, f) are staged in LDS as a bitmap first (each
// wave ballots 64 consecutive bits; one evaluation of pix per bit instead of one per output
// bit: config 4 reads each binned pixel bit in up to 9 patches).  Then each thread builds
// whole words:
// the pixel literals of one patch row are consecutive pixel values (f = patch origin +
// ry * image row + rx * dim2 + z, with rx * dim2 + z running over pd0 * dim2 values), so a
// word takes its pixel literals as a few bit ranges of the bitmap instead of bit by bit.  A
// word holds at most two runs of positive-literal indices: its positive literals, then
// (with appended negations) the negated ones.
constexpr int64_t kEncodeStagedMaxBits = 256 * 1024;  // a 32 KB LDS bitmap

// Several patches, or one patch of enough words to occupy a block (config 5: 625).
__host__ __device__ constexpr bool encode_staged_fits(const Geom& g) {
  return (g.P > 1 || g.W >= 128) && g.F <= kEncodeStagedMaxBits && g.P * g.W < (int64_t(1) << 31);
}

__host__ __device__ constexpr int64_t encode_staged_lds_bytes(const Geom& g) { return (g.F + 31) / 32 * 4; }

// Bits [lo, hi) of a 32-bit word (clamped to [0, 32)).
__device__ __forceinline__ uint32_t bit_range(int lo, int hi) {
  lo = lo < 0 ? 0 : lo;
  hi = hi > 32 ? 32 : hi;
  if (hi <= lo) return 0u;
  const uint32_t upto = hi == 32 ? 0xFFFFFFFFu : ((1u << hi) - 1u);
  return upto & ~((1u << lo) - 1u);
}

template <typename Pix>
__device__ __forceinline__ void encode_staged(const Pix& pix, int64_t N, uint32_t* __restrict__ out, const Geom& g) {
  extern __shared__ uint32_t s_bits[];  // [ceil(F / 32)]
  const int F = (int)g.F, FW = (F + 31) / 32;
  const int W = (int)g.W, PWw = (int)(g.P * g.W);
  const int xw = g.dim0 - g.pd0 + 1;
  const int ty = g.dim1 - g.pd1, tx = g.dim0 - g.pd0;
  const int row = g.pd0 * g.dim2;        // pixel literals per patch row
  const int img_row = g.dim0 * g.dim2;   // pixel values per image row
  const bool loc_on = g.encode_loc != 0;
  const int loc = loc_on ? ty + tx : 0;  // literals before the patch pixels
  const int L = (int)g.L, Lh = (int)g.Lh;
  const bool an = g.append_negated != 0;
  const int lane = (int)(threadIdx.x & (kWave - 1)), wv = (int)(threadIdx.x / kWave);
  const int nwv = (int)(blockDim.x / kWave);
  for (int64_t e = blockIdx.x; e < N; e += gridDim.x) {
    __syncthreads();  // the previous sample's bits are no longer read
    for (int f0 = wv * kWave; f0 < F; f0 += nwv * kWave) {
      const int f = f0 + lane;
      const unsigned long long m = __ballot(f < F && pix.bit32(e, f));
      if (lane == 0) s_bits[f0 >> 5] = (uint32_t)m;
      if (lane == 1 && (f0 >> 5) + 1 < FW) s_bits[(f0 >> 5) + 1] = (uint32_t)(m >> 32);
    }
    __syncthreads();
    uint32_t* oe = out + e * (int64_t)PWw;
    for (int idx = threadIdx.x; idx < PWw; idx += blockDim.x) {
      const int p = idx / W, w = idx - p * W;
      const int py = p / xw, px = p - py * xw;
      const int base = py * img_row + px * g.dim2;  // pixel value of the patch origin
      const int l0 = w * 32, l1 = l0 + 32 < L ? l0 + 32 : L;
      uint32_t word = 0u;
      for (int seg = 0; seg < 2; ++seg) {
        const bool neg = seg == 1;
        if (neg && !an) break;
        int l = neg ? (l0 > Lh ? l0 : Lh) : l0;
        const int bnd = (an && !neg) ? (l1 < Lh ? l1 : Lh) : l1;
        int li = neg ? l - Lh : l;  // positive literal index
        for (; l < bnd && li < loc; ++l, ++li) {  // the position thermometers (encode_loc)
          const uint32_t bit = li < ty ? (li < py ? 1u : 0u) : ((li - ty) < px ? 1u : 0u);
          word |= (bit ^ (neg ? 1u : 0u)) << (l - l0);
        }
        while (l < bnd) {  // pixel literals, up to the end of a patch row at a time
          const int pi = li - loc;
          const int ry = pi / row, c = pi - ry * row;
          const int k = row - c < bnd - l ? row - c : bnd - l;  // 1..32
          const int f = base + ry * img_row + c;
          const int w0 = f >> 5;
          const unsigned long long two =
              (unsigned long long)s_bits[w0] | ((unsigned long long)s_bits[w0 + 1 < FW ? w0 + 1 : w0] << 32);
          const uint32_t keep = k == 32 ? 0xFFFFFFFFu : ((1u << k) - 1u);
          uint32_t bits = (uint32_t)(two >> (f & 31)) & keep;
          // without encode_loc the thermometers still overwrite the first pixel literals
          // (positive_literal): literal li + t with li + t < py or ty <= li + t < ty + px
          if (!loc_on) bits |= (bit_range(0, py - li) | bit_range(ty - li, ty + px - li)) & keep;
          if (neg) bits = ~bits & keep;
          word |= bits << (l - l0);
          l += k;
          li += k;
        }
      }
      oe[idx] = word;
    }
  }
}

}  // namespace ytm

#endif  // YTM_ENCODE_H
