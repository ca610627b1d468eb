// ytm_device.h -- device-side building blocks shared by the YTM kernels (gfx950).
//
//  * Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel Random Numbers: As Easy as
//    1, 2, 3", SC'11) and the draw-site layout of the model's random stream.
//  * Bit-sliced Tsetlin-automaton state: the TA state of 32 literals is held as NP
//    32-bit planes (plane j = bit j of s' = s + OFF).  OFF is chosen so that
//    "literal included" (s > number_of_ta_states/2, src/cutm/cuda/kernel.cu:177-190)
//    is exactly "plane NP-1 set": the include mask of a clause is its top plane.
//  * wave64 helpers.
#pragma once
#include "ytm_types.h"

namespace ytm {

constexpr int kWave = 64;
constexpr int kMaxPlanes = 32;  // every int32 number_of_ta_states fits (np <= 31)

constexpr uint32_t TAG_SEL = 1;   // reservoir draw of the r-th firing patch
constexpr uint32_t TAG_CK = 2;    // per (clause, class): Q-skip draw, update draw
constexpr uint32_t TAG_LIT = 3;   // literal draws, 24 bit-planes per literal word
constexpr uint32_t TAG_INIT = 4;  // weight initialisation

struct U4 {
  uint32_t x, y, z, w;
};

__device__ __forceinline__ U4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                            uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
    c1 = (uint32_t)p1;
    c3 = (uint32_t)p0;
    c0 = n0;
    c2 = n2;
  }
  return U4{c0, c1, c2, c3};
}

// Counter of a draw site: (step low word, clause, tag | step high bits, site index).
__device__ __forceinline__ U4 site_words(uint64_t seed, uint64_t t, uint32_t c, uint32_t tag,
                                         uint32_t site) {
  return philox4x32_10((uint32_t)t, c, (tag << 28) | (uint32_t)((t >> 32) & 0x0fffffffu), site,
                       (uint32_t)seed, (uint32_t)(seed >> 32));
}

__device__ __forceinline__ uint32_t word_of(const U4& z, int i) {
  return i == 0 ? z.x : (i == 1 ? z.y : (i == 2 ? z.z : z.w));
}

// Uniform in (0, 1] from the top 24 bits of a word: ((z >> 8) + 1) * 2^-24, exact in fp32.
__device__ __forceinline__ float uniform_from_word(uint32_t z) {
  return (float)((z >> 8) + 1u) * (1.0f / 16777216.0f);
}

// ---------------------------------------------------------------- bit-sliced TA state
// Mask of the 32 lanes whose value (planes pl[0..np)) is < cst.  cst >= 2^np: all.
__device__ __forceinline__ uint32_t planes_lt(const uint32_t* pl, int np, uint32_t cst) {
  if (np < 32 && (cst >> np)) return 0xFFFFFFFFu;
  uint32_t lt = 0u, eq = 0xFFFFFFFFu;
#pragma unroll
  for (int j = kMaxPlanes - 1; j >= 0; --j) {
    if (j < np) {
      const uint32_t p = pl[j];
      if ((cst >> j) & 1u) {
        lt |= eq & ~p;
        eq &= p;
      } else {
        eq &= ~p;
      }
    }
  }
  return lt;
}

// Mask of the lanes whose value is > cst (cst < 2^np).
__device__ __forceinline__ uint32_t planes_gt(const uint32_t* pl, int np, uint32_t cst) {
  uint32_t gt = 0u, eq = 0xFFFFFFFFu;
#pragma unroll
  for (int j = kMaxPlanes - 1; j >= 0; --j) {
    if (j < np) {
      const uint32_t p = pl[j];
      if ((cst >> j) & 1u) {
        eq &= p;
      } else {
        gt |= eq & p;
        eq &= ~p;
      }
    }
  }
  return gt;
}

// +1 on the lanes of m (ripple carry through the planes).
__device__ __forceinline__ void planes_inc(uint32_t* pl, int np, uint32_t m) {
  uint32_t carry = m;
#pragma unroll
  for (int j = 0; j < kMaxPlanes; ++j) {
    if (j < np) {
      const uint32_t t = pl[j] & carry;
      pl[j] ^= carry;
      carry = t;
    }
  }
}

// -1 on the lanes of m (ripple borrow).
__device__ __forceinline__ void planes_dec(uint32_t* pl, int np, uint32_t m) {
  uint32_t borrow = m;
#pragma unroll
  for (int j = 0; j < kMaxPlanes; ++j) {
    if (j < np) {
      const uint32_t t = ~pl[j] & borrow;
      pl[j] ^= borrow;
      borrow = t;
    }
  }
}

// ---------------------------------------------------------------- wave64 helpers
// Inclusive scans over the 64 lanes with DPP (data-parallel primitives: VALU operands read
// from another lane), which avoid the LDS crossbar that lane shuffles go through: shifts by
// 1, 2, 4, 8 within each row of 16 lanes (Hillis-Steele), then row_bcast:15 (lane 15 of
// row r into row r+1, rows 1 and 3) and row_bcast:31 (lane 31 into rows 2 and 3).  A lane
// whose source is out of range receives the identity.  Call with every lane active.
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;

__device__ __forceinline__ int wave_scan_add_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr1, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr2, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr4, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr8, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowBcast15, 0xa, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowBcast31, 0xc, 0xf, false);
  return v;
}

__device__ __forceinline__ int wave_scan_max_i32(int v) {
  const int lo = (int)0x80000000;
  v = max(v, __builtin_amdgcn_update_dpp(lo, v, kDppRowShr1, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(lo, v, kDppRowShr2, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(lo, v, kDppRowShr4, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(lo, v, kDppRowShr8, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(lo, v, kDppRowBcast15, 0xa, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(lo, v, kDppRowBcast31, 0xc, 0xf, false));
  return v;
}

__device__ __forceinline__ uint32_t wave_scan_or_u32(uint32_t v) {
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowShr1, 0xf, 0xf, false);
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowShr2, 0xf, 0xf, false);
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowShr4, 0xf, 0xf, false);
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowShr8, 0xf, 0xf, false);
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowBcast15, 0xa, 0xf, false);
  v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kDppRowBcast31, 0xc, 0xf, false);
  return v;
}

// Value of lane `src` (wave-uniform) in every lane.
__device__ __forceinline__ int lane_value(int v, int src) { return __builtin_amdgcn_readlane(v, src); }

__device__ __forceinline__ int wave_sum_i32(int v) { return lane_value(wave_scan_add_i32(v), kWave - 1); }
__device__ __forceinline__ int wave_max_i32(int v) { return lane_value(wave_scan_max_i32(v), kWave - 1); }
__device__ __forceinline__ unsigned long long wave_or_u64(unsigned long long v) {
  const uint32_t lo = wave_scan_or_u32((uint32_t)v), hi = wave_scan_or_u32((uint32_t)(v >> 32));
  return ((unsigned long long)(uint32_t)lane_value((int)hi, kWave - 1) << 32) | (uint32_t)lane_value((int)lo, kWave - 1);
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

}  // namespace ytm
