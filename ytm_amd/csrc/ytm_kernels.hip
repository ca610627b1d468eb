// ytm_kernels.hip -- hand-written gfx950 kernels of the YTM Tsetlin Machine hot path.
//
// Data layout in HBM (per model):
//   planes  uint32 [C][np][W]   bit-sliced TA states; plane np-1 is the include mask
//   weights float  [C][K]       clause weights (integer-valued, as the reference keeps them)
//   patch_w int32  [C][P]       reservoir selection counts
// Encoded inputs keep the reference layout uint32 [N][P][W] (src/cutm/base.py:238).
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "ytm_device.h"
#include "ytm_encode.h"
#include "ytm_internal.h"
#include "ytm_train.h"

namespace ytm {

// ============================================================================ encode
// One thread per output word (encode_words, ytm_encode.h).
__global__ __launch_bounds__(256) void encode_kernel(const uint32_t* __restrict__ X, int64_t N,
                                                     uint32_t* __restrict__ out, Geom g) {
  encode_words(PlainPixels{X, g.F}, N, out, g);
}

// Several patches: a block per sample, its pixel bits staged in LDS (encode_staged).
__global__ __launch_bounds__(256) void encode_staged_kernel(const uint32_t* __restrict__ X, int64_t N,
                                                            uint32_t* __restrict__ out, Geom g) {
  encode_staged(PlainPixels{X, g.F}, N, out, g);
}

// Literal-major copy of encoded samples with several patches: bit b of XT[e][l][j] is
// literal l of patch 32j + b (0 beyond P), PW = ceil(P / 32) words per literal.  One wave
// per (sample, literal word w, chunk of 64 patches): lane q holds word w of patch
// 64*chunk + q, and one ballot per bit gives a literal's 64-patch bitset.
__global__ __launch_bounds__(256) void transpose_kernel(const uint32_t* __restrict__ X, int64_t N, Geom g,
                                                        uint32_t* __restrict__ XT) {
  const int lane = lane_id();
  const int64_t PW = (g.P + 31) / 32;
  const int64_t nchunk = (g.P + kWave - 1) / kWave;
  const int64_t items = N * g.W * nchunk;
  const int64_t wave = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) / kWave;
  const int64_t nwaves = (int64_t)gridDim.x * blockDim.x / kWave;
  for (int64_t item = wave; item < items; item += nwaves) {
    const int64_t e = item / (g.W * nchunk), rem = item % (g.W * nchunk);
    const int64_t w = rem / nchunk, ch = rem % nchunk;
    const int64_t p = ch * kWave + lane;
    const uint32_t xw = p < g.P ? X[(e * g.P + p) * g.W + w] : 0u;
    unsigned long long keep = 0ull;
#pragma unroll
    for (int b = 0; b < 32; ++b) {
      const unsigned long long bits = __ballot((xw >> b) & 1u);
      if (lane == b) keep = bits;
    }
    const int64_t l = 32 * w + lane;
    if (lane < 32 && l < g.L) {
      uint32_t* dst = XT + (e * g.L + l) * PW + 2 * ch;
      dst[0] = (uint32_t)keep;
      if (2 * ch + 1 < PW) dst[1] = (uint32_t)(keep >> 32);
    }
  }
}

// Clears *ok when some literal Lh + f of XT is not the complement of literal f in every
// patch (bits of patches >= P: 0 in both), i.e. when the training kernels may not stage
// only the first half of each sample's copy (TrainArgs::xt_halves).  *ok is set before.
__global__ __launch_bounds__(256) void xt_halves_kernel(const uint32_t* __restrict__ XT, int64_t N, Geom g,
                                                        int* ok) {
  const int64_t PW = (g.P + 31) / 32;
  const int64_t nh = g.Lh * PW;
  const uint32_t lastm = (g.P & 31) ? ((1u << (g.P & 31)) - 1u) : 0xFFFFFFFFu;
  const int64_t n = N * nh;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < n;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e = idx / nh, j = idx % nh;
    const uint32_t* row = XT + e * g.L * PW;
    if (row[nh + j] != (~row[j] & (j % PW == PW - 1 ? lastm : 0xFFFFFFFFu))) *ok = 0;
  }
}

// ===================================================================== TA state I/O
// uint32 (C, L) states <-> bit-planes.  Literals >= L of the last word hold s = 0 and are
// never updated or included.
__global__ __launch_bounds__(256) void ta_to_planes_kernel(const uint32_t* __restrict__ ta,
                                                           uint32_t* __restrict__ planes, Geom g) {
  const int64_t total = g.C * g.W;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t c = idx / g.W, w = idx % g.W;
    uint32_t pl[kMaxPlanes];
#pragma unroll
    for (int j = 0; j < kMaxPlanes; ++j) pl[j] = 0u;
    for (int b = 0; b < 32; ++b) {
      const int64_t l = w * 32 + b;
      const uint32_t s = (l < g.L ? ta[c * g.L + l] : 0u) + g.off;
#pragma unroll
      for (int j = 0; j < kMaxPlanes; ++j) pl[j] |= ((s >> j) & 1u) << b;
    }
    for (int j = 0; j < g.np; ++j) planes[(c * g.np + j) * g.W + w] = pl[j];
  }
}

__global__ __launch_bounds__(256) void planes_to_ta_kernel(const uint32_t* __restrict__ planes,
                                                           uint32_t* __restrict__ ta, Geom g) {
  const int64_t total = g.C * g.L;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t c = idx / g.L, l = idx % g.L;
    const int64_t w = l >> 5;
    const int b = (int)(l & 31);
    uint32_t s = 0u;
    for (int j = 0; j < g.np; ++j) s |= ((planes[(c * g.np + j) * g.W + w] >> b) & 1u) << j;
    ta[idx] = s - g.off;
  }
}

// Initial state: every TA at number_of_ta_states/2 (src/cutm/base.py:208-209) and the
// weights of init_weights (kernel.cu:46-73) with its random bit taken from the INIT site.
__global__ __launch_bounds__(256) void init_state_kernel(uint32_t* __restrict__ planes,
                                                         float* __restrict__ w, Geom g, uint64_t seed) {
  const int64_t nplane = g.C * g.W;
  const int64_t total = nplane > g.C * g.K ? nplane : g.C * g.K;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    if (idx < nplane) {
      const int64_t c = idx / g.W, wd = idx % g.W;
      const uint32_t valid = wd == g.W - 1 ? g.last_filter : 0xFFFFFFFFu;
      const uint32_t s_on = (uint32_t)g.half_state + g.off, s_off = g.off;
      for (int j = 0; j < g.np; ++j) {
        const uint32_t v = (((s_on >> j) & 1u) ? valid : 0u) | (((s_off >> j) & 1u) ? ~valid : 0u);
        planes[(c * g.np + j) * g.W + wd] = v;
      }
    }
    if (idx < g.C * g.K) {
      const int64_t c = idx / g.K, k = idx % g.K;
      float v;
      if (g.coalesced) {
        v = 1.0f;
        if (g.init_neg_weights) {
          const U4 z = site_words(seed, 0, (uint32_t)c, TAG_INIT, (uint32_t)k);
          v = 1.0f - 2.0f * (float)(z.x & 1u);
        }
      } else if (k == c / g.per_bank) {
        v = 1.0f;
        if (g.init_neg_weights && (c % g.per_bank) >= (g.per_bank / 2)) v = -1.0f;
      } else {
        v = 0.0f;
      }
      w[idx] = v;
    }
  }
}

// Number of included literals per clause (pack_clauses' total_count, kernel.cu:166-202).
__global__ __launch_bounds__(256) void ninc_kernel(const uint32_t* __restrict__ planes,
                                                   int32_t* __restrict__ ninc, Geom g) {
  const int lane = lane_id();
  const int64_t wave = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) / kWave;
  const int64_t nwaves = (int64_t)gridDim.x * blockDim.x / kWave;
  for (int64_t c = wave; c < g.C; c += nwaves) {
    const uint32_t* m = planes + (c * g.np + g.np - 1) * g.W;
    int cnt = 0;
    for (int64_t w = lane; w < g.W; w += kWave) cnt += __popc(m[w]);
    cnt = wave_sum_i32(cnt);
    if (lane == 0) ninc[c] = cnt;
  }
}

__global__ __launch_bounds__(256) void fill_u64_kernel(unsigned long long* p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0ull;
}

// ======================================================================== inference
// Does a non-empty clause (include mask m) match sample xe on at least one patch?
// clause_match (kernel.cu:207-216) with the early exit of calc_class_sums_infer_batch
// (kernel.cu:330-336).  Wave-uniform result.
template <bool VANILLA>
__device__ __forceinline__ bool clause_fires_any(const uint32_t* __restrict__ m,
                                                 const uint32_t* __restrict__ xe, const Geom& g) {
  const int lane = lane_id();
  if (VANILLA) {
    uint32_t bad = 0u;
    for (int64_t w = lane; w < g.W; w += kWave) bad |= m[w] & ~xe[w];
    return !__any(bad != 0u);
  } else {
    for (int64_t base = 0; base < g.P; base += kWave) {
      const int64_t p = base + lane;
      bool ok = p < g.P;
      if (ok) {
        const uint32_t* xp = xe + p * g.W;
        for (int64_t w = 0; w < g.W; ++w)
          if (m[w] & ~xp[w]) {
            ok = false;
            break;
          }
      }
      if (__any(ok)) return true;
    }
    return false;
  }
}

constexpr int kScoreChunk = 256;

// One block per (sample, chunk of clauses); waves take clauses; lane k accumulates the
// weight of class k over the firing clauses; integer atomics make the sum exact and
// order-independent.
template <bool VANILLA>
__global__ __launch_bounds__(256) void score_kernel(const uint32_t* __restrict__ planes,
                                                    const int32_t* __restrict__ ninc,
                                                    const float* __restrict__ w,
                                                    const uint32_t* __restrict__ X, int64_t N, Geom g,
                                                    long long* __restrict__ acc) {
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave, nw = blockDim.x / kWave;
  const int64_t nch = (g.C + kScoreChunk - 1) / kScoreChunk;
  for (int64_t blk = blockIdx.x; blk < N * nch; blk += gridDim.x) {
    const int64_t e = blk / nch, ch = blk % nch;
    const int64_t c0 = ch * kScoreChunk;
    const int64_t c1 = c0 + kScoreChunk < g.C ? c0 + kScoreChunk : g.C;
    const uint32_t* xe = X + e * g.P * g.W;
    long long sum = 0;
    for (int64_t c = c0 + wave; c < c1; c += nw) {
      if (ninc[c] == 0) continue;  // empty clauses do not vote (kernel.cu:328)
      if (clause_fires_any<VANILLA>(planes + (c * g.np + g.np - 1) * g.W, xe, g))
        if (lane < g.K) sum += (long long)w[c * g.K + lane];
    }
    if (lane < g.K && sum != 0)
      atomicAdd((unsigned long long*)&acc[e * g.K + lane], (unsigned long long)sum);
  }
}

// More than 64 classes: as score_kernel, but a firing clause's weights go into the block's
// LDS sums [K] (int64 atomics, 64 classes per wave step), which the block adds into acc at
// the end of its chunk.
template <bool VANILLA>
__global__ __launch_bounds__(256) void score_classes_kernel(const uint32_t* __restrict__ planes,
                                                            const int32_t* __restrict__ ninc,
                                                            const float* __restrict__ w,
                                                            const uint32_t* __restrict__ X, int64_t N, Geom g,
                                                            long long* __restrict__ acc) {
  extern __shared__ long long s_sum[];  // [K]
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave, nw = blockDim.x / kWave;
  const int64_t nch = (g.C + kScoreChunk - 1) / kScoreChunk;
  for (int64_t blk = blockIdx.x; blk < N * nch; blk += gridDim.x) {
    const int64_t e = blk / nch, ch = blk % nch;
    const int64_t c0 = ch * kScoreChunk;
    const int64_t c1 = c0 + kScoreChunk < g.C ? c0 + kScoreChunk : g.C;
    const uint32_t* xe = X + e * g.P * g.W;
    __syncthreads();  // the previous chunk's sums are flushed
    for (int64_t k = threadIdx.x; k < g.K; k += blockDim.x) s_sum[k] = 0;
    __syncthreads();
    for (int64_t c = c0 + wave; c < c1; c += nw) {
      if (ninc[c] == 0) continue;  // empty clauses do not vote (kernel.cu:328)
      if (clause_fires_any<VANILLA>(planes + (c * g.np + g.np - 1) * g.W, xe, g))
        for (int64_t k = lane; k < g.K; k += kWave) {
          const long long v = (long long)w[c * g.K + k];
          if (v != 0) atomicAdd((unsigned long long*)&s_sum[k], (unsigned long long)v);
        }
    }
    __syncthreads();
    for (int64_t k = threadIdx.x; k < g.K; k += blockDim.x)
      if (s_sum[k] != 0) atomicAdd((unsigned long long*)&acc[e * g.K + k], (unsigned long long)s_sum[k]);
  }
}

// One patch: lanes are samples.  A block takes a tile of 64 samples (staged transposed in
// LDS, [W][64], so that lane e reads word w of its own sample) and a chunk of clauses; each
// wave walks its clauses, reading a clause's mask words once and skipping the zero ones with
// scalar logic, so one instruction tests a mask word against 64 samples.  A lane whose
// sample the clause fires on adds the clause's weights to its int64 sums, which go to the
// exact accumulators at the end of the chunk (calc_class_sums_infer_batch, kernel.cu:319-343:
// empty clauses do not vote).
constexpr int kScoreTile = 64;
constexpr int kScoreTileChunk = 256;
constexpr int kScoreTileMaxK = 16;

__global__ __launch_bounds__(256) void score_tile_kernel(const uint32_t* __restrict__ planes,
                                                         const int32_t* __restrict__ ninc,
                                                         const float* __restrict__ w,
                                                         const uint32_t* __restrict__ X, int64_t N, Geom g,
                                                         long long* __restrict__ acc) {
  extern __shared__ uint32_t s_tile[];  // [W][64]
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave, nwv = blockDim.x / kWave;
  const int64_t ntile = (N + kScoreTile - 1) / kScoreTile;
  const int64_t nch = (g.C + kScoreTileChunk - 1) / kScoreTileChunk;
  for (int64_t blk = blockIdx.x; blk < ntile * nch; blk += gridDim.x) {
    const int64_t e0 = (blk / nch) * kScoreTile, ch = blk % nch;
    const int64_t c0 = ch * kScoreTileChunk;
    const int64_t c1 = c0 + kScoreTileChunk < g.C ? c0 + kScoreTileChunk : g.C;
    __syncthreads();  // the previous tile is no longer read
    for (int64_t j = threadIdx.x; j < kScoreTile * g.W; j += blockDim.x) {
      const int64_t sidx = j / g.W, ww = j % g.W, e = e0 + sidx;
      s_tile[ww * kScoreTile + sidx] = e < N ? X[e * g.W + ww] : 0u;
    }
    __syncthreads();
    long long sum[kScoreTileMaxK];
#pragma unroll
    for (int k = 0; k < kScoreTileMaxK; ++k) sum[k] = 0;
    for (int64_t c = c0 + wave; c < c1; c += nwv) {
      if (ninc[c] == 0) continue;  // empty clauses do not vote
      const uint32_t* m = planes + (c * g.np + g.np - 1) * g.W;
      bool alive = true;
      for (int64_t wb = 0; wb < g.W; wb += kWave) {
        const uint32_t mv = wb + lane < g.W ? m[wb + lane] : 0u;
        unsigned long long nz = __ballot(mv != 0u);  // the chunk's non-zero mask words
        int tested = 0;
        while (nz) {
          const int q = __ffsll((long long)nz) - 1;
          nz &= nz - 1ull;
          const uint32_t mw = (uint32_t)lane_value((int)mv, q);
          alive = alive && (mw & ~s_tile[(wb + q) * kScoreTile + lane]) == 0u;
          if ((++tested & 7) == 0 && !__any(alive)) break;
        }
        if (!__any(alive)) break;
      }
      if (alive) {
#pragma unroll
        for (int k = 0; k < kScoreTileMaxK; ++k)
          if (k < g.K) sum[k] += (long long)w[c * g.K + k];
      }
    }
    const int64_t e = e0 + lane;
    if (e < N) {
#pragma unroll
      for (int k = 0; k < kScoreTileMaxK; ++k)
        if (k < g.K && sum[k] != 0) atomicAdd((unsigned long long*)&acc[e * g.K + k], (unsigned long long)sum[k]);
    }
  }
}

// Literal order of the list walks (build_literal_list): the density of literal l over the
// first S samples, the share of their (sample, patch) pairs where l is 1, from the
// literal-major copy XT ([N][L][PW]) when given, else from X ([N][P][W]); literal l goes to
// bucket min(kOrderBuckets - 1, density * kOrderBuckets), literals past L to the last.  A
// block of 4 waves takes 64 literals (two words of the order), each wave a quarter of the
// rows.
__global__ __launch_bounds__(256) void literal_order_kernel(const uint32_t* __restrict__ X,
                                                            const uint32_t* __restrict__ XT, int64_t S, Geom g,
                                                            uint32_t* __restrict__ order) {
  __shared__ int64_t s_cnt[4][kWave];
  const int lane = lane_id(), part = threadIdx.x / kWave;
  const int64_t l = (int64_t)blockIdx.x * kWave + lane;
  const int64_t PW = (g.P + 31) / 32;
  int64_t cnt = 0;
  if (l < g.L) {
    if (XT) {
      for (int64_t e = part; e < S; e += 4)
        for (int64_t j = 0; j < PW; ++j) cnt += __popc(XT[(e * g.L + l) * PW + j]);
    } else {
      for (int64_t r = part; r < S * g.P; r += 4) cnt += (X[r * g.W + l / 32] >> (l % 32)) & 1u;
    }
  }
  s_cnt[part][lane] = cnt;
  __syncthreads();
  if (part != 0) return;
  const int64_t total = s_cnt[0][lane] + s_cnt[1][lane] + s_cnt[2][lane] + s_cnt[3][lane];
  const int64_t pairs = S * g.P;
  int b = pairs > 0 ? (int)(total * kOrderBuckets / pairs) : 0;
  b = (l >= g.L || b >= kOrderBuckets) ? kOrderBuckets - 1 : b;
  for (int k = 0; k < kOrderBuckets; ++k) {
    const unsigned long long bal = __ballot(b == k);
    const int64_t w0 = 2 * (int64_t)blockIdx.x;
    if (lane == 0 && w0 < g.W) order[k * g.W + w0] = (uint32_t)bal;
    if (lane == 0 && w0 + 1 < g.W) order[k * g.W + w0 + 1] = (uint32_t)(bal >> 32);
  }
}

// The buckets of literal_order_kernel from the first min(N, kOrderSamples) samples.
hipError_t launch_literal_order(const uint32_t* X, const uint32_t* XT, int64_t N, const Geom& g, uint32_t* order,
                                hipStream_t s) {
  const int64_t S = N < kOrderSamples ? N : kOrderSamples;
  literal_order_kernel<<<(unsigned)((g.W + 1) / 2), 256, 0, s>>>(X, XT, S, g, order);
  return hipGetLastError();
}

// The included literals of every clause as a list (build_literal_list) in the order of
// `order` (null: literal index order), [C][cap] with the include counts [C]; one wave per
// clause.
__global__ __launch_bounds__(256) void build_lists_kernel(const uint32_t* __restrict__ planes, Geom g, int cap,
                                                          const uint32_t* __restrict__ order,
                                                          uint16_t* __restrict__ lists, int32_t* __restrict__ nlit) {
  const int lane = lane_id();
  const int64_t wave = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) / kWave;
  const int64_t nwaves = (int64_t)gridDim.x * blockDim.x / kWave;
  for (int64_t c = wave; c < g.C; c += nwaves) {
    const int n = build_literal_list(g, planes + (c * g.np + g.np - 1) * g.W, lists + c * cap, cap, order);
    if (lane == 0) nlit[c] = n;
  }
}

// Firing bitmap from a literal list held in registers: lane q has entries [8q, 8q + 8) in
// lv (the list padded to a multiple of 8).  With at least two groups of PW lanes in the wave
// (the bitmap's PW words), group gq takes the runs 8(it * NG + gq) of step it, fetching
// them from their lanes with ds_bpermute, and the groups' bitmaps are AND-ed at the end
// (as firing_from_list); otherwise the runs are read 8 at a time with readlane.  FORM:
// list_form(g).
template <int FORM>
__device__ __forceinline__ uint32_t firing_from_list_regs(const Geom& g, uint4 lv, int n, const uint32_t* xt,
                                                          uint32_t acc) {
  const int lane = lane_id();
  const int PW = (int)((g.P + 31) / 32);
  const int NG = kWave / PW;
  if (NG >= 2) {
    const int GS = NG == 2 ? 32 : PW;  // two groups: one per 32-lane half
    const int q = lane / GS, w = lane - q * GS;
    const bool in_group = q < NG && w < PW;
    uint32_t part = in_group ? (w == PW - 1 && (g.P & 31) ? ((1u << (g.P & 31)) - 1u) : 0xFFFFFFFFu) : 0u;
    const unsigned long long gmask = (1ull << PW) - 1ull;
    const int nruns = (n + 7) / 8;
    for (int r0 = 0; r0 < nruns; r0 += NG) {
      const int run = r0 + (in_group ? q : 0);
      const int src = 4 * (run < kWave ? run : 0);
      const uint32_t e[4] = {(uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)lv.x),
                             (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)lv.y),
                             (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)lv.z),
                             (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)lv.w)};
      if (in_group && run < nruns) part &= and_listed_as<FORM>(g, e, xt, (uint32_t)w);
      // the walk ends when nothing fires: with two groups (the 32-lane halves) when the AND
      // of both partials is empty (the halves' words meet through one lane swap), else
      // when some group's partial is empty
      bool dead;
      if (NG == 2) {
        const auto sw = __builtin_amdgcn_permlane32_swap(part, part, false, false);
        dead = !__any((sw[0] & sw[1]) != 0u);
      } else {
        const unsigned long long live = __ballot(part != 0u);
        dead = __any(in_group && ((live >> (q * GS)) & gmask) == 0ull);
      }
      if (dead) return 0u;  // nothing fires: no combination of the groups
    }
    uint32_t r = part;
    for (int gq = 1; gq < NG; ++gq)
      r &= (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (w + gq * GS < kWave ? w + gq * GS : lane), (int)part);
    return lane < PW ? (r & acc) : 0u;
  }
  const int jl = lane < PW ? lane : 0;
  for (int j = 0; j < n; j += 8) {
    const int src = j >> 3;
    const uint32_t qv[4] = {(uint32_t)lane_value((int)lv.x, src), (uint32_t)lane_value((int)lv.y, src),
                            (uint32_t)lane_value((int)lv.z, src), (uint32_t)lane_value((int)lv.w, src)};
    acc &= and_listed_as<FORM>(g, qv, xt, (uint32_t)jl);
    if ((j & 8) && !__any(acc != 0u)) break;
  }
  return acc;
}

// Several patches (literal-major samples): one block per (sample, chunk of clauses); the
// sample's literal-major copy is staged in LDS and each wave decides, clause by clause,
// whether any patch fires (the AND of the included literals' bitsets, from the clause's
// literal list when it has one) -- calc_class_sums_infer_batch, kernel.cu:319-343 (empty
// clauses do not vote).  Lanes < K sum the weights of the firing clauses exactly.
constexpr int64_t kScoreLmChunk = 4096;
constexpr int kScoreListCap = 256;
// Block size: 16 waves when the sample's literal-major copy is large (it is staged once per
// block, and its LDS limits the blocks per CU, so only large blocks keep enough waves on a
// CU to hide the latency of each clause's list reads: config 4, 64 KB, 1.9x), else 4
// (config 3, 13 KB: 256 threads are 19% faster than 1024).
constexpr int kScoreLmThreads = 1024;
inline int score_lm_threads(const Geom& g) { return (g.L * ((g.P + 31) / 32)) * 4 > 32 * 1024 ? 1024 : 256; }
// Clauses per block of score_lm_kernel: kScoreLmChunk, or every clause when the sample's
// copy is large (1024-thread blocks) and the samples alone give enough blocks to fill the
// GPU: the copy is then staged once per sample instead of once per 4096 clauses (config 4,
// 10000 samples: 245K -> 256K samples/s in the kernel).  Small copies keep the chunks (config
// 3 with one block per sample: 879K -> 855K).  YTM_SCORE_WHOLE_MIN sets the samples needed
// (default 2048).
constexpr int64_t kScoreLmWholeMinSamples = 2048;
inline int64_t score_lm_chunk(const Geom& g, int64_t N) {
  const char* env = std::getenv("YTM_SCORE_WHOLE_MIN");
  const int64_t min_n = env && std::atoll(env) > 0 ? std::atoll(env) : kScoreLmWholeMinSamples;
  return score_lm_threads(g) == 1024 && N >= min_n && g.C > kScoreLmChunk ? g.C : kScoreLmChunk;
}

// Eight waves per SIMD (the compiler keeps at most 64 VGPRs and moves SGPRs it cannot keep
// to VGPR lanes): at the default seven, SGPR-bound, a CU held one 1024-thread block of a
// 64 KB copy; now two (config 4 inference 269K -> 327K samples/s in the kernel, config 3
// 930K -> 999K).  The one-patch tile and wide scorers lost with the same bound (config 1
// 430M -> 356M, config 2 160M -> 157M) and keep the default.
template <int FORM>
__global__ __launch_bounds__(kScoreLmThreads) __attribute__((amdgpu_waves_per_eu(8))) void score_lm_kernel(
    const uint32_t* __restrict__ planes, const uint16_t* __restrict__ lists, const int32_t* __restrict__ nlit,
    const float* __restrict__ w, const uint32_t* __restrict__ XT, int64_t N, Geom g, int64_t chunk,
    long long* __restrict__ acc) {
  extern __shared__ uint32_t s_xts[];  // [L][PW]
  const int lane = lane_id();
  // wave-uniform in a scalar register, so that the clause loop and its loads are scalar
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave)), nwv = blockDim.x / kWave;
  const int64_t xtw = g.L * ((g.P + 31) / 32);
  const int64_t nch = (g.C + chunk - 1) / chunk;
  for (int64_t blk = blockIdx.x; blk < N * nch; blk += gridDim.x) {
    const int64_t e = blk / nch, ch = blk % nch;
    const int64_t c0 = ch * chunk, c1 = c0 + chunk < g.C ? c0 + chunk : g.C;
    __syncthreads();  // the previous sample is no longer read
    copy_to_lds(s_xts, XT + e * xtw, xtw, threadIdx.x, blockDim.x);
    __syncthreads();
    long long sum = 0;
    for (int64_t c = c0 + wave; c < c1; c += nwv) {
      const int n = nlit[c];
      if (n == 0) continue;  // empty clauses do not vote
      uint32_t fire = all_patches_word(g);
      if (n <= kScoreListCap) {
        const uint4 lv = 8 * lane < n ? *(const uint4*)(lists + c * kScoreListCap + 8 * lane) : uint4{0u, 0u, 0u, 0u};
        fire = firing_from_list_regs<FORM>(g, lv, n, s_xts, fire);
      } else {
        fire = firing_from_mask(g, planes + (c * g.np + g.np - 1) * g.W, s_xts, fire);
      }
      if (__any(fire != 0u) && lane < g.K) sum += (long long)w[c * g.K + lane];
    }
    if (lane < g.K && sum != 0) atomicAdd((unsigned long long*)&acc[e * g.K + lane], (unsigned long long)sum);
  }
}

// Class sums from per-chunk slices parts[nch][N][K] (tile_kernel) plus the bias.
__global__ __launch_bounds__(256) void score_parts_finish_kernel(const long long* __restrict__ parts, int64_t nch,
                                                                 const float* __restrict__ bias, int64_t N, Geom g,
                                                                 float* __restrict__ out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < N * g.K;
       i += (int64_t)gridDim.x * blockDim.x) {
    long long v = (long long)bias[i % g.K];
    for (int64_t ch = 0; ch < nch; ++ch) v += parts[ch * N * g.K + i];
    out[i] = (float)v;
  }
}

__global__ __launch_bounds__(256) void score_finish_kernel(const long long* __restrict__ acc,
                                                           const float* __restrict__ bias, int64_t N,
                                                           Geom g, float* __restrict__ out) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < N * g.K;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = (float)(acc[i] + (long long)bias[i % g.K]);
}

// One patch, lanes = samples: a block stages kTileC clauses' include masks (rows padded to
// a multiple of 4 words, zero beyond W) in LDS; each of its four waves holds the
// complements of its own 64 samples' words in VGPRs and tests every staged clause with one
// AND-OR per word against a broadcast LDS row.  MODE 0 adds the firing clauses' weights into
// per-lane class sums (calc_class_sums_infer_batch, kernel.cu:319-343: empty clauses do not
// vote); MODE 1 writes clause outputs (transform, kernel.cu:346-368, and transform_patchwise
// with its single patch: empty clauses output 1) through per-clause ballots in LDS, so that
// each output row is written coalesced.  MAXQ bounds W by 4*MAXQ words.
constexpr int kTileC = 96;
constexpr int kTileMaxK = 16;
constexpr int kTileStage = 8;  // staged words in flight per thread

template <int MAXQ, int MODE, bool SUM32>
__global__ __launch_bounds__(256) void tile_kernel(const uint32_t* __restrict__ planes,
                                                   const int32_t* __restrict__ ninc, const float* __restrict__ w,
                                                   const uint32_t* __restrict__ X, int64_t N, Geom g,
                                                   long long* __restrict__ acc, uint32_t* __restrict__ out) {
  // SUM32: the class sums of a chunk are exact in int32 (the caller bounds |w| * kTileC < 2^31)
  using Sum = typename std::conditional<SUM32, int, long long>::type;
  __shared__ uint4 s_m[kTileC * MAXQ];
  __shared__ Sum s_w[MODE == 0 ? kTileC * kTileMaxK : 1];
  __shared__ int s_live[kTileC];
  __shared__ unsigned long long s_bal[MODE == 1 ? 4 * kTileC : 1];
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int Wq = (int)((g.W + 3) / 4);
  const int64_t nsg = (N + 255) / 256;
  const int64_t nch = (g.C + kTileC - 1) / kTileC;
  for (int64_t blk = blockIdx.x; blk < nsg * nch; blk += gridDim.x) {
    const int64_t e0 = (blk / nch) * 256 + wave * kWave, c0 = (blk % nch) * kTileC;
    const int nc = (int)(c0 + kTileC < g.C ? kTileC : g.C - c0);
    __syncthreads();  // the previous chunk is no longer read
    // Staging: every load reads a valid address (clamped) and is issued before any of the
    // batch is used, so a thread's loads overlap instead of waiting one by one.
    for (int j0 = threadIdx.x; j0 < nc * 4 * MAXQ; j0 += kTileStage * blockDim.x) {
      uint32_t v[kTileStage];
#pragma unroll
      for (int b = 0; b < kTileStage; ++b) {
        const int j = j0 + b * blockDim.x;
        const int cl = j / (4 * MAXQ), ww = j % (4 * MAXQ);
        const bool ok = j < nc * 4 * MAXQ && ww < g.W;
        v[b] = planes[ok ? ((c0 + cl) * g.np + g.np - 1) * g.W + ww : 0];
        v[b] = ok ? v[b] : 0u;
      }
#pragma unroll
      for (int b = 0; b < kTileStage; ++b)
        if (j0 + b * (int)blockDim.x < nc * 4 * MAXQ) ((uint32_t*)s_m)[j0 + b * blockDim.x] = v[b];
    }
    for (int j = threadIdx.x; j < nc; j += blockDim.x) s_live[j] = ninc[c0 + j] != 0;
    if (MODE == 0)
      for (int j0 = threadIdx.x; j0 < nc * (int)g.K; j0 += kTileStage * blockDim.x) {
        float v[kTileStage];
#pragma unroll
        for (int b = 0; b < kTileStage; ++b) {
          const int j = j0 + b * blockDim.x;
          v[b] = w[c0 * g.K + (j < nc * (int)g.K ? j : 0)];
        }
#pragma unroll
        for (int b = 0; b < kTileStage; ++b)
          if (j0 + b * (int)blockDim.x < nc * (int)g.K) s_w[j0 + b * blockDim.x] = (Sum)v[b];
      }
    const int64_t e = e0 + lane;
    const uint32_t* xr = X + (e < N ? e : N - 1) * g.W;  // lanes past N read the last sample and discard it
    uint32_t nx[4 * MAXQ];
#pragma unroll
    for (int ww = 0; ww < 4 * MAXQ; ++ww) nx[ww] = xr[ww < g.W ? ww : 0];
#pragma unroll
    for (int ww = 0; ww < 4 * MAXQ; ++ww) nx[ww] = (ww < g.W && e < N) ? ~nx[ww] : 0u;
    Sum sum[MODE == 0 ? kTileMaxK : 1];
#pragma unroll
    for (int k = 0; k < (MODE == 0 ? kTileMaxK : 1); ++k) sum[k] = 0;
    __syncthreads();
    for (int cl = 0; cl < nc; ++cl) {
      const uint4* row = s_m + cl * MAXQ;
      // Groups of up to 16 words: the group's LDS reads are issued together, the words go
      // into two independent AND-OR chains, and the wave stops once none of its samples can
      // satisfy the clause.
      uint32_t bad0 = 0u, bad1 = 0u;
#pragma unroll
      for (int q0 = 0; q0 < MAXQ; q0 += 4) {
        if (q0 < Wq && (q0 == 0 || __any((bad0 | bad1) == 0u))) {
          uint4 mv[MAXQ < 4 ? MAXQ : 4];
#pragma unroll
          for (int u = 0; u < (MAXQ < 4 ? MAXQ : 4); ++u) mv[u] = row[q0 + u];
#pragma unroll
          for (int u = 0; u < (MAXQ < 4 ? MAXQ : 4); ++u) {
            const int b = 4 * (q0 + u);
            bad0 |= mv[u].x & nx[b];
            bad1 |= mv[u].y & nx[b + 1];
            bad0 |= mv[u].z & nx[b + 2];
            bad1 |= mv[u].w & nx[b + 3];
          }
        }
      }
      const bool match = (bad0 | bad1) == 0u;
      const bool live = s_live[cl] != 0;
      if (MODE == 0) {
        const bool fire = live && match;
        if (__any(fire)) {
#pragma unroll
          for (int k = 0; k < kTileMaxK; ++k)
            if (k < g.K) sum[k] += fire ? s_w[cl * g.K + k] : (Sum)0;
        }
      } else {
        const unsigned long long bits = __ballot(!live || match);
        if (lane == 0) s_bal[wave * kTileC + cl] = bits;
      }
    }
    if (MODE == 0) {
      // the chunk's sums, stored (every value, zeros included) into its own slice
      // acc[chunk][N][K]; score_parts_finish_kernel adds the slices
      if (e < N) {
        long long* dst = acc + ((blk % nch) * N + e) * g.K;
#pragma unroll
        for (int k = 0; k < kTileMaxK; ++k)
          if (k < g.K) dst[k] = (long long)sum[k];
      }
    } else {
      __syncthreads();  // the ballots are complete
      const int rows = (int)(N - e0 < kWave ? N - e0 : kWave);
      for (int r = 0; r < rows; ++r)
        for (int cl = lane; cl < nc; cl += kWave)
          out[(e0 + r) * g.C + c0 + cl] = (uint32_t)(s_bal[wave * kTileC + cl] >> r) & 1u;
    }
  }
}

// Several patches, literal-major samples: clause outputs (transform / transform_patchwise,
// kernel.cu:346-394; an empty clause outputs 1 for every patch).  One block per (sample,
// chunk of clauses) with the sample's literal-major copy in LDS, one wave per clause: the
// firing bitmap over all patches is the AND of the included literals' bitsets (from the
// clause's literal list when it has one).  MODE 0: out[e][c] = some patch fires;
// MODE 1: out[e][c][p]; MODE 2: out[e][c][j] with bit b = patch 32j + b (0 beyond P).
// Eight waves per SIMD, as score_lm_kernel (configs 3 and 4, 1000 samples, six calls: 18.0 ->
// 13.0 ms in the kernel).
template <int MODE, int FORM>
__global__ __launch_bounds__(kScoreLmThreads) __attribute__((amdgpu_waves_per_eu(8))) void transform_lm_kernel(
    const uint32_t* __restrict__ planes, const uint16_t* __restrict__ lists, const int32_t* __restrict__ nlit,
    const uint32_t* __restrict__ XT, int64_t N, Geom g, uint32_t* __restrict__ out) {
  extern __shared__ uint32_t s_xts[];  // [L][PW]
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave)), nwv = blockDim.x / kWave;
  const int PW = (int)((g.P + 31) / 32);
  const int64_t xtw = g.L * PW;
  const int64_t nch = (g.C + kScoreLmChunk - 1) / kScoreLmChunk;
  for (int64_t blk = blockIdx.x; blk < N * nch; blk += gridDim.x) {
    const int64_t e = blk / nch, ch = blk % nch;
    const int64_t c0 = ch * kScoreLmChunk, c1 = c0 + kScoreLmChunk < g.C ? c0 + kScoreLmChunk : g.C;
    __syncthreads();  // the previous sample is no longer read
    copy_to_lds(s_xts, XT + e * xtw, xtw, threadIdx.x, blockDim.x);
    __syncthreads();
    for (int64_t c = c0 + wave; c < c1; c += nwv) {
      const int n = nlit[c];
      uint32_t fire = all_patches_word(g);
      if (n > 0) {
        if (n <= kScoreListCap) {
          const uint4 lv =
              8 * lane < n ? *(const uint4*)(lists + c * kScoreListCap + 8 * lane) : uint4{0u, 0u, 0u, 0u};
          fire = firing_from_list_regs<FORM>(g, lv, n, s_xts, fire);
        } else {
          fire = firing_from_mask(g, planes + (c * g.np + g.np - 1) * g.W, s_xts, fire);
        }
      }
      const int64_t ec = e * g.C + c;
      if (MODE == 0) {
        const bool any = __any(fire != 0u);
        if (lane == 0) out[ec] = any ? 1u : 0u;
      } else if (MODE == 2) {
        if (lane < PW) out[ec * PW + lane] = fire;
      } else {
        for (int base = 0; base < (int)g.P; base += kWave) {
          const int j = base >> 5;
          const uint32_t lo = (uint32_t)lane_value((int)fire, j);
          const uint32_t hi = j + 1 < PW ? (uint32_t)lane_value((int)fire, j + 1) : 0u;
          const uint32_t bit = lane < 32 ? (lo >> lane) & 1u : (hi >> (lane - 32)) & 1u;
          if (base + lane < (int)g.P) out[ec * g.P + base + lane] = bit;
        }
      }
    }
  }
}

// transform (kernel.cu:346-368) and transform_patchwise (kernel.cu:370-394) on the
// reference's sample layout, one wave per (sample, clause).  MODE 0: any patch; 1: per
// patch; 2: per patch, bit-packed as in transform_lm_kernel.
template <bool VANILLA, int MODE>
__global__ __launch_bounds__(256) void transform_kernel(const uint32_t* __restrict__ planes,
                                                        const int32_t* __restrict__ ninc,
                                                        const uint32_t* __restrict__ X, int64_t N, Geom g,
                                                        uint32_t* __restrict__ out) {
  const int lane = lane_id();
  const int64_t wave = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) / kWave;
  const int64_t nwaves = (int64_t)gridDim.x * blockDim.x / kWave;
  const int64_t PW = (g.P + 31) / 32;
  for (int64_t ec = wave; ec < N * g.C; ec += nwaves) {
    const int64_t e = ec / g.C, c = ec % g.C;
    const uint32_t* m = planes + (c * g.np + g.np - 1) * g.W;
    const uint32_t* xe = X + e * g.P * g.W;
    const bool empty = ninc[c] == 0;
    if (MODE == 0) {
      const bool v = empty ? true : clause_fires_any<VANILLA>(m, xe, g);
      if (lane == 0) out[ec] = v ? 1u : 0u;
    } else {
      for (int64_t base = 0; base < g.P; base += kWave) {
        const int64_t p = base + lane;
        uint32_t v = 0u;
        if (p < g.P) {
          v = 1u;
          if (!empty) {
            const uint32_t* xp = xe + p * g.W;
            for (int64_t w = 0; w < g.W; ++w)
              if (m[w] & ~xp[w]) {
                v = 0u;
                break;
              }
          }
          if (MODE == 1) out[ec * g.P + p] = v;
        }
        if (MODE == 2) {
          const unsigned long long bits = __ballot(v != 0u);
          const int64_t j = base / 32 + lane;
          if (lane < 2 && j < PW) out[ec * PW + j] = lane == 0 ? (uint32_t)bits : (uint32_t)(bits >> 32);
        }
      }
    }
  }
}

// ========================================================================= training
// Built-in instantiations of the training kernels (ytm_train.h), geometry at run time.
template <bool VANILLA, bool INJECT>
__global__ __launch_bounds__(kTrainThreads) void train_kernel(TrainArgs a) {
  train_global_body<VANILLA, INJECT>(a, a.g);
}

template <bool INJECT>
__global__ __launch_bounds__(kTrainThreads) void train_resident_kernel(TrainArgs a) {
  train_resident_body<INJECT>(a, a.g);
}

__global__ __launch_bounds__(kTrainThreads) void train_stream_kernel(TrainArgs a) { train_stream_body(a, a.g); }

// Per-sample training (one ordinary launch per sample), for clause banks (coalesced=False:
// clause c votes for and learns only its bank's class c / per_bank, kernel.cu:306-312,
// 563-565) and for models the persistent kernels do not take (more than 64 classes, or a
// grid whose state does not fit), a wave per clause at a time.  Launch i runs, for each
// clause, the feedback of sample i-1 (clause_update, kernel.cu:531-613, from the class
// totals the previous launch completed; with more than 64 classes decided and applied 64
// classes at a time, in increasing k, which is the reference's order: the decisions read
// only the evaluation's results) and then the evaluation of sample i (fast_eval and
// select_active, kernel.cu:255-316), which needs only the clause's own state: its selected
// patch and include count go to sel / ninc, its patch weight is counted and its votes added
// into sample i's class-sum row (int64).  The launch boundary orders the samples, so no
// workgroup ever waits on another.  Rows [3][K] cycle: launch i reads row (i-1) % 3, adds
// into row i % 3 and clears row (i+1) % 3, which the previous launch read and the next one
// adds into.  Launch 0 only evaluates and launch N only applies feedback.  Dynamic LDS:
// partial sums int64 [K], probabilities double [K], targets int [K] (step_lds_bytes).
template <bool ONE_PATCH, bool INJECT>
__global__ __launch_bounds__(256) void step_kernel(TrainArgs a, int i, long long* __restrict__ rows,
                                                   int* __restrict__ sel, int* __restrict__ ninc) {
  const Geom& g = a.g;
  extern __shared__ __attribute__((aligned(16))) long long step_lds[];
  long long* s_part = step_lds;                   // [K]
  double* s_prob = (double*)(s_part + g.K);       // [K]
  int* s_tgt = (int*)(s_prob + g.K);              // [K]
  __shared__ unsigned long long s_upd;
  const int lane = lane_id();
  const bool fb = i > 0, ev = i < a.N;
  const long long* sums_prev = rows + ((i + 2) % 3) * g.K;
  long long* sums_cur = rows + (i % 3) * g.K;
  long long* sums_next = rows + ((i + 1) % 3) * g.K;
  for (int64_t k = threadIdx.x; k < g.K; k += blockDim.x) {
    s_part[k] = 0;
    if (fb) class_targets(g, (int)k, sums_prev[k] + (long long)a.bias[k], a.Y + (int64_t)(i - 1) * g.K, s_tgt, s_prob);
    if (blockIdx.x == 0) sums_next[k] = 0;
  }
  if (threadIdx.x == 0) s_upd = 0ull;
  __syncthreads();
  if (fb && blockIdx.x == 0 && threadIdx.x < kWave) {  // samples where some class may update
    bool any = false;
    for (int64_t k = lane; k < g.K; k += kWave) any = any || s_prob[k] > 0.0;
    if (lane == 0 && __any(any)) atomicAdd(&a.counters[12], 1ull);
  }
  const int64_t wave0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int64_t nwaves = (int64_t)gridDim.x * blockDim.x / kWave;
  const int64_t cw = (int64_t)g.np * g.W;
  const uint64_t tp = a.step0 + (uint64_t)i - 1, t = a.step0 + (uint64_t)i;
  const float* injp = INJECT && fb ? a.inject + (int64_t)(i - 1) * a.inject_block : nullptr;
  const float* inj = INJECT && ev ? a.inject + (int64_t)i * a.inject_block : nullptr;
  const uint32_t* xp = a.X + (int64_t)(fb ? i - 1 : 0) * g.P * g.W;
  const uint32_t* xe = a.X + (int64_t)(ev ? i : 0) * g.P * g.W;
  const int64_t kspan = g.coalesced ? g.K : 1;  // classes a clause learns, 64 per decision
  for (int64_t c = wave0; c < g.C; c += nwaves) {
    if (fb && a.drop[c] != 1u) {  // a dropped clause gets no feedback (kernel.cu:555)
      const int sl = sel[c];
      bool updated = false;
      for (int64_t kc = 0; kc < kspan; kc += kWave) {
        const FbOps ops = decide<INJECT>(a, g, injp, c, tp, sl, ninc[c], s_tgt, s_prob, a.weights + c * g.K, nullptr,
                                         nullptr, false, kc);
        if ((ops.m1a | ops.m1b | ops.m2) != 0ull) {
          apply_ops<INJECT>(a, g, injp, c, tp, sl, ops, a.planes + c * cw, xp, nullptr, nullptr, 0, -1, kc);
          updated = true;
        }
      }
      if (updated) {
        if (lane == 0) atomicAdd(&s_upd, 1ull);
        __threadfence();  // the new planes (every lane's words) before the evaluation reads them
      }
    }
    if (ev) {
      const uint32_t* m = a.planes + c * cw + (int64_t)(g.np - 1) * g.W;
      int n = 0;
      const int sl = eval_select<ONE_PATCH, INJECT>(a, g, inj, c, t, m, xe, a.drop[c] == 1u, 0.0f, &n);
      if (lane == 0) {
        sel[c] = sl;
        ninc[c] = n;
        if (sl >= 0) a.patch_w[c * g.P + sl] += 1;
      }
      if (sl >= 0) {
        if (g.coalesced) {
          for (int64_t k = lane; k < g.K; k += kWave) {
            const long long v = (long long)a.weights[c * g.K + k];
            if (v != 0) atomicAdd((unsigned long long*)&s_part[k], (unsigned long long)v);
          }
        } else if (lane == 0) {
          const int64_t k = c / g.per_bank;
          atomicAdd((unsigned long long*)&s_part[k], (unsigned long long)(long long)a.weights[c * g.K + k]);
        }
      }
    }
  }
  __syncthreads();
  if (ev)
    for (int64_t k = threadIdx.x; k < g.K; k += blockDim.x)
      if (s_part[k] != 0) atomicAdd((unsigned long long*)&sums_cur[k], (unsigned long long)s_part[k]);
  if (threadIdx.x == 0 && s_upd) atomicAdd(&a.counters[0], s_upd);
}

// ========================================================================= launchers
static int grid_for(int64_t items, int block) {
  int64_t g = (items + block - 1) / block;
  if (g < 1) g = 1;
  if (g > 65536) g = 65536;
  return (int)g;
}

hipError_t launch_encode(const uint32_t* X, int64_t N, uint32_t* out, const Geom& g, hipStream_t s) {
  if (encode_staged_fits(g)) {
    if (N > 0)
      encode_staged_kernel<<<(int)(N < 65536 ? N : 65536), 256, encode_staged_lds_bytes(g), s>>>(X, N, out, g);
  } else {
    encode_kernel<<<grid_for(N * g.P * g.W, 256), 256, 0, s>>>(X, N, out, g);
  }
  return hipGetLastError();
}

hipError_t launch_transpose(const uint32_t* X, int64_t N, uint32_t* XT, const Geom& g, hipStream_t s) {
  const int64_t waves = N * g.W * ((g.P + kWave - 1) / kWave);
  transpose_kernel<<<grid_for(waves * kWave, 256), 256, 0, s>>>(X, N, g, XT);
  return hipGetLastError();
}

hipError_t launch_xt_halves_check(const uint32_t* XT, int64_t N, const Geom& g, int* ok, hipStream_t s) {
  xt_halves_kernel<<<grid_for(N * g.Lh * ((g.P + 31) / 32), 256), 256, 0, s>>>(XT, N, g, ok);
  return hipGetLastError();
}

hipError_t launch_ta_to_planes(const uint32_t* ta, uint32_t* planes, const Geom& g, hipStream_t s) {
  ta_to_planes_kernel<<<grid_for(g.C * g.W, 256), 256, 0, s>>>(ta, planes, g);
  return hipGetLastError();
}

hipError_t launch_planes_to_ta(const uint32_t* planes, uint32_t* ta, const Geom& g, hipStream_t s) {
  planes_to_ta_kernel<<<grid_for(g.C * g.L, 256), 256, 0, s>>>(planes, ta, g);
  return hipGetLastError();
}

hipError_t launch_init_state(uint32_t* planes, float* w, const Geom& g, uint64_t seed, hipStream_t s) {
  const int64_t n = g.C * g.W > g.C * g.K ? g.C * g.W : g.C * g.K;
  init_state_kernel<<<grid_for(n, 256), 256, 0, s>>>(planes, w, g, seed);
  return hipGetLastError();
}

hipError_t launch_ninc(const uint32_t* planes, int32_t* ninc, const Geom& g, hipStream_t s) {
  ninc_kernel<<<grid_for(g.C * kWave, 256), 256, 0, s>>>(planes, ninc, g);
  return hipGetLastError();
}

hipError_t launch_fill_u64(unsigned long long* p, int64_t n, hipStream_t s) {
  fill_u64_kernel<<<grid_for(n, 256), 256, 0, s>>>(p, n);
  return hipGetLastError();
}

// One patch, clauses wider than 16 words (score_wide_fits): a block takes kWideTile
// samples and every clause.  The samples are transposed in LDS into one word per literal
// (bit s: the literal is 1 in sample e0 + s), 32 ballots per pair of sample words.  A lane
// takes a clause and ANDs the words of its included literals, 8 per step from its literal
// list, stopping once no sample of the tile is left; the tile's samples that the clause
// fires on get its weights in LDS int64 sums (calc_class_sums_infer_batch, kernel.cu:319-343:
// empty clauses do not vote).  Clauses with more literals than the list holds are AND-ed
// by the whole wave from their include masks.  With few tiles the clauses are split into
// nch chunks over blocks; each block adds its chunk's exact sums into acc[e][k] (zeroed
// before the launch).  OUT: clause outputs instead (transform and transform_patchwise with
// their single patch, kernel.cu:346-394: an empty clause outputs 1), out[e][c], written by
// the clause's lane for each sample of the tile.
constexpr int kWideTile = 32;
constexpr int64_t kWideLdsBytes = 96 * 1024;

// MMA: class votes on the matrix cores (K >= 4; fewer classes keep the LDS atomics, and
// their kernel the registers of that path alone).
template <bool OUT, bool MMA = false>
__global__ __launch_bounds__(1024) void wide_kernel(const uint32_t* __restrict__ planes,
                                                    const uint16_t* __restrict__ lists,
                                                    const int32_t* __restrict__ nlit, const float* __restrict__ w,
                                                    const uint32_t* __restrict__ X, int64_t N, Geom g, int64_t nch,
                                                    long long* __restrict__ acc, uint32_t* __restrict__ out) {
  extern __shared__ uint32_t s_xw[];  // [W * 32]: word l = literal l over the tile's samples
  __shared__ long long s_sum[kWideTile * kTileMaxK];
  __shared__ __attribute__((aligned(16))) uint32_t s_fw[MMA ? 16 * kWave : 1];  // each wave's fire masks
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave, nwv = blockDim.x / kWave;
  const int sl = lane & 31, half = lane >> 5;  // transpose: sample sl of word 2 * pair + half
  const int64_t ntile = (N + kWideTile - 1) / kWideTile;
  const int64_t csz = ((g.C + nch - 1) / nch + kWave - 1) / kWave * kWave;  // clauses per chunk, whole waves
  for (int64_t blk = blockIdx.x; blk < ntile * nch; blk += gridDim.x) {
    const int64_t tile = blk / nch, cb = (blk % nch) * csz;
    const int64_t ce = cb + csz < g.C ? cb + csz : g.C;
    const int64_t e0 = tile * kWideTile;
    const int ns = (int)(N - e0 < kWideTile ? N - e0 : kWideTile);
    __syncthreads();  // the previous tile is no longer read
    for (int j = threadIdx.x; j < kWideTile * (int)g.K; j += blockDim.x) s_sum[j] = 0;
    for (int64_t pair = wave; pair < (g.W + 1) / 2; pair += nwv) {
      const int64_t wd = 2 * pair + half;
      const bool ok = wd < g.W && sl < ns;
      const uint32_t xr = X[(e0 + (sl < ns ? sl : 0)) * g.W + (wd < g.W ? wd : 0)];  // clamped, unconditional
      const uint32_t x = ok ? xr : 0u;
      uint32_t mine = 0u;
#pragma unroll
      for (int b = 0; b < 32; ++b) {
        const unsigned long long bal = __ballot((x >> b) & 1u);
        const uint32_t part = half ? (uint32_t)(bal >> 32) : (uint32_t)bal;
        mine = sl == b ? part : mine;
      }
      if (wd < g.W) s_xw[wd * 32 + sl] = mine;  // literal 32 * wd + sl
    }
    __syncthreads();
    const uint32_t live = ns == 32 ? 0xFFFFFFFFu : ((1u << ns) - 1u);
    const int np = g.np;
    for (int64_t c0 = cb + (int64_t)wave * kWave; c0 < ce; c0 += (int64_t)nwv * kWave) {
      const int64_t c = c0 + lane;
      const int n = c < ce ? nlit[c] : 0;
      uint32_t fire = (OUT && n == 0) ? live : 0u;  // empty clauses: output 1, no vote
      if (n > 0 && n <= kScoreListCap) {
        fire = live;
        const uint16_t* lst = lists + c * kScoreListCap;
        for (int j = 0; j < n && fire; j += 8) {  // the list is padded to a multiple of 8
          const uint4 q = *(const uint4*)(lst + j);
          fire &= s_xw[q.x & 0xFFFFu] & s_xw[q.x >> 16] & s_xw[q.y & 0xFFFFu] & s_xw[q.y >> 16] &
                  s_xw[q.z & 0xFFFFu] & s_xw[q.z >> 16] & s_xw[q.w & 0xFFFFu] & s_xw[q.w >> 16];
        }
      }
      if (!OUT) {
        // The wave's votes as one product on the matrix cores: sums[sample][k] = sum over
        // its 64 clauses of fire[sample][clause] * w[clause][k], eight clauses per
        // v_mfma_f32_32x32x8f16 (A: lane l row l % 32 = sample, B: lane l column l % 32 =
        // class, both with clauses 4 * (l / 32) + 0..3 of the step; D: lane l column
        // l % 32, rows 8 * (r / 4) + 4 * (l / 32) + r % 4).  Weights are integer-valued
        // (ytm_set_weights refuses others; training moves them by 1), so the product is exact
        // while every weight of the wave is at most 2048 in magnitude (f16 holds it, and
        // 64 * 2048 < 2^24 keeps the f32 sums exact); otherwise the firing samples' weights
        // go in one by one.
        const int K = (int)g.K;
        bool lane_ok = MMA;  // every weight this lane loads is within 2048
        typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
        typedef float float16_t __attribute__((ext_vector_type(16)));
        float16_t d;
#pragma unroll
        for (int r = 0; r < 16; ++r) d[r] = 0.0f;
        const int col = lane & 31, kq = 4 * (lane >> 5);
        if (MMA) {
          s_fw[wave * kWave + lane] = fire;
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
          __builtin_amdgcn_wave_barrier();
#pragma unroll 2
          for (int st = 0; st < kWave / 8; ++st) {
            const uint4 f4 = *(const uint4*)&s_fw[wave * kWave + 8 * st + kq];
            half4_t av, bv;
            av[0] = (_Float16)(float)((f4.x >> col) & 1u);
            av[1] = (_Float16)(float)((f4.y >> col) & 1u);
            av[2] = (_Float16)(float)((f4.z >> col) & 1u);
            av[3] = (_Float16)(float)((f4.w >> col) & 1u);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int64_t cc = c0 + 8 * st + kq + j;
              const float wf = cc < ce && col < K ? w[cc * g.K + col] : 0.0f;
              lane_ok = lane_ok && fabsf(wf) <= 2048.0f;
              bv[j] = (_Float16)wf;
            }
            d = __builtin_amdgcn_mfma_f32_32x32x8f16(av, bv, d, 0, 0, 0);
          }
        }
        if (__all(lane_ok)) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = 8 * (r >> 2) + kq + (r & 3);
            if (col < K && row < ns && d[r] != 0.0f)
              atomicAdd((unsigned long long*)&s_sum[row * g.K + col], (unsigned long long)(long long)d[r]);
          }
        } else if (fire) {
          for (int k = 0; k < K; ++k) {
            const long long v = (long long)w[c * g.K + k];
            for (uint32_t f = fire; f; f &= f - 1u)
              atomicAdd((unsigned long long*)&s_sum[(__ffs((int)f) - 1) * g.K + k], (unsigned long long)v);
          }
        }
      }
      unsigned long long over = __ballot(n > kScoreListCap);
      while (over) {  // wide clauses: the whole wave walks the include mask
        const int src = __ffsll((long long)over) - 1;
        over &= over - 1ull;
        const int64_t cc = c0 + src;
        const uint32_t* m = planes + (cc * np + np - 1) * g.W;
        uint32_t f2 = live;
        for (int64_t wb = 0; wb < g.W; wb += kWave) {
          const int64_t wd = wb + lane;
          for (uint32_t mw = wd < g.W ? m[wd] : 0u; mw; mw &= mw - 1u) f2 &= s_xw[wd * 32 + __ffs((int)mw) - 1];
        }
        for (int off = 32; off > 0; off >>= 1) f2 &= (uint32_t)__shfl_xor((int)f2, off);
        if (OUT && lane == src) fire = f2;
        if (!OUT && f2 && lane < g.K) {
          const long long v = (long long)w[cc * g.K + lane];
          for (uint32_t f = f2; f; f &= f - 1u)
            atomicAdd((unsigned long long*)&s_sum[(__ffs((int)f) - 1) * g.K + lane], (unsigned long long)v);
        }
      }
      if (OUT && c < ce)
        for (int sm = 0; sm < ns; ++sm) out[(e0 + sm) * g.C + c] = (fire >> sm) & 1u;
    }
    if (!OUT) {
      __syncthreads();
      for (int j = threadIdx.x; j < ns * (int)g.K; j += blockDim.x)
        if (s_sum[j] != 0) atomicAdd((unsigned long long*)&acc[e0 * g.K + j], (unsigned long long)s_sum[j]);
    }
  }
}

template <int MODE, bool SUM32>
static hipError_t launch_tile(const uint32_t* planes, const int32_t* ninc, const float* w, const uint32_t* X,
                              int64_t N, const Geom& g, long long* acc, uint32_t* out, hipStream_t s) {
  const int64_t blocks = ((N + 255) / 256) * ((g.C + kTileC - 1) / kTileC);
  const int grid = blocks < 65536 ? (int)blocks : 65536;
  if (g.W <= 4)
    tile_kernel<1, MODE, SUM32><<<grid, 256, 0, s>>>(planes, ninc, w, X, N, g, acc, out);
  else if (g.W <= 16)
    tile_kernel<4, MODE, SUM32><<<grid, 256, 0, s>>>(planes, ninc, w, X, N, g, acc, out);
  else
    tile_kernel<16, MODE, SUM32><<<grid, 256, 0, s>>>(planes, ninc, w, X, N, g, acc, out);
  return hipGetLastError();
}

static bool tile_fits(const Geom& g, int mode) {
  return g.P == 1 && g.W <= 64 && (mode == 1 || g.K <= kTileMaxK);
}

// Scratch of the list-based scorers: lists [C][kScoreListCap] uint16, include counts [C]
// int32, literal order [kOrderBuckets][W] uint32.
static size_t lists_scratch_bytes(const Geom& g) {
  return (size_t)g.C * kScoreListCap * 2 + (size_t)g.C * 4 + (size_t)kOrderBuckets * g.W * 4;
}
struct ListScratch {
  uint16_t* lists;
  int32_t* nlit;
  uint32_t* order;
};
static ListScratch list_scratch(void* scratch, const Geom& g) {
  ListScratch r;
  r.lists = (uint16_t*)scratch;
  r.nlit = (int32_t*)(r.lists + g.C * kScoreListCap);
  r.order = (uint32_t*)(r.nlit + g.C);
  return r;
}

size_t score_lists_bytes(const Geom& g) {
  if (!literal_major(g) || g.L > 65535 || (size_t)(g.L * ((g.P + 31) / 32)) * 4 > 120 * 1024) return 0;
  return lists_scratch_bytes(g);
}

size_t score_wide_bytes(const Geom& g) { return score_wide_fits(g) ? lists_scratch_bytes(g) : 0; }

// Literal order from the batch, then the lists in that order: several patches (XT given),
// whose walks end at the first AND over all patches that is empty (config 4: 149K -> 244K
// samples/s with the two-half test).  One-patch lists (wide_kernel, lanes = clauses over a
// tile of 32 samples) stay in literal index order, which measured faster there (config 2:
// 149M against 135M samples/s).  YTM_LIST_ORDER=0: index order everywhere.
static hipError_t build_lists(const uint32_t* planes, const uint32_t* X, const uint32_t* XT, int64_t N,
                              const Geom& g, const ListScratch& ls, hipStream_t s) {
  const char* env = std::getenv("YTM_LIST_ORDER");
  const bool ordered = XT != nullptr && !(env && std::atoi(env) == 0);
  if (ordered) {
    hipError_t e = launch_literal_order(X, XT, N, g, ls.order, s);
    if (e != hipSuccess) return e;
  }
  build_lists_kernel<<<grid_for(g.C * kWave, 256), 256, 0, s>>>(planes, g, kScoreListCap, ordered ? ls.order : nullptr,
                                                                  ls.lists, ls.nlit);
  return hipGetLastError();
}

hipError_t launch_score_lm(const uint32_t* planes, const float* w, const uint32_t* XT, int64_t N, const Geom& g,
                           void* scratch, long long* acc, hipStream_t s) {
  const ListScratch ls = list_scratch(scratch, g);
  hipError_t err = build_lists(planes, nullptr, XT, N, g, ls, s);
  if (err != hipSuccess) return err;
  uint16_t* lists = ls.lists;
  int32_t* nlit = ls.nlit;
  const int64_t chunk = score_lm_chunk(g, N);
  const int64_t blocks = N * ((g.C + chunk - 1) / chunk);
  const int grid = blocks < 65536 ? (int)blocks : 65536;
  const size_t lds = (size_t)(g.L * ((g.P + 31) / 32)) * 4;
  // the sample fits LDS (score_lists_bytes), so its word offsets fit 16 bits: no kListIndex
  if (list_form(g) == kListBytes)
    score_lm_kernel<kListBytes><<<grid, score_lm_threads(g), lds, s>>>(planes, lists, nlit, w, XT, N, g, chunk, acc);
  else
    score_lm_kernel<kListWords><<<grid, score_lm_threads(g), lds, s>>>(planes, lists, nlit, w, XT, N, g, chunk, acc);
  return hipGetLastError();
}

bool score_wide_fits(const Geom& g) {
  // From 17 words on, the literal lists beat the sample tiles held in registers (config 2,
  // 49 words: 167M against 70M samples/s in the kernel); narrower clauses keep the tiles.
  return g.P == 1 && g.W > 16 && g.K <= kTileMaxK && g.L <= 65535 && g.W * 32 * 4 <= kWideLdsBytes;
}

hipError_t launch_score_wide(const uint32_t* planes, const float* w, const uint32_t* X, int64_t N, const Geom& g,
                             void* scratch, bool lists_ready, long long* acc, hipStream_t s) {
  const ListScratch ls = list_scratch(scratch, g);
  if (!lists_ready) {
    hipError_t err = build_lists(planes, X, nullptr, N, g, ls, s);
    if (err != hipSuccess) return err;
  }
  uint16_t* lists = ls.lists;
  int32_t* nlit = ls.nlit;
  // enough blocks to fill the device (two per CU fit): split the clauses when tiles are few
  const int64_t tiles = (N + kWideTile - 1) / kWideTile;
  const int64_t want = (512 + tiles - 1) / tiles, most = (g.C + 1023) / 1024;
  const int64_t nch = want < most ? want : most;
  const int64_t blocks = tiles * (nch > 0 ? nch : 1);
  const int grid = blocks < 65536 ? (int)blocks : 65536;
  // 512 threads when two such blocks fit a CU's LDS: at 92 VGPRs a CU holds 20 waves, so one
  // 1024-thread block or two of 512, whose transposes, barriers and walks then overlap
  // (config 2, 6 KB per block: 159M -> 178M samples/s in the kernel); a transposed tile
  // above 64 KB keeps 1024 (config 5, 80 KB: one 512-thread block per CU would halve the
  // waves, 2.0M -> 1.05M).
  const size_t lds = (size_t)(g.W * 32) * 4;
  const int threads = lds <= 64 * 1024 ? 512 : 1024;
  if (g.K >= 4)  // votes on the matrix cores: config 2 inference 187M -> 234M samples/s in the kernel
    wide_kernel<false, true><<<grid, threads, lds, s>>>(planes, lists, nlit, w, X, N, g, nch > 0 ? nch : 1, acc, nullptr);
  else
    wide_kernel<false><<<grid, threads, lds, s>>>(planes, lists, nlit, w, X, N, g, nch > 0 ? nch : 1, acc, nullptr);
  return hipGetLastError();
}

hipError_t launch_transform_wide(const uint32_t* planes, const uint32_t* X, int64_t N, const Geom& g, void* scratch,
                                 bool lists_ready, uint32_t* out, hipStream_t s) {
  const ListScratch ls = list_scratch(scratch, g);
  if (!lists_ready) {
    hipError_t err = build_lists(planes, X, nullptr, N, g, ls, s);
    if (err != hipSuccess) return err;
  }
  uint16_t* lists = ls.lists;
  int32_t* nlit = ls.nlit;
  const int64_t tiles = (N + kWideTile - 1) / kWideTile;
  const int64_t want = (512 + tiles - 1) / tiles, most = (g.C + 1023) / 1024;
  const int64_t nch = want < most ? want : most;
  const int64_t blocks = tiles * (nch > 0 ? nch : 1);
  const int grid = blocks < 65536 ? (int)blocks : 65536;
  wide_kernel<true><<<grid, 1024, (size_t)(g.W * 32) * 4, s>>>(planes, lists, nlit, nullptr, X, N, g,
                                                                nch > 0 ? nch : 1, nullptr, out);
  return hipGetLastError();
}

int64_t score_tile_chunks(const Geom& g) { return tile_fits(g, 0) ? (g.C + kTileC - 1) / kTileC : 0; }

hipError_t launch_score_tile(const uint32_t* planes, const int32_t* ninc, const float* w, const uint32_t* X,
                             int64_t N, const Geom& g, long long* parts, double w_bound, hipStream_t s) {
  const bool sum32 = w_bound * kTileC < 2147483648.0;
  return sum32 ? launch_tile<0, true>(planes, ninc, w, X, N, g, parts, nullptr, s)
               : launch_tile<0, false>(planes, ninc, w, X, N, g, parts, nullptr, s);
}

hipError_t launch_score_parts_finish(const long long* parts, int64_t nch, const float* bias, int64_t N, const Geom& g,
                                     float* out, hipStream_t s) {
  score_parts_finish_kernel<<<grid_for(N * g.K, 256), 256, 0, s>>>(parts, nch, bias, N, g, out);
  return hipGetLastError();
}

hipError_t launch_score(const uint32_t* planes, const int32_t* ninc, const float* w, const uint32_t* X,
                        int64_t N, const Geom& g, long long* acc, hipStream_t s) {
  if (g.P == 1 && g.K <= kScoreTileMaxK && (size_t)g.W * kScoreTile * 4 <= 48 * 1024) {
    const int64_t blocks = ((N + kScoreTile - 1) / kScoreTile) * ((g.C + kScoreTileChunk - 1) / kScoreTileChunk);
    const int grid = blocks < 65536 ? (int)blocks : 65536;
    score_tile_kernel<<<grid, 256, (size_t)g.W * kScoreTile * 4, s>>>(planes, ninc, w, X, N, g, acc);
    return hipGetLastError();
  }
  const int64_t blocks = N * ((g.C + kScoreChunk - 1) / kScoreChunk);
  const int grid = blocks < 65536 ? (int)blocks : 65536;
  if (g.K > kWave) {
    const size_t lds = (size_t)g.K * 8;
    if (g.P == 1)
      score_classes_kernel<true><<<grid, 256, lds, s>>>(planes, ninc, w, X, N, g, acc);
    else
      score_classes_kernel<false><<<grid, 256, lds, s>>>(planes, ninc, w, X, N, g, acc);
    return hipGetLastError();
  }
  if (g.P == 1)
    score_kernel<true><<<grid, 256, 0, s>>>(planes, ninc, w, X, N, g, acc);
  else
    score_kernel<false><<<grid, 256, 0, s>>>(planes, ninc, w, X, N, g, acc);
  return hipGetLastError();
}

hipError_t launch_score_finish(const long long* acc, const float* bias, int64_t N, const Geom& g, float* out,
                               hipStream_t s) {
  score_finish_kernel<<<grid_for(N * g.K, 256), 256, 0, s>>>(acc, bias, N, g, out);
  return hipGetLastError();
}

hipError_t launch_transform(const uint32_t* planes, const int32_t* ninc, const uint32_t* X, int64_t N,
                            const Geom& g, int mode, uint32_t* out, hipStream_t s) {
  if (tile_fits(g, 1)) return launch_tile<1, false>(planes, ninc, nullptr, X, N, g, nullptr, out, s);
  const int grid = grid_for(N * g.C * kWave, 256);
  if (g.P == 1) {
    // One patch: per-patch output (packed or not) is the clause output.
    transform_kernel<true, 0><<<grid, 256, 0, s>>>(planes, ninc, X, N, g, out);
  } else if (mode == 0) {
    transform_kernel<false, 0><<<grid, 256, 0, s>>>(planes, ninc, X, N, g, out);
  } else if (mode == 1) {
    transform_kernel<false, 1><<<grid, 256, 0, s>>>(planes, ninc, X, N, g, out);
  } else {
    transform_kernel<false, 2><<<grid, 256, 0, s>>>(planes, ninc, X, N, g, out);
  }
  return hipGetLastError();
}

hipError_t launch_transform_lm(const uint32_t* planes, const uint32_t* XT, int64_t N, const Geom& g, int mode,
                               void* scratch, bool lists_ready, uint32_t* out, hipStream_t s) {
  const ListScratch ls = list_scratch(scratch, g);
  if (!lists_ready) {
    hipError_t err = build_lists(planes, nullptr, XT, N, g, ls, s);
    if (err != hipSuccess) return err;
  }
  uint16_t* lists = ls.lists;
  int32_t* nlit = ls.nlit;
  const int64_t blocks = N * ((g.C + kScoreLmChunk - 1) / kScoreLmChunk);
  const int grid = blocks < 65536 ? (int)blocks : 65536;
  const size_t lds = (size_t)(g.L * ((g.P + 31) / 32)) * 4;
  const int th = score_lm_threads(g);
  const bool bytes = list_form(g) == kListBytes;  // else kListWords: the sample fits LDS
  if (mode == 0) {
    if (bytes) transform_lm_kernel<0, kListBytes><<<grid, th, lds, s>>>(planes, lists, nlit, XT, N, g, out);
    else transform_lm_kernel<0, kListWords><<<grid, th, lds, s>>>(planes, lists, nlit, XT, N, g, out);
  } else if (mode == 1) {
    if (bytes) transform_lm_kernel<1, kListBytes><<<grid, th, lds, s>>>(planes, lists, nlit, XT, N, g, out);
    else transform_lm_kernel<1, kListWords><<<grid, th, lds, s>>>(planes, lists, nlit, XT, N, g, out);
  } else {
    if (bytes) transform_lm_kernel<2, kListBytes><<<grid, th, lds, s>>>(planes, lists, nlit, XT, N, g, out);
    else transform_lm_kernel<2, kListWords><<<grid, th, lds, s>>>(planes, lists, nlit, XT, N, g, out);
  }
  return hipGetLastError();
}

int train_rng_slots(int cpw, const Geom& g) {
  const size_t per_slot = (size_t)g.W * kPreGroups * 4 * sizeof(uint32_t) + 2 * sizeof(int);
  const size_t base = train_lds_bytes(TrainKind::kResident, cpw, 0, g);
  const size_t left = base < kResidentLdsLimit ? kResidentLdsLimit - base : 0;
  const size_t budget = std::min<size_t>(48 * 1024, left);
  return (int)std::max<size_t>(1, std::min<size_t>((size_t)cpw * g.K, budget / per_slot));
}

size_t train_lds_bytes(TrainKind kind, int cpw, int rng_slots, const Geom& g) {
  // literal lists (several patches): include counts [cpw, rounded to even] and lists [cpw][cap] u16
  const size_t cap = g.P > 1 ? (size_t)g.list_cap : 0;
  const size_t lists = cap > 0 ? (size_t)2 * ((cpw + 1) / 2) * 4 + (size_t)cpw * cap * 2 : 0;
  if (kind != TrainKind::kResident)  // task masks [cpw][3] u64; sel, ninc [2][cpw]; task clause / slot [cpw];
                                     // sample [L][PW]; with mask_lds include masks [cpw][W] and samples
                                     // [2][W]; weights [cpw][K]; drop flags [cpw]; with several
                                     // patches the reservoir thresholds [P+1] and rank bits [2][cpw]
    return (size_t)3 * cpw * 8 + (size_t)6 * cpw * sizeof(int) + lists +
           (literal_major_lds(g) ? (size_t)(g.L * ((g.P + 31) / 32)) * 4 : 0) +
           (g.mask_lds ? (size_t)(cpw + 2) * g.W * 4 : 0) + (size_t)cpw * g.K * 4 + (size_t)cpw * 4 +
           (g.P > 1 ? (size_t)(g.P + 1) * 4 + (size_t)2 * cpw * 4 : 0);
  // Resident kernel (layout of train_resident_body): task masks [cpw][3] u64; planes
  // [cpw][np][W]; weights [cpw][K]; samples [3][W]; sel, ninc [2][cpw]; drop, patch
  // weights [cpw]; targets [3][K]; bias [K]; rank-1 draws [3][cpw]; Q-skip and update
  // draws [3][cpw][K] each; task clause / first slot [cpw]; staged task weights [cpw][K];
  // slot clause / class [R]; slot plane groups [R][W][kPreGroups][4].
  // Several patches add the literal-major samples [2][L][PW] after the task masks and the
  // reservoir thresholds [P+1] at the end.
  const size_t C = (size_t)cpw, K = (size_t)g.K, W = (size_t)g.W, R = (size_t)rng_slots;
  const size_t xt = g.P > 1 ? (size_t)(2 * g.L * ((g.P + 31) / 32)) * 4 : 0;
  return 3 * C * 8 + lists + xt + C * (size_t)g.np * W * 4 + C * K * 4 + 3 * W * 4 + 4 * C * 4 + 2 * C * 4 + 3 * K * 4 +
         K * 4 + 3 * C * 4 + 6 * C * K * 4 + 2 * C * 4 + C * K * 4 + 2 * R * 4 + R * W * kPreGroups * 4 * 4 +
         (g.P > 1 ? (size_t)(g.P + 1) * 4 : 0);  // reservoir thresholds [P+1]
}

size_t stream_lds_bytes(const Geom& g, int threads) {
  // layout of train_stream_body: task masks [64][3] u64; planes [64][np][W]; weights [64][K]
  // f32 and [K][64] i32; include counts, drop, patch weights, task clauses, zeros, stop
  // selections [64] i32 each; targets ring [depth][K]; complemented samples ring [depth][Wp];
  // integer weights before a stop [K][64]; word-major include masks [Wp][64]
  (void)threads;
  const size_t C = kStreamClauses, K = (size_t)g.K, Wp = (size_t)((g.W + 3) & ~(int64_t)3);
  return 3 * C * 8 + C * (size_t)g.np * (size_t)g.W * 4 + 2 * C * K * 4 + 6 * C * 4 + (size_t)kStreamDepth * K * 4 +
         (size_t)kStreamDepth * Wp * 4 + K * C * 4 + Wp * C * 4 + (g.vote_table ? stream_vote_table_bytes(g) : 0);
}

// the vote nibble tables [16][16][K] (16-bit) of train_stream_body
size_t stream_vote_table_bytes(const Geom& g) { return (size_t)kStreamClauses / 4 * 16 * (size_t)g.K * 2; }

static const void* train_fn(TrainKind kind, bool inject) {
  switch (kind) {
    case TrainKind::kStream:
      return (const void*)train_stream_kernel;
    case TrainKind::kResident:
      return inject ? (const void*)train_resident_kernel<true> : (const void*)train_resident_kernel<false>;
    case TrainKind::kGlobalVanilla:
      return inject ? (const void*)train_kernel<true, true> : (const void*)train_kernel<true, false>;
    default:
      return inject ? (const void*)train_kernel<false, true> : (const void*)train_kernel<false, false>;
  }
}

hipError_t train_occupancy(TrainKind kind, bool inject, size_t lds_bytes, int* blocks_per_cu) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, train_fn(kind, inject), kTrainThreads,
                                                      lds_bytes);
}

hipError_t launch_train(const TrainArgs& a, int grid, size_t lds_bytes, TrainKind kind, bool inject,
                        hipStream_t s) {
  TrainArgs copy = a;
  void* args[] = {&copy};
  return hipLaunchCooperativeKernel(train_fn(kind, inject), dim3(grid), dim3(kTrainThreads), args,
                                    (unsigned)lds_bytes, s);
}

size_t step_lds_bytes(const Geom& g) { return (size_t)g.K * (8 + 8 + 4); }

hipError_t launch_step(const TrainArgs& a, int i, long long* rows, int* sel, int* ninc, bool inject, hipStream_t s) {
  const int grid = grid_for(a.g.C * kWave, 256);
  const bool one = a.g.P == 1;
  const size_t lds = step_lds_bytes(a.g);
  if (one && inject)
    step_kernel<true, true><<<grid, 256, lds, s>>>(a, i, rows, sel, ninc);
  else if (one)
    step_kernel<true, false><<<grid, 256, lds, s>>>(a, i, rows, sel, ninc);
  else if (inject)
    step_kernel<false, true><<<grid, 256, lds, s>>>(a, i, rows, sel, ninc);
  else
    step_kernel<false, false><<<grid, 256, lds, s>>>(a, i, rows, sel, ninc);
  return hipGetLastError();
}

}  // namespace ytm
