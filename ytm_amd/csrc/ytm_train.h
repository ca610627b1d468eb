// ytm_train.h -- device code of the YTM training kernels (gfx950).
//
// Included by the built-in kernels (ytm_kernels.hip) with the model geometry read from
// the kernel arguments, and compiled again at run time by hipRTC (ytm_jit.hip) with the
// geometry as a constexpr Geom, so that every size and hyperparameter folds to a
// constant.  Every function takes the geometry as `const Geom& g`.
#pragma once
#include "ytm_device.h"
#include "ytm_types.h"

namespace ytm {

// ========================================================================= training
// Persistent, cooperative kernel: one launch trains N consecutive samples.
// Workgroup b owns clauses [C*b/G, C*(b+1)/G) for the whole launch.  Per sample:
//   A. each wave takes own clauses: include mask (top plane) vs the sample, all patches
//      (fast_eval, kernel.cu:255-282), reservoir choice of the firing patch
//      (select_active, kernel.cu:285-316), patch weight, partial class sums in LDS;
//   B. the workgroup adds (1<<44 | partial) into its group's word of the sample's
//      class-sum row; a two-level tree of agent-scope atomics completes the sum and a
//      mailbox per group broadcasts it back (exchange_class_sums);
//   C. clip / target / update probability per class (kernel.cu:397,508-529,543-551);
//   D. feedback on own clauses (clause_update, kernel.cu:531-613): per class in order,
//      Q-skip and update draws, Type Ia / Ib / II, weight update, and the literal updates
//      applied bit-sliced to the clause's planes, 32 literals per lane.
// The only cross-workgroup traffic is the K class sums of each sample.

// Bounded wait for the class sums: at most kWaitTicks of the 100 MHz real-time counter
// (2 s), independent of how long one poll takes under contention.
constexpr uint64_t kWaitTicks = 200000000ull;

// The counter-stream words of a draw site (site_words).  With a.profile == 4 (counting
// runs) the lanes that compute a site are added up per kind: counters[3] Q-skip / update
// draws, [14] reservoir draws, [15] literal draws.  The counting is compiled in unless
// YTM_COUNT_DRAWS is 0 (kernels compiled per model leave it out of runs that do not count).
#ifndef YTM_COUNT_DRAWS
#define YTM_COUNT_DRAWS 1
#endif
__device__ __forceinline__ U4 counted_site(const TrainArgs& a, uint64_t t, uint32_t c, uint32_t tag, uint32_t site) {
  if (YTM_COUNT_DRAWS && a.profile == 4) {
    const unsigned long long m = __ballot(1);
    if ((int)(threadIdx.x & (kWave - 1)) == __ffsll((long long)m) - 1)
      atomicAdd(&a.counters[tag == TAG_LIT ? 15 : (tag == TAG_SEL ? 14 : 3)], (unsigned long long)__popcll(m));
  }
  return site_words(a.seed, t, c, tag, site);
}

// Plane groups (4 planes each, most significant first) of the literal draws that the
// resident kernel computes cooperatively ahead of applying an update.
constexpr int kPreGroups = 3;

// Plane groups that decide u <= S_INV, i.e. q < s_thr for the 24-bit integer q of a literal
// draw, taken most significant plane first.  Below the lowest set bit of s_thr nothing more
// can make q < s_thr: a literal still equal to s_thr on the planes above it is decided
// "not less", so only the groups down to that bit matter (one group for s_thr = 2^23,
// S_INV = 0.5).  None for s_thr = 0 or >= 2^24, which are decided without draws.
__device__ __forceinline__ int draw_groups(uint32_t s_thr) {
  return (s_thr == 0u || s_thr >= (1u << 24)) ? 0 : (23 - __builtin_ctz(s_thr)) / 4 + 1;
}

__device__ __forceinline__ int wave_inclusive_scan(int v) { return wave_scan_add_i32(v); }

// Literal-decrement mask of one (clause, class) update for the 32 literals of word w:
// bit b set iff need bit b is set and u(literal 32w+b) <= S_INV.
template <bool INJECT>
__device__ __forceinline__ uint32_t literal_draw_mask(const TrainArgs& a, const Geom& g, const float* inj, uint32_t need,
                                                      uint64_t t, int64_t c, int64_t k, int64_t w,
                                                      const uint32_t* pre, bool have_pre) {
  if (INJECT) {
    uint32_t res = 0u;
    if (need) {
      const float* u = inj + g.C * g.P + 2 * g.C * g.K + (c * g.K + k) * g.L + w * 32;
      for (int b = 0; b < 32; ++b)
        if (((need >> b) & 1u) && (double)u[b] <= g.s_inv) res |= 1u << b;
    }
    return res;
  } else {
    // u <= S_INV  <=>  q < s_thr for the 24-bit integer q of the literal; decided from the
    // most significant plane down, 4 planes per Philox call, until no lane of the wave
    // has an undecided literal.
    if (g.s_thr >= (1u << 24)) return need;
    if (g.s_thr == 0u) return 0u;
    uint32_t lt = 0u, eq = need;
    bool done = false;
    const int ngrp = draw_groups(g.s_thr);
#pragma unroll
    for (int grp = 0; grp < 6; ++grp) {  // unrolled (no break), which schedules the Philox rounds better
      if (done || grp >= ngrp) continue;
      if (!__any(eq != 0u)) {
        done = true;
        continue;
      }
      // a plane group computed ahead of time by the workgroup (zero words for idle lanes)
      const U4 z = (have_pre && grp < kPreGroups)
                       ? (pre ? U4{pre[grp * 4 + 0], pre[grp * 4 + 1], pre[grp * 4 + 2], pre[grp * 4 + 3]}
                              : U4{0u, 0u, 0u, 0u})
                       : counted_site(a, t, (uint32_t)c, TAG_LIT, (uint32_t)((k * g.W + w) * 6 + grp));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = 23 - 4 * grp - i;
        const uint32_t pl = word_of(z, i);
        if ((g.s_thr >> j) & 1u) {
          lt |= eq & ~pl;
          eq &= pl;
        } else {
          eq &= ~pl;
        }
      }
    }
    return lt;
  }
}

// The outcomes of ranks 1-4 of a clause's reservoir draws (the first Philox call of its
// TAG_SEL site): bit r - 1 set when the draw of rank r is below 1.0f / r (r <= P).  Computed
// by one lane per clause ahead of phase A, so that reservoir_rank needs no Philox call for
// clauses firing on at most 4 patches.
__device__ __forceinline__ int rank_bits(const TrainArgs& a, const Geom& g, int64_t c, uint64_t t,
                                         const float* inv_rank) {
  const U4 z = counted_site(a, t, (uint32_t)c, TAG_SEL, 0u);
  int m = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (j + 1 <= g.P && uniform_from_word(word_of(z, j)) < inv_rank[j + 1]) m |= 1 << j;
  return m;
}

// Reservoir choice among R >= 1 firing patches (select_active, kernel.cu:285-316): the rank
// r (1-based, in patch order) of the selected patch is the highest r whose draw is below
// 1.0f / r, or 0 when none is.  Ranks are scanned from R downward, 256 (64 Philox calls) at
// a time.  pre >= 0: the clause's rank_bits, which decide R <= 4 alone.  Wave-uniform.
template <bool INJECT>
__device__ __forceinline__ int reservoir_rank(const TrainArgs& a, const Geom& g, const float* inj, int64_t c, uint64_t t,
                                              int R, const float* inv_rank, int pre = -1) {
  const int lane = lane_id();
  if (!INJECT && pre >= 0 && R <= 4) {
    const unsigned hits = (unsigned)pre & ((1u << R) - 1u);
    return hits ? 32 - __builtin_clz(hits) : 0;
  }
  int best = 0;
  for (int g0 = (R - 1) >> 2; g0 >= 0; g0 -= kWave) {
    const int gl = g0 - lane;
    int lb = 0;
    if (gl >= 0) {
      if (INJECT) {
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * gl + 1 + j;
          if (r <= R && inj[c * g.P + (r - 1)] < inv_rank[r]) lb = r;
        }
      } else {
        const U4 z = counted_site(a, t, (uint32_t)c, TAG_SEL, (uint32_t)gl);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * gl + 1 + j;
          if (r <= R && uniform_from_word(word_of(z, j)) < inv_rank[r]) lb = r;
        }
      }
    }
    // lane q holds ranks 4(g0 - q) + 1 .. + 4, so the first lane with a hit has the best
    const unsigned long long hit = __ballot(lb > 0);
    if (hit) {
      best = lane_value(lb, __ffsll((long long)hit) - 1);
      break;
    }
  }
  return best;
}

// Patch of a clause with several patches from its firing bitmap (lane j: patch word j,
// j < PW): reservoir rank among the R firing patches, then the patch of that rank.
// Returns -1 when none is selected.  Wave-uniform.
template <bool INJECT>
__device__ __forceinline__ int select_from_bitmap(const TrainArgs& a, const Geom& g, const float* inj, int64_t c, uint64_t t,
                                                  uint32_t acc, const float* inv_rank, int pre = -1) {
  const int lane = lane_id();
  const int PW = (int)((g.P + 31) / 32);
  if (!__any(lane < PW && acc != 0u)) return -1;  // no patch fires (most clauses): no scan
  const int pc = lane < PW ? __popc(acc) : 0;
  const int incl = wave_inclusive_scan(pc);
  const int R = lane_value(incl, kWave - 1);
  if (R == 0) return -1;
  const int best = reservoir_rank<INJECT>(a, g, inj, c, t, R, inv_rank, pre);
  if (best == 0) return -1;
  const int excl = incl - pc;
  const bool here = lane < PW && best > excl && best <= incl;
  const unsigned long long hb = __ballot(here);
  const int src = __ffsll((long long)hb) - 1;
  int pos = 0;
  if (lane == src) {
    uint32_t v = acc;
    for (int q = 1; q < best - excl; ++q) v &= v - 1u;
    pos = src * 32 + __builtin_ctz(v);
  }
  return lane_value(pos, src);
}

// All-ones firing bitmap word of lane j (patches 32j .. 32j+31 that exist), 0 beyond PW.
__device__ __forceinline__ uint32_t all_patches_word(const Geom& g) {
  const int lane = lane_id();
  const int PW = (int)((g.P + 31) / 32);
  if (lane >= PW) return 0u;
  return (lane == PW - 1 && (g.P & 31)) ? ((1u << (g.P & 31)) - 1u) : 0xFFFFFFFFu;
}

// Form of a literal list entry, chosen per model so that a list walk turns an entry into an
// address without a multiply (v_mul_lo_u32 runs at a quarter of the VALU rate):
//   kListBytes: the literal's byte offset in the literal-major sample, l * 4 * ceil(P/32),
//     when every such offset fits 16 bits (several patches): one add per entry, which reads
//     the entry's half of the packed pair in place;
//   kListWords: its word offset l * ceil(P/32) when that fits 16 bits (every one-patch
//     model, where it is l): an extract and a shift-add;
//   kListIndex: the literal index l, multiplied by ceil(P/32) in the walk (several patches
//     whose literal-major sample exceeds 65536 words).
constexpr int kListIndex = 0, kListWords = 1, kListBytes = 2;
__host__ __device__ __forceinline__ int list_form(const Geom& g) {
  const int64_t last_word = (int64_t)(g.L - 1) * ((g.P + 31) / 32);
  if (g.P > 1 && last_word * 4 <= 0xFFFF) return kListBytes;
  return last_word <= 0xFFFF ? kListWords : kListIndex;
}
__device__ __forceinline__ uint32_t list_scale(const Geom& g) {
  const int f = list_form(g);
  const uint32_t PW = (uint32_t)((g.P + 31) / 32);
  return f == kListBytes ? 4u * PW : (f == kListWords ? PW : 1u);
}

// AND of word `word` of the bitsets of the 2 * NE literals whose list entries e holds (two
// per element) in the literal-major sample xt ([L][PW] words); FORM: list_form(g).
template <int FORM, int NE>
__device__ __forceinline__ uint32_t and_listed_as(const Geom& g, const uint32_t (&e)[NE], const uint32_t* xt,
                                                  uint32_t word) {
  uint32_t v = 0xFFFFFFFFu;
  if (FORM == kListBytes) {
    const char* xb = (const char*)(xt + word);
#pragma unroll
    for (int u = 0; u < NE; ++u) {
      v &= *(const uint32_t*)(xb + (e[u] & 0xFFFFu));
      v &= *(const uint32_t*)(xb + (e[u] >> 16));
    }
  } else if (FORM == kListWords) {
    const uint32_t* xw = xt + word;
#pragma unroll
    for (int u = 0; u < NE; ++u) {
      v &= xw[e[u] & 0xFFFFu];
      v &= xw[e[u] >> 16];
    }
  } else {
    const uint32_t PW = (uint32_t)((g.P + 31) / 32);
#pragma unroll
    for (int u = 0; u < NE; ++u) {
      v &= xt[(e[u] & 0xFFFFu) * PW + word];
      v &= xt[(e[u] >> 16) * PW + word];
    }
  }
  return v;
}

template <int NE>
__device__ __forceinline__ uint32_t and_listed(const Geom& g, const uint32_t (&e)[NE], const uint32_t* xt,
                                               uint32_t word) {
  switch (list_form(g)) {
    case kListBytes: return and_listed_as<kListBytes>(g, e, xt, word);
    case kListWords: return and_listed_as<kListWords>(g, e, xt, word);
    default: return and_listed_as<kListIndex>(g, e, xt, word);
  }
}

// Order of the literals in the lists: kOrderBuckets buckets of literal density, the share
// of (sample, patch) pairs of a few samples where the literal is 1 (literal_order_kernel),
// sparsest first, increasing literal index within a bucket.  A walk ends at the first step
// whose AND leaves no patch firing, so the literals most likely to be 0 go first; the AND,
// and so every result, is the same in any order.  order[b][w]: bit i set when literal
// 32w + i is in bucket b; each literal of the W words is in exactly one bucket.
// (kOrderBuckets, kOrderSamples: ytm_types.h)

// One round of build_literal_list: the literals mv of word w, lane by lane in lane order,
// appended to list[total...) (entries past cap dropped); updates total and last (the last
// literal appended).  Wave-uniform.
__device__ __forceinline__ void append_literals(uint32_t mv, int w, uint32_t scale, uint16_t* list, int cap,
                                                int* total, int* last) {
  const int pc = __popc(mv);
  const int incl = wave_inclusive_scan(pc);
  const int tot = lane_value(incl, kWave - 1);
  if (tot == 0) return;
  const unsigned long long nz = __ballot(mv != 0u);
  const int hi = 63 - __clzll((long long)nz);  // lane of the round's last literal
  *last = lane_value(32 * w + 31 - __clz((int)(mv | 1u)), hi);
  int pos = *total + incl - pc;
  while (mv) {
    const int bit = __ffs((int)mv) - 1;
    if (pos < cap) list[pos] = (uint16_t)((uint32_t)(32 * w + bit) * scale);
    ++pos;
    mv &= mv - 1u;
  }
  *total += tot;
}

// Included literals of a clause (include mask m, W words), bucket by bucket of `order`
// (literal index order when order is null), written to list[0, n) when n <= cap (as
// entries of list_form(g)), the entries from n to the next multiple of 8 repeating the
// last one (cap a multiple of 8).  Returns n, the include count.  Wave-uniform.
// BY_PAIRS: a round takes 64 (bucket, word) pairs in list order, one per lane, so that a
// model of W words needs ceil(kOrderBuckets * W / 64) rounds; else a round per bucket and
// 64 words.  The lists are the same; the kernels differ in what the inlined code costs
// them (the resident kernel rebuilds lists on its critical path and takes pairs, the
// global kernel rebuilds them rarely and runs its evaluation loop faster beside the
// per-bucket form).
template <bool BY_PAIRS = true>
__device__ int build_literal_list(const Geom& g, const uint32_t* m, uint16_t* list, int cap,
                                  const uint32_t* order = nullptr) {
  const int lane = lane_id();
  const uint32_t scale = list_scale(g);
  const int W = (int)g.W;
  int total = 0, last = 0;
  if (BY_PAIRS || !order) {
    // lane i takes pair (bucket b, word w) of each round (the words when there is no
    // order); a round moves it q64 buckets and r64 words on
    const int npairs = order ? kOrderBuckets * W : W;
    const int q64 = kWave / W, r64 = kWave - q64 * W;
    int b = lane / W, w = lane - b * W;
    for (int pb = 0; pb < npairs; pb += kWave) {
      uint32_t mv = pb + lane < npairs ? m[w] : 0u;
      if (order) mv &= pb + lane < npairs ? order[b * W + w] : 0u;
      append_literals(mv, w, scale, list, cap, &total, &last);
      b += q64;
      w += r64;
      if (w >= W) {
        w -= W;
        ++b;
      }
    }
  } else {
    for (int b = 0; b < kOrderBuckets; ++b)
      for (int wb = 0; wb < W; wb += kWave) {
        const int w = wb + lane;
        append_literals(w < W ? m[w] & order[b * W + w] : 0u, w, scale, list, cap, &total, &last);
      }
  }
  if (total > 0 && total <= cap) {
    const int pad_end = ((total + 7) & ~7) < cap ? ((total + 7) & ~7) : cap;
    for (int p = total + lane; p < pad_end; p += kWave) list[p] = (uint16_t)((uint32_t)last * scale);
  }
  return total;
}

// Firing bitmap of a clause from its literal list (n literals, padded to a multiple of 8)
// on the literal-major sample xt: acc (lane j: patch word j < PW, the all-patches mask)
// AND-ed with the bitsets of the listed literals, 16 per step (four 8-byte reads of the
// list); stops once nothing fires.  When at least two groups of PW lanes fit in the wave,
// each group walks its own runs of 16 literals and the groups' bitmaps are AND-ed at the
// end, so one step covers 16 * (64 / PW) literals.  list must be 8-byte aligned.
__device__ __forceinline__ uint32_t firing_from_list(const Geom& g, const uint16_t* list, int n, const uint32_t* xt,
                                                     uint32_t acc) {
  const int lane = lane_id();
  const int PW = (int)((g.P + 31) / 32);
  const int NG = kWave / PW;  // lane groups of PW lanes
  if (NG >= 2) {
    // Group q (lanes [q*GS, q*GS + PW)) ANDs the literal runs 16q, 16q + 16*NG, ... into its
    // own partial bitmap (lane q*GS + w: word w); a group whose partial is empty everywhere
    // ends the walk, and the groups' partials are AND-ed together at the end.  Two groups
    // sit in the two 32-lane halves, so that each half's reads come from one literal's row.
    const int GS = NG == 2 ? 32 : PW;
    const int q = lane / GS, w = lane - q * GS;
    const bool in_group = q < NG && w < PW;
    // word w of the all-patches mask
    uint32_t part = in_group ? (w == PW - 1 && (g.P & 31) ? ((1u << (g.P & 31)) - 1u) : 0xFFFFFFFFu) : 0u;
    const unsigned long long gmask = PW >= 64 ? ~0ull : ((1ull << PW) - 1ull);
    for (int j0 = 0; j0 < n; j0 += 16 * NG) {
      const int j = j0 + 16 * q;
      if (in_group && j < n) {
        // two runs of 8 per step, all 16 reads in flight together; without a second run the
        // first is read twice (the AND is idempotent)
        const int j1 = j + 8 < n ? j + 8 : j;
        const uint2 q0 = *(const uint2*)(list + j), q1 = *(const uint2*)(list + j + 4);
        const uint2 q2 = *(const uint2*)(list + j1), q3 = *(const uint2*)(list + j1 + 4);
        const uint32_t w8[8] = {q0.x, q0.y, q1.x, q1.y, q2.x, q2.y, q3.x, q3.y};
        part &= and_listed(g, w8, xt, (uint32_t)w);
      }
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
      if (dead) {
        part = 0u;
        break;
      }
    }
    // AND of the groups' partials: lane w (< PW) gathers word w of every group
    uint32_t r = part;
    for (int gq = 1; gq < NG; ++gq)
      r &= (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (w + gq * GS < kWave ? w + gq * GS : lane), (int)part);
    return lane < PW ? (r & acc) : 0u;
  }
  const int jl = lane < PW ? lane : 0;
  for (int j = 0; j < n; j += 16) {
    const int j1 = j + 8 < n ? j + 8 : j;  // second run of the step (the first again if none)
    const uint2 q0 = *(const uint2*)(list + j), q1 = *(const uint2*)(list + j + 4);
    const uint2 q2 = *(const uint2*)(list + j1), q3 = *(const uint2*)(list + j1 + 4);
    const uint32_t w8[8] = {q0.x, q0.y, q1.x, q1.y, q2.x, q2.y, q3.x, q3.y};
    acc &= and_listed(g, w8, xt, (uint32_t)jl);
    if (!__any(acc != 0u)) break;  // every 16 literals: stop once nothing fires
  }
  return acc;
}

// Firing bitmap of a clause by walking its include mask (no literal list), on the
// literal-major sample xt: lane j of each round of 64 finds the j-th included literal, and
// the literals are AND-ed 8 per step (a short last step repeats one).
__device__ __forceinline__ uint32_t firing_from_mask(const Geom& g, const uint32_t* m, const uint32_t* xt, uint32_t acc) {
  const int lane = lane_id();
  const int PW = (int)((g.P + 31) / 32);
  const int jl = lane < PW ? lane : 0;
  bool alive = true;
  for (int64_t wb = 0; wb < g.W && alive; wb += kWave) {
    const uint32_t mv = wb + lane < g.W ? m[wb + lane] : 0u;
    const int pc = __popc(mv);
    const int incl = wave_inclusive_scan(pc);
    const int tot = lane_value(incl, kWave - 1);
    const int nw = (int)(g.W - wb < kWave ? g.W - wb : kWave);
    for (int jb = 0; jb < tot && alive; jb += kWave) {
      const int j = jb + lane;
      uint32_t mw = 0u;
      int q = 0, ex = 0, before = 0;
      for (int w = 0; w < nw; ++w) {
        const int after = lane_value(incl, w);
        if (before <= j && j < after) {
          q = w;
          ex = before;
          mw = (uint32_t)lane_value((int)mv, w);
        }
        before = after;
      }
      int r = j - ex, pos = 0;
      uint32_t v = mw;
#pragma unroll
      for (int width = 16; width > 0; width >>= 1) {
        const int lowc = __popc(v & ((1u << width) - 1u));
        if (r >= lowc) {
          r -= lowc;
          v >>= width;
          pos += width;
        }
      }
      const int lit = (int)(32 * (wb + q)) + pos;  // valid for lanes j < tot
      const int cnt = tot - jb < kWave ? tot - jb : kWave;
      for (int jj = 0; jj < cnt; jj += 8) {
        uint32_t vv = 0xFFFFFFFFu;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int l = lane_value(lit, jj + u < cnt ? jj + u : jj);
          vv &= xt[l * PW + jl];
        }
        acc &= vv;
        if (((jj >> 3) & 1) && !__any(acc != 0u)) {
          alive = false;
          break;
        }
      }
    }
  }
  return acc;
}

// ---------------------------------------------------------------- lane groups
// Groups of S lanes (S = 16 or 32: one DPP row or two) that each take their own clause.
// Inclusive scan within each group (DPP row shifts; for S = 32 row_bcast:15 carries row 0
// into row 1 and row 2 into row 3).  Call with every lane active.
template <int S>
__device__ __forceinline__ int group_scan_add(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr1, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr2, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr4, 0xf, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, kDppRowShr8, 0xf, 0xf, false);
  if (S == 32) v += __builtin_amdgcn_update_dpp(0, v, kDppRowBcast15, 0xa, 0xf, false);
  return v;
}

// Value of lane src (any lane; every lane active).
__device__ __forceinline__ int lane_from(int v, int src) { return __builtin_amdgcn_ds_bpermute(4 * src, v); }

// Phase A of up to 64 / S clauses of a model with several patches at once, one per group of
// S lanes (S = 16 or 32, at least ceil(P/32)).  The calling lane's group takes clause c with
// the literal list `list` (n literals, padded to a multiple of 8) when valid, else nothing.
// Each group's result is eval_select_lm's for its clause: the firing bitmap over all patches
// is the AND of the listed literals' bitsets in the literal-major sample xt (fast_eval,
// kernel.cu:255-282; an empty clause fires on every patch), then the reservoir choice of the
// firing patch (select_active, kernel.cu:285-316) from the same draws (rank r: site
// (t, c, SEL, (r-1)/4), word (r-1)%4): a pass tests each open group's next 4*S ranks from the
// top, and a group closes at its first hit.  Returns the group's selected patch or -1, the
// same in every lane of the group.
template <bool INJECT, int S>
__device__ int eval_select_lm_group(const TrainArgs& a, const Geom& g, const float* inj, uint64_t t, int64_t c,
                                    bool valid, const uint16_t* list, int n, const uint32_t* xt, bool dropped,
                                    const float* inv_rank) {
  const int lane = lane_id();
  const int j = lane & (S - 1);
  const int gbase = lane - j;
  const uint32_t gmask = S == 32 ? 0xFFFFFFFFu : ((1u << S) - 1u);
  const int PW = (int)((g.P + 31) / 32);
  const bool live = valid && !dropped;
  // firing bitmap: lane j < PW of the group keeps patches [32j, 32j + 32)
  uint32_t acc = (live && j < PW) ? ((j == PW - 1 && (g.P & 31)) ? ((1u << (g.P & 31)) - 1u) : 0xFFFFFFFFu) : 0u;
  const int nn = live ? n : 0;
  const int nmax = wave_max_i32(nn);
  const uint32_t jl = (uint32_t)(j < PW ? j : 0);
  for (int s0 = 0; s0 < nmax; s0 += 16) {
    if (s0 < nn) {
      // two runs of 8 per step, all 16 reads in flight together; without a second run the
      // first is read twice (the AND is idempotent)
      const int s1 = s0 + 8 < nn ? s0 + 8 : s0;
      const uint2 q0 = *(const uint2*)(list + s0), q1 = *(const uint2*)(list + s0 + 4);
      const uint2 q2 = *(const uint2*)(list + s1), q3 = *(const uint2*)(list + s1 + 4);
      const uint32_t w8[8] = {q0.x, q0.y, q1.x, q1.y, q2.x, q2.y, q3.x, q3.y};
      acc &= and_listed(g, w8, xt, jl);
    }
    if (!__any(acc != 0u)) break;  // stop once nothing fires anywhere
  }
  if (!__any(acc != 0u)) return -1;  // no group's clause fires anywhere: no scan
  const int pc = __popc(acc);
  const int incl = group_scan_add<S>(pc);
  const int R = lane_from(incl, gbase + S - 1);  // firing patches of the group's clause
  // reservoir: the highest rank r <= R whose draw is below 1.0f / r
  int best = 0;
  bool open = R > 0;
  int g0 = (R - 1) >> 2;  // draw site of the group's top ranks
  while (__any(open)) {
    const int gl = g0 - j;
    int lb = 0;
    if (open && gl >= 0) {
      if (INJECT) {
        for (int q = 0; q < 4; ++q) {
          const int r = 4 * gl + 1 + q;
          if (r <= R && inj[c * g.P + (r - 1)] < inv_rank[r]) lb = r;
        }
      } else {
        const U4 z = counted_site(a, t, (uint32_t)c, TAG_SEL, (uint32_t)gl);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = 4 * gl + 1 + q;
          if (r <= R && uniform_from_word(word_of(z, q)) < inv_rank[r]) lb = r;
        }
      }
    }
    // lane j of a group holds ranks 4(g0 - j) + 1 .. + 4: the group's first lane with a hit
    // holds the best
    const uint32_t gh = (uint32_t)(__ballot(lb > 0) >> gbase) & gmask;
    const int hit_best = lane_from(lb, gh ? gbase + __ffs((int)gh) - 1 : lane);
    if (open) {
      if (gh) {
        best = hit_best;
        open = false;
      } else {
        g0 -= S;
        open = g0 >= 0;
      }
    }
  }
  // the patch of the best-th set bit of the group's firing bitmap
  const int excl = incl - pc;
  const bool here = best > 0 && j < PW && best > excl && best <= incl;
  int p_here = 0;
  if (here) {
    uint32_t v = acc;
    for (int q = 1; q < best - excl; ++q) v &= v - 1u;
    p_here = j * 32 + __builtin_ctz(v);
  }
  const uint32_t hb = (uint32_t)(__ballot(here) >> gbase) & gmask;
  const int p = lane_from(p_here, hb ? gbase + __ffs((int)hb) - 1 : lane);
  return best > 0 ? p : -1;
}

// Phase A for one clause of a model with several patches, on the literal-major sample xt
// ([L][PW] words, PW = ceil(P/32) <= 64; bit b of word j of literal l: literal l set in
// patch 32j + b).  The clause fires on the patches where every included literal is set, so
// its firing bitmap is the AND of its included literals' bitsets (fast_eval,
// kernel.cu:255-282), taken from the clause's literal list when it has one (nlist <= cap,
// cap > 0) and from its include mask otherwise.  Then the reservoir choice of the firing
// patch (select_active, kernel.cu:285-316).  An empty clause fires on every patch in
// training.  pre: the clause's rank_bits for this sample, or -1.  Wave-uniform.
template <bool INJECT>
__device__ int eval_select_lm(const TrainArgs& a, const Geom& g, const float* inj, int64_t c, uint64_t t, const uint32_t* m,
                              const uint16_t* list, int nlist, int cap, const uint32_t* xt, bool dropped,
                              int* ninc_out, const float* inv_rank, int pre = -1) {
  const int lane = lane_id();
  int ninc;
  if (cap > 0 && nlist <= cap) {
    ninc = nlist;
  } else {
    const bool exact_count = g.maxinc < g.L;
    int cnt = 0;
    uint32_t any = 0u;
    for (int64_t w = lane; w < g.W; w += kWave) {
      const uint32_t mw = m[w];
      if (exact_count) cnt += __popc(mw);
      any |= mw;
    }
    ninc = exact_count ? wave_sum_i32(cnt) : (__any(any != 0u) ? 1 : 0);
  }
  *ninc_out = ninc;
  if (dropped) return -1;
  uint32_t acc = all_patches_word(g);
  if (ninc != 0)
    acc = (cap > 0 && nlist <= cap) ? firing_from_list(g, list, nlist, xt, acc) : firing_from_mask(g, m, xt, acc);
  return select_from_bitmap<INJECT>(a, g, inj, c, t, acc, inv_rank, pre);
}

// Phase A for one clause (wave-uniform): returns the selected patch or -1 and the
// clause's include count.  m: the clause's include mask (W words), xe: the sample (P*W).
template <bool VANILLA, bool INJECT, bool PRE = false>
__device__ int eval_select(const TrainArgs& a, const Geom& g, const float* inj, int64_t c, uint64_t t, const uint32_t* m,
                           const uint32_t* xe, bool dropped, float u_pre, int* ninc_out) {
  const int lane = lane_id();
  // The include count only matters through "empty" and "<= MAX_INCLUDED_LITERALS"; when
  // that bound is at least L, a 0/1 emptiness flag stands in for it.
  const bool exact_count = g.maxinc < g.L;
  if (VANILLA) {
    uint32_t bad = 0u, any = 0u;
    int cnt = 0;
    for (int64_t w = lane; w < g.W; w += kWave) {
      const uint32_t mw = m[w];
      if (exact_count) cnt += __popc(mw);
      any |= mw;
      bad |= mw & ~xe[w];
    }
    const int ninc = exact_count ? wave_sum_i32(cnt) : (__any(any != 0u) ? 1 : 0);
    *ninc_out = ninc;
    const bool any_bad = __any(bad != 0u);
    if (dropped) return -1;
    if (ninc != 0 && any_bad) return -1;
    // One firing patch: its draw must be below 1.0f / 1.
    float u;
    if (INJECT)
      u = inj[c * g.P];
    else if (PRE)
      u = u_pre;
    else
      u = uniform_from_word(counted_site(a, t, (uint32_t)c, TAG_SEL, 0u).x);
    return u < 1.0f ? 0 : -1;  // 1.0f / 1
  } else {
    int cnt = 0;
    uint32_t any = 0u;
    for (int64_t w = lane; w < g.W; w += kWave) {
      const uint32_t mw = m[w];
      if (exact_count) cnt += __popc(mw);
      any |= mw;
    }
    const int ninc = exact_count ? wave_sum_i32(cnt) : (__any(any != 0u) ? 1 : 0);
    *ninc_out = ninc;
    if (dropped) return -1;
    // Firing patches of chunk ch, lane q: patch 64 ch + q.
    auto chunk_fire = [&](int ch) -> unsigned long long {
      const int64_t p = (int64_t)ch * kWave + lane;
      bool ok = p < g.P;
      if (ok && ninc != 0) {
        const uint32_t* xp = xe + p * g.W;
        for (int64_t w = 0; w < g.W; ++w)
          if (m[w] & ~xp[w]) {
            ok = false;
            break;
          }
      }
      return __ballot(ok);
    };
    // Firing bitmap: lane q keeps bits of patches [64q, 64q+64) (the first 64 chunks).
    unsigned long long myfire = 0ull;
    int R = 0;
    const int nch = (int)((g.P + kWave - 1) / kWave);
    for (int ch = 0; ch < nch; ++ch) {
      const unsigned long long b = chunk_fire(ch);
      if (lane == ch) myfire = b;
      R += __popcll(b);
    }
    if (R == 0) return -1;
    const int best = reservoir_rank<INJECT>(a, g, inj, c, t, R, a.inv_rank);
    if (best == 0) return -1;
    if (nch > kWave) {
      // more than 4096 patches: the chunks again, up to the one holding the best-th firing
      // patch
      int before = 0;
      for (int ch = 0; ch < nch; ++ch) {
        const unsigned long long b = chunk_fire(ch);
        const int pc = __popcll(b);
        if (before + pc >= best) {
          unsigned long long v = b;
          for (int q = 1; q < best - before; ++q) v &= v - 1ull;
          return ch * kWave + __ffsll((long long)v) - 1;
        }
        before += pc;
      }
      return -1;  // not reached: best <= R
    }
    // Patch of the best-th set bit of the firing bitmap.
    const int pc = lane < nch ? __popcll(myfire) : 0;
    const int incl = wave_inclusive_scan(pc);
    const int excl = incl - pc;
    const bool here = lane < nch && best > excl && best <= incl;
    const unsigned long long hb = __ballot(here);
    const int src = __ffsll((long long)hb) - 1;
    int pos = 0;
    if (lane == src) {
      unsigned long long v = myfire;
      for (int q = 1; q < best - excl; ++q) v &= v - 1ull;
      pos = src * kWave + __ffsll((long long)v) - 1;
    }
    return lane_value(pos, src);
  }
}

struct FbOps {
  unsigned long long m1a, m1b, m2;  // bit k - kb: class k runs Type Ia / Ib / II
};

// Phase D decisions for one non-dropped clause (clause_update, kernel.cu:567-610): per
// class, the Q-skip and update draws, the feedback type, and the weight update.  The
// literal updates are left to apply_ops.  Wave-uniform result.  Every input is loaded
// before any decision is taken and the decisions are selects, so the loads overlap
// instead of forming a chain of dependent LDS round trips.
// kc: with more than 64 classes (coalesced), the first of the 64 classes decided here.
template <bool INJECT, bool PRE = false>
__device__ FbOps decide(const TrainArgs& a, const Geom& g, const float* inj, int64_t c, uint64_t t, int sel, int ninc,
                        const int* s_tgt, const double* s_prob, float* wrow, const float* pre_uq,
                        const float* pre_uu, bool dropped = false, int64_t kc = 0) {
  const int lane = lane_id();
  const int64_t kb = g.coalesced ? kc : c / g.per_bank;
  const int kn = g.coalesced ? (int)(g.K - kc < kWave ? g.K - kc : kWave) : 1;
  const int64_t k = kb + (lane < kn ? lane : 0);  // idle lanes read class kb's inputs and discard them
  const bool act = lane < kn && !dropped;        // a dropped clause gets no feedback (kernel.cu:555)
  const int tgt = s_tgt[k];
  const double prob = s_prob[k];
  float* wp = wrow + k;
  const float w0 = *wp;
  float uq, uu;
  if (INJECT) {
    uq = inj[g.C * g.P + c * g.K + k];
    uu = inj[g.C * g.P + g.C * g.K + c * g.K + k];
  } else if (PRE) {
    uq = pre_uq[k];
    uu = pre_uu[k];
  } else {
    const U4 z = counted_site(a, t, (uint32_t)c, TAG_CK, (uint32_t)k);
    uq = uniform_from_word(z.x);
    uu = uniform_from_word(z.y);
  }
  const bool o = sel >= 0;
  const bool small = o && ninc <= g.maxinc;
  const bool skip = tgt == -1 && (double)uq > g.q_prob;
  const int sign = (w0 >= 0.0f) - (w0 < 0.0f);
  const bool upd = act && !skip && (double)uu <= prob;
  const int ts = tgt * sign;
  const bool t1a = upd && ts > 0 && small;
  const bool t1b = upd && ts > 0 && !small;
  const bool t2 = upd && ts < 0 && o;
  const float wa = w0 + (float)sign * 1.0f;
  float wb = w0 - (float)sign * 1.0f;
  if (!g.negative_polarity) wb = wb < 1.0f ? 1.0f : wb;
  if (t1a || t2) *wp = t1a ? wa : wb;
  return FbOps{__ballot(t1a), __ballot(t1b), __ballot(t2)};
}

// The decision of decide() for one (clause, class) pair held by the calling lane (its own
// clause c and class k), with the pre-drawn Q-skip and update draws uq, uu (or the
// injected ones).  The update test (double)uu <= prob is made as (double)uu * den <= num:
// den = 1, num = prob, or the exact division-free form of class_fb_exact.  Not
// wave-uniform: every lane may hold another clause.
struct PairOps {
  bool t1a, t1b, t2;
  float w_new;
};

// What a pair's decision needs besides its class's target and the update test's right-hand
// side: everything that is known before the class sums are (pair_pre), so that only
// pair_decide is left once they arrive.
struct PairPre {
  int flags;  // bit 0 act, 1 o (selected), 2 small (o and ninc <= MAXINC), 3 qskip, 4 w0 < 0, 5 w0 >= 0
  double ud;  // (double)uu * den
  float w0;
};

template <bool INJECT>
__device__ __forceinline__ PairPre pair_pre(const Geom& g, const float* inj, int64_t c, int64_t k, bool act, int sel,
                                            int ninc, double den, float w0, float uq, float uu) {
  if (INJECT) {
    uq = inj[g.C * g.P + c * g.K + k];
    uu = inj[g.C * g.P + g.C * g.K + c * g.K + k];
  }
  const bool o = sel >= 0;
  PairPre r;
  r.flags = (int)act | (int)o << 1 | (int)(o && ninc <= g.maxinc) << 2 | (int)((double)uq > g.q_prob) << 3 |
            (int)(w0 < 0.0f) << 4 | (int)(w0 >= 0.0f) << 5;
  r.ud = (double)uu * den;
  r.w0 = w0;
  return r;
}

// Keeps a PairPre computed where it stands (ahead of a wait) instead of where it is used.
__device__ __forceinline__ void pin(PairPre& q) { asm volatile("" : "+v"(q.flags), "+v"(q.ud), "+v"(q.w0)); }

__device__ __forceinline__ PairOps pair_decide(const Geom& g, const PairPre& q, int tgt, double num) {
  const bool act = q.flags & 1, o = (q.flags >> 1) & 1, small = (q.flags >> 2) & 1, qskip = (q.flags >> 3) & 1;
  const int sign = ((q.flags >> 5) & 1) - ((q.flags >> 4) & 1);  // (w0 >= 0) - (w0 < 0)
  const bool skip = tgt == -1 && qskip;
  const bool upd = act && !skip && q.ud <= num;
  const int ts = tgt * sign;
  PairOps r;
  r.t1a = upd && ts > 0 && small;
  r.t1b = upd && ts > 0 && !small;
  r.t2 = upd && ts < 0 && o;
  const float wa = q.w0 + (float)sign * 1.0f;
  float wb = q.w0 - (float)sign * 1.0f;
  if (!g.negative_polarity) wb = wb < 1.0f ? 1.0f : wb;
  r.w_new = r.t1a ? wa : wb;
  return r;
}

template <bool INJECT>
__device__ __forceinline__ PairOps decide_pair(const Geom& g, const float* inj, int64_t c, int64_t k, bool act, int sel,
                                               int ninc, int tgt, double num, double den, float w0, float uq, float uu) {
  return pair_decide(g, pair_pre<INJECT>(g, inj, c, k, act, sel, ninc, den, w0, uq, uu), tgt, num);
}

// Literal updates of one clause for the feedback decided in ops, applied class by class
// in increasing k to the clause's planes (cplanes, stride W).  pre, when given, holds the
// first kPreGroups plane groups of the literal draws of every Type Ia/Ib class, in the
// order of those classes: [op][W][kPreGroups][4].  kc: as in decide (bit b of ops is class
// kc + b of a coalesced model).
template <bool INJECT>
__device__ void apply_ops(const TrainArgs& a, const Geom& g, const float* inj, int64_t c, uint64_t t, int sel, FbOps ops,
                          uint32_t* cplanes, const uint32_t* xe, const uint32_t* pre, uint32_t* top_copy = nullptr,
                          int64_t wb_first = 0, int64_t wb_end = -1, int64_t kc = 0) {
  // words [wb_first, wb_end) of the clause (wb_first a multiple of 64; wb_end < 0: to W)
  const int lane = lane_id();
  const int64_t kb = g.coalesced ? kc : c / g.per_bank;
  const bool o = sel >= 0;
  const uint32_t* xsel = o ? xe + (int64_t)sel * g.W : nullptr;
  const int np = g.np;
  const unsigned long long all = ops.m1a | ops.m1b | ops.m2;
  const int64_t wend = wb_end < 0 || wb_end > g.W ? g.W : wb_end;
  for (int64_t wb = wb_first; wb < wend; wb += kWave) {
    const int64_t w = wb + lane;
    const bool act = w < g.W;
    const uint32_t F = act ? (w == g.W - 1 ? g.last_filter : 0xFFFFFFFFu) : 0u;
    uint32_t* pw = cplanes + w;
    uint32_t pl[kMaxPlanes];
#pragma unroll
    for (int j = 0; j < kMaxPlanes; ++j) pl[j] = (j < np && act) ? pw[(int64_t)j * g.W] : 0u;
    const uint32_t xb = (o && act) ? xsel[w] : 0u;
    unsigned long long rem = all;
    int rng_op = 0;
    while (rem) {
      const int b = __ffsll((long long)rem) - 1;
      rem &= rem - 1ull;
      const int64_t k = kb + b;
      if (((ops.m1a | ops.m1b) >> b) & 1ull) {
        // Type Ia (kernel.cu:410-443): literal 1 -> +1 below MAX, literal 0 -> -1 w.p. 1/s.
        // Type Ib (kernel.cu:453-470): every literal -1 w.p. 1/s.
        const bool t1a = (ops.m1a >> b) & 1ull;
        const uint32_t pos = planes_gt(pl, np, g.off) & F;
        const uint32_t need = t1a ? (~xb & pos) : pos;
        const uint32_t* pre_w = (pre && act) ? pre + ((int64_t)rng_op * g.W + w) * (kPreGroups * 4) : nullptr;
        const uint32_t dec = literal_draw_mask<INJECT>(a, g, inj, need, t, c, k, w, pre_w, pre != nullptr);
        if (t1a) planes_inc(pl, np, xb & planes_lt(pl, np, g.max_state_p) & F);
        planes_dec(pl, np, dec);
        ++rng_op;
      } else {
        // Type II (kernel.cu:481-506): literal 0 -> +1, no upper guard.
        planes_inc(pl, np, ~xb & F);
      }
    }
    if (act) {
#pragma unroll
      for (int j = 0; j < kMaxPlanes; ++j)
        if (j < np) pw[(int64_t)j * g.W] = pl[j];
      if (top_copy) top_copy[w] = pl[np - 1];  // the include mask, also kept in LDS
    }
  }
}

// Tasks per wave when ntask queued clause updates are spread over nwv waves, at most
// 64 / W of them packed into one wave: spread first, pack only what is left over.
__device__ __forceinline__ int tasks_per_wave(const Geom& g, int ntask, int nwv) {
  const int cap = kWave / (int)g.W;
  const int even = (ntask + nwv - 1) / nwv;
  return even < 1 ? 1 : (even > cap ? cap : even);
}

// Literal updates of several queued clauses at once, for models whose clauses have at most
// 32 literal words: lanes [g*W, g*W + W) of the wave take task tk0 + g (g < per <= 64 / W).
// Per class in increasing k, every clause with a feedback branch at that class applies it
// exactly as apply_ops does.  Tasks: clause s_task_idx[tk], masks s_task_m[tk][3] (bits
// relative to the clause's first class), first draw slot s_task_sb[tk] (s_rng null: draws
// computed here); sel_of[idx] the clause's selected patch; planes of clause idx at
// planes_base + idx * np * W; xe the sample's patch-major words.
// changed_lanes, when given, receives the ballot of the lanes whose include-mask word (top
// plane) changed: task tk0 + g changed its mask when a bit of [g * W, g * W + W) is set.
template <bool INJECT>
__device__ void apply_tasks(const TrainArgs& a, const Geom& g, const float* inj, int64_t c_begin, uint64_t t, int tk0,
                            int per, int ntask, const int* s_task_idx, const unsigned long long* s_task_m,
                            const int* s_task_sb, const int* sel_of, uint32_t* planes_base, const uint32_t* xe,
                            const uint32_t* s_rng, int R, uint32_t* top_base = nullptr,
                            unsigned long long* changed_lanes = nullptr) {
  const int lane = lane_id();
  const int W = (int)g.W;
  const int grp = lane / W, w = lane % W;
  const int tk = tk0 + grp;
  const bool act = grp < per && tk < ntask;
  int idx = 0, sb = 0, sel = -1;
  unsigned long long m1a = 0ull, m1b = 0ull, m2 = 0ull;
  if (act) {
    idx = s_task_idx[tk];
    m1a = s_task_m[tk * 3 + 0];
    m1b = s_task_m[tk * 3 + 1];
    m2 = s_task_m[tk * 3 + 2];
    sb = s_task_sb[tk];
    sel = sel_of[idx];
  }
  const int64_t c = c_begin + idx;
  const int64_t kb = g.coalesced ? 0 : c / g.per_bank;
  const int np = g.np;
  const uint32_t F = act ? (w == W - 1 ? g.last_filter : 0xFFFFFFFFu) : 0u;
  uint32_t* pw = planes_base + (int64_t)idx * np * W + w;
  uint32_t pl[kMaxPlanes];
#pragma unroll
  for (int j = 0; j < kMaxPlanes; ++j) pl[j] = (j < np && act) ? pw[(int64_t)j * W] : 0u;
  const uint32_t xb = (act && sel >= 0) ? xe[(int64_t)sel * W + w] : 0u;
  const unsigned long long t1 = m1a | m1b;
  const bool have = s_rng != nullptr && act && sb + __popcll(t1) <= R;
  unsigned long long u = wave_or_u64(m1a | m1b | m2);  // union of the wave's class bits
  int rng_op = 0;
  while (u) {
    const int b = __ffsll((long long)u) - 1;
    u &= u - 1ull;
    const int64_t k = kb + b;
    const bool is1 = (t1 >> b) & 1ull, is1a = (m1a >> b) & 1ull, is2 = (m2 >> b) & 1ull;
    if (__any(is1)) {
      // Type Ia (kernel.cu:410-443) / Type Ib (kernel.cu:453-470)
      const uint32_t pos = planes_gt(pl, np, g.off) & F;
      const uint32_t need = is1 ? (is1a ? (~xb & pos) : pos) : 0u;
      const uint32_t* pre_w = have ? s_rng + ((int64_t)(sb + rng_op) * W + w) * (kPreGroups * 4) : nullptr;
      const uint32_t dec = literal_draw_mask<INJECT>(a, g, inj, need, t, c, k, w, pre_w, have);
      planes_inc(pl, np, is1a ? (xb & planes_lt(pl, np, g.max_state_p) & F) : 0u);
      planes_dec(pl, np, dec);
      if (is1) ++rng_op;
    }
    // Type II (kernel.cu:481-506): literal 0 -> +1, no upper guard.
    if (__any(is2)) planes_inc(pl, np, is2 ? (~xb & F) : 0u);
  }
  if (changed_lanes) *changed_lanes = __ballot(act && pw[(int64_t)(np - 1) * W] != pl[np - 1]);
  if (act) {
#pragma unroll
    for (int j = 0; j < kMaxPlanes; ++j)
      if (j < np) pw[(int64_t)j * W] = pl[j];
    if (top_base) top_base[(int64_t)idx * W + w] = pl[np - 1];  // include masks kept in LDS ([idx][W])
  }
}

// Feedback target and update probability of one class.
struct ClassFb {
  int tgt;
  double prob;
};

// Class feedback from the class's exact total S and target y (kernel.cu:397,508-529,543-551):
// the sum clipped to +-T, target -1 when the clipped sum exceeds y, and the update
// probability (y - clip) / (2y) in double.
__device__ __forceinline__ ClassFb class_fb(const Geom& g, long long S, int y) {
  const float cs = (float)S;
  const float vclip = ((double)cs > g.thresh) ? (float)g.thresh : (((double)cs < -g.thresh) ? (float)(-g.thresh) : cs);
  return ClassFb{1 - 2 * (vclip > (float)y), ((double)y - (double)vclip) / (2.0 * (double)y)};
}

// class_fb(g, S, y).prob > 0.0 without the division: the quotient (y - vclip) / (2y) of two
// exact doubles is positive exactly when numerator and denominator have the same sign and
// the numerator is not zero; with y = 0 it is +inf (true) for y - vclip > 0, else -inf or NaN.
__device__ __forceinline__ bool class_may_update(const Geom& g, long long S, int y) {
  const float cs = (float)S;
  const float vclip = ((double)cs > g.thresh) ? (float)g.thresh : (((double)cs < -g.thresh) ? (float)(-g.thresh) : cs);
  const double d = (double)y - (double)vclip;
  return y >= 0 ? d > 0.0 : d < 0.0;
}

// class_fb without the int64 -> float conversion and the division, for an integral
// threshold 0 <= T < 2^24 and a target 0 < |y| < 2^28 (exact).  The clip is taken on the
// integer sum: for such T, (float)S > T exactly when S > T, and |S| <= T converts exactly,
// so clip((float)S) == (float)clip(S).  The update test (double)u <= prob with
// prob = RN((y - v) / (2y)) becomes u * |2y| <= (y - v) * sign(y), all terms exact in
// double: for a float u = m * 2^e (m < 2^24, |u| < 2^24) and q = (y - v) / (2y), q != u
// implies |q - u| >= 2^min(e, 0) / |2y| > half an ulp of u, so rounding q cannot cross u,
// and RN(q) >= u exactly when q >= u.  class_prep takes what depends on y only (ahead of
// the exchange); class_test returns {tgt, num, den} for decide_pair.
struct ClassPrep {
  int y;
  bool exact;
  double den;  // |2y| (exact) or 1
};

struct ClassTest {
  int tgt;
  double num, den;
};

__device__ __forceinline__ ClassPrep class_prep(const Geom& g, int y) {
  const bool tok = g.thresh >= 0.0 && g.thresh < 16777216.0 && g.thresh == (double)(int)g.thresh;
  const bool exact = tok && y != 0 && y > -(1 << 28) && y < (1 << 28);
  return ClassPrep{y, exact, exact ? (double)(y > 0 ? 2 * y : -2 * y) : 1.0};
}

__device__ __forceinline__ ClassTest class_test(const Geom& g, long long S, const ClassPrep& cp) {
  if (cp.exact) {
    const int T = (int)g.thresh;
    int v = S > (long long)T ? T : (S < -(long long)T ? -T : (int)S);
    asm volatile("" : "+v"(v));  // v is a 32-bit value from here on: one-instruction conversions
    return ClassTest{1 - 2 * ((float)v > (float)cp.y), (double)(cp.y > 0 ? cp.y - v : v - cp.y), cp.den};
  }
  const ClassFb r = class_fb(g, S, cp.y);
  return ClassTest{r.tgt, r.prob, 1.0};
}

// class_fb of class k, stored to s_tgt[k] / s_prob[k].
__device__ __forceinline__ void class_targets(const Geom& g, int k, long long S, const int32_t* y_row, int* s_tgt,
                                              double* s_prob) {
  const ClassFb r = class_fb(g, S, y_row[k]);
  s_tgt[k] = r.tgt;
  s_prob[k] = r.prob;
}

// Per sample, a two-level all-reduce of the K class sums over the grid, with a broadcast
// back (phases B/C, run by wave 0 of every workgroup):
//   1. lanes < K add (1<<44 | partial) into their group's word (groups of S workgroups);
//   2. for each word, the adder that completes its group (returned count == group size)
//      forwards the group total into the final word;
//   3. for each word, the forwarder that completes the final word (count == groups)
//      stores the total into every group's mailbox;
//   4. each workgroup polls its own group's mailbox (bounded in real time).
// Contention stays at <= S adders / pollers per word.  With one group the group words are
// polled directly; with one workgroup its partial sums are the totals.
struct ExchangeRow {
  unsigned long long* group_w;  // [D][ks]
  unsigned long long* final_w;  // [ks]
  unsigned long long* mbox;     // [D][ks]
  unsigned long long* poll;     // the words this workgroup waits on
  unsigned long long gsize;     // workgroups in this workgroup's group
  unsigned long long poll_count;
  int d, ks;
};

__device__ __forceinline__ ExchangeRow exchange_row(const TrainArgs& a, const Geom& g, int i) {
  ExchangeRow r;
  const int D = g.groups;
  r.d = (int)blockIdx.x / g.group_size;
  r.gsize = (unsigned long long)min(g.group_size, g.grid - r.d * g.group_size);
  r.ks = ((int)g.K + 15) & ~15;  // words per row (128-byte multiples)
  unsigned long long* row = a.slots + (int64_t)i * a.slot_stride;
  r.group_w = row;
  r.final_w = row + D * r.ks;
  r.mbox = r.final_w + r.ks;
  r.poll = D == 1 ? r.group_w : r.mbox + r.d * r.ks;
  r.poll_count = D == 1 ? r.gsize : (unsigned long long)D;
  return r;
}

// Steps 1-3: lanes < K publish the workgroup's partial sums of sample i (s_part, cleared;
// with one workgroup they stay in s_part for exchange_wait).
__device__ __forceinline__ void exchange_publish(const TrainArgs& a, const Geom& g, int i, long long* s_part) {
  const int lane = lane_id();
  if (g.grid == 1 || lane >= g.K) return;
  const ExchangeRow r = exchange_row(a, g, i);
  const long long part = s_part[lane];
  s_part[lane] = 0;
  const unsigned long long mine = (1ull << 44) + (unsigned long long)part;
  if (g.groups == 1) {
    __hip_atomic_fetch_add(&r.group_w[lane], mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    const unsigned long long now =
        __hip_atomic_fetch_add(&r.group_w[r.d * r.ks + lane], mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + mine;
    if (((now + (1ull << 43)) >> 44) == r.gsize) {
      const unsigned long long fwd = (1ull << 44) + (now - (r.gsize << 44));
      const unsigned long long now2 =
          __hip_atomic_fetch_add(&r.final_w[lane], fwd, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + fwd;
      if (((now2 + (1ull << 43)) >> 44) == (unsigned long long)g.groups)
        for (int m = 0; m < g.groups; ++m)
          __hip_atomic_store(&r.mbox[m * r.ks + lane], now2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Step 4: the whole wave waits until the total of every class is in; lanes with want set
// return the total of class kq (< K) in *S.  Returns false when the wait expired (s_abort
// and a.err record it).  With one workgroup the totals are read from s_part, which is then
// cleared.
__device__ __forceinline__ bool exchange_wait(const TrainArgs& a, const Geom& g, int i, int kq, bool want,
                                              long long* s_part, long long* S, int* s_abort, uint64_t* wait_ticks) {
  const int lane = lane_id();
  if (g.grid == 1) {
    if (want) *S = s_part[kq];
    __builtin_amdgcn_wave_barrier();  // every read of s_part before it is cleared
    if (lane < g.K) s_part[lane] = 0;
    return true;
  }
  const ExchangeRow r = exchange_row(a, g, i);
  const uint64_t t_start = __builtin_amdgcn_s_memrealtime();
  // a count no word reaches under the test hook: every wait then expires
  const unsigned long long complete = r.poll_count + (a.test_timeout ? 1ull : 0ull);
  unsigned long long v = 0;
  for (unsigned polls = 1;; ++polls) {
    bool ok = true;
    if (want) {
      v = __hip_atomic_load(&r.poll[kq], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ok = ((v + (1ull << 43)) >> 44) == complete;
    }
    if (__all(ok)) break;
    // the clock is read every 16th poll: each read is a scalar-memory round trip that would
    // otherwise lengthen every poll (the bound stays in real time)
    if ((polls & 15u) == 0u && __builtin_amdgcn_s_memrealtime() - t_start > (a.test_timeout ? 0 : kWaitTicks)) {
      // Record the first stall: err = {1, sample, workgroup, count seen by lane 0}.
      if (lane == 0) {
        *s_abort = 1;
        if (atomicCAS(a.err, 0, 1) == 0) {
          a.err[1] = i;
          a.err[2] = (int)blockIdx.x;
          a.err[3] = (int)((v + (1ull << 43)) >> 44);
        }
      }
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  *wait_ticks += __builtin_amdgcn_s_memrealtime() - t_start;
  if (want) *S = (long long)(v - (r.poll_count << 44));
  return true;
}

// The whole exchange of sample i; lanes < K then derive clip / target / update probability
// into s_tgt / s_prob.  Returns false when the wait expired.
__device__ __forceinline__ bool exchange_class_sums(const TrainArgs& a, const Geom& g, int i, const int32_t* y_row,
                                                    const float* bias, long long* s_part, int* s_tgt, double* s_prob,
                                                    int* s_abort, uint64_t* wait_ticks) {
  const int lane = lane_id();
  exchange_publish(a, g, i, s_part);
  long long S = 0;
  if (!exchange_wait(a, g, i, lane < g.K ? lane : 0, lane < g.K, s_part, &S, s_abort, wait_ticks)) return false;
  if (lane < g.K) class_targets(g, lane, S + (long long)bias[lane], y_row, s_tgt, s_prob);
  return true;
}

__device__ __forceinline__ void add_partial(const TrainArgs& a, const Geom& g, long long* s_part, int64_t c, const float* wrow) {
  const int lane = lane_id();
  if (g.coalesced) {
    if (lane < g.K) atomicAdd((unsigned long long*)&s_part[lane], (unsigned long long)(long long)wrow[lane]);
  } else if (lane == 0) {
    const int64_t k = c / g.per_bank;
    atomicAdd((unsigned long long*)&s_part[k], (unsigned long long)(long long)wrow[k]);
  }
}

// Phase timing of the training kernels: with TrainArgs::profile, wave 0 adds the ticks of
// the 100 MHz real-time counter since its previous mark to prof_acc[j] (locals `prof`,
// `prof_acc`, `prof_last` of the kernel body); the host reads the sums from counters[4..11].
#define YTM_PROF_MARK(j)                                      \
  if (prof) {                                                 \
    const uint64_t now_ = __builtin_amdgcn_s_memrealtime();   \
    prof_acc[j] += now_ - prof_last;                          \
    prof_last = now_;                                         \
  }

// Copies n words from global memory to LDS, threads [first, first + count) taking part,
// with up to kCopyBatch reads of each thread in flight before its LDS writes (a plain copy
// loop waits for every read in turn).  8-byte copies when n is even (both buffers are then
// 8-byte aligned).
constexpr int kCopyBatch = 8;

__device__ __forceinline__ void copy_to_lds(uint32_t* dst, const uint32_t* src, int64_t n, int first, int count) {
  if ((n & 1) == 0) {
    const uint2* s2 = (const uint2*)src;
    uint2* d2 = (uint2*)dst;
    const int64_t n2 = n / 2;
    for (int64_t j0 = first; j0 < n2; j0 += (int64_t)count * kCopyBatch) {
      uint2 v[kCopyBatch];
#pragma unroll
      for (int b = 0; b < kCopyBatch; ++b) {  // unconditional (clamped) loads, all in flight together
        const int64_t j = j0 + (int64_t)b * count;
        v[b] = s2[j < n2 ? j : n2 - 1];
      }
#pragma unroll
      for (int b = 0; b < kCopyBatch; ++b) {
        const int64_t j = j0 + (int64_t)b * count;
        if (j < n2) d2[j] = v[b];
      }
    }
  } else {
    for (int64_t j0 = first; j0 < n; j0 += (int64_t)count * kCopyBatch) {
      uint32_t v[kCopyBatch];
#pragma unroll
      for (int b = 0; b < kCopyBatch; ++b) {
        const int64_t j = j0 + (int64_t)b * count;
        v[b] = src[j < n ? j : n - 1];
      }
#pragma unroll
      for (int b = 0; b < kCopyBatch; ++b) {
        const int64_t j = j0 + (int64_t)b * count;
        if (j < n) dst[j] = v[b];
      }
    }
  }
}

// The literal-major copy of a sample whose literals Lh..L-1 are the complements of literals
// 0..Lh-1 (appended negations; TrainArgs::xt_halves): only the first half, nh = Lh * PW
// words, is read, and the second half is written as its complement with the bits of
// patches >= P (in each row's last word) kept 0, as the transposition leaves them.
__device__ __forceinline__ void copy_halves_to_lds(const Geom& g, uint32_t* dst, const uint32_t* src, int first,
                                                   int count) {
  const int64_t PW = (g.P + 31) / 32;
  const int64_t nh = g.Lh * PW;
  const uint32_t lastm = (g.P & 31) ? ((1u << (g.P & 31)) - 1u) : 0xFFFFFFFFu;
  for (int64_t j0 = first; j0 < nh; j0 += (int64_t)count * kCopyBatch) {
    uint32_t v[kCopyBatch];
#pragma unroll
    for (int b = 0; b < kCopyBatch; ++b) {  // unconditional (clamped) loads, all in flight together
      const int64_t j = j0 + (int64_t)b * count;
      v[b] = src[j < nh ? j : nh - 1];
    }
#pragma unroll
    for (int b = 0; b < kCopyBatch; ++b) {
      const int64_t j = j0 + (int64_t)b * count;
      if (j < nh) {
        dst[j] = v[b];
        dst[nh + j] = ~v[b] & (j % PW == PW - 1 ? lastm : 0xFFFFFFFFu);
      }
    }
  }
}

// Phase A of the global kernel for several patches with literal lists: waves claim 64 / S
// clauses at a time from *s_next and evaluate them in lane groups (eval_select_lm_group);
// clauses without a list take the include-mask walk in global memory, a wave each.  Results
// as the per-clause loop of train_global_body: selections, include counts, patch weights and
// votes into s_part.
template <bool INJECT, int S>
__device__ void global_eval_lm_groups(const TrainArgs& a, const Geom& g, const float* inj, uint64_t t, int64_t c_begin,
                                      int n_own, int* s_next, const uint16_t* s_lits, const int* s_nlit,
                                      const uint32_t* xt, int* s_sel, int* s_ninc, const float* s_wg, long long* s_part,
                                      const float* inv_rank, const int* s_drop) {
  constexpr int NG = kWave / S;
  const int lane = lane_id();
  const int q = lane / S, jj = lane & (S - 1);
  const int cap = g.list_cap;
  for (;;) {
    int idx0 = 0;
    if (lane == 0) idx0 = atomicAdd(s_next, NG);
    idx0 = lane_value(idx0, 0);
    if (idx0 >= n_own) break;
    const int idx = idx0 + q;
    const bool in = idx < n_own;
    const int ix = in ? idx : idx0;  // groups past the last clause read a valid one and discard it
    const int nl = s_nlit[ix];
    const bool listed = in && nl <= cap;
    const int64_t c = c_begin + ix;
    const int sel = eval_select_lm_group<INJECT, S>(a, g, inj, t, c, listed, s_lits + (int64_t)ix * cap, nl, xt,
                                                    s_drop[ix] != 0, inv_rank);
    if (listed) {
      if (jj == 0) {
        s_sel[idx] = sel;
        s_ninc[idx] = nl;
      }
      if (sel >= 0) {
        if (g.coalesced) {
          for (int k = jj; k < g.K; k += S)
            atomicAdd((unsigned long long*)&s_part[k], (unsigned long long)(long long)s_wg[(int64_t)ix * g.K + k]);
        } else if (jj == 0) {
          const int64_t k = c / g.per_bank;
          atomicAdd((unsigned long long*)&s_part[k], (unsigned long long)(long long)s_wg[(int64_t)ix * g.K + k]);
        }
      }
    }
    for (unsigned long long r = __ballot(in && !listed && jj == 0); r; r &= r - 1ull) {
      const int i2 = idx0 + (__ffsll((long long)r) - 1) / S;
      const int64_t c2 = c_begin + i2;
      int ninc;
      const uint32_t* m = a.planes + (c2 * g.np + g.np - 1) * g.W;
      const int sel2 = eval_select_lm<INJECT>(a, g, inj, c2, t, m, s_lits + (int64_t)i2 * cap, s_nlit[i2], cap, xt,
                                              s_drop[i2] != 0, &ninc, inv_rank);
      if (lane == 0) {
        s_sel[i2] = sel2;
        s_ninc[i2] = ninc;
      }
      if (sel2 >= 0) add_partial(a, g, s_part, c2, s_wg + (int64_t)i2 * g.K);
    }
  }
}

// Whether phase A of the global kernel evaluates four clauses to a wave
// (global_eval_lm_groups): bitmaps of at most 16 words and literal lists.
template <bool VANILLA>
__device__ __forceinline__ bool global_grouped(const Geom& g, int cap) {
  return !VANILLA && literal_major(g) && cap > 0 && (g.P + 31) / 32 <= 16;
}

// Phase A of sample j over the workgroup's clauses with state in global memory, claimed
// through *claim: selections and include counts into sel_out / ninc_out, the votes into
// part.  xt: the literal-major sample (several patches), xe: the sample's words (one
// patch: with mask_lds its LDS copy), masks: the LDS include masks (mask_lds); s_rb: the
// own clauses' rank_bits of sample j, or null.
template <bool VANILLA, bool INJECT>
__device__ __forceinline__ void global_phase_a(const TrainArgs& a, const Geom& g, int j, int64_t c_begin, int n_own,
                                               int* claim, const uint16_t* s_lits, const int* s_nlit, int cap,
                                               const uint32_t* xt, const uint32_t* xe, const uint32_t* s_mask,
                                               int* sel_out, int* ninc_out, const float* s_wg, long long* part,
                                               const float* inv_rank, const int* s_drop, const int* s_rb) {
  const int lane = lane_id();
  const uint64_t t = a.step0 + (uint64_t)j;
  const float* inj = INJECT ? a.inject + (int64_t)j * a.inject_block : nullptr;
  // Clauses with bitmaps of at most 16 words go four to a wave (eval_select_lm_group).  Two
  // to a wave (32-lane groups) lost on config 4: claims of two clauses balance the waves
  // worse (its phase A + barrier went from 10.8 to 11.5 us per sample).
  const bool grouped = global_grouped<VANILLA>(g, cap);
  if (grouped) {
    global_eval_lm_groups<INJECT, 16>(a, g, inj, t, c_begin, n_own, claim, s_lits, s_nlit, xt, sel_out, ninc_out, s_wg,
                                      part, inv_rank, s_drop);
    return;
  }
  for (;;) {
    int idx = 0;
    if (lane == 0) idx = atomicAdd(claim, 1);
    idx = lane_value(idx, 0);
    if (idx >= n_own) break;
    const int64_t c = c_begin + idx;
    int ninc;
    const uint32_t* m = g.mask_lds ? s_mask + (int64_t)idx * g.W : a.planes + (c * g.np + g.np - 1) * g.W;
    const int sel = (!VANILLA && literal_major(g))
                        ? eval_select_lm<INJECT>(a, g, inj, c, t, m, s_lits + (int64_t)idx * cap,
                                                 cap > 0 ? s_nlit[idx] : 0, cap, xt, s_drop[idx] != 0, &ninc, inv_rank,
                                                 s_rb ? s_rb[idx] : -1)
                        : eval_select<VANILLA, INJECT>(a, g, inj, c, t, m, xe, s_drop[idx] != 0, -1.0f, &ninc);
    if (lane == 0) {
      sel_out[idx] = sel;
      ninc_out[idx] = ninc;
    }
    if (sel >= 0) add_partial(a, g, part, c, s_wg + (int64_t)idx * g.K);
  }
}

// Clause state in global memory (L2/MALL resident across samples); any P.  A software
// pipeline over samples, like the resident kernel's; per sample i:
//   1. wave 0 adds the patch weights of sample i's selections (select_active,
//      kernel.cu:305) and publishes its partial class sums; then every wave stages sample
//      i+1 (its literal-major copy; with mask_lds its words) into LDS.
//   2. wave 0 waits for sample i's totals and derives the targets (phases B/C); the other
//      waves evaluate sample i+1 with the current state (phase A, speculative).
//   3. D: the feedback decisions of sample i (clause_update, kernel.cu:531-613) take
//      (clause, class) pairs, 64 / K clauses per claim (decide_pair), or a wave per clause
//      when K is above 32 (decide); a clause that changes takes back its speculative votes
//      for sample i+1 and is queued.  Then its literal updates: narrow clauses (W <= 32)
//      several to a wave, wide ones a 64-word chunk per wave.
//   4. the updated clauses rebuild their literal lists and are evaluated again for sample
//      i+1, so the result is exactly the sequential one.
// Phase A of sample i and its re-evaluations are over before sample i+1 is staged, so one
// literal-major buffer serves; the words of samples i and i+1 (mask_lds) take two.
template <bool VANILLA, bool INJECT>
__device__ __forceinline__ void train_global_body(const TrainArgs& a, const Geom& g) {
  extern __shared__ __attribute__((aligned(16))) long long dyn_lds[];  // 16-byte aligned: uint4 accesses
  __shared__ long long s_part[2][64];  // partial class sums by sample parity
  __shared__ int s_tgt[64];
  __shared__ double s_prob[64];
  __shared__ int s_next_a, s_next_d;  // clause claims of phase A and of the decisions
  __shared__ int s_abort;
  __shared__ int s_ntask;
  __shared__ int s_anyfb;  // some class of the current sample may update
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int nwv = (int)(blockDim.x / kWave);
  const int G = gridDim.x, wg = blockIdx.x;
  const int64_t c_begin = g.C * wg / G, c_end = g.C * (wg + 1) / G;
  const int n_own = (int)(c_end - c_begin);
  const int cpw = a.cpw;
  unsigned long long* s_task_m = (unsigned long long*)dyn_lds;  // [cpw][3] feedback masks
  int* s_sel = (int*)(s_task_m + 3 * cpw);                     // [2][cpw] by sample parity
  int* s_ninc = s_sel + 2 * cpw;                               // [2][cpw]
  int* s_task_idx = s_ninc + 2 * cpw;                          // [cpw]
  int* s_task_sb = s_task_idx + cpw;                           // [cpw] (zero: no precomputed draws)
  const int cap = VANILLA ? 0 : g.list_cap;                    // literal list capacity
  int* s_nlit = s_task_sb + cpw;                               // [cpw] include counts (cap > 0)
  uint16_t* s_lits = (uint16_t*)(s_nlit + (cap > 0 ? 2 * ((cpw + 1) / 2) : 0));  // [cpw][cap] literal lists
  uint32_t* s_xt = (uint32_t*)(s_lits + (int64_t)cpw * cap);  // [L][PW] when literal_major_lds(g)
  const int64_t cw = (int64_t)g.np * g.W;
  const int64_t xt_words = literal_major(g) ? g.L * ((g.P + 31) / 32) : 0;
  // mask_lds (one patch): the own clauses' include masks [cpw][W], kept current by the
  // literal updates, and the words of samples i and i+1 [2][W]
  uint32_t* s_mask = s_xt + (literal_major_lds(g) ? xt_words : 0);
  uint32_t* s_xs = s_mask + (g.mask_lds ? (int64_t)cpw * g.W : 0);
  float* s_wg = (float*)(s_xs + (g.mask_lds ? 2 * g.W : 0));  // the own clauses' weights [cpw][K]
  int* s_drop = (int*)(s_wg + (int64_t)cpw * g.K);              // [cpw] dropped (1) or not
  // several patches: the reservoir thresholds 1.0f / r, r = 0..P (a.inv_rank)
  float* s_invr = (float*)(s_drop + cpw);
  // several patches, counter stream, a clause per wave: the own clauses' rank_bits of
  // samples j, in buffer j & 1 [2][cpw]
  int* s_rb = (int*)(s_invr + (g.P > 1 ? g.P + 1 : 0));
  const bool lm = !VANILLA && literal_major(g);
  const bool use_rb = !INJECT && lm && !global_grouped<VANILLA>(g, cap);
  auto fill_rb = [&](int j, int first, int count) {
    for (int idx = first; idx < n_own; idx += count)
      s_rb[(j & 1) * cpw + idx] = rank_bits(a, g, c_begin + idx, a.step0 + (uint64_t)j, s_invr);
  };
  unsigned long long my_updates = 0ull, my_fb = 0ull;  // my_fb: samples where some class may update
  uint64_t wait_ticks = 0;
  const uint64_t t_kernel = __builtin_amdgcn_s_memrealtime();
  const bool prof = a.profile && wave == 0;
  uint64_t prof_acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  uint64_t prof_last = t_kernel;
  if (threadIdx.x < 128) (&s_part[0][0])[threadIdx.x] = 0;
  if (threadIdx.x == 0) {
    s_abort = 0;
    s_next_a = 0;
  }
  for (int64_t j = threadIdx.x; j < n_own * g.K; j += blockDim.x) s_wg[j] = a.weights[c_begin * g.K + j];
  for (int j = threadIdx.x; j < n_own; j += blockDim.x) s_drop[j] = a.drop[c_begin + j] == 1u;
  if (g.P > 1)
    for (int64_t j = threadIdx.x; j <= g.P; j += blockDim.x) s_invr[j] = a.inv_rank[j];
  if (g.mask_lds)  // include masks of the own clauses (visible after the first barrier below)
    for (int idx = wave; idx < n_own; idx += nwv)
      for (int64_t w = lane; w < g.W; w += kWave)
        s_mask[(int64_t)idx * g.W + w] = a.planes[(c_begin + idx) * cw + (int64_t)(g.np - 1) * g.W + w];
  if (cap > 0)  // literal lists of the own clauses (visible after the first barrier below)
    for (int idx = wave; idx < n_own; idx += nwv) {
      const int n = build_literal_list<false>(g, a.planes + (c_begin + idx) * cw + (int64_t)(g.np - 1) * g.W,
                                       s_lits + (int64_t)idx * cap, cap, a.lit_order);
      if (lane == 0) s_nlit[idx] = n;
    }
  if (use_rb) {  // the rank bits of samples 0 and 1 (from the thresholds, once they are in LDS)
    __syncthreads();
    for (int j = 0; j < 2 && j < a.N; ++j) fill_rb(j, threadIdx.x, blockDim.x);
  }
  // The LDS copy of sample j (threads [first, first + count)): literal-major words, or with
  // mask_lds the words into buffer j & 1.  The sample of phase A / re-evaluation: xt_of,
  // xe_of.
  auto stage = [&](int j, int first, int count) {
    if (g.mask_lds) copy_to_lds(s_xs + (int64_t)(j & 1) * g.W, a.X + (int64_t)j * g.W, g.W, first, count);
    if (lm && literal_major_lds(g)) {
      if (a.xt_halves)
        copy_halves_to_lds(g, s_xt, a.XT + (int64_t)j * xt_words, first, count);
      else
        copy_to_lds(s_xt, a.XT + (int64_t)j * xt_words, xt_words, first, count);
    }
  };
  // The same staging from registers, for the words of one-patch samples (mask_lds): each
  // thread's share of the sample after next is loaded one iteration ahead, so that staging
  // a sample is an LDS write (config 5: 373 -> 350 ms per epoch).  Not for literal-major
  // copies: their eight words per thread made config 4's kernel spill (499 -> 596 ms).
  constexpr int kStagePre = 8;
  const int64_t stage_n = g.mask_lds ? g.W : 0;
  const int per = (int)((stage_n + g.threads - 1) / g.threads);
  const bool prefetched = stage_n > 0 && per <= kStagePre;
  uint32_t pre[kStagePre];
  auto prefetch = [&](int j) {
    const uint32_t* src = a.X + (int64_t)j * g.W;
#pragma unroll
    for (int q = 0; q < kStagePre; ++q) {
      const int64_t idx = threadIdx.x + (int64_t)q * g.threads;
      if (q < per) pre[q] = src[idx < stage_n ? idx : stage_n - 1];  // clamped: every load unconditional
    }
  };
  auto commit = [&](int j) {
#pragma unroll
    for (int q = 0; q < kStagePre; ++q) {
      const int64_t idx = threadIdx.x + (int64_t)q * g.threads;
      if (q < per && idx < stage_n) {
        s_xs[(int64_t)(j & 1) * g.W + idx] = pre[q];
      }
    }
  };
  auto xt_of = [&](int j) -> const uint32_t* {
    return !lm ? nullptr : (literal_major_lds(g) ? s_xt : a.XT + (int64_t)j * xt_words);
  };
  auto xe_of = [&](int j) -> const uint32_t* {
    return g.mask_lds ? s_xs + (int64_t)(j & 1) * g.W : a.X + (int64_t)j * g.P * g.W;
  };
  const int kn = g.coalesced ? (int)g.K : 1;
  const int cpp = kWave / kn;
  if (prefetched && a.N > 0) prefetch(0);
  // i = -1 is the prologue: every wave stages sample 0 and takes part in its phase A
  for (int i = -1; i < a.N; ++i) {
    const uint64_t t = a.step0 + (uint64_t)i;
    const float* inj = INJECT && i >= 0 ? a.inject + (int64_t)i * a.inject_block : nullptr;
    const int b = i & 1, bn = b ^ 1;
    const bool more = i + 1 < a.N;
    int* sel_i = s_sel + b * cpw;
    int* ninc_i = s_ninc + b * cpw;
    int* sel_n = s_sel + bn * cpw;
    int* ninc_n = s_ninc + bn * cpw;

    // ---- 1: staging of sample i+1
    if (i >= 0 && wave == 0) {
      if (lane == 0) {
        s_next_a = 0;
        s_next_d = 0;
        s_ntask = 0;
      }
    }
    if (more) {
      if (prefetched) {
        commit(i + 1);
        if (i + 2 < a.N) prefetch(i + 2);
      } else {
        stage(i + 1, threadIdx.x, blockDim.x);
      }
    }
    __syncthreads();
    YTM_PROF_MARK(0);

    // ---- 2: the totals of sample i (wave 0, which publishes them first: the other waves
    // need not wait for that); speculative phase A of sample i+1 (the others)
    if (i >= 0 && wave == 0) {
      for (int idx = lane; idx < n_own; idx += kWave) {
        const int sl = sel_i[idx];
        if (sl >= 0) atomicAdd(&a.patch_w[(c_begin + idx) * g.P + sl], 1);
      }
      exchange_publish(a, g, i, s_part[b]);
      // the rank bits of sample i+2 while the sums are in flight (buffer i & 1: sample i's
      // phase A and re-evaluations are over)
      if (use_rb && i + 2 < a.N) fill_rb(i + 2, lane, kWave);
      long long S = 0;
      if (exchange_wait(a, g, i, lane < g.K ? lane : 0, lane < g.K, s_part[b], &S, &s_abort, &wait_ticks) &&
          lane < g.K)
        class_targets(g, lane, S + (long long)a.bias[lane], a.Y + (int64_t)i * g.K, s_tgt, s_prob);
      // samples where some class may update (workgroup 0 counts them); without one, the
      // sample's feedback (decisions, updates, re-evaluations) is skipped: every update needs
      // its draw u in (0, 1] at or below a probability above zero (kernel.cu:573-575)
      const bool anyfb = __ballot(lane < g.K && s_prob[lane < g.K ? lane : 0] > 0.0) != 0ull;
      if (wg == 0 && anyfb) ++my_fb;
      if (lane == 0) s_anyfb = anyfb;
      YTM_PROF_MARK(1);
    }
    // phase A of sample i+1: the other waves from the start, wave 0 once it has the totals
    if (more)
      global_phase_a<VANILLA, INJECT>(a, g, i + 1, c_begin, n_own, &s_next_a, s_lits, s_nlit, cap, xt_of(i + 1),
                                      xe_of(i + 1), s_mask, sel_n, ninc_n, s_wg, s_part[bn], s_invr, s_drop,
                                      use_rb ? s_rb + ((i + 1) & 1) * cpw : nullptr);
    __syncthreads();
    if (i < 0) {
      prof_last = __builtin_amdgcn_s_memrealtime();
      continue;
    }
    YTM_PROF_MARK(2);
    if (s_abort) break;
    if (!s_anyfb) continue;

    // ---- 3: decisions of sample i
    for (;;) {
      if (cpp < 2) break;  // decided a clause per wave below
      int base = 0;
      if (lane == 0) base = atomicAdd(&s_next_d, cpp);
      base = lane_value(base, 0);
      if (base >= n_own) break;
      const int jc = lane / kn, kk = lane - jc * kn;
      const int idx = base + jc;
      const bool valid = jc < cpp && idx < n_own;
      const int ix = valid ? idx : base;  // idle lanes read a valid clause and discard it
      const int64_t c = c_begin + ix;
      const int64_t k = (g.coalesced ? 0 : c / g.per_bank) + kk;
      float* wp = s_wg + (int64_t)ix * g.K + k;
      const float wold = *wp;
      float uq = 0.0f, uu = 0.0f;
      if (!INJECT) {
        const U4 z = counted_site(a, t, (uint32_t)c, TAG_CK, (uint32_t)k);
        uq = uniform_from_word(z.x);
        uu = uniform_from_word(z.y);
      }
      const PairOps po = decide_pair<INJECT>(g, inj, c, k, valid && s_drop[ix] == 0, sel_i[ix], ninc_i[ix], s_tgt[k],
                                             s_prob[k], 1.0, wold, uq, uu);
      if (po.t1a || po.t2) *wp = po.w_new;
      const unsigned long long b1a = __ballot(po.t1a), b1b = __ballot(po.t1b), bt2 = __ballot(po.t2);
      if ((b1a | b1b | bt2) == 0ull) continue;
      const unsigned long long seg = (1ull << kn) - 1ull;
      const int sh = jc * kn;
      const unsigned long long m1a = valid ? (b1a >> sh) & seg : 0ull;
      const unsigned long long m1b = valid ? (b1b >> sh) & seg : 0ull;
      const unsigned long long m2 = valid ? (bt2 >> sh) & seg : 0ull;
      const bool changes = (m1a | m1b | m2) != 0ull;
      // a changed clause takes back the votes it cast for sample i+1 with its old weights
      if (more && changes && sel_n[ix] >= 0)
        atomicAdd((unsigned long long*)&s_part[bn][k], (unsigned long long)(-(long long)wold));
      const bool leader = changes && kk == 0;
      my_updates += (unsigned long long)__popcll(__ballot(leader));
      if (leader) {
        const int tk = atomicAdd(&s_ntask, 1);
        s_task_idx[tk] = ix;
        s_task_sb[tk] = 0;
        s_task_m[tk * 3 + 0] = m1a;
        s_task_m[tk * 3 + 1] = m1b;
        s_task_m[tk * 3 + 2] = m2;
      }
    }
    for (;;) {
      if (cpp >= 2) break;  // decided in pairs above
      int idx = 0;
      if (lane == 0) idx = atomicAdd(&s_next_d, 1);
      idx = lane_value(idx, 0);
      if (idx >= n_own) break;
      const int64_t c = c_begin + idx;
      if (s_drop[idx]) continue;
      const int64_t kp = g.coalesced ? (lane < g.K ? lane : 0) : c / g.per_bank;
      const float wold = s_wg[(int64_t)idx * g.K + kp];
      const FbOps ops = decide<INJECT, false>(a, g, inj, c, t, sel_i[idx], ninc_i[idx], s_tgt, s_prob,
                                              s_wg + (int64_t)idx * g.K, nullptr, nullptr);
      if ((ops.m1a | ops.m1b | ops.m2) == 0ull) continue;
      if (more && sel_n[idx] >= 0 && (g.coalesced ? lane < g.K : lane == 0))
        atomicAdd((unsigned long long*)&s_part[bn][kp], (unsigned long long)(-(long long)wold));
      if (lane == 0) {
        ++my_updates;
        const int tk = atomicAdd(&s_ntask, 1);
        s_task_idx[tk] = idx;
        s_task_sb[tk] = 0;
        s_task_m[tk * 3 + 0] = ops.m1a;
        s_task_m[tk * 3 + 1] = ops.m1b;
        s_task_m[tk * 3 + 2] = ops.m2;
      }
    }
    __syncthreads();
    YTM_PROF_MARK(3);
    {
      const int ntask = s_ntask;
      const uint32_t* xe = xe_of(i);  // sample i's words, for the literal updates
      if (g.W <= 32) {
        // narrow clauses: up to 64 / W queued updates per wave at once
        const int per = tasks_per_wave(g, ntask, nwv);
        for (int tk0 = wave * per; tk0 < ntask; tk0 += nwv * per)
          apply_tasks<INJECT>(a, g, inj, c_begin, t, tk0, per, ntask, s_task_idx, s_task_m, s_task_sb, sel_i,
                              a.planes + c_begin * cw, xe, nullptr, 0, g.mask_lds ? s_mask : nullptr);
      } else {
        // wide clauses: (update, 64-word chunk) items over all waves; the chunks of one
        // clause touch disjoint literals
        const int nchunk = (int)((g.W + kWave - 1) / kWave);
        for (int item = wave; item < ntask * nchunk; item += nwv) {
          const int tk = item / nchunk, ch = item - tk * nchunk;
          const int idx = s_task_idx[tk];
          const FbOps ops{s_task_m[tk * 3 + 0], s_task_m[tk * 3 + 1], s_task_m[tk * 3 + 2]};
          apply_ops<INJECT>(a, g, inj, c_begin + idx, t, sel_i[idx], ops, a.planes + (c_begin + idx) * cw, xe, nullptr,
                            g.mask_lds ? s_mask + (int64_t)idx * g.W : nullptr, (int64_t)ch * kWave,
                            (int64_t)(ch + 1) * kWave);
        }
      }
    }
    __syncthreads();
    YTM_PROF_MARK(4);

    // ---- 4: the updated clauses' literal lists, and their phase A of sample i+1 again
    {
      const int ntask = s_ntask;
      const uint64_t tn = t + 1;
      const float* injn = INJECT && more ? a.inject + (int64_t)(i + 1) * a.inject_block : nullptr;
      for (int tk = wave; tk < ntask; tk += nwv) {
        const int idx = s_task_idx[tk];
        const int64_t c = c_begin + idx;
        const uint32_t* top = a.planes + c * cw + (int64_t)(g.np - 1) * g.W;
        if (cap > 0) {
          const int n = build_literal_list<false>(g, top, s_lits + (int64_t)idx * cap, cap, a.lit_order);
          if (lane == 0) s_nlit[idx] = n;
        }
        if (!more) continue;
        int ninc;
        const uint32_t* m = g.mask_lds ? s_mask + (int64_t)idx * g.W : top;
        const int sel = lm ? eval_select_lm<INJECT>(a, g, injn, c, tn, m, s_lits + (int64_t)idx * cap,
                                                    cap > 0 ? s_nlit[idx] : 0, cap, xt_of(i + 1), s_drop[idx] != 0,
                                                    &ninc, s_invr, use_rb ? s_rb[((i + 1) & 1) * cpw + idx] : -1)
                           : eval_select<VANILLA, INJECT>(a, g, injn, c, tn, m, xe_of(i + 1), s_drop[idx] != 0, -1.0f,
                                                          &ninc);
        if (lane == 0) {
          sel_n[idx] = sel;
          ninc_n[idx] = ninc;
        }
        if (sel >= 0) add_partial(a, g, s_part[bn], c, s_wg + (int64_t)idx * g.K);
      }
    }
    __syncthreads();
    YTM_PROF_MARK(5);
  }
  __syncthreads();
  for (int64_t j = threadIdx.x; j < n_own * g.K; j += blockDim.x) a.weights[c_begin * g.K + j] = s_wg[j];
  if (lane == 0 && my_updates) atomicAdd(&a.counters[0], my_updates);
  if (threadIdx.x == 0) {
    if (my_fb) atomicAdd(&a.counters[12], my_fb);
    atomicAdd(&a.counters[1], (unsigned long long)wait_ticks);
    atomicAdd(&a.counters[2], (unsigned long long)(__builtin_amdgcn_s_memrealtime() - t_kernel));
    if (prof)
      for (int j = 0; j < 8; ++j) atomicAdd(&a.counters[4 + j], (unsigned long long)prof_acc[j]);
  }
}

// Copies sample i (with one patch, its literal words; its K targets) into LDS buffer buf,
// threads [first, first + count) of the workgroup taking part.
__device__ __forceinline__ void stage_sample(const TrainArgs& a, const Geom& g, int i, int buf, uint32_t* s_x, int32_t* s_y,
                                             int first, int count) {
  if (g.P == 1)  // several patches: the clauses read the literal-major sample instead
    for (int64_t j = first; j < g.W; j += count) s_x[buf * g.W + j] = a.X[(int64_t)i * g.W + j];
  for (int64_t j = first; j < g.K; j += count) s_y[buf * g.K + j] = a.Y[(int64_t)i * g.K + j];
}

// Counter-stream draws of sample i for the workgroup's clauses, computed ahead of use
// into buffer buf: the reservoir draw of rank 1 (s_usel[buf][idx], one patch only) and the Q-skip / update
// draws (s_uq / s_uu [buf][idx][k]).  Threads [first, first + count) take part.
__device__ __forceinline__ void precompute_draws(const TrainArgs& a, const Geom& g, int i, int buf, int64_t c_begin,
                                                 int n_own, float* s_usel, float* s_uq, float* s_uu, int first,
                                                 int count) {
  const uint64_t t = a.step0 + (uint64_t)i;
  const int kn = g.coalesced ? (int)g.K : 1;
  const int per = kn + (g.P == 1 ? 1 : 0);  // the rank-1 draw serves one-patch models only
  for (int j = first; j < n_own * per; j += count) {
    const int idx = j / per, r = j % per;
    const int64_t c = c_begin + idx;
    if (r == kn) {
      s_usel[buf * a.cpw + idx] = uniform_from_word(counted_site(a, t, (uint32_t)c, TAG_SEL, 0u).x);
    } else {
      const int64_t k = (g.coalesced ? 0 : c / g.per_bank) + r;
      const U4 z = counted_site(a, t, (uint32_t)c, TAG_CK, (uint32_t)k);
      s_uq[((int64_t)buf * a.cpw + idx) * g.K + k] = uniform_from_word(z.x);
      s_uu[((int64_t)buf * a.cpw + idx) * g.K + k] = uniform_from_word(z.y);
    }
  }
}

// Copies the literal-major sample i ([L][PW] words) into LDS buffer buf of s_xt, threads
// [first, first + count) taking part.
__device__ __forceinline__ void stage_xt(const TrainArgs& a, const Geom& g, int i, int buf, uint32_t* s_xt, int first,
                                         int count) {
  const int64_t n = g.L * ((g.P + 31) / 32);
  copy_to_lds(s_xt + (int64_t)buf * n, a.XT + (int64_t)i * n, n, first, count);
}

// Staging of a literal-major sample around phase A: xt_prefetch issues the global loads of
// the first kXtPre word pairs per thread into registers, which nothing waits on until
// xt_commit stores them into LDS buffer buf and copies the rest (phase A in between reads
// only LDS).  Threads [first, first + count) take part.  An odd word count is copied whole
// by xt_commit.
constexpr int kXtPre = 2;
struct XtPre {
  uint2 v[kXtPre];
};
__device__ __forceinline__ void xt_prefetch(const TrainArgs& a, const Geom& g, int i, int first, int count, XtPre* r) {
  const int64_t n = g.L * ((g.P + 31) / 32);
  if (n & 1) return;
  const uint2* src = (const uint2*)(a.XT + (int64_t)i * n);
#pragma unroll
  for (int b = 0; b < kXtPre; ++b) {
    const int64_t j = first + (int64_t)b * count;
    if (j < n / 2) r->v[b] = src[j];
  }
}
__device__ __forceinline__ void xt_commit(const TrainArgs& a, const Geom& g, int i, int buf, uint32_t* s_xt, int first,
                                          int count, const XtPre& r) {
  const int64_t n = g.L * ((g.P + 31) / 32);
  if (n & 1) {
    stage_xt(a, g, i, buf, s_xt, first, count);
    return;
  }
  const uint2* src = (const uint2*)(a.XT + (int64_t)i * n);
  uint2* dst = (uint2*)(s_xt + (int64_t)buf * n);
#pragma unroll
  for (int b = 0; b < kXtPre; ++b) {
    const int64_t j = first + (int64_t)b * count;
    if (j < n / 2) dst[j] = r.v[b];
  }
  for (int64_t j = first + (int64_t)kXtPre * count; j < n / 2; j += count) dst[j] = src[j];
}

// Phase A of one resident clause (local index idx) on sample j, by one wave: selection
// (sel[idx]), include count (ninc[idx]), patch weight and the clause's votes added into
// part.  One patch: the sample's words are s_x[j % 3], the rank-1 draw s_usel[j % 3] and
// the patch weight s_pw[idx]; several patches: the literal-major sample is s_xt[j & 1] and
// the patch weight is counted in global memory.
template <bool INJECT>
__device__ __forceinline__ void resident_eval(const TrainArgs& a, const Geom& g, int j, int64_t c_begin, int idx,
                                              const uint32_t* s_planes, const float* s_w, const int* s_drop,
                                              const uint32_t* s_x, const uint32_t* s_xt, const float* s_usel,
                                              const float* inv_rank, const uint16_t* s_lits, const int* s_nlit,
                                              int* sel_out, int* ninc_out, int* s_pw, long long* part) {
  const int lane = lane_id();
  const int64_t c = c_begin + idx;
  const uint64_t t = a.step0 + (uint64_t)j;
  const float* inj = INJECT ? a.inject + (int64_t)j * a.inject_block : nullptr;
  // Inputs that do not depend on the evaluation are loaded first, so that their LDS reads
  // overlap those of the include mask and the sample.
  const int64_t kp = g.coalesced ? (lane < g.K ? lane : 0) : c / g.per_bank;
  const float wk = s_w[idx * g.K + kp];
  const bool dropped = s_drop[idx] != 0;
  const uint32_t* m = s_planes + (int64_t)idx * g.np * g.W + (int64_t)(g.np - 1) * g.W;
  int ninc, sel;
  if (g.P == 1)
    sel = eval_select<true, INJECT, !INJECT>(a, g, inj, c, t, m, s_x + (j % 3) * g.W, dropped,
                                             INJECT ? -1.0f : s_usel[(j % 3) * a.cpw + idx], &ninc);
  else
    sel = eval_select_lm<INJECT>(a, g, inj, c, t, m, s_lits + (int64_t)idx * g.list_cap, g.list_cap > 0 ? s_nlit[idx] : 0,
                                 g.list_cap, s_xt + (int64_t)(j & 1) * g.L * ((g.P + 31) / 32), dropped, &ninc,
                                 inv_rank);
  if (lane == 0) {
    sel_out[idx] = sel;
    ninc_out[idx] = ninc;
    if (sel >= 0 && g.P == 1) s_pw[idx] += 1;  // several patches: added once final (train_resident_body)
  }
  if (sel >= 0 && (g.coalesced ? lane < g.K : lane == 0))
    atomicAdd((unsigned long long*)&part[kp], (unsigned long long)(long long)wk);
}

// Phase A of resident clauses with several patches on sample j, 64 / S clauses per wave pass
// (eval_select_lm_group): passes b0, b0 + bstride, ... take clauses [b * 64/S, (b+1) * 64/S)
// below n_own.  Results as resident_eval: selections, include counts, patch weights (global
// memory) and the votes added into part.  Clauses without a literal list (more included
// literals than its capacity) take resident_eval's include-mask walk, a wave each.  Needs
// literal lists (list_cap > 0).
template <bool INJECT, int S>
__device__ void resident_eval_lm_groups(const TrainArgs& a, const Geom& g, int j, int64_t c_begin, int b0, int bstride,
                                        int n_own, const uint32_t* s_planes, const float* s_w, const int* s_drop,
                                        const uint32_t* s_x, const uint32_t* s_xt, const float* s_usel,
                                        const float* inv_rank, const uint16_t* s_lits, const int* s_nlit,
                                        int* sel_out, int* ninc_out, int* s_pw, long long* part) {
  constexpr int NG = kWave / S;
  const int lane = lane_id();
  const int q = lane / S, jj = lane & (S - 1);
  const uint64_t t = a.step0 + (uint64_t)j;
  const float* inj = INJECT ? a.inject + (int64_t)j * a.inject_block : nullptr;
  const int cap = g.list_cap;
  const uint32_t* xt = s_xt + (int64_t)(j & 1) * g.L * ((g.P + 31) / 32);
  for (int b = b0; b * NG < n_own; b += bstride) {
    const int idx = b * NG + q;
    const bool in = idx < n_own;
    const int ix = in ? idx : b * NG;  // groups past the last clause read a valid one and discard it
    const int nl = s_nlit[ix];
    const bool listed = in && nl <= cap;
    const int64_t c = c_begin + ix;
    const int sel = eval_select_lm_group<INJECT, S>(a, g, inj, t, c, listed, s_lits + (int64_t)ix * cap, nl, xt,
                                                    s_drop[ix] != 0, inv_rank);
    if (listed) {
      if (jj == 0) {
        sel_out[idx] = sel;
        ninc_out[idx] = nl;
      }
      if (sel >= 0) {
        if (g.coalesced) {
          for (int k = jj; k < g.K; k += S)
            atomicAdd((unsigned long long*)&part[k], (unsigned long long)(long long)s_w[(int64_t)ix * g.K + k]);
        } else if (jj == 0) {
          const int64_t k = c / g.per_bank;
          atomicAdd((unsigned long long*)&part[k], (unsigned long long)(long long)s_w[(int64_t)ix * g.K + k]);
        }
      }
    }
    // clauses without a literal list, a wave each
    for (unsigned long long r = __ballot(in && !listed && jj == 0); r; r &= r - 1ull)
      resident_eval<INJECT>(a, g, j, c_begin, b * NG + (__ffsll((long long)r) - 1) / S, s_planes, s_w, s_drop, s_x,
                            s_xt, s_usel, inv_rank, s_lits, s_nlit, sel_out, ninc_out, s_pw, part);
  }
}

// Phase A of the resident clauses idx0, idx0 + stride, ... with several patches on sample j:
// in lane groups when the literal lists and the patch bitmap allow, else a wave per clause.
template <bool INJECT>
__device__ __forceinline__ void resident_eval_lm(const TrainArgs& a, const Geom& g, int j, int64_t c_begin, int idx0,
                                                 int stride, int n_own, const uint32_t* s_planes, const float* s_w,
                                                 const int* s_drop, const uint32_t* s_x, const uint32_t* s_xt,
                                                 const float* s_usel, const float* inv_rank, const uint16_t* s_lits,
                                                 const int* s_nlit, int* sel_out, int* ninc_out, int* s_pw,
                                                 long long* part) {
  const int64_t PW = (g.P + 31) / 32;
  if (g.list_cap > 0 && PW <= 16)
    resident_eval_lm_groups<INJECT, 16>(a, g, j, c_begin, idx0, stride, n_own, s_planes, s_w, s_drop, s_x, s_xt, s_usel,
                                        inv_rank, s_lits, s_nlit, sel_out, ninc_out, s_pw, part);
  else if (g.list_cap > 0 && PW <= 32)
    resident_eval_lm_groups<INJECT, 32>(a, g, j, c_begin, idx0, stride, n_own, s_planes, s_w, s_drop, s_x, s_xt, s_usel,
                                        inv_rank, s_lits, s_nlit, sel_out, ninc_out, s_pw, part);
  else
    for (int idx = idx0; idx < n_own; idx += stride)
      resident_eval<INJECT>(a, g, j, c_begin, idx, s_planes, s_w, s_drop, s_x, s_xt, s_usel, inv_rank, s_lits, s_nlit,
                            sel_out, ninc_out, s_pw, part);
}

// Phase A of the one-patch clauses idx0, idx0 + stride, ... (below n_own) on sample j, by
// one wave, kEvalBatch clauses at a time: every LDS read of a batch is issued before any
// decision, and the batch's votes are summed in registers and added to part once.  The
// per-clause results are those of resident_eval (eval_select with one patch).
constexpr int kEvalBatch = 4;

// Most D1 passes (of 64 / kn clauses each) that wave 0 takes right after its exchange.
constexpr int kFusedPasses = 3;

template <bool INJECT>
__device__ void resident_eval_multi(const TrainArgs& a, const Geom& g, int j, int64_t c_begin, int idx0, int stride,
                                    int n_own, const uint32_t* s_planes, const float* s_w, const int* s_drop,
                                    const uint32_t* s_x, const float* s_usel, int* sel_out, int* ninc_out, int* s_pw,
                                    long long* part) {
  const int lane = lane_id();
  const float* inj = INJECT ? a.inject + (int64_t)j * a.inject_block : nullptr;
  const bool exact_count = g.maxinc < g.L;
  const uint32_t* x = s_x + (j % 3) * g.W;
  const int64_t cw = (int64_t)g.np * g.W;
  for (int r0 = idx0; r0 < n_own; r0 += kEvalBatch * stride) {
    uint32_t bad[kEvalBatch], any[kEvalBatch];
    int cnt[kEvalBatch];
#pragma unroll
    for (int b = 0; b < kEvalBatch; ++b) {
      bad[b] = 0u;
      any[b] = 0u;
      cnt[b] = 0;
    }
    for (int64_t w = lane; w < g.W; w += kWave) {
      const uint32_t nx = ~x[w];
#pragma unroll
      for (int b = 0; b < kEvalBatch; ++b) {
        const int idx = r0 + b * stride;
        if (idx < n_own) {
          const uint32_t mw = s_planes[idx * cw + (int64_t)(g.np - 1) * g.W + w];
          bad[b] |= mw & nx;
          any[b] |= mw;
          if (exact_count) cnt[b] += __popc(mw);
        }
      }
    }
    long long add = 0;  // lanes < K (coalesced): votes of the batch's selected clauses
#pragma unroll
    for (int b = 0; b < kEvalBatch; ++b) {
      const int idx = r0 + b * stride;
      if (idx >= n_own) continue;  // (no break: the loop must unroll for bad/any/cnt to stay in registers)
      const int64_t c = c_begin + idx;
      const int ninc = exact_count ? wave_sum_i32(cnt[b]) : (__any(any[b] != 0u) ? 1 : 0);
      const bool any_bad = __any(bad[b] != 0u);
      const float u = INJECT ? inj[c * g.P] : s_usel[(j % 3) * a.cpw + idx];
      // a clause fires on its one patch when it is empty or matches; it is selected when
      // its rank-1 draw is below 1.0f / 1 (eval_select)
      const int sel = (s_drop[idx] != 0 || (ninc != 0 && any_bad) || !(u < 1.0f)) ? -1 : 0;
      if (lane == 0) {
        sel_out[idx] = sel;
        ninc_out[idx] = ninc;
        if (sel >= 0) s_pw[idx] += 1;
      }
      if (sel >= 0) {
        if (g.coalesced) {
          if (lane < g.K) add += (long long)s_w[idx * g.K + lane];
        } else if (lane == 0) {
          const int64_t kb = c / g.per_bank;
          atomicAdd((unsigned long long*)&part[kb], (unsigned long long)(long long)s_w[idx * g.K + kb]);
        }
      }
    }
    if (g.coalesced && lane < g.K && add != 0) atomicAdd((unsigned long long*)&part[lane], (unsigned long long)add);
  }
}

// Patch weights of a sample's final selections with several patches (select_active,
// kernel.cu:305), added by wave 0 while it waits for the sample's class sums: the atomics'
// round trips then hold up no evaluation (a later load's wait would include them).  One
// patch keeps its patch weights in LDS instead.
__device__ __forceinline__ void flush_patch_weights(const TrainArgs& a, const Geom& g, int64_t c_begin, int n_own,
                                                    const int* sel) {
  if (g.P == 1) return;
  for (int idx = lane_id(); idx < n_own; idx += kWave) {
    const int sl = sel[idx];
    if (sl >= 0) atomicAdd(&a.patch_w[(c_begin + idx) * g.P + sl], 1);
  }
}

// Fused D1 (train_resident_body): the decisions of sample i were taken while other waves
// could still be reading the clause's weights for sample i+1, so the task's wave, before its
// literal updates, takes back the clause's speculative votes of sample i+1 (weights from
// before the update; spec_sel its selection there, -1 for none) and its patch-weight
// increment, then stores the new weights staged in task_w.  Lanes < K (coalesced) or lane 0
// (the own bank's class) take part.
__device__ __forceinline__ void commit_fused_task(const TrainArgs& a, const Geom& g, int64_t c_begin, int idx,
                                                  int spec_sel, const float* task_w, float* s_w, long long* part_next,
                                                  int* s_pw) {
  const int lane = lane_id();
  const int64_t c = c_begin + idx;
  const bool mine = g.coalesced ? lane < g.K : lane == 0;
  const int64_t k = g.coalesced ? (int64_t)lane : c / g.per_bank;
  if (mine) {
    float* wp = s_w + (int64_t)idx * g.K + k;
    if (spec_sel >= 0) atomicAdd((unsigned long long*)&part_next[k], (unsigned long long)(-(long long)*wp));
    *wp = task_w[k];
  }
  if (lane == 0 && spec_sel >= 0 && g.P == 1) s_pw[idx] -= 1;
}

// The votes of resident clause idx for the sample after the feedback again, with its new
// weights, when its literal updates left the include mask as it was: its evaluation (the
// selection sel and the include count) on that sample stands, so only what resident_eval
// adds after the evaluation is redone.
__device__ __forceinline__ void resident_revote(const Geom& g, int64_t c_begin, int idx, int sel, const float* s_w,
                                                int* s_pw, long long* part) {
  const int lane = lane_id();
  if (sel < 0) return;
  const int64_t c = c_begin + idx;
  const int64_t kp = g.coalesced ? (lane < g.K ? lane : 0) : c / g.per_bank;
  if (lane == 0 && g.P == 1) s_pw[idx] += 1;
  if (g.coalesced ? lane < g.K : lane == 0)
    atomicAdd((unsigned long long*)&part[kp], (unsigned long long)(long long)s_w[idx * g.K + kp]);
}

// Training with each workgroup's clause state resident in LDS for the whole launch:
// planes [own][np][W], weights [own][K] (and, with one patch, patch weights [own]) are
// loaded once, updated in place and written back at the end.  With several patches the
// clauses are evaluated on the literal-major samples, double-buffered in LDS.
//
// Per sample i, while wave 0 exchanges the class sums of sample i (phases B/C), the other
// waves evaluate sample i+1 speculatively against the state before i's feedback (phase A
// of i+1: selections, include counts, patch weights and partial sums), then stage sample
// i+2 and its counter-stream draws.  Feedback of sample i (phase D) then corrects the
// speculation exactly: a clause that runs any feedback branch takes back its speculative
// votes and patch-weight increment (with its weights from before the update), and after
// its literal updates its owning wave evaluates it again on sample i+1.  Clauses without
// feedback keep their speculative result, which is exact because their state did not
// change.  Samples, draws and selections are multi-buffered by sample index.
template <bool INJECT>
__device__ __forceinline__ void train_resident_body(const TrainArgs& a, const Geom& g) {
  extern __shared__ __attribute__((aligned(16))) long long dyn_lds[];  // 16-byte aligned: uint4 accesses
  __shared__ long long s_part[2][64];  // partial class sums of samples i and i+1
  __shared__ int s_tgt[64];
  __shared__ double s_prob[64];
  __shared__ int s_abort;
  __shared__ int s_ntask[2], s_nslot[2];  // queued tasks / draw slots, by sample parity
  __shared__ int s_anyfb;                  // some class of sample i may update (decisions after the exchange)
  __shared__ unsigned long long s_spec_max;  // profile: slowest wave's time in step 1 (waves >= 1)
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int nwv = blockDim.x / kWave;  // >= 2 (kTrainThreads)
  const int G = gridDim.x, wg = blockIdx.x;
  const int64_t c_begin = g.C * wg / G, c_end = g.C * (wg + 1) / G;
  const int n_own = (int)(c_end - c_begin);
  const int64_t cw = (int64_t)g.np * g.W;  // plane words per clause
  const int R = a.rng_slots;
  const int cpw = a.cpw;
  const int64_t xtw = g.P > 1 ? g.L * ((g.P + 31) / 32) : 0;     // literal-major sample words
  const int cap = g.P > 1 ? g.list_cap : 0;                       // literal list capacity
  unsigned long long* s_task_m = (unsigned long long*)dyn_lds;    // [cpw][3] feedback masks
  uint16_t* s_lits = (uint16_t*)(s_task_m + 3 * cpw);             // [cpw][cap] literal lists
  int* s_nlit = (int*)(s_lits + (int64_t)cpw * cap);              // [cpw] include counts
  uint32_t* s_xt = (uint32_t*)(s_nlit + (cap > 0 ? 2 * ((cpw + 1) / 2) : 0));  // [2][L][PW]
  uint32_t* s_planes = s_xt + 2 * xtw;                            // [cpw][np][W]
  float* s_w = (float*)(s_planes + cpw * cw);                     // [cpw][K]
  uint32_t* s_x = (uint32_t*)(s_w + cpw * g.K);                   // [3][W]
  int* s_sel = (int*)(s_x + 3 * g.W);                             // [2][cpw]
  int* s_ninc = s_sel + 2 * cpw;                                  // [2][cpw]
  int* s_drop = s_ninc + 2 * cpw;                                 // [cpw]
  int* s_pw = s_drop + cpw;                                       // [cpw]
  int32_t* s_y = s_pw + cpw;                                      // [3][K]
  float* s_bias = (float*)(s_y + 3 * g.K);                        // [K]
  float* s_usel = s_bias + g.K;                                   // [3][cpw]
  float* s_uq = s_usel + 3 * cpw;                                 // [3][cpw][K]
  float* s_uu = s_uq + 3 * cpw * g.K;                             // [3][cpw][K]
  int* s_task_idx = (int*)(s_uu + 3 * cpw * g.K);                 // [cpw]
  int* s_task_sb = s_task_idx + cpw;                              // [cpw] first draw slot
  float* s_task_w = (float*)(s_task_sb + cpw);                    // [cpw][K] new weights (fused D1)
  int* s_slot_idx = (int*)(s_task_w + cpw * g.K);                 // [R] clause of a draw slot
  int* s_slot_k = s_slot_idx + R;                                 // [R] class of a draw slot
  uint32_t* s_rng = (uint32_t*)(s_slot_k + R);                    // [R][W][kPreGroups][4]
  float* s_invr = (float*)(s_rng + (int64_t)R * g.W * kPreGroups * 4);  // [P+1] reservoir thresholds 1.0f / r
  unsigned long long my_updates = 0ull, my_fb = 0ull;  // my_fb: samples where some class may update
  uint64_t wait_ticks = 0;
  const uint64_t t_kernel = __builtin_amdgcn_s_memrealtime();
  // Optional phase timing (wave 0's view, 100 MHz real-time counter).
  const bool prof = a.profile && wave == 0;
  uint64_t prof_acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  uint64_t prof_last = 0;

  for (int64_t j = threadIdx.x; j < n_own * cw; j += blockDim.x) s_planes[j] = a.planes[c_begin * cw + j];
  for (int64_t j = threadIdx.x; j < n_own * g.K; j += blockDim.x) s_w[j] = a.weights[c_begin * g.K + j];
  for (int64_t j = threadIdx.x; j < n_own; j += blockDim.x) {
    s_drop[j] = a.drop[c_begin + j] == 1u;
    if (g.P == 1) s_pw[j] = a.patch_w[c_begin + j];
  }
  for (int64_t j = threadIdx.x; j < g.K; j += blockDim.x) s_bias[j] = a.bias[j];
  if (g.P > 1)
    for (int64_t j = threadIdx.x; j <= g.P; j += blockDim.x) s_invr[j] = a.inv_rank[j];
  for (int j = 0; j < 2 && j < a.N; ++j) {
    stage_sample(a, g, j, j, s_x, s_y, threadIdx.x, blockDim.x);
    if (g.P > 1) stage_xt(a, g, j, j, s_xt, threadIdx.x, blockDim.x);
    if (!INJECT) precompute_draws(a, g, j, j, c_begin, n_own, s_usel, s_uq, s_uu, threadIdx.x, blockDim.x);
  }
  if (threadIdx.x < 128) (&s_part[0][0])[threadIdx.x] = 0;
  if (threadIdx.x == 0) {
    s_abort = 0;
    s_ntask[0] = s_ntask[1] = 0;
    s_nslot[0] = s_nslot[1] = 0;
    s_spec_max = 0ull;
  }
  uint64_t spec_ticks = 0;  // profile: this wave's time in step 1 (waves >= 1)
  // Register prefetch of the one-patch samples (see step 1 below): thread q of waves >= 1,
  // counted from the last thread, holds word q (q < W) or target q - W (q < W + K).
  const int q = (int)blockDim.x - 1 - (int)threadIdx.x;
  const bool early = wave > 0 && g.P == 1 && g.W + g.K <= (int64_t)blockDim.x - kWave;
  uint32_t xq = 0u;
  int32_t yq = 0;
  if (early && a.N > 2) {
    if (q < g.W)
      xq = a.X[2 * g.W + q];
    else if (q < g.W + g.K)
      yq = a.Y[2 * g.K + (q - g.W)];
  }
  __syncthreads();
  if (cap > 0) {
    for (int idx = wave; idx < n_own; idx += nwv) {
      const int n = build_literal_list(g, s_planes + idx * cw + (int64_t)(g.np - 1) * g.W, s_lits + (int64_t)idx * cap,
                                       cap, a.lit_order);
      if (lane == 0) s_nlit[idx] = n;
    }
    __syncthreads();
  }
  // Phase A of sample 0, every wave.
  if (a.N > 0) {
    if (g.P == 1)
      resident_eval_multi<INJECT>(a, g, 0, c_begin, wave, nwv, n_own, s_planes, s_w, s_drop, s_x, s_usel, s_sel, s_ninc,
                                  s_pw, s_part[0]);
    else
      resident_eval_lm<INJECT>(a, g, 0, c_begin, wave, nwv, n_own, s_planes, s_w, s_drop, s_x, s_xt, s_usel, s_invr, s_lits,
                               s_nlit, s_sel, s_ninc, s_pw, s_part[0]);
  }
  __syncthreads();
  prof_last = __builtin_amdgcn_s_memrealtime();
  // Feedback decisions (D1) take lanes = (clause, class) pairs: kn classes per clause, cpp
  // clauses per pass of a wave.  When the classes are coalesced and the workgroup's clauses
  // fit in kFusedPasses passes, wave 0 takes the decisions itself as soon as its exchange
  // ends ("fused"): every lane polls the total of its own class and derives that class's
  // feedback, and the other inputs were loaded while the sums were in flight.  The other
  // waves may still be evaluating sample i+1 then, so the weight changes and the take-back
  // of speculative votes wait for the task's wave in D3 (commit_fused_task).  Otherwise D1
  // runs after a barrier, spread over the waves.
  const int kn = g.coalesced ? (int)g.K : 1;
  const int cpp = kWave / kn;
  const int jc = lane / kn, kk = lane - jc * kn;
  const unsigned long long seg = kn == kWave ? ~0ull : ((1ull << kn) - 1ull);
  // (from the geometry, which fixes cpw = ceil(C / grid) + 1, so that the specialised
  // kernels keep only one of the two paths)
  const int64_t cpw_g = (g.C + g.grid - 1) / g.grid + 1;
  const bool fused = g.coalesced && (cpw_g + cpp - 1) / cpp <= kFusedPasses;
  const long long bias_kk = (long long)s_bias[kk < g.K ? kk : 0];  // fused: class kk's bias (fixed for the launch)
  // Several patches: phase A of sample i+1 takes passes of lm_ng clauses, one per wave of
  // waves 1..; when that leaves two or more waves without a pass, those last waves
  // (stage_waves) stage sample i+2 while the others evaluate.  Staging threads are
  // [st_first, blockDim.x).  Decided from the geometry (g.threads is the launch's block
  // size, and no workgroup owns more than ceil(C / grid) clauses), so that a specialised
  // kernel keeps one of the two paths.
  const int64_t pw_words = (g.P + 31) / 32;
  const int lm_ng = g.list_cap > 0 && pw_words <= 16 ? 4 : (g.list_cap > 0 && pw_words <= 32 ? 2 : 1);
  const int64_t own_max = (g.C + g.grid - 1) / g.grid;
  const int lm_idle = (int)(g.threads / kWave - 1 - (own_max + lm_ng - 1) / lm_ng);
  const int stage_waves = g.P > 1 && lm_idle >= 2 ? lm_idle : 0;
  const int st_first = (nwv - (stage_waves ? stage_waves : nwv - 1)) * kWave;
  const int st_count = (int)blockDim.x - st_first;

  for (int i = 0; i < a.N; ++i) {
    const uint64_t t = a.step0 + (uint64_t)i;
    const float* inj = INJECT ? a.inject + (int64_t)i * a.inject_block : nullptr;
    const int b3 = i % 3, b3n = (i + 1) % 3, b2 = i & 1, b2n = b2 ^ 1;
    // the sample's patch-major words, for the literal updates
    const uint32_t* xe = g.P == 1 ? s_x + b3 * g.W : a.X + (int64_t)i * g.P * g.W;
    const bool more = i + 1 < a.N;

    // ---- B + C on wave 0; speculative A of sample i+1 and staging of i+2 on the others
    if (wave == 0) {
      if (lane == 0) {
        s_ntask[b2] = 0;
        s_nslot[b2] = 0;
      }
      if (fused) {
        exchange_publish(a, g, i, s_part[b2]);
        flush_patch_weights(a, g, c_begin, n_own, s_sel + b2 * cpw);
        // the decisions' inputs, loaded while the class sums are exchanged; lane (jc, kk)
        // takes class kk of clause p * cpp + jc in pass p
        const ClassPrep cp = class_prep(g, s_y[b3 * g.K + kk]);
        PairPre pre[kFusedPasses];
#pragma unroll
        for (int p = 0; p < kFusedPasses; ++p) {
          const int idx = p * cpp + jc;
          const bool valid = jc < cpp && idx < n_own;
          const int ix = valid ? idx : 0;  // idle lanes read clause 0 and discard it
          const int64_t k = kk;
          pre[p] = pair_pre<INJECT>(g, inj, c_begin + ix, k, valid && s_drop[ix] == 0, s_sel[b2 * cpw + ix],
                                    s_ninc[b2 * cpw + ix], cp.den, s_w[ix * g.K + k],
                                    INJECT ? 0.0f : s_uq[((int64_t)b3 * cpw + ix) * g.K + k],
                                    INJECT ? 0.0f : s_uu[((int64_t)b3 * cpw + ix) * g.K + k]);
          pin(pre[p]);
        }
        long long S = 0;
        const bool ok = exchange_wait(a, g, i, kk, true, s_part[b2], &S, &s_abort, &wait_ticks);
        YTM_PROF_MARK(0);
        if (ok) {
          const ClassTest fb = class_test(g, S + bias_kk, cp);  // every lane: class kk
          // samples where some class may update (workgroup 0 counts them)
          if (wg == 0 && __ballot(fb.num > 0.0) != 0ull) ++my_fb;
#pragma unroll
          for (int p = 0; p < kFusedPasses; ++p) {
            if (p * cpp >= n_own) continue;  // (no break: the loop must unroll for pre[] to stay in registers)
            const PairOps po = pair_decide(g, pre[p], fb.tgt, fb.num);
            const unsigned long long b1a = __ballot(po.t1a), b1b = __ballot(po.t1b), bt2 = __ballot(po.t2);
            if ((b1a | b1b | bt2) == 0ull) continue;
            const int idx = p * cpp + jc;
            const bool valid = jc < cpp && idx < n_own;
            const int ix = valid ? idx : 0;
            const int64_t k = kk;
            const int sh = jc * kn;
            const unsigned long long m1a = valid ? (b1a >> sh) & seg : 0ull;
            const unsigned long long m1b = valid ? (b1b >> sh) & seg : 0ull;
            const unsigned long long m2 = valid ? (bt2 >> sh) & seg : 0ull;
            const bool changes = (m1a | m1b | m2) != 0ull;
            const bool leader = changes && kk == 0;
            my_updates += (unsigned long long)__popcll(__ballot(leader));
            int tk = 0;
            if (leader) {
              const unsigned long long rng = INJECT ? 0ull : (m1a | m1b);
              tk = atomicAdd(&s_ntask[b2], 1);
              const int sb = INJECT ? 0 : atomicAdd(&s_nslot[b2], __popcll(rng));
              s_task_idx[tk] = ix;
              s_task_sb[tk] = sb;
              s_task_m[tk * 3 + 0] = m1a;
              s_task_m[tk * 3 + 1] = m1b;
              s_task_m[tk * 3 + 2] = m2;
              int jj = sb;
              for (unsigned long long r = rng; r; r &= r - 1ull, ++jj) {
                if (jj < R) {
                  s_slot_idx[jj] = ix;
                  s_slot_k[jj] = __ffsll((long long)r) - 1;
                }
              }
            }
            tk = __shfl(tk, sh);  // the clause's task, from its first lane
            if (changes) s_task_w[tk * g.K + k] = (po.t1a || po.t2) ? po.w_new : pre[p].w0;
          }
        }
        YTM_PROF_MARK(2);
      } else {
        exchange_publish(a, g, i, s_part[b2]);
        flush_patch_weights(a, g, c_begin, n_own, s_sel + b2 * cpw);
        long long S = 0;
        if (exchange_wait(a, g, i, lane < g.K ? lane : 0, lane < g.K, s_part[b2], &S, &s_abort, &wait_ticks) &&
            lane < g.K)
          class_targets(g, lane, S + (long long)s_bias[lane], s_y + b3 * g.K, s_tgt, s_prob);
        // samples where some class may update (workgroup 0 counts them); without one, D1 is
        // skipped (every update needs its draw u in (0, 1] at or below a probability above
        // zero, kernel.cu:573-575)
        const bool anyfb = __ballot(lane < g.K && s_prob[lane < g.K ? lane : 0] > 0.0) != 0ull;
        if (wg == 0 && anyfb) ++my_fb;
        if (lane == 0) s_anyfb = anyfb;
        YTM_PROF_MARK(0);
      }
    } else {
      const uint64_t spec_t0 = a.profile ? __builtin_amdgcn_s_memrealtime() : 0;
      // One patch: sample i+2 was read from global memory one iteration ago (one word or
      // target per thread of the last waves); it goes to LDS now, and sample i+3 is read
      // into the same registers, so no wait on the read latency remains.
      if (early) {
        if (i + 2 < a.N) {
          if (q < g.W)
            s_x[((i + 2) % 3) * g.W + q] = xq;
          else if (q < g.W + g.K)
            s_y[((i + 2) % 3) * g.K + (q - g.W)] = yq;
        }
        if (i + 3 < a.N) {
          if (q < g.W)
            xq = a.X[(int64_t)(i + 3) * g.W + q];
          else if (q < g.W + g.K)
            yq = a.Y[(int64_t)(i + 3) * g.K + (q - g.W)];
        }
      }
      // Several patches: the waves without a pass of phase A (stage_waves) stage sample i+2
      // meanwhile; without such waves, every wave stages it after phase A, its literal-major
      // words read into registers before.
      XtPre xpre;
      if (g.P > 1 && !stage_waves && i + 2 < a.N)
        xt_prefetch(a, g, i + 2, threadIdx.x - kWave, blockDim.x - kWave, &xpre);
      if (more) {
        if (g.P == 1)
          resident_eval_multi<INJECT>(a, g, i + 1, c_begin, wave - 1, nwv - 1, n_own, s_planes, s_w, s_drop, s_x, s_usel,
                                      s_sel + b2n * cpw, s_ninc + b2n * cpw, s_pw, s_part[b2n]);
        else
          resident_eval_lm<INJECT>(a, g, i + 1, c_begin, wave - 1, nwv - 1, n_own, s_planes, s_w, s_drop, s_x, s_xt, s_usel,
                                   s_invr, s_lits, s_nlit, s_sel + b2n * cpw, s_ninc + b2n * cpw, s_pw, s_part[b2n]);
      }
      if (a.profile == 2) spec_ticks += __builtin_amdgcn_s_memrealtime() - spec_t0;
      if (i + 2 < a.N && (int)threadIdx.x >= st_first) {
        const int b3nn = (i + 2) % 3;
        const int st = (int)threadIdx.x - st_first;
        if (!early) stage_sample(a, g, i + 2, b3nn, s_x, s_y, st, st_count);
        if (a.profile == 3) spec_ticks += __builtin_amdgcn_s_memrealtime() - spec_t0;
        if (g.P > 1) {
          if (stage_waves)
            stage_xt(a, g, i + 2, b2, s_xt, st, st_count);
          else
            xt_commit(a, g, i + 2, b2, s_xt, st, st_count, xpre);
        }
        if (!INJECT) precompute_draws(a, g, i + 2, b3nn, c_begin, n_own, s_usel, s_uq, s_uu, st, st_count);
      }
      if (a.profile == 1) spec_ticks += __builtin_amdgcn_s_memrealtime() - spec_t0;
    }
    __syncthreads();
    YTM_PROF_MARK(1);
    if (s_abort) break;

    // ---- D1: feedback decisions of sample i; the clauses that change take back their
    // speculative votes of sample i+1 and are queued.  With at most one clause per wave,
    // each wave decides its clause (decide, lanes = classes); with more, lanes take
    // (clause, class) pairs, kn classes per clause and 64 / kn clauses per wave pass
    // (decide_pair), and a clause is queued by its first lane.
    if (!fused) {
      if (!s_anyfb) continue;  // no class of sample i can update: nothing is queued
      if (n_own <= nwv) {
        for (int idx = wave; idx < n_own; idx += nwv) {
          const int64_t c = c_begin + idx;
          const int64_t kp = g.coalesced ? (lane < g.K ? lane : 0) : c / g.per_bank;
          const float wold = s_w[idx * g.K + kp];
          const FbOps ops = decide<INJECT, !INJECT>(a, g, inj, c, t, s_sel[b2 * cpw + idx], s_ninc[b2 * cpw + idx], s_tgt,
                                                    s_prob, s_w + idx * g.K, s_uq + ((int64_t)b3 * cpw + idx) * g.K,
                                                    s_uu + ((int64_t)b3 * cpw + idx) * g.K, s_drop[idx] != 0);
          if ((ops.m1a | ops.m1b | ops.m2) == 0ull) continue;
          const int spec_sel = more ? s_sel[b2n * cpw + idx] : -1;
          if (spec_sel >= 0) {
            if (g.coalesced ? lane < g.K : lane == 0)
              atomicAdd((unsigned long long*)&s_part[b2n][kp], (unsigned long long)(-(long long)wold));
            if (lane == 0 && g.P == 1) s_pw[idx] -= 1;
          }
          if (lane == 0) {
            ++my_updates;
            const unsigned long long rng = INJECT ? 0ull : (ops.m1a | ops.m1b);
            const int tk = atomicAdd(&s_ntask[b2], 1);
            const int sb = INJECT ? 0 : atomicAdd(&s_nslot[b2], __popcll(rng));
            s_task_idx[tk] = idx;
            s_task_sb[tk] = sb;
            s_task_m[tk * 3 + 0] = ops.m1a;
            s_task_m[tk * 3 + 1] = ops.m1b;
            s_task_m[tk * 3 + 2] = ops.m2;
            const int64_t kb = g.coalesced ? 0 : c / g.per_bank;
            int j = sb;
            for (unsigned long long r = rng; r; r &= r - 1ull, ++j) {
              if (j < R) {
                s_slot_idx[j] = idx;
                s_slot_k[j] = (int)(kb + __ffsll((long long)r) - 1);
              }
            }
          }
        }
      } else {
        for (int base = wave * cpp; base < n_own; base += nwv * cpp) {
          const int idx = base + jc;
          const bool valid = jc < cpp && idx < n_own;
          const int ix = valid ? idx : base;  // idle lanes read a valid clause and discard it
          const int64_t c = c_begin + ix;
          const int64_t k = (g.coalesced ? 0 : c / g.per_bank) + kk;
          float* wp = s_w + (int64_t)ix * g.K + k;
          const float wold = *wp;
          const PairOps po = decide_pair<INJECT>(g, inj, c, k, valid && s_drop[ix] == 0, s_sel[b2 * cpw + ix],
                                                 s_ninc[b2 * cpw + ix], s_tgt[k], s_prob[k], 1.0, wold,
                                                 s_uq[((int64_t)b3 * cpw + ix) * g.K + k],
                                                 s_uu[((int64_t)b3 * cpw + ix) * g.K + k]);
          if (po.t1a || po.t2) *wp = po.w_new;
          const unsigned long long b1a = __ballot(po.t1a), b1b = __ballot(po.t1b), bt2 = __ballot(po.t2);
          if ((b1a | b1b | bt2) == 0ull) continue;
          const int sh = jc * kn;
          const unsigned long long m1a = valid ? (b1a >> sh) & seg : 0ull;
          const unsigned long long m1b = valid ? (b1b >> sh) & seg : 0ull;
          const unsigned long long m2 = valid ? (bt2 >> sh) & seg : 0ull;
          const bool changes = (m1a | m1b | m2) != 0ull;
          const int spec_sel = more && changes ? s_sel[b2n * cpw + ix] : -1;
          if (spec_sel >= 0)
            atomicAdd((unsigned long long*)&s_part[b2n][k], (unsigned long long)(-(long long)wold));
          const bool leader = changes && kk == 0;
          my_updates += (unsigned long long)__popcll(__ballot(leader));
          if (leader) {
            if (spec_sel >= 0 && g.P == 1) s_pw[ix] -= 1;
            const unsigned long long rng = INJECT ? 0ull : (m1a | m1b);
            const int tk = atomicAdd(&s_ntask[b2], 1);
            const int sb = INJECT ? 0 : atomicAdd(&s_nslot[b2], __popcll(rng));
            s_task_idx[tk] = ix;
            s_task_sb[tk] = sb;
            s_task_m[tk * 3 + 0] = m1a;
            s_task_m[tk * 3 + 1] = m1b;
            s_task_m[tk * 3 + 2] = m2;
            const int64_t kb = g.coalesced ? 0 : c / g.per_bank;
            int jj = sb;
            for (unsigned long long r = rng; r; r &= r - 1ull, ++jj) {
              if (jj < R) {
                s_slot_idx[jj] = ix;
                s_slot_k[jj] = (int)(kb + __ffsll((long long)r) - 1);
              }
            }
          }
        }
      }
      YTM_PROF_MARK(2);
      __syncthreads();
      YTM_PROF_MARK(3);
    }
    const int ntask = s_ntask[b2];
    if (ntask == 0) continue;
    if (!INJECT) {
      // D2: the whole workgroup computes the leading plane groups of every queued draw
      const int nslot = min(s_nslot[b2], R);
      const int npre = draw_groups(g.s_thr) < kPreGroups ? draw_groups(g.s_thr) : kPreGroups;
      const int per_slot = (int)g.W * npre;
      for (int item = threadIdx.x; npre > 0 && item < nslot * per_slot; item += blockDim.x) {
        const int sl = item / per_slot, rem = item % per_slot;
        const int64_t w = rem / npre;
        const int grp = rem % npre;
        const int64_t k = s_slot_k[sl];
        const U4 z = counted_site(a, t, (uint32_t)(c_begin + s_slot_idx[sl]), TAG_LIT,
                                (uint32_t)((k * g.W + w) * 6 + grp));
        uint32_t* dst = s_rng + ((int64_t)sl * g.W + w) * (kPreGroups * 4) + grp * 4;
        dst[0] = z.x;
        dst[1] = z.y;
        dst[2] = z.z;
        dst[3] = z.w;
      }
      __syncthreads();
    }
    YTM_PROF_MARK(4);
    // D3: the waves apply the queued updates (round-robin), each then evaluating its clause
    // again on sample i+1 with the new state
    if (g.W <= 32) {
      // narrow clauses: up to 64 / W tasks per wave at once
      const int per = tasks_per_wave(g, ntask, nwv);
      for (int tk0 = wave * per; tk0 < ntask; tk0 += nwv * per) {
        if (fused)
          for (int tk = tk0; tk < tk0 + per && tk < ntask; ++tk) {
            const int idx = s_task_idx[tk];
            commit_fused_task(a, g, c_begin, idx, more ? s_sel[b2n * cpw + idx] : -1, s_task_w + tk * g.K, s_w,
                              s_part[b2n], s_pw);
          }
        unsigned long long chg = 0ull;
        apply_tasks<INJECT>(a, g, inj, c_begin, t, tk0, per, ntask, s_task_idx, s_task_m, s_task_sb,
                            s_sel + b2 * cpw, s_planes, xe, INJECT ? nullptr : s_rng, R, nullptr, &chg);
        const unsigned long long wmask = (1ull << g.W) - 1ull;
        // a task whose include mask is unchanged keeps its list and its evaluation of sample
        // i+1; only its votes come back with the new weights (resident_revote)
        if (cap > 0)
          for (int tk = tk0; tk < tk0 + per && tk < ntask; ++tk) {
            if (((chg >> ((tk - tk0) * g.W)) & wmask) == 0ull) continue;
            const int idx = s_task_idx[tk];
            const int n = build_literal_list(g, s_planes + idx * cw + (int64_t)(g.np - 1) * g.W,
                                             s_lits + (int64_t)idx * cap, cap, a.lit_order);
            if (lane == 0) s_nlit[idx] = n;
          }
        if (more)
          for (int tk = tk0; tk < tk0 + per && tk < ntask; ++tk) {
            const int idx = s_task_idx[tk];
            if (((chg >> ((tk - tk0) * g.W)) & wmask) == 0ull)
              resident_revote(g, c_begin, idx, s_sel[b2n * cpw + idx], s_w, s_pw, s_part[b2n]);
            else
              resident_eval<INJECT>(a, g, i + 1, c_begin, idx, s_planes, s_w, s_drop, s_x, s_xt, s_usel, s_invr,
                                    s_lits, s_nlit, s_sel + b2n * cpw, s_ninc + b2n * cpw, s_pw, s_part[b2n]);
          }
      }
    } else {
      for (int tk = wave; tk < ntask; tk += nwv) {  // tasks round-robin over the waves
        const int idx = s_task_idx[tk];
        if (fused)
          commit_fused_task(a, g, c_begin, idx, more ? s_sel[b2n * cpw + idx] : -1, s_task_w + tk * g.K, s_w,
                            s_part[b2n], s_pw);
        const FbOps ops{s_task_m[tk * 3 + 0], s_task_m[tk * 3 + 1], s_task_m[tk * 3 + 2]};
        const int sb = s_task_sb[tk];
        const bool have = !INJECT && sb + __popcll(ops.m1a | ops.m1b) <= R;
        apply_ops<INJECT>(a, g, inj, c_begin + idx, t, s_sel[b2 * cpw + idx], ops, s_planes + idx * cw, xe,
                          have ? s_rng + (int64_t)sb * g.W * (kPreGroups * 4) : nullptr);
        if (cap > 0) {
          const int n = build_literal_list(g, s_planes + idx * cw + (int64_t)(g.np - 1) * g.W,
                                           s_lits + (int64_t)idx * cap, cap, a.lit_order);
          if (lane == 0) s_nlit[idx] = n;
        }
        if (more)
          resident_eval<INJECT>(a, g, i + 1, c_begin, idx, s_planes, s_w, s_drop, s_x, s_xt, s_usel, s_invr, s_lits, s_nlit,
                                s_sel + b2n * cpw, s_ninc + b2n * cpw, s_pw, s_part[b2n]);
      }
    }
    YTM_PROF_MARK(5);
    __syncthreads();
    YTM_PROF_MARK(6);
  }
  __syncthreads();
  for (int64_t j = threadIdx.x; j < n_own * cw; j += blockDim.x) a.planes[c_begin * cw + j] = s_planes[j];
  for (int64_t j = threadIdx.x; j < n_own * g.K; j += blockDim.x) a.weights[c_begin * g.K + j] = s_w[j];
  if (g.P == 1)
    for (int64_t j = threadIdx.x; j < n_own; j += blockDim.x) a.patch_w[c_begin + j] = s_pw[j];
  if (lane == 0 && my_updates) atomicAdd(&a.counters[0], my_updates);
  if (a.profile && lane == 0 && wave > 0) atomicMax(&s_spec_max, (unsigned long long)spec_ticks);
  __syncthreads();
  if (threadIdx.x == 0) {
    if (my_fb) atomicAdd(&a.counters[12], my_fb);
    atomicAdd(&a.counters[1], (unsigned long long)wait_ticks);
    atomicAdd(&a.counters[2], (unsigned long long)(__builtin_amdgcn_s_memrealtime() - t_kernel));
    if (prof) {
      prof_acc[7] = s_spec_max;  // slot 7: the workgroup's slowest wave in step 1
      for (int j = 0; j < 8; ++j) atomicAdd(&a.counters[4 + j], (unsigned long long)prof_acc[j]);
    }
  }
}

// ========================================================================= streaming
// One-patch models, coalesced classes, counter stream, at most 64 clauses per workgroup
// (one lane each).  A sample changes the clause state only when some class has an update
// probability above zero: the update draw u lies in (0, 1] and a class updates only when
// u <= prob (kernel.cu:508-529,573-575), so with prob <= 0 for every class no weight and no
// TA state changes (the patch weights do, but nothing reads them during training).  Once a
// model is trained, most samples are like that (config 2 after five epochs: 96%).
//
// So the workgroups stream: each evaluates the samples ahead of the one being consumed with
// the current state and publishes their partial class sums (one flat row of K words per
// sample, every workgroup adding (1 << 44) | partial), while wave 0 consumes the completed
// rows in order.  A consumed sample whose classes all have prob <= 0 only commits its patch
// weights; the rows already published for later samples stay exact because nothing
// changed.  The first sample with some prob > 0 stops the stream in every workgroup (all
// see the same sums): the workgroup takes that sample's feedback decisions and literal
// updates (the same functions as the resident kernel).  The rows it published past the
// stop were evaluated with the state before the feedback; only its updated clauses vote
// differently now, so it adds their vote differences to each such row as one more unit,
// and streaming goes on at the next sample.  After k stops in a stream every row is
// complete at G * (k + 1) units: a row published from then on carries k + 1 units at once.
// The result is exactly the sequential one.
//
// Rows of a stream that starts at sample b with first row r0: row(s) = r0 + (s - b).  A
// workgroup publishes a sample only while it is fewer than kStreamDepth samples ahead of
// the one it consumes.  Once a stream has taken as many stops as the unit count allows
// (or a.stream_gens), the next one starts on fresh rows past the stop sample j: at row
// r0 + (j + 1 - b) + kStreamDepth, so the rows published past the stop are never read.
// Every workgroup derives the same rows from the same stops.
struct StreamCtl {
  int claim;    // next sample to evaluate
  int consume;  // next sample to consume: every earlier sample of this stream is final
  int stop;     // -1 while streaming; then the sample that needs feedback, or N
  int abort;
};

__device__ __forceinline__ int lds_load(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_store(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void train_stream_body(const TrainArgs& a, const Geom& g) {
  extern __shared__ __attribute__((aligned(16))) long long dyn_lds[];  // 16-byte aligned: uint4 accesses
  __shared__ StreamCtl ctl;
  __shared__ unsigned long long s_ring[kStreamDepth];  // selected clauses of in-flight samples
  __shared__ int s_pub[kStreamDepth];                  // the sample of each ring slot this workgroup published
  __shared__ int s_wmax;                               // bound on |integer weight| of the own clauses
  __shared__ long long s_S[64];                        // class sums + bias of the stop sample
  __shared__ int s_ntask;
  __shared__ int s_vdirty[64];                         // vote tables: nibble groups changed at a stop, per class
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int nwv = blockDim.x / kWave;
  const int G = gridDim.x, wg = blockIdx.x;
  const int64_t c_begin = g.C * wg / G, c_end = g.C * (wg + 1) / G;
  const int n_own = (int)(c_end - c_begin);  // <= kStreamClauses
  const int64_t cw = (int64_t)g.np * g.W;
  const int K = (int)g.K;
  const int64_t Wp = (g.W + 3) & ~(int64_t)3;
  constexpr int D = kStreamDepth;
  // LDS (sizes in stream_lds_bytes): task masks [64][3] u64; planes [64][np][W]; weights
  // [64][K]; transposed integer weights [K][64]; include counts, drop, patch weights, task
  // clauses, zeros, selections of the stop sample [64] each; targets ring [D][K];
  // complemented samples ring [D][Wp]; integer weights before a stop [K][64]; the include
  // masks again, word-major [Wp / 4][64] uint4 (lane = clause, four words per read).
  unsigned long long* s_task_m = (unsigned long long*)dyn_lds;
  uint32_t* s_planes = (uint32_t*)(s_task_m + 3 * kStreamClauses);
  float* s_w = (float*)(s_planes + (int64_t)kStreamClauses * cw);
  int* s_wt = (int*)(s_w + kStreamClauses * K);
  int* s_ninc = s_wt + K * kStreamClauses;
  int* s_drop = s_ninc + kStreamClauses;
  int* s_pw = s_drop + kStreamClauses;
  int* s_task_idx = s_pw + kStreamClauses;
  int* s_zero = s_task_idx + kStreamClauses;
  int* s_selj = s_zero + kStreamClauses;
  int32_t* s_yring = s_selj + kStreamClauses;
  uint32_t* s_nx = (uint32_t*)(s_yring + D * K);
  int* s_wt_old = (int*)(s_nx + (int64_t)D * Wp);  // [K][64] integer weights before a stop
  uint4* s_maskT = (uint4*)(s_wt_old + K * kStreamClauses);
  const int64_t Wq = Wp / 4;
  // g.vote_table: class votes from nibble tables [16][16][K] int16, entry (j, v, k) the sum
  // of the integer weights of class k of the clauses 4j + b with bit b of v set; a
  // selection mask then gives lane k its class's vote in 16 table reads.  Exact while every
  // own |weight| is below 512 (an entry stays within +-2044), as the paired reduction.
  short* s_vt = (short*)(s_maskT + Wq * kStreamClauses);
  auto vt_entry = [&](int e) -> short {  // entry e = (j * 16 + v) * K + k, from s_wt
    const int k = e % K, jv = e / K, j = jv >> 4, v = jv & 15;
    int sum = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b)
      if ((v >> b) & 1) sum += s_wt[k * kStreamClauses + 4 * j + b];
    return (short)sum;
  };
  // word group w4 of clause idx's include mask (zero past W and past the own clauses)
  auto mask_quad = [&](int idx, int64_t w4) -> uint4 {
    const uint32_t* mt = s_planes + idx * cw + (int64_t)(g.np - 1) * g.W;
    const int64_t w = 4 * w4;
    const bool ok = idx < n_own;
    return uint4{ok && w < g.W ? mt[w] : 0u, ok && w + 1 < g.W ? mt[w + 1] : 0u, ok && w + 2 < g.W ? mt[w + 2] : 0u,
                 ok && w + 3 < g.W ? mt[w + 3] : 0u};
  };
  const bool exact_count = g.maxinc < g.L;
  const int ks = (K + 15) & ~15;
  unsigned long long my_updates = 0ull, my_evals = 0ull, my_stops = 0ull;
  uint64_t wait_ticks = 0;
  const uint64_t t_kernel = __builtin_amdgcn_s_memrealtime();

  if (threadIdx.x == 0) s_wmax = 0;
  __syncthreads();
  for (int64_t j = threadIdx.x; j < n_own * cw; j += blockDim.x) s_planes[j] = a.planes[c_begin * cw + j];
  for (int64_t j = threadIdx.x; j < n_own * K; j += blockDim.x) {
    const float w = a.weights[c_begin * K + j];
    s_w[j] = w;
    s_wt[(j % K) * kStreamClauses + j / K] = (int)w;
    atomicMax(&s_wmax, (int)w < 0 ? -(int)w : (int)w);
  }
  for (int j = threadIdx.x; j < K * kStreamClauses; j += blockDim.x)
    if (j % kStreamClauses >= n_own) s_wt[j] = 0;  // clauses past the own ones (vote tables)
  if (threadIdx.x < 64) s_vdirty[threadIdx.x] = 0;
  for (int j = threadIdx.x; j < kStreamClauses; j += blockDim.x) {
    s_drop[j] = j < n_own ? a.drop[c_begin + j] == 1u : 1;
    s_pw[j] = j < n_own ? a.patch_w[c_begin + j] : 0;
    s_zero[j] = 0;
  }
  __syncthreads();
  for (int64_t j = threadIdx.x; j < Wq * kStreamClauses; j += blockDim.x)
    s_maskT[j] = mask_quad((int)(j % kStreamClauses), j / kStreamClauses);
  if (g.vote_table)
    for (int e = threadIdx.x; e < 256 * K; e += blockDim.x) s_vt[e] = vt_entry(e);
  // include counts (or emptiness when MAX_INCLUDED_LITERALS >= L), one clause per wave
  for (int idx = wave; idx < n_own; idx += nwv) {
    const uint32_t* m = s_planes + idx * cw + (int64_t)(g.np - 1) * g.W;
    int cnt = 0;
    for (int64_t w = lane; w < g.W; w += kWave) cnt += __popc(m[w]);
    cnt = wave_sum_i32(cnt);
    if (lane == 0) s_ninc[idx] = exact_count ? cnt : (cnt > 0);
  }

  // Profile (a.profile, wave 0's view, summed into counters[4..8]): streaming, draining the
  // evaluation waves after a stop, feedback decisions, literal updates and repairs, and
  // (within streaming) the wait for each phase's first row after a stop.
  const bool prof = a.profile && wave == 0;
  uint64_t prof_acc[5] = {0, 0, 0, 0, 0};
  uint64_t prof_last = t_kernel;
  int gen_start = 0;  // first sample of the stream (row row_base)
  int64_t row_base = 0;
  int next = 0;  // first sample of the current phase (after the last stop)
  int kgen = 0;  // stops in this stream: every row is complete at G * (kgen + 1) units
  // Stops a stream may take before a fresh one starts (the unit count of a row must stay
  // below 2^19); a.stream_gens lowers it (test hook).
  int kgen_cap = (1 << 19) / G - 2;
  if (a.stream_gens > 0 && a.stream_gens < kgen_cap) kgen_cap = a.stream_gens;
  // Lookahead at the start of a phase: 2 after a phase of one sample (a stop at every sample),
  // else eight times the previous phase's length, at most D: deep as soon as stops are a few
  // samples apart (the rows published past a stop are repaired, not discarded, so depth
  // costs little then).
  int depth0 = 2;
  for (int q = threadIdx.x; q < D; q += blockDim.x) s_pub[q] = -1;
  while (next < a.N) {
    if (threadIdx.x == 0) {
      ctl.claim = next;
      ctl.consume = next;
      ctl.stop = -1;
      ctl.abort = 0;
    }
    __syncthreads();
    if (wave == 0) {
      // ---- consumer: rows in order, up to 64 / K at a time (lane = (row q, class k))
      const int nq = K <= 32 ? kWave / K : 1;
      const int q = lane / K, k = lane - (lane / K) * K;
      const long long bias_k = (long long)a.bias[k];
      int j = next;
      int stop = -1;
      int pw_add = 0;
      bool first_row = next > 0;  // profile: the wait for a phase's first row after a stop
      const uint64_t t_phase = __builtin_amdgcn_s_memrealtime();
      // a count no word reaches under the test hook: every wait then expires
      const unsigned long long units = (unsigned long long)G * (unsigned long long)(kgen + 1);
      const unsigned long long complete = units + (a.test_timeout ? 1ull : 0ull);
      while (j < a.N) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        bool here = q < nq && j + q < a.N;  // this lane's (row, class) exists
        unsigned long long v = 0;
        int ncomp = 0;
        for (unsigned polls = 1;; ++polls) {
          bool ok = true;
          if (here) {
            v = __hip_atomic_load(&a.slots[(row_base + (j + q - gen_start)) * ks + k], __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
            ok = ((v + (1ull << 43)) >> 44) == complete;
          }
          // complete rows from j on: the first row with an incomplete word ends them
          const unsigned long long bad = __ballot(here && !ok);
          const int first_bad = bad ? (__ffsll((long long)bad) - 1) / K : nq;
          const int avail = a.N - j < nq ? a.N - j : nq;
          ncomp = first_bad < avail ? first_bad : avail;
          if (ncomp > 0) break;
          if ((polls & 15u) == 0u && lds_load(&ctl.abort)) break;  // an evaluation wave gave up
          if ((polls & 15u) == 0u && __builtin_amdgcn_s_memrealtime() - t0 > (a.test_timeout ? 0 : kWaitTicks)) {
            if (lane == 0) {
              lds_store(&ctl.abort, 1);
              if (atomicCAS(a.err, 0, 1) == 0) {
                a.err[1] = j;
                a.err[2] = wg;
                a.err[3] = (int)((v + (1ull << 43)) >> 44);
              }
            }
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
        wait_ticks += __builtin_amdgcn_s_memrealtime() - t0;
        if (prof && first_row) {
          prof_acc[4] += __builtin_amdgcn_s_memrealtime() - t_phase;
          first_row = false;
        }
        if (ncomp == 0) break;  // aborted
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");  // the rows' LDS rings are written
        // feedback possible in row q?  prob > 0 for some class (class_fb, kernel.cu:508-529)
        const bool live = here && q < ncomp;
        const long long S = (long long)(v - (units << 44)) + bias_k;
        // the selections of the complete rows, lane r holding row j + r's, read together with
        // the targets (instead of one LDS round trip per row below)
        const unsigned long long ringq = s_ring[(j + (lane < nq ? lane : 0)) & (D - 1)];
        const int yq = s_yring[((j + (q < nq ? q : 0)) & (D - 1)) * K + k];
        bool fb = false;
        if (live) {
          const int y = yq;
          fb = class_may_update(g, S, y);  // class_fb(g, S, y).prob > 0
        }
        const unsigned long long fbm = __ballot(fb);
        const int qf = fbm ? (__ffsll((long long)fbm) - 1) / K : ncomp;  // first row with feedback
        // patch weights of the rows before it (select_active, kernel.cu:305), counted in a
        // register of the clause's lane and added to LDS when the phase ends
        for (int r = 0; r < qf; ++r) {
          const unsigned long long rr =
              ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(ringq >> 32), r) << 32) |
              (unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)ringq, r);
          pw_add += (int)((rr >> lane) & 1ull);
        }
        if (qf < ncomp) {
          if (q == qf) s_S[k] = S;
          stop = j + qf;
          break;
        }
        j += ncomp;
        if (lane == 0) lds_store(&ctl.consume, j);
      }
      if (lane < n_own) s_pw[lane] += pw_add;
      if (lane == 0) lds_store(&ctl.stop, stop >= 0 ? stop : a.N);
    } else {
      // ---- evaluation: claim samples in order, evaluate with the current state, publish
      const bool own = lane < n_own;
      // per phase (drop flags never change, include counts only at stops): the lanes whose
      // clause takes part, and those whose clause is empty (an empty clause fires in training)
      const bool live = own && s_drop[lane] == 0;
      const bool empty = s_ninc[lane] == 0;
      // the last sample published before this phase (rows past the stop, repaired): later
      // samples need no look at the ring's publish marks
      int pub_hi = -1;
      {
        const int ps = lane < D ? s_pub[lane] : -1;
        pub_hi = wave_max_i32(ps);
      }
      for (;;) {
        // the stop flag, a claim and the consumer's position in one LDS round trip
        const int stop_now = __hip_atomic_load(&ctl.stop, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        int s = 0;
        if (lane == 0) s = atomicAdd(&ctl.claim, 1);
        int cons = lds_load(&ctl.consume);
        if (stop_now >= 0) break;
        s = lane_value(s, 0);
        if (s >= a.N) break;
        // the sample's targets and (one word per lane) its words, in flight while the
        // window is checked (every lane reads a valid entry)
        const int32_t yv = a.Y[(int64_t)s * K + (lane < K ? lane : 0)];
        const uint32_t xv0 = g.W <= kWave ? a.X[(int64_t)s * g.W + (lane < g.W ? lane : 0)] : 0u;
        // at most min(D, depth0 + consumed samples of this phase) ahead of the consumer
        bool skip = false;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        for (unsigned spins = 1;; ++spins) {
          if (spins > 1) cons = lds_load(&ctl.consume);
          const int ahead = depth0 + (cons - next) < D ? depth0 + (cons - next) : D;
          if (s < cons + ahead) break;
          if (lds_load(&ctl.stop) >= 0) {  // stopped before s: s is past the stop sample
            skip = true;
            break;
          }
          if ((spins & 15u) == 0u && __builtin_amdgcn_s_memrealtime() - t0 > 2 * kWaitTicks) {
            if (lane == 0) {
              lds_store(&ctl.abort, 1);
              if (atomicCAS(a.err, 0, 1) == 0) {
                a.err[1] = s;
                a.err[2] = wg;
                a.err[3] = -1;  // an evaluation wave, not the class-sum wait
              }
            }
            skip = true;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
        if (skip) break;
        if (s <= pub_hi && s_pub[s & (D - 1)] == s) continue;  // published before the last stop, and repaired
        // the sample's complemented words (broadcast reads below; kept in the sample's ring
        // slot for the repairs after a stop) and its targets
        uint32_t* nx = s_nx + (int64_t)(s & (D - 1)) * Wp;
        if (g.W <= kWave) {
          if (lane < g.W) nx[lane] = ~xv0;
        } else {
          for (int64_t w = lane; w < g.W; w += kWave) nx[w] = ~a.X[(int64_t)s * g.W + w];
        }
        if (lane < K) s_yring[(s & (D - 1)) * K + lane] = yv;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        // fast_eval (kernel.cu:255-282): an empty clause fires in training
        uint32_t bad = 0u;
        const uint4* nx4 = (const uint4*)nx;
#pragma unroll 2
        for (int64_t w4 = 0; w4 < Wq; ++w4) {
          const uint4 mv = s_maskT[w4 * kStreamClauses + lane], xv = nx4[w4];
          bad |= (mv.x & xv.x) | (mv.y & xv.y) | (mv.z & xv.z) | (mv.w & xv.w);
        }
        const bool fire = live && (empty || bad == 0u);
        // a stop set meanwhile lies before s: its row will not be read
        if (lds_load(&ctl.stop) >= 0) break;
        // select_active (kernel.cu:285-316) with one patch: selected when the rank-1 draw is
        // below 1.0f / 1
        bool sel = false;
        if (__any(fire)) {
          const U4 z = counted_site(a, a.step0 + (uint64_t)s, (uint32_t)(c_begin + (own ? lane : 0)), TAG_SEL, 0u);
          sel = fire && uniform_from_word(z.x) < 1.0f;
        }
        const unsigned long long smask = __ballot(sel);
        int mine = 0;
        if (smask) {
          // Two classes per 32-bit sum while |weight| < 512: each selected lane adds w + 512
          // (1 .. 1023) into a 16-bit field, so 64 lanes stay below 2^16 and no field carries
          // into the next; the bias of the selected lanes comes off again.
          int kk = 0;
          const bool small_w = lds_load(&s_wmax) < 512;
          if (g.vote_table && small_w) {
            // lane k < K: its class's vote from the 16 nibbles of the selection mask.  Every
            // lane reads (lanes >= K an entry of class 0), through a 32-bit LDS address, so
            // that the 16 reads go out together with no change of the exec mask.
            typedef const __attribute__((address_space(3))) short* LdsShorts;
            const LdsShorts vt_lane = (LdsShorts)(s_vt + (lane < K ? lane : 0));
            int e[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) e[j] = (int)vt_lane[(j * 16 + (int)((smask >> (4 * j)) & 15ull)) * K];
            int acc = 0;
#pragma unroll
            for (int j = 0; j < 16; ++j) acc += e[j];
            mine = lane < K ? acc : 0;
            kk = K;
          } else if (small_w) {
            const int nbias = 512 * __popcll(smask);
            for (; kk + 1 < K; kk += 2) {
              const int v0 = s_wt[kk * kStreamClauses + lane] + 512, v1 = s_wt[(kk + 1) * kStreamClauses + lane] + 512;
              const int p = wave_sum_i32(sel ? (v0 | (v1 << 16)) : 0);
              if (lane == kk) mine = (p & 0xFFFF) - nbias;
              if (lane == kk + 1) mine = (int)((unsigned)p >> 16) - nbias;
            }
          }
          for (; kk < K; ++kk) {
            const int p = wave_sum_i32(sel ? s_wt[kk * kStreamClauses + lane] : 0);
            if (lane == kk) mine = p;
          }
        }
        if (lane == 0) {
          s_ring[s & (D - 1)] = smask;
          s_pub[s & (D - 1)] = s;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // ring and targets before the publish
        if (lane < K)
          __hip_atomic_fetch_add(&a.slots[(row_base + (s - gen_start)) * ks + lane],
                                 ((unsigned long long)(kgen + 1) << 44) + (unsigned long long)(long long)mine,
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ++my_evals;
      }
    }
    if (prof) {
      const uint64_t now = __builtin_amdgcn_s_memrealtime();
      prof_acc[0] += now - prof_last;
      prof_last = now;
    }
    __syncthreads();
    if (prof) {
      const uint64_t now = __builtin_amdgcn_s_memrealtime();
      prof_acc[1] += now - prof_last;
      prof_last = now;
    }
    const int stop = ctl.stop;
    if (ctl.abort) break;
    if (stop >= a.N) break;

    // ---- feedback of sample `stop` (clause_update, kernel.cu:531-613), whole workgroup
    const uint64_t t = a.step0 + (uint64_t)stop;
    const unsigned long long selm = s_ring[stop & (D - 1)];
    if (threadIdx.x < kStreamClauses) s_selj[threadIdx.x] = ((selm >> threadIdx.x) & 1ull) ? 0 : -1;
    if (threadIdx.x == 0) s_ntask = 0;
    if (threadIdx.x < 64) s_vdirty[threadIdx.x] = 0;
    for (int j = threadIdx.x; j < K * kStreamClauses; j += blockDim.x) s_wt_old[j] = s_wt[j];
    ++my_stops;
    __syncthreads();
    {
      const int kn = K, cpp = kWave / kn;
      const int jc = lane / kn, kk = lane - jc * kn;
      const unsigned long long seg = kn == kWave ? ~0ull : ((1ull << kn) - 1ull);
      const ClassPrep cp = class_prep(g, s_yring[(stop & (D - 1)) * K + (kk < K ? kk : 0)]);
      const ClassTest ct = class_test(g, s_S[kk < K ? kk : 0], cp);
      for (int base = wave * cpp; base < n_own; base += nwv * cpp) {
        const int idx = base + jc;
        const bool valid = jc < cpp && idx < n_own;
        const int ix = valid ? idx : base;  // idle lanes read a valid clause and discard it
        const int64_t c = c_begin + ix;
        const float w0 = s_w[ix * K + kk];
        const U4 z = counted_site(a, t, (uint32_t)c, TAG_CK, (uint32_t)kk);
        const PairOps po = decide_pair<false>(g, nullptr, c, kk, valid && s_drop[ix] == 0, s_selj[ix], s_ninc[ix],
                                              ct.tgt, ct.num, ct.den, w0, uniform_from_word(z.x),
                                              uniform_from_word(z.y));
        if (valid && (po.t1a || po.t2)) {
          s_w[ix * K + kk] = po.w_new;
          s_wt[kk * kStreamClauses + ix] = (int)po.w_new;
          atomicMax(&s_wmax, (int)po.w_new < 0 ? -(int)po.w_new : (int)po.w_new);
          if (g.vote_table) atomicOr(&s_vdirty[kk], 1 << (ix >> 2));
        }
        const unsigned long long b1a = __ballot(po.t1a), b1b = __ballot(po.t1b), bt2 = __ballot(po.t2);
        if ((b1a | b1b | bt2) == 0ull) continue;
        const int sh = jc * kn;
        const unsigned long long m1a = valid ? (b1a >> sh) & seg : 0ull;
        const unsigned long long m1b = valid ? (b1b >> sh) & seg : 0ull;
        const unsigned long long m2 = valid ? (bt2 >> sh) & seg : 0ull;
        const bool leader = (m1a | m1b | m2) != 0ull && kk == 0;
        my_updates += (unsigned long long)__popcll(__ballot(leader));
        if (leader) {
          const int tk = atomicAdd(&s_ntask, 1);
          s_task_idx[tk] = ix;
          s_task_m[tk * 3 + 0] = m1a;
          s_task_m[tk * 3 + 1] = m1b;
          s_task_m[tk * 3 + 2] = m2;
        }
      }
    }
    __syncthreads();
    if (prof) {
      const uint64_t now = __builtin_amdgcn_s_memrealtime();
      prof_acc[2] += now - prof_last;
      prof_last = now;
    }
    if (g.vote_table) {
      // the vote-table entries of the changed weights' nibble groups (read after later
      // barriers): a wave per class, lanes 0..15 the 16 entries of each changed group
      for (int k = wave; k < K; k += nwv)
        for (int dm = s_vdirty[k]; dm; dm &= dm - 1) {
          const int j = __ffs(dm) - 1;
          if (lane < 16) s_vt[(j * 16 + lane) * K + k] = vt_entry((j * 16 + lane) * K + k);
        }
    }
    const int ntask = s_ntask;
    const uint32_t* xe = a.X + (int64_t)stop * g.W;  // the sample's words, for the literal updates
    if (g.W <= 32) {
      const int per = tasks_per_wave(g, ntask, nwv);
      for (int tk0 = wave * per; tk0 < ntask; tk0 += nwv * per)
        apply_tasks<false>(a, g, nullptr, c_begin, t, tk0, per, ntask, s_task_idx, s_task_m, s_zero, s_selj,
                           s_planes, xe, nullptr, 0);
    } else {
      for (int tk = wave; tk < ntask; tk += nwv) {
        const int idx = s_task_idx[tk];
        const FbOps ops{s_task_m[tk * 3 + 0], s_task_m[tk * 3 + 1], s_task_m[tk * 3 + 2]};
        apply_ops<false>(a, g, nullptr, c_begin + idx, t, s_selj[idx], ops, s_planes + idx * cw, xe, nullptr);
      }
    }
    __syncthreads();
    for (int tk = wave; tk < ntask; tk += nwv) {  // include counts of the updated clauses
      const int idx = s_task_idx[tk];
      const uint32_t* mt = s_planes + idx * cw + (int64_t)(g.np - 1) * g.W;
      int cnt = 0;
      for (int64_t w = lane; w < g.W; w += kWave) cnt += __popc(mt[w]);
      cnt = wave_sum_i32(cnt);
      if (lane == 0) s_ninc[idx] = exact_count ? cnt : (cnt > 0);
      for (int64_t w4 = lane; w4 < Wq; w4 += kWave) s_maskT[w4 * kStreamClauses + idx] = mask_quad(idx, w4);
    }
    if (wave == 0 && lane < n_own) s_pw[lane] += (int)((selm >> lane) & 1ull);  // the stop sample's
    depth0 = stop == next ? 2 : (8 * (stop + 1 - next) < D ? 8 * (stop + 1 - next) : D);
    next = stop + 1;
    if (kgen < kgen_cap) {
      // The stream goes on past the stop.  Every row this workgroup published past it was
      // evaluated with the state before the feedback; only the updated clauses' votes
      // differ now, so the row gets their difference as this workgroup's next unit, and a
      // row published from here on carries kgen + 1 units at once.
      ++kgen;
      __syncthreads();  // include counts of the updated clauses
      // the updated clauses, lane tk holding task tk's (read once for all the rows)
      const int tidx = lane < ntask ? s_task_idx[lane] : 0;
      // in row order from the next row, which the consumer waits for first
      for (int u = wave; u < D; u += nwv) {
        const int q = (next + u) & (D - 1);
        const int r = s_pub[q];
        if (r < next) continue;  // consumed (or none)
        // bit tk: updated clause s_task_idx[tk] has an included literal that is 0 in sample r
        // (the sample's complemented words are kept in its ring slot)
        unsigned long long badm = 0ull;
        const uint32_t* nxr = s_nx + (int64_t)q * Wp;
        for (int64_t w0 = 0; w0 < g.W; w0 += kWave) {
          const int64_t w = w0 + lane;
          const uint32_t nxw = w < g.W ? nxr[w] : 0u;
          for (int tk = 0; tk < ntask; ++tk) {
            const int tix = __builtin_amdgcn_readlane(tidx, tk);
            const uint32_t mw = w < g.W ? s_planes[tix * cw + (int64_t)(g.np - 1) * g.W + w] : 0u;
            if (__any((mw & nxw) != 0u)) badm |= 1ull << tk;
          }
        }
        // lane tk: the updated clause's selection for sample r (fast_eval and the rank-1
        // draw of select_active, as in the evaluation above)
        bool nsel = false;
        if (lane < ntask) {
          const int idx = tidx;
          if (s_ninc[idx] == 0 || ((badm >> lane) & 1ull) == 0ull)
            nsel = uniform_from_word(
                       counted_site(a, a.step0 + (uint64_t)r, (uint32_t)(c_begin + idx), TAG_SEL, 0u).x) < 1.0f;
        }
        const unsigned long long nb = __ballot(nsel);
        unsigned long long chg = 0ull, nsm = 0ull;
        for (int tk = 0; tk < ntask; ++tk) {
          const int idx = __builtin_amdgcn_readlane(tidx, tk);
          chg |= 1ull << idx;
          nsm |= ((nb >> tk) & 1ull) << idx;
        }
        const unsigned long long om = s_ring[q];
        if (lane < K) {
          long long delta = 0;
          for (int tk = 0; tk < ntask; ++tk) {
            const int idx = __builtin_amdgcn_readlane(tidx, tk);
            if ((nsm >> idx) & 1ull) delta += s_wt[lane * kStreamClauses + idx];
            if ((om >> idx) & 1ull) delta -= s_wt_old[lane * kStreamClauses + idx];
          }
          __hip_atomic_fetch_add(&a.slots[(row_base + (r - gen_start)) * ks + lane],
                                 (1ull << 44) + (unsigned long long)delta, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
        }
        if (lane == 0) s_ring[q] = (om & ~chg) | nsm;
      }
    } else {
      // a fresh stream on fresh rows: the rows published past the stop are never read
      row_base += (int64_t)(next - gen_start) + D;
      gen_start = next;
      kgen = 0;
      for (int q = threadIdx.x; q < D; q += blockDim.x) s_pub[q] = -1;
    }
    __syncthreads();
    if (prof) {
      const uint64_t now = __builtin_amdgcn_s_memrealtime();
      prof_acc[3] += now - prof_last;
      prof_last = now;
    }
  }
  __syncthreads();
  for (int64_t j = threadIdx.x; j < n_own * cw; j += blockDim.x) a.planes[c_begin * cw + j] = s_planes[j];
  for (int64_t j = threadIdx.x; j < n_own * K; j += blockDim.x) a.weights[c_begin * K + j] = s_w[j];
  for (int j = threadIdx.x; j < n_own; j += blockDim.x) a.patch_w[c_begin + j] = s_pw[j];
  if (lane == 0 && my_updates) atomicAdd(&a.counters[0], my_updates);
  if (lane == 0 && my_evals) atomicAdd(&a.counters[13], my_evals);
  if (threadIdx.x == 0) {
    atomicAdd(&a.counters[1], (unsigned long long)wait_ticks);
    atomicAdd(&a.counters[2], (unsigned long long)(__builtin_amdgcn_s_memrealtime() - t_kernel));
    if (wg == 0) atomicAdd(&a.counters[12], my_stops);
    if (prof)
      for (int j = 0; j < 5; ++j) atomicAdd(&a.counters[4 + j], (unsigned long long)prof_acc[j]);
  }
}

}  // namespace ytm
