// ytm_types.h -- structures shared by host code, the built-in kernels and the kernels
// specialised per model at run time (hipRTC compiles this header too).
#pragma once
#if !defined(__HIPCC_RTC__)
#include <hip/hip_runtime.h>
#include <stdint.h>
#else
// hipRTC's built-in preamble declares the fixed-width integer types in __hip_internal.
using __hip_internal::uint16_t;
using __hip_internal::int32_t;
using __hip_internal::int64_t;
using __hip_internal::uint32_t;
using __hip_internal::uint64_t;
#endif

namespace ytm {

constexpr int kTrainThreads = 512;  // workgroup size of the built-in training kernels
constexpr int kMaxPlanesHost = 32;  // must equal kMaxPlanes of ytm_device.h

// Resolved model geometry and hyperparameters.  Listed once (X-macro) so that host code
// can print a constexpr initializer in declaration order for a specialised compile.
#define YTM_GEOM_FIELDS(X)                                                                           \
  X(int64_t, C)            /* clauses */                                                             \
  X(int64_t, K)            /* classes */                                                             \
  X(int64_t, L)            /* literals */                                                            \
  X(int64_t, W)            /* literal words */                                                       \
  X(int64_t, P)            /* patches */                                                             \
  X(int64_t, Lh)           /* positive literals */                                                   \
  X(int64_t, F)            /* input features per sample */                                           \
  X(int, np)               /* TA bit-planes */                                                       \
  X(uint32_t, off)         /* stored plane value s' = s + off */                                     \
  X(uint32_t, max_state_p) /* number_of_ta_states + off */                                           \
  X(uint32_t, last_filter) /* valid-literal mask of word W-1 (kernel.cu:36-40) */                    \
  X(int, half_state)       /* number_of_ta_states / 2 */                                             \
  X(int, max_state)        /* number_of_ta_states */                                                 \
  X(int, per_bank)         /* clauses per bank (C when coalesced) */                                 \
  X(int, dim0)                                                                                       \
  X(int, dim1)                                                                                       \
  X(int, dim2)                                                                                       \
  X(int, pd0)                                                                                        \
  X(int, pd1)                                                                                        \
  X(int, append_negated)                                                                             \
  X(int, encode_loc)                                                                                 \
  X(int, coalesced)                                                                                  \
  X(int, negative_polarity)                                                                          \
  X(int, init_neg_weights)                                                                           \
  X(int, maxinc)           /* MAX_INCLUDED_LITERALS */                                               \
  X(double, thresh)        /* T */                                                                   \
  X(double, s_inv)         /* typed S_INV widened to double */                                       \
  X(double, q_prob)        /* typed Q_PROB widened to double */                                      \
  X(uint32_t, s_thr)       /* floor(s_inv * 2^24) clamped to [0, 2^24] */                             \
  X(int, threads)          /* training launch: threads per workgroup (0 outside training) */        \
  X(int, grid)             /* training launch: persistent workgroups (0 outside training) */         \
  X(int, group_size)       /* training launch: workgroups per class-sum group */                     \
  X(int, groups)           /* training launch: class-sum groups, ceil(grid / group_size) */          \
  X(int, list_cap)         /* training launch: literal-list capacity per clause (0: none) */       \
  X(int, mask_lds)         /* training launch, global one-patch kernel: include masks and sample in LDS */ \
  X(int, vote_table)       /* training launch, streaming kernel: class votes from nibble tables in LDS */

struct Geom {
#define YTM_GEOM_DECL(type, name) type name;
  YTM_GEOM_FIELDS(YTM_GEOM_DECL)
#undef YTM_GEOM_DECL
};

// Clauses of a model with several patches are evaluated on a literal-major copy of each
// sample (one bitset over the patches per literal), when a bitset fits one 32-bit word per
// wave lane.
__host__ __device__ constexpr bool literal_major(const Geom& g) { return g.P > 1 && (g.P + 31) / 32 <= 64; }
// The training kernel keeps the current literal-major sample in LDS when it fits 120 KiB.
__host__ __device__ constexpr bool literal_major_lds(const Geom& g) {
  return literal_major(g) && g.L * ((g.P + 31) / 32) * 4 <= 120 * 1024;
}

// Streaming training kernel (train_stream_body): in-flight samples per workgroup (a power
// of two), most clauses per workgroup (one lane each), and the class-sum rows a launch of n
// samples may use at most (every sample a stop).
constexpr int kStreamDepth = 32;
constexpr int kStreamClauses = 64;
__host__ __device__ constexpr int64_t stream_rows(int64_t n) { return n * (kStreamDepth + 1); }

// Literal order of the literal lists: buckets of literal density, and the samples whose
// densities set them (build_literal_list, literal_order_kernel).
constexpr int kOrderBuckets = 8;
constexpr int kOrderSamples = 32;

struct TrainArgs {
  uint32_t* planes;          // [C][np][W]
  float* weights;            // [C][K]
  int32_t* patch_w;          // [C][P]
  const float* bias;         // [K]
  const uint32_t* X;         // [N][P][W]  (first sample of this launch)
  const uint32_t* XT;        // [N][L][ceil(P/32)] literal-major samples (literal_major(g)), or null
  const int32_t* Y;          // [N][K]
  const uint32_t* drop;      // [C]
  const float* inject;       // [N][inject_block] or nullptr
  const float* inv_rank;     // [P + 1], inv_rank[r] = 1.0f / r
  unsigned long long* slots; // [N][slot_stride], zero on entry
  unsigned long long* counters;  // [0] updated clauses, [1] wait ticks, [2] kernel ticks, [4..11] phases,
                                 // [12] samples where some class may update (workgroup 0 counts; the
                                 // streaming kernel's stops), [13] evaluations (streaming kernel); with
                                 // profile 4, lane draws: [3] Q-skip/update, [14] reservoir, [15] literal
  int* err;                  // {1, sample, workgroup, count} when a bounded wait expires
  int64_t inject_block;
  uint64_t step0;
  uint64_t seed;
  int N;
  int64_t slot_stride;       // slot words per sample: groups == 1 ? ks : (2 groups + 1) ks, ks = K rounded to 16
  int cpw;                   // max clauses owned by one workgroup
  int rng_slots;             // literal-draw slots precomputed per sample (resident kernel)
  int profile;               // accumulate per-phase times into counters[4..11]; 4: count draws instead
  int test_timeout;          // test hook: class-sum waits never see their sums and expire at once
  int xt_halves;             // XT's literals Lh..L-1 are the complements of 0..Lh-1 (checked per dataset)
  int stream_gens;           // streaming kernel: stops per stream before fresh rows (0: as many as fit; test hook)
  const uint32_t* lit_order; // [kOrderBuckets][W] order of the literal lists (build_literal_list), or null
  Geom g;
};

}  // namespace ytm
