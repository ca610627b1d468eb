// ytm_internal.h -- host/device shared structures and kernel launchers of libytm.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ytm {

constexpr int kMaxPlanesHost = 16;  // must equal kMaxPlanes of ytm_device.h

// Resolved model geometry and hyperparameters (passed by value to every kernel).
struct Geom {
  int64_t C, K, L, W, P, Lh, F;  // clauses, classes, literals, literal words, patches,
                                 // positive literals, input features per sample
  int np;                        // TA bit-planes
  uint32_t off;                  // stored plane value s' = s + off
  uint32_t max_state_p;          // number_of_ta_states + off
  uint32_t last_filter;          // valid-literal mask of word W-1 (kernel.cu:36-40)
  int half_state;                // number_of_ta_states / 2
  int max_state;                 // number_of_ta_states
  int per_bank;                  // clauses per bank (C when coalesced)
  int dim0, dim1, dim2, pd0, pd1;
  int append_negated, encode_loc, coalesced, negative_polarity, init_neg_weights;
  int maxinc;                    // MAX_INCLUDED_LITERALS
  double thresh;                 // T
  double s_inv, q_prob;          // typed S_INV, Q_PROB widened to double
  uint32_t s_thr;                // floor(s_inv * 2^24) clamped to [0, 2^24]
};

struct TrainArgs {
  uint32_t* planes;          // [C][np][W]
  float* weights;            // [C][K]
  int32_t* patch_w;          // [C][P]
  const float* bias;         // [K]
  const uint32_t* X;         // [N][P][W]  (first sample of this launch)
  const int32_t* Y;          // [N][K]
  const uint32_t* drop;      // [C]
  const float* inject;       // [N][inject_block] or nullptr
  const float* inv_rank;     // [P + 1], inv_rank[r] = 1.0f / r
  unsigned long long* slots; // [N][slot_stride], zero on entry
  unsigned long long* counters;  // [0] updated clauses, [1] wait ticks, [2] kernel ticks, [4..11] phases
  int* err;                  // set to 1 when a bounded wait expires
  int64_t inject_block;
  uint64_t step0;
  uint64_t seed;
  int N;
  int S;                     // workgroups per class-sum group
  int D;                     // class-sum groups (ceil(grid / S))
  int64_t slot_stride;       // slot words per sample: D == 1 ? ks : (2D + 1) * ks, ks = K rounded up to 16
  int cpw;                   // max clauses owned by one workgroup
  int rng_slots;             // literal-draw slots precomputed per sample (resident kernel)
  int profile;               // accumulate per-phase times into counters[4..11]
  Geom g;
};

constexpr int kTrainThreads = 512;

hipError_t launch_encode(const uint32_t* X, int64_t N, uint32_t* out, const Geom& g, hipStream_t s);
hipError_t launch_ta_to_planes(const uint32_t* ta, uint32_t* planes, const Geom& g, hipStream_t s);
hipError_t launch_planes_to_ta(const uint32_t* planes, uint32_t* ta, const Geom& g, hipStream_t s);
hipError_t launch_init_state(uint32_t* planes, float* w, const Geom& g, uint64_t seed, hipStream_t s);
hipError_t launch_ninc(const uint32_t* planes, int32_t* ninc, const Geom& g, hipStream_t s);
hipError_t launch_fill_u64(unsigned long long* p, int64_t n, hipStream_t s);
hipError_t launch_score(const uint32_t* planes, const int32_t* ninc, const float* w, const uint32_t* X,
                        int64_t N, const Geom& g, long long* acc, hipStream_t s);
hipError_t launch_score_finish(const long long* acc, const float* bias, int64_t N, const Geom& g,
                               float* out, hipStream_t s);
hipError_t launch_transform(const uint32_t* planes, const int32_t* ninc, const uint32_t* X, int64_t N,
                            const Geom& g, int patchwise, uint32_t* out, hipStream_t s);
// Training kernel variants: clause state resident in LDS (one patch), or kept in global
// memory (one patch / several patches).
enum class TrainKind { kResident, kGlobalVanilla, kGlobalConv };
hipError_t train_occupancy(TrainKind kind, bool inject, size_t lds_bytes, int* blocks_per_cu);
hipError_t launch_train(const TrainArgs& a, int grid, size_t lds_bytes, TrainKind kind, bool inject, hipStream_t s);
size_t train_lds_bytes(TrainKind kind, int cpw, int rng_slots, const Geom& g);
// Literal-draw slots the resident kernel precomputes per sample within an LDS budget.
int train_rng_slots(int cpw, const Geom& g);

}  // namespace ytm
