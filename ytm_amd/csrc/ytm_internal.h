// ytm_internal.h -- host-side declarations of libytm's kernel launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "ytm.h"
#include "ytm_types.h"

namespace ytm {

hipError_t launch_encode(const uint32_t* X, int64_t N, uint32_t* out, const Geom& g, hipStream_t s);
// Literal-major copy of encoded samples (several patches): XT [N][L][ceil(P/32)].
hipError_t launch_transpose(const uint32_t* X, int64_t N, uint32_t* XT, const Geom& g, hipStream_t s);
// Clears *ok unless every literal Lh + f of XT is the complement of literal f (ok set before).
hipError_t launch_xt_halves_check(const uint32_t* XT, int64_t N, const Geom& g, int* ok, hipStream_t s);
hipError_t launch_ta_to_planes(const uint32_t* ta, uint32_t* planes, const Geom& g, hipStream_t s);
hipError_t launch_planes_to_ta(const uint32_t* planes, uint32_t* ta, const Geom& g, hipStream_t s);
hipError_t launch_init_state(uint32_t* planes, float* w, const Geom& g, uint64_t seed, hipStream_t s);
hipError_t launch_ninc(const uint32_t* planes, int32_t* ninc, const Geom& g, hipStream_t s);
hipError_t launch_fill_u64(unsigned long long* p, int64_t n, hipStream_t s);
// Class-sum accumulation into acc int64 [N][K] (zeroed by the caller).
hipError_t launch_score(const uint32_t* planes, const int32_t* ninc, const float* w, const uint32_t* X,
                        int64_t N, const Geom& g, long long* acc, hipStream_t s);
// One-patch models: the tiled scorer writes per-chunk sums parts int64 [chunks][N][K]
// (chunks = score_tile_chunks(g), 0 when the tiled scorer does not apply), which
// launch_score_parts_finish adds up with the bias.  w_bound: an upper bound of |weight|,
// which lets the kernel sum in int32 when that is exact.
int64_t score_tile_chunks(const Geom& g);
hipError_t launch_score_tile(const uint32_t* planes, const int32_t* ninc, const float* w, const uint32_t* X,
                             int64_t N, const Geom& g, long long* parts, double w_bound, hipStream_t s);
hipError_t launch_score_parts_finish(const long long* parts, int64_t nch, const float* bias, int64_t N, const Geom& g,
                                     float* out, hipStream_t s);
// Literal order of the literal lists, order [kOrderBuckets][W], from the densities of the
// first min(N, kOrderSamples) samples of XT (literal-major) when given, else of X.
hipError_t launch_literal_order(const uint32_t* X, const uint32_t* XT, int64_t N, const Geom& g, uint32_t* order,
                                hipStream_t s);
// Scoring of several-patch models on literal-major samples; scratch holds score_lists_bytes(g)
// (0: not available for this geometry).
size_t score_lists_bytes(const Geom& g);
hipError_t launch_score_lm(const uint32_t* planes, const float* w, const uint32_t* XT, int64_t N, const Geom& g,
                           void* scratch, long long* acc, hipStream_t s);
// One patch and clauses wider than 16 words: a tile of samples transposed in LDS, the
// clauses' literal lists AND-ed lane by lane; scratch holds score_wide_bytes(g); acc (zeroed
// first) receives each sample's exact sums.  lists_ready: scratch already holds the lists of
// these planes (a previous call on the unchanged model), which are then not rebuilt.
bool score_wide_fits(const Geom& g);
size_t score_wide_bytes(const Geom& g);  // 0 when score_wide_fits is false
hipError_t launch_score_wide(const uint32_t* planes, const float* w, const uint32_t* X, int64_t N, const Geom& g,
                             void* scratch, bool lists_ready, long long* acc, hipStream_t s);
hipError_t launch_score_finish(const long long* acc, const float* bias, int64_t N, const Geom& g,
                               float* out, hipStream_t s);
// Clause outputs; mode 0: any patch (N, C); 1: per patch (N, C, P); 2: per patch, bit-packed
// (N, C, ceil(P/32)).
hipError_t launch_transform(const uint32_t* planes, const int32_t* ninc, const uint32_t* X, int64_t N,
                            const Geom& g, int mode, uint32_t* out, hipStream_t s);
// One patch and clauses wider than 16 words (score_wide_fits), all modes alike: scratch holds
// score_wide_bytes(g), its literal lists built first unless lists_ready.
hipError_t launch_transform_wide(const uint32_t* planes, const uint32_t* X, int64_t N, const Geom& g, void* scratch,
                                 bool lists_ready, uint32_t* out, hipStream_t s);
// The same on literal-major samples; scratch holds score_lists_bytes(g), its literal lists
// built first unless lists_ready.
hipError_t launch_transform_lm(const uint32_t* planes, const uint32_t* XT, int64_t N, const Geom& g, int mode,
                               void* scratch, bool lists_ready, uint32_t* out, hipStream_t s);

// Binarizers (host preprocessing): element-wise thermometer / one-hot binning and the
// collapse of binned rows; see ytm_binarize / ytm_collapse_bins in ytm.h.
hipError_t launch_binarize(const void* X, int dtype, int64_t n, const void* t, bool int_thresholds, int nthr,
                           bool onehot, int edge, uint32_t* out, hipStream_t s);
// encode (launch_encode) of N samples of Fr raw values each (dtype YTM_DTYPE_*), each value
// binned into the levels of launch_binarize (width = nthr, or nthr - 1 + 2 edge for one-hot;
// g.F = Fr * width) where encode reads it; t: thresholds in device memory.
hipError_t launch_encode_binned(const void* X, int dtype, int64_t N, int64_t Fr, const void* t, bool int_thresholds,
                                int nthr, bool onehot, int edge, uint32_t* out, const Geom& g, hipStream_t s);
hipError_t launch_collapse_bins(const uint32_t* B, int64_t rows, int64_t width, bool onehot, int edge, int64_t* out,
                                hipStream_t s);

// LDS a resident training workgroup may use (gfx950 has 160 KiB per workgroup; the
// kernel's static LDS and some headroom are kept free).
constexpr size_t kResidentLdsLimit = 150 * 1024;

// Training kernel variants: clause state resident in LDS (one patch), or kept in global
// memory (one patch / several patches); kStream: one patch, clause state resident in LDS,
// class sums of the samples ahead exchanged speculatively (train_stream_body).
// kSteps: one ordinary launch per sample (launch_step): clause banks (coalesced=False), more
// than 64 classes, or a grid whose state does not fit.
enum class TrainKind { kResident, kGlobalVanilla, kGlobalConv, kStream, kSteps };
hipError_t train_occupancy(TrainKind kind, bool inject, size_t lds_bytes, int* blocks_per_cu);
hipError_t launch_train(const TrainArgs& a, int grid, size_t lds_bytes, TrainKind kind, bool inject, hipStream_t s);
// Launch i = 0 .. a.N of a per-sample fit over a.N samples: the feedback of sample i-1 and
// the evaluation of sample i; rows [3][K] int64 class sums (zero before launch 0); sel /
// ninc hold the clauses' selected patches and include counts from one launch to the next.
// Its dynamic LDS is step_lds_bytes(g) (partial sums, probabilities and targets per class).
hipError_t launch_step(const TrainArgs& a, int i, long long* rows, int* sel, int* ninc, bool inject, hipStream_t s);
size_t step_lds_bytes(const Geom& g);
size_t train_lds_bytes(TrainKind kind, int cpw, int rng_slots, const Geom& g);
// LDS of the streaming kernel for a workgroup of `threads` threads.
size_t stream_lds_bytes(const Geom& g, int threads);
// LDS of the streaming kernel's vote tables (Geom::vote_table).
size_t stream_vote_table_bytes(const Geom& g);
// Literal-draw slots the resident kernel precomputes per sample within an LDS budget.
int train_rng_slots(int cpw, const Geom& g);

// Training kernels compiled at run time (hipRTC) with the model's geometry and
// hyperparameters as compile-time constants.  Returns nullptr (and the reason) when the
// specialised compile is unavailable; the built-in kernels are used then.
// YTM_JIT=0 in the environment turns it off.
bool jit_enabled();
bool jit_compile(const Geom& g, TrainKind kind, bool inject, std::vector<char>* code, std::string* why);
hipFunction_t jit_train_kernel(const Geom& g, TrainKind kind, bool inject, std::string* why);
// Unloads every module jit_train_kernel loaded (each on its device, after a device
// synchronize) and empties the kernel cache; returns the number of modules that failed.
int jit_unload_all();
hipError_t jit_occupancy(hipFunction_t fn, int threads, size_t lds_bytes, int* blocks_per_cu);
hipError_t launch_train_jit(hipFunction_t fn, const TrainArgs& a, int grid, int threads, size_t lds_bytes,
                            hipStream_t s);

}  // namespace ytm
