// ytm_api.hip -- the extern "C" boundary of libytm.so (declared in include/ytm.h).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "ytm.h"
#include "ytm_internal.h"

using ytm::Geom;

struct ytm_model {
  ytm_params params;
  Geom g;
  int device = 0;
  int cus = 0;
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  uint32_t* d_planes = nullptr;
  float* d_w = nullptr;
  int32_t* d_pw = nullptr;
  float* d_bias = nullptr;
  int32_t* d_ninc = nullptr;
  float* d_inv_rank = nullptr;
  unsigned long long* d_counters = nullptr;
  int* d_err = nullptr;
  unsigned long long* d_slots = nullptr;
  size_t slots_bytes = 0;
  // Scoring buffers kept between calls (grow-only): class-sum accumulators, float sums,
  // literal lists.  Calls are synchronous, so a call never reuses a buffer still in use.
  void* d_sacc = nullptr;
  void* d_sout = nullptr;
  void* d_slists = nullptr;
  size_t sacc_bytes = 0, sout_bytes = 0, slists_bytes = 0;
  void* h_sout = nullptr;  // pinned host staging of the class sums (hipHostMalloc)
  size_t h_sout_bytes = 0;
  // The TA states change with every fit and ytm_set_ta_state (planes_version counts them);
  // the one-patch literal lists in d_slists hold those of version slists_version, so that
  // scoring again an unchanged model does not rebuild them.
  uint64_t planes_version = 0;
  uint64_t slists_version = ~0ull;
  // Upper bound of |clause weight|: 1 after initialisation, the largest loaded magnitude
  // after ytm_set_weights, and + 1 per trained sample (a sample moves a weight by at most 1).
  double w_bound = 1.0;
  // A training launch whose bounded wait expired stops each workgroup at its own sample, so
  // the state is then a mix of samples: the model refuses fit, score and transform until a
  // whole state is loaded again (the bits of the setters called since: 1 TA states, 2
  // weights, 4 patch weights).
  // share of the last fit's samples where some class could update; a new model updates at
  // nearly every sample (its class sums start near 0, with update probability about 1/2)
  double feedback_frac = 1.0;
  bool invalid = false;
  int reloaded = 0;
  ytm_stats stats;
};

struct ytm_dataset {
  ytm_model* m;
  uint32_t* d_X;   // [N][P][W]
  int32_t* d_Y;    // [N][K]
  int64_t N;
  uint32_t* d_XT;  // [N][L][ceil(P/32)] literal-major copy (several patches), or null
  int xt_halves;   // d_XT's literals Lh..L-1 are the complements of 0..Lh-1 (TrainArgs::xt_halves)
  uint32_t* d_order;  // [kOrderBuckets][W] literal order of the training lists (with d_XT), or null
};

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

#define HIP_TRY(expr)                                                                            \
  do {                                                                                           \
    hipError_t e_ = (expr);                                                                      \
    if (e_ != hipSuccess)                                                                        \
      return fail(YTM_EHIP, std::string(#expr) + " failed: " + hipGetErrorString(e_));           \
  } while (0)

int ceil_log2(int64_t x) {
  int b = 0;
  while (((int64_t)1 << b) < x) ++b;
  return b;
}

// Classes of a model: the per-sample training kernel keeps three int64/double/int values
// per class in LDS (step_lds_bytes), 80 KiB at this bound.
constexpr int kMaxClasses = 4096;

// Geometry of src/cutm/base.py:94-121 plus the bit-plane encoding of the TA states.
int resolve_geometry(const ytm_params& p, Geom* out) {
  Geom g{};
  if (p.clauses < 1 || p.classes < 1) return fail(YTM_EINVAL, "clauses and classes must be >= 1");
  if (p.classes > kMaxClasses) return fail(YTM_EINVAL, "at most 4096 classes are supported");
  if (p.dim0 < 1 || p.dim1 < 1 || p.dim2 < 1) return fail(YTM_EINVAL, "dim entries must be >= 1");
  if (p.patch_dim0 < 1 || p.patch_dim1 < 1 || p.patch_dim0 > p.dim0 || p.patch_dim1 > p.dim1)
    return fail(YTM_EINVAL, "patch_dim must lie within dim");
  if (p.number_of_ta_states < 1) return fail(YTM_EINVAL, "number_of_ta_states must be >= 1");
  if (!p.coalesced && p.clauses % p.classes != 0)
    return fail(YTM_EINVAL, "non-coalesced clause banks need clauses divisible by classes");
  g.C = p.clauses;
  g.K = p.classes;
  g.dim0 = p.dim0; g.dim1 = p.dim1; g.dim2 = p.dim2;
  g.pd0 = p.patch_dim0; g.pd1 = p.patch_dim1;
  int64_t base = (int64_t)p.patch_dim0 * p.patch_dim1 * p.dim2;
  if (p.encode_loc) base += (p.dim0 - p.patch_dim0) + (p.dim1 - p.patch_dim1);
  g.Lh = base;
  g.L = p.append_negated ? 2 * base : base;
  g.W = (g.L - 1) / 32 + 1;
  g.P = (int64_t)(p.dim0 - p.patch_dim0 + 1) * (p.dim1 - p.patch_dim1 + 1);
  g.F = (int64_t)p.dim0 * p.dim1 * p.dim2;
  if (g.K * g.W * 6 >= ((int64_t)1 << 32)) return fail(YTM_EINVAL, "classes * literal words too large");
  if (!p.encode_loc && g.P > 1) {
    // kernel.cu:101-121 writes the thermometer bits even without ENCODE_LOC; the result is
    // only defined while they stay inside the positive literals.
    const int64_t top = std::max<int64_t>(p.dim1 - p.patch_dim1, (p.dim1 - p.patch_dim1) + (p.dim0 - p.patch_dim0));
    if (top > g.Lh) return fail(YTM_EINVAL, "encode_loc=False with these patches writes outside the literals");
  }
  g.max_state = p.number_of_ta_states;
  g.half_state = p.number_of_ta_states / 2;
  const int64_t maxs = std::max<int64_t>(g.max_state, (int64_t)g.half_state + g.K);
  const int top = std::max(1, std::max(ceil_log2((int64_t)g.half_state + 1), ceil_log2(maxs - g.half_state)));
  g.np = top + 1;
  if (g.np > ytm::kMaxPlanesHost) return fail(YTM_EINVAL, "number_of_ta_states too large for the bit-plane state");
  g.off = (uint32_t)(((int64_t)1 << top) - g.half_state - 1);
  g.max_state_p = (uint32_t)g.max_state + g.off;
  g.last_filter = (g.L % 32) ? ~(0xFFFFFFFFu << (g.L % 32)) : 0xFFFFFFFFu;
  g.per_bank = (int)(p.coalesced ? g.C : g.C / g.K);
  g.append_negated = p.append_negated;
  g.encode_loc = p.encode_loc;
  g.coalesced = p.coalesced;
  g.negative_polarity = p.negative_polarity;
  g.init_neg_weights = p.init_neg_weights;
  g.maxinc = p.max_included_literals;
  g.thresh = (double)p.thresh;
  g.s_inv = p.s_inv;
  g.q_prob = p.q_prob;
  // u <= s_inv with u = (q + 1) * 2^-24  <=>  q < floor(s_inv * 2^24).
  const double scaled = std::floor(p.s_inv * 16777216.0);
  g.s_thr = !(scaled > 0.0) ? 0u : (scaled >= 16777216.0 ? (1u << 24) : (uint32_t)scaled);
  *out = g;
  return YTM_OK;
}

// A grow-only device buffer: *p holds at least bytes after a successful call.
hipError_t ensure_buffer(void** p, size_t* have, size_t bytes) {
  if (*have >= bytes && *p) return hipSuccess;
  if (*p) {
    const hipError_t e = hipFree(*p);
    if (e != hipSuccess) return e;
  }
  *p = nullptr;
  *have = 0;
  const hipError_t e = hipMalloc(p, bytes > 0 ? bytes : 4);
  if (e == hipSuccess) *have = bytes;
  return e;
}

int ensure_slots(ytm_model* m, size_t bytes) {
  if (m->slots_bytes >= bytes) return YTM_OK;
  if (m->d_slots) HIP_TRY(hipFree(m->d_slots));
  m->d_slots = nullptr;
  m->slots_bytes = 0;
  HIP_TRY(hipMalloc(&m->d_slots, bytes));
  m->slots_bytes = bytes;
  return YTM_OK;
}

// YTM_TRAIN_PROFILE: 0 off; 1-3 phase timings (TrainArgs::profile); 4 draw counts.
int prof_level() {
  const char* env = std::getenv("YTM_TRAIN_PROFILE");
  return env ? std::max(0, std::atoi(env)) : 0;
}

int check_valid(const ytm_model* m) {
  if (m->invalid)
    return fail(YTM_EINVAL, "the model's state is a mix of samples after a training launch timed out; load a whole "
                            "state (TA states, weights and patch weights) or create the model again");
  return YTM_OK;
}

// A setter of part of the state succeeded: once all three parts are loaded again the model
// is usable.
void note_reload(ytm_model* m, int part) {
  if (!m->invalid) return;
  m->reloaded |= part;
  if (m->reloaded == 7) {
    m->invalid = false;
    m->reloaded = 0;
  }
}

// Bytes per element of a binarizer input type (YTM_DTYPE_*), 0 for none.
size_t dtype_size(int dtype) {
  switch (dtype) {
    case YTM_DTYPE_U8:
    case YTM_DTYPE_I8:
      return 1;
    case YTM_DTYPE_U16:
    case YTM_DTYPE_I16:
      return 2;
    case YTM_DTYPE_U32:
    case YTM_DTYPE_I32:
    case YTM_DTYPE_F32:
      return 4;
    case YTM_DTYPE_I64:
    case YTM_DTYPE_F64:
      return 8;
    default:
      return 0;
  }
}

int upload(void** dst, const void* src, size_t bytes, hipStream_t s) {
  HIP_TRY(hipMalloc(dst, bytes > 0 ? bytes : 4));
  if (bytes) HIP_TRY(hipMemcpyAsync(*dst, src, bytes, hipMemcpyHostToDevice, s));
  return YTM_OK;
}

// Picks the persistent grid (one workgroup per CU at most, at least ~12 clauses each, and
// two workgroups for models of more than one clause) and the class-sum grouping (groups of
// <= 16 workgroups).  ~12 clauses per workgroup balance the per-sample exchange, which
// gets slower with more workgroups, against the per-workgroup evaluation and draws (config
// 2 on MI355X: 167 workgroups train 2.7% faster than 250, and 96-192 are within 1%).
void train_shape(int64_t C, int cus, int* grid, int* S, int* D, int* cpw) {
  const char* env = std::getenv("YTM_TRAIN_WGS");
  int64_t G = std::min<int64_t>(cus, std::max<int64_t>(std::min<int64_t>(C, 2), (C + 11) / 12));
  if (env && std::atoi(env) > 0) G = std::min<int64_t>(std::atoi(env), C);
  *grid = (int)G;
  const char* envs = std::getenv("YTM_TRAIN_GROUP");
  int s = envs && std::atoi(envs) > 0 ? std::atoi(envs) : 16;
  s = (int)std::min<int64_t>(s, G);
  *S = s;
  *D = (int)((G + s - 1) / s);
  *cpw = (int)((C + G - 1) / G) + 1;
}

// The model geometry plus the launch shape of a training run on `cus` compute units
// (train_shape).
// Fewer, fuller workgroups do not pay: the exchange gets cheaper (about 1.0 us at 16
// workgroups, 1.2 us at 32, 2.1 us at 250 on MI355X), but the per-sample evaluation and
// draws then run on fewer CUs and take longer than that.  YTM_TRAIN_WGS / YTM_TRAIN_GROUP
// / YTM_TRAIN_THREADS override.
Geom train_geometry(const Geom& model, int cus, int* cpw) {
  int grid, S, D;
  train_shape(model.C, cus, &grid, &S, &D, cpw);
  Geom g = model;
  // Workgroup size of the specialised kernels (the built-in ones use kTrainThreads): a wave
  // per two clauses plus one, 8 to 16 waves.  Workgroups with many clauses are latency
  // bound and gain from more waves (MI355X, 1024 against 512 threads: config 3 +24%,
  // config 4 +42%, config 5 +32%); config 2's 12 clauses per workgroup run best on 512.
  const char* envt = std::getenv("YTM_TRAIN_THREADS");
  const int t = envt ? std::atoi(envt) : 0;
  const int waves = std::min(16, std::max(8, 1 + (*cpw + 1) / 2));
  g.threads = (t >= 128 && t <= 1024 && t % 64 == 0) ? t : 64 * waves;
  g.grid = grid;
  g.group_size = S;
  g.groups = D;
  return g;
}

bool train_lds_fits(const Geom& g, ytm::TrainKind kind, int cpw, int cap) {
  Geom gc = g;
  gc.list_cap = cap;
  const int r = kind == ytm::TrainKind::kResident ? ytm::train_rng_slots(cpw, gc) : 0;
  return ytm::train_lds_bytes(kind, cpw, r, gc) <= ytm::kResidentLdsLimit;
}

// Literal-list capacity of a training kernel kind (several patches): the resident kernel
// keeps 64 per clause, the global one the largest of 256..64 that fits; 0 when none fits.
int train_list_cap(const Geom& g, ytm::TrainKind kind, int cpw) {
  if (!ytm::literal_major(g) || g.L > 65535) return 0;
  if (kind == ytm::TrainKind::kResident) return train_lds_fits(g, kind, cpw, 64) ? 64 : 0;
  for (int cap : {256, 192, 128, 64})
    if (train_lds_fits(g, kind, cpw, cap)) return cap;
  return 0;
}

// Keeps the workgroup's clause state resident in LDS when it fits (with several patches,
// together with two literal-major samples), else the global kernel; sets g->list_cap.
// A one-patch model on the global kernel keeps its include masks (and the sample) in LDS
// when they fit (g->mask_lds).
void set_mask_lds(Geom* g, ytm::TrainKind kind, int cpw) {
  g->mask_lds = 0;
  if (kind == ytm::TrainKind::kGlobalVanilla) {
    g->mask_lds = 1;
    if (!train_lds_fits(*g, kind, cpw, 0)) g->mask_lds = 0;
  }
}

// The streaming kernel (train_stream_body) takes one-patch models with coalesced classes in
// the counter stream when every workgroup's clauses fit one lane each and their state fits
// LDS: grid ceil(C / 64) (YTM_TRAIN_WGS may raise it, up to C), 16 waves (YTM_TRAIN_THREADS
// overrides).  False when the model does not fit that shape on `cus` compute units.
bool stream_shape(const Geom& mg, int cus, Geom* out) {
  if (mg.P != 1 || !mg.coalesced) return false;
  int64_t G = (mg.C + ytm::kStreamClauses - 1) / ytm::kStreamClauses;
  if (const char* e = std::getenv("YTM_TRAIN_WGS"))
    if (std::atoi(e) > 0) G = std::max<int64_t>(G, std::min<int64_t>(std::atoi(e), mg.C));
  if (G > cus || G > mg.C) return false;
  Geom g = mg;
  const char* envt = std::getenv("YTM_TRAIN_THREADS");
  const int t = envt ? std::atoi(envt) : 0;
  g.threads = (t >= 128 && t <= 1024 && t % 64 == 0) ? t : 1024;
  g.grid = (int)G;
  g.group_size = (int)G;
  g.groups = 1;
  g.list_cap = 0;
  g.mask_lds = 0;
  g.vote_table = 0;
  const size_t base = ytm::stream_lds_bytes(g, std::max(g.threads, ytm::kTrainThreads));
  if (base > ytm::kResidentLdsLimit) return false;
  // class votes from nibble tables when they fit (YTM_STREAM_VOTE_TABLE=0 turns them off)
  const char* vt_env = std::getenv("YTM_STREAM_VOTE_TABLE");
  g.vote_table = g.K <= 16 && base + ytm::stream_vote_table_bytes(g) <= ytm::kResidentLdsLimit &&
                 !(vt_env && std::atoi(vt_env) == 0);
  *out = g;
  return true;
}

// Whether a fit of `count` samples takes the streaming kernel: the counter stream (not
// injected draws), clause state not forced to global memory, the shape above, and int32
// partial class sums exact (every weight the launch can reach, times 64, below 2^31).
// YTM_TRAIN_STREAM=0 turns it off.
bool stream_geometry(const ytm_model* m, bool inject, bool force_global, int64_t count, Geom* out) {
  const char* env = std::getenv("YTM_TRAIN_STREAM");
  if ((env && std::atoi(env) == 0) || inject || force_global) return false;
  if (64.0 * (m->w_bound + (double)count) >= 2147483648.0) return false;
  return stream_shape(m->g, m->cus, out);
}

ytm::TrainKind choose_train_kind(Geom* g, int cpw, bool force_global) {
  ytm::TrainKind kind = g->P == 1 ? ytm::TrainKind::kGlobalVanilla : ytm::TrainKind::kGlobalConv;
  if (!force_global && (g->P == 1 || ytm::literal_major(*g))) {
    const int cap = train_list_cap(*g, ytm::TrainKind::kResident, cpw);
    if (train_lds_fits(*g, ytm::TrainKind::kResident, cpw, cap)) kind = ytm::TrainKind::kResident;
  }
  g->list_cap = train_list_cap(*g, kind, cpw);
  set_mask_lds(g, kind, cpw);
  return kind;
}

// Models that train one sample per ordinary launch (launch_step) instead of on a
// persistent kernel: clause banks (coalesced=False) and models of more than 64 classes
// (the persistent kernels keep a class per lane).
bool per_sample_training(const Geom& g) { return !g.coalesced || g.K > 64; }

// fit() with one ordinary launch per sample plus one (launch_step), no persistent kernel
// and no wait between workgroups: per_sample_training models, and models whose persistent
// grid does not fit the device.  Slot memory: three class-sum rows [3][K] int64, then sel
// [C] and ninc [C].
int fit_steps(ytm_model* m, const ytm_dataset* ds, int64_t first, int64_t count, const uint32_t* drop,
              const float* inject) {
  const Geom& g = m->g;
  const bool inj = inject != nullptr;
  const int64_t block = g.C * g.P + 2 * g.C * g.K + g.C * g.K * g.L;
  int64_t chunk = count;  // samples per copy of the injected blocks (<= 1 GiB)
  if (inj) chunk = std::min<int64_t>(chunk, std::max<int64_t>(1, ((int64_t)1 << 30) / (block * 4)));
  int rc = ensure_slots(m, (size_t)(3 * g.K * 8 + g.C * 8));
  if (rc) return rc;
  long long* sums = (long long*)m->d_slots;
  int* d_sel = (int*)(sums + 3 * g.K);
  int* d_ninc = d_sel + g.C;
  uint32_t* d_drop = nullptr;
  float* d_inj = nullptr;
  std::vector<uint32_t> zeros;
  if (!drop) {
    zeros.assign((size_t)g.C, 0u);
    drop = zeros.data();
  }
  rc = upload((void**)&d_drop, drop, (size_t)g.C * 4, m->stream);
  if (rc) return rc;
  if (inj) {
    hipError_t e = hipMalloc(&d_inj, (size_t)(chunk * block) * 4);
    if (e != hipSuccess) {
      (void)hipFree(d_drop);
      return fail(YTM_EHIP, std::string("hipMalloc(inject) failed: ") + hipGetErrorString(e));
    }
  }
  auto finish = [&](int code) {
    (void)hipStreamSynchronize(m->stream);
    (void)hipFree(d_drop);
    if (d_inj) (void)hipFree(d_inj);
    return code;
  };
#define BANK_TRY(expr)                                                                          \
  do {                                                                                          \
    hipError_t e_ = (expr);                                                                     \
    if (e_ != hipSuccess)                                                                       \
      return finish(fail(YTM_EHIP, std::string(#expr) + " failed: " + hipGetErrorString(e_)));  \
  } while (0)
  BANK_TRY(hipMemsetAsync(m->d_counters, 0, 128, m->stream));
  m->w_bound += (double)count;
  double ms_total = 0.0;
  int launches = 0;
  for (int64_t s = 0; s < count; s += chunk) {
    const int64_t n = std::min(chunk, count - s);
    if (inj)
      BANK_TRY(hipMemcpyAsync(d_inj, inject + s * block, (size_t)(n * block) * 4, hipMemcpyHostToDevice, m->stream));
    ytm::TrainArgs a{};
    a.planes = m->d_planes;
    a.weights = m->d_w;
    a.patch_w = m->d_pw;
    a.bias = m->d_bias;
    a.X = ds->d_X + (first + s) * g.P * g.W;
    a.Y = ds->d_Y + (first + s) * g.K;
    a.drop = d_drop;
    a.inject = d_inj;
    a.inv_rank = m->d_inv_rank;
    a.counters = m->d_counters;
    a.err = m->d_err;
    a.inject_block = block;
    a.step0 = m->stats.step + (uint64_t)s;
    a.seed = m->params.seed;
    a.N = (int)n;
    a.g = g;
    BANK_TRY(hipEventRecord(m->ev0, m->stream));
    BANK_TRY(ytm::launch_fill_u64((unsigned long long*)sums, 3 * g.K, m->stream));
    for (int64_t i = 0; i <= n; ++i) BANK_TRY(ytm::launch_step(a, (int)i, sums, d_sel, d_ninc, inj, m->stream));
    BANK_TRY(hipEventRecord(m->ev1, m->stream));
    BANK_TRY(hipEventSynchronize(m->ev1));
    float ms = 0.0f;
    BANK_TRY(hipEventElapsedTime(&ms, m->ev0, m->ev1));
    ms_total += ms;
    launches += (int)(n + 1);
  }
  unsigned long long cnt[16] = {0};
  BANK_TRY(hipMemcpy(cnt, m->d_counters, sizeof(cnt), hipMemcpyDeviceToHost));
#undef BANK_TRY
  for (int j = 0; j < 8; ++j) m->stats.last_fit_phase_us[j] = 0.0;
  m->stats.last_fit_stream = 0;
  m->stats.last_fit_feedback_samples = cnt[12];
  m->feedback_frac = (double)cnt[12] / (double)count;
  m->stats.last_fit_evaluations = (uint64_t)count;
  for (int j = 0; j < 3; ++j) m->stats.last_fit_draws[j] = 0;
  m->stats.last_fit_wait_frac = 0.0;
  m->stats.train_kind = (int32_t)ytm::TrainKind::kSteps;
  m->stats.train_specialised = 0;
  m->stats.train_workgroups = (int32_t)std::min<int64_t>((g.C * 64 + 255) / 256, 65536);  // per launch
  m->stats.step += (uint64_t)count;
  m->stats.last_fit_samples = (uint64_t)count;
  m->stats.last_fit_updates = cnt[0];
  m->stats.total_updates += cnt[0];
  m->stats.last_fit_kernel_ms = ms_total;
  m->stats.last_fit_launches = launches;
  return finish(YTM_OK);
}

}  // namespace

extern "C" {

const char* ytm_last_error(void) { return g_error.c_str(); }

int ytm_shutdown(void) {
  const int failed = ytm::jit_unload_all();
  if (failed) return fail(YTM_EHIP, std::to_string(failed) + " training-kernel module(s) failed to unload");
  return YTM_OK;
}

int ytm_create(const ytm_params* params, ytm_model** out) {
  if (!params || !out) return fail(YTM_EINVAL, "null argument");
  *out = nullptr;
  Geom g;
  int rc = resolve_geometry(*params, &g);
  if (rc) return rc;
  ytm_model* m = new ytm_model();
  m->params = *params;
  m->g = g;
  std::memset(&m->stats, 0, sizeof(m->stats));
  auto cleanup = [&](int code) {
    ytm_destroy(m);
    return code;
  };
  if (hipGetDevice(&m->device) != hipSuccess) return cleanup(fail(YTM_EHIP, "no HIP device"));
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, m->device) != hipSuccess) return cleanup(fail(YTM_EHIP, "device query failed"));
  m->cus = prop.multiProcessorCount;
  if (!prop.cooperativeLaunch) return cleanup(fail(YTM_EHIP, "device lacks cooperative launch"));
#define CREATE_TRY(expr)                                                                       \
  do {                                                                                         \
    hipError_t e_ = (expr);                                                                    \
    if (e_ != hipSuccess)                                                                      \
      return cleanup(fail(YTM_EHIP, std::string(#expr) + " failed: " + hipGetErrorString(e_))); \
  } while (0)
  CREATE_TRY(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking));
  CREATE_TRY(hipEventCreate(&m->ev0));
  CREATE_TRY(hipEventCreate(&m->ev1));
  CREATE_TRY(hipMalloc(&m->d_planes, (size_t)(g.C * g.np * g.W) * 4));
  CREATE_TRY(hipMalloc(&m->d_w, (size_t)(g.C * g.K) * 4));
  CREATE_TRY(hipMalloc(&m->d_pw, (size_t)(g.C * g.P) * 4));
  CREATE_TRY(hipMalloc(&m->d_bias, (size_t)g.K * 4));
  CREATE_TRY(hipMalloc(&m->d_ninc, (size_t)g.C * 4));
  CREATE_TRY(hipMalloc(&m->d_inv_rank, (size_t)(g.P + 1) * 4));
  CREATE_TRY(hipMalloc(&m->d_counters, 128));
  CREATE_TRY(hipMalloc(&m->d_err, 16));
  std::vector<float> inv((size_t)g.P + 1);
  inv[0] = 0.0f;
  for (int64_t r = 1; r <= g.P; ++r) inv[r] = 1.0f / (float)r;  // IEEE fp32 division
  CREATE_TRY(hipMemcpyAsync(m->d_inv_rank, inv.data(), inv.size() * 4, hipMemcpyHostToDevice, m->stream));
  CREATE_TRY(hipMemsetAsync(m->d_pw, 0, (size_t)(g.C * g.P) * 4, m->stream));
  CREATE_TRY(hipMemsetAsync(m->d_bias, 0, (size_t)g.K * 4, m->stream));
  CREATE_TRY(ytm::launch_init_state(m->d_planes, m->d_w, g, params->seed, m->stream));
  CREATE_TRY(hipStreamSynchronize(m->stream));
#undef CREATE_TRY
  *out = m;
  return YTM_OK;
}

void ytm_destroy(ytm_model* m) {
  if (!m) return;
  if (m->stream) (void)hipStreamSynchronize(m->stream);
  void* bufs[] = {m->d_planes, m->d_w,    m->d_pw,   m->d_bias, m->d_ninc,  m->d_inv_rank,
                  m->d_counters, m->d_err, m->d_slots, m->d_sacc, m->d_sout, m->d_slists};
  for (void* b : bufs)
    if (b) (void)hipFree(b);
  if (m->h_sout) (void)hipHostFree(m->h_sout);
  if (m->ev0) (void)hipEventDestroy(m->ev0);
  if (m->ev1) (void)hipEventDestroy(m->ev1);
  if (m->stream) (void)hipStreamDestroy(m->stream);
  delete m;
}

int ytm_load_train_kernels(ytm_model* m, int32_t kinds[4], int32_t* n_kinds) {
  if (!m || !kinds || !n_kinds) return fail(YTM_EINVAL, "null argument");
  *n_kinds = 0;
  if (per_sample_training(m->g) || !ytm::jit_enabled()) return YTM_OK;  // built-in kernels only
  const char* force_global = std::getenv("YTM_TRAIN_GLOBAL");
  const bool global = force_global && std::atoi(force_global) > 0;
  auto load = [&](const Geom& g, ytm::TrainKind kind) {
    std::string why;
    if (!ytm::jit_train_kernel(g, kind, false, &why)) return fail(YTM_EHIP, "training kernel: " + why);
    kinds[(*n_kinds)++] = (int32_t)kind;
    return (int)YTM_OK;
  };
  Geom gs;
  if (stream_geometry(m, false, global, 0, &gs))
    if (int rc = load(gs, ytm::TrainKind::kStream)) return rc;
  int cpw;
  Geom g = train_geometry(m->g, m->cus, &cpw);
  const ytm::TrainKind kind = choose_train_kind(&g, cpw, global);
  return load(g, kind);
}

int ytm_compile_train_kernel(const ytm_params* params, int train_kind, int injected, int compute_units) {
  if (!params) return fail(YTM_EINVAL, "null params");
  if (train_kind < 0 || train_kind > 3) return fail(YTM_EINVAL, "train_kind must be 0, 1, 2 or 3");
  if (compute_units < 0) return fail(YTM_EINVAL, "compute_units must be >= 0");
  Geom model;
  int rc = resolve_geometry(*params, &model);
  if (rc) return rc;
  if (per_sample_training(model))
    return fail(YTM_EINVAL, "clause banks (coalesced=False) and models of more than 64 classes train with built-in "
                            "kernels, one launch per sample; none is compiled per model");
  if (train_kind == 3) {
    Geom gs;
    if (injected || !stream_shape(model, compute_units > 0 ? compute_units : 256, &gs))
      return fail(YTM_EINVAL, "train_kind 3 (streaming) is for one-patch models with coalesced classes in the "
                              "counter stream, at most 64 clauses per workgroup");
    std::vector<char> code;
    std::string why;
    if (!ytm::jit_compile(gs, ytm::TrainKind::kStream, false, &code, &why)) return fail(YTM_EHIP, why);
    return YTM_OK;
  }
  int cpw;
  Geom g = train_geometry(model, compute_units > 0 ? compute_units : 256, &cpw);
  const bool valid = train_kind == 1 ? g.P == 1 : train_kind == 2 ? g.P > 1 : (g.P == 1 || ytm::literal_major(g));
  if (!valid)
    return fail(YTM_EINVAL, "train_kind 1 is for one patch, 2 for several, 0 for one patch or a literal-major model");
  g.list_cap = train_list_cap(g, (ytm::TrainKind)train_kind, cpw);
  set_mask_lds(&g, (ytm::TrainKind)train_kind, cpw);
  std::vector<char> code;
  std::string why;
  if (!ytm::jit_compile(g, (ytm::TrainKind)train_kind, injected != 0, &code, &why))
    return fail(YTM_EHIP, why);
  return YTM_OK;
}

int ytm_geometry(const ytm_model* m, int64_t out[4]) {
  if (!m || !out) return fail(YTM_EINVAL, "null argument");
  out[0] = m->g.L;
  out[1] = m->g.W;
  out[2] = m->g.P;
  out[3] = m->g.np;
  return YTM_OK;
}

int ytm_get_stats(const ytm_model* m, ytm_stats* out) {
  if (!m || !out) return fail(YTM_EINVAL, "null argument");
  *out = m->stats;
  return YTM_OK;
}

int ytm_set_seed(ytm_model* m, uint64_t seed) {
  if (!m) return fail(YTM_EINVAL, "null argument");
  m->params.seed = seed;
  m->stats.step = 0;
  return YTM_OK;
}

int ytm_encode(ytm_model* m, const uint32_t* X, int64_t N, uint32_t* out) {
  if (!m || (N > 0 && (!X || !out)) || N < 0) return fail(YTM_EINVAL, "bad encode arguments");
  if (N == 0) return YTM_OK;
  const Geom& g = m->g;
  // Chunk so that one chunk's encoded output stays below 1 GiB.
  const int64_t per = std::max<int64_t>(1, ((int64_t)1 << 30) / (g.P * g.W * 4));
  uint32_t *dX = nullptr, *dO = nullptr;
  const int64_t chunk = std::min(per, N);
  HIP_TRY(hipMalloc(&dX, (size_t)(chunk * g.F) * 4));
  hipError_t e = hipMalloc(&dO, (size_t)(chunk * g.P * g.W) * 4);
  if (e != hipSuccess) {
    (void)hipFree(dX);
    return fail(YTM_EHIP, std::string("hipMalloc failed: ") + hipGetErrorString(e));
  }
  double ms_total = 0.0;
  int rc = YTM_OK;
  for (int64_t s = 0; s < N && rc == YTM_OK; s += chunk) {
    const int64_t n = std::min(chunk, N - s);
    e = hipMemcpyAsync(dX, X + s * g.F, (size_t)(n * g.F) * 4, hipMemcpyHostToDevice, m->stream);
    if (e == hipSuccess) e = hipEventRecord(m->ev0, m->stream);
    if (e == hipSuccess) e = ytm::launch_encode(dX, n, dO, g, m->stream);
    if (e == hipSuccess) e = hipEventRecord(m->ev1, m->stream);
    if (e == hipSuccess)
      e = hipMemcpyAsync(out + s * g.P * g.W, dO, (size_t)(n * g.P * g.W) * 4, hipMemcpyDeviceToHost, m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, m->ev0, m->ev1);
    ms_total += ms;
    if (e != hipSuccess) rc = fail(YTM_EHIP, std::string("encode failed: ") + hipGetErrorString(e));
  }
  m->stats.last_encode_kernel_ms = ms_total;
  (void)hipFree(dX);
  (void)hipFree(dO);
  return rc;
}

int ytm_encode_binarized(ytm_model* m, const void* X, int x_dtype, int64_t N, const void* thresholds,
                         int int_thresholds, int nthr, int kind, int edge_bins, uint32_t* out) {
  if (!m || N < 0 || (N > 0 && (!X || !out)) || !thresholds) return fail(YTM_EINVAL, "bad encode arguments");
  const size_t es = dtype_size(x_dtype);
  if (es == 0) return fail(YTM_EINVAL, "unsupported binarizer input type");
  if (kind != 0 && kind != 1) return fail(YTM_EINVAL, "binarizer kind must be 0 (thermometer) or 1 (one-hot)");
  if (nthr < (kind == 1 ? 2 : 1)) return fail(YTM_EINVAL, "bad binarizer arguments");
  if (int_thresholds && (x_dtype == YTM_DTYPE_F32 || x_dtype == YTM_DTYPE_F64))
    return fail(YTM_EINVAL, "integer thresholds need integer input");
  const Geom& g = m->g;
  const int64_t width = kind == 0 ? nthr : nthr - 1 + (edge_bins ? 2 : 0);
  if (width < 1 || g.F % width != 0)
    return fail(YTM_EINVAL, "the binned values per sample (raw values x " + std::to_string(width) +
                                " levels) must be dim0 * dim1 * dim2 = " + std::to_string(g.F));
  if (N == 0) return YTM_OK;
  const int64_t Fr = g.F / width;  // raw values per sample
  // Chunk so that one chunk's encoded output stays below 1 GiB.
  const int64_t chunk = std::min(std::max<int64_t>(1, ((int64_t)1 << 30) / (g.P * g.W * 4)), N);
  void* dT = nullptr;
  void* dX = nullptr;
  uint32_t* dO = nullptr;
  int rc = upload(&dT, thresholds, (size_t)nthr * 8, m->stream);
  hipError_t e = hipSuccess;
  if (!rc) e = hipMalloc(&dX, (size_t)(chunk * Fr) * es);
  if (!rc && e == hipSuccess) e = hipMalloc((void**)&dO, (size_t)(chunk * g.P * g.W) * 4);
  double ms_total = 0.0;
  for (int64_t s = 0; !rc && e == hipSuccess && s < N; s += chunk) {
    const int64_t n = std::min(chunk, N - s);
    e = hipMemcpyAsync(dX, (const char*)X + (size_t)(s * Fr) * es, (size_t)(n * Fr) * es, hipMemcpyHostToDevice,
                       m->stream);
    if (e == hipSuccess) e = hipEventRecord(m->ev0, m->stream);
    if (e == hipSuccess)
      e = ytm::launch_encode_binned(dX, x_dtype, n, Fr, dT, int_thresholds != 0, nthr, kind == 1, edge_bins != 0, dO,
                                    g, m->stream);
    if (e == hipSuccess) e = hipEventRecord(m->ev1, m->stream);
    if (e == hipSuccess)
      e = hipMemcpyAsync(out + s * g.P * g.W, dO, (size_t)(n * g.P * g.W) * 4, hipMemcpyDeviceToHost, m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, m->ev0, m->ev1);
    ms_total += ms;
  }
  if (!rc && e != hipSuccess) rc = fail(YTM_EHIP, std::string("encode failed: ") + hipGetErrorString(e));
  m->stats.last_encode_kernel_ms = ms_total;
  if (dT) (void)hipFree(dT);
  if (dX) (void)hipFree(dX);
  if (dO) (void)hipFree(dO);
  return rc;
}

int ytm_dataset_create(ytm_model* m, const uint32_t* encX, const int32_t* encY, int64_t N, ytm_dataset** out) {
  if (!m || !out || N < 0 || (N > 0 && !encX)) return fail(YTM_EINVAL, "bad dataset arguments");
  *out = nullptr;
  const Geom& g = m->g;
  ytm_dataset* ds = new ytm_dataset{m, nullptr, nullptr, N, nullptr, 0, nullptr};
  int rc = upload((void**)&ds->d_X, encX, (size_t)(N * g.P * g.W) * 4, m->stream);
  if (!rc && encY) rc = upload((void**)&ds->d_Y, encY, (size_t)(N * g.K) * 4, m->stream);
  if (!rc && ytm::literal_major(g) && N > 0) {
    // Several patches: the training kernel evaluates clauses on a literal-major copy.
    const size_t bytes = (size_t)(N * g.L * ((g.P + 31) / 32)) * 4;
    hipError_t e = hipMalloc(&ds->d_XT, bytes);
    if (e == hipSuccess) e = ytm::launch_transpose(ds->d_X, N, ds->d_XT, g, m->stream);
    // the order of the training kernels' literal lists, from the densities of the first samples
    if (e == hipSuccess) e = hipMalloc(&ds->d_order, (size_t)ytm::kOrderBuckets * g.W * 4);
    if (e == hipSuccess) e = ytm::launch_literal_order(nullptr, ds->d_XT, N, g, ds->d_order, m->stream);
    if (e == hipSuccess && g.append_negated) {
      // Encoded samples hold the negations as complements (BaseTM.encode); samples encoded
      // elsewhere may not, so the training kernels rely on it only where this check holds.
      int* d_ok = nullptr;
      int ok = 1;
      e = hipMalloc(&d_ok, sizeof(int));
      if (e == hipSuccess) e = hipMemcpyAsync(d_ok, &ok, sizeof(int), hipMemcpyHostToDevice, m->stream);
      if (e == hipSuccess) e = ytm::launch_xt_halves_check(ds->d_XT, N, g, d_ok, m->stream);
      if (e == hipSuccess) e = hipMemcpyAsync(&ok, d_ok, sizeof(int), hipMemcpyDeviceToHost, m->stream);
      if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
      if (d_ok) (void)hipFree(d_ok);
      ds->xt_halves = e == hipSuccess && ok == 1;
    }
    if (e != hipSuccess) rc = fail(YTM_EHIP, std::string("literal-major copy: ") + hipGetErrorString(e));
  }
  if (!rc) {
    hipError_t e = hipStreamSynchronize(m->stream);
    if (e != hipSuccess) rc = fail(YTM_EHIP, hipGetErrorString(e));
  }
  if (rc) {
    ytm_dataset_destroy(ds);
    return rc;
  }
  *out = ds;
  return YTM_OK;
}

void ytm_dataset_destroy(ytm_dataset* ds) {
  if (!ds) return;
  if (ds->d_X) (void)hipFree(ds->d_X);
  if (ds->d_Y) (void)hipFree(ds->d_Y);
  if (ds->d_XT) (void)hipFree(ds->d_XT);
  if (ds->d_order) (void)hipFree(ds->d_order);
  delete ds;
}

namespace {
// Feedback share below which one-patch models stream: per sample the streaming kernel costs
// about 0.2 us plus 6-7 us per sample with feedback, the resident kernel about 3 us (config 2,
// epoch 1 in segments of 10000 samples: at 85% feedback streaming took 75 ms, at 53% 38 ms,
// at 35% 25 ms; resident 28-35 ms; config 1 at 96%: resident 11% faster).
constexpr double kStreamBelow = 0.55;
int fit_range(ytm_model* m, const ytm_dataset* ds, int64_t first, int64_t count, const uint32_t* drop,
              const float* inject);
}

// Samples [first, first + count) in order.  A fit of at least 8192 samples of a one-patch
// model that the streaming kernel can take goes in segments while its recent feedback share
// is at kStreamBelow or more (the resident kernel then, re-decided after each segment of a
// sixth of the fit, at least 4096 samples), the rest in one streaming launch: the first
// epoch of a new model starts with feedback at nearly every sample and ends with few (config
// 2: 85% of the first 10000 samples, 53% of the next, 19% of the last).  The statistics add
// up over the segments.
int ytm_fit_dataset(ytm_model* m, const ytm_dataset* ds, int64_t first, int64_t count, const uint32_t* drop,
                    const float* inject) {
  if (!m || !ds || ds->m != m) return fail(YTM_EINVAL, "dataset does not belong to this model");
  if (!ds->d_Y) return fail(YTM_EINVAL, "dataset has no targets");
  if (first < 0 || count < 0 || first + count > ds->N) return fail(YTM_EINVAL, "sample range out of bounds");
  if (int rc = check_valid(m)) return rc;
  const char* stream_env = std::getenv("YTM_TRAIN_STREAM");
  const char* force_global = std::getenv("YTM_TRAIN_GLOBAL");
  Geom gs;
  const bool segmented = !stream_env && !(force_global && std::atoi(force_global) > 0) && count >= 8192 &&
                         !per_sample_training(m->g) && stream_geometry(m, inject != nullptr, false, count, &gs);
  if (!segmented) return fit_range(m, ds, first, count, drop, inject);
  const int64_t seg = std::max<int64_t>(4096, count / 6);
  const int64_t block = m->g.C * m->g.P + 2 * m->g.C * m->g.K + m->g.C * m->g.K * m->g.L;  // injected floats per sample
  ytm_stats sum = m->stats;
  sum.last_fit_samples = sum.last_fit_updates = sum.last_fit_feedback_samples = sum.last_fit_evaluations = 0;
  sum.last_fit_kernel_ms = 0.0;
  sum.last_fit_launches = 0;
  double phase[8] = {0, 0, 0, 0, 0, 0, 0, 0}, wait_ms = 0.0;
  for (int64_t s = 0; s < count;) {
    const int64_t n = m->feedback_frac < kStreamBelow ? count - s : std::min(seg, count - s);
    if (int rc = fit_range(m, ds, first + s, n, drop, inject ? inject + s * block : nullptr)) return rc;
    const ytm_stats& st = m->stats;
    sum.last_fit_samples += st.last_fit_samples;
    sum.last_fit_updates += st.last_fit_updates;
    sum.last_fit_feedback_samples += st.last_fit_feedback_samples;
    sum.last_fit_evaluations += st.last_fit_evaluations;
    sum.last_fit_kernel_ms += st.last_fit_kernel_ms;
    sum.last_fit_launches += st.last_fit_launches;
    for (int j = 0; j < 8; ++j) phase[j] += st.last_fit_phase_us[j] * (double)n;
    wait_ms += st.last_fit_wait_frac * st.last_fit_kernel_ms;
    s += n;
  }
  ytm_stats& st = m->stats;  // step, total updates and the last segment's kernel stay as they are
  st.last_fit_samples = sum.last_fit_samples;
  st.last_fit_updates = sum.last_fit_updates;
  st.last_fit_feedback_samples = sum.last_fit_feedback_samples;
  st.last_fit_evaluations = sum.last_fit_evaluations;
  st.last_fit_kernel_ms = sum.last_fit_kernel_ms;
  st.last_fit_launches = sum.last_fit_launches;
  for (int j = 0; j < 8; ++j) st.last_fit_phase_us[j] = phase[j] / (double)count;
  st.last_fit_wait_frac = sum.last_fit_kernel_ms > 0.0 ? wait_ms / sum.last_fit_kernel_ms : 0.0;
  return YTM_OK;
}

namespace {
int fit_range(ytm_model* m, const ytm_dataset* ds, int64_t first, int64_t count, const uint32_t* drop,
              const float* inject) {
  ++m->planes_version;  // before any launch: also when the fit fails part-way
  m->stats.last_fit_samples = 0;
  m->stats.last_fit_updates = 0;
  m->stats.last_fit_kernel_ms = 0.0;
  m->stats.last_fit_launches = 0;
  if (count == 0) return YTM_OK;
  if (per_sample_training(m->g)) return fit_steps(m, ds, first, count, drop, inject);
  const bool inj = inject != nullptr;
  const char* force_global = std::getenv("YTM_TRAIN_GLOBAL");
  const bool global = force_global && std::atoi(force_global) > 0;
  int cpw;
  Geom g;
  ytm::TrainKind kind;
  int rng_slots = 0;
  size_t lds = 0;
  // The streaming kernel pays when few samples need feedback: it is taken unless the last
  // fit had feedback at kStreamBelow of its samples or more, or YTM_TRAIN_STREAM forces it
  // (1) or rules it out (0).
  const char* stream_env = std::getenv("YTM_TRAIN_STREAM");
  const bool stream_forced = stream_env && std::atoi(stream_env) > 0;
  if ((stream_forced || m->feedback_frac < kStreamBelow) && stream_geometry(m, inj, global, count, &g)) {
    kind = ytm::TrainKind::kStream;
    cpw = ytm::kStreamClauses;
    lds = ytm::stream_lds_bytes(g, g.threads);
  } else {
    g = train_geometry(m->g, m->cus, &cpw);  // the training kernels read both
    kind = choose_train_kind(&g, cpw, global);
    rng_slots = kind == ytm::TrainKind::kResident ? ytm::train_rng_slots(cpw, g) : 0;
    lds = ytm::train_lds_bytes(kind, cpw, rng_slots, g);
  }
  const int grid = g.grid, D = g.groups;
  // Kernel specialised for this model's geometry (hipRTC), else the built-in one.
  // YTM_JIT=0 selects the built-in kernel; YTM_JIT=2 makes an unavailable compile an error.
  hipFunction_t jit_fn = nullptr;
  if (ytm::jit_enabled()) {
    std::string why;
    jit_fn = ytm::jit_train_kernel(g, kind, inj, &why);
    const char* jit_env = std::getenv("YTM_JIT");
    if (!jit_fn && jit_env && std::atoi(jit_env) == 2)
      return fail(YTM_EHIP, "specialised training kernel unavailable: " + why);
  }
  if (!jit_fn) g.threads = ytm::kTrainThreads;
  int bpc = 0;
  if (jit_fn)
    HIP_TRY(ytm::jit_occupancy(jit_fn, g.threads, lds, &bpc));
  else
    HIP_TRY(ytm::train_occupancy(kind, inj, lds, &bpc));
  // a persistent grid that cannot be co-resident (its LDS, e.g. thresholds for very many
  // patches) trains one sample per launch instead
  if ((int64_t)bpc * m->cus < grid) return fit_steps(m, ds, first, count, drop, inject);
  m->stats.train_workgroups = grid;

  // Per-launch sample count: bounded by the class-sum slot memory (<= 256 MiB) and, in
  // injected mode, by the size of the injected block buffer (<= 1 GiB).
  const int64_t ks = (g.K + 15) & ~(int64_t)15;
  const int64_t slot_stride = D == 1 ? ks : (2 * (int64_t)D + 1) * ks;
  // the streaming kernel uses up to stream_rows(n) rows of ks words for n samples
  const int64_t slot_row = kind == ytm::TrainKind::kStream ? ytm::stream_rows(1) * ks * 8 : slot_stride * 8;
  int64_t per_launch = std::max<int64_t>(1, ((int64_t)256 << 20) / slot_row);
  const int64_t block = g.C * g.P + 2 * g.C * g.K + g.C * g.K * g.L;
  if (inj) per_launch = std::min<int64_t>(per_launch, std::max<int64_t>(1, ((int64_t)1 << 30) / (block * 4)));
  per_launch = std::min<int64_t>(per_launch, count);
  int rc = ensure_slots(m, (size_t)(per_launch * slot_row));
  if (rc) return rc;

  uint32_t* d_drop = nullptr;
  float* d_inj = nullptr;
  std::vector<uint32_t> zeros;
  if (!drop) {
    zeros.assign((size_t)g.C, 0u);
    drop = zeros.data();
  }
  rc = upload((void**)&d_drop, drop, (size_t)g.C * 4, m->stream);
  if (rc) return rc;
  if (inj) {
    hipError_t e = hipMalloc(&d_inj, (size_t)(per_launch * block) * 4);
    if (e != hipSuccess) {
      (void)hipFree(d_drop);
      return fail(YTM_EHIP, std::string("hipMalloc(inject) failed: ") + hipGetErrorString(e));
    }
  }
  auto finish = [&](int code) {
    (void)hipStreamSynchronize(m->stream);
    if (d_drop) (void)hipFree(d_drop);
    if (d_inj) (void)hipFree(d_inj);
    return code;
  };
#define FIT_TRY(expr)                                                                           \
  do {                                                                                          \
    hipError_t e_ = (expr);                                                                     \
    if (e_ != hipSuccess)                                                                       \
      return finish(fail(YTM_EHIP, std::string(#expr) + " failed: " + hipGetErrorString(e_)));  \
  } while (0)

  FIT_TRY(hipMemsetAsync(m->d_counters, 0, 128, m->stream));
  FIT_TRY(hipMemsetAsync(m->d_err, 0, 16, m->stream));
  double ms_total = 0.0;
  int launches = 0;
  m->w_bound += (double)count;  // before any launch: also holds if one fails part-way
  for (int64_t s = 0; s < count; s += per_launch) {
    const int64_t n = std::min(per_launch, count - s);
    if (inj)
      FIT_TRY(hipMemcpyAsync(d_inj, inject + s * block, (size_t)(n * block) * 4, hipMemcpyHostToDevice, m->stream));
    FIT_TRY(ytm::launch_fill_u64(m->d_slots, n * (slot_row / 8), m->stream));
    ytm::TrainArgs a{};
    a.planes = m->d_planes;
    a.weights = m->d_w;
    a.patch_w = m->d_pw;
    a.bias = m->d_bias;
    a.X = ds->d_X + (first + s) * g.P * g.W;
    a.XT = ds->d_XT ? ds->d_XT + (first + s) * g.L * ((g.P + 31) / 32) : nullptr;
    a.Y = ds->d_Y + (first + s) * g.K;
    a.drop = d_drop;
    a.inject = d_inj;
    a.inv_rank = m->d_inv_rank;
    a.slots = m->d_slots;
    a.counters = m->d_counters;
    a.err = m->d_err;
    a.inject_block = block;
    a.step0 = m->stats.step + (uint64_t)s;
    a.seed = m->params.seed;
    a.N = (int)n;
    a.slot_stride = slot_stride;
    a.cpw = cpw;
    a.rng_slots = rng_slots;
    a.profile = prof_level();
    const char* sg_env = std::getenv("YTM_TRAIN_STREAM_GENS");  // test hook: stops per stream
    a.stream_gens = sg_env ? std::max(0, std::atoi(sg_env)) : 0;
    const char* xh_env = std::getenv("YTM_TRAIN_XT_HALVES");  // 0: stage the whole literal-major copy
    a.xt_halves = ds->xt_halves && !(xh_env && std::atoi(xh_env) == 0);
    const char* lo_env = std::getenv("YTM_LIST_ORDER");  // 0: literal lists in index order
    a.lit_order = (lo_env && std::atoi(lo_env) == 0) ? nullptr : ds->d_order;
    const char* tt_env = std::getenv("YTM_TRAIN_TEST_TIMEOUT");  // test hook of the timeout path
    a.test_timeout = tt_env && std::atoi(tt_env) > 0;
    a.g = g;
    FIT_TRY(hipEventRecord(m->ev0, m->stream));
    if (jit_fn)
      FIT_TRY(ytm::launch_train_jit(jit_fn, a, grid, g.threads, lds, m->stream));
    else
      FIT_TRY(ytm::launch_train(a, grid, lds, kind, inj, m->stream));
    FIT_TRY(hipEventRecord(m->ev1, m->stream));
    FIT_TRY(hipEventSynchronize(m->ev1));
    float ms = 0.0f;
    FIT_TRY(hipEventElapsedTime(&ms, m->ev0, m->ev1));
    ms_total += ms;
    ++launches;
    int herr[4] = {0, 0, 0, 0};
    FIT_TRY(hipMemcpy(herr, m->d_err, sizeof(herr), hipMemcpyDeviceToHost));
    if (herr[0]) {
      m->invalid = true;
      m->reloaded = 0;
      return finish(fail(YTM_ETIMEOUT, "training kernel: the bounded wait for the class sums of sample " +
                                           std::to_string(s + herr[1]) + " expired in workgroup " +
                                           std::to_string(herr[2]) + " (count seen " + std::to_string(herr[3]) +
                                           ", grid " + std::to_string(grid) + ", groups " + std::to_string(D) + ")"));
    }
  }
  unsigned long long cnt[16] = {0};
  FIT_TRY(hipMemcpy(cnt, m->d_counters, sizeof(cnt), hipMemcpyDeviceToHost));
  // phase ticks are summed over workgroups and samples: average microseconds per sample
  for (int j = 0; j < 8; ++j) m->stats.last_fit_phase_us[j] = (double)cnt[4 + j] / 100.0 / (double)grid / (double)count;
  const unsigned long long upd = cnt[0];
  m->stats.last_fit_stream = kind == ytm::TrainKind::kStream;
  m->stats.last_fit_feedback_samples = cnt[12];
  m->feedback_frac = (double)cnt[12] / (double)count;
  m->stats.last_fit_evaluations = kind == ytm::TrainKind::kStream ? cnt[13] / (uint64_t)grid : (uint64_t)count;
  const bool counted = prof_level() == 4;
  m->stats.last_fit_draws[0] = counted ? cnt[14] : 0;
  m->stats.last_fit_draws[1] = counted ? cnt[3] : 0;
  m->stats.last_fit_draws[2] = counted ? cnt[15] : 0;
#undef FIT_TRY
  m->stats.last_fit_wait_frac = cnt[2] ? (double)cnt[1] / (double)cnt[2] : 0.0;
  m->stats.train_kind = (int32_t)kind;
  m->stats.train_specialised = jit_fn != nullptr;
  m->stats.step += (uint64_t)count;
  m->stats.last_fit_samples = (uint64_t)count;
  m->stats.last_fit_updates = upd;
  m->stats.total_updates += upd;
  m->stats.last_fit_kernel_ms = ms_total;
  m->stats.last_fit_launches = launches;
  return finish(YTM_OK);
}
}  // namespace

int ytm_fit(ytm_model* m, const uint32_t* encX, const int32_t* encY, int64_t N, const uint32_t* drop,
            const float* inject) {
  if (!m || N < 0 || (N > 0 && (!encX || !encY))) return fail(YTM_EINVAL, "bad fit arguments");
  ytm_dataset* ds = nullptr;
  int rc = ytm_dataset_create(m, encX, encY, N, &ds);
  if (rc) return rc;
  rc = ytm_fit_dataset(m, ds, 0, N, drop, inject);
  ytm_dataset_destroy(ds);
  return rc;
}

}  // extern "C"

namespace {

// Which scoring kernel a dataset takes, and the device buffers it needs besides the output:
// literal lists (lists_bytes, several patches or one patch with wide clauses) and the int64
// class-sum accumulators, acc_per_sample bytes per sample (per-chunk slices for the tiled
// one-patch scorer, chunks > 0).
struct ScorePlan {
  size_t lists_bytes;
  bool wide;
  int64_t chunks;
  size_t acc_per_sample;
};

ScorePlan score_plan(const Geom& g, bool has_xt) {
  ScorePlan p{};
  // the list-based and tiled scorers keep a class per lane: more than 64 classes take
  // launch_score's class-sum kernel
  const bool few = g.K <= 64;
  const size_t lm_bytes = has_xt && few ? ytm::score_lists_bytes(g) : 0;
  const size_t wide_bytes = lm_bytes || !few ? 0 : ytm::score_wide_bytes(g);
  p.lists_bytes = lm_bytes ? lm_bytes : wide_bytes;
  p.wide = wide_bytes > 0;
  p.chunks = p.lists_bytes ? 0 : ytm::score_tile_chunks(g);
  p.acc_per_sample = (size_t)g.K * (size_t)(p.chunks ? p.chunks : 1) * 8;
  return p;
}

// Class sums of N samples (X [N][P][W], XT its literal-major copy or null) into out (device
// float [N][K]), with the caller's buffers acc (plan.acc_per_sample * N bytes) and lists
// (plan.lists_bytes).  Enqueued on the model's stream; the include counts are current when
// the plan has no lists (the list-based scorers count the literals of their lists).
hipError_t score_samples(ytm_model* m, const ScorePlan& plan, const uint32_t* X, const uint32_t* XT, int64_t N,
                         long long* acc, void* lists, float* out, bool lists_ready = false) {
  const Geom& g = m->g;
  hipError_t e = hipSuccess;
  if (!plan.chunks) e = ytm::launch_fill_u64((unsigned long long*)acc, N * g.K, m->stream);
  if (e != hipSuccess) return e;
  if (plan.wide)
    e = ytm::launch_score_wide(m->d_planes, m->d_w, X, N, g, lists, lists_ready, acc, m->stream);
  else if (plan.lists_bytes)
    e = ytm::launch_score_lm(m->d_planes, m->d_w, XT, N, g, lists, acc, m->stream);
  else if (plan.chunks)
    e = ytm::launch_score_tile(m->d_planes, m->d_ninc, m->d_w, X, N, g, acc, m->w_bound, m->stream);
  else
    e = ytm::launch_score(m->d_planes, m->d_ninc, m->d_w, X, N, g, acc, m->stream);
  if (e != hipSuccess) return e;
  return plan.chunks ? ytm::launch_score_parts_finish(acc, plan.chunks, m->d_bias, N, g, out, m->stream)
                     : ytm::launch_score_finish(acc, m->d_bias, N, g, out, m->stream);
}

// ---- Scratch of the allocation-free scoring entry point: one static device array per GPU
// (each device that runs it holds its own copy, at its own address, until the process
// ends).  Host code never passes the array's name to a kernel: the name is a host-side
// stand-in, not a device address.  Its device address is looked up once per device, with
// that device current, and kept in g_scratch_ptr.
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu[kMaxDevices];  // held for a whole call: calls on one GPU share the array
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `device`'s scratch array.  The lookup is made with that device current
// (each device holds its own copy at its own address); the caller's current device is
// restored afterwards.
int scratch_address(int device, void** out) {
  if (device < 0 || device >= kMaxDevices) return fail(YTM_EINVAL, "device index out of range for the scratch table");
  if (!g_scratch_ptr[device]) {
    int prev = -1;
    hipError_t e = hipGetDevice(&prev);
    if (e == hipSuccess && prev != device) e = hipSetDevice(device);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (prev >= 0 && prev != device) (void)hipSetDevice(prev);
    if (e != hipSuccess || !p)
      return fail(YTM_EHIP, std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return YTM_OK;
}

}  // namespace

extern "C" {

int ytm_score_dataset(ytm_model* m, const ytm_dataset* ds, float* class_sums) {
  if (!m || !ds || ds->m != m || (ds->N > 0 && !class_sums)) return fail(YTM_EINVAL, "bad score arguments");
  if (int rc = check_valid(m)) return rc;
  const Geom& g = m->g;
  const int64_t N = ds->N;
  if (N == 0) return YTM_OK;
  const ScorePlan plan = score_plan(g, ds->d_XT != nullptr);
  hipError_t e = ensure_buffer(&m->d_sacc, &m->sacc_bytes, (size_t)N * plan.acc_per_sample);
  if (e == hipSuccess) e = ensure_buffer(&m->d_sout, &m->sout_bytes, (size_t)(N * g.K) * 4);
  const void* lists_before = m->d_slists;
  if (e == hipSuccess && plan.lists_bytes) e = ensure_buffer(&m->d_slists, &m->slists_bytes, plan.lists_bytes);
  if (m->d_slists != lists_before) m->slists_version = ~0ull;
  // one-patch lists (no literal order) depend on the TA states only: kept from the last call
  const bool lists_ready = plan.wide && m->slists_version == m->planes_version;
  float* dout = (float*)m->d_sout;
  int rc = YTM_OK;
  // the include counts, for the scorers that read them (the list-based ones count their lists)
  if (e == hipSuccess && !plan.lists_bytes) e = ytm::launch_ninc(m->d_planes, m->d_ninc, g, m->stream);
  if (e == hipSuccess) e = hipEventRecord(m->ev0, m->stream);
  if (e == hipSuccess)
    e = score_samples(m, plan, ds->d_X, ds->d_XT, N, (long long*)m->d_sacc, plan.lists_bytes ? m->d_slists : nullptr,
                      dout, lists_ready);
  m->slists_version = e == hipSuccess && plan.wide ? m->planes_version : ~0ull;
  if (e == hipSuccess) e = hipEventRecord(m->ev1, m->stream);
  // the sums come back through a pinned staging buffer of the model (a direct copy into
  // pageable memory goes through the runtime's own staging, in smaller pieces)
  const size_t out_bytes = (size_t)(N * g.K) * 4;
  if (e == hipSuccess && m->h_sout_bytes < out_bytes) {
    if (m->h_sout) (void)hipHostFree(m->h_sout);
    m->h_sout = nullptr;
    m->h_sout_bytes = 0;
    e = hipHostMalloc(&m->h_sout, out_bytes, hipHostMallocDefault);
    if (e == hipSuccess) m->h_sout_bytes = out_bytes;
  }
  if (e == hipSuccess) e = hipMemcpyAsync(m->h_sout, dout, out_bytes, hipMemcpyDeviceToHost, m->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
  if (e == hipSuccess) std::memcpy(class_sums, m->h_sout, out_bytes);
  float ms = 0.0f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, m->ev0, m->ev1);
  if (e != hipSuccess) rc = fail(YTM_EHIP, std::string("score failed: ") + hipGetErrorString(e));
  m->stats.last_score_kernel_ms = ms;
  return rc;
}

int ytm_score_dataset_noalloc(ytm_model* m, const ytm_dataset* ds, float* d_class_sums) {
  if (!m || !ds || ds->m != m || (ds->N > 0 && !d_class_sums)) return fail(YTM_EINVAL, "bad score arguments");
  if (int rc = check_valid(m)) return rc;
  const Geom& g = m->g;
  const int64_t N = ds->N;
  if (N == 0) return YTM_OK;
  const ScorePlan plan = score_plan(g, ds->d_XT != nullptr);
  const size_t lists_room = (plan.lists_bytes + 255) & ~(size_t)255;  // the sums start 256-byte aligned
  if (lists_room + plan.acc_per_sample > kNoAllocScratchBytes)
    return fail(YTM_EINVAL, "model too large for the allocation-free scorer: it needs " +
                                std::to_string(lists_room + plan.acc_per_sample) + " bytes of scratch for one sample, " +
                                "the scratch holds " + std::to_string(kNoAllocScratchBytes));
  if (m->device < 0 || m->device >= kMaxDevices) return fail(YTM_EINVAL, "device index out of range for the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu[m->device]);
  void* base = nullptr;
  int rc = scratch_address(m->device, &base);
  if (rc) return rc;
  void* lists = plan.lists_bytes ? base : nullptr;
  long long* acc = (long long*)((unsigned char*)base + lists_room);
  // samples per pass: as many as the accumulators of the rest of the scratch hold
  const int64_t per_pass = (int64_t)((kNoAllocScratchBytes - lists_room) / plan.acc_per_sample);
  const int64_t PW = (g.P + 31) / 32;
  hipError_t e = ytm::launch_ninc(m->d_planes, m->d_ninc, g, m->stream);
  if (e == hipSuccess) e = hipEventRecord(m->ev0, m->stream);
  for (int64_t first = 0; e == hipSuccess && first < N; first += per_pass) {
    const int64_t n = N - first < per_pass ? N - first : per_pass;
    e = score_samples(m, plan, ds->d_X + first * g.P * g.W, ds->d_XT ? ds->d_XT + first * g.L * PW : nullptr, n, acc,
                      lists, d_class_sums + first * g.K);
  }
  if (e == hipSuccess) e = hipEventRecord(m->ev1, m->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
  float ms = 0.0f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, m->ev0, m->ev1);
  if (e != hipSuccess) return fail(YTM_EHIP, std::string("score failed: ") + hipGetErrorString(e));
  m->stats.last_score_kernel_ms = ms;
  return YTM_OK;
}

int ytm_score(ytm_model* m, const uint32_t* encX, int64_t N, float* class_sums) {
  if (!m || N < 0 || (N > 0 && (!encX || !class_sums))) return fail(YTM_EINVAL, "bad score arguments");
  ytm_dataset* ds = nullptr;
  int rc = ytm_dataset_create(m, encX, nullptr, N, &ds);
  if (rc) return rc;
  rc = ytm_score_dataset(m, ds, class_sums);
  ytm_dataset_destroy(ds);
  return rc;
}

int ytm_transform(ytm_model* m, const uint32_t* encX, int64_t N, int mode, uint32_t* out) {
  if (!m || N < 0 || mode < 0 || mode > 2 || (N > 0 && (!encX || !out)))
    return fail(YTM_EINVAL, "bad transform arguments");
  if (int rc = check_valid(m)) return rc;
  if (N == 0) return YTM_OK;
  const Geom& g = m->g;
  const int64_t PW = (g.P + 31) / 32;
  const int64_t per_out = g.C * (mode == 0 ? 1 : (mode == 1 ? g.P : PW));  // uint32 per sample
  const size_t lm_bytes = ytm::score_lists_bytes(g);
  const bool lm = lm_bytes > 0;
  const size_t wide_bytes = lm ? 0 : ytm::score_wide_bytes(g);  // one patch, wide clauses
  const size_t lists_bytes = lm ? lm_bytes : wide_bytes;
  const int64_t per_in = g.P * g.W + (lm ? g.L * PW : 0);
  // Device buffers per pass stay within ~1 GiB; samples go through in chunks.
  int64_t chunk = ((int64_t)1 << 30) / ((per_out + per_in) * 4);
  if (const char* v = std::getenv("YTM_TRANSFORM_CHUNK")) chunk = std::atoll(v);  // samples per pass
  chunk = chunk < 1 ? 1 : (chunk > N ? N : chunk);
  uint32_t *dX = nullptr, *dXT = nullptr, *dO = nullptr;
  void* dL = nullptr;
  hipError_t e = hipMalloc(&dX, (size_t)(chunk * g.P * g.W) * 4);
  if (e == hipSuccess) e = hipMalloc(&dO, (size_t)(chunk * per_out) * 4);
  if (e == hipSuccess && lm) e = hipMalloc(&dXT, (size_t)(chunk * g.L * PW) * 4);
  if (e == hipSuccess && lists_bytes) e = hipMalloc(&dL, lists_bytes);
  if (e == hipSuccess) e = ytm::launch_ninc(m->d_planes, m->d_ninc, g, m->stream);
  for (int64_t first = 0; e == hipSuccess && first < N; first += chunk) {
    const int64_t n = N - first < chunk ? N - first : chunk;
    e = hipMemcpyAsync(dX, encX + first * g.P * g.W, (size_t)(n * g.P * g.W) * 4, hipMemcpyHostToDevice,
                       m->stream);
    if (e == hipSuccess && lm) {
      e = ytm::launch_transpose(dX, n, dXT, g, m->stream);
      if (e == hipSuccess) e = ytm::launch_transform_lm(m->d_planes, dXT, n, g, mode, dL, first > 0, dO, m->stream);
    } else if (e == hipSuccess && wide_bytes) {
      e = ytm::launch_transform_wide(m->d_planes, dX, n, g, dL, first > 0, dO, m->stream);
    } else if (e == hipSuccess) {
      e = ytm::launch_transform(m->d_planes, m->d_ninc, dX, n, g, mode, dO, m->stream);
    }
    if (e == hipSuccess)
      e = hipMemcpyAsync(out + first * per_out, dO, (size_t)(n * per_out) * 4, hipMemcpyDeviceToHost, m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
  }
  const int rc = e == hipSuccess ? YTM_OK : fail(YTM_EHIP, std::string("transform failed: ") + hipGetErrorString(e));
  if (dX) (void)hipFree(dX);
  if (dO) (void)hipFree(dO);
  if (dXT) (void)hipFree(dXT);
  if (dL) (void)hipFree(dL);
  return rc;
}

int ytm_get_ta_state(ytm_model* m, uint32_t* out) {
  if (!m || !out) return fail(YTM_EINVAL, "null argument");
  const Geom& g = m->g;
  uint32_t* d = nullptr;
  HIP_TRY(hipMalloc(&d, (size_t)(g.C * g.L) * 4));
  hipError_t e = ytm::launch_planes_to_ta(m->d_planes, d, g, m->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(out, d, (size_t)(g.C * g.L) * 4, hipMemcpyDeviceToHost, m->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
  (void)hipFree(d);
  if (e != hipSuccess) return fail(YTM_EHIP, std::string("get_ta_state failed: ") + hipGetErrorString(e));
  return YTM_OK;
}

int ytm_set_ta_state(ytm_model* m, const uint32_t* in) {
  if (!m || !in) return fail(YTM_EINVAL, "null argument");
  const Geom& g = m->g;
  ++m->planes_version;
  // Representable and closed under the feedback dynamics: s' = s + off < 2^np.
  const uint64_t limit = ((uint64_t)1 << g.np) - 1 - g.off;
  for (int64_t i = 0; i < g.C * g.L; ++i)
    if ((uint64_t)in[i] > limit)
      return fail(YTM_ERANGE, "TA state " + std::to_string(in[i]) + " exceeds the representable maximum " +
                                  std::to_string(limit));
  uint32_t* d = nullptr;
  int rc = upload((void**)&d, in, (size_t)(g.C * g.L) * 4, m->stream);
  if (rc) return rc;
  hipError_t e = ytm::launch_ta_to_planes(d, m->d_planes, g, m->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
  (void)hipFree(d);
  if (e != hipSuccess) return fail(YTM_EHIP, std::string("set_ta_state failed: ") + hipGetErrorString(e));
  note_reload(m, 1);
  return YTM_OK;
}

int ytm_get_weights(ytm_model* m, float* out) {
  if (!m || !out) return fail(YTM_EINVAL, "null argument");
  HIP_TRY(hipMemcpyAsync(out, m->d_w, (size_t)(m->g.C * m->g.K) * 4, hipMemcpyDeviceToHost, m->stream));
  HIP_TRY(hipStreamSynchronize(m->stream));
  return YTM_OK;
}

int ytm_set_weights(ytm_model* m, const float* in) {
  if (!m || !in) return fail(YTM_EINVAL, "null argument");
  for (int64_t i = 0; i < m->g.C * m->g.K; ++i) {
    const float v = in[i];
    if (!(std::fabs(v) < 2147483648.0f) || std::nearbyint(v) != v)
      return fail(YTM_ERANGE, "clause weights must be integer-valued floats below 2^31 in magnitude");
  }
  HIP_TRY(hipMemcpyAsync(m->d_w, in, (size_t)(m->g.C * m->g.K) * 4, hipMemcpyHostToDevice, m->stream));
  HIP_TRY(hipStreamSynchronize(m->stream));
  double bound = 0.0;
  for (int64_t i = 0; i < m->g.C * m->g.K; ++i) bound = std::max(bound, (double)std::fabs(in[i]));
  m->w_bound = bound;
  note_reload(m, 2);
  return YTM_OK;
}

int ytm_get_patch_weights(ytm_model* m, int32_t* out) {
  if (!m || !out) return fail(YTM_EINVAL, "null argument");
  HIP_TRY(hipMemcpyAsync(out, m->d_pw, (size_t)(m->g.C * m->g.P) * 4, hipMemcpyDeviceToHost, m->stream));
  HIP_TRY(hipStreamSynchronize(m->stream));
  return YTM_OK;
}

int ytm_set_patch_weights(ytm_model* m, const int32_t* in) {
  if (!m || !in) return fail(YTM_EINVAL, "null argument");
  HIP_TRY(hipMemcpyAsync(m->d_pw, in, (size_t)(m->g.C * m->g.P) * 4, hipMemcpyHostToDevice, m->stream));
  HIP_TRY(hipStreamSynchronize(m->stream));
  note_reload(m, 4);
  return YTM_OK;
}

int ytm_get_bias(ytm_model* m, float* out) {
  if (!m || !out) return fail(YTM_EINVAL, "null argument");
  HIP_TRY(hipMemcpyAsync(out, m->d_bias, (size_t)m->g.K * 4, hipMemcpyDeviceToHost, m->stream));
  HIP_TRY(hipStreamSynchronize(m->stream));
  return YTM_OK;
}

}  // extern "C"

// ---------------------------------------------------------------- binarizers
namespace {


}  // namespace

extern "C" {

int ytm_binarize(const void* X, int x_dtype, int64_t n, const void* thresholds, int int_thresholds, int nthr,
                 int kind, int edge_bins, uint32_t* out) {
  const size_t es = dtype_size(x_dtype);
  if (es == 0) return fail(YTM_EINVAL, "unsupported binarizer input type");
  if (kind != 0 && kind != 1) return fail(YTM_EINVAL, "binarizer kind must be 0 (thermometer) or 1 (one-hot)");
  if (n < 0 || nthr < (kind == 1 ? 2 : 1) || !thresholds || (n > 0 && (!X || !out)))
    return fail(YTM_EINVAL, "bad binarizer arguments");
  if (int_thresholds && (x_dtype == YTM_DTYPE_F32 || x_dtype == YTM_DTYPE_F64))
    return fail(YTM_EINVAL, "integer thresholds need integer input");
  const int64_t width = kind == 0 ? nthr : nthr - 1 + (edge_bins ? 2 : 0);
  if (n == 0) return YTM_OK;
  void* dX = nullptr;
  void* dT = nullptr;
  uint32_t* dO = nullptr;
  int rc = upload(&dX, X, (size_t)n * es, nullptr);
  if (!rc) rc = upload(&dT, thresholds, (size_t)nthr * 8, nullptr);
  hipError_t e = hipSuccess;
  if (!rc) e = hipMalloc(&dO, (size_t)(n * width) * 4);
  if (!rc && e == hipSuccess)
    e = ytm::launch_binarize(dX, x_dtype, n, dT, int_thresholds != 0, nthr, kind == 1, edge_bins != 0, dO, nullptr);
  if (!rc && e == hipSuccess) e = hipMemcpy(out, dO, (size_t)(n * width) * 4, hipMemcpyDeviceToHost);
  if (!rc && e != hipSuccess) rc = fail(YTM_EHIP, std::string("binarize failed: ") + hipGetErrorString(e));
  if (dX) (void)hipFree(dX);
  if (dT) (void)hipFree(dT);
  if (dO) (void)hipFree(dO);
  return rc;
}

int ytm_collapse_bins(const uint32_t* B, int64_t rows, int64_t width, int kind, int edge_bins, int64_t* out) {
  if (kind != 0 && kind != 1) return fail(YTM_EINVAL, "binarizer kind must be 0 (thermometer) or 1 (one-hot)");
  if (rows < 0 || width < 0 || (rows > 0 && (!B || !out))) return fail(YTM_EINVAL, "bad collapse arguments");
  if (rows == 0) return YTM_OK;
  void* dB = nullptr;
  int64_t* dO = nullptr;
  int rc = upload(&dB, B, (size_t)(rows * width) * 4, nullptr);
  hipError_t e = hipSuccess;
  if (!rc) e = hipMalloc(&dO, (size_t)rows * 8);
  if (!rc && e == hipSuccess)
    e = ytm::launch_collapse_bins((const uint32_t*)dB, rows, width, kind == 1, edge_bins != 0, dO, nullptr);
  if (!rc && e == hipSuccess) e = hipMemcpy(out, dO, (size_t)rows * 8, hipMemcpyDeviceToHost);
  if (!rc && e != hipSuccess) rc = fail(YTM_EHIP, std::string("collapse_bins failed: ") + hipGetErrorString(e));
  if (dB) (void)hipFree(dB);
  if (dO) (void)hipFree(dO);
  return rc;
}

}  // extern "C"
