/*
 * ytm.h -- C-ABI of libytm.so, the MI355X (gfx950) Tsetlin Machine hot path.
 *
 * This boundary replaces the reference's PyCUDA layer (src/cutm/base.py:128-206 compiles
 * src/cutm/cuda/kernel.cu and drives its 9 kernels with prepared_call).  Every entry point
 * below names the reference interface it stands in for.  Plain pointers and sizes only:
 * host arrays are caller-owned and borrowed for the duration of a call; device memory is
 * owned by the model / dataset handles.  Calls are synchronous on return, one HIP stream
 * per model, not re-entrant per handle.  Every function returns 0 on success and a
 * nonzero status otherwise; ytm_last_error() then describes the failure (thread-local).
 */
#ifndef YTM_H
#define YTM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
enum {
    YTM_OK = 0,
    YTM_EINVAL = 1,   /* bad argument / unsupported configuration */
    YTM_EHIP = 2,     /* HIP runtime error */
    YTM_ETIMEOUT = 3, /* a persistent kernel's bounded wait expired (2 s of real time, which
                         also runs while the GPU is preempted); the model's state is then a mix
                         of samples, and ytm_fit*, ytm_score* and ytm_transform refuse it
                         (YTM_EINVAL) until ytm_set_ta_state, ytm_set_weights and
                         ytm_set_patch_weights have all loaded a state again */
    YTM_ERANGE = 4    /* state value outside what the model can represent */
};

/* Element types of the binarizer inputs (ytm_binarize). */
enum {
    YTM_DTYPE_U8 = 0,
    YTM_DTYPE_I8 = 1,
    YTM_DTYPE_U16 = 2,
    YTM_DTYPE_I16 = 3,
    YTM_DTYPE_U32 = 4,
    YTM_DTYPE_I32 = 5,
    YTM_DTYPE_I64 = 6,
    YTM_DTYPE_F32 = 7,
    YTM_DTYPE_F64 = 8
};

/* Model hyperparameters, resolved on the host exactly as src/cutm/base.py:60-121,129-152
 * resolves them into #defines.  s_inv and q_prob are S_INV and Q_PROB as the reference's
 * C preprocessor types them (float or double, kernel.cu:31-32), widened to double. */
typedef struct ytm_params {
    int32_t clauses;               /* CLAUSES = banks * number_of_clauses_per_class */
    int32_t classes;               /* CLASSES */
    int32_t dim0, dim1, dim2;      /* DIM0 (width), DIM1 (height), DIM2 (channels) */
    int32_t patch_dim0, patch_dim1;/* PATCH_DIM0, PATCH_DIM1 */
    int32_t number_of_ta_states;   /* MAX_TA_STATE */
    int32_t max_included_literals; /* MAX_INCLUDED_LITERALS (resolved: LITERALS if None) */
    int32_t append_negated;        /* APPEND_NEGATED */
    int32_t encode_loc;            /* ENCODE_LOC */
    int32_t coalesced;             /* COALESCED (CLAUSE_BANKS = coalesced ? 1 : CLASSES) */
    int32_t negative_polarity;     /* NEGATIVE_CLAUSES */
    int32_t init_neg_weights;      /* INIT_NEG_WEIGHTS */
    int32_t thresh;                /* THRESH (T) */
    double s_inv;                  /* S_INV */
    double q_prob;                 /* Q_PROB */
    uint64_t seed;                 /* key of the counter-based random stream */
} ytm_params;

typedef struct ytm_model ytm_model;
typedef struct ytm_dataset ytm_dataset;

/* Per-model counters and timings of the most recent calls (HIP events on the model's
 * stream around the kernels named). */
typedef struct ytm_stats {
    uint64_t step;               /* samples trained so far (the random stream's step) */
    uint64_t last_fit_samples;
    uint64_t last_fit_updates;   /* (sample, clause) pairs that ran a Type Ia/Ib/II branch */
    uint64_t total_updates;
    double last_fit_kernel_ms;   /* sum over the training kernel launches of the last fit */
    int32_t last_fit_launches;
    int32_t train_workgroups;    /* persistent grid size used by the training kernel (clause
                                    banks: workgroups of each per-sample launch) */
    double last_score_kernel_ms; /* class-sum kernel of the last score */
    double last_encode_kernel_ms;
    double last_fit_wait_frac;   /* share of the training kernel's time workgroups spent
                                    waiting for the per-sample class sums */
    int32_t train_kind;          /* 0 = clause state resident in LDS, 1 = global (one
                                    patch), 2 = global (several patches), 3 = resident and
                                    streaming (one patch), 4 = one ordinary launch per
                                    sample: clause banks (coalesced=0), more than 64
                                    classes, or a persistent grid that does not fit */
    int32_t train_specialised;   /* 1 when the last fit ran a training kernel compiled at run
                                    time for this model's geometry (hipRTC), 0 when it ran the
                                    built-in kernel (YTM_JIT=0, or the compile was unavailable) */
    double last_fit_phase_us[8]; /* with YTM_TRAIN_PROFILE=1: average microseconds per sample
                                    that wave 0 of each workgroup spends in each phase of the
                                    training kernel (resident: exchange, barrier, D1, barrier,
                                    D2, D3, barrier, and the slowest other wave's time in the
                                    exchange step; global: staging, publish and exchange,
                                    wait for the next sample's evaluation, decisions, literal
                                    updates, re-evaluation of the updated clauses).  YTM_TRAIN_PROFILE=2 / =3 restrict that last
                                    resident slot to the next sample's evaluation / its
                                    evaluation and the staging of the sample after it */
    uint64_t last_fit_feedback_samples; /* samples of the last fit at which some class had an
                                    update probability above zero (the streaming kernel stops
                                    there to apply feedback); the sample count for the others */
    uint64_t last_fit_evaluations; /* clause evaluations of a sample per workgroup, averaged:
                                    the sample count plus the speculative ones discarded at
                                    stops (streaming kernel); the sample count for the others */
    int32_t last_fit_stream;     /* 1 when the last fit ran the streaming kernel (train_kind
                                    is then 3) */
    int32_t reserved;
    uint64_t last_fit_draws[3];  /* with YTM_TRAIN_PROFILE=4: counter-stream words computed
                                    by the last fit's training kernel, one per lane and draw
                                    site (a Philox4x32-10 call): reservoir draws, Q-skip /
                                    update draws, literal draws.  Zero otherwise */
} ytm_stats;

/* Thread-local description of the last failure. */
const char *ytm_last_error(void);

/* Unloads the training-kernel modules compiled at run time (each on its device, after a
 * device synchronize), so that nothing of the library is left on a GPU when the process
 * exits; call it after destroying every model and dataset.  A later fit loads what it needs
 * again.  Replaces the context teardown that `import pycuda.autoinit` registers for process
 * exit (src/cutm/base.py:5), which releases the modules SourceModule loaded
 * (src/cutm/base.py:155-159).  YTM_EHIP when a module fails to unload. */
int ytm_shutdown(void);

/* Model lifetime.  Replaces BaseTM._gpu_init / _reset_clauses / _reset_weights
 * (src/cutm/base.py:128-222; kernel.cu:46-73 init_weights): TA states start at
 * number_of_ta_states/2, weights from the INIT random site, patch weights and bias 0.
 * Geometry bounds: at most 4096 classes (the reference's kernels take any CLASSES; more
 * than 64 train one sample per launch), any number of patches, any int32
 * number_of_ta_states (up to 32 bit-planes), classes * literal words * 6 below 2^32 (the
 * 32-bit literal-draw site index of the counter stream).  YTM_EINVAL otherwise. */
int ytm_create(const ytm_params *params, ytm_model **out);
void ytm_destroy(ytm_model *m);
/* L, W (=number_of_literal_chunks), P (=number_of_patches), number of TA bit-planes. */
int ytm_geometry(const ytm_model *m, int64_t out[4]);
int ytm_get_stats(const ytm_model *m, ytm_stats *out);
/* Reseed the random stream and reset its step to 0 (what re-running __init__ does). */
int ytm_set_seed(ytm_model *m, uint64_t seed);
/* Compile (and cache for this process) the training kernel specialised for the geometry
 * of *params and the launch shape used on a device with compute_units CUs (0: 256, an
 * MI355X), without touching a GPU.  train_kind as in ytm_stats (0 resident: one patch, or
 * several with ceil(P/32) <= 64; 1 global one patch; 2 global several patches; 3 streaming:
 * one patch, coalesced, counter stream only); injected != 0 for the injected-draw variant.
 * Clause-bank models (coalesced = 0) and models of more than 64 classes train with built-in
 * kernels only (train_kind 4): YTM_EINVAL.
 * The counterpart of the per-model kernel compile in BaseTM.__init__
 * (src/cutm/base.py:129-159); ytm_fit compiles on first use anyway, so calling this is
 * optional (warm-up, or checking that the compiler is available).  YTM_EHIP with the
 * compiler log in ytm_last_error() on failure. */
int ytm_compile_train_kernel(const ytm_params *params, int train_kind, int injected,
                             int compute_units);
/* Compile (when not cached) and load onto the model's device every counter-stream training
 * kernel that ytm_fit may choose for this model (the streaming kernel of a one-patch model and
 * the resident or global one), so that no fit pays for it later; the kinds loaded (train_kind
 * values) go to kinds[0 .. *n_kinds).  The counterpart of the per-model kernel compile in
 * BaseTM.__init__ (src/cutm/base.py:129-159).  Nothing is loaded for clause banks or with
 * YTM_JIT=0 (*n_kinds = 0).  Optional: ytm_fit loads a kernel on first use anyway. */
int ytm_load_train_kernels(ytm_model *m, int32_t kinds[4], int32_t *n_kinds);

/* encode: BaseTM.encode (src/cutm/base.py:224-263; kernel.cu:76-152 encode_batch).
 * X: uint32 (N, dim0*dim1*dim2), any value > 0 is a set pixel.  out: uint32 (N, P, W). */
int ytm_encode(ytm_model *m, const uint32_t *X, int64_t N, uint32_t *out);

/* encode of binned raw values in one pass, without the binned array: the transform of
 * Binarizer / ThermometerBinarizer (src/tm_utils/binarizer.py:9-22,63-86) followed by
 * BaseTM.encode (src/cutm/base.py:224-263; kernel.cu:76-152).  X holds N samples of
 * dim0*dim1*dim2 / width raw values of type x_dtype (YTM_DTYPE_*); value i of a sample
 * becomes the width levels (kind 0 thermometer: width = nthr; kind 1 one-hot: width =
 * nthr - 1 + 2 * edge_bins) at positions [i * width, (i + 1) * width) of the binned row,
 * as ytm_binarize lays them out, with the same thresholds and comparison types.  out: uint32
 * (N, P, W), equal to ytm_encode of the binned rows. */
int ytm_encode_binarized(ytm_model *m, const void *X, int x_dtype, int64_t N, const void *thresholds,
                         int int_thresholds, int nthr, int kind, int edge_bins, uint32_t *out);

/* Device-resident training / scoring data, so repeated epochs do not re-copy it.
 * encX: uint32 (N, P, W); encY: int32 (N, classes) or NULL for score-only data. */
int ytm_dataset_create(ytm_model *m, const uint32_t *encX, const int32_t *encY, int64_t N,
                       ytm_dataset **out);
void ytm_dataset_destroy(ytm_dataset *ds);

/* fit: BaseTM._fit's per-sample loop (src/cutm/base.py:266-359; kernel.cu pack_clauses
 * :155-204, fast_eval :255-282, select_active :285-316, clause_update :531-613).
 * Samples [first, first+count) of ds, in order.  drop: uint32 (clauses) clause drop mask
 * (base.py:288-293) or NULL for none.  inject: NULL for the counter-based stream, or a
 * float buffer of count sample blocks [sel C*P | q C*K | upd C*K | lit C*K*L] replacing
 * every draw (test mode).  Advances the model's step by count. */
int ytm_fit_dataset(ytm_model *m, const ytm_dataset *ds, int64_t first, int64_t count,
                    const uint32_t *drop, const float *inject);
/* Host-array convenience form of the same (copies encX/encY in, like base.py:275-279). */
int ytm_fit(ytm_model *m, const uint32_t *encX, const int32_t *encY, int64_t N,
            const uint32_t *drop, const float *inject);

/* score: BaseTM._score_batch (src/cutm/base.py:375-420; kernel.cu:319-343).
 * class_sums: float (N, classes) = bias + sum of weights of non-empty firing clauses. */
int ytm_score_dataset(ytm_model *m, const ytm_dataset *ds, float *class_sums);
/* ytm_score_dataset without any device allocation.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  d_class_sums is a DEVICE pointer to
 * float (N, classes), written with the same values ytm_score_dataset returns.  The
 * kernels' literal lists and int64 class-sum accumulators live in a static per-GPU scratch
 * array of YTM_NOALLOC_SCRATCH_BYTES (32 MiB; it is part of libytm's code object, so every
 * GPU on which the library's kernels are loaded holds it until the process ends, whether or
 * not this entry point is called there); samples go through in passes that fit it.  YTM_EINVAL when the model's
 * lists plus one sample's accumulators do not fit (e.g. one-patch models of more than
 * about 65000 wide clauses).  Calls on one GPU share the array, so overlapping calls
 * would race: the library serialises them per GPU with a lock.  Synchronous on return. */
#define YTM_NOALLOC_SCRATCH_BYTES (32u << 20)
int ytm_score_dataset_noalloc(ytm_model *m, const ytm_dataset *ds, float *d_class_sums);
int ytm_score(ytm_model *m, const uint32_t *encX, int64_t N, float *class_sums);

/* transform / transform_patchwise (src/cutm/base.py:465-542; kernel.cu:346-394).
 * mode 0: out uint32 (N, clauses), 1 where some patch fires;
 * mode 1: out uint32 (N, clauses, P), one value per patch;
 * mode 2: out uint32 (N, clauses, ceil(P/32)), the mode-1 values bit-packed: bit b of word j
 *         is patch 32j + b, bits beyond P are 0 (an option the reference does not have, for
 *         outputs of C*P*N values that would not fit as one uint32 each).
 * Empty clauses output 1.  Samples are processed in chunks, so device memory stays bounded
 * whatever N is. */
int ytm_transform(ytm_model *m, const uint32_t *encX, int64_t N, int mode, uint32_t *out);

/* State accessors (src/cutm/base.py:423-461, 561-593), flat C-order.
 * ta_state: uint32 (clauses, L); weights: float (clauses, classes);
 * patch_weights: int32 (clauses, P); bias: float (classes). */
int ytm_get_ta_state(ytm_model *m, uint32_t *out);
int ytm_set_ta_state(ytm_model *m, const uint32_t *in);
int ytm_get_weights(ytm_model *m, float *out);
int ytm_set_weights(ytm_model *m, const float *in);
int ytm_get_patch_weights(ytm_model *m, int32_t *out);
int ytm_set_patch_weights(ytm_model *m, const int32_t *in);
int ytm_get_bias(ytm_model *m, float *out);

/* ---- Host preprocessing: the binarizers of src/tm_utils/binarizer.py (no model needed).
 *
 * ytm_binarize replaces the transform of Binarizer (binarizer.py:63-86, 107-113) and the
 * binarize_gray / binarize_rgb of ThermometerBinarizer (binarizer.py:9-22): X holds n values
 * of type x_dtype (YTM_DTYPE_*), thresholds nthr values, int64 when int_thresholds else
 * double.  Comparisons are made in int64 when X and the thresholds are integers, else in
 * double (numpy's promotion for these operands).
 *   kind 0, thermometer: out uint32 (n, nthr), out[i][j] = X[i] >= t[j];
 *   kind 1, one-hot: out uint32 (n, nthr - 1 + 2 * edge_bins); the nthr - 1 intervals
 *           t[j] <= X[i] < t[j + 1], preceded by X[i] < t[0] and followed by
 *           X[i] >= t[nthr - 1] when edge_bins.
 * ytm_collapse_bins replaces Binarizer.collapse_bins (binarizer.py:88-129): B uint32
 * (rows, width) -> out int64 (rows): kind 0, the index of the last non-zero value + 1 (0 if
 * none); kind 1, the index of the first maximum; minus 1 when edge_bins. */
int ytm_binarize(const void *X, int x_dtype, int64_t n, const void *thresholds, int int_thresholds, int nthr,
                 int kind, int edge_bins, uint32_t *out);
int ytm_collapse_bins(const uint32_t *B, int64_t rows, int64_t width, int kind, int edge_bins, int64_t *out);

#ifdef __cplusplus
}
#endif

#endif /* YTM_H */
