/*
 * ytm_oracle.c -- CPU restatement of the YTM (Mayur1009/YTM) Tsetlin Machine hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP product path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product (ytm_amd) never links, loads or calls it.
 *
 * What it restates (only the *called* kernel variants of the reference):
 *   encode_batch ............ src/cutm/cuda/kernel.cu:76-152     -> orc_encode
 *   pack_clauses ............ src/cutm/cuda/kernel.cu:155-204    -> include_mask()
 *   clause_match ............ src/cutm/cuda/kernel.cu:207-216    -> clause_match()
 *   fast_eval ............... src/cutm/cuda/kernel.cu:255-282    -> orc_fit (step 2)
 *   select_active ........... src/cutm/cuda/kernel.cu:285-316    -> orc_fit (step 3)
 *   clip_cs / update_probability / clause_update
 *                             src/cutm/cuda/kernel.cu:397,508-613 -> orc_fit (step 4)
 *   type1a_fb/type1b_fb/type2_fb (vectorised, called variants)
 *                             src/cutm/cuda/kernel.cu:410-443,453-470,481-506
 *   calc_class_sums_infer_batch src/cutm/cuda/kernel.cu:319-343  -> orc_score
 *   transform / transform_patchwise kernel.cu:346-394            -> orc_transform
 *   init_weights ............ src/cutm/cuda/kernel.cu:46-73      -> orc_init_weights
 *   per-sample driver ....... src/cutm/base.py:305-357           -> orc_fit
 *
 * Deliberate, documented replacements of things that cannot be reproduced off the
 * reference's exact NVIDIA setup (cuRAND XORWOW per-thread streams whose consumption
 * order depends on the launch grid, --use_fast_math reciprocal, float-atomic order):
 *   - randomness: Philox4x32-10 (Salmon et al., SC'11) keyed by the model seed, one
 *     counter per draw site (see "Random stream" below), or an injected float buffer;
 *   - 1.0f/count in the reservoir is IEEE-correctly-rounded float division;
 *   - class sums are exact integer sums of the (integer-valued) clause weights,
 *     rounded once to float32.  Identical to the reference whenever its own float
 *     atomics are exact (all partial sums below 2^24 in magnitude).
 *
 * Pinning (tests/): Philox against the Random123 known-answer vectors; encode,
 * evaluation, voting and transform against pure-Python brute force on small shapes and
 * hand-built cases; training against an independent pure-Python restatement driven by
 * the same injected random stream, plus hand-traced single-sample feedback cases.
 *
 * Random stream (shared definition with the HIP product; both must agree bit for bit):
 *   key = (seed & 0xffffffff, seed >> 32)
 *   ctr = (x0, x1, x2, x3) = ((u32)t, (u32)c, (tag << 28) | ((t >> 32) & 0x0fffffff), site)
 *   where t = global training step (samples trained by this model so far) and c = clause.
 *   A 32-bit output word z gives the uniform u = ((z >> 8) + 1) * 2^-24, in (0, 1].
 *   tag 1 SEL : reservoir draw for the r-th firing patch (r >= 1): site = (r-1) >> 2,
 *               word (r-1) & 3.
 *   tag 2 CK  : per (clause, class k): site = k; word 0 = Q-skip draw, word 1 = update draw.
 *   tag 3 LIT : literal draws of (clause, class k, literal word w): 24 bit-planes in 6
 *               groups g, site = (k*W + w)*6 + g, word i is plane j = 23 - 4g - i;
 *               bit b of plane j is bit j of the 24-bit integer q of literal 32w+b, and
 *               u = (q + 1) * 2^-24.
 *   tag 4 INIT: weight init, t = 0, site = k; w = 1 - 2*(word0 & 1).
 *   Injected mode replaces every draw by a float from a caller buffer laid out per
 *   sample i of the fit call as [sel C*P | q C*K | upd C*K | lit C*K*L]:
 *     sel[c*P + r-1], q[c*K + k], upd[c*K + k], lit[(c*K + k)*L + l].
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef struct {
    int32_t clauses;            /* total clauses C (banks * clauses per bank) */
    int32_t classes;            /* K */
    int32_t dim0, dim1, dim2;   /* image width, height, channels */
    int32_t patch_dim0, patch_dim1;
    int32_t number_of_ta_states;
    int32_t max_included_literals; /* resolved: L when None */
    int32_t append_negated, encode_loc, coalesced, negative_polarity, init_neg_weights;
    int32_t thresh;             /* T */
    double s_inv;               /* S_INV as the reference types it, widened to double */
    double q_prob;              /* Q_PROB likewise */
    uint64_t seed;
} orc_params;

typedef struct {
    int64_t L, W, P, Lh, C, K;
} geom;

static geom geometry(const orc_params *p) {
    /* src/cutm/base.py:108-121 */
    geom g;
    int64_t base = (int64_t)p->patch_dim0 * p->patch_dim1 * p->dim2;
    if (p->encode_loc) base += (p->dim0 - p->patch_dim0) + (p->dim1 - p->patch_dim1);
    g.Lh = base;
    g.L = p->append_negated ? 2 * base : base;
    g.W = (g.L - 1) / 32 + 1;
    g.P = (int64_t)(p->dim0 - p->patch_dim0 + 1) * (p->dim1 - p->patch_dim1 + 1);
    g.C = p->clauses;
    g.K = p->classes;
    return g;
}

void orc_geometry(const orc_params *p, int64_t out[4]) {
    geom g = geometry(p);
    out[0] = g.L; out[1] = g.W; out[2] = g.P; out[3] = g.Lh;
}

static int n_threads = 1;
void orc_set_threads(int n) { n_threads = n > 0 ? n : 1; }

/* ---------------------------------------------------------------- Philox4x32-10 */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; ++r) {
        if (r) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1; c3 = (uint32_t)p0; c0 = n0; c2 = n2;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

enum { TAG_SEL = 1, TAG_CK = 2, TAG_LIT = 3, TAG_INIT = 4 };

static void site_words(uint64_t seed, uint64_t t, uint32_t c, uint32_t tag, uint32_t site,
                       uint32_t out[4]) {
    uint32_t ctr[4] = {(uint32_t)t, c, (tag << 28) | (uint32_t)((t >> 32) & 0x0fffffffu), site};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    orc_philox4x32_10(ctr, key, out);
}

float orc_uniform_from_word(uint32_t z) {
    return (float)((z >> 8) + 1u) * (1.0f / 16777216.0f);
}

/* The literal draw u of literal l for (t, c, k) in counter mode, straight from the
 * definition: all 24 bit-planes assembled into q. */
float orc_u_lit(const orc_params *p, uint64_t t, int32_t c, int32_t k, int64_t l) {
    geom g = geometry(p);
    int64_t w = l / 32, b = l % 32;
    uint32_t q = 0;
    for (int grp = 0; grp < 6; ++grp) {
        uint32_t z[4];
        site_words(p->seed, t, (uint32_t)c, TAG_LIT, (uint32_t)((k * g.W + w) * 6 + grp), z);
        for (int i = 0; i < 4; ++i) {
            int j = 23 - 4 * grp - i;
            q |= ((z[i] >> b) & 1u) << j;
        }
    }
    return (float)(q + 1u) * (1.0f / 16777216.0f);
}

/* ---------------------------------------------------------------- init_weights */
void orc_init_weights(const orc_params *p, float *w) {
    /* src/cutm/cuda/kernel.cu:46-73 (random bit replaced by the INIT site) */
    geom g = geometry(p);
    int64_t per_bank = g.C / (p->coalesced ? 1 : g.K);
    for (int64_t c = 0; c < g.C; ++c) {
        for (int64_t k = 0; k < g.K; ++k) {
            float v;
            if (p->coalesced) {
                v = 1.0f;
                if (p->init_neg_weights) {
                    uint32_t z[4];
                    site_words(p->seed, 0, (uint32_t)c, TAG_INIT, (uint32_t)k, z);
                    v = 1.0f - 2.0f * (float)(z[0] & 1u);
                }
            } else {
                if (k == c / per_bank) {
                    v = 1.0f;
                    if (p->init_neg_weights && (c % per_bank) >= (per_bank / 2)) v = -1.0f;
                } else {
                    v = 0.0f;
                }
            }
            w[c * g.K + k] = v;
        }
    }
}

/* ---------------------------------------------------------------- encode */
static inline void set_bit(uint32_t *words, int64_t bit) { words[bit >> 5] |= 1u << (bit & 31); }
static inline void clr_bit(uint32_t *words, int64_t bit) { words[bit >> 5] &= ~(1u << (bit & 31)); }

void orc_encode(const orc_params *p, const uint32_t *X, int64_t N, uint32_t *out) {
    /* src/cutm/cuda/kernel.cu:76-152, executed in the same statement order */
    geom g = geometry(p);
    const int64_t F = (int64_t)p->dim0 * p->dim1 * p->dim2;
    const int64_t half = g.L / 2;
    memset(out, 0, (size_t)(N * g.P * g.W) * sizeof(uint32_t));
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int64_t ep = 0; ep < N * g.P; ++ep) {
        int64_t e = ep / g.P, patch = ep % g.P;
        int64_t py = patch / (p->dim0 - p->patch_dim0 + 1);
        int64_t px = patch % (p->dim0 - p->patch_dim0 + 1);
        uint32_t *o = out + (e * g.P + patch) * g.W;
        if (p->append_negated)
            for (int64_t l = half; l < g.L; ++l) set_bit(o, l);
        for (int64_t l = 0; l < py; ++l) {
            set_bit(o, l);
            if (p->append_negated) clr_bit(o, l + half);
        }
        for (int64_t l = 0; l < px; ++l) {
            int64_t lit = (p->dim1 - p->patch_dim1) + l;
            set_bit(o, lit);
            if (p->append_negated) clr_bit(o, lit + half);
        }
        for (int64_t y = py; y < py + p->patch_dim1; ++y)
            for (int64_t x = px; x < px + p->patch_dim0; ++x)
                for (int64_t z = 0; z < p->dim2; ++z) {
                    if (X[e * F + y * ((int64_t)p->dim0 * p->dim2) + x * p->dim2 + z] > 0) {
                        int64_t ry = y - py, rx = x - px;
                        int64_t lit = ry * p->patch_dim0 * p->dim2 + rx * p->dim2 + z;
                        if (p->encode_loc) lit += (p->dim1 - p->patch_dim1) + (p->dim0 - p->patch_dim0);
                        set_bit(o, lit);
                        if (p->append_negated) clr_bit(o, lit + half);
                    }
                }
    }
}

/* ---------------------------------------------------------------- evaluation */
static int64_t include_mask(const orc_params *p, const geom *g, const uint32_t *ta_row, uint32_t *mask) {
    /* pack_clauses, src/cutm/cuda/kernel.cu:155-204: bit l = ta > HALF_STATE */
    const uint32_t half_state = (uint32_t)(p->number_of_ta_states / 2);
    int64_t n = 0;
    for (int64_t w = 0; w < g->W; ++w) mask[w] = 0;
    for (int64_t l = 0; l < g->L; ++l)
        if (ta_row[l] > half_state) { mask[l >> 5] |= 1u << (l & 31); ++n; }
    return n;
}

static int clause_match(const geom *g, const uint32_t *mask, const uint32_t *x) {
    /* src/cutm/cuda/kernel.cu:207-216 */
    const uint32_t filter = (g->L % 32) ? ~(0xFFFFFFFFu << (g->L % 32)) : 0xFFFFFFFFu;
    for (int64_t w = 0; w < g->W - 1; ++w)
        if ((mask[w] & x[w]) != mask[w]) return 0;
    if ((mask[g->W - 1] & (x[g->W - 1] & filter)) != (mask[g->W - 1] & filter)) return 0;
    return 1;
}

void orc_score(const orc_params *p, const uint32_t *ta, const float *w, const float *bias,
               const uint32_t *X, int64_t N, float *cs_out) {
    /* calc_class_sums_infer_batch, src/cutm/cuda/kernel.cu:319-343; class sums start at
     * the bias (src/cutm/base.py:390-403).  Empty clauses are skipped (kernel.cu:328). */
    geom g = geometry(p);
    uint32_t *masks = (uint32_t *)malloc((size_t)(g.C * g.W) * sizeof(uint32_t));
    int64_t *ninc = (int64_t *)malloc((size_t)g.C * sizeof(int64_t));
    for (int64_t c = 0; c < g.C; ++c) ninc[c] = include_mask(p, &g, ta + c * g.L, masks + c * g.W);
#pragma omp parallel for num_threads(n_threads) schedule(dynamic, 16)
    for (int64_t e = 0; e < N; ++e) {
        int64_t acc[256];
        int64_t *sum = g.K <= 256 ? acc : (int64_t *)malloc((size_t)g.K * sizeof(int64_t));
        for (int64_t k = 0; k < g.K; ++k) sum[k] = 0;
        for (int64_t c = 0; c < g.C; ++c) {
            if (ninc[c] == 0) continue;
            int fired = 0;
            for (int64_t pt = 0; pt < g.P && !fired; ++pt)
                fired = clause_match(&g, masks + c * g.W, X + (e * g.P + pt) * g.W);
            if (fired)
                for (int64_t k = 0; k < g.K; ++k) sum[k] += (int64_t)w[c * g.K + k];
        }
        for (int64_t k = 0; k < g.K; ++k) cs_out[e * g.K + k] = (float)(sum[k] + (int64_t)bias[k]);
        if (sum != acc) free(sum);
    }
    free(masks);
    free(ninc);
}

void orc_transform(const orc_params *p, const uint32_t *ta, const uint32_t *X, int64_t N,
                   int patchwise, uint32_t *out) {
    /* transform / transform_patchwise, src/cutm/cuda/kernel.cu:346-394 */
    geom g = geometry(p);
    uint32_t *masks = (uint32_t *)malloc((size_t)(g.C * g.W) * sizeof(uint32_t));
    int64_t *ninc = (int64_t *)malloc((size_t)g.C * sizeof(int64_t));
    for (int64_t c = 0; c < g.C; ++c) ninc[c] = include_mask(p, &g, ta + c * g.L, masks + c * g.W);
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int64_t e = 0; e < N; ++e) {
        for (int64_t c = 0; c < g.C; ++c) {
            if (!patchwise) {
                uint32_t v = 1;
                if (ninc[c] != 0) {
                    v = 0;
                    for (int64_t pt = 0; pt < g.P && !v; ++pt)
                        v = (uint32_t)clause_match(&g, masks + c * g.W, X + (e * g.P + pt) * g.W);
                }
                out[e * g.C + c] = v;
            } else {
                for (int64_t pt = 0; pt < g.P; ++pt)
                    out[(e * g.C + c) * g.P + pt] =
                        ninc[c] == 0 ? 1u : (uint32_t)clause_match(&g, masks + c * g.W, X + (e * g.P + pt) * g.W);
            }
        }
    }
    free(masks);
    free(ninc);
}

/* ---------------------------------------------------------------- training */
typedef struct {
    const orc_params *p;
    geom g;
    uint64_t t;           /* global step of this sample */
    const float *inj;     /* injected block of this sample, or NULL */
} draws;

static float draw_sel(const draws *d, int64_t c, int64_t r) {
    if (d->inj) return d->inj[c * d->g.P + (r - 1)];
    uint32_t z[4];
    site_words(d->p->seed, d->t, (uint32_t)c, TAG_SEL, (uint32_t)((r - 1) >> 2), z);
    return orc_uniform_from_word(z[(r - 1) & 3]);
}

static float draw_ck(const draws *d, int64_t c, int64_t k, int which) {
    if (d->inj) return d->inj[d->g.C * d->g.P + which * d->g.C * d->g.K + c * d->g.K + k];
    uint32_t z[4];
    site_words(d->p->seed, d->t, (uint32_t)c, TAG_CK, (uint32_t)k, z);
    return orc_uniform_from_word(z[which]);
}

/* Literal draws: u of every literal of one (clause, class) update.  In counter mode the
 * 24 planes of each literal word are generated once per word and reused for its 32
 * literals; the resulting u is exactly orc_u_lit(). */
typedef struct {
    const draws *d;
    int64_t c, k;
    int64_t cached_word;
    uint32_t planes[24];
} lit_draws;

static float draw_lit(lit_draws *ld, int64_t l) {
    const draws *d = ld->d;
    if (d->inj) return d->inj[d->g.C * d->g.P + 2 * d->g.C * d->g.K + (ld->c * d->g.K + ld->k) * d->g.L + l];
    int64_t w = l >> 5;
    if (ld->cached_word != w) {
        for (int grp = 0; grp < 6; ++grp) {
            uint32_t z[4];
            site_words(d->p->seed, d->t, (uint32_t)ld->c, TAG_LIT,
                       (uint32_t)((ld->k * d->g.W + w) * 6 + grp), z);
            for (int i = 0; i < 4; ++i) ld->planes[23 - 4 * grp - i] = z[i];
        }
        ld->cached_word = w;
    }
    uint32_t q = 0;
    for (int j = 0; j < 24; ++j) q |= ((ld->planes[j] >> (l & 31)) & 1u) << j;
    return (float)(q + 1u) * (1.0f / 16777216.0f);
}

static inline uint32_t lit_bit(const uint32_t *patch, int64_t l) { return (patch[l >> 5] >> (l & 31)) & 1u; }

static void type1a_fb(const orc_params *p, const geom *g, lit_draws *ld, uint32_t *ta, const uint32_t *patch) {
    /* src/cutm/cuda/kernel.cu:410-443: increment included-candidate literals that are 1
     * (saturating at MAX_TA_STATE), decrement literals that are 0 with probability 1/s. */
    const uint32_t max_state = (uint32_t)p->number_of_ta_states;
    for (int64_t l = 0; l < g->L; ++l) {
        uint32_t bit = lit_bit(patch, l);
        if (bit == 1 && ta[l] < max_state) {
            ta[l] += 1;
        } else if (bit == 0 && ta[l] > 0 && (double)draw_lit(ld, l) <= p->s_inv) {
            ta[l] -= 1;
        }
    }
}

static void type1b_fb(const orc_params *p, const geom *g, lit_draws *ld, uint32_t *ta) {
    /* src/cutm/cuda/kernel.cu:453-470 */
    for (int64_t l = 0; l < g->L; ++l)
        if (ta[l] > 0 && (double)draw_lit(ld, l) <= p->s_inv) ta[l] -= 1;
}

static void type2_fb(const geom *g, uint32_t *ta, const uint32_t *patch) {
    /* src/cutm/cuda/kernel.cu:481-506 (the called variant: no upper guard) */
    for (int64_t l = 0; l < g->L; ++l)
        if (lit_bit(patch, l) == 0) ta[l] += 1;
}

/*
 * One fit() call over N samples (src/cutm/base.py:266-359).  State arrays are updated in
 * place: ta (C*L uint32), w (C*K float), pw (C*P int32).  bias is the K-vector the class
 * sums start from (base.py:327).  drop is the clause drop mask (base.py:288-293).
 * step0 is the model's global step before this call.  inject is NULL (counter stream) or
 * N sample blocks of the injected layout.  *updated_out accumulates the number of
 * (sample, clause) pairs that executed a Type Ia, Ib or II branch; *feedback_out (when
 * not NULL) the samples at which some class has an update probability above zero
 * (kernel.cu:508-529): only those can change a weight or a TA state, since every update
 * needs its draw u in (0, 1] at or below that probability (kernel.cu:573-575).
 */
void orc_fit(const orc_params *p, uint32_t *ta, float *w, int32_t *pw, const float *bias,
             const uint32_t *X, const int32_t *Y, int64_t N, const uint32_t *drop,
             uint64_t step0, const float *inject, uint64_t *updated_out, uint64_t *feedback_out) {
    geom g = geometry(p);
    const int64_t C = g.C, K = g.K, W = g.W, P = g.P, L = g.L;
    const int64_t per_bank = C / (p->coalesced ? 1 : K);
    const int64_t block = C * P + 2 * C * K + C * K * L;
    uint32_t *masks = (uint32_t *)malloc((size_t)(C * W) * sizeof(uint32_t));
    int64_t *ninc = (int64_t *)malloc((size_t)C * sizeof(int64_t));
    int64_t *sel = (int64_t *)malloc((size_t)C * sizeof(int64_t));
    int64_t *cs_int = (int64_t *)malloc((size_t)K * sizeof(int64_t));
    float *clipped = (float *)malloc((size_t)K * sizeof(float));
    int *target = (int *)malloc((size_t)K * sizeof(int));
    double *prob = (double *)malloc((size_t)K * sizeof(double));
    uint64_t updated = 0, feedback = 0;
    const float T = (float)p->thresh;

    for (int64_t e = 0; e < N; ++e) {
        draws d = {p, g, step0 + (uint64_t)e, inject ? inject + e * block : NULL};
        const uint32_t *x = X + e * P * W;
        const int32_t *y = Y + e * K;

        /* 1. pack_clauses (base.py:307-313) */
#pragma omp parallel for num_threads(n_threads) schedule(static)
        for (int64_t c = 0; c < C; ++c) ninc[c] = include_mask(p, &g, ta + c * L, masks + c * W);

        /* 2+3. fast_eval (kernel.cu:255-282) and select_active (kernel.cu:285-316):
         * reservoir over firing patches in increasing p; the r-th firing patch replaces
         * the selection when its draw is below 1/r. */
        for (int64_t k = 0; k < K; ++k) cs_int[k] = (int64_t)bias[k];
#pragma omp parallel num_threads(n_threads)
        {
            int64_t local[256];
            int64_t *part = K <= 256 ? local : (int64_t *)malloc((size_t)K * sizeof(int64_t));
            for (int64_t k = 0; k < K; ++k) part[k] = 0;
#pragma omp for schedule(static)
            for (int64_t c = 0; c < C; ++c) {
                int64_t count = 0, chosen = -1;
                if (drop[c] != 1) {
                    for (int64_t pt = 0; pt < P; ++pt) {
                        int out = ninc[c] == 0 ? 1 : clause_match(&g, masks + c * W, x + pt * W);
                        if (out) {
                            count++;
                            if (draw_sel(&d, c, count) < 1.0f / (float)count) chosen = pt;
                        }
                    }
                }
                sel[c] = chosen;
                if (chosen != -1) {
                    pw[c * P + chosen]++;
                    if (p->coalesced) {
                        for (int64_t k = 0; k < K; ++k) part[k] += (int64_t)w[c * K + k];
                    } else {
                        int64_t k = c / per_bank;
                        part[k] += (int64_t)w[c * K + k];
                    }
                }
            }
#pragma omp critical
            for (int64_t k = 0; k < K; ++k) cs_int[k] += part[k];
            if (part != local) free(part);
        }

        /* 4. clause_update (kernel.cu:531-613) */
        for (int64_t k = 0; k < K; ++k) {
            float cs = (float)cs_int[k];
            float v = (cs > T) ? T : ((cs < -T) ? -T : cs);           /* clip_cs, :397 */
            clipped[k] = v;
            target[k] = 1 - 2 * (v > (float)y[k]);                    /* :546,571 */
            prob[k] = ((double)y[k] - (double)v) / (2 * (double)y[k]); /* :508-529 */
        }
        for (int64_t k = 0; k < K; ++k) {
            if (prob[k] > 0.0) { feedback++; break; }
        }
        uint64_t upd_count = 0;
#pragma omp parallel for num_threads(n_threads) schedule(dynamic, 4) reduction(+ : upd_count)
        for (int64_t c = 0; c < C; ++c) {
            if (drop[c] == 1) continue;
            uint32_t *row = ta + c * L;
            const int clause_output = sel[c] > -1 ? 1 : 0;
            const uint32_t *patch = clause_output ? x + sel[c] * W : NULL;
            int64_t k_begin = 0, k_end = K;
            if (!p->coalesced) { k_begin = c / per_bank; k_end = k_begin + 1; }
            int touched = 0;
            for (int64_t k = k_begin; k < k_end; ++k) {
                if (target[k] == -1 && (double)draw_ck(&d, c, k, 0) > p->q_prob) continue;
                float *wp = &w[c * K + k];
                int sign = (*wp >= 0) - (*wp < 0);
                int should_update = (double)draw_ck(&d, c, k, 1) <= prob[k];
                int small = clause_output && ninc[c] <= p->max_included_literals;
                int type1a = (target[k] * sign) > 0 && small;
                int type1b = (target[k] * sign) > 0 && !small;
                int type2 = (target[k] * sign) < 0 && clause_output;
                if (!should_update) continue;
                lit_draws ld = {&d, c, k, -1, {0}};
                if (type1a) {
                    *wp += (float)sign * 1.0f;
                    type1a_fb(p, &g, &ld, row, patch);
                    touched = 1;
                } else if (type1b) {
                    type1b_fb(p, &g, &ld, row);
                    touched = 1;
                } else if (type2) {
                    *wp -= (float)sign * 1.0f;
                    if (!p->negative_polarity && *wp < 1) *wp = 1;
                    type2_fb(&g, row, patch);
                    touched = 1;
                }
            }
            upd_count += (uint64_t)touched;
        }
        updated += upd_count;
    }
    if (updated_out) *updated_out += updated;
    if (feedback_out) *feedback_out += feedback;
    free(masks); free(ninc); free(sel); free(cs_int); free(clipped); free(target); free(prob);
}
