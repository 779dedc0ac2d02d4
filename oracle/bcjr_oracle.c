/*
 * CPU oracle for the BCJR forward-backward path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only to check results against (or as the timed CPU baseline).  The
 * product path (quant-2bit_amd/) never links or calls it.
 *
 * It restates, in plain C, the algorithm of the reference's eager BCJR node and
 * its T->0 Viterbi mode:
 *   - codebook generators      src/codes/ref.py:33-41 (1MAD), :76-91 (3INST),
 *                              src/qat/ste.py:376-392 (HYB table build)
 *   - trellis structure        src/bcjr/forward_backward.py:62-86 (preds/succs)
 *   - emission                 src/bcjr/forward_backward.py:89-103
 *   - alpha / beta recursions  src/bcjr/forward_backward.py:106-187
 *   - logZ, marginals, soft    src/bcjr/forward_backward.py:219-228
 *   - gradient wrt sequences   src/bcjr/bcjr_monolithic.py:192-243 (analytic
 *                              form of the eager autograd backward)
 *   - Viterbi (direct form)    src/viterbi/encode.py:250-307 (viterbi_encode_v)
 *   - decode / walk replay     src/viterbi/encode.py:310-325, src/qat/ste.py:270-283
 *
 * The BCJR recursions run in double precision on the reduced bitshift state:
 * every destination state s shares its predecessor set with all states of the
 * same s >> kV, so alpha_t(s) = ll_t(s) + m_{t-1}(s >> kV) with
 * m_{t-1}(j) = LSE_p alpha_{t-1}(p * 2^(L-kV) + j); likewise
 * beta_t(s) = n_t(s mod 2^(L-kV)).  This is the same function as the
 * reference's gather-over-predecessors form (forward_backward.py:110-111,117-119),
 * evaluated without the redundant 2^kV-fold gather.
 *
 * The gradient uses the first-order expectation semiring: with
 * F = sum_t g_t . c(s_t) (+ g_Z * logZ), dL/dll_t(s) = P_t(s) (E[F|s_t=s] - E[F]),
 * where E[F|s_t=s] = phi_t(s) + psi_t(s) is carried by a forward recursion (phi,
 * reduced to mu) and a backward recursion (psi, reduced to nu) that reuse the
 * alpha/beta softmax weights.  d seq_t[v] = (2/T) sum_s dll_t(s) (c_v(s) - w_t[v]),
 * as in bcjr_monolithic.py:228-239.
 *
 * The Viterbi restatement runs in float32 with the reference numpy encoder's
 * exact operation order: local = sum_v fl((c_v - w_v)^2) without FMA contraction,
 * cum = min_p + local, lowest p wins a tie, lowest final state wins a tie.
 * Build with -ffp-contract=off (see oracle/Makefile).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_OK 0
#define ORACLE_EINVAL (-1)
#define ORACLE_ENOMEM (-2)

/* ------------------------------------------------------------------------- */
/* Codebook generators                                                        */
/* ------------------------------------------------------------------------- */

/* IEEE binary16 -> float, exact (normal, subnormal, inf/nan). */
static float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t exp = (uint32_t)(h >> 10) & 0x1Fu;
    uint32_t man = (uint32_t)h & 0x3FFu;
    float v;
    if (exp == 0) {
        v = ldexpf((float)man, -24);
    } else if (exp == 31) {
        v = man ? NAN : INFINITY;
    } else {
        v = ldexpf((float)(man | 0x400u), (int)exp - 25);
    }
    return sign ? -v : v;
}

/* src/codes/ref.py:33-41: LCG x = 34038481*s + 76625530 (mod 2^32), sum of the
 * four bytes, ((sum - 510) / 147.8) in float32. */
float oracle_code_1mad(uint32_t s) {
    uint32_t x = 34038481u * s + 76625530u;
    float b0 = (float)(x & 0xFFu), b1 = (float)((x >> 8) & 0xFFu);
    float b2 = (float)((x >> 16) & 0xFFu), b3 = (float)((x >> 24) & 0xFFu);
    float sum = ((b0 + b1) + b2) + b3;
    volatile float num = sum - 510.0f;
    volatile float den = 147.8f;
    return num / den;
}

/* src/codes/ref.py:76-91: LCG x = 89226354*s + 64248484, y = (x & 0x8FFF8FFF) ^
 * packed fp16(0.922), sum of the two fp16 halves, times float32(1/1.2447). */
float oracle_code_3inst(uint32_t s) {
    const uint32_t m_packed = 0x3B603B60u; /* fp16(0.922) = 0x3B60 in both halves */
    uint32_t x = 89226354u * s + 64248484u;
    uint32_t y = (x & 0x8FFF8FFFu) ^ m_packed;
    float lo = half_to_float((uint16_t)(y & 0xFFFFu));
    float hi = half_to_float((uint16_t)(y >> 16));
    volatile float sum = lo + hi;
    const float scale = (float)(1.0 / 1.2447);
    return sum * scale;
}

/* src/qat/ste.py:376-392 (and src/codes/ref.py:116-127): Klimov-Shamir
 * x = s*s + s, idx = (x >> (15-Q)) & (2^Q-1), second component negated when
 * bit 15 of x is set.  lut is (2^Q, 2) row-major. */
void oracle_code_hyb(uint32_t s, const float* lut, int Q, float* out2) {
    uint32_t x = s * s + s;
    uint32_t idx = (x >> (15 - Q)) & ((1u << Q) - 1u);
    out2[0] = lut[2 * idx + 0];
    out2[1] = (x & (1u << 15)) ? -lut[2 * idx + 1] : lut[2 * idx + 1];
}

/* Fill a (2^L, V) codebook.  code: 1=1MAD (V=1), 2=3INST (V=1), 3=HYB (V=2). */
int oracle_codebook(int code, int L, const float* lut, int Q, float* out) {
    if (L < 1 || L > 24) return ORACLE_EINVAL;
    uint32_t S = 1u << L;
    for (uint32_t s = 0; s < S; ++s) {
        if (code == 1) out[s] = oracle_code_1mad(s);
        else if (code == 2) out[s] = oracle_code_3inst(s);
        else if (code == 3) {
            if (!lut) return ORACLE_EINVAL;
            oracle_code_hyb(s, lut, Q, out + 2 * (size_t)s);
        } else return ORACLE_EINVAL;
    }
    return ORACLE_OK;
}

/* ------------------------------------------------------------------------- */
/* BCJR (double precision, natural-log domain)                                */
/* ------------------------------------------------------------------------- */

typedef struct {
    int L, KV, V, N;
    int64_t S, NT, R;
} trellis_t;

static int trellis_init(trellis_t* tr, int L, int KV, int V, int N) {
    if (L < 1 || L > 20 || KV < 1 || KV > L || V < 1 || V > 4 || N < 1) return ORACLE_EINVAL;
    tr->L = L; tr->KV = KV; tr->V = V; tr->N = N;
    tr->S = (int64_t)1 << L;
    tr->NT = (int64_t)1 << (L - KV);
    tr->R = (int64_t)1 << KV;
    return ORACLE_OK;
}

/* ll_t(s) for all s: -||c(s) - w_t||^2 / T (forward_backward.py:89-103). */
static void emission(const trellis_t* tr, const float* cb, const float* w, double invT, double* ll) {
    for (int64_t s = 0; s < tr->S; ++s) {
        double e = 0.0;
        for (int v = 0; v < tr->V; ++v) {
            double d = (double)cb[s * tr->V + v] - (double)w[v];
            e += d * d;
        }
        ll[s] = -e * invT;
    }
}

/* alpha sweep: writes m_t (t = 0..N-1) into m_all (N x NT); optional mu. */
static void alpha_sweep(const trellis_t* tr, const float* cb, const float* seq, double invT,
                        const double* f_all /* N x S or NULL */, double* m_all, double* mu_all,
                        double* ll, double* a) {
    const int64_t S = tr->S, NT = tr->NT, R = tr->R;
    const int KV = tr->KV;
    for (int t = 0; t < tr->N; ++t) {
        emission(tr, cb, seq + (size_t)t * tr->V, invT, ll);
        const double* mprev = t ? m_all + (size_t)(t - 1) * NT : NULL;
        const double* muprev = (t && mu_all) ? mu_all + (size_t)(t - 1) * NT : NULL;
        for (int64_t s = 0; s < S; ++s) {
            double mp = mprev ? mprev[s >> KV] : log((double)R); /* alpha_{-1} = 0 */
            a[s] = ll[s] + mp;
        }
        double* mcur = m_all + (size_t)t * NT;
        double* mucur = mu_all ? mu_all + (size_t)t * NT : NULL;
        for (int64_t j = 0; j < NT; ++j) {
            double mx = -INFINITY;
            for (int64_t p = 0; p < R; ++p) mx = fmax(mx, a[p * NT + j]);
            double sum = 0.0, acc = 0.0;
            for (int64_t p = 0; p < R; ++p) {
                int64_t s = p * NT + j;
                double e = exp(a[s] - mx);
                sum += e;
                if (mucur) {
                    double phi = f_all[(size_t)t * S + s] + (muprev ? muprev[s >> KV] : 0.0);
                    acc += e * phi;
                }
            }
            mcur[j] = mx + log(sum);
            if (mucur) mucur[j] = acc / sum;
        }
    }
}

static double lse_array(const double* x, int64_t n) {
    double mx = -INFINITY;
    for (int64_t i = 0; i < n; ++i) mx = fmax(mx, x[i]);
    double sum = 0.0;
    for (int64_t i = 0; i < n; ++i) sum += exp(x[i] - mx);
    return mx + log(sum);
}

typedef struct {
    double *ll, *a, *y, *m_all, *mu_all, *n_cur, *n_nxt, *nu_cur, *nu_nxt, *f_all;
} work_t;

static void work_free(work_t* w) {
    free(w->ll); free(w->a); free(w->y); free(w->m_all); free(w->mu_all);
    free(w->n_cur); free(w->n_nxt); free(w->nu_cur); free(w->nu_nxt); free(w->f_all);
    memset(w, 0, sizeof(*w));
}

static int work_alloc(work_t* w, const trellis_t* tr, int grad) {
    memset(w, 0, sizeof(*w));
    size_t S = (size_t)tr->S, NT = (size_t)tr->NT, N = (size_t)tr->N;
    w->ll = malloc(S * sizeof(double));
    w->a = malloc(S * sizeof(double));
    w->y = malloc(S * sizeof(double));
    w->m_all = malloc(N * NT * sizeof(double));
    w->n_cur = malloc(NT * sizeof(double));
    w->n_nxt = malloc(NT * sizeof(double));
    int ok = w->ll && w->a && w->y && w->m_all && w->n_cur && w->n_nxt;
    if (grad) {
        w->mu_all = malloc(N * NT * sizeof(double));
        w->nu_cur = malloc(NT * sizeof(double));
        w->nu_nxt = malloc(NT * sizeof(double));
        w->f_all = malloc(N * S * sizeof(double));
        ok = ok && w->mu_all && w->nu_cur && w->nu_nxt && w->f_all;
    }
    if (!ok) { work_free(w); return ORACLE_ENOMEM; }
    return ORACLE_OK;
}

/* One sequence, forward: soft (N x V), logZ and, when H is non-NULL, the
 * marginal entropy H_t = -sum_s P_t(s) ln P_t(s) (N) -- what entropy_diagnostic
 * (src/bcjr/anneal.py:175-179) reduces from P. */
static void fwd_one(const trellis_t* tr, const float* cb, const float* seq, double T,
                    float* soft, float* logZ_out, float* H, work_t* w) {
    const int64_t S = tr->S, NT = tr->NT, R = tr->R;
    const int KV = tr->KV, V = tr->V, N = tr->N;
    const double invT = 1.0 / T;
    alpha_sweep(tr, cb, seq, invT, NULL, w->m_all, NULL, w->ll, w->a);
    const double logZ = lse_array(w->m_all + (size_t)(N - 1) * NT, NT);
    *logZ_out = (float)logZ;
    for (int64_t j = 0; j < NT; ++j) w->n_cur[j] = 0.0; /* beta_{N-1} = 0 */
    for (int t = N - 1; t >= 0; --t) {
        emission(tr, cb, seq + (size_t)t * V, invT, w->ll);
        const double* mprev = t ? w->m_all + (size_t)(t - 1) * NT : NULL;
        double acc[4] = {0, 0, 0, 0}, h = 0.0;
        for (int64_t s = 0; s < S; ++s) {
            w->y[s] = w->ll[s] + w->n_cur[s & (NT - 1)];
            double mp = mprev ? mprev[s >> KV] : log((double)R);
            const double lp = w->y[s] + mp - logZ;
            double P = exp(lp);
            for (int v = 0; v < V; ++v) acc[v] += P * (double)cb[s * V + v];
            if (P > 0.0) h -= P * lp;
        }
        for (int v = 0; v < V; ++v) soft[(size_t)t * V + v] = (float)acc[v];
        if (H) H[t] = (float)h;
        for (int64_t u = 0; u < NT; ++u) w->n_nxt[u] = lse_array(w->y + u * R, R);
        double* tmp = w->n_cur; w->n_cur = w->n_nxt; w->n_nxt = tmp;
    }
}

/* One sequence, backward: d_seq (N x V) from g_soft (N x V) and g_Z. */
static void bwd_one(const trellis_t* tr, const float* cb, const float* seq, double T,
                    const float* g, double gZ, float* dseq, float* logZ_out, work_t* w) {
    const int64_t S = tr->S, NT = tr->NT, R = tr->R;
    const int KV = tr->KV, V = tr->V, N = tr->N;
    const double invT = 1.0 / T;
    for (int t = 0; t < N; ++t)
        for (int64_t s = 0; s < S; ++s) {
            double f = 0.0;
            for (int v = 0; v < V; ++v) f += (double)g[(size_t)t * V + v] * (double)cb[s * V + v];
            w->f_all[(size_t)t * S + s] = f;
        }
    alpha_sweep(tr, cb, seq, invT, w->f_all, w->m_all, w->mu_all, w->ll, w->a);
    const double* mlast = w->m_all + (size_t)(N - 1) * NT;
    const double* mulast = w->mu_all + (size_t)(N - 1) * NT;
    const double logZ = lse_array(mlast, NT);
    if (logZ_out) *logZ_out = (float)logZ;
    double EF = 0.0;
    for (int64_t j = 0; j < NT; ++j) EF += exp(mlast[j] - logZ) * mulast[j];
    for (int64_t j = 0; j < NT; ++j) { w->n_cur[j] = 0.0; w->nu_cur[j] = 0.0; }
    for (int t = N - 1; t >= 0; --t) {
        const float* wt = seq + (size_t)t * V;
        emission(tr, cb, wt, invT, w->ll);
        const double* mprev = t ? w->m_all + (size_t)(t - 1) * NT : NULL;
        const double* muprev = t ? w->mu_all + (size_t)(t - 1) * NT : NULL;
        const double* f = w->f_all + (size_t)t * S;
        double A0 = 0.0, A1[4] = {0, 0, 0, 0};
        for (int64_t s = 0; s < S; ++s) {
            w->y[s] = w->ll[s] + w->n_cur[s & (NT - 1)];
            double mp = mprev ? mprev[s >> KV] : log((double)R);
            double P = exp(w->y[s] + mp - logZ);
            double phi = f[s] + (muprev ? muprev[s >> KV] : 0.0);
            double psi = w->nu_cur[s & (NT - 1)];
            double dll = P * (phi + psi - EF + gZ);
            A0 += dll;
            for (int v = 0; v < V; ++v) A1[v] += dll * (double)cb[s * V + v];
        }
        for (int v = 0; v < V; ++v)
            dseq[(size_t)t * V + v] = (float)(2.0 * invT * (A1[v] - (double)wt[v] * A0));
        for (int64_t u = 0; u < NT; ++u) {
            const double* yy = w->y + u * R;
            double mx = -INFINITY;
            for (int64_t c = 0; c < R; ++c) mx = fmax(mx, yy[c]);
            double sum = 0.0, acc = 0.0;
            for (int64_t c = 0; c < R; ++c) {
                int64_t s = u * R + c;
                double e = exp(yy[c] - mx);
                sum += e;
                acc += e * (f[s] + w->nu_cur[s & (NT - 1)]);
            }
            w->n_nxt[u] = mx + log(sum);
            w->nu_nxt[u] = acc / sum;
        }
        double* tmp = w->n_cur; w->n_cur = w->n_nxt; w->n_nxt = tmp;
        tmp = w->nu_cur; w->nu_cur = w->nu_nxt; w->nu_nxt = tmp;
    }
}

static int set_threads(int nthreads) {
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
    return omp_get_max_threads();
#else
    (void)nthreads;
    return 1;
#endif
}

int oracle_num_threads(int nthreads) { return set_threads(nthreads); }

/* seq: (B, N, V); T: per-sequence (t_per_seq) or scalar; cb: (2^L, V). */
/* H: (B, N) marginal entropies in nats, or NULL. */
int oracle_bcjr_forward(int L, int KV, int V, int64_t B, int N, const float* seq, const float* T,
                        int t_per_seq, const float* cb, float* soft, float* logZ, float* H, int nthreads) {
    trellis_t tr;
    if (trellis_init(&tr, L, KV, V, N) || B < 0) return ORACLE_EINVAL;
    set_threads(nthreads);
    int err = ORACLE_OK;
#pragma omp parallel
    {
        work_t w;
        int e = work_alloc(&w, &tr, 0);
        if (e) {
#pragma omp atomic write
            err = e;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (int64_t b = 0; b < B; ++b) {
                double Tb = (double)(t_per_seq ? T[b] : T[0]);
                fwd_one(&tr, cb, seq + (size_t)b * N * V, Tb, soft + (size_t)b * N * V, logZ + b,
                        H ? H + (size_t)b * N : NULL, &w);
            }
            work_free(&w);
        }
    }
    return err;
}

int oracle_bcjr_backward(int L, int KV, int V, int64_t B, int N, const float* seq, const float* T,
                         int t_per_seq, const float* cb, const float* g_soft, const float* g_logZ,
                         float* d_seq, int nthreads) {
    trellis_t tr;
    if (trellis_init(&tr, L, KV, V, N) || B < 0) return ORACLE_EINVAL;
    set_threads(nthreads);
    int err = ORACLE_OK;
#pragma omp parallel
    {
        work_t w;
        int e = work_alloc(&w, &tr, 1);
        if (e) {
#pragma omp atomic write
            err = e;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (int64_t b = 0; b < B; ++b) {
                double Tb = (double)(t_per_seq ? T[b] : T[0]);
                double gZ = g_logZ ? (double)g_logZ[b] : 0.0;
                bwd_one(&tr, cb, seq + (size_t)b * N * V, Tb, g_soft + (size_t)b * N * V, gZ,
                        d_seq + (size_t)b * N * V, NULL, &w);
            }
            work_free(&w);
        }
    }
    return err;
}

/* ------------------------------------------------------------------------- */
/* Viterbi (float32, direct form; src/viterbi/encode.py:250-307)              */
/* ------------------------------------------------------------------------- */

/* One sequence.  With cons != 0, the constraint of viterbi_encode_constrained_v
 * (src/viterbi/encode.py:328-389): cum_0 of a state whose top ob bits differ
 * from ov becomes INF (:350-352, :364-365), the final argmin runs over states
 * whose bottom ob bits equal ov (:367-371), and a best cost >= INF/2 (the
 * reference raises, :372-375) is reported as start = -1. */
static int viterbi_one(const trellis_t* tr, const float* cb, const float* seq, int32_t* walk,
                       int32_t* bitstream, int32_t* start, float* recon, float* mse,
                       float* cum, float* ncum, uint8_t* bp /* N x NT */, int cons, int ob,
                       uint32_t ov_raw) {
    const int64_t S = tr->S, NT = tr->NT, R = tr->R;
    const int KV = tr->KV, V = tr->V, N = tr->N, L = tr->L;
    const float INF = 1e18f;
    const uint32_t omask = (1u << ob) - 1u;
    const uint32_t top_mask = omask << (L - ob), target_top = (ov_raw & omask) << (L - ob);
    const uint32_t target_bottom = ov_raw & omask;
    for (int64_t s = 0; s < S; ++s) cum[s] = 0.0f;
    for (int t = 0; t < N; ++t) {
        const float* w = seq + (size_t)t * V;
        uint8_t* bpt = bp + (size_t)t * NT;
        for (int64_t j = 0; j < NT; ++j) {
            float best = cum[j];
            int bi = 0;
            for (int64_t p = 1; p < R; ++p) {
                float v = cum[p * NT + j];
                if (v < best) { best = v; bi = (int)p; }
            }
            bpt[j] = (uint8_t)bi;
            /* every state whose predecessor group is j: s = R*j + c */
            for (int64_t c = 0; c < R; ++c) {
                int64_t s = j * R + c;
                float local = 0.0f;
                for (int v = 0; v < V; ++v) {
                    float d = cb[s * V + v] - w[v];
                    local = local + d * d;
                }
                ncum[s] = best + local;
            }
        }
        if (cons && t == 0)
            for (int64_t s = 0; s < S; ++s)
                if (((uint32_t)s & top_mask) != target_top) ncum[s] = INF;
        memcpy(cum, ncum, (size_t)S * sizeof(float));
    }
    if (cons)
        for (int64_t s = 0; s < S; ++s)
            if (((uint32_t)s & omask) != target_bottom) cum[s] = INF;
    int64_t fs = 0;
    for (int64_t s = 1; s < S; ++s)
        if (cum[s] < cum[fs]) fs = s;
    const int infeasible = cons && cum[fs] >= INF / 2;
    int64_t s = fs;
    walk[N - 1] = (int32_t)s;
    for (int t = N - 1; t > 0; --t) {
        int64_t j = s >> KV;
        s = (int64_t)bp[(size_t)t * NT + j] * NT + j;
        walk[t - 1] = (int32_t)s;
    }
    *start = infeasible ? -1 : (int32_t)((int64_t)bp[s >> KV] * NT + (s >> KV));
    double se = 0.0;
    for (int t = 0; t < N; ++t) {
        bitstream[t] = walk[t] & (int32_t)(R - 1);
        for (int v = 0; v < V; ++v) {
            float r = cb[(size_t)walk[t] * V + v];
            recon[(size_t)t * V + v] = r;
            double d = (double)r - (double)seq[(size_t)t * V + v];
            se += d * d;
        }
    }
    *mse = (float)(se / (double)(N * V));
    return ORACLE_OK;
}

/* overlap: (B,) or NULL (unconstrained); overlap_bits in [0, L]. */
int oracle_viterbi(int L, int KV, int V, int64_t B, int N, const float* seq, const float* cb,
                   int32_t* walk, int32_t* bitstream, int32_t* start, float* recon, float* mse,
                   int overlap_bits, const int32_t* overlap, int nthreads) {
    trellis_t tr;
    if (trellis_init(&tr, L, KV, V, N) || B < 0 || KV > 8) return ORACLE_EINVAL;
    if (overlap && (overlap_bits < 0 || overlap_bits > L || overlap_bits > 31)) return ORACLE_EINVAL;
    set_threads(nthreads);
    int err = ORACLE_OK;
#pragma omp parallel
    {
        float* cum = malloc((size_t)tr.S * sizeof(float));
        float* ncum = malloc((size_t)tr.S * sizeof(float));
        uint8_t* bp = malloc((size_t)tr.N * (size_t)tr.NT);
        if (!cum || !ncum || !bp) {
#pragma omp atomic write
            err = ORACLE_ENOMEM;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (int64_t b = 0; b < B; ++b) {
                size_t o = (size_t)b * N;
                viterbi_one(&tr, cb, seq + o * V, walk + o, bitstream + o, start + b, recon + o * V,
                            mse + b, cum, ncum, bp, overlap != NULL, overlap_bits,
                            overlap ? (uint32_t)overlap[b] : 0u);
            }
        }
        free(cum); free(ncum); free(bp);
    }
    return err;
}

/* Replay: states_t = ((s << kV) | bits_t) & mask, recon = c(states)
 * (src/viterbi/encode.py:310-325). */
int oracle_decode(int L, int KV, int V, int64_t B, int N, const int32_t* bitstream,
                  const int32_t* start, const float* cb, int32_t* walk, float* recon) {
    trellis_t tr;
    if (trellis_init(&tr, L, KV, V, N) || B < 0) return ORACLE_EINVAL;
    const uint32_t mask = (uint32_t)(tr.S - 1), kmask = (uint32_t)(tr.R - 1);
    for (int64_t b = 0; b < B; ++b) {
        uint32_t s = (uint32_t)start[b];
        for (int t = 0; t < N; ++t) {
            s = ((s << KV) | ((uint32_t)bitstream[(size_t)b * N + t] & kmask)) & mask;
            if (walk) walk[(size_t)b * N + t] = (int32_t)s;
            for (int v = 0; v < V; ++v) recon[((size_t)b * N + t) * V + v] = cb[(size_t)s * V + v];
        }
    }
    return ORACLE_OK;
}
