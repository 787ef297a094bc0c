/*
 * ssm_oracle.c -- CPU restatement of the Mamba SSM forward path (TEST INFRASTRUCTURE ONLY).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this file's
 * library, and only as the checker. Algorithms and citations are listed in ssm_oracle.h.
 * Every loop accumulates in double; inputs and outputs are float32.
 */
#include "ssm_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Threads the parallel loops use (1 without OpenMP). Every output element is computed by one
 * thread in a fixed order, so results do not depend on the thread count. */
int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static double softplus_d(double x) { return x > 20.0 ? x : log1p(exp(x)); }
static double silu_d(double x) { return x / (1.0 + exp(-x)); }

/* ---------------------------------------------------------------- conv1d */

void orc_causal_conv1d(const float* x, long ldx, const float* w, const float* bias,
                       float* y, long ldy, int B, int L, int C, int K, int silu,
                       const float* state_in, float* state_out) {
    for (int b = 0; b < B; ++b) {
        const float* xb = x + (long)b * L * ldx;
        float* yb = y + (long)b * L * ldy;
#pragma omp parallel for schedule(static)
        for (int t = 0; t < L; ++t) {
            for (int c = 0; c < C; ++c) {
                double acc = bias ? bias[c] : 0.0;
                for (int k = 0; k < K; ++k) {
                    int ts = t - (K - 1) + k;
                    double v;
                    if (ts >= 0) v = xb[(long)ts * ldx + c];
                    else if (state_in) v = state_in[((long)b * C + c) * (K - 1) + (K - 1) + ts];
                    else v = 0.0;
                    acc += (double)w[(long)c * K + k] * v;
                }
                yb[(long)t * ldy + c] = (float)(silu ? silu_d(acc) : acc);
            }
        }
        if (state_out) {
            for (int c = 0; c < C; ++c)
                for (int j = 0; j < K - 1; ++j) {
                    int ts = L - (K - 1) + j;
                    float v;
                    if (ts >= 0) v = xb[(long)ts * ldx + c];
                    else if (state_in) v = state_in[((long)b * C + c) * (K - 1) + (K - 1) + ts];
                    else v = 0.f;
                    state_out[((long)b * C + c) * (K - 1) + j] = v;
                }
        }
    }
}

void orc_conv_update(const float* x, const float* w, const float* bias, float* y,
                     float* state, int B, int C, int K, int silu) {
    for (int b = 0; b < B; ++b)
        for (int c = 0; c < C; ++c) {
            float* st = state + ((long)b * C + c) * (K - 1);
            double acc = bias ? bias[c] : 0.0;
            for (int k = 0; k < K - 1; ++k) acc += (double)w[(long)c * K + k] * st[k];
            acc += (double)w[(long)c * K + K - 1] * x[(long)b * C + c];
            for (int k = 0; k + 1 < K - 1; ++k) st[k] = st[k + 1];
            if (K > 1) st[K - 2] = x[(long)b * C + c];
            y[(long)b * C + c] = (float)(silu ? silu_d(acc) : acc);
        }
}

/* ------------------------------------------------------- Mamba-1 scan */

void orc_selective_scan(const float* u, long ldu, const float* dt, long lddt,
                        const float* dt_bias, int softplus, const float* A,
                        const float* Bm, long ldb, const float* Cm, long ldc,
                        const float* Dsk, const float* z, long ldz, float* y, long ldy,
                        int B, int L, int D, int N, const float* h0, float* hT) {
#pragma omp parallel
    {
    double* h = (double*)malloc(sizeof(double) * N);
#pragma omp for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
        for (int d = 0; d < D; ++d) {
            for (int n = 0; n < N; ++n) h[n] = h0 ? h0[((long)b * D + d) * N + n] : 0.0;
            for (int t = 0; t < L; ++t) {
                long r = (long)b * L + t;
                double delta = dt[r * lddt + d] + (dt_bias ? dt_bias[d] : 0.0);
                if (softplus) delta = softplus_d(delta);
                double uu = u[r * ldu + d];
                double acc = 0.0;
                for (int n = 0; n < N; ++n) {
                    double dA = exp(delta * A[(long)d * N + n]);
                    h[n] = dA * h[n] + delta * Bm[r * ldb + n] * uu;
                    acc += h[n] * Cm[r * ldc + n];
                }
                if (Dsk) acc += Dsk[d] * uu;
                if (z) acc *= silu_d(z[r * ldz + d]);
                y[r * ldy + d] = (float)acc;
            }
            if (hT)
                for (int n = 0; n < N; ++n) hT[((long)b * D + d) * N + n] = (float)h[n];
        }
    free(h);
    }
}

void orc_m1_state_update(const float* x, const float* dt, const float* dt_bias, int softplus,
                         const float* A, const float* Bm, const float* Cm, const float* Dsk,
                         const float* z, float* y, float* h, int B, int D, int N) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
        for (int d = 0; d < D; ++d) {
            double delta = dt[(long)b * D + d] + (dt_bias ? dt_bias[d] : 0.0);
            if (softplus) delta = softplus_d(delta);
            double xx = x[(long)b * D + d], acc = 0.0;
            float* hb = h + ((long)b * D + d) * N;
            for (int n = 0; n < N; ++n) {
                double v = exp(delta * A[(long)d * N + n]) * hb[n] + delta * Bm[(long)b * N + n] * xx;
                hb[n] = (float)v;
                acc += v * Cm[(long)b * N + n];
            }
            if (Dsk) acc += Dsk[d] * xx;
            if (z) acc *= silu_d(z[(long)b * D + d]);
            y[(long)b * D + d] = (float)acc;
        }
}

/* ------------------------------------------------------------ Mamba-2 SSD */

static double dt_eff(double raw, const float* dt_bias, int h, int softplus, float dt_min,
                     float dt_max) {
    double d = raw + (dt_bias ? dt_bias[h] : 0.0);
    if (softplus) d = softplus_d(d);
    if (d < dt_min) d = dt_min;
    if (d > dt_max) d = dt_max;
    return d;
}

void orc_ssd_sequential(const float* x, long ldx, const float* dt, long lddt,
                        const float* dt_bias, int softplus, float dt_min, float dt_max,
                        const float* A, const float* Bm, long ldb, const float* Cm, long ldc,
                        const float* Dsk, const float* z, long ldz, float* y, long ldy,
                        int B, int L, int H, int P, int G, int N,
                        const float* h0, float* hT) {
    int hpg = H / G;
#pragma omp parallel
    {
    double* h = (double*)malloc(sizeof(double) * (size_t)P * N);
#pragma omp for collapse(2) schedule(dynamic)
    for (int b = 0; b < B; ++b)
        for (int hh = 0; hh < H; ++hh) {
            int g = hh / hpg;
            long sbase = (((long)b * H + hh) * P) * N;
            for (long i = 0; i < (long)P * N; ++i) h[i] = h0 ? h0[sbase + i] : 0.0;
            for (int t = 0; t < L; ++t) {
                long r = (long)b * L + t;
                double delta = dt_eff(dt[r * lddt + hh], dt_bias, hh, softplus, dt_min, dt_max);
                double dA = exp(delta * A[hh]);
                const float* xr = x + r * ldx + (long)hh * P;
                const float* br = Bm + r * ldb + (long)g * N;
                const float* cr = Cm + r * ldc + (long)g * N;
                for (int p = 0; p < P; ++p) {
                    double acc = 0.0, dx = delta * xr[p];
                    for (int n = 0; n < N; ++n) {
                        double v = dA * h[(long)p * N + n] + dx * br[n];
                        h[(long)p * N + n] = v;
                        acc += v * cr[n];
                    }
                    if (Dsk) acc += Dsk[hh] * (double)xr[p];
                    if (z) acc *= silu_d(z[r * ldz + (long)hh * P + p]);
                    y[r * ldy + (long)hh * P + p] = (float)acc;
                }
            }
            if (hT)
                for (long i = 0; i < (long)P * N; ++i) hT[sbase + i] = (float)h[i];
        }
    free(h);
    }
}

void orc_ssd_chunked(const float* x, long ldx, const float* dt, long lddt,
                     const float* dt_bias, int softplus, float dt_min, float dt_max,
                     const float* A, const float* Bm, long ldb, const float* Cm, long ldc,
                     const float* Dsk, const float* z, long ldz, float* y, long ldy,
                     int B, int L, int H, int P, int G, int N, int Q,
                     const float* h0, float* hT) {
    int hpg = H / G;
#pragma omp parallel
    {
    double* S = (double*)malloc(sizeof(double) * (size_t)P * N);     /* state entering chunk */
    double* Sc = (double*)malloc(sizeof(double) * (size_t)P * N);    /* chunk-local state */
    double* acum = (double*)malloc(sizeof(double) * Q);
    double* dlt = (double*)malloc(sizeof(double) * Q);
#pragma omp for collapse(2) schedule(dynamic)
    for (int b = 0; b < B; ++b)
        for (int hh = 0; hh < H; ++hh) {
            int g = hh / hpg;
            long sbase = (((long)b * H + hh) * P) * N;
            for (long i = 0; i < (long)P * N; ++i) S[i] = h0 ? h0[sbase + i] : 0.0;
            for (int c0 = 0; c0 < L; c0 += Q) {
                int q = L - c0 < Q ? L - c0 : Q;
                double run = 0.0;
                for (int i = 0; i < q; ++i) {
                    long r = (long)b * L + c0 + i;
                    dlt[i] = dt_eff(dt[r * lddt + hh], dt_bias, hh, softplus, dt_min, dt_max);
                    run += dlt[i] * A[hh];
                    acum[i] = run;
                }
                /* outputs: Y_diag + Y_off */
                for (int i = 0; i < q; ++i) {
                    long ri = (long)b * L + c0 + i;
                    const float* ci = Cm + ri * ldc + (long)g * N;
                    for (int p = 0; p < P; ++p) {
                        double acc = 0.0;
                        for (int j = 0; j <= i; ++j) {
                            long rj = (long)b * L + c0 + j;
                            const float* bj = Bm + rj * ldb + (long)g * N;
                            double cb = 0.0;
                            for (int n = 0; n < N; ++n) cb += (double)ci[n] * bj[n];
                            acc += cb * exp(acum[i] - acum[j]) * dlt[j] *
                                   x[rj * ldx + (long)hh * P + p];
                        }
                        double off = 0.0;
                        for (int n = 0; n < N; ++n) off += (double)ci[n] * S[(long)p * N + n];
                        acc += exp(acum[i]) * off;
                        if (Dsk) acc += Dsk[hh] * (double)x[ri * ldx + (long)hh * P + p];
                        if (z) acc *= silu_d(z[ri * ldz + (long)hh * P + p]);
                        y[ri * ldy + (long)hh * P + p] = (float)acc;
                    }
                }
                /* chunk state and inter-chunk recurrence */
                for (int p = 0; p < P; ++p)
                    for (int n = 0; n < N; ++n) {
                        double s = 0.0;
                        for (int j = 0; j < q; ++j) {
                            long rj = (long)b * L + c0 + j;
                            s += exp(acum[q - 1] - acum[j]) * dlt[j] *
                                 x[rj * ldx + (long)hh * P + p] * Bm[rj * ldb + (long)g * N + n];
                        }
                        Sc[(long)p * N + n] = s;
                    }
                double a = exp(acum[q - 1]);
                for (long i = 0; i < (long)P * N; ++i) S[i] = a * S[i] + Sc[i];
            }
            if (hT)
                for (long i = 0; i < (long)P * N; ++i) hT[sbase + i] = (float)S[i];
        }
    free(S); free(Sc); free(acum); free(dlt);
    }
}

void orc_m2_state_update(const float* x, const float* dt, const float* dt_bias, int softplus,
                         float dt_min, float dt_max, const float* A, const float* Bm,
                         const float* Cm, const float* Dsk, const float* z, float* y, float* h,
                         int B, int H, int P, int G, int N) {
    int hpg = H / G;
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
        for (int hh = 0; hh < H; ++hh) {
            int g = hh / hpg;
            double delta = dt_eff(dt[(long)b * H + hh], dt_bias, hh, softplus, dt_min, dt_max);
            double dA = exp(delta * A[hh]);
            const float* br = Bm + ((long)b * G + g) * N;
            const float* cr = Cm + ((long)b * G + g) * N;
            for (int p = 0; p < P; ++p) {
                long xi = ((long)b * H + hh) * P + p;
                double xx = x[xi], acc = 0.0;
                float* hp = h + xi * N;
                for (int n = 0; n < N; ++n) {
                    double v = dA * hp[n] + delta * xx * br[n];
                    hp[n] = (float)v;
                    acc += v * cr[n];
                }
                if (Dsk) acc += Dsk[hh] * xx;
                if (z) acc *= silu_d(z[xi]);
                y[xi] = (float)acc;
            }
        }
}

/* ---------------------------------------------------------- dense glue */

void orc_linear(const float* x, long ldx, const float* W, const float* bias, float* y, long ldy,
                int M, int K, int Nout, int acc) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int m = 0; m < M; ++m)
        for (int o = 0; o < Nout; ++o) {
            double s = bias ? bias[o] : 0.0;
            const float* xr = x + (long)m * ldx;
            const float* wr = W + (long)o * K;
            for (int k = 0; k < K; ++k) s += (double)xr[k] * wr[k];
            if (acc) s += y[(long)m * ldy + o];
            y[(long)m * ldy + o] = (float)s;
        }
}

void orc_rmsnorm(const float* x, const float* w, float* y, int M, int n, float eps) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m) {
        double ss = 0.0;
        for (int i = 0; i < n; ++i) ss += (double)x[(long)m * n + i] * x[(long)m * n + i];
        double r = 1.0 / sqrt(ss / n + eps);
        for (int i = 0; i < n; ++i) y[(long)m * n + i] = (float)(x[(long)m * n + i] * r * w[i]);
    }
}

void orc_gated_rmsnorm(const float* x, long ldx, const float* z, long ldz, const float* w,
                       float* y, long ldy, int M, int n, int G, float eps) {
    int gs = n / G;
#pragma omp parallel
    {
    double* v = (double*)malloc(sizeof(double) * n);
#pragma omp for schedule(static)
    for (int m = 0; m < M; ++m) {
        for (int i = 0; i < n; ++i)
            v[i] = (double)x[(long)m * ldx + i] * silu_d(z[(long)m * ldz + i]);
        for (int g = 0; g < G; ++g) {
            double ss = 0.0;
            for (int i = g * gs; i < (g + 1) * gs; ++i) ss += v[i] * v[i];
            double r = 1.0 / sqrt(ss / gs + eps);
            for (int i = g * gs; i < (g + 1) * gs; ++i) y[(long)m * ldy + i] = (float)(v[i] * r * w[i]);
        }
    }
    free(v);
    }
}

/* ------------------------------------------------------------ sampleToken */

typedef struct {
    float e;
    int idx;
} orc_entry;

/* Array.prototype.sort with (a, b) => exps[b] - exps[a] is stable: descending e, and equal e
 * keep ascending index order (streaming.ts:74-75). */
static int entry_cmp(const void* pa, const void* pb) {
    const orc_entry* a = (const orc_entry*)pa;
    const orc_entry* b = (const orc_entry*)pb;
    if (a->e != b->e) return a->e > b->e ? -1 : 1;
    return a->idx < b->idx ? -1 : (a->idx > b->idx);
}

int orc_sample_token(const float* logits, int n, double temperature, int topK, double topP,
                     double u) {
    if (n < 1 || topK < 1) return -1;
    const double t = temperature > 1e-7 ? temperature : 1e-7;   /* streaming.ts:11,61 */
    float* scaled = (float*)malloc((size_t)n * sizeof(float));
    orc_entry* ent = (orc_entry*)malloc((size_t)n * sizeof(orc_entry));
    for (int i = 0; i < n; ++i) scaled[i] = (float)((double)logits[i] / t);   /* :60-61 */
    float maxL = -INFINITY;                                                     /* :64-65 */
    for (int i = 0; i < n; ++i)
        if (scaled[i] > maxL) maxL = scaled[i];
    double sumE = 0.0;                                                          /* :66-71 */
    for (int i = 0; i < n; ++i) {
        ent[i].e = (float)exp((double)scaled[i] - (double)maxL);
        ent[i].idx = i;
        sumE += (double)ent[i].e;
    }
    qsort(ent, (size_t)n, sizeof(orc_entry), entry_cmp);                       /* :74-76 */
    const int K = topK < n ? topK : n;
    double cum = 0.0;                                                           /* :79-85 */
    int m = 0;
    for (int k = 0; k < K; ++k) {
        cum += (double)ent[k].e / sumE;
        m = k + 1;
        if (cum >= topP) break;
    }
    double nsum = 0.0;                                                          /* :88-89 */
    for (int k = 0; k < m; ++k) nsum += (double)ent[k].e;
    const double thr = u * nsum;                                                /* :90 */
    double acc = 0.0;
    int pick = ent[m - 1].idx;                                                  /* :96 */
    for (int k = 0; k < m; ++k) {                                               /* :91-95 */
        acc += (double)ent[k].e;
        if (acc >= thr) {
            pick = ent[k].idx;
            break;
        }
    }
    free(scaled);
    free(ent);
    return pick;
}

/* ------------------------------------------------------------ model */

enum { LT_MAMBA1 = 1, LT_MAMBA2 = 2 };

typedef struct {
    int type;
    const float *norm_w, *in_proj, *conv_w, *conv_b, *x_proj, *dt_w, *dt_b, *A_log, *Dsk,
        *gnorm_w, *out_proj;
    float* A; /* -exp(A_log), owned */
} orc_layer;

struct orc_model {
    int V, d, nl, N, K, expand, H, G, R, chunk, eos;
    float eps;
    int D, P;
    float* payload; /* owned float32 copy of all tensors */
    const float* emb;
    const float* norm_f;
    orc_layer* layers;
};

struct orc_state {
    int B, nl;
    float** ssm;
    float** conv;
    size_t total;
};

static float half_to_float(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15), e = (h >> 10) & 0x1f, m = h & 0x3ff;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexp((double)(m | 0x400), (int)e - 25);
    return (float)(s ? -v : v);
}

static int layer_floats(const orc_model* m, int type, size_t* out) {
    int d = m->d, D = m->D, N = m->N, K = m->K, R = m->R, H = m->H, G = m->G;
    size_t n = (size_t)d; /* pre-norm */
    if (type == LT_MAMBA1)
        n += (size_t)2 * D * d + (size_t)D * K + D + (size_t)(R + 2 * N) * D + (size_t)D * R + D +
             (size_t)D * N + D + (size_t)d * D;
    else if (type == LT_MAMBA2)
        n += (size_t)(2 * D + 2 * G * N + H) * d + (size_t)(D + 2 * G * N) * K + (D + 2 * G * N) +
             3 * (size_t)H + D + (size_t)d * D;
    else
        return -1;
    *out = n;
    return 0;
}

orc_model* orc_model_open(const void* blob, size_t size, char* err, int errlen) {
    const unsigned char* p = (const unsigned char*)blob;
#define FAIL(msg) do { if (err) snprintf(err, errlen, "%s", msg); free(m->layers); free(m->payload); free(m); return NULL; } while (0)
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    if (size < 80 || memcmp(p, "SSMW", 4) != 0) FAIL("bad magic");
    uint32_t version, dtype, hdr;
    uint64_t payload_bytes;
    memcpy(&version, p + 4, 4); memcpy(&dtype, p + 8, 4); memcpy(&hdr, p + 12, 4);
    memcpy(&payload_bytes, p + 16, 8);
    if (version != 1) FAIL("unsupported version");
    if (dtype > 1) FAIL("unsupported dtype");
    int32_t f[11];
    memcpy(f, p + 24, 36);
    m->V = f[0]; m->d = f[1]; m->nl = f[2]; m->N = f[3]; m->K = f[4]; m->expand = f[5];
    m->H = f[6]; m->G = f[7]; m->R = f[8];
    memcpy(&m->eps, p + 60, 4);
    memcpy(&m->chunk, p + 64, 4); memcpy(&m->eos, p + 68, 4);
    m->D = m->expand * m->d;
    if (m->H <= 0 || m->G <= 0 || m->D % m->H || m->H % m->G) FAIL("bad head config");
    m->P = m->D / m->H;
    if (hdr < 80 + (uint32_t)m->nl || (size_t)hdr + payload_bytes != size) FAIL("size mismatch");
    m->layers = (orc_layer*)calloc(m->nl, sizeof(orc_layer));
    size_t total = (size_t)m->V * m->d + m->d;
    for (int l = 0; l < m->nl; ++l) {
        size_t n;
        m->layers[l].type = p[80 + l];
        if (layer_floats(m, m->layers[l].type, &n)) FAIL("bad layer type");
        total += n;
    }
    size_t esz = dtype ? 2 : 4;
    if (total * esz != payload_bytes) FAIL("payload size mismatch");
    m->payload = (float*)malloc(sizeof(float) * total);
    const unsigned char* src = p + hdr;
    if (dtype == 0) memcpy(m->payload, src, total * 4);
    else
        for (size_t i = 0; i < total; ++i) {
            uint16_t h; memcpy(&h, src + 2 * i, 2); m->payload[i] = half_to_float(h);
        }
    const float* q = m->payload;
    int d = m->d, D = m->D, N = m->N, K = m->K, R = m->R, H = m->H, G = m->G;
    m->emb = q; q += (size_t)m->V * d;
    for (int l = 0; l < m->nl; ++l) {
        orc_layer* L = &m->layers[l];
        L->norm_w = q; q += d;
        if (L->type == LT_MAMBA1) {
            L->in_proj = q; q += (size_t)2 * D * d;
            L->conv_w = q; q += (size_t)D * K;
            L->conv_b = q; q += D;
            L->x_proj = q; q += (size_t)(R + 2 * N) * D;
            L->dt_w = q; q += (size_t)D * R;
            L->dt_b = q; q += D;
            L->A_log = q; q += (size_t)D * N;
            L->Dsk = q; q += D;
            L->out_proj = q; q += (size_t)d * D;
            L->A = (float*)malloc(sizeof(float) * D * N);
            for (long i = 0; i < (long)D * N; ++i) L->A[i] = (float)(-exp((double)L->A_log[i]));
        } else {
            int cd = D + 2 * G * N;
            L->in_proj = q; q += (size_t)(2 * D + 2 * G * N + H) * d;
            L->conv_w = q; q += (size_t)cd * K;
            L->conv_b = q; q += cd;
            L->dt_b = q; q += H;
            L->A_log = q; q += H;
            L->Dsk = q; q += H;
            L->gnorm_w = q; q += D;
            L->out_proj = q; q += (size_t)d * D;
            L->A = (float*)malloc(sizeof(float) * H);
            for (int i = 0; i < H; ++i) L->A[i] = (float)(-exp((double)L->A_log[i]));
        }
    }
    m->norm_f = q;
    return m;
#undef FAIL
}

void orc_model_close(orc_model* m) {
    if (!m) return;
    for (int l = 0; l < m->nl; ++l) free(m->layers[l].A);
    free(m->layers);
    free(m->payload);
    free(m);
}

int orc_model_vocab(const orc_model* m) { return m->V; }

static size_t ssm_floats(const orc_model* m, int type, int B) {
    return type == LT_MAMBA1 ? (size_t)B * m->D * m->N : (size_t)B * m->H * m->P * m->N;
}
static size_t conv_floats(const orc_model* m, int type, int B) {
    int cd = type == LT_MAMBA1 ? m->D : m->D + 2 * m->G * m->N;
    return (size_t)B * cd * (m->K - 1);
}

orc_state* orc_state_new(const orc_model* m, int B) {
    orc_state* s = (orc_state*)calloc(1, sizeof(orc_state));
    s->B = B;
    s->ssm = (float**)calloc(m->nl, sizeof(float*));
    s->conv = (float**)calloc(m->nl, sizeof(float*));
    for (int l = 0; l < m->nl; ++l) {
        size_t a = ssm_floats(m, m->layers[l].type, B), c = conv_floats(m, m->layers[l].type, B);
        s->ssm[l] = (float*)calloc(a, sizeof(float));
        s->conv[l] = (float*)calloc(c, sizeof(float));
        s->total += a + c;
    }
    s->nl = m->nl;
    return s;
}

void orc_state_free(orc_state* s) {
    if (!s) return;
    for (int l = 0; l < s->nl; ++l) { free(s->ssm[l]); free(s->conv[l]); }
    free(s->ssm); free(s->conv); free(s);
}

size_t orc_state_floats(const orc_state* s) { return s->total; }

/* State image layout: for each layer l: ssm state then conv state. */
static void state_copy(const orc_model* m, orc_state* s, float* buf, int to_buf) {
    size_t off = 0;
    for (int l = 0; l < m->nl; ++l) {
        size_t a = ssm_floats(m, m->layers[l].type, s->B), c = conv_floats(m, m->layers[l].type, s->B);
        if (to_buf) { memcpy(buf + off, s->ssm[l], a * 4); memcpy(buf + off + a, s->conv[l], c * 4); }
        else { memcpy(s->ssm[l], buf + off, a * 4); memcpy(s->conv[l], buf + off + a, c * 4); }
        off += a + c;
    }
}

/* One mixer over (B, L) tokens; h is (B*L, d) normalized input; out (B*L, d) receives the
 * mixer output; ssm/conv state pointers may be NULL (zero initial, no write-back). */
static void mixer_forward(const orc_model* m, const orc_layer* Ly, const float* h, float* out,
                          int B, int L, float* ssm, float* conv, int update_state) {
    int d = m->d, D = m->D, N = m->N, K = m->K, R = m->R, H = m->H, G = m->G, P = m->P;
    long T = (long)B * L;
    if (Ly->type == LT_MAMBA1) {
        float* xz = (float*)malloc(sizeof(float) * T * 2 * D);
        float* xc = (float*)malloc(sizeof(float) * T * D);
        float* dbl = (float*)malloc(sizeof(float) * T * (R + 2 * N));
        float* dtv = (float*)malloc(sizeof(float) * T * D);
        float* y = (float*)malloc(sizeof(float) * T * D);
        float* cs_out = (float*)malloc(sizeof(float) * (size_t)B * D * (K - 1) + 4);
        orc_linear(h, d, Ly->in_proj, NULL, xz, 2 * D, (int)T, d, 2 * D, 0);
        orc_causal_conv1d(xz, 2 * D, Ly->conv_w, Ly->conv_b, xc, D, B, L, D, K, 1, conv, cs_out);
        orc_linear(xc, D, Ly->x_proj, NULL, dbl, R + 2 * N, (int)T, D, R + 2 * N, 0);
        orc_linear(dbl, R + 2 * N, Ly->dt_w, NULL, dtv, D, (int)T, R, D, 0);
        orc_selective_scan(xc, D, dtv, D, Ly->dt_b, 1, Ly->A, dbl + R, R + 2 * N, dbl + R + N,
                           R + 2 * N, Ly->Dsk, xz + D, 2 * D, y, D, B, L, D, N, ssm,
                           update_state ? ssm : NULL);
        if (update_state && conv) memcpy(conv, cs_out, sizeof(float) * (size_t)B * D * (K - 1));
        orc_linear(y, D, Ly->out_proj, NULL, out, d, (int)T, D, d, 0);
        free(xz); free(xc); free(dbl); free(dtv); free(y); free(cs_out);
    } else {
        int cd = D + 2 * G * N, nin = 2 * D + 2 * G * N + H;
        float* zx = (float*)malloc(sizeof(float) * T * nin);
        float* xbc = (float*)malloc(sizeof(float) * T * cd);
        float* y = (float*)malloc(sizeof(float) * T * D);
        float* yn = (float*)malloc(sizeof(float) * T * D);
        float* cs_out = (float*)malloc(sizeof(float) * (size_t)B * cd * (K - 1) + 4);
        orc_linear(h, d, Ly->in_proj, NULL, zx, nin, (int)T, d, nin, 0);
        orc_causal_conv1d(zx + D, nin, Ly->conv_w, Ly->conv_b, xbc, cd, B, L, cd, K, 1, conv, cs_out);
        orc_ssd_sequential(xbc, cd, zx + D + cd, nin, Ly->dt_b, 1, 0.f, INFINITY, Ly->A,
                           xbc + D, cd, xbc + D + G * N, cd, Ly->Dsk, NULL, 0, y, D,
                           B, L, H, P, G, N, ssm, update_state ? ssm : NULL);
        if (update_state && conv) memcpy(conv, cs_out, sizeof(float) * (size_t)B * cd * (K - 1));
        orc_gated_rmsnorm(y, D, zx, nin, Ly->gnorm_w, yn, D, (int)T, D, G, m->eps);
        orc_linear(yn, D, Ly->out_proj, NULL, out, d, (int)T, D, d, 0);
        free(zx); free(xbc); free(y); free(yn); free(cs_out);
    }
}

void orc_mixer_forward(const orc_model* m, int layer, const float* x, int B, int L, float* out) {
    mixer_forward(m, &m->layers[layer], x, out, B, L, NULL, NULL, 0);
}

/* Shared trunk: embeddings -> layers -> final norm; hidden (B*L, d) out. */
static void trunk(const orc_model* m, orc_state* s, const uint32_t* ids, int B, int L, float* hid) {
    int d = m->d;
    long T = (long)B * L;
    float* nrm = (float*)malloc(sizeof(float) * T * d);
    float* mo = (float*)malloc(sizeof(float) * T * d);
    for (long t = 0; t < T; ++t) memcpy(hid + t * d, m->emb + (size_t)ids[t] * d, sizeof(float) * d);
    for (int l = 0; l < m->nl; ++l) {
        orc_rmsnorm(hid, m->layers[l].norm_w, nrm, (int)T, d, m->eps);
        mixer_forward(m, &m->layers[l], nrm, mo, B, L, s ? s->ssm[l] : NULL, s ? s->conv[l] : NULL,
                      s != NULL);
        for (long i = 0; i < T * d; ++i) hid[i] += mo[i];
    }
    orc_rmsnorm(hid, m->norm_f, hid, (int)T, d, m->eps);
    free(nrm); free(mo);
}

void orc_model_forward(const orc_model* m, const uint32_t* ids, int B, int L, float* logits) {
    long T = (long)B * L;
    float* hid = (float*)malloc(sizeof(float) * T * m->d);
    trunk(m, NULL, ids, B, L, hid);
    orc_linear(hid, m->d, m->emb, NULL, logits, m->V, (int)T, m->d, m->V, 0);
    free(hid);
}

void orc_model_prefill(const orc_model* m, orc_state* s, const uint32_t* ids, int L,
                       float* last_logits) {
    int B = s->B;
    long T = (long)B * L;
    float* hid = (float*)malloc(sizeof(float) * T * m->d);
    float* last = (float*)malloc(sizeof(float) * (size_t)B * m->d);
    trunk(m, s, ids, B, L, hid);
    for (int b = 0; b < B; ++b)
        memcpy(last + (size_t)b * m->d, hid + ((long)b * L + L - 1) * m->d, sizeof(float) * m->d);
    orc_linear(last, m->d, m->emb, NULL, last_logits, m->V, B, m->d, m->V, 0);
    free(hid); free(last);
}

void orc_model_decode(const orc_model* m, orc_state* s, const uint32_t* ids, float* logits) {
    /* A single-token step is the L = 1 prefill continuing from the carried state: the conv
     * window comes from the conv state and the scan starts from the ssm state. */
    orc_model_prefill(m, s, ids, 1, logits);
}

void orc_state_read(const orc_model* m, const orc_state* s, float* out) {
    state_copy(m, (orc_state*)s, out, 1);
}
void orc_state_write(const orc_model* m, orc_state* s, const float* in) {
    state_copy(m, s, (float*)in, 0);
}
