/*
 * CPU oracle for the point-token hot path.  TEST INFRASTRUCTURE ONLY: this
 * file is compiled into oracle/liboracle.so and used by tests/, by
 * __graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline leg.
 * Nothing in affmae_amd/ may call it.
 *
 * Each function restates the reference algorithm it cites (paths relative to
 * the najafian-lab/affmae tree).  Floating-point work that the reference does
 * in fp32 (KNN distances) is done in fp32 with no contraction (this file is
 * built with -ffp-contract=off); attention and gathers are evaluated in fp64
 * from fp32 inputs.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ------------------------------------------------------------------ KNN --
 * knn.py:258-337, 422-471 (streaming top-K, strict '<' insertion in index
 * order => ties keep the lower index) and knn.py:1615-1648 (public API,
 * ascending order).  Key = (d2, index), d2 = fl(fl(dx*dx) + fl(dy*dy)) in
 * fp32 with dx = fl(q - r).  The k smallest keys are kept in a max-heap and
 * emitted in ascending order.
 */
static inline int key_less(float da, int ia, float db, int ib) {
    return da < db || (da == db && ia < ib);
}

static void heap_sift_down(float *hd, int *hi, int n, int i) {
    for (;;) {
        int l = 2 * i + 1, r = l + 1, m = i;
        if (l < n && key_less(hd[m], hi[m], hd[l], hi[l])) m = l;
        if (r < n && key_less(hd[m], hi[m], hd[r], hi[r])) m = r;
        if (m == i) return;
        float td = hd[i]; hd[i] = hd[m]; hd[m] = td;
        int ti = hi[i]; hi[i] = hi[m]; hi[m] = ti;
        i = m;
    }
}

/* query [B,M,D] and ref [B,N,D] contiguous fp32; out_idx [B,M,k] int64;
 * out_d2 [B,M,k] fp32 (may be NULL).  D in 1..8.  Returns 0 on success. */
int oracle_knn(const float *query, const float *ref, int B, int M, int N, int D, int k,
               int64_t *out_idx, float *out_d2) {
    if (k < 1 || k > N || D < 1 || D > 8) return 1;
    for (int b = 0; b < B; ++b) {
#pragma omp parallel for schedule(static)
        for (int m = 0; m < M; ++m) {
            float *hd = (float *)malloc(sizeof(float) * k);
            int *hi = (int *)malloc(sizeof(int) * k);
            const float *q = query + ((size_t)b * M + m) * D;
            int cnt = 0;
            for (int n = 0; n < N; ++n) {
                const float *r = ref + ((size_t)b * N + n) * D;
                float d2 = 0.f;
                for (int c = 0; c < D; ++c) {
                    float diff = q[c] - r[c];
                    float sq = diff * diff;
                    d2 = (c == 0) ? sq : d2 + sq;
                }
                if (cnt < k) {
                    /* push and sift up */
                    int i = cnt++;
                    hd[i] = d2; hi[i] = n;
                    while (i > 0) {
                        int p = (i - 1) / 2;
                        if (!key_less(hd[p], hi[p], hd[i], hi[i])) break;
                        float td = hd[i]; hd[i] = hd[p]; hd[p] = td;
                        int ti = hi[i]; hi[i] = hi[p]; hi[p] = ti;
                        i = p;
                    }
                } else if (key_less(d2, n, hd[0], hi[0])) {
                    hd[0] = d2; hi[0] = n;
                    heap_sift_down(hd, hi, k, 0);
                }
            }
            /* heap-sort into ascending order */
            int64_t *oi = out_idx + ((size_t)b * M + m) * k;
            float *od = out_d2 ? out_d2 + ((size_t)b * M + m) * k : NULL;
            for (int n = k; n > 0; --n) {
                oi[n - 1] = hi[0];
                if (od) od[n - 1] = hd[0];
                hd[0] = hd[n - 1]; hi[0] = hi[n - 1];
                heap_sift_down(hd, hi, n - 1, 0);
            }
            free(hd);
            free(hi);
        }
    }
    return 0;
}

/* ------------------------------------------------- neighbourhood attention --
 * local_attn.py:80-116 (_update_online_softmax_block), 119-215, 224-340
 * (_nbhood_attn_fwd): logits scale*<q,k_j> + bias_j; a masked neighbour takes
 * the logit -1e11 (bias dropped) and a zero value row; the blank token joins
 * the softmax; the running max starts at -1e11; lse = m + log(l + 1e-12) and
 * out = acc * exp(m - lse).  Out-of-range indices are treated as masked.
 *
 * q,k,v [B,H,N,D] fp32; idx [B,N,M] int64; bias [B,H,N,M] fp32 or NULL;
 * mask [B,H,N,M] uint8 or NULL; blank_k/blank_v [H,D] fp32 or NULL;
 * out [B,H,N,D] fp64; lse [B,H,N] fp64.
 */
int oracle_nbhd_attn(const float *q, const float *k, const float *v, const int64_t *idx,
                     const float *bias, const uint8_t *mask, const float *blank_k,
                     const float *blank_v, double scale, int B, int H, int N, int M, int D,
                     double *out, double *lse) {
    const double MASKED = -1e11;
    int64_t rows = (int64_t)B * H * N;
#pragma omp parallel for schedule(static)
    for (int64_t row = 0; row < rows; ++row) {
        int n = (int)(row % N);
        int64_t bh = row / N;
        int h = (int)(bh % H), b = (int)(bh / H);
        const float *qr = q + row * D;
        double *s = (double *)malloc(sizeof(double) * (M + 1));
        int *valid = (int *)malloc(sizeof(int) * (M + 1));
        double mx = MASKED;
        for (int j = 0; j < M; ++j) {
            int64_t id = idx[((int64_t)b * N + n) * M + j];
            int ok = id >= 0 && id < N;
            if (ok && mask) ok = mask[row * M + j] != 0;
            valid[j] = ok;
            if (ok) {
                const float *kr = k + ((int64_t)b * H + h) * N * D + id * D;
                double dot = 0.0;
                for (int c = 0; c < D; ++c) dot += (double)qr[c] * (double)kr[c];
                s[j] = scale * dot + (bias ? (double)bias[row * M + j] : 0.0);
            } else {
                s[j] = MASKED;
            }
            if (s[j] > mx) mx = s[j];
        }
        int nb = M;
        if (blank_k) {
            double dot = 0.0;
            for (int c = 0; c < D; ++c) dot += (double)qr[c] * (double)blank_k[h * D + c];
            s[M] = scale * dot;
            valid[M] = 1;
            if (s[M] > mx) mx = s[M];
            nb = M + 1;
        }
        double l = 0.0;
        for (int j = 0; j < nb; ++j) l += exp(s[j] - mx);
        double L = mx + log(l + 1e-12);
        double w = exp(mx - L);
        double *o = out + row * D;
        for (int c = 0; c < D; ++c) o[c] = 0.0;
        for (int j = 0; j < M; ++j) {
            if (!valid[j]) continue;
            int64_t id = idx[((int64_t)b * N + n) * M + j];
            const float *vr = v + ((int64_t)b * H + h) * N * D + id * D;
            double p = exp(s[j] - mx);
            for (int c = 0; c < D; ++c) o[c] += p * (double)vr[c];
        }
        if (blank_k) {
            double p = exp(s[M] - mx);
            for (int c = 0; c < D; ++c) o[c] += p * (double)blank_v[h * D + c];
        }
        for (int c = 0; c < D; ++c) o[c] *= w;
        lse[row] = L;
        free(s);
        free(valid);
    }
    return 0;
}

/* --------------------------------------------------- weighted features --
 * weighted_features.py:30-111 (kernel) and :440-457 (its PyTorch reference):
 *   out[b,i,ic,c] = sum_m w[b,i,m,ic] * f[b, idx[b,i,m], c]
 * weighted_gather (weighted_gather.py:21-102) is the IC = 1 case.
 * Indices outside [0, N) contribute nothing.  fp64 accumulation.
 * w [B,Nout,M,IC] f32; f [B,N,C] f32; idx [B,Nout,M] int64; out [B,Nout,IC,C] f64.
 */
int oracle_weighted_features(const float *w, const float *f, const int64_t *idx, int B, int Nout, int N,
                             int M, int C, int IC, double *out) {
    int64_t rows = (int64_t)B * Nout;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        int b = (int)(r / Nout);
        double *o = out + r * IC * C;
        for (int64_t t = 0; t < (int64_t)IC * C; ++t) o[t] = 0.0;
        for (int m = 0; m < M; ++m) {
            int64_t id = idx[r * M + m];
            if (id < 0 || id >= N) continue;
            const float *fr = f + ((int64_t)b * N + id) * C;
            for (int ic = 0; ic < IC; ++ic) {
                double wv = (double)w[(r * M + m) * IC + ic];
                for (int c = 0; c < C; ++c) o[ic * C + c] += wv * (double)fr[c];
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------ softmax merge --
 * knn -> w = softmax_m(-d_m / tau), d_m = |q_i - s_idx_m| -> weighted_gather
 * of features and coordinates (weighted_gather.py:21-102 applied twice).
 * qpos [B,Nout,2], spos [B,N,2], f [B,N,C] f32; idx [B,Nout,K] int64;
 * out [B,Nout,C], out_pos [B,Nout,2], out_w [B,Nout,K] f64.
 * Indices outside [0, N) get weight 0.
 */
int oracle_softmax_merge(const float *qpos, const float *spos, const float *f, const int64_t *idx,
                         int B, int Nout, int N, int K, int C, double tau, double *out, double *out_pos,
                         double *out_w) {
    int64_t rows = (int64_t)B * Nout;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        int b = (int)(r / Nout);
        double qx = qpos[r * 2], qy = qpos[r * 2 + 1];
        double *w = out_w + r * K;
        double mx = -INFINITY;
        for (int m = 0; m < K; ++m) {
            int64_t id = idx[r * K + m];
            if (id < 0 || id >= N) { w[m] = -INFINITY; continue; }
            double dx = qx - spos[((int64_t)b * N + id) * 2], dy = qy - spos[((int64_t)b * N + id) * 2 + 1];
            w[m] = -sqrt(dx * dx + dy * dy) / tau;
            if (w[m] > mx) mx = w[m];
        }
        double s = 0.0;
        for (int m = 0; m < K; ++m) { w[m] = exp(w[m] - mx); s += w[m]; }
        double *o = out + r * C;
        for (int c = 0; c < C; ++c) o[c] = 0.0;
        out_pos[r * 2] = out_pos[r * 2 + 1] = 0.0;
        for (int m = 0; m < K; ++m) {
            w[m] /= s;
            int64_t id = idx[r * K + m];
            if (id < 0 || id >= N) continue;
            const float *fr = f + ((int64_t)b * N + id) * C;
            for (int c = 0; c < C; ++c) o[c] += w[m] * (double)fr[c];
            out_pos[r * 2] += w[m] * (double)spos[((int64_t)b * N + id) * 2];
            out_pos[r * 2 + 1] += w[m] * (double)spos[((int64_t)b * N + id) * 2 + 1];
        }
    }
    return 0;
}

/* ------------------------------------------------------ deformable gather --
 * out[b,q,h,:] = sum_{s,j} w[b,q,h,s,j] * values[b, row[b,q,h,s,j], h, :]
 * (the value gather of fused_deform_attn.py:1188-1335 / msdetrpc.py:25-109),
 * rows < 0 skipped.  row, w [B,Nq,H,S,K]; values [B,Ntot,H,C] f32; out f64.
 */
int oracle_deform_gather(const int64_t *row, const double *w, const float *values, int B, int Nq, int H, int S,
                         int K, int Ntot, int C, double *out) {
    int64_t rows = (int64_t)B * Nq * H;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        int h = (int)(r % H);
        int b = (int)(r / ((int64_t)Nq * H));
        double *o = out + r * C;
        for (int c = 0; c < C; ++c) o[c] = 0.0;
        for (int t = 0; t < S * K; ++t) {
            int64_t id = row[r * S * K + t];
            if (id < 0 || id >= Ntot) continue;
            const float *v = values + (((int64_t)b * Ntot + id) * H + h) * C;
            double wv = w[r * S * K + t];
            for (int c = 0; c < C; ++c) o[c] += wv * (double)v[c];
        }
    }
    return 0;
}
