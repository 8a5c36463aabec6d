/*
 * gdn_oracle.c -- CPU oracle for the gated delta-rule (GDN) path.
 *
 * TEST INFRASTRUCTURE ONLY. This is the checker the HIP library is compared against; it is
 * never called by the library. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.
 *
 * The five legacy functions restate the double-precision host references that the
 * reference's acceptance test computes, with the same loop order and the same float/double
 * casts, so that "parity" means what it means there:
 *   ixo_step       tests/test_gdn.cu:22-26   (kernel: src/ix_gdn.cu:25-56)
 *   ixo_conv_step  tests/test_gdn.cu:36-37   (kernel: src/ix_gdn.cu:58-70)
 *   ixo_l2_norm    tests/test_gdn.cu:45      (kernel: src/ix_gdn.cu:73-84)
 *   ixo_out_norm   tests/test_gdn.cu:49-50   (kernel: src/ix_gdn.cu:87-100)
 *   ixo_beta_gate  tests/test_gdn.cu:54      (kernel: src/ix_gdn.cu:102-105)
 *
 * The fused decode and the prefill have no reference function. They compose the legacy
 * semantics (decay before the k^T S read, modulo head pairing, no q scale, conv without
 * activation: src/ix_gdn.cu:38, :49-53, :62-69) with closed forms:
 *   gate = -exp(A_log) * softplus(a + dt_bias), softplus as src/ix_gdn.cu:22
 *   beta = sigmoid(b), sigmoid as src/ix_gdn.cu:23
 *   q, k L2-normalised per head: x / sqrt(sum x^2 + eps), eps placement as src/ix_gdn.cu:82
 * The prefill is the token-by-token recurrence (T applications of the decode step).
 *
 * Parity pins (tests/test_oracle.py): known answers of the step (beta = 0 is pure decay;
 * a zero state gives S = beta k v^T; beta = 1 with a unit k gives S'^T k = v for any decay),
 * one-hot layout probes for the head map and the state index, brute force against the
 * product form S' = (I - beta k k^T) g S + beta k v^T, the L2 invariant, bit-exact conv
 * shift, closed forms of sigmoid/softplus, and B-independence / token-split invariance.
 */
#include "gdn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static inline double bf16_to_double(uint16_t u) {
    uint32_t bits = (uint32_t)u << 16;
    float f;
    memcpy(&f, &bits, sizeof f);
    return (double)f;
}

/* ------------------------------------------------------------------------------------------
 * Legacy functions (fp32 inputs, double references)
 * ------------------------------------------------------------------------------------------ */

/* tests/test_gdn.cu:22-26. State layout [S(i)][h_v][S(j)], element (h,i,j) at (i*h_v+h)*S+j
 * (src/ix_gdn.cu:47-48). Decay is applied before the k^T S contraction (src/ix_gdn.cu:49-50);
 * the output reads the updated state (src/ix_gdn.cu:52-53). */
void ixo_step(double* rs, const float* q, const float* k, const float* v, const float* gate,
              const float* beta, double* ro, int S, int hk, int hv) {
    for (int h = 0; h < hv; ++h) {
        const int src = h % hk;
        const double dec = exp((double)gate[h]);
        for (int j = 0; j < S; ++j) {
            double sk = 0;
            for (int i = 0; i < S; ++i) {
                const size_t e = ((size_t)i * hv + h) * S + j;
                const double s = rs[e] * dec;
                rs[e] = s;
                sk += s * k[src * S + i];
            }
            const double d = (v[h * S + j] - sk) * beta[h];
            double dot = 0;
            for (int i = 0; i < S; ++i) {
                const size_t e = ((size_t)i * hv + h) * S + j;
                const double s = rs[e] + k[src * S + i] * d;
                rs[e] = s;
                dot += s * q[src * S + i];
            }
            ro[h * S + j] = dot;
        }
    }
}

/* tests/test_gdn.cu:36-37. conv_state [C][dc-1] oldest first; w [C][dc]; the shift is exact. */
void ixo_conv_step(float* cs, const float* x, const float* w, double* out, int C, int dc) {
    for (int c = 0; c < C; ++c) {
        double acc = 0;
        for (int i = 0; i < dc - 1; ++i) acc += (double)cs[(size_t)c * (dc - 1) + i] * w[(size_t)c * dc + i];
        acc += (double)x[c] * w[(size_t)c * dc + dc - 1];
        out[c] = acc;
        for (int i = 0; i < dc - 2; ++i) cs[(size_t)c * (dc - 1) + i] = cs[(size_t)c * (dc - 1) + i + 1];
        cs[(size_t)c * (dc - 1) + dc - 2] = x[c];
    }
}

/* tests/test_gdn.cu:45: double sum of squares, inverse norm rounded to float, float product. */
void ixo_l2_norm(const float* x, double* r, int rows, int cols, float eps) {
    for (int i = 0; i < rows; ++i) {
        double s = 0;
        for (int c = 0; c < cols; ++c) s += (double)x[(size_t)i * cols + c] * x[(size_t)i * cols + c];
        const float inv = (float)(1.0 / sqrt(s + (double)eps));
        for (int c = 0; c < cols; ++c) r[(size_t)i * cols + c] = x[(size_t)i * cols + c] * inv;
    }
}

/* tests/test_gdn.cu:49-50: double mean square, float inverse, float o*inv*norm, double sigmoid. */
void ixo_out_norm(const float* o, const float* z, const float* nrm, double* r, int hv, int S, float eps) {
    for (int h = 0; h < hv; ++h) {
        double s = 0;
        for (int i = 0; i < S; ++i) s += (double)o[(size_t)h * S + i] * o[(size_t)h * S + i];
        const float inv = (float)(1.0 / sqrt(s / S + (double)eps));
        for (int i = 0; i < S; ++i)
            r[(size_t)h * S + i] = (double)(o[(size_t)h * S + i] * inv * nrm[i]) / (1.0 + exp(-(double)z[(size_t)h * S + i]));
    }
}

/* tests/test_gdn.cu:54 */
void ixo_beta_gate(const float* b, double* r, int n) {
    for (int i = 0; i < n; ++i) r[i] = 1.0 / (1.0 + exp(-(double)b[i]));
}

/* ------------------------------------------------------------------------------------------
 * Fused layer extensions
 * ------------------------------------------------------------------------------------------ */

int ixo_src_head(const ixo_cfg* c, int h) {
    if (c->head_map == 0) return h % c->h_k;        /* src/ix_gdn.cu:38 */
    return h / (c->h_v / c->h_k);
}

/* src/ix_gdn.cu:22 (threshold 20 is the reference's definition) */
double ixo_softplus(double x) { return x > 20.0 ? x : log1p(exp(x)); }
/* src/ix_gdn.cu:23 */
double ixo_sigmoid(double x) { return 1.0 / (1.0 + exp(-x)); }
double ixo_gate(float A_log, double a, float dt_bias) { return -exp((double)A_log) * ixo_softplus(a + (double)dt_bias); }

/* Conv over every channel of one sequence (src/ix_gdn.cu:58-70 semantics, bf16 storage),
 * then the optional activation. */
static void conv_row(const ixo_cfg* c, const uint16_t* x, uint16_t* cs, const uint16_t* w, double* y) {
    const int C = 2 * c->h_k * c->d_k + c->h_v * c->d_v, dc = c->d_conv;
    for (int ch = 0; ch < C; ++ch) {
        uint16_t* st = cs + (size_t)ch * (dc - 1);
        const uint16_t* wc = w + (size_t)ch * dc;
        double acc = 0;
        for (int i = 0; i < dc - 1; ++i) acc += bf16_to_double(st[i]) * bf16_to_double(wc[i]);
        acc += bf16_to_double(x[ch]) * bf16_to_double(wc[dc - 1]);
        for (int i = 0; i < dc - 2; ++i) st[i] = st[i + 1];
        st[dc - 2] = x[ch];
        if (c->conv_act == 1) acc = acc * ixo_sigmoid(acc);
        y[ch] = acc;
    }
}

/* One v-head of one token: normalise q/k of the paired head, gates, then the reference's
 * step loop (test_gdn.cu:23-26 order) on a [d_k][d_v] state. */
static void head_step(const ixo_cfg* c, const double* y, int h, double a, double b, float A_log,
                      float dt_bias, double* S, double* o) {
    const int dk = c->d_k, dv = c->d_v, src = ixo_src_head(c, h);
    const double* qr = y + (size_t)src * dk;
    const double* kr = y + (size_t)c->h_k * dk + (size_t)src * dk;
    const double* vr = y + 2 * (size_t)c->h_k * dk + (size_t)h * dv;
    double qq = 0, kk = 0;
    for (int i = 0; i < dk; ++i) { qq += qr[i] * qr[i]; kk += kr[i] * kr[i]; }
    const double iq = 1.0 / sqrt(qq + (double)c->l2_eps) * (double)c->q_scale;
    const double ik = 1.0 / sqrt(kk + (double)c->l2_eps);
    const double dec = exp(ixo_gate(A_log, a, dt_bias));
    const double beta = ixo_sigmoid(b);
    for (int j = 0; j < dv; ++j) {
        double sk = 0;
        for (int i = 0; i < dk; ++i) {
            const double s = S[(size_t)i * dv + j] * dec;
            S[(size_t)i * dv + j] = s;
            sk += s * (kr[i] * ik);
        }
        const double d = (vr[j] - sk) * beta;
        double dot = 0;
        for (int i = 0; i < dk; ++i) {
            const double s = S[(size_t)i * dv + j] + (kr[i] * ik) * d;
            S[(size_t)i * dv + j] = s;
            dot += s * (qr[i] * iq);
        }
        o[j] = dot;
    }
}

void ixo_decode(const ixo_cfg* c, int B, const uint16_t* x, uint16_t* cs, const uint16_t* w,
                const uint16_t* a, const uint16_t* b, const float* A_log, const float* dt_bias,
                double* state, double* o, int nthreads) {
    const int C = 2 * c->h_k * c->d_k + c->h_v * c->d_v, hv = c->h_v, dc = c->d_conv;
    const size_t tile = (size_t)c->d_k * c->d_v;
    double* y = (double*)malloc(sizeof(double) * (size_t)B * C);
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int bb = 0; bb < B; ++bb)
        conv_row(c, x + (size_t)bb * C, cs + (size_t)bb * C * (dc - 1), w, y + (size_t)bb * C);
#pragma omp parallel for num_threads(nthreads) schedule(static) collapse(2)
    for (int bb = 0; bb < B; ++bb)
        for (int h = 0; h < hv; ++h)
            head_step(c, y + (size_t)bb * C, h, bf16_to_double(a[(size_t)bb * hv + h]),
                      bf16_to_double(b[(size_t)bb * hv + h]), A_log[h], dt_bias[h],
                      state + ((size_t)bb * hv + h) * tile, o + ((size_t)bb * hv + h) * c->d_v);
    free(y);
}

void ixo_prefill(const ixo_cfg* c, int n_seq, const int32_t* cu, const uint16_t* x, uint16_t* cs,
                 const uint16_t* w, const uint16_t* a, const uint16_t* b, const float* A_log,
                 const float* dt_bias, double* state, double* o, int nthreads) {
    const int C = 2 * c->h_k * c->d_k + c->h_v * c->d_v, hv = c->h_v, dc = c->d_conv;
    const size_t tile = (size_t)c->d_k * c->d_v;
    double* y = (double*)malloc(sizeof(double) * (size_t)C);
    if (nthreads < 1) nthreads = 1;
    for (int s = 0; s < n_seq; ++s) {
        for (int t = cu[s]; t < cu[s + 1]; ++t) {
            conv_row(c, x + (size_t)t * C, cs + (size_t)s * C * (dc - 1), w, y);
#pragma omp parallel for num_threads(nthreads) schedule(static)
            for (int h = 0; h < hv; ++h)
                head_step(c, y, h, bf16_to_double(a[(size_t)t * hv + h]), bf16_to_double(b[(size_t)t * hv + h]),
                          A_log[h], dt_bias[h], state + ((size_t)s * hv + h) * tile, o + ((size_t)t * hv + h) * c->d_v);
        }
    }
    free(y);
}

/* ------------------------------------------------------------------------------------------
 * Input generator support (oracle/inputs.py): out[i] = mix(i + key) for i < n, with mix the
 * splitmix64 finaliser. Exact integer arithmetic, so it equals the numpy formulation bit for
 * bit; it only makes large seeded tensors cheap to generate.
 * ------------------------------------------------------------------------------------------ */
static inline uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void ixo_mix_counter(uint64_t key, uint64_t n, uint64_t* out) {
#pragma omp parallel for schedule(static) num_threads(8)
    for (long long i = 0; i < (long long)n; ++i) out[i] = splitmix64((uint64_t)i + key);
}
