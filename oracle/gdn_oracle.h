/*
 * gdn_oracle.h -- CPU oracle for the gated delta-rule (GDN) path.
 *
 * TEST INFRASTRUCTURE ONLY: this is the checker for the HIP library, never part of it.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * All arithmetic is double precision, following the reference's host references in
 * tests/test_gdn.cu. Per-function citations are in gdn_oracle.c.
 */
#ifndef IXO_GDN_ORACLE_H
#define IXO_GDN_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same field order and meaning as ix_gdn_cfg in include/ix_gdn.h. */
typedef struct ixo_cfg {
    int h_k, h_v;     /* q/k heads, v heads */
    int d_k, d_v;     /* head dims */
    int d_conv;       /* causal conv taps (>= 2) */
    int head_map;     /* 0: src = h mod h_k (reference); 1: src = h / (h_v / h_k) */
    int conv_act;     /* 0: none (reference); 1: SiLU after the conv */
    float q_scale;    /* multiplies the L2-normalised q; 1.0 in the reference */
    float l2_eps;     /* x * 1/sqrt(sum x^2 + eps) */
} ixo_cfg;

/* ---- legacy entry points (fp32 device API in the reference) ---- */
void ixo_step(double* state, const float* q, const float* k, const float* v, const float* gate,
              const float* beta, double* o, int S, int h_k, int h_v);
void ixo_conv_step(float* conv_state, const float* x, const float* w, double* out, int C, int d_conv);
void ixo_l2_norm(const float* x, double* out, int rows, int cols, float eps);
void ixo_out_norm(const float* o, const float* z, const float* ssm_norm, double* y, int h_v, int S, float eps);
void ixo_beta_gate(const float* b, double* out, int n);

/* ---- fused layer extensions (no reference function; closed forms) ---- */
int ixo_src_head(const ixo_cfg* c, int h);
double ixo_gate(float A_log, double a, float dt_bias);
double ixo_sigmoid(double x);
double ixo_softplus(double x);

/* One decode token for B sequences. x [B][C] bf16 (C = 2*h_k*d_k + h_v*d_v, order q|k|v);
 * conv_state [B][C][d_conv-1] bf16 oldest first (updated); w [C][d_conv] bf16; a, b [B][h_v] bf16;
 * A_log, dt_bias [h_v]; state [B][h_v][d_k][d_v] double (updated); o [B][h_v][d_v] double. */
void ixo_decode(const ixo_cfg* c, int B, const uint16_t* x, uint16_t* conv_state, const uint16_t* w,
                const uint16_t* a, const uint16_t* b, const float* A_log, const float* dt_bias,
                double* state, double* o, int nthreads);

/* Token-by-token prefill over packed sequences: cu_seqlens [n_seq+1]; x [T][C]; a, b [T][h_v];
 * conv_state [n_seq][C][d_conv-1]; state [n_seq][h_v][d_k][d_v]; o [T][h_v][d_v]. */
void ixo_prefill(const ixo_cfg* c, int n_seq, const int32_t* cu_seqlens, const uint16_t* x,
                 uint16_t* conv_state, const uint16_t* w, const uint16_t* a, const uint16_t* b,
                 const float* A_log, const float* dt_bias, double* state, double* o, int nthreads);

/* Input generator support: out[i] = splitmix64(i + key), i < n (oracle/inputs.py). */
void ixo_mix_counter(uint64_t key, uint64_t n, uint64_t* out);

#ifdef __cplusplus
}
#endif
#endif
