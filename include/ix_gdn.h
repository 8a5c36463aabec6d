/*
 * ix_gdn.h -- C ABI of libixgdn.so, the MI355X (gfx950) gated delta-rule (GDN) library.
 *
 * The first five entry points replace the reference's header-only inline launchers in
 * src/ix_gdn.cu one for one: same names, same parameter order and meaning, same shape
 * validation (hipErrorInvalidValue before any launch), same asynchronous contract (work is
 * enqueued on `s`, nothing is allocated, the caller synchronises). They are exported with C
 * linkage so any FFI can bind them; C++ callers get the reference's `s = 0` default.
 *
 * The fused decode and the chunked prefill are additions (no reference counterpart) for
 * serving a whole GDN layer: bf16 activations in, fp32 recurrent state, conv fused ahead of
 * the recurrence.
 *
 * Pointers are device pointers unless stated otherwise. bf16 values are passed as their
 * 16-bit patterns (uint16_t).
 */
#ifndef IX_GDN_H
#define IX_GDN_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
#define IX_GDN_DEFAULT_STREAM = 0
extern "C" {
#else
#define IX_GDN_DEFAULT_STREAM
#endif

/* ---------------------------------------------------------------------------------------
 * Legacy entry points (all fp32)
 * --------------------------------------------------------------------------------------- */

/* One decode token of the delta rule for h_v heads. Replaces ix_gdn_step, src/ix_gdn.cu:108-114.
 * state [S][h_v][S] (element (h,i,j) at (i*h_v+h)*S+j, updated in place); q, k [h_k][S];
 * v, o [h_v][S]; gate, beta [h_v] (gate is a log-decay, beta already sigmoided).
 * For head h: src = h mod h_k, S_h <- exp(gate) S_h; d = beta (v - S_h^T k); S_h += k d^T;
 * o = S_h^T q. Requires 0 < S <= 128, h_k > 0, h_v > 0. */
hipError_t ix_gdn_step(float* state, const float* q, const float* k, const float* v, const float* gate,
                       const float* beta, float* o, int S, int h_k, int h_v, hipStream_t s IX_GDN_DEFAULT_STREAM);

/* Depthwise causal conv over `channels` with a rolling state. Replaces ix_gdn_conv_step,
 * src/ix_gdn.cu:115-120. conv_state [channels][d_conv-1] oldest first (shifted in place, x
 * appended); kW [channels][d_conv]; out [channels] = sum(state*kW[..d_conv-1]) + x*kW[d_conv-1].
 * Requires channels > 0, d_conv >= 2. */
hipError_t ix_gdn_conv_step(float* conv_state, const float* x, const float* kW, float* out, int channels,
                            int d_conv, hipStream_t s IX_GDN_DEFAULT_STREAM);

/* In-place row L2 normalisation x <- x / sqrt(sum x^2 + eps) (double accumulation).
 * Replaces ix_gdn_l2_norm, src/ix_gdn.cu:121-125. Requires rows > 0, 0 < cols <= 1024. */
hipError_t ix_gdn_l2_norm(float* x, int rows, int cols, float eps, hipStream_t s IX_GDN_DEFAULT_STREAM);

/* In-place beta <- sigmoid(beta). Replaces ix_gdn_beta_gate, src/ix_gdn.cu:126-130.
 * Requires beta != NULL, h_v > 0. */
hipError_t ix_gdn_beta_gate(float* beta, int h_v, hipStream_t s IX_GDN_DEFAULT_STREAM);

/* Gated RMS output norm y = o / sqrt(mean(o^2) + eps) * ssm_norm * sigmoid(z), per head.
 * Replaces ix_gdn_out_norm, src/ix_gdn.cu:131-136. o, z, y [h_v][S]; ssm_norm [S].
 * Requires h_v > 0, S > 0. */
hipError_t ix_gdn_out_norm(const float* o, const float* z, const float* ssm_norm, float* y, int h_v, int S,
                           float eps, hipStream_t s IX_GDN_DEFAULT_STREAM);

/* ---------------------------------------------------------------------------------------
 * Fused layer entry points (additions; no reference counterpart)
 * --------------------------------------------------------------------------------------- */

enum { IX_GDN_HEAD_MOD = 0,   /* src = h mod h_k (the reference's pairing, src/ix_gdn.cu:38) */
       IX_GDN_HEAD_DIV = 1 }; /* src = h / (h_v / h_k) (contiguous groups) */
enum { IX_GDN_ACT_NONE = 0,   /* conv output used as is (the reference, src/ix_gdn.cu:64-67) */
       IX_GDN_ACT_SILU = 1 }; /* SiLU after the conv */

/* Host-side layer description (read on the host at call time). */
typedef struct ix_gdn_cfg {
    int h_k, h_v;     /* q/k heads and v heads */
    int d_k, d_v;     /* head dims; the fused kernels require d_k = d_v = 128 */
    int d_conv;       /* conv taps, 2..4 */
    int head_map;     /* IX_GDN_HEAD_MOD or IX_GDN_HEAD_DIV */
    int conv_act;     /* IX_GDN_ACT_NONE or IX_GDN_ACT_SILU */
    float q_scale;    /* multiplies the normalised q (1.0 in the reference) */
    float l2_eps;     /* q, k <- x / sqrt(sum x^2 + eps) */
} ix_gdn_cfg;

/* Mixed-projection channel count C = 2*h_k*d_k + h_v*d_v (order q | k | v). */
int ix_gdn_channels(const ix_gdn_cfg* cfg);

/* Fused state layout (decode and prefill): [B][h_v][d_v][d_k] fp32 -- each head's state S
 * (d_k x d_v, S[i][j] with i the k index and j the v index) is stored column by column, so
 * element (b, h, i, j) is at ((b*h_v + h)*d_v + j)*d_k + i and every column is contiguous. */

/* Bytes of the workspace ix_gdn_decode and ix_gdn_decode_gated can use for B sequences, or 0
 * for an invalid description. It holds one counter per (sequence, q/k head), which the
 * calls keep at zero. */
size_t ix_gdn_decode_workspace_size(const ix_gdn_cfg* cfg, int B);

/* Gated RMS output norm fused into a layer call's epilogue: for every token row and v head,
 *   y = o / sqrt(mean(o^2) + eps) * ssm_norm * sigmoid(z)
 * over the head's d_v outputs -- the semantics of ix_gdn_out_norm (src/ix_gdn.cu:87-100:
 * products in that order, sigmoid(x) = 1/(1+exp(-x))) with fp32 accumulation of the sum of
 * squares, taken as (sum of columns 0..63) + (sum of columns 64..127). Read on the host at
 * call time. */
typedef struct ix_gdn_out_gate {
    const uint16_t* z;        /* [rows][h_v][d_v] bf16 gate logits (from the in-projection) */
    const float* ssm_norm;    /* [d_v] fp32 norm weight shared by all heads */
    float eps;
    float* y;                 /* [rows][h_v][d_v] fp32, or NULL */
    uint16_t* y_bf16;         /* [rows][h_v][d_v] bf16 (RNE of the fp32 value), or NULL */
    void* y_q8_1;             /* [rows][h_v*d_v/32] q8_1 blocks of the fp32 value (the activation
                               * format of ix_mmvq_q8_0; see ix_q8_1_quantize), 4-byte aligned, or
                               * NULL */
} ix_gdn_out_gate;

/* One decode token for B independent sequences of one GDN layer, in one launch:
 * causal conv over the mixed q|k|v channels with its rolling state, per-head L2 norm of q
 * and k, gates g = exp(-exp(A_log) * softplus(a + dt_bias)) and beta = sigmoid(b), head map
 * of h_k q/k heads onto h_v v heads, and the delta-rule update of the fp32 state with the
 * output o = S'^T q.
 *   x          [B][C] bf16 (pre-conv mixed projection)
 *   conv_state [B][C][d_conv-1] bf16, oldest first, updated in place
 *   conv_w     [C][d_conv] bf16
 *   a, b       [B][h_v] bf16 gate and beta logits
 *   A_log, dt_bias [h_v] fp32
 *   state      [B][h_v][d_v][d_k] fp32 (layout above), updated in place, 16-byte aligned
 *   o          [B][h_v][d_v] fp32, or NULL
 *   o_bf16     [B][h_v][d_v] bf16 (round to nearest even of the fp32 output), or NULL
 *   workspace  NULL, or ix_gdn_decode_workspace_size(cfg, B) bytes of device memory that are
 *              all zero before the first call; every call leaves them all zero again. With a
 *              workspace the state streams through more, shorter workgroups (faster); calls
 *              that share one workspace must be ordered (same stream), since it holds
 *              per-call counters. x, conv_state, conv_w and workspace must be 4-byte aligned.
 * Calls on one stream are ordered; two streams must not share a state or conv-state buffer. */
hipError_t ix_gdn_decode(const ix_gdn_cfg* cfg, int B, const uint16_t* x, uint16_t* conv_state,
                         const uint16_t* conv_w, const uint16_t* a, const uint16_t* b, const float* A_log,
                         const float* dt_bias, float* state, float* o, uint16_t* o_bf16, void* workspace,
                         hipStream_t s IX_GDN_DEFAULT_STREAM);

/* ix_gdn_decode for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. It runs the kernel ix_gdn_decode runs with a workspace, with the group counters
 * in a library-owned static device array (one copy per GPU, 256 KiB, held until the process
 * ends; zero when the library is loaded, its address looked up on the first call on each
 * device) instead of a caller workspace, and calls no allocating routine; each call enqueues
 * the decode kernel only, so it may be captured into a HIP graph, first call included. Requires B * h_k <= 65536 (else hipErrorInvalidValue,
 * before any launch). Every call in this process on one GPU shares that GPU's array, which
 * each call leaves all zero: calls that overlap on one GPU (on two streams, or from two host
 * threads) race, so the caller must order them, e.g. on one stream. Arguments otherwise as
 * ix_gdn_decode. */
hipError_t ix_gdn_decode_noalloc(const ix_gdn_cfg* cfg, int B, const uint16_t* x, uint16_t* conv_state,
                                 const uint16_t* conv_w, const uint16_t* a, const uint16_t* b, const float* A_log,
                                 const float* dt_bias, float* state, float* o, uint16_t* o_bf16,
                                 hipStream_t s IX_GDN_DEFAULT_STREAM);

/* ix_gdn_decode followed by the gated output norm of each (sequence, v head), in the same
 * launch: gate->z, gate->y, gate->y_bf16 are [B][h_v][d_v]. o and o_bf16 may both be NULL.
 * gate must be non-NULL with z, ssm_norm and at least one of y, y_bf16 set. With a workspace
 * one workgroup per (sequence, v head) computes the head's outputs and applies the norm. */
hipError_t ix_gdn_decode_gated(const ix_gdn_cfg* cfg, int B, const uint16_t* x, uint16_t* conv_state,
                               const uint16_t* conv_w, const uint16_t* a, const uint16_t* b,
                               const float* A_log, const float* dt_bias, float* state, float* o,
                               uint16_t* o_bf16, const ix_gdn_out_gate* gate, void* workspace,
                               hipStream_t s IX_GDN_DEFAULT_STREAM);

/* Bytes of device workspace for ix_gdn_prefill over n_seq sequences and total_T tokens in
 * windows of at most 80 chunks of 64 tokens (1.83 MiB per chunk at the Qwen3-Next head layout:
 * 146 MiB at most, plus 16 bytes per chunk of tables). A batch of up to 5,120 tokens runs as
 * one window. Windows are never longer, whatever the workspace: a window's chunk operands then
 * stay in the GPU's Infinity Cache between the two kernels that write and read them. */
size_t ix_gdn_prefill_workspace_size(const ix_gdn_cfg* cfg, int n_seq, int total_T);

/* Bytes of device workspace for ix_gdn_prefill (gated = 0) or ix_gdn_prefill_gated (gated = 1)
 * in windows of window_chunks 64-token chunks: the chunk tables (16 bytes per chunk) plus the
 * chunk operands of one window. Any workspace of at least the size for window_chunks = 1 works;
 * the prefill then runs in windows of as many chunks as the workspace holds (at most 80), one
 * after the other, with results identical to the one-window run. 0 for invalid arguments. Addition; no
 * reference counterpart (for callers that bound device memory independently of total_T). */
size_t ix_gdn_prefill_window_workspace_size(const ix_gdn_cfg* cfg, int n_seq, int total_T, int window_chunks,
                                            int gated);

/* Chunked (64-token chunks) prefill of n_seq packed sequences, the same math as
 * total_T applications of ix_gdn_decode:
 *   cu_seqlens [n_seq+1] int32 device offsets (cu_seqlens[0] = 0, non-decreasing)
 *   x [total_T][C] bf16; a, b [total_T][h_v] bf16
 *   conv_state [n_seq][C][d_conv-1] bf16 in/out; state [n_seq][h_v][d_v][d_k] fp32 in/out
 *   (16-byte aligned)
 *   o [total_T][h_v][d_v] fp32 or NULL; o_bf16 likewise
 *   workspace: 256-byte aligned device memory of at least
 *   ix_gdn_prefill_window_workspace_size(cfg, n_seq, total_T, 1, 0) bytes (windows of one
 *   chunk); the prefill uses windows of as many chunks as the workspace holds, e.g.
 *   ix_gdn_prefill_workspace_size() bytes. */
hipError_t ix_gdn_prefill(const ix_gdn_cfg* cfg, int n_seq, int total_T, const int32_t* cu_seqlens,
                          const uint16_t* x, uint16_t* conv_state, const uint16_t* conv_w, const uint16_t* a,
                          const uint16_t* b, const float* A_log, const float* dt_bias, float* state, float* o,
                          uint16_t* o_bf16, void* workspace, size_t workspace_bytes,
                          hipStream_t s IX_GDN_DEFAULT_STREAM);

/* Bytes of device workspace ix_gdn_prefill_gated needs in the default windows (the
 * prefill's, plus room for one window's fp32 outputs, which the norm reads when the caller
 * passes no o). */
size_t ix_gdn_prefill_gated_workspace_size(const ix_gdn_cfg* cfg, int n_seq, int total_T);

/* ix_gdn_prefill followed by the gated output norm of every (token, v head) row:
 * gate->z, gate->y, gate->y_bf16 are [total_T][h_v][d_v]; workspace_bytes must be at least
 * ix_gdn_prefill_window_workspace_size(cfg, n_seq, total_T, 1, 1) (windows of one chunk;
 * ix_gdn_prefill_gated_workspace_size() gives the default windows). */
hipError_t ix_gdn_prefill_gated(const ix_gdn_cfg* cfg, int n_seq, int total_T, const int32_t* cu_seqlens,
                                const uint16_t* x, uint16_t* conv_state, const uint16_t* conv_w,
                                const uint16_t* a, const uint16_t* b, const float* A_log, const float* dt_bias,
                                float* state, float* o, uint16_t* o_bf16, const ix_gdn_out_gate* gate,
                                void* workspace, size_t workspace_bytes, hipStream_t s IX_GDN_DEFAULT_STREAM);

/* ---------------------------------------------------------------------------------------
 * Speculative windows (additions; no reference counterpart)
 *
 * A window is K draft tokens per sequence (1 <= K <= 16). ix_gdn_decode_window runs them
 * from the committed states and writes their outputs plus a window record, without
 * changing either state; ix_gdn_commit_window then advances the committed states by each
 * sequence's accepted prefix. Outputs are bit-identical to K ix_gdn_decode calls, and the
 * committed states to n calls for n accepted tokens.
 *
 * Window record (fp32, row = b*K + t; sections in this order, each 256-byte aligned):
 *   k_hat [B*K][h_k][d_k]  normalised key of each q/k head
 *   v     [B*K][h_v][d_v]  conv output of each v head's channels
 *   g     [B*K][h_v]       decay exp(-exp(A_log) * softplus(a + dt_bias))
 *   beta  [B*K][h_v]       sigmoid(b)
 * Both calls require every q/k head to feed at least one v head (IX_GDN_HEAD_DIV, or
 * h_v >= h_k with IX_GDN_HEAD_MOD).
 * --------------------------------------------------------------------------------------- */

/* Bytes of the window record for B sequences and K tokens, or 0 for an invalid request. */
size_t ix_gdn_window_record_size(const ix_gdn_cfg* cfg, int B, int K);

/* Verify a window: x [B][K][C] bf16, a, b [B][K][h_v] bf16; conv_state and state as in
 * ix_gdn_decode (read only here); o, o_bf16 [B][K][h_v][d_v] (either may be NULL); record:
 * ix_gdn_window_record_size() bytes, 256-byte aligned, written. */
hipError_t ix_gdn_decode_window(const ix_gdn_cfg* cfg, int B, int K, const uint16_t* x,
                                const uint16_t* conv_state, const uint16_t* conv_w, const uint16_t* a,
                                const uint16_t* b, const float* A_log, const float* dt_bias, const float* state,
                                float* o, uint16_t* o_bf16, void* record, hipStream_t s IX_GDN_DEFAULT_STREAM);

/* The same verify on the matrix cores: the committed state enters only through the products
 * S^T k_t and S^T q_t of the K tokens (split-bf16 MFMA, ~2^-16 relative), and the K steps are
 * unrolled in the K-token space. Outputs agree with K ix_gdn_decode calls to fp32 rounding
 * (within the decode tolerances of the reference's double recurrence), not bit for bit; the
 * record is bit-identical to ix_gdn_decode_window's, so ix_gdn_commit_window then gives the
 * same committed states. Arguments and requirements as ix_gdn_decode_window. */
hipError_t ix_gdn_decode_window_mfma(const ix_gdn_cfg* cfg, int B, int K, const uint16_t* x,
                                     const uint16_t* conv_state, const uint16_t* conv_w, const uint16_t* a,
                                     const uint16_t* b, const float* A_log, const float* dt_bias,
                                     const float* state, float* o, uint16_t* o_bf16, void* record,
                                     hipStream_t s IX_GDN_DEFAULT_STREAM);

/* Commit a window: accepted [B] int32 device array, each clamped to [0, K]; x and record as
 * given to ix_gdn_decode_window. Sequence b's conv_state and state advance by accepted[b]
 * tokens; a sequence with accepted[b] = 0 is not touched. */
hipError_t ix_gdn_commit_window(const ix_gdn_cfg* cfg, int B, int K, const int32_t* accepted, const uint16_t* x,
                                const void* record, uint16_t* conv_state, float* state,
                                hipStream_t s IX_GDN_DEFAULT_STREAM);

/* Commit one window in every GDN layer of a model, in one launch (the upstream layer-batched
 * commit the reference's project notes describe, STRATA_COMMITS_FULL.txt:3556; no counterpart
 * in the reference's sources). accepted [B] as for ix_gdn_commit_window, shared by the
 * layers; x, record, conv_state and state are DEVICE arrays of n_layers pointers, entry l
 * being what ix_gdn_commit_window would take for layer l (each state 16-byte and each record
 * 256-byte aligned; a layer whose pointers are null or misaligned is left untouched). The
 * result is bit-identical to n_layers ix_gdn_commit_window calls. Requires 1 <= n_layers <=
 * 65535 and the same description requirements as ix_gdn_commit_window. */
hipError_t ix_gdn_commit_window_layers(const ix_gdn_cfg* cfg, int n_layers, int B, int K, const int32_t* accepted,
                                       const uint16_t* const* x, const void* const* record,
                                       uint16_t* const* conv_state, float* const* state,
                                       hipStream_t s IX_GDN_DEFAULT_STREAM);

/* ---------------------------------------------------------------------------------------
 * Projections feeding the layer
 * --------------------------------------------------------------------------------------- */

/* bf16 GEMV y[o] = sum_i x[i] * w[o][i], fp32 accumulation and result; w [n_out][n_in] bf16,
 * x [n_in] bf16. Replaces ix_bf16_gemv, src/ix_bf16_gemv.cu:90-101. Requires n_in > 0,
 * n_out > 0. Summation order is this library's own (within float tolerance of a double
 * reference); rows are 16-byte loads when n_in % 8 == 0 and x, w are 16-byte aligned. */
hipError_t ix_bf16_gemv(const uint16_t* x, const uint16_t* w, float* y, long long n_in, long long n_out,
                        hipStream_t s IX_GDN_DEFAULT_STREAM);

/* Two GEMVs sharing x: y1 = w1 x (n_out1 rows), y2 = w2 x (n_out2 rows). Replaces
 * ix_bf16_gemv_pair, src/ix_bf16_gemv.cu:103-111. Each result is bit-identical to
 * ix_bf16_gemv on the same operands. Requires n_in > 0 and n_out1 > 0 or n_out2 > 0. */
hipError_t ix_bf16_gemv_pair(const uint16_t* x, const uint16_t* w1, float* y1, long long n_out1, const uint16_t* w2,
                             float* y2, long long n_out2, long long n_in, hipStream_t s IX_GDN_DEFAULT_STREAM);

/* GEMV with threads_per_row threads cooperating on each row. Replaces ix_bf16_gemv_split,
 * src/ix_bf16_gemv.cu:113-126: 64 is one wave per row (bit-identical to ix_bf16_gemv);
 * otherwise a power of two up to 1024, else hipErrorInvalidValue. */
hipError_t ix_bf16_gemv_split(const uint16_t* x, const uint16_t* w, float* y, long long n_in, long long n_out,
                              int threads_per_row, hipStream_t s IX_GDN_DEFAULT_STREAM);

/* Q8_0 weights times q8_1 activations for ncols (1..8) activation columns. Replaces
 * ix_mmvq::ix_mmvq_q8_0, src/ix_mmvq_wave.cu:120-123 (formats :22-25):
 *   weights [n_out][n_in/32] Q8_0 blocks (fp16 scale, 32 int8; 34 bytes, 2-byte aligned)
 *   x_q8_1  [ncols][n_in/32] q8_1 blocks (fp16 scale, fp16 sum, 32 int8; 36 bytes, 4-byte aligned)
 *   y       [ncols][n_out] fp32 = sum over blocks of d_w * d_x * (integer dot of the block)
 * Requires n_in > 0, n_in % 32 == 0, n_out > 0, 1 <= ncols <= 8, non-NULL pointers. A
 * column's result does not depend on ncols. */
hipError_t ix_mmvq_q8_0(const void* weights, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                        hipStream_t s IX_GDN_DEFAULT_STREAM);

/* q8_1 quantiser of fp32 activations for ix_mmvq_q8_0 (addition; the reference has the format,
 * src/ix_mmvq_wave.cu:20-24, and the division rule every q8_1 producer shares,
 * src/ix_q81_div.h:1-9, but no quantiser). x [n] fp32 -> y_q8_1 [n/32] blocks of 36 bytes:
 * for each 32 consecutive values, d = max|x| / 127 (IEEE division), qs = roundf(x / d) (0 when
 * d is 0), s = the sum of the 32 values in xor-butterfly order (16, 8, 4, 2, 1),
 * d and s stored as fp16 (RNE). The gated calls' y_q8_1 output goes through the same device
 * function, so it equals this quantiser applied to their fp32 y, byte for byte. d and s are
 * clamped to fp16's largest finite value 65504 before the conversion (a block with
 * max|x| > 127 * 65504 gets d = 65504 and codes saturated at +-127; smaller blocks are
 * unaffected). Requires n > 0, n % 32 == 0, 4-byte aligned x and y_q8_1, finite x. */
hipError_t ix_q8_1_quantize(const float* x, void* y_q8_1, long long n, hipStream_t s IX_GDN_DEFAULT_STREAM);

/* Output width N of the layer's input projection: C + h_v*d_v + 2*h_v (x | z | a | b), or 0
 * for an invalid description. */
int ix_gdn_in_proj_width(const ix_gdn_cfg* cfg);

/* Input projection of B token rows (addition; no reference counterpart -- the reference runs
 * per-token GEMVs): y = h W^T with h [B][hidden] bf16, W [N][hidden] bf16 (N as above), fp32
 * accumulation on bf16 MFMA, written as bf16 (RNE) pieces x [B][C], z [B][h_v][d_v],
 * a [B][h_v], b [B][h_v] -- the inputs of ix_gdn_decode(_gated) and ix_gdn_prefill(_gated) --
 * and, when y is not NULL, as fp32 y [B][N]. Requires hidden % 64 == 0, h and W 16-byte
 * aligned. */
hipError_t ix_gdn_in_proj(const ix_gdn_cfg* cfg, int B, int hidden, const uint16_t* h, const uint16_t* w,
                          uint16_t* x, uint16_t* z, uint16_t* a, uint16_t* b, float* y,
                          hipStream_t s IX_GDN_DEFAULT_STREAM);

/* Library version string ("ixgdn 0.5.0 gfx950"). 0.5.0: ix_gdn_out_gate ends with y_q8_1, so
 * callers compiled against an older header must be rebuilt. */
const char* ix_gdn_version(void);

#ifdef __cplusplus
}
/* The reference declares its Q8_0 launcher in namespace ix_mmvq (src/ix_mmvq_wave.cu:120-123),
 * and its caller spells it ix_mmvq::ix_mmvq_q8_0 (tests/test_mmvq_wave.cu:46); that spelling
 * names the C-linkage entry point above. */
namespace ix_mmvq {
using ::ix_mmvq_q8_0;
}
#endif
#endif /* IX_GDN_H */
