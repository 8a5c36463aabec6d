// gdn_window.hip -- speculative windows for the fused GDN decode (gfx950):
// ix_gdn_decode_window verifies K draft tokens per sequence, ix_gdn_commit_window advances
// the committed state by the accepted prefix.
//
// A serving engine that drafts K tokens per sequence needs the layer's outputs for all K
// positions, and afterwards the recurrent and conv states after the first n_b accepted
// tokens (0 <= n_b <= K, per sequence). Keeping a snapshot of the 64 KiB-per-head state after
// every draft position costs K + 2 sweeps of the state per window. Here:
//  * verify reads the committed state once, carries it through the K tokens in registers
//    (the same column math as ix_gdn_decode, so every output is bit-identical to K decode
//    calls), writes the K outputs and a window record, and leaves both states untouched;
//  * commit replays the first n_b tokens of the record onto the committed state (one read
//    and one write of the heads whose n_b > 0; nothing at all for n_b = 0) and shifts the
//    conv history by the n_b accepted inputs.
// Three sweeps per window, whatever K is.
//
// Window record, fp32, for token t of sequence b (row = b*K + t):
//   k_hat [B*K][h_k][128]  the normalised key of each q/k head (the value ix_gdn_decode
//                          multiplies into the state)
//   v     [B*K][h_v][128]  the conv output of each v head's channels
//   g     [B*K][h_v]       the decay exp(-exp(A_log) softplus(a + dt_bias))
//   beta  [B*K][h_v]       sigmoid(b)
// Each section is 256-byte aligned, in that order (ix_gdn_window_record_size).
//
// Work decomposition as the decode's slab kernel: one workgroup per (sequence, v head,
// 64-column half tile), lane l holding rows 4(l & 31)..+3 of column (l >> 5) of 8 column
// pairs. No workgroup writes anything another reads, so neither kernel needs counters.
#include "gdn_common.h"

namespace ixg {
namespace {

constexpr int kThreads = 256;
constexpr int kHalf = 64;                                 // columns per workgroup
constexpr int kPairs = kHalf / 2 / (kThreads / kWave);    // 8 column pairs per wave
constexpr int kMaxWindow = 16;
// Extra LDS a capped commit launch reserves: with the kernel's own 12 KiB, more than a fifth of
// a CU's 160 KiB.
constexpr unsigned kCommitLdsReserve = 24000;

struct WinRec {
    float* k;       // [B*K][h_k][128]
    float* v;       // [B*K][h_v][128]
    float* g;       // [B*K][h_v]
    float* bt;      // [B*K][h_v]
};

__host__ __device__ inline size_t rec_layout(int B, int K, int h_k, int h_v, size_t (&off)[4]) {
    const size_t rows = (size_t)B * K;
    const size_t sz[4] = {rows * h_k * kD * 4, rows * h_v * kD * 4, rows * h_v * 4, rows * h_v * 4};
    size_t at = 0;
    for (int i = 0; i < 4; ++i) { off[i] = at; at += (sz[i] + 255) & ~(size_t)255; }
    return at;
}

__host__ __device__ inline WinRec rec_bind(void* base, int B, int K, int h_k, int h_v) {
    size_t off[4];
    rec_layout(B, K, h_k, h_v, off);
    char* c = static_cast<char*>(base);
    return WinRec{reinterpret_cast<float*>(c + off[0]), reinterpret_cast<float*>(c + off[1]),
                  reinterpret_cast<float*>(c + off[2]), reinterpret_cast<float*>(c + off[3])};
}

struct WindowParams {
    Layer L;
    int K;
    const uint16_t* x;            // [B][K][C]
    uint16_t* conv_state;         // [B][C][dc-1]
    const uint16_t* a;            // [B][K][h_v]
    const uint16_t* b;            // [B][K][h_v]
    float* state;                 // [B][h_v][d_v][d_k]
    float* o;                     // [B][K][h_v][128] or null
    uint16_t* o_bf16;             // [B][K][h_v][128] or null
    const int32_t* accepted;      // [B] (commit)
    WinRec rec;
};

// ---------------------------------------------------------------------------------------
// verify: grid (2 h_v, B)
// The per-token inputs (conv outputs, squared norms, gates) do not depend on the state, so
// they are computed for all K tokens first, into LDS, while the state loads are in flight;
// after one barrier the K column updates run back to back in registers. The arithmetic and
// its order are those of the decode kernel, token by token.
// ---------------------------------------------------------------------------------------
template <int DC>
__global__ void __launch_bounds__(kThreads) window_verify_kernel(const WindowParams p) {
    __shared__ __align__(16) float q_s[kMaxWindow][kD], k_s[kMaxWindow][kD], v_s[kMaxWindow][kHalf];
    __shared__ float sq_s[kMaxWindow], sk_s[kMaxWindow], g_s[kMaxWindow], b_s[kMaxWindow];

    const Layer& L = p.L;
    const int tid = threadIdx.x, w = tid / kWave, lane = tid & (kWave - 1);
    const int half = lane >> 5, i4 = lane & 31;
    const int hf = blockIdx.x & 1, h = blockIdx.x >> 1, bseq = blockIdx.y;
    const int src = src_of(L, h);
    const int K = p.K;
    // One workgroup per q/k head records its normalised key.
    const bool rec_k = hf == 0 && h == mapped_head(L, src, 0);

    // Conv channel pair of this thread: 0..63 q, 64..127 k, 128..159 the half tile's v.
    int ch = 0, col = 0;
    if (tid < 64) { ch = q_channel(L, src, 2 * tid); col = 2 * tid; }
    else if (tid < 128) { ch = k_channel(L, src, 2 * (tid - 64)); col = 2 * (tid - 64); }
    else if (tid < 128 + kHalf / 2) { ch = v_channel(L, h, hf * kHalf + 2 * (tid - 128)); col = 2 * (tid - 128); }
    const bool conv_thread = tid < 128 + kHalf / 2;
    ConvPair<DC> cp;
    // The inputs of all K tokens are loaded at once (rows past K repeat row K-1), so the
    // token loop below never waits for a load it issued itself.
    uint32_t xk[kMaxWindow];
    if (conv_thread) {
        const uint32_t* hp = reinterpret_cast<const uint32_t*>(p.conv_state + ((size_t)bseq * L.C + ch) * (DC - 1));
#pragma unroll
        for (int i = 0; i < DC - 1; ++i) cp.h[i] = hp[i];
        const uint32_t* wp = reinterpret_cast<const uint32_t*>(L.conv_w + (size_t)ch * DC);
#pragma unroll
        for (int i = 0; i < DC; ++i) cp.w[i] = wp[i];
#pragma unroll
        for (int t = 0; t < kMaxWindow; ++t)
            xk[t] = *reinterpret_cast<const uint32_t*>(p.x + ((size_t)bseq * K + min(t, K - 1)) * L.C + ch);
    }

    // Gate inputs, one token per thread of the last kMaxWindow, and the head's decay
    // parameters: loaded by every thread (clamped addresses) ahead of the state.
    const int gt = tid - (kThreads - kMaxWindow);
    const size_t ab = ((size_t)bseq * K + min(max(gt, 0), K - 1)) * L.h_v + h;
    const uint16_t a_in = p.a[ab], b_in = p.b[ab];
    const float a_log = L.A_log[h], dt_b = L.dt_bias[h];

    const v4f* tile = reinterpret_cast<const v4f*>(p.state + ((size_t)bseq * L.h_v + h) * kD * kD) + i4;
    const int j0 = hf * kHalf + 2 * kPairs * w + half;
    v4f s[kPairs];
#pragma unroll
    for (int u = 0; u < kPairs; ++u) s[u] = __builtin_nontemporal_load(tile + (size_t)(j0 + 2 * u) * (kD / 4));

    // Phase 1: conv outputs, squared norms (waves 0 and 1) and gates of every token.
    if (conv_thread) {
        float* dst = tid < 64 ? q_s[0] : tid < 128 ? k_s[0] : v_s[0];
        const int stride = tid < 128 ? kD : kHalf;
#pragma unroll
        for (int t = 0; t < kMaxWindow; ++t) {
            if (t >= K) break;
            float y0, y1;
            uint32_t nh[DC - 1];
            cp.x = xk[t];
            conv_pair_eval<DC>(L, cp, y0, y1, nh);
            dst[t * stride + col] = y0;
            dst[t * stride + col + 1] = y1;
#pragma unroll
            for (int i = 0; i < DC - 1; ++i) cp.h[i] = nh[i];
            if (w < 2) {                                       // wave-uniform: q (wave 0), k (wave 1)
                const float r = wave_sum(fmaf(y0, y0, y1 * y1));
                if (lane == 0) (w == 0 ? sq_s : sk_s)[t] = r;
            }
        }
    }
    if (gt >= 0 && gt < K) {                                  // gates: one thread per token
        g_s[gt] = expf(log_gate(a_log, dt_b, bf16_to_f32(a_in)));
        b_s[gt] = sigmoid_f(bf16_to_f32(b_in));
    }
    lds_barrier();

    // Phase 2: the K tokens in order, the state slab in registers.
    for (int t = 0; t < K; ++t) {
        const size_t row = (size_t)bseq * K + t;
        const float inv_q = L.q_scale / sqrtf(sq_s[t] + L.l2_eps);
        const float inv_k = 1.0f / sqrtf(sk_s[t] + L.l2_eps);
        const float kq =
            wave_sum(fmaf(q_s[t][lane], k_s[t][lane], q_s[t][lane + kWave] * k_s[t][lane + kWave])) * inv_q * inv_k;
        v4f kr, qr;
        {
            const v4f kk = *reinterpret_cast<const v4f*>(&k_s[t][4 * i4]), qq = *reinterpret_cast<const v4f*>(&q_s[t][4 * i4]);
#pragma unroll
            for (int e = 0; e < 4; ++e) { kr[e] = kk[e] * inv_k; qr[e] = qq[e] * inv_q; }
        }
        const float g = g_s[t], bt = b_s[t];
        const size_t ob = (row * L.h_v + h) * kD;
#pragma unroll
        for (int u = 0; u < kPairs; ++u) {
            const int j = j0 + 2 * u;
            float ak = s[u][0] * kr[0], aq = s[u][0] * qr[0];
#pragma unroll
            for (int e = 1; e < 4; ++e) { ak = fmaf(s[u][e], kr[e], ak); aq = fmaf(s[u][e], qr[e], aq); }
            ak = half_sum(ak);
            aq = half_sum(aq);
            const float d = (v_s[t][j - hf * kHalf] - g * ak) * bt;
#pragma unroll
            for (int e = 0; e < 4; ++e) s[u][e] = fmaf(kr[e], d, s[u][e] * g);
            if (i4 == 0) {
                const float ov = fmaf(d, kq, g * aq);
                if (p.o) p.o[ob + j] = ov;
                if (p.o_bf16) p.o_bf16[ob + j] = f32_to_bf16(ov);
            }
        }
        // The record of this token.
        if (rec_k && tid < kD) p.rec.k[(row * L.h_k + src) * kD + tid] = k_s[t][tid] * inv_k;
        if (tid < kHalf) p.rec.v[(row * L.h_v + h) * kD + hf * kHalf + tid] = v_s[t][tid];
        if (hf == 0 && tid == 0) { p.rec.g[row * L.h_v + h] = g; p.rec.bt[row * L.h_v + h] = bt; }
    }
}

// ---------------------------------------------------------------------------------------
// verify on the matrix cores (ix_gdn_decode_window_mfma): grid (2 h_v, B), the workgroups of
// window_verify_kernel. With S the committed state, G_t = g_0 g_1 ... g_t and
// r(t, s) = g_{s+1} ... g_t (r(t, t) = 1), the K steps unroll to
//   d_t = beta_t (v_t - G_t (S^T k_t) - sum_{s<t} r(t, s) (k_t . k_s) d_s)
//   o_t = G_t (S^T q_t) + sum_{s<=t} r(t, s) (q_t . k_s) d_s
// (k, q normalised; q with its scale). The state enters only through the 2K products
// S^T k_t and S^T q_t: one split-bf16 MFMA product per wave with the state as the A operand
// (lane (li, lg) of wave w holds column j = 64 hf + 16 w + li at key rows 32 ks + kperm(lg, e)),
// loaded from HBM in whole lines, passed through the wave's own LDS tile into that layout,
// and never stored. The K x K
// products k_t . k_s and q_t . k_s come from the same token fragments. Each column then runs
// the K-step recurrence above in fp32. Outputs agree with K ix_gdn_decode calls to fp32
// rounding (not bit for bit); the record is computed exactly as window_verify_kernel computes
// it, so ix_gdn_commit_window gives the same committed states after either verify.
// ---------------------------------------------------------------------------------------
template <int DC, int KMAX>
__global__ void __launch_bounds__(kThreads, KMAX <= 8 ? 5 : 1) window_mfma_kernel(const WindowParams p) {
    static_assert(KMAX == 4 || KMAX == 8 || KMAX == 16, "window size class");
    constexpr int KP = KMAX + 1;                              // padded row of the token tables
    // q and k rows padded to 132 floats: the token fragments read 16 rows at one column
    // offset with 16-byte reads, which then meet in at most two ways per bank.
    constexpr int QS = kD + 4;
    __shared__ __align__(16) float q_s[KMAX][QS], k_s[KMAX][QS], v_s[KMAX][kHalf];
    __shared__ float sq_s[KMAX], sk_s[KMAX], g_s[KMAX], b_s[KMAX];
    __shared__ float kk_s[KMAX][KP], qk_s[KMAX][KP];         // k_t . k_s, q_t . k_s
    __shared__ float sk_t[kHalf][KP], sq_t[kHalf][KP];       // S^T k_t, S^T q_t per column
    // Each wave's 16 state columns, 32 rows (one k-step) at a time, column-major with rows
    // padded to SR floats: the coalesced loads write it and the fragment reads take it back
    // out, both without bank conflicts.
    constexpr int SR = 32 + 4;
    __shared__ __align__(16) float st_s[kThreads / kWave][16 * SR];

    const Layer& L = p.L;
    const int tid = threadIdx.x, w = tid / kWave, lane = tid & (kWave - 1);
    const int li = lane & 15, lg = lane >> 4;
    const int hf = blockIdx.x & 1, h = blockIdx.x >> 1, bseq = blockIdx.y;
    const int src = src_of(L, h);
    const int K = p.K;
    const bool rec_k = hf == 0 && h == mapped_head(L, src, 0);

    // Conv channel pair of this thread: 0..63 q, 64..127 k, 128..159 the half tile's v; the
    // inputs of all K tokens at once (rows past K repeat row K-1).
    int ch = 0, col = 0;
    if (tid < 64) { ch = q_channel(L, src, 2 * tid); col = 2 * tid; }
    else if (tid < 128) { ch = k_channel(L, src, 2 * (tid - 64)); col = 2 * (tid - 64); }
    else if (tid < 128 + kHalf / 2) { ch = v_channel(L, h, hf * kHalf + 2 * (tid - 128)); col = 2 * (tid - 128); }
    const bool conv_thread = tid < 128 + kHalf / 2;
    ConvPair<DC> cp;
    uint32_t xk[KMAX];
    if (conv_thread) {
        const uint32_t* hp = reinterpret_cast<const uint32_t*>(p.conv_state + ((size_t)bseq * L.C + ch) * (DC - 1));
#pragma unroll
        for (int i = 0; i < DC - 1; ++i) cp.h[i] = hp[i];
        const uint32_t* wp = reinterpret_cast<const uint32_t*>(L.conv_w + (size_t)ch * DC);
#pragma unroll
        for (int i = 0; i < DC; ++i) cp.w[i] = wp[i];
#pragma unroll
        for (int t = 0; t < KMAX; ++t)
            xk[t] = *reinterpret_cast<const uint32_t*>(p.x + ((size_t)bseq * K + min(t, K - 1)) * L.C + ch);
    }
    // Gate inputs, one token per thread of the last KMAX, and the head's decay parameters:
    // loaded by every thread (clamped addresses) ahead of the state, so that no branch waits
    // for them before the state loads go out and the gates do not wait for the state.
    const int gt = tid - (kThreads - KMAX);
    const size_t ab = ((size_t)bseq * K + min(max(gt, 0), K - 1)) * L.h_v + h;
    const uint16_t a_in = p.a[ab], b_in = p.b[ab];
    const float a_log = L.A_log[h], dt_b = L.dt_bias[h];

    // The wave's 16 state columns in whole 128-byte lines: load 2 ks + c8 brings column
    // 16 w + 8 c8 + lane / 8, rows 32 ks + 4 (lane % 8) .. + 3, i.e. eight whole lines per
    // instruction. The fragment layout (one column per li) is reached through the wave's
    // LDS tile in the product loop.
    const float* wcol = p.state + (((size_t)bseq * L.h_v + h) * kD + hf * kHalf + 16 * w + (lane >> 3)) * kD + 4 * (lane & 7);
    v4f sraw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        sraw[i] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(wcol + 8 * (i & 1) * kD + 32 * (i >> 1)));

    // Phase 1: conv outputs, squared norms (waves 0 and 1) and gates of every token.
    if (conv_thread) {
        float* dst = tid < 64 ? q_s[0] : tid < 128 ? k_s[0] : v_s[0];
        const int stride = tid < 128 ? QS : kHalf;
#pragma unroll
        for (int t = 0; t < KMAX; ++t) {
            if (t >= K) break;
            float y0, y1;
            uint32_t nh[DC - 1];
            cp.x = xk[t];
            conv_pair_eval<DC>(L, cp, y0, y1, nh);
            dst[t * stride + col] = y0;
            dst[t * stride + col + 1] = y1;
#pragma unroll
            for (int i = 0; i < DC - 1; ++i) cp.h[i] = nh[i];
            if (w < 2) {                                       // wave-uniform: q (wave 0), k (wave 1)
                const float r = wave_sum(fmaf(y0, y0, y1 * y1));
                if (lane == 0) (w == 0 ? sq_s : sk_s)[t] = r;
            }
        }
    }
    if (gt >= 0 && gt < K) {
        g_s[gt] = expf(log_gate(a_log, dt_b, bf16_to_f32(a_in)));
        b_s[gt] = sigmoid_f(bf16_to_f32(b_in));
    }
    lds_barrier();

    // Token fragments: the normalised k_t and q_t (the decode kernel's inverse norms) at this
    // lane's key rows. Up to 8 tokens share one 16-wide operand tile: column n < K is k_n,
    // K <= n < 2K is q_{n-K}; beyond that two tiles hold k (column n = token n) and q. With
    // the state fragments as A: S^T k and S^T q for this wave's 16 columns. The token
    // fragments also serve as A operands (row li of an A operand holds the same values):
    // wave 1 forms the token products k_t . k_s and q_t . k_s.
    v4 ak = {0.f, 0.f, 0.f, 0.f}, aq = ak, kk = ak, qk = ak;
    constexpr bool kShared = KMAX <= 8;
    // fragment 0: k_li (or, shared, k_li | q_{li-K}); fragment 1: q_li (unshared) or k_li (the B of k . k, q . k)
    const bool is_k0 = li < K, is_q0 = kShared && li >= K && li < 2 * K;
    const int row0 = is_k0 ? li : is_q0 ? li - K : 0;
    const float s0 = is_k0 ? 1.0f / sqrtf(sk_s[row0] + L.l2_eps)
                           : is_q0 ? L.q_scale / sqrtf(sq_s[row0] + L.l2_eps) : 0.0f;
    const float* base0 = is_q0 ? q_s[row0] : k_s[row0];
    const bool tok1 = li < K;
    const int row1 = tok1 ? li : 0;
    const float s1 = tok1 ? (kShared ? 1.0f / sqrtf(sk_s[row1] + L.l2_eps) : L.q_scale / sqrtf(sq_s[row1] + L.l2_eps))
                          : 0.0f;
    const float* base1 = kShared ? k_s[row1] : q_s[row1];
    float* tile = st_s[w];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        // Rows 32 ks .. 32 ks + 31 into the tile, then this lane's fragment rows back out.
#pragma unroll
        for (int c8 = 0; c8 < 2; ++c8)
            *reinterpret_cast<v4f*>(tile + (8 * c8 + (lane >> 3)) * SR + 4 * (lane & 7)) = sraw[2 * ks + c8];
        wave_lds_sync();
        const v4f st0 = *reinterpret_cast<const v4f*>(tile + li * SR + 4 * lg);
        const v4f st1 = *reinterpret_cast<const v4f*>(tile + li * SR + 4 * lg + 16);
        wave_lds_sync();                                        // read before the next rows are written
        float x0[8], x1[8], sx[8];
        const int i0 = 32 * ks + 4 * lg;                        // kperm: rows i0..i0+3, i0+16..i0+19
        const v4f a0 = *reinterpret_cast<const v4f*>(base0 + i0), a1 = *reinterpret_cast<const v4f*>(base0 + i0 + 16);
        const v4f c0 = *reinterpret_cast<const v4f*>(base1 + i0), c1 = *reinterpret_cast<const v4f*>(base1 + i0 + 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x0[e] = a0[e] * s0;
            x0[e + 4] = a1[e] * s0;
            x1[e] = c0[e] * s1;
            x1[e + 4] = c1[e] * s1;
            sx[e] = st0[e];
            sx[e + 4] = st1[e];
        }
        bf8 h0, l0, h1, l1, sh, sl;
        split8(x0, h0, l0);
        split8(x1, h1, l1);
        split8(sx, sh, sl);
        ak = mfma_split(sh, sl, h0, l0, ak);
        if constexpr (kShared) {
            if (w == 1) kk = mfma_split(h0, l0, h1, l1, kk);       // rows k_t then q_t, columns k_s
        } else {
            aq = mfma_split(sh, sl, h1, l1, aq);
            if (w == 1) kk = mfma_split(h0, l0, h0, l0, kk);
            if (w == 2) qk = mfma_split(h1, l1, h0, l0, qk);
        }
    }
    // The record, exactly as window_verify_kernel writes it. Its stores go out once the state
    // has been consumed: issued among the state loads, they would be waited for with them.
    for (int t = 0; t < K; ++t) {
        const size_t row = (size_t)bseq * K + t;
        if (rec_k && tid < kD) p.rec.k[(row * L.h_k + src) * kD + tid] = k_s[t][tid] * (1.0f / sqrtf(sk_s[t] + L.l2_eps));
        if (tid < kHalf) p.rec.v[(row * L.h_v + h) * kD + hf * kHalf + tid] = v_s[t][tid];
        if (hf == 0 && tid == 0) { p.rec.g[row * L.h_v + h] = g_s[t]; p.rec.bt[row * L.h_v + h] = b_s[t]; }
    }
    // Accumulator element r of lane (li, lg) is row 4 lg + r, column li.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int jr = 16 * w + 4 * lg + r, n = 4 * lg + r;
        if constexpr (kShared) {
            if (li < K) sk_t[jr][li] = ak[r];
            else if (li < 2 * K) sq_t[jr][li - K] = ak[r];
            if (w == 1 && li < K) {
                if (n < K) kk_s[n][li] = kk[r];
                else if (n < 2 * K) qk_s[n - K][li] = kk[r];
            }
        } else {
            if (li < KMAX) { sk_t[jr][li] = ak[r]; sq_t[jr][li] = aq[r]; }
            if (li < KMAX && n < KMAX) {
                if (w == 1) kk_s[n][li] = kk[r];
                if (w == 2) qk_s[n][li] = qk[r];
            }
        }
    }
    lds_barrier();

    // Phase 2: the K-step recurrence of each column (threads 0..63), outputs as they come.
    // G_t and r(t, s) are running products of the decays (no division: G_t may underflow).
    if (tid < kHalf) {
        const int j = hf * kHalf + tid;
        float d[KMAX], r[KMAX];
        float G = 1.0f;
#pragma unroll
        for (int t = 0; t < KMAX; ++t) {
            if (t >= K) break;
            const float g = g_s[t];
            G *= g;
#pragma unroll
            for (int s2 = 0; s2 < t; ++s2) r[s2] = s2 == t - 1 ? g : r[s2] * g;   // r(t, s) = r(t-1, s) g_t
            float u = G * sk_t[tid][t];
#pragma unroll
            for (int s2 = 0; s2 < t; ++s2) u = fmaf(r[s2] * kk_s[t][s2], d[s2], u);
            d[t] = (v_s[t][tid] - u) * b_s[t];
            float ov = fmaf(qk_s[t][t], d[t], G * sq_t[tid][t]);
#pragma unroll
            for (int s2 = 0; s2 < t; ++s2) ov = fmaf(r[s2] * qk_s[t][s2], d[s2], ov);
            const size_t ob = (((size_t)bseq * K + t) * L.h_v + h) * kD + j;
            if (p.o) p.o[ob] = ov;
            if (p.o_bf16) p.o_bf16[ob] = f32_to_bf16(ov);
        }
    }
}

// The window size class KMAX (4, 8 or 16 tokens) sizes the LDS tables and the registers.
template <int KMAX>
void launch_window_mfma(const ix_gdn_cfg* cfg, int B, const WindowParams& p, hipStream_t s) {
    const dim3 grid((unsigned)(2 * cfg->h_v), (unsigned)B), block(kThreads);
    switch (cfg->d_conv) {
        case 2: hipLaunchKernelGGL((window_mfma_kernel<2, KMAX>), grid, block, 0, s, p); break;
        case 3: hipLaunchKernelGGL((window_mfma_kernel<3, KMAX>), grid, block, 0, s, p); break;
        default: hipLaunchKernelGGL((window_mfma_kernel<4, KMAX>), grid, block, 0, s, p); break;
    }
}

// ---------------------------------------------------------------------------------------
// commit: grid (2 h_v, B)
// ---------------------------------------------------------------------------------------
// One workgroup's share of a commit: v head h, half tile hf, sequence bseq of the layer whose
// x, conv state, state and record p holds.
__device__ __forceinline__ void commit_tile(const WindowParams& p, int h, int hf, int bseq) {
    __shared__ __align__(16) float k_s[kMaxWindow][kD], v_s[kMaxWindow][kHalf];
    __shared__ float g_s[kMaxWindow], b_s[kMaxWindow];
    const Layer& L = p.L;
    const int tid = threadIdx.x, w = tid / kWave, lane = tid & (kWave - 1);
    const int half = lane >> 5, i4 = lane & 31;
    const int src = src_of(L, h);
    const int n = min(max(p.accepted[bseq], 0), p.K);
    if (n == 0) return;                                      // nothing accepted: both states stay
    const int dm = L.dc - 1;
    const size_t row0 = (size_t)bseq * p.K;

    // Every load is issued before anything waits: this workgroup's share of the record of
    // the n accepted tokens (key, the half tile's 64 values, gate, beta), the conv history
    // inputs, then the state. Indices are clamped, so the loads are unconditional; only the
    // stores are predicated.
    v4f kq[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int e = min(tid + r * kThreads, n * (kD / 4) - 1), t = e / (kD / 4), c4 = e % (kD / 4);
        kq[r] = *reinterpret_cast<const v4f*>(p.rec.k + ((row0 + t) * L.h_k + src) * kD + 4 * c4);
    }
    v4f vq;
    {
        const int e = min(tid, n * (kHalf / 4) - 1), t = e / (kHalf / 4), c4 = e % (kHalf / 4);
        vq = *reinterpret_cast<const v4f*>(p.rec.v + ((row0 + t) * L.h_v + h) * kD + hf * kHalf + 4 * c4);
    }
    const int tg = min(tid, n - 1);
    const float gq = p.rec.g[(row0 + tg) * L.h_v + h], bq = p.rec.bt[(row0 + tg) * L.h_v + h];

    // Conv history: the half tile's 64 v channels, and (one workgroup per q/k head) the 256
    // q and k channels. New history = the last dc-1 entries of (old history, x_0..x_{n-1}).
    const bool own_qk = hf == 0 && h == mapped_head(L, src, 0);
    const int nch = kHalf + (own_qk ? 2 * kD : 0);
    uint16_t hnew[2][3];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int e = min(tid + r * kThreads, nch - 1);
        const int c = e < kHalf ? v_channel(L, h, hf * kHalf + e)
                                : (e < kHalf + kD ? q_channel(L, src, e - kHalf) : k_channel(L, src, e - kHalf - kD));
        const uint16_t* hp = p.conv_state + ((size_t)bseq * L.C + c) * dm;
        uint16_t old[3], xin[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            old[i] = hp[min(i, dm - 1)];
            xin[i] = p.x[(row0 + min(max(n + i - dm, 0), p.K - 1)) * L.C + c];
        }
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int idx = n + i;                           // index into (old history, x_0, x_1, ...)
            hnew[r][i] = idx < dm ? (idx == 0 ? old[0] : idx == 1 ? old[1] : old[2]) : xin[i];
        }
    }

    v4f* tile = reinterpret_cast<v4f*>(p.state + ((size_t)bseq * L.h_v + h) * kD * kD) + i4;
    const int j0 = hf * kHalf + 2 * kPairs * w + half;
    v4f s[kPairs];
#pragma unroll
    for (int u = 0; u < kPairs; ++u) s[u] = __builtin_nontemporal_load(tile + (size_t)(j0 + 2 * u) * (kD / 4));

#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int e = tid + r * kThreads;
        if (e < n * (kD / 4)) *reinterpret_cast<v4f*>(&k_s[e / (kD / 4)][4 * (e % (kD / 4))]) = kq[r];
    }
    if (tid < n * (kHalf / 4)) *reinterpret_cast<v4f*>(&v_s[tid / (kHalf / 4)][4 * (tid % (kHalf / 4))]) = vq;
    if (tid < n) {
        g_s[tid] = gq;
        b_s[tid] = bq;
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int e = tid + r * kThreads;
        if (e >= nch) continue;
        const int c = e < kHalf ? v_channel(L, h, hf * kHalf + e)
                                : (e < kHalf + kD ? q_channel(L, src, e - kHalf) : k_channel(L, src, e - kHalf - kD));
        uint16_t* hp = p.conv_state + ((size_t)bseq * L.C + c) * dm;
#pragma unroll
        for (int i = 0; i < 3; ++i)
            if (i < dm) hp[i] = hnew[r][i];
    }
    lds_barrier();

    for (int t = 0; t < n; ++t) {
        const v4f kr = *reinterpret_cast<const v4f*>(&k_s[t][4 * i4]);
        const float g = g_s[t], bt = b_s[t];
#pragma unroll
        for (int u = 0; u < kPairs; ++u) {
            float ak = s[u][0] * kr[0];
#pragma unroll
            for (int e = 1; e < 4; ++e) ak = fmaf(s[u][e], kr[e], ak);
            ak = half_sum(ak);
            const float d = (v_s[t][j0 + 2 * u - hf * kHalf] - g * ak) * bt;
#pragma unroll
            for (int e = 0; e < 4; ++e) s[u][e] = fmaf(kr[e], d, s[u][e] * g);
        }
    }
#pragma unroll
    for (int u = 0; u < kPairs; ++u) __builtin_nontemporal_store(s[u], tile + (size_t)(j0 + 2 * u) * (kD / 4));
}

__global__ void __launch_bounds__(kThreads) window_commit_kernel(const WindowParams p) {
    commit_tile(p, blockIdx.x >> 1, blockIdx.x & 1, blockIdx.y);
}

// Per-layer buffers of a multi-layer commit: device arrays of n_layers pointers each.
struct LayerPtrs {
    const uint16_t* const* x;
    const void* const* record;
    uint16_t* const* conv_state;
    float* const* state;
};

// grid (2 h_v, B, n_layers): blockIdx.z picks the layer, whose pointers come from the device
// arrays; the work of each (layer, head, half tile, sequence) is the single-layer commit's.
// A layer whose pointers are null or misaligned (state 16 bytes, record 256 bytes) is skipped.
__global__ void __launch_bounds__(kThreads) window_commit_layers_kernel(const WindowParams base, const LayerPtrs lp,
                                                                      int B) {
    const int l = blockIdx.z;
    WindowParams p = base;
    p.x = lp.x[l];
    p.conv_state = lp.conv_state[l];
    p.state = lp.state[l];
    void* rec = const_cast<void*>(lp.record[l]);
    if (!p.x || !p.conv_state || !p.state || !rec || (reinterpret_cast<uintptr_t>(p.state) & 15) ||
        (reinterpret_cast<uintptr_t>(rec) & 255))
        return;
    p.rec = rec_bind(rec, B, p.K, p.L.h_k, p.L.h_v);
    commit_tile(p, blockIdx.x >> 1, blockIdx.x & 1, blockIdx.y);
}

}  // namespace
}  // namespace ixg

extern "C" hipError_t ix_gdn_check_cfg_(const ix_gdn_cfg* c);

extern "C" size_t ix_gdn_window_record_size(const ix_gdn_cfg* cfg, int B, int K) {
    if (ix_gdn_check_cfg_(cfg) != hipSuccess || B <= 0 || B > 65535 || K <= 0 || K > ixg::kMaxWindow) return 0;
    size_t off[4];
    return ixg::rec_layout(B, K, cfg->h_k, cfg->h_v, off);
}

static hipError_t window_params(const ix_gdn_cfg* cfg, int B, int K, const uint16_t* x, uint16_t* conv_state,
                                const uint16_t* conv_w, float* state, void* record, ixg::WindowParams& p) {
    const hipError_t e = ix_gdn_check_cfg_(cfg);
    if (e != hipSuccess) return e;
    if (B <= 0 || B > 65535 || K <= 0 || K > ixg::kMaxWindow) return hipErrorInvalidValue;
    // Every q/k head must feed a v head: the workgroups of its first v head carry its conv
    // history and record its key.
    if (cfg->head_map == IX_GDN_HEAD_MOD && cfg->h_v < cfg->h_k) return hipErrorInvalidValue;
    if (!x || !conv_state || !state || !record) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(state) & 15) || (reinterpret_cast<uintptr_t>(record) & 255))
        return hipErrorInvalidValue;
    p = ixg::WindowParams{};
    p.L = ixg::make_layer(cfg, conv_w, nullptr, nullptr);
    p.K = K;
    p.x = x; p.conv_state = conv_state; p.state = state;
    p.rec = ixg::rec_bind(record, B, K, cfg->h_k, cfg->h_v);
    return hipSuccess;
}

// Validation and parameters shared by the two verify entry points.
static hipError_t verify_params(const ix_gdn_cfg* cfg, int B, int K, const uint16_t* x, const uint16_t* conv_state,
                                const uint16_t* conv_w, const uint16_t* a, const uint16_t* b, const float* A_log,
                                const float* dt_bias, const float* state, float* o, uint16_t* o_bf16, void* record,
                                ixg::WindowParams& p) {
    const hipError_t e = window_params(cfg, B, K, x, const_cast<uint16_t*>(conv_state), conv_w,
                                       const_cast<float*>(state), record, p);
    if (e != hipSuccess) return e;
    if (!conv_w || !a || !b || !A_log || !dt_bias) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(conv_state) |
         reinterpret_cast<uintptr_t>(conv_w)) & 3)
        return hipErrorInvalidValue;                 // conv inputs are read as dwords
    if ((o && (reinterpret_cast<uintptr_t>(o) & 3)) || (o_bf16 && (reinterpret_cast<uintptr_t>(o_bf16) & 1)))
        return hipErrorInvalidValue;
    p.L.A_log = A_log; p.L.dt_bias = dt_bias;
    p.a = a; p.b = b; p.o = o; p.o_bf16 = o_bf16;
    return hipSuccess;
}

extern "C" hipError_t ix_gdn_decode_window(const ix_gdn_cfg* cfg, int B, int K, const uint16_t* x,
                                           const uint16_t* conv_state, const uint16_t* conv_w, const uint16_t* a,
                                           const uint16_t* b, const float* A_log, const float* dt_bias,
                                           const float* state, float* o, uint16_t* o_bf16, void* record,
                                           hipStream_t s) {
    ixg::WindowParams p;
    const hipError_t e = verify_params(cfg, B, K, x, conv_state, conv_w, a, b, A_log, dt_bias, state, o, o_bf16,
                                       record, p);
    if (e != hipSuccess) return e;
    const dim3 grid((unsigned)(2 * cfg->h_v), (unsigned)B), block(ixg::kThreads);
    switch (cfg->d_conv) {
        case 2: hipLaunchKernelGGL(ixg::window_verify_kernel<2>, grid, block, 0, s, p); break;
        case 3: hipLaunchKernelGGL(ixg::window_verify_kernel<3>, grid, block, 0, s, p); break;
        default: hipLaunchKernelGGL(ixg::window_verify_kernel<4>, grid, block, 0, s, p); break;
    }
    return hipGetLastError();
}

extern "C" hipError_t ix_gdn_decode_window_mfma(const ix_gdn_cfg* cfg, int B, int K, const uint16_t* x,
                                                const uint16_t* conv_state, const uint16_t* conv_w, const uint16_t* a,
                                                const uint16_t* b, const float* A_log, const float* dt_bias,
                                                const float* state, float* o, uint16_t* o_bf16, void* record,
                                                hipStream_t s) {
    ixg::WindowParams p;
    const hipError_t e = verify_params(cfg, B, K, x, conv_state, conv_w, a, b, A_log, dt_bias, state, o, o_bf16,
                                       record, p);
    if (e != hipSuccess) return e;
    if (K <= 4) ixg::launch_window_mfma<4>(cfg, B, p, s);
    else if (K <= 8) ixg::launch_window_mfma<8>(cfg, B, p, s);
    else ixg::launch_window_mfma<16>(cfg, B, p, s);
    return hipGetLastError();
}

extern "C" hipError_t ix_gdn_commit_window(const ix_gdn_cfg* cfg, int B, int K, const int32_t* accepted,
                                           const uint16_t* x, const void* record, uint16_t* conv_state,
                                           float* state, hipStream_t s) {
    ixg::WindowParams p;
    const hipError_t e = window_params(cfg, B, K, x, conv_state, nullptr, state, const_cast<void*>(record), p);
    if (e != hipSuccess) return e;
    if (!accepted) return hipErrorInvalidValue;
    p.accepted = accepted;
    // With at least 8 workgroups per CU to run (B >= 32 at h_v = 32), the launch reserves LDS that
    // no code touches, so that at most four workgroups share a CU (the decode's slab kernel does
    // the same with two): B = 64 47.5 against 48.1 us, B = 128 89.0 against 90.5; equal at
    // B = 32, slower at B = 16.
    const long long nwg = 2LL * cfg->h_v * B;
    const unsigned lds = nwg >= 8LL * ixg::device_cu_count(s) ? ixg::kCommitLdsReserve : 0;
    hipLaunchKernelGGL(ixg::window_commit_kernel, dim3((unsigned)(2 * cfg->h_v), (unsigned)B), dim3(ixg::kThreads),
                       lds, s, p);
    return hipGetLastError();
}

extern "C" hipError_t ix_gdn_commit_window_layers(const ix_gdn_cfg* cfg, int n_layers, int B, int K,
                                                  const int32_t* accepted, const uint16_t* const* x,
                                                  const void* const* record, uint16_t* const* conv_state,
                                                  float* const* state, hipStream_t s) {
    const hipError_t e = ix_gdn_check_cfg_(cfg);
    if (e != hipSuccess) return e;
    if (n_layers <= 0 || n_layers > 65535 || B <= 0 || B > 65535 || K <= 0 || K > ixg::kMaxWindow)
        return hipErrorInvalidValue;
    if (cfg->head_map == IX_GDN_HEAD_MOD && cfg->h_v < cfg->h_k) return hipErrorInvalidValue;
    if (!accepted || !x || !record || !conv_state || !state) return hipErrorInvalidValue;
    ixg::WindowParams p{};
    p.L = ixg::make_layer(cfg, nullptr, nullptr, nullptr);
    p.K = K;
    p.accepted = accepted;
    const ixg::LayerPtrs lp{x, record, conv_state, state};
    const long long nwg = 2LL * cfg->h_v * B * n_layers;
    const unsigned lds = nwg >= 8LL * ixg::device_cu_count(s) ? ixg::kCommitLdsReserve : 0;
    hipLaunchKernelGGL(ixg::window_commit_layers_kernel, dim3((unsigned)(2 * cfg->h_v), (unsigned)B, (unsigned)n_layers),
                       dim3(ixg::kThreads), lds, s, p, lp, B);
    return hipGetLastError();
}
