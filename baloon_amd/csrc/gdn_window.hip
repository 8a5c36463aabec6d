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

struct WinRec {
    float* k;       // [B*K][h_k][128]
    float* v;       // [B*K][h_v][128]
    float* g;       // [B*K][h_v]
    float* bt;      // [B*K][h_v]
};

inline size_t rec_layout(int B, int K, int h_k, int h_v, size_t (&off)[4]) {
    const size_t rows = (size_t)B * K;
    const size_t sz[4] = {rows * h_k * kD * 4, rows * h_v * kD * 4, rows * h_v * 4, rows * h_v * 4};
    size_t at = 0;
    for (int i = 0; i < 4; ++i) { off[i] = at; at += (sz[i] + 255) & ~(size_t)255; }
    return at;
}

inline WinRec rec_bind(void* base, int B, int K, int h_k, int h_v) {
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
    if (tid >= kThreads - kMaxWindow) {                       // gates: one thread per token
        const int t = tid - (kThreads - kMaxWindow);
        if (t < K) {
            const size_t ab = ((size_t)bseq * K + t) * L.h_v + h;
            g_s[t] = expf(log_gate(L, h, bf16_to_f32(p.a[ab])));
            b_s[t] = sigmoid_f(bf16_to_f32(p.b[ab]));
        }
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
// commit: grid (2 h_v, B)
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(kThreads) window_commit_kernel(const WindowParams p) {
    const Layer& L = p.L;
    const int tid = threadIdx.x, w = tid / kWave, lane = tid & (kWave - 1);
    const int half = lane >> 5, i4 = lane & 31;
    const int hf = blockIdx.x & 1, h = blockIdx.x >> 1, bseq = blockIdx.y;
    const int src = src_of(L, h);
    const int n = min(max(p.accepted[bseq], 0), p.K);
    if (n == 0) return;                                      // nothing accepted: both states stay
    const int dm = L.dc - 1;

    // Conv history: the half tile's 64 v channels, and (one workgroup per q/k head) the 256
    // q and k channels. New history = the last dc-1 entries of (old history, x_0..x_{n-1}).
    const bool own_qk = hf == 0 && h == mapped_head(L, src, 0);
    const int nch = kHalf + (own_qk ? 2 * kD : 0);
    for (int e = tid; e < nch; e += kThreads) {
        const int c = e < kHalf ? v_channel(L, h, hf * kHalf + e)
                                : (e < kHalf + kD ? q_channel(L, src, e - kHalf) : k_channel(L, src, e - kHalf - kD));
        uint16_t* hp = p.conv_state + ((size_t)bseq * L.C + c) * dm;
        uint16_t old[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) old[i] = i < dm ? hp[i] : 0;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            if (i >= dm) break;
            const int idx = n + i;                           // index into (old history, x_0, x_1, ...)
            hp[i] = idx < dm ? (idx == 0 ? old[0] : idx == 1 ? old[1] : old[2])
                             : p.x[((size_t)bseq * p.K + (idx - dm)) * L.C + c];
        }
    }

    v4f* tile = reinterpret_cast<v4f*>(p.state + ((size_t)bseq * L.h_v + h) * kD * kD) + i4;
    const int j0 = hf * kHalf + 2 * kPairs * w + half;
    v4f s[kPairs];
#pragma unroll
    for (int u = 0; u < kPairs; ++u) s[u] = __builtin_nontemporal_load(tile + (size_t)(j0 + 2 * u) * (kD / 4));
    for (int t = 0; t < n; ++t) {
        const size_t row = (size_t)bseq * p.K + t;
        const v4f kr = *reinterpret_cast<const v4f*>(p.rec.k + (row * L.h_k + src) * kD + 4 * i4);
        const float g = p.rec.g[row * L.h_v + h], bt = p.rec.bt[row * L.h_v + h];
        const float* vr = p.rec.v + (row * L.h_v + h) * kD;
#pragma unroll
        for (int u = 0; u < kPairs; ++u) {
            float ak = s[u][0] * kr[0];
#pragma unroll
            for (int e = 1; e < 4; ++e) ak = fmaf(s[u][e], kr[e], ak);
            ak = half_sum(ak);
            const float d = (vr[j0 + 2 * u] - g * ak) * bt;
#pragma unroll
            for (int e = 0; e < 4; ++e) s[u][e] = fmaf(kr[e], d, s[u][e] * g);
        }
    }
#pragma unroll
    for (int u = 0; u < kPairs; ++u) __builtin_nontemporal_store(s[u], tile + (size_t)(j0 + 2 * u) * (kD / 4));
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

extern "C" hipError_t ix_gdn_decode_window(const ix_gdn_cfg* cfg, int B, int K, const uint16_t* x,
                                           const uint16_t* conv_state, const uint16_t* conv_w, const uint16_t* a,
                                           const uint16_t* b, const float* A_log, const float* dt_bias,
                                           const float* state, float* o, uint16_t* o_bf16, void* record,
                                           hipStream_t s) {
    ixg::WindowParams p;
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
    const dim3 grid((unsigned)(2 * cfg->h_v), (unsigned)B), block(ixg::kThreads);
    switch (cfg->d_conv) {
        case 2: hipLaunchKernelGGL(ixg::window_verify_kernel<2>, grid, block, 0, s, p); break;
        case 3: hipLaunchKernelGGL(ixg::window_verify_kernel<3>, grid, block, 0, s, p); break;
        default: hipLaunchKernelGGL(ixg::window_verify_kernel<4>, grid, block, 0, s, p); break;
    }
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
    hipLaunchKernelGGL(ixg::window_commit_kernel, dim3((unsigned)(2 * cfg->h_v), (unsigned)B), dim3(ixg::kThreads),
                       0, s, p);
    return hipGetLastError();
}
