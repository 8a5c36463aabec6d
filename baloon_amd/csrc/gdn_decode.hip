// gdn_decode.hip -- fused, batched GDN decode for gfx950 (ix_gdn_decode).
//
// One launch does a whole GDN layer's recurrent part for one token of B sequences:
// causal depthwise conv (rolling state) over the q|k|v channels, L2 norm of q and k, the
// gates g = exp(-exp(A_log) softplus(a + dt_bias)) and beta = sigmoid(b), the head map, and
// the delta-rule update of the fp32 state with output o = S'^T q. The reference does these
// as separate launches (src/ix_gdn.cu:58-70, :73-84, :102-105, :25-56) and has no batch.
//
// Work decomposition: one workgroup per (sequence b, q/k head src). It owns the q and k
// channels of src and every v head mapped to src, so each conv-state channel and each state
// tile is read and written by exactly one workgroup: the in-place updates are race free
// without any cross-workgroup synchronisation.
//
// The state is the traffic (2 x 64 KiB per v head per token, ~0.9 FLOP/B): HBM-bound. Each
// 128x128 fp32 tile is handled by 4 waves; lane (c = lane & 31, r = lane >> 5) of wave w
// holds columns 4c..4c+3 of rows w*32 + 2m + r (m = 0..15) as 16 float4 registers, so every
// load/store instruction of a wave moves 1 KiB of contiguous state. The tile is loaded once
// (loads issued before the conv so HBM latency overlaps it), reduced once for both S^T k
// and S^T q (in-thread over 16 rows, v_permlane32_swap across the two row halves of a wave,
// LDS across the 4 waves), and written once:
//   u = g S^T k,  d = beta (v - u),  S' = g S + k d^T,  o = g S^T q + d (k . q).
#include "ix_gdn.h"
#include "wave64.h"

namespace ixg {
namespace {

constexpr int kD = 128;                 // d_k = d_v
constexpr int kTileThreads = 256;       // 4 waves per 128x128 tile
constexpr int kRowsPerLane = kD / (kTileThreads / 32);  // 16 rows (float4 column groups: 32 per row)

struct DecodeParams {
    const uint16_t* x;          // [B][C]
    uint16_t* conv_state;       // [B][C][dc-1]
    const uint16_t* conv_w;     // [C][dc]
    const uint16_t* a;          // [B][h_v]
    const uint16_t* b;          // [B][h_v]
    const float* A_log;         // [h_v]
    const float* dt_bias;       // [h_v]
    float* state;               // [B][h_v][128][128]
    float* o;                   // [B][h_v][128] or null
    uint16_t* o_bf16;           // [B][h_v][128] or null
    int h_k, h_v, C, dc, head_map, conv_act, per_src;
    float q_scale, l2_eps;
};

__device__ __forceinline__ int mapped_head(const DecodeParams& p, int src, int m) {
    return p.head_map == IX_GDN_HEAD_MOD ? src + m * p.h_k : src * p.per_src + m;
}

__device__ __forceinline__ int mapped_count(const DecodeParams& p, int src) {
    if (p.head_map == IX_GDN_HEAD_MOD) return src < p.h_v ? (p.h_v - src + p.h_k - 1) / p.h_k : 0;
    return p.per_src;
}

// Conv of one channel of one sequence; shifts the rolling state and returns the output.
__device__ __forceinline__ float conv_channel(const DecodeParams& p, int bseq, int ch) {
    const size_t row = (size_t)bseq * p.C + ch;
    uint16_t* st = p.conv_state + row * (p.dc - 1);
    const uint16_t* w = p.conv_w + (size_t)ch * p.dc;
    const uint16_t xu = p.x[row];
    uint16_t hist[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) hist[i] = (i < p.dc - 1) ? st[i] : (uint16_t)0;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 3; ++i)
        if (i < p.dc - 1) acc = fmaf(bf16_to_f32(hist[i]), bf16_to_f32(w[i]), acc);
    acc = fmaf(bf16_to_f32(xu), bf16_to_f32(w[p.dc - 1]), acc);
#pragma unroll
    for (int i = 0; i < 2; ++i)
        if (i < p.dc - 2) st[i] = hist[i + 1];
    st[p.dc - 2] = xu;
    if (p.conv_act == IX_GDN_ACT_SILU) acc = acc * sigmoid_f(acc);
    return acc;
}

template <int NV>
__global__ void __launch_bounds__(NV * kTileThreads)
decode_kernel(const DecodeParams p) {
    __shared__ __align__(16) float qk_raw[2][kD];   // post-conv q, k of src
    __shared__ __align__(16) float v_raw[NV][kD];   // post-conv v of each tile's head
    __shared__ float4 red[NV][4][2][kD / 4];        // per-wave column partials of S^T k, S^T q
    __shared__ float scal[4];                       // q.q, k.k, q.k
    __shared__ float gates[NV][2];                  // g, beta

    const int src = blockIdx.x, bseq = blockIdx.y;
    const int tid = threadIdx.x;
    const int t = tid / kTileThreads;               // tile (v head slot) of this thread
    const int ltid = tid % kTileThreads;
    const int w = ltid / kWave, lane = tid & (kWave - 1);
    const int cgrp = lane & 31, rsub = lane >> 5;
    const int count = mapped_count(p, src);

    for (int base = 0; base == 0 || base < count; base += NV) {
        const int slot = base + t;
        const bool active = slot < count;
        const int h = active ? mapped_head(p, src, slot) : 0;
        float4* tile = reinterpret_cast<float4*>(p.state + ((size_t)bseq * p.h_v + h) * kD * kD);

        // 1. State loads first: 16 x float4 per lane, all in flight during the conv.
        float4 s[kRowsPerLane];
        if (active) {
#pragma unroll
            for (int m = 0; m < kRowsPerLane; ++m) {
                const int i = w * 32 + 2 * m + rsub;
                s[m] = tile[i * (kD / 4) + cgrp];
            }
        }

        // 2. Conv: the first pass also covers q and k of src (256 channels, the first
        //    256 threads); each tile's 128 v channels go to the remaining threads.
        const int nwork = (base == 0 ? 2 * kD : 0) + NV * kD;
        for (int e = tid; e < nwork; e += NV * kTileThreads) {
            int ee = e - (base == 0 ? 2 * kD : 0);
            if (ee < 0) {
                const int which = e / kD, i = e % kD;     // 0: q, 1: k
                const int ch = which * p.h_k * kD + src * kD + i;
                qk_raw[which][i] = conv_channel(p, bseq, ch);
            } else {
                const int vt = ee / kD, i = ee % kD;
                if (base + vt < count) {
                    const int hv = mapped_head(p, src, base + vt);
                    v_raw[vt][i] = conv_channel(p, bseq, 2 * p.h_k * kD + hv * kD + i);
                }
            }
        }
        if (ltid == kWave && active) {              // one lane per tile computes its gates
            const float al = p.A_log[h], dt = p.dt_bias[h];
            const float av = bf16_to_f32(p.a[(size_t)bseq * p.h_v + h]);
            const float bv = bf16_to_f32(p.b[(size_t)bseq * p.h_v + h]);
            gates[t][0] = expf(-expf(al) * softplus_f(av + dt));
            gates[t][1] = sigmoid_f(bv);
        }
        __syncthreads();

        // 3. q.q, k.k, q.k over the 128 channels (wave 0 of the workgroup, first pass).
        if (base == 0 && tid < kWave) {
            const float q0 = qk_raw[0][tid], q1 = qk_raw[0][tid + kWave];
            const float k0 = qk_raw[1][tid], k1 = qk_raw[1][tid + kWave];
            const float qq = wave_sum(fmaf(q0, q0, q1 * q1));
            const float kk = wave_sum(fmaf(k0, k0, k1 * k1));
            const float qk = wave_sum(fmaf(q0, k0, q1 * k1));
            if (tid == 0) { scal[0] = qq; scal[1] = kk; scal[2] = qk; }
        }
        __syncthreads();

        const float inv_q = p.q_scale / sqrtf(scal[0] + p.l2_eps);
        const float inv_k = 1.0f / sqrtf(scal[1] + p.l2_eps);
        const float kq = scal[2] * inv_q * inv_k;

        // 4. Column partials over this lane's 16 rows.
        float4 ak = make_float4(0.f, 0.f, 0.f, 0.f), aq = ak;
        if (active) {
#pragma unroll
            for (int m = 0; m < kRowsPerLane; ++m) {
                const int i = w * 32 + 2 * m + rsub;
                const float ki = qk_raw[1][i] * inv_k, qi = qk_raw[0][i] * inv_q;
                ak.x = fmaf(s[m].x, ki, ak.x); ak.y = fmaf(s[m].y, ki, ak.y);
                ak.z = fmaf(s[m].z, ki, ak.z); ak.w = fmaf(s[m].w, ki, ak.w);
                aq.x = fmaf(s[m].x, qi, aq.x); aq.y = fmaf(s[m].y, qi, aq.y);
                aq.z = fmaf(s[m].z, qi, aq.z); aq.w = fmaf(s[m].w, qi, aq.w);
            }
        }
        ak.x = pair_sum32(ak.x); ak.y = pair_sum32(ak.y); ak.z = pair_sum32(ak.z); ak.w = pair_sum32(ak.w);
        aq.x = pair_sum32(aq.x); aq.y = pair_sum32(aq.y); aq.z = pair_sum32(aq.z); aq.w = pair_sum32(aq.w);
        if (rsub == 0) { red[t][w][0][cgrp] = ak; red[t][w][1][cgrp] = aq; }
        __syncthreads();

        // 5. Finish the reductions for this lane's 4 columns, update and write back.
        if (active) {
            const float g = gates[t][0], bt = gates[t][1];
            float4 A = red[t][0][0][cgrp], Q = red[t][0][1][cgrp];
#pragma unroll
            for (int ww = 1; ww < 4; ++ww) {
                const float4 a2 = red[t][ww][0][cgrp], q2 = red[t][ww][1][cgrp];
                A.x += a2.x; A.y += a2.y; A.z += a2.z; A.w += a2.w;
                Q.x += q2.x; Q.y += q2.y; Q.z += q2.z; Q.w += q2.w;
            }
            const float4 vv = reinterpret_cast<const float4*>(v_raw[t])[cgrp];
            float4 d;
            d.x = (vv.x - g * A.x) * bt; d.y = (vv.y - g * A.y) * bt;
            d.z = (vv.z - g * A.z) * bt; d.w = (vv.w - g * A.w) * bt;
#pragma unroll
            for (int m = 0; m < kRowsPerLane; ++m) {
                const int i = w * 32 + 2 * m + rsub;
                const float ki = qk_raw[1][i] * inv_k;
                float4 r;
                r.x = fmaf(ki, d.x, s[m].x * g); r.y = fmaf(ki, d.y, s[m].y * g);
                r.z = fmaf(ki, d.z, s[m].z * g); r.w = fmaf(ki, d.w, s[m].w * g);
                tile[i * (kD / 4) + cgrp] = r;
            }
            if (w == 0 && rsub == 0) {
                float4 ov;
                ov.x = fmaf(d.x, kq, g * Q.x); ov.y = fmaf(d.y, kq, g * Q.y);
                ov.z = fmaf(d.z, kq, g * Q.z); ov.w = fmaf(d.w, kq, g * Q.w);
                const size_t oo = ((size_t)bseq * p.h_v + h) * kD + 4 * cgrp;
                if (p.o) *reinterpret_cast<float4*>(p.o + oo) = ov;
                if (p.o_bf16) {
                    uint2 pk;
                    pk.x = pack_bf16x2(ov.x, ov.y);
                    pk.y = pack_bf16x2(ov.z, ov.w);
                    *reinterpret_cast<uint2*>(p.o_bf16 + oo) = pk;
                }
            }
        }
        if (base + NV >= count) break;
        __syncthreads();                              // LDS is reused by the next group
    }
}

}  // namespace
}  // namespace ixg

extern "C" int ix_gdn_channels(const ix_gdn_cfg* c) {
    return c ? 2 * c->h_k * c->d_k + c->h_v * c->d_v : 0;
}

extern "C" const char* ix_gdn_version(void) { return "ixgdn 0.1.0 gfx950"; }

// Shared validation of the fused layer description (also used by the prefill).
extern "C" hipError_t ix_gdn_check_cfg_(const ix_gdn_cfg* c) {
    if (!c) return hipErrorInvalidValue;
    if (c->h_k <= 0 || c->h_v <= 0) return hipErrorInvalidValue;
    if (c->d_k != 128 || c->d_v != 128) return hipErrorInvalidValue;
    if (c->d_conv < 2 || c->d_conv > 4) return hipErrorInvalidValue;
    if (c->head_map != IX_GDN_HEAD_MOD && c->head_map != IX_GDN_HEAD_DIV) return hipErrorInvalidValue;
    if (c->head_map == IX_GDN_HEAD_DIV && c->h_v % c->h_k != 0) return hipErrorInvalidValue;
    if (c->conv_act != IX_GDN_ACT_NONE && c->conv_act != IX_GDN_ACT_SILU) return hipErrorInvalidValue;
    if (!(c->l2_eps >= 0.0f)) return hipErrorInvalidValue;
    return hipSuccess;
}

extern "C" hipError_t ix_gdn_decode(const ix_gdn_cfg* cfg, int B, const uint16_t* x, uint16_t* conv_state,
                                    const uint16_t* conv_w, const uint16_t* a, const uint16_t* b,
                                    const float* A_log, const float* dt_bias, float* state, float* o,
                                    uint16_t* o_bf16, hipStream_t s) {
    const hipError_t e = ix_gdn_check_cfg_(cfg);
    if (e != hipSuccess) return e;
    if (B <= 0 || B > 65535) return hipErrorInvalidValue;
    if (!x || !conv_state || !conv_w || !a || !b || !A_log || !dt_bias || !state) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(state) & 15) || (o && (reinterpret_cast<uintptr_t>(o) & 15)) ||
        (o_bf16 && (reinterpret_cast<uintptr_t>(o_bf16) & 7)))
        return hipErrorInvalidValue;                 // float4 / uint2 accesses
    ixg::DecodeParams p;
    p.x = x; p.conv_state = conv_state; p.conv_w = conv_w; p.a = a; p.b = b;
    p.A_log = A_log; p.dt_bias = dt_bias; p.state = state; p.o = o; p.o_bf16 = o_bf16;
    p.h_k = cfg->h_k; p.h_v = cfg->h_v; p.C = ix_gdn_channels(cfg); p.dc = cfg->d_conv;
    p.head_map = cfg->head_map; p.conv_act = cfg->conv_act;
    p.per_src = cfg->head_map == IX_GDN_HEAD_DIV ? cfg->h_v / cfg->h_k : 0;
    p.q_scale = cfg->q_scale; p.l2_eps = cfg->l2_eps;
    hipLaunchKernelGGL(ixg::decode_kernel<2>, dim3((unsigned)cfg->h_k, (unsigned)B), dim3(2 * ixg::kTileThreads), 0, s, p);
    return hipGetLastError();
}
