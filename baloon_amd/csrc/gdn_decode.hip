// gdn_decode.hip -- fused, batched GDN decode for gfx950 (ix_gdn_decode).
//
// One launch does a whole GDN layer's recurrent part for one token of B sequences:
// causal depthwise conv (rolling state) over the q|k|v channels, L2 norm of q and k, the
// gates g = exp(-exp(A_log) softplus(a + dt_bias)) and beta = sigmoid(b), the head map, and
// the delta-rule update of the fp32 state with output o = S'^T q. The reference does these
// as separate launches (src/ix_gdn.cu:58-70, :73-84, :102-105, :25-56) and has no batch.
//
// Work decomposition: one 256-thread workgroup per (sequence b, q/k head src). It owns the
// q and k channels of src and every v head mapped to src, so each conv-state channel and
// each state element is read and written by exactly one workgroup: the in-place updates
// are race free without any cross-workgroup synchronisation.
//
// The state is the traffic (2 x 64 KiB per v head per token, ~0.9 FLOP/B): HBM-bound. A
// workgroup streams its tiles as 16 KiB slabs of 128 rows x 32 columns. Columns are
// independent in the update, so a slab is a complete unit of work:
//   u = g S^T k,  d = beta (v - u),  S' = g S + k d^T,  o = g S^T q + d (k . q)
// (the output identity lets one sweep produce both contractions, so every state element
// is read once and written once). Thread (c4 = tid & 7, r0 = tid >> 3) holds float4 column
// group c4 of rows r0 + 32 m, m = 0..3: each wave load/store instruction moves 8 full
// 128-byte lines. Column sums are reduced in-thread over 4 rows, across the 8 row groups of
// a wave with DPP row_ror and v_permlane16/32_swap, and across the 4 waves through LDS.
// Slabs are loaded two ahead of the one being processed (the first ones before the conv,
// so HBM latency overlaps it), with nontemporal loads and stores: the state is streamed
// once per token and never reused from cache.
#include "gdn_common.h"

namespace ixg {
namespace {

constexpr int kThreads = 256;                        // 4 waves
constexpr int kSlabCols = 32;                        // state columns per slab
constexpr int kSlabsPerTile = kD / kSlabCols;        // 4
constexpr int kRowsPerThread = kD / (kThreads / 8);  // 4: rows r0 + 32 m
constexpr int kMaxHeadsPerGroup = 16;                // v heads per q/k head

struct DecodeParams {
    Layer L;
    const uint16_t* x;          // [B][C]
    uint16_t* conv_state;       // [B][C][dc-1]
    const uint16_t* a;          // [B][h_v]
    const uint16_t* b;          // [B][h_v]
    float* state;               // [B][h_v][128][128]
    float* o;                   // [B][h_v][128] or null
    uint16_t* o_bf16;           // [B][h_v][128] or null
};

// Sum over the 8 row groups of a wave (lanes that share lane & 7), result in every lane.
__device__ __forceinline__ float rowgroup_sum(float v) {
    v += dpp_f32<kDppRowRor8>(v);
    return pair_sum32(pair_sum16(v));
}

// Conv inputs of two adjacent channels (ch even) of one sequence, as dwords: x of both,
// the (DC-1)-entry bf16 histories of ch then ch+1, and their DC bf16 weights each. Every
// access is 4-byte aligned because C, ch and the row offsets are even.
template <int DC>
struct ConvPair {
    uint32_t x;
    uint32_t h[DC - 1];
    uint32_t w[DC];
};

__device__ __forceinline__ uint16_t u16_at(const uint32_t* a, int e) {
    return (uint16_t)(a[e >> 1] >> (16 * (e & 1)));
}

template <int DC>
__device__ __forceinline__ void conv_pair_load(const DecodeParams& p, int bseq, int ch, ConvPair<DC>& c) {
    const size_t row = (size_t)bseq * p.L.C + ch;
    c.x = *reinterpret_cast<const uint32_t*>(p.x + row);
    const uint32_t* hp = reinterpret_cast<const uint32_t*>(p.conv_state + row * (DC - 1));
#pragma unroll
    for (int i = 0; i < DC - 1; ++i) c.h[i] = hp[i];
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(p.L.conv_w + (size_t)ch * DC);
#pragma unroll
    for (int i = 0; i < DC; ++i) c.w[i] = wp[i];
}

// Conv outputs of the pair (the same accumulation order as conv_eval) and the shifted
// histories written back in place.
template <int DC>
__device__ __forceinline__ void conv_pair_apply(const DecodeParams& p, int bseq, int ch, const ConvPair<DC>& c,
                                                float* y0, float* y1) {
    const uint16_t xs[2] = {(uint16_t)(c.x & 0xffff), (uint16_t)(c.x >> 16)};
    uint16_t nh[2 * (DC - 1)];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < DC - 1; ++i)
            acc = fmaf(bf16_to_f32(u16_at(c.h, q * (DC - 1) + i)), bf16_to_f32(u16_at(c.w, q * DC + i)), acc);
        acc = fmaf(bf16_to_f32(xs[q]), bf16_to_f32(u16_at(c.w, q * DC + DC - 1)), acc);
        if (p.L.conv_act == IX_GDN_ACT_SILU) acc = acc * sigmoid_f(acc);
        *(q == 0 ? y0 : y1) = acc;
#pragma unroll
        for (int i = 0; i < DC - 2; ++i) nh[q * (DC - 1) + i] = u16_at(c.h, q * (DC - 1) + i + 1);
        nh[q * (DC - 1) + DC - 2] = xs[q];
    }
    const size_t row = (size_t)bseq * p.L.C + ch;
    uint32_t* hp = reinterpret_cast<uint32_t*>(p.conv_state + row * (DC - 1));
#pragma unroll
    for (int i = 0; i < DC - 1; ++i) hp[i] = (uint32_t)nh[2 * i] | ((uint32_t)nh[2 * i + 1] << 16);
}

// Channel pair e of group (bseq, src): pairs 0..63 are q, 64..127 k, then 64 per mapped v head.
// Writes the conv outputs into q_s / k_s / v_s.
__device__ __forceinline__ int pair_channel(const Layer& L, int src, int e, float*& dst,
                                            float* q_s, float* k_s, float (*v_s)[kD]) {
    if (e < 64) { dst = q_s + 2 * e; return q_channel(L, src, 2 * e); }
    if (e < 128) { dst = k_s + 2 * (e - 64); return k_channel(L, src, 2 * (e - 64)); }
    const int t = (e - 128) / 64, j = 2 * ((e - 128) % 64);
    dst = v_s[t] + j;
    return v_channel(L, mapped_head(L, src, t), j);
}

template <int DC>
__global__ void __launch_bounds__(kThreads)
decode_kernel(const DecodeParams p) {
    __shared__ __align__(16) float q_s[kD], k_s[kD];
    __shared__ __align__(16) float v_s[kMaxHeadsPerGroup][kD];
    __shared__ float gate_s[kMaxHeadsPerGroup][2];
    __shared__ float scal_s[3];
    __shared__ v4f red_s[2][kThreads / kWave][kSlabCols / 4][2];   // [slab parity][wave][c4][u|q]

    const Layer& L = p.L;
    const int src = blockIdx.x, bseq = blockIdx.y;
    const int tid = threadIdx.x, w = tid / kWave, lane = tid & (kWave - 1);
    const int c4 = tid & 7, r0 = tid >> 3;
    const int count = mapped_count(L, src);
    const int nslab = count * kSlabsPerTile;

    // Address of this thread's first element of slab n (rows r0 + 32 m follow at stride 32 rows).
    auto slab_ptr = [&](int n) -> v4f* {
        const int h = mapped_head(L, src, n / kSlabsPerTile);
        float* tile = p.state + ((size_t)bseq * L.h_v + h) * kD * kD;
        return reinterpret_cast<v4f*>(tile + (size_t)r0 * kD + (n % kSlabsPerTile) * kSlabCols) + c4;
    };
    auto load_slab = [&](v4f (&buf)[kRowsPerThread], int n) {
        if (n < nslab) {
            const v4f* ptr = slab_ptr(n);
#pragma unroll
            for (int m = 0; m < kRowsPerThread; ++m)
                buf[m] = __builtin_nontemporal_load(ptr + (size_t)m * 32 * (kD / 4));
        }
    };

    // Conv over q, k of src and v of every mapped head, by channel pairs: the first pair of
    // each thread is loaded before the state so its inputs return first.
    const int npairs = 128 + count * 64;
    float* dst0;
    const int ch0 = tid < npairs ? pair_channel(L, src, tid, dst0, q_s, k_s, v_s) : 0;
    ConvPair<DC> cp;
    if (tid < npairs) conv_pair_load<DC>(p, bseq, ch0, cp);

    v4f s0[kRowsPerThread], s1[kRowsPerThread], s2[kRowsPerThread];
    load_slab(s0, 0);
    load_slab(s1, 1);
    load_slab(s2, 2);

    if (tid < npairs) conv_pair_apply<DC>(p, bseq, ch0, cp, dst0, dst0 + 1);
    for (int e = tid + kThreads; e < npairs; e += kThreads) {      // more than 2 v heads per q/k head
        float* dst;
        const int ch = pair_channel(L, src, e, dst, q_s, k_s, v_s);
        ConvPair<DC> c2;
        conv_pair_load<DC>(p, bseq, ch, c2);
        conv_pair_apply<DC>(p, bseq, ch, c2, dst, dst + 1);
    }
    if (tid < count) {
        const int h = mapped_head(L, src, tid);
        const size_t ab = (size_t)bseq * L.h_v + h;
        gate_s[tid][0] = expf(log_gate(L, h, bf16_to_f32(p.a[ab])));
        gate_s[tid][1] = sigmoid_f(bf16_to_f32(p.b[ab]));
    }
    __syncthreads();

    // q.q, k.k, q.k over the 128 dims (one wave each).
    if (w < 3) {
        const float* x0 = (w == 1) ? k_s : q_s;
        const float* x1 = (w == 0) ? q_s : k_s;
        const float r = wave_sum(fmaf(x0[lane], x1[lane], x0[lane + kWave] * x1[lane + kWave]));
        if (lane == 0) scal_s[w] = r;
    }
    __syncthreads();
    const float inv_q = L.q_scale / sqrtf(scal_s[0] + L.l2_eps);
    const float inv_k = 1.0f / sqrtf(scal_s[1] + L.l2_eps);
    const float kq = scal_s[2] * inv_q * inv_k;
    float kr[kRowsPerThread], qr[kRowsPerThread];
#pragma unroll
    for (int m = 0; m < kRowsPerThread; ++m) {
        kr[m] = k_s[r0 + 32 * m] * inv_k;
        qr[m] = q_s[r0 + 32 * m] * inv_q;
    }

    // One slab: column sums, update, write back, output.
    auto process = [&](v4f (&buf)[kRowsPerThread], int n) {
        const int t = n / kSlabsPerTile, sc = n % kSlabsPerTile;
        v4f ak = {0.f, 0.f, 0.f, 0.f}, aq = ak;
#pragma unroll
        for (int m = 0; m < kRowsPerThread; ++m) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                ak[e] = fmaf(buf[m][e], kr[m], ak[e]);
                aq[e] = fmaf(buf[m][e], qr[m], aq[e]);
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) { ak[e] = rowgroup_sum(ak[e]); aq[e] = rowgroup_sum(aq[e]); }
        if (lane < 8) { red_s[n & 1][w][c4][0] = ak; red_s[n & 1][w][c4][1] = aq; }
        __syncthreads();
        v4f A = red_s[n & 1][0][c4][0], Q = red_s[n & 1][0][c4][1];
#pragma unroll
        for (int ww = 1; ww < kThreads / kWave; ++ww) { A += red_s[n & 1][ww][c4][0]; Q += red_s[n & 1][ww][c4][1]; }
        const float g = gate_s[t][0], bt = gate_s[t][1];
        const v4f vv = *reinterpret_cast<const v4f*>(&v_s[t][sc * kSlabCols + 4 * c4]);
        v4f d;
#pragma unroll
        for (int e = 0; e < 4; ++e) d[e] = (vv[e] - g * A[e]) * bt;
        v4f* ptr = slab_ptr(n);
#pragma unroll
        for (int m = 0; m < kRowsPerThread; ++m) {
            v4f r;
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = fmaf(kr[m], d[e], buf[m][e] * g);
            __builtin_nontemporal_store(r, ptr + (size_t)m * 32 * (kD / 4));
        }
        if (r0 == 0) {
            v4f ov;
#pragma unroll
            for (int e = 0; e < 4; ++e) ov[e] = fmaf(d[e], kq, g * Q[e]);
            const int h = mapped_head(L, src, t);
            const size_t oo = ((size_t)bseq * L.h_v + h) * kD + sc * kSlabCols + 4 * c4;
            if (p.o) *reinterpret_cast<v4f*>(p.o + oo) = ov;
            if (p.o_bf16) {
                uint2 pk;
                pk.x = pack_bf16x2(ov[0], ov[1]);
                pk.y = pack_bf16x2(ov[2], ov[3]);
                *reinterpret_cast<uint2*>(p.o_bf16 + oo) = pk;
            }
        }
    };

    // Three rotating slab buffers: the loop body is unrolled so no register is copied
    // while its load is still in flight.
    for (int n = 0; n < nslab; n += 3) {
        process(s0, n);
        load_slab(s0, n + 3);
        if (n + 1 < nslab) {
            process(s1, n + 1);
            load_slab(s1, n + 4);
        }
        if (n + 2 < nslab) {
            process(s2, n + 2);
            load_slab(s2, n + 5);
        }
    }
}

}  // namespace
}  // namespace ixg

extern "C" int ix_gdn_channels(const ix_gdn_cfg* c) {
    return c ? 2 * c->h_k * c->d_k + c->h_v * c->d_v : 0;
}

extern "C" const char* ix_gdn_version(void) { return "ixgdn 0.2.0 gfx950"; }

// Shared validation of the fused layer description (also used by the prefill).
extern "C" hipError_t ix_gdn_check_cfg_(const ix_gdn_cfg* c) {
    if (!c) return hipErrorInvalidValue;
    if (c->h_k <= 0 || c->h_v <= 0) return hipErrorInvalidValue;
    if (c->d_k != 128 || c->d_v != 128) return hipErrorInvalidValue;
    if (c->d_conv < 2 || c->d_conv > 4) return hipErrorInvalidValue;
    if (c->head_map != IX_GDN_HEAD_MOD && c->head_map != IX_GDN_HEAD_DIV) return hipErrorInvalidValue;
    if (c->head_map == IX_GDN_HEAD_DIV && c->h_v % c->h_k != 0) return hipErrorInvalidValue;
    const int per_src = (c->h_v + c->h_k - 1) / c->h_k;     // most v heads on one q/k head
    if (per_src > ixg::kMaxHeadsPerGroup) return hipErrorInvalidValue;
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
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(conv_state) |
         reinterpret_cast<uintptr_t>(conv_w)) & 3)
        return hipErrorInvalidValue;                 // conv inputs are read as dwords
    ixg::DecodeParams p;
    p.L = ixg::make_layer(cfg, conv_w, A_log, dt_bias);
    p.x = x; p.conv_state = conv_state; p.a = a; p.b = b;
    p.state = state; p.o = o; p.o_bf16 = o_bf16;
    const dim3 grid((unsigned)cfg->h_k, (unsigned)B), block(ixg::kThreads);
    switch (cfg->d_conv) {
        case 2: hipLaunchKernelGGL(ixg::decode_kernel<2>, grid, block, 0, s, p); break;
        case 3: hipLaunchKernelGGL(ixg::decode_kernel<3>, grid, block, 0, s, p); break;
        default: hipLaunchKernelGGL(ixg::decode_kernel<4>, grid, block, 0, s, p); break;
    }
    return hipGetLastError();
}
