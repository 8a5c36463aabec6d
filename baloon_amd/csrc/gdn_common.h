// gdn_common.h -- layer description and per-channel helpers shared by the fused decode and
// the chunked prefill kernels (gfx950).
//
// Semantics follow the reference's GDN path (src/ix_gdn.cu): modulo head pairing
// (src = h mod h_k, :38), causal depthwise conv with a rolling history, oldest first
// (:58-70), softplus with threshold 20 and sigmoid (:22-23). The layer-level extensions
// (gate from A_log/dt_bias, beta = sigmoid(b), optional SiLU after the conv, the
// contiguous head map) are selected by ix_gdn_cfg.
#pragma once
#include <atomic>
#include "ix_gdn.h"
#include "wave64.h"

namespace ixg {

constexpr int kD = 128;   // d_k = d_v handled by the fused kernels

typedef float v4f __attribute__((ext_vector_type(4)));

// Device copy of the fields of ix_gdn_cfg the kernels use, plus the layer parameters.
struct Layer {
    const uint16_t* conv_w;   // [C][dc] bf16
    const float* A_log;       // [h_v]
    const float* dt_bias;     // [h_v]
    int h_k, h_v, C, dc, head_map, conv_act, per_src;
    float q_scale, l2_eps;
};

inline Layer make_layer(const ix_gdn_cfg* c, const uint16_t* conv_w, const float* A_log, const float* dt_bias) {
    Layer L;
    L.conv_w = conv_w; L.A_log = A_log; L.dt_bias = dt_bias;
    L.h_k = c->h_k; L.h_v = c->h_v; L.C = 2 * c->h_k * c->d_k + c->h_v * c->d_v; L.dc = c->d_conv;
    L.head_map = c->head_map; L.conv_act = c->conv_act;
    L.per_src = c->head_map == IX_GDN_HEAD_DIV ? c->h_v / c->h_k : 0;
    L.q_scale = c->q_scale; L.l2_eps = c->l2_eps;
    return L;
}

// v heads mapped onto q/k head `src`: slot m of `mapped_count` (ascending head index).
__device__ __forceinline__ int mapped_head(const Layer& L, int src, int m) {
    return L.head_map == IX_GDN_HEAD_MOD ? src + m * L.h_k : src * L.per_src + m;
}
__device__ __forceinline__ int mapped_count(const Layer& L, int src) {
    if (L.head_map == IX_GDN_HEAD_MOD) return src < L.h_v ? (L.h_v - src + L.h_k - 1) / L.h_k : 0;
    return L.per_src;
}
// q/k head feeding v head h.
__device__ __forceinline__ int src_of(const Layer& L, int h) {
    return L.head_map == IX_GDN_HEAD_MOD ? h % L.h_k : h / L.per_src;
}

// Channel offsets in the mixed projection (order q | k | v).
__device__ __forceinline__ int q_channel(const Layer& L, int src, int i) { return src * kD + i; }
__device__ __forceinline__ int k_channel(const Layer& L, int src, int i) { return (L.h_k + src) * kD + i; }
__device__ __forceinline__ int v_channel(const Layer& L, int h, int j) { return (2 * L.h_k + h) * kD + j; }

// Conv output of one channel from its history (oldest first, dc-1 values) and the current
// input; the accumulation order is the one both fused kernels use.
__device__ __forceinline__ float conv_eval(const Layer& L, const float* hist, float x, const uint16_t* w) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < 3; ++i)
        if (i < L.dc - 1) acc = fmaf(hist[i], bf16_to_f32(w[i]), acc);
    acc = fmaf(x, bf16_to_f32(w[L.dc - 1]), acc);
    if (L.conv_act == IX_GDN_ACT_SILU) acc = acc * sigmoid_f(acc);
    return acc;
}

// Log decay -exp(A_log) * softplus(a + dt_bias); the decay is exp() of it.
__device__ __forceinline__ float log_gate(float A_log, float dt_bias, float a) {
    return -expf(A_log) * softplus_f(a + dt_bias);
}
__device__ __forceinline__ float log_gate(const Layer& L, int h, float a) { return log_gate(L.A_log[h], L.dt_bias[h], a); }

// Sum over the 32 lanes of each half wave, result in all of them.
__device__ __forceinline__ float half_sum(float v) { return pair_sum16(row_sum16(v)); }

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

// Conv outputs of the pair (the accumulation order of conv_eval) and the shifted histories
// (each channel's history minus its oldest entry, then x), packed as dwords.
template <int DC>
__device__ __forceinline__ void conv_pair_eval(const Layer& L, const ConvPair<DC>& c, float& y0, float& y1,
                                               uint32_t (&nh)[DC - 1]) {
    const uint16_t xs[2] = {(uint16_t)(c.x & 0xffff), (uint16_t)(c.x >> 16)};
    uint16_t n16[2 * (DC - 1)];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < DC - 1; ++i)
            acc = fmaf(bf16_to_f32(u16_at(c.h, q * (DC - 1) + i)), bf16_to_f32(u16_at(c.w, q * DC + i)), acc);
        acc = fmaf(bf16_to_f32(xs[q]), bf16_to_f32(u16_at(c.w, q * DC + DC - 1)), acc);
        if (L.conv_act == IX_GDN_ACT_SILU) acc = acc * sigmoid_f(acc);
        (q == 0 ? y0 : y1) = acc;
#pragma unroll
        for (int i = 0; i < DC - 2; ++i) n16[q * (DC - 1) + i] = u16_at(c.h, q * (DC - 1) + i + 1);
        n16[q * (DC - 1) + DC - 2] = xs[q];
    }
#pragma unroll
    for (int i = 0; i < DC - 1; ++i) nh[i] = (uint32_t)n16[2 * i] | ((uint32_t)n16[2 * i + 1] << 16);
}

// Device copy of ix_gdn_out_gate.
struct OutGate {
    const uint16_t* z;
    const float* nrm;
    float eps;
    float* y;
    uint16_t* y_bf16;
    uint8_t* y_q8_1;
};

inline OutGate make_out_gate(const ix_gdn_out_gate* g) {
    OutGate o{};
    if (g) {
        o.z = g->z; o.nrm = g->ssm_norm; o.eps = g->eps; o.y = g->y; o.y_bf16 = g->y_bf16;
        o.y_q8_1 = static_cast<uint8_t*>(g->y_q8_1);
    }
    return o;
}

// Compute units of the device that stream s launches on (the calling thread's current device
// for the null stream), queried once per device (256 on MI355X).
inline int device_cu_count(hipStream_t s) {
    constexpr int kMaxDev = 64;
    static std::atomic<int> cached[kMaxDev];
    int dev = 0;
    if (s) {
        hipDevice_t d = 0;
        if (hipStreamGetDevice(s, &d) != hipSuccess) return 256;
        dev = (int)d;
    } else if (hipGetDevice(&dev) != hipSuccess) {
        return 256;
    }
    if (dev < 0 || dev >= kMaxDev) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// q8_1 block (36 bytes: half d, half s, int8 qs[32]; the activation format of the Q8_0 product,
// src/ix_mmvq_wave.cu:20-24) of the 32 values v held by the 32 lanes of this lane's half wave,
// lane & 31 being the value's position: d = max|v| / 127, qs = roundf(v / d) (0 when d is 0:
// an all-zero block, or one so small that d underflows), s = the sum of v in the
// xor-butterfly order 16, 8, 4, 2, 1; d and s rounded to half.
// Every q8_1 producer here (ix_q8_1_quantize and the gated epilogues) goes through this one
// function, so the same fp32 values give the same bytes, division included
// (src/ix_q81_div.h:1-9). The inputs are finite. All 64 lanes of the wave must call it (its
// reductions stay within each half wave); a half wave that passes blk == nullptr stores nothing.
// Range: d and s are stored as fp16, so both are clamped to its largest finite value, 65504,
// before the conversion. A block whose d would exceed it (max|v| > 127 * 65504, about 8.3e6)
// is quantised with d = 65504 and its codes saturate at +-127; below that bound the clamps
// change nothing. The reference names such a clamp (q8_1_finite, src/ix_q81_div.h:9) without
// defining it, so this rule is this library's own.
constexpr int kQ81Bytes = 36;
constexpr float kHalfMax = 65504.0f;
__device__ __forceinline__ void q81_store(float v, int lane, uint8_t* blk) {
    float amax = fabsf(v), sum = v;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) {
        amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
        sum = sum + __shfl_xor(sum, off, kWave);
    }
    const float d = fminf(amax / 127.0f, kHalfMax);
    const int q = d == 0.0f ? 0 : (int)fminf(fmaxf(roundf(v / d), -127.0f), 127.0f);
    if (!blk) return;
    blk[4 + (lane & 31)] = (uint8_t)(int8_t)q;
    if ((lane & 31) == 0) {
        const float sc = fminf(fmaxf(sum, -kHalfMax), kHalfMax);
        const uint32_t hd = __builtin_bit_cast(uint16_t, (_Float16)d), hs = __builtin_bit_cast(uint16_t, (_Float16)sc);
        *reinterpret_cast<uint32_t*>(blk) = hd | (hs << 16);
    }
}

// Sum of v^2 over the wave, the same bits in every lane and in every kernel that calls it:
// each square is rounded before the sums (left to itself the compiler fuses it into the
// first DPP add, whose result then differs between lanes), and lane 0's total is broadcast.
__device__ __forceinline__ float wave_sum_sq(float v) {
    float sq = v * v;
    __asm__("" : "+v"(sq));
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(wave_sum(sq))));
}

// Gated RMS norm of one head's 128 outputs, called by a whole wave: lane l holds o of
// columns l (lo) and 64 + l (hi); row is the offset of the head's first element in z and y.
// The sum of squares is (sum over columns 0..63) + (sum over 64..127), each a wave_sum_sq,
// so every kernel that holds the head in this form gets the same bits.
// out_gate_apply takes the two partial sums already reduced.
// The gate inputs of lane l's two columns (l and 64 + l), loaded ahead by a caller that
// has them early.
struct GateIn {
    float nrm[2];
    uint16_t z[2];
};
__device__ __forceinline__ GateIn gate_in(const OutGate& g, size_t row, int lane) {
    GateIn in;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        in.nrm[q] = g.nrm[lane + q * (kD / 2)];
        in.z[q] = g.z[row + lane + q * (kD / 2)];
    }
    return in;
}
__device__ __forceinline__ void out_gate_apply(const OutGate& g, size_t row, float lo, float hi, float ss_lo,
                                               float ss_hi, int lane, const GateIn& in) {
    const float ss = ss_lo + ss_hi;
    const float inv = 1.0f / sqrtf(ss * (1.0f / kD) + g.eps);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int j = lane + q * (kD / 2);
        const float y = (q ? hi : lo) * inv * in.nrm[q] * sigmoid_f(bf16_to_f32(in.z[q]));
        if (g.y) g.y[row + j] = y;
        if (g.y_bf16) g.y_bf16[row + j] = f32_to_bf16(y);
        if (g.y_q8_1) q81_store(y, lane, g.y_q8_1 + ((row + j) / 32) * kQ81Bytes);
    }
}
__device__ __forceinline__ void out_gate_head(const OutGate& g, size_t row, float lo, float hi, int lane,
                                              const GateIn& in) {
    out_gate_apply(g, row, lo, hi, wave_sum_sq(lo), wave_sum_sq(hi), lane, in);
}
__device__ __forceinline__ void out_gate_head(const OutGate& g, size_t row, float lo, float hi, int lane) {
    out_gate_head(g, row, lo, hi, lane, gate_in(g, row, lane));
}

// ---------------------------------------------------------------------------------------
// Split-bf16 products on v_mfma_f32_16x16x32_bf16: an fp32 operand x is split into
// hi = RNE(x) and lo = RNE(x - hi), and a product is hi*hi + hi*lo + lo*hi in fp32
// accumulators (relative error ~2^-16, against 2^-8 for one bf16 product).
// ---------------------------------------------------------------------------------------
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef uint32_t u4x __attribute__((ext_vector_type(4)));
typedef float v4 __attribute__((ext_vector_type(4)));

// k index of slot e (0..7) of lane group g (lane / 16) in an A or B operand: the row order of
// two stacked 16 x 16 accumulator tiles (lane group g holds rows 4g..4g+3 of each), so that
// an accumulator pair is the next product's operand as it stands, and so that a lane's 8
// values are two runs of 4 consecutive k (16-byte loads). A and B agree on it, so the k sum
// covers the same terms.
__device__ __forceinline__ int kperm(int g, int e) { return e < 4 ? 4 * g + e : 16 + 4 * g + (e - 4); }

// Split two fp32 values into packed bf16 pairs: hi = RNE(x), lo = RNE(x - hi). The hi values
// return to fp32 by a shift and a mask, so a pair costs one convert per plane.
__device__ __forceinline__ void split2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
    hi = pack_bf16x2(x0, x1);
    lo = pack_bf16x2(x0 - __uint_as_float(hi << 16), x1 - __uint_as_float(hi & 0xffff0000u));
}

// Split 8 fp32 values into hi and lo bf16 vectors.
__device__ __forceinline__ void split8(const float (&x)[8], bf8& hi, bf8& lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) split2(x[2 * i], x[2 * i + 1], h[i], l[i]);
    hi = __builtin_bit_cast(bf8, u4x{h[0], h[1], h[2], h[3]});
    lo = __builtin_bit_cast(bf8, u4x{l[0], l[1], l[2], l[3]});
}

__device__ __forceinline__ v4 mfma_bf16(const bf8& a, const bf8& b, const v4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// c += A B with both operands split: hi hi + hi lo + lo hi.
__device__ __forceinline__ v4 mfma_split(const bf8& ah, const bf8& al, const bf8& bh, const bf8& bl, v4 c) {
    c = mfma_bf16(ah, bh, c);
    c = mfma_bf16(ah, bl, c);
    return mfma_bf16(al, bh, c);
}

}  // namespace ixg
