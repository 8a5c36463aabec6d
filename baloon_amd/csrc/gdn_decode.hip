// gdn_decode.hip -- fused, batched GDN decode for gfx950 (ix_gdn_decode).
//
// One launch does a whole GDN layer's recurrent part for one token of B sequences:
// causal depthwise conv (rolling state) over the q|k|v channels, L2 norm of q and k, the
// gates g = exp(-exp(A_log) softplus(a + dt_bias)) and beta = sigmoid(b), the head map, and
// the delta-rule update of the fp32 state with output o = S'^T q. The reference does these
// as separate launches (src/ix_gdn.cu:58-70, :73-84, :102-105, :25-56) and has no batch.
//
// State layout: [B][h_v][d_v][d_k], i.e. each head's S (d_k x d_v) is stored column by
// column, so column j (all 128 k indices) is one contiguous 512-byte run. A column is a
// complete unit of the update:
//   u_j = g S_j . k,  d_j = beta (v_j - u_j),  S_j' = g S_j + d_j k,  o_j = g S_j . q + d_j (k . q)
// (the output identity lets one sweep produce both contractions, so every state element is
// read once and written once; ~0.9 FLOP per byte, HBM-bound). Lane l of a wave holds k
// indices 4 (l & 31) .. +3 of column (l >> 5) of a pair of adjacent columns: every wave
// load/store instruction moves 1 KiB of contiguous state, and the column sums are
// in-wave reductions over 32 lanes (DPP within rows, v_permlane16_swap across them).
//
// Kernels, chosen by the launcher:
//  * slab_kernel (a workspace of per-group counters is given): one workgroup per
//    (sequence, v head, 64-column half tile), 4096 workgroups at B=64 for a short,
//    well-balanced stream (512 threads instead of 256 when the grid does not fill the
//    CUs, B <= 4 at h_v = 32, so that each wave runs 4 column pairs instead of 8: B=1
//    replays at 3.98-4.01 against 4.13-4.25 us per token). Every workgroup evaluates the q/k conv of its q/k head
//    read-only; the conv history of those channels is written back by the last workgroup
//    of the (sequence, q/k head) group to finish reading it, found with one atomic counter
//    per group. The counter is reset by that workgroup, so the workspace is all zeros
//    again when the kernel ends. No workgroup ever waits for another.
//  * head_kernel (the gated decode, ix_gdn_decode_gated, with the counters): the same with
//    one 512-thread workgroup per (sequence, v head), so the head's 128 outputs meet in LDS
//    and the gated RMS output norm (the semantics of ix_gdn_out_norm, src/ix_gdn.cu:87-100)
//    is applied by one wave after one barrier.
//  * group_kernel (no workspace): one workgroup per (sequence, q/k head) that owns every
//    channel and tile of the group; race free by ownership. It has the gated variant too.
// The gated norm's sum of squares is the same two wave sums (columns 0..63, 64..127) in the
// head and group kernels, so they give the same bits.
//
// The group counter hand-off (slab and head kernels) rests on three facts, none of which is
// a guarantee of the HIP memory model (the counter add is a relaxed atomic with no
// release/acquire pairing, which at agent scope would wait for the state loads kept in
// flight across it):
//  1. Each member consumes its q/k conv-history loads before its LDS-only barrier: their
//     values feed the conv outputs that it stores to LDS ahead of that barrier, so the wave
//     has waited for those loads before it reaches the barrier.
//  2. The compiler keeps the global atomic add after the s_barrier (tests/test_codegen.py
//     checks this in the built code of every slab and head kernel), and a wave issues its
//     instructions in order, so the add is performed after the member's history reads.
//  3. The last member's history writes follow its add (they need its result), and the
//     next call on the stream starts after this kernel has ended.
// So the last arrival rewrites the history only after every member has read it.
// State loads use nontemporal hints and are issued right after the conv inputs so that
// HBM latency overlaps the conv; the state is streamed once per token.
#include "gdn_common.h"

#include <mutex>

namespace ixg {
namespace {

constexpr int kThreads = 256;                        // 4 waves
constexpr int kMaxHeadsPerGroup = 16;                // v heads per q/k head
constexpr int kHalfCols = 64;                        // columns per slab_kernel workgroup
constexpr int kSmallGridThreads = 512;               // slab workgroup size when the grid is below the CU count
constexpr int kPairsPerWave = kHalfCols / 2 / (kThreads / kWave);   // 8 column pairs (head kernel)

struct DecodeParams {
    Layer L;
    const uint16_t* x;          // [B][C]
    uint16_t* conv_state;       // [B][C][dc-1]
    const uint16_t* a;          // [B][h_v]
    const uint16_t* b;          // [B][h_v]
    float* state;               // [B][h_v][d_v][d_k]
    float* o;                   // [B][h_v][128] or null
    uint16_t* o_bf16;           // [B][h_v][128] or null
    OutGate og;                 // gated variant only
};

// Workspace: the group counters [B][h_k] (one per sequence and q/k head), zero between
// calls: each call's last group member resets its counter.
struct DecodeWs {
    int* group;
};

inline size_t decode_ws_bytes(int B, int h_k) { return ((size_t)B * h_k * 4 + 255) & ~(size_t)255; }

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

template <int DC>
__device__ __forceinline__ void hist_store(const DecodeParams& p, int bseq, int ch, const uint32_t (&nh)[DC - 1]) {
    uint32_t* hp = reinterpret_cast<uint32_t*>(p.conv_state + ((size_t)bseq * p.L.C + ch) * (DC - 1));
#pragma unroll
    for (int i = 0; i < DC - 1; ++i) hp[i] = nh[i];
}

// Gate and beta of head h of sequence bseq.
__device__ __forceinline__ void gates(const DecodeParams& p, int bseq, int h, float* gb) {
    const size_t ab = (size_t)bseq * p.L.h_v + h;
    gb[0] = expf(log_gate(p.L, h, bf16_to_f32(p.a[ab])));
    gb[1] = sigmoid_f(bf16_to_f32(p.b[ab]));
}

// The column update for one pair of columns held as one float4 per lane (see the header).
// kr, qr: this lane's 4 entries of the normalised k and q; vj: v of this lane's column.
// Returns the column's output (valid in every lane).
__device__ __forceinline__ float column_update(const DecodeParams& p, v4f s, v4f* dst, const v4f& kr, const v4f& qr,
                                              float vj, float g, float bt, float kq, size_t o_index, bool writer) {
    float ak = s[0] * kr[0], aq = s[0] * qr[0];
#pragma unroll
    for (int e = 1; e < 4; ++e) { ak = fmaf(s[e], kr[e], ak); aq = fmaf(s[e], qr[e], aq); }
    ak = half_sum(ak);
    aq = half_sum(aq);
    const float d = (vj - g * ak) * bt;
    v4f r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = fmaf(kr[e], d, s[e] * g);
    __builtin_nontemporal_store(r, dst);
    const float ov = fmaf(d, kq, g * aq);
    if (writer) {
        if (p.o) p.o[o_index] = ov;
        if (p.o_bf16) p.o_bf16[o_index] = f32_to_bf16(ov);
    }
    return ov;
}


// ---------------------------------------------------------------------------------------
// slab_kernel: grid (2 h_v, B); workgroup = (sequence bseq, v head h, half tile hf) of NT
// threads (kThreads, or kSmallGridThreads when the grid does not fill the CUs: more waves
// share the 32 column pairs, so each runs fewer of them in series)
// ---------------------------------------------------------------------------------------
template <int DC, int NT>
__global__ void __launch_bounds__(NT)
slab_kernel(const DecodeParams p, const DecodeWs ws) {
    constexpr int kPW = kHalfCols / 2 / (NT / kWave);         // column pairs per wave
    __shared__ __align__(16) float q_s[kD], k_s[kD], v_s[kHalfCols];
    int* __restrict__ counters = ws.group;
    __shared__ float scal_s[2], gb_s[2];
    __shared__ int last_s;

    const Layer& L = p.L;
    const int tid = threadIdx.x, w = tid / kWave, lane = tid & (kWave - 1);
    const int half = lane >> 5, i4 = lane & 31;
    const int hf = blockIdx.x & 1, h = blockIdx.x >> 1, bseq = blockIdx.y;
    const int src = src_of(L, h);

    // Conv inputs: threads 0..63 q pairs, 64..127 k pairs, 128..159 the v pairs of this half tile.
    int ch = 0;
    float* dst = nullptr;
    if (tid < 64) { ch = q_channel(L, src, 2 * tid); dst = q_s + 2 * tid; }
    else if (tid < 128) { ch = k_channel(L, src, 2 * (tid - 64)); dst = k_s + 2 * (tid - 64); }
    else if (tid < 128 + kHalfCols / 2) { ch = v_channel(L, h, hf * kHalfCols + 2 * (tid - 128)); dst = v_s + 2 * (tid - 128); }
    const bool conv_thread = tid < 128 + kHalfCols / 2;
    ConvPair<DC> cp;
    if (conv_thread) conv_pair_load<DC>(p, bseq, ch, cp);
    // The gate inputs too are loaded ahead of the state (by every thread, from one address:
    // a conditional load would make its branch wait for it before the state loads go out),
    // so that computing the gates does not wait for the state loads of the gate thread's wave.
    const size_t ab = (size_t)bseq * L.h_v + h;
    const uint16_t a_in = p.a[ab], b_in = p.b[ab];

    // State: wave w owns columns hf*64 + 2 kPW w + 2 u + half, u = 0..kPW-1.
    v4f* tile = reinterpret_cast<v4f*>(p.state + ((size_t)bseq * L.h_v + h) * kD * kD) + i4;
    const int j0 = hf * kHalfCols + 2 * kPW * w + half;
    v4f s[kPW];
#pragma unroll
    for (int u = 0; u < kPW; ++u) s[u] = __builtin_nontemporal_load(tile + (size_t)(j0 + 2 * u) * (kD / 4));

    uint32_t nh[DC - 1];
    float y0 = 0.0f, y1 = 0.0f;
    if (conv_thread) {
        conv_pair_eval<DC>(L, cp, y0, y1, nh);
        dst[0] = y0;
        dst[1] = y1;
        if (tid >= 128) hist_store<DC>(p, bseq, ch, nh);          // v channels: owned by this workgroup
    }
    if (w < 2) {                                                  // wave 0: q.q, wave 1: k.k
        const float r = wave_sum(fmaf(y0, y0, y1 * y1));
        if (lane == 0) scal_s[w] = r;
    }
    if (tid == NT - 1) {
        gb_s[0] = expf(log_gate(L, h, bf16_to_f32(a_in)));
        gb_s[1] = sigmoid_f(bf16_to_f32(b_in));
    }
    // Everything shared below is in LDS, and the conv history values were consumed above, so
    // their loads are complete: an LDS-only barrier, which leaves the state loads in flight.
    lds_barrier();

    // Every thread's reads of the q/k conv history are complete (fact 1 of the hand-off in
    // the file header): count this workgroup in. The result is needed only after the column
    // updates, so its round trip overlaps them.
    int old = 0;
    if (tid == 0) old = atomicAdd(counters + (size_t)bseq * L.h_k + src, 1);
    const float inv_q = L.q_scale / sqrtf(scal_s[0] + L.l2_eps);
    const float inv_k = 1.0f / sqrtf(scal_s[1] + L.l2_eps);
    const float kq = wave_sum(fmaf(q_s[lane], k_s[lane], q_s[lane + kWave] * k_s[lane + kWave])) * inv_q * inv_k;
    v4f kr, qr;
    {
        const v4f kk = *reinterpret_cast<const v4f*>(k_s + 4 * i4), qq = *reinterpret_cast<const v4f*>(q_s + 4 * i4);
#pragma unroll
        for (int e = 0; e < 4; ++e) { kr[e] = kk[e] * inv_k; qr[e] = qq[e] * inv_q; }
    }
    const float g = gb_s[0], bt = gb_s[1];
    const size_t ob = ((size_t)bseq * L.h_v + h) * kD;
#pragma unroll
    for (int u = 0; u < kPW; ++u) {
        const int j = j0 + 2 * u;
        column_update(p, s[u], tile + (size_t)j * (kD / 4), kr, qr, v_s[j - hf * kHalfCols], g, bt, kq, ob + j, i4 == 0);
    }

    if (tid == 0) last_s = old == mapped_count(L, src) * 2 - 1;
    lds_barrier();
    if (last_s) {
        if (tid < 128) hist_store<DC>(p, bseq, ch, nh);
        if (tid == 0) counters[(size_t)bseq * L.h_k + src] = 0;
    }
}

// ---------------------------------------------------------------------------------------
// head_kernel: grid (h_v, B); workgroup = (sequence bseq, v head h), 512 threads, gated
// ---------------------------------------------------------------------------------------
// The gated decode with one workgroup per head: the slab kernel's column math over all 128
// columns (wave w owns columns 16 w + 2 u + half, u = 0..7), o collected in LDS, and the
// gated RMS norm of the head applied by wave 0 after one barrier, so no two workgroups
// exchange anything. The q/k conv history is written by the group's last member, found
// with the same counters as the slab kernel (one arrival per head instead of two).
constexpr int kHeadThreads = 512;
template <int DC>
__global__ void __launch_bounds__(kHeadThreads)
head_kernel(const DecodeParams p, const DecodeWs ws) {
    __shared__ __align__(16) float q_s[kD], k_s[kD], v_s[kD], o_s[kD];
    __shared__ float scal_s[2], gb_s[2];
    __shared__ int last_s;
    int* __restrict__ counters = ws.group;

    const Layer& L = p.L;
    const int tid = threadIdx.x, w = tid / kWave, lane = tid & (kWave - 1);
    const int half = lane >> 5, i4 = lane & 31;
    const int h = blockIdx.x, bseq = blockIdx.y;
    const int src = src_of(L, h);

    // Conv inputs: threads 0..63 q pairs, 64..127 k pairs, 128..191 the head's v pairs.
    int ch = 0;
    float* dst = nullptr;
    if (tid < 64) { ch = q_channel(L, src, 2 * tid); dst = q_s + 2 * tid; }
    else if (tid < 128) { ch = k_channel(L, src, 2 * (tid - 64)); dst = k_s + 2 * (tid - 64); }
    else if (tid < 192) { ch = v_channel(L, h, 2 * (tid - 128)); dst = v_s + 2 * (tid - 128); }
    const bool conv_thread = tid < 192;
    ConvPair<DC> cp;
    if (conv_thread) conv_pair_load<DC>(p, bseq, ch, cp);
    const size_t ab = (size_t)bseq * L.h_v + h;
    const uint16_t a_in = p.a[ab], b_in = p.b[ab];
    const size_t ob = ((size_t)bseq * L.h_v + h) * kD;
    GateIn gin{};
    if (w == 0) gin = gate_in(p.og, ob, lane);                     // the norm's inputs, loaded ahead

    v4f* tile = reinterpret_cast<v4f*>(p.state + ((size_t)bseq * L.h_v + h) * kD * kD) + i4;
    const int j0 = 2 * kPairsPerWave * w + half;
    v4f s[kPairsPerWave];
#pragma unroll
    for (int u = 0; u < kPairsPerWave; ++u) s[u] = __builtin_nontemporal_load(tile + (size_t)(j0 + 2 * u) * (kD / 4));

    uint32_t nh[DC - 1];
    float y0 = 0.0f, y1 = 0.0f;
    if (conv_thread) {
        conv_pair_eval<DC>(L, cp, y0, y1, nh);
        dst[0] = y0;
        dst[1] = y1;
        if (tid >= 128) hist_store<DC>(p, bseq, ch, nh);
    }
    if (w < 2) {
        const float r = wave_sum(fmaf(y0, y0, y1 * y1));
        if (lane == 0) scal_s[w] = r;
    }
    if (tid == kHeadThreads - 1) {
        gb_s[0] = expf(log_gate(L, h, bf16_to_f32(a_in)));
        gb_s[1] = sigmoid_f(bf16_to_f32(b_in));
    }
    lds_barrier();

    int old = 0;
    if (tid == 0) old = atomicAdd(counters + (size_t)bseq * L.h_k + src, 1);
    const float inv_q = L.q_scale / sqrtf(scal_s[0] + L.l2_eps);
    const float inv_k = 1.0f / sqrtf(scal_s[1] + L.l2_eps);
    const float kq = wave_sum(fmaf(q_s[lane], k_s[lane], q_s[lane + kWave] * k_s[lane + kWave])) * inv_q * inv_k;
    v4f kr, qr;
    {
        const v4f kk = *reinterpret_cast<const v4f*>(k_s + 4 * i4), qq = *reinterpret_cast<const v4f*>(q_s + 4 * i4);
#pragma unroll
        for (int e = 0; e < 4; ++e) { kr[e] = kk[e] * inv_k; qr[e] = qq[e] * inv_q; }
    }
    const float g = gb_s[0], bt = gb_s[1];
#pragma unroll
    for (int u = 0; u < kPairsPerWave; ++u) {
        const int j = j0 + 2 * u;
        const float ov = column_update(p, s[u], tile + (size_t)j * (kD / 4), kr, qr, v_s[j], g, bt, kq, ob + j, i4 == 0);
        if (i4 == 0) o_s[j] = ov;
    }
    if (tid == 0) last_s = old == mapped_count(L, src) - 1;
    lds_barrier();
    if (w == 0) out_gate_head(p.og, ob, o_s[lane], o_s[lane + kWave], lane, gin);
    if (last_s) {
        if (tid < 128) hist_store<DC>(p, bseq, ch, nh);
        if (tid == 0) counters[(size_t)bseq * L.h_k + src] = 0;
    }
}

// ---------------------------------------------------------------------------------------
// group_kernel: grid (h_k, B); workgroup = (sequence bseq, q/k head src), all mapped heads
// ---------------------------------------------------------------------------------------
constexpr int kGroupBatch = 4;                       // column pairs per load batch and wave

// Channel pair e of group (bseq, src): pairs 0..63 are q, 64..127 k, then 64 per mapped v head.
__device__ __forceinline__ int pair_channel(const Layer& L, int src, int e, float*& dst,
                                            float* q_s, float* k_s, float (*v_s)[kD]) {
    if (e < 64) { dst = q_s + 2 * e; return q_channel(L, src, 2 * e); }
    if (e < 128) { dst = k_s + 2 * (e - 64); return k_channel(L, src, 2 * (e - 64)); }
    const int t = (e - 128) / 64, j = 2 * ((e - 128) % 64);
    dst = v_s[t] + j;
    return v_channel(L, mapped_head(L, src, t), j);
}

template <int DC, bool GATED>
__global__ void __launch_bounds__(kThreads)
group_kernel(const DecodeParams p) {
    __shared__ __align__(16) float q_s[kD], k_s[kD];
    __shared__ __align__(16) float v_s[kMaxHeadsPerGroup][kD];
    __shared__ float o_s[GATED ? kMaxHeadsPerGroup : 1][kD];
    __shared__ float gate_s[kMaxHeadsPerGroup][2];
    __shared__ float scal_s[3];

    const Layer& L = p.L;
    const int src = blockIdx.x, bseq = blockIdx.y;
    const int tid = threadIdx.x, w = tid / kWave, lane = tid & (kWave - 1);
    const int half = lane >> 5, i4 = lane & 31;
    const int count = mapped_count(L, src);
    const int per_wave = count * (kD / 2) / (kThreads / kWave);     // column pairs of this wave
    const int p0 = w * per_wave;

    // Column pair pr of the group (head slot pr / 64) -> this lane's float4 of it.
    auto col_ptr = [&](int pr) -> v4f* {
        const int col = 2 * pr + half, t = col / kD, j = col % kD;
        return reinterpret_cast<v4f*>(p.state + (((size_t)bseq * L.h_v + mapped_head(L, src, t)) * kD + j) * kD) + i4;
    };
    auto load = [&](v4f (&buf)[kGroupBatch], int base) {
#pragma unroll
        for (int u = 0; u < kGroupBatch; ++u)
            if (base + u < per_wave) buf[u] = __builtin_nontemporal_load(col_ptr(p0 + base + u));
    };

    const int npairs = 128 + count * 64;
    float* dst0;
    const int ch0 = tid < npairs ? pair_channel(L, src, tid, dst0, q_s, k_s, v_s) : 0;
    ConvPair<DC> cp;
    if (tid < npairs) conv_pair_load<DC>(p, bseq, ch0, cp);
    v4f b0[kGroupBatch], b1[kGroupBatch];
    load(b0, 0);
    load(b1, kGroupBatch);
    if (tid < npairs) {
        uint32_t nh[DC - 1];
        conv_pair_eval<DC>(L, cp, dst0[0], dst0[1], nh);
        hist_store<DC>(p, bseq, ch0, nh);
    }
    for (int e = tid + kThreads; e < npairs; e += kThreads) {      // more than 2 v heads per q/k head
        float* dst;
        const int ch = pair_channel(L, src, e, dst, q_s, k_s, v_s);
        ConvPair<DC> c2;
        uint32_t nh[DC - 1];
        conv_pair_load<DC>(p, bseq, ch, c2);
        conv_pair_eval<DC>(L, c2, dst[0], dst[1], nh);
        hist_store<DC>(p, bseq, ch, nh);
    }
    if (tid < count) gates(p, bseq, mapped_head(L, src, tid), gate_s[tid]);
    __syncthreads();

    if (w < 3) {                                                  // q.q, k.k, q.k
        const float* x0 = (w == 1) ? k_s : q_s;
        const float* x1 = (w == 0) ? q_s : k_s;
        const float r = wave_sum(fmaf(x0[lane], x1[lane], x0[lane + kWave] * x1[lane + kWave]));
        if (lane == 0) scal_s[w] = r;
    }
    __syncthreads();
    const float inv_q = L.q_scale / sqrtf(scal_s[0] + L.l2_eps);
    const float inv_k = 1.0f / sqrtf(scal_s[1] + L.l2_eps);
    const float kq = scal_s[2] * inv_q * inv_k;
    v4f kr, qr;
#pragma unroll
    for (int e = 0; e < 4; ++e) { kr[e] = k_s[4 * i4 + e] * inv_k; qr[e] = q_s[4 * i4 + e] * inv_q; }

    auto process = [&](v4f (&buf)[kGroupBatch], int base) {
#pragma unroll
        for (int u = 0; u < kGroupBatch; ++u) {
            if (base + u >= per_wave) break;
            const int pr = p0 + base + u, col = 2 * pr + half, t = col / kD, j = col % kD;
            const size_t oi = ((size_t)bseq * L.h_v + mapped_head(L, src, t)) * kD + j;
            const float ov =
                column_update(p, buf[u], col_ptr(pr), kr, qr, v_s[t][j], gate_s[t][0], gate_s[t][1], kq, oi, i4 == 0);
            if (GATED && i4 == 0) o_s[t][j] = ov;
        }
    };
    // Two batches in flight; the loop body is unrolled so no register is copied while its
    // load is outstanding.
    for (int base = 0; base < per_wave; base += 2 * kGroupBatch) {
        process(b0, base);
        load(b0, base + 2 * kGroupBatch);
        process(b1, base + kGroupBatch);
        load(b1, base + 3 * kGroupBatch);
    }
    if constexpr (GATED) {
        __syncthreads();
        for (int t = w; t < count; t += kThreads / kWave)
            out_gate_head(p.og, ((size_t)bseq * L.h_v + mapped_head(L, src, t)) * kD, o_s[t][lane],
                          o_s[t][lane + kWave], lane);
    }
}

// The slab kernel needs every q/k head to feed at least one v head (its history is written
// by the group's last member); otherwise, and without counters, one workgroup owns each
// group.
inline bool every_src_used(const ix_gdn_cfg* cfg) {
    return cfg->head_map == IX_GDN_HEAD_DIV || cfg->h_v >= cfg->h_k;
}

inline DecodeWs bind_decode_ws(void* workspace) { return DecodeWs{static_cast<int*>(workspace)}; }

// Occupancy cap of the slab kernel when every CU has at least kSlabCapPerCu workgroups to run
// (B >= 32 at h_v = 32): the launch reserves kSlabLdsReserve bytes of LDS per workgroup, which
// no code touches, so that at most two workgroups share a CU. With fewer workgroups in flight
// each one waits less behind the others' state loads (the whole launch stays HBM-bound), and
// B = 64 runs in exactly 8 rounds: 45.9-46.5 against 47.3-48.2 us per launch, B = 96 67.7
// against 69.9, B = 128 89.9 against 92.2. At B <= 24 the uncapped launch is faster.
constexpr int kSlabCapPerCu = 8;
constexpr unsigned kSlabLdsReserve = 64 * 1024;           // more than a third of a CU's 160 KiB

// ws: the group counters, or null for the group kernel.
template <bool GATED>
void launch_decode(const ix_gdn_cfg* cfg, int B, const DecodeParams& p, const DecodeWs* ws, hipStream_t s) {
    const dim3 block(kThreads);
    if (ws && every_src_used(cfg) && GATED) {
        const dim3 grid((unsigned)cfg->h_v, (unsigned)B), hblock(kHeadThreads);
        switch (cfg->d_conv) {
            case 2: hipLaunchKernelGGL(head_kernel<2>, grid, hblock, 0, s, p, *ws); break;
            case 3: hipLaunchKernelGGL(head_kernel<3>, grid, hblock, 0, s, p, *ws); break;
            default: hipLaunchKernelGGL(head_kernel<4>, grid, hblock, 0, s, p, *ws); break;
        }
    } else if (ws && every_src_used(cfg)) {
        const dim3 grid((unsigned)(2 * cfg->h_v), (unsigned)B);
        const long long nwg = 2LL * cfg->h_v * B;
        const int cus = device_cu_count(s);
        const unsigned lds = nwg >= (long long)kSlabCapPerCu * cus ? kSlabLdsReserve : 0;
        if (nwg <= cus) {                                     // B <= 4 at h_v = 32
            constexpr int NT = kSmallGridThreads;
            switch (cfg->d_conv) {
                case 2: hipLaunchKernelGGL((slab_kernel<2, NT>), grid, dim3(NT), 0, s, p, *ws); break;
                case 3: hipLaunchKernelGGL((slab_kernel<3, NT>), grid, dim3(NT), 0, s, p, *ws); break;
                default: hipLaunchKernelGGL((slab_kernel<4, NT>), grid, dim3(NT), 0, s, p, *ws); break;
            }
        } else {
            switch (cfg->d_conv) {
                case 2: hipLaunchKernelGGL((slab_kernel<2, kThreads>), grid, block, lds, s, p, *ws); break;
                case 3: hipLaunchKernelGGL((slab_kernel<3, kThreads>), grid, block, lds, s, p, *ws); break;
                default: hipLaunchKernelGGL((slab_kernel<4, kThreads>), grid, block, lds, s, p, *ws); break;
            }
        }
    } else {
        const dim3 grid((unsigned)cfg->h_k, (unsigned)B);
        switch (cfg->d_conv) {
            case 2: hipLaunchKernelGGL((group_kernel<2, GATED>), grid, block, 0, s, p); break;
            case 3: hipLaunchKernelGGL((group_kernel<3, GATED>), grid, block, 0, s, p); break;
            default: hipLaunchKernelGGL((group_kernel<4, GATED>), grid, block, 0, s, p); break;
        }
    }
}

}  // namespace
}  // namespace ixg

extern "C" int ix_gdn_channels(const ix_gdn_cfg* c) {
    return c ? 2 * c->h_k * c->d_k + c->h_v * c->d_v : 0;
}

extern "C" const char* ix_gdn_version(void) { return "ixgdn 0.5.0 gfx950"; }

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

extern "C" size_t ix_gdn_decode_workspace_size(const ix_gdn_cfg* cfg, int B) {
    if (ix_gdn_check_cfg_(cfg) != hipSuccess || B <= 0 || B > 65535) return 0;
    return ixg::decode_ws_bytes(B, cfg->h_k);
}

// Validation and parameter set-up shared by the plain and gated decode.
static hipError_t decode_params(const ix_gdn_cfg* cfg, int B, const uint16_t* x, uint16_t* conv_state,
                                const uint16_t* conv_w, const uint16_t* a, const uint16_t* b, const float* A_log,
                                const float* dt_bias, float* state, float* o, uint16_t* o_bf16, void* workspace,
                                ixg::DecodeParams& p) {
    const hipError_t e = ix_gdn_check_cfg_(cfg);
    if (e != hipSuccess) return e;
    if (B <= 0 || B > 65535) return hipErrorInvalidValue;
    if (!x || !conv_state || !conv_w || !a || !b || !A_log || !dt_bias || !state) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(state) & 15) || (o && (reinterpret_cast<uintptr_t>(o) & 3)) ||
        (o_bf16 && (reinterpret_cast<uintptr_t>(o_bf16) & 1)))
        return hipErrorInvalidValue;                 // float4 state accesses
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(conv_state) |
         reinterpret_cast<uintptr_t>(conv_w) | reinterpret_cast<uintptr_t>(workspace)) & 3)
        return hipErrorInvalidValue;                 // conv inputs and counters are dwords
    p.L = ixg::make_layer(cfg, conv_w, A_log, dt_bias);
    p.x = x; p.conv_state = conv_state; p.a = a; p.b = b;
    p.state = state; p.o = o; p.o_bf16 = o_bf16;
    p.og = ixg::OutGate{};
    return hipSuccess;
}

// The gate description of the gated calls: z and ssm_norm, at least one output, aligned.
extern "C" hipError_t ix_gdn_check_gate_(const ix_gdn_out_gate* g) {
    if (!g || !g->z || !g->ssm_norm || (!g->y && !g->y_bf16 && !g->y_q8_1)) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(g->z) & 1) || (reinterpret_cast<uintptr_t>(g->ssm_norm) & 3) ||
        (reinterpret_cast<uintptr_t>(g->y) & 3) || (reinterpret_cast<uintptr_t>(g->y_bf16) & 1) ||
        (reinterpret_cast<uintptr_t>(g->y_q8_1) & 3))
        return hipErrorInvalidValue;
    return hipSuccess;
}

extern "C" hipError_t ix_gdn_decode(const ix_gdn_cfg* cfg, int B, const uint16_t* x, uint16_t* conv_state,
                                    const uint16_t* conv_w, const uint16_t* a, const uint16_t* b,
                                    const float* A_log, const float* dt_bias, float* state, float* o,
                                    uint16_t* o_bf16, void* workspace, hipStream_t s) {
    ixg::DecodeParams p;
    const hipError_t e = decode_params(cfg, B, x, conv_state, conv_w, a, b, A_log, dt_bias, state, o, o_bf16,
                                       workspace, p);
    if (e != hipSuccess) return e;
    if (workspace) {
        const ixg::DecodeWs ws = ixg::bind_decode_ws(workspace);
        ixg::launch_decode<false>(cfg, B, p, &ws, s);
    } else {
        ixg::launch_decode<false>(cfg, B, p, nullptr, s);
    }
    return hipGetLastError();
}

extern "C" hipError_t ix_gdn_decode_gated(const ix_gdn_cfg* cfg, int B, const uint16_t* x, uint16_t* conv_state,
                                          const uint16_t* conv_w, const uint16_t* a, const uint16_t* b,
                                          const float* A_log, const float* dt_bias, float* state, float* o,
                                          uint16_t* o_bf16, const ix_gdn_out_gate* gate, void* workspace,
                                          hipStream_t s) {
    ixg::DecodeParams p;
    hipError_t e = decode_params(cfg, B, x, conv_state, conv_w, a, b, A_log, dt_bias, state, o, o_bf16,
                                 workspace, p);
    if (e != hipSuccess) return e;
    if ((e = ix_gdn_check_gate_(gate)) != hipSuccess) return e;
    p.og = ixg::make_out_gate(gate);
    if (workspace) {
        const ixg::DecodeWs ws = ixg::bind_decode_ws(workspace);
        ixg::launch_decode<true>(cfg, B, p, &ws, s);
    } else {
        ixg::launch_decode<true>(cfg, B, p, nullptr, s);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// ix_gdn_decode_noalloc: ix_gdn_decode's counter-workspace kernel with the group counters in
// a library-owned static device array instead of a caller workspace, so the call allocates
// nothing. Each GPU holds its own copy of the array (256 KiB) until the process ends.
// ---------------------------------------------------------------------------------------
constexpr int kNoAllocMaxGroups = 65536;                 // B * h_k counters
static __device__ __align__(256) int scratch[kNoAllocMaxGroups];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
int* g_scratch_dev[kMaxDevices];                         // device address of `scratch`, per GPU

// The current device's copy of `scratch`: its address, taken on the first call on a device
// (the host-side name is only a stand-in for it). The array is zero when the code object is
// loaded (static storage), and every kernel that counts in it resets each counter it used
// to zero, so it is all zero between calls; no call clears it, so nothing but the decode
// kernel itself is enqueued (also when the first call happens under graph capture).
hipError_t noalloc_counters(int** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_dev[dev] = static_cast<int*>(ptr);
    }
    *out = g_scratch_dev[dev];
    return hipSuccess;
}
}  // namespace

extern "C" hipError_t ix_gdn_decode_noalloc(const ix_gdn_cfg* cfg, int B, const uint16_t* x, uint16_t* conv_state,
                                            const uint16_t* conv_w, const uint16_t* a, const uint16_t* b,
                                            const float* A_log, const float* dt_bias, float* state, float* o,
                                            uint16_t* o_bf16, hipStream_t s) {
    ixg::DecodeParams p;
    hipError_t e = decode_params(cfg, B, x, conv_state, conv_w, a, b, A_log, dt_bias, state, o, o_bf16, nullptr, p);
    if (e != hipSuccess) return e;
    if ((long long)B * cfg->h_k > kNoAllocMaxGroups) return hipErrorInvalidValue;   // beyond the static array
    if (!ixg::every_src_used(cfg)) {                     // the group kernel needs no counters
        ixg::launch_decode<false>(cfg, B, p, nullptr, s);
        return hipGetLastError();
    }
    int* counters = nullptr;
    if ((e = noalloc_counters(&counters)) != hipSuccess) return e;
    const ixg::DecodeWs ws{counters};
    ixg::launch_decode<false>(cfg, B, p, &ws, s);
    return hipGetLastError();
}
