// gdn_prefill.hip -- chunked GDN prefill for gfx950 (ix_gdn_prefill).
//
// The same math as applying the fused decode token by token (conv, L2 norms, gates, head
// map, delta rule; the reference's step is src/ix_gdn.cu:25-56), regrouped into chunks of
// C = 64 tokens so that most of the work is dense contractions on the matrix cores.
//
// Within a chunk of one v head, with G_t the inclusive cumulative log decay, Gam_t =
// exp(G_t), beta_t, normalised keys k_t and queries q_t, and S the state at chunk start
// (d_k x d_v), unrolling S_t = g_t S_{t-1} + k_t d_t^T with
// d_t = beta_t (v_t - g_t S_{t-1}^T k_t) gives
//   A[t][s] = beta_t exp(G_t - G_s) (k_t . k_s)            (s < t)
//   T'      = (I + A)^-1 diag(beta)                         (lower triangular)
//   D       = T' (V - diag(Gam) K S)                        (rows d_t)
//   M[t][s] = exp(G_t - G_s) (q_t . k_s)                    (s <= t)
//   O       = diag(Gam) Q S + M D
//   S'      = Gam_last S + K^T diag(exp(G_last - G_s)) D
// (D is the WY form's U - W S with U = T' V and W = T' diag(Gam) K, applied to S without
// forming W.) Only differences G_t - G_s with t >= s are exponentiated, so no intermediate
// overflows however strong the decay (Gam_t itself may underflow to 0, its correct value).
//
// Kernels, in stream order, per window of chunks (the workspace holds one window's chunk
// operands; windows run one after the other, with identical results for any window size):
//   plan_kernel    (once, n_seq > 1 only) clamps cu_seqlens to a non-decreasing sequence in
//                  [0, total_T], builds the chunk table and lists the non-empty sequences;
//                  a single sequence's geometry comes from cu[0], cu[1] directly
//   tri_kernel     per (chunk, q/k head): conv and L2 norms of the chunk's q and k rows, the
//                  K K^T and Q K^T lower block triangles once for all the v heads mapped to the
//                  q/k head, then per v head the decay scan and beta, A and M, T = (I + A)^-1
//                  (diagonal blocks by substitution, the rest by block forward substitution)
//                  and T' = T diag(beta); it writes the chain's operands in their final
//                  layouts: key planes, Q, M and T' as split-bf16 MFMA fragments, decay factors
//   chain_kernel   per (v head, 16-column state strip, group of sequences): walks the window's
//                  chunks of its sequences in order, across sequence boundaries, two phases per
//                  chunk (roles below), and writes the outputs, the states and, after each
//                  sequence's last chunk, its new conv history
//   out_gate_*     (ix_gdn_prefill_gated) the gated RMS output norm of every (token, head) row
// Every dense product runs on split-bf16 MFMA (three bf16 products per fp32 product, ~2^-16
// relative error); only the 16 x 16 diagonal blocks of T are inverted in fp32 arithmetic.
// The chunked result stays within ~1e-5 (state) of the token-by-token recurrence in double.
#include "gdn_common.h"

namespace ixg {
namespace {

constexpr int kChunk = 64;
constexpr int kPlanThreads = 1024;

// ---------------------------------------------------------------------------------------
// Workspace layout (host and device agree through this struct)
// ---------------------------------------------------------------------------------------
// The chunk tables cover every chunk; the chunk operands cover one window of W chunks (the
// kernels run window by window, W chosen to fit the caller's workspace).
struct Ws {
    int32_t* seq_lo;     // [n_seq + 1] clamped token offsets
    int32_t* chunk_off;  // [n_seq + 1] first chunk of each sequence; chunk_off[n_seq] = #chunks
    int4* chunk_rec;     // [NC] {sequence, first token, sequence start, sequence end}
    uint8_t* Tf;         // [W][h_v] T' = (I + A)^-1 diag(beta) (64 x 64) as split-bf16 A fragments
                         // (the nonzero ones, kTriFragBytes per head)
    uint8_t* Mf;         // [W][h_v] M (64 x 64) as split-bf16 A fragments (kFragMBytes per head)
    float* G;            // [W][h_v][2][64] decay factors exp(G_last - G_t), then exp(G_t), of the
                         // inclusive cumulative log decay G (padded rows repeat the last)
    uint8_t* Kp;         // [W][h_k] normalised keys as split-bf16 planes in the chain's LDS layout
    uint16_t* Qf;        // [W][h_k] Q (64 x 128) as split-bf16 A fragments
};
constexpr int kWsSections = 8;
constexpr int kTriFragBytes = 10 * 1024;                // T' of one (chunk, v head)
constexpr int kFragMBytes = 16 * 1024;                  // M of one (chunk, v head)
constexpr int kPRow = 2 * 128;                          // key plane row: 128 bf16 as 16 chunks of 16 bytes
constexpr int kKPlane = 64 * kPRow;                     // one plane (hi or lo) of 64 keys
constexpr int kKSlot = 2 * kKPlane;                     // hi, then lo: 32 KiB
// Chunk j of key row t is stored at chunk j ^ kswz(t) of its row: the two 2-bit halves of
// t mod 16 swapped, so that the chain's 16-byte fragment reads (16 rows, one chunk column) and
// its transposing 8-byte reads (4 rows x 4 chunk columns per lane group) hit 16 distinct chunks.
__host__ __device__ constexpr int kswz(int t) { return ((t & 3) << 2) | ((t >> 2) & 3); }

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Chunks of (n_seq, T) at most: each sequence adds at most one partial chunk.
inline size_t max_chunks(int n_seq, int T) { return (size_t)(T + kChunk - 1) / kChunk + (size_t)n_seq; }

// Byte offsets of every workspace section for (n_seq, T) in windows of W chunks; returns the
// total size.
inline size_t ws_layout(const ix_gdn_cfg* c, int n_seq, int T, size_t W, size_t off[kWsSections]) {
    const size_t NC = max_chunks(n_seq, T);
    const size_t sz[kWsSections] = {
        sizeof(int32_t) * (n_seq + 1), sizeof(int32_t) * (n_seq + 1), sizeof(int4) * NC,
        (size_t)kTriFragBytes * W * c->h_v, (size_t)kFragMBytes * W * c->h_v, sizeof(float) * W * c->h_v * 2 * kChunk, (size_t)kKSlot * W * c->h_k,
        sizeof(uint16_t) * W * c->h_k * 4 * 4 * 2 * 512,
    };
    size_t pos = 0;
    for (int i = 0; i < kWsSections; ++i) { off[i] = pos; pos += align256(sz[i]); }
    return pos;
}

inline Ws ws_bind(char* base, const size_t off[kWsSections]) {
    Ws w;
    w.seq_lo = reinterpret_cast<int32_t*>(base + off[0]);
    w.chunk_off = reinterpret_cast<int32_t*>(base + off[1]);
    w.chunk_rec = reinterpret_cast<int4*>(base + off[2]);
    w.Tf = reinterpret_cast<uint8_t*>(base + off[3]);
    w.Mf = reinterpret_cast<uint8_t*>(base + off[4]);
    w.G = reinterpret_cast<float*>(base + off[5]);
    w.Kp = reinterpret_cast<uint8_t*>(base + off[6]);
    w.Qf = reinterpret_cast<uint16_t*>(base + off[7]);
    return w;
}

struct PrefillParams {
    Layer L;
    Ws ws;
    const int32_t* cu;          // [n_seq + 1]
    const uint16_t* x;          // [T][C]
    uint16_t* conv_state;       // [n_seq][C][dc-1]
    const uint16_t* a;          // [T][h_v]
    const uint16_t* b;          // [T][h_v]
    float* state;               // [n_seq][h_v][d_v][d_k]
    float* o;                   // [T][h_v][128], the window's rows (o_win), or null
    uint16_t* o_bf16;           // [T][h_v][128] or null
    int n_seq, T, NC;
    int single;                 // n_seq == 1: no plan pass; the geometry comes from cu[0], cu[1]
    int cb, W;                  // the window: chunks cb .. cb + W - 1
    int G;                      // chain workgroups per (v head, strip) in a window (1 for n_seq == 1)
    int o_win;                  // o holds the window's tokens only (row 0 = its first token)
};

// Clamped bounds [lo, hi) of sequence s: the plan's seq_lo (running maximum of the offsets,
// clamped to [0, T]), or for a single sequence the same two values from cu directly.
__device__ __forceinline__ void seq_bounds(const PrefillParams& p, int s, int& lo, int& hi) {
    if (p.single) {
        lo = min(max(p.cu[0], 0), p.T);
        hi = max(min(max(p.cu[1], 0), p.T), lo);
    } else {
        lo = p.ws.seq_lo[s];
        hi = p.ws.seq_lo[s + 1];
    }
}

// ---------------------------------------------------------------------------------------
// plan: one workgroup of 1024 threads, block scans in tiles of 1024 sequences
// ---------------------------------------------------------------------------------------
// Inclusive scan (max or sum) over the workgroup: within each wave by shuffles, then over
// the 16 wave totals by wave 0; two barriers.
template <bool IsMax>
__device__ int block_inclusive_scan(int v, int* wave_tot) {
    const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const int o = __shfl_up(v, off, kWave);
        if (lane >= off) v = IsMax ? max(v, o) : v + o;
    }
    if (lane == kWave - 1) wave_tot[w] = v;
    __syncthreads();
    if (w == 0) {
        int t = lane < kPlanThreads / kWave ? wave_tot[lane] : (IsMax ? INT_MIN : 0);
#pragma unroll
        for (int off = 1; off < kPlanThreads / kWave; off <<= 1) {
            const int o = __shfl_up(t, off, kWave);
            if (lane >= off) t = IsMax ? max(t, o) : t + o;
        }
        if (lane < kPlanThreads / kWave) wave_tot[lane] = t;          // inclusive totals
    }
    __syncthreads();
    if (w > 0) v = IsMax ? max(v, wave_tot[w - 1]) : v + wave_tot[w - 1];
    return v;
}

__global__ void __launch_bounds__(kPlanThreads) plan_kernel(const PrefillParams p) {
    __shared__ int wave_tot[kPlanThreads / kWave];
    __shared__ int carry;
    const int tid = threadIdx.x, n = p.n_seq;
    // seq_lo[s] = clamp(max(cu[0..s]), 0, T), s = 0..n
    int run = 0;                                                       // carry, same in every thread
    for (int base = 0; base <= n; base += kPlanThreads) {
        const int s = base + tid;
        int v = s <= n ? min(max(p.cu[s], 0), p.T) : 0;
        v = max(block_inclusive_scan<true>(v, wave_tot), run);
        if (s <= n) p.ws.seq_lo[s] = v;
        if (tid == kPlanThreads - 1) carry = v;
        __syncthreads();
        run = carry;
        __syncthreads();
    }
    // chunk_off = exclusive prefix sum of ceil(len / 64)
    run = 0;
    for (int base = 0; base <= n; base += kPlanThreads) {
        const int s = base + tid;
        const int cnt = s < n ? (p.ws.seq_lo[s + 1] - p.ws.seq_lo[s] + kChunk - 1) / kChunk : 0;
        const int inc = block_inclusive_scan<false>(cnt, wave_tot) + run;
        if (s <= n) p.ws.chunk_off[s] = inc - cnt;
        if (tid == kPlanThreads - 1) carry = inc;
        __syncthreads();
        run = carry;
        __syncthreads();
    }
    const int nc = run;
    // the chunk table: chunk c belongs to the last sequence s with chunk_off[s] <= c
    for (int c = tid; c < nc; c += kPlanThreads) {
        int lo = 0, hi = n - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (p.ws.chunk_off[mid] <= c) lo = mid; else hi = mid - 1;
        }
        const int s0 = p.ws.seq_lo[lo];
        p.ws.chunk_rec[c] = int4{lo, s0 + (c - p.ws.chunk_off[lo]) * kChunk, s0, p.ws.seq_lo[lo + 1]};
    }
}

// Chunk geometry: sequence, first token, tokens in the chunk, position of the first token
// within its sequence. Returns false for grid slots beyond the chunk count.
// One load for the whole geometry (the chunk count is read alongside, independently).
struct ChunkGeo { int s, t0, len, pos0, lo; };
__device__ __forceinline__ bool chunk_geo(const PrefillParams& p, int c, ChunkGeo& g) {
    if (p.single) {                                   // chunk c of the only sequence
        int lo, hi;
        seq_bounds(p, 0, lo, hi);
        const int t0 = lo + c * kChunk;
        if (t0 >= hi) return false;
        g.s = 0;
        g.t0 = t0;
        g.lo = lo;
        g.len = min(kChunk, hi - t0);
        g.pos0 = t0 - lo;
        return true;
    }
    const int nc = p.ws.chunk_off[p.n_seq];
    const int4 r = p.ws.chunk_rec[min(c, p.NC - 1)];
    if (c >= nc) return false;
    g.s = r.x;
    g.t0 = r.y;
    g.lo = r.z;
    g.len = min(kChunk, r.w - g.t0);
    g.pos0 = g.t0 - g.lo;
    return true;
}

// Tokens [t0, t1) of the window's chunks (consecutive chunks cover consecutive tokens); t0 = t1
// for a window past the last chunk.
__device__ __forceinline__ void window_tokens(const PrefillParams& p, int& t0, int& t1) {
    ChunkGeo a, b;
    t0 = t1 = 0;
    if (!chunk_geo(p, p.cb, a)) return;
    int nc;
    if (p.single) {
        int lo, hi;
        seq_bounds(p, 0, lo, hi);
        nc = (hi - lo + kChunk - 1) / kChunk;
    } else {
        nc = p.ws.chunk_off[p.n_seq];
    }
    chunk_geo(p, min(p.cb + p.W, nc) - 1, b);               // chunk cb exists, so this one does
    t0 = a.t0;
    t1 = b.t0 + b.len;
}

// ---------------------------------------------------------------------------------------
// Conv of 16 consecutive tokens of a chunk for the channel pair (ch, ch + 1), one pair per
// lane, so that every x access of a wave is one 256-byte row segment. Tokens tb .. tb + n - 1
// of the chunk (n wave-uniform, 1..16); the history of the first one comes from x or, before
// the sequence start, from the sequence's conv state ([C][dc-1] per sequence: channel ch's
// entries, then channel ch+1's).
// The loads and the arithmetic are separate steps, so that a wave can issue the loads well
// before it needs the rows (and before stores it issues in between, which its later waits
// would otherwise include).
// ---------------------------------------------------------------------------------------
constexpr int kConvTok = 16;

// The loads are unconditional and nothing touches the loaded words before conv_run: a
// load on one path only, or any use of a loaded value, makes the wave wait for every load
// it has in flight. Every row index is clamped into the chunk's tokens, so a wave whose
// rows all lie past the chunk end (n = 0) reads valid rows, whose results are discarded.
template <int DC>
struct ConvIn {
    uint32_t h0[DC - 1], h1[DC - 1];    // history of the first token (one bf16 each), oldest first
    uint32_t xs[kConvTok];              // bf16 pairs: inputs of the tokens (rows past n repeat row n-1)
    uint32_t w[DC];                     // bf16 pairs: conv weights of channel ch, then ch + 1
};

template <int DC>
__device__ __forceinline__ void conv_load(const PrefillParams& p, const ChunkGeo& g, int lo, int ch, int tb, int n,
                                          ConvIn<DC>& in) {
    const Layer& L = p.L;
#pragma unroll
    for (int i = 0; i < DC - 1; ++i) {
        const int pos = min(g.pos0 + tb - (DC - 1) + i, g.pos0 + g.len - 1);   // wave-uniform
        const uint16_t* xp = p.x + (size_t)(lo + max(pos, 0)) * L.C + ch;
        const uint16_t* sp = p.conv_state + ((size_t)g.s * L.C + ch) * (DC - 1) + (DC - 1) + min(pos, -1);
        in.h0[i] = *(pos >= 0 ? xp : sp);
        in.h1[i] = *(pos >= 0 ? xp + 1 : sp + (DC - 1));
    }
#pragma unroll
    for (int t = 0; t < kConvTok; ++t)
        in.xs[t] = *reinterpret_cast<const uint32_t*>(p.x + (size_t)(g.t0 + min(tb + min(t, n - 1), g.len - 1)) * L.C + ch);
    // conv_w is [C][dc]: the two channels' 2 dc weights are dc aligned words (ch is even)
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(L.conv_w + (size_t)ch * DC);
#pragma unroll
    for (int i = 0; i < DC; ++i) in.w[i] = wp[i];
}

__device__ __forceinline__ float bf16_half(uint32_t word, int half) {
    return __uint_as_float(half ? (word & 0xffff0000u) : (word << 16));
}

template <int DC, bool SILU>
__device__ __forceinline__ void conv_run(ConvIn<DC> in, float (&y0)[kConvTok], float (&y1)[kConvTok]) {
    // Pin the words here: the compiler would otherwise hoist their unpacking up to the loads,
    // which then wait for the data right after issue.
#pragma unroll
    for (int i = 0; i < DC - 1; ++i) { __asm__ volatile("" : "+v"(in.h0[i])); __asm__ volatile("" : "+v"(in.h1[i])); }
#pragma unroll
    for (int t = 0; t < kConvTok; ++t) __asm__ volatile("" : "+v"(in.xs[t]));
#pragma unroll
    for (int i = 0; i < DC; ++i) __asm__ volatile("" : "+v"(in.w[i]));
    float h0[DC - 1], h1[DC - 1], w0[DC], w1[DC];
#pragma unroll
    for (int i = 0; i < DC - 1; ++i) { h0[i] = __uint_as_float(in.h0[i] << 16); h1[i] = __uint_as_float(in.h1[i] << 16); }
#pragma unroll
    for (int i = 0; i < DC; ++i) {
        w0[i] = bf16_half(in.w[i >> 1], i & 1);
        w1[i] = bf16_half(in.w[(DC + i) >> 1], (DC + i) & 1);
    }
#pragma unroll
    for (int t = 0; t < kConvTok; ++t) {
        const float x0 = bf16_half(in.xs[t], 0), x1 = bf16_half(in.xs[t], 1);
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int i = 0; i < DC - 1; ++i) { a0 = fmaf(h0[i], w0[i], a0); a1 = fmaf(h1[i], w1[i], a1); }
        a0 = fmaf(x0, w0[DC - 1], a0);
        a1 = fmaf(x1, w1[DC - 1], a1);
        if constexpr (SILU) { a0 = a0 * sigmoid_f(a0); a1 = a1 * sigmoid_f(a1); }
        y0[t] = a0;
        y1[t] = a1;
#pragma unroll
        for (int i = 0; i < DC - 2; ++i) { h0[i] = h0[i + 1]; h1[i] = h1[i + 1]; }
        h0[DC - 2] = x0;
        h1[DC - 2] = x1;
    }
}

// ---------------------------------------------------------------------------------------
// commit: the rolling conv history of channel ch after sequence s, tokens lo .. lo+len-1
// (len > 0); run by the chain kernel after every read of the old history
// ---------------------------------------------------------------------------------------
// The new history's dc-1 values, loaded (hist_fetch), then stored (hist_put) once they have
// arrived, so that a wave can issue other loads in between.
struct HistNew { uint16_t v[3]; };
__device__ __forceinline__ HistNew hist_fetch(const PrefillParams& p, int ch, int lo, int len, int s) {
    const Layer& L = p.L;
    const uint16_t* st = p.conv_state + ((size_t)s * L.C + ch) * (L.dc - 1);
    // extended history [old (dc-1 values) | the sequence's inputs]; the new history is its
    // last dc-1 entries, i.e. entries len .. len+dc-2. An entry below dc-1 is old history.
    const uint16_t o0 = st[0], o1 = L.dc > 2 ? st[1] : (uint16_t)0, o2 = L.dc > 3 ? st[2] : (uint16_t)0;
    // Entries j >= dc-1 are not stored; their token index is clamped into the sequence, so
    // that no load reaches past its last token.
    HistNew h;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int ext = len + j;                               // index into the extended history
        const int pos = ext - (L.dc - 1);                      // token position when >= 0
        h.v[j] = pos >= 0 ? p.x[(size_t)(lo + min(pos, len - 1)) * L.C + ch] : (ext == 0 ? o0 : ext == 1 ? o1 : o2);
    }
    return h;
}
__device__ __forceinline__ void hist_put(const PrefillParams& p, int ch, int s, const HistNew& h) {
    const Layer& L = p.L;
    uint16_t* st = p.conv_state + ((size_t)s * L.C + ch) * (L.dc - 1);
    st[0] = h.v[0];
    if (L.dc > 2) st[1] = h.v[1];
    if (L.dc > 3) st[2] = h.v[2];
}

// ---------------------------------------------------------------------------------------
// Split-bf16 operand fragments.
//
// The chain runs its products on v_mfma_f32_16x16x32_bf16 with each fp32 operand x split
// into x_hi = bf16(x) and x_lo = bf16(x - x_hi); a product is hi*hi + hi*lo + lo*hi in fp32
// accumulators (relative error ~2^-16, against 2^-8 for one bf16 product). The chunk kernel
// writes the chain's A operands already split, in the instruction's A layout: fragment
// (m, ks) of a (rows x k) tile covers rows 16m..16m+15 and k = 32ks..32ks+31, and lane l of
// it holds row 16m + l%16 at the 8 k indices 32ks + kperm(l/16, e), e = 0..7, as 8 bf16
// (16 bytes). Stored [m][ks][plane hi, lo][lane][8]: one coalesced 16-byte load per lane
// per fragment and plane.
// kperm is the row order of two stacked MFMA accumulator tiles (lane group g holds rows
// 4g..4g+3 of each), so the chain feeds its accumulators (S, D) to the next product as B
// operands without moving them between lanes; A and B agree on the order of the k sum.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ size_t frag_at(int m, int ks, int nks, int plane, int lane) {
    return ((((size_t)m * nks + ks) * 2 + plane) * kWave + lane) * 8;       // in bf16 elements
}

__device__ __forceinline__ void store_frag(uint8_t* base, int m, int ks, int nks, int lane, const bf8& hi, const bf8& lo) {
    *reinterpret_cast<bf8*>(base + 2 * frag_at(m, ks, nks, 0, lane)) = hi;
    *reinterpret_cast<bf8*>(base + 2 * frag_at(m, ks, nks, 1, lane)) = lo;
}

// T' (64 x 64, lower triangular, split) stores its 6 nonzero fragments back to back, (0, 0),
// (1, 0), (2, 0), (2, 1), (3, 0), (3, 1); (0, 0) and (2, 1) pair a diagonal block with a zero
// block, so only entries 0..3 of each lane are stored (8 bytes a lane, 512 a plane). Byte offset
// of a lane's part of one plane:
__host__ __device__ constexpr bool tri_half(int m, int ks) { return (m == 0 && ks == 0) || (m == 2 && ks == 1); }
__device__ __forceinline__ int tri_frag_at(int m, int ks, int plane, int lane) {
    const int off = m == 0 ? 0 : m == 1 ? 1024 : m == 2 ? (ks ? 5120 : 3072) : (ks ? 8192 : 6144);
    return off + (tri_half(m, ks) ? plane * 512 + lane * 8 : plane * 1024 + lane * 16);
}
__device__ __forceinline__ void store_tri_frag(uint8_t* base, int m, int ks, int lane, const bf8& hi, const bf8& lo) {
    if (tri_half(m, ks)) {
        const u4x h = __builtin_bit_cast(u4x, hi), l = __builtin_bit_cast(u4x, lo);
        *reinterpret_cast<uint2*>(base + tri_frag_at(m, ks, 0, lane)) = uint2{h.x, h.y};
        *reinterpret_cast<uint2*>(base + tri_frag_at(m, ks, 1, lane)) = uint2{l.x, l.y};
    } else {
        *reinterpret_cast<bf8*>(base + tri_frag_at(m, ks, 0, lane)) = hi;
        *reinterpret_cast<bf8*>(base + tri_frag_at(m, ks, 1, lane)) = lo;
    }
}
// The whole fragment plane (zeros in a half fragment's entries 4..7); m and ks are compile-time
// constants where it is used.
__device__ __forceinline__ u4x load_tri_frag(const uint8_t* base, int m, int ks, int plane, int lane) {
    if (tri_half(m, ks)) {
        const uint2 v = *reinterpret_cast<const uint2*>(base + tri_frag_at(m, ks, plane, lane));
        return u4x{v.x, v.y, 0u, 0u};
    }
    return *reinterpret_cast<const u4x*>(base + tri_frag_at(m, ks, plane, lane));
}

// Fragment sizes in bf16 elements: (rows/16) x (k/32) fragments x 2 planes x 512.
constexpr size_t kFragW = 4 * 4 * 2 * 512;     // 64 x 128 (Q)

// ---------------------------------------------------------------------------------------
// chunk-local work (tri_kernel): grid (NC, h_k), 512 threads; workgroup = (chunk, q/k head)
// ---------------------------------------------------------------------------------------
constexpr int kTS = kChunk + 4;      // row stride of the A / M / T tiles
constexpr int kChunkThreads = 512;

// Normalised k and q rows in LDS as split-bf16 planes (hi, then lo; hi + lo is the fp32 value
// to ~2^-17): [64 tokens][128 channels] bf16, 256-byte rows whose 16-byte chunks are
// XOR-swizzled by (token & 15), so that a chunk read by 16 consecutive tokens (an MFMA
// operand) touches 16 different bank groups. Byte offset of (token t, channel ch) in a plane:
constexpr int kQKPlane = kChunk * 256;                   // bytes per plane
__device__ __forceinline__ int qk_off(int t, int ch) {
    return t * 256 + ((((ch >> 3) ^ (t & 15))) << 4) + ((ch & 7) << 1);
}
typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef short v4s __attribute__((ext_vector_type(4)));
// Transposing 8-byte LDS read of 16-bit elements (gfx950 ds_read_b64_tr_b16).
__device__ __forceinline__ uint2 lds_tr16(const lds_u8* a) {
    typedef __attribute__((address_space(3))) v4s lds_v4s;
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)a));
}

// The 10 blocks (br, bc) of the 4 x 4 lower block triangle, 16 x 16 each: wave w takes
// i = w, w+4, w+8. The order gives each wave whole 32-column halves of block rows: wave 0
// (1,0) (1,1) (0,0), wave 1 (2,0) (2,1) (2,2), wave 2 (3,0) (3,1), wave 3 (3,2) (3,3), so
// its first two blocks make one M fragment (block row br, k-step bc / 2), and waves 0, 1
// also hold the diagonal block whose right neighbour is zero.
__device__ __forceinline__ void tri_block(int i, int& br, int& bc) {
    br = (0x8f9f9 >> (2 * i)) & 3;                      // 1 2 3 3 1 2 3 3 0 2
    bc = (0x8d580 >> (2 * i)) & 3;                      // 0 0 0 2 1 1 1 3 0 2
}

// 16x16x16 bf16 MFMA operands: A lane l holds A[l%16][4 (l/16) + e], B lane l holds
// B[4 (l/16) + e][l%16], e = 0..3, and the accumulator's lane l holds C[4 (l/16) + r][l%16],
// so an accumulator split to bf16 is the next product's B operand as it stands.
typedef short bf4 __attribute__((ext_vector_type(4)));
struct Split4 { bf4 h, l; };
__device__ __forceinline__ Split4 split4(const v4& x) {
    uint32_t h0, l0, h1, l1;
    split2(x[0], x[1], h0, l0);
    split2(x[2], x[3], h1, l1);
    return Split4{__builtin_bit_cast(bf4, uint2{h0, h1}), __builtin_bit_cast(bf4, uint2{l0, l1})};
}
// c += A B on split operands (hi hi + hi lo + lo hi).
__device__ __forceinline__ v4 mfma16_split(const Split4& a, const Split4& b, v4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a.h, b.h, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a.h, b.l, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a.l, b.h, c, 0, 0, 0);
}
// A operand of the 16 x 16 block at (r0, c0) of an LDS matrix with row stride kTS, times s.
__device__ __forceinline__ Split4 block_a(const float* m, int r0, int c0, int lane, float s) {
    return split4(s * *reinterpret_cast<const v4*>(m + (r0 + (lane & 15)) * kTS + c0 + 4 * (lane >> 4)));
}

// Column block J of T = (I + A)^-1 below the diagonal, by forward substitution on the
// identity's block column: T_kj = -T_kk sum_{m=J}^{k-1} A_km T_mj, k = J+1..3, from the
// diagonal blocks T_kk already in T_s. Each block is chained to the next product in
// registers (its accumulator, split, is the B operand) and stored to T_s when done, at the
// mirrored block position (J, k): T shares its array with A (A's diagonal blocks are
// overwritten by T's in place, its blocks above the diagonal are never written), so T[t][s]
// of block (k, J), J <= k, sits at row 16 J + t % 16, column 16 k + s % 16.
template <int J>
__device__ __forceinline__ void t_column(const float* A_s, float* T_s, int lane) {
    const int li = lane & 15, lg4 = lane >> 4;
    Split4 xs[4];
    {
        v4 tj;                                            // T_JJ as a B operand
#pragma unroll
        for (int e = 0; e < 4; ++e) tj[e] = T_s[(16 * J + 4 * lg4 + e) * kTS + 16 * J + li];
        xs[J] = split4(tj);
    }
#pragma unroll
    for (int k = J + 1; k < 4; ++k) {
        v4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = J; m < k; ++m) acc = mfma16_split(block_a(A_s, 16 * k, 16 * m, lane, -1.0f), xs[m], acc);
        const v4 x = mfma16_split(block_a(T_s, 16 * k, 16 * k, lane, 1.0f), split4(acc), v4{0.f, 0.f, 0.f, 0.f});
        xs[k] = split4(x);
#pragma unroll
        for (int r = 0; r < 4; ++r) T_s[(16 * J + 4 * lg4 + r) * kTS + 16 * k + li] = x[r];
    }
}

// A and M of one v head from the raw products of this wave's triangle blocks (waves 0-3):
// A[t][s] = beta_t exp(G_t - G_s) (k_t . k_s) for s < t into LDS (the inverse's input), and
// M[t][s] = exp(G_t - G_s) (q_t . k_s) for s <= t straight into the chain's M fragments.
// The raw K K^T block (br, bc) holds (t = 16 br + 4 lg4 + r, s = 16 bc + li); the raw Q K^T
// block arrives transposed, (s = 16 bc + 4 lg4 + r, t = 16 br + li), which is the fragment
// layout: entries 4 (bc & 1) + r of lane (li, lg4) of fragment (br, bc / 2). The blocks above
// the diagonal of A are never written (nothing reads them); M's are written as zeros.
// Branch-free; the decay uses the hardware exp (relative error <= 4e-6 down to the fp32
// underflow of exp(G_t - G_s)).
__device__ __forceinline__ void am_head(const v4 (&kk)[3], const v4 (&qk)[3], const float* G, const float* Bt,
                                        float* A_s, uint8_t* Mf, int w, int lane) {
    const int li = lane & 15, lg4 = lane >> 4;
    float mv[3][4];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int i = w + 4 * j;
#pragma unroll
        for (int r = 0; r < 4; ++r) mv[j][r] = 0.0f;
        if (i >= 10) continue;
        int br, bc;
        tri_block(i, br, bc);
        {
            const int t0 = 16 * br + 4 * lg4, s = 16 * bc + li;
            const v4 gt = *reinterpret_cast<const v4*>(G + t0), bt = *reinterpret_cast<const v4*>(Bt + t0);
            const float gs = G[s];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = t0 + r;
                const float e = __expf(fminf(gt[r] - gs, 0.0f));    // used for s < t only
                A_s[t * kTS + s] = s < t ? bt[r] * e * kk[j][r] : 0.0f;
            }
        }
        {
            const int s0 = 16 * bc + 4 * lg4, t = 16 * br + li;
            const v4 gs = *reinterpret_cast<const v4*>(G + s0);
            const float gt = G[t];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __expf(fminf(gt - gs[r], 0.0f));    // used for s <= t only
                mv[j][r] = s0 + r <= t ? e * qk[j][r] : 0.0f;
            }
        }
    }
    // Blocks 0 and 1 of every wave: fragment (br, bc / 2) of the first. Block 2 of waves 0 and
    // 1 (a diagonal block, right neighbour zero). The fragments of block rows 0 and 1 at
    // k-step 1 are zero and not stored: the chain never reads them.
    int br, bc;
    tri_block(w, br, bc);
    float x[8];
    bf8 hi, lo;
#pragma unroll
    for (int r = 0; r < 4; ++r) { x[r] = mv[0][r]; x[4 + r] = mv[1][r]; }
    split8(x, hi, lo);
    store_frag(Mf, br, bc >> 1, 2, lane, hi, lo);
    if (w < 2) {
        tri_block(w + 8, br, bc);
#pragma unroll
        for (int r = 0; r < 4; ++r) { x[r] = mv[2][r]; x[4 + r] = 0.0f; }
        split8(x, hi, lo);
        store_frag(Mf, br, bc >> 1, 2, lane, hi, lo);
    }
}

// Row tile mt, k-step ks of T' = T diag(sc) as a split-bf16 A fragment: lane (li, lg4) holds
// T[16 mt + li][s] sc_s at the tokens s = 32 ks + kperm(lg4, e), zero above the diagonal
// blocks (T in its array shared with A: diagonal blocks in place, the others mirrored, so
// T[t][s] of block (k, J), J <= k, sits at row 16 J + t % 16, column 16 k + s % 16; the reads
// of blocks above the diagonal land in A and are discarded).
__device__ __forceinline__ void t_frag(const float* T_s, const float* sc, int mt, int ks, int li, int lg4, bf8& h,
                                       bf8& l) {
    const int s0 = 32 * ks + 4 * lg4;
    const v4 sc0 = *reinterpret_cast<const v4*>(sc + s0), sc1 = *reinterpret_cast<const v4*>(sc + s0 + 16);
    const float* tr = T_s + (32 * ks + li) * kTS + 16 * mt + 4 * lg4;
    const v4 t0 = *reinterpret_cast<const v4*>(tr), t1 = *reinterpret_cast<const v4*>(tr + 16 * kTS);
    const bool live0 = 2 * ks <= mt, live1 = 2 * ks + 1 <= mt;
    float av[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        av[e] = live0 ? t0[e] * sc0[e] : 0.0f;
        av[e + 4] = live1 ? t1[e] * sc1[e] : 0.0f;
    }
    split8(av, h, l);
}

// Decay scan of one v head over the chunk's tokens (one wave, lane = token): the inclusive
// cumulative log decay G and beta into LDS, the chain's decay factors exp(G_last - G_t) and
// exp(G_t) to the workspace. Rows past the chunk end add nothing (G repeats its last value)
// and have beta = 0.
__device__ __forceinline__ void decay_scan(const PrefillParams& p, const ChunkGeo& g, int h, size_t ch, uint16_t ra,
                                           uint16_t rb, float* G_s, float* B_s, int lane) {
    const Layer& L = p.L;
    const bool ok = lane < g.len;
    float lgt = ok ? log_gate(L, h, bf16_to_f32(ra)) : 0.0f;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const float o = __shfl_up(lgt, off, kWave);
        if (lane >= off) lgt += o;
    }
    G_s[lane] = lgt;
    B_s[lane] = ok ? sigmoid_f(bf16_to_f32(rb)) : 0.0f;
    const float glast = __shfl(lgt, kChunk - 1, kWave);
    float* E = p.ws.G + ch * 2 * kChunk;
    E[lane] = expf(glast - lgt);
    E[kChunk + lane] = expf(lgt);
}

// ---------------------------------------------------------------------------------------
// tri_kernel: grid (window chunks, h_k), 512 threads at most 128 VGPRs (two workgroups per
// CU); workgroup = (chunk, q/k head).
//   1. q rows (waves 0-3) and k rows (waves 4-7): conv and L2 norm into split-bf16 planes.
//   2. Each group of four waves (waves 0-3, waves 4-7) forms the raw K K^T and (Q K^T)^T
//      blocks of the lower block triangle in its registers (both groups the same blocks), and
//      its first wave the decay scan of its first v head.
//   3. Group g takes the mapped v heads g, g + 2, ...: A into its LDS array (the planes' space)
//      and M to its fragments, the diagonal blocks of T = (I + A)^-1 by substitution (the
//      group's first wave), the blocks below them by block forward substitution (three
//      waves), then T' = T diag(beta) as fragments (two per wave).
// At a sequence's first chunk the conv reads the old q/k history from conv_state; the chain,
// which runs after this kernel, writes the new history.
// Every barrier orders LDS only, so no wave waits for its own global stores.
// ---------------------------------------------------------------------------------------
template <int DC, bool SILU>
__global__ void __launch_bounds__(kChunkThreads) __attribute__((amdgpu_waves_per_eu(4))) tri_kernel(const PrefillParams p) {
    __shared__ __align__(16) uint8_t lds[4 * kQKPlane];   // k hi, k lo, q hi, q lo; then A/T of two heads
    __shared__ __align__(16) float G_s[2][kChunk], B_s[2][kChunk];
    uint8_t* Kp = lds;
    uint8_t* Qp = lds + 2 * kQKPlane;

    ChunkGeo g;
    const int c = p.cb + blockIdx.x, lc = blockIdx.x;       // chunk, and its place in the window
    if (!chunk_geo(p, c, g)) return;
    const Layer& L = p.L;
    const int src = blockIdx.y;
    const int nmap = mapped_count(L, src);
    if (nmap == 0) return;                                     // no v head reads this q/k head
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int grp = w >> 2, gw = w & 3;
    const int li = lane & 15, lg4 = lane >> 4, c2 = 2 * lane;
    const int tb = kConvTok * (w & 3), nt = min(max(g.len - tb, 0), kConvTok);

    // The gate inputs of the group's first v head, loaded first (lane = token, clamped rows).
    uint16_t ra = 0, rb = 0;
    if (gw == 0) {
        const size_t ab = (size_t)(g.t0 + min(lane, g.len - 1)) * L.h_v + mapped_head(L, src, min(grp, nmap - 1));
        ra = p.a[ab];
        rb = p.b[ab];
    }

    // q rows (waves 0-3) and k rows (waves 4-7), 16 tokens per wave: lane l carries channels
    // 2l, 2l+1, so every x access of a wave is a 256-byte row segment and each row's norm is
    // one wave sum. Rows past the chunk end are zero.
    const bool isk = w >= 4;
    {
        ConvIn<DC> in;
        conv_load<DC>(p, g, g.lo, isk ? k_channel(L, src, c2) : q_channel(L, src, c2), tb, nt, in);
        float y0[kConvTok], y1[kConvTok];
        conv_run<DC, SILU>(in, y0, y1);
        // The 16 row sums in one reduce-scatter: lane l holds the sum of row l >> 2, so one
        // rsqrt gives every row's factor, which each row then reads from lane 4 t.
        float ss[kConvTok];
#pragma unroll
        for (int t = 0; t < kConvTok; ++t) ss[t] = fmaf(y0[t], y0[t], y1[t] * y1[t]);
        const float scale = isk ? 1.0f : L.q_scale;
        const float inv_l = scale * rsqrtf(sum16_scatter(ss, lane) + L.l2_eps);
        uint8_t* dst = isk ? Kp : Qp;
#pragma unroll
        for (int t = 0; t < kConvTok; ++t) {
            const float inv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv_l), 4 * t));
            uint32_t hi = 0, lo = 0;
            if (t < nt) split2(y0[t] * inv, y1[t] * inv, hi, lo);
            const int o = qk_off(tb + t, c2);
            *reinterpret_cast<uint32_t*>(dst + o) = hi;
            *reinterpret_cast<uint32_t*>(dst + kQKPlane + o) = lo;
        }
    }
    lds_barrier();

    // The chain's key planes (row t: 128 bf16 with each 32-channel block in kperm order, its
    // 16-byte chunks swizzled by kswz(t); hi plane, then lo) and Q fragments (rows t, k = channel in kperm
    // order), from the swizzled planes: every thread moves 4 of the 16-byte key chunks and 4 Q
    // fragment chunks. Key chunk j of a row holds channels 32 (j / 4) + 4 (j % 4) .. +3, then
    // the 4 channels 16 later.
    {
        uint8_t* kg = p.ws.Kp + ((size_t)lc * L.h_k + src) * kKSlot;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = tid + u * kChunkThreads, pl = e >> 10, t = (e >> 4) & 63, cc = e & 15;
            const int c0 = 32 * (cc >> 2) + 4 * (cc & 3);
            const uint2 a = *reinterpret_cast<const uint2*>(Kp + pl * kQKPlane + qk_off(t, c0));
            const uint2 b = *reinterpret_cast<const uint2*>(Kp + pl * kQKPlane + qk_off(t, c0 + 16));
            *reinterpret_cast<u4x*>(kg + pl * kKPlane + t * kPRow + 16 * (cc ^ kswz(t))) = u4x{a.x, a.y, b.x, b.y};
        }
        uint16_t* Qg = p.ws.Qf + ((size_t)lc * L.h_k + src) * kFragW;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int e = tid + u * kChunkThreads, ln = e & (kWave - 1), f = e / kWave, m = f >> 2, ks = f & 3;
            const int row = 16 * m + (ln & 15), k0 = 32 * ks + 4 * (ln >> 4);      // kperm halves
            const int oa = qk_off(row, k0), ob = qk_off(row, k0 + 16);
#pragma unroll
            for (int pl = 0; pl < 2; ++pl) {
                const uint2 a = *reinterpret_cast<const uint2*>(Qp + pl * kQKPlane + oa);
                const uint2 b = *reinterpret_cast<const uint2*>(Qp + pl * kQKPlane + ob);
                *reinterpret_cast<u4x*>(Qg + frag_at(m, ks, 4, pl, ln)) = u4x{a.x, a.y, b.x, b.y};
            }
        }
    }

    // Raw K K^T and (Q K^T)^T of this wave's triangle blocks (16x16x32 split-bf16 MFMA,
    // operands straight from the planes: lane (li, lg4) supplies channels 32 ks + 8 lg4 .. +7
    // of token row li for both operands). The A and B register layouts are mirror images, so
    // swapping the operands of Q K^T gives its transpose.
    v4 kk[3], qk[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        kk[j] = v4{0.f, 0.f, 0.f, 0.f};
        qk[j] = kk[j];
        const int i = gw + 4 * j;
        if (i >= 10) continue;
        int br, bc;
        tri_block(i, br, bc);
        const int arow = 16 * br + li, brow = 16 * bc + li;
#pragma unroll
        for (int ks = 0; ks < kD / 32; ++ks) {
            const int ch = 32 * ks + 8 * lg4, oa = qk_off(arow, ch), ob = qk_off(brow, ch);
            const bf8 akh = *reinterpret_cast<const bf8*>(Kp + oa);
            const bf8 akl = *reinterpret_cast<const bf8*>(Kp + kQKPlane + oa);
            const bf8 aqh = *reinterpret_cast<const bf8*>(Qp + oa);
            const bf8 aql = *reinterpret_cast<const bf8*>(Qp + kQKPlane + oa);
            const bf8 bkh = *reinterpret_cast<const bf8*>(Kp + ob);
            const bf8 bkl = *reinterpret_cast<const bf8*>(Kp + kQKPlane + ob);
            kk[j] = mfma_bf16(akh, bkh, kk[j]);
            qk[j] = mfma_bf16(bkh, aqh, qk[j]);
            kk[j] = mfma_bf16(akh, bkl, kk[j]);
            qk[j] = mfma_bf16(bkl, aqh, qk[j]);
            kk[j] = mfma_bf16(akl, bkh, kk[j]);
            qk[j] = mfma_bf16(bkh, aql, qk[j]);
        }
    }
    if (gw == 0 && grp < nmap) {
        const int h = mapped_head(L, src, grp);
        decay_scan(p, g, h, (size_t)lc * L.h_v + h, ra, rb, G_s[grp], B_s[grp], lane);
    }
    lds_barrier();                                          // the planes' space becomes A/T

    float* A_s = reinterpret_cast<float*>(lds) + grp * (kChunk * kTS);
    float* T_s = A_s;                  // T over A: diagonal blocks in place, the others mirrored
    for (int it = 0; 2 * it < nmap; ++it) {
        const int m = 2 * it + grp;
        const bool live = m < nmap;
        const int h = mapped_head(L, src, min(m, nmap - 1));
        const size_t ch = (size_t)lc * L.h_v + h;
        if (it > 0) {                                       // the next head's decay scan
            if (live && gw == 0) {
                const size_t ab = (size_t)(g.t0 + min(lane, g.len - 1)) * L.h_v + h;
                decay_scan(p, g, h, ch, p.a[ab], p.b[ab], G_s[grp], B_s[grp], lane);
            }
            lds_barrier();
        }
        if (live) am_head(kk, qk, G_s[grp], B_s[grp], A_s, p.ws.Mf + ch * kFragMBytes, gw, lane);
        lds_barrier();
        // The group's first wave inverts the four unit lower-triangular diagonal blocks of
        // I + A (lane = 16 b + column cc).
        if (live && gw == 0) {
            const int b = lane >> 4, cc = lane & 15;
            const float* Ab = A_s + (16 * b) * kTS + 16 * b;
            float x[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float acc = r == cc ? 1.0f : 0.0f;
#pragma unroll
                for (int q = 0; q < r; ++q) acc = fmaf(-Ab[r * kTS + q], x[q], acc);
                x[r] = acc;
                if ((r & 3) == 3) __builtin_amdgcn_sched_barrier(0);   // loads hoisted 4 rows ahead at most
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) T_s[(16 * b + r) * kTS + 16 * b + cc] = x[r];
        }
        lds_barrier();
        // T below the diagonal blocks: wave j (0..2) of the group runs column block j.
        if (live) {
            if (gw == 0) t_column<0>(A_s, T_s, lane);
            else if (gw == 1) t_column<1>(A_s, T_s, lane);
            else if (gw == 2) t_column<2>(A_s, T_s, lane);
        }
        lds_barrier();
        // T' = T diag(beta) as the chain's A fragments (4 row tiles x 2 k-steps): wave gw
        // writes fragments gw and gw + 4, (row tile f / 2, k-step f % 2), except the zero ones
        // above the diagonal blocks (row tiles 0 and 1 at k-step 1), which the chain never reads.
        if (live) {
            uint8_t* Tf = p.ws.Tf + ch * kTriFragBytes;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int f = gw + 4 * u, mt = f >> 1, ks = f & 1;
                if (ks == 1 && mt < 2) continue;
                bf8 hi, lo;
                t_frag(T_s, B_s[grp], mt, ks, li, lg4, hi, lo);
                store_tri_frag(Tf, mt, ks, lane, hi, lo);
            }
        }
        if (2 * (it + 1) < nmap) lds_barrier();             // T and beta are read until here
    }
}

// ---------------------------------------------------------------------------------------
// chain: one workgroup per (v head, 16-column state strip, group), 8 waves
// ---------------------------------------------------------------------------------------
// Columns of the state are independent, so a head's chain splits into 8 strips of 16
// columns, and each strip's workgroup walks a run of the window's chunks in order: all of them
// (one group, when the h_v * 8 strips fill the CUs) or a share ending at a sequence start. At
// a sequence boundary the state waves store the finished state and continue with the next
// sequence's (loaded a chunk ahead); the other roles only follow each chunk's record. For
// chunk c_k, with S_k the strip at its start,
//     W_k     = K_k S_k                                            (64 x 16)
//     D_k     = T'_k (V_k - diag(Gam_k) W_k)
//     S_{k+1} = gam_k S_k + K_k^T Dg_k,  Dg_k = diag(E_k) D_k,  gam_k = Gam_k[63]
//     O_k     = diag(Gam_k) Q_k S_k + M_k D_k
// run in two phases per chunk, alpha_k and beta_k, each ended by a workgroup barrier:
//   alpha_k  the state waves (0, 1) each hold 64 rows of S in MFMA accumulators (row tile mt
//            of wave i: S[64 i + 16 mt + 4 lg4 + r][column li]); for k > 0 they finish
//            S_k = gam S_{k-1} + K_{k-1}^T Dg_{k-1} on their rows (K^T read in beta_{k-1}),
//            hand S_k over split and form their half of W_k (the sum over their 64 channels,
//            K read as the products need it);
//   beta_k   the D wave (4) and the feed wave (5) add the halves and form D_k, row tiles 0, 1
//            and 2, 3, handing over D_k (fp32) for the outputs and Dg_k (split) with gam_k
//            for the state waves.
// Products take their k index in accumulator row order (kperm), so an accumulator tile pair,
// split to bf16 hi/lo, is the next product's B operand as it stands. The D and feed waves keep
// their T' fragments in registers (loaded a chunk ahead) and read chunk c_k's V and decay
// factors from the value slot in alpha_k, while the state waves work.
// The output waves (2, 3, 6, 7; row tile r) form diag(Gam) Q S in beta_k and add M D in
// alpha_{k+1}, with Q and M loaded from the workspace two chunks ahead (Gam read from the value
// slot in alpha_k); they build row tile r of chunk c_{k+1}'s V (the conv of the strip's v
// channels), half in alpha_k and half in beta_k for r < 2, all in beta_k for r >= 2. The feed
// wave (5) copies chunk c_{k+1}'s key planes into key slot (k+1) mod 3 with direct
// global-to-LDS loads issued in alpha_k (the slot last held chunk c_{k-2}, read until
// beta_{k-2}), and writes the new rolling conv history of the workgroup's channels; the D
// wave writes chunk c_{k+1}'s decay factors into the value slot in beta_k from registers
// loaded in alpha_k.
// A last alpha_n finishes S_n (state waves) and O_{n-1} (output waves).
// Waves w and w + 4 share a SIMD: the state waves' partners (the D wave, the feed wave) only
// read and copy in alpha, where the state waves work.
constexpr int kStrip = 16;                              // state columns per chain workgroup
constexpr int kStrips = kD / kStrip;                    // 8
constexpr int kChainWaves = 8;
constexpr int kPlane = kWave * 16;                      // bytes of one fragment plane
constexpr int kKSlots = 3;                              // key slots in a ring
constexpr int kVSlot = 4 * kPlane + 2 * kChunk * 4;     // V (4 row tiles, accumulator layout), E, Gam
constexpr int kHandS = 8 * kPlane;                      // S: 4 k-steps x 2 planes
constexpr int kHandBytes = kHandS + 4 * kPlane;         // + D: 4 row tiles in fp32
constexpr int kWBytes = 2 * 4 * kPlane;                 // the two halves of W: 4 row tiles in fp32 each
constexpr int kDgBytes = 4 * kPlane + 16;               // Dg: 2 k-steps x 2 planes, then gam
constexpr int kOffK = 0, kOffV = kOffK + kKSlots * kKSlot, kOffH = kOffV + kVSlot;
constexpr int kXRows = 24;                              // an output wave's x staging: rows 16 r - 3 .. 16 r + 20
constexpr int kXBytes = 4 * kXRows * kStrip * 2;        // 16 bf16 channels per row, 4 output waves
constexpr int kOffW = kOffH + kHandBytes, kOffG = kOffW + kWBytes, kOffX = kOffG + kDgBytes;
constexpr int kMaxWindow = 80;                          // chunks of a window at most
constexpr int kOffR = kOffX + kXBytes;                  // the run's chunk records
constexpr int kOffV1 = kOffR + kMaxWindow * 16;         // V of odd chunks (even ones at kOffV)
constexpr int kChainLds = kOffV1 + 4 * kPlane;          // 135,952 bytes
// V of chunk c_k (4 row tiles, accumulator layout): written in alpha_{k-1}, read in alpha_k.
__device__ __forceinline__ int v_buf(int k) { return (k & 1) ? kOffV1 : kOffV; }

typedef __attribute__((address_space(3))) bf8 lds_bf8;
typedef __attribute__((address_space(3))) v4 lds_v4;

// This lane's address in an LDS area at byte offset off (which includes the lane's own part),
// made opaque to the compiler: reads and writes at base + (a constant below 64 KiB) then use
// the instruction's immediate offset, where the folded address of an area above 64 KiB
// would cost an add per access.
__device__ __forceinline__ lds_u8* lane_at(uint8_t* lds, int off) {
    lds_u8* b = (lds_u8*)lds + off;
    __asm__ volatile("" : "+v"(b));
    return b;
}

// B operand of one 32-wide k-step from two stacked accumulator tiles (kperm order), split.
__device__ __forceinline__ void split_tiles(const v4& a, const v4& b, bf8& hi, bf8& lo) {
    uint32_t h0, h1, h2, h3, l0, l1, l2, l3;
    split2(a[0], a[1], h0, l0);
    split2(a[2], a[3], h1, l1);
    split2(b[0], b[1], h2, l2);
    split2(b[2], b[3], h3, l3);
    hi = __builtin_bit_cast(bf8, u4x{h0, h1, h2, h3});
    lo = __builtin_bit_cast(bf8, u4x{l0, l1, l2, l3});
}

// Key slots hold each 32-channel block of a key row in kperm order: channels 4 a .. 4 a + 3,
// then 16 + 4 a .. 16 + 4 a + 3, for a = 0..3, i.e. channel 32 b + 16 h + 4 a + e sits at
// position 32 b + 8 a + 4 h + e.
// K fragment (token tile mt, channel k-step ks) of a key slot: A operand of K S. Lane
// (li, lg4) reads row 16 mt + li, channels 32 ks + 4 lg4 .. +3 and 32 ks + 16 + 4 lg4 .. +3:
// the 16 bytes of chunk 4 ks + lg4, stored at chunk (4 ks + lg4) ^ kswz(li) of the row.
__device__ __forceinline__ int k_lane(int li, int lg4, int ks) {
    return li * kPRow + 16 * ((4 * ks + lg4) ^ kswz(li));
}
// kb: the slot plus k_lane(li, lg4, ks).
__device__ __forceinline__ void k_frag(const lds_u8* kb, int mt, bf8& hi, bf8& lo) {
    const int o = mt * 16 * kPRow;
    hi = *(const lds_bf8*)(kb + o);
    lo = *(const lds_bf8*)(kb + kKPlane + o);
}

// K^T fragment (channel tile m, token k-step ks) of a key slot: A operand of K^T Dg, by
// transposing reads (ds_read_b64_tr_b16: within each 16-lane group, lane j receives element
// j & 3 of the 8-byte reads of lanes (j >> 2) + 4 e, e = 0..3). Lane i of lane group g reads
// channels 16 m + 4 (i & 3) .. +3 of token t = 32 ks + 4 g + (i >> 2) (then of the token 16
// later), so it receives channel 16 m + i at tokens 32 ks + 4 g + e (+ 16): entries e (4 + e)
// of its kperm fragment chunk. Those 4 channels are half m & 1 of chunk 4 (m / 2) + (i & 3),
// stored at chunk (4 (m / 2) + (i & 3)) ^ kswz(t) of the row (kswz(t) depends on i and g only).
__device__ __forceinline__ int kt_lane(int i, int g, int mh) {
    const int t = 4 * g + (i >> 2);
    return t * kPRow + 16 * ((4 * mh + (i & 3)) ^ kswz(t));
}
// tb: the slot plus kt_lane(i, g, m / 2); half = m & 1.
__device__ __forceinline__ void kt_frag(const lds_u8* tb, int half, int ks, bf8& hi, bf8& lo) {
    const int o = ks * 32 * kPRow + half * 8;
    const uint2 a = lds_tr16(tb + o), b = lds_tr16(tb + o + 16 * kPRow);
    const uint2 c = lds_tr16(tb + kKPlane + o), d = lds_tr16(tb + kKPlane + o + 16 * kPRow);
    hi = __builtin_bit_cast(bf8, u4x{a.x, a.y, b.x, b.y});
    lo = __builtin_bit_cast(bf8, u4x{c.x, c.y, d.x, d.y});
}

// acc[j] += A_j B for four row tiles, split products; the products go tile by tile within
// each of hi hi, hi lo, lo hi, so consecutive MFMAs never share an accumulator.
__device__ __forceinline__ void mfma4_split(const bf8 (&a)[4][2], const bf8& bh, const bf8& bl, v4* acc) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = mfma_bf16(a[j][0], bh, acc[j]);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = mfma_bf16(a[j][0], bl, acc[j]);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = mfma_bf16(a[j][1], bh, acc[j]);
}

// Interleaves two independent four-tile split products, MFMA by MFMA, so that the pipe
// always has an accumulator that is not waiting for its previous product.
__device__ __forceinline__ void mfma4x2_split(const bf8 (&a)[4][2], const bf8& ah, const bf8& al, v4* acc_a,
                                              const bf8 (&b)[4][2], const bf8& bh, const bf8& bl, v4* acc_b) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        acc_a[j] = mfma_bf16(a[j][0], ah, acc_a[j]);
        acc_b[j] = mfma_bf16(b[j][0], bh, acc_b[j]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        acc_a[j] = mfma_bf16(a[j][0], al, acc_a[j]);
        acc_b[j] = mfma_bf16(b[j][0], bl, acc_b[j]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        acc_a[j] = mfma_bf16(a[j][1], ah, acc_a[j]);
        acc_b[j] = mfma_bf16(b[j][1], bh, acc_b[j]);
    }
}

// acc[t] += A_t B for row tiles t = 0, 1 only, split products.
__device__ __forceinline__ void mfma2_split(const bf8 (&a)[4][2], const bf8& bh, const bf8& bl, v4* acc) {
#pragma unroll
    for (int t = 0; t < 2; ++t) acc[t] = mfma_bf16(a[t][0], bh, acc[t]);
#pragma unroll
    for (int t = 0; t < 2; ++t) acc[t] = mfma_bf16(a[t][0], bl, acc[t]);
#pragma unroll
    for (int t = 0; t < 2; ++t) acc[t] = mfma_bf16(a[t][1], bh, acc[t]);
}


// A chain workgroup's run: the window's chunks a .. a + n - 1, consecutive chunks of one or more
// consecutive sequences; wk = a - cb, the first one's place in the window; lo, hi: the bounds
// of the only sequence when n_seq == 1.
struct ChainRun { int a, n, wk, lo, hi; };
// Chunk c of a run: its sequence s, first token t0 and the sequence's bounds [lo, hi).
struct RunChunk {
    int s, t0, lo, hi;
    __device__ int len() const { return min(kChunk, hi - t0); }
    __device__ bool starts() const { return t0 == lo; }               // the sequence's first chunk
    __device__ bool ends() const { return t0 + kChunk >= hi; }        // its last
};
// Record k of the run, from the copy in LDS (kOffR) that every wave reads from before its
// first phase.
__device__ __forceinline__ RunChunk run_chunk(const uint8_t* lds, int k) {
    const u4x v = *(const __attribute__((address_space(3))) u4x*)((const lds_u8*)lds + kOffR + 16 * k);
    RunChunk r;
    r.s = (int)v.x;
    r.t0 = (int)v.y;
    r.lo = (int)v.z;
    r.hi = (int)v.w;
    return r;
}

// State role (waves 0 and 1, half = wave): rows 64 half .. 64 half + 63 of the strip, S[mt]
// the accumulator of row tile mt (rows 64 half + 16 mt + 4 lg4 + r, column li). The state
// is stored column by column ([d_v][d_k]), so the 4 rows of a lane are a float4. It is loaded
// at the run's first chunk and at each sequence start (the next sequence's state is loaded a
// chunk ahead), and stored after each sequence's last chunk and after the run's last.
__device__ __forceinline__ void chain_state_role(const PrefillParams& p, uint8_t* lds, int lane, const ChainRun& run,
                                                 int half, int h, int j0) {
    const int li = lane & 15, lg4 = lane >> 4, n = run.n;
    auto st_of = [&](int s) {
        return p.state + ((size_t)s * p.L.h_v + h) * kD * kD + (size_t)(j0 + li) * kD + 64 * half + 4 * lg4;
    };
    auto st_load = [&](int s, v4 (&X)[4]) {
        const float* st = st_of(s);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) X[mt] = *reinterpret_cast<const v4*>(st + 16 * mt);
    };
    auto st_store = [&](int s, const v4 (&X)[4]) {
        float* st = st_of(s);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) *reinterpret_cast<v4*>(st + 16 * mt) = X[mt];
    };
    // Chunks c_k, c_{k+1}, c_{k+2} (clamped to the run's last): each record is loaded two chunks
    // before the one that decides on it.
    RunChunk rc = run_chunk(lds, 0), rn = run_chunk(lds, min(1, n - 1)),
             rn2 = run_chunk(lds, min(2, n - 1));
    v4 S[4], Sn[4];
    st_load(rc.s, S);
    if (n > 1 && rn.starts()) st_load(rn.s, Sn);
    // Lane offsets in a key slot: K of k-steps 2 half + a, K^T of channel tiles 4 half + 2 a + j.
    int koff[2], toff[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
        koff[a] = k_lane(li, lg4, 2 * half + a);
        toff[a] = kt_lane(li, lg4, 2 * half + a);
    }
    lds_u8* hb = lane_at(lds, kOffH + 4 * half * kPlane + lane * 16);     // S k-steps 2 half, 2 half + 1
    lds_u8* wb = lane_at(lds, kOffW + 4 * half * kPlane + lane * 16);
    const lds_u8* gb = lane_at(lds, kOffG + lane * 16);
    // K: channel k-step 2 half + a, token tile mt; K^T: token k-step ks, channel tile 4 half + j.
    bf8 KF[2][4][2], KT[2][4][2];
    auto load_k = [&](int q) {
        const lds_u8* slot = (lds_u8*)lds + kOffK + q * kKSlot;
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) k_frag(slot + koff[a], mt, KF[a][mt][0], KF[a][mt][1]);
    };
    auto load_kt = [&](int q) {
        const lds_u8* slot = (lds_u8*)lds + kOffK + q * kKSlot;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int j = 0; j < 4; ++j) kt_frag(slot + toff[j >> 1], j & 1, ks, KT[ks][j][0], KT[ks][j][1]);
    };
    // S_k handed over split (the outputs' B operand) and this wave's half of W_k = K_k S_k.
    auto hand_and_w = [&]() {
        bf8 sh[2], sl[2];
        v4 W[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) W[mt] = v4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            split_tiles(S[2 * a], S[2 * a + 1], sh[a], sl[a]);
            *(lds_bf8*)(hb + (2 * a) * kPlane) = sh[a];
            *(lds_bf8*)(hb + (2 * a + 1) * kPlane) = sl[a];
            mfma4_split(KF[a], sh[a], sl[a], W);
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) *(lds_v4*)(wb + mt * kPlane) = W[mt];
    };

    lds_barrier();                                          // alpha_0: chunk c_0's keys in slot 0
    load_k(0);
    hand_and_w();
    int q = 0;                                              // key slot of chunk c_k: k mod 3
    for (int k = 0; k < n; ++k) {
        lds_barrier();                                      // beta_k
        const int q1 = q == kKSlots - 1 ? 0 : q + 1;
        // K^T of chunk c_k, for S_{k+1}, read in beta after a pause of about 768 cycles: issued
        // at once, its 32 reads would queue the D wave's W reads behind them; not issued
        // until alpha, their latency would open the next phase.
        __builtin_amdgcn_s_sleep(12);
        load_kt(q);
        lds_barrier();                                      // alpha_{k+1}: Dg_k, gam_k handed over
        bf8 dh[2], dl[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            dh[ks] = *(const lds_bf8*)(gb + (2 * ks) * kPlane);
            dl[ks] = *(const lds_bf8*)(gb + (2 * ks + 1) * kPlane);
        }
        // K of chunk c_{k+1} (in its slot since the end of beta_k) read now, behind Dg, so that
        // its latency passes under the S update.
        __asm__ volatile("" ::: "memory");
        load_k(q1);
        const float gam = *(const __attribute__((address_space(3))) float*)((lds_u8*)lds + kOffG + 4 * kPlane);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) S[mt] *= gam;
        // Row tiles 0, 1 first, so that their split and the first k-step of W need not wait
        // for the last products of tiles 2, 3.
#pragma unroll
        for (int pr = 0; pr < 2; ++pr)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int u = 0; u < 3; ++u)
#pragma unroll
                    for (int j = 2 * pr; j < 2 * pr + 2; ++j)
                        S[j] = mfma_bf16(KT[ks][j][u == 2], u == 1 ? dl[ks] : dh[ks], S[j]);
        if (k + 1 < n) {
            if (rn.starts()) {                              // chunk c_k ended its sequence
                st_store(rc.s, S);
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) S[mt] = Sn[mt];
            }
            rc = rn;
            rn = rn2;
            if (k + 2 < n && rn.starts()) st_load(rn.s, Sn);
            rn2 = run_chunk(lds, min(k + 3, n - 1));
            hand_and_w();
        }
        q = q1;
    }
    st_store(rc.s, S);
}

// The strip's v columns, built by the output waves: wave r builds row tile r of V. x rows
// 16 r - 3 + 8 i + (l >> 3), i = 0..2, of a chunk (relative to its first token) for the strip's
// 16 v channels, one channel pair per lane: lane l loads pair l & 7 as one word. Rows before the
// sequence start come from the old conv history, rows past its end repeat its last token
// (their V rows are zeroed).
// Every load is issued on every call (a row before the sequence start takes its history word
// in stage_conv), so each call issues the same memory operations and later waits can count them.
struct XStage {
    uint32_t w[3];
    uint32_t h0, h1;      // the history pair of row 0 and whether row 0 lies before the sequence
    bool hist;
};
template <int DC>
__device__ __forceinline__ void stage_load(const PrefillParams& p, const RunChunk& rc, int h, int strip, int r,
                                           int lane, XStage& xs) {
    const Layer& L = p.L;
    const int ch = v_channel(L, h, strip * kStrip + 2 * (lane & 7));
    const int pos0 = rc.t0 - rc.lo + 16 * r - 3, last = rc.hi - rc.lo - 1;
    const uint16_t* hist = p.conv_state + ((size_t)rc.s * L.C + ch) * (DC - 1) + (DC - 1);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int pos = pos0 + 8 * i + (lane >> 3);        // >= 0 for i > 0
        xs.w[i] = *reinterpret_cast<const uint32_t*>(p.x + (size_t)(rc.lo + max(min(pos, last), 0)) * L.C + ch);
    }
    const int pos = pos0 + (lane >> 3);
    const int hp = min(max(pos, -(DC - 1)), -1);            // rows before -(DC-1) feed no output
    xs.h0 = hist[hp];
    xs.h1 = hist[hp + (DC - 1)];
    xs.hist = pos < 0;
}
// The conv of the staged rows into row tile r of the value slot, in the D wave's accumulator
// layout: lane (li, lg4) holds V[16 r + 4 lg4 + e][channel li], e = 0..3, zero for rows at or
// past len. The rows pass through the wave's own LDS staging area (row 16 r - 3 + i at 32 i
// bytes). Same accumulation order as the fused kernels' conv.
// PART 0 stages the rows and forms entries 0, 1; PART 1 forms entries 2, 3 from the staged
// rows (the same wave, later); PART -1 does both.
template <int DC, bool SILU, int PART = -1>
__device__ __forceinline__ void stage_conv(uint8_t* lds, const XStage& xs, int r, int lane, const float (&w)[DC],
                                           int len, int vbuf) {
    typedef __attribute__((address_space(3))) uint32_t lds_u32;
    typedef __attribute__((address_space(3))) uint16_t lds_u16;
    typedef float f2 __attribute__((ext_vector_type(2)));
    lds_u8* xst = (lds_u8*)lds + kOffX + r * kXRows * 32;
    // The words go in as 32-bit and come back as 16-bit values: the fences keep the compiler
    // from reordering the two (the wave's own LDS accesses then complete in program order).
    __asm__ volatile("" ::: "memory");
    if constexpr (PART != 1) {
#pragma unroll
        for (int i = 0; i < 3; ++i)
            *(lds_u32*)(xst + (8 * i + (lane >> 3)) * 32 + 4 * (lane & 7)) =
                i == 0 && xs.hist ? xs.h0 | (xs.h1 << 16) : xs.w[i];
        __asm__ volatile("" ::: "memory");
    }
    constexpr int e0 = PART == 1 ? 2 : 0, ne = PART == -1 ? 4 : 2;
    const int li = lane & 15, lg4 = lane >> 4, t0 = 16 * r + 4 * lg4;
    float xv[ne + DC - 1];
#pragma unroll
    for (int j = 0; j < ne + DC - 1; ++j)
        xv[j] = __uint_as_float((uint32_t) * (const lds_u16*)(xst + (4 * lg4 - (DC - 1) + e0 + j + 3) * 32 + 2 * li)
                                << 16);
    float V[ne];
#pragma unroll
    for (int e = 0; e < ne; ++e) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < DC; ++i) acc = fmaf(xv[e + i], w[i], acc);
        if constexpr (SILU) acc = acc * sigmoid_f(acc);
        V[e] = t0 + e0 + e < len ? acc : 0.0f;
    }
    lds_u8* vd = (lds_u8*)lds + vbuf + r * kPlane + lane * 16;
    if constexpr (PART == -1) *(lds_v4*)vd = v4{V[0], V[1], V[2], V[3]};
    else *(__attribute__((address_space(3))) f2*)(vd + 4 * e0) = f2{V[0], V[1]};
    __asm__ volatile("" ::: "memory");
}

// D = T' X, X = V - diag(Gam) (W_0 + W_1), from the state waves' halves of W, with V, the decay
// factors and T' read in the preceding alpha; row tiles 0, 1 (T' (0, 0), (1, 0), tokens 0-31)
// by the D wave, row tiles 2, 3 (T' (2, 0), (3, 0), (2, 1), (3, 1)) by the feed wave, each
// handing over its tiles of D (fp32, for the outputs) and its k-step of Dg = diag(E) D (split,
// for the state waves).
// X row tiles mt .. mt + NT - 1 of one chunk.
template <int NT>
__device__ __forceinline__ void d_x(const lds_u8* wb, const v4* V, const v4* Gm, int mt0, v4* X) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int mt = mt0 + t;
        const v4 w0 = *(const lds_v4*)(wb + mt * kPlane), w1 = *(const lds_v4*)(wb + (4 + mt) * kPlane);
#pragma unroll
        for (int e = 0; e < 4; ++e) X[t][e] = fmaf(-Gm[t][e], w0[e] + w1[e], V[t][e]);
    }
}
// Dg k-step ks (row tiles 2 ks, 2 ks + 1) split, and the two D row tiles in fp32.
__device__ __forceinline__ void d_hand(uint8_t* lds, int lane, int ks, const v4* E, const v4* D) {
    bf8 dh, dl;
    split_tiles(E[0] * D[0], E[1] * D[1], dh, dl);
    lds_u8* gb = (lds_u8*)lds + kOffG + lane * 16;
    *(lds_bf8*)(gb + (2 * ks) * kPlane) = dh;
    *(lds_bf8*)(gb + (2 * ks + 1) * kPlane) = dl;
    lds_u8* hb = (lds_u8*)lds + kOffH + kHandS + lane * 16;
    *(lds_v4*)(hb + (2 * ks) * kPlane) = D[0];
    *(lds_v4*)(hb + (2 * ks + 1) * kPlane) = D[1];
}

// D role (wave 4): row tiles 0 and 1 of D (its T' fragments (0, 0), (1, 0) loaded into
// registers a chunk ahead, in one of two sets), and gam. In alpha_k it also loads chunk
// c_{k+1}'s decay factors and writes them (E, then Gam) into the value slot in beta_k, once the
// feed wave has read chunk c_k's.
struct DT {
    u4x f[4];             // T' (0, 0) hi, lo, (1, 0) hi, lo
};
__device__ __forceinline__ void chain_d_role(const PrefillParams& p, uint8_t* lds, int lane, const ChainRun& run,
                                             int h) {
    const int lg4 = lane >> 4, n = run.n;
    auto chh = [&](int k) { return (size_t)(run.wk + min(k, n - 1)) * p.L.h_v + h; };   // clamped
    auto tload = [&](int k, DT& t) {
        const uint8_t* tsrc = p.ws.Tf + chh(k) * kTriFragBytes;
#pragma unroll
        for (int i = 0; i < 4; ++i) t.f[i] = load_tri_frag(tsrc, i >> 1, 0, i & 1, lane);
    };
    v4 eg;
    auto eload = [&](int k) { eg = *reinterpret_cast<const v4*>(p.ws.G + chh(k) * 2 * kChunk + 4 * (lane & 31)); };
    auto eput = [&]() {
        if (lane < 32) *(lds_v4*)((lds_u8*)lds + kOffV + 4 * kPlane + lane * 16) = eg;
    };
    eload(0);
    eput();
    DT d0, d1;
    tload(0, d0);
    const lds_u8* vb0 = lane_at(lds, kOffV + lane * 16);
    const lds_u8* vb1 = lane_at(lds, kOffV1 + lane * 16);
    const lds_u8* eb = lane_at(lds, kOffV + 4 * kPlane + 16 * lg4);
    const lds_u8* wb = lane_at(lds, kOffW + lane * 16);
    // cur: chunk c_k's fragments; oth: reloaded with c_{k+1}'s (it held c_{k-1}'s).
    auto step = [&](int k, const DT& cur, DT& oth) {
        lds_barrier();                                      // alpha_k: chunk c_k in the value slot
        tload(k + 1, oth);
        eload(k + 1);
        const lds_u8* vb = (k & 1) ? vb1 : vb0;
        v4 V[2], E[2], Gm[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            V[mt] = *(const lds_v4*)(vb + mt * kPlane);
            E[mt] = *(const lds_v4*)(eb + mt * 64);
            Gm[mt] = *(const lds_v4*)(eb + 4 * kChunk + mt * 64);
        }
        const float gam = *(const __attribute__((address_space(3))) float*)((lds_u8*)lds + kOffV + 4 * kPlane +
                                                                            4 * kChunk + 4 * (kChunk - 1));
        lds_barrier();                                      // beta_k: both halves of W_k handed over
        bf8 F0[4][2];                                       // T' (mt, 0), mt = 0, 1
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int pl = 0; pl < 2; ++pl) F0[mt][pl] = __builtin_bit_cast(bf8, cur.f[2 * mt + pl]);
        v4 X[2];
        d_x<2>(wb, V, Gm, 0, X);
        bf8 xh, xl;
        split_tiles(X[0], X[1], xh, xl);
        v4 D[2] = {v4{0.f, 0.f, 0.f, 0.f}, v4{0.f, 0.f, 0.f, 0.f}};
        mfma2_split(F0, xh, xl, D);                         // tokens 0-31
        d_hand(lds, lane, 0, E, D);
        if (lane == 0) *(__attribute__((address_space(3))) float*)((lds_u8*)lds + kOffG + 4 * kPlane) = gam;
        eput();                                             // chunk c_{k+1}'s (clamped: harmless at the end)
    };
    for (int k = 0; k < n; k += 2) {
        step(k, d0, d1);
        if (k + 1 < n) step(k + 1, d1, d0);
    }
    lds_barrier();                                          // alpha_n
}

// Output role (waves 2, 3, 6, 7; row tile r): rows 16 r .. 16 r + 15 of every chunk's outputs,
// O = diag(Gam) Q S + M D, with Q and M from the workspace, loaded two chunks ahead into two
// alternating operand sets, and Gam from the value slot, read in alpha_k. In beta_k the wave
// forms diag(Gam) Q S of chunk c_k and the second half of row tile r of chunk c_{k+1}'s V, then
// loads chunk c_{k+2}'s Q; in alpha_{k+1} it adds M D, stores the rows, reads chunk c_{k+1}'s
// Gam, forms the first half of chunk c_{k+2}'s V tile (V is double-buffered: c_{k+2}'s is
// written while the D and feed waves read c_{k+1}'s) and loads c_{k+3}'s x rows and c_{k+2}'s
// M. Row tile r
// of chunk c_0's V is built before alpha_0, when the wave also reads the old conv history of
// the run's first sequence.
struct OutQ {
    bf8 qf[4][2];
};
struct OutM {
    bf8 mf[2][2];
};
__device__ __forceinline__ void chain_out_load_q(const PrefillParams& p, const ChainRun& run, int k, int h, int src,
                                                 int r, int lane, OutQ& x) {
    const size_t c = (size_t)(run.wk + min(k, run.n - 1));
    const uint16_t* Qf = p.ws.Qf + (c * p.L.h_k + src) * kFragW;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) x.qf[ks][pl] = *reinterpret_cast<const bf8*>(Qf + frag_at(r, ks, 4, pl, lane));
}
__device__ __forceinline__ void chain_out_load_m(const PrefillParams& p, const ChainRun& run, int k, int h, int r,
                                                 int lane, OutM& x) {
    const size_t c = (size_t)(run.wk + min(k, run.n - 1));
    const uint8_t* Mf = p.ws.Mf + (c * p.L.h_v + h) * kFragMBytes;
    // Row tiles 0 and 1 end before token 32: their k-step 1 of M (tokens 32..63) is zero and not
    // stored; they load k-step 0 again in its place (a fixed number of loads, no extra bytes;
    // M D does not use it).
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int pl = 0; pl < 2; ++pl)
                x.mf[ks][pl] = *reinterpret_cast<const bf8*>(Mf + 2 * frag_at(r, r >= 2 ? ks : 0, 2, pl, lane));
}

template <int DC, bool SILU>
__device__ __forceinline__ void chain_output_role(const PrefillParams& p, uint8_t* lds, int lane, int r,
                                                  const ChainRun& run, int h, int src, int strip) {
    const Layer& L = p.L;
    const int li = lane & 15, lg4 = lane >> 4, j0 = strip * kStrip;
    float cw[DC];                                           // conv weights of the lane's v channel
    {
        const uint16_t* wp = L.conv_w + (size_t)v_channel(L, h, j0 + li) * DC;
#pragma unroll
        for (int i = 0; i < DC; ++i) cw[i] = bf16_to_f32(wp[i]);
    }
    const int n = run.n;
    // Chunks c_k .. c_{k+3} of the run (clamped to its last).
    RunChunk r0 = run_chunk(lds, 0), r1 = run_chunk(lds, min(1, n - 1)), r2 = run_chunk(lds, min(2, n - 1)),
             r3 = run_chunk(lds, min(3, n - 1));
    // x rows of chunk c_j in set j mod 2, loaded in alpha_{j-2}; row tile r of c_j's V built
    // from them in alpha_{j-1} (entries 0, 1; for r >= 2 in beta_{j-1} too) and beta_{j-1}
    // (entries 2, 3); chunk c_0's before alpha_0. The work splits so because the output waves
    // have room in both phases, waves 6 and 7 (r = 3, 2: their M D is twice as long, and they
    // share SIMDs with waves 2 and 3) in beta only.
    XStage x0, x1;
    stage_load<DC>(p, r0, h, strip, r, lane, x0);
    stage_conv<DC, SILU>(lds, x0, r, lane, cw, r0.len(), v_buf(0));
    stage_load<DC>(p, r1, h, strip, r, lane, x1);
    OutQ q0, q1;
    OutM m0, m1;
    chain_out_load_q(p, run, 0, h, src, r, lane, q0);
    chain_out_load_m(p, run, 0, h, r, lane, m0);
    chain_out_load_q(p, run, 1, h, src, r, lane, q1);
    chain_out_load_m(p, run, 1, h, r, lane, m1);
    const lds_u8* hbase = lane_at(lds, kOffH + lane * 16);
    const size_t row = (size_t)L.h_v * kD;
    v4 o;
    // A window buffer for o starts at the window's first token.
    int tw0 = 0, tw1;
    if (p.o_win) window_tokens(p, tw0, tw1);
    tw0 = __builtin_amdgcn_readfirstlane(tw0);              // waited for here, not in the loop
    // exp(G_t) of chunk c_k at this lane's rows, read from the value slot in alpha_k (the D wave
    // writes chunk c_{k+1}'s there in beta_k).
    const lds_u8* gmb = lane_at(lds, kOffV + 4 * kPlane + 4 * kChunk + 64 * r + 16 * lg4);
    v4 gam_k;
    // o rows 16 r + 4 lg4 + i of a chunk at a lane offset fixed for the run, from a chunk base
    // held in scalar registers; a full chunk stores without per-row tests.
    const uint32_t lofs = (uint32_t)((16 * r + 4 * lg4) * (int)row + li);
    auto store = [&](const RunChunk& g) {
        const int t0 = __builtin_amdgcn_readfirstlane(g.t0), len = __builtin_amdgcn_readfirstlane(g.len());
        const int tl = 16 * r + 4 * lg4;
        if (p.o_bf16) {
            uint16_t* ob = p.o_bf16 + ((size_t)t0 * L.h_v + h) * kD + j0;
            if (len >= kChunk) {
#pragma unroll
                for (int i = 0; i < 4; ++i) ob[lofs + (uint32_t)(i * (int)row)] = f32_to_bf16(o[i]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (tl + i < len) ob[lofs + (uint32_t)(i * (int)row)] = f32_to_bf16(o[i]);
            }
        }
        if (p.o) {
            float* ow = p.o + ((size_t)(t0 - tw0) * L.h_v + h) * kD + j0;
            if (len >= kChunk) {
#pragma unroll
                for (int i = 0; i < 4; ++i) ow[lofs + (uint32_t)(i * (int)row)] = o[i];
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (tl + i < len) ow[lofs + (uint32_t)(i * (int)row)] = o[i];
            }
        }
    };
    auto step = [&](int k, OutQ& Q, OutM& M, XStage& xa, XStage& xb) {
        lds_barrier();                                      // beta_k: S_k handed over
        bf8 sb[4][2];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int pl = 0; pl < 2; ++pl) sb[ks][pl] = *(const lds_bf8*)(hbase + (2 * ks + pl) * kPlane);
        // The three split products in separate accumulators: three short dependency chains.
        v4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            a0 = mfma_bf16(Q.qf[ks][0], sb[ks][0], a0);
            a1 = mfma_bf16(Q.qf[ks][0], sb[ks][1], a1);
            a2 = mfma_bf16(Q.qf[ks][1], sb[ks][0], a2);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = (a0[i] + a1[i] + a2[i]) * gam_k[i];
        // Entries 2, 3 of row tile r of chunk c_{k+1}'s V (0, 1 formed in alpha_k), then chunk
        // c_{k+2}'s Q. Every step issues all its loads (clamped to the run's last chunk), so that
        // the waits for them count a fixed number of later operations.
        if (r >= 2) stage_conv<DC, SILU, 0>(lds, xb, r, lane, cw, r1.len(), v_buf(k + 1));
        stage_conv<DC, SILU, 1>(lds, xa, r, lane, cw, r1.len(), v_buf(k + 1));
        chain_out_load_q(p, run, k + 2, h, src, r, lane, Q);
        lds_barrier();                                      // alpha_{k+1}: D_k handed over
        // M D: tokens 0-31 for every row tile, tokens 32-63 for row tiles 2 and 3 only.
        bf8 db[2][2];
        {
            const v4 d0 = *(const lds_v4*)(hbase + kHandS), d1 = *(const lds_v4*)(hbase + kHandS + kPlane);
            split_tiles(d0, d1, db[0][0], db[0][1]);
        }
        a0 = o;
        a1 = v4{0.f, 0.f, 0.f, 0.f};
        a2 = a1;
        a0 = mfma_bf16(M.mf[0][0], db[0][0], a0);
        a1 = mfma_bf16(M.mf[0][0], db[0][1], a1);
        a2 = mfma_bf16(M.mf[0][1], db[0][0], a2);
        if (r >= 2) {
            const v4 d2 = *(const lds_v4*)(hbase + kHandS + 2 * kPlane), d3 = *(const lds_v4*)(hbase + kHandS + 3 * kPlane);
            split_tiles(d2, d3, db[1][0], db[1][1]);
            a0 = mfma_bf16(M.mf[1][0], db[1][0], a0);
            a1 = mfma_bf16(M.mf[1][0], db[1][1], a1);
            a2 = mfma_bf16(M.mf[1][1], db[1][0], a2);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = a0[i] + a1[i] + a2[i];
        store(r0);
        gam_k = *(const lds_v4*)gmb;                        // chunk c_{k+1}'s
        // Entries 0, 1 of row tile r of chunk c_{k+2}'s V (its x rows in xa), then chunk
        // c_{k+3}'s x rows into xb (chunk c_{k+1}'s, staged in alpha_k), and chunk c_{k+2}'s M.
        if (r < 2) stage_conv<DC, SILU, 0>(lds, xa, r, lane, cw, r2.len(), v_buf(k + 2));
        stage_load<DC>(p, r3, h, strip, r, lane, xb);
        chain_out_load_m(p, run, k + 2, h, r, lane, M);
        r0 = r1;
        r1 = r2;
        r2 = r3;
        r3 = run_chunk(lds, min(k + 4, n - 1));
    };
    lds_barrier();                                          // alpha_0
    gam_k = *(const lds_v4*)gmb;
    if (r < 2) stage_conv<DC, SILU, 0>(lds, x1, r, lane, cw, r1.len(), v_buf(1));
    stage_load<DC>(p, r2, h, strip, r, lane, x0);
    for (int k = 0; k < n; k += 2) {
        step(k, q0, m0, x0, x1);
        if (k + 1 < n) step(k + 1, q1, m1, x1, x0);
    }
}

// Feed role (wave 5). In alpha_k it starts copying chunk c_{k+1}'s key planes (written by the
// chunk kernel in this layout) into key slot (k+1) mod 3 with direct global-to-LDS loads and
// reads what row tiles 2 and 3 of D_k need; in beta_k it forms them and waits for the copies
// before the barrier. After a sequence's last chunk it also writes the new rolling conv history of the
// workgroup's channels: its share of the sequence's q/k channels (the h_v * 8 workgroups that
// run the sequence split them into contiguous ranges; the chunk kernel has read their old
// history) and the strip's 16 v channels (whose old history the output waves have read into
// the V of the sequence's first chunk by then, at the latest in beta of the chunk before it).
// Nothing else in this kernel writes conv_state.
__device__ __forceinline__ void chain_feed_role(const PrefillParams& p, uint8_t* lds, int lane, const ChainRun& run,
                                                int h, int strip, int src) {
    const Layer& L = p.L;
    auto copy_keys = [&](int k) {
        const uint8_t* g = p.ws.Kp + ((size_t)(run.wk + k) * L.h_k + src) * kKSlot + lane * 16;
        lds_u8* d = (lds_u8*)lds + kOffK + (k % kKSlots) * kKSlot;
#pragma unroll
        for (int i = 0; i < kKSlot / kPlane; ++i) __builtin_amdgcn_global_load_lds(g + i * kPlane, d + i * kPlane, 16, 0, 0);
    };
    // s_waitcnt lgkmcnt(0) alone (gfx9 layout: vmcnt bits 3:0 and 15:14 and expcnt 6:4 at their
    // maxima, lgkmcnt 11:8 zero).
    constexpr int kWaitLgkm0 = 0xc07f;
    auto wait_barrier = [&]() {
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0);                      // the copies have landed
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
    };

    const int n = run.n;
    // The lane's channels of a commit: q/k channel cq (at most 64 per workgroup, since
    // h_k <= h_v) and, in lanes 0-15, v channel cv.
    const int ng = L.h_v * kStrips, gi = h * kStrips + strip, cqk = 2 * L.h_k * kD, per = (cqk + ng - 1) / ng;
    const bool has_q = lane < per && gi * per + lane < cqk, has_v = lane < kStrip;
    const int cq = has_q ? gi * per + lane : 0, cv = v_channel(L, h, strip * kStrip + (lane & (kStrip - 1)));
    // T' (2, 0), (3, 0), (2, 1), (3, 1), hi and lo each, of a chunk, in registers (one of two
    // sets, loaded in alpha of the chunk before; clamped to the run's last chunk).
    struct FT {
        u4x f[8];
    };
    auto tload = [&](int k, FT& t) {
        const uint8_t* tsrc = p.ws.Tf + ((size_t)(run.wk + min(k, n - 1)) * L.h_v + h) * kTriFragBytes;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = i >> 1, mt = 2 + (e & 1), ks = e >> 1;
            t.f[i] = load_tri_frag(tsrc, mt, ks, i & 1, lane);
        }
    };
    RunChunk rc = run_chunk(lds, 0);                        // chunk c_k
    FT f0, f1;
    tload(0, f0);
    copy_keys(0);
    wait_barrier();                                         // alpha_0
    const int lg4 = lane >> 4;
    const lds_u8* vb0 = lane_at(lds, kOffV + lane * 16);
    const lds_u8* vb1 = lane_at(lds, kOffV1 + lane * 16);
    const lds_u8* eb = lane_at(lds, kOffV + 4 * kPlane + 16 * lg4);
    const lds_u8* wb = lane_at(lds, kOffW + lane * 16);
    // cur: chunk c_k's T'; oth: reloaded with c_{k+1}'s (it held c_{k-1}'s).
    auto step = [&](int k, const FT& cur, FT& oth) {
        // Row tiles 2, 3 of D_k: V and the decay factors of chunk c_k read in alpha_k.
        tload(k + 1, oth);
        v4 V[4], Gm[4], E[2];
        const lds_u8* vb = (k & 1) ? vb1 : vb0;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            V[mt] = *(const lds_v4*)(vb + mt * kPlane);
            Gm[mt] = *(const lds_v4*)(eb + 4 * kChunk + mt * 64);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) E[t] = *(const lds_v4*)(eb + (2 + t) * 64);
        // After a sequence's last chunk, its new histories: loaded before this chunk's copies
        // are issued, stored in beta_k.
        const RunChunk cc = rc;
        HistNew hq, hv;
        if (cc.ends()) {
            hq = hist_fetch(p, cq, cc.lo, cc.hi - cc.lo, cc.s);
            hv = hist_fetch(p, cv, cc.lo, cc.hi - cc.lo, cc.s);
        }
        if (k + 1 < n) rc = run_chunk(lds, k + 1);
        // Chunk c_{k+1}'s keys go to the slot of chunk c_{k-2}, whose K^T the state waves read
        // in beta_{k-2}; they are read from alpha_{k+1} on.
        if (k + 1 < n) copy_keys(k + 1);
        // beta_k: nothing this wave wrote to LDS is pending; the copies and loads stay in flight.
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
        {
            bf8 F0[4][2], F1[4][2];                         // T' (2, 0), (3, 0); T' (2, 1), (3, 1)
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int pl = 0; pl < 2; ++pl) {
                    F0[t][pl] = __builtin_bit_cast(bf8, cur.f[2 * t + pl]);
                    F1[t][pl] = __builtin_bit_cast(bf8, cur.f[4 + 2 * t + pl]);
                }
            v4 X[4];
            d_x<4>(wb, V, Gm, 0, X);
            bf8 xh[2], xl[2];
            split_tiles(X[0], X[1], xh[0], xl[0]);
            split_tiles(X[2], X[3], xh[1], xl[1]);
            v4 D[2] = {v4{0.f, 0.f, 0.f, 0.f}, v4{0.f, 0.f, 0.f, 0.f}};
            mfma2_split(F0, xh[0], xl[0], D);               // tokens 0-31
            mfma2_split(F1, xh[1], xl[1], D);               // tokens 32-63
            d_hand(lds, lane, 1, E, D);
        }
        if (cc.ends()) {
            if (has_q) hist_put(p, cq, cc.s, hq);
            if (has_v) hist_put(p, cv, cc.s, hv);
        }
        wait_barrier();                                     // alpha_{k+1}: the copies have landed
    };
    for (int k = 0; k < n; k += 2) {
        step(k, f0, f1);
        if (k + 1 < n) step(k + 1, f1, f0);
    }
}

template <int DC, bool SILU>
__global__ void __launch_bounds__(kChainWaves * kWave) chain_kernel(const PrefillParams p) {
    __shared__ __align__(16) uint8_t lds[kChainLds];

    const Layer& L = p.L;
    // XCD-aware mapping: the 8 strips of one (head, group) pair share an XCD, so its L2 serves
    // the chunk operands to all of them. Group g of G runs the window's chunks from the g-th of
    // G near-equal shares on, each share's start moved to the next sequence start (group 0
    // starts at the window's first chunk, continuing a sequence begun in an earlier window).
    const int lin = blockIdx.x, xcd = lin & 7, kq = lin >> 3;
    const int strip = kq & (kStrips - 1);
    const int pair = (kq / kStrips) * 8 + xcd;
    if (pair >= p.G * L.h_v) return;
    const int h = pair % L.h_v, grp = pair / L.h_v, src = src_of(L, h);
    int nc;
    if (p.single) {
        int lo, hi;
        seq_bounds(p, 0, lo, hi);
        nc = (hi - lo + kChunk - 1) / kChunk;
    } else {
        nc = p.ws.chunk_off[p.n_seq];
    }
    const int nw = min(p.W, nc - p.cb);                     // the window's chunks
    if (nw <= 0) return;
    auto share_start = [&](int g) {
        if (g == 0) return p.cb;
        if (g >= p.G) return p.cb + nw;
        const int x = p.cb + (int)((long long)g * nw / p.G);
        const int4 r = p.ws.chunk_rec[x];
        return r.y == r.z ? x : min(p.ws.chunk_off[r.x + 1], p.cb + nw);
    };
    ChainRun run;
    run.lo = run.hi = 0;
    if (p.single) seq_bounds(p, 0, run.lo, run.hi);
    run.a = share_start(grp);
    run.n = share_start(grp + 1) - run.a;
    if (run.n <= 0) return;
    run.wk = run.a - p.cb;
    // The run's chunk records, read by every role from LDS (n <= W <= kMaxWindow).
    if ((int)threadIdx.x < run.n) {
        const int t = threadIdx.x;
        const int4 v = p.single ? int4{0, run.lo + (run.a + t) * kChunk, run.lo, run.hi} : p.ws.chunk_rec[run.a + t];
        *(__attribute__((address_space(3))) u4x*)((lds_u8*)lds + kOffR + 16 * t) =
            u4x{(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
    }
    __syncthreads();
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x & (kWave - 1);
    const int j0 = strip * kStrip;

    if (w <= 1) {
        chain_state_role(p, lds, lane, run, w, h, j0);
    } else if (w == 4) {
        chain_d_role(p, lds, lane, run, h);
    } else if (w == 5) {
        chain_feed_role(p, lds, lane, run, h, strip, src);
    } else {
        // Row tiles 0, 1 on waves 2, 3 and 3, 2 on waves 6, 7: each SIMD's pair runs 3 of M D's
        // 6 k-steps (2-4% faster than tiles 2, 3 on waves 6, 7).
        chain_output_role<DC, SILU>(p, lds, lane, w < 4 ? w - 2 : 9 - w, run, h, src, strip);
    }
}

// ---------------------------------------------------------------------------------------
// out_gate_kernel: gated RMS output norm of every (token, v head) row, one wave per row,
// reading the fp32 outputs the chain wrote (ix_gdn_prefill_gated only).
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) out_gate_kernel(const float* __restrict__ o, const OutGate g, long long rows) {
    const long long r = (long long)blockIdx.x * 4 + threadIdx.x / kWave;
    if (r >= rows) return;
    const int lane = threadIdx.x & (kWave - 1);
    const size_t row = (size_t)r * kD;
    out_gate_head(g, row, o[row + lane], o[row + lane + kWave], lane);
}

// The same norm over one window's rows, for the gated prefill without a caller o: the chain
// wrote the window's fp32 outputs to p.o, row 0 being the window's first token.
__global__ void __launch_bounds__(256) out_gate_window_kernel(const PrefillParams p, const OutGate g) {
    int t0, t1;
    window_tokens(p, t0, t1);
    const long long r = (long long)blockIdx.x * 4 + threadIdx.x / kWave;       // row in the window
    if (r >= (long long)(t1 - t0) * p.L.h_v) return;
    const int lane = threadIdx.x & (kWave - 1);
    const size_t row = (size_t)r * kD;
    out_gate_head(g, (size_t)t0 * p.L.h_v * kD + row, p.o[row + lane], p.o[row + lane + kWave], lane);
}

}  // namespace
}  // namespace ixg

extern "C" hipError_t ix_gdn_check_cfg_(const ix_gdn_cfg* c);

extern "C" hipError_t ix_gdn_check_gate_(const ix_gdn_out_gate* g);

// Workspace bytes for windows of W chunks; with gwin, plus the window's fp32 outputs (the gated
// prefill's norm input when the caller passes no o).
static size_t prefill_ws_bytes(const ix_gdn_cfg* cfg, int n_seq, int T, size_t W, bool gwin) {
    size_t off[ixg::kWsSections];
    size_t b = ixg::ws_layout(cfg, n_seq, T, W, off);
    if (gwin) b += ixg::align256(W * ixg::kChunk * cfg->h_v * ixg::kD * sizeof(float));
    return b;
}

// Windows of at most kMaxWindow chunks (5,120 tokens): the chunk operands of one window (146 MiB
// at the Qwen3-Next head layout) then stay in MI355X's 256 MB Infinity Cache between the chunk
// kernel writing them and the chain reading them (configuration 4: 1.60 ms in 80-chunk windows,
// 1.80 ms in 112-chunk ones). The default workspace holds such a window, so it stops growing
// with total_T (only the chunk tables do, 16 bytes per chunk).
using ixg::kMaxWindow;

extern "C" size_t ix_gdn_prefill_workspace_size(const ix_gdn_cfg* cfg, int n_seq, int total_T) {
    if (ix_gdn_check_cfg_(cfg) != hipSuccess || n_seq <= 0 || total_T < 0) return 0;
    return prefill_ws_bytes(cfg, n_seq, total_T, std::min(ixg::max_chunks(n_seq, total_T), (size_t)kMaxWindow), false);
}

extern "C" size_t ix_gdn_prefill_gated_workspace_size(const ix_gdn_cfg* cfg, int n_seq, int total_T) {
    if (ix_gdn_check_cfg_(cfg) != hipSuccess || n_seq <= 0 || total_T < 0) return 0;
    return prefill_ws_bytes(cfg, n_seq, total_T, std::min(ixg::max_chunks(n_seq, total_T), (size_t)kMaxWindow), true);
}

extern "C" size_t ix_gdn_prefill_window_workspace_size(const ix_gdn_cfg* cfg, int n_seq, int total_T,
                                                       int window_chunks, int gated) {
    if (ix_gdn_check_cfg_(cfg) != hipSuccess || n_seq <= 0 || total_T < 0 || window_chunks < 1) return 0;
    const size_t W = std::min((size_t)window_chunks, ixg::max_chunks(n_seq, total_T));
    return prefill_ws_bytes(cfg, n_seq, total_T, W, gated != 0);
}

// One window: the chunk kernel, then the chain. The conv activation and width are template
// parameters: inlined into every unrolled conv output, a runtime choice would carry the
// activation's code in the kernels that do not use it.
template <int DC>
static void launch_prefill(const ixg::PrefillParams& p, dim3 tgrid, dim3 cgrid, dim3 cblock, bool silu,
                           hipStream_t s) {
    using namespace ixg;
    if (silu) {
        hipLaunchKernelGGL((tri_kernel<DC, true>), tgrid, dim3(kChunkThreads), 0, s, p);
        hipLaunchKernelGGL((chain_kernel<DC, true>), cgrid, cblock, 0, s, p);
    } else {
        hipLaunchKernelGGL((tri_kernel<DC, false>), tgrid, dim3(kChunkThreads), 0, s, p);
        hipLaunchKernelGGL((chain_kernel<DC, false>), cgrid, cblock, 0, s, p);
    }
}

static hipError_t prefill_impl(const ix_gdn_cfg* cfg, int n_seq, int total_T, const int32_t* cu_seqlens,
                               const uint16_t* x, uint16_t* conv_state, const uint16_t* conv_w, const uint16_t* a,
                               const uint16_t* b, const float* A_log, const float* dt_bias, float* state, float* o,
                               uint16_t* o_bf16, const ix_gdn_out_gate* gate, void* workspace,
                               size_t workspace_bytes, hipStream_t s) {
    using namespace ixg;
    hipError_t e = ix_gdn_check_cfg_(cfg);
    if (e != hipSuccess) return e;
    if (gate && (e = ix_gdn_check_gate_(gate)) != hipSuccess) return e;
    if (n_seq <= 0 || total_T < 0) return hipErrorInvalidValue;
    if (!cu_seqlens || !conv_state || !conv_w || !A_log || !dt_bias || !state) return hipErrorInvalidValue;
    if (total_T == 0) return hipSuccess;                       // nothing to consume
    if (!x || !a || !b || !workspace) return hipErrorInvalidValue;
    if (reinterpret_cast<uintptr_t>(workspace) & 255) return hipErrorInvalidValue;
    if (reinterpret_cast<uintptr_t>(state) & 15) return hipErrorInvalidValue;      // float4 state accesses
    // The window: as many chunks as the workspace holds (all of them with the full size).
    const bool gwin = gate && !o;
    const size_t NCmax = max_chunks(n_seq, total_T);
    if (workspace_bytes < prefill_ws_bytes(cfg, n_seq, total_T, 1, gwin)) return hipErrorInvalidValue;
    size_t W = 1, W_hi = std::min(NCmax, (size_t)kMaxWindow);
    while (W < W_hi) {
        const size_t mid = (W + W_hi + 1) / 2;
        if (prefill_ws_bytes(cfg, n_seq, total_T, mid, gwin) <= workspace_bytes) W = mid;
        else W_hi = mid - 1;
    }
    size_t off[kWsSections];
    const size_t need = ws_layout(cfg, n_seq, total_T, W, off);
    const long long NC = (long long)NCmax;
    if (NC * cfg->h_v > 0x7fffffffLL) return hipErrorInvalidValue;
    const long long rows = (long long)total_T * cfg->h_v;
    if (gate && (rows + 3) / 4 > 0x7fffffffLL) return hipErrorInvalidValue;

    PrefillParams p;
    p.L = make_layer(cfg, conv_w, A_log, dt_bias);
    p.ws = ws_bind(static_cast<char*>(workspace), off);
    p.cu = cu_seqlens; p.x = x; p.conv_state = conv_state; p.a = a; p.b = b;
    p.state = state; p.o = o; p.o_bf16 = o_bf16;
    p.n_seq = n_seq; p.T = total_T; p.NC = (int)NC;
    p.single = n_seq == 1;
    p.o_win = gwin;
    if (gwin) p.o = reinterpret_cast<float*>(static_cast<char*>(workspace) + need);   // the norm's input

    // Chain workgroups: (v head, strip, group), G groups splitting each window's chunks at
    // sequence starts; one group while the h_v * 8 (head, strip) runs fill every CU.
    p.G = 1;
    if (!p.single) p.G = std::max(1, std::min(n_seq, ixg::device_cu_count(s) / (cfg->h_v * kStrips)));

    if (!p.single) hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, p);
    const long long groups = ((long long)p.G * cfg->h_v + 7) / 8;
    const dim3 cgrid((unsigned)(groups * 8 * kStrips)), cblock(kChainWaves * kWave);
    const bool silu = cfg->conv_act == IX_GDN_ACT_SILU;
    const OutGate og = make_out_gate(gate);
    // Windows run in stream order: each chain resumes from the state and conv history the
    // previous one left; a window past the last chunk finds nothing to do.
    for (size_t cb = 0; cb < NCmax; cb += W) {
        p.cb = (int)cb;
        p.W = (int)std::min(W, NCmax - cb);
        const dim3 tgrid((unsigned)p.W, (unsigned)cfg->h_k);
        switch (cfg->d_conv) {
            case 2: launch_prefill<2>(p, tgrid, cgrid, cblock, silu, s); break;
            case 3: launch_prefill<3>(p, tgrid, cgrid, cblock, silu, s); break;
            default: launch_prefill<4>(p, tgrid, cgrid, cblock, silu, s); break;
        }
        if (gwin)
            hipLaunchKernelGGL(out_gate_window_kernel, dim3((unsigned)(((long long)p.W * kChunk * cfg->h_v + 3) / 4)),
                               dim3(256), 0, s, p, og);
    }
    if (gate && !gwin)
        hipLaunchKernelGGL(out_gate_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, p.o, og, rows);
    return hipGetLastError();
}

extern "C" hipError_t ix_gdn_prefill(const ix_gdn_cfg* cfg, int n_seq, int total_T, const int32_t* cu_seqlens,
                                     const uint16_t* x, uint16_t* conv_state, const uint16_t* conv_w,
                                     const uint16_t* a, const uint16_t* b, const float* A_log,
                                     const float* dt_bias, float* state, float* o, uint16_t* o_bf16,
                                     void* workspace, size_t workspace_bytes, hipStream_t s) {
    return prefill_impl(cfg, n_seq, total_T, cu_seqlens, x, conv_state, conv_w, a, b, A_log, dt_bias, state, o,
                        o_bf16, nullptr, workspace, workspace_bytes, s);
}

extern "C" hipError_t ix_gdn_prefill_gated(const ix_gdn_cfg* cfg, int n_seq, int total_T, const int32_t* cu_seqlens,
                                           const uint16_t* x, uint16_t* conv_state, const uint16_t* conv_w,
                                           const uint16_t* a, const uint16_t* b, const float* A_log,
                                           const float* dt_bias, float* state, float* o, uint16_t* o_bf16,
                                           const ix_gdn_out_gate* gate, void* workspace, size_t workspace_bytes,
                                           hipStream_t s) {
    if (!gate) return hipErrorInvalidValue;
    return prefill_impl(cfg, n_seq, total_T, cu_seqlens, x, conv_state, conv_w, a, b, A_log, dt_bias, state, o,
                        o_bf16, gate, workspace, workspace_bytes, s);
}
