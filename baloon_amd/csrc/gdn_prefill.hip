// gdn_prefill.hip -- chunked WY-form GDN prefill for gfx950 (ix_gdn_prefill).
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
//   T       = (I + A)^-1                                    (unit lower triangular)
//   W       = T diag(beta Gam) K,    U = T diag(beta) V     (64 x 128 each)
//   D       = U - W S                                       (rows d_t)
//   M[t][s] = exp(G_t - G_s) (q_t . k_s)                    (s <= t)
//   O       = diag(Gam) Q S + M D
//   S'      = Gam_last S + K^T diag(exp(G_last - G_s)) D
// Only differences G_t - G_s with t >= s are exponentiated, so no intermediate overflows
// however strong the decay (Gam_t itself may underflow to 0, which is its correct value).
//
// Kernels, in stream order:
//   plan_kernel    clamps cu_seqlens to a non-decreasing sequence in [0, total_T] and builds
//                  the chunk table (sequence and first token of each chunk)
//   chunk_kernel   per (chunk, q/k head): conv (history from conv_state at sequence starts),
//                  L2 norms of q and k; K K^T and Q K^T on fp32 MFMA (lower block triangle),
//                  once for all the v heads mapped to the q/k head; then per v head its
//                  decay and beta, its v rows, A and M, T = (I + A)^-1 by a blocked MFMA
//                  inverse, W = T diag(beta Gam) K and U = T diag(beta) V as MFMA GEMMs; the
//                  chain's operands W, M, K^T, Q written as split-bf16 MFMA fragments
//   commit_kernel  per sequence and channel: the new rolling conv history
//   chain_kernel   per (sequence, v head, 32-column state slice): walks the chunks in order
//                  carrying the state slice in MFMA accumulators; D, O and S' on split-bf16
//                  MFMA (three bf16 products per fp32 product), state and output work on
//                  separate waves. Columns of the state are independent, so 4 slices per
//                  head share a head's chain.
// fp32 MFMA for the chunk-local algebra and split-bf16 MFMA for the chain keep the chunked
// result within ~1e-5 (state) of the token-by-token recurrence in double.
#include "gdn_common.h"

namespace ixg {
namespace {

constexpr int kChunk = 64;
constexpr int kPlanThreads = 1024;

typedef float v4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4 mfma4(float a, float b, v4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------------------
// Workspace layout (host and device agree through this struct)
// ---------------------------------------------------------------------------------------
struct Ws {
    int32_t* seq_lo;     // [n_seq + 1] clamped token offsets
    int32_t* chunk_off;  // [n_seq + 1] first chunk of each sequence; chunk_off[n_seq] = #chunks
    int32_t* chunk_seq;  // [NC]
    int32_t* chunk_t0;   // [NC]
    uint16_t* Wf;        // [NC][h_v] W (64 x 128) as split-bf16 A fragments
    float* Ut;           // [NC][h_v][128][64]  U transposed (column j of U is row j)
    uint16_t* Mf;        // [NC][h_v] M (64 x 64) as split-bf16 A fragments
    float* G;            // [NC][h_v][64] cumulative log decay (padded rows repeat the last)
    uint16_t* Ktf;       // [NC][h_k] K^T (128 x 64, zero beyond the chunk length) as fragments
    uint16_t* Qf;        // [NC][h_k] Q (64 x 128, zero beyond the chunk length) as fragments
    float* sink;         // [16][64] target of the chain's stores for rows past a sequence end
};
constexpr int kWsSections = 11;

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Byte offsets of every workspace section for (n_seq, T); returns the total size.
inline size_t ws_layout(const ix_gdn_cfg* c, int n_seq, int T, size_t off[kWsSections]) {
    const size_t NC = (size_t)(T + kChunk - 1) / kChunk + (size_t)n_seq;
    const size_t sz[kWsSections] = {
        sizeof(int32_t) * (n_seq + 1), sizeof(int32_t) * (n_seq + 1), sizeof(int32_t) * NC, sizeof(int32_t) * NC,
        sizeof(float) * NC * c->h_v * kChunk * kD, sizeof(float) * NC * c->h_v * kChunk * kD,
        sizeof(float) * NC * c->h_v * kChunk * kChunk, sizeof(float) * NC * c->h_v * kChunk,
        sizeof(float) * NC * c->h_k * kD * kChunk, sizeof(float) * NC * c->h_k * kChunk * kD,
        sizeof(float) * 16 * kWave,
    };
    size_t pos = 0;
    for (int i = 0; i < kWsSections; ++i) { off[i] = pos; pos += align256(sz[i]); }
    return pos;
}

inline Ws ws_bind(char* base, const size_t off[kWsSections]) {
    Ws w;
    w.seq_lo = reinterpret_cast<int32_t*>(base + off[0]);
    w.chunk_off = reinterpret_cast<int32_t*>(base + off[1]);
    w.chunk_seq = reinterpret_cast<int32_t*>(base + off[2]);
    w.chunk_t0 = reinterpret_cast<int32_t*>(base + off[3]);
    w.Wf = reinterpret_cast<uint16_t*>(base + off[4]);
    w.Ut = reinterpret_cast<float*>(base + off[5]);
    w.Mf = reinterpret_cast<uint16_t*>(base + off[6]);
    w.G = reinterpret_cast<float*>(base + off[7]);
    w.Ktf = reinterpret_cast<uint16_t*>(base + off[8]);
    w.Qf = reinterpret_cast<uint16_t*>(base + off[9]);
    w.sink = reinterpret_cast<float*>(base + off[10]);
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
    float* o;                   // [T][h_v][128] or null
    uint16_t* o_bf16;           // [T][h_v][128] or null
    int n_seq, T, NC;
};

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
    // the chunk table: chunk c belongs to the last sequence s with chunk_off[s] <= c
    const int nc = run;
    for (int c = tid; c < nc; c += kPlanThreads) {
        int lo = 0, hi = n - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (p.ws.chunk_off[mid] <= c) lo = mid; else hi = mid - 1;
        }
        p.ws.chunk_seq[c] = lo;
        p.ws.chunk_t0[c] = p.ws.seq_lo[lo] + (c - p.ws.chunk_off[lo]) * kChunk;
    }
}

// Chunk geometry: sequence, first token, tokens in the chunk, position of the first token
// within its sequence. Returns false for grid slots beyond the chunk count.
struct ChunkGeo { int s, t0, len, pos0; };
__device__ __forceinline__ bool chunk_geo(const PrefillParams& p, int c, ChunkGeo& g) {
    if (c >= p.ws.chunk_off[p.n_seq]) return false;
    g.s = p.ws.chunk_seq[c];
    g.t0 = p.ws.chunk_t0[c];
    const int lo = p.ws.seq_lo[g.s], hi = p.ws.seq_lo[g.s + 1];
    g.len = min(kChunk, hi - g.t0);
    g.pos0 = g.t0 - lo;
    return true;
}

// ---------------------------------------------------------------------------------------
// Conv of 16 consecutive tokens of a chunk for the channel pair (ch, ch + 1), one pair per
// lane, so that every x access of a wave is one 256-byte row segment. Tokens tb .. tb + n - 1
// of the chunk (n wave-uniform, 1..16); the history of the first one comes from x or, before
// the sequence start, from the sequence's conv state ([C][dc-1] per sequence: channel ch's
// entries, then channel ch+1's). The loads and the arithmetic are separate steps, so that a
// wave can issue the loads well before it needs the rows (and before stores it issues in
// between, which its later waits would otherwise include).
// ---------------------------------------------------------------------------------------
constexpr int kConvTok = 16;

// The loads are unconditional and nothing touches the loaded words before conv_run: a
// load on one path only, or any use of a loaded value, makes the wave wait for every load
// it has in flight.
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
        const int pos = g.pos0 + tb - (DC - 1) + i;            // wave-uniform
        const uint16_t* xp = p.x + (size_t)(lo + max(pos, 0)) * L.C + ch;
        const uint16_t* sp = p.conv_state + ((size_t)g.s * L.C + ch) * (DC - 1) + (DC - 1) + min(pos, -1);
        in.h0[i] = *(pos >= 0 ? xp : sp);
        in.h1[i] = *(pos >= 0 ? xp + 1 : sp + (DC - 1));
    }
#pragma unroll
    for (int t = 0; t < kConvTok; ++t)
        in.xs[t] = *reinterpret_cast<const uint32_t*>(p.x + (size_t)(g.t0 + tb + min(t, n - 1)) * L.C + ch);
    // conv_w is [C][dc]: the two channels' 2 dc weights are dc aligned words (ch is even)
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(L.conv_w + (size_t)ch * DC);
#pragma unroll
    for (int i = 0; i < DC; ++i) in.w[i] = wp[i];
}

__device__ __forceinline__ float bf16_half(uint32_t word, int half) {
    return __uint_as_float(half ? (word & 0xffff0000u) : (word << 16));
}

template <int DC>
__device__ __forceinline__ void conv_run(const Layer& L, ConvIn<DC> in, float (&y0)[kConvTok],
                                         float (&y1)[kConvTok]) {
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
        if (L.conv_act == IX_GDN_ACT_SILU) { a0 = a0 * sigmoid_f(a0); a1 = a1 * sigmoid_f(a1); }
        y0[t] = a0;
        y1[t] = a1;
#pragma unroll
        for (int i = 0; i < DC - 2; ++i) { h0[i] = h0[i + 1]; h1[i] = h1[i + 1]; }
        h0[DC - 2] = x0;
        h1[DC - 2] = x1;
    }
}

// ---------------------------------------------------------------------------------------
// commit: the rolling conv history after each sequence, one thread per (sequence, channel)
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) commit_kernel(const PrefillParams p) {
    const Layer& L = p.L;
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)p.n_seq * L.C) return;
    const int s = (int)(idx / L.C), ch = (int)(idx % L.C);
    const int lo = p.ws.seq_lo[s], len = p.ws.seq_lo[s + 1] - lo;
    if (len == 0) return;
    uint16_t* st = p.conv_state + idx * (L.dc - 1);
    // extended history [old (dc-1 values) | the sequence's inputs]; the new history is its
    // last dc-1 entries, i.e. entries len .. len+dc-2. An entry below dc-1 is old history.
    const uint16_t o0 = st[0], o1 = L.dc > 2 ? st[1] : (uint16_t)0, o2 = L.dc > 3 ? st[2] : (uint16_t)0;
    uint16_t nw[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int ext = len + j;                               // index into the extended history
        const int pos = ext - (L.dc - 1);                      // token position when >= 0
        nw[j] = pos >= 0 ? p.x[(size_t)(lo + pos) * L.C + ch] : (ext == 0 ? o0 : ext == 1 ? o1 : o2);
    }
    st[0] = nw[0];
    if (L.dc > 2) st[1] = nw[1];
    if (L.dc > 3) st[2] = nw[2];
}

// ---------------------------------------------------------------------------------------
// Split-bf16 operand fragments.
//
// The chain runs its products on v_mfma_f32_16x16x32_bf16 with each fp32 operand x split
// into x_hi = bf16(x) and x_lo = bf16(x - x_hi); a product is hi*hi + hi*lo + lo*hi in fp32
// accumulators (relative error ~2^-16, against 2^-8 for one bf16 product). The chunk kernel
// writes the chain's A operands already split, in the instruction's A layout: fragment
// (m, ks) of a (rows x k) tile covers rows 16m..16m+15 and k = 32ks..32ks+31, and lane l of
// it holds row 16m + l%16, k = 32ks + 8(l/16) .. +7 as 8 bf16 (16 bytes). Stored
// [m][ks][plane hi, lo][lane][8]: one coalesced 16-byte load per lane per fragment and plane.
// ---------------------------------------------------------------------------------------
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef uint32_t u4x __attribute__((ext_vector_type(4)));

__device__ __forceinline__ size_t frag_at(int m, int ks, int nks, int plane, int lane) {
    return ((((size_t)m * nks + ks) * 2 + plane) * kWave + lane) * 8;       // in bf16 elements
}

// Split 8 fp32 values into hi and lo bf16 vectors.
__device__ __forceinline__ void split8(const float (&x)[8], bf8& hi, bf8& lo) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const __bf16 h = (__bf16)x[e];
        hi[e] = h;
        lo[e] = (__bf16)(x[e] - (float)h);
    }
}

__device__ __forceinline__ void store_frag(uint16_t* base, int m, int ks, int nks, int lane, const float (&x)[8]) {
    bf8 hi, lo;
    split8(x, hi, lo);
    *reinterpret_cast<bf8*>(base + frag_at(m, ks, nks, 0, lane)) = hi;
    *reinterpret_cast<bf8*>(base + frag_at(m, ks, nks, 1, lane)) = lo;
}

// Fragment sizes in bf16 elements: (rows/16) x (k/32) fragments x 2 planes x 512.
constexpr size_t kFragW = 4 * 4 * 2 * 512;     // 64 x 128 (W, Q)
constexpr size_t kFragM = 4 * 2 * 2 * 512;     // 64 x 64 (M)
constexpr size_t kFragKt = 8 * 2 * 2 * 512;    // 128 x 64 (K^T)

// ---------------------------------------------------------------------------------------
// chunk-local: grid (NC, h_k), 512 threads; workgroup = (chunk, q/k head) and, one after
// the other, the v heads mapped to that q/k head
// ---------------------------------------------------------------------------------------
constexpr int kKS = kD + 4;          // padded LDS row stride of the K / Q / V tiles
constexpr int kTS = kChunk + 4;      // row stride of the A / M / T tiles
constexpr int kChunkThreads = 512;
constexpr int kMaxMap = 16;          // v heads per q/k head (the configuration limit)

// The 10 blocks of the 4 x 4 lower block triangle, 16 x 16 each: wave w takes i = w, w+4, w+8.
__device__ __forceinline__ void tri_block(int i, int& br, int& bc) {
    br = i < 1 ? 0 : i < 3 ? 1 : i < 6 ? 2 : 3;
    bc = i - br * (br + 1) / 2;
}

// C += X (16 x 16 at x, row stride xs) * Y (16 x 16 at y, row stride ys) on fp32 MFMA
// (four 16x16x4 steps). Lane l supplies X[l%16][4k + l/16] and Y[4k + l/16][l%16]; C is in
// the MFMA layout (c[r] = C[4 (l/16) + r][l%16]).
__device__ __forceinline__ v4 mm16(const float* x, int xs, const float* y, int ys, v4 c, int lane) {
    const int r16 = lane & 15, k4 = lane >> 4;
#pragma unroll
    for (int k = 0; k < 4; ++k) c = mfma4(x[r16 * xs + 4 * k + k4], y[(4 * k + k4) * ys + r16], c);
    return c;
}
__device__ __forceinline__ void put16(float* z, int zs, const v4& c, int lane, float scale) {
#pragma unroll
    for (int r = 0; r < 4; ++r) z[(4 * (lane >> 4) + r) * zs + (lane & 15)] = scale * c[r];
}

// A and M of one v head from the raw products of this wave's triangle blocks (waves 0-3):
// A[t][s] = beta_t exp(G_t - G_s) (k_t . k_s) for s < t, M[t][s] = exp(G_t - G_s) (q_t . k_s)
// for s <= t, zero above the diagonal inside the diagonal blocks. The blocks above the
// diagonal are never written (nothing reads them).
__device__ __forceinline__ void am_head(const v4 (&kk)[3], const v4 (&qk)[3], const float* G, const float* Bt,
                                        float* A_s, float* M_s, int w, int li, int lg4) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int i = w + 4 * j;
        if (i >= 10) continue;
        int br, bc;
        tri_block(i, br, bc);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = 16 * br + 4 * lg4 + r, s = 16 * bc + li;
            float av = 0.0f, mv = 0.0f;
            if (s <= t) {
                const float e = expf(G[t] - G[s]);
                mv = e * qk[j][r];
                if (s < t) av = Bt[t] * e * kk[j][r];
            }
            A_s[t * kTS + s] = av;
            M_s[t * kTS + s] = mv;
        }
    }
}

// Phases (one workgroup, 8 waves; every barrier orders LDS only, so no wave ever waits for
// its own global stores):
//   gate inputs of the v heads | q and k rows of the chunk: conv, L2 norm, q scale, into LDS
//   (zero past the chunk end) | decay scan and beta of each v head | raw K K^T and Q K^T of
//   the lower block triangle on fp32 MFMA, kept in registers, while the other waves write
//   K^T and Q as split fragments | then, per mapped v head: M as fragments | T = (I + A)^-1:
//   the four 16 x 16 diagonal blocks by substitution (one wave, while four others compute
//   the next head's v rows), then the off-diagonal blocks T_ij = -T_ii sum_k A_ik T_kj in
//   three dependency levels of fp32 MFMA block products | W = T diag(beta Gam) K and
//   U = T diag(beta) V as fp32 MFMA GEMMs (the zero blocks of T skipped) | U^T stored from
//   the MFMA layout, W through LDS into fragments | A and M of the next head.
// The v rows of even and odd heads alternate between two tiles (the odd one is the q tile,
// free once the triangle and the Q fragments are done).
template <int DC>
__global__ void __launch_bounds__(kChunkThreads) chunk_kernel(const PrefillParams p) {
    __shared__ __align__(16) float lds[3 * kChunk * kKS + 2 * kChunk * kTS + 3 * 16 * 17];
    float (*K_s)[kKS] = reinterpret_cast<float (*)[kKS]>(lds);         // k rows
    float (*Q_s)[kKS] = K_s + kChunk;                                  // q rows, then v rows of odd heads
    float (*V_s)[kKS] = Q_s + kChunk;                                  // v rows of even heads
    float* A_s = lds + 3 * kChunk * kKS;                               // [64][kTS]
    float* M_s = A_s + kChunk * kTS;                                   // M, then T
    float* T_s = M_s;
    float (*W_s)[kKS] = reinterpret_cast<float (*)[kKS]>(A_s);        // W, over A and T
    float* P_s = M_s + kChunk * kTS;                                   // [3][16][17]
    static_assert(kChunk * kKS <= 2 * kChunk * kTS, "W fits over A and T");
    __shared__ float G_s[kMaxMap][kChunk], B_s[kMaxMap][kChunk], BG_s[kMaxMap][kChunk];

    ChunkGeo g;
    const int c = blockIdx.x;
    if (!chunk_geo(p, c, g)) return;
    const Layer& L = p.L;
    const int src = blockIdx.y, nmap = mapped_count(L, src);
    if (nmap == 0) return;
    const int lo = p.ws.seq_lo[g.s];
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int w = __builtin_amdgcn_readfirstlane(tid / kWave);        // wave-uniform: scalar branches
    const int li = lane & 15, lg4 = lane >> 4, c2 = 2 * lane;
    const size_t cs = (size_t)c * L.h_k + src;
    const int tb = kConvTok * (w & 3), nt = min(max(g.len - tb, 0), kConvTok);   // this wave's conv rows

    // Gate inputs of v heads w and w + 8 (lane = token), issued first.
    uint16_t ra[2] = {0, 0}, rb[2] = {0, 0};
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int hh = w + 8 * j;
        if (hh < nmap && lane < g.len) {
            const size_t ab = (size_t)(g.t0 + lane) * L.h_v + mapped_head(L, src, hh);
            ra[j] = p.a[ab];
            rb[j] = p.b[ab];
        }
    }

    // q rows (waves 0-3) and k rows (waves 4-7), 16 tokens per wave.
    {
        const bool isk = w >= 4;
        float y0[kConvTok], y1[kConvTok];
        if (nt > 0) {
            ConvIn<DC> in;
            conv_load<DC>(p, g, lo, isk ? k_channel(L, src, c2) : q_channel(L, src, c2), tb, nt, in);
            conv_run<DC>(L, in, y0, y1);
        } else {
#pragma unroll
            for (int t = 0; t < kConvTok; ++t) y0[t] = y1[t] = 0.0f;
        }
        // All 16 row sums first (independent, so their shuffle latencies overlap), then the
        // scaled rows; rows past the chunk end are zero.
        float ss[kConvTok];
#pragma unroll
        for (int t = 0; t < kConvTok; ++t) ss[t] = wave_sum(fmaf(y0[t], y0[t], y1[t] * y1[t]));
        const float scale = isk ? 1.0f : L.q_scale;
        float (*dst)[kKS] = isk ? K_s : Q_s;
#pragma unroll
        for (int t = 0; t < kConvTok; ++t) {
            const float inv = scale / sqrtf(ss[t] + L.l2_eps);
            *reinterpret_cast<float2*>(&dst[tb + t][c2]) = t < nt ? float2{y0[t] * inv, y1[t] * inv} : float2{0.0f, 0.0f};
        }
    }
    // Decay scan and beta of v heads w and w + 8.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int hh = w + 8 * j;
        if (hh >= nmap) continue;
        const int h = mapped_head(L, src, hh);
        const bool ok = lane < g.len;
        float lgt = ok ? log_gate(L, h, bf16_to_f32(ra[j])) : 0.0f;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {          // inclusive scan over the 64 lanes
            const float o = __shfl_up(lgt, off, kWave);
            if (lane >= off) lgt += o;
        }
        const float bt = ok ? sigmoid_f(bf16_to_f32(rb[j])) : 0.0f;
        G_s[hh][lane] = lgt;
        B_s[hh][lane] = bt;
        BG_s[hh][lane] = bt * expf(lgt);
        p.ws.G[((size_t)c * L.h_v + h) * kChunk + lane] = lgt;
    }
    lds_barrier();

    // Raw K K^T and Q K^T (waves 0-3). MFMA k index of (block 4m + e, lane group g) is
    // 16 m + 4 g + e for both operands. Waves 4-7 first issue the loads of the first v head's
    // rows, then write K^T (rows i, k = token t: 8 x 2 fragments) and Q (rows t, k = i:
    // 4 x 4 fragments) as split fragments.
    v4 kk[3], qk[3];
    ConvIn<DC> vin;
    if (w < 4) {
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int i = w + 4 * j;
            kk[j] = v4{0.f, 0.f, 0.f, 0.f};
            qk[j] = kk[j];
            if (i < 10) {
                int br, bc;
                tri_block(i, br, bc);
                const int arow = 16 * br + li;
#pragma unroll
                for (int m = 0; m < kD / 16; ++m) {
                    const v4 ak = *reinterpret_cast<const v4*>(&K_s[arow][16 * m + 4 * lg4]);
                    const v4 aq = *reinterpret_cast<const v4*>(&Q_s[arow][16 * m + 4 * lg4]);
                    const v4 bk = *reinterpret_cast<const v4*>(&K_s[16 * bc + li][16 * m + 4 * lg4]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        kk[j] = mfma4(ak[e], bk[e], kk[j]);
                        qk[j] = mfma4(aq[e], bk[e], qk[j]);
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);       // one block's operands live at a time
        }
    } else {
        if (nt > 0) conv_load<DC>(p, g, lo, v_channel(L, mapped_head(L, src, 0), c2), tb, nt, vin);
        const int t4 = tid - 4 * kWave;
        uint16_t* Ktf = p.ws.Ktf + cs * kFragKt;
        for (int u = t4; u < 8 * 2 * kWave; u += 4 * kWave) {
            const int ln = u & (kWave - 1), f = u / kWave, m = f >> 1, ks = f & 1;
            const int row = 16 * m + (ln & 15), k0 = 32 * ks + 8 * (ln >> 4);
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = K_s[k0 + e][row];
            store_frag(Ktf, m, ks, 2, ln, x);
        }
        uint16_t* Qf = p.ws.Qf + cs * kFragW;
        for (int u = t4; u < 4 * 4 * kWave; u += 4 * kWave) {
            const int ln = u & (kWave - 1), f = u / kWave, m = f >> 2, ks = f & 3;
            const int row = 16 * m + (ln & 15), k0 = 32 * ks + 8 * (ln >> 4);
            float x[8];
            const v4 a = *reinterpret_cast<const v4*>(&Q_s[row][k0]), b = *reinterpret_cast<const v4*>(&Q_s[row][k0 + 4]);
#pragma unroll
            for (int e = 0; e < 4; ++e) { x[e] = a[e]; x[e + 4] = b[e]; }
            store_frag(Qf, m, ks, 4, ln, x);
        }
    }
    lds_barrier();

    // v rows of the first head (waves 4-7); A and M of the first head (waves 0-3).
    if (w >= 4) {
        float y0[kConvTok], y1[kConvTok];
        if (nt > 0) conv_run<DC>(L, vin, y0, y1);
#pragma unroll
        for (int t = 0; t < kConvTok; ++t)
            *reinterpret_cast<float2*>(&V_s[tb + t][c2]) = t < nt ? float2{y0[t], y1[t]} : float2{0.0f, 0.0f};
    } else {
        am_head(kk, qk, G_s[0], B_s[0], A_s, M_s, w, li, lg4);
    }
    lds_barrier();

    for (int mi = 0; mi < nmap; ++mi) {
        const int h = mapped_head(L, src, mi);
        const size_t ch = (size_t)c * L.h_v + h;
        float (*Vb)[kKS] = (mi & 1) ? Q_s : V_s;                        // this head's v rows
        float (*Vn)[kKS] = (mi & 1) ? V_s : Q_s;                        // the next head's
        const bool next = mi + 1 < nmap, conv_next = w >= 4 && next && nt > 0;
        ConvIn<DC> nin;                    // the next head's conv inputs (waves 4-7)
        if (conv_next) conv_load<DC>(p, g, lo, v_channel(L, mapped_head(L, src, mi + 1), c2), tb, nt, nin);

        // M as fragments (4 x 2 fragments x 64 lanes: one unit per thread); the blocks
        // above the diagonal are zero.
        {
            uint16_t* Mf = p.ws.Mf + ch * kFragM;
            const int m = w >> 1, ks = w & 1;
            const int row = 16 * m + li, k0 = 32 * ks + 8 * lg4;
            float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (k0 < 16 * (m + 1)) {
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = M_s[row * kTS + k0 + e];
            }
            store_frag(Mf, m, ks, 2, lane, x);
        }
        lds_barrier();                     // M_s is read: T takes its place

        // Wave 0 inverts the four unit lower-triangular diagonal blocks of I + A (lane =
        // 16 b + column c); waves 4-7 compute the next head's v rows.
        if (w == 0) {
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
        } else if (w >= 4 && next) {
            float y0[kConvTok], y1[kConvTok];
            if (conv_next) conv_run<DC>(L, nin, y0, y1);
#pragma unroll
            for (int t = 0; t < kConvTok; ++t)
                *reinterpret_cast<float2*>(&Vn[tb + t][c2]) = t < nt ? float2{y0[t], y1[t]} : float2{0.0f, 0.0f};
        }
        lds_barrier();
        // Off-diagonal blocks: level 1 (1,0) (2,1) (3,2); level 2 (2,0) (3,1); level 3 (3,0).
        // T_ij = -T_ii P with P = sum_{k=j}^{i-1} A_ik T_kj (P through the wave's LDS scratch).
#pragma unroll
        for (int lev = 1; lev <= 3; ++lev) {
            if (w < 4 - lev) {
                const int j = w, i = w + lev;
                v4 pc = {0.f, 0.f, 0.f, 0.f};
                for (int k = j; k < i; ++k)
                    pc = mm16(A_s + (16 * i) * kTS + 16 * k, kTS, T_s + (16 * k) * kTS + 16 * j, kTS, pc, lane);
                float* Pw = P_s + w * 16 * 17;
                put16(Pw, 17, pc, lane, 1.0f);
                __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0): this wave's P stores done
                const v4 tc = mm16(T_s + (16 * i) * kTS + 16 * i, kTS, Pw, 17, v4{0.f, 0.f, 0.f, 0.f}, lane);
                put16(T_s + (16 * i) * kTS + 16 * j, kTS, tc, lane, -1.0f);
            }
            lds_barrier();
        }

        // W = T (beta Gam K) and U = T (beta V): wave w takes columns 16 w .. 16 w + 15 of
        // both, all four 16-row tiles; T[t][s] = 0 for s > t, so tile mt stops at k-step
        // 4 mt + 3.
        v4 wacc[4], uacc[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) { wacc[mt] = v4{0.f, 0.f, 0.f, 0.f}; uacc[mt] = wacc[mt]; }
        const int col = 16 * w + li;
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) {
            const int sr = 4 * ks + lg4;
            const float bw = K_s[sr][col] * BG_s[mi][sr], bu = B_s[mi][sr] * Vb[sr][col];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                if (ks > 4 * mt + 3) continue;               // compile-time after unrolling
                const float a = T_s[(16 * mt + li) * kTS + 4 * ks + lg4];
                wacc[mt] = mfma4(a, bw, wacc[mt]);
                uacc[mt] = mfma4(a, bu, uacc[mt]);
            }
            __builtin_amdgcn_sched_barrier(0);           // bounds the loads hoisted ahead
        }
        // U^T rows (column j of U: 4 consecutive tokens per lane and tile).
        float* Ut = p.ws.Ut + ch * kD * kChunk;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
            *reinterpret_cast<v4*>(Ut + (size_t)col * kChunk + 16 * mt + 4 * lg4) = uacc[mt];
        lds_barrier();                     // A and T are read: W takes their place
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) W_s[16 * mt + 4 * lg4 + r][col] = wacc[mt][r];
        lds_barrier();
        // W as fragments (4 x 4 x 64 = 1024 units, two per thread).
        uint16_t* Wf = p.ws.Wf + ch * kFragW;
#pragma unroll
        for (int rep = 0; rep < 2; ++rep) {
            const int u = tid + rep * kChunkThreads;
            const int ln = u & (kWave - 1), f = u / kWave, m = f >> 2, ks = f & 3;
            const int row = 16 * m + (ln & 15), k0 = 32 * ks + 8 * (ln >> 4);
            float x[8];
            const v4 a = *reinterpret_cast<const v4*>(&W_s[row][k0]), b = *reinterpret_cast<const v4*>(&W_s[row][k0 + 4]);
#pragma unroll
            for (int e = 0; e < 4; ++e) { x[e] = a[e]; x[e + 4] = b[e]; }
            store_frag(Wf, m, ks, 4, ln, x);
        }
        if (next) {
            lds_barrier();                 // W is read: the next head's A and M take its place
            if (w < 4) am_head(kk, qk, G_s[mi + 1], B_s[mi + 1], A_s, M_s, w, li, lg4);
            lds_barrier();
        }
    }
}

// ---------------------------------------------------------------------------------------
// chain: one workgroup per (sequence, v head, 32-column state slice), 512 threads
// ---------------------------------------------------------------------------------------
// The workgroup has 8 waves in two roles that meet at two barriers per chunk:
//   state waves (0-3): S -> LDS | W S, D = U - W S -> LDS | S' = Gam_last S + K^T (exp(G_last - G) D)
//   output waves (4-7):          | Q S                   | O = diag(Gam) Q S + M D
// All products are split-bf16 MFMA (16x16x32). The A operands (W, K^T, Q, M) come from the
// chunk kernel's fragments; the B operands (S, D, Dg) are split by their producer wave into
// LDS fragments of the B layout: fragment (ks, nt) covers k = 32ks..32ks+31 and columns
// 16nt..16nt+15; lane l holds column 16nt + l%16, k = 32ks + 8(l/16) .. +7.
// Lane (li = lane & 15, lg4 = lane >> 4) of role wave r: output rows 16r + 4lg4 + i in C layout;
// state wave r owns state rows 32r .. 32r + 31 (two 16-row m-tiles) of the slice's 32 columns.
// Each role loads the next chunk's operands (double buffer) while it computes the current one.
constexpr int kSlice = 32;                      // state columns per chain workgroup
constexpr int kSlices = kD / kSlice;            // 4
constexpr int kNT = kSlice / 16;                // 16-column tiles per slice

typedef float f4 __attribute__((ext_vector_type(4)));


// B-fragment LDS tiles of the chain (bf16 elements): S (k = state row, 4 ks), D and Dg (k = token, 2 ks).
constexpr int kBFrag = 2 * kWave * 8;                       // one (ks, nt) fragment, both planes
__device__ __forceinline__ int bfrag_at(int ks, int nt, int plane, int ln) {
    return ((ks * kNT + nt) * 2 + plane) * kWave * 8 + ln * 8;
}

// Write 4 consecutive k values (k = 4 q .. 4 q + 3 within the fragment's 32, q = 0..7) of
// column n (0..15) of fragment (ks, nt), split, into a B-fragment tile.
__device__ __forceinline__ void bfrag_put4(uint16_t* tile, int ks, int nt, int q, int n, const f4& v) {
    const int ln = 16 * (q >> 1) + n, e0 = 4 * (q & 1);
    uint16_t hi[4], lo[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const __bf16 hb = (__bf16)v[e];
        hi[e] = __builtin_bit_cast(uint16_t, hb);
        lo[e] = __builtin_bit_cast(uint16_t, (__bf16)(v[e] - (float)hb));
    }
    uint2 h2 = {(uint32_t)hi[0] | ((uint32_t)hi[1] << 16), (uint32_t)hi[2] | ((uint32_t)hi[3] << 16)};
    uint2 l2 = {(uint32_t)lo[0] | ((uint32_t)lo[1] << 16), (uint32_t)lo[2] | ((uint32_t)lo[3] << 16)};
    *reinterpret_cast<uint2*>(tile + bfrag_at(ks, nt, 0, ln) + e0) = h2;
    *reinterpret_cast<uint2*>(tile + bfrag_at(ks, nt, 1, ln) + e0) = l2;
}

struct StateOps {
    bf8 w[4][2];          // W fragments (m = r, ks 0..3), planes
    bf8 kt[2][2][2];      // K^T fragments (m = 2r + mt, ks 0..1), planes
    f4 u[kNT];            // U rows 16r + 4lg4 + i, columns j0 + 16nt + li
    f4 gv;                // G at those rows
    float glast;          // G of the chunk's last row
};
struct OutOps {
    bf8 q[4][2];          // Q fragments (m = r, ks 0..3), planes
    bf8 m[2][2];          // M fragments (m = r, ks 0..1), planes
    f4 gv;
    int t0, len;
};

struct ChainCtx {
    const PrefillParams* p;
    int h, src, seq_lo, seq_hi, c_begin, j0, r, li, lg4, lane;
};

__device__ __forceinline__ size_t chain_ch(const ChainCtx& x, int c) { return (size_t)c * x.p->L.h_v + x.h; }

__device__ __forceinline__ void load_state_ops(const ChainCtx& x, int c, StateOps& o) {
    const PrefillParams& p = *x.p;
    const size_t ch = chain_ch(x, c);
    const uint16_t* Wf = p.ws.Wf + ch * kFragW;
    const uint16_t* Kf = p.ws.Ktf + ((size_t)c * p.L.h_k + x.src) * kFragKt;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) o.w[ks][pl] = *reinterpret_cast<const bf8*>(Wf + frag_at(x.r, ks, 4, pl, x.lane));
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int pl = 0; pl < 2; ++pl)
                o.kt[mt][ks][pl] = *reinterpret_cast<const bf8*>(Kf + frag_at(2 * x.r + mt, ks, 2, pl, x.lane));
    const int crow = 16 * x.r + 4 * x.lg4;
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
        o.u[nt] = *reinterpret_cast<const f4*>(p.ws.Ut + (ch * kD + x.j0 + 16 * nt + x.li) * kChunk + crow);
    const float* Gc = p.ws.G + ch * kChunk;
    o.gv = *reinterpret_cast<const f4*>(Gc + crow);
    o.glast = Gc[kChunk - 1];
}

__device__ __forceinline__ void load_out_ops(const ChainCtx& x, int c, OutOps& o) {
    const PrefillParams& p = *x.p;
    const size_t ch = chain_ch(x, c);
    o.t0 = x.seq_lo + (c - x.c_begin) * kChunk;            // chunk c of the sequence (no table lookup)
    o.len = min(kChunk, x.seq_hi - o.t0);
    const uint16_t* Qf = p.ws.Qf + ((size_t)c * p.L.h_k + x.src) * kFragW;
    const uint16_t* Mf = p.ws.Mf + ch * kFragM;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) o.q[ks][pl] = *reinterpret_cast<const bf8*>(Qf + frag_at(x.r, ks, 4, pl, x.lane));
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) o.m[ks][pl] = *reinterpret_cast<const bf8*>(Mf + frag_at(x.r, ks, 2, pl, x.lane));
    o.gv = *reinterpret_cast<const f4*>(p.ws.G + ch * kChunk + 16 * x.r + 4 * x.lg4);
}

// State waves, one chunk: D = U - W S, S' = Gam_last S + K^T (exp(G_last - G) D).
// S[mt][nt]: rows 32r + 16mt + 4lg4 + i, columns 16nt + li of the slice.
__device__ __forceinline__ void state_step(const ChainCtx& x, const StateOps& o, f4 (&S)[2][kNT], uint16_t* S_f,
                                           uint16_t* D_f, uint16_t* Dg_f) {
    const int r = x.r, li = x.li, lg4 = x.lg4, lane = x.lane;
    // S into B fragments: state row i = 32r + 16mt + 4lg4 + e -> ks = r, q = 4mt + lg4
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) bfrag_put4(S_f, r, nt, 4 * mt + lg4, li, S[mt][nt]);
    lds_barrier();                                                    // (A) state slice visible

    // W S: the three split products and the column tiles accumulate separately (six
    // independent MFMA chains), and all B fragments of a k-step are read before its MFMAs.
    f4 ws[kNT][3];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
        for (int q = 0; q < 3; ++q) ws[nt][q] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        bf8 bh[kNT], bl[kNT];
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) {
            bh[nt] = *reinterpret_cast<const bf8*>(S_f + bfrag_at(ks, nt, 0, lane));
            bl[nt] = *reinterpret_cast<const bf8*>(S_f + bfrag_at(ks, nt, 1, lane));
        }
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) {
            ws[nt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.w[ks][0], bh[nt], ws[nt][0], 0, 0, 0);
            ws[nt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.w[ks][0], bl[nt], ws[nt][1], 0, 0, 0);
            ws[nt][2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.w[ks][1], bh[nt], ws[nt][2], 0, 0, 0);
        }
    }
    f4 d[kNT], dg[kNT];
    f4 eg;
#pragma unroll
    for (int i = 0; i < 4; ++i) eg[i] = expf(o.glast - o.gv[i]);
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            d[nt][i] = o.u[nt][i] - (ws[nt][0][i] + (ws[nt][1][i] + ws[nt][2][i]));
            dg[nt][i] = eg[i] * d[nt][i];
        }
    }
    // D, Dg into B fragments: token t = 16r + 4lg4 + e -> ks = r >> 1, q = 4 (r & 1) + lg4
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
        bfrag_put4(D_f, r >> 1, nt, 4 * (r & 1) + lg4, li, d[nt]);
        bfrag_put4(Dg_f, r >> 1, nt, 4 * (r & 1) + lg4, li, dg[nt]);
    }
    lds_barrier();                                                    // (B) D visible

    // S' = Gam_last S + K^T Dg: the state tile takes the hi*hi products; hi*lo and lo*hi
    // go to a second accumulator per tile, added at the end.
    const float gl = expf(o.glast);
    f4 sx[2][kNT];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) { S[mt][nt] *= gl; sx[mt][nt] = f4{0.f, 0.f, 0.f, 0.f}; }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        bf8 bh[kNT], bl[kNT];
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) {
            bh[nt] = *reinterpret_cast<const bf8*>(Dg_f + bfrag_at(ks, nt, 0, lane));
            bl[nt] = *reinterpret_cast<const bf8*>(Dg_f + bfrag_at(ks, nt, 1, lane));
        }
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < kNT; ++nt) {
                S[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.kt[mt][ks][0], bh[nt], S[mt][nt], 0, 0, 0);
                sx[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.kt[mt][ks][0], bl[nt], sx[mt][nt], 0, 0, 0);
                sx[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.kt[mt][ks][1], bh[nt], sx[mt][nt], 0, 0, 0);
            }
    }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) S[mt][nt] += sx[mt][nt];
}

// Output waves, one chunk: O = diag(Gam) Q S + M D for rows 16r..16r+15. OUT: bit 0 fp32 o,
// bit 1 bf16 o. Every store is issued (rows past the sequence end go to the sink), so the
// number of memory operations per chunk is fixed and the next chunk's operand loads never
// have to wait for this chunk's stores.
template <int OUT>
__device__ __forceinline__ void out_step(const ChainCtx& x, const OutOps& o, const uint16_t* S_f, const uint16_t* D_f) {
    const PrefillParams& p = *x.p;
    const int r = x.r, li = x.li, lg4 = x.lg4, lane = x.lane, crow = 16 * r + 4 * lg4;
    lds_barrier();                                                    // (A)
    f4 qs[kNT][3];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt)
#pragma unroll
        for (int q = 0; q < 3; ++q) qs[nt][q] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        bf8 bh[kNT], bl[kNT];
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) {
            bh[nt] = *reinterpret_cast<const bf8*>(S_f + bfrag_at(ks, nt, 0, lane));
            bl[nt] = *reinterpret_cast<const bf8*>(S_f + bfrag_at(ks, nt, 1, lane));
        }
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) {
            qs[nt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.q[ks][0], bh[nt], qs[nt][0], 0, 0, 0);
            qs[nt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.q[ks][0], bl[nt], qs[nt][1], 0, 0, 0);
            qs[nt][2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.q[ks][1], bh[nt], qs[nt][2], 0, 0, 0);
        }
    }
    lds_barrier();                                                    // (B)
    f4 eg;
#pragma unroll
    for (int i = 0; i < 4; ++i) eg[i] = expf(o.gv[i]);
    f4 md[kNT][2];
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) md[nt][0][i] = eg[i] * (qs[nt][0][i] + (qs[nt][1][i] + qs[nt][2][i]));
        md[nt][1] = f4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        bf8 bh[kNT], bl[kNT];
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) {
            bh[nt] = *reinterpret_cast<const bf8*>(D_f + bfrag_at(ks, nt, 0, lane));
            bl[nt] = *reinterpret_cast<const bf8*>(D_f + bfrag_at(ks, nt, 1, lane));
        }
#pragma unroll
        for (int nt = 0; nt < kNT; ++nt) {
            md[nt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.m[ks][0], bh[nt], md[nt][0], 0, 0, 0);
            md[nt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.m[ks][0], bl[nt], md[nt][1], 0, 0, 0);
            md[nt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.m[ks][1], bh[nt], md[nt][1], 0, 0, 0);
        }
    }
#pragma unroll
    for (int nt = 0; nt < kNT; ++nt) {
        const f4 ov = md[nt][0] + md[nt][1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = crow + i;
            const size_t oo = ((size_t)(o.t0 + t) * p.L.h_v + x.h) * kD + x.j0 + 16 * nt + li;
            const bool in = t < o.len;
            if constexpr ((OUT & 1) != 0) *(in ? p.o + oo : p.ws.sink + lane) = ov[i];
            if constexpr ((OUT & 2) != 0)
                *(in ? p.o_bf16 + oo : reinterpret_cast<uint16_t*>(p.ws.sink) + lane) = f32_to_bf16(ov[i]);
        }
    }
}

// As many stores as one out_step issues, all to the sink: issued once before the loop so
// that the memory operations in flight at the loop head are the same on entry as around the
// loop, and the compiler's wait for the next operands does not cover the last stores.
template <int OUT>
__device__ __forceinline__ void sink_stores(const PrefillParams& p, int lane) {
#pragma unroll
    for (int i = 0; i < kNT * 4; ++i) {            // distinct addresses: none of them is redundant
        if constexpr ((OUT & 1) != 0) p.ws.sink[i * kWave + lane] = 0.0f;
        if constexpr ((OUT & 2) != 0) reinterpret_cast<uint16_t*>(p.ws.sink + 8 * kWave)[i * kWave + lane] = 0;
    }
}

template <int OUT>
__global__ void __launch_bounds__(512) chain_kernel(const PrefillParams p) {
    __shared__ __align__(16) uint16_t S_f[4 * kNT * kBFrag];
    __shared__ __align__(16) uint16_t D_f[2 * kNT * kBFrag];
    __shared__ __align__(16) uint16_t Dg_f[2 * kNT * kBFrag];

    const Layer& L = p.L;
    // XCD-aware mapping: the 4 slices of one (sequence, head) pair share an XCD (and its L2).
    const int lin = blockIdx.x, xcd = lin & 7, k = lin >> 3;
    const int slice = k & (kSlices - 1);
    const int pair = (k / kSlices) * 8 + xcd;
    if (pair >= p.n_seq * L.h_v) return;
    const int s = pair / L.h_v, h = pair % L.h_v, src = src_of(L, h);
    const int c_begin = p.ws.chunk_off[s], c_end = p.ws.chunk_off[s + 1];
    if (c_begin >= c_end) return;
    const int tid = threadIdx.x, w = tid / kWave, lane = tid & (kWave - 1);

    ChainCtx x;
    x.p = &p;
    x.h = h;
    x.src = src;
    x.seq_lo = p.ws.seq_lo[s];
    x.seq_hi = p.ws.seq_lo[s + 1];
    x.c_begin = c_begin;
    x.j0 = slice * kSlice;
    x.r = w & 3;
    x.li = lane & 15;
    x.lg4 = lane >> 4;
    x.lane = lane;

    if (w < 4) {
        // State slice: rows 32 r + 16 mt + 4 lg4 + i (k index), columns j0 + 16 nt + li (v
        // index); the state is stored column by column ([d_v][d_k]), so the 4 rows are a float4.
        float* st = p.state + ((size_t)s * L.h_v + h) * kD * kD;
        f4 S[2][kNT];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < kNT; ++nt)
                S[mt][nt] = *reinterpret_cast<const f4*>(st + (size_t)(x.j0 + 16 * nt + x.li) * kD + 32 * x.r + 16 * mt + 4 * x.lg4);
        __builtin_amdgcn_s_waitcnt(0);             // the state is in registers before the loop
        // Prefetches are unconditional (past the last chunk they re-read it): a load that is
        // skipped on one path forces the compiler to wait for every load in flight.
        StateOps A, B;
        load_state_ops(x, c_begin, A);
        int c = c_begin;
        for (; c + 1 < c_end; c += 2) {
            load_state_ops(x, c + 1, B);
            state_step(x, A, S, S_f, D_f, Dg_f);
            __builtin_amdgcn_sched_barrier(0);     // keep A's reload after A's last use
            load_state_ops(x, min(c + 2, c_end - 1), A);
            state_step(x, B, S, S_f, D_f, Dg_f);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c < c_end) state_step(x, A, S, S_f, D_f, Dg_f);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < kNT; ++nt)
                *reinterpret_cast<f4*>(st + (size_t)(x.j0 + 16 * nt + x.li) * kD + 32 * x.r + 16 * mt + 4 * x.lg4) = S[mt][nt];
    } else {
        OutOps A, B;                               // same schedule as the state waves
        load_out_ops(x, c_begin, A);
        sink_stores<OUT>(p, lane);
        int c = c_begin;
        for (; c + 1 < c_end; c += 2) {
            load_out_ops(x, c + 1, B);
            out_step<OUT>(x, A, S_f, D_f);
            __builtin_amdgcn_sched_barrier(0);
            load_out_ops(x, min(c + 2, c_end - 1), A);
            out_step<OUT>(x, B, S_f, D_f);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c < c_end) out_step<OUT>(x, A, S_f, D_f);
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

}  // namespace
}  // namespace ixg

extern "C" hipError_t ix_gdn_check_cfg_(const ix_gdn_cfg* c);

extern "C" hipError_t ix_gdn_check_gate_(const ix_gdn_out_gate* g);

extern "C" size_t ix_gdn_prefill_workspace_size(const ix_gdn_cfg* cfg, int n_seq, int total_T) {
    if (ix_gdn_check_cfg_(cfg) != hipSuccess || n_seq <= 0 || total_T < 0) return 0;
    size_t off[ixg::kWsSections];
    return ixg::ws_layout(cfg, n_seq, total_T, off);
}

// The gated prefill's workspace: the prefill's, then [total_T][h_v][d_v] fp32 outputs.
extern "C" size_t ix_gdn_prefill_gated_workspace_size(const ix_gdn_cfg* cfg, int n_seq, int total_T) {
    const size_t base = ix_gdn_prefill_workspace_size(cfg, n_seq, total_T);
    if (!base) return 0;
    return base + (((size_t)total_T * cfg->h_v * ixg::kD * sizeof(float) + 255) & ~(size_t)255);
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
    size_t off[kWsSections];
    const size_t need = ws_layout(cfg, n_seq, total_T, off);
    if (workspace_bytes < (gate ? ix_gdn_prefill_gated_workspace_size(cfg, n_seq, total_T) : need))
        return hipErrorInvalidValue;
    const long long NC = (total_T + kChunk - 1) / kChunk + (long long)n_seq;
    const long long pairs = (long long)n_seq * cfg->h_v;
    if (NC > 0x7fffffffLL || pairs * kSlices > 0x7fffffffLL) return hipErrorInvalidValue;
    const long long rows = (long long)total_T * cfg->h_v;
    if (gate && (rows + 3) / 4 > 0x7fffffffLL) return hipErrorInvalidValue;

    PrefillParams p;
    p.L = make_layer(cfg, conv_w, A_log, dt_bias);
    p.ws = ws_bind(static_cast<char*>(workspace), off);
    p.cu = cu_seqlens; p.x = x; p.conv_state = conv_state; p.a = a; p.b = b;
    p.state = state; p.o = o; p.o_bf16 = o_bf16;
    p.n_seq = n_seq; p.T = total_T; p.NC = (int)NC;
    if (gate && !o) p.o = reinterpret_cast<float*>(static_cast<char*>(workspace) + need);   // the norm's input

    hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, p);
    const dim3 kgrid((unsigned)NC, (unsigned)cfg->h_k);
    switch (cfg->d_conv) {
        case 2: hipLaunchKernelGGL(chunk_kernel<2>, kgrid, dim3(kChunkThreads), 0, s, p); break;
        case 3: hipLaunchKernelGGL(chunk_kernel<3>, kgrid, dim3(kChunkThreads), 0, s, p); break;
        default: hipLaunchKernelGGL(chunk_kernel<4>, kgrid, dim3(kChunkThreads), 0, s, p); break;
    }
    // after the chunk kernel, which reads the old history at sequence starts
    const size_t nch = (size_t)n_seq * p.L.C;
    hipLaunchKernelGGL(commit_kernel, dim3((unsigned)((nch + 255) / 256)), dim3(256), 0, s, p);
    const long long groups = (pairs + 7) / 8;
    const dim3 cgrid((unsigned)(groups * 8 * kSlices));
    switch ((p.o ? 1 : 0) | (p.o_bf16 ? 2 : 0)) {
        case 0: hipLaunchKernelGGL(chain_kernel<0>, cgrid, dim3(512), 0, s, p); break;
        case 1: hipLaunchKernelGGL(chain_kernel<1>, cgrid, dim3(512), 0, s, p); break;
        case 2: hipLaunchKernelGGL(chain_kernel<2>, cgrid, dim3(512), 0, s, p); break;
        default: hipLaunchKernelGGL(chain_kernel<3>, cgrid, dim3(512), 0, s, p); break;
    }
    if (gate)
        hipLaunchKernelGGL(out_gate_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, p.o,
                           make_out_gate(gate), rows);
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
