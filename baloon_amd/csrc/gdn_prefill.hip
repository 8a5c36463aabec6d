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
//                  the chunk table (sequence and first token of each chunk); not launched
//                  for a single sequence, whose geometry the kernels derive from cu[0], cu[1]
//   qk_kernel      per (chunk, q/k head): conv (history from conv_state at sequence starts)
//                  and L2 norms of q and k; K K^T and Q K^T (lower block triangle) once for
//                  all the v heads mapped to the q/k head, stored raw; K^T and Q written as
//                  split-bf16 MFMA fragments
//   v_kernel       per (chunk, v head): decay factors and beta, v rows, A and M from the raw
//                  products, T = (I + A)^-1 (diagonal blocks by substitution, the rest by
//                  block forward substitution), U = T diag(beta) V by block forward
//                  substitution and W = T diag(beta Gam) K; the chain's operands W
//                  (negated, so the chain's D accumulates from U) and M as split-bf16
//                  fragments, U^T in fp32
//   chain_kernel   per (sequence, v head, 16-column state strip): walks the chunks in order.
//                  One wave carries the strip in MFMA accumulators with no barrier on its
//                  data path; four waves compute the outputs from the S and D it hands over;
//                  two waves copy the next chunk's W and the current chunk's K^T into LDS
//                  with direct loads and warm L2 ahead; before the first chunk the K^T
//                  wave writes the new rolling conv history of the pair's share of channels.
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
struct Ws {
    int32_t* seq_lo;     // [n_seq + 1] clamped token offsets
    int32_t* chunk_off;  // [n_seq + 1] first chunk of each sequence; chunk_off[n_seq] = #chunks
    int4* chunk_rec;     // [NC] {sequence, first token, sequence start, sequence end}
    uint16_t* Wf;        // [NC][h_v] -W (64 x 128) as split-bf16 A fragments
    float* Ut;           // [NC][h_v][128][64]  U transposed (column j of U is row j)
    uint16_t* Mf;        // [NC][h_v] M (64 x 64) as split-bf16 A fragments
    float* G;            // [NC][h_v][2][64] decay factors exp(G_last - G_t), then exp(G_t), of the
                         // inclusive cumulative log decay G (padded rows repeat the last)
    uint16_t* Ktf;       // [NC][h_k] K^T (128 x 64, zero beyond the chunk length) as fragments
    uint16_t* Qf;        // [NC][h_k] Q (64 x 128, zero beyond the chunk length) as fragments
    v4* raw;             // [NC][h_k][4][3][2][64] raw K K^T, (Q K^T)^T triangle blocks (accumulator layout)
};
constexpr int kWsSections = 10;

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Byte offsets of every workspace section for (n_seq, T); returns the total size.
inline size_t ws_layout(const ix_gdn_cfg* c, int n_seq, int T, size_t off[kWsSections]) {
    const size_t NC = (size_t)(T + kChunk - 1) / kChunk + (size_t)n_seq;
    const size_t sz[kWsSections] = {
        sizeof(int32_t) * (n_seq + 1), sizeof(int32_t) * (n_seq + 1), sizeof(int4) * NC,
        sizeof(float) * NC * c->h_v * kChunk * kD, sizeof(float) * NC * c->h_v * kChunk * kD,
        sizeof(float) * NC * c->h_v * kChunk * kChunk, sizeof(float) * NC * c->h_v * 2 * kChunk,
        sizeof(float) * NC * c->h_k * kD * kChunk, sizeof(float) * NC * c->h_k * kChunk * kD,
        sizeof(v4) * NC * c->h_k * 4 * 3 * 2 * kWave,
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
    w.Wf = reinterpret_cast<uint16_t*>(base + off[3]);
    w.Ut = reinterpret_cast<float*>(base + off[4]);
    w.Mf = reinterpret_cast<uint16_t*>(base + off[5]);
    w.G = reinterpret_cast<float*>(base + off[6]);
    w.Ktf = reinterpret_cast<uint16_t*>(base + off[7]);
    w.Qf = reinterpret_cast<uint16_t*>(base + off[8]);
    w.raw = reinterpret_cast<v4*>(base + off[9]);
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
    int single;                 // n_seq == 1: no plan pass; the geometry comes from cu[0], cu[1]
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
    // the chunk table: chunk c belongs to the last sequence s with chunk_off[s] <= c
    const int nc = run;
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
// commit: the rolling conv history of channel ch after sequence s, tokens lo .. lo+len-1
// (len > 0); run by the chain kernel, which starts after the chunk kernel has read the old
// history
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void commit_history(const PrefillParams& p, int ch, int lo, int len, int s) {
    const Layer& L = p.L;
    uint16_t* st = p.conv_state + ((size_t)s * L.C + ch) * (L.dc - 1);
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
__device__ __forceinline__ float qk_f32(const uint8_t* planes, int t, int ch) {
    const int o = qk_off(t, ch);
    return bf16_to_f32(*reinterpret_cast<const uint16_t*>(planes + o)) +
           bf16_to_f32(*reinterpret_cast<const uint16_t*>(planes + kQKPlane + o));
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
                                        float* A_s, uint16_t* Mf, int w, int lane) {
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
    // 1 (a diagonal block, right neighbour zero); waves 2 and 3 write the zero fragments of
    // block rows 0 and 1 at k-step 1.
    int br, bc;
    tri_block(w, br, bc);
    float x[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) { x[r] = mv[0][r]; x[4 + r] = mv[1][r]; }
    store_frag(Mf, br, bc >> 1, 2, lane, x);
    if (w < 2) {
        tri_block(w + 8, br, bc);
    } else {
        br = w - 2;
        bc = 2;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) { x[r] = mv[2][r]; x[4 + r] = 0.0f; }
    store_frag(Mf, br, bc >> 1, 2, lane, x);
}

// The chunk-local work runs as two kernels, so that each holds a fraction of the registers and
// LDS of a single one and two workgroups share a CU (one hides the other's load latency and
// barriers):
//   qk_kernel (chunk, q/k head): q and k rows (conv, L2 norm, q scale) as split-bf16 planes in
//     LDS; the lower block triangle of K K^T and Q K^T on split-bf16 MFMA, stored raw in the
//     accumulator layout for the v kernel; K^T and Q as the chain's fragments.
//   v_kernel (chunk, v head): decay scan and beta; v rows (conv); A and M from the raw
//     products; M fragments; T = (I + A)^-1 by a blocked inverse; U = T diag(beta) V and
//     W = T diag(beta Gam) K on split-bf16 MFMA (K from the K^T fragments); U^T and -W
//     fragments for the chain.
// Every barrier orders LDS only, so no wave waits for its own global stores.

// The v kernel's unit (chunk, v head) of 1-D workgroup id. Workgroups are dispatched to the
// 8 XCDs round robin (id % 8), so ids are first made XCD-major (XCD x runs units
// x * N/8 .. (x+1) * N/8 - 1, in order), and the units walk the v heads of one q/k head one
// after the other within a chunk: the heads that share a q/k head read the same K^T fragments
// and raw triangle blocks, and run back to back on one XCD, where the second reads hit L2.
__device__ __forceinline__ void v_unit(const Layer& L, int NC, int id, int& c, int& h) {
    const long long N = (long long)NC * L.h_v, per = N / 8;
    const long long u = id < per * 8 ? (long long)(id % 8) * per + id / 8 : id;
    c = (int)(u / L.h_v);
    const int k = (int)(u % L.h_v);
    if (L.head_map != IX_GDN_HEAD_MOD) {
        h = k;                                   // h / per_src: a q/k head's v heads are adjacent
        return;
    }
    // h mod h_k: q/k head s has v heads s, s + h_k, ...; the first h_v mod h_k heads have
    // one more than the others.
    const int lo = L.h_v / L.h_k, r = L.h_v % L.h_k, hi = lo + (r ? 1 : 0);
    int s, m;
    if (k < r * hi) {
        s = k / hi;
        m = k % hi;
    } else {
        const int k2 = k - r * hi;
        s = r + k2 / lo;
        m = k2 % lo;
    }
    h = s + m * L.h_k;
}

// Raw triangle products: per (chunk, q/k head), wave w (0..3) of the triangle and its block
// slot j (0..2, block i = w + 4 j), the K K^T then the transposed Q K^T accumulator (K of
// block bc times Q of block br, so that it lands in M's fragment layout), one 16-byte v4 per
// lane: [NC][h_k][4][3][2][64] v4.
__device__ __forceinline__ size_t raw_at(size_t cs, int w, int j, int kind, int lane) {
    return ((((cs * 4 + w) * 3 + j) * 2 + kind) * kWave + lane);
}

template <int DC>
__global__ void __launch_bounds__(kChunkThreads) qk_kernel(const PrefillParams p) {
    __shared__ __align__(16) uint8_t planes[4 * kQKPlane];     // k hi, k lo, q hi, q lo
    uint8_t* Kp = planes;
    uint8_t* Qp = planes + 2 * kQKPlane;

    ChunkGeo g;
    const int c = blockIdx.x;
    if (!chunk_geo(p, c, g)) return;
    const Layer& L = p.L;
    const int src = blockIdx.y;
    if (mapped_count(L, src) == 0) return;                     // no v head reads this q/k head
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int li = lane & 15, lg4 = lane >> 4, c2 = 2 * lane;
    const size_t cs = (size_t)c * L.h_k + src;
    const int tb = kConvTok * (w & 3), nt = min(max(g.len - tb, 0), kConvTok);   // this wave's rows

    // q rows (waves 0-3) and k rows (waves 4-7), 16 tokens per wave: lane l carries channels
    // 2l, 2l+1, so every x access of a wave is a 256-byte row segment and each row's norm is
    // one wave sum. Rows past the chunk end are zero.
    const bool isk = w >= 4;
    {
        ConvIn<DC> in;
        conv_load<DC>(p, g, g.lo, isk ? k_channel(L, src, c2) : q_channel(L, src, c2), tb, nt, in);
        float y0[kConvTok], y1[kConvTok];
        conv_run<DC>(L, in, y0, y1);
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

    if (w < 4) {
        // Raw K K^T and (Q K^T)^T of this wave's triangle blocks (16x16x32 split-bf16 MFMA,
        // operands straight from the planes: lane (li, lg4) supplies channels
        // 32 ks + 8 lg4 .. +7 of token row li for both operands), then stored. The A and B
        // register layouts are mirror images, so swapping the operands of Q K^T gives its
        // transpose.
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const int i = w + 4 * j;
            if (i >= 10) continue;
            v4 kk = {0.f, 0.f, 0.f, 0.f}, qk = kk;
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
                kk = mfma_bf16(akh, bkh, kk);
                qk = mfma_bf16(bkh, aqh, qk);
                kk = mfma_bf16(akh, bkl, kk);
                qk = mfma_bf16(bkl, aqh, qk);
                kk = mfma_bf16(akl, bkh, kk);
                qk = mfma_bf16(bkh, aql, qk);
            }
            p.ws.raw[raw_at(cs, w, j, 0, lane)] = kk;
            p.ws.raw[raw_at(cs, w, j, 1, lane)] = qk;
        }
    } else {
        // K^T (rows i, k = token t: 8 x 2 fragments) and Q (rows t, k = i: 4 x 4 fragments)
        // from the planes into split fragments, k in accumulator row order (kperm).
        const int t4 = tid - 4 * kWave;
        uint16_t* Ktf = p.ws.Ktf + cs * kFragKt;
        // K^T with the transposing LDS read (ds_read_b64_tr_b16): within each 16-lane group,
        // lane j receives element j & 3 of the 8-byte reads of lanes (j >> 2) + 4 e, e = 0..3.
        // Lane i of lane group g reads channels 16 m + 4 (i & 3) .. +3 of token
        // 32 ks + 4 g + (i >> 2) (then of the token 16 later), so it receives channel 16 m + i
        // at tokens 32 ks + 4 g + e (+ 16): entries e (4 + e) of its kperm fragment chunk.
        // Each wave takes whole fragments (m, ks), f = 2 m + ks = w - 4, w, w + 4, w + 8.
        const int ip = lane & 15, lgr = lane >> 4;
        const lds_u8* K3 = (const lds_u8*)Kp;
        for (int f = w - 4; f < 8 * 2; f += 4) {
            const int m = f >> 1, ks = f & 1;
            const int t0 = 32 * ks + 4 * lgr + (ip >> 2), c0 = 16 * m + 4 * (ip & 3);
            const int oa = qk_off(t0, c0), ob = qk_off(t0 + 16, c0);
            const uint2 ha = lds_tr16(K3 + oa), hb = lds_tr16(K3 + ob);
            const uint2 la = lds_tr16(K3 + kQKPlane + oa), lb = lds_tr16(K3 + kQKPlane + ob);
            *reinterpret_cast<u4x*>(Ktf + frag_at(m, ks, 2, 0, lane)) = u4x{ha.x, ha.y, hb.x, hb.y};
            *reinterpret_cast<u4x*>(Ktf + frag_at(m, ks, 2, 1, lane)) = u4x{la.x, la.y, lb.x, lb.y};
        }
        uint16_t* Qf = p.ws.Qf + cs * kFragW;
        for (int u = t4; u < 4 * 4 * kWave; u += 4 * kWave) {
            const int ln = u & (kWave - 1), f = u / kWave, m = f >> 2, ks = f & 3;
            const int row = 16 * m + (ln & 15), k0 = 32 * ks + 4 * (ln >> 4);      // kperm halves
            const int oa = qk_off(row, k0), ob = qk_off(row, k0 + 16);
            const uint2 ah = *reinterpret_cast<const uint2*>(Qp + oa), bh = *reinterpret_cast<const uint2*>(Qp + ob);
            const uint2 al = *reinterpret_cast<const uint2*>(Qp + kQKPlane + oa);
            const uint2 bl = *reinterpret_cast<const uint2*>(Qp + kQKPlane + ob);
            *reinterpret_cast<u4x*>(Qf + frag_at(m, ks, 4, 0, ln)) = u4x{ah.x, ah.y, bh.x, bh.y};
            *reinterpret_cast<u4x*>(Qf + frag_at(m, ks, 4, 1, ln)) = u4x{al.x, al.y, bl.x, bl.y};
        }
    }
}

// v_kernel: grid (NC, h_v), 512 threads; workgroup = (chunk, v head). Phases: decay scan and
// beta (wave 0, lane = token) and the raw products (waves 1-3 and 0) while waves 4-7 load and
// compute the v rows | A (to LDS) and M (to its fragments) (waves 0-3) | the four 16 x 16
// diagonal blocks of T by substitution (wave 0) | the blocks of T below them by forward
// substitution on the identity's block columns (waves 0-2) | U = T diag(beta) V (U^T stored
// from the MFMA layout) and W^T = K^T diag(beta Gam) T^T, whose accumulators are the chain's
// -W fragments as they stand, stored from registers, split evenly over the eight waves.
// T shares its LDS array with A, which keeps the workgroup at 51 KiB of LDS and 78 VGPRs:
// three workgroups per CU.
template <int DC>
__global__ void __launch_bounds__(kChunkThreads, 6) v_kernel(const PrefillParams p) {
    __shared__ __align__(16) float lds[kChunk * kKS + kChunk * kTS];
    float (*V_s)[kKS] = reinterpret_cast<float (*)[kKS]>(lds);        // v rows
    float* A_s = lds + kChunk * kKS;                                   // [64][kTS]
    float* T_s = A_s;                  // T over A: diagonal blocks in place, the others mirrored
    __shared__ __align__(16) float G_s[kChunk], B_s[kChunk], BG_s[kChunk];

    ChunkGeo g;
    const Layer& L = p.L;
    int c, h;
    v_unit(L, p.NC, blockIdx.x, c, h);
    if (!chunk_geo(p, c, g)) return;
    const int src = src_of(L, h);
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int li = lane & 15, lg4 = lane >> 4, c2 = 2 * lane;
    const size_t ch = (size_t)c * L.h_v + h, cs = (size_t)c * L.h_k + src;
    const int tb = kConvTok * (w & 3), nt = min(max(g.len - tb, 0), kConvTok);

    v4 kk[3], qk[3];
    if (w < 4) {
        uint16_t ra = 0, rb = 0;
        if (w == 0 && lane < g.len) {
            const size_t ab = (size_t)(g.t0 + lane) * L.h_v + h;
            ra = p.a[ab];
            rb = p.b[ab];
        }
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            kk[j] = v4{0.f, 0.f, 0.f, 0.f};
            qk[j] = kk[j];
            if (w + 4 * j < 10) {
                kk[j] = p.ws.raw[raw_at(cs, w, j, 0, lane)];
                qk[j] = p.ws.raw[raw_at(cs, w, j, 1, lane)];
            }
        }
        if (w == 0) {
            // Inclusive scan of the log decay over the chunk's tokens, beta, and the decay
            // factors the chain reads: exp(G_last - G_t), then exp(G_t).
            const bool ok = lane < g.len;
            float lgt = ok ? log_gate(L, h, bf16_to_f32(ra)) : 0.0f;
#pragma unroll
            for (int off = 1; off < kWave; off <<= 1) {
                const float o = __shfl_up(lgt, off, kWave);
                if (lane >= off) lgt += o;
            }
            const float bt = ok ? sigmoid_f(bf16_to_f32(rb)) : 0.0f;
            G_s[lane] = lgt;
            B_s[lane] = bt;
            BG_s[lane] = bt * expf(lgt);
            const float glast = __shfl(lgt, kChunk - 1, kWave);
            float* E = p.ws.G + ch * 2 * kChunk;
            E[lane] = expf(glast - lgt);
            E[kChunk + lane] = expf(lgt);
        }
    } else {
        // v rows of the head, 16 tokens per wave, zero past the chunk end.
        ConvIn<DC> vin;
        conv_load<DC>(p, g, g.lo, v_channel(L, h, c2), tb, nt, vin);
        float y0[kConvTok], y1[kConvTok];
        conv_run<DC>(L, vin, y0, y1);
#pragma unroll
        for (int t = 0; t < kConvTok; ++t)
            *reinterpret_cast<float2*>(&V_s[tb + t][c2]) = t < nt ? float2{y0[t], y1[t]} : float2{0.0f, 0.0f};
    }
    lds_barrier();
    if (w < 4) am_head(kk, qk, G_s, B_s, A_s, p.ws.Mf + ch * kFragM, w, lane);
    lds_barrier();

    // Wave 0 inverts the four unit lower-triangular diagonal blocks of I + A (lane = 16 b +
    // column c).
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
    }
    lds_barrier();
    // T below the diagonal blocks: wave j (0..2) runs column block j by forward substitution
    // (t_column), split-bf16 products on the 16x16x16 MFMA.
    if (w == 0) t_column<0>(A_s, T_s, lane);
    else if (w == 1) t_column<1>(A_s, T_s, lane);
    else if (w == 2) t_column<2>(A_s, T_s, lane);
    lds_barrier();

    // K^T fragments of row tiles 2 (w & 3) and 2 (w & 3) + 1 (the A operand of W^T below),
    // loaded here, so that the U product below hides their latency: held from the first
    // barrier on, they kept 32 more registers live through the inverse (90 VGPRs, two
    // workgroups per CU instead of three).
    const int kw = w & 3;
    bf8 kt[2][2][2];
    {
        const uint16_t* Ktf = p.ws.Ktf + cs * kFragKt;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int pl = 0; pl < 2; ++pl)
                    kt[t][ks][pl] = *reinterpret_cast<const bf8*>(Ktf + frag_at(2 * kw + t, ks, 2, pl, lane));
    }
    // U = (T diag beta) V and W = (T diag beta Gam) K on split-bf16 MFMA (16x16x32), every
    // wave taking a share of both of the same size. The k index (token s) runs in
    // kperm order, the order of the K^T fragments: lane (li, lg4) of k-step ks holds tokens
    // 32 ks + 4 lg4 .. +3 (the 16-token block 2 ks) and 32 ks + 16 + 4 lg4 .. +3 (block
    // 2 ks + 1). T[t][s] = 0 for s > t: tile mt needs the k-steps up to mt / 2, and the blocks
    // of T above the block diagonal (never written) are read as zeros.
    // Row tile mt of diag(sc) T^T as an MFMA operand: lane (li, lg4) holds sc_s T[16 mt + li][s]
    // at the tokens s of k-step ks (zero above the diagonal blocks), split.
    auto t_frag = [&](const float* sc, int mt, int ks, bf8& h, bf8& l) {
        const int s0 = 32 * ks + 4 * lg4;
        const v4 sc0 = *reinterpret_cast<const v4*>(sc + s0), sc1 = *reinterpret_cast<const v4*>(sc + s0 + 16);
        // T[16 mt + li][s] of blocks J = 2 ks, 2 ks + 1 (mirrored storage; the reads of blocks
        // above the diagonal land in A and are discarded below).
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
    };
    {
        // U: T diag(beta) as the A operand, the V columns 16 w .. 16 w + 15 as the B operand;
        // the accumulator of token tile mt holds U[16 mt + 4 lg4 + r][col], stored as U^T rows.
        const int col = 16 * w + li;
        v4 uacc[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) uacc[mt] = v4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int s0 = 32 * ks + 4 * lg4;
            float bv[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                bv[e] = V_s[s0 + e][col];
                bv[e + 4] = V_s[s0 + 16 + e][col];
            }
            bf8 bh, bl;
            split8(bv, bh, bl);
#pragma unroll
            for (int mt = 2 * ks; mt < 4; ++mt) {
                bf8 ah, al;
                t_frag(B_s, mt, ks, ah, al);
                uacc[mt] = mfma_bf16(ah, bh, uacc[mt]);
                uacc[mt] = mfma_bf16(ah, bl, uacc[mt]);
                uacc[mt] = mfma_bf16(al, bh, uacc[mt]);
            }
        }
        float* Ut = p.ws.Ut + ch * kD * kChunk;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
            *reinterpret_cast<v4*>(Ut + (size_t)col * kChunk + 16 * mt + 4 * lg4) = uacc[mt];
    }
    {
        // W^T = K^T diag(beta Gam) T^T, wave w taking W^T row tiles 2 kw, 2 kw + 1 (k-step kw of
        // the chain's W fragments) for token tiles 0 and 3 (waves 0-3) or 1 and 2 (waves 4-7),
        // three (token tile, k-step) pairs each: the K^T fragments
        // as the A operand and diag(beta Gam) T^T as the B operand, so the accumulator of (row
        // tile 2 kw + t, token tile mt) holds W[16 mt + li][32 kw + 16 t + 4 lg4 + r], r = 0..3:
        // entries 4 t + r of lane (li, lg4) of the chain's fragment (mt, kw) of -W, which the
        // wave then stores whole (negated, split) straight from the accumulators.
        v4 wacc[2][2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 2; ++j) wacc[t][j] = v4{0.f, 0.f, 0.f, 0.f};
        const int mts[2] = {w < 4 ? 0 : 1, w < 4 ? 3 : 2};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (2 * ks > mts[j]) continue;                  // T is zero there (wave-uniform)
                bf8 bh, bl;
                t_frag(BG_s, mts[j], ks, bh, bl);
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    wacc[t][j] = mfma_bf16(kt[t][ks][0], bh, wacc[t][j]);
                    wacc[t][j] = mfma_bf16(kt[t][ks][0], bl, wacc[t][j]);
                    wacc[t][j] = mfma_bf16(kt[t][ks][1], bh, wacc[t][j]);
                }
            }
        }
        uint16_t* Wf = p.ws.Wf + ch * kFragW;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float x[8];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                x[r] = -wacc[0][j][r];
                x[4 + r] = -wacc[1][j][r];
            }
            store_frag(Wf, mts[j], kw, 4, lane, x);
        }
    }
}
// ---------------------------------------------------------------------------------------
// chain: one workgroup per (sequence, v head, 16-column state strip), 7 waves
// ---------------------------------------------------------------------------------------
// Columns of the state are independent, so a head's chain splits into 8 strips of 16
// columns, and each strip's workgroup walks its sequence's chunks in order. Roles:
//   wave 0 (state) carries the strip S (128 x 16) in four-register MFMA accumulators and
//     per chunk computes
//       D  = U - W S                                   (64 x 16; W from LDS)
//       S' = Gam_last S + K^T Dg,  Dg = diag(exp(G_last - G)) D     (K^T from LDS)
//     The chunk kernel stores W, K^T, Q and M with their k index in accumulator row order
//     (kperm), so the accumulator tiles of S and D, split to bf16 hi/lo, are the next
//     product's B operands as they stand: the state path has no LDS round trip and never
//     waits at a barrier for data. It hands the split S and D of every chunk to the output
//     waves through a double-buffered LDS slot.
//   waves 1-4 (output): wave 1 + r computes rows 16 r .. 16 r + 15 of
//       O = diag(Gam) Q S + M D                        (Q, M from global, one chunk ahead)
//     from the S and D the state wave handed over.
//   waves 5, 6 (copy) move the next chunk's W and this chunk's K^T fragments (32 KiB each,
//     one wave each, so twice the loads are in flight) into LDS with direct global-to-LDS
//     loads, and wait for them before the barrier.
// The roles meet at one barrier per chunk. Between barriers c-1 and c the state wave
// finishes chunk c-1 (K^T from slot (c-1)&1) interleaved with the start of chunk c (W from
// slot c&1, hand-over slot c&1), the copy waves fill W slot (c+1)&1 and K^T slot c&1, and
// the output waves compute chunk c-1 from hand-over slot (c-1)&1. The state wave's code
// path issues no LDS DMA, so the compiler never makes it wait for the copies.
constexpr int kStrip = 16;                              // state columns per chain workgroup
constexpr int kStrips = kD / kStrip;                    // 8
constexpr int kChainWaves = 7;
constexpr int kPlane = kWave * 16;                      // bytes of one fragment plane
constexpr int kOpsBytes = 32 * kPlane;                  // W (4 x 4) or K^T (8 x 2) fragments, 2 planes
constexpr int kHandS = 8 * kPlane;                      // S: 4 k-steps x 2 planes
constexpr int kHandBytes = kHandS + 4 * kPlane;         // + D: 4 row tiles in fp32
constexpr int kChainSink = kPlane;                      // target of the L2 warm-up loads
constexpr int kChainLds = 4 * kOpsBytes + 2 * kHandBytes + kChainSink;   // 156,672 bytes
constexpr int kWarmAhead = 2;                           // chunks warmed ahead of their copy
constexpr int kWarmLoadsW = 9;                          // warm-up loads per chunk: W-copy wave
constexpr int kWarmLoadsK = 10;                         //                          K^T-copy wave

__device__ __forceinline__ bf8 lds_frag(const uint8_t* lds, int off, int lane) {
    return *reinterpret_cast<const bf8*>(lds + off + lane * 16);
}
__device__ __forceinline__ void lds_put(uint8_t* lds, int off, int lane, const bf8& v) {
    *reinterpret_cast<bf8*>(lds + off + lane * 16) = v;
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


__device__ __forceinline__ int chain_w_slot(int q) { return q * kOpsBytes; }
__device__ __forceinline__ int chain_k_slot(int q) { return (2 + q) * kOpsBytes; }
__device__ __forceinline__ int chain_h_slot(int q) { return 4 * kOpsBytes + q * kHandBytes; }

// State role: U of chunk c at this lane's rows 16 m + 4 lg4 + i (tokens), column j, the
// decay factors exp(G_last - G) at the same rows, and Gam_last = exp(G_last).
__device__ __forceinline__ void chain_load_ug(const PrefillParams& p, int c, int h, int j, int lg4, v4 (&u)[4],
                                              v4 (&e)[4], float& gam) {
    const size_t ch = (size_t)c * p.L.h_v + h;
    const float* Ut = p.ws.Ut + (ch * kD + j) * kChunk + 4 * lg4;
    const float* E = p.ws.G + ch * 2 * kChunk;
    gam = E[2 * kChunk - 1];
#pragma unroll
    for (int m = 0; m < 4; ++m) e[m] = *reinterpret_cast<const v4*>(E + 16 * m + 4 * lg4);
#pragma unroll
    for (int m = 0; m < 4; ++m) u[m] = *reinterpret_cast<const v4*>(Ut + 16 * m);
}

// Output role: Q and M fragments of row tile r of chunk c, and G at this lane's rows.
__device__ __forceinline__ void chain_load_qm(const PrefillParams& p, int c, int h, int src, int r, int lane,
                                              bf8 (&qf)[4][2], bf8 (&mf)[2][2], v4& g) {
    const size_t ch = (size_t)c * p.L.h_v + h;
    const uint16_t* Qf = p.ws.Qf + ((size_t)c * p.L.h_k + src) * kFragW;
    const uint16_t* Mf = p.ws.Mf + ch * kFragM;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) qf[ks][pl] = *reinterpret_cast<const bf8*>(Qf + frag_at(r, ks, 4, pl, lane));
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) mf[ks][pl] = *reinterpret_cast<const bf8*>(Mf + frag_at(r, ks, 2, pl, lane));
    g = *reinterpret_cast<const v4*>(p.ws.G + ch * 2 * kChunk + kChunk + 16 * r + 4 * (lane >> 4));   // exp(G_t)
}

// Copy role: the 32 one-KiB fragment planes of W (chunk c, v head h) or K^T (chunk c, q/k
// head src) into LDS at dst.
__device__ __forceinline__ void chain_copy(lds_u8* dst, const uint16_t* frags, int lane) {
    const uint8_t* g = reinterpret_cast<const uint8_t*>(frags) + lane * 16;
#pragma unroll
    for (int i = 0; i < 32; ++i) __builtin_amdgcn_global_load_lds(g + i * kPlane, dst + i * kPlane, 16, 0, 0);
}

// This lane's address in an LDS area at byte offset off, made opaque to the compiler: reads
// and writes at base + (a constant below 64 KiB) then use the instruction's immediate offset,
// where the folded address of an area above 64 KiB would cost an add per access.
__device__ __forceinline__ lds_u8* lane_base(uint8_t* lds, int off, int lane) {
    lds_u8* b = (lds_u8*)lds + off + lane * 16;
    __asm__ volatile("" : "+v"(b));
    return b;
}
// W fragments (row tiles m = 0..3, both planes) of k-step ks from the slot at wq (lane base).
__device__ __forceinline__ void chain_w_frags(const lds_u8* wq, int ks, bf8 (&f)[4][2]) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int o = (m * 4 + ks) * 2 * kPlane;
        f[m][0] = *(const __attribute__((address_space(3))) bf8*)(wq + o);
        f[m][1] = *(const __attribute__((address_space(3))) bf8*)(wq + o + kPlane);
    }
}
// K^T fragments (row tiles 4 g .. 4 g + 3, both planes) of k-step ks from the slot at kq.
__device__ __forceinline__ void chain_kt_frags(const lds_u8* kq, int ks, int g, bf8 (&f)[4][2]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int o = ((4 * g + j) * 2 + ks) * 2 * kPlane;
        f[j][0] = *(const __attribute__((address_space(3))) bf8*)(kq + o);
        f[j][1] = *(const __attribute__((address_space(3))) bf8*)(kq + o + kPlane);
    }
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

// State role (wave 0): the strip's whole chunk loop, S (128 x 16) in accumulators.
// Between barriers c-1 and c (c > c_begin) it finishes chunk c-1,
//     S <- Gam_{c-1} S + K^T Dg_{c-1}          (K^T from slot (c-1)&1; S arrives scaled)
// and runs chunk c:
//     S handed over (split), D = U - W S, D handed over, Dg = E D split, S *= Gam_c.
// W is stored negated, so the D accumulators start from U. The work is cut into regions
// of 12 MFMAs, each holding the VALU work (splits, scalings) that can overlap them. Three
// fragment groups (R0..R2) rotate through the K^T and W fragments, each refilled as soon
// as its last MFMA has issued.
__device__ __forceinline__ void chain_state_role(const PrefillParams& p, uint8_t* lds, int lane, int c_begin,
                                                 int c_end, int h, int j, int lg4, v4 (&S)[8]) {
    v4 U[4], E[4];
    float gam;
    bf8 dh[2], dl[2], sh[4], sl[4];
    v4 dg2, dg3;                       // Dg row tiles 2, 3, split at the start of part b
    bf8 R0[4][2], R1[4][2], R2[4][2];

    // Lane bases of the two W, K^T and hand-over slots.
    lds_u8* const wb[2] = {lane_base(lds, chain_w_slot(0), lane), lane_base(lds, chain_w_slot(1), lane)};
    lds_u8* const kb[2] = {lane_base(lds, chain_k_slot(0), lane), lane_base(lds, chain_k_slot(1), lane)};
    lds_u8* const hb[2] = {lane_base(lds, chain_h_slot(0), lane), lane_base(lds, chain_h_slot(1), lane)};
    typedef __attribute__((address_space(3))) bf8 lds_bf8;
    typedef __attribute__((address_space(3))) v4 lds_v4;
    auto put_s = [&](int q, int ks) {
        *(lds_bf8*)(hb[q] + (2 * ks) * kPlane) = sh[ks];
        *(lds_bf8*)(hb[q] + (2 * ks + 1) * kPlane) = sl[ks];
    };
    // Part b, row tiles 0-3 (K^T k-steps 0, 1 of slot qp in R0, R1); R2 and then R0 take
    // the row tiles 4-7.
    auto part_b_lo = [&](int qp) {
        chain_kt_frags(kb[qp], 0, 0, R0);
        chain_kt_frags(kb[qp], 1, 0, R1);
        split_tiles(dg2, dg3, dh[1], dl[1]);
        __builtin_amdgcn_sched_barrier(0);
        mfma4_split(R0, dh[0], dl[0], S);
        __builtin_amdgcn_sched_barrier(0);
        chain_kt_frags(kb[qp], 0, 1, R2);
        __builtin_amdgcn_sched_barrier(0);
        mfma4_split(R1, dh[1], dl[1], S);
        __builtin_amdgcn_sched_barrier(0);
        chain_kt_frags(kb[qp], 1, 1, R0);
        __builtin_amdgcn_sched_barrier(0);
    };
    // Part b, row tiles 4-7; with A, the split and hand-over of S row tiles 0-3 (final
    // after part_b_lo) and the reads of W k-steps 0, 1 (slot q) into R1, R2.
    auto part_b_hi = [&](int q, bool A) {
        mfma4_split(R2, dh[0], dl[0], S + 4);
        if (A) {
            split_tiles(S[0], S[1], sh[0], sl[0]);
            put_s(q, 0);
            chain_w_frags(wb[q], 0, R1);
        }
        __builtin_amdgcn_sched_barrier(0);
        mfma4_split(R0, dh[1], dl[1], S + 4);
        if (A) {
            split_tiles(S[2], S[3], sh[1], sl[1]);
            put_s(q, 1);
            chain_w_frags(wb[q], 1, R2);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // Part a from the W products on: D = U + (-W) S, hand-overs, Dg split, S *= Gam.
    auto part_a = [&](int q) {
        // W k-step 0 (R1); S row tiles 4, 5 split; S row tiles 0, 1 scaled; W k-step 2 -> R0.
        mfma4_split(R1, sh[0], sl[0], U);
        split_tiles(S[4], S[5], sh[2], sl[2]);
        put_s(q, 2);
        S[0] *= gam;
        S[1] *= gam;
        chain_w_frags(wb[q], 2, R0);
        __builtin_amdgcn_sched_barrier(0);
        // W k-step 1 (R2); S row tiles 6, 7 split; S row tiles 2, 3 scaled; W k-step 3 -> R1.
        mfma4_split(R2, sh[1], sl[1], U);
        split_tiles(S[6], S[7], sh[3], sl[3]);
        put_s(q, 3);
        S[2] *= gam;
        S[3] *= gam;
        chain_w_frags(wb[q], 3, R1);
        __builtin_amdgcn_sched_barrier(0);
        // W k-steps 2, 3 of row tiles 0, 1 (final after this); S row tiles 4-7 scaled.
        mfma2_split(R0, sh[2], sl[2], U);
        mfma2_split(R1, sh[3], sl[3], U);
#pragma unroll
        for (int mt = 4; mt < 8; ++mt) S[mt] *= gam;
        __builtin_amdgcn_sched_barrier(0);
        // W k-steps 2, 3 of row tiles 2, 3; D tiles 0, 1 handed over (fp32, the output
        // waves split it) and Dg tiles 0, 1 split.
        {
            bf8 a2[4][2], a3[4][2];
#pragma unroll
            for (int pl = 0; pl < 2; ++pl) {
                a2[0][pl] = R0[2][pl]; a2[1][pl] = R0[3][pl];
                a3[0][pl] = R1[2][pl]; a3[1][pl] = R1[3][pl];
            }
            mfma2_split(a2, sh[2], sl[2], U + 2);
            mfma2_split(a3, sh[3], sl[3], U + 2);
        }
#pragma unroll
        for (int m = 0; m < 2; ++m)
            *(lds_v4*)(hb[q] + kHandS + m * kPlane) = U[m];
        split_tiles(E[0] * U[0], E[1] * U[1], dh[0], dl[0]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int m = 2; m < 4; ++m)
            *(lds_v4*)(hb[q] + kHandS + m * kPlane) = U[m];
        dg2 = E[2] * U[2];
        dg3 = E[3] * U[3];
        __builtin_amdgcn_sched_barrier(0);
    };

    chain_load_ug(p, c_begin, h, j, lg4, U, E, gam);
    lds_barrier();                                            // W of the first chunk in LDS
    // Chunk c_begin: part a only.
    split_tiles(S[0], S[1], sh[0], sl[0]);
    put_s(0, 0);
    split_tiles(S[2], S[3], sh[1], sl[1]);
    put_s(0, 1);
    chain_w_frags(wb[0], 0, R1);
    chain_w_frags(wb[0], 1, R2);
    __builtin_amdgcn_sched_barrier(0);
    part_a(0);
    for (int c = c_begin + 1; c < c_end; ++c) {
        chain_load_ug(p, c, h, j, lg4, U, E, gam);
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();                                        // barrier c-1
        const int q = (c - c_begin) & 1;
        part_b_lo(q ^ 1);
        part_b_hi(q, true);
        part_a(q);
    }
    lds_barrier();                                            // barrier c_end-1
    part_b_lo((c_end - 1 - c_begin) & 1);
    part_b_hi(0, false);
}

struct ChainOut {
    bf8 qf[4][2], mf[2][2];
    v4 g;                 // exp(G_t) at this lane's rows
};

// Output role, one chunk: rows 16 r .. 16 r + 15 of O = diag(Gam) Q S + M D from hand-over
// slot q. Rows at or past len are not stored.
template <int OUT>
__device__ __forceinline__ void chain_out_step(const PrefillParams& p, const uint8_t* lds, int q, int lane, int r,
                                               const ChainOut& x, size_t o_base, int len) {
    lds_barrier();                                                // the chunk has been handed over
    bf8 sb[4][2], db[2][2];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) sb[ks][pl] = lds_frag(lds, chain_h_slot(q) + (2 * ks + pl) * kPlane, lane);
    v4 D[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) D[m] = *reinterpret_cast<const v4*>(lds + chain_h_slot(q) + kHandS + m * kPlane + lane * 16);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) split_tiles(D[2 * ks], D[2 * ks + 1], db[ks][0], db[ks][1]);
    v4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) o = mfma_split(x.qf[ks][0], x.qf[ks][1], sb[ks][0], sb[ks][1], o);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] *= x.g[i];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) o = mfma_split(x.mf[ks][0], x.mf[ks][1], db[ks][0], db[ks][1], o);
    const size_t row = (size_t)p.L.h_v * kD;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = 16 * r + 4 * (lane >> 4) + i;
        if (t < len) {
            const size_t oo = o_base + (size_t)t * row;
            if constexpr ((OUT & 1) != 0) p.o[oo] = o[i];
            if constexpr ((OUT & 2) != 0) p.o_bf16[oo] = f32_to_bf16(o[i]);
        }
    }
}

// Copy role: bring this strip's share of chunk c's operands into L2 ahead of their use (the
// 8 strips of a head share one XCD and its L2). Direct loads into a sink in LDS, so no
// register waits for them. The W-copy wave (kWarmLoadsW loads) takes an eighth of W and Q,
// and the decay factors; the K^T-copy wave (kWarmLoadsK loads) an eighth of K^T and M, and
// the strip's U rows.
__device__ __forceinline__ void chain_warm(const PrefillParams& p, lds_u8* sink, int c, int h, int src, int strip,
                                           int lane, bool w_wave) {
    const size_t ch = (size_t)c * p.L.h_v + h, cs = (size_t)c * p.L.h_k + src;
    if (w_wave) {
        const uint8_t* W = reinterpret_cast<const uint8_t*>(p.ws.Wf + ch * kFragW) + strip * 4 * kPlane + lane * 16;
        const uint8_t* Q = reinterpret_cast<const uint8_t*>(p.ws.Qf + cs * kFragW) + strip * 4 * kPlane + lane * 16;
        const uint8_t* G = reinterpret_cast<const uint8_t*>(p.ws.G + ch * 2 * kChunk) + (lane & 31) * 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_global_load_lds(W + i * kPlane, sink, 16, 0, 0);
            __builtin_amdgcn_global_load_lds(Q + i * kPlane, sink, 16, 0, 0);
        }
        __builtin_amdgcn_global_load_lds(G, sink, 16, 0, 0);
    } else {
        const uint8_t* K = reinterpret_cast<const uint8_t*>(p.ws.Ktf + cs * kFragKt) + strip * 4 * kPlane + lane * 16;
        const uint8_t* M = reinterpret_cast<const uint8_t*>(p.ws.Mf + ch * kFragM) + strip * 2 * kPlane + lane * 16;
        const uint8_t* U = reinterpret_cast<const uint8_t*>(p.ws.Ut + (ch * kD + strip * kStrip) * kChunk) + lane * 16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_global_load_lds(K + i * kPlane, sink, 16, 0, 0);
            __builtin_amdgcn_global_load_lds(U + i * kPlane, sink, 16, 0, 0);
        }
        __builtin_amdgcn_global_load_lds(M, sink, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(M + kPlane, sink, 16, 0, 0);
    }
}

// s_waitcnt that waits until at most N vector memory operations are outstanding (gfx9
// encoding: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left at their maximum).
// The field layout is gfx9-family (gfx950 here); another target would need its own encoding.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "wait_vmcnt encodes gfx950 s_waitcnt fields"
#endif
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int OUT>
__global__ void __launch_bounds__(kChainWaves * kWave) chain_kernel(const PrefillParams p) {
    __shared__ __align__(16) uint8_t lds[kChainLds];

    const Layer& L = p.L;
    // XCD-aware mapping: the 8 strips of one (sequence, head) pair share an XCD, so its L2
    // serves the pair's chunk operands to all of them.
    const int lin = blockIdx.x, xcd = lin & 7, k = lin >> 3;
    const int strip = k & (kStrips - 1);
    const int pair = (k / kStrips) * 8 + xcd;
    if (pair >= p.n_seq * L.h_v) return;
    const int s = pair / L.h_v, h = pair % L.h_v, src = src_of(L, h);
    int seq_lo, seq_hi;
    seq_bounds(p, s, seq_lo, seq_hi);
    const int c_begin = p.single ? 0 : p.ws.chunk_off[s];
    const int c_end = p.single ? (seq_hi - seq_lo + kChunk - 1) / kChunk : p.ws.chunk_off[s + 1];
    if (c_begin >= c_end) return;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x & (kWave - 1), li = lane & 15, lg4 = lane >> 4;
    const int j0 = strip * kStrip;

    if (w == 0) {
        // State strip: rows 16 mt + 4 lg4 + i (k index), column j0 + li (v index); the state
        // is stored column by column ([d_v][d_k]), so the 4 rows are a float4.
        float* st = p.state + ((size_t)s * L.h_v + h) * kD * kD + (size_t)(j0 + li) * kD + 4 * lg4;
        v4 S[8];
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) S[mt] = *reinterpret_cast<const v4*>(st + 16 * mt);
        chain_state_role(p, lds, lane, c_begin, c_end, h, j0 + li, lg4, S);
#pragma unroll
        for (int mt = 0; mt < 8; ++mt) *reinterpret_cast<v4*>(st + 16 * mt) = S[mt];
    } else if (w <= 4) {
        const int r = w - 1;
        ChainOut x;
        chain_load_qm(p, c_begin, h, src, r, lane, x.qf, x.mf, x.g);
        lds_barrier();
        for (int c = c_begin; c < c_end; ++c) {
            const int t0 = seq_lo + (c - c_begin) * kChunk;
            chain_out_step<OUT>(p, lds, (c - c_begin) & 1, lane, r, x, ((size_t)t0 * L.h_v + h) * kD + j0 + li,
                                min(kChunk, seq_hi - t0));
            __builtin_amdgcn_sched_barrier(0);                    // the reload after the last use
            chain_load_qm(p, min(c + 1, c_end - 1), h, src, r, lane, x.qf, x.mf, x.g);
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        const bool w_wave = w == 5;                               // wave 5: W; wave 6: K^T
        lds_u8* lds3 = (lds_u8*)lds;                              // the copies address LDS directly
        lds_u8* sink = lds3 + 4 * kOpsBytes + 2 * kHandBytes;
        auto w_of = [&](int cc) { return p.ws.Wf + ((size_t)cc * L.h_v + h) * kFragW; };
        auto kt_of = [&](int cc) { return p.ws.Ktf + ((size_t)cc * L.h_k + src) * kFragKt; };
        // Before the first barrier: W of the first chunk. Between barriers c-1 and c: W of
        // chunk c+1 (used after barrier c) and K^T of chunk c (used after barrier c); the
        // slots they replace were last read before barrier c-1.
        if (w_wave) chain_copy(lds3 + chain_w_slot(0), w_of(c_begin), lane);
#pragma unroll
        for (int a = 1; a <= kWarmAhead; ++a)
            chain_warm(p, sink, min(c_begin + a, c_end - 1), h, src, strip, lane, w_wave);
        if (!w_wave) {
            // The new rolling conv history (nothing in this kernel reads conv_state, and the
            // chunk kernel has read the old history): the sequence's h_v * 8 workgroups split
            // its C channels into contiguous ranges. Its round trip overlaps the W copy.
            const int G = L.h_v * kStrips, g = h * kStrips + strip, per = (L.C + G - 1) / G;
            const int ch_hi = min(L.C, (g + 1) * per);
            for (int ch = g * per + lane; ch < ch_hi; ch += kWave) commit_history(p, ch, seq_lo, seq_hi - seq_lo, s);
        }
        // The copies have landed in LDS; the warm-ups may still be in flight. Bare barriers
        // in this role: a release fence would also wait for the warm-up loads (LDS DMA counts
        // as LDS writes).
        if (w_wave) wait_vmcnt<kWarmAhead * kWarmLoadsW>();
        __builtin_amdgcn_s_barrier();
        for (int c = c_begin; c < c_end; ++c) {
            const int q = (c - c_begin) & 1;
            if (w_wave) {
                if (c + 1 < c_end) chain_copy(lds3 + chain_w_slot(q ^ 1), w_of(c + 1), lane);
            } else {
                chain_copy(lds3 + chain_k_slot(q), kt_of(c), lane);
            }
            chain_warm(p, sink, min(c + 1 + kWarmAhead, c_end - 1), h, src, strip, lane, w_wave);
            if (w_wave) wait_vmcnt<kWarmLoadsW>(); else wait_vmcnt<kWarmLoadsK>();   // this trip's copies done
            __builtin_amdgcn_s_barrier();                         // barrier c
        }
        __builtin_amdgcn_s_waitcnt(0);
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
    if (NC * cfg->h_v > 0x7fffffffLL || ((pairs + 7) / 8) * 8 * kStrips > 0x7fffffffLL) return hipErrorInvalidValue;
    const long long rows = (long long)total_T * cfg->h_v;
    if (gate && (rows + 3) / 4 > 0x7fffffffLL) return hipErrorInvalidValue;

    PrefillParams p;
    p.L = make_layer(cfg, conv_w, A_log, dt_bias);
    p.ws = ws_bind(static_cast<char*>(workspace), off);
    p.cu = cu_seqlens; p.x = x; p.conv_state = conv_state; p.a = a; p.b = b;
    p.state = state; p.o = o; p.o_bf16 = o_bf16;
    p.n_seq = n_seq; p.T = total_T; p.NC = (int)NC;
    p.single = n_seq == 1;
    if (gate && !o) p.o = reinterpret_cast<float*>(static_cast<char*>(workspace) + need);   // the norm's input

    if (!p.single) hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, p);
    const dim3 qgrid((unsigned)NC, (unsigned)cfg->h_k), vgrid((unsigned)(NC * cfg->h_v));
    switch (cfg->d_conv) {
        case 2:
            hipLaunchKernelGGL(qk_kernel<2>, qgrid, dim3(kChunkThreads), 0, s, p);
            hipLaunchKernelGGL(v_kernel<2>, vgrid, dim3(kChunkThreads), 0, s, p);
            break;
        case 3:
            hipLaunchKernelGGL(qk_kernel<3>, qgrid, dim3(kChunkThreads), 0, s, p);
            hipLaunchKernelGGL(v_kernel<3>, vgrid, dim3(kChunkThreads), 0, s, p);
            break;
        default:
            hipLaunchKernelGGL(qk_kernel<4>, qgrid, dim3(kChunkThreads), 0, s, p);
            hipLaunchKernelGGL(v_kernel<4>, vgrid, dim3(kChunkThreads), 0, s, p);
            break;
    }
    const long long groups = (pairs + 7) / 8;
    const dim3 cgrid((unsigned)(groups * 8 * kStrips)), cblock(kChainWaves * kWave);
    switch ((p.o ? 1 : 0) | (p.o_bf16 ? 2 : 0)) {
        case 0: hipLaunchKernelGGL(chain_kernel<0>, cgrid, cblock, 0, s, p); break;
        case 1: hipLaunchKernelGGL(chain_kernel<1>, cgrid, cblock, 0, s, p); break;
        case 2: hipLaunchKernelGGL(chain_kernel<2>, cgrid, cblock, 0, s, p); break;
        default: hipLaunchKernelGGL(chain_kernel<3>, cgrid, cblock, 0, s, p); break;
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
