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
//   prep_kernel    per (chunk, head): conv (history from conv_state at sequence starts), L2
//                  norm of q and k, log decay and beta; fp32 q, k, v into the workspace
//   commit_kernel  per sequence and channel: the new rolling conv history
//   chunk_kernel   per (chunk, v head): K K^T and Q K^T on fp32 MFMA (lower block triangle),
//                  A, M, and W | U by forward substitution (one column per thread)
//   chain_kernel   per (sequence, v head, 16-column state slice): walks the chunks in
//                  order carrying the state slice in MFMA accumulators; D, O and S' on fp32
//                  MFMA, state and output work on separate waves. Columns of the state are
//                  independent, so 8 slices per head fill the GPU even for a single sequence.
// The fp32 matrix cores (v_mfma_f32_16x16x4_f32) keep the chunked result within ~1e-6 of
// the token-by-token recurrence in double.
#include "gdn_common.h"

namespace ixg {
namespace {

constexpr int kChunk = 64;
constexpr int kSlice = 16;                     // state columns per chain workgroup
constexpr int kSlices = kD / kSlice;           // 8
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
    float* qn;           // [h_k][T][128] normalised (and scaled) q
    float* kn;           // [h_k][T][128] normalised k
    float* vv;           // [h_v][T][128] conv output v
    float* lg;           // [h_v][T] log decay
    float* bt;           // [h_v][T] beta
    float* W;            // [NC][h_v][64][128]
    float* Ut;           // [NC][h_v][128][64]  U transposed (column j of U is row j)
    float* M;            // [NC][h_v][64][64]
    float* G;            // [NC][h_v][64] cumulative log decay (padded rows repeat the last)
    float* Kt;           // [NC][h_k][128][64]  K transposed, zero beyond the chunk length
};
constexpr int kWsSections = 14;

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Byte offsets of every workspace section for (n_seq, T); returns the total size.
inline size_t ws_layout(const ix_gdn_cfg* c, int n_seq, int T, size_t off[kWsSections]) {
    const size_t NC = (size_t)(T + kChunk - 1) / kChunk + (size_t)n_seq;
    const size_t sz[kWsSections] = {
        sizeof(int32_t) * (n_seq + 1), sizeof(int32_t) * (n_seq + 1), sizeof(int32_t) * NC, sizeof(int32_t) * NC,
        sizeof(float) * c->h_k * (size_t)T * kD, sizeof(float) * c->h_k * (size_t)T * kD,
        sizeof(float) * c->h_v * (size_t)T * kD, sizeof(float) * c->h_v * (size_t)T,
        sizeof(float) * c->h_v * (size_t)T,
        sizeof(float) * NC * c->h_v * kChunk * kD, sizeof(float) * NC * c->h_v * kChunk * kD,
        sizeof(float) * NC * c->h_v * kChunk * kChunk, sizeof(float) * NC * c->h_v * kChunk,
        sizeof(float) * NC * c->h_k * kD * kChunk,
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
    w.qn = reinterpret_cast<float*>(base + off[4]);
    w.kn = reinterpret_cast<float*>(base + off[5]);
    w.vv = reinterpret_cast<float*>(base + off[6]);
    w.lg = reinterpret_cast<float*>(base + off[7]);
    w.bt = reinterpret_cast<float*>(base + off[8]);
    w.W = reinterpret_cast<float*>(base + off[9]);
    w.Ut = reinterpret_cast<float*>(base + off[10]);
    w.M = reinterpret_cast<float*>(base + off[11]);
    w.G = reinterpret_cast<float*>(base + off[12]);
    w.Kt = reinterpret_cast<float*>(base + off[13]);
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
template <bool IsMax>
__device__ int block_inclusive_scan(int v, int* sh) {
    const int tid = threadIdx.x;
    sh[tid] = v;
    __syncthreads();
    for (int off = 1; off < kPlanThreads; off <<= 1) {
        const int o = tid >= off ? sh[tid - off] : (IsMax ? INT_MIN : 0);
        __syncthreads();
        v = IsMax ? max(v, o) : v + o;
        sh[tid] = v;
        __syncthreads();
    }
    return v;
}

__global__ void __launch_bounds__(kPlanThreads) plan_kernel(const PrefillParams p) {
    __shared__ int sh[kPlanThreads];
    __shared__ int carry;
    const int tid = threadIdx.x, n = p.n_seq;
    // seq_lo[s] = clamp(max(cu[0..s]), 0, T), s = 0..n
    if (tid == 0) carry = 0;
    __syncthreads();
    for (int base = 0; base <= n; base += kPlanThreads) {
        const int s = base + tid;
        int v = s <= n ? min(max(p.cu[s], 0), p.T) : 0;
        v = max(block_inclusive_scan<true>(v, sh), carry);
        if (s <= n) p.ws.seq_lo[s] = v;
        __syncthreads();
        if (tid == kPlanThreads - 1) carry = v;
        __syncthreads();
    }
    // chunk_off = exclusive prefix sum of ceil(len / 64)
    if (tid == 0) carry = 0;
    __syncthreads();
    for (int base = 0; base <= n; base += kPlanThreads) {
        const int s = base + tid;
        const int cnt = s < n ? (p.ws.seq_lo[s + 1] - p.ws.seq_lo[s] + kChunk - 1) / kChunk : 0;
        const int inc = block_inclusive_scan<false>(cnt, sh) + carry;
        if (s <= n) p.ws.chunk_off[s] = inc - cnt;
        if (s < n)
            for (int j = 0; j < cnt; ++j) {
                p.ws.chunk_seq[inc - cnt + j] = s;
                p.ws.chunk_t0[inc - cnt + j] = p.ws.seq_lo[s] + j * kChunk;
            }
        __syncthreads();
        if (tid == kPlanThreads - 1) carry = inc;
        __syncthreads();
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
// prep: grid (NC, 2 h_k + h_v), 256 threads; workgroup = (chunk, one q, k or v head).
// Thread (c = tid & 127, th = tid >> 7) owns channel c of the head for tokens 32 th .. 32 th
// + 31 of the chunk: its history and all its inputs are loaded up front, then the conv runs
// along the tokens. q and k rows are L2-normalised (one wave sum per token and wave, two
// waves per token half).
// ---------------------------------------------------------------------------------------
constexpr int kPrepTok = kChunk / 2;

template <int DC>
__global__ void __launch_bounds__(256) prep_kernel(const PrefillParams p) {
    __shared__ float part[2][2][kPrepTok];          // [token half][wave of the half][token]
    ChunkGeo g;
    if (!chunk_geo(p, blockIdx.x, g)) return;
    const Layer& L = p.L;
    const int lo = p.ws.seq_lo[g.s];
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int c = tid & (kD - 1), th = tid >> 7, wh = (tid >> 6) & 1;
    const int y = blockIdx.y;
    const int kind = y < L.h_k ? 0 : (y < 2 * L.h_k ? 1 : 2);           // q, k, v
    const int head = kind == 0 ? y : (kind == 1 ? y - L.h_k : y - 2 * L.h_k);
    const int ch = kind == 0 ? q_channel(L, head, c) : (kind == 1 ? k_channel(L, head, c) : v_channel(L, head, c));
    const int tb = kPrepTok * th;                                          // first token of this thread
    const int n = min(max(g.len - tb, 0), kPrepTok);

    // History of the first token (only threads that own tokens read it: positions before
    // the sequence start come from its conv state, the others lie inside the sequence).
    float hist[DC - 1];
#pragma unroll
    for (int i = 0; i < DC - 1; ++i) {
        const int pos = g.pos0 + tb - (DC - 1) + i;
        uint16_t u = 0;
        if (n > 0)
            u = pos >= 0 ? p.x[(size_t)(lo + pos) * L.C + ch]
                         : p.conv_state[((size_t)g.s * L.C + ch) * (DC - 1) + (DC - 1) + pos];
        hist[i] = bf16_to_f32(u);
    }
    uint16_t xs[kPrepTok];
#pragma unroll
    for (int t = 0; t < kPrepTok; ++t) xs[t] = t < n ? p.x[(size_t)(g.t0 + tb + t) * L.C + ch] : (uint16_t)0;
    const uint16_t* wr = L.conv_w + (size_t)ch * DC;
    float wv[DC];
#pragma unroll
    for (int i = 0; i < DC; ++i) wv[i] = bf16_to_f32(wr[i]);

    float yv[kPrepTok];
#pragma unroll
    for (int t = 0; t < kPrepTok; ++t) {
        const float xv = bf16_to_f32(xs[t]);
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < DC - 1; ++i) acc = fmaf(hist[i], wv[i], acc);
        acc = fmaf(xv, wv[DC - 1], acc);
        if (L.conv_act == IX_GDN_ACT_SILU) acc = acc * sigmoid_f(acc);
        yv[t] = acc;
#pragma unroll
        for (int i = 0; i < DC - 2; ++i) hist[i] = hist[i + 1];
        hist[DC - 2] = xv;
    }

    if (kind == 2) {
        float* dst = p.ws.vv + ((size_t)head * p.T + g.t0 + tb) * kD + c;
#pragma unroll
        for (int t = 0; t < kPrepTok; ++t)
            if (t < n) dst[(size_t)t * kD] = yv[t];
        if (tid < g.len) {
            const size_t ab = (size_t)(g.t0 + tid) * L.h_v + head;
            p.ws.lg[(size_t)head * p.T + g.t0 + tid] = log_gate(L, head, bf16_to_f32(p.a[ab]));
            p.ws.bt[(size_t)head * p.T + g.t0 + tid] = sigmoid_f(bf16_to_f32(p.b[ab]));
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < kPrepTok; ++t) {
        const float r = wave_sum(yv[t] * yv[t]);
        if (lane == 0) part[th][wh][t] = r;
    }
    __syncthreads();
    const float scale = kind == 0 ? L.q_scale : 1.0f;
    float* dst = (kind == 0 ? p.ws.qn : p.ws.kn) + ((size_t)head * p.T + g.t0 + tb) * kD + c;
#pragma unroll
    for (int t = 0; t < kPrepTok; ++t)
        if (t < n) dst[(size_t)t * kD] = yv[t] * (scale / sqrtf(part[th][0][t] + part[th][1][t] + L.l2_eps));
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
// chunk-local: grid (NC, h_v), 256 threads; workgroup = (chunk, v head)
// ---------------------------------------------------------------------------------------
constexpr int kKS = kD + 4;          // padded LDS row stride of the K tile

// The 10 blocks of the 4 x 4 lower block triangle, 16 x 16 each: wave w takes i = w, w+4, w+8.
__device__ __forceinline__ void tri_block(int i, int& br, int& bc) {
    br = i < 1 ? 0 : i < 3 ? 1 : i < 6 ? 2 : 3;
    bc = i - br * (br + 1) / 2;
}

__global__ void __launch_bounds__(256) chunk_kernel(const PrefillParams p) {
    __shared__ __align__(16) float K_s[kChunk][kKS];
    __shared__ __align__(16) float A_s[kChunk][kChunk];
    __shared__ float G_s[kChunk], B_s[kChunk];

    ChunkGeo g;
    const int c = blockIdx.x;
    if (!chunk_geo(p, c, g)) return;
    const Layer& L = p.L;
    const int h = blockIdx.y, src = src_of(L, h);
    const int tid = threadIdx.x, w = tid / kWave, lane = tid & (kWave - 1);
    const int li = lane & 15, lg4 = lane >> 4;
    const size_t ch = (size_t)c * L.h_v + h;
    const float* kbase = p.ws.kn + ((size_t)src * p.T + g.t0) * kD;
    const float* qbase = p.ws.qn + ((size_t)src * p.T + g.t0) * kD;

    // Stage the K rows of the chunk (zero beyond its length); wave 0 also scans the decay.
    for (int e = tid; e < kChunk * (kD / 4); e += 256) {
        const int t = e / (kD / 4), c4 = e % (kD / 4);
        v4 kv = {0.f, 0.f, 0.f, 0.f};
        if (t < g.len) kv = *reinterpret_cast<const v4*>(kbase + (size_t)t * kD + 4 * c4);
        *reinterpret_cast<v4*>(&K_s[t][4 * c4]) = kv;
    }
    if (w == 0) {
        float lgt = lane < g.len ? p.ws.lg[(size_t)h * p.T + g.t0 + lane] : 0.0f;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {          // inclusive scan over the 64 lanes
            const float o = __shfl_up(lgt, off, kWave);
            if (lane >= off) lgt += o;
        }
        G_s[lane] = lgt;
        B_s[lane] = lane < g.len ? p.ws.bt[(size_t)h * p.T + g.t0 + lane] : 0.0f;
        p.ws.G[ch * kChunk + lane] = lgt;
    }
    __syncthreads();

    // K K^T and Q K^T on the lower block triangle, then A (into LDS) and M (to the workspace).
    // MFMA k index of (block 4m + e, lane group g) is 16 m + 4 g + e for both operands.
    float* Mg = p.ws.M + ch * kChunk * kChunk;
    for (int i = w; i < 10; i += 4) {
        int br, bc;
        tri_block(i, br, bc);
        const int arow = 16 * br + li;
        const bool qok = arow < g.len;
        v4 kk = {0.f, 0.f, 0.f, 0.f}, qk = kk;
#pragma unroll
        for (int m = 0; m < kD / 16; ++m) {
            const v4 ak = *reinterpret_cast<const v4*>(&K_s[arow][16 * m + 4 * lg4]);
            const v4 aq = qok ? *reinterpret_cast<const v4*>(qbase + (size_t)arow * kD + 16 * m + 4 * lg4)
                              : v4{0.f, 0.f, 0.f, 0.f};
            const v4 bk = *reinterpret_cast<const v4*>(&K_s[16 * bc + li][16 * m + 4 * lg4]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                kk = mfma4(ak[e], bk[e], kk);
                qk = mfma4(aq[e], bk[e], qk);
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = 16 * br + 4 * lg4 + r, s = 16 * bc + li;
            float av = 0.0f, mv = 0.0f;
            if (s <= t) {
                const float e = expf(G_s[t] - G_s[s]);
                mv = e * qk[r];
                if (s < t) av = B_s[t] * e * kk[r];
            }
            A_s[t][s] = av;
            Mg[t * kChunk + s] = mv;
        }
    }
    // the upper blocks of M are zero
    for (int e = tid; e < 6 * 256; e += 256) {
        const int i = e >> 8, r = (e >> 4) & 15, col = e & 15;
        const int br = i < 3 ? 0 : (i < 5 ? 1 : 2), bc = i < 3 ? i + 1 : (i < 5 ? i - 1 : 3);
        Mg[(16 * br + r) * kChunk + 16 * bc + col] = 0.0f;
    }
    __syncthreads();

    // Forward substitution (I + A) X = R for the 256 columns of R = [diag(beta Gam) K | diag(beta) V]:
    // waves 0-1 own the W columns, waves 2-3 the U columns (a wave-uniform split).
    {
        const int j = tid & (kD - 1);
        const bool is_w = tid < kD;
        float xr[kChunk];
        if (is_w) {
#pragma unroll
            for (int t = 0; t < kChunk; ++t) xr[t] = B_s[t] * expf(G_s[t]) * K_s[t][j];
        } else {
            const float* vsrc = p.ws.vv + ((size_t)h * p.T + g.t0) * kD + j;
#pragma unroll
            for (int t = 0; t < kChunk; ++t) xr[t] = t < g.len ? B_s[t] * vsrc[(size_t)t * kD] : 0.0f;
        }
        // Four partial sums per row keep the dependent FMA chain short.
#pragma unroll
        for (int t = 1; t < kChunk; ++t) {
            float r[4] = {xr[t], 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int q4 = 0; q4 < t; q4 += 4) {
                const v4 av = *reinterpret_cast<const v4*>(&A_s[t][q4]);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (q4 + e < t) r[e] = fmaf(-av[e], xr[q4 + e], r[e]);
            }
            xr[t] = (r[0] + r[1]) + (r[2] + r[3]);
        }
        if (is_w) {
            float* dst = p.ws.W + ch * kChunk * kD + j;
#pragma unroll
            for (int t = 0; t < kChunk; ++t) dst[(size_t)t * kD] = xr[t];
        } else {
            v4* dst = reinterpret_cast<v4*>(p.ws.Ut + (ch * kD + j) * kChunk);     // column j of U, contiguous
#pragma unroll
            for (int t4 = 0; t4 < kChunk / 4; ++t4) dst[t4] = v4{xr[4 * t4], xr[4 * t4 + 1], xr[4 * t4 + 2], xr[4 * t4 + 3]};
        }
    }
    // K^T of the chunk for the chain's state update, written once per (chunk, q/k head) by the
    // workgroup of its first mapped v head: thread (i = tid / 2, half = tid % 2) writes
    // tokens 32 half .. +31 of row i.
    if (mapped_head(L, src, 0) == h) {
        const int i = tid >> 1, t0h = 32 * (tid & 1);
        v4* dst = reinterpret_cast<v4*>(p.ws.Kt + (((size_t)c * L.h_k + src) * kD + i) * kChunk + t0h);
#pragma unroll
        for (int t4 = 0; t4 < 8; ++t4)
            dst[t4] = v4{K_s[t0h + 4 * t4][i], K_s[t0h + 4 * t4 + 1][i], K_s[t0h + 4 * t4 + 2][i], K_s[t0h + 4 * t4 + 3][i]};
    }
}

// ---------------------------------------------------------------------------------------
// chain: one workgroup per (sequence, v head, 16-column slice), 256 threads
// ---------------------------------------------------------------------------------------
// LDS tiles of the chain are stored column by column (4 padding words per column), so the
// 4 consecutive rows of one column that a lane needs are one 16-byte access.
constexpr int kSCol = kD + 4;          // state slice column stride
constexpr int kDCol = kChunk + 4;      // D tile column stride

// The chain workgroup has 8 waves in two roles that meet at two barriers per chunk:
//   state waves (0-3): S -> LDS | W S, D = U - W S -> LDS | S' = Gam_last S + K^T (exp(G_last - G) D)
//   output waves (4-7):          | Q S                   | O = diag(Gam) Q S + M D
// Each role loads the next chunk's operands (double buffer) while it computes the current one.
// Lane (li = lane & 15, lg4 = lane >> 4) of role wave r uses rows 16 r + li of the 64-row
// chunk tiles as MFMA A operands and rows 16 r + 4 lg4 + i in C layout; state wave r owns
// state rows (k index) 32 r .. 32 r + 31.
struct StateOps {
    v4 aw[8];             // W row 16r+li, k = 16 m + 4 lg4 + e
    v4 kt[2][4];          // K^T row 32 r + 16 tt + li, token 16 q + 4 lg4 + e
    v4 u;                 // U rows 16r + 4 lg4 + i, column j0 + li
    v4 gv;                // G at those rows
    float glast;          // G of the chunk's last row
};
struct OutOps {
    v4 aq[8];             // Q row 16r+li (the last row again past the chunk end)
    v4 am[4];             // M row 16r+li, s = 16 m + 4 lg4 + e
    v4 gv;
    int t0, len;
};

struct ChainCtx {
    const PrefillParams* p;
    const float* qbase;   // q rows of the head's q/k head
    int h, src, seq_lo, seq_hi, c_begin, j0, r, li, lg4;
};

__device__ __forceinline__ size_t chain_ch(const ChainCtx& x, int c) { return (size_t)c * x.p->L.h_v + x.h; }

__device__ __forceinline__ void load_state_ops(const ChainCtx& x, int c, StateOps& o) {
    const PrefillParams& p = *x.p;
    const size_t ch = chain_ch(x, c);
    const float* Wc = p.ws.W + ch * kChunk * kD;
    const float* Gc = p.ws.G + ch * kChunk;
    const float* Kc = p.ws.Kt + ((size_t)c * p.L.h_k + x.src) * kD * kChunk;
    const int arow = 16 * x.r + x.li, crow = 16 * x.r + 4 * x.lg4;
#pragma unroll
    for (int m = 0; m < 8; ++m) o.aw[m] = *reinterpret_cast<const v4*>(Wc + (size_t)arow * kD + 16 * m + 4 * x.lg4);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int q = 0; q < 4; ++q)
            o.kt[tt][q] = *reinterpret_cast<const v4*>(Kc + (size_t)(32 * x.r + 16 * tt + x.li) * kChunk + 16 * q + 4 * x.lg4);
    o.u = *reinterpret_cast<const v4*>(p.ws.Ut + (ch * kD + x.j0 + x.li) * kChunk + crow);
    o.gv = *reinterpret_cast<const v4*>(Gc + crow);
    o.glast = Gc[kChunk - 1];
}

__device__ __forceinline__ void load_out_ops(const ChainCtx& x, int c, OutOps& o) {
    const PrefillParams& p = *x.p;
    const size_t ch = chain_ch(x, c);
    o.t0 = x.seq_lo + (c - x.c_begin) * kChunk;            // chunk c of the sequence (no table lookup)
    o.len = min(kChunk, x.seq_hi - o.t0);
    const int arow = 16 * x.r + x.li, crow = 16 * x.r + 4 * x.lg4;
    // Q rows past the chunk end re-read its last row: an MFMA output row depends only on its
    // own A row, so those rows only produce output rows that are never stored.
    const float* qr = x.qbase + (size_t)(o.t0 + min(arow, o.len - 1)) * kD + 4 * x.lg4;
#pragma unroll
    for (int m = 0; m < 8; ++m) o.aq[m] = *reinterpret_cast<const v4*>(qr + 16 * m);
    const float* Mc = p.ws.M + ch * kChunk * kChunk;
#pragma unroll
    for (int m = 0; m < 4; ++m) o.am[m] = *reinterpret_cast<const v4*>(Mc + (size_t)arow * kChunk + 16 * m + 4 * x.lg4);
    o.gv = *reinterpret_cast<const v4*>(p.ws.G + ch * kChunk + crow);
}

// State waves, one chunk: D = U - W S, S' = Gam_last S + K^T (exp(G_last - G) D).
__device__ __forceinline__ void state_step(const ChainCtx& x, const StateOps& o, v4 (&S)[2], float* S_l,
                                           float* D_l, float* Dg_l) {
    const int r = x.r, li = x.li, lg4 = x.lg4, crow = 16 * r + 4 * lg4;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) *reinterpret_cast<v4*>(S_l + li * kSCol + 32 * r + 16 * tt + 4 * lg4) = S[tt];
    lds_barrier();                                                    // (A) state slice visible

    // W S for rows 16r..16r+15; k index of block (m, e), lane group g: 16 m + 4 g + e (each
    // load instruction of a wave then reads 64 contiguous bytes of 16 operand rows).
    v4 ws[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const v4 bv = *reinterpret_cast<const v4*>(S_l + li * kSCol + 16 * m + 4 * lg4);
#pragma unroll
        for (int e = 0; e < 4; ++e) ws[m & 1] = mfma4(o.aw[m][e], bv[e], ws[m & 1]);
    }
    v4 d, dg;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        d[i] = o.u[i] - (ws[0][i] + ws[1][i]);
        dg[i] = expf(o.glast - o.gv[i]) * d[i];
    }
    *reinterpret_cast<v4*>(D_l + li * kDCol + crow) = d;
    *reinterpret_cast<v4*>(Dg_l + li * kDCol + crow) = dg;
    lds_barrier();                                                    // (B) D visible

    // S' = Gam_last S + K^T Dg; token index of block (q, e): 16 q + 4 g + e.
    const float gl = expf(o.glast);
    v4 dgv[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) dgv[m] = *reinterpret_cast<const v4*>(Dg_l + li * kDCol + 16 * m + 4 * lg4);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        v4 acc = {0.f, 0.f, 0.f, 0.f};
        S[tt] *= gl;
#pragma unroll
        for (int b = 0; b < 16; ++b) {
            if (b & 1) acc = mfma4(o.kt[tt][b >> 2][b & 3], dgv[b >> 2][b & 3], acc);
            else S[tt] = mfma4(o.kt[tt][b >> 2][b & 3], dgv[b >> 2][b & 3], S[tt]);
        }
        S[tt] += acc;
    }
}

// Output waves, one chunk: O = diag(Gam) Q S + M D for rows 16r..16r+15.
__device__ __forceinline__ void out_step(const ChainCtx& x, const OutOps& o, const float* S_l, const float* D_l) {
    const PrefillParams& p = *x.p;
    const int r = x.r, li = x.li, lg4 = x.lg4, crow = 16 * r + 4 * lg4;
    lds_barrier();                                                    // (A)
    v4 qs[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        const v4 bv = *reinterpret_cast<const v4*>(S_l + li * kSCol + 16 * m + 4 * lg4);
#pragma unroll
        for (int e = 0; e < 4; ++e) qs[m & 1] = mfma4(o.aq[m][e], bv[e], qs[m & 1]);
    }
    lds_barrier();                                                    // (B)
    v4 ov[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) { ov[0][i] = expf(o.gv[i]) * (qs[0][i] + qs[1][i]); ov[1][i] = 0.0f; }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const v4 bv = *reinterpret_cast<const v4*>(D_l + li * kDCol + 16 * m + 4 * lg4);
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[m & 1] = mfma4(o.am[m][e], bv[e], ov[m & 1]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = crow + i;
        if (t < o.len) {
            const size_t oo = ((size_t)(o.t0 + t) * p.L.h_v + x.h) * kD + x.j0 + li;
            const float ovr = ov[0][i] + ov[1][i];
            if (p.o) p.o[oo] = ovr;
            if (p.o_bf16) p.o_bf16[oo] = f32_to_bf16(ovr);
        }
    }
}

__global__ void __launch_bounds__(512) chain_kernel(const PrefillParams p) {
    __shared__ __align__(16) float S_l[kSlice * kSCol];
    __shared__ __align__(16) float D_l[kSlice * kDCol];
    __shared__ __align__(16) float Dg_l[kSlice * kDCol];

    const Layer& L = p.L;
    // XCD-aware mapping: the 8 slices of one (sequence, head) pair share an XCD (and its L2).
    const int lin = blockIdx.x, xcd = lin & 7, k = lin >> 3;
    const int slice = k & 7;
    const int pair = (k >> 3) * 8 + xcd;
    if (pair >= p.n_seq * L.h_v) return;
    const int s = pair / L.h_v, h = pair % L.h_v, src = src_of(L, h);
    const int c_begin = p.ws.chunk_off[s], c_end = p.ws.chunk_off[s + 1];
    if (c_begin >= c_end) return;
    const int tid = threadIdx.x, w = tid / kWave, lane = tid & (kWave - 1);

    ChainCtx x;
    x.p = &p;
    x.qbase = p.ws.qn + (size_t)src * p.T * kD;
    x.h = h;
    x.src = src;
    x.seq_lo = p.ws.seq_lo[s];
    x.seq_hi = p.ws.seq_lo[s + 1];
    x.c_begin = c_begin;
    x.j0 = slice * kSlice;
    x.r = w & 3;
    x.li = lane & 15;
    x.lg4 = lane >> 4;

    if (w < 4) {
        // State slice: rows 32 r + 16 tt + 4 lg4 + i (k index), column j0 + li (v index); the
        // state is stored column by column ([d_v][d_k]), so the 4 rows are a float4.
        float* st = p.state + (((size_t)s * L.h_v + h) * kD + x.j0 + x.li) * kD + 32 * x.r + 4 * x.lg4;
        v4 S[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) S[tt] = *reinterpret_cast<const v4*>(st + 16 * tt);
        __builtin_amdgcn_s_waitcnt(0);             // the state is in registers before the loop
        // Prefetches are unconditional (past the last chunk they re-read it): a load that is
        // skipped on one path forces the compiler to wait for every load in flight.
        StateOps A, B;
        load_state_ops(x, c_begin, A);
        int c = c_begin;
        for (; c + 1 < c_end; c += 2) {
            load_state_ops(x, c + 1, B);
            state_step(x, A, S, S_l, D_l, Dg_l);
            __builtin_amdgcn_sched_barrier(0);     // keep A's reload after A's last use
            load_state_ops(x, min(c + 2, c_end - 1), A);
            state_step(x, B, S, S_l, D_l, Dg_l);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c < c_end) state_step(x, A, S, S_l, D_l, Dg_l);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) *reinterpret_cast<v4*>(st + 16 * tt) = S[tt];
    } else {
        OutOps A, B;                               // same schedule as the state waves
        load_out_ops(x, c_begin, A);
        int c = c_begin;
        for (; c + 1 < c_end; c += 2) {
            load_out_ops(x, c + 1, B);
            out_step(x, A, S_l, D_l);
            __builtin_amdgcn_sched_barrier(0);
            load_out_ops(x, min(c + 2, c_end - 1), A);
            out_step(x, B, S_l, D_l);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (c < c_end) out_step(x, A, S_l, D_l);
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
    const dim3 pgrid((unsigned)NC, (unsigned)(2 * cfg->h_k + cfg->h_v));
    switch (cfg->d_conv) {
        case 2: hipLaunchKernelGGL(prep_kernel<2>, pgrid, dim3(256), 0, s, p); break;
        case 3: hipLaunchKernelGGL(prep_kernel<3>, pgrid, dim3(256), 0, s, p); break;
        default: hipLaunchKernelGGL(prep_kernel<4>, pgrid, dim3(256), 0, s, p); break;
    }
    const size_t nch = (size_t)n_seq * p.L.C;
    hipLaunchKernelGGL(commit_kernel, dim3((unsigned)((nch + 255) / 256)), dim3(256), 0, s, p);
    hipLaunchKernelGGL(chunk_kernel, dim3((unsigned)NC, (unsigned)cfg->h_v), dim3(256), 0, s, p);
    const long long groups = (pairs + 7) / 8;
    hipLaunchKernelGGL(chain_kernel, dim3((unsigned)(groups * 64)), dim3(512), 0, s, p);
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
