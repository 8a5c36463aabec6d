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
//   prep_kernel    per chunk: conv (history from conv_state at sequence starts), L2 norm of
//                  q and k, log decay and beta; fp32 q, k, v into the workspace
//   commit_kernel  per sequence and channel: the new rolling conv history
//   chunk_kernel   per (chunk, q/k head): K K^T and Q K^T on fp32 MFMA, then per mapped v
//                  head A, M, and W | U by forward substitution (one column per thread)
//   chain_kernel   per (sequence, v head, 16-column state slice): walks the chunks in
//                  order carrying the state slice in MFMA accumulators; D, O and S' on fp32
//                  MFMA. Columns of the state are independent, so 8 slices per head fill
//                  the GPU even for a single sequence.
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
    float* U;            // [NC][h_v][64][128]
    float* M;            // [NC][h_v][64][64]
    float* G;            // [NC][h_v][64] cumulative log decay (padded rows repeat the last)
};

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Byte offsets of every workspace section for (n_seq, T); returns the total size.
inline size_t ws_layout(const ix_gdn_cfg* c, int n_seq, int T, size_t off[13]) {
    const size_t NC = (size_t)(T + kChunk - 1) / kChunk + (size_t)n_seq;
    const size_t sz[13] = {
        sizeof(int32_t) * (n_seq + 1), sizeof(int32_t) * (n_seq + 1), sizeof(int32_t) * NC, sizeof(int32_t) * NC,
        sizeof(float) * c->h_k * (size_t)T * kD, sizeof(float) * c->h_k * (size_t)T * kD,
        sizeof(float) * c->h_v * (size_t)T * kD, sizeof(float) * c->h_v * (size_t)T,
        sizeof(float) * c->h_v * (size_t)T,
        sizeof(float) * NC * c->h_v * kChunk * kD, sizeof(float) * NC * c->h_v * kChunk * kD,
        sizeof(float) * NC * c->h_v * kChunk * kChunk, sizeof(float) * NC * c->h_v * kChunk,
    };
    size_t pos = 0;
    for (int i = 0; i < 13; ++i) { off[i] = pos; pos += align256(sz[i]); }
    return pos;
}

inline Ws ws_bind(char* base, const size_t off[13]) {
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
    w.U = reinterpret_cast<float*>(base + off[10]);
    w.M = reinterpret_cast<float*>(base + off[11]);
    w.G = reinterpret_cast<float*>(base + off[12]);
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

// Conv output of channel ch at token position pos of sequence s (history from x, or from the
// sequence's conv state for the first dc-1 positions).
__device__ __forceinline__ float conv_at(const PrefillParams& p, int s, int lo, int pos, int ch) {
    const Layer& L = p.L;
    float hist[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        hist[i] = 0.0f;
        if (i < L.dc - 1) {
            const int hp = pos - (L.dc - 1) + i;
            const uint16_t u = hp >= 0 ? p.x[(size_t)(lo + hp) * L.C + ch]
                                       : p.conv_state[((size_t)s * L.C + ch) * (L.dc - 1) + (L.dc - 1) + hp];
            hist[i] = bf16_to_f32(u);
        }
    }
    const float xv = bf16_to_f32(p.x[(size_t)(lo + pos) * L.C + ch]);
    return conv_eval(L, hist, xv, L.conv_w + (size_t)ch * L.dc);
}

// ---------------------------------------------------------------------------------------
// prep: grid (NC, h_k + h_v), 256 threads
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) prep_kernel(const PrefillParams p) {
    ChunkGeo g;
    if (!chunk_geo(p, blockIdx.x, g)) return;
    const Layer& L = p.L;
    const int lo = p.ws.seq_lo[g.s];
    const int tid = threadIdx.x, w = tid / kWave, lane = tid & (kWave - 1);
    const int y = blockIdx.y;
    if (y < L.h_k) {
        // q and k of head src: one wave per token, lanes own dims lane and lane + 64.
        const int src = y;
        for (int t = w; t < g.len; t += 4) {
            const int pos = g.pos0 + t;
            const float q0 = conv_at(p, g.s, lo, pos, q_channel(L, src, lane));
            const float q1 = conv_at(p, g.s, lo, pos, q_channel(L, src, lane + kWave));
            const float k0 = conv_at(p, g.s, lo, pos, k_channel(L, src, lane));
            const float k1 = conv_at(p, g.s, lo, pos, k_channel(L, src, lane + kWave));
            const float qq = wave_sum(fmaf(q0, q0, q1 * q1));
            const float kk = wave_sum(fmaf(k0, k0, k1 * k1));
            const float inv_q = L.q_scale / sqrtf(qq + L.l2_eps);
            const float inv_k = 1.0f / sqrtf(kk + L.l2_eps);
            const size_t row = ((size_t)src * p.T + g.t0 + t) * kD;
            p.ws.qn[row + lane] = q0 * inv_q;
            p.ws.qn[row + lane + kWave] = q1 * inv_q;
            p.ws.kn[row + lane] = k0 * inv_k;
            p.ws.kn[row + lane + kWave] = k1 * inv_k;
        }
    } else {
        const int h = y - L.h_k;
        for (int e = tid; e < g.len * kD; e += 256) {
            const int t = e / kD, j = e % kD;
            p.ws.vv[((size_t)h * p.T + g.t0 + t) * kD + j] = conv_at(p, g.s, lo, g.pos0 + t, v_channel(L, h, j));
        }
        if (tid < g.len) {
            const size_t ab = (size_t)(g.t0 + tid) * L.h_v + h;
            p.ws.lg[(size_t)h * p.T + g.t0 + tid] = log_gate(L, h, bf16_to_f32(p.a[ab]));
            p.ws.bt[(size_t)h * p.T + g.t0 + tid] = sigmoid_f(bf16_to_f32(p.b[ab]));
        }
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
// chunk-local: grid (NC, h_k), 256 threads
// ---------------------------------------------------------------------------------------
constexpr int kKS = kD + 4;          // padded LDS row stride of K and Q tiles

__global__ void __launch_bounds__(256) chunk_kernel(const PrefillParams p) {
    __shared__ __align__(16) float K_s[kChunk][kKS];
    __shared__ __align__(16) float Q_s[kChunk][kKS];
    __shared__ __align__(16) float A_s[kChunk][kChunk];
    __shared__ float G_s[kChunk], B_s[kChunk];
    float (*KK_s)[kChunk] = reinterpret_cast<float (*)[kChunk]>(&Q_s[0][0]);              // after Q K^T
    float (*QK_s)[kChunk] = reinterpret_cast<float (*)[kChunk]>(&Q_s[0][0] + kChunk * kChunk);

    ChunkGeo g;
    const int c = blockIdx.x;
    if (!chunk_geo(p, c, g)) return;
    const Layer& L = p.L;
    const int src = blockIdx.y;
    const int tid = threadIdx.x, w = tid / kWave, lane = tid & (kWave - 1);
    const int li = lane & 15, lg4 = lane >> 4;

    // Stage K and Q rows of the chunk (zero beyond its length).
    for (int e = tid; e < kChunk * (kD / 4); e += 256) {
        const int t = e / (kD / 4), c4 = e % (kD / 4);
        v4 kv = {0.f, 0.f, 0.f, 0.f}, qv = kv;
        if (t < g.len) {
            const size_t row = ((size_t)src * p.T + g.t0 + t) * kD;
            kv = *reinterpret_cast<const v4*>(p.ws.kn + row + 4 * c4);
            qv = *reinterpret_cast<const v4*>(p.ws.qn + row + 4 * c4);
        }
        *reinterpret_cast<v4*>(&K_s[t][4 * c4]) = kv;
        *reinterpret_cast<v4*>(&Q_s[t][4 * c4]) = qv;
    }
    __syncthreads();

    // K K^T and Q K^T, lower block triangle: wave w owns block row w, blocks c <= w.
    // MFMA k index of (block 4m + e, lane group g) is 16 m + 4 g + e (same for A and B).
    v4 kk[4], qk[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) { kk[cb] = v4{0.f, 0.f, 0.f, 0.f}; qk[cb] = kk[cb]; }
#pragma unroll
    for (int m = 0; m < kD / 16; ++m) {
        const v4 ak = *reinterpret_cast<const v4*>(&K_s[16 * w + li][16 * m + 4 * lg4]);
        const v4 aq = *reinterpret_cast<const v4*>(&Q_s[16 * w + li][16 * m + 4 * lg4]);
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            if (cb <= w) {
                const v4 bk = *reinterpret_cast<const v4*>(&K_s[16 * cb + li][16 * m + 4 * lg4]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    kk[cb] = mfma4(ak[e], bk[e], kk[cb]);
                    qk[cb] = mfma4(aq[e], bk[e], qk[cb]);
                }
            }
        }
    }

    // Park both products in LDS (over Q_s, which is no longer read) to free the accumulators.
    __syncthreads();
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            KK_s[16 * w + 4 * lg4 + r][16 * cb + li] = kk[cb][r];
            QK_s[16 * w + 4 * lg4 + r][16 * cb + li] = qk[cb][r];
        }
    __syncthreads();

    const int count = mapped_count(L, src);
    for (int m = 0; m < count; ++m) {
        const int h = mapped_head(L, src, m);
        const size_t ch = (size_t)c * L.h_v + h;
        if (w == 0) {
            float lgt = lane < g.len ? p.ws.lg[(size_t)h * p.T + g.t0 + lane] : 0.0f;
            // inclusive scan over the 64 lanes
#pragma unroll
            for (int off = 1; off < kWave; off <<= 1) {
                const float o = __shfl_up(lgt, off, kWave);
                if (lane >= off) lgt += o;
            }
            G_s[lane] = lgt;
            B_s[lane] = lane < g.len ? p.ws.bt[(size_t)h * p.T + g.t0 + lane] : 0.0f;
            p.ws.G[ch * kChunk + lane] = lgt;
        }
        __syncthreads();

        // A into LDS, M into the workspace (C layout: row 16w + 4 lg4 + r, column 16 cb + li).
        float* Mg = p.ws.M + ch * kChunk * kChunk;
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * w + 4 * lg4 + r, s = 16 * cb + li;
                float av = 0.0f, mv = 0.0f;
                if (s <= t) {
                    const float e = expf(G_s[t] - G_s[s]);
                    mv = e * QK_s[t][s];
                    if (s < t) av = B_s[t] * e * KK_s[t][s];
                }
                A_s[t][s] = av;
                Mg[t * kChunk + s] = mv;
            }
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
#pragma unroll
            for (int t = 1; t < kChunk; ++t) {
                float r = xr[t];
#pragma unroll
                for (int q4 = 0; q4 < t; q4 += 4) {
                    const v4 av = *reinterpret_cast<const v4*>(&A_s[t][q4]);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (q4 + e < t) r = fmaf(-av[e], xr[q4 + e], r);
                }
                xr[t] = r;
            }
            float* dst = (is_w ? p.ws.W : p.ws.U) + ch * kChunk * kD + j;
#pragma unroll
            for (int t = 0; t < kChunk; ++t) dst[(size_t)t * kD] = xr[t];
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------
// chain: one workgroup per (sequence, v head, 16-column slice), 256 threads
// ---------------------------------------------------------------------------------------
// Rows r and r + 32 (state) or r and r + 16 (chunk rows) are read by the two lane groups
// of a half wave together; 16 padding words after every such block put them 16 banks apart.
__device__ __forceinline__ int s_idx(int row, int col) { return row * kSlice + col + 16 * (row >> 5); }
__device__ __forceinline__ int d_idx(int row, int col) { return row * kSlice + col + 16 * (row >> 4); }

__global__ void __launch_bounds__(256) chain_kernel(const PrefillParams p) {
    __shared__ float S_l[kD * kSlice + 16 * (kD / 32)];
    __shared__ float D_l[kChunk * kSlice + 16 * (kChunk / 16)];
    __shared__ float Dg_l[kChunk * kSlice + 16 * (kChunk / 16)];

    const Layer& L = p.L;
    // XCD-aware mapping: the 8 slices of one (sequence, head) pair share an XCD (and its L2).
    const int lin = blockIdx.x, xcd = lin & 7, k = lin >> 3;
    const int slice = k & 7;
    const int pair = (k >> 3) * 8 + xcd;
    if (pair >= p.n_seq * L.h_v) return;
    const int s = pair / L.h_v, h = pair % L.h_v, src = src_of(L, h);
    const int c_begin = p.ws.chunk_off[s], c_end = p.ws.chunk_off[s + 1];
    if (c_begin >= c_end) return;
    const int seq_hi = p.ws.seq_lo[s + 1];
    const int j0 = slice * kSlice;
    const int tid = threadIdx.x, w = tid / kWave, lane = tid & (kWave - 1);
    const int li = lane & 15, lg4 = lane >> 4;

    // State slice: wave w owns rows 32 w + 16 tt + 4 lg4 + r (k index), column j0 + li (v
    // index); the state is stored column by column ([d_v][d_k]), so the 4 rows are a float4.
    float* st = p.state + (((size_t)s * L.h_v + h) * kD + j0 + li) * kD + 32 * w + 4 * lg4;
    v4 S[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) S[tt] = *reinterpret_cast<const v4*>(st + 16 * tt);

    const float* qbase = p.ws.qn + (size_t)src * p.T * kD;
    const float* kbase = p.ws.kn + (size_t)src * p.T * kD;

    for (int c = c_begin; c < c_end; ++c) {
        const int t0 = p.ws.chunk_t0[c];
        const int len = min(kChunk, seq_hi - t0);
        const size_t ch = (size_t)c * L.h_v + h;
        const float* Wc = p.ws.W + ch * kChunk * kD;
        const float* Uc = p.ws.U + ch * kChunk * kD;
        const float* Mc = p.ws.M + ch * kChunk * kChunk;
        const float* Gc = p.ws.G + ch * kChunk;

        // Operands of this chunk (issued before the state exchange).
        const int arow = 16 * w + li;                          // A-operand row of this lane
        v4 aw[8], aq[8], am[4];
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            aw[m] = *reinterpret_cast<const v4*>(Wc + (size_t)arow * kD + 32 * lg4 + 4 * m);
            aq[m] = arow < len ? *reinterpret_cast<const v4*>(qbase + (size_t)(t0 + arow) * kD + 32 * lg4 + 4 * m)
                               : v4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) am[m] = *reinterpret_cast<const v4*>(Mc + (size_t)arow * kChunk + 16 * lg4 + 4 * m);
        const int crow = 16 * w + 4 * lg4;                     // C-layout rows crow + r
        float u[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) u[r] = Uc[(size_t)(crow + r) * kD + j0 + li];
        const v4 gv = *reinterpret_cast<const v4*>(Gc + crow);
        const float glast = Gc[kChunk - 1];

        // 1. state slice -> LDS
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int r = 0; r < 4; ++r) S_l[s_idx(32 * w + 16 * tt + 4 * lg4 + r, li)] = S[tt][r];
        __syncthreads();

        // 2. W S and Q S for rows 16w..16w+15 (k index of block b, lane group g: 32 g + b).
        v4 ws = {0.f, 0.f, 0.f, 0.f}, qs = ws;
#pragma unroll
        for (int m = 0; m < 8; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float bv = S_l[s_idx(32 * lg4 + 4 * m + e, li)];
                ws = mfma4(aw[m][e], bv, ws);
                qs = mfma4(aq[m][e], bv, qs);
            }

        // 3. D = U - W S; D and exp(G_last - G_t) D to LDS.
        v4 d;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            d[r] = u[r] - ws[r];
            D_l[d_idx(crow + r, li)] = d[r];
            Dg_l[d_idx(crow + r, li)] = expf(glast - gv[r]) * d[r];
        }
        __syncthreads();

        // 4. O = diag(Gam) Q S + M D (k index 16 g + b).
        v4 ov;
#pragma unroll
        for (int r = 0; r < 4; ++r) ov[r] = expf(gv[r]) * qs[r];
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) ov = mfma4(am[m][e], D_l[d_idx(16 * lg4 + 4 * m + e, li)], ov);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = crow + r;
            if (t < len) {
                const size_t oo = ((size_t)(t0 + t) * L.h_v + h) * kD + j0 + li;
                if (p.o) p.o[oo] = ov[r];
                if (p.o_bf16) p.o_bf16[oo] = f32_to_bf16(ov[r]);
            }
        }

        // 5. S' = Gam_last S + K^T (exp(G_last - G) D), k index 16 g + b over the chunk rows.
        const float gl = expf(glast);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            S[tt] *= gl;
            const int col = 32 * w + 16 * tt + li;            // A-operand row of K^T = k dim
#pragma unroll
            for (int b = 0; b < 16; ++b) {
                const int t = 16 * lg4 + b;
                const float kv = t < len ? kbase[(size_t)(t0 + t) * kD + col] : 0.0f;
                S[tt] = mfma4(kv, Dg_l[d_idx(t, li)], S[tt]);
            }
        }
    }

#pragma unroll
    for (int tt = 0; tt < 2; ++tt) *reinterpret_cast<v4*>(st + 16 * tt) = S[tt];
}

}  // namespace
}  // namespace ixg

extern "C" hipError_t ix_gdn_check_cfg_(const ix_gdn_cfg* c);

extern "C" size_t ix_gdn_prefill_workspace_size(const ix_gdn_cfg* cfg, int n_seq, int total_T) {
    if (ix_gdn_check_cfg_(cfg) != hipSuccess || n_seq <= 0 || total_T < 0) return 0;
    size_t off[13];
    return ixg::ws_layout(cfg, n_seq, total_T, off);
}

extern "C" hipError_t ix_gdn_prefill(const ix_gdn_cfg* cfg, int n_seq, int total_T, const int32_t* cu_seqlens,
                                     const uint16_t* x, uint16_t* conv_state, const uint16_t* conv_w,
                                     const uint16_t* a, const uint16_t* b, const float* A_log,
                                     const float* dt_bias, float* state, float* o, uint16_t* o_bf16,
                                     void* workspace, size_t workspace_bytes, hipStream_t s) {
    using namespace ixg;
    const hipError_t e = ix_gdn_check_cfg_(cfg);
    if (e != hipSuccess) return e;
    if (n_seq <= 0 || total_T < 0) return hipErrorInvalidValue;
    if (!cu_seqlens || !conv_state || !conv_w || !A_log || !dt_bias || !state) return hipErrorInvalidValue;
    if (total_T == 0) return hipSuccess;                       // nothing to consume
    if (!x || !a || !b || !workspace) return hipErrorInvalidValue;
    if (reinterpret_cast<uintptr_t>(workspace) & 255) return hipErrorInvalidValue;
    if (reinterpret_cast<uintptr_t>(state) & 15) return hipErrorInvalidValue;      // float4 state accesses
    size_t off[13];
    const size_t need = ws_layout(cfg, n_seq, total_T, off);
    if (workspace_bytes < need) return hipErrorInvalidValue;
    const long long NC = (total_T + kChunk - 1) / kChunk + (long long)n_seq;
    const long long pairs = (long long)n_seq * cfg->h_v;
    if (NC > 0x7fffffffLL || pairs * kSlices > 0x7fffffffLL) return hipErrorInvalidValue;

    PrefillParams p;
    p.L = make_layer(cfg, conv_w, A_log, dt_bias);
    p.ws = ws_bind(static_cast<char*>(workspace), off);
    p.cu = cu_seqlens; p.x = x; p.conv_state = conv_state; p.a = a; p.b = b;
    p.state = state; p.o = o; p.o_bf16 = o_bf16;
    p.n_seq = n_seq; p.T = total_T; p.NC = (int)NC;

    hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0, s, p);
    hipLaunchKernelGGL(prep_kernel, dim3((unsigned)NC, (unsigned)(cfg->h_k + cfg->h_v)), dim3(256), 0, s, p);
    const size_t nch = (size_t)n_seq * p.L.C;
    hipLaunchKernelGGL(commit_kernel, dim3((unsigned)((nch + 255) / 256)), dim3(256), 0, s, p);
    hipLaunchKernelGGL(chunk_kernel, dim3((unsigned)NC, (unsigned)cfg->h_k), dim3(256), 0, s, p);
    const long long groups = (pairs + 7) / 8;
    hipLaunchKernelGGL(chain_kernel, dim3((unsigned)(groups * 64)), dim3(256), 0, s, p);
    return hipGetLastError();
}
