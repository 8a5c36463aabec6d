// gdn_legacy.hip -- the five fp32 entry points of the reference's src/ix_gdn.cu, redesigned
// for gfx950 behind the same C signatures (include/ix_gdn.h).
//
//   ix_gdn_step       src/ix_gdn.cu:25-56, :108-114
//   ix_gdn_conv_step  src/ix_gdn.cu:58-70, :115-120
//   ix_gdn_l2_norm    src/ix_gdn.cu:73-84, :121-125
//   ix_gdn_beta_gate  src/ix_gdn.cu:102-105, :126-130
//   ix_gdn_out_norm   src/ix_gdn.cu:87-100, :131-136
//
// The step is the only kernel with real traffic. The reference sweeps each state column
// twice with one thread per column (2 reads + 2 writes per element, 128 dependent strided
// loads per thread). Here one 256-thread workgroup owns a head: every state element is
// loaded once into registers with coalesced row loads, both contractions S^T k and S^T q
// are reduced in one sweep (in-thread, then across the four waves through LDS), and the
// element is written once:
//   u = g S^T k,  d = beta (v - u),  S' = g S + k d^T,  o = S'^T q = g S^T q + d (k . q).
#include "ix_gdn.h"
#include "wave64.h"

namespace ixg {
namespace {

constexpr int kStepThreads = 256;                     // 4 waves per head
constexpr int kStepWaves = kStepThreads / kWave;
constexpr int kStepMaxS = 128;
constexpr int kStepRows = kStepMaxS / kStepWaves;     // rows per thread (row i = wave + 4*m)
constexpr int kStepCols = kStepMaxS / kWave;          // columns per lane (j = lane + 64*c)

__global__ void __launch_bounds__(kStepThreads)
step_kernel(float* __restrict__ state, const float* __restrict__ q, const float* __restrict__ k,
            const float* __restrict__ v, const float* __restrict__ gate, const float* __restrict__ beta,
            float* __restrict__ o, int S, int h_k, int h_v) {
    __shared__ float ks[kStepMaxS], qs[kStepMaxS];
    __shared__ float red[2][kStepWaves][kStepMaxS];
    __shared__ float kq_part[kStepWaves];

    const int h = blockIdx.x;
    const int src = h % h_k;                           // modulo head pairing, src/ix_gdn.cu:38
    const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
    const size_t row_stride = (size_t)h_v * S;         // layout [S][h_v][S], src/ix_gdn.cu:47-48
    float* base = state + (size_t)h * S;

    // Issue every state load of this thread first; they overlap the staging below.
    float s[kStepRows][kStepCols];
#pragma unroll
    for (int m = 0; m < kStepRows; ++m) {
        const int i = w + kStepWaves * m;
#pragma unroll
        for (int c = 0; c < kStepCols; ++c) {
            const int j = lane + kWave * c;
            s[m][c] = (i < S && j < S) ? base[(size_t)i * row_stride + j] : 0.0f;
        }
    }
    if (tid < S) { ks[tid] = k[(size_t)src * S + tid]; qs[tid] = q[(size_t)src * S + tid]; }
    const float g = expf(gate[h]);                     // decay, src/ix_gdn.cu:40
    const float bt = beta[h];
    __syncthreads();

    // k . q (needed for the output identity); wave w covers indices w*64 .. w*64+63.
    {
        const int i = tid;
        float p = (i < S && i < kStepMaxS) ? ks[i] * qs[i] : 0.0f;
        p = wave_sum(p);
        if (lane == 0) kq_part[w] = p;
    }

    float ak[kStepCols], aq[kStepCols];
#pragma unroll
    for (int c = 0; c < kStepCols; ++c) { ak[c] = 0.0f; aq[c] = 0.0f; }
#pragma unroll
    for (int m = 0; m < kStepRows; ++m) {
        const int i = w + kStepWaves * m;
        const float ki = (i < S) ? ks[i] : 0.0f, qi = (i < S) ? qs[i] : 0.0f;
#pragma unroll
        for (int c = 0; c < kStepCols; ++c) { ak[c] = fmaf(s[m][c], ki, ak[c]); aq[c] = fmaf(s[m][c], qi, aq[c]); }
    }
#pragma unroll
    for (int c = 0; c < kStepCols; ++c) { red[0][w][lane + kWave * c] = ak[c]; red[1][w][lane + kWave * c] = aq[c]; }
    __syncthreads();

    const float kq = kq_part[0] + kq_part[1] + kq_part[2] + kq_part[3];
    float d[kStepCols];
#pragma unroll
    for (int c = 0; c < kStepCols; ++c) {
        const int j = lane + kWave * c;
        const float A = red[0][0][j] + red[0][1][j] + red[0][2][j] + red[0][3][j];
        const float Bq = red[1][0][j] + red[1][1][j] + red[1][2][j] + red[1][3][j];
        const float vj = (j < S) ? v[(size_t)h * S + j] : 0.0f;
        d[c] = (vj - g * A) * bt;
        if (w == 0 && j < S) o[(size_t)h * S + j] = fmaf(d[c], kq, g * Bq);
    }
#pragma unroll
    for (int m = 0; m < kStepRows; ++m) {
        const int i = w + kStepWaves * m;
        if (i < S) {
            const float ki = ks[i];
#pragma unroll
            for (int c = 0; c < kStepCols; ++c) {
                const int j = lane + kWave * c;
                if (j < S) base[(size_t)i * row_stride + j] = fmaf(ki, d[c], s[m][c] * g);
            }
        }
    }
}

// One thread per channel (src/ix_gdn.cu:58-70). Memory-bound elementwise work.
__global__ void __launch_bounds__(256)
conv_kernel(float* __restrict__ cs, const float* __restrict__ x, const float* __restrict__ kW,
            float* __restrict__ out, int C, int dc) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= C) return;
    float* st = cs + (size_t)c * (dc - 1);
    const float* wc = kW + (size_t)c * dc;
    const float xc = x[c];
    float acc = 0.0f;
    for (int i = 0; i < dc - 1; ++i) acc = fmaf(st[i], wc[i], acc);
    out[c] = fmaf(xc, wc[dc - 1], acc);
    for (int i = 0; i < dc - 2; ++i) st[i] = st[i + 1];
    st[dc - 2] = xc;
}

// One wave per row, four rows per workgroup; double accumulation as src/ix_gdn.cu:75-82.
constexpr int kRowsPerBlock = 4;
__global__ void __launch_bounds__(kRowsPerBlock * kWave)
l2_kernel(float* __restrict__ x, int rows, int cols, float eps) {
    const int row = blockIdx.x * kRowsPerBlock + (int)(threadIdx.x / kWave);
    const int lane = threadIdx.x & (kWave - 1);
    if (row >= rows) return;                            // whole wave exits together
    float* p = x + (size_t)row * cols;
    double acc = 0.0;
    for (int i = lane; i < cols; i += kWave) acc += (double)p[i] * (double)p[i];
    acc = wave_sum_f64(acc);
    const float inv = (float)(1.0 / sqrt(acc + (double)eps));
    for (int i = lane; i < cols; i += kWave) p[i] *= inv;
}

// One wave per head (src/ix_gdn.cu:87-100).
__global__ void __launch_bounds__(kRowsPerBlock * kWave)
out_norm_kernel(const float* __restrict__ o, const float* __restrict__ z, const float* __restrict__ nrm,
                float* __restrict__ y, int h_v, int S, float eps) {
    const int h = blockIdx.x * kRowsPerBlock + (int)(threadIdx.x / kWave);
    const int lane = threadIdx.x & (kWave - 1);
    if (h >= h_v) return;
    const float* po = o + (size_t)h * S;
    const float* pz = z + (size_t)h * S;
    float* py = y + (size_t)h * S;
    double acc = 0.0;
    for (int i = lane; i < S; i += kWave) acc += (double)po[i] * (double)po[i];
    acc = wave_sum_f64(acc);
    const float inv = (float)(1.0 / sqrt(acc / (double)S + (double)eps));
    for (int i = lane; i < S; i += kWave) py[i] = po[i] * inv * nrm[i] * sigmoid_f(pz[i]);
}

__global__ void __launch_bounds__(256) beta_kernel(float* __restrict__ beta, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) beta[i] = sigmoid_f(beta[i]);
}

}  // namespace
}  // namespace ixg

extern "C" {

hipError_t ix_gdn_step(float* state, const float* q, const float* k, const float* v, const float* gate,
                       const float* beta, float* o, int S, int h_k, int h_v, hipStream_t s) {
    if (S <= 0 || h_k <= 0 || h_v <= 0 || S > ixg::kStepMaxS) return hipErrorInvalidValue;  // src/ix_gdn.cu:110
    hipLaunchKernelGGL(ixg::step_kernel, dim3((unsigned)h_v), dim3(ixg::kStepThreads), 0, s,
                       state, q, k, v, gate, beta, o, S, h_k, h_v);
    return hipGetLastError();
}

hipError_t ix_gdn_conv_step(float* conv_state, const float* x, const float* kW, float* out, int channels,
                            int d_conv, hipStream_t s) {
    if (channels <= 0 || d_conv < 2) return hipErrorInvalidValue;                           // src/ix_gdn.cu:117
    hipLaunchKernelGGL(ixg::conv_kernel, dim3((unsigned)((channels + 255) / 256)), dim3(256), 0, s,
                       conv_state, x, kW, out, channels, d_conv);
    return hipGetLastError();
}

hipError_t ix_gdn_l2_norm(float* x, int rows, int cols, float eps, hipStream_t s) {
    if (rows <= 0 || cols <= 0 || cols > 1024) return hipErrorInvalidValue;                  // src/ix_gdn.cu:122
    hipLaunchKernelGGL(ixg::l2_kernel, dim3((unsigned)((rows + ixg::kRowsPerBlock - 1) / ixg::kRowsPerBlock)),
                       dim3(ixg::kRowsPerBlock * ixg::kWave), 0, s, x, rows, cols, eps);
    return hipGetLastError();
}

hipError_t ix_gdn_beta_gate(float* beta, int h_v, hipStream_t s) {
    if (beta == nullptr || h_v <= 0) return hipErrorInvalidValue;                            // src/ix_gdn.cu:127
    hipLaunchKernelGGL(ixg::beta_kernel, dim3((unsigned)((h_v + 255) / 256)), dim3(256), 0, s, beta, h_v);
    return hipGetLastError();
}

hipError_t ix_gdn_out_norm(const float* o, const float* z, const float* ssm_norm, float* y, int h_v, int S,
                           float eps, hipStream_t s) {
    if (h_v <= 0 || S <= 0) return hipErrorInvalidValue;                                     // src/ix_gdn.cu:133
    hipLaunchKernelGGL(ixg::out_norm_kernel, dim3((unsigned)((h_v + ixg::kRowsPerBlock - 1) / ixg::kRowsPerBlock)),
                       dim3(ixg::kRowsPerBlock * ixg::kWave), 0, s, o, z, ssm_norm, y, h_v, S, eps);
    return hipGetLastError();
}

}  // extern "C"
