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
// loads per thread) and launches ceil(S/64) x h_v 64-thread blocks. Here the columns of a
// head are independent units of the update,
//   u_j = g S_j . k,  d_j = beta (v_j - u_j),  S_j' = g S_j + d_j k,  o_j = g S_j . q + d_j (k . q)
// (the output identity gives both contractions in one sweep), so a 256-thread workgroup
// owns a 32-column slice of one head: each thread holds one column of every eighth row in
// registers (every wave load is two 128-byte row segments), each element is read once and
// written once, and the two column sums are reduced in-thread and then over the slice's 8
// row groups through LDS. At the reference's shapes (S = 128, h_v = 48) that is 192
// workgroups instead of 48.
#include "ix_gdn.h"
#include "wave64.h"

namespace ixg {
namespace {

constexpr int kStepThreads = 256;
constexpr int kStepMaxS = 128;
constexpr int kStepSlice = 32;                               // columns per workgroup
constexpr int kStepGroups = kStepThreads / kStepSlice;       // 8 row groups
constexpr int kStepRows = kStepMaxS / kStepGroups;           // 16 rows per thread (i = r + 8 m)

__global__ void __launch_bounds__(kStepThreads)
step_kernel(float* __restrict__ state, const float* __restrict__ q, const float* __restrict__ k,
            const float* __restrict__ v, const float* __restrict__ gate, const float* __restrict__ beta,
            float* __restrict__ o, int S, int h_k, int h_v) {
    __shared__ float ks[kStepMaxS], qs[kStepMaxS];
    __shared__ float red[2][kStepGroups][kStepSlice];
    __shared__ float kq_part[kStepThreads / kWave];

    const int h = blockIdx.x;
    const int src = h % h_k;                           // modulo head pairing, src/ix_gdn.cu:38
    const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
    const int jj = tid & (kStepSlice - 1), r = tid / kStepSlice;
    const int j = blockIdx.y * kStepSlice + jj;
    const bool col = j < S;
    const size_t row_stride = (size_t)h_v * S;         // layout [S][h_v][S], src/ix_gdn.cu:47-48
    float* base = state + (size_t)h * S + j;

    // Issue every state load of this thread first; they overlap the staging below.
    float s[kStepRows];
#pragma unroll
    for (int m = 0; m < kStepRows; ++m) {
        const int i = r + kStepGroups * m;
        s[m] = (col && i < S) ? base[(size_t)i * row_stride] : 0.0f;
    }
    if (tid < S) { ks[tid] = k[(size_t)src * S + tid]; qs[tid] = q[(size_t)src * S + tid]; }
    const float g = expf(gate[h]);                     // decay, src/ix_gdn.cu:40
    const float bt = beta[h];
    const float vj = col ? v[(size_t)h * S + j] : 0.0f;
    __syncthreads();

    // k . q for the output identity: wave w covers indices 64 w .. 64 w + 63.
    {
        const float p = (tid < S) ? ks[tid] * qs[tid] : 0.0f;
        const float t = wave_sum(p);
        if (lane == 0) kq_part[w] = t;
    }
    float ak = 0.0f, aq = 0.0f;
#pragma unroll
    for (int m = 0; m < kStepRows; ++m) {
        const int i = r + kStepGroups * m;
        const float ki = (i < S) ? ks[i] : 0.0f, qi = (i < S) ? qs[i] : 0.0f;
        ak = fmaf(s[m], ki, ak);
        aq = fmaf(s[m], qi, aq);
    }
    red[0][r][jj] = ak;
    red[1][r][jj] = aq;
    __syncthreads();

    float A = 0.0f, Bq = 0.0f;
#pragma unroll
    for (int g8 = 0; g8 < kStepGroups; ++g8) { A += red[0][g8][jj]; Bq += red[1][g8][jj]; }
    const float kq = (kq_part[0] + kq_part[1]) + (kq_part[2] + kq_part[3]);
    const float d = (vj - g * A) * bt;
    if (r == 0 && col) o[(size_t)h * S + j] = fmaf(d, kq, g * Bq);
    if (!col) return;
#pragma unroll
    for (int m = 0; m < kStepRows; ++m) {
        const int i = r + kStepGroups * m;
        if (i < S) base[(size_t)i * row_stride] = fmaf(ks[i], d, s[m] * g);
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
    const dim3 grid((unsigned)h_v, (unsigned)((S + ixg::kStepSlice - 1) / ixg::kStepSlice));
    hipLaunchKernelGGL(ixg::step_kernel, grid, dim3(ixg::kStepThreads), 0, s, state, q, k, v, gate, beta, o, S, h_k,
                       h_v);
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
