// gdn_inproj.hip -- the GDN layer's input projection on gfx950 bf16 MFMA (ix_gdn_in_proj).
//
// For B token rows of hidden states h [B][K] and the projection weight W [N][K] (one row per
// output, as the reference's GEMV weights, src/ix_bf16_gemv.cu:36), computes
//   y = h W^T,  N = C + h_v*d_v + 2*h_v  (C = 2 h_k d_k + h_v d_v)
// with fp32 accumulation, and writes the four pieces a GDN layer consumes as bf16 (round to
// nearest even): the mixed conv input x [B][C] (columns 0..C), the output-gate logits
// z [B][h_v][d_v], and the gate and beta logits a, b [B][h_v]. This is the step to the left
// of the recurrence that the reference runs as per-token bf16 GEMVs.
//
// At decode batch sizes the product is a skinny GEMM that streams W once from HBM (about 2
// FLOP per weight byte at B = 64), so the work is moving bytes, not MFMA throughput. One
// workgroup owns 64 output columns and 64 rows; its 8 waves split K into contiguous ranges,
// and each wave runs v_mfma_f32_16x16x32_bf16 on all 4 x 4 tiles of the 64 x 64 output with
// operands loaded straight from memory. The k-slots of the instruction are filled so that a
// lane's two consecutive k-steps are adjacent in memory: for a 64-k super-step, lanes
// 16 g .. 16 g + 15 hold k = 16 g .. 16 g + 15 of their row (8 for each of two MFMAs), so four
// lanes read one full 128-byte line of each row per super-step. A and B use the same slot
// assignment, so the products are unchanged. The 8 partial tiles are added in wave order
// through LDS, so the result does not depend on timing.
#include "gdn_common.h"

namespace ixg {
namespace {

constexpr int kNt = 64;                 // output columns per workgroup (4 MFMA n-tiles)
constexpr int kMt = 64;                 // rows per workgroup (4 MFMA m-tiles)
constexpr int kWaves = 8;               // contiguous K ranges
constexpr int kSuper = 64;              // k per super-step (two MFMA k-steps)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct InProj {
    const uint16_t* h;          // [B][K]
    const uint16_t* w;          // [N][K]
    uint16_t* x;                // [B][C]
    uint16_t* z;                // [B][Z]
    uint16_t* a;                // [B][h_v]
    uint16_t* b;                // [B][h_v]
    float* y;                   // [B][N] fp32, or null
    int B, K, N, C, Z, hv;
};

__device__ __forceinline__ void store_out(const InProj& p, int row, int col, float v) {
    const uint16_t u = f32_to_bf16(v);
    if (col < p.C) p.x[(size_t)row * p.C + col] = u;
    else if (col < p.C + p.Z) p.z[(size_t)row * p.Z + (col - p.C)] = u;
    else if (col < p.C + p.Z + p.hv) p.a[(size_t)row * p.hv + (col - p.C - p.Z)] = u;
    else p.b[(size_t)row * p.hv + (col - p.C - p.Z - p.hv)] = u;
    if (p.y) p.y[(size_t)row * p.N + col] = v;
}

__global__ void __launch_bounds__(kWaves * kWave) in_proj_kernel(const InProj p) {
    __shared__ float red[kWaves][kMt][kNt + 1];

    const int tid = threadIdx.x, wv = tid / kWave, lane = tid & (kWave - 1);
    const int r16 = lane & 15, kg = lane >> 4;
    const int n0 = blockIdx.x * kNt, m0 = blockIdx.y * kMt;
    const int nsup = p.K / kSuper;                                   // super-steps in K
    const int s_lo = wv * nsup / kWaves, s_hi = (wv + 1) * nsup / kWaves;

    // Operand rows of this lane (clamped into range: rows and columns past the end compute
    // values that are never stored).
    const bf16x8* ap[4];
    const bf16x8* bp[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = min(m0 + 16 * i + r16, p.B - 1), c = min(n0 + 16 * i + r16, p.N - 1);
        ap[i] = reinterpret_cast<const bf16x8*>(p.h + (size_t)r * p.K + 16 * kg);
        bp[i] = reinterpret_cast<const bf16x8*>(p.w + (size_t)c * p.K + 16 * kg);
    }

    f32x4 acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll 2
    for (int sp = s_lo; sp < s_hi; ++sp) {
        bf16x8 av[4][2], bv[4][2];
        const int o = sp * (kSuper / 8);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int q = 0; q < 2; ++q) { bv[i][q] = bp[i][o + q]; av[i][q] = ap[i][o + q]; }
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int ni = 0; ni < 4; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[mi][q], bv[ni][q], acc[mi][ni], 0, 0, 0);
    }

    // acc[mi][ni][r] is output (row 16 mi + 4 kg + r, column 16 ni + r16) of this wave's K range.
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wv][16 * mi + 4 * kg + r][16 * ni + r16] = acc[mi][ni][r];
    __syncthreads();
    // 4096 outputs, 8 per thread: row tid / 8, columns 8 (tid % 8) .. +7.
    const int row = tid >> 3, c0 = 8 * (tid & 7);
    if (m0 + row < p.B) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int col = n0 + c0 + e;
            if (col < p.N) {
                float v = red[0][row][c0 + e];
#pragma unroll
                for (int q = 1; q < kWaves; ++q) v += red[q][row][c0 + e];
                store_out(p, m0 + row, col, v);
            }
        }
    }
}

}  // namespace
}  // namespace ixg

extern "C" hipError_t ix_gdn_check_cfg_(const ix_gdn_cfg* c);

extern "C" int ix_gdn_in_proj_width(const ix_gdn_cfg* cfg) {
    if (ix_gdn_check_cfg_(cfg) != hipSuccess) return 0;
    return 2 * cfg->h_k * cfg->d_k + cfg->h_v * cfg->d_v + cfg->h_v * cfg->d_v + 2 * cfg->h_v;
}

extern "C" hipError_t ix_gdn_in_proj(const ix_gdn_cfg* cfg, int B, int hidden, const uint16_t* h, const uint16_t* w,
                                     uint16_t* x, uint16_t* z, uint16_t* a, uint16_t* b, float* y, hipStream_t s) {
    using namespace ixg;
    const hipError_t e = ix_gdn_check_cfg_(cfg);
    if (e != hipSuccess) return e;
    if (B <= 0 || B > 65535 * kMt || hidden <= 0 || hidden % kSuper != 0) return hipErrorInvalidValue;
    if (!h || !w || !x || !z || !a || !b) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(w)) & 15) return hipErrorInvalidValue;
    if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(a) |
          reinterpret_cast<uintptr_t>(b)) & 1) || (reinterpret_cast<uintptr_t>(y) & 3))
        return hipErrorInvalidValue;
    InProj p;
    p.h = h; p.w = w; p.x = x; p.z = z; p.a = a; p.b = b; p.y = y;
    p.B = B; p.K = hidden;
    p.C = 2 * cfg->h_k * cfg->d_k + cfg->h_v * cfg->d_v;
    p.Z = cfg->h_v * cfg->d_v;
    p.hv = cfg->h_v;
    p.N = p.C + p.Z + 2 * p.hv;
    const dim3 grid((unsigned)((p.N + kNt - 1) / kNt), (unsigned)((B + kMt - 1) / kMt));
    hipLaunchKernelGGL(in_proj_kernel, grid, dim3(kWaves * kWave), 0, s, p);
    return hipGetLastError();
}
