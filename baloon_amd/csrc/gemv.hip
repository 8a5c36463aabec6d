// gemv.hip -- matrix-vector products feeding the GDN layer on gfx950: the bf16 GEMV family
// (ix_bf16_gemv, _pair, _split) and the Q8_0 x q8_1 product (ix_mmvq_q8_0).
//
// Drop-ins for the reference's src/ix_bf16_gemv.cu:97-126 and src/ix_mmvq_wave.cu:100-123:
// same names, argument order and meaning, same validation, fp32 results. The kernels are
// gfx950 designs: one wave64 per output row streaming the row in 16-byte loads (8 bf16 per
// lane) when the row is 16-byte aligned, and a 64-lane DPP/permlane reduction. As in the
// reference, results agree with a double reference within float tolerance (summation order
// is this build's own), and the pair product gives bit-identical results to the single one.
#include "gdn_common.h"

#include <algorithm>

namespace ixg {
namespace {

constexpr int kGemvThreads = 256;
constexpr int kRowsPerBlock = kGemvThreads / kWave;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// Partial dot product of one lane over a row: 8 values per 16-byte load when vec, else one
// value per step. The lane's partial is the same whichever kernel calls it.
__device__ __forceinline__ float row_partial(const uint16_t* __restrict__ x, const uint16_t* __restrict__ row,
                                             long long n_in, int lane, int step_lanes, bool vec) {
    float acc = 0.0f;
    if (vec) {
        const long long n8 = n_in >> 3;
        for (long long i = lane; i < n8; i += step_lanes) {
            const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row) + i);
            const u32x4 v = *(reinterpret_cast<const u32x4*>(x) + i);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc = fmaf(bf_lo(v[e]), bf_lo(w[e]), acc);
                acc = fmaf(bf_hi(v[e]), bf_hi(w[e]), acc);
            }
        }
    } else {
        for (long long i = lane; i < n_in; i += step_lanes) acc = fmaf(bf16_to_f32(x[i]), bf16_to_f32(row[i]), acc);
    }
    return acc;
}

// One wave per output row.
__global__ void __launch_bounds__(kGemvThreads)
gemv_wave_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, float* __restrict__ y,
                 long long n_in, long long n_out, bool vec) {
    const long long o = (long long)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave;
    if (o >= n_out) return;                                  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const float r = wave_sum(row_partial(x, w + o * n_in, n_in, lane, kWave, vec));
    if (lane == 0) y[o] = r;
}

// Two weight matrices against one x; row o of each with the same code as gemv_wave_kernel.
__global__ void __launch_bounds__(kGemvThreads)
gemv_pair_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1, float* __restrict__ y1,
                 long long n_out1, bool vec1, const uint16_t* __restrict__ w2, float* __restrict__ y2,
                 long long n_out2, bool vec2, long long n_in) {
    const long long o = (long long)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    if (o < n_out1) {
        const float r = wave_sum(row_partial(x, w1 + o * n_in, n_in, lane, kWave, vec1));
        if (lane == 0) y1[o] = r;
    }
    if (o < n_out2) {
        const float r = wave_sum(row_partial(x, w2 + o * n_in, n_in, lane, kWave, vec2));
        if (lane == 0) y2[o] = r;
    }
}

// tpr threads per row (a power of two other than 64). tpr < 64: 64/tpr rows per wave,
// reduced within lane groups; tpr > 64: one workgroup of tpr threads per row, reduced by
// waves and then through LDS.
__device__ __forceinline__ float group_sum(float v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__global__ void __launch_bounds__(kGemvThreads)
gemv_group_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, float* __restrict__ y,
                  long long n_in, long long n_out, int tpr, bool vec) {
    const int groups = kGemvThreads / tpr;
    const long long o = (long long)blockIdx.x * groups + threadIdx.x / tpr;
    const int t = threadIdx.x % tpr;
    float r = o < n_out ? row_partial(x, w + o * n_in, n_in, t, tpr, vec) : 0.0f;
    r = group_sum(r, tpr);                                   // every lane of the wave takes part
    if (o < n_out && t == 0) y[o] = r;
}

__global__ void __launch_bounds__(1024)
gemv_block_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, float* __restrict__ y,
                  long long n_in, int tpr, bool vec) {
    __shared__ float part[1024 / kWave];
    const long long o = blockIdx.x;
    const int t = threadIdx.x, lane = t & (kWave - 1), wv = t / kWave;
    const float r = wave_sum(row_partial(x, w + o * n_in, n_in, t, tpr, vec));
    if (lane == 0) part[wv] = r;
    __syncthreads();
    if (t == 0) {
        float s = part[0];
        for (int i = 1; i < tpr / kWave; ++i) s += part[i];
        y[o] = s;
    }
}

// ---------------------------------------------------------------------------------------
// Q8_0 weights x q8_1 activations (formats of src/ix_mmvq_wave.cu:22-25):
//   Q8_0 block: fp16 scale d, 32 int8 (34 bytes, 2-byte aligned); w [n_out][n_in/32]
//   q8_1 block: fp16 d, fp16 s (sum, unused by Q8_0), 32 int8 (36 bytes); x [ncols][n_in/32]
// y[c][r] = sum over blocks of d_w * d_x * (integer dot of the 32 pairs).
// One wave per row; each block is split over two lanes (16 values each: four v_dot4_i32_i8),
// the two integer halves are added exactly, then scaled once per block. Each column's sum is
// computed by the same code whatever the number of columns launched.
// ---------------------------------------------------------------------------------------
constexpr int kQ80Bytes = 34;                       // kQ81Bytes (36) is in gdn_common.h

__device__ __forceinline__ float half_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

template <int NC>
__global__ void __launch_bounds__(kGemvThreads)
mmvq_q8_0_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ x, float* __restrict__ y, int n_in,
                 int n_out) {
    const int row = blockIdx.x * kRowsPerBlock + threadIdx.x / kWave;
    if (row >= n_out) return;                                // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int nb = n_in / 32, hv = lane & 1;                 // hv: which 16 values of the block
    const uint8_t* wr = w + (size_t)row * nb * kQ80Bytes;
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = 0.0f;
    for (int kb = lane >> 1; kb < nb; kb += kWave / 2) {
        const uint8_t* wb = wr + (size_t)kb * kQ80Bytes;
        const uint16_t* wq = reinterpret_cast<const uint16_t*>(wb + 2 + 16 * hv);   // 2-byte aligned
        int wi[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) wi[i] = (int)((uint32_t)wq[2 * i] | ((uint32_t)wq[2 * i + 1] << 16));
        const float dw = half_to_f32(*reinterpret_cast<const uint16_t*>(wb));
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const uint8_t* xb = x + ((size_t)c * nb + kb) * kQ81Bytes;
            const int* xq = reinterpret_cast<const int*>(xb + 4 + 16 * hv);        // 4-byte aligned
            int s = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) s = __builtin_amdgcn_sdot4(wi[i], xq[i], s, false);
            s += __shfl_xor(s, 1, kWave);                    // the block's two halves, exactly
            const float dx = half_to_f32(*reinterpret_cast<const uint16_t*>(xb));
            if (hv == 0) acc[c] = fmaf(dw * dx, (float)s, acc[c]);
        }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const float r = wave_sum(acc[c]);
        if (lane == 0) y[(size_t)c * n_out + row] = r;
    }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
inline bool vec_rows(const uint16_t* x, const uint16_t* w, long long n_in) {
    return n_in % 8 == 0 && aligned16(x) && aligned16(w);
}
inline unsigned row_blocks(long long n_out) { return (unsigned)((n_out + kRowsPerBlock - 1) / kRowsPerBlock); }

// q8_1 quantiser: x [n] fp32 -> [n/32] q8_1 blocks; each wave takes 64 consecutive values
// (two blocks, one per half wave) per step, through the same q81_store as the gated epilogues.
__global__ void __launch_bounds__(256) q81_kernel(const float* __restrict__ x, uint8_t* __restrict__ y, long long nb) {
    const int lane = threadIdx.x & (kWave - 1);
    const long long waves = (long long)gridDim.x * (256 / kWave);
    for (long long wv = ((long long)blockIdx.x * 256 + threadIdx.x) / kWave; 2 * wv < nb; wv += waves) {
        const long long b = 2 * wv + (lane >> 5);            // this lane's block
        const bool live = b < nb;                             // false only in the upper half of the last wave
        const float v = live ? x[b * 32 + (lane & 31)] : 0.0f;
        q81_store(v, lane, live ? y + b * kQ81Bytes : nullptr);
    }
}

}  // namespace
}  // namespace ixg

using namespace ixg;

extern "C" hipError_t ix_bf16_gemv(const uint16_t* x, const uint16_t* w, float* y, long long n_in, long long n_out,
                                   hipStream_t s) {
    if (n_in <= 0 || n_out <= 0) return hipErrorInvalidValue;
    if ((n_out + kRowsPerBlock - 1) / kRowsPerBlock > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gemv_wave_kernel, dim3(row_blocks(n_out)), dim3(kGemvThreads), 0, s, x, w, y, n_in, n_out,
                       vec_rows(x, w, n_in));
    return hipGetLastError();
}

extern "C" hipError_t ix_bf16_gemv_pair(const uint16_t* x, const uint16_t* w1, float* y1, long long n_out1,
                                        const uint16_t* w2, float* y2, long long n_out2, long long n_in,
                                        hipStream_t s) {
    if (n_in <= 0 || (n_out1 <= 0 && n_out2 <= 0)) return hipErrorInvalidValue;
    const long long n_out = n_out1 > n_out2 ? n_out1 : n_out2;
    if ((n_out + kRowsPerBlock - 1) / kRowsPerBlock > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gemv_pair_kernel, dim3(row_blocks(n_out)), dim3(kGemvThreads), 0, s, x, w1, y1, n_out1,
                       vec_rows(x, w1, n_in), w2, y2, n_out2, vec_rows(x, w2, n_in), n_in);
    return hipGetLastError();
}

extern "C" hipError_t ix_bf16_gemv_split(const uint16_t* x, const uint16_t* w, float* y, long long n_in,
                                         long long n_out, int threads_per_row, hipStream_t s) {
    if (n_in <= 0 || n_out <= 0) return hipErrorInvalidValue;
    if (threads_per_row == kWave) return ix_bf16_gemv(x, w, y, n_in, n_out, s);     // one wave per row
    if (threads_per_row <= 0 || threads_per_row > 1024 || (threads_per_row & (threads_per_row - 1)) != 0)
        return hipErrorInvalidValue;
    const bool vec = vec_rows(x, w, n_in);
    if (threads_per_row < kWave) {
        const long long rows_per_block = kGemvThreads / threads_per_row;
        const long long blocks = (n_out + rows_per_block - 1) / rows_per_block;
        if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
        hipLaunchKernelGGL(gemv_group_kernel, dim3((unsigned)blocks), dim3(kGemvThreads), 0, s, x, w, y, n_in, n_out,
                           threads_per_row, vec);
    } else {
        if (n_out > 0x7fffffffLL) return hipErrorInvalidValue;
        hipLaunchKernelGGL(gemv_block_kernel, dim3((unsigned)n_out), dim3(threads_per_row), 0, s, x, w, y, n_in,
                           threads_per_row, vec);
    }
    return hipGetLastError();
}

extern "C" hipError_t ix_q8_1_quantize(const float* x, void* y_q8_1, long long n, hipStream_t s) {
    if (n <= 0 || n % 32 != 0 || !x || !y_q8_1) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(x) & 3) || (reinterpret_cast<uintptr_t>(y_q8_1) & 3)) return hipErrorInvalidValue;
    const long long nb = n / 32, waves = (nb + 1) / 2;
    const long long blocks = std::min<long long>((waves + 3) / 4, 65536);
    hipLaunchKernelGGL(ixg::q81_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, static_cast<uint8_t*>(y_q8_1), nb);
    return hipGetLastError();
}

extern "C" hipError_t ix_mmvq_q8_0(const void* weights, const void* x_q8_1, float* y, int n_in, int n_out, int ncols,
                                   hipStream_t s) {
    if (n_in <= 0 || n_in % 32 != 0 || n_out <= 0 || ncols < 1 || ncols > 8 || !weights || !x_q8_1 || !y)
        return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(weights) & 1) || (reinterpret_cast<uintptr_t>(x_q8_1) & 3) ||
        (reinterpret_cast<uintptr_t>(y) & 3))
        return hipErrorInvalidValue;                         // block alignment of the formats
    const auto* w = static_cast<const uint8_t*>(weights);
    const auto* x = static_cast<const uint8_t*>(x_q8_1);
    const dim3 grid(row_blocks(n_out)), block(kGemvThreads);
    switch (ncols) {
        case 1: hipLaunchKernelGGL(mmvq_q8_0_kernel<1>, grid, block, 0, s, w, x, y, n_in, n_out); break;
        case 2: hipLaunchKernelGGL(mmvq_q8_0_kernel<2>, grid, block, 0, s, w, x, y, n_in, n_out); break;
        case 3: hipLaunchKernelGGL(mmvq_q8_0_kernel<3>, grid, block, 0, s, w, x, y, n_in, n_out); break;
        case 4: hipLaunchKernelGGL(mmvq_q8_0_kernel<4>, grid, block, 0, s, w, x, y, n_in, n_out); break;
        case 5: hipLaunchKernelGGL(mmvq_q8_0_kernel<5>, grid, block, 0, s, w, x, y, n_in, n_out); break;
        case 6: hipLaunchKernelGGL(mmvq_q8_0_kernel<6>, grid, block, 0, s, w, x, y, n_in, n_out); break;
        case 7: hipLaunchKernelGGL(mmvq_q8_0_kernel<7>, grid, block, 0, s, w, x, y, n_in, n_out); break;
        default: hipLaunchKernelGGL(mmvq_q8_0_kernel<8>, grid, block, 0, s, w, x, y, n_in, n_out); break;
    }
    return hipGetLastError();
}
