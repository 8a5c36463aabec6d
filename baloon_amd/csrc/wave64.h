// wave64.h -- CDNA4 (gfx950) wavefront primitives for the GDN kernels.
//
// Replaces the role of the reference's src/ix_compat.h (IX_WARP_SIZE and the 64-lane
// butterfly reductions, ix_compat.h:12, :22-46, and ix_bf16_to_f32, :158-163) with native
// gfx950 code: DPP row operations for the in-row steps, v_permlane16_swap /
// v_permlane32_swap for the cross-row steps, and the hardware bf16 convert.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// Every kernel here is written for gfx950 alone: wave64, the gfx950 MFMA shapes and
// transposing LDS reads, hand-encoded s_waitcnt fields, and a decode counter hand-off that
// relies on this target's in-order wave issue (see gdn_decode.hip).
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "libixgdn device code targets gfx950 only"
#endif

namespace ixg {

constexpr int kWave = 64;

// DPP controls (GCN/CDNA encoding).
constexpr int kDppQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141; // lane i <- 7-i within each 8 lanes
constexpr int kDppRowMirror = 0x140;     // lane i <- 15-i within each 16-lane row
constexpr int kDppRowRor8 = 0x128;       // lane i <- lane (i + 8) mod 16 within each row (= i ^ 8)

template <int Ctrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xF, 0xF, false));
}

// v[l] + v[l ^ 32] in every lane (v_permlane32_swap: the two results hold the lower half
// swapped up and the upper half swapped down; their sum is the pair sum in both halves).
__device__ __forceinline__ float pair_sum32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// v[l] + v[l ^ 16] in every lane (v_permlane16_swap on 16-lane rows).
__device__ __forceinline__ float pair_sum16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over the 16 lanes of each row, result in every lane of the row.
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp_f32<kDppQuadXor1>(v);
    v += dpp_f32<kDppQuadXor2>(v);
    v += dpp_f32<kDppRowHalfMirror>(v);
    v += dpp_f32<kDppRowMirror>(v);
    return v;
}

// Sum over all 64 lanes, result in every lane.
__device__ __forceinline__ float wave_sum(float v) {
    return pair_sum32(pair_sum16(row_sum16(v)));
}

// Sixteen 64-lane sums at once, as a reduce-scatter: at lane distance 32, 16, 8 and 4 each
// step exchanges half of the remaining partial sums with the partner lane (which keeps the
// other half), so no partial sum is formed twice; the last two steps add within each quad.
// Lane l returns the total of v[l >> 2] (bit 5 of l picks bit 3 of the index, bit 4 bit 2,
// bit 3 bit 1, bit 2 bit 0). About 60 instructions against 16 x 8 for separate sums.
__device__ __forceinline__ float sum16_scatter(const float (&v)[16], int lane) {
    float a[8], b[4], c[2];
#pragma unroll
    for (int t = 0; t < 8; ++t) {            // lanes 0-31 keep index t, lanes 32-63 t + 8
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[t]), __float_as_uint(v[t + 8]), false, false);
        a[t] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {            // even rows keep index j, odd rows j + 4
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[j]), __float_as_uint(a[j + 4]), false, false);
        b[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    const bool h8 = lane & 8, h4 = lane & 4;
#pragma unroll
    for (int k = 0; k < 2; ++k) {            // lanes i ^ 8 within each row
        const float own = h8 ? b[k + 2] : b[k], send = h8 ? b[k] : b[k + 2];
        c[k] = own + dpp_f32<kDppRowRor8>(send);
    }
    const float own = h4 ? c[1] : c[0], send = h4 ? c[0] : c[1];
    float d = own + dpp_f32<kDppRowHalfMirror>(send);     // lanes i and 7 - i of each 8
    d += dpp_f32<kDppQuadXor1>(d);
    d += dpp_f32<kDppQuadXor2>(d);
    return d;
}

// Workgroup barrier that orders LDS accesses only. __syncthreads() also orders global
// memory, which makes every wave wait for all of its outstanding global loads (vmcnt(0))
// before the barrier -- including loads issued early on purpose to prefetch later work.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Orders one wave's LDS accesses across its lanes: reads issued after this point see the
// writes the wave's other lanes issued before it. A wave's LDS operations execute in issue
// order, so this only keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Double-precision 64-lane sum, result in every lane (xor butterfly on ds_swizzle/bpermute).
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// bf16 <-> fp32. bf16 -> fp32 is exact; fp32 -> bf16 uses the gfx950 hardware convert,
// round to nearest even.
__device__ __forceinline__ float bf16_to_f32(uint16_t u) { return __uint_as_float((uint32_t)u << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
// Two values in one v_cvt_pk_bf16_f32 (a vector conversion; packing two scalar conversions
// costs two converts and a merge).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// Scalar math with the reference's definitions (src/ix_gdn.cu:22-23).
__device__ __forceinline__ float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

}  // namespace ixg
