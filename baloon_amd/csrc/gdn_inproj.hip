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
// workgroup owns a 64 x 64 output tile over the whole of K. Two producer waves copy 64-k
// stages of the tile's 64 activation rows (one wave) and 64 weight rows (the other) into a
// ring of LDS stages with direct global-to-LDS loads: every load instruction moves 1 KiB =
// 8 whole 128-byte row segments, and the loads of three stages are in flight at once.
// Eight consumer waves each own a 32 x 16 eighth of the tile and run
// v_mfma_f32_16x16x32_bf16 on operands read from the ring; they issue no LDS DMA, so the
// compiler never makes their LDS reads wait for the copies in flight. Producers and
// consumers meet at one barrier per stage. In LDS the 16-byte chunk c of tile row r sits
// at position c ^ (r & 7) of the row's 128 bytes, so the eight rows an operand read touches
// at once fall in different banks; the producers apply the swizzle by choosing which chunk
// each lane fetches. The summation order over K is fixed, so results do not depend on
// timing.
#include "gdn_common.h"

namespace ixg {
namespace {

constexpr int kNt = 64;                 // output columns per workgroup (4 MFMA n-tiles)
constexpr int kMt = 64;                 // rows per workgroup (4 MFMA m-tiles)
constexpr int kKd = 64;                 // k per stage (two MFMA k-steps)
constexpr int kRowB = 2 * kKd;          // bytes of one tile row per stage
constexpr int kRowsPerCopy = 1024 / kRowB;          // tile rows per 1 KiB load instruction
constexpr int kHalf = 64 * kRowB;       // bytes of one operand tile per stage
constexpr int kStage = 2 * kHalf;       // activation tile, then weight tile
constexpr int kRing = 4;                // stages in the LDS ring (64 KiB)
constexpr int kCons = 8, kProd = 2;     // consumer and producer waves
constexpr int kTM = 2, kTN = 1;         // 16 x 16 output tiles per consumer wave (rows, columns)
static_assert(2 * 16 * kTM == kMt && (kCons / 2) * 16 * kTN == kNt, "the consumer waves cover the tile");
constexpr int kCopies = 2 * (64 / kRowsPerCopy) / kProd;   // load instructions per producer and stage

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) uint8_t lds_u8;

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

// s_waitcnt that waits until at most N vector memory operations are outstanding, in the
// gfx9-family field layout (gfx950 here: vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt
// left at their maximum); another target would need its own encoding.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "wait_vmcnt encodes gfx950 s_waitcnt fields"
#endif
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Byte offset in an operand tile of 16-byte chunk c of row r.
__device__ __forceinline__ int ring_off(int r, int c) { return r * kRowB + ((c ^ (r & 7)) << 4); }

__global__ void __launch_bounds__((kCons + kProd) * kWave) in_proj_kernel(const InProj p) {
    __shared__ __align__(16) uint8_t lds[kRing * kStage];

    const int lane = threadIdx.x & (kWave - 1);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int n0 = blockIdx.x * kNt, m0 = blockIdx.y * kMt;
    const int nst = p.K / kKd;

    if (w >= kCons) {
        // Producer: the first half of the producer waves copy activation rows, the second
        // half weight rows, kCopies load instructions each. Instruction g of a tile covers
        // rows kRowsPerCopy g .. +kRowsPerCopy-1; lane l writes position l % (kRowB / 16) of
        // row kRowsPerCopy g + l / (kRowB / 16), so it fetches chunk position ^ (row & 7) of
        // that row. Rows past the end are clamped (their results are never stored).
        const int pw = w - kCons;
        const bool act = pw < kProd / 2;
        const int g0 = (pw % (kProd / 2)) * kCopies;          // first load instruction of this wave
        const int rr = lane / (kRowB / 16), pos = lane % (kRowB / 16);
        const uint8_t* src[kCopies];
#pragma unroll
        for (int j = 0; j < kCopies; ++j) {
            const int r = kRowsPerCopy * (g0 + j) + rr;
            const int chunk = pos ^ (r & 7);
            const int row = act ? min(m0 + r, p.B - 1) : min(n0 + r, p.N - 1);
            src[j] = reinterpret_cast<const uint8_t*>(act ? p.h : p.w) + (size_t)row * p.K * 2 + chunk * 16;
        }
        lds_u8* dst = (lds_u8*)lds + (act ? 0 : kHalf) + g0 * 1024;
        // Virtual stage v goes to ring slot v % kRing; stages past the end repeat the last one,
        // so every trip issues the same number of loads.
        auto issue = [&](int v) {
            const int sv = min(v, nst - 1);
            lds_u8* d = dst + (v % kRing) * kStage;
#pragma unroll
            for (int j = 0; j < kCopies; ++j) __builtin_amdgcn_global_load_lds(src[j] + sv * kRowB, d + j * 1024, 16, 0, 0);
        };
#pragma unroll
        for (int v = 0; v < kRing - 1; ++v) issue(v);
        wait_vmcnt<kCopies * (kRing - 2)>();                   // stage 0 landed
        __builtin_amdgcn_s_barrier();
        for (int st = 0; st < nst; ++st) {
            // The slot of stage st + kRing - 1 held stage st - 1, read before this barrier.
            issue(st + kRing - 1);
            wait_vmcnt<kCopies * (kRing - 2)>();               // stage st + 1 landed
            __builtin_amdgcn_s_barrier();
        }
        __builtin_amdgcn_s_waitcnt(0);
        return;
    }

    // Consumer wave w: rows 32 (w & 1) .. +31, columns 16 (w >> 1) .. +15 of the tile.
    const int li = lane & 15, lg = lane >> 4;
    const int rbase = 16 * kTM * (w & 1), cbase = 16 * kTN * (w >> 1);
    f32x4 acc[kTM][kTN];
#pragma unroll
    for (int mt = 0; mt < kTM; ++mt)
#pragma unroll
        for (int nt = 0; nt < kTN; ++nt) acc[mt][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // Operand offsets inside a stage: lane (li, lg) of k-step ks holds k = 32 ks + 8 lg .. +7
    // of its row (chunk 4 ks + lg).
    constexpr int kSteps = kKd / 32;
    int ao[kTM][kSteps], bo[kTN][kSteps];
#pragma unroll
    for (int ks = 0; ks < kSteps; ++ks) {
#pragma unroll
        for (int t = 0; t < kTM; ++t) ao[t][ks] = ring_off(rbase + 16 * t + li, 4 * ks + lg);
#pragma unroll
        for (int t = 0; t < kTN; ++t) bo[t][ks] = kHalf + ring_off(cbase + 16 * t + li, 4 * ks + lg);
    }
    lds_barrier();
    for (int st = 0; st < nst; ++st) {
        const uint8_t* sp = lds + (st % kRing) * kStage;
        bf16x8 av[kTM][kSteps], bv[kTN][kSteps];
#pragma unroll
        for (int ks = 0; ks < kSteps; ++ks) {
#pragma unroll
            for (int t = 0; t < kTM; ++t) av[t][ks] = *reinterpret_cast<const bf16x8*>(sp + ao[t][ks]);
#pragma unroll
            for (int t = 0; t < kTN; ++t) bv[t][ks] = *reinterpret_cast<const bf16x8*>(sp + bo[t][ks]);
        }
#pragma unroll
        for (int ks = 0; ks < kSteps; ++ks)
#pragma unroll
            for (int mt = 0; mt < kTM; ++mt)
#pragma unroll
                for (int nt = 0; nt < kTN; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[mt][ks], bv[nt][ks], acc[mt][nt], 0, 0, 0);
        lds_barrier();                                          // this slot may be refilled
    }

    // acc[mt][nt][r] is output (row rbase + 16 mt + 4 lg + r, column cbase + 16 nt + li).
#pragma unroll
    for (int mt = 0; mt < kTM; ++mt)
#pragma unroll
        for (int nt = 0; nt < kTN; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + rbase + 16 * mt + 4 * lg + r, col = n0 + cbase + 16 * nt + li;
                if (row < p.B && col < p.N) store_out(p, row, col, acc[mt][nt][r]);
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
    if (B <= 0 || B > 65535 * kMt || hidden <= 0 || hidden % kKd != 0) return hipErrorInvalidValue;
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
    hipLaunchKernelGGL(in_proj_kernel, grid, dim3((kCons + kProd) * kWave), 0, s, p);
    return hipGetLastError();
}
