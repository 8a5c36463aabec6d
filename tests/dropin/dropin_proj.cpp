// dropin_proj.cpp -- a compiled C++ caller of libixgdn.so's projection entry points through
// include/ix_gdn.h, written the way the reference's projection tests call their launchers:
//   tests/test_bf16_gemv.cu:27-38  ix_bf16_gemv, ix_bf16_gemv_split (64 and 32/128/256 threads
//                                  per row), ix_bf16_gemv_pair -- int sizes, stream defaulted
//   tests/test_mmvq_wave.cu:46     ix_mmvq::ix_mmvq_q8_0(dw, dx, dy, n_in, n_out, nc)
// with the same shape sweeps and checks: every GEMV within 2e-5 of the sum of |terms| of a
// double reference, the pair's first result bit-identical to the 64-thread split, the Q8_0
// product within 1e-5 of its double reference scaled by the sum of |terms|, and a column's
// Q8_0 result the same for 1 and 8 columns. Inputs come from std::mt19937 like the reference
// tests (its own seeds 5 and 20261029), so the shapes, magnitudes and block formats match.
//
//   dropin_proj --validate   the launchers' argument checks only; needs no GPU
//   dropin_proj              the checks above on the current GPU
// Exit status 0 means every check passed.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "ix_gdn.h"

namespace {

#define CK(expr)                                                                                \
    do {                                                                                        \
        const hipError_t e_ = (expr);                                                           \
        if (e_ != hipSuccess) {                                                                 \
            std::printf("HIP error %s at line %d: %s\n", hipGetErrorString(e_), __LINE__, #expr); \
            std::exit(2);                                                                       \
        }                                                                                       \
    } while (0)

uint16_t f2bf(float f) {   // round to nearest even
    uint32_t b;
    std::memcpy(&b, &f, 4);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}
float bf2f(uint16_t h) {
    const uint32_t b = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}
uint16_t half_bits(float f) {   // exact for the k/1024 scales drawn below
    const _Float16 h = (_Float16)f;
    uint16_t u;
    std::memcpy(&u, &h, 2);
    return u;
}
float half_val(uint16_t u) {
    _Float16 h;
    std::memcpy(&h, &u, 2);
    return (float)h;
}

int worst_of(const char* name, int nin, int nout, const std::vector<float>& y, const std::vector<double>& ref,
             const std::vector<double>& mag) {
    int bad = 0;
    double worst = 0;
    for (size_t o = 0; o < ref.size(); ++o) {
        const double e = std::fabs((double)y[o] - ref[o]) / (2e-5 * mag[o] + 1e-30);
        worst = std::fmax(worst, e);
        bad += e > 1.0;
    }
    std::printf("%-18s n_in=%-5d n_out=%-5d bad=%d worst_err/tol=%.3f\n", name, nin, nout, bad, worst);
    return bad;
}

template <class T>
T* dev_copy(const std::vector<T>& h) {
    T* p = nullptr;
    CK(hipMalloc(&p, h.size() * sizeof(T)));
    CK(hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return p;
}
std::vector<float> host_copy(const float* d, size_t n) {
    std::vector<float> h(n);
    CK(hipMemcpy(h.data(), d, n * sizeof(float), hipMemcpyDeviceToHost));
    return h;
}

int gemv_checks() {
    int bad = 0;
    std::mt19937 rng(5);
    std::normal_distribution<float> nd(0.f, 1.f);
    for (int nin : {2560, 5120, 100, 63, 64, 65})
        for (int nout : {1, 48, 64, 130, 1000}) {
            std::vector<uint16_t> x(nin), w((size_t)nin * nout), w2((size_t)nin * (nout + 17));
            for (auto& v : x) v = f2bf(nd(rng));
            for (auto& v : w) v = f2bf(nd(rng) * 0.05f);
            for (auto& v : w2) v = f2bf(nd(rng) * 0.05f);
            std::vector<double> ref(nout), mag(nout), ref2(nout + 17), mag2(nout + 17);
            for (int o = 0; o < nout; ++o)
                for (int i = 0; i < nin; ++i) {
                    const double p = (double)bf2f(x[i]) * bf2f(w[(size_t)o * nin + i]);
                    ref[o] += p;
                    mag[o] += std::fabs(p);
                }
            for (int o = 0; o < nout + 17; ++o)
                for (int i = 0; i < nin; ++i) {
                    const double p = (double)bf2f(x[i]) * bf2f(w2[(size_t)o * nin + i]);
                    ref2[o] += p;
                    mag2[o] += std::fabs(p);
                }
            uint16_t *dx = dev_copy(x), *dw = dev_copy(w), *dw2 = dev_copy(w2);
            float *dy, *dy1, *dy2, *dyw;
            CK(hipMalloc(&dy, nout * 4));
            CK(hipMalloc(&dy1, nout * 4));
            CK(hipMalloc(&dy2, (nout + 17) * 4));
            CK(hipMalloc(&dyw, nout * 4));
            // the reference test's calls, in its order
            CK(ix_bf16_gemv(dx, dw, dy, nin, nout));
            CK(hipDeviceSynchronize());
            bad += worst_of("gemv(entry)", nin, nout, host_copy(dy, nout), ref, mag);
            CK(ix_bf16_gemv_split(dx, dw, dyw, nin, nout, 64));
            CK(hipDeviceSynchronize());
            const std::vector<float> yw = host_copy(dyw, nout);
            bad += worst_of("split(64)=warp", nin, nout, yw, ref, mag);
            for (int tpr : {32, 128, 256}) {
                CK(ix_bf16_gemv_split(dx, dw, dy, nin, nout, tpr));
                CK(hipDeviceSynchronize());
                char nm[32];
                std::snprintf(nm, sizeof nm, "split(%d)", tpr);
                bad += worst_of(nm, nin, nout, host_copy(dy, nout), ref, mag);
            }
            CK(ix_bf16_gemv_pair(dx, dw, dy1, nout, dw2, dy2, nout + 17, nin));
            CK(hipDeviceSynchronize());
            const std::vector<float> y1 = host_copy(dy1, nout), y2 = host_copy(dy2, nout + 17);
            int pb = 0;
            for (int o = 0; o < nout; ++o) pb += std::memcmp(&y1[o], &yw[o], 4) != 0;
            bad += pb + worst_of("pair.y2", nin, nout + 17, y2, ref2, mag2);
            std::printf("%-18s n_in=%-5d n_out=%-5d bitwise mismatches vs split(64)=%d\n", "pair.y1", nin, nout, pb);
            (void)hipFree(dx); (void)hipFree(dw); (void)hipFree(dw2);
            (void)hipFree(dy); (void)hipFree(dy1); (void)hipFree(dy2); (void)hipFree(dyw);
        }
    return bad;
}

// Q8_0 weight block (34 bytes: fp16 d, 32 int8) and q8_1 activation block (36 bytes: fp16 d,
// fp16 s, 32 int8), packed as the formats of src/ix_mmvq_wave.cu:20-25 lay them out.
int mmvq_checks() {
    std::mt19937 rng(20261029);
    long cases = 0, fail_ref = 0, fail_cols = 0;
    for (int n_in : {32, 96, 256, 2048, 4096, 7 * 32})
        for (int n_out : {1, 3, 4, 5, 100, 333}) {
            const int bpr = n_in / 32, ncols = 8;
            std::vector<uint8_t> wp((size_t)n_out * bpr * 34), xp((size_t)ncols * bpr * 36);
            std::vector<float> wd((size_t)n_out * bpr), xd((size_t)ncols * bpr);
            std::vector<int8_t> wq((size_t)n_out * bpr * 32), xq((size_t)ncols * bpr * 32);
            for (size_t b = 0; b < wd.size(); ++b) {
                const uint16_t d = half_bits(float(1 + rng() % 2047) / 1024.f);
                wd[b] = half_val(d);
                std::memcpy(&wp[b * 34], &d, 2);
                for (int i = 0; i < 32; ++i) wq[b * 32 + i] = int8_t(int(rng() % 255) - 127);
                std::memcpy(&wp[b * 34 + 2], &wq[b * 32], 32);
            }
            for (size_t b = 0; b < xd.size(); ++b) {
                const uint16_t d = half_bits(float(1 + rng() % 2047) / 1024.f), s = 0;
                xd[b] = half_val(d);
                std::memcpy(&xp[b * 36], &d, 2);
                std::memcpy(&xp[b * 36 + 2], &s, 2);
                for (int i = 0; i < 32; ++i) xq[b * 32 + i] = int8_t(int(rng() % 255) - 127);
                std::memcpy(&xp[b * 36 + 4], &xq[b * 32], 32);
            }
            uint8_t *dw = dev_copy(wp), *dx = dev_copy(xp);
            float* dy;
            CK(hipMalloc(&dy, sizeof(float) * n_out * ncols));
            std::vector<float> y8, y1;
            for (int nc : {8, 1, 3}) {
                CK(hipMemset(dy, 0xFF, sizeof(float) * n_out * ncols));
                CK(ix_mmvq::ix_mmvq_q8_0(dw, dx, dy, n_in, n_out, nc));
                CK(hipDeviceSynchronize());
                const std::vector<float> y = host_copy(dy, (size_t)n_out * nc);
                if (nc == 8) y8 = y;
                if (nc == 1) y1 = y;
                for (int c = 0; c < nc; ++c)
                    for (int r = 0; r < n_out; ++r) {
                        ++cases;
                        double ref = 0, sc = 0;
                        for (int k = 0; k < bpr; ++k) {
                            const size_t wb = (size_t)r * bpr + k, xb = (size_t)c * bpr + k;
                            long dot = 0;
                            for (int i = 0; i < 32; ++i) dot += (long)wq[wb * 32 + i] * xq[xb * 32 + i];
                            ref += (double)wd[wb] * xd[xb] * dot;
                            sc += std::fabs((double)wd[wb] * xd[xb]) * 32 * 127 * 127;
                        }
                        if (!(std::fabs(y[(size_t)c * n_out + r] - ref) / sc <= 1e-5)) ++fail_ref;
                    }
            }
            for (int r = 0; r < n_out; ++r) fail_cols += std::memcmp(&y1[r], &y8[r], 4) != 0;
            (void)hipFree(dw); (void)hipFree(dx); (void)hipFree(dy);
        }
    std::printf("mmvq_q8_0 cases=%ld ref_fail=%ld column_dependence=%ld\n", cases, fail_ref, fail_cols);
    return (int)(fail_ref + fail_cols);
}

// The launchers refuse what the reference's launchers refuse (src/ix_bf16_gemv.cu:92, :106,
// :115, :121; src/ix_mmvq_wave.cu:103-105), before any device work.
int validate() {
    int bad = 0;
    auto want_invalid = [&](const char* what, hipError_t e) {
        const bool ok = e == hipErrorInvalidValue;
        std::printf("%-36s %s\n", what, ok ? "ok" : "FAIL");
        bad += !ok;
    };
    const uint16_t* nx = nullptr;
    float* ny = nullptr;
    want_invalid("gemv n_in=0", ix_bf16_gemv(nx, nx, ny, 0, 64));
    want_invalid("gemv n_out=0", ix_bf16_gemv(nx, nx, ny, 64, 0));
    want_invalid("gemv_pair both n_out<=0", ix_bf16_gemv_pair(nx, nx, ny, 0, nx, ny, 0, 64));
    want_invalid("gemv_split threads_per_row=48", ix_bf16_gemv_split(nx, nx, ny, 64, 64, 48));
    want_invalid("gemv_split threads_per_row=2048", ix_bf16_gemv_split(nx, nx, ny, 64, 64, 2048));
    want_invalid("ix_mmvq::ix_mmvq_q8_0 n_in=48", ix_mmvq::ix_mmvq_q8_0(nullptr, nullptr, ny, 48, 4, 1));
    want_invalid("ix_mmvq::ix_mmvq_q8_0 ncols=9", ix_mmvq::ix_mmvq_q8_0(nullptr, nullptr, ny, 64, 4, 9));
    want_invalid("ix_mmvq::ix_mmvq_q8_0 NULL weights", ix_mmvq::ix_mmvq_q8_0(nullptr, nullptr, ny, 64, 4, 1));
    return bad;
}

}  // namespace

int main(int argc, char** argv) {
    int bad = validate();
    if (argc > 1 && std::strcmp(argv[1], "--validate") == 0) {
        std::printf("drop-in projection caller (validation only): %s\n", bad ? "FAIL" : "PASS");
        return bad != 0;
    }
    bad += gemv_checks();
    bad += mmvq_checks();
    std::printf("drop-in projection caller, libixgdn %s: %s\n", ix_gdn_version(), bad ? "FAIL" : "PASS");
    return bad != 0;
}
