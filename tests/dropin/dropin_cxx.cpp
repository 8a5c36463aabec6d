// dropin_cxx.cpp -- a compiled C++ caller of libixgdn.so through include/ix_gdn.h.
//
// It makes the reference acceptance test's five launcher calls (tests/test_gdn.cu:28, :39,
// :46, :51, :55) the way that test makes them: positional arguments with the stream left to
// its default (ix_gdn.h gives C++ callers the reference's `s = 0`), a device synchronise
// after each. Inputs come from the reference test's generator -- std::mt19937 seeded with 9
// and std::normal_distribution<float>, drawn in the same order and scaled the same way
// (tests/test_gdn.cu:15, :20-21, :34, :44, :48, :54) -- so with the same C++ standard library
// they are the same values. Every result is compared with the CPU oracle's double reference
// (oracle/liboracle.so, test infrastructure) under the reference test's norm
// max|gpu - ref| <= tol * max|ref| (tests/test_gdn.cu:10-13) and its tolerances.
//
//   dropin_cxx --validate   the launchers' shape checks only; needs no GPU
//   dropin_cxx              the reference test's checks on the current GPU
// Exit status 0 means every check passed.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "gdn_oracle.h"
#include "ix_gdn.h"

namespace {

#define HIP_OK(expr)                                                                           \
    do {                                                                                       \
        const hipError_t e_ = (expr);                                                          \
        if (e_ != hipSuccess) {                                                                \
            std::printf("HIP error %s at line %d: %s\n", hipGetErrorString(e_), __LINE__, #expr); \
            std::exit(2);                                                                      \
        }                                                                                      \
    } while (0)

// Device copy of a host vector (or uninitialised device memory), freed at scope exit.
template <class T>
class DevBuf {
public:
    explicit DevBuf(const std::vector<T>& h) : n_(h.size()) {
        HIP_OK(hipMalloc(&p_, n_ * sizeof(T)));
        HIP_OK(hipMemcpy(p_, h.data(), n_ * sizeof(T), hipMemcpyHostToDevice));
    }
    explicit DevBuf(size_t n) : n_(n) { HIP_OK(hipMalloc(&p_, n_ * sizeof(T))); }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() { (void)hipFree(p_); }
    T* get() const { return p_; }
    std::vector<T> host() const {
        std::vector<T> h(n_);
        HIP_OK(hipMemcpy(h.data(), p_, n_ * sizeof(T), hipMemcpyDeviceToHost));
        return h;
    }

private:
    T* p_ = nullptr;
    size_t n_;
};

// The reference test's comparison: max|got - ref| <= tol * max|ref|.
int compare(const char* name, const std::vector<float>& got, const std::vector<double>& ref, double tol) {
    double worst = 0.0, scale = 1e-30;
    for (size_t i = 0; i < ref.size(); ++i) {
        worst = std::fmax(worst, std::fabs(got[i] - ref[i]));
        scale = std::fmax(scale, std::fabs(ref[i]));
    }
    const bool ok = worst <= tol * scale;
    std::printf("%-24s max|d| %.3g  scale %.3g  rel %.3g  %s\n", name, worst, scale, worst / scale, ok ? "ok" : "FAIL");
    return ok ? 0 : 1;
}

class Normals {
public:
    float operator()() { return dist_(rng_); }
    void fill(std::vector<float>& v, float scale = 1.0f) {
        for (float& x : v) x = (*this)() * scale;
    }

private:
    std::mt19937 rng_{9};
    std::normal_distribution<float> dist_{0.0f, 1.0f};
};

int check_step(Normals& nd, int hk) {
    const int S = 128, hv = 48;
    std::vector<float> st((size_t)S * hv * S), q(hk * S), k(hk * S), v(hv * S), gate(hv), beta(hv);
    nd.fill(st, 0.1f);
    nd.fill(q, 0.1f);
    nd.fill(k, 0.1f);
    nd.fill(v);
    for (float& g : gate) g = -std::fabs(nd());
    for (float& b : beta) b = 0.5f + 0.4f * std::tanh(nd());
    std::vector<double> ref_state(st.begin(), st.end()), ref_o((size_t)hv * S);
    ixo_step(ref_state.data(), q.data(), k.data(), v.data(), gate.data(), beta.data(), ref_o.data(), S, hk, hv);

    DevBuf<float> d_st(st), d_q(q), d_k(k), d_v(v), d_g(gate), d_b(beta), d_o((size_t)hv * S);
    HIP_OK(ix_gdn_step(d_st.get(), d_q.get(), d_k.get(), d_v.get(), d_g.get(), d_b.get(), d_o.get(), S, hk, hv));
    HIP_OK(hipDeviceSynchronize());
    char name[40];
    std::snprintf(name, sizeof name, "step.o     h_k=%d", hk);
    int bad = compare(name, d_o.host(), ref_o, 1e-4);
    std::snprintf(name, sizeof name, "step.state h_k=%d", hk);
    return bad + compare(name, d_st.host(), ref_state, 1e-4);
}

int check_conv(Normals& nd) {
    const int C = 8192 + 5, dc = 4;
    std::vector<float> cs((size_t)C * (dc - 1)), x(C), w((size_t)C * dc);
    nd.fill(cs);
    nd.fill(x);
    nd.fill(w);
    std::vector<float> ref_cs = cs;
    std::vector<double> ref_out(C);
    ixo_conv_step(ref_cs.data(), x.data(), w.data(), ref_out.data(), C, dc);

    DevBuf<float> d_cs(cs), d_x(x), d_w(w), d_out(C);
    HIP_OK(ix_gdn_conv_step(d_cs.get(), d_x.get(), d_w.get(), d_out.get(), C, dc));
    HIP_OK(hipDeviceSynchronize());
    const int bad = compare("conv.out", d_out.host(), ref_out, 1e-5);
    return bad + compare("conv.state", d_cs.host(), std::vector<double>(ref_cs.begin(), ref_cs.end()), 0.0);
}

int check_l2(Normals& nd, int cols) {
    const int rows = 33;
    const float eps = 1e-6f;
    std::vector<float> x((size_t)rows * cols);
    nd.fill(x);
    std::vector<double> ref(x.size());
    ixo_l2_norm(x.data(), ref.data(), rows, cols, eps);

    DevBuf<float> d_x(x);
    HIP_OK(ix_gdn_l2_norm(d_x.get(), rows, cols, eps));
    HIP_OK(hipDeviceSynchronize());
    char name[40];
    std::snprintf(name, sizeof name, "l2 cols=%d", cols);
    return compare(name, d_x.host(), ref, 1e-6);
}

int check_out_norm(Normals& nd, int S) {
    const int hv = 48;
    const float eps = 1e-6f;
    std::vector<float> o((size_t)hv * S), z((size_t)hv * S), nrm(S);
    nd.fill(o);
    nd.fill(z);
    for (float& n : nrm) n = 1.0f + 0.1f * nd();
    std::vector<double> ref((size_t)hv * S);
    ixo_out_norm(o.data(), z.data(), nrm.data(), ref.data(), hv, S, eps);

    DevBuf<float> d_o(o), d_z(z), d_n(nrm), d_y((size_t)hv * S);
    HIP_OK(ix_gdn_out_norm(d_o.get(), d_z.get(), d_n.get(), d_y.get(), hv, S, eps));
    HIP_OK(hipDeviceSynchronize());
    char name[40];
    std::snprintf(name, sizeof name, "out_norm S=%d", S);
    return compare(name, d_y.host(), ref, 1e-5);
}

int check_beta(Normals& nd) {
    const int n = 48;
    std::vector<float> b(n);
    nd.fill(b, 3.0f);
    std::vector<double> ref(n);
    ixo_beta_gate(b.data(), ref.data(), n);

    DevBuf<float> d_b(b);
    HIP_OK(ix_gdn_beta_gate(d_b.get(), n));
    HIP_OK(hipDeviceSynchronize());
    return compare("beta_gate", d_b.host(), ref, 1e-6);
}

// The launchers refuse what the reference's launchers refuse, before any device work.
int validate() {
    int bad = 0;
    auto want_invalid = [&](const char* what, hipError_t e) {
        const bool ok = e == hipErrorInvalidValue;
        std::printf("%-32s %s\n", what, ok ? "ok" : "FAIL");
        bad += !ok;
    };
    float* none = nullptr;
    want_invalid("step S=129", ix_gdn_step(none, none, none, none, none, none, none, 129, 16, 48));
    want_invalid("step h_v=0", ix_gdn_step(none, none, none, none, none, none, none, 128, 16, 0));
    want_invalid("conv_step d_conv=1", ix_gdn_conv_step(none, none, none, none, 8197, 1));
    want_invalid("l2_norm rows=0", ix_gdn_l2_norm(none, 0, 128, 1e-6f));
    want_invalid("l2_norm cols=1025", ix_gdn_l2_norm(none, 33, 1025, 1e-6f));
    want_invalid("beta_gate NULL", ix_gdn_beta_gate(nullptr, 48));
    want_invalid("out_norm h_v=0", ix_gdn_out_norm(none, none, none, none, 0, 128, 1e-6f));
    return bad;
}

}  // namespace

int main(int argc, char** argv) {
    int bad = validate();
    if (argc > 1 && std::strcmp(argv[1], "--validate") == 0) {
        std::printf("drop-in C++ caller (validation only): %s\n", bad ? "FAIL" : "PASS");
        return bad != 0;
    }
    Normals nd;
    for (int hk : {16, 48}) bad += check_step(nd, hk);
    bad += check_conv(nd);
    for (int cols : {128, 100, 7, 64, 65, 1024}) bad += check_l2(nd, cols);
    for (int S : {128, 100, 65}) bad += check_out_norm(nd, S);
    bad += check_beta(nd);
    std::printf("drop-in C++ caller, libixgdn %s: %s\n", ix_gdn_version(), bad ? "FAIL" : "PASS");
    return bad != 0;
}
