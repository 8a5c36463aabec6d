// gdn_prefill.hip -- chunked WY-form GDN prefill for gfx950 (ix_gdn_prefill).
#include "ix_gdn.h"
#include "wave64.h"

extern "C" hipError_t ix_gdn_check_cfg_(const ix_gdn_cfg* c);

extern "C" size_t ix_gdn_prefill_workspace_size(const ix_gdn_cfg* cfg, int n_seq, int total_T) {
    if (ix_gdn_check_cfg_(cfg) != hipSuccess || n_seq <= 0 || total_T < 0) return 0;
    return 256;
}

extern "C" hipError_t ix_gdn_prefill(const ix_gdn_cfg* cfg, int n_seq, int total_T, const int32_t* cu_seqlens,
                                     const uint16_t* x, uint16_t* conv_state, const uint16_t* conv_w,
                                     const uint16_t* a, const uint16_t* b, const float* A_log,
                                     const float* dt_bias, float* state, float* o, uint16_t* o_bf16,
                                     void* workspace, size_t workspace_bytes, hipStream_t s) {
    (void)n_seq; (void)total_T; (void)cu_seqlens; (void)x; (void)conv_state; (void)conv_w; (void)a; (void)b;
    (void)A_log; (void)dt_bias; (void)state; (void)o; (void)o_bf16; (void)workspace; (void)workspace_bytes; (void)s;
    const hipError_t e = ix_gdn_check_cfg_(cfg);
    if (e != hipSuccess) return e;
    return hipErrorNotSupported;
}
