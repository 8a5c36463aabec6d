/*
 * dropin_c.c -- a C caller of libixgdn.so through include/ix_gdn.h (C mode: no default stream
 * argument, so every call passes one). It needs no GPU: each call below is refused by the
 * library's validation before anything is enqueued, and the program checks the codes --
 * the shapes the reference's launchers refuse (src/ix_gdn.cu:110, :117, :122, :127, :133)
 * and the fused entry points' description checks. Exit status 0 means every check passed.
 */
#include <stdio.h>
#include <string.h>

#include "ix_gdn.h"

static int failures = 0;

static void expect(const char* what, hipError_t got, hipError_t want) {
    const int ok = got == want;
    printf("%-44s %s (got %d, want %d)\n", what, ok ? "ok" : "FAIL", (int)got, (int)want);
    failures += !ok;
}

int main(void) {
    const hipStream_t s = NULL;
    float* none = NULL;
    /* the reference launchers' shape checks */
    expect("ix_gdn_step S=129", ix_gdn_step(none, none, none, none, none, none, none, 129, 16, 48, s),
           hipErrorInvalidValue);
    expect("ix_gdn_step S=0", ix_gdn_step(none, none, none, none, none, none, none, 0, 16, 48, s),
           hipErrorInvalidValue);
    expect("ix_gdn_step h_k=0", ix_gdn_step(none, none, none, none, none, none, none, 128, 0, 48, s),
           hipErrorInvalidValue);
    expect("ix_gdn_conv_step d_conv=1", ix_gdn_conv_step(none, none, none, none, 8197, 1, s), hipErrorInvalidValue);
    expect("ix_gdn_conv_step channels=0", ix_gdn_conv_step(none, none, none, none, 0, 4, s), hipErrorInvalidValue);
    expect("ix_gdn_l2_norm cols=1025", ix_gdn_l2_norm(none, 33, 1025, 1e-6f, s), hipErrorInvalidValue);
    expect("ix_gdn_beta_gate NULL", ix_gdn_beta_gate(NULL, 48, s), hipErrorInvalidValue);
    expect("ix_gdn_out_norm S=0", ix_gdn_out_norm(none, none, none, none, 48, 0, 1e-6f, s), hipErrorInvalidValue);

    /* the fused entry points: a C struct for the layer description */
    ix_gdn_cfg cfg;
    memset(&cfg, 0, sizeof cfg);
    cfg.h_k = 16; cfg.h_v = 32; cfg.d_k = 128; cfg.d_v = 128; cfg.d_conv = 4;
    cfg.head_map = IX_GDN_HEAD_MOD; cfg.conv_act = IX_GDN_ACT_NONE; cfg.q_scale = 1.0f; cfg.l2_eps = 1e-6f;
    if (ix_gdn_channels(&cfg) != 8192) { printf("ix_gdn_channels FAIL\n"); ++failures; }
    if (ix_gdn_in_proj_width(&cfg) != 8192 + 4096 + 64) { printf("ix_gdn_in_proj_width FAIL\n"); ++failures; }
    if (ix_gdn_decode_workspace_size(&cfg, 64) == 0) { printf("ix_gdn_decode_workspace_size FAIL\n"); ++failures; }
    if (ix_gdn_prefill_workspace_size(&cfg, 1, 4096) == 0) { printf("ix_gdn_prefill_workspace_size FAIL\n"); ++failures; }
    expect("ix_gdn_decode B=0", ix_gdn_decode(&cfg, 0, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL,
                                               NULL, s), hipErrorInvalidValue);
    ix_gdn_cfg bad = cfg;
    bad.d_k = 64;
    expect("ix_gdn_decode d_k=64", ix_gdn_decode(&bad, 1, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL,
                                                  NULL, s), hipErrorInvalidValue);
    expect("ix_gdn_prefill n_seq=0", ix_gdn_prefill(&cfg, 0, 64, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL,
                                                     NULL, NULL, NULL, 0, s), hipErrorInvalidValue);
    expect("ix_gdn_decode_window K=17", ix_gdn_decode_window(&cfg, 2, 17, NULL, NULL, NULL, NULL, NULL, NULL, NULL,
                                                              NULL, NULL, NULL, NULL, s), hipErrorInvalidValue);
    printf("libixgdn %s, C caller: %s\n", ix_gdn_version(), failures ? "FAIL" : "PASS");
    return failures != 0;
}
