/*
 * A reference-side C11 caller of libvx27_hip, compiled unchanged against
 * the headers in include/ (as src/vx27_qfwd.c includes the reference's own
 * vx27_deltanet.h, vx27_gqa.h and vx27_rope.h) and linked to the library.
 *
 * It runs the host-only functions (state sizing, KV-head map, gate
 * parameters, RoPE table, pack sizes), takes the address of every other
 * exported function (so the link resolves each one), and prints
 * sizeof/offsetof of every descriptor field for tests/test_c_boundary.py to
 * compare with the ctypes mirrors in vx27_amd/lib.py.  It needs no GPU.
 */
#include <stddef.h>
#include <stdio.h>

#include "vx27_deltanet.h"
#include "vx27_gqa.h"
#include "vx27_hip.h"
#include "vx27_rope.h"

#include "layout.inc"   /* generated: print_layout() */

typedef void (*any_fn)(void);
#define REF(f) (any_fn)(f)

int main(void) {
    /* every declared entry point, by address */
    static const any_fn fns[] = {
        REF(vx27_deltanet_update_ref), REF(vx27_deltanet_retrieve_ref), REF(vx27_deltanet_update_tiled),
        REF(vx27_deltanet_retrieve_tiled), REF(vx27_deltanet_update_avx2), REF(vx27_deltanet_retrieve_avx2),
        REF(vx27_deltanet_l2norm), REF(vx27_deltanet_step_exact), REF(vx27_conv1d_step), REF(vx27_rmsnorm),
        REF(vx27_attn_1q), REF(vx27_rope_apply), REF(vx27_mrope_cos_sin_text),
        REF(vx27_hip_open), REF(vx27_hip_close), REF(vx27_hip_sync), REF(vx27_hip_set_stream),
        REF(vx27_hip_get_stream), REF(vx27_hip_last_error), REF(vx27_hip_device_count), REF(vx27_hip_version),
        REF(vx27_hip_prof_enable), REF(vx27_hip_prof_read), REF(vx27_hip_default_ctx), REF(vx27_hip_enable),
        REF(vx27_hip_disable), REF(vx27_hip_enabled), REF(vx27_hip_set_error_mode), REF(vx27_hip_alloc),
        REF(vx27_hip_free), REF(vx27_hip_h2d), REF(vx27_hip_d2h), REF(vx27_hip_d2d), REF(vx27_hip_memset),
        REF(vx27_hip_dn_decode), REF(vx27_hip_dn_prefill), REF(vx27_hip_dn_commit), REF(vx27_hip_gqa_decode), REF(vx27_hip_gqa_decode_noalloc), REF(vx27_hip_gqa_prefill),
        REF(vx27_hip_kv_write), REF(vx27_hip_kv_read), REF(vx27_hip_rope_table), REF(vx27_hip_gemv_bf16),
        REF(vx27_hip_pack_weights_bf16), REF(vx27_hip_dn_layer_decode), REF(vx27_hip_gqa_layer_decode),
        REF(vx27_hip_dn_layer_prefill), REF(vx27_hip_gqa_layer_prefill),
        REF(vx27_hip_pack_bytes), REF(vx27_hip_pack_x), REF(vx27_hip_advance_pos), REF(vx27_hip_graph_begin),
        REF(vx27_hip_graph_end), REF(vx27_hip_graph_launch), REF(vx27_hip_graph_destroy),
        REF(vx27_hip_fill_normal_f32), REF(vx27_hip_fill_normal_bf16), REF(vx27_hip_step_exact),
        REF(vx27_hip_update_simple), REF(vx27_hip_retrieve_simple), REF(vx27_hip_l2norm), REF(vx27_hip_rmsnorm),
        REF(vx27_hip_conv1d_step), REF(vx27_hip_rope_apply), REF(vx27_hip_attn_1q), REF(vx27_hip_staging),
        REF(vx27_hip_get_error_mode),
    };
    int null_fns = 0;
    for (size_t i = 0; i < sizeof fns / sizeof fns[0]; i++) null_fns += fns[i] == NULL;

    /* host-only reference functions (tests/test_deltanet.c:24-27, test_gqa.c) */
    double beta = 0.0, g_log = 0.0;
    vx27_deltanet_gate_params(0.3, -0.5, 1.2, 0.05, &beta, &g_log);
    float c[32], s[32];
    vx27_rope_cos_sin(131072, c, s, 64, 1e7f, 1.0f);
    printf("fns %zu null %d\n", sizeof fns / sizeof fns[0], null_fns);
    printf("state_per_layer %d\n", vx27_deltanet_state_per_layer());
    printf("state_total %d\n", vx27_deltanet_state_total());
    printf("kv_for_q_23 %d\n", vx27_gqa_kv_for_q(23));
    printf("gate %.17g %.17g\n", beta, g_log);
    printf("rope_c0_131072 %.9g\n", (double)c[0]);
    printf("pack_bytes_5120 %zu\n", vx27_hip_pack_bytes(5120, 4));
    printf("version %s\n", vx27_hip_version());
    print_layout();
    return 0;
}
