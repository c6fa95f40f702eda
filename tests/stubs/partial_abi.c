/* A stand-in for libffn_mi355x.so that exports the planning half of include/ffn_mi355x.h and,
 * unless PARTIAL_ABI_NO_PLAN is defined, plans every problem onto one 64x64x64 tile variant.
 * It exports no launch entry point (ffn_mi355x_run and its relatives): a stale or partial
 * build as the host would meet it.  Built by the host tests with gcc; it touches no GPU. */
#include <string.h>
#include "ffn_mi355x.h"

int ffn_mi355x_query(int device, int* cu_count, char* arch, int arch_len) {
    (void)device;
    *cu_count = 256;
    strncpy(arch, "gfx950", (size_t)arch_len);
    return FFN_MI355X_OK;
}

#ifndef PARTIAL_ABI_NO_PLAN
int ffn_mi355x_make_plan(int m, int mp, int kp, int hp, int np, int dtype, int down_impl,
                         int activation, int block_num, int up_variant, int down_variant,
                         ffn_mi355x_plan* plan) {
    (void)up_variant;
    (void)down_variant;
    memset(plan, 0, sizeof *plan);
    plan->m = m, plan->mp = mp, plan->kp = kp, plan->hp = hp, plan->np = np;
    plan->dtype = dtype, plan->down_impl = down_impl, plan->activation = activation;
    plan->block_num = block_num;
    plan->up_bm = plan->up_bn = plan->up_bk = 64;
    plan->down_bm = plan->down_bn = plan->down_bk = 64;
    plan->k = kp, plan->h = hp, plan->n = np, plan->ldx = kp, plan->ldw1 = kp, plan->ldw2 = hp;
    return FFN_MI355X_OK;
}
#endif

int ffn_mi355x_set_operands(ffn_mi355x_plan* plan, int k, int h, int n, int ldx, int ldw1, int ldw2) {
    plan->k = k, plan->h = h, plan->n = n, plan->ldx = ldx, plan->ldw1 = ldw1, plan->ldw2 = ldw2;
    return FFN_MI355X_OK;
}

int ffn_mi355x_set_x_rows(ffn_mi355x_plan* plan, int d1, int d2, int s0, int s1, int s2) {
    plan->x_d1 = d1, plan->x_d2 = d2, plan->x_s0 = s0, plan->x_s1 = s1, plan->x_s2 = s2;
    return FFN_MI355X_OK;
}

int ffn_mi355x_set_single_launch(ffn_mi355x_plan* plan, int on) {
    plan->single_launch = 0;
    return on ? FFN_MI355X_ENOT_APPLICABLE : FFN_MI355X_OK;
}

int ffn_mi355x_workspace_bytes(const ffn_mi355x_plan* plan, size_t* bytes) {
    *bytes = plan->workspace_bytes;
    return FFN_MI355X_OK;
}

int ffn_mi355x_workspace_counter_bytes(const ffn_mi355x_plan* plan, size_t* bytes) {
    (void)plan;
    *bytes = 0;
    return FFN_MI355X_OK;
}

int ffn_mi355x_num_variants(void) { return 1; }

int ffn_mi355x_variant_info(int variant, int* bm, int* bn, int* bk, int* waves, int* stages, int* lds_bytes) {
    if (variant != 0) return FFN_MI355X_EINVAL;
    *bm = *bn = *bk = 64, *waves = 4, *stages = 2, *lds_bytes = 32768;
    return FFN_MI355X_OK;
}

int ffn_mi355x_variant_refill_waves(int variant) { return variant == 0 ? 0 : FFN_MI355X_EINVAL; }

int ffn_mi355x_variant_mfma_edge(int variant) { return variant == 0 ? 32 : FFN_MI355X_EINVAL; }

const char* ffn_mi355x_last_error(void) { return ""; }

const char* ffn_mi355x_strerror(int code) { return code ? "error" : "ok"; }

const char* ffn_mi355x_version(void) { return "partial ABI stand-in"; }
