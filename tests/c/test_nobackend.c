/*
 * test_nobackend.c — the engine's CPU-only build: engine_tu.c without the
 * library. The stubs decline, the hook table stays all-NULL, so every call
 * site (c/bf16.h:717-719, 743-745; c/gdsa.h:529-531) runs its CPU kernel.
 * Exit 0 = as expected.
 */
#include <stdio.h>
#include <string.h>

#include "backend_hip.h"

int main(void) {
    char err[256] = "";
    int rc = apus_ghip_enable(err, sizeof err);
    int ok = rc != 0 && strcmp(err, "HIP backend not linked") == 0
          && apus_ghip_is_enabled() == 0 && apus_ghip_hooks.bf16_gemm == NULL
          && apus_ghip_hooks.fp8blk_linear == NULL
          && apus_ghip_register_region(&rc, sizeof rc) != 0;
    apus_ghip_disable();
    apus_ghip_unregister_region(&rc);
    printf("nobackend: enable rc=%d (%s), hooks %s\n", rc, err,
           apus_ghip_hooks.bf16_gemm || apus_ghip_hooks.fp8blk_linear ? "SET" : "NULL");
    printf(ok ? "PASS\n" : "FAIL\n");
    return ok ? 0 : 1;
}
