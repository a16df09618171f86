/*
 * engine_tu.c — the engine-side lines a maintainer adds next to the Metal
 * hook table in the bf16.h implementation TU (c/bf16.h:157-172): the
 * engine's own (strong) hook table, all-NULL until apus_ghip_enable fills
 * it, and -- in a build that does not link libapus_ghip.so -- stubs that
 * decline, so the plain CPU build still links.
 *
 * The stubs are compiled only when the library is NOT linked
 * (APUS_GHIP_LINKED undefined). A weak stub defined in the executable is
 * not replaced by the shared library's definition at run time (the
 * executable's own definition binds first), so stubs in a build that also
 * links the library would keep the backend off for good; the C tests link
 * this file both ways.
 */
#include <stdio.h>

#include "backend_hip.h"

ApusGhipHooks apus_ghip_hooks;          /* all-NULL: the CPU kernels run */

#ifndef APUS_GHIP_LINKED
int apus_ghip_enable(char *err, size_t errcap) {
    if (err && errcap) snprintf(err, errcap, "HIP backend not linked");
    return -1;
}
void apus_ghip_disable(void) {}
int apus_ghip_is_enabled(void) { return 0; }
int apus_ghip_register_region(const void *p, size_t n) { (void)p; (void)n; return 1; }
void apus_ghip_unregister_region(const void *p) { (void)p; }
#endif
