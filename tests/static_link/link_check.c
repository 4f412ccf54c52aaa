/* Links libvicinity_gpu.a into a C program (the way a Rust build.rs links it)
 * and calls entry points whose argument checks fail before any device call,
 * so the program runs on a host with no GPU. */
#include <stdio.h>
#include <string.h>

#include "vicinity_gpu.h"

int main(void) {
    vgpu_ivfpq *h = 0;
    int rc = vgpu_ivfpq_new(16, 0, &h);
    if (rc != VGPU_ERR_INVALID_PARAMETER) {
        printf("vgpu_ivfpq_new(null params) returned %d\n", rc);
        return 1;
    }
    if (strlen(vgpu_last_error()) == 0) {
        printf("no error message\n");
        return 1;
    }
    vgpu_ivfpq_free(0);
    printf("static link ok: %s\n", vgpu_last_error());
    return 0;
}
