/* v4_check_main.c — TEST DRIVER for a host sanitizer build (ASan + UBSan) of the CPW1 v4
 * parser and writer (cachepotato_amd/csrc/engine/cpw4.c), built by tests/test_sanitize.py.
 *
 *   v4_check FILE...       cpw4_check_file on each file; prints "rc message" per file
 *   v4_check --write FILE  writes a two-tensor file (one f32 vector, one Q4_0 matrix, a
 *                          region over both) with the streaming writer, then checks it */
#include "cpw4.h"
#include "qwen3_moe.h"

#include <stdio.h>
#include <string.h>

static int fill(void *user, int t, uint8_t *dst, size_t nbytes) {
    (void)user;
    for (size_t i = 0; i < nbytes; i++) dst[i] = (uint8_t)(i * 131u + (unsigned)t * 7u);
    return 0;
}

static int write_small(const char *path) {
    cpw4_writer *w = cpw4_writer_create();
    if (!w) return -2;
    const uint32_t d1[1] = {64}, d2[2] = {64, 128};
    int rc = 0;
    const int a = cpw4_add_tensor(w, "norm", QW3_ENC_F32, 1, d1, CPW4_ROLE_NORM);
    const int b = cpw4_add_tensor(w, "matrix", QW3_ENC_Q4, 2, d2, CPW4_ROLE_OTHER);
    if (a < 0 || b < 0) rc = -1;
    if (!rc) rc = cpw4_add_region(w, a, b + 1, CPW4_REG_TENSOR, 0xFFFF, 0, 1);
    char err[256] = {0};
    if (rc >= 0) rc = cpw4_write(w, path, NULL, fill, NULL, err, sizeof err);
    cpw4_writer_destroy(w);
    if (rc) fprintf(stderr, "write: %d %s\n", rc, err);
    return rc;
}

int main(int argc, char **argv) {
    int first = 1;
    if (argc > 2 && strcmp(argv[1], "--write") == 0) {
        if (write_small(argv[2])) return 2;
        first = 2;
    }
    for (int i = first; i < argc; i++) {
        char err[256] = {0};
        const int rc = cpw4_check_file(argv[i], err, sizeof err);
        printf("%d %s\n", rc, err);
    }
    return 0;
}
