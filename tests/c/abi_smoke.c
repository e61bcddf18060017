/* A C99 program against include/tomoul_hip.h, linked to libtomoul_hip.so:
 * shows that the boundary is a plain C ABI (what a Zig `extern "c"` shim
 * binds) and exercises the entry points that need no GPU -- the .tl reader
 * on the reference's own fixture (tests/fixtures/linear/model.tl: y = 2x + 1,
 * src/core/loader.zig:650-693) and the error codes -- plus tml_hip_init,
 * which reports TML_ERR_NO_DEVICE on a host without a GPU. */
#include <stdio.h>
#include <string.h>

#include "tomoul_hip.h"

static int fail(int code, const char *what) {
    printf("FAIL %s (%d: %s)\n", what, code, tml_hip_last_error());
    return 1;
}

int main(int argc, char **argv) {
    if (argc < 2) return fail(0, "usage: abi_smoke <linear_model.tl>");
    tml_tl_t f = NULL;
    int rc = tml_tl_open(argv[1], &f);
    if (rc != TML_OK) return fail(rc, "tml_tl_open");
    if (tml_tl_format(f) != TML_FMT_F32) return fail(tml_tl_format(f), "format");
    if (tml_tl_count(f) != 2) return fail((int)tml_tl_count(f), "tensor count");
    if (tml_tl_name(f, 0) == NULL || strcmp(tml_tl_name(f, 0), "weight") != 0) return fail(0, "first name");
    if (tml_tl_name(f, 2) != NULL) return fail(0, "name past the end");

    int64_t dims[4] = {0, 0, 0, 0};
    int ndim = 0;
    uint64_t off = 0, size = 0;
    rc = tml_tl_info(f, "weight", dims, 4, &ndim, &off, &size);
    if (rc != TML_OK || ndim != 2 || dims[0] != 1 || dims[1] != 1 || size != 4) return fail(rc, "weight info");

    float w = 0.0f, b = 0.0f;
    rc = tml_tl_read(f, "weight", TML_FMT_F32, &w, NULL, NULL);
    if (rc != TML_OK) return fail(rc, "read weight");
    rc = tml_tl_read(f, "bias", TML_FMT_F32, &b, NULL, NULL);
    if (rc != TML_OK) return fail(rc, "read bias");
    if (tml_tl_read(f, "missing", TML_FMT_F32, &w, NULL, NULL) != TML_ERR_TENSOR_NOT_FOUND)
        return fail(0, "missing tensor");
    float scale = 0.0f;
    int8_t q = 0;
    if (tml_tl_read(f, "weight", TML_FMT_Q8_0, &q, NULL, &scale) != TML_ERR_UNSUPPORTED_QUANT_FORMAT)
        return fail(0, "Q8_0 getter on an f32 file");
    tml_tl_close(f);

    tml_tl_t g = NULL;
    if (tml_tl_open("/nonexistent/path/model.tl", &g) != TML_ERR_FILE_NOT_FOUND || g != NULL)
        return fail(0, "missing file");

    rc = tml_hip_init();
    if (rc != TML_OK && rc != TML_ERR_NO_DEVICE) return fail(rc, "tml_hip_init");
    printf("y(10) = %g; init = %d\n", 10.0f * w + b, rc);
    return 0;
}
