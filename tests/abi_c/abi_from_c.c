/*
 * The C ABI used from plain C99, as a cgo / JNI / FFI binding would use it: the header compiles as
 * C, every call below links against libcannbench_amd.so, and each returns its validation status
 * before touching a device (no GPU needed).  Prints "ok" and exits 0 when every check holds.
 */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "cannbench_amd.h"

static int failures = 0;

static void expect(const char* what, int got, int want)
{
    if (got != want) {
        printf("%s: status %d (%s), expected %d (%s)\n", what, got, cb_status_string(got), want,
               cb_status_string(want));
        ++failures;
    }
}

int main(void)
{
    /* a non-NULL pointer value that is never dereferenced: validation fails first */
    void* fake = (void*)(uintptr_t)0x1000;
    const int64_t gl_ok[2] = {4, 8};
    const int64_t gl_short[2] = {4, 7};
    int64_t ws;

    if (strstr(cb_version(), "gfx950") == NULL) {
        printf("cb_version: %s\n", cb_version());
        ++failures;
    }
    /* GroupedMatmulSwigluQuant: odd N, group total, empty M (returns before any launch) */
    expect("gmsq odd N",
           cb_grouped_matmul_swiglu_quant((const int8_t*)fake, (const int8_t*)fake, (const float*)fake,
                                          (const float*)fake, gl_ok, 2, 8, 64, 7, 2, (int8_t*)fake,
                                          (float*)fake, fake, 1 << 20, NULL),
           CB_ERR_N_ODD);
    expect("gmsq group total",
           cb_grouped_matmul_swiglu_quant((const int8_t*)fake, (const int8_t*)fake, (const float*)fake,
                                          (const float*)fake, gl_short, 2, 8, 64, 8, 2, (int8_t*)fake,
                                          (float*)fake, fake, 1 << 20, NULL),
           CB_ERR_GROUP_TOTAL);
    expect("gmsq empty M",
           cb_grouped_matmul_swiglu_quant((const int8_t*)fake, (const int8_t*)fake, (const float*)fake,
                                          (const float*)fake, gl_ok, 2, 0, 64, 8, 2, (int8_t*)fake,
                                          (float*)fake, fake, 1 << 20, NULL),
           CB_OK);
    ws = cb_grouped_matmul_swiglu_quant_workspace_size(131072, 7168, 4096, 256);
    if (ws <= 0 || ws > (64 << 20)) {
        printf("gmsq workspace size %lld\n", (long long)ws);
        ++failures;
    }
    /* AddRmsNormDynamicQuant: a dtype it does not take */
    expect("ardq dtype",
           cb_add_rms_norm_dynamic_quant(fake, fake, fake, CB_DT_INT8, 4, 64, 1e-6f, (int8_t*)fake, fake,
                                         (float*)fake, NULL),
           CB_ERR_DTYPE);
    /* MoeGatingTopKSoftmax: k above the expert count */
    expect("gating k > E",
           cb_moe_gating_top_k_softmax(fake, CB_DT_FLOAT32, 4, 8, NULL, 9, fake, (int32_t*)fake, (int32_t*)fake,
                                       NULL),
           CB_ERR_SHAPE);
    if (strcmp(cb_status_string(CB_ERR_N_ODD), "N must be even") != 0) {
        printf("status string: %s\n", cb_status_string(CB_ERR_N_ODD));
        ++failures;
    }
    if (failures == 0) printf("ok\n");
    return failures == 0 ? 0 : 1;
}
