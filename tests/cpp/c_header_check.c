/* The C ABI header must compile as plain C11 and declare every entry point with C linkage. */
#include <rocmkernels_attention.h>

int main(void) {
    rocmkernels_strides s = {0, 0, 0};
    float x = 0.0f;
    bool m = true;
    /* Invalid sizes: returns hipErrorInvalidValue (1) before any HIP call, so this runs without a GPU. */
    return attention_fp32_forward_flash(&x, &x, &x, &m, &x, &x, 0, 1, 1, 1, -1, s, s, s, s, NULL) == 1 ? 0 : 1;
}
