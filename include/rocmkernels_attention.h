/*
 * C ABI of the MI355X (gfx950) FP32 attention library, libROCmKernels.Kernels.Shared.so.
 *
 * Every entry point keeps the name, argument order, argument meaning and return convention of the
 * reference's exported symbol, so a caller that binds the reference shared library by symbol name
 * (ctypes, dlsym, or the C++ wrappers in ROCmKernels/Kernels/Attention headers) binds this one unchanged.
 *
 * Conventions shared by all entry points:
 *   - Tensors are FP32 `[batch][head][token][D]` with element strides {batch, head, token} given by a
 *     Strides value; features are contiguous. D is 32 for attention_fp32_* and 64 for attention64_fp32_*.
 *   - mask is `[batch][keys]` bytes, shared across heads; a zero byte excludes the key.
 *   - radius < 0 attends globally; otherwise a key is visible when |query - key| <= radius (raw indices).
 *   - The softmax scale is fixed at 1/sqrt(D).
 *   - lse is packed `[batch][head][query][2]` = {row maximum of the scaled scores, sum of exp(score - maximum)}.
 *     A row with no visible key gets output 0 and lse {-inf, 0}; a NaN sum gives NaN output and lse {NaN, NaN}.
 *   - output honours its strides; gradient_q/k/v are packed `[batch][head][token][D]`; delta is packed
 *     `[batch][head][query]` and receives sum(upstream * output) per query row.
 *   - Return value is a hipError_t as int: 0 on success, 1 (hipErrorInvalidValue) on invalid arguments,
 *     detected before any HIP call, otherwise hipGetLastError() after the launches.
 *   - Work is enqueued asynchronously on `stream` (NULL = default stream); the library never allocates,
 *     frees or synchronises device memory, and keeps no device state. Host-side it caches what it can recompute:
 *     each device's CU count (process-wide) and, per host thread, the work tables of the last shape it launched.
 *   - Limits of the attention entry points: every (batch, head) sequence of every tensor, plus one 32-row tile, must
 *     span less than 2 GiB, and token strides must be >= 0 (batch and head strides may be negative); otherwise
 *     hipErrorInvalidValue.
 *
 * The *_ex entry points have no counterpart in the reference: they add `int flags` after `radius`, where
 * bit 0 (ROCMKERNELS_ATTENTION_CAUSAL) restricts every query to keys <= query. For the backward, the flags also
 * choose between two implementations of the same maths:
 *   - fused: one kernel forms dK, dV and dQ from each recomputed score tile (5 matrix products per tile); dQ is
 *     accumulated with FP32 atomics, and so are dK/dV of the key blocks whose query range is split over several
 *     workgroups, so those values' low-order bits may differ from run to run (delta is bit-reproducible);
 *   - deterministic: the reference's arrangement, a query-major dQ kernel and a key-major dK/dV kernel (7 matrix
 *     products per tile, S and dP computed in both); bit-identical results run to run.
 *   With neither bit 1 nor bit 2 set the library takes the faster one for the call: fused for inputs with 128-bit
 *   access (16-byte aligned pointers, strides multiples of 4), under a radius window the band kernel when there are at
 *   least 5/8 as many 128-key blocks (batch x heads x ceil(keys / 128)) as compute units; deterministic otherwise.
 *   Bit 1 (ROCMKERNELS_ATTENTION_FUSED_BACKWARD) asks for fused wherever it exists (inputs with 128-bit access); bit 2
 *   (ROCMKERNELS_ATTENTION_DETERMINISTIC) asks for deterministic. Setting both, or any other bit, returns
 *   hipErrorInvalidValue.
 * The reference-named backward entry points always run the deterministic kernels, as the reference's do.
 */
#ifndef ROCMKERNELS_ATTENTION_H
#define ROCMKERNELS_ATTENTION_H

#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__ 1
#endif
#include <hip/hip_runtime_api.h>

#ifndef __cplusplus
#include <stdbool.h>
#endif

#if defined(__HIP_DEVICE_COMPILE__)
#define ROCMKERNELS_EXPORT
#else
#define ROCMKERNELS_EXPORT __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Element strides of a [batch][head][token] tensor (reference: ROCmKernels.Kernels/include/ROCmKernels/Kernels/Strides.hpp:5-9). */
typedef struct rocmkernels_strides {
    int batch;
    int head;
    int token;
} rocmkernels_strides;

#define ROCMKERNELS_ATTENTION_CAUSAL 1
#define ROCMKERNELS_ATTENTION_FUSED_BACKWARD 2
#define ROCMKERNELS_ATTENTION_DETERMINISTIC 4

/* ---- 32-wide forward family ------------------------------------------------------------------ */

/* Replaces attention_fp32_forward (reference Attention.hpp:9-11, Attention.hip:194-203). */
ROCMKERNELS_EXPORT int attention_fp32_forward(const float *q, const float *k, const float *v, const bool *mask, float *output,
        float *lse, int batch, int heads, int queries, int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks,
        rocmkernels_strides vs, rocmkernels_strides os, hipStream_t stream);

/* Replaces attention_fp32_forward_tiled (reference Attention.hpp:12-14, Attention.hip:225-233). */
ROCMKERNELS_EXPORT int attention_fp32_forward_tiled(const float *q, const float *k, const float *v, const bool *mask, float *output,
        float *lse, int batch, int heads, int queries, int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks,
        rocmkernels_strides vs, rocmkernels_strides os, hipStream_t stream);

/* Replaces attention_fp32_statistics (reference Attention.hpp:23-24, Attention.hip:252-261): lse only. */
ROCMKERNELS_EXPORT int attention_fp32_statistics(const float *q, const float *k, const bool *mask, float *lse, int batch, int heads,
        int queries, int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks, hipStream_t stream);

/* Replaces attention_fp32_forward_tuned (reference Attention.hpp:25-27, Attention.hip:358-370).
 * group must be one of 2, 8, 4, 84, 164, 1164, 1264. */
ROCMKERNELS_EXPORT int attention_fp32_forward_tuned(const float *q, const float *k, const float *v, const bool *mask, float *output,
        float *lse, int batch, int heads, int queries, int keys, int radius, int group, rocmkernels_strides qs,
        rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os, hipStream_t stream);

/* Replaces attention_fp32_forward_flash (reference Attention.hpp:28-30, Attention.hip:372-390). */
ROCMKERNELS_EXPORT int attention_fp32_forward_flash(const float *q, const float *k, const float *v, const bool *mask, float *output,
        float *lse, int batch, int heads, int queries, int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks,
        rocmkernels_strides vs, rocmkernels_strides os, hipStream_t stream);

/* Replaces attention_fp32_forward_flash_tuned (reference Attention.hpp:31-33, Attention.hip:392-417). variant is 0..18. */
ROCMKERNELS_EXPORT int attention_fp32_forward_flash_tuned(const float *q, const float *k, const float *v, const bool *mask,
        float *output, float *lse, int batch, int heads, int queries, int keys, int radius, int variant, rocmkernels_strides qs,
        rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os, hipStream_t stream);

/* ---- 32-wide backward family ----------------------------------------------------------------- */

/* Replaces attention_fp32_backward (reference Attention.hpp:15-18, Attention.hip:205-223). */
ROCMKERNELS_EXPORT int attention_fp32_backward(const float *q, const float *k, const float *v, const bool *mask, const float *output,
        const float *lse, const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, int batch,
        int heads, int queries, int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs,
        rocmkernels_strides os, rocmkernels_strides us, hipStream_t stream);

/* Replaces attention_fp32_backward_tiled (reference Attention.hpp:19-22, Attention.hip:235-250). */
ROCMKERNELS_EXPORT int attention_fp32_backward_tiled(const float *q, const float *k, const float *v, const bool *mask,
        const float *output, const float *lse, const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v,
        float *delta, int batch, int heads, int queries, int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks,
        rocmkernels_strides vs, rocmkernels_strides os, rocmkernels_strides us, hipStream_t stream);

/* Replaces attention_fp32_backward_tuned (reference Attention.hpp:34-37, Attention.hip:419-438).
 * group must be one of 2, 8, 4, 84, 164, 1164, 1264. */
ROCMKERNELS_EXPORT int attention_fp32_backward_tuned(const float *q, const float *k, const float *v, const bool *mask,
        const float *output, const float *lse, const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v,
        float *delta, int batch, int heads, int queries, int keys, int radius, int group, rocmkernels_strides qs,
        rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os, rocmkernels_strides us, hipStream_t stream);

/* Replaces the exported-but-undeclared attention_fp32_backward_profile (reference Attention.hip:327-337).
 * stage 1 writes delta only, 2 writes gradient_q only (reading delta), 3 writes gradient_k/v only (reading delta).
 * Requires queries >= 32, as the reference does. */
ROCMKERNELS_EXPORT int attention_fp32_backward_profile(const float *q, const float *k, const float *v, const bool *mask,
        const float *output, const float *lse, const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v,
        float *delta, int batch, int heads, int queries, int keys, int radius, int stage, rocmkernels_strides qs,
        rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os, rocmkernels_strides us, hipStream_t stream);

/* Replaces the exported-but-undeclared attention_fp32_query_profile (reference Attention.hip:339-356): writes
 * gradient_q only, reading delta. tuning must be one of 14, 18, 116, 24, 28, 44. Requires queries >= 32. */
ROCMKERNELS_EXPORT int attention_fp32_query_profile(const float *q, const float *k, const float *v, const bool *mask,
        const float *output, const float *lse, const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v,
        float *delta, int batch, int heads, int queries, int keys, int radius, int tuning, rocmkernels_strides qs,
        rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os, rocmkernels_strides us, hipStream_t stream);

/* ---- 64-wide ---------------------------------------------------------------------------------- */

/* Replaces attention64_fp32_forward (reference Attention64.hpp:9-11, Attention64.hip:193-202). */
ROCMKERNELS_EXPORT int attention64_fp32_forward(const float *q, const float *k, const float *v, const bool *mask, float *output,
        float *lse, int batch, int heads, int queries, int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks,
        rocmkernels_strides vs, rocmkernels_strides os, hipStream_t stream);

/* Replaces attention64_fp32_backward (reference Attention64.hpp:12-15, Attention64.hip:204-220). */
ROCMKERNELS_EXPORT int attention64_fp32_backward(const float *q, const float *k, const float *v, const bool *mask,
        const float *output, const float *lse, const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v,
        float *delta, int batch, int heads, int queries, int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks,
        rocmkernels_strides vs, rocmkernels_strides os, rocmkernels_strides us, hipStream_t stream);

/* ---- causal-capable extensions (no reference counterpart; the reference has no causal mask) ------ */

/* attention_fp32_forward_flash plus flags (bit 0 = causal). */
ROCMKERNELS_EXPORT int attention_fp32_forward_flash_ex(const float *q, const float *k, const float *v, const bool *mask,
        float *output, float *lse, int batch, int heads, int queries, int keys, int radius, int flags, rocmkernels_strides qs,
        rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os, hipStream_t stream);

/* attention_fp32_backward plus flags (bit 0 = causal; bits 1 and 2 choose fused or deterministic, see above). */
ROCMKERNELS_EXPORT int attention_fp32_backward_ex(const float *q, const float *k, const float *v, const bool *mask,
        const float *output, const float *lse, const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v,
        float *delta, int batch, int heads, int queries, int keys, int radius, int flags, rocmkernels_strides qs,
        rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os, rocmkernels_strides us, hipStream_t stream);

/* attention64_fp32_forward plus flags (bit 0 = causal). */
ROCMKERNELS_EXPORT int attention64_fp32_forward_ex(const float *q, const float *k, const float *v, const bool *mask,
        float *output, float *lse, int batch, int heads, int queries, int keys, int radius, int flags, rocmkernels_strides qs,
        rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os, hipStream_t stream);

/* attention64_fp32_backward plus flags (bit 0 = causal; bits 1 and 2 choose fused or deterministic, see above). */
ROCMKERNELS_EXPORT int attention64_fp32_backward_ex(const float *q, const float *k, const float *v, const bool *mask,
        const float *output, const float *lse, const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v,
        float *delta, int batch, int heads, int queries, int keys, int radius, int flags, rocmkernels_strides qs,
        rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os, rocmkernels_strides us, hipStream_t stream);

/* ---- generic forward (16-, 32- or 64-wide heads, fp32 or fp16 storage) --------------------------------- */

/* Storage type of attention_generic_forward's q, k, v and output; accumulation is always fp32 (reference:
 * ROCmKernels.Kernels/include/ROCmKernels/Kernels/DType.hpp:7-8, `enum class DType : unsigned char { Float32, Float16 }`). */
typedef unsigned char rocmkernels_dtype;
#define ROCMKERNELS_DTYPE_FLOAT32 0
#define ROCMKERNELS_DTYPE_FLOAT16 1

/* Replaces attention_generic_forward (reference Generic/AttentionGeneric.hpp:10-13,
 * Generic/Attention/AttentionGeneric.hip:291-309): windowed forward for headWidth 16, 32 or 64 with q, k, v and
 * output of type dtype (fp32 lse). No causal mask. hipErrorInvalidValue for null pointers, non-positive sizes,
 * radius < -1, another headWidth or an unknown dtype. fp16 rows are read with 128-bit loads when every pointer is
 * 16-byte aligned and every stride a multiple of 8 elements. */
ROCMKERNELS_EXPORT int attention_generic_forward(const void *q, const void *k, const void *v, const bool *mask, void *output,
        float *lse, int batch, int heads, int queries, int keys, int headWidth, int radius, rocmkernels_strides qs,
        rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os, rocmkernels_dtype dtype, hipStream_t stream);

/* ---- rotary position embedding (the step that prepares Q and K) ---------------------------------------- */

/* Replaces rotary_fp32 (reference Positional/Rotary.hpp:9-11, Positional/Rotary.hip:44-56): 32-wide heads, q and k
 * honour qs and ks, cos and sin hold 32 values per (batch, token) and honour the batch and token entries of cs and
 * ss. Outputs oq and ok are token-major packed [batch][token][head][32]. backward != 0 applies the transposed
 * rotation. hipErrorInvalidValue for null pointers or non-positive sizes. */
ROCMKERNELS_EXPORT int rotary_fp32(const float *q, const float *k, const float *cos, const float *sin, float *oq, float *ok, int batch,
        int heads, int length, int backward, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides cs,
        rocmkernels_strides ss, hipStream_t stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* ROCMKERNELS_ATTENTION_H */
