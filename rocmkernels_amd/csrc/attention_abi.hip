// The library's C entry points: argument validation with the reference's return codes, then one launch
// path per direction. Every reference entry point computes the same maths with a different RDNA2 tiling
// (simple, tiled, tuned group codes, flash variants, profile stages); on gfx950 they all run the same MFMA
// kernels, and the codes that selected an RDNA2 tiling are validated and otherwise ignored.
#include <rocmkernels_attention.h>

#include "attention_launch.hpp"

namespace {

using rk::BackwardArgs;
using rk::ForwardArgs;

constexpr int kInvalid = hipErrorInvalidValue;

bool bad_dims(const int batch, const int heads, const int queries, const int keys) {
    return batch <= 0 || heads <= 0 || queries <= 0 || keys <= 0;
}

bool bad_forward_pointers(const float *q, const float *k, const float *v, const bool *mask, const float *output, const float *lse) {
    return !q || !k || !v || !mask || !output || !lse;
}

bool bad_backward_pointers(const float *q, const float *k, const float *v, const bool *mask, const float *output, const float *lse,
        const float *upstream, const float *gq, const float *gk, const float *gv, const float *delta) {
    return !q || !k || !v || !mask || !output || !lse || !upstream || !gq || !gk || !gv || !delta;
}

int forward(const int D, const int flags, const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse,
        const int batch, const int heads, const int queries, const int keys, const int radius, const rocmkernels_strides qs,
        const rocmkernels_strides ks, const rocmkernels_strides vs, const rocmkernels_strides os, hipStream_t stream) {
    if (bad_forward_pointers(q, k, v, mask, output, lse) || bad_dims(batch, heads, queries, keys)) return kInvalid;
    const ForwardArgs a{q, k, v, mask, output, lse, batch, heads, queries, keys, radius < 0 ? -1 : radius, flags & 1, qs, ks, vs, os};
    return rk::launch_forward(D, false, a, stream);
}

int backward(const int D, const int flags, const rk::BackwardStage stage, const float *q, const float *k, const float *v,
        const bool *mask, const float *output, const float *lse, const float *upstream, float *gq, float *gk, float *gv, float *delta,
        const int batch, const int heads, const int queries, const int keys, const int radius, const rocmkernels_strides qs,
        const rocmkernels_strides ks, const rocmkernels_strides vs, const rocmkernels_strides os, const rocmkernels_strides us,
        hipStream_t stream) {
    if (bad_backward_pointers(q, k, v, mask, output, lse, upstream, gq, gk, gv, delta) || bad_dims(batch, heads, queries, keys))
        return kInvalid;
    const BackwardArgs a{q, k, v, mask, output, lse, upstream, gq, gk, gv, delta, batch, heads, queries, keys, radius < 0 ? -1 : radius,
            flags & 1, qs, ks, vs, os, us};
    return rk::launch_backward(D, stage, a, stream);
}

// _ex backward flags: causal, and at most one of fused / deterministic.
bool bad_backward_flags(const int flags) {
    constexpr int kKnown = ROCMKERNELS_ATTENTION_CAUSAL | ROCMKERNELS_ATTENTION_FUSED_BACKWARD | ROCMKERNELS_ATTENTION_DETERMINISTIC;
    constexpr int kBoth = ROCMKERNELS_ATTENTION_FUSED_BACKWARD | ROCMKERNELS_ATTENTION_DETERMINISTIC;
    return (flags & ~kKnown) != 0 || (flags & kBoth) == kBoth;
}

rk::BackwardStage backward_stage(const int flags) {
    if (flags & ROCMKERNELS_ATTENTION_DETERMINISTIC) return rk::kBackwardAll;
    if (flags & ROCMKERNELS_ATTENTION_FUSED_BACKWARD) return rk::kBackwardFused;
    return rk::kBackwardAuto;
}

bool valid_group(const int group) {
    // Group codes accepted by the reference (Attention.hip:361-369 forward, :423-437 backward).
    return group == 2 || group == 8 || group == 4 || group == 84 || group == 164 || group == 1164 || group == 1264;
}

bool valid_tuning(const int tuning) {
    // Tuning codes accepted by the reference's query profile (Attention.hip:347-355).
    return tuning == 14 || tuning == 18 || tuning == 116 || tuning == 24 || tuning == 28 || tuning == 44;
}

} // namespace

extern "C" {

// Reference Attention.hip:194-203: validates pointers and dims; radius < -1 behaves as global.
int attention_fp32_forward(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse, int batch,
        int heads, int queries, int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs,
        rocmkernels_strides os, hipStream_t stream) {
    return forward(32, 0, q, k, v, mask, output, lse, batch, heads, queries, keys, radius, qs, ks, vs, os, stream);
}

// Reference Attention.hip:225-233. Validated as attention_fp32_forward (the reference skips validation when
// queries >= 32; rejecting null pointers there changes nothing for valid calls).
int attention_fp32_forward_tiled(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse, int batch,
        int heads, int queries, int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs,
        rocmkernels_strides os, hipStream_t stream) {
    return forward(32, 0, q, k, v, mask, output, lse, batch, heads, queries, keys, radius, qs, ks, vs, os, stream);
}

// Reference Attention.hip:252-261.
int attention_fp32_statistics(const float *q, const float *k, const bool *mask, float *lse, int batch, int heads, int queries, int keys,
        int radius, rocmkernels_strides qs, rocmkernels_strides ks, hipStream_t stream) {
    if (!q || !k || !mask || !lse || bad_dims(batch, heads, queries, keys) || radius < -1) return kInvalid;
    const rocmkernels_strides none{0, 0, 0};
    const ForwardArgs a{q, k, nullptr, mask, nullptr, lse, batch, heads, queries, keys, radius, 0, qs, ks, none, none};
    return rk::launch_forward(32, true, a, stream);
}

// Reference Attention.hip:358-370.
int attention_fp32_forward_tuned(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse, int batch,
        int heads, int queries, int keys, int radius, int group, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs,
        rocmkernels_strides os, hipStream_t stream) {
    if (!valid_group(group)) return kInvalid;
    return forward(32, 0, q, k, v, mask, output, lse, batch, heads, queries, keys, radius, qs, ks, vs, os, stream);
}

// Reference Attention.hip:372-390: additionally rejects radius < -1.
int attention_fp32_forward_flash(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse, int batch,
        int heads, int queries, int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs,
        rocmkernels_strides os, hipStream_t stream) {
    if (radius < -1) return kInvalid;
    return forward(32, 0, q, k, v, mask, output, lse, batch, heads, queries, keys, radius, qs, ks, vs, os, stream);
}

// Reference Attention.hip:392-417: variants 0..18.
int attention_fp32_forward_flash_tuned(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse,
        int batch, int heads, int queries, int keys, int radius, int variant, rocmkernels_strides qs, rocmkernels_strides ks,
        rocmkernels_strides vs, rocmkernels_strides os, hipStream_t stream) {
    if (variant < 0 || variant > 18 || radius < -1) return kInvalid;
    return forward(32, 0, q, k, v, mask, output, lse, batch, heads, queries, keys, radius, qs, ks, vs, os, stream);
}

// Reference Attention.hip:205-223.
int attention_fp32_backward(const float *q, const float *k, const float *v, const bool *mask, const float *output, const float *lse,
        const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, int batch, int heads, int queries,
        int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os,
        rocmkernels_strides us, hipStream_t stream) {
    return backward(32, 0, rk::kBackwardAll, q, k, v, mask, output, lse, upstream, gradient_q, gradient_k, gradient_v, delta, batch, heads,
            queries, keys, radius, qs, ks, vs, os, us, stream);
}

// Reference Attention.hip:235-250.
int attention_fp32_backward_tiled(const float *q, const float *k, const float *v, const bool *mask, const float *output, const float *lse,
        const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, int batch, int heads, int queries,
        int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os,
        rocmkernels_strides us, hipStream_t stream) {
    return backward(32, 0, rk::kBackwardAll, q, k, v, mask, output, lse, upstream, gradient_q, gradient_k, gradient_v, delta, batch, heads,
            queries, keys, radius, qs, ks, vs, os, us, stream);
}

// Reference Attention.hip:419-438.
int attention_fp32_backward_tuned(const float *q, const float *k, const float *v, const bool *mask, const float *output, const float *lse,
        const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, int batch, int heads, int queries,
        int keys, int radius, int group, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os,
        rocmkernels_strides us, hipStream_t stream) {
    if (!valid_group(group)) return kInvalid;
    return backward(32, 0, rk::kBackwardAll, q, k, v, mask, output, lse, upstream, gradient_q, gradient_k, gradient_v, delta, batch, heads,
            queries, keys, radius, qs, ks, vs, os, us, stream);
}

// Reference Attention.hip:327-337.
int attention_fp32_backward_profile(const float *q, const float *k, const float *v, const bool *mask, const float *output,
        const float *lse, const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, int batch,
        int heads, int queries, int keys, int radius, int stage, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs,
        rocmkernels_strides os, rocmkernels_strides us, hipStream_t stream) {
    if (stage < 1 || stage > 3 || queries < 32 || radius < -1) return kInvalid;
    return backward(32, 0, static_cast<rk::BackwardStage>(stage), q, k, v, mask, output, lse, upstream, gradient_q, gradient_k, gradient_v,
            delta, batch, heads, queries, keys, radius, qs, ks, vs, os, us, stream);
}

// Reference Attention.hip:339-356.
int attention_fp32_query_profile(const float *q, const float *k, const float *v, const bool *mask, const float *output,
        const float *lse, const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, int batch,
        int heads, int queries, int keys, int radius, int tuning, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs,
        rocmkernels_strides os, rocmkernels_strides us, hipStream_t stream) {
    if (queries < 32 || radius < -1 || !valid_tuning(tuning)) return kInvalid;
    return backward(32, 0, rk::kBackwardQuery, q, k, v, mask, output, lse, upstream, gradient_q, gradient_k, gradient_v, delta, batch,
            heads, queries, keys, radius, qs, ks, vs, os, us, stream);
}

// Reference Attention64.hip:193-202.
int attention64_fp32_forward(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse, int batch,
        int heads, int queries, int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs,
        rocmkernels_strides os, hipStream_t stream) {
    return forward(64, 0, q, k, v, mask, output, lse, batch, heads, queries, keys, radius, qs, ks, vs, os, stream);
}

// Reference Attention64.hip:204-220.
int attention64_fp32_backward(const float *q, const float *k, const float *v, const bool *mask, const float *output, const float *lse,
        const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, int batch, int heads, int queries,
        int keys, int radius, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os,
        rocmkernels_strides us, hipStream_t stream) {
    return backward(64, 0, rk::kBackwardAll, q, k, v, mask, output, lse, upstream, gradient_q, gradient_k, gradient_v, delta, batch, heads,
            queries, keys, radius, qs, ks, vs, os, us, stream);
}

int attention_fp32_forward_flash_ex(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse,
        int batch, int heads, int queries, int keys, int radius, int flags, rocmkernels_strides qs, rocmkernels_strides ks,
        rocmkernels_strides vs, rocmkernels_strides os, hipStream_t stream) {
    if ((flags & ~ROCMKERNELS_ATTENTION_CAUSAL) != 0 || radius < -1) return kInvalid;
    return forward(32, flags, q, k, v, mask, output, lse, batch, heads, queries, keys, radius, qs, ks, vs, os, stream);
}

int attention_fp32_backward_ex(const float *q, const float *k, const float *v, const bool *mask, const float *output, const float *lse,
        const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, int batch, int heads, int queries,
        int keys, int radius, int flags, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os,
        rocmkernels_strides us, hipStream_t stream) {
    if (bad_backward_flags(flags) || radius < -1) return kInvalid;
    return backward(32, flags, backward_stage(flags), q, k, v, mask, output, lse, upstream, gradient_q, gradient_k, gradient_v, delta, batch,
            heads, queries, keys, radius, qs, ks, vs, os, us, stream);
}

int attention64_fp32_forward_ex(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse, int batch,
        int heads, int queries, int keys, int radius, int flags, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs,
        rocmkernels_strides os, hipStream_t stream) {
    if ((flags & ~ROCMKERNELS_ATTENTION_CAUSAL) != 0 || radius < -1) return kInvalid;
    return forward(64, flags, q, k, v, mask, output, lse, batch, heads, queries, keys, radius, qs, ks, vs, os, stream);
}

int attention64_fp32_backward_ex(const float *q, const float *k, const float *v, const bool *mask, const float *output, const float *lse,
        const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, int batch, int heads, int queries,
        int keys, int radius, int flags, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs, rocmkernels_strides os,
        rocmkernels_strides us, hipStream_t stream) {
    if (bad_backward_flags(flags) || radius < -1) return kInvalid;
    return backward(64, flags, backward_stage(flags), q, k, v, mask, output, lse, upstream, gradient_q, gradient_k, gradient_v, delta, batch,
            heads, queries, keys, radius, qs, ks, vs, os, us, stream);
}

// Reference Generic/Attention/AttentionGeneric.hip:291-309.
int attention_generic_forward(const void *q, const void *k, const void *v, const bool *mask, void *output, float *lse, int batch, int heads,
        int queries, int keys, int headWidth, int radius, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides vs,
        rocmkernels_strides os, rocmkernels_dtype dtype, hipStream_t stream) {
    if (!q || !k || !v || !mask || !output || !lse || bad_dims(batch, heads, queries, keys)) return kInvalid;
    if (headWidth != 16 && headWidth != 32 && headWidth != 64) return kInvalid;
    if (radius < -1) return kInvalid;
    if (dtype == ROCMKERNELS_DTYPE_FLOAT32) {
        const ForwardArgs a{static_cast<const float *>(q), static_cast<const float *>(k), static_cast<const float *>(v), mask,
                static_cast<float *>(output), lse, batch, heads, queries, keys, radius, 0, qs, ks, vs, os};
        return rk::launch_forward(headWidth, false, a, stream);
    }
    if (dtype == ROCMKERNELS_DTYPE_FLOAT16) {
        const rk::HalfForwardArgs a{q, k, v, mask, output, lse, batch, heads, queries, keys, radius, qs, ks, vs, os};
        return rk::launch_forward_f16(headWidth, a, stream);
    }
    return kInvalid;
}

// Reference Positional/Rotary.hip:44-56.
int rotary_fp32(const float *q, const float *k, const float *cos, const float *sin, float *oq, float *ok, int batch, int heads, int length,
        int backward, rocmkernels_strides qs, rocmkernels_strides ks, rocmkernels_strides cs, rocmkernels_strides ss, hipStream_t stream) {
    if (!q || !k || !cos || !sin || !oq || !ok || batch <= 0 || heads <= 0 || length <= 0) return kInvalid;
    const rk::RotaryArgs a{q, k, cos, sin, oq, ok, batch, heads, length, backward != 0, qs, ks, cs, ss};
    return rk::launch_rotary(a, stream);
}

} // extern "C"
