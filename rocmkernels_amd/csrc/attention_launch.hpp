// Host-side launch interface between the C entry points (attention_abi.hip) and the kernels
// (attention_forward.hip, attention_backward.hip). Arguments are already validated when these are called.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>

#include <rocmkernels_attention.h>

namespace rk {

struct ForwardArgs {
    const float *q, *k, *v;
    const bool *mask;
    float *output, *lse;
    int batch, heads, queries, keys, radius, causal;
    rocmkernels_strides qs, ks, vs, os;
};

// fp16 storage (attention_generic_forward with dtype Float16): Q/K/V/output hold _Float16, lse stays fp32.
struct HalfForwardArgs {
    const void *q, *k, *v;
    const bool *mask;
    void *output;
    float *lse;
    int batch, heads, queries, keys, radius;
    rocmkernels_strides qs, ks, vs, os;
};

struct BackwardArgs {
    const float *q, *k, *v;
    const bool *mask;
    const float *output, *lse, *upstream;
    float *gradient_q, *gradient_k, *gradient_v, *delta;
    int batch, heads, queries, keys, radius, causal;
    rocmkernels_strides qs, ks, vs, os, us;
};

// Buffer resources address one (batch, head) sequence with 32-bit byte offsets. Kernels read up to one 32-row
// tile past the end (those reads return 0) and use offset 2^31 as "no row", so every sequence of every tensor,
// padded by one tile, must span less than 2 GiB. Offsets from the sequence start are unsigned, so the token stride
// must be non-negative (a token-reversed view is rejected); batch and head strides may have either sign.
inline bool sequence_fits(const int rows, const rocmkernels_strides &s, const int width) {
    const long long extent = (static_cast<long long>(rows) + 32) * s.token + width;
    return s.token >= 0 && extent * 4 < (1ll << 31);
}

// Waves per 32-row work item (see WorkItem in attention_device.hpp): split the streamed dimension over several waves
// when there are too few items to give every SIMD of the MI355X (1024) several waves of its own, not at all for
// large grids. Measured on MI355X for the forward: 4 waves per item below 4096 items; 2 from 4096 to 8191 (3-6.5%
// faster than 1 there, e.g. config 5, 4096 items at d=64: 105.6 -> 98.7 us); 1 from 8192 (2 is 3-5% slower there).
// The backward kernels, which hold twice the accumulators and merge them through LDS, prefer 2 from 2048 items.
inline int forward_split_for(const long long items) { return items >= 8192 ? 1 : items >= 4096 ? 2 : 4; }
inline int backward_split_for(const long long items) { return items >= 4096 ? 1 : items >= 2048 ? 2 : 4; }

// Compute units of the current device (256 on MI355X), queried once per device and then read from a process-wide
// cache (a device's CU count never changes), so a launch costs one hipGetDevice instead of an attribute query.
constexpr int kMaxCachedDevices = 64;
inline hipError_t compute_units(int &cus) {
    static std::atomic<int> cached[kMaxCachedDevices] = {};
    int device = 0;
    const hipError_t error = hipGetDevice(&device);
    if (error != hipSuccess) return error;
    const bool cacheable = device >= 0 && device < kMaxCachedDevices;
    if (cacheable) {
        const int known = cached[device].load(std::memory_order_relaxed);
        if (known > 0) {
            cus = known;
            return hipSuccess;
        }
    }
    const hipError_t query = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (query == hipSuccess && cacheable && cus > 0) cached[device].store(cus, std::memory_order_relaxed);
    return query;
}

// Workgroups of 4 waves covering `items` items of `split` waves each.
inline unsigned workgroups_for(const long long items, const int split) {
    const int per_group = 4 / split;
    return static_cast<unsigned>((items + per_group - 1) / per_group);
}

// Forward pass for head width D (16, 32 or 64). statistics_only writes lse and skips V and the output.
hipError_t launch_forward(int D, bool statistics_only, const ForwardArgs &a, hipStream_t stream);

struct RotaryArgs {
    const float *q, *k, *cos, *sin;
    float *oq, *ok;
    int batch, heads, length, backward;
    rocmkernels_strides qs, ks, cs, ss;
};

// 32-wide rotary embedding of Q and K (rotary.hip); outputs token-major [batch][token][head][32].
hipError_t launch_rotary(const RotaryArgs &a, hipStream_t stream);

// fp16-storage forward for head width D (16, 32 or 64) on the FP16 matrix cores.
hipError_t launch_forward_f16(int D, const HalfForwardArgs &a, hipStream_t stream);

enum BackwardStage {
    kBackwardAll = 0,    // delta, then dQ, then dK/dV
    kBackwardDelta = 1,  // delta only
    kBackwardQuery = 2,  // dQ only, reading delta
    kBackwardKeyValue = 3, // dK/dV only, reading delta
    kBackwardFused = 4,    // delta and dQ = 0, then dK/dV with dQ accumulated by atomics (not bit-reproducible)
    kBackwardAuto = 5,     // the faster of kBackwardFused and kBackwardAll for the call
};

hipError_t launch_backward(int D, BackwardStage stage, const BackwardArgs &a, hipStream_t stream);

// Fused single-kernel backward over key blocks (attention_backward_fused.hip) for D = 32 or 64 with 128-bit access
// (every pointer 16-byte aligned, every stride a multiple of 4); called by launch_backward for kBackwardFused.
hipError_t launch_fused_backward(int D, const BackwardArgs &a, int cus, hipStream_t stream);

// The fused backward's pre-pass alone: delta = sum(dO * O) per query row and dQ = 0 (dK/dV untouched).
hipError_t launch_backward_prepass(int D, const BackwardArgs &a, hipStream_t stream);

// Fused backward for radius windows (attention_backward_band.hip), D = 32 or 64 with 128-bit access: runs the pre-pass,
// then one persistent workgroup per CU over whole 128-key blocks with skewed query tiles.
hipError_t launch_band_backward(int D, const BackwardArgs &a, int cus, hipStream_t stream);

} // namespace rk
