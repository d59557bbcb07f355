// GPU run of every namespaced C++ wrapper (include/ROCmKernels/...), the way the reference's tests drive its kernels
// (ROCmKernels.Tests/AttentionTests.cpp:162-224,254-264): device buffers, one call per wrapper on the default stream,
// results copied back. Built as a small shared library; tests/test_wrappers_gpu.py writes the inputs, calls
// wrapper_gpu_check() in its own process through ctypes (no child process: a process that has initialised the GPU must
// not exec another program) and compares every output bit for bit with the same call made through the C entry points,
// so a wrapper that swapped or dropped an argument fails.
//
// int wrapper_gpu_check(const char *dir, int B, int H, int L): returns the number of outputs written, or -1.
//   dir holds the inputs as raw little-endian arrays: q32 v32 (float, token-major [B][L][H][32]), k32 u32 (float,
//   [B][H][L][32] packed), q64 v64 (token-major [B][L][H][64]), k64 u64 ([B][H][L][64]), h64q h64k h64v (fp16 bits,
//   [B][H][L][64]), cos sin (float, [B][L][32]), mask (bytes, [B][L]). Every output is written to dir/out_<name>
//   (float, or fp16 bits for the generic fp16 output).
// Layouts: Q and V are read token-major ([B][L][H][D] storage, viewed through strides), K, dO and the outputs packed,
// so a qs/ks or vs/os mix-up changes the results.
#include <ROCmKernels/Kernels/Attention/Attention.hpp>
#include <ROCmKernels/Kernels/Attention/Attention64.hpp>
#include <ROCmKernels/Kernels/Generic/AttentionGeneric.hpp>
#include <ROCmKernels/Kernels/Positional/Rotary.hpp>

#include <cstdint>
#include <cstdio>
#include <type_traits>
#include <string>
#include <vector>

namespace {

struct Failure {
    std::string what;
};

// Device allocations of one run, freed when it ends (normally or by a Failure).
struct Buffers {
    std::vector<void *> all;
    ~Buffers() {
        for (void *p : all) (void)hipFree(p);
    }
    void *allocate(const size_t bytes) {
        void *p = nullptr;
        check(hipMalloc(&p, bytes), "hipMalloc");
        all.push_back(p);
        return p;
    }
    static void check(const hipError_t error, const char *what) {
        if (error != hipSuccess) throw Failure{std::string(what) + ": " + hipGetErrorString(error)};
    }
};

std::string dir;

template<class T>
std::vector<T> read_file(const std::string &name, const size_t count) {
    std::vector<T> data(count);
    FILE *f = std::fopen((dir + "/" + name).c_str(), "rb");
    const bool ok = f && std::fread(data.data(), sizeof(T), count, f) == count;
    if (f) std::fclose(f);
    if (!ok) throw Failure{"cannot read " + name};
    return data;
}

struct Output {
    std::string name;
    void *device;
    size_t bytes;
};

} // namespace

extern "C" __attribute__((visibility("default"))) int wrapper_gpu_check(const char *directory, const int B, const int H, const int L) {
    using namespace ROCmKernels::Kernels;
    dir = directory;
    Buffers buffers;
    std::vector<Output> outputs;
    const auto upload = [&](const auto &host) {
        using T = typename std::decay_t<decltype(host)>::value_type;
        void *p = buffers.allocate(host.size() * sizeof(T));
        Buffers::check(hipMemcpy(p, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy H2D");
        return static_cast<const T *>(p);
    };
    const auto output_of = [&](const std::string &name, const size_t count, const size_t size) {
        void *p = buffers.allocate(count * size);
        Buffers::check(hipMemset(p, 0xff, count * size), "hipMemset"); // NaN-filled: an output left unwritten is visible
        outputs.push_back(Output{name, p, count * size});
        return p;
    };
    const auto output = [&](const std::string &name, const size_t count) { return static_cast<float *>(output_of(name, count, 4)); };
    try {
        const size_t n32 = static_cast<size_t>(B) * H * L * 32, n64 = n32 * 2, rows = static_cast<size_t>(B) * H * L;

        const float *q32 = upload(read_file<float>("q32", n32)), *k32 = upload(read_file<float>("k32", n32));
        const float *v32 = upload(read_file<float>("v32", n32)), *u32 = upload(read_file<float>("u32", n32));
        const float *q64 = upload(read_file<float>("q64", n64)), *k64 = upload(read_file<float>("k64", n64));
        const float *v64 = upload(read_file<float>("v64", n64)), *u64 = upload(read_file<float>("u64", n64));
        const uint16_t *hq = upload(read_file<uint16_t>("h64q", n64)), *hk = upload(read_file<uint16_t>("h64k", n64));
        const uint16_t *hv = upload(read_file<uint16_t>("h64v", n64));
        const float *cosine = upload(read_file<float>("cos", static_cast<size_t>(B) * L * 32));
        const float *sine = upload(read_file<float>("sin", static_cast<size_t>(B) * L * 32));
        const bool *mask = reinterpret_cast<const bool *>(upload(read_file<uint8_t>("mask", static_cast<size_t>(B) * L)));

        // Token-major [B][L][H][D] storage for Q and V, packed [B][H][L][D] for everything else.
        const auto token_major = [&](const int D) { return Strides{L * H * D, D, H * D}; };
        const auto packed = [&](const int D) { return Strides{H * L * D, L * D, D}; };
        const Strides tm32 = token_major(32), pk32 = packed(32), tm64 = token_major(64), pk64 = packed(64);
        const Strides tables{L * 32, 0, 32};

        // 32-wide forward family.
        struct Fwd {
            float *o, *lse;
        };
        const auto fwd32 = [&](const std::string &name) { return Fwd{output(name + "_o", n32), output(name + "_lse", 2 * rows)}; };
        const Fwd simple = fwd32("forward");
        AttentionForward(q32, k32, v32, mask, simple.o, simple.lse, B, H, L, L, -1, tm32, pk32, tm32, pk32);
        const Fwd tiled = fwd32("forward_tiled");
        AttentionForwardTiled(q32, k32, v32, mask, tiled.o, tiled.lse, B, H, L, L, 5, tm32, pk32, tm32, pk32);
        const Fwd flash = fwd32("forward_flash");
        AttentionForwardFlash(q32, k32, v32, mask, flash.o, flash.lse, B, H, L, L, -1, tm32, pk32, tm32, pk32);
        const Fwd flash_tuned = fwd32("forward_flash_tuned");
        AttentionForwardFlashTuned(q32, k32, v32, mask, flash_tuned.o, flash_tuned.lse, B, H, L, L, 7, 13, tm32, pk32, tm32, pk32);
        const Fwd tuned = fwd32("forward_tuned");
        AttentionForwardTuned(q32, k32, v32, mask, tuned.o, tuned.lse, B, H, L, L, -1, 84, tm32, pk32, tm32, pk32);
        float *stats = output("statistics_lse", 2 * rows);
        AttentionStatistics(q32, k32, mask, stats, B, H, L, L, 9, tm32, pk32);
        const Fwd causal = fwd32("forward_flash_ex");
        AttentionForwardFlashEx(q32, k32, v32, mask, causal.o, causal.lse, B, H, L, L, -1, ROCMKERNELS_ATTENTION_CAUSAL, tm32, pk32, tm32, pk32);

        // 32-wide backward family, on the flash forward's O and lse (radius -1) and the causal forward's.
        struct Bwd {
            float *gq, *gk, *gv, *delta;
        };
        const auto bwd = [&](const std::string &name, const size_t n) {
            return Bwd{output(name + "_gq", n), output(name + "_gk", n), output(name + "_gv", n), output(name + "_delta", rows)};
        };
        const Bwd back = bwd("backward", n32);
        AttentionBackward(q32, k32, v32, mask, flash.o, flash.lse, u32, back.gq, back.gk, back.gv, back.delta, B, H, L, L, -1, tm32, pk32,
                tm32, pk32, pk32);
        const Bwd back_tiled = bwd("backward_tiled", n32);
        AttentionBackwardTiled(q32, k32, v32, mask, flash.o, flash.lse, u32, back_tiled.gq, back_tiled.gk, back_tiled.gv, back_tiled.delta, B, H,
                L, L, -1, tm32, pk32, tm32, pk32, pk32);
        const Bwd back_tuned = bwd("backward_tuned", n32);
        AttentionBackwardTuned(q32, k32, v32, mask, flash.o, flash.lse, u32, back_tuned.gq, back_tuned.gk, back_tuned.gv, back_tuned.delta, B, H,
                L, L, -1, 164, tm32, pk32, tm32, pk32, pk32);
        const Bwd back_ex = bwd("backward_ex", n32);
        AttentionBackwardEx(q32, k32, v32, mask, causal.o, causal.lse, u32, back_ex.gq, back_ex.gk, back_ex.gv, back_ex.delta, B, H, L, L, -1,
                ROCMKERNELS_ATTENTION_CAUSAL | ROCMKERNELS_ATTENTION_DETERMINISTIC, tm32, pk32, tm32, pk32, pk32);

        // 64-wide.
        float *o64 = output("forward64_o", n64), *lse64 = output("forward64_lse", 2 * rows);
        Attention64Forward(q64, k64, v64, mask, o64, lse64, B, H, L, L, 11, tm64, pk64, tm64, pk64);
        const Bwd back64 = bwd("backward64", n64);
        Attention64Backward(q64, k64, v64, mask, o64, lse64, u64, back64.gq, back64.gk, back64.gv, back64.delta, B, H, L, L, 11, tm64, pk64,
                tm64, pk64, pk64);
        float *o64c = output("forward64_ex_o", n64), *lse64c = output("forward64_ex_lse", 2 * rows);
        Attention64ForwardEx(q64, k64, v64, mask, o64c, lse64c, B, H, L, L, -1, ROCMKERNELS_ATTENTION_CAUSAL, tm64, pk64, tm64, pk64);
        const Bwd back64_ex = bwd("backward64_ex", n64);
        Attention64BackwardEx(q64, k64, v64, mask, o64c, lse64c, u64, back64_ex.gq, back64_ex.gk, back64_ex.gv, back64_ex.delta, B, H, L, L, -1,
                ROCMKERNELS_ATTENTION_CAUSAL | ROCMKERNELS_ATTENTION_DETERMINISTIC, tm64, pk64, tm64, pk64, pk64);

        // Generic forward: fp32 storage at width 32, fp16 storage at width 64.
        float *go = output("generic32_o", n32), *glse = output("generic32_lse", 2 * rows);
        AttentionGenericForward(q32, k32, v32, mask, go, glse, B, H, L, L, 32, 3, tm32, pk32, tm32, pk32, DType::Float32);
        uint16_t *ho = static_cast<uint16_t *>(output_of("generic16_o", n64, 2));
        float *hlse = output("generic16_lse", 2 * rows);
        AttentionGenericForward(hq, hk, hv, mask, ho, hlse, B, H, L, L, 64, -1, pk64, pk64, pk64, pk64, DType::Float16);

        // Rotary, forward and backward: Q token-major, K packed; outputs token-major packed [B][L][H][32].
        float *rq = output("rotary_q", n32), *rk = output("rotary_k", n32);
        Rotary(q32, k32, cosine, sine, rq, rk, B, H, L, false, tm32, pk32, tables, tables);
        float *bq = output("rotary_back_q", n32), *bk = output("rotary_back_k", n32);
        Rotary(q32, k32, cosine, sine, bq, bk, B, H, L, true, tm32, pk32, tables, tables);

        Buffers::check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        for (const Output &out : outputs) {
            std::vector<unsigned char> host(out.bytes);
            Buffers::check(hipMemcpy(host.data(), out.device, out.bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
            FILE *f = std::fopen((dir + "/out_" + out.name).c_str(), "wb");
            const bool ok = f && std::fwrite(host.data(), 1, out.bytes, f) == out.bytes;
            if (f) std::fclose(f);
            if (!ok) throw Failure{"cannot write out_" + out.name};
        }
    } catch (const Failure &failure) {
        std::fprintf(stderr, "wrapper_gpu_check: %s\n", failure.what.c_str());
        return -1;
    } catch (const ROCmKernels::HipError &error) {
        std::fprintf(stderr, "wrapper_gpu_check: %s\n", error.what());
        return -1;
    }
    return static_cast<int>(outputs.size());
}
