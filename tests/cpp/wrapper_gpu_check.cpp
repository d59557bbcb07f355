// GPU run of every namespaced C++ wrapper (include/ROCmKernels/...), the way the reference's tests drive its kernels
// (ROCmKernels.Tests/AttentionTests.cpp:162-224,254-264): device buffers, one call per wrapper on the default stream,
// results copied back. tests/test_wrappers_gpu.py writes the inputs, runs this program and compares every output bit
// for bit with the same call made through the C entry points (ctypes), so a wrapper that swapped or dropped an argument
// fails.
//
// usage: wrapper_gpu_check DIR B H L
//   DIR holds the inputs as raw little-endian arrays: q32 k32 v32 u32 (float, [B][H][L][32] packed), q64 k64 v64 u64
//   (float, [B][H][L][64]), h64q h64k h64v (fp16 bits, [B][H][L][64]), cos sin (float, [B][L][32]), mask (bytes,
//   [B][L]). Every output is written to DIR/out_<name> (float, or fp16 bits for the generic fp16 output).
// Layouts: Q and V are read token-major ([B][L][H][D] storage, viewed through strides), K, dO and the outputs packed,
// so a qs/ks or vs/os mix-up changes the results.
#include <ROCmKernels/Kernels/Attention/Attention.hpp>
#include <ROCmKernels/Kernels/Attention/Attention64.hpp>
#include <ROCmKernels/Kernels/Generic/AttentionGeneric.hpp>
#include <ROCmKernels/Kernels/Positional/Rotary.hpp>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

namespace {

std::string dir;

void check(const hipError_t error, const char *what) {
    if (error != hipSuccess) {
        std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(error));
        std::exit(2);
    }
}

template<class T>
std::vector<T> read_file(const std::string &name, const size_t count) {
    std::vector<T> data(count);
    FILE *f = std::fopen((dir + "/" + name).c_str(), "rb");
    if (!f || std::fread(data.data(), sizeof(T), count, f) != count) {
        std::fprintf(stderr, "cannot read %s (%zu values)\n", name.c_str(), count);
        std::exit(2);
    }
    std::fclose(f);
    return data;
}

template<class T>
T *upload(const std::vector<T> &host) {
    void *p = nullptr;
    check(hipMalloc(&p, host.size() * sizeof(T)), "hipMalloc");
    check(hipMemcpy(p, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy H2D");
    return static_cast<T *>(p);
}

struct Output {
    std::string name;
    void *device;
    size_t bytes;
};
std::vector<Output> outputs;

template<class T = float>
T *output(const std::string &name, const size_t count) {
    void *p = nullptr;
    check(hipMalloc(&p, count * sizeof(T)), "hipMalloc");
    check(hipMemset(p, 0xff, count * sizeof(T)), "hipMemset"); // NaN-filled: an output left unwritten is visible
    outputs.push_back(Output{name, p, count * sizeof(T)});
    return static_cast<T *>(p);
}

} // namespace

int main(int argc, char **argv) {
    using namespace ROCmKernels::Kernels;
    if (argc != 5) {
        std::fprintf(stderr, "usage: %s DIR B H L\n", argv[0]);
        return 2;
    }
    dir = argv[1];
    const int B = std::atoi(argv[2]), H = std::atoi(argv[3]), L = std::atoi(argv[4]);
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
    uint16_t *ho = output<uint16_t>("generic16_o", n64);
    float *hlse = output("generic16_lse", 2 * rows);
    AttentionGenericForward(hq, hk, hv, mask, ho, hlse, B, H, L, L, 64, -1, pk64, pk64, pk64, pk64, DType::Float16);

    // Rotary, forward and backward: Q token-major, K packed; outputs token-major packed [B][L][H][32].
    float *rq = output("rotary_q", n32), *rk = output("rotary_k", n32);
    Rotary(q32, k32, cosine, sine, rq, rk, B, H, L, false, tm32, pk32, tables, tables);
    float *bq = output("rotary_back_q", n32), *bk = output("rotary_back_k", n32);
    Rotary(q32, k32, cosine, sine, bq, bk, B, H, L, true, tm32, pk32, tables, tables);

    check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    for (const Output &out : outputs) {
        std::vector<unsigned char> host(out.bytes);
        check(hipMemcpy(host.data(), out.device, out.bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
        FILE *f = std::fopen((dir + "/out_" + out.name).c_str(), "wb");
        if (!f || std::fwrite(host.data(), 1, out.bytes, f) != out.bytes) {
            std::fprintf(stderr, "cannot write out_%s\n", out.name.c_str());
            return 2;
        }
        std::fclose(f);
    }
    std::printf("%zu outputs written\n", outputs.size());
    return 0;
}
