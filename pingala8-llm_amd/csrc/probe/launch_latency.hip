// launch_latency.hip -- what a freshly launched workgroup waits for before it can work, on one MI355X: per workgroup
// s_memrealtime stamps (100 MHz) at kernel entry, after its first kernel-argument word is in, after a dependent
// load from device memory, and around two passes over one 4 KB block of straight-line code (1024 s_nop): the first
// pass fetches the block if the instruction cache does not hold it from an earlier launch, the second cannot miss,
// so their difference is the instruction-fetch cost and the second pass the issue rate of one wave. 256
// workgroups, 200 launches back to back on one stream; medians over workgroups, then over launches. Not part of the
// library; `make -C pingala8-llm_amd/csrc probe` builds ../p8x/launch_latency.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <vector>

#define CHECK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { std::printf("%s: %s\n", #x, hipGetErrorString(e_)); return 1; } } while (0)

typedef unsigned long long u64;

struct Args {
    const unsigned *dev;   // a device word the kernel reads after its arguments
    u64 *rec;              // [launches][256][5]
    int launch;
};

#define NOP8 "s_nop 0\n s_nop 0\n s_nop 0\n s_nop 0\n s_nop 0\n s_nop 0\n s_nop 0\n s_nop 0\n"
#define NOP64 NOP8 NOP8 NOP8 NOP8 NOP8 NOP8 NOP8 NOP8

__global__ __launch_bounds__(64) void k_probe(Args a) {
    const u64 t0 = __builtin_amdgcn_s_memrealtime();
    const int launch = a.launch;   // first kernel-argument words
    __asm__ volatile("" ::"s"(launch));
    const u64 t1 = __builtin_amdgcn_s_memrealtime();
    const unsigned v = *(const __attribute__((address_space(4))) unsigned *)a.dev;   // dependent scalar load
    __asm__ volatile("" ::"s"(v));
    const u64 t2 = __builtin_amdgcn_s_memrealtime();
    u64 pass[2];
#pragma unroll 1
    for (int it = 0; it < 2; ++it) {   // one copy of the block, run twice
        const u64 ta = __builtin_amdgcn_s_memrealtime();
        // 4 KB of code (1024 four-byte s_nop): 64 instruction-cache lines of 64 bytes
        __asm__ volatile(NOP64 NOP64 NOP64 NOP64 NOP64 NOP64 NOP64 NOP64 NOP64 NOP64 NOP64 NOP64 NOP64 NOP64 NOP64 NOP64);
        pass[it] = __builtin_amdgcn_s_memrealtime() - ta;
    }
    if (threadIdx.x == 0) {
        u64 *r = a.rec + ((size_t)launch * gridDim.x + blockIdx.x) * 5;
        r[0] = t0; r[1] = t1 - t0; r[2] = t2 - t1 + (v & 0u); r[3] = pass[0]; r[4] = pass[1];
    }
}

int main() {
    const int L = 200, G = 256;
    unsigned *dev = nullptr;
    u64 *rec = nullptr;
    CHECK(hipMalloc(&dev, 256));
    CHECK(hipMemset(dev, 0, 256));
    CHECK(hipMalloc(&rec, sizeof(u64) * L * G * 5));
    hipStream_t st;
    CHECK(hipStreamCreate(&st));
    for (int l = 0; l < L; ++l) {
        Args a{dev, rec, l};
        hipLaunchKernelGGL(k_probe, dim3(G), dim3(64), 0, st, a);
    }
    CHECK(hipStreamSynchronize(st));
    std::vector<u64> h((size_t)L * G * 5);
    CHECK(hipMemcpy(h.data(), rec, h.size() * sizeof(u64), hipMemcpyDeviceToHost));
    const char *names[4] = {"first kernel-argument word in", "dependent device-memory scalar load", "4 KB of code, first pass",
                            "the same 4 KB, second pass"};
    for (int k = 1; k <= 4; ++k) {
        std::vector<double> per_launch;
        for (int l = 10; l < L; ++l) {   // the first launches warm the code and the runtime
            std::vector<double> v;
            for (int g = 0; g < G; ++g) v.push_back(h[((size_t)l * G + g) * 5 + k] / 100.0);
            std::sort(v.begin(), v.end());
            per_launch.push_back(v[G / 2]);
        }
        std::sort(per_launch.begin(), per_launch.end());
        std::printf("%-40s median %.2f us (launch medians from %.2f to %.2f)\n", names[k - 1], per_launch[per_launch.size() / 2], per_launch.front(),
                    per_launch.back());
    }
    std::vector<double> ramp;
    for (int l = 10; l < L; ++l) {
        u64 lo = ~0ull, hi = 0;
        for (int g = 0; g < G; ++g) { lo = std::min(lo, h[((size_t)l * G + g) * 5]); hi = std::max(hi, h[((size_t)l * G + g) * 5]); }
        ramp.push_back((hi - lo) / 100.0);
    }
    std::sort(ramp.begin(), ramp.end());
    std::printf("%-40s median %.2f us\n", "dispatch ramp (last start - first start)", ramp[ramp.size() / 2]);
    CHECK(hipFree(dev));
    CHECK(hipFree(rec));
    return 0;
}
