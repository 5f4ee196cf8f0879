// hbm_read.hip -- the read stream one MI355X sustains: a kernel that only reads a large buffer (16-byte loads,
// each workgroup a contiguous run, four loads in flight per lane) and writes one word per workgroup. Not part of the
// library; `make -C pingala8-llm_amd/csrc probe` builds ../p8x/hbm_read. Prints GB/s for 1 and 4 GiB over 20 runs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <vector>

#define CHECK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { std::printf("%s: %s\n", #x, hipGetErrorString(e_)); return 1; } } while (0)

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// workgroup b reads 16-byte words [b * per, (b + 1) * per) of src (per a multiple of 4 x 256), sums them, and
// writes the sum to out[b] so that nothing is optimized away
__global__ __launch_bounds__(256) void k_read(const u32x4 *__restrict__ src, size_t per, unsigned *__restrict__ out) {
    const u32x4 *p = src + (size_t)blockIdx.x * per;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (size_t i = threadIdx.x; i < per; i += 4 * 256) {
        const u32x4 a = __builtin_nontemporal_load(p + i), b = __builtin_nontemporal_load(p + i + 256);
        const u32x4 c = __builtin_nontemporal_load(p + i + 512), d = __builtin_nontemporal_load(p + i + 768);
        acc += a ^ b ^ c ^ d;
    }
    const unsigned v = acc.x ^ acc.y ^ acc.z ^ acc.w;
    __shared__ unsigned s[256];
    s[threadIdx.x] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned t = 0;
        for (int i = 0; i < 256; ++i) t ^= s[i];
        out[blockIdx.x] = t;
    }
}

int main() {
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    for (size_t gib : {1, 4}) {
        const size_t bytes = gib << 30, words = bytes / 16;
        const int grid = 2048;                       // 8 workgroups per CU
        const size_t per = words / grid;             // a multiple of 1024 for these sizes
        u32x4 *src = nullptr;
        unsigned *out = nullptr;
        CHECK(hipMalloc(&src, bytes));
        CHECK(hipMalloc(&out, grid * sizeof(unsigned)));
        CHECK(hipMemset(src, 1, bytes));
        std::vector<float> ms(20);
        for (int r = -2; r < 20; ++r) {
            CHECK(hipEventRecord(e0));
            hipLaunchKernelGGL(k_read, dim3(grid), dim3(256), 0, 0, src, per, out);
            CHECK(hipEventRecord(e1));
            CHECK(hipEventSynchronize(e1));
            if (r >= 0) CHECK(hipEventElapsedTime(&ms[r], e0, e1));
        }
        std::sort(ms.begin(), ms.end());
        std::printf("read %zu GiB: median %.1f us, %.0f GB/s (best %.0f GB/s)\n", gib, ms[10] * 1e3, bytes / (ms[10] * 1e-3) / 1e9,
                    bytes / (ms[0] * 1e-3) / 1e9);
        CHECK(hipFree(src));
        CHECK(hipFree(out));
    }
    return 0;
}
