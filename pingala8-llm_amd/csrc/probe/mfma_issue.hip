// mfma_issue.hip -- what the prompt GEMM's inner loop can reach on one MI355X: v_mfma_f32_32x32x16_f16 throughput
// alone, with independent VALU instructions between the MFMAs, and with the GEMM's per-step mix of LDS operand
// reads, table reads and VALU (the decode). Not part of the library; `make -C pingala8-llm_amd/csrc probe` builds
// ../p8x/mfma_issue. One workgroup of four waves per CU (one wave per SIMD) unless stated; no global memory traffic
// inside the timed loops.
#include <hip/hip_runtime.h>

#include <cstdio>

typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

#define CHECK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { std::printf("%s: %s\n", #x, hipGetErrorString(e_)); return 1; } } while (0)

// 8 independent accumulators; V v_pk_add_f16 (inline asm, so the count is exact) after each MFMA
template <int V>
__global__ __launch_bounds__(256) void k_mix(float *out, int iters) {
    half8v a, b;
    for (int i = 0; i < 8; ++i) { a[i] = (_Float16)(threadIdx.x * 0.001f + i); b[i] = (_Float16)(i * 0.5f); }
    float16v acc[8];
    for (int k = 0; k < 8; ++k) acc[k] = float16v{};
    uint32_t x[8], y = threadIdx.x;
    for (int k = 0; k < 8; ++k) x[k] = threadIdx.x * (k + 1);
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[k], 0, 0, 0);
#pragma unroll
            for (int v = 0; v < V; ++v) __asm__ volatile("v_pk_add_f16 %0, %0, %1" : "+v"(x[v & 7]) : "v"(y));
        }
    }
    float s = 0.f;
    uint32_t xs = 0;
    for (int k = 0; k < 8; ++k) {
        for (int q = 0; q < 16; ++q) s += acc[k][q];
        xs += x[k];
    }
    out[blockIdx.x * 256 + threadIdx.x] = s + (float)xs;
}

// One GEMM step shape: NA 16-byte x' operand reads and NT table-word reads from LDS (read one step ahead), V VALU,
// 16 MFMAs (NA token tiles x 16 / NA row tiles); the next step's LDS addresses depend on this step's VALU.
template <int NA, int NT, int V>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_step(float *out, int iters) {
    constexpr int NR = 16 / NA;
    __shared__ __attribute__((aligned(16))) _Float16 xs[NA * 32 * 128];
    __shared__ uint32_t tab[8192];
    const int lane = threadIdx.x & 63, j = lane & 31, kh = lane >> 5;
    for (int i = threadIdx.x; i < NA * 32 * 128; i += 256) xs[i] = (_Float16)(i & 7);
    for (int i = threadIdx.x; i < 8192; i += 256) tab[i] = i * 2654435761u;
    __syncthreads();
    float16v acc[NA][NR];
    for (int a = 0; a < NA; ++a)
        for (int r = 0; r < NR; ++r) acc[a][r] = float16v{};
    half8v A[NA], B[NR];
    uint32_t W[NT > 0 ? NT : 1] = {};
    for (int r = 0; r < NR; ++r)
        for (int i = 0; i < 8; ++i) B[r][i] = (_Float16)(0.01f * (r + i));
    uint32_t addr = (lane * 4) & 8191;
    for (int a = 0; a < NA; ++a) A[a] = half8v{};
    for (int it = 0; it < iters; ++it) {
        const int s8 = it & 7;
        half8v An[NA];
        uint32_t Wn[NT > 0 ? NT : 1];
#pragma unroll
        for (int a = 0; a < NA; ++a) An[a] = *reinterpret_cast<const half8v *>(xs + (32 * a + j) * 128 + 8 * ((8 * kh + s8) ^ (j & 15)));
#pragma unroll
        for (int t = 0; t < NT; ++t) Wn[t] = tab[(addr + 64 * t + 256 * s8) & 8191];
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int r = 0; r < NR; ++r) acc[a][r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[a], B[r], acc[a][r], 0, 0, 0);
        uint32_t x0 = 0, x1 = 0, x2 = 0, x3 = 0;
#pragma unroll
        for (int v = 0; v < V / 4; ++v) {
            __asm__ volatile("v_pk_add_f16 %0, %0, %1" : "+v"(x0) : "v"(W[0]));
            __asm__ volatile("v_pk_add_f16 %0, %0, %1" : "+v"(x1) : "v"(W[NT > 1 ? 1 : 0]));
            __asm__ volatile("v_pk_add_f16 %0, %0, %1" : "+v"(x2) : "v"(W[NT > 2 ? 2 : 0]));
            __asm__ volatile("v_pk_add_f16 %0, %0, %1" : "+v"(x3) : "v"(W[NT > 3 ? 3 : 0]));
        }
        addr = (addr + x0 + x1 + x2 + x3) & 8191 & ~3u;
        for (int a = 0; a < NA; ++a) A[a] = An[a];
        for (int t = 0; t < NT; ++t) W[t] = Wn[t];
    }
    float s = 0.f;
    for (int a = 0; a < NA; ++a)
        for (int r = 0; r < NR; ++r)
            for (int q = 0; q < 16; ++q) s += acc[a][r][q];
    out[blockIdx.x * 256 + threadIdx.x] = s + (float)addr;
}

static hipEvent_t e0, e1;

template <int V>
static int run_mix(float *out, int wg_per_cu) {
    const int grid = 256 * wg_per_cu, iters = 2000;
    hipLaunchKernelGGL(k_mix<V>, dim3(grid), dim3(256), 0, 0, out, iters);
    CHECK(hipEventRecord(e0));
    hipLaunchKernelGGL(k_mix<V>, dim3(grid), dim3(256), 0, 0, out, iters);
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    const double fl = 2.0 * 32 * 32 * 16 * 8.0 * iters * grid * 4;
    std::printf("mix: %2d VALU after each MFMA, %d wave(s) per SIMD: %7.1f TFLOP/s, %5.1f ns per MFMA per wave\n", V, wg_per_cu,
                fl / (ms * 1e-3) / 1e12, ms * 1e6 / (8.0 * iters));
    return 0;
}

template <int NA, int NT, int V>
static int run_step(float *out) {
    const int iters = 2000;
    hipLaunchKernelGGL((k_step<NA, NT, V>), dim3(256), dim3(256), 0, 0, out, iters);
    CHECK(hipEventRecord(e0));
    hipLaunchKernelGGL((k_step<NA, NT, V>), dim3(256), dim3(256), 0, 0, out, iters);
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    std::printf("step: %d x' reads, %2d table reads, %2d VALU per 16 MFMAs: %5.1f ns per MFMA per wave\n", NA, NT, V, ms * 1e6 / (16.0 * iters));
    return 0;
}

int main() {
    float *out = nullptr;
    CHECK(hipMalloc(&out, 512 * 256 * sizeof(float)));   // the largest grid: 512 workgroups x 256 threads
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    int rc = 0;
    for (int wpc = 1; wpc <= 2 && !rc; ++wpc)
        rc = run_mix<0>(out, wpc) || run_mix<2>(out, wpc) || run_mix<4>(out, wpc) || run_mix<6>(out, wpc) || run_mix<8>(out, wpc) || run_mix<12>(out, wpc);
    if (!rc)
        rc = run_step<4, 0, 0>(out) || run_step<4, 8, 0>(out) || run_step<4, 8, 48>(out) || run_step<4, 8, 76>(out) || run_step<8, 0, 0>(out) ||
             run_step<8, 4, 0>(out) || run_step<8, 4, 24>(out) || run_step<8, 4, 36>(out) || run_step<8, 4, 48>(out);
    CHECK(hipDeviceSynchronize());
    CHECK(hipFree(out));
    return rc;
}
