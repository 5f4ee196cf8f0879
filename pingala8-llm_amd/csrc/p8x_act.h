// p8x_act.h -- activation prep shared by the standalone launches and the fused single-GEMV staging:
// x' = FWHT256(x * ic) / 16 per 256-block (CPU.patch:533-554), quantized to 8 bits per 128 columns
// (CPU.patch:559-571). Global address-space views only (no FLAT accesses in the kernels that include this).
#pragma once
#include <hip/hip_runtime.h>

#include "p8x_lane.h"

namespace p8x {

// correctly rounded f32 quotient via f64 (53 >= 2*24 + 2 bits: no double-rounding error)
__device__ __forceinline__ float div_rn(float a, float b) { return (float)((double)a / (double)b); }

typedef float f32x4 __attribute__((ext_vector_type(4)));

// the lane's 4 consecutive elements of one 256-block of x and of ic
struct BlockLane {
    f32x4 x, c;
    __device__ __forceinline__ void load(const float *__restrict__ xb, const float *__restrict__ icb, int lane) {
        x = as_global(reinterpret_cast<const f32x4 *>(xb))[lane];
        c = as_global(reinterpret_cast<const f32x4 *>(icb))[lane];
    }
};

// The 32-bit value held by lane (lane ^ M). M = 1, 2, 4, 8 stay inside 16-lane rows and use DPP row moves (VALU,
// no LDS traffic): quad_perm [1,0,3,2] and [2,3,0,1], row_ror:8, and for M = 4 row_ror:12 (lane i reads lane
// (i + 4) mod 16, the partner of lanes with bit 2 clear) or row_ror:4 (lane i - 4, for bit 2 set). M = 16 and 32
// use gfx950's lane swaps on two copies of the value (VALU): v_permlane16_swap exchanges the odd 16-lane rows of its
// first operand with the even rows of its second, so the copy that received row r ^ 1 is the second for even rows
// and the first for odd rows; v_permlane32_swap exchanges the upper 32 lanes of the first with the lower 32 of the
// second, so lanes 0..31 take the second copy and lanes 32..63 the first. Only the data movement differs from
// __shfl_xor; the arithmetic on the values is unchanged.
template <int M, typename T>
__device__ __forceinline__ T lane_xor(T v, int lane) {
    static_assert(sizeof(T) == 4, "32-bit values");
    const int iv = __builtin_bit_cast(int, v);
    int r;
    if constexpr (M == 1) r = __builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xF, 0xF, false);
    else if constexpr (M == 2) r = __builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xF, 0xF, false);
    else if constexpr (M == 4) {
        const int up = __builtin_amdgcn_update_dpp(0, iv, 0x12C, 0xF, 0xF, false);
        const int down = __builtin_amdgcn_update_dpp(0, iv, 0x124, 0xF, 0xF, false);
        r = (lane & 4) ? down : up;
    } else if constexpr (M == 8) r = __builtin_amdgcn_update_dpp(0, iv, 0x128, 0xF, 0xF, false);
    else if constexpr (M == 16) {
        const auto sw = __builtin_amdgcn_permlane16_swap((unsigned)iv, (unsigned)iv, false, false);
        r = (int)((lane & 16) ? sw[0] : sw[1]);
    } else if constexpr (M == 32) {
        const auto sw = __builtin_amdgcn_permlane32_swap((unsigned)iv, (unsigned)iv, false, false);
        r = (int)((lane & 32) ? sw[0] : sw[1]);
    } else r = __shfl_xor(iv, M);
    return __builtin_bit_cast(T, r);
}

// one butterfly stage across lanes: the lower index gets a + b, the upper a - b, with a the lower operand. Computed
// as p + s v with s = -1 for the upper lanes and +1 for the lower: s v is exact and the one rounding of the add gives
// p - v and v + p bit for bit (IEEE defines x - y as x + (-y)); the partner's value p reaches the add through its DPP
// operand, so a stage costs a multiply and an add instead of an add, a move, a subtract and a select.
template <int M>
__device__ __forceinline__ void fwht_lane_stage(float (&v)[4], int lane) {
    const float s = (lane & M) ? -1.f : 1.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float sv = s * v[e];
        v[e] = lane_xor<M>(v[e], lane) + sv;
    }
}

// x' for one 256-block from its loaded elements: lane holds 4 consecutive elements
__device__ __forceinline__ void rotate_block_lane(const BlockLane &in, int lane, float (&v)[4]) {
    const f32x4 xv = in.x, cv = in.c;
    v[0] = xv.x * cv.x; v[1] = xv.y * cv.y; v[2] = xv.z * cv.z; v[3] = xv.w * cv.w;
    // h = 1, 2 inside the lane
    { const float a0 = v[0], b0 = v[1], a1 = v[2], b1 = v[3]; v[0] = a0 + b0; v[1] = a0 - b0; v[2] = a1 + b1; v[3] = a1 - b1; }
    { const float a0 = v[0], b0 = v[2], a1 = v[1], b1 = v[3]; v[0] = a0 + b0; v[2] = a0 - b0; v[1] = a1 + b1; v[3] = a1 - b1; }
    // h = 4 .. 128 across lanes
    fwht_lane_stage<1>(v, lane);
    fwht_lane_stage<2>(v, lane);
    fwht_lane_stage<4>(v, lane);
    fwht_lane_stage<8>(v, lane);
    fwht_lane_stage<16>(v, lane);
    fwht_lane_stage<32>(v, lane);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] *= 0.0625f;
}

__device__ __forceinline__ float half_wave_max(float v, int lane) {
    v = fmaxf(v, lane_xor<1>(v, lane));
    v = fmaxf(v, lane_xor<2>(v, lane));
    v = fmaxf(v, lane_xor<4>(v, lane));
    v = fmaxf(v, lane_xor<8>(v, lane));
    return fmaxf(v, lane_xor<16>(v, lane));
}

__device__ __forceinline__ int half_wave_sum(int v, int lane) {
    v += lane_xor<1>(v, lane);
    v += lane_xor<2>(v, lane);
    v += lane_xor<4>(v, lane);
    v += lane_xor<8>(v, lane);
    return v + lane_xor<16>(v, lane);
}

// one 256-block to 8 bits per 128 columns: lane l gets the packed int8 of x' elements 4l..4l+3, the scale of its
// half (max |x'| / 127, correctly rounded) and the integer sum of its four values
__device__ __forceinline__ void quantize_loaded_q8_128(const BlockLane &in, int lane, uint32_t &packed, float &dd, int &sum) {
    float v[4];
    rotate_block_lane(in, lane, v);
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    am = half_wave_max(am, lane);
    dd = div_rn(am, 127.f);
    const float id = dd > 0.f ? div_rn(1.f, dd) : 0.f;
    int qi[4];
    sum = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) { qi[e] = __float2int_rn(v[e] * id); sum += qi[e]; }
    packed = (uint32_t)(uint8_t)qi[0] | ((uint32_t)(uint8_t)qi[1] << 8) | ((uint32_t)(uint8_t)qi[2] << 16) | ((uint32_t)(uint8_t)qi[3] << 24);
}

__device__ __forceinline__ void quantize_block_q8_128(const float *__restrict__ x, const float *__restrict__ ic, int lane, uint32_t &packed,
                                                      float &dd, int &sum) {
    BlockLane in;
    in.load(x, ic, lane);
    quantize_loaded_q8_128(in, lane, packed, dd, sum);
}

// ggml block_q8_1 of one rotated 256-block (quantize_row_q8_1_ref convention): lane l holds values 4l..4l+3, so the
// eight lanes 8i..8i+7 form 32-block i: d = max|x'| / 127 over it, q = round-half-away(x' / d), s = d * sum(q).
// dd and s are the float values the block stores as fp16.
__device__ __forceinline__ void quantize_block_q8_1(const float *__restrict__ x, const float *__restrict__ ic, int lane, uint32_t &packed,
                                                    float &dd, float &s) {
    BlockLane in;
    in.load(x, ic, lane);
    float v[4];
    rotate_block_lane(in, lane, v);
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) am = fmaxf(am, __shfl_xor(am, m));
    dd = div_rn(am, 127.f);
    const float id = dd != 0.f ? div_rn(1.f, dd) : 0.f;
    int qi[4], sum = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) { qi[e] = (int)roundf(v[e] * id); sum += qi[e]; }
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) sum += __shfl_xor(sum, m);
    s = (float)sum * dd;
    packed = (uint32_t)(uint8_t)qi[0] | ((uint32_t)(uint8_t)qi[1] << 8) | ((uint32_t)(uint8_t)qi[2] << 16) | ((uint32_t)(uint8_t)qi[3] << 24);
}

}  // namespace p8x
