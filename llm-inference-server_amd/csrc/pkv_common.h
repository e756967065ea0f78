// Internal helpers shared by the libpagedkv kernels: dtype tags, 16-byte vector
// access, bf16/fp16 <-> fp32 conversion, wave64 cross-lane reductions, and the
// thread-local error string behind pkv_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pagedkv.h"

namespace pkv {

// ------------------------------------------------------------------ errors
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// Checks hipGetLastError() after a launch; returns PKV_OK or fail(PKV_EHIP, ...).
int check_launch(const char* what);

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ------------------------------------------------------------------ element types
// Storage types: fp32 as float, fp16 as _Float16, bf16 as raw 16-bit words (the
// conversions below are exact widening and round-to-nearest-even narrowing, the
// same rounding torch's `.to(bfloat16)` applies).
struct bf16_t {
    uint16_t bits;
};

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16_t x) {
    return __builtin_bit_cast(float, (uint32_t)x.bits << 16);
}

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float x) { return (_Float16)x; }
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) {
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
        return bf16_t{(uint16_t)((u >> 16) | 0x0040u)};  // quiet NaN stays NaN
    }
    u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest, ties to even
    return bf16_t{(uint16_t)(u >> 16)};
}

// The two fp32 values packed in one 32-bit word of a 16-bit dtype (element 2k in the
// low half, 2k+1 in the high half, i.e. memory order).
template <typename T>
struct Pair;
template <>
struct Pair<_Float16> {
    __device__ __forceinline__ static float lo(uint32_t w) {
        return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
    }
    __device__ __forceinline__ static float hi(uint32_t w) {
        return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
    }
    // acc + a.lo * b.lo + a.hi * b.hi in one v_dot2_f32_f16.
    __device__ __forceinline__ static float dot2(uint32_t a, uint32_t b, float acc) {
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b),
                                      acc, false);
    }
};
template <>
struct Pair<bf16_t> {
    __device__ __forceinline__ static float lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
    __device__ __forceinline__ static float hi(uint32_t w) {
        return __builtin_bit_cast(float, w & 0xffff0000u);
    }
    __device__ __forceinline__ static float dot2(uint32_t a, uint32_t b, float acc) {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                               __builtin_bit_cast(bf16x2_t, b), acc, false);
    }
};

// 16 bytes, the widest global load/store a lane issues (global_load_dwordx4).
struct alignas(16) Vec16 {
    uint32_t w[4];
};
__device__ __forceinline__ Vec16 load16(const void* p) {
    uint4 v = *reinterpret_cast<const uint4*>(p);
    return Vec16{{v.x, v.y, v.z, v.w}};
}
__device__ __forceinline__ void store16(void* p, const Vec16& v) {
    *reinterpret_cast<uint4*>(p) = make_uint4(v.w[0], v.w[1], v.w[2], v.w[3]);
}

// Streaming (nontemporal) loads for data read exactly once, such as K/V rows in
// decode: the `nt` hint keeps them from displacing reusable lines in L2/MALL. A plain
// read-only stream measured 6.8 TB/s on MI355X with these against 6.4 TB/s without.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ Vec16 load16_stream(const void* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return Vec16{{v.x, v.y, v.z, v.w}};
}
__device__ __forceinline__ uint2 load8_stream(const void* p) {
    const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    return make_uint2(v.x, v.y);
}

// ------------------------------------------------------------------ wave64 lanes
__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63u); }

// A 64-bit value of one lane, broadcast (wave-uniform, lands in SGPRs).
__device__ __forceinline__ int64_t readlane64(int64_t v, int lane) {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)(uint64_t)v, lane);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)v >> 32), lane);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// DPP moves within a row of 16 lanes (bound_ctrl: every lane reads a valid source).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}
constexpr int kDppQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141; // lane i <-> 7-i within each half row
constexpr int kDppRowMirror = 0x140;     // lane i <-> 15-i within each row
constexpr int kDppRowRor8 = 0x128;       // lane i <- (i+8) mod 16 (i.e. i ^ 8)

__device__ __forceinline__ float quad_sum(float x) {
    x += dpp_f32<kDppQuadXor1>(x);
    x += dpp_f32<kDppQuadXor2>(x);
    return x;
}
// Sum over each aligned group of 8 lanes (every lane of the group gets it).
__device__ __forceinline__ float octet_sum(float x) {
    x = quad_sum(x);
    x += dpp_f32<kDppRowHalfMirror>(x);
    return x;
}

// Value of lane (id ^ 16) / (id ^ 32), from gfx950's permlane swaps: with both
// operands equal, one result holds this lane's own value and the other its partner's,
// so op(r0, r1) == op(own, partner) for a commutative op.
struct SwapPair {
    float a, b;
};
__device__ __forceinline__ SwapPair swap16(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                              false, false);
    return SwapPair{__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
}
__device__ __forceinline__ SwapPair swap32(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                              false, false);
    return SwapPair{__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
}
// x combined with its value in the lane 32 apart, in every lane: swap32 of two copies of
// x leaves the lower half's value in one result and the upper half's in the other, so no
// select of the partner's value is needed.
__device__ __forceinline__ float max_across32(float x) {
    const SwapPair s = swap32(x);
    return fmaxf(s.a, s.b);
}
__device__ __forceinline__ float sum_across32(float x) {
    const SwapPair s = swap32(x);
    return s.a + s.b;
}

// Reductions over each row of 16 lanes (every lane of the row gets its row's result).
__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp_f32<kDppQuadXor1>(x));
    x = fmaxf(x, dpp_f32<kDppQuadXor2>(x));
    x = fmaxf(x, dpp_f32<kDppRowHalfMirror>(x));
    return fmaxf(x, dpp_f32<kDppRowMirror>(x));
}
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_f32<kDppQuadXor1>(x);
    x += dpp_f32<kDppQuadXor2>(x);
    x += dpp_f32<kDppRowHalfMirror>(x);
    return x + dpp_f32<kDppRowMirror>(x);
}

// Full-wave reductions: DPP inside each 16-lane row, then the two permlane swaps.
// Every lane ends with the result.
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp_f32<kDppQuadXor1>(x));
    x = fmaxf(x, dpp_f32<kDppQuadXor2>(x));
    x = fmaxf(x, dpp_f32<kDppRowHalfMirror>(x));
    x = fmaxf(x, dpp_f32<kDppRowMirror>(x));
    SwapPair s = swap16(x);
    x = fmaxf(s.a, s.b);
    s = swap32(x);
    return fmaxf(s.a, s.b);
}
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp_f32<kDppQuadXor1>(x);
    x += dpp_f32<kDppQuadXor2>(x);
    x += dpp_f32<kDppRowHalfMirror>(x);
    x += dpp_f32<kDppRowMirror>(x);
    SwapPair s = swap16(x);
    x = s.a + s.b;
    s = swap32(x);
    return s.a + s.b;
}

// Sum over the lanes that share (lane % STRIDE), STRIDE in {8, 16, 32, 64}.
template <int STRIDE>
__device__ __forceinline__ float fold_lanes(float x) {
    if constexpr (STRIDE <= 8) x += dpp_f32<kDppRowRor8>(x);
    if constexpr (STRIDE <= 16) {
        SwapPair s = swap16(x);
        x = s.a + s.b;
    }
    if constexpr (STRIDE <= 32) {
        SwapPair s = swap32(x);
        x = s.a + s.b;
    }
    return x;
}

// Workgroup barrier that orders LDS only. __syncthreads() also fences global memory,
// which makes every wave wait for ALL of its outstanding global loads at the barrier;
// this one lets prefetched loads stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Orders one wave's LDS writes before its own later LDS reads, including reads by
// other lanes of the same wave, without a workgroup barrier: the DS instructions of a
// wave execute in order, so this only has to stop the compiler from moving memory
// operations across it.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// 2^x on the hardware exponential unit (v_exp_f32). Softmax here runs in the base-2
// domain: scores are pre-multiplied by log2(e), so exp(s - m) == exp2(s' - m').
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// s_waitcnt immediate (gfx9 encoding) waiting until at most N vector-memory operations
// are outstanding, leaving the export and LDS/scalar counters unconstrained.
template <int N>
constexpr int kWaitVm = (N & 0xf) | (0x7 << 4) | (0xf << 8) | (((N >> 4) & 0x3) << 14);
// s_waitcnt immediate waiting until no LDS (or scalar-memory) operation of this wave is
// outstanding, leaving the vector-memory and export counters unconstrained.
constexpr int kWaitLgkm0 = 0xf | (0x7 << 4) | (0x0 << 8) | (0x3 << 14);
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// A score as the reference's gather path holds it when its softmax reads it
// (core/attention.py:146, :176): the q.k dot product rounded to the pool dtype (the
// matmul's output tensor), times `scale` and rounded again (the `* scale` on that
// tensor), then carried into the base-2 domain for exp2. For fp32 pools both roundings
// are the identity and the product is rounded once, as in fp32 torch.
template <typename T>
__device__ __forceinline__ float ref_score_log2(float dot, float scale) {
    return to_f32(from_f32<T>(to_f32(from_f32<T>(dot)) * scale)) * kLog2e;
}

}  // namespace pkv
