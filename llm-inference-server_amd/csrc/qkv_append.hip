// QKV projection with the KV append in its epilogue (fp16/bf16, gfx950).
//
// Per layer of a decode step the reference projects the hidden rows with the fused
// QKV weight (HF GPT-2's c_attn, a Conv1D: addmm(bias, x, W) with W [in, q + 2 kv]),
// splits the result, transposes K and V to [T, Hkv, D] views and scatters them into
// the pool (core/paged_executor.py:116-125: pool.k[l].view(-1, H, D).index_copy_(0,
// write_slots, k), the same for V). Here one launch computes out = x · W + b and, in
// the epilogue, stores each K and V element both into `out` (so the caller's tensor
// is the complete projection) and at its row's pool slot: no strided transpose, no
// index_copy_, no append launch.
//
//  * The weight is taken transposed, Wt [N, in] with `in` contiguous (the caller keeps
//    one transposed copy per layer), so both MFMA operands are 16-byte loads of 8
//    consecutive k of a weight row and a hidden row.
//  * Few rows (decode batches) make this a GEMV over the weight: a workgroup takes one
//    16-column tile of the output (v_mfma_f32_16x16x32; 32-column tiles on 32x32x16
//    when `in` is not a multiple of 32) and its waves split the `in` dimension; their
//    fp32 partial tiles are summed through LDS by wave 0 (in wave order, so the result
//    is deterministic), which adds the bias, rounds once to the model dtype and stores.
//  * Each lane holds 4 consecutive output columns of one row, so it stores 8 bytes at a
//    time: into `out`, and for K / V columns into the pool row of its slot (4
//    consecutive head_dim elements of one head).
// Slots outside the pool are skipped (the host layer raises before the call).
#include "pkv_common.h"

namespace pkv {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct QkvMfma;
template <>
struct QkvMfma<_Float16> {
    __device__ __forceinline__ static f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
};
template <>
struct QkvMfma<bf16_t> {
    __device__ __forceinline__ static f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    }
};

template <typename T>
__device__ __forceinline__ uint16_t bits_of(float x) {
    return __builtin_bit_cast(uint16_t, from_f32<T>(x));
}

struct QkvArgs {
    const void* x;             // [rows, in], row stride x_st (elements)
    const void* wt;            // [N, in], row stride wt_st
    const void* bias;          // [N] or null
    void* out;                 // [rows, N], row stride out_st
    char* k_pool;
    char* v_pool;
    const int64_t* slots;      // [rows]
    int64_t x_st, wt_st, out_st;
    int64_t sb, ss, sh;        // pool strides in bytes: block, slot, head
    int64_t num_slots;         // num_blocks * block_size
    int block_size;
    int rows, in, n, nq;       // nq = query columns; then K (kvw columns), then V (kvw)
    int kvw, head_dim;
};

constexpr int kKS = 8;   // waves per workgroup, splitting the `in` dimension
constexpr int kU = 4;    // k-steps (16 elements each) per load block

// 32-column tiles on v_mfma_f32_32x32x16 (16-element k steps): the kernel for an
// `in` that is a multiple of 16 but not of 32. A = 8 elements of weight row n0 + (lane
// % 32), B = 8 of hidden row m0 + (lane % 32); accumulator register r of lane l is
// output column n0 + 8 (r / 4) + 4 (l / 32) + r % 4 of row m0 + l % 32.
template <typename T>
__global__ __launch_bounds__(kKS * 64) void qkv_append_kernel(const QkvArgs a) {
    __shared__ f32x4 red[kKS - 1][4][64];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int col = lane & 31;
    const int half = lane >> 5;
    const int n0 = (int)blockIdx.x * 32;
    const int ksteps = a.in / 16;
    const int per = (ksteps + kKS - 1) / kKS;
    const int kb0 = min(ksteps, wave * per);
    const int kb1 = min(ksteps, kb0 + per);
    const int nsteps = kb1 - kb0;
    // Columns past N re-read the last row of Wt; their results are never stored.
    const T* wp = static_cast<const T*>(a.wt) + (int64_t)min(n0 + col, a.n - 1) * a.wt_st + half * 8 + 16 * kb0;
    // The epilogue's inputs (this lane's 16 bias values, its row's slot) are loaded
    // before the GEMM so the epilogue issues no dependent global load.
    float bias[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int n = n0 + 8 * (r >> 2) + 4 * half + (r & 3);
        bias[r] = (a.bias && n < a.n) ? to_f32(static_cast<const T*>(a.bias)[n]) : 0.f;
    }
    int64_t slot_next = a.slots[min(col, a.rows - 1)];

    for (int m0 = 0; m0 < a.rows; m0 += 32) {
        const int64_t slot = slot_next;
        if (m0 + 32 < a.rows) slot_next = a.slots[min(m0 + 32 + col, a.rows - 1)];
        const T* xp = static_cast<const T*>(a.x) + (int64_t)min(m0 + col, a.rows - 1) * a.x_st + half * 8 + 16 * kb0;
        f32x16 acc = f32x16{};
        const int nblk = nsteps / kU;
        u32x4 a0[kU], b0[kU], a1[kU], b1[kU];
        auto load_blk = [&](u32x4(&wa)[kU], u32x4(&xb)[kU], int kb) {
#pragma unroll
            for (int u = 0; u < kU; ++u) wa[u] = *reinterpret_cast<const u32x4*>(wp + kb + 16 * u);
#pragma unroll
            for (int u = 0; u < kU; ++u) xb[u] = *reinterpret_cast<const u32x4*>(xp + kb + 16 * u);
        };
        auto mma_blk = [&](const u32x4(&wa)[kU], const u32x4(&xb)[kU]) {
#pragma unroll
            for (int u = 0; u < kU; ++u) acc = QkvMfma<T>::run(wa[u], xb[u], acc);
        };
        int i = 0;
        if (nblk > 0) load_blk(a0, b0, 0);
        for (; i + 1 < nblk; i += 2) {
            load_blk(a1, b1, (i + 1) * 16 * kU);
            mma_blk(a0, b0);
            if (i + 2 < nblk) load_blk(a0, b0, (i + 2) * 16 * kU);
            mma_blk(a1, b1);
        }
        if (i < nblk) mma_blk(a0, b0);
        for (int k = nblk * 16 * kU; k < nsteps * 16; k += 16)
            acc = QkvMfma<T>::run(*reinterpret_cast<const u32x4*>(wp + k), *reinterpret_cast<const u32x4*>(xp + k), acc);

        if (wave > 0) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                red[wave - 1][q][lane] = f32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll 1
            for (int w = 0; w < kKS - 1; ++w)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const f32x4 y = red[w][q][lane];
                    acc[4 * q] += y[0];
                    acc[4 * q + 1] += y[1];
                    acc[4 * q + 2] += y[2];
                    acc[4 * q + 3] += y[3];
                }
            const int m = m0 + col;
            if (m < a.rows) {
                const bool in_pool = (uint64_t)slot < (uint64_t)a.num_slots;
                const int64_t slot_ofs = in_pool ? (slot / a.block_size) * a.sb + (slot % a.block_size) * a.ss : 0;
                char* orow = static_cast<char*>(a.out) + (int64_t)m * a.out_st * 2;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int n = n0 + 8 * j + 4 * half;
                    if (n >= a.n) continue;
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = acc[4 * j + e] + bias[4 * j + e];
                    const uint2 word = make_uint2((uint32_t)bits_of<T>(v[0]) | ((uint32_t)bits_of<T>(v[1]) << 16),
                                                  (uint32_t)bits_of<T>(v[2]) | ((uint32_t)bits_of<T>(v[3]) << 16));
                    *reinterpret_cast<uint2*>(orow + (int64_t)n * 2) = word;
                    if (n >= a.nq && in_pool) {
                        const int idx = n - a.nq;
                        const bool is_v = idx >= a.kvw;
                        const int hd = is_v ? idx - a.kvw : idx;
                        char* dst = (is_v ? a.v_pool : a.k_pool) + slot_ofs + (int64_t)(hd / a.head_dim) * a.sh +
                                    (int64_t)(hd % a.head_dim) * 2;
                        *reinterpret_cast<uint2*>(dst) = word;
                    }
                }
            }
        }
        __syncthreads();
    }
}

template <typename T>
struct QkvMfma16;
template <>
struct QkvMfma16<_Float16> {
    __device__ __forceinline__ static f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
};
template <>
struct QkvMfma16<bf16_t> {
    __device__ __forceinline__ static f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    }
};

// The default kernel (in_features a multiple of 32): 16-column tiles on
// v_mfma_f32_16x16x32, so a GPT-2 c_attn weight is streamed by 144 workgroups (the
// 32-column kernel above has 72: too few compute units to read 3.5 MB quickly). A = 8
// elements of weight row n0 + (lane % 16) at k offset 8 (lane / 16), B = the same of
// hidden row m0 + (lane % 16); accumulator register r of lane l is output column
// n0 + 4 (l / 16) + r of row m0 + l % 16. KS waves split `in` (their fp32 partials
// summed through LDS in wave order), blocks of U k-steps double-buffered, MT 16-row
// tiles of the batch per pass.
template <typename T, int MT, int KS, int U>
__global__ __launch_bounds__(KS * 64) void qkv_append16_kernel(const QkvArgs a) {
    __shared__ f32x4 red[KS - 1][MT][64];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int r16 = lane & 15;
    const int kq = lane >> 4;
    const int n0 = (int)blockIdx.x * 16;
    const int ksteps = a.in / 32;
    const int per = (ksteps + KS - 1) / KS;
    const int kb0 = min(ksteps, wave * per);
    const int kb1 = min(ksteps, kb0 + per);
    const T* wp = static_cast<const T*>(a.wt) + (int64_t)min(n0 + r16, a.n - 1) * a.wt_st + 8 * kq;
    const int ncol = n0 + 4 * kq;            // this lane's first output column
    float bias[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
        bias[r] = (a.bias && ncol + r < a.n) ? to_f32(static_cast<const T*>(a.bias)[ncol + r]) : 0.f;

    for (int m0 = 0; m0 < a.rows; m0 += 16 * MT) {
        int64_t slot[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) slot[t] = a.slots[min(m0 + 16 * t + r16, a.rows - 1)];
        const T* xp[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t)
            xp[t] = static_cast<const T*>(a.x) + (int64_t)min(m0 + 16 * t + r16, a.rows - 1) * a.x_st + 8 * kq;
        f32x4 acc[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        u32x4 wa[2][U], xb[2][U][MT];
        auto load = [&](int b, int k0) {
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (k0 + u < kb1) {
                    wa[b][u] = *reinterpret_cast<const u32x4*>(wp + 32 * (k0 + u));
#pragma unroll
                    for (int t = 0; t < MT; ++t) xb[b][u][t] = *reinterpret_cast<const u32x4*>(xp[t] + 32 * (k0 + u));
                }
        };
        auto mma = [&](int b, int k0) {
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (k0 + u < kb1) {
#pragma unroll
                    for (int t = 0; t < MT; ++t) acc[t] = QkvMfma16<T>::run(wa[b][u], xb[b][u][t], acc[t]);
                }
        };
        if (kb0 < kb1) load(0, kb0);
        for (int k0 = kb0; k0 < kb1; k0 += 2 * U) {
            if (k0 + U < kb1) load(1, k0 + U);
            mma(0, k0);
            if (k0 + 2 * U < kb1) load(0, k0 + 2 * U);
            if (k0 + U < kb1) mma(1, k0 + U);
        }
        if (wave > 0) {
#pragma unroll
            for (int t = 0; t < MT; ++t) red[wave - 1][t][lane] = acc[t];
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll 1
            for (int w = 0; w < KS - 1; ++w)
#pragma unroll
                for (int t = 0; t < MT; ++t) acc[t] += red[w][t][lane];
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const int m = m0 + 16 * t + r16;
                if (m >= a.rows || ncol >= a.n) continue;
                const uint2 word = make_uint2(
                    (uint32_t)bits_of<T>(acc[t][0] + bias[0]) | ((uint32_t)bits_of<T>(acc[t][1] + bias[1]) << 16),
                    (uint32_t)bits_of<T>(acc[t][2] + bias[2]) | ((uint32_t)bits_of<T>(acc[t][3] + bias[3]) << 16));
                *reinterpret_cast<uint2*>(static_cast<char*>(a.out) + ((int64_t)m * a.out_st + ncol) * 2) = word;
                if (ncol >= a.nq && (uint64_t)slot[t] < (uint64_t)a.num_slots) {
                    const int idx = ncol - a.nq;
                    const bool is_v = idx >= a.kvw;
                    const int hd = is_v ? idx - a.kvw : idx;
                    char* dst = (is_v ? a.v_pool : a.k_pool) + (slot[t] / a.block_size) * a.sb +
                                (slot[t] % a.block_size) * a.ss + (int64_t)(hd / a.head_dim) * a.sh +
                                (int64_t)(hd % a.head_dim) * 2;
                    *reinterpret_cast<uint2*>(dst) = word;
                }
            }
        }
        __syncthreads();
    }
}

}  // namespace
}  // namespace pkv

using namespace pkv;

extern "C" int pkv_qkv_append(const void* x, int64_t x_stride, const void* weight_t, int64_t weight_stride,
                              const void* bias, int64_t num_rows, int64_t in_features, int64_t q_features,
                              int64_t num_kv_heads, int64_t head_dim, void* out, int64_t out_stride, void* k_pool,
                              void* v_pool, int64_t pool_stride_block, int64_t pool_stride_slot,
                              int64_t pool_stride_head, int64_t num_blocks, int64_t block_size, const int64_t* slots,
                              int dtype, hipStream_t stream) {
    clear_error();
    if (num_rows < 0 || in_features <= 0 || q_features < 0 || num_kv_heads <= 0 || head_dim <= 0 ||
        num_blocks < 0 || block_size <= 0)
        return fail(PKV_EINVAL, "qkv_append: bad sizes");
    if (num_rows == 0) return PKV_OK;
    if (!x || !weight_t || !out || !k_pool || !v_pool || !slots) return fail(PKV_EINVAL, "qkv_append: null pointer");
    if (dtype != PKV_FLOAT16 && dtype != PKV_BFLOAT16)
        return fail(PKV_EUNSUPPORTED, "qkv_append: dtype %d has no kernel (fp16 and bf16 only)", dtype);
    const int64_t kvw = num_kv_heads * head_dim;
    const int64_t n = q_features + 2 * kvw;
    if (in_features % 16 || x_stride % 8 || weight_stride % 8 || x_stride < in_features ||
        weight_stride < in_features || ((uintptr_t)x | (uintptr_t)weight_t) % 16)
        return fail(PKV_EUNSUPPORTED, "qkv_append: needs in_features %% 16 == 0, row strides %% 8 == 0 and "
                                      "16-byte aligned x and weight rows");
    if (q_features % 4 || head_dim % 4 || out_stride % 4 || out_stride < n || (uintptr_t)out % 8 ||
        ((pool_stride_block | pool_stride_slot | pool_stride_head) * 2) % 8 || ((uintptr_t)k_pool | (uintptr_t)v_pool) % 8)
        return fail(PKV_EUNSUPPORTED, "qkv_append: needs 8-byte aligned output and pool rows "
                                      "(q_features, head_dim and strides multiples of 4 elements)");
    if (num_rows > 0x7fffffff || in_features > 0x7fffffff || n > 0x7fffffff)
        return fail(PKV_EUNSUPPORTED, "qkv_append: sizes beyond int32");
    QkvArgs a;
    a.x = x;
    a.wt = weight_t;
    a.bias = bias;
    a.out = out;
    a.k_pool = static_cast<char*>(k_pool);
    a.v_pool = static_cast<char*>(v_pool);
    a.slots = slots;
    a.x_st = x_stride;
    a.wt_st = weight_stride;
    a.out_st = out_stride;
    a.sb = pool_stride_block * 2;
    a.ss = pool_stride_slot * 2;
    a.sh = pool_stride_head * 2;
    a.num_slots = num_blocks * block_size;
    a.block_size = (int)block_size;
    a.rows = (int)num_rows;
    a.in = (int)in_features;
    a.n = (int)n;
    a.nq = (int)q_features;
    a.kvw = (int)kvw;
    a.head_dim = (int)head_dim;
    if (in_features % 32 == 0) {
        // Two waves per 16-column tile; GPT-2 c_attn fp16 per call (HIP-graph replays):
        // 3.5 / 3.7 / 4.0 / 5.0 / 6.7 us at 1 / 8 / 16 / 32 / 64 rows, against 6.5 / 4.6 /
        // 4.6 / 6.5 / 7.6 us for hipBLASLt's addmm alone and 5.9 / 6.2 / 6.4 / 7.0 / 10.9
        // for the 32-column kernel; 4 or 8 waves were 0.1-0.4 us slower, deeper blocks
        // and splitting the batch's row tiles over more workgroups no better.
        constexpr int KS = 2;
        const dim3 grid((unsigned)ceil_div(n, 16));
#define PKV_Q16(MT_, U_)                                                             \
    if (dtype == PKV_FLOAT16)                                                         \
        qkv_append16_kernel<_Float16, MT_, KS, U_><<<grid, KS * 64, 0, stream>>>(a);  \
    else                                                                              \
        qkv_append16_kernel<bf16_t, MT_, KS, U_><<<grid, KS * 64, 0, stream>>>(a);
        if (num_rows <= 16) {
            PKV_Q16(1, 4)
        } else if (num_rows <= 32) {
            PKV_Q16(2, 4)
        } else {
            PKV_Q16(4, 2)
        }
#undef PKV_Q16
        return check_launch("qkv_append");
    }
    const dim3 grid((unsigned)ceil_div(n, 32));
    if (dtype == PKV_FLOAT16)
        qkv_append_kernel<_Float16><<<grid, kKS * 64, 0, stream>>>(a);
    else
        qkv_append_kernel<bf16_t><<<grid, kKS * 64, 0, stream>>>(a);
    return check_launch("qkv_append");
}
