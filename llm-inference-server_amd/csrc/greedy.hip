// Greedy sampling fused into the LM head (gfx950, fp16/bf16): ids[r] is the argmax over
// the vocabulary of hidden[r] · weight[v], without materialising the [rows, vocab] logits.
//
// Replaces `logits[0, ends - 1, :].argmax(-1)` of the paged executor
// (inference_server/core/paged_executor.py:194-203), where `logits` is the model's LM
// head (a bias-free Linear whose weight is [vocab, hidden], GPT-2's tied token
// embedding) applied to the sampled rows. Semantics kept from that expression:
//
//  * each logit is accumulated in fp32 and rounded to the model dtype before the
//    comparison — the LM head's output tensor is fp16/bf16, so two vocabulary entries
//    whose logits round to the same value tie, as they do in the reference;
//  * ties go to the lowest vocabulary index (torch.argmax returns the first maximum);
//  * -0.0 equals +0.0; any NaN ranks above every number (the first NaN wins), as
//    torch's argmax treats NaN as the maximum.
//
// Shape of the work: the weight (77 MB for GPT-2) is read once per 32·NT sampled rows
// and the hidden rows are re-read from L2 by every wave: 2·B flop per weight element,
// below MFMA's ridge, so the bound is the weight stream for a few rows and the hidden
// re-reads as B grows (GPT-2 fp16 on MI355X: 19 us at B = 1, 22.9 us at B = 32 and
// 29.7 us at B = 64 against 34-36 us for the LM-head GEMM + argmax; even at B = 128,
// 42.8 vs 41.3 us; the GEMM wins at 256, 79 vs 61 us). The contraction runs on
// v_mfma_f32_32x32x16_{f16,bf16}:
//
//  * one wave = VT x 32 vocabulary rows (VT MFMA row tiles) x 32·NT sampled rows (NT
//    MFMA column tiles); A = 8 consecutive weight elements of row (lane % 32), B = 8 consecutive
//    hidden elements of sampled row (lane % 32), both one 16-byte load straight from
//    global memory, no LDS. One load instruction takes 32 bytes of each of 32 weight
//    rows, so each 128-byte line is read by four consecutive k steps: the weight loads
//    are plain cached loads (nontemporal ones let the line go between them: 37.7 vs
//    21.7 us for one GPT-2 row). Loads run one block of 8 k steps ahead of the MFMAs.
//  * accumulator register r of lane l holds the logit of vocabulary row
//    8·(r/4) + 4·(l/32) + r%4 of its tile for sampled row l % 32, so each lane ranks
//    16·VT candidates of one sampled row locally and one permlane32 swap merges the two
//    lane halves.
//  * each wave writes one 64-bit key per sampled row into the partials; a second
//    kernel takes the maximum key of each row. A key is the order-preserving integer
//    image of the rounded logit (high word) over the complemented vocabulary index (low
//    word), so the maximum key is the largest logit with the lowest index, and the
//    whole reduction is integer max — deterministic, with no atomics and no
//    initialisation (graph-capture safe).
#include "pkv_common.h"

namespace pkv {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;      // waves per workgroup (independent vocabulary tiles)
constexpr int kVocabTile = 32; // vocabulary rows per wave

template <typename T>
struct LmMfma;
template <>
struct LmMfma<_Float16> {
    __device__ __forceinline__ static f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
    // The logit as the LM head's fp16 output holds it.
    __device__ __forceinline__ static float round(float x) { return (float)(_Float16)x; }
};
template <>
struct LmMfma<bf16_t> {
    __device__ __forceinline__ static f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    }
    __device__ __forceinline__ static float round(float x) { return to_f32(from_f32<bf16_t>(x)); }
};

// Order-preserving key: larger logit -> larger key; equal logits -> lower index larger.
// Every NaN (either sign, any payload) takes the top ordinal, so a NaN outranks every
// number and among NaNs the lowest index wins, as torch.argmax treats NaN.
__device__ __forceinline__ uint64_t rank_key(float x, int v) {
    if (x == 0.0f) x = 0.0f;  // -0.0 ranks as +0.0
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    if (x != x) ord = 0xffffffffu;
    return ((uint64_t)ord << 32) | (uint32_t)(0xffffffffu - (uint32_t)v);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ u32x4 load16v(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// partials[row * num_tasks + task] = best key of wave task `task` (VT consecutive
// 32-row vocabulary tiles) for each sampled row.
template <typename T, int NT, int VT, int U>
__global__ __launch_bounds__(kWaves * 64) void lm_head_argmax_kernel(const T* __restrict__ hidden, int64_t hs,
                                                                     const T* __restrict__ weight, int64_t wsd,
                                                                     int rows, int dim, int vocab, int num_tasks,
                                                                     uint64_t* __restrict__ partials) {
    const int lane = lane_id();
    const int task = (int)blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    if (task >= num_tasks) return;  // whole waves; the kernel has no barrier
    const int col = lane & 31;
    const int half = lane >> 5;
    const int v0 = task * kVocabTile * VT;
    const T* wp[VT];
#pragma unroll
    for (int t = 0; t < VT; ++t)  // rows past the vocabulary re-read the last one, ranked out below
        wp[t] = weight + (int64_t)min(v0 + kVocabTile * t + col, vocab - 1) * wsd + half * 8;

    for (int n0 = 0; n0 < rows; n0 += 32 * NT) {
        const T* hp[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) hp[j] = hidden + (int64_t)min(n0 + 32 * j + col, rows - 1) * hs + half * 8;
        f32x16 acc[VT][NT];
#pragma unroll
        for (int t = 0; t < VT; ++t)
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[t][j] = f32x16{};
        // Two register blocks of U k steps: block i + 1's loads are issued before block
        // i's MFMAs. Each hidden fragment feeds VT MFMAs, each weight fragment NT.
        const int nblk = dim / (16 * U);
        u32x4 a0[VT][U], b0[NT][U], a1[VT][U], b1[NT][U];
        auto load_blk = [&](u32x4(&a)[VT][U], u32x4(&b)[NT][U], int kb) {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int t = 0; t < VT; ++t) a[t][u] = load16v(wp[t] + kb + 16 * u);
#pragma unroll
            for (int j = 0; j < NT; ++j)
#pragma unroll
                for (int u = 0; u < U; ++u) b[j][u] = load16v(hp[j] + kb + 16 * u);
        };
        auto mma_blk = [&](const u32x4(&a)[VT][U], const u32x4(&b)[NT][U]) {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int t = 0; t < VT; ++t)
#pragma unroll
                    for (int j = 0; j < NT; ++j) acc[t][j] = LmMfma<T>::run(a[t][u], b[j][u], acc[t][j]);
        };
        int i = 0;
        if (nblk > 0) load_blk(a0, b0, 0);
        for (; i + 1 < nblk; i += 2) {
            load_blk(a1, b1, (i + 1) * 16 * U);
            mma_blk(a0, b0);
            if (i + 2 < nblk) load_blk(a0, b0, (i + 2) * 16 * U);
            mma_blk(a1, b1);
        }
        if (i < nblk) mma_blk(a0, b0);
        for (int k = nblk * 16 * U; k < dim; k += 16) {
            u32x4 b[NT];
#pragma unroll
            for (int j = 0; j < NT; ++j) b[j] = load16v(hp[j] + k);
#pragma unroll
            for (int t = 0; t < VT; ++t) {
                const u32x4 a = load16v(wp[t] + k);
#pragma unroll
                for (int j = 0; j < NT; ++j) acc[t][j] = LmMfma<T>::run(a, b[j], acc[t][j]);
            }
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            uint64_t best = 0;  // below every real key
#pragma unroll
            for (int t = 0; t < VT; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int v = v0 + kVocabTile * t + 8 * (r >> 2) + 4 * half + (r & 3);
                    if (v < vocab) best = max_u64(best, rank_key(LmMfma<T>::round(acc[t][j][r]), v));
                }
            // Merge with lane ^ 32 (the other four rows of each group of eight).
            const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)best, (uint32_t)best, false, false);
            const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(best >> 32), (uint32_t)(best >> 32), false,
                                                             false);
            const uint64_t k0 = ((uint64_t)(uint32_t)hi[0] << 32) | (uint32_t)lo[0];
            const uint64_t k1 = ((uint64_t)(uint32_t)hi[1] << 32) | (uint32_t)lo[1];
            best = max_u64(k0, k1);
            const int n = n0 + 32 * j + col;
            if (half == 0 && n < rows) partials[(int64_t)n * num_tasks + task] = best;
        }
    }
}

// ids[row] = vocabulary index of the largest key among the row's num_tiles partials
// (one per wave task).
__global__ __launch_bounds__(256) void argmax_merge_kernel(const uint64_t* __restrict__ partials, int num_tiles,
                                                           int64_t* __restrict__ ids) {
    __shared__ uint64_t wave_best[4];
    const uint64_t* p = partials + (int64_t)blockIdx.x * num_tiles;
    uint64_t best = 0;
    for (int t = (int)threadIdx.x; t < num_tiles; t += 256) best = max_u64(best, p[t]);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)best, m, 64);
        const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(best >> 32), m, 64);
        best = max_u64(best, ((uint64_t)hi << 32) | lo);
    }
    if (lane_id() == 0) wave_best[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        best = max_u64(max_u64(wave_best[0], wave_best[1]), max_u64(wave_best[2], wave_best[3]));
        ids[blockIdx.x] = (int64_t)(0xffffffffu - (uint32_t)best);
    }
}

// Wave tasks for `vocab` rows at VT tiles per task; the workspace is sized for VT = 1.
int64_t num_tasks(int64_t vocab, int vt) { return ceil_div(vocab, (int64_t)kVocabTile * vt); }

template <typename T, int NT, int VT, int U>
int launch_kernel(const void* hidden, int64_t hs, const void* weight, int64_t ws, int rows, int dim, int vocab,
                  uint64_t* partials, int& tasks, hipStream_t stream) {
    tasks = (int)num_tasks(vocab, VT);
    lm_head_argmax_kernel<T, NT, VT, U><<<dim3((unsigned)ceil_div(tasks, kWaves)), kWaves * 64, 0, stream>>>(
        static_cast<const T*>(hidden), hs, static_cast<const T*>(weight), ws, rows, dim, vocab, tasks, partials);
    return check_launch("lm_head_argmax");
}

template <typename T>
int launch(const void* hidden, int64_t hs, const void* weight, int64_t ws, int rows, int dim, int vocab,
           uint64_t* partials, int64_t* ids, hipStream_t stream) {
    int tasks = 0, rc;
    // VT = 2: one hidden fragment feeds two vocabulary tiles (GPT-2 fp16, 32 rows: 22.9 us
    // vs 28.3 at VT = 1; VT = 4 leaves too few waves for small batches, 34.9 us).
    if (rows <= 32)
        rc = launch_kernel<T, 1, 2, 8>(hidden, hs, weight, ws, rows, dim, vocab, partials, tasks, stream);
    else if (rows <= 64)
        rc = launch_kernel<T, 2, 2, 4>(hidden, hs, weight, ws, rows, dim, vocab, partials, tasks, stream);
    else
        rc = launch_kernel<T, 4, 2, 4>(hidden, hs, weight, ws, rows, dim, vocab, partials, tasks, stream);
    if (rc) return rc;
    argmax_merge_kernel<<<dim3((unsigned)rows), 256, 0, stream>>>(partials, tasks, ids);
    return check_launch("lm_head_argmax merge");
}

}  // namespace
}  // namespace pkv

using namespace pkv;

extern "C" int64_t pkv_lm_head_argmax_workspace_bytes(int64_t num_rows, int64_t vocab_size) {
    if (num_rows <= 0 || vocab_size <= 0) return 0;
    return ceil_div(num_rows * num_tasks(vocab_size, 1) * (int64_t)sizeof(uint64_t), 256) * 256;
}

extern "C" int pkv_lm_head_argmax(const void* hidden, int64_t hidden_stride, const void* weight,
                                  int64_t weight_stride, int64_t num_rows, int64_t hidden_size, int64_t vocab_size,
                                  int dtype, int64_t* out_ids, void* workspace, int64_t workspace_bytes,
                                  hipStream_t stream) {
    clear_error();
    if (num_rows < 0 || hidden_size <= 0 || vocab_size <= 0) return fail(PKV_EINVAL, "lm_head_argmax: bad sizes");
    if (num_rows == 0) return PKV_OK;
    if (!hidden || !weight || !out_ids || !workspace) return fail(PKV_EINVAL, "lm_head_argmax: null pointer");
    if (dtype != PKV_FLOAT16 && dtype != PKV_BFLOAT16)
        return fail(PKV_EUNSUPPORTED, "lm_head_argmax: dtype %d has no fused kernel (fp16 and bf16 only)", dtype);
    if (hidden_size % 16 || hidden_stride % 8 || weight_stride % 8 || hidden_stride < hidden_size ||
        weight_stride < hidden_size || ((uintptr_t)hidden | (uintptr_t)weight) % 16)
        return fail(PKV_EUNSUPPORTED,
                    "lm_head_argmax: needs hidden_size %% 16 == 0, row strides %% 8 == 0 and 16-byte aligned rows");
    if (num_rows > 0x7fffffff || hidden_size > 0x7fffffff || vocab_size > 0x7fffffff)
        return fail(PKV_EUNSUPPORTED, "lm_head_argmax: sizes beyond int32");
    const int64_t need = pkv_lm_head_argmax_workspace_bytes(num_rows, vocab_size);
    if (workspace_bytes < need)
        return fail(PKV_EWORKSPACE, "lm_head_argmax: workspace %lld bytes, needs %lld", (long long)workspace_bytes,
                    (long long)need);
    uint64_t* partials = static_cast<uint64_t*>(workspace);
    if (dtype == PKV_FLOAT16)
        return launch<_Float16>(hidden, hidden_stride, weight, weight_stride, (int)num_rows, (int)hidden_size,
                                (int)vocab_size, partials, out_ids, stream);
    return launch<bf16_t>(hidden, hidden_stride, weight, weight_stride, (int)num_rows, (int)hidden_size,
                          (int)vocab_size, partials, out_ids, stream);
}
