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
//  * -0.0 equals +0.0; a positive NaN ranks above every number, as torch's argmax
//    treats NaN as the maximum.
//
// Shape of the work: the weight (77 MB for GPT-2) is read once per 32·NT sampled rows
// and the hidden rows are re-read from L2 by every wave: 2·B flop per weight element,
// below MFMA's ridge, so the bound is the weight stream for a few rows and the hidden
// re-reads as B grows (GPT-2 fp16 on MI355X: 20 us at B = 1, 29 us at B = 32 against
// 33-35 us for the LM-head GEMM + argmax; 41 vs 36 us at B = 64, where the separate GEMM
// wins). The contraction runs on v_mfma_f32_32x32x16_{f16,bf16}:
//
//  * one wave = 32 vocabulary rows (the MFMA's M) x 32·NT sampled rows (NT MFMA column
//    tiles); A = 8 consecutive weight elements of row (lane % 32), B = 8 consecutive
//    hidden elements of sampled row (lane % 32), both one 16-byte load straight from
//    global memory, no LDS. One load instruction takes 32 bytes of each of 32 weight
//    rows, so each 128-byte line is read by four consecutive k steps: the weight loads
//    are plain cached loads (nontemporal ones let the line go between them: 37.7 vs
//    21.7 us for one GPT-2 row). Loads run one block of 8 k steps ahead of the MFMAs.
//  * accumulator register r of lane l holds the logit of vocabulary row
//    8·(r/4) + 4·(l/32) + r%4 for sampled row l % 32, so each lane ranks 16 candidates
//    of one sampled row locally and one permlane32 swap merges the two lane halves.
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
constexpr int kUnroll = 8;     // 16-element k steps loaded together

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
__device__ __forceinline__ uint64_t rank_key(float x, int v) {
    if (x == 0.0f) x = 0.0f;  // -0.0 ranks as +0.0
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint32_t)(0xffffffffu - (uint32_t)v);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ u32x4 load16v(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// partials[row * num_tiles + tile] = best key of vocabulary tile `tile` for sampled row.
template <typename T, int NT>
__global__ __launch_bounds__(kWaves * 64) void lm_head_argmax_kernel(const T* __restrict__ hidden, int64_t hs,
                                                                     const T* __restrict__ weight, int64_t wsd,
                                                                     int rows, int dim, int vocab, int num_tiles,
                                                                     uint64_t* __restrict__ partials) {
    const int lane = lane_id();
    const int tile = (int)blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    if (tile >= num_tiles) return;  // whole waves; the kernel has no barrier
    const int col = lane & 31;
    const int half = lane >> 5;
    const int v0 = tile * kVocabTile;
    const int vrow = min(v0 + col, vocab - 1);  // rows past the vocabulary re-read the last one, ranked out below
    const T* wp = weight + (int64_t)vrow * wsd + half * 8;

    for (int n0 = 0; n0 < rows; n0 += 32 * NT) {
        const T* hp[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) hp[j] = hidden + (int64_t)min(n0 + 32 * j + col, rows - 1) * hs + half * 8;
        f32x16 acc[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[j] = f32x16{};
        // Two register blocks: block i + 1's loads are issued before block i's MFMAs.
        const int nblk = dim / (16 * kUnroll);
        u32x4 a0[kUnroll], b0[NT][kUnroll], a1[kUnroll], b1[NT][kUnroll];
        auto load_blk = [&](u32x4(&a)[kUnroll], u32x4(&b)[NT][kUnroll], int kb) {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) a[u] = load16v(wp + kb + 16 * u);
#pragma unroll
            for (int j = 0; j < NT; ++j)
#pragma unroll
                for (int u = 0; u < kUnroll; ++u) b[j][u] = load16v(hp[j] + kb + 16 * u);
        };
        auto mma_blk = [&](const u32x4(&a)[kUnroll], const u32x4(&b)[NT][kUnroll]) {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u)
#pragma unroll
                for (int j = 0; j < NT; ++j) acc[j] = LmMfma<T>::run(a[u], b[j][u], acc[j]);
        };
        int i = 0;
        if (nblk > 0) load_blk(a0, b0, 0);
        for (; i + 1 < nblk; i += 2) {
            load_blk(a1, b1, (i + 1) * 16 * kUnroll);
            mma_blk(a0, b0);
            if (i + 2 < nblk) load_blk(a0, b0, (i + 2) * 16 * kUnroll);
            mma_blk(a1, b1);
        }
        if (i < nblk) mma_blk(a0, b0);
        int k = nblk * 16 * kUnroll;
        for (; k < dim; k += 16) {
            const u32x4 a = load16v(wp + k);
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[j] = LmMfma<T>::run(a, load16v(hp[j] + k), acc[j]);
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            uint64_t best = 0;  // below every real key
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int v = v0 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (v < vocab) best = max_u64(best, rank_key(LmMfma<T>::round(acc[j][r]), v));
            }
            // Merge with lane ^ 32 (the other four rows of each group of eight).
            const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)best, (uint32_t)best, false, false);
            const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(best >> 32), (uint32_t)(best >> 32), false,
                                                             false);
            const uint64_t k0 = ((uint64_t)(uint32_t)hi[0] << 32) | (uint32_t)lo[0];
            const uint64_t k1 = ((uint64_t)(uint32_t)hi[1] << 32) | (uint32_t)lo[1];
            best = max_u64(k0, k1);
            const int n = n0 + 32 * j + col;
            if (half == 0 && n < rows) partials[(int64_t)n * num_tiles + tile] = best;
        }
    }
}

// ids[row] = vocabulary index of the largest key among the row's num_tiles partials.
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

int64_t num_vocab_tiles(int64_t vocab) { return ceil_div(vocab, kVocabTile); }

template <typename T>
int launch(const void* hidden, int64_t hs, const void* weight, int64_t ws, int rows, int dim, int vocab,
           uint64_t* partials, int64_t* ids, hipStream_t stream) {
    const int tiles = (int)num_vocab_tiles(vocab);
    const dim3 grid((unsigned)ceil_div(tiles, kWaves));
    const T* h = static_cast<const T*>(hidden);
    const T* w = static_cast<const T*>(weight);
    if (rows <= 32)
        lm_head_argmax_kernel<T, 1><<<grid, kWaves * 64, 0, stream>>>(h, hs, w, ws, rows, dim, vocab, tiles, partials);
    else if (rows <= 64)
        lm_head_argmax_kernel<T, 2><<<grid, kWaves * 64, 0, stream>>>(h, hs, w, ws, rows, dim, vocab, tiles, partials);
    else
        lm_head_argmax_kernel<T, 4><<<grid, kWaves * 64, 0, stream>>>(h, hs, w, ws, rows, dim, vocab, tiles, partials);
    int rc = check_launch("lm_head_argmax");
    if (rc) return rc;
    argmax_merge_kernel<<<dim3((unsigned)rows), 256, 0, stream>>>(partials, tiles, ids);
    return check_launch("lm_head_argmax merge");
}

}  // namespace
}  // namespace pkv

using namespace pkv;

extern "C" int64_t pkv_lm_head_argmax_workspace_bytes(int64_t num_rows, int64_t vocab_size) {
    if (num_rows <= 0 || vocab_size <= 0) return 0;
    return ceil_div(num_rows * num_vocab_tiles(vocab_size) * (int64_t)sizeof(uint64_t), 256) * 256;
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
