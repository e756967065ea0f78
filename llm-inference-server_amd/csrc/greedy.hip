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
// Shape of the work: 2·B flop per weight element, far below MFMA's ridge, so the bound
// is the weight stream (77 MB for GPT-2). One launch per call, of one of two kernels,
// each merging its producers' keys of each row inside the launch (below):
//
//  * lm_head_argmax_stream_kernel (hidden size a multiple of 128, the default): one
//    workgroup of 16 waves per compute unit stages up to 64 sampled rows of the hidden
//    states in LDS once (LDS DMA, XOR-swizzled rows); each wave streams one 16-row
//    vocabulary unit of the weight through a register ring on
//    v_mfma_f32_16x16x32_{f16,bf16}, reading the hidden fragments from LDS; each
//    workgroup contributes one key per sampled row. GPT-2 fp16 on MI355X, per call:
//    16.3 us at B = 1, 17.6 at B = 32, 20.0 at B = 64, against ~35 us for the LM-head
//    GEMM + argmax.
//  * lm_head_argmax_kernel (other hidden sizes): one wave = VT x 32 vocabulary rows x
//    32·NT sampled rows on v_mfma_f32_32x32x16, both operands 16-byte loads straight
//    from global memory (the hidden rows re-read from L2 by every wave); one key per
//    wave and sampled row.
//
// A key is the order-preserving integer image of the rounded logit (high word) over the
// complemented vocabulary index (low word), so the maximum key is the largest logit with
// the lowest index, and every reduction is an integer max: the result does not depend on
// the order the producers' keys arrive in. The merge keeps its state (an arrival counter
// and the keys) in the caller's workspace, zero when a call starts and zero again when
// it completes: the workspace is zero-filled once, before its first use, and needs no
// clearing between calls or graph replays.
//
// Tile-kernel details:
//
//  * A = 8 consecutive weight elements of row (lane % 32), B = 8 consecutive hidden
//    elements of sampled row (lane % 32). One load instruction takes 32 bytes of each of
//    32 weight rows, so each 128-byte line is read by four consecutive k steps: the
//    weight loads are plain cached loads (nontemporal ones let the line go between them:
//    37.7 vs 21.7 us for one GPT-2 row). Loads run one block of 8 k steps ahead.
//  * accumulator register r of lane l holds the logit of vocabulary row
//    8·(r/4) + 4·(l/32) + r%4 of its tile for sampled row l % 32, so each lane ranks
//    16·VT candidates of one sampled row locally and one permlane32 swap merges the two
//    lane halves.
#include <algorithm>
#include <atomic>

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

// ---- the merge inside the launch. The workspace holds an arrival counter (offset 0)
// and kKeyCopies copies of one 64-bit key per sampled row (from kKeysOffset, copy c of
// row r at c * rows_pad + r, rows_pad = rows rounded up to 16: whole 128-byte lines),
// all zero when a call starts. Every producer (a workgroup of the streaming kernel, a
// wave of the tile kernel) folds its best key of each row into copy producer % 8 by an
// agent-scope atomic max: one copy took 242 updates of each address per GPT-2 call and
// those serialise (32 rows: 19.0 us per call against 17.6 with 8 copies; 16 or 32
// copies cost more in the final read than they save). The producer then waits until
// its updates are performed (s_waitcnt vmcnt(0): acknowledged by the memory system,
// where agent-scope atomics are performed) and counts itself in; the last of
// `producers` to arrive reads and clears every copy of every row by atomic exchange,
// writes the ids and returns the counter to zero, so each completed call leaves the
// workspace zero for the next. Against a second launch that merged per-producer keys:
// GPT-2 fp16, 1 / 16 / 32 / 64 rows, 16.3 / 16.4 / 17.6 / 20.0 us vs 16.7 / 17.3 / 17.9 /
// 20.2 us per call, one launch instead of two.
constexpr int64_t kKeysOffset = 256;
constexpr int kKeyCopies = 8;

__device__ __forceinline__ int key_rows_pad(int rows) { return (rows + 15) & ~15; }

__device__ __forceinline__ void fold_key(uint64_t* keys, int rows, int producer, int row, uint64_t key) {
    __hip_atomic_fetch_max(keys + (int64_t)(producer % kKeyCopies) * key_rows_pad(rows) + row,
                           (unsigned long long)key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every row's key over all copies, cleared on the way, as the row's vocabulary index.
__device__ __forceinline__ void finish_rows(uint64_t* keys, int rows, int64_t* ids, int first, int step) {
    for (int r = first; r < rows; r += step) {
        uint64_t k = 0;
#pragma unroll
        for (int c = 0; c < kKeyCopies; ++c)
            k = max_u64(k, __hip_atomic_exchange(keys + (int64_t)c * key_rows_pad(rows) + r, 0ull, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT));
        ids[r] = (int64_t)(0xffffffffu - (uint32_t)k);
    }
}

__device__ __forceinline__ u32x4 load16v(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// Wave task `task` (VT consecutive 32-row vocabulary tiles) ranks its candidates of each
// sampled row; the workgroup's 4 waves combine theirs in LDS and fold one key per row
// into the keys (a fold per wave took 28.3 us per call for GPT-2 rows at hidden 1040,
// against 23.3 with the second merge launch: ~1,600 updates of each key); the last
// workgroup to arrive writes the ids.
template <typename T, int NT, int VT, int U>
__global__ __launch_bounds__(kWaves * 64) void lm_head_argmax_kernel(const T* __restrict__ hidden, int64_t hs,
                                                                     const T* __restrict__ weight, int64_t wsd,
                                                                     int rows, int dim, int vocab, int num_tasks,
                                                                     uint64_t* __restrict__ keys,
                                                                     uint32_t* __restrict__ arrivals,
                                                                     int64_t* __restrict__ ids) {
    __shared__ uint64_t s_best[kWaves][32 * NT];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int task_raw = (int)blockIdx.x * kWaves + wave;
    // A wave past the last task computes task num_tasks - 1 again (its keys are a copy,
    // harmless under max) so that every wave reaches the workgroup's barriers.
    const int task = task_raw < num_tasks ? task_raw : num_tasks - 1;
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
            if (half == 0) s_best[wave][32 * j + col] = best;
        }
        __syncthreads();
        if ((int)threadIdx.x < 32 * NT && n0 + (int)threadIdx.x < rows) {
            uint64_t b = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) b = max_u64(b, s_best[w][threadIdx.x]);
            fold_key(keys, rows, (int)blockIdx.x, n0 + (int)threadIdx.x, b);
        }
        __syncthreads();  // s_best is rewritten by the next pass
    }
    // Arrival of this workgroup once its key updates are performed.
    __shared__ uint32_t s_arrived;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        s_arrived = __hip_atomic_fetch_add(arrivals, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_arrived != gridDim.x - 1) return;
    finish_rows(keys, rows, ids, (int)threadIdx.x, kWaves * 64);
    if (threadIdx.x == 0) __hip_atomic_store(arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------
// Weight-streaming kernel (hidden_size % 128 == 0 and the hidden rows of one pass in
// LDS). One workgroup of 16 waves per compute unit stages RT = 16·NT sampled rows of
// the hidden states in LDS once; every wave then streams ONE 16-row vocabulary unit of
// the weight through a register ring of DEPTH 128-element chunks on
// v_mfma_f32_16x16x32_{f16,bf16}, reading each hidden fragment from LDS. So the weight
// is the only HBM stream, the grid is one round (at most 16 units per workgroup, one
// workgroup per CU) and no wave re-reads the hidden rows from L2.
//
//  * A = 8 consecutive weight elements of vocabulary row (lane % 16) at k offset
//    32 s + 8 (lane / 16): each load instruction covers 64 contiguous bytes of 16 rows.
//    B = the same k offsets of sampled row (lane % 16) of column tile j, from LDS.
//  * accumulator register i of lane l holds the logit of vocabulary row
//    4 (l / 16) + i of the unit for sampled row 16 j + l % 16; two xor shuffles
//    (16, 32) merge the four lane groups into one best key per sampled row.
//  * the waves' best keys meet in LDS; lane r of the workgroup folds the best key of
//    sampled row r into the keys (fold_key), and the workgroup counts itself in.
//  * measured and dropped: every chunk of a unit in flight at once (two units per wave,
//    8 waves of 256 registers: 18.4 vs 16.9 us at one row), 32x32x16 tiles (below), and
//    an arrival-counter merge that had the last workgroup read every workgroup's keys
//    (20.5 / 25.9 us at 32 / 64 rows).
constexpr int kChunk = 128;       // k elements per ring chunk of the weight-streaming kernel
constexpr int kGroupsTarget = 256;  // workgroups per launch (one per MI355X compute unit)
constexpr int kLdsBudget = 150 * 1024;  // hidden-row bytes one workgroup may stage (of 160 KiB)

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct LmMfma16;
template <>
struct LmMfma16<_Float16> {
    __device__ __forceinline__ static f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
};
template <>
struct LmMfma16<bf16_t> {
    __device__ __forceinline__ static f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    }
};

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t x, int m) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)x, m, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(x >> 32), m, 64);
    return ((uint64_t)hi << 32) | lo;
}

// The MFMA tile of the weight-streaming kernel: a unit is M = 16 vocabulary rows (the
// A operand, from registers), a column tile M sampled rows (the B operand, from LDS);
// each MFMA contracts KSTEP = 32 elements, lane l supplying 8 of them at offset
// 8 (l / 16). (A 32x32x16 variant with 32-row units, 8 waves of 256 registers, halved
// the LDS bytes per weight byte beyond 16 rows but ran slower: GPT-2, 32 rows 24.1 vs
// 20.3 us, both with the merge then inside the launch.)
template <int M>
struct StreamTile;
template <>
struct StreamTile<16> {  // v_mfma_f32_16x16x32: 16 waves per workgroup (128 registers)
    static constexpr int KSTEP = 32, WAVES = 16, NACC = 4;
    typedef f32x4 acc_t;
    template <typename T>
    __device__ __forceinline__ static acc_t mma(u32x4 a, u32x4 b, acc_t c) { return LmMfma16<T>::run(a, b, c); }
    // Vocabulary row (within the unit) of accumulator register r of lane l.
    __device__ __forceinline__ static int row_of(int r, int l) { return 4 * (l >> 4) + r; }
};

template <typename T, int M, int NT, int DEPTH>
__global__ __launch_bounds__(StreamTile<M>::WAVES * 64) void lm_head_argmax_stream_kernel(
    const T* __restrict__ hidden, int64_t hs, const T* __restrict__ weight, int64_t wsd, int rows, int dim,
    int vocab, int units, int units_per_group, int num_groups, uint64_t* __restrict__ keys,
    uint32_t* __restrict__ arrivals, int64_t* __restrict__ ids) {
    using Tile = StreamTile<M>;
    constexpr int WAVES = Tile::WAVES;
    constexpr int KSTEP = Tile::KSTEP;
    constexpr int KC = kChunk / KSTEP;  // k steps per 128-element chunk
    constexpr int RT = M * NT;          // sampled rows per pass
    constexpr int CPS = KSTEP / 8;      // 16-byte chunks of a row per k step
    constexpr int SPB = 16 / CPS;       // k steps per 16-chunk swizzle block
    extern __shared__ __attribute__((aligned(16))) uint16_t s_hidden[];
    __shared__ uint64_t s_best[WAVES][RT];

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int group = (int)blockIdx.x;
    const int nchunks = dim / kChunk;
    const int u_first = group * units_per_group;
    const int u = u_first + wave;  // this wave's unit
    const bool has_unit = u < min(units, u_first + units_per_group);
    const int h = lane / M;        // which 8 elements of a k step this lane supplies

    const int cpr = dim / 8;             // 16-byte chunks per hidden row
    const int n_dma = RT * cpr / 64;     // DMA instructions per pass (1 KiB each)
    // Vocabulary rows past the end re-read the last one; their keys are ranked out below.
    const T* wrow = weight + (int64_t)min(u * M + lane % M, vocab - 1) * wsd + 8 * h;
    for (int r0 = 0; r0 < rows; r0 += RT) {
        // Stage sampled rows r0 .. r0 + RT by LDS DMA (rows past the end repeat the last
        // one; their keys are never stored). Instruction i fills LDS bytes [1 KiB i, +1 KiB):
        // physical chunk P = 64 i + lane = row r, slot p, which holds logical chunk
        // p ^ (r % 16) of the row (an XOR swizzle in place of padding: the 16 rows a
        // B-fragment read pass touches land on 16 different bank groups).
        for (int i = wave; i < n_dma; i += WAVES) {
            const int P = 64 * i + lane;
            const int r = P / cpr, p = P - r * cpr;
            const char* src = reinterpret_cast<const char*>(hidden + (int64_t)min(r0 + r, rows - 1) * hs) +
                              16 * (p ^ (r & 15));
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(s_hidden + 512 * i), 16, 0,
                                             0);
        }
        asm volatile("" ::: "memory");  // the weight loads below are issued after the DMAs
        // Then the first DEPTH chunks of this wave's unit, before anything waits.
        u32x4 a[DEPTH][KC];
        if (has_unit) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d)
#pragma unroll
                for (int k = 0; k < KC; ++k) a[d][k] = load16v(wrow + KSTEP * (d * KC + k));
            // The DMAs are older than the weight loads: wait for them only.
            __builtin_amdgcn_s_waitcnt(kWaitVm<DEPTH * KC>);
        } else {
            __builtin_amdgcn_s_waitcnt(kWaitVm<0>);
        }
        // Every wave's DMAs have landed once all have passed this barrier. A fenced
        // barrier would make the compiler wait for the weight loads as well (it cannot
        // tell them from the DMAs), so: a plain s_barrier that memory operations are
        // not moved across.
        asm volatile("s_barrier" ::: "memory");

        uint64_t best[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j) best[j] = 0;
        if (has_unit) {
            // Lane (c = lane % 16, h) reads row M j + lane % M, logical chunk CPS s + h, at
            // physical chunk 16 (s / SPB) + ((CPS (s % SPB) + h) ^ c): SPB per-lane offsets,
            // the rest immediates. They do not depend on the pass; without the asm the
            // compiler hoists every fragment read out of the pass loop (and spills them).
            const int c16 = lane & 15;
            int hoff[SPB];
#pragma unroll
            for (int t = 0; t < SPB; ++t) {
                hoff[t] = (lane % M) * dim + 8 * ((CPS * t + h) ^ c16);
                asm volatile("" : "+v"(hoff[t]));
            }
            typename Tile::acc_t acc[NT];
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[j] = typename Tile::acc_t{};
            auto read_b = [&](u32x4(&b)[NT], int s) {
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    b[j] = *reinterpret_cast<const u32x4*>(s_hidden + hoff[s % SPB] + M * j * dim + 128 * (s / SPB));
            };
            // Chunk c: KC k steps, the hidden fragments of step s + 1 read before the
            // MFMAs of step s so the LDS latency overlaps them.
            auto mma_chunk = [&](const u32x4(&ac)[KC], int c) {
                u32x4 b[2][NT];
                read_b(b[0], c * KC);
#pragma unroll
                for (int k = 0; k < KC; ++k) {
                    if (k + 1 < KC) read_b(b[(k + 1) & 1], c * KC + k + 1);
#pragma unroll
                    for (int j = 0; j < NT; ++j) acc[j] = Tile::template mma<T>(ac[k], b[k & 1][j], acc[j]);
                }
            };
            // Chunk c lives in ring slot c % DEPTH. Groups of DEPTH chunks: every group but
            // the last refills each slot with the next group's chunk as soon as it has
            // been used, so the loop body issues its loads in the same slot order as the
            // prologue and the compiler's load counting stays exact (chunk c waits only
            // for its own loads, never for younger ones).
            const int ngroups = nchunks / DEPTH;
            for (int g = 0; g + 1 < ngroups; ++g) {
#pragma unroll
                for (int d = 0; d < DEPTH; ++d) {
                    mma_chunk(a[d], g * DEPTH + d);
#pragma unroll
                    for (int k = 0; k < KC; ++k) a[d][k] = load16v(wrow + KSTEP * (((g + 1) * DEPTH + d) * KC + k));
                    // Keep the refill here: left to itself the scheduler sinks every refill
                    // of the group below its last MFMA, draining the ring once per group.
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) mma_chunk(a[d], (ngroups - 1) * DEPTH + d);
#pragma unroll
            for (int j = 0; j < NT; ++j)
#pragma unroll
                for (int r = 0; r < Tile::NACC; ++r) {
                    const int v = u * M + Tile::row_of(r, lane);
                    if (v < vocab) best[j] = max_u64(best[j], rank_key(LmMfma<T>::round(acc[j][r]), v));
                }
        }
        // Lanes l, l ^ 16, l ^ 32 and l ^ 48 hold the same sampled row.
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            uint64_t b = best[j];
            b = max_u64(b, shfl_xor_u64(b, 16));
            b = max_u64(b, shfl_xor_u64(b, 32));
            if (lane < M) s_best[wave][M * j + lane] = b;
        }
        lds_barrier();
        if ((int)threadIdx.x < RT && r0 + (int)threadIdx.x < rows) {
            uint64_t b = 0;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) b = max_u64(b, s_best[w][threadIdx.x]);
            fold_key(keys, rows, group, r0 + (int)threadIdx.x, b);
        }
        lds_barrier();  // s_hidden and s_best are rewritten by the next pass
    }
    // Arrival of this workgroup once its key updates are performed.
    __shared__ uint32_t s_arrived;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        s_arrived = __hip_atomic_fetch_add(arrivals, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_arrived != (uint32_t)(num_groups - 1)) return;
    finish_rows(keys, rows, ids, (int)threadIdx.x, WAVES * 64);
    if (threadIdx.x == 0) __hip_atomic_store(arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wave tasks for `vocab` rows at VT tiles per task; the workspace is sized for VT = 1.
int64_t num_tasks(int64_t vocab, int vt) { return ceil_div(vocab, (int64_t)kVocabTile * vt); }

template <typename T, int NT, int VT, int U>
int launch_kernel(const void* hidden, int64_t hs, const void* weight, int64_t ws, int rows, int dim, int vocab,
                  uint64_t* keys, uint32_t* arrivals, int64_t* ids, hipStream_t stream) {
    const int tasks = (int)num_tasks(vocab, VT);
    lm_head_argmax_kernel<T, NT, VT, U><<<dim3((unsigned)ceil_div(tasks, kWaves)), kWaves * 64, 0, stream>>>(
        static_cast<const T*>(hidden), hs, static_cast<const T*>(weight), ws, rows, dim, vocab, tasks, keys,
        arrivals, ids);
    return check_launch("lm_head_argmax");
}

// Launch shape of the weight-streaming kernel, or NT = 0 when it does not apply.
struct StreamShape {
    int m = 0, nt = 0, depth = 0, waves = 0, units = 0, units_per_group = 0, groups = 0;
    size_t lds = 0;
};

StreamShape stream_shape(int64_t rows, int64_t dim, int64_t vocab) {
    StreamShape s;
    if (dim % kChunk || rows <= 0 || vocab <= 0) return s;
    // Column tiles per pass: the fewest 16-row tiles that hold the rows, at most 4 (passes
    // of 64 rows beyond that), and no more than the LDS budget allows. Each pass streams
    // the whole weight again; the host layer sends batches that need more than one pass
    // to the GEMM + argmax instead (Llama-sized [32000, 4096] fp16 head: 47.6 us fused vs
    // 55.3 us at 16 rows, one pass; 86.7 vs 54.0 us at 32 rows, two passes; the tile kernel
    // below is no better there: 92 us).
    s.m = 16;
    int nt = rows <= 16 ? 1 : rows <= 32 ? 2 : 4;
    while (nt > 0 && (int64_t)s.m * nt * dim * 2 > kLdsBudget) nt /= 2;
    if (nt == 0) return s;
    // Ring depth in 128-element chunks: the chunk count must be a multiple of it.
    const int64_t nchunks = dim / kChunk;
    s.depth = nchunks % 3 == 0 ? 3 : nchunks % 2 == 0 ? 2 : 0;
    if (s.depth == 0) return s;
    s.nt = nt;
    s.waves = StreamTile<16>::WAVES;
    s.units = (int)ceil_div(vocab, s.m);
    s.units_per_group = (int)std::min<int64_t>(s.waves, ceil_div(s.units, kGroupsTarget));
    s.groups = (int)ceil_div(s.units, s.units_per_group);
    s.lds = (size_t)s.m * nt * dim * 2;
    return s;
}

template <typename T, int M, int NT, int DEPTH>
int launch_stream(const StreamShape& sh, const void* hidden, int64_t hs, const void* weight, int64_t ws, int rows,
                  int dim, int vocab, uint64_t* keys, uint32_t* arrivals, int64_t* ids, hipStream_t stream) {
    // Dynamic LDS beyond 64 KiB needs an opt-in, once per device (a function attribute
    // belongs to the device's context). Setting it is idempotent, so two threads making
    // the first call on a device at once may both set it.
    static std::atomic<uint64_t> attr_set{0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(PKV_EHIP, "lm_head_argmax: hipGetDevice failed");
    const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t)1 << dev : 0;
    if (!bit || !(attr_set.load(std::memory_order_relaxed) & bit)) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&lm_head_argmax_stream_kernel<T, M, NT, DEPTH>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBudget) != hipSuccess)
            return fail(PKV_EHIP, "lm_head_argmax: cannot raise the dynamic LDS limit");
        attr_set.fetch_or(bit, std::memory_order_relaxed);
    }
    lm_head_argmax_stream_kernel<T, M, NT, DEPTH>
        <<<dim3((unsigned)sh.groups), StreamTile<M>::WAVES * 64, sh.lds, stream>>>(
            static_cast<const T*>(hidden), hs, static_cast<const T*>(weight), ws, rows, dim, vocab, sh.units,
            sh.units_per_group, sh.groups, keys, arrivals, ids);
    return check_launch("lm_head_argmax");
}

template <typename T>
int launch(const void* hidden, int64_t hs, const void* weight, int64_t ws, int rows, int dim, int vocab,
           char* workspace, int64_t* ids, hipStream_t stream) {
    uint32_t* arrivals = reinterpret_cast<uint32_t*>(workspace);
    uint64_t* keys = reinterpret_cast<uint64_t*>(workspace + kKeysOffset);
    int rc = PKV_EUNSUPPORTED;
    const StreamShape sh = stream_shape(rows, dim, vocab);
    if (sh.nt) {
#define PKV_STREAM(M_, NT_, D_)                      \
    if (rc == PKV_EUNSUPPORTED && sh.m == M_ && sh.nt == NT_ && sh.depth == D_) \
        rc = launch_stream<T, M_, NT_, D_>(sh, hidden, hs, weight, ws, rows, dim, vocab, keys, arrivals, ids, stream);
        PKV_STREAM(16, 1, 3) PKV_STREAM(16, 2, 3) PKV_STREAM(16, 4, 3)
        PKV_STREAM(16, 1, 2) PKV_STREAM(16, 2, 2) PKV_STREAM(16, 4, 2)
#undef PKV_STREAM
        if (rc == PKV_EUNSUPPORTED)
            return fail(PKV_EUNSUPPORTED, "lm_head_argmax: no streaming kernel for %d x %d-row tiles at depth %d",
                        sh.nt, sh.m, sh.depth);
        return rc;
    }
    if (rows <= 32) {
        // VT = 2: one hidden fragment feeds two vocabulary tiles (GPT-2 fp16, 32 rows: 22.9 us
        // vs 28.3 at VT = 1; VT = 4 leaves too few waves for small batches, 34.9 us).
        return launch_kernel<T, 1, 2, 8>(hidden, hs, weight, ws, rows, dim, vocab, keys, arrivals, ids, stream);
    }
    if (rows <= 64)
        return launch_kernel<T, 2, 2, 4>(hidden, hs, weight, ws, rows, dim, vocab, keys, arrivals, ids, stream);
    return launch_kernel<T, 4, 2, 4>(hidden, hs, weight, ws, rows, dim, vocab, keys, arrivals, ids, stream);
}

}  // namespace
}  // namespace pkv

using namespace pkv;

extern "C" int64_t pkv_lm_head_argmax_workspace_bytes(int64_t num_rows, int64_t vocab_size) {
    if (num_rows <= 0 || vocab_size <= 0) return 0;
    // The arrival counter's 256 bytes, then kKeyCopies keys per row (rows rounded up to 16).
    return kKeysOffset + ceil_div((int64_t)kKeyCopies * ((num_rows + 15) & ~(int64_t)15) * 8, 256) * 256;
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
    char* ws = static_cast<char*>(workspace);
    if (dtype == PKV_FLOAT16)
        return launch<_Float16>(hidden, hidden_stride, weight, weight_stride, (int)num_rows, (int)hidden_size,
                                (int)vocab_size, ws, out_ids, stream);
    return launch<bf16_t>(hidden, hidden_stride, weight, weight_stride, (int)num_rows, (int)hidden_size,
                          (int)vocab_size, ws, out_ids, stream);
}
