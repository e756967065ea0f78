// Persistent paged decode attention on MFMA (gfx950), fp16/bf16, block size 16,
// head_dim 64/128, GQA group 1/2/4/8, for batches large enough to fill the GPU.
//
// Decode reads every K/V byte of the context once; the work per byte is small, so the
// kernel is organised to keep HBM busy and to spend as few instructions per byte as
// possible (the VALU form of this contraction needs ~220 VALU instructions per 4 KiB
// of K/V, enough to make the SIMDs, not HBM, the limit when the core clock drops):
//
//  * Work decomposition (stream-K over the flattened batch). The batch's work is a
//    list of units = (sequence, KV-head group, 16-key block), sequence-major, one
//    group = the NW KV heads a workgroup's NW waves serve (wave w = KV head
//    group * NW + w). A persistent grid of P workgroups (every CU's share, sized by
//    occupancy) takes equal contiguous runs of ceil(units / P) units. Each wave walks
//    its run as a chain of 16-key blocks across sequence boundaries, so the grid is
//    balanced whatever the context lengths are, no workgroup starts or ends mid-launch,
//    and the 32 KiB of one pool block (all KV heads of 16 slots) is fetched by one CU
//    in one window. A sequence lying inside one run is finished in place; one cut by a
//    run boundary leaves a partial (max, denominator, unnormalised output) per cut
//    piece, which a small second kernel on the same stream merges (log-sum-exp rule,
//    pieces in run order). The decode kernel itself never waits on its stores: an
//    in-kernel merge (store, wait, count the arrival with an atomic) stalled each wave's
//    ring for two memory round trips per piece and cost 9% of config 4's time.
//  * Streaming: per wave a two-slot ring of whole blocks in LDS (K and V, 16 rows of
//    one KV head), filled by DMA (global_load_lds_dwordx4). A block's K and V
//    fragments are read from its slot into registers first and the slot is refilled
//    with block n + 2 at once, so two blocks are in flight while block n is computed.
//    All ring waits are explicit s_waitcnt vmcnt counts; the loop issues no other
//    vector-memory instruction, so the counts are exact.
//  * Contraction on the matrix cores, the formulation of the prefill kernel:
//    S^T = K · Q^T (v_mfma_f32_16x16x32: A = 16 K rows from LDS, B = Q^T in registers,
//    heads padded to 16 columns with zeros), so lane (g, n) ends with the scores of
//    keys 4g .. 4g+3 for head n; P^T goes straight from those registers into the
//    B operand of O^T += V^T · P^T (v_mfma_f32_16x16x16, A = V^T through gfx950's
//    transposing LDS read, four keys of one head_dim column per lane). Softmax
//    reductions over a block are lane-local plus two permlane swaps.
//  * Numerics follow the reference gather path (core/attention.py:130-153) as the
//    other decode kernels do: each score is the fp32 dot product rounded to the pool
//    dtype, times scale and rounded again; softmax in fp32; probabilities rounded to
//    the pool dtype before P·V (as exp2(s - m) against a running max m that is raised
//    lazily, only when a block exceeds it by more than 2^8); P·V accumulates in fp32
//    and the output is rounded once.
#include "attention.h"

#include <mutex>

namespace pkv {
namespace {

constexpr int kBS = 16;
constexpr int kMaxSeqs = kDecodeMfmaMaxSeqs;  // prefix table in LDS
constexpr float kLazyMax = 8.f;               // raise the running max past 2^8 only
// Cache policy of the K/V DMAs: nontemporal. The rows are read exactly once per call;
// a DMA-only stream of this access pattern (config 4's blocks, 8 waves per CU, two
// blocks in flight per wave) runs at 7.05 TB/s with it and 6.28 TB/s without.
constexpr int kNontemporal = 2;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// The two MFMA shapes (lane layouts pinned on the MI355X with an in-bounds probe):
//  16x16x32: A[i][k] at lane i + 16 (k / 8), element k % 8; B[k][j] at lane
//            j + 16 (k / 8), element k % 8; D[i][j] at lane j + 16 (i / 4), reg i % 4.
//  16x16x16: the same with 4 elements per lane (k / 4, k % 4).
template <typename T>
struct DMfma;
template <>
struct DMfma<bf16_t> {
    __device__ __forceinline__ static f32x4 qk(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    }
    __device__ __forceinline__ static f32x4 pv(uint2 a, uint2 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4, a), __builtin_bit_cast(bf16x4, b),
                                                         c, 0, 0, 0);
    }
    __device__ __forceinline__ static uint32_t pack(float lo, float hi) {
        bf16x2_t v = {(__bf16)lo, (__bf16)hi};
        return __builtin_bit_cast(uint32_t, v);
    }
    // x rounded to the pool dtype and back (round to nearest even).
    __device__ __forceinline__ static float round(float x) { return (float)(__bf16)x; }
};
template <>
struct DMfma<_Float16> {
    __device__ __forceinline__ static f32x4 qk(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
    __device__ __forceinline__ static f32x4 pv(uint2 a, uint2 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c,
                                                     0, 0, 0);
    }
    __device__ __forceinline__ static uint32_t pack(float lo, float hi) {
        half2_t v = {(_Float16)lo, (_Float16)hi};
        return __builtin_bit_cast(uint32_t, v);
    }
    __device__ __forceinline__ static float round(float x) { return (float)(_Float16)x; }
};

// Transposing LDS read (gfx950 ds_read_b64_tr_b16, issued in RingRead below): within
// each group of 16 lanes the 16 addresses name 4 consecutive 16-bit elements each; lane
// i of the group receives elements i, i + 16, i + 32, i + 48 of those 64 taken in
// (lane, element) order. With source lane c pointing at V[key0 + c / 4][d0 + 4 (c % 4)],
// lane i receives V[key0 .. key0 + 3][d0 + i].

// Physical 16-byte slot of logical chunk c of ring row r: c ^ swz(r). Over any 16
// consecutive rows the swizzle is a permutation, so the b128 K reads (one logical chunk
// of 16 rows per 16 lanes) are free of bank conflicts (D = 64 rows are 128 bytes: the
// row parity picks the bank half and the swizzle spreads each parity over 8 slots).
template <int D>
__device__ __forceinline__ int ring_swizzle(int r) {
    if constexpr (D == 128) return ((r & 3) << 2) | ((r >> 2) & 3);
    else return (((r >> 1) & 1) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1);
}

// 32-bit LDS address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* ptr) {
    return (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) char*)ptr);
}

// A block's MFMA operands from its ring slot, and the wait for them, in one asm
// statement: KSTEPS b128 K reads and VTILES transposing V reads, then lgkmcnt(0). The
// compiler's own wait insertion cannot tell these reads from the DMAs still filling the
// other slot and would drain every outstanding DMA (vmcnt(0)) before them; the explicit
// vmcnt wait that precedes them is exact, so they are issued where the compiler does
// not see them. The results are defined only once the asm (with its wait) completes.
template <int D>
struct RingRead;
template <>
struct RingRead<128> {
    __device__ __forceinline__ static void run(const uint32_t (&ka)[4], const uint32_t (&va)[8], u32x4 (&kf)[4],
                                               uint2 (&vf)[8]) {
        asm volatile(
            "ds_read_b128 %0, %12\n\t"
            "ds_read_b128 %1, %13\n\t"
            "ds_read_b128 %2, %14\n\t"
            "ds_read_b128 %3, %15\n\t"
            "ds_read_b64_tr_b16 %4, %16\n\t"
            "ds_read_b64_tr_b16 %5, %17\n\t"
            "ds_read_b64_tr_b16 %6, %18\n\t"
            "ds_read_b64_tr_b16 %7, %19\n\t"
            "ds_read_b64_tr_b16 %8, %20\n\t"
            "ds_read_b64_tr_b16 %9, %21\n\t"
            "ds_read_b64_tr_b16 %10, %22\n\t"
            "ds_read_b64_tr_b16 %11, %23\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(kf[0]), "=&v"(kf[1]), "=&v"(kf[2]), "=&v"(kf[3]), "=&v"(vf[0]), "=&v"(vf[1]), "=&v"(vf[2]),
              "=&v"(vf[3]), "=&v"(vf[4]), "=&v"(vf[5]), "=&v"(vf[6]), "=&v"(vf[7])
            : "v"(ka[0]), "v"(ka[1]), "v"(ka[2]), "v"(ka[3]), "v"(va[0]), "v"(va[1]), "v"(va[2]), "v"(va[3]),
              "v"(va[4]), "v"(va[5]), "v"(va[6]), "v"(va[7])
            : "memory");
    }
};
template <>
struct RingRead<64> {
    __device__ __forceinline__ static void run(const uint32_t (&ka)[2], const uint32_t (&va)[4], u32x4 (&kf)[2],
                                               uint2 (&vf)[4]) {
        asm volatile(
            "ds_read_b128 %0, %6\n\t"
            "ds_read_b128 %1, %7\n\t"
            "ds_read_b64_tr_b16 %2, %8\n\t"
            "ds_read_b64_tr_b16 %3, %9\n\t"
            "ds_read_b64_tr_b16 %4, %10\n\t"
            "ds_read_b64_tr_b16 %5, %11\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(kf[0]), "=&v"(kf[1]), "=&v"(vf[0]), "=&v"(vf[1]), "=&v"(vf[2]), "=&v"(vf[3])
            : "v"(ka[0]), "v"(ka[1]), "v"(va[0]), "v"(va[1]), "v"(va[2]), "v"(va[3])
            : "memory");
    }
};

// One 16-byte LDS read and its wait, hidden from the compiler's wait insertion for the
// same reason (the query rows staged by DMA).
__device__ __forceinline__ u32x4 lds_read16_waited(uint32_t addr) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(addr) : "memory");
    return v;
}

// Read-only data the kernel indexes with wave-uniform offsets, through the constant
// address space so the loads are scalar (SMEM): they are waited for with the LDS
// counter, which every block waits on anyway, and never join the vector-memory queue
// whose counts the ring's waits rely on.
__device__ __forceinline__ int64_t const_load64(const int64_t* base, int64_t idx) {
    return *((const __attribute__((address_space(4))) int64_t*)base + idx);
}

// Context length as every decode kernel clamps it (never past the table row).
__device__ __forceinline__ int clamp_ctx(int64_t c, int64_t width) {
    const int64_t cap = width * kBS;
    c = c < 0 ? 0 : (c > cap ? cap : c);
    return (int)c;
}

// Position in the flattened unit list: sequence s, KV-head group g, block b of the
// sequence's nb blocks; u is the global unit index; last = valid keys of block nb - 1.
struct Cursor {
    int u, s, g, b, nb, last;
};

template <typename T, int D, int G, int NW>
__global__ __launch_bounds__(NW * 64) void paged_decode_mfma_kernel(const AttnParams p) {
    constexpr int ROWB = D * 2;               // bytes per (token, head) row
    constexpr int CPR = ROWB / 16;            // 16-byte chunks per row
    constexpr int RPI = 1024 / ROWB;          // rows per DMA instruction (64 lanes x 16 B)
    constexpr int IPB = kBS / RPI;            // DMA instructions per block, K or V
    constexpr int KSTEPS = D / 32;            // S^T MFMAs per block
    constexpr int VTILES = D / 16;            // P·V MFMAs per block
    constexpr int NT = NW * 64;
    constexpr int PER = (kMaxSeqs + NT - 1) / NT;
    static_assert(G <= 16 && kBS % RPI == 0, "shape");

    // Ring: slot 0 / slot 1 of every wave, K and V in separate arrays (distinct objects,
    // so the compiler can tell a DMA into one slot from reads of the other).
    __shared__ __attribute__((aligned(1024))) uint16_t s_k0[NW][kBS * D];
    __shared__ __attribute__((aligned(1024))) uint16_t s_v0[NW][kBS * D];
    __shared__ __attribute__((aligned(1024))) uint16_t s_k1[NW][kBS * D];
    __shared__ __attribute__((aligned(1024))) uint16_t s_v1[NW][kBS * D];
    // Query rows of the segment a wave starts next (G rows of head_dim, unswizzled).
    __shared__ __attribute__((aligned(1024))) uint16_t s_q[NW][G * D];
    __shared__ int s_pfx[kMaxSeqs + 1];       // units before sequence s
    __shared__ int s_scan[NT];
    __shared__ int s_prog[NW];                // blocks computed by each wave (priority balance)

    const int tid = (int)threadIdx.x;
    const int B = p.num_seqs;
    const int ngrp = p.num_kv_heads / NW;
    const int64_t width = p.table_width;

    // ---- prefix sums of the units per sequence (one pass over context_lens)
    {
        int units[PER];
        int sum = 0;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int s = tid * PER + i;
            int u = 0;
            if (s < B) u = (clamp_ctx(p.ctx_lens[s], width) + kBS - 1) / kBS * ngrp;
            units[i] = u;
            sum += u;
        }
        s_scan[tid] = sum;
        if (tid < NW) s_prog[tid] = 0;
        lds_barrier();
        for (int off = 1; off < NT; off <<= 1) {
            const int v = tid >= off ? s_scan[tid - off] : 0;
            lds_barrier();
            s_scan[tid] += v;
            lds_barrier();
        }
        int run = s_scan[tid] - sum;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int s = tid * PER + i;
            if (s < B) s_pfx[s] = run;
            run += units[i];
        }
        if (tid == NT - 1) s_pfx[B] = s_scan[NT - 1];
        lds_barrier();
        // The merge kernel reads the same table.
        if (blockIdx.x == 0)
            for (int s = tid; s <= B; s += NT) p.ws_pfx[s] = s_pfx[s];
    }
    const int U = s_pfx[B];
    const int P = (int)gridDim.x;
    const int S = (U + P - 1) / P;
    const int w = (int)blockIdx.x;
    const int u_begin = w * S;
    const int u_end = u_begin + S < U ? u_begin + S : U;
    if (u_begin >= u_end) return;             // no barrier follows

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lg = lane >> 4;                 // MFMA lane group
    const int ln = lane & 15;                 // MFMA row / column index

    // The sequence holding unit u_begin: the last s with pfx[s] <= u_begin.
    Cursor start;
    {
        int lo = 0, hi = B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (s_pfx[mid] <= u_begin) lo = mid;
            else hi = mid - 1;
        }
        start.s = __builtin_amdgcn_readfirstlane(lo);
        const int base = __builtin_amdgcn_readfirstlane(s_pfx[start.s]);
        const int ctx = clamp_ctx(const_load64(p.ctx_lens, start.s), width);
        start.nb = (ctx + kBS - 1) / kBS;
        start.last = ctx - kBS * (start.nb - 1);
        start.u = u_begin;
        start.g = (u_begin - base) / start.nb;
        start.b = (u_begin - base) - start.g * start.nb;
    }
    // Next unit; sequences with no context are skipped.
    auto advance = [&](Cursor& c) {
        ++c.u;
        if (++c.b < c.nb) return;
        c.b = 0;
        if (++c.g < ngrp) return;
        c.g = 0;
        int ctx = 0;
        while (ctx == 0 && c.s + 1 < B) {
            ++c.s;
            ctx = clamp_ctx(const_load64(p.ctx_lens, c.s), width);
        }
        c.nb = (ctx + kBS - 1) / kBS;
        c.last = ctx - kBS * (c.nb - 1);
    };

    const int64_t slot_bytes = p.ss * 2;
    const int64_t block_bytes = p.sb * 2;
    const int64_t head_bytes = p.sh * 2;
    const char* kpool = reinterpret_cast<const char*>(p.k);
    const char* vpool = reinterpret_cast<const char*>(p.v);

    // ---- fused append: rows of the sequences whose last block this run holds, written
    // before any DMA of this wave reads them (only this wave reads that block).
    if (p.app_slots) {
        Cursor c = start;
        while (c.u < u_end) {
            // Jump to the last unit of the current (sequence, group) run.
            const int to_last = c.nb - 1 - c.b;
            if (c.u + to_last < u_end) {
                const int kvh = c.g * NW + wave;
                const int64_t slot = const_load64(p.app_slots, c.s);
                if (slot >= 0 && slot < p.num_blocks * kBS) {
                    const int64_t dst = (slot / kBS) * block_bytes + (slot % kBS) * slot_bytes + kvh * head_bytes;
                    const int64_t src = ((int64_t)c.s * p.app_st + (int64_t)kvh * p.app_sh) * 2;
                    constexpr int WORDS = ROWB / 4;
                    for (int i = lane; i < 2 * WORDS; i += 64) {
                        const bool is_v = i >= WORDS;
                        const int off = 4 * (is_v ? i - WORDS : i);
                        const uint32_t x = *reinterpret_cast<const uint32_t*>(
                            reinterpret_cast<const char*>(is_v ? p.app_v : p.app_k) + src + off);
                        *reinterpret_cast<uint32_t*>(const_cast<char*>(is_v ? vpool : kpool) + dst + off) = x;
                    }
                }
            }
            c.u += to_last;
            c.b = c.nb - 1;
            advance(c);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }

    // ---- DMA of one block (unit cursor c) into a ring slot: 16 rows of K and V of
    // this wave's KV head; rows past the context re-read row 0 (a valid key, masked),
    // an id outside the pool reads block 0 (memory-safe garbage, out of contract).
    const int dma_row = lane / CPR;
    const int dma_slot = lane % CPR;
    uint32_t full_off[IPB];
#pragma unroll
    for (int j = 0; j < IPB; ++j) {
        const int r = j * RPI + dma_row;
        full_off[j] = (uint32_t)(r * slot_bytes) + (uint32_t)((dma_slot ^ ring_swizzle<D>(r)) * 16);
    }
    auto dma_block = [&](const Cursor& c, int64_t id, uint16_t* dk, uint16_t* dv) {
        const int kvh = c.g * NW + wave;
        const int64_t bofs = ((uint64_t)id < (uint64_t)p.num_blocks ? id : 0) * block_bytes + kvh * head_bytes;
        const char* kb = kpool + bofs;
        const char* vb = vpool + bofs;
        const int rows = c.b == c.nb - 1 ? c.last : kBS;
#pragma unroll
        for (int j = 0; j < IPB; ++j) {
            const int r = j * RPI + dma_row;
            const uint32_t off = rows == kBS || r < rows
                                     ? full_off[j]
                                     : (uint32_t)((dma_slot ^ ring_swizzle<D>(r)) * 16);
            const char* ks = kb + off;
            const char* vs = vb + off;
            __builtin_amdgcn_global_load_lds(ks, (__attribute__((address_space(3))) void*)((char*)dk + j * 1024), 16,
                                             0, kNontemporal);
            __builtin_amdgcn_global_load_lds(vs, (__attribute__((address_space(3))) void*)((char*)dv + j * 1024), 16,
                                             0, kNontemporal);
        }
    };
    auto block_id = [&](const Cursor& c) -> int64_t {
        return const_load64(p.tables, (int64_t)c.s * p.table_stride + c.b);
    };

    // ---- per-lane operand addresses inside a ring slot (bytes from the slot's start)
    // K (S^T A operand): row ln, logical chunk 4 j + lg.
    uint32_t k_addr[KSTEPS];
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) k_addr[j] = (uint32_t)(ln * ROWB + (((4 * j + lg) ^ ring_swizzle<D>(ln)) << 4));
    // V^T (P·V A operand, transposing read): source lane c = ln of group lg points at
    // row 4 lg + c / 4, columns 16 t + 4 (c % 4): logical chunk 2 t + (c % 4) / 2,
    // 8-byte half (c % 2).
    const int v_row = 4 * lg + (ln >> 2);
    const int v_swz = ring_swizzle<D>(v_row);
    uint32_t v_addr[VTILES];
#pragma unroll
    for (int t = 0; t < VTILES; ++t)
        v_addr[t] = (uint32_t)(v_row * ROWB + (((2 * t + ((ln & 3) >> 1)) ^ v_swz) << 4) + 8 * (ln & 1));

    // ---- compute state of the current segment
    u32x4 qf[KSTEPS];
    f32x4 o[VTILES];
    float m_run = kNegInf, l_part = 0.f;
    int seg_b0 = 0;                           // first block of the segment in this run
    bool seg_first = true;                    // the run's first segment
    const float scale = p.scale;

    // Query rows of (sequence, KV head) by DMA into this wave's s_q: lane i copies
    // 16-byte chunk i % CPR of head i / CPR of the group (QI instructions).
    constexpr int QI = (G * CPR + 63) / 64;
    auto dma_q = [&](const Cursor& c) {
        const int kvh = c.g * NW + wave;
#pragma unroll
        for (int j = 0; j < QI; ++j) {
            const int i = j * 64 + lane;
            if (i < G * CPR) {
                const char* src = reinterpret_cast<const char*>(p.q) +
                                  ((int64_t)c.s * p.q_st + (int64_t)(kvh * G + i / CPR) * p.q_sh) * 2 + (i % CPR) * 16;
                __builtin_amdgcn_global_load_lds(
                    src, (__attribute__((address_space(3))) void*)((char*)s_q[wave] + j * 1024), 16, 0, 0);
            }
        }
    };
    // Q^T B operand from s_q: lane (lg, ln) takes head ln, dims 32 j + 8 lg .. +8 (zero
    // for the padding columns ln >= G).
    const uint32_t q_addr = lds_addr(s_q[wave]) + (uint32_t)(ln * ROWB + lg * 16);
    auto read_q = [&]() {
#pragma unroll
        for (int j = 0; j < KSTEPS; ++j) {
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (ln < G) v = lds_read16_waited(q_addr + (uint32_t)(4 * j * 16));
            qf[j] = v;
        }
    };

    // The run's first segment, when a run boundary cut it, is finished mid-run: its
    // partial stays in registers until the run's last block and is stored then. A store
    // issued mid-run would hold up the wave's next ring waits (vector-memory operations
    // retire in issue order, and a store's acknowledgement comes back late while the
    // memory system is saturated with reads): storing the partials as they came measured
    // 5% slower on config 4.
    f32x4 o_first[VTILES];
    float m_first = 0.f, l_first = 0.f;
    bool first_pending = false;
    auto store_partial = [&](int side, const f32x4 (&ov)[VTILES], float m, float l) {
        const int64_t slot = ((int64_t)(w * 2 + side) * NW + wave) * G + ln;
        float* po = p.ws_o + slot * D + 4 * lg;
#pragma unroll
        for (int t = 0; t < VTILES; ++t)
            *reinterpret_cast<float4*>(po + 16 * t) = make_float4(ov[t][0], ov[t][1], ov[t][2], ov[t][3]);
        if (lg == 0) *reinterpret_cast<float2*>(p.ws_ml + slot * 2) = make_float2(m, l);
    };

    // Finish the segment that ends with compute cursor c: the normalised output when the
    // run holds the whole (sequence, group), else this piece's partial for the merge
    // kernel (slot (workgroup, side, wave, head): side 0 for the run's first segment, 1
    // for its last; a run's middle segments are whole sequences). No waits here: stores
    // go out before the step's next DMAs.
    auto finish = [&](const Cursor& c) {
        // Denominator over all 16 keys of each block: the four lane groups' sums.
        float l = l_part;
        {
            SwapPair sp = swap16(l);
            l = sp.a + sp.b;
            sp = swap32(l);
            l = sp.a + sp.b;
        }
        if (ln >= G) return;
        const int kvh = c.g * NW + wave;
        if (seg_b0 == 0 && c.b == c.nb - 1) {
            const float inv = 1.f / l;
            T* orow = reinterpret_cast<T*>(p.out) + (int64_t)c.s * p.out_st + (int64_t)(kvh * G + ln) * p.out_sh;
#pragma unroll
            for (int t = 0; t < VTILES; ++t) {
                const uint32_t w0 = DMfma<T>::pack(o[t][0] * inv, o[t][1] * inv);
                const uint32_t w1 = DMfma<T>::pack(o[t][2] * inv, o[t][3] * inv);
                *reinterpret_cast<uint2*>(orow + 16 * t + 4 * lg) = make_uint2(w0, w1);
            }
            return;
        }
        if (seg_first && c.u != u_end - 1) {
#pragma unroll
            for (int t = 0; t < VTILES; ++t) o_first[t] = o[t];
            m_first = m_run;
            l_first = l;
            first_pending = true;
            return;
        }
        store_partial(seg_first ? 0 : 1, o, m_run, l);
    };

    // ---- one block: wait for its DMA, read its K and V^T fragments, refill the slot with
    // block n + 2, then the contraction and the online softmax from registers.
    constexpr int kBlockDmas = 2 * IPB;
    Cursor cc = start;                        // compute cursor: block n
    Cursor dc = start;                        // DMA cursor: block n + 2 once primed
    int64_t next_id = 0;                      // table entry of dc, loaded a step ahead
    int remaining = u_end - u_begin;          // blocks left to compute
    int to_issue = remaining;                 // blocks left to DMA

    bool seg_start = true;
    // Balance between the two waves of a SIMD. With 8 waves, waves w and w + 4 share a
    // SIMD and walk the same blocks (different KV heads); when both are ready the older
    // one issues first, refills its ring first and stays ahead: on config 4 waves 0-3
    // ended their runs at ~226 us and waves 4-7 at ~317 us, streaming alone (half the
    // bytes in flight per CU) for the last ~90 us. Each wave publishes its block count in
    // LDS and raises its priority while it is behind its SIMD partner: the waves of a
    // workgroup then end within ~4 us of each other (config 4: 344.7 -> 334.0 us per call,
    // output bit-identical). Both LDS accesses are inline asm for the same reason as the
    // ring reads (a compiler-visible LDS read would drain the ring with vmcnt(0)).
    int done = 0;
    const uint32_t prog_me = lds_addr(&s_prog[wave]);
    const uint32_t prog_partner = lds_addr(&s_prog[wave ^ (NW / 2)]);
    auto step = [&](const uint16_t* ck, const uint16_t* cv, uint16_t* nk, uint16_t* nv) {
        // Block n's DMA (and any query DMA issued before block n + 1's) is done when at
        // most block n + 1's DMAs are outstanding: every step that leaves a later step
        // issues exactly those kBlockDmas after them.
        if (remaining > 1) __builtin_amdgcn_s_waitcnt(kWaitVm<kBlockDmas>);
        else __builtin_amdgcn_s_waitcnt(kWaitVm<0>);
        u32x4 kf[KSTEPS];
        uint2 vf[VTILES];
        {
            uint32_t ka[KSTEPS], va[VTILES];
            const uint32_t kb = lds_addr(ck), vb = lds_addr(cv);
#pragma unroll
            for (int j = 0; j < KSTEPS; ++j) ka[j] = kb + k_addr[j];
#pragma unroll
            for (int t = 0; t < VTILES; ++t) va[t] = vb + v_addr[t];
            RingRead<D>::run(ka, va, kf, vf);
        }
        if (seg_start) read_q();
        if constexpr (NW == 8) {
            ++done;
            asm volatile("ds_write_b32 %0, %1" : : "v"(prog_me), "v"(done) : "memory");
            int other;
            asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(other) : "v"(prog_partner) : "memory");
            if (__builtin_amdgcn_readfirstlane(done < other ? 1 : 0)) __builtin_amdgcn_s_setprio(1);
            else __builtin_amdgcn_s_setprio(0);
        }
        // The slot and s_q are free now (the reads above waited for themselves).
        // Segment end: the sequence's last block for this group, or the run's last block.
        const bool seg_end = cc.b == cc.nb - 1 || cc.u == u_end - 1;
        // Next DMAs: the next segment's queries (if block n + 1 starts one), then block
        // n + 2. At a segment end they follow the finish's stores (below), so that the
        // next step's ring wait, which leaves only block n + 2's DMAs outstanding, also
        // retires the stores; elsewhere they go out before the compute.
        auto issue_next = [&]() {
            if (seg_end && remaining > 1) {
                Cursor nx = cc;
                advance(nx);
                dma_q(nx);
            }
            if (to_issue > 0) {
                dma_block(dc, next_id, nk, nv);
                --to_issue;
                advance(dc);
                if (to_issue > 0) next_id = block_id(dc);
            }
        };
        if (!seg_end) issue_next();
        if (seg_start) {
#pragma unroll
            for (int t = 0; t < VTILES; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            m_run = kNegInf;
            l_part = 0.f;
        }

        // S^T for the 16 keys: lane (lg, ln) holds keys 4 lg + r of head ln.
        f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < KSTEPS; ++j) st = DMfma<T>::qk(kf[j], qf[j], st);
        const int valid = cc.b == cc.nb - 1 ? cc.last : kBS;
        float bmax = kNegInf;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float x = DMfma<T>::round(DMfma<T>::round(st[r]) * scale) * kLog2e;
            st[r] = 4 * lg + r < valid ? x : kNegInf;
            bmax = fmaxf(bmax, st[r]);
        }
        {
            SwapPair sp = swap16(bmax);
            bmax = fmaxf(sp.a, sp.b);
            sp = swap32(bmax);
            bmax = fmaxf(sp.a, sp.b);
        }
        const bool raise = bmax > m_run + kLazyMax;
        if (__builtin_amdgcn_ballot_w64(raise)) {
            const float m_new = raise ? bmax : m_run;
            const float alpha = !raise ? 1.f : (m_run == kNegInf ? 0.f : fast_exp2(m_run - m_new));
#pragma unroll
            for (int t = 0; t < VTILES; ++t) o[t] *= alpha;
            l_part *= alpha;
            m_run = m_new;
        }
        const float m_off = m_run == kNegInf ? 0.f : m_run;
        float pr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            pr[r] = fast_exp2(st[r] - m_off);
            l_part += pr[r];
        }
        const uint2 pb = make_uint2(DMfma<T>::pack(pr[0], pr[1]), DMfma<T>::pack(pr[2], pr[3]));
#pragma unroll
        for (int t = 0; t < VTILES; ++t) o[t] = DMfma<T>::pv(vf[t], pb, o[t]);

        if (seg_end) {
            finish(cc);
            seg_first = false;
            issue_next();
        }
        --remaining;
        advance(cc);
        seg_start = seg_end;
        seg_b0 = seg_end ? cc.b : seg_b0;
    };

    // Prime the ring: the first segment's queries, then blocks 0 and 1 of the run.
    dma_q(start);
    next_id = block_id(dc);
    dma_block(dc, next_id, s_k0[wave], s_v0[wave]);
    --to_issue;
    advance(dc);
    if (to_issue > 0) {
        next_id = block_id(dc);
        dma_block(dc, next_id, s_k1[wave], s_v1[wave]);
        --to_issue;
        advance(dc);
        if (to_issue > 0) next_id = block_id(dc);
    }
    seg_b0 = start.b;
    while (remaining > 0) {
        step(s_k0[wave], s_v0[wave], s_k0[wave], s_v0[wave]);
        if (remaining > 0) step(s_k1[wave], s_v1[wave], s_k1[wave], s_v1[wave]);
    }
    if (first_pending) store_partial(0, o_first, m_first, l_first);
}

// Split-KV merge of the pieces a run boundary cut: one workgroup per (sequence, KV-head
// group), launched after the decode kernel on the same stream (stream order is the only
// synchronisation). Pieces are combined in run order with the log-sum-exp rule; a
// (sequence, group) held by one run was finished by the decode kernel and is skipped.
template <int NW, int G, int D>
constexpr int kMergeThreads = NW * G * D / 4 < 1024 ? NW * G * D / 4 : 1024;

template <typename T, int D, int G, int NW>
__global__ __launch_bounds__((kMergeThreads<NW, G, D>)) void paged_decode_mfma_merge_kernel(const AttnParams p,
                                                                                        int grid) {
    const int s = (int)blockIdx.x;
    const int g = (int)blockIdx.y;
    const int U = p.ws_pfx[p.num_seqs];
    const int units = p.ws_pfx[s + 1] - p.ws_pfx[s];
    if (U == 0 || units == 0) return;
    const int S = (U + grid - 1) / grid;
    const int nb = units / (p.num_kv_heads / NW);
    const int u_first = p.ws_pfx[s] + g * nb;
    const int w_first = u_first / S;
    const int pieces = (u_first + nb - 1) / S - w_first + 1;
    if (pieces == 1) return;
    constexpr int EL = NW * G * D;            // (wave, head, dim) elements, 4 per thread
    constexpr int CH = 8;                     // pieces whose loads are in flight together
    for (int e = (int)threadIdx.x * 4; e < EL; e += kMergeThreads<NW, G, D> * 4) {
        const int wave = e / (G * D);
        const int h = (e / D) % G;
        const int d = e % D;
        float M = kNegInf, L = 0.f;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int k0 = 0; k0 < pieces; k0 += CH) {
            float2 ml[CH];
            float4 ov[CH];
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int k = k0 + j;
                ml[j] = make_float2(kNegInf, 0.f);
                ov[j] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (k < pieces) {
                    const int wk = w_first + k;
                    const int64_t slot =
                        ((int64_t)(wk * 2 + (k == 0 && u_first != wk * S ? 1 : 0)) * NW + wave) * G + h;
                    ml[j] = *reinterpret_cast<const float2*>(p.ws_ml + slot * 2);
                    ov[j] = *reinterpret_cast<const float4*>(p.ws_o + slot * D + d);
                }
            }
            float Mc = M;
#pragma unroll
            for (int j = 0; j < CH; ++j) Mc = fmaxf(Mc, ml[j].x);
            const float rs = M == kNegInf ? 0.f : fast_exp2(M - Mc);
            L *= rs;
            acc.x *= rs;
            acc.y *= rs;
            acc.z *= rs;
            acc.w *= rs;
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const float sc = ml[j].x == kNegInf ? 0.f : fast_exp2(ml[j].x - Mc);
                L += sc * ml[j].y;
                acc.x += sc * ov[j].x;
                acc.y += sc * ov[j].y;
                acc.z += sc * ov[j].z;
                acc.w += sc * ov[j].w;
            }
            M = Mc;
        }
        const float inv = 1.f / L;
        T* orow = reinterpret_cast<T*>(p.out) + (int64_t)s * p.out_st + (int64_t)((g * NW + wave) * G + h) * p.out_sh;
        *reinterpret_cast<uint2*>(orow + d) =
            make_uint2(DMfma<T>::pack(acc.x * inv, acc.y * inv), DMfma<T>::pack(acc.z * inv, acc.w * inv));
    }
}

// Workgroups per CU of each instantiation (from the occupancy API, once per device),
// capped at kMaxWgsPerCu.
constexpr int kMaxDevices = 64;
constexpr int kMaxWgsPerCu = 2;
std::mutex g_cu_mu;
int g_cus[kMaxDevices] = {};

int device_cus() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    std::lock_guard<std::mutex> lock(g_cu_mu);
    if (!g_cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
        g_cus[dev] = n;
    }
    return g_cus[dev];
}

template <typename T, int D, int G, int NW>
int occupancy() {
    static std::mutex mu;
    static int per_cu[kMaxDevices] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    std::lock_guard<std::mutex> lock(mu);
    if (!per_cu[dev]) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, paged_decode_mfma_kernel<T, D, G, NW>, NW * 64, 0) !=
                hipSuccess ||
            n <= 0)
            return 0;
        per_cu[dev] = n;
    }
    return per_cu[dev];
}

int waves_per_group(int num_kv_heads) { return num_kv_heads % 8 == 0 ? 8 : (num_kv_heads % 4 == 0 ? 4 : 0); }

template <typename T, int D, int G, int NW>
int launch_nw(const AttnParams& p, hipStream_t stream) {
    const int cus = device_cus();
    int occ = occupancy<T, D, G, NW>();
    if (cus <= 0 || occ <= 0) return PKV_EUNSUPPORTED;
    // At most two workgroups per CU: the workspace's partials are sized for that grid.
    occ = occ < kMaxWgsPerCu ? occ : kMaxWgsPerCu;
    const int64_t grid = (int64_t)cus * occ;
    paged_decode_mfma_kernel<T, D, G, NW><<<dim3((unsigned)grid), NW * 64, 0, stream>>>(p);
    const int rc = check_launch("paged decode attention (mfma)");
    if (rc) return rc;
    paged_decode_mfma_merge_kernel<T, D, G, NW>
        <<<dim3((unsigned)p.num_seqs, (unsigned)(p.num_kv_heads / NW)), kMergeThreads<NW, G, D>, 0, stream>>>(
            p, (int)grid);
    return check_launch("paged decode merge (mfma)");
}

template <typename T, int D, int G>
int launch_g(const AttnParams& p, hipStream_t stream) {
    if (waves_per_group(p.num_kv_heads) == 8) return launch_nw<T, D, G, 8>(p, stream);
    return launch_nw<T, D, G, 4>(p, stream);
}

template <typename T, int D>
int launch_d(const AttnParams& p, hipStream_t stream) {
    switch (p.group) {
        case 1: return launch_g<T, D, 1>(p, stream);
        case 2: return launch_g<T, D, 2>(p, stream);
        case 4: return launch_g<T, D, 4>(p, stream);
        case 8: return launch_g<T, D, 8>(p, stream);
        default: return PKV_EUNSUPPORTED;
    }
}

}  // namespace

// Largest grid any instantiation takes on this device (workgroups), for sizing.
int64_t decode_mfma_max_grid() {
    const int cus = device_cus();
    return cus > 0 ? (int64_t)cus * kMaxWgsPerCu : 0;
}

int64_t decode_mfma_partial_floats(int64_t num_kv_heads, int64_t group, int64_t head_dim) {
    const int nw = waves_per_group((int)num_kv_heads);
    if (!nw) return 0;
    return decode_mfma_max_grid() * 2 * nw * group * (head_dim + 2);
}

bool decode_mfma_sizes_apply(int64_t num_seqs, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                             int64_t max_context_len) {
    if (num_kv_heads <= 0 || num_heads % num_kv_heads) return false;
    const int64_t group = num_heads / num_kv_heads;
    if (head_dim != 64 && head_dim != 128) return false;
    if (group != 1 && group != 2 && group != 4 && group != 8) return false;
    if (!waves_per_group((int)num_kv_heads) || num_seqs > kMaxSeqs || num_seqs < 1) return false;
    // Launches whose K/V (bounded by the longest context) reach 512 MiB. Measured against
    // the partition kernels over 400 back-to-back calls (us, MFMA vs partition): config 4
    // 348 vs 391; 128 x 512-8192 tokens GQA 2 365 vs 414; 64 x 1024-8192 GQA 8 196 vs
    // 362; 128 x 1024-4096 d64 GQA 4 115 vs 143; 32 x 4096 89 vs 100. Smaller launches
    // stay on the partition kernels: 16 x 2048 30.5 vs 31.2 and config 2 (64 x 12 heads x
    // d64, up to 2048 tokens) 23.6 vs 25.0 gain little and config 2 lost it in a
    // 40-call run after a 5-call warm-up (28.6 vs 25 us); GPT-2's decode shape
    // (32 x 100-700 tokens) 14.8 vs 13.5: runs of a few blocks each leave the persistent
    // grid's fixed costs (prefix scan, ring fill, merge launch) uncovered.
    return max_context_len >= 1 && num_seqs * num_kv_heads * max_context_len * head_dim * 4 >= ((int64_t)512 << 20);
}

bool decode_mfma_applies(const AttnParams& p, int dtype, int64_t max_context_len) {
    if (dtype != PKV_FLOAT16 && dtype != PKV_BFLOAT16) return false;
    if (p.block_size != kBS || p.num_blocks < 1) return false;
    if (!decode_mfma_sizes_apply(p.num_seqs, p.num_heads, p.num_kv_heads, p.head_dim, max_context_len)) return false;
    // Unit indices in int32.
    const int64_t ngrp = p.num_kv_heads / waves_per_group(p.num_kv_heads);
    if ((int64_t)p.num_seqs * p.table_width * ngrp >= ((int64_t)1 << 31) - 4096) return false;
    const uint64_t probe = (uint64_t)(uintptr_t)p.q | (uint64_t)(uintptr_t)p.k | (uint64_t)(uintptr_t)p.v |
                           (uint64_t)(uintptr_t)p.out | (uint64_t)(p.q_st * 2) | (uint64_t)(p.q_sh * 2) |
                           (uint64_t)(p.sb * 2) | (uint64_t)(p.ss * 2) | (uint64_t)(p.sh * 2) |
                           (uint64_t)(p.out_st * 2) | (uint64_t)(p.out_sh * 2);
    if (probe % 16) return false;
    // Slot offsets inside a block in 32 bits.
    if (kBS * p.ss * 2 >= ((int64_t)1 << 32)) return false;
    return decode_mfma_max_grid() > 0;
}

int launch_decode_mfma(const AttnParams& p, int dtype, hipStream_t stream) {
    if (!p.ws_pfx || !p.ws_o || !p.ws_ml) return PKV_EUNSUPPORTED;
    if (dtype == PKV_FLOAT16) {
        if (p.head_dim == 64) return launch_d<_Float16, 64>(p, stream);
        return launch_d<_Float16, 128>(p, stream);
    }
    if (p.head_dim == 64) return launch_d<bf16_t, 64>(p, stream);
    return launch_d<bf16_t, 128>(p, stream);
}

}  // namespace pkv
