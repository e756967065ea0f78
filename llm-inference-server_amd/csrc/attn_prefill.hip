// Paged prefill / chunked-prefill attention on MFMA (gfx950), fp16/bf16, block
// size 16, head_dim 64/128, GQA group 1/2/4/8. Other shapes take the generic kernel.
//
// Prefill is compute-bound (config 4 chunks: ~926 flop per byte touched), so the
// contraction runs on v_mfma_f32_32x32x16_{bf16,f16}. The formulation is chosen so
// the softmax needs almost no cross-lane traffic:
//
//  * S^T = K · Q^T per 32-key x 32-query tile: A = K rows (from LDS), B = Q^T
//    (registers, loaded once). MFMA result register r of lane l holds
//    S^T[key 8*(r/4) + 4*(l/32) + r%4][query l%32], so every lane owns ONE query's
//    column: row max / row sum are lane-local over 32 values plus one permlane32 swap
//    with the lane holding the other half of the keys.
//  * P^T feeds the P·V MFMA as its B operand straight from the S^T accumulator
//    registers, cast to the pool dtype at the point where the reference casts
//    `probs.to(v.dtype)` — but as the unnormalised weights exp2(s - m) <= 2^8 of fp32
//    scores, divided by the fp32 row sum only at the end, where the reference rounds
//    its fp16 scores and then the normalised probabilities. The key order inside a
//    lane's 8 slots is the accumulator's, and the A operand V^T is read from LDS in that
//    same key order, so no data moves between the two MFMAs.
//  * V^T: the 64-key V tile is staged row-major like K and read through gfx950's
//    transposing LDS load (ds_read_b64_tr_b16): two 8-byte reads per MFMA give each
//    lane its 8 keys of one head_dim column.
//  * Work unit: one workgroup = (sequence, KV head, 32-query tile) x 4 waves. With a
//    GQA group of G >= 4 the waves are 4 query heads of one KV head and share every
//    staged K/V tile (G = 8 uses two workgroups); with G < 4 they are 4/G consecutive
//    query tiles x G heads. K/V tiles are 64 keys (4 blocks) walked through the block
//    table up to the causal bound of the workgroup's last query.
//  * Two waves per SIMD (registers capped at 256 per lane): with one, every MFMA ->
//    softmax -> MFMA dependency and every load wait idles the matrix core; two
//    workgroups per CU interleave (config 4 chunks: 311 -> 486 TFLOP/s).
//  * XCD-aware order: the hardware hands workgroup L to XCD L % 8 and each XCD has its
//    own L2. Work items are numbered query block fastest, then sequence, then KV head,
//    and XCD x takes the x-th contiguous eighth, so the workgroups that re-read one
//    sequence's K/V tiles share an L2 instead of fetching them from HBM once per XCD.
//    Within a sequence the query blocks go last-first (longest causal range first).
//  * Staging: K/V tiles move HBM -> LDS by DMA (global_load_lds_dwordx4), double
//    buffered: tile t+1 streams into one buffer pair while tile t is computed from the
//    other, one barrier per tile, no staging registers and no LDS store instructions.
//    A wave's whole-block DMA takes the block base as a uniform (scalar) base and a
//    fixed per-lane 32-bit offset, so an issue costs no vector address arithmetic (the
//    DMAs are inline asm, hidden from the compiler's wait counting: dma16); only
//    a block crossing the causal bound takes the per-row path. The LDS reads likewise
//    take per-lane offsets computed once and carry the buffer and key-group part as
//    immediates (config 4 chunks: 337 -> 328 us for the two together).
//    Rows are unpadded with an XOR swizzle of their 16-byte chunks (lds_swizzle), which
//    keeps the K and transposed V reads free of bank conflicts. The tile's 4 block ids
//    come from one vector load issued a tile ahead, so no DMA waits on a table read.
//  * Online softmax in fp32, base-2 domain, with lazy rescaling (the running max is
//    raised only when a tile exceeds it by more than 2^8); causal mask key <= query
//    position, applied only on tiles that cross the workgroup's first query position,
//    with positions from context_lens - query_lens (reference core/attention.py:44-53).
//
// MFMA lane layouts (A, B, C of the 32x32x16 f16/bf16 forms) were pinned on the MI355X
// with a one-hot probe before this kernel was written.
#include "attention.h"

namespace pkv {
namespace {

constexpr int kBS = 16;
constexpr int kKT = 64;          // keys per staged tile
constexpr int kQT = 32;          // queries per wave task

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma;
template <>
struct Mfma<_Float16> {
    __device__ __forceinline__ static f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
    __device__ __forceinline__ static uint32_t pack(float lo, float hi) {
        half2_t v = {(_Float16)lo, (_Float16)hi};
        return __builtin_bit_cast(uint32_t, v);
    }
};
template <>
struct Mfma<bf16_t> {
    __device__ __forceinline__ static f32x16 run(u32x4 a, u32x4 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    }
    __device__ __forceinline__ static uint32_t pack(float lo, float hi) {
        bf16x2_t v = {(__bf16)lo, (__bf16)hi};
        return __builtin_bit_cast(uint32_t, v);
    }
};

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Transposing LDS read (gfx950 ds_read_b64_tr_b16). Within each group of 16 lanes the
// 16 source addresses name 4 consecutive 16-bit elements each; taking those 64
// elements in (lane, element) order, result lane i receives elements i, i+16, i+32
// and i+48. With source lane c of a group pointing at V[key0 + c/4][d0 + 4*(c%4)] of a
// row-major tile, lane i therefore receives V[key0 .. key0+3][d0 + i]: four keys of
// one head_dim column, the MFMA A-operand slice of V^T. (Semantics pinned on the
// MI355X with an in-bounds probe.)
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* ptr) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(ptr));
    return __builtin_bit_cast(uint2, v);
}

// XOR swizzle of a K/V tile row in LDS: logical 16-byte chunk c of row r sits in
// physical slot c ^ lds_swizzle<D>(r) of the unpadded row (period 16 rows). Two
// constraints, for 16- and 32-lane LDS passes alike:
//  * a b128 K read takes one logical chunk of 16 consecutive rows: the swizzle is a
//    permutation over any 16 aligned rows, so the 16 reads hit 16 distinct slots;
//  * 32 lanes of a transposing V read take 4 aligned rows x 4 consecutive logical
//    chunks (one aligned 4-chunk block): the 4 rows' swizzles move that block to 4
//    different blocks, so the 16 reads are distinct too.
// D = 128 (16 chunks = 256 bytes per row, one bank sweep): slot c ^ (4 (r % 4) + r / 4 % 4).
// D = 64 (8 chunks per 128-byte row, two rows per bank sweep): rows of one parity share
// the sweep half, so the same two rules apply to each parity: c ^ (4 bit1 + 2 bit2 + bit3).
template <int D>
__device__ __forceinline__ int lds_swizzle(int r) {
    if constexpr (D == 128) return ((r & 3) << 2) | ((r >> 2) & 3);
    else return (((r >> 1) & 1) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1);
}

// Softmax maxima are only raised when a tile's max exceeds the running one by more
// than 2^8: until then probabilities are exp2(s - m) <= 256 (exact enough in fp32 and
// in the pool dtype), and the O accumulators need no rescale — FlashAttention-3's lazy
// rescaling, which removes the per-tile multiply of every accumulator.
constexpr float kRescaleThreshold = 8.f;

__device__ __forceinline__ uint32_t lds_u32(const void* p) {
    return (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) char*)p);
}
// 16 bytes per lane by LDS DMA to LDS address lds + 16 lane (M0 = lds), from the uniform
// base sbase plus the lane's 32-bit offset, or from the lane's own 64-bit address. Issued
// from inline asm, so the compiler's wait counting never sees an LDS DMA in flight: with
// one in flight it cannot count LDS reads in order and waits for all of them (lgkmcnt(0))
// before every MFMA step (config 4 chunks: 314 -> 310 us). The tile's s_waitcnt(0) and
// barrier order the DMA's data for its readers. M0 is reserved to the compiler (a clobber
// of it is not honoured), so no compiler-generated code of this kernel may rely on M0:
// all of its LDS DMAs go through these helpers.
__device__ __forceinline__ void dma16(const char* sbase, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(lds), "v"(voff), "s"(sbase)
                 : "memory");
}
__device__ __forceinline__ void dma16(const char* addr, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(lds), "v"(addr)
                 : "memory");
}

// One whole live 16-row block of K and V by LDS DMA: the block bases are uniform (SGPR
// pairs) and each lane adds its fixed 32-bit offset inside the block, so an issue costs
// one address add instead of a 64-bit multiply-add and a select per instruction.
template <int IPB, int RPI, int ROWB>
__device__ __forceinline__ void dma_whole_block(const char* kb, const char* vb, const uint32_t* off,
                                                uint16_t* sk, uint16_t* sv, int row0) {
#pragma unroll
    for (int j = 0; j < IPB; ++j) {
        const int dst = (row0 + j * RPI) * ROWB;
        dma16(kb, off[j], lds_u32((char*)sk + dst));
        dma16(vb, off[j], lds_u32((char*)sv + dst));
    }
}

template <typename T, int D, int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void paged_prefill_kernel(
    const AttnParams p) {
    constexpr int NH = G >= 4 ? 4 : G;        // query heads per workgroup
    constexpr int NQT = 4 / NH;               // 32-query tiles per workgroup
    constexpr int HGROUPS = G / NH;           // workgroups per KV head per query block
    constexpr int DSTEPS = D / 16;            // QK^T contraction steps
    constexpr int DTILES = D / 32;            // P·V output d tiles
    constexpr int ROWB = D * 2;               // bytes per K/V row
    constexpr int RPI = 1024 / ROWB;          // rows per DMA instruction (64 lanes x 16 B)
    constexpr int IPB = kBS / RPI;            // DMA instructions per 16-row block, K or V
    constexpr int CPR = ROWB / 16;            // 16-byte chunks per row

    // Two K/V tile buffers, distinct objects so the compiler can tell a DMA into one
    // from reads of the other (it waits on a pending LDS DMA only before reading the
    // buffer that DMA targets).
    __shared__ __attribute__((aligned(1024))) uint16_t s_k0[kKT * D];
    __shared__ __attribute__((aligned(1024))) uint16_t s_v0[kKT * D];
    __shared__ __attribute__((aligned(1024))) uint16_t s_k1[kKT * D];
    __shared__ __attribute__((aligned(1024))) uint16_t s_v1[kKT * D];

    // XCD-ordered work item of this workgroup (the grid is padded to a multiple of 8).
    const int64_t n_qb = (p.max_query_len + NQT * kQT - 1) / (NQT * kQT);
    const int64_t n_items = n_qb * p.num_seqs * p.num_kv_heads * HGROUPS;
    const int64_t per_xcd = (n_items + 7) / 8;
    const int64_t item = (int64_t)(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (item >= n_items) return;
    // Query blocks of a sequence run last-first: the last block sees the most keys
    // (causal), so the longest workgroups are dispatched first and the short ones fill
    // the tail (config 4 chunks 335 -> 331 us).
    const int qblock = (int)(n_qb - 1 - item % n_qb);
    const int seq_slot = (int)((item / n_qb) % p.num_seqs);
    const int hy = (int)(item / (n_qb * p.num_seqs));
    const int kvh = hy / HGROUPS;
    const int hgroup = hy % HGROUPS;
    // Sequences longest first (prefill_seq, attention.h).
    const PrefillSeq ps = prefill_seq(p, seq_slot, kBS);
    const int seq = ps.seq;
    const int64_t q_first = ps.q_first;
    const int q_len = ps.q_len;
    const int ctx = ps.ctx;
    const int q0 = qblock * NQT * kQT;        // first query (within the sequence) of this workgroup
    if (q0 >= q_len) return;
    const int pos0 = ctx - q_len;             // position of query 0
    const int q_last = (q0 + NQT * kQT < q_len ? q0 + NQT * kQT : q_len) - 1;
    const int kmax = pos0 + q_last + 1;       // keys [0, kmax) are visible to this workgroup
    if (kmax <= 0) return;
    const int first_pos = pos0 + q0;          // smallest query position in the workgroup

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int h = lane >> 5;                  // half of the wave
    const int col = lane & 31;                // query column / MFMA row-col index
    const int head = kvh * G + hgroup * NH + wave % NH;
    const int qt = q0 + (wave / NH) * kQT;    // this wave's first query
    const int my_q = qt + col;                // this lane's query (may be >= q_len: not stored)
    const int my_pos = pos0 + my_q;

    // Q^T B operand: lane supplies Q[query my_q][d = 16*step + 8*h .. +8].
    u32x4 qfrag[DSTEPS];
    {
        const int qq = my_q < q_len ? my_q : q_len - 1;
        const char* qrow = reinterpret_cast<const char*>(p.q) +
                           ((q_first + qq) * p.q_st + (int64_t)head * p.q_sh) * (int64_t)sizeof(T);
#pragma unroll
        for (int s = 0; s < DSTEPS; ++s) {
            const Vec16 v = load16(qrow + (s * 16 + h * 8) * (int)sizeof(T));
            qfrag[s] = u32x4{v.w[0], v.w[1], v.w[2], v.w[3]};
        }
    }

    // Fused KV append (p.app_k set): this workgroup's own query tokens' new K/V rows go
    // to their pool slots (KV-head group 0 of the KV head writes them). Nothing in this
    // launch reads those slots: every workgroup stages positions >= pos0 from the
    // source rows instead (dma_tile), so no workgroup waits for another.
    const bool fused = p.app_k != nullptr;
    if (fused && hgroup == 0) {
        constexpr int LPR = ROWB / 16;          // lanes per row, 16 bytes each
        constexpr int RPW = 64 / LPR;           // rows per wave instruction
        const int n_tok = q_len - q0 < NQT * kQT ? q_len - q0 : NQT * kQT;
        const int64_t pool_slots = p.num_blocks * kBS;
        for (int i = wave * RPW + lane / LPR; i < n_tok; i += 4 * RPW) {
            const int64_t tok = q_first + q0 + i;
            const int64_t slot = p.app_slots[tok];
            if ((uint64_t)slot >= (uint64_t)pool_slots) continue;     // outside the pool: skipped
            const int64_t src = (tok * p.app_st + (int64_t)kvh * p.app_sh) * (int64_t)sizeof(T) + (lane % LPR) * 16;
            const int64_t dst = ((slot / kBS) * p.sb + (slot % kBS) * p.ss + (int64_t)kvh * p.sh) * (int64_t)sizeof(T) +
                                (lane % LPR) * 16;
            store16(reinterpret_cast<char*>(const_cast<void*>(p.k)) + dst,
                    load16(reinterpret_cast<const char*>(p.app_k) + src));
            store16(reinterpret_cast<char*>(const_cast<void*>(p.v)) + dst,
                    load16(reinterpret_cast<const char*>(p.app_v) + src));
        }
    }

    f32x16 o[DTILES];
#pragma unroll
    for (int t = 0; t < DTILES; ++t) o[t] = f32x16{};
    float m_run = kNegInf, l_run = 0.f;       // running max (scaled, base 2) and denominator

    const int64_t* table = p.tables + (int64_t)seq * p.table_stride;
    const char* kbase = reinterpret_cast<const char*>(p.k) + (int64_t)kvh * p.sh * (int64_t)sizeof(T);
    const char* vbase = reinterpret_cast<const char*>(p.v) + (int64_t)kvh * p.sh * (int64_t)sizeof(T);
    const int64_t block_bytes = p.sb * (int64_t)sizeof(T);
    const int64_t slot_bytes = p.ss * (int64_t)sizeof(T);

    // Block ids of 64-key tile kt: lane l holds entry 4 kt + l % 4, the index clamped to
    // the last block with a visible key, so every lane loads a valid table entry without
    // a branch (kmax <= context <= table width x 16). A block at or beyond kmax is staged
    // by position, never from its id: dma_tile sends it to the redirect path.
    const int nb_last = (kmax - 1) / kBS;
    auto tile_ids = [&](int kt) -> int64_t {
        const int b = kt * (kKT / kBS) + (lane & 3);
        return table[b < nb_last ? b : nb_last];
    };
    // Tile staging by LDS DMA (global_load_lds_dwordx4: lane i's 16 bytes land at the
    // instruction's LDS base + 16 i, no registers involved). Wave w stages block w of
    // the tile (16 rows) for K and V; instruction j covers rows 16 w + RPI j .. +RPI.
    // Rows at or beyond kmax, and blocks whose id is outside the pool, are redirected
    // to the tile's first row (a valid key): masked to -inf in S, so their finite V rows
    // get probability 0.
    const int dma_row = lane / CPR;           // row within the instruction's RPI rows
    const int dma_slot = lane % CPR;          // physical 16-byte slot written by this lane
    // This lane's byte offset inside a block for each of its DMA instructions (the row
    // within the block and the swizzled source chunk), fixed for the whole kernel.
    uint32_t lane_off[IPB];
#pragma unroll
    for (int j = 0; j < IPB; ++j) {
        const int r = wave * kBS + j * RPI + dma_row;
        lane_off[j] = (uint32_t)((r % kBS) * slot_bytes) + (uint32_t)((dma_slot ^ lds_swizzle<D>(r)) * 16);
    }
    const bool offs_fit = kBS * slot_bytes + ROWB <= (int64_t)0xffffffff;
    // With a fused append, key positions >= pos0 (this pass's new tokens) come from the
    // source rows: key position j is packed token q_first + j - pos0.
    const int new_from = fused ? pos0 : 0x7fffffff;
    const char* knew = fused ? reinterpret_cast<const char*>(p.app_k) + (int64_t)kvh * p.app_sh * (int64_t)sizeof(T)
                             : nullptr;
    const char* vnew = fused ? reinterpret_cast<const char*>(p.app_v) + (int64_t)kvh * p.app_sh * (int64_t)sizeof(T)
                             : nullptr;
    const int64_t new_row_bytes = p.app_st * (int64_t)sizeof(T);
    auto dma_tile = [&](int kt, int64_t ids, uint16_t* sk, uint16_t* sv) {
        const int64_t id0 = readlane64(ids, 0);
        const int64_t idw = readlane64(ids, wave);
        const bool okw = (uint64_t)idw < (uint64_t)p.num_blocks;
        const int row0 = kt * kKT + wave * kBS;                       // first key of this wave's block
        // The common case; one uniform branch (bitwise &: no short-circuit branches).
        if (okw & offs_fit & (row0 + kBS <= kmax) & (row0 + kBS <= new_from)) {
            dma_whole_block<IPB, RPI, ROWB>(kbase + idw * block_bytes, vbase + idw * block_bytes, lane_off, sk, sv,
                                            wave * kBS);
            return;
        }
        // The redirect target, key kt * kKT: with a fused append it is a new row when it
        // lies at or past pos0 (its pool slot may be mid-write in this launch and its old
        // contents need not be finite, and a 0 probability times a NaN V is NaN).
        const int key0 = kt * kKT;
        const char* ksafe;
        const char* vsafe;
        if (key0 >= new_from) {
            const int64_t o = (q_first + key0 - pos0) * new_row_bytes;
            ksafe = knew + o;
            vsafe = vnew + o;
        } else {
            const int64_t o = (uint64_t)id0 < (uint64_t)p.num_blocks ? id0 * block_bytes : 0;
            ksafe = kbase + o;
            vsafe = vbase + o;
        }
#pragma unroll
        for (int j = 0; j < IPB; ++j) {
            const int r = wave * kBS + j * RPI + dma_row;
            const int key = kt * kKT + r;
            const int64_t chunk = (int64_t)((dma_slot ^ lds_swizzle<D>(r)) * 16);
            const char* ks;
            const char* vs;
            if (key >= new_from && key < kmax) {                      // a new row: from the source
                const int64_t off = (q_first + key - pos0) * new_row_bytes + chunk;
                ks = knew + off;
                vs = vnew + off;
            } else if (okw && key < kmax) {
                const int64_t off = idw * block_bytes + (int64_t)(r % kBS) * slot_bytes + chunk;
                ks = kbase + off;
                vs = vbase + off;
            } else {
                ks = ksafe + chunk;
                vs = vsafe + chunk;
            }
            const int dst = (wave * kBS + j * RPI) * ROWB;
            dma16(ks, lds_u32((char*)sk + dst));
            dma16(vs, lds_u32((char*)sv + dst));
        }
    };

    // Transposed V^T reads: source lane c of each 16-lane group points at key row
    // c / 4 of its 4-key group, head_dim column d0 + 4 * (c % 4); groups 0/2 cover
    // columns 0-15 of the 32-wide d tile, groups 1/3 columns 16-31.
    const int grp = lane >> 4;
    const int tr_key = (lane & 15) >> 2;
    const int tr_col = 16 * (grp & 1) + 4 * (lane & 3);

    // Swizzled LDS addresses (bytes) of this lane's operands. K: row half*32 + col,
    // logical chunk 2 s + h. V (transposing reads): rows kk + tr_key and kk + tr_key + 8
    // of the step's 16-key group kk, logical chunk (32 t + tr_col) / 8, 8-byte half
    // (lane & 1); the swizzle of those rows does not depend on the group.
    const int k_swz = lds_swizzle<D>(col);
    const int v_cb = (tr_col >> 3);
    const int v_lo_swz = lds_swizzle<D>(4 * (grp >> 1) + tr_key);
    const int v_hi_swz = lds_swizzle<D>(4 * (grp >> 1) + tr_key + 8);
    const int v_byte = 8 * (lane & 1);
    // Per-lane byte offsets inside a tile buffer, fixed for the kernel: the K read of
    // step s (row col) and the V^T reads of d tile t (rows tr_key, tr_key + 8 of a 16-key
    // group). Everything else in an LDS address — the buffer, the 32-key half, the key
    // group — is a constant the read instruction carries as its immediate offset.
    uint32_t koff[DSTEPS], voff_lo[DTILES], voff_hi[DTILES];
#pragma unroll
    for (int s = 0; s < DSTEPS; ++s) {
        koff[s] = (uint32_t)(col * ROWB + (((2 * s + h) ^ k_swz) << 4));
        asm volatile("" : "+v"(koff[s]));
    }
#pragma unroll
    for (int t = 0; t < DTILES; ++t) {
        voff_lo[t] = (uint32_t)((4 * (grp >> 1) + tr_key) * ROWB + v_byte + (((4 * t + v_cb) ^ v_lo_swz) << 4));
        voff_hi[t] = (uint32_t)((4 * (grp >> 1) + tr_key + 8) * ROWB + v_byte + (((4 * t + v_cb) ^ v_hi_swz) << 4));
        asm volatile("" : "+v"(voff_lo[t]), "+v"(voff_hi[t]));
    }

    const int n_tiles = (kmax + kKT - 1) / kKT;
    int64_t ids = tile_ids(0);
    dma_tile(0, ids, s_k0, s_v0);
    ids = tile_ids(1);
    // One tile: wait for this wave's DMA of tile kt, meet the other waves (their DMAs
    // have landed and they are done with tile kt-1, so its buffer is free), compute S^T,
    // start the DMA of tile kt+1 into the free buffer, then the softmax and P·V.
    auto tile = [&](int kt, const uint16_t* tile_k, const uint16_t* tile_v, uint16_t* nk, uint16_t* nv) {
        __builtin_amdgcn_s_waitcnt(0);
        lds_barrier();

        // ---- S^T for 64 keys: two 32-key MFMA tiles.
        // Both 32-key halves' K fragments first, then the two accumulators' MFMAs
        // interleaved, so each LDS read feeds MFMAs of both halves; the phase runs at
        // raised wave priority so the SIMD's other wave fills the gaps with its softmax
        // rather than holding these MFMAs back (config 4 chunks: 348.5 -> 341 us).
        __builtin_amdgcn_s_setprio(1);
        f32x16 st[2];
        {
            u32x4 kf[2][DSTEPS];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const char* kt0 = reinterpret_cast<const char*>(tile_k) + half * 32 * ROWB;
#pragma unroll
                for (int s = 0; s < DSTEPS; ++s) {
                    const uint4 a = *reinterpret_cast<const uint4*>(kt0 + koff[s]);
                    kf[half][s] = u32x4{a.x, a.y, a.z, a.w};
                }
            }
            st[0] = f32x16{};
            st[1] = f32x16{};
#pragma unroll
            for (int s = 0; s < DSTEPS; ++s) {
                st[0] = Mfma<T>::run(kf[0][s], qfrag[s], st[0]);
                st[1] = Mfma<T>::run(kf[1][s], qfrag[s], st[1]);
            }
        }
        __builtin_amdgcn_s_setprio(0);
        // The next tile's DMA goes out after the S^T MFMAs (issued at the tile's top, it
        // delayed them: config 4 chunks 332 -> 325 us for the move, with the DMA still
        // visible to the compiler; 318 vs 310 us between the two places with it hidden).
        if (kt + 1 < n_tiles) {
            dma_tile(kt + 1, ids, nk, nv);
            ids = tile_ids(kt + 2);
        }
        // ---- causal mask only on tiles that cross the workgroup's first query position.
        if (kt * kKT + kKT - 1 > first_pos) {
#pragma unroll
            for (int half = 0; half < 2; ++half)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kt * kKT + half * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (key > my_pos) st[half][r] = kNegInf;
                }
        }
        // ---- tile max of this query over our 32 keys and the partner lane's 32.
        float mt = kNegInf;
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
            for (int r = 0; r < 16; ++r) mt = fmaxf(mt, st[half][r]);
        mt = max_across32(mt) * p.scale_log2;   // scale > 0: max commutes with it
        asm("" : "+v"(mt));   // mt stays rounded: m_run - mt below is not contracted into an fma
        // Raise the running max only when this tile exceeds it by more than 2^8.
        const bool raise = mt > m_run + kRescaleThreshold;
        const float m_new = raise ? mt : m_run;
        const float alpha = raise ? fast_exp2(m_run - mt) : 1.f;   // exp2(-inf) = 0 for m_run = -inf
        if (__builtin_amdgcn_ballot_w64(raise)) {
#pragma unroll
            for (int t = 0; t < DTILES; ++t) o[t] *= alpha;
        }
        m_run = m_new;
        // A query with no visible key yet keeps m = -inf; its scores are all -inf, so any
        // finite offset gives exp2(-inf) = 0 without a per-element select.
        const float m_off = m_new == kNegInf ? 0.f : m_new;
        float psum = 0.f;
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float e = fast_exp2(fmaf(st[half][r], p.scale_log2, -m_off));
                st[half][r] = e;
                psum += e;
            }
        psum = sum_across32(psum);
        l_run = l_run * alpha + psum;

        // ---- O^T += V^T · P^T, 16 keys per MFMA step. Step s uses accumulator
        // registers 8*(s%2) .. +8 of tile s/2: keys 16*(s%2) + 4h + {0..3} and +8.
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const f32x16& sv = st[s >> 1];
            const int r0 = 8 * (s & 1);
            const u32x4 pb = {Mfma<T>::pack(sv[r0 + 0], sv[r0 + 1]), Mfma<T>::pack(sv[r0 + 2], sv[r0 + 3]),
                              Mfma<T>::pack(sv[r0 + 4], sv[r0 + 5]), Mfma<T>::pack(sv[r0 + 6], sv[r0 + 7])};
            // This lane's 4-key groups: rows 4 (grp / 2) .. +3 and +8 .. +11 of the step's
            // 16-key group (lane groups 0-1: h = 0, groups 2-3: h = 1), in voff_lo / voff_hi.
            const char* vgrp = reinterpret_cast<const char*>(tile_v) + ((s >> 1) * 32 + 16 * (s & 1)) * ROWB;
#pragma unroll
            for (int t = 0; t < DTILES; ++t) {
                const uint2 lo = lds_read_tr16(reinterpret_cast<const uint16_t*>(vgrp + voff_lo[t]));
                const uint2 hi = lds_read_tr16(reinterpret_cast<const uint16_t*>(vgrp + voff_hi[t]));
                o[t] = Mfma<T>::run(u32x4{lo.x, lo.y, hi.x, hi.y}, pb, o[t]);
            }
        }
    };
    // Two tiles per trip, so every buffer reference names a fixed array.
    for (int kt = 0; kt < n_tiles; kt += 2) {
        tile(kt, s_k0, s_v0, s_k1, s_v1);
        if (kt + 1 < n_tiles) tile(kt + 1, s_k1, s_v1, s_k0, s_v0);
    }

    // ---- normalise and store: lane holds query my_q, d = 32 t + 8 (r/4) + 4 h + r%4.
    if (my_q < q_len) {
        const float inv = 1.f / l_run;
        T* orow = reinterpret_cast<T*>(p.out) + (q_first + my_q) * p.out_st + (int64_t)head * p.out_sh;
#pragma unroll
        for (int t = 0; t < DTILES; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 32 * t + 8 * i + 4 * h;
                const uint32_t w0 = Mfma<T>::pack(o[t][4 * i] * inv, o[t][4 * i + 1] * inv);
                const uint32_t w1 = Mfma<T>::pack(o[t][4 * i + 2] * inv, o[t][4 * i + 3] * inv);
                *reinterpret_cast<uint2*>(orow + d) = make_uint2(w0, w1);
            }
    }
}

// Workgroups of the MFMA kernel's flat grid for group size `group`: the work items
// padded to a multiple of 8 (the kernel maps the grid to work items XCD by XCD and
// retires the padding). -1 for a group the kernel has no instance of.
int64_t prefill_workgroups(const AttnParams& p, int group) {
    if (group != 1 && group != 2 && group != 4 && group != 8) return -1;
    const int nh = group >= 4 ? 4 : group;
    const int nqt = 4 / nh;
    const int64_t items = ceil_div(p.max_query_len, nqt * kQT) * p.num_seqs * p.num_kv_heads * (group / nh);
    return ceil_div(items, 8) * 8;
}

template <typename T, int D, int G>
int launch_g(const AttnParams& p, hipStream_t stream) {
    const int64_t wgs = prefill_workgroups(p, G);
    if (wgs == 0) return PKV_OK;
    paged_prefill_kernel<T, D, G><<<dim3((unsigned)wgs), 256, 0, stream>>>(p);
    return check_launch("paged prefill attention");
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

template <typename T>
int launch_t(const AttnParams& p, hipStream_t stream) {
    if (p.head_dim == 64) return launch_d<T, 64>(p, stream);
    if (p.head_dim == 128) return launch_d<T, 128>(p, stream);
    return PKV_EUNSUPPORTED;
}

}  // namespace

bool prefill_tuned(const AttnParams& p, int dtype) {
    if (p.block_size != kBS) return false;
    if (p.head_dim != 64 && p.head_dim != 128) return false;
    if (dtype != PKV_FLOAT16 && dtype != PKV_BFLOAT16) return false;
    // Instances exist for GQA groups 1/2/4/8 only, and the grid is one dimension.
    const int64_t wgs = prefill_workgroups(p, p.group);
    if (wgs < 0 || wgs > 0x7fffffff) return false;
    // Masked-off rows are staged from a valid row of the pool: needs a non-empty pool.
    if (p.num_blocks < 1) return false;
    // 16-byte rows and 8-byte output stores need aligned pointers and strides; so do the
    // source rows of a fused append, which are staged by the same 16-byte DMA.
    uint64_t probe = (uint64_t)(uintptr_t)p.q | (uint64_t)(uintptr_t)p.k | (uint64_t)(uintptr_t)p.v |
                     (uint64_t)(uintptr_t)p.out | (uint64_t)(p.q_st * 2) | (uint64_t)(p.q_sh * 2) |
                     (uint64_t)(p.sb * 2) | (uint64_t)(p.ss * 2) | (uint64_t)(p.sh * 2) |
                     (uint64_t)(p.out_st * 2) | (uint64_t)(p.out_sh * 2);
    if (p.app_k)
        probe |= (uint64_t)(uintptr_t)p.app_k | (uint64_t)(uintptr_t)p.app_v | (uint64_t)(p.app_st * 2) |
                 (uint64_t)(p.app_sh * 2);
    return probe % 16 == 0;
}

int launch_prefill_attention(const AttnParams& p, int dtype, hipStream_t stream) {
    if (!prefill_tuned(p, dtype)) return PKV_EUNSUPPORTED;
    if (p.num_seqs == 0 || p.num_tokens == 0) return PKV_OK;
    if (dtype == PKV_FLOAT16) return launch_t<_Float16>(p, stream);
    return launch_t<bf16_t>(p, stream);
}

}  // namespace pkv
