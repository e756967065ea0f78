// Paged prefill / chunked-prefill attention over float32 pools on the matrix cores
// (v_mfma_f32_32x32x2_f32, gfx950): block size 16, head_dim 64/128, GQA group
// 1/2/4/8. Replaces, for float32 pools, the reference's ragged loop
// (inference_server/core/attention.py:156-187) where the tiled fp32 kernel
// (attn_f32.hip) does the arithmetic on the vector ALUs.
//
//  * Work unit as in the 16-bit MFMA kernel (attn_prefill.hip): a workgroup of 4 waves =
//    (sequence, KV head, query block); with a GQA group G >= 4 the waves are 4 query
//    heads sharing every staged K/V tile, with G < 4 they are 4/G consecutive 32-query
//    tiles x G heads. XCD-ordered grid, each sequence's query blocks last-first.
//  * S^T = K · Q^T per 32-key x 32-query tile: A = K (LDS), B = Q^T (registers, loaded
//    once). The 32x32x2 instruction contracts two head_dim elements, one per half-wave:
//    step s takes elements s (lanes 0-31) and s + D/2 (lanes 32-63), so one 16-byte LDS
//    read of a K row feeds four steps. Accumulator register r of lane l holds
//    S^T[key 8 (r/4) + 4 (l/32) + r%4][query l%32].
//  * O^T += V^T · P^T: register r of the S^T accumulator, as it stands, is the B operand
//    of one P·V step over the two keys 8 (r/4) + r%4 (lanes 0-31) and that key + 4
//    (lanes 32-63); the A operand is V^T: lane i reads V[that key][32 t + i] (one 4-byte
//    LDS read). No data moves between the two products.
//  * Online softmax in fp32, base 2, lazy rescaling (the running max is raised only when
//    a tile exceeds it by more than 2^8); causal mask only on tiles that cross the
//    workgroup's first query position (positions context_lens - query_lens + i,
//    core/attention.py:44-53). Nothing is rounded below fp32 (the reference's fp32
//    path: probs.to(v.dtype) is a no-op).
//  * Staging: 32-key tiles (two blocks) of K and V move HBM -> LDS by DMA, double
//    buffered, one barrier per tile; wave w stages rows 8w .. 8w + 7 of both. The DMAs
//    are inline asm, hidden from the compiler's wait counting (with an LDS DMA in
//    flight it waits for every LDS read before each MFMA); the tile's s_waitcnt(0) and
//    barrier order their data. Rows are unpadded and XOR-swizzled in 16-byte chunks:
//    K row r's chunk c sits at c ^ (r % 16) (a K read takes one chunk of 16 rows per
//    pass), V row r's at c ^ 8 (bit 2 of r) (a V read takes 32 consecutive elements of
//    one row in each half-wave, rows 4 apart).
// Rows past the visible keys and blocks whose id is outside the pool are staged from a
// valid row (masked to -inf, so their finite V rows get probability 0).
#include "attention.h"

namespace pkv {
namespace {

constexpr int kBS = 16;
constexpr int kKT = 32;   // keys per staged tile (two blocks)
constexpr int kQT = 32;   // queries per wave task

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x16 mfma32x2(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t lds_u32(const void* p) {
    return (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) char*)p);
}
// 16 bytes per lane by LDS DMA to LDS address lds + 16 lane (M0 = lds), from the uniform
// base sbase plus the lane's 32-bit offset, or from the lane's own 64-bit address; inline
// asm, so the compiler's wait counting never sees an LDS DMA in flight. M0 is reserved to
// the compiler (a clobber of it is not honoured): no compiler-generated code of this
// kernel may rely on M0, so all of its LDS DMAs go through these helpers.
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

// Raise the running max only when a tile exceeds it by more than 2^8 (until then the
// unnormalised weights exp2(s - m) stay <= 256 and the accumulators need no rescale).
constexpr float kRescaleThreshold = 8.f;

template <int D, int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void paged_prefill_f32_kernel(const AttnParams p) {
    constexpr int NH = G >= 4 ? 4 : G;        // query heads per workgroup
    constexpr int NQT = 4 / NH;               // 32-query tiles per workgroup
    constexpr int HGROUPS = G / NH;           // workgroups per KV head per query block
    constexpr int QS = D / 2;                 // S^T contraction steps
    constexpr int KR = D / 8;                 // 16-byte K reads per tile (4 steps each)
    constexpr int DT = D / 32;                // P·V output d tiles
    constexpr int ROWB = D * 4;               // bytes per K/V row
    constexpr int CPR = ROWB / 16;            // 16-byte chunks per row (16 or 32)
    constexpr int RPI = 1024 / ROWB;          // rows per DMA instruction (64 lanes x 16 B)
    constexpr int NI = (kKT / 4) / RPI;       // DMA instructions per wave per tile and side
    static_assert(CPR >= 16 && NI >= 1, "unsupported head_dim");

    __shared__ __attribute__((aligned(1024))) float s_k0[kKT * D];
    __shared__ __attribute__((aligned(1024))) float s_v0[kKT * D];
    __shared__ __attribute__((aligned(1024))) float s_k1[kKT * D];
    __shared__ __attribute__((aligned(1024))) float s_v1[kKT * D];

    // XCD-ordered work item of this workgroup (the grid is padded to a multiple of 8).
    const int64_t n_qb = (p.max_query_len + NQT * kQT - 1) / (NQT * kQT);
    const int64_t n_items = n_qb * p.num_seqs * p.num_kv_heads * HGROUPS;
    const int64_t per_xcd = (n_items + 7) / 8;
    const int64_t item = (int64_t)(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (item >= n_items) return;
    const int qblock = (int)(n_qb - 1 - item % n_qb);
    const int hy = (int)(item / (n_qb * p.num_seqs));
    const int kvh = hy / HGROUPS;
    const int hgroup = hy % HGROUPS;
    // Sequences longest first (prefill_seq, attention.h).
    const PrefillSeq ps = prefill_seq(p, (int)((item / n_qb) % p.num_seqs), kBS);
    const int seq = ps.seq;
    const int64_t q_first = ps.q_first;
    const int q_len = ps.q_len;
    const int q0 = qblock * NQT * kQT;
    if (q0 >= q_len) return;
    const int ctx = ps.ctx;
    const int pos0 = ctx - q_len;             // position of query 0
    const int q_last = (q0 + NQT * kQT < q_len ? q0 + NQT * kQT : q_len) - 1;
    const int kmax = pos0 + q_last + 1;       // keys [0, kmax) are visible to this workgroup
    if (kmax <= 0) return;
    const int first_pos = pos0 + q0;

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int h = lane >> 5;                  // half-wave
    const int col = lane & 31;                // query column / key row of the MFMA tile
    const int head = kvh * G + hgroup * NH + wave % NH;
    const int my_q = q0 + (wave / NH) * kQT + col;
    const int my_pos = pos0 + my_q;

    // Q^T B operand: step s takes element s + (D/2) h of this lane's query row.
    float qf[QS];
    {
        const int qq = my_q < q_len ? my_q : q_len - 1;
        const float* qrow = static_cast<const float*>(p.q) + (q_first + qq) * p.q_st + (int64_t)head * p.q_sh + h * QS;
#pragma unroll
        for (int c = 0; c < QS / 4; ++c) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(qrow + 4 * c);
            qf[4 * c] = v[0];
            qf[4 * c + 1] = v[1];
            qf[4 * c + 2] = v[2];
            qf[4 * c + 3] = v[3];
        }
    }

    f32x16 o[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] = f32x16{};
    float m_run = kNegInf, l_run = 0.f;

    const int64_t* table = p.tables + (int64_t)seq * p.table_stride;
    const char* kbase = reinterpret_cast<const char*>(p.k) + (int64_t)kvh * p.sh * 4;
    const char* vbase = reinterpret_cast<const char*>(p.v) + (int64_t)kvh * p.sh * 4;
    const int64_t block_bytes = p.sb * 4;
    const int64_t slot_bytes = p.ss * 4;

    // Block ids of tile kt: lane l holds entry 2 kt + l % 2, the index clamped to the last
    // block with a visible key, so every lane loads a valid table entry without a branch
    // (kmax <= context <= table width x 16). A block at or beyond kmax is staged by
    // position, never from its id: dma_tile sends it to the redirect path.
    const int nb_last = (kmax - 1) / kBS;
    auto tile_ids = [&](int kt) -> int64_t {
        const int b = kt * (kKT / kBS) + (lane & 1);
        return table[b < nb_last ? b : nb_last];
    };
    // This lane's DMA sources: instruction j covers tile rows 8 wave + RPI j .. + RPI;
    // lane writes physical chunk dma_p of row 8 wave + RPI j + lane / CPR, which holds
    // logical chunk dma_p ^ (row % 16) (K) or dma_p ^ 8 (bit 2 of row) (V).
    const int dma_p = lane % CPR;
    uint32_t koff[NI], voff_dma[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const int rt = 8 * wave + RPI * j + lane / CPR;       // row within the tile
        const int rb = rt % kBS;                               // row within its block
        koff[j] = (uint32_t)(rb * slot_bytes) + (uint32_t)((dma_p ^ (rt & 15)) * 16);
        voff_dma[j] = (uint32_t)(rb * slot_bytes) + (uint32_t)((dma_p ^ (8 * ((rt >> 2) & 1))) * 16);
    }
    const bool offs_fit = kBS * slot_bytes + ROWB <= (int64_t)0xffffffff;
    auto dma_tile = [&](int kt, int64_t ids, float* sk, float* sv) {
        const int blk = wave >> 1;                             // this wave's block of the tile
        const int64_t idw = readlane64(ids, blk);
        const bool okw = (uint64_t)idw < (uint64_t)p.num_blocks;
        const int row0 = kt * kKT + 8 * wave;                  // first key this wave stages
        if (okw & offs_fit & (row0 + 8 <= kmax)) {              // the common case (one branch)
            const char* kb = kbase + idw * block_bytes;
            const char* vb = vbase + idw * block_bytes;
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                const int dst = (8 * wave + RPI * j) * ROWB;
                dma16(kb, koff[j], lds_u32((char*)sk + dst));
                dma16(vb, voff_dma[j], lds_u32((char*)sv + dst));
            }
            return;
        }
        // Rows at or past kmax and blocks outside the pool read the tile's first row
        // (block id0, or block 0 when that id is out of the pool too).
        const int64_t id0 = readlane64(ids, 0);
        const int64_t safe = (uint64_t)id0 < (uint64_t)p.num_blocks ? id0 * block_bytes : 0;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int rt = 8 * wave + RPI * j + lane / CPR;
            const int key = kt * kKT + rt;
            const int64_t kc = (int64_t)((dma_p ^ (rt & 15)) * 16);
            const int64_t vc = (int64_t)((dma_p ^ (8 * ((rt >> 2) & 1))) * 16);
            const int64_t row = (okw && key < kmax) ? idw * block_bytes + (int64_t)(rt % kBS) * slot_bytes : safe;
            const int dst = (8 * wave + RPI * j) * ROWB;
            dma16(kbase + row + kc, lds_u32((char*)sk + dst));
            dma16(vbase + row + vc, lds_u32((char*)sv + dst));
        }
    };

    // LDS read offsets, fixed for the kernel. K: row col, logical chunk KR h + g of
    // read g (elements 4 g .. +3 of the lane's half) at physical chunk that ^ (col % 16).
    // V^T: row 8 (r/4) + 4 h + r%4 of step r, element 32 t + col, i.e. physical chunk
    // (8 t + col / 4) ^ 8 h; the row part that depends on r is an immediate.
    const uint32_t k_row = (uint32_t)(col * ROWB);
    const int k_swz = col & 15;
    uint32_t vr_off[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) {
        vr_off[t] = (uint32_t)(4 * h * ROWB + 4 * col + 128 * (t ^ h));
        asm volatile("" : "+v"(vr_off[t]));
    }

    const int n_tiles = (kmax + kKT - 1) / kKT;
    int64_t ids = tile_ids(0);
    dma_tile(0, ids, s_k0, s_v0);
    ids = tile_ids(1);
    auto tile = [&](int kt, const float* tile_k, const float* tile_v, float* nk, float* nv) {
        __builtin_amdgcn_s_waitcnt(0);
        lds_barrier();
        // ---- S^T for 32 keys x 32 queries.
        f32x16 st = f32x16{};
        {
            const char* kt0 = reinterpret_cast<const char*>(tile_k) + k_row;
#pragma unroll
            for (int g = 0; g < KR; ++g) {
                const f32x4 a = *reinterpret_cast<const f32x4*>(kt0 + (((KR * h + g) ^ k_swz) << 4));
#pragma unroll
                for (int u = 0; u < 4; ++u) st = mfma32x2(a[u], qf[4 * g + u], st);
            }
        }
        if (kt + 1 < n_tiles) {
            dma_tile(kt + 1, ids, nk, nv);
            ids = tile_ids(kt + 2);
        }
        // ---- causal mask only on tiles that cross the workgroup's first query position.
        if (kt * kKT + kKT - 1 > first_pos) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kt * kKT + 8 * (r >> 2) + 4 * h + (r & 3);
                if (key > my_pos) st[r] = kNegInf;
            }
        }
        float mt = kNegInf;
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = fmaxf(mt, st[r]);
        mt = max_across32(mt) * p.scale_log2;      // scale > 0: max commutes with it
        asm("" : "+v"(mt));   // mt stays rounded: m_run - mt below is not contracted into an fma
        const bool raise = mt > m_run + kRescaleThreshold;
        const float m_new = raise ? mt : m_run;
        const float alpha = raise ? fast_exp2(m_run - mt) : 1.f;   // exp2(-inf) = 0 for m_run = -inf
        if (__builtin_amdgcn_ballot_w64(raise)) {
#pragma unroll
            for (int t = 0; t < DT; ++t) o[t] *= alpha;
        }
        m_run = m_new;
        // A query with no visible key yet keeps m = -inf; its scores are all -inf, so any
        // finite offset gives exp2(-inf) = 0.
        const float m_off = m_new == kNegInf ? 0.f : m_new;
        float psum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float e = fast_exp2(fmaf(st[r], p.scale_log2, -m_off));
            st[r] = e;
            psum += e;
        }
        psum = sum_across32(psum);
        l_run = l_run * alpha + psum;
        // ---- O^T += V^T · P^T: step r takes keys 8 (r/4) + r%4 and + 4.
        const char* tv = reinterpret_cast<const char*>(tile_v);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const char* vrow = tv + (8 * (r >> 2) + (r & 3)) * ROWB;
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                const float a = *reinterpret_cast<const float*>(vrow + vr_off[t]);
                o[t] = mfma32x2(a, st[r], o[t]);
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
        float* orow = static_cast<float*>(p.out) + (q_first + my_q) * p.out_st + (int64_t)head * p.out_sh;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<f32x4*>(orow + 32 * t + 8 * i + 4 * h) =
                    f32x4{o[t][4 * i] * inv, o[t][4 * i + 1] * inv, o[t][4 * i + 2] * inv, o[t][4 * i + 3] * inv};
    }
}

int64_t workgroups(const AttnParams& p, int group) {
    const int nh = group >= 4 ? 4 : group;
    const int nqt = 4 / nh;
    const int64_t items = ceil_div(p.max_query_len, nqt * kQT) * p.num_seqs * p.num_kv_heads * (group / nh);
    return ceil_div(items, 8) * 8;
}

template <int D, int G>
int launch_g(const AttnParams& p, hipStream_t stream) {
    const int64_t wgs = workgroups(p, G);
    if (wgs == 0) return PKV_OK;
    paged_prefill_f32_kernel<D, G><<<dim3((unsigned)wgs), 256, 0, stream>>>(p);
    return check_launch("fp32 MFMA prefill attention");
}

template <int D>
int launch_d(const AttnParams& p, hipStream_t stream) {
    switch (p.group) {
        case 1: return launch_g<D, 1>(p, stream);
        case 2: return launch_g<D, 2>(p, stream);
        case 4: return launch_g<D, 4>(p, stream);
        case 8: return launch_g<D, 8>(p, stream);
        default: return PKV_EUNSUPPORTED;
    }
}

}  // namespace

int launch_prefill_f32_mfma(const AttnParams& p, hipStream_t stream) {
    if (!p.qsl || p.app_k || p.block_size != kBS || (p.head_dim != 64 && p.head_dim != 128)) return PKV_EUNSUPPORTED;
    // Batches of 1-token rows only stay on the tiled fp32 kernel: a 32-query tile would
    // carry one query (64 rows of ctx 100-2000, d64: 341 vs 222 us). Any longer row and
    // the tiles pay (8 x 128-token prefills + 56 one-token rows: 360 vs 835 us; config 1's
    // 8 prompts: 24 vs 51 us; 16 x 512-token chunks at d128, GQA 4: 2.46 vs 13.5 ms).
    if (p.max_query_len <= 1) return PKV_EUNSUPPORTED;
    if (p.group != 1 && p.group != 2 && p.group != 4 && p.group != 8) return PKV_EUNSUPPORTED;
    if (p.num_blocks < 1) return PKV_EUNSUPPORTED;
    // 16-byte rows: query, pool and output pointers and strides.
    const uint64_t probe = (uint64_t)(uintptr_t)p.q | (uint64_t)(uintptr_t)p.k | (uint64_t)(uintptr_t)p.v |
                           (uint64_t)(uintptr_t)p.out | (uint64_t)(p.q_st * 4) | (uint64_t)(p.q_sh * 4) |
                           (uint64_t)(p.sb * 4) | (uint64_t)(p.ss * 4) | (uint64_t)(p.sh * 4) |
                           (uint64_t)(p.out_st * 4) | (uint64_t)(p.out_sh * 4);
    if (probe % 16) return PKV_EUNSUPPORTED;
    if (workgroups(p, p.group) > 0x7fffffff) return PKV_EUNSUPPORTED;
    if (p.num_seqs == 0 || p.num_tokens == 0) return PKV_OK;
    return p.head_dim == 64 ? launch_d<64>(p, stream) : launch_d<128>(p, stream);
}

}  // namespace pkv
