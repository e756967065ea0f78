// fp32 paged attention on 16-key tiles (one block each) over a float32 pool with block
// size 16 and head_dim 64 or 128: decode batches at head_dim 128, prefill-entry batches
// of 1-token rows, and prefill batches the fp32 MFMA kernel (attn_prefill_f32.hip)
// declines. Replaces, for float32 pools, the reference's ragged loop and batched decode
// (inference_server/core/attention.py:130-187) where the only other kernel walks the
// keys one at a time.
//
//  * A wave owns SLOTS = 64 / LPQ (query token, query head) slots of one sequence and
//    one KV head: the G query heads of the GQA group times SLOTS / G consecutive query
//    tokens. Lane (slot, part) holds DPL = D / LPQ consecutive elements (16 or 4) of its
//    slot's query and output accumulator in registers; a score is the LPQ parts'
//    partial dot products summed by DPP. All G heads and all tokens of the wave share
//    one staged copy of every K/V row.
//  * Keys are walked one block at a time. The block's 16 K rows and 16 V rows of the
//    KV head move HBM -> LDS by DMA (global_load_lds_dwordx4) into one of two buffer
//    pairs; block t + 1's DMA is in flight while block t is computed. Lanes read the
//    rows back with 16-byte LDS reads that every slot of the wave shares (one address
//    per part); the 16-byte chunks of a row are stored XOR-swizzled (chunk c at
//    c ^ ((c >> 3) & 7)) so the parts of one read instruction fall in different banks.
//  * Softmax per block, as the reference's mirror folds keys block by block
//    (core/attention_triton.py:309-384): block maximum, rescale of the running
//    denominator and accumulator, then exp2 of the base-2 scores (scores are
//    dot * scale * log2(e)). Everything stays in fp32; the output is acc / l.
//
// Rows past the keys the wave needs re-read the block's first row (a valid key) and
// are masked; a block id outside the pool reads block 0 (memory-safe, out of contract).
#include "attention.h"

namespace pkv {
namespace {

constexpr int kTile = 16;  // keys per tile = the block size this kernel takes

// Sum over the LPQ consecutive lanes of a slot; every lane of the slot gets it.
template <int LPQ>
__device__ __forceinline__ float slot_sum(float x) {
    if constexpr (LPQ >= 2) x += dpp_f32<kDppQuadXor1>(x);
    if constexpr (LPQ >= 4) x += dpp_f32<kDppQuadXor2>(x);
    if constexpr (LPQ >= 8) x += dpp_f32<kDppRowHalfMirror>(x);
    if constexpr (LPQ >= 16) x += dpp_f32<kDppRowMirror>(x);
    if constexpr (LPQ >= 32) {
        const SwapPair s = swap16(x);
        x = s.a + s.b;
    }
    return x;
}

// Position of global 16-byte chunk c within a staged row.
__device__ __forceinline__ constexpr int f32_swz(int c) { return c ^ ((c >> 3) & 7); }

typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <int D, int LPQ, int G>
__global__ __launch_bounds__(64) void paged_f32_kernel(const AttnParams p) {
    constexpr int SLOTS = 64 / LPQ;
    constexpr int TPW = SLOTS / G;          // query tokens per wave
    constexpr int DPL = D / LPQ;            // elements per lane
    constexpr int CPL = DPL / 4;            // 16-byte chunks per lane
    constexpr int RB = D * 4;               // bytes per staged row
    constexpr int NI = kTile * RB / 1024;   // DMA instructions per block side
    static_assert(SLOTS % G == 0 && TPW >= 1 && DPL % 4 == 0 && NI >= 1, "unsupported shape");

    // Two buffer pairs as four distinct objects (explicit waits order them).
    __shared__ __attribute__((aligned(1024))) float s_k0[kTile * D];
    __shared__ __attribute__((aligned(1024))) float s_v0[kTile * D];
    __shared__ __attribute__((aligned(1024))) float s_k1[kTile * D];
    __shared__ __attribute__((aligned(1024))) float s_v1[kTile * D];

    const int lane = lane_id();
    const int kvh = (int)blockIdx.y;
    const int seq = (int)blockIdx.z;
    const int64_t q_first = p.qsl ? p.qsl[seq] : (int64_t)seq;
    const int q_len = p.qsl ? (int)(p.qsl[seq + 1] - q_first) : 1;
    const int t0 = (int)blockIdx.x * TPW;   // the wave's first query token (index within the sequence)
    if (t0 >= q_len) return;
    int64_t ctx = p.ctx_lens[seq];
    const int64_t cap = (int64_t)p.table_width * kTile;
    ctx = ctx < cap ? ctx : cap;
    const int pos0 = (int)(ctx - q_len);    // position of the sequence's first query token

    const int slot = lane / LPQ;
    const int part = lane % LPQ;
    const int tok = t0 + slot / G;
    const int head = kvh * G + slot % G;
    const bool live = tok < q_len;
    const int tq = live ? tok : q_len - 1;
    const int qpos = pos0 + tq;             // this slot sees keys 0 .. qpos

    float q[DPL];
    {
        const float* qrow = reinterpret_cast<const float*>(p.q) + (q_first + tq) * p.q_st + (int64_t)head * p.q_sh +
                            part * DPL;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const f32x4_t v = *reinterpret_cast<const f32x4_t*>(qrow + 4 * c);
            q[4 * c] = v.x;
            q[4 * c + 1] = v.y;
            q[4 * c + 2] = v.z;
            q[4 * c + 3] = v.w;
        }
    }

    const int last = t0 + TPW < q_len ? t0 + TPW : q_len;
    const int kmax = pos0 + last;           // keys the wave needs: 0 .. kmax - 1
    const int n_tiles = (kmax + kTile - 1) / kTile;

    // DMA instruction j, lane l fills bytes [1024 j + 16 l, +16) of a buffer: row r,
    // position P; it loads global chunk f32_swz(P) of row r (f32_swz is an involution).
    const int64_t slot_bytes = p.ss * 4;
    const int64_t block_bytes = p.sb * 4;
    int row_of[NI];
    int64_t off[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const int b = 1024 * j + 16 * lane;
        row_of[j] = b / RB;
        off[j] = (int64_t)row_of[j] * slot_bytes + (int64_t)f32_swz((b % RB) / 16) * 16;
    }
    const int64_t* trow = p.tables + (int64_t)seq * p.table_stride;
    const char* kbase = reinterpret_cast<const char*>(p.k) + (int64_t)kvh * p.sh * 4;
    const char* vbase = reinterpret_cast<const char*>(p.v) + (int64_t)kvh * p.sh * 4;
    auto dma = [&](int t, float* dk, float* dv) {
        int64_t id = *(const __attribute__((address_space(4))) int64_t*)(trow + t);
        id = (uint64_t)id < (uint64_t)p.num_blocks ? id : 0;
        const int valid = kmax - t * kTile;
        const char* kblk = kbase + id * block_bytes;
        const char* vblk = vbase + id * block_bytes;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int64_t o = row_of[j] < valid ? off[j] : off[j] - (int64_t)row_of[j] * slot_bytes;
            const char* ks = kblk + o;
            const char* vs = vblk + o;
            __builtin_amdgcn_global_load_lds(ks, (__attribute__((address_space(3))) void*)(dk + 256 * j), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(vs, (__attribute__((address_space(3))) void*)(dv + 256 * j), 16, 0, 0);
        }
    };

    float m = kNegInf, l = 0.f;
    float acc[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[e] = 0.f;

    auto compute = [&](int t, const float* ck, const float* cv) {
        float s[kTile];
#pragma unroll
        for (int j = 0; j < kTile; ++j) {
            const float* row = ck + j * D;
            float a = 0.f;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const f32x4_t kv = *reinterpret_cast<const f32x4_t*>(row + 4 * f32_swz(part * CPL + c));
                a = __builtin_fmaf(q[4 * c], kv.x, a);
                a = __builtin_fmaf(q[4 * c + 1], kv.y, a);
                a = __builtin_fmaf(q[4 * c + 2], kv.z, a);
                a = __builtin_fmaf(q[4 * c + 3], kv.w, a);
            }
            s[j] = a;
        }
        float mb = kNegInf;
#pragma unroll
        for (int j = 0; j < kTile; ++j) {
            const float x = ref_score_log2<float>(slot_sum<LPQ>(s[j]), p.scale);
            s[j] = t * kTile + j <= qpos ? x : kNegInf;
            mb = fmaxf(mb, s[j]);
        }
        const float m_new = fmaxf(m, mb);
        const float mref = m_new == kNegInf ? 0.f : m_new;   // no key yet: every weight stays 0
        const float alpha = fast_exp2(m - mref);
        l *= alpha;
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[e] *= alpha;
#pragma unroll
        for (int j = 0; j < kTile; ++j) {
            const float pj = fast_exp2(s[j] - mref);
            l += pj;
            const float* row = cv + j * D;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const f32x4_t vv = *reinterpret_cast<const f32x4_t*>(row + 4 * f32_swz(part * CPL + c));
                acc[4 * c] = __builtin_fmaf(pj, vv.x, acc[4 * c]);
                acc[4 * c + 1] = __builtin_fmaf(pj, vv.y, acc[4 * c + 1]);
                acc[4 * c + 2] = __builtin_fmaf(pj, vv.z, acc[4 * c + 2]);
                acc[4 * c + 3] = __builtin_fmaf(pj, vv.w, acc[4 * c + 3]);
            }
        }
        m = m_new;
    };

    if (n_tiles > 0) dma(0, s_k0, s_v0);   // none only for out-of-contract lengths
    for (int t = 0; t < n_tiles; ++t) {
        const bool odd = t & 1;
        if (t + 1 < n_tiles) {
            // The other buffer pair was read by tile t - 1: those LDS reads must be done
            // before a DMA may overwrite it (DMA writes are not ordered behind them).
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
            if (odd) dma(t + 1, s_k0, s_v0);
            else dma(t + 1, s_k1, s_v1);
            __builtin_amdgcn_s_waitcnt(kWaitVm<2 * NI>);      // tile t landed; t + 1 in flight
        } else {
            __builtin_amdgcn_s_waitcnt(kWaitVm<0>);
        }
        if (odd) compute(t, s_k1, s_v1);
        else compute(t, s_k0, s_v0);
    }

    if (live) {
        float* orow = reinterpret_cast<float*>(p.out) + (q_first + tok) * p.out_st + (int64_t)head * p.out_sh +
                      part * DPL;
        const float inv = 1.f / l;
#pragma unroll
        for (int c = 0; c < CPL; ++c)
            *reinterpret_cast<f32x4_t*>(orow + 4 * c) =
                f32x4_t{acc[4 * c] * inv, acc[4 * c + 1] * inv, acc[4 * c + 2] * inv, acc[4 * c + 3] * inv};
    }
}

template <int D, int LPQ, int G>
int launch_one(const AttnParams& p, int max_q, hipStream_t stream) {
    constexpr int TPW = 64 / LPQ / G;
    const int64_t gx = ceil_div((int64_t)max_q, (int64_t)TPW);
    paged_f32_kernel<D, LPQ, G><<<dim3((unsigned)gx, (unsigned)p.num_kv_heads, (unsigned)p.num_seqs), 64, 0, stream>>>(p);
    return check_launch("fp32 paged attention");
}

// Two lane shapes per (D, G): 16 elements per lane (16 / G query tokens per wave at
// D = 64, 8 / G at D = 128) or 4 (4x fewer tokens per wave). The launch takes the
// 16-element shape when its tokens per wave do not exceed the longest query and it
// gives at least one wave per SIMD, else the 4-element one where the group fits its
// slots. A 64-element shape (one query per lane at D = 64) measured slower on large
// batches (16 x 512-token chunks at D = 128, GQA 4: 18.8 ms vs 11.4 ms; 64 x 256 tokens
// at D = 64: 398 vs 333 us; 256+ registers, one wave per SIMD) and equal on small ones.
template <int D, int G>
int launch_dg(const AttnParams& p, hipStream_t stream) {
    constexpr int L1 = D / 16, L2 = D / 4;
    constexpr int T1 = 64 / L1 / G;
    constexpr int T2 = (64 / L2) / G;  // 0 when the group exceeds the narrow shape's slots
    const int64_t mq = p.qsl ? p.max_query_len : 1;
    const int64_t tokens = p.qsl ? p.num_tokens : p.num_seqs;
    const int64_t waves = (tokens / T1 + p.num_seqs) * (int64_t)p.num_kv_heads;
    const int max_q = (int)(mq > 0 ? mq : 1);
    if constexpr (T2 >= 1) {
        if (T1 > mq || waves < 1024) return launch_one<D, L2, G>(p, max_q, stream);
    }
    return launch_one<D, L1, G>(p, max_q, stream);
}

template <int D>
int launch_d(const AttnParams& p, hipStream_t stream) {
    switch (p.group) {
        case 1: return launch_dg<D, 1>(p, stream);
        case 2: return launch_dg<D, 2>(p, stream);
        case 4: return launch_dg<D, 4>(p, stream);
        case 8: return launch_dg<D, 8>(p, stream);
    }
    return PKV_EUNSUPPORTED;
}

}  // namespace

int launch_f32_attention(const AttnParams& p, hipStream_t stream) {
    if (p.block_size != kTile || (p.head_dim != 64 && p.head_dim != 128)) return PKV_EUNSUPPORTED;
    if (p.group != 1 && p.group != 2 && p.group != 4 && p.group != 8) return PKV_EUNSUPPORTED;
    if (p.num_blocks < 1 || p.num_kv_heads > 65535 || p.num_seqs > 65535) return PKV_EUNSUPPORTED;
    // 16-byte vector access to query, pool and output rows.
    const uint64_t probe = (uint64_t)(uintptr_t)p.q | (uint64_t)(uintptr_t)p.k | (uint64_t)(uintptr_t)p.v |
                           (uint64_t)(uintptr_t)p.out | (uint64_t)(p.q_st * 4) | (uint64_t)(p.q_sh * 4) |
                           (uint64_t)(p.sb * 4) | (uint64_t)(p.ss * 4) | (uint64_t)(p.sh * 4) |
                           (uint64_t)(p.out_st * 4) | (uint64_t)(p.out_sh * 4);
    if (probe % 16) return PKV_EUNSUPPORTED;
    // Byte offsets inside a block fit the 32-bit-friendly range the DMA offsets assume.
    if ((int64_t)kTile * p.ss * 4 > 0x7fffffff) return PKV_EUNSUPPORTED;
    if (p.num_seqs == 0 || (p.qsl && p.num_tokens == 0)) return PKV_OK;
    return p.head_dim == 64 ? launch_d<64>(p, stream) : launch_d<128>(p, stream);
}

}  // namespace pkv
