// Tuned paged decode attention for block_size 16, head_dim 64/128, GQA group
// 1/2/4/8, fp16/bf16/fp32.
//
// Single-query decode is a bandwidth-bound GEMV: every K/V byte of the context is
// read once and used for 2*G flops per element, where G = num_heads / num_kv_heads.
// The kernel is therefore organised around HBM traffic and latency, not arithmetic:
//
//  * Work unit = (KV head, 256-token partition, sequence): one 256-thread workgroup
//    of 4 wave64s, 64 tokens (4 blocks) per wave. All G query heads of the GQA group
//    are served by the same K/V read, so K/V are fetched once per KV head, never once
//    per query head (the reference's kernel design re-reads them G times,
//    core/attention_triton.py:181).
//  * Latency chain per wave: ONE vector load of the wave's 4 block-table entries
//    (broadcast with readlane), then all K loads of the 4 blocks at once, the scores,
//    then all V loads at once — issued before the softmax so they are in flight while
//    it runs. No load waits on another load except through the block table.
//  * Split-KV: contexts are cut into partitions so the grid has thousands of
//    workgroups for 256 CUs. A sequence that fits one partition is finished in
//    place; otherwise each partition writes its partial (max, denominator,
//    unnormalised output) and a small second kernel on the same stream merges them
//    with the log-sum-exp rule. Stream order is the only synchronisation: an
//    in-kernel "last workgroup merges" scheme needs an agent-scope release fence per
//    workgroup, which writes back the XCD's L2 and was measured to serialise the
//    whole launch (time grew with the workgroup count, 2.4 ms -> 3.5 ms when the
//    partition was halved).
//  * K layout: lane (token = lane / 4, quarter = lane % 4) holds 16-byte chunks
//    quarter, quarter + 4, ... of its token's K row: one block per load step with
//    fully used 64-byte segments; a quad DPP reduction finishes each score.
//    fp16/bf16 dot products use v_dot2_f32_{f16,bf16} (two MACs, fp32 accumulate).
//  * V layout: lane (chunk = lane % C, slot = lane / C), C = row bytes / 16, so lanes
//    own disjoint head_dim slices and accumulate P·V with no per-token cross-lane
//    traffic; the token slots are folded once at the end with DPP/permlane swaps.
//
// Numerics follow the reference gather path (core/attention.py:130-153): fp32
// scores and softmax, fp32 accumulation, one rounding of the output to the pool
// dtype. Keys at or beyond context_lens are never loaded.
#include "attention.h"

namespace pkv {
namespace {

constexpr int kBS = 16;
constexpr int kWaves = kDecodePart / 64;  // 64 tokens per wave
constexpr int kTPW = 64;
constexpr int kBPW = kTPW / kBS;          // blocks per wave

template <typename T>
struct Elem;
template <>
struct Elem<float> {
    static constexpr int kPerChunk = 4;
    __device__ __forceinline__ static float get(const Vec16& v, int e) { return __builtin_bit_cast(float, v.w[e]); }
};
template <>
struct Elem<_Float16> {
    static constexpr int kPerChunk = 8;
    __device__ __forceinline__ static float get(const Vec16& v, int e) {
        return (e & 1) ? Pair<_Float16>::hi(v.w[e >> 1]) : Pair<_Float16>::lo(v.w[e >> 1]);
    }
};
template <>
struct Elem<bf16_t> {
    static constexpr int kPerChunk = 8;
    __device__ __forceinline__ static float get(const Vec16& v, int e) {
        return (e & 1) ? Pair<bf16_t>::hi(v.w[e >> 1]) : Pair<bf16_t>::lo(v.w[e >> 1]);
    }
};

// Partial dot product of one 16-byte chunk of K with the matching chunk of q.
template <typename T>
struct ChunkDot {
    __device__ __forceinline__ static float run(const Vec16& k, const Vec16& q, float acc) {
#pragma unroll
        for (int w = 0; w < 4; ++w) acc = Pair<T>::dot2(k.w[w], q.w[w], acc);
        return acc;
    }
};
template <>
struct ChunkDot<float> {
    __device__ __forceinline__ static float run(const Vec16& k, const Vec16& q, float acc) {
#pragma unroll
        for (int w = 0; w < 4; ++w)
            acc = fmaf(__builtin_bit_cast(float, k.w[w]), __builtin_bit_cast(float, q.w[w]), acc);
        return acc;
    }
};

__device__ __forceinline__ int64_t readlane64(int64_t v, int lane) {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)(uint64_t)v, lane);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)v >> 32), lane);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

template <typename T, int D, int G>
__global__ __launch_bounds__(kWaves * 64) void paged_decode_kernel(const AttnParams p) {
    constexpr int ISZ = (int)sizeof(T);
    constexpr int EPC = Elem<T>::kPerChunk;   // elements per 16-byte chunk
    constexpr int CHUNKS = D / EPC;           // chunks per (token, head) row
    constexpr int CPL = CHUNKS / 4;           // K: chunks per lane
    constexpr int TSV = 64 / CHUNKS;          // V: tokens per load step
    constexpr int VSTEPS = kTPW / TSV;        // V: load steps per wave
    static_assert(CHUNKS % 4 == 0 && 64 % CHUNKS == 0 && kBS % TSV == 0, "unsupported head_dim");

    __shared__ float s_p[kWaves][kTPW][G];    // scores, then probabilities
    __shared__ float s_acc[kWaves][G][D];
    __shared__ float s_ml[kWaves][G][2];

    const int kvh = (int)blockIdx.x;
    const int part = (int)blockIdx.y;
    const int seq = (int)blockIdx.z;
    // Memory safety for out-of-contract input: never walk past the table row or the
    // partitions the grid/workspace were sized for (the host guarantees neither
    // bound binds for valid input).
    int64_t ctx64 = p.ctx_lens[seq];
    ctx64 = ctx64 < (int64_t)p.table_width * kBS ? ctx64 : (int64_t)p.table_width * kBS;
    ctx64 = ctx64 < (int64_t)p.max_parts * kDecodePart ? ctx64 : (int64_t)p.max_parts * kDecodePart;
    const int ctx = (int)ctx64;
    const int part_start = part * kDecodePart;
    if (part_start >= ctx) return;
    const int n_parts = (ctx + kDecodePart - 1) / kDecodePart;

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int wstart = part_start + wave * kTPW;  // multiple of 16
    const char* kbase = reinterpret_cast<const char*>(p.k) + (int64_t)kvh * p.sh * ISZ;
    const char* vbase = reinterpret_cast<const char*>(p.v) + (int64_t)kvh * p.sh * ISZ;

    // ------------------------------------------------------------ block ids + q
    // Lane b < kBPW fetches the wave's b-th block id; -1 marks "beyond the context"
    // and ids outside the pool are treated the same way (never dereferenced).
    int64_t my_blk = -1;
    if (lane < kBPW && wstart + lane * kBS < ctx)
        my_blk = p.tables[(int64_t)seq * p.table_stride + wstart / kBS + lane];
    const int quarter = lane & 3;
    const int ktok = lane >> 2;  // token within a block
    Vec16 q[G][CPL];
    {
        const char* qrow = reinterpret_cast<const char*>(p.q) + ((int64_t)seq * p.q_st + (int64_t)kvh * G * p.q_sh) * ISZ;
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < CPL; ++i) q[g][i] = load16(qrow + (int64_t)g * p.q_sh * ISZ + (i * 4 + quarter) * 16);
    }
    int64_t blk[kBPW];
    bool live[kBPW];
#pragma unroll
    for (int b = 0; b < kBPW; ++b) {
        blk[b] = readlane64(my_blk, b);
        live[b] = (uint64_t)blk[b] < (uint64_t)p.num_blocks;
    }

    // ------------------------------------------------------------ K: all blocks in flight
    Vec16 kv[kBPW][CPL];
#pragma unroll
    for (int b = 0; b < kBPW; ++b) {
        if (live[b]) {
            const char* row = kbase + (blk[b] * p.sb + (int64_t)ktok * p.ss) * ISZ;
#pragma unroll
            for (int i = 0; i < CPL; ++i) kv[b][i] = load16(row + (i * 4 + quarter) * 16);
        } else {
#pragma unroll
            for (int i = 0; i < CPL; ++i) kv[b][i] = Vec16{{0u, 0u, 0u, 0u}};
        }
    }
#pragma unroll
    for (int b = 0; b < kBPW; ++b) {
        const int t_rel = b * kBS + ktok;
        const bool valid = live[b] && wstart + t_rel < ctx;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < CPL; ++i) s = ChunkDot<T>::run(kv[b][i], q[g][i], s);
            s = quad_sum(s) * p.scale_log2;
            if ((g & 3) == quarter) s_p[wave][t_rel][g] = valid ? s : kNegInf;
        }
    }

    // ------------------------------------------------------------ V: issue before softmax
    const int vchunk = lane % CHUNKS;
    const int vslot = lane / CHUNKS;
    Vec16 vv[VSTEPS];
#pragma unroll
    for (int st = 0; st < VSTEPS; ++st) {
        const int b = (st * TSV) / kBS;
        const int t_rel = st * TSV + vslot;
        vv[st] = Vec16{{0u, 0u, 0u, 0u}};
        if (live[b] && wstart + t_rel < ctx)
            vv[st] = load16(vbase + (blk[b] * p.sb + (int64_t)(t_rel % kBS) * p.ss) * ISZ + vchunk * 16);
    }
    lds_barrier();

    // ------------------------------------------------------------ softmax (lane = token)
    float m_w[G], l_w[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float a = s_p[wave][lane][g];
        const float m = wave_max(a);
        const float pr = m == kNegInf ? 0.f : fast_exp2(a - m);
        s_p[wave][lane][g] = pr;
        m_w[g] = m;
        l_w[g] = wave_sum(pr);
    }
    lds_barrier();

    // ------------------------------------------------------------ P·V
    float acc[G][EPC];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPC; ++e) acc[g][e] = 0.f;
#pragma unroll
    for (int st = 0; st < VSTEPS; ++st) {
        const int t_rel = st * TSV + vslot;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float pg = s_p[wave][t_rel][g];
#pragma unroll
            for (int e = 0; e < EPC; ++e) acc[g][e] = fmaf(pg, Elem<T>::get(vv[st], e), acc[g][e]);
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPC; ++e) acc[g][e] = fold_lanes<CHUNKS>(acc[g][e]);
    if (vslot == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < EPC; ++e) s_acc[wave][g][vchunk * EPC + e] = acc[g][e];
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            s_ml[wave][g][0] = m_w[g];
            s_ml[wave][g][1] = l_w[g];
        }
    }
    lds_barrier();

    // ------------------------------------------------------------ merge the waves
    const int head0 = kvh * G;
    for (int idx = (int)threadIdx.x; idx < G * D; idx += kWaves * 64) {
        const int g = idx / D, d = idx - g * D;
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_ml[w][g][0]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float mw = s_ml[w][g][0];
            const float sc = mw == kNegInf ? 0.f : fast_exp2(mw - M);
            L += sc * s_ml[w][g][1];
            O += sc * s_acc[w][g][d];
        }
        if (n_parts == 1) {
            T* orow = reinterpret_cast<T*>(p.out) + (int64_t)seq * p.out_st + (int64_t)(head0 + g) * p.out_sh;
            orow[d] = from_f32<T>(O / L);
        } else {
            const int64_t slot = ((int64_t)seq * p.num_heads + head0 + g) * p.max_parts + part;
            p.ws_o[slot * D + d] = O;
            if (d == 0) {
                p.ws_ml[slot * 2] = M;
                p.ws_ml[slot * 2 + 1] = L;
            }
        }
    }
}

// Split-KV merge, launched after paged_decode_kernel on the same stream (stream
// order is the only synchronisation: no fences, no atomics). One workgroup per
// (KV head, sequence) merges the partitions' (max, denominator, output) with the
// log-sum-exp rule; sequences that fit one partition were finished by the first
// kernel and are skipped.
template <typename T, int D, int G>
__global__ __launch_bounds__(256) void paged_decode_combine_kernel(const AttnParams p) {
    const int kvh = (int)blockIdx.x;
    const int seq = (int)blockIdx.y;
    int64_t ctx64 = p.ctx_lens[seq];
    ctx64 = ctx64 < (int64_t)p.table_width * kBS ? ctx64 : (int64_t)p.table_width * kBS;
    ctx64 = ctx64 < (int64_t)p.max_parts * kDecodePart ? ctx64 : (int64_t)p.max_parts * kDecodePart;
    const int n_parts = (int)((ctx64 + kDecodePart - 1) / kDecodePart);
    if (n_parts <= 1) return;
    const int head0 = kvh * G;
    constexpr int CH = 16;  // partitions whose loads are in flight together
    for (int idx = (int)threadIdx.x; idx < G * D; idx += 256) {
        const int g = idx / D, d = idx - g * D;
        const int64_t base = ((int64_t)seq * p.num_heads + head0 + g) * p.max_parts;
        const float2* ml = reinterpret_cast<const float2*>(p.ws_ml) + base;
        const float* o = p.ws_o + base * D + d;
        // Online log-sum-exp over the partitions, CH at a time.
        float M = kNegInf, L = 0.f, O = 0.f;
        for (int pt0 = 0; pt0 < n_parts; pt0 += CH) {
            float2 mlv[CH];
            float ov[CH];
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const bool in = pt0 + j < n_parts;
                mlv[j] = in ? ml[pt0 + j] : make_float2(kNegInf, 0.f);
                ov[j] = in ? o[(int64_t)(pt0 + j) * D] : 0.f;
            }
            float Mc = M;
#pragma unroll
            for (int j = 0; j < CH; ++j) Mc = fmaxf(Mc, mlv[j].x);
            const float rescale = M == kNegInf ? 0.f : fast_exp2(M - Mc);
            L *= rescale;
            O *= rescale;
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const float sc = mlv[j].x == kNegInf ? 0.f : fast_exp2(mlv[j].x - Mc);
                L += sc * mlv[j].y;
                O += sc * ov[j];
            }
            M = Mc;
        }
        T* orow = reinterpret_cast<T*>(p.out) + (int64_t)seq * p.out_st + (int64_t)(head0 + g) * p.out_sh;
        orow[d] = from_f32<T>(O / L);
    }
}

// Instantiated only where the query registers (G * D * itemsize / 64 bytes per lane)
// leave room for the in-flight K loads without spilling: at most 64 VGPRs of query
// per lane. Larger combinations take the generic kernel.
template <typename T, int D, int G>
constexpr bool kDecodeFits = G * D * (int)sizeof(T) <= 1024 && !(sizeof(T) == 4 && D > 64);

template <typename T, int D, int G>
int launch_g(const AttnParams& p, dim3 grid, hipStream_t stream) {
    if constexpr (kDecodeFits<T, D, G>) {
        paged_decode_kernel<T, D, G><<<grid, kWaves * 64, 0, stream>>>(p);
        int rc = check_launch("paged decode attention");
        if (rc || p.max_parts == 1) return rc;
        paged_decode_combine_kernel<T, D, G><<<dim3(grid.x, grid.z), 256, 0, stream>>>(p);
        return check_launch("paged decode combine");
    }
    return PKV_EUNSUPPORTED;
}

template <typename T, int D>
int launch_d(const AttnParams& p, dim3 grid, hipStream_t stream) {
    switch (p.group) {
        case 1: return launch_g<T, D, 1>(p, grid, stream);
        case 2: return launch_g<T, D, 2>(p, grid, stream);
        case 4: return launch_g<T, D, 4>(p, grid, stream);
        case 8: return launch_g<T, D, 8>(p, grid, stream);
        default: return PKV_EUNSUPPORTED;
    }
}

template <typename T>
int launch_t(const AttnParams& p, dim3 grid, hipStream_t stream) {
    if (p.head_dim == 64) return launch_d<T, 64>(p, grid, stream);
    if (p.head_dim == 128) return launch_d<T, 128>(p, grid, stream);
    return PKV_EUNSUPPORTED;
}

}  // namespace

int launch_decode_attention(const AttnParams& p, int dtype, hipStream_t stream) {
    if (p.block_size != kBS) return PKV_EUNSUPPORTED;
    if (p.group != 1 && p.group != 2 && p.group != 4 && p.group != 8) return PKV_EUNSUPPORTED;
    if (p.head_dim != 64 && p.head_dim != 128) return PKV_EUNSUPPORTED;
    if (p.num_kv_heads > 65535 || p.max_parts > 65535 || p.num_seqs > 65535) return PKV_EUNSUPPORTED;
    if (p.max_parts > 1 && (!p.ws_o || !p.ws_ml)) return PKV_EUNSUPPORTED;
    // 16-byte chunk loads need 16-byte aligned rows.
    const int isz = dtype == PKV_FLOAT32 ? 4 : 2;
    const uint64_t probe = (uint64_t)(uintptr_t)p.q | (uint64_t)(uintptr_t)p.k | (uint64_t)(uintptr_t)p.v |
                           (uint64_t)(p.q_st * isz) | (uint64_t)(p.q_sh * isz) | (uint64_t)(p.sb * isz) |
                           (uint64_t)(p.ss * isz) | (uint64_t)(p.sh * isz);
    if (probe % 16) return PKV_EUNSUPPORTED;
    if (p.num_seqs == 0) return PKV_OK;
    dim3 grid((unsigned)p.num_kv_heads, (unsigned)p.max_parts, (unsigned)p.num_seqs);
    switch (dtype) {
        case PKV_FLOAT32: return launch_t<float>(p, grid, stream);
        case PKV_FLOAT16: return launch_t<_Float16>(p, grid, stream);
        case PKV_BFLOAT16: return launch_t<bf16_t>(p, grid, stream);
    }
    return PKV_EUNSUPPORTED;
}

}  // namespace pkv
