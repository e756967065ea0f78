// Tuned paged decode attention for block_size 16, head_dim 64/128, GQA group
// 1/2/4/8, fp16/bf16/fp32.
//
// Single-query decode is a bandwidth-bound GEMV: every K/V byte of the context is
// read once and used for 2*G flops per element, where G = num_heads / num_kv_heads.
// The kernel is therefore organised around HBM traffic, not arithmetic:
//
//  * Work unit = (KV head, 512-token partition, sequence): one 256-thread workgroup
//    (4 wave64s, 128 tokens each). All G query heads of the GQA group are served by
//    the same K/V read, so K/V are fetched once per KV head, never once per query
//    head (the reference's design re-reads them G times, core/attention_triton.py:181).
//  * Split-KV: long contexts are cut into partitions so the grid has thousands of
//    workgroups to spread over 256 CUs. Partials (max, denominator, unnormalised
//    output) are merged with the log-sum-exp rule by the LAST workgroup of each
//    (sequence, KV head) to finish — an arrival counter in the workspace — so one
//    launch produces the final output and no combine kernel is needed.
//  * K phase: lane (token = lane/4, quarter = lane%4) loads 16-byte chunks
//    quarter, quarter+4, ... of its token's K row; a wave covers one 16-token block
//    per step with fully used 64-byte segments, and a quad DPP reduction finishes
//    each score. fp16/bf16 dot products use v_dot2_f32_{f16,bf16} (two MACs, fp32
//    accumulate). Scores go to LDS.
//  * Softmax over the wave's 128 scores in LDS (fp32, base-2 domain).
//  * V phase: lane (chunk = lane % C, slot = lane / C), C = row bytes / 16, so lanes
//    own disjoint head_dim slices and accumulate P·V with no per-token cross-lane
//    traffic; the token slots are folded once at the end.
//  * Loads are batched (16 outstanding 16-byte loads per lane) so each CU keeps well
//    over 100 KB in flight, what HBM3E needs to approach its 8 TB/s peak.
//
// Numerics follow the reference gather path (core/attention.py:130-153): fp32
// scores and softmax, fp32 accumulation, one rounding of the output to the pool
// dtype. Keys at or beyond context_lens are never loaded.
#include "attention.h"

namespace pkv {
namespace {

constexpr int kBS = 16;
constexpr int kWaves = 4;
constexpr int kTPW = kDecodePart / kWaves;  // tokens per wave

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

template <typename T, int D, int G>
__global__ __launch_bounds__(256, 2) void paged_decode_kernel(const AttnParams p) {
    constexpr int ISZ = (int)sizeof(T);
    constexpr int EPC = Elem<T>::kPerChunk;   // elements per 16-byte chunk
    constexpr int CHUNKS = D / EPC;           // chunks per (token, head) row
    constexpr int CPL = CHUNKS / 4;           // K phase: chunks per lane
    constexpr int KSTEPS = kTPW / kBS;        // K phase: one block per step
    constexpr int KU = (16 / CPL) < KSTEPS ? (16 / CPL) : KSTEPS;
    constexpr int TSV = 64 / CHUNKS;          // V phase: tokens per step
    constexpr int VSTEPS = kTPW / TSV;
    constexpr int VU = 16 < VSTEPS ? 16 : VSTEPS;
    static_assert(CHUNKS % 4 == 0 && 64 % CHUNKS == 0 && kBS % TSV == 0, "unsupported head_dim");
    static_assert(KSTEPS % KU == 0 && VSTEPS % VU == 0, "step batching");

    __shared__ float s_p[kWaves][kTPW][G];    // scores, then probabilities
    __shared__ float s_acc[kWaves][G][D];
    __shared__ float s_ml[kWaves][G][2];
    __shared__ int s_last;

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
    const int64_t* table = p.tables + (int64_t)seq * p.table_stride;
    const char* kbase = reinterpret_cast<const char*>(p.k) + (int64_t)kvh * p.sh * ISZ;
    const char* vbase = reinterpret_cast<const char*>(p.v) + (int64_t)kvh * p.sh * ISZ;

    // ---------------------------------------------------------------- K phase
    const int quarter = lane & 3;
    const int ktok = lane >> 2;  // token within the step's block
    Vec16 q[G][CPL];
    {
        const char* qrow = reinterpret_cast<const char*>(p.q) + ((int64_t)seq * p.q_st + (int64_t)kvh * G * p.q_sh) * ISZ;
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < CPL; ++i) q[g][i] = load16(qrow + (int64_t)g * p.q_sh * ISZ + (i * 4 + quarter) * 16);
    }

#pragma unroll
    for (int ks0 = 0; ks0 < KSTEPS; ks0 += KU) {
        Vec16 kv[KU][CPL];
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const int bstart = wstart + (ks0 + u) * kBS;
            const int64_t blk = bstart < ctx ? table[bstart / kBS] : -1;
            if ((uint64_t)blk < (uint64_t)p.num_blocks) {
                const char* row = kbase + (blk * p.sb + (int64_t)ktok * p.ss) * ISZ;
#pragma unroll
                for (int i = 0; i < CPL; ++i) kv[u][i] = load16(row + (i * 4 + quarter) * 16);
            } else {
#pragma unroll
                for (int i = 0; i < CPL; ++i) kv[u][i] = Vec16{{0u, 0u, 0u, 0u}};
            }
        }
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const int t_rel = (ks0 + u) * kBS + ktok;
            const bool valid = wstart + t_rel < ctx;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float s = 0.f;
#pragma unroll
                for (int i = 0; i < CPL; ++i) s = ChunkDot<T>::run(kv[u][i], q[g][i], s);
                s = quad_sum(s) * p.scale_log2;
                if ((g & 3) == quarter) s_p[wave][t_rel][g] = valid ? s : kNegInf;
            }
        }
    }
    __syncthreads();

    // ---------------------------------------------------------------- softmax
    float m_w[G], l_w[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float a0 = s_p[wave][lane][g];
        const float a1 = s_p[wave][lane + 64][g];
        const float m = wave_max(fmaxf(a0, a1));
        const float p0 = m == kNegInf ? 0.f : fast_exp2(a0 - m);
        const float p1 = m == kNegInf ? 0.f : fast_exp2(a1 - m);
        s_p[wave][lane][g] = p0;
        s_p[wave][lane + 64][g] = p1;
        m_w[g] = m;
        l_w[g] = wave_sum(p0 + p1);
    }
    __syncthreads();

    // ---------------------------------------------------------------- V phase
    const int vchunk = lane % CHUNKS;
    const int vslot = lane / CHUNKS;
    float acc[G][EPC];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPC; ++e) acc[g][e] = 0.f;

#pragma unroll
    for (int vs0 = 0; vs0 < VSTEPS; vs0 += VU) {
        Vec16 vv[VU];
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int sstart = wstart + (vs0 + u) * TSV;  // first token of the step
            const int tok = sstart + vslot;
            vv[u] = Vec16{{0u, 0u, 0u, 0u}};
            const int64_t blk = sstart < ctx ? table[sstart / kBS] : -1;
            if ((uint64_t)blk < (uint64_t)p.num_blocks) {
                if (tok < ctx)
                    vv[u] = load16(vbase + (blk * p.sb + (int64_t)(tok % kBS) * p.ss) * ISZ + vchunk * 16);
            }
        }
#pragma unroll
        for (int u = 0; u < VU; ++u) {
            const int t_rel = (vs0 + u) * TSV + vslot;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float pg = s_p[wave][t_rel][g];
#pragma unroll
                for (int e = 0; e < EPC; ++e) acc[g][e] = fmaf(pg, Elem<T>::get(vv[u], e), acc[g][e]);
            }
        }
    }
    // Fold the token slots: lanes with equal vchunk hold partial sums of one slice.
#pragma unroll
    for (int msk = CHUNKS; msk < 64; msk <<= 1)
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < EPC; ++e) acc[g][e] += shfl_xor_f32(acc[g][e], msk);
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
    __syncthreads();

    // ---------------------------------------------------------------- merge waves
    const int head0 = kvh * G;
    for (int idx = (int)threadIdx.x; idx < G * D; idx += 256) {
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
    if (n_parts == 1) return;

    // ---------------------------------------------------------------- split-KV merge
    // Release this partition's partials, count arrivals; the last arrival merges.
    __threadfence();
    __syncthreads();
    int* counter = p.ws_cnt + (int64_t)seq * p.num_kv_heads + kvh;
    if (threadIdx.x == 0) s_last = atomicAdd(counter, 1) == n_parts - 1;
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int idx = (int)threadIdx.x; idx < G * D; idx += 256) {
        const int g = idx / D, d = idx - g * D;
        const int64_t base = ((int64_t)seq * p.num_heads + head0 + g) * p.max_parts;
        float M = kNegInf;
        for (int pt = 0; pt < n_parts; ++pt) M = fmaxf(M, p.ws_ml[(base + pt) * 2]);
        float L = 0.f, O = 0.f;
        for (int pt = 0; pt < n_parts; ++pt) {
            const float sc = fast_exp2(p.ws_ml[(base + pt) * 2] - M);
            L += sc * p.ws_ml[(base + pt) * 2 + 1];
            O += sc * p.ws_o[(base + pt) * D + d];
        }
        T* orow = reinterpret_cast<T*>(p.out) + (int64_t)seq * p.out_st + (int64_t)(head0 + g) * p.out_sh;
        orow[d] = from_f32<T>(O / L);
    }
    if (threadIdx.x == 0) *counter = 0;  // ready for the next call on this workspace
}

// Instantiated only where the query registers (G * D * itemsize / 64 bytes per lane)
// leave room for 16 outstanding 16-byte loads without spilling: at most 64 VGPRs of
// query per lane. Larger combinations take the generic kernel.
template <typename T, int D, int G>
constexpr bool kDecodeFits = G * D * (int)sizeof(T) <= 1024 && !(sizeof(T) == 4 && D > 64);

template <typename T, int D, int G>
int launch_g(const AttnParams& p, dim3 grid, hipStream_t stream) {
    if constexpr (kDecodeFits<T, D, G>) {
        paged_decode_kernel<T, D, G><<<grid, 256, 0, stream>>>(p);
        return check_launch("paged decode attention");
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
