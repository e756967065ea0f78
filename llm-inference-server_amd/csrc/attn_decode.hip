// Tuned paged decode attention for block_size 16, head_dim 64/128, GQA group
// 1/2/4/8. Two partition kernels and a split-KV merge kernel:
//   paged_decode_stream_kernel (fp16/bf16, further down): K/V stream HBM -> LDS by
//     DMA through a per-wave ring, so every wave keeps its next chunk in flight;
//   paged_decode_kernel (fp32, and any 16-bit call on an empty pool): K/V staged in
//     registers, described first.
//
// Single-query decode is a bandwidth-bound GEMV: every K/V byte of the context is
// read once and used for 2*G flops per element, where G = num_heads / num_kv_heads.
// The kernels are therefore organised around HBM traffic and latency, not arithmetic:
//
//  * Work unit = (KV head, 256-token partition, sequence): one 256-thread workgroup
//    of 4 wave64s, 64 tokens (4 blocks) per wave. All G query heads of the GQA group
//    are served by the same K/V read, so K/V are fetched once per KV head, never once
//    per query head (the reference's kernel design re-reads them G times,
//    core/attention_triton.py:181).
//  * Latency chain per wave: ONE vector load of the wave's 4 block-table entries
//    (broadcast with readlane), then all K loads of the 4 blocks at once, the scores,
//    then all V loads at once — issued before the softmax so they are in flight while
//    it runs. No load waits on another load except through the block table. Block
//    bases live in SGPRs and lane offsets are 32-bit, so every load is a
//    `global_load ... saddr` with no per-lane 64-bit address arithmetic.
//  * Split-KV: contexts are cut into partitions so the grid has thousands of
//    workgroups for 256 CUs. A sequence that fits one partition is finished in
//    place; otherwise each partition writes its partial (max, denominator,
//    unnormalised output) and the partials are merged with the log-sum-exp rule:
//    by the streaming kernel's last partition of each (sequence, KV head) to finish
//    (agent-scope partial stores, a completion wait and one relaxed atomic counter per
//    pair; no agent-scope fence, which writes back the XCD's L2 and was measured to
//    serialise the whole launch), or by a small second kernel on the same stream (the
//    register kernel, and streaming launches of few long (sequence, KV head) pairs).
//  * K layout: lane (token = lane / 8, j = lane % 8) holds 16-byte chunks j, j + 8,
//    ... of its token's K row, so each load instruction reads 8 tokens x one whole
//    128-byte line; a 3-step DPP reduction over the 8 lanes finishes each score.
//    fp16/bf16 dot products use v_dot2_f32_{f16,bf16} (two MACs, fp32 accumulate).
//  * V layout: lane (chunk = lane % C, slot = lane / C), C = row bytes / 8, so lanes
//    own disjoint 8-byte head_dim slices and accumulate P·V with no per-token
//    cross-lane traffic. For fp16/bf16, two tokens' values of one element are packed
//    into one register and multiplied by the packed pair of their probabilities with
//    v_dot2 (probabilities rounded to the pool dtype first, as the reference's
//    `softmax(...).to(v.dtype)` rounds them before its P·V matmul,
//    core/attention.py:152). The token slots are folded once at the end with permlane
//    swaps.
//
// Numerics against the reference gather path (core/attention.py:130-153):
//  * scores are rounded where the gather path rounds them: q·k (fp32 dot products)
//    rounded to the pool dtype, as the matmul's output tensor is, then times scale and
//    rounded again, as `* scale` on that tensor is (ref_score_log2);
//  * the softmax runs in fp32 on those scores, as softmax(dtype=float32) does;
//  * the reference rounds the NORMALISED probabilities exp(s - max) / sum to the pool
//    dtype; a streaming kernel does not know the global max and sum while it reads V,
//    so here the rounded weights are exp(s - m) against the running max m of the
//    partition, and the division by the sum (and the rescale between partitions)
//    happens in fp32 afterwards. Each weight is still rounded once to the pool dtype,
//    so the two differ by that rounding (half an ulp of the pool dtype per weight),
//    not by its size; outputs are checked against oracle.gather at 2e-2 (fp16/bf16);
//  * P·V accumulates in fp32 and the output is rounded once to the pool dtype.
// Keys at or beyond context_lens are never loaded.
#include <type_traits>

#include "attention.h"

namespace pkv {
namespace {

constexpr int kBS = 16;
constexpr int kWaves = kDecodePart / 64;  // 64 tokens per wave
constexpr int kTPW = 64;
constexpr int kBPW = kTPW / kBS;          // blocks per wave

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

// Two probabilities packed (round to nearest even) into the 16-bit pool dtype.
template <typename T>
__device__ __forceinline__ uint32_t pack_probs(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack_probs<bf16_t>(float lo, float hi) {
    bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}
template <>
__device__ __forceinline__ uint32_t pack_probs<_Float16>(float lo, float hi) {
    half2_t v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// K/V rows are read exactly once per launch: streaming loads (config 4: 5.02 TB/s
// with them, 4.80 TB/s with cached loads).
__device__ __forceinline__ Vec16 kv_load16(const void* ptr) { return load16_stream(ptr); }
__device__ __forceinline__ uint2 kv_load8(const void* ptr) { return load8_stream(ptr); }
// Cache-policy operand of global_load_lds for the same streaming data: nontemporal.
constexpr int kDmaNontemporal = 2;

template <typename T, int D, int G>
__global__ __launch_bounds__(kWaves * 64) void paged_decode_kernel(const AttnParams p) {
    constexpr int ISZ = (int)sizeof(T);
    constexpr int CHUNKS = D * ISZ / 16;      // K: 16-byte chunks per (token, head) row
    constexpr int KLPT = 8;                   // K: lanes per token (8 x 16 B = one 128-byte line)
    constexpr int CPL = CHUNKS / KLPT;        // K: chunks per lane
    constexpr int KGRP = kBS * KLPT / 64;     // K: load groups per block (8 tokens each)
    constexpr int EPV = 8 / ISZ;              // V: elements per 8-byte chunk
    constexpr int VLPT = D * ISZ / 8;         // V: lanes per token
    constexpr int TSV = 64 / VLPT;            // V: tokens per load step
    constexpr int VSTEPS = kTPW / TSV;        // V: load steps per wave
    constexpr bool kPacked = ISZ == 2;        // fp16/bf16: P·V through v_dot2
    static_assert(CHUNKS % KLPT == 0 && G <= KLPT && 64 % VLPT == 0 && kBS % TSV == 0 && VSTEPS % 2 == 0,
                  "unsupported head_dim / group");

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
    const uint32_t slot_bytes = (uint32_t)(p.ss * ISZ);
    const int64_t block_bytes = p.sb * ISZ;

    // ------------------------------------------------------------ block ids + q
    // Lane b < kBPW fetches the wave's b-th block id; -1 marks "beyond the context"
    // and ids outside the pool are treated the same way (never dereferenced).
    int64_t my_blk = -1;
    if (lane < kBPW && wstart + lane * kBS < ctx)
        my_blk = p.tables[(int64_t)seq * p.table_stride + wstart / kBS + lane];
    const int kj = lane % KLPT;   // which 16-byte chunks of the row: kj, kj + 8, ...
    const int ktok = lane / KLPT; // token within a load group
    Vec16 q[G][CPL];
    {
        const char* qrow = reinterpret_cast<const char*>(p.q) + ((int64_t)seq * p.q_st + (int64_t)kvh * G * p.q_sh) * ISZ;
        const uint32_t q_head_bytes = (uint32_t)(p.q_sh * ISZ);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < CPL; ++i) q[g][i] = load16(qrow + (g * q_head_bytes + (uint32_t)((i * KLPT + kj) * 16)));
    }
    const char* kblk[kBPW];
    const char* vblk[kBPW];
    bool live[kBPW];
#pragma unroll
    for (int b = 0; b < kBPW; ++b) {
        const int64_t id = readlane64(my_blk, b);
        live[b] = (uint64_t)id < (uint64_t)p.num_blocks;
        kblk[b] = kbase + id * block_bytes;
        vblk[b] = vbase + id * block_bytes;
    }

    // ------------------------------------------------------------ K, scores, V issue
    // Fast path (wave-uniform): all 64 tokens inside the context and all 4 block ids
    // inside the pool. Its loads are unconditional and nothing is zero-filled; the other
    // waves (at most the last two of a sequence) predicate every load and zero what they
    // skip, which costs ~15% more VALU instructions.
    bool full = wstart + kTPW <= ctx;
#pragma unroll
    for (int b = 0; b < kBPW; ++b) full = full && live[b];
    // K: each load instruction reads 8 tokens x one whole 128-byte line of their rows.
    const uint32_t k_lane_off = ktok * slot_bytes + (uint32_t)(kj * 16);
    const int vchunk = lane % VLPT;
    const int vslot = lane / VLPT;
    Vec16 kv[kBPW][KGRP][CPL];
    uint2 vv[VSTEPS];
    auto stream = [&](auto full_tag) {
        constexpr bool FULL = decltype(full_tag)::value;
#pragma unroll
        for (int b = 0; b < kBPW; ++b)
#pragma unroll
            for (int gr = 0; gr < KGRP; ++gr) {
                if (FULL || live[b]) {
#pragma unroll
                    for (int i = 0; i < CPL; ++i)
                        kv[b][gr][i] = kv_load16(kblk[b] + (k_lane_off + (uint32_t)(gr * 8) * slot_bytes +
                                                            (uint32_t)(i * KLPT * 16)));
                } else {
#pragma unroll
                    for (int i = 0; i < CPL; ++i) kv[b][gr][i] = Vec16{{0u, 0u, 0u, 0u}};
                }
            }
#pragma unroll
        for (int b = 0; b < kBPW; ++b)
#pragma unroll
            for (int gr = 0; gr < KGRP; ++gr) {
                const int t_rel = b * kBS + gr * 8 + ktok;
                const bool valid = FULL || (live[b] && wstart + t_rel < ctx);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    float s = 0.f;
#pragma unroll
                    for (int i = 0; i < CPL; ++i) s = ChunkDot<T>::run(kv[b][gr][i], q[g][i], s);
                    s = ref_score_log2<T>(octet_sum(s), p.scale);
                    if (g == kj) s_p[wave][t_rel][g] = valid ? s : kNegInf;
                }
            }
        // V: issued before the softmax so the loads are in flight while it runs.
#pragma unroll
        for (int st = 0; st < VSTEPS; ++st) {
            const int b = (st * TSV) / kBS;
            const int t_rel = st * TSV + vslot;
            const uint32_t off = (uint32_t)(t_rel % kBS) * slot_bytes + (uint32_t)(vchunk * 8);
            if (FULL) {
                vv[st] = kv_load8(vblk[b] + off);
            } else {
                vv[st] = make_uint2(0u, 0u);
                if (live[b] && wstart + t_rel < ctx) vv[st] = kv_load8(vblk[b] + off);
            }
        }
    };
    if (full) stream(std::true_type{});
    else stream(std::false_type{});
    // Scores, softmax and P·V stay inside the wave's own slice of s_p, so the waves only
    // order their own LDS traffic here; the workgroup meets once, at the merge.
    wave_lds_sync();

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
    wave_lds_sync();

    // ------------------------------------------------------------ P·V
    float acc[G][EPV];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPV; ++e) acc[g][e] = 0.f;
    if constexpr (kPacked) {
#pragma unroll
        for (int st = 0; st < VSTEPS; st += 2) {
            const int t0 = st * TSV + vslot;
            const int t1 = t0 + TSV;
            // (token t0, token t1) values of each element, packed for v_dot2.
            uint32_t vp[EPV];
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                const uint32_t a = w ? vv[st].y : vv[st].x;
                const uint32_t c = w ? vv[st + 1].y : vv[st + 1].x;
                // One v_perm_b32 each: bytes {a.0, a.1, c.0, c.1} and {a.2, a.3, c.2, c.3}.
                vp[2 * w] = __builtin_amdgcn_perm(c, a, 0x05040100u);
                vp[2 * w + 1] = __builtin_amdgcn_perm(c, a, 0x07060302u);
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const uint32_t pp = pack_probs<T>(s_p[wave][t0][g], s_p[wave][t1][g]);
#pragma unroll
                for (int e = 0; e < EPV; ++e) acc[g][e] = Pair<T>::dot2(vp[e], pp, acc[g][e]);
            }
        }
    } else {
#pragma unroll
        for (int st = 0; st < VSTEPS; ++st) {
            const int t_rel = st * TSV + vslot;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float pg = s_p[wave][t_rel][g];
                acc[g][0] = fmaf(pg, __builtin_bit_cast(float, vv[st].x), acc[g][0]);
                acc[g][1] = fmaf(pg, __builtin_bit_cast(float, vv[st].y), acc[g][1]);
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPV; ++e) acc[g][e] = fold_lanes<VLPT>(acc[g][e]);
    if (vslot == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < EPV; ++e) s_acc[wave][g][vchunk * EPV + e] = acc[g][e];
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

// Split-KV merge, launched after the partition kernel on the same stream (stream
// order is the only synchronisation: no fences, no atomics). One workgroup per
// (KV head, sequence) merges the partitions' (max, denominator, output) with the
// log-sum-exp rule; sequences that fit one PART-token partition were finished by the
// partition kernel and are skipped.
// Threads of a merge workgroup: the G * D / 2 element pairs of one KV head, in whole
// waves, at most 256 (one wave for a head_dim-64 group of one).
template <int G, int D>
constexpr int kCombineThreads = (G * D / 2 + 63) / 64 * 64 < 256 ? (G * D / 2 + 63) / 64 * 64 : 256;

template <typename T, int D, int G, int PART>
__global__ __launch_bounds__((kCombineThreads<G, D>)) void paged_decode_combine_kernel(const AttnParams p) {
    const int kvh = (int)blockIdx.x;
    const int seq = (int)blockIdx.y;
    int64_t ctx64 = p.ctx_lens[seq];
    ctx64 = ctx64 < (int64_t)p.table_width * kBS ? ctx64 : (int64_t)p.table_width * kBS;
    ctx64 = ctx64 < (int64_t)p.max_parts * kDecodePart ? ctx64 : (int64_t)p.max_parts * kDecodePart;
    const int n_parts = (int)((ctx64 + PART - 1) / PART);
    if (n_parts <= 1) return;
    const int head0 = kvh * G;
    constexpr int CH = 16;  // partitions whose loads are in flight together
    static_assert(D % 2 == 0, "pairs of head_dim elements");
    // Each thread merges two adjacent head_dim elements (8-byte loads), so G * D <= 512
    // (every shape the partition kernels take) is one pass of dependent loads.
    for (int idx = (int)threadIdx.x; idx < G * D / 2; idx += kCombineThreads<G, D>) {
        const int g = (2 * idx) / D, d = 2 * idx - g * D;
        const int64_t base = ((int64_t)seq * p.num_heads + head0 + g) * p.max_parts;
        const float2* ml = reinterpret_cast<const float2*>(p.ws_ml) + base;
        const float2* o = reinterpret_cast<const float2*>(p.ws_o + base * D + d);
        // Online log-sum-exp over the partitions, CH at a time.
        float M = kNegInf, L = 0.f, O0 = 0.f, O1 = 0.f;
        for (int pt0 = 0; pt0 < n_parts; pt0 += CH) {
            float2 mlv[CH], ov[CH];
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const bool in = pt0 + j < n_parts;
                mlv[j] = in ? ml[pt0 + j] : make_float2(kNegInf, 0.f);
                ov[j] = in ? o[(int64_t)(pt0 + j) * (D / 2)] : make_float2(0.f, 0.f);
            }
            float Mc = M;
#pragma unroll
            for (int j = 0; j < CH; ++j) Mc = fmaxf(Mc, mlv[j].x);
            const float rescale = M == kNegInf ? 0.f : fast_exp2(M - Mc);
            L *= rescale;
            O0 *= rescale;
            O1 *= rescale;
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const float sc = mlv[j].x == kNegInf ? 0.f : fast_exp2(mlv[j].x - Mc);
                L += sc * mlv[j].y;
                O0 += sc * ov[j].x;
                O1 += sc * ov[j].y;
            }
            M = Mc;
        }
        T* orow = reinterpret_cast<T*>(p.out) + (int64_t)seq * p.out_st + (int64_t)(head0 + g) * p.out_sh;
        orow[d] = from_f32<T>(O0 / L);
        orow[d + 1] = from_f32<T>(O1 / L);
    }
}

// Context length of `seq` clamped like the kernels above: never past the table row or
// the partitions the workspace was sized for (neither binds for valid input).
__device__ __forceinline__ int clamped_ctx(const AttnParams& p, int seq) {
    int64_t c = p.ctx_lens[seq];
    c = c < (int64_t)p.table_width * kBS ? c : (int64_t)p.table_width * kBS;
    c = c < (int64_t)p.max_parts * kDecodePart ? c : (int64_t)p.max_parts * kDecodePart;
    return (int)c;
}

// ============================================================ streaming decode (fp16/bf16)
//
// The 16-bit pools take this kernel instead of the one above. Its waves stream their
// K/V through LDS instead of registers, so each keeps its next block in flight while
// it computes the current one:
//
//  * Work unit = (KV head, 768-token partition, sequence), 4 waves; wave w owns tokens
//    [192 w, 192 w + 192) of the partition as 24 chunks of 8 tokens (half a block);
//    grouped heads whose merge runs in this kernel use 8 waves x 96 tokens instead.
//    Launches that take 256-token partitions (below) run 8 waves x 32 tokens or 4 x 64.
//  * Each wave has a private two-buffer ring in LDS. A chunk's K and V rows move
//    HBM -> LDS by DMA (global_load_lds_dwordx4, nontemporal); the DMA of chunk c + 2
//    is issued as soon as chunk c is done, so one chunk is always in flight while the
//    other is computed. No registers hold in-flight data and no workgroup barrier is
//    needed until the final merge. (The register-staged kernel holds 16 KB per wave in VGPRs for one
//    phase at a time; counters showed it keeping ~10 KB of reads in flight per CU where
//    a plain read stream of the same pattern keeps ~15 KB and runs 25% faster.)
//  * Online softmax across the chunks, per head, with the per-head state in the lanes
//    of one 8-lane group (group-local DPP reductions); the probabilities of token pairs
//    (t, t + TSV) are stored next to each other so P·V reads each pair with one load.
//  * Scores and P·V use the same lane layouts and v_dot2 arithmetic as the kernel
//    above (K: 8 lanes per token; V: lanes own 8-byte head_dim slices, two tokens'
//    values packed against their two probabilities), so the numerics are identical.
// Partition size: a template parameter, 768 or 256 tokens. Sweep on config 4 (GB/s,
// 8-token chunks): 256 -> 5084, 512 -> 5340, 640 -> 5462, 768 -> 5399-5471, 896 ->
// 5336, 1024 -> 5320: longer partitions amortise a workgroup's start and merge. A wave
// walks its quarter of the partition as a chain of dependent chunk DMAs, so on short
// contexts (batches that cannot fill the GPU with long partitions) 768 leaves a few
// long chains where 256 has many short ones; the launch picks per call.
constexpr int kSPartLong = 768;
constexpr int kSPartShort = 256;
constexpr int kSCT = 8;                      // tokens per chunk (half a block)

// K rows in LDS are stored with their two 128-byte halves swapped on odd rows (D = 128)
// so the 2 rows x 8 chunks of a 16-lane b128 read hit distinct banks; D = 64 rows are
// 128 bytes and need no swizzle.
template <int D>
__device__ __forceinline__ int stream_kswz(int r) {
    return D == 128 ? 8 * (r & 1) : 0;
}

// kSCT rows of one KV head, K and V, HBM -> LDS by DMA (global_load_lds_dwordx4: lane
// i's 16 bytes land at the instruction's LDS base + 16 i). `kblock`/`vblock` point at
// the chunk's first row; rows >= `rows` re-read that row (a valid token). K rows are
// stored swizzled (stream_kswz).
template <int D>
__device__ __forceinline__ void stream_dma_chunk(const char* kblock, const char* vblock, int64_t slot_bytes, int rows,
                                                 int dma_row, int dma_slot, uint16_t* dk, uint16_t* dv) {
    constexpr int ROWB = D * 2;
    constexpr int RPI = 1024 / ROWB;
    static_assert(kSCT % RPI == 0, "chunk must be whole DMA instructions");
#pragma unroll
    for (int j = 0; j < kSCT / RPI; ++j) {
        const int r = j * RPI + dma_row;
        const int64_t row = (int64_t)(r < rows ? r : 0) * slot_bytes;
        // (Offsets computed outside the builtin's argument list: a device-function call
        // inside it makes clang's host pass drop this kernel's launch stub silently.)
        const char* ksrc = kblock + row + ((dma_slot ^ stream_kswz<D>(r)) << 4);
        const char* vsrc = vblock + row + (dma_slot << 4);
        __builtin_amdgcn_global_load_lds(ksrc, (__attribute__((address_space(3))) void*)((char*)dk + j * RPI * ROWB),
                                         16, 0, kDmaNontemporal);
        __builtin_amdgcn_global_load_lds(vsrc, (__attribute__((address_space(3))) void*)((char*)dv + j * RPI * ROWB),
                                         16, 0, kDmaNontemporal);
    }
}

// Max / sum over each aligned group of R lanes (R = 8 or 16; every lane gets its
// group's result).
template <int R>
__device__ __forceinline__ float group_max(float x) {
    x = fmaxf(x, dpp_f32<kDppQuadXor1>(x));
    x = fmaxf(x, dpp_f32<kDppQuadXor2>(x));
    x = fmaxf(x, dpp_f32<kDppRowHalfMirror>(x));
    if constexpr (R == 16) x = fmaxf(x, dpp_f32<kDppRowMirror>(x));
    return x;
}
template <int R>
__device__ __forceinline__ float group_sum(float x) {
    x = octet_sum(x);
    if constexpr (R == 16) x += dpp_f32<kDppRowMirror>(x);
    return x;
}

template <typename T, int D, int G, int PART, int W>
__global__ __launch_bounds__(W * 64) void paged_decode_stream_kernel(const AttnParams p) {
    constexpr int kSSlice = PART / W;         // tokens per wave
    // PART >= the workspace's 256-token partition: never more partials than it holds.
    // A wave's block ids live one per lane: at most 64 blocks per wave.
    static_assert(kSSlice % kSCT == 0 && PART >= kDecodePart && kSSlice <= 64 * kBS, "partition shape");
    constexpr int ISZ = 2;
    constexpr int ROWB = D * ISZ;             // bytes per (token, head) row
    constexpr int CPR = ROWB / 16;            // 16-byte chunks per row
    constexpr int KLPT = 8;                   // K: lanes per token
    constexpr int CPL = CPR / KLPT;           // K: 16-byte chunks per lane
    constexpr int KROUNDS = kSCT * KLPT / 64; // K: 8-token rounds per chunk
    constexpr int EPV = 8 / ISZ;              // V: elements per 8-byte slice
    constexpr int VLPT = ROWB / 8;            // V: lanes per token
    constexpr int TSV = 64 / VLPT;            // V: tokens per step
    constexpr int VSTEPS = kSCT / TSV;        // V: steps per chunk
    constexpr int HPR = 64 / kSCT;            // softmax: heads per 64-lane round
    constexpr int SROUNDS = (G + HPR - 1) / HPR;
    static_assert(CPR % KLPT == 0 && G <= KLPT && KROUNDS >= 1 && VSTEPS % 2 == 0 && kSCT % TSV == 0,
                  "unsupported head_dim / group");
    // The merge writes a wave's [G][D] fp32 partial output over its own s_b0 slice.
    static_assert(G * D * 4 <= 2 * kSCT * D * ISZ, "partial output must fit a wave's s_b0 slice");

    // The two ring buffers are distinct objects (the waits on their DMAs are explicit).
    __shared__ __attribute__((aligned(1024))) uint16_t s_b0[W][2][kSCT * D];
    __shared__ __attribute__((aligned(1024))) uint16_t s_b1[W][2][kSCT * D];
    __shared__ float s_sc[W][G][kSCT];  // chunk scores, then probabilities
    __shared__ float s_ml[W][G][2];     // per-wave (max, denominator) for the merge

    const int kvh = (int)blockIdx.x;
    const int part = (int)blockIdx.y;
    const int seq = (int)blockIdx.z;
    const int ctx = clamped_ctx(p, seq);
    const int part_start = part * PART;
    if (part_start >= ctx) return;
    const int n_parts = (ctx + PART - 1) / PART;

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int wstart = part_start + wave * kSSlice;
    int wtok = ctx - wstart;                  // tokens of this wave inside the context
    wtok = wtok < 0 ? 0 : (wtok > kSSlice ? kSSlice : wtok);
    const int nchunk = (wtok + kSCT - 1) / kSCT;
    const char* kbase = reinterpret_cast<const char*>(p.k) + (int64_t)kvh * p.sh * ISZ;
    const char* vbase = reinterpret_cast<const char*>(p.v) + (int64_t)kvh * p.sh * ISZ;
    const int64_t slot_bytes = p.ss * ISZ;
    const int64_t block_bytes = p.sb * ISZ;

    // Fused append (decode steps): the wave whose slice holds the context's last token
    // writes that token's new K and V rows for this KV head into their pool slot before
    // any of its DMAs, and waits until the stores are done. In a valid step the slot is
    // the one the block table gives for position ctx - 1 and no other sequence's table
    // reaches it (copy-on-write made the block private), so only this wave reads it.
    if (p.app_slots && part == n_parts - 1 && ctx - 1 >= wstart && ctx - 1 < wstart + kSSlice) {
        const int64_t slot = p.app_slots[seq];
        if (slot >= 0 && slot < p.num_blocks * kBS) {
            const int64_t dst = ((slot / kBS) * p.sb + (slot % kBS) * p.ss + (int64_t)kvh * p.sh) * ISZ;
            const int64_t src = ((int64_t)seq * p.app_st + (int64_t)kvh * p.app_sh) * ISZ;
            constexpr int WORDS = ROWB / 4;  // 4-byte words per row
            for (int w = lane; w < 2 * WORDS; w += 64) {
                const bool is_v = w >= WORDS;
                const int off = 4 * (is_v ? w - WORDS : w);
                const uint32_t x = *reinterpret_cast<const uint32_t*>(
                    reinterpret_cast<const char*>(is_v ? p.app_v : p.app_k) + src + off);
                *reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(const_cast<void*>(is_v ? p.v : p.k)) + dst +
                                             off) = x;
            }
            __builtin_amdgcn_s_waitcnt(kWaitVm<0>);  // stores done before this wave's DMAs read the slot
        }
    }

    // Lane b holds the id of the wave's b-th block, for the blocks inside the context
    // (wstart / 16 + b < ceil(ctx / 16) <= table_width).
    int64_t my_blk = -1;
    if (lane < (wtok + kBS - 1) / kBS) my_blk = p.tables[(int64_t)seq * p.table_stride + wstart / kBS + lane];

    const int kj = lane % KLPT;               // K: 16-byte chunks kj, kj + 8, ... of the row
    const int ktok = lane / KLPT;             // K: token within an 8-token round
    Vec16 q[G][CPL];
    {
        const char* qrow = reinterpret_cast<const char*>(p.q) + ((int64_t)seq * p.q_st + (int64_t)kvh * G * p.q_sh) * ISZ;
        const uint32_t q_head_bytes = (uint32_t)(p.q_sh * ISZ);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < CPL; ++i) q[g][i] = load16(qrow + (g * q_head_bytes + (uint32_t)((i * KLPT + kj) * 16)));
    }

    // DMA of chunk c: rows past the context re-read the chunk's first row (a valid token,
    // probability 0); an id outside the pool reads block 0 (memory-safe garbage for an
    // out-of-contract table).
    const int dma_row = lane / CPR;
    const int dma_slot = lane % CPR;
    auto dma_chunk = [&](int c, uint16_t* dk, uint16_t* dv) {
        // The buffer was just read by the previous chunk's LDS loads, and an LDS DMA
        // write is not ordered behind this wave's outstanding LDS reads (it arrives by
        // the vector-memory path). The compiler issues these DMAs before waiting for
        // those reads, so wait here: otherwise a fast DMA can overwrite V rows before
        // P·V has read them.
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
        const int64_t id = readlane64(my_blk, (c * kSCT) / kBS);
        const int64_t bofs = ((uint64_t)id < (uint64_t)p.num_blocks ? id : 0) * block_bytes +
                             (int64_t)((c * kSCT) % kBS) * slot_bytes;
        stream_dma_chunk<D>(kbase + bofs, vbase + bofs, slot_bytes, wtok - c * kSCT, dma_row, dma_slot, dk, dv);
    };

    // Per-head online-softmax state, held by the lanes of the head's group: lane
    // (group lane / kSCT) of softmax round sr owns head lane / kSCT + HPR * sr.
    const int stok = lane % kSCT;
    const int shr = lane / kSCT;
    float m_row[SROUNDS], l_row[SROUNDS];
#pragma unroll
    for (int sr = 0; sr < SROUNDS; ++sr) {
        m_row[sr] = kNegInf;
        l_row[sr] = 0.f;
    }
    const int vchunk = lane % VLPT;
    const int vslot = lane / VLPT;
    float acc[G][EPV];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPV; ++e) acc[g][e] = 0.f;
    // Pair-ordered probability slot of token t: t and t + TSV side by side.
    auto pair_slot = [](int t) { return 2 * ((t / (2 * TSV)) * TSV + t % TSV) + (t / TSV) % 2; };

    auto compute = [&](int c, const uint16_t* ck, const uint16_t* cv) {
        // ---- scores: K rows from LDS against the query registers
#pragma unroll
        for (int kr = 0; kr < KROUNDS; ++kr) {
            const int t = kr * 8 + ktok;
            const char* krow = reinterpret_cast<const char*>(ck) + t * ROWB;
            Vec16 k[CPL];
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const uint4 v = *reinterpret_cast<const uint4*>(krow + (((i * KLPT + kj) ^ stream_kswz<D>(t)) << 4));
                k[i] = Vec16{{v.x, v.y, v.z, v.w}};
            }
            const bool valid = c * kSCT + t < wtok;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float sc = 0.f;
#pragma unroll
                for (int i = 0; i < CPL; ++i) sc = ChunkDot<T>::run(k[i], q[g][i], sc);
                sc = ref_score_log2<T>(octet_sum(sc), p.scale);
                if (g == kj) s_sc[wave][g][t] = valid ? sc : kNegInf;
            }
        }
        wave_lds_sync();
        // ---- online softmax, one head per group of kSCT lanes
        float alpha[G];
#pragma unroll
        for (int sr = 0; sr < SROUNDS; ++sr) {
            const int g = shr + HPR * sr;
            const float a = g < G ? s_sc[wave][g < G ? g : 0][stok] : kNegInf;
            const float m_new = fmaxf(m_row[sr], group_max<kSCT>(a));
            const float al = m_row[sr] == kNegInf ? 1.f : fast_exp2(m_row[sr] - m_new);
            const float pr = m_new == kNegInf ? 0.f : fast_exp2(a - m_new);
            l_row[sr] = l_row[sr] * al + group_sum<kSCT>(pr);
            m_row[sr] = m_new;
            if (g < G) s_sc[wave][g][pair_slot(stok)] = pr;
#pragma unroll
            for (int gg = HPR * sr; gg < HPR * sr + HPR && gg < G; ++gg)
                alpha[gg] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, al),
                                                                               kSCT * (gg - HPR * sr)));
        }
        wave_lds_sync();
        // ---- rescale only the heads whose running max moved (wave-uniform test)
#pragma unroll
        for (int g = 0; g < G; ++g)
            if (alpha[g] != 1.f) {
#pragma unroll
                for (int e = 0; e < EPV; ++e) acc[g][e] *= alpha[g];
            }
        // ---- P·V, two tokens per v_dot2
        uint2 vv[VSTEPS];
#pragma unroll
        for (int st = 0; st < VSTEPS; ++st)
            vv[st] = *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(cv) + (st * TSV + vslot) * ROWB +
                                                     vchunk * 8);
#pragma unroll
        for (int st = 0; st < VSTEPS; st += 2) {
            uint32_t vp[EPV];
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                const uint32_t a = w ? vv[st].y : vv[st].x;
                const uint32_t b = w ? vv[st + 1].y : vv[st + 1].x;
                vp[2 * w] = __builtin_amdgcn_perm(b, a, 0x05040100u);
                vp[2 * w + 1] = __builtin_amdgcn_perm(b, a, 0x07060302u);
            }
            const int t0 = st * TSV + vslot;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float2 pp = *reinterpret_cast<const float2*>(&s_sc[wave][g][pair_slot(t0)]);
                const uint32_t pk = pack_probs<T>(pp.x, pp.y);
#pragma unroll
                for (int e = 0; e < EPV; ++e) acc[g][e] = Pair<T>::dot2(vp[e], pk, acc[g][e]);
            }
        }
        wave_lds_sync();                       // the next chunk rewrites s_sc
    };

    // ---- the ring: chunk c lives in buffer c % 2; chunk c + 2 is issued once c is done
    uint16_t* k0 = s_b0[wave][0];
    uint16_t* v0 = s_b0[wave][1];
    uint16_t* k1 = s_b1[wave][0];
    uint16_t* v1 = s_b1[wave][1];
    // The compiler does not order these reads after the DMA that fills the buffer, so
    // each chunk waits explicitly: the only vector-memory operations issued inside the
    // loop are the DMAs, so "all but the newer chunk's instructions" is exact.
    constexpr int kChunkDmas = 2 * kSCT / (1024 / ROWB);
    auto wait_chunk = [&](int c) {
        if (c + 1 < nchunk) __builtin_amdgcn_s_waitcnt(kWaitVm<kChunkDmas>);
        else __builtin_amdgcn_s_waitcnt(kWaitVm<0>);
    };
    if (nchunk > 0) dma_chunk(0, k0, v0);
    if (nchunk > 1) dma_chunk(1, k1, v1);
    for (int c = 0; c < nchunk; c += 2) {
        wait_chunk(c);
        compute(c, k0, v0);
        if (c + 2 < nchunk) dma_chunk(c + 2, k0, v0);
        if (c + 1 < nchunk) {
            wait_chunk(c + 1);
            compute(c + 1, k1, v1);
            if (c + 3 < nchunk) dma_chunk(c + 3, k1, v1);
        }
    }

    // ---- this wave's unnormalised output over its own s_b0 slice (no longer in use)
    // and its (max, denominator) in s_ml, then one workgroup barrier and the merge.
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPV; ++e) acc[g][e] = fold_lanes<VLPT>(acc[g][e]);
    float* w_acc = reinterpret_cast<float*>(s_b0[wave][0]);   // [G][D]
    if (vslot == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < EPV; ++e) w_acc[g * D + vchunk * EPV + e] = acc[g][e];
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int src = kSCT * (g % HPR);
        const float mg = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m_row[g / HPR]), src));
        const float lg = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l_row[g / HPR]), src));
        if (lane == 0) {
            s_ml[wave][g][0] = mg;
            s_ml[wave][g][1] = lg;
        }
    }
    lds_barrier();

    const int head0 = kvh * G;
    for (int idx = (int)threadIdx.x; idx < G * D; idx += W * 64) {
        const int g = idx / D, d = idx - g * D;
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, s_ml[w][g][0]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float mw = s_ml[w][g][0];
            const float sc = mw == kNegInf ? 0.f : fast_exp2(mw - M);
            L += sc * s_ml[w][g][1];
            O += sc * reinterpret_cast<const float*>(s_b0[w][0])[g * D + d];
        }
        if (n_parts == 1) {
            T* orow = reinterpret_cast<T*>(p.out) + (int64_t)seq * p.out_st + (int64_t)(head0 + g) * p.out_sh;
            orow[d] = from_f32<T>(O / L);
        } else {
            const int64_t slot = ((int64_t)seq * p.num_heads + head0 + g) * p.max_parts + part;
            if (p.ws_cnt) {
                // Agent-scope stores: written through to the point of coherence that
                // every XCD's agent-scope loads read (the merging workgroup may run on
                // another XCD, behind another L2).
                __hip_atomic_store(&p.ws_o[slot * D + d], O, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (d == 0) {
                    __hip_atomic_store(&p.ws_ml[slot * 2], M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(&p.ws_ml[slot * 2 + 1], L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            } else {
                p.ws_o[slot * D + d] = O;
                if (d == 0) {
                    p.ws_ml[slot * 2] = M;
                    p.ws_ml[slot * 2 + 1] = L;
                }
            }
        }
    }
    if (n_parts == 1 || !p.ws_cnt) return;

    // ---- in-kernel split-KV merge. Every partition of a (sequence, KV head), once its
    // partial stores are complete (s_waitcnt: performed at the coherence point), counts
    // itself in; the one that finds all others counted merges the partials, writes the
    // output and returns the counter to zero for the next call. Nothing waits for
    // another workgroup, and the merge reads partials in partition order, so the result
    // is the separate merge kernel's, bit for bit.
    // Ordering: the partial stores above must be performed before the counter update
    // below. s_waitcnt vmcnt(0) holds the wave until every store it issued has been
    // acknowledged by the memory system (on CDNA an agent-scope store is acknowledged
    // once it is visible at the agent's coherence point, which the merging workgroup's
    // agent-scope loads read); the asm's "memory" clobber stops the compiler from
    // moving the stores below it or the counter update above it. No agent-scope
    // release fence is used: on this chip it also writes back the XCD's L2 and was
    // measured to serialise the launch.
    __shared__ uint32_t s_arrived;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    uint32_t* cnt = p.ws_cnt + ((int64_t)seq * p.num_kv_heads + kvh);
    if (threadIdx.x == 0) s_arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_arrived != (uint32_t)(n_parts - 1)) return;
    if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    constexpr int CH = 16;  // partitions whose loads are in flight together
    for (int idx = (int)threadIdx.x; idx < G * D; idx += W * 64) {
        const int g = idx / D, d = idx - g * D;
        const int64_t base = ((int64_t)seq * p.num_heads + head0 + g) * p.max_parts;
        float* ml = p.ws_ml + base * 2;
        float* o = p.ws_o + base * D + d;
        // The separate merge kernel's arithmetic, per element.
        float M = kNegInf, L = 0.f, O = 0.f;
        for (int pt0 = 0; pt0 < n_parts; pt0 += CH) {
            float mx[CH], ly[CH], ov[CH];
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const bool in = pt0 + j < n_parts;
                mx[j] = in ? __hip_atomic_load(ml + 2 * (pt0 + j), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : kNegInf;
                ly[j] = in ? __hip_atomic_load(ml + 2 * (pt0 + j) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
                ov[j] = in ? __hip_atomic_load(o + (int64_t)(pt0 + j) * D, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                           : 0.f;
            }
            float Mc = M;
#pragma unroll
            for (int j = 0; j < CH; ++j) Mc = fmaxf(Mc, mx[j]);
            const float rescale = M == kNegInf ? 0.f : fast_exp2(M - Mc);
            L *= rescale;
            O *= rescale;
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const float sc = mx[j] == kNegInf ? 0.f : fast_exp2(mx[j] - Mc);
                L += sc * ly[j];
                O += sc * ov[j];
            }
            M = Mc;
        }
        T* orow = reinterpret_cast<T*>(p.out) + (int64_t)seq * p.out_st + (int64_t)(head0 + g) * p.out_sh;
        orow[d] = from_f32<T>(O / L);
    }
}

// Instantiated only where the query registers (G * D * itemsize / 32 VGPRs per lane)
// leave room for the in-flight K and V loads without spilling: at most 64 VGPRs of
// query per lane, and no fp32 head_dim 128 (its V step alone would take 128 VGPRs).
// Other combinations take the generic kernel.
template <typename T, int D, int G>
constexpr bool kDecodeFits = G * D * (int)sizeof(T) <= 2048 && !(sizeof(T) == 4 && D > 64);

// Batches whose 768-token partitions would make fewer workgroups than this (counted
// at the batch's longest context) take 256-token partitions: four short chains per
// workgroup instead of a few long ones. Measured (us, 768 vs 256): config 4 402 vs
// 442; Llama shape, 16 sequences at 512 / 1024 / 2048 / 4096 tokens 26.7 / 29.5 /
// 37.7 / 55.6 vs 16.7 / 20.0 / 30.6 / 53.4; 128 sequences at 512 tokens 51.3 vs 54.9;
// GPT-2 shape, 20 sequences at 100-700 tokens 15.4 vs 12.7; config 2 27.5 vs 27.1.
constexpr int64_t kShortPartBelow = 1024;
constexpr int64_t kEightWaveMaxWorkgroups = 512;

// Merge in the partition kernel (its last partition of each (sequence, KV head)) or in
// a second kernel. In-kernel, every multi-partition workgroup waits for its partial
// stores to complete and the merges run where each (sequence, KV head) finishes: a
// win wherever contexts are ragged or short (config 4 -1.9%, config 2 -8%, GPT-2
// decode shapes -5% per call), a loss for a few long, equal contexts in 768-token
// partitions, whose merges all land at the end of the launch (32 sequences x 4096
// tokens +14%). The second kernel is kept for 768-token launches of at most 512
// (sequence, KV head) pairs spanning 4+ partitions.
constexpr int64_t kSeparateMergeMaxPairs = 512;
constexpr int kSeparateMergeMinParts = 4;

template <typename T, int D, int G, int PART, int W>
int launch_stream(const AttnParams& p0, dim3 grid, hipStream_t stream) {
    const int parts = (p0.max_parts * kDecodePart + PART - 1) / PART;
    AttnParams p = p0;
    if (PART == kSPartLong && (int64_t)p.num_seqs * p.num_kv_heads <= kSeparateMergeMaxPairs &&
        parts >= kSeparateMergeMinParts)
        p.ws_cnt = nullptr;
    paged_decode_stream_kernel<T, D, G, PART, W><<<dim3(grid.x, parts, grid.z), W * 64, 0, stream>>>(p);
    int rc = check_launch("paged decode attention");
    if (rc || parts == 1 || p.ws_cnt) return rc;
    paged_decode_combine_kernel<T, D, G, PART><<<dim3(grid.x, grid.z), kCombineThreads<G, D>, 0, stream>>>(p);
    return check_launch("paged decode combine");
}

template <typename T, int D, int G>
int launch_g(const AttnParams& p, dim3 grid, hipStream_t stream) {
    if constexpr (sizeof(T) == 2) {
        // 16-bit pools: the streaming kernel (its redirected rows need a non-empty pool).
        if (p.num_blocks >= 1) {
            const int64_t long_parts = ((int64_t)p.max_parts * kDecodePart + kSPartLong - 1) / kSPartLong;
            if ((int64_t)p.num_seqs * p.num_kv_heads * long_parts >= kShortPartBelow) {
                // 768-token partitions: 8 waves x 96 tokens for grouped heads whose merge
                // runs in the partition kernel, else 4 waves x 192. Measured (us, 4 vs 8
                // waves): config 4 394.7 vs 391.2; 128 x 512-8192 tokens at GQA 2 420 vs
                // 409; head_dim 64 GQA 4, 128 x 1024-4096 149.0 vs 141.8; GQA 8 359.6 vs
                // 359.4; GQA 1 (config 2) 24.8 vs 25.6; 32 x 4096 with the separate merge
                // 96.0 vs 97.8.
                const bool separate_merge = (int64_t)p.num_seqs * p.num_kv_heads <= kSeparateMergeMaxPairs &&
                                            long_parts >= kSeparateMergeMinParts;
                if (G >= 2 && !separate_merge) return launch_stream<T, D, G, kSPartLong, 8>(p, grid, stream);
                return launch_stream<T, D, G, kSPartLong, 4>(p, grid, stream);
            }
            // Short partitions: 8 waves x 32 tokens (four-chunk chains) where the
            // workgroups fit one round at the 8-wave kernel's LDS (all of head_dim 64,
            // head_dim 128 up to 512 workgroups), else 4 waves x 64 tokens. Measured (us,
            // 4 vs 8 waves): GPT-2 shape 32 x 100-700 tokens 12.7 vs 11.6, 24 x 16-400
            // 9.8 vs 8.5, 8 x 200-900 8.6 vs 7.6; Llama shape 16 x 1024 18.7 vs 17.4,
            // 8 x 4096 (1024 workgroups) 31.5 vs 34.4.
            const int64_t short_wgs = (int64_t)p.num_seqs * p.num_kv_heads *
                                      (((int64_t)p.max_parts * kDecodePart + kSPartShort - 1) / kSPartShort);
            if (D == 64 || short_wgs <= kEightWaveMaxWorkgroups)
                return launch_stream<T, D, G, kSPartShort, 8>(p, grid, stream);
            return launch_stream<T, D, G, kSPartShort, 4>(p, grid, stream);
        }
    }
    if constexpr (kDecodeFits<T, D, G>) {
        paged_decode_kernel<T, D, G><<<grid, kWaves * 64, 0, stream>>>(p);
        int rc = check_launch("paged decode attention");
        if (rc || p.max_parts == 1) return rc;
        paged_decode_combine_kernel<T, D, G, kDecodePart><<<dim3(grid.x, grid.z), kCombineThreads<G, D>, 0, stream>>>(p);
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

bool decode_streams(const AttnParams& p, int dtype) {
    if (dtype == PKV_FLOAT32 || p.num_blocks < 1 || p.block_size != kBS) return false;
    if (p.group != 1 && p.group != 2 && p.group != 4 && p.group != 8) return false;
    if (p.head_dim != 64 && p.head_dim != 128) return false;
    if (p.num_kv_heads > 65535 || p.max_parts > 65535 || p.num_seqs > 65535) return false;
    if (p.max_parts > 1 && (!p.ws_o || !p.ws_ml)) return false;
    const uint64_t probe = (uint64_t)(uintptr_t)p.q | (uint64_t)(uintptr_t)p.k | (uint64_t)(uintptr_t)p.v |
                           (uint64_t)(p.q_st * 2) | (uint64_t)(p.q_sh * 2) | (uint64_t)(p.sb * 2) |
                           (uint64_t)(p.ss * 2) | (uint64_t)(p.sh * 2);
    return probe % 16 == 0;
}

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
