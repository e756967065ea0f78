// Launch parameters shared by the paged-attention kernels (internal to libpagedkv).
#pragma once

#include "pkv_common.h"

namespace pkv {

struct AttnParams {
    void* out;
    int64_t out_st, out_sh;          // elements
    const void* q;
    int64_t q_st, q_sh;              // elements
    const void* k;
    const void* v;
    int64_t sb, ss, sh;              // pool strides (elements): block, slot, head
    int64_t num_blocks;
    int block_size, num_kv_heads, head_dim;
    const int64_t* tables;
    int64_t table_stride, table_width;
    const int64_t* ctx_lens;
    const int64_t* qsl;              // query_start_loc [num_seqs+1]; null => token i is seq i
    int num_seqs, num_heads, group;
    int64_t num_tokens;
    int max_query_len;
    float scale_log2;                // scale * log2(e): scores live in the base-2 domain
    float scale;                     // softmax scale, applied to the rounded dot product
    // split-KV decode workspace
    float* ws_o;                     // [num_seqs, num_heads, max_parts, head_dim]
    float* ws_ml;                    // [num_seqs, num_heads, max_parts, 2] = (max, denominator)
    int max_parts;
    // Split-KV merge counters, one per (sequence, KV head), zero between calls (null:
    // the partials are merged by a second kernel). With them the streaming kernel's
    // last partition of a (sequence, KV head) to finish does the merge itself.
    uint32_t* ws_cnt;
    // Fused KV append (null = none). Decode (streaming kernel): row seq of app_k / app_v
    // ([num_seqs, num_kv_heads, head_dim], element strides app_st, app_sh) goes to flat
    // pool slot app_slots[seq] before the attention reads it. Prefill (MFMA kernel): row
    // t of [num_tokens, num_kv_heads, head_dim] goes to app_slots[t] and the kernel reads
    // the new positions from these rows.
    const void* app_k;
    const void* app_v;
    int64_t app_st, app_sh;
    const int64_t* app_slots;
    // Persistent MFMA decode: units (blocks x KV-head groups) before each sequence,
    // [num_seqs + 1], written by the decode kernel for its merge kernel.
    int* ws_pfx;
};

// True when launch_decode_attention runs the streaming kernel for these parameters
// (the only decode kernel that performs a fused append).
bool decode_streams(const AttnParams& p, int dtype);
// True when launch_prefill_attention runs the MFMA kernel for these parameters (with
// p.app_* set: including the fused append, whose source rows must be 16-byte aligned).
bool prefill_tuned(const AttnParams& p, int dtype);

// Bytes reserved for the merge counters at the front of a decode workspace (a fixed
// size, so counters never overlap another call's partials in a reused workspace).
constexpr int64_t kMergeCounterBytes = 256 * 1024;

// Tokens per split-KV partition of the decode kernel (one workgroup's share).
// Measured on config 4 (ragged contexts 512-8192): 256 -> 5.03 TB/s, 512 -> 4.81,
// 128 -> 4.80 (512 wins only for uniform long contexts, 5.44 vs 5.31).
constexpr int kDecodePart = 256;

// Persistent MFMA decode (attn_decode_mfma.hip): whether it takes a batch of these
// parameters (16-bit pools, block size 16, head_dim 64/128, GQA 1/2/4/8, a multiple of
// 4 KV heads, at most 1024 sequences, at least 512 MiB of K/V at the longest context),
// the floats its split-KV partials
// need (0 when it never applies to such sizes), and the launch (PKV_EUNSUPPORTED
// without an error when the device does not fit). It needs p.ws_pfx, p.ws_ml, p.ws_o.
constexpr int kDecodeMfmaMaxSeqs = 1024;
bool decode_mfma_applies(const AttnParams& p, int dtype, int64_t max_context_len);
bool decode_mfma_sizes_apply(int64_t num_seqs, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                             int64_t max_context_len);
int64_t decode_mfma_partial_floats(int64_t num_kv_heads, int64_t group, int64_t head_dim);
int launch_decode_mfma(const AttnParams& p, int dtype, hipStream_t stream);

int launch_generic_attention(const AttnParams& p, int dtype, hipStream_t stream);
// fp32 pools, block size 16, head_dim 64/128, GQA 1/2/4/8, 16-byte aligned rows: the
// tiled fp32 kernel (any query lengths; p.qsl null for a decode batch). Returns
// PKV_EUNSUPPORTED (without setting an error) for anything else.
int launch_f32_attention(const AttnParams& p, hipStream_t stream);
// fp32 pools, prefill / chunked-prefill batches (p.qsl set, no fused append, a row of at
// least 2 tokens), block size 16, head_dim 64/128, GQA 1/2/4/8, 16-byte aligned rows: the
// fp32 MFMA kernel. Returns PKV_EUNSUPPORTED (without setting an error) for anything else.
int launch_prefill_f32_mfma(const AttnParams& p, hipStream_t stream);
// Returns PKV_EUNSUPPORTED (without setting an error) when no tuned kernel matches.
int launch_decode_attention(const AttnParams& p, int dtype, hipStream_t stream);
int launch_prefill_attention(const AttnParams& p, int dtype, hipStream_t stream);

// ---- prefill dispatch order (the MFMA prefill kernels, 256-thread workgroups).
// A prefill grid walks (sequence slot, query block) items; sequence slot i runs the
// sequence with the i-th largest context (ties by index), so the workgroups with the
// longest causal ranges start first and the end of the launch is left to short ones
// (bf16 config 4 chunks: the occupancy drained over the last ~50 of ~345 us in index
// order; 314.2 -> 306.7 us per call). Ordering every (sequence, query block) pair
// longest first instead was slower (322-325 us): it scatters a sequence's query blocks,
// whose K/V tiles one L2 otherwise serves to all of them. Every workgroup ranks the
// batch's contexts itself (one load per sequence, replacing its own context and query
// start loads); batches of more than kPrefillSortSeqs sequences keep index order.
constexpr int kPrefillSortSeqs = 256;   // one sequence per thread

struct PrefillSeq {
    int seq;
    int64_t q_first;
    int q_len;
    int ctx;                            // context length clamped to the table width
};

// Called by every thread of a 256-thread workgroup (it holds two barriers).
__device__ __forceinline__ PrefillSeq prefill_seq(const AttnParams& p, int seq_slot, int block_size) {
    const int64_t cap = p.table_width * (int64_t)block_size;
    PrefillSeq r;
    if (p.num_seqs > kPrefillSortSeqs) {
        r.seq = seq_slot;
        r.q_first = p.qsl[seq_slot];
        r.q_len = (int)(p.qsl[seq_slot + 1] - r.q_first);
        const int64_t c = p.ctx_lens[seq_slot];
        r.ctx = (int)(c < cap ? c : cap);
        return r;
    }
    __shared__ int s_ctx[kPrefillSortSeqs];
    __shared__ int s_order[kPrefillSortSeqs];
    __shared__ int64_t s_qsl[kPrefillSortSeqs + 1];
    const int t = (int)threadIdx.x;
    if (t < p.num_seqs) {
        const int64_t c = p.ctx_lens[t];
        s_ctx[t] = (int)(c < cap ? c : cap);
        s_qsl[t] = p.qsl[t];
    }
    if (t == 0) s_qsl[p.num_seqs] = p.qsl[p.num_seqs];
    __syncthreads();
    if (t < p.num_seqs) {
        const int ct = s_ctx[t];
        int rank = 0;
        for (int u = 0; u < p.num_seqs; ++u) {
            const int cu = s_ctx[u];
            rank += (cu > ct || (cu == ct && u < t)) ? 1 : 0;
        }
        s_order[rank] = t;
    }
    __syncthreads();
    r.seq = s_order[seq_slot];
    r.q_first = s_qsl[r.seq];
    r.q_len = (int)(s_qsl[r.seq + 1] - r.q_first);
    r.ctx = s_ctx[r.seq];
    return r;
}

}  // namespace pkv
