// Generic paged attention: any block size, any head_dim <= 512, any GQA group, any
// mix of prefill and decode tokens, fp32/fp16/bf16.
//
// One wave64 owns one (query token, query head) — the program decomposition of the
// reference's kernel design (core/attention_triton.py:13-32, grid (tokens, heads)
// at :288) — and walks that token's keys 0..q_pos through the block table with an
// online softmax in fp32. Lanes split head_dim (lane d, d+64, ...), so each key row
// is one coalesced load and the score is one wave reduction. This path exists for
// shapes the tuned kernels do not cover (block sizes 4/6, head_dim 8/12 in the unit
// tests, fp32 prefill); the tuned decode and MFMA prefill kernels take every
// production shape.
#include "attention.h"

namespace pkv {
namespace {

template <typename T, int EPL>
__global__ __launch_bounds__(256) void generic_attention_kernel(const AttnParams p) {
    const int wave = (int)(threadIdx.x >> 6);
    const int lane = lane_id();
    const int64_t tok = (int64_t)blockIdx.x * 4 + wave;
    const int head = (int)blockIdx.y;
    if (tok >= p.num_tokens) return;

    // Token -> sequence: the last s with query_start_loc[s] <= tok (empty sequences
    // share a start with their successor, so the last one is the owner).
    int seq;
    int64_t q_len, q_start;
    if (p.qsl) {
        int lo = 0, hi = p.num_seqs;  // answer in [lo, hi)
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (p.qsl[mid] <= tok) lo = mid; else hi = mid;
        }
        seq = lo;
        q_start = p.qsl[seq];
        q_len = p.qsl[seq + 1] - q_start;
    } else {
        seq = (int)tok;
        q_start = tok;
        q_len = 1;
    }
    const int64_t ctx = p.ctx_lens[seq];
    // Logical position of this token: the LAST q_len positions of the context
    // (core/attention.py:44-53); it sees keys 0..q_pos (core/attention_triton.py:185).
    const int64_t q_pos = ctx - q_len + (tok - q_start);
    const int64_t n_keys = q_pos + 1;
    const int kvh = head / p.group;

    const T* qrow = reinterpret_cast<const T*>(p.q) + tok * p.q_st + (int64_t)head * p.q_sh;
    float q[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const int d = lane + 64 * e;
        q[e] = d < p.head_dim ? to_f32(qrow[d]) : 0.f;
    }

    const T* kbase = reinterpret_cast<const T*>(p.k) + (int64_t)kvh * p.sh;
    const T* vbase = reinterpret_cast<const T*>(p.v) + (int64_t)kvh * p.sh;
    const int64_t* table = p.tables + (int64_t)seq * p.table_stride;

    float m = kNegInf, l = 0.f, acc[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] = 0.f;

    // Out-of-contract input stays in bounds: keys beyond the table row are not
    // walked and block ids outside the pool read as zero.
    const int64_t key_cap = p.table_width * p.block_size;
    const int64_t n_walk = n_keys < key_cap ? n_keys : key_cap;
    for (int64_t j = 0; j < n_walk; ++j) {
        int64_t blk = table[j / p.block_size];
        const bool blk_ok = (uint64_t)blk < (uint64_t)p.num_blocks;
        blk = blk_ok ? blk : 0;
        const int64_t row = blk * p.sb + (j % p.block_size) * p.ss;
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int d = lane + 64 * e;
            if (d < p.head_dim && blk_ok) s += q[e] * to_f32(kbase[row + d]);
        }
        s = ref_score_log2<T>(wave_sum(s), p.scale);
        const float m_new = fmaxf(m, s);
        const float alpha = fast_exp2(m - m_new);  // 0 on the first key (m = -inf)
        const float pj = fast_exp2(s - m_new);
        l = l * alpha + pj;
        // P.V takes the probability in the pool dtype (the reference's probs.to(v.dtype)).
        const float pv = to_f32(from_f32<T>(pj));
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int d = lane + 64 * e;
            const float vd = (d < p.head_dim && blk_ok) ? to_f32(vbase[row + d]) : 0.f;
            acc[e] = acc[e] * alpha + pv * vd;
        }
        m = m_new;
    }

    T* orow = reinterpret_cast<T*>(p.out) + tok * p.out_st + (int64_t)head * p.out_sh;
    const float inv = 1.f / l;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const int d = lane + 64 * e;
        if (d < p.head_dim) orow[d] = from_f32<T>(acc[e] * inv);
    }
}

template <typename T>
int launch_t(const AttnParams& p, hipStream_t stream) {
    const int64_t gx = ceil_div(p.num_tokens, 4);
    if (gx > 0x7fffffff || p.num_heads > 65535) return fail(PKV_EUNSUPPORTED, "attention: grid too large");
    dim3 grid((unsigned)gx, (unsigned)p.num_heads);
    const int epl = (int)ceil_div(p.head_dim, 64);
    if (epl <= 1) generic_attention_kernel<T, 1><<<grid, 256, 0, stream>>>(p);
    else if (epl <= 2) generic_attention_kernel<T, 2><<<grid, 256, 0, stream>>>(p);
    else if (epl <= 4) generic_attention_kernel<T, 4><<<grid, 256, 0, stream>>>(p);
    else if (epl <= 8) generic_attention_kernel<T, 8><<<grid, 256, 0, stream>>>(p);
    else return fail(PKV_EUNSUPPORTED, "attention: head_dim %d > 512", p.head_dim);
    return check_launch("generic attention");
}

}  // namespace

int launch_generic_attention(const AttnParams& p, int dtype, hipStream_t stream) {
    if (p.num_tokens == 0) return PKV_OK;
    switch (dtype) {
        case PKV_FLOAT32: return launch_t<float>(p, stream);
        case PKV_FLOAT16: return launch_t<_Float16>(p, stream);
        case PKV_BFLOAT16: return launch_t<bf16_t>(p, stream);
    }
    return fail(PKV_EINVAL, "attention: unknown dtype %d", dtype);
}

}  // namespace pkv
