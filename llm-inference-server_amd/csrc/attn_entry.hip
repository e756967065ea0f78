// extern "C" paged-attention entry points: argument checks, workspace carving, and
// dispatch to the tuned kernels (decode split-KV, MFMA prefill) or the generic one.
#include <mutex>

#include "attention.h"

// Split-KV partials of pkv_paged_attention_decode_noalloc: a static device buffer, one
// copy per device. In host code this name is a host-side stand-in, not a device
// address: host code uses only the address hipGetSymbolAddress returns for the current
// device (looked up once per device, kept in g_scratch below).
static __device__ __align__(256) unsigned char scratch[PKV_DECODE_SCRATCH_BYTES];

namespace pkv {
namespace {

int itemsize(int dtype) { return dtype == PKV_FLOAT32 ? 4 : (dtype == PKV_FLOAT16 || dtype == PKV_BFLOAT16) ? 2 : 0; }

int fill_common(AttnParams& p, const char* what, void* out, int64_t out_st, int64_t out_sh, const void* query,
                int64_t q_st, int64_t q_sh, const void* k_pool, const void* v_pool, int64_t sb, int64_t ss,
                int64_t sh, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
                const int64_t* tables, int64_t table_stride, int64_t table_width, const int64_t* ctx_lens,
                int64_t num_seqs, int64_t num_heads, float scale, int dtype) {
    if (!itemsize(dtype)) return fail(PKV_EINVAL, "%s: unknown dtype %d", what, dtype);
    if (num_seqs < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks < 0 ||
        table_width < 0)
        return fail(PKV_EINVAL, "%s: bad sizes", what);
    if (num_heads % num_kv_heads)
        return fail(PKV_EINVAL, "%s: %lld query heads not divisible by %lld kv heads", what, (long long)num_heads,
                    (long long)num_kv_heads);
    if (num_seqs > 0x7fffffff || num_heads > 65535 || head_dim > 0x7fffffff || block_size > 0x7fffffff)
        return fail(PKV_EUNSUPPORTED, "%s: sizes beyond int32", what);
    p = AttnParams{};
    p.out = out;
    p.out_st = out_st;
    p.out_sh = out_sh;
    p.q = query;
    p.q_st = q_st;
    p.q_sh = q_sh;
    p.k = k_pool;
    p.v = v_pool;
    p.sb = sb;
    p.ss = ss;
    p.sh = sh;
    p.num_blocks = num_blocks;
    p.block_size = (int)block_size;
    p.num_kv_heads = (int)num_kv_heads;
    p.head_dim = (int)head_dim;
    p.tables = tables;
    p.table_stride = table_stride;
    p.table_width = table_width;
    p.ctx_lens = ctx_lens;
    p.num_seqs = (int)num_seqs;
    p.num_heads = (int)num_heads;
    p.group = (int)(num_heads / num_kv_heads);
    p.scale_log2 = scale * kLog2e;
    p.scale = scale;
    return PKV_OK;
}

// Layout: [merge counters, kMergeCounterBytes][ml][o] when any context spans more than
// one partition; empty otherwise.
// Behind the counters two layouts share the space: the partition kernels' partials
// ([ml][o] per (sequence, head, 256-token partition)) and the persistent MFMA kernel's
// ([prefix table][ml][o], partials per (workgroup, side, wave, head)); the workspace
// holds the larger. The MFMA kernel never touches the counters, so they stay zero.
struct DecodeWorkspace {
    int64_t cnt_bytes, ml_bytes, o_bytes;
    int64_t mfma_pfx_bytes, mfma_ml_bytes, mfma_o_bytes;
    int max_parts;
    int64_t total() const {
        const int64_t part = ml_bytes + o_bytes;
        const int64_t mfma = mfma_pfx_bytes + mfma_ml_bytes + mfma_o_bytes;
        return cnt_bytes + (part > mfma ? part : mfma);
    }
    int64_t mfma_total() const { return cnt_bytes + mfma_pfx_bytes + mfma_ml_bytes + mfma_o_bytes; }
};

DecodeWorkspace decode_workspace(int64_t num_seqs, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                 int64_t max_context_len) {
    DecodeWorkspace w;
    w.max_parts = (int)(max_context_len > 0 ? ceil_div(max_context_len, kDecodePart) : 1);
    auto round256 = [](int64_t b) { return ceil_div(b, 256) * 256; };
    w.ml_bytes = round256(num_seqs * num_heads * w.max_parts * 2 * 4);
    w.o_bytes = round256(num_seqs * num_heads * w.max_parts * head_dim * 4);
    w.cnt_bytes = kMergeCounterBytes;
    w.mfma_pfx_bytes = w.mfma_ml_bytes = w.mfma_o_bytes = 0;
    if (decode_mfma_sizes_apply(num_seqs, num_heads, num_kv_heads, head_dim, max_context_len)) {
        const int64_t slots = decode_mfma_partial_floats(num_kv_heads, num_heads / num_kv_heads, head_dim) /
                              (head_dim + 2);
        if (slots > 0) {
            w.mfma_pfx_bytes = round256((kDecodeMfmaMaxSeqs + 1) * 4);
            w.mfma_ml_bytes = round256(slots * 2 * 4);
            w.mfma_o_bytes = round256(slots * head_dim * 4);
        }
    }
    if (w.max_parts == 1) w.cnt_bytes = w.ml_bytes = w.o_bytes = 0;  // single partition: no partials
    return w;
}

}  // namespace
}  // namespace pkv

using namespace pkv;

extern "C" int64_t pkv_paged_attention_decode_workspace_bytes(int64_t num_seqs, int64_t num_heads,
                                                              int64_t num_kv_heads, int64_t head_dim,
                                                              int64_t max_context_len) {
    if (num_seqs < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0) return 0;
    DecodeWorkspace w = decode_workspace(num_seqs, num_heads, num_kv_heads, head_dim, max_context_len);
    return w.total();
}

namespace pkv {
namespace {

struct DecodeAppend {
    const void* k_new;
    const void* v_new;
    int64_t st, sh;
    const int64_t* slots;
};

int decode_impl(void* out, int64_t out_stride_t, int64_t out_stride_h, const void* query, int64_t q_stride_t,
                int64_t q_stride_h, const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                int64_t pool_stride_slot, int64_t pool_stride_head, int64_t num_blocks, int64_t block_size,
                int64_t num_kv_heads, int64_t head_dim, const int64_t* block_tables, int64_t table_stride,
                int64_t table_width, const int64_t* context_lens, int64_t num_seqs, int64_t num_heads,
                int64_t max_context_len, float scale, int dtype, void* workspace, int64_t workspace_bytes,
                const DecodeAppend* app, hipStream_t stream) {
    AttnParams p;
    int rc = fill_common(p, "paged_attention_decode", out, out_stride_t, out_stride_h, query, q_stride_t,
                         q_stride_h, k_pool, v_pool, pool_stride_block, pool_stride_slot, pool_stride_head,
                         num_blocks, block_size, num_kv_heads, head_dim, block_tables, table_stride, table_width,
                         context_lens, num_seqs, num_heads, scale, dtype);
    if (rc) return rc;
    if (num_seqs == 0) return PKV_OK;
    if (!out || !query || !k_pool || !v_pool || !block_tables || !context_lens)
        return fail(PKV_EINVAL, "paged_attention_decode: null pointer");
    if (max_context_len <= 0 || max_context_len > table_width * block_size) max_context_len = table_width * block_size;
    p.num_tokens = num_seqs;
    p.max_query_len = 1;

    DecodeWorkspace w = decode_workspace(num_seqs, num_heads, num_kv_heads, head_dim, max_context_len);
    // A single partition writes the output directly and touches no workspace.
    if (w.max_parts > 1) {
        const int64_t need = w.total();
        if (!workspace || workspace_bytes < need)
            return fail(PKV_EWORKSPACE, "paged_attention_decode: workspace of %lld bytes, need %lld",
                        (long long)workspace_bytes, (long long)need);
        // Counters only while every (sequence, KV head) has one.
        p.ws_cnt = num_seqs * num_kv_heads <= w.cnt_bytes / 4 ? (uint32_t*)workspace : nullptr;
        p.ws_ml = (float*)((char*)workspace + w.cnt_bytes);
        p.ws_o = (float*)((char*)workspace + w.cnt_bytes + w.ml_bytes);
    }
    p.max_parts = w.max_parts;

    // Long contexts over a large batch: the persistent MFMA kernel, when the workspace
    // holds its partials (it always needs the counters).
    const bool mfma = decode_mfma_applies(p, dtype, max_context_len) && w.mfma_pfx_bytes > 0 &&
                      w.mfma_total() <= workspace_bytes;
    if (mfma) {
        p.ws_pfx = (int*)((char*)workspace + w.cnt_bytes);
        p.ws_ml = (float*)((char*)workspace + w.cnt_bytes + w.mfma_pfx_bytes);
        p.ws_o = (float*)((char*)workspace + w.cnt_bytes + w.mfma_pfx_bytes + w.mfma_ml_bytes);
    }

    if (app) {
        // The streaming kernel writes the rows itself (4-byte copies: even strides and
        // 4-byte aligned sources); any other kernel gets the append launch first.
        const bool fuse = decode_streams(p, dtype) && app->st % 2 == 0 && app->sh % 2 == 0 &&
                          ((uintptr_t)app->k_new | (uintptr_t)app->v_new) % 4 == 0;
        if (fuse) {
            p.app_k = app->k_new;
            p.app_v = app->v_new;
            p.app_st = app->st;
            p.app_sh = app->sh;
            p.app_slots = app->slots;
        } else {
            rc = pkv_kv_append(const_cast<void*>(k_pool), const_cast<void*>(v_pool), pool_stride_block,
                               pool_stride_slot, pool_stride_head, num_blocks, block_size, num_kv_heads, head_dim,
                               app->k_new, app->v_new, app->st, app->sh, app->slots, num_seqs, dtype, stream);
            if (rc) return rc;
        }
    }
    if (mfma) {
        rc = launch_decode_mfma(p, dtype, stream);
        if (rc != PKV_EUNSUPPORTED) return rc;
        clear_error();
        // Not launched after all (no occupancy on this device): the partition kernels,
        // with their own partial layout.
        p.ws_pfx = nullptr;
        p.ws_ml = (float*)((char*)workspace + w.cnt_bytes);
        p.ws_o = (float*)((char*)workspace + w.cnt_bytes + w.ml_bytes);
    }
    rc = launch_decode_attention(p, dtype, stream);
    if (rc != PKV_EUNSUPPORTED) return rc;
    clear_error();
    if (dtype == PKV_FLOAT32) {
        rc = launch_f32_attention(p, stream);
        if (rc != PKV_EUNSUPPORTED) return rc;
    }
    return launch_generic_attention(p, dtype, stream);
}

}  // namespace
}  // namespace pkv

extern "C" int pkv_paged_attention_decode(
    void* out, int64_t out_stride_t, int64_t out_stride_h, const void* query, int64_t q_stride_t,
    int64_t q_stride_h, const void* k_pool, const void* v_pool, int64_t pool_stride_block, int64_t pool_stride_slot,
    int64_t pool_stride_head, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
    const int64_t* block_tables, int64_t table_stride, int64_t table_width, const int64_t* context_lens,
    int64_t num_seqs, int64_t num_heads, int64_t max_context_len, float scale, int dtype, void* workspace,
    int64_t workspace_bytes, hipStream_t stream) {
    clear_error();
    return decode_impl(out, out_stride_t, out_stride_h, query, q_stride_t, q_stride_h, k_pool, v_pool,
                       pool_stride_block, pool_stride_slot, pool_stride_head, num_blocks, block_size, num_kv_heads,
                       head_dim, block_tables, table_stride, table_width, context_lens, num_seqs, num_heads,
                       max_context_len, scale, dtype, workspace, workspace_bytes, nullptr, stream);
}

extern "C" int pkv_paged_attention_decode_append(
    void* out, int64_t out_stride_t, int64_t out_stride_h, const void* query, int64_t q_stride_t,
    int64_t q_stride_h, void* k_pool, void* v_pool, int64_t pool_stride_block, int64_t pool_stride_slot,
    int64_t pool_stride_head, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
    const void* k_new, const void* v_new, int64_t new_stride_t, int64_t new_stride_h, const int64_t* slots,
    const int64_t* block_tables, int64_t table_stride, int64_t table_width, const int64_t* context_lens,
    int64_t num_seqs, int64_t num_heads, int64_t max_context_len, float scale, int dtype, void* workspace,
    int64_t workspace_bytes, hipStream_t stream) {
    clear_error();
    if (num_seqs > 0 && (!k_new || !v_new || !slots))
        return fail(PKV_EINVAL, "paged_attention_decode_append: null pointer");
    const DecodeAppend app{k_new, v_new, new_stride_t, new_stride_h, slots};
    return decode_impl(out, out_stride_t, out_stride_h, query, q_stride_t, q_stride_h, k_pool, v_pool,
                       pool_stride_block, pool_stride_slot, pool_stride_head, num_blocks, block_size, num_kv_heads,
                       head_dim, block_tables, table_stride, table_width, context_lens, num_seqs, num_heads,
                       max_context_len, scale, dtype, workspace, workspace_bytes, &app, stream);
}

namespace pkv {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

// Device address of `scratch` on the current device.
int scratch_address(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return fail(PKV_EHIP, "paged_attention_decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(PKV_EUNSUPPORTED, "paged_attention_decode_noalloc: device %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(PKV_EHIP, "paged_attention_decode_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    return PKV_OK;
}

}  // namespace
}  // namespace pkv

extern "C" int pkv_paged_attention_decode_noalloc(
    void* out, int64_t out_stride_t, int64_t out_stride_h, const void* query, int64_t q_stride_t,
    int64_t q_stride_h, const void* k_pool, const void* v_pool, int64_t pool_stride_block, int64_t pool_stride_slot,
    int64_t pool_stride_head, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
    const int64_t* block_tables, int64_t table_stride, int64_t table_width, const int64_t* context_lens,
    int64_t num_seqs, int64_t num_heads, int64_t max_context_len, float scale, int dtype, hipStream_t stream) {
    clear_error();
    void* ws = nullptr;
    if (num_seqs > 0 && num_heads > 0 && num_kv_heads > 0 && head_dim > 0 && block_size > 0 && table_width >= 0 &&
        table_width <= ((int64_t)1 << 40) / block_size) {
        int64_t bound = max_context_len;
        if (bound <= 0 || bound > table_width * block_size) bound = table_width * block_size;
        const DecodeWorkspace w = decode_workspace(num_seqs, num_heads, num_kv_heads, head_dim, bound);
        const int64_t need = w.total();
        if (need > PKV_DECODE_SCRATCH_BYTES)
            return fail(PKV_EWORKSPACE,
                        "paged_attention_decode_noalloc: the batch needs %lld bytes of split-KV partials, "
                        "the static scratch holds %lld (use pkv_paged_attention_decode with a workspace)",
                        (long long)need, (long long)PKV_DECODE_SCRATCH_BYTES);
        if (need > 0) {
            const int rc = scratch_address(&ws);
            if (rc) return rc;
        }
    }
    return decode_impl(out, out_stride_t, out_stride_h, query, q_stride_t, q_stride_h, k_pool, v_pool,
                       pool_stride_block, pool_stride_slot, pool_stride_head, num_blocks, block_size, num_kv_heads,
                       head_dim, block_tables, table_stride, table_width, context_lens, num_seqs, num_heads,
                       max_context_len, scale, dtype, ws, ws ? PKV_DECODE_SCRATCH_BYTES : 0, nullptr, stream);
}

namespace pkv {
namespace {

int prefill_impl(void* out, int64_t out_stride_t, int64_t out_stride_h, const void* query, int64_t q_stride_t,
                 int64_t q_stride_h, const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                 int64_t pool_stride_slot, int64_t pool_stride_head, int64_t num_blocks, int64_t block_size,
                 int64_t num_kv_heads, int64_t head_dim, const int64_t* block_tables, int64_t table_stride,
                 int64_t table_width, const int64_t* context_lens, const int64_t* query_start_loc,
                 int64_t num_seqs, int64_t num_heads, int64_t num_tokens, int64_t max_query_len, float scale,
                 int dtype, const DecodeAppend* app, hipStream_t stream) {
    AttnParams p;
    int rc = fill_common(p, "paged_attention_prefill", out, out_stride_t, out_stride_h, query, q_stride_t,
                         q_stride_h, k_pool, v_pool, pool_stride_block, pool_stride_slot, pool_stride_head,
                         num_blocks, block_size, num_kv_heads, head_dim, block_tables, table_stride, table_width,
                         context_lens, num_seqs, num_heads, scale, dtype);
    if (rc) return rc;
    if (num_tokens < 0 || max_query_len < 0) return fail(PKV_EINVAL, "paged_attention_prefill: bad sizes");
    if (num_tokens == 0 || num_seqs == 0) return PKV_OK;
    if (!out || !query || !k_pool || !v_pool || !block_tables || !context_lens || !query_start_loc)
        return fail(PKV_EINVAL, "paged_attention_prefill: null pointer");
    p.qsl = query_start_loc;
    p.num_tokens = num_tokens;
    // No sequence has more queries than the batch has tokens: num_tokens is always a
    // valid bound, and replaces a missing (0) or larger one.
    if (max_query_len <= 0 || max_query_len > num_tokens) max_query_len = num_tokens;
    p.max_query_len = (int)(max_query_len > 0x7fffffff ? 0x7fffffff : max_query_len);
    if (app) {
        p.app_k = app->k_new;
        p.app_v = app->v_new;
        p.app_st = app->st;
        p.app_sh = app->sh;
        p.app_slots = app->slots;
        if (!prefill_tuned(p, dtype)) {
            // Any other kernel reads the pool only: append first, on the same stream.
            p.app_k = p.app_v = nullptr;
            p.app_slots = nullptr;
            rc = pkv_kv_append(const_cast<void*>(k_pool), const_cast<void*>(v_pool), pool_stride_block,
                               pool_stride_slot, pool_stride_head, num_blocks, block_size, num_kv_heads, head_dim,
                               app->k_new, app->v_new, app->st, app->sh, app->slots, num_tokens, dtype, stream);
            if (rc) return rc;
        }
    }
    rc = launch_prefill_attention(p, dtype, stream);
    if (rc != PKV_EUNSUPPORTED) return rc;
    clear_error();
    if (p.app_slots) {
        // prefill_tuned() promised the MFMA kernel would write the rows; it did not run,
        // so append them before the pool-only kernels below read it.
        p.app_k = p.app_v = nullptr;
        p.app_slots = nullptr;
        rc = pkv_kv_append(const_cast<void*>(k_pool), const_cast<void*>(v_pool), pool_stride_block,
                           pool_stride_slot, pool_stride_head, num_blocks, block_size, num_kv_heads, head_dim,
                           app->k_new, app->v_new, app->st, app->sh, app->slots, num_tokens, dtype, stream);
        if (rc) return rc;
    }
    if (dtype == PKV_FLOAT32) {
        rc = launch_prefill_f32_mfma(p, stream);
        if (rc != PKV_EUNSUPPORTED) return rc;
        rc = launch_f32_attention(p, stream);
        if (rc != PKV_EUNSUPPORTED) return rc;
    }
    return launch_generic_attention(p, dtype, stream);
}

}  // namespace
}  // namespace pkv

extern "C" int pkv_paged_attention_prefill(
    void* out, int64_t out_stride_t, int64_t out_stride_h, const void* query, int64_t q_stride_t,
    int64_t q_stride_h, const void* k_pool, const void* v_pool, int64_t pool_stride_block, int64_t pool_stride_slot,
    int64_t pool_stride_head, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
    const int64_t* block_tables, int64_t table_stride, int64_t table_width, const int64_t* context_lens,
    const int64_t* query_start_loc, int64_t num_seqs, int64_t num_heads, int64_t num_tokens, int64_t max_query_len,
    float scale, int dtype, hipStream_t stream) {
    clear_error();
    return prefill_impl(out, out_stride_t, out_stride_h, query, q_stride_t, q_stride_h, k_pool, v_pool,
                        pool_stride_block, pool_stride_slot, pool_stride_head, num_blocks, block_size, num_kv_heads,
                        head_dim, block_tables, table_stride, table_width, context_lens, query_start_loc, num_seqs,
                        num_heads, num_tokens, max_query_len, scale, dtype, nullptr, stream);
}

extern "C" int pkv_paged_attention_prefill_append(
    void* out, int64_t out_stride_t, int64_t out_stride_h, const void* query, int64_t q_stride_t,
    int64_t q_stride_h, void* k_pool, void* v_pool, int64_t pool_stride_block, int64_t pool_stride_slot,
    int64_t pool_stride_head, int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
    const void* k_new, const void* v_new, int64_t new_stride_t, int64_t new_stride_h, const int64_t* slots,
    const int64_t* block_tables, int64_t table_stride, int64_t table_width, const int64_t* context_lens,
    const int64_t* query_start_loc, int64_t num_seqs, int64_t num_heads, int64_t num_tokens, int64_t max_query_len,
    float scale, int dtype, hipStream_t stream) {
    clear_error();
    if (num_tokens > 0 && (!k_new || !v_new || !slots))
        return fail(PKV_EINVAL, "paged_attention_prefill_append: null pointer");
    const DecodeAppend app{k_new, v_new, new_stride_t, new_stride_h, slots};
    return prefill_impl(out, out_stride_t, out_stride_h, query, q_stride_t, q_stride_h, k_pool, v_pool,
                        pool_stride_block, pool_stride_slot, pool_stride_head, num_blocks, block_size, num_kv_heads,
                        head_dim, block_tables, table_stride, table_width, context_lens, query_start_loc, num_seqs,
                        num_heads, num_tokens, max_query_len, scale, dtype, &app, stream);
}
