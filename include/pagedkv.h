/*
 * pagedkv.h — C ABI of the MI355X (gfx950) paged-KV library `libpagedkv.so`.
 *
 * The library holds the device half of a paged-KV serving path: paged attention
 * (decode and prefill / chunked prefill), the KV append scatter, block copy for
 * copy-on-write, the gather/scatter halves of swap-out/swap-in, and greedy sampling
 * fused into the LM head. Everything else
 * (validation with the reference's exception texts, allocation, host bookkeeping)
 * stays in the Python host layer that binds this header with ctypes.
 *
 * Conventions shared by every entry point
 *   - Plain pointers and integers only. Device pointers are `void*` into HBM; the
 *     caller (PyTorch's caching allocator in the host layer) owns every buffer,
 *     including workspaces and pinned host buffers. The library never allocates or
 *     frees memory.
 *   - Strides are in ELEMENTS, not bytes. The innermost (head_dim) stride of every
 *     tensor operand must be 1.
 *   - `dtype` is one of PKV_FLOAT32 / PKV_FLOAT16 / PKV_BFLOAT16 and applies to the
 *     query, the output and both pools (they share one dtype, as in the reference).
 *   - Integer metadata (block tables, lengths, slots, block lists) is int64, exactly
 *     the LongTensors the reference builds, read in place with no conversion launch.
 *   - Every call is stream-ordered on the trailing `hipStream_t` (pass
 *     torch.cuda.current_stream().cuda_stream) and returns 0 on success or a
 *     PKV_E* code; `pkv_last_error()` then holds a message for the calling thread.
 *   - Library-wide state: the thread-local error string; per device, three lazily
 *     filled caches guarded by mutexes (the static split-KV scratch's device
 *     address, the CU count and each decode kernel's occupancy, the greedy kernel's
 *     dynamic-LDS opt-in); and the static scratch of pkv_paged_attention_decode_noalloc
 *     itself, shared by every call of that entry point on a device. Calls are
 *     reentrant; concurrent calls are safe when they use distinct workspaces and
 *     (for the no-alloc entry point) distinct devices.
 *   - The workspaces of the decode and greedy-sampling entry points carry the state of
 *     a merge inside the launch (arrival counters, keys): zero-fill each once, before
 *     its first use; every call that completes leaves that state zero again.
 *
 * Citations are to akshajravi/llm-inference-server, paths relative to its root.
 */
#ifndef PAGEDKV_H
#define PAGEDKV_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PKV_ABI_VERSION 1

enum pkv_dtype { PKV_FLOAT32 = 0, PKV_FLOAT16 = 1, PKV_BFLOAT16 = 2 };

enum pkv_status {
    PKV_OK = 0,
    PKV_EINVAL = 1,        /* bad argument: null pointer, negative size, bad stride */
    PKV_EUNSUPPORTED = 2,  /* shape/dtype combination this build has no kernel for */
    PKV_EWORKSPACE = 3,    /* workspace smaller than pkv_*_workspace_bytes() says */
    PKV_EHIP = 4           /* a HIP runtime call failed; message has hipGetErrorString */
};

/* ABI version of the loaded library; the host layer refuses a mismatch. */
int pkv_abi_version(void);

/* Message for the last non-zero return on this thread ("" if none). */
const char* pkv_last_error(void);

/* Count the nodes of a captured (not yet destroyed) hipGraph_t by type: counts[t]
 * += nodes of hipGraphNodeType t for t < num_types; types >= num_types land in
 * counts[num_types - 1]. counts is host memory the caller zeroes. No counterpart in
 * the reference: it is for callers that capture these kernels into HIP graphs (the
 * paged engine's decode-step graphs) and must show a graph holds no memset node
 * before instantiating it. Runs on this library's own HIP runtime, the one its
 * kernels launch through. */
int pkv_graph_node_counts(void* graph, int64_t* counts, int64_t num_types);

/* ------------------------------------------------------------------ attention
 * Paged attention over a block-major pool, the contract of the reference's
 * `paged_attention(query, k_pool, v_pool, block_tables, context_lens, query_lens,
 * scale)` (inference_server/core/attention.py:19-58, :73-88):
 *
 *   query        [num_tokens, num_heads, head_dim]      strides (q_stride_t, q_stride_h, 1)
 *   k/v pool     [num_blocks, block_size, num_kv_heads, head_dim]
 *                strides (pool_stride_block, pool_stride_slot, pool_stride_head, 1),
 *                identical for K and V
 *   block_tables int64 [num_seqs, table_width], row stride table_stride, 0-padded
 *   context_lens int64 [num_seqs]  tokens in the cache INCLUDING this pass's
 *   out          [num_tokens, num_heads, head_dim]      strides (out_stride_t, out_stride_h, 1)
 *
 * Token t of sequence i sits at logical position context_lens[i] - query_lens[i] + t
 * and attends to keys 0..that position (attention.py:44-53, :178-181). Query head h
 * reads KV head h / (num_heads / num_kv_heads) (attention.py:190-199). Softmax and
 * the P·V accumulator are float32, probabilities are rounded to dtype before P·V
 * (un-normalised, against a running max, where the gather path rounds normalised
 * ones), and the output is rounded once to dtype. Decode rounds the scores as the
 * gather path's tensors hold them (q·k rounded to dtype, then times scale rounded to
 * dtype); the MFMA prefill kernel keeps them in float32.
 * Keys at or beyond context_lens[i] are never read, so 0-padded table entries are
 * never dereferenced (tests/test_paged_attention.py:139-145).
 */

/* Workspace bytes pkv_paged_attention_decode needs for this batch shape: 256 KiB of
 * split-KV merge counters (one 32-bit word per (sequence, KV head)) followed by the
 * larger of two partial layouts: the partition kernels' (per sequence, query head and
 * 256-token partition: the running max, the softmax denominator and the unnormalised
 * output row, fp32; 768-token partitions use the first third of each row) and, for
 * batches the persistent MFMA kernel may take, its own (a prefix table plus one
 * partial per (workgroup, side, wave, head)). 0 when every context fits one 256-token
 * partition and the MFMA kernel does not apply (the output is then written directly).
 *
 * The counters must read zero when a call starts: zero-fill the workspace once before
 * its first use. Every call that runs to completion leaves them zero again (the
 * partition kernel's last partition of each (sequence, KV head) merges in place and
 * resets its counter; the MFMA kernel never touches them), and the partials need no
 * initialisation, so one workspace serves any later call on the same stream without
 * clearing. After a call that did not complete (a failed launch, an aborted stream, a
 * device reset) the counters may be dirty: zero-fill the workspace again (or use a
 * fresh zeroed one) before the next call. (A contract change: earlier builds of this
 * library needed no initialisation of the workspace.) */
int64_t pkv_paged_attention_decode_workspace_bytes(int64_t num_seqs, int64_t num_heads,
                                                   int64_t num_kv_heads, int64_t head_dim,
                                                   int64_t max_context_len);

/* Decode: every sequence has exactly one query token (query row i belongs to
 * sequence i). Replaces the all-decode branch of paged_attention_gather,
 * `_decode_batched` (inference_server/core/attention.py:125-153).
 * max_context_len is an upper bound on context_lens (table_width * block_size is
 * always valid); it sizes the split-KV grid, so a tight bound saves empty launches.
 * Kernels: fp16/bf16 batches whose K/V bound (num_seqs x num_kv_heads x
 * max_context_len x head_dim x 4 bytes) reaches 512 MiB, with a multiple of 4 KV heads
 * and at most 1024 sequences, run the persistent MFMA kernel (equal runs of 16-key
 * blocks per workgroup, then a small merge kernel for the sequences the runs cut);
 * other 16-bit batches run the partition kernel (768- or 256-token partitions, merged
 * in place or by a small second kernel), fp32 the register kernel plus its merge
 * kernel. All launch on the same stream; calls that overlap in time (different
 * streams) need distinct workspaces. */
int pkv_paged_attention_decode(
    void* out, int64_t out_stride_t, int64_t out_stride_h,
    const void* query, int64_t q_stride_t, int64_t q_stride_h,
    const void* k_pool, const void* v_pool,
    int64_t pool_stride_block, int64_t pool_stride_slot, int64_t pool_stride_head,
    int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
    const int64_t* block_tables, int64_t table_stride, int64_t table_width,
    const int64_t* context_lens,
    int64_t num_seqs, int64_t num_heads, int64_t max_context_len,
    float scale, int dtype,
    void* workspace, int64_t workspace_bytes,
    hipStream_t stream);

/* Decode step with its KV append fused in: writes row i of k_new / v_new
 * ([num_seqs, num_kv_heads, head_dim], element strides new_stride_t / new_stride_h,
 * unit innermost stride) into flat pool slot slots[i], then computes exactly what
 * pkv_paged_attention_decode computes over the updated pool (context_lens include the
 * new token). Replaces, per layer of a decode step, `_PagedCache.update`
 * (inference_server/core/paged_executor.py:116-125) followed by the decode attention
 * (inference_server/core/attention.py:130-153). With 16-bit pools on the tuned shapes
 * the streaming kernel writes each row itself, from the wave that reads that token
 * (no append launch); otherwise the append kernel runs first. Contract: slots[i] is
 * the slot of position context_lens[i] - 1 of sequence i, and no other sequence's
 * table reaches it (the reference's copy-on-write guarantees both); slots outside the
 * pool are skipped. Same workspace as pkv_paged_attention_decode. */
int pkv_paged_attention_decode_append(
    void* out, int64_t out_stride_t, int64_t out_stride_h,
    const void* query, int64_t q_stride_t, int64_t q_stride_h,
    void* k_pool, void* v_pool,
    int64_t pool_stride_block, int64_t pool_stride_slot, int64_t pool_stride_head,
    int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
    const void* k_new, const void* v_new, int64_t new_stride_t, int64_t new_stride_h,
    const int64_t* slots,
    const int64_t* block_tables, int64_t table_stride, int64_t table_width,
    const int64_t* context_lens,
    int64_t num_seqs, int64_t num_heads, int64_t max_context_len,
    float scale, int dtype,
    void* workspace, int64_t workspace_bytes,
    hipStream_t stream);

/* Bytes of the static device scratch that pkv_paged_attention_decode_noalloc keeps its
 * split-KV partials in: one buffer per device, held from the library's load onto that
 * device until the process ends. */
#define PKV_DECODE_SCRATCH_BYTES (96ll * 1024 * 1024)

/* No counterpart in the reference: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * pkv_paged_attention_decode without the workspace: the split-KV partials go to the
 * library's static scratch of PKV_DECODE_SCRATCH_BYTES on the current device (call it
 * with the stream's device current). Allocates nothing (no hipMalloc, hipFree or
 * allocating library routine). A batch whose partials need more than the scratch
 * (pkv_paged_attention_decode_workspace_bytes > PKV_DECODE_SCRATCH_BYTES) is refused
 * with PKV_EWORKSPACE before anything is launched. Every call on one device shares that
 * device's scratch and leaves its partials there: calls that overlap in time on one
 * device (different streams) race. The scratch needs no clearing: it starts zeroed,
 * every call leaves its merge counters zero again, and a call reads only the partials
 * it wrote. Output identical to pkv_paged_attention_decode's. */
int pkv_paged_attention_decode_noalloc(
    void* out, int64_t out_stride_t, int64_t out_stride_h,
    const void* query, int64_t q_stride_t, int64_t q_stride_h,
    const void* k_pool, const void* v_pool,
    int64_t pool_stride_block, int64_t pool_stride_slot, int64_t pool_stride_head,
    int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
    const int64_t* block_tables, int64_t table_stride, int64_t table_width,
    const int64_t* context_lens,
    int64_t num_seqs, int64_t num_heads, int64_t max_context_len,
    float scale, int dtype,
    hipStream_t stream);

/* General ragged batch: prefill, chunked prefill, recompute, or a mix with decode.
 * Replaces the `_ragged_loop` branch (inference_server/core/attention.py:156-187)
 * and the Triton launcher's per-token walk (core/attention_triton.py:239-305).
 * query_start_loc int64 [num_seqs + 1] is the exclusive prefix sum of query_lens
 * (`cu_query_lens` of core/attention_triton.py:129-150); tokens at or beyond
 * query_start_loc[num_seqs] belong to no sequence (a caller padding the batch to a
 * fixed size) and their output rows are unspecified. max_query_len bounds query_lens
 * (sizes the tile grid); 0 or a value above num_tokens is replaced by num_tokens. */
int pkv_paged_attention_prefill(
    void* out, int64_t out_stride_t, int64_t out_stride_h,
    const void* query, int64_t q_stride_t, int64_t q_stride_h,
    const void* k_pool, const void* v_pool,
    int64_t pool_stride_block, int64_t pool_stride_slot, int64_t pool_stride_head,
    int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
    const int64_t* block_tables, int64_t table_stride, int64_t table_width,
    const int64_t* context_lens, const int64_t* query_start_loc,
    int64_t num_seqs, int64_t num_heads, int64_t num_tokens, int64_t max_query_len,
    float scale, int dtype,
    hipStream_t stream);

/* Prefill / chunked-prefill step with its KV append fused in: row t of k_new / v_new
 * ([num_tokens, num_kv_heads, head_dim], element strides new_stride_t / new_stride_h,
 * unit innermost stride) goes to flat pool slot slots[t], and the attention is what
 * pkv_paged_attention_prefill computes over the updated pool. Replaces, per layer of a
 * prefill step, `_PagedCache.update` (inference_server/core/paged_executor.py:116-125)
 * followed by `_ragged_loop` (inference_server/core/attention.py:156-187). With 16-bit
 * pools on the tuned shapes (and 16-byte aligned rows) the MFMA kernel stages each
 * sequence's new positions straight from k_new / v_new and the workgroups write their
 * own tokens' rows into the pool (no append launch, no wait between workgroups);
 * otherwise the append kernel runs first. Contract: slots[t] is the slot of token t's
 * position (context_lens[i] - query_lens[i] + its index) in its own sequence's table,
 * private to it (the reference's copy-on-write guarantees it); slots outside the pool
 * are skipped, and tokens at or beyond query_start_loc[num_seqs] (padding) must carry
 * such slots. */
int pkv_paged_attention_prefill_append(
    void* out, int64_t out_stride_t, int64_t out_stride_h,
    const void* query, int64_t q_stride_t, int64_t q_stride_h,
    void* k_pool, void* v_pool,
    int64_t pool_stride_block, int64_t pool_stride_slot, int64_t pool_stride_head,
    int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
    const void* k_new, const void* v_new, int64_t new_stride_t, int64_t new_stride_h,
    const int64_t* slots,
    const int64_t* block_tables, int64_t table_stride, int64_t table_width,
    const int64_t* context_lens, const int64_t* query_start_loc,
    int64_t num_seqs, int64_t num_heads, int64_t num_tokens, int64_t max_query_len,
    float scale, int dtype,
    hipStream_t stream);

/* ------------------------------------------------------------------ KV append
 * Scatter this pass's new K/V rows into their pool slots. Replaces
 * `_PagedCache.update` (inference_server/core/paged_executor.py:116-125):
 *   pool.k[layer].view(-1, H, D).index_copy_(0, write_slots, k)   (and V)
 * k_new/v_new [num_tokens, num_kv_heads, head_dim] with strides (new_stride_t,
 * new_stride_h, 1) — the strided `key_states[0].transpose(0, 1)` view is accepted
 * as is. slots int64 [num_tokens], flat slot = block * block_size + offset
 * (core/block_table.py:143-159); slots must be distinct. Bytes are copied
 * bit-for-bit. Slots outside [0, num_blocks * block_size) are skipped (the host
 * layer raises before the call, as index_copy_ does). */
int pkv_kv_append(
    void* k_pool, void* v_pool,
    int64_t pool_stride_block, int64_t pool_stride_slot, int64_t pool_stride_head,
    int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
    const void* k_new, const void* v_new, int64_t new_stride_t, int64_t new_stride_h,
    const int64_t* slots, int64_t num_tokens, int dtype,
    hipStream_t stream);

/* QKV projection with the KV append in its epilogue (decode steps). Replaces, per
 * layer, HF GPT-2's fused QKV projection `c_attn` (Conv1D: addmm(bias, x, W), W
 * [in, q + 2 kv], split into Q, K, V) followed by `_PagedCache.update`
 * (inference_server/core/paged_executor.py:116-125): out[m] = x[m] . W + bias for
 * num_rows hidden rows, every column rounded once to the model dtype, and each K
 * and V element also stored at pool slot slots[m] (head (c - q_features) / head_dim
 * of the K or V part). weight_t is W transposed, [N, in_features] with row stride
 * weight_stride (in_features contiguous); N = q_features + 2 * num_kv_heads *
 * head_dim; out [num_rows, N] with row stride out_stride holds the whole projection;
 * bias [N] or NULL. fp16/bf16 only (else PKV_EUNSUPPORTED); in_features % 16 == 0,
 * x and weight rows 16-byte aligned, q_features and head_dim multiples of 4, output
 * and pool rows 8-byte aligned (else PKV_EUNSUPPORTED). Slots outside the pool are
 * skipped; slots must be distinct. Sized for decode batches (the weight is read once
 * per 16 to 64 rows). */
int pkv_qkv_append(
    const void* x, int64_t x_stride, const void* weight_t, int64_t weight_stride, const void* bias,
    int64_t num_rows, int64_t in_features, int64_t q_features, int64_t num_kv_heads, int64_t head_dim,
    void* out, int64_t out_stride,
    void* k_pool, void* v_pool,
    int64_t pool_stride_block, int64_t pool_stride_slot, int64_t pool_stride_head,
    int64_t num_blocks, int64_t block_size, const int64_t* slots, int dtype,
    hipStream_t stream);

/* All layers in one launch: k_pools/v_pools are DEVICE arrays of num_layers pool
 * base pointers (contiguous pools of one shape); layer l's new rows start at
 * k_new + l * new_stride_layer elements. Same per-layer semantics as
 * pkv_kv_append; one launch instead of 2 * num_layers index_copy_ calls. */
int pkv_kv_append_layers(
    void* const* k_pools, void* const* v_pools, int64_t num_layers,
    int64_t num_blocks, int64_t block_size, int64_t num_kv_heads, int64_t head_dim,
    const void* k_new, const void* v_new,
    int64_t new_stride_layer, int64_t new_stride_t, int64_t new_stride_h,
    const int64_t* slots, int64_t num_tokens, int dtype,
    hipStream_t stream);

/* ------------------------------------------------------------------ block copy
 * Copy-on-write: for every (src, dst) pair and every one of num_tensors pool
 * tensors, pool[dst] = pool[src] bit-for-bit. Replaces PagedExecutor._copy_block
 * (inference_server/core/paged_executor.py:265-270), reached through
 * BlockTable.ensure_private (core/block_table.py:110-134) — one launch for all
 * layers of K and V and any number of pairs, instead of 2 * L copy_ calls per pair.
 * tensors: DEVICE array of num_tensors contiguous pool base pointers (all K layers
 * then all V layers). pairs: int64 [num_pairs, 2] = (src, dst) block indices.
 * A dst must not also be a src of another pair in the same call. */
int pkv_copy_blocks(
    void* const* tensors, int64_t num_tensors, int64_t num_blocks, int64_t block_bytes,
    const int64_t* pairs, int64_t num_pairs,
    hipStream_t stream);

/* ------------------------------------------------------------------ swap
 * The device halves of a swap, for callers that run the host transfer on a copy
 * stream of their own. Gather: blocks[0..n) of every pool tensor into `staging`
 * (device, num_tensors * n * block_bytes, tensor-major then block order) — replaces
 * the per-layer `layer.index_select(0, idx)` of PagedKVPool.swap_out
 * (inference_server/core/kv_pool.py:157-161). Scatter: block i of every tensor in
 * `staging` into blocks[i] — replaces the per-layer `dst.index_copy_(0, idx, ...)` of
 * PagedKVPool.swap_in (inference_server/core/kv_pool.py:177-182). Stream-ordered;
 * ids outside [0, num_blocks) are skipped (never dereferenced; the host layer
 * range-checks first). */
int pkv_gather_blocks(
    void* const* tensors, int64_t num_tensors, int64_t num_blocks, int64_t block_bytes,
    const int64_t* blocks, int64_t num_swap_blocks,
    void* staging,
    hipStream_t stream);
int pkv_scatter_blocks(
    void* const* tensors, int64_t num_tensors, int64_t num_blocks, int64_t block_bytes,
    const int64_t* blocks, int64_t num_swap_blocks,
    const void* staging,
    hipStream_t stream);

/* Swap-out: gather blocks[0..n) of every pool tensor into `staging` (device,
 * num_tensors * n * block_bytes, tensor-major then block order) and copy it with
 * one hipMemcpyAsync into `host_dst` (pinned, same size and layout), so host_dst
 * holds [num_tensors][n][block] — the reference's HostBlocks per-layer
 * [n, block_size, kv_heads, head_dim] tensors back to back. Replaces
 * PagedKVPool.swap_out (inference_server/core/kv_pool.py:142-166). The copy is
 * stream-ordered: synchronize the stream before reading host_dst on the host. */
int pkv_swap_out(
    void* const* tensors, int64_t num_tensors, int64_t num_blocks, int64_t block_bytes,
    const int64_t* blocks, int64_t num_swap_blocks,
    void* staging, void* host_dst,
    hipStream_t stream);

/* Swap-in: one hipMemcpyAsync of host_src (pinned, layout as swap_out writes it)
 * into `staging`, then scatter block i of every tensor into blocks[i] (which need
 * not be the blocks it left). Replaces PagedKVPool.swap_in
 * (inference_server/core/kv_pool.py:168-182); the block-count check that raises
 * ValueError there lives in the host layer. host_src must stay alive and
 * unmodified until the stream passes this call. */
int pkv_swap_in(
    void* const* tensors, int64_t num_tensors, int64_t num_blocks, int64_t block_bytes,
    const int64_t* blocks, int64_t num_swap_blocks,
    void* staging, const void* host_src,
    hipStream_t stream);

/* ------------------------------------------------------------------ greedy sampling
 * Greedy next-token ids straight from the LM head, without the logits: out_ids[r] =
 * argmax over v < vocab_size of dot(hidden[r, :], weight[v, :]), each dot product
 * accumulated in fp32 and rounded to `dtype` before ranking, ties to the lowest index.
 * Replaces `logits[0, ends - 1, :].argmax(-1)` of PagedExecutor.execute
 * (inference_server/core/paged_executor.py:194-203), whose logits are the model's
 * bias-free LM head applied to the sampled rows; the [num_rows, vocab_size] logits
 * are never written. hidden: [num_rows, hidden_size], row stride hidden_stride;
 * weight: [vocab_size, hidden_size] (the LM head / tied embedding), row stride
 * weight_stride; both `dtype`, which must be PKV_FLOAT16 or PKV_BFLOAT16 (else
 * PKV_EUNSUPPORTED: the host layer keeps the matmul + argmax for fp32). hidden_size %
 * 16 == 0, strides % 8 == 0 and 16-byte aligned base pointers, else PKV_EUNSUPPORTED.
 * out_ids: int64 [num_rows]. One kernel launch; the keys of the rows are merged inside
 * it, and the merge keeps its state in `workspace`: at least
 * pkv_lm_head_argmax_workspace_bytes(num_rows, vocab_size) bytes (an arrival counter
 * and 8 keys per row), which must be zero-filled before its first use. Every call that
 * completes leaves it zero again, so one buffer serves every later call (any row count
 * it is large enough for) and every graph replay with no clearing. After a call that
 * did not complete (a launch error, a reset device) zero-fill it again. Calls that
 * overlap in time on one workspace (different streams) race. */
int64_t pkv_lm_head_argmax_workspace_bytes(int64_t num_rows, int64_t vocab_size);
int pkv_lm_head_argmax(
    const void* hidden, int64_t hidden_stride, const void* weight, int64_t weight_stride,
    int64_t num_rows, int64_t hidden_size, int64_t vocab_size, int dtype,
    int64_t* out_ids, void* workspace, int64_t workspace_bytes,
    hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PAGEDKV_H */
