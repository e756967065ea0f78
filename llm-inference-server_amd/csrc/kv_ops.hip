// KV append, block copy (copy-on-write) and the device halves of swap-out/in.
//
// All four are pure byte movement and HBM-bound: no arithmetic touches the data, so
// the kernels are written around one rule — every lane moves the widest unit the
// operands' alignment allows (16 bytes in every production shape), and consecutive
// lanes touch consecutive bytes of one row or block, so each wave issues fully
// coalesced 1 KiB loads and stores.
#include "pkv_common.h"

namespace pkv {
namespace {

// Widest power-of-two unit (<= 16 bytes) that divides every byte offset and pointer.
inline int copy_unit(uint64_t v) {
    if (v % 16 == 0) return 16;
    if (v % 8 == 0) return 8;
    if (v % 4 == 0) return 4;
    if (v % 2 == 0) return 2;
    return 1;
}

template <int U>
struct UnitT;
template <>
struct UnitT<16> { typedef uint4 type; };
template <>
struct UnitT<8> { typedef uint2 type; };
template <>
struct UnitT<4> { typedef uint32_t type; };
template <>
struct UnitT<2> { typedef uint16_t type; };
template <>
struct UnitT<1> { typedef uint8_t type; };

// ------------------------------------------------------------------ append
struct AppendArgs {
    char* k_pool;            // single-layer call: the layer's pools
    char* v_pool;
    void* const* k_pools;    // all-layer call: device tables of pool bases (else null)
    void* const* v_pools;
    const char* k_new;
    const char* v_new;
    const int64_t* slots;
    int64_t pool_stride_block, pool_stride_slot, pool_stride_head;  // bytes
    int64_t new_stride_layer, new_stride_t, new_stride_h;           // bytes
    int64_t num_slots;       // num_blocks * block_size
    int64_t block_size;
    int64_t num_tokens, num_kv_heads;
    int64_t units_per_row;   // head_dim * itemsize / unit
};

// Thread i copies unit (i % units_per_row) of row (i / units_per_row); a row is one
// (token, kv_head) slice of head_dim elements. blockIdx.y = layer * 2 + (0:K, 1:V).
template <int U>
__global__ __launch_bounds__(256) void kv_append_kernel(const AppendArgs a) {
    typedef typename UnitT<U>::type unit_t;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t rows = a.num_tokens * a.num_kv_heads;
    if (i >= rows * a.units_per_row) return;
    const int layer = (int)(blockIdx.y >> 1);
    const bool is_v = blockIdx.y & 1;
    const int64_t row = i / a.units_per_row;
    const int64_t u = i - row * a.units_per_row;
    const int64_t t = row / a.num_kv_heads;
    const int64_t h = row - t * a.num_kv_heads;
    const int64_t slot = a.slots[t];
    if (slot < 0 || slot >= a.num_slots) return;  // host layer raises before launch
    char* pool;
    if (a.k_pools) {
        pool = (char*)(is_v ? a.v_pools[layer] : a.k_pools[layer]);
    } else {
        pool = is_v ? a.v_pool : a.k_pool;
    }
    const char* src = (is_v ? a.v_new : a.k_new) + layer * a.new_stride_layer + t * a.new_stride_t +
                      h * a.new_stride_h;
    const int64_t blk = slot / a.block_size;
    const int64_t off = slot - blk * a.block_size;
    char* dst = pool + blk * a.pool_stride_block + off * a.pool_stride_slot + h * a.pool_stride_head;
    reinterpret_cast<unit_t*>(dst)[u] = reinterpret_cast<const unit_t*>(src)[u];
}

int launch_append(const AppendArgs& a0, int64_t head_dim, int itemsize, int64_t grid_y, uint64_t align_probe,
                  hipStream_t stream) {
    AppendArgs a = a0;
    const int U = copy_unit(align_probe | (uint64_t)(head_dim * itemsize));
    a.units_per_row = head_dim * itemsize / U;
    const int64_t total = a.num_tokens * a.num_kv_heads * a.units_per_row;
    if (total == 0) return PKV_OK;
    const int64_t grid_x = ceil_div(total, 256);
    if (grid_x > 0x7fffffff || grid_y > 65535) return fail(PKV_EUNSUPPORTED, "kv_append: grid too large");
    dim3 grid((unsigned)grid_x, (unsigned)grid_y);
    switch (U) {
        case 16: kv_append_kernel<16><<<grid, 256, 0, stream>>>(a); break;
        case 8: kv_append_kernel<8><<<grid, 256, 0, stream>>>(a); break;
        case 4: kv_append_kernel<4><<<grid, 256, 0, stream>>>(a); break;
        case 2: kv_append_kernel<2><<<grid, 256, 0, stream>>>(a); break;
        default: kv_append_kernel<1><<<grid, 256, 0, stream>>>(a); break;
    }
    return check_launch("kv_append");
}

int itemsize_of(int dtype) {
    switch (dtype) {
        case PKV_FLOAT32: return 4;
        case PKV_FLOAT16:
        case PKV_BFLOAT16: return 2;
        default: return 0;
    }
}

// ------------------------------------------------------------------ block moves
// One workgroup moves one block of one tensor: blockIdx.x = entry (pair or swap
// index), blockIdx.y = tensor. MODE 0: copy pool[src] -> pool[dst] (pairs);
// MODE 1: gather pool[blocks[i]] -> staging[tensor][i]; MODE 2: scatter back.
struct MoveArgs {
    void* const* tensors;
    const int64_t* index;    // pairs [n,2] (MODE 0) or blocks [n]
    char* staging;
    int64_t num_entries;
    int64_t num_blocks;
    int64_t block_bytes;
    int64_t units_per_block;
};

template <int MODE, int U>
__global__ __launch_bounds__(256) void block_move_kernel(const MoveArgs a) {
    typedef typename UnitT<U>::type unit_t;
    const int64_t e = blockIdx.x;
    const int64_t tensor = blockIdx.y;
    char* base = (char*)a.tensors[tensor];
    const unit_t* src;
    unit_t* dst;
    if (MODE == 0) {
        const int64_t s = a.index[2 * e], d = a.index[2 * e + 1];
        if (s < 0 || s >= a.num_blocks || d < 0 || d >= a.num_blocks) return;
        src = reinterpret_cast<const unit_t*>(base + s * a.block_bytes);
        dst = reinterpret_cast<unit_t*>(base + d * a.block_bytes);
    } else {
        const int64_t b = a.index[e];
        if (b < 0 || b >= a.num_blocks) return;
        char* pool_block = base + b * a.block_bytes;
        char* stage_block = a.staging + (tensor * a.num_entries + e) * a.block_bytes;
        src = reinterpret_cast<const unit_t*>(MODE == 1 ? pool_block : stage_block);
        dst = reinterpret_cast<unit_t*>(MODE == 1 ? stage_block : pool_block);
    }
    // 4 independent units in flight per lane before the stores.
    int64_t u = threadIdx.x;
    for (; u + 3 * 256 < a.units_per_block; u += 4 * 256) {
        unit_t x0 = src[u], x1 = src[u + 256], x2 = src[u + 512], x3 = src[u + 768];
        dst[u] = x0;
        dst[u + 256] = x1;
        dst[u + 512] = x2;
        dst[u + 768] = x3;
    }
    for (; u < a.units_per_block; u += 256) dst[u] = src[u];
}

template <int MODE>
int launch_move(MoveArgs a, int64_t num_tensors, uint64_t align_probe, hipStream_t stream, const char* what) {
    if (a.num_entries == 0 || num_tensors == 0 || a.block_bytes == 0) return PKV_OK;
    const int U = copy_unit(align_probe | (uint64_t)a.block_bytes);
    a.units_per_block = a.block_bytes / U;
    if (a.num_entries > 0x7fffffff || num_tensors > 65535) return fail(PKV_EUNSUPPORTED, "%s: grid too large", what);
    dim3 grid((unsigned)a.num_entries, (unsigned)num_tensors);
    switch (U) {
        case 16: block_move_kernel<MODE, 16><<<grid, 256, 0, stream>>>(a); break;
        case 8: block_move_kernel<MODE, 8><<<grid, 256, 0, stream>>>(a); break;
        case 4: block_move_kernel<MODE, 4><<<grid, 256, 0, stream>>>(a); break;
        case 2: block_move_kernel<MODE, 2><<<grid, 256, 0, stream>>>(a); break;
        default: block_move_kernel<MODE, 1><<<grid, 256, 0, stream>>>(a); break;
    }
    return check_launch(what);
}

int check_move_args(const char* what, void* const* tensors, int64_t num_tensors, int64_t num_blocks,
                    int64_t block_bytes, const void* index, int64_t n) {
    if (num_tensors < 0 || num_blocks < 0 || block_bytes < 0 || n < 0)
        return fail(PKV_EINVAL, "%s: negative size", what);
    if (n > 0 && num_tensors > 0 && (!tensors || !index)) return fail(PKV_EINVAL, "%s: null pointer", what);
    return PKV_OK;
}

}  // namespace
}  // namespace pkv

using namespace pkv;

extern "C" int pkv_kv_append(void* k_pool, void* v_pool, int64_t pool_stride_block, int64_t pool_stride_slot,
                             int64_t pool_stride_head, int64_t num_blocks, int64_t block_size,
                             int64_t num_kv_heads, int64_t head_dim, const void* k_new, const void* v_new,
                             int64_t new_stride_t, int64_t new_stride_h, const int64_t* slots,
                             int64_t num_tokens, int dtype, hipStream_t stream) {
    clear_error();
    const int isz = itemsize_of(dtype);
    if (!isz) return fail(PKV_EINVAL, "kv_append: unknown dtype %d", dtype);
    if (num_tokens < 0 || num_blocks <= 0 || block_size <= 0 || num_kv_heads <= 0 || head_dim <= 0)
        return fail(PKV_EINVAL, "kv_append: bad sizes");
    if (num_tokens == 0) return PKV_OK;
    if (!k_pool || !v_pool || !k_new || !v_new || !slots) return fail(PKV_EINVAL, "kv_append: null pointer");
    AppendArgs a = {};
    a.k_pool = (char*)k_pool;
    a.v_pool = (char*)v_pool;
    a.k_new = (const char*)k_new;
    a.v_new = (const char*)v_new;
    a.slots = slots;
    a.pool_stride_block = pool_stride_block * isz;
    a.pool_stride_slot = pool_stride_slot * isz;
    a.pool_stride_head = pool_stride_head * isz;
    a.new_stride_t = new_stride_t * isz;
    a.new_stride_h = new_stride_h * isz;
    a.num_slots = num_blocks * block_size;
    a.block_size = block_size;
    a.num_tokens = num_tokens;
    a.num_kv_heads = num_kv_heads;
    const uint64_t probe = (uint64_t)(uintptr_t)k_pool | (uint64_t)(uintptr_t)v_pool | (uint64_t)(uintptr_t)k_new |
                           (uint64_t)(uintptr_t)v_new | (uint64_t)a.pool_stride_block |
                           (uint64_t)a.pool_stride_slot | (uint64_t)a.pool_stride_head |
                           (uint64_t)a.new_stride_t | (uint64_t)a.new_stride_h;
    return launch_append(a, head_dim, isz, 2, probe, stream);
}

extern "C" int pkv_kv_append_layers(void* const* k_pools, void* const* v_pools, int64_t num_layers,
                                    int64_t num_blocks, int64_t block_size, int64_t num_kv_heads,
                                    int64_t head_dim, const void* k_new, const void* v_new,
                                    int64_t new_stride_layer, int64_t new_stride_t, int64_t new_stride_h,
                                    const int64_t* slots, int64_t num_tokens, int dtype, hipStream_t stream) {
    clear_error();
    const int isz = itemsize_of(dtype);
    if (!isz) return fail(PKV_EINVAL, "kv_append_layers: unknown dtype %d", dtype);
    if (num_tokens < 0 || num_layers < 0 || num_blocks <= 0 || block_size <= 0 || num_kv_heads <= 0 ||
        head_dim <= 0)
        return fail(PKV_EINVAL, "kv_append_layers: bad sizes");
    if (num_tokens == 0 || num_layers == 0) return PKV_OK;
    if (!k_pools || !v_pools || !k_new || !v_new || !slots)
        return fail(PKV_EINVAL, "kv_append_layers: null pointer");
    if (num_layers * 2 > 65535) return fail(PKV_EUNSUPPORTED, "kv_append_layers: too many layers");
    AppendArgs a = {};
    a.k_pools = k_pools;
    a.v_pools = v_pools;
    a.k_new = (const char*)k_new;
    a.v_new = (const char*)v_new;
    a.slots = slots;
    // Pools are contiguous [num_blocks, block_size, num_kv_heads, head_dim].
    a.pool_stride_head = head_dim * isz;
    a.pool_stride_slot = num_kv_heads * a.pool_stride_head;
    a.pool_stride_block = block_size * a.pool_stride_slot;
    a.new_stride_layer = new_stride_layer * isz;
    a.new_stride_t = new_stride_t * isz;
    a.new_stride_h = new_stride_h * isz;
    a.num_slots = num_blocks * block_size;
    a.block_size = block_size;
    a.num_tokens = num_tokens;
    a.num_kv_heads = num_kv_heads;
    // Pool bases come from torch's allocator (>= 256-byte aligned); probe the rest.
    const uint64_t probe = (uint64_t)(uintptr_t)k_new | (uint64_t)(uintptr_t)v_new | (uint64_t)a.new_stride_layer |
                           (uint64_t)a.new_stride_t | (uint64_t)a.new_stride_h | (uint64_t)a.pool_stride_head;
    return launch_append(a, head_dim, isz, 2 * num_layers, probe, stream);
}

extern "C" int pkv_copy_blocks(void* const* tensors, int64_t num_tensors, int64_t num_blocks, int64_t block_bytes,
                               const int64_t* pairs, int64_t num_pairs, hipStream_t stream) {
    clear_error();
    int rc = check_move_args("copy_blocks", tensors, num_tensors, num_blocks, block_bytes, pairs, num_pairs);
    if (rc) return rc;
    MoveArgs a = {};
    a.tensors = tensors;
    a.index = pairs;
    a.num_entries = num_pairs;
    a.num_blocks = num_blocks;
    a.block_bytes = block_bytes;
    return launch_move<0>(a, num_tensors, 0, stream, "copy_blocks");
}

namespace {
// Gather (MODE 1: blocks -> contiguous staging) or scatter (MODE 2: staging -> blocks)
// of every tensor's named blocks; staging is [num_tensors][n][block_bytes].
template <int MODE>
int move_staging(const char* what, void* const* tensors, int64_t num_tensors, int64_t num_blocks,
                 int64_t block_bytes, const int64_t* blocks, int64_t n, void* staging, hipStream_t stream) {
    int rc = check_move_args(what, tensors, num_tensors, num_blocks, block_bytes, blocks, n);
    if (rc) return rc;
    if (num_tensors * n * block_bytes == 0) return PKV_OK;
    if (!staging) return fail(PKV_EINVAL, "%s: null staging buffer", what);
    MoveArgs a = {};
    a.tensors = tensors;
    a.index = blocks;
    a.staging = (char*)staging;
    a.num_entries = n;
    a.num_blocks = num_blocks;
    a.block_bytes = block_bytes;
    return launch_move<MODE>(a, num_tensors, (uint64_t)(uintptr_t)staging, stream, what);
}
}  // namespace

extern "C" int pkv_gather_blocks(void* const* tensors, int64_t num_tensors, int64_t num_blocks, int64_t block_bytes,
                                 const int64_t* blocks, int64_t num_swap_blocks, void* staging, hipStream_t stream) {
    clear_error();
    return move_staging<1>("gather_blocks", tensors, num_tensors, num_blocks, block_bytes, blocks, num_swap_blocks,
                           staging, stream);
}

extern "C" int pkv_scatter_blocks(void* const* tensors, int64_t num_tensors, int64_t num_blocks, int64_t block_bytes,
                                  const int64_t* blocks, int64_t num_swap_blocks, const void* staging,
                                  hipStream_t stream) {
    clear_error();
    return move_staging<2>("scatter_blocks", tensors, num_tensors, num_blocks, block_bytes, blocks, num_swap_blocks,
                           const_cast<void*>(staging), stream);
}

extern "C" int pkv_swap_out(void* const* tensors, int64_t num_tensors, int64_t num_blocks, int64_t block_bytes,
                            const int64_t* blocks, int64_t num_swap_blocks, void* staging, void* host_dst,
                            hipStream_t stream) {
    clear_error();
    const int64_t total = num_tensors * num_swap_blocks * block_bytes;
    if (total > 0 && !host_dst) return fail(PKV_EINVAL, "swap_out: null host buffer");
    int rc = move_staging<1>("swap_out", tensors, num_tensors, num_blocks, block_bytes, blocks, num_swap_blocks,
                             staging, stream);
    if (rc || total <= 0) return rc;
    hipError_t e = hipMemcpyAsync(host_dst, staging, (size_t)total, hipMemcpyDeviceToHost, stream);
    if (e != hipSuccess) return fail(PKV_EHIP, "swap_out: hipMemcpyAsync: %s", hipGetErrorString(e));
    return PKV_OK;
}

extern "C" int pkv_swap_in(void* const* tensors, int64_t num_tensors, int64_t num_blocks, int64_t block_bytes,
                           const int64_t* blocks, int64_t num_swap_blocks, void* staging, const void* host_src,
                           hipStream_t stream) {
    clear_error();
    int rc = check_move_args("swap_in", tensors, num_tensors, num_blocks, block_bytes, blocks, num_swap_blocks);
    if (rc) return rc;
    const int64_t total = num_tensors * num_swap_blocks * block_bytes;
    if (total == 0) return PKV_OK;
    if (!staging || !host_src) return fail(PKV_EINVAL, "swap_in: null staging or host buffer");
    hipError_t e = hipMemcpyAsync(staging, host_src, (size_t)total, hipMemcpyHostToDevice, stream);
    if (e != hipSuccess) return fail(PKV_EHIP, "swap_in: hipMemcpyAsync: %s", hipGetErrorString(e));
    return move_staging<2>("swap_in", tensors, num_tensors, num_blocks, block_bytes, blocks, num_swap_blocks,
                           staging, stream);
}
