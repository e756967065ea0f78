// ABI version, the thread-local error string shared by every entry point, and the
// graph-node census for callers that capture the kernels into HIP graphs.
#include <stdarg.h>
#include <stdio.h>

#include <vector>

#include "pkv_common.h"

namespace pkv {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(PKV_EHIP, "%s: %s", what, hipGetErrorString(e));
    return PKV_OK;
}

}  // namespace pkv

extern "C" int pkv_abi_version(void) { return PKV_ABI_VERSION; }

extern "C" const char* pkv_last_error(void) { return pkv::g_last_error; }

extern "C" int pkv_graph_node_counts(void* graph, int64_t* counts, int64_t num_types) {
    pkv::clear_error();
    if (!graph || !counts || num_types <= 0) return pkv::fail(PKV_EINVAL, "graph_node_counts: bad argument");
    size_t n = 0;
    hipError_t e = hipGraphGetNodes(static_cast<hipGraph_t>(graph), nullptr, &n);
    if (e != hipSuccess) return pkv::fail(PKV_EHIP, "graph_node_counts: hipGraphGetNodes: %s", hipGetErrorString(e));
    std::vector<hipGraphNode_t> nodes(n);
    if (n) {
        e = hipGraphGetNodes(static_cast<hipGraph_t>(graph), nodes.data(), &n);
        if (e != hipSuccess)
            return pkv::fail(PKV_EHIP, "graph_node_counts: hipGraphGetNodes: %s", hipGetErrorString(e));
    }
    for (size_t i = 0; i < n; ++i) {
        hipGraphNodeType t;
        e = hipGraphNodeGetType(nodes[i], &t);
        if (e != hipSuccess)
            return pkv::fail(PKV_EHIP, "graph_node_counts: hipGraphNodeGetType: %s", hipGetErrorString(e));
        const int64_t k = (int64_t)t < num_types && (int64_t)t >= 0 ? (int64_t)t : num_types - 1;
        counts[k] += 1;
    }
    return PKV_OK;
}
