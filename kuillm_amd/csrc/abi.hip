// Library-level C ABI entry points: version, status strings and workspace
// sizing for every op that takes a workspace.
#include "common.hpp"

namespace kuiops {
size_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K);
size_t gemv_workspace_bytes(int64_t M, int64_t N, int64_t K);
size_t decode_workspace_bytes(int64_t rows, int64_t kv_len, int64_t ev);
size_t topk_workspace_bytes(int64_t rows, int64_t n, int64_t k);
size_t sort_workspace_bytes(int64_t m, int64_t n);
size_t decode_rows_batched_workspace_bytes(int64_t M, int64_t N, int64_t K);
}  // namespace kuiops

extern "C" int kuiops_abi_version(void) { return KUIOPS_ABI_VERSION; }

extern "C" const char *kuiops_status_string(int status) {
    switch (status) {
        case KUIOPS_OK: return "ok";
        case KUIOPS_E_UNSUPPORTED: return "unsupported shape or dtype";
        case KUIOPS_E_INVALID: return "invalid argument";
        case KUIOPS_E_HIP: return "HIP runtime error";
        case KUIOPS_E_WORKSPACE: return "workspace missing or too small";
        default: return "unknown status";
    }
}

extern "C" size_t kuiops_query_workspace(int op, int64_t a, int64_t b, int64_t c) {
    if (a < 0 || b < 0 || c < 0) return 0;
    switch (op) {
        case KUIOPS_OP_ADDMM: return kuiops::gemm_workspace_bytes(a, b, c);
        case KUIOPS_OP_GEMV_SPLITK: return kuiops::gemv_workspace_bytes(a, b, c);
        case KUIOPS_OP_SDPA_DECODE: return kuiops::decode_workspace_bytes(a, b, c);
        case KUIOPS_OP_TOPK: return kuiops::topk_workspace_bytes(a, b, c);
        case KUIOPS_OP_SORT: return kuiops::sort_workspace_bytes(a, b);
        case KUIOPS_OP_DECODE_ROWS_BATCHED: return kuiops::decode_rows_batched_workspace_bytes(a, b, c);
        default: return 0;
    }
}
