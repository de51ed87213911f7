// Index data movement for gfx950: torch.gather, aten.scatter.src and
// single-tensor aten.index.
// Pure data movement (bit-exact): each thread copies whole elements, and
// aten.index copies 16-byte chunks of the trailing (inner) block when the
// element run allows it.  Indices are consumed as int64 directly (no u32
// narrowing pass as in the reference's include/kuiops.h:28-36).
// Semantics: aten.gather (kuipy/kuiops.py:717-754,
// kuiops/gather/Kuiops.Gather.fst:482-486), aten.scatter.src
// (kuipy/kuiops.py:757-807) and aten.index.Tensor.
#include "common.hpp"

namespace kuiops {

constexpr int kMaxRank = 8;

struct GatherShape {
    int rank, dim;
    int64_t inp[kMaxRank], idx[kMaxRank];
    int64_t inp_stride[kMaxRank];
};

template <typename E>
__global__ __launch_bounds__(256) void gather_kernel(GatherShape g, int64_t total, const E *inp,
                                                     const int64_t *idx, E *out, int *err) {
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < total; o += (int64_t)gridDim.x * 256) {
        int64_t rem = o, off = 0;
        bool ok = true;
        const int64_t iv = idx[o];
        for (int d = g.rank - 1; d >= 0; --d) {
            const int64_t c = rem % g.idx[d];
            rem /= g.idx[d];
            int64_t cc = c;
            if (d == g.dim) {
                cc = iv;
                if (iv < 0 || iv >= g.inp[d]) ok = false;
            }
            off += cc * g.inp_stride[d];
        }
        if (ok) out[o] = inp[off];
        else {
            out[o] = E(0);
            if (err) *err = 1;
        }
    }
}

// out[x with axis dim replaced by idx[x]] = src[x] for every x of idx's shape
// (src has idx's shape); out already holds a copy of self.  Where indices
// repeat along dim, which of the writers lands is unspecified, as in aten.
template <typename E>
__global__ __launch_bounds__(256) void scatter_kernel(GatherShape g, int64_t total, const E *src,
                                                      const int64_t *idx, E *out, int *err) {
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < total; o += (int64_t)gridDim.x * 256) {
        int64_t rem = o, off = 0;
        bool ok = true;
        const int64_t iv = idx[o];
        for (int d = g.rank - 1; d >= 0; --d) {
            const int64_t c = rem % g.idx[d];
            rem /= g.idx[d];
            int64_t cc = c;
            if (d == g.dim) {
                cc = iv;
                if (iv < 0 || iv >= g.inp[d]) ok = false;
            }
            off += cc * g.inp_stride[d];
        }
        if (ok) out[off] = src[o];
        else if (err) *err = 1;
    }
}

// out[o][j][i] = inp[o][idx[j]][i];  V = copy unit (element or 16-byte chunk).
template <typename V>
__global__ __launch_bounds__(256) void index_kernel(int64_t outer, int64_t size, int64_t inner_v, int64_t n_idx,
                                                    const V *inp, const int64_t *idx, V *out, int *err) {
    const int64_t total = outer * n_idx * inner_v;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
        const int64_t i = t % inner_v;
        const int64_t r = t / inner_v;
        const int64_t j = r % n_idx, o = r / n_idx;
        int64_t v = idx[j];
        if (v < 0) v += size;
        if (v >= 0 && v < size) out[t] = inp[(o * size + v) * inner_v + i];
        else {
            out[t] = V{};
            if (err) *err = 1;
        }
    }
}

// aten.index.Tensor with k <= 8 index tensors on adjacent axes: inp viewed
// as (outer, size[0..k), inner), the k index tensors broadcast to n_pos
// positions (contiguous int64 each); out (outer, n_pos, inner).
constexpr int kMaxIdx = 8;
struct MultiIndex {
    const int64_t *idx[kMaxIdx];
    int64_t size[kMaxIdx];
    int k;
};

template <typename V>
__global__ __launch_bounds__(256) void index_multi_kernel(int64_t outer, int64_t span, int64_t inner_v, int64_t n_pos,
                                                          MultiIndex mi, const V *inp, V *out, int *err) {
    const int64_t total = outer * n_pos * inner_v;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
        const int64_t i = t % inner_v;
        const int64_t r = t / inner_v;
        const int64_t j = r % n_pos, o = r / n_pos;
        int64_t lin = 0;
        bool ok = true;
        for (int d = 0; d < mi.k; ++d) {
            int64_t v = mi.idx[d][j];
            if (v < 0) v += mi.size[d];
            ok = ok && v >= 0 && v < mi.size[d];
            lin = lin * mi.size[d] + v;
        }
        if (ok) out[t] = inp[(o * span + lin) * inner_v + i];
        else {
            out[t] = V{};
            if (err) *err = 1;
        }
    }
}

static unsigned grid_for(int64_t total) {
    int64_t b = cdiv(total, 256);
    if (b > 65536) b = 65536;
    return (unsigned)(b < 1 ? 1 : b);
}

}  // namespace kuiops

using namespace kuiops;

extern "C" int kuiops_gather(int rank, const int64_t *inp_shape, const int64_t *idx_shape, int dim, int elem_bytes,
                             const void *inp, const int64_t *idx, void *out, int *err_flag, void *stream) {
    if (rank < 1 || rank > kMaxRank || !inp_shape || !idx_shape || dim < 0 || dim >= rank) return KUIOPS_E_INVALID;
    GatherShape g{};
    g.rank = rank; g.dim = dim;
    int64_t total = 1;
    for (int d = 0; d < rank; ++d) {
        g.inp[d] = inp_shape[d];
        g.idx[d] = idx_shape[d];
        if (g.idx[d] < 0 || g.inp[d] < 0) return KUIOPS_E_INVALID;
        if (d != dim && g.idx[d] > g.inp[d]) return KUIOPS_E_INVALID;
        total *= g.idx[d];
    }
    if (total == 0) return KUIOPS_OK;
    if (!inp || !idx || !out) return KUIOPS_E_INVALID;
    int64_t st = 1;
    for (int d = rank - 1; d >= 0; --d) { g.inp_stride[d] = st; st *= g.inp[d]; }
    hipStream_t s = as_stream(stream);
    const unsigned grid = grid_for(total);
    switch (elem_bytes) {
        case 1: hipLaunchKernelGGL(gather_kernel<uint8_t>, dim3(grid), dim3(256), 0, s, g, total, (const uint8_t *)inp, idx, (uint8_t *)out, err_flag); break;
        case 2: hipLaunchKernelGGL(gather_kernel<uint16_t>, dim3(grid), dim3(256), 0, s, g, total, (const uint16_t *)inp, idx, (uint16_t *)out, err_flag); break;
        case 4: hipLaunchKernelGGL(gather_kernel<uint32_t>, dim3(grid), dim3(256), 0, s, g, total, (const uint32_t *)inp, idx, (uint32_t *)out, err_flag); break;
        case 8: hipLaunchKernelGGL(gather_kernel<uint64_t>, dim3(grid), dim3(256), 0, s, g, total, (const uint64_t *)inp, idx, (uint64_t *)out, err_flag); break;
        default: return KUIOPS_E_UNSUPPORTED;
    }
    return launch_status();
}

extern "C" int kuiops_scatter(int rank, const int64_t *out_shape, const int64_t *idx_shape, int dim, int elem_bytes,
                              const void *src, const int64_t *idx, void *out, int *err_flag, void *stream) {
    if (rank < 1 || rank > kMaxRank || !out_shape || !idx_shape || dim < 0 || dim >= rank) return KUIOPS_E_INVALID;
    GatherShape g{};
    g.rank = rank; g.dim = dim;
    int64_t total = 1;
    for (int d = 0; d < rank; ++d) {
        g.inp[d] = out_shape[d];
        g.idx[d] = idx_shape[d];
        if (g.idx[d] < 0 || g.inp[d] < 0) return KUIOPS_E_INVALID;
        if (d != dim && g.idx[d] > g.inp[d]) return KUIOPS_E_INVALID;
        total *= g.idx[d];
    }
    if (total == 0) return KUIOPS_OK;
    if (!src || !idx || !out) return KUIOPS_E_INVALID;
    int64_t st = 1;
    for (int d = rank - 1; d >= 0; --d) { g.inp_stride[d] = st; st *= g.inp[d]; }
    hipStream_t s = as_stream(stream);
    const unsigned grid = grid_for(total);
    switch (elem_bytes) {
        case 1: hipLaunchKernelGGL(scatter_kernel<uint8_t>, dim3(grid), dim3(256), 0, s, g, total, (const uint8_t *)src, idx, (uint8_t *)out, err_flag); break;
        case 2: hipLaunchKernelGGL(scatter_kernel<uint16_t>, dim3(grid), dim3(256), 0, s, g, total, (const uint16_t *)src, idx, (uint16_t *)out, err_flag); break;
        case 4: hipLaunchKernelGGL(scatter_kernel<uint32_t>, dim3(grid), dim3(256), 0, s, g, total, (const uint32_t *)src, idx, (uint32_t *)out, err_flag); break;
        case 8: hipLaunchKernelGGL(scatter_kernel<uint64_t>, dim3(grid), dim3(256), 0, s, g, total, (const uint64_t *)src, idx, (uint64_t *)out, err_flag); break;
        default: return KUIOPS_E_UNSUPPORTED;
    }
    return launch_status();
}

extern "C" int kuiops_index(int64_t outer, int64_t size, int64_t inner, int64_t n_idx, int elem_bytes, const void *inp,
                            const int64_t *idx, void *out, int *err_flag, void *stream) {
    if (outer < 0 || size < 0 || inner < 0 || n_idx < 0) return KUIOPS_E_INVALID;
    if (outer * n_idx * inner == 0) return KUIOPS_OK;
    if (!inp || !idx || !out) return KUIOPS_E_INVALID;
    hipStream_t s = as_stream(stream);
    const int64_t row_bytes = inner * elem_bytes;
    if (row_bytes % 16 == 0 && aligned16(inp) && aligned16(out)) {
        const int64_t iv = row_bytes / 16;
        hipLaunchKernelGGL(index_kernel<u32x4>, dim3(grid_for(outer * n_idx * iv)), dim3(256), 0, s, outer, size, iv,
                           n_idx, (const u32x4 *)inp, idx, (u32x4 *)out, err_flag);
        return launch_status();
    }
    const unsigned grid = grid_for(outer * n_idx * inner);
    switch (elem_bytes) {
        case 1: hipLaunchKernelGGL(index_kernel<uint8_t>, dim3(grid), dim3(256), 0, s, outer, size, inner, n_idx, (const uint8_t *)inp, idx, (uint8_t *)out, err_flag); break;
        case 2: hipLaunchKernelGGL(index_kernel<uint16_t>, dim3(grid), dim3(256), 0, s, outer, size, inner, n_idx, (const uint16_t *)inp, idx, (uint16_t *)out, err_flag); break;
        case 4: hipLaunchKernelGGL(index_kernel<uint32_t>, dim3(grid), dim3(256), 0, s, outer, size, inner, n_idx, (const uint32_t *)inp, idx, (uint32_t *)out, err_flag); break;
        case 8: hipLaunchKernelGGL(index_kernel<uint64_t>, dim3(grid), dim3(256), 0, s, outer, size, inner, n_idx, (const uint64_t *)inp, idx, (uint64_t *)out, err_flag); break;
        default: return KUIOPS_E_UNSUPPORTED;
    }
    return launch_status();
}

extern "C" int kuiops_index_multi(int64_t outer, int k, const int64_t *sizes, int64_t inner, int64_t n_pos,
                                  const int64_t *const *idx, int elem_bytes, const void *inp, void *out,
                                  int *err_flag, void *stream) {
    if (outer < 0 || inner < 0 || n_pos < 0 || k < 1 || !sizes || !idx) return KUIOPS_E_INVALID;
    if (k > kMaxIdx) return KUIOPS_E_UNSUPPORTED;
    MultiIndex mi{};
    mi.k = k;
    int64_t span = 1;
    for (int d = 0; d < k; ++d) {
        if (sizes[d] < 0) return KUIOPS_E_INVALID;
        mi.size[d] = sizes[d];
        mi.idx[d] = idx[d];
        span *= sizes[d];
    }
    if (outer * n_pos * inner == 0) return KUIOPS_OK;
    if (!inp || !out) return KUIOPS_E_INVALID;
    for (int d = 0; d < k; ++d)
        if (!idx[d]) return KUIOPS_E_INVALID;
    hipStream_t s = as_stream(stream);
    const int64_t row_bytes = inner * elem_bytes;
    if (row_bytes % 16 == 0 && aligned16(inp) && aligned16(out)) {
        const int64_t iv = row_bytes / 16;
        hipLaunchKernelGGL(index_multi_kernel<u32x4>, dim3(grid_for(outer * n_pos * iv)), dim3(256), 0, s, outer, span,
                           iv, n_pos, mi, (const u32x4 *)inp, (u32x4 *)out, err_flag);
        return launch_status();
    }
    const unsigned grid = grid_for(outer * n_pos * inner);
    switch (elem_bytes) {
        case 1: hipLaunchKernelGGL(index_multi_kernel<uint8_t>, dim3(grid), dim3(256), 0, s, outer, span, inner, n_pos, mi, (const uint8_t *)inp, (uint8_t *)out, err_flag); break;
        case 2: hipLaunchKernelGGL(index_multi_kernel<uint16_t>, dim3(grid), dim3(256), 0, s, outer, span, inner, n_pos, mi, (const uint16_t *)inp, (uint16_t *)out, err_flag); break;
        case 4: hipLaunchKernelGGL(index_multi_kernel<uint32_t>, dim3(grid), dim3(256), 0, s, outer, span, inner, n_pos, mi, (const uint32_t *)inp, (uint32_t *)out, err_flag); break;
        case 8: hipLaunchKernelGGL(index_multi_kernel<uint64_t>, dim3(grid), dim3(256), 0, s, outer, span, inner, n_pos, mi, (const uint64_t *)inp, (uint64_t *)out, err_flag); break;
        default: return KUIOPS_E_UNSUPPORTED;
    }
    return launch_status();
}
