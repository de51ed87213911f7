// Elementwise maps, last-axis mean and concatenation: the decoder glue that
// the reference's ElementwiseImpl / MeanImpl / CatImpl families serve
// (kuipy/kuiops.py:150-320, 810-921).  All three are HBM-bound byte movers:
// every kernel reads each input element once and writes each output element
// once, with 16-byte accesses wherever the layout allows.
//
//   * ew_contig_kernel: every tensor operand is contiguous with the output's
//     shape (or a single broadcast element); a thread maps 8 consecutive
//     elements with vector loads sized by each operand's dtype.
//   * ew_strided_kernel: broadcasting / strided operands; the host collapses
//     the iteration space to its fewest dims, each thread decomposes its
//     linear output index once and walks every operand's strides.
//   * mean_rows_kernel: one wave (n < 8192) or one 256-thread work-group per
//     row, fp32 (fp64 for fp64) accumulation, times 1/n as aten's mean.
//   * cat_kernel: grid.y = input; each input's rows are copied into their
//     column range of the output rows, 16 bytes per lane when aligned.
//
// Arithmetic follows aten's "opmath" rule: 16-bit floats are computed in fp32
// and rounded once on store; python scalars enter as the compute type,
// unrounded.  Floating-point contraction is off so that a*b + c rounds as
// aten's separate operations do; add / sub with alpha use an explicit fma as
// aten's alpha kernels do.
#include "common.hpp"

#include <type_traits>

#pragma clang fp contract(off)

namespace kuiops {

constexpr int kEwMaxIn = 3;
constexpr int kEwMaxRank = 8;

struct EwArgs {
    const void *in[kEwMaxIn];
    int in_dt[kEwMaxIn];
    int64_t in_stride[kEwMaxIn][kEwMaxRank];   // elements; 0 = broadcast
    int64_t shape[kEwMaxRank];
    int rank;
    int n_in;
    int out_dt;
    void *out;
    int64_t numel;
    double s0, s1;                              // alpha / exponent, scalar operand
};

// ------------------------------------------------------------- load / store
template <typename C>
__device__ __forceinline__ C load_one(const void *p, int64_t i, int dt) {
    switch (dt) {
        case KUIOPS_F32: return (C)reinterpret_cast<const float *>(p)[i];
        case KUIOPS_BF16: return (C)(float)reinterpret_cast<const bf16_t *>(p)[i];
        case KUIOPS_F16: return (C)(float)reinterpret_cast<const f16_t *>(p)[i];
        case KUIOPS_F64: return (C)reinterpret_cast<const double *>(p)[i];
        case KUIOPS_I64: return (C)reinterpret_cast<const int64_t *>(p)[i];
        case KUIOPS_I32: return (C)reinterpret_cast<const int32_t *>(p)[i];
        case KUIOPS_I16: return (C)reinterpret_cast<const int16_t *>(p)[i];
        case KUIOPS_I8: return (C)reinterpret_cast<const int8_t *>(p)[i];
        default: return (C)reinterpret_cast<const uint8_t *>(p)[i];     // U8, BOOL
    }
}

template <typename C>
__device__ __forceinline__ void store_one(void *p, int64_t i, int dt, C v) {
    switch (dt) {
        case KUIOPS_F32: reinterpret_cast<float *>(p)[i] = (float)v; break;
        case KUIOPS_BF16: reinterpret_cast<bf16_t *>(p)[i] = (bf16_t)(float)v; break;
        case KUIOPS_F16: reinterpret_cast<f16_t *>(p)[i] = (f16_t)(float)v; break;
        case KUIOPS_F64: reinterpret_cast<double *>(p)[i] = (double)v; break;
        case KUIOPS_I64: reinterpret_cast<int64_t *>(p)[i] = (int64_t)v; break;
        case KUIOPS_I32: reinterpret_cast<int32_t *>(p)[i] = (int32_t)v; break;
        case KUIOPS_I16: reinterpret_cast<int16_t *>(p)[i] = (int16_t)v; break;
        case KUIOPS_I8: reinterpret_cast<int8_t *>(p)[i] = (int8_t)v; break;
        case KUIOPS_BOOL: reinterpret_cast<uint8_t *>(p)[i] = v != (C)0; break;
        default: reinterpret_cast<uint8_t *>(p)[i] = (uint8_t)v; break;
    }
}

// 8 consecutive elements starting at i (16-byte aligned groups; the host
// checks every base pointer is 16-byte aligned).
template <typename C>
__device__ __forceinline__ void load8(const void *p, int64_t i, int dt, C v[8]) {
    switch (dt) {
        case KUIOPS_BF16: case KUIOPS_F16: {
            const u32x4 w = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const uint16_t *>(p) + i);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (dt == KUIOPS_BF16) {
                    v[2 * j] = (C)bf16lo(w[j]);
                    v[2 * j + 1] = (C)bf16hi(w[j]);
                } else {
                    v[2 * j] = (C)(float)__builtin_bit_cast(f16_t, (uint16_t)(w[j] & 0xffffu));
                    v[2 * j + 1] = (C)(float)__builtin_bit_cast(f16_t, (uint16_t)(w[j] >> 16));
                }
            }
            break;
        }
        case KUIOPS_F32: {
            const f32x4 *q = reinterpret_cast<const f32x4 *>(reinterpret_cast<const float *>(p) + i);
            const f32x4 a = q[0], b = q[1];
#pragma unroll
            for (int j = 0; j < 4; ++j) { v[j] = (C)a[j]; v[4 + j] = (C)b[j]; }
            break;
        }
        case KUIOPS_BOOL: case KUIOPS_U8: case KUIOPS_I8: {
            const u32x2 w = *reinterpret_cast<const u32x2 *>(reinterpret_cast<const uint8_t *>(p) + i);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t b = (w[j >> 2] >> (8 * (j & 3))) & 0xffu;
                v[j] = dt == KUIOPS_I8 ? (C)(int8_t)b : (C)b;
            }
            break;
        }
        default:
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = load_one<C>(p, i + j, dt);
    }
}

template <typename C>
__device__ __forceinline__ void store8(void *p, int64_t i, int dt, const C v[8]) {
    switch (dt) {
        case KUIOPS_BF16: case KUIOPS_F16: {
            u32x4 w;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint16_t lo, hi;
                if (dt == KUIOPS_BF16) {
                    lo = __builtin_bit_cast(uint16_t, (bf16_t)(float)v[2 * j]);
                    hi = __builtin_bit_cast(uint16_t, (bf16_t)(float)v[2 * j + 1]);
                } else {
                    lo = __builtin_bit_cast(uint16_t, (f16_t)(float)v[2 * j]);
                    hi = __builtin_bit_cast(uint16_t, (f16_t)(float)v[2 * j + 1]);
                }
                w[j] = (uint32_t)lo | ((uint32_t)hi << 16);
            }
            *reinterpret_cast<u32x4 *>(reinterpret_cast<uint16_t *>(p) + i) = w;
            break;
        }
        case KUIOPS_F32: {
            f32x4 a, b;
#pragma unroll
            for (int j = 0; j < 4; ++j) { a[j] = (float)v[j]; b[j] = (float)v[4 + j]; }
            f32x4 *q = reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(p) + i);
            q[0] = a;
            q[1] = b;
            break;
        }
        case KUIOPS_BOOL: {
            u32x2 w = {0u, 0u};
#pragma unroll
            for (int j = 0; j < 8; ++j) w[j >> 2] |= (uint32_t)(v[j] != (C)0) << (8 * (j & 3));
            *reinterpret_cast<u32x2 *>(reinterpret_cast<uint8_t *>(p) + i) = w;
            break;
        }
        default:
#pragma unroll
            for (int j = 0; j < 8; ++j) store_one<C>(p, i + j, dt, v[j]);
    }
}

// ------------------------------------------------------------------- ops
__device__ __forceinline__ double pow_scalar(double x, double e) {
    // aten's pow(Tensor, Scalar) special cases (exact products / roots)
    if (e == 2.0) return x * x;
    if (e == 3.0) return x * x * x;
    if (e == 1.0) return x;
    if (e == 0.5) return sqrt(x);
    if (e == -0.5) return 1.0 / sqrt(x);
    if (e == -1.0) return 1.0 / x;
    if (e == -2.0) return 1.0 / (x * x);
    return pow(x, e);
}
// 16-bit results: aten multiplies the integer powers in the storage type,
// so the square is rounded to it before the third factor / the reciprocal.
__device__ __forceinline__ float round_to(float x, int dt) {
    if (dt == KUIOPS_BF16) return (float)(bf16_t)x;
    if (dt == KUIOPS_F16) return (float)(f16_t)x;
    return x;
}

__device__ __forceinline__ float pow_scalar(float x, double e, int out_dt) {
    if (e == 2.0) return x * x;
    if (e == 3.0) return round_to(x * x, out_dt) * x;
    if (e == 1.0) return x;
    if (e == 0.5) return sqrtf(x);
    if (e == -0.5) return rsqrtf(x);
    if (e == -1.0) return 1.0f / x;
    if (e == -2.0) return 1.0f / round_to(x * x, out_dt);
    return powf(x, (float)e);
}
__device__ __forceinline__ double pow_scalar(double x, double e, int) { return pow_scalar(x, e); }

__device__ __forceinline__ float ew_fma(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double ew_fma(double a, double b, double c) { return __builtin_fma(a, b, c); }
__device__ __forceinline__ int64_t ew_fma(int64_t a, int64_t b, int64_t c) { return a * b + c; }

__device__ __forceinline__ float ew_rsqrt(float x) { return rsqrtf(x); }
__device__ __forceinline__ double ew_rsqrt(double x) { return 1.0 / sqrt(x); }
__device__ __forceinline__ float ew_exp(float x) { return expf(x); }
__device__ __forceinline__ double ew_exp(double x) { return exp(x); }

constexpr bool float_only_op(int op) {
    return op == KUIOPS_EW_DIV || op == KUIOPS_EW_SILU || op == KUIOPS_EW_RSQRT || op == KUIOPS_EW_COS ||
           op == KUIOPS_EW_SIN || op == KUIOPS_EW_EXP || op == KUIOPS_EW_SQRT || op == KUIOPS_EW_POW_SCALAR;
}

template <int OP, typename C>
__device__ __forceinline__ C apply(C a, C b, C c, double s0, int out_dt) {
    if constexpr (OP == KUIOPS_EW_ADD) return s0 == 1.0 ? a + b : ew_fma((C)s0, b, a);
    else if constexpr (OP == KUIOPS_EW_SUB) return s0 == 1.0 ? a - b : ew_fma((C)(-s0), b, a);
    else if constexpr (OP == KUIOPS_EW_MUL) return a * b;
    else if constexpr (OP == KUIOPS_EW_NEG) return -a;
    else if constexpr (OP == KUIOPS_EW_EQ) return (C)(a == b);
    else if constexpr (OP == KUIOPS_EW_NE) return (C)(a != b);
    else if constexpr (OP == KUIOPS_EW_LE) return (C)(a <= b);
    else if constexpr (OP == KUIOPS_EW_LT) return (C)(a < b);
    else if constexpr (OP == KUIOPS_EW_GE) return (C)(a >= b);
    else if constexpr (OP == KUIOPS_EW_GT) return (C)(a > b);
    else if constexpr (OP == KUIOPS_EW_WHERE) return a != (C)0 ? b : c;
    else if constexpr (std::is_integral<C>::value) return a;      // float-only ops: refused on the host
    else if constexpr (OP == KUIOPS_EW_DIV) return a / b;
    else if constexpr (OP == KUIOPS_EW_SILU) return a / ((C)1 + ew_exp(-a));
    else if constexpr (OP == KUIOPS_EW_RSQRT) return ew_rsqrt(a);
    else if constexpr (OP == KUIOPS_EW_COS) return cos(a);
    else if constexpr (OP == KUIOPS_EW_SIN) return sin(a);
    else if constexpr (OP == KUIOPS_EW_EXP) return ew_exp(a);
    else if constexpr (OP == KUIOPS_EW_SQRT) return sqrt(a);
    else if constexpr (OP == KUIOPS_EW_POW_SCALAR) return pow_scalar(a, s0, out_dt);
    else return a;
}

// Bitwise ops on integer / bool operands (computed in int64).
template <int OP>
__device__ __forceinline__ int64_t apply_bits(int64_t a, int64_t b, int out_dt) {
    switch (OP) {
        case KUIOPS_EW_BITWISE_NOT: return out_dt == KUIOPS_BOOL ? (int64_t)(a == 0) : ~a;
        case KUIOPS_EW_BITWISE_AND: return a & b;
        case KUIOPS_EW_BITWISE_OR: return a | b;
        default: return a;
    }
}

constexpr bool is_bit_op(int op) {
    return op == KUIOPS_EW_BITWISE_NOT || op == KUIOPS_EW_BITWISE_AND || op == KUIOPS_EW_BITWISE_OR;
}

template <int OP, typename C>
__device__ __forceinline__ C apply_any(C a, C b, C c, const EwArgs &A) {
    if constexpr (is_bit_op(OP)) return (C)apply_bits<OP>((int64_t)a, (int64_t)b, A.out_dt);
    else return apply<OP, C>(a, b, c, A.s0, A.out_dt);
}

// Operand j of the op: an input tensor, or (binary ops given one tensor) the
// scalar s1.
template <typename C>
__device__ __forceinline__ C scalar_operand(const EwArgs &A) { return (C)A.s1; }

template <int OP, typename C>
__global__ __launch_bounds__(256) void ew_contig_kernel(EwArgs A) {
    const int64_t groups = A.numel >> 3;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups; g += stride) {
        const int64_t i = g << 3;
        C v[kEwMaxIn][8];
#pragma unroll
        for (int k = 0; k < kEwMaxIn; ++k) {
            if (k < A.n_in) {
                if (A.in_stride[k][0] == 0) {        // a single broadcast element
                    const C x = load_one<C>(A.in[k], 0, A.in_dt[k]);
#pragma unroll
                    for (int j = 0; j < 8; ++j) v[k][j] = x;
                } else {
                    load8<C>(A.in[k], i, A.in_dt[k], v[k]);
                }
            } else {
                const C x = scalar_operand<C>(A);
#pragma unroll
                for (int j = 0; j < 8; ++j) v[k][j] = x;
            }
        }
        C r[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = apply_any<OP, C>(v[0][j], v[1][j], v[2][j], A);
        store8<C>(A.out, i, A.out_dt, r);
    }
    // tail (numel % 8 elements): the first threads of block 0
    const int64_t t = (groups << 3) + threadIdx.x;
    if (blockIdx.x == 0 && t < A.numel) {
        C x[kEwMaxIn];
#pragma unroll
        for (int k = 0; k < kEwMaxIn; ++k)
            x[k] = k < A.n_in ? load_one<C>(A.in[k], A.in_stride[k][0] == 0 ? 0 : t, A.in_dt[k])
                              : scalar_operand<C>(A);
        store_one<C>(A.out, t, A.out_dt, apply_any<OP, C>(x[0], x[1], x[2], A));
    }
}

template <int OP, typename C>
__global__ __launch_bounds__(256) void ew_strided_kernel(EwArgs A) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < A.numel; i += stride) {
        int64_t off[kEwMaxIn] = {0, 0, 0};
        int64_t rem = i;
        for (int d = A.rank - 1; d >= 0; --d) {
            const int64_t sz = A.shape[d];
            const int64_t q = rem / sz;
            const int64_t c = rem - q * sz;
            rem = q;
#pragma unroll
            for (int k = 0; k < kEwMaxIn; ++k) off[k] += c * A.in_stride[k][d];
        }
        C x[kEwMaxIn];
#pragma unroll
        for (int k = 0; k < kEwMaxIn; ++k)
            x[k] = k < A.n_in ? load_one<C>(A.in[k], off[k], A.in_dt[k]) : scalar_operand<C>(A);
        store_one<C>(A.out, i, A.out_dt, apply_any<OP, C>(x[0], x[1], x[2], A));
    }
}

// ---------------------------------------------------------------- host side
static bool is_float_dt(int dt) { return dt == KUIOPS_F32 || dt == KUIOPS_F16 || dt == KUIOPS_BF16 || dt == KUIOPS_F64; }
static bool is_int_dt(int dt) {
    return dt == KUIOPS_I64 || dt == KUIOPS_I32 || dt == KUIOPS_I16 || dt == KUIOPS_I8 || dt == KUIOPS_U8 ||
           dt == KUIOPS_BOOL;
}

static int ew_arity(int op) {
    switch (op) {
        case KUIOPS_EW_NEG: case KUIOPS_EW_SILU: case KUIOPS_EW_RSQRT: case KUIOPS_EW_COS: case KUIOPS_EW_SIN:
        case KUIOPS_EW_EXP: case KUIOPS_EW_SQRT: case KUIOPS_EW_POW_SCALAR: case KUIOPS_EW_BITWISE_NOT:
            return 1;
        case KUIOPS_EW_WHERE: return 3;
        case KUIOPS_EW_ADD: case KUIOPS_EW_SUB: case KUIOPS_EW_MUL: case KUIOPS_EW_DIV: case KUIOPS_EW_EQ:
        case KUIOPS_EW_NE: case KUIOPS_EW_LE: case KUIOPS_EW_LT: case KUIOPS_EW_GE: case KUIOPS_EW_GT:
        case KUIOPS_EW_BITWISE_AND: case KUIOPS_EW_BITWISE_OR:
            return 2;
        default: return 0;
    }
}

template <int OP, typename C>
static int ew_launch(const EwArgs &a, bool contig, hipStream_t st) {
    const int64_t work = contig ? cdiv(a.numel, 8) : a.numel;
    int64_t blocks = cdiv(work, 256);
    const int64_t cap = (int64_t)num_cus() * 16;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    if (contig) hipLaunchKernelGGL((ew_contig_kernel<OP, C>), dim3((unsigned)blocks), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((ew_strided_kernel<OP, C>), dim3((unsigned)blocks), dim3(256), 0, st, a);
    return launch_status();
}

template <int OP>
static int ew_by_compute(const EwArgs &a, int compute_dt, bool contig, hipStream_t st) {
    if constexpr (is_bit_op(OP)) {
        return ew_launch<OP, int64_t>(a, contig, st);
    } else {
        switch (compute_dt) {
            case KUIOPS_F64: return ew_launch<OP, double>(a, contig, st);
            case KUIOPS_I64: return ew_launch<OP, int64_t>(a, contig, st);
            default: return ew_launch<OP, float>(a, contig, st);
        }
    }
}

static int ew_dispatch(int op, const EwArgs &a, int compute_dt, bool contig, hipStream_t st) {
    switch (op) {
#define KUIOPS_EW_CASE(X) case X: return ew_by_compute<X>(a, compute_dt, contig, st);
        KUIOPS_EW_CASE(KUIOPS_EW_ADD) KUIOPS_EW_CASE(KUIOPS_EW_SUB) KUIOPS_EW_CASE(KUIOPS_EW_MUL)
        KUIOPS_EW_CASE(KUIOPS_EW_DIV) KUIOPS_EW_CASE(KUIOPS_EW_NEG) KUIOPS_EW_CASE(KUIOPS_EW_SILU)
        KUIOPS_EW_CASE(KUIOPS_EW_RSQRT) KUIOPS_EW_CASE(KUIOPS_EW_COS) KUIOPS_EW_CASE(KUIOPS_EW_SIN)
        KUIOPS_EW_CASE(KUIOPS_EW_EXP) KUIOPS_EW_CASE(KUIOPS_EW_SQRT) KUIOPS_EW_CASE(KUIOPS_EW_POW_SCALAR)
        KUIOPS_EW_CASE(KUIOPS_EW_EQ) KUIOPS_EW_CASE(KUIOPS_EW_NE) KUIOPS_EW_CASE(KUIOPS_EW_LE)
        KUIOPS_EW_CASE(KUIOPS_EW_LT) KUIOPS_EW_CASE(KUIOPS_EW_GE) KUIOPS_EW_CASE(KUIOPS_EW_GT)
        KUIOPS_EW_CASE(KUIOPS_EW_WHERE) KUIOPS_EW_CASE(KUIOPS_EW_BITWISE_NOT)
        KUIOPS_EW_CASE(KUIOPS_EW_BITWISE_AND) KUIOPS_EW_CASE(KUIOPS_EW_BITWISE_OR)
#undef KUIOPS_EW_CASE
        default: return KUIOPS_E_INVALID;
    }
}

}  // namespace kuiops

using namespace kuiops;

extern "C" int kuiops_elementwise(int op, int rank, const int64_t *shape, int n_in, const int *in_dtypes,
                                  const void *const *in_ptrs, const int64_t *in_strides, double s0, double s1,
                                  int compute_dtype, int out_dtype, void *out, void *stream) {
    const int arity = ew_arity(op);
    if (arity == 0 || rank < 0 || rank > kEwMaxRank || (rank > 0 && !shape)) return KUIOPS_E_INVALID;
    // binary ops may take their second operand as the scalar s1
    if (!(n_in == arity || (arity == 2 && n_in == 1))) return KUIOPS_E_INVALID;
    if (n_in > 0 && (!in_dtypes || !in_ptrs || (rank > 0 && !in_strides))) return KUIOPS_E_INVALID;
    int64_t numel = 1;
    for (int d = 0; d < rank; ++d) {
        if (shape[d] < 0) return KUIOPS_E_INVALID;
        numel *= shape[d];
    }
    if (numel == 0) return KUIOPS_OK;
    if (!out) return KUIOPS_E_INVALID;
    if (dtype_bytes(out_dtype) == 0) return KUIOPS_E_INVALID;
    if (compute_dtype != KUIOPS_F32 && compute_dtype != KUIOPS_F64 && compute_dtype != KUIOPS_I64)
        return KUIOPS_E_UNSUPPORTED;
    const bool bitop = op == KUIOPS_EW_BITWISE_NOT || op == KUIOPS_EW_BITWISE_AND || op == KUIOPS_EW_BITWISE_OR;
    if (float_only_op(op) && compute_dtype == KUIOPS_I64) return KUIOPS_E_UNSUPPORTED;
    if (bitop && !is_int_dt(out_dtype)) return KUIOPS_E_UNSUPPORTED;

    EwArgs a{};
    a.n_in = n_in;
    a.rank = rank;
    a.out = out;
    a.out_dt = out_dtype;
    a.numel = numel;
    a.s0 = s0;
    a.s1 = s1;
    bool contig = ((uintptr_t)out & 15) == 0;
    for (int k = 0; k < n_in; ++k) {
        if (!in_ptrs[k] || dtype_bytes(in_dtypes[k]) == 0) return KUIOPS_E_INVALID;
        if (bitop && !is_int_dt(in_dtypes[k])) return KUIOPS_E_UNSUPPORTED;
        if (!bitop && !(is_float_dt(in_dtypes[k]) || is_int_dt(in_dtypes[k]))) return KUIOPS_E_UNSUPPORTED;
        a.in[k] = in_ptrs[k];
        a.in_dt[k] = in_dtypes[k];
        // contiguous with the output's shape, or one broadcast element
        bool full = ((uintptr_t)in_ptrs[k] & 15) == 0, single = true;
        int64_t expect = 1;
        for (int d = rank - 1; d >= 0; --d) {
            const int64_t s = in_strides[k * rank + d];
            a.in_stride[k][d] = s;
            if (shape[d] != 1 && s != expect) full = false;
            if (shape[d] != 1 && s != 0) single = false;
            expect *= shape[d];
        }
        if (single) {
            for (int d = 0; d < kEwMaxRank; ++d) a.in_stride[k][d] = 0;
        } else if (!full) {
            contig = false;
        } else if (rank > 0) {
            a.in_stride[k][0] = 1;      // marker: contiguous (read as a flat array)
        }
    }
    for (int d = 0; d < rank; ++d) a.shape[d] = shape[d];
    if (contig && rank == 0) {
        for (int k = 0; k < n_in; ++k) a.in_stride[k][0] = 0;
    }
    if (!contig) {
        // the strided kernel reads the real strides again
        for (int k = 0; k < n_in; ++k)
            for (int d = 0; d < rank; ++d) a.in_stride[k][d] = in_strides[k * rank + d];
    }
    return ew_dispatch(op, a, compute_dtype, contig, as_stream(stream));
}

// ------------------------------------------------------------------- mean
namespace kuiops {

template <typename T, typename Acc, typename Tout>
__global__ __launch_bounds__(256) void mean_rows_kernel(const T *x, int64_t ldx, Tout *out, int64_t m, int64_t n,
                                                        Acc factor, int wave_rows) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (wave_rows) {
        const int64_t row = (int64_t)blockIdx.x * 4 + wave;
        if (row >= m) return;
        const T *xr = x + row * ldx;
        Acc acc = 0;
        for (int64_t j = lane; j < n; j += 64) acc += (Acc)to_f32_or_self(xr[j]);
        acc = wave_sum(acc);
        if (lane == 0) out[row] = (Tout)(acc * factor);
        return;
    }
    __shared__ Acc part[4];
    const int64_t row = blockIdx.x;
    const T *xr = x + row * ldx;
    Acc acc = 0;
    for (int64_t j = threadIdx.x; j < n; j += 256) acc += (Acc)to_f32_or_self(xr[j]);
    acc = wave_sum(acc);
    if (lane == 0) part[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[row] = (Tout)(((part[0] + part[1]) + (part[2] + part[3])) * factor);
}

template <typename T, typename Acc>
static int mean_launch(const void *x, int64_t ldx, void *out, int64_t m, int64_t n, hipStream_t st) {
    // aten scales the sum by (output numel / input numel), computed in the
    // accumulation type
    const Acc factor = (Acc)m / (Acc)(m * n);
    const int wave_rows = n < 8192;
    const dim3 grid((unsigned)(wave_rows ? cdiv(m, 4) : m));
    hipLaunchKernelGGL((mean_rows_kernel<T, Acc, T>), grid, dim3(256), 0, st, reinterpret_cast<const T *>(x), ldx,
                       reinterpret_cast<T *>(out), m, n, factor, wave_rows);
    return launch_status();
}

}  // namespace kuiops

extern "C" int kuiops_mean_lastdim(int64_t m, int64_t n, int dtype, const void *x, int64_t ldx, void *out,
                                   void *stream) {
    if (m < 0 || n < 0 || ldx < n) return KUIOPS_E_INVALID;
    if (m == 0) return KUIOPS_OK;
    if (!x || !out) return KUIOPS_E_INVALID;
    if (n == 0 || m > 0x7fffffff) return KUIOPS_E_UNSUPPORTED;
    hipStream_t st = as_stream(stream);
    switch (dtype) {
        case KUIOPS_F32: return mean_launch<float, float>(x, ldx, out, m, n, st);
        case KUIOPS_BF16: return mean_launch<bf16_t, float>(x, ldx, out, m, n, st);
        case KUIOPS_F16: return mean_launch<f16_t, float>(x, ldx, out, m, n, st);
        case KUIOPS_F64: return mean_launch<double, double>(x, ldx, out, m, n, st);
        default: return KUIOPS_E_UNSUPPORTED;
    }
}

// -------------------------------------------------------------------- cat
namespace kuiops {

constexpr int kCatMax = 32;

struct CatArgs {
    const char *in[kCatMax];
    int64_t width[kCatMax];      // bytes of one outer row of input i
    int64_t stride[kCatMax];     // bytes between outer rows of input i
    int64_t col[kCatMax];        // byte offset of input i inside an output row
    char *out;
    int64_t out_row;             // bytes of one output row
    int64_t outer;
};

template <int VB>
__global__ __launch_bounds__(256) void cat_kernel(CatArgs a) {
    typedef typename std::conditional<VB == 16, u32x4, typename std::conditional<VB == 8, u32x2,
            typename std::conditional<VB == 4, uint32_t, typename std::conditional<VB == 2, uint16_t,
            uint8_t>::type>::type>::type>::type V;
    const int i = blockIdx.y;
    const int64_t w = a.width[i] / VB;
    const int64_t total = w * a.outer;
    const char *src = a.in[i];
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += step) {
        const int64_t o = e / w;
        const int64_t j = e - o * w;
        *reinterpret_cast<V *>(a.out + o * a.out_row + a.col[i] + j * VB) =
            *reinterpret_cast<const V *>(src + o * a.stride[i] + j * VB);
    }
}

}  // namespace kuiops

extern "C" int kuiops_cat(int n_inputs, const void *const *inputs, const int64_t *widths,
                          const int64_t *outer_strides, int64_t outer, int elem_bytes, void *out, void *stream) {
    if (n_inputs < 0 || outer < 0 || (n_inputs > 0 && (!inputs || !widths || !outer_strides))) return KUIOPS_E_INVALID;
    if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) return KUIOPS_E_INVALID;
    if (n_inputs > kCatMax) return KUIOPS_E_UNSUPPORTED;
    CatArgs a{};
    int64_t row = 0;
    int vb = 16;
    for (int i = 0; i < n_inputs; ++i) {
        if (widths[i] < 0 || outer_strides[i] < 0) return KUIOPS_E_INVALID;
        if (widths[i] > 0 && outer > 0 && !inputs[i]) return KUIOPS_E_INVALID;
        a.in[i] = reinterpret_cast<const char *>(inputs[i]);
        a.width[i] = widths[i] * elem_bytes;
        a.stride[i] = outer_strides[i] * elem_bytes;
        a.col[i] = row;
        row += a.width[i];
        const uintptr_t bits = (uintptr_t)inputs[i] | (uintptr_t)a.width[i] | (uintptr_t)a.stride[i] | (uintptr_t)a.col[i];
        while (vb > elem_bytes && (bits & (vb - 1))) vb >>= 1;
    }
    if (row == 0 || outer == 0) return KUIOPS_OK;
    if (!out) return KUIOPS_E_INVALID;
    const uintptr_t obits = (uintptr_t)out | (uintptr_t)row;
    while (vb > elem_bytes && (obits & (vb - 1))) vb >>= 1;
    a.out = reinterpret_cast<char *>(out);
    a.out_row = row;
    a.outer = outer;
    int64_t maxw = 0;
    for (int i = 0; i < n_inputs; ++i) maxw = a.width[i] > maxw ? a.width[i] : maxw;
    int64_t blocks = cdiv(maxw / vb * outer, 256);
    const int64_t cap = (int64_t)num_cus() * 8;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    const dim3 grid((unsigned)blocks, (unsigned)n_inputs);
    hipStream_t st = as_stream(stream);
    switch (vb) {
        case 16: hipLaunchKernelGGL(cat_kernel<16>, grid, dim3(256), 0, st, a); break;
        case 8: hipLaunchKernelGGL(cat_kernel<8>, grid, dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL(cat_kernel<4>, grid, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL(cat_kernel<2>, grid, dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL(cat_kernel<1>, grid, dim3(256), 0, st, a); break;
    }
    return launch_status();
}
