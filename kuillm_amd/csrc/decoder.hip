// Decoder-layer glue around the hot path: residual add + RMSNorm, SwiGLU
// (silu(gate) * up), and rotary embedding fused with the KV-cache append.
//
// All three are HBM-bound elementwise/row kernels; each reads its operands
// once and writes its results once, 16 bytes per lane.  Rounding follows the
// bf16/f16 module code these kernels replace (each torch op rounds its
// result to the tensor dtype), so a decoder built on them tracks the stock
// PyTorch model op for op.  Floating-point contraction is off in this file:
// an FMA would skip the rounding of a product that the stock ops round.
#include "common.hpp"

#pragma clang fp contract(off)

namespace kuiops {

template <typename T>
__device__ __forceinline__ float rnd(float x) { return to_f32(from_f32<T>(x)); }

template <typename T>
__device__ __forceinline__ void unpack8(u32x4 raw, float *f) {
    typedef T t8 __attribute__((ext_vector_type(8)));
    const t8 v = __builtin_bit_cast(t8, raw);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = to_f32(v[e]);
}

template <typename T>
__device__ __forceinline__ u32x4 pack8f(const float *f) {
    typedef T t8 __attribute__((ext_vector_type(8)));
    t8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = from_f32<T>(f[e]);
    return __builtin_bit_cast(u32x4, v);
}

// ------------------------------------------------------------ RMSNorm

struct RmsArgs {
    int64_t m, n;
    const void *x; int64_t ldx;
    const void *res; int64_t ldr;      // optional residual added first
    void *res_out; int64_t ldro;       // optional: x + res (the new residual)
    const void *w;
    float eps;
    void *y; int64_t ldy;
};

// One work-group (256 lanes) per row; lane t holds chunks t, t + 256, ...
// of 8 elements in registers (n <= 8 * 256 * NC).
//   h = x (+ res, rounded)      y = w * round(h * rsqrt(mean(h^2) + eps))
template <typename T, int NC>
__global__ __launch_bounds__(256) void rmsnorm_kernel(RmsArgs a) {
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const T *x = reinterpret_cast<const T *>(a.x) + row * a.ldx;
    const T *r = a.res ? reinterpret_cast<const T *>(a.res) + row * a.ldr : nullptr;
    T *ro = a.res_out ? reinterpret_cast<T *>(a.res_out) + row * a.ldro : nullptr;
    float h[NC][8];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int64_t i = ((int64_t)c * 256 + tid) * 8;
        if (i < a.n) {
            unpack8<T>(*reinterpret_cast<const u32x4 *>(x + i), h[c]);
            if (r) {
                float rv[8];
                unpack8<T>(*reinterpret_cast<const u32x4 *>(r + i), rv);
#pragma unroll
                for (int e = 0; e < 8; ++e) h[c][e] = rnd<T>(h[c][e] + rv[e]);
            }
            if (ro) *reinterpret_cast<u32x4 *>(ro + i) = pack8f<T>(h[c]);
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += h[c][e] * h[c][e];
        }
    }
    __shared__ float part[4];
    ss = wave_sum(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    const float tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float inv = rsqrtf(tot / (float)a.n + a.eps);
    const T *w = reinterpret_cast<const T *>(a.w);
    T *y = reinterpret_cast<T *>(a.y) + row * a.ldy;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int64_t i = ((int64_t)c * 256 + tid) * 8;
        if (i < a.n) {
            float wv[8], o[8];
            unpack8<T>(*reinterpret_cast<const u32x4 *>(w + i), wv);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = wv[e] * rnd<T>(h[c][e] * inv);
            *reinterpret_cast<u32x4 *>(y + i) = pack8f<T>(o);
        }
    }
}

// ------------------------------------------------------------- SwiGLU

struct SiluMulArgs {
    int64_t m, n;
    const void *gu; int64_t ldg;       // row: [gate (n) | up (n)]
    void *out; int64_t ldo;
    int64_t chunks;                     // m * n / 8
};

//   out = round(round(silu(gate)) * up)
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(SiluMulArgs a) {
    const int64_t cpr = a.n / 8;
    for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < a.chunks; c += (int64_t)gridDim.x * 256) {
        const int64_t row = c / cpr, i = (c % cpr) * 8;
        const T *g = reinterpret_cast<const T *>(a.gu) + row * a.ldg + i;
        float gv[8], uv[8], o[8];
        unpack8<T>(*reinterpret_cast<const u32x4 *>(g), gv);
        unpack8<T>(*reinterpret_cast<const u32x4 *>(g + a.n), uv);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = rnd<T>(gv[e] / (1.f + expf(-gv[e]))) * uv[e];
        *reinterpret_cast<u32x4 *>(reinterpret_cast<T *>(a.out) + row * a.ldo + i) = pack8f<T>(o);
    }
}

// ------------------------------------------- rotary + KV-cache append

struct RopeArgs {
    int64_t n, t, hq, hkv, hd;
    const void *qkv; int64_t ld_tok, ld_batch;
    const float *inv_freq;             // [hd / 2]
    const int32_t *pos0;               // [n] first position of the t tokens (device), or null = 0
    void *q; int64_t sq0, sq1, sq2;
    void *kc; int64_t sk0, sk1, sk2;
    void *vc; int64_t sv0, sv1, sv2;
    int64_t cap;                       // cache positions; tokens at pos >= cap are not stored
};

// One work-group per (token, batch entry).  Rotation is the split-half form
// (x1, x2) -> (x1 cos - x2 sin, x2 cos + x1 sin) with angle pos * inv_freq[i]
// in fp32, cos / sin rounded to the tensor dtype, and each product and the
// sum rounded, as in the stock module code.
template <typename T>
__global__ __launch_bounds__(256) void rope_kv_kernel(RopeArgs a) {
    const int64_t ti = blockIdx.x, b = blockIdx.y;
    const int tid = threadIdx.x;
    const int64_t pos = (a.pos0 ? (int64_t)a.pos0[b] : 0) + ti;
    const bool store_kv = pos >= 0 && pos < a.cap;
    const T *row = reinterpret_cast<const T *>(a.qkv) + b * a.ld_batch + ti * a.ld_tok;
    const int64_t half = a.hd / 2;
    const int64_t nrot = (a.hq + a.hkv) * half;
    for (int64_t idx = tid; idx < nrot; idx += 256) {
        const int64_t h = idx / half, i = idx % half;
        const T *src = row + h * a.hd;
        const float x1 = to_f32(src[i]), x2 = to_f32(src[i + half]);
        const float ang = (float)pos * a.inv_freq[i];
        const float c = rnd<T>(cosf(ang)), s = rnd<T>(sinf(ang));
        const T o1 = from_f32<T>(rnd<T>(x1 * c) + rnd<T>(-x2 * s));
        const T o2 = from_f32<T>(rnd<T>(x2 * c) + rnd<T>(x1 * s));
        if (h < a.hq) {
            T *q = reinterpret_cast<T *>(a.q) + b * a.sq0 + h * a.sq1 + ti * a.sq2;
            q[i] = o1;
            q[i + half] = o2;
        } else if (store_kv) {
            T *k = reinterpret_cast<T *>(a.kc) + b * a.sk0 + (h - a.hq) * a.sk1 + pos * a.sk2;
            k[i] = o1;
            k[i + half] = o2;
        }
    }
    if (!store_kv) return;
    const int64_t cph = a.hd / 8;                     // 16-byte chunks per head
    const T *vsrc = row + (a.hq + a.hkv) * a.hd;
    for (int64_t idx = tid; idx < a.hkv * cph; idx += 256) {
        const int64_t h = idx / cph, c = idx % cph;
        T *v = reinterpret_cast<T *>(a.vc) + b * a.sv0 + h * a.sv1 + pos * a.sv2 + c * 8;
        *reinterpret_cast<u32x4 *>(v) = *reinterpret_cast<const u32x4 *>(vsrc + h * a.hd + c * 8);
    }
}

}  // namespace kuiops

using namespace kuiops;

extern "C" int kuiops_rmsnorm(int64_t m, int64_t n, int dtype, const void *x, int64_t ldx, const void *residual,
                              int64_t ldr, void *res_out, int64_t ldro, const void *weight, float eps, void *y,
                              int64_t ldy, void *stream) {
    if (m < 0 || n < 0) return KUIOPS_E_INVALID;
    if (m == 0 || n == 0) return KUIOPS_OK;
    if (!x || !weight || !y) return KUIOPS_E_INVALID;
    if (dtype != KUIOPS_BF16 && dtype != KUIOPS_F16) return KUIOPS_E_UNSUPPORTED;
    if (n % 8 || ldx % 8 || ldy % 8 || (residual && ldr % 8) || (res_out && ldro % 8)) return KUIOPS_E_UNSUPPORTED;
    if (!aligned16(x) || !aligned16(weight) || !aligned16(y) || (residual && !aligned16(residual)) ||
        (res_out && !aligned16(res_out)))
        return KUIOPS_E_UNSUPPORTED;
    if (m > INT32_MAX || n > 8 * 256 * 4) return KUIOPS_E_UNSUPPORTED;
    RmsArgs a{m, n, x, ldx, residual, ldr, res_out, ldro, weight, eps, y, ldy};
    hipStream_t st = as_stream(stream);
    const int nc = (int)cdiv(n, 8 * 256);
    const dim3 grid((unsigned)m);
#define KUIOPS_RMS(T)                                                                          \
    switch (nc) {                                                                              \
        case 1: hipLaunchKernelGGL((rmsnorm_kernel<T, 1>), grid, dim3(256), 0, st, a); break;  \
        case 2: hipLaunchKernelGGL((rmsnorm_kernel<T, 2>), grid, dim3(256), 0, st, a); break;  \
        default: hipLaunchKernelGGL((rmsnorm_kernel<T, 4>), grid, dim3(256), 0, st, a); break; \
    }
    if (dtype == KUIOPS_BF16) { KUIOPS_RMS(bf16_t) } else { KUIOPS_RMS(f16_t) }
#undef KUIOPS_RMS
    return launch_status();
}

extern "C" int kuiops_silu_mul(int64_t m, int64_t n, int dtype, const void *gate_up, int64_t ldg, void *out,
                               int64_t ldo, void *stream) {
    if (m < 0 || n < 0) return KUIOPS_E_INVALID;
    if (m == 0 || n == 0) return KUIOPS_OK;
    if (!gate_up || !out) return KUIOPS_E_INVALID;
    if (dtype != KUIOPS_BF16 && dtype != KUIOPS_F16) return KUIOPS_E_UNSUPPORTED;
    if (n % 8 || ldg % 8 || ldo % 8 || !aligned16(gate_up) || !aligned16(out)) return KUIOPS_E_UNSUPPORTED;
    SiluMulArgs a{m, n, gate_up, ldg, out, ldo, m * n / 8};
    int64_t blocks = cdiv(a.chunks, 256);
    if (blocks > 4096) blocks = 4096;
    hipStream_t st = as_stream(stream);
    if (dtype == KUIOPS_BF16) hipLaunchKernelGGL((silu_mul_kernel<bf16_t>), dim3((unsigned)blocks), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((silu_mul_kernel<f16_t>), dim3((unsigned)blocks), dim3(256), 0, st, a);
    return launch_status();
}

extern "C" int kuiops_rope_kv_append(int64_t n, int64_t t, int64_t hq, int64_t hkv, int64_t hd, int dtype,
                                     const void *qkv, int64_t ld_tok, int64_t ld_batch, const float *inv_freq,
                                     const int32_t *pos0, void *q_out, const int64_t sq[3], void *k_cache,
                                     const int64_t sk[3], void *v_cache, const int64_t sv[3], int64_t cache_cap,
                                     void *stream) {
    if (n < 0 || t < 0 || hq < 0 || hkv < 0 || hd <= 0 || cache_cap < 0) return KUIOPS_E_INVALID;
    if (n == 0 || t == 0) return KUIOPS_OK;
    if (!qkv || !inv_freq || !q_out || !k_cache || !v_cache || !sq || !sk || !sv) return KUIOPS_E_INVALID;
    if (dtype != KUIOPS_BF16 && dtype != KUIOPS_F16) return KUIOPS_E_UNSUPPORTED;
    if (hd % 8 || ld_tok % 8 || ld_batch % 8 || sv[0] % 8 || sv[1] % 8 || sv[2] % 8) return KUIOPS_E_UNSUPPORTED;
    if (!aligned16(qkv) || !aligned16(v_cache)) return KUIOPS_E_UNSUPPORTED;
    if (t > INT32_MAX || n > 65535) return KUIOPS_E_UNSUPPORTED;
    RopeArgs a{n, t, hq, hkv, hd, qkv, ld_tok, ld_batch, inv_freq, pos0,
               q_out, sq[0], sq[1], sq[2], k_cache, sk[0], sk[1], sk[2], v_cache, sv[0], sv[1], sv[2], cache_cap};
    const dim3 grid((unsigned)t, (unsigned)n);
    hipStream_t st = as_stream(stream);
    if (dtype == KUIOPS_BF16) hipLaunchKernelGGL((rope_kv_kernel<bf16_t>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((rope_kv_kernel<f16_t>), grid, dim3(256), 0, st, a);
    return launch_status();
}
