// Greedy decode tail shared by the sampling library and the persistent
// decode-step kernel: softmax of one row followed by its arg-max (top-1 with
// aten.topk's ordering), and the decode-state advance.
#pragma once

#include "common.hpp"

namespace kuiops {

__device__ __forceinline__ float acc_exp(float x) { return __expf(x); }
__device__ __forceinline__ double acc_exp(double x) { return exp(x); }

// 32-bit key whose unsigned order is the float order (largest) or its
// reverse; NaN sorts above +inf, as aten.topk treats it.
__device__ __forceinline__ uint32_t order_key(float v, bool largest) {
    uint32_t b = __float_as_uint(v);
    uint32_t k;
    if (v != v) k = 0xffffffffu;                       // NaN: above everything
    else k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return largest ? k : ~k;                           // smallest: NaN lands last
}

constexpr int kSmThreads = 1024;
constexpr int kSmCache = 32;

// softmax + top-1 of the row X[0 .. n) (n <= kSmThreads * kSmCache), run by
// NTH threads of one work-group (NTH divides kSmThreads).  The arithmetic is
// that of a kSmThreads-thread work-group (virtual thread vt = tid + NTH * f
// holds elements vt + kSmThreads * j; sums run per virtual thread, per
// virtual wave, then over the virtual waves in order), so the probabilities
// are bitwise those of the softmax kernel.  The arg-max takes the largest
// probability at the lowest index (NaN largest).  Thread 0 writes the index
// (and the probability), records it at history[pos] when given, then
// advances the decode state: pos += 1, kv_len += 1 when given.  IO carries
// the reads of x.
template <typename T, int NTH, typename IO = PlainIO>
__device__ __forceinline__ void softmax_top1_row(int64_t n, const T *x, float *prob, int64_t *index, int32_t *pos,
                                                 int32_t *kv_len, int64_t *history, int64_t hist_len,
                                                 __attribute__((address_space(3))) char *stage = nullptr) {
    static_assert(kSmThreads % NTH == 0 && NTH % 64 == 0, "thread count");
    constexpr int F = kSmThreads / NTH;            // virtual threads per thread
    constexpr int VW = kSmThreads / 64;            // virtual waves
    typedef float A;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ A s_a[VW], s_b[VW];
    // the decode state is read up front, so the final writes wait on nothing
    int32_t pos0 = 0, kv0 = 0;
    if (tid == 0) {
        if (pos) pos0 = *pos;
        if (kv_len) kv0 = *kv_len;
    }
    A v[F][kSmCache];
    A m = -(A)INFINITY;
    // every load is issued before any is used: an index past the row reads
    // the last element (masked below), so no load sits behind a branch
    // (32-bit indices: n <= kSmThreads * kSmCache)
    const int nn = (int)n;
    if constexpr (__is_same(IO, PlainIO)) {
#pragma unroll
        for (int f = 0; f < F; ++f)
#pragma unroll
            for (int j = 0; j < kSmCache; ++j) {
                const int i = tid + NTH * f + kSmThreads * j;
                v[f][j] = (A)to_f32_or_self(x[i < nn ? i : nn - 1]);
            }
    } else {
        // written by other work-groups of the launch: the row goes through
        // `stage` (LDS, n * 2 bytes) by 16-byte agent-coherent (sc1) buffer
        // loads (2-byte coherent loads each cost a request past the L2)
        static_assert(sizeof(T) == 2, "coherent rows: 16-bit elements");
        typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
        typedef __attribute__((address_space(3))) T lds_t;
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<T *>(x), (short)0, nn * 2, 0x00020000);
        const int nch = (nn + 7) / 8;          // (a chunk past the row reads as zeros)
        constexpr int CPT = (kSmThreads * kSmCache / 8 + NTH - 1) / NTH;
        u32x4 c[CPT];
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int ch = tid + NTH * k;
            c[k] = ch < nch ? __builtin_amdgcn_raw_buffer_load_b128(rs, ch * 16, 0, kSc1Aux) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int ch = tid + NTH * k;
            if (ch < nch) reinterpret_cast<lds_u32x4 *>(stage)[ch] = c[k];
        }
        __syncthreads();
#pragma unroll
        for (int f = 0; f < F; ++f)
#pragma unroll
            for (int j = 0; j < kSmCache; ++j) {
                const int i = tid + NTH * f + kSmThreads * j;
                v[f][j] = (A)to_f32(reinterpret_cast<lds_t *>(stage)[i < nn ? i : nn - 1]);
            }
    }
    // maximum (a NaN anywhere makes it NaN, as aten's max does)
    bool has_nan = false;
#pragma unroll
    for (int f = 0; f < F; ++f)
#pragma unroll
        for (int j = 0; j < kSmCache; ++j) {
            const int i = tid + NTH * f + kSmThreads * j;
            if (i >= nn) v[f][j] = -(A)INFINITY;
            has_nan |= v[f][j] != v[f][j];
            m = fmaxf(m, v[f][j]);
        }
    m = wave_max(m);
    if (lane == 0) s_a[wave] = m;
    if (__syncthreads_or(has_nan)) m = __builtin_nanf("");
    else {
        m = s_a[0];
#pragma unroll
        for (int w = 1; w < NTH / 64; ++w) m = fmaxf(m, s_a[w]);
    }
    // Sums of e = exp(x - m) in the order of the kSmThreads-thread kernel.
    // The arg-max of p = e * (1 / sum): with m finite, e <= 1 and e == 1 at
    // the maximum, so the largest probability is exactly 1 / sum; another
    // element ties with it only when its e is 1, or 1 - 2^-24 and
    // (1 - 2^-24) / sum rounds to 1 / sum (any smaller e gives a smaller
    // product).  So the winner is the lowest index with e == 1, or with
    // e >= 1 - 2^-24 in that rounding case.  With m not finite (a NaN or an
    // infinity in the row) every probability is NaN: the winner is index 0.
    constexpr float kBelow1 = 1.f - 0x1p-24f;
    int i1 = INT32_MAX, i2 = INT32_MAX;
#pragma unroll
    for (int f = 0; f < F; ++f) {
        A s = 0;
#pragma unroll
        for (int j = 0; j < kSmCache; ++j) {
            const int i = tid + NTH * f + kSmThreads * j;
            const A e = acc_exp(v[f][j] - m);
            if (i < nn) s += e;
            i1 = (e == 1.f && i < i1) ? i : i1;
            i2 = (e == kBelow1 && i < i2) ? i : i2;
        }
        s = wave_sum(s);
        if (lane == 0) s_b[wave + (NTH / 64) * f] = s;
    }
    i1 = wave_min_i32(i1);
    i2 = wave_min_i32(i2);
    __shared__ int s_i1[NTH / 64], s_i2[NTH / 64];
    if (lane == 0) { s_i1[wave] = i1; s_i2[wave] = i2; }
    __syncthreads();
    if (tid == 0) {
        A sum = 0;
#pragma unroll
        for (int w = 0; w < VW; ++w) sum += s_b[w];
        const A inv = (A)1 / sum;
        int64_t i = 0;
        float p = __builtin_nanf("");
        if (m - m == 0.f) {                    // m finite
            int b1 = s_i1[0], b2 = s_i2[0];
#pragma unroll
            for (int w = 1; w < NTH / 64; ++w) {
                b1 = min(b1, s_i1[w]);
                b2 = min(b2, s_i2[w]);
            }
            i = (kBelow1 * inv == inv) ? min(b1, b2) : b1;
            p = inv;
        }
        *index = i;
        if (prob) *prob = p;
        if (history && pos && pos0 >= 0 && pos0 < hist_len) history[pos0] = i;
        if (pos) *pos = pos0 + 1;
        if (kv_len) *kv_len = kv0 + 1;
    }
}

}  // namespace kuiops
