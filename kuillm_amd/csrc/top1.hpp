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

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long v, int off) {
    const uint32_t lo = __shfl_xor((uint32_t)v, off, 64), hi = __shfl_xor((uint32_t)(v >> 32), off, 64);
    return ((unsigned long long)hi << 32) | lo;
}

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
                                                 int32_t *kv_len, int64_t *history, int64_t hist_len) {
    static_assert(kSmThreads % NTH == 0 && NTH % 64 == 0, "thread count");
    constexpr int F = kSmThreads / NTH;            // virtual threads per thread
    constexpr int VW = kSmThreads / 64;            // virtual waves
    typedef float A;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ A s_a[VW], s_b[VW];
    __shared__ unsigned long long s_k[VW];
    // the decode state is read up front, so the final writes wait on nothing
    int32_t pos0 = 0, kv0 = 0;
    if (tid == 0) {
        if (pos) pos0 = *pos;
        if (kv_len) kv0 = *kv_len;
    }
    A v[F][kSmCache];
    A m = -(A)INFINITY;
    // every load is issued before any is used: an index past the row reads
    // the last element (masked below), so no load sits behind a branch (a
    // coherent load there would wait for its own round trip)
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
        // written by other work-groups of the launch: agent-coherent (sc1)
        // buffer loads, which unlike atomic loads issue back to back
        static_assert(sizeof(T) == 2, "coherent rows: 16-bit elements");
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<T *>(x), (short)0, nn * 2, 0x00020000);
#pragma unroll
        for (int f = 0; f < F; ++f)
#pragma unroll
            for (int j = 0; j < kSmCache; ++j) {
                const int i = tid + NTH * f + kSmThreads * j;
                const unsigned short b = __builtin_amdgcn_raw_buffer_load_b16(rs, (i < nn ? i : nn - 1) * 2, 0, kSc1Aux);
                v[f][j] = (A)to_f32(__builtin_bit_cast(T, b));
            }
    }
#pragma unroll
    for (int f = 0; f < F; ++f)
#pragma unroll
        for (int j = 0; j < kSmCache; ++j) {
            const int i = tid + NTH * f + kSmThreads * j;
            if (i >= nn) v[f][j] = -(A)INFINITY;
            m = (v[f][j] > m || v[f][j] != v[f][j]) ? v[f][j] : m;
        }
    m = wave_max(m);
    if (lane == 0) s_a[wave] = m;
    __syncthreads();
    m = s_a[0];
#pragma unroll
    for (int w = 1; w < NTH / 64; ++w) m = (s_a[w] > m || s_a[w] != s_a[w]) ? s_a[w] : m;
#pragma unroll
    for (int f = 0; f < F; ++f) {
        A s = 0;
#pragma unroll
        for (int j = 0; j < kSmCache; ++j) {
            v[f][j] = acc_exp(v[f][j] - m);
            if (tid + NTH * f + kSmThreads * j < nn) s += v[f][j];
        }
        s = wave_sum(s);
        if (lane == 0) s_b[wave + (NTH / 64) * f] = s;
    }
    __syncthreads();
    A s = 0;
#pragma unroll
    for (int w = 0; w < VW; ++w) s += s_b[w];
    const A inv = (A)1 / s;
    // (order key of the probability, complement of the index): the maximum
    // is the largest probability at the lowest index
    unsigned long long best = 0ull;
#pragma unroll
    for (int f = 0; f < F; ++f)
#pragma unroll
        for (int j = 0; j < kSmCache; ++j) {
            const int i = tid + NTH * f + kSmThreads * j;
            if (i >= nn) continue;
            const unsigned long long k = ((unsigned long long)order_key(v[f][j] * inv, true) << 32) |
                                         (0xffffffffu - (uint32_t)i);
            best = k > best ? k : best;
        }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = shfl_xor_u64(best, off);
        best = o > best ? o : best;
    }
    if (lane == 0) s_k[wave] = best;
    __syncthreads();
    if (tid == 0) {
        best = s_k[0];
#pragma unroll
        for (int w = 1; w < NTH / 64; ++w) best = s_k[w] > best ? s_k[w] : best;
        const int64_t i = (int64_t)(0xffffffffu - (uint32_t)best);
        *index = i;
        // the winner's probability is in the key: order_key of a value >= 0
        // is its bit pattern with the top bit set (NaN: all ones)
        const uint32_t pk = (uint32_t)(best >> 32);
        if (prob) *prob = pk == 0xffffffffu ? __builtin_nanf("") : __uint_as_float(pk & 0x7fffffffu);
        if (history && pos && pos0 >= 0 && pos0 < hist_len) history[pos0] = i;
        if (pos) *pos = pos0 + 1;
        if (kv_len) *kv_len = kv0 + 1;
    }
}

}  // namespace kuiops
