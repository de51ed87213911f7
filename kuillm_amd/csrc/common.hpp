// Shared device helpers for the gfx950 kuiops kernels: vector types, bf16/f16
// conversions, MFMA wrappers, wave64 reductions and launch-status plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include "kuiops.h"

namespace kuiops {

typedef __bf16 bf16_t;
typedef _Float16 f16_t;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- numerics
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(double x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return (float)x; }
__device__ __forceinline__ float to_f32(f16_t x) { return (float)x; }

// Accumulation-type view of an element: fp64 stays fp64, everything else fp32.
__device__ __forceinline__ float to_f32_or_self(float x) { return x; }
__device__ __forceinline__ double to_f32_or_self(double x) { return x; }
__device__ __forceinline__ float to_f32_or_self(bf16_t x) { return (float)x; }
__device__ __forceinline__ float to_f32_or_self(f16_t x) { return (float)x; }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ double from_f32<double>(float x) { return x; }
// bf16 / f16 conversions round to nearest even (the hardware converts used by
// the compiler on gfx950), matching torch's float -> bf16 / half casts.
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) { return (bf16_t)x; }
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float x) { return (f16_t)x; }

// Two raw 16-bit floats packed in a dword -> fp32 (bf16 is the top half of fp32).
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ------------------------------------------------------------------- MFMA
// 32x32x16 and 16x16x32 half-precision MFMAs of CDNA4.  Operand lanes hold 8
// consecutive K values; for 32x32: lane l -> row/col (l % 32), k 8*(l/32)..+7,
// acc[4*j+i] -> row 8*j + 4*(l/32) + i, col l % 32.  For 16x16: lane l ->
// row/col (l % 16), k 8*(l/16)..+7, acc[i] -> row 4*(l/16) + i, col l % 16.
template <typename T> struct Mfma;
template <> struct Mfma<bf16_t> {
    typedef bf16x8 frag;
    static __device__ __forceinline__ f32x16 m32(frag a, frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 m16(frag a, frag b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma<f16_t> {
    typedef f16x8 frag;
    static __device__ __forceinline__ f32x16 m32(frag a, frag b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ f32x4 m16(frag a, frag b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

template <typename F> __device__ __forceinline__ F as_frag(u32x4 v) {
    return __builtin_bit_cast(F, v);
}

// 8x8 transpose of 16-bit elements held as 8 rows of 4 dwords: in[r] holds
// row r (element c in half (c & 1) of dword c / 2); out[c] receives column c
// (element r in half (r & 1) of dword r / 2).
__device__ __forceinline__ void transpose8x8_b16(const u32x4 in[8], u32x4 out[8]) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint32_t lo = in[2 * e][c >> 1];
            uint32_t hi = in[2 * e + 1][c >> 1];
            // v_perm_b32 selector: bytes of (hi:lo); pick the low or high half of each.
            out[c][e] = (c & 1) ? __builtin_amdgcn_perm(hi, lo, 0x07060302u)
                                : __builtin_amdgcn_perm(hi, lo, 0x05040100u);
        }
    }
}

// 4x8 variant: in[r] (r < 4) rows of 8 elements; out[c] (c < 8) two dwords
// holding column c's 4 elements.
__device__ __forceinline__ void transpose4x8_b16(const u32x4 in[4], u32x2 out[8]) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            uint32_t lo = in[2 * e][c >> 1];
            uint32_t hi = in[2 * e + 1][c >> 1];
            out[c][e] = (c & 1) ? __builtin_amdgcn_perm(hi, lo, 0x07060302u)
                                : __builtin_amdgcn_perm(hi, lo, 0x05040100u);
        }
    }
}

// ------------------------------------------------------ I/O policies
// Loads / stores of the activations that the shared kernel bodies exchange.
// PlainIO: ordinary accesses (the data crosses a kernel boundary).
// CoherentIO: agent-scope relaxed atomic accesses, which gfx942 / gfx950
// perform with sc1 (stores written through the per-XCD L2, loads served
// past the non-coherent L1 / L2), for data exchanged between work-groups of
// one launch on different XCDs.  16-byte transfers go as two 8-byte atomics.
//
// Vector accesses used by the shared bodies (16-bit elements; idx an element
// index, a multiple of 8 for ld8 / st8 and of 2 for st2; ep the epoch of an
// epoch-tagged vector, ignored by the plain forms): ld8 reads 8 elements and
// reports whether they are the expected write (always, here), st8 / st2
// write 8 / 2 elements.
// Buffer-load cache policy bits for an agent-coherent (sc1) read.
constexpr int kSc1Aux = 16;

struct PlainIO {
    static constexpr bool kLL = false;
    template <typename V> static __device__ __forceinline__ V ld(const V *p) { return *p; }
    template <typename V> static __device__ __forceinline__ void st(V *p, V v) { *p = v; }
    static __device__ __forceinline__ bool ld8(const void *base, int64_t idx, uint32_t, u32x4 &v) {
        v = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const char *>(base) + idx * 2);
        return true;
    }
    static __device__ __forceinline__ void st8(void *base, int64_t idx, uint32_t, u32x4 v) {
        *reinterpret_cast<u32x4 *>(reinterpret_cast<char *>(base) + idx * 2) = v;
    }
    template <typename T> static __device__ __forceinline__ void st2(T *base, int64_t idx, T v0, T v1, uint32_t) {
        base[idx] = v0;
        base[idx + 1] = v1;
    }
};
struct CoherentIO {
    static constexpr bool kLL = false;
    template <typename V> static __device__ __forceinline__ V ld(const V *p) {
        static_assert(sizeof(V) == 16 || sizeof(V) == 8 || sizeof(V) == 4 || sizeof(V) == 2, "size");
        if constexpr (sizeof(V) == 16) {
            const uint64_t *q = reinterpret_cast<const uint64_t *>(p);
            typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
            const u64x2 r = {__hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                             __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)};
            return __builtin_bit_cast(V, r);
        } else if constexpr (sizeof(V) == 8) {
            return __builtin_bit_cast(V, __hip_atomic_load(reinterpret_cast<const uint64_t *>(p), __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT));
        } else if constexpr (sizeof(V) == 4) {
            return __builtin_bit_cast(V, __hip_atomic_load(reinterpret_cast<const uint32_t *>(p), __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT));
        } else {
            return __builtin_bit_cast(V, __hip_atomic_load(reinterpret_cast<const uint16_t *>(p), __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT));
        }
    }
    template <typename V> static __device__ __forceinline__ void st(V *p, V v) {
        static_assert(sizeof(V) == 16 || sizeof(V) == 8 || sizeof(V) == 4 || sizeof(V) == 2, "size");
        if constexpr (sizeof(V) == 16) {
            typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
            const u64x2 r = __builtin_bit_cast(u64x2, v);
            uint64_t *q = reinterpret_cast<uint64_t *>(p);
            __hip_atomic_store(q, r[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(q + 1, r[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else if constexpr (sizeof(V) == 8) {
            __hip_atomic_store(reinterpret_cast<uint64_t *>(p), __builtin_bit_cast(uint64_t, v), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        } else if constexpr (sizeof(V) == 4) {
            __hip_atomic_store(reinterpret_cast<uint32_t *>(p), __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        } else {
            __hip_atomic_store(reinterpret_cast<uint16_t *>(p), __builtin_bit_cast(uint16_t, v), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    static __device__ __forceinline__ bool ld8(const void *base, int64_t idx, uint32_t, u32x4 &v) {
        v = ld(reinterpret_cast<const u32x4 *>(reinterpret_cast<const char *>(base) + idx * 2));
        return true;
    }
    static __device__ __forceinline__ void st8(void *base, int64_t idx, uint32_t, u32x4 v) {
        st(reinterpret_cast<u32x4 *>(reinterpret_cast<char *>(base) + idx * 2), v);
    }
    template <typename T> static __device__ __forceinline__ void st2(T *base, int64_t idx, T v0, T v1, uint32_t) {
        st(base + idx, v0);
        st(base + idx + 1, v1);
    }
};


// Epoch-tagged vectors for data handed between work-groups of one launch:
// element pair (2w, 2w + 1) and the epoch of its write share the 8-byte word
// w (element 2w in the low 16 bits, the epoch in the high 32), written with
// one agent-coherent (sc1) store.  A reader knows which write it needs (its
// epoch) and polls the words themselves: no completion counter, and no
// wait for store acknowledgements before signalling.
struct LLIO {
    static constexpr bool kLL = true;
    static __device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7fffffff, 0x00020000);
    }
    static constexpr int kLdAux = kSc1Aux | (int)(1u << 31);     // sc1, volatile
    static __device__ __forceinline__ uint64_t word(const void *base, int64_t w) {
        return __hip_atomic_load(reinterpret_cast<const uint64_t *>(base) + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    static __device__ __forceinline__ void put(void *base, int64_t w, uint32_t pair, uint32_t ep) {
        __hip_atomic_store(reinterpret_cast<uint64_t *>(base) + w, (uint64_t)pair | ((uint64_t)ep << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // 8 elements (4 words) as two 16-byte agent-coherent (sc1) buffer
    // accesses; each 8-byte word of a 16-byte access is read or written
    // whole, so a word still carries its own element pair and epoch (a
    // reader may see one half of a chunk before the other, and then reads
    // again).  The loads are volatile: a polling loop re-issues them.
    static __device__ __forceinline__ bool ld8(const void *base, int64_t idx, uint32_t ep, u32x4 &v) {
        const __amdgpu_buffer_rsrc_t rs = rsrc(base);
        const uint32_t off = (uint32_t)(idx / 2) * 8u;
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, kLdAux);
        const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16u, 0, kLdAux);
        v = u32x4{a[0], a[2], b[0], b[2]};
        return a[1] == ep && a[3] == ep && b[1] == ep && b[3] == ep;
    }
    static __device__ __forceinline__ void st8(void *base, int64_t idx, uint32_t ep, u32x4 v) {
        const __amdgpu_buffer_rsrc_t rs = rsrc(base);
        const uint32_t off = (uint32_t)(idx / 2) * 8u;
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{v[0], ep, v[1], ep}, rs, off, 0, kSc1Aux);
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{v[2], ep, v[3], ep}, rs, off + 16u, 0, kSc1Aux);
    }
    template <typename T> static __device__ __forceinline__ void st2(T *base, int64_t idx, T v0, T v1, uint32_t ep) {
        const uint32_t pair = (uint32_t)__builtin_bit_cast(uint16_t, v0) | ((uint32_t)__builtin_bit_cast(uint16_t, v1) << 16);
        put(base, idx / 2, pair, ep);
    }
};

// ------------------------------------------------------- wave64 reductions
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ int wave_min_i32(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ double wave_max(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmax(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sum over aligned groups of N (2, 4, 8 or 16) lanes with DPP lane moves
// (no LDS round trip): quad swaps, then the half-row and row mirrors.  Each
// step adds two partial sums that are equal in both lanes of a pair, so every
// lane of a group ends with the bitwise same total.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(N == 2 || N == 4 || N == 8 || N == 16, "group size");
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));  // lane ^ 1
    if (N >= 4) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));  // lane ^ 2
    if (N >= 8) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)); // 7 - lane (in 8)
    if (N >= 16) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)); // 15 - lane (in 16)
    return v;
}

// Lane exchanges across lane bit 5, 4 or 3 without an LDS round trip
// (v_permlane32_swap / v_permlane16_swap on gfx950, DPP row rotate by 8).
// swap_rows<B>(x, y): in every lane, the pair {p, q} with p + q the sum of
// x over the lane and its partner (lane ^ B) when the lane's bit B is clear,
// and the sum of y over the pair when it is set.  Float addition commutes,
// so both partners' sums have the same bits.
template <int B>
__device__ __forceinline__ void swap_rows(float x, float y, float &p, float &q) {
    static_assert(B == 8 || B == 16 || B == 32, "lane bit");
    if constexpr (B == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
        p = __uint_as_float(r[0]);
        q = __uint_as_float(r[1]);
    } else if constexpr (B == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
        p = __uint_as_float(r[0]);
        q = __uint_as_float(r[1]);
    } else {
        const bool hi = (__lane_id() & 8) != 0;
        p = hi ? y : x;
        q = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(hi ? x : y), 0x128, 0xF, 0xF, false));
    }
}
// v + v of lane ^ B, the same bits in both lanes
template <int B>
__device__ __forceinline__ float xor_add(float v) {
    float p, q;
    swap_rows<B>(v, v, p, q);
    return p + q;
}
template <int B>
__device__ __forceinline__ float xor_max(float v) {
    float p, q;
    swap_rows<B>(v, v, p, q);
    return fmaxf(p, q);
}

// Value of lane ^ B, for lanes with bit B clear (lane + B).
template <int B>
__device__ __forceinline__ float from_lane_above(float v) {
    float p, q;
    swap_rows<B>(v, v, p, q);
    return q;
}
// Value of lane ^ 1 (DPP quad permute).
__device__ __forceinline__ int lane_xor1(int v) { return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false); }

// Wave total by lane moves only (DPP within rows of 16, then lane swaps
// across rows): every lane ends with the same bits.  (A different order
// from wave_sum.)
__device__ __forceinline__ float wave_sum_swaps(float v) {
    v = group_sum<16>(v);
    v = xor_add<16>(v);
    return xor_add<32>(v);
}

// a.x * b.x + a.y * b.y + c for packed pairs (fp32 accumulate)
template <typename T>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    if constexpr (__is_same(T, bf16_t)) {
        typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a), __builtin_bit_cast(bf2, b), c, false);
    } else {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
    }
}

constexpr unsigned kLLSpinLimit = 1u << 20;      // polls of one epoch-tagged wait (~1 s)
// s_sleep argument (units of 64 clocks) between two polls of an epoch-tagged
// wait: a poll reads past the per-XCD L2, so a longer pause trades wake-up
// latency for fabric traffic (persistent Llama-1B step: sleep 4 / 16 cost
// 3 / 17 us per token more than 1)
#ifndef KUIOPS_LL_SLEEP
#define KUIOPS_LL_SLEEP 1
#endif
constexpr int kLLSleep = KUIOPS_LL_SLEEP;

// Epoch-tagged waits spin per wave: a wave polls its own input words until
// all carry the expected epoch (a wave vote, no work-group reduction per
// poll), then the work-group meets at one barrier.  The expired-wait flag is
// read by each wave's lane 0 together with the wave's poll loads (checking
// it adds no memory round trip to a poll).
__device__ __forceinline__ unsigned ll_err_read(const unsigned *err) {
    return (err && (threadIdx.x & 63) == 0) ? __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                             : 0u;
}

// True (wave-uniform) when the wave's wait must stop at iteration `it`: its
// bound is reached (then *err is raised), or `e`, the flag read with the
// wave's last poll, shows that another wait raised it.  A stopped wait lets
// the work-group run on; the step's results are then void (*err is set).
__device__ __forceinline__ bool ll_expired(unsigned it, unsigned e, unsigned *err) {
    if (it >= kLLSpinLimit) {
        if (err && (threadIdx.x & 63) == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return true;
    }
    return __builtin_amdgcn_readfirstlane(e) != 0;
}

// --------------------------------------------------------------- host side
inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

inline int launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? KUIOPS_OK : KUIOPS_E_HIP;
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Compute units of the current device (queried once per device, then cached).
inline int num_cus() {
    static int cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

__host__ __device__ inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

inline int dtype_bytes(int dt) {
    switch (dt) {
        case KUIOPS_F32: case KUIOPS_I32: return 4;
        case KUIOPS_F16: case KUIOPS_BF16: case KUIOPS_I16: return 2;
        case KUIOPS_F64: case KUIOPS_I64: return 8;
        case KUIOPS_I8: case KUIOPS_U8: case KUIOPS_BOOL: return 1;
        default: return 0;
    }
}

}  // namespace kuiops
