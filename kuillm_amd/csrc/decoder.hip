// Decoder-layer glue around the hot path: residual add + RMSNorm, SwiGLU
// (silu(gate) * up), and rotary embedding fused with the KV-cache append.
//
// All three are HBM-bound elementwise/row kernels; each reads its operands
// once and writes its results once, 16 bytes per lane.  Rounding follows the
// bf16/f16 module code these kernels replace (each torch op rounds its
// result to the tensor dtype), so a decoder built on them tracks the stock
// PyTorch model op for op.  Floating-point contraction is off in this file:
// an FMA would skip the rounding of a product that the stock ops round.
#include "decode_rows.hpp"

#pragma clang fp contract(off)

namespace kuiops {

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
    // the norm weight is loaded with x (one memory round trip, not two)
    const T *w = reinterpret_cast<const T *>(a.w);
    u32x4 wr[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int64_t i = ((int64_t)c * 256 + tid) * 8;
        wr[c] = i < a.n ? *reinterpret_cast<const u32x4 *>(w + i) : u32x4{0, 0, 0, 0};
    }
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
    T *y = reinterpret_cast<T *>(a.y) + row * a.ldy;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int64_t i = ((int64_t)c * 256 + tid) * 8;
        if (i < a.n) {
            float wv[8], o[8];
            unpack8<T>(wr[c], wv);
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

// One 64-lane work-group per (token, batch entry, head) of the qkv row:
// q and k heads are rotated (lane i < hd / 2 owns the pair (i, i + hd / 2)),
// v heads are copied (lane i owns elements i, i + 64, ...).  Rotation is the
// split-half form (x1, x2) -> (x1 cos - x2 sin, x2 cos + x1 sin) with angle
// pos * inv_freq[i] in fp32, cos / sin rounded to the tensor dtype, and each
// product and the sum rounded, as in the stock module code.
template <typename T>
__global__ __launch_bounds__(64) void rope_kv_kernel(RopeArgs a) {
    const int64_t ti = blockIdx.x, b = blockIdx.y, h = blockIdx.z;
    const int lane = threadIdx.x;
    const int64_t pos = (a.pos0 ? (int64_t)a.pos0[b] : 0) + ti;
    const bool store_kv = pos >= 0 && pos < a.cap;
    const T *row = reinterpret_cast<const T *>(a.qkv) + b * a.ld_batch + ti * a.ld_tok;
    const int64_t half = a.hd / 2;
    if (h < a.hq + a.hkv) {
        if (h >= a.hq && !store_kv) return;
        for (int64_t i = lane; i < half; i += 64) {
            const float x1 = to_f32(row[h * a.hd + i]), x2 = to_f32(row[h * a.hd + i + half]);
            const float ang = (float)pos * a.inv_freq[i];
            const float c = rnd<T>(cosf(ang)), s = rnd<T>(sinf(ang));
            const T o1 = from_f32<T>(rnd<T>(x1 * c) + rnd<T>(-x2 * s));
            const T o2 = from_f32<T>(rnd<T>(x2 * c) + rnd<T>(x1 * s));
            T *dst = h < a.hq ? reinterpret_cast<T *>(a.q) + b * a.sq0 + h * a.sq1 + ti * a.sq2
                              : reinterpret_cast<T *>(a.kc) + b * a.sk0 + (h - a.hq) * a.sk1 + pos * a.sk2;
            dst[i] = o1;
            dst[i + half] = o2;
        }
        return;
    }
    if (!store_kv) return;
    const int64_t hv = h - a.hq - a.hkv;
    T *v = reinterpret_cast<T *>(a.vc) + b * a.sv0 + hv * a.sv1 + pos * a.sv2;
    for (int64_t i = lane; i < a.hd; i += 64) v[i] = row[h * a.hd + i];
}

template <typename T, int XK, int OK>
static void decode_rows_launch(const DecLinArgs &a, unsigned grid, hipStream_t st) {
    const int kc = (int)cdiv(a.K, 512);
    if (kc <= 4) hipLaunchKernelGGL((decode_rows_kernel<T, XK, 4, OK>), dim3(grid), dim3(256), 0, st, a);
    else if (kc <= 8) hipLaunchKernelGGL((decode_rows_kernel<T, XK, 8, OK>), dim3(grid), dim3(256), 0, st, a);
    else if constexpr (OK == kOutPlain) {
        if (kc <= 12) hipLaunchKernelGGL((decode_rows_kernel<T, XK, 12, OK>), dim3(grid), dim3(256), 0, st, a);
        else hipLaunchKernelGGL((decode_rows_kernel<T, XK, 16, OK>), dim3(grid), dim3(256), 0, st, a);
    }
}

template <typename T, int OK>
static void decode_rows_dispatch(const DecLinArgs &a, int x_kind, unsigned grid, hipStream_t st) {
    if (x_kind == kXPlain) decode_rows_launch<T, kXPlain, OK>(a, grid, st);
    else if (x_kind == kXRmsNorm) decode_rows_launch<T, kXRmsNorm, OK>(a, grid, st);
    else decode_rows_launch<T, kXSwiGlu, OK>(a, grid, st);
}

// log2(v) when v is a power of two, else -1.
static int log2_exact(int64_t v) {
    if (v <= 0 || (v & (v - 1))) return -1;
    int k = 0;
    while ((int64_t(1) << k) < v) ++k;
    return k;
}

// Shared host path of the decode projections: argument checks, rows per
// wave (the register group's size) and the launch.
template <int OK>
static int decode_linear_run(DecLinArgs a, int dtype, int x_kind, void *stream) {
    if (a.N < 0 || a.K < 0) return KUIOPS_E_INVALID;
    if (x_kind != kXPlain && x_kind != kXRmsNorm && x_kind != kXSwiGlu) return KUIOPS_E_INVALID;
    if (a.N == 0) return KUIOPS_OK;
    if (!a.in || !a.W || !a.out || (x_kind == kXRmsNorm && !a.norm_w)) return KUIOPS_E_INVALID;
    if (dtype != KUIOPS_BF16 && dtype != KUIOPS_F16) return KUIOPS_E_UNSUPPORTED;
    if (a.K == 0 || a.K % 8 || a.K > kDecodeMaxK || a.ldw % 8 || a.ldw < a.K) return KUIOPS_E_UNSUPPORTED;
    if (!aligned16(a.in) || !aligned16(a.W) || (a.in_add && !aligned16(a.in_add)) ||
        (a.norm_w && !aligned16(a.norm_w)) || (a.h_out && !aligned16(a.h_out)))
        return KUIOPS_E_UNSUPPORTED;
    if (a.in_row && (a.ld_in % 8 || a.in_rows <= 0)) return KUIOPS_E_UNSUPPORTED;
    if (a.h_out && (a.h_out == a.in || a.h_out == a.in_add)) return KUIOPS_E_INVALID;
    const int kc = (int)cdiv(a.K, 512);
    const int rg = kc <= 4 ? 4 : (kc <= 8 ? 2 : 1);
    if (OK != kOutPlain && rg < 2) return KUIOPS_E_UNSUPPORTED;
    // A wave loads all RG rows of its register group, so it owns exactly RG
    // rows (fewer would re-read its neighbours' rows).  Measured with the
    // weights streamed from HBM: 4 rows per wave beat 1 or 2 for every
    // K <= 2048 decode shape (o 2048x2048: 5.3 -> 4.3 us).
    a.rpw = rg;
    const int64_t grid = cdiv(a.N, 4 * (int64_t)a.rpw);
    if (grid > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    hipStream_t st = as_stream(stream);
    if (dtype == KUIOPS_BF16) decode_rows_dispatch<bf16_t, OK>(a, x_kind, (unsigned)grid, st);
    else decode_rows_dispatch<f16_t, OK>(a, x_kind, (unsigned)grid, st);
    return launch_status();
}

// ---------------------------------- batched decode projection (2..16 rows)

// The decode projection for a batch of M <= 16 sequences: the same fused
// input stage (plain / residual add + RMSNorm / SwiGLU) and epilogues (plain,
// SwiGLU pair, rotary + KV append) as decode_rows_kernel, per row, with the
// dot products on 16x16x32 MFMAs: an nn.Linear weight row is K-contiguous,
// so a 16-byte load of it is already the B operand (8 k of one output), and
// the normalised rows of x, staged in LDS, are the A operand (rows past M
// are zero).  A work-group owns 16 outputs (8 pairs for the paired
// epilogues); its NW waves split K and are summed in wave order.  In a 64-k
// step the 4 lanes of a row read its 128 bytes as two 64-byte runs (one per
// MFMA: k = 8 * cq and 32 + 8 * cq); PF steps are in flight.
struct DecMArgs {
    int64_t M, N, K;
    const void *in; int64_t ld_in;
    const int64_t *in_row; int64_t in_rows;  // optional per-row index into `in` (embedding lookup)
    const void *in_add; int64_t ld_add;
    const void *norm_w; float eps;
    void *h_out; int64_t ld_h;
    const void *W; int64_t ldw;
    void *out; int64_t ld_out;
    int64_t pair_off; int pair_shift;
    int64_t hq, hkv, hd;
    const float *inv_freq;
    const int32_t *pos;                      // [M] device positions (rotary epilogue)
    void *kc; int64_t sk0, sk1, sk2;         // k cache: batch, head, position strides
    void *vc; int64_t sv0, sv1, sv2;
    int64_t cap;
    int64_t kq;                              // k per wave, a multiple of 64
    int64_t ldsx;                            // LDS row stride of the staged x rows (elements)
    float *part;                             // (wide kernel, K split over work-groups) fp32 sums
    int64_t ks;                              //   [split][group][row][16]; k per split (multiple of 64)
};

__device__ __forceinline__ int64_t pair_div_m(const DecMArgs &a, int64_t p) {
    return a.pair_shift >= 0 ? p >> a.pair_shift : p / a.pair_off;
}

// Epilogue of decode_mrows_kernel for x row m, output o of group g (the
// group's 16 sums in vals[m][0..15]).
template <typename T, int OK>
__device__ __forceinline__ void decode_mrows_epilogue(const DecMArgs &a, int64_t g, int m, int o,
                                                      const float (*vals)[17]) {
    if constexpr (OK == kOutPlain) {
        const int64_t r = g * 16 + o;
        if (r < a.N) reinterpret_cast<T *>(a.out)[m * a.ld_out + r] = from_f32<T>(vals[m][o]);
    } else if constexpr (OK == kOutSwiGlu) {
        const int64_t p = g * 8 + o;
        if (o < 8 && p < a.N / 2) {
            const float x1 = rnd<T>(vals[m][o]), x2 = rnd<T>(vals[m][o + 8]);
            reinterpret_cast<T *>(a.out)[m * a.ld_out + p] = from_f32<T>(rnd<T>(x1 / (1.f + expf(-x1))) * x2);
        }
    } else {
        const int64_t p = g * 8 + (o & 7), e = o >> 3;
        if (p >= a.N / 2) return;
        const int64_t half = a.pair_off, head = pair_div_m(a, p), i = p - head * half + e * half;
        const float x1 = rnd<T>(vals[m][o & 7]), x2 = rnd<T>(vals[m][(o & 7) + 8]);
        const int64_t pos = a.pos ? (int64_t)a.pos[m] : 0;
        float res;
        if (head < a.hq + a.hkv) {
            const float ang = (float)pos * a.inv_freq[p - head * half];
            const float c = rnd<T>(cosf(ang)), sn = rnd<T>(sinf(ang));
            res = e == 0 ? rnd<T>(x1 * c) + rnd<T>(-x2 * sn) : rnd<T>(x2 * c) + rnd<T>(x1 * sn);
        } else {
            res = e == 0 ? x1 : x2;
        }
        T *dst;
        if (head < a.hq) {
            dst = reinterpret_cast<T *>(a.out) + m * a.ld_out + head * a.hd + i;
        } else {
            if (pos < 0 || pos >= a.cap) return;
            dst = head < a.hq + a.hkv
                      ? reinterpret_cast<T *>(a.kc) + m * a.sk0 + (head - a.hq) * a.sk1 + pos * a.sk2 + i
                      : reinterpret_cast<T *>(a.vc) + m * a.sv0 + (head - a.hq - a.hkv) * a.sv1 + pos * a.sv2 + i;
        }
        *dst = from_f32<T>(res);
    }
}

template <typename T, int XK, int OK, int NW, bool SPLIT = false>
__global__ __launch_bounds__(NW * 64) void decode_mrows_kernel(DecMArgs a) {
    typedef typename Mfma<T>::frag frag;
    constexpr int PF = 32 / NW;                       // 64-k steps in flight per wave (64 KB per work-group)
    extern __shared__ __attribute__((aligned(16))) char dsm[];
    T *sx = reinterpret_cast<T *>(dsm);               // [M][ldsx] normalised rows of x
    __shared__ float red[NW][4][64];
    __shared__ float vals[16][17];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, cq = lane >> 4;
    const int M = (int)a.M;

    // ---- output groups: a work-group owns groups blockIdx.x + i * gridDim.x
    // (16 outputs, or 8 pairs, each) and stages x once for all of them
    const int64_t ngroups = OK == kOutPlain ? (a.N + 15) / 16 : (a.N / 2 + 7) / 8;
    // W row of this lane's logical output n in group g (row 0, never
    // stored, for outputs past N)
    auto w_row = [&](int64_t g) __attribute__((always_inline)) -> uint32_t {
        int64_t wrow;
        bool wvalid;
        if constexpr (OK == kOutPlain) {
            wrow = g * 16 + n;
            wvalid = wrow < a.N;
        } else {
            const int64_t p = g * 8 + (n & 7), e = n >> 3;
            wvalid = p < a.N / 2;
            if constexpr (OK == kOutSwiGlu) {
                wrow = p + e * a.pair_off;
            } else {
                const int64_t half = a.pair_off, head = pair_div_m(a, p);
                wrow = head * a.hd + (p - head * half) + e * half;
            }
        }
        return (uint32_t)((wvalid ? wrow : 0) * a.ldw * 2);   // byte offset (W spans < 2 GiB)
    };
    // every wave runs the same padded step count (steps past its K range
    // load nothing), so group boundaries line up for the barriers
    // (SPLIT, plain x only: this work-group's K slice is split blockIdx.y;
    // k below counts from the slice's start, x is staged for the slice)
    const int64_t kb0 = SPLIT ? (int64_t)blockIdx.y * a.ks : 0;
    const int64_t klen = SPLIT ? min(a.K - kb0, a.ks) : a.K;
    const int64_t kbeg = (int64_t)wave * a.kq;
    const int64_t kend = min(klen, kbeg + a.kq);
    const int nsp = (int)(((a.kq / 64) + PF - 1) / PF) * PF;
    // ---- input stage: wave w normalises rows w, w + NW, ... into LDS.  A
    // lane issues XB chunk loads (and their residual / up halves) before it
    // uses any, so a row costs one memory round trip per 64 * XB chunks.
    constexpr int XB = 4;
    const int nch = (int)(klen / 8);
    const T *addp = reinterpret_cast<const T *>(a.in_add);
    auto x_row = [&](int m) __attribute__((always_inline)) {
        return reinterpret_cast<const T *>(a.in) + kb0 +
               (a.in_row ? max((int64_t)0, min(a.in_row[m], a.in_rows - 1)) : (int64_t)m) * a.ld_in;
    };
    // (every load is issued, from chunk 0 when the chunk is past the row or
    // there is no residual; consume_x skips those values.  With no
    // conditional loads and no use right after them, the compiler waits for
    // exactly these, leaving younger W loads in flight.)
    auto issue_x = [&](int m, int c0, u32x4 *v0, u32x4 *v1) __attribute__((always_inline)) {
        const T *in = x_row(m);
        const T *ap = addp ? addp + m * a.ld_add : in;
#pragma unroll
        for (int j = 0; j < XB; ++j) {
            const int c = c0 + 64 * j;
            const int cc = c < nch ? c : 0;
            v0[j] = *reinterpret_cast<const u32x4 *>(in + cc * 8);
            v1[j] = u32x4{0, 0, 0, 0};
            if constexpr (XK == kXSwiGlu) v1[j] = *reinterpret_cast<const u32x4 *>(in + a.K + cc * 8);
            if constexpr (XK == kXRmsNorm) v1[j] = *reinterpret_cast<const u32x4 *>(ap + cc * 8);
        }
    };
    auto consume_x = [&](int m, int c0, const u32x4 *v0, const u32x4 *v1, float &ss) __attribute__((always_inline)) {
        T *srow = sx + (int64_t)m * a.ldsx;
#pragma unroll
        for (int j = 0; j < XB; ++j) {
            const int c = c0 + 64 * j;
            if (c >= nch) continue;
            float h[8], o[8];
            unpack8<T>(v0[j], h);
            if constexpr (XK == kXRmsNorm) {
                if (addp) {
                    unpack8<T>(v1[j], o);
#pragma unroll
                    for (int e = 0; e < 8; ++e) h[e] = rnd<T>(h[e] + o[e]);
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += h[e] * h[e];
                // the summed row goes to LDS first (rounded: exact), normalised below
                *reinterpret_cast<u32x4 *>(srow + c * 8) = pack8f<T>(h);
                if (a.h_out && blockIdx.x == 0)
                    *reinterpret_cast<u32x4 *>(reinterpret_cast<T *>(a.h_out) + m * a.ld_h + c * 8) = pack8f<T>(h);
            } else if constexpr (XK == kXSwiGlu) {
                unpack8<T>(v1[j], o);
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = rnd<T>(h[e] / (1.f + expf(-h[e]))) * o[e];
                *reinterpret_cast<u32x4 *>(srow + c * 8) = pack8f<T>(h);
            } else {
                *reinterpret_cast<u32x4 *>(srow + c * 8) = v0[j];
            }
        }
    };
    auto norm_pass = [&](int m, float ss, const u32x4 *nw) __attribute__((always_inline)) {
        // RMSNorm's second pass over a staged row; the norm weight chunks
        // come from `nw` (loaded with the row: one chunk batch) or memory
        if constexpr (XK == kXRmsNorm) {
            T *srow = sx + (int64_t)m * a.ldsx;
            ss = wave_sum(ss);
            const float inv = rsqrtf(ss / (float)a.K + a.eps);
            auto one = [&](int c, u32x4 wv) __attribute__((always_inline)) {
                float h[8], w8[8], xo[8];
                unpack8<T>(*reinterpret_cast<const u32x4 *>(srow + c * 8), h);
                unpack8<T>(wv, w8);
#pragma unroll
                for (int e = 0; e < 8; ++e) xo[e] = w8[e] * rnd<T>(h[e] * inv);
                *reinterpret_cast<u32x4 *>(srow + c * 8) = pack8f<T>(xo);
            };
            if (nw) {
#pragma unroll
                for (int j = 0; j < XB; ++j)
                    if (lane + 64 * j < nch) one(lane + 64 * j, nw[j]);
            } else {
                for (int c = lane; c < nch; c += 64)
                    one(c, *reinterpret_cast<const u32x4 *>(reinterpret_cast<const T *>(a.norm_w) + c * 8));
            }
        }
    };
    // W steps as buffer loads: a step that is switched off (past this
    // wave's K range, or past the work-group's last group) gets an offset
    // past the descriptor's range and reads zeros without touching memory,
    // so no load is conditional and the compiler's waits count them exactly
    u32x4 wr[PF][2];
    const __amdgpu_buffer_rsrc_t rsW =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.W), (short)0, 0x7fffffff, 0x00020000);
    auto load_w = [&](uint32_t wrow, int st, bool live, u32x4 *dst) __attribute__((always_inline)) {
        const int64_t k = kbeg + (int64_t)st * 64 + 8 * cq;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const bool ok = live && k + 32 * h < kend;
            dst[h] = __builtin_amdgcn_raw_buffer_load_b128(rsW, ok ? wrow + (uint32_t)((kb0 + k + 32 * h) * 2) : 0x80000000u,
                                                           0, 0);
        }
    };
    const int64_t G = gridDim.x;
    int64_t g = blockIdx.x;
    uint32_t Wc = w_row(g);
    const bool one_batch = nch <= 64 * XB;
    int m_rest = wave;                                // first row still to stage
    if (one_batch) {
        // one chunk batch per row: this wave's first row (and the norm
        // weights) is loaded, then the first group's W steps, and the row is
        // staged while those are in flight (loads return in issue order)
        u32x4 v0[XB], v1[XB], nw[XB];
        const bool has = wave < M;
        if (has) {
            issue_x(wave, lane, v0, v1);
            if constexpr (XK == kXRmsNorm) {
#pragma unroll
                for (int j = 0; j < XB; ++j) {
                    const int c = lane + 64 * j;        // (chunks past the row are not used)
                    nw[j] = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const T *>(a.norm_w) + (c < nch ? c : 0) * 8);
                }
            }
        }
#pragma unroll
        for (int st = 0; st < PF; ++st) load_w(Wc, st, true, wr[st]);
        if (has) {
            float ss = 0.f;
            consume_x(wave, lane, v0, v1, ss);
            norm_pass(wave, ss, nw);
        }
        m_rest = wave + NW;
    }
    for (int m = m_rest; m < M; m += NW) {
        float ss = 0.f;
        for (int c0 = lane; c0 < nch; c0 += 64 * XB) {
            u32x4 v0[XB], v1[XB];
            issue_x(m, c0, v0, v1);
            consume_x(m, c0, v0, v1, ss);
        }
        norm_pass(m, ss, nullptr);
    }
    if (!one_batch) {
#pragma unroll
        for (int st = 0; st < PF; ++st) load_w(Wc, st, true, wr[st]);
    }

    __syncthreads();

    const bool mrow = n < M;                          // A operand row (x row n of this lane)
    for (; g < ngroups; g += G) {
        // ---- MFMAs over this wave's K range; the last PF steps prefetch
        // the next group's first PF
        const bool has_next = g + G < ngroups;
        const uint32_t Wn = w_row(has_next ? g + G : g);
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
        // PF steps: MFMAs on the loaded W, each step's registers refilled
        // with step nst0 + j of W row offset nrow (switched off: zeros)
        auto steps = [&](int s0, uint32_t nrow, int nst0, bool live) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < PF; ++j) {
                const int st = s0 + j;
                const int64_t k = kbeg + (int64_t)st * 64 + 8 * cq;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const bool in_k = k + 32 * h < kend;
                    const u32x4 xa = (mrow && in_k)
                                         ? *reinterpret_cast<const u32x4 *>(sx + (int64_t)n * a.ldsx + k + 32 * h)
                                         : u32x4{0, 0, 0, 0};
                    acc = Mfma<T>::m16(as_frag<frag>(xa), as_frag<frag>(wr[j][h]), acc);
                }
                load_w(nrow, nst0 + j, live, wr[j]);
            }
        };
        int s0 = 0;
        for (; s0 + PF < nsp; s0 += PF) steps(s0, Wc, s0 + PF, true);
        steps(s0, Wn, 0, has_next);               // the last PF steps prefetch the next group's first
        // acc[i]: x row 4 * cq + i, output n.  Waves summed in wave order.
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][i][lane] = acc[i];
        __syncthreads();
        if (tid < 256) {
            const int m = tid >> 4, o = tid & 15;
            const int l = (m >> 2) * 16 + o, i = m & 3;
            float v = red[0][i][l];
#pragma unroll
            for (int w = 1; w < NW; ++w) v += red[w][i][l];
            vals[m][o] = v;
        }
        __syncthreads();
        if (tid < 256 && (tid >> 4) < M) {
            if constexpr (SPLIT)
                a.part[(((int64_t)blockIdx.y * ngroups + g) * M) * 16 + tid] = vals[tid >> 4][tid & 15];
            else
                decode_mrows_epilogue<T, OK>(a, g, tid >> 4, tid & 15, vals);
        }
        Wc = Wn;
    }
}

// Wide batched decode projection (17..64 rows of plain x, or rows too long
// to stage): each lane reads its A operand (8 k of one row of x, 16 bytes)
// straight from global memory, where x (at most 64 rows) stays in L2; MB
// blocks of 16 rows share each W fragment and GW output groups share each x
// fragment.  A work-group owns GW consecutive 16-output groups, its NW waves
// split K, the wave sums meet in LDS in wave order and the plain / SwiGLU /
// rotary epilogues follow.  PF = 2 steps of W and x in flight per wave.
template <typename T, int OK, int NW, int MB, int GW, bool SPLIT = false>
__global__ __launch_bounds__(NW * 64) void decode_mrows_wide_kernel(DecMArgs a) {
    typedef typename Mfma<T>::frag frag;
    constexpr int PF = 2;
    __shared__ float red[NW][MB][4][64];
    __shared__ float vals[64][17];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, cq = lane >> 4;
    const int M = (int)a.M;
    const int64_t ngroups = OK == kOutPlain ? (a.N + 15) / 16 : (a.N / 2 + 7) / 8;
    const int64_t g0 = (int64_t)blockIdx.x * GW;
    const T *Wr[GW];
#pragma unroll
    for (int gi = 0; gi < GW; ++gi) {
        const int64_t g = g0 + gi;
        int64_t wrow;
        bool wvalid;
        if constexpr (OK == kOutPlain) {
            wrow = g * 16 + n;
            wvalid = wrow < a.N;
        } else {
            const int64_t p = g * 8 + (n & 7), e = n >> 3;
            wvalid = p < a.N / 2;
            if constexpr (OK == kOutSwiGlu) {
                wrow = p + e * a.pair_off;
            } else {
                const int64_t half = a.pair_off, head = pair_div_m(a, p);
                wrow = head * a.hd + (p - head * half) + e * half;
            }
        }
        Wr[gi] = reinterpret_cast<const T *>(a.W) + (wvalid ? wrow : 0) * a.ldw;
    }
    const T *X = reinterpret_cast<const T *>(a.in);
    // (SPLIT: this work-group's K slice is split blockIdx.y)
    const int64_t kb0 = SPLIT ? (int64_t)blockIdx.y * a.ks : 0;
    const int64_t kfin = SPLIT ? min(a.K, kb0 + a.ks) : a.K;
    const int64_t kbeg = kb0 + (int64_t)wave * a.kq;
    const int64_t kend = min(kfin, kbeg + a.kq);
    const int nsp = (int)(((a.kq / 64) + PF - 1) / PF) * PF;
    u32x4 wr[PF][GW][2], xr[PF][MB][2];
    auto load = [&](int st, int j) __attribute__((always_inline)) {
        const int64_t k = kbeg + (int64_t)st * 64 + 8 * cq;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const bool in_k = k + 32 * h < kend;
#pragma unroll
            for (int gi = 0; gi < GW; ++gi)
                wr[j][gi][h] = in_k ? *reinterpret_cast<const u32x4 *>(Wr[gi] + k + 32 * h) : u32x4{0, 0, 0, 0};
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int m = mb * 16 + n;
                xr[j][mb][h] = (in_k && m < M) ? *reinterpret_cast<const u32x4 *>(X + m * a.ld_in + k + 32 * h)
                                               : u32x4{0, 0, 0, 0};
            }
        }
    };
#pragma unroll
    for (int j = 0; j < PF; ++j) load(j, j);
    f32x4 acc[GW][MB];
#pragma unroll
    for (int gi = 0; gi < GW; ++gi)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[gi][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < nsp; s0 += PF) {
#pragma unroll
        for (int j = 0; j < PF; ++j) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int gi = 0; gi < GW; ++gi)
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb)
                        acc[gi][mb] = Mfma<T>::m16(as_frag<frag>(xr[j][mb][h]), as_frag<frag>(wr[j][gi][h]),
                                                   acc[gi][mb]);
            if (s0 + j + PF < nsp) load(s0 + j + PF, j);
        }
    }
    // acc[gi][mb][i]: x row 16 * mb + 4 * cq + i, output n of group g0 + gi.
    // Waves summed in wave order, one group at a time.
#pragma unroll
    for (int gi = 0; gi < GW; ++gi) {
        if (gi > 0) __syncthreads();                  // the previous group's epilogue has read vals
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave][mb][i][lane] = acc[gi][mb][i];
        __syncthreads();
        for (int idx = tid; idx < M * 16; idx += NW * 64) {
            const int m = idx >> 4, o = idx & 15, mb = m >> 4, mm = m & 15;
            const int l = (mm >> 2) * 16 + o, i = mm & 3;
            float v = red[0][mb][i][l];
#pragma unroll
            for (int w = 1; w < NW; ++w) v += red[w][mb][i][l];
            vals[m][o] = v;
        }
        __syncthreads();
        if (g0 + gi < ngroups) {
            if constexpr (SPLIT) {
                float *pp = a.part + (((int64_t)blockIdx.y * ngroups + g0 + gi) * M) * 16;
                for (int idx = tid; idx < M * 16; idx += NW * 64) pp[idx] = vals[idx >> 4][idx & 15];
            } else {
                for (int idx = tid; idx < M * 16; idx += NW * 64)
                    decode_mrows_epilogue<T, OK>(a, g0 + gi, idx >> 4, idx & 15, vals);
            }
        }
    }
}

// The K splits of decode_mrows_wide_kernel<..., SPLIT>: one work-group per
// output group and 16 rows, one thread per (row, output); a thread loads
// all its splits' sums before adding them in split order, then the group's
// epilogue runs for those rows.
constexpr int kMaxWideSplits = 16;
template <typename T, int OK>
__global__ __launch_bounds__(256) void decode_wide_merge_kernel(DecMArgs a, int splits) {
    __shared__ float vals[64][17];
    const int tid = threadIdx.x;
    const int M = (int)a.M;
    const int64_t ngroups = OK == kOutPlain ? (a.N + 15) / 16 : (a.N / 2 + 7) / 8;
    const int64_t g = blockIdx.x;
    const int m = (int)blockIdx.y * 16 + (tid >> 4), o = tid & 15;
    if (m < M) {
        const float *pp = a.part + (g * M + m) * 16 + o;
        const int64_t stride = ngroups * M * 16;
        float p[kMaxWideSplits];
#pragma unroll
        for (int sp = 0; sp < kMaxWideSplits; ++sp) p[sp] = sp < splits ? pp[sp * stride] : 0.f;
        float v = p[0];
#pragma unroll
        for (int sp = 1; sp < kMaxWideSplits; ++sp)
            if (sp < splits) v += p[sp];
        vals[m][o] = v;
    }
    __syncthreads();
    if (m < M) decode_mrows_epilogue<T, OK>(a, g, m, o, vals);
}

template <typename T, int OK, int NW, int GW, bool SPLIT = false>
static void decode_wide_launch2(const DecMArgs &a, dim3 grid, hipStream_t st) {
    switch ((a.M + 15) / 16) {
        case 1: hipLaunchKernelGGL((decode_mrows_wide_kernel<T, OK, NW, 1, GW, SPLIT>), grid, dim3(NW * 64), 0, st, a); break;
        case 2: hipLaunchKernelGGL((decode_mrows_wide_kernel<T, OK, NW, 2, GW, SPLIT>), grid, dim3(NW * 64), 0, st, a); break;
        case 3: hipLaunchKernelGGL((decode_mrows_wide_kernel<T, OK, NW, 3, GW, SPLIT>), grid, dim3(NW * 64), 0, st, a); break;
        default: hipLaunchKernelGGL((decode_mrows_wide_kernel<T, OK, NW, 4, GW, SPLIT>), grid, dim3(NW * 64), 0, st, a); break;
    }
}

// Wide-kernel shapes: output groups per work-group (x reuse) traded against
// waves per work-group (K split), within the registers of a lane:
// (GW, NW) = (4, 4) or (1, 16).
template <typename T, int OK>
static void decode_wide_launch1(const DecMArgs &a, int gw, unsigned grid, int splits, hipStream_t st) {
    if (splits > 1) {
        // K split over grid.y work-groups (4 groups x 4 waves each), then the merge
        decode_wide_launch2<T, OK, 4, 4, true>(a, dim3(grid, (unsigned)splits), st);
        const int64_t ngroups = OK == kOutPlain ? (a.N + 15) / 16 : (a.N / 2 + 7) / 8;
        hipLaunchKernelGGL((decode_wide_merge_kernel<T, OK>), dim3((unsigned)ngroups, (unsigned)((a.M + 15) / 16)),
                           dim3(256), 0, st, a, splits);
    } else if (gw == 4) {
        decode_wide_launch2<T, OK, 4, 4>(a, dim3(grid), st);
    } else {
        decode_wide_launch2<T, OK, 16, 1>(a, dim3(grid), st);
    }
}

template <typename T>
static void decode_wide_launch(const DecMArgs &a, int out_kind, int gw, unsigned grid, int splits, hipStream_t st) {
    switch (out_kind) {
        case kOutPlain: decode_wide_launch1<T, kOutPlain>(a, gw, grid, splits, st); break;
        case kOutSwiGlu: decode_wide_launch1<T, kOutSwiGlu>(a, gw, grid, splits, st); break;
        default: decode_wide_launch1<T, kOutRope>(a, gw, grid, splits, st); break;
    }
}

// dynamic LDS for the staged rows of x; with the 17 KiB of static reduction
// arrays of 16 waves it stays within the CU's 160 KiB
constexpr int64_t kDecMaxLds = 140 * 1024;

// K split of the wide kernel over work-groups, for K >= 4096: 4 output
// groups per work-group (x read once per 64 outputs) and enough K slices (of
// at least 256 k, at most 16) for about one work-group per CU, so each
// work-group reads only its slice of x.  Measured at M = 64 with cold W:
// 2048 x 5632 (down) 32.0 -> 24.1 us (25.7 at half the slices, 35.7 at
// twice); at K = 2048 the merge launch outweighs it (11264 x 2048: 27.2 ->
// 35.3 us, 2048 x 2048: 12.2 -> 19.3 us), so those stay unsplit.
struct WideSplit { int64_t splits, ks; };
static WideSplit wide_split_plan(int64_t ngroups, int64_t K) {
    if (K < 4096) return {1, K};
    const int64_t ngs = cdiv(ngroups, 4);
    const int64_t sp = std::max<int64_t>(1, std::min<int64_t>({(int64_t)kMaxWideSplits, K / 256, cdiv((int64_t)num_cus(), ngs)}));
    const int64_t ks = cdiv(cdiv(K, sp), 64) * 64;
    return {cdiv(K, ks), ks};
}
// K split of the staged kernel (plain x, K >= 4096, fewer output groups than
// CUs): enough slices for about one work-group per CU.
static WideSplit staged_split_plan(int64_t ngroups, int64_t K) {
    if (K < 4096 || ngroups >= num_cus()) return {1, K};
    const int64_t sp = std::max<int64_t>(1, std::min<int64_t>({(int64_t)kMaxWideSplits, K / 512,
                                                               cdiv((int64_t)num_cus(), ngroups)}));
    const int64_t ks = cdiv(cdiv(K, sp), 64) * 64;
    return {cdiv(K, ks), ks};
}

// Workspace of kuiops_decode_rows_batched (the K splits; a plain-x bound).
size_t decode_rows_batched_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0 || M > 64) return 0;
    const bool wide = M > 16 || M * K * 2 > kDecMaxLds;
    const int64_t ngroups = cdiv(N, 16);
    const WideSplit p = wide ? wide_split_plan(ngroups, K) : staged_split_plan(ngroups, K);
    return p.splits > 1 ? (size_t)(p.splits * ngroups * M * 16 * sizeof(float)) : 0;
}


template <typename T, int XK, int OK, int NW, bool SPLIT = false>
static hipError_t decode_mrows_launch1(const DecMArgs &a, dim3 grid, size_t lds, hipStream_t st) {
    // more than 64 KB of dynamic LDS has to be allowed per kernel first
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void *>(&decode_mrows_kernel<T, XK, OK, NW, SPLIT>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDecMaxLds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((decode_mrows_kernel<T, XK, OK, NW, SPLIT>), grid, dim3(NW * 64), lds, st, a);
    return hipSuccess;
}

// Plain x with K split over grid.y work-groups, then the split merge.
template <typename T, int OK>
static hipError_t decode_mrows_split_launch(const DecMArgs &a, int nw, unsigned grid, int splits, size_t lds,
                                            hipStream_t st) {
    const dim3 g(grid, (unsigned)splits);
    hipError_t e;
    if (nw == 16) e = decode_mrows_launch1<T, kXPlain, OK, 16, true>(a, g, lds, st);
    else if (nw == 8) e = decode_mrows_launch1<T, kXPlain, OK, 8, true>(a, g, lds, st);
    else e = decode_mrows_launch1<T, kXPlain, OK, 4, true>(a, g, lds, st);
    if (e != hipSuccess) return e;
    const int64_t ngroups = OK == kOutPlain ? (a.N + 15) / 16 : (a.N / 2 + 7) / 8;
    hipLaunchKernelGGL((decode_wide_merge_kernel<T, OK>), dim3((unsigned)ngroups, (unsigned)((a.M + 15) / 16)),
                       dim3(256), 0, st, a, splits);
    return hipSuccess;
}

template <typename T, int XK, int OK>
static hipError_t decode_mrows_launch2(const DecMArgs &a, int nw, unsigned grid, size_t lds, hipStream_t st) {
    if (nw == 16) return decode_mrows_launch1<T, XK, OK, 16>(a, dim3(grid), lds, st);
    if (nw == 8) return decode_mrows_launch1<T, XK, OK, 8>(a, dim3(grid), lds, st);
    return decode_mrows_launch1<T, XK, OK, 4>(a, dim3(grid), lds, st);
}

template <typename T, int XK>
static hipError_t decode_mrows_launch(const DecMArgs &a, int out_kind, int nw, unsigned grid, size_t lds,
                                      hipStream_t st) {
    switch (out_kind) {
        case kOutPlain: return decode_mrows_launch2<T, XK, kOutPlain>(a, nw, grid, lds, st);
        case kOutSwiGlu: return decode_mrows_launch2<T, XK, kOutSwiGlu>(a, nw, grid, lds, st);
        default: return decode_mrows_launch2<T, XK, kOutRope>(a, nw, grid, lds, st);
    }
}

}  // namespace kuiops

using namespace kuiops;

extern "C" int kuiops_decode_rows_batched(
    int64_t M, int64_t N, int64_t K, int dtype, int x_kind, int out_kind, const void *in, int64_t ld_in,
    const int64_t *in_row, int64_t in_rows, const void *in_add, int64_t ld_add, const void *norm_w, float eps,
    void *h_out, int64_t ld_h, const void *W, int64_t ldw, void *out, int64_t ld_out, int64_t pair_off,
    int64_t hq, int64_t hkv, int64_t hd, const float *inv_freq, const int32_t *pos, void *k_cache,
    const int64_t sk[3], void *v_cache, const int64_t sv[3], int64_t cache_cap, void *workspace,
    size_t workspace_bytes, void *stream) {
    if (M < 0 || N < 0 || K < 0) return KUIOPS_E_INVALID;
    if (x_kind != kXPlain && x_kind != kXRmsNorm && x_kind != kXSwiGlu) return KUIOPS_E_INVALID;
    if (out_kind != kOutPlain && out_kind != kOutSwiGlu && out_kind != kOutRope) return KUIOPS_E_INVALID;
    if (M == 0 || N == 0) return KUIOPS_OK;
    if (!in || !W || !out || (x_kind == kXRmsNorm && !norm_w)) return KUIOPS_E_INVALID;
    if (dtype != KUIOPS_BF16 && dtype != KUIOPS_F16) return KUIOPS_E_UNSUPPORTED;
    if (M > 64 || K == 0 || K % 8 || ldw % 8 || ldw < K || ld_in % 8 || (in_add && ld_add % 8) ||
        (h_out && ld_h % 8))
        return KUIOPS_E_UNSUPPORTED;
    if (x_kind == kXSwiGlu ? ld_in < 2 * K : (ld_in < K && !in_row && M > 1)) return KUIOPS_E_INVALID;
    // x rows staged in LDS (any input stage) up to 16 rows and 140 KiB; the
    // wide kernel takes 17..64 rows of plain x read from L2
    const bool wide = M > 16 || (int64_t)M * K * 2 > kDecMaxLds;
    if (wide ? (x_kind != kXPlain || in_row) : (int64_t)M * K * 2 > kDecMaxLds) return KUIOPS_E_UNSUPPORTED;
    // the staged kernel addresses W by 32-bit buffer offsets
    if (!wide && N > 0 && ((N - 1) * ldw + K) * 2 >= 0x7fffffff) return KUIOPS_E_UNSUPPORTED;
    if (!aligned16(in) || !aligned16(W) || (in_add && !aligned16(in_add)) || (norm_w && !aligned16(norm_w)) ||
        (h_out && !aligned16(h_out)))
        return KUIOPS_E_UNSUPPORTED;
    if (in_row && (in_rows <= 0)) return KUIOPS_E_INVALID;
    if (out_kind != kOutPlain && (N % 2 || pair_off <= 0)) return KUIOPS_E_INVALID;
    if (out_kind == kOutRope) {
        if (hq < 0 || hkv < 0 || hd <= 0 || hd % 2 || 2 * pair_off != hd || N != (hq + 2 * hkv) * hd) return KUIOPS_E_INVALID;
        if (!inv_freq || !k_cache || !v_cache || !sk || !sv || !pos) return KUIOPS_E_INVALID;
    }
    DecMArgs a{};
    a.M = M; a.N = N; a.K = K; a.in = in; a.ld_in = ld_in; a.in_row = in_row; a.in_rows = in_rows;
    a.in_add = in_add; a.ld_add = ld_add; a.norm_w = norm_w; a.eps = eps; a.h_out = h_out; a.ld_h = ld_h;
    a.W = W; a.ldw = ldw; a.out = out; a.ld_out = ld_out;
    a.pair_off = pair_off; a.pair_shift = log2_exact(pair_off);
    a.hq = hq; a.hkv = hkv; a.hd = hd; a.inv_freq = inv_freq; a.pos = pos;
    if (out_kind == kOutRope) {
        a.kc = k_cache; a.sk0 = sk[0]; a.sk1 = sk[1]; a.sk2 = sk[2];
        a.vc = v_cache; a.sv0 = sv[0]; a.sv1 = sv[1]; a.sv2 = sv[2];
    }
    a.cap = cache_cap;
    // At most one work-group per CU, each staging x once and taking every
    // G-th output group (one group per work-group in the wide kernel, which
    // stages nothing).  A second work-group on a CU queues its x loads
    // behind the first one's W loads and doubles that CU's groups: with 704
    // groups on 352 work-groups (batch 8 gate|up), 96 CUs carried 4 groups
    // and staged x 6 us late (17.3 us); 256 work-groups carry at most 3
    // (13.9 us).
    const int64_t ngroups = out_kind == kOutPlain ? cdiv(N, 16) : cdiv(N / 2, 8);
    const int64_t grid = wide ? ngroups : std::min<int64_t>(ngroups, (int64_t)num_cus());
    if (grid > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    hipStream_t st = as_stream(stream);
    if (!wide && x_kind == kXPlain) {
        // Plain x with K >= 4096 and fewer output groups than CUs (batch
        // down projection): K split over work-groups, each staging only its
        // slice of x, when the workspace allows (see staged_split_plan).
        const WideSplit sp = staged_split_plan(ngroups, K);
        const size_t need = sp.splits > 1 ? (size_t)(sp.splits * ngroups * M * 16 * sizeof(float)) : 0;
        if (need > 0 && workspace && workspace_bytes >= need && aligned16(workspace)) {
            a.part = static_cast<float *>(workspace);
            a.ks = sp.ks;
            int snw = 4;
            while (snw < 16 && grid * sp.splits * snw < 2048 && sp.ks >= (int64_t)snw * 2 * 128) snw *= 2;
            a.kq = cdiv(cdiv(sp.ks, snw), 64) * 64;
            a.ldsx = (int64_t)M * (sp.ks + 8) * 2 <= kDecMaxLds ? sp.ks + 8 : sp.ks;
            const size_t slds = (size_t)M * a.ldsx * 2;
            hipError_t e;
            switch (out_kind) {
                case kOutPlain:
                    e = dtype == KUIOPS_BF16 ? decode_mrows_split_launch<bf16_t, kOutPlain>(a, snw, (unsigned)grid, (int)sp.splits, slds, st)
                                             : decode_mrows_split_launch<f16_t, kOutPlain>(a, snw, (unsigned)grid, (int)sp.splits, slds, st);
                    break;
                case kOutSwiGlu:
                    e = dtype == KUIOPS_BF16 ? decode_mrows_split_launch<bf16_t, kOutSwiGlu>(a, snw, (unsigned)grid, (int)sp.splits, slds, st)
                                             : decode_mrows_split_launch<f16_t, kOutSwiGlu>(a, snw, (unsigned)grid, (int)sp.splits, slds, st);
                    break;
                default:
                    e = dtype == KUIOPS_BF16 ? decode_mrows_split_launch<bf16_t, kOutRope>(a, snw, (unsigned)grid, (int)sp.splits, slds, st)
                                             : decode_mrows_split_launch<f16_t, kOutRope>(a, snw, (unsigned)grid, (int)sp.splits, slds, st);
                    break;
            }
            if (e != hipSuccess) return KUIOPS_E_HIP;
            return launch_status();
        }
    }
    // Waves per work-group: K is split over more waves when the output
    // groups alone would leave CUs idle (N = 2048 is 128 work-groups), as
    // long as each wave keeps at least two 64-k steps.
    int nw = 4;
    while (nw < 16 && grid * nw < 2048 && K >= (int64_t)nw * 2 * 128) nw *= 2;
    a.kq = cdiv(cdiv(K, nw), 64) * 64;
    // The 16 lanes of an MFMA A-operand read sit in 16 rows of x at one k:
    // rows 16 bytes apart modulo the 64 banks (stride K + 8) spread them over
    // the banks (a row stride of K, a multiple of 256 bytes, puts all 16 in
    // one bank group); kept unpadded when the padding would not fit.
    a.ldsx = (int64_t)M * (K + 8) * 2 <= kDecMaxLds ? K + 8 : K;
    const size_t lds = (size_t)M * a.ldsx * 2;
#define KUIOPS_DECM(T)                                                                                   \
    switch (x_kind) {                                                                                    \
        case kXPlain: err = decode_mrows_launch<T, kXPlain>(a, out_kind, nw, (unsigned)grid, lds, st); break;     \
        case kXRmsNorm: err = decode_mrows_launch<T, kXRmsNorm>(a, out_kind, nw, (unsigned)grid, lds, st); break; \
        default: err = decode_mrows_launch<T, kXSwiGlu>(a, out_kind, nw, (unsigned)grid, lds, st); break;         \
    }
    if (wide) {
        // groups per work-group: 4 (x read once per 64 outputs) once that
        // still leaves ~128 work-groups, else 1 with K split over 16 waves.
        // Measured at M = 64 / 32, cold W: 11264 x 2048 25.9 / 19.4 us with
        // 4 groups against 32.5 / 22.5 (2) and 37.7 / 25.2 (1); 32000 x 2048
        // 50.8 / 37.1 against 93.4 / 62.6; 2048-output shapes are fastest
        // with 1 group (2048 x 5632: 31.5 against 55.1 with 4).
        // With a workspace, K is split over work-groups instead (each reads
        // only its slice of x; see wide_split_plan).
        const WideSplit sp = wide_split_plan(ngroups, K);
        const size_t need = sp.splits > 1 ? (size_t)(sp.splits * ngroups * M * 16 * sizeof(float)) : 0;
        if (need > 0 && workspace && workspace_bytes >= need && aligned16(workspace)) {
            a.part = static_cast<float *>(workspace);
            a.ks = sp.ks;
            a.kq = cdiv(cdiv(sp.ks, 4), 64) * 64;
            const unsigned sgrid = (unsigned)cdiv(ngroups, 4);
            if (dtype == KUIOPS_BF16) decode_wide_launch<bf16_t>(a, out_kind, 4, sgrid, (int)sp.splits, st);
            else decode_wide_launch<f16_t>(a, out_kind, 4, sgrid, (int)sp.splits, st);
            return launch_status();
        }
        const int gw = ngroups >= 512 ? 4 : 1;
        const int wnw = gw == 4 ? 4 : 16;
        a.kq = cdiv(cdiv(K, wnw), 64) * 64;
        const unsigned wgrid = (unsigned)cdiv(ngroups, gw);
        if (dtype == KUIOPS_BF16) decode_wide_launch<bf16_t>(a, out_kind, gw, wgrid, 1, st);
        else decode_wide_launch<f16_t>(a, out_kind, gw, wgrid, 1, st);
        return launch_status();
    }
    hipError_t err;
    if (dtype == KUIOPS_BF16) { KUIOPS_DECM(bf16_t) } else { KUIOPS_DECM(f16_t) }
    if (err != hipSuccess) return KUIOPS_E_HIP;
#undef KUIOPS_DECM
    return launch_status();
}

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
    if (t > INT32_MAX || n > 65535 || hq + 2 * hkv > 65535) return KUIOPS_E_UNSUPPORTED;
    RopeArgs a{n, t, hq, hkv, hd, qkv, ld_tok, ld_batch, inv_freq, pos0,
               q_out, sq[0], sq[1], sq[2], k_cache, sk[0], sk[1], sk[2], v_cache, sv[0], sv[1], sv[2], cache_cap};
    const dim3 grid((unsigned)t, (unsigned)n, (unsigned)(hq + 2 * hkv));
    hipStream_t st = as_stream(stream);
    if (dtype == KUIOPS_BF16) hipLaunchKernelGGL((rope_kv_kernel<bf16_t>), grid, dim3(64), 0, st, a);
    else hipLaunchKernelGGL((rope_kv_kernel<f16_t>), grid, dim3(64), 0, st, a);
    return launch_status();
}

extern "C" int kuiops_decode_linear(int64_t N, int64_t K, int dtype, int x_kind, const void *in, const void *in_add,
                                    const void *norm_w, float eps, void *h_out, const void *W, int64_t ldw,
                                    const void *bias, void *out, void *stream) {
    DecLinArgs a{};
    a.N = N; a.K = K; a.in = in; a.in_add = in_add; a.norm_w = norm_w; a.eps = eps; a.h_out = h_out;
    a.W = W; a.ldw = ldw; a.bias = bias; a.out = out;
    return decode_linear_run<kOutPlain>(a, dtype, x_kind, stream);
}

extern "C" int kuiops_decode_gate_up(int64_t ffn, int64_t K, int dtype, int x_kind, const void *in,
                                     const void *in_add, const void *norm_w, float eps, void *h_out, const void *W,
                                     int64_t ldw, void *out, void *stream) {
    if (ffn < 0) return KUIOPS_E_INVALID;
    DecLinArgs a{};
    a.N = 2 * ffn; a.K = K; a.in = in; a.in_add = in_add; a.norm_w = norm_w; a.eps = eps; a.h_out = h_out;
    a.W = W; a.ldw = ldw; a.out = out; a.pair_off = ffn; a.pair_shift = log2_exact(ffn);
    return decode_linear_run<kOutSwiGlu>(a, dtype, x_kind, stream);
}

extern "C" int kuiops_decode_qkv_rope(int64_t hq, int64_t hkv, int64_t hd, int64_t K, int dtype, int x_kind,
                                      const void *in, const int64_t *in_row, int64_t ld_in, int64_t in_rows,
                                      const void *in_add, const void *norm_w, float eps, void *h_out,
                                      const void *W, int64_t ldw, const float *inv_freq, const int32_t *pos,
                                      void *q_out, void *k_cache, int64_t sk_head, int64_t sk_pos, void *v_cache,
                                      int64_t sv_head, int64_t sv_pos, int64_t cache_cap, void *stream) {
    if (hq < 0 || hkv < 0 || hd <= 0 || hd % 2 || cache_cap < 0) return KUIOPS_E_INVALID;
    if (!inv_freq || !k_cache || !v_cache) return KUIOPS_E_INVALID;
    DecLinArgs a{};
    a.N = (hq + 2 * hkv) * hd; a.K = K; a.in = in; a.in_add = in_add; a.norm_w = norm_w; a.eps = eps;
    a.h_out = h_out; a.W = W; a.ldw = ldw; a.out = q_out;
    a.in_row = in_row; a.ld_in = ld_in; a.in_rows = in_rows;
    a.pair_off = hd / 2; a.pair_shift = log2_exact(hd / 2); a.hq = hq; a.hkv = hkv; a.hd = hd; a.inv_freq = inv_freq; a.pos = pos;
    a.kc = k_cache; a.sk1 = sk_head; a.sk2 = sk_pos; a.vc = v_cache; a.sv1 = sv_head; a.sv2 = sv_pos;
    a.cap = cache_cap;
    return decode_linear_run<kOutRope>(a, dtype, x_kind, stream);
}
