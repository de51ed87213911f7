// Batch-1 decode projection (one wave's dot product per weight row, with the
// RMSNorm / SwiGLU input stage and the SwiGLU / rotary + KV-append
// epilogues), shared by the decoder library and the persistent decode-step
// kernel.  Floating-point contraction is off in these bodies: an FMA would
// skip the rounding of a product that the stock ops round.
#pragma once

#include "common.hpp"

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

// ------------------------------------- batch-1 decode projection

constexpr int kXPlain = 1, kXRmsNorm = 2, kXSwiGlu = 3;   // kuiops_x_kind
constexpr int kDecodeMaxK = 8192;

constexpr int kOutPlain = 0, kOutSwiGlu = 1, kOutRope = 2;   // decode_rows_kernel epilogues

struct DecLinArgs {
    int64_t N, K;
    const void *in, *in_add;           // x source; RMSNorm: h = round(in + in_add)
    const void *norm_w;
    float eps;
    void *h_out;
    const void *W; int64_t ldw;        // [N, K] rows, K contiguous
    const void *bias;
    void *out;
    int rpw;                           // rows per wave
    // optional device row index of `in` (in += in_row[0] * ld_in, clamped to
    // in_rows), or (row_ll) an epoch-tagged word holding the row index in its
    // low 32 bits, awaited with epoch ep_row before the input is read
    const int64_t *in_row; int64_t ld_in, in_rows;
    const void *row_ll; uint32_t ep_row;
    // paired epilogues: logical row 2p + e is W row base(p) + e * pair_off
    int64_t pair_off;
    int pair_shift;                    // log2(pair_off) when a power of two, else -1
    // rotary epilogue (kOutRope): rows are [q heads | k heads | v heads] of hd
    int64_t hq, hkv, hd;
    const float *inv_freq;
    const int32_t *pos;                // device position of the token
    int64_t pos_val; int use_pos_val;  // or the position itself
    void *kc; int64_t sk1, sk2;        // k cache: head, position strides
    void *vc; int64_t sv1, sv2;
    int64_t cap;
    // epoch-tagged exchange (the persistent decode step): the epochs of the
    // input, addend and output writes, and epoch-tagged copies [hkv * hd]
    // of the new k / v rows (kOutRope, optional)
    uint32_t ep_in, ep_add, ep_out;
    void *kfresh, *vfresh;
    unsigned *err;                     // raised when an epoch-tagged wait expires
};

// W row of logical row j: identity, or the pair mapping of the paired
// epilogues (SwiGLU: rows p and p + ffn; rotary: rows i and i + hd/2 of a
// head, so that one wave holds both halves of each rotated pair).
// p / pair_off (a shift for the power-of-two head halves of real models: a
// 64-bit division would sit on the W loads' address path)
__device__ __forceinline__ int64_t pair_div(const DecLinArgs &a, int64_t p) {
    return a.pair_shift >= 0 ? p >> a.pair_shift : p / a.pair_off;
}

template <int OK>
__device__ __forceinline__ int64_t dec_row(const DecLinArgs &a, int64_t j) {
    if constexpr (OK == kOutPlain) return j;
    const int64_t p = j >> 1, e = j & 1;
    if constexpr (OK == kOutSwiGlu) return p + e * a.pair_off;
    const int64_t half = a.pair_off, head = pair_div(a, p);
    return head * a.hd + (p - head * half) + e * half;
}

// out[n] = dot(W[n, :], x) (+ bias[n]) with x computed by every work-group
// into LDS (the fused input stage), then held in registers: lane l owns
// 16-byte chunks l, l + 64, ... of x and of each W row, so a wave reads a row
// as whole 1 KB segments and the row's dot product is a wave sum.  A wave
// owns rpw <= RG rows; their W loads are issued before the input stage, so
// the stage's own global reads and reduction hide under the W latency.
//   kXPlain    x = in
//   kXRmsNorm  h = round(in + in_add), x = round(w * round(h * rsqrt(mean(h^2) + eps)));
//              work-group 0 stores h to h_out
//   kXSwiGlu   x = round(round(silu(in[k])) * in[K + k])      (in = [gate | up])
// Epilogues (OK):
//   kOutPlain   out[n] = round(dot) (+ bias)
//   kOutSwiGlu  rows (p, p + ffn) of a [gate; up] weight: out[p] = round(round(silu(g)) * u),
//               g, u the rounded projections (as silu_mul_kernel)
//   kOutRope    rows (i, i + hd/2) of each head of a fused qkv weight: q and k
//               pairs rotated at position pos (as rope_kv_kernel), q to out
//               [hq * hd], k and v stored into the caches at pos (if < cap)
// Wave sums of RG per-lane partial rows in one pass: log2(RG) exchange steps
// in which each lane sends half of its remaining rows to the partner across
// lane bit 5, 4, 3 (keeping the half that lane bit selects), then the one
// remaining row is summed over the low lanes with DPP moves.  Returns, in
// every lane, the total of row lane / (64 / RG).  (RG separate butterflies
// would take RG x 6 dependent cross-lane exchanges.)
template <int N, int MASK>
__device__ __forceinline__ void halve_rows(float *v, int lane) {
    // the lane keeps row i (bit MASK clear) or i + N / 2 (set) and adds its
    // partner's value of that row
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
        float p, q;
        swap_rows<MASK>(v[i], v[i + N / 2], p, q);
        v[i] = p + q;
    }
}

template <int RG>
__device__ __forceinline__ float multi_row_sum(float *v, int lane) {
    // Every row is summed over lane bits 5, 4, 3 (halving steps or
    // butterflies: a + b and b + a are the same sum), then over bits 0-2
    // by DPP, so a row's total has the same bits whatever RG is.
    static_assert(RG == 1 || RG == 2 || RG == 4 || RG == 8, "rows");
    if constexpr (RG >= 2) halve_rows<RG, 32>(v, lane);
    else v[0] = xor_add<32>(v[0]);
    if constexpr (RG >= 4) halve_rows<RG / 2, 16>(v, lane);
    else v[0] = xor_add<16>(v[0]);
    if constexpr (RG >= 8) halve_rows<2, 8>(v, lane);
    else v[0] = xor_add<8>(v[0]);
    return group_sum<8>(v[0]);
}

struct NoWait {
    __device__ __forceinline__ void operator()() const {}
};

// One work-group of NWV waves (NWV = 4 or 8) of decode_rows_kernel, owning
// rows from blk * NWV * rpw.  `wait` runs after the W loads are issued and
// before the input stage reads `in` / `in_add` (the persistent decode step
// waits there for the producers of its input; the plain kernel waits for
// nothing).  IO carries the activation reads and every output store
// (PlainIO, or CoherentIO when consumers in the same launch read them).  The input stage runs on the first 256 threads, so its sums
// are those of the 4-wave kernel whatever NWV is.
typedef __attribute__((address_space(3))) char lds_bytes;

// RGL > 0: each wave owns RGL more rows whose W chunks go global -> LDS
// (LDS-DMA, issued with the register loads) into `wl` (NWV * RGL * KC KB,
// wave w's rows at w * RGL * KC KB), so a work-group keeps more weight
// bytes in flight than its registers hold.
// xs (non-null): LDS for the staged input x (K * 2 bytes) in place of the
// body's own array (the persistent decode step shares one buffer between its
// job kinds).
// IO reads the input vectors, OIO writes the outputs (epoch-tagged LLIO
// inputs are polled until the expected write is there, bounded: on expiry
// *a_err (if set) is raised and the stale values are used).
template <typename T, int XK, int KC, int OK, int NWV, typename Wait, typename IO = PlainIO, int RGO = 0, int RGL = 0,
          bool EXTX = false, typename OIO = IO>
__device__ __forceinline__ void decode_rows_block(const DecLinArgs &a, int64_t blk, const Wait &wait,
                                                  lds_bytes *wl = nullptr, lds_bytes *xs = nullptr) {
#pragma clang fp contract(off)
    static_assert(NWV == 4 || NWV == 8, "waves");
    static_assert(RGL == 0 || OK != kOutRope, "LDS rows: plain or SwiGLU epilogues");
    static_assert(OK == kOutPlain || RGL % 2 == 0, "paired epilogues: whole pairs of LDS rows");
    // register rows per wave; RGO overrides the default (a row's dot product
    // is the same whichever wave computes it).  Host: rpw == RG + RGL.
    constexpr int RG = RGO ? RGO : (KC <= 4 ? 4 : (KC <= 8 ? 2 : 1));
    static_assert(OK == kOutPlain || RG % 2 == 0, "paired epilogues need two rows per wave");
    static_assert(!OIO::kLL || OK == kOutPlain || (RG % 2 == 0 && RGL % 2 == 0),
                  "epoch-tagged paired outputs: whole pairs per wave");
    constexpr int XCH = KC * 64 / 256 > 0 ? KC * 64 / 256 : 1;   // x chunks per thread in the input stage (K <= 512 KC)
    typedef T t8 __attribute__((ext_vector_type(8)));
    typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
    lds_u32x4 *sx;
    if constexpr (EXTX) {
        sx = (lds_u32x4 *)xs;
    } else {
        __shared__ u32x4 sx_own[KC * 64];
        sx = (lds_u32x4 *)sx_own;
    }
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nch = (int)(a.K / 8);
    const T *in = reinterpret_cast<const T *>(a.in);
    if (a.in_row) in += max((int64_t)0, min(a.in_row[0], a.in_rows - 1)) * a.ld_in;

    // ---- this wave's W rows, in flight during the input stage
    const T *W = reinterpret_cast<const T *>(a.W);
    const int64_t r0 = (blk * NWV + wave) * a.rpw;
    const int64_t r1 = min(a.N, r0 + a.rpw);
    // Rotary epilogue operands (the token position and the pair's inverse
    // frequency), loaded first so that their latency hides under the W loads
    // instead of following the dot products.
    int64_t rope_pos = 0;
    float rope_freq = 0.f;
    if constexpr (OK == kOutRope) {
        rope_pos = a.use_pos_val ? a.pos_val : (a.pos ? (int64_t)a.pos[0] : 0);
        if (lane % (128 / RG) == 0) {               // the lane that finishes pair lane / (128 / RG)
            const int g = 2 * (lane / (128 / RG));
            const int64_t p = (r0 + g) >> 1, half = a.pair_off, head = pair_div(a, p);
            if (head < a.hq + a.hkv && r0 + g + 1 < r1) rope_freq = a.inv_freq[p - head * half];
        }
    }
    u32x4 wv[RG][KC];
#pragma unroll
    for (int g = 0; g < RG; ++g) {
        const int64_t r = dec_row<OK>(a, min(r0 + g, a.N - 1));   // clamped: never stored
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const int ch = j * 64 + lane;
            wv[g][j] = ch < nch ? *reinterpret_cast<const u32x4 *>(W + r * a.ldw + ch * 8) : u32x4{0, 0, 0, 0};
        }
    }
    if constexpr (RGL > 0) {
        // chunks past K read a valid neighbour; x is zero there
#pragma unroll
        for (int g = 0; g < RGL; ++g) {
            const int64_t r = dec_row<OK>(a, min(r0 + RG + g, a.N - 1));
#pragma unroll
            for (int j = 0; j < KC; ++j) {
                const int ch = min(j * 64 + lane, nch - 1);
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(W + r * a.ldw + ch * 8),
                                                 wl + ((wave * RGL + g) * KC + j) * 1024, 16, 0, 0);
            }
        }
    }
    // Rotary cos / sin of this lane's pair, computed while the W rows are in
    // flight (their loads were issued after the two operands above, so only
    // those are waited for); computed in the epilogue they would lengthen
    // the kernel's final dependency chain by ~0.7 us.
    float rope_c = 0.f, rope_s = 0.f;
    if constexpr (OK == kOutRope) {
        if (lane % (128 / RG) == 0) {
            const float ang = (float)rope_pos * rope_freq;
            rope_c = rnd<T>(cosf(ang));
            rope_s = rnd<T>(sinf(ang));
        }
    }
    // ---- input stage (threads 0 .. 255); the RMSNorm weight does not
    // depend on the input, so it is loaded before the wait
    const bool stage = tid < 256;
    u32x4 nwv[XK == kXRmsNorm ? XCH : 1];
    if constexpr (XK == kXRmsNorm) {
#pragma unroll
        for (int c = 0; c < XCH; ++c) {
            const int ch = c * 256 + tid;
            nwv[c] = (stage && ch < nch) ? *reinterpret_cast<const u32x4 *>(reinterpret_cast<const T *>(a.norm_w) + ch * 8)
                                         : u32x4{0, 0, 0, 0};
        }
    }
    wait();
    // raw input chunks (and the addend's / SwiGLU up half's), read through IO
    const bool has_add = XK == kXRmsNorm && a.in_add;
    u32x4 rin[XCH], radd[XCH];
    auto load_input = [&]() -> bool {
        bool ok = true;
#pragma unroll
        for (int c = 0; c < XCH; ++c) {
            const int ch = c * 256 + tid;
            if (!stage || ch >= nch) continue;
            ok = IO::ld8(in, (int64_t)ch * 8, a.ep_in, rin[c]) && ok;
            if (has_add) ok = IO::ld8(a.in_add, (int64_t)ch * 8, a.ep_add, radd[c]) && ok;
            if constexpr (XK == kXSwiGlu) ok = IO::ld8(in, a.K + (int64_t)ch * 8, a.ep_in, radd[c]) && ok;
        }
        return ok;
    };
    if constexpr (IO::kLL) {
        // every thread reads its chunks; while a chunk is not the expected
        // write it probes only the chunk's first word (8 bytes per poll), then
        // reads the chunk again; each wave spins on its own chunks, then the
        // work-group meets
        auto probe = [&]() -> bool {
            bool ok = true;
#pragma unroll
            for (int c = 0; c < XCH; ++c) {
                const int ch = c * 256 + tid;
                if (!stage || ch >= nch) continue;
                ok = ok && (uint32_t)(LLIO::word(in, (int64_t)ch * 4) >> 32) == a.ep_in;
                if (has_add) ok = ok && (uint32_t)(LLIO::word(a.in_add, (int64_t)ch * 4) >> 32) == a.ep_add;
            }
            return ok;
        };
        bool ok = load_input();
        unsigned e = ll_err_read(a.err);
        for (unsigned it = 0; !__all(ok); ++it) {
            if (ll_expired(it, e, a.err)) break;
            __builtin_amdgcn_s_sleep(kLLSleep);
            if (!ok && probe()) ok = load_input();
            e = ll_err_read(a.err);
        }
        __syncthreads();
    } else {
        if (a.row_ll) {
            // the row index comes from another work-group of the launch
            uint64_t w = LLIO::word(a.row_ll, 0);
            unsigned e = ll_err_read(a.err);
            for (unsigned it = 0; !__all((uint32_t)(w >> 32) == a.ep_row); ++it) {
                if (ll_expired(it, e, a.err)) break;
                __builtin_amdgcn_s_sleep(kLLSleep);
                w = LLIO::word(a.row_ll, 0);
                e = ll_err_read(a.err);
            }
            in = reinterpret_cast<const T *>(a.in) +
                 max((int64_t)0, min((int64_t)(uint32_t)w, a.in_rows - 1)) * a.ld_in;
        }
        load_input();
    }
    float h[XCH][8];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < XCH; ++c) {
        const int ch = c * 256 + tid;
        if (!stage || ch >= nch) continue;
        unpack8<T>(rin[c], h[c]);
        if constexpr (XK == kXRmsNorm) {
            if (has_add) {
                float o[8];
                unpack8<T>(radd[c], o);
#pragma unroll
                for (int e = 0; e < 8; ++e) h[c][e] = rnd<T>(h[c][e] + o[e]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += h[c][e] * h[c][e];
        }
    }
    float inv = 0.f;
    if constexpr (XK == kXRmsNorm) {
        ss = wave_sum_swaps(ss);
        if (lane == 0 && stage) red[wave] = ss;
        __syncthreads();
        inv = rsqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)a.K + a.eps);
    }
    const bool store_h = XK == kXRmsNorm && a.h_out && blk == 0;
#pragma unroll
    for (int c = 0; c < XCH; ++c) {
        const int ch = c * 256 + tid;
        if (!stage || ch >= nch) continue;
        float xo[8];
        if constexpr (XK == kXRmsNorm) {
            float wv[8];
            unpack8<T>(nwv[c], wv);
#pragma unroll
            for (int e = 0; e < 8; ++e) xo[e] = wv[e] * rnd<T>(h[c][e] * inv);
            if (store_h) OIO::st8(a.h_out, (int64_t)ch * 8, a.ep_out, pack8f<T>(h[c]));
        } else if constexpr (XK == kXSwiGlu) {
            float uv[8];
            unpack8<T>(radd[c], uv);
#pragma unroll
            for (int e = 0; e < 8; ++e) xo[e] = rnd<T>(h[c][e] / (1.f + expf(-h[c][e]))) * uv[e];
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) xo[e] = h[c][e];
        }
        sx[ch] = pack8f<T>(xo);
    }
    __syncthreads();

    // ---- rows
    // x stays packed (bf16 / f16 pairs): v_dot2 takes a W pair and an x pair
    // per instruction (products exact in fp32, fp32 accumulate)
    u32x4 xv[KC];
#pragma unroll
    for (int j = 0; j < KC; ++j) {
        const int ch = j * 64 + lane;
        xv[j] = ch < nch ? sx[ch] : u32x4{0, 0, 0, 0};
    }
    float accs[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < KC; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = dot2<T>(wv[g][j][e], xv[j][e], acc);
        accs[g] = acc;
    }
    // row lane / (64 / RG)'s total in every lane of its group; the next row's
    // total comes from the group above (paired epilogues: rows 2q, 2q + 1)
    const float tot = multi_row_sum<RG>(accs, lane);
    // the LDS rows RG .. RG + RGL - 1 (their own reduction: the same sums)
    float totl = 0.f;
    if constexpr (RGL > 0) {
        __builtin_amdgcn_s_waitcnt(0);              // this wave's LDS-DMA has landed
        float accl[RGL];
#pragma unroll
        for (int g = 0; g < RGL; ++g) {
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < KC; ++j) {
                const u32x4 w = *(const __attribute__((address_space(3))) u32x4 *)(wl + ((wave * RGL + g) * KC + j) * 1024 + lane * 16);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc = dot2<T>(w[e], xv[j][e], acc);
            }
            accl[g] = acc;
        }
        totl = multi_row_sum<RGL>(accl, lane);
    }
    if constexpr (OK == kOutPlain) {
        auto val = [&](int64_t r, float acc) {
            if (a.bias) acc += to_f32(reinterpret_cast<const T *>(a.bias)[r]);
            return from_f32<T>(acc);
        };
        if constexpr (OIO::kLL) {
            // the work-group's rows (consecutive from blk * NWV * rpw) meet in
            // LDS, then go out as row pairs, one epoch-tagged word each
            constexpr int RW = RG + RGL, RJ = NWV * RW;
            static_assert(RJ % 2 == 0, "whole row pairs per work-group");
            __shared__ __attribute__((aligned(16))) T s_rows[RJ];
            const int64_t rj0 = blk * RJ;
            if (lane % (64 / RG) == 0) {
                const int64_t r = r0 + lane / (64 / RG);
                if (r < r1) s_rows[r - rj0] = val(r, tot);
            }
            if constexpr (RGL > 0) {
                if (lane % (64 / RGL) == 0) {
                    const int64_t r = r0 + RG + lane / (64 / RGL);
                    if (r < r1) s_rows[r - rj0] = val(r, totl);
                }
            }
            __syncthreads();
            const int64_t nr = min((int64_t)RJ, a.N - rj0);
            if (2 * tid < nr)
                OIO::st2(reinterpret_cast<T *>(a.out), rj0 + 2 * tid, s_rows[2 * tid],
                         2 * tid + 1 < nr ? s_rows[2 * tid + 1] : from_f32<T>(0.f), a.ep_out);
        } else {
            auto put = [&](int64_t r, float acc) {
                if (r < r1) OIO::st(reinterpret_cast<T *>(a.out) + r, val(r, acc));
            };
            if (lane % (64 / RG) == 0) put(r0 + lane / (64 / RG), tot);
            if constexpr (RGL > 0)
                if (lane % (64 / RGL) == 0) put(r0 + RG + lane / (64 / RGL), totl);
        }
    } else {
        const float nxt = from_lane_above<64 / RG>(tot);
        float nxtl = 0.f;
        if constexpr (RGL >= 2) nxtl = from_lane_above<64 / RGL>(totl);
        // lane 2q * (64 / RG) finishes pair q, so the pairs' epilogues run
        // side by side.  The results go through LDS: the work-group's pairs
        // are consecutive (pg0 ..), so each output half is one contiguous
        // run, stored as 16-byte writes (2-byte stores from every wave of
        // every work-group cost the qkv kernel ~1.5 us).
        constexpr int PW = (RG + RGL) / 2, PG = NWV * PW;   // pairs per wave / work-group
        __shared__ __attribute__((aligned(16))) T s_o[2][PG];
        const int64_t pg0 = blk * PG;
        const int np = (int)min((int64_t)PG, a.N / 2 - pg0);
        const int64_t pos = rope_pos;
        const bool store_kv = pos >= 0 && pos < a.cap;
        auto finish_pair = [&](int g, float t1, float t2) {
            const int64_t r = r0 + g;                    // even: rows r, r + 1 form pair r / 2
            const int64_t p = r >> 1;
            const int slot = wave * PW + g / 2;
            const float x1 = rnd<T>(t1), x2 = rnd<T>(t2);
            if (r + 1 < r1) {
                if constexpr (OK == kOutSwiGlu) {
                    s_o[0][slot] = from_f32<T>(rnd<T>(x1 / (1.f + expf(-x1))) * x2);
                } else {
                    const int64_t head = pair_div(a, p);
                    if (head < a.hq + a.hkv) {
                        const float c = rope_c, sn = rope_s;
                        s_o[0][slot] = from_f32<T>(rnd<T>(x1 * c) + rnd<T>(-x2 * sn));
                        s_o[1][slot] = from_f32<T>(rnd<T>(x2 * c) + rnd<T>(x1 * sn));
                    } else {
                        s_o[0][slot] = from_f32<T>(x1);
                        s_o[1][slot] = from_f32<T>(x2);
                    }
                }
            }
        };
        if (lane % (128 / RG) == 0) finish_pair(2 * (lane / (128 / RG)), tot, nxt);
        if constexpr (RGL >= 2)
            if (lane % (128 / RGL) == 0) finish_pair(RG + 2 * (lane / (128 / RGL)), totl, nxtl);
        __syncthreads();
        // destination of pair p's half e: SwiGLU out[p]; rotary q -> out,
        // k -> k cache, v -> v cache at position pos (element i, or i + hd/2),
        // plus the epoch-tagged fresh k / v rows when given.  kind: 0 out,
        // 1 k, 2 v, -1 nothing; idx: element index in out, or within the head.
        auto dst_of = [&](int64_t p, int e, int &kind, int64_t &head_kv) -> int64_t {
            if constexpr (OK == kOutSwiGlu) {
                kind = 0;
                return p;
            } else {
                const int64_t half = a.pair_off, head = pair_div(a, p), i = p - head * half + e * half;
                if (head < a.hq) { kind = 0; return head * a.hd + i; }
                kind = head < a.hq + a.hkv ? 1 : 2;
                head_kv = kind == 1 ? head - a.hq : head - a.hq - a.hkv;
                return i;
            }
        };
        T *const kc = reinterpret_cast<T *>(a.kc), *const vc = reinterpret_cast<T *>(a.vc);
        auto cache_idx = [&](int kind, int64_t hkv, int64_t i) {
            return kind == 1 ? hkv * a.sk1 + pos * a.sk2 + i : hkv * a.sv1 + pos * a.sv2 + i;
        };
        constexpr int NE = OK == kOutSwiGlu ? 1 : 2;
        // a run of whole 16-byte pieces goes out as NV vector stores
        constexpr bool VEC = PG * sizeof(T) % 16 == 0;
        constexpr int NV = VEC ? PG * (int)sizeof(T) / 16 : 1;
        if (tid < NE * NV && np > 0) {
            const int e = tid / NV, v = tid % NV;
            int kind0 = -1;
            int64_t hkv0 = 0;
            const int64_t i0 = dst_of(pg0, e, kind0, hkv0);
            // one run when all pairs are present and share the first pair's head
            const bool one_run = np == PG && (OK == kOutSwiGlu || (pg0 - pair_div(a, pg0) * a.pair_off) + PG <= a.pair_off);
            const u32x4 piece = reinterpret_cast<const u32x4 *>(s_o[e])[v];
            if (VEC && one_run && (i0 & 7) == 0 && (kind0 == 0 || (store_kv && (cache_idx(kind0, hkv0, i0) & 7) == 0))) {
                if (kind0 == 0) {
                    OIO::st8(a.out, i0 + v * 8, a.ep_out, piece);
                } else {
                    PlainIO::st8(kind0 == 1 ? a.kc : a.vc, cache_idx(kind0, hkv0, i0) + v * 8, 0, piece);
                    void *fr = kind0 == 1 ? a.kfresh : a.vfresh;
                    if (fr) OIO::st8(fr, hkv0 * a.hd + i0 + v * 8, a.ep_out, piece);
                }
            } else if (v == 0) {
                // element by element (pairs for epoch-tagged vectors: the run
                // starts at an even element and holds whole pairs)
                for (int k = 0; k < np; k += (OIO::kLL ? 2 : 1)) {
                    int kind = -1;
                    int64_t hkv = 0;
                    const int64_t i = dst_of(pg0 + k, e, kind, hkv);
                    const T x0 = s_o[e][k], x1 = OIO::kLL && k + 1 < np ? s_o[e][k + 1] : from_f32<T>(0.f);
                    if (kind == 0) {
                        if constexpr (OIO::kLL) OIO::st2(reinterpret_cast<T *>(a.out), i, x0, x1, a.ep_out);
                        else OIO::st(reinterpret_cast<T *>(a.out) + i, x0);
                    } else if (kind > 0 && store_kv) {
                        T *c = kind == 1 ? kc : vc;
                        c[cache_idx(kind, hkv, i)] = x0;
                        if constexpr (OIO::kLL) {
                            if (k + 1 < np) c[cache_idx(kind, hkv, i) + 1] = x1;
                            void *fr = kind == 1 ? a.kfresh : a.vfresh;
                            if (fr) OIO::st2(reinterpret_cast<T *>(fr), hkv * a.hd + i, x0, x1, a.ep_out);
                        }
                    }
                }
            }
        }
    }
}

template <typename T, int XK, int KC, int OK = kOutPlain>
__global__ __launch_bounds__(256) void decode_rows_kernel(DecLinArgs a) {
    decode_rows_block<T, XK, KC, OK, 4>(a, blockIdx.x, NoWait{});
}

}  // namespace kuiops
