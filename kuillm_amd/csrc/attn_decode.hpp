// Split-KV decode attention (few query rows per head over a long KV cache),
// shared by the attention library and the persistent decode-step kernel.
#pragma once

#include "common.hpp"

namespace kuiops {

struct AttnArgs {
    int64_t n, hq, hkv, l, s;
    const void *Q, *K, *V;
    void *O;
    int64_t sq0, sq1, sq2, sk0, sk1, sk2, sv0, sv1, sv2, so0, so1, so2;
    float *lse;
    float scale_log2;   // softmax scale * log2(e)
    int causal;
    int nqb;            // query blocks per (batch, head)
    int pair;           // causal prefill: a work-group runs query blocks p and nqb-1-p
    // decode
    int splits;
    int64_t chunk;      // keys per split
    int rows_per_group; // query rows handled by one work-group
    int row_groups;
    float *ws_ml;       // [rows_total][splits][2]
    float *ws_o;        // [rows_total][splits][ev]
    unsigned *counters; // [n][hkv][row_groups] split arrival counters (zero between calls)
    const int32_t *kv_len;  // decode: per-batch key count in device memory (<= s), or null
    // additive attention bias (fa_fwd_kernel BIAS): element (b, h, q, key) at
    // bias + b*sb0 + h*sb1 + q*sb2 + key, in the dtype of Q; added to the raw
    // scores pre-divided by the scale (softmax(scale * (QK^T + bias / scale)))
    const void *bias;
    int64_t sb0, sb1, sb2;
    float inv_scale;
    // epoch-tagged exchange (the persistent decode step, IO = LLIO): the
    // epochs of the query and output writes, epoch-tagged copies [hkv * e]
    // of the new k / v rows (key `fresh`), and the expired-wait flag
    uint32_t ep_q, ep_o;
    const void *kfresh, *vfresh;
    unsigned *err;
    // one-pass form: the key count itself (use_s_len), and the keys
    // fresh_lo .. fresh read from epoch-tagged slots: key fresh_lo + i at
    // kfresh / vfresh + i * fresh_stride elements, written with epoch
    // ep_fresh0 + i * ep_fresh_step
    int64_t s_len; int use_s_len;
    int64_t fresh_lo, fresh_stride;
    uint32_t ep_fresh0, ep_fresh_step;
};

constexpr float kLn2 = 0.69314718055994530942f;

// Split arrival counters sit kAttnCounterStride words (64 bytes) apart: agent-scope
// atomics on one cache line serialise, and the row groups' counts all arrive
// at the end of the launch (4096-key bench case: 20.8 -> 19.7 us).
constexpr int kAttnCounterStride = 16;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }


// Merges online-softmax state (m2, l2, o2) into (m1, l1, o1).
template <int ND>
__device__ __forceinline__ void merge_state(float &m1, float &l1, float *o1, float m2, float l2, const float *o2) {
    const float M = fmaxf(m1, m2);
    const float Mu = (M == -INFINITY) ? 0.f : M;
    const float a1 = fast_exp2(m1 - Mu), a2 = fast_exp2(m2 - Mu);
    l1 = l1 * a1 + l2 * a2;
#pragma unroll
    for (int d = 0; d < ND; ++d) o1[d] = o1[d] * a1 + o2[d] * a2;
    m1 = M;
}

// One work-group of fa_decode_kernel: split `split` of the row group `unit`
// (KV head * row_groups + row group) of batch entry b.  The query is read
// first, then every step loads its keys.
template <typename T, int HD, int R, int NWV = 4, int NB = 4, bool KVFIRST = true>
__device__ __forceinline__ void fa_decode_block(const AttnArgs &a, int split, int unit, int64_t b) {
    // NB: keys per lane group per step; all K / V loads of a step are issued
    // before any is used, so a step is one memory round trip.  KVFIRST: the
    // first step's loads are issued with the query's (else after the query
    // is converted: fewer registers live across the query's arrival).
    constexpr int NT = NWV * 64;
    constexpr int LPK = HD / 8;       // lanes per key (8 d values each)
    constexpr int KPW = 64 / LPK;     // keys per wave step
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kg = lane / LPK, dl = lane % LPK;
    const int hk = unit / a.row_groups, rg = unit % a.row_groups;
    // head / query index arithmetic in 32 bits (a 64-bit division is a long
    // instruction sequence ahead of the Q loads); decode row counts are small
    const int G = (int)a.hq / (int)a.hkv;
    const int LQ = (int)a.l;
    const int rows_kv = G * (int)a.l;            // query rows sharing this KV head
    const int r0 = rg * a.rows_per_group;

    const T *Kp = reinterpret_cast<const T *>(a.K) + b * a.sk0 + hk * a.sk1;
    const T *Vp = reinterpret_cast<const T *>(a.V) + b * a.sv0 + hk * a.sv1;
    // keys of this batch entry: s, or the cache length read from device
    // memory (a graph-captured decode step keeps s at the cache capacity)
    const int64_t s_b = a.kv_len ? max((int64_t)0, min((int64_t)a.kv_len[b], a.s)) : a.s;
    const int64_t kbeg = (int64_t)split * a.chunk;
    const int64_t kend = min(s_b, kbeg + a.chunk);

    float m[R], lsum[R], o[R][8];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        m[r] = -INFINITY;
        lsum[r] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[r][e] = 0.f;
    }

    // The loop runs over the split's keys within the capacity s (known at
    // launch), not over the device key count: the K / V loads then need not
    // wait for kv_len.  Keys at or past kend are masked after loading.
    const int64_t kend_cap = min(a.s, kbeg + a.chunk);
    u32x4 kr[NB], vr[NB];
    auto load_kv = [&](int64_t kb) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int64_t key = min(kb + j * KPW + kg, kend_cap - 1);    // in-bounds address (s = 0: zero strides)
            kr[j] = *reinterpret_cast<const u32x4 *>(Kp + key * a.sk2 + dl * 8);
            vr[j] = *reinterpret_cast<const u32x4 *>(Vp + key * a.sv2 + dl * 8);
        }
    };
    const int64_t kb0 = kbeg + (int64_t)wave * KPW * NB;

    // Query rows: row r -> head hk*G + (r / l), query index r % l.
    float q[R][8];
    int64_t last_key[R];
    u32x4 qraw[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int rr = r0 + r;
        const bool ok = rr < rows_kv && r < a.rows_per_group;
        const int64_t head = hk * G + (ok ? rr / LQ : 0);
        const int64_t qi = ok ? rr % LQ : 0;
        qraw[r] = ok ? *reinterpret_cast<const u32x4 *>(reinterpret_cast<const T *>(a.Q) + b * a.sq0 + head * a.sq1 +
                                                        qi * a.sq2 + dl * 8)
                     : u32x4{0, 0, 0, 0};
    }
    // The first step's K / V loads go out right behind the query's, so the
    // query's conversion waits for the query alone and the key stream does
    // not start a memory round trip later (later steps load at the end of
    // the previous one).  Unconditional (a conditional load makes the
    // compiler wait for every load before the query is used): addresses are
    // clamped into the split's keys, and an empty cache (s = 0) is given K / V
    // pointers into the workspace with zero strides by the host.
    const int64_t kstep = (int64_t)NWV * KPW * NB;
    if constexpr (KVFIRST) load_kv(kb0);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int rr = r0 + r;
        const bool ok = rr < rows_kv && r < a.rows_per_group;
        const int64_t qi = ok ? rr % LQ : 0;
        typedef T t8 __attribute__((ext_vector_type(8)));
        t8 qv = __builtin_bit_cast(t8, qraw[r]);
#pragma unroll
        for (int e = 0; e < 8; ++e) q[r][e] = to_f32(qv[e]) * a.scale_log2;
        // keys visible to this row (exclusive bound)
        last_key[r] = ok ? (a.causal ? s_b - a.l + qi + 1 : s_b) : 0;
    }

    for (int64_t kb = kb0; kb < kend_cap; kb += kstep) {
        float s[R][NB];
        if constexpr (!KVFIRST) load_kv(kb);
        // keys past the device count are zeroed (their scores are masked
        // below; a zero V keeps a NaN in unused cache rows out of the sum)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            if (kb + j * KPW + kg >= kend) {
                kr[j] = u32x4{0, 0, 0, 0};
                vr[j] = u32x4{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            typedef T t8 __attribute__((ext_vector_type(8)));
            t8 kv = __builtin_bit_cast(t8, kr[j]);
            float kf[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) kf[e] = to_f32(kv[e]);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) d += q[r][e] * kf[e];
                d = group_sum<LPK>(d);
                s[r][j] = d;
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float mb = -INFINITY;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int64_t key = kb + j * KPW + kg;
                if (key >= kend || key >= last_key[r]) s[r][j] = -INFINITY;
                mb = fmaxf(mb, s[r][j]);
            }
            const float m_new = fmaxf(m[r], mb);
            const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
            const float alpha = fast_exp2(m[r] - m_use);
            float p[NB], ps = 0.f;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                p[j] = fast_exp2(s[r][j] - m_use);
                ps += p[j];
            }
            lsum[r] = lsum[r] * alpha + ps;
            m[r] = m_new;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[r][e] *= alpha;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                typedef T t8 __attribute__((ext_vector_type(8)));
                t8 vv = __builtin_bit_cast(t8, vr[j]);
#pragma unroll
                for (int e = 0; e < 8; ++e) o[r][e] += p[j] * to_f32(vv[e]);
            }
        }
        if constexpr (KVFIRST)
            if (kb + kstep < kend_cap) load_kv(kb + kstep);
    }

    // Merge the KPW key slots of a wave (lanes with equal dl) by a butterfly
    // over the lane bits above dl: partners compute the same commutative
    // merge, so every lane ends with the wave's bitwise-same state.  Then the
    // waves' states merge through LDS in wave order; a single split writes
    // the normalised output, otherwise the split's state goes to the
    // workspace.
#pragma unroll
    for (int sh = LPK; sh < 64; sh <<= 1) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float m2 = __shfl_xor(m[r], sh, 64), l2 = __shfl_xor(lsum[r], sh, 64);
            float o2[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o2[e] = __shfl_xor(o[r][e], sh, 64);
            merge_state<8>(m[r], lsum[r], o[r], m2, l2, o2);
        }
    }
    constexpr int NSL = NWV;
    __shared__ float sm[NSL][R], sl[NSL][R], so[NSL][R][HD];
    if (kg == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (dl == 0) { sm[wave][r] = m[r]; sl[wave][r] = lsum[r]; }
#pragma unroll
            for (int e = 0; e < 8; ++e) so[wave][r][dl * 8 + e] = o[r][e];
        }
    }
    __syncthreads();
    const int nrows = min(a.rows_per_group, rows_kv - r0);
    for (int idx = tid; idx < R * HD; idx += NT) {
        const int r = idx / HD, d = idx % HD;
        if (r >= nrows) continue;
        // max over the slots, then one weight per slot for its sum and output
        // (independent terms, summed in slot order)
        float mm = -INFINITY;
        for (int sv = 0; sv < NSL; ++sv) mm = fmaxf(mm, sm[sv][r]);
        const float mu = (mm == -INFINITY) ? 0.f : mm;
        float ll = 0.f, oo = 0.f;
        for (int sv = 0; sv < NSL; ++sv) {
            const float wgt = fast_exp2(sm[sv][r] - mu);
            ll = __builtin_fmaf(sl[sv][r], wgt, ll);
            oo = __builtin_fmaf(so[sv][r][d], wgt, oo);
        }
        const int rr = r0 + r;
        const int64_t head = hk * G + rr / LQ, qi = rr % LQ;
        const int64_t grow = (b * a.hq + head) * a.l + qi;
        if (a.splits == 1) {
            const T ov = from_f32<T>(oo * (ll > 0.f ? 1.f / ll : 0.f));
            const int64_t oidx = b * a.so0 + head * a.so1 + qi * a.so2 + d;
            reinterpret_cast<T *>(a.O)[oidx] = ov;
            if (a.lse && d == 0) a.lse[grow] = ll > 0.f ? (mm + __log2f(ll)) * kLn2 : -INFINITY;
            continue;
        }
        if (!a.counters) {
            // merged by the separate merge kernel
            a.ws_o[(grow * a.splits + split) * HD + d] = oo;
            if (d == 0) {
                a.ws_ml[(grow * a.splits + split) * 2 + 0] = mm;
                a.ws_ml[(grow * a.splits + split) * 2 + 1] = ll;
            }
            continue;
        }
        // agent-coherent stores (written through the XCD's L2): the
        // work-group that merges the splits may run on another XCD
        __hip_atomic_store(&a.ws_o[(grow * a.splits + split) * HD + d], oo, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        if (d == 0) {
            __hip_atomic_store(&a.ws_ml[(grow * a.splits + split) * 2 + 0], mm, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&a.ws_ml[(grow * a.splits + split) * 2 + 1], ll, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (a.splits == 1 || !a.counters) return;

    // The last of the group's split work-groups to arrive merges the splits
    // in split order (bitwise repeatable whatever the arrival order).
    // Ordering (as in the decode GEMM's merge): the split states are
    // agent-scope relaxed atomic stores (`global_store sc1`, written through
    // the per-XCD L2); each thread waits for their acknowledgements
    // (s_waitcnt(0)) before the barrier that precedes tid 0's agent-scope
    // counter RMW, and the merging work-group reads them with sc1 buffer
    // loads, which miss the non-coherent caches.  This relies on the hardware
    // rule that an acknowledged sc1 store is visible at the agent's coherence
    // point before a later RMW of the same agent, not on a release / acquire
    // pair (which would add an L2 write-back per XCD to every work-group).
    __shared__ int s_last;
    __shared__ float s_w[R][64];
    __shared__ float s_M[R], s_L[R];
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    unsigned *ctr = a.counters + ((b * a.hkv + hk) * a.row_groups + rg) * kAttnCounterStride;
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (unsigned)(a.splits - 1);
    __syncthreads();
    if (!s_last) return;
    // The split states are read with agent-coherent (sc1) buffer loads, which
    // unlike atomics can be batched.  Wave w turns row w's split maxima into
    // weights (splits <= 64, one per lane); thread (r, d) then sums
    // weight * o[split][d] in split order.
    const __amdgpu_buffer_rsrc_t rs_ml = __builtin_amdgcn_make_buffer_rsrc((void *)a.ws_ml, (short)0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs_o = __builtin_amdgcn_make_buffer_rsrc((void *)a.ws_o, (short)0, 0x7fffffff, 0x00020000);
    constexpr int kSc1 = kSc1Aux;
    auto grow_of = [&](int r) {
        const int rr = r0 + r;
        return (b * a.hq + hk * G + rr / LQ) * a.l + rr % LQ;
    };
    // Thread (r, d) = tid issues its o loads (at most 32 splits) before the
    // weights are known, so both arrive in one memory round trip.
    constexpr int kMaxSplits = 32;
    float ov[kMaxSplits];
    const bool pre = a.splits <= kMaxSplits && nrows * HD <= NT && tid < nrows * HD;
    if (pre) {
        const uint32_t base = (uint32_t)((grow_of(tid / HD) * a.splits * HD + tid % HD) * 4);
#pragma unroll
        for (int z = 0; z < kMaxSplits; ++z)
            ov[z] = z < a.splits ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                                       rs_o, base + (uint32_t)(z * HD * 4), 0, kSc1))
                                 : 0.f;
    }
    for (int r = wave; r < nrows; r += NWV) {
        const uint32_t base = (uint32_t)(grow_of(r) * a.splits * 2) * 4;
        // (the b32 loads return raw bits)
        const float mz = lane < a.splits
                             ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs_ml, base + lane * 8, 0, kSc1))
                             : -INFINITY;
        const float lz = lane < a.splits
                             ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs_ml, base + lane * 8 + 4, 0, kSc1))
                             : 0.f;
        const float M = wave_max(mz);
        const float Mu = (M == -INFINITY) ? 0.f : M;
        const float w = lane < a.splits ? fast_exp2(mz - Mu) : 0.f;
        s_w[r][lane] = w;
        const float L = wave_sum(w * lz);
        if (lane == 0) { s_M[r] = M; s_L[r] = L; }
    }
    __syncthreads();
    for (int idx = tid; idx < nrows * HD; idx += NT) {
        const int r = idx / HD, d = idx % HD;
        const int64_t grow = grow_of(r);
        float acc = 0.f;
        if (pre) {
#pragma unroll
            for (int z = 0; z < kMaxSplits; ++z)
                if (z < a.splits) acc += s_w[r][z] * ov[z];
        } else {
            const uint32_t base = (uint32_t)((grow * a.splits * HD + d) * 4);
            for (int z0 = 0; z0 < a.splits; z0 += 8) {
                float o8[8];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    o8[j] = z0 + j < a.splits ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                                                    rs_o, base + (uint32_t)((z0 + j) * HD * 4), 0, kSc1))
                                              : 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (z0 + j < a.splits) acc += s_w[r][z0 + j] * o8[j];
            }
        }
        const float L = s_L[r];
        const float inv = L > 0.f ? 1.f / L : 0.f;
        const int rr = r0 + r;
        const int64_t head = hk * G + rr / LQ, qi = rr % LQ;
        T *Op = reinterpret_cast<T *>(a.O) + b * a.so0 + head * a.so1 + qi * a.so2;
        Op[d] = from_f32<T>(acc * inv);
        if (a.lse && d == 0) a.lse[grow] = L > 0.f ? (s_M[r] + __log2f(L)) * kLn2 : -INFINITY;
    }
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One query row (unit = KV head * row_groups + row, rows_per_group 1) over a
// cache whose capacity a.s fits one step of the work-group (a.s <= NWV *
// KPW * NB keys): lane group kg of wave w holds keys j * NWV * KPW + w * KPW
// + kg (j < NB), all loaded at once; interleaved so that every wave holds
// about the same number of visible keys, and a j whose keys are all past the
// visible count is skipped by the whole wave.  Scores are dot products of
// the bf16 / f16 query and key pairs (exact products, fp32 sums) times
// scale * log2(e).  The work-group's maximum score is found first, so the
// key slots' sums of p = exp2(score - max) and p * v merge by plain addition
// (lanes of a wave by a butterfly, then the waves in wave order), with no
// rescaling.
//
// With PF the K / V loads are issued before the query is read (the
// persistent decode step reads the query, and key `fresh` >= 0, through IO
// from work-groups of the same launch, polling epoch-tagged words).
template <typename T, int HD, int NWV, int NB, typename IO = PlainIO, bool PF = false>
__device__ __forceinline__ void fa_decode_onepass_block(const AttnArgs &a, int unit, int64_t b, int64_t fresh = -1) {
    constexpr int LPK = HD / 8;       // lanes per key (8 d values each)
    constexpr int KPW = 64 / LPK;     // keys per wave per j
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kg = lane / LPK, dl = lane % LPK;
    const int G = (int)a.hq / (int)a.hkv;
    const int LQ = (int)a.l;
    const int hk = unit / a.row_groups, rr = unit % a.row_groups;
    const int head = hk * G + rr / LQ, qi = rr % LQ;
    const T *Kp = reinterpret_cast<const T *>(a.K) + b * a.sk0 + hk * a.sk1;
    const T *Vp = reinterpret_cast<const T *>(a.V) + b * a.sv0 + hk * a.sv1;
    const int64_t s_b = a.use_s_len ? max((int64_t)0, min(a.s_len, a.s))
                                    : a.kv_len ? max((int64_t)0, min((int64_t)a.kv_len[b], a.s)) : a.s;
    constexpr int KPJ = NWV * KPW;                                 // keys per j
    const int64_t kw = (int64_t)wave * KPW + kg;                  // this lane group's key j = 0

    u32x4 kr[NB], vr[NB];
    auto load_kv = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int64_t key = min(kw + j * KPJ, a.s - 1);          // in-bounds address
            kr[j] = *reinterpret_cast<const u32x4 *>(Kp + key * a.sk2 + dl * 8);
            vr[j] = *reinterpret_cast<const u32x4 *>(Vp + key * a.sv2 + dl * 8);
        }
    };
    if constexpr (PF) load_kv();

    // this lane's key among fresh_lo .. fresh (keys of a lane are KPJ apart,
    // so at most one when the range is shorter than KPJ): its j, or -1
    int jw = -1;
    int64_t sw = 0;
    if (IO::kLL && fresh >= 0) {
        const int64_t lo = min(a.fresh_lo, fresh);
        const int64_t jj = lo > kw ? (lo - kw + KPJ - 1) / KPJ : 0;
        if (jj < NB && kw + jj * KPJ <= fresh) {
            jw = (int)jj;
            sw = kw + jj * KPJ - lo;
        }
    }
    u32x4 qraw, kfr = {0, 0, 0, 0}, vfr = {0, 0, 0, 0};
    auto load_q = [&]() -> bool {
        bool ok = IO::ld8(a.Q, b * a.sq0 + head * a.sq1 + qi * a.sq2 + dl * 8, a.ep_q, qraw);
        if constexpr (IO::kLL) {
            if (jw >= 0) {
                const int64_t e = sw * a.fresh_stride + hk * HD + dl * 8;
                const uint32_t ep = a.ep_fresh0 + (uint32_t)sw * a.ep_fresh_step;
                ok = IO::ld8(a.kfresh, e, ep, kfr) && ok;
                ok = IO::ld8(a.vfresh, e, ep, vfr) && ok;
            }
        }
        return ok;
    };
    if constexpr (IO::kLL) {
        // every lane reads its query chunk (and the new k / v chunk) until it
        // is the expected write (each wave on its own), then the work-group meets
        bool ok = load_q();
        unsigned e = ll_err_read(a.err);
        for (unsigned it = 0; !__all(ok); ++it) {
            if (ll_expired(it, e, a.err)) break;
            __builtin_amdgcn_s_sleep(kLLSleep);
            if (!ok) ok = load_q();
            e = ll_err_read(a.err);
        }
        __syncthreads();
    } else {
        load_q();
    }
    // the query's load stays ahead of the K / V loads in issue order (the
    // compiler would hoist them above it), so its wait leaves them in flight
    // and the scores start as K arrives (batch-8 step 0.779 -> 0.777 ms)
    if constexpr (!PF) __builtin_amdgcn_sched_barrier(0);
    if constexpr (!PF) load_kv();
    if (PF && fresh >= 0) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            if (IO::kLL ? j == jw : kw + j * KPJ == fresh) {
                if constexpr (IO::kLL) {
                    kr[j] = kfr;
                    vr[j] = vfr;
                } else {
                    kr[j] = IO::ld(reinterpret_cast<const u32x4 *>(Kp + fresh * a.sk2 + dl * 8));
                    vr[j] = IO::ld(reinterpret_cast<const u32x4 *>(Vp + fresh * a.sv2 + dl * 8));
                }
            }
        }
    }

    // keys visible to this row (exclusive bound); V of the others is zeroed
    // (their p is 0, and a NaN in an unused cache row stays out of the sums)
    const int64_t lim = min(s_b, a.causal ? s_b - a.l + qi + 1 : s_b);
    // j < nj: the j whose keys of this wave are not all past lim (uniform)
    const int64_t w0 = (int64_t)wave * KPW;
    const int nj = lim > w0 ? (int)min((int64_t)NB, (lim - w0 + KPJ - 1) / KPJ) : 0;
    float sc[NB];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        sc[j] = -INFINITY;
        if (j < nj) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) d = dot2<T>(kr[j][e], qraw[e], d);
            d = group_sum<LPK>(d);
            const bool vis = kw + j * KPJ < lim;
            sc[j] = vis ? d * a.scale_log2 : -INFINITY;
            if (!vis) vr[j] = u32x4{0, 0, 0, 0};
            mx = fmaxf(mx, sc[j]);
        }
    }
    if constexpr (LPK <= 8) mx = xor_max<8>(mx);
    if constexpr (LPK <= 16) mx = xor_max<16>(mx);
    mx = xor_max<32>(mx);
    __shared__ float s_mx[NWV], s_l[NWV], s_o[NWV][HD];
    if (lane == 0) s_mx[wave] = mx;
    __syncthreads();
    float M = s_mx[0];
#pragma unroll
    for (int w = 1; w < NWV; ++w) M = fmaxf(M, s_mx[w]);
    const float Mu = (M == -INFINITY) ? 0.f : M;

    float l = 0.f, o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.f;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        if (j < nj) {
            const float pj = fast_exp2(sc[j] - Mu);
            l += pj;
            typedef T t8 __attribute__((ext_vector_type(8)));
            const t8 vv = __builtin_bit_cast(t8, vr[j]);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = __builtin_fmaf(pj, to_f32(vv[e]), o[e]);
        }
    }
    // lanes with equal dl: sums commute, so partners hold bitwise-equal totals
    if constexpr (LPK <= 8) {
        l = xor_add<8>(l);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = xor_add<8>(o[e]);
    }
    if constexpr (LPK <= 16) {
        l = xor_add<16>(l);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = xor_add<16>(o[e]);
    }
    l = xor_add<32>(l);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = xor_add<32>(o[e]);
    if (kg == 0) {
        if (dl == 0) s_l[wave] = l;
#pragma unroll
        for (int e = 0; e < 8; ++e) s_o[wave][dl * 8 + e] = o[e];
    }
    __syncthreads();
    if (tid >= HD) return;
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < NWV; ++w) {
        L += s_l[w];
        O += s_o[w][tid];
    }
    const T ov = from_f32<T>(O * (L > 0.f ? 1.f / L : 0.f));
    const int64_t oidx = b * a.so0 + (int64_t)head * a.so1 + (int64_t)qi * a.so2 + tid;
    if constexpr (IO::kLL) {
        // element pairs (d, d + 1) in one epoch-tagged word (neighbour lanes)
        const uint16_t nb = (uint16_t)lane_xor1((int)__builtin_bit_cast(uint16_t, ov));
        if ((tid & 1) == 0) IO::st2(reinterpret_cast<T *>(a.O), oidx, ov, __builtin_bit_cast(T, nb), a.ep_o);
    } else {
        IO::st(reinterpret_cast<T *>(a.O) + oidx, ov);
    }
    if (a.lse && tid == 0) a.lse[((int64_t)b * a.hq + head) * a.l + qi] = L > 0.f ? (M + __log2f(L)) * kLn2 : -INFINITY;
}

template <typename T, int HD, int NWV, int NB>
__global__ __launch_bounds__(NWV * 64) void fa_decode_onepass_kernel(AttnArgs a) {
    // consecutive (KV head, row) units spread so that all rows of a KV head
    // run on one XCD (its K / V then come from that XCD's L2 after the first read)
    int unit = blockIdx.y;
    if ((gridDim.y & 7) == 0) unit = (unit & 7) * (gridDim.y >> 3) + (unit >> 3);
    fa_decode_onepass_block<T, HD, NWV, NB>(a, unit, blockIdx.z);
}

template <typename T, int HD, int R, int NWV = 4, int NB = 4, bool KVFIRST = true>
__global__ __launch_bounds__(NWV * 64) void fa_decode_kernel(AttnArgs a) {
    // One split, many row groups: work-groups are dispatched round-robin
    // over the 8 XCDs, so consecutive (KV head, row group) units are spread
    // to give all row groups of a KV head one XCD (its K / V then come from
    // that XCD's L2 after the first read).
    int unit = blockIdx.y;
    if (gridDim.x == 1 && (gridDim.y & 7) == 0) unit = (unit & 7) * (gridDim.y >> 3) + (unit >> 3);
    fa_decode_block<T, HD, R, NWV, NB, KVFIRST>(a, blockIdx.x, unit, blockIdx.z);
}

}  // namespace kuiops
