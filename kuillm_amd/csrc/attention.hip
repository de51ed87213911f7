// Scaled dot-product attention for gfx950.
//
// fa_fwd_kernel -- flash-attention forward (prefill), bf16/f16, head dim 64/128.
//   A work-group owns 128 queries of one (batch, head) and walks the keys in
//   blocks of 64 staged through LDS (two stages, register prefetch).  Each of
//   the 4 waves owns 32 queries and computes the TRANSPOSED score tile
//   S^T = K Q^T with 32x32x16 MFMAs, so a lane holds 32 scores of a single
//   query: the row max / row sum of the online softmax are in-lane reductions
//   plus one cross-half swap (lane ^ 32).  The output is accumulated
//   transposed as well, O^T += V^T P^T, with P^T taken straight from the
//   score registers.  MFMA sums over K in any order, so the keys of one
//   16-key step are numbered in the order the score accumulator holds them;
//   V is transposed into LDS in that same order ([d][key], 4-key groups
//   permuted 0,2,1,3 inside each 16) and one ds_read_b128 yields an operand.
//   Softmax runs in the log2 domain (exp2 on the hardware exp unit) in fp32.
//   Causal grids that give every CU a work-group pair query blocks p and
//   nqb-1-p in one work-group (equal work everywhere; the second block walks
//   its keys backwards so all work-groups stream the same key blocks);
//   smaller ones run single blocks heaviest-first.  All q-blocks of one head
//   are mapped to one XCD so its K / V stay in that XCD's L2.
//
// fa_decode_kernel -- decode (few queries per head) over a long KV cache:
//   HBM-bound, so the keys are split over work-groups (split-KV); each
//   work-group streams its key range once for all query rows that share the
//   KV head (grouped-query attention), keeps fp32 online-softmax state per
//   row and writes (max, sum, unnormalised output) to the workspace; the last
//   work-group of a row group to finish merges the splits in split order.
//
// Semantics: aten scaled_dot_product_attention (the reference's fallthrough,
// kuipy/kuiops.py:627-681 rejects is_causal; tests/test_jit_ops.py:173-193).
#include <algorithm>

#include "attn_decode.hpp"

namespace kuiops {



__device__ __forceinline__ int swz8(int row) { return (row ^ (row >> 3)) & 7; }

template <typename T>
__device__ __forceinline__ u32x4 pack8(const float *v) {
    typedef T t8 __attribute__((ext_vector_type(8)));
    t8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = from_f32<T>(v[i]);
    return __builtin_bit_cast(u32x4, r);
}

typedef __attribute__((address_space(3))) char lds_char;
typedef short s16x4 __attribute__((ext_vector_type(4)));

// Generic -> LDS pointer with provenance kept (see the GEMM kernels).
__device__ __forceinline__ lds_char *to_lds(const void *p) { return (lds_char *)(const_cast<void *>(p)); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
// 16 bytes per lane from (descriptor, lane offset, uniform offset) into
// dst + 16 * lane; reads past the descriptor's size return zeros.
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, const void *dst) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)to_lds(dst), 16,
                                             (int)voff, (int)soff, 0, 0);
}

// Threshold (log2 domain) by which the running max may grow before O and l
// are rescaled: probabilities stay below 2^8 meanwhile.
constexpr float kRescaleSlack = 8.0f;

template <typename T, int HD, bool CAUSAL, int NWV, bool BIAS = false, bool PRIO = true>
__global__ __launch_bounds__(NWV * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void fa_fwd_kernel(AttnArgs a) {
    constexpr int BQ = 32 * NWV, BKV = 64;          // 32 queries per wave
    constexpr int RB = HD * 2;                      // bytes per K / V row
    constexpr int CPR = HD / 8;                     // 16-byte chunks per row
    constexpr int TILE = BKV * RB;                  // bytes per K or V tile
    constexpr int DPW = TILE / 1024 / NWV;          // 1 KB DMA blocks per wave per tile
    constexpr int RPB = 1024 / RB;                  // rows per DMA block
    constexpr int DT = HD / 32;                     // 32-row d tiles of O^T
    typedef typename Mfma<T>::frag frag;
    static_assert(DPW >= 1, "tile split");

    // LDS swizzles (64 banks = 256 bytes per cycle).  K rows, read with
    // ds_read_b128 (16 consecutive rows per cycle): chunk c sits at c ^ kswz(r),
    // which gives those 16 rows distinct 16-byte slots.  V rows, read with
    // ds_read_b64_tr_b16 (8 rows x 64 bytes per instruction): chunk c sits at
    // c ^ vswz(r), spreading each group of 4 rows over the whole bank width.
    auto kswz = [](int r) { return CPR == 16 ? (r & 15) : ((r >> 1) & 7); };
    auto vswz = [](int r) { return CPR == 16 ? 4 * (r & 3) : 4 * ((r >> 1) & 1); };
    __shared__ __attribute__((aligned(1024))) char sK0[TILE], sV0[TILE], sK1[TILE], sV1[TILE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lq = lane & 31, lh = lane >> 5;
    const int G = lane >> 4, qq = lane & 15;

    const int nblocks = gridDim.x, bid = blockIdx.x;
    // (PRIO: the work-groups dispatched second to a CU run one priority level
    // above the first ones, which otherwise win the age-ordered issue ties)
    const bool young = PRIO && bid >= nblocks / 2;
    int w = bid;
    if ((nblocks & 7) == 0) w = (bid & 7) * (nblocks >> 3) + (bid >> 3);
    // Work units per (batch, head): one query block each, or (causal, paired)
    // the pair of blocks p and nqb - 1 - p, which together cost nqb + 1 key
    // blocks whatever p is, so every work-group has the same work.
    const int upb = a.pair ? a.nqb >> 1 : a.nqb;
    const int hb = w / upb;
    const int unit = w - hb * upb;
    const int64_t b = hb / a.hq, h = hb - b * a.hq;
    const int64_t hk = h / (a.hq / a.hkv);

    const T *Qp = reinterpret_cast<const T *>(a.Q) + b * a.sq0 + h * a.sq1;
    const char *Kb = reinterpret_cast<const char *>(reinterpret_cast<const T *>(a.K) + b * a.sk0 + hk * a.sk1);
    const char *Vb = reinterpret_cast<const char *>(reinterpret_cast<const T *>(a.V) + b * a.sv0 + hk * a.sv1);
    // Descriptors end at the last key: the rows of a partial last block read 0.
    const uint32_t kbytes = (uint32_t)min((int64_t)0x7fffffff, ((a.s - 1) * a.sk2 + HD) * 2);
    const uint32_t vbytes = (uint32_t)min((int64_t)0x7fffffff, ((a.s - 1) * a.sv2 + HD) * 2);
    const __amdgpu_buffer_rsrc_t rsK = make_rsrc(Kb, a.s > 0 ? kbytes : 0);
    const __amdgpu_buffer_rsrc_t rsV = make_rsrc(Vb, a.s > 0 ? vbytes : 0);

    for (int pass = 0; pass < (a.pair ? 2 : 1); ++pass) {
    // heaviest block first: the last (causal) block of the pair, or of the head
    const int qb = CAUSAL ? (pass == 0 ? a.nqb - 1 - unit : unit) : unit;
    if (pass) __syncthreads();      // every wave is done with the LDS slots
    const int64_t q0 = (int64_t)qb * BQ;
    const int64_t qw = q0 + wave * 32;
    const int64_t myq = qw + lq;

    frag qf[HD / 16];
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) {
        const int ch = 2 * kk + lh;
        qf[kk] = as_frag<frag>(myq < a.l ? *reinterpret_cast<const u32x4 *>(Qp + myq * a.sq2 + ch * 8)
                                         : u32x4{0, 0, 0, 0});
    }

    int64_t kv_end = a.s;
    if (CAUSAL) kv_end = min(a.s, q0 + BQ);
    const int nkv = (int)((kv_end + BKV - 1) / BKV);

    // Per-lane DMA byte offsets within a KV block (uniform part: block start).
    uint32_t offK[DPW], offV[DPW];
#pragma unroll
    for (int j = 0; j < DPW; ++j) {
        const int blk = wave * DPW + j;
        const int r = blk * RPB + lane / CPR;
        const int p = lane % CPR;
        offK[j] = (uint32_t)((r * a.sk2 + ((p ^ kswz(r)) * 8)) * 2);
        offV[j] = (uint32_t)((r * a.sv2 + ((p ^ vswz(r)) * 8)) * 2);
    }
    auto issue_k = [&](int kt, char *sk) __attribute__((always_inline)) {
        const uint32_t kb = (uint32_t)((int64_t)kt * BKV * a.sk2 * 2);
#pragma unroll
        for (int j = 0; j < DPW; ++j) dma16_buf(rsK, offK[j], kb, sk + (wave * DPW + j) * 1024);
    };
    auto issue_v = [&](int kt, char *sv) __attribute__((always_inline)) {
        const uint32_t vb = (uint32_t)((int64_t)kt * BKV * a.sv2 * 2);
#pragma unroll
        for (int j = 0; j < DPW; ++j) dma16_buf(rsV, offV[j], vb, sv + (wave * DPW + j) * 1024);
    };

    // LDS offsets of this lane's operands.  K (A operand of S^T = K Q^T): key
    // row 32t + lq, chunk 2kk + lh.  V^T (A operand of O^T += V^T P^T): d row
    // 32dt + lq; the 8 key slots of lane half lh are keys 4lh..4lh+3 and
    // 8+4lh..8+4lh+3 of each 16-key step (the order the score accumulator
    // holds them), each 4 fetched by one transposing read.
    int offKr[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) offKr[t] = (t * 32 + lq) * RB;
    const int kpos = kswz(lq);                      // == kswz(32t + lq)
    int offVr[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
        const int krow = 4 * (G >> 1) + (qq >> 2);   // + 16 * step (+ 8 for the second read)
        const int d = dt * 32 + 16 * (G & 1) + 4 * (qq & 3);
        offVr[dt] = krow * RB + (((d >> 3) ^ vswz(krow)) << 4) + ((d >> 2) & 1) * 8;   // vswz(krow + 16s + 8h) == vswz(krow)
    }

    f32x16 o[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[t][e] = 0.f;
    float m_used = -INFINITY, l_run = 0.f;

    // Bias of this lane's query for the 32 score slots of a key block: slot
    // (t, e) is key kv0 + 32t + 8(e/4) + 4lh + e%4, so each (t, e/4) is 4
    // consecutive keys, one 8-byte load.  Loaded one block ahead (br), added
    // (times 1/scale) to the raw scores at the start of the block's step.
    typedef T t4v __attribute__((ext_vector_type(4)));
    t4v br[8];
    const T *brow = nullptr;
    if constexpr (BIAS) {
        const int64_t qrow = myq < a.l ? myq : a.l - 1;
        brow = reinterpret_cast<const T *>(a.bias) + b * a.sb0 + h * a.sb1 + qrow * a.sb2;
    }
    auto load_bias = [&](int64_t kv0) __attribute__((always_inline)) {
        if constexpr (BIAS) {
            if (kv0 + BKV <= a.s) {
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    br[i] = *reinterpret_cast<const t4v *>(brow + kv0 + 32 * (i >> 2) + 8 * (i & 3) + 4 * lh);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const int64_t key = kv0 + 32 * (i >> 2) + 8 * (i & 3) + 4 * lh + c;
                        br[i][c] = key < a.s ? brow[key] : (T)0.f;
                    }
            }
        }
    };
    auto add_bias = [&](f32x16 *sc) __attribute__((always_inline)) {
        if constexpr (BIAS) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    sc[t][e] = __builtin_fmaf(to_f32(br[4 * t + (e >> 2)][e & 3]), a.inv_scale, sc[t][e]);
        }
    };

    // S^T block = K_blk Q^T: sc[t][e] = score of key kv0 + 32t + 8(e/4) + 4lh + e%4, query myq.
    auto qk = [&](const char *pk, f32x16 *sc) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) sc[t][e] = 0.f;
#pragma unroll
        for (int kk = 0; kk < HD / 16; ++kk) {
            const int pos = ((2 * kk + lh) ^ kpos) << 4;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const frag kf = as_frag<frag>(*reinterpret_cast<const u32x4 *>(pk + offKr[t] + pos));
                sc[t] = Mfma<T>::m32(kf, qf[kk], sc[t]);
            }
        }
    };
    // One pipeline step on score block `cur` (keys kv0 ..): mask and row
    // max, lazy rescale, then exp(cur) interleaved with the MFMAs of the next
    // block's scores (K slot `pk`, into `nxt`), then O^T += V^T P^T.
    auto step = [&](f32x16 *cur, f32x16 *nxt, const char *pk, const char *pv, int64_t kv0, int64_t kv_next)
        __attribute__((always_inline)) {
        if constexpr (BIAS) {
            add_bias(cur);
            if (kv_next >= 0) load_bias(kv_next);
        }
        const bool need_mask = (kv0 + BKV > a.s) || (CAUSAL && kv0 + BKV - 1 > qw);
        if (need_mask) {
            // key offset within the block of lane-slot (t, e) is 32t + 8(e/4) + 4lh + e%4
            const int64_t last = CAUSAL ? min(myq, a.s - 1) : a.s - 1;   // last visible key
            const int64_t lim = last - kv0 - 4 * lh;                       // its offset (minus 4lh)
            const int lim32 = (int)max((int64_t)-1, min(lim, (int64_t)BKV));
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    if (t * 32 + (e >> 2) * 8 + (e & 3) > lim32) cur[t][e] = -INFINITY;
        }
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) mx = fmaxf(mx, cur[t][e]);
        mx = xor_max<32>(mx) * a.scale_log2;
        // Lazy rescale: move the reference max only when it grew by more
        // than the slack (or is still -inf), for the whole wave at once.
        if (__any(mx > m_used + kRescaleSlack)) {
            const float m_new = fmaxf(m_used, mx);
            const float alpha = (m_new == -INFINITY) ? 1.f : fast_exp2(m_used - m_new);
            l_run *= alpha;
#pragma unroll
            for (int t = 0; t < DT; ++t)
#pragma unroll
                for (int e = 0; e < 16; ++e) o[t][e] *= alpha;
            m_used = m_new;
        }
        const float mref = (m_used == -INFINITY) ? 0.f : m_used;
        float rs = 0.f;
        constexpr int KS = HD / 16;                 // MFMA k-steps of one score block
        constexpr int EPK = 32 / KS;                // exps per k-step
        // K fragments are read KPF k-steps ahead of their MFMAs (a ring of
        // registers), so the LDS latency hides behind the MFMAs in flight.
        constexpr int KPF = 3;
        frag kr[KPF][2];
        auto load_k = [&](int kk, frag *dst) __attribute__((always_inline)) {
            const int pos = ((2 * kk + lh) ^ kpos) << 4;
#pragma unroll
            for (int t = 0; t < 2; ++t) dst[t] = as_frag<frag>(*reinterpret_cast<const u32x4 *>(pk + offKr[t] + pos));
        };
        // With two waves per SIMD (PRIO), a wave in the MFMA phases (scores +
        // exps, then P V) runs at raised priority, so the other wave's row max
        // and rescale fill its gaps: 2% at causal S=4096.  With one wave per
        // SIMD the priority changes only constrain the schedule (2% slower
        // at S=2048), so that instance has none.
        if constexpr (PRIO) {
            if (young) __builtin_amdgcn_s_setprio(2);
            else __builtin_amdgcn_s_setprio(1);
        }
#pragma unroll
        for (int kk = 0; kk < KPF - 1; ++kk) load_k(kk, kr[kk]);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            if (kk + KPF - 1 < KS) load_k(kk + KPF - 1, kr[(kk + KPF - 1) % KPF]);
#pragma unroll
            for (int t = 0; t < 2; ++t)      // (the first k-step starts from a zero accumulator operand)
                nxt[t] = Mfma<T>::m32(kr[kk % KPF][t], qf[kk], kk == 0 ? f32x16{} : nxt[t]);
#pragma unroll
            for (int i = 0; i < EPK; ++i) {
                const int idx = kk * EPK + i, t = idx >> 4, e = idx & 15;
                const float p = fast_exp2(__builtin_fmaf(cur[t][e], a.scale_log2, -mref));
                cur[t][e] = p;
                rs += p;
            }
        }
        l_run += rs;
        // V^T fragments (two transposing reads each), VPF MFMAs ahead.
        constexpr int NV = 4 * DT, VPF = 3;
        frag vr[VPF];
        auto load_v = [&](int idx, frag &dst) __attribute__((always_inline)) {
            const int b16 = idx / DT, dt = idx % DT;
            const char *vb = pv + offVr[dt] + b16 * 16 * RB;
            const s16x4 t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4 *)to_lds(vb));
            const s16x4 t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4 *)to_lds(vb + 8 * RB));
            const u32x2 h0 = __builtin_bit_cast(u32x2, t0), h1 = __builtin_bit_cast(u32x2, t1);
            dst = as_frag<frag>(u32x4{h0[0], h0[1], h1[0], h1[1]});
        };
#pragma unroll
        for (int i = 0; i < VPF - 1; ++i) load_v(i, vr[i]);
        frag pf;
#pragma unroll
        for (int idx = 0; idx < NV; ++idx) {
            const int b16 = idx / DT, dt = idx % DT;
            if (dt == 0) {
                const int t = b16 >> 1, u = b16 & 1;
                float pv8[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) pv8[i] = cur[t][8 * u + i];
                pf = as_frag<frag>(pack8<T>(pv8));
            }
            if (idx + VPF - 1 < NV) load_v(idx + VPF - 1, vr[(idx + VPF - 1) % VPF]);
            o[dt] = Mfma<T>::m32(vr[idx % VPF], pf, o[dt]);
        }
        if constexpr (PRIO) {
            if (young) __builtin_amdgcn_s_setprio(1);
            else __builtin_amdgcn_s_setprio(0);
        }
    };

    // Software pipeline over KV blocks: step j runs the softmax of block j
    // (VALU) interleaved with the score MFMAs of block j + 1, then
    // O += P_j V_j, so each wave keeps both pipes fed.  LDS slots: K_j and
    // V_j in slot j % 2.  Step j needs K_{j+1} and V_j; it refills slot j % 2
    // with K_{j+2} (K_j was consumed at step j - 1) and slot (j + 1) % 2 with
    // V_{j+1} (V_{j-1} was consumed at step j - 1).  The last step computes
    // scores of a stale K slot, which are never used: no branch in the step.
    // Waves whose queries are all masked in a block still run it (their
    // probabilities are 0).
    const bool live = qw < a.l;
    // Key-block order: the second block of a causal pair walks its keys
    // backwards.  At step t of a work-group, pair p is at key block t during
    // its first block (2(nqb - p) steps) and at 2p + 1 - (t - 2(nqb - p)) =
    // 2 nqb + 1 - t during its second: whatever p, every work-group of the
    // launch is at one of just two key blocks, so the K / V blocks they
    // stream stay shared in L2.  The online softmax is order-independent up
    // to rounding.
    const bool rev = CAUSAL && a.pair && pass == 1;
    auto kvb = [&](int j) { return rev ? nkv - 1 - j : j; };
    f32x16 scA[2], scB[2];
    if (nkv > 0) {
        if (live) load_bias((int64_t)kvb(0) * BKV);
        issue_k(kvb(0), sK0);
        issue_v(kvb(0), sV0);
        if (nkv > 1) issue_k(kvb(1), sK1);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (live) qk(sK0, scA);
    }
    for (int j0 = 0; j0 < nkv; j0 += 2) {
#pragma unroll
        for (int hs = 0; hs < 2; ++hs) {
            const int j = j0 + hs;
            if (j >= nkv) break;
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (j + 2 < nkv) issue_k(kvb(j + 2), hs ? sK1 : sK0);
            if (j + 1 < nkv) issue_v(kvb(j + 1), hs ? sV0 : sV1);
            if (live) step(hs ? scB : scA, hs ? scA : scB, hs ? sK0 : sK1, hs ? sV1 : sV0, (int64_t)kvb(j) * BKV,
                           j + 1 < nkv ? (int64_t)kvb(j + 1) * BKV : -1);
        }
    }

    const float l_tot = xor_add<32>(l_run);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (myq < a.l) {
        T *Op = reinterpret_cast<T *>(a.O) + b * a.so0 + h * a.so1 + myq * a.so2;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = dt * 32 + j * 8 + lh * 4;
                typedef T t4 __attribute__((ext_vector_type(4)));
                t4 v;
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = from_f32<T>(o[dt][4 * j + i] * inv);
                *reinterpret_cast<t4 *>(Op + d) = v;
            }
        if (a.lse && lh == 0)
            a.lse[(b * a.hq + h) * a.l + myq] = l_tot > 0.f ? (m_used + __log2f(l_tot)) * kLn2 : -INFINITY;
    }
    }   // pass
}

// Separate merge for many splits (one work-group per query row; see the
// host launch): wave 0 turns the split maxima into weights
// (splits <= 64, one per lane), then thread d sums weight * o[split][d] over
// the splits in split order.
template <typename T, int HD>
__global__ __launch_bounds__(128) void fa_decode_combine_kernel(AttnArgs a) {
    const int64_t grow = blockIdx.x;            // (b * hq + head) * l + qi
    const int tid = threadIdx.x;
    const int64_t qi = grow % a.l, bh = grow / a.l;
    const int64_t head = bh % a.hq, b = bh / a.hq;
    __shared__ float s_w[64];
    __shared__ float s_M, s_L;
    const float *ml = a.ws_ml + grow * a.splits * 2;
    // The partial outputs do not depend on the weights: load (up to 32 of)
    // them together with the split maxima, so the kernel is one round trip.
    constexpr int PRE = 32;
    const float *o = a.ws_o + grow * a.splits * HD + min(tid, HD - 1);
    float op[PRE];
#pragma unroll
    for (int z = 0; z < PRE; ++z) op[z] = z < a.splits ? o[z * HD] : 0.f;
    if (tid < 64) {
        const float mz = tid < a.splits ? ml[2 * tid] : -INFINITY;
        const float lz = tid < a.splits ? ml[2 * tid + 1] : 0.f;
        const float M = wave_max(mz);
        const float Mu = (M == -INFINITY) ? 0.f : M;
        const float w = tid < a.splits ? fast_exp2(mz - Mu) : 0.f;
        s_w[tid] = w;
        const float L = wave_sum(w * lz);
        if (tid == 0) { s_M = M; s_L = L; }
    }
    __syncthreads();
    const float L = s_L, M = s_M;
    const float inv = L > 0.f ? 1.f / L : 0.f;
    if (tid < HD) {
        float acc = 0.f;
#pragma unroll
        for (int z = 0; z < PRE; ++z)
            if (z < a.splits) acc += s_w[z] * op[z];
        for (int z = PRE; z < a.splits; ++z) acc += s_w[z] * o[z * HD];
        T *Op = reinterpret_cast<T *>(a.O) + b * a.so0 + head * a.so1 + qi * a.so2;
        Op[tid] = from_f32<T>(acc * inv);
    }
    if (a.lse && tid == 0) a.lse[grow] = L > 0.f ? (M + __log2f(L)) * kLn2 : -INFINITY;
}

// ------------------------------------------------------------------------
// sdpa_general_kernel -- every other SDPA: fp32 / fp64 (and 16-bit) inputs,
// head dims e != ev, head dims past the MFMA kernels' 64 / 128, an optional
// additive bias of any alignment.  The reference's own family takes any float
// dtype and any (e, ev) (kuipy/kuiops.py:640-648), with a plain launcher
// (sdpa/wrapper_sdpa.cu.j2:21-30); this is the matching coverage path, SIMT in
// the accumulation type (fp32, fp64 for fp64 inputs).  One wave per query
// row, 4 rows per work-group: the query row sits in LDS; keys go in chunks
// of 64, lane j scoring key c0 + j (a dot product over its own K row), the
// chunk's maximum moves the running maximum (online softmax, natural
// exponent), the chunk's probabilities pass through LDS and each lane
// accumulates its output columns d = lane + 64 t from the chunk's V rows
// (coalesced).  score = scale * q.k + bias (aten's order), masked keys
// (causal: key j > query i) weigh 0; rows with no visible key give 0 and
// LSE = -inf.
constexpr int kGenRows = 4;          // query rows (waves) per work-group
constexpr int kGenMaxE = 1024;       // head dims served
constexpr int kGenAcc = kGenMaxE / 64;

template <typename T> struct GenAcc { typedef float type; };
template <> struct GenAcc<double> { typedef double type; };

__device__ __forceinline__ float gen_exp(float x) { return expf(x); }
__device__ __forceinline__ double gen_exp(double x) { return exp(x); }
__device__ __forceinline__ float gen_log(float x) { return logf(x); }
__device__ __forceinline__ double gen_log(double x) { return log(x); }
// accumulation type -> element type (fp64 stays fp64)
template <typename T, typename Acc> __device__ __forceinline__ T gen_out(Acc v) {
    if constexpr (sizeof(T) == 8) return v;
    else return from_f32<T>((float)v);
}

struct GenArgs {
    int64_t n, hq, hkv, l, s, e, ev;
    const void *Q, *K, *V, *bias;
    void *O;
    float *lse;
    int64_t sq0, sq1, sq2, sk0, sk1, sk2, sv0, sv1, sv2, so0, so1, so2, sb0, sb1, sb2;
    double scale;
    int causal;
};

template <typename T, int NACC>
__global__ __launch_bounds__(kGenRows * 64) void sdpa_general_kernel(GenArgs a) {
    typedef typename GenAcc<T>::type Acc;
    __shared__ Acc s_q[kGenRows][kGenMaxE];
    __shared__ Acc s_p[kGenRows][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row = (int64_t)blockIdx.x * kGenRows + wave;     // (b, h, i) flattened
    if (row >= a.n * a.hq * a.l) return;                            // whole wave leaves
    const int64_t i = row % a.l, bh = row / a.l, h = bh % a.hq, b = bh / a.hq;
    const int64_t hk = h / (a.hq / a.hkv);
    const T *Q = reinterpret_cast<const T *>(a.Q) + b * a.sq0 + h * a.sq1 + i * a.sq2;
    const T *K = reinterpret_cast<const T *>(a.K) + b * a.sk0 + hk * a.sk1;
    const T *V = reinterpret_cast<const T *>(a.V) + b * a.sv0 + hk * a.sv1;
    const T *B = a.bias ? reinterpret_cast<const T *>(a.bias) + b * a.sb0 + h * a.sb1 + i * a.sb2 : nullptr;
    for (int64_t d = lane; d < a.e; d += 64) s_q[wave][d] = (Acc)to_f32_or_self(Q[d]);
    __builtin_amdgcn_wave_barrier();
    const Acc scale = (Acc)a.scale;
    const int64_t kend = a.causal ? min(a.s, i + 1) : a.s;
    Acc m = -INFINITY, lsum = 0;
    Acc o[NACC];
#pragma unroll
    for (int t = 0; t < NACC; ++t) o[t] = 0;
    for (int64_t c0 = 0; c0 < kend; c0 += 64) {
        const int64_t key = c0 + lane;
        Acc sc = -INFINITY;
        if (key < kend) {
            const T *kr = K + key * a.sk2;
            Acc dot = 0;
            for (int64_t d = 0; d < a.e; ++d) dot += s_q[wave][d] * (Acc)to_f32_or_self(kr[d]);
            sc = scale * dot;
            if (B) sc += (Acc)to_f32_or_self(B[key]);
        }
        const Acc mc = wave_max(sc);
        const Acc m_new = m > mc ? m : mc;
        if (m_new == -INFINITY) continue;            // nothing visible yet (bias -inf)
        const Acc alpha = m == -INFINITY ? (Acc)0 : gen_exp(m - m_new);
        const Acc pj = sc == -INFINITY ? (Acc)0 : gen_exp(sc - m_new);
        lsum = lsum * alpha + wave_sum(pj);
#pragma unroll
        for (int t = 0; t < NACC; ++t) o[t] *= alpha;
        m = m_new;
        s_p[wave][lane] = pj;
        __builtin_amdgcn_wave_barrier();
        const int nk = (int)min((int64_t)64, kend - c0);
        for (int j = 0; j < nk; ++j) {
            const Acc p = s_p[wave][j];
            const T *vr = V + (c0 + j) * a.sv2;
#pragma unroll
            for (int t = 0; t < NACC; ++t) {
                const int64_t d = lane + 64 * t;
                if (d < a.ev) o[t] += p * (Acc)to_f32_or_self(vr[d]);
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
    T *O = reinterpret_cast<T *>(a.O) + b * a.so0 + h * a.so1 + i * a.so2;
    const Acc inv = lsum > 0 ? (Acc)1 / lsum : (Acc)0;
#pragma unroll
    for (int t = 0; t < NACC; ++t) {
        const int64_t d = lane + 64 * t;
        if (d < a.ev) O[d] = gen_out<T, Acc>(o[t] * inv);
    }
    if (a.lse && lane == 0) a.lse[row] = lsum > 0 ? (float)(m + gen_log(lsum)) : -INFINITY;
}

// ------------------------------------------------------------ host side

static bool attn_common_ok(int64_t n, int64_t hq, int64_t hkv, int64_t l, int64_t s, int64_t e, int64_t ev,
                           int dtype, const void *Q, const int64_t *sq, const void *K, const int64_t *sk,
                           const void *V, const int64_t *sv, void *O, const int64_t *so, int &status) {
    status = KUIOPS_OK;
    if (n < 0 || hq < 0 || hkv < 0 || l < 0 || s < 0 || e <= 0 || ev <= 0 || !sq || !sk || !sv || !so) {
        status = KUIOPS_E_INVALID;
        return false;
    }
    if (hkv == 0 || hq % hkv) { status = KUIOPS_E_INVALID; return false; }
    if (!Q || !K || !V || !O) { status = KUIOPS_E_INVALID; return false; }
    if (dtype != KUIOPS_BF16 && dtype != KUIOPS_F16) { status = KUIOPS_E_UNSUPPORTED; return false; }
    if (e != ev || (e != 64 && e != 128)) { status = KUIOPS_E_UNSUPPORTED; return false; }
    if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(O)) { status = KUIOPS_E_UNSUPPORTED; return false; }
    for (int i = 0; i < 3; ++i)
        if (sq[i] % 8 || sk[i] % 8 || sv[i] % 8 || so[i] % 4) { status = KUIOPS_E_UNSUPPORTED; return false; }
    return true;
}

// fa_fwd_kernel addresses one (batch, head)'s K / V through a buffer
// descriptor whose size field is 31 bits, with 32-bit byte offsets: the last
// key row must end below 2^31 bytes, and the offsets of the padding rows of
// the last 64-key block (which read zero past the descriptor) below 2^32.
static bool fwd_offsets_fit(int64_t s, int64_t e, int64_t sk2, int64_t sv2) {
    if (s == 0) return true;
    if (sk2 < 0 || sv2 < 0) return false;
    const int64_t st = sk2 > sv2 ? sk2 : sv2;
    if (((s - 1) * st + e) * 2 >= (int64_t(1) << 31)) return false;
    return ((s + 64) * st + e) * 2 < (int64_t(1) << 32);
}

static void fill_args(AttnArgs &a, int64_t n, int64_t hq, int64_t hkv, int64_t l, int64_t s, const void *Q,
                      const int64_t *sq, const void *K, const int64_t *sk, const void *V, const int64_t *sv,
                      void *O, const int64_t *so, float *lse, float scale, int causal) {
    a.n = n; a.hq = hq; a.hkv = hkv; a.l = l; a.s = s;
    a.Q = Q; a.K = K; a.V = V; a.O = O;
    a.sq0 = sq[0]; a.sq1 = sq[1]; a.sq2 = sq[2];
    a.sk0 = sk[0]; a.sk1 = sk[1]; a.sk2 = sk[2];
    a.sv0 = sv[0]; a.sv1 = sv[1]; a.sv2 = sv[2];
    a.so0 = so[0]; a.so1 = so[1]; a.so2 = so[2];
    a.lse = lse;
    a.scale_log2 = scale * 1.44269504088896340736f;
    a.causal = causal;
}

// Keys per split for the decode kernel: enough splits to fill the GPU, at
// least 64 keys each.
constexpr int kFusedMergeMaxSplits = 16;

static int64_t decode_chunk(int64_t s) {
    int64_t c = cdiv(cdiv(s, 32), 64) * 64;   // at most 32 splits
    return c < 64 ? 64 : c;
}

// Query rows per work-group (the rows sharing a KV head, up to 8).
static int decode_rows_per_group(int rows_kv) {
    return rows_kv <= 1 ? 1 : rows_kv <= 2 ? 2 : rows_kv <= 4 ? 4 : 8;
}

// Waves of the single-split kernel (as many as the row state's registers allow).
static int decode_single_waves(int R) { return R <= 2 ? 16 : 4; }   // the one-split launch's waves

// A cache that one work-group streams in a single step takes a single split
// (no workspace round trip): keys per step = waves x keys per wave-step.
// Longer caches are faster split: each step of a work-group is a dependent
// memory round trip, while splits overlap theirs.
static bool decode_single_split(int64_t s, int64_t ev, int R) {
    const int64_t per_step = (int64_t)decode_single_waves(R) * (64 / (ev / 8)) * 4;
    return s <= per_step;
}

// Caches of at most kDecodeWideWaves x (keys per wave step) x kDecodeWideNB
// keys (768 at head dim 64, 384 at 128) take the one-step row-wide kernel.
// Measured on the Llama-1B decode step (32 q / 8 kv heads, 640-key cache):
// 8 waves x 12 keys 6.2 us, 16 x 6 6.6 us, 4 x 20 6.7 us; 2 rows per
// work-group 8.6 us, 4 rows 16.2 us; split-KV with in-kernel merge 10.6 us.
// With many query rows (a batch of sequences) the row groups alone fill the
// GPU, and one work-group per row would re-read each KV head once per query
// head of its group, so the row-wide kernel is kept for at most
// kDecodeWideMaxRows rows.
constexpr int kDecodeWideWaves = 8, kDecodeWideNB = 12, kDecodeWideMaxRows = 256;
static bool decode_row_wide(int64_t s, int64_t hd, int64_t rows) {
    return s <= kDecodeWideWaves * (64 / (hd / 8)) * kDecodeWideNB && rows <= kDecodeWideMaxRows;
}

// Keys per split for a launch of `groups` row-group work-groups per split:
// enough splits for about two work-groups per CU, at most 32, and never
// fewer keys than decode_chunk (the workspace is sized by it).
static int64_t decode_chunk_for(int64_t s, int64_t groups) {
    const int64_t want = cdiv(2 * (int64_t)num_cus(), groups > 0 ? groups : 1);
    const int64_t splits = want < 1 ? 1 : (want > 32 ? 32 : want);
    const int64_t c = cdiv(cdiv(s, splits), 64) * 64;
    return c < decode_chunk(s) ? decode_chunk(s) : c;
}

// Workspace: split arrival counters (one per work-group row group, at most
// one per query row; zero between calls), then the split states.
static size_t decode_counter_bytes(int64_t rows) { return (size_t)cdiv(rows * 4 * kAttnCounterStride, 256) * 256; }

size_t decode_workspace_bytes(int64_t rows, int64_t kv_len, int64_t ev) {
    const int64_t splits = cdiv(kv_len > 0 ? kv_len : 1, decode_chunk(kv_len));
    return decode_counter_bytes(rows) + (size_t)rows * splits * (ev + 2) * sizeof(float) + 256;
}

template <typename T, int HD>
static int launch_fwd(AttnArgs a, hipStream_t st) {
    // 4 waves, 128 queries per work-group, two work-groups per CU.  (256
    // queries per work-group as 4 waves of 64 would halve the LDS reads per
    // MFMA, but needs more than 256 registers per wave; the compiler then
    // keeps the scores in accumulation registers and copies them for every
    // softmax step: 1.5x slower, measured.  8 waves of 32 queries, pairs of
    // 256-query blocks one per CU, halve the L2 -> LDS traffic but were 9%
    // slower at causal S=4096.  At S=2048 (one work-group per CU) an 8-wave
    // form in which two 4-wave groups split a pair's key blocks evenly, each
    // in its own LDS half, and merge the shared block's softmax state through
    // LDS was 5% slower (62.9 against 59.9 us): 256 VGPRs with spills.)
    a.nqb = (int)cdiv(a.l, 128);
    // Causal: pair the query blocks of a head (equal work per work-group)
    // when the pairs still give every CU a work-group.  Single blocks, even
    // heaviest first, end with the longest block alone: at S=2048 (32 heads,
    // 256 pairs, one per CU) pairing is 9% faster than 512 single blocks at
    // two per CU (64.5 -> 59.2 us); at S=4096 the 512 pairs fill both slots.
    const int64_t singles = (int64_t)a.nqb * a.n * a.hq;
    a.pair = (a.causal && (a.nqb & 1) == 0 && singles / 2 >= (int64_t)num_cus()) ? 1 : 0;
    const int64_t blocks = a.pair ? singles / 2 : singles;
    if (blocks > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    if (a.bias) {
        if (a.causal) hipLaunchKernelGGL((fa_fwd_kernel<T, HD, true, 4, true>), dim3((unsigned)blocks), dim3(256), 0, st, a);
        else hipLaunchKernelGGL((fa_fwd_kernel<T, HD, false, 4, true>), dim3((unsigned)blocks), dim3(256), 0, st, a);
    } else if (blocks < 2 * (int64_t)num_cus()) {
        // one work-group per CU: one wave per SIMD, no priority changes
        if (a.causal) hipLaunchKernelGGL((fa_fwd_kernel<T, HD, true, 4, false, false>), dim3((unsigned)blocks), dim3(256), 0, st, a);
        else hipLaunchKernelGGL((fa_fwd_kernel<T, HD, false, 4, false, false>), dim3((unsigned)blocks), dim3(256), 0, st, a);
    } else if (a.causal) {
        hipLaunchKernelGGL((fa_fwd_kernel<T, HD, true, 4>), dim3((unsigned)blocks), dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL((fa_fwd_kernel<T, HD, false, 4>), dim3((unsigned)blocks), dim3(256), 0, st, a);
    }
    return launch_status();
}

template <typename T, int HD>
static int launch_decode(AttnArgs a, hipStream_t st) {
    const int G = (int)(a.hq / a.hkv);
    const int rows_kv = G * (int)a.l;
    if (decode_row_wide(a.s, HD, a.n * a.hkv * rows_kv) && a.hkv * rows_kv <= 65535) {
        // short caches: one 8-wave work-group per query row loads every key
        // in one step (one memory round trip, no split merge); the rows of a
        // KV head share its K / V through L2
        a.rows_per_group = 1;
        a.row_groups = rows_kv;
        dim3 grid(1u, (unsigned)(a.hkv * rows_kv), (unsigned)a.n);
        hipLaunchKernelGGL((fa_decode_onepass_kernel<T, HD, kDecodeWideWaves, kDecodeWideNB>), grid,
                           dim3(kDecodeWideWaves * 64), 0, st, a);
        return launch_status();
    }
    const int R = decode_rows_per_group(rows_kv);
    a.rows_per_group = R;
    a.row_groups = (int)cdiv(rows_kv, R);
    dim3 grid((unsigned)a.splits, (unsigned)(a.hkv * a.row_groups), (unsigned)a.n);
    if (a.splits == 1) {
        // short caches: one work-group per row group streams every key (no
        // workspace round trip).  Four rows take 4-wave work-groups: at 180
        // VGPRs two of them fit a CU, so batch 64's 512 row groups run in one
        // round instead of two 8-wave rounds (27 -> ~22 us per layer).
        switch (R) {
            case 1: hipLaunchKernelGGL((fa_decode_kernel<T, HD, 1, 16>), grid, dim3(1024), 0, st, a); break;
            case 2: hipLaunchKernelGGL((fa_decode_kernel<T, HD, 2, 16>), grid, dim3(1024), 0, st, a); break;
            // (query first: the early K / V loads cost this instance 24 VGPRs
            // and measured 1.697 against 1.683 ms per batch-64 step)
            case 4: hipLaunchKernelGGL((fa_decode_kernel<T, HD, 4, 4, 4, false>), grid, dim3(256), 0, st, a); break;
            default: hipLaunchKernelGGL((fa_decode_kernel<T, HD, 8, 4>), grid, dim3(256), 0, st, a); break;
        }
        return launch_status();
    }
    // The last split work-group of a row group merges the splits in-kernel
    // (one launch) when there are few; with many, each split work-group
    // would wait for its write-through stores, so a second kernel merges.
    const bool fused = a.splits <= kFusedMergeMaxSplits;
    if (!fused) a.counters = nullptr;
    switch (R) {
        // one or two rows: 8 keys per lane group, so a split of up to 128
        // (head dim 128) or 256 (64) keys is a single load round trip
        case 1: hipLaunchKernelGGL((fa_decode_kernel<T, HD, 1, 4, 8>), grid, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL((fa_decode_kernel<T, HD, 2, 4, 8>), grid, dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL((fa_decode_kernel<T, HD, 4>), grid, dim3(256), 0, st, a); break;
        default: hipLaunchKernelGGL((fa_decode_kernel<T, HD, 8>), grid, dim3(256), 0, st, a); break;
    }
    if (!fused)
        hipLaunchKernelGGL((fa_decode_combine_kernel<T, HD>), dim3((unsigned)(a.n * a.hq * a.l)), dim3(128), 0, st, a);
    return launch_status();
}

}  // namespace kuiops

using namespace kuiops;

extern "C" int kuiops_sdpa_fwd(int64_t n, int64_t hq, int64_t hkv, int64_t l, int64_t s, int64_t e, int64_t ev,
                               int dtype, const void *Q, const int64_t sq[3], const void *K, const int64_t sk[3],
                               const void *V, const int64_t sv[3], void *O, const int64_t so[3], float *lse,
                               float scale, int causal, void *stream) {
    int status;
    if (!attn_common_ok(n, hq, hkv, l, s, e, ev, dtype, Q, sq, K, sk, V, sv, O, so, status)) {
        if (status == KUIOPS_E_INVALID || n * hq * l != 0) return status;
    }
    if (n == 0 || hq == 0 || l == 0) return KUIOPS_OK;
    if (hq > 65535 || n > 65535) return KUIOPS_E_UNSUPPORTED;
    if (!fwd_offsets_fit(s, e, sk[2], sv[2])) return KUIOPS_E_UNSUPPORTED;
    AttnArgs a{};
    fill_args(a, n, hq, hkv, l, s, Q, sq, K, sk, V, sv, O, so, lse, scale, causal);
    hipStream_t st = as_stream(stream);
    if (dtype == KUIOPS_BF16) return e == 128 ? launch_fwd<bf16_t, 128>(a, st) : launch_fwd<bf16_t, 64>(a, st);
    return e == 128 ? launch_fwd<f16_t, 128>(a, st) : launch_fwd<f16_t, 64>(a, st);
}

extern "C" int kuiops_sdpa_fwd_bias(int64_t n, int64_t hq, int64_t hkv, int64_t l, int64_t s, int64_t e,
                                    int64_t ev, int dtype, const void *Q, const int64_t sq[3], const void *K,
                                    const int64_t sk[3], const void *V, const int64_t sv[3], void *O,
                                    const int64_t so[3], float *lse, float scale, int causal, const void *bias,
                                    const int64_t sb[3], void *stream) {
    if (!bias) return kuiops_sdpa_fwd(n, hq, hkv, l, s, e, ev, dtype, Q, sq, K, sk, V, sv, O, so, lse, scale,
                                      causal, stream);
    if (!sb) return KUIOPS_E_INVALID;
    int status;
    if (!attn_common_ok(n, hq, hkv, l, s, e, ev, dtype, Q, sq, K, sk, V, sv, O, so, status)) {
        if (status == KUIOPS_E_INVALID || n * hq * l != 0) return status;
    }
    if (n == 0 || hq == 0 || l == 0) return KUIOPS_OK;
    if (hq > 65535 || n > 65535) return KUIOPS_E_UNSUPPORTED;
    if (!fwd_offsets_fit(s, e, sk[2], sv[2])) return KUIOPS_E_UNSUPPORTED;
    if (!(scale > 0.f)) return KUIOPS_E_UNSUPPORTED;
    // 8-byte loads of 4 consecutive keys: row starts 8-byte aligned
    if ((reinterpret_cast<uintptr_t>(bias) & 7) || sb[0] % 4 || sb[1] % 4 || sb[2] % 4) return KUIOPS_E_UNSUPPORTED;
    if (sb[0] < 0 || sb[1] < 0 || sb[2] < 0) return KUIOPS_E_UNSUPPORTED;
    AttnArgs a{};
    fill_args(a, n, hq, hkv, l, s, Q, sq, K, sk, V, sv, O, so, lse, scale, causal);
    a.bias = bias;
    a.sb0 = sb[0]; a.sb1 = sb[1]; a.sb2 = sb[2];
    a.inv_scale = 1.f / scale;
    hipStream_t st = as_stream(stream);
    if (dtype == KUIOPS_BF16) return e == 128 ? launch_fwd<bf16_t, 128>(a, st) : launch_fwd<bf16_t, 64>(a, st);
    return e == 128 ? launch_fwd<f16_t, 128>(a, st) : launch_fwd<f16_t, 64>(a, st);
}

extern "C" int kuiops_sdpa_decode(int64_t n, int64_t hq, int64_t hkv, int64_t l, int64_t s, int64_t e,
                                  int64_t ev, int dtype, const void *Q, const int64_t sq[3], const void *K,
                                  const int64_t sk[3], const void *V, const int64_t sv[3], void *O,
                                  const int64_t so[3], float *lse, float scale, int causal,
                                  const int32_t *kv_len, void *workspace, size_t workspace_bytes,
                                  void *stream) {
    int status;
    if (!attn_common_ok(n, hq, hkv, l, s, e, ev, dtype, Q, sq, K, sk, V, sv, O, so, status)) {
        if (status == KUIOPS_E_INVALID || n * hq * l != 0) return status;
    }
    if (n == 0 || hq == 0 || l == 0) return KUIOPS_OK;
    if (causal && l > s) return KUIOPS_E_UNSUPPORTED;
    if (n > 65535 || hkv * cdiv((hq / hkv) * l, 8) > 65535) return KUIOPS_E_UNSUPPORTED;
    AttnArgs a{};
    fill_args(a, n, hq, hkv, l, s, Q, sq, K, sk, V, sv, O, so, lse, scale, causal);
    a.kv_len = kv_len;
    const int64_t ss = s > 0 ? s : 1;
    const int R = decode_rows_per_group((int)((hq / hkv) * l));
    a.chunk = decode_chunk_for(ss, n * hkv * cdiv((hq / hkv) * l, R));
    if (decode_row_wide(ss, ev, n * hq * l) || decode_single_split(ss, ev, R)) a.chunk = ss;
    a.splits = (int)cdiv(ss, a.chunk);
    const int64_t rows = n * hq * l;
    const size_t need = decode_workspace_bytes(rows, s, ev);
    if ((int64_t)(need - decode_counter_bytes(rows)) >= INT32_MAX) return KUIOPS_E_UNSUPPORTED;  // 32-bit offsets
    if (!workspace || workspace_bytes < need) return KUIOPS_E_WORKSPACE;
    if (!aligned16(workspace)) return KUIOPS_E_WORKSPACE;
    a.counters = reinterpret_cast<unsigned *>(workspace);
    a.ws_ml = reinterpret_cast<float *>(reinterpret_cast<char *>(workspace) + decode_counter_bytes(rows));
    a.ws_o = a.ws_ml + rows * a.splits * 2;
    if ((reinterpret_cast<uintptr_t>(a.ws_o) & 15) != 0) {
        // keep o rows 16-byte aligned
        a.ws_o = reinterpret_cast<float *>((reinterpret_cast<uintptr_t>(a.ws_o) + 15) & ~uintptr_t(15));
    }
    if (s == 0) {
        // empty cache: the kernels' first K / V loads are issued before the
        // key count is tested; point them at the workspace (zero strides)
        a.K = a.V = workspace;
        a.sk0 = a.sk1 = a.sk2 = a.sv0 = a.sv1 = a.sv2 = 0;
    }
    hipStream_t st = as_stream(stream);
    if (dtype == KUIOPS_BF16) return e == 128 ? launch_decode<bf16_t, 128>(a, st) : launch_decode<bf16_t, 64>(a, st);
    return e == 128 ? launch_decode<f16_t, 128>(a, st) : launch_decode<f16_t, 64>(a, st);
}

// General SDPA entry point (any float dtype, e != ev, head dims up to 1024,
// optional bias of any alignment); see sdpa_general_kernel.
template <typename T>
static int launch_general(const GenArgs &a, hipStream_t st) {
    const int64_t rows = a.n * a.hq * a.l;
    const dim3 grid((unsigned)cdiv(rows, kGenRows)), block(kGenRows * 64);
    const int64_t w = std::max(a.ev, (int64_t)1);
    if (w <= 64) hipLaunchKernelGGL((sdpa_general_kernel<T, 1>), grid, block, 0, st, a);
    else if (w <= 128) hipLaunchKernelGGL((sdpa_general_kernel<T, 2>), grid, block, 0, st, a);
    else if (w <= 256) hipLaunchKernelGGL((sdpa_general_kernel<T, 4>), grid, block, 0, st, a);
    else if (w <= 512) hipLaunchKernelGGL((sdpa_general_kernel<T, 8>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((sdpa_general_kernel<T, 16>), grid, block, 0, st, a);
    return launch_status();
}

extern "C" int kuiops_sdpa_general(int64_t n, int64_t hq, int64_t hkv, int64_t l, int64_t s, int64_t e, int64_t ev,
                                   int dtype, const void *Q, const int64_t sq[3], const void *K, const int64_t sk[3],
                                   const void *V, const int64_t sv[3], void *O, const int64_t so[3], float *lse,
                                   double scale, int causal, const void *bias, const int64_t sb[3], void *stream) {
    if (n < 0 || hq < 0 || hkv <= 0 || l < 0 || s < 0 || e <= 0 || ev <= 0 || !sq || !sk || !sv || !so)
        return KUIOPS_E_INVALID;
    if (hq % hkv || !Q || !K || !V || !O || (bias && !sb)) return KUIOPS_E_INVALID;
    if (dtype != KUIOPS_BF16 && dtype != KUIOPS_F16 && dtype != KUIOPS_F32 && dtype != KUIOPS_F64)
        return KUIOPS_E_UNSUPPORTED;
    if (e > kGenMaxE || ev > kGenMaxE) return KUIOPS_E_UNSUPPORTED;
    if (!(scale > 0.0)) return KUIOPS_E_UNSUPPORTED;
    const int64_t rows = n * hq * l;
    if (rows == 0) return KUIOPS_OK;
    if (cdiv(rows, kGenRows) > INT32_MAX) return KUIOPS_E_UNSUPPORTED;
    GenArgs a{};
    a.n = n; a.hq = hq; a.hkv = hkv; a.l = l; a.s = s; a.e = e; a.ev = ev;
    a.Q = Q; a.K = K; a.V = V; a.O = O; a.lse = lse; a.bias = bias;
    a.sq0 = sq[0]; a.sq1 = sq[1]; a.sq2 = sq[2];
    a.sk0 = sk[0]; a.sk1 = sk[1]; a.sk2 = sk[2];
    a.sv0 = sv[0]; a.sv1 = sv[1]; a.sv2 = sv[2];
    a.so0 = so[0]; a.so1 = so[1]; a.so2 = so[2];
    if (bias) { a.sb0 = sb[0]; a.sb1 = sb[1]; a.sb2 = sb[2]; }
    a.scale = scale;
    a.causal = causal ? 1 : 0;
    hipStream_t st = as_stream(stream);
    switch (dtype) {
        case KUIOPS_BF16: return launch_general<bf16_t>(a, st);
        case KUIOPS_F16: return launch_general<f16_t>(a, st);
        case KUIOPS_F32: return launch_general<float>(a, st);
        default: return launch_general<double>(a, st);
    }
}
