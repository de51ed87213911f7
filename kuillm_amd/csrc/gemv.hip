// Skinny decode GEMM with deterministic split-K:  out[M, N] = x[M, K] @ W[K, N] (+ bias[N]),
// 1 <= M <= 64, bf16 / f16 in, fp32 accumulate.  HBM-bound on W (K*N*2 bytes,
// read exactly once), so each kernel is built around how W streams from HBM.
//
//   * gemv_rows_kernel (row-major W, M <= 2): VALU dot products; a wave reads
//     1 KB row segments (512 columns, 8 per lane), a work-group walks a K
//     range of one 512-column block; K splits merged in-kernel.
//   * gemv_strip_kernel (row-major W, 3 <= M <= 64): a work-group owns a
//     64-column strip, streams its rows through LDS by buffer DMA and feeds
//     16x16x32 MFMAs with x as the A operand (transposing LDS reads give the
//     W operand); the waves' K ranges are summed in LDS in wave order.
//   * gemv_splitk_kernel (K-contiguous W, i.e. an nn.Linear weight seen
//     through .t(), or shapes the others refuse): one 16-byte load per lane is
//     already an MFMA operand; `splits` work-groups share a strip and
//     gemv_reduce_kernel sums their partials in split order.
//
// Wherever K is split over work-groups the partials are summed in split
// order 0..splits-1, so results are bitwise repeatable.
#include <stdlib.h>

#include "common.hpp"

#include <mutex>

namespace kuiops {

struct GemvArgs {
    int64_t M, N, K;
    const void *x; int64_t ldx;
    const void *W; int64_t ldw;
    const void *bias;
    void *out; int64_t ldo;
    int splits;
    int64_t k_per_split;      // multiple of 128
    int64_t k_part;           // strip kernel: k rows per wave (multiple of 32 * stages)
    float *partial;           // [splits][M][N]
    unsigned *counters;       // strip kernel: per-strip arrival counters (zero between calls)
};

constexpr int kGemvStrip = 128;

template <typename T, bool WCOL, typename Tout, int MB>
__global__ __launch_bounds__(256) void gemv_splitk_kernel(GemvArgs a) {
    typedef typename Mfma<T>::frag frag;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int strip = blockIdx.x, split = blockIdx.y;
    const int64_t n0 = (int64_t)strip * kGemvStrip;
    const int64_t kbeg = (int64_t)split * a.k_per_split;
    const int64_t kend = min(a.K, kbeg + a.k_per_split);
    const T *x = reinterpret_cast<const T *>(a.x);
    const T *W = reinterpret_cast<const T *>(a.W);

    const int lc = lane & 15, lg = lane >> 4;
    f32x4 acc[MB][8];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[mb][c] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll 2
    for (int64_t k0 = kbeg + (int64_t)wave * 32; k0 < kend; k0 += 4 * 32) {
        const int64_t kl = k0 + lg * 8;          // first of this lane's 8 k values
        const bool kin = kl < kend;               // K % 8 == 0: all 8 in or out
        u32x4 wb[8];
        if constexpr (!WCOL) {
            const int64_t gn = n0 + lc * 8;
            const bool ok = kin && gn < a.N;
            u32x4 rows[8];
#pragma unroll
            for (int r = 0; r < 8; ++r)
                rows[r] = ok ? *reinterpret_cast<const u32x4 *>(W + (kl + r) * a.ldw + gn)
                             : u32x4{0, 0, 0, 0};
            transpose8x8_b16(rows, wb);
        } else {
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const int64_t gn = n0 + lc * 8 + c;
                wb[c] = (kin && gn < a.N) ? *reinterpret_cast<const u32x4 *>(W + gn * a.ldw + kl)
                                          : u32x4{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int64_t m = mb * 16 + lc;
            const u32x4 xv = (kin && m < a.M) ? *reinterpret_cast<const u32x4 *>(x + m * a.ldx + kl)
                                              : u32x4{0, 0, 0, 0};
            const frag fa = as_frag<frag>(xv);
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[mb][c] = Mfma<T>::m16(fa, as_frag<frag>(wb[c]), acc[mb][c]);
        }
    }

    // acc[mb][c][i]: row 16*mb + 4*lg + i, column n0 + 8*lc + c.
    // Cross-wave sum in wave order through LDS; wave w ends up owning row
    // offset i = w of every 4-row group, 8 adjacent columns per lane.
    __shared__ float red[4][MB][32][64];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave][mb][i * 8 + c][lane] = acc[mb][c][i];
    __syncthreads();

    float part[MB][8];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int e = wave * 8 + c;
            part[mb][c] = ((red[0][mb][e][lane] + red[1][mb][e][lane]) + red[2][mb][e][lane]) +
                          red[3][mb][e][lane];
        }

    const int64_t col0 = n0 + lc * 8;
    const bool col_ok = col0 < a.N;   // N % 8 == 0 is not required: mask per column below
    if (a.splits == 1) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int64_t row = mb * 16 + lg * 4 + wave;
            if (row >= a.M || !col_ok) continue;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const int64_t col = col0 + c;
                if (col >= a.N) break;
                float v = part[mb][c];
                if (a.bias) v += to_f32(reinterpret_cast<const T *>(a.bias)[col]);
                reinterpret_cast<Tout *>(a.out)[row * a.ldo + col] = from_f32<Tout>(v);
            }
        }
        return;
    }

    // Split partials: this work-group's fp32 tile goes to the workspace; the
    // reduce kernel sums the splits in order.
    const int64_t MN = a.M * a.N;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int64_t row = mb * 16 + lg * 4 + wave;
        if (row >= a.M || !col_ok) continue;
        float *dst = a.partial + split * MN + row * a.N + col0;
        if (col0 + 8 <= a.N) {
            *reinterpret_cast<f32x4 *>(dst) = f32x4{part[mb][0], part[mb][1], part[mb][2], part[mb][3]};
            *reinterpret_cast<f32x4 *>(dst + 4) = f32x4{part[mb][4], part[mb][5], part[mb][6], part[mb][7]};
        } else {
#pragma unroll
            for (int c = 0; c < 8; ++c)
                if (col0 + c < a.N) dst[c] = part[mb][c];
        }
    }
}

// out[m, n] = sum_{z = 0..splits-1} partial[z, m, n] (+ bias[n]), summed in
// split order; 4 adjacent columns per thread.
template <typename T, typename Tout>
__global__ __launch_bounds__(256) void gemv_reduce_kernel(GemvArgs a) {
    const int64_t MN = a.M * a.N;
    const int64_t nq = (a.N + 3) / 4;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < a.M * nq; t += (int64_t)gridDim.x * 256) {
        const int64_t row = t / nq, col0 = (t - row * nq) * 4;
        const float *src = a.partial + row * a.N + col0;
        float s[4] = {0.f, 0.f, 0.f, 0.f};
        const int nc = (int)min((int64_t)4, a.N - col0);
        if (nc == 4 && (a.N & 3) == 0) {
            for (int z = 0; z < a.splits; ++z) {
                const f32x4 v = *reinterpret_cast<const f32x4 *>(src + z * MN);
                s[0] += v[0]; s[1] += v[1]; s[2] += v[2]; s[3] += v[3];
            }
        } else {
            for (int z = 0; z < a.splits; ++z)
                for (int c = 0; c < nc; ++c) s[c] += src[z * MN + c];
        }
        for (int c = 0; c < nc; ++c) {
            float v = s[c];
            if (a.bias) v += to_f32(reinterpret_cast<const T *>(a.bias)[col0 + c]);
            reinterpret_cast<Tout *>(a.out)[row * a.ldo + col0 + c] = from_f32<Tout>(v);
        }
    }
}

// ------------------------------------------------------------------------
// Strip variant (row-major W): one NW-wave work-group per (SW-column strip,
// K range).  Enough work-groups to keep ~2 per CU resident matter more for
// HBM throughput than long contiguous runs: 128-byte row segments stream at
// full speed once ~600 work-groups are in flight.  Each wave owns
// k_part rows of the strip and streams them through NS private LDS stages of
// 32 rows with buffer_load ... lds (DMA, no VGPR staging, no barriers: a wave
// only reads what it loaded itself).  The MFMA B operand (8 consecutive k of
// one column) comes from two ds_read_b64_tr_b16 on W's natural row-major
// layout; x is the A operand straight from global memory (it is tiny and
// stays in L2).  The wave partials are summed in wave order through LDS; with
// several K ranges, fp32 partials go to the workspace for gemv_reduce_kernel.
typedef __attribute__((address_space(3))) char lds_char_g;
typedef short s16x4g __attribute__((ext_vector_type(4)));
__device__ __forceinline__ lds_char_g *to_lds_g(const void *p) { return (lds_char_g *)(const_cast<void *>(p)); }

template <int N>
__device__ __forceinline__ void wait_vmcnt_g() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <typename T, typename Tout, int SW, int NS, int MB, int NW>
__global__ __launch_bounds__(NW * 64) void gemv_strip_kernel(GemvArgs a) {
    constexpr int RB = SW * 2;                      // bytes per LDS row (one W row of the strip)
    constexpr int STG = 32 * RB;                    // bytes per stage per wave (32 k rows)
    constexpr int DPS = STG / 1024;                 // 1 KB DMA blocks per stage
    constexpr int RPB = 1024 / RB;                  // rows per DMA block
    constexpr int CPR = RB / 16;                    // 16-byte chunks per row
    constexpr int CG = SW / 16;                     // 16-column MFMA groups
    static_assert(DPS >= 1 && CPR >= 2, "strip width");
    typedef typename Mfma<T>::frag frag;
    // one array per stage (distinct objects: see the GEMM kernels)
    static_assert(NS >= 2 && NS <= 8, "stages");
    __shared__ __attribute__((aligned(1024))) char st0[NW * STG], st1[NW * STG];
    __shared__ __attribute__((aligned(1024))) char st2[NS > 2 ? NW * STG : 16], st3[NS > 3 ? NW * STG : 16];
    __shared__ __attribute__((aligned(1024))) char st4[NS > 4 ? NW * STG : 16], st5[NS > 5 ? NW * STG : 16];
    __shared__ __attribute__((aligned(1024))) char st6[NS > 6 ? NW * STG : 16], st7[NS > 7 ? NW * STG : 16];
    char *const ST[8] = {st0, st1, st2, st3, st4, st5, st6, st7};

    const int tid = threadIdx.x, lane = tid & 63;
    // wave-uniform by construction; readfirstlane lets the compiler keep the
    // buffer descriptor built from it in SGPRs
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Strips handed to one XCD (dispatch is round-robin over the 8 XCDs) form
    // a contiguous range of columns, so the work-groups running together on
    // an XCD read adjacent segments of the same W rows.
    const int nb = gridDim.x, bid = blockIdx.x;
    const int xcd = bid & 7, q8 = nb >> 3, r8 = nb & 7;
    const int strip = xcd * q8 + (xcd < r8 ? xcd : r8) + (bid >> 3);
    const int64_t n0 = (int64_t)strip * SW;
    // Rows past the split's end (or K) lie outside the buffer range below and
    // load as zeros.
    const int split = blockIdx.y;
    // A split covers NW * k_part rows; its waves take the 32-row stages in
    // turn (wave w: rows kbeg + 32 * (NW * kt + w)), so the waves of a
    // work-group read neighbouring rows at any moment (cold W streams ~5%
    // faster than with one contiguous K range per wave).
    const int64_t kbeg = (int64_t)split * NW * a.k_part + 32 * wave;
    const int64_t kend = min(a.K, ((int64_t)split + 1) * NW * a.k_part);
    constexpr int64_t rowstep = 32 * NW;
    const int nst = (int)(a.k_part / 32);
    const T *x = reinterpret_cast<const T *>(a.x);

    // chunk c of row r sits at c ^ swz(r).  One transposing read touches rows
    // 8G + 4h + {0..3} (G = 0..3) x 32 bytes; swz spreads them over the
    // 256-byte bank width (each 16-byte slot twice, the minimum for 512 bytes)
    // and is the same for rows r and r + 4, which the second read (h = 1)
    // relies on.
    auto swz = [](int r) { return CPR == 8 ? 2 * ((r >> 3) & 3) : 2 * (((r >> 3) & 3) | ((r & 1) << 2)); };

    const char *wbase = reinterpret_cast<const char *>(reinterpret_cast<const T *>(a.W) + kbeg * a.ldw + n0);
    // the range ends after row kend - 1 (its columns up to N): row kend and
    // beyond read zeros
    const uint32_t wbytes =
        kbeg < kend ? (uint32_t)min((int64_t)0x7fffffff, ((kend - 1 - kbeg) * a.ldw + (a.N - n0)) * 2) : 0u;
    const __amdgpu_buffer_rsrc_t rsW = __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(wbase), (short)0,
                                                                         (int)wbytes, 0x00020000);
    uint32_t goff[DPS];
#pragma unroll
    for (int j = 0; j < DPS; ++j) {
        const int r = j * RPB + lane / CPR;
        const int c = (lane % CPR) ^ swz(r);
        // columns past N read the next row (or zeros past the end); not stored
        goff[j] = (uint32_t)(((int64_t)r * a.ldw + c * 8) * 2);
    }
    const uint32_t step = (uint32_t)(rowstep * a.ldw * 2);
    const int lc = lane & 15, G = lane >> 4;
    // x fragments (A operand) travel with their stage's DMA: vmcnt counts in
    // issue order, so a later, separate x load would make every wait drain
    // all DMA in flight.
    u32x4 xr[NS][MB];
    auto issue = [&](int kt, char *st, u32x4 *xs) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < DPS; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rsW, (__attribute__((address_space(3))) void *)to_lds_g(st + wave * STG + j * 1024), 16,
                (int)(goff[j] + kt * step), 0, 0, 0);
        const int64_t kl = min(kbeg + (int64_t)kt * rowstep + 8 * G, a.K - 8);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            // unconditional load from a clamped row (no branch around the
            // load); rows past M are zeroed where the fragment is used
            const int64_t m = mb * 16 + lc;
            xs[mb] = *reinterpret_cast<const u32x4 *>(x + min(m, a.M - 1) * a.ldx + kl);
        }
    };

    // transposing-read offsets: lane group G holds k rows 8G..8G+7 of column
    // 16cg + (lane % 16); read h covers rows 8G + 4h .. + 3.
    const int q = lane & 15;
    int offB[CG];
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
        const int r = 8 * G + (q >> 2);
        const int n = 16 * cg + 4 * (q & 3);
        offB[cg] = r * RB + (((n >> 3) ^ swz(r)) << 4) + ((n >> 2) & 1) * 8;
    }

    f32x4 acc[MB][CG];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) acc[mb][cg] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int kt, const char *stg, const u32x4 *xs) __attribute__((always_inline)) {
        // x columns of rows outside [kbeg, kend) meet zero W rows but are
        // zeroed too, so an Inf or NaN there cannot leak into the sum
        const bool kin = kbeg + (int64_t)kt * rowstep + 8 * G < kend;
        const char *sw = stg + wave * STG;
        frag fb[CG];
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) {
            const s16x4g t0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4g *)to_lds_g(sw + offB[cg]));
            const s16x4g t1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) s16x4g *)to_lds_g(sw + offB[cg] + 4 * RB));
            const u32x2 h0 = __builtin_bit_cast(u32x2, t0), h1 = __builtin_bit_cast(u32x2, t1);
            fb[cg] = as_frag<frag>(u32x4{h0[0], h0[1], h1[0], h1[1]});
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const frag fa = as_frag<frag>(kin && mb * 16 + lc < a.M ? xs[mb] : u32x4{0, 0, 0, 0});
#pragma unroll
            for (int cg = 0; cg < CG; ++cg) acc[mb][cg] = Mfma<T>::m16(fa, fb[cg], acc[mb][cg]);
        }
    };
    constexpr int PER = DPS + MB;                   // vector-memory instructions per stage
    // nst is a multiple of NS (k_part is a multiple of 32 * NS).  Straight-line code
    // (no branch between issue and use) lets the compiler track which LDS
    // array each DMA targets and keep NS - 1 stages in flight.
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) issue(s, ST[s], xr[s]);
    for (int kt0 = 0; kt0 + NS < nst; kt0 += NS) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            issue(kt0 + s + NS - 1, ST[(s + NS - 1) % NS], xr[(s + NS - 1) % NS]);
            wait_vmcnt_g<(NS - 1) * PER>();
            compute(kt0 + s, ST[s], xr[s]);
        }
    }
    // last NS stages: one more issue, then drain
    issue(nst - 1, ST[NS - 1], xr[NS - 1]);
    wait_vmcnt_g<(NS - 1) * PER>();
    compute(nst - NS, ST[0], xr[0]);
#pragma unroll
    for (int s = 1; s < NS; ++s) {
        // stages issued after this one: NS - 1 - s
        switch (NS - 1 - s) {
            case 6: wait_vmcnt_g<(NS > 7 ? 6 * PER : 0)>(); break;
            case 5: wait_vmcnt_g<(NS > 6 ? 5 * PER : 0)>(); break;
            case 4: wait_vmcnt_g<(NS > 5 ? 4 * PER : 0)>(); break;
            case 3: wait_vmcnt_g<(NS > 4 ? 3 * PER : 0)>(); break;
            case 2: wait_vmcnt_g<(NS > 3 ? 2 * PER : 0)>(); break;
            case 1: wait_vmcnt_g<(NS > 2 ? 1 * PER : 0)>(); break;
            default: wait_vmcnt_g<0>(); break;
        }
        compute(nst - NS + s, ST[s], xr[s]);
    }

    // acc[mb][cg][i]: row 16mb + 4G + i, column n0 + 16cg + lc.  Sum the
    // waves in wave order through LDS, one 16-row block at a time (the DMA
    // stages are free: every wave waited for its last stage before its last
    // reads, and the barrier orders them).
    float *red = reinterpret_cast<float *>(st0);    // [wave][CG * 4][64] floats <= NW * STG bytes
    constexpr int E = CG * 4;
    static_assert(NW * E * 64 * 4 <= NW * STG, "reduction buffer");
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        __syncthreads();
#pragma unroll
        for (int cg = 0; cg < CG; ++cg)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[(wave * E + cg * 4 + i) * 64 + lane] = acc[mb][cg][i];
        __syncthreads();
        for (int idx = tid; idx < E * 64; idx += NW * 64) {
            const int e = idx / 64, l = idx % 64;
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) v += red[(w * E + e) * 64 + l];
            const int cg = e / 4, i = e % 4;
            const int64_t row = mb * 16 + 4 * (l >> 4) + i;
            const int64_t col = n0 + 16 * cg + (l & 15);
            if (row < a.M && col < a.N) {
                if (a.splits > 1) {
                    // agent-coherent store (written through the XCD's L2):
                    // the work-group that sums the partials may run on another XCD
                    __hip_atomic_store(&a.partial[((int64_t)split * a.M + row) * a.N + col], v, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                } else {
                    if (a.bias) v += to_f32(reinterpret_cast<const T *>(a.bias)[col]);
                    reinterpret_cast<Tout *>(a.out)[row * a.ldo + col] = from_f32<Tout>(v);
                }
            }
        }
    }
    if (a.splits > 1) {
        // The last work-group of the strip to arrive sums the partials in
        // split order (bitwise repeatable whatever the arrival order).
        // Ordering: the partials are agent-scope relaxed atomic stores, which
        // the gfx942 / gfx950 memory model lowers to `global_store sc1`
        // (written through the per-XCD L2 to the agent's coherence point);
        // s_waitcnt(0) waits for their acknowledgements, the barrier orders
        // every wave's acknowledged stores before tid 0's relaxed agent-scope
        // counter RMW (performed at the coherence point), and the summing
        // work-group reads with agent-scope relaxed atomic loads (`sc1`, which
        // miss the non-coherent caches).  Relaxed atomics alone do not order
        // two locations in the formal model; this relies on the hardware rule
        // that an acknowledged sc1 store is visible at the coherence point
        // before a later RMW of the same agent.  A release / acquire pair would
        // add an L2 write-back per XCD to every work-group.
        __shared__ int s_last;
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0)
            s_last = __hip_atomic_fetch_add(&a.counters[strip], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     (unsigned)(a.splits - 1);
        __syncthreads();
        if (s_last) {
            for (int idx = tid; idx < MB * 16 * SW; idx += NW * 64) {
                const int64_t row = idx / SW, col = n0 + idx % SW;
                if (row >= a.M || col >= a.N) continue;
                float v = 0.f;
                for (int z = 0; z < a.splits; ++z)
                    v += __hip_atomic_load(&a.partial[((int64_t)z * a.M + row) * a.N + col], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                if (a.bias) v += to_f32(reinterpret_cast<const T *>(a.bias)[col]);
                reinterpret_cast<Tout *>(a.out)[row * a.ldo + col] = from_f32<Tout>(v);
            }
            if (tid == 0) __hip_atomic_store(&a.counters[strip], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Row-streaming decode GEMM for row-major W and at most 2 rows of x
// (VALU v_dot2, no MFMA; beyond 2 rows the VALU work bounds it): lane l of a wave owns 8 adjacent output columns, so one
// 16-byte load per lane covers 512 columns (1 KB) of a W row, and a
// work-group of 8 waves walks a K range of its 512-column block in groups of
// 8 rows (wave w takes groups w, w + 8, ...; two groups, 16 loads per lane,
// in flight).  Cold W (not in the MALL) streams from HBM far better in
// these 1 KB row segments than in the 128-byte segments of the strip kernel.
// The waves' sums meet in LDS in wave order; the K splits of one column
// block are summed in split order by the last work-group of that block to
// arrive (agent-coherent partials and counter, as in the strip kernel), so
// the result is bitwise repeatable.
//

template <typename T, typename Tout, int MR, int P>
__global__ __launch_bounds__(512) void gemv_rows_kernel(GemvArgs a) {
    constexpr int NW = 8, CB = 512;                 // waves, columns per block; P groups in flight
    __shared__ float red[NW * CB];
    __shared__ int s_last;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int cb = blockIdx.x, split = blockIdx.y;
    const int64_t n0 = (int64_t)cb * CB;
    // columns past N read a valid neighbouring 16 bytes (not stored)
    const int64_t colc = min(n0 + 8 * lane, a.N - 8);
    const int64_t kbeg = (int64_t)split * a.k_part;
    const int64_t kend = min(a.K, kbeg + a.k_part);
    const int ngroups = kend > kbeg ? (int)((kend - kbeg) / 8) : 0;   // k_part, K multiples of 8
    const T *W = reinterpret_cast<const T *>(a.W);
    const T *x = reinterpret_cast<const T *>(a.x);

    float acc[MR][8];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[m][c] = 0.f;

    u32x4 wr[P][8];
    auto load = [&](int g, u32x4 *w) __attribute__((always_inline)) {
        const T *p = W + (kbeg + 8 * (int64_t)g) * a.ldw + colc;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            w[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p + j * a.ldw));
    };
    // rows 2p and 2p + 1 of a group pair up for v_dot2 (two products and the
    // accumulator per instruction): one v_perm_b32 gathers a column's two W
    // values, and x's consecutive k pair is already one 32-bit word.
    auto dot8 = [&](int g, const u32x4 *w) __attribute__((always_inline)) {
        const int64_t k = kbeg + 8 * (int64_t)g;
        u32x4 xv[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m)   // rows past M repeat row M - 1 (not stored)
            xv[m] = *reinterpret_cast<const u32x4 *>(x + (int64_t)min(m, (int)a.M - 1) * a.ldx + k);
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const uint32_t wp = __builtin_amdgcn_perm(w[2 * pp + 1][i], w[2 * pp][i], e ? 0x07060302u : 0x05040100u);
#pragma unroll
                    for (int m = 0; m < MR; ++m) acc[m][2 * i + e] = dot2<T>(xv[m][pp], wp, acc[m][2 * i + e]);
                }
            }
        }
    };
    // wave w: groups w, w + NW, ...; P groups in flight
    int g = wave;
#pragma unroll
    for (int p = 0; p < P; ++p)
        if (g + p * NW < ngroups) load(g + p * NW, wr[p]);
    for (; g < ngroups; g += P * NW) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int gg = g + p * NW;
            if (gg < ngroups) {
                dot8(gg, wr[p]);
                if (gg + P * NW < ngroups) load(gg + P * NW, wr[p]);
            }
        }
    }

    // waves summed in wave order; thread t then owns column n0 + t
    const int64_t col = n0 + tid;
    float res[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        if (m) __syncthreads();
#pragma unroll
        for (int c = 0; c < 8; ++c) red[wave * CB + 8 * lane + c] = acc[m][c];
        __syncthreads();
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += red[w * CB + tid];
        res[m] = v;
    }
    if (a.splits == 1) {
        if (col < a.N) {
            const float b = a.bias ? to_f32(reinterpret_cast<const T *>(a.bias)[col]) : 0.f;
#pragma unroll
            for (int m = 0; m < MR; ++m)
                if (m < a.M) reinterpret_cast<Tout *>(a.out)[m * a.ldo + col] = from_f32<Tout>(res[m] + b);
        }
        return;
    }
    if (col < a.N) {
#pragma unroll
        for (int m = 0; m < MR; ++m)
            if (m < a.M)
                __hip_atomic_store(&a.partial[((int64_t)split * a.M + m) * a.N + col], res[m], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(&a.counters[cb], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (unsigned)(a.splits - 1);
    __syncthreads();
    if (!s_last) return;
    if (col < a.N) {
        const float b = a.bias ? to_f32(reinterpret_cast<const T *>(a.bias)[col]) : 0.f;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if (m >= a.M) break;
            float v = 0.f;
            int z = 0;
            for (; z + 8 <= a.splits; z += 8) {
                float t[8];
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    t[i] = __hip_atomic_load(&a.partial[((int64_t)(z + i) * a.M + m) * a.N + col], __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                for (int i = 0; i < 8; ++i) v += t[i];
            }
            for (; z < a.splits; ++z)
                v += __hip_atomic_load(&a.partial[((int64_t)z * a.M + m) * a.N + col], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            reinterpret_cast<Tout *>(a.out)[m * a.ldo + col] = from_f32<Tout>(v + b);
        }
    }
    if (tid == 0) __hip_atomic_store(&a.counters[cb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int kRowsCB = 512;        // columns per work-group of the row-streaming kernel
constexpr int kRowsMaxM = 2;

// K splits of the row-streaming kernel: at most ~192 work-groups (one per
// CU).  Every split adds the merge tail (write-through partials, counter,
// re-read) to its column block, so fewer, longer K ranges win: 4096 x 11008,
// M = 1, cold W: 8 splits 17.5 us, 11 18.0, 16 19.9, 32 19.8, 64 24.0.
static int rows_splits(int64_t N, int64_t K) {
    const int64_t cbs = cdiv(N, kRowsCB);
    int64_t s = 192 / cbs;
    const int64_t maxs = cdiv(K, 64);                // at least one group per wave
    if (s > maxs) s = maxs;
    if (s > 64) s = 64;
    return s < 1 ? 1 : (int)s;
}

static int gemv_choose_splits(int64_t M, int64_t N, int64_t K) {
    (void)M;
    const int64_t strips = cdiv(N, kGemvStrip);
    const int64_t ksteps = cdiv(K, 128);            // 128 = 4 waves x 32
    int64_t s = cdiv(768, strips);                   // aim for ~3 work-groups per CU
    if (s > ksteps) s = ksteps;
    if (s > 64) s = 64;
    return s < 1 ? 1 : (int)s;
}

static int strip_splits(int64_t N, int64_t K);

// Workspace layout: the strip kernel's arrival counters (one per strip,
// zero between calls) occupy a fixed head region that no call uses for
// anything else; fp32 partials follow it.
constexpr size_t kGemvCounterBytes = 16384;       // 4096 strips: N <= 262144

size_t gemv_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    const int s = gemv_choose_splits(M, N, K);
    const int s2 = strip_splits(N, K);
    const int s3 = M <= kRowsMaxM ? rows_splits(N, K) : 1;
    const int mx = max(max(s, s2), s3);
    return kGemvCounterBytes + (mx > 1 ? (size_t)mx * M * N * sizeof(float) : 0);
}

template <typename T, typename Tout, int MB>
static void gemv_launch(const GemvArgs &a, bool wcol, hipStream_t st) {
    dim3 grid((unsigned)cdiv(a.N, kGemvStrip), (unsigned)a.splits);
    if (wcol) hipLaunchKernelGGL((gemv_splitk_kernel<T, true, Tout, MB>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((gemv_splitk_kernel<T, false, Tout, MB>), grid, dim3(256), 0, st, a);
}

template <typename T, typename Tout>
static int gemv_dispatch(const GemvArgs &a, bool wcol, hipStream_t st) {
    switch (cdiv(a.M, 16)) {
        case 1: gemv_launch<T, Tout, 1>(a, wcol, st); break;
        case 2: gemv_launch<T, Tout, 2>(a, wcol, st); break;
        case 3: gemv_launch<T, Tout, 3>(a, wcol, st); break;
        case 4: gemv_launch<T, Tout, 4>(a, wcol, st); break;
        default: return KUIOPS_E_UNSUPPORTED;
    }
    if (a.splits > 1) {
        int64_t blocks = cdiv(a.M * cdiv(a.N, 4), 256);
        if (blocks > 2048) blocks = 2048;
        hipLaunchKernelGGL((gemv_reduce_kernel<T, Tout>), dim3((unsigned)blocks), dim3(256), 0, st, a);
    }
    return launch_status();
}

constexpr int kStripW = 64;      // 128-byte row segments: narrower ones halve HBM efficiency
// Work-group shape (128 KB of LDS, one work-group per CU): up to 16 rows of
// x and 33..64 rows take 8 waves x 4 stages of 4 KB, so three stages per wave
// stay in flight while it computes on the fourth (4096 x 11008, M = 1 / 4 /
// 16: 15.3 / 15.5 / 16.1 us, against 15.7 / 15.9 / 16.4 us for 16 waves x 2
// stages and 15.6 / 15.7 / 16.2 us for 4 waves x 8 stages; 2 or 3 K splits
// per strip were slower, 17.8-21 us); 17..32 rows
// keep 16 waves x 2 stages (128 VGPRs per lane).
constexpr int kStripWaves = 16, kStripStages = 2;
constexpr int kStripWavesWide = 8, kStripStagesWide = 4;

// K splits for the strip kernel.  A split costs a second (reduce) launch, so
// one work-group per strip is kept while that still occupies >= 128 CUs
// (N = 11008 gives 172 strips); narrower problems, once split anyway, are
// split until every CU has a work-group.
static int strip_splits(int64_t N, int64_t K) {
    const int64_t strips = cdiv(N, kStripW);
    if (strips >= 128) return 1;
    int s = 1;
    while (strips * s < 256 && s < 16 && K >= (int64_t)2 * s * 1024) s *= 2;
    return s;
}

// rows per wave: K / (splits * NW) rounded up to whole pipelines (32 * NS)
static int64_t strip_part(int64_t K, int splits, int nw, int ns) {
    const int64_t g = 32 * ns;
    return cdiv(cdiv(K, (int64_t)splits * nw), g) * g;
}

static bool strip_eligible(const GemvArgs &a, bool wcol) {
    if (wcol || a.N % 8 || a.ldw % 8 || a.K % 8 || cdiv(a.N, kStripW) * 4 > (int64_t)kGemvCounterBytes) return false;
    if (cdiv(a.N, kStripW) * strip_splits(a.N, a.K) < 128) return false;
    return ((a.K - 1) * a.ldw + a.N) * 2 < ((int64_t)1 << 31);
}

template <typename T, typename Tout, int MB, int NW, int NS>
static void strip_launch(GemvArgs a, hipStream_t st) {
    a.k_part = strip_part(a.K, a.splits, NW, NS);
    dim3 grid((unsigned)cdiv(a.N, kStripW), (unsigned)a.splits);
    hipLaunchKernelGGL((gemv_strip_kernel<T, Tout, kStripW, NS, MB, NW>), grid, dim3(NW * 64), 0, st, a);
}

template <typename T, typename Tout>
static int strip_dispatch(const GemvArgs &a, hipStream_t st) {
    switch (cdiv(a.M, 16)) {
        case 1: strip_launch<T, Tout, 1, kStripWavesWide, kStripStagesWide>(a, st); break;
        case 2: strip_launch<T, Tout, 2, kStripWaves, kStripStages>(a, st); break;
        case 3: strip_launch<T, Tout, 3, kStripWavesWide, kStripStagesWide>(a, st); break;
        case 4: strip_launch<T, Tout, 4, kStripWavesWide, kStripStagesWide>(a, st); break;
        default: return KUIOPS_E_UNSUPPORTED;
    }
    return launch_status();
}

static bool rows_eligible(const GemvArgs &a, bool wcol) {
    if (wcol || a.M > kRowsMaxM || a.N % 8 || a.ldw % 8 || a.K % 8 || a.N < kRowsCB) return false;
    if (cdiv(a.N, kRowsCB) * 4 > (int64_t)kGemvCounterBytes) return false;
    return true;
}

template <typename T, typename Tout>
static int rows_dispatch(const GemvArgs &a, hipStream_t st) {
    dim3 grid((unsigned)cdiv(a.N, kRowsCB), (unsigned)a.splits);
    switch (a.M) {
        case 1: hipLaunchKernelGGL((gemv_rows_kernel<T, Tout, 1, 2>), grid, dim3(512), 0, st, a); break;
        case 2: hipLaunchKernelGGL((gemv_rows_kernel<T, Tout, 2, 2>), grid, dim3(512), 0, st, a); break;
        default: return KUIOPS_E_UNSUPPORTED;
    }
    return launch_status();
}

}  // namespace kuiops

using namespace kuiops;

static void clear_counters_on(unsigned *counters, int64_t n, hipStream_t st);

static int gemv_run(int64_t M, int64_t N, int64_t K, int in_dtype, const void *x, int64_t ldx, const void *W,
                    int64_t ldw, int w_layout, const void *bias, int out_dtype, void *out, int64_t ldo, int splits,
                    void *workspace, size_t workspace_bytes, bool clear_counters, void *stream);

extern "C" int kuiops_gemv_splitk(int64_t M, int64_t N, int64_t K, int in_dtype, const void *x, int64_t ldx,
                                  const void *W, int64_t ldw, int w_layout, const void *bias, int out_dtype,
                                  void *out, int64_t ldo, int splits, void *workspace, size_t workspace_bytes,
                                  void *stream) {
    return gemv_run(M, N, K, in_dtype, x, ldx, W, ldw, w_layout, bias, out_dtype, out, ldo, splits, workspace,
                    workspace_bytes, false, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free variant: the same kernels with their workspace in a
// file-scope device array instead of caller / torch memory.  Each GPU holds
// its own copy of `scratch` (at its own address, found once per device with
// hipGetSymbolAddress) for the life of the process.  Calls that overlap on
// one GPU share it and race.
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static void *g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

__global__ void clear_u32_kernel(unsigned *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

static int scratch_for_current_device(void **ptr) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return KUIOPS_E_HIP;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return KUIOPS_E_HIP;
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return KUIOPS_OK;
}

// The arrival counters must be zero when a split kernel starts.  The kernels
// leave them at zero, but the shared array keeps whatever the previous call
// on this GPU left, so every allocation-free call clears the counters it
// uses first (a fill kernel, not a memset, so the call can be captured).
static void clear_counters_on(unsigned *counters, int64_t n, hipStream_t st) {
    hipLaunchKernelGGL(clear_u32_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st, counters, (int)n);
}

extern "C" size_t kuiops_gemv_splitk_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int kuiops_gemv_splitk_noalloc(int64_t M, int64_t N, int64_t K, int in_dtype, const void *x,
                                          int64_t ldx, const void *W, int64_t ldw, int w_layout, const void *bias,
                                          int out_dtype, void *out, int64_t ldo, int splits, void *stream) {
    if (M < 0 || N < 0 || K < 0) return KUIOPS_E_INVALID;
    if (M == 0 || N == 0) return KUIOPS_OK;
    if (M <= 64 && gemv_workspace_bytes(M, N, K) > kNoAllocScratchBytes) return KUIOPS_E_WORKSPACE;
    void *ws = nullptr;
    const int st = scratch_for_current_device(&ws);
    if (st != KUIOPS_OK) return st;
    return gemv_run(M, N, K, in_dtype, x, ldx, W, ldw, w_layout, bias, out_dtype, out, ldo, splits, ws,
                    kNoAllocScratchBytes, true, stream);
}

static int gemv_run(int64_t M, int64_t N, int64_t K, int in_dtype, const void *x, int64_t ldx, const void *W,
                    int64_t ldw, int w_layout, const void *bias, int out_dtype, void *out, int64_t ldo, int splits,
                    void *workspace, size_t workspace_bytes, bool clear_counters, void *stream) {
    if (M < 0 || N < 0 || K < 0) return KUIOPS_E_INVALID;
    if (w_layout != KUIOPS_B_ROW && w_layout != KUIOPS_B_COL) return KUIOPS_E_INVALID;
    if (M == 0 || N == 0) return KUIOPS_OK;
    if (!x || !W || !out) return KUIOPS_E_INVALID;
    if (M > 64) return KUIOPS_E_UNSUPPORTED;
    if (in_dtype != KUIOPS_BF16 && in_dtype != KUIOPS_F16) return KUIOPS_E_UNSUPPORTED;
    if (out_dtype != in_dtype && out_dtype != KUIOPS_F32) return KUIOPS_E_UNSUPPORTED;
    const bool wcol = w_layout == KUIOPS_B_COL;
    if (K % 8 || ldx % 8 || ldw % 8 || !aligned16(x) || !aligned16(W)) return KUIOPS_E_UNSUPPORTED;
    if (!wcol && N % 8) return KUIOPS_E_UNSUPPORTED;
    if (K == 0) return KUIOPS_E_UNSUPPORTED;

    GemvArgs a{};
    a.M = M; a.N = N; a.K = K;
    a.x = x; a.ldx = ldx; a.W = W; a.ldw = ldw; a.bias = bias;
    a.out = out; a.ldo = ldo;
    hipStream_t st0 = as_stream(stream);
    if (splits <= 0 && rows_eligible(a, wcol)) {
        a.splits = rows_splits(N, K);
        a.k_part = cdiv(cdiv(K, a.splits), 8) * 8;
        a.splits = (int)cdiv(K, a.k_part);
        if (a.splits > 1) {
            const size_t need = kGemvCounterBytes + (size_t)a.splits * M * N * sizeof(float);
            if (!workspace || workspace_bytes < need || !aligned16(workspace)) return KUIOPS_E_WORKSPACE;
            a.counters = reinterpret_cast<unsigned *>(workspace);
            a.partial = reinterpret_cast<float *>(reinterpret_cast<char *>(workspace) + kGemvCounterBytes);
            if (clear_counters) clear_counters_on(a.counters, cdiv(N, kRowsCB), st0);
        }
        if (in_dtype == KUIOPS_BF16)
            return out_dtype == KUIOPS_F32 ? rows_dispatch<bf16_t, float>(a, st0) : rows_dispatch<bf16_t, bf16_t>(a, st0);
        return out_dtype == KUIOPS_F32 ? rows_dispatch<f16_t, float>(a, st0) : rows_dispatch<f16_t, f16_t>(a, st0);
    }
    if (splits <= 0 && strip_eligible(a, wcol)) {
        a.splits = strip_splits(N, K);
        if (a.splits > 1) {
            const size_t need = kGemvCounterBytes + (size_t)a.splits * M * N * sizeof(float);
            if (!workspace || workspace_bytes < need || !aligned16(workspace)) return KUIOPS_E_WORKSPACE;
            a.counters = reinterpret_cast<unsigned *>(workspace);
            a.partial = reinterpret_cast<float *>(reinterpret_cast<char *>(workspace) + kGemvCounterBytes);
            if (clear_counters) clear_counters_on(a.counters, cdiv(N, kStripW), st0);
        }
        if (in_dtype == KUIOPS_BF16)
            return out_dtype == KUIOPS_F32 ? strip_dispatch<bf16_t, float>(a, st0) : strip_dispatch<bf16_t, bf16_t>(a, st0);
        return out_dtype == KUIOPS_F32 ? strip_dispatch<f16_t, float>(a, st0) : strip_dispatch<f16_t, f16_t>(a, st0);
    }
    int s = splits > 0 ? splits : gemv_choose_splits(M, N, K);
    int64_t kps = cdiv(cdiv(K, s), 128) * 128;
    s = (int)cdiv(K, kps);
    a.splits = s;
    a.k_per_split = kps;
    if (s > 1) {
        const size_t need = kGemvCounterBytes + (size_t)s * M * N * sizeof(float);
        if (!workspace || workspace_bytes < need || !aligned16(workspace)) return KUIOPS_E_WORKSPACE;
        a.partial = reinterpret_cast<float *>(reinterpret_cast<char *>(workspace) + kGemvCounterBytes);
    }
    hipStream_t st = st0;
    if (in_dtype == KUIOPS_BF16)
        return out_dtype == KUIOPS_F32 ? gemv_dispatch<bf16_t, float>(a, wcol, st)
                                       : gemv_dispatch<bf16_t, bf16_t>(a, wcol, st);
    return out_dtype == KUIOPS_F32 ? gemv_dispatch<f16_t, float>(a, wcol, st)
                                   : gemv_dispatch<f16_t, f16_t>(a, wcol, st);
}

