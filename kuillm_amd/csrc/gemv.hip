// Skinny decode GEMM with deterministic split-K:  out[M, N] = x[M, K] @ W[K, N] (+ bias[N]),
// 1 <= M <= 64, bf16 / f16 in, fp32 accumulate.
//
// The kernel is HBM-bound on W (K*N*2 bytes, read exactly once), so the design
// goal is many bytes in flight and no re-reads:
//   * A wave owns a 128-column strip and consumes W in 32(k) x 128(n) steps
//     with 16x16x32 MFMAs; x (at most 64 rows) is the MFMA A operand, padded to
//     16-row blocks with zeros.
//   * Row-major W ([K, N], N contiguous): lane l loads an 8(k) x 8(n) block
//     (8 x 16 bytes, rows k0 + 8*(l/16) .. +7, columns 8*(l%16) .. +7) and
//     transposes it in registers; MFMA number c then covers columns
//     {8*i + c}, so each lane ends with 8 adjacent output columns.
//     K-contiguous W ([N, K] storage): the same operand is one 16-byte load.
//   * A work-group is 4 waves on one strip, interleaving their K steps; the
//     four partial tiles are summed through LDS in wave order.
//   * `splits` work-groups share a strip.  Each writes its fp32 partial tile to
//     the workspace and a second kernel sums the partials in split order
//     0..splits-1, adds the bias and converts, so the result is bitwise
//     repeatable.  (Reducing in the last-arriving work-group instead would
//     need device-scope fences, which on a chip with one L2 per XCD write
//     back that L2.)
#include "common.hpp"

namespace kuiops {

struct GemvArgs {
    int64_t M, N, K;
    const void *x; int64_t ldx;
    const void *W; int64_t ldw;
    const void *bias;
    void *out; int64_t ldo;
    int splits;
    int64_t k_per_split;      // multiple of 128
    float *partial;           // [splits][M][N]
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

static int gemv_choose_splits(int64_t M, int64_t N, int64_t K) {
    (void)M;
    const int64_t strips = cdiv(N, kGemvStrip);
    const int64_t ksteps = cdiv(K, 128);            // 128 = 4 waves x 32
    int64_t s = cdiv(768, strips);                   // aim for ~3 work-groups per CU
    if (s > ksteps) s = ksteps;
    if (s > 64) s = 64;
    return s < 1 ? 1 : (int)s;
}

size_t gemv_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    const int s = gemv_choose_splits(M, N, K);
    return s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
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

}  // namespace kuiops

using namespace kuiops;

extern "C" int kuiops_gemv_splitk(int64_t M, int64_t N, int64_t K, int in_dtype, const void *x, int64_t ldx,
                                  const void *W, int64_t ldw, int w_layout, const void *bias, int out_dtype,
                                  void *out, int64_t ldo, int splits, void *workspace, size_t workspace_bytes,
                                  void *stream) {
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
    int s = splits > 0 ? splits : gemv_choose_splits(M, N, K);
    int64_t kps = cdiv(cdiv(K, s), 128) * 128;
    s = (int)cdiv(K, kps);
    a.splits = s;
    a.k_per_split = kps;
    if (s > 1) {
        const size_t need = (size_t)s * M * N * sizeof(float);
        if (!workspace || workspace_bytes < need || !aligned16(workspace)) return KUIOPS_E_WORKSPACE;
        a.partial = reinterpret_cast<float *>(workspace);
    }
    hipStream_t st = as_stream(stream);
    if (in_dtype == KUIOPS_BF16)
        return out_dtype == KUIOPS_F32 ? gemv_dispatch<bf16_t, float>(a, wcol, st)
                                       : gemv_dispatch<bf16_t, bf16_t>(a, wcol, st);
    return out_dtype == KUIOPS_F32 ? gemv_dispatch<f16_t, float>(a, wcol, st)
                                   : gemv_dispatch<f16_t, f16_t>(a, wcol, st);
}
