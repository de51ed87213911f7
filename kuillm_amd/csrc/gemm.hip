// GEMM family for gfx950: mm / addmm / bmm.
//
// Fast path (bf16 / f16 in, fp32 accumulate): LDS-tiled MFMA kernel.
//   * Work-group tile BM x BN x 64, WM x WN waves, each wave a
//     (BM/WM) x (BN/WN) sub-tile built from 32x32x16 MFMAs.
//   * A and B tiles are staged K-contiguous in LDS ([row][64] with the 16-byte
//     chunk index XOR-swizzled by the row), so one ds_read_b128 feeds one MFMA
//     operand.  A row-major B ([K, N], N contiguous) is transposed on its way
//     into LDS: each thread loads a 4(k) x 8(n) block and permutes it in
//     registers; a K-contiguous B (nn.Linear weight seen through .t()) is
//     copied like A.
//   * Two LDS stages; the global loads of tile k+1 are issued before the
//     MFMAs of tile k, one barrier per K step.
//   * Work-group ids are remapped so that neighbouring output tiles run on the
//     same XCD (dispatch is round-robin over the 8 XCDs) and are visited in
//     groups of 8 tile-rows for L2 reuse.
//   * Split-K writes fp32 partial tiles to the workspace; a second kernel
//     sums them in split order (deterministic) and applies the epilogue.
// Anything else (f32 / f64, unaligned or odd shapes) takes a plain LDS-tiled
// SIMT kernel with the same epilogue.
//
// Semantics follow aten mm / addmm / bmm (the reference's fallthrough and
// test oracle, kuipy/kuiops.py:403-564, tests/test_jit_ops.py:51-112).
#include "common.hpp"

namespace kuiops {

struct GemmArgs {
    int64_t M, N, K;
    const void *A; int64_t lda, stride_a;
    const void *B; int64_t ldb, stride_b;
    void *out; int64_t ldo, stride_o;
    const void *cin; int64_t ldcin; int c_kind;
    float alpha, beta;
    int64_t k_per_split;   // multiple of 64
    int splits;
    int tiles_m, tiles_n;
    float *partial;        // split-K workspace [splits][M][N]
};

__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }

// Maps a linear work-group id so that ids dispatched to one XCD become a
// contiguous range, then orders tiles in groups of 8 tile-rows.
__device__ __forceinline__ void tile_coords(int bid, int nblocks, int tiles_m, int tiles_n,
                                            int &tm, int &tn) {
    const int xcd = bid & 7, idx = bid >> 3;
    const int q = nblocks >> 3, r = nblocks & 7;
    const int pid = xcd * q + (xcd < r ? xcd : r) + idx;
    const int G = 8;
    const int width = G * tiles_n;
    const int group = pid / width;
    const int first_m = group * G;
    const int gsz = min(tiles_m - first_m, G);
    const int in_group = pid - group * width;
    tm = first_m + in_group % gsz;
    tn = in_group / gsz;
}

template <typename Tout>
__device__ __forceinline__ void epilogue_store(const GemmArgs &a, Tout *out, const Tout *cin,
                                               int64_t row, int64_t col, float acc) {
    float v = a.alpha * acc;
    if (a.c_kind == KUIOPS_C_FULL) v += a.beta * to_f32(cin[row * a.ldcin + col]);
    else if (a.c_kind == KUIOPS_C_ROW) v += a.beta * to_f32(cin[col]);
    out[row * a.ldo + col] = from_f32<Tout>(v);
}

template <typename T, int BM, int BN, int WM, int WN, bool BCOL, typename Tout, bool SPLIT>
__global__ __launch_bounds__(WM * WN * 64) void gemm_mfma_kernel(GemmArgs a) {
    constexpr int NT = WM * WN * 64;
    constexpr int BK = 64;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int CA = BM * 8 / NT;            // 16-byte chunks of A per thread
    constexpr int CBC = BN * 8 / NT;           // B chunks per thread (K-contiguous B)
    constexpr int CBR = 2 * BN / NT;           // 4x8 B blocks per thread (row-major B)
    static_assert(CA >= 1 && BM * 8 % NT == 0, "A tile / thread mismatch");
    static_assert(BCOL ? (CBC >= 1 && BN * 8 % NT == 0) : (CBR >= 1 && 2 * BN % NT == 0),
                  "B tile / thread mismatch");
    typedef typename Mfma<T>::frag frag;

    __shared__ __attribute__((aligned(16))) T sA[2][BM * BK];
    __shared__ __attribute__((aligned(16))) T sB[2][BN * BK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, a.tiles_m, a.tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int zb = blockIdx.y;
    const int split = SPLIT ? zb : 0;
    const int64_t batch = SPLIT ? 0 : zb;

    const T *A = reinterpret_cast<const T *>(a.A) + batch * a.stride_a;
    const T *B = reinterpret_cast<const T *>(a.B) + batch * a.stride_b;
    const int64_t kbeg = (int64_t)split * a.k_per_split;
    const int64_t kend = min(a.K, kbeg + a.k_per_split);
    const int nk = (int)((kend - kbeg + BK - 1) / BK);

    u32x4 ra[CA];
    u32x4 rb[BCOL ? CBC : CBR * 4];

    auto load_tile = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int c = tid + i * NT, r = c >> 3, kc = c & 7;
            const int64_t gm = m0 + r, gk = k0 + kc * 8;
            if (gm < a.M && gk < kend)
                ra[i] = *reinterpret_cast<const u32x4 *>(A + gm * a.lda + gk);
            else
                ra[i] = u32x4{0, 0, 0, 0};
        }
        if constexpr (BCOL) {
#pragma unroll
            for (int i = 0; i < CBC; ++i) {
                const int c = tid + i * NT, r = c >> 3, kc = c & 7;
                const int64_t gn = n0 + r, gk = k0 + kc * 8;
                if (gn < a.N && gk < kend)
                    rb[i] = *reinterpret_cast<const u32x4 *>(B + gn * a.ldb + gk);
                else
                    rb[i] = u32x4{0, 0, 0, 0};
            }
        } else {
#pragma unroll
            for (int i = 0; i < CBR; ++i) {
                const int c = tid + i * NT;
                const int nb = c % (BN / 8), kb4 = c / (BN / 8);
                const int64_t gn = n0 + nb * 8;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t gk = k0 + kb4 * 4 + r;
                    if (gn < a.N && gk < kend)
                        rb[i * 4 + r] = *reinterpret_cast<const u32x4 *>(B + gk * a.ldb + gn);
                    else
                        rb[i * 4 + r] = u32x4{0, 0, 0, 0};
                }
            }
        }
    };

    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const int c = tid + i * NT, r = c >> 3, kc = c & 7;
            *reinterpret_cast<u32x4 *>(&sA[buf][r * BK + ((kc ^ swz(r)) << 3)]) = ra[i];
        }
        if constexpr (BCOL) {
#pragma unroll
            for (int i = 0; i < CBC; ++i) {
                const int c = tid + i * NT, r = c >> 3, kc = c & 7;
                *reinterpret_cast<u32x4 *>(&sB[buf][r * BK + ((kc ^ swz(r)) << 3)]) = rb[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < CBR; ++i) {
                const int c = tid + i * NT;
                const int nb = c % (BN / 8), kb4 = c / (BN / 8);
                u32x2 t[8];
                transpose4x8_b16(&rb[i * 4], t);
#pragma unroll
                for (int cc = 0; cc < 8; ++cc) {
                    const int n = nb * 8 + cc;
                    *reinterpret_cast<u32x2 *>(
                        &sB[buf][n * BK + (((kb4 >> 1) ^ swz(n)) << 3) + (kb4 & 1) * 4]) = t[cc];
                }
            }
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    if (nk > 0) {
        load_tile(kbeg);
        store_tile(0);
    }
    __syncthreads();

    const int lrow = lane & 31, lk = lane >> 5;
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load_tile(kbeg + (int64_t)(kt + 1) * BK);
        const T *pa = sA[buf];
        const T *pb = sB[buf];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            frag fa[TM], fb[TN];
            const int chunk = 2 * kk + lk;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int r = wm * WTM + i * 32 + lrow;
                fa[i] = as_frag<frag>(*reinterpret_cast<const u32x4 *>(&pa[r * BK + ((chunk ^ swz(r)) << 3)]));
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int r = wn * WTN + j * 32 + lrow;
                fb[j] = as_frag<frag>(*reinterpret_cast<const u32x4 *>(&pb[r * BK + ((chunk ^ swz(r)) << 3)]));
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<T>::m32(fa[i], fb[j], acc[i][j]);
        }
        if (kt + 1 < nk) store_tile(buf ^ 1);
        __syncthreads();
    }

    // Epilogue: lane holds column (lane % 32) and rows 8*j + 4*(lane/32) + i.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int64_t col = n0 + wn * WTN + j * 32 + lrow;
            if (col >= a.N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int64_t row = m0 + wm * WTM + i * 32 + (e >> 2) * 8 + lk * 4 + (e & 3);
                if (row >= a.M) continue;
                if constexpr (SPLIT) {
                    a.partial[((int64_t)split * a.M + row) * a.N + col] = acc[i][j][e];
                } else {
                    Tout *out = reinterpret_cast<Tout *>(a.out) + batch * a.stride_o;
                    epilogue_store<Tout>(a, out, reinterpret_cast<const Tout *>(a.cin), row, col,
                                         acc[i][j][e]);
                }
            }
        }
    }
}

// Sums split-K partials in split order, then applies alpha / beta / addend.
template <typename Tout>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs a) {
    const int64_t total = a.M * a.N;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * 256) {
        float s = 0.f;
        for (int z = 0; z < a.splits; ++z) s += a.partial[(int64_t)z * total + idx];
        const int64_t row = idx / a.N, col = idx - row * a.N;
        epilogue_store<Tout>(a, reinterpret_cast<Tout *>(a.out), reinterpret_cast<const Tout *>(a.cin),
                             row, col, s);
    }
}

// Generic LDS-tiled SIMT GEMM (any strides / shapes / float dtypes): 64x64
// tile, 256 threads each owning a 4x4 strided patch, K step 16.
template <typename Tin, typename Tacc, typename Tout>
__global__ __launch_bounds__(256) void gemm_simt_kernel(GemmArgs a, int b_col) {
    __shared__ Tacc sA[16][65];
    __shared__ Tacc sB[16][65];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int64_t m0 = (int64_t)blockIdx.x * 64, n0 = (int64_t)blockIdx.y * 64;
    const int64_t batch = blockIdx.z;
    const Tin *A = reinterpret_cast<const Tin *>(a.A) + batch * a.stride_a;
    const Tin *B = reinterpret_cast<const Tin *>(a.B) + batch * a.stride_b;
    Tacc acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0;
    for (int64_t k0 = 0; k0 < a.K; k0 += 16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = tid + 256 * i;
            const int m = e >> 4, kk = e & 15;
            const int64_t gm = m0 + m, gk = k0 + kk;
            sA[kk][m] = (gm < a.M && gk < a.K) ? (Tacc)A[gm * a.lda + gk] : (Tacc)0;
            const int kb = e >> 6, n = e & 63;
            const int64_t gn = n0 + n, gkb = k0 + kb;
            Tacc bv = 0;
            if (gn < a.N && gkb < a.K) bv = (Tacc)(b_col ? B[gn * a.ldb + gkb] : B[gkb * a.ldb + gn]);
            sB[kb][n] = bv;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            Tacc av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = sA[kk][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = sB[kk][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] += av[i] * bv[j];
        }
        __syncthreads();
    }
    Tout *out = reinterpret_cast<Tout *>(a.out) + batch * a.stride_o;
    const Tout *cin = reinterpret_cast<const Tout *>(a.cin);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t row = m0 + ty + 16 * i;
        if (row >= a.M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t col = n0 + tx + 16 * j;
            if (col >= a.N) continue;
            Tacc v = (Tacc)a.alpha * acc[i][j];
            if (a.c_kind == KUIOPS_C_FULL) v += (Tacc)a.beta * (Tacc)cin[row * a.ldcin + col];
            else if (a.c_kind == KUIOPS_C_ROW) v += (Tacc)a.beta * (Tacc)cin[col];
            out[row * a.ldo + col] = (Tout)v;
        }
    }
}

// ------------------------------------------------------------ host dispatch

struct TileCfg { int bm, bn; };

static TileCfg pick_tile(int64_t M, int64_t N, int64_t batch) {
    // 256x256 tiles only when they still give a full wave of work-groups.
    if (M >= 2048 && N >= 2048 && cdiv(M, 256) * cdiv(N, 256) * batch >= 192) return {256, 256};
    return {128, 128};
}

static int choose_splits(int64_t M, int64_t N, int64_t K, int64_t batch, TileCfg t) {
    const int64_t tiles = cdiv(M, t.bm) * cdiv(N, t.bn) * batch;
    if (batch != 1 || tiles >= 128 || K < 1024) return 1;
    int64_t s = cdiv(256, tiles);
    s = s < (K / 512) ? s : (K / 512);
    if (s > 16) s = 16;
    return s < 1 ? 1 : (int)s;
}

template <typename T, typename Tout, bool SPLIT>
static void launch_mfma(const GemmArgs &a, TileCfg t, bool bcol, int64_t gz, hipStream_t st) {
    const int64_t tiles = (int64_t)a.tiles_m * a.tiles_n;
    dim3 grid((unsigned)tiles, (unsigned)gz);
#define KUIOPS_GEMM_LAUNCH(BM, BN, WM, WN)                                                        \
    do {                                                                                          \
        if (bcol)                                                                                 \
            hipLaunchKernelGGL((gemm_mfma_kernel<T, BM, BN, WM, WN, true, Tout, SPLIT>), grid,    \
                               dim3(WM * WN * 64), 0, st, a);                                     \
        else                                                                                      \
            hipLaunchKernelGGL((gemm_mfma_kernel<T, BM, BN, WM, WN, false, Tout, SPLIT>), grid,   \
                               dim3(WM * WN * 64), 0, st, a);                                     \
    } while (0)
    if (t.bm == 256) KUIOPS_GEMM_LAUNCH(256, 256, 2, 2);
    else KUIOPS_GEMM_LAUNCH(128, 128, 2, 2);
#undef KUIOPS_GEMM_LAUNCH
}

template <typename T, typename Tout>
static int run_mfma(GemmArgs a, int64_t batch, bool bcol, int splits_req, void *ws, size_t ws_bytes,
                    hipStream_t st) {
    TileCfg t = pick_tile(a.M, a.N, batch);
    a.tiles_m = (int)cdiv(a.M, t.bm);
    a.tiles_n = (int)cdiv(a.N, t.bn);
    int splits = splits_req > 0 ? splits_req : choose_splits(a.M, a.N, a.K, batch, t);
    if (batch != 1) splits = 1;
    int64_t kps = cdiv(cdiv(a.K, splits), 64) * 64;
    splits = (int)cdiv(a.K, kps);
    if (splits <= 1) {
        a.splits = 1;
        a.k_per_split = cdiv(a.K, 64) * 64;
        if (a.K == 0) a.k_per_split = 64;
        launch_mfma<T, Tout, false>(a, t, bcol, batch, st);
        return launch_status();
    }
    const size_t need = (size_t)splits * a.M * a.N * sizeof(float);
    if (!ws || ws_bytes < need) return KUIOPS_E_WORKSPACE;
    a.splits = splits;
    a.k_per_split = kps;
    a.partial = reinterpret_cast<float *>(ws);
    launch_mfma<T, Tout, true>(a, t, bcol, splits, st);
    int64_t blocks = cdiv(a.M * a.N, 256);
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(splitk_reduce_kernel<Tout>, dim3((unsigned)blocks), dim3(256), 0, st, a);
    return launch_status();
}

template <typename Tin, typename Tacc, typename Tout>
static int run_simt(const GemmArgs &a, int64_t batch, bool bcol, hipStream_t st) {
    dim3 grid((unsigned)cdiv(a.M, 64), (unsigned)cdiv(a.N, 64), (unsigned)batch);
    hipLaunchKernelGGL((gemm_simt_kernel<Tin, Tacc, Tout>), grid, dim3(256), 0, st, a, bcol ? 1 : 0);
    return launch_status();
}

static bool mfma_eligible(const GemmArgs &a, int in_dt, bool bcol, int64_t batch) {
    if (in_dt != KUIOPS_BF16 && in_dt != KUIOPS_F16) return false;
    if (a.K % 8 || a.lda % 8 || !aligned16(a.A) || !aligned16(a.B) || a.ldb % 8) return false;
    if (batch > 1 && (a.stride_a % 8 || a.stride_b % 8)) return false;
    if (!bcol && a.N % 8) return false;
    if (a.M > INT32_MAX / 2 || a.N > INT32_MAX / 2) return false;
    return true;
}

// Shared entry for mm / addmm / bmm.
static int gemm_entry(GemmArgs a, int64_t batch, int in_dt, int out_dt, int b_layout, int splits,
                      void *ws, size_t ws_bytes, void *stream) {
    if (a.M < 0 || a.N < 0 || a.K < 0 || batch < 0) return KUIOPS_E_INVALID;
    if (b_layout != KUIOPS_B_ROW && b_layout != KUIOPS_B_COL) return KUIOPS_E_INVALID;
    if (a.c_kind < KUIOPS_C_NONE || a.c_kind > KUIOPS_C_ROW) return KUIOPS_E_INVALID;
    if (a.M == 0 || a.N == 0 || batch == 0) return KUIOPS_OK;
    if (!a.A || !a.B || !a.out || (a.c_kind != KUIOPS_C_NONE && !a.cin)) return KUIOPS_E_INVALID;
    const bool bcol = b_layout == KUIOPS_B_COL;
    hipStream_t st = as_stream(stream);
    if (batch > 65535) return KUIOPS_E_UNSUPPORTED;
    if (mfma_eligible(a, in_dt, bcol, batch)) {
        if (in_dt == KUIOPS_BF16 && out_dt == KUIOPS_BF16) return run_mfma<bf16_t, bf16_t>(a, batch, bcol, splits, ws, ws_bytes, st);
        if (in_dt == KUIOPS_BF16 && out_dt == KUIOPS_F32) return run_mfma<bf16_t, float>(a, batch, bcol, splits, ws, ws_bytes, st);
        if (in_dt == KUIOPS_F16 && out_dt == KUIOPS_F16) return run_mfma<f16_t, f16_t>(a, batch, bcol, splits, ws, ws_bytes, st);
        if (in_dt == KUIOPS_F16 && out_dt == KUIOPS_F32) return run_mfma<f16_t, float>(a, batch, bcol, splits, ws, ws_bytes, st);
        return KUIOPS_E_UNSUPPORTED;
    }
    if (cdiv(a.M, 64) > 65535 * 32 || cdiv(a.N, 64) > 65535) return KUIOPS_E_UNSUPPORTED;
    if (in_dt == KUIOPS_F32 && out_dt == KUIOPS_F32) return run_simt<float, float, float>(a, batch, bcol, st);
    if (in_dt == KUIOPS_F64 && out_dt == KUIOPS_F64) return run_simt<double, double, double>(a, batch, bcol, st);
    if (in_dt == KUIOPS_BF16 && out_dt == KUIOPS_BF16) return run_simt<bf16_t, float, bf16_t>(a, batch, bcol, st);
    if (in_dt == KUIOPS_BF16 && out_dt == KUIOPS_F32) return run_simt<bf16_t, float, float>(a, batch, bcol, st);
    if (in_dt == KUIOPS_F16 && out_dt == KUIOPS_F16) return run_simt<f16_t, float, f16_t>(a, batch, bcol, st);
    if (in_dt == KUIOPS_F16 && out_dt == KUIOPS_F32) return run_simt<f16_t, float, float>(a, batch, bcol, st);
    return KUIOPS_E_UNSUPPORTED;
}

size_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    TileCfg t = pick_tile(M, N, 1);
    int s = choose_splits(M, N, K, 1, t);
    if (s <= 1) return 0;
    return (size_t)s * M * N * sizeof(float);
}

}  // namespace kuiops

using namespace kuiops;

extern "C" int kuiops_mm(int64_t M, int64_t N, int64_t K, int in_dtype, const void *A, int64_t lda,
                         const void *B, int64_t ldb, int b_layout, int out_dtype, void *C, int64_t ldc,
                         void *stream) {
    GemmArgs a{};
    a.M = M; a.N = N; a.K = K;
    a.A = A; a.lda = lda; a.B = B; a.ldb = ldb;
    a.out = C; a.ldo = ldc;
    a.c_kind = KUIOPS_C_NONE; a.alpha = 1.f; a.beta = 0.f;
    return gemm_entry(a, 1, in_dtype, out_dtype, b_layout, 1, nullptr, 0, stream);
}

extern "C" int kuiops_addmm(int64_t M, int64_t K, int64_t N, double alpha, double beta, int in_dtype,
                            const void *A, int64_t lda, const void *B, int64_t ldb, int b_layout,
                            const void *Cin, int c_kind, int64_t ldcin, int out_dtype, void *out,
                            int64_t ldo, int splits, void *workspace, size_t workspace_bytes,
                            void *stream) {
    GemmArgs a{};
    a.M = M; a.N = N; a.K = K;
    a.A = A; a.lda = lda; a.B = B; a.ldb = ldb;
    a.out = out; a.ldo = ldo;
    a.cin = Cin; a.c_kind = c_kind; a.ldcin = ldcin;
    a.alpha = (float)alpha; a.beta = (float)beta;
    if (c_kind != KUIOPS_C_NONE && out_dtype != in_dtype) return KUIOPS_E_UNSUPPORTED;
    return gemm_entry(a, 1, in_dtype, out_dtype, b_layout, splits, workspace, workspace_bytes, stream);
}

extern "C" int kuiops_bmm(int64_t batch, int64_t M, int64_t K, int64_t N, int in_dtype, const void *A,
                          int64_t stride_a, int64_t lda, const void *B, int64_t stride_b, int64_t ldb,
                          int b_layout, int out_dtype, void *C, int64_t stride_c, int64_t ldc,
                          void *stream) {
    GemmArgs a{};
    a.M = M; a.N = N; a.K = K;
    a.A = A; a.lda = lda; a.stride_a = stride_a;
    a.B = B; a.ldb = ldb; a.stride_b = stride_b;
    a.out = C; a.ldo = ldc; a.stride_o = stride_c;
    a.c_kind = KUIOPS_C_NONE; a.alpha = 1.f; a.beta = 0.f;
    return gemm_entry(a, batch, in_dtype, out_dtype, b_layout, 1, nullptr, 0, stream);
}
